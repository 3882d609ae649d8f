"""CPU tier: the C-ABI library loads, exports every symbol the header declares,
and rejects invalid arguments on the host before touching a device.

No call here reaches a kernel launch: every call carries an argument the host
validation refuses (or is a pure-host query such as the workspace size).
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT
from pallas_flash import _lib

HEADER = os.path.join(ROOT, "include", "pallas_flash_amd.h")


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(pf_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


def test_header_declares_expected_entry_points():
    names = _declared_functions()
    for want in ("pf_attn_fwd", "pf_attn_fwd_rope", "pf_attn_fwd_rope_workspace_size",
                 "pf_attn_bwd", "pf_attn_bwd_delta",
                 "pf_attn_bwd_dq", "pf_attn_bwd_dkv", "pf_attn_decode",
                 "pf_attn_decode_workspace_size", "pf_paged_attn", "pf_paged_attn_workspace_size",
                 "pf_rope", "pf_kv_cache_write", "pf_paged_cache_write", "pf_attn_decode_step",
                 "pf_attn_decode_step_workspace_size", "pf_version"):
        assert want in names


def test_library_exports_every_declared_symbol(L):
    for name in _declared_functions():
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature in _lib.py"


def test_version(L):
    assert b"gfx950" in L.pf_version()


def test_struct_sizes_match_c_layout():
    # pointers 8 bytes; int32/float 4; size_t 8 (x86-64 SysV)
    assert ctypes.sizeof(_lib.FwdArgs) == 5 * 8 + 10 * 4
    assert ctypes.sizeof(_lib.FwdRopeArgs) == ctypes.sizeof(_lib.FwdArgs) + 4 * 8 + 8 + 8
    assert ctypes.sizeof(_lib.BwdArgs) == 10 * 8 + 10 * 4
    assert ctypes.sizeof(_lib.DecodeArgs) == 4 * 8 + 8 * 4 + 8 + 8
    assert ctypes.sizeof(_lib.PagedArgs) == 6 * 8 + 9 * 4 + 4 + 8 + 8
    assert ctypes.sizeof(_lib.RopeArgs) == 4 * 8 + 7 * 4 + 4
    assert ctypes.sizeof(_lib.KvWriteArgs) == 5 * 8 + 8 * 4
    assert ctypes.sizeof(_lib.PagedWriteArgs) == 6 * 8 + 9 * 4 + 4
    # 7 pointers, stride + pad, cos/sin, 9 x 4-byte fields + pad, workspace, size_t
    assert ctypes.sizeof(_lib.DecodeStepArgs) == 7 * 8 + 8 + 2 * 8 + 9 * 4 + 4 + 8 + 8
    assert _lib.DecodeStepArgs.cos.offset == 7 * 8 + 8
    assert _lib.DecodeStepArgs.workspace.offset == 7 * 8 + 8 + 2 * 8 + 9 * 4 + 4


def _fwd(**over):
    base = dict(q=8, k=8, v=8, o=8, lse=None, batch=1, num_heads=4, num_kv_heads=2, seq_len_q=16,
                seq_len_k=16, head_dim=128, kv_len=16, causal=0, sm_scale=0.1, dtype=1)
    base.update(over)
    return _lib.FwdArgs(**base)


@pytest.mark.parametrize("over,status", [
    (dict(num_heads=6, num_kv_heads=4), _lib.PF_ERR_INVALID),        # flash_attention.py:537
    (dict(kv_len=0), _lib.PF_ERR_INVALID),                           # :544
    (dict(kv_len=17), _lib.PF_ERR_INVALID),
    (dict(num_kv_heads=0), _lib.PF_ERR_INVALID),
    (dict(q=None), _lib.PF_ERR_INVALID),
    (dict(sm_scale=float("nan")), _lib.PF_ERR_INVALID),
    (dict(head_dim=96), _lib.PF_ERR_UNSUPPORTED),                  # kernels: 64, 128, 256 (16-bit)
    (dict(head_dim=192), _lib.PF_ERR_UNSUPPORTED),
    (dict(head_dim=512), _lib.PF_ERR_UNSUPPORTED),
    (dict(head_dim=256, dtype=0), _lib.PF_ERR_UNSUPPORTED),        # float32 stops at 128
    (dict(dtype=7), _lib.PF_ERR_UNSUPPORTED),
])
def test_fwd_rejects_on_host(L, over, status):
    assert L.pf_attn_fwd(_fwd(**over), None) == status


def test_fwd_null_args(L):
    assert L.pf_attn_fwd(None, None) == _lib.PF_ERR_INVALID


def test_rope_requires_tables(L):
    args = _lib.FwdRopeArgs(_fwd(), None, None, None, None, 256, 1 << 20)
    assert L.pf_attn_fwd_rope(args, None) == _lib.PF_ERR_INVALID


def test_rope_workspace_size_and_rejection(L):
    # rotated-K workspace = K's bytes (bf16 [1, 2, 16, 128]), rounded up to 256
    args = _lib.FwdRopeArgs(_fwd(), 8, 8, 8, 8, None, 0)
    assert L.pf_attn_fwd_rope_workspace_size(args) == 2 * 16 * 128 * 2
    assert L.pf_attn_fwd_rope(args, None) == _lib.PF_ERR_WORKSPACE
    args.workspace, args.workspace_bytes = 256, 2 * 16 * 128 * 2 - 1
    assert L.pf_attn_fwd_rope(args, None) == _lib.PF_ERR_WORKSPACE
    args.workspace, args.workspace_bytes = 264, 1 << 20  # not 256-byte aligned
    assert L.pf_attn_fwd_rope(args, None) == _lib.PF_ERR_WORKSPACE
    args.base.head_dim = 96
    assert L.pf_attn_fwd_rope_workspace_size(args) == 0


def test_bwd_requires_buffers(L):
    a = _lib.BwdArgs(q=8, k=8, v=8, o=8, do_=8, lse=8, delta=8, dq=8, dk=8, dv=None, batch=1,
                     num_heads=2, num_kv_heads=2, seq_len_q=8, seq_len_k=8, head_dim=128, kv_len=8,
                     causal=1, sm_scale=0.1, dtype=0)
    for fn in (L.pf_attn_bwd, L.pf_attn_bwd_dkv, L.pf_attn_bwd_dq):
        assert fn(a, None) == _lib.PF_ERR_INVALID
    a.dv = 8
    a.num_heads = 3
    assert L.pf_attn_bwd(a, None) == _lib.PF_ERR_INVALID


@pytest.mark.parametrize("sq,sk", [(1 << 22, 8), (8, 1 << 22), (1 << 23, 1 << 23)])
def test_bwd_rejects_sequences_past_32bit_offsets(L, sq, sk):
    """The backward kernels address one head's rows with 32-bit byte offsets
    (buffer descriptors): longer sequences are refused, never wrapped."""
    a = _lib.BwdArgs(q=8, k=8, v=8, o=8, do_=8, lse=8, delta=8, dq=8, dk=8, dv=8, batch=1,
                     num_heads=1, num_kv_heads=1, seq_len_q=sq, seq_len_k=sk, head_dim=128, kv_len=sk,
                     causal=0, sm_scale=0.1, dtype=1)
    for fn in (L.pf_attn_bwd, L.pf_attn_bwd_dkv, L.pf_attn_bwd_dq, L.pf_attn_bwd_delta):
        assert fn(a, None) == _lib.PF_ERR_UNSUPPORTED


def _dec(**over):
    base = dict(q=8, k_cache=8, v_cache=8, o=8, batch=64, num_heads=32, num_kv_heads=8,
                cache_size=8192, head_dim=128, cache_len=6000, sm_scale=0.1, dtype=1,
                workspace=None, workspace_bytes=0)
    base.update(over)
    return _lib.DecodeArgs(**base)


def test_decode_workspace_and_rejections(L):
    ws = L.pf_attn_decode_workspace_size(_dec())
    assert ws > 0 and ws % 256 == 0
    # workspace missing -> rejected before launch
    assert L.pf_attn_decode(_dec(), None) == _lib.PF_ERR_WORKSPACE
    assert L.pf_attn_decode(_dec(workspace=256, workspace_bytes=ws - 1), None) == _lib.PF_ERR_WORKSPACE
    assert L.pf_attn_decode(_dec(workspace=100, workspace_bytes=ws), None) == _lib.PF_ERR_WORKSPACE
    assert L.pf_attn_decode(_dec(cache_len=0), None) == _lib.PF_ERR_INVALID
    assert L.pf_attn_decode(_dec(cache_len=8193), None) == _lib.PF_ERR_INVALID
    assert L.pf_attn_decode_workspace_size(_dec(num_heads=30)) == 0


def _paged(**over):
    base = dict(q=8, k_pages=8, v_pages=8, block_tables=8, context_lens=8, o=8, batch=128,
                num_heads=32, num_kv_heads=8, num_pages=16384, page_size=64, head_dim=128,
                pages_per_seq=128, sm_scale=0.1, dtype=1, workspace=None, workspace_bytes=0)
    base.update(over)
    return _lib.PagedArgs(**base)


def test_paged_workspace_and_rejections(L):
    ws = L.pf_paged_attn_workspace_size(_paged())
    assert ws > 0
    assert L.pf_paged_attn(_paged(), None) == _lib.PF_ERR_WORKSPACE
    assert L.pf_paged_attn(_paged(num_heads=12), None) == _lib.PF_ERR_INVALID
    assert L.pf_paged_attn(_paged(context_lens=None, workspace=256, workspace_bytes=ws), None) == _lib.PF_ERR_INVALID
    # any head_dim up to 256 (16-bit) or 128 (float32) whose rows are whole
    # 16-byte chunks is read in place
    assert L.pf_paged_attn_workspace_size(_paged(head_dim=80)) > 0
    assert L.pf_paged_attn_workspace_size(_paged(head_dim=96, dtype=0)) > 0
    assert L.pf_paged_attn_workspace_size(_paged(head_dim=136)) > 0
    assert L.pf_paged_attn_workspace_size(_paged(head_dim=256, dtype=2)) > 0
    for bad in (dict(head_dim=84), dict(head_dim=264), dict(head_dim=0), dict(head_dim=6, dtype=0),
                dict(head_dim=136, dtype=0)):
        assert L.pf_paged_attn(_paged(**bad), None) == _lib.PF_ERR_UNSUPPORTED, bad
        assert L.pf_paged_attn_workspace_size(_paged(**bad)) == 0, bad


def test_decode_head_dims_read_in_place(L):
    """pf_attn_decode takes head_dim 8..256 (16-bit) or 4..128 (float32) in
    steps of one 16-byte chunk (8 elements for 16-bit dtypes, 4 for
    float32); the workspace holds the partials at the compute width (64,
    128 or 256)."""
    for d, dt in ((80, 1), (96, 2), (8, 1), (36, 0), (100, 0), (136, 1), (200, 2), (256, 1)):
        ws = L.pf_attn_decode_workspace_size(_dec(head_dim=d, dtype=dt))
        assert ws > 0 and ws % 256 == 0, (d, dt)
    # the generic kernel's partials are the compute width wide: 256 above 128
    assert (L.pf_attn_decode_workspace_size(_dec(head_dim=136, dtype=1))
            > L.pf_attn_decode_workspace_size(_dec(head_dim=96, dtype=1)))
    for d, dt in ((84, 1), (100, 1), (6, 0), (132, 0), (264, 1), (256, 0)):
        assert L.pf_attn_decode(_dec(head_dim=d, dtype=dt), None) == _lib.PF_ERR_UNSUPPORTED, (d, dt)


def test_status_mapping():
    _lib.check(_lib.PF_OK, "x")
    with pytest.raises(ValueError):
        _lib.check(_lib.PF_ERR_INVALID, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.PF_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.PF_ERR_LAUNCH, "x")


def _kvw(**over):
    base = dict(k=8, v=8, k_cache=8, v_cache=8, positions=8, positions_stride=1, batch=2,
                num_kv_heads=2, seq_len=3, cache_size=16, head_dim=128, ring=0, dtype=1)
    base.update(over)
    return _lib.KvWriteArgs(**base)


@pytest.mark.parametrize("over,status", [
    (dict(batch=-1), _lib.PF_ERR_INVALID),
    (dict(positions_stride=2), _lib.PF_ERR_INVALID),
    (dict(ring=3), _lib.PF_ERR_INVALID),
    (dict(cache_size=0), _lib.PF_ERR_INVALID),
    (dict(positions=None), _lib.PF_ERR_INVALID),
    (dict(dtype=9), _lib.PF_ERR_UNSUPPORTED),
    (dict(head_dim=84), _lib.PF_ERR_UNSUPPORTED),                   # rows of whole 16-byte chunks only
    (dict(head_dim=264), _lib.PF_ERR_UNSUPPORTED),
    (dict(head_dim=132, dtype=0), _lib.PF_ERR_UNSUPPORTED),          # float32 stops at 128
    (dict(seq_len=0, k=None, v=None, positions=None), _lib.PF_OK),  # nothing to write
])
def test_kv_cache_write_rejects_on_host(L, over, status):
    assert L.pf_kv_cache_write(_kvw(**over), None) == status


def _pw(**over):
    base = dict(k=8, v=8, k_pages=8, v_pages=8, block_tables=8, positions=8, positions_stride=0,
                batch=2, num_kv_heads=2, seq_len=1, num_pages=10, page_size=16, head_dim=128,
                pages_per_seq=4, dtype=1)
    base.update(over)
    return _lib.PagedWriteArgs(**base)


@pytest.mark.parametrize("over,status", [
    (dict(num_pages=0), _lib.PF_ERR_INVALID),
    (dict(page_size=0), _lib.PF_ERR_INVALID),
    (dict(pages_per_seq=-1), _lib.PF_ERR_INVALID),
    (dict(block_tables=None), _lib.PF_ERR_INVALID),
    (dict(positions_stride=5), _lib.PF_ERR_INVALID),
    (dict(dtype=4), _lib.PF_ERR_UNSUPPORTED),
    (dict(head_dim=100), _lib.PF_ERR_UNSUPPORTED),
    (dict(head_dim=256, dtype=0), _lib.PF_ERR_UNSUPPORTED),
    (dict(pages_per_seq=0, block_tables=None), _lib.PF_OK),  # no page to write into
])
def test_paged_cache_write_rejects_on_host(L, over, status):
    assert L.pf_paged_cache_write(_pw(**over), None) == status


def _step(**over):
    base = dict(q=8, k_new=8, v_new=8, k_cache=8, v_cache=8, o=8, positions=8, positions_stride=1,
                cos=8, sin=8, rope_len=8192, batch=64, num_heads=32, num_kv_heads=8, cache_size=8192,
                head_dim=128, ring=0, sm_scale=0.1, dtype=1, workspace=None, workspace_bytes=0)
    base.update(over)
    return _lib.DecodeStepArgs(**base)


def test_decode_step_workspace_and_rejections(L):
    ws = L.pf_attn_decode_step_workspace_size(_step())
    assert ws > 0 and ws % 256 == 0
    # one streaming-decode launch: the same split partials as a plain decode
    # of that cache (the rotation and the cache write happen in the kernel)
    plain = L.pf_attn_decode_workspace_size(_dec(batch=64, num_heads=32, num_kv_heads=8, cache_size=8192))
    assert ws == plain
    assert L.pf_attn_decode_step(_step(), None) == _lib.PF_ERR_WORKSPACE
    assert L.pf_attn_decode_step(_step(workspace=256, workspace_bytes=ws - 1), None) == _lib.PF_ERR_WORKSPACE
    assert L.pf_attn_decode_step(_step(workspace=100, workspace_bytes=ws), None) == _lib.PF_ERR_WORKSPACE
    for over, status in [(dict(sin=None), _lib.PF_ERR_INVALID),       # tables come in pairs
                         (dict(rope_len=0), _lib.PF_ERR_INVALID),
                         (dict(num_heads=12), _lib.PF_ERR_INVALID),
                         (dict(positions_stride=2), _lib.PF_ERR_INVALID),
                         (dict(ring=2), _lib.PF_ERR_INVALID),
                         (dict(sm_scale=float("inf")), _lib.PF_ERR_INVALID),
                         (dict(dtype=0), _lib.PF_ERR_UNSUPPORTED),     # streaming path: 16-bit only
                         (dict(head_dim=64), _lib.PF_ERR_UNSUPPORTED)]:
        assert L.pf_attn_decode_step(_step(**over), None) == status, over
        assert L.pf_attn_decode_step_workspace_size(_step(**over)) == 0, over
    # no tables: no rotation, still valid
    assert L.pf_attn_decode_step_workspace_size(_step(cos=None, sin=None, rope_len=0)) == ws


def _rope_args(**over):
    base = dict(x=8, out=8, cos=8, sin=8, batch=1, heads=2, seq_len=64, head_dim=128, rope_len=64,
                inverse=0, dtype=1)
    base.update(over)
    return _lib.RopeArgs(**base)


@pytest.mark.parametrize("over,status", [
    (dict(rope_len=63), _lib.PF_ERR_INVALID),        # table shorter than the rows
    (dict(head_dim=127), _lib.PF_ERR_INVALID),       # odd head_dim (fused_rope.py:168-169)
    (dict(inverse=2), _lib.PF_ERR_INVALID),
    (dict(sin=None), _lib.PF_ERR_INVALID),
    (dict(head_dim=96), _lib.PF_ERR_UNSUPPORTED),
    (dict(head_dim=256, dtype=0), _lib.PF_ERR_UNSUPPORTED),
    (dict(seq_len=0, x=None, out=None), _lib.PF_OK),
])
def test_rope_rejects_on_host(L, over, status):
    assert L.pf_rope(_rope_args(**over), None) == status


# pf_tuning defaults (capi.hip: Tuning)
TUNING_DEFAULTS = {"tail_dynamic_pct": 30, "decode_stages": 2, "decode_waves": 0}


def test_tuning_round_trip_and_rejections(L):
    """pf_get_tuning / pf_set_tuning: defaults (no PF_* variables in this
    environment), out-of-range values refused without changing anything,
    and the context manager restores the previous values."""
    import os
    if any(v in os.environ for v in ("PF_TAIL_DYNAMIC_PCT", "PF_DECODE_STAGES", "PF_DECODE_WAVES")):
        pytest.skip("tuning variables set in this environment")
    assert _lib.get_tuning() == TUNING_DEFAULTS
    for bad in (dict(tail_dynamic_pct=-1), dict(tail_dynamic_pct=101), dict(decode_stages=1),
                dict(decode_stages=5), dict(decode_waves=-1)):
        t = _lib.Tuning(**{**_lib.get_tuning(), **bad})
        assert L.pf_set_tuning(ctypes.byref(t)) == _lib.PF_ERR_INVALID
        assert _lib.get_tuning() == TUNING_DEFAULTS
    assert L.pf_set_tuning(None) == _lib.PF_ERR_INVALID
    assert L.pf_get_tuning(None) == _lib.PF_ERR_INVALID
    with _lib.tuning(tail_dynamic_pct=37, decode_waves=7) as t:
        assert t == _lib.get_tuning() == {**TUNING_DEFAULTS, "tail_dynamic_pct": 37, "decode_waves": 7}
    assert _lib.get_tuning() == TUNING_DEFAULTS
    with pytest.raises(TypeError):
        with _lib.tuning(block_q=64):
            pass


def test_paged_noalloc_refuses_on_host(L):
    """pf_paged_attn_noalloc validates like pf_paged_attn and refuses, before
    any HIP call, a problem whose partials exceed its static array."""
    text = open(HEADER).read()
    m = re.search(r"#define PF_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    scratch = int(m.group(1)) << int(m.group(2))
    bad = _lib.PagedArgs(q=8, k_pages=8, v_pages=8, block_tables=8, context_lens=8, o=8, batch=2,
                         num_heads=3, num_kv_heads=2, num_pages=4, page_size=5, head_dim=128,
                         pages_per_seq=2, sm_scale=0.1, dtype=0, workspace=None, workspace_bytes=0)
    assert L.pf_paged_attn_noalloc(bad, None) == _lib.PF_ERR_INVALID  # 3 % 2 heads
    big = _lib.PagedArgs(q=8, k_pages=8, v_pages=8, block_tables=8, context_lens=8, o=8, batch=4096,
                         num_heads=32, num_kv_heads=8, num_pages=8, page_size=5, head_dim=128,
                         pages_per_seq=2, sm_scale=0.1, dtype=0, workspace=None, workspace_bytes=0)
    assert L.pf_paged_attn_workspace_size(big) > scratch
    assert L.pf_paged_attn_noalloc(big, None) == _lib.PF_ERR_WORKSPACE
