"""GPU tier: decode-loop primitives vs the oracle.

* write_kv_cache (pf_kv_cache_write): the decode loop's ``_cache_write`` and
  the ring scatter (model.py:257-262, :437, :447-448, :475) -- index work,
  checked bit-exactly against oracle.cache_write_ref;
* write_to_paged_cache (pf_paged_cache_write): paged.py:205-223, batched --
  bit-exact against oracle.paged_write_ref, then read back by the paged
  kernel;
* flash_attention_decode_step (pf_attn_decode_step): RoPE at the position,
  cache write, attention over the live slots (model.py:340-347, :475-491) --
  against oracle.decode_step_ref: untouched slots bit-identical, the written
  slot and o within the bf16/f16 bar, a multi-step ring loop, invalid
  positions, and a captured step replayed with positions advanced on device.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import DEV, TORCH_DT, check_fwd, dev, host, max_abs, note
from oracle import cache_write_ref, decode_step_ref, paged_ref, paged_write_ref, precompute_rope_ref
from pallas_flash import (flash_attention_decode_step, paged_flash_attention, precompute_rope,
                          write_kv_cache, write_to_paged_cache)

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    """Raw storage bits (exact comparisons, NaN-safe)."""
    t = t.detach().contiguous().cpu()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).numpy()


def _rounder(dt):
    """What the device keeps of a float64 value: rounded to the storage dtype."""
    return lambda x: torch.as_tensor(np.asarray(x)).to(TORCH_DT[dt]).double().numpy()


# --------------------------------------------------------- contiguous write --
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("D", [64, 96, 128, 200, 256])
@pytest.mark.parametrize("ring,L,pos", [(False, 1, [3, 0, 9]), (False, 5, [7, 14, 0]),
                                        (True, 1, [17, 3, 40]), (True, 23, [2, 0, 31])])
def test_kv_cache_write_exact(dt, D, ring, L, pos):
    """Kernel head dims (64, 128, 16-bit 256) and any other row of whole
    16-byte chunks (96; 200 for 16-bit); float32 stops at 128."""
    note(f"kv_cache_write dt={dt} D={D} ring={ring} L={L} pos={pos}")
    rng = np.random.default_rng(11)
    B, Hkv, C = 3, 2, 16
    kc = dev(rng.standard_normal((B, Hkv, C, D)), dt)
    vc = dev(rng.standard_normal((B, Hkv, C, D)), dt)
    k = dev(rng.standard_normal((B, Hkv, L, D)), dt)
    v = dev(rng.standard_normal((B, Hkv, L, D)), dt)
    if dt == "f32" and D > 128:
        with pytest.raises(NotImplementedError):
            write_kv_cache(kc, vc, k, v, torch.tensor(pos, dtype=torch.int32, device=DEV), ring=ring)
        return
    want_k = cache_write_ref(_bits(kc), _bits(k), pos, ring=ring)
    want_v = cache_write_ref(_bits(vc), _bits(v), pos, ring=ring)
    out_k, out_v = write_kv_cache(kc, vc, k, v, torch.tensor(pos, dtype=torch.int32, device=DEV), ring=ring)
    torch.cuda.synchronize()
    assert out_k is kc and out_v is vc
    assert np.array_equal(_bits(kc), want_k)
    assert np.array_equal(_bits(vc), want_v)


def test_kv_cache_write_scalar_position_broadcasts():
    rng = np.random.default_rng(12)
    kc = dev(np.zeros((2, 1, 8, 128)), "bf16")
    vc = dev(np.zeros((2, 1, 8, 128)), "bf16")
    k = dev(rng.standard_normal((2, 1, 3, 128)), "bf16")
    write_kv_cache(kc, vc, k, k, 4)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kc), cache_write_ref(np.zeros((2, 1, 8, 128), np.int16), _bits(k), 4))


# -------------------------------------------------------------- paged write --
@pytest.mark.parametrize("dt,D", [("f32", 128), ("bf16", 128), ("f32", 96), ("bf16", 200), ("bf16", 256)])
@pytest.mark.parametrize("page_size", [16, 64])
def test_paged_cache_write_exact_then_read(dt, D, page_size):
    note(f"paged_cache_write dt={dt} D={D} page={page_size}")
    rng = np.random.default_rng(13)
    B, Hkv, Hq, num_pages, pps = 3, 2, 4, 24, 6
    lens = [page_size * 2 + 5, page_size * 6, 1]
    perm = rng.permutation(num_pages)
    table = np.full((B, pps), -1, np.int32)
    cur = 0
    for b in range(B):
        n = -(-lens[b] // page_size)
        table[b, :n] = perm[cur:cur + n]
        cur += n
    kp = dev(np.full((num_pages, Hkv, page_size, D), np.nan), dt)
    vp = dev(np.full((num_pages, Hkv, page_size, D), np.nan), dt)
    L = max(lens)
    rows_k = rng.standard_normal((B, Hkv, L, D))
    rows_v = rng.standard_normal((B, Hkv, L, D))
    tt = torch.as_tensor(table, device=DEV)
    want_k, want_v = _bits(kp), _bits(vp)
    # write each sequence's tokens in two chunks at device positions (prefill, then a step)
    for lo, hi in ((0, 3), (3, L)):
        k = dev(rows_k[:, :, lo:hi], dt)
        v = dev(rows_v[:, :, lo:hi], dt)
        want_k = paged_write_ref(want_k, _bits(k), table, lo)
        want_v = paged_write_ref(want_v, _bits(v), table, lo)
        write_to_paged_cache(kp, vp, k, v, tt, torch.full((B,), lo, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kp), want_k)
    assert np.array_equal(_bits(vp), want_v)
    # pages that no live token maps to keep their NaN fill; the paged kernel reads the rest
    q = rng.standard_normal((B, Hq, 1, D))
    out = host(paged_flash_attention(dev(q, dt), kp, vp, tt, torch.as_tensor(lens, dtype=torch.int32)))
    ref = paged_ref(host(dev(q, dt)), host(kp), host(vp), table, np.array(lens))
    check_fwd(out, ref, dt)


def test_write_to_paged_cache_reference_signature():
    """paged.py:205-223: one token, batch 1, table row [pages_per_seq], int position."""
    rng = np.random.default_rng(14)
    kp = dev(np.zeros((5, 2, 16, 128)), "bf16")
    vp = dev(np.zeros((5, 2, 16, 128)), "bf16")
    k = dev(rng.standard_normal((1, 2, 1, 128)), "bf16")
    v = dev(rng.standard_normal((1, 2, 1, 128)), "bf16")
    table = torch.tensor([3, 0, 4], dtype=torch.int32)
    out_k, out_v = write_to_paged_cache(kp, vp, k, v, table, 21)  # logical page 1 -> physical 0, offset 5
    torch.cuda.synchronize()
    assert out_k is kp and out_v is vp
    want = np.zeros((5, 2, 16, 128), np.int16)
    want[0, :, 5] = _bits(k)[0, :, 0]
    assert np.array_equal(_bits(kp), want)
    # position past the table: nothing written
    write_to_paged_cache(kp, vp, k, v, table, 3 * 16)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kp), want)


@pytest.mark.parametrize("which", ["paged", "contiguous"])
def test_cache_writes_out_of_place(which):
    """inplace=False: the given cache or pool is left bit-identical and the
    returned copies hold exactly what the in-place write produces (the
    reference's functional update, paged.py:205-223 / model.py:257-262)."""
    note(f"cache write out of place: {which}")
    rng = np.random.default_rng(15)
    if which == "paged":
        kp = dev(rng.standard_normal((6, 2, 16, 128)), "bf16")
        vp = dev(rng.standard_normal((6, 2, 16, 128)), "bf16")
        k = dev(rng.standard_normal((2, 2, 3, 128)), "bf16")
        table = torch.tensor([[4, 1, -1], [0, 5, 2]], dtype=torch.int32)
        pos = torch.tensor([14, 20], dtype=torch.int32, device=DEV)
        call = lambda a, b, inplace: write_to_paged_cache(a, b, k, k, table, pos, inplace=inplace)
    else:
        kp = dev(rng.standard_normal((2, 2, 16, 96)), "f16")
        vp = dev(rng.standard_normal((2, 2, 16, 96)), "f16")
        k = dev(rng.standard_normal((2, 2, 5, 96)), "f16")
        call = lambda a, b, inplace: write_kv_cache(a, b, k, k, [3, 13], ring=True, inplace=inplace)
    before_k, before_v = _bits(kp), _bits(vp)
    nk, nv = call(kp, vp, False)
    torch.cuda.synchronize()
    assert nk.data_ptr() != kp.data_ptr() and nv.data_ptr() != vp.data_ptr()
    assert np.array_equal(_bits(kp), before_k) and np.array_equal(_bits(vp), before_v)
    assert not np.array_equal(_bits(nk), before_k)
    ik, iv = call(kp, vp, True)
    torch.cuda.synchronize()
    assert ik is kp and iv is vp
    assert np.array_equal(_bits(nk), _bits(kp)) and np.array_equal(_bits(nv), _bits(vp))


# -------------------------------------------------------------- decode step --
def _step_inputs(rng, B, Hq, Hkv, C, D, dt):
    return (dev(rng.standard_normal((B, Hq, 1, D)), dt), dev(rng.standard_normal((B, Hkv, 1, D)), dt),
            dev(rng.standard_normal((B, Hkv, 1, D)), dt), dev(rng.standard_normal((B, Hkv, C, D)), dt),
            dev(rng.standard_normal((B, Hkv, C, D)), dt))


def _check_step(dt, q, kn, vn, kc0, vc0, kc, vc, o, pos, cos, sin, ring):
    """o within the bar; the written slots within one storage rounding of the
    oracle; every other slot bit-identical to before."""
    C = kc0.shape[2]
    store = _rounder(dt)
    o_ref, kc_ref, vc_ref = decode_step_ref(host(q), host(kn), host(vn), host(kc0), host(vc0), pos,
                                            None if cos is None else host(cos),
                                            None if sin is None else host(sin), ring=ring, store=store)
    check_fwd(host(o), o_ref, dt)
    B = q.shape[0]
    posv = np.broadcast_to(np.asarray(pos).reshape(-1), (B,))
    bits_k, bits_k0, bits_v, bits_v0 = _bits(kc), _bits(kc0), _bits(vc), _bits(vc0)
    for b in range(B):
        p = int(posv[b])
        valid = p >= 0 and (ring or p < C) and (cos is None or p < cos.shape[0])
        slot = (p % C if ring else p) if valid else -1
        keep = [s for s in range(C) if s != slot]
        assert np.array_equal(bits_k[b][:, keep], bits_k0[b][:, keep])
        assert np.array_equal(bits_v[b][:, keep], bits_v0[b][:, keep])
        if valid:
            assert np.array_equal(bits_v[b][:, slot], _bits(vn)[b][:, 0])
            assert max_abs(host(kc)[b][:, slot], kc_ref[b][:, slot]) <= 2e-2


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("Hq,Hkv", [(8, 2), (32, 8), (4, 4), (32, 1), (24, 1)])
@pytest.mark.parametrize("ring", [False, True])
def test_decode_step_matches_oracle(dt, Hq, Hkv, ring):
    """(32, 1) and (24, 1): the group spans two 16-head slices, each of which
    streams (and patches) the new token's stage; only slice 0 writes the cache."""
    note(f"decode_step dt={dt} Hq={Hq} Hkv={Hkv} ring={ring}")
    rng = np.random.default_rng(15)
    B, C, D = 4, 200, 128
    q, kn, vn, kc, vc = _step_inputs(rng, B, Hq, Hkv, C, D, dt)
    kc0, vc0 = kc.clone(), vc.clone()
    cos, sin = precompute_rope(1024, D, 10000.0, device=DEV)
    pos = [0, 77, 199, 531] if ring else [0, 77, 199, 31]
    o = flash_attention_decode_step(q, kn, vn, kc, vc, torch.tensor(pos, dtype=torch.int32, device=DEV),
                                    cos, sin, ring=ring)
    torch.cuda.synchronize()
    _check_step(dt, q, kn, vn, kc0, vc0, kc, vc, o, pos, cos, sin, ring)


def test_decode_step_without_rope_and_scalar_position():
    rng = np.random.default_rng(16)
    q, kn, vn, kc, vc = _step_inputs(rng, 3, 8, 2, 96, 128, "bf16")
    kc0, vc0 = kc.clone(), vc.clone()
    o = flash_attention_decode_step(q, kn, vn, kc, vc, 40)
    torch.cuda.synchronize()
    _check_step("bf16", q, kn, vn, kc0, vc0, kc, vc, o, 40, None, None, False)


def test_decode_step_invalid_positions_write_nothing():
    rng = np.random.default_rng(17)
    q, kn, vn, kc, vc = _step_inputs(rng, 4, 8, 2, 64, 128, "bf16")
    kc0, vc0 = kc.clone(), vc.clone()
    cos, sin = precompute_rope(100, 128, 10000.0, device=DEV)
    pos = [-3, 64, 10, 100]  # negative, past the capacity, valid, past the RoPE table
    o = flash_attention_decode_step(q, kn, vn, kc, vc, torch.tensor(pos, dtype=torch.int32, device=DEV),
                                    cos, sin)
    torch.cuda.synchronize()
    oh = host(o)
    assert not oh[[0, 1, 3]].any()
    _check_step("bf16", q, kn, vn, kc0, vc0, kc, vc, o, pos, cos, sin, False)


def test_decode_step_ring_loop_matches_oracle():
    """A generate_streaming-style loop (model.py:406-531) on the attention
    path: every step writes one token into a ring of 40 slots and attends the
    live window; sequences start at different positions and wrap."""
    note("decode_step ring loop")
    rng = np.random.default_rng(18)
    B, Hq, Hkv, C, D, T = 3, 8, 2, 40, 128, 90
    cos, sin = precompute_rope(512, D, 10000.0, device=DEV)
    kc = dev(np.zeros((B, Hkv, C, D)), "bf16")
    vc = dev(np.zeros((B, Hkv, C, D)), "bf16")
    kc_ref = np.zeros((B, Hkv, C, D))
    vc_ref = np.zeros((B, Hkv, C, D))
    start = np.array([0, 0, 0], np.int64)
    pos = torch.tensor(start, dtype=torch.int32, device=DEV)
    worst = 0.0
    for t in range(T):
        q = dev(rng.standard_normal((B, Hq, 1, D)), "bf16")
        kn = dev(rng.standard_normal((B, Hkv, 1, D)), "bf16")
        vn = dev(rng.standard_normal((B, Hkv, 1, D)), "bf16")
        o = flash_attention_decode_step(q, kn, vn, kc, vc, pos, cos, sin, ring=True)
        o_ref, kc_ref, vc_ref = decode_step_ref(host(q), host(kn), host(vn), kc_ref, vc_ref, start + t,
                                                host(cos), host(sin), ring=True, store=_rounder("bf16"))
        worst = max(worst, max_abs(host(o), o_ref))
        pos += 1
    torch.cuda.synchronize()
    assert worst <= 2e-2, f"ring loop max-abs error {worst:.3e}"
    assert max_abs(host(kc), kc_ref) <= 2e-2 and np.array_equal(host(vc), vc_ref)


def test_decode_step_graph_replay_advances_positions_on_device():
    """One captured decode step replayed while the positions advance on the
    GPU (no host-side value depends on them): every replay equals the eager
    step at that position."""
    note("decode_step graph replay")
    rng = np.random.default_rng(19)
    B, Hq, Hkv, C, D = 2, 8, 2, 64, 128
    cos, sin = precompute_rope(256, D, 10000.0, device=DEV)
    q, kn, vn, kc, vc = _step_inputs(rng, B, Hq, Hkv, C, D, "bf16")
    kc_e, vc_e = kc.clone(), vc.clone()
    pos = torch.tensor([5, 30], dtype=torch.int32, device=DEV)
    pos_e = pos.clone()
    # warm up on a side stream (allocator), then capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        flash_attention_decode_step(q, kn, vn, kc.clone(), vc.clone(), pos.clone(), cos, sin, ring=True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_g = flash_attention_decode_step(q, kn, vn, kc, vc, pos, cos, sin, ring=True)
    for step in range(70):  # wraps the 64-slot ring
        graph.replay()
        o_e = flash_attention_decode_step(q, kn, vn, kc_e, vc_e, pos_e, cos, sin, ring=True)
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e), f"replay {step}"
        pos += 1
        pos_e += 1
    assert torch.equal(kc, kc_e) and torch.equal(vc, vc_e)


def test_decode_step_config4_shape():
    """BASELINE config 4's shape as a decode step: B=64, Hq=32, Hkv=8, capacity
    8192, new token at position 5999 (kv_len 6000); oracle on 4 sequences."""
    note("decode_step config4 shape")
    rng = np.random.default_rng(20)
    B, Hq, Hkv, C, D = 64, 32, 8, 8192, 128
    g = torch.Generator(device=DEV).manual_seed(20)
    kc = torch.randn((B, Hkv, C, D), generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn((B, Hkv, C, D), generator=g, device=DEV).to(torch.bfloat16)
    kc[:, :, 6000:] = float("nan")
    vc[:, :, 6000:] = float("nan")
    q = dev(rng.standard_normal((B, Hq, 1, D)), "bf16")
    kn = dev(rng.standard_normal((B, Hkv, 1, D)), "bf16")
    vn = dev(rng.standard_normal((B, Hkv, 1, D)), "bf16")
    cos, sin = precompute_rope(C, D, 10000.0, device=DEV)
    sel = [0, 17, 40, 63]
    kc0 = host(kc[sel, :, :6000])
    vc0 = host(vc[sel, :, :6000])
    o = flash_attention_decode_step(q, kn, vn, kc, vc, 5999, cos, sin)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()
    kfull = np.concatenate([kc0, np.zeros((4, Hkv, 1, D))], axis=2)
    vfull = np.concatenate([vc0, np.zeros((4, Hkv, 1, D))], axis=2)
    o_ref, _, _ = decode_step_ref(host(q)[sel], host(kn)[sel], host(vn)[sel], kfull, vfull, 5999,
                                  host(cos), host(sin), store=_rounder("bf16"))
    check_fwd(host(o)[sel], o_ref, "bf16")


@pytest.mark.parametrize("Hq,Hkv", [(8, 2), (4, 4)])
def test_decode_loop_matches_full_causal_attention(Hq, Hkv):
    """test_model.py::test_cached_matches_recompute on the attention path:
    prefill a prompt (write_kv_cache + causal flash_attention on the rotated
    q/k), then feed the remaining tokens one at a time through
    flash_attention_decode_step -- every step's output equals the matching row
    of causal attention over the whole sequence computed at once."""
    from pallas_flash import apply_rope, flash_attention
    note(f"decode loop vs full causal Hq={Hq} Hkv={Hkv}")
    rng = np.random.default_rng(25)
    B, D, P, T, C = 2, 128, 37, 70, 96  # prompt 37 tokens, 33 decode steps, cache 96
    q = dev(rng.standard_normal((B, Hq, T, D)), "bf16")
    k = dev(rng.standard_normal((B, Hkv, T, D)), "bf16")
    v = dev(rng.standard_normal((B, Hkv, T, D)), "bf16")
    cos, sin = precompute_rope(C, D, 10000.0, device=DEV)
    # recompute: rotate the whole sequence (float32, rounded once), causal attention
    qr = apply_rope(q.float(), cos[:T], sin[:T]).to(torch.bfloat16)
    kr = apply_rope(k.float(), cos[:T], sin[:T]).to(torch.bfloat16)
    full = host(flash_attention(qr, kr, v, causal=True))
    # cached: prefill writes the rotated prompt keys, then one decode step per token
    kc = torch.zeros((B, Hkv, C, D), dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    write_kv_cache(kc, vc, kr[:, :, :P], v[:, :, :P], 0)
    pos = torch.full((B,), P, dtype=torch.int32, device=DEV)
    worst = 0.0
    for t in range(P, T):
        o = flash_attention_decode_step(q[:, :, t:t + 1], k[:, :, t:t + 1], v[:, :, t:t + 1], kc, vc, pos,
                                        cos, sin)
        worst = max(worst, max_abs(host(o)[:, :, 0], full[:, :, t]))
        pos += 1
    torch.cuda.synchronize()
    assert worst <= 2e-2, f"cached vs recompute max-abs {worst:.3e}"
    # the cache now holds exactly the rotated keys and values of all T tokens
    assert max_abs(host(kc[:, :, :T]), host(kr)) <= 2e-2
    assert torch.equal(vc[:, :, :T], v)
