"""GPU tier: the streaming (persistent, work-balanced) decode kernel.

bf16/f16 caches at head_dim 128 go through one wave per resident slot, each
taking an equal contiguous share of the global list of 32-key stages over
all (batch, kv head, head slice) sequences. These cases pin the partition
logic against the oracle (flash_attention.py:555-589 decode on the cache
prefix; paged.py:45-99 via the gathered-pages oracle, test_paged.py:25-28):
sequences finished inside one wave, sequences cut across several waves, waves
spanning many short sequences (grid forced small through the decode_waves tuning),
zero-length paged batches, page sizes that are and are not multiples of the
32-key stage, GQA groups of 1..32 heads, and exact NaN-tail invariance.
"""

from __future__ import annotations

import contextlib

import numpy as np
import pytest
import torch

from gpu_util import check_fwd, dev, host, note
from oracle import decode_ref, paged_ref
from pallas_flash import _lib, flash_attention_decode, paged_flash_attention

pytestmark = pytest.mark.gpu

WAVES = [None, 1, 3, 7, 50]


@pytest.fixture
def waves():
    """set_waves(w): route this test's decodes through a persistent grid of w
    waves (None: one per resident slot) via the library's tuning."""
    stack = contextlib.ExitStack()

    def set_waves(w):
        stack.enter_context(_lib.tuning(decode_waves=0 if w is None else w))
    with stack:
        yield set_waves


@pytest.mark.parametrize("w", WAVES)
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("B,Hq,Hkv,cap,L", [
    (3, 8, 2, 512, 500),    # g = 4
    (2, 16, 2, 300, 257),   # g = 8 (16-row query slots)
    (2, 32, 1, 160, 33),    # g = 32: two head slices per kv head
    (5, 2, 2, 64, 1),       # one key
])
def test_stream_decode_partitions(waves, w, dt, B, Hq, Hkv, cap, L):
    waves(w)
    note(f"stream decode waves={w} dt={dt} B={B} Hq={Hq} Hkv={Hkv} cap={cap} L={L}")
    rng = np.random.default_rng(5)
    q = rng.standard_normal((B, Hq, 1, 128))
    k = rng.standard_normal((B, Hkv, cap, 128))
    v = rng.standard_normal((B, Hkv, cap, 128))
    k[:, :, L:] = np.nan
    v[:, :, L:] = np.nan
    tq, tk, tv = dev(q, dt), dev(k, dt), dev(v, dt)
    out = host(flash_attention_decode(tq, tk, tv, L))
    ref = decode_ref(host(tq), host(tk), host(tv), L)
    check_fwd(out, ref, dt)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, L:] = 3.0
    v2[:, :, L:] = -1.0
    out2 = host(flash_attention_decode(tq, dev(k2, dt), dev(v2, dt), L))
    np.testing.assert_array_equal(out, out2)


def _pool(rng, B, Hkv, page, pps, npages, lens):
    kp = rng.standard_normal((npages, Hkv, page, 128))
    vp = rng.standard_normal((npages, Hkv, page, 128))
    perm = rng.permutation(npages)
    table = np.full((B, pps), -1, np.int32)
    cur = 0
    for b, L in enumerate(lens):
        n = -(-min(int(L), pps * page) // page)
        table[b, :n] = perm[cur:cur + n]
        cur += n
    return kp, vp, table


@pytest.mark.parametrize("w", WAVES)
@pytest.mark.parametrize("page", [4, 12, 16, 32, 64, 96])
def test_stream_paged_partitions(waves, w, page):
    waves(w)
    rng = np.random.default_rng(page)
    B, Hq, Hkv, pps = 6, 8, 2, 24
    lens = np.array([0, 1, 31, 33, 5 * page + 3, pps * page], np.int32)
    npages = int(sum(-(-int(L) // page) for L in lens)) + 5
    kp, vp, table = _pool(rng, B, Hkv, page, pps, npages, lens)
    q = rng.standard_normal((B, Hq, 1, 128))
    note(f"stream paged waves={w} page={page}")
    tq, tk, tv = dev(q, "bf16"), dev(kp, "bf16"), dev(vp, "bf16")
    tt, tl = torch.as_tensor(table), torch.as_tensor(lens)
    out = host(paged_flash_attention(tq, tk, tv, tt, tl))
    ref = paged_ref(host(tq), host(tk), host(tv), np.where(table < 0, 0, table), lens)
    check_fwd(out, ref, "bf16")
    assert (out[0] == 0).all()
    # unreferenced pages and the tail past each length -> NaN: bitwise the same
    used = np.zeros(npages, bool)
    kn, vn = kp.copy(), vp.copy()
    for b, L in enumerate(lens):
        n = -(-int(L) // page)
        used[table[b, :n]] = True
        if n and L % page:
            kn[table[b, n - 1], :, L % page:] = np.nan
            vn[table[b, n - 1], :, L % page:] = np.nan
    kn[~used] = np.nan
    vn[~used] = np.nan
    out2 = host(paged_flash_attention(tq, dev(kn, "bf16"), dev(vn, "bf16"), tt, tl))
    np.testing.assert_array_equal(out, out2)


@pytest.mark.parametrize("w", [None, 64])
def test_stream_paged_many_sequences(waves, w):
    """Waves spanning many whole sequences plus cut ones (cfg5's shape, scaled)."""
    waves(w)
    rng = np.random.default_rng(21)
    B, Hq, Hkv, page, pps = 32, 32, 8, 64, 20
    lens = rng.integers(0, pps * page + 1, B).astype(np.int32)
    lens[3] = 0
    npages = int(sum(-(-int(L) // page) for L in lens)) + 3
    kp, vp, table = _pool(rng, B, Hkv, page, pps, npages, lens)
    q = rng.standard_normal((B, Hq, 1, 128))
    note(f"stream paged many waves={w}")
    tq, tk, tv = dev(q, "bf16"), dev(kp, "bf16"), dev(vp, "bf16")
    out = host(paged_flash_attention(tq, tk, tv, torch.as_tensor(table), torch.as_tensor(lens)))
    ref = paged_ref(host(tq), host(tk), host(tv), np.where(table < 0, 0, table), lens)
    check_fwd(out, ref, "bf16")
