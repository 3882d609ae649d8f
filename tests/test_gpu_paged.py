"""GPU tier: paged decode kernel vs the oracle on gathered pages.

Re-expresses the reference's test_paged.py (contiguous-equivalence cases
:31-58, shared pages :61-74, NaN pages past ctx :77-91, write-helper round
trip :94-115) plus -1 table padding, zero/over-long context lengths, bf16.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import check_fwd, dev, host, max_abs, note
from oracle import attention_ref, paged_ref
from pallas_flash import init_paged_cache, paged_flash_attention, write_to_paged_cache

pytestmark = pytest.mark.gpu


def _scrambled_table(batch, pages_per_seq, num_pages, seed):
    rng = np.random.default_rng(seed)
    return np.stack([rng.choice(num_pages, size=pages_per_seq, replace=False) for _ in range(batch)]
                    ).astype(np.int32)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("batch,n_heads,n_kv_heads,page_size,context_lens", [
    (1, 2, 2, 64, [100]),
    (3, 4, 2, 64, [10, 130, 200]),
    (2, 4, 1, 128, [128, 5]),
    (4, 2, 2, 32, [1, 33, 64, 90]),
])
def test_paged_matches_contiguous(dt, batch, n_heads, n_kv_heads, page_size, context_lens):
    note(f"paged dt={dt} B={batch} Hq={n_heads} Hkv={n_kv_heads} page={page_size} lens={context_lens}")
    dim, num_pages = 128, 32
    pps = max(context_lens) // page_size + 1
    rng = np.random.default_rng(0)
    q = rng.standard_normal((batch, n_heads, 1, dim))
    kp = rng.standard_normal((num_pages, n_kv_heads, page_size, dim))
    vp = rng.standard_normal((num_pages, n_kv_heads, page_size, dim))
    table = _scrambled_table(batch, pps, num_pages, seed=batch)
    tq, tk, tv = dev(q, dt), dev(kp, dt), dev(vp, dt)
    out = paged_flash_attention(tq, tk, tv, torch.as_tensor(table),
                                torch.as_tensor(np.array(context_lens, np.int32)), interpret=True)
    assert out.shape == tq.shape
    ref = paged_ref(host(tq), host(tk), host(tv), table, np.array(context_lens))
    check_fwd(host(out), ref, dt)
    if dt == "f32":
        assert max_abs(host(out), ref) < 2e-3


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("page_size", [1, 5, 7])
def test_paged_page_size_not_multiple_of_4(dt, page_size):
    """16-bit D = 128 pools whose page size is not a multiple of 4 run the
    generic split-KV kernel (the streaming kernel's 4-row loads need a page
    boundary every 4 rows); the reference takes any page size (paged.py:
    102-192). Scrambled table, -1 padding past the live pages, a zero and an
    over-long length, and NaN in every page no sequence reads."""
    batch, n_heads, n_kv_heads, dim = 4, 8, 2, 128
    lens = np.array([1, 0, 3 * page_size + 2, 40 * page_size], np.int32)
    pps = 24
    num_pages = 4 * pps + 8
    note(f"paged odd page dt={dt} page={page_size} lens={lens.tolist()}")
    rng = np.random.default_rng(100 + page_size)
    q = rng.standard_normal((batch, n_heads, 1, dim))
    kp = rng.standard_normal((num_pages, n_kv_heads, page_size, dim))
    vp = rng.standard_normal((num_pages, n_kv_heads, page_size, dim))
    perm = rng.permutation(num_pages)
    table = np.full((batch, pps), -1, np.int32)
    used = np.zeros(num_pages, bool)
    cur = 0
    for b in range(batch):
        n = min(-(-int(lens[b]) // page_size), pps)
        table[b, :n] = perm[cur:cur + n]
        used[perm[cur:cur + n]] = True
        cur += n
    tq, tk, tv = dev(q, dt), dev(kp, dt), dev(vp, dt)
    tt, tl = torch.as_tensor(table), torch.as_tensor(lens)
    out = paged_flash_attention(tq, tk, tv, tt, tl)
    ref = paged_ref(host(tq), host(tk), host(tv), table, lens)
    check_fwd(host(out), ref, dt)
    assert not host(out)[1].any()  # zero length -> zeros
    kn, vn = tk.clone(), tv.clone()
    unused = torch.as_tensor(np.nonzero(~used)[0], device=tk.device)
    kn[unused] = float("nan")
    vn[unused] = float("nan")
    for b in range(batch):  # rows past each length in its last live page
        L = min(int(lens[b]), pps * page_size)
        n = -(-L // page_size)
        if n and L < n * page_size:
            kn[int(table[b, n - 1]), :, L - (n - 1) * page_size:] = float("nan")
            vn[int(table[b, n - 1]), :, L - (n - 1) * page_size:] = float("nan")
    out_nan = paged_flash_attention(tq, kn, vn, tt, tl)
    torch.cuda.synchronize()
    assert torch.equal(out, out_nan)


def test_pages_are_shareable():
    rng = np.random.default_rng(7)
    q1 = rng.standard_normal((1, 2, 1, 128))
    q = np.concatenate([q1, q1])
    kp = rng.standard_normal((8, 2, 64, 128))
    vp = rng.standard_normal((8, 2, 64, 128))
    note("paged shared pages")
    out = host(paged_flash_attention(dev(q, "f32"), dev(kp, "f32"), dev(vp, "f32"),
                                     torch.tensor([[3, 5], [3, 5]], dtype=torch.int32),
                                     torch.tensor([100, 100], dtype=torch.int32)))
    np.testing.assert_array_equal(out[0], out[1])


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_unwritten_pages_do_not_leak(dt):
    page_size, dim = 64, 128
    kp = np.concatenate([np.ones((1, 2, page_size, dim)), np.full((1, 2, page_size, dim), np.nan)])
    q = np.ones((1, 2, 1, dim))
    note(f"paged nan KAT {dt}")
    out = host(paged_flash_attention(dev(q, dt), dev(kp, dt), dev(kp, dt),
                                     torch.tensor([[0, 1]], dtype=torch.int32),
                                     torch.tensor([page_size], dtype=torch.int32)))
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, 1.0, atol=1e-5)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_minus_one_padding_zero_and_overlong_lengths(dt):
    rng = np.random.default_rng(11)
    B, Hq, Hkv, page, pps, npages = 5, 8, 2, 16, 12, 64
    q = rng.standard_normal((B, Hq, 1, 128))
    kp = rng.standard_normal((npages, Hkv, page, 128))
    vp = rng.standard_normal((npages, Hkv, page, 128))
    table = np.stack([rng.permutation(npages)[:pps] for _ in range(B)]).astype(np.int32)
    lens = np.array([0, 1, 150, pps * page, pps * page + 40], np.int32)  # last: capped
    padded = table.copy()
    for b, L in enumerate(lens):
        padded[b, -(-min(L, pps * page) // page):] = -1
    used = {int(table[b, p]) for b, L in enumerate(lens) for p in range(-(-min(L, pps * page) // page))}
    kp_nan, vp_nan = kp.copy(), vp.copy()
    for p in set(range(npages)) - used:
        kp_nan[p] = np.nan
        vp_nan[p] = np.nan
    note(f"paged padding dt={dt}")
    tq = dev(q, dt)
    out = host(paged_flash_attention(tq, dev(kp_nan, dt), dev(vp_nan, dt), torch.as_tensor(padded),
                                     torch.as_tensor(lens)))
    ref = paged_ref(host(tq), host(dev(kp, dt)), host(dev(vp, dt)), table, lens)
    check_fwd(out, ref, dt)
    assert (out[0] == 0).all()
    out_clean = host(paged_flash_attention(tq, dev(kp, dt), dev(vp, dt), torch.as_tensor(table),
                                           torch.as_tensor(lens)))
    np.testing.assert_array_equal(out, out_clean)


def test_page_permutation_invariance():
    rng = np.random.default_rng(12)
    q = rng.standard_normal((1, 4, 1, 128))
    kp = rng.standard_normal((16, 2, 32, 128))
    vp = rng.standard_normal((16, 2, 32, 128))
    table = rng.permutation(16)[:6].astype(np.int32)[None]
    note("paged permutation")
    out1 = host(paged_flash_attention(dev(q, "f32"), dev(kp, "f32"), dev(vp, "f32"),
                                      torch.as_tensor(table), torch.tensor([170], dtype=torch.int32)))
    kid, vid = kp[table[0]], vp[table[0]]
    out2 = host(paged_flash_attention(dev(q, "f32"), dev(kid, "f32"), dev(vid, "f32"),
                                      torch.arange(6, dtype=torch.int32)[None],
                                      torch.tensor([170], dtype=torch.int32)))
    np.testing.assert_array_equal(out1, out2)


def test_write_to_paged_cache_roundtrip():
    page_size, dim, n_kv = 32, 128, 2
    num_pages, length = 4, 70
    kpg, vpg = init_paged_cache(num_pages, n_kv, page_size, dim, device="cuda")
    table = torch.tensor([0, 2, 1, 3], dtype=torch.int32)
    rng = np.random.default_rng(11)
    k_seq = rng.standard_normal((1, n_kv, length, dim))
    v_seq = rng.standard_normal((1, n_kv, length, dim))
    tk, tv = dev(k_seq, "f32"), dev(v_seq, "f32")
    note("paged write roundtrip")
    for pos in range(length):
        kpg, vpg = write_to_paged_cache(kpg, vpg, tk[:, :, pos:pos + 1], tv[:, :, pos:pos + 1],
                                        table, pos)
    q = rng.standard_normal((1, 2, 1, dim))
    out = host(paged_flash_attention(dev(q, "f32"), kpg, vpg, table[None],
                                     torch.tensor([length], dtype=torch.int32), interpret=True))
    ref, _ = attention_ref(q, k_seq, v_seq)
    assert max_abs(out, ref) < 1e-5
