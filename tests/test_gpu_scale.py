"""GPU tier: parity at BASELINE's full sizes (configs 2-5).

The other GPU tests pin semantics against the float64 oracle at sizes it
finishes in seconds; those grids are small enough that every workgroup has a
CU to itself. These cases run the kernels at the benchmarked shapes, where
several workgroups share each CU's LDS and the persistent decode grid spans
the whole chip, against a float32 PyTorch restatement of the same algorithm
(flash_attention.py:61-159 and :233-442 forward/backward, fused_rope.py:43-113,
paged.py:45-99) computed on the GPU one (batch, KV-head group) at a time.
Inputs are rounded to bf16 first, so both sides see the same values.

Bars (north star): bf16 outputs <= 2e-2 max-abs; bf16 gradients <= 5e-2
relative (max-abs error / max-abs reference); LSE <= 1e-3 max-abs; masking
exact (NaN in never-attended slots must not change a single output bit).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import note
from pallas_flash import (flash_attention, flash_attention_decode, flash_attention_rope,
                          flash_attention_with_lse, paged_flash_attention, precompute_rope)

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _randn(g, *shape):
    return torch.randn(shape, generator=g, device=DEV, dtype=torch.float32).to(torch.bfloat16)


def _attn_group(qg, kh, vh, scale, causal, dog=None):
    """float32 attention of one GQA group: qg [g, Sq, D], kh/vh [Sk, D].
    Returns o, lse and, with dog, the group's dq and group-summed dk, dv."""
    s = torch.matmul(qg, kh.t().contiguous()) * scale
    if causal:
        Sq, Sk = s.shape[1], s.shape[2]
        s.masked_fill_(torch.ones(Sq, Sk, dtype=torch.bool, device=DEV).triu(1), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse[..., None])
    del s
    o = torch.matmul(p, vh)
    if dog is None:
        return o, lse
    dp = torch.matmul(dog, vh.t().contiguous())
    delta = (dog * o).sum(-1, keepdim=True)
    ds = p * (dp - delta)
    del dp
    dq = torch.matmul(ds, kh) * scale
    dk = torch.matmul(ds.transpose(1, 2).contiguous(), qg).sum(0) * scale
    dv = torch.matmul(p.transpose(1, 2).contiguous(), dog).sum(0)
    return o, lse, dq, dk, dv


def _rel(got, want):
    return float((got.float() - want).abs().max() / want.abs().max())


def test_config3_forward_backward_full_size():
    """bf16 causal GQA B=2 Hq=16 Hkv=4 S=8192 D=128, fwd + bwd."""
    B, Hq, Hkv, S, D = 2, 16, 4, 8192, 128
    g = Hq // Hkv
    gen = torch.Generator(device=DEV).manual_seed(0)
    q, k, v, do = _randn(gen, B, Hq, S, D), _randn(gen, B, Hkv, S, D), _randn(gen, B, Hkv, S, D), \
        _randn(gen, B, Hq, S, D)
    note("scale cfg3 fwd+bwd")
    tq, tk, tv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = flash_attention(tq, tk, tv, causal=True)
    out.backward(do)
    _, lse = flash_attention_with_lse(q, k, v, causal=True)
    torch.cuda.synchronize()
    scale = 1.0 / D ** 0.5
    worst = {"o": 0.0, "lse": 0.0, "dq": 0.0, "dk": 0.0, "dv": 0.0}
    for b in range(B):
        for h in range(Hkv):
            sl = slice(h * g, (h + 1) * g)
            o_r, lse_r, dq_r, dk_r, dv_r = _attn_group(
                q[b, sl].float(), k[b, h].float(), v[b, h].float(), scale, True, do[b, sl].float())
            worst["o"] = max(worst["o"], float((out[b, sl].float() - o_r).abs().max()))
            worst["lse"] = max(worst["lse"], float((lse[b, sl] - lse_r).abs().max()))
            worst["dq"] = max(worst["dq"], _rel(tq.grad[b, sl], dq_r))
            worst["dk"] = max(worst["dk"], _rel(tk.grad[b, h], dk_r))
            worst["dv"] = max(worst["dv"], _rel(tv.grad[b, h], dv_r))
            del o_r, lse_r, dq_r, dk_r, dv_r
    note(f"scale cfg3 worst {worst}")
    assert worst["o"] <= 2e-2
    assert worst["lse"] <= 1e-3
    for name in ("dq", "dk", "dv"):
        assert worst[name] <= 5e-2, (name, worst[name])


def test_config2_fused_rope_full_size():
    """flash_attention_rope bf16 causal B=4 Hq=32 Hkv=8 S=4096,
    tables from precompute_rope(4096, 128, 1e4)."""
    B, Hq, Hkv, S, D = 4, 32, 8, 4096, 128
    g = Hq // Hkv
    gen = torch.Generator(device=DEV).manual_seed(1)
    q, k, v = _randn(gen, B, Hq, S, D), _randn(gen, B, Hkv, S, D), _randn(gen, B, Hkv, S, D)
    cos, sin = precompute_rope(S, D, 10000.0, device=DEV)
    note("scale cfg2 rope")
    out = flash_attention_rope(q, k, v, cos, sin, causal=True)
    torch.cuda.synchronize()

    def rot(x):  # fused_rope.py:43-50 in float32
        x = x.float()
        half = D // 2
        return x * cos + torch.cat([-x[..., half:], x[..., :half]], dim=-1) * sin

    worst, worst_rounded = 0.0, 0.0
    for b in range(B):
        for h in range(Hkv):
            sl = slice(h * g, (h + 1) * g)
            qr, kr = rot(q[b, sl]), rot(k[b, h])
            o_r, _ = _attn_group(qr, kr, v[b, h].float(), 1.0 / D ** 0.5, True)
            worst = max(worst, float((out[b, sl].float() - o_r).abs().max()))
            # the kernel's own rounding of the rotated q and k to bf16
            o_b, _ = _attn_group(qr.bfloat16().float(), kr.bfloat16().float(), v[b, h].float(),
                                 1.0 / D ** 0.5, True)
            worst_rounded = max(worst_rounded, float((out[b, sl].float() - o_b).abs().max()))
            del o_r, o_b
    note(f"scale cfg2 worst {worst:.3e} (vs a reference with the rotated q, k rounded to bf16: "
         f"{worst_rounded:.3e})")
    # Measured 9.02e-3 against the float32 rotation of fused_rope.py:75-78
    # (deterministic inputs and kernel); the bar keeps a third of headroom
    # for reordered arithmetic, under the north star's 2e-2.
    assert worst <= 1.2e-2


def test_config4_decode_full_size():
    """decode bf16 B=64 Hq=32 Hkv=8, cache 8192, kv_len 6000,
    slots past 6000 NaN (never read: a finite tail gives bitwise the same)."""
    B, Hq, Hkv, cap, L, D = 64, 32, 8, 8192, 6000, 128
    g = Hq // Hkv
    gen = torch.Generator(device=DEV).manual_seed(2)
    q = _randn(gen, B, Hq, 1, D)
    kc, vc = _randn(gen, B, Hkv, cap, D), _randn(gen, B, Hkv, cap, D)
    kn, vn = kc.clone(), vc.clone()
    kn[:, :, L:] = float("nan")
    vn[:, :, L:] = float("nan")
    note("scale cfg4 decode")
    out = flash_attention_decode(q, kn, vn, L)
    out_finite = flash_attention_decode(q, kc, vc, L)
    torch.cuda.synchronize()
    assert torch.equal(out, out_finite)
    qf = q[:, :, 0].float().view(B, Hkv, g, D)
    s = torch.matmul(qf, kc[:, :, :L].float().transpose(2, 3).contiguous()) / D ** 0.5
    o_r = torch.matmul(torch.softmax(s, dim=-1), vc[:, :, :L].float()).view(B, Hq, 1, D)
    err = float((out.float() - o_r).abs().max())
    note(f"scale cfg4 err {err:.3e}")
    assert err <= 2e-2


def test_config5_paged_full_size():
    """paged decode bf16, 128 sequences, Hq=32 Hkv=8, page 64,
    lengths U[512, 8192] (numpy default_rng(0)), 16384-page pool dealt out by a
    seeded permutation, -1-padded [128, 128] table; unreferenced pages and the
    tail past each length NaN (bitwise the same as finite)."""
    B, Hq, Hkv, D, page, npages, pps = 128, 32, 8, 128, 64, 16384, 128
    g = Hq // Hkv
    rng = np.random.default_rng(0)
    lens = rng.integers(512, 8193, B)
    perm = rng.permutation(npages)
    table = np.full((B, pps), -1, np.int32)
    cur = 0
    for b in range(B):
        n = -(-int(lens[b]) // page)
        table[b, :n] = perm[cur:cur + n]
        cur += n
    gen = torch.Generator(device=DEV).manual_seed(3)
    q = _randn(gen, B, Hq, 1, D)
    kp, vp = _randn(gen, npages, Hkv, page, D), _randn(gen, npages, Hkv, page, D)
    tt = torch.as_tensor(table, device=DEV)
    tl = torch.as_tensor(lens.astype(np.int32), device=DEV)
    note("scale cfg5 paged")
    out_finite = paged_flash_attention(q, kp, vp, tt, tl)
    used = torch.zeros(npages, dtype=torch.bool, device=DEV)
    used[torch.as_tensor(perm[:cur], device=DEV)] = True
    kn, vn = kp.clone(), vp.clone()
    kn[~used] = float("nan")
    vn[~used] = float("nan")
    for b in range(B):
        n = -(-int(lens[b]) // page)
        tail = int(lens[b]) - (n - 1) * page
        kn[int(table[b, n - 1]), :, tail:] = float("nan")
        vn[int(table[b, n - 1]), :, tail:] = float("nan")
    out = paged_flash_attention(q, kn, vn, tt, tl)
    torch.cuda.synchronize()
    assert torch.equal(out, out_finite)
    worst = 0.0
    for b in range(B):
        L = int(lens[b])
        n = -(-L // page)
        pages = torch.as_tensor(table[b, :n].astype(np.int64), device=DEV)
        kb = kp[pages].permute(1, 0, 2, 3).reshape(Hkv, n * page, D)[:, :L].float()
        vb = vp[pages].permute(1, 0, 2, 3).reshape(Hkv, n * page, D)[:, :L].float()
        qb = q[b, :, 0].float().view(Hkv, g, D)
        s = torch.matmul(qb, kb.transpose(1, 2).contiguous()) / D ** 0.5
        o_r = torch.matmul(torch.softmax(s, dim=-1), vb).reshape(Hq, D)
        worst = max(worst, float((out[b, :, 0].float() - o_r).abs().max()))
    note(f"scale cfg5 worst {worst:.3e}")
    assert worst <= 2e-2
