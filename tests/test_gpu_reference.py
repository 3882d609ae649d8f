"""GPU tier: ``pallas_flash.reference_attention``, the materialising torch
baseline (reference.py:22-66), against the float64 oracle.

Its arithmetic follows reference.py:55-66: the score product in the input
dtype (bf16 scores are rounded to bf16), then float32 softmax and a float32
product with V. Float32 inputs must match the oracle to the north-star fp32
bar; bf16 inputs are compared with an oracle that rounds the scores the same
way, and with the unrounded oracle and the fused kernel at the bf16 bar.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import check_fwd, dev, host, max_abs, note, qkv
from oracle import attention_ref
from pallas_flash import flash_attention, reference_attention

pytestmark = pytest.mark.gpu


def _oracle_rounded_scores(q, k, v, causal, scale):
    """float64 attention whose q k^T is rounded to bf16 before scaling
    (reference.py:55 on bf16 inputs), GQA by head repetition (:49-53)."""
    g = q.shape[1] // k.shape[1]
    k = np.repeat(k, g, axis=1)
    v = np.repeat(v, g, axis=1)
    s = np.einsum("bhqd,bhkd->bhqk", q, k)
    s = torch.as_tensor(s.astype(np.float32)).to(torch.bfloat16).double().numpy() * scale
    if causal:
        Sq, Sk = s.shape[-2:]
        s = np.where(np.arange(Sq)[:, None] >= np.arange(Sk)[None, :], s, -1e30)
    s = s - s.max(axis=-1, keepdims=True)
    w = np.exp(s)
    w /= w.sum(axis=-1, keepdims=True)
    return w @ v


@pytest.mark.parametrize("Hq,Hkv,Sq,Sk,causal", [(4, 4, 128, 128, False), (8, 2, 200, 200, True),
                                                 (4, 1, 96, 160, True), (2, 2, 64, 300, False)])
def test_reference_attention_f32(Hq, Hkv, Sq, Sk, causal):
    note(f"reference_attention f32 Hq={Hq} Hkv={Hkv} Sq={Sq} Sk={Sk} causal={causal}")
    q, k, v = qkv(np.random.default_rng(40), 2, Hq, Hkv, Sq, Sk)
    tq, tk, tv = dev(q, "f32"), dev(k, "f32"), dev(v, "f32")
    out = reference_attention(tq, tk, tv, causal=causal)
    assert out.dtype == torch.float32 and out.shape == tq.shape
    ref, _ = attention_ref(q, k, v, causal=causal)
    check_fwd(host(out), ref, "f32")


@pytest.mark.parametrize("Hq,Hkv,causal", [(4, 2, True), (4, 4, False)])
def test_reference_attention_bf16_scores_in_input_dtype(Hq, Hkv, causal):
    note(f"reference_attention bf16 Hq={Hq} Hkv={Hkv} causal={causal}")
    q, k, v = qkv(np.random.default_rng(41), 1, Hq, Hkv, 256, 256)
    tq, tk, tv = dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16")
    out = reference_attention(tq, tk, tv, causal=causal)
    assert out.dtype == torch.bfloat16
    qh, kh, vh = host(tq), host(tk), host(tv)
    rounded = _oracle_rounded_scores(qh, kh, vh, causal, 1.0 / np.sqrt(128))
    plain, _ = attention_ref(qh, kh, vh, causal=causal)
    o = host(out)
    m_rounded, m_plain = float(np.abs(o - rounded).mean()), float(np.abs(o - plain).mean())
    note(f"reference_attention bf16: mean abs error vs rounded-score oracle {m_rounded:.3e}, "
         f"vs float64 oracle {m_plain:.3e}")
    # the bf16 score rounding is visible: the rounded-score oracle is closer
    assert m_rounded < m_plain
    check_fwd(o, rounded, "bf16")
    check_fwd(o, plain, "bf16")
    fused = flash_attention(tq, tk, tv, causal=causal)
    assert max_abs(host(fused), host(out)) <= 2e-2
