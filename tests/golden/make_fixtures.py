"""Generate the golden fixtures in this directory from the float64 oracle.

    python tests/golden/make_fixtures.py

The reference ships no golden vectors (its tests compare kernels against
jnp on jax.random inputs) and jax is not installed, so these fixtures hold
inputs drawn from np.random.default_rng and the expected outputs of this
repository's pinned oracle (oracle/attention.py; see tests/test_oracle.py for
how each function is pinned). Inputs are rounded to bfloat16-representable
float32 values so the same fixture drives the float32 and bfloat16 kernels
with identical inputs. Expected outputs are stored as float32 (6e-8 relative,
far below every tolerance they are checked against).
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import (attention_bwd_ref, attention_ref, decode_ref, paged_ref,  # noqa: E402
                    precompute_rope_ref, rope_attention_ref)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float64 values to the nearest bfloat16 (ties to even), as float32."""
    f = np.asarray(x, np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def build() -> dict:
    rng = np.random.default_rng(20240601)
    n = lambda *s: bf16_round(rng.standard_normal(s))
    fx = {}
    # forward: GQA, Sq != Sk, causal, kv_len < Sk (flash_attention.py:61-159)
    q, k, v = n(1, 4, 70, 128), n(1, 2, 90, 128), n(1, 2, 90, 128)
    o, lse = attention_ref(q, k, v, causal=True, kv_len=83)
    fx.update(fwd_q=q, fwd_k=k, fwd_v=v, fwd_o=o, fwd_lse=lse)
    # backward: MQA, causal, ragged (flash_attention.py:354-442)
    q, k, v, do = n(1, 2, 72, 128), n(1, 1, 72, 128), n(1, 1, 72, 128), n(1, 2, 72, 128)
    dq, dk, dv = attention_bwd_ref(q, k, v, do, causal=True)
    fx.update(bwd_q=q, bwd_k=k, bwd_v=v, bwd_do=do, bwd_dq=dq, bwd_dk=dk, bwd_dv=dv)
    # decode: cache prefix (flash_attention.py:555-589)
    q, kc, vc = n(2, 8, 1, 128), n(2, 2, 160, 128), n(2, 2, 160, 128)
    fx.update(dec_q=q, dec_k=kc, dec_v=vc, dec_len=np.int32(131), dec_o=decode_ref(q, kc, vc, 131))
    # paged: scrambled table with -1 padding, zero-length sequence (paged.py:45-192)
    q, kp, vp = n(3, 4, 1, 128), n(12, 2, 16, 128), n(12, 2, 16, 128)
    table = np.array([[7, 2, 9, -1, -1], [0, 11, 3, 5, 8], [4, -1, -1, -1, -1]], np.int32)
    lens = np.array([40, 80, 0], np.int32)
    fx.update(pg_q=q, pg_k=kp, pg_v=vp, pg_table=table, pg_lens=lens,
              pg_o=paged_ref(q, kp, vp, table, lens))
    # fused RoPE: tables from precompute_rope (fused_rope.py:53-113; model.py:41-51)
    q, k, v = n(1, 4, 66, 128), n(1, 2, 66, 128), n(1, 2, 66, 128)
    cos, sin = precompute_rope_ref(66, 128, 10000.0)
    cos, sin = cos.astype(np.float32), sin.astype(np.float32)
    fx.update(rope_q=q, rope_k=k, rope_v=v, rope_cos=cos, rope_sin=sin,
              rope_o=rope_attention_ref(q, k, v, cos, sin, causal=True))
    return fx


if __name__ == "__main__":
    out = os.path.join(HERE, "fixtures.npz")
    fx = {k: (v.astype(np.float32) if v.dtype == np.float64 else v) for k, v in build().items()}
    np.savez_compressed(out, **fx)
    print(f"wrote {out} ({os.path.getsize(out) / 1024:.0f} KiB)")
