"""DiT differential cross-attention, restated in NumPy (oracle; test infrastructure only).

`cross_xla` follows the reference's XLA chain: sa3jax/dit.py:274-284 (`_cross_kv`: to_kv output split into
k, k_diff, v; k and k_diff RMS-normed with k_norm; v as is), 203-215 (`_cross_attention`: to_q output split into
q, q_diff; no RoPE, no mask), 150-176 (`_attend`: q RMSNorm with q_norm), 131-147 (`_attend_out`: SDPA x2 and the
subtraction), 113-119 (SDPA) and 45-57 (RMSNorm). It reuses the dense oracle's pieces, so the cast points are
those of the DiT chain: RMSNorm in fp32 cast to the compute dtype, logits, weights and PV in the compute dtype,
the subtraction cast once.

Generalisation beyond the reference (reduces to it at the default): a per-head `lam` multiplies the second
branch (lam = 1 is the reference).
"""
from __future__ import annotations

import numpy as np

from oracle.bf16 import cast
from oracle.dense import F32, _lam, heads, merge, rms, sdpa


def prepare_kv(kv: np.ndarray, k_weight: np.ndarray, num_heads: int, head_dim: int, eps: float, compute: str):
    """`(B, Nk, 3*H*D)` to_kv output -> `(k, k_diff, v)`, each `(B, H, Nk, D)` (dit.py:278-281, 122-128)."""
    x = cast(kv, compute)
    width = num_heads * head_dim
    if x.shape[-1] != 3 * width:
        raise ValueError(f"kv width {x.shape[-1]} != 3 * {num_heads} * {head_dim}")
    k, kd, v = (heads(t, num_heads, head_dim) for t in np.split(x, 3, axis=-1))
    return rms(k, k_weight, eps, compute), rms(kd, k_weight, eps, compute), v


def cross_xla(q_proj: np.ndarray, kv: np.ndarray, q_weight: np.ndarray, k_weight: np.ndarray, num_heads: int,
              head_dim: int, eps: float = 1e-6, lam: np.ndarray | None = None, compute: str = "bf16",
              accum=np.float64) -> np.ndarray:
    """`(B, L, 2*H*D)` to_q output and `(B, Nk, 3*H*D)` to_kv output -> `(B, L, H*D)`:
    `out = SDPA(q, k, v) - lam * SDPA(q_diff, k_diff, v)` over all Nk keys (dit.py:203-215, 131-147)."""
    x = cast(q_proj, compute)
    width = num_heads * head_dim
    if x.shape[-1] != 2 * width:
        raise ValueError(f"q width {x.shape[-1]} != 2 * {num_heads} * {head_dim}")
    q, qd = (heads(t, num_heads, head_dim) for t in np.split(x, 2, axis=-1))
    q, qd = rms(q, q_weight, eps, compute), rms(qd, q_weight, eps, compute)
    k, kd, v = prepare_kv(kv, k_weight, num_heads, head_dim, eps, compute)
    lam = _lam(lam, num_heads)
    out = np.zeros(q.shape, F32)
    for bi in range(q.shape[0]):
        for h in range(num_heads):
            first = sdpa(q[bi, h], k[bi, h], v[bi, h], compute, accum)
            second = sdpa(qd[bi, h], kd[bi, h], v[bi, h], compute, accum)
            out[bi, h] = cast(first - lam[h] * second, compute)
    return merge(out)
