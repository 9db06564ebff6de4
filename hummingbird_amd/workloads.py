"""Synthetic inputs for the two attention workloads, drawn with NumPy's PCG64 (`default_rng(seed)`) in a fixed
order so every consumer (tests, benchmark, smoke check) sees identical values.

Dense (DiT self-attention): qkv ~ N(0,1) `(B, L, 5*H*D)`; q/k RMSNorm gains ~ 1 + N(0, 0.02) `(D,)`; rotary
half-width `half` (default D/2) with inv_freq_i = 10000^(-2i/(2*half)); per-head lambda ~ U(0.2, 0.8); a value
mask of ones with the last `mask_tail` tokens of every row zeroed (or a ragged tail of 0-25 % per row).
Band (SAME-L): qkv ~ N(0,1) `(B, S, 5*H*D)`; DyT alpha = 0.5, gamma ~ 1 + N(0, 0.02), beta ~ N(0, 0.02) for q and
for k; the same RoPE and lambda recipe.
Cross (DiT cross-attention): the block's to_q output ~ N(0,1) `(B, L, 2*H*D)`, the context's to_kv output
~ N(0,1) `(B, Nk, 3*H*D)`, q/k RMSNorm gains and lambda as for dense.
Draw order: qkv (cross: q, then kv), q-gain (or q DyT), k-gain (or k DyT), lambda, mask.
"""
from __future__ import annotations

import numpy as np

# The measured configurations (sizes from the workload definitions the benchmark reports against).
DENSE_120S = dict(batch=2, length=2584, heads=24, head_dim=64)      # DiT at a 120 s clip, CFG batch 2
BAND_120S = dict(batch=1, length=82688, heads=8, head_dim=64, window=128)  # SAME-L decoder at 120 s
CROSS_120S = dict(batch=2, length=2584, context=257, heads=24, head_dim=64)  # DiT cross-attention, 257 tokens
DENSE_CALLS_PER_CLIP = 192  # 8 sampler steps x 24 DiT blocks (the cross-attention calls as many times)
BAND_CALLS_PER_CLIP = 12    # 12 SAME-L decoder blocks


def inv_freq(half: int, base: float = 10000.0) -> np.ndarray:
    """RotaryEmbedding's inverse frequencies for a `2*half`-dim rotary part: base^(-2i/(2*half))."""
    if half == 0:
        return np.zeros(0, np.float32)
    return (1.0 / base ** (np.arange(0, 2 * half, 2, dtype=np.float64) / (2 * half))).astype(np.float32)


def _bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even), returned as float32."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


def _as(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values of the input dtype: 'bf16' and 'fp16' round to nearest even, 'fp32' keeps them."""
    if dtype == "bf16":
        return _bf16(x)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float32)
    return x


def dense_inputs(batch: int, length: int, heads: int, head_dim: int, seed: int = 0, dtype: str = "bf16",
                 half: int | None = None, mask_tail: int = 16, ragged: bool = False, gain_std: float = 0.02,
                 gain_mean: float = 1.0) -> dict:
    """Dense workload inputs as float32 NumPy arrays (qkv holds values of `dtype`: 'bf16', 'fp16' or 'fp32')."""
    rng = np.random.default_rng(seed)
    half = head_dim // 2 if half is None else half
    qkv = _as(rng.standard_normal((batch, length, 5 * heads * head_dim), dtype=np.float32), dtype)
    q_weight = (gain_mean + gain_std * rng.standard_normal(head_dim)).astype(np.float32)
    k_weight = (gain_mean + gain_std * rng.standard_normal(head_dim)).astype(np.float32)
    lam = rng.uniform(0.2, 0.8, heads).astype(np.float32)
    valid = np.ones((batch, length), np.float32)
    if ragged:
        for b in range(batch):
            tail = int(rng.integers(0, length // 4 + 1))
            if tail:
                valid[b, length - tail:] = 0.0
    elif mask_tail:
        valid[:, max(0, length - mask_tail):] = 0.0
    return dict(qkv=qkv, q_weight=q_weight, k_weight=k_weight, inv_freq=inv_freq(half), lam=lam, valid=valid,
                heads=heads, head_dim=head_dim, half=half, eps=1e-6)


def band_inputs(batch: int, length: int, heads: int, head_dim: int, window: int, seed: int = 1,
                dtype: str = "bf16", half: int | None = None, alpha: float = 0.5, gamma_mean: float = 1.0) -> dict:
    """Band workload inputs as float32 NumPy arrays (qkv holds values of `dtype`: 'bf16', 'fp16' or 'fp32')."""
    rng = np.random.default_rng(seed)
    half = head_dim // 2 if half is None else half
    qkv = _as(rng.standard_normal((batch, length, 5 * heads * head_dim), dtype=np.float32), dtype)

    def dyt():
        gamma = (gamma_mean + 0.02 * rng.standard_normal(head_dim)).astype(np.float32)
        beta = (0.02 * rng.standard_normal(head_dim)).astype(np.float32)
        return {"alpha": np.float32(alpha), "gamma": gamma, "beta": beta}

    q_norm = dyt()
    k_norm = dyt()
    lam = rng.uniform(0.2, 0.8, heads).astype(np.float32)
    return dict(qkv=qkv, q_norm=q_norm, k_norm=k_norm, inv_freq=inv_freq(half), lam=lam, heads=heads,
                head_dim=head_dim, half=half, window=window)


def cross_inputs(batch: int, length: int, context: int, heads: int, head_dim: int, seed: int = 0,
                 dtype: str = "bf16", gain_std: float = 0.02, gain_mean: float = 1.0) -> dict:
    """Cross-attention inputs as float32 NumPy arrays (q and kv hold values of `dtype`)."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((batch, length, 2 * heads * head_dim), dtype=np.float32)
    kv = rng.standard_normal((batch, context, 3 * heads * head_dim), dtype=np.float32)
    q, kv = _as(q, dtype), _as(kv, dtype)
    q_weight = (gain_mean + gain_std * rng.standard_normal(head_dim)).astype(np.float32)
    k_weight = (gain_mean + gain_std * rng.standard_normal(head_dim)).astype(np.float32)
    lam = rng.uniform(0.2, 0.8, heads).astype(np.float32)
    return dict(q=q, kv=kv, q_weight=q_weight, k_weight=k_weight, lam=lam, heads=heads, head_dim=head_dim,
                eps=1e-6)


def cross_flops(batch: int, length: int, context: int, heads: int, head_dim: int) -> float:
    """Algorithmic FLOPs of one cross-attention call: 2 branches x (QK^T + PV) x 2 flops per MAC."""
    return 8.0 * batch * heads * length * context * head_dim


def dense_flops(batch: int, length: int, heads: int, head_dim: int) -> float:
    """Algorithmic FLOPs of one dense call: 2 branches x (QK^T + PV) x 2 flops per MAC = 8 B H L^2 D."""
    return 8.0 * batch * heads * length * length * head_dim


def dense_bytes(batch: int, length: int, heads: int, head_dim: int, elem: int = 2) -> float:
    """Algorithmic HBM bytes of one dense call: read qkv (5 H D per token) once, write out (H D) once."""
    return float(batch * length * 6 * heads * head_dim * elem)


def band_pairs(length: int, window: int) -> int:
    """Number of (query, key) pairs with |k - q| <= window inside [0, S)."""
    w = min(window, length - 1)
    return length * (2 * w + 1) - w * (w + 1)


def band_flops(batch: int, length: int, heads: int, head_dim: int, window: int) -> float:
    """Algorithmic FLOPs of one band call: 8 B H D x (in-band pairs)."""
    return 8.0 * batch * heads * head_dim * band_pairs(length, window)


def band_bytes(batch: int, length: int, heads: int, head_dim: int, elem: int = 2) -> float:
    """Algorithmic HBM bytes of one band call: read qkv once, write out once."""
    return float(batch * length * 6 * heads * head_dim * elem)
