"""SAME-L sliding-window (band) differential attention, restated in NumPy (oracle; test infrastructure only).

* `band_xla`     -- the reference's XLA chain, the parity contract: sa3jax/same_l.py:151-169 (split, DyT, RoPE,
  two SDPAs, fp32 subtraction, one cast), 58-69 (DyT, fp32 island), 84-100 (RoPE, kept fp32),
  134-148 (SDPA: fp32 logits scaled, -inf outside the band, fp32 softmax, fp32 P @ V).
  The band is `|k - q| <= w` with `0 <= k < S` (same_l.py:14-16, 103-115; band_attention.py:108-110).
* `band_grouped` -- the reference's own grouped form (same_l.py:103-148: query groups of `w`, three
  consecutive KV groups, the `(groups, w, 3w)` mask), which needs `S % w == 0`; used to pin `band_xla`.
* `band_fused`   -- the fused TPU kernel's cast points (band_attention.py:61-120): q*scale and k rounded to bf16
  after DyT/RoPE, fp32 scores with -1e30 outside the band, unnormalised exp, bf16 P and V, fp32 subtraction.

Generalisations beyond the reference (each reduces to it at the default): per-head `lam` on the second branch
(lam = 1 is the reference); a general half-width `w` and any `S` (the reference hard-wires w = 17 and S = 17 T,
same_l.py:140, 160); head_dim 128.
"""
from __future__ import annotations

import math

import numpy as np

from oracle.bf16 import cast
from oracle.dense import heads, merge, rope, rope_tables

F32 = np.float32


def dyt(x: np.ndarray, alpha, gamma: np.ndarray, beta: np.ndarray) -> np.ndarray:
    """`gamma * tanh(alpha * x) + beta` in fp32, returned in fp32 (same_l.py:58-69)."""
    x32 = np.asarray(x, dtype=F32)
    a = F32(np.asarray(alpha, dtype=F32).reshape(()))
    return (np.asarray(gamma, F32) * np.tanh(a * x32).astype(F32) + np.asarray(beta, F32)).astype(F32)


def prepare(qkv: np.ndarray, q_norm: dict, k_norm: dict, inv_freq: np.ndarray, num_heads: int, head_dim: int,
            compute: str):
    """Split into heads, DyT and RoPE as the XLA chain does (same_l.py:162-167). q/k stay fp32 (DyT returns
    fp32 and `_rope` casts back to that dtype); v keeps the compute dtype."""
    x = cast(qkv, compute)
    b, length, width = x.shape
    if width != 5 * num_heads * head_dim:
        raise ValueError(f"qkv width {width} != 5 * {num_heads} * {head_dim}")
    q, k, v, qd, kd = (heads(t, num_heads, head_dim) for t in np.split(x, 5, axis=-1))
    cos, sin = rope_tables(length, inv_freq)
    qn = (q_norm["alpha"], q_norm["gamma"], q_norm["beta"])
    kn = (k_norm["alpha"], k_norm["gamma"], k_norm["beta"])
    q = rope(dyt(q, *qn), cos, sin, "fp32")
    k = rope(dyt(k, *kn), cos, sin, "fp32")
    qd = rope(dyt(qd, *qn), cos, sin, "fp32")
    kd = rope(dyt(kd, *kn), cos, sin, "fp32")
    return q, k, v, qd, kd


def band_sdpa(q: np.ndarray, k: np.ndarray, v: np.ndarray, window: int, block: int = 512,
              accum=np.float64) -> np.ndarray:
    """One head's band attention in fp32: softmax over keys `|k - q| <= window`, `0 <= k < S`, of the
    fp32 logits `q k^T / sqrt(D)`, then fp32 P @ V (same_l.py:134-148). Processed in query blocks so only
    `block x (block + 2 window)` logits exist at a time. `q`/`k`/`v` are `(S, D)`; `accum` is the matmul
    accumulation dtype (float64 for checking, float32 for the timed CPU baseline)."""
    s, d = q.shape
    scale = F32(1.0 / math.sqrt(d))
    out = np.empty((s, d), F32)
    for q0 in range(0, s, block):
        q1 = min(s, q0 + block)
        k0, k1 = max(0, q0 - window), min(s, q1 + window)
        logits = ((q[q0:q1].astype(accum) @ k[k0:k1].astype(accum).T).astype(F32) * scale).astype(F32)
        qpos = np.arange(q0, q1)[:, None]
        kpos = np.arange(k0, k1)[None, :]
        logits = np.where(np.abs(kpos - qpos) <= window, logits, -np.inf)
        e = np.exp(logits - logits.max(-1, keepdims=True)).astype(F32)
        w = (e / e.sum(-1, keepdims=True, dtype=np.float64).astype(F32)).astype(F32)
        out[q0:q1] = (w.astype(accum) @ v[k0:k1].astype(accum)).astype(F32)
    return out


def _lam(lam, num_heads: int) -> np.ndarray:
    return np.ones(num_heads, F32) if lam is None else np.asarray(lam, dtype=F32).reshape(num_heads)


def band_xla(qkv: np.ndarray, q_norm: dict, k_norm: dict, inv_freq: np.ndarray, num_heads: int, head_dim: int,
             window: int, lam: np.ndarray | None = None, compute: str = "bf16", accum=np.float64) -> np.ndarray:
    """`(B, S, 5*H*D)` -> `(B, S, H*D)`: `SDPA(q,k,v) - lam * SDPA(q_d,k_d,v)` in fp32, cast once
    (same_l.py:168-169)."""
    if window < 0:
        raise ValueError("window must be >= 0")
    q, k, v, qd, kd = prepare(qkv, q_norm, k_norm, inv_freq, num_heads, head_dim, compute)
    lam = _lam(lam, num_heads)
    out = np.empty(q.shape, F32)
    for bi in range(qkv.shape[0]):
        for h in range(num_heads):
            first = band_sdpa(q[bi, h], k[bi, h], v[bi, h], window, accum=accum)
            second = band_sdpa(qd[bi, h], kd[bi, h], v[bi, h], window, accum=accum)
            out[bi, h] = cast(first - lam[h] * second, compute)
    return merge(out)


def swa_mask(groups: int, stride: int) -> np.ndarray:
    """The static `(groups, stride, 3*stride)` band of the grouped form (same_l.py:103-115): query `q` of
    group `g` is position `stride*g + q`; slot `w` is position `stride*g + w - stride`."""
    q = np.arange(stride)[None, :, None]
    w = np.arange(3 * stride)[None, None, :]
    pos = np.arange(groups)[:, None, None] * stride + w - stride
    return (w >= q) & (w <= q + 2 * stride) & (pos >= 0) & (pos < groups * stride)


def windows(t: np.ndarray, groups: int, stride: int) -> np.ndarray:
    """`(S, D) -> (groups, 3*stride, D)`: each query group's three consecutive KV groups, zero-padded by one
    group on each side (same_l.py:118-131)."""
    s, d = t.shape
    padded = np.pad(t, ((stride, stride), (0, 0)))
    parts = [padded[off: off + s].reshape(groups, stride, d) for off in (0, stride, 2 * stride)]
    return np.concatenate(parts, axis=1)


def band_grouped_sdpa(q: np.ndarray, k: np.ndarray, v: np.ndarray, window: int) -> np.ndarray:
    """The reference's grouped band SDPA for one head (same_l.py:134-148) with `stride = window`; needs
    `S % window == 0` and `window >= 1`."""
    s, d = q.shape
    if window < 1 or s % window:
        raise ValueError("grouped form needs window >= 1 and S % window == 0")
    groups = s // window
    mask = swa_mask(groups, window)
    qg = q.reshape(groups, window, d).astype(np.float64)
    kw, vw = windows(k, groups, window).astype(np.float64), windows(v, groups, window).astype(np.float64)
    logits = (np.einsum("gqd,gwd->gqw", qg, kw).astype(F32) * F32(1.0 / math.sqrt(d))).astype(F32)
    logits = np.where(mask, logits, -np.inf)
    e = np.exp(logits - logits.max(-1, keepdims=True)).astype(F32)
    w = (e / e.sum(-1, keepdims=True, dtype=np.float64).astype(F32)).astype(F32)
    return np.einsum("gqw,gwd->gqd", w.astype(np.float64), vw).astype(F32).reshape(s, d)


def fused_band_attend(qq: np.ndarray, kk: np.ndarray, vv: np.ndarray, window: int, block: int = 512) -> np.ndarray:
    """One branch of the fused kernel's `attend` (band_attention.py:96-101) for one head of bf16 `qq` (scaled
    queries), `kk` and `vv`, all `(S, D)`: fp32 logits, -1e30 outside `|k - q| <= window` (and `0 <= k < S`),
    `w = exp(l - max)` in fp32, `bf16(w) @ V` accumulated in fp32 over the fp32 row sum of the unrounded `w`."""
    s = qq.shape[0]
    res = np.empty(qq.shape, F32)
    for q0 in range(0, s, block):
        q1 = min(s, q0 + block)
        k0, k1 = max(0, q0 - window), min(s, q1 + window)
        logits = (qq[q0:q1].astype(np.float64) @ kk[k0:k1].astype(np.float64).T).astype(F32)
        band = np.abs(np.arange(k0, k1)[None, :] - np.arange(q0, q1)[:, None]) <= window
        logits = np.where(band, logits, F32(-1e30))
        e = np.exp(logits - logits.max(-1, keepdims=True)).astype(F32)
        res[q0:q1] = ((cast(e, "bf16").astype(np.float64) @ vv[k0:k1].astype(np.float64))
                      / e.sum(-1, keepdims=True, dtype=np.float64)).astype(F32)
    return res


def band_fused(qkv: np.ndarray, q_norm: dict, k_norm: dict, inv_freq: np.ndarray, num_heads: int, head_dim: int,
               window: int, lam: np.ndarray | None = None, compute: str = "bf16") -> np.ndarray:
    """The fused TPU kernel's cast points (band_attention.py:82-120): q*scale and k rounded to bf16 after DyT and
    RoPE in fp32 (85, 104), v rounded to bf16 (94), fp32 scores masked with -1e30, `exp(l - max)`,
    `bf16(P) @ V / sum` (`fused_band_attend`), fp32 subtraction cast once to the compute dtype (120)."""
    q, k, v, qd, kd = prepare(qkv, q_norm, k_norm, inv_freq, num_heads, head_dim, compute)
    lam = _lam(lam, num_heads)
    scale = F32(1.0 / math.sqrt(head_dim))
    q, qd = cast(q * scale, "bf16"), cast(qd * scale, "bf16")
    k, kd, v = cast(k, "bf16"), cast(kd, "bf16"), cast(v, "bf16")
    out = np.empty(q.shape, F32)
    for bi in range(qkv.shape[0]):
        for h in range(num_heads):
            out[bi, h] = cast(fused_band_attend(q[bi, h], k[bi, h], v[bi, h], window)
                              - lam[h] * fused_band_attend(qd[bi, h], kd[bi, h], v[bi, h], window), compute)
    return merge(out)
