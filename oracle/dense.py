"""DiT dense differential self-attention, restated in NumPy (oracle; test infrastructure only).

Two cast profiles are provided:

* `dense_xla`   -- the reference's XLA chain, the parity contract: sa3jax/dit.py:185-200 (split, heads),
  122-128 (k RMSNorm), 150-176 (q RMSNorm, RoPE, V-mask), 131-147 (SDPA x2 and the subtraction),
  113-119 (SDPA), 45-57 (RMSNorm), 82-98 (RoPE tables and rotate-half), 101-110 (head split/merge).
* `dense_fused` -- the cast points of the reference's fused TPU kernel, sa3jax/dense_attention.py:43-94
  (fp32 scores, unnormalised exp, bf16 P and V, fp32 subtraction, one cast).

Generalisations beyond the reference (each reduces to it at the default): a per-head `lam` multiplies the
second branch (lam = 1 is the reference); `half` follows from `inv_freq.shape[0]` (the reference uses 16 of
a 64-dim head, config.py:67-70); head_dim 128 is allowed (the XLA chain is general in D, dit.py:113-119).

Arrays are float32 holding values of the compute dtype ('bf16' / 'fp16' values are exactly representable in that
type). The compute dtype follows the reference's presets (sa3jax/dtypes.py:40-58): 'bf16', 'fp16' or 'fp32'.
"""
from __future__ import annotations

import math

import numpy as np

from oracle.bf16 import cast

F32 = np.float32


def rope_tables(length: int, inv_freq: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """`(L, 2*half)` cos/sin: angles = fp32(arange(L)) * fp32(inv_freq), duplicated (dit.py:82-87).

    The angle is the fp32 product, as in the reference; cos/sin of that fp32 angle are evaluated in float64
    and rounded once to float32 (XLA's own cos/sin are within a few ulp of this)."""
    angles = np.arange(length, dtype=F32)[:, None] * np.asarray(inv_freq, dtype=F32)[None, :]
    freqs = np.concatenate([angles, angles], axis=-1).astype(np.float64)
    return np.cos(freqs).astype(F32), np.sin(freqs).astype(F32)


def rms(x: np.ndarray, weight: np.ndarray, eps: float, compute: str) -> np.ndarray:
    """RMSNorm over the last axis with an fp32 island, cast back to the compute dtype (dit.py:45-57)."""
    x32 = np.asarray(x, dtype=F32)
    mean_sq = np.mean(x32.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(F32)
    inv = (F32(1.0) / np.sqrt(mean_sq + F32(eps))).astype(F32)
    return cast(x32 * inv * np.asarray(weight, dtype=F32), compute)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, compute: str) -> np.ndarray:
    """Half-half rotate_half RoPE on the first `cos.shape[-1]` dims, fp32, cast back (dit.py:90-98)."""
    x32 = np.asarray(x, dtype=F32)
    rot_dim = cos.shape[-1]
    if rot_dim == 0:
        return cast(x32, compute)
    rot, rest = x32[..., :rot_dim], x32[..., rot_dim:]
    rotated = np.concatenate([-rot[..., rot_dim // 2:], rot[..., : rot_dim // 2]], axis=-1)
    return cast(np.concatenate([rot * cos + rotated * sin, rest], axis=-1), compute)


def heads(x: np.ndarray, num_heads: int, head_dim: int) -> np.ndarray:
    """`b n (h d) -> b h n d` (dit.py:101-104)."""
    b, n, _ = x.shape
    return x.reshape(b, n, num_heads, head_dim).transpose(0, 2, 1, 3)


def merge(x: np.ndarray) -> np.ndarray:
    """`b h n d -> b n (h d)` (dit.py:107-110)."""
    b, h, n, d = x.shape
    return x.transpose(0, 2, 1, 3).reshape(b, n, h * d)


def softmax(x: np.ndarray) -> np.ndarray:
    """fp32 softmax over the last axis: exp(x - max) / sum (jax.nn.softmax, called at dit.py:118)."""
    x = np.asarray(x, dtype=F32)
    e = np.exp(x - x.max(axis=-1, keepdims=True)).astype(F32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float64).astype(F32)).astype(F32)


def sdpa(q: np.ndarray, k: np.ndarray, v: np.ndarray, compute: str, accum=np.float64) -> np.ndarray:
    """One head's `softmax(q k^T / sqrt(D)) v` with the XLA path's cast points (dit.py:113-119):
    logits in the compute dtype, scale applied to them, fp32 softmax, weights cast to the compute dtype,
    P @ V accumulated and cast. `q` (Lq, D), `k`/`v` (Lk, D). `accum` is the matmul accumulation dtype
    (float64 for checking; float32, as XLA:CPU accumulates, for the timed CPU baseline)."""
    d = q.shape[-1]
    logits = cast(q.astype(accum) @ k.astype(accum).T, compute)
    logits = cast(logits * cast(np.array(1.0 / math.sqrt(d), dtype=F32), compute), compute)
    weights = cast(softmax(logits), compute)
    return cast(weights.astype(accum) @ v.astype(accum), compute)


def prepare(qkv: np.ndarray, q_weight, k_weight, inv_freq, valid, num_heads: int, head_dim: int,
            eps: float, compute: str):
    """Split, RMSNorm, RoPE and V-mask exactly as the XLA chain does (dit.py:196-200, 122-128, 167-175).
    Returns `(q, k, v, q_diff, k_diff)`, each `(B, H, L, D)` float32 holding compute-dtype values."""
    x = cast(qkv, compute)
    b, length, width = x.shape
    if width != 5 * num_heads * head_dim:
        raise ValueError(f"qkv width {width} != 5 * {num_heads} * {head_dim}")
    q, k, v, qd, kd = (heads(t, num_heads, head_dim) for t in np.split(x, 5, axis=-1))
    k, kd = rms(k, k_weight, eps, compute), rms(kd, k_weight, eps, compute)
    q, qd = rms(q, q_weight, eps, compute), rms(qd, q_weight, eps, compute)
    cos, sin = rope_tables(length, inv_freq)
    q, k, qd, kd = (rope(t, cos, sin, compute) for t in (q, k, qd, kd))
    if valid is not None:
        mask = cast(np.asarray(valid, dtype=F32), compute)[:, None, :, None]
        v = cast(v * mask, compute)
    return q, k, v, qd, kd


def _lam(lam, num_heads: int) -> np.ndarray:
    return np.ones(num_heads, F32) if lam is None else np.asarray(lam, dtype=F32).reshape(num_heads)


def dense_xla(qkv: np.ndarray, q_weight: np.ndarray, k_weight: np.ndarray, inv_freq: np.ndarray,
              valid: np.ndarray | None, num_heads: int, head_dim: int, eps: float = 1e-6,
              lam: np.ndarray | None = None, compute: str = "bf16", accum=np.float64,
              heads_subset: list | None = None, query_rows: np.ndarray | None = None) -> np.ndarray:
    """`(B, L, 5*H*D)` -> `(B, L, H*D)`: the XLA chain of dit._self_attention (dit.py:185-200).

    `heads_subset` (a list of (batch, head) pairs) restricts the attention to those heads (the others stay 0);
    the timed CPU baseline uses it to run a bounded sample of the work. `query_rows` (indices into L) restricts
    it to those queries against all keys (the other rows stay 0), so long sequences can be checked row by row
    without the whole `(L, L)` score matrix.

    `out = SDPA(q, k, v) - lam * SDPA(q_diff, k_diff, v)` (dit.py:144-146; lam = 1 in the reference), with
    the subtraction's result cast once to the compute dtype. Heads are processed one at a time so the
    `(L, L)` scores stay small."""
    q, k, v, qd, kd = prepare(qkv, q_weight, k_weight, inv_freq, valid, num_heads, head_dim, eps, compute)
    lam = _lam(lam, num_heads)
    b = qkv.shape[0]
    out = np.zeros(q.shape, F32)
    pairs = heads_subset if heads_subset is not None else [(bi, h) for bi in range(b) for h in range(num_heads)]
    rows = slice(None) if query_rows is None else np.asarray(query_rows)
    for bi, h in pairs:
        first = sdpa(q[bi, h][rows], k[bi, h], v[bi, h], compute, accum)
        second = sdpa(qd[bi, h][rows], kd[bi, h], v[bi, h], compute, accum)
        out[bi, h][rows] = cast(first - lam[h] * second, compute)
    return merge(out)


def fused_attend(qq: np.ndarray, kk: np.ndarray, vv: np.ndarray) -> np.ndarray:
    """One branch of the fused kernel's `attend` (dense_attention.py:79-83) for bf16 `qq` (scaled queries), `kk`
    and `vv`: fp32 logits, `w = exp(l - max)` in fp32, `bf16(w) @ V` accumulated in fp32, divided by the fp32 row
    sum of the unrounded `w`."""
    logits = (qq.astype(np.float64) @ kk.astype(np.float64).T).astype(F32)
    w = np.exp(logits - logits.max(-1, keepdims=True)).astype(F32)
    return ((cast(w, "bf16").astype(np.float64) @ vv.astype(np.float64))
            / w.sum(-1, keepdims=True, dtype=np.float64)).astype(F32)


def dense_fused(qkv: np.ndarray, q_weight: np.ndarray, k_weight: np.ndarray, inv_freq: np.ndarray,
                valid: np.ndarray | None, num_heads: int, head_dim: int, eps: float = 1e-6,
                lam: np.ndarray | None = None, compute: str = "bf16") -> np.ndarray:
    """The fused TPU kernel's cast points (dense_attention.py:61-94): RMSNorm and RoPE cast to the compute dtype
    (62-69), then K, K_diff and masked V rounded to bf16 whatever the compute dtype (75-77), q * scale rounded to
    bf16 (87-90); fp32 scores, unnormalised exp, `bf16(P) @ V` over the fp32 row sum (`fused_attend`); the fp32
    subtraction cast once to the compute dtype (94)."""
    q, k, v, qd, kd = prepare(qkv, q_weight, k_weight, inv_freq, valid, num_heads, head_dim, eps, compute)
    lam = _lam(lam, num_heads)
    scale = F32(1.0 / math.sqrt(head_dim))
    k, kd, v = cast(k, "bf16"), cast(kd, "bf16"), cast(v, "bf16")
    q, qd = cast(q * scale, "bf16"), cast(qd * scale, "bf16")
    out = np.empty(q.shape, F32)
    for bi in range(qkv.shape[0]):
        for h in range(num_heads):
            out[bi, h] = cast(fused_attend(q[bi, h], k[bi, h], v[bi, h])
                              - lam[h] * fused_attend(qd[bi, h], kd[bi, h], v[bi, h]), compute)
    return merge(out)


def tables(length: int, inv_freq: np.ndarray, valid: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Per-clip tables in the kernel-native layout: `(L, half)` fp32 cos and sin of the fp32 angles
    (the reference's lane tables, dense_attention.py:97-101, hold the same values spread over lanes) and a
    `(B, L)` float32 V-mask."""
    half = np.asarray(inv_freq).shape[0]
    cos, sin = rope_tables(length, inv_freq)
    return cos[:, :half].copy(), sin[:, :half].copy(), np.asarray(valid, dtype=F32)
