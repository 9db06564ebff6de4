"""The reference's plain (non-kernel) attention chains, restated in torch for `attention="xla"`.

These run wherever torch runs and keep the reference's cast points: bf16 logits, weights and subtraction for
the DiT self- and cross-attention chains (sa3jax/dit.py:113-119, 131-176, 203-215, 274-284), fp32
DyT/RoPE/softmax/subtraction for the SAME-L chain
(sa3jax/same_l.py:58-69, 92-100, 134-169). They are what `attention="xla"` selects; the `"hip"` path never
falls back to them.
"""
from __future__ import annotations

import math

import torch

F32 = torch.float32


def rope_tables(length: int, inv_freq: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """`(L, 2*half)` cos/sin of `fp32(arange) * inv_freq`, duplicated (sa3jax/dit.py:82-87). The fp32 angle is
    evaluated in float64 and rounded once."""
    angles = torch.arange(length, dtype=F32, device=inv_freq.device)[:, None] * inv_freq.to(F32)[None, :]
    freqs = torch.cat([angles, angles], dim=-1).double()
    return torch.cos(freqs).to(F32), torch.sin(freqs).to(F32)


def rms(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm with an fp32 island, cast back (sa3jax/dit.py:45-57)."""
    x32 = x.to(F32)
    normed = x32 * torch.rsqrt(torch.mean(x32 * x32, dim=-1, keepdim=True) + eps)
    return (normed * weight.to(F32)).to(x.dtype)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """Half-half rotate_half on the first `cos.shape[-1]` dims in fp32 (sa3jax/dit.py:90-98)."""
    rot_dim = cos.shape[-1]
    x32 = x.to(F32)
    if rot_dim == 0:
        return x32.to(out_dtype)
    rot, rest = x32[..., :rot_dim], x32[..., rot_dim:]
    rotated = torch.cat([-rot[..., rot_dim // 2:], rot[..., : rot_dim // 2]], dim=-1)
    return torch.cat([rot * cos + rotated * sin, rest], dim=-1).to(out_dtype)


def heads(x: torch.Tensor, num_heads: int, head_dim: int) -> torch.Tensor:
    b, n, _ = x.shape
    return x.reshape(b, n, num_heads, head_dim).permute(0, 2, 1, 3)


def merge(x: torch.Tensor) -> torch.Tensor:
    b, h, n, d = x.shape
    return x.permute(0, 2, 1, 3).reshape(b, n, h * d)


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, dtype: torch.dtype) -> torch.Tensor:
    """One head's SDPA with the DiT chain's cast points (sa3jax/dit.py:113-119): logits formed in fp32 and
    rounded to the compute dtype (as XLA's einsum does), scaled in that dtype, fp32 softmax, weights and PV in
    the compute dtype."""
    logits = (q.to(F32) @ k.to(F32).transpose(-1, -2)).to(dtype)
    logits = (logits.to(F32) * scale).to(dtype)
    weights = torch.softmax(logits.to(F32), dim=-1).to(dtype)
    return (weights.to(F32) @ v.to(F32)).to(dtype)


def dense_chain(qkv: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor, inv_freq: torch.Tensor,
                valid: torch.Tensor | None, num_heads: int, head_dim: int, eps: float,
                lam: torch.Tensor | None = None) -> torch.Tensor:
    """The DiT XLA chain (sa3jax/dit.py:196-200 -> 150-176 -> 131-147): per head, one head at a time so the
    `(L, L)` scores stay bounded. The scores are formed in fp32 and rounded to the compute dtype, as XLA's
    einsum does."""
    dtype = qkv.dtype
    length = qkv.shape[1]
    q, k, v, qd, kd = (heads(t, num_heads, head_dim) for t in qkv.split(num_heads * head_dim, dim=-1))
    k, kd, q, qd = (rms(t, w, eps) for t, w in ((k, k_weight), (kd, k_weight), (q, q_weight), (qd, q_weight)))
    cos, sin = rope_tables(length, inv_freq)
    q, k, qd, kd = (rope(t, cos, sin, dtype) for t in (q, k, qd, kd))
    if valid is not None:
        v = v * valid.to(dtype)[:, None, :, None]
    return _subtract(q, k, v, qd, kd, head_dim, dtype, lam)


def _subtract(q, k, v, qd, kd, head_dim: int, dtype: torch.dtype, lam: torch.Tensor | None) -> torch.Tensor:
    """`SDPA(q, k, v) - lam * SDPA(q_diff, k_diff, v)` per head, cast once (sa3jax/dit.py:131-147)."""
    num_heads = q.shape[1]
    scale = torch.tensor(1.0 / math.sqrt(head_dim), dtype=dtype).item()
    lam_v = torch.ones(num_heads, dtype=F32, device=q.device) if lam is None else lam.to(F32)
    out = torch.empty_like(q)
    for b in range(q.shape[0]):
        for h in range(num_heads):
            first = sdpa(q[b, h], k[b, h], v[b, h], scale, dtype)
            second = sdpa(qd[b, h], kd[b, h], v[b, h], scale, dtype)
            out[b, h] = (first.to(F32) - lam_v[h] * second.to(F32)).to(dtype)
    return merge(out)


def cross_kv(kv: torch.Tensor, k_weight: torch.Tensor, num_heads: int, head_dim: int,
             eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The hoisted context K/V (sa3jax/dit.py:274-284): the `(B, Nk, 3*H*D)` to_kv output split into k, k_diff and
    v, heads first; k and k_diff RMS-normed (dit.py:122-128), v as is."""
    k, kd, v = (heads(t, num_heads, head_dim) for t in kv.split(num_heads * head_dim, dim=-1))
    return rms(k, k_weight, eps), rms(kd, k_weight, eps), v


def cross_chain(q_proj: torch.Tensor, context: tuple[torch.Tensor, torch.Tensor, torch.Tensor],
                q_weight: torch.Tensor, num_heads: int, head_dim: int, eps: float,
                lam: torch.Tensor | None = None) -> torch.Tensor:
    """The DiT cross-attention chain (sa3jax/dit.py:203-215 -> 150-176 -> 131-147) for a `(B, L, 2*H*D)` to_q
    output against `cross_kv(...)`: q and q_diff RMS-normed, no RoPE, no mask."""
    q, qd = (heads(t, num_heads, head_dim) for t in q_proj.split(num_heads * head_dim, dim=-1))
    q, qd = rms(q, q_weight, eps), rms(qd, q_weight, eps)
    k, kd, v = context
    return _subtract(q, k, v, qd, kd, head_dim, q_proj.dtype, lam)


def dyt(x: torch.Tensor, alpha, gamma: torch.Tensor, beta: torch.Tensor) -> torch.Tensor:
    """`gamma * tanh(alpha * x) + beta` in fp32 (sa3jax/same_l.py:58-69)."""
    a = torch.as_tensor(alpha, dtype=F32, device=x.device)
    return gamma.to(F32) * torch.tanh(a * x.to(F32)) + beta.to(F32)


def band_chain(qkv: torch.Tensor, q_norm: dict, k_norm: dict, inv_freq: torch.Tensor, num_heads: int,
               head_dim: int, window: int, lam: torch.Tensor | None = None, block: int = 1024) -> torch.Tensor:
    """The SAME-L XLA chain (sa3jax/same_l.py:162-169) generalised to any S and half-width `window`: fp32
    softmax over `|k - q| <= window`, `0 <= k < S`, fp32 P @ V, fp32 subtraction, one cast. Queries are
    processed in blocks so only `block x (block + 2 window)` logits exist at once."""
    dtype = qkv.dtype
    length = qkv.shape[1]
    q, k, v, qd, kd = (heads(t, num_heads, head_dim) for t in qkv.split(num_heads * head_dim, dim=-1))
    cos, sin = rope_tables(length, inv_freq)

    def prep(t, norm):
        return rope(dyt(t, norm["alpha"], norm["gamma"], norm["beta"]), cos, sin, F32)

    q, qd = prep(q, q_norm), prep(qd, q_norm)
    k, kd = prep(k, k_norm), prep(kd, k_norm)
    v32 = v.to(F32)
    scale = 1.0 / math.sqrt(head_dim)
    lam_v = torch.ones(num_heads, dtype=F32, device=qkv.device) if lam is None else lam.to(F32)

    def band(qq, kk, vv):
        out = torch.empty_like(qq)
        for q0 in range(0, length, block):
            q1 = min(length, q0 + block)
            k0, k1 = max(0, q0 - window), min(length, q1 + window)
            logits = (qq[..., q0:q1, :] @ kk[..., k0:k1, :].transpose(-1, -2)) * scale
            dist = (torch.arange(k0, k1, device=qq.device)[None, :] - torch.arange(q0, q1, device=qq.device)[:, None])
            logits = logits.masked_fill(dist.abs() > window, float("-inf"))
            out[..., q0:q1, :] = torch.softmax(logits, dim=-1) @ vv[..., k0:k1, :]
        return out

    diff = band(q, k, v32) - lam_v[None, :, None, None] * band(qd, kd, v32)
    return merge(diff.to(dtype))


def dyt_cast(x: torch.Tensor, norm: dict) -> torch.Tensor:
    """DyT in fp32 cast back to `x.dtype` (sa3jax/same_l.py:58-69, 191-192)."""
    return dyt(x, norm["alpha"], norm["gamma"], norm["beta"]).to(x.dtype)


def glu(proj: torch.Tensor, sinusoidal: bool) -> torch.Tensor:
    """`value * act(gate)` for the glu_proj output `[value | gate]` (sa3jax/same_l.py:172-183) with the XLA chain's
    intermediate arrays in the compute dtype: SiLU as gate * sigmoid(gate) (jax.nn.silu), sin(pi * gate) with pi
    itself in the compute dtype (a Python float times an array takes the array's dtype in JAX)."""
    value, gate = proj.chunk(2, dim=-1)
    if sinusoidal:
        act = torch.sin(torch.tensor(math.pi, dtype=proj.dtype, device=proj.device) * gate)
    else:
        act = gate * torch.sigmoid(gate)
    return value * act
