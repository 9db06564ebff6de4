"""The DiT attention call sites with the `attention="hip"` dispatch: self-attention (sa3jax/dit.py:179-200) with
the per-clip tables it reads (sa3jax/dit.py:317-336), and cross-attention (sa3jax/dit.py:203-215) with its context
K/V hoisted out of the sampler loop (sa3jax/dit.py:274-284).

Only the attention steps of a DiT block are here: `to_qkv` -> differential self-attention -> `to_out`, and
`to_q` -> differential cross-attention against the prepared context -> `to_out`. The rest of the block (adaLN,
feed-forward) is outside this package.
"""
from __future__ import annotations

import torch

from hummingbird_amd import cross_attention as xattn
from hummingbird_amd import dense_attention, projection, xla_chain
from hummingbird_amd.config import DiTConfig
from hummingbird_amd.dtypes import Dtype


def use_hip(cfg: DiTConfig, qkv: torch.Tensor) -> bool:
    """Dispatch predicate (reference: dit._fused, dit.py:179-182): the HIP kernel when selected, the model is
    differential and the tensors live on a ROCm device. There is no token floor. Selecting "hip" for CPU
    tensors is an error rather than a silent fallback."""
    if cfg.attention != "hip" or not cfg.differential:
        return False
    if not qkv.is_cuda:
        raise ValueError('attention="hip" needs ROCm device tensors; use attention="xla" on the CPU')
    return True


def static_tables(inv_freq: torch.Tensor, valid: torch.Tensor, cfg: DiTConfig,
                  compute: torch.dtype | Dtype) -> dict[str, torch.Tensor]:
    """Per-clip tables (reference: dit._static, dit.py:317-336). `valid` is the `(B, T)` padding mask of the
    latents; the mask is extended over the memory tokens (dit.py:320). `compute` is the compute dtype or a `Dtype`
    preset."""
    if isinstance(compute, Dtype):
        compute = compute.compute
    batch = valid.shape[0]
    ones = torch.ones((batch, cfg.num_memory_tokens), dtype=torch.bool, device=valid.device)
    full = torch.cat([ones, valid.to(torch.bool)], dim=-1)
    length = full.shape[1]
    static = {"inv_freq": inv_freq, "valid": full}
    if cfg.attention == "hip":
        static["hip_cos"], static["hip_sin"], static["hip_mask"] = dense_attention.tables(
            length, inv_freq, full, cfg.head_dim, compute)
    return static


def self_attention(h: torch.Tensor, block: dict, static: dict, cfg: DiTConfig,
                   lam: torch.Tensor | None = None, dtype: Dtype | None = None,
                   projections: str = "torch") -> torch.Tensor:
    """`to_qkv` -> differential self-attention -> `to_out` (reference: dit._self_attention, dit.py:185-200).
    `block["self_attn"]` holds `to_qkv.weight (5E, E)`, `to_out.weight (E, E)`, `q_norm.weight`, `k_norm.weight`.
    `dtype` (a preset of hummingbird_amd.dtypes, as the reference's `dtype` argument) casts `h` and the projection
    weights to its compute dtype; without it they are used as given.

    `projections` picks the GEMMs around the HIP kernel: "torch" (hipBLASLt, then the kernel's own key
    preparation) or "hip" (this package's matrix-core GEMMs with the key preparation in the to_qkv epilogue, so
    `qkv` is never stored; bf16 or fp16, head_dim 64, heads a multiple of 4). Both compute the same cast points; the
    choice only affects speed."""
    attn = block["self_attn"]
    if dtype is not None:
        h = h.to(dtype.compute)
    half = cfg.rope_dim // 2
    if projections not in ("torch", "hip"):
        raise ValueError(f'projections must be "torch" or "hip", got {projections!r}')
    if (projections == "hip" and use_hip(cfg, h)
            and projection.fused_supported(h.dtype, cfg.num_heads, cfg.head_dim, h.shape[-1], half)):
        qq, ws = projection.qkv_projection(h, attn["to_qkv"]["weight"], attn["k_norm"]["weight"], static["hip_cos"],
                                           static["hip_sin"], static["hip_mask"], cfg.num_heads, cfg.head_dim, half,
                                           cfg.qk_norm_eps)
        out = projection.attend_projected(qq, attn["q_norm"]["weight"], attn["k_norm"]["weight"], static["hip_cos"],
                                          static["hip_sin"], cfg.num_heads, cfg.head_dim, half, cfg.qk_norm_eps, ws,
                                          lam=lam)
        w_out = attn["to_out"]["weight"]
        if projection.linear_supported(out.dtype, *w_out.shape):
            return projection.linear(out, w_out)
        return out @ w_out.to(out.dtype).t()
    qkv = h @ attn["to_qkv"]["weight"].to(h.dtype).t()
    if use_hip(cfg, qkv):
        out = dense_attention.dense_attention(qkv, attn["q_norm"]["weight"], attn["k_norm"]["weight"],
                                              static["hip_cos"], static["hip_sin"], static["hip_mask"],
                                              cfg.num_heads, cfg.head_dim, cfg.rope_dim // 2, cfg.qk_norm_eps,
                                              lam=lam)
    else:
        if not cfg.differential:
            raise NotImplementedError("only the differential self-attention is on this package's path")
        out = xla_chain.dense_chain(qkv, attn["q_norm"]["weight"], attn["k_norm"]["weight"], static["inv_freq"],
                                    static["valid"], cfg.num_heads, cfg.head_dim, cfg.qk_norm_eps, lam=lam)
    return out @ attn["to_out"]["weight"].to(out.dtype).t()


def cross_context(block: dict, ctx: torch.Tensor, cfg: DiTConfig):
    """The context's K/V for one block, computed once per clip (reference: dit._cross_kv, dit.py:274-284):
    `to_kv` -> split -> k_norm on k and k_diff. With `attention="hip"` the result is a prepared
    `cross_attention.CrossKV` on the device, otherwise the `(k, k_diff, v)` tensors of the XLA chain.
    `block["cross_attn"]` holds `to_kv.weight (3E, C)`, `to_q.weight (2E, E)`, `to_out.weight (E, E)`,
    `q_norm.weight`, `k_norm.weight`."""
    attn = block["cross_attn"]
    kv = ctx @ attn["to_kv"]["weight"].t()
    if use_hip(cfg, kv):
        return xattn.prepare_cross_kv(kv, attn["k_norm"]["weight"], cfg.num_heads, cfg.head_dim, cfg.qk_norm_eps)
    if not cfg.differential:
        raise NotImplementedError("only the differential cross-attention is on this package's path")
    return xla_chain.cross_kv(kv, attn["k_norm"]["weight"], cfg.num_heads, cfg.head_dim, cfg.qk_norm_eps)


def cross_attention(h: torch.Tensor, block: dict, context, cfg: DiTConfig,
                    lam: torch.Tensor | None = None) -> torch.Tensor:
    """`to_q` -> differential cross-attention -> `to_out` (reference: dit._cross_attention, dit.py:203-215)
    against `cross_context(...)` of the same block."""
    attn = block["cross_attn"]
    q = h @ attn["to_q"]["weight"].t()
    if use_hip(cfg, q):
        if not isinstance(context, xattn.CrossKV):
            raise TypeError('attention="hip" needs the context prepared by cross_context with attention="hip"')
        out = xattn.cross_attention(q, context, attn["q_norm"]["weight"], cfg.qk_norm_eps, lam=lam)
    else:
        if not cfg.differential:
            raise NotImplementedError("only the differential cross-attention is on this package's path")
        out = xla_chain.cross_chain(q, context, attn["q_norm"]["weight"], cfg.num_heads, cfg.head_dim,
                                    cfg.qk_norm_eps, lam=lam)
    return out @ attn["to_out"]["weight"].t()
