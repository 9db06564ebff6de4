"""The SAME-L attention call site with the `attention="hip"` dispatch (sa3jax/same_l.py:151-169).

Only the attention step of a decoder block is here: `to_qkv` -> differential band attention -> `to_out`.
"""
from __future__ import annotations

import torch

from hummingbird_amd import band_attention, xla_chain
from hummingbird_amd.config import SameConfig


def use_hip(cfg: SameConfig, qkv: torch.Tensor) -> bool:
    """Dispatch predicate (reference: same_l.py:158): the HIP kernel when selected on ROCm device tensors."""
    if cfg.attention != "hip":
        return False
    if not qkv.is_cuda:
        raise ValueError('attention="hip" needs ROCm device tensors; use attention="xla" on the CPU')
    return True


def attention(x: torch.Tensor, block: dict, cfg: SameConfig, lam: torch.Tensor | None = None) -> torch.Tensor:
    """`to_qkv` -> differential band attention at half-width `sub_chunk_size` -> `to_out` (reference:
    same_l._attention, same_l.py:151-169). `block` holds `self_attn.{to_qkv,to_out}.weight`,
    `self_attn.{q_norm,k_norm}` DyT params and `rope_inv_freq`."""
    attn = block["self_attn"]
    qkv = x @ attn["to_qkv"]["weight"].t()
    if use_hip(cfg, qkv):
        out = band_attention.band_attention(qkv, attn["q_norm"], attn["k_norm"], block["rope_inv_freq"],
                                            cfg.num_heads, cfg.dim_heads, cfg.sub_chunk_size, lam=lam)
    else:
        out = xla_chain.band_chain(qkv, attn["q_norm"], attn["k_norm"], block["rope_inv_freq"], cfg.num_heads,
                                   cfg.dim_heads, cfg.sub_chunk_size, lam=lam)
    return out @ attn["to_out"]["weight"].t()
