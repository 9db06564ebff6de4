"""Rotary half-widths that are not a multiple of 8.

The reference's rotate-half RoPE (sa3jax/dit.py:90-98, sa3jax/same_l.py:92-100) rotates dim d with dim d + half
for d < half and leaves dims 2 half .. D - 1 alone, for any half. The HIP kernels hold a head's dims in 16-byte
groups of 8 and pair group m with group m + half / 8, so the C ABI takes half % 8 == 0. For another half the
wrappers run the kernels on the same heads with their q and k dims reordered:

  - kernel position d (d < half) holds dim d and position ha + d holds dim half + d, where ha = half rounded up to
    a multiple of 8; the unrotated dims fill the other positions in order;
  - the kernels then rotate with half-width ha; the RoPE tables get ha - half more columns of angle 0 (cos 1,
    sin 0), which leave the unrotated dims that land in those pairs unchanged (x cos - y sin = x exactly);
  - the per-dim norm parameters (RMSNorm gains, DyT gamma and beta) are reordered the same way.

A dot product does not depend on the order of the dims, so the logits, the softmax and the output (v and out are
not reordered) are those of the reference's layout; only the fp32 summation order of each logit differs. The
reordering costs one copy of `qkv` per call.
"""
from __future__ import annotations

import functools

import torch

ALIGN = 8  # dims per 16-byte group of bf16


def aligned_half(half: int) -> int:
    """`half` rounded up to a multiple of 8: the kernels' rotary half-width for a reordered head."""
    return -(-half // ALIGN) * ALIGN


def head_order(head_dim: int, half: int) -> list[int]:
    """`order[p]`: the dim of the reference's head layout that kernel position p holds (see the module comment)."""
    ha = aligned_half(half)
    if 2 * ha > head_dim:
        raise ValueError(f"half {half} rounded up to {ha} exceeds head_dim / 2 = {head_dim // 2}")
    order = [-1] * head_dim
    for d in range(half):
        order[d] = d
        order[ha + d] = half + d
    rest = iter(range(2 * half, head_dim))
    for p in range(head_dim):
        if order[p] < 0:
            order[p] = next(rest)
    return order


@functools.lru_cache(maxsize=64)
def _columns(num_heads: int, head_dim: int, half: int, sections: tuple[bool, ...], device: torch.device
             ) -> torch.Tensor:
    order = torch.tensor(head_order(head_dim, half), dtype=torch.long)
    ident = torch.arange(head_dim, dtype=torch.long)
    cols = []
    for s, reorder in enumerate(sections):
        for h in range(num_heads):
            cols.append((s * num_heads + h) * head_dim + (order if reorder else ident))
    return torch.cat(cols).to(device)


def reorder_sections(x: torch.Tensor, num_heads: int, head_dim: int, half: int,
                     sections: tuple[bool, ...]) -> torch.Tensor:
    """A contiguous copy of `x` `(..., len(sections) * H * D)` with the heads of the sections marked True in the
    kernels' order (`head_order`) and the others as they are."""
    cols = _columns(num_heads, head_dim, half, tuple(sections), x.device)
    return x.index_select(-1, cols)


def reorder_dims(v: torch.Tensor, head_dim: int, half: int) -> torch.Tensor:
    """A per-dim parameter `(D,)` in the kernels' order."""
    order = torch.tensor(head_order(head_dim, half), dtype=torch.long, device=v.device)
    return v.reshape(-1).index_select(0, order)


def pad_tables(cos: torch.Tensor, sin: torch.Tensor, half: int) -> tuple[torch.Tensor, torch.Tensor]:
    """`(N, half)` RoPE tables widened to `(N, aligned_half(half))` with angle-0 columns (cos 1, sin 0)."""
    extra = aligned_half(half) - half
    n = cos.shape[0]
    ones = torch.ones((n, extra), dtype=cos.dtype, device=cos.device)
    zeros = torch.zeros((n, extra), dtype=sin.dtype, device=sin.device)
    return torch.cat([cos, ones], dim=1).contiguous(), torch.cat([sin, zeros], dim=1).contiguous()
