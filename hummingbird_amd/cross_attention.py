"""DiT differential cross-attention on MI355X: the `attention="hip"` counterpart of the reference's XLA chain
`dit._cross_attention` (sa3jax/dit.py:203-215) and its hoisted context K/V `dit._cross_kv` (dit.py:274-284).

`prepare_cross_kv` does once per clip what `_cross_kv` does: split the context's `to_kv` output into k, k_diff
and v and RMS-norm k and k_diff (dit.py:278-281, 122-128). Its result holds them on the device in the dense
kernels' layout. `cross_attention` then does what `_cross_attention` does up to `to_out`, for one block and
sampler step: split the `to_q` output into q and q_diff, RMS-norm them (dit.py:166-168), and subtract the two
softmax attentions over the context (dit.py:131-147). There is no RoPE and no mask (dit.py:204-205). Both run
through the C ABI (`hb_cross_prep`, `hb_cross_attend`) on torch's current stream.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from hummingbird_amd import _lib
from hummingbird_amd.dense_attention import SUPPORTED_HEAD_DIMS, _f32, _require_gpu, _row_stride, dtype_code


@dataclass(frozen=True)
class CrossKV:
    """The prepared context of one block: k, k_diff (normed) and v in the kernel-native layout."""
    workspace: torch.Tensor  # uint8, hb_cross_workspace_size bytes
    k_weight: torch.Tensor   # (D,) fp32: bounds the logits in the attention kernel
    dtype: torch.dtype
    batch: int
    length: int              # Nk context tokens
    num_heads: int
    head_dim: int


def workspace_bytes(dtype: torch.dtype, batch: int, length: int, num_heads: int, head_dim: int) -> int:
    """Bytes of device memory `prepare_cross_kv` fills for a context of `length` tokens."""
    return int(_lib.load().hb_cross_workspace_size(dtype_code(dtype), batch, length, num_heads, head_dim))


def _check_head_dim(head_dim: int) -> None:
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"cross_attention needs head_dim in {SUPPORTED_HEAD_DIMS} (head_dim={head_dim})")


def prepare_cross_kv(kv: torch.Tensor, k_weight: torch.Tensor, num_heads: int, head_dim: int, eps: float, *,
                     workspace: torch.Tensor | None = None) -> CrossKV:
    """`(B, Nk, 3 * H * D)` context `to_kv` output -> the prepared context (reference: dit._cross_kv,
    dit.py:274-284; the reference computes it once per clip and reuses it in every sampler step).
    `k_weight` is the block's k_norm scale `(D,)`. `workspace` optionally supplies the device memory
    (`workspace_bytes(...)` bytes of uint8); it must stay alive and unmodified while the result is in use."""
    _require_gpu(kv, "kv")
    _check_head_dim(head_dim)
    if kv.dim() != 3 or kv.shape[-1] != 3 * num_heads * head_dim:
        raise ValueError(f"kv must be (B, Nk, 3*H*D) = (., ., {3 * num_heads * head_dim}), got {tuple(kv.shape)}")
    dev = kv.device
    code = dtype_code(kv.dtype)
    batch, length, _ = kv.shape
    kw = _f32(k_weight, dev).reshape(-1)
    if kw.numel() != head_dim:
        raise ValueError("k_weight must have head_dim elements")
    lib = _lib.load()
    need = int(lib.hb_cross_workspace_size(code, batch, length, num_heads, head_dim))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    elif workspace.numel() * workspace.element_size() < need or workspace.device != dev:
        raise ValueError(f"workspace must hold {need} bytes on {dev}")
    stream = torch.cuda.current_stream(dev).cuda_stream
    status = lib.hb_cross_prep(stream, kv.data_ptr(), code, _row_stride(kv), kw.data_ptr(), batch, length, num_heads,
                               head_dim, float(eps), workspace.data_ptr(), workspace.numel() * workspace.element_size())
    _lib.check(status, "prepare_cross_kv")
    return CrossKV(workspace, kw, kv.dtype, batch, length, num_heads, head_dim)


def cross_attention(q: torch.Tensor, context: CrossKV, q_weight: torch.Tensor, eps: float, *,
                    lam: torch.Tensor | None = None) -> torch.Tensor:
    """`(B, L, 2 * H * D)` block `to_q` output -> `(B, L, H * D)` differential cross-attention against a prepared
    context, in `q.dtype` (reference: dit._cross_attention, dit.py:203-215, up to `to_out`). `q_weight` is the
    block's q_norm scale `(D,)`; `lam` `(H,)` optionally weights the second branch (`A - lam * B`; default 1, the
    reference)."""
    _require_gpu(q, "q")
    heads, dim = context.num_heads, context.head_dim
    if q.dim() != 3 or q.shape[-1] != 2 * heads * dim:
        raise ValueError(f"q must be (B, L, 2*H*D) = (., ., {2 * heads * dim}), got {tuple(q.shape)}")
    if q.dtype != context.dtype:
        raise TypeError(f"q is {q.dtype} but the context was prepared as {context.dtype}")
    batch, length, _ = q.shape
    if batch != context.batch:
        raise ValueError(f"q has batch {batch}, the context {context.batch}")
    dev = q.device
    if context.workspace.device != dev:
        raise ValueError("q and the prepared context must be on the same device")
    qw = _f32(q_weight, dev).reshape(-1)
    if qw.numel() != dim:
        raise ValueError("q_weight must have head_dim elements")
    lam_p = 0
    if lam is not None:
        lam = _f32(lam, dev).reshape(-1)
        if lam.numel() != heads:
            raise ValueError("lam must have num_heads elements")
        lam_p = lam.data_ptr()
    out = torch.empty((batch, length, heads * dim), dtype=q.dtype, device=dev)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws = context.workspace
    status = lib.hb_cross_attend(stream, q.data_ptr(), dtype_code(q.dtype), _row_stride(q), qw.data_ptr(),
                                 context.k_weight.data_ptr(), lam_p, out.data_ptr(), batch, length, context.length,
                                 heads, dim, float(eps), ws.data_ptr(), ws.numel() * ws.element_size())
    _lib.check(status, "cross_attention")
    return out
