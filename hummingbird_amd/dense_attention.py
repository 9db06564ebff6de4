"""DiT dense differential self-attention on MI355X: the `attention="hip"` counterpart of the reference's
`sa3jax/dense_attention.py` (same function names, argument meaning and error behaviour).

`tables` builds the per-clip inputs once (reference: dense_attention.py:97-101, called from dit.py:334-336);
`dense_attention` runs RMSNorm -> RoPE -> V-mask -> both softmax branches -> subtract on the GPU through the
C ABI (`hb_dense_diffattn`), replacing the Pallas kernel (dense_attention.py:104-153). Tensors are torch
tensors on a ROCm device; work is enqueued on torch's current stream for that device.
"""
from __future__ import annotations

import torch

from hummingbird_amd import _lib, rotary
from hummingbird_amd._lib import HB_BF16, HB_F16, HB_F32

SUPPORTED_HEAD_DIMS = (64, 128)

# The compute dtypes of the reference's presets (sa3jax/dtypes.py:40-58): BF16, FP16 and FP32_PARITY.
_DTYPE_CODES = {torch.bfloat16: HB_BF16, torch.float16: HB_F16, torch.float32: HB_F32}


def dtype_code(dtype: torch.dtype) -> int:
    """The C ABI's code for a compute dtype: bf16, fp16 (both with bf16 attention operands, as the reference's
    fused kernels) or fp32."""
    code = _DTYPE_CODES.get(dtype)
    if code is None:
        raise TypeError(f"hummingbird_amd kernels take bfloat16, float16 or float32 inputs, got {dtype}")
    return code


def _require_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a ROCm device tensor (hummingbird_amd has no CPU path)")


def _f32(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    return t.to(device=device, dtype=torch.float32).contiguous()


def _row_stride(qkv: torch.Tensor) -> int:
    """Row stride (elements) of a `(B, N, W)` tensor whose batch and sequence axes share one stride."""
    b, n, _ = qkv.shape
    s0, s1, s2 = qkv.stride()
    if s2 != 1 or (b > 1 and s0 != n * s1):
        raise ValueError("qkv must have unit stride on the feature axis and stride(0) == N * stride(1)")
    return s1


def rope_tables(length: int, inv_freq: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """`(length, half)` fp32 cos and sin of `fp32(n) * inv_freq[j]` (sa3jax/dit.py:82-87: the same values, not
    duplicated over the two rotary halves), built on the device by `hb_rope_tables`."""
    _require_gpu(inv_freq, "inv_freq")
    half = inv_freq.shape[0]
    freq = _f32(inv_freq, inv_freq.device)
    cos = torch.empty((length, half), dtype=torch.float32, device=inv_freq.device)
    sin = torch.empty_like(cos)
    lib = _lib.load()
    stream = torch.cuda.current_stream(inv_freq.device).cuda_stream
    _lib.check(lib.hb_rope_tables(stream, freq.data_ptr(), half, length, cos.data_ptr(), sin.data_ptr()),
               "rope_tables")
    return cos, sin


def tables(length: int, inv_freq: torch.Tensor, valid: torch.Tensor, head_dim: int,
           compute: torch.dtype) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per-clip inputs (reference: dense_attention.py:97-101): RoPE cos/sin `(L, half)` fp32 and the V-mask
    `(B, L)` fp32. The reference returns lane tables `(L, 128)` and a lane mask `(B, L, 128)`; the tables are
    opaque to the caller, so the kernel-native layout is returned instead. `head_dim` and `compute` are kept
    for signature compatibility (the mask is 0/1 and exact in every dtype)."""
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"dense_attention needs head_dim in {SUPPORTED_HEAD_DIMS} (head_dim={head_dim})")
    cos, sin = rope_tables(length, inv_freq)
    mask = valid.to(device=inv_freq.device, dtype=torch.float32).reshape(valid.shape[0], length).contiguous()
    return cos, sin, mask


def workspace_bytes(dtype: torch.dtype, batch: int, length: int, num_heads: int, head_dim: int) -> int:
    """Bytes of scratch `dense_attention` needs (prepared k, k_diff and v in the kernel-native layout)."""
    return int(_lib.load().hb_dense_workspace_size(dtype_code(dtype), batch, length, num_heads, head_dim))


def dense_attention(qkv: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor, mask: torch.Tensor | None, num_heads: int, head_dim: int, half: int,
                    eps: float, *, rows: int | None = None, stack: bool = True, interpret: bool = False,
                    lam: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """`(B, L, 5 * H * D)` DiT `to_qkv` output -> `(B, L, H * D)` differential self-attention, in `qkv.dtype`.

    Same contract as the reference (sa3jax/dense_attention.py:104-114): `q_weight`/`k_weight` are the q/k RMSNorm
    scales `(D,)`, `cos`/`sin`/`mask` come from `tables`, `half` is the rotate-half width. `rows`, `stack` and
    `interpret` are the TPU kernel's tiling knobs and are accepted and ignored (the HIP tiling is fixed).
    `lam` `(H,)` optionally weights the second branch (`A - lam * B`; default 1, the reference).
    `workspace` optionally supplies the scratch (`workspace_bytes(...)` bytes of uint8 on the same device).
    Any `half` in `[0, head_dim / 2]` is taken; one that is not a multiple of 8 runs on a copy of `qkv` with the q
    and k dims reordered (`hummingbird_amd.rotary`). Raises ValueError for unsupported shapes, like the reference
    does at trace time.
    """
    del rows, stack, interpret
    _require_gpu(qkv, "qkv")
    if qkv.dim() != 3:
        raise ValueError(f"qkv must be (B, L, 5*H*D), got shape {tuple(qkv.shape)}")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"dense_attention needs head_dim in {SUPPORTED_HEAD_DIMS} (head_dim={head_dim})")
    batch, length, width = qkv.shape
    if width != 5 * num_heads * head_dim:
        raise ValueError(f"qkv width {width} != 5 * num_heads * head_dim = {5 * num_heads * head_dim}")
    if not 0 <= half <= head_dim // 2:
        raise ValueError(f"half {half} outside [0, head_dim/2]")
    dev = qkv.device
    code = dtype_code(qkv.dtype)
    rs = _row_stride(qkv)
    qw, kw = _f32(q_weight, dev).reshape(-1), _f32(k_weight, dev).reshape(-1)
    if qw.numel() != head_dim or kw.numel() != head_dim:
        raise ValueError("q_weight and k_weight must have head_dim elements")
    cos_p = sin_p = 0
    if half > 0:
        cos, sin = _f32(cos, dev), _f32(sin, dev)
        if tuple(cos.shape) != (length, half) or tuple(sin.shape) != (length, half):
            raise ValueError(f"cos/sin must be (L, half) = ({length}, {half}) from tables(), got {tuple(cos.shape)}")
        cos_p, sin_p = cos.data_ptr(), sin.data_ptr()
    if half % rotary.ALIGN:  # the kernels pair 8-dim groups: reorder the q and k dims (see rotary)
        qkv = rotary.reorder_sections(qkv, num_heads, head_dim, half, (True, True, False, True, True))
        rs = qkv.shape[-1]
        qw, kw = rotary.reorder_dims(qw, head_dim, half), rotary.reorder_dims(kw, head_dim, half)
        cos, sin = rotary.pad_tables(cos, sin, half)
        cos_p, sin_p = cos.data_ptr(), sin.data_ptr()
        half = rotary.aligned_half(half)
    mask_p = 0
    if mask is not None:
        mask = _f32(mask, dev)
        if mask.numel() != batch * length:
            raise ValueError(f"mask must be (B, L) = ({batch}, {length}) from tables(), got {tuple(mask.shape)}")
        mask_p = mask.data_ptr()
    lam_p = 0
    if lam is not None:
        lam = _f32(lam, dev).reshape(-1)
        if lam.numel() != num_heads:
            raise ValueError("lam must have num_heads elements")
        lam_p = lam.data_ptr()
    lib = _lib.load()
    need = int(lib.hb_dense_workspace_size(code, batch, length, num_heads, head_dim))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    elif workspace.numel() * workspace.element_size() < need or workspace.device != dev:
        raise ValueError(f"workspace must hold {need} bytes on {dev}")
    out = torch.empty((batch, length, num_heads * head_dim), dtype=qkv.dtype, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    status = lib.hb_dense_diffattn(stream, qkv.data_ptr(), code, rs, qw.data_ptr(), kw.data_ptr(), cos_p, sin_p, half,
                                   mask_p, lam_p, out.data_ptr(), batch, length, num_heads, head_dim, float(eps),
                                   workspace.data_ptr(), workspace.numel() * workspace.element_size())
    _lib.check(status, "dense_attention")
    return out
