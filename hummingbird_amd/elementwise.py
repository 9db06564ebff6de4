"""The elementwise steps of a SAME-L decoder block on MI355X (`hb_dyt`, `hb_glu`): the `attention="hip"`
counterparts of `same_l._dyt` followed by the block's cast to the compute dtype (sa3jax/same_l.py:58-69,
191-192) and of the GLU gate of `same_l._feed_forward` (sa3jax/same_l.py:172-183). Tensors are torch tensors on a
ROCm device; work is enqueued on torch's current stream.
"""
from __future__ import annotations

import torch

from hummingbird_amd import _lib
from hummingbird_amd.band_attention import pack_dyt
from hummingbird_amd.dense_attention import _require_gpu, dtype_code


def _rows(t: torch.Tensor, name: str) -> tuple[int, int]:
    """(rows, row stride in elements) of a tensor whose leading axes flatten onto equally spaced rows: contiguous,
    or a column slice of a wider contiguous tensor."""
    if t.dim() < 1 or t.stride(-1) != 1:
        raise ValueError(f"{name} must have unit stride on its last axis")
    rows = t.numel() // t.shape[-1]
    if t.dim() == 1:
        return 1, t.shape[-1]
    stride = t.stride(-2)
    step = stride
    for size, st in zip(reversed(t.shape[:-1]), reversed(t.stride()[:-1])):
        if size > 1 and st != step:
            raise ValueError(f"{name}'s leading axes must flatten onto rows of one stride")
        step *= size
    return rows, stride


def dyt(x: torch.Tensor, norm: dict) -> torch.Tensor:
    """`cast(gamma * tanh(alpha * x) + beta)` over the last axis, computed in fp32 and returned in `x.dtype`
    (reference: same_l._dyt + `.astype(dtype.compute)`, same_l.py:58-69, 191-192). `norm` holds the DyT params
    `{alpha: scalar, gamma: (C,), beta: (C,)}`."""
    _require_gpu(x, "x")
    channels = x.shape[-1]
    params = pack_dyt(norm, channels, x.device)
    rows, stride = _rows(x, "x")
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(_lib.load().hb_dyt(stream, x.data_ptr(), dtype_code(x.dtype), stride, params.data_ptr(), out.data_ptr(),
                                  channels, rows, channels), "dyt")
    return out


def glu(proj: torch.Tensor, sinusoidal: bool, bias: torch.Tensor | None = None) -> torch.Tensor:
    """`value * act(gate)` for `[value | gate]` = the two halves of the last axis of the glu_proj output
    (reference: same_l._feed_forward, same_l.py:172-183); act = SiLU, or sin(pi * gate) when `sinusoidal`.
    `bias` (2F), if given, is the glu_proj layer's bias and `proj` the bare matmul: the bias is added in the
    compute dtype first (same_l._linear), in the same pass."""
    _require_gpu(proj, "proj")
    width = proj.shape[-1]
    if width % 2:
        raise ValueError(f"the glu_proj output width {width} is not even")
    inner = width // 2
    rows, stride = _rows(proj, "proj")
    bias_p = 0
    if bias is not None:
        bias = bias.to(device=proj.device, dtype=torch.float32).contiguous().reshape(-1)
        if bias.numel() != width:
            raise ValueError(f"bias must have {width} elements")
        bias_p = bias.data_ptr()
    out = torch.empty((*proj.shape[:-1], inner), dtype=proj.dtype, device=proj.device)
    stream = torch.cuda.current_stream(proj.device).cuda_stream
    _lib.check(_lib.load().hb_glu(stream, proj.data_ptr(), dtype_code(proj.dtype), stride, bias_p,
                                  int(bool(sinusoidal)), out.data_ptr(), inner, rows, inner), "glu")
    return out
