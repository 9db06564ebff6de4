"""The elementwise steps of a SAME-L decoder block (`hb_dyt`, `hb_glu`) and of a DiT block (`hb_rms_modulate`,
`hb_gated_residual`) on MI355X: the `attention="hip"` counterparts of `same_l._dyt` followed by the block's cast to
the compute dtype (sa3jax/same_l.py:58-69, 191-192), of the GLU gate of `same_l._feed_forward`
(sa3jax/same_l.py:172-183; the DiT's SwiGLU, sa3jax/dit.py:218-221, is the same gate), and of the DiT block's
norms, adaLN modulations and residuals (sa3jax/dit.py:224-251). Tensors are torch tensors on a ROCm device; work
is enqueued on torch's current stream.
"""
from __future__ import annotations

import torch

from hummingbird_amd import _lib
from hummingbird_amd._derived import f32_vector
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
        bias = f32_vector(bias, proj.device)
        if bias.numel() != width:
            raise ValueError(f"bias must have {width} elements")
        bias_p = bias.data_ptr()
    out = torch.empty((*proj.shape[:-1], inner), dtype=proj.dtype, device=proj.device)
    stream = torch.cuda.current_stream(proj.device).cuda_stream
    _lib.check(_lib.load().hb_glu(stream, proj.data_ptr(), dtype_code(proj.dtype), stride, bias_p,
                                  int(bool(sinusoidal)), out.data_ptr(), inner, rows, inner), "glu")
    return out


def residual_dyt(h: torch.Tensor, x: torch.Tensor, bias: torch.Tensor | None = None,
                 norm: dict | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """`(h + (x + bias), cast(DyT(h + (x + bias))))` in one pass: a residual add of the SAME-L block (reference:
    same_l._block, same_l.py:191-192) after the projection's bias add (same_l._linear), each sum held in the compute
    dtype, and with `norm` (DyT params) the DyT of the sum cast back, the next GEMM's input. `x` is the bare
    projection output; `bias` (C values) may be None. Without `norm` the second result is None."""
    _require_gpu(h, "h")
    if h.shape != x.shape or h.dtype != x.dtype:
        raise ValueError(f"h {tuple(h.shape)} {h.dtype} and x {tuple(x.shape)} {x.dtype} must match")
    channels = h.shape[-1]
    rows, hs = _rows(h, "h")
    _, xs = _rows(x, "x")
    bias_p = 0
    if bias is not None:
        bias = f32_vector(bias, h.device)
        if bias.numel() != channels:
            raise ValueError(f"bias must have {channels} elements")
        bias_p = bias.data_ptr()
    params = pack_dyt(norm, channels, h.device) if norm is not None else None
    out_h = torch.empty(h.shape, dtype=h.dtype, device=h.device)
    out_y = torch.empty(h.shape, dtype=h.dtype, device=h.device) if norm is not None else None
    stream = torch.cuda.current_stream(h.device).cuda_stream
    _lib.check(_lib.load().hb_residual_dyt(stream, h.data_ptr(), dtype_code(h.dtype), hs, x.data_ptr(), xs, bias_p,
                                           params.data_ptr() if params is not None else 0, out_h.data_ptr(),
                                           out_y.data_ptr() if out_y is not None else 0, channels, rows, channels),
               "residual_dyt")
    return out_h, out_y


def _per_batch(t: torch.Tensor | None, batch: int, channels: int, dtype: torch.dtype, name: str):
    """(pointer, batch stride) of a `(B, C)` (or `(B, 1, C)`) per-batch row tensor in `dtype`, possibly a view into a
    wider row (the adaLN chunks of `(B, 6 E)`); (0, 0) for None."""
    if t is None:
        return 0, 0
    if t.dtype != dtype:
        raise TypeError(f"{name} is {t.dtype}, expected {dtype}")
    t2 = t.reshape(t.shape[0], t.shape[-1]) if t.dim() == 3 and t.shape[1] == 1 else t
    if t2.dim() != 2 or tuple(t2.shape) != (batch, channels) or t2.stride(-1) != 1:
        raise ValueError(f"{name} must be (B, C) = ({batch}, {channels}) with unit stride on C, got {tuple(t.shape)}")
    return t2.data_ptr(), (t2.stride(0) if batch > 1 else channels)


def rms_modulate(x: torch.Tensor, weight: torch.Tensor, eps: float, scale: torch.Tensor | None = None,
                 shift: torch.Tensor | None = None) -> torch.Tensor:
    """The DiT block norm on `(B, L, C)`: `cast(x * rsqrt(mean(x^2) + eps) * weight)` with an fp32 island
    (sa3jax/dit.py:44-57), then with `scale` / `shift` `(B, C)` the adaLN modulation `* (1 + scale) + shift`
    (sa3jax/dit.py:231-233, 246-247), each step in `x.dtype`. One pass (`hb_rms_modulate`)."""
    _require_gpu(x, "x")
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, C), got {tuple(x.shape)}")
    batch, length, channels = x.shape
    rows, stride = _rows(x, "x")
    w = weight.to(device=x.device, dtype=torch.float32).contiguous().reshape(-1)
    if w.numel() != channels:
        raise ValueError(f"weight must have {channels} elements")
    if (scale is None) != (shift is None):
        raise ValueError("scale and shift are given together or not at all")
    sp, ms = _per_batch(scale, batch, channels, x.dtype, "scale")
    hp, ms2 = _per_batch(shift, batch, channels, x.dtype, "shift")
    if scale is not None and ms != ms2:
        raise ValueError("scale and shift must share their batch stride")
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(_lib.load().hb_rms_modulate(stream, x.data_ptr(), dtype_code(x.dtype), stride, w.data_ptr(), float(eps),
                                           sp, hp, ms, length, out.data_ptr(), channels, rows, channels),
               "rms_modulate")
    return out


def gated_residual(h: torch.Tensor, x: torch.Tensor, gate: torch.Tensor | None = None,
                   x_bias: torch.Tensor | None = None, local: torch.Tensor | None = None,
                   memory: int = 0) -> torch.Tensor:
    """`h + (x + x_bias) * sigmoid(1 - gate)` on `(B, L, C)` (sa3jax/dit.py:234, 249-251), or `h + x` without
    `gate`, then `+ local` on the tokens at or past `memory` (sa3jax/dit.py:237-241); each step in `h.dtype`.
    `gate` is `(B, C)`, `x_bias` and `local` `(C,)`. One pass (`hb_gated_residual`)."""
    _require_gpu(h, "h")
    if h.dim() != 3 or x.shape != h.shape or x.dtype != h.dtype:
        raise ValueError(f"h and x must be (B, L, C) of one shape and dtype, got {tuple(h.shape)}, {tuple(x.shape)}")
    batch, length, channels = h.shape
    _, hs = _rows(h, "h")
    rows, xs = _rows(x, "x")
    gp, gs = _per_batch(gate, batch, channels, h.dtype, "gate")

    def vec(t, name):
        if t is None:
            return 0
        if t.dtype != h.dtype or t.numel() != channels or t.stride(-1) != 1:
            raise ValueError(f"{name} must be ({channels},) of {h.dtype} with unit stride")
        return t.data_ptr()
    out = torch.empty(h.shape, dtype=h.dtype, device=h.device)
    stream = torch.cuda.current_stream(h.device).cuda_stream
    _lib.check(_lib.load().hb_gated_residual(stream, h.data_ptr(), dtype_code(h.dtype), hs, x.data_ptr(), xs,
                                             vec(x_bias, "x_bias"), gp, gs, vec(local, "local"), int(memory), length,
                                             out.data_ptr(), channels, rows, channels), "gated_residual")
    return out


def residual_rms(h: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, eps: float,
                 gate: torch.Tensor | None = None, x_bias: torch.Tensor | None = None,
                 local: torch.Tensor | None = None, memory: int = 0, scale: torch.Tensor | None = None,
                 shift: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """`gated_residual(h, x, gate, x_bias, local, memory)` and then `rms_modulate` of its result with `weight`, `eps`,
    `scale`, `shift`, in one pass per row (`hb_residual_rms`; rows of at most 2048 values):
    returns `(h', norm(h'))`, the same values as the two calls. A DiT block's residuals each feed the next norm
    (sa3jax/dit.py:234-236, 237-247, 249-251 into the next block's 231-233)."""
    _require_gpu(h, "h")
    if h.dim() != 3 or x.shape != h.shape or x.dtype != h.dtype:
        raise ValueError(f"h and x must be (B, L, C) of one shape and dtype, got {tuple(h.shape)}, {tuple(x.shape)}")
    batch, length, channels = h.shape
    _, hs = _rows(h, "h")
    rows, xs = _rows(x, "x")
    gp, gs = _per_batch(gate, batch, channels, h.dtype, "gate")
    if (scale is None) != (shift is None):
        raise ValueError("scale and shift are given together or not at all")
    sp, ms = _per_batch(scale, batch, channels, h.dtype, "scale")
    hp, ms2 = _per_batch(shift, batch, channels, h.dtype, "shift")
    if scale is not None and ms != ms2:
        raise ValueError("scale and shift must share their batch stride")
    w = weight.to(device=h.device, dtype=torch.float32).contiguous().reshape(-1)
    if w.numel() != channels:
        raise ValueError(f"weight must have {channels} elements")

    def vec(t, name):
        if t is None:
            return 0
        if t.dtype != h.dtype or t.numel() != channels or t.stride(-1) != 1:
            raise ValueError(f"{name} must be ({channels},) of {h.dtype} with unit stride")
        return t.data_ptr()
    out_h = torch.empty(h.shape, dtype=h.dtype, device=h.device)
    out_y = torch.empty(h.shape, dtype=h.dtype, device=h.device)
    stream = torch.cuda.current_stream(h.device).cuda_stream
    _lib.check(_lib.load().hb_residual_rms(stream, h.data_ptr(), dtype_code(h.dtype), hs, x.data_ptr(), xs,
                                           vec(x_bias, "x_bias"), gp, gs, vec(local, "local"), int(memory),
                                           w.data_ptr(), float(eps), sp, hp, ms, length, out_h.data_ptr(),
                                           out_y.data_ptr(), channels, rows, channels), "residual_rms")
    return out_h, out_y


def residual_rms_supported(dtype: torch.dtype, channels: int) -> bool:
    """Whether `residual_rms` takes rows of `channels` values of `dtype` (held in registers)."""
    return channels <= 2048 and channels % (8 if dtype in (torch.bfloat16, torch.float16) else 4) == 0
