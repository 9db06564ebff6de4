"""The projections around the attention kernels on MI355X. The DiT self-attention's: `to_qkv` with the dense
kernel's key preparation in its epilogue, and `to_out` (reference: sa3jax/dit.py:190 and 195, `_linear` without
bias). The SAME-L block's: `glu_proj` with the GLU in its epilogue, and `to_out` / `proj_out` with the residual add
and the next DyT in theirs (reference: sa3jax/same_l.py:161, 181-184, 191-192).

`qkv_projection` runs `hb_dit_qkv_proj`: one matrix-core GEMM `h @ W_qkv^T` that never stores `qkv`; it writes the
queries as rows `[q | q_diff]` and the prepared keys and values (RMSNorm, RoPE, value mask) into the attention
workspace. `attend_projected` runs the attention against them (`hb_dense_attend_qq`), and `linear` is `x @ W^T`
(`hb_proj`). Together they compute what `h @ W_qkv^T -> dense_attention -> @ W_o^T` computes, in the same cast points.
"""
from __future__ import annotations

import torch

from hummingbird_amd import _lib
from hummingbird_amd._derived import f32_vector
from hummingbird_amd.band_attention import pack_dyt
from hummingbird_amd.dense_attention import _f32, _require_gpu, dtype_code

FUSED_DTYPES = (torch.bfloat16, torch.float16)


def _rows(t: torch.Tensor, name: str) -> tuple[int, int]:
    """(rows, row stride) of a tensor whose leading axes flatten onto rows of one stride with unit stride inside."""
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must have unit stride on its last axis")
    rows = t.numel() // t.shape[-1]
    stride = t.stride(-2) if t.dim() > 1 else t.shape[-1]
    step = stride
    for size, st in zip(reversed(t.shape[:-1]), reversed(t.stride()[:-1])):
        if size > 1 and st != step:
            raise ValueError(f"{name}'s leading axes must flatten onto rows of one stride")
        step *= size
    return rows, stride


def fused_supported(dtype: torch.dtype, num_heads: int, head_dim: int, embed_dim: int, half: int) -> bool:
    """Whether `qkv_projection` takes this geometry (bf16 or half, head_dim 64, heads a multiple of 4, model width a
    multiple of 64, rotary half-width a multiple of 8 up to 32)."""
    return (dtype in FUSED_DTYPES and head_dim == 64 and num_heads % 4 == 0 and embed_dim % 64 == 0
            and 0 <= half <= 32 and half % 8 == 0)


def linear_supported(dtype: torch.dtype, out_features: int, in_features: int) -> bool:
    """Whether `linear` takes this product (bf16 or half, out_features a multiple of 256, in_features of 64)."""
    return dtype in FUSED_DTYPES and out_features % 256 == 0 and in_features % 64 == 0 and out_features > 0


def qkv_projection(h: torch.Tensor, w_qkv: torch.Tensor, k_weight: torch.Tensor, cos: torch.Tensor | None,
                   sin: torch.Tensor | None, mask: torch.Tensor | None, num_heads: int, head_dim: int, half: int,
                   eps: float, workspace: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """`(B, L, E)` block input -> (`qq` `(B, L, 2 H D)` = `[q | q_diff]` of `h @ W_qkv^T`, the attention workspace
    holding the prepared k, k_diff and v). `w_qkv` is the layer weight `(5 H D, E)` (out x in); `cos`, `sin`, `mask`
    come from `dense_attention.tables`. Raises ValueError for geometries outside `fused_supported`."""
    _require_gpu(h, "h")
    if h.dim() != 3:
        raise ValueError(f"h must be (B, L, E), got {tuple(h.shape)}")
    batch, length, width = h.shape
    if not fused_supported(h.dtype, num_heads, head_dim, width, half):
        raise ValueError(f"the fused projection does not take dtype {h.dtype}, H={num_heads}, D={head_dim}, E={width}, "
                         f"half={half}")
    dev = h.device
    w = w_qkv.to(device=dev, dtype=h.dtype)
    if tuple(w.shape) != (5 * num_heads * head_dim, width):
        raise ValueError(f"w_qkv must be (5*H*D, E) = ({5 * num_heads * head_dim}, {width}), got {tuple(w.shape)}")
    _, hs = _rows(h, "h")
    _, ws_ = _rows(w, "w_qkv")
    kw = _f32(k_weight, dev).reshape(-1)
    cos_p = sin_p = 0
    if half > 0:
        cos, sin = _f32(cos, dev), _f32(sin, dev)
        cos_p, sin_p = cos.data_ptr(), sin.data_ptr()
    mask_p = 0
    if mask is not None:
        mask = _f32(mask, dev)
        mask_p = mask.data_ptr()
    lib = _lib.load()
    code = dtype_code(h.dtype)
    need = int(lib.hb_dense_workspace_size(code, batch, length, num_heads, head_dim))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    elif workspace.numel() * workspace.element_size() < need or workspace.device != dev:
        raise ValueError(f"workspace must hold {need} bytes on {dev}")
    qq = torch.empty((batch, length, 2 * num_heads * head_dim), dtype=h.dtype, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(lib.hb_dit_qkv_proj(stream, h.data_ptr(), code, hs, w.data_ptr(), ws_, width, kw.data_ptr(), cos_p,
                                   sin_p, half, mask_p, qq.data_ptr(), batch, length, num_heads, head_dim, float(eps),
                                   workspace.data_ptr(), workspace.numel() * workspace.element_size()), "qkv_projection")
    return qq, workspace


def attend_projected(qq: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor, cos: torch.Tensor | None,
                     sin: torch.Tensor | None, num_heads: int, head_dim: int, half: int, eps: float,
                     workspace: torch.Tensor, lam: torch.Tensor | None = None) -> torch.Tensor:
    """The differential self-attention of `dense_attention` for queries in `qq` (from `qkv_projection`) against the
    workspace it filled: `(B, L, H D)` in `qq.dtype`."""
    _require_gpu(qq, "qq")
    batch, length, _ = qq.shape
    dev = qq.device
    _, rs = _rows(qq, "qq")
    qw, kw = _f32(q_weight, dev).reshape(-1), _f32(k_weight, dev).reshape(-1)
    cos_p = sin_p = 0
    if half > 0:
        cos, sin = _f32(cos, dev), _f32(sin, dev)
        cos_p, sin_p = cos.data_ptr(), sin.data_ptr()
    lam_p = 0
    if lam is not None:
        lam = _f32(lam, dev).reshape(-1)
        lam_p = lam.data_ptr()
    out = torch.empty((batch, length, num_heads * head_dim), dtype=qq.dtype, device=dev)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(lib.hb_dense_attend_qq(stream, qq.data_ptr(), dtype_code(qq.dtype), rs, qw.data_ptr(), kw.data_ptr(),
                                      cos_p, sin_p, half, lam_p, out.data_ptr(), batch, length, num_heads, head_dim,
                                      float(eps), workspace.data_ptr(), workspace.numel() * workspace.element_size()),
               "attend_projected")
    return out


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """`x @ W^T` on the matrix cores (the reference's `_linear` without bias), fp32 accumulation, one rounding to
    `x.dtype`. `weight` is `(F, K)` (out x in) with F a multiple of 256 and K of 64."""
    _require_gpu(x, "x")
    if x.dtype not in FUSED_DTYPES:
        raise TypeError(f"linear takes bfloat16 or float16 inputs, got {x.dtype}")
    w = weight.to(device=x.device, dtype=x.dtype)
    n, xs = _rows(x, "x")
    _, wstride = _rows(w, "weight")
    f, k = w.shape
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} columns, weight {k}")
    out = torch.empty((*x.shape[:-1], f), dtype=x.dtype, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(_lib.load().hb_proj(stream, x.data_ptr(), dtype_code(x.dtype), xs, w.data_ptr(), wstride, out.data_ptr(),
                                   f, n, k, f), "linear")
    return out


def glu_linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, sinusoidal: bool) -> torch.Tensor:
    """`value * act(gate)` of `[value | gate] = x @ W^T (+ bias)` without storing the product (`hb_proj_glu`): the
    SAME-L feed-forward's `glu_proj` and GLU (reference: same_l._feed_forward, same_l.py:181-183), with the cast
    points of `elementwise.glu` on the rounded product. `weight` is the layer's `(2F, K)` (out x in), `bias` `(2F,)`
    or None; act = sin(pi * gate) when `sinusoidal`, else SiLU. F a multiple of 128, K of 64."""
    _require_gpu(x, "x")
    if x.dtype not in FUSED_DTYPES:
        raise TypeError(f"glu_linear takes bfloat16 or float16 inputs, got {x.dtype}")
    w = weight.to(device=x.device, dtype=x.dtype)
    n, xs = _rows(x, "x")
    _, wstride = _rows(w, "weight")
    f2, k = w.shape
    if x.shape[-1] != k or f2 % 2:
        raise ValueError(f"x has {x.shape[-1]} columns, weight is {tuple(w.shape)}")
    f = f2 // 2
    bias_p = 0
    if bias is not None:
        bias = f32_vector(bias, x.device)
        if bias.numel() != f2:
            raise ValueError(f"bias must have {f2} elements")
        bias_p = bias.data_ptr()
    out = torch.empty((*x.shape[:-1], f), dtype=x.dtype, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(_lib.load().hb_proj_glu(stream, x.data_ptr(), dtype_code(x.dtype), xs, w.data_ptr(), wstride, bias_p,
                                       int(bool(sinusoidal)), out.data_ptr(), f, n, k, f), "glu_linear")
    return out


def residual_linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, h: torch.Tensor,
                    norm: dict | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
    """`(h + (x @ W^T + bias), cast(DyT(...)))` with the residual add and the next DyT in the GEMM's epilogue
    (`hb_proj_residual`): the SAME-L `to_out` / `proj_out` and the residual add after them (reference:
    same_l._block, same_l.py:191-192, and same_l._linear), with the cast points of `elementwise.residual_dyt` on the
    rounded product. `weight` is `(F, K)` (out x in), `bias` `(F,)` or None, `h` the residual `(..., F)`; without
    `norm` (DyT params) the second result is None. F a multiple of 256, K of 64."""
    _require_gpu(x, "x")
    if x.dtype not in FUSED_DTYPES:
        raise TypeError(f"residual_linear takes bfloat16 or float16 inputs, got {x.dtype}")
    w = weight.to(device=x.device, dtype=x.dtype)
    n, xs = _rows(x, "x")
    _, wstride = _rows(w, "weight")
    f, k = w.shape
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} columns, weight {k}")
    if h.shape[:-1] != x.shape[:-1] or h.shape[-1] != f or h.dtype != x.dtype:
        raise ValueError(f"h must be {(*x.shape[:-1], f)} of {x.dtype}, got {tuple(h.shape)} {h.dtype}")
    _, hs = _rows(h, "h")
    bias_p = 0
    if bias is not None:
        bias = f32_vector(bias, x.device)
        if bias.numel() != f:
            raise ValueError(f"bias must have {f} elements")
        bias_p = bias.data_ptr()
    params = pack_dyt(norm, f, x.device) if norm is not None else None
    out_h = torch.empty(h.shape, dtype=x.dtype, device=x.device)
    out_y = torch.empty(h.shape, dtype=x.dtype, device=x.device) if norm is not None else None
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(_lib.load().hb_proj_residual(stream, x.data_ptr(), dtype_code(x.dtype), xs, w.data_ptr(), wstride,
                                            bias_p, h.data_ptr(), hs, params.data_ptr() if params is not None else 0,
                                            out_h.data_ptr(), out_y.data_ptr() if out_y is not None else 0, f, n, k,
                                            f), "residual_linear")
    return out_h, out_y


def same_l_supported(dtype: torch.dtype, dim: int, ff_inner: int, qkv_width: int) -> bool:
    """Whether the SAME-L block's projections take the fused kernels: bf16 or half, model width a multiple of 256,
    feed-forward width a multiple of 256 (its GLU half of 128 and proj_out's reduction of 64), the to_qkv width a
    multiple of 256."""
    return (dtype in FUSED_DTYPES and dim % 256 == 0 and ff_inner % 256 == 0 and qkv_width % 256 == 0 and dim > 0
            and ff_inner > 0)
