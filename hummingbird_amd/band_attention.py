"""SAME-L band differential attention on MI355X: the `attention="hip"` counterpart of the reference's
`sa3jax/band_attention.py` (same function names, argument meaning and error behaviour).

`band_attention` runs DyT -> RoPE -> both windowed softmax branches -> subtract on the GPU through the C ABI
(`hb_band_diffattn`), replacing the Pallas kernel (band_attention.py:123-180). `rope_tables` replaces the
reference's lane tables (band_attention.py:43-58) with `(length, half)` fp32 tables built on the device.
"""
from __future__ import annotations

import torch

from hummingbird_amd import _lib, rotary
from hummingbird_amd._derived import derived
from hummingbird_amd.dense_attention import (SUPPORTED_HEAD_DIMS, _f32, _require_gpu, _row_stride, dtype_code,
                                             rope_tables)

__all__ = ["band_attention", "band_workspace", "rope_tables", "pack_dyt"]

# fp32 calls given no workspace allocate one (it lets every key be prepared once) only up to this size; above it they
# run the kernel that prepares each query block's key window itself, which needs none.
FP32_WORKSPACE_CAP = 256 << 20


def _cached_tables(inv_freq: torch.Tensor, length: int, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """The RoPE tables of `inv_freq` at `length`, built once per live, unedited caller tensor (a decoder's blocks
    share one inv_freq buffer, so its repeated calls reuse one table instead of rebuilding it per call)."""
    return derived((inv_freq,), ("rope", length, device),
                   lambda: rope_tables(length, inv_freq.to(device) if inv_freq.device != device else inv_freq))


def _pack_dyt(norm: dict, head_dim: int, device: torch.device) -> torch.Tensor:
    alpha = torch.as_tensor(norm["alpha"]).to(device=device, dtype=torch.float32).reshape(-1)
    gamma = torch.as_tensor(norm["gamma"]).to(device=device, dtype=torch.float32).reshape(-1)
    beta = torch.as_tensor(norm["beta"]).to(device=device, dtype=torch.float32).reshape(-1)
    if alpha.numel() != 1 or gamma.numel() != head_dim or beta.numel() != head_dim:
        raise ValueError(f"DyT params need a scalar alpha and (head_dim={head_dim},) gamma and beta")
    return torch.cat([alpha, gamma, beta]).contiguous()


def pack_dyt(norm: dict, head_dim: int, device: torch.device) -> torch.Tensor:
    """`{alpha: scalar, gamma: (D,), beta: (D,)}` (the DyT params of sa3jax/same_l.py:58-69) -> the C ABI's
    `[alpha, gamma[0..D), beta[0..D)]` fp32 vector. When the three are tensors the vector is built once per live,
    unedited set of them (a decoder passes the same params on every call); a Python-number alpha packs anew."""
    parts = (norm["alpha"], norm["gamma"], norm["beta"])
    if not all(isinstance(t, torch.Tensor) for t in parts):
        return _pack_dyt(norm, head_dim, device)
    return derived(parts, ("dyt", head_dim, device), lambda: _pack_dyt(norm, head_dim, device))


def _workspace_bytes(dtype: torch.dtype, batch: int, length: int, num_heads: int, head_dim: int, half: int,
                     window: int) -> int:
    half = rotary.aligned_half(half) if half % rotary.ALIGN else half
    return int(_lib.load().hb_band_workspace_size(dtype_code(dtype), batch, length, num_heads, head_dim, half,
                                                  int(window)))


def band_workspace(batch: int, length: int, num_heads: int, head_dim: int, window: int, half: int,
                   dtype: torch.dtype, device) -> torch.Tensor | None:
    """A workspace that `band_attention` calls of this shape can share (`workspace=`), or None when they need none:
    the bf16 shapes outside the streaming kernel require one; fp32 calls use one if given (every key prepared once).
    The decoder's block loop allocates it once for all its blocks."""
    need = _workspace_bytes(dtype, batch, length, num_heads, head_dim, half, window)
    return torch.empty(need, dtype=torch.uint8, device=device) if need else None


def band_attention(qkv: torch.Tensor, q_norm: dict, k_norm: dict, inv_freq: torch.Tensor, num_heads: int,
                   head_dim: int, window: int, *, rows: int = 1024, halo: int = 32, sub: int = 256,
                   stack: bool = True, interpret: bool = False, lam: torch.Tensor | None = None,
                   tables: tuple[torch.Tensor, torch.Tensor] | None = None,
                   workspace: torch.Tensor | None = None) -> torch.Tensor:
    """`(B, S, 5 * H * D)` projection output -> `(B, S, H * D)` differential band attention, in `qkv.dtype`.

    Same contract as the reference (sa3jax/band_attention.py:123-135): `q_norm`/`k_norm` are the block's DyT
    params (`alpha` scalar, `gamma`/`beta` `(D,)`), shared by both branches; a query at position p sees keys
    `|k - p| <= window` inside `[0, S)`. `rows`, `halo`, `sub`, `stack` and `interpret` are the TPU kernel's
    tiling knobs and are accepted and ignored (the reference's `halo >= window` constraint does not apply: the
    HIP kernel takes any window >= 0). `lam` `(H,)` optionally weights the second branch (default 1, the
    reference). `tables` optionally supplies `(cos, sin)` from `rope_tables(S, inv_freq)`. `workspace` optionally
    supplies the scratch that bf16 shapes outside the streaming kernel (window > 128 or head_dim 128) need, and that
    fp32 calls use to prepare every key once: `hb_band_workspace_size` bytes of uint8 on the same device
    (`band_workspace`). When absent it is allocated here for those bf16 shapes, and for fp32 only up to
    `FP32_WORKSPACE_CAP` bytes (larger fp32 calls run without one). Any rotary
    half-width `inv_freq.shape[0]` in `[0, head_dim / 2]` is taken; one that is not a multiple of 8 runs on a copy
    of `qkv` with the q and k dims reordered (`hummingbird_amd.rotary`).
    """
    del rows, halo, sub, stack, interpret
    _require_gpu(qkv, "qkv")
    if qkv.dim() != 3:
        raise ValueError(f"qkv must be (B, S, 5*H*D), got shape {tuple(qkv.shape)}")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"band_attention needs head_dim in {SUPPORTED_HEAD_DIMS} (head_dim={head_dim})")
    if window < 0:
        raise ValueError(f"band_attention needs window >= 0 (window={window})")
    batch, length, width = qkv.shape
    if width != 5 * num_heads * head_dim:
        raise ValueError(f"qkv width {width} != 5 * num_heads * head_dim = {5 * num_heads * head_dim}")
    dev = qkv.device
    half = inv_freq.shape[0]
    if not 0 <= half <= head_dim // 2:
        raise ValueError(f"inv_freq has {half} entries; the rotary half-width must be in [0, head_dim/2]")
    code = dtype_code(qkv.dtype)
    rs = _row_stride(qkv)
    qd, kd = pack_dyt(q_norm, head_dim, dev), pack_dyt(k_norm, head_dim, dev)
    cos_p = sin_p = 0
    if half > 0:
        if tables is None:
            cos, sin = _cached_tables(inv_freq, length, dev)
        else:
            cos, sin = (_f32(t, dev) for t in tables)
            if tuple(cos.shape) != (length, half) or tuple(sin.shape) != (length, half):
                raise ValueError(f"tables must be (S, half) = ({length}, {half})")
        if half % rotary.ALIGN:  # the kernels pair 8-dim groups: reorder the q and k dims (see rotary)
            qkv = rotary.reorder_sections(qkv, num_heads, head_dim, half, (True, True, False, True, True))
            rs = qkv.shape[-1]
            qd, kd = (torch.cat([p[:1], rotary.reorder_dims(p[1:1 + head_dim], head_dim, half),
                                 rotary.reorder_dims(p[1 + head_dim:], head_dim, half)]) for p in (qd, kd))
            cos, sin = rotary.pad_tables(cos, sin, half)
            half = rotary.aligned_half(half)
        cos_p, sin_p = cos.data_ptr(), sin.data_ptr()
    lam_p = 0
    if lam is not None:
        lam = _f32(lam, dev).reshape(-1)
        if lam.numel() != num_heads:
            raise ValueError("lam must have num_heads elements")
        lam_p = lam.data_ptr()
    out = torch.empty((batch, length, num_heads * head_dim), dtype=qkv.dtype, device=dev)
    lib = _lib.load()
    need = int(lib.hb_band_workspace_size(code, batch, length, num_heads, head_dim, half, int(window)))
    ws_p, ws_bytes = 0, 0
    if need:  # shapes outside the streaming kernel, and fp32, prepare their keys into scratch
        if workspace is None and not (code == _lib.HB_F32 and need > FP32_WORKSPACE_CAP):
            workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        if workspace is not None:
            if workspace.numel() * workspace.element_size() < need or workspace.device != dev:
                raise ValueError(f"workspace must hold {need} bytes on {dev}")
            ws_p, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    stream = torch.cuda.current_stream(dev).cuda_stream
    status = lib.hb_band_diffattn(stream, qkv.data_ptr(), code, rs, qd.data_ptr(), kd.data_ptr(), cos_p, sin_p, half,
                                  int(window), lam_p, out.data_ptr(), batch, length, num_heads, head_dim, ws_p,
                                  ws_bytes)
    _lib.check(status, "band_attention")
    return out
