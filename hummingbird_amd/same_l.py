"""The SAME-L decoder block with the `attention="hip"` dispatch: its attention step (sa3jax/same_l.py:151-169),
its feed-forward (sa3jax/same_l.py:172-183), the block around them (sa3jax/same_l.py:186-192) and the decoder's
loop over its blocks (sa3jax/same_l.py:236-237).

`attention="hip"` runs the band attention, the DyT norms, the GLU gate and the residual adds (fused with the DyT or
the bias add next to them) as HIP kernels and the projections as torch GEMMs (hipBLASLt); with `projections="hip"`
the projections run on this package's GEMMs instead, `glu_proj` with the GLU in its epilogue and `to_out` /
`proj_out` with the residual add and the next DyT in theirs. `attention="xla"` runs the torch restatement of the
reference's chain.
"""
from __future__ import annotations

import torch

from hummingbird_amd import band_attention, elementwise, projection, xla_chain
from hummingbird_amd.config import SameConfig
from hummingbird_amd.dtypes import Dtype


def use_hip(cfg: SameConfig, qkv: torch.Tensor) -> bool:
    """Dispatch predicate (reference: same_l.py:158): the HIP kernel when selected on ROCm device tensors."""
    if cfg.attention != "hip":
        return False
    if not qkv.is_cuda:
        raise ValueError('attention="hip" needs ROCm device tensors; use attention="xla" on the CPU')
    return True


def attention(x: torch.Tensor, block: dict, cfg: SameConfig, lam: torch.Tensor | None = None,
              dtype: Dtype | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """`to_qkv` -> differential band attention at half-width `sub_chunk_size` -> `to_out` (reference:
    same_l._attention, same_l.py:151-169). `block` holds `self_attn.{to_qkv,to_out}.weight`,
    `self_attn.{q_norm,k_norm}` DyT params and `rope_inv_freq`. `dtype` (a preset of hummingbird_amd.dtypes) casts
    `x` and the projection weights to its compute dtype; without it they are used as given. `workspace` (from
    `band_attention.band_workspace`) is passed to the band kernel."""
    attn = block["self_attn"]
    if dtype is not None:
        x = x.to(dtype.compute)
    qkv = x @ attn["to_qkv"]["weight"].to(x.dtype).t()
    if use_hip(cfg, qkv):
        out = band_attention.band_attention(qkv, attn["q_norm"], attn["k_norm"], block["rope_inv_freq"],
                                            cfg.num_heads, cfg.dim_heads, cfg.sub_chunk_size, lam=lam,
                                            workspace=workspace)
    else:
        out = xla_chain.band_chain(qkv, attn["q_norm"], attn["k_norm"], block["rope_inv_freq"], cfg.num_heads,
                                   cfg.dim_heads, cfg.sub_chunk_size, lam=lam)
    return out @ attn["to_out"]["weight"].to(out.dtype).t()


def _linear(x: torch.Tensor, layer: dict) -> torch.Tensor:
    """`x @ W^T (+ b)` in the compute dtype (reference: same_l._linear)."""
    y = x @ layer["weight"].t()
    return y if layer.get("bias") is None else y + layer["bias"]


def feed_forward(x: torch.Tensor, block: dict, index: int, cfg: SameConfig) -> torch.Tensor:
    """`glu_proj` -> value * act(gate) -> `proj_out` (reference: same_l._feed_forward, same_l.py:172-183); act is
    sin(pi x) on the last `sinusoidal_blocks` blocks and SiLU before them."""
    ff = block["ff"]
    sine = cfg.sinusoidal(index)
    if use_hip(cfg, x):  # the bias add runs inside the GLU kernel, with the same roundings
        gated = elementwise.glu(x @ ff["glu_proj"]["weight"].t(), sine, bias=ff["glu_proj"].get("bias"))
    else:
        gated = xla_chain.glu(_linear(x, ff["glu_proj"]), sine)
    return _linear(gated, ff["proj_out"])


def _fused_projections(cfg: SameConfig, x: torch.Tensor, params: dict, projections: str) -> bool:
    """Whether this block runs its projections on the fused GEMMs: `projections="hip"` and a geometry they take."""
    if projections not in ("torch", "hip"):
        raise ValueError(f'projections must be "torch" or "hip", got {projections!r}')
    if projections != "hip":
        return False
    dim = x.shape[-1]
    ff = params["ff"]["proj_out"]["weight"].shape[-1]
    qkv_width = params["self_attn"]["to_qkv"]["weight"].shape[0]
    return projection.same_l_supported(x.dtype, dim, ff, qkv_width)


def block(x: torch.Tensor, params: dict, index: int, cfg: SameConfig,
          lam: torch.Tensor | None = None, projections: str = "torch") -> torch.Tensor:
    """One decoder block (reference: same_l._block, same_l.py:186-192):
    `h = x + attention(DyT(x; pre_norm))`, then `h + feed_forward(DyT(h; ff_norm))`, each DyT in fp32 and cast
    back to `x.dtype` before its GEMM. `params` holds `pre_norm`, `ff_norm` (DyT params), `self_attn`,
    `rope_inv_freq` (as `attention` reads them) and `ff.{glu_proj,proj_out}.{weight,bias}`."""
    if not use_hip(cfg, x):
        h = x + attention(xla_chain.dyt_cast(x, params["pre_norm"]), params, cfg, lam=lam)
        return h + feed_forward(xla_chain.dyt_cast(h, params["ff_norm"]), params, index, cfg)
    out, _ = _block_hip(x, elementwise.dyt(x, params["pre_norm"]), params, index, cfg, lam, None,
                        projections=projections)
    return out


def _block_hip(x: torch.Tensor, y: torch.Tensor, params: dict, index: int, cfg: SameConfig,
               lam: torch.Tensor | None, next_norm: dict | None,
               workspace: torch.Tensor | None = None,
               projections: str = "torch") -> tuple[torch.Tensor, torch.Tensor | None]:
    """A block from its input `x` and `y` = DyT(x; pre_norm) cast: `(out, DyT(out; next_norm) or None)`. The residual
    adds run fused with what surrounds them, with the same roundings: the first with the ff_norm DyT that follows it,
    the second with proj_out's bias add before it and, given `next_norm`, the next block's pre_norm DyT after it.
    With `projections="hip"` (and a geometry the fused GEMMs take) they move into the GEMMs' epilogues: to_out's
    for the first, proj_out's for the second, and the GLU into glu_proj's."""
    if _fused_projections(cfg, y, params, projections):
        attn, ff = params["self_attn"], params["ff"]
        qkv = projection.linear(y, attn["to_qkv"]["weight"])
        a = band_attention.band_attention(qkv, attn["q_norm"], attn["k_norm"], params["rope_inv_freq"], cfg.num_heads,
                                          cfg.dim_heads, cfg.sub_chunk_size, lam=lam, workspace=workspace)
        h, y = projection.residual_linear(a, attn["to_out"]["weight"], attn["to_out"].get("bias"), x,
                                          params["ff_norm"])
        gated = projection.glu_linear(y, ff["glu_proj"]["weight"], ff["glu_proj"].get("bias"), cfg.sinusoidal(index))
        return projection.residual_linear(gated, ff["proj_out"]["weight"], ff["proj_out"].get("bias"), h, next_norm)
    a = attention(y, params, cfg, lam=lam, workspace=workspace)
    h, y = elementwise.residual_dyt(x, a, norm=params["ff_norm"])
    ff = params["ff"]
    gated = elementwise.glu(y @ ff["glu_proj"]["weight"].t(), cfg.sinusoidal(index), bias=ff["glu_proj"].get("bias"))
    return elementwise.residual_dyt(h, gated @ ff["proj_out"]["weight"].t(), bias=ff["proj_out"].get("bias"),
                                    norm=next_norm)


def blocks(x: torch.Tensor, params: list, cfg: SameConfig, lam: torch.Tensor | None = None,
           projections: str = "torch") -> torch.Tensor:
    """The decoder's block loop (reference: same_l.decode, `for index, block in enumerate(params["blocks"])`,
    same_l.py:236-237): `block` over `params` in order. With `attention="hip"` each block hands the next one its
    pre_norm DyT from the pass that finishes its own residual, so a chain of n blocks makes one DyT pass instead of
    n; the values are those of the block-by-block loop. The band kernel's workspace, where the shape takes one
    (fp32, or bf16 outside the streaming kernel), is allocated once for the whole loop. `projections` as `block`."""
    if not use_hip(cfg, x):
        for index, p in enumerate(params):
            x = block(x, p, index, cfg, lam=lam, projections=projections)
        return x
    y = elementwise.dyt(x, params[0]["pre_norm"])
    half = params[0]["rope_inv_freq"].shape[0]
    ws = band_attention.band_workspace(x.shape[0], x.shape[1], cfg.num_heads, cfg.dim_heads, cfg.sub_chunk_size, half,
                                       x.dtype, x.device)
    for index, p in enumerate(params):
        nxt = params[index + 1]["pre_norm"] if index + 1 < len(params) else None
        x, y = _block_hip(x, y, p, index, cfg, lam, nxt, workspace=ws, projections=projections)
    return x
