"""The DiT around the attention kernels, in torch: the attention call sites with the `attention="hip"` dispatch
(self-attention, sa3jax/dit.py:179-200; cross-attention against its context K/V hoisted out of the sampler loop,
sa3jax/dit.py:203-215, 274-284), the per-clip state (`prepare_static`, sa3jax/dit.py:287-337) and the denoiser
(`dit_forward`, sa3jax/dit.py:340-361, with the adaLN block of sa3jax/dit.py:224-251).

Everything that does not depend on `x` or `t` is built once per clip in `prepare_static`: the RoPE tables and
value mask in the kernels' layout, the attention workspace, every block's prepared cross-attention context, the
projected global condition and the blocks' constant local embeddings. `dit_forward` is then a fixed sequence of
launches with no host synchronisation, so the sampler can capture it in a HIP graph.

Cast points: each elementwise step rounds to the compute dtype (as the reference's JAX arrays hold them), the
block norms run in fp32 and cast back, the timestep features are fp32 (sa3jax/dit.py:44-79).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from hummingbird_amd import cross_attention as xattn
from hummingbird_amd import dense_attention, projection, xla_chain
from hummingbird_amd import elementwise as ew
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
                                           cfg.qk_norm_eps, workspace=static.get("hip_workspace"))
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
                                              lam=lam, workspace=static.get("hip_workspace"))
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


# ---------------------------------------------------------------------------------------------------------------
# The denoiser around the attention call sites.

def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """`nn.Linear` with the weight stored (out, in) (sa3jax/dit.py:31-34): the product rounded to `x.dtype`, then
    the bias added."""
    y = x @ weight.to(x.dtype).t()
    return y if bias is None else y + bias.to(x.dtype)


def silu(x: torch.Tensor) -> torch.Tensor:
    """`jax.nn.silu` as `x * sigmoid(x)` with the sigmoid held in `x.dtype`."""
    return x * torch.sigmoid(x)


def sequential(seq: dict, x: torch.Tensor) -> torch.Tensor:
    """`Linear -> SiLU -> Linear` (sa3jax/dit.py:37-41); the biases are optional per layer."""
    inner, outer = seq["in"], seq["out"]
    return linear(silu(linear(x, inner["weight"], inner.get("bias"))), outer["weight"], outer.get("bias"))


def conv1x1(x: torch.Tensor, kernel: torch.Tensor) -> torch.Tensor:
    """1x1 `Conv1d` on a `(B, C, T)` tensor as a channel product (sa3jax/dit.py:60-68), kernel `(out, in, 1)`.
    Evaluated as `(x^T W^T)^T` so that the batched operand is never a transposed view on the right."""
    return (x.transpose(1, 2) @ kernel[:, :, 0].to(x.dtype).t()).transpose(1, 2)


def expo_fourier(t: torch.Tensor, dim: int) -> torch.Tensor:
    """`ExpoFourierFeatures(dim, 0.5, 10000)` (sa3jax/dit.py:71-79): frequencies `exp(linspace(0, 1) *
    (ln 10000 - ln 0.5) + ln 0.5)`, angles `2 pi t f`, `[cos | sin]` in fp32, cast to `t.dtype`."""
    f32 = torch.float32
    freqs = torch.exp(torch.linspace(0.0, 1.0, dim // 2, dtype=f32, device=t.device)
                      * (math.log(10000.0) - math.log(0.5)) + math.log(0.5))
    args = t.to(f32)[:, None] * freqs
    args = args * (2.0 * math.pi)
    return torch.cat([torch.cos(args), torch.sin(args)], dim=-1).to(t.dtype)


def feed_forward(x: torch.Tensor, ff: dict) -> torch.Tensor:
    """SwiGLU (sa3jax/dit.py:218-221): `glu_proj` (+bias) -> `value * silu(gate)` -> `proj_out` (+bias)."""
    value, gate = linear(x, ff["glu_proj"]["weight"], ff["glu_proj"]["bias"]).chunk(2, dim=-1)
    return linear(value * silu(gate), ff["proj_out"]["weight"], ff["proj_out"]["bias"])


def local_constants(blocks: list, compute: torch.dtype) -> torch.Tensor:
    """`(depth, E)`: each block's `to_local_embed` output for the all-zero local condition of text-to-audio,
    `W2 silu(b1) + b2` (sa3jax/dit.py:254-271)."""
    return torch.stack([linear(silu(b["to_local_embed"]["in"]["bias"].to(compute)), b["to_local_embed"]["out"]["weight"],
                               b["to_local_embed"]["out"]["bias"]) for b in blocks])


def block_forward(h: torch.Tensor, block: dict, static: dict, gcond: torch.Tensor, index: int, cfg: DiTConfig,
                  projections: str = "torch", adaln: torch.Tensor | None = None) -> torch.Tensor:
    """One transformer block with adaLN (sa3jax/dit.py:224-251): `h + attn(rms(h) (1 + scale) + shift) *
    sigmoid(1 - gate)`, `h + cross(rms(h))`, the local constant on the latent tokens, then the feed-forward the
    same way as the self-attention. `gcond` is `(B, 6 E)`; `adaln`, if given, is the block's
    `to_scale_shift_gate + gcond` computed by the caller (the same values)."""
    compute = h.dtype
    if adaln is None:
        adaln = block["to_scale_shift_gate"].to(compute) + gcond
    scale_self, shift_self, gate_self, scale_ff, shift_ff, gate_ff = adaln[:, None, :].chunk(6, dim=-1)
    if use_hip(cfg, h):
        return _block_fused(h, block, static, (scale_self, shift_self, gate_self, scale_ff, shift_ff, gate_ff), index,
                            cfg, projections)
    x = xla_chain.rms(h, block["pre_norm"]["weight"], cfg.norm_eps)
    x = x * (1 + scale_self) + shift_self
    x = self_attention(x, block, static, cfg, projections=projections)
    h = h + x * torch.sigmoid(1 - gate_self)

    x = xla_chain.rms(h, block["cross_attend_norm"]["weight"], cfg.norm_eps)
    h = h + cross_attention(x, block, static["cross"][index], cfg)

    # the memory tokens receive no local condition (sa3jax/dit.py:239-241)
    memory = cfg.num_memory_tokens
    h = torch.cat([h[:, :memory], h[:, memory:] + static["local"][index]], dim=1)

    x = xla_chain.rms(h, block["ff_norm"]["weight"], cfg.norm_eps)
    x = x * (1 + scale_ff) + shift_ff
    x = feed_forward(x, block["ff"])
    return h + x * torch.sigmoid(1 - gate_ff)


def _blocks_fused(h: torch.Tensor, blocks: list, static: dict, adaln: torch.Tensor, cfg: DiTConfig,
                  projections: str) -> torch.Tensor:
    """Every block of `dit_forward` with the elementwise steps in HIP kernels, residual and following norm fused
    (`hb_residual_rms`): the feed-forward residual of block i computes block i + 1's modulated input in the same
    pass. Same values as `block_forward` block after block. `adaln` is `(depth, B, 6 E)`."""
    eps, E = cfg.norm_eps, h.shape[-1]
    depth = len(blocks)

    def chunks(i):
        return adaln[i].reshape(adaln.shape[1], 6, E).unbind(1)  # (B, E) views: scale, shift, gate x 2
    s_self, sh_self, g_self, s_ff, sh_ff, g_ff = chunks(0)
    x = ew.rms_modulate(h, blocks[0]["pre_norm"]["weight"], eps, s_self, sh_self)
    for i, block in enumerate(blocks):
        s_self, sh_self, g_self, s_ff, sh_ff, g_ff = chunks(i)
        a = self_attention(x, block, static, cfg, projections=projections)
        h, x = ew.residual_rms(h, a, block["cross_attend_norm"]["weight"], eps, gate=g_self)
        c = cross_attention(x, block, static["cross"][i], cfg)
        h, x = ew.residual_rms(h, c, block["ff_norm"]["weight"], eps, local=static["local"][i],
                               memory=cfg.num_memory_tokens, scale=s_ff, shift=sh_ff)
        ff = block["ff"]
        f = linear(ew.glu(linear(x, ff["glu_proj"]["weight"]), False, bias=ff["glu_proj"]["bias"]),
                   ff["proj_out"]["weight"])
        bias = ff["proj_out"]["bias"].to(h.dtype)
        if i + 1 < depth:
            ns, nsh = chunks(i + 1)[:2]
            h, x = ew.residual_rms(h, f, blocks[i + 1]["pre_norm"]["weight"], eps, gate=g_ff, x_bias=bias, scale=ns,
                                   shift=nsh)
        else:
            h = ew.gated_residual(h, f, gate=g_ff, x_bias=bias)
    return h


def _block_fused(h: torch.Tensor, block: dict, static: dict, adaln: tuple, index: int, cfg: DiTConfig,
                 projections: str) -> torch.Tensor:
    """`block_forward` with the elementwise steps in HIP kernels, same cast points: `hb_rms_modulate` for the three
    norms (with the adaLN modulation where the block has it), `hb_gated_residual` for the three residuals (the gates,
    proj_out's bias and the local constant folded in), `hb_glu` for the SwiGLU with glu_proj's bias."""
    scale_self, shift_self, gate_self, scale_ff, shift_ff, gate_ff = (t[:, 0] for t in adaln)
    x = ew.rms_modulate(h, block["pre_norm"]["weight"], cfg.norm_eps, scale_self, shift_self)
    x = self_attention(x, block, static, cfg, projections=projections)
    h = ew.gated_residual(h, x, gate=gate_self)

    x = ew.rms_modulate(h, block["cross_attend_norm"]["weight"], cfg.norm_eps)
    x = cross_attention(x, block, static["cross"][index], cfg)
    h = ew.gated_residual(h, x, local=static["local"][index], memory=cfg.num_memory_tokens)

    x = ew.rms_modulate(h, block["ff_norm"]["weight"], cfg.norm_eps, scale_ff, shift_ff)
    ff = block["ff"]
    x = ew.glu(linear(x, ff["glu_proj"]["weight"]), False, bias=ff["glu_proj"]["bias"])
    x = linear(x, ff["proj_out"]["weight"])
    return ew.gated_residual(h, x, gate=gate_ff, x_bias=ff["proj_out"]["bias"].to(h.dtype))


def _fp32_norms(block: dict) -> dict:
    """A view of a block's parameters with its norm scales and glu_proj's bias in fp32, the forms the HIP kernels take
    (the other tensors shared), so that no call converts them again."""
    out = dict(block)
    for key in ("pre_norm", "cross_attend_norm", "ff_norm"):
        out[key] = {"weight": block[key]["weight"].float().contiguous()}
    for attn in ("self_attn", "cross_attn"):
        out[attn] = dict(block[attn])
        for norm in ("q_norm", "k_norm"):
            out[attn][norm] = {"weight": block[attn][norm]["weight"].float().contiguous()}
    glu = block["ff"]["glu_proj"]
    if glu.get("bias") is not None:  # hb_glu reads it in fp32; the torch route casts it to the compute dtype again
        out["ff"] = {**block["ff"], "glu_proj": {**glu, "bias": glu["bias"].float().contiguous()}}
    return out


def prepare_static(params: dict, cond: dict, padding_mask: torch.Tensor, cfg: DiTConfig, dtype: Dtype) -> dict:
    """Everything `dit_forward` reads that does not depend on `x` or `t` (sa3jax/dit.py:287-337), built once per
    clip: the tables of `static_tables`, the projected context and every block's prepared cross-attention
    context (`cross_context`), the projected global condition, the blocks' local constants and, with
    `attention="hip"`, the dense attention workspace that every self-attention call of the clip reuses.

    `cond` holds `cross_attn_cond (B, Nk, cond_token_dim)`, `global_cond (B, global_cond_dim)` and optionally
    `local_add_cond`, which must be all zero (text-to-audio), as the reference requires (sa3jax/dit.py:296-301)."""
    local = cond.get("local_add_cond")
    if local is not None and bool(torch.any(local != 0)):
        raise ValueError("local_add_cond is non-zero (inpaint): the constant to_local_embed shortcut holds only for "
                         "an all-zero input")
    net = params["transformer"]
    compute = dtype.compute
    static = static_tables(net["rope_inv_freq"], padding_mask, cfg, dtype)
    ctx = sequential(params["to_cond_embed"], cond["cross_attn_cond"].to(compute))
    static["cross"] = [cross_context(b, ctx, cfg) for b in net["blocks"]]
    static["gcond_proj"] = sequential(params["to_global_embed"], cond["global_cond"].to(compute))
    static["local"] = local_constants(net["blocks"], compute)
    static["adaln"] = torch.stack([b["to_scale_shift_gate"].to(compute) for b in net["blocks"]])  # (depth, 6 E)
    if cfg.attention == "hip":  # the kernels take the norm scales in fp32: convert them once per clip
        static["blocks"] = [_fp32_norms(b) for b in net["blocks"]]
    if cfg.attention == "hip" and cfg.differential:
        batch, length = padding_mask.shape[0], cfg.num_memory_tokens + padding_mask.shape[1]
        need = dense_attention.workspace_bytes(compute, batch, length, cfg.num_heads, cfg.head_dim)
        static["hip_workspace"] = torch.empty(need, dtype=torch.uint8, device=padding_mask.device)
    return static


def dit_forward(params: dict, x: torch.Tensor, t: torch.Tensor, static: dict, cfg: DiTConfig, dtype: Dtype,
                projections: str = "torch") -> torch.Tensor:
    """One denoiser evaluation (sa3jax/dit.py:340-361): `(B, io_channels, T)` latents and `(B,)` timesteps -> the
    velocity, same shape, in the compute dtype. `static` comes from `prepare_static`. `projections` is passed to
    `self_attention`."""
    net = params["transformer"]
    compute = dtype.compute
    h = x.to(compute)
    h = conv1x1(h, params["preprocess_conv"]["weight"]) + h
    h = linear(h.transpose(1, 2), net["project_in"]["weight"])
    memory = net["memory_tokens"].to(compute).expand(h.shape[0], cfg.num_memory_tokens, cfg.embed_dim)
    h = torch.cat([memory, h], dim=1)

    timestep = sequential(params["to_timestep_embed"], expo_fourier(t.to(compute), cfg.fourier_dim))
    gcond = sequential(net["global_cond_embedder"], static["gcond_proj"] + timestep)

    adaln = static["adaln"][:, None, :] + gcond[None] if "adaln" in static else None  # every block's, one launch
    blocks = static.get("blocks", net["blocks"])
    if adaln is not None and blocks and use_hip(cfg, h) and ew.residual_rms_supported(h.dtype, cfg.embed_dim):
        h = _blocks_fused(h, blocks, static, adaln, cfg, projections)
    else:
        for index, block in enumerate(blocks):
            h = block_forward(h, block, static, gcond, index, cfg, projections,
                              adaln=None if adaln is None else adaln[index])

    h = linear(h[:, cfg.num_memory_tokens:, :], net["project_out"]["weight"])
    v = h.transpose(1, 2)
    return conv1x1(v, params["postprocess_conv"]["weight"]) + v


def init_params(cfg: DiTConfig, dtype: Dtype, device="cpu", seed: int = 0) -> dict:
    """Random-initialised DiT weights in the reference's pytree layout (sa3jax/weights.py:90-120), stored in
    `dtype.weight` (the RoPE `inv_freq` in `dtype.rope`): linear weights N(0, 1/fan_in), biases N(0, 0.02^2),
    norm scales 1 + N(0, 0.02^2), adaLN offsets N(0, 0.02^2), drawn on `device` from a generator seeded with
    `seed`. For tests and benchmarks (no checkpoint here)."""
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)  # drawn where they live: no host copy of the weights
    E, wd = cfg.embed_dim, dtype.weight

    def randn(*shape):
        return torch.randn(shape, generator=gen, device=device)

    def w(o, i):
        return (randn(o, i) / math.sqrt(i)).to(wd)

    def b(n, std=0.02):
        return (std * randn(n)).to(wd)

    def norm(n):
        return {"weight": (1 + 0.02 * randn(n)).to(wd)}

    def seq(i, o_in, o_out, bias):
        s = {"in": {"weight": w(o_in, i)}, "out": {"weight": w(o_out, o_in)}}
        if bias:
            s["in"]["bias"], s["out"]["bias"] = b(o_in), b(o_out)
        return s
    H, D = cfg.num_heads, cfg.head_dim
    blocks = []
    for _ in range(cfg.depth):
        qkv_width = (5 if cfg.differential else 3) * H * D
        blocks.append({
            "to_scale_shift_gate": b(cfg.adaln_dim),
            "pre_norm": norm(E), "cross_attend_norm": norm(E), "ff_norm": norm(E),
            "self_attn": {"to_qkv": {"weight": w(qkv_width, E)}, "to_out": {"weight": w(E, H * D)},
                          "q_norm": norm(D), "k_norm": norm(D)},
            "cross_attn": {"to_q": {"weight": w((2 if cfg.differential else 1) * H * D, E)},
                           "to_kv": {"weight": w((3 if cfg.differential else 2) * H * D, E)},
                           "to_out": {"weight": w(E, H * D)}, "q_norm": norm(D), "k_norm": norm(D)},
            "ff": {"glu_proj": {"weight": w(2 * cfg.ff_inner, E), "bias": b(2 * cfg.ff_inner)},
                   "proj_out": {"weight": w(E, cfg.ff_inner), "bias": b(E)}},
            "to_local_embed": seq(cfg.local_add_cond_dim, E, E, True),
        })
    half = cfg.rope_dim // 2
    inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, 2 * half, 2, dtype=torch.float64) / (2 * half)))
    io = cfg.io_channels
    return {
        "preprocess_conv": {"weight": w(io, io)[:, :, None]},
        "postprocess_conv": {"weight": w(io, io)[:, :, None]},
        "to_timestep_embed": seq(cfg.fourier_dim, E, E, True),
        "to_cond_embed": seq(cfg.cond_token_dim, E, E, False),
        "to_global_embed": seq(cfg.global_cond_dim, E, E, False),
        "transformer": {
            "project_in": {"weight": w(E, io)},
            "project_out": {"weight": w(io, E)},
            "memory_tokens": randn(cfg.num_memory_tokens, E).to(wd),
            "rope_inv_freq": inv_freq.to(device, dtype.rope),
            "global_cond_embedder": seq(E, E, cfg.adaln_dim, True),
            "blocks": blocks,
        },
    }
