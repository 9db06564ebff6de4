"""The DiT denoiser and its per-clip state, restated in NumPy (oracle; test infrastructure only).

Follows sa3jax/dit.py: `_linear` (31-34), `_sequential` (37-41), `_rms` (44-57), `_conv1x1` (60-68),
`_expo_fourier` (71-79), `_feed_forward` (218-221), `_block` (224-251), `_local_constants` (254-271), `_cross_kv`
(274-284), `_static` (304-337) and `dit_forward` (340-361). The self-attention is `oracle.dense.dense_xla` on the
`to_qkv` output and the cross-attention `oracle.cross.cross_xla`, both pinned on their own.

Cast points: every elementwise step is evaluated exactly (float64 on compute-dtype values) and rounded once to
the compute dtype, as the reference's JAX arrays hold each intermediate; products accumulate in float64 and
round once; the norms run in fp32 and cast back; the timestep features are evaluated exactly and rounded once
(see `expo_fourier`). `compute` is "bf16", "fp16" or "fp32".
"""
from __future__ import annotations

import math

import numpy as np

from oracle import cross as ocross
from oracle import dense as odense
from oracle.bf16 import cast

F64 = np.float64


def linear(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None, compute: str) -> np.ndarray:
    """`x @ W^T` (W stored (out, in)) rounded once, then `+ b` rounded (dit.py:31-34)."""
    y = cast(np.asarray(cast(x, compute), F64) @ np.asarray(cast(weight, compute), F64).T, compute)
    if bias is None:
        return y
    return cast(y.astype(F64) + np.asarray(cast(bias, compute), F64), compute)


def silu(x: np.ndarray, compute: str) -> np.ndarray:
    """`x * sigmoid(x)` with the sigmoid rounded, then the product (jax.nn.silu)."""
    x64 = np.asarray(x, F64)
    sig = cast(1.0 / (1.0 + np.exp(-x64)), compute)
    return cast(x64 * sig.astype(F64), compute)


def sigmoid(x: np.ndarray, compute: str) -> np.ndarray:
    return cast(1.0 / (1.0 + np.exp(-np.asarray(x, F64))), compute)


def sequential(seq: dict, x: np.ndarray, compute: str) -> np.ndarray:
    """`Linear -> SiLU -> Linear` (dit.py:37-41)."""
    inner, outer = seq["in"], seq["out"]
    return linear(silu(linear(x, inner["weight"], inner.get("bias"), compute), compute), outer["weight"],
                  outer.get("bias"), compute)


def rms(x: np.ndarray, weight: np.ndarray, eps: float, compute: str) -> np.ndarray:
    """The block RMSNorm, fp32 island, cast back (dit.py:44-57)."""
    return odense.rms(cast(x, compute), np.asarray(weight, np.float32), eps, compute)


def conv1x1(x: np.ndarray, kernel: np.ndarray, compute: str) -> np.ndarray:
    """`einsum("bct,oc->bot")` with the `(out, in, 1)` kernel (dit.py:60-68), rounded once."""
    k = np.asarray(cast(kernel[:, :, 0], compute), F64)
    return cast(np.einsum("bct,oc->bot", np.asarray(x, F64), k), compute)


def expo_fourier(t: np.ndarray, dim: int, compute: str) -> np.ndarray:
    """`[cos | sin](2 pi t f)` with `f = exp(linspace(0, 1, dim/2) (ln 10000 - ln 0.5) + ln 0.5)` (dit.py:71-79),
    evaluated exactly (float64) from the fp32 `t` and rounded once to fp32, then to the compute dtype.

    The reference evaluates each step in fp32. At the high frequencies the angle reaches 2 pi * 10000 t, where one
    fp32 ulp of the frequency or of the angle moves cos / sin by up to |angle| * 2^-23 (about 7e-3 at t = 1):
    two fp32 evaluations of the same formula (XLA's, torch's) differ there by that much, so the oracle keeps the
    exact value and the checks of an fp32 evaluation against it allow that bound."""
    lin = np.arange(dim // 2, dtype=F64) / max(dim // 2 - 1, 1)
    freqs = np.exp(lin * (math.log(10000.0) - math.log(0.5)) + math.log(0.5))
    args = 2.0 * math.pi * np.asarray(t, np.float32).astype(F64)[:, None] * freqs
    return cast(np.concatenate([np.cos(args), np.sin(args)], axis=-1).astype(np.float32), compute)


def fourier_bound(t: np.ndarray, dim: int) -> np.ndarray:
    """Per-feature bound on an fp32 evaluation's distance from `expo_fourier`: a few ulps of the fp32 angle and
    frequency, |angle| * 2^-21, plus one fp32 ulp of the result."""
    lin = np.arange(dim // 2, dtype=F64) / max(dim // 2 - 1, 1)
    freqs = np.exp(lin * (math.log(10000.0) - math.log(0.5)) + math.log(0.5))
    angle = 2.0 * math.pi * np.abs(np.asarray(t, F64))[:, None] * freqs
    b = angle * 2.0 ** -21 + 2.0 ** -23
    return np.concatenate([b, b], axis=-1)


def add(a, b, compute: str) -> np.ndarray:
    return cast(np.asarray(a, F64) + np.asarray(b, F64), compute)


def mul(a, b, compute: str) -> np.ndarray:
    return cast(np.asarray(a, F64) * np.asarray(b, F64), compute)


def feed_forward(x: np.ndarray, ff: dict, compute: str) -> np.ndarray:
    """`value * silu(gate)` between `glu_proj` and `proj_out`, both with bias (dit.py:218-221)."""
    proj = linear(x, ff["glu_proj"]["weight"], ff["glu_proj"]["bias"], compute)
    value, gate = np.split(proj, 2, axis=-1)
    return linear(mul(value, silu(gate, compute), compute), ff["proj_out"]["weight"], ff["proj_out"]["bias"], compute)


def local_constants(blocks: list, compute: str) -> np.ndarray:
    """`(depth, E)`: `W2 silu(b1) + b2` per block (dit.py:254-271)."""
    return np.stack([linear(silu(cast(b["to_local_embed"]["in"]["bias"], compute), compute),
                            b["to_local_embed"]["out"]["weight"], b["to_local_embed"]["out"]["bias"], compute)
                     for b in blocks])


def block(h: np.ndarray, blk: dict, static: dict, gcond: np.ndarray, index: int, cfg, compute: str) -> np.ndarray:
    """One adaLN transformer block (dit.py:224-251)."""
    ssg = add(cast(blk["to_scale_shift_gate"], compute), gcond, compute)[:, None, :]
    scale_self, shift_self, gate_self, scale_ff, shift_ff, gate_ff = np.split(ssg, 6, axis=-1)
    one = 1.0

    x = rms(h, blk["pre_norm"]["weight"], cfg.norm_eps, compute)
    x = add(mul(x, add(one, scale_self, compute), compute), shift_self, compute)
    attn = blk["self_attn"]
    qkv = linear(x, attn["to_qkv"]["weight"], None, compute)
    out = odense.dense_xla(qkv, attn["q_norm"]["weight"], attn["k_norm"]["weight"], static["inv_freq"],
                           static["valid"], cfg.num_heads, cfg.head_dim, cfg.qk_norm_eps, None, compute)
    x = linear(out, attn["to_out"]["weight"], None, compute)
    h = add(h, mul(x, sigmoid(add(one, -np.asarray(gate_self, F64), compute), compute), compute), compute)

    x = rms(h, blk["cross_attend_norm"]["weight"], cfg.norm_eps, compute)
    cattn = blk["cross_attn"]
    q = linear(x, cattn["to_q"]["weight"], None, compute)
    out = ocross.cross_xla(q, static["cross_kv"][index], cattn["q_norm"]["weight"], cattn["k_norm"]["weight"],
                           cfg.num_heads, cfg.head_dim, cfg.qk_norm_eps, None, compute)
    h = add(h, linear(out, cattn["to_out"]["weight"], None, compute), compute)

    memory = cfg.num_memory_tokens
    h = h.copy()
    h[:, memory:, :] = add(h[:, memory:, :], static["local"][index], compute)

    x = rms(h, blk["ff_norm"]["weight"], cfg.norm_eps, compute)
    x = add(mul(x, add(one, scale_ff, compute), compute), shift_ff, compute)
    x = feed_forward(x, blk["ff"], compute)
    return add(h, mul(x, sigmoid(add(one, -np.asarray(gate_ff, F64), compute), compute), compute), compute)


def prepare_static(params: dict, cond: dict, padding_mask: np.ndarray, cfg, compute: str) -> dict:
    """Per-clip state (dit.py:304-337): the validity mask over memory + latent tokens, the RoPE `inv_freq`, each
    block's `to_kv` output over the projected context (the oracle's cross-attention prepares k/k_diff/v from it),
    the projected global condition and the local constants."""
    net = params["transformer"]
    batch = padding_mask.shape[0]
    valid = np.concatenate([np.ones((batch, cfg.num_memory_tokens), bool), np.asarray(padding_mask, bool)], axis=-1)
    ctx = sequential(params["to_cond_embed"], cast(cond["cross_attn_cond"], compute), compute)
    return {
        "valid": valid,
        "inv_freq": np.asarray(net["rope_inv_freq"], np.float32),
        "cross_kv": [linear(ctx, b["cross_attn"]["to_kv"]["weight"], None, compute) for b in net["blocks"]],
        "gcond_proj": sequential(params["to_global_embed"], cast(cond["global_cond"], compute), compute),
        "local": local_constants(net["blocks"], compute),
    }


def dit_forward(params: dict, x: np.ndarray, t: np.ndarray, static: dict, cfg, compute: str,
                features: np.ndarray | None = None) -> np.ndarray:
    """`(B, io, T)` latents and `(B,)` timesteps -> velocity (dit.py:340-361). `features` optionally replaces
    `expo_fourier(t)` (the `(B, fourier_dim)` timestep features in the compute dtype), so that a comparison with an
    fp32 evaluation of them can share one set."""
    net = params["transformer"]
    h = cast(x, compute)
    h = add(conv1x1(h, params["preprocess_conv"]["weight"], compute), h, compute)
    h = linear(np.swapaxes(h, 1, 2), net["project_in"]["weight"], None, compute)
    memory = np.broadcast_to(cast(net["memory_tokens"], compute), (h.shape[0], cfg.num_memory_tokens, cfg.embed_dim))
    h = np.concatenate([memory, h], axis=1)
    if features is None:
        features = expo_fourier(cast(t, compute), cfg.fourier_dim, compute)
    timestep = sequential(params["to_timestep_embed"], cast(features, compute), compute)
    gcond = sequential(net["global_cond_embedder"], add(static["gcond_proj"], timestep, compute), compute)
    for index, blk in enumerate(net["blocks"]):
        h = block(h, blk, static, gcond, index, cfg, compute)
    h = linear(h[:, cfg.num_memory_tokens:, :], net["project_out"]["weight"], None, compute)
    v = np.swapaxes(h, 1, 2)
    return add(conv1x1(v, params["postprocess_conv"]["weight"], compute), v, compute)


def build_schedule(steps: int, sigma_max: float, anchor_logsnr: float, logsnr_end: float) -> np.ndarray:
    """`(steps + 1,)` fp32 (sa3jax/sampling.py:65-78): the shifted sigmoid of a linear logSNR, endpoints pinned,
    `t[0] = sigma_max`. Each step in fp32."""
    f32 = np.float32
    t = np.linspace(sigma_max, 0.0, steps + 1, dtype=f32)
    logsnr = (f32(logsnr_end) - (t * f32(logsnr_end - anchor_logsnr)).astype(f32)).astype(f32)
    t_out = (1.0 / (1.0 + np.exp(logsnr.astype(F64)))).astype(f32)
    t_out = np.where(t <= 0.0, f32(0.0), t_out)
    t_out = np.where(t >= 1.0, f32(1.0), t_out)
    t_out[0] = sigma_max
    return t_out.astype(f32)


def pingpong(forward, x0: np.ndarray, schedule: np.ndarray, noise: np.ndarray, compute: str):
    """`(x_final, trajectory)` of the pingpong sampler (sa3jax/sampling.py:81-118): per step
    `v = forward(x, t_curr)`, `denoised = x - t_curr v`, `x = (1 - t_next) denoised + t_next noise[i]`, every
    step rounded to the compute dtype; the schedule is broadcast to `(B, steps + 1)` and cast first."""
    t = np.asarray(schedule, np.float32)
    if t.ndim == 1:
        t = np.broadcast_to(t, (x0.shape[0], t.shape[-1]))
    t = cast(t, compute)
    x = cast(x0, compute)
    vs = []
    for i in range(t.shape[-1] - 1):
        tc, tn = t[:, i][:, None, None], t[:, i + 1][:, None, None]
        v = forward(x, t[:, i])
        denoised = add(x, -mul(tc, v, compute).astype(F64), compute)
        x = add(mul(add(1.0, -tn.astype(F64), compute), denoised, compute), mul(tn, cast(noise[i], compute), compute),
                compute)
        vs.append(v)
    return x, np.stack(vs)
