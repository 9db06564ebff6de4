"""The sampler loop and the denoiser around the attention path, on the CPU (reference: sa3jax/sampling.py:65-118,
sa3jax/dit.py:31-79, 218-361).

How the oracle (oracle/dit.py) is pinned:
* the schedule against the values the reference documents for the shipped sampler (steps 8, sigma_max 1, the
  LogSNR shift -6.2 / 2.0): t[1] rounds to 0.99609375 in bf16 and to 0.994140625 in half
  (sa3jax/sampling.py:17-20); its end points, the sigma_max re-anchoring, and the constant-logSNR special case;
* the pingpong step against closed forms with a stub denoiser (v = 0, v = x), and the reference's statement
  that the last step's noise is multiplied away;
* the timestep features against their end-point frequencies (0.5 and 10000) and the [cos | sin] order;
* the 1x1 convolution's orientation against a brute-force sum; the depth-0 denoiser against a float64
  composition of its four linear maps;
* the adaLN block against known cases: a block whose branches cancel exactly is the identity; the local constant
  lands on the latent tokens only; the gate is sigmoid(1 - gate); the scale / shift modulation
  `x (1 + scale) + shift` through a feed-forward that is exactly the identity.
Each known case is also shown to tell a plausible mistake apart (sigmoid(gate), the local constant on every token,
a transposed convolution, no re-anchoring, x * scale instead of x * (1 + scale), [sin | cos]).
The torch mirror (hummingbird_amd.dit / .sampling, attention="xla") is then checked against the pinned oracle.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np
import pytest
import torch

from hummingbird_amd import dit, sampling
from hummingbird_amd.config import ANCHOR_LOGSNR, LOGSNR_END, DiTConfig
from hummingbird_amd.dtypes import BF16, FP32_PARITY
from oracle import bf16 as obf16
from oracle import dit as odit
from tests.util import assert_bf16_parity, stats

TINY = DiTConfig(io_channels=16, embed_dim=128, depth=2, num_heads=2, cond_token_dim=24, global_cond_dim=20,
                 local_add_cond_dim=12, num_memory_tokens=4, ff_mult=2.0, differential=True, fourier_dim=16,
                 attention="xla")


def to_np(tree):
    if isinstance(tree, dict):
        return {k: to_np(v) for k, v in tree.items()}
    if isinstance(tree, list):
        return [to_np(v) for v in tree]
    return tree.detach().cpu().float().numpy() if tree.is_floating_point() else tree.cpu().numpy()


def cond_case(cfg: DiTConfig, batch: int, tokens: int, seed: int = 3, ctx_tokens: int = 9):
    gen = torch.Generator().manual_seed(seed)
    cond = {"cross_attn_cond": torch.randn((batch, ctx_tokens, cfg.cond_token_dim), generator=gen),
            "global_cond": torch.randn((batch, cfg.global_cond_dim), generator=gen)}
    mask = torch.ones((batch, tokens), dtype=torch.bool)
    mask[-1, tokens - 5:] = False
    x = torch.randn((batch, cfg.io_channels, tokens), generator=gen)
    return cond, mask, x


# ---------------------------------------------------------------------------------------------------------------
# schedule

@pytest.mark.parametrize("impl", ["oracle", "torch"])
def test_schedule_matches_the_documented_values(impl):
    t = (odit.build_schedule(8, 1.0, ANCHOR_LOGSNR, LOGSNR_END) if impl == "oracle"
         else sampling.build_schedule(8).numpy())
    assert t.dtype == np.float32 and t.shape == (9,)
    assert t[0] == 1.0 and t[-1] == 0.0
    assert float(obf16.round_bf16(t[1:2])[0]) == 0.99609375   # sa3jax/sampling.py:19
    assert float(obf16.round_fp16(t[1:2])[0]) == 0.994140625  # "0.994141"
    assert np.all(np.diff(t) < 0)


def test_schedule_reanchors_and_constant_logsnr():
    t = odit.build_schedule(8, 0.8, ANCHOR_LOGSNR, LOGSNR_END)
    assert t[0] == np.float32(0.8)  # re-anchored: the shifted value there would be sigmoid(4.56) = 0.9897
    flat = odit.build_schedule(4, 1.0, 2.0, 2.0)  # logsnr constant at 2: interior points are sigmoid(-2)
    np.testing.assert_allclose(flat[1:-1], 1 / (1 + math.exp(2.0)), rtol=1e-6)
    np.testing.assert_allclose(sampling.build_schedule(8, 0.8).numpy(), t, rtol=2.5e-7)  # fp32 sigmoid ulps


def test_planted_schedule_without_reanchor_fails():
    f32 = np.float32
    t = np.linspace(0.8, 0.0, 9, dtype=f32)
    wrong = (1 / (1 + np.exp(f32(2.0) - t * f32(8.2)))).astype(f32)
    assert wrong[0] != f32(0.8)


# ---------------------------------------------------------------------------------------------------------------
# pingpong step

def test_pingpong_closed_forms():
    rng = np.random.default_rng(0)
    x0 = rng.standard_normal((2, 3, 5)).astype(np.float32)
    noise = rng.standard_normal((8, 2, 3, 5)).astype(np.float32)
    t = odit.build_schedule(8, 1.0, ANCHOR_LOGSNR, LOGSNR_END).astype(np.float64)
    # v = 0: x_{i+1} = (1 - t_{i+1}) x_i + t_{i+1} eps_i
    x, traj = odit.pingpong(lambda x, tc: np.zeros_like(x), x0, t, noise, "fp32")
    ref = x0.astype(np.float64)
    for i in range(8):
        ref = (1 - t[i + 1]) * ref + t[i + 1] * noise[i]
    np.testing.assert_allclose(x, ref, rtol=1e-5, atol=1e-6)
    assert traj.shape == (8, 2, 3, 5) and not traj.any()
    # v = x: denoised = (1 - t_i) x
    x, _ = odit.pingpong(lambda x, tc: x, x0, t, noise, "fp32")
    ref = x0.astype(np.float64)
    for i in range(8):
        ref = (1 - t[i + 1]) * (1 - t[i]) * ref + t[i + 1] * noise[i]
    np.testing.assert_allclose(x, ref, rtol=1e-5, atol=1e-6)


def test_pingpong_last_noise_is_multiplied_away():
    rng = np.random.default_rng(1)
    x0 = rng.standard_normal((1, 2, 4)).astype(np.float32)
    noise = rng.standard_normal((8, 1, 2, 4)).astype(np.float32)
    fwd = lambda x, tc: np.tanh(x) * tc[:, None, None]  # noqa: E731
    t = odit.build_schedule(8, 1.0, ANCHOR_LOGSNR, LOGSNR_END)
    a, _ = odit.pingpong(fwd, x0, t, noise, "bf16")
    noise[-1] = 1e3
    b, _ = odit.pingpong(fwd, x0, t, noise, "bf16")
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("compute", ["fp32", "bf16"])
def test_torch_pingpong_equals_oracle_with_a_stub_denoiser(compute):
    """The per-step arithmetic, cast points included, is bit-identical between the torch loop and the oracle."""
    rng = np.random.default_rng(2)
    x0 = rng.standard_normal((2, 3, 6)).astype(np.float32)
    noise = rng.standard_normal((8, 2, 3, 6)).astype(np.float32)
    dtype = FP32_PARITY if compute == "fp32" else BF16

    def stub(params, x, t, static, cfg, dt, projections="torch"):  # v = x t + 1/4, each step rounded
        return x * t[:, None, None] + 0.25
    got, traj = sampling.pingpong(None, torch.from_numpy(x0), sampling.build_schedule(8), torch.from_numpy(noise),
                                  None, TINY, dtype, forward=stub)
    ref, ref_traj = odit.pingpong(lambda x, tc: odit.add(odit.mul(x, tc[:, None, None], compute), 0.25, compute),
                                  x0, sampling.build_schedule(8).numpy(), noise, compute)
    np.testing.assert_array_equal(got.float().numpy(), ref)
    np.testing.assert_array_equal(traj.float().numpy(), ref_traj)


# ---------------------------------------------------------------------------------------------------------------
# timestep features, convolution, depth-0 denoiser

def test_expo_fourier_end_frequencies():
    dim = 16
    zero = odit.expo_fourier(np.zeros(1, np.float32), dim, "fp32")[0]
    np.testing.assert_array_equal(zero, np.r_[np.ones(dim // 2), np.zeros(dim // 2)])  # [cos | sin] at t = 0
    half = odit.expo_fourier(np.array([0.5], np.float32), dim, "fp32")[0]
    assert abs(half[0]) < 1e-6 and abs(half[dim // 2] - 1) < 1e-6     # f0 = 0.5: angle pi / 2
    last = odit.expo_fourier(np.array([1 / 40000], np.float32), dim, "fp32")[0]
    assert abs(last[dim // 2 - 1]) < 1e-4 and abs(last[-1] - 1) < 1e-6  # f_last = 10000: angle pi / 2
    t = np.array([0.0, 0.5, 1 / 40000, 0.35, 0.9, 1.0], np.float32)
    got = dit.expo_fourier(torch.from_numpy(t), dim).numpy()  # fp32 steps, as the reference evaluates them
    diff = np.abs(got - odit.expo_fourier(t, dim, "fp32"))
    assert (diff <= odit.fourier_bound(t, dim)).all(), diff.max()
    planted = np.concatenate([np.sin(2 * np.pi * t[:, None] * 0.5), np.cos(2 * np.pi * t[:, None] * 0.5)], -1)
    assert not np.allclose(odit.expo_fourier(t, 2, "fp32"), planted, atol=1e-3)  # [sin | cos] order


def test_conv1x1_orientation():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 5)).astype(np.float32)
    k = rng.standard_normal((4, 3, 1)).astype(np.float32)
    brute = np.zeros((2, 4, 5))
    for b in range(2):
        for o in range(4):
            for t in range(5):
                brute[b, o, t] = sum(float(k[o, c, 0]) * float(x[b, c, t]) for c in range(3))
    np.testing.assert_allclose(odit.conv1x1(x, k, "fp32"), brute, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(dit.conv1x1(torch.from_numpy(x), torch.from_numpy(k)).numpy(), brute, rtol=1e-5,
                               atol=1e-6)
    square = rng.standard_normal((3, 3, 1)).astype(np.float32)
    planted = np.einsum("bct,co->bot", x.astype(np.float64), square[:, :, 0].astype(np.float64))  # transposed
    assert not np.allclose(odit.conv1x1(x, square, "fp32"), planted, atol=1e-3)


def test_depth0_denoiser_is_its_linear_maps():
    cfg = dataclasses.replace(TINY, depth=0)
    params = to_np(dit.init_params(cfg, FP32_PARITY, seed=5))
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, cfg.io_channels, 7)).astype(np.float32)
    static = {"gcond_proj": np.zeros((2, cfg.embed_dim), np.float32)}
    got = odit.dit_forward(params, x, np.array([0.3, 0.7], np.float32), static, cfg, "fp32")
    pre = params["preprocess_conv"]["weight"][:, :, 0].astype(np.float64)
    post = params["postprocess_conv"]["weight"][:, :, 0].astype(np.float64)
    p_in = params["transformer"]["project_in"]["weight"].astype(np.float64)
    p_out = params["transformer"]["project_out"]["weight"].astype(np.float64)
    eye = np.eye(cfg.io_channels)
    ref = np.einsum("oc,bct->bot", (post + eye) @ p_out @ p_in @ (pre + eye), x.astype(np.float64))
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------------------------------------------------------
# the adaLN block

def cancelling_block(cfg: DiTConfig, seed: int = 6) -> dict:
    """Random block whose three branches are exactly zero: q_diff/k_diff rows equal q/k rows (self and cross;
    the two softmaxes are then identical and the differential output is 0), and the feed-forward's and the
    local embedding's output layers are zero."""
    blk = to_np(dit.init_params(dataclasses.replace(cfg, depth=1), FP32_PARITY, seed=seed))["transformer"]["blocks"][0]
    E = cfg.embed_dim
    qkv = blk["self_attn"]["to_qkv"]["weight"]
    qkv[3 * E:4 * E], qkv[4 * E:5 * E] = qkv[0:E], qkv[E:2 * E]
    blk["cross_attn"]["to_q"]["weight"][E:] = blk["cross_attn"]["to_q"]["weight"][:E]
    blk["cross_attn"]["to_kv"]["weight"][E:2 * E] = blk["cross_attn"]["to_kv"]["weight"][:E]
    for layer in (blk["ff"]["proj_out"], blk["to_local_embed"]["out"]):
        layer["weight"][:] = 0
        layer["bias"][:] = 0
    return blk


def block_static(cfg: DiTConfig, blk: dict, batch: int, tokens: int, seed: int = 7) -> dict:
    rng = np.random.default_rng(seed)
    ctx = rng.standard_normal((batch, 5, cfg.embed_dim)).astype(np.float32)
    return {"valid": np.ones((batch, cfg.num_memory_tokens + tokens), bool),
            "inv_freq": np.asarray(dit.init_params(dataclasses.replace(cfg, depth=0), FP32_PARITY)["transformer"]
                                   ["rope_inv_freq"].numpy()),
            "cross_kv": [odit.linear(ctx, blk["cross_attn"]["to_kv"]["weight"], None, "fp32")],
            "local": odit.local_constants([blk], "fp32")}


def test_block_with_cancelling_branches_is_the_identity():
    cfg = TINY
    blk = cancelling_block(cfg)
    h = np.random.default_rng(8).standard_normal((2, cfg.num_memory_tokens + 6, cfg.embed_dim)).astype(np.float32)
    static = block_static(cfg, blk, 2, 6)
    gcond = np.random.default_rng(9).standard_normal((2, cfg.adaln_dim)).astype(np.float32)
    np.testing.assert_array_equal(odit.block(h, blk, static, gcond, 0, cfg, "fp32"), h)


def test_block_local_constant_lands_on_latent_tokens_only():
    cfg = TINY
    blk = cancelling_block(cfg)
    blk["to_local_embed"]["out"]["bias"][:] = 0.25
    h = np.random.default_rng(8).standard_normal((1, cfg.num_memory_tokens + 6, cfg.embed_dim)).astype(np.float32)
    static = block_static(cfg, blk, 1, 6)
    out = odit.block(h, blk, static, np.zeros((1, cfg.adaln_dim), np.float32), 0, cfg, "fp32")
    M = cfg.num_memory_tokens
    np.testing.assert_array_equal(out[:, :M], h[:, :M])
    np.testing.assert_array_equal(out[:, M:], (h[:, M:] + np.float32(0.25)).astype(np.float32))
    planted = h + np.float32(0.25)  # the local constant on every token
    assert not np.array_equal(out, planted)


def test_block_gate_is_sigmoid_of_one_minus_gate():
    cfg = TINY
    blk = cancelling_block(cfg)
    E = cfg.embed_dim
    blk["ff"]["proj_out"]["bias"][:] = 0.5  # the feed-forward outputs the constant 0.5
    g = 2.0
    blk["to_scale_shift_gate"][:] = 0
    blk["to_scale_shift_gate"][5 * E:] = g
    h = np.random.default_rng(10).standard_normal((1, cfg.num_memory_tokens + 3, E)).astype(np.float32)
    static = block_static(cfg, blk, 1, 3)
    out = odit.block(h, blk, static, np.zeros((1, cfg.adaln_dim), np.float32), 0, cfg, "fp32")
    expect = h.astype(np.float64) + 0.5 / (1 + math.exp(-(1 - g)))  # sigmoid(1 - 2) = 0.2689
    np.testing.assert_allclose(out, expect, rtol=1e-6, atol=1e-6)
    planted = h.astype(np.float64) + 0.5 / (1 + math.exp(-g))  # sigmoid(gate): 0.8808
    assert not np.allclose(out, planted, atol=1e-2)


def test_block_modulation_through_an_identity_feed_forward():
    """glu_proj's value rows are the identity and its gate rows are 0 with bias 32 (silu(32) = 32 exactly in
    fp32), proj_out is I / 32: the feed-forward is exactly the identity, so the block adds
    `(rms(h) (1 + scale) + shift) * sigmoid(1 - gate)` for the feed-forward's adaLN slices."""
    cfg = TINY
    E, F = cfg.embed_dim, cfg.ff_inner
    blk = cancelling_block(cfg)
    glu = blk["ff"]["glu_proj"]
    glu["weight"][:] = 0
    glu["weight"][:E, :E] = np.eye(E)
    glu["bias"][:] = 0
    glu["bias"][F:] = 32.0
    blk["ff"]["proj_out"]["weight"][:] = 0
    blk["ff"]["proj_out"]["weight"][:, :E] = np.eye(E) / 32
    blk["ff_norm"]["weight"][:] = 1
    s, sh, g = 0.5, 0.125, -1.0
    ssg = np.zeros(6 * E, np.float32)
    ssg[3 * E:4 * E], ssg[4 * E:5 * E], ssg[5 * E:] = s, sh, g
    blk["to_scale_shift_gate"] = ssg
    rng = np.random.default_rng(11)
    h = np.where(rng.random((1, cfg.num_memory_tokens + 3, E)) < 0.5, -1.0, 1.0).astype(np.float32)  # mean(h^2) = 1
    static = block_static(cfg, blk, 1, 3)
    out = odit.block(h, blk, static, np.zeros((1, cfg.adaln_dim), np.float32), 0, cfg, "fp32")
    r = 1 / math.sqrt(1 + cfg.norm_eps)
    gate = 1 / (1 + math.exp(-(1 - g)))
    expect = h + (h * r * (1 + s) + sh) * gate
    np.testing.assert_allclose(out, expect, rtol=2e-6, atol=2e-6)
    planted = h + (h * r * s + sh) * gate  # x * scale
    assert not np.allclose(out, planted, atol=1e-2)


def test_prepare_static_rejects_a_nonzero_local_condition():
    params = dit.init_params(dataclasses.replace(TINY, depth=1), FP32_PARITY)
    cond, mask, _ = cond_case(TINY, 1, 6)
    cond["local_add_cond"] = torch.zeros((1, TINY.local_add_cond_dim, 6))
    dit.prepare_static(params, cond, mask, dataclasses.replace(TINY, depth=1), FP32_PARITY)
    cond["local_add_cond"][0, 0, 0] = 1
    with pytest.raises(ValueError, match="local_add_cond"):
        dit.prepare_static(params, cond, mask, dataclasses.replace(TINY, depth=1), FP32_PARITY)


# ---------------------------------------------------------------------------------------------------------------
# the torch mirror against the oracle

def forward_case(cfg: DiTConfig, dtype, batch=2, tokens=20, seed=12):
    params = dit.init_params(cfg, dtype, seed=seed)
    cond, mask, x = cond_case(cfg, batch, tokens, seed)
    t = torch.tensor([0.9, 0.35][:batch])
    return params, cond, mask, x, t


def test_dit_forward_xla_mirror_vs_oracle_fp32():
    cfg = TINY
    params, cond, mask, x, t = forward_case(cfg, FP32_PARITY)
    static = dit.prepare_static(params, cond, mask, cfg, FP32_PARITY)
    got = dit.dit_forward(params, x, t, static, cfg, FP32_PARITY).numpy()
    np_params = to_np(params)
    ostatic = odit.prepare_static(np_params, to_np(cond), mask.numpy(), cfg, "fp32")
    feats = dit.expo_fourier(t, cfg.fourier_dim).numpy()
    ref = odit.dit_forward(np_params, x.numpy(), t.numpy(), ostatic, cfg, "fp32", features=feats)
    s = stats(got, ref)
    assert s["max_abs"] <= 1e-5 * max(1.0, float(np.abs(ref).max())), s


def test_dit_forward_xla_mirror_vs_oracle_bf16():
    cfg = TINY
    params, cond, mask, x, t = forward_case(cfg, BF16)
    static = dit.prepare_static(params, cond, mask, cfg, BF16)
    got = dit.dit_forward(params, x, t, static, cfg, BF16).float().numpy()
    np_params = to_np(params)
    ostatic = odit.prepare_static(np_params, to_np(cond), mask.numpy(), cfg, "bf16")
    feats = dit.expo_fourier(t.to(torch.bfloat16), cfg.fourier_dim).float().numpy()
    ref = odit.dit_forward(np_params, x.numpy(), t.numpy(), ostatic, cfg, "bf16", features=feats)
    scale = float(np.abs(ref).max())
    assert_bf16_parity(got / scale, ref / scale, "dit_forward bf16 (normalised by max)")


def test_sampler_xla_mirror_vs_oracle_fp32():
    cfg = TINY
    params, cond, mask, x, _ = forward_case(cfg, FP32_PARITY, batch=1, tokens=12)
    noise = torch.randn((3, 1, cfg.io_channels, 12), generator=torch.Generator().manual_seed(13))
    schedule = sampling.build_schedule(3)
    static = dit.prepare_static(params, cond, mask, cfg, FP32_PARITY)
    got, traj = sampling.pingpong(params, x, schedule, noise, static, cfg, FP32_PARITY)
    np_params = to_np(params)
    ostatic = odit.prepare_static(np_params, to_np(cond), mask.numpy(), cfg, "fp32")
    def forward(xx, tc):
        feats = dit.expo_fourier(torch.from_numpy(np.array(tc)), cfg.fourier_dim).numpy()
        return odit.dit_forward(np_params, xx, tc, ostatic, cfg, "fp32", features=feats)
    ref, ref_traj = odit.pingpong(forward, x.numpy(), schedule.numpy(), noise.numpy(), "fp32")
    assert stats(got.numpy(), ref)["max_abs"] <= 2e-5 * float(np.abs(ref).max())
    assert stats(traj.numpy(), ref_traj)["max_abs"] <= 2e-5 * float(np.abs(ref_traj).max())
