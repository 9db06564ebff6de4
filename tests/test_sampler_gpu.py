"""The denoiser and the sampler loop on the GPU with attention="hip" (reference: sa3jax/dit.py:287-361,
sa3jax/sampling.py:81-118).

* the denoiser (a 2-block DiT with 2 heads of 64) in fp32 against the oracle, and three sampler steps likewise
  (tolerance: 2e-5 of the output's largest magnitude; the attention calls alone hold 1e-5 relative, the GEMMs,
  norms and residuals around them add fp32 rounding of the same order);
* the `medium` geometry (width 1536, 24 heads, 2 blocks, 300 latents, batch 2) under the BF16 and FP16 presets
  against attention="xla" on the same device, with hipBLASLt and with this package's projection GEMMs, at the bf16
  contract applied to the output divided by its largest magnitude;
* the whole sampler loop captured as a HIP graph against the eager loop: bit-identical on three replays with new
  inputs, with eager work and synchronisations in between.
The timestep features are shared between the mirror and the oracle (oracle.dit.expo_fourier explains why).
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from hummingbird_amd import dit, sampling
from hummingbird_amd.config import MEDIUM_DIT
from hummingbird_amd.dtypes import BF16, FP16, FP32_PARITY
from oracle import dit as odit
from tests.test_sampler import TINY, cond_case, to_np
from tests.util import assert_bf16_parity, stats

pytestmark = pytest.mark.gpu
DEV = "cuda"
HIP_TINY = dataclasses.replace(TINY, attention="hip")


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def dev(tree):
    if isinstance(tree, dict):
        return {k: dev(v) for k, v in tree.items()}
    if isinstance(tree, list):
        return [dev(v) for v in tree]
    return tree.to(DEV)


def case(cfg, dtype, batch, tokens, seed=21, ctx_tokens=9):
    params = dit.init_params(cfg, dtype, device=DEV, seed=seed)
    cond, mask, x = cond_case(cfg, batch, tokens, seed, ctx_tokens)
    return params, dev(cond), mask.to(DEV), x.to(DEV)


def oracle_forward(np_params, ostatic, cfg, compute):
    def forward(xx, tc):
        feats = dit.expo_fourier(torch.from_numpy(np.array(tc)), cfg.fourier_dim).numpy()
        return odit.dit_forward(np_params, xx, tc, ostatic, cfg, compute, features=feats)
    return forward


def test_dit_forward_hip_fp32_vs_oracle():
    announce("dit_forward hip fp32 vs oracle (2 blocks, 2 heads)")
    cfg = HIP_TINY
    params, cond, mask, x = case(cfg, FP32_PARITY, 2, 40)
    t = torch.tensor([0.9, 0.35], device=DEV)
    static = dit.prepare_static(params, cond, mask, cfg, FP32_PARITY)
    got = dit.dit_forward(params, x, t, static, cfg, FP32_PARITY).cpu().numpy()
    np_params = to_np(params)
    ostatic = odit.prepare_static(np_params, to_np(cond), mask.cpu().numpy(), cfg, "fp32")
    ref = oracle_forward(np_params, ostatic, cfg, "fp32")(x.cpu().numpy(), t.cpu().numpy())
    s = stats(got, ref)
    assert s["max_abs"] <= 2e-5 * float(np.abs(ref).max()), s


def test_sampler_hip_fp32_vs_oracle():
    announce("pingpong 3 steps hip fp32 vs oracle")
    cfg = HIP_TINY
    params, cond, mask, x = case(cfg, FP32_PARITY, 1, 24, seed=22)
    noise = torch.randn((3, 1, cfg.io_channels, 24), generator=torch.Generator().manual_seed(23)).to(DEV)
    schedule = sampling.build_schedule(3, device=DEV)
    static = dit.prepare_static(params, cond, mask, cfg, FP32_PARITY)
    got, traj = sampling.pingpong(params, x, schedule, noise, static, cfg, FP32_PARITY)
    np_params = to_np(params)
    ostatic = odit.prepare_static(np_params, to_np(cond), mask.cpu().numpy(), cfg, "fp32")
    ref, ref_traj = odit.pingpong(oracle_forward(np_params, ostatic, cfg, "fp32"), x.cpu().numpy(),
                                  schedule.cpu().numpy(), noise.cpu().numpy(), "fp32")
    assert stats(got.cpu().numpy(), ref)["max_abs"] <= 2e-5 * float(np.abs(ref).max())
    assert stats(traj.cpu().numpy(), ref_traj)["max_abs"] <= 2e-5 * float(np.abs(ref_traj).max())


MEDIUM2 = dataclasses.replace(MEDIUM_DIT, depth=2)


@pytest.mark.parametrize("projections,preset", [("torch", "bf16"), ("hip", "bf16"), ("torch", "fp16"),
                                                ("hip", "fp16")])
def test_dit_forward_medium_hip_vs_xla(projections, preset):
    announce(f"dit_forward medium {preset} hip ({projections} projections) vs xla")
    dtype = {"bf16": BF16, "fp16": FP16}[preset]
    params, cond, mask, x = case(MEDIUM2, dtype, 2, 300, seed=24, ctx_tokens=257)
    t = torch.tensor([0.9, 0.35], device=DEV)
    static = dit.prepare_static(params, cond, mask, MEDIUM2, dtype)
    got = dit.dit_forward(params, x, t, static, MEDIUM2, dtype, projections=projections).float().cpu().numpy()
    xcfg = dataclasses.replace(MEDIUM2, attention="xla")
    xstatic = dit.prepare_static(params, cond, mask, xcfg, dtype)
    ref = dit.dit_forward(params, x, t, xstatic, xcfg, dtype).float().cpu().numpy()
    scale = float(np.abs(ref).max())
    assert_bf16_parity(got / scale, ref / scale, f"medium dit_forward {preset} ({projections}) / max")


@pytest.mark.parametrize("projections", ["torch", "hip"])
def test_sampler_graph_replays_equal_the_eager_loop(projections):
    announce(f"PingpongGraph vs eager pingpong ({projections} projections)")
    params, cond, mask, x = case(MEDIUM2, BF16, 1, 200, seed=25, ctx_tokens=257)
    static = dit.prepare_static(params, cond, mask, MEDIUM2, BF16)
    gen = torch.Generator().manual_seed(26)
    noise = torch.randn((3, 1, MEDIUM2.io_channels, 200), generator=gen).to(DEV)
    graph = sampling.PingpongGraph(params, static, MEDIUM2, BF16, x, noise, projections=projections)
    schedule = sampling.build_schedule(3, device=DEV)
    for rep in range(3):
        x_r = torch.randn(x.shape, generator=gen).to(DEV)
        n_r = torch.randn(noise.shape, generator=gen).to(DEV)
        got = graph(x_r, n_r).clone()
        torch.cuda.synchronize()
        ref, _ = sampling.pingpong(params, x_r, schedule, n_r, static, MEDIUM2, BF16, trajectory=False,
                                   projections=projections)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"replay {rep}: {stats(got.float().cpu().numpy(), ref.float().cpu().numpy())}"
        _ = (torch.randn(1000, device=DEV) * 2).sum().item()  # unrelated eager work between replays


def test_tuned_gemms_keep_parity_and_graph_replays():
    """After sampling.tune_gemms (TunableOp picks each GEMM's solution) the medium denoiser still matches the XLA
    chain at the contract, and a graph captured afterwards replays bit-identically to the eager loop."""
    announce("tune_gemms: parity and graph replay")
    params, cond, mask, x = case(MEDIUM2, BF16, 1, 200, seed=27, ctx_tokens=257)
    static = dit.prepare_static(params, cond, mask, MEDIUM2, BF16)
    noise = torch.randn((2, 1, MEDIUM2.io_channels, 200), generator=torch.Generator().manual_seed(28)).to(DEV)
    schedule = sampling.build_schedule(2, device=DEV)

    def eager():
        return sampling.pingpong(params, x, schedule, noise, static, MEDIUM2, BF16, trajectory=False)[0]
    try:
        sampling.tune_gemms(eager)
        assert torch.cuda.tunable.is_enabled() and not torch.cuda.tunable.tuning_is_enabled()
        t = torch.tensor([0.7], device=DEV)
        got = dit.dit_forward(params, x, t, static, MEDIUM2, BF16).float().cpu().numpy()
        xcfg = dataclasses.replace(MEDIUM2, attention="xla")
        ref = dit.dit_forward(params, x, t, dit.prepare_static(params, cond, mask, xcfg, BF16), xcfg,
                              BF16).float().cpu().numpy()
        scale = float(np.abs(ref).max())
        assert_bf16_parity(got / scale, ref / scale, "tuned medium dit_forward / max")
        graph = sampling.PingpongGraph(params, static, MEDIUM2, BF16, x, noise)
        for _ in range(2):
            out = graph(x, noise).clone()
            torch.cuda.synchronize()
            assert torch.equal(out, eager())
    finally:
        torch.cuda.tunable.tuning_enable(False)
        torch.cuda.tunable.enable(False)
