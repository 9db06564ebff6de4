"""The sampler loop that drives the DiT attention calls: the LogSNR-shift schedule and the pingpong sampler
(sa3jax/sampling.py:65-118), plus `PingpongGraph`, the whole loop captured once as a HIP graph.

One clip is `steps` denoiser evaluations (8 for the shipped sampler), each `depth` blocks, so 8 x 24 = 192 dense
self-attention calls and as many cross-attention calls for the `medium` DiT. Per-clip state (tables, prepared
cross-attention contexts, the attention workspace) comes from `dit.prepare_static` and is reused by every step.

The reference runs the loop as one `lax.scan` with the carry `x` and per-step slices of the schedule and the
noise (sa3jax/sampling.py:107-118). Here the eager form is a Python loop over the same per-step arithmetic, and
`PingpongGraph` records all of its launches into one HIP graph with static input and output buffers, so a clip
is one graph launch: no host work per step or per block, the same fixed shapes the scan requires.
"""
from __future__ import annotations

from typing import Callable

import torch

from hummingbird_amd import dit
from hummingbird_amd.config import ANCHOR_LOGSNR, LOGSNR_END, SIGMA_MAX, DiTConfig
from hummingbird_amd.dtypes import Dtype

Forward = Callable[..., torch.Tensor]


def build_schedule(steps: int, sigma_max: float = SIGMA_MAX, anchor_logsnr: float = ANCHOR_LOGSNR,
                   logsnr_end: float = LOGSNR_END, device=None) -> torch.Tensor:
    """`(steps + 1,)` fp32 timesteps (sa3jax/sampling.py:65-78): `t = linspace(sigma_max, 0)`, `logsnr =
    logsnr_end - t (logsnr_end - anchor_logsnr)`, `t_out = sigmoid(-logsnr)`, pinned to 0 where `t <= 0` and to
    1 where `t >= 1`, and `t_out[0] = sigma_max`."""
    f32 = torch.float32
    t = torch.linspace(sigma_max, 0.0, steps + 1, dtype=f32, device=device)
    t_out = torch.sigmoid(-(logsnr_end - t * (logsnr_end - anchor_logsnr)))
    t_out = torch.where(t <= 0.0, torch.zeros_like(t_out), t_out)
    t_out = torch.where(t >= 1.0, torch.ones_like(t_out), t_out)
    t_out[0] = sigma_max
    return t_out


def _per_element(schedule: torch.Tensor, batch: int, latent: torch.dtype) -> torch.Tensor:
    """`(B, steps + 1)` in the latent dtype: a 1-D schedule is broadcast over the batch, then cast, as the
    reference does before the DiT sees it (sa3jax/sampling.py:99-104)."""
    t = schedule
    if t.dim() == 1:
        t = t.expand(batch, t.shape[-1])
    return t.to(latent)


def _step(x: torch.Tensor, v: torch.Tensor, t_curr: torch.Tensor, t_next: torch.Tensor,
          eps: torch.Tensor) -> torch.Tensor:
    """`denoised = x - t_curr v`, `x_next = (1 - t_next) denoised + t_next eps` (sa3jax/sampling.py:109-114)."""
    denoised = x - t_curr[:, None, None] * v
    return (1 - t_next[:, None, None]) * denoised + t_next[:, None, None] * eps


def pingpong(params: dict, x0: torch.Tensor, schedule: torch.Tensor, noise: torch.Tensor, static: dict,
             cfg: DiTConfig, dtype: Dtype, *, trajectory: bool = True, forward: Forward | None = None,
             projections: str = "torch") -> tuple[torch.Tensor, torch.Tensor | None]:
    """`(x_final, velocity trajectory)` of the pingpong sampler (sa3jax/sampling.py:81-118).

    `x0` `(B, io_channels, T)` and `noise` `(steps, B, io_channels, T)` are cast to the compute dtype;
    `schedule` is `(steps + 1,)` or `(B, steps + 1)`. The trajectory is `(steps, B, io_channels, T)` of the
    per-step velocities, or None with `trajectory=False`. `forward` replaces `dit.dit_forward` (same
    arguments); `projections` is passed to it."""
    forward = forward or dit.dit_forward
    latent = dtype.compute
    t = _per_element(schedule, x0.shape[0], latent)
    steps = t.shape[-1] - 1
    if noise.shape[0] != steps:
        raise ValueError(f"noise has {noise.shape[0]} steps, the schedule {steps}")
    x = x0.to(latent)
    vs = []
    for i in range(steps):
        v = forward(params, x, t[:, i], static, cfg, dtype, projections=projections)
        x = _step(x, v, t[:, i], t[:, i + 1], noise[i].to(latent))
        if trajectory:
            vs.append(v)
    return x, (torch.stack(vs) if trajectory else None)


class PingpongGraph:
    """The whole sampler loop for one clip shape as one HIP graph (`torch.cuda.CUDAGraph` on ROCm).

    Built for fixed `(steps, B, io_channels, T)`, weights and per-clip `static` (the graph reads them where they
    lie, so they must stay alive and unchanged). `__call__(x0, noise)` copies the inputs into the graph's
    static buffers, replays the graph on the current stream and returns the final latents in the graph's
    static output buffer (overwritten by the next call: clone it to keep it). The schedule is fixed at
    construction. Every launch of `pingpong` is recorded: the denoiser's GEMMs and elementwise work, the
    attention kernels (their workspaces come from `static`), and the sampler arithmetic.
    """

    def __init__(self, params: dict, static: dict, cfg: DiTConfig, dtype: Dtype, x0: torch.Tensor,
                 noise: torch.Tensor, schedule: torch.Tensor | None = None, *, projections: str = "torch",
                 warmup: int = 1):
        latent = dtype.compute
        steps = noise.shape[0]
        dev = x0.device
        if schedule is None:
            schedule = build_schedule(steps, device=dev)
        self.x0 = x0.to(latent).clone()
        self.noise = noise.to(latent).clone()
        self.schedule = _per_element(schedule.to(dev), x0.shape[0], latent).contiguous()

        def run():
            out, _ = pingpong(params, self.x0, self.schedule, self.noise, static, cfg, dtype, trajectory=False,
                              projections=projections)
            return out

        # The first launches initialise library state (GEMM handles, kernel modules) outside the capture.
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                run()
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = run()

    def __call__(self, x0: torch.Tensor, noise: torch.Tensor) -> torch.Tensor:
        self.x0.copy_(x0)
        self.noise.copy_(noise)
        self.graph.replay()
        return self.out


def tune_gemms(run: Callable[[], object], filename: str | None = None) -> None:
    """Let PyTorch's TunableOp pick, per GEMM shape, the fastest hipBLASLt / rocBLAS solution for the GEMMs that
    `run()` issues (the denoiser's projections and feed-forward), then keep those choices for later calls in this
    process. Opt-in and process-wide: it enables `torch.cuda.tunable`. `filename` keeps the results for a later
    process (`torch.cuda.tunable.read_file`). Call it before capturing a `PingpongGraph`, since capture does not
    tune."""
    tunable = torch.cuda.tunable
    tunable.enable(True)
    if filename is not None:
        tunable.set_filename(filename)
    tunable.tuning_enable(True)
    try:
        run()
        torch.cuda.synchronize()
    finally:
        tunable.tuning_enable(False)
