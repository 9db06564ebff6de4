"""Benchmark: milliseconds of DiT + SAME-L differential attention per 120 s clip on one MI355X.

One step is one clip's worth of the hot path with inputs resident in HBM:
  192 dense calls  (8 sampler steps x 24 DiT blocks), B=2 (CFG), L=2584 tokens, 24 heads x 64, bf16
  + 12 band calls (12 SAME-L decoder blocks), B=1, S=82688 frames, 8 heads x 64, half-width w=128, bf16
Each call is the full C-ABI operation (dense: prep + attention kernels; band: one kernel) on preallocated
buffers. Inputs follow the seeded recipe of `hummingbird_amd.workloads` (synthetic data, random gains).

The JSON line also carries, for the dominant kernel (dense attention), a roofline object computed from its
average launch duration measured here with HIP events on its own stream, and the same for the band kernel
(`roofline_band`); plus the CPU baseline: the NumPy restatement of the reference XLA chains (the oracle, fp32
accumulation) timed on this host on whole config-0, config-1 and config-2 calls, the clip composed from the
per-call times.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import dataclasses
import itertools
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E
# HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE passes over `bench.py --kernels-only`
# (written by hummingbird_amd.rocprof_summary); reported as roofline.traffic when present.
TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_120s_clip.json"
# Kernels that the two calls launch at these shapes (D = 64; window 128 takes the two-tile ring variant).
DENSE_KERNEL = "dense_attend_bf16<64,128,4>"
BAND_KERNEL = "band_ring_bf16<2>"


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--kernel-iters", type=int, default=50, help="launches per live kernel timing")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU-baseline sample time")
    ap.add_argument("--sweep", action="store_true",
                    help="instead of the clip benchmark: the mixed-shape sweep (DiT L in {216, 1292, 2584} x "
                         "D in {64, 128}, SAME-L S=16384 with w in {64, 128, 256}; bf16 and fp32), one JSON line "
                         "per shape with its timing, roofline fraction and parity against the torch XLA chain")
    ap.add_argument("--ceiling", action="store_true",
                    help="instead of the clip benchmark: the data dependence of the matrix cores -- torch bf16 "
                         "GEMMs (8192^3) and the dense call with N(0,1), all-zero and all-one inputs")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the per-call timings at the reference-true and 380 s shapes")
    ap.add_argument("--sampler-only", action="store_true",
                    help="instead of the clip benchmark: the whole 120 s render of the medium DiT (8 pingpong steps "
                         "x 24 blocks, eager and as one HIP graph), one JSON line; for profiling under rocprofv3")
    ap.add_argument("--decoder-only", action="store_true",
                    help="instead of the clip benchmark: the SAME-L decoder's 12 blocks for a 120 s clip at the "
                         "reference's decoder geometry, chained and block by block, one JSON line; for profiling")
    ap.add_argument("--no-tune", action="store_true",
                    help="skip the sampler timing with TunableOp-selected GEMMs (whose search launches thousands of "
                         "candidate kernels; for profiling the loop itself)")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the per-kernel timing loops plus one 256 MiB device copy (the traffic-counter "
                         "calibration kernel); for profiling under rocprofv3")
    return ap.parse_args()


def _median_time(fn, target_s: float, min_runs: int = 5, warm: bool = True) -> tuple[float, int]:
    """Median wall time (s) of runs of `fn` (after one untimed run when `warm`): at least `min_runs`, more until
    about `target_s` has passed."""
    if warm:
        fn()
    times = []
    t_end = time.perf_counter() + target_s
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def config0_inputs(seed: int = 0) -> dict:
    """The CPU configuration: x ~ N(0,1) (1, 216, 1536); W_qkv (7680, 1536) and W_o (1536, 1536) ~ N(0, 1/1536);
    RMSNorm gains ~ 1 + N(0, 0.02); RoPE base 10000 over the full head_dim (half 32); per-pair lambda ~ U(0.2, 0.8);
    value mask ones except the last 16 tokens; 24 heads of 64; seed 0."""
    rng = np.random.default_rng(seed)
    E, L, H, D = 1536, 216, 24, 64
    x = rng.standard_normal((1, L, E), dtype=np.float32)
    w_qkv = (rng.standard_normal((5 * E, E)) / np.sqrt(E)).astype(np.float32)
    w_o = (rng.standard_normal((E, E)) / np.sqrt(E)).astype(np.float32)
    qw = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    kw = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    lam = rng.uniform(0.2, 0.8, H).astype(np.float32)
    valid = np.ones((1, L), np.float32)
    valid[:, L - 16:] = 0.0
    from hummingbird_amd import workloads as wl
    return dict(x=x, w_qkv=w_qkv, w_o=w_o, q_weight=qw, k_weight=kw, lam=lam, valid=valid, inv_freq=wl.inv_freq(32),
                heads=H, head_dim=D)


def cpu_baseline(target_s: float) -> dict:
    """The oracle (NumPy restatement of the reference XLA chains, fp32 with fp32 accumulation, as XLA:CPU runs them)
    on this host, each workload whole: config 0 (to_qkv -> attention -> to_out at L=216; the median of at least 5
    warm runs), one config-1 dense call (B=2, L=2584, 24 heads) and one config-2 band call (S=82688, 8 heads,
    w=128), each the median of 3 runs (multi-second calls: no untimed warm-up run)."""
    from threadpoolctl import threadpool_info

    from hummingbird_amd import workloads as wl
    from oracle import band as oband
    from oracle import dense as odense

    rows = {}
    # config 0, whole
    c0 = config0_inputs()

    def config0():
        qkv = (c0["x"] @ c0["w_qkv"].T).astype(np.float32)
        out = odense.dense_xla(qkv, c0["q_weight"], c0["k_weight"], c0["inv_freq"], c0["valid"], c0["heads"],
                               c0["head_dim"], 1e-6, c0["lam"], "fp32", np.float32)
        return (out @ c0["w_o"].T).astype(np.float32)

    t0, n0 = _median_time(config0, target_s / 3)
    rows["config0"] = {"ms": round(1e3 * t0, 2), "runs": n0, "sampled": "no (whole call, L=216, to_qkv -> "
                       "attention -> to_out)"}
    # config 1: one whole dense call
    d, b = wl.DENSE_120S, wl.BAND_120S
    inp = wl.dense_inputs(d["batch"], d["length"], d["heads"], d["head_dim"], seed=0, dtype="fp32")
    args = (inp["qkv"], inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"], d["heads"], d["head_dim"],
            1e-6, inp["lam"], "fp32", np.float32)
    t1, n1 = _median_time(lambda: odense.dense_xla(*args), 0.0, min_runs=3, warm=False)  # seconds per run
    rows["config1_dense_call"] = {"ms": round(1e3 * t1, 1), "runs": n1,
                                  "sampled": f"no (whole call, B={d['batch']}, L={d['length']}, H={d['heads']})"}
    del inp, args
    # config 2: one whole band call
    binp = wl.band_inputs(b["batch"], b["length"], b["heads"], b["head_dim"], b["window"], seed=1, dtype="fp32")
    bargs = (binp["qkv"], binp["q_norm"], binp["k_norm"], binp["inv_freq"], b["heads"], b["head_dim"], b["window"],
             binp["lam"], "fp32", np.float32)
    t2, n2 = _median_time(lambda: oband.band_xla(*bargs), 0.0, min_runs=3, warm=False)
    rows["config2_band_call"] = {"ms": round(1e3 * t2, 1), "runs": n2,
                                 "sampled": f"no (whole call, S={b['length']}, H={b['heads']}, w={b['window']})"}
    del binp, bargs
    threads = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    ms_clip = (wl.DENSE_CALLS_PER_CLIP * rows["config1_dense_call"]["ms"]
               + wl.BAND_CALLS_PER_CLIP * rows["config2_band_call"]["ms"])
    return {"value": round(ms_clip, 1), "unit": "ms/120s-clip", "cores": int(threads), "kind": "port",
            "sample": (f"oracle (NumPy fp32 XLA-chain restatement, not XLA: jax is absent), whole calls, medians of "
                       f"3 runs (config 0: >= 5 warm runs); clip = {wl.DENSE_CALLS_PER_CLIP} config-1 dense calls + "
                       f"{wl.BAND_CALLS_PER_CLIP} config-2 band calls at the measured per-call times; "
                       f"host cpus={len(os.sched_getaffinity(0))}"),
            "rows": rows}


def call_percentiles(fn, n: int, stream) -> dict:
    """Per-call duration percentiles (us) from HIP events around each of `n` warm calls on `stream`."""
    import torch

    fn()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    ev[0].record(stream)
    for i in range(n):
        fn()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    us = np.array([ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(n)])
    return {"p10": round(float(np.percentile(us, 10)), 2), "p50": round(float(np.median(us)), 2),
            "p90": round(float(np.percentile(us, 90)), 2)}


# Extra shapes, timed per call (not part of the clip value):
#   reference-true 120 s geometry: DiT B=1, L=1422, 24 heads, rotary half 16; SAME-L S=23086, 24 heads, w=17
#   380 s clip: DiT B=2, L=8180; SAME-L S=261760, 8 heads, w=128
EXTRA_DENSE = {"ref_true_120s": (1, 1422, 24, 64, 16), "clip_380s": (2, 8180, 24, 64, 32)}
EXTRA_BAND = {"ref_true_120s": (1, 23086, 24, 64, 17, 16), "clip_380s": (1, 261760, 8, 64, 128, 32)}


def extra_shapes(lib, sp, stream, dev) -> dict:
    """Per-call p10/p50/p90 and roofline fractions of the dense and band calls at the extra shapes, of the DiT
    cross-attention and of a SAME-L decoder block at the 120 s clip (synthetic N(0,1) inputs drawn on the device,
    unit gains, lam = 1)."""
    import torch

    from hummingbird_amd import _lib
    from hummingbird_amd import band_attention as ba
    from hummingbird_amd import dense_attention as da
    from hummingbird_amd import workloads as wl

    gen = torch.Generator(device=dev).manual_seed(7)
    res = {}
    for name, (B, L, H, D, half) in EXTRA_DENSE.items():
        qkv = torch.randn((B, L, 5 * H * D), device=dev, generator=gen).to(torch.bfloat16)
        ones = torch.ones(D, device=dev)
        cos, sin, mask = da.tables(L, torch.from_numpy(wl.inv_freq(half)).to(dev), torch.ones((B, L), device=dev),
                                   D, torch.bfloat16)
        wsb = int(lib.hb_dense_workspace_size(_lib.HB_BF16, B, L, H, D))
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        out = torch.empty((B, L, H * D), dtype=torch.bfloat16, device=dev)

        def call():
            _lib.check(lib.hb_dense_diffattn(sp, qkv.data_ptr(), _lib.HB_BF16, 5 * H * D, ones.data_ptr(),
                                             ones.data_ptr(), cos.data_ptr(), sin.data_ptr(), half, mask.data_ptr(),
                                             0, out.data_ptr(), B, L, H, D, 1e-6, ws.data_ptr(), wsb), "dense")
        pc = call_percentiles(call, 20, stream)
        tf = wl.dense_flops(B, L, H, D) / (pc["p50"] * 1e-6) / 1e12
        res[f"dense_{name}"] = {"shape": {"B": B, "L": L, "H": H, "D": D, "half": half}, "us_per_call": pc,
                                "tflops_p50": round(tf, 1), "mfma_frac_p50": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}
        del qkv, ws, out
    for name, (B, S, H, D, W, half) in EXTRA_BAND.items():
        qkv = torch.randn((B, S, 5 * H * D), device=dev, generator=gen).to(torch.bfloat16)
        dyt = {"alpha": torch.tensor(0.5), "gamma": torch.ones(D), "beta": torch.zeros(D)}
        qd, kd = ba.pack_dyt(dyt, D, dev), ba.pack_dyt(dyt, D, dev)
        cos, sin = ba.rope_tables(S, torch.from_numpy(wl.inv_freq(half)).to(dev))
        out = torch.empty((B, S, H * D), dtype=torch.bfloat16, device=dev)

        def bcall():
            _lib.check(lib.hb_band_diffattn(sp, qkv.data_ptr(), _lib.HB_BF16, 5 * H * D, qd.data_ptr(), kd.data_ptr(),
                                            cos.data_ptr(), sin.data_ptr(), half, W, 0, out.data_ptr(), B, S, H, D,
                                            0, 0), "band")
        pc = call_percentiles(bcall, 10, stream)
        gbs = wl.band_bytes(B, S, H, D) / (pc["p50"] * 1e-6) / 1e9
        res[f"band_{name}"] = {"shape": {"B": B, "S": S, "H": H, "D": D, "w": W, "half": half}, "us_per_call": pc,
                               "gbs_p50": round(gbs, 1), "hbm_frac_p50": round(gbs / HBM_PEAK_GBS, 4),
                               "tflops_p50": round(wl.band_flops(B, S, H, D, W) / (pc["p50"] * 1e-6) / 1e12, 1)}
        del qkv, out
    # DiT cross-attention of the same clip (as many calls as the self-attention): the context's K/V prepared
    # once, then the attention per call against it.
    c = wl.CROSS_120S
    B, L, Nk, H, D = c["batch"], c["length"], c["context"], c["heads"], c["head_dim"]
    q = torch.randn((B, L, 2 * H * D), device=dev, generator=gen).to(torch.bfloat16)
    kv = torch.randn((B, Nk, 3 * H * D), device=dev, generator=gen).to(torch.bfloat16)
    ones = torch.ones(D, device=dev)
    wsb = int(lib.hb_cross_workspace_size(_lib.HB_BF16, B, Nk, H, D))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    out = torch.empty((B, L, H * D), dtype=torch.bfloat16, device=dev)

    def prep():
        _lib.check(lib.hb_cross_prep(sp, kv.data_ptr(), _lib.HB_BF16, 3 * H * D, ones.data_ptr(), B, Nk, H, D, 1e-6,
                                     ws.data_ptr(), wsb), "cross_prep")

    def attend():
        _lib.check(lib.hb_cross_attend(sp, q.data_ptr(), _lib.HB_BF16, 2 * H * D, ones.data_ptr(), ones.data_ptr(),
                                       0, out.data_ptr(), B, L, Nk, H, D, 1e-6, ws.data_ptr(), wsb), "cross_attend")
    pp = call_percentiles(prep, 20, stream)
    pc = call_percentiles(attend, 20, stream)
    tf = wl.cross_flops(B, L, Nk, H, D) / (pc["p50"] * 1e-6) / 1e12
    res["cross_120s"] = {"shape": {"B": B, "L": L, "Nk": Nk, "H": H, "D": D}, "prep_us_per_context": pp,
                         "us_per_call": pc, "tflops_p50": round(tf, 1),
                         "mfma_frac_p50": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                         "ms_per_clip": round(wl.DENSE_CALLS_PER_CLIP * pc["p50"] / 1e3, 3)}
    del q, kv, ws, out
    res["same_l_block_120s"] = block_shape(lib, sp, stream, dev, gen)
    res["same_l_decoder_120s"] = decoder_shape(dev, gen)
    res["dit_self_attention_120s"] = dit_self_attention_shape(stream, dev, gen)
    res["sampler_120s"] = sampler_shape(dev)
    # the matrix cores' data dependence: what the dense kernel's roofline fraction is measured against in practice
    res["mfma_ceiling"] = ceiling_summary(lib, sp, stream, dev)
    return res


def sampler_shape(dev, tune: bool = True) -> dict:
    """The whole denoising of one 120 s clip as the reference renders it: the `medium` DiT (24 blocks, width 1536,
    24 heads; random weights), batch 1, 1358 latents + 64 memory tokens (L = 1422), a 257-token context, 8 pingpong
    steps, bf16, attention="hip" (192 dense self-attention and 192 cross-attention calls). Per-clip state from
    `dit.prepare_static` (not timed); then ms per clip for the eager loop and for the loop captured as one HIP
    graph (median of 3 each), and for the graph again after `sampling.tune_gemms` has let PyTorch's TunableOp pick
    each GEMM's solution (the tuning itself is not timed; TunableOp is switched off again afterwards)."""
    import torch

    from hummingbird_amd import dit, sampling
    from hummingbird_amd.config import MEDIUM_DIT, SAMPLER_STEPS
    from hummingbird_amd.dtypes import BF16

    cfg, T, steps = MEDIUM_DIT, 1358, SAMPLER_STEPS
    gen = torch.Generator(device=dev).manual_seed(11)
    params = dit.init_params(cfg, BF16, device=dev, seed=11)
    cond = {"cross_attn_cond": torch.randn((1, 257, cfg.cond_token_dim), device=dev, generator=gen),
            "global_cond": torch.randn((1, cfg.global_cond_dim), device=dev, generator=gen)}
    mask = torch.ones((1, T), dtype=torch.bool, device=dev)
    x0 = torch.randn((1, cfg.io_channels, T), device=dev, generator=gen)
    noise = torch.zeros((steps, 1, cfg.io_channels, T), device=dev)  # the "zeros" renoise the ports ship
    static = dit.prepare_static(params, cond, mask, cfg, BF16)
    schedule = sampling.build_schedule(steps, device=dev)

    def clip_ms(fn, n=3) -> float:
        fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(n):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b))
        return round(float(np.median(times)), 2)
    def eager_clip():
        return sampling.pingpong(params, x0, schedule, noise, static, cfg, BF16, trajectory=False)
    eager = clip_ms(eager_clip)
    graph = sampling.PingpongGraph(params, static, cfg, BF16, x0, noise)
    replay = clip_ms(lambda: graph(x0, noise))
    del graph
    shape = {"B": 1, "latents": T, "L": T + cfg.num_memory_tokens, "context": 257, "depth": cfg.depth,
             "E": cfg.embed_dim, "H": cfg.num_heads, "steps": steps}
    calls = {"dense": steps * cfg.depth, "cross": steps * cfg.depth}
    if not tune:
        return {"shape": shape, "eager_ms_per_clip": eager, "graph_ms_per_clip": replay,
                "attention_calls_per_clip": calls}
    # GEMM solutions chosen per shape by PyTorch's TunableOp (tuning untimed), then the graph captured again
    import tempfile
    import time
    with tempfile.TemporaryDirectory() as tmp:
        t0 = time.perf_counter()
        sampling.tune_gemms(eager_clip, filename=f"{tmp}/tunableop_results.csv")
        tune_s = time.perf_counter() - t0
        graph = sampling.PingpongGraph(params, static, cfg, BF16, x0, noise)
        tuned = clip_ms(lambda: graph(x0, noise))
        del graph
        torch.cuda.tunable.enable(False)
    return {"shape": shape, "eager_ms_per_clip": eager, "graph_ms_per_clip": replay,
            "graph_ms_per_clip_tuned_gemms": tuned, "gemm_tuning_s": round(tune_s, 1),
            "attention_calls_per_clip": calls}


def dit_self_attention_shape(stream, dev, gen) -> dict:
    """One DiT self-attention (to_qkv -> differential attention -> to_out) at the 120 s clip (B=2, L=2584, width 1536
    = 24 heads of 64, rotary half 16, bf16), with the projections on hipBLASLt ("torch": GEMM, then the kernel's own
    key preparation) and on this package's GEMMs ("hip": key preparation in the to_qkv epilogue), per call."""
    import dataclasses

    import torch

    from hummingbird_amd import dit
    from hummingbird_amd import workloads as wl
    from hummingbird_amd.config import MEDIUM_DIT

    d = wl.DENSE_120S
    cfg = dataclasses.replace(MEDIUM_DIT, num_memory_tokens=0)
    B, L, E, H = d["batch"], d["length"], cfg.embed_dim, cfg.num_heads
    h = torch.randn((B, L, E), device=dev, generator=gen).to(torch.bfloat16)

    def w(o, i):
        return (torch.randn((o, i), device=dev, generator=gen) / i ** 0.5).to(torch.bfloat16)
    block = {"self_attn": {"to_qkv": {"weight": w(5 * E, E)}, "to_out": {"weight": w(E, E)},
                           "q_norm": {"weight": torch.ones(64, device=dev)},
                           "k_norm": {"weight": torch.ones(64, device=dev)}}}
    static = dit.static_tables(torch.from_numpy(wl.inv_freq(cfg.rope_dim // 2)).to(dev),
                               torch.ones((B, L), dtype=torch.bool, device=dev), cfg, torch.bfloat16)
    res = {"shape": {"B": B, "L": L, "E": E, "H": H, "D": 64, "half": cfg.rope_dim // 2}}
    for proj in ("torch", "hip"):
        res[f"{proj}_us_per_call"] = call_percentiles(
            lambda: dit.self_attention(h, block, static, cfg, projections=proj), 10, stream)
    return res


def block_shape(lib, sp, stream, dev, gen) -> dict:
    """One SAME-L decoder block at the 120 s clip (S=82688 frames, dim 512 = 8 heads of 64, ff 1536, w=128):
    hb_dyt and hb_glu per call with their HBM fractions, and the whole block (DyT -> to_qkv -> band attention ->
    to_out -> residual -> DyT -> glu_proj -> GLU -> proj_out -> residual; GEMMs on torch/hipBLASLt)."""
    import torch

    from hummingbird_amd import _lib, same_l
    from hummingbird_amd import workloads as wl
    from hummingbird_amd.config import SameConfig

    S, dim, ff = wl.BAND_120S["length"], 8 * 64, 8 * 64 * 3
    x = torch.randn((1, S, dim), device=dev, generator=gen).to(torch.bfloat16)
    dyt = torch.cat([torch.tensor([0.5], device=dev), torch.ones(dim, device=dev), torch.zeros(dim, device=dev)])
    y = torch.empty_like(x)
    proj = torch.randn((1, S, 2 * ff), device=dev, generator=gen).to(torch.bfloat16)
    g = torch.empty((1, S, ff), dtype=torch.bfloat16, device=dev)
    bias = torch.zeros(2 * ff, device=dev)

    def dyt_call():
        _lib.check(lib.hb_dyt(sp, x.data_ptr(), _lib.HB_BF16, dim, dyt.data_ptr(), y.data_ptr(), dim, S, dim), "dyt")

    def glu_call():
        _lib.check(lib.hb_glu(sp, proj.data_ptr(), _lib.HB_BF16, 2 * ff, bias.data_ptr(), 1, g.data_ptr(), ff, S, ff),
                   "glu")
    pd, pg = call_percentiles(dyt_call, 20, stream), call_percentiles(glu_call, 20, stream)
    dyt_bytes, glu_bytes = 2.0 * S * dim * 2, float(S) * 3 * ff * 2

    def w(o, i):
        return (torch.randn((o, i), device=dev, generator=gen) / i ** 0.5).to(torch.bfloat16)

    def norm(c):
        return {"alpha": torch.tensor(0.5, device=dev), "gamma": torch.ones(c, device=dev),
                "beta": torch.zeros(c, device=dev)}
    params = {"pre_norm": norm(dim), "ff_norm": norm(dim),
              "rope_inv_freq": torch.from_numpy(wl.inv_freq(32)).to(dev),
              "self_attn": {"to_qkv": {"weight": w(5 * dim, dim)}, "to_out": {"weight": w(dim, dim)},
                            "q_norm": norm(64), "k_norm": norm(64)},
              "ff": {"glu_proj": {"weight": w(2 * ff, dim), "bias": torch.zeros(2 * ff, device=dev, dtype=torch.bfloat16)},
                     "proj_out": {"weight": w(dim, ff), "bias": torch.zeros(dim, device=dev, dtype=torch.bfloat16)}}}
    cfg = SameConfig(channels=128, c_mults=(4,), stride=127, transformer_depth=12, sinusoidal_blocks=8,
                     attention="hip")  # dim 512, half-width 128
    pb = call_percentiles(lambda: same_l.block(x, params, 11, cfg), 10, stream)
    return {"shape": {"S": S, "dim": dim, "ff": ff, "w": cfg.sub_chunk_size},
            "dyt_us_per_call": pd, "dyt_hbm_frac_p50": round(dyt_bytes / (pd["p50"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "glu_us_per_call": pg, "glu_hbm_frac_p50": round(glu_bytes / (pg["p50"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "block_us_per_call": pb}


def stream_of(dev):
    import torch
    return torch.cuda.current_stream(dev)


def decoder_gemms(x, p, cfg, stream) -> dict:
    """One decoder block's glu_proj and proj_out at the clip's shape (p50 of interleaved calls, µs): hipBLASLt
    followed by this package's GLU / residual kernels against the fused GEMMs that do the same work in their
    epilogues."""
    from hummingbird_amd import elementwise, projection
    ff, dim = p["ff"], x.shape[-1]
    y = x[0]
    g = projection.glu_linear(y, ff["glu_proj"]["weight"], ff["glu_proj"]["bias"], True)
    cases = {
        "glu_proj_torch_then_glu": lambda: elementwise.glu(y @ ff["glu_proj"]["weight"].t(), True,
                                                           bias=ff["glu_proj"]["bias"]),
        "glu_proj_fused": lambda: projection.glu_linear(y, ff["glu_proj"]["weight"], ff["glu_proj"]["bias"], True),
        "proj_out_torch_then_residual_dyt": lambda: elementwise.residual_dyt(
            y, g @ ff["proj_out"]["weight"].t(), bias=ff["proj_out"]["bias"], norm=p["pre_norm"]),
        "proj_out_fused": lambda: projection.residual_linear(g, ff["proj_out"]["weight"], ff["proj_out"]["bias"], y,
                                                             p["pre_norm"]),
        "to_out_torch_then_residual_dyt": lambda: elementwise.residual_dyt(
            y, y @ p["self_attn"]["to_out"]["weight"].t(), norm=p["ff_norm"]),
        "to_out_fused": lambda: projection.residual_linear(y, p["self_attn"]["to_out"]["weight"], None, y,
                                                           p["ff_norm"]),
    }
    rows = {k: [] for k in cases}
    for _ in range(3):
        for k, fn in cases.items():
            rows[k].append(call_percentiles(fn, 10, stream)["p50"])
    del g
    return {k: round(float(np.median(v)), 2) for k, v in rows.items()}


def decoder_shape(dev, gen) -> dict:
    """The SAME-L decoder's 12 blocks for a 120 s clip at the reference's medium geometry (1358 latents x 17 = 23086
    frames, dim 1536 = 24 heads of 64, ff 4608, half-width 17, the last 8 blocks with the sine gate; random weights,
    bf16): ms per clip for the chained loop (`same_l.blocks`, each block handing the next its pre_norm DyT), for the
    block-by-block loop and for the chained loop on this package's projection GEMMs with fused epilogues
    (projections="hip"), medians of 7 interleaved runs after one warm-up each; then each projection of one block
    timed alone, fused against hipBLASLt plus the elementwise kernel (`decoder_gemms`). The reference's published
    figure for its whole decode (these blocks plus the bottleneck, token interleave and output mapping) is 61 ms on
    a TPU v6e-1."""
    import torch

    from hummingbird_amd import same_l
    from hummingbird_amd import workloads as wl
    from hummingbird_amd.config import MEDIUM_SAME_L

    cfg = dataclasses.replace(MEDIUM_SAME_L, attention="hip")
    latents = 1358
    S, dim, ff = latents * cfg.sub_chunk_size, cfg.dim, cfg.ff_inner

    def w(o, i):
        return (torch.randn((o, i), device=dev, generator=gen) / i ** 0.5).to(torch.bfloat16)

    def norm(c):
        return {"alpha": torch.tensor(0.5, device=dev), "gamma": torch.ones(c, device=dev),
                "beta": torch.zeros(c, device=dev)}

    def zeros(n):
        return torch.zeros(n, device=dev, dtype=torch.bfloat16)
    inv_freq = torch.from_numpy(wl.inv_freq(16)).to(dev)
    params = [{"pre_norm": norm(dim), "ff_norm": norm(dim), "rope_inv_freq": inv_freq,
               "self_attn": {"to_qkv": {"weight": w(5 * dim, dim)}, "to_out": {"weight": w(dim, dim)},
                             "q_norm": norm(64), "k_norm": norm(64)},
               "ff": {"glu_proj": {"weight": w(2 * ff, dim), "bias": zeros(2 * ff)},
                      "proj_out": {"weight": w(dim, ff), "bias": zeros(dim)}}}
              for _ in range(cfg.transformer_depth)]
    x = torch.randn((1, S, dim), device=dev, generator=gen).to(torch.bfloat16)

    def chained():
        return same_l.blocks(x, params, cfg)

    def one_by_one():
        h = x
        for i, p in enumerate(params):
            h = same_l.block(h, p, i, cfg)
        return h

    def fused_projections():
        return same_l.blocks(x, params, cfg, projections="hip")

    def once(fn) -> float:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b)
    chained(), one_by_one(), fused_projections()
    torch.cuda.synchronize()
    times = {"chained": [], "one_by_one": [], "fused": []}
    for _ in range(7):  # the loops interleaved, so that a drift of the clock touches them alike
        times["chained"].append(once(chained))
        times["one_by_one"].append(once(one_by_one))
        times["fused"].append(once(fused_projections))
    res = {"shape": {"S": S, "dim": dim, "heads": cfg.num_heads, "ff": ff, "w": cfg.sub_chunk_size,
                     "blocks": cfg.transformer_depth, "sine_blocks": cfg.sinusoidal_blocks},
           "chained_ms_per_clip": round(float(np.median(times["chained"])), 3),
           "block_by_block_ms_per_clip": round(float(np.median(times["one_by_one"])), 3),
           "hip_projections_ms_per_clip": round(float(np.median(times["fused"])), 3),
           "projection_gemms_us": decoder_gemms(x, params[0], cfg, stream_of(dev)),
           "reference_whole_decode_ms_tpu_v6e": 61.0}
    del params
    return res


FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA


def parity(got, ref, dtype: str) -> dict:
    """max-abs, cosine and relative error against the torch restatement of the XLA chain, and whether they are
    within the contract (bf16: max-abs <= 2e-2 and cosine >= 0.9999; fp32: <= 1e-5 relative)."""
    g, r = got.double().flatten(), ref.double().flatten()
    err = (g - r).abs().max().item()
    cos = (g @ r / (g.norm() * r.norm())).item()
    rel = err / max(r.abs().max().item(), 1e-30)
    ok = (err <= 2e-2 and cos >= 0.9999) if dtype == "bf16" else rel <= 1e-5
    return {"max_abs": float(f"{err:.3g}"), "cosine": round(cos, 7), "rel": float(f"{rel:.3g}"), "within_tolerance": ok}


def sweep(lib, sp, stream, dev) -> None:
    """Mixed-shape sweep: per shape, p50 per-call time, roofline fraction and parity (one JSON line each).
    Dense: B=2, H = 1536 / D, ragged value mask (0-25 % tail per row). Band: B=1, S=16384, 8 heads of 64 or 4
    of 128, half-widths 64-512."""
    import torch

    from hummingbird_amd import _lib
    from hummingbird_amd import band_attention as ba
    from hummingbird_amd import dense_attention as da
    from hummingbird_amd import workloads as wl
    from hummingbird_amd import xla_chain

    tdt = {"bf16": torch.bfloat16, "fp32": torch.float32}
    for length in (216, 1292, 2584):
        for D in (64, 128):
            for dt in ("bf16", "fp32"):
                B, H = 2, 1536 // D
                inp = wl.dense_inputs(B, length, H, D, seed=length + D, dtype=dt, ragged=True)
                qkv = torch.from_numpy(inp["qkv"]).to(dev, tdt[dt])
                qw, kw = torch.from_numpy(inp["q_weight"]).to(dev), torch.from_numpy(inp["k_weight"]).to(dev)
                lam, freq = torch.from_numpy(inp["lam"]).to(dev), torch.from_numpy(inp["inv_freq"]).to(dev)
                valid = torch.from_numpy(inp["valid"]).to(dev)
                cos, sin, mask = da.tables(length, freq, valid, D, tdt[dt])
                code = _lib.HB_BF16 if dt == "bf16" else _lib.HB_F32
                wsb = int(lib.hb_dense_workspace_size(code, B, length, H, D))
                ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
                out = torch.empty((B, length, H * D), dtype=tdt[dt], device=dev)

                def call():  # the C ABI directly, so host-side checks do not show up as GPU idle time
                    _lib.check(lib.hb_dense_diffattn(sp, qkv.data_ptr(), code, 5 * H * D, qw.data_ptr(), kw.data_ptr(),
                                                     cos.data_ptr(), sin.data_ptr(), inp["half"], mask.data_ptr(),
                                                     lam.data_ptr(), out.data_ptr(), B, length, H, D, inp["eps"],
                                                     ws.data_ptr(), wsb), "dense")
                pc = call_percentiles(call, 20, stream)
                ref = xla_chain.dense_chain(qkv, qw, kw, freq, valid, H, D, inp["eps"], lam=lam)
                tf = wl.dense_flops(B, length, H, D) / (pc["p50"] * 1e-6) / 1e12
                peak = MFMA_BF16_PEAK_TFLOPS if dt == "bf16" else FP32_MFMA_PEAK_TFLOPS
                print(json.dumps({"sweep": "dense", "B": B, "L": length, "H": H, "D": D, "dtype": dt,
                                  "us_per_call": pc, "tflops_p50": round(tf, 1), "peak_tflops": peak,
                                  "peak_frac_p50": round(tf / peak, 4), **parity(out.float(), ref.float(), dt)}),
                      flush=True)
                del qkv, ws, out, ref
    for (H, D), w in itertools.product(((8, 64), (4, 128)), (64, 128, 256, 512)):
        for dt in ("bf16", "fp32"):
            S = 16384
            inp = wl.band_inputs(1, S, H, D, w, seed=w, dtype=dt)
            qkv = torch.from_numpy(inp["qkv"]).to(dev, tdt[dt])
            qn = {k: torch.as_tensor(np.asarray(v)).to(dev) for k, v in inp["q_norm"].items()}
            kn = {k: torch.as_tensor(np.asarray(v)).to(dev) for k, v in inp["k_norm"].items()}
            lam, freq = torch.from_numpy(inp["lam"]).to(dev), torch.from_numpy(inp["inv_freq"]).to(dev)
            cos, sin = ba.rope_tables(S, freq)
            qd, kd = ba.pack_dyt(qn, D, dev), ba.pack_dyt(kn, D, dev)
            code = _lib.HB_BF16 if dt == "bf16" else _lib.HB_F32
            out = torch.empty((1, S, H * D), dtype=tdt[dt], device=dev)
            wsb = int(lib.hb_band_workspace_size(code, 1, S, H, D, inp["half"], w))
            ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev)

            def call():
                _lib.check(lib.hb_band_diffattn(sp, qkv.data_ptr(), code, 5 * H * D, qd.data_ptr(), kd.data_ptr(),
                                                cos.data_ptr(), sin.data_ptr(), inp["half"], w, lam.data_ptr(),
                                                out.data_ptr(), 1, S, H, D, ws.data_ptr(), wsb), "band")
            pc = call_percentiles(call, 10, stream)
            ref = xla_chain.band_chain(qkv, qn, kn, freq, H, D, w, lam=lam)
            elem = 2 if dt == "bf16" else 4
            gbs = wl.band_bytes(1, S, H, D, elem) / (pc["p50"] * 1e-6) / 1e9
            print(json.dumps({"sweep": "band", "B": 1, "S": S, "H": H, "D": D, "w": w, "window": 2 * w,
                              "dtype": dt, "us_per_call": pc, "gbs_p50": round(gbs, 1),
                              "hbm_frac_p50": round(gbs / HBM_PEAK_GBS, 4),
                              "tflops_p50": round(wl.band_flops(1, S, H, D, w) / (pc["p50"] * 1e-6) / 1e12, 1),
                              **parity(out.float(), ref.float(), dt)}), flush=True)
            del qkv, out, ref


def ceiling(lib, sp, stream, dev) -> None:
    """Throughput of the matrix cores as a function of the operand data (`ceiling_rows`), one JSON line per case."""
    for row in ceiling_rows(lib, sp, stream, dev):
        print(json.dumps(row), flush=True)


def ceiling_summary(lib, sp, stream, dev) -> dict:
    """`ceiling_rows` in short, for the default bench line: TFLOP/s at p50 per (kernel, data) and the dense kernel's
    N(0,1) rate as a fraction of the vendor GEMM's N(0,1) rate, the practical ceiling on random operands."""
    rows = ceiling_rows(lib, sp, stream, dev)
    out = {f"{'gemm' if r['ceiling'].startswith('torch') else 'dense_attend'}_{r['data']}_tflops": r["tflops_p50"]
           for r in rows}
    out["gemm_shape"] = [8192, 8192, 8192]
    out["dense_vs_gemm_randn"] = round(out["dense_attend_randn_tflops"] / out["gemm_randn_tflops"], 3)
    return out


def ceiling_rows(lib, sp, stream, dev, rounds: int = 3) -> list[dict]:
    """The vendor GEMM (torch -> hipBLASLt, bf16 8192^3) and the dense call at B=2, L=2584, H=24, D=64, each with
    N(0,1), all-zero and all-one inputs: per-call percentiles and TFLOP/s at p50. The six cases are interleaved
    over `rounds` rounds and each reports the round with the median p50: the matrix cores slow down as the chip
    heats, so cases timed one after the other would compare different power states."""
    import torch

    from hummingbird_amd import _lib
    from hummingbird_amd import dense_attention as da
    from hummingbird_amd import workloads as wl

    n = 8192
    d = wl.DENSE_120S
    B, L, H, D = d["batch"], d["length"], d["heads"], d["head_dim"]
    inp = wl.dense_inputs(B, L, H, D, seed=0)
    qw, kw = torch.from_numpy(inp["q_weight"]).to(dev), torch.from_numpy(inp["k_weight"]).to(dev)
    cos, sin, mask = da.tables(L, torch.from_numpy(inp["inv_freq"]).to(dev), torch.from_numpy(inp["valid"]).to(dev),
                               D, torch.bfloat16)
    wsb = int(lib.hb_dense_workspace_size(_lib.HB_BF16, B, L, H, D))
    out = torch.empty((B, L, H * D), dtype=torch.bfloat16, device=dev)
    cases = []
    for kind in ("randn", "zeros", "ones"):
        a = getattr(torch, kind)((n, n), device=dev, dtype=torch.bfloat16)
        b = getattr(torch, kind)((n, n), device=dev, dtype=torch.bfloat16)
        cases.append(({"ceiling": "torch.mm bf16", "shape": [n, n, n], "data": kind}, 2 * n ** 3, 20,
                      lambda a=a, b=b: torch.mm(a, b)))
    for kind in ("randn", "zeros", "ones"):
        qkv = getattr(torch, kind)((B, L, 5 * H * D), device=dev, dtype=torch.bfloat16)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        _lib.check(lib.hb_dense_prep(sp, qkv.data_ptr(), _lib.HB_BF16, 5 * H * D, qw.data_ptr(), kw.data_ptr(),
                                     cos.data_ptr(), sin.data_ptr(), inp["half"], mask.data_ptr(), B, L, H, D, 1e-6,
                                     ws.data_ptr(), wsb), "prep")

        def attend(qkv=qkv, ws=ws):
            _lib.check(lib.hb_dense_attend(sp, qkv.data_ptr(), _lib.HB_BF16, 5 * H * D, qw.data_ptr(), kw.data_ptr(),
                                           cos.data_ptr(), sin.data_ptr(), inp["half"], 0, out.data_ptr(), B, L, H,
                                           D, 1e-6, ws.data_ptr(), wsb), "attend")
        cases.append(({"ceiling": DENSE_KERNEL, "shape": [B, L, H, D], "data": kind}, wl.dense_flops(B, L, H, D), 50,
                      attend))
    runs: list[list[dict]] = [[] for _ in cases]
    for _ in range(rounds):
        for i, (_, _, iters, fn) in enumerate(cases):
            runs[i].append(call_percentiles(fn, iters, stream))
    rows = []
    for (head, flops, _, _), pcs in zip(cases, runs):
        pc = sorted(pcs, key=lambda p: p["p50"])[len(pcs) // 2]
        rows.append({**head, "us_per_call": pc, "tflops_p50": round(flops / (pc["p50"] * 1e-6) / 1e12, 1),
                     "rounds": rounds})
    return rows


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU only; run with --gpus 1 (the kernels shard by "
                                   "(batch, head) and by sequence with a halo, which is described but not built)"}))
        return 2

    import torch

    from hummingbird_amd import _lib
    from hummingbird_amd import band_attention as ba
    from hummingbird_amd import dense_attention as da
    from hummingbird_amd import workloads as wl

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    if args.sweep:
        sweep(lib, sp, stream, dev)
        return 0
    if args.ceiling:
        ceiling(lib, sp, stream, dev)
        return 0
    if args.sampler_only:
        print(json.dumps({"sampler_120s": sampler_shape(dev, tune=not args.no_tune)}), flush=True)
        return 0
    if args.decoder_only:
        gen = torch.Generator(device=dev).manual_seed(0)
        print(json.dumps({"same_l_decoder_120s": decoder_shape(dev, gen)}), flush=True)
        return 0

    # ---- dense inputs (two qkv buffers alternate, as consecutive blocks would) ----
    d = wl.DENSE_120S
    B, L, H, D = d["batch"], d["length"], d["heads"], d["head_dim"]
    dinp = wl.dense_inputs(B, L, H, D, seed=0)
    gen = torch.Generator(device=dev).manual_seed(0)
    qkv_d = [torch.from_numpy(dinp["qkv"]).to(dev, torch.bfloat16),
             torch.randn((B, L, 5 * H * D), device=dev, generator=gen).to(torch.bfloat16)]
    qw = torch.from_numpy(dinp["q_weight"]).to(dev)
    kw = torch.from_numpy(dinp["k_weight"]).to(dev)
    lam_d = torch.from_numpy(dinp["lam"]).to(dev)
    cos_d, sin_d, mask_d = da.tables(L, torch.from_numpy(dinp["inv_freq"]).to(dev),
                                     torch.from_numpy(dinp["valid"]).to(dev), D, torch.bfloat16)
    half_d = dinp["half"]
    ws_bytes = int(lib.hb_dense_workspace_size(_lib.HB_BF16, B, L, H, D))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    out_d = torch.empty((B, L, H * D), dtype=torch.bfloat16, device=dev)

    # ---- band inputs ----
    bcfg = wl.BAND_120S
    S, HB, DB, W = bcfg["length"], bcfg["heads"], bcfg["head_dim"], bcfg["window"]
    binp = wl.band_inputs(1, S, HB, DB, W, seed=1)
    qkv_b = torch.from_numpy(binp["qkv"]).to(dev, torch.bfloat16)
    qdyt = ba.pack_dyt({k: torch.as_tensor(np.asarray(v)) for k, v in binp["q_norm"].items()}, DB, dev)
    kdyt = ba.pack_dyt({k: torch.as_tensor(np.asarray(v)) for k, v in binp["k_norm"].items()}, DB, dev)
    cos_b, sin_b = ba.rope_tables(S, torch.from_numpy(binp["inv_freq"]).to(dev))
    lam_b = torch.from_numpy(binp["lam"]).to(dev)
    out_b = torch.empty((1, S, HB * DB), dtype=torch.bfloat16, device=dev)
    half_b = binp["half"]
    del dinp, binp

    def dense_call(i: int) -> None:
        q = qkv_d[i & 1]
        _lib.check(lib.hb_dense_diffattn(sp, q.data_ptr(), _lib.HB_BF16, 5 * H * D, qw.data_ptr(), kw.data_ptr(),
                                         cos_d.data_ptr(), sin_d.data_ptr(), half_d, mask_d.data_ptr(),
                                         lam_d.data_ptr(), out_d.data_ptr(), B, L, H, D, 1e-6, ws.data_ptr(),
                                         ws_bytes), "dense")

    def band_call() -> None:
        _lib.check(lib.hb_band_diffattn(sp, qkv_b.data_ptr(), _lib.HB_BF16, 5 * HB * DB, qdyt.data_ptr(),
                                        kdyt.data_ptr(), cos_b.data_ptr(), sin_b.data_ptr(), half_b, W,
                                        lam_b.data_ptr(), out_b.data_ptr(), 1, S, HB, DB, 0, 0), "band")

    def step() -> None:
        for i in range(wl.DENSE_CALLS_PER_CLIP):
            dense_call(i)
        for _ in range(wl.BAND_CALLS_PER_CLIP):
            band_call()

    if args.kernels_only:
        for _ in range(args.warmup):  # clocks settle as in the timed run
            step()
        src = torch.empty(1 << 28, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)  # 256 MiB read + 256 MiB written: calibrates FETCH_SIZE / WRITE_SIZE
        torch.cuda.synchronize()
        del src, dst
        ms_clip, host_s = float("nan"), 0.0
    else:
        print(f"[bench] warmup {args.warmup} clip(s)", file=sys.stderr, flush=True)
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        print(f"[bench] timing {args.steps} clip(s)", file=sys.stderr, flush=True)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t_host = time.perf_counter()
        start.record(stream)
        for _ in range(args.steps):
            step()
        stop.record(stream)
        torch.cuda.synchronize()
        host_s = time.perf_counter() - t_host
        ms_clip = start.elapsed_time(stop) / args.steps

    # ---- live per-kernel timing (HIP events on the launch stream) ----
    def timed(fn, n: int) -> float:
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(n):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n * 1e-3  # seconds per launch

    dense_call(0)  # workspace now holds the prepared k/v of qkv_d[0] for the attention-only timing
    attend_s = timed(lambda: _lib.check(lib.hb_dense_attend(sp, qkv_d[0].data_ptr(), _lib.HB_BF16, 5 * H * D,
                                                            qw.data_ptr(), kw.data_ptr(), cos_d.data_ptr(),
                                                            sin_d.data_ptr(), half_d, lam_d.data_ptr(),
                                                            out_d.data_ptr(), B, L, H, D, 1e-6, ws.data_ptr(),
                                                            ws_bytes), "attend"), args.kernel_iters)
    prep_s = timed(lambda: _lib.check(lib.hb_dense_prep(sp, qkv_d[0].data_ptr(), _lib.HB_BF16, 5 * H * D,
                                                        qw.data_ptr(), kw.data_ptr(), cos_d.data_ptr(),
                                                        sin_d.data_ptr(), half_d, mask_d.data_ptr(), B, L, H, D, 1e-6,
                                                        ws.data_ptr(), ws_bytes), "prep"), args.kernel_iters)
    band_s = timed(band_call, max(5, args.kernel_iters // 5))
    dense_pc = call_percentiles(lambda: dense_call(0), args.kernel_iters, stream)
    band_pc = call_percentiles(band_call, max(5, args.kernel_iters // 5), stream)
    dense_fl, dense_by = wl.dense_flops(B, L, H, D), wl.dense_bytes(B, L, H, D)
    band_fl, band_by = wl.band_flops(1, S, HB, DB, W), wl.band_bytes(1, S, HB, DB)
    attend_tf = dense_fl / attend_s / 1e12
    band_gbs = band_by / band_s / 1e9

    result = {
        "metric": "ms/120s-clip for DiT+SAME-L attention; % bf16 MFMA peak and % HBM GB/s",
        "value": round(ms_clip, 3),
        "unit": "ms/120s-clip",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_clip, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) qkv, random gains; hummingbird_amd.workloads)",
        "config": {"workload": "120 s clip: 192 x DiT dense diff-attn (B=2, L=2584, H=24, D=64) + 12 x SAME-L "
                               "band diff-attn (B=1, S=82688, H=8, D=64, w=128)",
                   "dense_ms_per_call": round((attend_s + prep_s) * 1e3, 4),
                   "band_ms_per_call": round(band_s * 1e3, 4),
                   "dense_call_us": dense_pc, "band_call_us": band_pc,
                   "host_wall_s": round(host_s, 3)},
        "roofline": {"bound": "mfma", "achieved": round(attend_tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(attend_tf / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": DENSE_KERNEL, "avg_us": round(attend_s * 1e6, 2),
                     "flops_per_launch": dense_fl},
        "roofline_band": {"bound": "hbm", "achieved": round(band_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(band_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                          "kernel": BAND_KERNEL, "avg_us": round(band_s * 1e6, 2),
                          "bytes_per_launch": band_by, "tflops": round(band_fl / band_s / 1e12, 1)},
        # prep reads the k, v and k_diff sections and writes them back prepared: 2 x 3 H D bf16 per token
        "dense_prep": {"avg_us": round(prep_s * 1e6, 2), "gbs": round(2 * B * L * 3 * H * D * 2 / prep_s / 1e9, 1)},
    }
    if TRAFFIC_FILE.exists():
        measured = json.loads(TRAFFIC_FILE.read_text())["hbm_bytes_per_launch"]
        for key, kernel in (("roofline", DENSE_KERNEL), ("roofline_band", BAND_KERNEL)):
            result[key]["traffic"] = measured.get(kernel)
            result[key]["traffic_source"] = str(TRAFFIC_FILE.relative_to(ROOT))
    if not args.no_extras and not args.kernels_only:
        print("[bench] extra shapes", file=sys.stderr, flush=True)
        result["extra_shapes"] = extra_shapes(lib, sp, stream, dev)
    if not args.no_cpu and not args.kernels_only:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
