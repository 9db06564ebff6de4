"""GPU parity of the band differential attention (hb_band_diffattn) against the oracle.

Small shapes (including the edges of the sequence, windows of 0, 1, 17, 64, 128 and 400, head_dim 128) run
against the NumPy oracle's XLA-chain profile (the contract) and the fused-kernel profile (tighter); multi-block
shapes on both kernels (the streaming ring for w <= 128 at head_dim 64, the tiled kernels otherwise) and the
120 s and 380 s shapes run against the torch restatement of the XLA chain on the GPU and through
size-independent properties.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hummingbird_amd import band_attention as ba
from hummingbird_amd import workloads, xla_chain
from oracle import band as oband
from tests.util import assert_bf16_parity, assert_fp32_parity, stats

pytestmark = pytest.mark.gpu
DEV = "cuda"


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def norm_t(n: dict) -> dict:
    return {k: torch.as_tensor(np.asarray(v)).to(DEV) for k, v in n.items()}


def run_hip(inp: dict, dtype=torch.bfloat16, lam=True, qkv_override=None) -> np.ndarray:
    qkv = torch.from_numpy(inp["qkv"] if qkv_override is None else qkv_override).to(DEV, dtype)
    out = ba.band_attention(qkv, norm_t(inp["q_norm"]), norm_t(inp["k_norm"]), torch.from_numpy(inp["inv_freq"]).to(DEV),
                            inp["heads"], inp["head_dim"], inp["window"],
                            lam=torch.from_numpy(inp["lam"]).to(DEV) if lam else None)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def oracle(inp: dict, profile="xla", compute="bf16", lam=True, qkv_override=None) -> np.ndarray:
    fn = oband.band_xla if profile == "xla" else oband.band_fused
    qkv = inp["qkv"] if qkv_override is None else qkv_override
    return fn(qkv, inp["q_norm"], inp["k_norm"], inp["inv_freq"], inp["heads"], inp["head_dim"], inp["window"],
              inp["lam"] if lam else None, compute)


SMALL = [  # (B, S, H, D, window, half)
    (1, 1, 2, 64, 17, 32), (2, 17, 2, 64, 17, 16), (1, 100, 2, 64, 0, 32), (1, 100, 2, 64, 1, 32),
    (1, 300, 2, 64, 17, 16), (2, 300, 2, 64, 64, 32), (1, 700, 2, 64, 128, 32), (1, 333, 1, 64, 400, 32),
    (1, 260, 2, 128, 64, 64), (1, 200, 2, 64, 128, 0),
    # rotary half-widths that are not a multiple of 8 (the wrapper reorders the q and k dims): ring and tiled
    (1, 300, 2, 64, 17, 12), (1, 700, 2, 64, 128, 20), (1, 260, 2, 128, 64, 36), (1, 333, 1, 64, 200, 5),
]


@pytest.mark.parametrize("shape", SMALL, ids=lambda s: "B%dS%dH%dD%dw%dh%d" % s)
def test_band_small_vs_oracle(shape):
    b, s, h, d, w, half = shape
    announce(f"band bf16 {shape}")
    inp = workloads.band_inputs(b, s, h, d, w, seed=s + w, half=half)
    got = run_hip(inp)
    assert_bf16_parity(got, oracle(inp, "xla"), f"xla {shape}")
    # tighter check against the fused-kernel cast points (the max-free path also folds log2(e) into bf16 q)
    st = stats(got, oracle(inp, "fused"))
    assert st["max_abs"] <= 8e-3 and st["cosine"] >= 0.99995, f"fused-profile {shape}: {st}"


def test_band_large_gamma_takes_running_max_path():
    """gamma ~ 8 makes the logit bound exceed 64, so the running-max softmax runs. Logits reach ~50 here and
    the XLA chain keeps q/k in fp32 while both fused kernels (the reference's and this one) round them to bf16,
    so the reference's own fused kernel already sits ~0.09 from its XLA chain (> the 2e-2 contract). The
    contract is therefore held against the fused-kernel cast points, and the XLA deviation is bounded by the
    reference kernel's own."""
    announce("band bf16 gamma 8 (running-max path)")
    inp = workloads.band_inputs(1, 400, 2, 64, 64, seed=3, gamma_mean=8.0)
    got, xla, fused = run_hip(inp), oracle(inp, "xla"), oracle(inp, "fused")
    assert_bf16_parity(got, fused, "large gamma vs fused profile")
    ours, theirs = stats(got, xla), stats(fused, xla)
    assert ours["max_abs"] <= 1.25 * theirs["max_abs"] and ours["cosine"] >= 1 - 1.25 * (1 - theirs["cosine"]), \
        (ours, theirs)


def test_band_identical_branches_cancel():
    announce("band bf16 identical branches")
    inp = workloads.band_inputs(1, 500, 2, 64, 128, seed=4)
    qkv = inp["qkv"].copy()
    hd = 2 * 64
    qkv[..., 3 * hd:4 * hd] = qkv[..., 0:hd]
    qkv[..., 4 * hd:5 * hd] = qkv[..., hd:2 * hd]
    inp["q_norm"] = inp["k_norm"] = inp["q_norm"]
    assert np.count_nonzero(run_hip(inp, lam=False, qkv_override=qkv)) == 0


def test_band_wide_window_equals_dense_attention():
    # w >= S - 1: every key is in band, so each branch is plain softmax attention over the whole sequence.
    announce("band bf16 window >= S-1")
    inp = workloads.band_inputs(1, 190, 2, 64, 189, seed=5)
    wide = dict(inp, window=1000)
    a, b = run_hip(inp), run_hip(wide)
    assert np.array_equal(a, b)


FP32_SHAPES = [  # (B, S, H, D, window, half)
    (1, 300, 2, 64, 17, 32), (1, 100, 2, 64, 0, 32), (2, 257, 2, 64, 64, 16), (1, 300, 2, 128, 17, 64),
    (1, 50, 2, 64, 60, 0), (1, 1000, 1, 64, 128, 32), (1, 300, 2, 64, 17, 12), (1, 257, 2, 128, 64, 44),
]


@pytest.mark.parametrize("shape", FP32_SHAPES, ids=lambda s: "B%dS%dH%dD%dw%dh%d" % s)
def test_band_fp32_vs_oracle(shape):
    b, length, h, d, w, half = shape
    announce(f"band fp32 {shape}")
    inp = workloads.band_inputs(b, length, h, d, w, seed=6 + length, dtype="fp32", half=half)
    got = run_hip(inp, dtype=torch.float32)
    assert_fp32_parity(got, oracle(inp, "xla", compute="fp32"), f"fp32 {shape}")


@pytest.mark.parametrize("shape", FP32_SHAPES[:4] + [(1, 1000, 1, 64, 100, 32)], ids=lambda s: "B%dS%dH%dD%dw%dh%d" % s)
def test_band_fp32_without_workspace_vs_oracle(shape):
    """The fp32 band call with a NULL workspace (each query block prepares its own key window) against the oracle
    and against the call with a workspace (every key prepared once), through the C ABI."""
    from hummingbird_amd import _lib

    b, length, h, d, w, half = shape
    announce(f"band fp32 without workspace {shape}")
    inp = workloads.band_inputs(b, length, h, d, w, seed=16 + length, dtype="fp32", half=half)
    lib = _lib.load()
    qkv = torch.from_numpy(inp["qkv"]).to(DEV)
    qd, kd = ba.pack_dyt(norm_t(inp["q_norm"]), d, DEV), ba.pack_dyt(norm_t(inp["k_norm"]), d, DEV)
    cos, sin = ba.rope_tables(length, torch.from_numpy(inp["inv_freq"]).to(DEV))
    lam = torch.from_numpy(inp["lam"]).to(DEV)
    need = int(lib.hb_band_workspace_size(_lib.HB_F32, b, length, h, d, half, w))
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    outs = []
    stream = torch.cuda.current_stream().cuda_stream
    for ws_p, ws_b in ((0, 0), (ws.data_ptr(), need)):
        out = torch.empty((b, length, h * d), dtype=torch.float32, device=DEV)
        _lib.check(lib.hb_band_diffattn(stream, qkv.data_ptr(), _lib.HB_F32, 5 * h * d, qd.data_ptr(), kd.data_ptr(),
                                        cos.data_ptr() if half else 0, sin.data_ptr() if half else 0, half, w,
                                        lam.data_ptr(), out.data_ptr(), b, length, h, d, ws_p, ws_b), "band fp32")
        outs.append(out.cpu().numpy())
    ref = oracle(inp, "xla", compute="fp32")
    assert_fp32_parity(outs[0], ref, f"fp32 no workspace {shape}")
    assert_fp32_parity(outs[1], ref, f"fp32 workspace {shape}")
    assert_fp32_parity(outs[0], outs[1], f"fp32 with vs without workspace {shape}")


def test_band_fp32_large_call_allocates_no_workspace(monkeypatch):
    """An fp32 call whose workspace would exceed band_attention.FP32_WORKSPACE_CAP, given none, runs without one
    (the kernel that prepares each query block's key window) instead of allocating it; with the cap lowered below
    a small call's need, the small call's output is the same as with its own workspace (fp32 parity)."""
    announce("band fp32 workspace cap")
    b, length, h, d, w, half = 1, 1000, 2, 64, 100, 32
    inp = workloads.band_inputs(b, length, h, d, w, seed=44, dtype="fp32", half=half)
    with_ws = run_hip(inp, dtype=torch.float32)
    allocs = []
    real_empty = torch.empty

    def spy(*a, **kw):
        if kw.get("dtype") is torch.uint8:
            allocs.append(a)
        return real_empty(*a, **kw)

    monkeypatch.setattr(ba, "FP32_WORKSPACE_CAP", 1024)
    monkeypatch.setattr(torch, "empty", spy)
    without = run_hip(inp, dtype=torch.float32)
    monkeypatch.undo()
    assert not allocs
    assert_fp32_parity(without, with_ws, "fp32 above the workspace cap vs with a workspace")
    assert_fp32_parity(without, oracle(inp, "xla", compute="fp32"), "fp32 above the workspace cap vs oracle")


def test_band_fp32_identical_branches_cancel():
    announce("band fp32 identical branches")
    inp = workloads.band_inputs(1, 300, 2, 64, 40, seed=5, dtype="fp32")
    qkv = inp["qkv"].copy()
    hd = 2 * 64
    qkv[..., 3 * hd:4 * hd] = qkv[..., 0:hd]
    qkv[..., 4 * hd:5 * hd] = qkv[..., hd:2 * hd]
    assert np.count_nonzero(run_hip(inp, dtype=torch.float32, lam=False, qkv_override=qkv)) == 0


def test_band_120s_vs_torch_chain():
    cfg = workloads.BAND_120S
    announce(f"band bf16 120s {cfg}")
    inp = workloads.band_inputs(cfg["batch"], cfg["length"], cfg["heads"], cfg["head_dim"], cfg["window"], seed=1)
    got = run_hip(inp)
    qkv = torch.from_numpy(inp["qkv"]).to(DEV, torch.bfloat16)
    ref = xla_chain.band_chain(qkv, norm_t(inp["q_norm"]), norm_t(inp["k_norm"]),
                               torch.from_numpy(inp["inv_freq"]).to(DEV), cfg["heads"], cfg["head_dim"], cfg["window"],
                               lam=torch.from_numpy(inp["lam"]).to(DEV)).float().cpu().numpy()
    assert_bf16_parity(got, ref, "120s")
    # the last 700 positions of head 3 against the oracle (the sequence end is an edge of the band)
    h, tail = 3, 700
    hd = cfg["heads"] * cfg["head_dim"]
    cols = np.concatenate([np.arange(s * hd + h * 64, s * hd + h * 64 + 64) for s in range(5)])
    full_head = dict(inp, qkv=np.ascontiguousarray(inp["qkv"][:, :, cols]), heads=1, lam=inp["lam"][h:h + 1])
    ref_head = oracle(full_head, "xla")[0]
    assert_bf16_parity(got[0, -tail:, h * 64:(h + 1) * 64], ref_head[-tail:], "120s head 3 tail vs oracle")


def test_band_380s_vs_torch_chain():
    """The 380 s clip shape (S=261760 frames, 8 heads of 64, w=128): 4090 steps per head over the ring, checked
    against the torch restatement of the XLA chain on the GPU (inputs drawn on the device)."""
    S, H, D, w = 261760, 8, 64, 128
    announce(f"band bf16 380s S={S} H={H} w={w}")
    gen = torch.Generator(device=DEV).manual_seed(381)
    qkv = torch.randn((1, S, 5 * H * D), device=DEV, generator=gen).to(torch.bfloat16)
    norm = lambda: {"alpha": torch.tensor(0.5, device=DEV),  # noqa: E731
                    "gamma": 1 + 0.02 * torch.randn(D, device=DEV, generator=gen),
                    "beta": 0.02 * torch.randn(D, device=DEV, generator=gen)}
    qn, kn = norm(), norm()
    lam = 0.2 + 0.6 * torch.rand(H, device=DEV, generator=gen)
    freq = torch.from_numpy(workloads.inv_freq(32)).to(DEV)
    got = ba.band_attention(qkv, qn, kn, freq, H, D, w, lam=lam).float().cpu().numpy()
    ref = xla_chain.band_chain(qkv, qn, kn, freq, H, D, w, lam=lam).float().cpu().numpy()
    assert_bf16_parity(got, ref, "380s")
    # the last head through the oracle (all positions, so RoPE keeps its absolute angles), checked at both ends
    h = H - 1
    cols = torch.from_numpy(np.concatenate([np.arange(sec * H * D + h * D, sec * H * D + (h + 1) * D)
                                            for sec in range(5)])).to(DEV)
    head_qkv = qkv.index_select(2, cols).float().cpu().numpy()
    host = lambda n: {k: v.float().cpu().numpy() for k, v in n.items()}  # noqa: E731
    exp = oband.band_xla(head_qkv, host(qn), host(kn), freq.cpu().numpy(), 1, D, w, lam[h:h + 1].cpu().numpy())[0]
    for lo, hi in ((0, 300), (S - 300, S)):
        assert_bf16_parity(got[0, lo:hi, h * D:(h + 1) * D], exp[lo:hi], f"380s last head [{lo},{hi}) vs oracle")


RUNS = [  # (B, S, H, window, half, gamma_mean): several 64-query steps per workgroup, runs crossing heads/batches
    (2, 9000, 3, 128, 32, 1.0), (1, 20000, 2, 64, 16, 1.0), (2, 7001, 3, 17, 32, 1.0), (1, 18000, 1, 0, 32, 1.0),
    (1, 16500, 2, 100, 8, 1.0), (1, 9000, 3, 128, 24, 1.0), (2, 8000, 2, 128, 32, 8.0),
]


def check_vs_torch_chain(b, s, h, d, w, half, gm, label):
    """The whole output against the torch restatement of the XLA chain, and the first and last 300 positions of
    the last head against the oracle (the sequence edges)."""
    inp = workloads.band_inputs(b, s, h, d, w, seed=s + h + w, half=half, gamma_mean=gm)
    got = run_hip(inp)
    qkv = torch.from_numpy(inp["qkv"]).to(DEV, torch.bfloat16)
    ref = xla_chain.band_chain(qkv, norm_t(inp["q_norm"]), norm_t(inp["k_norm"]),
                               torch.from_numpy(inp["inv_freq"]).to(DEV), h, d, w,
                               lam=torch.from_numpy(inp["lam"]).to(DEV)).float().cpu().numpy()
    if gm == 1.0:
        assert_bf16_parity(got, ref, label)
    else:  # logits reach ~50 here: the XLA chain keeps q/k in fp32, the fused cast points round them to bf16
        assert stats(got, ref)["cosine"] >= 0.999, f"{label}: {stats(got, ref)}"
    hh = h - 1
    cols = np.concatenate([np.arange(sec * h * d + hh * d, sec * h * d + hh * d + d) for sec in range(5)])
    head = dict(inp, qkv=np.ascontiguousarray(inp["qkv"][-1:, :, cols]), heads=1, lam=inp["lam"][hh:hh + 1])
    if gm == 1.0:
        exp = oracle(head, "xla")[0]
        for lo, hi in ((0, 300), (s - 300, s)):
            assert_bf16_parity(got[-1, lo:hi, hh * d:(hh + 1) * d], exp[lo:hi], f"{label} [{lo},{hi}) vs oracle")
    else:  # the whole head against the fused-kernel cast points under the bf16 contract
        assert_bf16_parity(got[-1, :, hh * d:(hh + 1) * d], oracle(head, "fused")[0], f"{label} head vs fused oracle")


@pytest.mark.parametrize("shape", RUNS, ids=lambda s: "B%dS%dH%dw%dh%dg%g" % s)
def test_band_multistep_runs_vs_torch_chain(shape):
    """Shapes with more 64-query steps than CUs, so each workgroup streams a run of steps and some runs cross a
    (batch, head) boundary."""
    b, s, h, w, half, gm = shape
    announce(f"band bf16 multistep {shape}")
    check_vs_torch_chain(b, s, h, 64, w, half, gm, f"multistep {shape}")


# At least 16 steps per CU, with a (batch, head) count that does not divide the CU count: the ring kernel then
# splits the steps weighted by ring fills, so the workgroups that cross a (batch, head) boundary get fewer steps.
FILL_WEIGHTED = [  # (B, S, H, window, half, gamma_mean)
    (1, 23086, 24, 17, 16, 1.0),  # the reference decoder geometry
    (1, 50000, 6, 40, 32, 1.0),
    (2, 30000, 5, 128, 32, 1.0),
    (1, 90000, 3, 0, 32, 1.0),    # w = 0: the diagonal half only
]


@pytest.mark.parametrize("shape", FILL_WEIGHTED, ids=lambda s: "B%dS%dH%dw%dh%dg%g" % s)
def test_band_fill_weighted_split_vs_torch_chain(shape):
    b, s, h, w, half, gm = shape
    announce(f"band bf16 fill-weighted split {shape}")
    assert torch.cuda.get_device_properties(0).multi_processor_count % (b * h) != 0
    check_vs_torch_chain(b, s, h, 64, w, half, gm, f"fill-weighted {shape}")


# Windows at the edges of the ring kernel's interior-step patterns. For w in (64 (C - 1), 64 C] an interior
# step's attention wave attends the 32-key halves t = -T .. T around its own queries, T = floor((w + 31) / 32), and
# masks those with |t| >= M = floor((w + 1) / 32); the pattern changes at w = 64 C - 33, 64 C - 31 and 64 C - 1.
PATTERN_WINDOWS = [30, 31, 32, 33, 62, 63, 65, 94, 95, 96, 97, 126, 127]


@pytest.mark.parametrize("w", PATTERN_WINDOWS)
def test_band_interior_pattern_windows_vs_torch_chain(w):
    """Every interior-step pattern of the ring kernel, on both sides of each change, over multistep runs."""
    announce(f"band bf16 pattern window {w}")
    check_vs_torch_chain(1, 6000, 2, 64, w, 32, 1.0, f"pattern w={w}")


@pytest.mark.parametrize("w", [17, 40])
def test_band_interior_patterns_running_max_vs_fused_oracle(w):
    """Interior patterns with masked halves on the running-max softmax (gamma ~ 8 lifts the logit bound). Over so
    few keys the outputs reach magnitudes where one bf16 step exceeds the contract's absolute bound, so the
    contract is applied to the output divided by the reference's largest magnitude."""
    announce(f"band bf16 pattern window {w} gamma 8")
    inp = workloads.band_inputs(1, 6000, 2, 64, w, seed=6000 + w, half=32, gamma_mean=8.0)
    got = run_hip(inp)
    ref = oracle(inp, "fused")
    scale = float(np.abs(ref).max())
    assert_bf16_parity(got / scale, ref / scale, f"pattern w={w} gamma 8 vs fused oracle (scaled by {scale:.3g})")


TILED = [  # (B, S, H, D, window, half, gamma_mean): windows past 128 and head_dim 128 (the tiled kernels)
    (1, 5000, 2, 64, 256, 32, 1.0), (2, 3001, 2, 64, 129, 16, 1.0), (1, 4100, 1, 64, 700, 24, 1.0),
    (2, 3000, 2, 128, 128, 64, 1.0), (1, 4000, 2, 128, 300, 48, 1.0), (1, 3000, 2, 128, 17, 0, 1.0),
    (1, 3000, 2, 64, 200, 32, 8.0),
]


@pytest.mark.parametrize("shape", TILED, ids=lambda s: "B%dS%dH%dD%dw%dh%dg%g" % s)
def test_band_tiled_vs_torch_chain(shape):
    """Several 128-query blocks per head whose key windows overlap, partly in-band tiles, ragged last tiles."""
    b, s, h, d, w, half, gm = shape
    announce(f"band bf16 tiled {shape}")
    check_vs_torch_chain(b, s, h, d, w, half, gm, f"tiled {shape}")


def test_band_errors_are_value_errors():
    announce("band argument errors")
    qkv = torch.zeros((1, 8, 5 * 2 * 64), device=DEV, dtype=torch.bfloat16)
    n = {"alpha": 0.5, "gamma": torch.ones(64, device=DEV), "beta": torch.zeros(64, device=DEV)}
    with pytest.raises(ValueError):
        ba.band_attention(qkv, n, n, torch.ones(16, device=DEV), 2, 64, -1)
    with pytest.raises(ValueError):
        ba.band_attention(qkv, n, n, torch.ones(40, device=DEV), 2, 64, 4)


@pytest.mark.parametrize("half", [32, 12])
def test_band_explicit_tables_equal_the_built_ones(half):
    """`tables=(cos, sin)` from `rope_tables(S, inv_freq)` gives the output of the call that builds them itself, bit
    for bit, also for a rotary width that is not a multiple of 8 (padded and reordered inside); tables of another
    shape are refused."""
    announce(f"band explicit tables half={half}")
    inp = workloads.band_inputs(1, 500, 2, 64, 64, seed=77, half=half)
    qkv = torch.from_numpy(inp["qkv"]).to(DEV, torch.bfloat16)
    freq = torch.from_numpy(inp["inv_freq"]).to(DEV)
    qn, kn = norm_t(inp["q_norm"]), norm_t(inp["k_norm"])
    lam = torch.from_numpy(inp["lam"]).to(DEV)
    built = ba.band_attention(qkv, qn, kn, freq, 2, 64, 64, lam=lam)
    tabs = ba.rope_tables(500, freq)
    given = ba.band_attention(qkv, qn, kn, freq, 2, 64, 64, lam=lam, tables=tabs)
    torch.cuda.synchronize()
    assert torch.equal(built, given)
    with pytest.raises(ValueError):
        ba.band_attention(qkv, qn, kn, freq, 2, 64, 64, tables=(tabs[0][:499], tabs[1][:499]))
