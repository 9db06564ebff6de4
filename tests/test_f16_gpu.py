"""The reference's FP16 preset (sa3jax/dtypes.py:50-58) on the GPU: half-precision qkv and out.

Under it the reference's fused kernels round the RMSNorm and RoPE outputs to half (dense_attention.py:66, 69), then
K, q * scale, P and V to bf16 for the matrix unit (75-77, 83, 90; band_attention.py:85, 94, 101), and cast the fp32
difference to half (dense_attention.py:94, band_attention.py:120). The kernels here follow those cast points.

Each case is checked against the oracle's fp16 XLA-chain profile at the bf16 contract (max-abs <= 2e-2, cosine >=
0.9999; the operands are bf16 as in the reference's kernels) and, where small, against the fp16 fused-kernel
profile more tightly; the 120 s shapes against the torch restatement of the XLA chain in half on the GPU plus one
head against the oracle; the caller mirrors with the FP16 preset against attention="xla"; the DyT and GLU kernels
within one half step of the oracle.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from hummingbird_amd import dit, elementwise, same_l, workloads, xla_chain
from hummingbird_amd.config import MEDIUM_DIT, MEDIUM_SAME_L, SameConfig
from hummingbird_amd.dtypes import FP16
from oracle import band as oband
from oracle import block as oblock
from oracle import cross as ocross
from oracle import dense as odense
from tests.test_band_gpu import norm_t
from tests.test_band_gpu import run_hip as band_hip
from tests.test_callers import dit_case
from tests.test_cross_gpu import run_hip as cross_hip
from tests.test_dense_gpu import run_hip as dense_hip
from tests.util import assert_bf16_parity, stats

pytestmark = pytest.mark.gpu
DEV = "cuda"
H16 = torch.float16


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def head_columns(h: int, heads: int, d: int) -> np.ndarray:
    hd = heads * d
    return np.concatenate([np.arange(s * hd + h * d, s * hd + h * d + d) for s in range(5)])


DENSE = [  # (B, L, H, D, half)
    (2, 7, 2, 64, 16), (1, 216, 24, 64, 16), (2, 129, 2, 64, 32), (1, 300, 2, 64, 0), (2, 216, 2, 128, 64),
    (1, 150, 2, 128, 40),
]


@pytest.mark.parametrize("shape", DENSE, ids=lambda s: "B%dL%dH%dD%dh%d" % s)
def test_dense_f16_vs_oracle(shape):
    b, length, h, d, half = shape
    announce(f"dense fp16 {shape}")
    inp = workloads.dense_inputs(b, length, h, d, seed=length + d + 16, half=half, dtype="fp16", ragged=True)
    got = dense_hip(inp, dtype=H16)
    args = (inp["qkv"], inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"], h, d, inp["eps"], inp["lam"])
    assert_bf16_parity(got, odense.dense_xla(*args, "fp16"), f"fp16 {shape} vs xla")
    s = stats(got, odense.dense_fused(*args, "fp16"))
    assert s["max_abs"] <= 8e-3 and s["cosine"] >= 0.99995, f"fp16 {shape} vs fused profile: {s}"


def test_dense_f16_120s_vs_torch_chain():
    cfg = workloads.DENSE_120S
    announce(f"dense fp16 120s {cfg}")
    B, L, H, D = cfg["batch"], cfg["length"], cfg["heads"], cfg["head_dim"]
    inp = workloads.dense_inputs(B, L, H, D, seed=16, dtype="fp16")
    got = dense_hip(inp, dtype=H16)
    t = lambda a: torch.from_numpy(a).to(DEV)  # noqa: E731
    ref = xla_chain.dense_chain(t(inp["qkv"]).to(H16), t(inp["q_weight"]), t(inp["k_weight"]), t(inp["inv_freq"]),
                                t(inp["valid"]), H, D, inp["eps"], lam=t(inp["lam"])).float().cpu().numpy()
    assert_bf16_parity(got, ref, "fp16 120s vs torch chain")
    h = 7
    sub = np.ascontiguousarray(inp["qkv"][1:2, :, head_columns(h, H, D)])
    exp = odense.dense_xla(sub, inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"][1:2], 1, D,
                           inp["eps"], inp["lam"][h:h + 1], "fp16")[0]
    assert_bf16_parity(got[1, :, h * D:(h + 1) * D], exp, "fp16 120s head 7 vs oracle")


BAND = [  # (B, S, H, D, window, half): the ring kernel (D = 64, w <= 128) and the tiled pair (w = 256, D = 128)
    (1, 300, 2, 64, 17, 16), (2, 700, 2, 64, 128, 32), (1, 9000, 3, 64, 64, 32), (1, 3000, 2, 64, 256, 32),
    (1, 2000, 2, 128, 128, 64), (1, 6000, 2, 64, 40, 32), (1, 6000, 2, 64, 100, 32),
]


@pytest.mark.parametrize("shape", BAND, ids=lambda s: "B%dS%dH%dD%dw%dh%d" % s)
def test_band_f16_vs_oracle(shape):
    b, s, h, d, w, half = shape
    announce(f"band fp16 {shape}")
    inp = workloads.band_inputs(b, s, h, d, w, seed=s + w + 16, half=half, dtype="fp16")
    got = band_hip(inp, dtype=H16)
    args = (inp["qkv"], inp["q_norm"], inp["k_norm"], inp["inv_freq"], h, d, w, inp["lam"])
    assert_bf16_parity(got, oband.band_xla(*args, "fp16"), f"fp16 {shape} vs xla")
    st = stats(got, oband.band_fused(*args, "fp16"))
    assert st["max_abs"] <= 8e-3 and st["cosine"] >= 0.99995, f"fp16 {shape} vs fused profile: {st}"


def test_band_f16_120s_vs_torch_chain():
    cfg = workloads.BAND_120S
    S, H, D, w = cfg["length"], cfg["heads"], cfg["head_dim"], cfg["window"]
    announce(f"band fp16 120s S={S} H={H} w={w}")
    inp = workloads.band_inputs(1, S, H, D, w, seed=17, dtype="fp16")
    got = band_hip(inp, dtype=H16)
    t = lambda a: torch.from_numpy(np.asarray(a)).to(DEV)  # noqa: E731
    ref = xla_chain.band_chain(t(inp["qkv"]).to(H16), norm_t(inp["q_norm"]), norm_t(inp["k_norm"]),
                               t(inp["inv_freq"]), H, D, w, lam=t(inp["lam"])).float().cpu().numpy()
    assert_bf16_parity(got, ref, "fp16 120s vs torch chain")
    h = H - 1
    qkv = np.ascontiguousarray(inp["qkv"][:, :, head_columns(h, H, D)])
    exp = oband.band_xla(qkv, inp["q_norm"], inp["k_norm"], inp["inv_freq"], 1, D, w, inp["lam"][h:h + 1], "fp16")[0]
    for lo, hi in ((0, 700), (S - 700, S)):
        assert_bf16_parity(got[0, lo:hi, h * D:(h + 1) * D], exp[lo:hi], f"fp16 120s rows [{lo},{hi}) vs oracle")


@pytest.mark.parametrize("shape", [(2, 100, 17, 2, 64), (1, 300, 257, 2, 64), (2, 216, 64, 3, 128)],
                         ids=lambda s: "B%dL%dNk%dH%dD%d" % s)
def test_cross_f16_vs_oracle(shape):
    b, length, nk, h, d = shape
    announce(f"cross fp16 {shape}")
    inp = workloads.cross_inputs(b, length, nk, h, d, seed=length + nk + 16, dtype="fp16")
    ref = ocross.cross_xla(inp["q"], inp["kv"], inp["q_weight"], inp["k_weight"], h, d, inp["eps"], inp["lam"],
                           "fp16")
    assert_bf16_parity(cross_hip(inp, H16), ref, f"cross fp16 {shape}")


def assert_within_one_half_step(got: np.ndarray, ref: np.ndarray, what: str, atol: float = 0.0) -> None:
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    step = np.maximum(np.abs(ref), 6.1e-5) * 2.0 ** -10 + atol  # the spacing of half values around ref (bound)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert (np.abs(got - ref) <= step).all(), f"{what}: {int((np.abs(got - ref) > step).sum())} elements off"
    assert float((got != ref).mean()) <= 0.01, f"{what}: {float((got != ref).mean()):.3%} of the elements differ"


@pytest.mark.parametrize("sine", [False, True], ids=["silu", "sine"])
def test_dyt_and_glu_f16_vs_oracle(sine):
    rng = np.random.default_rng(16)
    announce(f"dyt + glu fp16 sine={sine}")
    n, c, f = 500, 512, 1536
    x = torch.from_numpy((rng.standard_normal((n, c)) * 3).astype(np.float32)).to(DEV, H16)
    norm = {"alpha": np.float32(0.7), "gamma": (1 + 0.3 * rng.standard_normal(c)).astype(np.float32),
            "beta": (0.1 * rng.standard_normal(c)).astype(np.float32)}
    got = elementwise.dyt(x, {k: torch.as_tensor(v).to(DEV) for k, v in norm.items()}).float().cpu().numpy()
    scale = float(np.max(np.abs(norm["gamma"]) + np.abs(norm["beta"])))
    assert_within_one_half_step(got, oblock.dyt_cast(x.float().cpu().numpy(), norm, "fp16"), "dyt fp16",
                                atol=scale * 2.0 ** -21)
    proj = torch.from_numpy((rng.standard_normal((n, 2 * f)) * 2).astype(np.float32)).to(DEV, H16)
    got = elementwise.glu(proj, sine).float().cpu().numpy()
    assert_within_one_half_step(got, oblock.glu(proj.float().cpu().numpy(), sine, "fp16"), "glu fp16")


def test_dit_self_attention_fp16_preset_hip_vs_xla_and_oracle():
    """Config 0's geometry (L = 216 = 64 memory + 152 latent tokens, 24 heads of 64, partial rotary half 16) with the
    FP16 preset: to_qkv -> attention -> to_out, attention="hip" against attention="xla" on the same device, and the
    attention output against the oracle's fp16 profile."""
    announce("dit.self_attention FP16 preset")
    cfg = MEDIUM_DIT
    h, valid, inv_freq, block, lam = dit_case(cfg, 1, 216 - cfg.num_memory_tokens, seed=16)
    h = h.to(DEV)
    block = {"self_attn": {k: {"weight": v["weight"].to(DEV)} for k, v in block["self_attn"].items()}}
    inv_freq, valid, lam = inv_freq.to(DEV), valid.to(DEV), lam.to(DEV)
    got = dit.self_attention(h, block, dit.static_tables(inv_freq, valid, cfg, FP16), cfg, lam=lam, dtype=FP16)
    assert got.dtype == H16
    xcfg = dataclasses.replace(cfg, attention="xla")
    ref = dit.self_attention(h, block, dit.static_tables(inv_freq, valid, xcfg, FP16), xcfg, lam=lam, dtype=FP16)
    s = stats(got.float().cpu().numpy(), ref.float().cpu().numpy())
    assert s["cosine"] >= 0.9999 and s["max_abs"] <= 2e-2 * max(1.0, float(ref.abs().max())), f"dit fp16: {s}"
    # the attention step alone against the oracle (the projections are the same torch GEMM in both paths)
    qkv = (h.to(H16) @ block["self_attn"]["to_qkv"]["weight"].to(H16).t()).float().cpu().numpy()
    statics = dit.static_tables(inv_freq, valid, cfg, FP16)
    from hummingbird_amd import dense_attention as da
    att = da.dense_attention(torch.from_numpy(qkv).to(DEV, H16), block["self_attn"]["q_norm"]["weight"],
                             block["self_attn"]["k_norm"]["weight"], statics["hip_cos"], statics["hip_sin"],
                             statics["hip_mask"], cfg.num_heads, cfg.head_dim, cfg.rope_dim // 2, cfg.qk_norm_eps,
                             lam=lam).float().cpu().numpy()
    exp = odense.dense_xla(qkv, block["self_attn"]["q_norm"]["weight"].cpu().numpy(),
                           block["self_attn"]["k_norm"]["weight"].cpu().numpy(), inv_freq.cpu().numpy(),
                           statics["valid"].float().cpu().numpy(), cfg.num_heads, cfg.head_dim, cfg.qk_norm_eps,
                           lam.cpu().numpy(), "fp16")
    assert_bf16_parity(att, exp, "dit fp16 attention vs oracle")


def test_same_l_attention_fp16_preset_hip_vs_xla():
    announce("same_l.attention FP16 preset")
    cfg = MEDIUM_SAME_L
    rng = np.random.default_rng(161)
    S, E = 1500, cfg.dim
    x = torch.from_numpy(rng.standard_normal((1, S, E)).astype(np.float32)).to(DEV)
    w = lambda *s: torch.from_numpy((rng.standard_normal(s) / np.sqrt(E)).astype(np.float32)).to(DEV)  # noqa: E731
    dyt = lambda: {"alpha": torch.tensor(0.5, device=DEV), "gamma": torch.from_numpy(  # noqa: E731
        (1 + 0.02 * rng.standard_normal(64)).astype(np.float32)).to(DEV),
        "beta": torch.from_numpy((0.02 * rng.standard_normal(64)).astype(np.float32)).to(DEV)}
    block = {"self_attn": {"to_qkv": {"weight": w(5 * E, E)}, "to_out": {"weight": w(E, E)}, "q_norm": dyt(),
                           "k_norm": dyt()}, "rope_inv_freq": torch.from_numpy(workloads.inv_freq(16)).to(DEV)}
    lam = torch.from_numpy(rng.uniform(0.2, 0.8, cfg.num_heads).astype(np.float32)).to(DEV)
    got = same_l.attention(x, block, cfg, lam=lam, dtype=FP16)
    assert got.dtype == H16
    ref = same_l.attention(x, block, dataclasses.replace(cfg, attention="xla"), lam=lam, dtype=FP16)
    assert_bf16_parity(got.float().cpu().numpy(), ref.float().cpu().numpy(), "same_l fp16")


def test_same_l_blocks_fp16_hip_vs_xla():
    """Two SAME-L decoder blocks (a SiLU and a sine block; dim 128 = 2 heads of 64, ff 384, half-width 17) in half
    through `same_l.blocks`: attention="hip" (band kernel, hb_dyt, hb_glu, hb_residual_dyt) against "xla", at the
    contract on the output divided by its largest magnitude."""
    announce("same_l.blocks FP16")
    from tests.block_util import block_params, to_torch
    kw = dict(channels=64, c_mults=(2,), stride=16, transformer_depth=2, sinusoidal_blocks=2)  # block 1 has the sine
    ps = [to_torch(block_params(128, 2, 384, seed=90 + i), DEV, H16) for i in (2, 3)]
    x = torch.from_numpy(np.random.default_rng(91).standard_normal((1, 700, 128)).astype(np.float32)).to(DEV, H16)
    cfg = SameConfig(**kw, attention="hip")
    assert not cfg.sinusoidal(0) and cfg.sinusoidal(1)
    got = same_l.blocks(x, ps, cfg)
    ref = same_l.blocks(x, ps, dataclasses.replace(cfg, attention="xla"))
    assert got.dtype == H16 and ref.dtype == H16
    scale = max(1.0, float(ref.float().abs().max()))
    assert_bf16_parity(got.float().cpu().numpy() / scale, ref.float().cpu().numpy() / scale, "blocks fp16 (/max)")
