"""The DiT projections on the GPU: hb_proj (`x @ W^T`), hb_dit_qkv_proj (to_qkv with the key preparation in its
epilogue) and hb_dense_attend_qq (the attention over its output).

* hb_proj against the product computed in float64 on the CPU and rounded once to the compute dtype: every element
  within one rounding step, nearly all equal (the fp32 accumulation order differs);
* hb_dit_qkv_proj's q / q_diff rows the same way, and the workspace rows past L zero;
* the fused block (qkv_proj -> attend_qq -> hb_proj) against the unfused one (torch GEMM -> hb_dense_diffattn ->
  torch GEMM), and config 0 (to_qkv -> attention -> to_out at L = 216, 24 heads, bf16) against the oracle at the
  bf16 contract (max-abs <= 2e-2, cosine >= 0.9999).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hummingbird_amd import dense_attention as da
from hummingbird_amd import projection, workloads
from oracle import bf16 as obf16
from oracle import dense as odense
from tests.util import assert_bf16_parity, stats

pytestmark = pytest.mark.gpu
DEV = "cuda"


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def within_one_step(got: np.ndarray, ref: np.ndarray, what: str, frac_equal: float = 0.98, atol: float = 1e-5,
                    bits: int = 8) -> None:
    """Every element within one step (`bits` significant bits: 8 for bf16, 11 for half) of the float64 product
    rounded once, plus `atol` for the fp32 accumulation's absolute error where the product nearly cancels (about
    sqrt(K) * 2^-24 at these scales); nearly all elements equal."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    step = np.ldexp(1.0, np.frexp(np.maximum(np.abs(ref), np.abs(got)))[1] - bits) + atol  # one step (bound)
    diff = np.abs(got - ref)
    assert np.isfinite(got).all(), f"{what}: non-finite"
    assert (diff <= step).all(), f"{what}: {int((diff > step).sum())} elements over one step"
    assert (diff == 0).mean() >= frac_equal, f"{what}: only {(diff == 0).mean():.4f} equal"


def rand(shape, std, gen, dtype=torch.bfloat16):
    return (torch.randn(shape, device=DEV, generator=gen) * std).to(dtype)


ROUND = {torch.bfloat16: (obf16.round_bf16, 8), torch.float16: (obf16.round_fp16, 11)}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("n,k,f", [(1, 64, 256), (300, 128, 512), (5168, 1536, 1536)], ids=lambda v: str(v))
def test_linear_vs_float64(n, k, f, dtype):
    announce(f"hb_proj N={n} K={k} F={f} {dtype}")
    gen = torch.Generator(device=DEV).manual_seed(n + k)
    x, w = rand((n, k), 1.0, gen, dtype), rand((f, k), k ** -0.5, gen, dtype)
    got = projection.linear(x, w).float().cpu().numpy()
    rnd, bits = ROUND[dtype]
    ref = rnd((x.double().cpu() @ w.double().cpu().T).numpy().astype(np.float32))
    within_one_step(got, ref, f"linear {n}x{k}x{f}", bits=bits)


def qkv_case(B, L, H, half, seed, E=None, dtype=torch.bfloat16):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    D = 64
    E = E or H * D
    h = rand((B, L, E), 1.0, gen, dtype)
    w_qkv = rand((5 * H * D, E), E ** -0.5, gen, dtype)
    w_o = rand((E, H * D), (H * D) ** -0.5, gen, dtype)
    qw = 1 + 0.02 * torch.randn(D, device=DEV, generator=gen)
    kw = 1 + 0.02 * torch.randn(D, device=DEV, generator=gen)
    lam = 0.2 + 0.6 * torch.rand(H, device=DEV, generator=gen)
    valid = torch.ones((B, L), device=DEV)
    for b in range(B):
        valid[b, L - (16 + 37 * b) % max(1, L // 3):] = 0
    cos, sin, mask = da.tables(L, torch.from_numpy(workloads.inv_freq(half)).to(DEV), valid, D, dtype)
    return dict(B=B, L=L, H=H, D=D, E=E, half=half, h=h, w_qkv=w_qkv, w_o=w_o, qw=qw, kw=kw, lam=lam, valid=valid,
                cos=cos, sin=sin, mask=mask)


@pytest.mark.parametrize("shape", [(1, 7, 4, 32, "bf16"), (2, 150, 4, 16, "bf16"), (2, 300, 8, 0, "bf16"),
                                   (1, 216, 24, 32, "bf16"), (2, 150, 4, 16, "fp16")],
                         ids=lambda s: "B%dL%dH%dh%d_%s" % s)
def test_qkv_proj_queries_and_padding(shape):
    B, L, H, half, name = shape
    dtype = {"bf16": torch.bfloat16, "fp16": torch.float16}[name]
    announce(f"qkv_proj queries {shape}")
    c = qkv_case(B, L, H, half, seed=L + H, dtype=dtype)
    qq, ws = projection.qkv_projection(c["h"], c["w_qkv"], c["kw"], c["cos"], c["sin"], c["mask"], H, 64, half, 1e-6)
    HD = H * 64
    rnd, bits = ROUND[dtype]
    ref = rnd((c["h"].double().cpu() @ c["w_qkv"].double().cpu().T).numpy().astype(np.float32))
    got = qq.float().cpu().numpy()
    within_one_step(got[..., :HD], ref[..., :HD], "q", bits=bits)
    within_one_step(got[..., HD:], ref[..., 3 * HD:4 * HD], "q_diff", bits=bits)
    # workspace rows past L (up to the 128-row padding) are zero in all three regions
    Lp = -(-L // 128) * 128
    region = B * H * Lp * 64
    wsv = ws.view(torch.bfloat16)[:3 * region].float().reshape(3, B, H, Lp, 64)  # -0.0 counts as zero
    if Lp > L:
        assert bool((wsv[:2, :, :, L:] == 0).all())
    vt = wsv[2].reshape(B, H, Lp // 64, 64, 64)  # [tile][d][pos]
    last, keys = L // 64, L % 64
    if keys:  # positions of keys >= L in the last tile hold zeros
        pos = [p for p in range(64) if (p & ~12 | ((p & 4) << 1) | ((p & 8) >> 1)) >= keys]
        assert bool((vt[:, :, last, :, pos] == 0).all())
    assert bool((vt[:, :, last + 1:] == 0).all())


@pytest.mark.parametrize("shape", [(2, 150, 4, 16, "bf16"), (1, 333, 8, 32, "bf16"), (2, 2584, 24, 32, "bf16"),
                                   (1, 333, 8, 32, "fp16")], ids=lambda s: "B%dL%dH%dh%d_%s" % s)
def test_fused_block_vs_unfused(shape):
    """qkv_proj -> attend_qq -> hb_proj against torch's GEMM -> hb_dense_diffattn -> torch's GEMM on the same
    weights: the only differences are the GEMMs' fp32 summation orders."""
    B, L, H, half, name = shape
    announce(f"fused block vs unfused {shape}")
    c = qkv_case(B, L, H, half, seed=7 * L + H, dtype={"bf16": torch.bfloat16, "fp16": torch.float16}[name])
    qq, ws = projection.qkv_projection(c["h"], c["w_qkv"], c["kw"], c["cos"], c["sin"], c["mask"], H, 64, half, 1e-6)
    att = projection.attend_projected(qq, c["qw"], c["kw"], c["cos"], c["sin"], H, 64, half, 1e-6, ws, lam=c["lam"])
    fused = projection.linear(att, c["w_o"])
    qkv = c["h"] @ c["w_qkv"].t()
    att_ref = da.dense_attention(qkv, c["qw"], c["kw"], c["cos"], c["sin"], c["mask"], H, 64, half, 1e-6, lam=c["lam"])
    unfused = att_ref @ c["w_o"].t()
    s_att = stats(att.float().cpu().numpy(), att_ref.float().cpu().numpy())
    assert s_att["max_abs"] <= 2e-2 and s_att["cosine"] >= 0.99995, f"attention: {s_att}"
    s = stats(fused.float().cpu().numpy(), unfused.float().cpu().numpy())
    assert s["max_abs"] <= 2e-2 and s["cosine"] >= 0.99995, f"block: {s}"


def test_config0_fused_block_vs_oracle():
    """Config 0 in bf16 on the GPU: x ~ N(0,1) (1, 216, 1536), W ~ N(0, 1/1536), gains 1 + N(0, 0.02), RoPE over the
    full head_dim (half 32), lambda ~ U(0.2, 0.8), the last 16 tokens masked; to_qkv -> attention -> to_out through
    the fused projections, against the oracle's XLA chain with the bf16 cast points (qkv rounded, the attention of
    oracle.dense.dense_xla, the to_out product rounded)."""
    from bench import config0_inputs

    announce("config 0 fused block vs oracle")
    c0 = config0_inputs()
    H, D = c0["heads"], c0["head_dim"]
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    x = to(obf16.round_bf16(c0["x"])).to(torch.bfloat16)
    w_qkv, w_o = to(c0["w_qkv"]).to(torch.bfloat16), to(c0["w_o"]).to(torch.bfloat16)
    cos, sin, mask = da.tables(216, to(c0["inv_freq"]), to(c0["valid"]), D, torch.bfloat16)
    qq, ws = projection.qkv_projection(x, w_qkv, to(c0["k_weight"]), cos, sin, mask, H, D, 32, 1e-6)
    att = projection.attend_projected(qq, to(c0["q_weight"]), to(c0["k_weight"]), cos, sin, H, D, 32, 1e-6, ws,
                                      lam=to(c0["lam"]))
    got = projection.linear(att, w_o).float().cpu().numpy()
    xf, wq, wo = x.double().cpu().numpy(), w_qkv.double().cpu().numpy(), w_o.double().cpu().numpy()
    qkv = obf16.round_bf16((xf @ wq.T).astype(np.float32))
    att_ref = odense.dense_xla(qkv, c0["q_weight"], c0["k_weight"], c0["inv_freq"], c0["valid"], H, D, 1e-6, c0["lam"],
                               "bf16")
    ref = obf16.round_bf16((att_ref.astype(np.float64) @ wo.T).astype(np.float32))
    assert_bf16_parity(att.float().cpu().numpy(), att_ref, "config 0 attention vs oracle")
    assert_bf16_parity(got, ref, "config 0 block vs oracle")
