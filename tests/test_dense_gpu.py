"""GPU parity of the dense differential attention (hb_dense_diffattn) against the oracle.

Small shapes run against the NumPy oracle's XLA-chain profile (the contract) and its fused-kernel profile
(tighter); the 120 s shape runs against the torch restatement of the XLA chain on the GPU and through
size-independent properties. Every case prints its name before touching the GPU.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hummingbird_amd import dense_attention as da
from hummingbird_amd import workloads, xla_chain
from oracle import dense as odense
from tests.util import assert_bf16_parity, assert_fp32_parity, stats

pytestmark = pytest.mark.gpu
DEV = "cuda"


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def run_hip(inp: dict, dtype=torch.bfloat16, lam=True, mask=True, qkv_override=None) -> np.ndarray:
    qkv = torch.from_numpy(inp["qkv"] if qkv_override is None else qkv_override).to(DEV, dtype)
    freq = torch.from_numpy(inp["inv_freq"]).to(DEV)
    valid = torch.from_numpy(inp["valid"]).to(DEV)
    cos, sin, m = da.tables(qkv.shape[1], freq, valid, inp["head_dim"], dtype)
    out = da.dense_attention(qkv, torch.from_numpy(inp["q_weight"]).to(DEV), torch.from_numpy(inp["k_weight"]).to(DEV),
                             cos, sin, m if mask else None, inp["heads"], inp["head_dim"], inp["half"], inp["eps"],
                             lam=torch.from_numpy(inp["lam"]).to(DEV) if lam else None)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def oracle(inp: dict, profile="xla", compute="bf16", lam=True, mask=True, qkv_override=None) -> np.ndarray:
    fn = odense.dense_xla if profile == "xla" else odense.dense_fused
    qkv = inp["qkv"] if qkv_override is None else qkv_override
    return fn(qkv, inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"] if mask else None, inp["heads"],
              inp["head_dim"], inp["eps"], inp["lam"] if lam else None, compute)


SMALL = [  # (B, L, H, D, half)
    (2, 1, 2, 64, 32), (2, 7, 2, 64, 16), (1, 64, 3, 64, 32), (2, 129, 2, 64, 16), (2, 216, 4, 64, 32),
    (1, 300, 2, 64, 0), (2, 216, 2, 128, 64), (1, 131, 2, 128, 32),
    # rotary half-widths whose RoPE partner group sits in the other half of a query row's lanes
    (1, 200, 2, 64, 24), (2, 100, 2, 64, 8), (1, 150, 2, 128, 40),
    # rotary half-widths that are not a multiple of 8 (the wrapper reorders the q and k dims)
    (1, 150, 2, 64, 12), (2, 129, 2, 64, 5), (1, 90, 2, 64, 31), (1, 100, 2, 128, 36),
]


@pytest.mark.parametrize("shape", SMALL, ids=lambda s: "B%dL%dH%dD%dh%d" % s)
def test_dense_small_vs_oracle(shape):
    b, length, h, d, half = shape
    announce(f"dense bf16 {shape}")
    inp = workloads.dense_inputs(b, length, h, d, seed=length + d, half=half, mask_tail=min(16, length // 4))
    got = run_hip(inp)
    assert_bf16_parity(got, oracle(inp, "xla"), f"xla {shape}")
    # tighter check against the fused-kernel cast points (the max-free path also folds log2(e) into bf16 q)
    s = stats(got, oracle(inp, "fused"))
    assert s["max_abs"] <= 8e-3 and s["cosine"] >= 0.99995, f"fused-profile {shape}: {s}"


def test_dense_ragged_mask_and_no_lambda():
    announce("dense bf16 ragged mask, lam=None")
    inp = workloads.dense_inputs(2, 200, 2, 64, seed=5, ragged=True)
    got = run_hip(inp, lam=False)
    assert_bf16_parity(got, oracle(inp, "xla", lam=False), "ragged")


def test_dense_no_mask_matches_all_ones_mask():
    announce("dense bf16 mask=None vs ones")
    inp = workloads.dense_inputs(1, 96, 2, 64, seed=6, mask_tail=0)
    assert np.array_equal(run_hip(inp, mask=False), run_hip(inp, mask=True))


def test_dense_large_gains_take_running_max_path():
    """Gains of 4 put the a-priori logit bound (about 11.5 * 16) above 64: the running-max softmax runs. Logits
    reach ~100 here, and the XLA chain rounds them to bf16 (an error of ~0.2 each), so the reference's own
    fused kernel sits ~0.18 from its XLA chain (> the 2e-2 contract). The contract is therefore held against
    the fused-kernel cast points, and the XLA deviation is bounded by the reference kernel's own."""
    announce("dense bf16 large gains (running-max path)")
    inp = workloads.dense_inputs(1, 150, 2, 64, seed=7, gain_mean=4.0, gain_std=0.5)
    got, xla, fused = run_hip(inp), oracle(inp, "xla"), oracle(inp, "fused")
    assert_bf16_parity(got, fused, "large gains vs fused profile")
    ours, theirs = stats(got, xla), stats(fused, xla)
    assert ours["max_abs"] <= 1.25 * theirs["max_abs"] and ours["cosine"] >= 1 - 1.25 * (1 - theirs["cosine"]), \
        (ours, theirs)


def test_dense_identical_branches_cancel():
    # q_diff = q and k_diff = k make both branches bit-identical: out is exactly 0 at lambda = 1.
    announce("dense bf16 identical branches")
    inp = workloads.dense_inputs(1, 333, 3, 64, seed=8)
    qkv = inp["qkv"].copy()
    hd = 3 * 64
    qkv[..., 3 * hd:4 * hd] = qkv[..., 0:hd]
    qkv[..., 4 * hd:5 * hd] = qkv[..., hd:2 * hd]
    got = run_hip(inp, lam=False, qkv_override=qkv)
    assert np.count_nonzero(got) == 0


def test_dense_lambda_linearity():
    announce("dense bf16 lambda linearity")
    inp = workloads.dense_inputs(1, 100, 2, 64, seed=9)
    qkv = torch.from_numpy(inp["qkv"]).to(DEV, torch.bfloat16)
    freq = torch.from_numpy(inp["inv_freq"]).to(DEV)
    cos, sin, m = da.tables(100, freq, torch.from_numpy(inp["valid"]).to(DEV), 64, torch.bfloat16)
    qw, kw = torch.from_numpy(inp["q_weight"]).to(DEV), torch.from_numpy(inp["k_weight"]).to(DEV)

    def run(lam):
        return da.dense_attention(qkv, qw, kw, cos, sin, m, 2, 64, 32, 1e-6,
                                  lam=torch.full((2,), lam, device=DEV)).float().cpu().numpy()
    a0, a1, ah = run(0.0), run(1.0), run(0.5)
    # out(0.5) = (out(0) + out(1)) / 2 up to the bf16 rounding of each output
    assert np.abs(ah - 0.5 * (a0 + a1)).max() <= 4e-3 * max(1.0, np.abs(a0).max())


FP32_SHAPES = [  # (B, L, H, D, half, ragged)
    (2, 1, 2, 64, 32, False), (2, 150, 2, 64, 32, False), (2, 216, 4, 64, 16, True), (1, 300, 2, 64, 0, False),
    (2, 129, 2, 128, 64, True), (1, 70, 3, 128, 32, False), (1, 100, 2, 64, 24, False), (1, 90, 2, 128, 56, True),
    (1, 100, 2, 64, 20, True), (1, 90, 2, 128, 45, False),
]


@pytest.mark.parametrize("shape", FP32_SHAPES, ids=lambda s: "B%dL%dH%dD%dh%d%s" % (*s[:5], "r" if s[5] else ""))
def test_dense_fp32_vs_oracle(shape):
    b, length, h, d, half, ragged = shape
    announce(f"dense fp32 {shape}")
    inp = workloads.dense_inputs(b, length, h, d, seed=10 + length, dtype="fp32", half=half, ragged=ragged,
                                 mask_tail=min(16, length // 4))
    got = run_hip(inp, dtype=torch.float32)
    assert_fp32_parity(got, oracle(inp, "xla", compute="fp32"), f"fp32 {shape}")


def test_dense_fp32_5s_clip():
    """The 5 s clip shape with fp32 inputs: B=1, L=216, 24 heads of 64, rotary half 32, last 16 tokens masked."""
    announce("dense fp32 B1 L216 H24 D64")
    inp = workloads.dense_inputs(1, 216, 24, 64, seed=0, dtype="fp32", half=32, mask_tail=16)
    got = run_hip(inp, dtype=torch.float32)
    assert_fp32_parity(got, oracle(inp, "xla", compute="fp32"), "fp32 5 s clip")


def test_dense_fp32_identical_branches_cancel():
    announce("dense fp32 identical branches")
    inp = workloads.dense_inputs(2, 100, 2, 64, seed=4, dtype="fp32")
    x = inp["qkv"].reshape(2, 100, 5, 2 * 64).copy()
    x[:, :, 3], x[:, :, 4] = x[:, :, 0], x[:, :, 1]
    got = run_hip(inp, dtype=torch.float32, lam=False, qkv_override=x.reshape(2, 100, -1))
    assert np.count_nonzero(got) == 0


def test_dense_120s_vs_torch_chain():
    cfg = workloads.DENSE_120S
    announce(f"dense bf16 120s {cfg}")
    inp = workloads.dense_inputs(cfg["batch"], cfg["length"], cfg["heads"], cfg["head_dim"], seed=0)
    got = run_hip(inp)
    qkv = torch.from_numpy(inp["qkv"]).to(DEV, torch.bfloat16)
    ref = xla_chain.dense_chain(qkv, torch.from_numpy(inp["q_weight"]).to(DEV),
                                torch.from_numpy(inp["k_weight"]).to(DEV), torch.from_numpy(inp["inv_freq"]).to(DEV),
                                torch.from_numpy(inp["valid"]).to(DEV), cfg["heads"], cfg["head_dim"], 1e-6,
                                lam=torch.from_numpy(inp["lam"]).to(DEV)).float().cpu().numpy()
    assert_bf16_parity(got, ref, "120s")
    # heads are independent: head 5 of the full call equals the oracle on that head alone (batch row 1)
    h = 5
    hd = cfg["heads"] * cfg["head_dim"]
    cols = np.concatenate([np.arange(s * hd + h * 64, s * hd + h * 64 + 64) for s in range(5)])
    sub = dict(inp, qkv=np.ascontiguousarray(inp["qkv"][1:2, :, cols]), heads=1, lam=inp["lam"][h:h + 1],
               valid=inp["valid"][1:2])
    assert_bf16_parity(got[1, :, h * 64:(h + 1) * 64], oracle(sub, "xla")[0], "120s head 5 vs oracle")


BALANCED = [  # (B, L, H, half): 257 to 384 workgroups of 128 queries, where the 64-query workgroups run
    (1, 1422, 24, 16), (2, 700, 24, 32), (1, 2000, 20, 8), (3, 513, 25, 24),
]


@pytest.mark.parametrize("shape", BALANCED, ids=lambda s: "B%dL%dH%dh%d" % s)
def test_dense_64_query_workgroups_vs_torch_chain(shape):
    """Grids of between one and one and a half 128-query workgroups per CU run 64-query workgroups (three per CU);
    the first shape is the reference's own 120 s DiT geometry (B=1, L=1422 = 64 memory + 1358 latent tokens,
    half=16). Checked against the torch restatement of the XLA chain, and the last head against the oracle."""
    B, L, H, half = shape
    blocks = B * H * -(-L // 128)
    assert 256 < blocks <= 384, blocks
    announce(f"dense bf16 64-query workgroups {shape} ({blocks} x 128 queries)")
    inp = workloads.dense_inputs(B, L, H, 64, seed=L + H, half=half, ragged=True)
    got = run_hip(inp)
    qkv = torch.from_numpy(inp["qkv"]).to(DEV, torch.bfloat16)
    ref = xla_chain.dense_chain(qkv, torch.from_numpy(inp["q_weight"]).to(DEV),
                                torch.from_numpy(inp["k_weight"]).to(DEV), torch.from_numpy(inp["inv_freq"]).to(DEV),
                                torch.from_numpy(inp["valid"]).to(DEV), H, 64, 1e-6,
                                lam=torch.from_numpy(inp["lam"]).to(DEV)).float().cpu().numpy()
    assert_bf16_parity(got, ref, f"{shape} vs torch chain")
    h = H - 1
    hd = H * 64
    cols = np.concatenate([np.arange(sec * hd + h * 64, sec * hd + h * 64 + 64) for sec in range(5)])
    sub = dict(inp, qkv=np.ascontiguousarray(inp["qkv"][-1:, :, cols]), heads=1, lam=inp["lam"][h:h + 1],
               valid=inp["valid"][-1:])
    assert_bf16_parity(got[-1, :, h * 64:(h + 1) * 64], oracle(sub, "xla")[0], f"{shape} last head vs oracle")


def test_dense_380s_vs_torch_chain():
    """The 380 s clip shape (B=2, L=8180, 24 heads of 64): long-sequence accumulation over 128 key tiles, checked
    against the torch restatement of the XLA chain on the GPU (inputs drawn on the device)."""
    B, L, H, D = 2, 8180, 24, 64
    announce(f"dense bf16 380s B={B} L={L} H={H}")
    gen = torch.Generator(device=DEV).manual_seed(380)
    qkv = torch.randn((B, L, 5 * H * D), device=DEV, generator=gen).to(torch.bfloat16)
    qw = 1 + 0.02 * torch.randn(D, device=DEV, generator=gen)
    kw = 1 + 0.02 * torch.randn(D, device=DEV, generator=gen)
    lam = 0.2 + 0.6 * torch.rand(H, device=DEV, generator=gen)
    valid = torch.ones((B, L), device=DEV)
    valid[0, L - 700:] = 0
    valid[1, L - 16:] = 0
    freq = torch.from_numpy(workloads.inv_freq(32)).to(DEV)
    cos, sin, mask = da.tables(L, freq, valid, D, torch.bfloat16)
    got = da.dense_attention(qkv, qw, kw, cos, sin, mask, H, D, 32, 1e-6, lam=lam).float().cpu().numpy()
    ref = xla_chain.dense_chain(qkv, qw, kw, freq, valid, H, D, 1e-6, lam=lam).float().cpu().numpy()
    assert_bf16_parity(got, ref, "380s")
    # the last head of batch row 0 (700 masked values at its end) against the oracle: its first and last 300
    # queries, each against all 8180 keys
    h, hd = H - 1, H * D
    cols = np.concatenate([np.arange(sec * hd + h * D, sec * hd + (h + 1) * D) for sec in range(5)])
    host = lambda t: t.float().cpu().numpy()  # noqa: E731
    rows = np.r_[0:300, L - 300:L]
    sub = odense.dense_xla(np.ascontiguousarray(host(qkv)[0:1, :, cols]), host(qw), host(kw), workloads.inv_freq(32),
                           host(valid)[0:1], 1, D, 1e-6, host(lam)[h:h + 1], "bf16", query_rows=rows)
    assert_bf16_parity(got[0, rows, h * D:(h + 1) * D], sub[0, rows], "380s last head vs oracle")


@pytest.mark.parametrize("half", [16, 32])
def test_rope_tables_at_the_380s_band_length_match_the_oracle(half):
    """hb_rope_tables at S = 261760 (the 380 s decoder sequence, angles up to 2.6e5 rad) against the oracle's
    tables: the same fp32 angle, cos / sin evaluated in double and rounded once, so they agree to the last bit
    except where a double result lies within a rounding error of an fp32 rounding boundary (at most 1 ulp)."""
    S = 261760
    announce(f"rope tables S={S} half={half}")
    freq = workloads.inv_freq(half)
    cos, sin = da.rope_tables(S, torch.from_numpy(freq).to(DEV))
    rc, rs = odense.rope_tables(S, freq)
    for got, ref, name in ((cos, rc[:, :half], "cos"), (sin, rs[:, :half], "sin")):
        g = got.cpu().numpy().reshape(S, half)
        assert np.isfinite(g).all()
        ulps = np.abs(g.view(np.int32).astype(np.int64) - np.ascontiguousarray(ref).view(np.int32).astype(np.int64))
        exact = (ulps == 0).mean()
        print(f"  {name}: max {ulps.max()} ulp, {exact:.7f} exact", flush=True)
        assert ulps.max() <= 1, name
        assert exact >= 0.99999, name


def test_dense_split_entry_points_match_the_fused_call():
    """hb_dense_prep + hb_dense_attend (the two stages the fused entry point runs) give bit-identical output, and
    repeated hb_dense_attend calls on one prepared workspace are stable (the benchmark times them that way)."""
    from hummingbird_amd import _lib

    announce("dense split entry points")
    B, L, H, D = 2, 333, 3, 64
    inp = workloads.dense_inputs(B, L, H, D, seed=33, half=16, ragged=True)
    qkv = torch.from_numpy(inp["qkv"]).to(DEV, torch.bfloat16)
    qw, kw = torch.from_numpy(inp["q_weight"]).to(DEV), torch.from_numpy(inp["k_weight"]).to(DEV)
    lam = torch.from_numpy(inp["lam"]).to(DEV)
    cos, sin, mask = da.tables(L, torch.from_numpy(inp["inv_freq"]).to(DEV), torch.from_numpy(inp["valid"]).to(DEV),
                               D, torch.bfloat16)
    lib = _lib.load()
    wsb = int(lib.hb_dense_workspace_size(_lib.HB_BF16, B, L, H, D))
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    full = torch.empty((B, L, H * D), dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.hb_dense_diffattn(s, qkv.data_ptr(), _lib.HB_BF16, 5 * H * D, qw.data_ptr(), kw.data_ptr(),
                                     cos.data_ptr(), sin.data_ptr(), 16, mask.data_ptr(), lam.data_ptr(),
                                     full.data_ptr(), B, L, H, D, 1e-6, ws.data_ptr(), wsb), "diffattn")
    ws.fill_(0xFF)  # the stages must not depend on what the workspace held
    _lib.check(lib.hb_dense_prep(s, qkv.data_ptr(), _lib.HB_BF16, 5 * H * D, qw.data_ptr(), kw.data_ptr(),
                                 cos.data_ptr(), sin.data_ptr(), 16, mask.data_ptr(), B, L, H, D, 1e-6, ws.data_ptr(),
                                 wsb), "prep")
    outs = []
    for _ in range(3):
        o = torch.empty_like(full)
        _lib.check(lib.hb_dense_attend(s, qkv.data_ptr(), _lib.HB_BF16, 5 * H * D, qw.data_ptr(), kw.data_ptr(),
                                       cos.data_ptr(), sin.data_ptr(), 16, lam.data_ptr(), o.data_ptr(), B, L, H, D,
                                       1e-6, ws.data_ptr(), wsb), "attend")
        outs.append(o)
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), full.view(torch.int16))
    assert_bf16_parity(full.float().cpu().numpy(), oracle(inp, "xla"), "split entry points vs oracle")


def test_dense_errors_are_value_errors():
    announce("dense argument errors")
    qkv = torch.zeros((1, 8, 5 * 2 * 96), device=DEV, dtype=torch.bfloat16)
    w = torch.ones(96, device=DEV)
    with pytest.raises(ValueError):
        da.dense_attention(qkv, w, w, None, None, None, 2, 96, 0, 1e-6)
    qkv = torch.zeros((1, 8, 5 * 2 * 64), device=DEV, dtype=torch.bfloat16)
    w = torch.ones(64, device=DEV)
    with pytest.raises(ValueError):
        da.dense_attention(qkv, w, w, None, None, None, 2, 64, 40, 1e-6)
    with pytest.raises(TypeError):
        da.dense_attention(qkv.double(), w, w, None, None, None, 2, 64, 0, 1e-6)
