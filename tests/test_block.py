"""The SAME-L decoder block on the CPU (no GPU here):

* the oracle's GLU against torch's SiLU and sine in float64 (which half is the value, which the gate), and the
  whole block against independent torch compositions where one branch is switched off (zero output weights);
* the torch restatement that `attention="xla"` runs against the oracle;
* the C ABI's host-side checks of hb_dyt and hb_glu (no kernel is launched).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from hummingbird_amd import _lib, same_l, workloads
from hummingbird_amd.config import SameConfig
from oracle import band as oband
from oracle import block as oblock
from tests.block_util import block_params, rounded, to_torch
from tests.util import assert_bf16_parity, assert_fp32_parity

RNG = np.random.default_rng(31)


@pytest.mark.parametrize("sine", [False, True])
def test_glu_matches_torch_float64(sine):
    proj = RNG.standard_normal((7, 2 * 24)).astype(np.float32) * 2
    t = torch.from_numpy(proj).double()
    value, gate = t[:, :24], t[:, 24:]
    ref = value * (torch.sin(math.pi * gate) if sine else F.silu(gate))
    np.testing.assert_allclose(oblock.glu(proj, sine, "fp32"), ref.numpy(), atol=2e-6, rtol=1e-5)


def test_glu_bf16_cast_points():
    # gate 1: pi is held in bf16 (3.140625), so sin(pi * gate) is sin(3.140625), not ~0
    proj = np.array([[1.0, 1.0]], np.float32)
    expect = oblock.cast(np.array([math.sin(3.140625)]), "bf16")
    assert np.array_equal(oblock.glu(proj, True, "bf16")[0], expect)
    # gate 0 gives 0 for both activations; every bf16 output is a bf16 value
    proj = RNG.standard_normal((5, 16)).astype(np.float32)
    proj[:, 8:] = 0.0
    for sine in (False, True):
        assert np.count_nonzero(oblock.glu(proj, sine, "bf16")) == 0
    out = oblock.glu(RNG.standard_normal((5, 16)).astype(np.float32), False, "bf16")
    assert np.array_equal(out, oblock.cast(out, "bf16"))


def test_block_with_both_branches_off_is_identity():
    p = block_params(128, 2, 384, seed=1, zero_attn=True, zero_ff=True)
    x = RNG.standard_normal((1, 50, 128)).astype(np.float32)
    for compute in ("fp32", "bf16"):
        assert np.array_equal(oblock.block_xla(x, p, 2, 64, 17, False, None, compute), oblock.cast(x, compute))


@pytest.mark.parametrize("sine", [False, True])
def test_block_feed_forward_branch_matches_torch(sine):
    """Attention off (to_out = 0): the block is x + FF(DyT(x)), composed here from torch's tanh, matmuls, SiLU and
    sine in float64."""
    p = block_params(128, 2, 384, seed=2, zero_attn=True)
    x = RNG.standard_normal((2, 30, 128)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    n, ff = p["ff_norm"], p["ff"]
    h = t(x)
    y = t(n["gamma"]) * torch.tanh(float(n["alpha"]) * h) + t(n["beta"])
    proj = y @ t(ff["glu_proj"]["weight"]).T + t(ff["glu_proj"]["bias"])
    value, gate = proj[..., :384], proj[..., 384:]
    act = torch.sin(math.pi * gate) if sine else F.silu(gate)
    ref = h + (value * act) @ t(ff["proj_out"]["weight"]).T + t(ff["proj_out"]["bias"])
    np.testing.assert_allclose(oblock.block_xla(x, p, 2, 64, 17, sine, None, "fp32"), ref.numpy(), atol=2e-5,
                               rtol=1e-4)


def test_block_attention_branch_matches_torch_band_sdpa():
    """FF off (proj_out = 0): the block is x + to_out(band attention(to_qkv(DyT(x)))), with the attention from
    torch's SDPA under an explicit band mask (the band oracle's own pin) in float64."""
    p = block_params(128, 2, 384, seed=3, zero_ff=True)
    x = RNG.standard_normal((1, 80, 128)).astype(np.float32)
    w, H = 17, 2
    a = p["self_attn"]
    y = oband.dyt(x, p["pre_norm"]["alpha"], p["pre_norm"]["gamma"], p["pre_norm"]["beta"]).astype(np.float64)
    qkv = y @ a["to_qkv"]["weight"].astype(np.float64).T
    q, k, v, qd, kd = oband.prepare(qkv.astype(np.float32), a["q_norm"], a["k_norm"], p["rope_inv_freq"], H, 64,
                                    "fp32")
    pos = np.arange(80)
    mask = torch.from_numpy(np.abs(pos[:, None] - pos[None, :]) <= w)
    tt = lambda z: torch.from_numpy(np.ascontiguousarray(z)).double()  # noqa: E731
    att = (F.scaled_dot_product_attention(tt(q), tt(k), tt(v), attn_mask=mask)
           - F.scaled_dot_product_attention(tt(qd), tt(kd), tt(v), attn_mask=mask))
    out = att.permute(0, 2, 1, 3).reshape(1, 80, 128).numpy() @ a["to_out"]["weight"].astype(np.float64).T
    ref = x.astype(np.float64) + out + p["ff"]["proj_out"]["bias"]
    np.testing.assert_allclose(oblock.block_xla(x, p, H, 64, w, False, None, "fp32"), ref, atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("compute", ["fp32", "bf16"])
def test_torch_chain_block_matches_oracle(compute):
    dim, heads, ff = 128, 2, 384
    cfg = SameConfig(channels=64, c_mults=(2,), stride=16, transformer_depth=4, sinusoidal_blocks=2,
                     attention="xla")
    dt = torch.float32 if compute == "fp32" else torch.bfloat16
    for index in (0, 3):  # SiLU block, sine block
        p = block_params(dim, heads, ff, seed=4 + index)
        x = RNG.standard_normal((1, 70, dim)).astype(np.float32)
        tp = to_torch(p, "cpu", dt)
        got = same_l.block(torch.from_numpy(x).to(dt), tp, index, cfg).float().numpy()
        ref = oblock.block_xla(torch.from_numpy(x).to(dt).float().numpy(), rounded(p, compute), heads, 64,
                               cfg.sub_chunk_size, cfg.sinusoidal(index), None, compute)
        scale = max(1.0, float(np.abs(ref).max()))  # the residual stream's magnitude (one bf16 step at 4 is 0.03)
        (assert_fp32_parity if compute == "fp32" else assert_bf16_parity)(got / scale, ref / scale,
                                                                          f"block {index} {compute}")


def test_blocks_chain_matches_oracle_chain():
    """same_l.blocks (attention="xla", fp32) over four blocks against the oracle's block applied four times: the
    loop runs the blocks in order with their own index (the sine gate from block index 3 on)."""
    dim, heads, ff = 128, 2, 384
    cfg = SameConfig(channels=64, c_mults=(2,), stride=16, transformer_depth=4, sinusoidal_blocks=2,
                     attention="xla")
    ps = [block_params(dim, heads, ff, seed=9 + i) for i in range(4)]
    x = RNG.standard_normal((1, 60, dim)).astype(np.float32)
    got = same_l.blocks(torch.from_numpy(x), [to_torch(p) for p in ps], cfg).numpy()
    ref = x
    for i, p in enumerate(ps):
        ref = oblock.block_xla(ref, p, heads, 64, cfg.sub_chunk_size, cfg.sinusoidal(i), None, "fp32")
    scale = max(1.0, float(np.abs(ref).max()))
    assert_fp32_parity(got / scale, ref / scale, "4 blocks fp32")


# ---- the C ABI's host-side checks ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libhummingbird_amd.so is not built: run `python -m hummingbird_amd._build`")
    return _lib.load()


def test_elementwise_errors_before_any_launch(lib):
    x, o, p = 0x10000, 0x20000, 0x30000  # fake, 16-byte aligned, never dereferenced
    dyt = lambda xp=x, dt=0, xs=512, os_=512, n=10, c=512, par=p: lib.hb_dyt(None, xp, dt, xs, par, o, os_, n, c)  # noqa: E731
    assert dyt(dt=3) == 3                     # dtype
    assert dyt(c=500) == 2                    # bf16 channels must be a multiple of 8
    assert dyt(dt=1, c=502, xs=504, os_=504) == 2   # fp32: multiple of 4
    assert dyt(xs=500) == 7 and dyt(os_=516 - 12) == 7  # stride below C / not a multiple of 8
    assert dyt(xp=x + 8) == 7                 # misaligned input
    assert dyt(xp=None) == 1 and dyt(par=None) == 1
    assert dyt(n=0) == 2
    glu = lambda ps=1024, f=512, pp=x: lib.hb_glu(None, pp, 0, ps, None, 0, o, f, 10, f)  # noqa: E731
    assert glu(ps=1016) == 7                  # proj rows hold 2F
    assert glu(pp=None) == 1
    assert "glu" in lib.hb_last_error().decode()
