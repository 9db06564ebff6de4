"""GPU parity of the SAME-L block's elementwise kernels (hb_dyt, hb_glu) and of the block mirror with
`attention="hip"`.

hb_dyt and hb_glu run against the oracle; hb_residual_dyt against the torch additions it fuses (bit-identical:
the same roundings) followed by hb_dyt (bit-identical: the same DyT code). fp32 within 1e-5 relative; bf16 within one bf16 step of the oracle's
value on every element (the kernels' tanh, exp and sine are not bit-identical to NumPy's, so a value that lands
next to a rounding boundary may round the other way), plus for the DyT a few fp32 units of its operands' scale
(where gamma * tanh(alpha x) nearly cancels beta, both evaluations carry that absolute error in a tiny result),
and equal on all but a small fraction. The block with
`attention="hip"` runs against `attention="xla"` on the GPU and against the oracle, with the attention contract
(bf16: max-abs <= 2e-2 and cosine >= 0.9999; fp32: 1e-5 relative) applied to the output divided by its largest
magnitude: the block's output is the residual stream, which carries the block input (values to about 4.5 here),
and one bf16 step at that magnitude is 0.03.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hummingbird_amd import elementwise, same_l
from hummingbird_amd.config import SameConfig
from oracle import block as oblock
from tests.block_util import block_params, rounded, to_torch
from tests.util import assert_bf16_parity, assert_fp32_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"
RNG = np.random.default_rng(41)


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def dev(a, dtype=torch.float32) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV, dtype)


def assert_within_one_bf16_step(got: np.ndarray, ref: np.ndarray, what: str, atol: float = 0.0,
                                max_frac: float = 0.01) -> None:
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    step = np.maximum(np.abs(ref), 1e-30) * 2.0 ** -7 + atol  # the spacing of bf16 values around ref (upper bound)
    diff = np.abs(got - ref)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert (diff <= step).all(), f"{what}: {int((diff > step).sum())} elements more than one bf16 step away"
    frac = float((diff > 0).mean())
    assert frac <= max_frac, f"{what}: {frac:.3%} of the elements differ (allowed {max_frac:.1%})"


DYT_SHAPES = [(1, 8), (100, 512), (3000, 768), (37, 1536)]


@pytest.mark.parametrize("shape", DYT_SHAPES, ids=lambda s: "N%dC%d" % s)
@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_dyt_vs_oracle(shape, dtype):
    n, c = shape
    announce(f"dyt {dtype} {shape}")
    x = (RNG.standard_normal((n, c)) * 3).astype(np.float32)
    norm = {"alpha": np.float32(0.7), "gamma": (1 + 0.3 * RNG.standard_normal(c)).astype(np.float32),
            "beta": (0.1 * RNG.standard_normal(c)).astype(np.float32)}
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    xt = dev(x, tdt)
    got = elementwise.dyt(xt, {k: torch.as_tensor(v).to(DEV) for k, v in norm.items()}).float().cpu().numpy()
    ref = oblock.dyt_cast(xt.float().cpu().numpy(), norm, dtype)
    if dtype == "fp32":
        assert_fp32_parity(got, ref, f"dyt {shape}")
    else:
        scale = float(np.max(np.abs(norm["gamma"]) + np.abs(norm["beta"])))
        assert_within_one_bf16_step(got, ref, f"dyt {shape}", atol=scale * 2.0 ** -21)


GLU_SHAPES = [(1, 8), (200, 1536), (1000, 4608)]


@pytest.mark.parametrize("shape", GLU_SHAPES, ids=lambda s: "N%dF%d" % s)
@pytest.mark.parametrize("sine", [False, True], ids=["silu", "sine"])
@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_glu_vs_oracle(shape, sine, dtype):
    n, f = shape
    announce(f"glu {dtype} sine={sine} {shape}")
    proj = (RNG.standard_normal((n, 2 * f)) * 2).astype(np.float32)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    pt = dev(proj, tdt)
    got = elementwise.glu(pt, sine).float().cpu().numpy()
    ref = oblock.glu(pt.float().cpu().numpy(), sine, dtype)
    if dtype == "fp32":
        assert_fp32_parity(got, ref, f"glu {shape}")
    else:
        assert_within_one_bf16_step(got, ref, f"glu {shape}")


@pytest.mark.parametrize("sine", [False, True], ids=["silu", "sine"])
@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_glu_with_bias_vs_oracle(sine, dtype):
    """The glu_proj bias added inside the kernel equals the bias added to the matmul output in the compute dtype
    first (same_l._linear), then the GLU."""
    announce(f"glu with bias {dtype} sine={sine}")
    n, f = 300, 1536
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    pt = dev((RNG.standard_normal((n, 2 * f)) * 2).astype(np.float32), tdt)
    bias = dev(0.5 * RNG.standard_normal(2 * f), tdt)  # a parameter of the compute dtype
    got = elementwise.glu(pt, sine, bias=bias).float().cpu().numpy()
    summed = oblock.cast(pt.float().cpu().numpy().astype(np.float64) + bias.float().cpu().numpy(), dtype)
    ref = oblock.glu(summed, sine, dtype)
    if dtype == "fp32":
        assert_fp32_parity(got, ref, "glu with bias")
    else:
        assert_within_one_bf16_step(got, ref, "glu with bias")


@pytest.mark.parametrize("scale", [40.0, 400.0, 30000.0], ids=["gate40", "gate400", "gate30000"])
def test_glu_sine_large_gates_vs_oracle(scale):
    """bf16 sine gates far outside the usual range: pi * gate reaches ~500 rad (scale 40) and ~5000 rad (scale
    400); the kernel reduces the argument by 2 pi before the hardware sine."""
    announce(f"glu sine large gates x{scale}")
    proj = (RNG.standard_normal((256, 2 * 512)) * np.r_[np.ones(512), np.full(512, scale)]).astype(np.float32)
    pt = dev(proj, torch.bfloat16)
    got = elementwise.glu(pt, True).float().cpu().numpy()
    ref = oblock.glu(pt.float().cpu().numpy(), True, "bf16")
    assert_within_one_bf16_step(got, ref, f"glu sine x{scale}", max_frac=0.02)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_glu_sine_every_gate_vs_oracle(dtype):
    """Every finite gate value of the dtype (value 1, so the output is the rounded activation) through the sine GLU
    against the oracle's float64 sine: the kernel's argument reductions (Cody-Waite and the hardware sine for bf16,
    with the exact table reduction once |pi g| > 2^16; the three-term split and the polynomial for half) on every
    input they can receive. Gates whose product pi g overflows give NaN on both sides."""
    announce(f"glu sine every {dtype} gate")
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    gates = bits.view(tdt).float()
    gates = gates[torch.isfinite(gates)]
    f = 256
    rows = -(-gates.numel() // f)
    g = torch.zeros(rows * f)
    g[: gates.numel()] = gates
    proj = torch.cat([torch.ones(rows, f), g.reshape(rows, f)], dim=1).to(DEV, tdt)
    got = elementwise.glu(proj, True).float().cpu().numpy()
    with np.errstate(invalid="ignore"):
        ref = oblock.glu(proj.float().cpu().numpy(), True, dtype)
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    assert (nan_g == nan_r).all(), f"NaN at {int((nan_g != nan_r).sum())} positions that differ"
    keep = ~nan_r
    got, ref = got[keep], ref[keep]
    bits_ = 8 if dtype == "bf16" else 11
    step = np.ldexp(1.0, np.frexp(np.maximum(np.abs(ref), 2.0 ** -126))[1] - bits_)
    diff = np.abs(got.astype(np.float64) - ref)
    assert (diff <= step).all(), f"{int((diff > step).sum())} activations more than one step from the oracle"
    assert (diff == 0).mean() >= 0.999, f"only {(diff == 0).mean():.5f} of the activations equal the oracle's"


def test_elementwise_padded_rows():
    """Column slices of wider tensors (row stride > width) give the same values as contiguous inputs."""
    announce("dyt / glu padded rows")
    x = dev(RNG.standard_normal((64, 520)), torch.bfloat16)
    norm = {"alpha": torch.tensor(0.5, device=DEV), "gamma": torch.ones(512, device=DEV),
            "beta": torch.zeros(512, device=DEV)}
    assert torch.equal(elementwise.dyt(x[:, :512], norm), elementwise.dyt(x[:, :512].contiguous(), norm))
    p = dev(RNG.standard_normal((2, 32, 3 * 256)), torch.bfloat16)[..., : 2 * 256]
    assert torch.equal(elementwise.glu(p, False), elementwise.glu(p.contiguous(), False))


CFG = SameConfig(channels=64, c_mults=(2,), stride=16, transformer_depth=4, sinusoidal_blocks=2)


@pytest.mark.parametrize("index", [0, 3], ids=["silu_block", "sine_block"])
@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_block_hip_vs_xla_and_oracle(index, dtype):
    """A decoder block (dim 128 = 2 heads of 64, ff 384, half-width 17) with attention="hip" against "xla" on the
    GPU and against the oracle."""
    announce(f"same-l block {dtype} index {index}")
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    p = block_params(128, 2, 384, seed=50 + index)
    x = RNG.standard_normal((1, 900, 128)).astype(np.float32)
    xt = dev(x, tdt)
    outs = {}
    for mode in ("hip", "xla"):
        cfg = SameConfig(channels=64, c_mults=(2,), stride=16, transformer_depth=4, sinusoidal_blocks=2,
                         attention=mode)
        outs[mode] = same_l.block(xt, to_torch(p, DEV, tdt), index, cfg).float().cpu().numpy()
    check = assert_bf16_parity if dtype == "bf16" else assert_fp32_parity
    scale = max(1.0, float(np.abs(outs["xla"]).max()))
    check(outs["hip"] / scale, outs["xla"] / scale, f"block {index} hip vs xla (/{scale:.3g})")
    ref = oblock.block_xla(xt.float().cpu().numpy(), rounded(p, dtype), 2, 64, CFG.sub_chunk_size,
                           CFG.sinusoidal(index), None, dtype)
    check(outs["hip"] / scale, ref / scale, f"block {index} hip vs oracle (/{scale:.3g})")


@pytest.mark.parametrize("with_bias", [False, True], ids=["no_bias", "bias"])
@pytest.mark.parametrize("with_dyt", [False, True], ids=["no_dyt", "dyt"])
@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
def test_residual_dyt_equals_the_ops_it_fuses(dtype, with_dyt, with_bias):
    """out_h = h + (x + bias) equals torch's additions in the compute dtype (each sum rounded once, as the reference
    holds them) bit for bit, and out_y equals hb_dyt of out_h bit for bit, on a row slice of a wider tensor."""
    announce(f"residual_dyt {dtype} dyt={with_dyt} bias={with_bias}")
    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dtype]
    c = 512
    h = dev(2 * RNG.standard_normal((3, 333, c)), tdt)
    x = dev(RNG.standard_normal((3, 333, c + 64)), tdt)[..., :c]
    bias = dev(0.1 * RNG.standard_normal(c), tdt) if with_bias else None
    norm = ({"alpha": torch.tensor(0.7, device=DEV), "gamma": dev(1 + 0.1 * RNG.standard_normal(c)),
             "beta": dev(0.1 * RNG.standard_normal(c))} if with_dyt else None)
    out_h, out_y = elementwise.residual_dyt(h, x, bias=bias, norm=norm)
    ref_h = h + ((x + bias) if with_bias else x)
    assert ref_h.dtype == tdt and torch.equal(out_h, ref_h)
    if with_dyt:
        assert torch.equal(out_y, elementwise.dyt(ref_h, norm))
    else:
        assert out_y is None


def test_residual_dyt_in_place():
    """The C ABI allows out_h to be h itself: the sum lands where h was, and out_y is unchanged by the aliasing."""
    announce("residual_dyt in place")
    from hummingbird_amd import _lib
    c = 256
    h = dev(RNG.standard_normal((100, c)), torch.bfloat16)
    x = dev(RNG.standard_normal((100, c)), torch.bfloat16)
    norm = {"alpha": torch.tensor(0.5, device=DEV), "gamma": dev(np.ones(c)), "beta": dev(np.zeros(c))}
    ref_h, ref_y = elementwise.residual_dyt(h, x, norm=norm)
    params = elementwise.pack_dyt(norm, c, h.device)
    y = torch.empty_like(h)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.load().hb_residual_dyt(stream, h.data_ptr(), _lib.HB_BF16, c, x.data_ptr(), c, 0, params.data_ptr(),
                                           h.data_ptr(), y.data_ptr(), c, 100, c), "residual_dyt")
    torch.cuda.synchronize()
    assert torch.equal(h, ref_h) and torch.equal(y, ref_y)


def test_row_ops_on_interleaved_column_slices():
    """Inputs and outputs as interleaved column slices of one wide buffer (same row stride, no element shared) pass
    the C ABI's overlap check, and hb_residual_dyt, hb_dyt, hb_rms_modulate and hb_residual_rms write exactly what
    they write into separate tensors, leaving the other columns untouched."""
    announce("row ops on interleaved column slices")
    from hummingbird_amd import _lib
    lib, stream = _lib.load(), torch.cuda.current_stream().cuda_stream
    n, c = 300, 256
    buf = dev(RNG.standard_normal((n, 6 * c)), torch.bfloat16)
    keep = buf.clone()
    h, x, oh, oy, od, orm = (buf[:, i * c:(i + 1) * c] for i in range(6))
    norm = {"alpha": torch.tensor(0.6, device=DEV), "gamma": dev(1 + 0.1 * RNG.standard_normal(c)),
            "beta": dev(0.1 * RNG.standard_normal(c))}
    ref_h, ref_y = elementwise.residual_dyt(h.contiguous(), x.contiguous(), norm=norm)
    ref_d = elementwise.dyt(h.contiguous(), norm)
    w = dev(1 + 0.1 * RNG.standard_normal(c))
    ref_r = elementwise.rms_modulate(x.contiguous().unsqueeze(0), w, 1e-6)[0]
    params = elementwise.pack_dyt(norm, c, h.device)
    rs = 6 * c
    _lib.check(lib.hb_residual_dyt(stream, h.data_ptr(), _lib.HB_BF16, rs, x.data_ptr(), rs, 0, params.data_ptr(),
                                   oh.data_ptr(), oy.data_ptr(), rs, n, c), "residual_dyt")
    _lib.check(lib.hb_dyt(stream, h.data_ptr(), _lib.HB_BF16, rs, params.data_ptr(), od.data_ptr(), rs, n, c), "dyt")
    _lib.check(lib.hb_rms_modulate(stream, x.data_ptr(), _lib.HB_BF16, rs, w.data_ptr(), 1e-6, None, None, c, n,
                                   orm.data_ptr(), rs, n, c), "rms_modulate")
    torch.cuda.synchronize()
    assert torch.equal(oh, ref_h) and torch.equal(oy, ref_y) and torch.equal(od, ref_d) and torch.equal(orm, ref_r)
    assert torch.equal(buf[:, :2 * c], keep[:, :2 * c])  # the inputs
    # hb_residual_rms: h and x in columns 0 and 1, the two outputs in columns 2 and 3 of a fresh copy
    buf2 = keep.clone()
    h2, x2, oh2, oy2 = (buf2[:, i * c:(i + 1) * c] for i in range(4))
    ref_h2, ref_y2 = elementwise.residual_rms(h2.contiguous().unsqueeze(0), x2.contiguous().unsqueeze(0), w, 1e-6)
    _lib.check(lib.hb_residual_rms(stream, h2.data_ptr(), _lib.HB_BF16, rs, x2.data_ptr(), rs, None, None, c, None,
                                   0, w.data_ptr(), 1e-6, None, None, c, n, oh2.data_ptr(), oy2.data_ptr(), rs, n, c),
               "residual_rms")
    torch.cuda.synchronize()
    assert torch.equal(oh2, ref_h2[0]) and torch.equal(oy2, ref_y2[0])
    assert torch.equal(buf2[:, :2 * c], keep[:, :2 * c]) and torch.equal(buf2[:, 4 * c:], keep[:, 4 * c:])


def test_block_graph_replays_equal_eager():
    """The whole SAME-L block with attention="hip" (hb_dyt, the band kernel, hb_glu, hb_residual_dyt and the torch
    GEMMs) captured as one HIP graph: three replays with new inputs, eager work in between, each bit-identical to
    the eager block on the same input."""
    announce("same-l block graph replays")
    cfg = SameConfig(channels=64, c_mults=(2,), stride=16, transformer_depth=4, sinusoidal_blocks=2, attention="hip")
    p = to_torch(block_params(128, 2, 384, seed=60), DEV, torch.bfloat16)
    static_x = dev(RNG.standard_normal((1, 700, 128)), torch.bfloat16)
    same_l.block(static_x, p, 3, cfg)  # warm-up: table caches, library load
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        same_l.block(static_x, p, 3, cfg)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = same_l.block(static_x, p, 3, cfg)
    for replay in range(3):
        x = dev(RNG.standard_normal((1, 700, 128)), torch.bfloat16)
        static_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        ref = same_l.block(x, p, 3, cfg)
        torch.cuda.synchronize()
        assert torch.equal(static_out, ref), f"replay {replay}"
        _ = (torch.randn(1 << 16, device=DEV) * 2).sum().item()  # unrelated eager work between replays


def test_blocks_chain_equals_block_by_block():
    """same_l.blocks with attention="hip" (each block's last residual pass also making the next block's pre_norm DyT)
    gives the block-by-block loop's values bit for bit, over four blocks (SiLU and sine gates), and matches the
    "xla" chain at the contract on the output divided by its largest magnitude."""
    announce("same-l blocks chain")
    cfg_hip = SameConfig(channels=64, c_mults=(2,), stride=16, transformer_depth=4, sinusoidal_blocks=2,
                         attention="hip")
    cfg_xla = SameConfig(channels=64, c_mults=(2,), stride=16, transformer_depth=4, sinusoidal_blocks=2,
                         attention="xla")
    ps = [to_torch(block_params(128, 2, 384, seed=70 + i), DEV, torch.bfloat16) for i in range(4)]
    x = dev(RNG.standard_normal((1, 600, 128)), torch.bfloat16)
    chained = same_l.blocks(x, ps, cfg_hip)
    h = x
    for i, p in enumerate(ps):
        h = same_l.block(h, p, i, cfg_hip)
    assert torch.equal(chained, h)
    ref = same_l.blocks(x, ps, cfg_xla).float().cpu().numpy()
    got = chained.float().cpu().numpy()
    scale = max(1.0, float(np.abs(ref).max()))
    assert_bf16_parity(got / scale, ref / scale, f"4 blocks hip vs xla (/{scale:.3g})")


def test_blocks_chain_shares_one_band_workspace_fp32(monkeypatch):
    """In fp32 the band kernel prepares every key once into a workspace; same_l.blocks allocates one for the whole
    loop and hands the same buffer to every block's band call. The values are the block-by-block loop's (whose
    calls each allocate their own) bit for bit."""
    announce("same-l blocks fp32 shared workspace")
    cfg = SameConfig(channels=64, c_mults=(2,), stride=16, transformer_depth=3, sinusoidal_blocks=1, attention="hip")
    ps = [to_torch(block_params(128, 2, 384, seed=90 + i), DEV, torch.float32) for i in range(3)]
    x = dev(RNG.standard_normal((1, 500, 128)), torch.float32)
    seen = []
    orig = same_l.band_attention.band_attention

    def spy(*a, **kw):
        seen.append(kw.get("workspace"))
        return orig(*a, **kw)

    monkeypatch.setattr(same_l.band_attention, "band_attention", spy)
    chained = same_l.blocks(x, ps, cfg)
    monkeypatch.undo()
    assert len(seen) == 3 and seen[0] is not None and all(w is seen[0] for w in seen)
    h = x
    for i, p in enumerate(ps):
        h = same_l.block(h, p, i, cfg)
    assert torch.equal(chained, h)
