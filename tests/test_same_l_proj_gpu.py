"""The SAME-L block's projections with the work next to them in their epilogues, on the GPU.

* hb_proj_glu (glu_proj + GLU) against hb_proj's product of the whole [value | gate] weight followed by hb_glu:
  bit for bit (both GEMMs accumulate in fp32 over K in the same order and round once; the epilogue then repeats
  hb_glu's arithmetic), in bf16 and half, SiLU and sine, with and without bias, on ragged and full decoder shapes;
  and against the oracle's linear + GLU at the bf16 contract;
* hb_proj_residual (to_out / proj_out + bias + residual + next DyT) against hb_proj followed by hb_residual_dyt, bit
  for bit, with and without bias and DyT, and in place (out_h = h);
* same_l.blocks with projections="hip" against projections="torch" (hipBLASLt) at the bf16 contract, against the
  oracle block, and falling back to the torch projections where the fused GEMMs do not take the geometry.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hummingbird_amd import _lib, elementwise, projection, same_l
from hummingbird_amd.config import SameConfig
from hummingbird_amd.dense_attention import dtype_code
from oracle import block as oblock
from oracle.bf16 import cast
from tests.block_util import block_params, rounded, to_torch
from tests.util import assert_bf16_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def rand(shape, std, gen, dtype):
    return (torch.randn(shape, device=DEV, generator=gen) * std).to(dtype)


def same_bits(a: torch.Tensor, b: torch.Tensor, what: str) -> None:
    assert a.shape == b.shape and a.dtype == b.dtype, what
    ai, bi = a.view(torch.int16), b.view(torch.int16)
    diff = int((ai != bi).sum())
    assert diff == 0, f"{what}: {diff} of {a.numel()} elements differ"


DTYPES = [torch.bfloat16, torch.float16]


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16"])
@pytest.mark.parametrize("sine", [False, True], ids=["silu", "sine"])
@pytest.mark.parametrize("with_bias", [False, True], ids=["no_bias", "bias"])
@pytest.mark.parametrize("n,k,f", [(1, 64, 128), (300, 128, 256), (1000, 512, 384)], ids=lambda v: str(v))
def test_glu_linear_equals_linear_then_glu(n, k, f, with_bias, sine, dtype):
    announce(f"proj_glu N={n} K={k} F={f} bias={with_bias} sine={sine} {dtype}")
    gen = torch.Generator(device=DEV).manual_seed(n + 7 * k + f)
    x, w = rand((n, k), 1.0, gen, dtype), rand((2 * f, k), k ** -0.5, gen, dtype)
    bias = rand((2 * f,), 0.05, gen, dtype) if with_bias else None
    got = projection.glu_linear(x, w, bias, sine)
    ref = elementwise.glu(projection.linear(x, w), sine, bias=bias)
    assert not torch.isnan(got.float()).any()
    same_bits(got, ref, "glu_linear vs linear -> glu")


@pytest.mark.parametrize("sine", [False, True], ids=["silu", "sine"])
def test_glu_linear_at_the_decoder_shape(sine):
    """The SAME-L decoder's glu_proj (23086 frames, 1536 -> 2 x 4608) with its bias, against the unfused kernels."""
    announce(f"proj_glu decoder shape sine={sine}")
    gen = torch.Generator(device=DEV).manual_seed(5)
    x, w = rand((23086, 1536), 1.0, gen, torch.bfloat16), rand((9216, 1536), 1536 ** -0.5, gen, torch.bfloat16)
    bias = rand((9216,), 0.02, gen, torch.bfloat16)
    same_bits(projection.glu_linear(x, w, bias, sine), elementwise.glu(projection.linear(x, w), sine, bias=bias),
              "decoder glu_proj")


@pytest.mark.parametrize("sine", [False, True], ids=["silu", "sine"])
def test_glu_linear_vs_oracle(sine):
    announce(f"proj_glu vs oracle sine={sine}")
    gen = torch.Generator(device=DEV).manual_seed(11)
    n, k, f = 333, 256, 256
    x, w = rand((n, k), 1.0, gen, torch.bfloat16), rand((2 * f, k), k ** -0.5, gen, torch.bfloat16)
    bias = rand((2 * f,), 0.05, gen, torch.bfloat16)
    got = projection.glu_linear(x, w, bias, sine).float().cpu().numpy()
    host = lambda t: t.float().cpu().numpy()  # noqa: E731
    ref = oblock.glu(oblock.linear(host(x), {"weight": host(w), "bias": host(bias)}, "bf16"), sine, "bf16")
    assert_bf16_parity(got, ref, "glu_linear vs oracle")


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16"])
@pytest.mark.parametrize("with_dyt", [False, True], ids=["no_dyt", "dyt"])
@pytest.mark.parametrize("with_bias", [False, True], ids=["no_bias", "bias"])
@pytest.mark.parametrize("n,k,f", [(1, 64, 256), (700, 192, 512)], ids=lambda v: str(v))
def test_residual_linear_equals_linear_then_residual_dyt(n, k, f, with_bias, with_dyt, dtype):
    check_residual(n, k, f, with_bias, with_dyt, dtype)


def test_residual_linear_at_the_decoder_shape():
    """The SAME-L decoder's proj_out (23086 frames, 4608 -> 1536) with its bias, the residual and the next block's
    pre_norm DyT, against the unfused kernels."""
    check_residual(23086, 4608, 1536, True, True, torch.bfloat16)


def check_residual(n, k, f, with_bias, with_dyt, dtype):
    announce(f"proj_residual N={n} K={k} F={f} bias={with_bias} dyt={with_dyt} {dtype}")
    gen = torch.Generator(device=DEV).manual_seed(n + k + 3 * f)
    x, w = rand((n, k), 1.0, gen, dtype), rand((f, k), k ** -0.5, gen, dtype)
    h = rand((n, f), 1.5, gen, dtype)
    bias = rand((f,), 0.05, gen, dtype) if with_bias else None
    norm = None
    if with_dyt:
        norm = {"alpha": torch.tensor(0.5, device=DEV),
                "gamma": 1 + 0.02 * torch.randn(f, device=DEV, generator=gen),
                "beta": 0.02 * torch.randn(f, device=DEV, generator=gen)}
    got_h, got_y = projection.residual_linear(x, w, bias, h, norm)
    ref_h, ref_y = elementwise.residual_dyt(h, projection.linear(x, w), bias=bias, norm=norm)
    same_bits(got_h, ref_h, "out_h")
    if with_dyt:
        same_bits(got_y, ref_y, "out_y")
    else:
        assert got_y is None


def test_residual_linear_in_place():
    """out_h = h itself (the C ABI allows it: each residual element is read and written by one lane)."""
    announce("proj_residual in place")
    gen = torch.Generator(device=DEV).manual_seed(21)
    n, k, f = 513, 256, 512
    x, w = rand((n, k), 1.0, gen, torch.bfloat16), rand((f, k), k ** -0.5, gen, torch.bfloat16)
    h = rand((n, f), 1.0, gen, torch.bfloat16)
    bias = rand((f,), 0.05, gen, torch.bfloat16)
    ref_h, _ = projection.residual_linear(x, w, bias, h)
    b32 = bias.float()
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.hb_proj_residual(stream, x.data_ptr(), dtype_code(x.dtype), k, w.data_ptr(), k, b32.data_ptr(),
                                    h.data_ptr(), f, 0, h.data_ptr(), 0, f, n, k, f), "in place")
    same_bits(h, ref_h, "in place")


def _cfg(attention: str) -> SameConfig:
    # 256 = 4 heads of 64, half-width 17 (the reference decoder's window), two sinusoidal blocks of four
    return SameConfig(channels=128, c_mults=(2,), stride=16, transformer_depth=4, sinusoidal_blocks=2,
                      attention=attention)


def test_blocks_fused_projections_vs_hipblaslt_and_oracle():
    """Four decoder blocks (dim 256 = 4 heads, ff 512; SiLU and sine gates) with projections="hip" against
    projections="torch" at the bf16 contract on the output divided by its largest magnitude, and one block against
    the oracle."""
    announce("same-l blocks fused projections")
    cfg = _cfg("hip")
    rng = np.random.default_rng(3)
    ps_np = [block_params(256, 4, 512, seed=90 + i) for i in range(4)]
    ps = [to_torch(p, DEV, torch.bfloat16) for p in ps_np]
    x = torch.as_tensor(rng.standard_normal((1, 700, 256)).astype(np.float32)).to(DEV, torch.bfloat16)
    fused = same_l.blocks(x, ps, cfg, projections="hip")
    ref = same_l.blocks(x, ps, cfg, projections="torch")
    got, want = fused.float().cpu().numpy(), ref.float().cpu().numpy()
    scale = max(1.0, float(np.abs(want).max()))
    assert_bf16_parity(got / scale, want / scale, f"4 blocks fused vs hipBLASLt (/{scale:.3g})")
    # one block against the oracle
    one = same_l.block(x, ps[3], 3, cfg, projections="hip").float().cpu().numpy()
    oref = oblock.block_xla(cast(x.float().cpu().numpy(), "bf16"), rounded(ps_np[3], "bf16"), 4, 64,
                            cfg.sub_chunk_size, cfg.sinusoidal(3), None, "bf16")
    s1 = max(1.0, float(np.abs(oref).max()))
    assert_bf16_parity(one / s1, oref / s1, f"block 3 fused vs oracle (/{s1:.3g})")


def test_blocks_fall_back_where_the_fused_gemms_do_not_apply():
    """dim 128 (not a multiple of 256): projections="hip" runs the torch projections, bit for bit."""
    announce("same-l blocks fused projections fallback")
    cfg = SameConfig(channels=64, c_mults=(2,), stride=16, transformer_depth=4, sinusoidal_blocks=2, attention="hip")
    ps = [to_torch(block_params(128, 2, 384, seed=95 + i), DEV, torch.bfloat16) for i in range(2)]
    gen = torch.Generator(device=DEV).manual_seed(31)
    x = torch.randn((1, 300, 128), device=DEV, generator=gen).to(torch.bfloat16)
    same_bits(same_l.blocks(x, ps, cfg, projections="hip"), same_l.blocks(x, ps, cfg, projections="torch"),
              "fallback")
    with pytest.raises(ValueError):
        same_l.blocks(x, ps, cfg, projections="cuda")
