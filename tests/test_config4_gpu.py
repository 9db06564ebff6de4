"""The mixed-shape sweep on the GPU: DiT dense differential attention at L in {1292, 2584} (B = 2) with head_dim 64
(24 heads) and 128 (12 heads), bf16 and fp32, ragged value masks zeroing a random 0-25 % tail per batch row; SAME-L
band attention over S = 16384 frames at half-widths w in {64, 128, 256} (windows 128, 256, 512) with head_dim 64 (8
heads: the streaming ring kernel for w <= 128, the tiled kernels for w = 256) and 128 (4 heads: the tiled kernels),
bf16 and fp32. Seeded N(0, 1) inputs.

Every case checks the whole output against the torch restatement of the reference's XLA chain on the GPU
(hummingbird_amd.xla_chain, itself tied to the oracle in tests/test_chains.py), and the first and last 300 rows of
one head against the NumPy oracle. Tolerances: bf16 max-abs <= 2e-2 and cosine >= 0.9999; fp32 max error <= 1e-5
relative to the output's largest magnitude.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hummingbird_amd import workloads, xla_chain
from oracle import band as oband
from oracle import dense as odense
from tests.test_band_gpu import norm_t
from tests.test_band_gpu import run_hip as band_hip
from tests.test_dense_gpu import run_hip as dense_hip
from tests.util import assert_bf16_parity, assert_fp32_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"
TORCH = {"bf16": torch.bfloat16, "fp32": torch.float32}


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def check(got: np.ndarray, ref: np.ndarray, dtype: str, what: str) -> None:
    (assert_bf16_parity if dtype == "bf16" else assert_fp32_parity)(got, ref, what)


def head_columns(h: int, heads: int, d: int) -> np.ndarray:
    """Columns of head h in each of the five sections of a packed qkv row."""
    hd = heads * d
    return np.concatenate([np.arange(s * hd + h * d, s * hd + h * d + d) for s in range(5)])


DENSE = [(length, d, dtype) for length in (1292, 2584) for d in (64, 128) for dtype in ("bf16", "fp32")]


@pytest.mark.parametrize("length,d,dtype", DENSE, ids=lambda v: str(v))
def test_dense_sweep(length, d, dtype):
    B, H = 2, 1536 // d
    announce(f"dense sweep {dtype} B={B} L={length} H={H} D={d} ragged")
    inp = workloads.dense_inputs(B, length, H, d, seed=length + d, dtype=dtype, ragged=True)
    got = dense_hip(inp, dtype=TORCH[dtype])
    t = lambda a: torch.from_numpy(a).to(DEV)  # noqa: E731
    ref = xla_chain.dense_chain(t(inp["qkv"]).to(TORCH[dtype]), t(inp["q_weight"]), t(inp["k_weight"]),
                                t(inp["inv_freq"]), t(inp["valid"]), H, d, inp["eps"],
                                lam=t(inp["lam"])).float().cpu().numpy()
    check(got, ref, dtype, f"dense sweep L={length} D={d} {dtype} vs torch chain")
    h, b = H - 1, B - 1  # the last head of the last batch row (its own ragged tail)
    sub = dict(inp, qkv=np.ascontiguousarray(inp["qkv"][b:b + 1, :, head_columns(h, H, d)]), heads=1,
               lam=inp["lam"][h:h + 1], valid=inp["valid"][b:b + 1])
    exp = odense.dense_xla(sub["qkv"], sub["q_weight"], sub["k_weight"], sub["inv_freq"], sub["valid"], 1, d,
                           sub["eps"], sub["lam"], dtype)[0]
    for lo, hi in ((0, 300), (length - 300, length)):
        check(got[b, lo:hi, h * d:(h + 1) * d], exp[lo:hi], dtype, f"dense sweep rows [{lo},{hi}) vs oracle")


BAND = [(d, w, dtype) for d in (64, 128) for w in (64, 128, 256) for dtype in ("bf16", "fp32")]


@pytest.mark.parametrize("d,w,dtype", BAND, ids=lambda v: str(v))
def test_band_sweep(d, w, dtype):
    S, H = 16384, 512 // d
    announce(f"band sweep {dtype} S={S} H={H} D={d} w={w}")
    inp = workloads.band_inputs(1, S, H, d, w, seed=S + w + d, dtype=dtype)
    got = band_hip(inp, dtype=TORCH[dtype])
    t = lambda a: torch.from_numpy(np.asarray(a)).to(DEV)  # noqa: E731
    ref = xla_chain.band_chain(t(inp["qkv"]).to(TORCH[dtype]), norm_t(inp["q_norm"]), norm_t(inp["k_norm"]),
                               t(inp["inv_freq"]), H, d, w, lam=t(inp["lam"])).float().cpu().numpy()
    check(got, ref, dtype, f"band sweep D={d} w={w} {dtype} vs torch chain")
    h = H - 1  # the oracle over the whole last head (RoPE positions stay absolute), checked at both sequence ends
    qkv = np.ascontiguousarray(inp["qkv"][:, :, head_columns(h, H, d)])
    exp = oband.band_xla(qkv, inp["q_norm"], inp["k_norm"], inp["inv_freq"], 1, d, w, inp["lam"][h:h + 1], dtype)[0]
    for lo, hi in ((0, 300), (S - 300, S)):
        check(got[0, lo:hi, h * d:(h + 1) * d], exp[lo:hi], dtype, f"band sweep rows [{lo},{hi}) vs oracle")
