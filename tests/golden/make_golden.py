"""Writes the golden fixtures of this directory: seeded inputs and the oracle's outputs for small dense and band
cases, one compressed .npz per case.

The reference ships no golden vectors, so these come from the oracle (the NumPy restatement of the reference's
XLA chains, sa3jax/dit.py:185-200 and sa3jax/same_l.py:151-169, cast points as the reference's bf16 and
fp32-parity presets). They freeze its outputs so that the GPU parity tests read fixed data and a later change to
the oracle shows up as a fixture mismatch. Inputs come from `hummingbird_amd.workloads` (NumPy PCG64,
`default_rng(seed)`, fixed draw order); every case stores its seed and generator arguments.

bf16 inputs are stored as their bf16 bit patterns (uint16), fp32 inputs as float32; outputs as float32.

Usage (from the repository root): python -m tests.golden.make_golden
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from hummingbird_amd import workloads
from oracle import band as oband
from oracle import dense as odense

HERE = Path(__file__).resolve().parent

# (B, L, H, D, half, dtype, seed, mask recipe)
DENSE_CASES = [
    (2, 1, 2, 64, 32, "bf16", 101, "tail"),
    (2, 7, 2, 64, 16, "bf16", 102, "tail"),
    (1, 64, 2, 64, 32, "bf16", 103, "tail"),
    (2, 129, 2, 64, 16, "bf16", 104, "ragged"),
    (1, 216, 1, 64, 32, "fp32", 105, "tail"),
    (1, 129, 1, 128, 32, "bf16", 106, "ragged"),
    (1, 100, 1, 128, 64, "fp32", 107, "tail"),
    (1, 90, 2, 64, 24, "bf16", 108, "tail"),
]
# (B, S, H, D, window, half, dtype, seed)
BAND_CASES = [
    (1, 1, 2, 64, 17, 32, "bf16", 201),
    (1, 17, 2, 64, 17, 16, "bf16", 202),
    (1, 100, 2, 64, 0, 32, "bf16", 203),
    (1, 100, 1, 64, 1, 32, "fp32", 204),
    (1, 300, 1, 64, 64, 32, "bf16", 205),
    (1, 300, 2, 64, 128, 32, "bf16", 206),
    (1, 150, 1, 64, 17, 16, "fp32", 207),
    (1, 200, 1, 128, 128, 64, "bf16", 208),
]


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """Bit patterns of float32 values that are exactly bf16-representable."""
    bits = np.ascontiguousarray(x, np.float32).view(np.uint32)
    assert not (bits & 0xFFFF).any(), "value is not bf16-representable"
    return (bits >> 16).astype(np.uint16)


def dense_name(c) -> str:
    b, length, h, d, half, dtype, _, mask = c
    return f"dense_B{b}L{length}H{h}D{d}h{half}_{mask}_{dtype}"


def band_name(c) -> str:
    b, s, h, d, w, half, dtype, _ = c
    return f"band_B{b}S{s}H{h}D{d}w{w}h{half}_{dtype}"


def make_dense(c) -> dict:
    b, length, h, d, half, dtype, seed, mask = c
    inp = workloads.dense_inputs(b, length, h, d, seed=seed, dtype=dtype, half=half,
                                 mask_tail=min(16, length // 4), ragged=mask == "ragged")
    out = odense.dense_xla(inp["qkv"], inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"], h, d,
                           inp["eps"], inp["lam"], dtype)
    qkv = bf16_bits(inp["qkv"]) if dtype == "bf16" else inp["qkv"]
    return dict(qkv=qkv, q_weight=inp["q_weight"], k_weight=inp["k_weight"], inv_freq=inp["inv_freq"],
                lam=inp["lam"], valid=inp["valid"], out=np.asarray(out, np.float32),
                meta=np.array(json.dumps(dict(kind="dense", batch=b, length=length, heads=h, head_dim=d, half=half,
                                              dtype=dtype, seed=seed, mask=mask, eps=inp["eps"],
                                              generator="hummingbird_amd.workloads.dense_inputs",
                                              expected="oracle.dense.dense_xla"))))


def make_band(c) -> dict:
    b, s, h, d, w, half, dtype, seed = c
    inp = workloads.band_inputs(b, s, h, d, w, seed=seed, dtype=dtype, half=half)
    out = oband.band_xla(inp["qkv"], inp["q_norm"], inp["k_norm"], inp["inv_freq"], h, d, w, inp["lam"], dtype)
    qkv = bf16_bits(inp["qkv"]) if dtype == "bf16" else inp["qkv"]
    qn, kn = inp["q_norm"], inp["k_norm"]
    return dict(qkv=qkv, q_dyt=np.concatenate([[qn["alpha"]], qn["gamma"], qn["beta"]]).astype(np.float32),
                k_dyt=np.concatenate([[kn["alpha"]], kn["gamma"], kn["beta"]]).astype(np.float32),
                inv_freq=inp["inv_freq"], lam=inp["lam"], out=np.asarray(out, np.float32),
                meta=np.array(json.dumps(dict(kind="band", batch=b, length=s, heads=h, head_dim=d, window=w,
                                              half=half, dtype=dtype, seed=seed,
                                              generator="hummingbird_amd.workloads.band_inputs",
                                              expected="oracle.band.band_xla"))))


def main() -> None:
    for c in DENSE_CASES:
        np.savez_compressed(HERE / f"{dense_name(c)}.npz", **make_dense(c))
    for c in BAND_CASES:
        np.savez_compressed(HERE / f"{band_name(c)}.npz", **make_band(c))
    print(f"wrote {len(DENSE_CASES) + len(BAND_CASES)} fixtures to {HERE}")


if __name__ == "__main__":
    main()
