"""Comparison helpers and the parity tolerances of the two kernels.

Tolerances (bf16 inputs): fp32 max-abs error <= 2e-2 and cosine similarity >= 0.9999 against the reference's
XLA chain (the oracle); fp32 inputs: max-abs error <= 1e-5 relative to the reference output's max-abs.
"""
from __future__ import annotations

import numpy as np

BF16_MAX_ABS = 2e-2
BF16_COSINE = 0.9999
FP32_REL = 1e-5


def stats(got: np.ndarray, ref: np.ndarray) -> dict:
    g = np.asarray(got, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    err = np.abs(g - r)
    denom = np.linalg.norm(g) * np.linalg.norm(r)
    cos = float(g @ r / denom) if denom > 0 else (1.0 if np.allclose(g, r) else 0.0)
    scale = float(np.abs(r).max()) if r.size else 0.0
    return {"max_abs": float(err.max()) if err.size else 0.0, "cosine": cos,
            "rel": float(err.max() / scale) if scale > 0 and err.size else float(err.max() if err.size else 0.0),
            "finite": bool(np.isfinite(g).all())}


def assert_bf16_parity(got: np.ndarray, ref: np.ndarray, what: str = "") -> dict:
    s = stats(got, ref)
    assert s["finite"], f"{what}: non-finite output"
    assert s["max_abs"] <= BF16_MAX_ABS, f"{what}: max-abs {s['max_abs']:.3g} > {BF16_MAX_ABS} ({s})"
    assert s["cosine"] >= BF16_COSINE, f"{what}: cosine {s['cosine']:.7f} < {BF16_COSINE} ({s})"
    return s


def assert_fp32_parity(got: np.ndarray, ref: np.ndarray, what: str = "") -> dict:
    s = stats(got, ref)
    assert s["finite"], f"{what}: non-finite output"
    assert s["rel"] <= FP32_REL, f"{what}: relative max error {s['rel']:.3g} > {FP32_REL} ({s})"
    return s
