"""The committed golden fixtures against their generator and the oracle (CPU).

Each fixture holds seeded inputs and the oracle's output at the time it was written (tests/golden/make_golden.py).
Here the inputs must be reproduced exactly from the stored seed and recipe, and the oracle run on them today must
still give the stored output; the GPU kernels are checked against the same files in test_golden_gpu.py.
"""
from __future__ import annotations

import numpy as np
import pytest

from hummingbird_amd import workloads
from oracle import band as oband
from oracle import dense as odense
from tests.golden_util import fixtures, load
from tests.util import stats

DENSE = fixtures("dense")
BAND = fixtures("band")


def test_fixture_set_is_complete():
    assert len(DENSE) >= 8 and len(BAND) >= 8


@pytest.mark.parametrize("path", DENSE, ids=lambda p: p.stem)
def test_dense_fixture(path):
    f = load(path)
    inp = workloads.dense_inputs(f["batch"], f["length"], f["heads"], f["head_dim"], seed=f["seed"], dtype=f["dtype"],
                                 half=f["half"], mask_tail=min(16, f["length"] // 4), ragged=f["mask"] == "ragged")
    for key in ("qkv", "q_weight", "k_weight", "inv_freq", "lam", "valid"):
        assert np.array_equal(inp[key], f[key]), key
    out = odense.dense_xla(f["qkv"], f["q_weight"], f["k_weight"], f["inv_freq"], f["valid"], f["heads"],
                           f["head_dim"], f["eps"], f["lam"], f["dtype"])
    s = stats(out, f["out"])
    if f["dtype"] == "fp32":
        assert s["rel"] <= 1e-6, s
    else:  # bf16 outputs: at most a rounding flip from a different BLAS summation order
        assert s["max_abs"] <= 8e-3 and s["cosine"] >= 0.999999, s


@pytest.mark.parametrize("path", BAND, ids=lambda p: p.stem)
def test_band_fixture(path):
    f = load(path)
    inp = workloads.band_inputs(f["batch"], f["length"], f["heads"], f["head_dim"], f["window"], seed=f["seed"],
                                dtype=f["dtype"], half=f["half"])
    for key in ("qkv", "inv_freq", "lam"):
        assert np.array_equal(inp[key], f[key]), key
    for name in ("q_norm", "k_norm"):
        for k in ("alpha", "gamma", "beta"):
            assert np.array_equal(np.asarray(inp[name][k]), np.asarray(f[name][k])), (name, k)
    out = oband.band_xla(f["qkv"], f["q_norm"], f["k_norm"], f["inv_freq"], f["heads"], f["head_dim"], f["window"],
                         f["lam"], f["dtype"])
    s = stats(out, f["out"])
    if f["dtype"] == "fp32":
        assert s["rel"] <= 1e-6, s
    else:
        assert s["max_abs"] <= 8e-3 and s["cosine"] >= 0.999999, s
