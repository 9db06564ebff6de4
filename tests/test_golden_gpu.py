"""The HIP kernels against the committed golden fixtures (inputs and oracle outputs read from tests/golden).

bf16 cases: max-abs <= 2e-2 and cosine >= 0.9999; fp32 cases: max-abs <= 1e-5 relative to the fixture's max-abs.
"""
from __future__ import annotations

import pytest
import torch

from hummingbird_amd import band_attention as ba
from hummingbird_amd import dense_attention as da
from tests.golden_util import fixtures, load
from tests.util import assert_bf16_parity, assert_fp32_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = {"bf16": torch.bfloat16, "fp32": torch.float32}


def t(x):
    return torch.as_tensor(x).to(DEV)


@pytest.mark.parametrize("path", fixtures("dense"), ids=lambda p: p.stem)
def test_dense_vs_golden(path):
    print(f"\n[case] golden {path.stem}", flush=True)
    f = load(path)
    dtype = DTYPES[f["dtype"]]
    qkv = t(f["qkv"]).to(dtype)
    cos, sin, mask = da.tables(f["length"], t(f["inv_freq"]), t(f["valid"]), f["head_dim"], dtype)
    out = da.dense_attention(qkv, t(f["q_weight"]), t(f["k_weight"]), cos, sin, mask, f["heads"], f["head_dim"],
                             f["half"], f["eps"], lam=t(f["lam"]))
    got = out.float().cpu().numpy()
    check = assert_bf16_parity if f["dtype"] == "bf16" else assert_fp32_parity
    check(got, f["out"], path.stem)


@pytest.mark.parametrize("path", fixtures("band"), ids=lambda p: p.stem)
def test_band_vs_golden(path):
    print(f"\n[case] golden {path.stem}", flush=True)
    f = load(path)
    dtype = DTYPES[f["dtype"]]
    qkv = t(f["qkv"]).to(dtype)
    norms = [{k: t(v) for k, v in f[name].items()} for name in ("q_norm", "k_norm")]
    out = ba.band_attention(qkv, norms[0], norms[1], t(f["inv_freq"]), f["heads"], f["head_dim"], f["window"],
                            lam=t(f["lam"]))
    got = out.float().cpu().numpy()
    check = assert_bf16_parity if f["dtype"] == "bf16" else assert_fp32_parity
    check(got, f["out"], path.stem)
