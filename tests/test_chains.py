"""The torch restatements that `attention="xla"` runs (hummingbird_amd.xla_chain) against the oracle on the CPU, at
the bf16 and fp16 presets with RoPE and the value mask, and the band wrapper's RoPE-table cache (host logic only).

The GPU tests at full size compare the HIP kernels with these torch chains; this file ties the chains to the
pinned oracle. Both restate the same cast points, so they agree except where a rounding tie falls differently
under a different summation order: every element within one rounding step of the compute dtype, nearly all equal.
"""
from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

from hummingbird_amd import _derived
from hummingbird_amd import band_attention as ba
from hummingbird_amd import workloads, xla_chain
from oracle import band as oband
from oracle import dense as odense

TORCH = {"bf16": torch.bfloat16, "fp16": torch.float16}
FRAC_BITS = {"bf16": 7, "fp16": 10}
MIN_EXP = {"bf16": -126, "fp16": -14}


def _spacing(x: np.ndarray, compute: str) -> np.ndarray:
    """Distance between adjacent values of the compute dtype at |x| (the larger one at a power of two)."""
    e = np.maximum(np.frexp(np.abs(x).astype(np.float64))[1] - 1, MIN_EXP[compute])
    return np.ldexp(1.0, e - FRAC_BITS[compute])


def _close_in_steps(got: np.ndarray, ref: np.ndarray, compute: str, exact_frac: float) -> None:
    """Every element within one rounding step at the scale of the largest output (a branch result that rounds
    the other way moves the difference by one step at the branch's scale), and nearly all elements equal."""
    err = np.abs(got.astype(np.float64) - ref)
    step = float(_spacing(np.abs(ref).max(), compute))
    assert err.max() <= step, f"max error {err.max():.3g} over one rounding step {step:.3g}"
    assert np.mean(err == 0) >= exact_frac, f"only {np.mean(err == 0):.4f} of the elements are equal"


@pytest.mark.parametrize("compute", ["bf16", "fp16"])
@pytest.mark.parametrize("head_dim,half,ragged", [(64, 32, False), (64, 16, True), (128, 64, True)])
def test_dense_torch_chain_matches_oracle(compute, head_dim, half, ragged):
    inp = workloads.dense_inputs(2, 97, 2, head_dim, seed=21, dtype=compute, half=half, ragged=ragged)
    qkv = inp["qkv"]
    if compute == "fp16":
        qkv = qkv.astype(np.float16).astype(np.float32)
    ref = odense.dense_xla(qkv, inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"], 2, head_dim,
                           inp["eps"], inp["lam"], compute)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    got = xla_chain.dense_chain(t(qkv).to(TORCH[compute]), t(inp["q_weight"]), t(inp["k_weight"]), t(inp["inv_freq"]),
                                t(inp["valid"]), 2, head_dim, inp["eps"], t(inp["lam"]))
    _close_in_steps(got.float().numpy(), ref, compute, 0.99)


@pytest.mark.parametrize("compute", ["bf16", "fp16"])
@pytest.mark.parametrize("window", [17, 64])
def test_band_torch_chain_matches_oracle(compute, window):
    inp = workloads.band_inputs(1, 300, 2, 64, window, seed=22, dtype=compute)
    qkv = inp["qkv"]
    if compute == "fp16":
        qkv = qkv.astype(np.float16).astype(np.float32)
    ref = oband.band_xla(qkv, inp["q_norm"], inp["k_norm"], inp["inv_freq"], 2, 64, window, inp["lam"], compute)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(np.asarray(a)))  # noqa: E731
    norm = lambda n: {k: t(v) for k, v in n.items()}  # noqa: E731
    got = xla_chain.band_chain(t(qkv).to(TORCH[compute]), norm(inp["q_norm"]), norm(inp["k_norm"]), t(inp["inv_freq"]),
                               2, 64, window, t(inp["lam"]))
    _close_in_steps(got.float().numpy(), ref, compute, 0.99)


def test_band_table_cache_follows_tensor_lifetime(monkeypatch):
    """The band wrapper caches RoPE tables per caller tensor (id, length, device), rebuilds after an in-place edit,
    and drops an entry when its tensor is garbage-collected."""
    built = []

    def fake_tables(length, inv_freq):
        built.append(length)
        return torch.zeros(length, inv_freq.shape[0]), torch.zeros(length, inv_freq.shape[0])

    monkeypatch.setattr(ba, "rope_tables", fake_tables)
    monkeypatch.setattr(_derived, "_CACHE", {})
    dev = torch.device("cpu")
    f = torch.ones(4)
    a = ba._cached_tables(f, 10, dev)
    assert ba._cached_tables(f, 10, dev)[0] is a[0] and built == [10]
    f.mul_(2.0)  # an in-place edit bumps the version: rebuilt
    ba._cached_tables(f, 10, dev)
    assert built == [10, 10] and len(_derived._CACHE) == 1
    ba._cached_tables(f, 12, dev)
    assert len(_derived._CACHE) == 2
    for _ in range(5):  # a fresh tensor per call does not pile up entries
        ba._cached_tables(torch.ones(4), 10, dev)
        gc.collect()
    assert len(_derived._CACHE) == 2
    del f, a
    gc.collect()
    assert len(_derived._CACHE) == 0


def test_dyt_params_and_bias_vectors_are_converted_once_per_tensor(monkeypatch):
    """A decoder passes the same DyT params and biases to every call: the packed `[alpha | gamma | beta]` vector and
    the fp32 bias are built once per live, unedited set of tensors, rebuilt after an in-place edit of any of them,
    and dropped with them; a Python-number alpha, or an fp32 vector already in place, is used without an entry."""
    monkeypatch.setattr(_derived, "_CACHE", {})
    dev = torch.device("cpu")
    norm = {"alpha": torch.tensor(0.5), "gamma": torch.arange(4.0), "beta": torch.full((4,), 2.0)}
    p = ba.pack_dyt(norm, 4, dev)
    assert p.tolist() == [0.5, 0, 1, 2, 3, 2, 2, 2, 2] and ba.pack_dyt(norm, 4, dev) is p
    norm["beta"].add_(1.0)  # an edit of any one of the three rebuilds the vector
    q = ba.pack_dyt(norm, 4, dev)
    assert q is not p and q.tolist()[-1] == 3.0 and len(_derived._CACHE) == 1
    with pytest.raises(ValueError, match="scalar alpha"):
        ba.pack_dyt(norm, 3, dev)
    assert ba.pack_dyt({**norm, "alpha": 0.25}, 4, dev).tolist()[0] == 0.25 and len(_derived._CACHE) == 1
    b16 = torch.linspace(-1, 1, 6).to(torch.bfloat16)
    v = _derived.f32_vector(b16, dev)
    assert v.dtype == torch.float32 and torch.equal(v, b16.float()) and _derived.f32_vector(b16, dev) is v
    f = torch.ones(3)
    assert _derived.f32_vector(f, dev).data_ptr() == f.data_ptr() and len(_derived._CACHE) == 2
    del norm, p, q, b16, v
    gc.collect()
    assert len(_derived._CACHE) == 0
    with torch.inference_mode():  # inference tensors have no version counter: converted per call, nothing kept
        inf = {"alpha": torch.tensor(0.5), "gamma": torch.ones(4), "beta": torch.zeros(4)}
        assert ba.pack_dyt(inf, 4, dev).tolist() == [0.5, 1, 1, 1, 1, 0, 0, 0, 0]
        assert torch.equal(_derived.f32_vector(torch.ones(3, dtype=torch.bfloat16), dev), torch.ones(3))
    assert len(_derived._CACHE) == 0
