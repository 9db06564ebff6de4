"""DiT differential cross-attention on the CPU (no GPU here):

* the oracle's restatement (oracle/cross.py) pinned against torch's SDPA in float64, against the dense oracle
  (already pinned) on inputs where the two chains coincide, and against closed-form special cases; planted
  mistakes must fail those pins;
* the torch restatement that `attention="xla"` runs, and the caller mirror, against the oracle;
* the C ABI's host-side checks of the cross-attention entry points (no kernel is launched).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from hummingbird_amd import _lib, dit, workloads, xla_chain
from hummingbird_amd.config import DiTConfig
from oracle import cross as ocross
from oracle import dense as odense
from tests.util import assert_bf16_parity, assert_fp32_parity


def _split_heads(x: np.ndarray, i: int, heads: int, dim: int) -> np.ndarray:
    b, n, _ = x.shape
    return x[..., i * heads * dim:(i + 1) * heads * dim].reshape(b, n, heads, dim).transpose(0, 2, 1, 3)


def _torch_cross(inp: dict, lam: np.ndarray) -> np.ndarray:
    """Independent composition: sections sliced by index, the oracle's (separately pinned) RMSNorm in fp32, then
    torch's SDPA in float64 over all context keys, and the subtraction."""
    H, D, eps = inp["heads"], inp["head_dim"], inp["eps"]
    q, qd = (odense.rms(_split_heads(inp["q"], i, H, D), inp["q_weight"], eps, "fp32") for i in (0, 1))
    k, kd = (odense.rms(_split_heads(inp["kv"], i, H, D), inp["k_weight"], eps, "fp32") for i in (0, 1))
    v = _split_heads(inp["kv"], 2, H, D)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).double()  # noqa: E731
    out = (F.scaled_dot_product_attention(t(q), t(k), t(v))
           - torch.from_numpy(lam).double()[None, :, None, None] * F.scaled_dot_product_attention(t(qd), t(kd), t(v)))
    return odense.merge(out.numpy())


def _oracle(inp: dict, compute: str, lam=None) -> np.ndarray:
    return ocross.cross_xla(inp["q"], inp["kv"], inp["q_weight"], inp["k_weight"], inp["heads"], inp["head_dim"],
                            inp["eps"], inp["lam"] if lam is None else lam, compute)


@pytest.mark.parametrize("shape", [(2, 37, 17, 3, 64), (1, 20, 300, 2, 128), (1, 5, 1, 2, 64)],
                         ids=lambda s: "B%dL%dNk%dH%dD%d" % s)
def test_cross_fp32_matches_torch_sdpa(shape):
    b, length, nk, h, d = shape
    inp = workloads.cross_inputs(b, length, nk, h, d, seed=length + nk, dtype="fp32")
    np.testing.assert_allclose(_oracle(inp, "fp32"), _torch_cross(inp, inp["lam"]), atol=2e-6, rtol=1e-5)


@pytest.mark.parametrize("compute", ["bf16", "fp32"])
def test_cross_equals_dense_without_rope_and_mask(compute):
    """With as many context tokens as queries, cross-attention is the dense chain on the packed row
    [q | k | v | q_diff | k_diff] without RoPE (half = 0) and without a mask: bit-identical."""
    inp = workloads.cross_inputs(2, 40, 40, 2, 64, seed=11, dtype=compute)
    E = 2 * 64
    q, kv = inp["q"], inp["kv"]
    qkv = np.concatenate([q[..., :E], kv[..., :E], kv[..., 2 * E:], q[..., E:], kv[..., E:2 * E]], axis=-1)
    dense = odense.dense_xla(qkv, inp["q_weight"], inp["k_weight"], workloads.inv_freq(0), None, 2, 64, inp["eps"],
                             inp["lam"], compute)
    assert np.array_equal(_oracle(inp, compute), dense)


def test_cross_special_cases():
    # one context token: each softmax is 1 on it, so every query gets (1 - lam) * v
    one = workloads.cross_inputs(1, 9, 1, 2, 64, seed=12, dtype="fp32")
    v = one["kv"][0, 0, 2 * 128:]
    expect = v * np.repeat(1.0 - one["lam"], 64)
    np.testing.assert_allclose(_oracle(one, "fp32")[0], np.tile(expect, (9, 1)), atol=1e-6)
    # q = q_diff = 0: uniform weights over the context, so every query gets (1 - lam) * mean(v)
    inp = workloads.cross_inputs(1, 7, 33, 2, 64, seed=13, dtype="fp32")
    inp["q"] = np.zeros_like(inp["q"])
    mean = inp["kv"][0, :, 2 * 128:].mean(0)
    np.testing.assert_allclose(_oracle(inp, "fp32")[0], np.tile(mean * np.repeat(1.0 - inp["lam"], 64), (7, 1)),
                               atol=1e-6)


def test_cross_identical_branches_cancel_and_linearity():
    inp = workloads.cross_inputs(1, 30, 50, 2, 64, seed=14)
    E = 128
    inp["q"][..., E:] = inp["q"][..., :E]
    inp["kv"][..., E:2 * E] = inp["kv"][..., :E]
    assert np.count_nonzero(_oracle(inp, "bf16", lam=np.ones(2, np.float32))) == 0
    base = workloads.cross_inputs(1, 30, 50, 2, 64, seed=15, dtype="fp32")
    f = lambda lam: _oracle(base, "fp32", lam=np.full(2, lam, np.float32))  # noqa: E731
    np.testing.assert_allclose(f(0.3), 0.7 * f(0.0) + 0.3 * f(1.0), atol=1e-6)


@pytest.mark.parametrize("compute", ["bf16", "fp32"])
def test_torch_chain_matches_oracle(compute):
    inp = workloads.cross_inputs(2, 100, 57, 3, 64, seed=16, dtype=compute)
    dt = torch.bfloat16 if compute == "bf16" else torch.float32
    ctx = xla_chain.cross_kv(torch.from_numpy(inp["kv"]).to(dt), torch.from_numpy(inp["k_weight"]), 3, 64, inp["eps"])
    got = xla_chain.cross_chain(torch.from_numpy(inp["q"]).to(dt), ctx, torch.from_numpy(inp["q_weight"]), 3, 64,
                                inp["eps"], lam=torch.from_numpy(inp["lam"])).float().numpy()
    check = assert_bf16_parity if compute == "bf16" else assert_fp32_parity
    check(got, _oracle(inp, compute), f"torch chain {compute}")


def test_caller_mirror_xla_on_cpu_matches_oracle():
    """dit.cross_context + dit.cross_attention with attention="xla" (fp32 on the CPU): to_kv and to_q
    projections, the chain, to_out; against the oracle composed with the same projections."""
    rng = np.random.default_rng(17)
    H, D, C = 2, 64, 96
    E = H * D
    cfg = DiTConfig(embed_dim=E, num_heads=H, attention="xla", differential=True)
    w = lambda *s: (rng.standard_normal(s) / np.sqrt(s[-1])).astype(np.float32)  # noqa: E731
    block = {"cross_attn": {"to_kv": {"weight": torch.from_numpy(w(3 * E, C))},
                            "to_q": {"weight": torch.from_numpy(w(2 * E, E))},
                            "to_out": {"weight": torch.from_numpy(w(E, E))},
                            "q_norm": {"weight": torch.from_numpy((1 + 0.02 * rng.standard_normal(D)).astype(np.float32))},
                            "k_norm": {"weight": torch.from_numpy((1 + 0.02 * rng.standard_normal(D)).astype(np.float32))}}}
    ctx = rng.standard_normal((2, 19, C)).astype(np.float32)
    h = rng.standard_normal((2, 33, E)).astype(np.float32)
    context = dit.cross_context(block, torch.from_numpy(ctx), cfg)
    got = dit.cross_attention(torch.from_numpy(h), block, context, cfg).numpy()
    a = block["cross_attn"]
    kv = ctx @ a["to_kv"]["weight"].numpy().T
    q = h @ a["to_q"]["weight"].numpy().T
    ref = ocross.cross_xla(q, kv, a["q_norm"]["weight"].numpy(), a["k_norm"]["weight"].numpy(), H, D,
                           cfg.qk_norm_eps, None, "fp32") @ a["to_out"]["weight"].numpy().T
    np.testing.assert_allclose(got, ref, atol=1e-5, rtol=1e-4)


# ---- planted mistakes: each must be caught by one of the pins above -------------------------------------------
def test_planted_swapped_kv_sections_are_caught(monkeypatch):
    orig = ocross.prepare_kv

    def wrong(kv, k_weight, num_heads, head_dim, eps, compute):  # v taken from the k_diff section and vice versa
        k, kd, v = orig(kv, k_weight, num_heads, head_dim, eps, compute)
        return k, v, kd
    monkeypatch.setattr(ocross, "prepare_kv", wrong)
    with pytest.raises(AssertionError):
        test_cross_fp32_matches_torch_sdpa((2, 37, 17, 3, 64))


def test_planted_missing_q_norm_is_caught(monkeypatch):
    orig = ocross.rms
    calls = {"n": 0}

    def wrong(x, weight, eps, compute):  # the first two calls are q and q_diff: leave them un-normed
        calls["n"] += 1
        return odense.cast(np.asarray(x, np.float32), compute) if calls["n"] <= 2 else orig(x, weight, eps, compute)
    monkeypatch.setattr(ocross, "rms", wrong)
    with pytest.raises(AssertionError):
        test_cross_fp32_matches_torch_sdpa((2, 37, 17, 3, 64))


# ---- the C ABI's host-side checks ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libhummingbird_amd.so is not built: run `python -m hummingbird_amd._build`")
    return _lib.load()


@pytest.mark.parametrize("kw,status", [
    ({}, 0), ({"D": 128, "H": 12}, 0), ({"D": 96}, 4), ({"dtype": 5}, 3), ({"Nk": 0}, 2), ({"L": 0}, 2),
    ({"qs": 2 * 24 * 64 - 8}, 7), ({"kvs": 3 * 24 * 64 + 4}, 7), ({"eps": float("nan")}, 10),
])
def test_cross_validate(lib, kw, status):
    a = {**dict(dtype=0, qs=2 * 24 * 64, kvs=3 * 24 * 64, B=2, L=2584, Nk=257, H=24, D=64, eps=1e-6), **kw}
    if "H" in kw:
        a["qs"], a["kvs"] = 2 * a["H"] * a["D"], 3 * a["H"] * a["D"]
    assert lib.hb_cross_validate(a["dtype"], a["qs"], a["kvs"], a["B"], a["L"], a["Nk"], a["H"], a["D"],
                                 a["eps"]) == status
    if status:
        assert lib.hb_last_error()


def test_cross_workspace_size(lib):
    # three (B, H, round_up(Nk, 128), D) regions: k, k_diff, v prepared
    assert lib.hb_cross_workspace_size(0, 2, 257, 24, 64) == 3 * 2 * 24 * 384 * 64 * 2
    assert lib.hb_cross_workspace_size(1, 1, 1, 1, 128) == 3 * 128 * 128 * 4
    assert lib.hb_cross_workspace_size(0, 1, 10, 1, 96) == 0


def test_cross_errors_before_any_launch(lib):
    """Missing, short or misaligned buffers are rejected with their status codes before any GPU call (fake,
    never dereferenced addresses; the checks read only the pointer values)."""
    B, L, Nk, H, D = 1, 100, 30, 2, 64
    need = lib.hb_cross_workspace_size(0, B, Nk, H, D)
    x, w, ws, out = 0x10000, 0x20000, 0x40000, 0x50000
    prep = lambda kv=x, kw=w, wsp=ws, wsb=need: lib.hb_cross_prep(None, kv, 0, 3 * H * D, kw, B, Nk, H, D,  # noqa: E731
                                                                   ctypes.c_float(1e-6), wsp, wsb)
    assert prep(kv=None) == 1 and prep(kw=None) == 1 and prep(wsp=None) == 1
    assert prep(kv=x + 2) == 7                    # kv not 16-byte aligned
    assert prep(wsb=need - 1) == 8 and prep(wsp=ws + 64) == 8
    attend = lambda q=x, o=out, wsp=ws, wsb=need: lib.hb_cross_attend(None, q, 0, 2 * H * D, w, w, None, o, B, L,  # noqa: E731
                                                                       Nk, H, D, ctypes.c_float(1e-6), wsp, wsb)
    assert attend(q=None) == 1 and attend(o=None) == 1
    assert attend(q=x + 4) == 7 and attend(o=out + 2) == 7
    assert attend(wsb=need - 1) == 8
    assert "workspace" in lib.hb_last_error().decode()
