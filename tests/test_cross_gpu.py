"""GPU parity of the DiT differential cross-attention (hb_cross_prep + hb_cross_attend) against the oracle.

Small shapes (context lengths 1 to 300 with ragged last key tiles, query counts that are not multiples of the
128-query block, head_dim 64 and 128, bf16 and fp32) run against the NumPy oracle of the XLA chain; the 120 s
shape (B=2, L=2584, 257 context tokens, 24 heads) runs against the torch restatement on the GPU and one head
against the oracle; a prepared context is reused by several query sets; the caller mirror with
`attention="hip"` runs against `attention="xla"`.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hummingbird_amd import cross_attention as xattn
from hummingbird_amd import dit, workloads, xla_chain
from hummingbird_amd.config import DiTConfig
from oracle import cross as ocross
from tests.util import assert_bf16_parity, assert_fp32_parity, stats

pytestmark = pytest.mark.gpu
DEV = "cuda"


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def dev(a: np.ndarray, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return t.to(dtype) if dtype is not None else t


def run_hip(inp: dict, dtype=torch.bfloat16, lam=True) -> np.ndarray:
    ctx = xattn.prepare_cross_kv(dev(inp["kv"], dtype), dev(inp["k_weight"]), inp["heads"], inp["head_dim"],
                                 inp["eps"])
    out = xattn.cross_attention(dev(inp["q"], dtype), ctx, dev(inp["q_weight"]), inp["eps"],
                                lam=dev(inp["lam"]) if lam else None)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def oracle(inp: dict, compute: str, lam=True) -> np.ndarray:
    return ocross.cross_xla(inp["q"], inp["kv"], inp["q_weight"], inp["k_weight"], inp["heads"], inp["head_dim"],
                            inp["eps"], inp["lam"] if lam else None, compute)


SMALL = [  # (B, L, Nk, H, D)
    (1, 1, 1, 2, 64), (2, 100, 17, 2, 64), (1, 300, 257, 2, 64), (2, 216, 64, 3, 128), (1, 129, 300, 2, 64),
    (1, 70, 129, 2, 128), (1, 200, 1, 2, 64), (2, 131, 65, 1, 64),
]


@pytest.mark.parametrize("shape", SMALL, ids=lambda s: "B%dL%dNk%dH%dD%d" % s)
def test_cross_small_vs_oracle(shape):
    b, length, nk, h, d = shape
    announce(f"cross bf16 {shape}")
    inp = workloads.cross_inputs(b, length, nk, h, d, seed=length + nk)
    assert_bf16_parity(run_hip(inp), oracle(inp, "bf16"), f"cross {shape}")


@pytest.mark.parametrize("shape", SMALL[:6], ids=lambda s: "B%dL%dNk%dH%dD%d" % s)
def test_cross_fp32_vs_oracle(shape):
    b, length, nk, h, d = shape
    announce(f"cross fp32 {shape}")
    inp = workloads.cross_inputs(b, length, nk, h, d, seed=length + nk + 1, dtype="fp32")
    assert_fp32_parity(run_hip(inp, torch.float32), oracle(inp, "fp32"), f"cross fp32 {shape}")


def test_cross_no_lambda_and_identical_branches():
    announce("cross bf16 lam=None, identical branches")
    inp = workloads.cross_inputs(1, 150, 40, 2, 64, seed=3)
    assert_bf16_parity(run_hip(inp, lam=False), oracle(inp, "bf16", lam=False), "cross lam=None")
    E = 128
    inp["q"][..., E:] = inp["q"][..., :E]
    inp["kv"][..., E:2 * E] = inp["kv"][..., :E]
    assert np.count_nonzero(run_hip(inp, lam=False)) == 0


def test_cross_large_gains_take_running_max_path():
    """Gains ~ 6 make the logit bound exceed 64, so the running-max softmax runs; checked at the contract
    against the oracle (bf16 logits in the XLA chain, fp32 logits here)."""
    announce("cross bf16 gains 6 (running-max path)")
    inp = workloads.cross_inputs(1, 200, 77, 2, 64, seed=4, gain_mean=6.0)
    got, ref = run_hip(inp), oracle(inp, "bf16")
    assert stats(got, ref)["cosine"] >= 0.999, stats(got, ref)


def test_cross_context_reused_by_several_query_sets():
    """One prepared context, three query sets (as one block's cross-attention over the sampler steps): each
    result is bit-identical to a fresh preparation and within the contract of the oracle."""
    announce("cross bf16 context reuse")
    inp = workloads.cross_inputs(2, 260, 257, 3, 64, seed=5)
    ctx = xattn.prepare_cross_kv(dev(inp["kv"], torch.bfloat16), dev(inp["k_weight"]), 3, 64, inp["eps"])
    for step in range(3):
        q = workloads.cross_inputs(2, 260, 1, 3, 64, seed=100 + step)["q"]
        out = xattn.cross_attention(dev(q, torch.bfloat16), ctx, dev(inp["q_weight"]), inp["eps"],
                                    lam=dev(inp["lam"])).float().cpu().numpy()
        fresh = run_hip(dict(inp, q=q))
        assert np.array_equal(out, fresh), f"step {step}: reused context differs from a fresh one"
        assert_bf16_parity(out, oracle(dict(inp, q=q), "bf16"), f"reuse step {step}")


def test_cross_120s_vs_torch_chain():
    """The 120 s clip's cross-attention (B=2, L=2584 queries, 257 context tokens, 24 heads of 64) against the
    torch restatement of the XLA chain on the GPU, and one head against the oracle."""
    c = workloads.CROSS_120S
    B, L, Nk, H, D = c["batch"], c["length"], c["context"], c["heads"], c["head_dim"]
    announce(f"cross bf16 120s B={B} L={L} Nk={Nk} H={H}")
    inp = workloads.cross_inputs(B, L, Nk, H, D, seed=6)
    got = run_hip(inp)
    q, kv = dev(inp["q"], torch.bfloat16), dev(inp["kv"], torch.bfloat16)
    context = xla_chain.cross_kv(kv, dev(inp["k_weight"]), H, D, inp["eps"])
    ref = xla_chain.cross_chain(q, context, dev(inp["q_weight"]), H, D, inp["eps"],
                                lam=dev(inp["lam"])).float().cpu().numpy()
    assert_bf16_parity(got, ref, "cross 120s vs torch chain")
    hh = H - 1
    E = H * D
    qcols = np.concatenate([np.arange(s * E + hh * D, s * E + hh * D + D) for s in range(2)])
    kcols = np.concatenate([np.arange(s * E + hh * D, s * E + hh * D + D) for s in range(3)])
    head = dict(inp, q=np.ascontiguousarray(inp["q"][-1:, :, qcols]), kv=np.ascontiguousarray(inp["kv"][-1:, :, kcols]),
                heads=1, lam=inp["lam"][hh:hh + 1])
    assert_bf16_parity(got[-1, :, hh * D:(hh + 1) * D], oracle(head, "bf16")[0], "cross 120s last head vs oracle")


def test_cross_reference_geometry_64_query_workgroups():
    """The reference's own 120 s geometry (B=1, L=1422, 257 context tokens, 24 heads: 288 workgroups of 128
    queries, run as 64-query workgroups) against the torch restatement."""
    B, L, Nk, H, D = 1, 1422, 257, 24, 64
    announce(f"cross bf16 reference geometry B={B} L={L} Nk={Nk} H={H}")
    inp = workloads.cross_inputs(B, L, Nk, H, D, seed=8)
    got = run_hip(inp)
    context = xla_chain.cross_kv(dev(inp["kv"], torch.bfloat16), dev(inp["k_weight"]), H, D, inp["eps"])
    ref = xla_chain.cross_chain(dev(inp["q"], torch.bfloat16), context, dev(inp["q_weight"]), H, D, inp["eps"],
                                lam=dev(inp["lam"])).float().cpu().numpy()
    assert_bf16_parity(got, ref, "cross reference geometry vs torch chain")


def test_cross_caller_mirror_hip_vs_xla():
    """dit.cross_context + dit.cross_attention with attention="hip" against attention="xla" on the GPU (bf16):
    to_kv and to_q projections, the attention, to_out."""
    announce("cross caller mirror")
    rng = np.random.default_rng(7)
    H, D, C = 4, 64, 96
    E = H * D
    w = lambda *s: dev((rng.standard_normal(s) / np.sqrt(s[-1])).astype(np.float32), torch.bfloat16)  # noqa: E731
    block = {"cross_attn": {"to_kv": {"weight": w(3 * E, C)}, "to_q": {"weight": w(2 * E, E)},
                            "to_out": {"weight": w(E, E)},
                            "q_norm": {"weight": dev((1 + 0.02 * rng.standard_normal(D)).astype(np.float32))},
                            "k_norm": {"weight": dev((1 + 0.02 * rng.standard_normal(D)).astype(np.float32))}}}
    ctx = dev(rng.standard_normal((2, 57, C)).astype(np.float32), torch.bfloat16)
    h = dev(rng.standard_normal((2, 333, E)).astype(np.float32), torch.bfloat16)
    outs = {}
    for mode in ("hip", "xla"):
        cfg = DiTConfig(embed_dim=E, num_heads=H, attention=mode, differential=True)
        context = dit.cross_context(block, ctx, cfg)
        outs[mode] = dit.cross_attention(h, block, context, cfg).float().cpu().numpy()
    assert_bf16_parity(outs["hip"], outs["xla"], "caller mirror hip vs xla")


def test_cross_errors_are_value_errors():
    announce("cross argument errors")
    kv = torch.zeros((1, 8, 3 * 2 * 64), device=DEV, dtype=torch.bfloat16)
    ones = torch.ones(64, device=DEV)
    with pytest.raises(ValueError):
        xattn.prepare_cross_kv(kv[..., :-8], ones, 2, 64, 1e-6)
    with pytest.raises(ValueError):
        xattn.prepare_cross_kv(torch.zeros((1, 8, 3 * 2 * 96), device=DEV, dtype=torch.bfloat16), torch.ones(96), 2,
                               96, 1e-6)
    ctx = xattn.prepare_cross_kv(kv, ones, 2, 64, 1e-6)
    with pytest.raises(ValueError):
        xattn.cross_attention(torch.zeros((1, 4, 3 * 2 * 64), device=DEV, dtype=torch.bfloat16), ctx, ones, 1e-6)
    with pytest.raises(TypeError):
        xattn.cross_attention(torch.zeros((1, 4, 2 * 2 * 64), device=DEV), ctx, ones, 1e-6)
    with pytest.raises(ValueError):
        xattn.cross_attention(torch.zeros((2, 4, 2 * 2 * 64), device=DEV, dtype=torch.bfloat16), ctx, ones, 1e-6)
