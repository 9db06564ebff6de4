"""The caller mirrors with attention="hip" on the GPU against attention="xla" (the torch restatement of the
reference's plain chain) on the same device and weights: config 0 geometry (L=216, 24 heads of 64, partial rotary
half 16) in fp32 and bf16 for the DiT, a MEDIUM-width SAME-L block (24 heads, half-width 17) for the band.
Reference: sa3jax/dit.py:185-200, sa3jax/same_l.py:151-169."""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from hummingbird_amd import dit, same_l, workloads
from hummingbird_amd.config import MEDIUM_DIT, MEDIUM_SAME_L
from tests.test_callers import dit_case
from tests.util import assert_bf16_parity, assert_fp32_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"


def to(x, dtype):
    if isinstance(x, dict):
        return {k: to(v, dtype) for k, v in x.items()}
    return x.to(DEV, dtype if x.is_floating_point() else x.dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_dit_self_attention_hip_vs_xla(dtype):
    print(f"\n[case] dit.self_attention hip vs xla {dtype}", flush=True)
    cfg = MEDIUM_DIT
    h, valid, inv_freq, block, lam = dit_case(cfg, 2, 216 - cfg.num_memory_tokens)
    h, block = to(h, dtype), to(block, dtype)
    for norm in ("q_norm", "k_norm"):  # the gains stay fp32, as in the reference's norm params
        block["self_attn"][norm]["weight"] = block["self_attn"][norm]["weight"].float()
    inv_freq, valid, lam = inv_freq.to(DEV), valid.to(DEV), lam.to(DEV)
    got = dit.self_attention(h, block, dit.static_tables(inv_freq, valid, cfg, dtype), cfg, lam=lam)
    xcfg = dataclasses.replace(cfg, attention="xla")
    ref = dit.self_attention(h, block, dit.static_tables(inv_freq, valid, xcfg, dtype), xcfg, lam=lam)
    check = assert_fp32_parity if dtype == torch.float32 else assert_bf16_parity
    check(got.float().cpu().numpy(), ref.float().cpu().numpy(), f"dit {dtype}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_dit_self_attention_hip_projections_vs_xla(dtype):
    """projections="hip" (the fused to_qkv GEMM + attention over its output + the to_out GEMM) against the XLA
    chain on the same weights, and against projections="torch" at the bf16 contract."""
    from hummingbird_amd import projection

    print(f"\n[case] dit.self_attention hip projections {dtype}", flush=True)
    cfg = MEDIUM_DIT
    assert projection.fused_supported(dtype, cfg.num_heads, cfg.head_dim, cfg.embed_dim, cfg.rope_dim // 2)
    h, valid, inv_freq, block, lam = dit_case(cfg, 2, 216 - cfg.num_memory_tokens)
    h, block = to(h, dtype), to(block, dtype)
    for norm in ("q_norm", "k_norm"):
        block["self_attn"][norm]["weight"] = block["self_attn"][norm]["weight"].float()
    inv_freq, valid, lam = inv_freq.to(DEV), valid.to(DEV), lam.to(DEV)
    static = dit.static_tables(inv_freq, valid, cfg, dtype)
    got = dit.self_attention(h, block, static, cfg, lam=lam, projections="hip")
    unfused = dit.self_attention(h, block, static, cfg, lam=lam, projections="torch")
    xcfg = dataclasses.replace(cfg, attention="xla")
    ref = dit.self_attention(h, block, dit.static_tables(inv_freq, valid, xcfg, dtype), xcfg, lam=lam)
    assert_bf16_parity(got.float().cpu().numpy(), unfused.float().cpu().numpy(), f"hip vs torch projections {dtype}")
    assert_bf16_parity(got.float().cpu().numpy(), ref.float().cpu().numpy(), f"hip projections vs xla {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_same_l_attention_hip_vs_xla(dtype):
    print(f"\n[case] same_l.attention hip vs xla {dtype}", flush=True)
    cfg = MEDIUM_SAME_L
    rng = np.random.default_rng(9)
    S, E = 1500, cfg.dim
    x = torch.from_numpy(rng.standard_normal((1, S, E)).astype(np.float32)).to(DEV, dtype)
    w = lambda *s: torch.from_numpy((rng.standard_normal(s) / np.sqrt(E)).astype(np.float32)).to(DEV, dtype)  # noqa: E731
    dyt = lambda: {"alpha": torch.tensor(0.5, device=DEV), "gamma": torch.from_numpy(  # noqa: E731
        (1 + 0.02 * rng.standard_normal(64)).astype(np.float32)).to(DEV),
        "beta": torch.from_numpy((0.02 * rng.standard_normal(64)).astype(np.float32)).to(DEV)}
    block = {"self_attn": {"to_qkv": {"weight": w(5 * E, E)}, "to_out": {"weight": w(E, E)}, "q_norm": dyt(),
                           "k_norm": dyt()}, "rope_inv_freq": torch.from_numpy(workloads.inv_freq(16)).to(DEV)}
    lam = torch.from_numpy(rng.uniform(0.2, 0.8, cfg.num_heads).astype(np.float32)).to(DEV)
    got = same_l.attention(x, block, cfg, lam=lam)
    ref = same_l.attention(x, block, dataclasses.replace(cfg, attention="xla"), lam=lam)
    check = assert_fp32_parity if dtype == torch.float32 else assert_bf16_parity
    check(got.float().cpu().numpy(), ref.float().cpu().numpy(), f"same_l {dtype}")
