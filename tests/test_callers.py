"""The caller mirrors (dit.self_attention, same_l.attention, their dispatch predicates and per-clip tables) on
the CPU: the attention="xla" path against the oracle, with the projections either side (config 0: to_qkv ->
differential self-attention -> to_out at L=216, fp32). Reference: sa3jax/dit.py:179-200, 317-336;
sa3jax/same_l.py:151-169."""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from hummingbird_amd import dit, same_l, workloads
from hummingbird_amd.config import MEDIUM_DIT, DiTConfig, SameConfig
from oracle import band as oband
from oracle import dense as odense
from tests.util import assert_fp32_parity


def dit_block(cfg: DiTConfig, seed: int) -> tuple[dict, torch.Tensor]:
    """Config-0 style weights: W ~ N(0, 1/E), RMSNorm gains ~ 1 + N(0, 0.02), per-head lambda ~ U(0.2, 0.8)."""
    rng = np.random.default_rng(seed)
    E = cfg.embed_dim
    w = lambda *s: torch.from_numpy((rng.standard_normal(s) / np.sqrt(E)).astype(np.float32))  # noqa: E731
    g = lambda: torch.from_numpy((1 + 0.02 * rng.standard_normal(cfg.head_dim)).astype(np.float32))  # noqa: E731
    block = {"self_attn": {"to_qkv": {"weight": w(5 * E, E)}, "to_out": {"weight": w(E, E)},
                           "q_norm": {"weight": g()}, "k_norm": {"weight": g()}}}
    lam = torch.from_numpy(rng.uniform(0.2, 0.8, cfg.num_heads).astype(np.float32))
    return block, lam


def dit_case(cfg: DiTConfig, batch: int, tokens: int, seed: int = 0):
    rng = np.random.default_rng(seed + 100)
    length = cfg.num_memory_tokens + tokens
    h = torch.from_numpy(rng.standard_normal((batch, length, cfg.embed_dim)).astype(np.float32))
    valid = torch.ones((batch, tokens), dtype=torch.bool)
    valid[:, tokens - 16:] = False  # the last 16 latents are padding
    inv_freq = torch.from_numpy(workloads.inv_freq(cfg.rope_dim // 2))
    block, lam = dit_block(cfg, seed)
    return h, valid, inv_freq, block, lam


def test_dit_dispatch_predicate():
    x = torch.zeros(1, 4, 5 * 64)
    assert not dit.use_hip(DiTConfig(attention="xla", differential=True), x)
    assert not dit.use_hip(DiTConfig(attention="fused", differential=True), x)
    assert not dit.use_hip(DiTConfig(attention="hip", differential=False), x)
    with pytest.raises(ValueError):  # no silent fallback for CPU tensors
        dit.use_hip(DiTConfig(attention="hip", differential=True), x)


def test_same_l_dispatch_predicate():
    x = torch.zeros(1, 4, 5 * 64)
    assert not same_l.use_hip(SameConfig(attention="xla"), x)
    assert not same_l.use_hip(SameConfig(attention="pallas"), x)
    with pytest.raises(ValueError):
        same_l.use_hip(SameConfig(attention="hip"), x)


def test_dit_static_tables_prepend_memory_tokens():
    cfg = DiTConfig(embed_dim=128, num_heads=2, differential=True)
    valid = torch.tensor([[1, 1, 0], [1, 0, 0]], dtype=torch.bool)
    st = dit.static_tables(torch.ones(16), valid, cfg, torch.float32)
    assert st["valid"].shape == (2, cfg.num_memory_tokens + 3)
    assert bool(st["valid"][:, : cfg.num_memory_tokens].all())
    assert torch.equal(st["valid"][:, cfg.num_memory_tokens:], valid)
    assert "hip_cos" not in st  # the kernel-native tables are built only for attention="hip"


def test_dit_self_attention_config0_matches_oracle():
    """Config 0: B=1, L=216 (64 memory tokens + 152 latents, the last 16 masked), 24 heads of 64, partial rotary
    (rope_dim 32, half 16), fp32: to_qkv -> differential attention -> to_out against the oracle's XLA chain."""
    cfg = dataclasses.replace(MEDIUM_DIT, attention="xla")
    h, valid, inv_freq, block, lam = dit_case(cfg, 1, 216 - cfg.num_memory_tokens)
    st = dit.static_tables(inv_freq, valid, cfg, torch.float32)
    got = dit.self_attention(h, block, st, cfg, lam=lam).numpy()
    attn = block["self_attn"]
    qkv = (h @ attn["to_qkv"]["weight"].t()).numpy()
    core = odense.dense_xla(qkv, attn["q_norm"]["weight"].numpy(), attn["k_norm"]["weight"].numpy(),
                            inv_freq.numpy(), st["valid"].numpy().astype(np.float32), cfg.num_heads, cfg.head_dim,
                            cfg.qk_norm_eps, lam.numpy(), "fp32")
    ref = core @ attn["to_out"]["weight"].numpy().T
    assert_fp32_parity(got, ref, "config 0 self-attention")


def test_same_l_attention_matches_oracle():
    """A small SAME-L block (dim 128 = 2 heads of 64, half-width 17 = stride + 1), fp32, against the oracle."""
    cfg = SameConfig(channels=64, c_mults=(2,), stride=16, attention="xla")
    rng = np.random.default_rng(5)
    S, E = 300, cfg.dim
    x = torch.from_numpy(rng.standard_normal((1, S, E)).astype(np.float32))
    w = lambda *s: torch.from_numpy((rng.standard_normal(s) / np.sqrt(E)).astype(np.float32))  # noqa: E731
    dyt = lambda: {"alpha": torch.tensor(0.5), "gamma": torch.from_numpy(  # noqa: E731
        (1 + 0.02 * rng.standard_normal(64)).astype(np.float32)),
        "beta": torch.from_numpy((0.02 * rng.standard_normal(64)).astype(np.float32))}
    block = {"self_attn": {"to_qkv": {"weight": w(5 * E, E)}, "to_out": {"weight": w(E, E)}, "q_norm": dyt(),
                           "k_norm": dyt()}, "rope_inv_freq": torch.from_numpy(workloads.inv_freq(16))}
    lam = torch.from_numpy(rng.uniform(0.2, 0.8, cfg.num_heads).astype(np.float32))
    got = same_l.attention(x, block, cfg, lam=lam).numpy()
    attn = block["self_attn"]
    qkv = (x @ attn["to_qkv"]["weight"].t()).numpy()
    norm = lambda n: {k: np.asarray(v) for k, v in n.items()}  # noqa: E731
    core = oband.band_xla(qkv, norm(attn["q_norm"]), norm(attn["k_norm"]), block["rope_inv_freq"].numpy(),
                          cfg.num_heads, cfg.dim_heads, cfg.sub_chunk_size, lam.numpy(), "fp32")
    ref = core @ attn["to_out"]["weight"].numpy().T
    assert_fp32_parity(got, ref, "SAME-L attention")
