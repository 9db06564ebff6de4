"""Random SAME-L block parameters in the reference's layout, shared by the CPU and GPU block tests."""
from __future__ import annotations

import math

import numpy as np
import torch

from hummingbird_amd import workloads
from oracle.bf16 import cast


def block_params(dim: int, heads: int, ff: int, seed: int, zero_attn: bool = False, zero_ff: bool = False) -> dict:
    """Weights ~ N(0, 1/fan_in), biases ~ N(0, 0.02), DyT alpha 0.5, gamma ~ 1 + N(0, 0.02), beta ~ N(0, 0.02);
    `zero_attn` / `zero_ff` zero the output layer of that branch (which then adds nothing, or only its bias)."""
    rng = np.random.default_rng(seed)

    def w(o, i, zero=False):
        return np.zeros((o, i), np.float32) if zero else (rng.standard_normal((o, i)) / math.sqrt(i)).astype(np.float32)

    def b(o, zero=False):
        return np.zeros(o, np.float32) if zero else (0.02 * rng.standard_normal(o)).astype(np.float32)

    def dyt(c):
        return {"alpha": np.float32(0.5), "gamma": (1 + 0.02 * rng.standard_normal(c)).astype(np.float32),
                "beta": (0.02 * rng.standard_normal(c)).astype(np.float32)}
    d = heads * 64
    return {"pre_norm": dyt(dim), "ff_norm": dyt(dim), "rope_inv_freq": workloads.inv_freq(32),
            "self_attn": {"to_qkv": {"weight": w(5 * d, dim)}, "to_out": {"weight": w(dim, d, zero_attn)},
                          "q_norm": dyt(64), "k_norm": dyt(64)},
            "ff": {"glu_proj": {"weight": w(2 * ff, dim), "bias": b(2 * ff)},
                   "proj_out": {"weight": w(dim, ff, zero_ff), "bias": b(dim, zero_ff)}}}


def to_torch(p, device: str = "cpu", dtype: torch.dtype = torch.float32, key: str = ""):
    """The parameters as torch tensors on `device`: layer weights and biases in the compute dtype `dtype`,
    everything else (DyT parameters, RoPE frequencies) in fp32."""
    if isinstance(p, dict):
        return {k: to_torch(v, device, dtype, k) for k, v in p.items()}
    t = torch.as_tensor(np.asarray(p, np.float32)).to(device)
    return t.to(dtype) if key in ("weight", "bias") else t


def rounded(p, compute: str, key: str = ""):
    """The parameters as the oracle should see them for `compute`: layer weights and biases rounded to the compute
    dtype (the values the device holds), everything else unchanged."""
    if isinstance(p, dict):
        return {k: rounded(v, compute, k) for k, v in p.items()}
    return cast(np.asarray(p, np.float32), compute) if key in ("weight", "bias") else p
