"""The SAME-L decoder block, restated in NumPy (oracle; test infrastructure only).

Follows the reference's XLA chain: sa3jax/same_l.py:186-192 (`_block`: two residual branches, each DyT in fp32
cast back to the compute dtype), 151-169 (`_attention`: to_qkv, band attention, to_out; the band attention itself
is `oracle.band.band_xla`), 172-183 (`_feed_forward`: glu_proj, value * act(gate), proj_out), 58-69 (`_dyt`) and
the `_linear` layers (a matmul in the compute dtype, then the bias added in it).

Cast points for bf16 (where the XLA chain holds a bf16 array): every GEMM output and bias add; the DyT output; in
the GLU the sigmoid, the SiLU product, pi itself (a Python float times a bf16 array takes bf16 in JAX), pi * gate,
the sine, and value * act; each residual add. Parity unpinned: how XLA evaluates a bf16 `logistic` or `sin`
internally is XLA's own behaviour (jax is not installed here); this restatement evaluates each elementwise
function in float64 and rounds its result once to the compute dtype.
"""
from __future__ import annotations

import math

import numpy as np

from oracle import band as oband
from oracle.bf16 import cast

F32 = np.float32


def dyt_cast(x: np.ndarray, norm: dict, compute: str) -> np.ndarray:
    """DyT in fp32 (same_l.py:58-69), cast back to the compute dtype (same_l.py:191-192)."""
    return cast(oband.dyt(x, norm["alpha"], norm["gamma"], norm["beta"]), compute)


def glu(proj: np.ndarray, sinusoidal: bool, compute: str) -> np.ndarray:
    """`value * act(gate)` for `[value | gate]` = the halves of the last axis (same_l.py:172-183)."""
    value, gate = np.split(np.asarray(proj, F32), 2, axis=-1)
    g = gate.astype(np.float64)
    if sinusoidal:
        t = cast(cast(np.array(math.pi, F32), compute).astype(np.float64) * g, compute)
        act = cast(np.sin(t.astype(np.float64)), compute)
    else:
        sig = cast(1.0 / (1.0 + np.exp(-g)), compute)
        act = cast(g * sig.astype(np.float64), compute)
    return cast(value.astype(np.float64) * act.astype(np.float64), compute)


def linear(x: np.ndarray, layer: dict, compute: str) -> np.ndarray:
    """`x @ W^T` accumulated in float64 and cast, then `+ b` cast (same_l._linear)."""
    y = cast(np.asarray(x, np.float64) @ np.asarray(layer["weight"], np.float64).T, compute)
    if layer.get("bias") is None:
        return y
    return cast(y.astype(np.float64) + np.asarray(layer["bias"], np.float64), compute)


def attention(x: np.ndarray, params: dict, num_heads: int, head_dim: int, window: int, lam, compute: str):
    """to_qkv -> band attention -> to_out (same_l.py:151-169)."""
    attn = params["self_attn"]
    qkv = linear(x, attn["to_qkv"], compute)
    out = oband.band_xla(qkv, attn["q_norm"], attn["k_norm"], params["rope_inv_freq"], num_heads, head_dim, window,
                         lam, compute)
    return linear(out, attn["to_out"], compute)


def feed_forward(x: np.ndarray, params: dict, sinusoidal: bool, compute: str) -> np.ndarray:
    ff = params["ff"]
    return linear(glu(linear(x, ff["glu_proj"], compute), sinusoidal, compute), ff["proj_out"], compute)


def block_xla(x: np.ndarray, params: dict, num_heads: int, head_dim: int, window: int, sinusoidal: bool,
              lam=None, compute: str = "bf16") -> np.ndarray:
    """`h = x + attention(DyT(x))`, `out = h + feed_forward(DyT(h))` (same_l.py:186-192)."""
    x = cast(x, compute)
    h = cast(x.astype(np.float64) + attention(dyt_cast(x, params["pre_norm"], compute), params, num_heads, head_dim,
                                              window, lam, compute), compute)
    return cast(h.astype(np.float64) + feed_forward(dyt_cast(h, params["ff_norm"], compute), params, sinusoidal,
                                                    compute), compute)
