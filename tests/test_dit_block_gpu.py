"""The DiT block's fused elementwise kernels on the GPU (reference: sa3jax/dit.py:44-57, 224-251): hb_rms_modulate
and hb_gated_residual against the oracle's chain of the same steps (oracle.dit: rms, add, mul, sigmoid, each rounded
to the compute dtype) and against the torch ops of the mirror, in bf16, half and fp32.

Contract: fp32 within 2e-6 relative to the row's scale; bf16 and half within one rounding step of the oracle on every
element (two steps after the adaLN modulation, which carries a step of the norm through x (1 + scale) and the
shift), the step taken at the larger of the result and the operands of a final sum that can cancel (shift,
residual), and equal on at least 99.5 % (the fp32 mean of squares and the fp32 sigmoid may differ from the oracle's exactly
rounded ones in the last fp32 bit, which moves a rounded intermediate by one step when it sits on a tie).
The whole block with these kernels is covered by tests/test_sampler_gpu.py (attention="hip" against "xla" and
the oracle).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hummingbird_amd import elementwise as ew
from hummingbird_amd import xla_chain
from oracle import dit as odit

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = {"bf16": (torch.bfloat16, 8), "fp16": (torch.float16, 11), "fp32": (torch.float32, 24)}


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def check(got: torch.Tensor, ref: np.ndarray, name: str, what: str, operands: np.ndarray | None = None,
          steps: int = 1) -> None:
    """`operands`: the magnitude of the last step's operands where it can cancel (the step is taken at the larger of
    that and the result: one step of an operand survives a cancelling sum). `steps`: steps allowed."""
    got = got.float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.isfinite(got).all(), what
    if name == "fp32":
        scale = np.maximum(np.abs(ref).max(axis=-1, keepdims=True), 1e-30)
        assert (np.abs(got - ref) <= 2e-6 * scale).all(), f"{what}: {np.abs(got - ref).max()}"
        return
    bits = DTYPES[name][1]
    mag = np.maximum(np.abs(ref), np.abs(got))
    if operands is not None:
        mag = np.maximum(mag, np.abs(operands))
    step = steps * np.ldexp(1.0, np.frexp(mag)[1] - bits)
    diff = np.abs(got - ref)
    worst = np.unravel_index(np.argmax(diff / step), diff.shape)
    assert (diff <= step).all(), (f"{what}: {int((diff > step).sum())} elements beyond {steps} step(s); worst at "
                                  f"{worst}: got {got[worst]}, ref {ref[worst]}, allowed {step[worst]}")
    assert (diff == 0).mean() >= 0.995, f"{what}: only {(diff == 0).mean():.4f} equal"


def rand(shape, gen, dtype, std=1.0, mean=0.0):
    return (mean + std * torch.randn(shape, device=DEV, generator=gen)).to(dtype)


@pytest.mark.parametrize("name", list(DTYPES))
@pytest.mark.parametrize("B,L,C,modulate", [(2, 37, 64, True), (1, 1422, 1536, True), (2, 300, 1536, False),
                                            (3, 5, 256, True)])
def test_rms_modulate_vs_oracle(name, B, L, C, modulate):
    announce(f"rms_modulate {name} B={B} L={L} C={C} modulate={modulate}")
    dtype = DTYPES[name][0]
    gen = torch.Generator(device=DEV).manual_seed(B * L + C)
    x = rand((B, L, C), gen, dtype, std=2.0)
    w = 1 + 0.1 * torch.randn(C, device=DEV, generator=gen)
    ssg = rand((B, 6 * C), gen, dtype, std=0.3)  # the adaLN row: scale and shift are views into it
    scale, shift = (ssg[:, :C], ssg[:, C:2 * C]) if modulate else (None, None)
    got = ew.rms_modulate(x, w, 1e-5, scale, shift)
    comp = "fp16" if name == "fp16" else name
    xs = x.float().cpu().numpy()
    ref = odit.rms(xs, w.cpu().numpy(), 1e-5, comp)
    operands = None
    if modulate:
        s = ssg[:, :C].float().cpu().numpy()[:, None, :]
        t = ssg[:, C:2 * C].float().cpu().numpy()[:, None, :]
        prod = odit.mul(ref, odit.add(1.0, s, comp), comp)
        operands = np.maximum(np.abs(prod), np.abs(t))  # the shift can cancel the product
        ref = odit.add(prod, t, comp)
    # a tie-rounding step of the norm survives x (1 + scale) (at most 2x) and the shift: two operand steps
    check(got, ref, name, "rms_modulate vs oracle", operands, steps=2 if modulate else 1)
    mirror = xla_chain.rms(x, w, 1e-5)
    if modulate:
        mirror = mirror * (1 + ssg[:, None, :C]) + ssg[:, None, C:2 * C]
    check(got, mirror.float().cpu().numpy(), name, "rms_modulate vs torch ops", operands, steps=2 if modulate else 1)


@pytest.mark.parametrize("name", list(DTYPES))
@pytest.mark.parametrize("B,L,C,mode", [(2, 37, 64, "gate"), (1, 1422, 1536, "gate_bias"), (2, 300, 1536, "local"),
                                        (3, 70, 256, "plain")])
def test_gated_residual_vs_oracle(name, B, L, C, mode):
    announce(f"gated_residual {name} B={B} L={L} C={C} {mode}")
    dtype = DTYPES[name][0]
    comp = name
    gen = torch.Generator(device=DEV).manual_seed(7 * B * L + C)
    h = rand((B, L, C), gen, dtype, std=3.0)
    x = rand((B, L, C), gen, dtype)
    ssg = rand((B, 6 * C), gen, dtype, std=1.5)
    gate = ssg[:, 2 * C:3 * C] if mode.startswith("gate") else None
    xb = rand((C,), gen, dtype, std=0.1) if mode == "gate_bias" else None
    local = rand((C,), gen, dtype, std=0.5) if mode == "local" else None
    memory = 16 if mode == "local" else 0
    got = ew.gated_residual(h, x, gate=gate, x_bias=xb, local=local, memory=memory)
    hn, xn = h.float().cpu().numpy(), x.float().cpu().numpy()
    if xb is not None:
        xn = odit.add(xn, xb.float().cpu().numpy(), comp)
    if gate is not None:
        g = gate.float().cpu().numpy()[:, None, :]
        xn = odit.mul(xn, odit.sigmoid(odit.add(1.0, -g, comp), comp), comp)
    ref = odit.add(hn, xn, comp)
    operands = np.maximum(np.abs(hn), np.abs(xn))  # the residual sum can cancel
    if local is not None:
        operands[:, memory:] = np.maximum(np.abs(ref[:, memory:]), np.abs(local.float().cpu().numpy()))
        ref[:, memory:] = odit.add(ref[:, memory:], local.float().cpu().numpy(), comp)
    check(got, ref, name, "gated_residual vs oracle", operands)
    mirror = x if xb is None else x + xb
    if gate is not None:
        mirror = mirror * torch.sigmoid(1 - gate[:, None, :])
    mirror = h + mirror
    if local is not None:
        mirror = torch.cat([mirror[:, :memory], mirror[:, memory:] + local], dim=1)
    check(got, mirror.float().cpu().numpy(), name, "gated_residual vs torch ops", operands)


@pytest.mark.parametrize("name", list(DTYPES))
@pytest.mark.parametrize("B,L,C,mode", [(2, 37, 64, "gate"), (1, 1422, 1536, "gate_bias_mod"),
                                        (2, 300, 1536, "local_mod"), (3, 70, 1024, "plain")])
def test_residual_rms_equals_the_two_kernels(name, B, L, C, mode):
    """hb_residual_rms against hb_gated_residual followed by hb_rms_modulate on the same inputs: bit-identical (the
    same roundings, the mean of squares in the same order); both of those are held to the oracle above."""
    announce(f"residual_rms {name} B={B} L={L} C={C} {mode}")
    dtype = DTYPES[name][0]
    gen = torch.Generator(device=DEV).manual_seed(3 * B * L + C)
    h = rand((B, L, C), gen, dtype, std=3.0)
    x = rand((B, L, C), gen, dtype)
    ssg = rand((B, 6 * C), gen, dtype, std=0.5)
    w = 1 + 0.1 * torch.randn(C, device=DEV, generator=gen)
    gate = ssg[:, 2 * C:3 * C] if mode.startswith("gate") else None
    xb = rand((C,), gen, dtype, std=0.1) if "bias" in mode else None
    local = rand((C,), gen, dtype, std=0.5) if mode.startswith("local") else None
    memory = 16 if local is not None else 0
    scale, shift = (ssg[:, :C], ssg[:, C:2 * C]) if mode.endswith("mod") else (None, None)
    got_h, got_y = ew.residual_rms(h, x, w, 1e-5, gate=gate, x_bias=xb, local=local, memory=memory, scale=scale,
                                   shift=shift)
    ref_h = ew.gated_residual(h, x, gate=gate, x_bias=xb, local=local, memory=memory)
    ref_y = ew.rms_modulate(ref_h, w, 1e-5, scale, shift)
    assert torch.equal(got_h, ref_h), "residual differs"
    assert torch.equal(got_y, ref_y), f"norm differs: {(got_y != ref_y).sum().item()} elements"
