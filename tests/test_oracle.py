"""Pins the NumPy oracle (CPU only).

Each oracle function is checked against something it does not share code with: a library routine (torch's
bf16 conversion, tanh and scaled_dot_product_attention in float64), a closed form (complex rotation for RoPE,
unit RMS), or an invariant (identical branches cancel, linearity in lambda, band = brute force). The
`test_planted_*` tests plant plausible mistakes in the oracle and check that the pins catch them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from hummingbird_amd import workloads
from oracle import band as oband
from oracle import bf16 as obf16
from oracle import dense as odense

RNG = np.random.default_rng(1234)


# ---- bf16 rounding --------------------------------------------------------------------------------------------
def test_round_bf16_matches_torch():
    x = np.concatenate([RNG.standard_normal(100000).astype(np.float32) * 10.0 ** RNG.integers(-30, 30, 100000),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3.0e38, 1e-40, np.inf, -np.inf],
                                 np.float32)]).astype(np.float32)
    ours = obf16.round_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours, ref)


def test_round_bf16_ties_to_even():
    # 1 + 2^-8 is halfway between 1 and 1 + 2^-7: ties go to the even mantissa (1.0)
    assert obf16.round_bf16(np.float32(1.0 + 2.0 ** -8)) == np.float32(1.0)
    assert obf16.round_bf16(np.float32(1.0 + 3 * 2.0 ** -8)) == np.float32(1.0 + 2.0 ** -6)


# ---- RMSNorm --------------------------------------------------------------------------------------------------
def test_rms_unit_rms_and_scale_invariance():
    x = RNG.standard_normal((50, 64)).astype(np.float32) * 3.0
    y = odense.rms(x, np.ones(64, np.float32), 0.0, "fp32")
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(-1)), 1.0, rtol=1e-6)
    np.testing.assert_allclose(odense.rms(7.5 * x, np.ones(64, np.float32), 0.0, "fp32"), y, rtol=2e-6, atol=1e-6)


def test_rms_weight_and_eps():
    x = RNG.standard_normal((8, 64)).astype(np.float32)
    w = RNG.uniform(0.5, 2.0, 64).astype(np.float32)
    np.testing.assert_allclose(odense.rms(x, w, 0.0, "fp32"), odense.rms(x, np.ones(64, np.float32), 0.0, "fp32") * w,
                               rtol=1e-6)
    tiny = x * 1e-6  # mean square 1e-12 << eps = 1: the norm divides by ~sqrt(eps) = 1
    np.testing.assert_allclose(odense.rms(tiny, w, 1.0, "fp32"), tiny * w, rtol=1e-5)


# ---- RoPE -----------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("half", [16, 32])
def test_rope_is_complex_rotation_of_pairs(half):
    length, d = 300, 64
    freq = workloads.inv_freq(half)
    cos, sin = odense.rope_tables(length, freq)
    x = RNG.standard_normal((2, length, d)).astype(np.float32)
    y = odense.rope(x, cos, sin, "fp32")
    theta = np.arange(length, dtype=np.float32)[:, None] * freq[None, :]  # fp32 angle, as the reference
    z = (x[..., :half] + 1j * x[..., half:2 * half]).astype(np.complex128) * np.exp(1j * theta.astype(np.float64))
    np.testing.assert_allclose(y[..., :half], z.real, rtol=0, atol=2e-6 * np.abs(x).max())
    np.testing.assert_allclose(y[..., half:2 * half], z.imag, rtol=0, atol=2e-6 * np.abs(x).max())
    assert np.array_equal(y[..., 2 * half:], x[..., 2 * half:])


def test_rope_identity_and_relative_position():
    x = RNG.standard_normal((40, 64)).astype(np.float32)
    cos, sin = odense.rope_tables(40, np.zeros(32, np.float32))
    assert np.array_equal(odense.rope(x, cos, sin, "fp32"), x)
    cos, sin = odense.rope_tables(200, workloads.inv_freq(32))
    q = RNG.standard_normal(64).astype(np.float32)
    k = RNG.standard_normal(64).astype(np.float32)
    dots = []
    for p in (0, 50, 120):  # rotate q at p + 7 and k at p: the dot product depends only on the offset 7
        qr = odense.rope(np.tile(q, (200, 1)), cos, sin, "fp32")[p + 7]
        kr = odense.rope(np.tile(k, (200, 1)), cos, sin, "fp32")[p]
        dots.append(float(qr.astype(np.float64) @ kr))
    np.testing.assert_allclose(dots, dots[0], rtol=1e-4)


def test_rope_tables_fp32_angle():
    freq = workloads.inv_freq(16)
    cos, sin = odense.rope_tables(5000, freq)
    ang = np.arange(5000, dtype=np.float32)[:, None] * freq[None, :]
    np.testing.assert_allclose(cos[:, :16], np.cos(ang.astype(np.float64)), atol=6e-8)
    assert np.array_equal(cos[:, :16], cos[:, 16:]) and np.array_equal(sin[:, :16], sin[:, 16:])


# ---- dense chain ----------------------------------------------------------------------------------------------
def _torch_dense(inp, lam):
    """Independent composition: the oracle's (separately pinned) norm/RoPE prep, then torch's SDPA in float64."""
    q, k, v, qd, kd = odense.prepare(inp["qkv"], inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"],
                                     inp["heads"], inp["head_dim"], inp["eps"], "fp32")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).double()  # noqa: E731
    a = F.scaled_dot_product_attention(t(q), t(k), t(v))
    b = F.scaled_dot_product_attention(t(qd), t(kd), t(v))
    out = a - torch.from_numpy(lam).double()[None, :, None, None] * b
    return odense.merge(out.numpy())


def test_dense_fp32_matches_torch_sdpa():
    inp = workloads.dense_inputs(2, 70, 3, 64, seed=3, dtype="fp32", half=16)
    ours = odense.dense_xla(inp["qkv"], inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"], 3, 64,
                            inp["eps"], inp["lam"], "fp32")
    np.testing.assert_allclose(ours, _torch_dense(inp, inp["lam"]), atol=2e-6, rtol=1e-5)


def test_dense_d128_fp32_matches_torch_sdpa():
    inp = workloads.dense_inputs(1, 40, 2, 128, seed=4, dtype="fp32")
    ours = odense.dense_xla(inp["qkv"], inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"], 2, 128,
                            inp["eps"], inp["lam"], "fp32")
    np.testing.assert_allclose(ours, _torch_dense(inp, inp["lam"]), atol=2e-6, rtol=1e-5)


def test_dense_special_cases():
    inp = workloads.dense_inputs(1, 30, 2, 64, seed=5, dtype="fp32", mask_tail=5)
    hd = 2 * 64
    qkv = inp["qkv"].copy()
    qkv[..., 0:hd] = 0.0  # q = 0: uniform weights over all 30 keys (the mask zeroes values, not keys)
    qkv[..., 3 * hd:4 * hd] = 0.0
    out = odense.dense_xla(qkv, inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"], 2, 64, 1e-6,
                           np.array([1.0, 0.25], np.float32), "fp32")
    v = qkv[0, :, 2 * hd:3 * hd] * inp["valid"][0][:, None]
    mean = v.mean(0)
    expect = np.concatenate([mean[:64] * 0.0, mean[64:] * 0.75])
    np.testing.assert_allclose(out[0], np.tile(expect, (30, 1)), atol=1e-6)
    one = workloads.dense_inputs(1, 1, 2, 64, seed=6, dtype="fp32", mask_tail=0)
    o1 = odense.dense_xla(one["qkv"], one["q_weight"], one["k_weight"], one["inv_freq"], None, 2, 64, 1e-6,
                          one["lam"], "fp32")
    v1 = one["qkv"][0, 0, 2 * hd:3 * hd]
    np.testing.assert_allclose(o1[0, 0], v1 * np.repeat(1.0 - one["lam"], 64), atol=1e-6)


def test_dense_identical_branches_and_linearity():
    inp = workloads.dense_inputs(1, 50, 2, 64, seed=7)
    qkv = inp["qkv"].copy()
    hd = 128
    qkv[..., 3 * hd:4 * hd], qkv[..., 4 * hd:5 * hd] = qkv[..., 0:hd], qkv[..., hd:2 * hd]
    args = (inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"], 2, 64, 1e-6)
    assert np.count_nonzero(odense.dense_xla(qkv, *args, None, "bf16")) == 0
    f = lambda lam: odense.dense_xla(inp["qkv"], *args, np.full(2, lam, np.float32), "fp32")  # noqa: E731
    np.testing.assert_allclose(f(0.3), 0.7 * f(0.0) + 0.3 * f(1.0), atol=1e-6)


def test_dense_query_rows_are_the_full_call_rows():
    """Restricting the chain to some query rows gives exactly those rows of the full call (each query sees every
    key either way) and zeros elsewhere."""
    inp = workloads.dense_inputs(2, 90, 2, 64, seed=9)
    args = (inp["qkv"], inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"], 2, 64, 1e-6, inp["lam"])
    full = odense.dense_xla(*args)
    rows = np.r_[0:7, 60:90]
    part = odense.dense_xla(*args, query_rows=rows)
    np.testing.assert_array_equal(part[:, rows], full[:, rows])
    assert np.count_nonzero(np.delete(part, rows, axis=1)) == 0


def test_dense_profiles_agree_within_contract():
    inp = workloads.dense_inputs(2, 120, 2, 64, seed=8)
    args = (inp["qkv"], inp["q_weight"], inp["k_weight"], inp["inv_freq"], inp["valid"], 2, 64, 1e-6, inp["lam"])
    a, b = odense.dense_xla(*args), odense.dense_fused(*args)
    assert np.abs(a - b).max() <= 2e-2


# ---- band chain -----------------------------------------------------------------------------------------------
def test_dyt_matches_torch_tanh_and_special_cases():
    x = RNG.standard_normal((10, 64)).astype(np.float32) * 4
    g = RNG.standard_normal(64).astype(np.float32)
    b = RNG.standard_normal(64).astype(np.float32)
    ref = (torch.from_numpy(g).double() * torch.tanh(0.7 * torch.from_numpy(x).double()) + torch.from_numpy(b).double())
    np.testing.assert_allclose(oband.dyt(x, 0.7, g, b), ref.numpy(), atol=1e-6 * np.abs(g).max() + 1e-6)
    np.testing.assert_allclose(oband.dyt(x, 0.0, g, b), np.broadcast_to(b, x.shape))
    np.testing.assert_allclose(oband.dyt(x, 0.7, np.zeros(64, np.float32), b), np.broadcast_to(b, x.shape))


@pytest.mark.parametrize("s,w", [(1, 3), (17, 17), (100, 0), (100, 1), (300, 17), (257, 64), (90, 200)])
def test_band_sdpa_matches_masked_torch_sdpa(s, w):
    q, k, v = (RNG.standard_normal((s, 64)).astype(np.float32) for _ in range(3))
    ours = oband.band_sdpa(q, k, v, w, block=37)
    pos = np.arange(s)
    mask = torch.from_numpy(np.abs(pos[None, :] - pos[:, None]) <= w)
    t = lambda a: torch.from_numpy(a).double()  # noqa: E731
    ref = F.scaled_dot_product_attention(t(q), t(k), t(v), attn_mask=mask).numpy()
    np.testing.assert_allclose(ours, ref, atol=2e-6)


@pytest.mark.parametrize("s,w", [(17 * 6, 17), (64 * 5, 64), (40, 1)])
def test_band_grouped_form_equals_brute_force(s, w):
    q, k, v = (RNG.standard_normal((s, 64)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(oband.band_grouped_sdpa(q, k, v, w), oband.band_sdpa(q, k, v, w), atol=2e-6)


def test_band_translation_equivariance_away_from_edges():
    s, w = 400, 20
    q, k, v = (RNG.standard_normal((s, 64)).astype(np.float32) for _ in range(3))
    full = oband.band_sdpa(q, k, v, w)
    shifted = oband.band_sdpa(q[100:], k[100:], v[100:], w)
    np.testing.assert_allclose(shifted[w:-w], full[100 + w:-w], atol=1e-6)


def test_band_chain_identical_branches_and_wide_window():
    inp = workloads.band_inputs(1, 120, 2, 64, 17, seed=9)
    qkv = inp["qkv"].copy()
    hd = 128
    qkv[..., 3 * hd:4 * hd], qkv[..., 4 * hd:5 * hd] = qkv[..., 0:hd], qkv[..., hd:2 * hd]
    n = inp["q_norm"]
    assert np.count_nonzero(oband.band_xla(qkv, n, n, inp["inv_freq"], 2, 64, 17)) == 0
    a = oband.band_xla(inp["qkv"], n, inp["k_norm"], inp["inv_freq"], 2, 64, 119, compute="fp32")
    b = oband.band_xla(inp["qkv"], n, inp["k_norm"], inp["inv_freq"], 2, 64, 10000, compute="fp32")
    assert np.array_equal(a, b)


def test_band_profiles_agree_within_contract():
    inp = workloads.band_inputs(1, 300, 2, 64, 64, seed=10)
    args = (inp["qkv"], inp["q_norm"], inp["k_norm"], inp["inv_freq"], 2, 64, 64, inp["lam"])
    assert np.abs(oband.band_xla(*args) - oband.band_fused(*args)).max() <= 2e-2


# ---- planted mistakes: each must be caught by one of the pins above -------------------------------------------
def test_planted_rope_sign_error_is_caught(monkeypatch):
    def wrong(x, cos, sin, compute):
        x32 = np.asarray(x, np.float32)
        rd = cos.shape[-1]
        rot, rest = x32[..., :rd], x32[..., rd:]
        rotated = np.concatenate([rot[..., rd // 2:], -rot[..., : rd // 2]], axis=-1)  # signs swapped
        return obf16.cast(np.concatenate([rot * cos + rotated * sin, rest], axis=-1), compute)
    monkeypatch.setattr(odense, "rope", wrong)
    with pytest.raises(AssertionError):
        test_rope_is_complex_rotation_of_pairs(16)


def test_planted_missing_scale_is_caught(monkeypatch):
    orig = odense.sdpa

    def wrong(q, k, v, compute, accum=np.float64):  # the 1/sqrt(D) factor dropped
        return orig(q * np.float32(8.0), k, v, compute, accum)
    monkeypatch.setattr(odense, "sdpa", wrong)
    with pytest.raises(AssertionError):
        test_dense_fp32_matches_torch_sdpa()


def test_planted_band_off_by_one_is_caught(monkeypatch):
    orig = oband.band_sdpa
    monkeypatch.setattr(oband, "band_sdpa", lambda q, k, v, window, block=512: orig(q, k, v, window + 1, block))
    with pytest.raises(AssertionError):
        test_band_sdpa_matches_masked_torch_sdpa(100, 1)


def test_planted_mask_on_keys_is_caught(monkeypatch):
    # A key mask (instead of zeroing values) changes the q = 0 special case: weights renormalise over 25 keys.
    orig = odense.sdpa

    def wrong(q, k, v, compute, accum=np.float64):
        keep = np.abs(v).sum(-1) > 0
        return orig(q, k[keep], v[keep], compute, accum)
    monkeypatch.setattr(odense, "sdpa", wrong)
    with pytest.raises(AssertionError):
        test_dense_special_cases()
