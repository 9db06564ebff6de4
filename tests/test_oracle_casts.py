"""Known-case pins of the oracle's cast points (CPU only).

Each case is a tiny input built so that one rounding step changes the result, with the expected output derived
by hand for that input: the logits, weights and partial sums are written out for the case and every rounding is
done with torch's bf16 / fp16 conversion (a library routine, not the oracle's). The `test_planted_*` tests plant
each cast point's plausible mistake (the rounding dropped, or added where the reference keeps fp32) into the
oracle and check that one of these pins fails.

Cast points (where the reference rounds to the compute dtype on each chain):
  XLA dense chain (oracle.dense.dense_xla / sdpa): RMSNorm cast (dit.py:57), RoPE cast (dit.py:98), bf16 logits
  (dit.py:117), the scale multiply in bf16 (dit.py:117), bf16 weights (dit.py:118), bf16 P @ V (dit.py:119), bf16
  subtraction (dit.py:146).
  Fused dense kernel (oracle.dense.dense_fused / fused_attend): K rounded to bf16 (dense_attention.py:75-76), q *
  scale rounded to bf16 (87-90), bf16 P over the fp32 sum of the unrounded weights (80-83), fp32 subtraction with
  one cast (94).
  XLA band chain (oracle.band.band_xla): q and k stay fp32 after DyT and RoPE (same_l.py:65-69, 95-100), fp32
  softmax and P @ V, fp32 subtraction with one cast (same_l.py:144-148, 168-169).
  Fused band kernel (oracle.band.band_fused / fused_band_attend): q * scale and k rounded to bf16
  (band_attention.py:85, 104), bf16 P over the fp32 sum (99-101), V rounded to bf16 (94).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import band as oband
from oracle import bf16 as obf16
from oracle import dense as odense

F32 = np.float32


def bf(x: float) -> float:
    """Nearest bfloat16 of the float32 value of x (torch's conversion, ties to even)."""
    return float(torch.tensor(float(np.float32(x)), dtype=torch.float32).to(torch.bfloat16).float())


def fp16(x: float) -> float:
    """Nearest IEEE half of the float32 value of x (torch's conversion)."""
    return float(torch.tensor(float(np.float32(x)), dtype=torch.float32).to(torch.float16).float())


def f32(x: float) -> float:
    return float(np.float32(x))


def row(d: int, **entries) -> np.ndarray:
    """A length-d vector with the given entries (keys like e0=8.0), zero elsewhere."""
    v = np.zeros(d, F32)
    for k, val in entries.items():
        v[int(k[1:])] = val
    return v


# ---- fp16 emulation -------------------------------------------------------------------------------------------
def test_round_fp16_matches_torch():
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(100000).astype(F32) * F32(10.0) ** rng.integers(-9, 6, 100000),
                        np.array([0.0, -0.0, 65504.0, 65520.0, 1e6, 6e-8, 2.98e-8, 1 + 2 ** -11, np.inf],
                                 F32)]).astype(F32)
    ref = torch.from_numpy(x).to(torch.float16).float().numpy()
    with np.errstate(over="ignore"):
        assert np.array_equal(obf16.round_fp16(x), ref)
    assert obf16.cast(np.float32(1 + 2 ** -11), "fp16") == 1.0  # tie to even
    with np.errstate(over="ignore"):
        assert obf16.cast(np.float32(65520.0), "fp16") == np.inf  # overflow


# ---- XLA dense chain: sdpa -------------------------------------------------------------------------------------
def sdpa_case_logit():
    """One query, two keys, D = 64. q . k0 = 64.25 rounds to the bf16 logit 64 (a tie between 64 and 64.5, to
    even), scaled by 1/8 to 8; q . k1 = 0. Weights softmax(8, 0), rounded; v0 = 0, v1 = 1 in dim 0."""
    q = row(64, e0=8.0, e1=1.0)[None]
    k = np.stack([row(64, e0=8.0, e1=0.25), row(64)])
    v = np.stack([row(64), row(64, e0=1.0)])
    w1 = f32(math.exp(-8.0) / (1.0 + math.exp(-8.0)))
    return q, k, v, bf(bf(w1) * 1.0)


def test_sdpa_bf16_logits_known_case():
    q, k, v, expect = sdpa_case_logit()
    out = odense.sdpa(q, k, v, "bf16")
    assert out[0, 0] == expect
    assert expect != bf(f32(math.exp(-8.03125) / (1.0 + math.exp(-8.03125))))  # the unrounded logit differs


def test_sdpa_bf16_logits_d128_known_case():
    """At D = 64 the logit rounding and the scale multiply round one value twice by a power of two, which is one
    rounding; at D = 128 they differ. q = (1, 1), k0 = (60.5, 0.375): q . k0 = 60.875 rounds to the bf16 logit 61
    (a tie between 60.75 and 61, to even), times bf16(1/sqrt(128)) = 5.4043 -> 5.40625; unrounded, 60.875 times it
    is 5.3803 -> 5.375. k1 = 0; v = (0, 1) in dim 0."""
    q = row(128, e0=1.0, e1=1.0)[None]
    k = np.stack([row(128, e0=60.5, e1=0.375), row(128)])
    v = np.stack([row(128), row(128, e0=1.0)])
    sb = bf(1.0 / math.sqrt(128))
    scaled = bf(bf(60.875) * sb)
    assert bf(60.875) == 61.0 and scaled == 5.40625 and bf(60.875 * sb) == 5.375
    expect = bf(bf(f32(math.exp(-scaled) / (1.0 + math.exp(-scaled)))))
    assert odense.sdpa(q, k, v, "bf16")[0, 0] == expect
    assert expect != bf(bf(f32(math.exp(-5.375) / (1.0 + math.exp(-5.375)))))


def sdpa_case_weights():
    """Scaled logits (0.5, 0): w = (sigma(0.5), sigma(-0.5)) = (0.62246, 0.37754), rounded to (0.62109375,
    0.376953125). Dim 0: v = (1, -1) gives bf(0.62109375 - 0.376953125) = 0.244140625 (the unrounded weights would
    give bf(0.24492) = 0.2451171875). Dim 1: v = (1, bf(1/3)) gives the P @ V sum 0.74699..., rounded to
    0.74609375."""
    q = row(64, e0=2.0)[None]
    k = np.stack([row(64, e0=2.0), row(64)])
    third = bf(1.0 / 3.0)
    v = np.stack([row(64, e0=1.0, e1=1.0), row(64, e0=-1.0, e1=third)])
    w0, w1 = f32(1.0 / (1.0 + math.exp(-0.5))), f32(1.0 / (1.0 + math.exp(0.5)))
    return q, k, v, (bf(bf(w0) - bf(w1)), bf(bf(w0) + bf(w1) * third))


def test_sdpa_bf16_weights_and_pv_known_case():
    q, k, v, (e0, e1) = sdpa_case_weights()
    out = odense.sdpa(q, k, v, "bf16")
    assert (out[0, 0], out[0, 1]) == (e0, e1) == (0.244140625, 0.74609375)


def test_sdpa_scale_in_bf16_known_case():
    """D = 128: the scale 1/sqrt(128) = 0.0883883 is a bf16 value, 0.08837890625, before it multiplies the bf16
    logit (a Python float times a bf16 array is a bf16 multiply). The logit 113.5 times it is 10.0309 -> bf16
    10.0; times the exact scale, 10.0322 -> bf16 10.0625. Two keys: the second logit is 0; v = (0, 1) in dim 0."""
    q = row(128, e0=1.0)[None]
    k = np.stack([row(128, e0=113.5), row(128)])
    v = np.stack([row(128), row(128, e0=1.0)])
    scaled = bf(113.5 * bf(1.0 / math.sqrt(128)))
    assert scaled == 10.0 and bf(113.5 / math.sqrt(128)) == 10.0625
    expect = bf(bf(f32(math.exp(-scaled) / (1.0 + math.exp(-scaled)))))
    assert odense.sdpa(q, k, v, "bf16")[0, 0] == expect
    assert expect != bf(bf(f32(math.exp(-10.0625) / (1.0 + math.exp(-10.0625)))))


def test_sdpa_fp16_known_case():
    """The fp16 preset (dtypes.py:50-58) rounds at the same points to IEEE half. q = (32, 1); k0 = (32, 0.25): q . k0
    = 1024.25 -> fp16 1024 (spacing 1 there), scaled by 1/8 to 128; k1 = (32, 1): 1025, scaled 128.125. Weights
    (sigma(-0.125), sigma(0.125)) in fp16; v = identity rows. Unrounded logits would give sigma(-+0.09375)."""
    q = row(64, e0=32.0, e1=1.0)[None]
    k = np.stack([row(64, e0=32.0, e1=0.25), row(64, e0=32.0, e1=1.0)])
    v = np.stack([row(64, e0=1.0), row(64, e1=1.0)])
    out = odense.sdpa(q, k, v, "fp16")
    w0, w1 = f32(1.0 / (1.0 + math.exp(0.125))), f32(1.0 / (1.0 + math.exp(-0.125)))
    assert (out[0, 0], out[0, 1]) == (fp16(w0), fp16(w1))
    assert fp16(w0) != fp16(1.0 / (1.0 + math.exp(0.09375)))


# ---- XLA dense chain: norm, rope, subtraction (through dense_xla) ----------------------------------------------
def test_rms_bf16_cast_known_case():
    """x = (3, 4, 0...), D = 64: mean square 25/64, rsqrt 1.6; the normalised (4.8, 6.4) is rounded to bf16
    (4.8125, 6.40625) (dit.py:57)."""
    x = row(64, e0=3.0, e1=4.0)[None]
    y = odense.rms(x, np.ones(64, F32), 0.0, "bf16")
    assert (y[0, 0], y[0, 1]) == (bf(4.8), bf(6.4)) == (4.8125, 6.40625)
    assert np.count_nonzero(y[0, 2:]) == 0


def test_rope_bf16_cast_known_case():
    """Position 1 with inv_freq 1 rotates (1, 0) by one radian to (cos 1, sin 1) = (0.5403, 0.8415), rounded to
    bf16 (0.5390625, 0.83984375) (dit.py:98)."""
    cos, sin = odense.rope_tables(2, np.ones(1, F32))
    x = np.array([[1.0, 0.0, 5.0, 7.0], [1.0, 0.0, 5.0, 7.0]], F32)
    y = odense.rope(x, cos, sin, "bf16")
    assert tuple(y[1]) == (bf(math.cos(1.0)), bf(math.sin(1.0)), 5.0, 7.0) == (0.5390625, 0.83984375, 5.0, 7.0)
    assert tuple(y[0]) == (1.0, 0.0, 5.0, 7.0)


def dense_qkv(rows: list[dict], d: int = 64) -> np.ndarray:
    """(1, L, 5 d) qkv for one head from per-token dicts of section -> vector (q, k, v, qd, kd)."""
    out = np.zeros((1, len(rows), 5 * d), F32)
    for i, r in enumerate(rows):
        for s, name in enumerate(("q", "k", "v", "qd", "kd")):
            if name in r:
                out[0, i, s * d:(s + 1) * d] = r[name]
    return out


def subtraction_case():
    """Two tokens, one head, no RoPE, RMSNorm with unit gains and eps = 0, so each row 8 e_i stays 8 e_i.
    Branch 1: q = 8 e0, keys 8 e2 and 8 e3: logits 0, 0, weights (0.5, 0.5). Branch 2: q_d = 8 e0, keys 8 e0 and
    8 e1: scaled logits 8 and 0, weights (bf(sigma(8)), bf(sigma(-8))) = (1, 3.357e-4). v = (2^-9, 2) in dim 0.
    first = bf(0.5 * 2^-9 + 0.5 * 2) = 1; second = bf(2^-9 + 2 bf(sigma(-8))); out = bf(first - second) (dit.py:146).
    The first query is the only one checked."""
    e = lambda i: row(64, **{f"e{i}": 8.0})  # noqa: E731
    qkv = dense_qkv([dict(q=e(0), k=e(2), v=row(64, e0=2.0 ** -9), qd=e(0), kd=e(0)),
                     dict(q=e(0), k=e(3), v=row(64, e0=2.0), qd=e(0), kd=e(1))])
    s8 = f32(1.0 / (1.0 + math.exp(8.0)))
    first = bf(0.5 * 2.0 ** -9 + 0.5 * 2.0)
    second = bf(bf(1.0 - s8) * 2.0 ** -9 + bf(s8) * 2.0)
    return qkv, first, second


def run_dense_xla(qkv, compute="bf16", lam=None):
    return odense.dense_xla(qkv, np.ones(64, F32), np.ones(64, F32), np.zeros(0, F32), None, 1, 64, 0.0, lam, compute)


def test_dense_xla_subtraction_known_case():
    qkv, first, second = subtraction_case()
    assert first == 1.0
    out = run_dense_xla(qkv)
    assert out[0, 0, 0] == bf(first - second)
    assert bf(first - second) != f32(first - second)  # the difference itself is not a bf16 value


# ---- fused dense profile ----------------------------------------------------------------------------------------
def fused_case(wq0: float = 1.0, wk0: float = 1.0, compute: str = "fp32", lam=0.0):
    """Two tokens, one head, no RoPE, eps = 0. q = 8 wq0 e0 (scaled by 1/8 to wq0 e0); keys 8 wk0 e0 and 8 e1:
    logits (8 wq0 wk0, 0) with K and q*scale rounded to bf16 first. v0 = (1, 0), v1 = (0, 1). Branch 2 is
    switched off with lam = 0 unless given."""
    e = lambda i: row(64, **{f"e{i}": 8.0})  # noqa: E731
    qkv = dense_qkv([dict(q=e(0), k=e(0), v=row(64, e0=1.0), qd=e(5), kd=e(2)),
                     dict(q=e(0), k=e(1), v=row(64, e1=1.0), qd=e(5), kd=e(3))])
    qw, kw = np.ones(64, F32), np.ones(64, F32)
    qw[0], kw[0] = wq0, wk0
    return odense.dense_fused(qkv, qw, kw, np.zeros(0, F32), None, 1, 64, 0.0, np.array([lam], F32), compute)


def fused_expect(logit0: float) -> tuple[float, float]:
    """fused_attend for logits (l0, 0), l0 >= 0: w = (1, e^-l0) in fp32, P = bf16(w), divided by 1 + w1 (fp32 sum
    of the unrounded weights): dims 0 and 1 are 1 / (1 + w1) and bf(w1) / (1 + w1)."""
    w1 = f32(math.exp(-logit0))
    return f32(1.0 / (1.0 + w1)), f32(bf(w1) / (1.0 + w1))


def test_fused_dense_k_rounding_known_case():
    """k gain 1 + 2^-10: k0 = 8.0078125 in fp32 (FP32_PARITY compute), rounded to bf16 8.0 before the product
    (dense_attention.py:75-76): the logit is 8, not 8.0078125."""
    out = fused_case(wk0=1.0 + 2.0 ** -10)
    assert (out[0, 0, 0], out[0, 0, 1]) == fused_expect(8.0)
    assert fused_expect(8.0)[1] != fused_expect(8.0078125)[1]


def test_fused_dense_q_rounding_known_case():
    """q gain 1 + 2^-10: q * scale = 1.0009765625 rounded to bf16 1.0 (dense_attention.py:87-90)."""
    out = fused_case(wq0=1.0 + 2.0 ** -10)
    assert (out[0, 0, 0], out[0, 0, 1]) == fused_expect(8.0)


def test_fused_dense_p_rounding_and_fp32_denominator_known_case():
    """k gain 1/16: logits (0.5, 0), w = (1, e^-0.5 = 0.60653); P1 = bf16 0.60546875 in the numerator, the fp32
    1.60653 in the denominator (dense_attention.py:80-83)."""
    out = fused_case(wk0=1.0 / 16.0)
    e0, e1 = fused_expect(0.5)
    assert (out[0, 0, 0], out[0, 0, 1]) == (e0, e1)
    w1 = f32(math.exp(-0.5))
    assert e1 != f32(w1 / (1.0 + w1)) and e0 != f32(1.0 / (1.0 + bf(w1)))


# The fused kernel subtracts in fp32 and casts once (dense_attention.py:94); the XLA chain rounds each branch
# first. Branch 1 as in the P case (dim 1 = bf(w1) / (1 + w1) = 0.376879), branch 2 uniform over two keys (q_d =
# 8 e5 against keys 8 e2, 8 e3: weights 1, 1 -> dim 1 = 0.5); lam 0.5502 puts the exact difference just past a
# bf16 rounding boundary that the rounded branch result does not: 0.1015625 against 0.10205078125.
FUSED_LAM = 0.5502


def test_fused_dense_single_cast_known_case():
    a = fused_expect(0.5)[1]
    b = f32(0.5)
    expect = bf(f32(a - f32(FUSED_LAM) * b))
    out = fused_case(wk0=1.0 / 16.0, compute="bf16", lam=FUSED_LAM)
    assert out[0, 0, 1] == expect
    assert expect != bf(bf(a) - f32(FUSED_LAM) * b)


# ---- band chains --------------------------------------------------------------------------------------------------
def band_case(gq0: float = 1.0 + 2.0 ** -9, gk: float = 512.0):
    """S = 2, w = 1, one head, D = 64, no RoPE. DyT with alpha = 100 saturates tanh to +-1 (exact in fp32), so a
    row x gives gamma * sign(x) on its nonzero dims and beta = 0 elsewhere. q rows: x = (1, 1) with gamma_q =
    (gq0, 1): q = (gq0, 1). k0 = (gk, 0), k1 = (0, gk). Query 0 sees both keys: logits gq0 gk / 8 and gk / 8,
    i.e. 64.125 and 64 at the defaults. v0 = (1, 0), v1 = (0, 1). Branch 2 off (lam = 0)."""
    d = 64
    qkv = np.zeros((1, 2, 5 * d), F32)
    for t in range(2):
        qkv[0, t, 0:2] = 1.0          # q
        qkv[0, t, 3 * d:3 * d + 2] = 1.0  # q_diff (unused, lam = 0)
    qkv[0, 0, d + 0] = 1.0  # k0 = (gk, 0)
    qkv[0, 1, d + 1] = 1.0  # k1 = (0, gk)
    qkv[0, 0, 2 * d + 0] = 1.0  # v0
    qkv[0, 1, 2 * d + 1] = 1.0  # v1
    qkv[0, :, 4 * d:5 * d] = qkv[0, :, d:2 * d]
    gamma_q = row(d, e0=gq0, e1=1.0)
    gamma_k = row(d, e0=gk, e1=gk)
    qn = {"alpha": F32(100.0), "gamma": gamma_q, "beta": np.zeros(d, F32)}
    kn = {"alpha": F32(100.0), "gamma": gamma_k, "beta": np.zeros(d, F32)}
    return qkv, qn, kn


def test_band_xla_keeps_q_fp32_known_case():
    """The XLA band chain keeps DyT and RoPE outputs in fp32 (same_l.py:65-69, 95-100): q0 = 1 + 2^-9 is not a
    bf16 value, and the logits 64.125 and 64 give query 0 the weights (sigma(0.125), sigma(-0.125)); dims 0 and 1
    are those weights, cast to bf16 once at the end (same_l.py:168-169). A bf16 q would give (0.5, 0.5)."""
    qkv, qn, kn = band_case()
    out = oband.band_xla(qkv, qn, kn, np.zeros(0, F32), 1, 64, 1, np.zeros(1, F32), "bf16")
    s = 1.0 / (1.0 + math.exp(-0.125))
    assert (out[0, 0, 0], out[0, 0, 1]) == (bf(s), bf(1.0 - s)) == (0.53125, 0.46875)


def test_band_xla_fp32_branches_cast_once_known_case():
    """Same input, compute fp32 throughout, lam = 1 with branch 2 the same as branch 1: exact cancellation; with
    lam = 0.5 the output is half of branch 1 in fp32, no rounding of the branches."""
    qkv, qn, kn = band_case()
    s = f32(1.0 / (1.0 + math.exp(-0.125)))
    out = oband.band_xla(qkv, qn, kn, np.zeros(0, F32), 1, 64, 1, np.full(1, 0.5, F32), "fp32")
    assert abs(out[0, 0, 0] - 0.5 * s) <= 2e-7 and out[0, 0, 0] != bf(0.5 * s)
    assert np.count_nonzero(oband.band_xla(qkv, qn, kn, np.zeros(0, F32), 1, 64, 1, None, "bf16")) == 0


def test_band_fused_q_rounding_known_case():
    """The fused band kernel rounds q * scale to bf16 (band_attention.py:85, 104): (1 + 2^-9) / 8 -> 1/8, so both
    logits are 64 and query 0 weighs its two keys equally: (0.5, 0.5) exactly (compute fp32)."""
    qkv, qn, kn = band_case()
    out = oband.band_fused(qkv, qn, kn, np.zeros(0, F32), 1, 64, 1, np.zeros(1, F32), "fp32")
    assert (out[0, 0, 0], out[0, 0, 1]) == (0.5, 0.5)


def test_band_fused_k_rounding_and_p_known_case():
    """q exact (gq0 = 1), k gain 512 (1 + 2^-8 + 2^-9) = 514.5 -> bf16 514 for both keys: logits 64.25 and 64.25
    -> equal weights (0.5, 0.5). With gq0 = 1 + 2^-7 (a bf16 value) and k gain 512: logits 64.5 and 64 -> w =
    (1, e^-0.5); P = bf16 and the fp32 sum in the denominator (band_attention.py:99-101)."""
    qkv, qn, kn = band_case(gq0=1.0, gk=512.0 * (1.0 + 2.0 ** -8 + 2.0 ** -9))
    out = oband.band_fused(qkv, qn, kn, np.zeros(0, F32), 1, 64, 1, np.zeros(1, F32), "fp32")
    assert (out[0, 0, 0], out[0, 0, 1]) == (0.5, 0.5)
    qkv, qn, kn = band_case(gq0=1.0 + 2.0 ** -7, gk=512.0)
    out = oband.band_fused(qkv, qn, kn, np.zeros(0, F32), 1, 64, 1, np.zeros(1, F32), "fp32")
    assert (out[0, 0, 0], out[0, 0, 1]) == fused_expect(0.5)


def test_band_fused_v_rounding_known_case():
    """fp16 compute: v0 = 1 + 2^-9 is an fp16 value but not a bf16 one; the fused kernel rounds V to bf16
    (band_attention.py:94) before P @ V, the XLA chain does not (fp32(V), same_l.py:147)."""
    qkv, qn, kn = band_case(gq0=1.0, gk=512.0)
    qkv[0, 0, 2 * 64] = 1.0 + 2.0 ** -9
    fused = oband.band_fused(qkv, qn, kn, np.zeros(0, F32), 1, 64, 1, np.zeros(1, F32), "fp16")
    xla = oband.band_xla(qkv, qn, kn, np.zeros(0, F32), 1, 64, 1, np.zeros(1, F32), "fp16")
    assert fused[0, 0, 0] == fp16(0.5 * 1.0)                 # bf16(1 + 2^-9) = 1; equal weights
    assert xla[0, 0, 0] == fp16(0.5 * (1.0 + 2.0 ** -9))


# ---- planted mistakes -----------------------------------------------------------------------------------------------
def _sdpa_without(step: str):
    """oracle.dense.sdpa with one of its cast points dropped."""
    def sdpa(q, k, v, compute, accum=np.float64):
        c = (lambda x: x) if step == "all" else (lambda x: obf16.cast(x, compute))
        keep = lambda name, x: np.asarray(x, F32) if step == name else c(x)  # noqa: E731
        d = q.shape[-1]
        logits = keep("logits", q.astype(accum) @ k.astype(accum).T)
        logits = keep("scale", logits * (F32(1.0 / math.sqrt(d)) if step == "scale" else c(np.array(1.0 / math.sqrt(d), F32))))
        weights = keep("weights", odense.softmax(logits))
        return keep("pv", weights.astype(accum) @ v.astype(accum))
    return sdpa


@pytest.mark.parametrize("step,pin", [
    ("logits", test_sdpa_bf16_logits_d128_known_case),
    ("all", test_sdpa_bf16_logits_known_case),
    ("scale", test_sdpa_scale_in_bf16_known_case),
    ("weights", test_sdpa_bf16_weights_and_pv_known_case),
    ("pv", test_sdpa_bf16_weights_and_pv_known_case),
])
def test_planted_dropped_sdpa_cast_is_caught(monkeypatch, step, pin):
    monkeypatch.setattr(odense, "sdpa", _sdpa_without(step))
    with pytest.raises(AssertionError):
        pin()


def test_planted_dropped_norm_and_rope_casts_are_caught(monkeypatch):
    orig_rms, orig_rope = odense.rms, odense.rope
    monkeypatch.setattr(odense, "rms", lambda x, w, eps, compute: orig_rms(x, w, eps, "fp32"))
    with pytest.raises(AssertionError):
        test_rms_bf16_cast_known_case()
    monkeypatch.setattr(odense, "rms", orig_rms)
    monkeypatch.setattr(odense, "rope", lambda x, c, s, compute: orig_rope(x, c, s, "fp32"))
    with pytest.raises(AssertionError):
        test_rope_bf16_cast_known_case()


def test_planted_dropped_subtraction_cast_is_caught(monkeypatch):
    def dense_xla(qkv, qw, kw, inv_freq, valid, num_heads, head_dim, eps=1e-6, lam=None, compute="bf16", **kw_):
        q, k, v, qd, kd = odense.prepare(qkv, qw, kw, inv_freq, valid, num_heads, head_dim, eps, compute)
        first = odense.sdpa(q[0, 0], k[0, 0], v[0, 0], compute)
        second = odense.sdpa(qd[0, 0], kd[0, 0], v[0, 0], compute)
        return (first - second)[None]  # fp32 difference, no cast
    monkeypatch.setattr(odense, "dense_xla", dense_xla)
    with pytest.raises(AssertionError):
        test_dense_xla_subtraction_known_case()


def test_planted_fused_dense_mistakes_are_caught(monkeypatch):
    orig_cast = odense.cast
    # K (and q) not rounded to bf16 before the products: the fused profile keeps them in the compute dtype
    monkeypatch.setattr(odense, "cast", lambda x, c: orig_cast(x, "fp32") if c == "bf16" else orig_cast(x, c))
    with pytest.raises(AssertionError):
        test_fused_dense_k_rounding_known_case()
    with pytest.raises(AssertionError):
        test_fused_dense_q_rounding_known_case()
    monkeypatch.setattr(odense, "cast", orig_cast)

    def no_p_round(qq, kk, vv):
        logits = (qq.astype(np.float64) @ kk.astype(np.float64).T).astype(F32)
        w = np.exp(logits - logits.max(-1, keepdims=True)).astype(F32)
        return ((w.astype(np.float64) @ vv.astype(np.float64)) / w.sum(-1, keepdims=True, dtype=np.float64)).astype(F32)

    def bf16_denominator(qq, kk, vv):
        logits = (qq.astype(np.float64) @ kk.astype(np.float64).T).astype(F32)
        p = orig_cast(np.exp(logits - logits.max(-1, keepdims=True)).astype(F32), "bf16")
        return ((p.astype(np.float64) @ vv.astype(np.float64)) / p.sum(-1, keepdims=True, dtype=np.float64)).astype(F32)

    for planted in (no_p_round, bf16_denominator):
        monkeypatch.setattr(odense, "fused_attend", planted)
        with pytest.raises(AssertionError):
            test_fused_dense_p_rounding_and_fp32_denominator_known_case()


def test_planted_fused_dense_branch_rounding_is_caught(monkeypatch):
    orig = odense.fused_attend
    monkeypatch.setattr(odense, "fused_attend", lambda q, k, v: obf16.round_bf16(orig(q, k, v)))
    with pytest.raises(AssertionError):
        test_fused_dense_single_cast_known_case()


def test_planted_band_q_cast_is_caught(monkeypatch):
    orig_rope = oband.rope
    # q and k cast to the compute dtype after RoPE, as the dense chain does, instead of kept in fp32
    monkeypatch.setattr(oband, "rope", lambda x, c, s, compute: orig_rope(x, c, s, "bf16"))
    with pytest.raises(AssertionError):
        test_band_xla_keeps_q_fp32_known_case()


def test_planted_band_branch_rounding_is_caught(monkeypatch):
    orig = oband.band_sdpa
    monkeypatch.setattr(oband, "band_sdpa", lambda *a, **k: obf16.round_bf16(orig(*a, **k)))
    with pytest.raises(AssertionError):
        test_band_xla_fp32_branches_cast_once_known_case()


def test_planted_fused_band_mistakes_are_caught(monkeypatch):
    orig_cast = oband.cast
    monkeypatch.setattr(oband, "cast", lambda x, c: orig_cast(x, "fp32") if c == "bf16" else orig_cast(x, c))
    with pytest.raises(AssertionError):
        test_band_fused_q_rounding_known_case()
    with pytest.raises(AssertionError):
        test_band_fused_k_rounding_and_p_known_case()
    with pytest.raises(AssertionError):
        test_band_fused_v_rounding_known_case()
    monkeypatch.setattr(oband, "cast", orig_cast)
    orig = oband.fused_band_attend

    def bf16_denominator(qq, kk, vv, window, block=512):
        # the row sum taken over the rounded probabilities instead of the fp32 weights
        s = qq.shape[0]
        logits = (qq.astype(np.float64) @ kk.astype(np.float64).T).astype(F32)
        band = np.abs(np.arange(s)[None, :] - np.arange(s)[:, None]) <= window
        p = orig_cast(np.exp(np.where(band, logits, F32(-1e30)) - np.where(band, logits, F32(-1e30)).max(
            -1, keepdims=True)).astype(F32), "bf16")
        return ((p.astype(np.float64) @ vv.astype(np.float64)) / p.sum(-1, keepdims=True, dtype=np.float64)).astype(F32)
    del orig
    monkeypatch.setattr(oband, "fused_band_attend", bf16_denominator)
    with pytest.raises(AssertionError):
        test_band_fused_k_rounding_and_p_known_case()
