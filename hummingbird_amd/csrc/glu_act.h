// The GLU activation of same_l._feed_forward (sa3jax/same_l.py:172-183), shared by the elementwise GLU kernel and
// the GLU epilogue of the glu_proj GEMM so that both compute it with the same instructions.
#pragma once

#include <math.h>

#include "common.h"

namespace hb {

// How sin(t) is evaluated for the sine gate, by compute dtype. None of the device paths calls the math library, so
// a GEMM epilogue that inlines them keeps its accumulators in registers.
enum SineMode {
  kSineLibrary = 0,  // fp32: the library sine (any finite t)
  kSineBf16 = 1,     // bf16: Cody-Waite by 2 pi and the hardware sine; |t| > 2^16 reduced exactly from a table
  kSineHalf = 2,     // half: three-term Cody-Waite by pi and an odd polynomial (relative accuracy near the zeros)
};

// 2^e mod 2 pi for e = 9 .. 120, to double precision: every bf16 value above 2^16 is m 2^e with an integer
// m in [128, 256) and e in that range. Written by gen_sine_table.py (this directory) from pi to 120 digits.
__device__ constexpr double kPow2Mod2Pi[112] = {
    3.0619901184534952, 6.1239802369069904, 5.964775166634395, 5.646365026089203,
    5.009544744998821, 3.7359041828180546, 1.188623058456523, 2.377246116913046,
    4.754492233826092, 3.2257991604725964, 0.1684130137656059, 0.3368260275312118,
    0.6736520550624236, 1.3473041101248473, 2.6946082202496946, 5.389216440499389,
    4.495247573819193, 2.707309840458799, 5.414619680917598, 4.546054054655609,
    2.8089228021316304, 5.617845604263261, 4.952505901346936, 3.621826495514285,
    0.960467683848984, 1.920935367697968, 3.841870735395936, 1.400556163612285,
    2.80111232722457, 5.60222465444914, 4.921264001718693, 3.5593426962577985,
    0.8355000853360102, 1.6710001706720203, 3.3420003413440407, 0.4008153755084947,
    0.8016307510169894, 1.6032615020339789, 3.2065230040679578, 0.12986070095632937,
    0.25972140191265874, 0.5194428038253175, 1.038885607650635, 2.07777121530127,
    4.15554243060254, 2.0278995540254936, 4.055799108050987, 1.8284129089223877,
    3.6568258178447755, 1.030466328509965, 2.06093265701993, 4.12186531403986,
    1.9605453209001322, 3.9210906418002645, 1.5589959764209427, 3.1179919528418854,
    6.235983905683771, 6.188782504187955, 6.094379701196324, 5.905574095213061,
    5.527962883246536, 4.772740459313485, 3.262295611447383, 0.24140591571517903,
    0.48281183143035805, 0.9656236628607161, 1.9312473257214322, 3.8624946514428644,
    1.4418039957061426, 2.883607991412285, 5.76721598282457, 5.251246658469554,
    4.219308009759521, 2.1554307123394554, 4.310861424678911, 2.338537542178235,
    4.67707508435647, 3.0709648615333527, 6.141929723066705, 6.000674138953824,
    5.718162970728061, 5.153140634276536, 4.0230959613734845, 1.7630066155673831,
    3.5260132311347663, 0.7688411550899459, 1.5376823101798918, 3.0753646203597835,
    6.150729240719567, 6.018273174259547, 5.753361041339508, 5.223536775499429,
    4.1638882438192715, 2.0445911804589567, 4.089182360917913, 1.895179414656241,
    3.790358829312482, 1.297532351445378, 2.595064702890756, 5.190129405781512,
    4.097073504383439, 1.9109617015872908, 3.8219234031745817, 1.360661499169577,
    2.721322998339154, 5.442645996678308, 4.602106686177028, 2.9210280651744704,
    5.842056130348941, 5.4009269535182955, 4.518668599857005, 2.754151892534424,
};

// sin(t) for a bf16 value t with |t| > 2^16: t = m 2^e exactly, so t mod 2 pi = m (2^e mod 2 pi) mod 2 pi, with
// m (2^e mod 2 pi) < 1606 reduced by a two-term 2 pi in double, then the hardware sine of the remainder.
__device__ __forceinline__ float sin_bf16_large(float t) {
  if (!isfinite(t)) return __int_as_float(0x7fc00000);  // sin(inf) is NaN
  int ex;
  const float f = frexpf(fabsf(t), &ex);  // |t| = f 2^ex, f in [0.5, 1), ex in [17, 128]
  const double u = static_cast<double>(f * 256.f) * kPow2Mod2Pi[ex - 17];
  const double k = rint(u * 0.15915494309189535);  // 1 / (2 pi)
  double r = fma(-k, 6.283185307179586, u);        // 2 pi = 6.283185307179586 + 2.4492935982947064e-16
  r = fma(-k, 2.4492935982947064e-16, r);
  const float s = __builtin_amdgcn_sinf(static_cast<float>(r * 0.15915494309189535));  // argument in revolutions
  return t < 0.f ? -s : s;
}

// sin(t) for |t| <= 65504 (every finite half): k = rint(t / pi); t - k pi by a three-term Cody-Waite split of pi
// (P1 = 201 / 64 and P2 = 507 / 2^19 have few enough bits that k P1 and k P2 are exact for |k| < 2^15, and each
// subtraction is exact or rounds relative to its result), then the odd Taylor polynomial of degree 11 on
// [-pi/2, pi/2] (truncation error below 6e-8) and the sign (-1)^k.
__device__ __forceinline__ float sin_half_range(float t) {
  const float k = rintf(t * 0.31830988618379067f);
  float r = __fmaf_rn(-k, 3.140625f, t);
  r = __fmaf_rn(-k, 9.670257568359375e-4f, r);
  r = __fmaf_rn(-k, 6.2783295e-7f, r);
  const float r2 = r * r;
  float p = -2.5052108385441720e-8f;           // -1/11!
  p = __fmaf_rn(p, r2, 2.7557319223985893e-6f);  // 1/9!
  p = __fmaf_rn(p, r2, -1.9841269841269841e-4f); // -1/7!
  p = __fmaf_rn(p, r2, 8.3333333333333333e-3f);  // 1/5!
  p = __fmaf_rn(p, r2, -1.6666666666666667e-1f); // -1/3!
  const float s = __fmaf_rn(r * r2, p, r);
  return (static_cast<int>(k) & 1) ? -s : s;
}

// act(g) with the XLA chain's intermediate arrays held in the compute dtype (`round`): SiLU(g) = g * sigmoid(g)
// (jax.nn.silu), the sigmoid rounded before the product; or, with SINE, sin(pi * g) with pi taken in the compute
// dtype (a Python float times a bf16 array is a bf16 multiply in JAX) and the product rounded before the sine. The
// caller rounds the activation before multiplying it into the value.
// kSineBf16, |t| <= 2^16: Cody-Waite reduction of t by 2 pi = C1 + C2 (C1 = 6.28125 has 8 significant bits, so
// k * C1 is exact for |k| < 2^16), then the hardware sine (v_sin_f32, argument in revolutions) of the remainder,
// |rev| <= 1/2; its error is far inside the bf16 rounding of the result.
template <bool SINE, int MODE, class Round>
__device__ __forceinline__ float glu_act(float g, Round round) {
  if constexpr (SINE) {
    const float t = round(round(static_cast<float>(M_PI)) * g);
    if constexpr (MODE == kSineBf16) {
      constexpr float inv2pi = static_cast<float>(0.5 / M_PI);
      if (__builtin_expect(fabsf(t) > 65536.f, 0)) return sin_bf16_large(t);
      const float k = rintf(t * inv2pi);
      const float r = __fmaf_rn(-k, 1.9353071795864769e-3f, __fmaf_rn(-k, 6.28125f, t));
      return __builtin_amdgcn_sinf(r * inv2pi);
    } else if constexpr (MODE == kSineHalf) {
      return sin_half_range(t);
    } else {
      return sinf(t);
    }
  } else {
    return g * round(__builtin_amdgcn_rcpf(1.f + fast_exp2(-kLog2e * g)));
  }
}

}  // namespace hb
