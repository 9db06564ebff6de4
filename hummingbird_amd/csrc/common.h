// Shared device helpers for the gfx950 differential-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hb {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

// bf16 <-> fp32. The float -> bf16 conversion rounds to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }
__device__ __forceinline__ float round_bf16(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v;
  v[0] = static_cast<__bf16>(lo);
  v[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, v);
}

// Element type of qkv and out (the compute dtype of the reference's bf16 and fp16 presets, sa3jax/dtypes.py:40-58).
// The attention operands themselves (K, q * scale, P, V) are bf16 under both, as in the reference's fused kernels
// (dense_attention.py:75-77, 83, 90; band_attention.py:85, 94, 101); the type sets how inputs are read, where the
// compute-dtype casts of the norms round (dense_attention.py:66, 69) and how the output is written.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct Bf16Io {
  __device__ static __forceinline__ void unpack8(u32x4 v, float (&x)[8]);
  __device__ static __forceinline__ float round(float f);
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi);
  // 8 input elements as 8 bf16 (the fused kernels' `.astype(bf16)` of V)
  __device__ static __forceinline__ u32x4 to_bf16x8(u32x4 v) { return v; }
};

struct F16Io {
  // The whole 16 bytes are reinterpreted at once: hipcc miscompiles __builtin_bit_cast of a single element v[i] of
  // an ext_vector (every i read element 0).
  __device__ static __forceinline__ void unpack8(u32x4 v, float (&x)[8]) {
    const f16x8 h = __builtin_bit_cast(f16x8, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(h[i]);
  }
  // IEEE half round to nearest even (v_cvt_f16_f32 in the default rounding mode) of an fp32 value. The empty asm
  // makes the fp32 value exist before the conversion: otherwise the compiler may fold the multiply or subtract
  // that produced it into a mixed-precision FMA (v_fma_mixlo_f16), which rounds the exact result to half once,
  // where the source (and the reference's fp32 arithmetic followed by a cast) rounds to fp32 first. The two differ
  // by one half step when the fp32 result lies exactly on a half-precision tie.
  __device__ static __forceinline__ float round(float f) {
    asm volatile("" : "+v"(f));
    return static_cast<float>(static_cast<_Float16>(f));
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    asm volatile("" : "+v"(lo), "+v"(hi));
    f16x2 h;
    h[0] = static_cast<_Float16>(lo);
    h[1] = static_cast<_Float16>(hi);
    return __builtin_bit_cast(uint32_t, h);
  }
  __device__ static __forceinline__ u32x4 to_bf16x8(u32x4 v);
};

// 16-byte global load / store of 8 bf16.
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

__device__ __forceinline__ void unpack8(u32x4 v, float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(v[i] << 16);
    x[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ u32x4 pack8(const float (&x)[8]) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
  return v;
}

__device__ __forceinline__ void Bf16Io::unpack8(u32x4 v, float (&x)[8]) { hb::unpack8(v, x); }
__device__ __forceinline__ float Bf16Io::round(float f) { return round_bf16(f); }
__device__ __forceinline__ uint32_t Bf16Io::pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
__device__ __forceinline__ u32x4 F16Io::to_bf16x8(u32x4 v) {
  float x[8];
  unpack8(v, x);  // exact: every half is a float
  return pack8(x);
}

__device__ __forceinline__ f32x16 mfma_bf16_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_f16_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}
// The 32x32x16 product of 16-bit operands stored in the IO type's own format (bf16 or half), fp32 accumulation.
template <class IO>
__device__ __forceinline__ f32x16 mfma_io_32x32x16(u32x4 a, u32x4 b, f32x16 c);
template <>
__device__ __forceinline__ f32x16 mfma_io_32x32x16<Bf16Io>(u32x4 a, u32x4 b, f32x16 c) {
  return mfma_bf16_32x32x16(a, b, c);
}
template <>
__device__ __forceinline__ f32x16 mfma_io_32x32x16<F16Io>(u32x4 a, u32x4 b, f32x16 c) {
  return mfma_f16_32x32x16(a, b, c);
}
__device__ __forceinline__ f32x16 mfma_f32_32x32x2(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Sum of the two bf16 halves of `p` added to `acc` in fp32 (v_dot2_f32_bf16 against (1, 1)).
__device__ __forceinline__ float add_bf16_pair(uint32_t p, float acc) {
  const uint32_t ones = 0x3f803f80u;
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p), __builtin_bit_cast(bf16x2, ones), acc,
                                         false);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// A zero the compiler cannot see through. Adding it to an address inside a loop keeps loop-invariant loads
// in the loop (where their registers are short-lived) instead of hoisted and held across the whole loop.
__device__ __forceinline__ int opaque_zero() {
  int z;
  asm volatile("s_mov_b32 %0, 0" : "=s"(z));
  return z;
}

// Index of this wave inside the workgroup as a scalar: branches on it become scalar branches instead of
// exec-masked diamonds (the compiler cannot prove threadIdx.x / 64 uniform on its own).
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// The two 8-dim groups of RoPE pair p of a head (rotate_half over the first 2*half dims, half % 8 == 0).
// With h8 = half / 8 rotary pairs, pair p < h8 couples groups p and p + h8 (dims d and d + half, which
// rotate_half mixes); the remaining groups are not rotated and are paired in order. A thread that owns one pair
// therefore has each rotation partner in its own registers.
__device__ __forceinline__ void pair_groups(int p, int h8, int& m1, int& m2) {
  if (p < h8) {
    m1 = p;
    m2 = p + h8;
  } else {
    m1 = 2 * h8 + 2 * (p - h8);
    m2 = m1 + 1;
  }
}

// DyT(x) = gamma * tanh(alpha x) + beta (sa3jax/same_l.py:58-69) with tanh(y) = 1 - 2 / (1 + 2^(2 log2(e) y)):
// (gamma + beta) + (-2 gamma) / (1 + 2^(a2 x)), a2 = 2 log2(e) alpha, g2 = -2 gamma, gb = gamma + beta. Two
// transcendental instructions.
__device__ __forceinline__ float dyt_tanh(float x, float a2, float g2, float gb) {
  return __fmaf_rn(g2, __builtin_amdgcn_rcpf(1.f + fast_exp2(a2 * x)), gb);
}

// Bound on the norm of a DyT output row: |DyT(x)_d| <= |gamma_d| + |beta_d|, so |y| <= sqrt(sum_d (|gamma_d| +
// |beta_d|)^2) for `dyt` = [alpha, gamma[D], beta[D]]; reduced over the wave (every lane gets the value).
template <int D>
__device__ __forceinline__ float dyt_row_bound(const float* __restrict__ dyt) {
  const int lane = threadIdx.x & 63;
  float acc = 0.f;
  for (int d = lane; d < D; d += 64) {
    const float v = fabsf(dyt[1 + d]) + fabsf(dyt[1 + D + d]);
    acc = __fmaf_rn(v, v, acc);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, kWave);
  return sqrtf(acc);
}

// Workgroup index remap that keeps consecutive logical tiles on one XCD (its own L2). Hardware dispatches
// workgroup p to XCD p % 8; logical tile `start(x) + p / 8` is given to it, so each XCD walks a contiguous
// range of the logical order.
__device__ __forceinline__ int xcd_remap(int p, int n) {
  const int per = n >> 3, rem = n & 7, x = p & 7, idx = p >> 3;
  return x * per + (x < rem ? x : rem) + idx;
}

}  // namespace hb
