// One 64-key step of the two-branch differential attention, shared by the dense and band kernels.
//
// Per wave: 32 queries (MFMA columns) against 64 keys (two 32-row MFMA tiles), both branches.
//   S^T[key][query] = K Q^T        v_mfma_f32_32x32x16_bf16, A = K rows from LDS, B = Q held in registers
//   P = exp2(S^T) or exp2(S^T c - m)   see SoftmaxPlan
//   O^T[d][query] += V^T P^T       A = V^T rows from LDS, B = P straight from the S^T accumulators
// The C layout of a 32x32 MFMA gives lane l the column l % 32 and, in register r, the row
// 8*(r/4) + 4*(l/32) + r%4. Row sums therefore stay lane-local; the two lane halves hold different keys of the
// same query and are combined once at the end.
#pragma once

#include "common.h"

namespace hb {

__device__ __forceinline__ u32x4 lds16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Key (relative to the tile start) held by accumulator register r of row tile rt in lane half lh.
__device__ __forceinline__ int acc_key(int rt, int r, int lh) { return 32 * rt + 8 * (r >> 2) + 4 * lh + (r & 3); }

// Position of key `k` (0..63) inside a transposed V tile: the 8 elements at column 16c + 8h are the keys
// {16c + 8*(j/4) + 4*h + j%4 : j < 8}, which is the order in which accumulator registers 8c..8c+7 of lane
// half h feed the B operand of the PV MFMA.
__device__ __forceinline__ int vt_slot(int k) {
  const int g = k >> 4, r = k & 15;
  return (g << 4) + (((r >> 2) & 1) << 3) + ((r >> 3) << 2) + (r & 3);
}

// How the softmax scale 1/sqrt(D) and the exp -> exp2 factor log2(e) are applied.
//   fast:  the logits are known to lie in [-64, 64] (log2 units): q carries log2(e)/sqrt(D) before its bf16
//          rounding, and P = exp2(S) needs neither a running max nor any per-score arithmetic.
//   !fast: q carries only the exact power of two 1/8 (as the reference's fused kernel does,
//          dense_attention.py:86-87), and P = exp2(S * c - m) with c = log2(e)/sqrt(D)*8 in fp32 and m the
//          running max of S * c, which costs one FMA per score in place of the subtraction.
struct SoftmaxPlan {
  bool fast;
  float qscale;  // folded into q before its bf16 rounding
  float c;       // applied to the raw logits in the running-max path
};

// `qn`, `kn`: upper bounds of |q| and |k| after normalisation and RoPE (before any scale).
__device__ __forceinline__ SoftmaxPlan softmax_plan(float qn, float kn, int D) {
  const float full = kLog2e / sqrtf(static_cast<float>(D));
  const float bound = qn * kn * full * 1.03f;  // 1.03 covers the bf16 roundings of q and k
  SoftmaxPlan p;
  p.fast = bound <= 64.f;  // false for NaN gains too
  p.qscale = p.fast ? full : 0.125f;
  p.c = p.fast ? 1.f : full * 8.f;
  return p;
}

// MASKED: `valid(key_in_tile)` decides per score whether the key takes part (false -> weight 0).
template <int D, bool FAST, bool MASKED, class Valid>
__device__ __forceinline__ void attend_tile(const uint16_t* __restrict__ sK, const uint16_t* __restrict__ sKd,
                                            const uint16_t* __restrict__ sVt, int kp, int vp,
                                            const u32x4 (&qf)[2][D / 16], f32x16 (&o)[2][D / 32],
                                            float (&lsum)[2], float (&m)[2], float c, Valid valid) {
  const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5;
  f32x16 sc[2][2];
#pragma unroll
  for (int br = 0; br < 2; ++br) {
    const uint16_t* sk = br ? sKd : sK;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      f32x16 acc = {};
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk)
        acc = mfma_bf16_32x32x16(lds16(sk + (32 * rt + lr) * kp + 16 * kk + 8 * lh), qf[br][kk], acc);
      sc[br][rt] = acc;
    }
  }
  if constexpr (MASKED) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (!valid(acc_key(rt, r, lh))) {
          sc[0][rt][r] = -INFINITY;
          sc[1][rt][r] = -INFINITY;
        }
  }

  u32x4 pb[2][2][2];  // [branch][row tile][16-key half]: 8 bf16 probabilities each
#pragma unroll
  for (int br = 0; br < 2; ++br) {
    float mb = 0.f;
    if constexpr (!FAST) {
      float mt = -INFINITY;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sc[br][rt][r]);
      mt = fmaxf(mt, __shfl_xor(mt, 32, kWave)) * c;
      const float mn = fmaxf(m[br], mt);
      // mn == -inf only while every key seen so far is masked; keep the state at zero then.
      const float alpha = mn == -INFINITY ? 1.f : fast_exp2(m[br] - mn);
      m[br] = mn;
      lsum[br] *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) o[br][dt] *= alpha;
      mb = mn == -INFINITY ? 0.f : mn;
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float e0, e1;
          if constexpr (FAST) {
            e0 = fast_exp2(sc[br][rt][8 * h + 2 * j]);
            e1 = fast_exp2(sc[br][rt][8 * h + 2 * j + 1]);
          } else {
            e0 = fast_exp2(__fmaf_rn(sc[br][rt][8 * h + 2 * j], c, -mb));
            e1 = fast_exp2(__fmaf_rn(sc[br][rt][8 * h + 2 * j + 1], c, -mb));
          }
          const uint32_t p = pack_bf16x2(e0, e1);
          pb[br][rt][h][j] = p;
          lsum[br] = add_bf16_pair(p, lsum[br]);
        }
  }

#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u32x4 a = lds16(sVt + (32 * dt + lr) * vp + 16 * g + 8 * lh);
      o[0][dt] = mfma_bf16_32x32x16(a, pb[0][g >> 1][g & 1], o[0][dt]);
      o[1][dt] = mfma_bf16_32x32x16(a, pb[1][g >> 1][g & 1], o[1][dt]);
    }
}

// out[q, h*D + d] = O1/l1 - lam * O2/l2 for this lane's query, written as bf16 in groups of 4 dims.
template <int D>
__device__ __forceinline__ void store_diff_bf16(uint16_t* __restrict__ orow, const f32x16 (&o)[2][D / 32],
                                                const float (&lsum)[2], float lam) {
  const int lh = (threadIdx.x & 63) >> 5;
  const float l0 = lsum[0] + __shfl_xor(lsum[0], 32, kWave);
  const float l1 = lsum[1] + __shfl_xor(lsum[1], 32, kWave);
  // Same correctly rounded reciprocal for both branches, so identical branches give identical factors.
  const float i0 = __frcp_rn(l0), i1 = __fmul_rn(lam, __frcp_rn(l1));
  if (!orow) return;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)  // rounded products: identical branches cancel exactly, as in the reference
        v[j] = __fsub_rn(__fmul_rn(o[0][dt][4 * g + j], i0), __fmul_rn(o[1][dt][4 * g + j], i1));
      u32x2 pk;
      pk[0] = pack_bf16x2(v[0], v[1]);
      pk[1] = pack_bf16x2(v[2], v[3]);
      *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * g + 4 * lh) = pk;
    }
}

}  // namespace hb
