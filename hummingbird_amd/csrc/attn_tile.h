// One 64-key step of the two-branch differential attention, shared by the dense and band kernels.
//
// Per wave: 32 queries (MFMA columns) against 64 keys (two 32-row MFMA tiles), both branches.
//   S^T[key][query] = K Q^T        v_mfma_f32_32x32x16_bf16, A = K rows from LDS, B = Q held in registers
//   P = exp2(S^T) or exp2(S^T c - m)   see SoftmaxPlan
//   O^T[d][query] += V^T P^T       A = V^T via transposing reads of row-major V in LDS, B = P straight from the
//                                  S^T accumulators
// The C layout of a 32x32 MFMA gives lane l the column l % 32 and, in register r, the row
// 8*(r/4) + 4*(l/32) + r%4. Row sums therefore stay lane-local; the two lane halves hold different keys of the
// same query and are combined once at the end.
#pragma once

#include "common.h"

namespace hb {

__device__ __forceinline__ u32x4 lds16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Key (relative to the tile start) held by accumulator register r of row tile rt in lane half lh.
__device__ __forceinline__ int acc_key(int rt, int r, int lh) { return 32 * rt + 8 * (r >> 2) + 4 * lh + (r & 3); }

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// A operand of the PV MFMA for d-tile dt and 16-key group g, read from a row-major V tile (pitch vp elements)
// with gfx950's transposing LDS read. ds_read_b64_tr_b16 hands lane m of each 16-lane group element m of the
// four 8-byte row chunks the group addressed; addressing rows k0 + m/4 at columns d0 + 4*(m%4) therefore gives
// lane (lr, lh) the column d = 32*dt + lr of rows k0 .. k0+3. The eight keys returned,
// {16g + 8*(j/4) + 4*lh + j%4 : j < 8}, are exactly the keys that accumulator registers 8c..8c+7 (c = g % 2) of
// lane half lh feed to the B operand, so P can be used straight from the S^T accumulators.
__device__ __forceinline__ u32x4 v_frag(const uint16_t* __restrict__ sV, int vp, int dt, int g) {
  const int lane = threadIdx.x & 63, grp = lane >> 4, m = lane & 15;
  const int row = 16 * g + 4 * (grp >> 1) + (m >> 2);
  const int col = 32 * dt + 16 * (grp & 1) + 4 * (m & 3);
  // generic -> LDS address-space casts (sV points into __shared__ memory)
  lds_i16x4* p0 = (lds_i16x4*)(sV + row * vp + col);
  lds_i16x4* p1 = (lds_i16x4*)(sV + (row + 8) * vp + col);
  const i16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p0);
  const i16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p1);
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return u32x4{ua[0], ua[1], ub[0], ub[1]};
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

// One 64-key step for NB differential branches (1 or 2) and NCT column tiles of 32 queries each. Every K
// fragment read from LDS feeds NCT MFMAs and every V fragment NB * NCT MFMAs. One code path for every tile:
// `masked` (wave-uniform) only switches on the per-score masking step, so masked and unmasked tiles share
// registers; `valid(key_in_tile, ct)` then decides whether a key takes part for column tile ct (false -> weight
// 0). Branches run one after the other up to their probabilities, so only one branch's scores are live at a time.
// `kf(b, rt, kk)` is the A operand of S^T for branch slot b: this lane's 8 bf16 of key row 32 rt + lr, dims
// 16 kk + 8 lh .. +8. `vf(dt, g)` is the A operand of O^T: dim 32 dt + lr of the eight keys
// {16 g + 8 (j / 4) + 4 lh + j % 4 : j < 8} that the lane's probability registers hold (see v_frag).
// `qf(b, ct, kk)` is the B operand (8 bf16 of this lane's query in column tile ct) for branch slot b and dims
// 16 kk + 8 lh .. +8. RT: 32-key row tiles attended (2 = the whole tile; 1 = its first 32 keys only, for a last
// tile whose other keys do not exist: their probabilities would be 0 and their products add nothing).
template <int D, int NB, int NCT, bool FAST, int RT = 2, class KFrag, class VFrag, class QFrag, class Valid>
__device__ __forceinline__ void attend_tile(KFrag kf, VFrag vf, QFrag qf, f32x16 (&o)[NB][NCT][D / 32],
                                            float (&lsum)[NB][NCT], float (&m)[NB][NCT], float c, bool masked,
                                            Valid valid) {
  static_assert(RT == 1 || RT == 2, "a tile is one or two 32-key row tiles");
  const int lane = threadIdx.x & 63, lh = lane >> 5;
  u32x4 pb[NB][NCT][2][2];  // [branch][column tile][row tile][16-key half]: 8 bf16 probabilities each
#pragma unroll
  for (int br = 0; br < NB; ++br) {
    f32x16 sc[NCT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      f32x16 acc[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) acc[ct] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        const u32x4 a = kf(br, rt, kk);
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc[ct] = mfma_bf16_32x32x16(a, qf(br, ct, kk), acc[ct]);
      }
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) sc[ct][rt] = acc[ct];
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      if (masked) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            sc[ct][rt][r] = valid(acc_key(rt, r, lh), ct) ? sc[ct][rt][r] : -INFINITY;
      }
      float mb = 0.f;
      if constexpr (!FAST) {
        float mt = -INFINITY;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sc[ct][rt][r]);
        mt = fmaxf(mt, __shfl_xor(mt, 32, kWave)) * c;
        const float mn = fmaxf(m[br][ct], mt);
        // mn == -inf only while every key seen so far is masked; keep the state at zero then.
        const float alpha = mn == -INFINITY ? 1.f : fast_exp2(m[br][ct] - mn);
        m[br][ct] = mn;
        lsum[br][ct] *= alpha;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) o[br][ct][dt] *= alpha;
        mb = mn == -INFINITY ? 0.f : mn;
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float e0, e1;
            if constexpr (FAST) {
              e0 = fast_exp2(sc[ct][rt][8 * h + 2 * j]);
              e1 = fast_exp2(sc[ct][rt][8 * h + 2 * j + 1]);
            } else {
              e0 = fast_exp2(__fmaf_rn(sc[ct][rt][8 * h + 2 * j], c, -mb));
              e1 = fast_exp2(__fmaf_rn(sc[ct][rt][8 * h + 2 * j + 1], c, -mb));
            }
            const uint32_t p = pack_bf16x2(e0, e1);
            pb[br][ct][rt][h][j] = p;
            lsum[br][ct] = add_bf16_pair(p, lsum[br][ct]);
          }
    }
  }

#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int g = 0; g < 2 * RT; ++g) {
      const u32x4 a = vf(dt, g);
#pragma unroll
      for (int br = 0; br < NB; ++br)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
          o[br][ct][dt] = mfma_bf16_32x32x16(a, pb[br][ct][g >> 1][g & 1], o[br][ct][dt]);
    }
}

// 1 / (sum of this lane's query over both lane halves) for branch slot br, column tile ct: the same correctly
// rounded reciprocal for both branches, so identical branches give identical factors.
template <int NB, int NCT>
__device__ __forceinline__ float inv_rowsum(const float (&lsum)[NB][NCT], int br, int ct) {
  return __frcp_rn(lsum[br][ct] + __shfl_xor(lsum[br][ct], 32, kWave));
}

// out[q, h*D + d] = O1/l1 - lam * O2/l2 for this lane's query of column tile ct, written in the output type IO
// (bf16 or half) in groups of 4 dims. Every lane must call it (it combines the two lane halves); `orow` may be null
// for queries >= N.
template <int D, int NCT, class IO = Bf16Io>
__device__ __forceinline__ void store_diff_bf16(uint16_t* __restrict__ orow, const f32x16 (&o)[2][NCT][D / 32],
                                                const float (&lsum)[2][NCT], int ct, float lam) {
  const int lh = (threadIdx.x & 63) >> 5;
  const float i0 = inv_rowsum(lsum, 0, ct), i1 = __fmul_rn(lam, inv_rowsum(lsum, 1, ct));
  if (!orow) return;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)  // rounded products: identical branches cancel exactly, as in the reference
        v[j] = __fsub_rn(__fmul_rn(o[0][ct][dt][4 * g + j], i0), __fmul_rn(o[1][ct][dt][4 * g + j], i1));
      u32x2 pk;
      pk[0] = IO::pack2(v[0], v[1]);
      pk[1] = IO::pack2(v[2], v[3]);
      *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * g + 4 * lh) = pk;
    }
}

}  // namespace hb
