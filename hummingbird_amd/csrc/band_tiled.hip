// SAME-L sliding-window (band) differential attention for the shapes the streaming ring kernel does not take:
// half-widths w > 128 (whose key window does not fit an LDS ring) and head_dim 128, bf16 or half inputs (bf16
// operands either way).
//
// Replaces the reference's fused TPU kernel sa3jax/band_attention.py:61-180 and the XLA chain
// sa3jax/same_l.py:151-169 on those shapes. Two kernels run back to back on the caller's stream, on the dense
// kernel's tiling (tiles.h):
//
//   band_prep    one pass over the key side of qkv: DyT (same_l.py:58-69) and rotate-half RoPE
//                (same_l.py:92-100) of k and k_diff in fp32 with one bf16 rounding, and V, written to a
//                workspace of three (B, H, Sp, D) regions; V is stored transposed per 64-key tile in the order
//                the PV MFMA consumes it. Keys at or past S are zero.
//   band_attend  one workgroup of 4 waves per (batch, head, 128-query block): each lane prepares one query row
//                (DyT, RoPE and the softmax scale, one rounding), then the 64-key tiles of the block's window
//                [q0 - w, q0 + 128 + w) stream through LDS (global_load_lds, double-buffered). Each wave skips
//                the tiles outside its band, runs the tiles inside |k - q| <= w for all of its queries unmasked
//                and masks the others per score (band_attention.py:108-110); the branches are subtracted in fp32
//                with one cast (same_l.py:168-169).
//
// Every key is prepared once per call and read back from L2 by the blocks whose window covers it.
#include "api.h"
#include "attn_tile.h"
#include "common.h"
#include "tiles.h"

namespace hb {
namespace band_tiled {

// DyT + RoPE of k and k_diff (and V transposed) for 64 keys of one head. Thread task = (key, RoPE group pair) as
// in the dense prep: the rotation partner and the cos / sin slice are in the thread's own registers.
// `kdyt` = [alpha, gamma[D], beta[D]]; `half` % 8 == 0 (checked on the host).
// IO: the element type of qkv (bf16 or half); the keys are prepared in bf16 either way.
template <class IO, int D>
__global__ __launch_bounds__(256) void band_prep(const uint16_t* __restrict__ qkv, int64_t rs,
                                                 const float* __restrict__ kdyt, const float* __restrict__ cosT,
                                                 const float* __restrict__ sinT, int half, int S, int Sp, int H,
                                                 int64_t region, uint16_t* __restrict__ ws) {
  constexpr int PAIRS = D / 16;
  constexpr int TASKS = 64 * PAIRS / 256;
  constexpr int VCH = 64 * D / 8 / 256;
  const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z, t = threadIdx.x;
  const int l0 = tile * 64;
  const int64_t bh = static_cast<int64_t>(b) * H + h;
  const int64_t HD = static_cast<int64_t>(H) * D;
  const int h8 = half / 8;
  const float a2 = 2.f * kLog2e * kdyt[0];

  u32x4 raw[TASKS][2][2];
  f32x4 cs[TASKS][4];
  int tm1[TASKS], tm2[TASKS];
  bool trot[TASKS];
#pragma unroll
  for (int i = 0; i < TASKS; ++i) {
    const int task = t + 256 * i, p = task % PAIRS, l = l0 + task / PAIRS;
    pair_groups(p, h8, tm1[i], tm2[i]);
    trot[i] = p < h8;
    const int lc = l < S ? l : S - 1;
    const uint16_t* row = qkv + (static_cast<int64_t>(b) * S + lc) * rs + h * D;
#pragma unroll
    for (int si = 0; si < 2; ++si) {
      const int sec = 1 + 3 * si;  // k, k_diff
      raw[i][si][0] = ld16(row + sec * HD + 8 * tm1[i]);
      raw[i][si][1] = ld16(row + sec * HD + 8 * tm2[i]);
    }
    if (trot[i]) {
      const float* c = cosT + static_cast<int64_t>(lc) * half + 8 * tm1[i];
      const float* s = sinT + static_cast<int64_t>(lc) * half + 8 * tm1[i];
      cs[i][0] = *reinterpret_cast<const f32x4*>(c);
      cs[i][1] = *reinterpret_cast<const f32x4*>(c + 4);
      cs[i][2] = *reinterpret_cast<const f32x4*>(s);
      cs[i][3] = *reinterpret_cast<const f32x4*>(s + 4);
    } else {
      cs[i][0] = cs[i][1] = f32x4{1.f, 1.f, 1.f, 1.f};
      cs[i][2] = cs[i][3] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  u32x4 vraw[VCH];
#pragma unroll
  for (int i = 0; i < VCH; ++i) {
    const int ch = t + 256 * i, l = l0 + ch / (D / 8), col = (ch % (D / 8)) * 8;
    vraw[i] = l < S ? ld16(qkv + (static_cast<int64_t>(b) * S + l) * rs + 2 * HD + h * D + col)
                    : u32x4{0u, 0u, 0u, 0u};
  }

#pragma unroll
  for (int i = 0; i < TASKS; ++i) {
    const int task = t + 256 * i, l = l0 + task / PAIRS;
    const int m1 = tm1[i], m2 = tm2[i];
    const float c[8] = {cs[i][0][0], cs[i][0][1], cs[i][0][2], cs[i][0][3],
                        cs[i][1][0], cs[i][1][1], cs[i][1][2], cs[i][1][3]};
    const float s[8] = {cs[i][2][0], cs[i][2][1], cs[i][2][2], cs[i][2][3],
                        cs[i][3][0], cs[i][3][1], cs[i][3][2], cs[i][3][3]};
#pragma unroll
    for (int si = 0; si < 2; ++si) {
      float x1[8], x2[8], o1[8], o2[8];
      IO::unpack8(raw[i][si][0], x1);
      IO::unpack8(raw[i][si][1], x2);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float g1 = kdyt[1 + 8 * m1 + j], b1 = kdyt[1 + D + 8 * m1 + j];
        const float g2 = kdyt[1 + 8 * m2 + j], b2 = kdyt[1 + D + 8 * m2 + j];
        const float y1 = dyt_tanh(x1[j], a2, -2.f * g1, g1 + b1);
        const float y2 = dyt_tanh(x2[j], a2, -2.f * g2, g2 + b2);
        // rotate_half: d < half takes -x[d + half], d >= half takes x[d - half]; fp32, one rounding
        o1[j] = l < S ? __fmaf_rn(y1, c[j], -(y2 * s[j])) : 0.f;
        o2[j] = l < S ? __fmaf_rn(y2, c[j], y1 * s[j]) : 0.f;
      }
      uint16_t* dst = ws + si * region + (bh * Sp + l) * D;
      st16(dst + 8 * m1, pack8(o1));
      st16(dst + 8 * m2, pack8(o2));
    }
  }

  // V (rounded to bf16, band_attention.py:94), transposed per 64-key tile (v_tile_key order) through LDS, the
  // 16-byte chunks of row r XOR-swizzled by (r / 8) % 8.
  __shared__ __attribute__((aligned(16))) uint16_t vt[64 * D];
  auto vt_at = [](int row, int col) { return row * D + 8 * ((col >> 3) ^ ((row >> 3) & 7)) + (col & 7); };
#pragma unroll
  for (int i = 0; i < VCH; ++i) {
    const int ch = t + 256 * i, key = ch / (D / 8), col = (ch % (D / 8)) * 8;
    *reinterpret_cast<u32x4*>(vt + vt_at(key, col)) = IO::to_bf16x8(vraw[i]);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < VCH; ++i) {
    const int ch = t + 256 * i, d = ch / 8, pos0 = (ch % 8) * 8;
    uint16_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = vt[vt_at(v_tile_key(pos0 + j), d)];
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = static_cast<uint32_t>(e[2 * j]) | (static_cast<uint32_t>(e[2 * j + 1]) << 16);
    st16(ws + 2 * region + (bh * Sp + l0) * D + d * 64 + pos0, w);
  }
}

// DyT, rotate-half RoPE over the first 2 * 8 H8 dims and the softmax scale of one query row held whole by this
// lane, in fp32 with one bf16 rounding (the reference fused kernel's cast points, band_attention.py:82-85, 104).
// `row`: its D elements in qkv; `cs` / `sn`: its (half) columns of the tables; `qdyt` = [alpha, gamma, beta].
template <class IO, int D, int H8>
__device__ __forceinline__ void prep_q_row(const uint16_t* __restrict__ row, const float* __restrict__ qdyt,
                                           const float* __restrict__ cs, const float* __restrict__ sn, float qscale,
                                           u32x4 (&out)[D / 8]) {
  u32x4 raw[D / 8];
#pragma unroll
  for (int c = 0; c < D / 8; ++c) raw[c] = ld16(row + 8 * c);
  float cv[8 * H8 + 1], sv[8 * H8 + 1];
#pragma unroll
  for (int j4 = 0; j4 < 2 * H8; ++j4) {
    const f32x4 c4 = *reinterpret_cast<const f32x4*>(cs + 4 * j4);
    const f32x4 s4 = *reinterpret_cast<const f32x4*>(sn + 4 * j4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      cv[4 * j4 + e] = c4[e];
      sv[4 * j4 + e] = s4[e];
    }
  }
  const float a2 = 2.f * kLog2e * qdyt[0];
  float y[D];
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    float x[8];
    IO::unpack8(raw[c], x);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int d = 8 * c + j;
      const float g = qdyt[1 + d], be = qdyt[1 + D + d];
      y[d] = dyt_tanh(x[j], a2, -2.f * g, g + be);
    }
  }
#pragma unroll
  for (int d = 0; d < 8 * H8; ++d) {
    const float y1 = y[d], y2 = y[d + 8 * H8];
    y[d] = __fmaf_rn(y1, cv[d], -(y2 * sv[d]));
    y[d + 8 * H8] = __fmaf_rn(y2, cv[d], y1 * sv[d]);
  }
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = y[8 * c + j] * qscale;
    out[c] = pack8(o);  // the single bf16 rounding
  }
}

// The window's tiles, double-buffered: tile t_lo has already been issued into stage A by the caller. A wave
// attends a tile only if it meets its band, unmasked when every (key, query) pair of the tile and the wave is in
// band and the keys exist; `qa` is the wave's first query, `nq` its query count (64 or 32).
template <int D, bool FAST>
__device__ __forceinline__ void band_tiles(const TileCopy<D>& issue, int S, int w, int t_lo, int t_hi, int qa, int nq,
                                           int br0, uint16_t* sA, uint16_t* sB,
                                           const u32x4 (&qf)[DenseTile<D>::NB][DenseTile<D>::NCT][D / 16],
                                           f32x16 (&o)[DenseTile<D>::NB][DenseTile<D>::NCT][D / 32],
                                           float (&lsum)[DenseTile<D>::NB][DenseTile<D>::NCT], float c) {
  using T = DenseTile<D>;
  constexpr int NB = T::NB, NCT = T::NCT;
  float m[NB][NCT];
#pragma unroll
  for (int br = 0; br < NB; ++br)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) m[br][ct] = -INFINITY;
  const int lr = threadIdx.x & 31, lh = (threadIdx.x >> 5) & 1;
  const int qlast = qa + nq - 1;
  const int wlo = qa - w > 0 ? qa - w : 0;          // the wave's union band
  const int whi = qlast + w < S - 1 ? qlast + w : S - 1;
  const uint32_t ldsA = lds_addr(sA), ldsB = lds_addr(sB);
  auto attend = [&](const uint16_t* s, int t) {
    const int k0 = 64 * t, k1 = k0 + 63;
    if (k0 > whi || k1 < wlo) return;  // outside the band of every query of the wave
    const bool inside = k0 >= qlast - w && k1 <= qa + w && k1 < S;
    attend_tile<D, NB, NCT, FAST>(
        [&](int b, int rt, int kk) { return lds16(s + (br0 + b) * T::K_ELEMS + swz<D>(32 * rt + lr, 2 * kk + lh)); },
        [&](int dt, int g) { return lds16(s + 2 * T::K_ELEMS + swz<64>(32 * dt + lr, 2 * g + lh)); },
        [&](int b, int ct, int kk) { return qf[b][ct][kk]; }, o, lsum, m, c, !inside, [&](int k, int ct) {
          const int key = k0 + k, dist = key - (qa + 32 * ct + lr);
          return (key < S) & (dist <= w) & (dist >= -w);
        });
  };
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int t = t_lo;
  for (; t + 1 <= t_hi; t += 2) {
    issue(t + 1, ldsB);  // stage B was last read in tile t - 1
    attend(sA, t);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t + 2 <= t_hi) issue(t + 2, ldsA);
    attend(sB, t + 1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if (t == t_hi) {  // an odd tile count: the last one sits in stage A
    attend(sA, t);
    __syncthreads();
  }
}

// IO: the element type of qkv and out (bf16 or half); the operands are bf16 either way.
template <class IO, int D>
__global__ __launch_bounds__(256, D == 64 ? 2 : 1) void band_attend(
    const uint16_t* __restrict__ qkv, int64_t rs, const float* __restrict__ qdyt, const float* __restrict__ kdyt,
    const float* __restrict__ cosT, const float* __restrict__ sinT, int half, int w, const uint16_t* __restrict__ ws,
    int64_t region, int B, int S, int Sp, int H, const float* __restrict__ lam, uint16_t* __restrict__ out) {
  using T = DenseTile<D>;
  constexpr int NB = T::NB, NCT = T::NCT;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * T::STAGE];
  const int nqb = (S + 127) / 128;
  const int tile = xcd_remap(blockIdx.x, B * H * nqb);
  const int qb = tile % nqb, bh = tile / nqb, h = bh % H, b = bh / H;
  const int lane = threadIdx.x & 63, wave = wave_id(), lr = lane & 31, lh = lane >> 5;
  const int br0 = T::SPLIT ? wave >> 1 : 0;
  const int q0 = qb * 128;
  const int qa = q0 + (T::SPLIT ? (wave & 1) * 64 : wave * 32);  // this wave's first query
  const int64_t rowbase = static_cast<int64_t>(bh) * Sp;

  // Launch-uniform softmax plan from the DyT bounds (|DyT(x)_d| <= |gamma_d| + |beta_d|; RoPE is a rotation).
  const SoftmaxPlan plan = softmax_plan(dyt_row_bound<D>(qdyt), dyt_row_bound<D>(kdyt), D);

  // The queries: each lane prepares one whole row (D = 64: row qa + lane of this wave's branch; D = 128: row
  // qa + lane % 32 of branch lane / 32), then v_permlane32_swap moves the chunks into the MFMA B-operand layout
  // (as in the dense kernel). Rows at or past S are prepared from row S - 1 and never stored.
  u32x4 qf[NB][NCT][D / 16];
  {
    const int64_t HD = static_cast<int64_t>(H) * D;
    const int qrow = T::SPLIT ? qa + lane : qa + lr;
    const int sec = 3 * (T::SPLIT ? br0 : lh);  // q is section 0 of a qkv row, q_diff section 3
    const int qc = qrow < S ? qrow : S - 1;
    const uint16_t* row = qkv + (static_cast<int64_t>(b) * S + qc) * rs + sec * HD + h * D;
    const float* cs = cosT + static_cast<int64_t>(qc) * half;
    const float* sn = sinT + static_cast<int64_t>(qc) * half;
    u32x4 whole[D / 8];
    switch (half / 8) {  // half % 8 == 0 and half <= D / 2 are checked on the host
      case 0: prep_q_row<IO, D, 0>(row, qdyt, cs, sn, plan.qscale, whole); break;
      case 1: prep_q_row<IO, D, 1>(row, qdyt, cs, sn, plan.qscale, whole); break;
      case 2: prep_q_row<IO, D, 2>(row, qdyt, cs, sn, plan.qscale, whole); break;
      case 3: prep_q_row<IO, D, 3>(row, qdyt, cs, sn, plan.qscale, whole); break;
      default:
        if constexpr (D == 64) {
          prep_q_row<IO, D, 4>(row, qdyt, cs, sn, plan.qscale, whole);
        } else {
          switch (half / 8) {
            case 4: prep_q_row<IO, D, 4>(row, qdyt, cs, sn, plan.qscale, whole); break;
            case 5: prep_q_row<IO, D, 5>(row, qdyt, cs, sn, plan.qscale, whole); break;
            case 6: prep_q_row<IO, D, 6>(row, qdyt, cs, sn, plan.qscale, whole); break;
            case 7: prep_q_row<IO, D, 7>(row, qdyt, cs, sn, plan.qscale, whole); break;
            default: prep_q_row<IO, D, 8>(row, qdyt, cs, sn, plan.qscale, whole); break;
          }
        }
    }
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const auto r = __builtin_amdgcn_permlane32_swap(whole[2 * kk][e], whole[2 * kk + 1][e], false, false);
        if constexpr (T::SPLIT) {
          qf[0][0][kk][e] = r[0];
          qf[0][1][kk][e] = r[1];
        } else {
          qf[0][0][kk][e] = r[0];
          qf[1][0][kk][e] = r[1];
        }
      }
  }

  f32x16 o[NB][NCT][D / 32];
  float lsum[NB][NCT];
#pragma unroll
  for (int bi = 0; bi < NB; ++bi)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      lsum[bi][ct] = 0.f;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) o[bi][ct][dt] = f32x16{};
    }

  // The block's key window [q0 - w, q0 + 127 + w] clipped to [0, S), in 64-key tiles.
  const int klo = q0 - w > 0 ? q0 - w : 0;
  const int khi = q0 + 127 + w < S - 1 ? q0 + 127 + w : S - 1;
  const int t_lo = klo / 64, t_hi = khi / 64;
  const TileCopy<D> copy(ws + rowbase * D, ws + region + rowbase * D, ws + 2 * region + rowbase * D);
  copy(t_lo, lds_addr(smem));
  const int nq = T::SPLIT ? 64 : 32;
  if (plan.fast)
    band_tiles<D, true>(copy, S, w, t_lo, t_hi, qa, nq, br0, smem, smem + T::STAGE, qf, o, lsum, plan.c);
  else
    band_tiles<D, false>(copy, S, w, t_lo, t_hi, qa, nq, br0, smem, smem + T::STAGE, qf, o, lsum, plan.c);

  static_assert(2 * NCT * (D / 32) * 16 * 64 * 4 <= 2 * T::STAGE * 2, "exchange buffer exceeds the two stages");
  store_diff_split<D, 128, IO>(out, b, S, H, h, qa, br0, lam ? lam[h] : 1.f, o, lsum, smem);
}

}  // namespace band_tiled

DenseLayout band_tiled_layout(int B, int S, int H, int D) { return dense_layout(HB_BF16, B, S, H, D); }

int launch_band_tiled(hipStream_t stream, int dtype, const void* qkv, int64_t rs, const float* q_dyt,
                      const float* k_dyt, const float* cosT, const float* sinT, int half, int window, const float* lam,
                      void* out, int B, int S, int H, int D, void* workspace) {
  using namespace band_tiled;
  const DenseLayout lay = band_tiled_layout(B, S, H, D);
  const int Sp = static_cast<int>(lay.Lp);
  const uint16_t* x = static_cast<const uint16_t*>(qkv);
  uint16_t* ws = static_cast<uint16_t*>(workspace);
  uint16_t* o = static_cast<uint16_t*>(out);
  const dim3 pgrid(static_cast<unsigned>(Sp / 64), static_cast<unsigned>(H), static_cast<unsigned>(B));
  const int nblocks = B * H * ((S + 127) / 128);
  const bool f16 = dtype == HB_F16;
  auto prep = D == 64 ? (f16 ? band_prep<F16Io, 64> : band_prep<Bf16Io, 64>)
                      : (f16 ? band_prep<F16Io, 128> : band_prep<Bf16Io, 128>);
  auto attend = D == 64 ? (f16 ? band_attend<F16Io, 64> : band_attend<Bf16Io, 64>)
                        : (f16 ? band_attend<F16Io, 128> : band_attend<Bf16Io, 128>);
  hipLaunchKernelGGL(prep, pgrid, dim3(256), 0, stream, x, rs, k_dyt, cosT, sinT, half, S, Sp, H, lay.region_elems,
                     ws);
  hipLaunchKernelGGL(attend, dim3(nblocks), dim3(256), 0, stream, x, rs, q_dyt, k_dyt, cosT, sinT, half, window, ws,
                     lay.region_elems, B, S, Sp, H, lam, o);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HB_ERR_LAUNCH, "band_tiled launch failed: %s", hipGetErrorString(e));
  return HB_OK;
}

}  // namespace hb
