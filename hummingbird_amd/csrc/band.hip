// SAME-L sliding-window (band) differential attention for gfx950 (MI355X).
//
// Replaces the reference's fused TPU kernel sa3jax/band_attention.py:61-180 and the XLA chain
// sa3jax/same_l.py:151-169, in one pass over qkv. One workgroup owns 128 consecutive queries of one
// (batch, head); its four waves hold 32 queries each in registers. The keys that can reach the block,
// [q0 - w, q0 + 128 + w) clipped to [0, S), stream through LDS in 64-key tiles:
//   - each tile's k and k_diff rows get DyT (same_l.py:58-69, fp32) and rotate-half RoPE (same_l.py:92-100,
//     fp32) and are rounded once to bf16; the v rows are transposed for the MFMA A operand;
//   - a wave skips tiles entirely outside its band, runs unmasked tiles that lie entirely inside it, and masks
//     `|k - q| <= w, k < S` per score only on the band's edge tiles (band_attention.py:108-110);
//   - the scores, softmax and both branches follow attn_tile.h; the subtraction is fp32 with one cast
//     (same_l.py:168-169).
// q and q_diff get the same DyT/RoPE plus the softmax scale before their single bf16 rounding.
//
// Softmax without a running max when DyT bounds the logits: |DyT(x)_d| <= |gamma_d| + |beta_d|, RoPE is a
// rotation, so |s| <= |q|max |k|max log2(e)/sqrt(D); when that is <= 64 exp2 needs no max, otherwise the
// running-max softmax runs (SoftmaxPlan in attn_tile.h).
#include "api.h"
#include "attn_tile.h"
#include "common.h"

namespace hb {

template <int D>
struct BandTile {
  static constexpr int KP = D + 8;
  static constexpr int VP = 64 + 8;
  static constexpr int K_ELEMS = 64 * KP;
  static constexpr int V_ELEMS = D * VP;
  static constexpr int STAGE = 2 * K_ELEMS + V_ELEMS;  // K, K_diff, V^T of one 64-key tile
  static constexpr int QSTAGE = 2 * 128 * KP;           // q, q_diff of the 128-query block
  static constexpr int ELEMS = STAGE > QSTAGE ? STAGE : QSTAGE;
  static constexpr int CH = D / 8;
  static constexpr int RPP = 256 / CH;
  static constexpr int PASSES = 64 / RPP;
};

// DyT + RoPE of 64 rows (sequence positions p0 .. p0+63) of one qkv section into bf16 LDS rows of pitch KP.
// Rows outside [0, S) are written as zeros.
template <int D>
__device__ __forceinline__ void band_prep_rows(const uint16_t* __restrict__ src, int64_t rs, int p0, int S,
                                               float alpha, const float (&gamma)[8], const float (&beta)[8],
                                               const float* __restrict__ cosT, const float* __restrict__ sinT,
                                               int half, float scale, float (*ybuf)[D + 1],
                                               uint16_t* __restrict__ dst) {
  using T = BandTile<D>;
  const int t = threadIdx.x, ch = t % T::CH, rsub = t / T::CH;
  float y[T::PASSES][8];
#pragma unroll
  for (int p = 0; p < T::PASSES; ++p) {
    const int row = p * T::RPP + rsub, pos = p0 + row;
    float x[8];
    if (pos >= 0 && pos < S) {
      unpack8(ld16(src + static_cast<int64_t>(pos) * rs + ch * 8), x);
#pragma unroll
      for (int i = 0; i < 8; ++i) y[p][i] = __fadd_rn(__fmul_rn(gamma[i], tanhf(__fmul_rn(alpha, x[i]))), beta[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) y[p][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ybuf[row][ch * 8 + i] = y[p][i];
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < T::PASSES; ++p) {
    const int row = p * T::RPP + rsub, pos = p0 + row;
    const bool in = pos >= 0 && pos < S;
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int d = ch * 8 + i;
      float r = y[p][i];
      if (d < 2 * half && in) {
        const int j = d < half ? d : d - half;
        const float c = cosT[static_cast<int64_t>(pos) * half + j];
        const float s = sinT[static_cast<int64_t>(pos) * half + j];
        const float partner = d < half ? -ybuf[row][d + half] : ybuf[row][d - half];
        r = __fadd_rn(__fmul_rn(r, c), __fmul_rn(partner, s));
      }
      o[i] = in ? __fmul_rn(r, scale) : 0.f;
    }
    *reinterpret_cast<u32x4*>(dst + row * T::KP + ch * 8) = pack8(o);
  }
  __syncthreads();
}

// |DyT(x)| bound: sqrt(sum_d (|gamma_d| + |beta_d|)^2), reduced over the wave.
template <int D>
__device__ __forceinline__ float dyt_norm_bound(const float* __restrict__ dyt) {
  const int lane = threadIdx.x & 63;
  float acc = 0.f;
  for (int d = lane; d < D; d += 64) {
    const float v = fabsf(dyt[1 + d]) + fabsf(dyt[1 + D + d]);
    acc += v * v;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, kWave);
  return sqrtf(acc);
}

template <int D, bool FAST>
__device__ __forceinline__ void band_loop(const uint16_t* __restrict__ xb, int64_t rs, int64_t HD, int h, int S,
                                          int window, int q0, const float* __restrict__ k_dyt,
                                          const float* __restrict__ cosT, const float* __restrict__ sinT, int half,
                                          float (*ybuf)[D + 1], uint16_t* smem, const u32x4 (&qf)[2][D / 16],
                                          f32x16 (&o)[2][D / 32], float (&lsum)[2], float c) {
  using T = BandTile<D>;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, lr = lane & 31;
  const int ch = t % T::CH, rsub = t / T::CH;
  const float ka = k_dyt[0];
  float kg[8], kbeta[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    kg[i] = k_dyt[1 + ch * 8 + i];
    kbeta[i] = k_dyt[1 + D + ch * 8 + i];
  }
  float m[2] = {-INFINITY, -INFINITY};
  const int qa = q0 + 32 * wave;  // this wave's first query
  const int q = qa + lr;           // this lane's query
  const int kbeg = q0 - window > 0 ? q0 - window : 0;
  const int kend = q0 + 128 + window < S ? q0 + 128 + window : S;
  uint16_t* sK = smem;
  uint16_t* sKd = smem + T::K_ELEMS;
  uint16_t* sVt = smem + 2 * T::K_ELEMS;

  for (int kt0 = kbeg; kt0 < kend; kt0 += 64) {
    band_prep_rows<D>(xb + 1 * HD + h * D, rs, kt0, S, ka, kg, kbeta, cosT, sinT, half, 1.f, ybuf, sK);
    band_prep_rows<D>(xb + 4 * HD + h * D, rs, kt0, S, ka, kg, kbeta, cosT, sinT, half, 1.f, ybuf, sKd);
    // V rows, transposed with the MFMA key permutation; positions >= S are zero.
#pragma unroll
    for (int p = 0; p < T::PASSES; ++p) {
      const int row = p * T::RPP + rsub, pos = kt0 + row;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (pos < S) v = ld16(xb + static_cast<int64_t>(pos) * rs + 2 * HD + h * D + ch * 8);
      const int slot = vt_slot(row);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sVt[(ch * 8 + 2 * i) * T::VP + slot] = static_cast<uint16_t>(v[i] & 0xffffu);
        sVt[(ch * 8 + 2 * i + 1) * T::VP + slot] = static_cast<uint16_t>(v[i] >> 16);
      }
    }
    __syncthreads();

    // Wave-uniform band classification of this tile against the wave's 32 queries.
    const int klast = kt0 + 63;
    const bool touches = kt0 <= qa + 31 + window && klast >= qa - window;
    if (touches) {
      const bool inside = kt0 >= qa + 31 - window && klast <= qa + window && klast < S;
      if (inside) {
        attend_tile<D, FAST, false>(sK, sKd, sVt, T::KP, T::VP, qf, o, lsum, m, c, [](int) { return true; });
      } else {
        attend_tile<D, FAST, true>(sK, sKd, sVt, T::KP, T::VP, qf, o, lsum, m, c, [&](int k) {
          const int key = kt0 + k, dist = key - q;
          return key < S && dist <= window && dist >= -window;
        });
      }
    }
    __syncthreads();
  }
}

template <int D>
__global__ __launch_bounds__(256) void band_attend_bf16(const uint16_t* __restrict__ qkv, int64_t rs, int B, int S,
                                                        int H, int window, const float* __restrict__ q_dyt,
                                                        const float* __restrict__ k_dyt,
                                                        const float* __restrict__ cosT,
                                                        const float* __restrict__ sinT, int half,
                                                        const float* __restrict__ lam,
                                                        uint16_t* __restrict__ out) {
  using T = BandTile<D>;
  __shared__ float ybuf[64][D + 1];
  __shared__ __attribute__((aligned(16))) uint16_t smem[T::ELEMS];
  const int nqb = (S + 127) / 128;
  const int tile = xcd_remap(blockIdx.x, B * H * nqb);
  const int qb = tile % nqb, bh = tile / nqb, h = bh % H, b = bh / H;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, lr = lane & 31, lh = lane >> 5;
  const int ch = t % T::CH;
  const int q0 = qb * 128;
  const int64_t HD = static_cast<int64_t>(H) * D;
  const uint16_t* xb = qkv + static_cast<int64_t>(b) * S * rs;

  const SoftmaxPlan plan = softmax_plan(dyt_norm_bound<D>(q_dyt), dyt_norm_bound<D>(k_dyt), D);

  // q and q_diff of the block: DyT, RoPE, * log2(e)/sqrt(D), bf16, staged in LDS then loaded as B fragments.
  {
    const float qa = q_dyt[0];
    float qg[8], qbeta[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qg[i] = q_dyt[1 + ch * 8 + i];
      qbeta[i] = q_dyt[1 + D + ch * 8 + i];
    }
#pragma unroll
    for (int br = 0; br < 2; ++br)
#pragma unroll
      for (int half_blk = 0; half_blk < 2; ++half_blk)
        band_prep_rows<D>(xb + (br ? 3 : 0) * HD + h * D, rs, q0 + 64 * half_blk, S, qa, qg, qbeta, cosT, sinT, half,
                          plan.qscale, ybuf, smem + br * 128 * T::KP + 64 * half_blk * T::KP);
  }
  u32x4 qf[2][D / 16];
#pragma unroll
  for (int br = 0; br < 2; ++br)
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
      qf[br][kk] = lds16(smem + br * 128 * T::KP + (32 * wave + lr) * T::KP + 16 * kk + 8 * lh);
  __syncthreads();

  f32x16 o[2][D / 32];
#pragma unroll
  for (int br = 0; br < 2; ++br)
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) o[br][dt] = f32x16{};
  float lsum[2] = {0.f, 0.f};
  if (plan.fast)
    band_loop<D, true>(xb, rs, HD, h, S, window, q0, k_dyt, cosT, sinT, half, ybuf, smem, qf, o, lsum, plan.c);
  else
    band_loop<D, false>(xb, rs, HD, h, S, window, q0, k_dyt, cosT, sinT, half, ybuf, smem, qf, o, lsum, plan.c);

  const int q = q0 + 32 * wave + lr;
  uint16_t* orow = q < S ? out + (static_cast<int64_t>(b) * S + q) * HD + h * D : nullptr;
  store_diff_bf16<D>(orow, o, lsum, lam ? lam[h] : 1.f);
}

}  // namespace hb

using namespace hb;

extern "C" int hb_band_diffattn(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride,
                                const float* q_dyt, const float* k_dyt, const float* cos, const float* sin, int half,
                                int window, const float* lam, void* out, int B, int S, int H, int D) {
  int st = hb_band_validate(dtype, row_stride, B, S, H, D, half, window);
  if (st) return st;
  if (!qkv || !q_dyt || !k_dyt || !out) return fail(HB_ERR_NULL, "qkv, q_dyt, k_dyt and out must be non-NULL");
  if (half > 0 && (!cos || !sin)) return fail(HB_ERR_NULL, "cos and sin must be non-NULL when half > 0");
  if (reinterpret_cast<uintptr_t>(qkv) % 16) return fail(HB_ERR_STRIDE, "qkv must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(out) % 8) return fail(HB_ERR_STRIDE, "out must be 8-byte aligned");
  if (dtype != HB_BF16) return fail(HB_ERR_DTYPE, "band fp32 path not built yet");
  const int nblocks = B * H * ((S + 127) / 128);
  const uint16_t* x = static_cast<const uint16_t*>(qkv);
  uint16_t* o = static_cast<uint16_t*>(out);
  if (D == 64)
    hipLaunchKernelGGL(band_attend_bf16<64>, dim3(nblocks), dim3(256), 0, stream, x, row_stride, B, S, H, window,
                       q_dyt, k_dyt, cos, sin, half, lam, o);
  else
    hipLaunchKernelGGL(band_attend_bf16<128>, dim3(nblocks), dim3(256), 0, stream, x, row_stride, B, S, H, window,
                       q_dyt, k_dyt, cos, sin, half, lam, o);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HB_ERR_LAUNCH, "band_attend launch failed: %s", hipGetErrorString(e));
  return HB_OK;
}
