// SAME-L sliding-window (band) differential attention for gfx950 (MI355X).
//
// Replaces the reference's fused TPU kernel sa3jax/band_attention.py:61-180 and the XLA chain
// sa3jax/same_l.py:151-169, in one pass over qkv.
//
// Work split. One workgroup (8 waves, 512 threads) owns 256 consecutive queries of one (batch, head); each
// wave attends 32 of them. The keys that can reach the block,
// [q0 - w, q0 + 256 + w) clipped to [0, S), stream through LDS in 64-key tiles, double-buffered with one
// barrier per tile:
//   - waves 0-3 prepare K and K_diff of the tile: DyT (same_l.py:58-69, fp32) and rotate-half RoPE
//     (same_l.py:92-100, fp32), one bf16 rounding; each thread owns a pair of 8-dim groups that RoPE couples
//     (d and d + half), so the rotation partner is in the thread's own registers and the cos/sin row is
//     loaded once for k and k_diff;
//   - waves 4-7 copy the tile's V rows (row-major; the MFMA operand is read with transposing LDS loads);
//   - the raw rows of the next tile are loaded into registers while the current tile is attended (the cos/sin
//     slices, shared by all heads and L2-resident, are read at prep time);
//   - q and q_diff of the block stay in LDS (prepared once) and are re-read as MFMA B operands each tile, which
//     keeps the register budget within two waves per SIMD;
//   - every wave then attends the tile if it intersects its band: unmasked when the tile lies inside
//     `|k - q| <= w` for all its 32 queries, masked per score on the band edges (band_attention.py:108-110).
// Scores, softmax and both branches follow attn_tile.h; the subtraction is fp32 with one cast
// (same_l.py:168-169). tanh is evaluated as 1 - 2 / (1 + 2^(2 log2(e) x)): two transcendental
// instructions instead of a libm call, absolute error ~1e-7.
//
// Softmax without a running max when DyT bounds the logits: |DyT(x)_d| <= |gamma_d| + |beta_d| and RoPE is
// a rotation, so |s| <= |q|max |k|max log2(e)/sqrt(D); when that is <= 64 exp2 needs no max, otherwise the
// running-max softmax runs (SoftmaxPlan in attn_tile.h).
#include "api.h"
#include "attn_tile.h"
#include "common.h"

namespace hb {

template <int D>
struct BandCfg {
  static constexpr int NW = 8;              // waves per workgroup
  static constexpr int NT = 64 * NW;        // threads
  static constexpr int QB = 32 * NW;        // queries per workgroup
  static constexpr int KT = 64;             // keys per tile
  static constexpr int KP = D + 8;          // K / K_diff / V / Q row pitch (elements)
  static constexpr int K_ELEMS = KT * KP;
  static constexpr int STAGE = 3 * K_ELEMS;           // K, K_diff, V of one tile, all row-major
  static constexpr int QSTAGE = 2 * QB * KP;          // q, q_diff of the block
  // D = 64: q stays in LDS and is re-read every tile (keeps two waves per SIMD without spills).
  // D = 128: q does not fit beside the tiles; it is staged through the tile buffers into registers.
  static constexpr bool Q_IN_LDS = D == 64;
  static constexpr int TILE_BASE = Q_IN_LDS ? QSTAGE : 0;
  static constexpr int LDS_ELEMS = Q_IN_LDS ? QSTAGE + 2 * STAGE : (QSTAGE > 2 * STAGE ? QSTAGE : 2 * STAGE);
  static constexpr int PAIRS = D / 16;                // 16-dim group pairs per row
  static constexpr int KTASK = KT * PAIRS / 256;      // (key, pair) tasks per prep thread (waves 0-3)
  static constexpr int VTASK = KT * D / 8 / 256;      // 16-byte V chunks per copy thread (waves 4-7)
  static constexpr int QTASK = QB * PAIRS / NT;       // (query, pair) tasks per thread at the start
};

// Raw inputs of one (position, pair) task for two tensors of one section pair, plus its RoPE table slice.
struct PairRaw {
  u32x4 a1, a2;  // tensor A (q or k): groups m1, m2
  u32x4 b1, b2;  // tensor B (q_diff or k_diff): groups m1, m2
  f32x4 c0, c1, s0, s1;  // cos / sin of the 8 rotary frequencies 8*m1 .. 8*m1+7
};

__device__ __forceinline__ void load_rows(PairRaw& r, const uint16_t* __restrict__ rowA,
                                          const uint16_t* __restrict__ rowB, int pos, int S, int m1, int m2) {
  if (pos >= 0 && pos < S) {
    r.a1 = ld16(rowA + 8 * m1);
    r.a2 = ld16(rowA + 8 * m2);
    r.b1 = ld16(rowB + 8 * m1);
    r.b2 = ld16(rowB + 8 * m2);
  } else {
    r.a1 = r.a2 = r.b1 = r.b2 = u32x4{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void load_table(PairRaw& r, const float* __restrict__ cosT,
                                           const float* __restrict__ sinT, int pos, int S, int half, int m1,
                                           bool rot) {
  if (rot && pos >= 0 && pos < S) {
    const float* c = cosT + static_cast<int64_t>(pos) * half + 8 * m1;
    const float* s = sinT + static_cast<int64_t>(pos) * half + 8 * m1;
    r.c0 = *reinterpret_cast<const f32x4*>(c);
    r.c1 = *reinterpret_cast<const f32x4*>(c + 4);
    r.s0 = *reinterpret_cast<const f32x4*>(s);
    r.s1 = *reinterpret_cast<const f32x4*>(s + 4);
  }
}

// gamma * tanh(alpha * x) + beta with tanh(y) = 1 - 2 / (1 + 2^(2 log2(e) y)); `a2` = 2 log2(e) alpha.
__device__ __forceinline__ float dyt(float x, float a2, float g, float b) {
  const float e = fast_exp2(a2 * x);
  const float t = __fmaf_rn(-2.f, __builtin_amdgcn_rcpf(1.f + e), 1.f);
  return __fmaf_rn(g, t, b);
}

// DyT + RoPE (+ scale) of one tensor's 16 dims (groups m1, m2), written as bf16 into an LDS row.
__device__ __forceinline__ void prep_pair(u32x4 v1, u32x4 v2, const PairRaw& r, bool rot, bool in, float a2,
                                          const float* __restrict__ dyt_g, const float* __restrict__ dyt_b,
                                          int m1, int m2, float scale, uint16_t* __restrict__ dst) {
  float x1[8], x2[8];
  unpack8(v1, x1);
  unpack8(v2, x2);
  float y1[8], y2[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    y1[j] = dyt(x1[j], a2, dyt_g[8 * m1 + j], dyt_b[8 * m1 + j]);
    y2[j] = dyt(x2[j], a2, dyt_g[8 * m2 + j], dyt_b[8 * m2 + j]);
  }
  float o1[8], o2[8];
  if (rot) {
    const float cs[8] = {r.c0[0], r.c0[1], r.c0[2], r.c0[3], r.c1[0], r.c1[1], r.c1[2], r.c1[3]};
    const float sn[8] = {r.s0[0], r.s0[1], r.s0[2], r.s0[3], r.s1[0], r.s1[1], r.s1[2], r.s1[3]};
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // rotate_half: d < half takes -x[d + half], d >= half takes x[d - half]
      o1[j] = __fmul_rn(__fadd_rn(__fmul_rn(y1[j], cs[j]), __fmul_rn(-y2[j], sn[j])), scale);
      o2[j] = __fmul_rn(__fadd_rn(__fmul_rn(y2[j], cs[j]), __fmul_rn(y1[j], sn[j])), scale);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o1[j] = __fmul_rn(y1[j], scale);
      o2[j] = __fmul_rn(y2[j], scale);
    }
  }
  if (!in) {
#pragma unroll
    for (int j = 0; j < 8; ++j) o1[j] = o2[j] = 0.f;
  }
  *reinterpret_cast<u32x4*>(dst + 8 * m1) = pack8(o1);
  *reinterpret_cast<u32x4*>(dst + 8 * m2) = pack8(o2);
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

template <int D, bool FAST, class QFrag>
__device__ __forceinline__ void band_loop(const uint16_t* __restrict__ xb, int64_t rs, int64_t HD, int h, int S,
                                          int window, int half, int q0, const float* __restrict__ cosT,
                                          const float* __restrict__ sinT, float ka2, const float* sdyt_kg,
                                          const float* sdyt_kb, uint16_t* smem, QFrag qf,
                                          f32x16 (&o)[2][1][D / 32], float (&lsum)[2][1], float c) {
  using C = BandCfg<D>;
  const int t = threadIdx.x, lane = t & 63, wave = wave_id(), lr = lane & 31;
  const int h8 = half / 8;
  float m[2][1] = {{-INFINITY}, {-INFINITY}};
  uint16_t* tiles = smem + C::TILE_BASE;
  const int qa = q0 + 32 * wave;  // this wave's first query
  const int q = qa + lr;           // this lane's query
  const int kbeg = q0 - window > 0 ? q0 - window : 0;
  const int kend = q0 + C::QB + window < S ? q0 + C::QB + window : S;
  const bool producer = wave < 4;  // waves 0-3 prepare K / K_diff, waves 4-7 copy V
  const int pt = t & 255;          // thread index inside its half of the workgroup

  // Per-thread task geometry (fixed for every tile).
  int tk_key[C::KTASK], tk_m1[C::KTASK], tk_m2[C::KTASK];
  bool tk_rot[C::KTASK];
#pragma unroll
  for (int i = 0; i < C::KTASK; ++i) {
    const int task = pt + 256 * i, p = task % C::PAIRS;
    tk_key[i] = task / C::PAIRS;
    pair_groups(p, h8, tk_m1[i], tk_m2[i]);
    tk_rot[i] = p < h8;
  }
  PairRaw kraw[C::KTASK];
  u32x4 vraw[C::VTASK];

  auto gload = [&](int kt0) {
    if (producer) {
#pragma unroll
      for (int i = 0; i < C::KTASK; ++i) {
        const int pos = kt0 + tk_key[i];
        const uint16_t* row = xb + static_cast<int64_t>(pos) * rs + h * D;
        load_rows(kraw[i], row + 1 * HD, row + 4 * HD, pos, S, tk_m1[i], tk_m2[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < C::VTASK; ++i) {
        const int ch = pt + 256 * i, key = ch / (D / 8), col = (ch % (D / 8)) * 8, pos = kt0 + key;
        vraw[i] = pos < S ? ld16(xb + static_cast<int64_t>(pos) * rs + 2 * HD + h * D + col) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto prep = [&](int kt0, uint16_t* s) {
    if (producer) {
      const int z = opaque_zero();  // re-read gamma/beta every tile rather than pin 32 registers for them
#pragma unroll
      for (int i = 0; i < C::KTASK; ++i) {
        const int pos = kt0 + tk_key[i];
        const bool in = pos < S;
        load_table(kraw[i], cosT, sinT, pos, S, half, tk_m1[i], tk_rot[i]);  // L2-resident, read at prep time
        uint16_t* rowK = s + tk_key[i] * C::KP;
        prep_pair(kraw[i].a1, kraw[i].a2, kraw[i], tk_rot[i], in, ka2, sdyt_kg + z, sdyt_kb + z, tk_m1[i],
                  tk_m2[i], 1.f, rowK);
        prep_pair(kraw[i].b1, kraw[i].b2, kraw[i], tk_rot[i], in, ka2, sdyt_kg + z, sdyt_kb + z, tk_m1[i],
                  tk_m2[i], 1.f, rowK + C::K_ELEMS);
      }
    } else {
      uint16_t* sv = s + 2 * C::K_ELEMS;
#pragma unroll
      for (int i = 0; i < C::VTASK; ++i) {
        const int ch = pt + 256 * i, key = ch / (D / 8), col = (ch % (D / 8)) * 8;
        *reinterpret_cast<u32x4*>(sv + key * C::KP + col) = vraw[i];
      }
    }
  };

  if (kbeg < kend) gload(kbeg);
  int stage = 0;
  for (int kt0 = kbeg; kt0 < kend; kt0 += C::KT, stage ^= 1) {
    uint16_t* s = tiles + stage * C::STAGE;
    prep(kt0, s);
    if (kt0 + C::KT < kend) gload(kt0 + C::KT);
    __syncthreads();

    // Wave-uniform band classification of this tile against the wave's 32 queries: skipped when it lies
    // outside the band, unmasked when `|k - q| <= w` holds for every pair, masked per score otherwise.
    const int klast = kt0 + C::KT - 1;
    if (kt0 <= qa + 31 + window && klast >= qa - window) {
      const bool inside = kt0 >= qa + 31 - window && klast <= qa + window && klast < S;
      const int klh = (threadIdx.x >> 5) & 1;
      attend_tile<D, 2, 1, FAST>(
          [&](int br, int rt, int kk) { return lds16(s + br * C::K_ELEMS + (32 * rt + lr) * C::KP + 16 * kk + 8 * klh); },
          [&](int dt, int g) { return v_frag(s + 2 * C::K_ELEMS, C::KP, dt, g); }, qf, o, lsum, m, c, !inside,
          [&](int k, int) {
                             const int key = kt0 + k, dist = key - q;
                             return (key < S) & (dist <= window) & (dist >= -window);
                           });
    }
  }
}

template <int D>
__global__ __launch_bounds__(512) void band_attend_bf16(const uint16_t* __restrict__ qkv, int64_t rs, int B, int S,
                                                        int H, int window, const float* __restrict__ q_dyt,
                                                        const float* __restrict__ k_dyt,
                                                        const float* __restrict__ cosT,
                                                        const float* __restrict__ sinT, int half,
                                                        const float* __restrict__ lam,
                                                        uint16_t* __restrict__ out) {
  using C = BandCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[C::LDS_ELEMS];
  __shared__ float sdyt[4 * D];  // q gamma, q beta, k gamma, k beta
  const int nqb = (S + C::QB - 1) / C::QB;
  // Logical order: query block major, (batch, head) minor. Each XCD walks a contiguous range, so the heads of a
  // query block (which read the same RoPE table rows) and its neighbours (which share the key halo) run
  // together on one XCD and meet in its L2.
  const int tile = xcd_remap(blockIdx.x, B * H * nqb);
  const int qb = tile / (B * H), bh = tile % (B * H), h = bh % H, b = bh / H;
  const int t = threadIdx.x, lane = t & 63, wave = wave_id(), lr = lane & 31, lh = lane >> 5;
  const int q0 = qb * C::QB;
  const int64_t HD = static_cast<int64_t>(H) * D;
  const uint16_t* xb = qkv + static_cast<int64_t>(b) * S * rs;
  const int h8 = half / 8;

  for (int i = t; i < D; i += C::NT) {
    sdyt[i] = q_dyt[1 + i];
    sdyt[D + i] = q_dyt[1 + D + i];
    sdyt[2 * D + i] = k_dyt[1 + i];
    sdyt[3 * D + i] = k_dyt[1 + D + i];
  }
  const SoftmaxPlan plan = softmax_plan(dyt_norm_bound<D>(q_dyt), dyt_norm_bound<D>(k_dyt), D);
  const float qa2 = 2.f * kLog2e * q_dyt[0], ka2 = 2.f * kLog2e * k_dyt[0];
  __syncthreads();

  // q and q_diff of the block: DyT, RoPE and the softmax scale, one bf16 rounding, staged in LDS.
#pragma unroll
  for (int i = 0; i < C::QTASK; ++i) {
    const int task = t + C::NT * i, p = task % C::PAIRS, row = task / C::PAIRS, pos = q0 + row;
    int m1, m2;
    pair_groups(p, h8, m1, m2);
    const bool rot = p < h8;
    PairRaw r;
    const uint16_t* src = xb + static_cast<int64_t>(pos) * rs + h * D;
    load_rows(r, src, src + 3 * HD, pos, S, m1, m2);
    load_table(r, cosT, sinT, pos, S, half, m1, rot);
    const bool in = pos < S;
    prep_pair(r.a1, r.a2, r, rot, in, qa2, sdyt, sdyt + D, m1, m2, plan.qscale, smem + row * C::KP);
    prep_pair(r.b1, r.b2, r, rot, in, qa2, sdyt, sdyt + D, m1, m2, plan.qscale, smem + (C::QB + row) * C::KP);
  }
  f32x16 o[2][1][D / 32];
#pragma unroll
  for (int br = 0; br < 2; ++br)
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) o[br][0][dt] = f32x16{};
  float lsum[2][1] = {{0.f}, {0.f}};
  if constexpr (C::Q_IN_LDS) {
    // the first barrier inside band_loop publishes the staged q rows
    const uint16_t* sq = smem + (32 * wave + lr) * C::KP + 8 * lh;  // this lane's query row (branch 0)
    // the opaque zero keeps these loop-invariant reads inside the tile loop instead of pinning 32 registers
    auto qf = [=](int br, int, int kk) { return lds16(sq + opaque_zero() + br * C::QB * C::KP + 16 * kk); };
    if (plan.fast)
      band_loop<D, true>(xb, rs, HD, h, S, window, half, q0, cosT, sinT, ka2, sdyt + 2 * D, sdyt + 3 * D, smem, qf,
                         o, lsum, plan.c);
    else
      band_loop<D, false>(xb, rs, HD, h, S, window, half, q0, cosT, sinT, ka2, sdyt + 2 * D, sdyt + 3 * D, smem, qf,
                          o, lsum, plan.c);
  } else {
    __syncthreads();
    u32x4 qr[2][D / 16];
#pragma unroll
    for (int br = 0; br < 2; ++br)
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk)
        qr[br][kk] = lds16(smem + (br * C::QB + 32 * wave + lr) * C::KP + 16 * kk + 8 * lh);
    __syncthreads();  // the tile buffers alias the staging area
    auto qf = [&](int br, int, int kk) { return qr[br][kk]; };
    if (plan.fast)
      band_loop<D, true>(xb, rs, HD, h, S, window, half, q0, cosT, sinT, ka2, sdyt + 2 * D, sdyt + 3 * D, smem, qf,
                         o, lsum, plan.c);
    else
      band_loop<D, false>(xb, rs, HD, h, S, window, half, q0, cosT, sinT, ka2, sdyt + 2 * D, sdyt + 3 * D, smem, qf,
                          o, lsum, plan.c);
  }

  const int q = q0 + 32 * wave + lr;
  uint16_t* orow = q < S ? out + (static_cast<int64_t>(b) * S + q) * HD + h * D : nullptr;
  store_diff_bf16<D, 1>(orow, o, lsum, 0, lam ? lam[h] : 1.f);
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
  if (half % 8 != 0) return fail(HB_ERR_HALF, "band kernel needs half %% 8 == 0 (half=%d)", half);
  // A half-width of S or more reaches every key; clamping keeps the kernels' key-range arithmetic within int.
  if (window > S) window = S;
  if (reinterpret_cast<uintptr_t>(qkv) % 16) return fail(HB_ERR_STRIDE, "qkv must be 16-byte aligned");
  if (half > 0 && (reinterpret_cast<uintptr_t>(cos) % 16 || reinterpret_cast<uintptr_t>(sin) % 16))
    return fail(HB_ERR_STRIDE, "cos and sin must be 16-byte aligned");
  if (dtype == HB_F32) {
    if (reinterpret_cast<uintptr_t>(out) % 16) return fail(HB_ERR_STRIDE, "fp32 out must be 16-byte aligned");
    return launch_band_f32(stream, qkv, row_stride, q_dyt, k_dyt, cos, sin, half, window, lam, out, B, S, H, D);
  }
  if (reinterpret_cast<uintptr_t>(out) % 8) return fail(HB_ERR_STRIDE, "out must be 8-byte aligned");
  if (band_ring_supported(dtype, D, half, window))
    return launch_band_ring(stream, qkv, row_stride, q_dyt, k_dyt, cos, sin, half, window, lam, out, B, S, H);
  const int nblocks = B * H * ((S + BandCfg<64>::QB - 1) / BandCfg<64>::QB);
  const uint16_t* x = static_cast<const uint16_t*>(qkv);
  uint16_t* o = static_cast<uint16_t*>(out);
  if (D == 64)
    hipLaunchKernelGGL(band_attend_bf16<64>, dim3(nblocks), dim3(BandCfg<64>::NT), 0, stream, x, row_stride, B, S, H,
                       window, q_dyt, k_dyt, cos, sin, half, lam, o);
  else
    hipLaunchKernelGGL(band_attend_bf16<128>, dim3(nblocks), dim3(BandCfg<128>::NT), 0, stream, x, row_stride, B, S,
                       H, window, q_dyt, k_dyt, cos, sin, half, lam, o);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HB_ERR_LAUNCH, "band_attend launch failed: %s", hipGetErrorString(e));
  return HB_OK;
}
