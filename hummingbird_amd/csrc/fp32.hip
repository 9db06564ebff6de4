// fp32 inputs: the dense and band differential attentions computed in fp32 throughout.
//
// This is the parity path of the reference's FP32_PARITY preset (sa3jax/dtypes.py:41-49), under which every
// cast of the XLA chain is a no-op: RMSNorm or DyT, RoPE, the logits, the softmax, P V and the subtraction all
// stay fp32 (sa3jax/dit.py:45-57, 90-98, 113-119, 146; sa3jax/same_l.py:58-69, 92-100, 134-148, 168-169).
// Nothing is rounded to bf16, so both products run on the fp32 matrix cores (v_mfma_f32_32x32x2_f32):
//
//   S^T[key][query] = K Q^T   A = K rows from LDS, B = q held in registers; the reduction over d is split as
//                             d = (D/2) * (lane / 32) + j, so each lane reads one contiguous half-row of K
//   P = exp2(S^T c - m)       c = log2(e)/sqrt(D), m the running max of S^T c (online softmax), one FMA per
//                             score; masked scores are -inf and give exactly 0
//   O^T[d][query] += V^T P^T  A = V rows from LDS (lane reads V[key][d], consecutive d across lanes), B = P
//                             straight from the S^T accumulators (their keys are the MFMA's k index)
//
// Work split: a workgroup (4 waves) owns 64 queries of one (batch, head); waves 0-1 run branch 1 on 32 queries
// each, waves 2-3 branch 2, and the branch-2 waves hand lam * O2 / l2 to the branch-1 waves through LDS. Keys
// stream through LDS in 64-key tiles (K, K_diff, V). The dense kernel reads the fp32 workspace written by its
// prep kernel. The band call prepares every key once into a workspace (band_keys_f32: DyT with the device tanhf,
// RoPE) and streams the prepared tiles (band_attend_ws_f32, the next tile fetched into registers while the current
// one is attended); without a workspace it prepares the K / K_diff tiles
// of each query block's window itself (band_attend_f32).
#include "api.h"
#include "attn_tile.h"
#include "common.h"

namespace hb {

template <int D>
struct F32Tile {
  static constexpr int KP = D + 4;  // row pitch in floats: conflict-free 16-byte K reads down a column of rows
  static constexpr int TILE = 64 * KP;
  static constexpr int LDS_FLOATS = 3 * TILE;  // K, K_diff, V
  static constexpr int XBUF = 2 * (D / 32) * 16 * 64;  // epilogue hand-over, aliases the tiles
  static_assert(XBUF <= LDS_FLOATS, "epilogue buffer must fit in the tile area");
};

__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }

// The next 64-key tile of prepared K, K_diff and V (three workspace regions of D-float rows) held in registers:
// fetched from global memory while the current tile is attended, stored into the LDS tile rows after the
// barrier that retires it, so the loads' latency is hidden behind the tile's MFMAs.
template <int D>
struct TileRegs {
  f32x4 v[3][D / 16];
  __device__ __forceinline__ void fetch(const float* const (&src)[3], int k0) {
#pragma unroll
    for (int s3 = 0; s3 < 3; ++s3)
#pragma unroll
      for (int i = 0; i < D / 16; ++i) {
        const int ch = threadIdx.x + 256 * i, row = ch / (D / 4), col = (ch % (D / 4)) * 4;
        v[s3][i] = ld4(src[s3] + static_cast<int64_t>(k0 + row) * D + col);
      }
  }
  __device__ __forceinline__ void store(float* __restrict__ smem) const {
#pragma unroll
    for (int s3 = 0; s3 < 3; ++s3)
#pragma unroll
      for (int i = 0; i < D / 16; ++i) {
        const int ch = threadIdx.x + 256 * i, row = ch / (D / 4), col = (ch % (D / 4)) * 4;
        st4(smem + s3 * F32Tile<D>::TILE + row * F32Tile<D>::KP + col, v[s3][i]);
      }
  }
};

// One 64-key tile for one wave: 32 queries (lane % 32) of one branch. `valid(k)` says whether key k of the tile
// (0..63) takes part for this lane's query.
template <int D, class Valid>
__device__ __forceinline__ void attend_tile_f32(const float* __restrict__ sK, const float* __restrict__ sV,
                                                const float (&qreg)[D / 2], f32x16 (&o)[D / 32], float& lsum,
                                                float& m, float c, Valid valid) {
  constexpr int KP = F32Tile<D>::KP;
  const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5;
  f32x16 s[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    s[rt] = f32x16{};
    const float* krow = sK + (32 * rt + lr) * KP + lh * (D / 2);
#pragma unroll
    for (int j4 = 0; j4 < D / 8; ++j4) {
      const f32x4 kv = ld4(krow + 4 * j4);
#pragma unroll
      for (int e = 0; e < 4; ++e) s[rt] = mfma_f32_32x32x2(kv[e], qreg[4 * j4 + e], s[rt]);
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float v = valid(acc_key(rt, r, lh)) ? s[rt][r] : -INFINITY;
      s[rt][r] = v;
      mx = fmaxf(mx, v);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
  const float mnew = fmaxf(m, mx * c);
  const float muse = mnew == -INFINITY ? 0.f : mnew;  // a query with no valid key so far keeps O = l = 0
  const float alpha = fast_exp2(m - muse);
  m = mnew;
  lsum *= alpha;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) o[dt] *= alpha;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(__fmaf_rn(s[rt][r], c, -muse));
      s[rt][r] = p;
      lsum += p;
    }
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float* vrow = sV + acc_key(rt, j, lh) * KP + lr;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) o[dt] = mfma_f32_32x32x2(vrow[32 * dt], s[rt][j], o[dt]);
    }
}

// Epilogue shared by both kernels: out[q] = O1 / l1 - lam * O2 / l2 in fp32, each product rounded on its own so
// that identical branches cancel exactly. Must follow a barrier after the last use of the tiles.
template <int D>
__device__ __forceinline__ void store_diff_f32(float* __restrict__ smem, const f32x16 (&o)[D / 32], float lsum,
                                               int br, float lamh, float* __restrict__ orow) {
  const int lane = threadIdx.x & 63, lh = lane >> 5, wave = wave_id();
  const int slot0 = (wave & 1) * (D / 32) * 16;
  const float inv = __frcp_rn(lsum + __shfl_xor(lsum, 32, kWave));
  if (br == 1) {
    const float i1 = __fmul_rn(lamh, inv);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) smem[(slot0 + dt * 16 + r) * 64 + lane] = __fmul_rn(o[dt][r], i1);
  }
  __syncthreads();
  if (br == 0 && orow) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * g + j;
          v[j] = __fsub_rn(__fmul_rn(o[dt][r], inv), smem[(slot0 + dt * 16 + r) * 64 + lane]);
        }
        st4(orow + 32 * dt + 8 * g + 4 * lh, v);
      }
  }
}

// RMSNorm (dit.py:45-57) and rotate-half RoPE (dit.py:90-98) of k and k_diff and V * mask for 64 tokens of one
// head, all in fp32, into the workspace regions k', k_diff', v'. Thread task = (token, RoPE group pair) as in the
// bf16 prep: the rotation partner of every dim is in the thread's own registers.
template <int D>
__global__ __launch_bounds__(256) void dense_prep_f32(const float* __restrict__ qkv, int64_t rs, int sk, int skd,
                                                      int sv, const float* __restrict__ kw,
                                                      const float* __restrict__ cosT,
                                                      const float* __restrict__ sinT,
                                                      int half, const float* __restrict__ vmask, int L, int Lp, int H,
                                                      float eps, int64_t region, float* __restrict__ ws) {
  constexpr int PAIRS = D / 16;
  constexpr int TASKS = 64 * PAIRS / 256;
  constexpr int VCH = 64 * D / 4 / 256;
  const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z, t = threadIdx.x;
  const int l0 = tile * 64;
  const int64_t bh = static_cast<int64_t>(b) * H + h;
  const int64_t HD = static_cast<int64_t>(H) * D;
  const int h8 = half / 8;
#pragma unroll
  for (int i = 0; i < TASKS; ++i) {
    const int task = t + 256 * i, p = task % PAIRS, l = l0 + task / PAIRS;
    int m1, m2;
    pair_groups(p, h8, m1, m2);
    const bool rot = p < h8, in = l < L;
    const float* row = qkv + (static_cast<int64_t>(b) * L + (in ? l : 0)) * rs + h * D;
    float c[8] = {}, s[8] = {};
    if (rot && in) {
      const float* cp = cosT + static_cast<int64_t>(l) * half + 8 * m1;
      const float* sp = sinT + static_cast<int64_t>(l) * half + 8 * m1;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        c[j] = cp[j];
        s[j] = sp[j];
      }
    }
#pragma unroll
    for (int si = 0; si < 2; ++si) {
      const int sec = si == 0 ? sk : skd;
      const float* w = kw;
      float x1[8] = {}, x2[8] = {};
      if (in) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          x1[j] = row[sec * HD + 8 * m1 + j];
          x2[j] = row[sec * HD + 8 * m2 + j];
        }
      }
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __fmaf_rn(x2[j], x2[j], __fmaf_rn(x1[j], x1[j], ss));
#pragma unroll
      for (int off = 1; off < PAIRS; off <<= 1) ss += __shfl_xor(ss, off, kWave);
      const float inv = rsqrtf(ss / static_cast<float>(D) + eps);
      float o1[8], o2[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float y1 = __fmul_rn(__fmul_rn(x1[j], inv), w[8 * m1 + j]);
        const float y2 = __fmul_rn(__fmul_rn(x2[j], inv), w[8 * m2 + j]);
        if (rot) {
          o1[j] = __fadd_rn(__fmul_rn(y1, c[j]), __fmul_rn(-y2, s[j]));
          o2[j] = __fadd_rn(__fmul_rn(y2, c[j]), __fmul_rn(y1, s[j]));
        } else {
          o1[j] = y1;
          o2[j] = y2;
        }
        if (!in) o1[j] = o2[j] = 0.f;
      }
      float* dst = ws + si * region + (bh * Lp + l) * D;
      st4(dst + 8 * m1, f32x4{o1[0], o1[1], o1[2], o1[3]});
      st4(dst + 8 * m1 + 4, f32x4{o1[4], o1[5], o1[6], o1[7]});
      st4(dst + 8 * m2, f32x4{o2[0], o2[1], o2[2], o2[3]});
      st4(dst + 8 * m2 + 4, f32x4{o2[4], o2[5], o2[6], o2[7]});
    }
  }
#pragma unroll
  for (int i = 0; i < VCH; ++i) {
    const int ch = t + 256 * i, key = ch / (D / 4), col = (ch % (D / 4)) * 4, l = l0 + key;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    if (l < L) {
      v = ld4(qkv + (static_cast<int64_t>(b) * L + l) * rs + sv * HD + h * D + col);
      v *= vmask ? vmask[static_cast<int64_t>(b) * L + l] : 1.f;
    }
    st4(ws + 2 * region + (bh * Lp + l) * D + col, v);
  }
}

template <int D>
__global__ __launch_bounds__(256) void dense_attend_f32(const float* __restrict__ qkv, int64_t rs, int sqd,
                                                        const float* __restrict__ qw, const float* __restrict__ cosT,
                                                        const float* __restrict__ sinT, int half, float eps,
                                                        const float* __restrict__ ws, int64_t region, int B, int L,
                                                        int Lp, int Lk, int Lkp, int H,
                                                        const float* __restrict__ lam, float* __restrict__ out) {
  using T = F32Tile<D>;
  __shared__ __attribute__((aligned(16))) float smem[T::LDS_FLOATS];
  const int nqb = Lp / 64;
  const int tile = xcd_remap(blockIdx.x, B * H * nqb);
  const int qb = tile % nqb, bh = tile / nqb, h = bh % H, b = bh / H;
  const int lane = threadIdx.x & 63, wave = wave_id(), lr = lane & 31, lh = lane >> 5;
  const int br = wave >> 1, q0 = qb * 64 + (wave & 1) * 32;
  const int64_t rowbase = static_cast<int64_t>(bh) * Lkp;

  // RMSNorm (dit.py:45-57) and rotate-half RoPE (dit.py:90-98) of this lane's half row (dims lh D/2 ..) of q
  // (branch 1, section 0) or q_diff (branch 2, section sqd), from qkv; the RoPE partner (d +- half) of each group
  // of 4 dims is loaded directly. Rows at or past L give zeros.
  float qreg[D / 2];
  {
    const int q = q0 + lr, qc = q < L ? q : L - 1, h4 = half / 4;
    const float* row = qkv + (static_cast<int64_t>(b) * L + qc) * rs + static_cast<int64_t>(br ? sqd : 0) * H * D + h * D;
    float xp[D / 2];
    float ss = 0.f;
#pragma unroll
    for (int j4 = 0; j4 < D / 8; ++j4) {
      const int g = lh * (D / 8) + j4;
      const int pg = g < h4 ? g + h4 : g < 2 * h4 ? g - h4 : g;
      const f32x4 v = ld4(row + 4 * g), p = ld4(row + 4 * pg);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qreg[4 * j4 + e] = v[e];
        xp[4 * j4 + e] = p[e];
        ss = __fmaf_rn(v[e], v[e], ss);
      }
    }
    ss += __shfl_xor(ss, 32, kWave);
    const float inv = rsqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
    for (int j = 0; j < D / 2; ++j) {
      const int d = lh * (D / 2) + j;
      const bool first = d < half, rot = d < 2 * half;
      const int pd = first ? d + half : rot ? d - half : d;
      const float y = __fmul_rn(__fmul_rn(qreg[j], inv), qw[d]);
      const float yp = __fmul_rn(__fmul_rn(xp[j], inv), qw[pd]);
      float r = y;
      if (rot) {  // d < half takes -x[d + half], d >= half takes x[d - half]
        const int64_t t = static_cast<int64_t>(qc) * half + (first ? d : d - half);
        r = first ? __fadd_rn(__fmul_rn(y, cosT[t]), __fmul_rn(-yp, sinT[t]))
                  : __fadd_rn(__fmul_rn(y, cosT[t]), __fmul_rn(yp, sinT[t]));
      }
      qreg[j] = q < L ? r : 0.f;
    }
  }
  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) o[dt] = f32x16{};
  float lsum = 0.f, m = -INFINITY;
  const float c = kLog2e / sqrtf(static_cast<float>(D));

  const float* src[3] = {ws + rowbase * D, ws + region + rowbase * D, ws + 2 * region + rowbase * D};
  const int nkt = (Lk + 63) / 64;
  // Loaded through registers into one LDS stage per tile: a register prefetch of the next tile (TileRegs, as in the
  // band kernel) measured 1.6 % slower here, where the 48 extra registers leave the waves less room.
  for (int t = 0; t < nkt; ++t) {
    // 3 tensors x 64 rows x D floats; rows past Lk are the zero padding of the workspace (t * 64 + 63 < Lkp)
#pragma unroll
    for (int s3 = 0; s3 < 3; ++s3)
#pragma unroll
      for (int i = 0; i < D / 16; ++i) {
        const int ch = threadIdx.x + 256 * i, row = ch / (D / 4), col = (ch % (D / 4)) * 4;
        st4(smem + s3 * T::TILE + row * T::KP + col, ld4(src[s3] + static_cast<int64_t>(t * 64 + row) * D + col));
      }
    __syncthreads();
    const int k0 = t * 64;
    attend_tile_f32<D>(smem + br * T::TILE, smem + 2 * T::TILE, qreg, o, lsum, m, c,
                       [&](int k) { return k0 + k < Lk; });
    __syncthreads();
  }
  const int q = q0 + lr;
  float* orow = q < L ? out + (static_cast<int64_t>(b) * L + q) * (static_cast<int64_t>(H) * D) + h * D : nullptr;
  store_diff_f32<D>(smem, o, lsum, br, lam ? lam[h] : 1.f, orow);
}

// DyT (same_l.py:58-69) and RoPE (same_l.py:92-100) in fp32 of two tensors (sections secA, secB) for the 64
// positions pos0 .. pos0+63 into rows of pitch P floats (LDS rows by default, or workspace rows); positions
// outside [0, S) give zero rows. `dyt` = [alpha, gamma[0..D), beta[0..D)].
template <int D, int P = F32Tile<D>::KP>
__device__ __forceinline__ void band_prep_f32(const float* __restrict__ xb, int64_t rs, int64_t offA, int64_t offB,
                                              int pos0, int S, int half, const float* __restrict__ dyt,
                                              const float* __restrict__ cosT, const float* __restrict__ sinT,
                                              float* __restrict__ dA, float* __restrict__ dB) {
  constexpr int PAIRS = D / 16, TASKS = 64 * PAIRS / 256, KP = P;
  const int h8 = half / 8;
  const float alpha = dyt[0];
  const float* gamma = dyt + 1;
  const float* beta = dyt + 1 + D;
#pragma unroll
  for (int i = 0; i < TASKS; ++i) {
    const int task = threadIdx.x + 256 * i, p = task % PAIRS, r = task / PAIRS, pos = pos0 + r;
    int m1, m2;
    pair_groups(p, h8, m1, m2);
    const bool rot = p < h8, in = pos >= 0 && pos < S;
    float c[8] = {}, s[8] = {};
    if (rot && in) {
      const float* cp = cosT + static_cast<int64_t>(pos) * half + 8 * m1;
      const float* sp = sinT + static_cast<int64_t>(pos) * half + 8 * m1;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        c[j] = cp[j];
        s[j] = sp[j];
      }
    }
    const float* row = xb + static_cast<int64_t>(in ? pos : 0) * rs;
#pragma unroll
    for (int tsr = 0; tsr < 2; ++tsr) {
      const float* x = row + (tsr ? offB : offA);
      float* dst = (tsr ? dB : dA) + r * KP;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int d1 = 8 * m1 + j, d2 = 8 * m2 + j;
        const float y1 = in ? __fadd_rn(__fmul_rn(gamma[d1], tanhf(__fmul_rn(alpha, x[d1]))), beta[d1]) : 0.f;
        const float y2 = in ? __fadd_rn(__fmul_rn(gamma[d2], tanhf(__fmul_rn(alpha, x[d2]))), beta[d2]) : 0.f;
        if (rot) {
          dst[d1] = __fadd_rn(__fmul_rn(y1, c[j]), __fmul_rn(-y2, s[j]));
          dst[d2] = __fadd_rn(__fmul_rn(y2, c[j]), __fmul_rn(y1, s[j]));
        } else {
          dst[d1] = y1;
          dst[d2] = y2;
        }
      }
    }
  }
}

template <int D>
__global__ __launch_bounds__(256) void band_attend_f32(const float* __restrict__ qkv, int64_t rs, int B, int S, int H,
                                                       int w, const float* __restrict__ qdyt,
                                                       const float* __restrict__ kdyt, const float* __restrict__ cosT,
                                                       const float* __restrict__ sinT, int half,
                                                       const float* __restrict__ lam, float* __restrict__ out) {
  using T = F32Tile<D>;
  __shared__ __attribute__((aligned(16))) float smem[T::LDS_FLOATS];
  // query-block-major order: the heads of one query block run together and share key rows in L2
  const int qb = blockIdx.x / (B * H), bh = blockIdx.x % (B * H), h = bh % H, b = bh / H;
  const int lane = threadIdx.x & 63, wave = wave_id(), lr = lane & 31, lh = lane >> 5;
  const int br = wave >> 1, q0 = qb * 64, qw0 = q0 + (wave & 1) * 32, q = qw0 + lr;
  const int64_t HD = static_cast<int64_t>(H) * D;
  const float* xb = qkv + static_cast<int64_t>(b) * S * rs + h * D;
  float* sA = smem;
  float* sB = smem + T::TILE;
  float* sV = smem + 2 * T::TILE;

  // q and q_diff of the block, then each wave takes its branch's half-rows into registers
  band_prep_f32<D>(xb, rs, 0, 3 * HD, q0, S, half, qdyt, cosT, sinT, sA, sB);
  __syncthreads();
  float qreg[D / 2];
  const float* qrow = (br ? sB : sA) + ((wave & 1) * 32 + lr) * T::KP + lh * (D / 2);
#pragma unroll
  for (int j4 = 0; j4 < D / 8; ++j4) {
    const f32x4 v = ld4(qrow + 4 * j4);
#pragma unroll
    for (int e = 0; e < 4; ++e) qreg[4 * j4 + e] = v[e];
  }
  __syncthreads();

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) o[dt] = f32x16{};
  float lsum = 0.f, m = -INFINITY;
  const float c = kLog2e / sqrtf(static_cast<float>(D));
  const int kbeg = q0 - w > 0 ? q0 - w : 0;
  const int kend = q0 + 64 + w < S ? q0 + 64 + w : S;
  for (int k0 = kbeg; k0 < kend; k0 += 64) {
    band_prep_f32<D>(xb, rs, HD, 4 * HD, k0, S, half, kdyt, cosT, sinT, sA, sB);
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
      const int ch = threadIdx.x + 256 * i, row = ch / (D / 4), col = (ch % (D / 4)) * 4, pos = k0 + row;
      st4(sV + row * T::KP + col, pos < S ? ld4(xb + static_cast<int64_t>(pos) * rs + 2 * HD + col)
                                          : f32x4{0.f, 0.f, 0.f, 0.f});
    }
    __syncthreads();
    // the tile reaches this wave's band iff k0 <= qw0 + 31 + w and k0 + 63 >= qw0 - w
    if (k0 <= qw0 + 31 + w && k0 + 63 >= qw0 - w)
      attend_tile_f32<D>(br ? sB : sA, sV, qreg, o, lsum, m, c, [&](int k) {
        const int kk = k0 + k, dist = kk - q;
        return kk < S && dist <= w && -dist <= w;
      });
    __syncthreads();
  }
  float* orow = q < S ? out + (static_cast<int64_t>(b) * S + q) * HD + h * D : nullptr;
  store_diff_f32<D>(smem, o, lsum, br, lam ? lam[h] : 1.f, orow);
}

// The keys of the band prepared once: DyT and RoPE of k and k_diff (the same steps as band_prep_f32 inside
// band_attend_f32) and V as it is, for 64-key tile blockIdx.x of (batch blockIdx.z, head blockIdx.y), into the
// fp32 workspace regions k', k_diff', v' (rows of D floats, Sp rows per (batch, head), zeros past S).
template <int D>
__global__ __launch_bounds__(256) void band_keys_f32(const float* __restrict__ qkv, int64_t rs, int S, int Sp, int H,
                                                     const float* __restrict__ kdyt, const float* __restrict__ cosT,
                                                     const float* __restrict__ sinT, int half, int64_t region,
                                                     float* __restrict__ ws) {
  const int t = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t HD = static_cast<int64_t>(H) * D, bh = static_cast<int64_t>(b) * H + h;
  const float* xb = qkv + static_cast<int64_t>(b) * S * rs + h * D;
  float* kA = ws + (bh * Sp + 64 * t) * D;
  band_prep_f32<D, D>(xb, rs, HD, 4 * HD, 64 * t, S, half, kdyt, cosT, sinT, kA, kA + region);
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    const int ch = threadIdx.x + 256 * i, row = ch / (D / 4), col = (ch % (D / 4)) * 4, pos = 64 * t + row;
    st4(ws + 2 * region + (bh * Sp + pos) * D + col,
        pos < S ? ld4(xb + static_cast<int64_t>(pos) * rs + 2 * HD + col) : f32x4{0.f, 0.f, 0.f, 0.f});
  }
}

// band_attend_f32 over prepared keys: the 64-aligned key tiles that meet the block's band are loaded from the
// workspace of band_keys_f32 instead of being prepared per query block.
template <int D>
__global__ __launch_bounds__(256) void band_attend_ws_f32(const float* __restrict__ qkv, int64_t rs, int B, int S,
                                                          int Sp, int H, int w, const float* __restrict__ qdyt,
                                                          const float* __restrict__ cosT,
                                                          const float* __restrict__ sinT, int half,
                                                          const float* __restrict__ ws, int64_t region,
                                                          const float* __restrict__ lam, float* __restrict__ out) {
  using T = F32Tile<D>;
  __shared__ __attribute__((aligned(16))) float smem[T::LDS_FLOATS];
  // query-block-major order: the heads of one query block run together and share key rows in L2
  const int qb = blockIdx.x / (B * H), bh = blockIdx.x % (B * H), h = bh % H, b = bh / H;
  const int lane = threadIdx.x & 63, wave = wave_id(), lr = lane & 31, lh = lane >> 5;
  const int br = wave >> 1, q0 = qb * 64, qw0 = q0 + (wave & 1) * 32, q = qw0 + lr;
  const int64_t HD = static_cast<int64_t>(H) * D;
  const float* xb = qkv + static_cast<int64_t>(b) * S * rs + h * D;

  band_prep_f32<D>(xb, rs, 0, 3 * HD, q0, S, half, qdyt, cosT, sinT, smem, smem + T::TILE);
  __syncthreads();
  float qreg[D / 2];
  const float* qrow = smem + br * T::TILE + ((wave & 1) * 32 + lr) * T::KP + lh * (D / 2);
#pragma unroll
  for (int j4 = 0; j4 < D / 8; ++j4) {
    const f32x4 v = ld4(qrow + 4 * j4);
#pragma unroll
    for (int e = 0; e < 4; ++e) qreg[4 * j4 + e] = v[e];
  }
  __syncthreads();

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) o[dt] = f32x16{};
  float lsum = 0.f, m = -INFINITY;
  const float c = kLog2e / sqrtf(static_cast<float>(D));
  const int64_t rowbase = static_cast<int64_t>(bh) * Sp;
  const float* const src[3] = {ws + rowbase * D, ws + region + rowbase * D, ws + 2 * region + rowbase * D};
  const int kbeg = (q0 - w > 0 ? q0 - w : 0) / 64 * 64;
  const int kend = q0 + 64 + w < S ? q0 + 64 + w : S;
  TileRegs<D> nxt;  // every tile's rows k0 .. k0 + 63 lie below Sp: Sp is a multiple of 128 and k0 < S
  nxt.fetch(src, kbeg);
  nxt.store(smem);
  __syncthreads();
  for (int k0 = kbeg; k0 < kend; k0 += 64) {
    const bool more = k0 + 64 < kend;
    if (more) nxt.fetch(src, k0 + 64);
    if (k0 <= qw0 + 31 + w && k0 + 63 >= qw0 - w)
      attend_tile_f32<D>(smem + br * T::TILE, smem + 2 * T::TILE, qreg, o, lsum, m, c, [&](int k) {
        const int kk = k0 + k, dist = kk - q;
        return kk < S && dist <= w && -dist <= w;
      });
    __syncthreads();
    if (more) {
      nxt.store(smem);
      __syncthreads();
    }
  }
  float* orow = q < S ? out + (static_cast<int64_t>(b) * S + q) * HD + h * D : nullptr;
  store_diff_f32<D>(smem, o, lsum, br, lam ? lam[h] : 1.f, orow);
}

static int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HB_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return HB_OK;
}

int launch_dense_prep_f32(hipStream_t stream, const void* qkv, int64_t rs, int sk, int skd, int sv, const float* kw,
                          const float* cosT, const float* sinT, int half, const float* vmask, int B, int L, int H, int D,
                          float eps, const DenseLayout& lay, void* ws) {
  const dim3 grid(static_cast<unsigned>(lay.Lp / 64), static_cast<unsigned>(H), static_cast<unsigned>(B));
  const float* x = static_cast<const float*>(qkv);
  float* w = static_cast<float*>(ws);
  const int Lp = static_cast<int>(lay.Lp);
  if (D == 64)
    hipLaunchKernelGGL(dense_prep_f32<64>, grid, dim3(256), 0, stream, x, rs, sk, skd, sv, kw, cosT, sinT, half, vmask,
                       L, Lp, H, eps, lay.region_elems, w);
  else
    hipLaunchKernelGGL(dense_prep_f32<128>, grid, dim3(256), 0, stream, x, rs, sk, skd, sv, kw, cosT, sinT, half,
                       vmask, L, Lp, H, eps, lay.region_elems, w);
  return launched("dense_prep_f32");
}

int launch_dense_attend_f32(hipStream_t stream, const void* qkv, int64_t rs, int sqd, const float* qw,
                            const float* cosT, const float* sinT, int half, float eps, const void* ws, const float* lam,
                            void* out, int B, int L, int Lk, int H, int D, const DenseLayout& lay) {
  const int Lp = (L + 127) / 128 * 128;
  const int nblocks = B * H * (Lp / 64);
  const float* x = static_cast<const float*>(qkv);
  const float* w = static_cast<const float*>(ws);
  float* o = static_cast<float*>(out);
  const int Lkp = static_cast<int>(lay.Lp);
  if (D == 64)
    hipLaunchKernelGGL(dense_attend_f32<64>, dim3(nblocks), dim3(256), 0, stream, x, rs, sqd, qw, cosT, sinT, half, eps,
                       w, lay.region_elems, B, L, Lp, Lk, Lkp, H, lam, o);
  else
    hipLaunchKernelGGL(dense_attend_f32<128>, dim3(nblocks), dim3(256), 0, stream, x, rs, sqd, qw, cosT, sinT, half,
                       eps, w, lay.region_elems, B, L, Lp, Lk, Lkp, H, lam, o);
  return launched("dense_attend_f32");
}

int launch_band_f32_ws(hipStream_t stream, const void* qkv, int64_t rs, const float* qdyt, const float* kdyt,
                       const float* cosT, const float* sinT, int half, int window, const float* lam, void* out, int B,
                       int S, int H, int D, void* workspace) {
  const DenseLayout lay = dense_layout(HB_F32, B, S, H, D);
  const int Sp = static_cast<int>(lay.Lp);
  const float* x = static_cast<const float*>(qkv);
  float* ws = static_cast<float*>(workspace);
  float* o = static_cast<float*>(out);
  const dim3 kgrid(static_cast<unsigned>(Sp / 64), static_cast<unsigned>(H), static_cast<unsigned>(B));
  const int nblocks = B * H * ((S + 63) / 64);
  if (D == 64) {
    hipLaunchKernelGGL(band_keys_f32<64>, kgrid, dim3(256), 0, stream, x, rs, S, Sp, H, kdyt, cosT, sinT, half,
                       lay.region_elems, ws);
    hipLaunchKernelGGL(band_attend_ws_f32<64>, dim3(nblocks), dim3(256), 0, stream, x, rs, B, S, Sp, H, window, qdyt,
                       cosT, sinT, half, ws, lay.region_elems, lam, o);
  } else {
    hipLaunchKernelGGL(band_keys_f32<128>, kgrid, dim3(256), 0, stream, x, rs, S, Sp, H, kdyt, cosT, sinT, half,
                       lay.region_elems, ws);
    hipLaunchKernelGGL(band_attend_ws_f32<128>, dim3(nblocks), dim3(256), 0, stream, x, rs, B, S, Sp, H, window,
                       qdyt, cosT, sinT, half, ws, lay.region_elems, lam, o);
  }
  return launched("band_attend_ws_f32");
}

int launch_band_f32(hipStream_t stream, const void* qkv, int64_t rs, const float* qdyt, const float* kdyt,
                    const float* cosT, const float* sinT, int half, int window, const float* lam, void* out, int B,
                    int S, int H, int D) {
  const int nblocks = B * H * ((S + 63) / 64);
  const float* x = static_cast<const float*>(qkv);
  float* o = static_cast<float*>(out);
  if (D == 64)
    hipLaunchKernelGGL(band_attend_f32<64>, dim3(nblocks), dim3(256), 0, stream, x, rs, B, S, H, window, qdyt, kdyt,
                       cosT, sinT, half, lam, o);
  else
    hipLaunchKernelGGL(band_attend_f32<128>, dim3(nblocks), dim3(256), 0, stream, x, rs, B, S, H, window, qdyt, kdyt,
                       cosT, sinT, half, lam, o);
  return launched("band_attend_f32");
}

}  // namespace hb
