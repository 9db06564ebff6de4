// DiT dense differential self-attention for gfx950 (MI355X).
//
// Replaces the reference's fused TPU kernel sa3jax/dense_attention.py:43-153 and the XLA chain
// sa3jax/dit.py:185-200. Two kernels run back to back on the caller's stream:
//
//   dense_prep    one pass over the key side of qkv: per-head RMSNorm (dit.py:45-57) and rotate-half RoPE
//                 (dit.py:90-98) of k and k_diff, and V * mask (dit.py:174-175), written in bf16 to a workspace;
//                 V is stored transposed per 64-key tile, in the order the PV MFMA consumes it.
//   dense_attend  flash-style single pass per (batch, head, 128-query block). Each lane first prepares one
//                 query row straight from qkv (RMSNorm, RoPE and the softmax scale, the same cast points), so
//                 q and q_diff never round-trip through HBM. K, K_diff and V tiles of 64 keys are then
//                 double-buffered through LDS; S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_32x32x16_bf16 with
//                 fp32 accumulation; both branches share each V tile; scores never leave registers; the
//                 subtraction is done in fp32 with one cast (dense_attention.py:94).
//
// Softmax without a running max. The logits are bounded a priori: after RMSNorm every row has
// |x| <= sqrt(D) * max|w|, and RoPE is a rotation, so |s| <= D * max|w_q| * max|w_k| * log2(e)/sqrt(D). When
// that bound is <= 64 (true for unit-scale gains: about 11.5), exp2(s) lies in [2^-64, 2^64] and needs no
// max subtraction, which removes a compare and a subtract per score. Larger gains take the classic online
// softmax (running max with rescaling) with the reference fused kernel's cast points; the choice is uniform
// for the whole launch (SoftmaxPlan in attn_tile.h).
#include <mutex>
#include <type_traits>

#include "api.h"
#include "attn_tile.h"
#include "common.h"
#include "tiles.h"

namespace hb {

// After RMSNorm a row has |x| <= sqrt(D) * max|w|, so the plan depends only on the two gain vectors and is the
// same for every wave of the launch.
template <int D>
__device__ __forceinline__ SoftmaxPlan dense_plan(const float* __restrict__ qw, const float* __restrict__ kw) {
  const int lane = threadIdx.x & 63;
  float mq = 0.f, mk = 0.f;
  for (int d = lane; d < D; d += 64) {
    mq = fmaxf(mq, fabsf(qw[d]));
    mk = fmaxf(mk, fabsf(kw[d]));
  }
  const float rd = sqrtf(static_cast<float>(D));
  return softmax_plan(rd * wave_max(mq), rd * wave_max(mk), D);
}

// RMSNorm + RoPE of k and k_diff and V * mask for 64 tokens of one head. Thread task = (token, RoPE group pair):
// the thread loads the pair's 16 dims of both key sections and the pair's cos/sin slice once, so every load is
// issued before any arithmetic; the RMS statistic is reduced over the D/16 lanes of a token. RoPE reads the
// (L, half) fp32 tables; `half` is a multiple of 8 (checked on the host). Workspace regions: k', k_diff', V'^T.
// `sk`, `skd`, `sv`: the sections of k, k_diff and v in a row of `qkv`, in units of H * D elements (self-attention
// reads a to_qkv row [q | k | v | q_diff | k_diff], cross-attention a to_kv row [k | k_diff | v]).
// IO: the element type of qkv (bf16 or half); the RMSNorm and RoPE outputs round to it (the compute dtype,
// dense_attention.py:66, 69) and then to bf16 for the workspace (75-77).
template <class IO, int D>
__global__ __launch_bounds__(256) void dense_prep(const uint16_t* __restrict__ qkv, int64_t rs, int sk, int skd, int sv,
                                                  const float* __restrict__ kw, const float* __restrict__ cosT,
                                                  const float* __restrict__ sinT, int half,
                                                  const float* __restrict__ vmask, int L, int Lp, int H, float eps,
                                                  int64_t region, uint16_t* __restrict__ ws) {
  constexpr int PAIRS = D / 16;            // group pairs per row; the lanes of one token are consecutive
  constexpr int TASKS = 64 * PAIRS / 256;  // (token, pair) tasks per thread
  constexpr int VCH = 64 * D / 8 / 256;    // 16-byte V chunks per thread
  const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x;
  const int l0 = tile * 64;
  const int64_t bh = static_cast<int64_t>(b) * H + h;
  const int64_t HD = static_cast<int64_t>(H) * D;
  const int h8 = half / 8;

  // Issue every global load first: 2 sections x 2 groups of data, the cos/sin slice and the V chunks.
  u32x4 raw[TASKS][2][2];
  f32x4 cs[TASKS][4];
  int tm1[TASKS], tm2[TASKS];
  bool trot[TASKS];
#pragma unroll
  for (int i = 0; i < TASKS; ++i) {
    const int task = t + 256 * i, p = task % PAIRS, l = l0 + task / PAIRS;
    pair_groups(p, h8, tm1[i], tm2[i]);
    trot[i] = p < h8;
    const uint16_t* row = qkv + (static_cast<int64_t>(b) * L + (l < L ? l : 0)) * rs + h * D;
#pragma unroll
    for (int si = 0; si < 2; ++si) {
      const int sec = si == 0 ? sk : skd;
      raw[i][si][0] = l < L ? ld16(row + sec * HD + 8 * tm1[i]) : u32x4{0u, 0u, 0u, 0u};
      raw[i][si][1] = l < L ? ld16(row + sec * HD + 8 * tm2[i]) : u32x4{0u, 0u, 0u, 0u};
    }
    if (trot[i] && l < L) {
      const float* c = cosT + static_cast<int64_t>(l) * half + 8 * tm1[i];
      const float* s = sinT + static_cast<int64_t>(l) * half + 8 * tm1[i];
      cs[i][0] = *reinterpret_cast<const f32x4*>(c);
      cs[i][1] = *reinterpret_cast<const f32x4*>(c + 4);
      cs[i][2] = *reinterpret_cast<const f32x4*>(s);
      cs[i][3] = *reinterpret_cast<const f32x4*>(s + 4);
    }
  }
  u32x4 vraw[VCH];
  float vm[VCH];
#pragma unroll
  for (int i = 0; i < VCH; ++i) {
    const int ch = t + 256 * i, l = l0 + ch / (D / 8), col = (ch % (D / 8)) * 8;
    vraw[i] = l < L ? ld16(qkv + (static_cast<int64_t>(b) * L + l) * rs + sv * HD + h * D + col)
                    : u32x4{0u, 0u, 0u, 0u};
    vm[i] = l < L ? (vmask ? vmask[static_cast<int64_t>(b) * L + l] : 1.f) : 0.f;
  }

#pragma unroll
  for (int i = 0; i < TASKS; ++i) {
    const int task = t + 256 * i, l = l0 + task / PAIRS;
    const int m1 = tm1[i], m2 = tm2[i];
#pragma unroll
    for (int si = 0; si < 2; ++si) {
      float x1[8], x2[8];
      IO::unpack8(raw[i][si][0], x1);
      IO::unpack8(raw[i][si][1], x2);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __fmaf_rn(x2[j], x2[j], __fmaf_rn(x1[j], x1[j], ss));
#pragma unroll
      for (int off = 1; off < PAIRS; off <<= 1) ss += __shfl_xor(ss, off, kWave);
      const float inv = rsqrtf(ss / static_cast<float>(D) + eps);
      float y1[8], y2[8], o1[8], o2[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {  // RMSNorm (dit.py:56-57): x * rsqrt(mean + eps), * w, cast
        y1[j] = IO::round((x1[j] * inv) * kw[8 * m1 + j]);
        y2[j] = IO::round((x2[j] * inv) * kw[8 * m2 + j]);
      }
      if (trot[i]) {
        const float c[8] = {cs[i][0][0], cs[i][0][1], cs[i][0][2], cs[i][0][3],
                            cs[i][1][0], cs[i][1][1], cs[i][1][2], cs[i][1][3]};
        const float s[8] = {cs[i][2][0], cs[i][2][1], cs[i][2][2], cs[i][2][3],
                            cs[i][3][0], cs[i][3][1], cs[i][3][2], cs[i][3][3]};
#pragma unroll
        for (int j = 0; j < 8; ++j) {  // rotate_half (dit.py:96-98): d < half takes -x[d+half], else x[d-half]
          o1[j] = IO::round(y1[j] * c[j] + (-y2[j]) * s[j]);
          o2[j] = IO::round(y2[j] * c[j] + y1[j] * s[j]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          o1[j] = y1[j];
          o2[j] = y2[j];
        }
      }
      if (l >= L) {
#pragma unroll
        for (int j = 0; j < 8; ++j) o1[j] = o2[j] = 0.f;
      }
      uint16_t* dst = ws + si * region + (bh * Lp + l) * D;
      st16(dst + 8 * m1, pack8(o1));  // bf16 (exact for bf16 IO; the fused kernel's second cast for half)
      st16(dst + 8 * m2, pack8(o2));
    }
  }

  // V * mask, transposed per 64-key tile (v_tile_key order): the attention kernel then reads its PV operand
  // with full-rate 16-byte LDS loads instead of transposing ones. The tile is staged in LDS row-major first, with
  // the 16-byte chunks of row r XOR-swizzled by (r / 8) % 8: the column reads below take one dim of 8 rows that
  // are 8 apart, which then fall in 8 different chunks (distinct banks) instead of one.
  __shared__ __attribute__((aligned(16))) uint16_t vt[64 * D];
  auto vt_at = [](int row, int col) { return row * D + 8 * ((col >> 3) ^ ((row >> 3) & 7)) + (col & 7); };
#pragma unroll
  for (int i = 0; i < VCH; ++i) {
    const int ch = t + 256 * i, key = ch / (D / 8), col = (ch % (D / 8)) * 8;
    float x[8];
    IO::unpack8(vraw[i], x);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] *= vm[i];
    *reinterpret_cast<u32x4*>(vt + vt_at(key, col)) = pack8(x);
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
    st16(ws + 2 * region + (bh * Lp + l0) * D + d * 64 + pos0, w);
  }
}

// The key loop. Tile 0 has already been issued into stage A by the caller.
template <int D, int QB, int NW, bool FAST>
__device__ __forceinline__ void dense_attend_loop(
    const TileCopy<D, NW>& issue, int L, int br0, uint16_t* sA, uint16_t* sB,
    const u32x4 (&qf)[DenseTile<D, QB, NW>::NB][DenseTile<D, QB, NW>::NCT][D / 16],
    f32x16 (&o)[DenseTile<D, QB, NW>::NB][DenseTile<D, QB, NW>::NCT][D / 32],
    float (&lsum)[DenseTile<D, QB, NW>::NB][DenseTile<D, QB, NW>::NCT], float c) {
  using T = DenseTile<D, QB, NW>;
  constexpr int NB = T::NB, NCT = T::NCT;
  const int tid = threadIdx.x;
  const int nkt = (L + 63) / 64;
  float m[NB][NCT];
#pragma unroll
  for (int br = 0; br < NB; ++br)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) m[br][ct] = -INFINITY;

  // The next tile is copied into the other LDS stage while the current one is attended; one wait and one
  // barrier per tile.
  const int lr = tid & 31, lh = (tid >> 5) & 1;
  auto attend = [&](const uint16_t* s, bool masked, int kt0, auto row_tiles) {
    attend_tile<D, NB, NCT, FAST, decltype(row_tiles)::value>(
        [&](int b, int rt, int kk) { return lds16(s + (br0 + b) * T::K_ELEMS + swz<D>(32 * rt + lr, 2 * kk + lh)); },
        [&](int dt, int g) { return lds16(s + 2 * T::K_ELEMS + swz<64>(32 * dt + lr, 2 * g + lh)); },
        [&](int b, int ct, int kk) { return qf[b][ct][kk]; }, o, lsum, m, c, masked,
        [&](int k, int) { return kt0 + k < L; });
  };

  // Full tiles run unmasked; the ragged last tile (keys >= L do not exist) is peeled off after the loop so the
  // loop body has a single code path and the accumulators keep their registers.
  // The loop is unrolled over the two stages so that both stage addresses are fixed in each half.
  // A copy has landed once this wave's vector-memory counter drains (s_waitcnt 0); the barrier then publishes
  // every wave's copies.
  const int nfull = L / 64;
  const uint32_t ldsA = lds_addr(sA), ldsB = lds_addr(sB);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const std::integral_constant<int, 2> whole;
  const std::integral_constant<int, 1> first_half;
  int t = 0;
  for (; t + 1 < nfull; t += 2) {
    issue(t + 1, ldsB);  // stage B was last read in tile t - 1
    attend(sA, false, 0, whole);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t + 2 < nkt) issue(t + 2, ldsA);
    attend(sB, false, 0, whole);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if (t < nfull) {  // an odd number of full tiles: the last one sits in stage A
    if (t + 1 < nkt) issue(t + 1, ldsB);
    attend(sA, false, 0, whole);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    ++t;
  }
  if (nfull < nkt) {  // the ragged last tile; at D = 64 with at most 32 keys left only its first row tile is
                      // attended (at D = 128 the extra inlined copy would spill registers)
    const uint16_t* s = (nfull & 1) ? sB : sA;
    if (D == 64 && L - nfull * 64 <= 32)
      attend(s, true, nfull * 64, first_half);
    else
      attend(s, true, nfull * 64, whole);
  }
}

// RMSNorm (dit.py:45-57), rotate-half RoPE over the first 2 * 8 H8 dims (dit.py:90-98) and the softmax scale of
// one query row, held whole by this lane: `row` points at its D elements in qkv, `cs` / `sn` at its (half)
// columns of the tables. Cast points are those of the reference fused kernel: the compute dtype IO after the gain
// and after the rotation, bf16 after the scale. The rotary width is a template parameter so that the partner of every dim is a
// fixed register. Rows at or past L are prepared from row L - 1 (the caller clamps `row`); their outputs are
// never stored, and real rows keep the logits within the softmax plan's bound.
template <class IO, int D, int H8, bool STREAM>
__device__ __forceinline__ void prep_q_row(const uint16_t* __restrict__ row, const float* __restrict__ qw,
                                           const float* __restrict__ cs, const float* __restrict__ sn, float eps,
                                           float qscale, u32x4 (&out)[D / 8]) {
  u32x4 raw[D / 8];
#pragma unroll
  for (int c = 0; c < D / 8; ++c) raw[c] = ld16(row + 8 * c);
  float cv[8 * H8 + 1], sv[8 * H8 + 1];
#pragma unroll
  for (int j4 = 0; j4 < (STREAM ? 0 : 2 * H8); ++j4) {  // the streamed form loads its slices chunk by chunk
    const f32x4 c4 = *reinterpret_cast<const f32x4*>(cs + 4 * j4);
    const f32x4 s4 = *reinterpret_cast<const f32x4*>(sn + 4 * j4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      cv[4 * j4 + e] = c4[e];
      sv[4 * j4 + e] = s4[e];
    }
  }
  if constexpr (STREAM) {
    // The same arithmetic chunk pair by chunk pair, so that the whole fp32 row and its tables are never live at
    // once (head_dim 128 with two waves per SIMD, at most 256 registers each).
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      float t[8];
      IO::unpack8(raw[c], t);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __fmaf_rn(t[j], t[j], ss);
    }
    const float inv = rsqrtf(ss / static_cast<float>(D) + eps);
    auto normed = [&](int c, float (&y)[8]) {
      IO::unpack8(raw[c], y);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = IO::round((y[j] * inv) * qw[8 * c + j]);
    };
    auto emit = [&](int c, const float (&y)[8]) {
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = y[j] * qscale;
      out[c] = pack8(o);
    };
#pragma unroll
    for (int c = 0; c < H8; ++c) {  // chunk c rotates with chunk c + H8 (dims d and d + half)
      float y1[8], y2[8], r1[8], r2[8];
      normed(c, y1);
      normed(c + H8, y2);
      const f32x4 c0 = *reinterpret_cast<const f32x4*>(cs + 8 * c), c1 = *reinterpret_cast<const f32x4*>(cs + 8 * c + 4);
      const f32x4 s0 = *reinterpret_cast<const f32x4*>(sn + 8 * c), s1 = *reinterpret_cast<const f32x4*>(sn + 8 * c + 4);
      const float cvv[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
      const float svv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        r1[j] = IO::round(y1[j] * cvv[j] + (-y2[j]) * svv[j]);
        r2[j] = IO::round(y2[j] * cvv[j] + y1[j] * svv[j]);
      }
      emit(c, r1);
      emit(c + H8, r2);
    }
#pragma unroll
    for (int c = 2 * H8; c < D / 8; ++c) {
      float y[8];
      normed(c, y);
      emit(c, y);
    }
    return;
  }
  float y[D];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    IO::unpack8(raw[c], *reinterpret_cast<float(*)[8]>(y + 8 * c));
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __fmaf_rn(y[8 * c + j], y[8 * c + j], ss);
  }
  const float inv = rsqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
  for (int d = 0; d < D; ++d) y[d] = IO::round((y[d] * inv) * qw[d]);
#pragma unroll
  for (int d = 0; d < 8 * H8; ++d) {  // d < half takes -x[d + half], d >= half takes x[d - half]
    const float y1 = y[d], y2 = y[d + 8 * H8];
    y[d] = IO::round(y1 * cv[d] + (-y2) * sv[d]);
    y[d + 8 * H8] = IO::round(y2 * cv[d] + y1 * sv[d]);
  }
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = y[8 * c + j] * qscale;
    out[c] = pack8(o);  // the packing conversion is the final bf16 rounding
  }
}

// `qkv` rows hold q at section 0 and q_diff at section `sqd` (units of H * D); the L queries are padded to Lp (a
// multiple of 128), the Lk keys of the workspace to Lkp. Self-attention has Lk = L. QB: queries per workgroup;
// the 64-query form runs three workgroups per CU.
// IO: the element type of qkv and out (bf16 or half); the attention operands are bf16 either way. QB: queries per
// workgroup; the 64-query form runs three workgroups per CU.
template <class IO, int D, int QB, int NW>
__global__ __launch_bounds__(64 * NW, D == 64 ? (QB == 64 ? 3 : 2) : 1) void dense_attend(
    const uint16_t* __restrict__ qkv, int64_t rs, int sqd, const float* __restrict__ cosT,
    const float* __restrict__ sinT, int half, float eps, const uint16_t* __restrict__ ws, int64_t region, int B,
    int L, int Lp, int Lk, int Lkp, int H, const float* __restrict__ qw, const float* __restrict__ kw,
    const float* __restrict__ lam, uint16_t* __restrict__ out) {
  using T = DenseTile<D, QB, NW>;
  constexpr int NB = T::NB, NCT = T::NCT;
  // Stages A and B of the K/V tiles; the epilogue reuses the array as its exchange buffer.
  __shared__ __attribute__((aligned(16))) uint16_t smem[T::SMEM_ELEMS];
  const int nqb = Lp / QB;
  const int tile = xcd_remap(blockIdx.x, B * H * nqb);
  const int qb = tile % nqb, bh = tile / nqb, h = bh % H, b = bh / H;
  const int lane = threadIdx.x & 63, wave = wave_id(), lr = lane & 31, lh = lane >> 5;
  const int br0 = T::SPLIT ? wave / (NW / 2) : 0;                                 // first branch of this wave
  const int q0 = qb * QB + (T::SPLIT ? (wave % (NW / 2)) * 32 * NCT : wave * 32);  // first query of this wave
  const int64_t rowbase = static_cast<int64_t>(bh) * Lkp;

  constexpr bool kStream = D == 128 && NW == 8;  // the query prologue in the register budget of two waves per SIMD
  // Launch-uniform choice between the max-free and the running-max softmax (see the file comment).
  const SoftmaxPlan plan = dense_plan<D>(qw, kw);

  // The queries: each lane prepares one whole row from qkv (D = 64: row q0 + lane of this wave's branch, or
  // q0 + lane % 32 with one column tile; D = 128: row q0 + lane % 32 of branch lane / 32), then v_permlane32_swap
  // moves the 16-byte chunks into the MFMA B operand layout (lane (lr, lh) holds chunks 2 kk + lh of its row): for
  // chunk pair (2 kk, 2 kk + 1) the swap gives [lanes 0-31 of chunk 2 kk | lanes 0-31 of chunk 2 kk + 1] and the
  // same for lanes 32-63. With one column tile both lane halves hold the same rows and the first half suffices.
  u32x4 qf[NB][NCT][D / 16];
  {
    const int64_t HD = static_cast<int64_t>(H) * D;
    const int qrow = T::SPLIT && NCT == 2 ? q0 + lane : q0 + lr;
    const int sec = (T::SPLIT ? br0 : lh) ? sqd : 0;
    const int qc = qrow < L ? qrow : L - 1;
    const uint16_t* row = qkv + (static_cast<int64_t>(b) * L + qc) * rs + sec * HD + h * D;
    const float* cs = cosT + static_cast<int64_t>(qc) * half;
    const float* sn = sinT + static_cast<int64_t>(qc) * half;
    u32x4 whole[D / 8];
    switch (half / 8) {  // half % 8 == 0 and half <= D / 2 are checked on the host
      case 0: prep_q_row<IO, D, 0, kStream>(row, qw, cs, sn, eps, plan.qscale, whole); break;
      case 1: prep_q_row<IO, D, 1, kStream>(row, qw, cs, sn, eps, plan.qscale, whole); break;
      case 2: prep_q_row<IO, D, 2, kStream>(row, qw, cs, sn, eps, plan.qscale, whole); break;
      case 3: prep_q_row<IO, D, 3, kStream>(row, qw, cs, sn, eps, plan.qscale, whole); break;
      default:
        if constexpr (D == 64) {
          prep_q_row<IO, D, 4, kStream>(row, qw, cs, sn, eps, plan.qscale, whole);
        } else {
          switch (half / 8) {
            case 4: prep_q_row<IO, D, 4, kStream>(row, qw, cs, sn, eps, plan.qscale, whole); break;
            case 5: prep_q_row<IO, D, 5, kStream>(row, qw, cs, sn, eps, plan.qscale, whole); break;
            case 6: prep_q_row<IO, D, 6, kStream>(row, qw, cs, sn, eps, plan.qscale, whole); break;
            case 7: prep_q_row<IO, D, 7, kStream>(row, qw, cs, sn, eps, plan.qscale, whole); break;
            default: prep_q_row<IO, D, 8, kStream>(row, qw, cs, sn, eps, plan.qscale, whole); break;
          }
        }
    }
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const auto r = __builtin_amdgcn_permlane32_swap(whole[2 * kk][e], whole[2 * kk + 1][e], false, false);
        if constexpr (T::SPLIT && NCT == 2) {  // lanes 0-31 held rows q0 .. q0 + 31 (column tile 0), 32-63 the next
          qf[0][0][kk][e] = r[0];
          qf[0][1][kk][e] = r[1];
        } else if constexpr (T::SPLIT) {  // both lane halves held rows q0 .. q0 + 31
          qf[0][0][kk][e] = r[0];
        } else {  // lanes 0-31 held branch 1, lanes 32-63 branch 2, both for rows q0 .. q0 + 31
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

  const TileCopy<D, NW> copy(ws + rowbase * D, ws + region + rowbase * D, ws + 2 * region + rowbase * D);
  copy(0, lds_addr(smem));
  if (plan.fast)
    dense_attend_loop<D, QB, NW, true>(copy, Lk, br0, smem, smem + T::STAGE, qf, o, lsum, plan.c);
  else
    dense_attend_loop<D, QB, NW, false>(copy, Lk, br0, smem, smem + T::STAGE, qf, o, lsum, plan.c);

  // Both stages are free once every wave is past its last tile; the exchange reuses them.
  static_assert(T::XBUF_BYTES <= T::SMEM_ELEMS * 2, "exchange buffer exceeds the workgroup's LDS");
  if constexpr (T::SPLIT) __syncthreads();
  store_diff_split<D, QB, IO, NW>(out, b, L, H, h, q0, br0, lam ? lam[h] : 1.f, o, lsum, smem);
}

__global__ void rope_tables_kernel(const float* __restrict__ inv_freq, int half, int length, float* __restrict__ cosT,
                                   float* __restrict__ sinT) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(length) * half) return;
  const int n = static_cast<int>(i / half), j = static_cast<int>(i % half);
  const double angle = static_cast<double>(__fmul_rn(static_cast<float>(n), inv_freq[j]));
  cosT[i] = static_cast<float>(cos(angle));
  sinT[i] = static_cast<float>(sin(angle));
}

}  // namespace hb

using namespace hb;

static int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HB_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return HB_OK;
}

static int dense_args(const void* qkv, const float* qw, const float* kw, const float* cos, const float* sin, int half,
                      const void* ws, size_t wsb, size_t need) {
  if (!qkv || !qw || !kw || !ws) return fail(HB_ERR_NULL, "qkv, q_weight, k_weight and workspace must be non-NULL");
  if (half > 0 && (!cos || !sin)) return fail(HB_ERR_NULL, "cos and sin must be non-NULL when half > 0");
  if (reinterpret_cast<uintptr_t>(qkv) % 16) return fail(HB_ERR_STRIDE, "qkv must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(ws) % 256) return fail(HB_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (wsb < need) return fail(HB_ERR_WORKSPACE, "workspace holds %zu bytes, needs %zu", wsb, need);
  return HB_OK;
}

extern "C" int hb_rope_tables(hipStream_t stream, const float* inv_freq, int half, int length, float* cosT,
                              float* sinT) {
  clear_error();
  if (half < 0 || length < 0) return fail(HB_ERR_SHAPE, "half %d and length %d must be >= 0", half, length);
  const int64_t n = static_cast<int64_t>(length) * half;
  if (n == 0) return HB_OK;
  if (!inv_freq || !cosT || !sinT) return fail(HB_ERR_NULL, "inv_freq, cos and sin must be non-NULL");
  hipLaunchKernelGGL(rope_tables_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, inv_freq,
                     half, length, cosT, sinT);
  return launch_status("rope_tables");
}

// Checks shared by both stages: shapes, pointers, alignment and the workspace size.
static int dense_checks(const void* qkv, int dtype, int64_t row_stride, const float* qw, const float* kw,
                        const float* cos, const float* sin, int half, int B, int L, int H, int D, float eps,
                        const void* workspace, size_t workspace_bytes, DenseLayout& lay) {
  int st = hb_dense_validate(dtype, row_stride, B, L, H, D, half, eps);
  if (st) return st;
  lay = dense_layout(dtype, B, L, H, D);
  st = dense_args(qkv, qw, kw, cos, sin, half, workspace, workspace_bytes, lay.total_bytes);
  if (st) return st;
  if (half % 8 != 0) return fail(HB_ERR_HALF, "dense kernel needs half %% 8 == 0 (half=%d)", half);
  if (half > 0 && (reinterpret_cast<uintptr_t>(cos) % 16 || reinterpret_cast<uintptr_t>(sin) % 16))
    return fail(HB_ERR_STRIDE, "cos and sin must be 16-byte aligned");
  return HB_OK;
}

namespace hb {

int launch_dense_prep_16bit(hipStream_t stream, int dtype, const void* kv, int64_t rs, int sk, int skd, int sv,
                            const float* kw, const float* cos, const float* sin, int half, const float* vmask, int B,
                            int Lk, int H, int D, float eps, const DenseLayout& lay, void* workspace) {
  const dim3 grid(static_cast<unsigned>(lay.Lp / 64), static_cast<unsigned>(H), static_cast<unsigned>(B));
  const uint16_t* x = static_cast<const uint16_t*>(kv);
  uint16_t* ws = static_cast<uint16_t*>(workspace);
  const int Lkp = static_cast<int>(lay.Lp);
  const bool f16 = dtype == HB_F16;
  auto kernel = D == 64 ? (f16 ? dense_prep<F16Io, 64> : dense_prep<Bf16Io, 64>)
                        : (f16 ? dense_prep<F16Io, 128> : dense_prep<Bf16Io, 128>);
  hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, x, rs, sk, skd, sv, kw, cos, sin, half, vmask, Lk, Lkp, H,
                     eps, lay.region_elems, ws);
  return launch_status("dense_prep");
}

int launch_dense_attend_16bit(hipStream_t stream, int dtype, const void* q, int64_t rs, int sqd, const float* qw,
                              const float* kw, const float* cos, const float* sin, int half, float eps,
                              const float* lam, void* out, int B, int L, int Lk, int H, int D, const DenseLayout& lay,
                              const void* workspace) {
  const int Lp = (L + 127) / 128 * 128;
  const uint16_t* x = static_cast<const uint16_t*>(q);
  const uint16_t* ws = static_cast<const uint16_t*>(workspace);
  uint16_t* o = static_cast<uint16_t*>(out);
  const int Lkp = static_cast<int>(lay.Lp);
  const bool f16 = dtype == HB_F16;
  // 128-query workgroups run two per CU. With between one and one and a half of them per CU, some CUs would run
  // two while most run one; 64-query workgroups (three per CU) spread the same work more evenly (measured: 6 %
  // faster at 288 workgroups on 256 CUs; slower at exactly one per CU and at nearly two, where they cost more per
  // query than they gain in balance). Just past two per CU (a nearly empty second round of 128-query workgroups)
  // they win again: 3 % at 528 workgroups on 256 CUs (B = 2, L = 1292, H = 24). And on grids of at most half a
  // 128-query workgroup per CU they halve the work of each busy CU: 9.8 against 11.4 us at B = 1, L = 216, H = 24.
  const int64_t blocks128 = static_cast<int64_t>(B) * H * (Lp / 128);
  const int64_t ncu = device_cus();
  const bool spread = 2 * blocks128 <= ncu || (blocks128 > ncu && 2 * blocks128 <= 3 * ncu) ||
                      (blocks128 > 2 * ncu && 8 * blocks128 <= 17 * ncu);
  if (D == 64 && spread) {
    const int nblocks = B * H * (Lp / 64);
    auto kernel = f16 ? dense_attend<F16Io, 64, 64, 4> : dense_attend<Bf16Io, 64, 64, 4>;
    hipLaunchKernelGGL(kernel, dim3(nblocks), dim3(DenseTile<64, 64>::NT), 0, stream, x, rs, sqd, cos, sin, half, eps,
                       ws, lay.region_elems, B, L, Lp, Lk, Lkp, H, qw, kw, lam, o);
  } else {
    // head_dim 128: 8 waves of one branch each (two per SIMD) once the grid fills the GPU; below that the 4-wave
    // form, whose fixed part per workgroup is smaller (measured: 7 % faster at L = 1292 and 2584, 17 % slower at
    // L = 216 with 48 workgroups)
    const bool w8 = D == 128 && blocks128 >= ncu;
    auto kernel = D == 64 ? (f16 ? dense_attend<F16Io, 64, 128, 4> : dense_attend<Bf16Io, 64, 128, 4>)
                  : w8    ? (f16 ? dense_attend<F16Io, 128, 128, 8> : dense_attend<Bf16Io, 128, 128, 8>)
                          : (f16 ? dense_attend<F16Io, 128, 128, 4> : dense_attend<Bf16Io, 128, 128, 4>);
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks128)), dim3(w8 ? 512 : 256), 0, stream, x, rs, sqd,
                       cos, sin, half, eps, ws, lay.region_elems, B, L, Lp, Lk, Lkp, H, qw, kw, lam, o);
  }
  return launch_status("dense_attend");
}

}  // namespace hb

// Sections of a to_qkv row [q | k | v | q_diff | k_diff] (dit.py:196-198), in units of H * D.
constexpr int kSecK = 1, kSecV = 2, kSecQd = 3, kSecKd = 4;

// The output of the attention stage: alignment, and no byte shared with qkv or the workspace it reads.
static int out_checks(const void* qkv, int dtype, int64_t row_stride, const void* out, int B, int L, int H, int D,
                      const void* workspace, const DenseLayout& lay) {
  if (reinterpret_cast<uintptr_t>(out) % (dtype == HB_F32 ? 16 : 8))
    return fail(HB_ERR_STRIDE, "out must be %d-byte aligned", dtype == HB_F32 ? 16 : 8);
  const int es = dtype == HB_F32 ? 4 : 2;
  const int64_t HD = static_cast<int64_t>(H) * D, rows = static_cast<int64_t>(B) * L, ob = rows * HD * es;
  int st = check_disjoint("dense_attend", "out", out, ob, "qkv", qkv, rows_bytes(rows, row_stride, 5 * HD, es));
  if (st) return st;
  return check_disjoint("dense_attend", "out", out, ob, "workspace", workspace, static_cast<int64_t>(lay.total_bytes));
}

extern "C" int hb_dense_prep(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride, const float* q_weight,
                             const float* k_weight, const float* cos, const float* sin, int half, const float* vmask,
                             int B, int L, int H, int D, float eps, void* workspace, size_t workspace_bytes) {
  DenseLayout lay;
  const int st = dense_checks(qkv, dtype, row_stride, q_weight, k_weight, cos, sin, half, B, L, H, D, eps, workspace,
                              workspace_bytes, lay);
  if (st) return st;
  const int es = dtype == HB_F32 ? 4 : 2;
  if (const int ov = check_disjoint("dense_prep", "workspace", workspace, static_cast<int64_t>(lay.total_bytes), "qkv",
                                    qkv, rows_bytes(static_cast<int64_t>(B) * L, row_stride,
                                                    static_cast<int64_t>(5) * H * D, es)))
    return ov;
  if (dtype == HB_F32)
    return launch_dense_prep_f32(stream, qkv, row_stride, kSecK, kSecKd, kSecV, k_weight, cos, sin, half, vmask, B, L,
                                 H, D, eps, lay, workspace);
  return launch_dense_prep_16bit(stream, dtype, qkv, row_stride, kSecK, kSecKd, kSecV, k_weight, cos, sin, half, vmask,
                                 B, L, H, D, eps, lay, workspace);
}

extern "C" int hb_dense_attend(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride,
                               const float* q_weight, const float* k_weight, const float* cos, const float* sin,
                               int half, const float* lam, void* out, int B, int L, int H, int D, float eps,
                               const void* workspace, size_t workspace_bytes) {
  if (!out) {
    clear_error();
    return fail(HB_ERR_NULL, "out must be non-NULL");
  }
  DenseLayout lay;
  int st = dense_checks(qkv, dtype, row_stride, q_weight, k_weight, cos, sin, half, B, L, H, D, eps, workspace,
                        workspace_bytes, lay);
  if (st) return st;
  if ((st = out_checks(qkv, dtype, row_stride, out, B, L, H, D, workspace, lay))) return st;
  if (dtype == HB_F32)
    return launch_dense_attend_f32(stream, qkv, row_stride, kSecQd, q_weight, cos, sin, half, eps, workspace, lam, out,
                                   B, L, L, H, D, lay);
  return launch_dense_attend_16bit(stream, dtype, qkv, row_stride, kSecQd, q_weight, k_weight, cos, sin, half, eps, lam,
                                   out, B, L, L, H, D, lay, workspace);
}

extern "C" int hb_dense_diffattn(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride,
                                 const float* q_weight, const float* k_weight, const float* cos, const float* sin,
                                 int half, const float* vmask, const float* lam, void* out, int B, int L, int H, int D,
                                 float eps, void* workspace, size_t workspace_bytes) {
  if (!out) {
    clear_error();
    return fail(HB_ERR_NULL, "out must be non-NULL");
  }
  {  // everything the attention stage checks, before the prep stage launches
    DenseLayout lay;
    int st = dense_checks(qkv, dtype, row_stride, q_weight, k_weight, cos, sin, half, B, L, H, D, eps, workspace,
                          workspace_bytes, lay);
    if (st) return st;
    if ((st = out_checks(qkv, dtype, row_stride, out, B, L, H, D, workspace, lay))) return st;
  }
  int st = hb_dense_prep(stream, qkv, dtype, row_stride, q_weight, k_weight, cos, sin, half, vmask, B, L, H, D, eps,
                         workspace, workspace_bytes);
  if (st) return st;
  return hb_dense_attend(stream, qkv, dtype, row_stride, q_weight, k_weight, cos, sin, half, lam, out, B, L, H, D, eps,
                         workspace, workspace_bytes);
}

// ---- The no-allocation entry point ------------------------------------------------------------------------------
// hb_dense_diffattn_noalloc runs the same two kernels as hb_dense_diffattn with their workspace in `scratch`, a
// file-scope device array of kNoAllocScratchBytes that every GPU the library runs on holds until the process ends.
// Host code never passes the array's name to a kernel (on the host it is only a stand-in for the symbol): the
// device address comes from hipGetSymbolAddress, once per device with that device current, and is kept per device.
// The prep kernel writes every workspace row the attention kernel reads (zeros past L included), so nothing in the
// array has to start at zero; each call on a GPU overwrites what the last one left there, so calls that overlap on
// one GPU (different streams, no ordering between them) race on the array.
namespace {

constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;  // holds the 120 s clip's 49.5 MB bf16 workspace
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device; null until the first call there
std::mutex g_scratch_mutex;

// Device address of `scratch` on the current device, or null (with the error recorded) if it cannot be had.
void* device_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(HB_ERR_LAUNCH, "no current HIP device (or device index %d >= %d)", dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(HB_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" size_t hb_dense_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int hb_dense_diffattn_noalloc(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride,
                                         const float* q_weight, const float* k_weight, const float* cos,
                                         const float* sin, int half, const float* vmask, const float* lam, void* out,
                                         int B, int L, int H, int D, float eps) {
  int st = hb_dense_validate(dtype, row_stride, B, L, H, D, half, eps);
  if (st) return st;
  const size_t need = dense_layout(dtype, B, L, H, D).total_bytes;
  if (need > kNoAllocScratchBytes)
    return fail(HB_ERR_WORKSPACE,
                "this shape needs %zu bytes of workspace, more than the %zu-byte no-allocation scratch; call "
                "hb_dense_diffattn with a workspace instead", need, kNoAllocScratchBytes);
  if (!qkv || !q_weight || !k_weight || !out) return fail(HB_ERR_NULL, "qkv, q_weight, k_weight and out must be non-NULL");
  if (half > 0 && (!cos || !sin)) return fail(HB_ERR_NULL, "cos and sin must be non-NULL when half > 0");
  void* ws = device_scratch();
  if (!ws) return HB_ERR_LAUNCH;
  return hb_dense_diffattn(stream, qkv, dtype, row_stride, q_weight, k_weight, cos, sin, half, vmask, lam, out, B, L,
                           H, D, eps, ws, kNoAllocScratchBytes);
}
