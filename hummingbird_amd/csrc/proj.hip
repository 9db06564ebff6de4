// The DiT self-attention's projections on the matrix cores, for gfx950 (MI355X).
//
// Replaces the two GEMMs around the reference's fused kernel (sa3jax/dit.py:190 `qkv = _linear(h, to_qkv)` and
// dit.py:195 `_linear(out, to_out)`), with the dense kernel's key-side preparation moved into the first one:
//
//   qkv_proj  C^T = W_qkv h^T on v_mfma_f32_32x32x16_bf16 (or _f16 for half inputs), one 256-feature x 128-token tile per workgroup. The
//             fp32 accumulators are rounded to the compute dtype (the stored `qkv` of the reference), then each
//             four-head feature tile is finished by section ([q | k | v | q_diff | k_diff], dit.py:196-198):
//               q, q_diff -> written as they are to a (B, L, 2 H D) buffer [q | q_diff], which the attention
//                            kernel reads (it prepares the queries itself);
//               k, k_diff -> RMSNorm (dit.py:45-57) and rotate-half RoPE (dit.py:90-98) with the fused kernel's
//                            cast points, written in bf16 to the attention workspace (k', k_diff');
//               v         -> times the value mask, written in bf16 to the workspace transposed per 64-key tile in
//                            the order the attention kernel's PV operand takes (v'^T).
//             So the `qkv` tensor is never written, and the separate preparation pass (one read and one write of
//             the key side) disappears.
//   out_proj  C^T = W_o x^T with the accumulators rounded to the compute dtype and written row-major.
//
// The orientation C^T (features x tokens) puts one token in each lane and 16 of its features in the registers of
// one 32 x 32 accumulator tile (feature 8 (r / 4) + 4 (lane / 32) + r % 4 in register r), so a head's 64 features
// live in two tiles of one lane and its partner lane (lane ^ 32): the RMSNorm sum needs one cross-lane add, and
// every RoPE partner (d + half, half a multiple of 8) sits in the same lane.
//
// Operands stream through LDS in 64-column steps, double-buffered, copied straight from global memory with
// global_load_lds (no registers) into rows XOR-swizzled by 16-byte chunk, as in the attention kernel. Each of the
// four waves computes one head (64 features) for all 128 tokens: 8 MFMAs per 16 columns from 2 + 4 fragment reads.
#include <math.h>

#include <type_traits>

#include "api.h"
#include "common.h"
#include "glu_act.h"
#include "tiles.h"

namespace hb {
namespace proj {

constexpr int FT = 256;  // features per workgroup tile (four heads of 64)
constexpr int KS = 64;   // columns of the reduction per step
constexpr int kStages = 3;  // LDS stages of the operand ring (the host side picks the token tile to fit)
constexpr int A_ELEMS = FT * KS;        // one stage of W rows (32 KB)
constexpr int AB = A_ELEMS * 2 / 1024;  // 1 KB blocks of a stage's A tile (32)

// A workgroup of NW waves (4 or 8) computes FT features x TT tokens (TT = 128 or 256). Wave w computes head w % 4 of
// the tile (two 32-feature MFMA tiles) for TW token tiles of 32, starting at token tile (w / 4) * TW.
template <int NW, int TT>
struct Cfg {
  static constexpr int NT = 64 * NW;
  static constexpr int TW = (TT / 32) / (NW / 4);
  static constexpr int B_ELEMS = TT * KS;          // one stage of token rows
  static constexpr int STAGE = A_ELEMS + B_ELEMS;  // elements per LDS stage
  static constexpr int BB = B_ELEMS * 2 / 1024;    // 1 KB blocks of a stage's B tile
  static_assert(NW == 4 || NW == 8, "four or eight waves");
  static_assert(TW >= 1, "at least one token tile per wave");
};

enum Epilogue { kQkvPrep = 0, kPlain = 1, kResidual = 2 };

// Tokens are tiled over the padded token space: B batches of Lp rows (Lp a multiple of 128), token p of it being row
// p % Lp of batch p / Lp; rows at or past L of a batch, and past the last batch, are padding.
struct Args {
  const uint16_t* w;  // (F, K) row-major, row stride w_rs elements
  const uint16_t* x;  // token rows, row stride x_rs elements
  int64_t w_rs, x_rs;
  int K;              // reduction length (multiple of 64)
  int F;              // output features (multiple of 256)
  int B, L, Lp;       // kQkvPrep: batches of L tokens padded to Lp; kPlain: B = 1, L = token count
  int nF, nT;         // feature tiles, token tiles
  // kQkvPrep
  int H, half;
  float eps;
  const float* kw;    // k RMSNorm gains (64)
  const float* cosT;  // (L, half)
  const float* sinT;
  const float* vmask;  // (B, L) or null
  uint16_t* qq;       // (B, L, 2 H 64): [q | q_diff]
  uint16_t* ws;       // workspace: k', k_diff', v'^T regions of `region` elements
  int64_t region;
  // kPlain, kResidual
  uint16_t* out;      // (tokens, F) row-major, row stride out_rs (kResidual: out_h)
  int64_t out_rs;
  // kResidual
  const uint16_t* res;  // (tokens, F) residual rows, row stride res_rs (may be `out` itself)
  int64_t res_rs;
  const float* bias;    // F values of the compute dtype, or null
  const float* dyt;     // [alpha, gamma[F], beta[F]], or null
  uint16_t* out_y;      // (tokens, F), row stride out_rs, when dyt is given
};

// The workgroup's tile: groups of four feature tiles walk the token tiles together (consecutive workgroups share
// their W rows and token rows in L2), and the XCD remap keeps consecutive tiles on one XCD.
__device__ __forceinline__ void tile_of(const Args& a, int& ft, int& tt) {
  constexpr int GF = 4;
  const int id = xcd_remap(blockIdx.x, a.nF * a.nT);
  const int per_group = GF * a.nT;
  const int g = id / per_group, first = g * GF;
  const int gsize = a.nF - first < GF ? a.nF - first : GF;
  const int in = id - g * per_group;
  ft = first + in % gsize;
  tt = in / gsize;
}

// Asynchronous copy of one k-step's operands into an LDS stage. Each wave copies A blocks wv, wv + NW, ... and B
// blocks likewise; lane i lands at byte 16 i of its 1 KB block (row i / 8, position i % 8), so it fetches the
// logical chunk that swz<64> puts there: (i % 8) ^ (i / 8) ^ (block & 1), the block parity being wv & 1.
template <int NW, int TT>
struct OperandCopy {
  using C = Cfg<NW, TT>;
  uint32_t aoff[AB / NW];
  uint32_t boff[C::BB / NW];
  int wv;

  // p0: the tile's first token in the padded token space.
  __device__ OperandCopy(const Args& a, int p0) {
    const int ln = threadIdx.x & 63;
    wv = wave_id();
    const int r8 = ln >> 3, c = (ln & 7) ^ r8 ^ (wv & 1);
#pragma unroll
    for (int u = 0; u < AB / NW; ++u) {
      const int row = 8 * (wv + NW * u) + r8;
      aoff[u] = static_cast<uint32_t>(row * a.w_rs * 2 + 16 * c);
    }
#pragma unroll
    for (int u = 0; u < C::BB / NW; ++u) {
      const int p = p0 + 8 * (wv + NW * u) + r8;
      int b = p / a.Lp, l = p - b * a.Lp;
      if (b >= a.B) b = a.B - 1;  // padding rows read a real row; their results are not stored
      if (l >= a.L) l = a.L - 1;
      boff[u] = static_cast<uint32_t>((static_cast<int64_t>(b) * a.L + l) * a.x_rs * 2 + 16 * c);
    }
  }

  // Step k of the operands (w0, x0: the tile's rows at column 0) into the stage at LDS byte address `stage`.
  __device__ __forceinline__ void operator()(const uint16_t* w0, const uint16_t* x0, int k, uint32_t stage) const {
    const uint16_t* wk = w0 + static_cast<int64_t>(k) * KS;
    const uint16_t* xk = x0 + static_cast<int64_t>(k) * KS;
#pragma unroll
    for (int u = 0; u < AB / NW; ++u) lds_dma16(wk, aoff[u], stage + (wv + NW * u) * 1024);
#pragma unroll
    for (int u = 0; u < C::BB / NW; ++u) lds_dma16(xk, boff[u], stage + 2 * A_ELEMS + (wv + NW * u) * 1024);
  }
};

// One k-step (64 columns) of a wave: its two feature tiles against its TW token tiles, in four 16-column MFMA steps.
// The fragments are double-buffered in registers: those of sub-step kk + 1 are read from LDS while the MFMAs of
// sub-step kk run.
template <class IO, int NW, int TT>
__device__ __forceinline__ void mma_kstep(const uint16_t* s, int wv, f32x16 (&acc)[2][Cfg<NW, TT>::TW]) {
  constexpr int TW = Cfg<NW, TT>::TW;
  const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5;
  const int head = wv & 3, tb = (wv >> 2) * TW;
  u32x4 af[2][2], bf[2][TW];
  auto load = [&](int kk, int buf) {
#pragma unroll
    for (int f = 0; f < 2; ++f) af[buf][f] = lds16(s + swz<64>(64 * head + 32 * f + lr, 2 * kk + lh));
#pragma unroll
    for (int t = 0; t < TW; ++t) bf[buf][t] = lds16(s + A_ELEMS + swz<64>(32 * (tb + t) + lr, 2 * kk + lh));
  };
  load(0, 0);
#pragma unroll
  for (int kk = 0; kk < KS / 16; ++kk) {
    if (kk + 1 < KS / 16) load(kk + 1, (kk + 1) & 1);
    // keep the reads ahead of this sub-step's MFMAs (and so in registers of their own)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int t = 0; t < TW; ++t) acc[f][t] = mfma_io_32x32x16<IO>(af[kk & 1][f], bf[kk & 1][t], acc[f][t]);
  }
}

// The accumulators of token tile t as the lane's 32 features of its token, x[a][j] = feature 8 a + 4 lh + j, rounded
// to the compute dtype (the reference's `qkv` values).
template <class IO, int TW>
__device__ __forceinline__ void token_values(const f32x16 (&acc)[2][TW], int t, float (&x)[8][4]) {
#pragma unroll
  for (int a = 0; a < 8; ++a)
#pragma unroll
    for (int j = 0; j < 4; ++j) x[a][j] = IO::round(acc[a >> 2][t][4 * (a & 3) + j]);
}

// RMSNorm (dit.py:45-57) and rotate-half RoPE over the first 2 * 8 H8 features (dit.py:90-98) of one key row held
// by this lane and its partner lane (features 8 a + 4 lh + j), with the cast points of the preparation kernel: the
// compute dtype after the gain and after the rotation. `cs` / `sn`: the row's (half) table entries.
template <class IO, int H8>
__device__ __forceinline__ void norm_rope(float (&x)[8][4], const float* __restrict__ kw, const float* __restrict__ cs,
                                         const float* __restrict__ sn, float eps) {
  const int lh = (threadIdx.x & 63) >> 5;
  float ss = 0.f;
#pragma unroll
  for (int a = 0; a < 8; ++a)
#pragma unroll
    for (int j = 0; j < 4; ++j) ss = __fmaf_rn(x[a][j], x[a][j], ss);
  ss += __shfl_xor(ss, 32, kWave);
  const float inv = rsqrtf(ss / 64.f + eps);
#pragma unroll
  for (int a = 0; a < 8; ++a) {
    const f32x4 w4 = *reinterpret_cast<const f32x4*>(kw + 8 * a + 4 * lh);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[a][j] = IO::round((x[a][j] * inv) * w4[j]);
  }
#pragma unroll
  for (int a = 0; a < H8; ++a) {  // d < half takes -x[d + half], d >= half takes x[d - half]
    const f32x4 c4 = *reinterpret_cast<const f32x4*>(cs + 8 * a + 4 * lh);
    const f32x4 s4 = *reinterpret_cast<const f32x4*>(sn + 8 * a + 4 * lh);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float y1 = x[a][j], y2 = x[a + H8][j];
      x[a][j] = IO::round(y1 * c4[j] + (-y2) * s4[j]);
      x[a + H8][j] = IO::round(y2 * c4[j] + y1 * s4[j]);
    }
  }
}

// Four features of one row as 8 bytes of the output type (IO) or of bf16.
template <class IO>
__device__ __forceinline__ u32x2 pack4_io(const float (&v)[4]) {
  return u32x2{IO::pack2(v[0], v[1]), IO::pack2(v[2], v[3])};
}
__device__ __forceinline__ u32x2 pack4_bf16(const float (&v)[4]) {
  return u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
}

// Token tile t of this wave: its batch and the lane's row in it (-1 past the last batch). A 32-token tile never
// straddles batches (Lp is a multiple of 128).
__device__ __forceinline__ void token_of(const Args& a, int p, int& b, int& l) {
  b = p / a.Lp;
  l = p - b * a.Lp + (threadIdx.x & 31);
  if (b >= a.B) b = -1;
}

template <class IO, int NW, int TT>
__device__ __forceinline__ void epilogue_qkv(const Args& a, const f32x16 (&acc)[2][Cfg<NW, TT>::TW], int ft, int p0) {
  constexpr int TW = Cfg<NW, TT>::TW;
  const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5, wv = wave_id();
  const int64_t HD = static_cast<int64_t>(a.H) * 64;
  const int fb = ft * FT + 64 * (wv & 3);  // this wave's first feature: one head of one section
  const int sec = static_cast<int>(fb / HD), h = static_cast<int>(fb % HD) / 64;
  p0 += 32 * TW * (wv >> 2);  // this wave's first token
#pragma unroll
  for (int t = 0; t < TW; ++t) {
    int b, tok;
    token_of(a, p0 + 32 * t, b, tok);  // tok < Lp
    if (b < 0) continue;  // wave-uniform
    const bool real = tok < a.L;
    const int tc = real ? tok : a.L - 1;  // table and mask rows are read at a real position
    const int64_t bh = static_cast<int64_t>(b) * a.H + h;
    float x[8][4];
    token_values<IO, TW>(acc, t, x);
    if (sec == 0 || sec == 3) {  // q, q_diff: the attention kernel prepares them
      if (real) {
        uint16_t* row = a.qq + (static_cast<int64_t>(b) * a.L + tok) * 2 * HD + (sec == 3 ? HD : 0) + h * 64;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          const float v[4] = {x[g][0], x[g][1], x[g][2], x[g][3]};
          *reinterpret_cast<u32x2*>(row + 8 * g + 4 * lh) = pack4_io<IO>(v);
        }
      }
    } else if (sec == 1 || sec == 4) {  // k, k_diff: RMSNorm + RoPE, bf16 rows of the workspace
      const float* cs = a.cosT + static_cast<int64_t>(tc) * a.half;
      const float* sn = a.sinT + static_cast<int64_t>(tc) * a.half;
      switch (a.half / 8) {  // half % 8 == 0 and half <= 32 are checked on the host
        case 0: norm_rope<IO, 0>(x, a.kw, cs, sn, a.eps); break;
        case 1: norm_rope<IO, 1>(x, a.kw, cs, sn, a.eps); break;
        case 2: norm_rope<IO, 2>(x, a.kw, cs, sn, a.eps); break;
        case 3: norm_rope<IO, 3>(x, a.kw, cs, sn, a.eps); break;
        default: norm_rope<IO, 4>(x, a.kw, cs, sn, a.eps); break;
      }
      uint16_t* row = a.ws + (sec == 4 ? a.region : 0) + (bh * a.Lp + tok) * 64;
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const float v[4] = {real ? x[g][0] : 0.f, real ? x[g][1] : 0.f, real ? x[g][2] : 0.f, real ? x[g][3] : 0.f};
        *reinterpret_cast<u32x2*>(row + 8 * g + 4 * lh) = pack4_bf16(v);
      }
    } else {  // v: times the value mask, bf16, transposed per 64-key tile (v_tile_key order)
      const float m = real ? (a.vmask ? a.vmask[static_cast<int64_t>(b) * a.L + tok] : 1.f) : 0.f;
      uint16_t* tile = a.ws + 2 * a.region + (bh * a.Lp + (tok & ~63)) * 64;
      const int pos = v_tile_key(tok & 63);  // even for even lanes: the pair (pos, pos + 1) is one dword
#pragma unroll
      for (int g = 0; g < 8; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float mine = x[g][j] * m;
          const float odd = __shfl_xor(mine, 1, kWave);  // the next token's value of this feature
          if (!(lr & 1))
            *reinterpret_cast<uint32_t*>(tile + (8 * g + 4 * lh + j) * 64 + pos) = pack_bf16x2(mine, odd);
        }
    }
  }
}

template <class IO, int NW, int TT>
__device__ __forceinline__ void epilogue_plain(const Args& a, const f32x16 (&acc)[2][Cfg<NW, TT>::TW], int ft, int p0) {
  constexpr int TW = Cfg<NW, TT>::TW;
  const int lane = threadIdx.x & 63, lh = lane >> 5, wv = wave_id();
  const int fb = ft * FT + 64 * (wv & 3);
  p0 += 32 * TW * (wv >> 2);
#pragma unroll
  for (int t = 0; t < TW; ++t) {
    int b, tok;
    token_of(a, p0 + 32 * t, b, tok);
    if (b < 0 || tok >= a.L) continue;
    float x[8][4];
    token_values<IO, TW>(acc, t, x);
    uint16_t* row = a.out + static_cast<int64_t>(tok) * a.out_rs + fb;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const float v[4] = {x[g][0], x[g][1], x[g][2], x[g][3]};
      *reinterpret_cast<u32x2*>(row + 8 * g + 4 * lh) = pack4_io<IO>(v);
    }
  }
}

// The residual add of same_l._block (sa3jax/same_l.py:191-192) after the projection (same_l._linear: the matmul,
// then the bias add): out_h = h + (x W^T + bias), each of the three held in the compute dtype, and with `dyt`
// out_y = cast(DyT(out_h)), the input of the next GEMM; the same arithmetic as hb_residual_dyt on the stored product.
// Each element of the residual is read and its out_h written by one lane, so out_h may be the residual itself.
template <class IO, int NW, int TT>
__device__ __forceinline__ void epilogue_residual(const Args& a, const f32x16 (&acc)[2][Cfg<NW, TT>::TW], int ft,
                                                  int p0) {
  constexpr int TW = Cfg<NW, TT>::TW;
  const int lane = threadIdx.x & 63, lh = lane >> 5, wv = wave_id();
  const int fb = ft * FT + 64 * (wv & 3);
  const float a2 = a.dyt ? 2.f * kLog2e * a.dyt[0] : 0.f;
  p0 += 32 * TW * (wv >> 2);
#pragma unroll
  for (int t = 0; t < TW; ++t) {
    int b, tok;
    token_of(a, p0 + 32 * t, b, tok);
    if (b < 0 || tok >= a.L) continue;
    float x[8][4];
    token_values<IO, TW>(acc, t, x);
    const uint16_t* hrow = a.res + static_cast<int64_t>(tok) * a.res_rs + fb;
    uint16_t* orow = a.out + static_cast<int64_t>(tok) * a.out_rs + fb;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const int f0 = 8 * g + 4 * lh;  // this lane's four features of group g, relative to fb
      const u32x2 hp = *reinterpret_cast<const u32x2*>(hrow + f0);
      float hv[4];
      {
        float e8[8];
        IO::unpack8(u32x4{hp[0], hp[1], 0u, 0u}, e8);
#pragma unroll
        for (int j = 0; j < 4; ++j) hv[j] = e8[j];
      }
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float xv = x[g][j];
        if (a.bias) xv = IO::round(xv + a.bias[fb + f0 + j]);
        v[j] = IO::round(hv[j] + xv);
      }
      *reinterpret_cast<u32x2*>(orow + f0) = pack4_io<IO>(v);
      if (a.dyt) {
        float y[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float gm = a.dyt[1 + fb + f0 + j], be = a.dyt[1 + a.F + fb + f0 + j];
          y[j] = dyt_tanh(v[j], a2, -2.f * gm, gm + be);
        }
        *reinterpret_cast<u32x2*>(a.out_y + static_cast<int64_t>(tok) * a.out_rs + fb + f0) = pack4_io<IO>(y);
      }
    }
  }
}

// Waits until at most N vector-memory operations of this wave are outstanding (vmcnt N; expcnt and lgkmcnt at their
// maxima, i.e. not waited on). Loads complete in issue order, so this retires all but the N most recent copies.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <class IO, int EPI, int NW, int TT>
__global__ __launch_bounds__(64 * NW) void proj_gemm(Args a) {
  using C = Cfg<NW, TT>;
  constexpr int TW = C::TW;
  constexpr int NS = kStages;                         // LDS stages: copies run NS - 1 steps ahead
  static_assert(NS == 2 || NS == 3, "the waits below count the copies of a two- or three-stage ring");
  constexpr int PER_COPY = AB / NW + C::BB / NW;      // global_load_lds instructions per wave per step
  __shared__ __attribute__((aligned(16))) uint16_t smem[NS * C::STAGE];
  int ft, tt;
  tile_of(a, ft, tt);
  const int p0 = tt * TT;  // the tile's first token in the padded token space
  const int wv = wave_id();

  const OperandCopy<NW, TT> copy(a, p0);
  const uint16_t* w0 = a.w + static_cast<int64_t>(ft) * FT * a.w_rs;
  const uint16_t* x0 = a.x;  // token rows are addressed by the per-lane offsets
  f32x16 acc[2][TW];
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int t = 0; t < TW; ++t) acc[f][t] = f32x16{};

  const int nk = a.K / KS;
  const uint32_t lds0 = lds_addr(smem);
  // Steps 0 .. NS - 2 in flight; then per step: copy step k + NS - 1 into the stage step k - 1 used, multiply step
  // k, wait for step k + 1's copy (all but the newest copy retired) and pass one barrier.
#pragma unroll
  for (int i = 0; i < NS - 1; ++i)
    if (i < nk) copy(w0, x0, i, lds0 + i * C::STAGE * 2);
  if (nk > 1) wait_vmcnt<(NS - 2) * PER_COPY>(); else wait_vmcnt<0>();
  __syncthreads();
  for (int k = 0; k < nk; ++k) {
    const int ahead = k + NS - 1;
    if (ahead < nk) copy(w0, x0, ahead, lds0 + (ahead % NS) * C::STAGE * 2);
    const uint16_t* st = smem + (k % NS) * C::STAGE;
    mma_kstep<IO, NW, TT>(st, wv, acc);
    // step k + 1 must have landed; copies of later steps may stay in flight
    if (ahead < nk) wait_vmcnt<(NS - 2) * PER_COPY>();
    else if (k + 2 < nk) wait_vmcnt<(NS - 3 > 0 ? NS - 3 : 0) * PER_COPY>();
    else wait_vmcnt<0>();
    __syncthreads();
  }

  if constexpr (EPI == kQkvPrep)
    epilogue_qkv<IO, NW, TT>(a, acc, ft, p0);
  else if constexpr (EPI == kResidual)
    epilogue_residual<IO, NW, TT>(a, acc, ft, p0);
  else
    epilogue_plain<IO, NW, TT>(a, acc, ft, p0);
}

}  // namespace proj

// The feed-forward's glu_proj with the GLU in its epilogue (sa3jax/same_l.py:181-183): out = value * act(gate) for
// [value | gate] = x [W_value | W_gate]^T (+ bias), so the 2F-wide product is never stored.
//
// Workgroup tiles of 256 W rows x 256 tokens, four waves of 128 x 128 (4 x 4 tiles of v_mfma_f32_32x32x16, the 256
// accumulators in the accumulation registers, one wave per SIMD), K in 64-column steps through two 64 KB LDS
// stages filled by global_load_lds (next step's copy issued at the start of the current one). The 256 W rows of a
// tile are gathered so that each wave holds the value rows of 64 output features in its MFMA tiles 0 and 1 and the
// gate rows of the same features in tiles 2 and 3: a lane then has the value and the gate of each of its outputs in
// the same register of two tiles, and the epilogue needs no exchange. A tile writes 128 output features.
namespace proj_wide {

constexpr int KS = 64;                 // reduction columns per step
constexpr int TROWS = 256;             // W rows and tokens per tile
constexpr int STAGE = 2 * TROWS * KS;  // elements per LDS stage: W rows, then token rows (64 KB)

struct Args {
  const uint16_t* w;  // (2F, K): value rows 0 .. F - 1, gate rows F .. 2F - 1
  const uint16_t* x;  // (N, K) token rows
  int64_t w_rs, x_rs;
  int K, N, F;        // F: output features (value width)
  int nF, nT;         // feature tiles (F / 128), token tiles
  const float* bias;  // 2F values of the compute dtype, or null
  uint16_t* out;      // (N, F)
  int64_t out_rs;
};

// W row of tile row r of feature tile ft: wave half wm = r / 128 covers output features 128 ft + 64 wm .. + 64, its
// MFMA tile i = (r / 32) % 4 holds value rows (i = 0, 1) or the gate rows of the same features (i = 2, 3).
__device__ __forceinline__ int w_row(const Args& a, int ft, int r) {
  const int wm = r >> 7, i = (r >> 5) & 3;
  const int f = 128 * ft + 64 * wm + 32 * (i & 1) + (r & 31);
  return i < 2 ? f : a.F + f;
}

template <class IO, bool SINE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void proj_glu(Args a) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE];
  int ft, tt;
  {  // groups of four feature tiles walk the token tiles together; the XCD remap keeps consecutive tiles on one XCD
    constexpr int GF = 4;
    const int id = xcd_remap(blockIdx.x, a.nF * a.nT);
    const int g = id / (GF * a.nT), first = g * GF;
    const int gsize = a.nF - first < GF ? a.nF - first : GF;
    const int in = id - g * GF * a.nT;
    ft = first + in % gsize;
    tt = in / gsize;
  }
  const int lane = threadIdx.x & 63, wv = wave_id(), wm = wv >> 1, wn = wv & 1;
  const int lr = lane & 31, lh = lane >> 5;

  // Copies: wave wv fills 1 KB blocks wv + 4 u (u < 8) of each operand, block b holding tile rows 8 b .. 8 b + 7;
  // lane i lands at row 8 b + i / 8, physical chunk i % 8, so it fetches the logical chunk that swz<64> puts there.
  uint32_t aoff[8], boff[8];
  {
    const int r8 = lane >> 3, c = (lane & 7) ^ r8 ^ (wv & 1);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int row = 8 * (wv + 4 * u) + r8;
      aoff[u] = static_cast<uint32_t>(static_cast<int64_t>(w_row(a, ft, row)) * a.w_rs * 2 + 16 * c);
      int tok = tt * TROWS + row;
      if (tok >= a.N) tok = a.N - 1;  // padding rows read a real row; their results are not stored
      boff[u] = static_cast<uint32_t>(static_cast<int64_t>(tok) * a.x_rs * 2 + 16 * c);
    }
  }
  const uint32_t lds0 = lds_addr(smem);
  auto copy = [&](int k, int s) {
    const uint32_t st = lds0 + s * STAGE * 2;
    const uint16_t* wk = a.w + static_cast<int64_t>(k) * KS;
    const uint16_t* xk = a.x + static_cast<int64_t>(k) * KS;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      lds_dma16(wk, aoff[u], st + (wv + 4 * u) * 1024);
      lds_dma16(xk, boff[u], st + TROWS * KS * 2 + (wv + 4 * u) * 1024);
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  // Fragments of 16-column sub-step kk, double-buffered in registers (sub-step kk + 1 is read during kk's MFMAs).
  u32x4 fa[2][4], fb[2][4];
  auto fread = [&](const uint16_t* st, int kk, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[buf][i] = lds16(st + swz<64>(128 * wm + 32 * i + lr, 2 * kk + lh));
      fb[buf][i] = lds16(st + TROWS * KS + swz<64>(128 * wn + 32 * i + lr, 2 * kk + lh));
    }
  };

  const int nk = a.K / KS;
  copy(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int k = 0; k < nk; ++k) {
    const uint16_t* st = smem + (k & 1) * STAGE;
    fread(st, 0, 0);
    if (k + 1 < nk) copy(k + 1, (k + 1) & 1);  // into the stage step k - 1 used (every wave is past its barrier)
#pragma unroll
    for (int kk = 0; kk < KS / 16; ++kk) {
      if (kk + 1 < KS / 16) fread(st, kk + 1, (kk + 1) & 1);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma_io_32x32x16<IO>(fa[kk & 1][i], fb[kk & 1][j], acc[i][j]);
    }
    __builtin_amdgcn_s_waitcnt(0);  // step k + 1 has landed
    __syncthreads();
  }

  // Epilogue: lane lr of token tile j holds, in register 4 q + e of MFMA tile i, feature 8 q + 4 lh + e of that
  // tile. Value (tiles 0, 1) and gate (tiles 2, 3) are rounded to the compute dtype (the reference's stored
  // glu_proj output), the bias added and rounded, then value * round(act(gate)) as hb_glu computes it.
  auto round = [](float v) { return IO::round(v); };
  constexpr int kSine = std::is_same<IO, Bf16Io>::value ? kSineBf16 : kSineHalf;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tok = tt * TROWS + 128 * wn + 32 * j + lr;
    if (tok >= a.N) continue;
    uint16_t* orow = a.out + static_cast<int64_t>(tok) * a.out_rs;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int f = 128 * ft + 64 * wm + 32 * i + 8 * q + 4 * lh;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float val = IO::round(acc[i][j][4 * q + e]), g = IO::round(acc[i + 2][j][4 * q + e]);
          if (a.bias) {
            val = IO::round(val + a.bias[f + e]);
            g = IO::round(g + a.bias[a.F + f + e]);
          }
          v[e] = val * IO::round(glu_act<SINE, kSine>(g, round));
        }
        *reinterpret_cast<u32x2*>(orow + f) = u32x2{IO::pack2(v[0], v[1]), IO::pack2(v[2], v[3])};
      }
  }
}

}  // namespace proj_wide
}  // namespace hb

using namespace hb;

namespace {

constexpr int kProjWaves = 8;    // waves per projection workgroup
constexpr int kProjTokens = 128;  // tokens per projection workgroup

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HB_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return HB_OK;
}

// Byte offsets of operand rows are 32-bit (global_load_lds takes a 32-bit per-lane offset from a scalar base).
bool offsets_fit(int64_t rows, int64_t row_stride) { return rows * row_stride * 2 < (int64_t(1) << 32); }

int check_operand(const char* what, const void* p, int64_t rows, int64_t rs, int64_t cols) {
  if (!p) return fail(HB_ERR_NULL, "%s must be non-NULL", what);
  if (reinterpret_cast<uintptr_t>(p) % 16) return fail(HB_ERR_STRIDE, "%s must be 16-byte aligned", what);
  if (rs < cols || rs % 8) return fail(HB_ERR_STRIDE, "%s row stride %lld must be >= %lld and a multiple of 8", what,
                                       static_cast<long long>(rs), static_cast<long long>(cols));
  if (const int st = check_extent("projection", what, rows, rs, cols)) return st;
  if (!offsets_fit(rows, rs)) return fail(HB_ERR_SHAPE, "%s spans 4 GiB or more", what);
  return HB_OK;
}

}  // namespace

extern "C" int hb_dit_qkv_proj(hipStream_t stream, const void* h, int dtype, int64_t h_row_stride, const void* w_qkv,
                               int64_t w_row_stride, int E, const float* k_weight, const float* cos, const float* sin,
                               int half, const float* vmask, void* qq, int B, int L, int H, int D, float eps,
                               void* workspace, size_t workspace_bytes) {
  clear_error();
  if (dtype != HB_BF16 && dtype != HB_F16)
    return fail(HB_ERR_DTYPE, "the fused projection takes HB_BF16 or HB_F16 (dtype %d)", dtype);
  if (D != 64) return fail(HB_ERR_HEAD_DIM, "the fused projection needs head_dim 64 (D=%d)", D);
  if (B < 1 || L < 1 || H < 1 || B > 65535 || L > (1 << 24))
    return fail(HB_ERR_SHAPE, "need 1 <= B <= 65535, 1 <= L <= 2^24, H >= 1 (B=%d, L=%d, H=%d)", B, L, H);
  if (H % 4) return fail(HB_ERR_SHAPE, "the fused projection needs the head count to be a multiple of 4 (H=%d)", H);
  if (E < 64 || E % 64) return fail(HB_ERR_SHAPE, "the model width E=%d must be a positive multiple of 64", E);
  if (half < 0 || half > 32 || half % 8) return fail(HB_ERR_HALF, "half %d must be a multiple of 8 in [0, 32]", half);
  if (!(eps >= 0.0f) || !isfinite(eps)) return fail(HB_ERR_EPS, "eps %g must be finite and >= 0", eps);
  const int64_t HD = static_cast<int64_t>(H) * D;
  int st = check_operand("h", h, static_cast<int64_t>(B) * L, h_row_stride, E);
  if (st) return st;
  st = check_operand("w_qkv", w_qkv, 5 * HD, w_row_stride, E);
  if (st) return st;
  if (!k_weight || !qq) return fail(HB_ERR_NULL, "k_weight and qq must be non-NULL");
  if (half > 0 && (!cos || !sin)) return fail(HB_ERR_NULL, "cos and sin must be non-NULL when half > 0");
  if (half > 0 && (reinterpret_cast<uintptr_t>(cos) % 16 || reinterpret_cast<uintptr_t>(sin) % 16))
    return fail(HB_ERR_STRIDE, "cos and sin must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(k_weight) % 16) return fail(HB_ERR_STRIDE, "k_weight must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(qq) % 8) return fail(HB_ERR_STRIDE, "qq must be 8-byte aligned");
  const DenseLayout lay = dense_layout(dtype, B, L, H, D);
  if (!workspace) return fail(HB_ERR_NULL, "workspace must be non-NULL");
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(HB_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (workspace_bytes < lay.total_bytes)
    return fail(HB_ERR_WORKSPACE, "workspace holds %zu bytes, needs %zu", workspace_bytes, lay.total_bytes);
  {
    const int64_t hb = rows_bytes(static_cast<int64_t>(B) * L, h_row_stride, E, 2);
    const int64_t wb = rows_bytes(5 * HD, w_row_stride, E, 2), qb = static_cast<int64_t>(B) * L * 2 * HD * 2;
    const int64_t sb = static_cast<int64_t>(lay.total_bytes);
    const char* w = "qkv_proj";
    if ((st = check_disjoint(w, "qq", qq, qb, "h", h, hb)) || (st = check_disjoint(w, "qq", qq, qb, "w_qkv", w_qkv, wb)) ||
        (st = check_disjoint(w, "workspace", workspace, sb, "h", h, hb)) ||
        (st = check_disjoint(w, "workspace", workspace, sb, "w_qkv", w_qkv, wb)) ||
        (st = check_disjoint(w, "workspace", workspace, sb, "qq", qq, qb)))
      return st;
  }

  proj::Args a{};
  a.w = static_cast<const uint16_t*>(w_qkv);
  a.x = static_cast<const uint16_t*>(h);
  a.w_rs = w_row_stride;
  a.x_rs = h_row_stride;
  a.K = E;
  a.F = static_cast<int>(5 * HD);
  a.B = B;
  a.L = L;
  a.Lp = static_cast<int>(lay.Lp);
  a.nF = a.F / proj::FT;
  a.nT = static_cast<int>((static_cast<int64_t>(B) * a.Lp + kProjTokens - 1) / kProjTokens);
  a.H = H;
  a.half = half;
  a.eps = eps;
  a.kw = k_weight;
  a.cosT = cos;
  a.sinT = sin;
  a.vmask = vmask;
  a.qq = static_cast<uint16_t*>(qq);
  a.ws = static_cast<uint16_t*>(workspace);
  a.region = lay.region_elems;
  const unsigned grid = static_cast<unsigned>(a.nF * a.nT);
  if (dtype == HB_F16)
    hipLaunchKernelGGL((proj::proj_gemm<F16Io, proj::kQkvPrep, kProjWaves, kProjTokens>), dim3(grid),
                       dim3(64 * kProjWaves), 0, stream, a);
  else
    hipLaunchKernelGGL((proj::proj_gemm<Bf16Io, proj::kQkvPrep, kProjWaves, kProjTokens>), dim3(grid),
                       dim3(64 * kProjWaves), 0, stream, a);
  return launched("qkv_proj");
}

extern "C" int hb_proj(hipStream_t stream, const void* x, int dtype, int64_t x_row_stride, const void* w,
                       int64_t w_row_stride, void* out, int64_t out_row_stride, int64_t N, int K, int F) {
  clear_error();
  if (dtype != HB_BF16 && dtype != HB_F16)
    return fail(HB_ERR_DTYPE, "the projection takes HB_BF16 or HB_F16 (dtype %d)", dtype);
  if (N < 1 || N > (1 << 24)) return fail(HB_ERR_SHAPE, "need 1 <= N <= 2^24 rows (N=%lld)", static_cast<long long>(N));
  if (K < 64 || K % 64) return fail(HB_ERR_SHAPE, "the reduction length K=%d must be a positive multiple of 64", K);
  if (F < 256 || F % 256) return fail(HB_ERR_SHAPE, "the output width F=%d must be a positive multiple of 256", F);
  int st = check_operand("x", x, N, x_row_stride, K);
  if (st) return st;
  st = check_operand("w", w, F, w_row_stride, K);
  if (st) return st;
  if (!out) return fail(HB_ERR_NULL, "out must be non-NULL");
  if (reinterpret_cast<uintptr_t>(out) % 8 || out_row_stride < F || out_row_stride % 4)
    return fail(HB_ERR_STRIDE, "out must be 8-byte aligned with a row stride >= F and a multiple of 4");
  if ((st = check_extent("proj", "out", N, out_row_stride, F))) return st;
  {
    const int64_t ob = rows_bytes(N, out_row_stride, F, 2);
    if ((st = check_disjoint("proj", "out", out, ob, "x", x, rows_bytes(N, x_row_stride, K, 2))) ||
        (st = check_disjoint("proj", "out", out, ob, "w", w, rows_bytes(F, w_row_stride, K, 2))))
      return st;
  }
  proj::Args a{};
  a.w = static_cast<const uint16_t*>(w);
  a.x = static_cast<const uint16_t*>(x);
  a.w_rs = w_row_stride;
  a.x_rs = x_row_stride;
  a.K = K;
  a.F = F;
  a.B = 1;
  a.L = static_cast<int>(N);
  a.Lp = static_cast<int>(round_up(N, 128));
  a.nF = F / proj::FT;
  a.nT = static_cast<int>((a.Lp + kProjTokens - 1) / kProjTokens);
  a.out = static_cast<uint16_t*>(out);
  a.out_rs = out_row_stride;
  const unsigned grid = static_cast<unsigned>(a.nF * a.nT);
  if (dtype == HB_F16)
    hipLaunchKernelGGL((proj::proj_gemm<F16Io, proj::kPlain, kProjWaves, kProjTokens>), dim3(grid),
                       dim3(64 * kProjWaves), 0, stream, a);
  else
    hipLaunchKernelGGL((proj::proj_gemm<Bf16Io, proj::kPlain, kProjWaves, kProjTokens>), dim3(grid),
                       dim3(64 * kProjWaves), 0, stream, a);
  return launched("proj");
}

extern "C" int hb_proj_glu(hipStream_t stream, const void* x, int dtype, int64_t x_row_stride, const void* w,
                           int64_t w_row_stride, const float* bias, int sinusoidal, void* out, int64_t out_row_stride,
                           int64_t N, int K, int F) {
  clear_error();
  if (dtype != HB_BF16 && dtype != HB_F16)
    return fail(HB_ERR_DTYPE, "the GLU projection takes HB_BF16 or HB_F16 (dtype %d)", dtype);
  if (N < 1 || N > (1 << 24)) return fail(HB_ERR_SHAPE, "need 1 <= N <= 2^24 rows (N=%lld)", static_cast<long long>(N));
  if (K < 64 || K % 64) return fail(HB_ERR_SHAPE, "the reduction length K=%d must be a positive multiple of 64", K);
  if (F < 128 || F % 128 || F > (1 << 24))
    return fail(HB_ERR_SHAPE, "the output width F=%d must be a positive multiple of 128", F);
  int st = check_operand("x", x, N, x_row_stride, K);
  if (st) return st;
  st = check_operand("w", w, static_cast<int64_t>(2) * F, w_row_stride, K);
  if (st) return st;
  if (!out) return fail(HB_ERR_NULL, "out must be non-NULL");
  if (reinterpret_cast<uintptr_t>(out) % 8 || out_row_stride < F || out_row_stride % 4)
    return fail(HB_ERR_STRIDE, "out must be 8-byte aligned with a row stride >= F and a multiple of 4");
  if ((st = check_extent("proj_glu", "out", N, out_row_stride, F))) return st;
  {
    const int64_t ob = rows_bytes(N, out_row_stride, F, 2);
    if ((st = check_disjoint("proj_glu", "out", out, ob, "x", x, rows_bytes(N, x_row_stride, K, 2))) ||
        (st = check_disjoint("proj_glu", "out", out, ob, "w", w, rows_bytes(2 * static_cast<int64_t>(F), w_row_stride,
                                                                             K, 2))) ||
        (st = check_disjoint("proj_glu", "out", out, ob, "bias", bias, static_cast<int64_t>(2) * F * 4)))
      return st;
  }
  proj_wide::Args a{};
  a.w = static_cast<const uint16_t*>(w);
  a.x = static_cast<const uint16_t*>(x);
  a.w_rs = w_row_stride;
  a.x_rs = x_row_stride;
  a.K = K;
  a.N = static_cast<int>(N);
  a.F = F;
  a.nF = F / 128;
  a.nT = static_cast<int>((N + proj_wide::TROWS - 1) / proj_wide::TROWS);
  a.bias = bias;
  a.out = static_cast<uint16_t*>(out);
  a.out_rs = out_row_stride;
  const dim3 grid(static_cast<unsigned>(a.nF * a.nT)), block(256);
  if (dtype == HB_F16) {
    if (sinusoidal)
      hipLaunchKernelGGL((proj_wide::proj_glu<F16Io, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((proj_wide::proj_glu<F16Io, false>), grid, block, 0, stream, a);
  } else {
    if (sinusoidal)
      hipLaunchKernelGGL((proj_wide::proj_glu<Bf16Io, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((proj_wide::proj_glu<Bf16Io, false>), grid, block, 0, stream, a);
  }
  return launched("proj_glu");
}

extern "C" int hb_proj_residual(hipStream_t stream, const void* x, int dtype, int64_t x_row_stride, const void* w,
                                int64_t w_row_stride, const float* bias, const void* h, int64_t h_row_stride,
                                const float* dyt, void* out_h, void* out_y, int64_t out_row_stride, int64_t N, int K,
                                int F) {
  clear_error();
  if (dtype != HB_BF16 && dtype != HB_F16)
    return fail(HB_ERR_DTYPE, "the residual projection takes HB_BF16 or HB_F16 (dtype %d)", dtype);
  if (N < 1 || N > (1 << 24)) return fail(HB_ERR_SHAPE, "need 1 <= N <= 2^24 rows (N=%lld)", static_cast<long long>(N));
  if (K < 64 || K % 64) return fail(HB_ERR_SHAPE, "the reduction length K=%d must be a positive multiple of 64", K);
  if (F < 256 || F % 256 || F > (1 << 24))
    return fail(HB_ERR_SHAPE, "the output width F=%d must be a positive multiple of 256", F);
  int st = check_operand("x", x, N, x_row_stride, K);
  if (st) return st;
  st = check_operand("w", w, F, w_row_stride, K);
  if (st) return st;
  if (!h || !out_h) return fail(HB_ERR_NULL, "h and out_h must be non-NULL");
  if (!dyt != !out_y) return fail(HB_ERR_NULL, "dyt and out_y are given together or not at all");
  if (reinterpret_cast<uintptr_t>(h) % 8 || h_row_stride < F || h_row_stride % 4)
    return fail(HB_ERR_STRIDE, "h must be 8-byte aligned with a row stride >= F and a multiple of 4");
  if (reinterpret_cast<uintptr_t>(out_h) % 8 || (out_y && reinterpret_cast<uintptr_t>(out_y) % 8) ||
      out_row_stride < F || out_row_stride % 4)
    return fail(HB_ERR_STRIDE, "out_h and out_y must be 8-byte aligned with a row stride >= F and a multiple of 4");
  if ((st = check_extent("proj_residual", "h", N, h_row_stride, F)) ||
      (st = check_extent("proj_residual", "out", N, out_row_stride, F)))
    return st;
  {
    const char* wn = "proj_residual";
    const int64_t ob = rows_bytes(N, out_row_stride, F, 2), xb = rows_bytes(N, x_row_stride, K, 2);
    const int64_t wb = rows_bytes(F, w_row_stride, K, 2), cb = static_cast<int64_t>(F) * 4;
    if ((st = check_no_overlap(wn, "out_h", out_h, out_row_stride, F, "h", h, h_row_stride, F, N, 2, true)) ||
        (st = check_no_overlap(wn, "out_y", out_y, out_row_stride, F, "h", h, h_row_stride, F, N, 2, false)) ||
        (st = check_no_overlap(wn, "out_y", out_y, out_row_stride, F, "out_h", out_h, out_row_stride, F, N, 2,
                               false)) ||
        (st = check_disjoint(wn, "out_h", out_h, ob, "x", x, xb)) ||
        (st = check_disjoint(wn, "out_h", out_h, ob, "w", w, wb)) ||
        (st = check_disjoint(wn, "out_h", out_h, ob, "bias", bias, cb)) ||
        (st = check_disjoint(wn, "out_h", out_h, ob, "dyt parameters", dyt, 2 * cb + 4)) ||
        (st = check_disjoint(wn, "out_y", out_y, ob, "x", x, xb)) ||
        (st = check_disjoint(wn, "out_y", out_y, ob, "w", w, wb)) ||
        (st = check_disjoint(wn, "out_y", out_y, ob, "bias", bias, cb)) ||
        (st = check_disjoint(wn, "out_y", out_y, ob, "dyt parameters", dyt, 2 * cb + 4)))
      return st;
  }
  proj::Args a{};
  a.w = static_cast<const uint16_t*>(w);
  a.x = static_cast<const uint16_t*>(x);
  a.w_rs = w_row_stride;
  a.x_rs = x_row_stride;
  a.K = K;
  a.F = F;
  a.B = 1;
  a.L = static_cast<int>(N);
  a.Lp = static_cast<int>(round_up(N, 128));
  a.nF = F / proj::FT;
  a.nT = static_cast<int>((a.Lp + kProjTokens - 1) / kProjTokens);
  a.out = static_cast<uint16_t*>(out_h);
  a.out_rs = out_row_stride;
  a.res = static_cast<const uint16_t*>(h);
  a.res_rs = h_row_stride;
  a.bias = bias;
  a.dyt = dyt;
  a.out_y = static_cast<uint16_t*>(out_y);
  const unsigned grid = static_cast<unsigned>(a.nF * a.nT);
  if (dtype == HB_F16)
    hipLaunchKernelGGL((proj::proj_gemm<F16Io, proj::kResidual, kProjWaves, kProjTokens>), dim3(grid),
                       dim3(64 * kProjWaves), 0, stream, a);
  else
    hipLaunchKernelGGL((proj::proj_gemm<Bf16Io, proj::kResidual, kProjWaves, kProjTokens>), dim3(grid),
                       dim3(64 * kProjWaves), 0, stream, a);
  return launched("proj_residual");
}

// The attention over a projection: q and q_diff from rows [q | q_diff] (the qq buffer of hb_dit_qkv_proj) against
// the workspace that hb_dit_qkv_proj filled.
extern "C" int hb_dense_attend_qq(hipStream_t stream, const void* qq, int dtype, int64_t row_stride,
                                  const float* q_weight, const float* k_weight, const float* cos, const float* sin,
                                  int half, const float* lam, void* out, int B, int L, int H, int D, float eps,
                                  const void* workspace, size_t workspace_bytes) {
  clear_error();
  if (dtype != HB_BF16 && dtype != HB_F16)
    return fail(HB_ERR_DTYPE, "hb_dense_attend_qq takes HB_BF16 or HB_F16 (dtype %d)", dtype);
  int st = check_common(dtype, static_cast<int64_t>(5) * H * D, B, L, H, D, half);
  if (st) return st;
  if (!(eps >= 0.0f) || !isfinite(eps)) return fail(HB_ERR_EPS, "eps %g must be finite and >= 0", eps);
  if (row_stride < static_cast<int64_t>(2) * H * D || row_stride % 8)
    return fail(HB_ERR_STRIDE, "qq row_stride %lld must be >= 2*H*D and a multiple of 8",
                static_cast<long long>(row_stride));
  if ((st = check_extent("dense_attend_qq", "qq", static_cast<int64_t>(B) * L, row_stride,
                         static_cast<int64_t>(2) * H * D)))
    return st;
  if (half % 8) return fail(HB_ERR_HALF, "half %d must be a multiple of 8", half);
  if (!qq || !q_weight || !k_weight || !out) return fail(HB_ERR_NULL, "qq, q_weight, k_weight and out must be non-NULL");
  if (half > 0 && (!cos || !sin)) return fail(HB_ERR_NULL, "cos and sin must be non-NULL when half > 0");
  if (reinterpret_cast<uintptr_t>(qq) % 16) return fail(HB_ERR_STRIDE, "qq must be 16-byte aligned");
  if (half > 0 && (reinterpret_cast<uintptr_t>(cos) % 16 || reinterpret_cast<uintptr_t>(sin) % 16))
    return fail(HB_ERR_STRIDE, "cos and sin must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(out) % 8) return fail(HB_ERR_STRIDE, "out must be 8-byte aligned");
  const DenseLayout lay = dense_layout(dtype, B, L, H, D);
  if (!workspace) return fail(HB_ERR_NULL, "workspace must be non-NULL");
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(HB_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (workspace_bytes < lay.total_bytes)
    return fail(HB_ERR_WORKSPACE, "workspace holds %zu bytes, needs %zu", workspace_bytes, lay.total_bytes);
  {
    const int64_t HD = static_cast<int64_t>(H) * D, rows = static_cast<int64_t>(B) * L, ob = rows * HD * 2;
    if ((st = check_disjoint("dense_attend_qq", "out", out, ob, "qq", qq, rows_bytes(rows, row_stride, 2 * HD, 2))) ||
        (st = check_disjoint("dense_attend_qq", "out", out, ob, "workspace", workspace,
                             static_cast<int64_t>(lay.total_bytes))))
      return st;
  }
  return launch_dense_attend_16bit(stream, dtype, qq, row_stride, 1, q_weight, k_weight, cos, sin, half, eps, lam, out, B,
                                   L, L, H, D, lay, workspace);
}
