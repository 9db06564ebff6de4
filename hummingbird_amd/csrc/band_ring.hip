// SAME-L sliding-window (band) differential attention, streaming form, for gfx950 (MI355X).
//
// Replaces the reference's fused TPU kernel sa3jax/band_attention.py:61-180 and the XLA chain
// sa3jax/same_l.py:151-169 for head_dim 64, half-width w <= 128, bf16, rotary half-width a multiple of 8.
//
// One workgroup of 8 waves per CU walks a contiguous run of 64-query steps along the sequence of one
// (batch, head). The keys step j can reach, [64j - 64C, 64j + 64 + 64C) with C = ceil(w / 64), live in an LDS
// ring of 2C + 1 tiles of 64 keys, each holding K and K_diff after DyT (same_l.py:58-69) and rotate-half RoPE
// (same_l.py:92-100) rounded once to bf16, and the raw V rows. A step retires the oldest tile and adds one,
// so every key is prepared once per run (the reference's kernel prepares each key block three times, once per
// halo; band_attention.py:155-169).
//
// The waves have two roles, one of each on every SIMD, so that one role's VALU work runs while the other
// waits on LDS, memory or the matrix core:
//   - attention waves 0-3, wave = (query half, branch): 32 queries of one differential branch. Per ring tile
//     that meets their band: S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_32x32x16_bf16 (attn_tile.h layouts),
//     32-key halves outside the band skipped and the halves cut by its edge masked per score
//     (|k - q| <= w, 0 <= k < S; band_attention.py:108-110). At the end of the step the branch-2 waves hand
//     lam * O2 / l2 to the branch-1 waves through LDS, which write O1 / l1 - lam * O2 / l2 in fp32 with one
//     bf16 cast (same_l.py:168-169).
//   - prep waves 4-7: meanwhile load and prepare the next step's key tile (k, k_diff: DyT + RoPE; v: copied)
//     and its 64 queries (q, q_diff: DyT + RoPE + softmax scale), one (row, RoPE group pair) task each, so the
//     rotation partner and the cos/sin slice are in the thread's own registers.
// Two barriers per step: after the first the prep waves store the new tile into the retired slot and the new
// queries into the query buffer; the second publishes them.
//
// Rows are 128 B without padding; 16-byte chunks are XOR-swizzled per row so that the K fragment reads
// (ds_read_b128, 8 or 16 rows per cycle), the transposing V reads (ds_read_b64_tr_b16, 4 rows x 32 B per 16
// lanes) and the Q reads hit distinct banks.
//
// The runs are the flattened (batch, head, step) range split evenly over one workgroup per CU; consecutive
// workgroups go to different XCDs, so the same run position of every head (the same RoPE rows) shares an L2.
#include "api.h"
#include "attn_tile.h"
#include "common.h"

namespace hb {
namespace band_ring {

constexpr int D = 64;
constexpr int NT = 512;       // 8 waves
constexpr int QT = 64;        // queries per step
constexpr int KT = 64;        // keys per ring tile
constexpr int TE = KT * D;    // elements of one tensor in a tile (8 KB)
constexpr int TILE = 3 * TE;  // K, K_diff, V
constexpr int XF = 2 * 2 * 16 * 64;  // exchange floats: 2 query halves x 2 d-tiles x 16 registers x 64 lanes

// Physical element offset of logical 16-byte chunk c of row r. K, K_diff, q, q_diff: the MFMA operand reads
// take one chunk of 8 (or 16) consecutive rows per cycle. V: the transposing read takes two adjacent chunks of
// 4 consecutive rows per 16 lanes.
__device__ __forceinline__ int kofs(int r, int c) { return r * D + 8 * (c ^ (r & 7) ^ ((r >> 3) & 1)); }
__device__ __forceinline__ int vofs(int r, int c) { return r * D + 8 * (c ^ ((r & 3) << 1)); }

// DyT(x) = gamma * tanh(alpha x) + beta with tanh(y) = 1 - 2 / (1 + 2^(2 log2(e) y)):
// y = (gamma + beta) + (-2 gamma) / (1 + 2^(a2 x)), a2 = 2 log2(e) alpha. Two transcendental instructions.
__device__ __forceinline__ float dyt(float x, float a2, float g2, float gb) {
  return __fmaf_rn(g2, __builtin_amdgcn_rcpf(1.f + fast_exp2(a2 * x)), gb);
}

// Raw inputs of one prep task: groups m1, m2 of tensors A and B (k and k_diff, or q and q_diff) of one row,
// and the cos / sin slice of frequencies 8 m1 .. 8 m1 + 7 (1 and 0 when the pair is not rotated).
struct Raw {
  u32x4 a1, a2, b1, b2;
  f32x4 c0, c1, s0, s1;
};
struct Prepped {
  u32x4 a1, a2, b1, b2;
};

// DyT + RoPE (+ scale) of one task; A and B share the DyT parameters `par` = [-2 gamma (D) | gamma + beta (D)].
__device__ __forceinline__ void prep_task(const Raw& r, int m1, int m2, float a2, const float* __restrict__ par,
                                          float scale, Prepped& o) {
  const float cs[8] = {r.c0[0], r.c0[1], r.c0[2], r.c0[3], r.c1[0], r.c1[1], r.c1[2], r.c1[3]};
  const float sn[8] = {r.s0[0], r.s0[1], r.s0[2], r.s0[3], r.s1[0], r.s1[1], r.s1[2], r.s1[3]};
#pragma unroll
  for (int tsr = 0; tsr < 2; ++tsr) {
    float x1[8], x2[8], o1[8], o2[8];
    unpack8(tsr ? r.b1 : r.a1, x1);
    unpack8(tsr ? r.b2 : r.a2, x2);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float y1 = dyt(x1[j], a2, par[8 * m1 + j], par[D + 8 * m1 + j]);
      const float y2 = dyt(x2[j], a2, par[8 * m2 + j], par[D + 8 * m2 + j]);
      // rotate_half: d < half takes -x[d + half], d >= half takes x[d - half]
      o1[j] = __fmaf_rn(y1, cs[j], -(y2 * sn[j])) * scale;
      o2[j] = __fmaf_rn(y2, cs[j], y1 * sn[j]) * scale;
    }
    if (tsr) {
      o.b1 = pack8(o1);
      o.b2 = pack8(o2);
    } else {
      o.a1 = pack8(o1);
      o.a2 = pack8(o2);
    }
  }
}

// One ring tile for an attention wave: 32 queries, one branch. EDGE = false: every key of the tile is in the
// band of every query. EDGE = true: 32-key half rt takes part if act_rt and is masked per score if msk_rt;
// [lo, hi] are the keys (relative to the tile start, minus 4 lh) this lane's query may see.
template <bool FAST, bool EDGE>
__device__ __forceinline__ void tile_step(const uint16_t* __restrict__ sk, const uint16_t* __restrict__ sv,
                                          const int (&koff)[4], const int (&voff)[2], const u32x4 (&qf)[4],
                                          f32x16 (&o)[2], float& lsum, float& m, float c, bool act0, bool act1,
                                          bool msk0, bool msk1, int lo, int hi) {
  const bool act[2] = {EDGE ? act0 : true, EDGE ? act1 : true};
  const bool msk[2] = {EDGE && msk0, EDGE && msk1};
  f32x16 sc[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    sc[rt] = f32x16{};
    if (act[rt]) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) sc[rt] = mfma_bf16_32x32x16(lds16(sk + rt * 32 * D + koff[kk]), qf[kk], sc[rt]);
    }
  }
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    if (msk[rt]) {
      const unsigned span = static_cast<unsigned>(hi - lo);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kc = 32 * rt + 8 * (r >> 2) + (r & 3);
        sc[rt][r] = static_cast<unsigned>(kc - lo) <= span ? sc[rt][r] : -INFINITY;
      }
    }
  }
  float mb = 0.f;
  if constexpr (!FAST) {
    float mt = -INFINITY;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
      if (act[rt]) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sc[rt][r]);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 32, kWave)) * c;
    const float mn = fmaxf(m, mt);
    // mn == -inf only while every key seen so far is masked; keep the state at zero then.
    const float alpha = mn == -INFINITY ? 1.f : fast_exp2(m - mn);
    m = mn;
    lsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) o[dt] *= alpha;
    mb = mn == -INFINITY ? 0.f : mn;
  }
  u32x4 pb[2][2];  // [rt][16-key half]: 8 bf16 probabilities each
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    if (!act[rt]) continue;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float e0, e1;
        if constexpr (FAST) {
          e0 = fast_exp2(sc[rt][8 * hh + 2 * j]);
          e1 = fast_exp2(sc[rt][8 * hh + 2 * j + 1]);
        } else {
          e0 = fast_exp2(__fmaf_rn(sc[rt][8 * hh + 2 * j], c, -mb));
          e1 = fast_exp2(__fmaf_rn(sc[rt][8 * hh + 2 * j + 1], c, -mb));
        }
        const uint32_t p = pack_bf16x2(e0, e1);
        pb[rt][hh][j] = p;
        lsum = add_bf16_pair(p, lsum);
      }
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    if (!act[g >> 1]) continue;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      lds_i16x4* p0 = (lds_i16x4*)(sv + g * 16 * D + voff[dt]);
      lds_i16x4* p1 = (lds_i16x4*)(sv + g * 16 * D + 8 * D + voff[dt]);
      const u32x2 ua = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(p0));
      const u32x2 ub = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(p1));
      o[dt] = mfma_bf16_32x32x16(u32x4{ua[0], ua[1], ub[0], ub[1]}, pb[g >> 1][g & 1], o[dt]);
    }
  }
}

struct Args {
  const uint16_t* qkv;
  int64_t rs;
  int S, H, w, half, NS;
  int64_t total;  // B * H * NS steps
  const float* q_dyt;
  const float* k_dyt;
  const float* cosT;
  const float* sinT;
  const float* lam;
  uint16_t* out;
};

template <int C, bool FAST>
__device__ __forceinline__ void run(const Args& a, uint16_t* ring, uint16_t* qbuf, float* xbuf, const float* qpar,
                                    const float* kpar, float qa2, float ka2, const SoftmaxPlan& plan) {
  constexpr int RING = 2 * C + 1;
  const int t = threadIdx.x, lane = t & 63, wave = wave_id(), lr = lane & 31, lh = lane >> 5;
  const bool prep_role = wave >= 4;  // uniform per wave
  const int S = a.S, H = a.H, w = a.w, half = a.half;
  const int64_t HD = static_cast<int64_t>(H) * D;
  const int h8 = half >> 3;
  const int64_t G = gridDim.x, gi = blockIdx.x;
  const int64_t f_beg = a.total * gi / G, f_end = a.total * (gi + 1) / G;

  // Prep geometry (waves 4-7): task row pt / 4, RoPE group pair pt % 4; V chunks pt and pt + 256.
  const int pt = t & 255, prow = pt >> 2, pp = pt & 3;
  int m1, m2;
  pair_groups(pp, h8, m1, m2);
  const bool prot = pp < h8;
  // Attention geometry (waves 0-3): query half, branch, per-lane LDS fragment offsets.
  const int qhalf = wave & 1, br = (wave >> 1) & 1;
  const int kswz = (lr & 7) ^ ((lr >> 3) & 1);
  int koff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) koff[kk] = lr * D + 8 * ((2 * kk + lh) ^ kswz);
  const int grp = lane >> 4, mm = lane & 15;
  int voff[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    const int col = 32 * dt + 16 * (grp & 1) + 4 * (mm & 3);
    voff[dt] = (4 * (grp >> 1) + (mm >> 2)) * D + 8 * ((col >> 3) ^ ((mm >> 2) << 1)) + (col & 7);
  }

  for (int64_t f = f_beg; f < f_end;) {
    const int bh = static_cast<int>(f / a.NS);
    const int j0 = static_cast<int>(f % a.NS);
    const int j1 = static_cast<int>(f_end - f < a.NS - j0 ? j0 + (f_end - f) : a.NS);
    const int b = bh / H, h = bh % H;
    const uint16_t* xb = a.qkv + static_cast<int64_t>(b) * S * a.rs + h * D;

    // ---- prep role -------------------------------------------------------------------------------------
    Raw kr, qr;
    Prepped ko, qo;
    u32x4 vr[2];
    // Raw rows of key tile kt (this thread's task row, two V chunks) and of the queries of step jj. Rows
    // outside [0, S) are read from a clamped position: their keys are always masked, their V chunks are
    // replaced by zeros and their queries are never stored.
    auto load_raw = [&](Raw& r, int pos, int sa, int sb) {
      const int cp = pos < 0 ? 0 : (pos < S ? pos : S - 1);
      const uint16_t* row = xb + static_cast<int64_t>(cp) * a.rs;
      r.a1 = ld16(row + sa * HD + 8 * m1);
      r.a2 = ld16(row + sa * HD + 8 * m2);
      r.b1 = ld16(row + sb * HD + 8 * m1);
      r.b2 = ld16(row + sb * HD + 8 * m2);
      if (half > 0) {
        const int64_t toff = static_cast<int64_t>(cp) * half + (prot ? 8 * m1 : 0);
        const f32x4 one = {1.f, 1.f, 1.f, 1.f}, zero = {0.f, 0.f, 0.f, 0.f};
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(a.cosT + toff);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(a.cosT + toff + 4);
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(a.sinT + toff);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(a.sinT + toff + 4);
        r.c0 = prot ? c0 : one;
        r.c1 = prot ? c1 : one;
        r.s0 = prot ? s0 : zero;
        r.s1 = prot ? s1 : zero;
      } else {
        r.c0 = r.c1 = f32x4{1.f, 1.f, 1.f, 1.f};
        r.s0 = r.s1 = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    };
    auto load_tile = [&](int kt) {
      load_raw(kr, KT * kt + prow, 1, 4);  // k, k_diff
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ch = pt + 256 * u, vpos = KT * kt + (ch >> 3);
        const int vc = vpos < 0 ? 0 : (vpos < S ? vpos : S - 1);
        const u32x4 v = ld16(xb + static_cast<int64_t>(vc) * a.rs + 2 * HD + 8 * (ch & 7));
        vr[u] = vpos == vc ? v : u32x4{0u, 0u, 0u, 0u};
      }
    };
    auto store_tile = [&](int kt) {
      uint16_t* base = ring + ((kt % RING + RING) % RING) * TILE;
      *reinterpret_cast<u32x4*>(base + kofs(prow, m1)) = ko.a1;
      *reinterpret_cast<u32x4*>(base + kofs(prow, m2)) = ko.a2;
      *reinterpret_cast<u32x4*>(base + TE + kofs(prow, m1)) = ko.b1;
      *reinterpret_cast<u32x4*>(base + TE + kofs(prow, m2)) = ko.b2;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ch = pt + 256 * u;
        *reinterpret_cast<u32x4*>(base + 2 * TE + vofs(ch >> 3, ch & 7)) = vr[u];
      }
    };
    auto store_q = [&]() {
      *reinterpret_cast<u32x4*>(qbuf + kofs(prow, m1)) = qo.a1;
      *reinterpret_cast<u32x4*>(qbuf + kofs(prow, m2)) = qo.a2;
      *reinterpret_cast<u32x4*>(qbuf + TE + kofs(prow, m1)) = qo.b1;
      *reinterpret_cast<u32x4*>(qbuf + TE + kofs(prow, m2)) = qo.b2;
    };

    // Fill the ring for step j0 (tiles j0 - C .. j0 + C) and the query buffer.
    if (prep_role) {
#pragma unroll 1
      for (int i = 0; i < RING; ++i) {
        load_tile(j0 - C + i);
        prep_task(kr, m1, m2, ka2, kpar, 1.f, ko);
        store_tile(j0 - C + i);
      }
      load_raw(qr, QT * j0 + prow, 0, 3);  // q, q_diff
      prep_task(qr, m1, m2, qa2, qpar, plan.qscale, qo);
      store_q();
    }
    __syncthreads();

#pragma unroll 1
    for (int j = j0; j < j1; ++j) {
      const bool next = j + 1 < j1;
      if (prep_role) {
        if (next) {
          load_tile(j + 1 + C);
          load_raw(qr, QT * (j + 1) + prow, 0, 3);
          prep_task(kr, m1, m2, ka2, kpar, 1.f, ko);
          prep_task(qr, m1, m2, qa2, qpar, plan.qscale, qo);
        }
        __syncthreads();  // the attention waves are done with the oldest tile and the query buffer
        if (next) {
          store_tile(j + 1 + C);
          store_q();
        }
        __syncthreads();
      } else {
        // ---- attention role ----------------------------------------------------------------------------
        u32x4 qf[4];
        const uint16_t* qsrc = qbuf + br * TE + 32 * qhalf * D;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) qf[kk] = lds16(qsrc + koff[kk]);
        f32x16 o[2] = {f32x16{}, f32x16{}};
        float lsum = 0.f, m = -INFINITY;
        const int qa = QT * j + 32 * qhalf;  // this wave's first query
        const int q = qa + lr;
        const int ulo = qa - w > 0 ? qa - w : 0;  // union band of the wave's queries
        const int uhi = qa + 31 + w < S - 1 ? qa + 31 + w : S - 1;
        const int qlo = q - w > 0 ? q - w : 0;    // this lane's band
        const int qhi = q + w < S - 1 ? q + w : S - 1;
#pragma unroll 1
        for (int i = 0; i < RING; ++i) {
          const int kt = j - C + i, kt0 = KT * kt;
          const uint16_t* base = ring + ((kt % RING + RING) % RING) * TILE;
          bool act[2], full[2];
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const int k0 = kt0 + 32 * rt, k1 = k0 + 31;
            act[rt] = k1 >= ulo && k0 <= uhi;
            full[rt] = k0 >= qa + 31 - w && k1 <= qa + w && k0 >= 0 && k1 <= S - 1;
          }
          if (!act[0] && !act[1]) continue;
          if (act[0] && act[1] && full[0] && full[1])
            tile_step<FAST, false>(base + br * TE, base + 2 * TE, koff, voff, qf, o, lsum, m, plan.c, true, true,
                                   false, false, 0, 0);
          else
            tile_step<FAST, true>(base + br * TE, base + 2 * TE, koff, voff, qf, o, lsum, m, plan.c, act[0],
                                  act[1], act[0] && !full[0], act[1] && !full[1], qlo - kt0 - 4 * lh,
                                  qhi - kt0 - 4 * lh);
        }
        // Branch 2 publishes lam * O2 / l2 (rounded per element); branch 1 subtracts it from O1 / l1.
        const float inv = __frcp_rn(lsum + __shfl_xor(lsum, 32, kWave));
        float* xs = xbuf + qhalf * (2 * 16 * 64);
        if (br == 1) {
          const float li = __fmul_rn(a.lam ? a.lam[h] : 1.f, inv);
#pragma unroll
          for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) xs[(dt * 16 + r) * 64 + lane] = __fmul_rn(o[dt][r], li);
        }
        __syncthreads();
        if (br == 0) {
          uint16_t* orow = a.out + (static_cast<int64_t>(b) * S + q) * HD + h * D;
#pragma unroll
          for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              float v[4];
#pragma unroll
              for (int jj = 0; jj < 4; ++jj) {
                const int r = 4 * g + jj;
                v[jj] = __fsub_rn(__fmul_rn(o[dt][r], inv), xs[(dt * 16 + r) * 64 + lane]);
              }
              if (q < S) {
                u32x2 pk;
                pk[0] = pack_bf16x2(v[0], v[1]);
                pk[1] = pack_bf16x2(v[2], v[3]);
                *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * g + 4 * lh) = pk;
              }
            }
        }
        __syncthreads();
      }
    }
    f += j1 - j0;
  }
}

// |DyT(x)| bound: sqrt(sum_d (|gamma_d| + |beta_d|)^2), reduced over the wave.
__device__ __forceinline__ float dyt_bound(const float* __restrict__ dyt) {
  const int lane = threadIdx.x & 63;
  const float v = fabsf(dyt[1 + lane]) + fabsf(dyt[1 + D + lane]);
  float acc = v * v;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, kWave);
  return sqrtf(acc);
}

template <int C>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void band_ring_bf16(Args a) {
  constexpr int RING = 2 * C + 1;
  __shared__ __attribute__((aligned(16))) uint16_t ring[RING * TILE];
  __shared__ __attribute__((aligned(16))) uint16_t qbuf[2 * TE];  // q, q_diff of the step (64 rows each)
  __shared__ __attribute__((aligned(16))) float xbuf[XF];
  __shared__ __attribute__((aligned(16))) float par[4 * D];  // q: -2 gamma, gamma + beta; k: the same
  const int t = threadIdx.x;
  if (t < D) {
    const float qg = a.q_dyt[1 + t], qb = a.q_dyt[1 + D + t], kg = a.k_dyt[1 + t], kb = a.k_dyt[1 + D + t];
    par[t] = -2.f * qg;
    par[D + t] = qg + qb;
    par[2 * D + t] = -2.f * kg;
    par[3 * D + t] = kg + kb;
  }
  const SoftmaxPlan plan = softmax_plan(dyt_bound(a.q_dyt), dyt_bound(a.k_dyt), D);
  const float qa2 = 2.f * kLog2e * a.q_dyt[0], ka2 = 2.f * kLog2e * a.k_dyt[0];
  __syncthreads();
  if (plan.fast)
    run<C, true>(a, ring, qbuf, xbuf, par, par + 2 * D, qa2, ka2, plan);
  else
    run<C, false>(a, ring, qbuf, xbuf, par, par + 2 * D, qa2, ka2, plan);
}

}  // namespace band_ring

bool band_ring_supported(int dtype, int D, int half, int window) {
  return dtype == HB_BF16 && D == band_ring::D && half % 8 == 0 && window <= 128;
}

int launch_band_ring(hipStream_t stream, const void* qkv, int64_t rs, const float* q_dyt, const float* k_dyt,
                     const float* cosT, const float* sinT, int half, int window, const float* lam, void* out, int B,
                     int S, int H) {
  using namespace band_ring;
  static int cu_count[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  int ncu = dev < 64 ? cu_count[dev] : 0;
  if (ncu <= 0) {
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0) ncu = 256;
    if (dev < 64) cu_count[dev] = ncu;
  }
  Args a;
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.rs = rs;
  a.S = S;
  a.H = H;
  a.w = window;
  a.half = half;
  a.NS = (S + QT - 1) / QT;
  a.total = static_cast<int64_t>(B) * H * a.NS;
  a.q_dyt = q_dyt;
  a.k_dyt = k_dyt;
  a.cosT = cosT;
  a.sinT = sinT;
  a.lam = lam;
  a.out = static_cast<uint16_t*>(out);
  const int64_t grid = a.total < ncu ? a.total : ncu;
  const int C = (window + 63) / 64;
  if (C == 0)
    hipLaunchKernelGGL(band_ring_bf16<0>, dim3(static_cast<unsigned>(grid)), dim3(NT), 0, stream, a);
  else if (C == 1)
    hipLaunchKernelGGL(band_ring_bf16<1>, dim3(static_cast<unsigned>(grid)), dim3(NT), 0, stream, a);
  else
    hipLaunchKernelGGL(band_ring_bf16<2>, dim3(static_cast<unsigned>(grid)), dim3(NT), 0, stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HB_ERR_LAUNCH, "band_ring launch failed: %s", hipGetErrorString(e));
  return HB_OK;
}

}  // namespace hb
