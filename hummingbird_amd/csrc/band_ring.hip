// SAME-L sliding-window (band) differential attention, streaming form, for gfx950 (MI355X).
//
// Replaces the reference's fused TPU kernel sa3jax/band_attention.py:61-180 and the XLA chain
// sa3jax/same_l.py:151-169 for head_dim 64, half-width w <= 128, bf16 or half inputs (bf16 operands either way),
// rotary half-width a multiple of 8.
//
// One workgroup of 8 waves per CU walks a contiguous run of 64-query steps along the sequence of one
// (batch, head). The keys step j can reach, [64j - 64C, 64j + 64 + 64C) with C = ceil(w / 64), live in an LDS
// ring of 2C + 1 tiles of 64 keys, each holding K and K_diff after DyT (same_l.py:58-69) and rotate-half RoPE
// (same_l.py:92-100) rounded once to bf16, and the raw V rows (K and K_diff in one ring, V in another). A step
// retires the oldest tile and adds one, so every key is prepared once per run (the reference's kernel prepares
// each key block three times, once per halo; band_attention.py:155-169).
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
//     rotation partner and the cos/sin slice are in the thread's own registers. For bf16 inputs with C <= 1 the
//     V rows skip the prep waves: the attention waves copy them from HBM straight into a spare V ring slot
//     (global_load_lds) a step ahead.
// Two barriers per step: after the first the prep waves store the new tile into the retired slot and the new
// queries into the query buffer; the second publishes them. The prep waves run at a higher issue priority, except
// that at C <= 1 the attention waves' exchange and epilogue go first.
//
// Steps away from the sequence ends (all but a few per run) have a tile pattern fixed by w alone: the wave's
// 32-key halves t = -T .. T around the half that holds its own queries take part (T = floor((w + 31) / 32)), and
// those with |t| >= M = floor((w + 1) / 32) are cut by one band edge (both when t = 0). Those steps run a separate,
// fully unrolled loop with their pattern built in (four patterns per C); the general loop covers the rest.
//
// Rows are 128 B without padding; 16-byte chunks are XOR-swizzled per row so that the K fragment reads
// (ds_read_b128, 8 or 16 rows per cycle), the transposing V reads (ds_read_b64_tr_b16, 4 rows x 32 B per 16
// lanes) and the Q reads hit distinct banks.
//
// The runs are the flattened (batch, head, step) range split over one workgroup per CU, evenly, or weighted by
// ring fills where (batch, head) boundaries fall inside workgroups (Range); consecutive workgroups go to
// different XCDs, so the same run position of every head (the same RoPE rows) shares an L2.
#include <type_traits>

#include "api.h"
#include "attn_tile.h"
#include "common.h"
#include "tiles.h"

namespace hb {
namespace band_ring {

constexpr int D = 64;
constexpr int NT = 512;       // 8 waves
constexpr int QT = 64;        // queries per step
constexpr int KT = 64;        // keys per ring tile
constexpr int TE = KT * D;    // elements of one tensor in a tile (8 KB)
constexpr int KTILE = 2 * TE; // K, K_diff of one ring slot
constexpr int XF = 2 * 2 * 16 * 64;  // exchange floats: 2 query halves x 2 d-tiles x 16 registers x 64 lanes

// Physical element offset of logical 16-byte chunk c of row r. K, K_diff, q, q_diff: the MFMA operand reads
// take one chunk of 8 (or 16) consecutive rows per cycle. V: the transposing read takes two adjacent chunks of
// 4 consecutive rows per 16 lanes.
__device__ __forceinline__ int kofs(int r, int c) { return r * D + 8 * (c ^ (r & 7) ^ ((r >> 3) & 1)); }
__device__ __forceinline__ int vofs(int r, int c) { return r * D + 8 * (c ^ ((r & 3) << 1)); }

// Raw inputs of one prep task: groups m1, m2 of tensors A and B (k and k_diff, or q and q_diff) of one row,
// and the cos / sin slice of frequencies 8 m1 .. 8 m1 + 7 (unused when the pair is not rotated, or half = 0).
struct Raw {
  u32x4 a1, a2, b1, b2;
  f32x4 c0, c1, s0, s1;
};
struct Prepped {
  u32x4 a1, a2, b1, b2;
};

struct Par {
  float g1[8], b1[8], g2[8], b2[8];
};
// -2 gamma and gamma + beta of groups m1, m2 from `dyt` = [alpha, gamma[D], beta[D]].
__device__ __forceinline__ Par load_par(const float* __restrict__ dyt, int m1, int m2) {
  Par p;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float ga = dyt[1 + 8 * m1 + j], be = dyt[1 + D + 8 * m1 + j];
    const float gc = dyt[1 + 8 * m2 + j], bd = dyt[1 + D + 8 * m2 + j];
    p.g1[j] = -2.f * ga;
    p.b1[j] = ga + be;
    p.g2[j] = -2.f * gc;
    p.b2[j] = gc + bd;
  }
  return p;
}
// DyT + RoPE (+ scale) of one task; A and B share the DyT parameters `p` (-2 gamma, gamma + beta per dim).
// `rot`: the pair is rotated (otherwise cos 1, sin 0).
template <class IO>
__device__ __forceinline__ void prep_task(const Raw& r, bool rot, float a2, const Par& p, float scale, Prepped& o) {
  float cs[8] = {r.c0[0], r.c0[1], r.c0[2], r.c0[3], r.c1[0], r.c1[1], r.c1[2], r.c1[3]};
  float sn[8] = {r.s0[0], r.s0[1], r.s0[2], r.s0[3], r.s1[0], r.s1[1], r.s1[2], r.s1[3]};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    cs[j] = rot ? cs[j] : 1.f;
    sn[j] = rot ? sn[j] : 0.f;
  }
#pragma unroll
  for (int tsr = 0; tsr < 2; ++tsr) {
    float x1[8], x2[8], o1[8], o2[8];
    IO::unpack8(tsr ? r.b1 : r.a1, x1);
    IO::unpack8(tsr ? r.b2 : r.a2, x2);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float y1 = dyt_tanh(x1[j], a2, p.g1[j], p.b1[j]);
      const float y2 = dyt_tanh(x2[j], a2, p.g2[j], p.b2[j]);
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

// K fragments of one ring tile for an attention wave (key row 32 rt + lr, dims 16 kk + 8 lh .. +8), for the
// 32-key halves that take part (act0, act1: wave-uniform, constants in the unrolled interior loops).
__device__ __forceinline__ void kload(const uint16_t* __restrict__ sk, const int (&koff)[4], u32x4 (&kf)[2][4],
                                      bool act0 = true, bool act1 = true) {
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    if (!(rt == 0 ? act0 : act1)) continue;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) kf[rt][kk] = lds16(sk + rt * 32 * D + koff[kk]);
  }
}

// S^T of one ring tile for an attention wave: 64 keys x its 32 queries, for the 32-key halves that take part
// (act0, act1: wave-uniform; a half that does not keeps its registers and is never read).
__device__ __forceinline__ void qk(const u32x4 (&kf)[2][4], const u32x4 (&qf)[4], f32x16 (&sc)[2], bool act0,
                                   bool act1) {
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    if (!(rt == 0 ? act0 : act1)) continue;
    sc[rt] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) sc[rt] = mfma_bf16_32x32x16(kf[rt][kk], qf[kk], sc[rt]);
  }
}

// Softmax and PV of one ring tile from its scores `sc` (read only, so the caller's score buffers keep their
// registers). act_rt: 32-key half rt takes part; msk_rt: it is cut by the band edge or the sequence end and is
// masked per score to the keys [lo, lo + span] (relative to the tile start, minus 4 lh) this lane's query may
// see. Both flags are wave-uniform.
template <bool FAST>
__device__ __forceinline__ void soft_pv(const f32x16 (&sc)[2], const uint16_t* __restrict__ sv, const int (&voff)[2],
                                        f32x16 (&o)[2], float& lsum, float& m, float c, bool act0, bool act1,
                                        int mode0, int mode1, int lo, unsigned span) {
  const bool act[2] = {act0, act1};
  const int mode[2] = {mode0, mode1};
  const bool msk[2] = {mode0 != 0, mode1 != 0};

  // A masked-out score's probability is exp2(-inf) = 0. Mode bit 0: the lower band edge cuts the half (keep
  // kc >= lo), bit 1: the upper one (keep kc <= lo + span); a half cut by one edge only pays one compare.
  auto score = [&](int rt, int r) {
    const int kc = 32 * rt + 8 * (r >> 2) + (r & 3);
    bool out;
    if (mode[rt] == 1)
      out = kc < lo;
    else if (mode[rt] == 2)
      out = kc > lo + static_cast<int>(span);
    else
      out = static_cast<unsigned>(kc - lo) > span;
    return msk[rt] && out ? -INFINITY : sc[rt][r];
  };
  float mb = 0.f;
  if constexpr (!FAST) {
    float mt = -INFINITY;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
      if (act[rt]) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, score(rt, r));
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
  // Masked and unmasked halves are separate code, so unmasked halves pay nothing for the band edges.
  auto probs = [&](int rt, auto sval) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float s0 = sval(8 * hh + 2 * j), s1 = sval(8 * hh + 2 * j + 1);
        float e0, e1;
        if constexpr (FAST) {
          e0 = fast_exp2(s0);
          e1 = fast_exp2(s1);
        } else {
          e0 = fast_exp2(__fmaf_rn(s0, c, -mb));
          e1 = fast_exp2(__fmaf_rn(s1, c, -mb));
        }
        const uint32_t p = pack_bf16x2(e0, e1);
        pb[rt][hh][j] = p;
        lsum = add_bf16_pair(p, lsum);
      }
  };
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    if (!act[rt]) continue;
    if (msk[rt])
      probs(rt, [&](int r) { return score(rt, r); });
    else
      probs(rt, [&](int r) { return sc[rt][r]; });
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
  int fillw;      // the cost of a run's ring fill, in steps (see Range)
  int64_t total;  // B * H * NS steps
  const float* q_dyt;
  const float* k_dyt;
  const float* cosT;
  const float* sinT;
  const float* lam;
  uint16_t* out;
};

// The flattened (batch, head, step) range of this workgroup, walked as runs of consecutive steps of one
// (batch, head). Both roles walk it identically and meet at the same barriers: one after each run's ring fill,
// two per step. A workgroup whose range crosses into the next (batch, head) fills its ring twice, so the split
// is even in a cost that counts each (batch, head) as NS + fillw steps, the first fillw of them standing for
// the fill at its start (fillw = 0: an even split of the steps).
struct Range {
  int64_t beg, end;
  __device__ Range(const Args& a) {
    const int64_t G = gridDim.x, gi = blockIdx.x;
    const int64_t per = a.NS + a.fillw, cost = a.total / a.NS * per;
    beg = step_of(a, cost * gi / G, per);
    end = step_of(a, cost * (gi + 1) / G, per);
  }
  __device__ static int64_t step_of(const Args& a, int64_t c, int64_t per) {
    const int64_t bh = c / per, off = c - bh * per;
    return bh * a.NS + (off > a.fillw ? off - a.fillw : 0);
  }
};

// Raw rows of one step for a prep thread: its key task (k, k_diff), its two V chunks, its query task (q, q_diff).
struct Stage {
  Raw k, q;
  u32x4 v[2];
};

// V rows reach the ring by DMA (global_load_lds, issued by the attention waves a step ahead, into one spare ring
// slot) for bf16 inputs and windows of at most 64 keys, where the prep waves' row loads set the pace. Half inputs
// are converted to bf16 on the way, so their V rows pass through the prep waves' registers; at C = 2 the spare
// slot would fill the LDS, and the copy measured no faster there, so the prep waves load V as well.
template <class IO, int C>
constexpr bool kVdma = std::is_same<IO, Bf16Io>::value && C <= 1;
// V ring slots: one more than the key ring when the next tile's copy lands a step ahead.
template <class IO, int C>
constexpr int kVring = 2 * C + 1 + (kVdma<IO, C> ? 1 : 0);

// The fixed pattern of an interior step for query half QH (see the file comment): the halves t = -T .. T around
// ring half QH + 2C take part, and those with |t| >= M are masked by the band edge on their side.
template <int QH, int T, int M>
struct Interior {
  static constexpr int qh = QH, t = T, m = M;
};
struct General {};

// Ring slot of key tile kt (kt >= -C) in a ring of n slots.
__device__ __forceinline__ int ring_slot(int kt, int n) { return (kt % n + n) % n; }

// Prep waves (4-7): fill the ring at the start of each run, then prepare step j + 1 during step j from rows
// loaded during step j - 1. The step loop is unrolled by two over stage buffers A and B, so a buffer is loaded
// in one step and consumed in the next without being copied (a copy would wait for the loads to land).
template <class IO, int C, bool ALLROT>
__device__ __forceinline__ void prep_waves(const Args& a, uint16_t* kring, uint16_t* vring, uint16_t* qbuf,
                                           float qa2, float ka2, float qscale) {
  constexpr int RING = 2 * C + 1;
  constexpr bool VDMA = kVdma<IO, C>;
  constexpr int VR = kVring<IO, C>;
  const int t = threadIdx.x;
  const int S = a.S, H = a.H, half = a.half;
  const int64_t HD = static_cast<int64_t>(H) * D;
  const int h8 = half >> 3;
  // Task row pt / 4, RoPE group pair pt % 4; V chunks pt and pt + 256.
  const int pt = t & 255, prow = pt >> 2, pp = pt & 3;
  int m1, m2;
  pair_groups(pp, h8, m1, m2);
  const bool prot = ALLROT || pp < h8;
  const Par kp = load_par(a.k_dyt, m1, m2), qp = load_par(a.q_dyt, m1, m2);
  const Range rg(a);

  for (int64_t f = rg.beg; f < rg.end;) {
    const int bh = static_cast<int>(f / a.NS);
    const int j0 = static_cast<int>(f % a.NS);
    const int j1 = static_cast<int>(rg.end - f < a.NS - j0 ? j0 + (rg.end - f) : a.NS);
    const int b = bh / H, h = bh % H;
    const uint16_t* xb = a.qkv + static_cast<int64_t>(b) * S * a.rs + h * D;

    // Rows outside [0, S) are read from a clamped position: their keys are always masked, their V chunks are
    // replaced by zeros when stored and their queries are never stored. The RoPE slice of a pair that is not
    // rotated is read from column 0 and replaced by (1, 0) in prep_task. Nothing here depends on the loaded
    // values, so nothing waits for them until they are used.
    auto load_raw = [&](int pos, int sa, int sb) {
      Raw r;
      const int cp = pos < 0 ? 0 : (pos < S ? pos : S - 1);
      const uint16_t* row = xb + static_cast<int64_t>(cp) * a.rs;
      r.a1 = ld16(row + sa * HD + 8 * m1);
      r.a2 = ld16(row + sa * HD + 8 * m2);
      r.b1 = ld16(row + sb * HD + 8 * m1);
      r.b2 = ld16(row + sb * HD + 8 * m2);
      if (half > 0) {
        const int64_t toff = static_cast<int64_t>(cp) * half + (prot ? 8 * m1 : 0);
        r.c0 = *reinterpret_cast<const f32x4*>(a.cosT + toff);
        r.c1 = *reinterpret_cast<const f32x4*>(a.cosT + toff + 4);
        r.s0 = *reinterpret_cast<const f32x4*>(a.sinT + toff);
        r.s1 = *reinterpret_cast<const f32x4*>(a.sinT + toff + 4);
      } else {
        r.c0 = r.c1 = f32x4{1.f, 1.f, 1.f, 1.f};
        r.s0 = r.s1 = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      return r;
    };
    // Step jj's rows: key tile jj + C and the queries of step jj; the tile's V rows only when `withv`.
    auto load_stage = [&](int jj, bool withv) {
      Stage st;
      const int kt = jj + C;
      st.k = load_raw(KT * kt + prow, 1, 4);  // k, k_diff
      if (withv) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int ch = pt + 256 * u, vpos = KT * kt + (ch >> 3);
          const int vc = vpos < 0 ? 0 : (vpos < S ? vpos : S - 1);
          st.v[u] = ld16(xb + static_cast<int64_t>(vc) * a.rs + 2 * HD + 8 * (ch & 7));
        }
      }
      st.q = load_raw(QT * jj + prow, 0, 3);  // q, q_diff
      return st;
    };
    auto store_k = [&](int kt, const Prepped& ko) {
      uint16_t* base = kring + ring_slot(kt, RING) * KTILE;
      *reinterpret_cast<u32x4*>(base + kofs(prow, m1)) = ko.a1;
      *reinterpret_cast<u32x4*>(base + kofs(prow, m2)) = ko.a2;
      *reinterpret_cast<u32x4*>(base + TE + kofs(prow, m1)) = ko.b1;
      *reinterpret_cast<u32x4*>(base + TE + kofs(prow, m2)) = ko.b2;
    };
    auto store_v = [&](int kt, const u32x4 (&v)[2]) {
      uint16_t* base = vring + ring_slot(kt, VR) * TE;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ch = pt + 256 * u, vpos = KT * kt + (ch >> 3);
        const bool in = vpos >= 0 && vpos < S;
        *reinterpret_cast<u32x4*>(base + vofs(ch >> 3, ch & 7)) = in ? IO::to_bf16x8(v[u]) : u32x4{0u, 0u, 0u, 0u};
      }
    };
    auto store_q = [&](const Prepped& qo) {
      *reinterpret_cast<u32x4*>(qbuf + kofs(prow, m1)) = qo.a1;
      *reinterpret_cast<u32x4*>(qbuf + kofs(prow, m2)) = qo.a2;
      *reinterpret_cast<u32x4*>(qbuf + TE + kofs(prow, m1)) = qo.b1;
      *reinterpret_cast<u32x4*>(qbuf + TE + kofs(prow, m2)) = qo.b2;
    };

    // Ring fill for step j0: tiles j0 - C .. j0 + C, and the queries of j0.
    Prepped ko, qo;
#pragma unroll 1
    for (int i = 0; i < RING; ++i) {
      const Stage st = load_stage(j0 - 2 * C + i, true);  // key tile j0 - C + i (its query rows are not used)
      prep_task<IO>(st.k, prot, ka2, kp, 1.f, ko);
      store_k(j0 - C + i, ko);
      store_v(j0 - C + i, st.v);
      if (i == RING - 1) {
        const Stage sq = load_stage(j0, false);
        prep_task<IO>(sq.q, prot, qa2, qp, qscale, qo);
        store_q(qo);
      }
    }
    // Loads beyond the run's last step read clamped rows and are never stored.
    Stage A = load_stage(j0 + 1 < j1 ? j0 + 1 : j0, !VDMA);
    __syncthreads();

    // One step: prepare step jj + 1 from `cur`, load step jj + 2 into `nxt`, then store after the first barrier.
    auto step = [&](int jj, const Stage& cur, Stage& nxt) {
      const bool next = jj + 1 < j1;
      prep_task<IO>(cur.k, prot, ka2, kp, 1.f, ko);
      prep_task<IO>(cur.q, prot, qa2, qp, qscale, qo);
      // The prepared values are only consumed by the stores after the barrier; pin their computation here, while
      // the attention waves are still busy, instead of letting the compiler sink it past the barrier.
      asm volatile("" ::"v"(ko.a1), "v"(ko.a2), "v"(ko.b1), "v"(ko.b2), "v"(qo.a1), "v"(qo.a2), "v"(qo.b1),
                   "v"(qo.b2));
      nxt = load_stage(jj + 2 < j1 ? jj + 2 : jj, !VDMA);
      __syncthreads();  // the attention waves are done with the oldest tile and the query buffer
      if (next) {
        store_k(jj + 1 + C, ko);
        if constexpr (!VDMA) store_v(jj + 1 + C, cur.v);
        store_q(qo);
      }
      __syncthreads();
    };
#pragma unroll 1
    for (int j = j0; j < j1; j += 2) {
      Stage B;
      step(j, A, B);
      if (j + 1 >= j1) break;
      step(j + 1, B, A);
    }
    f += j1 - j0;
  }
}

// Attention waves (0-3), wave = (query half, branch).
template <class IO, int C, bool FAST>
__device__ __forceinline__ void attn_waves(const Args& a, uint16_t* kring, uint16_t* vring, uint16_t* qbuf,
                                           float* xbuf, float c) {
  constexpr int RING = 2 * C + 1;
  constexpr bool VDMA = kVdma<IO, C>;
  constexpr int VR = kVring<IO, C>;
  const int lane = threadIdx.x & 63, wave = wave_id(), lr = lane & 31, lh = lane >> 5;
  const int S = a.S, H = a.H, w = a.w;
  const int64_t HD = static_cast<int64_t>(H) * D;
  const int qhalf = wave & 1, br = (wave >> 1) & 1;
  // Per-lane LDS fragment offsets.
  const int kswz = (lr & 7) ^ ((lr >> 3) & 1);
  int koff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) koff[kk] = lr * D + 8 * ((2 * kk + lh) ^ kswz);
  const int grp = lane >> 4, mm = lane & 15;
  // Accumulator o[0] holds the d-tile this wave writes out (dims 32 br .. 32 br + 31), o[1] the one it hands to
  // the other branch's wave: the branch-2 waves read the V d-tiles in swapped order.
  int voff[2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    const int col = 32 * (dt ^ br) + 16 * (grp & 1) + 4 * (mm & 3);
    voff[dt] = (4 * (grp >> 1) + (mm >> 2)) * D + 8 * ((col >> 3) ^ ((mm >> 2) << 1)) + (col & 7);
  }
  const Range rg(a);

  for (int64_t f = rg.beg; f < rg.end;) {
    const int bh = static_cast<int>(f / a.NS);
    const int j0 = static_cast<int>(f % a.NS);
    const int j1 = static_cast<int>(rg.end - f < a.NS - j0 ? j0 + (rg.end - f) : a.NS);
    const int b = bh / H, h = bh % H;
    const float lamh = a.lam ? a.lam[h] : 1.f;
    const uint16_t* xb = a.qkv + static_cast<int64_t>(b) * S * a.rs + h * D;
    __syncthreads();  // ring fill

    // V rows of key tile kt copied from qkv straight into their ring slot (the slot of tile kt - RING - 1, which
    // no wave reads after the previous step); each attention wave copies two 1 KB blocks of 8 rows, lane i the
    // 16-byte chunk that the swizzled layout puts at byte 16 i of its block. Rows at or past S are zeroed
    // instead (their probabilities are 0, and 0 * V must stay 0). The copy has the whole step to land; the wave
    // waits for it before the step's first barrier.
    auto v_dma = [&](int kt) {
      const uint16_t* tb = xb + static_cast<int64_t>(KT * kt) * a.rs;
      uint16_t* vt = vring + ring_slot(kt, VR) * TE;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int blk = 2 * wave + u, r = 8 * blk + (lane >> 3), ch = (lane & 7) ^ ((r & 3) << 1);
        if (KT * kt + r < S)
          lds_dma16(tb, static_cast<uint32_t>((r * a.rs + 2 * HD + 8 * ch) * 2), lds_addr(vt + blk * 512));
        else
          *reinterpret_cast<u32x4*>(vt + blk * 512 + 8 * lane) = u32x4{0u, 0u, 0u, 0u};
      }
    };

    // One step of 64 queries: `mode` is General (any step) or the Interior pattern of an interior step.
    auto do_step = [&](int j, auto mode) {
      using Mode = decltype(mode);
      if constexpr (VDMA) {
        if (j + 1 < j1) v_dma(j + 1 + C);
      }
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
      // The wave's tiles form one contiguous range of the ring; the scores of tile i + 1 are issued on the
      // matrix core before the softmax of tile i, so the two overlap.
      const int ilo = (ulo >> 6) - (j - C), ihi = (uhi >> 6) - (j - C);
      // The wave's tiles span at most RING consecutive slots, starting at the slot of tile ilo (kt0 >= 0).
      const int kt0 = j - C + ilo, slot0 = kt0 % RING, vslot0 = kt0 % VR;
      auto tile_ptr = [&](int i) {
        const int sl = slot0 + (i - ilo);
        return kring + (sl >= RING ? sl - RING : sl) * KTILE;
      };
      auto vtile_ptr = [&](int i) {
        const int sl = vslot0 + (i - ilo);
        return vring + (sl >= VR ? sl - VR : sl) * TE;
      };
      // 32-key half rt of tile i takes part: it meets the band of at least one query of the wave.
      auto active = [&](int i, int rt) {
        const int k0 = KT * (j - C + i) + 32 * rt;
        return k0 + 31 >= ulo && k0 <= uhi;
      };
      auto scores = [&](int i, const u32x4 (&kf)[2][4], f32x16 (&sc)[2]) {
        qk(kf, qf, sc, active(i, 0), active(i, 1));
      };
      auto frags = [&](int i, u32x4 (&kf)[2][4], bool act0 = true, bool act1 = true) {
        kload(tile_ptr(i) + br * TE, koff, kf, act0, act1);
      };
      auto finish = [&](int i, const f32x16 (&sc)[2]) {
        const int kt0 = KT * (j - C + i);
        bool act[2], full[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const int k0 = kt0 + 32 * rt, k1 = k0 + 31;
          act[rt] = active(i, rt);
          full[rt] = k0 >= qa + 31 - w && k1 <= qa + w && k0 >= 0 && k1 <= S - 1;
        }
        soft_pv<FAST>(sc, vtile_ptr(i), voff, o, lsum, m, c, act[0], act[1], full[0] ? 0 : 3,
                      full[1] ? 0 : 3, qlo - kt0 - 4 * lh, static_cast<unsigned>(qhi - qlo));
      };
      // Interior steps (every key of the wave's halves inside [0, S), so the band is |k - q| <= w unclipped):
      // ring half h = 2 i + rt sits t = h - (QH + 2C) halves from the wave's own queries; it takes part iff
      // |t| <= T, and it is cut by the lower band edge (t < 0), the upper one (t > 0) or both (t = 0) iff
      // |t| >= M. That pattern is known at compile time, so the tile loop over tiles IL .. IH is unrolled with no
      // per-tile scalar work, each half's softmax is the masked or unmasked code only, and the fragments of
      // halves that take no part are not read.
      auto run_interior = [&](auto pattern) {
        using P = decltype(pattern);
        constexpr int QH = P::qh, T = P::t, M = P::m, H0 = QH + 2 * C;
        constexpr int IL = (H0 - T) / 2, IH = (H0 + T) / 2;
        static_assert(T >= 0 && M >= 0 && M <= T + 1 && IH < RING, "interior pattern");
        auto act = [](int hh) { return hh - H0 >= -T && hh - H0 <= T; };
        auto msk = [](int hh) { return (hh - H0 <= -M ? 1 : 0) | (hh - H0 >= M ? 2 : 0); };
        auto fin = [&](int i, const f32x16 (&sc)[2]) {
          const int kt0 = KT * (j - C + i);
          soft_pv<FAST>(sc, vtile_ptr(i), voff, o, lsum, m, c, act(2 * i), act(2 * i + 1), msk(2 * i),
                        msk(2 * i + 1), qlo - kt0 - 4 * lh, static_cast<unsigned>(qhi - qlo));
          // Each tile's code is scheduled on its own, as in the general loop (measured 2% faster than one
          // schedule over the whole unrolled step).
          __builtin_amdgcn_sched_barrier(0);
        };
        u32x4 ka[2][4], kb[2][4];
        f32x16 sa[2], sb[2];
        auto fr = [&](int i, u32x4 (&kf)[2][4]) { frags(i, kf, act(2 * i), act(2 * i + 1)); };
        fr(IL, ka);
        if (IL + 1 <= IH) fr(IL + 1, kb);
        qk(ka, qf, sa, act(2 * IL), act(2 * IL + 1));
#pragma unroll
        for (int i = IL; i <= IH; i += 2) {
          if (i + 2 <= IH) fr(i + 2, ka);
          if (i + 1 <= IH) qk(kb, qf, sb, act(2 * i + 2), act(2 * i + 3));
          fin(i, sa);
          if (i + 1 > IH) break;
          if (i + 3 <= IH) fr(i + 3, kb);
          if (i + 2 <= IH) qk(ka, qf, sa, act(2 * i + 4), act(2 * i + 5));
          fin(i + 1, sb);
        }
      };
      if constexpr (!std::is_same<Mode, General>::value) {
        run_interior(mode);
      } else {
        // The K fragments are read one tile ahead of their MFMAs. The loop is unrolled over the two score and
        // fragment buffers so that all of them stay in fixed registers.
        f32x16 sa[2], sb[2];
        u32x4 ka[2][4], kb[2][4];
        frags(ilo, ka);
        if (ilo + 1 <= ihi) frags(ilo + 1, kb);
        scores(ilo, ka, sa);
#pragma unroll 1
        for (int i = ilo;;) {
          if (i + 2 <= ihi) frags(i + 2, ka);
          if (i + 1 <= ihi) scores(i + 1, kb, sb);
          finish(i, sa);
          if (++i > ihi) break;
          if (i + 2 <= ihi) frags(i + 2, kb);
          if (i + 1 <= ihi) scores(i + 1, ka, sa);
          finish(i, sb);
          if (++i > ihi) break;
        }
      }

      // out = O1 / l1 - lam * O2 / l2, each product rounded on its own. The two branch waves of a query half
      // split the work by output dims: branch 1 writes dims 0-31 (d-tile 0), branch 2 dims 32-63 (d-tile 1); each
      // first publishes the product the other one needs (branch 1: O1 / l1 of d-tile 1; branch 2: lam * O2 / l2
      // of d-tile 0).
      // At C <= 1 the exchange and the epilogue, the same work at every window, are a fifth of the step; the wave
      // issues them ahead of the prep waves (measured 4 % faster at w = 17, no change at w = 64 or at C = 2).
      if constexpr (C <= 1) __builtin_amdgcn_s_setprio(2);
      const float inv = __frcp_rn(lsum + __shfl_xor(lsum, 32, kWave));
      const float li = br == 1 ? __fmul_rn(lamh, inv) : inv;  // this branch's factor
      f32x4* xs = reinterpret_cast<f32x4*>(xbuf) + qhalf * (2 * 4 * 64);  // [d-tile][register / 4][lane][4]
      const int give = 1 - br;                                           // the d-tile the other wave stores
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 v;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) v[jj] = __fmul_rn(o[1][4 * g + jj], li);
        xs[(give * 4 + g) * 64 + lane] = v;
      }
      // This step's V copy (and the previous step's output stores) are complete before the barrier.
      if constexpr (VDMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      {
        const int dt = br;  // the d-tile this wave stores
        uint16_t* orow = a.out + (static_cast<int64_t>(b) * S + q) * HD + h * D + 32 * dt;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 other = xs[(dt * 4 + g) * 64 + lane];
          float v[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const float mine = __fmul_rn(o[0][4 * g + jj], li);
            v[jj] = br == 0 ? __fsub_rn(mine, other[jj]) : __fsub_rn(other[jj], mine);
          }
          if (q < S) {
            u32x2 pk;
            pk[0] = IO::pack2(v[0], v[1]);
            pk[1] = IO::pack2(v[2], v[3]);
            *reinterpret_cast<u32x2*>(orow + 8 * g + 4 * lh) = pk;
          }
        }
      }
      if constexpr (C <= 1) __builtin_amdgcn_s_setprio(0);
      __syncthreads();
    };
    // Interior steps [ja, jb): every query's band inside [0, S), i.e. 64 j - w >= 0 (j >= C, since
    // 64 C >= w) and 64 j + 63 + w <= S - 1. Each range is its own loop, so that the unrolled interior code
    // shares no control flow with the general path.
    int ja = j0, jb = j0;
    if (S - QT - w >= 0) {
      ja = j0 > C ? j0 : C;
      jb = (S - QT - w) / QT + 1;
      if (jb > j1) jb = j1;
      if (jb < ja) ja = jb = j0;
    }
#pragma unroll 1
    for (int j = j0; j < ja; ++j) do_step(j, General{});
    auto interior = [&](auto pattern) {
#pragma unroll 1
      for (int j = ja; j < jb; ++j) do_step(j, pattern);
    };
    // The pattern of w: T = 2C - 1 for w <= 64 C - 32, else 2C; M = T - 1 except for w in {64C - 33, 64C - 32}
    // (T = M = 2C - 1) and w >= 64 C - 1 (T = M = 2C). C = 0 means w = 0: the diagonal half only, both edges.
    auto by_pattern = [&](auto qh) {
      constexpr int QH = decltype(qh)::value;
      if constexpr (C == 0) {
        interior(Interior<QH, 0, 0>{});
      } else {
        const int tw = (w + 31) / 32, mw = (w + 1) / 32;
        if (tw == 2 * C)
          mw == 2 * C ? interior(Interior<QH, 2 * C, 2 * C>{}) : interior(Interior<QH, 2 * C, 2 * C - 1>{});
        else
          mw == 2 * C - 1 ? interior(Interior<QH, 2 * C - 1, 2 * C - 1>{})
                          : interior(Interior<QH, 2 * C - 1, 2 * C - 2>{});
      }
    };
    if (qhalf == 0)
      by_pattern(std::integral_constant<int, 0>{});
    else
      by_pattern(std::integral_constant<int, 1>{});
#pragma unroll 1
    for (int j = jb; j < j1; ++j) do_step(j, General{});
    f += j1 - j0;
  }
}

// IO: the element type of qkv and out (bf16 or half); the operands are bf16 either way.
template <class IO, int C>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void band_ring(Args a) {
  constexpr int RING = 2 * C + 1;
  // K and K_diff of RING tiles; V of RING tiles, plus the spare slot that takes the next tile's copy.
  __shared__ __attribute__((aligned(16))) uint16_t kring[RING * KTILE];
  __shared__ __attribute__((aligned(16))) uint16_t vring[kVring<IO, C> * TE];
  __shared__ __attribute__((aligned(16))) uint16_t qbuf[2 * TE];  // q, q_diff of the step (64 rows each)
  __shared__ __attribute__((aligned(16))) float xbuf[XF];
  const SoftmaxPlan plan = softmax_plan(dyt_row_bound<D>(a.q_dyt), dyt_row_bound<D>(a.k_dyt), D);
  const float qa2 = 2.f * kLog2e * a.q_dyt[0], ka2 = 2.f * kLog2e * a.k_dyt[0];
  if (wave_id() >= 4) {
    // The prep waves issue first when both roles of a SIMD are ready: measured 6% faster than equal priority.
    __builtin_amdgcn_s_setprio(1);
    if (a.half == D / 2)
      prep_waves<IO, C, true>(a, kring, vring, qbuf, qa2, ka2, plan.qscale);
    else
      prep_waves<IO, C, false>(a, kring, vring, qbuf, qa2, ka2, plan.qscale);
  }
  else if (plan.fast)
    attn_waves<IO, C, true>(a, kring, vring, qbuf, xbuf, plan.c);
  else
    attn_waves<IO, C, false>(a, kring, vring, qbuf, xbuf, plan.c);
}

}  // namespace band_ring

bool band_ring_supported(int dtype, int D, int half, int window) {
  return (dtype == HB_BF16 || dtype == HB_F16) && D == band_ring::D && half % 8 == 0 && window <= 128;
}

int launch_band_ring(hipStream_t stream, int dtype, const void* qkv, int64_t rs, const float* q_dyt, const float* k_dyt,
                     const float* cosT, const float* sinT, int half, int window, const float* lam, void* out, int B,
                     int S, int H) {
  using namespace band_ring;
  const int ncu = device_cus();
  Args a;
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.rs = rs;
  a.S = S;
  a.H = H;
  a.w = window;
  a.half = half;
  a.NS = (S + QT - 1) / QT;
  a.total = static_cast<int64_t>(B) * H * a.NS;
  // A ring fill costs about one step. Where the (batch, head) boundaries do not fall between workgroups
  // (the CU count is not a multiple of B * H), the workgroups whose range holds a boundary fill twice; weighting
  // the split by the fills balances them (reference decoder geometry: 121.5 -> 120.0 us; S = 50000 with six
  // heads and w = 40: 78.7 -> 70.5 us). Short ranges keep the even split, where a step more would cost more.
  a.fillw = (ncu % (B * H) != 0 && a.total >= 16 * static_cast<int64_t>(ncu)) ? 1 : 0;
  a.q_dyt = q_dyt;
  a.k_dyt = k_dyt;
  a.cosT = cosT;
  a.sinT = sinT;
  a.lam = lam;
  a.out = static_cast<uint16_t*>(out);
  const int64_t grid = a.total < ncu ? a.total : ncu;
  const int C = (window + 63) / 64;
  const bool f16 = dtype == HB_F16;
  auto kernel = C == 0 ? (f16 ? hb::band_ring::band_ring<F16Io, 0> : hb::band_ring::band_ring<Bf16Io, 0>)
                : C == 1 ? (f16 ? hb::band_ring::band_ring<F16Io, 1> : hb::band_ring::band_ring<Bf16Io, 1>)
                         : (f16 ? hb::band_ring::band_ring<F16Io, 2> : hb::band_ring::band_ring<Bf16Io, 2>);
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(NT), 0, stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HB_ERR_LAUNCH, "band_ring launch failed: %s", hipGetErrorString(e));
  return HB_OK;
}

}  // namespace hb
