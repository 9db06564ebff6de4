// Key tiles of the flash-style attention kernels (dense, and band with a wide window): the prepared-tile
// layout in the workspace and in LDS, the global -> LDS copier, and the differential epilogue of a 4-wave
// workgroup. Shared by dense.hip and band_tiled.hip.
#pragma once

#include "attn_tile.h"
#include "common.h"

namespace hb {

// Layout of a prepared 64-key V tile: transposed, V^T[d][pos], with the keys of every 16-key group in the order
// that the probability registers of a lane hold them. Lane half lh of the PV MFMA takes the keys
// {16 g + 8 (j / 4) + 4 lh + j % 4 : j < 8}; storing key 16 g + 8 a + 4 b + c at position 16 g + 8 b + 4 a + c
// (bits 2 and 3 swapped, an involution) puts them at the eight consecutive positions 16 g + 8 lh .. +8.
__device__ __forceinline__ int v_tile_key(int pos) { return (pos & ~12) | ((pos & 4) << 1) | ((pos & 8) >> 1); }

// Asynchronous 16-byte copy global -> LDS for a whole wave: lane i's 16 bytes at `sbase` + `voff` bytes
// (`sbase` wave-uniform) land at byte 16 i of the 1 KB LDS block at byte address `lds` (wave-uniform). Issued as inline assembly
// so that the compiler does not serialise it against the LDS reads of the other stage; the caller waits for it
// (s_waitcnt vmcnt(0)) before the barrier that publishes the stage. The assembly writes M0 (the LDS address of
// the copy); nothing else in these kernels reads M0, so the compiler's note that a reserved register in a
// clobber list may not be preserved has no consumer here.
__device__ __forceinline__ void lds_dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(sbase) : "m0");
}

// Byte address of an LDS location (the operand M0 and the LDS instructions take).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

// XOR swizzle of the 16-byte chunks of an LDS row of RL elements, so that the MFMA operand reads (one chunk of
// 16 consecutive rows per cycle) hit distinct banks.
template <int RL>
__device__ __forceinline__ int swz(int row, int chunk) {
  if constexpr (RL == 64) return row * 64 + 8 * (chunk ^ (row & 7) ^ ((row >> 3) & 1));
  else return row * RL + 8 * (chunk ^ (row & 15));
}

// Attention tiling: a workgroup of NW waves attends QB queries.
//   - Split layouts (D = 64 with 4 waves; D = 128 with 8 waves): each wave owns one differential branch of
//     32 * NCT queries; the first NW / 2 waves run branch 1 (q, k), the others branch 2 (q_diff, k_diff), and each
//     branch-2 wave hands its normalised result to the branch-1 wave of the same queries through LDS at the end.
//     D = 64: QB = 128 (two MFMA column tiles per wave, so every K fragment read from LDS feeds two MFMAs while a
//     wave's registers still fit two waves per SIMD) or 64 for grids too small to fill the GPU. D = 128: QB = 128
//     over 8 waves, one column tile each, so two waves share each SIMD in the one workgroup per CU that the 96 KB
//     of K/V stages allow.
//   - D = 128 with 4 waves (the tiled band kernels): each wave owns both branches of 32 queries.
template <int D, int QB = 128, int NW = 4>
struct DenseTile {
  static_assert((NW == 4 && (QB == 128 || (D == 64 && QB == 64))) || (NW == 8 && D == 128 && QB == 128),
                "tilings: D = 64 with 4 waves (QB 128 or 64), D = 128 with 4 or 8 waves (QB 128)");
  static constexpr bool SPLIT = D == 64 || NW == 8;         // one branch per wave
  static constexpr int NB = SPLIT ? 1 : 2;                   // branches per wave
  static constexpr int NCT = SPLIT ? QB / (16 * NW) : 1;     // 32-query column tiles per wave
  static constexpr int NT = 64 * NW;                         // threads per workgroup
  static constexpr int K_ELEMS = 64 * D;     // one tensor of a 64-key tile: K, K_diff [key][d]; V^T [d][pos]
  static constexpr int STAGE = 3 * K_ELEMS;  // K, K_diff, V^T of one 64-key tile, swizzled rows
  static constexpr int BPT = 64 * D * 2 / 1024;  // 1 KB blocks per tensor of a 64-key tile
  static constexpr int NBLK = 3 * BPT;            // blocks per tile (a multiple of the waves)
  // the split epilogue's hand-over (fp32 accumulators of every branch-2 wave), and the LDS a workgroup declares
  static constexpr int XBUF_BYTES = SPLIT ? (NW / 2) * NCT * (D / 32) * 16 * 64 * 4 : 0;
  static constexpr int SMEM_ELEMS = 2 * STAGE > XBUF_BYTES / 2 ? 2 * STAGE : XBUF_BYTES / 2;
};

// Copies 64-key tile t of K, K_diff and V'^T from the workspace straight into an LDS stage (global_load_lds, no
// registers). Each wave copies 1 KB blocks: lane i lands at byte 16 i of its block, so it fetches the chunk that
// the swizzled layout puts there.
template <int D, int NW = 4>
struct TileCopy {
  const uint16_t* Kb;
  const uint16_t* Kdb;
  const uint16_t* Vb;
  int wv;
  uint32_t off64, off128;  // byte offset of this lane's chunk inside its wave's 1 KB block, per row length

  __device__ TileCopy(const uint16_t* k, const uint16_t* kd, const uint16_t* v) : Kb(k), Kdb(kd), Vb(v) {
    const int ln = threadIdx.x & 63;
    wv = wave_id();
    // The same for every block of a tensor, since the swizzle depends on the row only through bits the block
    // index does not change.
    const int r64 = ln >> 3;   // rows of 64 elements: 8 per block
    off64 = static_cast<uint32_t>(wv * 1024 + r64 * 128 + 16 * ((ln & 7) ^ (r64 & 7) ^ (wv & 1)));
    const int r128 = ln >> 4;  // rows of 128 elements: 4 per block
    off128 = static_cast<uint32_t>(wv * 1024 + r128 * 256 + 16 * ((ln & 15) ^ (4 * (wv & 3) + r128)));
  }

  // Tile t into the stage at LDS byte address `stage`.
  __device__ __forceinline__ void operator()(int t, uint32_t stage) const {
    using T = DenseTile<D>;
#pragma unroll
    for (int tsr = 0; tsr < 3; ++tsr) {  // K, K_diff [key][d]; V^T [d][pos]
      const uint16_t* base = (tsr == 0 ? Kb : tsr == 1 ? Kdb : Vb) + static_cast<int64_t>(t) * 64 * D;
      const uint32_t off = tsr < 2 && D == 128 ? off128 : off64;
#pragma unroll
      for (int u = 0; u < T::BPT / NW; ++u)  // blocks wv, wv + NW, ...
        lds_dma16(base, off + u * NW * 1024, stage + 2 * tsr * T::K_ELEMS + (wv + NW * u) * 1024);
    }
  }
};

// out[q, h*D + d] = O1 / l1 - lam * O2 / l2 for the QB queries of a 4-wave workgroup laid out as DenseTile<D, QB>
// describes (q0w: this wave's first query, br0: its first branch), written in the output type IO for q < N.
// D = 64: the branch-2 waves publish lam * O2 / l2 (rounded per element) through LDS (`xbuf_mem`, at least
// 32 KB, free of tile reads: the caller has passed a barrier after its last tile) and the branch-1 waves
// subtract it from O1 / l1; D = 128: each wave holds both branches. Every lane of the workgroup must call it.
template <int D, int QB = 128, class IO = Bf16Io, int NW = 4>
__device__ __forceinline__ void store_diff_split(
    uint16_t* __restrict__ out, int64_t b, int N, int H, int h, int q0w, int br0, float lamh,
    const f32x16 (&o)[DenseTile<D, QB, NW>::NB][DenseTile<D, QB, NW>::NCT][D / 32],
    const float (&lsum)[DenseTile<D, QB, NW>::NB][DenseTile<D, QB, NW>::NCT], uint16_t* xbuf_mem) {
  using T = DenseTile<D, QB, NW>;
  constexpr int NCT = T::NCT;
  const int lane = threadIdx.x & 63, wave = wave_id(), lr = lane & 31, lh = lane >> 5;
  const int64_t HD = static_cast<int64_t>(H) * D;
  if constexpr (T::SPLIT) {
    float* xbuf = reinterpret_cast<float*>(xbuf_mem);  // 2 query halves x NCT x D/32 x 16 registers x 64 lanes
    const int slot0 = (wave % (NW / 2)) * NCT * (D / 32) * 16;
    if (br0 == 1) {
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const float i1 = __fmul_rn(lamh, inv_rowsum(lsum, 0, ct));
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            xbuf[(slot0 + (ct * (D / 32) + dt) * 16 + r) * 64 + lane] = __fmul_rn(o[0][ct][dt][r], i1);
      }
    }
    __syncthreads();
    if (br0 == 0) {
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const float i0 = inv_rowsum(lsum, 0, ct);
        const int q = q0w + 32 * ct + lr;
        uint16_t* orow = out + (b * N + q) * HD + h * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int r = 4 * g + j;
              v[j] = __fsub_rn(__fmul_rn(o[0][ct][dt][r], i0), xbuf[(slot0 + (ct * (D / 32) + dt) * 16 + r) * 64 + lane]);
            }
            if (q < N) {
              u32x2 pk;
              pk[0] = IO::pack2(v[0], v[1]);
              pk[1] = IO::pack2(v[2], v[3]);
              *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * g + 4 * lh) = pk;
            }
          }
      }
    }
  } else {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const int q = q0w + 32 * ct + lr;
      uint16_t* orow = q < N ? out + (b * N + q) * HD + h * D : nullptr;
      store_diff_bf16<D, NCT, IO>(orow, o, lsum, ct, lamh);
    }
  }
}

}  // namespace hb
