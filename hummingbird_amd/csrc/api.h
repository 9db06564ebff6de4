// Host-side helpers shared by the launchers: status reporting, validation and the dense workspace layout.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/hummingbird_amd.h"

namespace hb {

// Records `msg` (printf-style) as this thread's last error and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Queries per dense attention workgroup; the prepared sequence is padded to a multiple of this.
constexpr int kDenseQueryBlock = 128;
// Keys per LDS tile in the dense attention loop.
constexpr int kDenseKeyTile = 64;

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// The dense workspace holds three equally sized (B, H, Lp, D) regions of prepared key-side rows, Lp = L rounded
// up to kDenseQueryBlock and zero-filled past L: k' and k_diff' (normalised and rotated) and v' (V * mask).
// Elements are bf16 for HB_BF16 and fp32 for HB_F32. The queries are prepared inside the attention kernel.
struct DenseLayout {
  int64_t Lp;
  int64_t region_elems;  // B * H * Lp * D
  size_t elem_bytes;
  size_t region_bytes;
  size_t total_bytes;
};
DenseLayout dense_layout(int dtype, int B, int L, int H, int D);

int check_common(int dtype, int64_t row_stride, int B, int N, int H, int D, int half);

// Whether two row-strided regions share a byte: N rows of ca (cb) elements of `esize` bytes, starting at a (b),
// rows `as` (`bs`) elements apart (strides >= the row widths). With equal strides the test is exact, so column
// slices of one wider buffer that interleave without sharing elements do not overlap; with different strides it is
// the conservative test of the two byte extents. NULL never overlaps.
bool regions_overlap(const void* a, int64_t as, int64_t ca, const void* b, int64_t bs, int64_t cb, int64_t N,
                     int esize);
// Fails with HB_ERR_STRIDE unless N >= 1 rows of C elements, `stride` elements apart, span fewer than 2^48
// elements (computed without overflow), so that every extent and offset the validators and launchers compute for
// the buffer fits in int64. Every entry point checks each strided buffer with it before using rows_bytes.
int check_extent(const char* what, const char* name, int64_t N, int64_t stride, int64_t C);
// Bytes spanned by N rows of C elements of `esize` bytes, rows `stride` elements apart (after check_extent).
inline int64_t rows_bytes(int64_t N, int64_t stride, int64_t C, int esize) { return ((N - 1) * stride + C) * esize; }
// Fails with HB_ERR_STRIDE if the byte ranges [a, a + a_bytes) and [b, b + b_bytes) intersect (NULL never does):
// an output or workspace of the attention and projection entry points against the buffers the same call reads.
int check_disjoint(const char* what, const char* a_name, const void* a, int64_t a_bytes, const char* b_name,
                   const void* b, int64_t b_bytes);
// The aliasing rule of the row-wise entry points for an output `out` (N x out_cols) against an input `in`
// (N x in_cols): when `in_place_ok` the output may be the input itself (same pointer, row stride and width: every
// element is read before it is written, by the thread that writes it); otherwise, and for any other placement, the
// two must share no element.
int check_no_overlap(const char* what, const char* out_name, const void* out, int64_t out_stride, int64_t out_cols,
                     const char* in_name, const void* in, int64_t in_stride, int64_t in_cols, int64_t N, int esize,
                     bool in_place_ok);
// Multiprocessor (CU) count of the current device, queried once per device (256 if the query fails).
int device_cus();

// Dense kernels (dense.hip: bf16 and half, fp32.hip: fp32). Arguments are validated by the exported entry points before
// these are called. The prep reads k, k_diff and v from sections sk, skd and sv of the rows of `kv` (units of
// H * D elements) for Lk keys into the workspace described by `lay` (laid out for Lk keys); the attention reads
// q and q_diff from sections 0 and sqd of the rows of `q` for L queries and attends over the Lk prepared keys.
// 16-bit inputs (dtype HB_BF16 or HB_F16: bf16 or half qkv and out; the operands are bf16 in both).
int launch_dense_prep_16bit(hipStream_t stream, int dtype, const void* kv, int64_t rs, int sk, int skd, int sv,
                            const float* kw, const float* cos, const float* sin, int half, const float* vmask, int B,
                            int Lk, int H, int D, float eps, const DenseLayout& lay, void* workspace);
int launch_dense_attend_16bit(hipStream_t stream, int dtype, const void* q, int64_t rs, int sqd, const float* qw,
                              const float* kw, const float* cos, const float* sin, int half, float eps,
                              const float* lam, void* out, int B, int L, int Lk, int H, int D, const DenseLayout& lay,
                              const void* workspace);
int launch_dense_prep_f32(hipStream_t stream, const void* qkv, int64_t rs, int sk, int skd, int sv, const float* kw,
                          const float* cosT, const float* sinT, int half, const float* vmask, int B, int L, int H, int D,
                          float eps, const DenseLayout& lay, void* ws);
int launch_dense_attend_f32(hipStream_t stream, const void* qkv, int64_t rs, int sqd, const float* qw,
                            const float* cosT, const float* sinT, int half, float eps, const void* ws, const float* lam,
                            void* out, int B, int L, int Lk, int H, int D, const DenseLayout& lay);
// Streaming band kernel (band_ring.hip): bf16 or half, D = 64, half % 8 == 0, window <= 128. Arguments are
// validated by hb_band_diffattn before the launch.
bool band_ring_supported(int dtype, int D, int half, int window);
int launch_band_ring(hipStream_t stream, int dtype, const void* qkv, int64_t rs, const float* q_dyt, const float* k_dyt,
                     const float* cosT, const float* sinT, int half, int window, const float* lam, void* out, int B,
                     int S, int H);
// Tiled band kernels (band_tiled.hip): bf16 or half, any head_dim and half-width; the workspace holds the prepared
// keys in the dense layout (three (B, H, round_up(S, 128), D) bf16 regions: k', k_diff', v'^T).
DenseLayout band_tiled_layout(int B, int S, int H, int D);
int launch_band_tiled(hipStream_t stream, int dtype, const void* qkv, int64_t rs, const float* q_dyt, const float* k_dyt,
                      const float* cosT, const float* sinT, int half, int window, const float* lam, void* out, int B,
                      int S, int H, int D, void* workspace);
// fp32 band with its keys prepared once into a workspace of dense_layout(HB_F32, B, S, H, D).total_bytes.
int launch_band_f32_ws(hipStream_t stream, const void* qkv, int64_t rs, const float* qdyt, const float* kdyt,
                       const float* cosT, const float* sinT, int half, int window, const float* lam, void* out, int B,
                       int S, int H, int D, void* workspace);
int launch_band_f32(hipStream_t stream, const void* qkv, int64_t rs, const float* qdyt, const float* kdyt,
                    const float* cosT, const float* sinT, int half, int window, const float* lam, void* out, int B,
                    int S, int H, int D);

}  // namespace hb
