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

// The dense workspace holds five equally sized (B, H, Lp, D) regions of prepared (normalised, rotated or
// masked) rows, Lp = L rounded up to kDenseQueryBlock and zero-filled past L. Elements are bf16
// for HB_BF16 and fp32 for HB_F32. Region order: q', k', q_diff', k_diff', v'.
struct DenseLayout {
  int64_t Lp;
  int64_t region_elems;  // B * H * Lp * D
  size_t elem_bytes;
  size_t region_bytes;
  size_t total_bytes;
};
DenseLayout dense_layout(int dtype, int B, int L, int H, int D);

int check_common(int dtype, int64_t row_stride, int B, int N, int H, int D, int half);

}  // namespace hb
