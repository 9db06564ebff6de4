// DiT differential cross-attention: the C ABI (host code; the kernels are the dense ones, dense.hip and fp32.hip).
//
// Replaces the XLA chain of dit._cross_attention (sa3jax/dit.py:203-215): q and q_diff come from the block's
// to_q output [q | q_diff] (dit.py:207-209) and are RMS-normed with q_norm (dit.py:166-168); k, k_diff and v come
// from the context's to_kv output [k | k_diff | v], k and k_diff RMS-normed with k_norm, hoisted out of the
// sampler loop (dit._cross_kv, dit.py:274-284). No RoPE and no mask (dit.py:204-205, 214-215). The two softmax
// attentions share v and are subtracted (dit.py:131-147).
//
// hb_cross_prep prepares k, k_diff and v of the context once into a workspace in the dense kernels' layout;
// hb_cross_attend then runs the dense attention kernel with the queries of one block against it, as often as
// the sampler needs (the reference computes the context's K/V once per clip).
#include "api.h"

#include <math.h>

using namespace hb;

namespace {

// Sections (units of H * D elements): a to_q row is [q | q_diff], a to_kv row [k | k_diff | v] (dit.py:208, 279).
constexpr int kQdSec = 1;
constexpr int kKSec = 0, kKdSec = 1, kVSec = 2;

// `rows` rows of `min_elems` elements, `row_stride` apart.
int check_stride(const char* what, int64_t row_stride, int64_t min_elems, int64_t rows) {
  if (row_stride < min_elems || row_stride % 8 != 0)
    return fail(HB_ERR_STRIDE, "%s row_stride %lld must be >= %lld and a multiple of 8", what,
                static_cast<long long>(row_stride), static_cast<long long>(min_elems));
  return check_extent("cross_attention", what, rows, row_stride, min_elems);
}

int check_shape(int dtype, int B, int L, int Nk, int H, int D, float eps) {
  if (dtype != HB_BF16 && dtype != HB_F32 && dtype != HB_F16)
    return fail(HB_ERR_DTYPE, "dtype %d is not HB_BF16 (0), HB_F32 (1) or HB_F16 (2)", dtype);
  if (D != 64 && D != 128) return fail(HB_ERR_HEAD_DIM, "head_dim %d is not 64 or 128", D);
  if (B < 1 || L < 1 || Nk < 1 || H < 1)
    return fail(HB_ERR_SHAPE, "need B, L, Nk, H >= 1 (B=%d, L=%d, Nk=%d, H=%d)", B, L, Nk, H);
  if (B > 65535 || H > 65535 || L > (1 << 28) || Nk > (1 << 28))
    return fail(HB_ERR_SHAPE, "shape out of range (B=%d, H=%d <= 65535; L=%d, Nk=%d <= 2^28)", B, H, L, Nk);
  if (static_cast<int64_t>(B) * (L > Nk ? L : Nk) * H * D > (int64_t(1) << 40))
    return fail(HB_ERR_SHAPE, "B*max(L,Nk)*H*D exceeds 2^40 elements");
  if (!(eps >= 0.0f) || !isfinite(eps)) return fail(HB_ERR_EPS, "eps %g must be finite and >= 0", eps);
  return HB_OK;
}

int check_workspace(const void* ws, size_t bytes, size_t need) {
  if (!ws) return fail(HB_ERR_NULL, "workspace must be non-NULL");
  if (reinterpret_cast<uintptr_t>(ws) % 256) return fail(HB_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (bytes < need) return fail(HB_ERR_WORKSPACE, "workspace holds %zu bytes, needs %zu", bytes, need);
  return HB_OK;
}

}  // namespace

extern "C" {

size_t hb_cross_workspace_size(int dtype, int B, int Nk, int H, int D) {
  if ((dtype != HB_BF16 && dtype != HB_F32 && dtype != HB_F16) || B < 1 || Nk < 1 || H < 1 || (D != 64 && D != 128)) return 0;
  return dense_layout(dtype, B, Nk, H, D).total_bytes;
}

int hb_cross_validate(int dtype, int64_t q_row_stride, int64_t kv_row_stride, int B, int L, int Nk, int H, int D,
                      float eps) {
  clear_error();
  int st = check_shape(dtype, B, L, Nk, H, D, eps);
  if (st) return st;
  st = check_stride("q", q_row_stride, static_cast<int64_t>(2) * H * D, static_cast<int64_t>(B) * L);
  if (st) return st;
  return check_stride("kv", kv_row_stride, static_cast<int64_t>(3) * H * D, static_cast<int64_t>(B) * Nk);
}

int hb_cross_prep(hipStream_t stream, const void* kv, int dtype, int64_t row_stride, const float* k_weight, int B,
                  int Nk, int H, int D, float eps, void* workspace, size_t workspace_bytes) {
  clear_error();
  int st = check_shape(dtype, B, 1, Nk, H, D, eps);
  if (st) return st;
  st = check_stride("kv", row_stride, static_cast<int64_t>(3) * H * D, static_cast<int64_t>(B) * Nk);
  if (st) return st;
  if (!kv || !k_weight) return fail(HB_ERR_NULL, "kv and k_weight must be non-NULL");
  if (reinterpret_cast<uintptr_t>(kv) % 16) return fail(HB_ERR_STRIDE, "kv must be 16-byte aligned");
  const DenseLayout lay = dense_layout(dtype, B, Nk, H, D);
  st = check_workspace(workspace, workspace_bytes, lay.total_bytes);
  if (st) return st;
  const int es = dtype == HB_F32 ? 4 : 2;
  if ((st = check_disjoint("cross_prep", "workspace", workspace, static_cast<int64_t>(lay.total_bytes), "kv", kv,
                           rows_bytes(static_cast<int64_t>(B) * Nk, row_stride, static_cast<int64_t>(3) * H * D, es))))
    return st;
  if (dtype == HB_F32)
    return launch_dense_prep_f32(stream, kv, row_stride, kKSec, kKdSec, kVSec, k_weight, nullptr, nullptr, 0, nullptr,
                                 B, Nk, H, D, eps, lay, workspace);
  return launch_dense_prep_16bit(stream, dtype, kv, row_stride, kKSec, kKdSec, kVSec, k_weight, nullptr, nullptr, 0,
                                 nullptr, B, Nk, H, D, eps, lay, workspace);
}

int hb_cross_attend(hipStream_t stream, const void* q, int dtype, int64_t row_stride, const float* q_weight,
                    const float* k_weight, const float* lam, void* out, int B, int L, int Nk, int H, int D, float eps,
                    const void* workspace, size_t workspace_bytes) {
  clear_error();
  int st = check_shape(dtype, B, L, Nk, H, D, eps);
  if (st) return st;
  st = check_stride("q", row_stride, static_cast<int64_t>(2) * H * D, static_cast<int64_t>(B) * L);
  if (st) return st;
  if (!q || !q_weight || !k_weight || !out) return fail(HB_ERR_NULL, "q, q_weight, k_weight and out must be non-NULL");
  if (reinterpret_cast<uintptr_t>(q) % 16) return fail(HB_ERR_STRIDE, "q must be 16-byte aligned");
  const DenseLayout lay = dense_layout(dtype, B, Nk, H, D);
  st = check_workspace(workspace, workspace_bytes, lay.total_bytes);
  if (st) return st;
  {
    const int es = dtype == HB_F32 ? 4 : 2;
    const int64_t HD = static_cast<int64_t>(H) * D, rows = static_cast<int64_t>(B) * L, ob = rows * HD * es;
    if ((st = check_disjoint("cross_attend", "out", out, ob, "q", q, rows_bytes(rows, row_stride, 2 * HD, es))) ||
        (st = check_disjoint("cross_attend", "out", out, ob, "workspace", workspace,
                             static_cast<int64_t>(lay.total_bytes))))
      return st;
  }
  if (dtype == HB_F32) {
    if (reinterpret_cast<uintptr_t>(out) % 16) return fail(HB_ERR_STRIDE, "fp32 out must be 16-byte aligned");
    return launch_dense_attend_f32(stream, q, row_stride, kQdSec, q_weight, nullptr, nullptr, 0, eps, workspace, lam,
                                   out, B, L, Nk, H, D, lay);
  }
  if (reinterpret_cast<uintptr_t>(out) % 8) return fail(HB_ERR_STRIDE, "out must be 8-byte aligned");
  return launch_dense_attend_16bit(stream, dtype, q, row_stride, kQdSec, q_weight, k_weight, nullptr, nullptr, 0, eps, lam,
                                   out, B, L, Nk, H, D, lay, workspace);
}

}  // extern "C"
