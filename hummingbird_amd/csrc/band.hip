// SAME-L band differential attention: the C ABI entry points and the choice between the two bf16 kernels.
//
// Replaces the reference's fused TPU kernel sa3jax/band_attention.py:123-180 (and the XLA chain
// sa3jax/same_l.py:151-169):
//   - bf16 or half, head_dim 64, half-width w <= 128: the streaming ring kernel (band_ring.hip), which keeps the
//     whole key window of a 64-query step in LDS and prepares every key once per run; no workspace;
//   - bf16 or half, w > 128 or head_dim 128: the tiled kernels (band_tiled.hip), which prepare the keys into a
//     caller-supplied workspace and stream each 128-query block's window through LDS;
//   - fp32: the fp32 kernels (fp32.hip): with a workspace every key is prepared once and the attention streams the
//     prepared tiles; without one (NULL, as before) each query block prepares its own window.
#include "api.h"

using namespace hb;

static bool band_needs_workspace(int dtype, int D, int half, int window) {
  return dtype != HB_F32 && !band_ring_supported(dtype, D, half, window);
}

// fp32: the workspace of the prepared keys, which the call uses when it is given one (it is optional there).
extern "C" size_t hb_band_workspace_size(int dtype, int B, int S, int H, int D, int half, int window) {
  if ((dtype != HB_BF16 && dtype != HB_F32 && dtype != HB_F16) || B < 1 || S < 1 || H < 1 || (D != 64 && D != 128))
    return 0;
  if (dtype == HB_F32) return dense_layout(HB_F32, B, S, H, D).total_bytes;
  if (!band_needs_workspace(dtype, D, half, window > S ? S : window)) return 0;
  return band_tiled_layout(B, S, H, D).total_bytes;
}

extern "C" int hb_band_diffattn(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride,
                                const float* q_dyt, const float* k_dyt, const float* cos, const float* sin, int half,
                                int window, const float* lam, void* out, int B, int S, int H, int D, void* workspace,
                                size_t workspace_bytes) {
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
  // Outputs against the buffers the call reads, checked after the workspace is known to be valid.
  auto overlaps = [&]() {
    const int es = dtype == HB_F32 ? 4 : 2;
    const int64_t HD = static_cast<int64_t>(H) * D, rows = static_cast<int64_t>(B) * S, ob = rows * HD * es;
    const int64_t qb = rows_bytes(rows, row_stride, 5 * HD, es);
    // the bytes of the workspace this call writes (none when the ring kernel runs)
    const int64_t wb = workspace ? static_cast<int64_t>(hb_band_workspace_size(dtype, B, S, H, D, half, window)) : 0;
    int ov;
    if ((ov = check_disjoint("band", "out", out, ob, "qkv", qkv, qb)) ||
        (ov = check_disjoint("band", "workspace", workspace, wb, "qkv", qkv, qb)) ||
        (ov = check_disjoint("band", "workspace", workspace, wb, "out", out, ob)))
      return ov;
    return static_cast<int>(HB_OK);
  };
  if (dtype == HB_F32) {
    if (reinterpret_cast<uintptr_t>(out) % 16) return fail(HB_ERR_STRIDE, "fp32 out must be 16-byte aligned");
    if (workspace) {
      const size_t need = dense_layout(HB_F32, B, S, H, D).total_bytes;
      if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(HB_ERR_WORKSPACE, "workspace must be 256-byte aligned");
      if (workspace_bytes < need) return fail(HB_ERR_WORKSPACE, "workspace holds %zu bytes, needs %zu", workspace_bytes, need);
      if ((st = overlaps())) return st;
      return launch_band_f32_ws(stream, qkv, row_stride, q_dyt, k_dyt, cos, sin, half, window, lam, out, B, S, H, D,
                                workspace);
    }
    if ((st = overlaps())) return st;
    return launch_band_f32(stream, qkv, row_stride, q_dyt, k_dyt, cos, sin, half, window, lam, out, B, S, H, D);
  }
  if (reinterpret_cast<uintptr_t>(out) % 8) return fail(HB_ERR_STRIDE, "out must be 8-byte aligned");
  if (band_ring_supported(dtype, D, half, window)) {
    if ((st = overlaps())) return st;
    return launch_band_ring(stream, dtype, qkv, row_stride, q_dyt, k_dyt, cos, sin, half, window, lam, out, B, S, H);
  }
  const size_t need = band_tiled_layout(B, S, H, D).total_bytes;
  if (!workspace) return fail(HB_ERR_WORKSPACE, "this shape needs a workspace of %zu bytes (hb_band_workspace_size)", need);
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(HB_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (workspace_bytes < need) return fail(HB_ERR_WORKSPACE, "workspace holds %zu bytes, needs %zu", workspace_bytes, need);
  if ((st = overlaps())) return st;
  return launch_band_tiled(stream, dtype, qkv, row_stride, q_dyt, k_dyt, cos, sin, half, window, lam, out, B, S, H, D,
                           workspace);
}
