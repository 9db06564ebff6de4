// Status reporting and argument validation for the C ABI (host code only; no kernels here).
#include "api.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

namespace hb {

namespace {
thread_local char g_last_error[512] = "";
}

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_last_error[0] = '\0'; }

DenseLayout dense_layout(int dtype, int B, int L, int H, int D) {
  DenseLayout lay;
  lay.Lp = round_up(L, kDenseQueryBlock);
  lay.region_elems = static_cast<int64_t>(B) * H * lay.Lp * D;
  lay.elem_bytes = dtype == HB_F32 ? 4 : 2;
  lay.region_bytes = static_cast<size_t>(lay.region_elems) * lay.elem_bytes;
  lay.total_bytes = 3 * lay.region_bytes;
  return lay;
}

int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];  // zero-initialised (static storage); 0 = not yet queried
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  if (dev < kMaxDevices) {
    const int n = cached[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev < kMaxDevices) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

int check_common(int dtype, int64_t row_stride, int B, int N, int H, int D, int half) {
  if (dtype != HB_BF16 && dtype != HB_F32 && dtype != HB_F16)
    return fail(HB_ERR_DTYPE, "dtype %d is not HB_BF16 (0), HB_F32 (1) or HB_F16 (2)", dtype);
  if (D != 64 && D != 128) return fail(HB_ERR_HEAD_DIM, "head_dim %d is not 64 or 128", D);
  if (B < 1 || N < 1 || H < 1) return fail(HB_ERR_SHAPE, "need B, N, H >= 1 (B=%d, N=%d, H=%d)", B, N, H);
  if (B > 65535 || H > 65535 || N > (1 << 28))
    return fail(HB_ERR_SHAPE, "shape out of range (B=%d <= 65535, H=%d <= 65535, N=%d <= 2^28)", B, H, N);
  if (static_cast<int64_t>(B) * N * H * D > (int64_t(1) << 40))
    return fail(HB_ERR_SHAPE, "B*N*H*D exceeds 2^40 elements");
  if (half < 0 || 2 * half > D) return fail(HB_ERR_HALF, "half %d outside [0, D/2=%d]", half, D / 2);
  if (row_stride < static_cast<int64_t>(5) * H * D || row_stride % 8 != 0)
    return fail(HB_ERR_STRIDE, "row_stride %lld must be >= 5*H*D=%lld and a multiple of 8",
                static_cast<long long>(row_stride), static_cast<long long>(5) * H * D);
  return check_extent("attention", "qkv", static_cast<int64_t>(B) * N, row_stride, static_cast<int64_t>(5) * H * D);
}

int check_extent(const char* what, const char* name, int64_t N, int64_t stride, int64_t C) {
  constexpr __int128 kLimit = static_cast<__int128>(1) << 48;
  const __int128 ext = static_cast<__int128>(N > 1 ? N - 1 : 0) * stride + C;
  if (stride < 0 || C < 0 || ext >= kLimit)
    return fail(HB_ERR_STRIDE, "%s: %s spans 2^48 elements or more (%lld rows, row stride %lld)", what, name,
                static_cast<long long>(N), static_cast<long long>(stride));
  return HB_OK;
}

namespace {
int64_t floor_div(int64_t a, int64_t b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }  // b > 0
}  // namespace

bool regions_overlap(const void* a, int64_t as, int64_t ca, const void* b, int64_t bs, int64_t cb, int64_t N,
                     int esize) {
  if (!a || !b || N < 1 || ca < 1 || cb < 1) return false;
  const int64_t pa = static_cast<int64_t>(reinterpret_cast<uintptr_t>(a));
  const int64_t pb = static_cast<int64_t>(reinterpret_cast<uintptr_t>(b));
  const int64_t wa = ca * esize, wb = cb * esize;  // bytes of one row of each
  if (as == bs) {
    // Row i of a, [pa + i S, pa + i S + wa), meets row j of b iff -wa < d + k S < wb with d = pa - pb and
    // k = i - j in [-(N - 1), N - 1]: an interval of k, checked exactly.
    const int64_t S = as * esize, d = pa - pb;
    int64_t lo = floor_div(-wa - d, S) + 1, hi = -floor_div(d - wb, S) - 1;
    if (lo < -(N - 1)) lo = -(N - 1);
    if (hi > N - 1) hi = N - 1;
    return lo <= hi;
  }
  const int64_t ea = pa + (N - 1) * as * esize + wa, eb = pb + (N - 1) * bs * esize + wb;
  return pa < eb && pb < ea;
}

int check_no_overlap(const char* what, const char* out_name, const void* out, int64_t out_stride, int64_t out_cols,
                     const char* in_name, const void* in, int64_t in_stride, int64_t in_cols, int64_t N, int esize,
                     bool in_place_ok) {
  if (in_place_ok && out == in && out_stride == in_stride && out_cols == in_cols) return HB_OK;
  if (regions_overlap(out, out_stride, out_cols, in, in_stride, in_cols, N, esize))
    return fail(HB_ERR_STRIDE, "%s: %s overlaps %s%s", what, out_name, in_name,
                in_place_ok ? " (only the same buffer with the same row stride may be updated in place)" : "");
  return HB_OK;
}

int check_disjoint(const char* what, const char* a_name, const void* a, int64_t a_bytes, const char* b_name,
                   const void* b, int64_t b_bytes) {
  if (!a || !b || a_bytes <= 0 || b_bytes <= 0) return HB_OK;
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  if (pa < pb + static_cast<uintptr_t>(b_bytes) && pb < pa + static_cast<uintptr_t>(a_bytes))
    return fail(HB_ERR_STRIDE, "%s: %s overlaps %s", what, a_name, b_name);
  return HB_OK;
}

}  // namespace hb

extern "C" {

const char* hb_last_error(void) { return hb::g_last_error; }

const char* hb_version(void) { return "hummingbird_amd 0.1.0 (gfx950)"; }

const char* hb_status_name(int status) {
  switch (status) {
    case HB_OK: return "HB_OK";
    case HB_ERR_NULL: return "HB_ERR_NULL";
    case HB_ERR_SHAPE: return "HB_ERR_SHAPE";
    case HB_ERR_DTYPE: return "HB_ERR_DTYPE";
    case HB_ERR_HEAD_DIM: return "HB_ERR_HEAD_DIM";
    case HB_ERR_HALF: return "HB_ERR_HALF";
    case HB_ERR_WINDOW: return "HB_ERR_WINDOW";
    case HB_ERR_STRIDE: return "HB_ERR_STRIDE";
    case HB_ERR_WORKSPACE: return "HB_ERR_WORKSPACE";
    case HB_ERR_LAUNCH: return "HB_ERR_LAUNCH";
    case HB_ERR_EPS: return "HB_ERR_EPS";
    default: return "HB_ERR_UNKNOWN";
  }
}

size_t hb_dense_workspace_size(int dtype, int B, int L, int H, int D) {
  if ((dtype != HB_BF16 && dtype != HB_F32 && dtype != HB_F16) || B < 1 || L < 1 || H < 1 || (D != 64 && D != 128))
    return 0;
  return hb::dense_layout(dtype, B, L, H, D).total_bytes;
}

int hb_dense_validate(int dtype, int64_t row_stride, int B, int L, int H, int D, int half, float eps) {
  hb::clear_error();
  int st = hb::check_common(dtype, row_stride, B, L, H, D, half);
  if (st) return st;
  if (!(eps >= 0.0f) || !isfinite(eps)) return hb::fail(HB_ERR_EPS, "eps %g must be finite and >= 0", eps);
  return HB_OK;
}

int hb_band_validate(int dtype, int64_t row_stride, int B, int S, int H, int D, int half, int window) {
  hb::clear_error();
  int st = hb::check_common(dtype, row_stride, B, S, H, D, half);
  if (st) return st;
  if (window < 0) return hb::fail(HB_ERR_WINDOW, "window %d must be >= 0", window);
  return HB_OK;
}

}  // extern "C"
