// The two elementwise steps of a SAME-L decoder block around the band attention, for gfx950 (MI355X).
//
// Replaces the XLA chain of same_l._block (sa3jax/same_l.py:186-192) between its GEMMs:
//   dyt   out = cast(gamma * tanh(alpha * x) + beta), the fp32 island of same_l._dyt (same_l.py:58-69) cast back
//         to the compute dtype before the next GEMM, as the block does (same_l.py:191-192);
//   glu   out = value * act(gate) for the glu_proj output [value | gate] (same_l._feed_forward, same_l.py:172-183),
//         act = SiLU, or sin(pi * gate) on the sinusoidal blocks.
// Both are single HBM passes: every thread moves 16-byte chunks (8 bf16 or half, or 4 fp32 elements) of one row,
// the per-channel parameters come from L1/L2. Cast points are the reference's: bf16 and half runs round where the
// XLA chain holds an array of the compute dtype (after the DyT; pi itself, pi * gate and the sine; the sigmoid and
// the SiLU; the product); fp32 runs do not round.
#include "api.h"
#include "common.h"
#include "glu_act.h"

namespace hb {
namespace ew {

template <typename T>
struct Vec;
template <>
struct Vec<uint16_t> {  // bf16: 8 elements per 16 bytes
  static constexpr int N = 8;
  static constexpr int kSine = kSineBf16;
  __device__ static void load(const uint16_t* p, float (&x)[8]) { unpack8(ld16(p), x); }
  __device__ static void store(uint16_t* p, const float (&x)[8]) { st16(p, pack8(x)); }
  __device__ static float round(float x) { return round_bf16(x); }
};
template <>
struct Vec<_Float16> {  // IEEE half (the fp16 preset): 8 elements per 16 bytes
  static constexpr int N = 8;
  static constexpr int kSine = kSineHalf;
  __device__ static void load(const _Float16* p, float (&x)[8]) { F16Io::unpack8(ld16(p), x); }
  __device__ static void store(_Float16* p, const float (&x)[8]) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = F16Io::pack2(x[2 * i], x[2 * i + 1]);
    st16(p, v);
  }
  __device__ static float round(float x) { return F16Io::round(x); }
};
template <>
struct Vec<float> {  // fp32: 4 elements per 16 bytes
  static constexpr int N = 4;
  static constexpr int kSine = kSineLibrary;
  __device__ static void load(const float* p, float (&x)[4]) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p);
    for (int i = 0; i < 4; ++i) x[i] = v[i];
  }
  __device__ static void store(float* p, const float (&x)[4]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
  }
  __device__ static float round(float x) { return x; }
};

// Both kernels walk the (row, 16-byte chunk) pairs of the tensor with a grid stride, consecutive threads taking
// consecutive chunks of a row, so every wave moves whole 1 KB runs whatever the row length.
template <typename T>
__global__ __launch_bounds__(256) void dyt_kernel(const T* __restrict__ x, int64_t xs, const float* __restrict__ dyt,
                                                  T* __restrict__ out, int64_t os, int64_t N, int C) {
  constexpr int V = Vec<T>::N;
  const int chunks = C / V;
  const float a2 = 2.f * kLog2e * dyt[0];
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < N * chunks;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t n = i / chunks;
    const int c0 = static_cast<int>(i - n * chunks) * V;
    float v[V];
    Vec<T>::load(x + n * xs + c0, v);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float g = dyt[1 + c0 + j], b = dyt[1 + C + c0 + j];
      v[j] = dyt_tanh(v[j], a2, -2.f * g, g + b);
    }
    Vec<T>::store(out + n * os + c0, v);  // the store's conversion is the single cast
  }
}

// The activation with the XLA chain's intermediate arrays (glu_act.h), rounded before the product.
// `bias` (2F values of the compute dtype, or null): the glu_proj layer's bias, added to the GEMM output in the
// compute dtype first (same_l._linear: the matmul, then the bias add, each held in the compute dtype).
template <typename T, bool SINE>
__global__ __launch_bounds__(256) void glu_kernel(const T* __restrict__ proj, int64_t ps,
                                                  const float* __restrict__ bias, T* __restrict__ out, int64_t os,
                                                  int64_t N, int F) {
  constexpr int V = Vec<T>::N;
  const int chunks = F / V;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < N * chunks;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t n = i / chunks;
    const int c0 = static_cast<int>(i - n * chunks) * V;
    float val[V], g[V];
    Vec<T>::load(proj + n * ps + c0, val);
    Vec<T>::load(proj + n * ps + F + c0, g);
    if (bias) {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        val[i] = Vec<T>::round(val[i] + bias[c0 + i]);
        g[i] = Vec<T>::round(g[i] + bias[F + c0 + i]);
      }
    }
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float act = glu_act<SINE, Vec<T>::kSine>(g[i], [](float x) { return Vec<T>::round(x); });
      val[i] = val[i] * Vec<T>::round(act);
    }
    Vec<T>::store(out + n * os + c0, val);
  }
}

// The block's residual adds with what surrounds them (same_l.py:191-192): out_h = h + (x + bias), the projection's
// bias added first (same_l._linear: the matmul, then the bias add) and each sum held in the compute dtype; then,
// with `dyt`, out_y = cast(DyT(out_h)), the input of the next GEMM (ff_norm inside the block, or the next block's
// pre_norm). One pass where the XLA chain makes two or three. `bias` (C values of the compute dtype as fp32) and
// `dyt` (packed as for dyt_kernel) may be null; out_h may be h itself.
template <typename T>
__global__ __launch_bounds__(256) void residual_dyt_kernel(const T* h, int64_t hs, const T* __restrict__ x,
                                                           int64_t xs, const float* __restrict__ bias,
                                                           const float* __restrict__ dyt, T* out_h,
                                                           T* __restrict__ out_y, int64_t os, int64_t N, int C) {
  constexpr int V = Vec<T>::N;
  const int chunks = C / V;
  const float a2 = dyt ? 2.f * kLog2e * dyt[0] : 0.f;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < N * chunks;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t n = i / chunks;
    const int c0 = static_cast<int>(i - n * chunks) * V;
    float hv[V], xv[V];
    Vec<T>::load(h + n * hs + c0, hv);
    Vec<T>::load(x + n * xs + c0, xv);
    if (bias) {
#pragma unroll
      for (int j = 0; j < V; ++j) xv[j] = Vec<T>::round(xv[j] + bias[c0 + j]);
    }
#pragma unroll
    for (int j = 0; j < V; ++j) hv[j] = Vec<T>::round(hv[j] + xv[j]);
    Vec<T>::store(out_h + n * os + c0, hv);
    if (dyt) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float g = dyt[1 + c0 + j], b = dyt[1 + C + c0 + j];
        hv[j] = dyt_tanh(hv[j], a2, -2.f * g, g + b);
      }
      Vec<T>::store(out_y + n * os + c0, hv);  // the store's conversion is the single cast
    }
  }
}

}  // namespace ew
}  // namespace hb

using namespace hb;

namespace {

int check_rows(const char* what, int dtype, const void* in, int64_t in_stride, const void* out, int64_t out_stride,
               int64_t N, int C, int64_t in_min) {
  if (dtype != HB_BF16 && dtype != HB_F32 && dtype != HB_F16)
    return fail(HB_ERR_DTYPE, "dtype %d is not HB_BF16 (0), HB_F32 (1) or HB_F16 (2)", dtype);
  if (N < 1 || C < 1 || N > (int64_t(1) << 31)) return fail(HB_ERR_SHAPE, "%s needs 1 <= N <= 2^31 and C >= 1", what);
  const int vec = dtype == HB_F32 ? 4 : 8;
  if (C % vec) return fail(HB_ERR_SHAPE, "%s needs the channel count (%d) to be a multiple of %d", what, C, vec);
  if (in_stride < in_min || out_stride < C || in_stride % vec || out_stride % vec)
    return fail(HB_ERR_STRIDE, "%s row strides (%lld, %lld) must be >= (%lld, %d) and multiples of %d", what,
                static_cast<long long>(in_stride), static_cast<long long>(out_stride),
                static_cast<long long>(in_min), C, vec);
  if (!in || !out) return fail(HB_ERR_NULL, "%s input and output must be non-NULL", what);
  if (reinterpret_cast<uintptr_t>(in) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
    return fail(HB_ERR_STRIDE, "%s input and output must be 16-byte aligned", what);
  int st = check_extent(what, "input", N, in_stride, in_min);
  if (st) return st;
  return check_extent(what, "output", N, out_stride, C);
}

// Enough 256-thread blocks for every chunk, at most 16 per CU (the rest is walked with the grid stride).
dim3 row_grid(int64_t N, int chunks) {
  const int64_t need = (N * chunks + 255) / 256, cap = 16 * static_cast<int64_t>(device_cus());
  return dim3(static_cast<unsigned>(need < cap ? need : cap));
}

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HB_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return HB_OK;
}

}  // namespace

extern "C" {

int hb_dyt(hipStream_t stream, const void* x, int dtype, int64_t x_row_stride, const float* dyt, void* out,
           int64_t out_row_stride, int64_t N, int C) {
  clear_error();
  int st = check_rows("dyt", dtype, x, x_row_stride, out, out_row_stride, N, C, C);
  if (st) return st;
  if (!dyt) return fail(HB_ERR_NULL, "dyt parameters must be non-NULL");
  const int es = dtype == HB_F32 ? 4 : 2;
  if ((st = check_no_overlap("dyt", "out", out, out_row_stride, C, "x", x, x_row_stride, C, N, es, false))) return st;
  if ((st = check_disjoint("dyt", "out", out, rows_bytes(N, out_row_stride, C, es), "dyt parameters", dyt,
                           (1 + 2 * static_cast<int64_t>(C)) * 4)))
    return st;
  const int chunks = C / (dtype == HB_F32 ? 4 : 8);
  if (dtype == HB_BF16)
    hipLaunchKernelGGL(ew::dyt_kernel<uint16_t>, row_grid(N, chunks), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(x), x_row_stride, dyt, static_cast<uint16_t*>(out), out_row_stride,
                       N, C);
  else if (dtype == HB_F16)
    hipLaunchKernelGGL(ew::dyt_kernel<_Float16>, row_grid(N, chunks), dim3(256), 0, stream,
                       static_cast<const _Float16*>(x), x_row_stride, dyt, static_cast<_Float16*>(out), out_row_stride,
                       N, C);
  else
    hipLaunchKernelGGL(ew::dyt_kernel<float>, row_grid(N, chunks), dim3(256), 0, stream, static_cast<const float*>(x),
                       x_row_stride, dyt, static_cast<float*>(out), out_row_stride, N, C);
  return launched("dyt");
}

int hb_glu(hipStream_t stream, const void* proj, int dtype, int64_t proj_row_stride, const float* bias,
           int sinusoidal, void* out, int64_t out_row_stride, int64_t N, int F) {
  clear_error();
  int st = check_rows("glu", dtype, proj, proj_row_stride, out, out_row_stride, N, F, static_cast<int64_t>(2) * F);
  if (st) return st;
  // A thread reads the value and gate chunks of its output chunk, which other threads' outputs could cover.
  if ((st = check_no_overlap("glu", "out", out, out_row_stride, F, "proj", proj, proj_row_stride,
                             static_cast<int64_t>(2) * F, N, dtype == HB_F32 ? 4 : 2, false)))
    return st;
  if ((st = check_disjoint("glu", "out", out, rows_bytes(N, out_row_stride, F, dtype == HB_F32 ? 4 : 2), "bias", bias,
                           static_cast<int64_t>(2) * F * 4)))
    return st;
  const int chunks = F / (dtype == HB_F32 ? 4 : 8);
  const dim3 grid = row_grid(N, chunks);
  if (dtype == HB_F16) {
    const _Float16* p = static_cast<const _Float16*>(proj);
    _Float16* o = static_cast<_Float16*>(out);
    if (sinusoidal)
      hipLaunchKernelGGL((ew::glu_kernel<_Float16, true>), grid, dim3(256), 0, stream, p, proj_row_stride, bias,
                         o, out_row_stride, N, F);
    else
      hipLaunchKernelGGL((ew::glu_kernel<_Float16, false>), grid, dim3(256), 0, stream, p, proj_row_stride, bias,
                         o, out_row_stride, N, F);
  } else if (dtype == HB_BF16) {
    const uint16_t* p = static_cast<const uint16_t*>(proj);
    uint16_t* o = static_cast<uint16_t*>(out);
    if (sinusoidal)
      hipLaunchKernelGGL((ew::glu_kernel<uint16_t, true>), grid, dim3(256), 0, stream, p, proj_row_stride, bias,
                         o, out_row_stride, N, F);
    else
      hipLaunchKernelGGL((ew::glu_kernel<uint16_t, false>), grid, dim3(256), 0, stream, p, proj_row_stride, bias,
                         o, out_row_stride, N, F);
  } else {
    const float* p = static_cast<const float*>(proj);
    float* o = static_cast<float*>(out);
    if (sinusoidal)
      hipLaunchKernelGGL((ew::glu_kernel<float, true>), grid, dim3(256), 0, stream, p, proj_row_stride, bias,
                         o, out_row_stride, N, F);
    else
      hipLaunchKernelGGL((ew::glu_kernel<float, false>), grid, dim3(256), 0, stream, p, proj_row_stride, bias,
                         o, out_row_stride, N, F);
  }
  return launched("glu");
}

int hb_residual_dyt(hipStream_t stream, const void* h, int dtype, int64_t h_row_stride, const void* x,
                    int64_t x_row_stride, const float* bias, const float* dyt, void* out_h, void* out_y,
                    int64_t out_row_stride, int64_t N, int C) {
  clear_error();
  int st = check_rows("residual_dyt", dtype, h, h_row_stride, out_h, out_row_stride, N, C, C);
  if (st) return st;
  st = check_rows("residual_dyt", dtype, x, x_row_stride, out_h, out_row_stride, N, C, C);
  if (st) return st;
  if (!dyt != !out_y) return fail(HB_ERR_NULL, "residual_dyt: dyt and out_y are given together or not at all");
  if (out_y && reinterpret_cast<uintptr_t>(out_y) % 16)
    return fail(HB_ERR_STRIDE, "residual_dyt: out_y must be 16-byte aligned");
  const int es = dtype == HB_F32 ? 4 : 2;
  const char* w = "residual_dyt";
  if ((st = check_no_overlap(w, "out_h", out_h, out_row_stride, C, "h", h, h_row_stride, C, N, es, true)) ||
      (st = check_no_overlap(w, "out_h", out_h, out_row_stride, C, "x", x, x_row_stride, C, N, es, false)) ||
      (st = check_no_overlap(w, "out_y", out_y, out_row_stride, C, "h", h, h_row_stride, C, N, es, false)) ||
      (st = check_no_overlap(w, "out_y", out_y, out_row_stride, C, "x", x, x_row_stride, C, N, es, false)) ||
      (st = check_no_overlap(w, "out_y", out_y, out_row_stride, C, "out_h", out_h, out_row_stride, C, N, es, false)))
    return st;
  {
    const int64_t ob = rows_bytes(N, out_row_stride, C, es), cb = static_cast<int64_t>(C) * 4;
    if ((st = check_disjoint(w, "out_h", out_h, ob, "bias", bias, cb)) ||
        (st = check_disjoint(w, "out_h", out_h, ob, "dyt parameters", dyt, cb * 2 + 4)) ||
        (st = check_disjoint(w, "out_y", out_y, ob, "bias", bias, cb)) ||
        (st = check_disjoint(w, "out_y", out_y, ob, "dyt parameters", dyt, cb * 2 + 4)))
      return st;
  }
  const dim3 grid = row_grid(N, C / (dtype == HB_F32 ? 4 : 8));
  if (dtype == HB_BF16)
    hipLaunchKernelGGL(ew::residual_dyt_kernel<uint16_t>, grid, dim3(256), 0, stream, static_cast<const uint16_t*>(h),
                       h_row_stride, static_cast<const uint16_t*>(x), x_row_stride, bias, dyt,
                       static_cast<uint16_t*>(out_h), static_cast<uint16_t*>(out_y), out_row_stride, N, C);
  else if (dtype == HB_F16)
    hipLaunchKernelGGL(ew::residual_dyt_kernel<_Float16>, grid, dim3(256), 0, stream, static_cast<const _Float16*>(h),
                       h_row_stride, static_cast<const _Float16*>(x), x_row_stride, bias, dyt,
                       static_cast<_Float16*>(out_h), static_cast<_Float16*>(out_y), out_row_stride, N, C);
  else
    hipLaunchKernelGGL(ew::residual_dyt_kernel<float>, grid, dim3(256), 0, stream, static_cast<const float*>(h),
                       h_row_stride, static_cast<const float*>(x), x_row_stride, bias, dyt,
                       static_cast<float*>(out_h), static_cast<float*>(out_y), out_row_stride, N, C);
  return launched("residual_dyt");
}

}  // extern "C"
