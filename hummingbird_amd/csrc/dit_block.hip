// The elementwise steps of a DiT block around its GEMMs and attention calls, for gfx950 (MI355X).
//
// Replaces the chain of dit._block between the matmuls (sa3jax/dit.py:224-251), which the reference leaves to
// XLA as separate array operations:
//   rms_modulate    x = rms(h) * (1 + scale) + shift: the block RMSNorm (dit.py:44-57; fp32 mean of squares,
//                   the stored scale applied in fp32, cast back) followed by the adaLN modulation of the self-
//                   attention or feed-forward input (dit.py:231-233, 246-247), or the plain norm (no scale and
//                   shift) of the cross-attention input (dit.py:236);
//   gated_residual  out = h + (x + bias) * sigmoid(1 - gate): the gated residuals of the self-attention and the
//                   feed-forward (dit.py:234, 249-251; the bias is proj_out's, dit.py:221), or the plain residual
//                   of the cross-attention (dit.py:237) followed by the constant local embedding on the latent
//                   tokens (dit.py:239-241);
//   residual_rms    the two back to back on one row: a residual, then the norm (and modulation) that consumes it
//                   (the cross-attention input after the self-attention residual, the feed-forward input after the
//                   cross-attention residual, the next block's input after the feed-forward residual).
// Each is one HBM pass over 16-byte chunks. bf16 and half round where the reference holds an array of the compute
// dtype: after the norm, 1 + scale, the product, the shift; x + bias, 1 - gate, the sigmoid, the product, the
// residual sum, the local sum. fp32 does not round.
#include <cmath>

#include "api.h"
#include "common.h"

namespace hb {
namespace blk {

template <typename T>
struct Vec;
template <>
struct Vec<uint16_t> {  // bf16
  static constexpr int N = 8;
  __device__ static void load(const uint16_t* p, float (&x)[8]) { unpack8(ld16(p), x); }
  __device__ static void store(uint16_t* p, const float (&x)[8]) { st16(p, pack8(x)); }
  __device__ static float round(float x) { return round_bf16(x); }
};
template <>
struct Vec<_Float16> {  // IEEE half
  static constexpr int N = 8;
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
struct Vec<float> {  // fp32
  static constexpr int N = 4;
  __device__ static void load(const float* p, float (&x)[4]) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = v[i];
  }
  __device__ static void store(float* p, const float (&x)[4]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
  }
  __device__ static float round(float x) { return x; }
};

// The logistic function with the hardware exponential and reciprocal (v_exp_f32, v_rcp_f32): within a few fp32
// units of the exactly rounded value, which the compute dtype's rounding that follows hides but for values on a
// tie; in fp32 a relative error of about 1e-6 at |u| = 10. The library expf and the IEEE division took a fifth of
// a gated residual pass (10.0 against 8.1 us for 1422 rows of 1536 bf16 values with the norm).
__device__ __forceinline__ float sigmoid(float u) { return __builtin_amdgcn_rcpf(1.f + fast_exp2(-kLog2e * u)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// One wave per row: the mean of squares over the row (fp32), then the normalised row scaled by `w` (fp32), cast,
// and with `scale` the modulation by the row's batch entry of `scale` / `shift` (`mod_stride` elements apart per
// batch, `L` rows per batch). The row is read twice; the second read hits the cache.
template <typename T>
__global__ __launch_bounds__(256) void rms_modulate_kernel(const T* __restrict__ x, int64_t xs,
                                                           const float* __restrict__ w, float eps,
                                                           const T* __restrict__ scale, const T* __restrict__ shift,
                                                           int64_t mod_stride, int L, T* __restrict__ out, int64_t os,
                                                           int64_t N, int C) {
  constexpr int V = Vec<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 4 + wave_id();
  if (n >= N) return;  // wave-uniform
  const T* row = x + n * xs;
  float ss = 0.f;
  for (int c0 = lane * V; c0 < C; c0 += 64 * V) {
    float v[V];
    Vec<T>::load(row + c0, v);
#pragma unroll
    for (int j = 0; j < V; ++j) ss = ss + v[j] * v[j];
  }
  const float inv = rsqrtf(wave_sum(ss) * (1.f / static_cast<float>(C)) + eps);
  const int64_t b = n / L;
  const T* sc = scale ? scale + b * mod_stride : nullptr;
  const T* sh = shift ? shift + b * mod_stride : nullptr;
  T* orow = out + n * os;
  for (int c0 = lane * V; c0 < C; c0 += 64 * V) {
    float v[V];
    Vec<T>::load(row + c0, v);
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = Vec<T>::round((v[j] * inv) * w[c0 + j]);
    if (sc) {
      float s[V], t[V];
      Vec<T>::load(sc + c0, s);
      Vec<T>::load(sh + c0, t);
#pragma unroll
      for (int j = 0; j < V; ++j) v[j] = Vec<T>::round(Vec<T>::round(v[j] * Vec<T>::round(1.f + s[j])) + t[j]);
    }
    Vec<T>::store(orow + c0, v);
  }
}

// Grid-stride walk over the (row, 16-byte chunk) pairs. Row n belongs to batch n / L at token n % L.
template <typename T>
__global__ __launch_bounds__(256) void gated_residual_kernel(const T* __restrict__ h, int64_t hs,
                                                             const T* __restrict__ x, int64_t xs,
                                                             const T* __restrict__ xbias, const T* __restrict__ gate,
                                                             int64_t gate_stride, const T* __restrict__ local,
                                                             int memory, int L, T* __restrict__ out, int64_t os,
                                                             int64_t N, int C) {
  constexpr int V = Vec<T>::N;
  const int chunks = C / V;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < N * chunks;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t n = i / chunks;
    const int c0 = static_cast<int>(i - n * chunks) * V;
    float hv[V], xv[V];
    Vec<T>::load(h + n * hs + c0, hv);
    Vec<T>::load(x + n * xs + c0, xv);
    if (xbias) {
      float bv[V];
      Vec<T>::load(xbias + c0, bv);
#pragma unroll
      for (int j = 0; j < V; ++j) xv[j] = Vec<T>::round(xv[j] + bv[j]);
    }
    if (gate) {
      float g[V];
      Vec<T>::load(gate + (n / L) * gate_stride + c0, g);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float u = Vec<T>::round(1.f - g[j]);
        xv[j] = Vec<T>::round(xv[j] * Vec<T>::round(sigmoid(u)));
      }
    }
#pragma unroll
    for (int j = 0; j < V; ++j) hv[j] = Vec<T>::round(hv[j] + xv[j]);
    if (local && static_cast<int>(n % L) >= memory) {
      float lv[V];
      Vec<T>::load(local + c0, lv);
#pragma unroll
      for (int j = 0; j < V; ++j) hv[j] = Vec<T>::round(hv[j] + lv[j]);
    }
    Vec<T>::store(out + n * os + c0, hv);
  }
}

// residual then norm of the same row, one wave per row with the row in registers (at most KMAX chunks per lane):
// h' = the gated_residual of (h, x) with the same optional operands and roundings, stored; then
// y = rms_modulate(h') with the same optional modulation, stored. The sum of squares runs over the rounded h' in
// the order rms_modulate_kernel uses, so y equals what the two kernels produce one after the other.
template <typename T, int KMAX>
__global__ __launch_bounds__(256) void residual_rms_kernel(
    const T* __restrict__ h, int64_t hs, const T* __restrict__ x, int64_t xs, const T* __restrict__ xbias,
    const T* __restrict__ gate, int64_t gate_stride, const T* __restrict__ local, int memory,
    const float* __restrict__ w, float eps, const T* __restrict__ scale, const T* __restrict__ shift,
    int64_t mod_stride, int L, T* __restrict__ out_h, T* __restrict__ out_y, int64_t os, int64_t N, int C) {
  constexpr int V = Vec<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 4 + wave_id();
  if (n >= N) return;  // wave-uniform
  const int64_t b = n / L;
  const bool latent = static_cast<int>(n - b * L) >= memory;
  // Every load of the row first (chunks past C are not read), so the wave waits for memory once.
  float r[KMAX][V], xv[KMAX][V], g[KMAX][V], bv[KMAX][V], lv[KMAX][V];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int c0 = (lane + 64 * k) * V;
    if (c0 < C) {
      Vec<T>::load(h + n * hs + c0, r[k]);
      Vec<T>::load(x + n * xs + c0, xv[k]);
      if (xbias) Vec<T>::load(xbias + c0, bv[k]);
      if (gate) Vec<T>::load(gate + b * gate_stride + c0, g[k]);
      if (local && latent) Vec<T>::load(local + c0, lv[k]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int c0 = (lane + 64 * k) * V;
    if (c0 < C) {
      if (xbias) {
#pragma unroll
        for (int j = 0; j < V; ++j) xv[k][j] = Vec<T>::round(xv[k][j] + bv[k][j]);
      }
      if (gate) {
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const float u = Vec<T>::round(1.f - g[k][j]);
          xv[k][j] = Vec<T>::round(xv[k][j] * Vec<T>::round(sigmoid(u)));
        }
      }
#pragma unroll
      for (int j = 0; j < V; ++j) r[k][j] = Vec<T>::round(r[k][j] + xv[k][j]);
      if (local && latent) {
#pragma unroll
        for (int j = 0; j < V; ++j) r[k][j] = Vec<T>::round(r[k][j] + lv[k][j]);
      }
      Vec<T>::store(out_h + n * os + c0, r[k]);
#pragma unroll
      for (int j = 0; j < V; ++j) ss = ss + r[k][j] * r[k][j];
    }
  }
  const float inv = rsqrtf(wave_sum(ss) * (1.f / static_cast<float>(C)) + eps);
  const T* sc = scale ? scale + b * mod_stride : nullptr;
  const T* sh = shift ? shift + b * mod_stride : nullptr;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int c0 = (lane + 64 * k) * V;
    if (c0 < C) {
      float v[V];
#pragma unroll
      for (int j = 0; j < V; ++j) v[j] = Vec<T>::round((r[k][j] * inv) * w[c0 + j]);
      if (sc) {
        float s[V], t[V];
        Vec<T>::load(sc + c0, s);
        Vec<T>::load(sh + c0, t);
#pragma unroll
        for (int j = 0; j < V; ++j) v[j] = Vec<T>::round(Vec<T>::round(v[j] * Vec<T>::round(1.f + s[j])) + t[j]);
      }
      Vec<T>::store(out_y + n * os + c0, v);
    }
  }
}

}  // namespace blk
}  // namespace hb

using namespace hb;

namespace {

int vec_of(int dtype) { return dtype == HB_F32 ? 4 : 8; }

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int check_common(const char* what, int dtype, int64_t N, int C, int L) {
  if (dtype != HB_BF16 && dtype != HB_F32 && dtype != HB_F16)
    return fail(HB_ERR_DTYPE, "dtype %d is not HB_BF16 (0), HB_F32 (1) or HB_F16 (2)", dtype);
  if (N < 1 || C < 1 || N > (int64_t(1) << 31) || L < 1)
    return fail(HB_ERR_SHAPE, "%s needs 1 <= N <= 2^31, C >= 1 and rows_per_batch >= 1", what);
  if (C % vec_of(dtype)) return fail(HB_ERR_SHAPE, "%s needs C (%d) to be a multiple of %d", what, C, vec_of(dtype));
  return HB_OK;
}

// `rows` rows of `min_stride` elements, `stride` apart.
int check_tensor(const char* what, const char* name, const void* p, int64_t stride, int64_t min_stride, int dtype,
                 bool required, int64_t rows) {
  if (!p) return required ? fail(HB_ERR_NULL, "%s: %s must be non-NULL", what, name) : HB_OK;
  if (!aligned16(p)) return fail(HB_ERR_STRIDE, "%s: %s must be 16-byte aligned", what, name);
  if (stride < min_stride || stride % vec_of(dtype))
    return fail(HB_ERR_STRIDE, "%s: %s stride %lld must be >= %lld and a multiple of %d", what, name,
                static_cast<long long>(stride), static_cast<long long>(min_stride), vec_of(dtype));
  return check_extent(what, name, rows, stride, min_stride);
}

// An output region (bytes) against every vector the call reads: a per-channel vector of C elements of `es` bytes
// (x_bias, local; fp32 weight) or the per-batch rows of the adaLN operands (scale, shift, gate: nb rows `bs`
// elements apart). Workgroups read these while others write their output rows, so they may share no byte.
struct Reads {
  const char* name;
  const void* p;
  int64_t bytes;
};
int check_out_vs_reads(const char* what, const char* oname, const void* out, int64_t ob, const Reads* r, int n) {
  for (int i = 0; i < n; ++i) {
    const int st = check_disjoint(what, oname, out, ob, r[i].name, r[i].p, r[i].bytes);
    if (st) return st;
  }
  return HB_OK;
}

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HB_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return HB_OK;
}

template <typename T>
void launch_rms(hipStream_t s, const void* x, int64_t xs, const float* w, float eps, const void* scale,
                const void* shift, int64_t ms, int L, void* out, int64_t os, int64_t N, int C) {
  const dim3 grid(static_cast<unsigned>((N + 3) / 4));
  hipLaunchKernelGGL(blk::rms_modulate_kernel<T>, grid, dim3(256), 0, s, static_cast<const T*>(x), xs, w, eps,
                     static_cast<const T*>(scale), static_cast<const T*>(shift), ms, L, static_cast<T*>(out), os, N,
                     C);
}

template <typename T>
void launch_residual(hipStream_t s, const void* h, int64_t hs, const void* x, int64_t xs, const void* xbias,
                     const void* gate, int64_t gs, const void* local, int memory, int L, void* out, int64_t os,
                     int64_t N, int C) {
  const int64_t chunks = C / blk::Vec<T>::N;
  const int64_t need = (N * chunks + 255) / 256, cap = 16 * static_cast<int64_t>(device_cus());
  hipLaunchKernelGGL(blk::gated_residual_kernel<T>, dim3(static_cast<unsigned>(need < cap ? need : cap)), dim3(256),
                     0, s, static_cast<const T*>(h), hs, static_cast<const T*>(x), xs, static_cast<const T*>(xbias),
                     static_cast<const T*>(gate), gs, static_cast<const T*>(local), memory, L, static_cast<T*>(out), os,
                     N, C);
}

// 16-byte chunks of a row per lane: rows of up to 2048 values (4 chunks of 8 bf16 / half, 8 chunks of 4 fp32).
template <typename T>
constexpr int kResidualRmsChunks = sizeof(T) == 4 ? 8 : 4;
constexpr int kResidualRmsMaxC = 2048;

template <typename T>
void launch_residual_rms(hipStream_t s, const void* h, int64_t hs, const void* x, int64_t xs, const void* xbias,
                         const void* gate, int64_t gs, const void* local, int memory, const float* w, float eps,
                         const void* scale, const void* shift, int64_t ms, int L, void* out_h, void* out_y, int64_t os,
                         int64_t N, int C) {
  hipLaunchKernelGGL((blk::residual_rms_kernel<T, kResidualRmsChunks<T>>), dim3(static_cast<unsigned>((N + 3) / 4)),
                     dim3(256), 0, s, static_cast<const T*>(h), hs, static_cast<const T*>(x), xs,
                     static_cast<const T*>(xbias), static_cast<const T*>(gate), gs, static_cast<const T*>(local), memory,
                     w, eps, static_cast<const T*>(scale), static_cast<const T*>(shift), ms, L, static_cast<T*>(out_h),
                     static_cast<T*>(out_y), os, N, C);
}

}  // namespace

extern "C" {

int hb_rms_modulate(hipStream_t stream, const void* x, int dtype, int64_t x_row_stride, const float* weight,
                    float eps, const void* scale, const void* shift, int64_t mod_batch_stride, int rows_per_batch,
                    void* out, int64_t out_row_stride, int64_t N, int C) {
  clear_error();
  int st = check_common("rms_modulate", dtype, N, C, rows_per_batch);
  if (st) return st;
  if ((st = check_tensor("rms_modulate", "x", x, x_row_stride, C, dtype, true, N))) return st;
  if ((st = check_tensor("rms_modulate", "out", out, out_row_stride, C, dtype, true, N))) return st;
  if (!weight) return fail(HB_ERR_NULL, "rms_modulate: weight must be non-NULL");
  if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(HB_ERR_EPS, "rms_modulate: eps %g must be finite and >= 0", eps);
  if (!scale != !shift) return fail(HB_ERR_NULL, "rms_modulate: scale and shift are given together or not at all");
  if (scale) {
    if (N % rows_per_batch) return fail(HB_ERR_SHAPE, "rms_modulate: N must be a multiple of rows_per_batch");
    const int64_t stride = N / rows_per_batch > 1 ? mod_batch_stride : C;  // unused with a single batch
    if ((st = check_tensor("rms_modulate", "scale", scale, stride, C, dtype, true, N / rows_per_batch))) return st;
    if ((st = check_tensor("rms_modulate", "shift", shift, stride, C, dtype, true, N / rows_per_batch))) return st;
  }
  if ((st = check_no_overlap("rms_modulate", "out", out, out_row_stride, C, "x", x, x_row_stride, C, N,
                             dtype == HB_F32 ? 4 : 2, false)))
    return st;
  {
    const int es = dtype == HB_F32 ? 4 : 2;
    const int64_t nb = scale ? N / rows_per_batch : 1, ms = nb > 1 ? mod_batch_stride : C;
    const Reads r[] = {{"weight", weight, static_cast<int64_t>(C) * 4},
                       {"scale", scale, rows_bytes(nb, ms, C, es)},
                       {"shift", shift, rows_bytes(nb, ms, C, es)}};
    if ((st = check_out_vs_reads("rms_modulate", "out", out, rows_bytes(N, out_row_stride, C, es), r, 3))) return st;
  }
  if (dtype == HB_BF16)
    launch_rms<uint16_t>(stream, x, x_row_stride, weight, eps, scale, shift, mod_batch_stride, rows_per_batch, out,
                         out_row_stride, N, C);
  else if (dtype == HB_F16)
    launch_rms<_Float16>(stream, x, x_row_stride, weight, eps, scale, shift, mod_batch_stride, rows_per_batch, out,
                         out_row_stride, N, C);
  else
    launch_rms<float>(stream, x, x_row_stride, weight, eps, scale, shift, mod_batch_stride, rows_per_batch, out,
                      out_row_stride, N, C);
  return launched("rms_modulate");
}

int hb_gated_residual(hipStream_t stream, const void* h, int dtype, int64_t h_row_stride, const void* x,
                      int64_t x_row_stride, const void* x_bias, const void* gate, int64_t gate_batch_stride,
                      const void* local, int memory, int rows_per_batch, void* out, int64_t out_row_stride,
                      int64_t N, int C) {
  clear_error();
  int st = check_common("gated_residual", dtype, N, C, rows_per_batch);
  if (st) return st;
  if ((st = check_tensor("gated_residual", "h", h, h_row_stride, C, dtype, true, N))) return st;
  if ((st = check_tensor("gated_residual", "x", x, x_row_stride, C, dtype, true, N))) return st;
  if ((st = check_tensor("gated_residual", "out", out, out_row_stride, C, dtype, true, N))) return st;
  if ((st = check_tensor("gated_residual", "x_bias", x_bias, C, C, dtype, false, 1))) return st;
  if ((st = check_tensor("gated_residual", "local", local, C, C, dtype, false, 1))) return st;
  if (gate) {
    if (N % rows_per_batch) return fail(HB_ERR_SHAPE, "gated_residual: N must be a multiple of rows_per_batch");
    const bool several = N / rows_per_batch > 1;
    if ((st = check_tensor("gated_residual", "gate", gate, several ? gate_batch_stride : C, C, dtype, true,
                           N / rows_per_batch)))
      return st;
  }
  if (memory < 0) return fail(HB_ERR_SHAPE, "gated_residual: memory must be >= 0");
  {
    const int es = dtype == HB_F32 ? 4 : 2;
    if ((st = check_no_overlap("gated_residual", "out", out, out_row_stride, C, "h", h, h_row_stride, C, N, es,
                               false)) ||
        (st = check_no_overlap("gated_residual", "out", out, out_row_stride, C, "x", x, x_row_stride, C, N, es,
                               false)))
      return st;
    const int64_t nb = gate ? N / rows_per_batch : 1, gs = nb > 1 ? gate_batch_stride : C;
    const Reads r[] = {{"x_bias", x_bias, static_cast<int64_t>(C) * es},
                       {"local", local, static_cast<int64_t>(C) * es},
                       {"gate", gate, rows_bytes(nb, gs, C, es)}};
    if ((st = check_out_vs_reads("gated_residual", "out", out, rows_bytes(N, out_row_stride, C, es), r, 3))) return st;
  }
  if (dtype == HB_BF16)
    launch_residual<uint16_t>(stream, h, h_row_stride, x, x_row_stride, x_bias, gate, gate_batch_stride, local,
                              memory, rows_per_batch, out, out_row_stride, N, C);
  else if (dtype == HB_F16)
    launch_residual<_Float16>(stream, h, h_row_stride, x, x_row_stride, x_bias, gate, gate_batch_stride, local,
                              memory, rows_per_batch, out, out_row_stride, N, C);
  else
    launch_residual<float>(stream, h, h_row_stride, x, x_row_stride, x_bias, gate, gate_batch_stride, local, memory,
                           rows_per_batch, out, out_row_stride, N, C);
  return launched("gated_residual");
}

int hb_residual_rms(hipStream_t stream, const void* h, int dtype, int64_t h_row_stride, const void* x,
                    int64_t x_row_stride, const void* x_bias, const void* gate, int64_t gate_batch_stride,
                    const void* local, int memory, const float* weight, float eps, const void* scale,
                    const void* shift, int64_t mod_batch_stride, int rows_per_batch, void* out_h, void* out_y,
                    int64_t out_row_stride, int64_t N, int C) {
  clear_error();
  int st = check_common("residual_rms", dtype, N, C, rows_per_batch);
  if (st) return st;
  if (C > kResidualRmsMaxC)
    return fail(HB_ERR_SHAPE, "residual_rms holds a row in registers: C (%d) must be <= %d", C, kResidualRmsMaxC);
  if ((st = check_tensor("residual_rms", "h", h, h_row_stride, C, dtype, true, N))) return st;
  if ((st = check_tensor("residual_rms", "x", x, x_row_stride, C, dtype, true, N))) return st;
  if ((st = check_tensor("residual_rms", "out_h", out_h, out_row_stride, C, dtype, true, N))) return st;
  if ((st = check_tensor("residual_rms", "out_y", out_y, out_row_stride, C, dtype, true, N))) return st;
  if ((st = check_tensor("residual_rms", "x_bias", x_bias, C, C, dtype, false, 1))) return st;
  if ((st = check_tensor("residual_rms", "local", local, C, C, dtype, false, 1))) return st;
  if (!weight) return fail(HB_ERR_NULL, "residual_rms: weight must be non-NULL");
  if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(HB_ERR_EPS, "residual_rms: eps %g must be finite and >= 0", eps);
  if (!scale != !shift) return fail(HB_ERR_NULL, "residual_rms: scale and shift are given together or not at all");
  if (memory < 0) return fail(HB_ERR_SHAPE, "residual_rms: memory must be >= 0");
  if (gate || scale) {
    if (N % rows_per_batch) return fail(HB_ERR_SHAPE, "residual_rms: N must be a multiple of rows_per_batch");
    const bool several = N / rows_per_batch > 1;
    const int64_t nb = N / rows_per_batch;
    if (gate && (st = check_tensor("residual_rms", "gate", gate, several ? gate_batch_stride : C, C, dtype, true, nb)))
      return st;
    if (scale &&
        ((st = check_tensor("residual_rms", "scale", scale, several ? mod_batch_stride : C, C, dtype, true, nb)) ||
         (st = check_tensor("residual_rms", "shift", shift, several ? mod_batch_stride : C, C, dtype, true, nb))))
      return st;
  }
  {
    const int es = dtype == HB_F32 ? 4 : 2;
    const char* w = "residual_rms";
    if ((st = check_no_overlap(w, "out_h", out_h, out_row_stride, C, "h", h, h_row_stride, C, N, es, false)) ||
        (st = check_no_overlap(w, "out_h", out_h, out_row_stride, C, "x", x, x_row_stride, C, N, es, false)) ||
        (st = check_no_overlap(w, "out_y", out_y, out_row_stride, C, "h", h, h_row_stride, C, N, es, false)) ||
        (st = check_no_overlap(w, "out_y", out_y, out_row_stride, C, "x", x, x_row_stride, C, N, es, false)) ||
        (st = check_no_overlap(w, "out_y", out_y, out_row_stride, C, "out_h", out_h, out_row_stride, C, N, es, false)))
      return st;
    const int64_t nb = (gate || scale) ? N / rows_per_batch : 1;
    const int64_t gs = nb > 1 ? gate_batch_stride : C, ms = nb > 1 ? mod_batch_stride : C;
    const Reads r[] = {{"x_bias", x_bias, static_cast<int64_t>(C) * es},
                       {"local", local, static_cast<int64_t>(C) * es},
                       {"weight", weight, static_cast<int64_t>(C) * 4},
                       {"gate", gate, rows_bytes(nb, gs, C, es)},
                       {"scale", scale, rows_bytes(nb, ms, C, es)},
                       {"shift", shift, rows_bytes(nb, ms, C, es)}};
    const int64_t ob = rows_bytes(N, out_row_stride, C, es);
    if ((st = check_out_vs_reads(w, "out_h", out_h, ob, r, 6)) || (st = check_out_vs_reads(w, "out_y", out_y, ob, r, 6)))
      return st;
  }
  if (dtype == HB_BF16)
    launch_residual_rms<uint16_t>(stream, h, h_row_stride, x, x_row_stride, x_bias, gate, gate_batch_stride, local,
                                  memory, weight, eps, scale, shift, mod_batch_stride, rows_per_batch, out_h, out_y,
                                  out_row_stride, N, C);
  else if (dtype == HB_F16)
    launch_residual_rms<_Float16>(stream, h, h_row_stride, x, x_row_stride, x_bias, gate, gate_batch_stride, local,
                                  memory, weight, eps, scale, shift, mod_batch_stride, rows_per_batch, out_h, out_y,
                                  out_row_stride, N, C);
  else
    launch_residual_rms<float>(stream, h, h_row_stride, x, x_row_stride, x_bias, gate, gate_batch_stride, local,
                               memory, weight, eps, scale, shift, mod_batch_stride, rows_per_batch, out_h, out_y,
                               out_row_stride, N, C);
  return launched("residual_rms");
}

}  // extern "C"
