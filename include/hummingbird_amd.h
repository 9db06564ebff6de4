/* hummingbird_amd: MI355X (gfx950) differential-attention kernels behind a plain C ABI.
 *
 * Two operations replace the reference's two fused TPU kernels (kelechi-c/hummingbird, sa3jax/); the others
 * replace XLA chains next to them (the DiT cross-attention, the SAME-L block's elementwise steps):
 *
 *   hb_dense_diffattn  replaces  dense_attention.dense_attention  (sa3jax/dense_attention.py:104-153),
 *                      called from dit._self_attention (sa3jax/dit.py:191-195);
 *   hb_band_diffattn   replaces  band_attention.band_attention    (sa3jax/band_attention.py:123-180),
 *                      called from same_l._attention (sa3jax/same_l.py:158-161);
 *   hb_cross_prep +    replace   the XLA chain of dit._cross_attention and its hoisted context K/V
 *   hb_cross_attend              (sa3jax/dit.py:203-215, 274-284), which the reference runs without a kernel;
 *   hb_dyt, hb_glu,    replace   the elementwise steps of same_l._block around its GEMMs (sa3jax/same_l.py:58-69,
 *   hb_residual_dyt              172-192), an XLA chain in the reference;
 *   hb_dit_qkv_proj,   replace   the GEMMs either side of the DiT kernel (sa3jax/dit.py:190, 195), the first with the
 *   hb_dense_attend_qq,          dense kernel's key preparation in its epilogue;
 *   hb_proj
 *   hb_rms_modulate,   replace   the elementwise steps of dit._block around its GEMMs and attention calls
 *   hb_gated_residual,           (sa3jax/dit.py:224-251), an XLA chain in the reference;
 *   hb_residual_rms
 *   hb_rope_tables     replaces  band_attention.rope_tables / dit._rope_tables
 *                      (sa3jax/band_attention.py:43-58, sa3jax/dit.py:82-87) in a kernel-native layout.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers except where stated. Nothing is allocated: scratch is the caller's
 *     `workspace` (size from hb_dense_workspace_size).
 *   - Work is enqueued on `stream`; no entry point synchronises the host.
 *   - The packed input `qkv` is (B, N, 5*H*D) = [q | k | v | q_diff | k_diff], head-major inside each section
 *     (sa3jax/dit.py:196-198, sa3jax/same_l.py:162). Element (b, n, c) sits at
 *     qkv[(b*N + n) * row_stride + c]; row_stride >= 5*H*D and a multiple of 8 elements; qkv 16-byte aligned.
 *   - The output `out` is dense (B, N, H*D) in `b n (h d)` order (sa3jax/dit.py:107-110), dtype = input dtype.
 *   - Outputs and workspaces share no byte with the buffers the same call reads, nor with each other, as the
 *     reference's functional calls never alias; an overlap is refused with HB_ERR_STRIDE before any launch. The
 *     row-wise block entry points below state their exact rule (in-place hb_residual_dyt).
 *   - `lam` (H floats, or NULL for all ones) weights the second branch: out = A - lam[h] * B. lam = 1 is the
 *     reference's unweighted difference (sa3jax/dit.py:146, sa3jax/same_l.py:168).
 *   - Return value: HB_OK, or an HB_ERR_* code; hb_last_error() then describes the failure (thread-local).
 *     Shape errors correspond to the reference's trace-time ValueErrors (sa3jax/dense_attention.py:119-120,
 *     sa3jax/band_attention.py:138-140).
 */
#ifndef HUMMINGBIRD_AMD_H
#define HUMMINGBIRD_AMD_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum hb_status {
  HB_OK = 0,
  HB_ERR_NULL = 1,      /* a required pointer is NULL */
  HB_ERR_SHAPE = 2,     /* B, N or H out of range */
  HB_ERR_DTYPE = 3,     /* dtype is not HB_BF16, HB_F32 or HB_F16 */
  HB_ERR_HEAD_DIM = 4,  /* D is not 64 or 128 */
  HB_ERR_HALF = 5,      /* rotary half-width outside [0, D/2] or not a multiple of 8 */
  HB_ERR_WINDOW = 6,    /* band half-width < 0 */
  HB_ERR_STRIDE = 7,    /* row_stride < 5*H*D, not a multiple of 8, or qkv misaligned */
  HB_ERR_WORKSPACE = 8, /* workspace missing, too small or misaligned */
  HB_ERR_LAUNCH = 9,    /* the HIP runtime rejected a launch */
  HB_ERR_EPS = 10       /* eps < 0 or not finite */
};

/* The element type of the 16- or 32-bit inputs and outputs: the compute dtype of the reference's presets
 * (sa3jax/dtypes.py:40-58). HB_BF16 is the bf16 preset and HB_F16 the fp16 preset; under both the attention
 * operands (K, q * scale, P, V) are rounded to bf16 as in the reference's fused kernels
 * (sa3jax/dense_attention.py:75-77, 83, 90; sa3jax/band_attention.py:85, 94, 101), while the RMSNorm and RoPE
 * outputs round to the compute dtype (sa3jax/dense_attention.py:66, 69) and the output is written in it. HB_F32
 * is the FP32_PARITY preset: fp32 throughout (the XLA chain's arithmetic). */
enum hb_dtype { HB_BF16 = 0, HB_F32 = 1, HB_F16 = 2 };

/* Message for the last failing call on this thread ("" if none). */
const char* hb_last_error(void);
/* Static name of a status code. */
const char* hb_status_name(int status);
/* Library version string. */
const char* hb_version(void);

/* ---- RoPE tables ---------------------------------------------------------------------------------------
 * cos[n*half + j] = cos(fp32(n) * inv_freq[j]), sin likewise, for n in [0, length), j in [0, half).
 * The angle is the fp32 product, as in the reference (sa3jax/dit.py:85, sa3jax/same_l.py:87); its cosine and
 * sine are evaluated in double precision and rounded once. These (length, half) tables hold the same values
 * as the reference's duplicated (length, 2*half) tables and its lane tables (sa3jax/band_attention.py:49-58). */
int hb_rope_tables(hipStream_t stream, const float* inv_freq, int half, int length, float* cos, float* sin);

/* ---- DiT dense differential self-attention --------------------------------------------------------------
 * Replaces dense_attention.dense_attention (sa3jax/dense_attention.py:104-153) and the XLA chain it stands
 * in for (sa3jax/dit.py:185-200). Per (batch b, head h), with `x` the head's D-slice of a section:
 *   q, q_diff <- RoPE(RMSNorm(x; q_weight, eps)),   k, k_diff <- RoPE(RMSNorm(x; k_weight, eps)),
 *   v <- v * vmask[b, n],
 *   out = softmax(q k^T / sqrt(D)) v - lam[h] * softmax(q_diff k_diff^T / sqrt(D)) v,
 * with RMSNorm as sa3jax/dit.py:45-57 and half-half rotate_half RoPE over the first 2*half dims as
 * sa3jax/dit.py:90-98. The softmax sees every key; vmask zeroes values only (sa3jax/dit.py:113-116).
 *   q_weight, k_weight : D floats (RMSNorm scales)
 *   cos, sin           : (L, half) floats from hb_rope_tables (ignored when half == 0)
 *   vmask              : (B, L) floats, or NULL for all ones
 *   dtype              : HB_BF16, HB_F16 or HB_F32 (of qkv and out)
 *   D                  : 64 or 128;  0 <= half <= D/2 with half % 8 == 0;  eps >= 0
 *   workspace          : >= hb_dense_workspace_size(dtype, B, L, H, D) bytes, 256-byte aligned; holds the
 *                        prepared k, k_diff and v for the duration of the call (stream-ordered).
 * Internally two kernels run on `stream`: hb_dense_prep then hb_dense_attend (exported separately below). */
size_t hb_dense_workspace_size(int dtype, int B, int L, int H, int D);
int hb_dense_validate(int dtype, int64_t row_stride, int B, int L, int H, int D, int half, float eps);
int hb_dense_diffattn(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride,
                      const float* q_weight, const float* k_weight, const float* cos, const float* sin, int half,
                      const float* vmask, const float* lam, void* out, int B, int L, int H, int D, float eps,
                      void* workspace, size_t workspace_bytes);
/* No-allocation variant of hb_dense_diffattn. It has no counterpart in the reference: it is for callers that
 * cannot allocate device memory or pass a workspace (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). The workspace is a file-scope device array of hb_dense_noalloc_max_bytes() bytes (64 MiB,
 * which holds the 120 s clip's bf16 workspace), held by every GPU the library runs on until the process ends; its
 * device address is looked up once per device. Shapes whose hb_dense_workspace_size exceeds it are rejected with
 * HB_ERR_WORKSPACE before anything runs. The call allocates nothing and otherwise behaves as hb_dense_diffattn.
 * All calls on one GPU share that GPU's array: calls that overlap on one GPU (streams with no ordering between
 * them) race and must not be issued. */
size_t hb_dense_noalloc_max_bytes(void);
int hb_dense_diffattn_noalloc(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride,
                              const float* q_weight, const float* k_weight, const float* cos, const float* sin,
                              int half, const float* vmask, const float* lam, void* out, int B, int L, int H, int D,
                              float eps);
/* Stage 1: RMSNorm + RoPE of k and k_diff and V-masking into `workspace` (kernel-native layout). q_weight is
 * checked but not read. */
int hb_dense_prep(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride,
                  const float* q_weight, const float* k_weight, const float* cos, const float* sin, int half,
                  const float* vmask, int B, int L, int H, int D, float eps, void* workspace,
                  size_t workspace_bytes);
/* Stage 2: RMSNorm + RoPE of q and q_diff (read from the same qkv), both softmax attentions and the
 * subtraction, against a workspace that hb_dense_prep filled from this qkv. Arguments as hb_dense_diffattn. */
int hb_dense_attend(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride,
                    const float* q_weight, const float* k_weight, const float* cos, const float* sin, int half,
                    const float* lam, void* out, int B, int L, int H, int D, float eps,
                    const void* workspace, size_t workspace_bytes);

/* ---- DiT self-attention projections ---------------------------------------------------------------------
 * hb_dit_qkv_proj replaces `qkv = _linear(h, to_qkv)` (sa3jax/dit.py:190) together with the key-side half of
 * dense_attention.dense_attention (the preparation of sa3jax/dense_attention.py:61-77): one matrix-core GEMM
 * h (B*L, E) x W_qkv^T (E, 5*H*D) whose fp32 accumulators are rounded to the compute dtype (the reference's `qkv`)
 * and then finished by section [q | k | v | q_diff | k_diff] (sa3jax/dit.py:196-198): q and q_diff are written to
 * `qq` (B, L, 2*H*D) as rows [q | q_diff]; k and k_diff are RMS-normed with k_weight and rotated, v is multiplied
 * by vmask, and all three are written to `workspace` in the layout hb_dense_prep produces. `qkv` itself is never
 * stored. hb_dense_attend_qq then runs the attention of hb_dense_attend with its queries read from `qq`.
 *   h      : (B, L, E) rows with stride h_row_stride (>= E, a multiple of 8), 16-byte aligned
 *   w_qkv  : (5*H*D, E) row-major with stride w_row_stride (the layer's weight as stored, out x in)
 *   dtype  : HB_BF16 or HB_F16;  D = 64;  H a multiple of 4;  E a multiple of 64;  half a multiple of 8 <= 32
 *   cos, sin, vmask, k_weight, eps, workspace: as hb_dense_diffattn (workspace >= hb_dense_workspace_size)
 * hb_proj replaces `_linear(x, W)` without bias (sa3jax/dit.py:195, the to_out projection): out (N, F) = x (N, K)
 * x W^T (K, F) on the matrix cores, fp32 accumulation, one rounding to dtype; K a multiple of 64, F of 256. */
int hb_dit_qkv_proj(hipStream_t stream, const void* h, int dtype, int64_t h_row_stride, const void* w_qkv,
                    int64_t w_row_stride, int E, const float* k_weight, const float* cos, const float* sin, int half,
                    const float* vmask, void* qq, int B, int L, int H, int D, float eps, void* workspace,
                    size_t workspace_bytes);
int hb_dense_attend_qq(hipStream_t stream, const void* qq, int dtype, int64_t row_stride, const float* q_weight,
                       const float* k_weight, const float* cos, const float* sin, int half, const float* lam, void* out,
                       int B, int L, int H, int D, float eps, const void* workspace, size_t workspace_bytes);
int hb_proj(hipStream_t stream, const void* x, int dtype, int64_t x_row_stride, const void* w, int64_t w_row_stride,
            void* out, int64_t out_row_stride, int64_t N, int K, int F);

/* ---- SAME-L decoder block: projections with the work next to them in their epilogues ----------------------
 * hb_proj_glu replaces the feed-forward's `glu_proj` and the GLU after it (same_l._feed_forward,
 *   sa3jax/same_l.py:181-183): out (N, F) = value * act(gate) for [value | gate] = x (N, K) x W^T (K, 2F), W (2F, K)
 *   the layer's weight as stored (out x in; value rows first). The product is rounded to dtype (the reference's
 *   stored glu_proj output), `bias` (2F floats holding values of dtype, or NULL) added and rounded, then act and the
 *   product with hb_glu's cast points (act = SiLU, or sin(pi * gate) when `sinusoidal` != 0); the 2F-wide product is
 *   never stored. K a multiple of 64, F of 128; dtype HB_BF16 or HB_F16.
 * hb_proj_residual replaces `to_out` / `proj_out` and the residual add after them (sa3jax/same_l.py:161, 184 with
 *   191, 192): out_h (N, F) = h + (x W^T + bias) and, with `dyt` (packed as for hb_dyt), out_y = cast(DyT(out_h)),
 *   the next GEMM's input; the product, the bias add and the sum are each rounded to dtype, as hb_residual_dyt
 *   computes them from the stored product. W (F, K); K a multiple of 64, F of 256; bias: F floats or NULL; `dyt`
 *   and `out_y` both given or both NULL. out_h may be h itself (same row stride); otherwise no output shares an
 *   element with h, x, w, bias, dyt or the other output (HB_ERR_STRIDE).
 * Both: x rows with stride x_row_stride (>= K, a multiple of 8), x and w 16-byte aligned, outputs 8-byte aligned
 *   with row strides >= F and multiples of 4; fp32 accumulation over K in order. */
int hb_proj_glu(hipStream_t stream, const void* x, int dtype, int64_t x_row_stride, const void* w,
                int64_t w_row_stride, const float* bias, int sinusoidal, void* out, int64_t out_row_stride, int64_t N,
                int K, int F);
int hb_proj_residual(hipStream_t stream, const void* x, int dtype, int64_t x_row_stride, const void* w,
                     int64_t w_row_stride, const float* bias, const void* h, int64_t h_row_stride, const float* dyt,
                     void* out_h, void* out_y, int64_t out_row_stride, int64_t N, int K, int F);

/* ---- SAME-L band differential attention -----------------------------------------------------------------
 * Replaces band_attention.band_attention (sa3jax/band_attention.py:123-180) and the XLA chain it stands in
 * for (sa3jax/same_l.py:151-169). Per (batch b, head h):
 *   q, q_diff <- RoPE(DyT(x; q_dyt)),   k, k_diff <- RoPE(DyT(x; k_dyt)),   DyT(x) = gamma*tanh(alpha*x)+beta,
 *   out[i] = sum_{|j-i|<=window, 0<=j<S} softmax_j(q_i . k_j / sqrt(D)) v_j - lam[h] * (same with q_diff, k_diff)
 * with DyT as sa3jax/same_l.py:58-69 and RoPE as sa3jax/same_l.py:92-100; `window` is the reference's band
 * half-width (`|k - q| <= window`, sa3jax/band_attention.py:110).
 *   q_dyt, k_dyt : 1 + 2*D floats each: [alpha, gamma[0..D), beta[0..D)]
 *   cos, sin     : (S, half) floats from hb_rope_tables (ignored when half == 0)
 *   dtype        : HB_BF16, HB_F16 or HB_F32;  D: 64 or 128;  0 <= half <= D/2 with half % 8 == 0;  window >= 0
 *   workspace    : >= hb_band_workspace_size(dtype, B, S, H, D, half, window) bytes, 256-byte aligned; that size
 *                  is 0 (and workspace may be NULL) for 16-bit inputs with D = 64 and window <= 128, which run
 *                  without one. For fp32 the workspace is optional: given, it holds the prepared keys; NULL runs the
 *                  kernel that prepares each query block's key window itself. Otherwise it holds the prepared keys
 *                  for the duration of the call.
 * Kernels: 16-bit inputs with D = 64 and window <= 128 run one streaming kernel; other 16-bit shapes, and fp32 with
 * a workspace, run a key preparation kernel and an attention kernel over the workspace; fp32 without one runs one
 * kernel. */
size_t hb_band_workspace_size(int dtype, int B, int S, int H, int D, int half, int window);
int hb_band_validate(int dtype, int64_t row_stride, int B, int S, int H, int D, int half, int window);
int hb_band_diffattn(hipStream_t stream, const void* qkv, int dtype, int64_t row_stride,
                     const float* q_dyt, const float* k_dyt, const float* cos, const float* sin, int half,
                     int window, const float* lam, void* out, int B, int S, int H, int D, void* workspace,
                     size_t workspace_bytes);

/* ---- DiT differential cross-attention -------------------------------------------------------------------
 * Replaces the XLA chain of dit._cross_attention (sa3jax/dit.py:203-215) with its hoisted context K/V
 * (dit._cross_kv, sa3jax/dit.py:274-284). Per (batch b, head h):
 *   q, q_diff <- RMSNorm(x; q_weight, eps) of the block's to_q output rows, q at section 0, q_diff at section 1
 *                (a row is [q | q_diff], sa3jax/dit.py:207-209);
 *   k, k_diff <- RMSNorm(x; k_weight, eps), v <- x, of the context's to_kv output rows (a row is
 *                [k | k_diff | v], sa3jax/dit.py:279-281);
 *   out = softmax(q k^T / sqrt(D)) v - lam[h] * softmax(q_diff k_diff^T / sqrt(D)) v   (sa3jax/dit.py:131-147),
 * over all Nk context keys: no RoPE and no mask (sa3jax/dit.py:204-205, 214-215).
 *   q      : (B, L, >= 2*H*D) with row stride `row_stride` (a multiple of 8), 16-byte aligned
 *   kv     : (B, Nk, >= 3*H*D) with row stride `row_stride` (a multiple of 8), 16-byte aligned
 *   dtype  : HB_BF16, HB_F16 or HB_F32 (of q, kv and out);  D: 64 or 128;  eps >= 0
 *   workspace : >= hb_cross_workspace_size(dtype, B, Nk, H, D) bytes, 256-byte aligned.
 * hb_cross_prep writes the prepared k, k_diff and v of the context into the workspace; hb_cross_attend reads
 * them, for as many query sets as the caller has (the reference computes them once per clip and reuses them in
 * every sampler step). k_weight is passed to hb_cross_attend too: it bounds the logits for the softmax. */
size_t hb_cross_workspace_size(int dtype, int B, int Nk, int H, int D);
int hb_cross_validate(int dtype, int64_t q_row_stride, int64_t kv_row_stride, int B, int L, int Nk, int H, int D,
                      float eps);
int hb_cross_prep(hipStream_t stream, const void* kv, int dtype, int64_t row_stride, const float* k_weight, int B,
                  int Nk, int H, int D, float eps, void* workspace, size_t workspace_bytes);
int hb_cross_attend(hipStream_t stream, const void* q, int dtype, int64_t row_stride, const float* q_weight,
                    const float* k_weight, const float* lam, void* out, int B, int L, int Nk, int H, int D, float eps,
                    const void* workspace, size_t workspace_bytes);

/* ---- SAME-L decoder block: the elementwise steps around the GEMMs ---------------------------------------
 * Replace the XLA chain of same_l._block between its GEMMs (sa3jax/same_l.py:186-192).
 *   hb_dyt : out[n, c] = cast(gamma[c] * tanh(alpha * x[n, c]) + beta[c]), computed in fp32 as same_l._dyt
 *            (sa3jax/same_l.py:58-69) and cast back to `dtype` before the next GEMM (sa3jax/same_l.py:191-192);
 *            `dyt` = [alpha, gamma[0..C), beta[0..C)].
 *   hb_glu : out[n, f] = value * act(gate) with [value | gate] = [proj[n, 0:F] | proj[n, F:2F]]
 *            (same_l._feed_forward, sa3jax/same_l.py:172-183); act = SiLU(gate) = gate * sigmoid(gate), or
 *            sin(pi * gate) when `sinusoidal` != 0. For bf16 and half the intermediate arrays of the XLA chain are
 *            rounded to the compute dtype where it holds them (the sigmoid and the SiLU; pi, pi * gate and the sine).
 *            `bias` (2F floats holding values of the compute dtype, or NULL) is the glu_proj layer's bias: proj
 *            holds the bare matmul and the bias is added first, rounded to the compute dtype as same_l._linear
 *            holds it.
 *   x, proj, out : N rows with row strides in elements (multiples of 8 for bf16 and half, 4 for fp32), 16-byte
 *                  aligned; C and F multiples of 8 (bf16, half) or 4 (fp32);  dtype: HB_BF16, HB_F16 or HB_F32 (input
 *                  and output). out shares no element with the input (HB_ERR_STRIDE otherwise; column slices of one
 *                  wider buffer that interleave without sharing elements are fine). */
int hb_dyt(hipStream_t stream, const void* x, int dtype, int64_t x_row_stride, const float* dyt, void* out,
           int64_t out_row_stride, int64_t N, int C);
int hb_glu(hipStream_t stream, const void* proj, int dtype, int64_t proj_row_stride, const float* bias,
           int sinusoidal, void* out, int64_t out_row_stride, int64_t N, int F);

/*   hb_residual_dyt : out_h = h + (x + bias), the residual adds of same_l._block (sa3jax/same_l.py:191, 192) after
 *                     the projection's bias add (same_l._linear), each sum rounded to the compute dtype; `bias` (C
 *                     floats holding values of the compute dtype) may be NULL. With `dyt` (packed as for hb_dyt) also
 *                     out_y = cast(DyT(out_h)), the input of the next GEMM (ff_norm, or the next block's pre_norm);
 *                     `dyt` and `out_y` are both given or both NULL. out_h may be h itself (same row stride) and
 *                     otherwise shares no element with h or x; out_y shares none with h, x or out_h. out_h and out_y
 *                     share `out_row_stride`. One pass where the XLA chain makes two or three. */
int hb_residual_dyt(hipStream_t stream, const void* h, int dtype, int64_t h_row_stride, const void* x,
                    int64_t x_row_stride, const float* bias, const float* dyt, void* out_h, void* out_y,
                    int64_t out_row_stride, int64_t N, int C);

/* ---- DiT block: the elementwise steps around the GEMMs and attention calls ---------------------------------
 * Replace the array operations of dit._block between its matmuls (sa3jax/dit.py:224-251).
 *   hb_rms_modulate   : y = cast(x * rsqrt(mean(x^2) + eps) * weight), the block RMSNorm (sa3jax/dit.py:44-57:
 *                       fp32 mean of squares, `weight` applied in fp32, cast back); with `scale` and `shift` (both
 *                       or neither) then out = y * (1 + scale) + shift, the adaLN modulation (dit.py:231-233,
 *                       246-247), each step rounded to the compute dtype; without them out = y (dit.py:236).
 *                       scale, shift: one row of C values per batch, `mod_batch_stride` elements apart; row n of x
 *                       belongs to batch n / rows_per_batch. weight: C floats.
 *   hb_gated_residual : out = h + (x + x_bias) * sigmoid(1 - gate) (dit.py:234, 249-251; x_bias is proj_out's bias,
 *                       dit.py:221), each step rounded to the compute dtype; without `gate` out = h + (x + x_bias);
 *                       without `x_bias` the bias step is skipped; with `local` the constant local embedding is
 *                       then added to the rows whose token index n % rows_per_batch is >= `memory` (dit.py:237-241).
 *                       gate: one row of C values per batch, `gate_batch_stride` elements apart; x_bias, local: C
 *                       values.
 *   All tensors are of `dtype` (HB_BF16, HB_F16 or HB_F32) except `weight`; row strides in elements, multiples of
 *   8 (bf16, half) or 4 (fp32); every pointer 16-byte aligned; C a multiple of 8 (bf16, half) or 4 (fp32). The
 *   row outputs (out; out_h and out_y) share no element with the row inputs (x; h and x) or with each other
 *   (HB_ERR_STRIDE otherwise). */
int hb_rms_modulate(hipStream_t stream, const void* x, int dtype, int64_t x_row_stride, const float* weight,
                    float eps, const void* scale, const void* shift, int64_t mod_batch_stride, int rows_per_batch,
                    void* out, int64_t out_row_stride, int64_t N, int C);
int hb_gated_residual(hipStream_t stream, const void* h, int dtype, int64_t h_row_stride, const void* x,
                      int64_t x_row_stride, const void* x_bias, const void* gate, int64_t gate_batch_stride,
                      const void* local, int memory, int rows_per_batch, void* out, int64_t out_row_stride,
                      int64_t N, int C);
/*   hb_residual_rms   : hb_gated_residual into out_h, then hb_rms_modulate of out_h into out_y, in one pass that
 *                       holds the row in registers (C <= 2048); out_h and out_y
 *                       share out_row_stride. The block's three residuals each feed a norm (dit.py:234-236,
 *                       237-247, and 249-251 into the next block's 231-233). */
int hb_residual_rms(hipStream_t stream, const void* h, int dtype, int64_t h_row_stride, const void* x,
                    int64_t x_row_stride, const void* x_bias, const void* gate, int64_t gate_batch_stride,
                    const void* local, int memory, const float* weight, float eps, const void* scale,
                    const void* shift, int64_t mod_batch_stride, int rows_per_batch, void* out_h, void* out_y,
                    int64_t out_row_stride, int64_t N, int C);

#ifdef __cplusplus
}
#endif

#endif /* HUMMINGBIRD_AMD_H */
