/*
 * gsvk.h — C ABI of the MI355X (gfx950) fused layer kernels for GPT-SoVITS-native.
 *
 * Every entry point enqueues work on a HIP stream and returns without waiting. Pointers named
 * "device" must be device-accessible memory (hipMalloc or equivalent); all sizes are element counts.
 * The stream argument is a hipStream_t passed as void* (NULL = the legacy default stream), so the
 * header needs no HIP include and binds directly from ctypes / cgo / JNI.
 *
 * Status: every function returns GSVK_OK (0) or a negative gsvk_status. Argument checks happen on the
 * host before anything is launched, so a rejected call leaves the stream untouched.
 *
 * Storage vs math: activations are stored as f32, f16 or bf16 (gsvk_dtype); all arithmetic is fp32
 * (fp64 where the reference finalizes in double) and results are rounded to the storage type once,
 * round-to-nearest-even. Per-column parameters (gamma, beta, bias) and the PE table are always fp32,
 * as the reference keeps them (t2s_engine.cpp:615-626, hubert.cpp:135-139).
 *
 * Aliasing: y == x (exact same pointer, same layout) is allowed wherever the reference calls the
 * primitive in place; any other overlap between an output and an input is rejected (GSVK_E_ALIAS).
 */
#ifndef GSVK_H
#define GSVK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum gsvk_dtype {
  GSVK_F32 = 0,
  GSVK_F16 = 1,
  GSVK_BF16 = 2,
} gsvk_dtype;

typedef enum gsvk_index_type {
  GSVK_I64 = 0, /* int64_t ids, as T2SEngine::generate takes them (t2s_engine.hpp:114-115) */
  GSVK_I32 = 1, /* int32_t ids, as the sampler returns them (t2s_engine.hpp:168-175) */
} gsvk_index_type;

typedef enum gsvk_act {
  GSVK_ACT_NONE = 0,       /* y = x + bias                                         */
  GSVK_ACT_RELU = 1,       /* kern::relu after the bias pass (kern.cpp:85-91)      */
  GSVK_ACT_GELU_ERF = 2,   /* bert::gelu_erf / HubertEngine::gelu (bert_ops.hpp:25-27) */
  GSVK_ACT_LEAKY_RELU = 3, /* sovits::leaky_relu_write semantics (nn_ops.hpp:64-74) */
} gsvk_act;

typedef enum gsvk_conv_epi {
  GSVK_CONV_EPI_BIAS = 0,       /* y = conv + bias                           (conv1d.hpp:193-202) */
  GSVK_CONV_EPI_LRELU = 1,      /* y = lrelu(conv + bias)         conv1 then leaky_relu_io (dec.hpp:323-324) */
  GSVK_CONV_EPI_RES_LRELU = 2,  /* cur += conv + bias; y = lrelu(cur)  conv2, add_inplace, next
                                   leaky_relu_write (dec.hpp:325-326, 322) */
  GSVK_CONV_EPI_RES = 3,        /* cur += conv + bias (y unused)      a branch's last conv2 (dec.hpp:325-326) */
  GSVK_CONV_EPI_DUAL = 4,       /* y = conv + bias and cur = lrelu(y)  upsampler + the first pair's
                                   leaky_relu_write (dec.hpp:285, 322) */
  GSVK_CONV_EPI_TANH = 5,       /* y = tanh(conv + bias)              conv_post then tanh (dec.hpp:343-344) */
  /* Flag OR-ed into epi: the convolution reads lrelu(x, slope) instead of x (the same slope as
     the epilogue's), i.e. leaky_relu_write into t_in then the conv (dec.hpp:322-323) in one pass
     without t_in. */
  GSVK_CONV_X_LRELU = 0x100,
} gsvk_conv_epi;

typedef enum gsvk_status {
  GSVK_OK = 0,
  GSVK_E_NULL = -1,   /* a required pointer is NULL                                  */
  GSVK_E_SIZE = -2,   /* zero or out-of-range size, or ld < n                         */
  GSVK_E_DTYPE = -3,  /* unknown dtype / index type / activation                      */
  GSVK_E_ALIAS = -4,  /* output overlaps an input other than the allowed exact alias  */
  GSVK_E_ARG = -5,    /* other invalid argument (negative or non-finite eps, odd D, …) */
  GSVK_E_HIP = -6,    /* the HIP runtime reported an error at launch                  */
  GSVK_E_FORMAT = -7, /* malformed .gsv container (gsvk_gsv.h)                         */
  GSVK_E_IO = -8,     /* a file could not be opened or mapped                          */
} gsvk_status;

/* Library identification and error text (host only, no GPU needed). */
const char* gsvk_version(void);
const char* gsvk_status_string(int status);

/* ------------------------------------------------------------------------------------------------
 * Residual add + LayerNorm over rows.
 *   h[r,c] = (x[r,c] + bias[c]) + residual[r,c]        (bias / residual may be NULL)
 *   y[r,c] = (h - mean_r) * rstd_r * gamma[c] + beta[c] (gamma / beta may be NULL: 1 / 0)
 * mean and biased variance per row; rstd = 1/sqrt(var + eps) finalized in double.
 * Replaces gsv::kern::layernorm(const float* x, const float* g, const float* b, float* y, size_t n,
 * double eps) (src/kern/kern.hpp:25, kern.cpp:27-59) called once per row, together with the residual
 * and bias loops that feed it: T2S prefill t2s_engine.cpp:980-987 and 1018-1025, decode 1096-1098
 * and 1117-1119, HuBERT hubert.cpp:697-703 and 725-731, and bert::LayerNorm1D::forward
 * (src/bert/bert_ops.hpp:261-286, eps 1e-12) after the residual add at bert_ops.hpp:389 and 397.
 * Layout: row-major [rows, n] with row stride ld >= n (elements) shared by x, residual and y.
 * y == x and y == residual are allowed (in place).
 * ------------------------------------------------------------------------------------------------ */
int gsvk_add_layernorm(int dtype, const void* x, const float* bias, const void* residual,
                       const float* gamma, const float* beta, void* y, size_t rows, size_t n,
                       size_t ld, double eps, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Bias + activation epilogue over rows: y[r,c] = act(x[r,c] + bias[c]).
 * Replaces the bias loop + gsv::kern::relu(const float* x, float* y, size_t n) (kern.hpp:33,
 * kern.cpp:85-91; t2s_engine.cpp:995-996, 1111-1112), the Linear bias + bert::gelu_erf pass
 * (bert_ops.hpp:25-27, 255-257, 394), and HubertEngine::gelu after the f1 bias (hubert.cpp:233-236,
 * 714-716). bias may be NULL. slope is used by GSVK_ACT_LEAKY_RELU only. y == x allowed.
 * ReLU keeps NaN and maps -0 to +0 (vmaxq_f32 semantics); LeakyReLU keeps -0 and NaN.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_bias_act(int dtype, int act, const void* x, const float* bias, void* y, size_t rows,
                  size_t n, size_t ld, float slope, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Batched decode GEMV with fp16 weights and fp32 accumulation, epilogue fused into the store.
 *   xr[k]  = x[r, k] as fp32; with x_dtype F32 and round_x != 0 it is first rounded to fp16
 *   acc    = sum_k float(w[n, k]) * xr[k]                       (fp32 sum of the products)
 *   v      = act(acc + bias[n])                                 (no add when bias is NULL)
 *   y[r,n] = residual ? v + residual[r, n] : v                  (rounded once to y_dtype)
 * for rows r < rows (B sequences, one GEMV each), n < out, k < in.
 * Replaces kern::gemv_f16w_f32acc(const uint16_t* w, const float* x, float* y, size_t out,
 * size_t in) (src/kern/gemv.cpp:112-127; x_dtype F32, round_x = 0) and T2SEngine::gemv_fmlal ->
 * kern::gemv_f16x_fmlal (t2s_engine.cpp:696-700, src/kern/gemv_fmlal.cpp:113-132; x rounded to
 * fp16: x_dtype F16, or F32 with round_x = 1), each called once per sequence, together with the
 * loops after them in block_decode_impl: QKV + bias (t2s_engine.cpp:1044-1049), out-proj + bias +
 * residual (1090-1095), W1 + bias + ReLU (1105-1112), W2 + bias + residual (1113-1116).
 * act is a gsvk_act (slope for LeakyReLU); bias, residual may be NULL.
 * Layout: x [rows, in] with row stride ldx (x_dtype F32 or F16); w [out, in] row-major fp16 bit
 * patterns (the .gsv weight layout); residual and y [rows, out] with row stride ldy (y_dtype).
 * residual == y is allowed (in-place accumulate); y must not overlap x, w or bias.
 * The sum is formed in a different order from the reference (matrix-core tiles, then a fixed-order
 * sum of per-wave partials): results agree within fp32 accumulation noise,
 * |y - ref| <= 1e-5 * max(1, max_n |ref[r, n]|) (the reference's own NEON-vs-scalar rule,
 * tests/test_kern.cpp:111-118). Deterministic: the same inputs give the same bits on every call.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_gemv_f16w(int x_dtype, int round_x, const void* x, size_t ldx, const uint16_t* w,
                   const float* bias, int act, float slope, const void* residual, int y_dtype,
                   void* y, size_t ldy, size_t rows, size_t out, size_t in, void* stream);

/* ------------------------------------------------------------------------------------------------
 * LayerNorm folded into the GEMV that consumes it:
 *   h[r, :] = LN(z[r, :]; gamma, beta, eps)      as gsvk_add_layernorm(x_dtype, z, NULL, NULL,
 *                                                gamma, beta, h, rows, in, ., eps)
 *   y       = gsvk_gemv_f16w(x_dtype, round_x, h, ...)   on that h, with the same bits
 * in one launch: every workgroup forms its rows' statistics from the activations it has loaded
 * for the products, normalizes them as it stages them, and the first column block stores h. The
 * statistics are summed in another order than gsvk_add_layernorm's: h agrees with it within the
 * LayerNorm tolerance, not bit for bit. No reference function has this form; it is
 * the post-LN of block_decode_impl followed by the GEMV that reads it: norm1 then W1
 * (t2s_engine.cpp:1097-1110), norm2 then the next layer's QKV (1119, 1044) or the logits.
 * The fused form needs every wave of the GEMV's launch plan to hold all its k blocks at once
 * (in <= 128, 193..256, 449..512 or 961..1024 at decode batch sizes), in % 8 == 0 and 16-byte
 * aligned rows and vectors; otherwise the call runs the two launches, with their exact results
 * (then ldz == ldh is required: E_ARG).
 * h is required and overlaps none of z, w, gamma, beta, y; y overlaps none of z, h, w, bias;
 * residual == y is allowed. Same tolerance and determinism as gsvk_gemv_f16w.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_gemv_f16w_ln(int x_dtype, int round_x, const void* z, size_t ldz, const float* gamma,
                      const float* beta, double eps, void* h, size_t ldh, const uint16_t* w,
                      const float* bias, int act, float slope, const void* residual, int y_dtype,
                      void* y, size_t ldy, size_t rows, size_t out, size_t in, void* stream);

/* ------------------------------------------------------------------------------------------------
 * T2S decode attention with the KV append, B sequences at once.
 *   for each sequence b, p = pos[b]:
 *     k_cache[b, p, :] = k, v_cache[b, p, :] = v      (k, v = qkv[b, D:2D], qkv[b, 2D:3D], rounded
 *                                                       once to kv_dtype)
 *     for each head h:  s_j = (q_h . K[b, j, h]) * (1 / sqrtf(head_dim)),  j = 0 .. p
 *                       out[b, h*HD : (h+1)*HD] = sum_j softmax(s)_j V[b, j, h]
 * Replaces the append and the single-query SDPA of T2SEngine::block_decode_impl
 * (t2s_engine.cpp:1051-1087: kern::f32_to_f16 into k16 / v16 or the fp32 memcpy, then per head
 * ar_neon::dot_f16kv / dot_f32, kern::softmax (kern.cpp:62-74) and ar_neon::accum_f16kv /
 * accum_f32, t2s_engine.cpp:40-145), for every sequence in one call.
 * Layout: qkv [batch, ldq >= 3D] fp32 as the QKV GEMV writes it (q | k | v, bias included);
 * k_cache / v_cache [batch, max_len, D] of kv_dtype, token-major (row j holds every head, as the
 * reference's k16[j * D + h * HD + e]); out [batch, ldo >= D] of out_dtype. D = heads * head_dim
 * <= 512, head_dim a multiple of 8 with head_dim / 8 a power of two; rows 16-byte aligned.
 * len_bound: a host-side upper bound of pos[b] + 1 (e.g. the longest sequence so far) that sets how
 * many key chunks a sequence is split into (0 = max_len); results agree within the tolerance below
 * whatever its value (the partition of the keys, so the rounding, follows it). With more
 * than one chunk the partial states go through `workspace` (gsvk_decode_attention_workspace_bytes
 * bytes, 16-byte aligned; no initialisation needed); with a NULL or smaller workspace every sequence
 * runs as one chunk. Cache rows at and past pos[b] may hold any bits (stale, Inf, NaN): none of
 * them enters the result. A position outside [0, max_len) (undefined in the reference) writes a
 * NaN row, leaves the caches untouched and stores 1 into *err when err != NULL.
 * The softmax is formed online (running maximum, rescaled sums) in another order than the
 * reference's; results agree within fp32 rounding: |out - ref| <= 1e-5 * max(1, max |v|).
 * ------------------------------------------------------------------------------------------------ */
int gsvk_decode_attention(int kv_dtype, int out_dtype, const float* qkv, size_t ldq, void* k_cache,
                          void* v_cache, size_t max_len, const int64_t* pos, void* out, size_t ldo,
                          size_t batch, size_t heads, size_t head_dim, size_t len_bound,
                          void* workspace, size_t workspace_bytes, int32_t* err, void* stream);
/* Workspace bytes gsvk_decode_attention uses for these sizes (0: none). Host only. len_bound 0:
 * the size for the longest context, an upper bound of what the call needs for any max_len. */
size_t gsvk_decode_attention_workspace_bytes(size_t batch, size_t heads, size_t head_dim,
                                             size_t len_bound);
/* gsvk_decode_attention without a workspace argument, for callers that cannot allocate (code under
 * HIP graph capture, serving loops that forbid hipMalloc). No counterpart in the reference. The
 * key-chunk states live in a 4 MiB device array owned by the library, one copy per GPU, kept until
 * the process ends; the call allocates nothing. Every call on a GPU shares that copy, so calls in
 * flight at once on one GPU (different streams) race on it. Same arguments (minus the workspace)
 * and the same bits as gsvk_decode_attention with a workspace of
 * gsvk_decode_attention_workspace_bytes. GSVK_E_SIZE, before any launch, when the chunk states
 * would exceed 4 MiB (batch x chunks x 3 KiB, 1365 states: on a 256-CU MI355X every batch of up to
 * 256 sequences fits at any length, and up to 682 sequences at contexts of at most 256 keys);
 * GSVK_E_HIP when the array's device address cannot be looked up. The lookup runs on the first
 * call on each device (hipGetSymbolAddress, not a stream operation); a caller that captures every
 * call into a graph makes one ordinary call on that device before capturing. */
int gsvk_decode_attention_noalloc(int kv_dtype, int out_dtype, const float* qkv, size_t ldq,
                                  void* k_cache, void* v_cache, size_t max_len, const int64_t* pos,
                                  void* out, size_t ldo, size_t batch, size_t heads,
                                  size_t head_dim, size_t len_bound, int32_t* err, void* stream);

/* ------------------------------------------------------------------------------------------------
 * SoVITS Conv1d, same padding with dilation, and the ResBlock passes that follow it.
 *   v[o, t] = bias[o] + sum_{i < c_in, kk < k} w[o, i, kk] * x[i, t + kk*dilation - pad],
 *   pad = (k - 1) * dilation / 2, x = 0 outside [0, T); the output has T columns.
 *   epi (gsvk_conv_epi): BIAS y = v; LRELU y = lrelu(v, slope); RES_LRELU cur = r + v, y =
 *   lrelu(cur, slope) (from the fp32 sum); RES cur = r + v (y may be NULL); DUAL y = v, cur =
 *   lrelu(v, slope); TANH y = tanhf(v). With GSVK_CONV_X_LRELU OR-ed into epi, every x value is
 *   replaced by lrelu(x, slope) as it is read (x itself unchanged; the sum then runs on that value:
 *   as an fp32 value for F32, rounded to fp16 with round_x or F16 storage, as a stored lrelu(x)
 *   would be).
 *   For RES_LRELU / RES the residual r is read from `res`
 *   (row stride ldc) or, when res is NULL or equal to cur, from cur itself (in place): a branch's
 *   first pair can then add onto the stage input without copying it into cur first.
 * Replaces Conv1d::forward (src/sovits/conv1d.hpp:109-194: im2col, sgemm, add_bias) and, fused
 * into its store, the ResBlock passes after each convolution in Generator::forward
 * (src/sovits/dec.hpp:322-326: leaky_relu_io after conv1, add_inplace after conv2 and the next
 * pair's leaky_relu_write).
 * Layout: channel-major [channels, T] rows with strides ldx, ldc, ldy >= T; x, cur, y of dtype
 * (F32 or F16); bias fp32 [c_out] or NULL (conv_post has none, conv1d.hpp:82-88); w_packed from
 * gsvk_conv1d_pack, 16-byte aligned. dtype F32 keeps the fp32 activations as a hi/lo pair of fp16
 * halves, x to about 2^-22 relative, not exactly (round_x = 0, the reference's sgemm path;
 * |x| < 65504), or rounds them to fp16 (round_x = 1, as the reference's AMX path packs them,
 * conv1d.hpp:130-151); F16 storage rounds each output once.
 * (k - 1) * dilation <= 256; 32 rows of x and the packed weights each under 2 GiB (GSVK_E_SIZE
 * otherwise). y and cur must not overlap x, the weights, the bias or each other
 * (the reference's in-place x == y goes through a copy; here the caller keeps them apart); res may
 * equal cur but must not otherwise overlap an output.
 * The sum is formed in the matrix cores' order: |y - ref| <= 1e-5 * max(1, max_t |ref[o, t]|)
 * against the fp32 reference (fp32 storage). Deterministic.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_conv1d(int dtype, int round_x, const void* x, size_t ldx, const uint16_t* w_packed,
                const float* bias, int epi, float slope, void* cur, const void* res, size_t ldc,
                void* y, size_t ldy, size_t c_in, size_t c_out, size_t T, size_t k,
                size_t dilation, void* stream);
/* Elements (uint16_t) of the packed weights of a [c_out, c_in, k] filter bank (0 for a zero size).
 * Host only. */
size_t gsvk_conv1d_packed_elems(size_t c_out, size_t c_in, size_t k);
/* Pack a torch-layout [c_out, c_in, k] fp16 filter bank (the .gsv layout; Conv1d::load,
 * conv1d.hpp:74-107, packs its AMX panel once the same way) into the layout gsvk_conv1d reads:
 * [c_in / 32][k][c_out padded to 64][32], zero padded. Runs on the GPU, once per model load. */
int gsvk_conv1d_pack(const uint16_t* w, size_t c_out, size_t c_in, size_t k, uint16_t* w_packed,
                     size_t packed_elems, void* stream);

/* ------------------------------------------------------------------------------------------------
 * SoVITS ConvTranspose1d (the upsampler), stride u, pad_t = (k - u) / 2, output length T * u:
 *   v[o, t] = bias[o] + sum over (j, d) with j*u + d - pad_t = t of sum_i w[i, o, d] * x[i, j]
 *   followed by the same epilogues as gsvk_conv1d (epi, slope, cur, res), on [c_out, T * u]
 *   outputs.
 * Replaces ConvT1d::forward (src/sovits/conv1d.hpp:250-340: one sgemm per tap d, scatter-add into
 * y at j*u + d - pad, then the bias), computed here per output phase r = (t + pad_t) mod u as a
 * short convolution over x (ceil((k - r) / u) taps), all phases in one launch.
 * Layout: x [c_in, T] (stride ldx >= T); y / cur [c_out, T * u] (strides >= T * u); bias fp32 or
 * NULL; w_packed from gsvk_convt1d_pack. Requires k >= u (the reference's pad formula) and
 * ceil(k / u) <= 65. Same dtype / round_x / aliasing rules and tolerance as gsvk_conv1d.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_convt1d(int dtype, int round_x, const void* x, size_t ldx, const uint16_t* w_packed,
                 const float* bias, int epi, float slope, void* cur, const void* res, size_t ldc,
                 void* y, size_t ldy, size_t c_in, size_t c_out, size_t T, size_t k,
                 size_t stride, void* stream);
/* Elements of the packed transposed filter bank (0 for a zero size or k < stride). Host only. */
size_t gsvk_convt1d_packed_elems(size_t c_out, size_t c_in, size_t k, size_t stride);
/* Pack a torch-layout [c_in, c_out, k] fp16 ConvTranspose1d filter bank (the .gsv layout;
 * ConvT1d::load, conv1d.hpp:219-237, re-slices it per tap the same way) for gsvk_convt1d. */
int gsvk_convt1d_pack(const uint16_t* w, size_t c_out, size_t c_in, size_t k, size_t stride,
                      uint16_t* w_packed, size_t packed_elems, void* stream);

/* ------------------------------------------------------------------------------------------------
 * GroupNorm with one group per channel, optionally followed by GELU(erf).
 *   mean_c, var_c over the T frames of channel c (biased); y = (x - mean)*rstd*gamma[c] + beta[c];
 *   y = gelu_erf(y) when apply_gelu != 0.
 * Replaces the HuBERT conv-layer-0 GroupNorm loop and the GELU pass after it
 * (src/encoder/hubert.cpp:487-503). Layout: channel-major [channels, T] with channel stride ld >= T.
 * gamma / beta may be NULL (1 / 0). y == x allowed.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_groupnorm_gelu(int dtype, const void* x, const float* gamma, const float* beta, void* y,
                        size_t channels, size_t T, size_t ld, double eps, int apply_gelu,
                        void* stream);

/* ------------------------------------------------------------------------------------------------
 * LeakyReLU over a flat buffer: y[k] = x[k] < 0 ? x[k]*slope : x[k].
 * x == y is sovits::leaky_relu_io (nn_ops.hpp:48-59); x != y is leaky_relu_write (nn_ops.hpp:64-74).
 * Call sites: Generator::forward stage entry and final slope 0.01 (dec.hpp:284, 342), ResBlock
 * pre-conv (dec.hpp:322, 324).
 * ------------------------------------------------------------------------------------------------ */
int gsvk_leaky_relu(int dtype, const void* x, void* y, size_t n, float slope, void* stream);

/* ------------------------------------------------------------------------------------------------
 * ResBlock residual step: cur[k] += t_b[k]; then, if t_in != NULL, t_in[k] = lrelu(cur[k], slope).
 * Fuses sovits::add_inplace (nn_ops.hpp:77-83; dec.hpp:326) with the next conv pair's
 * leaky_relu_write (dec.hpp:322; batched prepare hook dec.hpp:226-228).
 * cur, t_b and t_in must not overlap (the reference marks them __restrict).
 * ------------------------------------------------------------------------------------------------ */
int gsvk_resblock_add_lrelu(int dtype, void* cur, const void* t_b, void* t_in, size_t n,
                            float slope, void* stream);

/* ------------------------------------------------------------------------------------------------
 * ResBlock branch average (+ the next stage's LeakyReLU):
 *   v_j = cur[j][k] (+ t_b[j][k] when t_b != NULL and t_b[j] != NULL),  kinv = 1.f / nbranch
 *   s = v_0 * kinv;  s = s + v_j * kinv  for j = 1..nbranch-1   (multiply and add rounded separately)
 *   out[k] = apply_lrelu ? lrelu(s, slope) : s
 * Fuses the last add_inplace of each branch, sovits::mul_write / add_scaled_inplace
 * (nn_ops.hpp:86-105; dec.hpp:328-333, batched dec.hpp:247-254) and the next stage's
 * leaky_relu_io (dec.hpp:284, slope 0.1; dec.hpp:342, slope 0.01). nbranch in 1..4 (the reference
 * uses 3). out must not overlap any input.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_resblock_branch_mean(int dtype, const void* const* cur, const void* const* t_b,
                              int nbranch, void* out, size_t n, int apply_lrelu, float slope,
                              void* stream);

/* ------------------------------------------------------------------------------------------------
 * Scaled accumulate: out[k] = acc ? acc[k] + src[k]*scale : src[k]*scale (multiply and add rounded
 * separately). acc == out is sovits::add_scaled_inplace (nn_ops.hpp:86-95); acc == NULL is
 * sovits::mul_write (nn_ops.hpp:98-105). out must not overlap src; acc is either out or disjoint.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_scaled_add(int dtype, const void* acc, const void* src, void* out, size_t n, float scale,
                    void* stream);

/* ------------------------------------------------------------------------------------------------
 * fp32 -> fp16 storage: y[k] = fp16(x[k]) rounded to nearest even (subnormals kept, overflow to
 * inf, NaN stays NaN), bit-exact. Replaces kern::f32_to_f16 (src/kern/gemv_fmlal.cpp:23-35), the
 * conversion load_tensor_f16 applies to a weight stored without an fp16 copy
 * (src/sovits/sovits_types.hpp:76-87). x and y must not overlap.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_f32_to_f16(const float* x, uint16_t* y, size_t n, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Token-embedding gather fused with the scaled sinusoidal positional add, bit-exact.
 *   p = pos ? pos[r] : pos0 + r
 *   e = float(table[id_r, :])                           (exact upcast of f16 / bf16 / f32 rows)
 *   without mm:  out[r, :] = fmaf(alpha, pe[p, :], e (+ bias))                 (audio / decode)
 *   with mm:     out[r, :] = fmaf(alpha, pe[p, :], mm[r, :] + (e (+ bias)))    (text rows)
 * Replaces the T2S input rebuild loops: text rows t2s_engine.cpp:1774-1780, prompt rows 1781-1786,
 * the decode-step input 1866-1869, with the PE row of T2SEngine::pe_row (t2s_engine.cpp:711-720)
 * read from a table made by gsvk_pe_table. An id outside [0, vocab) or a position outside
 * [0, max_pos) (undefined behaviour in the reference) writes a NaN row and, when err != NULL,
 * stores 1 into *err (device int32); nothing is read out of bounds.
 * Layout: table [vocab, D] (table_dtype), pe [max_pos, D] f32, mm / out [rows, D] (out_dtype),
 * bias [D] f32 (or NULL). D must be even.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_embed_pe(int out_dtype, int table_dtype, int index_type, const void* table, size_t vocab,
                  const void* ids, const int64_t* pos, int64_t pos0, const float* pe,
                  size_t max_pos, float alpha, const void* mm, const float* bias, void* out,
                  size_t rows, size_t D, int32_t* err, void* stream);

/* ------------------------------------------------------------------------------------------------
 * The T2S prefill input xy [T + P, D] in one launch: the text rows and the prompt rows, which both
 * take positions 0, 1, ... (T2SEngine::generate, t2s_engine.cpp:1770-1786):
 *   xy[t, :]     = fmaf(alpha_text,  pe[t, :], mm[t, :] + (e_text[phones[t]] (+ bias)))  t < T
 *   xy[T + t, :] = fmaf(alpha_audio, pe[t, :], e_audio[prompt[t]])                       t < P
 * Each output row has the bits of gsvk_embed_pe with pos0 = 0 (mm / bias: the text form, as there;
 * mm may be NULL). The PE row of position t is read once for both rows. mm is the bert_proj output
 * [T, D] in out_dtype: xy itself (the reference writes it into xy first, t2s_engine.cpp:1772) or a
 * buffer that does not overlap xy. Both tables have table_dtype, phones / prompt index_type.
 * Out-of-range ids and positions >= max_pos write NaN rows and set *err, as gsvk_embed_pe.
 * D must be even and T, P at most 2^24; rows that are not 16-byte aligned, or D % 8 != 0, run as
 * two gsvk_embed_pe launches (the same results).
 * ------------------------------------------------------------------------------------------------ */
int gsvk_t2s_prefill_input(int out_dtype, int table_dtype, int index_type, const void* text_table,
                           size_t text_vocab, const void* phones, size_t T, const void* mm,
                           const float* bias, float alpha_text, const void* audio_table,
                           size_t audio_vocab, const void* prompt, size_t P, float alpha_audio,
                           const float* pe, size_t max_pos, void* xy, size_t D, int32_t* err,
                           void* stream);

/* ------------------------------------------------------------------------------------------------
 * Host helper: the sinusoidal PE table, row p = T2SEngine::pe_row(pe, p) (t2s_engine.cpp:711-720):
 *   log_inc = float(-ln(10000)/D); div = expf(float(d)*log_inc); pe[2i] = sinf(p*div),
 *   pe[2i+1] = cosf(p*div), all in fp32. host_out holds max_pos * D floats. Host memory, no GPU.
 * ------------------------------------------------------------------------------------------------ */
int gsvk_pe_table(float* host_out, size_t max_pos, size_t D);
/* One row of it: T2SEngine::pe_row(pe, pos) (t2s_engine.hpp:187) for a model of width D, into
 * host_out[0 .. D). The same values as row `pos` of gsvk_pe_table. Host memory, no GPU. */
int gsvk_pe_row(float* host_out, size_t pos, size_t D);

#ifdef __cplusplus
}
#endif

#endif /* GSVK_H */
