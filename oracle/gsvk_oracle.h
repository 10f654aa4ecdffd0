/*
 * gsvk_oracle.h — CPU restatement of the reference's fused-layer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. The HIP kernels are compared against these results, and this is the
 * timed CPU baseline; the product library never links, loads or calls it. Only tests/, the smoke check
 * and the benchmark's CPU-baseline leg may use it.
 *
 * Each function follows the reference's operation order (cited per function in gsvk_oracle.c).
 * Contraction: the reference is built by AppleClang with its default -ffp-contract=on, which fuses
 * `a*b + c` / `c - a*b` written in ONE expression into an fma; those places are written here with
 * an explicit fma/fmaf and the file is compiled with -ffp-contract=off so nothing else is fused.
 * Storage: dtype 0 = f32, 1 = f16, 2 = bf16 (same values as gsvk_dtype); 16-bit values are
 * upcast exactly and results are rounded to nearest even once, in software.
 */
#ifndef GSVK_ORACLE_H
#define GSVK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* conversions (accel.cpp:10-23 exact upcast; gemv_fmlal.cpp:23-35 RNE downcast) */
float oracle_h2f(uint16_t h);
uint16_t oracle_f2h(float f);
float oracle_bf2f(uint16_t h);
uint16_t oracle_f2bf(float f);
void oracle_to_f32(int dtype, const void* src, float* dst, size_t n);
void oracle_from_f32(int dtype, const float* src, void* dst, size_t n);

/* a1: kern::layernorm on one fp32 row (kern.cpp:27-59) */
void oracle_layernorm_row(const float* x, const float* g, const float* b, float* y, size_t n,
                          double eps);
/* a3: bert::LayerNorm1D::forward on one row, two-pass fp32 (bert_ops.hpp:269-285) */
void oracle_layernorm1d_row(float* r, const float* g, const float* b, size_t n, float eps);

/* a1+a2 (+a3): h = (x + bias) + residual, then mode 0 = kern::layernorm, 1 = LayerNorm1D.
 * bias / residual / gamma / beta may be NULL. */
int oracle_add_layernorm(int dtype, const void* x, const float* bias, const void* residual,
                         const float* gamma, const float* beta, void* y, size_t rows, size_t n,
                         size_t ld, double eps, int mode);

/* a4/a5/a7: y = act(x + bias) over rows; act as gsvk_act (0 none, 1 relu, 2 gelu, 3 leaky) */
int oracle_bias_act(int dtype, int act, const void* x, const float* bias, void* y, size_t rows,
                    size_t n, size_t ld, float slope);
/* kern::relu over a flat buffer (kern.cpp:85-91): 4-wide vmaxq body, scalar tail */
void oracle_relu(const float* x, float* y, size_t n);
float oracle_gelu_erf(float x);

/* a6: HuBERT GroupNorm(groups = C) + GELU (hubert.cpp:487-503) */
int oracle_groupnorm_gelu(int dtype, const void* x, const float* gamma, const float* beta, void* y,
                          size_t channels, size_t T, size_t ld, double eps, int apply_gelu);

/* a7: leaky_relu_io / leaky_relu_write (nn_ops.hpp:48-74) */
int oracle_leaky_relu(int dtype, const void* x, void* y, size_t n, float slope);
/* a8 (+a7): add_inplace then leaky_relu_write (nn_ops.hpp:77-83; dec.hpp:322-326) */
int oracle_resblock_add_lrelu(int dtype, void* cur, const void* t_b, void* t_in, size_t n,
                              float slope);
/* a9 (+a7): mul_write / add_scaled_inplace over branches, then leaky_relu_io (dec.hpp:326-336, 284) */
int oracle_resblock_branch_mean(int dtype, const void* const* cur, const void* const* t_b,
                                int nbranch, void* out, size_t n, int apply_lrelu, float slope);
/* add_scaled_inplace / mul_write (nn_ops.hpp:86-105) */
int oracle_scaled_add(int dtype, const void* acc, const void* src, void* out, size_t n,
                      float scale);

/* Decode GEMV: gemv_f16x_fmlal (x rounded to fp16: x_dtype 1, or 0 with round_x) or
 * gemv_f16w_f32acc (x_dtype 0, round_x 0), then bias, act (gsvk_act), residual, per row. */
int oracle_gemv_f16w(int x_dtype, int round_x, const void* x, size_t ldx, const uint16_t* w,
                     const float* bias, int act, float slope, const void* residual, int y_dtype,
                     void* y, size_t ldy, size_t rows, size_t out, size_t in);

/* SoVITS Conv1d (conv1d.hpp:155-196) + ResBlock epilogue epi (0 bias, 1 + leaky_relu_io,
 * 2 cur += y then y = lrelu(cur), 3 cur += y). x [cin, T] (stride ldx), w [cout][cin][k] fp16 bits,
 * bias [cout] fp32 or NULL, cur / y [cout, T] (strides ldc / ldy), storage dtype for x / cur / y. */
int oracle_conv1d(int dtype, const void* x, size_t ldx, const uint16_t* w, const float* bias, int epi,
                  float slope, void* cur, size_t ldc, void* y, size_t ldy, size_t cin, size_t cout,
                  size_t T, size_t k, size_t dil);

/* SoVITS ConvTranspose1d: w [cin][cout][k] fp16 bits, stride u, pad (k-u)/2, output [cout][T u]
 * (rows ldy / ldc), the reference's per-tap GEMM + scatter order, bias last, then epi as conv1d. */
int oracle_convt1d(int dtype, const void* x, size_t ldx, const uint16_t* w, const float* bias,
                   int epi, float slope, void* cur, size_t ldc, void* y, size_t ldy, size_t cin,
                   size_t cout, size_t T, size_t k, size_t u);

/* Decode attention: KV append at pos[b] and single-query SDPA over keys 0..pos[b] per head
 * (t2s_engine.cpp:1051-1087). kv_dtype 0 = fp32 cache, 1 = fp16 cache. Caches [B][max_len][H*HD];
 * qkv rows [q | k | v] fp32 with stride ldq; out [B][H*HD] fp32 with stride ldo (NaN rows for a
 * position outside [0, max_len)). scale = 1 / sqrtf(HD). */
int oracle_decode_attention(int kv_dtype, const float* qkv, size_t ldq, void* kcache, void* vcache,
                            size_t max_len, const int64_t* pos, float* out, size_t ldo, size_t B,
                            size_t H, size_t HD);
/* kern::softmax on one row (kern.cpp:62-74) */
void oracle_softmax(const float* x, float* y, size_t n);

/* a10: T2SEngine::pe_row (t2s_engine.cpp:711-720) and the gather + alpha*PE loops
 * (t2s_engine.cpp:1774-1786, 1866-1869). index_type 0 = int64, 1 = int32. Returns the number of
 * rows whose id / position was out of range (those rows are NaN, as the GPU writes them). */
void oracle_pe_row(float* pe, size_t pos, size_t D);
long oracle_embed_pe(int out_dtype, int table_dtype, int index_type, const void* table,
                     size_t vocab, const void* ids, const int64_t* pos, int64_t pos0,
                     const float* pe, size_t max_pos, float alpha, const void* mm,
                     const float* bias, void* out, size_t rows, size_t D);

/* The epilogue part of one T2S decode step for B sequences (gsvk_t2s.h order), with the B rows
 * split over `threads` std-thread-like row bands (each band runs the whole row-local chain).
 * Per-layer arrays hold `layers` pointers. dtype: activation storage. */
int oracle_t2s_step(int dtype, size_t B, size_t D, size_t FF, size_t layers, double eps,
                    const void* table, int table_dtype, size_t vocab, const int64_t* ids,
                    const int64_t* pos, const float* pe, size_t max_pos, float alpha, void* x,
                    void* h, const void* const* attn_out, const float* const* bout,
                    const float* const* n1g, const float* const* n1b, void* const* ff,
                    const float* const* b1, const void* const* ffn_out, const float* const* b2,
                    const float* const* n2g, const float* const* n2b, int threads);

#ifdef __cplusplus
}
#endif

#endif
