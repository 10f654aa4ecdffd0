/*
 * gsvk_oracle.c — CPU restatement of the reference's fused-layer arithmetic (see gsvk_oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the results the HIP kernels are compared with and the timed CPU
 * baseline. It is never linked into, loaded by or called from the product library.
 *
 * Build: gcc -O3 -mavx2 -mfma -ffp-contract=off (oracle/Makefile). With contraction off, an fma
 * happens exactly where this file writes fma()/fmaf(), which is where AppleClang's default
 * -ffp-contract=on fuses the reference's single-expression `a*b + c`.
 *
 * Pinning (what checks each function, tests/test_oracle.py):
 *   layernorm_row        reference golden tests/kern_golden/ln_*.f32 (test_kern.cpp:207-216),
 *                        float64 closed form, planted-mistake checks
 *   relu                 reference golden act_v/act_relu, bit-exact (test_kern.cpp:231-239)
 *   f16 / bf16           reference special values (test_accel.cpp:69-83), numpy float16 on all
 *                        65536 half patterns and on random floats, torch bfloat16 rounding
 *   pe_row               reference closed-form test at pos {0,1,7,166,1234} (test_ar_unit.cpp:35-52)
 *   embed_pe             alpha = 0 exact-upcast identity, exact-rational fma check
 *   layernorm1d_row      float64 closed form, gamma=1/beta=0 moments       (no reference vector)
 *   gelu_erf             float64 math.erf closed form, odd-part identity   (no reference vector)
 *   groupnorm_gelu       float64 closed form, T = 1 -> beta                (no reference vector)
 *   leaky / add / mean   exact-rational closed forms, slope identities     (no reference vector)
 *   conv1d               float64 closed form via numpy correlation, k = 1 matmul, delta inputs
 *                        give the taps, padding / dilation planted mistakes (no reference vector)
 *   decode_attention     reference softmax golden sm_x / sm_y (test_kern.cpp:219-229) for the
 *                        softmax step, float64 closed form, one-key and equal-key identities
 *   gemv_f16w            reference golden gemv_a / gemv_b (test_kern.cpp:96-120) at its own
 *                        tolerance, exact small-integer products (sum order free), fp16-rounded x
 *                        identity between the two modes, epilogue order
 * Functions marked "no reference vector" are pinned by mathematics only: the reference holds no
 * golden data for them.
 *
 * Parity unpinned at the last bit: whether the reference binary fuses embed_pe's e + alpha * pe
 * (taken here as one fmaf) and branch_mean's product and sum (taken here as two roundings) is a
 * choice of its compiler that no reference vector records; the two readings differ by at most one
 * rounding of the product per term.
 */
#include "gsvk_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------------
 * Conversions. accel::f16_to_f32 is an exact upcast (accel.cpp:10-23); kern::f32_to_f16 is the
 * hardware round-to-nearest-even (gemv_fmlal.cpp:23-35). Written from the IEEE 754 binary16 and
 * bfloat16 definitions.
 * --------------------------------------------------------------------------------------------- */

static inline uint32_t f_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bits_f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float oracle_h2f(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    const float v = (float)m * 0x1p-24f; /* subnormal or zero, exact */
    return bits_f(f_bits(v) | s);
  }
  if (e == 31) return bits_f(s | 0x7f800000u | (m << 13));
  return bits_f(s | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_f2h(float f) {
  const uint32_t u = f_bits(f);
  const uint32_t s = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(s | 0x7e00u | ((a >> 13) & 0x3ffu)); /* quiet NaN */
  if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u); /* >= 65520 rounds to infinity */
  if (a < 0x38800000u) {                                /* below 2^-14: subnormal half */
    const float t = bits_f(a) * 0x1p24f;                 /* exact: units of 2^-24 */
    return (uint16_t)(s | (uint32_t)nearbyintf(t));      /* ties to even; 1024 = min normal */
  }
  uint32_t hb = (((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13);
  const uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (hb & 1u))) ++hb; /* carry may step the exponent */
  return (uint16_t)(s | hb);
}

float oracle_bf2f(uint16_t h) { return bits_f((uint32_t)h << 16); }

uint16_t oracle_f2bf(float f) {
  const uint32_t u = f_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u; /* canonical quiet NaN */
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

void oracle_to_f32(int dtype, const void* src, float* dst, size_t n) {
  if (dtype == 0) {
    memcpy(dst, src, n * 4);
  } else {
    const uint16_t* s = (const uint16_t*)src;
    for (size_t i = 0; i < n; ++i) dst[i] = dtype == 1 ? oracle_h2f(s[i]) : oracle_bf2f(s[i]);
  }
}

void oracle_from_f32(int dtype, const float* src, void* dst, size_t n) {
  if (dtype == 0) {
    memcpy(dst, src, n * 4);
  } else {
    uint16_t* d = (uint16_t*)dst;
    for (size_t i = 0; i < n; ++i) d[i] = dtype == 1 ? oracle_f2h(src[i]) : oracle_f2bf(src[i]);
  }
}

static size_t esize(int dtype) { return dtype == 0 ? 4 : 2; }
static const void* row_ptr(const void* base, int dtype, size_t off) {
  return (const char*)base + off * esize(dtype);
}
static void* row_ptr_w(void* base, int dtype, size_t off) {
  return (char*)base + off * esize(dtype);
}

/* ---------------------------------------------------------------------------------------------
 * a1: gsv::kern::layernorm (kern.cpp:27-59).
 * NEON body over blocks of 8: lane accumulators s0/s1 (vaddq_f32) and q0/q1 (vfmaq_f32, fused),
 * horizontal vaddvq_f32 = pairwise (l0+l1)+(l2+l3), the two halves added in float and widened;
 * the tail (n % 8) accumulates in double with a contracted `sqsum += x*x`.
 * mean = float(sum/n); var = float(sqsum/n - mean*mean) contracted to one double fma; two-pass
 * double fallback when var is not >= 0; rstd = float(1/sqrt(var + eps)) in double;
 * y = (x - mean)*rstd*g + b with the final multiply-add fused.
 * --------------------------------------------------------------------------------------------- */
static inline float vaddv4(const float l[4]) { return (l[0] + l[1]) + (l[2] + l[3]); }

void oracle_layernorm_row(const float* x, const float* g, const float* b, float* y, size_t n,
                          double eps) {
  const size_t vec_end = n & ~(size_t)7;
  float s0[4] = {0, 0, 0, 0}, s1[4] = {0, 0, 0, 0}, q0[4] = {0, 0, 0, 0}, q1[4] = {0, 0, 0, 0};
  size_t i = 0;
  for (; i < vec_end; i += 8) {
    for (int k = 0; k < 4; ++k) {
      const float a = x[i + k], c = x[i + 4 + k];
      s0[k] = s0[k] + a;
      s1[k] = s1[k] + c;
      q0[k] = fmaf(a, a, q0[k]);
      q1[k] = fmaf(c, c, q1[k]);
    }
  }
  double sum = (double)(vaddv4(s0) + vaddv4(s1));
  double sqsum = (double)(vaddv4(q0) + vaddv4(q1));
  for (; i < n; ++i) {
    sum += x[i];
    sqsum = fma((double)x[i], (double)x[i], sqsum);
  }
  const double dn = (double)n;
  const float mean = (float)(sum / dn);
  float var = (float)fma(-(double)mean, (double)mean, sqsum / dn);
  if (!(var >= 0.0f)) {
    double s2 = 0;
    for (size_t j = 0; j < n; ++j) {
      const double d = (double)x[j] - mean;
      s2 = fma(d, d, s2);
    }
    var = (float)(s2 / dn);
  }
  const float rstd = (float)(1.0 / sqrt((double)var + eps));
  for (size_t j = 0; j < n; ++j) y[j] = fmaf((x[j] - mean) * rstd, g ? g[j] : 1.f, b ? b[j] : 0.f);
}

/* a3: bert::LayerNorm1D::forward (bert_ops.hpp:269-285): sequential fp32 sums, contracted
 * `var += dv*dv`, float eps, 1.f/sqrtf, fused final multiply-add. In place. */
void oracle_layernorm1d_row(float* r, const float* g, const float* b, size_t n, float eps) {
  float mean = 0.f;
  for (size_t i = 0; i < n; ++i) mean += r[i];
  mean /= (float)n;
  float var = 0.f;
  for (size_t i = 0; i < n; ++i) {
    const float dv = r[i] - mean;
    var = fmaf(dv, dv, var);
  }
  var /= (float)n;
  const float inv = 1.f / sqrtf(var + eps);
  for (size_t i = 0; i < n; ++i) r[i] = fmaf((r[i] - mean) * inv, g ? g[i] : 1.f, b ? b[i] : 0.f);
}

/* a2 + a1/a3: h = (x + bias) + residual — the decode order `xb += bout; xb += x`
 * (t2s_engine.cpp:1096-1097, 1117-1118; also prefill 980/1018 and HuBERT 697-700) — then LN. */
int oracle_add_layernorm(int dtype, const void* x, const float* bias, const void* residual,
                         const float* gamma, const float* beta, void* y, size_t rows, size_t n,
                         size_t ld, double eps, int mode) {
  float* h = (float*)malloc(n * 4);
  float* r = (float*)malloc(n * 4);
  float* o = (float*)malloc(n * 4);
  if (!h || !r || !o) {
    free(h);
    free(r);
    free(o);
    return -1;
  }
  for (size_t row = 0; row < rows; ++row) {
    oracle_to_f32(dtype, row_ptr(x, dtype, row * ld), h, n);
    if (bias)
      for (size_t j = 0; j < n; ++j) h[j] = h[j] + bias[j];
    if (residual) {
      oracle_to_f32(dtype, row_ptr(residual, dtype, row * ld), r, n);
      for (size_t j = 0; j < n; ++j) h[j] = h[j] + r[j];
    }
    if (mode == 1) {
      oracle_layernorm1d_row(h, gamma, beta, n, (float)eps);
      memcpy(o, h, n * 4);
    } else {
      oracle_layernorm_row(h, gamma, beta, o, n, eps);
    }
    oracle_from_f32(dtype, o, row_ptr_w(y, dtype, row * ld), n);
  }
  free(h);
  free(r);
  free(o);
  return 0;
}

/* ---------------------------------------------------------------------------------------------
 * a4 / a5 / a7: activations after the separate bias pass.
 * --------------------------------------------------------------------------------------------- */

/* vmaxq_f32(v, 0): NaN in -> that NaN made quiet; -0 -> +0. */
static inline float relu_vec(float v) {
  if (v != v) return bits_f(f_bits(v) | 0x00400000u);
  return v > 0.f ? v : 0.f;
}

/* kern::relu (kern.cpp:85-91): 4-wide body, scalar tail `x > 0 ? x : 0` (NaN -> 0 there). */
void oracle_relu(const float* x, float* y, size_t n) {
  const size_t vec_end = n & ~(size_t)3;
  size_t i = 0;
  for (; i < vec_end; ++i) y[i] = relu_vec(x[i]);
  for (; i < n; ++i) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

/* bert::gelu_erf (bert_ops.hpp:25-27) == HubertEngine::gelu (hubert.cpp:233-236):
 * (0.5f * x) * (1.f + erff(x * 0.70710678f)); nothing here contracts. */
float oracle_gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752440f)); }

static inline float leaky(float v, float slope) { return v < 0.f ? v * slope : v; }

int oracle_bias_act(int dtype, int act, const void* x, const float* bias, void* y, size_t rows,
                    size_t n, size_t ld, float slope) {
  float* v = (float*)malloc(n * 4);
  if (!v) return -1;
  for (size_t row = 0; row < rows; ++row) {
    oracle_to_f32(dtype, row_ptr(x, dtype, row * ld), v, n);
    for (size_t j = 0; j < n; ++j) {
      float t = bias ? v[j] + bias[j] : v[j];
      if (act == 1) t = relu_vec(t);
      else if (act == 2) t = oracle_gelu_erf(t);
      else if (act == 3) t = leaky(t, slope);
      v[j] = t;
    }
    oracle_from_f32(dtype, v, row_ptr_w(y, dtype, row * ld), n);
  }
  free(v);
  return 0;
}

/* ---------------------------------------------------------------------------------------------
 * Decode GEMV with fp16 weights (next-tier row 1) and the bias / activation / residual loops that
 * follow it in block_decode_impl (t2s_engine.cpp:1044-1049, 1090-1095, 1105-1116).
 *
 * x rounded to fp16 (T2SEngine::gemv_fmlal, t2s_engine.cpp:696-700 -> kern::f32_to_f16 then
 * kern::gemv_f16x_fmlal, gemv_fmlal.cpp:23-35 and 40-132): per row, eight 4-lane fp32 accumulators
 * a0..a7; each 64-element block adds, into lane l of a_j, w*x of elements 8j+l (vfmlalq_low) then
 * 8j+4+l (vfmlalq_high), every fp16 x fp16 product exact and one rounding per accumulate (fma);
 * s = vaddv(a0) + vaddv(a1) + ... + vaddv(a7) left to right with vaddv = (l0 + l1) + (l2 + l3);
 * then the tail elements one by one.
 *
 * x in fp32 (kern::gemv_f16w_f32acc, gemv.cpp:36-127, the 4-row kernel): two 4-lane accumulators,
 * acc0 lane l += w[i+l] * x[i+l], acc1 lane l += w[i+4+l] * x[i+4+l] per 8 elements (vfmaq: fma);
 * s = vaddv(acc0 + acc1), then the tail with the contracted s += w*x (fma). (The reference sums the
 * last out % 4 rows of each thread's range as vaddv(acc0) + vaddv(acc1) instead; which rows those
 * are depends on its core count, so the 4-row order is used for every row. The difference is one
 * fp32 rounding, far inside the comparison tolerance.)
 * --------------------------------------------------------------------------------------------- */
static inline float vaddv4q(const float a[4]) { return (a[0] + a[1]) + (a[2] + a[3]); }

static float dot_fmlal(const uint16_t* w, const float* xh, size_t in) {
  float a[8][4];
  memset(a, 0, sizeof a);
  const size_t vec_end = in & ~(size_t)63;
  size_t i = 0;
  for (; i < vec_end; i += 64)
    for (int j = 0; j < 8; ++j)
      for (int half = 0; half < 2; ++half)
        for (int l = 0; l < 4; ++l) {
          const size_t e = i + 8 * (size_t)j + 4 * (size_t)half + (size_t)l;
          a[j][l] = fmaf(oracle_h2f(w[e]), xh[e], a[j][l]);
        }
  float s = vaddv4q(a[0]);
  for (int j = 1; j < 8; ++j) s = s + vaddv4q(a[j]);
  for (; i < in; ++i) s = fmaf(oracle_h2f(w[i]), xh[i], s);
  return s;
}

static float dot_f32acc(const uint16_t* w, const float* x, size_t in) {
  float a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
  const size_t vec_end = in & ~(size_t)7;
  size_t i = 0;
  for (; i < vec_end; i += 8)
    for (int l = 0; l < 4; ++l) {
      a0[l] = fmaf(oracle_h2f(w[i + l]), x[i + l], a0[l]);
      a1[l] = fmaf(oracle_h2f(w[i + 4 + l]), x[i + 4 + l], a1[l]);
    }
  float t[4];
  for (int l = 0; l < 4; ++l) t[l] = a0[l] + a1[l];
  float s = vaddv4q(t);
  for (; i < in; ++i) s = fmaf(oracle_h2f(w[i]), x[i], s);
  return s;
}

int oracle_gemv_f16w(int x_dtype, int round_x, const void* x, size_t ldx, const uint16_t* w,
                     const float* bias, int act, float slope, const void* residual, int y_dtype,
                     void* y, size_t ldy, size_t rows, size_t out, size_t in) {
  float* xr = (float*)malloc(in * 4);
  float* v = (float*)malloc(out * 4);
  float* r = (float*)malloc(out * 4);
  if (!xr || !v || !r) {
    free(xr);
    free(v);
    free(r);
    return -1;
  }
  const int fmlal = x_dtype == 1 || round_x;
  for (size_t row = 0; row < rows; ++row) {
    oracle_to_f32(x_dtype, row_ptr(x, x_dtype, row * ldx), xr, in);
    if (x_dtype == 0 && round_x)
      for (size_t k = 0; k < in; ++k) xr[k] = oracle_h2f(oracle_f2h(xr[k]));
    for (size_t n = 0; n < out; ++n) {
      const uint16_t* wr = w + n * in;
      float t = fmlal ? dot_fmlal(wr, xr, in) : dot_f32acc(wr, xr, in);
      if (bias) t = t + bias[n];
      if (act == 1) t = relu_vec(t);
      else if (act == 2) t = oracle_gelu_erf(t);
      else if (act == 3) t = leaky(t, slope);
      v[n] = t;
    }
    if (residual) {
      oracle_to_f32(y_dtype, row_ptr(residual, y_dtype, row * ldy), r, out);
      for (size_t n = 0; n < out; ++n) v[n] = v[n] + r[n];
    }
    oracle_from_f32(y_dtype, v, row_ptr_w(y, y_dtype, row * ldy), out);
  }
  free(xr);
  free(v);
  free(r);
  return 0;
}

/* ---------------------------------------------------------------------------------------------
 * SoVITS Conv1d with the ResBlock epilogues (next-tier row 4): Conv1d::forward's fallback path
 * (conv1d.hpp:155-196): same padding pad_l = (k-1)*dilation/2, im2col K index = i*k + kk, fp32
 * weights (the fp16 weights upcast), y = W col + b ("yr[t] += bc" after the GEMM); then, per epi:
 *   0: y                                   1: leaky_relu_io(y, slope)      (dec.hpp:323-324)
 *   2: cur += y; y_out = lrelu(cur, slope) (add_inplace then the next leaky_relu_write, 322-326)
 *   3: cur += y                            (add_inplace only: the branch's last pair)
 *   4: y, and cur = lrelu(y, slope)        (the upsampler's output and the first pair's input)
 *   5: tanh(y)                             (conv_post then std::tanh, dec.hpp:343-344)
 * The GEMM sums over K in order with one rounding per step (fmaf); Accelerate's sgemm order is not
 * published, so parity with it is tolerance-based in any case.
 * --------------------------------------------------------------------------------------------- */
/* The epilogue of one fp32 output row (n columns) of output channel o, per epi (see above). */
static int conv_epilogue(int dtype, float* row, size_t o, int epi, float slope, void* cur, size_t ldc,
                         void* y, size_t ldy, size_t n) {
  if (epi == 1) {
    for (size_t t = 0; t < n; ++t) row[t] = leaky(row[t], slope);
    oracle_from_f32(dtype, row, row_ptr_w(y, dtype, o * ldy), n);
  } else if (epi == 2 || epi == 3) {
    float* c = (float*)malloc(n * 4);
    if (!c) return -1;
    oracle_to_f32(dtype, row_ptr(cur, dtype, o * ldc), c, n);
    for (size_t t = 0; t < n; ++t) c[t] = c[t] + row[t];
    oracle_from_f32(dtype, c, row_ptr_w(cur, dtype, o * ldc), n);
    if (epi == 2) {
      for (size_t t = 0; t < n; ++t) row[t] = leaky(c[t], slope);
      oracle_from_f32(dtype, row, row_ptr_w(y, dtype, o * ldy), n);
    }
    free(c);
  } else if (epi == 4) {  /* y = v; cur = lrelu(v): the upsampler and the first pair's input */
    oracle_from_f32(dtype, row, row_ptr_w(y, dtype, o * ldy), n);
    for (size_t t = 0; t < n; ++t) row[t] = leaky(row[t], slope);
    oracle_from_f32(dtype, row, row_ptr_w(cur, dtype, o * ldc), n);
  } else if (epi == 5) {  /* y = tanh(v): conv_post then std::tanh (dec.hpp:343-344) */
    for (size_t t = 0; t < n; ++t) row[t] = tanhf(row[t]);
    oracle_from_f32(dtype, row, row_ptr_w(y, dtype, o * ldy), n);
  } else {
    oracle_from_f32(dtype, row, row_ptr_w(y, dtype, o * ldy), n);
  }
  return 0;
}

int oracle_conv1d(int dtype, const void* x, size_t ldx, const uint16_t* w, const float* bias, int epi,
                  float slope, void* cur, size_t ldc, void* y, size_t ldy, size_t cin, size_t cout,
                  size_t T, size_t k, size_t dil) {
  float* xr = (float*)malloc(cin * T * 4);
  float* wf = (float*)malloc(cout * cin * k * 4);
  float* row = (float*)malloc(T * 4);
  int rc = 0;
  if (!xr || !wf || !row) {
    rc = -1;
    goto done;
  }
  for (size_t i = 0; i < cin; ++i) oracle_to_f32(dtype, row_ptr(x, dtype, i * ldx), xr + i * T, T);
  for (size_t e = 0; e < cout * cin * k; ++e) wf[e] = oracle_h2f(w[e]);
  const long pad = (long)((k - 1) * dil) / 2;
  for (size_t o = 0; o < cout && rc == 0; ++o) {
    for (size_t t = 0; t < T; ++t) {
      float s = 0.f;
      for (size_t i = 0; i < cin; ++i)
        for (size_t kk = 0; kk < k; ++kk) {
          const long src = (long)t + (long)(kk * dil) - pad;
          const float xv = (src >= 0 && src < (long)T) ? xr[i * T + (size_t)src] : 0.f;
          s = fmaf(wf[(o * cin + i) * k + kk], xv, s);
        }
      row[t] = bias ? s + bias[o] : s;
    }
    rc = conv_epilogue(dtype, row, o, epi, slope, cur, ldc, y, ldy, T);
  }
done:
  free(xr);
  free(wf);
  free(row);
  return rc;
}

/* ---------------------------------------------------------------------------------------------
 * SoVITS ConvTranspose1d (next-tier row 4): ConvT1d::forward's fallback path (conv1d.hpp:250-340).
 * Weights w[i][o][d] (torch layout, upcast from fp16), stride u, pad = (k - u) / 2, T_out = T u:
 *   y = 0; for d = 0 .. k-1: tmp[o][j] = sum_i W[i][o][d] x[i][j] (one sgemm per tap, the sum in
 *   order with fmaf), then y[o][j u + d - pad] += tmp[o][j] where inside [0, T_out) (scatter_raw);
 *   finally y += b, and the epilogue of Conv1d (epi 0 .. 3) on the T_out-column rows.
 * --------------------------------------------------------------------------------------------- */
int oracle_convt1d(int dtype, const void* x, size_t ldx, const uint16_t* w, const float* bias,
                   int epi, float slope, void* cur, size_t ldc, void* y, size_t ldy, size_t cin,
                   size_t cout, size_t T, size_t k, size_t u) {
  if (k < u || u == 0) return -2;
  const size_t Tout = T * u;
  const long pad = (long)(k - u) / 2;
  float* xr = (float*)malloc(cin * T * 4);
  float* wf = (float*)malloc(cin * cout * k * 4);
  float* acc = (float*)calloc(Tout, 4);
  int rc = 0;
  if (!xr || !wf || !acc) {
    rc = -1;
    goto done;
  }
  for (size_t i = 0; i < cin; ++i) oracle_to_f32(dtype, row_ptr(x, dtype, i * ldx), xr + i * T, T);
  for (size_t e = 0; e < cin * cout * k; ++e) wf[e] = oracle_h2f(w[e]);
  for (size_t o = 0; o < cout && rc == 0; ++o) {
    for (size_t t = 0; t < Tout; ++t) acc[t] = 0.f;
    for (size_t d = 0; d < k; ++d)
      for (size_t j = 0; j < T; ++j) {
        float s = 0.f;
        for (size_t i = 0; i < cin; ++i) s = fmaf(wf[(i * cout + o) * k + d], xr[i * T + j], s);
        const long pos = (long)(j * u + d) - pad;
        if (pos >= 0 && pos < (long)Tout) acc[pos] += s;
      }
    if (bias)
      for (size_t t = 0; t < Tout; ++t) acc[t] += bias[o];
    rc = conv_epilogue(dtype, acc, o, epi, slope, cur, ldc, y, ldy, Tout);
  }
done:
  free(xr);
  free(wf);
  free(acc);
  return rc;
}

/* ---------------------------------------------------------------------------------------------
 * Decode attention (next-tier row 2): block_decode_impl's KV append and single-query SDPA per head
 * (t2s_engine.cpp:1051-1087), per sequence b at position pos[b]:
 *   K[pos] = k, V[pos] = v (rounded to the cache type: kern::f32_to_f16 for fp16 caches, 1051-1058)
 *   for each head h, keys k < len = pos + 1:
 *     s_k = dot(q_h, K[k, h]) * scale        ar_neon::dot_f16kv / dot_f32 (t2s_engine.cpp:40-103)
 *     p = kern::softmax(s)                    (kern.cpp:62-74)
 *     o_h = sum_k p_k V[k, h]                 ar_neon::accum_f16kv / accum_f32 (105-145)
 * dot: four 4-lane accumulators over 16-element groups (fma), (a0 + a1) + (a2 + a3) lane-wise,
 * then (l0 + l2) + (l1 + l3); tail elements with the contracted dot += q*k. softmax: sequential max,
 * e = expf(x - max), sequential sum, then x * (1 / sum). accum: ov[e] = ov[e] + p * v[e] with the
 * product rounded first (vmulq then vaddq) in 16-element groups, tail contracted (fma).
 * --------------------------------------------------------------------------------------------- */
static float attn_dot(const float* q, const float* k, size_t HD) {
  float a[4][4];
  memset(a, 0, sizeof a);
  size_t e = 0;
  for (; e + 16 <= HD; e += 16)
    for (int j = 0; j < 4; ++j)
      for (int l = 0; l < 4; ++l) a[j][l] = fmaf(q[e + 4 * j + l], k[e + 4 * j + l], a[j][l]);
  float t[4];
  for (int l = 0; l < 4; ++l) t[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
  float dot = (t[0] + t[2]) + (t[1] + t[3]);
  for (; e < HD; ++e) dot = fmaf(q[e], k[e], dot);
  return dot;
}

static void attn_accum(float* o, const float* v, float p, size_t HD) {
  size_t e = 0;
  for (; e + 16 <= HD; e += 16)
    for (int i = 0; i < 16; ++i) o[e + i] = o[e + i] + p * v[e + i];
  for (; e < HD; ++e) o[e] = fmaf(p, v[e], o[e]);
}

void oracle_softmax(const float* x, float* y, size_t n) {
  float m = x[0];
  for (size_t i = 1; i < n; ++i) m = m < x[i] ? x[i] : m;
  float sum = 0.f;
  for (size_t i = 0; i < n; ++i) {
    const float e = expf(x[i] - m);
    y[i] = e;
    sum += e;
  }
  const float inv = 1.0f / sum;
  for (size_t i = 0; i < n; ++i) y[i] *= inv;
}

int oracle_decode_attention(int kv_dtype, const float* qkv, size_t ldq, void* kcache, void* vcache,
                            size_t max_len, const int64_t* pos, float* out, size_t ldo, size_t B,
                            size_t H, size_t HD) {
  const size_t D = H * HD;
  const float scale = 1.0f / sqrtf((float)HD);
  float* sc = (float*)malloc((max_len ? max_len : 1) * 4);
  float* kr = (float*)malloc(D * 4);
  float* vr = (float*)malloc(D * 4);
  if (!sc || !kr || !vr) {
    free(sc);
    free(kr);
    free(vr);
    return -1;
  }
  const size_t esz = esize(kv_dtype);
  for (size_t b = 0; b < B; ++b) {
    float* ob = out + b * ldo;
    const int64_t p = pos[b];
    if (p < 0 || (size_t)p >= max_len) {
      for (size_t i = 0; i < D; ++i) ob[i] = bits_f(0x7fc00000u);
      continue;
    }
    const float* qb = qkv + b * ldq;
    char* kb = (char*)kcache + b * max_len * D * esz;
    char* vb = (char*)vcache + b * max_len * D * esz;
    oracle_from_f32(kv_dtype, qb + D, kb + (size_t)p * D * esz, D);
    oracle_from_f32(kv_dtype, qb + 2 * D, vb + (size_t)p * D * esz, D);
    const size_t len = (size_t)p + 1;
    for (size_t h = 0; h < H; ++h) {
      const float* qh = qb + h * HD;
      for (size_t k = 0; k < len; ++k) {
        oracle_to_f32(kv_dtype, kb + (k * D + h * HD) * esz, kr, HD);
        sc[k] = attn_dot(qh, kr, HD) * scale;
      }
      float m = sc[0];
      for (size_t k = 1; k < len; ++k) m = m < sc[k] ? sc[k] : m;
      float sum = 0.f;
      for (size_t k = 0; k < len; ++k) {
        const float e = expf(sc[k] - m);
        sc[k] = e;
        sum += e;
      }
      const float inv = 1.0f / sum;
      for (size_t k = 0; k < len; ++k) sc[k] *= inv;
      float* oh = ob + h * HD;
      for (size_t e = 0; e < HD; ++e) oh[e] = 0.f;
      for (size_t k = 0; k < len; ++k) {
        oracle_to_f32(kv_dtype, vb + (k * D + h * HD) * esz, vr, HD);
        attn_accum(oh, vr, sc[k], HD);
      }
    }
  }
  free(sc);
  free(kr);
  free(vr);
  return 0;
}

/* ---------------------------------------------------------------------------------------------
 * a6: HuBERT conv-layer-0 GroupNorm(groups = C) + GELU (hubert.cpp:487-503): per channel, double
 * sequential mean, double two-pass variance with the contracted `var += (p-mu)*(p-mu)`,
 * rstd = 1/sqrt(var + eps), p = float((p - mu)*rstd*g + b) with the double multiply-add fused;
 * then GELU over the buffer in fp32.
 * --------------------------------------------------------------------------------------------- */
int oracle_groupnorm_gelu(int dtype, const void* x, const float* gamma, const float* beta, void* y,
                          size_t channels, size_t T, size_t ld, double eps, int apply_gelu) {
  float* p = (float*)malloc(T * 4);
  if (!p) return -1;
  const double inv = 1.0 / (double)T;
  for (size_t ch = 0; ch < channels; ++ch) {
    oracle_to_f32(dtype, row_ptr(x, dtype, ch * ld), p, T);
    double mu = 0.0, var = 0.0;
    for (size_t t = 0; t < T; ++t) mu += p[t];
    mu *= inv;
    for (size_t t = 0; t < T; ++t) var = fma(p[t] - mu, p[t] - mu, var);
    var *= inv;
    const double rstd = 1.0 / sqrt(var + eps);
    const double g = gamma ? gamma[ch] : 1.0, b = beta ? beta[ch] : 0.0;
    for (size_t t = 0; t < T; ++t) p[t] = (float)fma((p[t] - mu) * rstd, g, b);
    if (apply_gelu)
      for (size_t t = 0; t < T; ++t) p[t] = oracle_gelu_erf(p[t]);
    oracle_from_f32(dtype, p, row_ptr_w(y, dtype, ch * ld), T);
  }
  free(p);
  return 0;
}

/* ---------------------------------------------------------------------------------------------
 * a7 / a8 / a9: SoVITS element-wise steps (nn_ops.hpp:48-105; dec.hpp:283-342).
 * --------------------------------------------------------------------------------------------- */

/* Element-wise helpers over 16-bit storage convert one value at a time (same result as a row). */
static inline float ld1(int dtype, const void* p, size_t i) {
  if (dtype == 0) return ((const float*)p)[i];
  const uint16_t h = ((const uint16_t*)p)[i];
  return dtype == 1 ? oracle_h2f(h) : oracle_bf2f(h);
}
static inline void st1(int dtype, void* p, size_t i, float v) {
  if (dtype == 0) ((float*)p)[i] = v;
  else ((uint16_t*)p)[i] = dtype == 1 ? oracle_f2h(v) : oracle_f2bf(v);
}

/* leaky_relu_io / leaky_relu_write: v < 0 ? v*slope : v (vcltzq + vbslq; -0 and NaN kept). */
int oracle_leaky_relu(int dtype, const void* x, void* y, size_t n, float slope) {
  for (size_t i = 0; i < n; ++i) st1(dtype, y, i, leaky(ld1(dtype, x, i), slope));
  return 0;
}

/* add_inplace(cur, t_b) (dec.hpp:326) then leaky_relu_write(cur, t_in, 0.1) (dec.hpp:322). */
int oracle_resblock_add_lrelu(int dtype, void* cur, const void* t_b, void* t_in, size_t n,
                              float slope) {
  for (size_t i = 0; i < n; ++i) {
    const float v = ld1(dtype, cur, i) + ld1(dtype, t_b, i);
    st1(dtype, cur, i, v);
    if (t_in) st1(dtype, t_in, i, leaky(v, slope));
  }
  return 0;
}

/* For each branch j: cur_j += t_b_j (dec.hpp:326, the last conv pair); j = 0: sum = cur*kInv
 * (mul_write); j > 0: sum = sum + cur*kInv (add_scaled_inplace; vmlaq_f32 is a multiply and an
 * add, rounded separately); kInv = 1.f/3 (dec.hpp:295). Then the next stage's leaky_relu_io. */
int oracle_resblock_branch_mean(int dtype, const void* const* cur, const void* const* t_b,
                                int nbranch, void* out, size_t n, int apply_lrelu, float slope) {
  const float kinv = 1.f / (float)nbranch;
  for (size_t i = 0; i < n; ++i) {
    float acc = 0.f;
    for (int j = 0; j < nbranch; ++j) {
      float v = ld1(dtype, cur[j], i);
      if (t_b && t_b[j]) v = v + ld1(dtype, t_b[j], i);
      const float prod = v * kinv;
      acc = j == 0 ? prod : acc + prod;
    }
    st1(dtype, out, i, apply_lrelu ? leaky(acc, slope) : acc);
  }
  return 0;
}

int oracle_scaled_add(int dtype, const void* acc, const void* src, void* out, size_t n,
                      float scale) {
  for (size_t i = 0; i < n; ++i) {
    const float prod = ld1(dtype, src, i) * scale;
    st1(dtype, out, i, acc ? ld1(dtype, acc, i) + prod : prod);
  }
  return 0;
}

/* ---------------------------------------------------------------------------------------------
 * a10: T2SEngine::pe_row (t2s_engine.cpp:711-720) and the input gathers.
 * --------------------------------------------------------------------------------------------- */
void oracle_pe_row(float* pe, size_t pos, size_t D) {
  const float log_inc = (float)(-log(10000.0) / (double)D);
  const float p = (float)pos;
  for (size_t d = 0; d < D; d += 2) {
    const float div = expf((float)d * log_inc);
    pe[d] = sinf(p * div);
    pe[d + 1] = cosf(p * div);
  }
}

/* audio / decode rows: x = e + alpha*pe (t2s_engine.cpp:1785, 1869), one fused multiply-add;
 * text rows: x = mm; x += e + b; x += alpha*pe (1777, 1779), the last one fused. */
long oracle_embed_pe(int out_dtype, int table_dtype, int index_type, const void* table,
                     size_t vocab, const void* ids, const int64_t* pos, int64_t pos0,
                     const float* pe, size_t max_pos, float alpha, const void* mm,
                     const float* bias, void* out, size_t rows, size_t D) {
  long bad = 0;
  for (size_t r = 0; r < rows; ++r) {
    const int64_t id = index_type == 1 ? (int64_t)((const int32_t*)ids)[r] : ((const int64_t*)ids)[r];
    const int64_t p = pos ? pos[r] : pos0 + (int64_t)r;
    const int ok = id >= 0 && (uint64_t)id < vocab && p >= 0 && (uint64_t)p < max_pos;
    if (!ok) ++bad;
    for (size_t d = 0; d < D; ++d) {
      float o = nanf("");
      if (ok) {
        float e = ld1(table_dtype, table, (size_t)id * D + d);
        if (bias) e = e + bias[d];
        if (mm) e = ld1(out_dtype, mm, r * D + d) + e;
        o = fmaf(alpha, pe[(size_t)p * D + d], e);
      }
      st1(out_dtype, out, r * D + d, o);
    }
  }
  return bad;
}

/* ---------------------------------------------------------------------------------------------
 * One T2S decode step's epilogue chain over B rows, split into row bands over threads.
 * --------------------------------------------------------------------------------------------- */
typedef struct {
  int dtype;
  size_t D, FF, layers, r0, r1;
  double eps;
  const void* table;
  int table_dtype;
  size_t vocab;
  const int64_t* ids;
  const int64_t* pos;
  const float* pe;
  size_t max_pos;
  float alpha;
  void* x;
  void* h;
  const void* const* attn_out;
  const float* const* bout;
  const float* const* n1g;
  const float* const* n1b;
  void* const* ff;
  const float* const* b1;
  const void* const* ffn_out;
  const float* const* b2;
  const float* const* n2g;
  const float* const* n2b;
} StepBand;

static const float* at(const float* const* a, size_t l) { return a ? a[l] : NULL; }

static void* step_band(void* arg) {
  const StepBand* s = (const StepBand*)arg;
  const size_t rows = s->r1 - s->r0, D = s->D, FF = s->FF;
  if (!rows) return NULL;
  const int dt = s->dtype;
  oracle_embed_pe(dt, s->table_dtype, 0, s->table, s->vocab, s->ids + s->r0,
                  s->pos ? s->pos + s->r0 : NULL, 0, s->pe, s->max_pos, s->alpha, NULL, NULL,
                  row_ptr_w(s->x, dt, s->r0 * D), rows, D);
  for (size_t l = 0; l < s->layers; ++l) {
    oracle_add_layernorm(dt, row_ptr(s->attn_out[l], dt, s->r0 * D), at(s->bout, l),
                         row_ptr(s->x, dt, s->r0 * D), at(s->n1g, l), at(s->n1b, l),
                         row_ptr_w(s->h, dt, s->r0 * D), rows, D, D, s->eps, 0);
    oracle_bias_act(dt, 1, row_ptr(s->ff[l], dt, s->r0 * FF), at(s->b1, l),
                    row_ptr_w(s->ff[l], dt, s->r0 * FF), rows, FF, FF, 0.f);
    oracle_add_layernorm(dt, row_ptr(s->ffn_out[l], dt, s->r0 * D), at(s->b2, l),
                         row_ptr(s->h, dt, s->r0 * D), at(s->n2g, l), at(s->n2b, l),
                         row_ptr_w(s->x, dt, s->r0 * D), rows, D, D, s->eps, 0);
  }
  return NULL;
}

int oracle_t2s_step(int dtype, size_t B, size_t D, size_t FF, size_t layers, double eps,
                    const void* table, int table_dtype, size_t vocab, const int64_t* ids,
                    const int64_t* pos, const float* pe, size_t max_pos, float alpha, void* x,
                    void* h, const void* const* attn_out, const float* const* bout,
                    const float* const* n1g, const float* const* n1b, void* const* ff,
                    const float* const* b1, const void* const* ffn_out, const float* const* b2,
                    const float* const* n2g, const float* const* n2b, int threads) {
  if (threads < 1) threads = 1;
  if ((size_t)threads > B) threads = (int)B;
  StepBand* bands = (StepBand*)calloc((size_t)threads, sizeof(StepBand));
  pthread_t* tid = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
  if (!bands || !tid) {
    free(bands);
    free(tid);
    return -1;
  }
  for (int t = 0; t < threads; ++t) {
    StepBand* s = &bands[t];
    s->dtype = dtype;
    s->D = D;
    s->FF = FF;
    s->layers = layers;
    s->r0 = B * (size_t)t / (size_t)threads;
    s->r1 = B * (size_t)(t + 1) / (size_t)threads;
    s->eps = eps;
    s->table = table;
    s->table_dtype = table_dtype;
    s->vocab = vocab;
    s->ids = ids;
    s->pos = pos;
    s->pe = pe;
    s->max_pos = max_pos;
    s->alpha = alpha;
    s->x = x;
    s->h = h;
    s->attn_out = attn_out;
    s->bout = bout;
    s->n1g = n1g;
    s->n1b = n1b;
    s->ff = ff;
    s->b1 = b1;
    s->ffn_out = ffn_out;
    s->b2 = b2;
    s->n2g = n2g;
    s->n2b = n2b;
  }
  int rc = 0;
  for (int t = 1; t < threads; ++t)
    if (pthread_create(&tid[t], NULL, step_band, &bands[t]) != 0) rc = -1;
  step_band(&bands[0]);
  for (int t = 1; t < threads; ++t)
    if (tid[t]) pthread_join(tid[t], NULL);
  free(bands);
  free(tid);
  return rc;
}
