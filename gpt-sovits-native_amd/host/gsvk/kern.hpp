// gsvk/kern.hpp — C++ host mirror of the reference's kernel-layer interface over the gsvk C ABI.
//
// The functions keep the reference's names, argument order and argument meaning so an engine's
// call sites compile unchanged after swapping the include:
//   gsv::kern::layernorm / relu                      (src/kern/kern.hpp:25, 33)
//   gsv::kern::gemv_f16w_f32acc / gemv_f16x_fmlal / f32_to_f16-free batched forms
//                                                    (src/kern/gemv.cpp:112, gemv_fmlal.cpp:113)
//   gsv::sovits::leaky_relu_io / leaky_relu_write / add_inplace / add_scaled_inplace / mul_write
//                                                    (src/sovits/nn_ops.hpp:48-105)
//   gsv::bert::gelu_erf over a buffer                (src/bert/bert_ops.hpp:25-27, 394)
//   gsv::bert::Matrix / LayerNorm1D::forward(Matrix&) (src/bert/bert_io.hpp:18-27,
//                                                     bert_ops.hpp:261-286), device storage
//   gsv::sovits::Tensor2D                            (src/sovits/sovits_types.hpp:21-36)
//   gsv::ar::PeRows::pe_row(float*, size_t)          (src/ar/t2s_engine.hpp:187)
//   gsv::sovits::Conv1d / ConvT1d, device-resident   (src/sovits/conv1d.hpp:56-360)
// Differences, all deliberate: pointers are device pointers; every call is enqueued on the calling
// thread's current stream (gsvk::set_stream) and returns before the GPU finishes (call
// gsvk::sync() before reading results on the host); a rejected argument or a HIP launch failure
// throws std::runtime_error (the reference's error style at load time, t2s_engine.cpp:559-562)
// instead of being undefined behaviour. Row-batched forms (one launch per tensor) sit next to the
// per-row ones, because a GPU call per row is the wrong granularity.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "gsvk.h"

namespace gsvk {

inline hipStream_t& current_stream_ref() {
  static thread_local hipStream_t s = nullptr;
  return s;
}
inline void set_stream(hipStream_t s) { current_stream_ref() = s; }
inline hipStream_t current_stream() { return current_stream_ref(); }

inline void check(int rc, const char* what) {
  if (rc != GSVK_OK)
    throw std::runtime_error(std::string(what) + ": " + gsvk_status_string(rc));
}
inline void sync() {
  if (hipStreamSynchronize(current_stream()) != hipSuccess)
    throw std::runtime_error("gsvk::sync: hipStreamSynchronize failed");
}

// Owning device buffer with the parts of std::vector the reference's containers use (data(),
// size(), assign(n, 0)), so their call sites (`f(x.d.data(), x.d.size(), ...)`) compile unchanged
// with device storage. Allocation happens in resize / assign, as the reference allocates in its
// containers' reset / load; the kernels themselves allocate nothing.
template <class T>
class DeviceVector {
 public:
  DeviceVector() = default;
  explicit DeviceVector(size_t n) { resize(n); }
  DeviceVector(const DeviceVector&) = delete;
  DeviceVector& operator=(const DeviceVector&) = delete;
  DeviceVector(DeviceVector&& o) noexcept : p_(o.p_), n_(o.n_), cap_(o.cap_) {
    o.p_ = nullptr;
    o.n_ = o.cap_ = 0;
  }
  DeviceVector& operator=(DeviceVector&& o) noexcept {
    if (this != &o) {
      release();
      p_ = o.p_, n_ = o.n_, cap_ = o.cap_;
      o.p_ = nullptr;
      o.n_ = o.cap_ = 0;
    }
    return *this;
  }
  ~DeviceVector() { release(); }

  // n elements; the contents are unspecified after a reallocation.
  void resize(size_t n) {
    if (n > cap_) {
      release();
      if (hipMalloc(reinterpret_cast<void**>(&p_), n * sizeof(T)) != hipSuccess)
        throw std::runtime_error("gsvk::DeviceVector: hipMalloc failed");
      cap_ = n;
    }
    n_ = n;
  }
  // n zero elements (std::vector::assign(n, 0) of the reference's reset()).
  void assign(size_t n, T zero) {
    if (zero != T(0)) throw std::runtime_error("gsvk::DeviceVector::assign: only zero fill");
    resize(n);
    if (n && hipMemsetAsync(p_, 0, n * sizeof(T), current_stream()) != hipSuccess)
      throw std::runtime_error("gsvk::DeviceVector::assign: hipMemsetAsync failed");
  }
  // Both copies run on the thread's current stream, after the work already queued there (a zero
  // fill from assign(), a kernel writing the buffer), and return once the copy has completed.
  void copy_from_host(const T* host, size_t n) {
    resize(n);
    if (n && (hipMemcpyAsync(p_, host, n * sizeof(T), hipMemcpyHostToDevice, current_stream()) !=
                  hipSuccess ||
              hipStreamSynchronize(current_stream()) != hipSuccess))
      throw std::runtime_error("gsvk::DeviceVector: host-to-device copy failed");
  }
  void copy_to_host(T* host) const {
    if (n_ && (hipMemcpyAsync(host, p_, n_ * sizeof(T), hipMemcpyDeviceToHost, current_stream()) !=
                   hipSuccess ||
               hipStreamSynchronize(current_stream()) != hipSuccess))
      throw std::runtime_error("gsvk::DeviceVector: device-to-host copy failed");
  }
  T* data() { return p_; }
  const T* data() const { return p_; }
  size_t size() const { return n_; }
  bool empty() const { return n_ == 0; }

 private:
  void release() {
    if (p_) (void)hipFree(p_);
    p_ = nullptr;
    n_ = cap_ = 0;
  }
  T* p_ = nullptr;
  size_t n_ = 0, cap_ = 0;
};

}  // namespace gsvk

namespace gsv::kern {

// y = (x - mean) / sqrt(var + eps) * g + b over one row of n floats (kern.hpp:25). y may be x.
inline void layernorm(const float* x, const float* g, const float* b, float* y, size_t n,
                      double eps) {
  gsvk::check(gsvk_add_layernorm(GSVK_F32, x, nullptr, nullptr, g, b, y, 1, n, n, eps,
                                 gsvk::current_stream()),
              "gsv::kern::layernorm");
}

// The same over `rows` consecutive rows: one launch replaces the per-row loops at
// t2s_engine.cpp:985-987 / hubert.cpp:701-703.
inline void layernorm_rows(const float* x, const float* g, const float* b, float* y, size_t rows,
                           size_t n, double eps) {
  gsvk::check(gsvk_add_layernorm(GSVK_F32, x, nullptr, nullptr, g, b, y, rows, n, n, eps,
                                 gsvk::current_stream()),
              "gsv::kern::layernorm_rows");
}

// y = LN((mm + bias) + residual): the residual/bias loop and the LayerNorm that follows it
// (t2s_engine.cpp:1096-1098, 1117-1119) in one launch.
inline void add_layernorm(const float* mm, const float* bias, const float* residual, const float* g,
                          const float* b, float* y, size_t rows, size_t n, double eps) {
  gsvk::check(gsvk_add_layernorm(GSVK_F32, mm, bias, residual, g, b, y, rows, n, n, eps,
                                 gsvk::current_stream()),
              "gsv::kern::add_layernorm");
}

// y = max(x, 0) (kern.hpp:33).
inline void relu(const float* x, float* y, size_t n) {
  gsvk::check(gsvk_bias_act(GSVK_F32, GSVK_ACT_RELU, x, nullptr, y, 1, n, n, 0.f,
                            gsvk::current_stream()),
              "gsv::kern::relu");
}

// ff = relu(ff + b1) over [rows, n] (t2s_engine.cpp:995-996, 1111-1112).
inline void bias_relu(float* ff, const float* b1, size_t rows, size_t n) {
  gsvk::check(gsvk_bias_act(GSVK_F32, GSVK_ACT_RELU, ff, b1, ff, rows, n, n, 0.f,
                            gsvk::current_stream()),
              "gsv::kern::bias_relu");
}

// y[out] = W16 x, fp32 activations, fp32 accumulation (gemv.cpp:112-127).
inline void gemv_f16w_f32acc(const uint16_t* w, const float* x, float* y, size_t out, size_t in) {
  gsvk::check(gsvk_gemv_f16w(GSVK_F32, 0, x, in, w, nullptr, GSVK_ACT_NONE, 0.f, nullptr, GSVK_F32,
                             y, out, 1, out, in, gsvk::current_stream()),
              "gsv::kern::gemv_f16w_f32acc");
}

// y[out] = W16 xh with xh already fp16 bit patterns (gemv_fmlal.cpp:113-132).
inline void gemv_f16x_fmlal(const uint16_t* w, const uint16_t* xh, float* y, size_t out,
                            size_t in) {
  gsvk::check(gsvk_gemv_f16w(GSVK_F16, 1, xh, in, w, nullptr, GSVK_ACT_NONE, 0.f, nullptr, GSVK_F32,
                             y, out, 1, out, in, gsvk::current_stream()),
              "gsv::kern::gemv_f16x_fmlal");
}

// B sequences at once, x rounded to fp16 as T2SEngine::gemv_fmlal does (t2s_engine.cpp:696-700),
// with the loops after the GEMV fused: y = act(W16 x + bias) (+ residual). x [rows, in],
// y / residual [rows, out]; residual may be y.
inline void gemv_fmlal_rows(const uint16_t* w, const float* x, float* y, size_t rows, size_t out,
                            size_t in, const float* bias = nullptr, int act = GSVK_ACT_NONE,
                            const float* residual = nullptr) {
  gsvk::check(gsvk_gemv_f16w(GSVK_F32, 1, x, in, w, bias, act, 0.f, residual, GSVK_F32, y, out,
                             rows, out, in, gsvk::current_stream()),
              "gsv::kern::gemv_fmlal_rows");
}

// The post-LN of block_decode_impl followed by the GEMV that reads its output, in one launch:
// h = layernorm(z; g, b, eps) (kern.hpp:25) is stored and y = act(W16 h + bias) (+ residual)
// (norm1 then W1, t2s_engine.cpp:1097-1112; norm2 then the next QKV, 1119 / 1044). z, h
// [rows, in] (h must not overlap z), y / residual [rows, out].
inline void layernorm_gemv_fmlal_rows(const float* z, const float* g, const float* b, double eps,
                                      float* h, const uint16_t* w, float* y, size_t rows,
                                      size_t out, size_t in, const float* bias = nullptr,
                                      int act = GSVK_ACT_NONE, const float* residual = nullptr) {
  gsvk::check(gsvk_gemv_f16w_ln(GSVK_F32, 1, z, in, g, b, eps, h, in, w, bias, act, 0.f, residual,
                                GSVK_F32, y, out, rows, out, in, gsvk::current_stream()),
              "gsv::kern::layernorm_gemv_fmlal_rows");
}

}  // namespace gsv::kern

namespace gsv::bert {

// x = gelu_erf(x + bias) over [rows, n]; bias may be nullptr (bert_ops.hpp:255-257 then 394).
inline void bias_gelu_erf(float* x, const float* bias, size_t rows, size_t n) {
  gsvk::check(gsvk_bias_act(GSVK_F32, GSVK_ACT_GELU_ERF, x, bias, x, rows, n, n, 0.f,
                            gsvk::current_stream()),
              "gsv::bert::bias_gelu_erf");
}

// LayerNorm1D::forward on a [rows, cols] matrix in place, eps 1e-12 (bert_ops.hpp:261-286).
inline void layernorm1d_forward(float* x, const float* g, const float* bta, size_t rows,
                                size_t cols, float eps = 1e-12f) {
  gsvk::check(gsvk_add_layernorm(GSVK_F32, x, nullptr, nullptr, g, bta, x, rows, cols, cols, eps,
                                 gsvk::current_stream()),
              "gsv::bert::layernorm1d_forward");
}

// bert::Matrix (bert_io.hpp:18-27) with the same members over device storage: row-major
// [rows = T, cols = C], d.data() a device pointer.
struct Matrix {
  size_t rows = 0, cols = 0;
  gsvk::DeviceVector<float> d;
  void reset(size_t r, size_t c) {
    rows = r;
    cols = c;
    d.assign(r * c, 0.f);
  }
  size_t size() const { return d.size(); }
};

// bert::LayerNorm1D (bert_ops.hpp:261-286): members g, bta, eps; forward(Matrix&) in place, one
// launch for all rows. load() takes the host vectors the reference's load() reads from the .gsv
// file (weight, bias of length c).
struct LayerNorm1D {
  gsvk::DeviceVector<float> g, bta;
  float eps = 1e-12f;
  void load(const float* weight, const float* bias, size_t c, float e) {
    eps = e;
    g.copy_from_host(weight, c);
    bta.copy_from_host(bias, c);
  }
  void forward(Matrix& x) const {
    if (g.size() != x.cols || bta.size() != x.cols)
      throw std::runtime_error("gsv::bert::LayerNorm1D::forward: width mismatch");
    layernorm1d_forward(x.d.data(), g.data(), bta.data(), x.rows, x.cols, eps);
  }
};

// The scalar gelu_erf(float) (bert_ops.hpp:25-27) is called inside host loops over host floats;
// on the GPU its loops become bias_gelu_erf over a device buffer (one launch per tensor).

}  // namespace gsv::bert

namespace gsv::encoder {

// HuBERT conv layer 0: GroupNorm(groups = C) then GELU, in place on [C, T] (hubert.cpp:487-503).
inline void groupnorm_gelu(float* x, const float* g, const float* b, size_t C, size_t T,
                           double eps) {
  gsvk::check(gsvk_groupnorm_gelu(GSVK_F32, x, g, b, x, C, T, T, eps, 1, gsvk::current_stream()),
              "gsv::encoder::groupnorm_gelu");
}

// HubertEngine::gelu(float* x, size_t n) (hubert.cpp:233-236).
inline void gelu(float* x, size_t n) {
  gsvk::check(gsvk_bias_act(GSVK_F32, GSVK_ACT_GELU_ERF, x, nullptr, x, 1, n, n, 0.f,
                            gsvk::current_stream()),
              "gsv::encoder::gelu");
}

}  // namespace gsv::encoder

namespace gsv::sovits {

// sovits::Tensor2D (sovits_types.hpp:21-36) with the same members over device storage: [C, T]
// rows contiguous, d.data() / row(c) device pointers.
struct Tensor2D {
  size_t C = 0, T = 0;
  gsvk::DeviceVector<float> d;

  Tensor2D() = default;
  Tensor2D(size_t c, size_t t) { reset(c, t); }

  void reset(size_t c, size_t t) {
    C = c;
    T = t;
    d.assign(c * t, 0.f);
  }
  float* row(size_t c) { return d.data() + c * T; }
  const float* row(size_t c) const { return d.data() + c * T; }
};

inline void leaky_relu_io(float* io, size_t n, float slope) {
  gsvk::check(gsvk_leaky_relu(GSVK_F32, io, io, n, slope, gsvk::current_stream()),
              "gsv::sovits::leaky_relu_io");
}

inline void leaky_relu_write(const float* src, float* dst, size_t n, float slope) {
  gsvk::check(gsvk_leaky_relu(GSVK_F32, src, dst, n, slope, gsvk::current_stream()),
              "gsv::sovits::leaky_relu_write");
}

inline void add_inplace(float* dst, const float* src, size_t n) {
  gsvk::check(gsvk_resblock_add_lrelu(GSVK_F32, dst, src, nullptr, n, 0.f, gsvk::current_stream()),
              "gsv::sovits::add_inplace");
}

inline void add_scaled_inplace(float* acc, const float* src, size_t n, float scale) {
  gsvk::check(gsvk_scaled_add(GSVK_F32, acc, src, acc, n, scale, gsvk::current_stream()),
              "gsv::sovits::add_scaled_inplace");
}

inline void mul_write(float* dst, const float* src, size_t n, float scale) {
  gsvk::check(gsvk_scaled_add(GSVK_F32, nullptr, src, dst, n, scale, gsvk::current_stream()),
              "gsv::sovits::mul_write");
}

// cur += t_b; t_in = lrelu(cur, slope): add_inplace (dec.hpp:326) fused with the next conv pair's
// leaky_relu_write (dec.hpp:322).
inline void add_then_leaky_write(float* cur, const float* t_b, float* t_in, size_t n, float slope) {
  gsvk::check(gsvk_resblock_add_lrelu(GSVK_F32, cur, t_b, t_in, n, slope, gsvk::current_stream()),
              "gsv::sovits::add_then_leaky_write");
}

// x_next = lrelu(sum_j (cur_j + t_b_j) / 3, slope): the end of a Generator stage (dec.hpp:326-336)
// fused with the next stage's leaky_relu_io (dec.hpp:284 / 342).
inline void branch_mean_leaky(const float* const cur[3], const float* const t_b[3], float* x_next,
                              size_t n, float slope) {
  const void* c[3] = {cur[0], cur[1], cur[2]};
  const void* t[3] = {t_b ? t_b[0] : nullptr, t_b ? t_b[1] : nullptr, t_b ? t_b[2] : nullptr};
  gsvk::check(gsvk_resblock_branch_mean(GSVK_F32, c, t, 3, x_next, n, 1, slope,
                                        gsvk::current_stream()),
              "gsv::sovits::branch_mean_leaky");
}

// Device-resident Conv1d (conv1d.hpp:56-203): the reference's members out_c / in_c / k / dilation
// and b, the fp16 [out, in, k] weights packed once at load, forward(x, y) on [C, T] rows. The
// ResBlock passes after a convolution can be fused into it: epi = GSVK_CONV_EPI_LRELU is conv1 +
// leaky_relu_io (dec.hpp:323-324); GSVK_CONV_EPI_RES_LRELU is conv2 + add_inplace into `cur` +
// the next pair's leaky_relu_write into y (dec.hpp:325-326, 322).
class Conv1d {
 public:
  size_t out_c = 0, in_c = 0, k = 0, dilation = 1;
  const float* b = nullptr;      // device fp32 [out_c], or nullptr (conv_post has no bias)
  uint16_t* w_packed = nullptr;  // device, owned

  Conv1d() = default;
  Conv1d(const Conv1d&) = delete;
  Conv1d& operator=(const Conv1d&) = delete;
  ~Conv1d() {
    if (w_packed) (void)hipFree(w_packed);
  }

  // w_f16: device [o, i, kk] fp16 bits (for example inside a .gsv arena); bias: device or nullptr.
  void load(const uint16_t* w_f16, const float* bias, size_t o, size_t i, size_t kk,
            size_t dil = 1) {
    out_c = o, in_c = i, k = kk, dilation = dil, b = bias;
    const size_t n = gsvk_conv1d_packed_elems(o, i, kk);
    if (!w_packed && hipMalloc(&w_packed, n * 2) != hipSuccess)
      throw std::runtime_error("gsv::sovits::Conv1d::load: hipMalloc failed");
    gsvk::check(gsvk_conv1d_pack(w_f16, o, i, kk, w_packed, n, gsvk::current_stream()),
                "gsv::sovits::Conv1d::load");
  }

  // y[out_c, T] = conv(x[in_c, T]) + b, then the epilogue (x and y must not overlap).
  // res: the residual source of the RES epilogues when it is not cur itself.
  void forward(const float* x, float* y, size_t T, int epi = GSVK_CONV_EPI_BIAS,
               float slope = 0.1f, float* cur = nullptr, const float* res = nullptr) const {
    gsvk::check(gsvk_conv1d(GSVK_F32, 0, x, T, w_packed, b, epi, slope, cur, res, T, y, T, in_c,
                            out_c, T, k, dilation, gsvk::current_stream()),
                "gsv::sovits::Conv1d::forward");
  }
};

// Device-resident ConvT1d (conv1d.hpp:205-360): the torch-layout [in, out, k] weights packed once
// per output phase, forward(x, y) with y [out_c, T * stride_u].
class ConvT1d {
 public:
  size_t out_c = 0, in_c = 0, k = 0, stride_u = 1;
  const float* b = nullptr;
  uint16_t* w_packed = nullptr;

  ConvT1d() = default;
  ConvT1d(const ConvT1d&) = delete;
  ConvT1d& operator=(const ConvT1d&) = delete;
  ~ConvT1d() {
    if (w_packed) (void)hipFree(w_packed);
  }

  void load(const uint16_t* w_f16, const float* bias, size_t i, size_t o, size_t kk, size_t u) {
    in_c = i, out_c = o, k = kk, stride_u = u, b = bias;
    const size_t n = gsvk_convt1d_packed_elems(o, i, kk, u);
    if (!w_packed && hipMalloc(&w_packed, n * 2) != hipSuccess)
      throw std::runtime_error("gsv::sovits::ConvT1d::load: hipMalloc failed");
    gsvk::check(gsvk_convt1d_pack(w_f16, o, i, kk, u, w_packed, n, gsvk::current_stream()),
                "gsv::sovits::ConvT1d::load");
  }

  void forward(const float* x, float* y, size_t T, int epi = GSVK_CONV_EPI_BIAS,
               float slope = 0.1f, float* cur = nullptr, const float* res = nullptr) const {
    gsvk::check(gsvk_convt1d(GSVK_F32, 0, x, T, w_packed, b, epi, slope, cur, res, T * stride_u, y,
                             T * stride_u, in_c, out_c, T, k, stride_u, gsvk::current_stream()),
                "gsv::sovits::ConvT1d::forward");
  }
};

}  // namespace gsv::sovits

namespace gsv::ar {

// T2SEngine::pe_row for every position 0..max_pos-1 into host memory (t2s_engine.cpp:711-720).
inline void pe_table(float* host_out, size_t max_pos, size_t d_model) {
  gsvk::check(gsvk_pe_table(host_out, max_pos, d_model), "gsv::ar::pe_table");
}

// T2SEngine::pe_row(float* pe, size_t pos) (t2s_engine.hpp:187) as a member of anything that
// knows d_model: an engine holding (or deriving from) this keeps its pe_row(pe, pos) call sites.
// Host memory: the rows feed gsvk_embed_pe through a table uploaded once.
struct PeRows {
  size_t d_model = 0;
  void pe_row(float* pe, size_t pos) const {
    gsvk::check(gsvk_pe_row(pe, pos, d_model), "gsv::ar::PeRows::pe_row");
  }
};

// x[r] = e[id_r] + alpha * pe[pos_r] over B rows (t2s_engine.cpp:1781-1786, 1866-1869).
inline void embed_pe(const uint16_t* table_f16, size_t vocab, const int64_t* ids,
                     const int64_t* pos, const float* pe, size_t max_pos, float alpha, float* x,
                     size_t rows, size_t D, int32_t* err = nullptr) {
  gsvk::check(gsvk_embed_pe(GSVK_F32, GSVK_F16, GSVK_I64, table_f16, vocab, ids, pos, 0, pe,
                            max_pos, alpha, nullptr, nullptr, x, rows, D, err,
                            gsvk::current_stream()),
              "gsv::ar::embed_pe");
}

// The prefill input xy[T + P, D] of T2SEngine::generate (t2s_engine.cpp:1770-1786) in one launch:
// text rows xy[t] += (text_emb[phones[t]] + bert_b) then += alpha_text * pe(t), over the bert_proj
// rows already in xy (the reference's order), then prompt rows xy[T + t] = audio_emb[prompt[t]] +
// alpha_audio * pe(t). fp32 activations, fp16 tables, int64 ids, device pointers.
inline void prefill_input(const uint16_t* text_emb_f16, size_t text_vocab, const int64_t* phones,
                          size_t T, const float* bert_b, float alpha_text,
                          const uint16_t* audio_emb_f16, size_t audio_vocab,
                          const int64_t* prompt, size_t P, float alpha_audio, const float* pe,
                          size_t max_pos, float* xy, size_t D, int32_t* err = nullptr) {
  gsvk::check(gsvk_t2s_prefill_input(GSVK_F32, GSVK_F16, GSVK_I64, text_emb_f16, text_vocab,
                                     phones, T, xy, bert_b, alpha_text, audio_emb_f16,
                                     audio_vocab, prompt, P, alpha_audio, pe, max_pos, xy, D, err,
                                     gsvk::current_stream()),
              "gsv::ar::prefill_input");
}

}  // namespace gsv::ar
