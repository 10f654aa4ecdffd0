// gsvk/sovits.hpp — C++ host mirror of the reference's SoVITS decoder classes over the gsvk C ABI:
// gsv::sovits::ResBlock1 and gsv::sovits::Generator (src/sovits/dec.hpp:18-345) with the
// reference's members, load() from a .gsv by the names Generator::load reads (dec.hpp:54-75) and
// forward(z, ge, out) running gsvk_sovits_decoder (103 fused launches).
// Differences, all deliberate: tensors are device pointers ([C, T] channel-major fp32, as
// sovits::Tensor2D lays them out), the .gsv is uploaded to device arenas first (gsvk_gsv_upload),
// forward enqueues on the thread's current stream (gsvk::set_stream) and returns before the GPU
// finishes, no debug dumps, and errors throw std::runtime_error.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "gsvk.h"
#include "gsvk/kern.hpp"
#include "gsvk_gsv.h"
#include "gsvk_sovits.h"

namespace gsv::sovits {

// The .gsv uploaded to the device: both segment arenas, and each tensor by name as
// load_tensor_f16 / load_tensor_f32 take it (sovits_types.hpp:76-87).
class GsvDevice {
 public:
  const gsvk_gsv* f = nullptr;
  void* arena16 = nullptr;
  void* arena32 = nullptr;

  GsvDevice() = default;
  GsvDevice(const GsvDevice&) = delete;
  GsvDevice& operator=(const GsvDevice&) = delete;
  ~GsvDevice() {
    for (void* p : scratch_) (void)hipFree(p);
    if (arena16) (void)hipFree(arena16);
    if (arena32) (void)hipFree(arena32);
  }

  void upload(const gsvk_gsv* file) {
    f = file;
    for (int kind : {GSVK_F16, GSVK_F32}) {
      uint64_t base = 0, bytes = 0;
      gsvk::check(gsvk_gsv_arena(f, kind, &base, &bytes), "GsvDevice::upload");
      void*& arena = kind == GSVK_F16 ? arena16 : arena32;
      if (hipMalloc(&arena, bytes ? bytes : 16) != hipSuccess)
        throw std::runtime_error("GsvDevice::upload: hipMalloc failed");
      if (bytes)
        gsvk::check(gsvk_gsv_upload(f, kind, arena, bytes, gsvk::current_stream()),
                    "GsvDevice::upload");
    }
  }

  bool has(const std::string& name) const { return gsvk_gsv_find(f, name.c_str()) >= 0; }

  // fp16 bits of a weight: the fp16 copy when the file has one, else its fp32 values rounded to
  // fp16 on the device (gsvk_f32_to_f16; kept until this object goes away).
  const uint16_t* f16(const std::string& name) {
    const long i = index(name);
    if (const void* p = gsvk_gsv_device_ptr(f, GSVK_F16, arena16, static_cast<size_t>(i)))
      return static_cast<const uint16_t*>(p);
    const float* src = f32(name);
    gsvk_gsv_tensor t{};
    gsvk::check(gsvk_gsv_tensor_at(f, static_cast<size_t>(i), &t), "GsvDevice::f16");
    void* dst = nullptr;
    if (hipMalloc(&dst, t.numel * 2) != hipSuccess)
      throw std::runtime_error("GsvDevice::f16: hipMalloc failed");
    scratch_.push_back(dst);
    gsvk::check(gsvk_f32_to_f16(src, static_cast<uint16_t*>(dst), t.numel, gsvk::current_stream()),
                "GsvDevice::f16");
    return static_cast<const uint16_t*>(dst);
  }

  // fp32 values (biases), or nullptr when the tensor is absent (conv_post has no bias).
  const float* f32_or_null(const std::string& name) {
    return has(name) ? f32(name) : nullptr;
  }

  const float* f32(const std::string& name) {
    const void* p =
        gsvk_gsv_device_ptr(f, GSVK_F32, arena32, static_cast<size_t>(index(name)));
    if (!p) throw std::runtime_error("missing fp32 data: " + name);
    return static_cast<const float*>(p);
  }

 private:
  long index(const std::string& name) const {
    const long i = gsvk_gsv_find(f, name.c_str());
    if (i < 0) throw std::runtime_error("missing tensor: " + name);
    return i;
  }
  std::vector<void*> scratch_;
};

// ResBlock1 (dec.hpp:18-43): convs1 with dilations {1, 3, 5}, convs2 with dilation 1.
class ResBlock1 {
 public:
  size_t channels = 0, kernel_size = 0;
  Conv1d convs1[3];
  Conv1d convs2[3];

  void load(GsvDevice& f, const std::string& prefix, size_t ch, size_t k,
            const size_t (&dil)[3]) {
    channels = ch, kernel_size = k;
    for (size_t j = 0; j < 3; ++j) {
      const std::string p1 = prefix + ".convs1." + std::to_string(j);
      const std::string p2 = prefix + ".convs2." + std::to_string(j);
      convs1[j].load(f.f16(p1 + ".weight"), f.f32_or_null(p1 + ".bias"), ch, ch, k, dil[j]);
      convs2[j].load(f.f16(p2 + ".weight"), f.f32_or_null(p2 + ".bias"), ch, ch, k, 1);
    }
  }
};

// Generator (dec.hpp:44-345): 768 channels after conv_pre, upsample rates 10, 8, 2, 2, 2 with
// kernels 20, 16, 8, 2, 2, ResBlock1 kernels 3 / 7 / 11; channel counts are read from the
// tensors' shapes. forward(z [c_z, frames], ge [g_in] fp32 column, out [frames * 640]).
class Generator {
 public:
  static constexpr size_t kStages = 5;
  static constexpr size_t kResKernels = 3;
  Conv1d conv_pre;
  ConvT1d ups[kStages];
  ResBlock1 resblocks[kStages][kResKernels];
  Conv1d conv_post;
  const uint16_t* cond_w = nullptr;  // [c0, g_in] fp16 (the k = 1 weight as stored)
  const float* cond_b = nullptr;
  size_t c_z = 0, c0 = 0, g_in = 0;

  Generator() = default;
  Generator(const Generator&) = delete;
  Generator& operator=(const Generator&) = delete;
  ~Generator() {
    if (ws_) (void)hipFree(ws_);
  }

  void load(GsvDevice& f) {
    static const size_t kUpsU[kStages] = {10, 8, 2, 2, 2};
    static const size_t kUpsK[kStages] = {20, 16, 8, 2, 2};
    static const size_t kResK[kResKernels] = {3, 7, 11};
    static const size_t kResDil[3] = {1, 3, 5};
    c0 = dim(f, "dec.conv_pre.weight", 0);
    c_z = dim(f, "dec.conv_pre.weight", 1);
    conv_pre.load(f.f16("dec.conv_pre.weight"), f.f32_or_null("dec.conv_pre.bias"), c0, c_z, 7);
    if (f.has("dec.cond.weight")) {
      g_in = dim(f, "dec.cond.weight", 1);
      cond_w = f.f16("dec.cond.weight");
      cond_b = f.f32_or_null("dec.cond.bias");
    }
    size_t cin = c0;
    for (size_t i = 0; i < kStages; ++i) {
      const size_t cout = cin / 2;
      const std::string up = "dec.ups." + std::to_string(i);
      ups[i].load(f.f16(up + ".weight"), f.f32_or_null(up + ".bias"), cin, cout, kUpsK[i],
                  kUpsU[i]);
      for (size_t j = 0; j < kResKernels; ++j)
        resblocks[i][j].load(f, "dec.resblocks." + std::to_string(i * kResKernels + j), cout,
                             kResK[j], kResDil);
      cin = cout;
    }
    conv_post.load(f.f16("dec.conv_post.weight"), nullptr, 1, cin, 7);
  }

  // z [c_z, frames] -> out [1, frames * 640], values in [-1, 1] (device pointers, fp32).
  void forward(const float* z, size_t frames, const float* ge, float* out) {
    gsvk_sovits_stage st[kStages];
    for (size_t i = 0; i < kStages; ++i) {
      gsvk_sovits_stage& S = st[i];
      S = gsvk_sovits_stage{};
      S.c_in = ups[i].in_c, S.c_out = ups[i].out_c, S.ups_k = ups[i].k, S.ups_u = ups[i].stride_u;
      S.ups_w = ups[i].w_packed, S.ups_b = ups[i].b;
      for (size_t j = 0; j < kResKernels; ++j) {
        const ResBlock1& rb = resblocks[i][j];
        S.res_k[j] = rb.kernel_size;
        for (size_t m = 0; m < 3; ++m) {
          S.res_dil[m] = rb.convs1[m].dilation;
          S.w1[j][m] = rb.convs1[m].w_packed, S.b1[j][m] = rb.convs1[m].b;
          S.w2[j][m] = rb.convs2[m].w_packed, S.b2[j][m] = rb.convs2[m].b;
        }
      }
    }
    gsvk_sovits_decoder_desc d{};
    d.dtype = GSVK_F32;
    d.frames = frames, d.c_z = c_z, d.c0 = c0, d.pre_k = conv_pre.k;
    d.pre_w = conv_pre.w_packed, d.pre_b = conv_pre.b;
    d.g_in = cond_w ? g_in : 0, d.cond_w = cond_w, d.cond_b = cond_b;
    d.n_stages = kStages, d.stage = st;
    d.post_k = conv_post.k, d.post_w = conv_post.w_packed;
    d.z = z, d.ge = cond_w ? ge : nullptr, d.out = out;
    const size_t need = gsvk_sovits_decoder_workspace_bytes(&d);
    if (!need) throw std::runtime_error("gsv::sovits::Generator::forward: bad shapes");
    if (need > ws_bytes_) {  // grows once per longest input (the reference's thread_local scratch)
      if (ws_) (void)hipFree(ws_);
      ws_ = nullptr, ws_bytes_ = 0;
      if (hipMalloc(&ws_, need) != hipSuccess)
        throw std::runtime_error("gsv::sovits::Generator::forward: hipMalloc failed");
      ws_bytes_ = need;
    }
    d.workspace = ws_, d.workspace_bytes = ws_bytes_;
    gsvk::check(gsvk_sovits_decoder_eager(&d, gsvk::current_stream()),
                "gsv::sovits::Generator::forward");
  }

 private:
  static size_t dim(GsvDevice& f, const std::string& name, int axis) {
    gsvk_gsv_tensor t{};
    gsvk::check(gsvk_gsv_tensor_at(f.f, static_cast<size_t>(gsvk_gsv_find(f.f, name.c_str())), &t),
                "gsv::sovits::Generator::load");
    if (axis >= static_cast<int>(t.rank)) throw std::runtime_error("bad rank: " + name);
    return t.dims[axis];
  }
  void* ws_ = nullptr;
  size_t ws_bytes_ = 0;
};

}  // namespace gsv::sovits
