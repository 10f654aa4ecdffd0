// sovits_run.cpp — the C++ host mirror used as an engine would use it: load a SoVITS .gsv, bind
// gsv::sovits::Generator (the reference's dec.hpp:44-345 class) to its tensors and run one decoder
// pass on the GPU.
//
//   sovits_run MODEL.gsv Z.f32 FRAMES GE.f32|- OUT.f32
//
// Z.f32 holds z [c_z, FRAMES] and GE.f32 the speaker vector ge [g_in] ("-": the model has no cond),
// both raw little-endian fp32; OUT.f32 receives the waveform [FRAMES * 640] fp32.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <exception>
#include <fstream>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "gsvk/sovits.hpp"

namespace {

std::vector<float> read_f32(const char* path, size_t n) {
  std::ifstream f(path, std::ios::binary);
  std::vector<float> v(n);
  if (!f.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(n * sizeof(float))))
    throw std::runtime_error(std::string("cannot read ") + std::to_string(n) + " floats from " +
                             path);
  return v;
}

struct DeviceBuf {
  void* p = nullptr;
  explicit DeviceBuf(size_t bytes) {
    if (hipMalloc(&p, bytes) != hipSuccess) throw std::runtime_error("hipMalloc failed");
  }
  ~DeviceBuf() { (void)hipFree(p); }
  float* f() const { return static_cast<float*>(p); }
};

void to_device(const std::vector<float>& h, const DeviceBuf& d) {
  if (hipMemcpy(d.p, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
    throw std::runtime_error("hipMemcpy to device failed");
}

int run(int argc, char** argv) {
  if (argc != 6) {
    std::fprintf(stderr, "usage: %s MODEL.gsv Z.f32 FRAMES GE.f32|- OUT.f32\n", argv[0]);
    return 2;
  }
  const size_t frames = std::strtoull(argv[3], nullptr, 10);
  if (frames == 0) throw std::runtime_error("FRAMES must be positive");

  gsvk_gsv* file = nullptr;
  gsvk::check(gsvk_gsv_open(argv[1], &file), "gsvk_gsv_open");
  std::unique_ptr<gsvk_gsv, void (*)(gsvk_gsv*)> file_guard(file, gsvk_gsv_close);

  gsv::sovits::GsvDevice weights;
  weights.upload(file);
  gsv::sovits::Generator dec;
  dec.load(weights);

  const std::vector<float> z = read_f32(argv[2], dec.c_z * frames);
  DeviceBuf z_d(z.size() * sizeof(float));
  to_device(z, z_d);
  const bool has_ge = std::string(argv[4]) != "-";
  if (dec.cond_w && !has_ge) throw std::runtime_error("the model has cond: GE.f32 is required");
  std::vector<float> ge = has_ge ? read_f32(argv[4], dec.g_in) : std::vector<float>(1, 0.f);
  DeviceBuf ge_d(ge.size() * sizeof(float));
  to_device(ge, ge_d);

  const size_t n_out = frames * 640;
  DeviceBuf out_d(n_out * sizeof(float));
  dec.forward(z_d.f(), frames, ge_d.f(), out_d.f());
  gsvk::sync();

  std::vector<float> out(n_out);
  if (hipMemcpy(out.data(), out_d.p, n_out * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess)
    throw std::runtime_error("hipMemcpy to host failed");
  std::ofstream o(argv[5], std::ios::binary);
  o.write(reinterpret_cast<const char*>(out.data()),
          static_cast<std::streamsize>(n_out * sizeof(float)));
  if (!o) throw std::runtime_error(std::string("cannot write ") + argv[5]);
  std::printf("sovits_run: %zu frames -> %zu samples\n", frames, n_out);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    return run(argc, argv);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "sovits_run: %s\n", e.what());
    return 1;
  }
}
