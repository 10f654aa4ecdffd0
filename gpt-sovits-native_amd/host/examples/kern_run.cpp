// kern_run.cpp — the reference-named kernel layer (gsvk/kern.hpp) called the way the reference's
// engines call it, on device buffers, one call per entry point; used by the test suite to check
// the C++ boundary end to end.
//
//   kern_run IN.f32 OUT.f32 R N M
//
// IN.f32 holds, as raw little-endian fp32: x [R, N], g [N], b [N], v [M], w [M], then slope,
// scale, eps (one float each). OUT.f32 receives, in this order:
//   gsv::kern::layernorm(x[0], g, b, y, N, eps)                   N        (kern.hpp:25)
//   gsv::kern::layernorm_rows(x, g, b, y, R, N, eps)              R * N
//   gsv::kern::relu(v, y, M)                                      M        (kern.hpp:33)
//   gsv::sovits::leaky_relu_io(v copy, M, slope)                  M        (nn_ops.hpp:48)
//   gsv::sovits::leaky_relu_write(v, y, M, slope)                 M        (nn_ops.hpp:64)
//   gsv::sovits::add_inplace(v copy, w, M)                        M        (nn_ops.hpp:77)
//   gsv::sovits::add_scaled_inplace(v copy, w, M, scale)          M        (nn_ops.hpp:86)
//   gsv::sovits::mul_write(y, w, M, scale)                        M        (nn_ops.hpp:98)
//   gsv::bert::LayerNorm1D{g, b, 1e-12}.forward(Matrix x)         R * N    (bert_ops.hpp:269)
//   leaky_relu_io(t.d.data(), t.d.size(), 0.01) on Tensor2D t(3, M / 3) of v   3 * (M / 3)
//   gsv::ar::PeRows{N}.pe_row(pe, p), p = 0, 1, 7, 166, 1234, 2047 6 * N   (t2s_engine.hpp:187)
//   gsv::ar::prefill_input(...) (the block at t2s_engine.cpp:1770-1786)      4 R * N
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <exception>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "gsvk/kern.hpp"

namespace {

using gsvk::DeviceVector;

DeviceVector<float> upload(const float* host, size_t n) {
  DeviceVector<float> d;
  d.copy_from_host(host, n);
  return d;
}

void append(std::vector<float>& out, const DeviceVector<float>& d, size_t n) {
  gsvk::sync();
  std::vector<float> h(d.size());
  d.copy_to_host(h.data());
  out.insert(out.end(), h.begin(), h.begin() + static_cast<long>(n));
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 6) {
    std::fprintf(stderr, "usage: %s IN.f32 OUT.f32 R N M\n", argv[0]);
    return 2;
  }
  try {
    const size_t R = std::strtoull(argv[3], nullptr, 10), N = std::strtoull(argv[4], nullptr, 10),
                 M = std::strtoull(argv[5], nullptr, 10);
    const size_t n_in = R * N + 2 * N + 2 * M + 3;
    std::vector<float> in(n_in);
    std::ifstream f(argv[1], std::ios::binary);
    if (!f.read(reinterpret_cast<char*>(in.data()), static_cast<std::streamsize>(n_in * 4)))
      throw std::runtime_error("cannot read the input file");
    const float* x = in.data();
    const float* g = x + R * N;
    const float* b = g + N;
    const float* v = b + N;
    const float* w = v + M;
    const float slope = w[M], scale = w[M + 1], eps = w[M + 2];

    std::vector<float> out;
    DeviceVector<float> X = upload(x, R * N), G = upload(g, N), B = upload(b, N);
    DeviceVector<float> V = upload(v, M), W = upload(w, M), Y(R * N > M ? R * N : M);

    gsv::kern::layernorm(X.data(), G.data(), B.data(), Y.data(), N, eps);
    append(out, Y, N);
    gsv::kern::layernorm_rows(X.data(), G.data(), B.data(), Y.data(), R, N, eps);
    append(out, Y, R * N);
    gsv::kern::relu(V.data(), Y.data(), M);
    append(out, Y, M);
    {
      DeviceVector<float> T = upload(v, M);
      gsv::sovits::leaky_relu_io(T.data(), M, slope);
      append(out, T, M);
    }
    gsv::sovits::leaky_relu_write(V.data(), Y.data(), M, slope);
    append(out, Y, M);
    {
      DeviceVector<float> T = upload(v, M);
      gsv::sovits::add_inplace(T.data(), W.data(), M);
      append(out, T, M);
    }
    {
      DeviceVector<float> T = upload(v, M);
      gsv::sovits::add_scaled_inplace(T.data(), W.data(), M, scale);
      append(out, T, M);
    }
    gsv::sovits::mul_write(Y.data(), W.data(), M, scale);
    append(out, Y, M);
    {
      gsv::bert::Matrix m;
      m.reset(R, N);
      m.d.copy_from_host(x, R * N);
      gsv::bert::LayerNorm1D ln;
      ln.load(g, b, N, 1e-12f);
      ln.forward(m);
      append(out, m.d, R * N);
    }
    {
      gsv::sovits::Tensor2D t(3, M / 3);
      t.d.copy_from_host(v, t.C * t.T);
      gsv::sovits::leaky_relu_io(t.d.data(), t.d.size(), 0.01f);
      append(out, t.d, t.C * t.T);
    }
    {
      const gsv::ar::PeRows rows{N};
      std::vector<float> pe(N);
      for (size_t p : {0ul, 1ul, 7ul, 166ul, 1234ul, 2047ul}) {
        rows.pe_row(pe.data(), p);
        out.insert(out.end(), pe.begin(), pe.end());
      }
    }
    {
      // gsv::ar::prefill_input: both tables are the fp16 rounding of x's R rows, text ids t mod R,
      // prompt ids R - 1 - (t mod R), T = P = 2R; the bert_proj rows already in xy are w's first
      // 2R N values, bias b, alphas 0.75 / 1.25, PE rows 0 .. 2R - 1 of the 2048-row table.
      const size_t T = 2 * R, P = 2 * R;
      if (M < T * N) throw std::runtime_error("prefill_input needs M >= 2 R N");
      DeviceVector<uint16_t> tab(R * N);
      gsvk::check(gsvk_f32_to_f16(X.data(), tab.data(), R * N, gsvk::current_stream()),
                  "gsvk_f32_to_f16");
      std::vector<int64_t> ph(T), pr(P);
      for (size_t t = 0; t < T; ++t) ph[t] = static_cast<int64_t>(t % R);
      for (size_t t = 0; t < P; ++t) pr[t] = static_cast<int64_t>(R - 1 - t % R);
      DeviceVector<int64_t> PH, PR;
      PH.copy_from_host(ph.data(), T);
      PR.copy_from_host(pr.data(), P);
      std::vector<float> pe_host(2048 * N);
      gsv::ar::pe_table(pe_host.data(), 2048, N);
      DeviceVector<float> PE = upload(pe_host.data(), 2048 * N), XY((T + P) * N);
      XY.copy_from_host(w, T * N);
      XY.resize((T + P) * N);
      gsv::ar::prefill_input(tab.data(), R, PH.data(), T, B.data(), 0.75f, tab.data(), R, PR.data(),
                             P, 1.25f, PE.data(), 2048, XY.data(), N);
      append(out, XY, (T + P) * N);
    }
    std::ofstream o(argv[2], std::ios::binary);
    if (!o.write(reinterpret_cast<const char*>(out.data()),
                 static_cast<std::streamsize>(out.size() * 4)))
      throw std::runtime_error("cannot write the output file");
    std::printf("kern_run: %zu floats written\n", out.size());
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "kern_run: %s\n", e.what());
    return 1;
  }
}
