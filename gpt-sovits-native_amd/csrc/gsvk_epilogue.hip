// gsvk_epilogue.hip — bias + activation over rows, LeakyReLU, and the SoVITS ResBlock element-wise
// steps (residual add + LeakyReLU, 3-branch average + next-stage LeakyReLU) for gfx950.
//
// All of these are pure streams: each output element depends on the same element of the inputs
// (plus a per-column bias). Threads move 16-byte chunks; each thread issues UNROLL independent
// chunk loads before it computes and stores, which gives every wave several 1 KiB requests in
// flight. Bit-exactness: every result is the reference's sequence of single-rounded fp32 operations
// (this file is built with -ffp-contract=off, so no multiply-add is fused unless written as fmaf).
#include <cmath>

#include "gsvk_common.hpp"

namespace gsvk {
namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 4;
constexpr long kMaxBlocks = 2048;  // 8 workgroups per CU on 256 CUs; threads stride over the rest

// ---- activations (reference semantics) ----------------------------------------------------------

// vmaxq_f32(x, 0): a NaN input comes out as that NaN made quiet, -0 -> +0 (kern.cpp:85-91,
// vector body).
__device__ __forceinline__ float relu_ref(float v) {
  if (v != v) return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) | 0x00400000u);
  return v > 0.f ? v : 0.f;
}
// v < 0 ? v * slope : v — keeps -0 and NaN (nn_ops.hpp:48-74).
__device__ __forceinline__ float lrelu_ref(float v, float slope) { return v < 0.f ? v * slope : v; }
// 0.5f * x * (1 + erff(x * 0.70710678f)) (bert_ops.hpp:25-27; hubert.cpp:233-236).
__device__ __forceinline__ float gelu_ref(float v) {
  return 0.5f * v * (1.f + erff(v * 0.70710678118654752440f));
}

template <int ACT>
__device__ __forceinline__ float act_apply(float v, float slope) {
  if constexpr (ACT == GSVK_ACT_RELU) return relu_ref(v);
  else if constexpr (ACT == GSVK_ACT_GELU_ERF) return gelu_ref(v);
  else if constexpr (ACT == GSVK_ACT_LEAKY_RELU) return lrelu_ref(v, slope);
  else return v;
}

// ---- bias + activation over [rows, n] ------------------------------------------------------------

struct BaArgs {
  const void* x;
  const float* bias;
  void* y;
  long rows;
  long n;
  long ld;
  float slope;
};

// grid.x covers the 16-byte column chunks of a row, grid.y strides over rows. Each thread keeps its
// bias chunk in VGPRs and walks rows blockIdx.y, +gridDim.y, ... in groups of kUnroll.
template <int DT, int ACT>
__global__ __launch_bounds__(kBlock) void bias_act_vec(BaArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  const long cc = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x;
  if (cc >= a.n / V) return;
  float bi[V];
#pragma unroll
  for (int k = 0; k < V; k += 4) {
    if (a.bias) load_f32x4(a.bias, static_cast<size_t>(cc) * V + k, &bi[k]);
    else bi[k] = bi[k + 1] = bi[k + 2] = bi[k + 3] = 0.f;
  }
  const long step = gridDim.y;
  for (long r0 = blockIdx.y; r0 < a.rows; r0 += step * kUnroll) {
    float v[kUnroll][V];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const long r = r0 + u * step;
      if (r < a.rows) S::load(a.x, static_cast<size_t>(r) * a.ld + cc * V, v[u]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const long r = r0 + u * step;
      if (r < a.rows) {
#pragma unroll
        for (int k = 0; k < V; ++k) v[u][k] = act_apply<ACT>(v[u][k] + bi[k], a.slope);
        S::store(a.y, static_cast<size_t>(r) * a.ld + cc * V, v[u]);
      }
    }
  }
}

template <int DT, int ACT>
__global__ __launch_bounds__(kBlock) void bias_act_generic(BaArgs a) {
  using S = Store<DT>;
  const long total = a.rows * a.n;
  const long stride = static_cast<long>(gridDim.x) * kBlock;
  for (long i = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride) {
    const long r = i / a.n, c = i - r * a.n;
    const size_t off = static_cast<size_t>(r) * a.ld + c;
    const float b = a.bias ? a.bias[c] : 0.f;
    S::store1(a.y, off, act_apply<ACT>(S::load1(a.x, off) + b, a.slope));
  }
}

// ---- flat element-wise streams -------------------------------------------------------------------

struct EwArgs {
  const void* in[8];  // operands (see each kernel)
  void* out[2];
  long n;
  float slope;
  int flag;
  int nbranch;
};

// Each thread handles kUnroll chunks spaced one grid-stride apart, then moves kUnroll strides on.
// Elements past the last whole chunk are done one per thread by the scalar tail pass.
template <typename Body>
__device__ __forceinline__ void flat_chunks(long nchunks, Body body) {
  const long stride = static_cast<long>(gridDim.x) * kBlock;
  for (long c0 = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; c0 < nchunks;
       c0 += stride * kUnroll)
    body(c0, stride);
}

// y = lrelu(x, slope)
template <int DT>
__global__ __launch_bounds__(kBlock) void lrelu_vec(EwArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  const long nch = a.n / V;
  flat_chunks(nch, [&](long c0, long stride) {
    float v[kUnroll][V];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (c0 + u * stride < nch) S::load(a.in[0], (c0 + u * stride) * V, v[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (c0 + u * stride < nch) {
#pragma unroll
        for (int k = 0; k < V; ++k) v[u][k] = lrelu_ref(v[u][k], a.slope);
        S::store(a.out[0], (c0 + u * stride) * V, v[u]);
      }
  });
  const long i = nch * V + static_cast<long>(blockIdx.x) * kBlock + threadIdx.x;
  if (i < a.n) S::store1(a.out[0], i, lrelu_ref(S::load1(a.in[0], i), a.slope));
}

// cur += t_b; t_in = lrelu(cur)   (flag = 1 when t_in is written)
template <int DT>
__global__ __launch_bounds__(kBlock) void res_add_lrelu_vec(EwArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  const long nch = a.n / V;
  void* cur = a.out[0];
  void* tin = a.out[1];
  flat_chunks(nch, [&](long c0, long stride) {
    float c[kUnroll][V], t[kUnroll][V];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (c0 + u * stride < nch) {
        S::load(cur, (c0 + u * stride) * V, c[u]);
        S::load(a.in[0], (c0 + u * stride) * V, t[u]);
      }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (c0 + u * stride < nch) {
#pragma unroll
        for (int k = 0; k < V; ++k) c[u][k] = c[u][k] + t[u][k];
        S::store(cur, (c0 + u * stride) * V, c[u]);
        if (a.flag) {
#pragma unroll
          for (int k = 0; k < V; ++k) t[u][k] = lrelu_ref(c[u][k], a.slope);
          S::store(tin, (c0 + u * stride) * V, t[u]);
        }
      }
  });
  const long i = nch * V + static_cast<long>(blockIdx.x) * kBlock + threadIdx.x;
  if (i < a.n) {
    const float v = S::load1(cur, i) + S::load1(a.in[0], i);
    S::store1(cur, i, v);
    if (a.flag) S::store1(tin, i, lrelu_ref(v, a.slope));
  }
}

// out = lrelu( sum_j (cur_j [+ tb_j]) * kinv ), summed left to right with separate roundings.
// in[0..3] = cur_j, in[4..7] = tb_j (NULL when absent); flag = apply_lrelu. All 2*NB operand
// chunks of U chunk positions are loaded before any arithmetic, so U*2*NB loads are in flight.
template <int DT, int NB>
__global__ __launch_bounds__(kBlock) void branch_mean_vec(EwArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  constexpr int U = DT == GSVK_F32 ? kUnroll : kUnroll / 2;
  constexpr float kInv = 1.f / static_cast<float>(NB);
  const long nch = a.n / V;
  const long stride = static_cast<long>(gridDim.x) * kBlock;
  for (long c0 = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; c0 < nch; c0 += stride * U) {
    float cv[U][NB][V], tv[U][NB][V];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long c = c0 + u * stride;
      if (c < nch) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          S::load(a.in[j], c * V, cv[u][j]);
          if (a.in[4 + j]) S::load(a.in[4 + j], c * V, tv[u][j]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long c = c0 + u * stride;
      if (c < nch) {
        float acc[V];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const bool has_t = a.in[4 + j] != nullptr;
#pragma unroll
          for (int k = 0; k < V; ++k) {
            const float v = has_t ? cv[u][j][k] + tv[u][j][k] : cv[u][j][k];
            acc[k] = j == 0 ? v * kInv : acc[k] + v * kInv;
          }
        }
        if (a.flag) {
#pragma unroll
          for (int k = 0; k < V; ++k) acc[k] = lrelu_ref(acc[k], a.slope);
        }
        S::store(a.out[0], c * V, acc);
      }
    }
  }
  const long i = nch * V + static_cast<long>(blockIdx.x) * kBlock + threadIdx.x;
  if (i < a.n) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      float v = S::load1(a.in[j], i);
      if (a.in[4 + j]) v = v + S::load1(a.in[4 + j], i);
      acc = j == 0 ? v * kInv : acc + v * kInv;
    }
    S::store1(a.out[0], i, a.flag ? lrelu_ref(acc, a.slope) : acc);
  }
}

// out = acc + src * scale (acc optional); in[0] = acc, in[1] = src, slope carries the scale.
template <int DT>
__global__ __launch_bounds__(kBlock) void scaled_add_vec(EwArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  const long nch = a.n / V;
  const bool has_acc = a.in[0] != nullptr;
  flat_chunks(nch, [&](long c0, long stride) {
    float s[kUnroll][V], q[kUnroll][V];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (c0 + u * stride < nch) {
        S::load(a.in[1], (c0 + u * stride) * V, s[u]);
        if (has_acc) S::load(a.in[0], (c0 + u * stride) * V, q[u]);
      }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (c0 + u * stride < nch) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
          const float v = s[u][k] * a.slope;
          s[u][k] = has_acc ? q[u][k] + v : v;
        }
        S::store(a.out[0], (c0 + u * stride) * V, s[u]);
      }
  });
  const long i = nch * V + static_cast<long>(blockIdx.x) * kBlock + threadIdx.x;
  if (i < a.n) {
    const float v = S::load1(a.in[1], i) * a.slope;
    S::store1(a.out[0], i, has_acc ? S::load1(a.in[0], i) + v : v);
  }
}

// Scalar fallbacks for buffers that are not 16-byte aligned.
template <int DT>
__global__ __launch_bounds__(kBlock) void ew_scalar(EwArgs a, int op) {
  using S = Store<DT>;
  const long stride = static_cast<long>(gridDim.x) * kBlock;
  for (long i = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; i < a.n; i += stride) {
    if (op == 0) {
      S::store1(a.out[0], i, lrelu_ref(S::load1(a.in[0], i), a.slope));
    } else if (op == 1) {
      const float v = S::load1(a.out[0], i) + S::load1(a.in[0], i);
      S::store1(a.out[0], i, v);
      if (a.flag) S::store1(a.out[1], i, lrelu_ref(v, a.slope));
    } else if (op == 3) {
      const float v = S::load1(a.in[1], i) * a.slope;
      S::store1(a.out[0], i, a.in[0] ? S::load1(a.in[0], i) + v : v);
    } else {
      const float kinv = 1.f / static_cast<float>(a.nbranch);
      float acc = 0.f;
      for (int j = 0; j < a.nbranch; ++j) {
        float v = S::load1(a.in[j], i);
        if (a.in[4 + j]) v = v + S::load1(a.in[4 + j], i);
        acc = j == 0 ? v * kinv : acc + v * kinv;
      }
      S::store1(a.out[0], i, a.flag ? lrelu_ref(acc, a.slope) : acc);
    }
  }
}

// ---- launch helpers -------------------------------------------------------------------------------

unsigned flat_grid(long nchunks) {
  long b = (nchunks + kBlock - 1) / kBlock;
  if (b < 1) b = 1;  // the tail pass needs one block even when there is no whole chunk
  return static_cast<unsigned>(b < kMaxBlocks ? b : kMaxBlocks);
}

template <int ACT>
int launch_bias_act(int dt, const BaArgs& a, bool vec_ok, hipStream_t st) {
  const int V = dt == GSVK_F32 ? 4 : 8;
  if (vec_ok) {
    const long nch = a.n / V;
    const unsigned gx = static_cast<unsigned>((nch + kBlock - 1) / kBlock);
    long gy = kMaxBlocks / gx;
    if (gy < 1) gy = 1;
    if (gy > a.rows) gy = a.rows;
    if (gy > 65535) gy = 65535;
    const dim3 grid(gx, static_cast<unsigned>(gy));
    switch (dt) {
      case GSVK_F32: hipLaunchKernelGGL((bias_act_vec<GSVK_F32, ACT>), grid, dim3(kBlock), 0, st, a); break;
      case GSVK_F16: hipLaunchKernelGGL((bias_act_vec<GSVK_F16, ACT>), grid, dim3(kBlock), 0, st, a); break;
      default: hipLaunchKernelGGL((bias_act_vec<GSVK_BF16, ACT>), grid, dim3(kBlock), 0, st, a); break;
    }
  } else {
    const unsigned g = flat_grid(a.rows * a.n);
    switch (dt) {
      case GSVK_F32: hipLaunchKernelGGL((bias_act_generic<GSVK_F32, ACT>), dim3(g), dim3(kBlock), 0, st, a); break;
      case GSVK_F16: hipLaunchKernelGGL((bias_act_generic<GSVK_F16, ACT>), dim3(g), dim3(kBlock), 0, st, a); break;
      default: hipLaunchKernelGGL((bias_act_generic<GSVK_BF16, ACT>), dim3(g), dim3(kBlock), 0, st, a); break;
    }
  }
  return launch_status();
}

template <int DT>
void launch_scalar(const EwArgs& a, int op, hipStream_t st) {
  hipLaunchKernelGGL((ew_scalar<DT>), dim3(flat_grid(a.n)), dim3(kBlock), 0, st, a, op);
}

void launch_scalar_dt(int dt, const EwArgs& a, int op, hipStream_t st) {
  switch (dt) {
    case GSVK_F32: launch_scalar<GSVK_F32>(a, op, st); break;
    case GSVK_F16: launch_scalar<GSVK_F16>(a, op, st); break;
    default: launch_scalar<GSVK_BF16>(a, op, st); break;
  }
}

template <int DT>
void launch_branch_mean(const EwArgs& a, hipStream_t st) {
  const unsigned g = flat_grid(a.n / Store<DT>::VEC);
  switch (a.nbranch) {
    case 1: hipLaunchKernelGGL((branch_mean_vec<DT, 1>), dim3(g), dim3(kBlock), 0, st, a); break;
    case 2: hipLaunchKernelGGL((branch_mean_vec<DT, 2>), dim3(g), dim3(kBlock), 0, st, a); break;
    case 3: hipLaunchKernelGGL((branch_mean_vec<DT, 3>), dim3(g), dim3(kBlock), 0, st, a); break;
    default: hipLaunchKernelGGL((branch_mean_vec<DT, 4>), dim3(g), dim3(kBlock), 0, st, a); break;
  }
}

}  // namespace
}  // namespace gsvk

using namespace gsvk;

extern "C" int gsvk_bias_act(int dtype, int act, const void* x, const float* bias, void* y,
                             size_t rows, size_t n, size_t ld, float slope, void* stream) {
  if (!valid_dtype(dtype)) return GSVK_E_DTYPE;
  if (act < GSVK_ACT_NONE || act > GSVK_ACT_LEAKY_RELU) return GSVK_E_DTYPE;
  if (!x || !y) return GSVK_E_NULL;
  if (rows == 0 || n == 0 || ld < n || rows > (1ul << 40) || n > (1ul << 40)) return GSVK_E_SIZE;
  const size_t esz = dtype_size(dtype);
  const size_t span = span_bytes(rows, n, ld, esz);
  if (y != x && overlaps(y, span, x, span)) return GSVK_E_ALIAS;
  if (bias && overlaps(y, span, bias, n * sizeof(float))) return GSVK_E_ALIAS;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % esz) return GSVK_E_ARG;
  const int V = dtype == GSVK_F32 ? 4 : 8;
  const bool vec_ok = n % V == 0 && ld % V == 0 && aligned16(x) && aligned16(y) &&
                      (!bias || aligned16(bias));
  BaArgs a{x, bias, y, static_cast<long>(rows), static_cast<long>(n), static_cast<long>(ld), slope};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (act) {
    case GSVK_ACT_NONE: return launch_bias_act<GSVK_ACT_NONE>(dtype, a, vec_ok, st);
    case GSVK_ACT_RELU: return launch_bias_act<GSVK_ACT_RELU>(dtype, a, vec_ok, st);
    case GSVK_ACT_GELU_ERF: return launch_bias_act<GSVK_ACT_GELU_ERF>(dtype, a, vec_ok, st);
    default: return launch_bias_act<GSVK_ACT_LEAKY_RELU>(dtype, a, vec_ok, st);
  }
}

extern "C" int gsvk_leaky_relu(int dtype, const void* x, void* y, size_t n, float slope,
                               void* stream) {
  if (!valid_dtype(dtype)) return GSVK_E_DTYPE;
  if (!x || !y) return GSVK_E_NULL;
  if (n == 0 || n > (1ul << 40)) return GSVK_E_SIZE;
  const size_t esz = dtype_size(dtype);
  if (y != x && overlaps(y, n * esz, x, n * esz)) return GSVK_E_ALIAS;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % esz) return GSVK_E_ARG;
  EwArgs a{};
  a.in[0] = x;
  a.out[0] = y;
  a.n = static_cast<long>(n);
  a.slope = slope;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (aligned16(x) && aligned16(y)) {
    const unsigned g = flat_grid(a.n / (dtype == GSVK_F32 ? 4 : 8));
    switch (dtype) {
      case GSVK_F32: hipLaunchKernelGGL((lrelu_vec<GSVK_F32>), dim3(g), dim3(kBlock), 0, st, a); break;
      case GSVK_F16: hipLaunchKernelGGL((lrelu_vec<GSVK_F16>), dim3(g), dim3(kBlock), 0, st, a); break;
      default: hipLaunchKernelGGL((lrelu_vec<GSVK_BF16>), dim3(g), dim3(kBlock), 0, st, a); break;
    }
  } else {
    launch_scalar_dt(dtype, a, 0, st);
  }
  return launch_status();
}

extern "C" int gsvk_resblock_add_lrelu(int dtype, void* cur, const void* t_b, void* t_in, size_t n,
                                       float slope, void* stream) {
  if (!valid_dtype(dtype)) return GSVK_E_DTYPE;
  if (!cur || !t_b) return GSVK_E_NULL;
  if (n == 0 || n > (1ul << 40)) return GSVK_E_SIZE;
  const size_t esz = dtype_size(dtype), bytes = n * esz;
  if (overlaps(cur, bytes, t_b, bytes) || overlaps(t_in, bytes, cur, bytes) ||
      overlaps(t_in, bytes, t_b, bytes))
    return GSVK_E_ALIAS;
  if ((reinterpret_cast<uintptr_t>(cur) | reinterpret_cast<uintptr_t>(t_b) |
       reinterpret_cast<uintptr_t>(t_in)) % esz)
    return GSVK_E_ARG;
  EwArgs a{};
  a.in[0] = t_b;
  a.out[0] = cur;
  a.out[1] = t_in;
  a.n = static_cast<long>(n);
  a.slope = slope;
  a.flag = t_in != nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (aligned16(cur) && aligned16(t_b) && (!t_in || aligned16(t_in))) {
    const unsigned g = flat_grid(a.n / (dtype == GSVK_F32 ? 4 : 8));
    switch (dtype) {
      case GSVK_F32: hipLaunchKernelGGL((res_add_lrelu_vec<GSVK_F32>), dim3(g), dim3(kBlock), 0, st, a); break;
      case GSVK_F16: hipLaunchKernelGGL((res_add_lrelu_vec<GSVK_F16>), dim3(g), dim3(kBlock), 0, st, a); break;
      default: hipLaunchKernelGGL((res_add_lrelu_vec<GSVK_BF16>), dim3(g), dim3(kBlock), 0, st, a); break;
    }
  } else {
    launch_scalar_dt(dtype, a, 1, st);
  }
  return launch_status();
}

extern "C" int gsvk_resblock_branch_mean(int dtype, const void* const* cur, const void* const* t_b,
                                         int nbranch, void* out, size_t n, int apply_lrelu,
                                         float slope, void* stream) {
  if (!valid_dtype(dtype)) return GSVK_E_DTYPE;
  if (!cur || !out) return GSVK_E_NULL;
  if (nbranch < 1 || nbranch > 4) return GSVK_E_ARG;
  if (n == 0 || n > (1ul << 40)) return GSVK_E_SIZE;
  const size_t esz = dtype_size(dtype), bytes = n * esz;
  EwArgs a{};
  bool aligned = aligned16(out);
  uintptr_t ormask = reinterpret_cast<uintptr_t>(out);
  for (int j = 0; j < nbranch; ++j) {
    if (!cur[j]) return GSVK_E_NULL;
    a.in[j] = cur[j];
    a.in[4 + j] = t_b ? t_b[j] : nullptr;
    for (const void* p : {a.in[j], a.in[4 + j]}) {
      if (!p) continue;
      if (overlaps(out, bytes, p, bytes)) return GSVK_E_ALIAS;
      aligned = aligned && aligned16(p);
      ormask |= reinterpret_cast<uintptr_t>(p);
    }
  }
  if (ormask % esz) return GSVK_E_ARG;
  a.out[0] = out;
  a.n = static_cast<long>(n);
  a.slope = slope;
  a.flag = apply_lrelu ? 1 : 0;
  a.nbranch = nbranch;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (aligned) {
    switch (dtype) {
      case GSVK_F32: launch_branch_mean<GSVK_F32>(a, st); break;
      case GSVK_F16: launch_branch_mean<GSVK_F16>(a, st); break;
      default: launch_branch_mean<GSVK_BF16>(a, st); break;
    }
  } else {
    launch_scalar_dt(dtype, a, 2, st);
  }
  return launch_status();
}

extern "C" int gsvk_scaled_add(int dtype, const void* acc, const void* src, void* out, size_t n,
                               float scale, void* stream) {
  if (!valid_dtype(dtype)) return GSVK_E_DTYPE;
  if (!src || !out) return GSVK_E_NULL;
  if (n == 0 || n > (1ul << 40)) return GSVK_E_SIZE;
  const size_t esz = dtype_size(dtype), bytes = n * esz;
  if (overlaps(out, bytes, src, bytes)) return GSVK_E_ALIAS;
  if (acc && acc != out && overlaps(out, bytes, acc, bytes)) return GSVK_E_ALIAS;
  if ((reinterpret_cast<uintptr_t>(acc) | reinterpret_cast<uintptr_t>(src) |
       reinterpret_cast<uintptr_t>(out)) % esz)
    return GSVK_E_ARG;
  EwArgs a{};
  a.in[0] = acc;
  a.in[1] = src;
  a.out[0] = out;
  a.n = static_cast<long>(n);
  a.slope = scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (aligned16(src) && aligned16(out) && (!acc || aligned16(acc))) {
    const unsigned g = flat_grid(a.n / (dtype == GSVK_F32 ? 4 : 8));
    switch (dtype) {
      case GSVK_F32: hipLaunchKernelGGL((scaled_add_vec<GSVK_F32>), dim3(g), dim3(kBlock), 0, st, a); break;
      case GSVK_F16: hipLaunchKernelGGL((scaled_add_vec<GSVK_F16>), dim3(g), dim3(kBlock), 0, st, a); break;
      default: hipLaunchKernelGGL((scaled_add_vec<GSVK_BF16>), dim3(g), dim3(kBlock), 0, st, a); break;
    }
  } else {
    launch_scalar_dt(dtype, a, 3, st);
  }
  return launch_status();
}
