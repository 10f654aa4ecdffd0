// gsvk_gemv.hip — batched decode GEMV with fp16 weights on the gfx950 matrix cores, with the bias /
// activation / residual epilogue fused into the store.
//
// y[r, n] = act(sum_k float(w[n, k]) * x[r, k] + bias[n]) (+ residual[r, n]), for B sequences
// (rows) at once. At B = 64 a weight element feeds 64 multiply-adds: 64 flop per weight byte,
// above the fp32 VALU ridge of MI355X (157 TFLOP/s / 8 TB/s = 20) and far below the fp16 matrix
// core one (2.5 PFLOP/s / 8 TB/s = 312), so the products go to v_mfma_f32_16x16x32_f16 and the
// kernel stays bound by the weight stream from HBM.
//
// Tiles. Operand A of one MFMA is a 16 x 32 slice of W (16 output columns n, 32 k), operand B a
// 32 x 16 slice of X^T (32 k, 16 rows r): lane l feeds row/column (l & 15) with the 8 k values of
// its lane group (l >> 4). The accumulator then holds, in lane l, four consecutive outputs
// n = 4 (l >> 4) .. +3 of row (l & 15), stored as one vector. A and B use the same k slots, so
// which 8 k a lane group holds is free: lane group g holds k = 64 kb + 16 g + 8 h .. +7 for the two
// MFMAs h = 0, 1 of a 64-wide k block, which makes every wave load 128 contiguous bytes of each
// weight row per k block.
// A workgroup covers 64 rows x 16 NF columns; its WK waves split K into contiguous ranges and their
// partial sums are added in wave order through LDS (a fixed order: results do not depend on
// timing). Products fp16 x fp16 are exact in fp32; the sum is fp32.
//
// x in fp32: round_x = 1 rounds it to fp16 first (T2SEngine::gemv_fmlal, t2s_engine.cpp:696-700);
// round_x = 0 keeps the fp32 value (kern::gemv_f16w_f32acc, gemv.cpp:112-127) by feeding
// hi = f16(x) and lo = f16(x - hi) through two MFMAs: x - hi is exact and lo holds the next 11
// bits, so hi + lo equals x to about 2^-22 relative (|x| < 65504).
#include <algorithm>

#include "gsvk_common.hpp"

namespace gsvk {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f8v __attribute__((ext_vector_type(8)));

enum XMode { kXF16 = 0, kXRound = 1, kXSplit = 2 };

constexpr int kRowsPerGroup = 64;  // 4 fragments of 16 rows
constexpr long kMaxRowGroups = 65535;

struct GvArgs {
  const void* x;
  const uint16_t* w;
  const float* bias;
  const void* res;
  void* y;
  long M, N, K, ldx, ldy;
  int act;
  int ydt;
  float slope;
  bool vec_store;
};

// 8 consecutive k of one weight row; zero when the k block lies past K (the address is clamped to
// the row's last 8 values, so the load itself stays in bounds and outside any branch).
__device__ __forceinline__ h8 load_w8(const uint16_t* w, size_t off, bool ok) {
  u32x4 q = ld16<false>(w + off);
  if (!ok) q = u32x4{0u, 0u, 0u, 0u};
  return __builtin_bit_cast(h8, q);
}

// 8 consecutive k of one activation row as fp16 (hi) and, in split mode, the fp16 remainder (lo).
template <int XM>
__device__ __forceinline__ void load_x8(const void* x, size_t off, bool ok, h8& hi, h8& lo) {
  if constexpr (XM == kXF16) {
    u32x4 q = ld16<false>(static_cast<const uint16_t*>(x) + off);
    if (!ok) q = u32x4{0u, 0u, 0u, 0u};
    hi = __builtin_bit_cast(h8, q);
  } else {
    const float* p = static_cast<const float*>(x) + off;
    const u32x4 q0 = ld16<false>(p), q1 = ld16<false>(p + 4);
    uint32_t u[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      u[k] = q0[k];
      u[4 + k] = q1[k];
    }
    f8v f;
#pragma unroll
    for (int k = 0; k < 8; ++k) f[k] = ok ? __builtin_bit_cast(float, u[k]) : 0.f;
    hi = __builtin_convertvector(f, h8);
    if constexpr (XM == kXSplit) {
      const f8v rest = f - __builtin_convertvector(hi, f8v);
      lo = __builtin_convertvector(rest, h8);
    }
  }
}

__device__ __forceinline__ float act_rt(int act, float v, float slope) {
  switch (act) {
    case GSVK_ACT_RELU: return relu_ref(v);
    case GSVK_ACT_GELU_ERF: return gelu_erf(v);
    case GSVK_ACT_LEAKY_RELU: return lrelu_ref(v, slope);
    default: return v;
  }
}

__device__ __forceinline__ float load_y(int dt, const void* p, size_t i) {
  switch (dt) {
    case GSVK_F32: return static_cast<const float*>(p)[i];
    case GSVK_F16: return h2f(static_cast<const uint16_t*>(p)[i]);
    default: return bf2f(static_cast<const uint16_t*>(p)[i]);
  }
}

__device__ __forceinline__ void store_y(int dt, void* p, size_t i, float v) {
  switch (dt) {
    case GSVK_F32: static_cast<float*>(p)[i] = v; break;
    case GSVK_F16: static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f2h(v)); break;
    default: static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f2bf(v)); break;
  }
}

// One output: v = act(acc + bias[n]) (+ residual[m, n]). The bias add is skipped, not replaced by
// + 0, when there is no bias (x + 0 would turn -0 into +0).
__device__ __forceinline__ float epilogue(const GvArgs& a, long m, long n, float v) {
  if (a.bias) v = v + a.bias[n];
  v = act_rt(a.act, v, a.slope);
  if (a.res) v = v + load_y(a.ydt, a.res, static_cast<size_t>(m) * a.ldy + n);
  return v;
}

// Four consecutive outputs n .. n+3 of row m.
__device__ __forceinline__ void finish4(const GvArgs& a, long m, long n, f4v s) {
  if (m >= a.M) return;
  const size_t off = static_cast<size_t>(m) * a.ldy + n;
  if (a.vec_store && n + 4 <= a.N) {
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = epilogue(a, m, n + q, s[q]);
    if (a.ydt == GSVK_F32) {
      *reinterpret_cast<float4*>(static_cast<float*>(a.y) + off) = float4{v[0], v[1], v[2], v[3]};
    } else {
      uint32_t h[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) h[q] = a.ydt == GSVK_F16 ? f2h(v[q]) : f2bf(v[q]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.y) + off) =
          uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if (n + q < a.N) store_y(a.ydt, a.y, off + q, epilogue(a, m, n + q, s[q]));
}

template <int XM, int NF, int WK>
__global__ __launch_bounds__(kWave * WK) void gemv_mfma(GvArgs a) {
  __shared__ f4v red[WK > 1 ? WK : 1][4 * NF][kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int r16 = lane & 15, grp = lane >> 4;
  const long m0 = static_cast<long>(blockIdx.y) * kRowsPerGroup;
  const long n0 = static_cast<long>(blockIdx.x) * (16 * NF);
  const long nkb = (a.K + 63) >> 6;
  const long per = (nkb + WK - 1) / WK;
  const long kb0 = min(nkb, wave * per), kb1 = min(nkb, kb0 + per);

  size_t xoff[4], woff[NF];
#pragma unroll
  for (int i = 0; i < 4; ++i) xoff[i] = static_cast<size_t>(min(m0 + 16 * i + r16, a.M - 1)) * a.ldx;
#pragma unroll
  for (int j = 0; j < NF; ++j) woff[j] = static_cast<size_t>(min(n0 + 16 * j + r16, a.N - 1)) * a.K;

  f4v acc[4][NF];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};

  // Fragments of one 64-wide k block: [h][j] weights, [h][i] activations.
  h8 wv[2][NF], xh[2][4], xl[2][4];
  auto load = [&](long kb) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const long k = kb * 64 + grp * 16 + h * 8;
      const bool ok = k < a.K;
      const size_t kc = static_cast<size_t>(ok ? k : a.K - 8);
#pragma unroll
      for (int j = 0; j < NF; ++j) wv[h][j] = load_w8(a.w, woff[j] + kc, ok);
#pragma unroll
      for (int i = 0; i < 4; ++i) load_x8<XM>(a.x, xoff[i] + kc, ok, xh[h][i], xl[h][i]);
    }
  };
  for (long kb = kb0; kb < kb1; ++kb) {
    load(kb);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv[h][j], xh[h][i], acc[i][j], 0, 0, 0);
          if constexpr (XM == kXSplit)
            acc[i][j] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(wv[h][j], xl[h][i], acc[i][j], 0, 0, 0);
        }
  }

  if constexpr (WK == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NF; ++j)
        finish4(a, m0 + 16 * i + r16, n0 + 16 * j + 4 * grp, acc[i][j]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NF; ++j) red[wave][i * NF + j][lane] = acc[i][j];
    __syncthreads();
    for (int t = wave; t < 4 * NF; t += WK) {
      f4v s = red[0][t][lane];
#pragma unroll
      for (int w = 1; w < WK; ++w) s = s + red[w][t][lane];
      const int i = t / NF, j = t % NF;
      finish4(a, m0 + 16 * i + r16, n0 + 16 * j + 4 * grp, s);
    }
  }
}

// Any shape or alignment: one thread per output, k in order with fmaf (the product of an fp16
// weight and an fp16 or fp32 activation is formed exactly or rounded once, then added: the
// reference's vfmaq / fmlal step). Used when K % 8 != 0 or a row is not 16-byte aligned.
template <int XM>
__global__ __launch_bounds__(256) void gemv_generic(GvArgs a) {
  const long total = a.M * a.N;
  for (long t = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
       t += static_cast<long>(gridDim.x) * blockDim.x) {
    const long m = t / a.N, n = t % a.N;
    const uint16_t* wr = a.w + static_cast<size_t>(n) * a.K;
    const size_t xr = static_cast<size_t>(m) * a.ldx;
    float s = 0.f;
    for (long k = 0; k < a.K; ++k) {
      float xv;
      if constexpr (XM == kXF16) {
        xv = h2f(static_cast<const uint16_t*>(a.x)[xr + k]);
      } else {
        xv = static_cast<const float*>(a.x)[xr + k];
        if constexpr (XM == kXRound) xv = h2f(f2h(xv));
      }
      s = __builtin_fmaf(h2f(wr[k]), xv, s);
    }
    store_y(a.ydt, a.y, static_cast<size_t>(m) * a.ldy + n, epilogue(a, m, n, s));
  }
}

template <int XM, int NF, int WK>
void launch_tiles(const GvArgs& a, hipStream_t st) {
  const long gx = (a.N + 16 * NF - 1) / (16 * NF);
  const long gy = (a.M + kRowsPerGroup - 1) / kRowsPerGroup;
  hipLaunchKernelGGL((gemv_mfma<XM, NF, WK>), dim3(static_cast<unsigned>(gx),
                                                   static_cast<unsigned>(gy)),
                     dim3(kWave * WK), 0, st, a);
}

template <int XM>
void launch_xm(const GvArgs& a, bool tiled, hipStream_t st) {
  if (!tiled) {
    const long blocks = std::min<long>((a.M * a.N + 255) / 256, 4096);
    hipLaunchKernelGGL((gemv_generic<XM>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                       a);
    return;
  }
  const long tiles16 = (a.N + 15) / 16 * ((a.M + kRowsPerGroup - 1) / kRowsPerGroup);
  const long nkb = (a.K + 63) >> 6;
  // Many column tiles (a long weight stream): 64 columns per workgroup so the activations are
  // re-read once per 64 columns instead of once per 16. Few tiles (decode shapes): 16 columns per
  // workgroup and K split over up to 8 waves to put more requests in flight per CU.
  if (tiles16 >= 4096) return launch_tiles<XM, 4, 4>(a, st);
  if (nkb >= 8) return launch_tiles<XM, 1, 8>(a, st);
  if (nkb >= 4) return launch_tiles<XM, 1, 4>(a, st);
  if (nkb >= 2) return launch_tiles<XM, 1, 2>(a, st);
  launch_tiles<XM, 1, 1>(a, st);
}

}  // namespace
}  // namespace gsvk

using namespace gsvk;

extern "C" int gsvk_gemv_f16w(int x_dtype, int round_x, const void* x, size_t ldx,
                              const uint16_t* w, const float* bias, int act, float slope,
                              const void* residual, int y_dtype, void* y, size_t ldy, size_t rows,
                              size_t out, size_t in, void* stream) {
  if (x_dtype != GSVK_F32 && x_dtype != GSVK_F16) return GSVK_E_DTYPE;
  if (!valid_dtype(y_dtype)) return GSVK_E_DTYPE;
  if (act < GSVK_ACT_NONE || act > GSVK_ACT_LEAKY_RELU) return GSVK_E_DTYPE;
  if (!x || !w || !y) return GSVK_E_NULL;
  if (rows == 0 || out == 0 || in == 0 || ldx < in || ldy < out) return GSVK_E_SIZE;
  if (rows > static_cast<size_t>(kMaxRowGroups) * kRowsPerGroup || out > (1ul << 31) ||
      in > (1ul << 31) || ldx > (1ul << 40) || ldy > (1ul << 40))
    return GSVK_E_SIZE;
  const size_t xsz = dtype_size(x_dtype), ysz = dtype_size(y_dtype);
  const size_t ybytes = span_bytes(rows, out, ldy, ysz);
  if (overlaps(y, ybytes, x, span_bytes(rows, in, ldx, xsz)) ||
      overlaps(y, ybytes, w, out * in * 2) || overlaps(y, ybytes, bias, bias ? out * 4 : 0))
    return GSVK_E_ALIAS;
  if (residual && residual != y && overlaps(y, ybytes, residual, ybytes)) return GSVK_E_ALIAS;

  GvArgs a{x, w, bias, residual, y, static_cast<long>(rows), static_cast<long>(out),
           static_cast<long>(in), static_cast<long>(ldx), static_cast<long>(ldy), act, y_dtype,
           slope, false};
  const size_t yalign = y_dtype == GSVK_F32 ? 16 : 8;
  a.vec_store = ldy % 4 == 0 && reinterpret_cast<uintptr_t>(y) % yalign == 0;
  // Matrix-core tiles need 16-byte rows: K % 8 == 0, and aligned x rows and weights.
  const bool tiled = in % 8 == 0 && aligned16(w) && aligned16(x) && (ldx * xsz) % 16 == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int xm = x_dtype == GSVK_F16 ? kXF16 : (round_x ? kXRound : kXSplit);
  switch (xm) {
    case kXF16: launch_xm<kXF16>(a, tiled, st); break;
    case kXRound: launch_xm<kXRound>(a, tiled, st); break;
    default: launch_xm<kXSplit>(a, tiled, st); break;
  }
  return launch_status();
}
