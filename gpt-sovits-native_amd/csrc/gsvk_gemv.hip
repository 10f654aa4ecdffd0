// gsvk_gemv.hip — batched decode GEMV with fp16 weights on the gfx950 matrix cores, with the bias /
// activation / residual epilogue fused into the store.
//
// y[r, n] = act(sum_k float(w[n, k]) * x[r, k] + bias[n]) (+ residual[r, n]), for B sequences
// (rows) at once. At B = 64 a weight element feeds 64 multiply-adds: 64 flop per weight byte,
// above the fp32 VALU ridge of MI355X (157 TFLOP/s / 8 TB/s = 20) and far below the fp16 matrix
// core one (2.5 PFLOP/s / 8 TB/s = 312), so the products go to v_mfma_f32_16x16x32_f16 and the
// kernel stays bound by memory.
//
// Tiles. Operand A of one MFMA is a 16 x 32 slice of W (16 output columns n, 32 k), operand B a
// 32 x 16 slice of X^T (32 k, 16 rows r): lane l feeds row/column (l & 15) with 8 k values chosen
// by its lane group (l >> 4). The accumulator then holds, in lane l, four consecutive outputs
// n = 4 (l >> 4) .. +3 of row (l & 15), stored as one vector. A and B use the same k slots, so
// which 8 k a lane group holds is free: lane group g holds k = 64 kb + 16 g + 8 h .. +7 for the two
// MFMAs h = 0, 1 of a 64-wide k block.
//
// Staging. Read straight into that fragment layout, every 16-byte load instruction would touch 16
// rows (one 128-byte line per row, half used), which runs at a fraction of the CU's load rate. So
// each wave loads its k block as 8 rows x 128 contiguous bytes per instruction, writes it to a
// private, padded LDS tile and reads the fragments back from there. A wave's LDS accesses execute
// in issue order; a wavefront fence keeps the compiler from reordering them.
//
// Work split. A workgroup covers 16 MF rows x 16 NF columns over all of K; its WK waves split K
// into contiguous k-block ranges and keep up to D k blocks of global loads in flight each. The
// per-wave partial sums are added in wave order through LDS (a fixed order: results do not depend
// on timing). Products fp16 x fp16 are exact in fp32; the sums are fp32.
//
// x in fp32: round_x = 1 rounds it to fp16 first (T2SEngine::gemv_fmlal, t2s_engine.cpp:696-700);
// round_x = 0 keeps the fp32 value (kern::gemv_f16w_f32acc, gemv.cpp:112-127) by feeding
// hi = f16(x) and lo = f16(x - hi) through two MFMAs: x - hi is exact and lo holds the next 11
// bits, so hi + lo equals x to about 2^-22 relative (|x| < 65504).
#include <algorithm>
#include <cmath>

#include "gsvk_common.hpp"

namespace gsvk {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));

enum XMode { kXF16 = 0, kXRound = 1, kXSplit = 2 };

constexpr long kMaxRowGroups = 65535;
constexpr int kRowHalves = 72;  // LDS row: 64 k + 8 halves of padding (144 bytes)

struct GvArgs {
  const void* x;
  const uint16_t* w;
  const float* bias;
  const void* res;
  void* y;
  long M, N, K, ldx, ldy;
  int act;
  float slope;
  bool vec_store;
  // LayerNorm prologue (the LN instantiations): x holds the pre-norm rows, the products use
  // h = LN(x) (gamma / beta may be null: ones / zeros), and column-block 0 stores h to ln_y.
  const float* ln_g = nullptr;
  const float* ln_b = nullptr;
  void* ln_y = nullptr;
  long ldh = 0;
  float ln_eps = 0.f;
  double inv_n = 0.0;  // 1.0 / K, computed on the host
};

__device__ __forceinline__ float act_rt(int act, float v, float slope) {
  switch (act) {
    case GSVK_ACT_RELU: return relu_ref(v);
    case GSVK_ACT_GELU_ERF: return gelu_erf(v);
    case GSVK_ACT_LEAKY_RELU: return lrelu_ref(v, slope);
    default: return v;
  }
}

template <int YDT>
__device__ __forceinline__ float load_y(const void* p, size_t i) {
  if constexpr (YDT == GSVK_F32) return static_cast<const float*>(p)[i];
  else if constexpr (YDT == GSVK_F16) return h2f(static_cast<const uint16_t*>(p)[i]);
  else return bf2f(static_cast<const uint16_t*>(p)[i]);
}

template <int YDT>
__device__ __forceinline__ void store_y(void* p, size_t i, float v) {
  if constexpr (YDT == GSVK_F32) static_cast<float*>(p)[i] = v;
  else if constexpr (YDT == GSVK_F16) static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f2h(v));
  else static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f2bf(v));
}

// Epilogue operands of four consecutive outputs n .. n+3 of row m: bias[n + q] and
// residual[m, n + q], read from clamped indices (an in-bounds dummy when absent: the value is then
// not used) so the loads need no branch.
struct EpiIn {
  float b[4];
  float r[4];
};

template <int YDT>
__device__ __forceinline__ EpiIn epi_load(const GvArgs& a, long m, long n) {
  EpiIn e;
  const size_t mr = static_cast<size_t>(min(m, a.M - 1)) * a.ldy;
  const float* bp = a.bias ? a.bias : kZeros8;
  const void* rp = a.res ? a.res : static_cast<const void*>(kZeros8);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const long nq = min(n + q, a.N - 1);
    e.b[q] = bp[a.bias ? nq : 0];
    e.r[q] = load_y<YDT>(rp, a.res ? mr + nq : 0);
  }
  return e;
}

// The streaming kernel's form of the same operands, as loaded: 4 in-range columns n .. n+3
// (n % 4 == 0) of an in-range row, one 16-byte bias load and one residual load of 4 elements (the
// host has checked that bias, residual and the row stride keep them aligned). They stay raw until
// the store: converting them right after the load would make the wave wait for it there.
struct EpiRaw {
  u32x4 b;
  u32x4 r;  // 4 fp32, or 4 16-bit values in the low two words
};

template <int YDT>
__device__ __forceinline__ EpiRaw epi_load_raw(const GvArgs& a, long m, long n) {
  EpiRaw e;
  e.b = ld16<false>(a.bias ? a.bias + n : kZeros8);
  if constexpr (YDT == GSVK_F32) {
    e.r = ld16<false>(a.res ? static_cast<const float*>(a.res) + static_cast<size_t>(m) * a.ldy + n
                            : kZeros8);
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(
        a.res ? static_cast<const uint16_t*>(a.res) + static_cast<size_t>(m) * a.ldy + n
              : reinterpret_cast<const uint16_t*>(kZeros8));
    e.r = u32x4{v.x, v.y, 0u, 0u};
  }
  return e;
}

// Four outputs of the streaming kernel: act(s + b) + r with the activation fixed at compile time,
// stored as one vector when the row and the 4 columns are in range (N % 4 == 0). An absent bias or
// residual is -0, which added leaves every value as it is (-0 included): no branch.
template <int YDT, int ACT>
__device__ __forceinline__ void finish4s(const GvArgs& a, long m, long n, f4v s, const EpiRaw& e,
                                         bool live) {
  float b[4], r[4];
  const f4v bf = __builtin_bit_cast(f4v, e.b);
  if constexpr (YDT == GSVK_F32) {
    const f4v rf = __builtin_bit_cast(f4v, e.r);
#pragma unroll
    for (int q = 0; q < 4; ++q) r[q] = rf[q];
  } else {
    const uint32_t h[4] = {e.r[0] & 0xffffu, e.r[0] >> 16, e.r[1] & 0xffffu, e.r[1] >> 16};
#pragma unroll
    for (int q = 0; q < 4; ++q) r[q] = YDT == GSVK_F16 ? h2f(h[q]) : bf2f(h[q]);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    b[q] = a.bias ? bf[q] : -0.f;
    r[q] = a.res ? r[q] : -0.f;
  }
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = act_apply<ACT>(s[q] + b[q], a.slope) + r[q];
  if (live && m < a.M && n < a.N) {
    const size_t off = static_cast<size_t>(m) * a.ldy + n;
    if constexpr (YDT == GSVK_F32) {
      *reinterpret_cast<float4*>(static_cast<float*>(a.y) + off) = float4{v[0], v[1], v[2], v[3]};
    } else {
      uint32_t h[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) h[q] = YDT == GSVK_F16 ? f2h(v[q]) : f2bf(v[q]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.y) + off) =
          uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
  }
}

// v = act(acc + bias[n]) (+ residual[m, n]). The bias add is skipped, not replaced by + 0, when
// there is no bias (x + 0 would turn -0 into +0); likewise the residual add.
__device__ __forceinline__ float epilogue(const GvArgs& a, float v, float b, float r) {
  if (a.bias) v = v + b;
  v = act_rt(a.act, v, a.slope);
  if (a.res) v = v + r;
  return v;
}

// Four consecutive outputs n .. n+3 of row m.
template <int YDT>
__device__ __forceinline__ void finish4(const GvArgs& a, long m, long n, f4v s, const EpiIn& e) {
  if (m >= a.M) return;
  const size_t off = static_cast<size_t>(m) * a.ldy + n;
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = epilogue(a, s[q], e.b[q], e.r[q]);
  if (a.vec_store && n + 4 <= a.N) {
    if constexpr (YDT == GSVK_F32) {
      *reinterpret_cast<float4*>(static_cast<float*>(a.y) + off) = float4{v[0], v[1], v[2], v[3]};
    } else {
      uint32_t h[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) h[q] = YDT == GSVK_F16 ? f2h(v[q]) : f2bf(v[q]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.y) + off) =
          uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if (n + q < a.N) store_y<YDT>(a.y, off + q, v[q]);
}

// One k block as loaded from global memory. 16-bit rows: 128 bytes per row, instruction q covers
// rows 8q .. 8q+7 (lane l: row l / 8, bytes 16 (l % 8)). fp32 rows: 256 bytes per row,
// instruction q covers rows 4q .. 4q+3 (lane l: row l / 16, bytes 16 (l % 16)).
template <int XM>
constexpr int x_insts() { return XM == kXF16 ? 2 : 4; }

// The in-range flags travel with the data: zeroing a value right after its load would make the
// wave wait for that load there, so k blocks past K are zeroed only when they are staged (and only
// in the TAIL instantiation, for K % 64 != 0).
template <int XM, int MF, int NF>
struct Raw {
  u32x4 w[NF][2];
  u32x4 x[MF][x_insts<XM>()];
  u32x4 g[XM == kXF16 ? 2 : 1], b[XM == kXF16 ? 2 : 1];  // LN: gamma / beta of the lane's k
  long kb;                                                // LN: the block (for the h store)
  bool okw, okx;
};

// Per-wave LDS tile of one k block: NF weight fragments, MF activation fragments (and MF
// remainders in split mode), 16 rows of kRowHalves each.
template <int XM, int MF, int NF>
constexpr int stage_halves() {
  return (NF + MF * (XM == kXSplit ? 2 : 1)) * 16 * kRowHalves;
}

template <int XM, int YDT, int MF, int NF, int WK, int D, bool TAIL, bool LN>
__global__ __launch_bounds__(kWave * WK) void gemv_mfma(GvArgs a) {
  constexpr int T = MF * NF;  // 16 x 16 output tiles of the workgroup
  constexpr int SH = stage_halves<XM, MF, NF>();
  constexpr int kStageBytes = WK * SH * 2;
  constexpr int kRedBytes = WK > 1 ? WK * T * kWave * 16 : 16;
  __shared__ __attribute__((aligned(16))) char smem[kStageBytes > kRedBytes ? kStageBytes
                                                                              : kRedBytes];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int r16 = lane & 15, grp = lane >> 4;
  const long m0 = static_cast<long>(blockIdx.y) * (16 * MF);
  const long n0 = static_cast<long>(blockIdx.x) * (16 * NF);
  const long nkb = (a.K + 63) >> 6;
  const long per = (nkb + WK - 1) / WK;
  const long kb0 = min(nkb, wave * per), kb1 = min(nkb, kb0 + per);

  // Each wave finishes tiles wave, wave + WK, ... (TPW of them at most). With few enough tiles it
  // fetches their epilogue operands first, so that latency hides under the main loads.
  constexpr int TPW = (T + WK - 1) / WK;
  constexpr bool kPrefetch = TPW <= 4;
  EpiIn pre[kPrefetch ? TPW : 1];
  if constexpr (kPrefetch) {
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const int t = min(wave + u * WK, T - 1);
      pre[u] = epi_load<YDT>(a, m0 + 16 * (t / NF) + r16, n0 + 16 * (t % NF) + 4 * grp);
    }
  }

  // Global rows this lane loads (clamped: rows past M or N load a valid row that is never stored).
  constexpr int XQ = x_insts<XM>();
  constexpr int XLPR = XQ == 2 ? 8 : 16;  // lanes per x row in one instruction
  size_t wrow[NF][2], xrow[MF][XQ];
#pragma unroll
  for (int j = 0; j < NF; ++j)
#pragma unroll
    for (int q = 0; q < 2; ++q)
      wrow[j][q] = static_cast<size_t>(min(n0 + 16 * j + 8 * q + lane / 8, a.N - 1)) * a.K;
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int q = 0; q < XQ; ++q)
      xrow[i][q] =
          static_cast<size_t>(min(m0 + 16 * i + (16 / XQ) * q + lane / XLPR, a.M - 1)) * a.ldx;

  auto load = [&](Raw<XM, MF, NF>& r, long kb) {
    r.kb = kb;
    const long kw = kb * 64 + (lane % 8) * 8;  // 8 halves per lane
    r.okw = !TAIL || kw < a.K;
    const size_t kcw = static_cast<size_t>(r.okw ? kw : a.K - 8);
#pragma unroll
    for (int j = 0; j < NF; ++j)
#pragma unroll
      for (int q = 0; q < 2; ++q) r.w[j][q] = ld16<false>(a.w + wrow[j][q] + kcw);
    if constexpr (XM == kXF16) {
      r.okx = r.okw;
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int q = 0; q < 2; ++q)
          r.x[i][q] = ld16<false>(static_cast<const uint16_t*>(a.x) + xrow[i][q] + kcw);
    } else {
      const long kx = kb * 64 + (lane % 16) * 4;  // 4 floats per lane
      r.okx = !TAIL || kx < a.K;
      const size_t kcx = static_cast<size_t>(r.okx ? kx : a.K - 4);
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          r.x[i][q] = ld16<false>(static_cast<const float*>(a.x) + xrow[i][q] + kcx);
    }
    if constexpr (LN) {
      // the lane's 8 (16-bit x) or 4 (fp32 x) k of this block, clamped like the x loads
      const size_t kc = XM == kXF16 ? kcw
                                    : static_cast<size_t>(!TAIL || kb * 64 + (lane % 16) * 4 < a.K
                                                              ? kb * 64 + (lane % 16) * 4
                                                              : a.K - 4);
#pragma unroll
      for (int q = 0; q < (XM == kXF16 ? 2 : 1); ++q) {
        r.g[q] = ld16<false>(param_or(a.ln_g, kc + 4 * q, kOnes8));
        r.b[q] = ld16<false>(param_or(a.ln_b, kc + 4 * q, kZeros8));
      }
    }
  };

  // LayerNorm prologue (LN). The host launches it only when every wave's k blocks fit in its D
  // load slots, so the activations of the workgroup's 16 MF rows over all of K are in registers
  // once the first loads land: the statistics come from them, with no second read. Per row:
  // each lane sums its in-range values in k order, the lanes that share the row add up with DPP,
  // and the per-wave partials are added in wave order through LDS; mean = float(sum * (1/K)) in
  // double, then the centred second moment the same way, rstd = rsq(var + eps): ln_rows_tile's
  // formulas (csrc/gsvk_norm.hip) in another summation order.
  __shared__ float ln_part[LN ? 2 * WK * 16 * MF : 1];  // one area per pass: two barriers in all
  float lmean[MF][XQ], lrstd[MF][XQ];
  const bool store_h = LN && a.ln_y != nullptr && blockIdx.x == 0;
  auto row_sum = [&](float v) {  // over the XLPR consecutive lanes that hold one row
    v += dpp_f32<0xB1>(v);       // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);       // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);      // row_half_mirror: 8 lanes
    if constexpr (XLPR == 16) v += dpp_f32<0x140>(v);  // row_mirror: 16 lanes
    return v;
  };
  // pass 0: sum of x; pass 1: sum of (x - mean)^2. Lanes past K and blocks past the wave's range
  // add nothing.
  auto ln_pass = [&](const Raw<XM, MF, NF>(&f)[D], int pass, float (&out)[MF][XQ]) {
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int q = 0; q < XQ; ++q) {
        float p = 0.f;
#pragma unroll
        for (int s = 0; s < D; ++s) {
          if (kb0 + s < kb1 && f[s].okx) {
            float v[XQ == 2 ? 8 : 4];
            if constexpr (XM == kXF16) Store<GSVK_F16>::unpack(f[s].x[i][q], v);
            else Store<GSVK_F32>::unpack(f[s].x[i][q], v);
#pragma unroll
            for (int k = 0; k < (XQ == 2 ? 8 : 4); ++k) {
              if (pass == 0) {
                p += v[k];
              } else {
                const float d = v[k] - lmean[i][q];
                p = __builtin_fmaf(d, d, p);
              }
            }
          }
        }
        p = row_sum(p);
        if (lane % XLPR == 0)
          ln_part[(pass * WK + wave) * 16 * MF + 16 * i + (16 / XQ) * q + lane / XLPR] = p;
      }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int q = 0; q < XQ; ++q) {
        const int rr = pass * WK * 16 * MF + 16 * i + (16 / XQ) * q + lane / XLPR;
        float t = ln_part[rr];
#pragma unroll
        for (int w = 1; w < WK; ++w) t += ln_part[w * 16 * MF + rr];
        out[i][q] = static_cast<float>(static_cast<double>(t) * a.inv_n);
      }
  };
  auto ln_prologue = [&](const Raw<XM, MF, NF>(&f)[D]) {
    ln_pass(f, 0, lmean);
    float var[MF][XQ];
    ln_pass(f, 1, var);
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int q = 0; q < XQ; ++q) lrstd[i][q] = __builtin_amdgcn_rsqf(var[i][q] + a.ln_eps);
  };

  _Float16* st_w = reinterpret_cast<_Float16*>(smem) + wave * SH;
  _Float16* st_x = st_w + NF * 16 * kRowHalves;
  _Float16* st_l = st_x + MF * 16 * kRowHalves;  // split mode: remainders

  auto stage = [&](const Raw<XM, MF, NF>& r) {
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < NF; ++j)
#pragma unroll
      for (int q = 0; q < 2; ++q)
        *reinterpret_cast<u32x4*>(st_w + (j * 16 + 8 * q + lane / 8) * kRowHalves +
                                  (lane % 8) * 8) = r.okw ? r.w[j][q] : zero;
    if constexpr (XM == kXF16) {
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          u32x4 v = r.x[i][q];
          if constexpr (LN) {
            float h[8], o[8];
            Store<GSVK_F16>::unpack(v, h);
            const f4v g0 = __builtin_bit_cast(f4v, r.g[0]), g1 = __builtin_bit_cast(f4v, r.g[1]);
            const f4v b0 = __builtin_bit_cast(f4v, r.b[0]), b1 = __builtin_bit_cast(f4v, r.b[1]);
#pragma unroll
            for (int k = 0; k < 8; ++k)
              o[k] = __builtin_fmaf((h[k] - lmean[i][q]) * lrstd[i][q], k < 4 ? g0[k] : g1[k - 4],
                                    k < 4 ? b0[k] : b1[k - 4]);
            v = Store<GSVK_F16>::pack(o);
            const long row = m0 + 16 * i + 8 * q + lane / 8;
            if (store_h && r.okx && row < a.M)
              st16<false>(static_cast<uint16_t*>(a.ln_y) + static_cast<size_t>(row) * a.ldh +
                              r.kb * 64 + (lane % 8) * 8,
                          v);
          }
          *reinterpret_cast<u32x4*>(st_x + (i * 16 + 8 * q + lane / 8) * kRowHalves +
                                    (lane % 8) * 8) = r.okx ? v : zero;
        }
    } else {
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f4v f = __builtin_bit_cast(f4v, r.x[i][q]);
          if constexpr (LN) {
            const f4v g = __builtin_bit_cast(f4v, r.g[0]), b = __builtin_bit_cast(f4v, r.b[0]);
#pragma unroll
            for (int k = 0; k < 4; ++k)
              f[k] = __builtin_fmaf((f[k] - lmean[i][q]) * lrstd[i][q], g[k], b[k]);
            const long row = m0 + 16 * i + 4 * q + lane / 16;
            if (store_h && r.okx && row < a.M)
              st16<false>(static_cast<float*>(a.ln_y) + static_cast<size_t>(row) * a.ldh +
                              r.kb * 64 + (lane % 16) * 4,
                          __builtin_bit_cast(u32x4, f));
          }
          if (!r.okx) f = __builtin_bit_cast(f4v, zero);
          const h4 hi = __builtin_convertvector(f, h4);
          const int off = (i * 16 + 4 * q + lane / 16) * kRowHalves + (lane % 16) * 4;
          *reinterpret_cast<h4*>(st_x + off) = hi;
          if constexpr (XM == kXSplit) {
            const f4v rest = f - __builtin_convertvector(hi, f4v);
            *reinterpret_cast<h4*>(st_l + off) = __builtin_convertvector(rest, h4);
          }
        }
    }
  };

  f4v acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};

  auto compute = [&]() {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int col = grp * 16 + h * 8;
      h8 wv[NF], xh[MF], xl[MF];
#pragma unroll
      for (int j = 0; j < NF; ++j)
        wv[j] = *reinterpret_cast<const h8*>(st_w + (j * 16 + r16) * kRowHalves + col);
#pragma unroll
      for (int i = 0; i < MF; ++i) {
        xh[i] = *reinterpret_cast<const h8*>(st_x + (i * 16 + r16) * kRowHalves + col);
        if constexpr (XM == kXSplit)
          xl[i] = *reinterpret_cast<const h8*>(st_l + (i * 16 + r16) * kRowHalves + col);
      }
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv[j], xh[i], acc[i][j], 0, 0, 0);
          if constexpr (XM == kXSplit)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv[j], xl[i], acc[i][j], 0, 0, 0);
        }
    }
  };
  // Stage a block, read its fragments, multiply. The fences keep this wave's LDS writes and reads
  // in program order (the LDS executes one wave's accesses in issue order).
  auto process = [&](const Raw<XM, MF, NF>& r) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    stage(r);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    compute();
  };

  // Rolling prefetch: D k blocks of global loads in flight. Block indices past the wave's range
  // are clamped to its last block (an in-bounds reload whose result is not used), so no load sits
  // under a branch.
  Raw<XM, MF, NF> f[D];
  if constexpr (LN) {
    // All of the wave's blocks (at most D), then the statistics. A wave with no blocks
    // (kb0 == kb1 == nkb) loads the last block and never uses it.
#pragma unroll
    for (int s = 0; s < D; ++s) load(f[s], max(0L, min(kb0 + s, kb1 - 1)));
    ln_prologue(f);
  }
  if (kb0 < kb1) {
    const long nr = (kb1 - kb0 + D - 1) / D;
    if constexpr (!LN) {
#pragma unroll
      for (int s = 0; s < D; ++s) load(f[s], min(kb0 + s, kb1 - 1));
    }
    for (long r = 0; r + 1 < nr; ++r) {
#pragma unroll
      for (int s = 0; s < D; ++s) {
        process(f[s]);
        load(f[s], min(kb0 + (r + 1) * D + s, kb1 - 1));
      }
    }
    const long kl = kb0 + (nr - 1) * D;
#pragma unroll
    for (int s = 0; s < D; ++s)
      if (kl + s < kb1) process(f[s]);
  }

  // Workgroup sum of the wave partials, tile t by wave t % WK, waves added in order. The reduction
  // area reuses the staging LDS, so every wave must be done with it first.
  f4v* red = reinterpret_cast<f4v*>(smem);
  if constexpr (WK > 1) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int j = 0; j < NF; ++j) red[(wave * T + i * NF + j) * kWave + lane] = acc[i][j];
    __syncthreads();
  }
  for (int t = wave; t < T; t += WK) {
    f4v s;
    if constexpr (WK > 1) {
      s = red[t * kWave + lane];
#pragma unroll
      for (int w = 1; w < WK; ++w) s = s + red[(w * T + t) * kWave + lane];
    } else {
      s = acc[0][0];
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j)
          if (i * NF + j == t) s = acc[i][j];
    }
    const long m = m0 + 16 * (t / NF) + r16, n = n0 + 16 * (t % NF) + 4 * grp;
    if constexpr (kPrefetch) {
      EpiIn e = pre[0];
#pragma unroll
      for (int u = 1; u < TPW; ++u)
        if (wave + u * WK == t) e = pre[u];
      finish4<YDT>(a, m, n, s, e);
    } else {
      finish4<YDT>(a, m, n, s, epi_load<YDT>(a, m, n));
    }
  }
}

// Any shape or alignment: one thread per output, k in order with fmaf (the product of an fp16
// weight and an fp16 or fp32 activation is formed exactly or rounded once, then added: the
// reference's vfmaq / fmlal step). Used when K % 8 != 0 or a row is not 16-byte aligned.
template <int XM, int YDT>
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
    const size_t off = static_cast<size_t>(m) * a.ldy + n;
    const float b = a.bias ? a.bias[n] : 0.f;
    const float r = a.res ? load_y<YDT>(a.res, off) : 0.f;
    store_y<YDT>(a.y, off, epilogue(a, s, b, r));
  }
}

// ---- long weight streams -------------------------------------------------------------------------
//
// A weight stream far larger than the launch's CUs can cover in one round of tiles (many thousands of
// 16-column tiles at up to 64 rows) runs on persistent workgroups instead. Each wave owns a fixed
// k slice (KB blocks of 64) and keeps the workgroup's activations of that slice in registers for the
// whole launch, loaded once; the workgroup then walks column batches (NT tiles of 16 columns)
// blockIdx.x, + gridDim.x, ... with D batches of weight loads in flight per wave. A lane reads
// its weight fragments straight from global memory: for k block b and MFMA half h, lane (column c,
// lane group g) takes the 16 bytes at k = 64 b + 16 g + 8 h of column c, the k assignment of the
// tiled kernel above, so a batch needs no staging. The waves' partial sums meet in LDS (double
// buffered, one barrier per batch) and are added in wave order, as in the tiled kernel: for a k
// slice of 128 per wave (KB = 2) the two kernels give the same bits.
//
// The epilogue operands of a batch (bias, residual) travel in its load slot, so no wave waits for a
// load issued after the weights it is about to use.
template <int XM, int MF, int KB>
struct StreamX {
  h8 hi[MF][2 * KB];
  h8 lo[XM == kXSplit ? MF : 1][XM == kXSplit ? 2 * KB : 1];
};

template <int MF, int NT, int KB, int FPW>
struct StreamSlot {
  u32x4 w[NT][2 * KB];  // tile t, k block b, half h at [t][2 b + h]
  EpiRaw e[NT][FPW];    // epilogue operands of the row fragments this wave finishes
};

template <int XM, int YDT, int ACT, int MF, int KB, int WK, int NT, int D>
__global__ __launch_bounds__(kWave * WK) void gemv_stream(GvArgs a) {
  constexpr int FPW = (MF + WK - 1) / WK;  // row fragments each wave finishes per tile
  constexpr int kRed = WK > 1 ? 2 * WK * NT * MF * kWave : 1;
  __shared__ f4v red[kRed];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int r16 = lane & 15, grp = lane >> 4;
  const long m0 = static_cast<long>(blockIdx.y) * (16 * MF);
  const long kw = static_cast<long>(wave) * (64 * KB);  // first k of this wave's slice
  const long nb = (a.N + 16 * NT - 1) / (16 * NT);     // column batches

  // Activations of the slice, once: lane (row r16, group grp), block b, half h holds k =
  // kw + 64 b + 16 grp + 8 h .. +7 of row m0 + 16 i + r16 (clamped: rows past M are never stored).
  StreamX<XM, MF, KB> xf;
#pragma unroll
  for (int i = 0; i < MF; ++i) {
    const size_t row = static_cast<size_t>(min(m0 + 16 * i + r16, a.M - 1)) * a.ldx;
#pragma unroll
    for (int q = 0; q < 2 * KB; ++q) {
      const size_t k = static_cast<size_t>(kw + 64 * (q >> 1) + 16 * grp + 8 * (q & 1));
      if constexpr (XM == kXF16) {
        xf.hi[i][q] = __builtin_bit_cast(h8, ld16<false>(static_cast<const uint16_t*>(a.x) + row + k));
      } else {
        const float* xp = static_cast<const float*>(a.x) + row + k;
        const f4v f0 = __builtin_bit_cast(f4v, ld16<false>(xp));
        const f4v f1 = __builtin_bit_cast(f4v, ld16<false>(xp + 4));
        const h4 h0 = __builtin_convertvector(f0, h4), h1 = __builtin_convertvector(f1, h4);
        xf.hi[i][q] = h8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
        if constexpr (XM == kXSplit) {
          const h4 l0 = __builtin_convertvector(f0 - __builtin_convertvector(h0, f4v), h4);
          const h4 l1 = __builtin_convertvector(f1 - __builtin_convertvector(h1, f4v), h4);
          xf.lo[i][q] = h8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
        }
      }
    }
  }

  // The loop never waits for the activations: their loads go out first and are waited for here,
  // behind nothing else (a wait inside the loop would also wait for every weight load in flight).
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int q = 0; q < 2 * KB; ++q) {
      asm volatile("" ::"v"(xf.hi[i][q]));
      if constexpr (XM == kXSplit) asm volatile("" ::"v"(xf.lo[i][q]));
    }

  // Loads of batch j (clamped to the last batch: a reload past the end is never used): the weights,
  // then, once the previous contents of the slot are used, the epilogue operands.
  auto n0_of = [&](long j) {
    return min(static_cast<long>(blockIdx.x) + static_cast<long>(gridDim.x) * j, nb - 1) *
           (16 * NT);
  };
  auto load_w = [&](StreamSlot<MF, NT, KB, FPW>& f, long j) {
    const long n0 = n0_of(j);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const size_t col = static_cast<size_t>(min(n0 + 16 * t + r16, a.N - 1)) * a.K;
#pragma unroll
      for (int q = 0; q < 2 * KB; ++q)
        f.w[t][q] = ld16<false>(a.w + col + kw + 64 * (q >> 1) + 16 * grp + 8 * (q & 1));
    }
  };
  auto load_e = [&](StreamSlot<MF, NT, KB, FPW>& f, long j) {
    const long n0 = n0_of(j);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int u = 0; u < FPW; ++u) {
        const int fr = min(wave + u * WK, MF - 1);
        // N % 4 == 0 here: a group past N reads the last 4 columns (never stored)
        f.e[t][u] = epi_load_raw<YDT>(a, min(m0 + 16 * fr + r16, a.M - 1),
                                      min(n0 + 16 * t + 4 * grp, a.N - 4));
      }
  };

  StreamSlot<MF, NT, KB, FPW> f[D];
#pragma unroll
  for (int s = 0; s < D; ++s) {
    load_w(f[s], s);
    load_e(f[s], s);
  }

  const long nbw = blockIdx.x < nb ? (nb - 1 - blockIdx.x) / gridDim.x + 1 : 0;  // own batches

  // Batch j of this workgroup covers columns n0_of(j) ..; process() multiplies, sums the waves and
  // stores it (the slot's weights are reloaded for batch j + D as soon as the products are issued,
  // its epilogue operands once they are used).
  auto process = [&](StreamSlot<MF, NT, KB, FPW>& f, long j, bool reload) {
    f4v acc[NT][MF];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < MF; ++i) acc[t][i] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 2 * KB; ++q)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const h8 wv = __builtin_bit_cast(h8, f.w[t][q]);
#pragma unroll
        for (int i = 0; i < MF; ++i) {
          acc[t][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv, xf.hi[i][q], acc[t][i], 0, 0, 0);
          if constexpr (XM == kXSplit)
            acc[t][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv, xf.lo[i][q], acc[t][i], 0, 0, 0);
        }
      }
    if (reload) load_w(f, j + D);

    const long n0 = n0_of(j);
    // A batch past the workgroup's own (the rounding of its count to whole rounds) stores nothing:
    // with the residual read from y itself it would add the residual twice.
    const bool live = j < nbw;
    if constexpr (WK == 1) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < MF; ++i)
          finish4s<YDT, ACT>(a, m0 + 16 * i + r16, n0 + 16 * t + 4 * grp, acc[t][i], f.e[t][i],
                             live);
    } else {
      f4v* rb = red + (j & 1) * (WK * NT * MF * kWave);
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < MF; ++i) rb[((wave * NT + t) * MF + i) * kWave + lane] = acc[t][i];
      lds_barrier();
#pragma unroll
      for (int u = 0; u < FPW; ++u) {
        const int fr = wave + u * WK;
        if (FPW * WK == MF || fr < MF) {  // every wave has a fragment when WK divides MF
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            f4v sum = rb[(t * MF + fr) * kWave + lane];
#pragma unroll
            for (int w = 1; w < WK; ++w) sum = sum + rb[((w * NT + t) * MF + fr) * kWave + lane];
            finish4s<YDT, ACT>(a, m0 + 16 * fr + r16, n0 + 16 * t + 4 * grp, sum, f.e[t][u], live);
          }
        }
      }
    }
    if (reload) load_e(f, j + D);
  };

  // The workgroup's batches run in whole rounds of D with no exit inside a round (an exit there
  // would merge into the loop's entry, and the compiler's wait counts at the top of the loop would
  // then assume that path's few loads in flight). Batches past the workgroup's last one load the
  // last batch of the launch again (n0_of clamps) and store nothing.
  for (long j = 0; j < nbw; j += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) process(f[s], j + s, true);
  }
}

// ---- launch plan ---------------------------------------------------------------------------------

template <int XM, int YDT, int MF, int NF, int WK, int D, bool LN>
void launch_tiles(const GvArgs& a, hipStream_t st) {
  const long gx = (a.N + 16 * NF - 1) / (16 * NF);
  const long gy = (a.M + 16 * MF - 1) / (16 * MF);
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
  // K a multiple of 64 (every decode shape) needs no zeroing of a partial last k block.
  if (a.K % 64 == 0)
    hipLaunchKernelGGL((gemv_mfma<XM, YDT, MF, NF, WK, D, false, LN>), grid, dim3(kWave * WK), 0,
                       st, a);
  else
    hipLaunchKernelGGL((gemv_mfma<XM, YDT, MF, NF, WK, D, true, LN>), grid, dim3(kWave * WK), 0,
                       st, a);
}

// LN (the LayerNorm prologue) is only launched tiled: the host checks the tile conditions first.
// The tile plan for a shape: 16 MF rows x 16 NF columns per workgroup, K over WK waves with D
// k blocks in flight each.
struct Plan {
  int mf, nf, wk, d;
};
// A long weight stream (many 16 x 16 tiles): 64-row tiles, so the weights are re-read from L2
// once per 64 rows, and 32 or 64 columns. Decode shapes: 16 x 16 tiles (the most workgroups),
// K over 4 or 8 waves with two k blocks each in flight (measured best on MI355X at B = 64 for
// K = 512 and 2048).
Plan plan_for(long M, long N, long K) {
  const long nkb = (K + 63) / 64;
  const long tiles = (N + 15) / 16 * ((M + 15) / 16);
  if (tiles >= 16384) return nkb > 16 ? Plan{4, 4, 2, 2} : Plan{4, 2, 4, 2};
  if (nkb >= 16) return {1, 1, 8, 2};
  if (nkb >= 8) return {1, 1, 4, 2};
  if (nkb >= 4) return {1, 1, 4, 1};
  if (nkb >= 2) return {1, 1, 2, 1};
  return {1, 1, 1, 1};
}

// Long weight streams at K = 512 or 1024 (k slices of 128 over 4 or 8 waves), no activation or
// ReLU, with aligned bias / residual / output rows: the persistent streaming kernel, one
// workgroup per CU (more per CU measured slower on MI355X), two 16-column tiles per batch and two
// batches of loads in flight (of 1-4 and 1-3 tried, the best on the replicated decode shapes).
constexpr int kStreamNT = 2, kStreamD = 2;

// (fp32 x kept as hi + lo needs twice the activation registers: K = 512 only.)
bool stream_ok(const GvArgs& a, bool tiled, long tiles, size_t ysz, bool split) {
  if (!tiled || tiles < 16384 || a.N % 4 || !a.vec_store) return false;
  if (a.K != 512 && (a.K != 1024 || split)) return false;
  if (a.act != GSVK_ACT_NONE && a.act != GSVK_ACT_RELU) return false;
  if (a.bias && !aligned16(a.bias)) return false;
  return !a.res || reinterpret_cast<uintptr_t>(a.res) % (4 * ysz) == 0;
}

template <int XM, int YDT, int ACT, int WK>
void launch_stream_wk(const GvArgs& a, hipStream_t st) {
  constexpr int MF = 4, KB = 2;
  const long nb = (a.N + 16 * kStreamNT - 1) / (16 * kStreamNT);
  const dim3 grid(static_cast<unsigned>(std::min<long>(nb, device_cus())),
                  static_cast<unsigned>((a.M + 16 * MF - 1) / (16 * MF)));
  hipLaunchKernelGGL((gemv_stream<XM, YDT, ACT, MF, KB, WK, kStreamNT, kStreamD>), grid,
                     dim3(kWave * WK), 0, st, a);
}

template <int XM, int YDT>
void launch_stream(const GvArgs& a, hipStream_t st) {
  if constexpr (XM == kXSplit) {
    if (a.act == GSVK_ACT_RELU) return launch_stream_wk<XM, YDT, GSVK_ACT_RELU, 4>(a, st);
    return launch_stream_wk<XM, YDT, GSVK_ACT_NONE, 4>(a, st);
  } else {
    if (a.act == GSVK_ACT_RELU)
      return a.K == 512 ? launch_stream_wk<XM, YDT, GSVK_ACT_RELU, 4>(a, st)
                        : launch_stream_wk<XM, YDT, GSVK_ACT_RELU, 8>(a, st);
    return a.K == 512 ? launch_stream_wk<XM, YDT, GSVK_ACT_NONE, 4>(a, st)
                      : launch_stream_wk<XM, YDT, GSVK_ACT_NONE, 8>(a, st);
  }
}

template <int XM, int YDT, bool LN>
void launch_plan(const GvArgs& a, bool tiled, hipStream_t st) {
  if constexpr (!LN) {
    const long tiles = (a.N + 15) / 16 * ((a.M + 15) / 16);
    if (stream_ok(a, tiled, tiles, YDT == GSVK_F32 ? 4 : 2, XM == kXSplit))
      return launch_stream<XM, YDT>(a, st);
  }
  if (!tiled && !LN) {
    const long blocks = std::min<long>((a.M * a.N + 255) / 256, 4096);
    hipLaunchKernelGGL((gemv_generic<XM, YDT>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       st, a);
    return;
  }
  const Plan p = plan_for(a.M, a.N, a.K);
  if (p.mf == 4) {
    if (p.nf == 4) return launch_tiles<XM, YDT, 4, 4, 2, 2, LN>(a, st);
    return launch_tiles<XM, YDT, 4, 2, 4, 2, LN>(a, st);
  }
  switch (p.wk * 10 + p.d) {
    case 82: return launch_tiles<XM, YDT, 1, 1, 8, 2, LN>(a, st);
    case 42: return launch_tiles<XM, YDT, 1, 1, 4, 2, LN>(a, st);
    case 41: return launch_tiles<XM, YDT, 1, 1, 4, 1, LN>(a, st);
    case 21: return launch_tiles<XM, YDT, 1, 1, 2, 1, LN>(a, st);
    default: return launch_tiles<XM, YDT, 1, 1, 1, 1, LN>(a, st);
  }
}

// Whether the plan for this shape gives every wave at most D k blocks (all of them in registers
// at once), which the LayerNorm prologue needs; decode plans (16-row tiles) only.
bool ln_resident(long M, long N, long K) {
  const Plan p = plan_for(M, N, K);
  const long nkb = (K + 63) / 64;
  return p.mf == 1 && (nkb + p.wk - 1) / p.wk <= p.d;
}

template <int XM, bool LN = false>
void launch_xm(int ydt, const GvArgs& a, bool tiled, hipStream_t st) {
  switch (ydt) {
    case GSVK_F32: return launch_plan<XM, GSVK_F32, LN>(a, tiled, st);
    case GSVK_F16: return launch_plan<XM, GSVK_F16, LN>(a, tiled, st);
    default: return launch_plan<XM, GSVK_BF16, LN>(a, tiled, st);
  }
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
  if (rows > static_cast<size_t>(kMaxRowGroups) * 16 || out > (1ul << 31) || in > (1ul << 31) ||
      ldx > (1ul << 40) || ldy > (1ul << 40))
    return GSVK_E_SIZE;
  const size_t xsz = dtype_size(x_dtype), ysz = dtype_size(y_dtype);
  const size_t ybytes = span_bytes(rows, out, ldy, ysz);
  if (overlaps(y, ybytes, x, span_bytes(rows, in, ldx, xsz)) ||
      overlaps(y, ybytes, w, out * in * 2) || overlaps(y, ybytes, bias, bias ? out * 4 : 0))
    return GSVK_E_ALIAS;
  if (residual && residual != y && overlaps(y, ybytes, residual, ybytes)) return GSVK_E_ALIAS;

  GvArgs a{x, w, bias, residual, y, static_cast<long>(rows), static_cast<long>(out),
           static_cast<long>(in), static_cast<long>(ldx), static_cast<long>(ldy), act, slope,
           false};
  const size_t yalign = y_dtype == GSVK_F32 ? 16 : 8;
  a.vec_store = ldy % 4 == 0 && reinterpret_cast<uintptr_t>(y) % yalign == 0;
  // Matrix-core tiles need 16-byte rows: K % 8 == 0, aligned x rows and weights.
  const bool tiled = in % 8 == 0 && aligned16(w) && aligned16(x) && (ldx * xsz) % 16 == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int xm = x_dtype == GSVK_F16 ? kXF16 : (round_x ? kXRound : kXSplit);
  switch (xm) {
    case kXF16: launch_xm<kXF16>(y_dtype, a, tiled, st); break;
    case kXRound: launch_xm<kXRound>(y_dtype, a, tiled, st); break;
    default: launch_xm<kXSplit>(y_dtype, a, tiled, st); break;
  }
  return launch_status();
}

extern "C" int gsvk_gemv_f16w_ln(int x_dtype, int round_x, const void* z, size_t ldz,
                                 const float* gamma, const float* beta, double eps, void* h,
                                 size_t ldh, const uint16_t* w, const float* bias, int act,
                                 float slope, const void* residual, int y_dtype, void* y,
                                 size_t ldy, size_t rows, size_t out, size_t in, void* stream) {
  if (x_dtype != GSVK_F32 && x_dtype != GSVK_F16) return GSVK_E_DTYPE;
  if (!valid_dtype(y_dtype)) return GSVK_E_DTYPE;
  if (act < GSVK_ACT_NONE || act > GSVK_ACT_LEAKY_RELU) return GSVK_E_DTYPE;
  if (!z || !h || !w || !y) return GSVK_E_NULL;
  if (rows == 0 || out == 0 || in == 0 || ldz < in || ldh < in || ldy < out) return GSVK_E_SIZE;
  if (rows > static_cast<size_t>(kMaxRowGroups) * 16 || out > (1ul << 31) || in > (1ul << 30) ||
      ldz > (1ul << 40) || ldh > (1ul << 40) || ldy > (1ul << 40))
    return GSVK_E_SIZE;
  if (!(eps >= 0.0) || !std::isfinite(eps)) return GSVK_E_ARG;
  const size_t xsz = dtype_size(x_dtype), ysz = dtype_size(y_dtype);
  const size_t zbytes = span_bytes(rows, in, ldz, xsz), hbytes = span_bytes(rows, in, ldh, xsz);
  const size_t ybytes = span_bytes(rows, out, ldy, ysz);
  // Other workgroups still read z while column block 0 writes h, and every one reads h's
  // parameters and the weights: h overlaps none of them, nor y.
  if (overlaps(h, hbytes, z, zbytes) || overlaps(h, hbytes, w, out * in * 2) ||
      overlaps(h, hbytes, gamma, gamma ? in * 4 : 0) || overlaps(h, hbytes, beta, beta ? in * 4 : 0))
    return GSVK_E_ALIAS;
  if (overlaps(y, ybytes, z, zbytes) || overlaps(y, ybytes, h, hbytes) ||
      overlaps(y, ybytes, w, out * in * 2) || overlaps(y, ybytes, bias, bias ? out * 4 : 0))
    return GSVK_E_ALIAS;
  if (residual && residual != y && overlaps(y, ybytes, residual, ybytes)) return GSVK_E_ALIAS;

  hipStream_t st = static_cast<hipStream_t>(stream);
  // The fused form needs the matrix-core tiles (16-byte rows of z and h, K % 8 == 0, 16-byte
  // parameter vectors) and a launch plan whose waves hold all their k blocks at once (K up to
  // 1024 at decode batch sizes). Otherwise: the two launches it stands for.
  const bool fused = in % 8 == 0 && ln_resident(static_cast<long>(rows), static_cast<long>(out),
                                                static_cast<long>(in)) &&
                     aligned16(w) && aligned16(z) && aligned16(h) && (ldz * xsz) % 16 == 0 &&
                     (ldh * xsz) % 16 == 0 && (!gamma || aligned16(gamma)) &&
                     (!beta || aligned16(beta));
  if (!fused) {
    if (ldz != ldh) return GSVK_E_ARG;  // the LayerNorm launch takes one row stride
    const int rc = gsvk_add_layernorm(x_dtype, z, nullptr, nullptr, gamma, beta, h, rows, in, ldz,
                                      eps, stream);
    if (rc) return rc;
    return gsvk_gemv_f16w(x_dtype, round_x, h, ldh, w, bias, act, slope, residual, y_dtype, y, ldy,
                          rows, out, in, stream);
  }
  GvArgs a{z, w, bias, residual, y, static_cast<long>(rows), static_cast<long>(out),
           static_cast<long>(in), static_cast<long>(ldz), static_cast<long>(ldy), act, slope,
           false};
  a.ln_g = gamma;
  a.ln_b = beta;
  a.ln_y = h;
  a.ldh = static_cast<long>(ldh);
  a.ln_eps = static_cast<float>(eps);
  a.inv_n = 1.0 / static_cast<double>(in);
  const size_t yalign = y_dtype == GSVK_F32 ? 16 : 8;
  a.vec_store = ldy % 4 == 0 && reinterpret_cast<uintptr_t>(y) % yalign == 0;
  const int xm = x_dtype == GSVK_F16 ? kXF16 : (round_x ? kXRound : kXSplit);
  switch (xm) {
    case kXF16: launch_xm<kXF16, true>(y_dtype, a, true, st); break;
    case kXRound: launch_xm<kXRound, true>(y_dtype, a, true, st); break;
    default: launch_xm<kXSplit, true>(y_dtype, a, true, st); break;
  }
  return launch_status();
}
