// gsvk_norm.hip — residual-add + LayerNorm over rows and per-channel GroupNorm + GELU for gfx950.
//
// LayerNorm: one wave64 per row, R consecutive rows per wave, one-shot grid. Each lane owns the
// 16-byte chunks lane, lane+64, ... of its rows (so every load/store instruction of the wave covers
// 1 KiB contiguously), keeps them in VGPRs, and the row statistics are an exact two-pass mean /
// centred second moment over those registers, reduced with DPP + ds_swizzle. gamma / beta / bias
// chunks for the lane's columns are loaded once per wave and reused for its R rows.
//
// GroupNorm(groups = channels): one 1024-thread workgroup per channel row of length T, the whole
// row held in VGPRs (up to 8 chunks of 16 bytes per thread: T <= 32768 fp32 / 65536 fp16),
// double-precision block reduction through LDS, then normalize + GELU(erf) and a single write:
// one HBM read and one write per element.
#include <atomic>
#include <cmath>

#include "gsvk_common.hpp"

namespace gsvk {
namespace {

struct LnArgs {
  const void* x;
  const float* bias;
  const void* res;
  const float* gamma;
  const float* beta;
  void* y;
  long rows;
  int n;
  long ld;
  double eps;
  double inv_n;  // 1.0 / n, computed on the host
};

// Workgroup size of the generic path; the tiled path takes it as a template parameter (one wave
// per workgroup for latency-bound calls, four for large ones).
constexpr int kLnBlock = 256;

__device__ __forceinline__ float finish_rstd(float var, double eps) {
  return static_cast<float>(1.0 / sqrt(static_cast<double>(var) + eps));
}

// Vector path: n % VEC == 0, every row start 16-byte aligned, n <= 64 * CPL * VEC.
// Wave w of workgroup b owns rows (WG*b + w)*R ... (WG*b + w)*R + R - 1 (WG waves per workgroup),
// so a workgroup's WG*R rows are consecutive: one contiguous tile for row-major data, visited once
// (one-shot grid). All x / residual chunks of the wave's R rows are loaded (packed) before any
// arithmetic. The statistics are finalized with the host's 1/n and v_rsq_f32 (1 ulp): the latency
// of a double-precision divide and square root sits on the critical path of every small call.
// Per-lane partial sums are balanced trees per chunk (chunk_sum / chunk_sumsq), chunks added in
// order. The one-launch decode step (gsvk_step.hip) shares that tree order but not the statistics
// (it takes one pass, E[x^2] - mean^2, where this kernel takes a centred second pass), so the two
// agree within the LayerNorm tolerance, not bit for bit.
template <int DT, int CPL, int R, bool NT, int BLOCK, bool HAS_RES>
__global__ __launch_bounds__(BLOCK) void ln_rows_tile(LnArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  constexpr bool kCache = CPL * V <= 16;  // keep per-column parameters in VGPRs for all R rows
  constexpr size_t kEsz = DT == GSVK_F32 ? 4 : 2;
  const int lane = threadIdx.x & (kWave - 1);
  const long row0 = (static_cast<long>(blockIdx.x) * (BLOCK / kWave) + threadIdx.x / kWave) * R;
  if (row0 >= a.rows) return;  // wave-uniform; this kernel has no workgroup barriers
  const int nch = a.n / V;
  const bool has_bias = a.bias != nullptr;

  // Every load is unconditional (see param_or): a lane past the row end (idx >= nch) and a row
  // past the last one read a clamped, valid chunk whose value is never used; absent parameters
  // read constant rows.
  auto load_params = [&](int idx, float (&g)[V], float (&b)[V], float (&bi)[V]) {
    const size_t i = static_cast<size_t>(idx) * V;
    const float* gp = param_or(a.gamma, i, kOnes8);
    const float* bp = param_or(a.beta, i, kZeros8);
    const float* bip = param_or(a.bias, i, kZeros8);
#pragma unroll
    for (int k = 0; k < V; k += 4) {
      load_f32x4(gp, k, &g[k]);
      load_f32x4(bp, k, &b[k]);
      load_f32x4(bip, k, &bi[k]);
    }
  };

  u32x4 xq[R][CPL], rq[R][CPL];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long row = row0 + r < a.rows ? row0 + r : a.rows - 1;
    const size_t base = static_cast<size_t>(row) * static_cast<size_t>(a.ld);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int idx = lane + c * kWave < nch ? lane + c * kWave : nch - 1;
      const size_t off = (base + static_cast<size_t>(idx) * V) * kEsz;
      xq[r][c] = ld16<NT>(static_cast<const char*>(a.x) + off);
      if constexpr (HAS_RES) rq[r][c] = ld16<NT>(static_cast<const char*>(a.res) + off);
    }
  }
  float pg[kCache ? CPL : 1][V], pb[kCache ? CPL : 1][V], pbias[kCache ? CPL : 1][V];
  if constexpr (kCache) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int idx = lane + c * kWave < nch ? lane + c * kWave : nch - 1;
      load_params(idx, pg[c], pb[c], pbias[c]);
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long row = row0 + r;
    if (row >= a.rows) break;  // wave-uniform
    const size_t base = static_cast<size_t>(row) * static_cast<size_t>(a.ld);
    float h[CPL][V];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int idx = lane + c * kWave;
      if (idx < nch) {
        S::unpack(xq[r][c], h[c]);
        if (has_bias) {
          float bi[V];
          if constexpr (kCache) {
#pragma unroll
            for (int k = 0; k < V; ++k) bi[k] = pbias[c][k];
          } else {
            const float* bip = param_or(a.bias, static_cast<size_t>(idx) * V, kZeros8);
#pragma unroll
            for (int k = 0; k < V; k += 4) load_f32x4(bip, k, &bi[k]);
          }
#pragma unroll
          for (int k = 0; k < V; ++k) h[c][k] = h[c][k] + bi[k];
        }
        if constexpr (HAS_RES) {
          float rv[V];
          S::unpack(rq[r][c], rv);
#pragma unroll
          for (int k = 0; k < V; ++k) h[c][k] = h[c][k] + rv[k];
        }
        s = c == 0 ? chunk_sum(h[c]) : s + chunk_sum(h[c]);
      } else {
#pragma unroll
        for (int k = 0; k < V; ++k) h[c][k] = 0.f;
      }
    }
    const float sum = wave_sum(s);
    const float mean = static_cast<float>(static_cast<double>(sum) * a.inv_n);
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int idx = lane + c * kWave;
      if (idx < nch) q = c == 0 ? chunk_sumsq(h[c], mean) : q + chunk_sumsq(h[c], mean);
    }
    const float sq = wave_sum(q);
    const float var = static_cast<float>(static_cast<double>(sq) * a.inv_n);
    const float rstd = __builtin_amdgcn_rsqf(var + static_cast<float>(a.eps));
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int idx = lane + c * kWave;
      if (idx < nch) {
        float g[V], b[V], bi_unused[V];
        if constexpr (kCache) {
#pragma unroll
          for (int k = 0; k < V; ++k) {
            g[k] = pg[c][k];
            b[k] = pb[c][k];
          }
        } else {
          load_params(idx, g, b, bi_unused);
        }
        float o[V];
#pragma unroll
        for (int k = 0; k < V; ++k) o[k] = __builtin_fmaf((h[c][k] - mean) * rstd, g[k], b[k]);
        S::template store<NT>(a.y, base + static_cast<size_t>(idx) * V, o);
      }
    }
  }
}

// Generic path: any n, any alignment. One wave per row, three strided sweeps (the row is re-read
// from cache instead of held in registers).
template <int DT>
__global__ __launch_bounds__(kLnBlock) void ln_rows_generic(LnArgs a) {
  using S = Store<DT>;
  const int lane = threadIdx.x & (kWave - 1);
  const long wave = static_cast<long>(blockIdx.x) * (kLnBlock / kWave) + (threadIdx.x / kWave);
  const long nwaves = static_cast<long>(gridDim.x) * (kLnBlock / kWave);
  for (long row = wave; row < a.rows; row += nwaves) {
    const size_t base = static_cast<size_t>(row) * static_cast<size_t>(a.ld);
    auto hval = [&](int j) {
      float v = S::load1(a.x, base + j);
      if (a.bias) v = v + a.bias[j];
      if (a.res) v = v + S::load1(a.res, base + j);
      return v;
    };
    float s = 0.f;
    for (int j = lane; j < a.n; j += kWave) s += hval(j);
    const float mean = static_cast<float>(static_cast<double>(wave_sum(s)) / static_cast<double>(a.n));
    float q = 0.f;
    for (int j = lane; j < a.n; j += kWave) {
      const float d = hval(j) - mean;
      q = __builtin_fmaf(d, d, q);
    }
    const float var = static_cast<float>(static_cast<double>(wave_sum(q)) / static_cast<double>(a.n));
    const float rstd = finish_rstd(var, a.eps);
    // Every lane has read all of its elements before any lane writes: the sweeps above end in a
    // wave-wide reduction, so in-place (y == x or y == res) is safe.
    for (int j = lane; j < a.n; j += kWave) {
      const float g = a.gamma ? a.gamma[j] : 1.f, b = a.beta ? a.beta[j] : 0.f;
      S::store1(a.y, base + j, __builtin_fmaf((hval(j) - mean) * rstd, g, b));
    }
  }
}

// ---- GroupNorm(groups = channels) + GELU --------------------------------------------------------

struct GnArgs {
  const void* x;
  const float* gamma;
  const float* beta;
  void* y;
  long channels;
  long T;
  long ld;
  double eps;
  int gelu;
};

constexpr int kGnBlock = 1024;
constexpr int kGnWaves = kGnBlock / kWave;


// Sum over the 1024-thread block of one float per thread (each a partial over ~T/1024 values):
// DPP wave sums in fp32, the 16 wave sums accumulated in double. Every thread gets the same value.
// (A double-precision shuffle reduction costs six LDS permutes per step of latency on the
// pipeline's critical path between two channels.)
__device__ __forceinline__ double block_sum(float v, double* red) {
  const float w_sum = wave_sum(v);
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = static_cast<double>(w_sum);
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int i = 0; i < kGnWaves; ++i) t += red[i];
  __syncthreads();
  return t;
}

// ---- GroupNorm with one channel per 512-thread workgroup, the row resident in registers ----------
// For rows of up to 512 * 16 chunks (32768 fp32 / 65536 16-bit elements): every workgroup loads
// its whole channel row with all 16-byte loads in flight, reduces, and writes it back normalized,
// two workgroups per CU. With as many workgroups as channels the hardware dispatcher starts the
// next channel on a CU as soon as one finishes, so no in-kernel pipeline is needed, and at the
// configuration's [512, 31999] every channel is resident at once: the call is one read of the
// tensor, the reductions, and one write.
constexpr int kGrBlock = 512;
constexpr int kGrWaves = kGrBlock / kWave;

__device__ __forceinline__ double block_sum512(float v, double* red) {
  const float w_sum = wave_sum(v);
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = static_cast<double>(w_sum);
  lds_barrier();
  double t = 0.0;
#pragma unroll
  for (int i = 0; i < kGrWaves; ++i) t += red[i];
  lds_barrier();
  return t;
}

// A channel row as this thread sees it: head elements up to the first 128-byte boundary, nbody
// 16-byte chunks (thread t owns chunks t, t + 1024, ...), then fewer than one chunk of tail
// elements. Thread t also owns head element t (t < head) or tail element t - head (head <= t <
// head + tail). Starting the body on a cache line keeps every wave access (1 KiB) on 8 lines
// instead of 9 when rows are not line-aligned ([512, 31999] fp32 rows are 127,996 bytes apart).
// x and y rows share their 16-byte phase (checked on the host).
struct GnRow {
  size_t base;   // element index of the row start
  size_t body0;  // element index of the first aligned chunk
  long nbody;
  long e_idx;    // this thread's head / tail element within the row, or -1
};

template <int DT>
__device__ __forceinline__ GnRow gn_row(const GnArgs& a, long ch) {
  constexpr int ESZ = DT == GSVK_F32 ? 4 : 2;
  constexpr int V = Store<DT>::VEC;
  GnRow r;
  r.base = static_cast<size_t>(ch) * static_cast<size_t>(a.ld);
  const uintptr_t addr = reinterpret_cast<uintptr_t>(a.x) + r.base * ESZ;
  long head = static_cast<long>(((128u - (addr & 127u)) & 127u) / ESZ);
  if (head > a.T) head = a.T;
  r.nbody = (a.T - head) / V;
  const long tail = a.T - head - r.nbody * V;
  r.body0 = r.base + head;
  const int t = threadIdx.x;
  r.e_idx = t < head ? t : (t < head + tail ? head + r.nbody * V + (t - head) : -1);
  return r;
}

// Issue the loads of one row into registers (raw 16-byte chunks: packed halves stay packed, 4
// VGPRs per chunk for every dtype).
template <int DT, int CPT, bool NT>
__device__ __forceinline__ void gn_load(const GnArgs& a, const GnRow& r, u32x4 (&raw)[CPT],
                                        float& e) {
  constexpr int ESZ = DT == GSVK_F32 ? 4 : 2;
  const char* xb = static_cast<const char*>(a.x) + r.body0 * ESZ;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const long k = threadIdx.x + static_cast<long>(c) * kGnBlock;
    if (k < r.nbody) raw[c] = ld16<NT>(xb + static_cast<size_t>(k) * 16);
    else raw[c] = u32x4{0u, 0u, 0u, 0u};  // zero bits are 0.0 in every dtype
  }
  e = r.e_idx >= 0 ? Store<DT>::load1(a.x, r.base + r.e_idx) : 0.f;
}

// Mean and rstd of one row held in registers (raw chunks + the head / tail element e). Contains
// workgroup barriers: every thread of the workgroup calls it for the same channel.
template <int DT, int CPT>
__device__ __forceinline__ void gn_stats(const GnArgs& a, const GnRow& r, const u32x4 (&raw)[CPT],
                                         float e, double* red, float& mean, float& rstd) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  float s = e;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    float v[V];
    S::unpack(raw[c], v);  // chunks past the row end hold zeros
#pragma unroll
    for (int i = 0; i < V; ++i) s += v[i];
  }
  const double mean_d = block_sum(s, red) / static_cast<double>(a.T);
  mean = static_cast<float>(mean_d);
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const long k = threadIdx.x + static_cast<long>(c) * kGnBlock;
    if (k < r.nbody) {
      float v[V];
      S::unpack(raw[c], v);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float d = v[i] - mean;
        q = __builtin_fmaf(d, d, q);
      }
    }
  }
  if (r.e_idx >= 0) {
    const float d = e - mean;
    q = __builtin_fmaf(d, d, q);
  }
  // Centred on the fp32 mean, corrected by (mean_d - mean)^2 so the variance is about mean_d.
  const double dm = mean_d - static_cast<double>(mean);
  const double var = block_sum(q, red) / static_cast<double>(a.T) - dm * dm;
  rstd = static_cast<float>(1.0 / sqrt((var > 0.0 ? var : 0.0) + a.eps));
}

// Workgroup b normalizes channels b, b + G, b + 2G, ... (G = gridDim.x, about one workgroup per
// CU) as a two-stage pipeline. Once a channel's statistics are known, its chunks are parked in LDS
// (each thread writes and later reads back only its own 16-byte slots, so no barrier orders them),
// the registers take the loads of the next channel, and the parked channel is normalized, passed
// through GELU and stored from LDS while those loads are in flight, so HBM keeps streaming during
// the compute phase. (With one channel per workgroup, the two co-resident workgroups of a CU load,
// compute and store in lockstep and HBM idles while the CU computes.) No workgroup waits for
// another.
template <int DT, int CPT, bool NT>
__global__ __launch_bounds__(kGnBlock) void gn_gelu_vec(GnArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  extern __shared__ u32x4 stage[];  // CPT * kGnBlock chunks; thread t owns stage[c * kGnBlock + t]
  __shared__ double red[kGnWaves];
  const long G = gridDim.x;
  long ch = blockIdx.x;  // workgroup-uniform
  GnRow r = gn_row<DT>(a, ch);
  u32x4 raw[CPT];
  float e;
  gn_load<DT, CPT, NT>(a, r, raw, e);
  while (ch < a.channels) {
    float mean, rstd;
    gn_stats<DT, CPT>(a, r, raw, e, red, mean, rstd);
#pragma unroll
    for (int c = 0; c < CPT; ++c) stage[c * kGnBlock + threadIdx.x] = raw[c];
    const GnRow cur = r;
    const float e_cur = e;
    const long next = ch + G;
    if (next < a.channels) {
      r = gn_row<DT>(a, next);
      gn_load<DT, CPT, NT>(a, r, raw, e);
    }
    const float g = a.gamma ? a.gamma[ch] : 1.f;
    const float b = a.beta ? a.beta[ch] : 0.f;
    // One chunk per iteration (8 or 4 independent elements): the prefetched channel occupies
    // CPT chunks of VGPRs meanwhile.
#pragma unroll 1
    for (int c = 0; c < CPT; ++c) {
      const long k = threadIdx.x + static_cast<long>(c) * kGnBlock;
      if (k < cur.nbody) {
        float v[V], o[V];
        S::unpack(stage[c * kGnBlock + threadIdx.x], v);
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const float y = __builtin_fmaf((v[i] - mean) * rstd, g, b);
          o[i] = a.gelu ? gelu_erf(y) : y;
        }
        S::template store<NT>(a.y, cur.body0 + static_cast<size_t>(k) * V, o);
      }
    }
    if (cur.e_idx >= 0) {
      const float y = __builtin_fmaf((e_cur - mean) * rstd, g, b);
      S::store1(a.y, cur.base + cur.e_idx, a.gelu ? gelu_erf(y) : y);
    }
    ch = next;
  }
}

// One channel per workgroup. The row layout is gn_row's (head to the first 128-byte line, 16-byte
// body chunks, tail), for 512 threads: thread t owns body chunks t, t + 512, ... and head / tail
// element t. Chunks past the body load the body's last chunk and count as zero (every load is
// unconditional, so all of them are in flight together). The statistics are gn_gelu_vec's: fp32
// partial sums, wave sums in fp32, the block sum in double, the centred second moment corrected by
// the fp32 mean's offset. Launch bounds of four waves per SIMD (at most 128 VGPRs) keep a second
// channel resident on every CU.
template <int DT, int CPT, bool NT>
__global__ __launch_bounds__(kGrBlock, 4) void gn_gelu_row(GnArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  constexpr int ESZ = DT == GSVK_F32 ? 4 : 2;
  __shared__ double red[kGrWaves];
  const long ch = blockIdx.x;
  const size_t base = static_cast<size_t>(ch) * static_cast<size_t>(a.ld);
  const uintptr_t addr = reinterpret_cast<uintptr_t>(a.x) + base * ESZ;
  long head = static_cast<long>(((128u - (addr & 127u)) & 127u) / ESZ);
  if (head > a.T) head = a.T;
  const long nbody = (a.T - head) / V;
  const long tail = a.T - head - nbody * V;
  const size_t body0 = base + head;
  const int t = threadIdx.x;
  const long e_idx = t < head ? t : (t < head + tail ? head + nbody * V + (t - head) : -1);
  const char* xb = static_cast<const char*>(a.x) + body0 * ESZ;
  const float g = *(a.gamma ? a.gamma + ch : kOnes8);
  const float b = *(a.beta ? a.beta + ch : kZeros8);
  u32x4 raw[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const long k = t + static_cast<long>(c) * kGrBlock;
    raw[c] = ld16<NT>(xb + static_cast<size_t>(k < nbody ? k : nbody - 1) * 16);
  }
  const float e_raw = S::load1(a.x, base + (e_idx >= 0 ? e_idx : 0));
  const float e = e_idx >= 0 ? e_raw : 0.f;
  float s = e;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const long k = t + static_cast<long>(c) * kGrBlock;
    float v[V];
    S::unpack(raw[c], v);
    float cs = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) cs += v[i];
    s += k < nbody ? cs : 0.f;
  }
  const double mean_d = block_sum512(s, red) / static_cast<double>(a.T);
  const float mean = static_cast<float>(mean_d);
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const long k = t + static_cast<long>(c) * kGrBlock;
    float v[V];
    S::unpack(raw[c], v);
    float cq = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float d = v[i] - mean;
      cq = __builtin_fmaf(d, d, cq);
    }
    q += k < nbody ? cq : 0.f;
  }
  if (e_idx >= 0) {
    const float d = e - mean;
    q = __builtin_fmaf(d, d, q);
  }
  const double dm = mean_d - static_cast<double>(mean);
  const double var = block_sum512(q, red) / static_cast<double>(a.T) - dm * dm;
  const float rstd = static_cast<float>(1.0 / sqrt((var > 0.0 ? var : 0.0) + a.eps));
  // Every thread has read all of its elements before any thread writes (the reductions above end
  // in workgroup barriers), so y == x in place is safe.
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const long k = t + static_cast<long>(c) * kGrBlock;
    if (k < nbody) {
      float v[V], o[V];
      S::unpack(raw[c], v);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float y = __builtin_fmaf((v[i] - mean) * rstd, g, b);
        o[i] = a.gelu ? gelu_erf(y) : y;
      }
      S::template store<NT>(a.y, body0 + static_cast<size_t>(k) * V, o);
    }
  }
  if (e_idx >= 0) {
    const float y = __builtin_fmaf((e - mean) * rstd, g, b);
    S::store1(a.y, base + e_idx, a.gelu ? gelu_erf(y) : y);
  }
}

// Any T / alignment: three strided sweeps over the channel row.
template <int DT>
__global__ __launch_bounds__(kGnBlock) void gn_gelu_generic(GnArgs a) {
  using S = Store<DT>;
  __shared__ double red[kGnWaves];
  const long ch = blockIdx.x;
  const size_t base = static_cast<size_t>(ch) * static_cast<size_t>(a.ld);
  float s = 0.f;
  for (long j = threadIdx.x; j < a.T; j += kGnBlock) s += S::load1(a.x, base + j);
  const double mean_d = block_sum(s, red) / static_cast<double>(a.T);
  const float mean = static_cast<float>(mean_d);
  float q = 0.f;
  for (long j = threadIdx.x; j < a.T; j += kGnBlock) {
    const float d = S::load1(a.x, base + j) - mean;
    q = __builtin_fmaf(d, d, q);
  }
  const double dm = mean_d - static_cast<double>(mean);
  const double var = block_sum(q, red) / static_cast<double>(a.T) - dm * dm;
  const float rstd = static_cast<float>(1.0 / sqrt((var > 0.0 ? var : 0.0) + a.eps));
  const float g = a.gamma ? a.gamma[ch] : 1.f;
  const float b = a.beta ? a.beta[ch] : 0.f;
  // block_sum ends with a barrier after every thread's last read, so in-place writes are safe.
  for (long j = threadIdx.x; j < a.T; j += kGnBlock) {
    const float y = __builtin_fmaf((S::load1(a.x, base + j) - mean) * rstd, g, b);
    S::store1(a.y, base + j, a.gelu ? gelu_erf(y) : y);
  }
}

// ---- launchers ----------------------------------------------------------------------------------

int ln_grid(long rows) {
  // generic path: 2048 workgroups (8 per CU on 256 CUs); waves stride over the rest
  const long need = (rows + (kLnBlock / kWave) - 1) / (kLnBlock / kWave);
  return static_cast<int>(need < 2048 ? need : 2048);
}

// Workgroups per launch of the tiled path (a dispatch holds at most 2^32 - 1 work-items).
constexpr long kLnMaxGrid = 1L << 22;

template <int DT, int CPL, int R, bool NT, int BLOCK>
void launch_ln_tile(LnArgs a, hipStream_t st) {
  const bool has_res = a.res != nullptr;
  constexpr size_t esz = DT == GSVK_F32 ? 4 : 2;
  const long rows_per_block = (BLOCK / kWave) * R;
  const long rows_per_launch = kLnMaxGrid * rows_per_block;
  const long total = a.rows;
  const void* x0 = a.x;
  const void* r0p = a.res;
  void* y0 = a.y;
  for (long r0 = 0; r0 < total; r0 += rows_per_launch) {
    const size_t off = static_cast<size_t>(r0) * a.ld * esz;
    a.rows = total - r0 < rows_per_launch ? total - r0 : rows_per_launch;
    a.x = static_cast<const char*>(x0) + off;
    a.res = r0p ? static_cast<const char*>(r0p) + off : nullptr;
    a.y = static_cast<char*>(y0) + off;
    const unsigned grid = static_cast<unsigned>((a.rows + rows_per_block - 1) / rows_per_block);
    if (has_res)
      hipLaunchKernelGGL((ln_rows_tile<DT, CPL, R, NT, BLOCK, true>), dim3(grid), dim3(BLOCK), 0, st, a);
    else
      hipLaunchKernelGGL((ln_rows_tile<DT, CPL, R, NT, BLOCK, false>), dim3(grid), dim3(BLOCK), 0, st, a);
  }
}

// Short jobs (latency-bound, e.g. one decode step's [64, 512]): one row per wave, one wave per
// workgroup (measured on MI355X: 2.35 us per launch against 2.59 with four-wave workgroups and a
// double-precision finalize). Long jobs: four-wave workgroups, two rows per wave up to 1024 f16 /
// 512 f32 columns (f16 rows of 512: 77% of 8 TB/s with two rows per wave, 61% with four).
constexpr long kLnManyRows = 8192;

template <int DT, bool NT>
void launch_ln_vec(const LnArgs& a, int nch, hipStream_t st) {
  const bool many = a.rows >= kLnManyRows;
  if (nch <= 1 * kWave) {
    if (many) launch_ln_tile<DT, 1, 2, NT, 256>(a, st);
    else launch_ln_tile<DT, 1, 1, NT, 64>(a, st);
  } else if (nch <= 2 * kWave) {
    if (many) launch_ln_tile<DT, 2, 2, NT, 256>(a, st);
    else launch_ln_tile<DT, 2, 1, NT, 64>(a, st);
  } else if (nch <= 4 * kWave) {
    if (many) launch_ln_tile<DT, 4, 1, NT, 256>(a, st);
    else launch_ln_tile<DT, 4, 1, NT, 64>(a, st);
  } else {
    if (many) launch_ln_tile<DT, 8, 1, NT, 256>(a, st);
    else launch_ln_tile<DT, 8, 1, NT, 64>(a, st);
  }
}

template <int DT>
int launch_ln(const LnArgs& a, bool vec_ok, hipStream_t st) {
  constexpr int V = Store<DT>::VEC;
  const int nch = a.n / V;
  if (vec_ok && nch <= 8 * kWave) {
    const size_t bytes = static_cast<size_t>(a.rows) * a.n * (DT == GSVK_F32 ? 4 : 2) * (a.res ? 3 : 2);
    if (bytes >= kStreamBytes) launch_ln_vec<DT, true>(a, nch, st);
    else launch_ln_vec<DT, false>(a, nch, st);
  } else {
    hipLaunchKernelGGL((ln_rows_generic<DT>), dim3(ln_grid(a.rows)), dim3(kLnBlock), 0, st, a);
  }
  return launch_status();
}

// False (nothing launched) when the runtime refuses the LDS the tile needs.
template <int DT, int CPT, bool NT>
bool launch_gn_cpt(const GnArgs& a, hipStream_t st) {
  constexpr size_t lds = static_cast<size_t>(CPT) * kGnBlock * 16;  // 16-128 KiB of the 160 KiB
  static std::atomic<bool> lds_ok[kMaxDevices];
  if (lds > 64 * 1024 &&
      !allow_dynamic_lds(reinterpret_cast<const void*>(&gn_gelu_vec<DT, CPT, NT>), lds, lds_ok))
    return false;
  // one workgroup per CU (two when the staging buffer leaves room for a second one)
  const long slots = device_cus() * (lds <= 64 * 1024 ? 2 : 1);
  const dim3 grid(static_cast<unsigned>(a.channels < slots ? a.channels : slots));
  hipLaunchKernelGGL((gn_gelu_vec<DT, CPT, NT>), grid, dim3(kGnBlock), lds, st, a);
  return true;
}

template <int DT, bool NT>
bool launch_gn_vec(const GnArgs& a, hipStream_t st) {
  constexpr int V = Store<DT>::VEC;
  const long nb = a.T / V + 1;  // upper bound on body chunks
  if (nb <= 1L * kGnBlock) return launch_gn_cpt<DT, 1, NT>(a, st);
  if (nb <= 2L * kGnBlock) return launch_gn_cpt<DT, 2, NT>(a, st);
  if (nb <= 4L * kGnBlock) return launch_gn_cpt<DT, 4, NT>(a, st);
  if (nb <= 8L * kGnBlock) return launch_gn_cpt<DT, 8, NT>(a, st);
  return false;
}

template <int DT, bool NT>
void launch_gn_row(const GnArgs& a, long nb, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(a.channels));
  if (nb <= 4L * kGrBlock)
    hipLaunchKernelGGL((gn_gelu_row<DT, 4, NT>), grid, dim3(kGrBlock), 0, st, a);
  else if (DT != GSVK_F32 || nb <= 8L * kGrBlock)
    hipLaunchKernelGGL((gn_gelu_row<DT, 8, NT>), grid, dim3(kGrBlock), 0, st, a);
  else if constexpr (DT == GSVK_F32)
    hipLaunchKernelGGL((gn_gelu_row<DT, 16, NT>), grid, dim3(kGrBlock), 0, st, a);
}

template <int DT>
int launch_gn(const GnArgs& a, bool vec_ok, hipStream_t st) {
  constexpr long kEsz = DT == GSVK_F32 ? 4 : 2;
  constexpr int V = Store<DT>::VEC;
  const size_t bytes = 2 * static_cast<size_t>(a.channels) * a.T * kEsz;
  const long nb = a.T / V + 1;  // upper bound on body chunks
  // The resident-row kernel: rows of at least two 128-byte lines (its clamped loads need one whole
  // body chunk) and at most 16 chunks per thread for fp32, 8 for 16-bit types (32768 elements;
  // 16 chunks of packed 16-bit values do not fit 128 VGPRs with their fp32 temporaries).
  if (vec_ok && a.T >= 2 * (128 / kEsz) && nb <= (DT == GSVK_F32 ? 16L : 8L) * kGrBlock) {
    if (bytes >= kStreamBytes) launch_gn_row<DT, true>(a, nb, st);
    else launch_gn_row<DT, false>(a, nb, st);
    return launch_status();
  }
  if (vec_ok) vec_ok = bytes >= kStreamBytes ? launch_gn_vec<DT, true>(a, st) : launch_gn_vec<DT, false>(a, st);
  if (!vec_ok)
    hipLaunchKernelGGL((gn_gelu_generic<DT>), dim3(static_cast<unsigned>(a.channels)), dim3(kGnBlock), 0, st, a);
  return launch_status();
}

}  // namespace
}  // namespace gsvk

using namespace gsvk;

extern "C" int gsvk_add_layernorm(int dtype, const void* x, const float* bias, const void* residual,
                                  const float* gamma, const float* beta, void* y, size_t rows,
                                  size_t n, size_t ld, double eps, void* stream) {
  if (!valid_dtype(dtype)) return GSVK_E_DTYPE;
  if (!x || !y) return GSVK_E_NULL;
  if (rows == 0 || n == 0 || ld < n || n > (1u << 30) || rows > (1ul << 40)) return GSVK_E_SIZE;
  if (!(eps >= 0.0) || !std::isfinite(eps)) return GSVK_E_ARG;
  const size_t esz = dtype_size(dtype);
  const size_t span = span_bytes(rows, n, ld, esz);
  // y may be exactly x or exactly residual; any other overlap with an input is rejected.
  if (y != x && overlaps(y, span, x, span)) return GSVK_E_ALIAS;
  if (residual && y != residual && overlaps(y, span, residual, span)) return GSVK_E_ALIAS;
  for (const float* p : {bias, gamma, beta})
    if (p && overlaps(y, span, p, n * sizeof(float))) return GSVK_E_ALIAS;

  LnArgs a{x, bias, residual, gamma, beta, y, static_cast<long>(rows), static_cast<int>(n),
           static_cast<long>(ld), eps, 1.0 / static_cast<double>(n)};
  const int V = dtype == GSVK_F32 ? 4 : 8;
  bool vec_ok = (n % V == 0) && (ld % V == 0) && aligned16(x) && aligned16(y) &&
                (!residual || aligned16(residual));
  for (const float* p : {bias, gamma, beta}) vec_ok = vec_ok && (!p || aligned16(p));
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case GSVK_F32: return launch_ln<GSVK_F32>(a, vec_ok, st);
    case GSVK_F16: return launch_ln<GSVK_F16>(a, vec_ok, st);
    default: return launch_ln<GSVK_BF16>(a, vec_ok, st);
  }
}

extern "C" int gsvk_groupnorm_gelu(int dtype, const void* x, const float* gamma, const float* beta,
                                   void* y, size_t channels, size_t T, size_t ld, double eps,
                                   int apply_gelu, void* stream) {
  if (!valid_dtype(dtype)) return GSVK_E_DTYPE;
  if (!x || !y) return GSVK_E_NULL;
  // one 1024-thread workgroup per channel: a dispatch holds at most 2^32 - 1 work-items
  if (channels == 0 || T == 0 || ld < T || channels >= (1ul << 22) || T > (1ul << 40))
    return GSVK_E_SIZE;
  if (!(eps >= 0.0) || !std::isfinite(eps)) return GSVK_E_ARG;
  const size_t esz = dtype_size(dtype);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % esz) return GSVK_E_ARG;
  const size_t span = span_bytes(channels, T, ld, esz);
  if (y != x && overlaps(y, span, x, span)) return GSVK_E_ALIAS;
  for (const float* p : {gamma, beta})
    if (p && overlaps(y, span, p, channels * sizeof(float))) return GSVK_E_ALIAS;
  GnArgs a{x, gamma, beta, y, static_cast<long>(channels), static_cast<long>(T),
           static_cast<long>(ld), eps, apply_gelu ? 1 : 0};
  // The register path needs x and y rows in the same 16-byte phase.
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(x) - reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case GSVK_F32: return launch_gn<GSVK_F32>(a, vec_ok, st);
    case GSVK_F16: return launch_gn<GSVK_F16>(a, vec_ok, st);
    default: return launch_gn<GSVK_BF16>(a, vec_ok, st);
  }
}
