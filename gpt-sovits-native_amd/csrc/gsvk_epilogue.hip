// gsvk_epilogue.hip — bias + activation over rows, LeakyReLU, and the SoVITS ResBlock element-wise
// steps (residual add + LeakyReLU, 3-branch average + next-stage LeakyReLU) for gfx950.
//
// All of these are pure streams: each output element depends on the same element of the inputs
// (plus a per-column bias). Tiling is one-shot: workgroup b owns one contiguous tile of 16-byte
// chunks and exits after a single load-compute-store pass, so the waves in flight on the chip always
// cover one compact window of memory that advances with the dispatch order. Each thread loads all of
// its chunks before it computes. Calls that move more than the MALL holds read and write their
// operands non-temporally (kStreamBytes).
// (Measured on MI355X: persistent grid-stride loops over the same data plateau at ~57% of 8 TB/s,
// one-shot tiles of 4-16 KiB per operand reach 75-80%.)
//
// Bit-exactness: every result is the reference's sequence of single-rounded fp32 operations (this
// file is built with -ffp-contract=off, so no multiply-add is fused unless written as fmaf).
#include <cmath>

#include <algorithm>

#include "gsvk_common.hpp"

namespace gsvk {
namespace {

constexpr int kBlock = 256;
// Workgroups per launch: a dispatch holds at most 2^32 - 1 work-items per dimension, so larger jobs
// are split into several launches on the host.
constexpr long kMaxGrid = 1L << 22;

// ---- bias + activation over [rows, n] ------------------------------------------------------------

struct BaArgs {
  const void* x;
  const float* bias;
  void* y;
  long rows;   // rows in this launch
  long n;
  long ld;
  long nch;    // 16-byte chunks per row
  int wshift;  // log2 of W, the threads per row slice (64, 128 or 256)
  float slope;
};

// Workgroup (bx, by) covers column tile bx (W chunks) of row group by (P = kBlock / W row slices of
// U rows each, P*U consecutive rows); x-fastest dispatch order walks a row group's column tiles
// back to back. A thread keeps its bias chunk in VGPRs for its U rows. When a row is shorter than
// kBlock chunks, one workgroup covers several whole rows, so the tile stays contiguous for
// row-major data.
template <int DT, int ACT, int U, bool NT>
__global__ __launch_bounds__(kBlock) void bias_act_tile(BaArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  const long bx = blockIdx.x, by = blockIdx.y;
  const int P = kBlock >> a.wshift;  // shifts, not divisions: nothing delays the first load
  const int tc = threadIdx.x & ((1 << a.wshift) - 1), tr = threadIdx.x >> a.wshift;
  const long c = (bx << a.wshift) + tc;
  if (c >= a.nch) return;  // no barriers below: idle lanes of a partial tile just leave
  float bi[V];
  // no bias: add -0, which changes nothing (the reference applies no bias add at all)
  const float* bp = param_or(a.bias, static_cast<size_t>(c) * V, kNegZeros8);
#pragma unroll
  for (int k = 0; k < V; k += 4) load_f32x4(bp, k, &bi[k]);
  const long r0 = by * static_cast<long>(P) * U + tr;
  float v[U][V];
#pragma unroll
  for (int u = 0; u < U; ++u) {  // rows past the end re-read the last row (discarded)
    long r = r0 + static_cast<long>(u) * P;
    r = r < a.rows ? r : a.rows - 1;
    S::template load<NT>(a.x, static_cast<size_t>(r) * a.ld + c * V, v[u]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long r = r0 + static_cast<long>(u) * P;
    if (r < a.rows) {
#pragma unroll
      for (int k = 0; k < V; ++k) v[u][k] = act_apply<ACT>(v[u][k] + bi[k], a.slope);
      S::template store<NT>(a.y, static_cast<size_t>(r) * a.ld + c * V, v[u]);
    }
  }
}

// Any width / alignment: one element per thread, grid-stride (fallback path).
template <int DT, int ACT>
__global__ __launch_bounds__(kBlock) void bias_act_generic(BaArgs a) {
  using S = Store<DT>;
  const long total = a.rows * a.n;
  const long stride = static_cast<long>(gridDim.x) * kBlock;
  for (long i = static_cast<long>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride) {
    const long r = i / a.n, c = i - r * a.n;
    const size_t off = static_cast<size_t>(r) * a.ld + c;
    const float b = a.bias ? a.bias[c] : -0.f;
    S::store1(a.y, off, act_apply<ACT>(S::load1(a.x, off) + b, a.slope));
  }
}

// ---- flat element-wise streams -------------------------------------------------------------------

struct EwArgs {
  const void* in[8];  // operands (see each kernel)
  void* out[2];
  long n;             // elements
  float slope;
  int flag;
  int nbranch;
};

// Chunk u of this thread in the workgroup's tile: tile b = chunks [b*kBlock*U, (b+1)*kBlock*U).
template <int U>
__device__ __forceinline__ long tile_chunk(int u) {
  return static_cast<long>(blockIdx.x) * (kBlock * U) + u * kBlock + threadIdx.x;
}
// Chunk to load for tile_chunk(u): clamped to the last whole chunk (nch > 0), so loads need no
// branch; the value loaded for an out-of-range chunk is discarded.
template <int U>
__device__ __forceinline__ long load_chunk(int u, long nch) {
  const long c = tile_chunk<U>(u);
  return c < nch ? c : nch - 1;
}
// The n % VEC trailing elements are handled one per thread by the last workgroup.
template <int V>
__device__ __forceinline__ long tail_elem(long n) {
  if (blockIdx.x != gridDim.x - 1) return -1;
  const long i = (n / V) * V + threadIdx.x;
  return i < n ? i : -1;
}

// y = lrelu(x, slope)
template <int DT, int U, bool NT>
__global__ __launch_bounds__(kBlock) void lrelu_tile(EwArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  const long nch = a.n / V;
  if (nch > 0) {
    float v[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u) S::template load<NT>(a.in[0], load_chunk<U>(u, nch) * V, v[u]);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (tile_chunk<U>(u) < nch) {
#pragma unroll
        for (int k = 0; k < V; ++k) v[u][k] = lrelu_ref(v[u][k], a.slope);
        S::template store<NT>(a.out[0], tile_chunk<U>(u) * V, v[u]);
      }
  }
  const long i = tail_elem<V>(a.n);
  if (i >= 0) S::store1(a.out[0], i, lrelu_ref(S::load1(a.in[0], i), a.slope));
}

// cur += t_b; t_in = lrelu(cur)   (flag = 1 when t_in is written)
template <int DT, int U, bool NT>
__global__ __launch_bounds__(kBlock) void res_add_lrelu_tile(EwArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  const long nch = a.n / V;
  void* cur = a.out[0];
  void* tin = a.out[1];
  if (nch > 0) {
    float c[U][V], t[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      S::template load<NT>(cur, load_chunk<U>(u, nch) * V, c[u]);
      S::template load<NT>(a.in[0], load_chunk<U>(u, nch) * V, t[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (tile_chunk<U>(u) < nch) {
#pragma unroll
        for (int k = 0; k < V; ++k) c[u][k] = c[u][k] + t[u][k];
        S::template store<NT>(cur, tile_chunk<U>(u) * V, c[u]);
        if (a.flag) {
#pragma unroll
          for (int k = 0; k < V; ++k) t[u][k] = lrelu_ref(c[u][k], a.slope);
          S::template store<NT>(tin, tile_chunk<U>(u) * V, t[u]);
        }
      }
  }
  const long i = tail_elem<V>(a.n);
  if (i >= 0) {
    const float v = S::load1(cur, i) + S::load1(a.in[0], i);
    S::store1(cur, i, v);
    if (a.flag) S::store1(tin, i, lrelu_ref(v, a.slope));
  }
}

// out = lrelu( sum_j (cur_j [+ tb_j]) * kinv ), summed left to right with separate roundings.
// in[0..3] = cur_j, in[4..7] = tb_j (NULL when absent); flag = apply_lrelu. All 2*NB operand
// chunks are loaded before any arithmetic.
// HAS_T: every branch has its t_b operand (the launcher takes the scalar kernel when only some do).
template <int DT, int NB, bool NT, bool HAS_T>
__global__ __launch_bounds__(kBlock) void branch_mean_tile(EwArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  constexpr float kInv = 1.f / static_cast<float>(NB);
  const long nch = a.n / V;
  const long c = tile_chunk<1>(0);
  if (c < nch) {  // one chunk per thread: this branch holds every load of the thread
    float cv[NB][V], tv[NB][V];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      S::template load<NT>(a.in[j], c * V, cv[j]);
      if constexpr (HAS_T) S::template load<NT>(a.in[4 + j], c * V, tv[j]);
    }
    float acc[V];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
#pragma unroll
      for (int k = 0; k < V; ++k) {
        const float v = HAS_T ? cv[j][k] + tv[j][k] : cv[j][k];
        acc[k] = j == 0 ? v * kInv : acc[k] + v * kInv;
      }
    }
    if (a.flag) {
#pragma unroll
      for (int k = 0; k < V; ++k) acc[k] = lrelu_ref(acc[k], a.slope);
    }
    S::template store<NT>(a.out[0], c * V, acc);
  }
  const long i = tail_elem<V>(a.n);
  if (i >= 0) {
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
template <int DT, int U, bool NT>
__global__ __launch_bounds__(kBlock) void scaled_add_tile(EwArgs a) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  const long nch = a.n / V;
  const bool has_acc = a.in[0] != nullptr;
  // Without acc the src chunk is read twice instead of branching around the acc load.
  const void* accp = has_acc ? a.in[0] : a.in[1];
  if (nch > 0) {
    float s[U][V], q[U][V];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      S::template load<NT>(a.in[1], load_chunk<U>(u, nch) * V, s[u]);
      S::template load<NT>(accp, load_chunk<U>(u, nch) * V, q[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (tile_chunk<U>(u) < nch) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
          const float v = s[u][k] * a.slope;
          s[u][k] = has_acc ? q[u][k] + v : v;
        }
        S::template store<NT>(a.out[0], tile_chunk<U>(u) * V, s[u]);
      }
  }
  const long i = tail_elem<V>(a.n);
  if (i >= 0) {
    const float v = S::load1(a.in[1], i) * a.slope;
    S::store1(a.out[0], i, has_acc ? S::load1(a.in[0], i) + v : v);
  }
}

// Scalar fallbacks for buffers that are not 16-byte aligned (grid-stride).
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

unsigned stride_grid(long items) {
  long b = (items + kBlock - 1) / kBlock;
  if (b < 1) b = 1;
  return static_cast<unsigned>(b < 2048 ? b : 2048);
}

// One-shot grid over nch chunks with U chunks per thread; at least one workgroup so that the
// tail elements are handled even when there is no whole chunk.
unsigned tile_grid(long nch, int U) {
  const long per = static_cast<long>(kBlock) * U;
  long b = (nch + per - 1) / per;
  return static_cast<unsigned>(b < 1 ? 1 : b);
}

// log2 of the threads per row slice: the width (64, 128 or 256) that leaves the fewest idle lanes
// in the last column tile, preferring the wider one on a tie.
int slice_shift(long nch) {
  int best = 8;
  long best_idle = -1;
  for (int sh : {8, 7, 6}) {
    const long w = 1L << sh;
    const long idle = ((nch + w - 1) / w) * w - nch;
    if (best_idle < 0 || idle < best_idle) {
      best = sh;
      best_idle = idle;
    }
  }
  return best;
}

// Rows per thread in bias_act_tile: several for streaming calls (more bytes in flight per thread:
// four for 16-bit storage, two for fp32), one for small calls (more workgroups: latency-bound
// launches finish sooner). Row groups go on grid.y, at most 65535 per launch.
template <int DT, int ACT, int U, bool NT>
void launch_bias_act_tile(BaArgs a, hipStream_t st) {
  const long W = 1L << a.wshift;
  const long rows_per_group = (kBlock / W) * U;
  const long rows_per_launch = 65535L * rows_per_group;
  const unsigned gx = static_cast<unsigned>((a.nch + W - 1) / W);
  const long total_rows = a.rows;
  const void* x0 = a.x;
  void* y0 = a.y;
  constexpr size_t esz = DT == GSVK_F32 ? 4 : 2;
  for (long r0 = 0; r0 < total_rows; r0 += rows_per_launch) {
    a.rows = total_rows - r0 < rows_per_launch ? total_rows - r0 : rows_per_launch;
    a.x = static_cast<const char*>(x0) + static_cast<size_t>(r0) * a.ld * esz;
    a.y = static_cast<char*>(y0) + static_cast<size_t>(r0) * a.ld * esz;
    const unsigned gy = static_cast<unsigned>((a.rows + rows_per_group - 1) / rows_per_group);
    hipLaunchKernelGGL((bias_act_tile<DT, ACT, U, NT>), dim3(gx, gy), dim3(kBlock), 0, st, a);
  }
}

template <int ACT>
int launch_bias_act(int dt, BaArgs a, bool vec_ok, hipStream_t st) {
  if (vec_ok) {
    a.nch = a.n / (dt == GSVK_F32 ? 4 : 8);
    a.wshift = slice_shift(a.nch);
    const bool stream = 2 * static_cast<size_t>(a.rows) * a.n * dtype_size(dt) >= kStreamBytes;
    switch (dt) {
      case GSVK_F32:
        if (stream) launch_bias_act_tile<GSVK_F32, ACT, 2, true>(a, st);
        else launch_bias_act_tile<GSVK_F32, ACT, 1, false>(a, st);
        break;
      case GSVK_F16:
        if (stream) launch_bias_act_tile<GSVK_F16, ACT, 4, true>(a, st);
        else launch_bias_act_tile<GSVK_F16, ACT, 1, false>(a, st);
        break;
      default:
        if (stream) launch_bias_act_tile<GSVK_BF16, ACT, 4, true>(a, st);
        else launch_bias_act_tile<GSVK_BF16, ACT, 1, false>(a, st);
        break;
    }
  } else {
    const unsigned g = stride_grid(a.rows * a.n);
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
  hipLaunchKernelGGL((ew_scalar<DT>), dim3(stride_grid(a.n)), dim3(kBlock), 0, st, a, op);
}

void launch_scalar_dt(int dt, const EwArgs& a, int op, hipStream_t st) {
  switch (dt) {
    case GSVK_F32: launch_scalar<GSVK_F32>(a, op, st); break;
    case GSVK_F16: launch_scalar<GSVK_F16>(a, op, st); break;
    default: launch_scalar<GSVK_BF16>(a, op, st); break;
  }
}

// Chunks per thread of the flat kernels: one for the single-operand LeakyReLU and the six-operand
// branch mean, two for the two-operand residual add and scaled add.
constexpr int kLreluU = 1, kResU = 2, kScaledU = 2;

// Runs `launch(args, grid)` over the n elements in segments of at most kMaxGrid workgroups of
// kBlock*U chunks each; every operand pointer is advanced to the segment start. Segment lengths are
// multiples of the chunk size, so only the last segment has tail elements.
template <int DT, typename L>
void launch_flat(const EwArgs& a, int U, hipStream_t st, L launch) {
  constexpr long V = Store<DT>::VEC;
  constexpr size_t esz = DT == GSVK_F32 ? 4 : 2;
  const long seg = kMaxGrid * kBlock * U * V;
  for (long off = 0; off < a.n; off += seg) {
    EwArgs b = a;
    b.n = a.n - off < seg ? a.n - off : seg;
    for (int i = 0; i < 8; ++i)
      if (a.in[i]) b.in[i] = static_cast<const char*>(a.in[i]) + static_cast<size_t>(off) * esz;
    for (int i = 0; i < 2; ++i)
      if (a.out[i]) b.out[i] = static_cast<char*>(a.out[i]) + static_cast<size_t>(off) * esz;
    launch(b, tile_grid(b.n / V, U), st);
  }
}

// Streaming (non-temporal) access when the call moves `operands` arrays of n elements totalling at
// least kStreamBytes.
template <int DT>
bool streams(const EwArgs& a, int operands) {
  return static_cast<size_t>(operands) * a.n * (DT == GSVK_F32 ? 4 : 2) >= kStreamBytes;
}

template <int DT, int NB, bool NT>
void launch_branch_mean_nb(const EwArgs& a, hipStream_t st) {
  if (a.in[4]) {
    launch_flat<DT>(a, 1, st, [](const EwArgs& b, unsigned g, hipStream_t s) {
      hipLaunchKernelGGL((branch_mean_tile<DT, NB, NT, true>), dim3(g), dim3(kBlock), 0, s, b);
    });
  } else {
    launch_flat<DT>(a, 1, st, [](const EwArgs& b, unsigned g, hipStream_t s) {
      hipLaunchKernelGGL((branch_mean_tile<DT, NB, NT, false>), dim3(g), dim3(kBlock), 0, s, b);
    });
  }
}

template <int DT, bool NT>
void launch_branch_mean_nt(const EwArgs& a, hipStream_t st) {
  switch (a.nbranch) {
    case 1: launch_branch_mean_nb<DT, 1, NT>(a, st); break;
    case 2: launch_branch_mean_nb<DT, 2, NT>(a, st); break;
    case 3: launch_branch_mean_nb<DT, 3, NT>(a, st); break;
    default: launch_branch_mean_nb<DT, 4, NT>(a, st); break;
  }
}

template <int DT>
void launch_branch_mean(const EwArgs& a, hipStream_t st) {
  int ops = 1;
  for (int j = 0; j < a.nbranch; ++j) ops += 1 + (a.in[4 + j] != nullptr);
  if (streams<DT>(a, ops)) launch_branch_mean_nt<DT, true>(a, st);
  else launch_branch_mean_nt<DT, false>(a, st);
}

template <int DT, bool NT>
void launch_lrelu_nt(const EwArgs& a, hipStream_t st) {
  launch_flat<DT>(a, kLreluU, st, [](const EwArgs& b, unsigned g, hipStream_t s) {
    hipLaunchKernelGGL((lrelu_tile<DT, kLreluU, NT>), dim3(g), dim3(kBlock), 0, s, b);
  });
}

template <int DT>
void launch_lrelu(const EwArgs& a, hipStream_t st) {
  if (streams<DT>(a, 2)) launch_lrelu_nt<DT, true>(a, st);
  else launch_lrelu_nt<DT, false>(a, st);
}

template <int DT, bool NT>
void launch_res_add_nt(const EwArgs& a, hipStream_t st) {
  launch_flat<DT>(a, kResU, st, [](const EwArgs& b, unsigned g, hipStream_t s) {
    hipLaunchKernelGGL((res_add_lrelu_tile<DT, kResU, NT>), dim3(g), dim3(kBlock), 0, s, b);
  });
}

template <int DT>
void launch_res_add(const EwArgs& a, hipStream_t st) {
  if (streams<DT>(a, a.flag ? 4 : 3)) launch_res_add_nt<DT, true>(a, st);
  else launch_res_add_nt<DT, false>(a, st);
}

template <int DT, bool NT>
void launch_scaled_add_nt(const EwArgs& a, hipStream_t st) {
  launch_flat<DT>(a, kScaledU, st, [](const EwArgs& b, unsigned g, hipStream_t s) {
    hipLaunchKernelGGL((scaled_add_tile<DT, kScaledU, NT>), dim3(g), dim3(kBlock), 0, s, b);
  });
}

template <int DT>
void launch_scaled_add(const EwArgs& a, hipStream_t st) {
  if (streams<DT>(a, a.in[0] ? 3 : 2)) launch_scaled_add_nt<DT, true>(a, st);
  else launch_scaled_add_nt<DT, false>(a, st);
}

// fp32 -> fp16 storage, round to nearest even (subnormals kept, overflow to inf, NaN stays NaN):
// kern::f32_to_f16 (gemv_fmlal.cpp:23-35, vcvt_f16_f32). 8 elements per thread per step from 32
// aligned bytes (vec), else one.
__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float* __restrict__ x,
                                                         uint16_t* __restrict__ y, long n, int vec) {
  const long stride = static_cast<long>(gridDim.x) * blockDim.x;
  const long t0 = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (vec) {
    const long n8 = n / 8;
    for (long i = t0; i < n8; i += stride) {
      const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
      const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
      reinterpret_cast<uint4*>(y)[i] =
          uint4{f2h2(a.x, a.y), f2h2(a.z, a.w), f2h2(b.x, b.y), f2h2(b.z, b.w)};
    }
    for (long i = n8 * 8 + t0; i < n; i += stride) y[i] = static_cast<uint16_t>(f2h(x[i]));
  } else {
    for (long i = t0; i < n; i += stride) y[i] = static_cast<uint16_t>(f2h(x[i]));
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
  if (rows == 0 || n == 0 || ld < n || rows > (1ul << 40) || n > (1ul << 30) || ld > (1ul << 40) ||
      rows * ld > (1ul << 42))
    return GSVK_E_SIZE;
  const size_t esz = dtype_size(dtype);
  const size_t span = span_bytes(rows, n, ld, esz);
  if (y != x && overlaps(y, span, x, span)) return GSVK_E_ALIAS;
  if (bias && overlaps(y, span, bias, n * sizeof(float))) return GSVK_E_ALIAS;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % esz) return GSVK_E_ARG;
  const int V = dtype == GSVK_F32 ? 4 : 8;
  const bool vec_ok = n % V == 0 && ld % V == 0 && aligned16(x) && aligned16(y) &&
                      (!bias || aligned16(bias));
  BaArgs a{x, bias, y, static_cast<long>(rows), static_cast<long>(n), static_cast<long>(ld), 0, 8,
           slope};
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
    switch (dtype) {
      case GSVK_F32: launch_lrelu<GSVK_F32>(a, st); break;
      case GSVK_F16: launch_lrelu<GSVK_F16>(a, st); break;
      default: launch_lrelu<GSVK_BF16>(a, st); break;
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
    switch (dtype) {
      case GSVK_F32: launch_res_add<GSVK_F32>(a, st); break;
      case GSVK_F16: launch_res_add<GSVK_F16>(a, st); break;
      default: launch_res_add<GSVK_BF16>(a, st); break;
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
  bool all_t = true, any_t = false;
  for (int j = 0; j < nbranch; ++j) {
    all_t = all_t && a.in[4 + j] != nullptr;
    any_t = any_t || a.in[4 + j] != nullptr;
  }
  if (any_t && !all_t) aligned = false;  // mixed presence: the scalar kernel handles it per branch
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
    switch (dtype) {
      case GSVK_F32: launch_scaled_add<GSVK_F32>(a, st); break;
      case GSVK_F16: launch_scaled_add<GSVK_F16>(a, st); break;
      default: launch_scaled_add<GSVK_BF16>(a, st); break;
    }
  } else {
    launch_scalar_dt(dtype, a, 3, st);
  }
  return launch_status();
}

extern "C" int gsvk_f32_to_f16(const float* x, uint16_t* y, size_t n, void* stream) {
  if (!x || !y) return GSVK_E_NULL;
  if (n == 0 || n > (1ul << 40)) return GSVK_E_SIZE;
  if (overlaps(y, n * 2, x, n * 4)) return GSVK_E_ALIAS;
  if (reinterpret_cast<uintptr_t>(x) % 4 || reinterpret_cast<uintptr_t>(y) % 2) return GSVK_E_ARG;
  const int vec = aligned16(x) && aligned16(y);
  const long blocks = std::min<long>((static_cast<long>(n) / 8 + 255) / 256 + 1, 8192);
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, y, static_cast<long>(n), vec);
  return launch_status();
}
