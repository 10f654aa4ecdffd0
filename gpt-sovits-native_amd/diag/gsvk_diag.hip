// gsvk_diag.hip — measurement kernels for the access patterns the library's kernels are built on.
// Not part of the library's interface: bench.py --diag times them to give the ceilings that the
// streaming kernels are compared with (a copy issued the way a resident-row kernel must issue it,
// and the load forms a weight stream can use), so those comparisons can be re-run from the tree.
//
//   gsvk_diag_copy(form, x, y, rows, row_bytes, stream): y = x, rows of row_bytes bytes, one launch.
//     form 0  one row per 512-thread workgroup; each thread loads all of its 16-byte chunks
//             (t, t + 512, ..., up to 16) before it stores any: the access order of a kernel that
//             must see a whole row before writing it (GroupNorm). Non-temporal loads and stores.
//     form 1  form 0 with ordinary (cached) stores.
//     form 2  one-shot blocks of 256 threads x 8 chunks (32 KiB per workgroup, wave-contiguous):
//             the element-wise streams' order. Non-temporal loads and stores.
//     form 3  form 2 with ordinary stores.
//   gsvk_diag_stream_read(form, w, rows, sink, stream): reads rows of 1 KiB once, in batches of 32
//     rows walked by one 4-wave workgroup per CU (the long-stream GEMV's partition: wave w owns
//     bytes 256 w .. 256 w + 255 of every row of a batch in form 0; whole rows in forms 1-3), and
//     folds what it reads into one word (written to sink only if it hits a fixed value).
//     form 0  the GEMV's fragment loads: lane (r16, grp) reads 16 bytes of row 16 t + r16 at byte
//             256 w + 128 (q / 2) + 32 grp + 16 (q % 2): 16 rows x 64 bytes per instruction;
//             two batches in flight.
//     form 1  contiguous rows into registers: 1 KiB per instruction; two batches in flight.
//     form 2  the same rows straight into LDS (global_load_lds_dwordx4), read back per wave;
//             two batches in flight.
//     form 3  form 2 with four batches in flight (128 KiB of LDS per workgroup).
//     form 4  one-shot blocks of 256 threads x 8 chunks (a plain read).
// Return: 0, -1 (unknown form), -2 (sizes or alignment the form does not take), -3 (HIP error).
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kWave = 64;

template <bool NT>
__device__ __forceinline__ u32x4 ld(const u32x4* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT>
__device__ __forceinline__ void st(u32x4* p, u32x4 v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}
__device__ __forceinline__ uint32_t fold(u32x4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

// ---- copies ------------------------------------------------------------------------------------

constexpr int kRowThreads = 512, kRowChunks = 16;

// rc: 16-byte chunks per row (<= 512 * 16). Chunks past the row load the row's last chunk.
template <bool NS>
__global__ __launch_bounds__(kRowThreads, 4) void copy_row(const u32x4* x, u32x4* y, long rc) {
  const long r = blockIdx.x;
  const int t = threadIdx.x;
  u32x4 v[kRowChunks];
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const long k = t + static_cast<long>(c) * kRowThreads;
    v[c] = ld<true>(x + r * rc + (k < rc ? k : rc - 1));
  }
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const long k = t + static_cast<long>(c) * kRowThreads;
    if (k < rc) st<NS>(y + r * rc + k, v[c]);
  }
}

constexpr int kBlk = 256, kBlkChunks = 8;

// grid * 256 * 8 == total chunks (checked on the host)
template <bool NS>
__global__ __launch_bounds__(kBlk) void copy_block(const u32x4* x, u32x4* y) {
  const long b = static_cast<long>(blockIdx.x) * kBlk * kBlkChunks + threadIdx.x;
  u32x4 v[kBlkChunks];
#pragma unroll
  for (int u = 0; u < kBlkChunks; ++u) v[u] = ld<true>(x + b + u * static_cast<long>(kBlk));
#pragma unroll
  for (int u = 0; u < kBlkChunks; ++u) st<NS>(y + b + u * static_cast<long>(kBlk), v[u]);
}

// ---- weight-stream reads -----------------------------------------------------------------------

constexpr long kRowBytes = 1024, kBatchRows = 32;

__device__ __forceinline__ long batch_of(long j, long nb) {
  const long b = static_cast<long>(blockIdx.x) + static_cast<long>(gridDim.x) * j;
  return b < nb ? b : nb - 1;  // loads past the workgroup's batches re-read the last one
}

// Batches blockIdx.x, + gridDim.x, ...: rounded up to whole rounds of D, the extra ones re-read
// the last batch (in bounds).
template <int D, bool FRAG>
__global__ __launch_bounds__(4 * kWave) void read_regs(const char* w, long nb, uint32_t* sink) {
  const int l = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  const long nbw = (nb - 1 - blockIdx.x) / gridDim.x + 1;
  u32x4 f[D][8];
  auto load = [&](u32x4 (&s)[8], long j) {
    const long b = batch_of(j, nb);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const long off =
          FRAG ? (kBatchRows * b + 16 * (u / 4) + (l & 15)) * kRowBytes + 256 * wv +
                     128 * ((u & 3) >> 1) + 32 * (l >> 4) + 16 * (u & 1)
               : (kBatchRows * b + 8 * wv + u) * kRowBytes + 16 * l;
      s[u] = *reinterpret_cast<const u32x4*>(w + off);
    }
  };
  uint32_t acc = 0;
#pragma unroll
  for (int s = 0; s < D; ++s) load(f[s], s);
  for (long j = 0; j < nbw; j += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += fold(f[s][u]);
      load(f[s], j + s + D);
    }
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

// s_waitcnt with only the vector-memory count set (gfx9 encoding: vmcnt bits 3:0 and 15:14;
// expcnt 6:4 and lgkmcnt 11:8 at their maxima, i.e. not waited for).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
}

// Each wave streams its own 8 rows of a batch into its own LDS slots (8 KiB per slot, D slots),
// waits for the oldest slot (vmcnt counts this wave's loads, issued in order), reads it back,
// then refills it once its reads have returned (lgkmcnt 0). No other wave touches the slot.
template <int D>
__global__ __launch_bounds__(4 * kWave) void read_lds(const char* w, long nb, uint32_t* sink) {
  extern __shared__ u32x4 slots[];  // [4 waves][D][8 rows][64 lanes]
  const int l = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  const long nbw = (nb - 1 - blockIdx.x) / gridDim.x + 1;
  u32x4* mine = slots + static_cast<size_t>(wv) * D * 8 * kWave;
  auto load = [&](int s, long j) {
    const long b = batch_of(j, nb);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      __builtin_amdgcn_global_load_lds(
          static_cast<const void*>(w + (kBatchRows * b + 8 * wv + u) * kRowBytes + 16 * l),
          (lds_void*)(mine + (s * 8 + u) * kWave), 16, 0, 0);
  };
  uint32_t acc = 0;
#pragma unroll
  for (int s = 0; s < D; ++s) load(s, s);
  for (long j = 0; j < nbw; j += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      wait_vmcnt<8 * (D - 1)>();
      __builtin_amdgcn_sched_barrier(0);
      u32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = mine[(s * 8 + u) * kWave + (l ^ u)];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += fold(v[u]);
      wait_lgkmcnt0();
      __builtin_amdgcn_sched_barrier(0);
      load(s, j + s + D);
    }
  }
  wait_vmcnt<0>();  // the refills past the last batch land before the workgroup ends
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

__global__ __launch_bounds__(kBlk) void read_block(const u32x4* x, uint32_t* sink) {
  const long b = static_cast<long>(blockIdx.x) * kBlk * kBlkChunks + threadIdx.x;
  u32x4 v[kBlkChunks];
#pragma unroll
  for (int u = 0; u < kBlkChunks; ++u) v[u] = ld<false>(x + b + u * static_cast<long>(kBlk));
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < kBlkChunks; ++u) acc += fold(v[u]);
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

int cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return n;
}

int status() { return hipGetLastError() == hipSuccess ? 0 : -3; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int gsvk_diag_copy(int form, const void* x, void* y, size_t rows, size_t row_bytes,
                              void* stream) {
  if (form < 0 || form > 3) return -1;
  if (!x || !y || !aligned16(x) || !aligned16(y) || rows == 0 || row_bytes == 0 ||
      row_bytes % 16 || rows > (1u << 30))
    return -2;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const auto* xs = static_cast<const u32x4*>(x);
  auto* ys = static_cast<u32x4*>(y);
  const long rc = static_cast<long>(row_bytes / 16);
  if (form <= 1) {
    if (rc > static_cast<long>(kRowThreads) * kRowChunks) return -2;
    const dim3 grid(static_cast<unsigned>(rows));
    if (form == 0) hipLaunchKernelGGL(copy_row<true>, grid, dim3(kRowThreads), 0, st, xs, ys, rc);
    else hipLaunchKernelGGL(copy_row<false>, grid, dim3(kRowThreads), 0, st, xs, ys, rc);
    return status();
  }
  const size_t chunks = rows * (row_bytes / 16), per = static_cast<size_t>(kBlk) * kBlkChunks;
  if (chunks % per || chunks / per > (1u << 31)) return -2;
  const dim3 grid(static_cast<unsigned>(chunks / per));
  if (form == 2) hipLaunchKernelGGL(copy_block<true>, grid, dim3(kBlk), 0, st, xs, ys);
  else hipLaunchKernelGGL(copy_block<false>, grid, dim3(kBlk), 0, st, xs, ys);
  return status();
}

extern "C" int gsvk_diag_stream_read(int form, const void* w, size_t rows, uint32_t* sink,
                                     void* stream) {
  if (form < 0 || form > 4) return -1;
  if (!w || !sink || !aligned16(w) || rows == 0 || rows % kBatchRows || rows > (1u << 26)) return -2;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const char* wb = static_cast<const char*>(w);
  const long nb = static_cast<long>(rows / kBatchRows);
  const int n = cus();
  if (n <= 0) return -3;
  const dim3 grid(static_cast<unsigned>(nb < n ? nb : n)), block(4 * kWave);
  switch (form) {
    case 0: hipLaunchKernelGGL((read_regs<2, true>), grid, block, 0, st, wb, nb, sink); break;
    case 1: hipLaunchKernelGGL((read_regs<2, false>), grid, block, 0, st, wb, nb, sink); break;
    case 2: {
      constexpr size_t lds = 4 * 2 * 8 * kWave * 16;
      hipLaunchKernelGGL((read_lds<2>), grid, block, lds, st, wb, nb, sink);
      break;
    }
    case 3: {
      constexpr size_t lds = 4 * 4 * 8 * kWave * 16;  // 128 KiB: above the default 64 KiB limit
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(&read_lds<4>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) !=
          hipSuccess)
        return -3;
      hipLaunchKernelGGL((read_lds<4>), grid, block, lds, st, wb, nb, sink);
      break;
    }
    default: {
      const size_t chunks = rows * (kRowBytes / 16), per = static_cast<size_t>(kBlk) * kBlkChunks;
      if (chunks % per) return -2;
      hipLaunchKernelGGL(read_block, dim3(static_cast<unsigned>(chunks / per)), dim3(kBlk), 0, st,
                         reinterpret_cast<const u32x4*>(wb), sink);
    }
  }
  return status();
}
