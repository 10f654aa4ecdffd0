// gsvk_common.hpp — storage traits, 128-bit row access and wave64 reductions shared by the gfx950
// kernels. Everything here is device code for CDNA4 (wave64); nothing is portable on purpose.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>

#include "gsvk.h"

namespace gsvk {

constexpr int kWave = 64;

// ---- scalar conversions (exact upcast, round-to-nearest-even downcast) -------------------------

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}
__device__ __forceinline__ uint32_t f2h(float v) {
  // The value must be rounded to fp32 first and then to fp16 (the reference computes in fp32 and
  // the fp16 store rounds that result). Without the empty asm below, the compiler folds a
  // producing fmaf into v_fma_mixlo_f16, which rounds the exact result to fp16 once and differs
  // in the last bit for some inputs; the asm makes v an opaque fp32 register value.
  __asm__("" : "+v"(v));
  // v_cvt_f16_f32: round to nearest even (checked on MI355X against numpy on every half-subnormal
  // midpoint, its neighbours and 200k random values), overflow to inf, NaN kept.
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two values to one packed word (lo = a, hi = b) with one v_cvt_pk_f16_f32: round to nearest
// even, the same results as f2h (checked the same way). The asm keeps fmaf + downcast unfused.
__device__ __forceinline__ uint32_t f2h2(float a, float b) {
  __asm__("" : "+v"(a), "+v"(b));
  const f32x2 p = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(p, f16x2));
}
__device__ __forceinline__ float bf2f(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}
__device__ __forceinline__ uint32_t f2bf(float v) {
  // Round to nearest even on the top 16 bits; every NaN becomes the canonical quiet NaN 0x7FC0.
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// ---- storage traits: one 16-byte chunk = VEC elements ----------------------------------------

template <int DT>
struct Store;

// 16-byte global access. NT = true marks the access non-temporal (the line is not kept in the caches
// after use): streaming kernels read and write each byte once, so caching it only evicts data that
// other waves still need.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ u32x4 ld16(const void* p) {
  const u32x4* q = static_cast<const u32x4*>(p);
  if constexpr (NT) return __builtin_nontemporal_load(q);
  else return *q;
}
template <bool NT>
__device__ __forceinline__ void st16(void* p, u32x4 v) {
  u32x4* q = static_cast<u32x4*>(p);
  if constexpr (NT) __builtin_nontemporal_store(v, q);
  else *q = v;
}

template <>
struct Store<GSVK_F32> {
  using T = float;
  static constexpr int VEC = 4;
  __device__ static __forceinline__ void unpack(const u32x4& q, float (&v)[VEC]) {
    // Copy the lanes out first: __builtin_bit_cast applied directly to an ext_vector element
    // (q.y) was compiled by this clang as a cast of element 0.
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = __builtin_bit_cast(float, w[k]);
  }
  __device__ static __forceinline__ u32x4 pack(const float (&v)[VEC]) {
    u32x4 q;
    q.x = __builtin_bit_cast(uint32_t, v[0]);
    q.y = __builtin_bit_cast(uint32_t, v[1]);
    q.z = __builtin_bit_cast(uint32_t, v[2]);
    q.w = __builtin_bit_cast(uint32_t, v[3]);
    return q;
  }
  template <bool NT = false>
  __device__ static __forceinline__ void load(const void* base, size_t i, float (&v)[VEC]) {
    unpack(ld16<NT>(static_cast<const float*>(base) + i), v);
  }
  template <bool NT = false>
  __device__ static __forceinline__ void store(void* base, size_t i, const float (&v)[VEC]) {
    st16<NT>(static_cast<float*>(base) + i, pack(v));
  }
  __device__ static __forceinline__ float load1(const void* base, size_t i) {
    return static_cast<const float*>(base)[i];
  }
  __device__ static __forceinline__ void store1(void* base, size_t i, float v) {
    static_cast<float*>(base)[i] = v;
  }
};

template <int DT>
struct Store16 {  // f16 and bf16 share the 16-bit packing
  static constexpr int VEC = 8;
  __device__ static __forceinline__ float up(uint32_t b) { return DT == GSVK_F16 ? h2f(b) : bf2f(b); }
  __device__ static __forceinline__ uint32_t down(float v) { return DT == GSVK_F16 ? f2h(v) : f2bf(v); }
  __device__ static __forceinline__ void unpack(const u32x4& q, float (&v)[VEC]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = up(w[k] & 0xffffu);
      v[2 * k + 1] = up(w[k] >> 16);
    }
  }
  __device__ static __forceinline__ u32x4 pack(const float (&v)[VEC]) {
    u32x4 q;
    if constexpr (DT == GSVK_F16) {
      q.x = f2h2(v[0], v[1]);
      q.y = f2h2(v[2], v[3]);
      q.z = f2h2(v[4], v[5]);
      q.w = f2h2(v[6], v[7]);
    } else {
      q.x = down(v[0]) | (down(v[1]) << 16);
      q.y = down(v[2]) | (down(v[3]) << 16);
      q.z = down(v[4]) | (down(v[5]) << 16);
      q.w = down(v[6]) | (down(v[7]) << 16);
    }
    return q;
  }
  template <bool NT = false>
  __device__ static __forceinline__ void load(const void* base, size_t i, float (&v)[VEC]) {
    unpack(ld16<NT>(static_cast<const uint16_t*>(base) + i), v);
  }
  template <bool NT = false>
  __device__ static __forceinline__ void store(void* base, size_t i, const float (&v)[VEC]) {
    st16<NT>(static_cast<uint16_t*>(base) + i, pack(v));
  }
  __device__ static __forceinline__ float load1(const void* base, size_t i) {
    return up(static_cast<const uint16_t*>(base)[i]);
  }
  __device__ static __forceinline__ void store1(void* base, size_t i, float v) {
    static_cast<uint16_t*>(base)[i] = static_cast<uint16_t>(down(v));
  }
};
template <>
struct Store<GSVK_F16> : Store16<GSVK_F16> {};
template <>
struct Store<GSVK_BF16> : Store16<GSVK_BF16> {};

// Loads stay outside branches. A load under `if (in_bounds)` or `if (ptr)` ends a basic block, and
// the compiler then waits for it (s_waitcnt vmcnt(0)) before the next load is issued: a thread
// keeps one request in flight instead of all of them. So out-of-range indices are clamped to a
// valid element (the value is discarded) and only stores are guarded, and an absent parameter
// vector reads one of these constant rows instead of being skipped.
static __device__ __attribute__((aligned(16))) float kZeros8[8] = {0.f, 0.f, 0.f, 0.f,
                                                                    0.f, 0.f, 0.f, 0.f};
static __device__ __attribute__((aligned(16))) float kOnes8[8] = {1.f, 1.f, 1.f, 1.f,
                                                                   1.f, 1.f, 1.f, 1.f};
// An absent addend that must leave every value as it is: x + (-0) == x for all x, -0 included
// (x + 0 turns -0 into +0).
static __device__ __attribute__((aligned(16))) float kNegZeros8[8] = {-0.f, -0.f, -0.f, -0.f,
                                                                       -0.f, -0.f, -0.f, -0.f};

// Address of the 8-float parameter chunk starting at element i, or of a constant row when the
// vector is absent.
__device__ __forceinline__ const float* param_or(const float* p, size_t i, const float* fill) {
  return p ? p + i : fill;
}

// fp32 parameter vectors (gamma / beta / bias): 4 floats per 16 bytes.
__device__ __forceinline__ void load_f32x4(const float* p, size_t i, float* v) {
  const float4 q = *reinterpret_cast<const float4*>(p + i);
  v[0] = q.x;
  v[1] = q.y;
  v[2] = q.z;
  v[3] = q.w;
}

// ---- GELU(erf) ------------------------------------------------------------------------------------
// gelu(x) = 0.5 x (1 + erf(x / sqrt2)), the reference's bert::gelu_erf / HubertEngine::gelu
// (bert_ops.hpp:25-27, hubert.cpp:233-236). With e = erfc(|x| / sqrt2) one branch-free form holds
// for both signs: gelu(x) = 0.5 (x + |x| (1 - e)) (x >= 0: x - 0.5 x e; x < 0: 0.5 x e).
// erfc(z) = t (a1 + a2 t + a3 t^2 + a4 t^3 + a5 t^4) exp(-z^2), t = 1 / (1 + p z): Abramowitz &
// Stegun, Handbook of Mathematical Functions, formula 7.1.26, absolute error below 1.5e-7 for every
// z >= 0. The rounding of 1 - e adds at most |x| 2^-25 absolute. Both stay below the fp32 tolerance
// of this path (1e-6 + 1e-5 |gelu|) over the whole range; past |x| ~ 13 e underflows to 0 and the
// result is exactly x (x > 0) or -0 (x < 0). The result takes the sign of x: the reference's
// product 0.5f * x * (1 + erf) is -0 wherever it is zero for a negative x (x = -0, and every x
// whose erff rounds to -1), and the sum above would give +0 there. +inf gives inf, -inf and NaN
// give NaN, like the reference. 13 VALU operations plus two transcendentals (v_rcp_f32,
// v_exp_f32) per element.
__device__ __forceinline__ float gelu_erf(float x) {
  const float ax = __builtin_fabsf(x);
  const float zz = ax * 0.84932180028801904f;  // |x| sqrt(log2(e) / 2): exp(-x^2/2) = 2^-(zz^2)
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.23164189925183054f, ax, 1.f));
  float p = 1.061405429f;
  p = __builtin_fmaf(p, t, -1.453152027f);
  p = __builtin_fmaf(p, t, 1.421413741f);
  p = __builtin_fmaf(p, t, -0.284496736f);
  p = __builtin_fmaf(p, t, 0.254829592f);
  const float e = (p * t) * __builtin_amdgcn_exp2f(-(zz * zz));
  return __builtin_copysignf(0.5f * __builtin_fmaf(ax, 1.f - e, x), x);
}

// ---- streaming threshold ---------------------------------------------------------------------------
// A call that moves at least this many bytes streams its operands non-temporally: its working set
// exceeds the 256 MB MALL, so caching its lines only evicts what other kernels still use. Smaller
// calls keep normal cached access (their operands are often still in L2 / MALL from the producing
// kernel, and their outputs are read next).
constexpr size_t kStreamBytes = size_t(256) << 20;

// ---- wave64 reductions -------------------------------------------------------------------------
// Inside each 16-lane DPP row: quad_perm xor-1, quad_perm xor-2, row_half_mirror, row_mirror give
// every lane its row's sum r_k (bitwise the same on all 16 lanes: each step adds a pair in either
// order). Then row_bcast:15 adds row k's lane 15 into row k + 1 (rows 1 and 3 only) and
// row_bcast:31 adds lane 31 into rows 2 and 3, so lane 63 holds (r3 + r2) + (r1 + r0), read once
// with v_readlane. The result is wave-uniform; the two broadcasts replace an LDS swizzle and a
// second readlane on the critical path of every row reduction (the sum is the same bits as
// (r0 + r1) + (r2 + r3): fp32 addition is commutative).
// (v_permlane16/32_swap would keep the sum in VGPRs, but this compiler folds the two results of
// a swap whose operands are the same value into one: it emitted s.x + s.x for s.x + s.y.)

// Whole-row DPP move with bound_ctrl set: every lane has its source lane for these controls, so
// the values are the plain move's, and the compiler can fold the move into the add that follows
// (v_add_f32_dpp: one instruction per reduction step instead of two).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
// DPP move restricted to ROW_MASK rows; the other rows get 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_rows_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xf, false));
}

// Workgroup barrier that orders LDS only (__syncthreads() would also wait for the thread's
// outstanding global stores and loads).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The two cross-row steps: rows 1 and 3 add lane 15 of the row before (row_bcast:15), then rows 2
// and 3 add lane 31 (row_bcast:31), each as one v_add_f32_dpp whose other rows keep v (where
// v + dpp_rows_f32 computes v + 0: the same value up to the sign of a zero, in rows that are never
// read). Written as dpp_rows_f32 + add, each step is three instructions: the move with a zero old
// value is not folded into the add when the row mask is partial. The compiler does not see inside
// the asm, so it carries the wait states DPP needs after a VALU write of its source: two before
// each DPP read, two after for the v_readlane of the result.
__device__ __forceinline__ float add_row_bcasts(float v) {
  asm volatile(
      "s_nop 1\n\t"
      "v_add_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_add_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
      "s_nop 1"
      : "+v"(v));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  v = add_row_bcasts(v);   // rows 1, 3 then 2, 3: lane 63 holds (r3 + r2) + (r1 + r0)
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// add_row_bcasts for two independent values, the steps of one interleaved with the other's (each
// DPP read is then two or more wait states after the VALU write of its source).
__device__ __forceinline__ void add_row_bcasts2(float& a, float& b) {
  asm volatile(
      "s_nop 1\n\t"
      "v_add_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
      "v_add_f32_dpp %1, %1, %1 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_add_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
      "v_add_f32_dpp %1, %1, %1 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
      "s_nop 1"
      : "+v"(a), "+v"(b));
}

// Two wave sums at once (each the same bits as wave_sum of that value): the two dependent chains
// interleave, so the pair costs about one chain's latency.
__device__ __forceinline__ void wave_sum2(float a, float b, float& ra, float& rb) {
  a += dpp_f32<0xB1>(a);
  b += dpp_f32<0xB1>(b);
  a += dpp_f32<0x4E>(a);
  b += dpp_f32<0x4E>(b);
  a += dpp_f32<0x141>(a);
  b += dpp_f32<0x141>(b);
  a += dpp_f32<0x140>(a);
  b += dpp_f32<0x140>(b);
  add_row_bcasts2(a, b);
  ra = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 63));
  rb = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, b), 63));
}

// Per-lane partial sums of one 16-byte chunk (4 or 8 values) as a balanced tree: depth 2-3
// instead of a 3-7 long dependent chain (each dependent VALU step costs ~11 cycles on MI355X, and
// the LayerNorm reductions sit on the critical path of latency-bound calls).
template <int V>
__device__ __forceinline__ float chunk_sum(const float (&v)[V]) {
  static_assert(V == 4 || V == 8, "chunk of 4 or 8 values");
  if constexpr (V == 4) return (v[0] + v[1]) + (v[2] + v[3]);
  else return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}
// Sum of v^2 over one chunk: pairs fma(v1, v1, v0 * v0), then a tree of the pairs.
template <int V>
__device__ __forceinline__ float chunk_sq(const float (&v)[V]) {
  float q[V / 2];
#pragma unroll
  for (int k = 0; k < V / 2; ++k) q[k] = __builtin_fmaf(v[2 * k + 1], v[2 * k + 1], v[2 * k] * v[2 * k]);
  if constexpr (V == 4) return q[0] + q[1];
  else return (q[0] + q[1]) + (q[2] + q[3]);
}
// Sum of (v - mean)^2 over one chunk: pairs fma(d1, d1, d0 * d0), then a tree of the pairs.
template <int V>
__device__ __forceinline__ float chunk_sumsq(const float (&v)[V], float mean) {
  float q[V / 2];
#pragma unroll
  for (int k = 0; k < V / 2; ++k) {
    const float d0 = v[2 * k] - mean, d1 = v[2 * k + 1] - mean;
    q[k] = __builtin_fmaf(d1, d1, d0 * d0);
  }
  if constexpr (V == 4) return q[0] + q[1];
  else return (q[0] + q[1]) + (q[2] + q[3]);
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// ---- activations (reference semantics) -----------------------------------------------------------

// vmaxq_f32(x, 0): a NaN input comes out as that NaN made quiet, -0 -> +0 (kern.cpp:85-91,
// vector body).
__device__ __forceinline__ float relu_ref(float v) {
  if (v != v) return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) | 0x00400000u);
  return v > 0.f ? v : 0.f;
}
// v < 0 ? v * slope : v — keeps -0 and NaN (nn_ops.hpp:48-74).
__device__ __forceinline__ float lrelu_ref(float v, float slope) { return v < 0.f ? v * slope : v; }

template <int ACT>
__device__ __forceinline__ float act_apply(float v, float slope) {
  if constexpr (ACT == GSVK_ACT_RELU) return relu_ref(v);
  else if constexpr (ACT == GSVK_ACT_GELU_ERF) return gelu_erf(v);
  else if constexpr (ACT == GSVK_ACT_LEAKY_RELU) return lrelu_ref(v, slope);
  else return v;
}

// ---- host-side helpers shared by the launchers ------------------------------------------------

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline size_t dtype_size(int dt) { return dt == GSVK_F32 ? 4 : 2; }

inline bool valid_dtype(int dt) { return dt == GSVK_F32 || dt == GSVK_F16 || dt == GSVK_BF16; }

// True when [a, a+abytes) and [b, b+bbytes) intersect.
inline bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
  if (!a || !b || !abytes || !bbytes) return false;
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
  return a0 < b0 + bbytes && b0 < a0 + abytes;
}

// Bytes spanned by a [rows, n] view with row stride ld.
inline size_t span_bytes(size_t rows, size_t n, size_t ld, size_t esz) {
  return rows ? ((rows - 1) * ld + n) * esz : 0;
}

int launch_status();  // GSVK_OK, or GSVK_E_HIP after a failed launch (reads hipGetLastError)

constexpr int kMaxDevices = 64;

// Allow `bytes` of dynamic LDS (above the 64 KiB default) for kernel `fn` on the current device:
// once per kernel and device, `done` being that kernel's flags (setting it twice from racing first
// calls is harmless). False when the device cannot be queried or the runtime refuses.
inline bool allow_dynamic_lds(const void* fn, size_t bytes,
                              std::atomic<bool> (&done)[kMaxDevices]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  if (done[dev].load(std::memory_order_acquire)) return true;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(bytes)) != hipSuccess)
    return false;
  done[dev].store(true, std::memory_order_release);
  return true;
}

// Compute units of the current device (cached per device; 256 on MI355X). A racing first call
// stores the same value twice.
inline int device_cus() {
  static std::atomic<int> cus[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace gsvk
