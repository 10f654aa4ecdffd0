// gsvk_conv.hip — SoVITS Conv1d (same padding, dilation) on the gfx950 matrix cores, with the
// ResBlock element-wise passes that follow a convolution fused into its store.
//
// y[o, t] = bias[o] + sum_{i, kk} w[o, i, kk] x[i, t + kk dil - pad], pad = (k - 1) dil / 2, zero
// outside [0, T) (Conv1d::forward, conv1d.hpp:109-194: im2col col[(i k + kk), t] then
// y = W[o, i k] col, then add_bias). Channel-major activations [C, T] with rows of stride ld, fp16 weights.
//
// Implicit GEMM: M = T, N = C_out, K = C_in x k, never materialised. One MFMA
// v_mfma_f32_16x16x32_f16 multiplies a 16 t x 32 channel slice of X^T (operand A) by a 32 channel
// x 16 o slice of W^T for one tap (operand B); lane l feeds row / column (l & 15) with 8 channels
// chosen by its lane group (l >> 4), and the accumulator holds, in lane l, four consecutive t
// 4 (l >> 4) .. +3 of output row o = (l & 15): one 16-byte store per fragment.
//
// Workgroup: 4 waves side by side along t, NT fragments (16 NT t) each, all on the same 16 NO
// output rows. Input channels go in chunks of 32. A chunk of x, with the halo of (k - 1) dil
// columns the taps reach past the tile, is staged once in LDS and read k times, once per tap at
// shift kk dil: layout [plane][channel group g = 0..3][t][8 channels], so a fragment read is 16
// consecutive 16-byte rows (no bank conflicts) and the tap shift is a row offset. The weights are
// packed once (gsvk_conv1d_pack) as [chunk][tap][channel group][o][8 channels] and staged through
// LDS in groups of kTapGroup taps of a chunk, laid out like x (a B fragment read is 16 consecutive
// 16-byte rows); each group's weights are loaded into registers while the group before it
// multiplies, and the next chunk of x while the current chunk's first group does.
//
// x in fp32: round_x = 1 rounds it to fp16 (the reference's AMX packing, im2col_to_panel_f16);
// round_x = 0 keeps fp32 (the reference's default sgemm path) by multiplying hi = f16(x) and
// lo = f16(x - hi) separately: hi + lo equals x to about 2^-22 relative (|x| < 65504), and the
// products with fp16 weights are exact in fp32. Sums are fp32 in the matrix cores' order.
#include <algorithm>
#include <type_traits>

#include "gsvk_common.hpp"

namespace gsvk {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

enum XMode { kXF16 = 0, kXRound = 1, kXSplit = 2 };

constexpr int kChunk = 32;  // input channels per LDS chunk: one MFMA k depth
constexpr int kOPad = 64;   // packed output rows: a multiple of the largest wave tile
constexpr int kWaves = 4;   // waves per workgroup, side by side along t
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxHalo = 256;
#ifndef GSVK_CONV_TAP_GROUP
#define GSVK_CONV_TAP_GROUP 4
#endif
constexpr int kTapGroup = GSVK_CONV_TAP_GROUP;  // taps whose weights share one LDS refill

struct ConvArgs {
  const void* x;
  const uint16_t* wp;
  const float* bias;
  void* cur;
  const void* res;  // residual source of epi 2 / 3 (row stride ldc); nullptr: cur itself
  void* y;
  long cin, cout, T, ldx, ldc, ldy;  // T: input columns
  int k, dil, pad, nch, opad;
  int epi;
  float slope;
  bool vec;
  bool xact;  // x read as lrelu(x, slope)
  int up;     // 0: Conv1d; u: transposed convolution with stride u (phase r = blockIdx.z)
  long Tout;  // transposed: output columns T u
  int pad_t;  // transposed: (k - u) / 2
  long xspan;  // time tiles per XCD (the grid's x extent / kXcds), 0: x index = time tile
};

// Workgroups are dispatched to the 8 XCDs of the chip round-robin by linear id, and each XCD has
// its own L2. The grid's x extent is padded to a multiple of kXcds and x index b computes time
// tile (b % kXcds) xspan + b / kXcds: each XCD walks a contiguous range of tiles in order, so a
// tile's halo columns were just read into the same L2 by its neighbour, and the output-row blocks
// of one tile (grid y) land on the same XCD and share its x columns there. Grids of fewer than
// kXcdMinTiles time tiles keep the identity order: there, whole XCDs would sit idle (20 tiles of
// the 384-channel decoder stage: 1% slower remapped).
constexpr int kXcds = 8;
constexpr long kXcdMinTiles = 64;

// What one workgroup computes. Conv1d: output column t reads x columns t - pad + kk dil over the
// k taps. Transposed convolution, phase r (ConvT1d, conv1d.hpp:250-340; y[j u + d - pad_t] +=
// W[:, :, d] x[:, j]): the outputs t_out = q u + r - pad_t take the taps d = r + m u < k with
// x column q - m, i.e. kn = ceil((k - r) / u) taps in reverse order (packed so, slot kk = kn - 1 -
// m) over x columns q - (kn - 1) + kk. Position t of the phase is q = qlo + t, written to column
// obase + t ostr.
struct Map {
  int kn;       // taps
  long nq;      // output positions
  long xoff;    // x column of position 0, tap 0
  long ostr;    // output column stride
  long obase;   // output column of position 0
  const uint16_t* wp;
};

__device__ __forceinline__ long ceil_div(long a, long b) { return a >= 0 ? (a + b - 1) / b : -((-a) / b); }
__device__ __forceinline__ long floor_div(long a, long b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }

__device__ __forceinline__ Map block_map(const ConvArgs& a) {
  Map m;
  if (!a.up) {
    m.kn = a.k, m.nq = a.T, m.xoff = -a.pad, m.ostr = 1, m.obase = 0, m.wp = a.wp;
    return m;
  }
  const int u = a.up, r = blockIdx.z;
  m.kn = (a.k - r + u - 1) / u;
  size_t taps_before = 0;
  for (int r2 = 0; r2 < r; ++r2) taps_before += static_cast<size_t>((a.k - r2 + u - 1) / u);
  m.wp = a.wp + taps_before * a.nch * a.opad * kChunk;
  const long qlo = ceil_div(a.pad_t - r, u), qhi = floor_div(a.Tout - 1 + a.pad_t - r, u);
  m.nq = qhi - qlo + 1;
  m.xoff = qlo - (m.kn - 1);
  m.ostr = u;
  m.obase = qlo * u + r - a.pad_t;
  return m;
}

template <int XM>
constexpr int planes() { return XM == kXSplit ? 2 : 1; }

// The staging conversions below cost a few VALU instructions per staged value, and they sit
// between a workgroup's barriers, on the path of every chunk.
//
// lrelu(v, s) for 0 < s <= 1 as max(v, v s): the same bits as lrelu_ref (v < 0: v s > v; v >= 0:
// v s <= v; -0 and +-inf give themselves; NaN stays NaN). One v_max_f32: fmaxf would first quiet
// each operand with an instruction of its own.
__device__ __forceinline__ float lrelu_max(float v, float s) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(v), "v"(v * s));
  return r;
}

// Two values to one packed fp16 word (RNE), v_cvt_pk_f16_f32.
__device__ __forceinline__ uint32_t pack_h2(float v0, float v1) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  const f2v p = {v0, v1};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(p, h2v));
}

// The remainders of the hi / lo split of two values, hi = pack_h2(v0, v1): f16(v0 - hi.lo) |
// f16(v1 - hi.hi) << 16. Each is one v_fma_mix (the half converted, multiplied by m1 = -1, added
// to v and the sum rounded to f16): v - hi is exact in fp32, so that is the value of a separate
// conversion, subtraction and rounding. m1 is -1 held where the compiler cannot see it (a
// constant -1 would turn the fma into a subtraction, which is not matched to v_fma_mix). An
// infinite v leaves inf - inf = NaN there, which the packed max with -65504 (maxNum: the non-NaN
// operand) turns into -65504: hi w + lo w is then still inf w (NaN for w = 0), as with a zero
// remainder. Finite remainders are far inside +-65504.
__device__ __forceinline__ uint32_t split_rest2(uint32_t hi, float v0, float v1, float m1) {
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  const h2v h = __builtin_bit_cast(h2v, hi);
  const h2v r = {static_cast<_Float16>(__builtin_fmaf(static_cast<float>(h[0]), m1, v0)),
                 static_cast<_Float16>(__builtin_fmaf(static_cast<float>(h[1]), m1, v1))};
  const h2v lim = {static_cast<_Float16>(-65504.f), static_cast<_Float16>(-65504.f)};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(r, lim));
}

template <int XM>
constexpr int storage_dt() { return XM == kXF16 ? GSVK_F16 : GSVK_F32; }

// Packed weights, step s = c k + kk (chunk c, tap kk), channel group g = 0..3 of the chunk:
// wp[((s 4 + g) opad + o) 8 + j] = w[o, 32 c + 8 g + j, kk], zero past C_out / C_in. One step's
// group g is opad contiguous 16-byte rows, the layout of the B fragments in LDS.
__device__ __forceinline__ void unpack_index(long e, long opad, long& s, long& g, long& o, long& j) {
  j = e % 8;
  o = (e / 8) % opad;
  g = (e / (8 * opad)) % 4;
  s = e / (kChunk * opad);
}

__global__ __launch_bounds__(256) void conv_pack(const uint16_t* __restrict__ w,
                                                 uint16_t* __restrict__ wp, long cout, long cin,
                                                 long k, long opad, long total) {
  for (long e = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<long>(gridDim.x) * blockDim.x) {
    long s, g, o, j;
    unpack_index(e, opad, s, g, o, j);
    const long c = s / k, kk = s % k, i = c * kChunk + 8 * g + j;
    wp[e] = (o < cout && i < cin) ? w[(o * cin + i) * k + kk] : uint16_t(0);
  }
}

// Transposed weights, torch layout w[i, o, d] (ConvT1d::load, conv1d.hpp:219-237), packed per
// phase r = 0 .. u-1 one after another, each like conv_pack with kn_r = ceil((k - r) / u) taps:
// slot kk holds tap d = r + (kn_r - 1 - kk) u.
__global__ __launch_bounds__(256) void convt_pack(const uint16_t* __restrict__ w,
                                                  uint16_t* __restrict__ wp, long cout, long cin,
                                                  long k, long u, long nch, long opad, long total) {
  for (long e = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<long>(gridDim.x) * blockDim.x) {
    long rest = e, r = 0, kn = (k + u - 1) / u;
    while (rest >= nch * kn * opad * kChunk) {  // at most u - 1 steps
      rest -= nch * kn * opad * kChunk;
      ++r;
      kn = (k - r + u - 1) / u;
    }
    long s, g, o, j;
    unpack_index(rest, opad, s, g, o, j);
    const long c = s / kn, kk = s % kn, i = c * kChunk + 8 * g + j, d = r + (kn - 1 - kk) * u;
    wp[e] = (o < cout && i < cin) ? w[(i * cout + o) * k + d] : uint16_t(0);
  }
}

template <int DT>
__device__ __forceinline__ float ld1(const void* p, size_t i) { return Store<DT>::load1(p, i); }

// cur[o, t .. t+3] for the residual epilogues (positions t .. t+3 of the map), read before any
// result is stored so that all fragments' loads are in flight together: one vector load for a whole
// group of contiguous, aligned columns, otherwise element loads at clamped positions (values past
// the end are not used).
template <int DT>
__device__ __forceinline__ f4v load_cur(const ConvArgs& a, const Map& m, long o, long t) {
  const size_t row = static_cast<size_t>(min(o, a.cout - 1)) * a.ldc + m.obase;
  const void* src = a.res ? a.res : a.cur;
  f4v c;
  if (a.vec && m.ostr == 1 && t + 4 <= m.nq) {
    if constexpr (DT == GSVK_F32) {
      c = *reinterpret_cast<const f4v*>(static_cast<const float*>(src) + row + t);
    } else {
      const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(src) + row + t);
      c = f4v{h2f(q.x & 0xffffu), h2f(q.x >> 16), h2f(q.y & 0xffffu), h2f(q.y >> 16)};
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) c[q] = ld1<DT>(src, row + min(t + q, m.nq - 1) * m.ostr);
  }
  return c;
}

template <int DT>
__device__ __forceinline__ void store4(void* base, size_t off, long stride, const float (&v)[4],
                                       bool full, long valid) {
  if (full) {
    if constexpr (DT == GSVK_F32)
      *reinterpret_cast<float4*>(static_cast<float*>(base) + off) = float4{v[0], v[1], v[2], v[3]};
    else
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + off) =
          uint2{f2h2(v[0], v[1]), f2h2(v[2], v[3])};
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (q < valid) Store<DT>::store1(base, off + q * stride, v[q]);
  }
}

// Positions t .. t+3 of row o: bias, epilogue, stores. Vector stores when the four columns are
// contiguous, inside the output and aligned.
template <int DT>
__device__ __forceinline__ void finish4(const ConvArgs& a, const Map& m, long o, long t, f4v s,
                                        float b, f4v cur) {
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = a.bias ? s[q] + b : s[q];
  const size_t yo = static_cast<size_t>(o) * a.ldy + m.obase + t * m.ostr;
  const size_t co = static_cast<size_t>(o) * a.ldc + m.obase + t * m.ostr;
  const bool full = a.vec && m.ostr == 1 && t + 4 <= m.nq;
  const long valid = m.nq - t;
  switch (a.epi) {
    case GSVK_CONV_EPI_RES_LRELU:
    case GSVK_CONV_EPI_RES: {  // cur = res + conv (+ b); RES_LRELU also writes y = lrelu(cur)
      float c[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) c[q] = cur[q] + v[q];
      store4<DT>(a.cur, co, m.ostr, c, full, valid);
      if (a.epi == GSVK_CONV_EPI_RES) return;
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = lrelu_ref(c[q], a.slope);
      break;
    }
    case GSVK_CONV_EPI_DUAL: {  // y = conv (+ b) and cur = lrelu(y)
      float l[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) l[q] = lrelu_ref(v[q], a.slope);
      store4<DT>(a.cur, co, m.ostr, l, full, valid);
      break;
    }
    case GSVK_CONV_EPI_LRELU:
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = lrelu_ref(v[q], a.slope);
      break;
    case GSVK_CONV_EPI_TANH:
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = tanhf(v[q]);
      break;
    default:
      break;
  }
  store4<DT>(a.y, yo, m.ostr, v, full, valid);
}

// Fragment shapes. FS = 16: v_mfma_f32_16x16x32_f16, one 32-channel step per MFMA (above). FS =
// 32: v_mfma_f32_32x32x16_f16 on 32 t x 32 o fragments, two 16-channel halves h of the chunk per
// step: operand A is a 32 t x 16 channel slice of X^T (lane l: position l & 31, the 8 channels of
// group 2 h + (l >> 5)), operand B a 16 channel x 32 o slice of W^T (lane l: output row l & 31),
// and the accumulator holds in lane l output row (l & 31) at positions 8 q + 4 (l >> 5) .. +3,
// q = 0..3: four runs of four consecutive positions, one 16-byte store each. A wave tile of
// 64 t x 64 o in 32-wide fragments reads a quarter fewer LDS bytes per multiply than 32 t x 64 o in
// 16-wide ones, and each refill of LDS (x per chunk, weights per tap group) feeds twice the
// matrix-core work of a workgroup.
//
// At least two waves per SIMD: the register budget is sized for them (the compiler would
// otherwise keep two steps' fragments live); at two, every tile fits without spilling. The
// fp16-storage 32-wide tiles take three (168 VGPRs, a few spilled): with the decoder's ResBlocks
// sharing the chip, its fp16-storage graph measured 4% faster; the exact split's tiles were slower
// so.
template <int XM>
constexpr int conv_waves_per_eu(int fs) { return XM == kXF16 && fs == 32 ? 3 : 2; }
template <int XM, int NT, int NO, int HMAX, int FS>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(conv_waves_per_eu<XM>(FS)))) void conv1d_mfma(ConvArgs a) {
  constexpr int DT = storage_dt<XM>();
  constexpr int P = planes<XM>();
  constexpr int TT = kWaves * FS * NT;  // output columns of the workgroup
  constexpr int TTH = TT + HMAX;        // staged columns (tile + halo)
  // HMAX 16: the tile's columns in whole-wave blocks and the halo in one slab of 16 columns (two
  // loads per lane); otherwise every staged column in whole-wave blocks.
  constexpr bool kSlab = HMAX == 16;
  constexpr int NI = (kSlab ? TT : TTH) / kWave;  // whole-wave column blocks per lane
  extern __shared__ __attribute__((aligned(16))) _Float16 xs[];  // [P][4][TTH][8]
  static_assert(FS == 16 || FS == 32, "fragment size");

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int r16 = lane & 15, grp = lane >> 4;
  const int r32 = lane & 31, hl = lane >> 5;
  const long t0 =
      (a.xspan ? static_cast<long>(blockIdx.x % kXcds) * a.xspan + blockIdx.x / kXcds
               : static_cast<long>(blockIdx.x)) *
      TT;
  const long o0 = static_cast<long>(blockIdx.y) * (FS * NO);
  const Map m = block_map(a);
  if (t0 >= m.nq) return;  // a phase with fewer positions than the grid covers (whole workgroup)

  // ---- x chunk: global -> registers -> LDS ------------------------------------------------------
  // Wave g stages channel group g (channels 8 g .. 8 g + 7 of the chunk) over all TTH columns:
  // lane l holds column tp = l + 64 u (x column t0 + xoff + tp, clamped into [0, T)). The row
  // is wave-uniform, so each load is a buffer load with the column as its 32-bit offset and the
  // row, clamped to the chunk's last row, as a scalar offset: every load reads inside x. Clamped
  // values are zeroed when staged (a zero pad, and no 0 * inf from channels past C_in).
  // The slab (HMAX 16): lane l holds halo column TT + (l & 15) of channels j = 2 (l >> 4) and
  // j + 1 (one load each; 16 lanes read 16 consecutive columns of one row), so a halo of up to 16
  // columns costs two loads and two values per lane instead of a whole-wave block of 64 columns.
  static_assert(kSlab ? TT % kWave == 0 : TTH % kWave == 0, "staged columns: whole waves");
  constexpr int ESZ = DT == GSVK_F32 ? 4 : 2;
  const int g = __builtin_amdgcn_readfirstlane(wave);
  const int row_bytes = static_cast<int>(a.ldx) * ESZ;
  int tcol[NI];
#pragma unroll
  for (int u = 0; u < NI; ++u)
    tcol[u] = static_cast<int>(min(max(t0 + m.xoff + lane + kWave * u, 0l), a.T - 1)) * ESZ;
  uint32_t raw[NI][8];  // bit patterns; converted when staged so the loads stay in flight
  const int hj = 2 * (lane >> 4);  // slab: the lane's first channel of the group
  const int hcol =
      static_cast<int>(min(max(t0 + m.xoff + TT + (lane & 15), 0l), a.T - 1)) * ESZ;
  uint32_t rawh[2];
  auto xload = [&](int c) {
    const long ch0 = static_cast<long>(c) * kChunk;
    const int last = static_cast<int>(min(a.cin - ch0, static_cast<long>(kChunk))) - 1;
    const char* base = static_cast<const char*>(a.x) + static_cast<size_t>(ch0) * row_bytes;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(base), 0, last * row_bytes + static_cast<int>(a.T) * ESZ, 0x00020000);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int srow = min(8 * g + j, last) * row_bytes;
#pragma unroll
      for (int u = 0; u < NI; ++u) {
        if constexpr (DT == GSVK_F32)
          raw[u][j] = __builtin_amdgcn_raw_buffer_load_b32(rs, tcol[u], srow, 0);
        else
          raw[u][j] = __builtin_amdgcn_raw_buffer_load_b16(rs, tcol[u], srow, 0);
      }
    }
    if constexpr (kSlab) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int off = hcol + min(8 * g + hj + q, last) * row_bytes;
        if constexpr (DT == GSVK_F32)
          rawh[q] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
        else
          rawh[q] = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
      }
    }
  };
  // Tiles whose staged columns all lie inside [0, T), with a whole channel group, skip the
  // per-element zeroing of padding columns and channels; the input LeakyReLU (act 1: the max form
  // for slopes in (0, 1], 2: lrelu_ref) is chosen once per chunk. The values staged are the same
  // either way.
  const bool interior = t0 + m.xoff >= 0 && t0 + m.xoff + TTH <= a.T;
  float m1 = -1.f;
  asm("" : "+s"(m1));
  auto stage_rows = [&](auto fast, auto act, int c) {
    const long ch0 = static_cast<long>(c) * kChunk + 8 * g;
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      const int tp = lane + kWave * u;
      const long t = t0 + m.xoff + tp;
      const bool tok = t >= 0 && t < a.T;
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[j] = DT == GSVK_F32 ? __builtin_bit_cast(float, raw[u][j]) : h2f(raw[u][j]);
        if constexpr (!decltype(fast)::value) v[j] = tok && ch0 + j < a.cin ? v[j] : 0.f;
        if constexpr (decltype(act)::value == 1) v[j] = lrelu_max(v[j], a.slope);
        else if constexpr (decltype(act)::value == 2) v[j] = lrelu_ref(v[j], a.slope);
      }
      if constexpr (P == 2) {  // the exact split: hi and lo planes
        const u32x4 hi = {pack_h2(v[0], v[1]), pack_h2(v[2], v[3]), pack_h2(v[4], v[5]),
                          pack_h2(v[6], v[7])};
        const u32x4 lo = {split_rest2(hi[0], v[0], v[1], m1), split_rest2(hi[1], v[2], v[3], m1),
                          split_rest2(hi[2], v[4], v[5], m1), split_rest2(hi[3], v[6], v[7], m1)};
        *reinterpret_cast<u32x4*>(xs + (static_cast<size_t>(g) * TTH + tp) * 8) = hi;
        *reinterpret_cast<u32x4*>(xs + (static_cast<size_t>(4 + g) * TTH + tp) * 8) = lo;
      } else {
        // f2h2 rounds the LeakyReLU's product to fp32 before the rounding to fp16, as a LeakyReLU
        // stored first would: with fp16 x the compiler would otherwise fuse both into one
        // v_fma_mixlo (rounded once), another value where the fp32 product is an fp16 halfway case
        // (slope 0.1: products in the fp16 subnormal range).
        const u32x4 hi = {f2h2(v[0], v[1]), f2h2(v[2], v[3]), f2h2(v[4], v[5]), f2h2(v[6], v[7])};
        *reinterpret_cast<u32x4*>(xs + (static_cast<size_t>(g) * TTH + tp) * 8) = hi;
      }
    }
    if constexpr (kSlab) {  // the halo slab: channels hj, hj + 1 of column TT + (lane & 15)
      const int tp = TT + (lane & 15);
      const long t = t0 + m.xoff + tp;
      const bool tok = t >= 0 && t < a.T;
      float v[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        v[q] = DT == GSVK_F32 ? __builtin_bit_cast(float, rawh[q]) : h2f(rawh[q]);
        if constexpr (!decltype(fast)::value) v[q] = tok && ch0 + hj + q < a.cin ? v[q] : 0.f;
        if constexpr (decltype(act)::value == 1) v[q] = lrelu_max(v[q], a.slope);
        else if constexpr (decltype(act)::value == 2) v[q] = lrelu_ref(v[q], a.slope);
      }
      const size_t at = (static_cast<size_t>(g) * TTH + tp) * 8 + hj;
      if constexpr (P == 2) {
        const uint32_t hi = pack_h2(v[0], v[1]);
        *reinterpret_cast<uint32_t*>(xs + at) = hi;
        *reinterpret_cast<uint32_t*>(xs + at + static_cast<size_t>(4) * TTH * 8) =
            split_rest2(hi, v[0], v[1], m1);
      } else {
        *reinterpret_cast<uint32_t*>(xs + at) = f2h2(v[0], v[1]);
      }
    }
  };
  // The max form pays off in the exact split, where the staging is longest; the one-plane modes
  // (round_x, fp16 storage) measured faster with lrelu_ref.
  const int actk = !a.xact ? 0 : P == 2 && a.slope > 0.f && a.slope <= 1.f ? 1 : 2;
  auto stage = [&](int c) {
    using A0 = std::integral_constant<int, 0>;
    using A1 = std::integral_constant<int, 1>;
    using A2 = std::integral_constant<int, 2>;
    if (interior && static_cast<long>(c) * kChunk + 8 * g + 8 <= a.cin) {
      if constexpr (P == 2) {
        if (actk == 1) return stage_rows(std::true_type{}, A1{}, c);
      }
      if (actk) stage_rows(std::true_type{}, A2{}, c);
      else stage_rows(std::true_type{}, A0{}, c);
    } else {
      if (actk) stage_rows(std::false_type{}, A2{}, c);
      else stage_rows(std::false_type{}, A0{}, c);
    }
  };

  // ---- weights: groups of up to kTapGroup taps of the chunk through LDS ------------------------
  // Group q covers chunk c = q / ng, taps kk0 = kTapGroup (q % ng) and the next kTapGroup - 1
  // (fewer at the end of k). In LDS, ws[tap][channel group][16 NO rows][8]: a B fragment read is
  // then 16 consecutive 16-byte rows, like the x reads (no bank conflicts). Item it = tid + 256 u
  // is tap it / (64 NO), channel group (it / (16 NO)) % 4, row it % (16 NO): consecutive lanes read
  // consecutive 16-byte rows of the packed weights and write consecutive rows of LDS.
  constexpr int TO = FS * NO;
  constexpr int WITEMS = kTapGroup * 4 * TO;                 // 16-byte rows per group
  constexpr int WPT = (WITEMS + kThreads - 1) / kThreads;   // per thread
  _Float16* ws = xs + static_cast<size_t>(P) * 4 * TTH * 8;  // [kTapGroup][4][TO][8]
  const int ng = (m.kn + kTapGroup - 1) / kTapGroup;
  const int Q = a.nch * ng;
  // The packed weights as a buffer: a group's first tap as the scalar offset, each item's place
  // in the group (tap slot, channel group, row) as a 32-bit vector offset fixed for the launch;
  // only a chunk's short last group clamps the tap slot. (The entry points keep the packed weights
  // under 2 GiB.)
  const int tap_bytes = static_cast<int>(a.opad) * 4 * 16;  // one tap of a chunk: 4 x opad rows
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(m.wp), 0, 0x7FFFFFFF, 0x00020000);
  int wofs[WPT], wtap[WPT];
#pragma unroll
  for (int u = 0; u < WPT; ++u) {
    const int it = min(tid + kThreads * u, WITEMS - 1);
    wtap[u] = it / (4 * TO);
    wofs[u] = (((it / TO) & 3) * static_cast<int>(a.opad) + static_cast<int>(o0) + it % TO) * 16;
  }
  u32x4 wraw[WPT];
  auto wload = [&](int q) {
    const int c = q / ng, kk0 = (q - c * ng) * kTapGroup, nt = min(kTapGroup, m.kn - kk0);
    const int s0 = (c * m.kn + kk0) * tap_bytes;
#pragma unroll
    for (int u = 0; u < WPT; ++u)
      wraw[u] = __builtin_amdgcn_raw_buffer_load_b128(
          wrs, wofs[u] + min(wtap[u], nt - 1) * tap_bytes, s0, 0);
  };
  auto wstage = [&]() {
#pragma unroll
    for (int u = 0; u < WPT; ++u) {
      const int it = tid + kThreads * u;  // = ((tap 4 + group) TO + row): the LDS row
      if (WITEMS % kThreads == 0 || it < WITEMS)
        *reinterpret_cast<u32x4*>(ws + static_cast<size_t>(it) * 8) = wraw[u];
    }
  };

  const int orow = FS == 16 ? r16 : r32;  // this lane's output row within a fragment
  float bias[NO];
#pragma unroll
  for (int n = 0; n < NO; ++n)
    bias[n] = a.bias ? a.bias[min(o0 + FS * n + orow, a.cout - 1)] : 0.f;

  using Acc = typename std::conditional<FS == 16, f4v, f16v>::type;
  Acc acc[NT][NO];
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int n = 0; n < NO; ++n) acc[i][n] = Acc{};

  // One step: tap kk0 + tl (slot tl of the group) of the staged chunk. Only LDS reads feed the
  // MFMAs.
  auto step = [&](int kk, int tl) {
    const int sh = kk * a.dil;
    if constexpr (FS == 16) {
      const _Float16* xw = xs + (static_cast<size_t>(grp) * TTH + wave * 16 * NT + r16) * 8;
      const _Float16* wr = ws + (static_cast<size_t>(grp) * TO + r16) * 8;
      h8 xf[NT][P], wf[NO];
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int i = 0; i < NT; ++i)
          xf[i][p] = *reinterpret_cast<const h8*>(
              xw + (static_cast<size_t>(p) * 4 * TTH + 16 * i + sh) * 8);
#pragma unroll
      for (int n = 0; n < NO; ++n)
        wf[n] = *reinterpret_cast<const h8*>(wr + (static_cast<size_t>(tl) * 4 * TO + 16 * n) * 8);
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int n = 0; n < NO; ++n)
#pragma unroll
          for (int i = 0; i < NT; ++i)
            acc[i][n] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[i][p], wf[n], acc[i][n], 0, 0, 0);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int gq = 2 * h + hl;  // channel group this lane feeds
        const _Float16* xw = xs + (static_cast<size_t>(gq) * TTH + wave * 32 * NT + r32) * 8;
        const _Float16* wr = ws + (static_cast<size_t>(gq) * TO + r32) * 8;
        h8 xf[NT][P], wf[NO];
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int i = 0; i < NT; ++i)
            xf[i][p] = *reinterpret_cast<const h8*>(
                xw + (static_cast<size_t>(p) * 4 * TTH + 32 * i + sh) * 8);
#pragma unroll
        for (int n = 0; n < NO; ++n)
          wf[n] =
              *reinterpret_cast<const h8*>(wr + (static_cast<size_t>(tl) * 4 * TO + 32 * n) * 8);
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int n = 0; n < NO; ++n)
#pragma unroll
            for (int i = 0; i < NT; ++i)
              acc[i][n] =
                  __builtin_amdgcn_mfma_f32_32x32x16_f16(xf[i][p], wf[n], acc[i][n], 0, 0, 0);
      }
    }
  };

  // Group g of chunk c: refill LDS from the registers loaded one group earlier (x only at g = 0),
  // then load ahead: the next group's weights first, then, at g = 0, the next chunk's x. Issued in
  // that order, each weight load can be waited for without waiting for the x loads, which get the
  // whole chunk to arrive. The last group reloads in-bounds data that is not used. The groups of
  // a chunk are laid out in straight-line code (at most three for k <= 12; further groups loop) so
  // the compiler can count the loads in flight exactly.
  auto group = [&](int c, int g) {
    const int kk0 = g * kTapGroup, nt = min(kTapGroup, m.kn - kk0);
    if (c > 0 || g > 0) __syncthreads();  // every wave is done with the previous group
    if (g == 0) stage(c);
    wstage();
    __syncthreads();
    // (Unconditional, with clamped indices past the end: loads under a branch would make the
    // compiler assume the worst order and wait for the x loads here.)
    wload(min(c * ng + g + 1, Q - 1));
    __builtin_amdgcn_sched_barrier(0);  // keep the weight loads ahead of the x loads
    if (g == 0) xload(min(c + 1, a.nch - 1));
#pragma unroll
    for (int tl = 0; tl < kTapGroup; ++tl)
      if (tl < nt) step(kk0 + tl, tl);
  };

  xload(0);
  wload(0);
  for (int c = 0; c < a.nch; ++c) {
    group(c, 0);
    if (ng > 1) group(c, 1);
    if (ng > 2) group(c, 2);
    for (int g = 3; g < ng; ++g) group(c, g);
  }

  // ---- epilogue ---------------------------------------------------------------------------------
  // A lane's results come in runs of four consecutive positions of one output row: per fragment
  // one run (FS 16) or four (FS 32, q = 0..3). Output-row block n at a time; the residual
  // epilogues read block n + 1's cur before block n is finished, so each block's loads are in
  // flight together (two blocks of registers at most).
  constexpr int RUNS = FS == 16 ? 1 : 4;
  auto run_t = [&](int i, int q) -> long {
    if constexpr (FS == 16) return t0 + wave * 16 * NT + 16 * i + 4 * grp;
    else return t0 + wave * 32 * NT + 32 * i + 8 * q + 4 * hl;
  };
  auto run_v = [&](int i, int n, int q) -> f4v {
    if constexpr (FS == 16) return acc[i][n];
    else return f4v{acc[i][n][4 * q], acc[i][n][4 * q + 1], acc[i][n][4 * q + 2], acc[i][n][4 * q + 3]};
  };
  f4v cur[2][NT * RUNS];
  auto load_block = [&](f4v (&c)[NT * RUNS], int n) {
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
      for (int q = 0; q < RUNS; ++q)
        c[i * RUNS + q] = load_cur<DT>(a, m, o0 + FS * n + orow, run_t(i, q));
  };
  const bool has_res = a.epi == GSVK_CONV_EPI_RES_LRELU || a.epi == GSVK_CONV_EPI_RES;
  if (has_res) load_block(cur[0], 0);
#pragma unroll
  for (int n = 0; n < NO; ++n) {
    if (has_res && n + 1 < NO) load_block(cur[(n + 1) & 1], n + 1);
    const long o = o0 + FS * n + orow;
    if (o >= a.cout) continue;
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
      for (int q = 0; q < RUNS; ++q) {
        const long t = run_t(i, q);
        if (t < m.nq) finish4<DT>(a, m, o, t, run_v(i, n, q), bias[n], cur[n & 1][i * RUNS + q]);
      }
  }
}

template <int XM, int NT, int NO, int HMAX, int FS>
constexpr size_t lds_bytes() {
  return static_cast<size_t>(planes<XM>()) * 4 * (kWaves * FS * NT + HMAX) * 16 +
         static_cast<size_t>(kTapGroup) * 4 * FS * NO * 16;
}

template <int XM, int NT, int NO, int HMAX, int FS = 16>
int launch_tiles(const ConvArgs& a, hipStream_t st) {
  constexpr size_t lds = lds_bytes<XM, NT, NO, HMAX, FS>();
  auto kern = conv1d_mfma<XM, NT, NO, HMAX, FS>;
  if constexpr (lds > 64 * 1024) {
    static std::atomic<bool> lds_ok[kMaxDevices];
    if (!allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds, lds_ok)) return GSVK_E_HIP;
  }
  const long npos = a.up ? a.T + 1 : a.T;  // a phase of a transposed convolution: <= T + 1
  const long gx = (npos + kWaves * FS * NT - 1) / (kWaves * FS * NT);
  const long gy = (a.cout + FS * NO - 1) / (FS * NO);
  ConvArgs b = a;
  // padding workgroups (tile >= gx) return at once
  b.xspan = gx >= kXcdMinTiles ? (gx + kXcds - 1) / kXcds : 0;
  const long gxl = b.xspan ? b.xspan * kXcds : gx;
  hipLaunchKernelGGL(kern,
                     dim3(static_cast<unsigned>(gxl), static_cast<unsigned>(gy),
                          static_cast<unsigned>(a.up ? a.up : 1)),
                     dim3(kThreads), lds, st, b);
  return launch_status();
}

template <int XM, int NT, int HMAX>
int launch_no(const ConvArgs& a, int no, hipStream_t st) {
  switch (no) {
    case 1: return launch_tiles<XM, NT, 1, HMAX>(a, st);
    case 2: return launch_tiles<XM, NT, 2, HMAX>(a, st);
    case 3: return launch_tiles<XM, NT, 3, HMAX>(a, st);
    default: return launch_tiles<XM, NT, 4, HMAX>(a, st);
  }
}

// Output rows per wave: the largest fragment count (4..1) that pads at most a sixth of the rows
// it computes, and whose last tile stays inside the packed rows. Columns per wave: 32 (128 per
// workgroup, three workgroups per CU). Measured on the decoder stages: more, smaller workgroups in
// flight beat larger register tiles (64 columns or 96 rows per wave cut the LDS bytes per MFMA but
// were slower on every stage: the group refills, not LDS bandwidth, set the pace).
template <int XM>
int launch_plan(const ConvArgs& a, hipStream_t st) {
  const long ofr = (a.cout + 15) / 16;
  int no = 1;
  for (int c = 4; c > 1; --c) {
    const long rows = (ofr + c - 1) / c * c;
    if (6 * (rows - ofr) <= rows && rows * 16 <= a.opad) {
      no = c;
      break;
    }
  }
  // Halos of up to 16 columns (k 3 at dilations up to 8, every dilation-1 ResBlock convolution,
  // the upsamplers) take the kernels with the 16-column halo slab; measured on the decoder
  // graph, 3% faster exact than staging a 64-column halo block for them.
  const int halo = a.up ? (a.k + a.up - 1) / a.up - 1 : (a.k - 1) * a.dil;
  if (halo <= 64 && a.cout >= 24) {
    // 32-wide fragments, 64 positions x 64 output rows per wave (256 x 64 per workgroup), when
    // 64-row tiles pad at most a sixth of the rows and the grid still holds about 1.5 workgroups
    // per CU of the 256 (two fit on a CU). Measured on the decoder stages: 3-10% faster than the
    // 16-wide tiles at 192 channels; with 32-row tiles (96, 48, 24 channels) slower, so those keep
    // the 16-wide kernel.
    const long r64 = (a.cout + 63) / 64 * 64;
    const int nw = 6 * (r64 - a.cout) <= r64 ? 2 : 1;
    const long npos = a.up ? a.T + 1 : a.T;
    const long groups = (npos + 255) / 256 * ((a.cout + 32 * nw - 1) / (32 * nw)) * (a.up ? a.up : 1);
    if (nw == 2 && groups >= 384)
      return halo <= 16 ? launch_tiles<XM, 2, 2, 16, 32>(a, st)
                        : launch_tiles<XM, 2, 2, 64, 32>(a, st);
  }
  if (halo <= 64) {
    // A grid of fewer than 512 workgroups (two per CU) leaves matrix cores idle: the 384-channel
    // stage, its upsampler and conv_pre launch 48-240. There, two 16-row fragments per wave
    // instead of three or four give 1.5-2x the workgroups; measured on the whole decoder graph
    // (alternating on one box): exact 3955-4035 -> 3767-3852 us, round_x 3090-3106 -> 2981-2987,
    // fp16 storage 2946-2959 -> 2864. Smaller time tiles instead (32 columns per workgroup) or
    // both were slower.
    // With the exact split (two staged planes per chunk), such grids instead take 64-column time
    // tiles at the full fragment count: about as many workgroups, half the staging per product.
    // Alternating on one box: the 384-channel stage 5% faster exact, the decoder graph 3506-3518
    // -> 3465-3474 us; with one plane (round_x, fp16 storage) the same tiles were 7% slower there.
    const long npos = a.up ? a.T + 1 : a.T;
    const long groups =
        (npos + 127) / 128 * ((a.cout + 16 * no - 1) / (16 * no)) * (a.up ? a.up : 1);
    if constexpr (XM == kXSplit) {
      if (groups < 512)
        return halo <= 16 ? launch_no<XM, 1, 16>(a, no, st) : launch_no<XM, 1, 64>(a, no, st);
    }
    if (groups < 512 && no > 2 && (a.cout + 31) / 32 * 32 <= a.opad) no = 2;
    return halo <= 16 ? launch_no<XM, 2, 16>(a, no, st) : launch_no<XM, 2, 64>(a, no, st);
  }
  return launch_no<XM, 1, kMaxHalo>(a, no, st);
}

}  // namespace
}  // namespace gsvk

using namespace gsvk;

extern "C" size_t gsvk_conv1d_packed_elems(size_t c_out, size_t c_in, size_t k) {
  if (!c_out || !c_in || !k) return 0;
  return (c_in + kChunk - 1) / kChunk * k * ((c_out + kOPad - 1) / kOPad * kOPad) * kChunk;
}

extern "C" int gsvk_conv1d_pack(const uint16_t* w, size_t c_out, size_t c_in, size_t k,
                                uint16_t* w_packed, size_t packed_elems, void* stream) {
  if (!w || !w_packed) return GSVK_E_NULL;
  if (!c_out || !c_in || !k || c_out > (1ul << 24) || c_in > (1ul << 24) || k > 4096)
    return GSVK_E_SIZE;
  const size_t total = gsvk_conv1d_packed_elems(c_out, c_in, k);
  if (packed_elems < total) return GSVK_E_SIZE;
  if (overlaps(w, c_out * c_in * k * 2, w_packed, total * 2)) return GSVK_E_ALIAS;
  const long opad = static_cast<long>((c_out + kOPad - 1) / kOPad * kOPad);
  const long blocks = std::min<long>((static_cast<long>(total) + 255) / 256, 16384);
  hipLaunchKernelGGL(conv_pack, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w, w_packed, static_cast<long>(c_out),
                     static_cast<long>(c_in), static_cast<long>(k), opad,
                     static_cast<long>(total));
  return launch_status();
}

namespace gsvk {
namespace {

// Validation and launch shared by both entry points. T: input columns; Tout: output columns.
int conv_entry(ConvArgs a, int dtype, int round_x, size_t T, size_t Tout, size_t wb,
               hipStream_t st) {
  if (dtype != GSVK_F32 && dtype != GSVK_F16) return GSVK_E_DTYPE;
  a.xact = (a.epi & GSVK_CONV_X_LRELU) != 0;
  a.epi &= ~GSVK_CONV_X_LRELU;
  if (a.epi < GSVK_CONV_EPI_BIAS || a.epi > GSVK_CONV_EPI_TANH) return GSVK_E_DTYPE;
  const bool reads_res = a.epi == GSVK_CONV_EPI_RES_LRELU || a.epi == GSVK_CONV_EPI_RES;
  const bool has_cur = reads_res || a.epi == GSVK_CONV_EPI_DUAL;
  const bool has_y = a.epi != GSVK_CONV_EPI_RES;
  if (!a.x || !a.wp || (has_y && !a.y) || (has_cur && !a.cur)) return GSVK_E_NULL;
  const size_t ldx = static_cast<size_t>(a.ldx), ldy = static_cast<size_t>(a.ldy),
               ldc = static_cast<size_t>(a.ldc);
  if (ldx < T || (has_y && ldy < Tout) || (has_cur && ldc < Tout)) return GSVK_E_SIZE;
  if (kChunk * ldx * dtype_size(dtype) >= (1ul << 31)) return GSVK_E_SIZE;
  if (wb >= (1ul << 31)) return GSVK_E_SIZE;  // packed weights: 32-bit buffer offsets
  if (!aligned16(a.wp)) return GSVK_E_ARG;
  if (!has_y) a.y = nullptr, a.ldy = 0;
  if (!has_cur) a.cur = nullptr, a.ldc = 0;
  if (!reads_res || a.res == a.cur) a.res = nullptr;
  const size_t esz = dtype_size(dtype);
  const size_t xb = span_bytes(static_cast<size_t>(a.cin), T, ldx, esz);
  const size_t bb = a.bias ? static_cast<size_t>(a.cout) * 4 : 0;
  const size_t yb = has_y ? span_bytes(static_cast<size_t>(a.cout), Tout, ldy, esz) : 0;
  const size_t cb = has_cur ? span_bytes(static_cast<size_t>(a.cout), Tout, ldc, esz) : 0;
  const void* outs[2] = {a.y, a.cur};
  const size_t outb[2] = {yb, cb};
  for (int i = 0; i < 2; ++i)
    if (overlaps(outs[i], outb[i], a.x, xb) || overlaps(outs[i], outb[i], a.wp, wb) ||
        overlaps(outs[i], outb[i], a.bias, bb) || overlaps(outs[i], outb[i], a.res, cb))
      return GSVK_E_ALIAS;
  if (overlaps(a.y, yb, a.cur, cb)) return GSVK_E_ALIAS;
  const size_t va = esz * 4;  // one vector: four elements
  a.vec = Tout >= 4 && (!a.y || (ldy % 4 == 0 && reinterpret_cast<uintptr_t>(a.y) % va == 0)) &&
          (!a.cur || (ldc % 4 == 0 && reinterpret_cast<uintptr_t>(a.cur) % va == 0)) &&
          (!a.res || reinterpret_cast<uintptr_t>(a.res) % va == 0);
  if (a.up && a.up != 1) a.vec = false;  // interleaved phases: element stores
  if (dtype == GSVK_F16) return launch_plan<kXF16>(a, st);
  return round_x ? launch_plan<kXRound>(a, st) : launch_plan<kXSplit>(a, st);
}

}  // namespace
}  // namespace gsvk

extern "C" int gsvk_conv1d(int dtype, int round_x, const void* x, size_t ldx,
                           const uint16_t* w_packed, const float* bias, int epi, float slope,
                           void* cur, const void* res, size_t ldc, void* y, size_t ldy,
                           size_t c_in, size_t c_out, size_t T, size_t k, size_t dilation,
                           void* stream) {
  if (!c_in || !c_out || !T || !k || !dilation) return GSVK_E_SIZE;
  if (c_in > (1ul << 24) || c_out > (1ul << 24) || k > 4096 || dilation > 4096 ||
      T > (1ul << 31) - 512 || ldx > (1ul << 40) || ldy > (1ul << 40) || ldc > (1ul << 40))
    return GSVK_E_SIZE;
  if ((k - 1) * dilation > static_cast<size_t>(kMaxHalo)) return GSVK_E_ARG;
  ConvArgs a{};
  a.x = x, a.wp = w_packed, a.bias = bias, a.cur = cur, a.res = res, a.y = y;
  a.cin = static_cast<long>(c_in), a.cout = static_cast<long>(c_out), a.T = static_cast<long>(T);
  a.ldx = static_cast<long>(ldx), a.ldc = static_cast<long>(ldc), a.ldy = static_cast<long>(ldy);
  a.k = static_cast<int>(k), a.dil = static_cast<int>(dilation);
  a.pad = static_cast<int>((k - 1) * dilation / 2);
  a.nch = static_cast<int>((c_in + kChunk - 1) / kChunk);
  a.opad = static_cast<int>((c_out + kOPad - 1) / kOPad * kOPad);
  a.epi = epi, a.slope = slope;
  return conv_entry(a, dtype, round_x, T, T, gsvk_conv1d_packed_elems(c_out, c_in, k) * 2,
                    static_cast<hipStream_t>(stream));
}

extern "C" size_t gsvk_convt1d_packed_elems(size_t c_out, size_t c_in, size_t k, size_t stride) {
  if (!c_out || !c_in || !k || !stride || k < stride) return 0;
  // the phases' tap counts ceil((k - r) / u) add up to k
  return (c_in + kChunk - 1) / kChunk * k * ((c_out + kOPad - 1) / kOPad * kOPad) * kChunk;
}

extern "C" int gsvk_convt1d_pack(const uint16_t* w, size_t c_out, size_t c_in, size_t k,
                                 size_t stride, uint16_t* w_packed, size_t packed_elems,
                                 void* stream) {
  if (!w || !w_packed) return GSVK_E_NULL;
  if (!c_out || !c_in || !k || !stride || c_out > (1ul << 24) || c_in > (1ul << 24) || k > 4096 ||
      stride > 4096)
    return GSVK_E_SIZE;
  if (k < stride) return GSVK_E_ARG;
  const size_t total = gsvk_convt1d_packed_elems(c_out, c_in, k, stride);
  if (packed_elems < total) return GSVK_E_SIZE;
  if (overlaps(w, c_out * c_in * k * 2, w_packed, total * 2)) return GSVK_E_ALIAS;
  const long opad = static_cast<long>((c_out + kOPad - 1) / kOPad * kOPad);
  const long nch = static_cast<long>((c_in + kChunk - 1) / kChunk);
  const long blocks = std::min<long>((static_cast<long>(total) + 255) / 256, 16384);
  hipLaunchKernelGGL(convt_pack, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w, w_packed, static_cast<long>(c_out),
                     static_cast<long>(c_in), static_cast<long>(k), static_cast<long>(stride), nch,
                     opad, static_cast<long>(total));
  return launch_status();
}

extern "C" int gsvk_convt1d(int dtype, int round_x, const void* x, size_t ldx,
                            const uint16_t* w_packed, const float* bias, int epi, float slope,
                            void* cur, const void* res, size_t ldc, void* y, size_t ldy,
                            size_t c_in, size_t c_out, size_t T, size_t k, size_t stride,
                            void* stream) {
  if (!c_in || !c_out || !T || !k || !stride) return GSVK_E_SIZE;
  if (c_in > (1ul << 24) || c_out > (1ul << 24) || k > 4096 || stride > 4096 ||
      T > (1ul << 31) / stride - 512 || ldx > (1ul << 40) || ldy > (1ul << 40) ||
      ldc > (1ul << 40))
    return GSVK_E_SIZE;
  // pad = (k - u) / 2 needs k >= u (ConvT1d, conv1d.hpp:262); each phase's taps share one LDS tile
  if (k < stride || (k + stride - 1) / stride - 1 > 64) return GSVK_E_ARG;
  ConvArgs a{};
  a.x = x, a.wp = w_packed, a.bias = bias, a.cur = cur, a.res = res, a.y = y;
  a.cin = static_cast<long>(c_in), a.cout = static_cast<long>(c_out), a.T = static_cast<long>(T);
  a.ldx = static_cast<long>(ldx), a.ldc = static_cast<long>(ldc), a.ldy = static_cast<long>(ldy);
  a.k = static_cast<int>(k), a.dil = 1, a.pad = 0;
  a.nch = static_cast<int>((c_in + kChunk - 1) / kChunk);
  a.opad = static_cast<int>((c_out + kOPad - 1) / kOPad * kOPad);
  a.epi = epi, a.slope = slope;
  a.up = static_cast<int>(stride), a.Tout = static_cast<long>(T * stride);
  a.pad_t = static_cast<int>((k - stride) / 2);
  return conv_entry(a, dtype, round_x, T, T * stride,
                    gsvk_convt1d_packed_elems(c_out, c_in, k, stride) * 2,
                    static_cast<hipStream_t>(stream));
}
