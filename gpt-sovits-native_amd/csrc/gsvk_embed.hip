// gsvk_embed.hip — token-embedding gather fused with the scaled sinusoidal positional add (gfx950).
//
// Three row kernels. embed_pe_vec (short calls, latency-bound): one wave64 per output row, the
// wave's id and position read once, then each lane moves 8 consecutive columns: the table row chunk
// (16 B for f16/bf16, 32 B for f32), the PE row chunk (32 B fp32), optionally the mm row chunk and
// the bias chunk, and writes 8 output columns. embed_pe_rows (long calls): RPW consecutive rows per
// wave, their ids and positions read with one vector load, U rows' loads in flight at once.
// prefill_input_rows (the T2S prefill input): the text row and the prompt row at one position
// share a single read of the PE row. Table and PE rows are read through the caches (ids repeat);
// output rows of calls beyond kStreamBytes are written non-temporally. The arithmetic is the
// reference's exactly (fmaf is the contraction AppleClang applies to `e + alpha * pe`), so the
// result is bit-identical to the CPU restatement for every input.
#include "gsvk_common.hpp"

namespace gsvk {
namespace {

struct EmbArgs {
  const void* table;
  const void* ids;
  const int64_t* pos;
  const float* pe;
  const void* mm;
  const float* bias;
  void* out;
  int32_t* err;
  long vocab;
  long max_pos;
  long rows;
  long D;
  int64_t pos0;
  float alpha;
  int ids32;
};

constexpr int kBlock = 256;
#ifndef GSVK_EMBED_U
#define GSVK_EMBED_U 8
#endif
#ifndef GSVK_EMBED_RPW
#define GSVK_EMBED_RPW 32
#endif

// 8 consecutive elements starting at element i (i multiple of 8, 16-byte aligned for every dtype).
template <int DT>
__device__ __forceinline__ void load8(const void* p, size_t i, float (&v)[8]) {
  if constexpr (DT == GSVK_F32) {
    float a[4], b[4];
    Store<GSVK_F32>::load(p, i, a);
    Store<GSVK_F32>::load(p, i + 4, b);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[k] = a[k];
      v[4 + k] = b[k];
    }
  } else {
    Store<DT>::load(p, i, v);
  }
}
template <int DT, bool NT>
__device__ __forceinline__ void store8(void* p, size_t i, const float (&v)[8]) {
  if constexpr (DT == GSVK_F32) {
    const float a[4] = {v[0], v[1], v[2], v[3]}, b[4] = {v[4], v[5], v[6], v[7]};
    Store<GSVK_F32>::store<NT>(p, i, a);
    Store<GSVK_F32>::store<NT>(p, i + 4, b);
  } else {
    Store<DT>::template store<NT>(p, i, v);
  }
}

// Row check shared by both paths: returns the table row and PE row element offsets, or -1.
__device__ __forceinline__ bool row_source(const EmbArgs& a, long r, size_t& trow, size_t& prow) {
  const int64_t id = a.ids32 ? static_cast<int64_t>(static_cast<const int32_t*>(a.ids)[r])
                             : static_cast<const int64_t*>(a.ids)[r];
  const int64_t p = a.pos ? a.pos[r] : a.pos0 + r;
  if (id < 0 || id >= a.vocab || p < 0 || p >= a.max_pos) return false;
  trow = static_cast<size_t>(id) * a.D;
  prow = static_cast<size_t>(p) * a.D;
  return true;
}

template <int OUT, int TAB, bool NT, int BLOCK>
__global__ __launch_bounds__(BLOCK) void embed_pe_vec(EmbArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const long wave = static_cast<long>(blockIdx.x) * (BLOCK / kWave) + (threadIdx.x / kWave);
  const long nwaves = static_cast<long>(gridDim.x) * (BLOCK / kWave);
  const long nch = a.D / 8;
  for (long r = wave; r < a.rows; r += nwaves) {
    size_t trow = 0, prow = 0;
    const bool ok = row_source(a, r, trow, prow);
    const size_t orow = static_cast<size_t>(r) * a.D;
    if (!ok) {
      if (lane == 0 && a.err) *a.err = 1;
      float nan8[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) nan8[k] = __builtin_nanf("");
      for (long c = lane; c < nch; c += kWave) store8<OUT, NT>(a.out, orow + c * 8, nan8);
      continue;
    }
    for (long c = lane; c < nch; c += kWave) {
      float e[8], pe[8], o[8];
      load8<TAB>(a.table, trow + c * 8, e);
      load8<GSVK_F32>(a.pe, prow + c * 8, pe);
      if (a.bias) {
        float b[8];
        load8<GSVK_F32>(a.bias, c * 8, b);
#pragma unroll
        for (int k = 0; k < 8; ++k) e[k] = e[k] + b[k];
      }
      if (a.mm) {
        float m[8];
        load8<OUT>(a.mm, orow + c * 8, m);
#pragma unroll
        for (int k = 0; k < 8; ++k) e[k] = m[k] + e[k];
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) o[k] = __builtin_fmaf(a.alpha, pe[k], e[k]);
      store8<OUT, NT>(a.out, orow + c * 8, o);
    }
  }
}

// Long calls: each wave owns RPW consecutive rows (one-shot). Lanes 0 .. RPW-1 read the rows' ids
// and positions with one vector load each (a per-row scalar load put a dependent HBM round trip in
// front of every row), then the rows go in groups of U: every table / PE (/ mm) chunk of the group
// is loaded before the group's arithmetic and stores, so U rows are in flight per wave. The bias
// chunk is the same for every row of the wave and is loaded once. Lane l moves the 8 columns
// 8l .. 8l + 7 (D <= 512); the arithmetic is embed_pe_vec's, so the results are the same bits.
// Measured on the replicated prefill gather (524,288 rows of 512): 32 rows per wave in groups of
// 8 moved 3.6 TB/s of floor bytes against 3.0 TB/s with one row per wave.
template <int OUT, int TAB, bool NT, int RPW, int U, bool MM>
__global__ __launch_bounds__(kBlock) void embed_pe_rows(EmbArgs a) {
  static_assert(RPW % U == 0 && RPW <= kWave, "groups of U rows within RPW <= 64");
  const int lane = threadIdx.x & (kWave - 1);
  const long wave = static_cast<long>(blockIdx.x) * (kBlock / kWave) + (threadIdx.x / kWave);
  const long r0 = wave * RPW;
  if (r0 >= a.rows) return;  // wave-uniform; no barriers
  const long nch = a.D / 8;
  const bool lane_on = lane < nch;
  const size_t col = static_cast<size_t>(lane_on ? lane : 0) * 8;
  // row r0 + j's id / position live in lane j
  const long rj = r0 + (lane < RPW ? lane : 0) < a.rows ? r0 + (lane < RPW ? lane : 0) : a.rows - 1;
  const int64_t my_id = a.ids32 ? static_cast<int64_t>(static_cast<const int32_t*>(a.ids)[rj])
                                : static_cast<const int64_t*>(a.ids)[rj];
  const int64_t my_pos = a.pos ? a.pos[rj] : a.pos0 + rj;
  const bool my_ok = my_id >= 0 && my_id < a.vocab && my_pos >= 0 && my_pos < a.max_pos;
  float bi[8];
  if (a.bias) load8<GSVK_F32>(a.bias, col, bi);
#pragma unroll
  for (int g = 0; g < RPW; g += U) {
    float e[U][8], pe[U][8], mm[MM ? U : 1][8];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = g + u;
      const int64_t id = (static_cast<int64_t>(__builtin_amdgcn_readlane(
                              static_cast<int>(static_cast<uint64_t>(my_id) >> 32), j)) << 32) |
                         static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(my_id), j));
      const int64_t p = (static_cast<int64_t>(__builtin_amdgcn_readlane(
                             static_cast<int>(static_cast<uint64_t>(my_pos) >> 32), j)) << 32) |
                        static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(my_pos), j));
      ok[u] = __builtin_amdgcn_readlane(static_cast<int>(my_ok), j) != 0;
      const size_t trow = static_cast<size_t>(ok[u] ? id : 0) * a.D;
      const size_t prow = static_cast<size_t>(ok[u] ? p : 0) * a.D;
      load8<TAB>(a.table, trow + col, e[u]);
      load8<GSVK_F32>(a.pe, prow + col, pe[u]);
      if constexpr (MM) {
        const long r = r0 + j < a.rows ? r0 + j : a.rows - 1;
        load8<OUT>(a.mm, static_cast<size_t>(r) * a.D + col, mm[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long r = r0 + g + u;
      if (r >= a.rows) break;  // wave-uniform
      const size_t orow = static_cast<size_t>(r) * a.D;
      float o[8];
      if (ok[u]) {
        if (a.bias) {
#pragma unroll
          for (int k = 0; k < 8; ++k) e[u][k] = e[u][k] + bi[k];
        }
        if constexpr (MM) {
#pragma unroll
          for (int k = 0; k < 8; ++k) e[u][k] = mm[u][k] + e[u][k];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = __builtin_fmaf(a.alpha, pe[u][k], e[u][k]);
      } else {
        if (lane == 0 && a.err) *a.err = 1;
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = __builtin_nanf("");
      }
      if (lane_on) store8<OUT, NT>(a.out, orow + col, o);
    }
  }
}

template <int OUT, int TAB>
__global__ __launch_bounds__(kBlock) void embed_pe_scalar(EmbArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const long wave = static_cast<long>(blockIdx.x) * (kBlock / kWave) + (threadIdx.x / kWave);
  const long nwaves = static_cast<long>(gridDim.x) * (kBlock / kWave);
  for (long r = wave; r < a.rows; r += nwaves) {
    size_t trow = 0, prow = 0;
    const bool ok = row_source(a, r, trow, prow);
    const size_t orow = static_cast<size_t>(r) * a.D;
    if (!ok && lane == 0 && a.err) *a.err = 1;
    for (long d = lane; d < a.D; d += kWave) {
      float o = __builtin_nanf("");
      if (ok) {
        float e = Store<TAB>::load1(a.table, trow + d);
        if (a.bias) e = e + a.bias[d];
        if (a.mm) e = Store<OUT>::load1(a.mm, orow + d) + e;
        o = __builtin_fmaf(a.alpha, a.pe[prow + d], e);
      }
      Store<OUT>::store1(a.out, orow + d, o);
    }
  }
}

// Calls with fewer rows than this are latency-bound: one wave per workgroup.
constexpr long kSmallRows = 8192;
// Rows per launch: a dispatch holds at most 2^32 - 1 work-items, so longer jobs are split.
constexpr long kMaxRowsPerLaunch = (1L << 22) * (kBlock / kWave);

template <int OUT, int TAB>
void launch_embed(EmbArgs a, bool vec_ok, hipStream_t st) {
  constexpr size_t osz = OUT == GSVK_F32 ? 4 : 2;
  const size_t isz = a.ids32 ? 4 : 8;
  const long total = a.rows;
  const EmbArgs a0 = a;
  for (long r0 = 0; r0 < total; r0 += kMaxRowsPerLaunch) {
    a.rows = total - r0 < kMaxRowsPerLaunch ? total - r0 : kMaxRowsPerLaunch;
    a.ids = static_cast<const char*>(a0.ids) + static_cast<size_t>(r0) * isz;
    a.pos = a0.pos ? a0.pos + r0 : nullptr;
    a.pos0 = a0.pos0 + r0;
    a.mm = a0.mm ? static_cast<const char*>(a0.mm) + static_cast<size_t>(r0) * a.D * osz : nullptr;
    a.out = static_cast<char*>(a0.out) + static_cast<size_t>(r0) * a.D * osz;
    const unsigned g = static_cast<unsigned>((a.rows + (kBlock / kWave) - 1) / (kBlock / kWave));
    const bool nt = static_cast<size_t>(total) * a.D * osz >= kStreamBytes;
    if (vec_ok && a.D <= 512 && a.rows >= kSmallRows) {
      constexpr int kRpw = GSVK_EMBED_RPW;
      const long waves = (a.rows + kRpw - 1) / kRpw;
      const unsigned gw = static_cast<unsigned>((waves + (kBlock / kWave) - 1) / (kBlock / kWave));
      constexpr int kU = GSVK_EMBED_U;
      if (nt && a.mm)
        hipLaunchKernelGGL((embed_pe_rows<OUT, TAB, true, kRpw, kU, true>), dim3(gw), dim3(kBlock), 0, st, a);
      else if (nt)
        hipLaunchKernelGGL((embed_pe_rows<OUT, TAB, true, kRpw, kU, false>), dim3(gw), dim3(kBlock), 0, st, a);
      else if (a.mm)
        hipLaunchKernelGGL((embed_pe_rows<OUT, TAB, false, kRpw, kU, true>), dim3(gw), dim3(kBlock), 0, st, a);
      else
        hipLaunchKernelGGL((embed_pe_rows<OUT, TAB, false, kRpw, kU, false>), dim3(gw), dim3(kBlock), 0, st, a);
    } else if (vec_ok && nt) {
      hipLaunchKernelGGL((embed_pe_vec<OUT, TAB, true, kBlock>), dim3(g), dim3(kBlock), 0, st, a);
    } else if (vec_ok && total < kSmallRows) {
      hipLaunchKernelGGL((embed_pe_vec<OUT, TAB, false, kWave>), dim3(static_cast<unsigned>(a.rows)),
                         dim3(kWave), 0, st, a);
    } else if (vec_ok) {
      hipLaunchKernelGGL((embed_pe_vec<OUT, TAB, false, kBlock>), dim3(g), dim3(kBlock), 0, st, a);
    } else {
      hipLaunchKernelGGL((embed_pe_scalar<OUT, TAB>), dim3(g), dim3(kBlock), 0, st, a);
    }
  }
}

template <int OUT>
void launch_embed_tab(int tab, const EmbArgs& a, bool vec_ok, hipStream_t st) {
  switch (tab) {
    case GSVK_F32: launch_embed<OUT, GSVK_F32>(a, vec_ok, st); break;
    case GSVK_F16: launch_embed<OUT, GSVK_F16>(a, vec_ok, st); break;
    default: launch_embed<OUT, GSVK_BF16>(a, vec_ok, st); break;
  }
}

// ---- the T2S prefill input: text rows and prompt rows sharing each PE row ----------------------
//
// T2SEngine::generate builds xy[T + P, D] from two gathers that both start at position 0
// (t2s_engine.cpp:1770-1786): text row t = bert_proj row + (text_emb[phones[t]] + b) + a_t pe(t),
// prompt row T + t = audio_emb[prompt[t]] + a_a pe(t). One wave takes RPW consecutive positions t
// and, per position, reads the PE row once for both rows: 3 row reads and 2 row writes where two
// embed_pe launches make 4 and 2. The rows' ids come in one vector load per wave (lanes 0 .. RPW-1)
// and the position's loads are unconditional (a missing row, t >= T or t >= P, reads row 0 and
// stores nothing), U positions in flight. The arithmetic is embed_pe_vec's, the same bits. The
// launches use RPW = U = 1 (the measured best, below); the template keeps the multi-position form.
struct PfArgs {
  const void* ttab;
  const void* atab;
  const void* phones;
  const void* prompt;
  const void* mm;
  const float* bias;
  const float* pe;
  void* xy;
  int32_t* err;
  long T, P, D, tvocab, avocab, max_pos;
  float at, aa;
  int ids32;
};

__device__ __forceinline__ int64_t id_at(const void* ids, bool ids32, long i) {
  return ids32 ? static_cast<int64_t>(static_cast<const int32_t*>(ids)[i])
               : static_cast<const int64_t*>(ids)[i];
}
__device__ __forceinline__ int64_t lane_i64(int64_t v, int j) {
  return (static_cast<int64_t>(__builtin_amdgcn_readlane(
              static_cast<int>(static_cast<uint64_t>(v) >> 32), j))
          << 32) |
         static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), j));
}

template <int OUT, int TAB, bool NT, int RPW, int U, int BLOCK>
__global__ __launch_bounds__(BLOCK) void prefill_input_rows(PfArgs a) {
  static_assert(RPW % U == 0 && RPW <= kWave, "groups of U positions within RPW <= 64");
  const int lane = threadIdx.x & (kWave - 1);
  const long wave = static_cast<long>(blockIdx.x) * (BLOCK / kWave) + (threadIdx.x / kWave);
  const long n = a.T > a.P ? a.T : a.P;
  const long t0 = wave * RPW;
  if (t0 >= n) return;  // wave-uniform; no barriers
  const long nch = a.D / 8;
  // position t0 + j's ids live in lane j (clamped reads: an absent id is never used)
  const long tj = t0 + (lane < RPW ? lane : 0);
  const int64_t my_ph = id_at(a.phones, a.ids32, (tj < a.T ? tj : a.T - 1));
  const int64_t my_pr = id_at(a.prompt, a.ids32, (tj < a.P ? tj : a.P - 1));
  for (long c = lane; c - lane < nch; c += kWave) {  // wave-uniform trip count
    const bool col_on = c < nch;
    const size_t col = static_cast<size_t>(col_on ? c : 0) * 8;
    float bi[8];
    if (a.bias) load8<GSVK_F32>(a.bias, col, bi);
#pragma unroll
    for (int g = 0; g < RPW; g += U) {
      float te[U][8], ae[U][8], pe[U][8], mm[U][8];
      bool tok[U], aok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const long t = t0 + g + u;
        const int64_t ph = lane_i64(my_ph, g + u), pr = lane_i64(my_pr, g + u);
        const bool pos_ok = t < a.max_pos;
        tok[u] = pos_ok && ph >= 0 && ph < a.tvocab;
        aok[u] = pos_ok && pr >= 0 && pr < a.avocab;
        load8<TAB>(a.ttab, static_cast<size_t>(tok[u] ? ph : 0) * a.D + col, te[u]);
        load8<TAB>(a.atab, static_cast<size_t>(aok[u] ? pr : 0) * a.D + col, ae[u]);
        load8<GSVK_F32>(a.pe, static_cast<size_t>(pos_ok ? t : 0) * a.D + col, pe[u]);
        if (a.mm) {
          const long r = t < a.T ? t : a.T - 1;
          load8<OUT>(a.mm, static_cast<size_t>(r) * a.D + col, mm[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const long t = t0 + g + u;
        if (t >= n) break;  // wave-uniform
        if (t < a.T) {
          float o[8];
          if (tok[u]) {
            if (a.bias) {
#pragma unroll
              for (int k = 0; k < 8; ++k) te[u][k] = te[u][k] + bi[k];
            }
            if (a.mm) {
#pragma unroll
              for (int k = 0; k < 8; ++k) te[u][k] = mm[u][k] + te[u][k];
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = __builtin_fmaf(a.at, pe[u][k], te[u][k]);
          } else {
            if (lane == 0 && a.err) *a.err = 1;
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = __builtin_nanf("");
          }
          if (col_on) store8<OUT, NT>(a.xy, static_cast<size_t>(t) * a.D + col, o);
        }
        if (t < a.P) {
          float o[8];
          if (aok[u]) {
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = __builtin_fmaf(a.aa, pe[u][k], ae[u][k]);
          } else {
            if (lane == 0 && a.err) *a.err = 1;
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = __builtin_nanf("");
          }
          if (col_on) store8<OUT, NT>(a.xy, static_cast<size_t>(a.T + t) * a.D + col, o);
        }
      }
    }
  }
}

template <int OUT, int TAB>
void launch_prefill(const PfArgs& a, hipStream_t st) {
  constexpr size_t osz = OUT == GSVK_F32 ? 4 : 2;
  const long n = a.T > a.P ? a.T : a.P;
  const bool nt = static_cast<size_t>(a.T + a.P) * a.D * osz >= kStreamBytes;
  if (n < kSmallRows) {  // latency-bound: one position per one-wave workgroup
    hipLaunchKernelGGL((prefill_input_rows<OUT, TAB, false, 1, 1, kWave>),
                       dim3(static_cast<unsigned>(n)), dim3(kWave), 0, st, a);
    return;
  }
  // Long calls: one position per wave too, four waves per workgroup. Measured on 262,144
  // positions whose PE rows are each read once from HBM (floor bytes / time, % of 8 TB/s), by
  // positions per wave x positions in flight: 1 x 1 74.1%, 2 x 2 73.6%, 4 x 4 73.4%, 8 x 4 67.7%,
  // 16 x 4 63.0%, 32 x 8 58.1%: the more waves, the more PE rows in flight.
  constexpr int kRpw = 1, kU = 1;
  const long waves = (n + kRpw - 1) / kRpw;
  const unsigned g = static_cast<unsigned>((waves + (kBlock / kWave) - 1) / (kBlock / kWave));
  if (nt)
    hipLaunchKernelGGL((prefill_input_rows<OUT, TAB, true, kRpw, kU, kBlock>), dim3(g),
                       dim3(kBlock), 0, st, a);
  else
    hipLaunchKernelGGL((prefill_input_rows<OUT, TAB, false, kRpw, kU, kBlock>), dim3(g),
                       dim3(kBlock), 0, st, a);
}

template <int OUT>
void launch_prefill_tab(int tab, const PfArgs& a, hipStream_t st) {
  switch (tab) {
    case GSVK_F32: launch_prefill<OUT, GSVK_F32>(a, st); break;
    case GSVK_F16: launch_prefill<OUT, GSVK_F16>(a, st); break;
    default: launch_prefill<OUT, GSVK_BF16>(a, st); break;
  }
}

}  // namespace
}  // namespace gsvk

using namespace gsvk;

extern "C" int gsvk_embed_pe(int out_dtype, int table_dtype, int index_type, const void* table,
                             size_t vocab, const void* ids, const int64_t* pos, int64_t pos0,
                             const float* pe, size_t max_pos, float alpha, const void* mm,
                             const float* bias, void* out, size_t rows, size_t D, int32_t* err,
                             void* stream) {
  if (!valid_dtype(out_dtype) || !valid_dtype(table_dtype)) return GSVK_E_DTYPE;
  if (index_type != GSVK_I64 && index_type != GSVK_I32) return GSVK_E_DTYPE;
  if (!table || !ids || !pe || !out) return GSVK_E_NULL;
  if (rows == 0 || D == 0 || vocab == 0 || max_pos == 0 || rows > (1ul << 40) ||
      D > (1ul << 30) || vocab > (1ul << 40) || max_pos > (1ul << 40))
    return GSVK_E_SIZE;
  if (D % 2) return GSVK_E_ARG;
  const size_t osz = dtype_size(out_dtype), obytes = rows * D * osz;
  const size_t isz = index_type == GSVK_I64 ? 8 : 4;
  if (mm && mm != out && overlaps(out, obytes, mm, obytes)) return GSVK_E_ALIAS;
  if (overlaps(out, obytes, table, vocab * D * dtype_size(table_dtype)) ||
      overlaps(out, obytes, ids, rows * isz) || overlaps(out, obytes, pos, pos ? rows * 8 : 0) ||
      overlaps(out, obytes, pe, max_pos * D * 4) || overlaps(out, obytes, bias, bias ? D * 4 : 0) ||
      overlaps(out, obytes, err, err ? 4 : 0))
    return GSVK_E_ALIAS;
  EmbArgs a{table, ids, pos, pe, mm, bias, out, err, static_cast<long>(vocab),
            static_cast<long>(max_pos), static_cast<long>(rows), static_cast<long>(D), pos0,
            alpha, index_type == GSVK_I32};
  const bool vec_ok = D % 8 == 0 && aligned16(table) && aligned16(pe) && aligned16(out) &&
                      (!mm || aligned16(mm)) && (!bias || aligned16(bias));
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case GSVK_F32: launch_embed_tab<GSVK_F32>(table_dtype, a, vec_ok, st); break;
    case GSVK_F16: launch_embed_tab<GSVK_F16>(table_dtype, a, vec_ok, st); break;
    default: launch_embed_tab<GSVK_BF16>(table_dtype, a, vec_ok, st); break;
  }
  return launch_status();
}

extern "C" int gsvk_t2s_prefill_input(int out_dtype, int table_dtype, int index_type,
                                      const void* text_table, size_t text_vocab,
                                      const void* phones, size_t T, const void* mm,
                                      const float* bias, float alpha_text,
                                      const void* audio_table, size_t audio_vocab,
                                      const void* prompt, size_t P, float alpha_audio,
                                      const float* pe, size_t max_pos, void* xy, size_t D,
                                      int32_t* err, void* stream) {
  if (!valid_dtype(out_dtype) || !valid_dtype(table_dtype)) return GSVK_E_DTYPE;
  if (index_type != GSVK_I64 && index_type != GSVK_I32) return GSVK_E_DTYPE;
  if (!text_table || !audio_table || !pe || !xy || (T && !phones) || (P && !prompt))
    return GSVK_E_NULL;
  // (positions <= 2^24: one wave each, so a launch stays under 2^32 work-items)
  if (T + P == 0 || D == 0 || text_vocab == 0 || audio_vocab == 0 || max_pos == 0 ||
      T > (1ul << 24) || P > (1ul << 24) || D > (1ul << 30) || text_vocab > (1ul << 40) ||
      audio_vocab > (1ul << 40) || max_pos > (1ul << 40))
    return GSVK_E_SIZE;
  if (D % 2) return GSVK_E_ARG;
  const size_t osz = dtype_size(out_dtype), tsz = dtype_size(table_dtype);
  const size_t isz = index_type == GSVK_I64 ? 8 : 4;
  const size_t obytes = (T + P) * D * osz, mbytes = T * D * osz;
  // mm is the text rows' bert_proj output: xy itself (the reference's order, in place) or apart
  if (mm && mm != xy && overlaps(xy, obytes, mm, mbytes)) return GSVK_E_ALIAS;
  if (overlaps(xy, obytes, text_table, text_vocab * D * tsz) ||
      overlaps(xy, obytes, audio_table, audio_vocab * D * tsz) ||
      overlaps(xy, obytes, phones, T * isz) || overlaps(xy, obytes, prompt, P * isz) ||
      overlaps(xy, obytes, pe, max_pos * D * 4) || overlaps(xy, obytes, bias, bias ? D * 4 : 0) ||
      overlaps(xy, obytes, err, err ? 4 : 0))
    return GSVK_E_ALIAS;
  const bool vec_ok = D % 8 == 0 && aligned16(text_table) && aligned16(audio_table) &&
                      aligned16(pe) && aligned16(xy) && (!mm || aligned16(mm)) &&
                      (!bias || aligned16(bias));
  if (!vec_ok || !T || !P) {  // the two gathers one after the other: the same results
    int rc = GSVK_OK;
    if (T)
      rc = gsvk_embed_pe(out_dtype, table_dtype, index_type, text_table, text_vocab, phones,
                         nullptr, 0, pe, max_pos, alpha_text, mm, bias, xy, T, D, err, stream);
    if (rc == GSVK_OK && P)
      rc = gsvk_embed_pe(out_dtype, table_dtype, index_type, audio_table, audio_vocab, prompt,
                         nullptr, 0, pe, max_pos, alpha_audio, nullptr, nullptr,
                         static_cast<char*>(xy) + T * D * osz, P, D, err, stream);
    return rc;
  }
  PfArgs a{text_table, audio_table, phones, prompt, mm, bias, pe, xy, err,
           static_cast<long>(T), static_cast<long>(P), static_cast<long>(D),
           static_cast<long>(text_vocab), static_cast<long>(audio_vocab),
           static_cast<long>(max_pos), alpha_text, alpha_audio, index_type == GSVK_I32};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case GSVK_F32: launch_prefill_tab<GSVK_F32>(table_dtype, a, st); break;
    case GSVK_F16: launch_prefill_tab<GSVK_F16>(table_dtype, a, st); break;
    default: launch_prefill_tab<GSVK_BF16>(table_dtype, a, st); break;
  }
  return launch_status();
}
