// gsvk_step.hip — the epilogue chain of one T2S decode step as ONE launch (gfx950).
//
// The chain (include/gsvk_t2s.h; block_decode_impl, t2s_engine.cpp:1096-1119, and the decode input,
// 1866-1869) for B sequences is:
//   x = audio_emb[id] + alpha * pe[pos]
//   per layer l:  h = LN1((attn_out[l] + bout) + x);  ff[l] = relu(ff[l] + b1);
//                 x = LN2((ffn_out[l] + b2) + h)
// Every dependency of the LayerNorm chain stays inside one row: row b of layer l + 1 needs only row b
// of layer l. So wave b walks the whole chain of sequence b with its row in VGPRs (the gather, then
// 2 x layers LayerNorms), storing every h and x exactly as the per-op launches do, while the other
// waves of the same launch stream the ReLU tiles of all layers (they depend on nothing in the chain).
// No wave waits for another and there is no barrier: the 1 + 3 x layers launches of the graph form
// become one dispatch, and its duration is the chain's critical path (2 x layers dependent row
// reductions) instead of 73 launch latencies.
//
// The chain wave prefetches the next layers' inputs (attn_out / ffn_out rows and the six parameter
// vectors) three layers ahead into a register ring, so HBM latency is paid once, not per LayerNorm.
// Its row reductions are DPP only: no LDS round trip per LayerNorm.
//
// What bounds it: one wave issues at most one instruction per four cycles (a wave64 VALU op takes
// four passes of the 16-lane SIMD), and the chain wave issues ~5,400 of them (rocprofv3 counters:
// SQ_INSTS, SQ_INSTS_VALU, SQ_ACTIVE_INST_VALU per wave with the ReLU waves removed). So the chain
// is shortened by issuing fewer instructions, not by shorter dependences: the next LayerNorm's
// input + bias conversions fill the issue slots in which the DPP reduction steps would wait out
// their hazards (no s_nop there), fp16 halves are converted and added by v_fma_mix_f32 that the
// compiler sees (an opaque fp16 one as the multiplier: around inline asm the compiler adds wait
// states), and the lane's sum of squares is one fma chain.
//
// Numerics: each LayerNorm takes its statistics in one pass, as kern::layernorm does
// (kern.cpp:27-59: the row's sum and sum of squares, var = E[x^2] - mean^2, a centred second pass
// only where that comes out negative), so its two row reductions run together and the chain pays
// one reduction latency per LayerNorm. The per-op kernel (ln_rows_tile) takes exact two-pass
// statistics; the two forms agree within the LayerNorm tolerance, not bit for bit. The gather and
// the ReLU tiles are embed_pe_vec's and bias_act_tile's arithmetic (bit-exact), and each stored
// h / x is re-read as its rounded storage value (unpack of the packed store), so every LayerNorm
// sees exactly the residual the per-op form would read back.
#include <cmath>
#include <mutex>

#include "gsvk_common.hpp"
#include "gsvk_t2s.h"

namespace gsvk {
namespace {

constexpr int kMaxStepLayers = 32;  // the layer records travel in the kernel arguments
constexpr int kReluRows = 4;        // rows per ReLU wave (the bias chunk is reused across them)

struct StepLayer {
  const void* attn_out;
  const float* bout;
  const float* n1g;
  const float* n1b;
  void* ff;
  const float* b1;
  const void* ffn_out;
  const float* b2;
  const float* n2g;
  const float* n2b;
};

struct StepArgs {
  const void* table;
  const void* ids;
  const int64_t* pos;
  const float* pe;
  int32_t* err;
  void* x;
  void* h;
  long vocab, max_pos, B, D, FF;
  long relu_waves_per_layer;  // ceil(B / kReluRows) * ceil(FF chunks / 64)
  int relu_col_tiles;         // ceil(FF chunks / 64)
  double inv_n;               // 1 / D, computed on the host
  float inv_n_f;              // the same in fp32 (exact when D is a power of two)
  float eps;
  float alpha;
  int ids32;
  int tab_dt;
  int layers;
  StepLayer L[kMaxStepLayers];
};

// V consecutive elements of a row of storage type T at element index i, as fp32 (the table may have
// another storage type than the activations, so 8, 16 or 32 bytes).
template <int T, int V>
__device__ __forceinline__ void load_elems(const void* p, size_t i, float (&v)[V]) {
  if constexpr (T == GSVK_F32) {
#pragma unroll
    for (int k = 0; k < V; k += 4) {
      float q[4];
      Store<GSVK_F32>::load(p, i + k, q);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[k + j] = q[j];
    }
  } else if constexpr (V == 8) {
    Store<T>::load(p, i, v);
  } else {  // four 16-bit values: one 8-byte load
    const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    v[0] = Store<T>::up(w.x & 0xffffu);
    v[1] = Store<T>::up(w.x >> 16);
    v[2] = Store<T>::up(w.y & 0xffffu);
    v[3] = Store<T>::up(w.y >> 16);
  }
}

template <int V>
__device__ __forceinline__ void load_param(const float* p, size_t i, const float* fill,
                                           float (&v)[V]) {
  const float* q = param_or(p, i, fill);
#pragma unroll
  for (int k = 0; k < V; k += 4) load_f32x4(q, k, &v[k]);
}

// One layer's inputs for this lane's CPL chunks, in flight until the layer runs.
template <int DT, int CPL>
struct LayerIn {
  static constexpr int V = Store<DT>::VEC;
  u32x4 att[CPL], ffo[CPL];
  float bo[CPL][V], g1[CPL][V], be1[CPL][V], b2[CPL][V], g2[CPL][V], be2[CPL][V];
};

// Rows an absent parameter vector reads instead (d_model <= 1024 here). The host puts their
// device addresses into the layer records in place of null pointers, so the chain wave spends no
// instruction choosing between a given vector and these: each lane only adds its own 32-bit offset
// to the record's pointer (the scalar-base + 32-bit-offset address form).
static __device__ __attribute__((aligned(16))) float kRowZeros[1024] = {};
static __device__ __attribute__((aligned(16))) float kRowOnes[1024] = {[0 ... 1023] = 1.f};

template <int DT, int CPL>
__device__ __forceinline__ void load_layer(const StepLayer& L, size_t row_off,
                                           const uint32_t (&eo)[CPL], LayerIn<DT, CPL>& f) {
  constexpr uint32_t kEsz = DT == GSVK_F32 ? 4 : 2;
  const char* att = static_cast<const char*>(L.attn_out) + row_off * kEsz;  // wave-uniform
  const char* ffo = static_cast<const char*>(L.ffn_out) + row_off * kEsz;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    f.att[c] = ld16<false>(att + eo[c] * kEsz);
    f.ffo[c] = ld16<false>(ffo + eo[c] * kEsz);
  }
  const float *bo = L.bout, *g1 = L.n1g, *be1 = L.n1b, *b2 = L.b2, *g2 = L.n2g, *be2 = L.n2b;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
#pragma unroll
    for (int k = 0; k < Store<DT>::VEC; k += 4) {
      load_f32x4(bo + eo[c], k, &f.bo[c][k]);
      load_f32x4(g1 + eo[c], k, &f.g1[c][k]);
      load_f32x4(be1 + eo[c], k, &f.be1[c][k]);
      load_f32x4(b2 + eo[c], k, &f.b2[c][k]);
      load_f32x4(g2 + eo[c], k, &f.g2[c][k]);
      load_f32x4(be2 + eo[c], k, &f.be2[c][k]);
    }
  }
}

// The rounded value of a stored row chunk as the next LayerNorm reads it back: fp16 rows stay
// packed (the next residual add takes the halves directly), other types as fp32.
template <int DT, int CPL>
struct RowVal {
  float f[CPL][Store<DT>::VEC];
};
template <int CPL>
struct RowVal<GSVK_F16, CPL> {
  u32x4 p[CPL];
};

// float(half) + b with one rounding: v_fma_mix_f32 h, one, b, the half converted exactly and
// multiplied by one exactly (the same bits as the conversion and the add). `one` is an opaque fp16
// 1.0 in a VGPR: with a literal 1.0 the compiler folds the fma into a conversion and an add.
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
template <bool HI>
__device__ __forceinline__ float add_half(uint32_t w, float b, _Float16 one) {
  const h2v h = __builtin_bit_cast(h2v, w);
  return __builtin_fmaf(static_cast<float>(HI ? h.y : h.x), static_cast<float>(one), b);
}

// t = in + bias as fp32 (the first rounding of the reference's (in + bias) + res).
template <int DT>
__device__ __forceinline__ void add_bias(const u32x4& in, const float (&bias)[Store<DT>::VEC],
                                         float (&t)[Store<DT>::VEC], _Float16 one) {
  if constexpr (DT == GSVK_F16) {
    const uint32_t hw[4] = {in.x, in.y, in.z, in.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      t[2 * k] = add_half<false>(hw[k], bias[2 * k], one);
      t[2 * k + 1] = add_half<true>(hw[k], bias[2 * k + 1], one);
    }
  } else {
    Store<DT>::unpack(in, t);
#pragma unroll
    for (int k = 0; k < Store<DT>::VEC; ++k) t[k] = t[k] + bias[k];
  }
}

// y = LN(t + res), t = in + bias already rounded, over one row held by the wave: per-lane chunk
// trees of the values and of their squares added in chunk order, both wave sums at once,
// var = E[x^2] - mean^2 (the centred second moment where that is negative), rstd = rsq(var + eps),
// y = fmaf((v - mean) rstd, g, b). Stores y and returns its rounded storage value in `yr` (what the
// next LayerNorm reads back as its residual). The next LayerNorm's nt = nin + nbias (independent of
// this one) is computed between the steps of the wave reduction, in the issue slots the DPP reads
// would otherwise wait out.
template <int DT, int CPL, bool FULL>
__device__ __forceinline__ void ln_row(const StepArgs& a, const float (&t)[CPL][Store<DT>::VEC],
                                       const RowVal<DT, CPL>& res,
                                       const float (&g)[CPL][Store<DT>::VEC],
                                       const float (&b)[CPL][Store<DT>::VEC],
                                       const bool (&on)[CPL], void* y, size_t row_off,
                                       const uint32_t (&eo)[CPL], RowVal<DT, CPL>& yr,
                                       _Float16 one, const u32x4 (&nin)[CPL],
                                       const float (&nbias)[CPL][Store<DT>::VEC],
                                       float (&nt)[CPL][Store<DT>::VEC]) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  float v[CPL][V];
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    if (FULL || on[c]) {
      if constexpr (DT == GSVK_F16) {
        const uint32_t rw[4] = {res.p[c].x, res.p[c].y, res.p[c].z, res.p[c].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          v[c][2 * k] = add_half<false>(rw[k], t[c][2 * k], one);
          v[c][2 * k + 1] = add_half<true>(rw[k], t[c][2 * k + 1], one);
        }
      } else {
#pragma unroll
        for (int k = 0; k < V; ++k) v[c][k] = t[c][k] + res.f[c][k];
      }
      s = c == 0 ? chunk_sum(v[c]) : s + chunk_sum(v[c]);
    } else {
#pragma unroll
      for (int k = 0; k < V; ++k) v[c][k] = 0.f;
    }
  }
  // One pass, as kern::layernorm (kern.cpp:29-48): the row's sum and sum of squares are reduced
  // together (two interleaved DPP chains), then var = E[x^2] - mean^2, and only a row where that
  // comes out negative or NaN (cancellation) takes the second, centred pass (kern.cpp:49-56).
  // With FULL rows n = 64 * CPL * VEC is a power of two, so scaling by 1/n is exact in fp32 and
  // commutes with every rounding of the sums: the lane partials are scaled before the reduction,
  // and fmaf(-mean, mean, E[x^2]) rounds the exact difference once, as the reference's
  // float(double(sqsum) / n - double(mean)^2) does (mean^2 is exact in double).
  // The lane's sum of squares is one fma chain (V instructions; a tree takes V + V / 2 - 1): the
  // chain wave is bound by instruction issue, not by the depth of its dependences.
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c)
    if (FULL || on[c]) {
#pragma unroll
      for (int k = 0; k < V; ++k)
        q = (c == 0 && k == 0) ? v[c][k] * v[c][k] : __builtin_fmaf(v[c][k], v[c][k], q);
    }
  // the wave reduction (wave_sum2's steps) with nt computed in the issue slots between them
  float ra = FULL ? s * a.inv_n_f : s, rb = FULL ? q * a.inv_n_f : q;
  if constexpr (DT == GSVK_F16 && CPL == 1 && FULL) {
    // One block: two DPP chains of six steps (each DPP read two issue slots after the write of its
    // source, filled by the other chain's step and one conversion of nt) and the eight v_fma_mix
    // that form nt = float(nin) + nbias. Lane 63 ends with (r3 + r2) + (r1 + r0) of both values.
    float* o = nt[0];
    asm volatile(
        "v_fma_mix_f32 %2, %10, 1.0, %14 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mix_f32 %3, %10, 1.0, %15 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_add_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %1, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_fma_mix_f32 %4, %11, 1.0, %16 op_sel_hi:[1,0,0]\n\t"
        "v_add_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %1, %1, %1 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_fma_mix_f32 %5, %11, 1.0, %17 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_add_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %1, %1, %1 row_half_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_fma_mix_f32 %6, %12, 1.0, %18 op_sel_hi:[1,0,0]\n\t"
        "v_add_f32_dpp %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %1, %1, %1 row_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_fma_mix_f32 %7, %12, 1.0, %19 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_add_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %1, %1, %1 row_bcast:15 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_fma_mix_f32 %8, %13, 1.0, %20 op_sel_hi:[1,0,0]\n\t"
        "v_add_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_add_f32_dpp %1, %1, %1 row_bcast:31 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "v_fma_mix_f32 %9, %13, 1.0, %21 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "s_nop 1"
        : "+v"(ra), "+v"(rb), "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]),
          "=&v"(o[5]), "=&v"(o[6]), "=&v"(o[7])
        : "v"(nin[0].x), "v"(nin[0].y), "v"(nin[0].z), "v"(nin[0].w), "v"(nbias[0][0]),
          "v"(nbias[0][1]), "v"(nbias[0][2]), "v"(nbias[0][3]), "v"(nbias[0][4]), "v"(nbias[0][5]),
          "v"(nbias[0][6]), "v"(nbias[0][7]));
  } else {
#pragma unroll
    for (int c = 0; c < CPL; ++c) add_bias<DT>(nin[c], nbias[c], nt[c], one);
    ra += dpp_f32<0xB1>(ra);
    rb += dpp_f32<0xB1>(rb);
    ra += dpp_f32<0x4E>(ra);
    rb += dpp_f32<0x4E>(rb);
    ra += dpp_f32<0x141>(ra);
    rb += dpp_f32<0x141>(rb);
    ra += dpp_f32<0x140>(ra);
    rb += dpp_f32<0x140>(rb);
    ra += dpp_f32<0x142>(ra);
    rb += dpp_f32<0x142>(rb);
    ra += dpp_f32<0x143>(ra);
    rb += dpp_f32<0x143>(rb);
  }
  const float SA = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ra), 63));
  const float SB = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, rb), 63));
  float mean, var;
  if constexpr (FULL) {
    mean = SA;
    var = __builtin_fmaf(-mean, mean, SB);
  } else {
    mean = static_cast<float>(static_cast<double>(SA) * a.inv_n);
    const double m = mean;
    var = static_cast<float>(static_cast<double>(SB) * a.inv_n - m * m);
  }
  if (!(var >= 0.f)) {  // wave-uniform
    float m2 = mean;
    asm volatile("" : "+v"(m2));
    float q2 = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      if (FULL || on[c]) q2 = c == 0 ? chunk_sumsq(v[c], m2) : q2 + chunk_sumsq(v[c], m2);
    var = FULL ? wave_sum(q2 * a.inv_n_f)
               : static_cast<float>(static_cast<double>(wave_sum(q2)) * a.inv_n);
  }
  const float rstd = __builtin_amdgcn_rsqf(var + a.eps);
  constexpr uint32_t kEsz = DT == GSVK_F32 ? 4 : 2;
  char* yrow = static_cast<char*>(y) + row_off * kEsz;  // wave-uniform
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    float o[V];
#pragma unroll
    for (int k = 0; k < V; ++k) o[k] = __builtin_fmaf((v[c][k] - mean) * rstd, g[c][k], b[c][k]);
    const u32x4 packed = S::pack(o);
    if (FULL || on[c]) st16<false>(yrow + eo[c] * kEsz, packed);
    if constexpr (DT == GSVK_F16) yr.p[c] = packed;
    else S::unpack(packed, yr.f[c]);
  }
}

// The chain of sequence b: gather + alpha*PE, then LN1 / LN2 of every layer. FULL: every lane
// holds CPL whole chunks (D = 64 * CPL * VEC), so no store needs a guard.
//
// The layer loop runs in threes with no condition inside: layer l sits in ring slot l % 3 and the
// slot is refilled with layer l + 3 (clamped to the last layer: an in-bounds reread whose values
// are never used) right after it runs. With no branch between the loads and their uses, the
// compiler's wait before each layer covers only that layer's loads (the other slots' loads stay in
// flight); the last L mod 3 layers run after the loop from slots 0 and 1.
template <int DT, int CPL, bool FULL>
__device__ __forceinline__ void chain_row(const StepArgs& a, long b) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  const int lane = threadIdx.x;
  const int nch = static_cast<int>(a.D / V);
  uint32_t eo[CPL];  // element offset of the lane's chunk c within a row
  bool on[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int i = lane + c * kWave;
    on[c] = FULL || i < nch;
    // clamped: loads stay unconditional, stores are guarded
    eo[c] = static_cast<uint32_t>(on[c] ? i : nch - 1) * V;
  }
  const size_t row_off = static_cast<size_t>(b) * static_cast<size_t>(a.D);

  // Decode input (embed_pe_vec's arithmetic): x = fmaf(alpha, pe[pos], e[id]). Both index words are
  // read unconditionally (int32 ids read word b twice) so no branch separates the loads.
  const uint32_t* idw = static_cast<const uint32_t*>(a.ids);
  const size_t w0 = a.ids32 ? static_cast<size_t>(b) : 2 * static_cast<size_t>(b);
  const uint32_t id_lo = idw[w0], id_hi = idw[a.ids32 ? w0 : w0 + 1];
  const int64_t p = a.pos[b];

  // Layers 0, 1 and 2 are in flight while the gather resolves its id.
  const int L = a.layers;
  LayerIn<DT, CPL> f[3];
  load_layer<DT, CPL>(a.L[0], row_off, eo, f[0]);
  load_layer<DT, CPL>(a.L[L > 1 ? 1 : 0], row_off, eo, f[1]);
  load_layer<DT, CPL>(a.L[L > 2 ? 2 : L - 1], row_off, eo, f[2]);

  const int64_t id = a.ids32 ? static_cast<int64_t>(static_cast<int32_t>(id_lo))
                             : static_cast<int64_t>((static_cast<uint64_t>(id_hi) << 32) | id_lo);
  const bool ok = id >= 0 && id < a.vocab && p >= 0 && p < a.max_pos;
  const size_t trow = static_cast<size_t>(ok ? id : 0) * static_cast<size_t>(a.D);
  const size_t prow = static_cast<size_t>(ok ? p : 0) * static_cast<size_t>(a.D);
  RowVal<DT, CPL> xr;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const size_t i = eo[c];
    float e[V], pe[V], o[V];
    switch (a.tab_dt) {  // wave-uniform
      case GSVK_F32: load_elems<GSVK_F32, V>(a.table, trow + i, e); break;
      case GSVK_F16: load_elems<GSVK_F16, V>(a.table, trow + i, e); break;
      default: load_elems<GSVK_BF16, V>(a.table, trow + i, e); break;
    }
    load_elems<GSVK_F32, V>(a.pe, prow + i, pe);
#pragma unroll
    for (int k = 0; k < V; ++k) o[k] = ok ? __builtin_fmaf(a.alpha, pe[k], e[k]) : __builtin_nanf("");
    const u32x4 packed = S::pack(o);
    if (FULL || on[c])
      st16<false>(static_cast<char*>(a.x) + (row_off + i) * (DT == GSVK_F32 ? 4 : 2), packed);
    if constexpr (DT == GSVK_F16) xr.p[c] = packed;
    else S::unpack(packed, xr.f[c]);
  }
  if (!ok && lane == 0 && a.err) *a.err = 1;

  RowVal<DT, CPL> hr;
  _Float16 one = static_cast<_Float16>(1.f);
  asm volatile("" : "+v"(one));
  float t[CPL][V], nt[CPL][V];
#pragma unroll
  for (int c = 0; c < CPL; ++c) add_bias<DT>(f[0].att[c], f[0].bo[c], t[c], one);
  // fn: the ring slot of the next layer (its attention row + bias is the next LN1's input)
  auto layer = [&](LayerIn<DT, CPL>& fi, LayerIn<DT, CPL>& fn) {
    ln_row<DT, CPL, FULL>(a, t, xr, fi.g1, fi.be1, on, a.h, row_off, eo, hr, one, fi.ffo, fi.b2, nt);
    ln_row<DT, CPL, FULL>(a, nt, hr, fi.g2, fi.be2, on, a.x, row_off, eo, xr, one, fn.att, fn.bo, t);
  };
  // sched_barrier(0) keeps the scheduler from hoisting the next layer's arithmetic (and so its
  // loads' waits) into the current layer's reductions: measured, that put a wait on loads issued
  // half a layer earlier into every LayerNorm.
  // The layer records (ten pointers each, in the kernel arguments) are read into registers one
  // layer before the refill that uses them: a record read right before its loads put a scalar-load
  // round trip (the kernel-argument lines miss the scalar cache) in front of every refill.
  StepLayer rec = a.L[L > 3 ? 3 : L - 1];
  auto refill = [&](LayerIn<DT, CPL>& fi, int l) {
    __builtin_amdgcn_sched_barrier(0);
    load_layer<DT, CPL>(rec, row_off, eo, fi);
    rec = a.L[l + 1 < L ? l + 1 : L - 1];
    __builtin_amdgcn_sched_barrier(0);
  };
  int l = 0;
  for (; l + 2 < L; l += 3) {
    layer(f[0], f[1]);
    refill(f[0], l + 3);
    layer(f[1], f[2]);
    refill(f[1], l + 4);
    layer(f[2], f[0]);
    refill(f[2], l + 5);
  }
  // the last 1 or 2 layers (L mod 3), already in slots 0 and 1
  if (l < L) layer(f[0], f[1]);
  if (l + 1 < L) layer(f[1], f[2]);
}

// ReLU wave w of the launch: layer w / waves_per_layer, rows r0 .. r0 + kReluRows - 1, one column
// tile of 64 chunks. bias_act_tile's arithmetic: relu(x + b1) in place.
template <int DT>
__device__ __forceinline__ void relu_tile(const StepArgs& a, long w) {
  using S = Store<DT>;
  constexpr int V = S::VEC;
  const long l = w / a.relu_waves_per_layer;
  const long rem = w - l * a.relu_waves_per_layer;
  const long rg = rem / a.relu_col_tiles, ct = rem - rg * a.relu_col_tiles;
  const long nch = a.FF / V;
  const long c = ct * kWave + threadIdx.x;
  if (c >= nch) return;
  const StepLayer& L = a.L[l];
  float bi[V];
  load_param(L.b1, static_cast<size_t>(c) * V, kZeros8, bi);
  const long r0 = rg * kReluRows;
  float v[kReluRows][V];
#pragma unroll
  for (int u = 0; u < kReluRows; ++u) {
    const long r = r0 + u < a.B ? r0 + u : a.B - 1;
    S::load(L.ff, static_cast<size_t>(r) * a.FF + c * V, v[u]);
  }
#pragma unroll
  for (int u = 0; u < kReluRows; ++u) {
    if (r0 + u < a.B) {
#pragma unroll
      for (int k = 0; k < V; ++k) v[u][k] = relu_ref(v[u][k] + bi[k]);
      S::store(L.ff, static_cast<size_t>(r0 + u) * a.FF + c * V, v[u]);
    }
  }
}

// Workgroups 0 .. B-1 (dispatched first) run the chains at raised wave priority, so a ReLU wave
// sharing their SIMD does not delay the critical path; the rest run the ReLU tiles.
template <int DT, int CPL, bool FULL>
__global__ __launch_bounds__(kWave) void t2s_step_fused(StepArgs a) {
  const long blk = blockIdx.x;
  if (blk < a.B) {
    __builtin_amdgcn_s_setprio(3);
    chain_row<DT, CPL, FULL>(a, blk);
  } else {
    relu_tile<DT>(a, blk - a.B);
  }
}

template <int DT>
int launch_step(const StepArgs& a, hipStream_t st) {
  constexpr int V = Store<DT>::VEC;
  const long nch = a.D / V;
  const unsigned grid = static_cast<unsigned>(a.B + a.layers * a.relu_waves_per_layer);
  if (nch == kWave)
    hipLaunchKernelGGL((t2s_step_fused<DT, 1, true>), dim3(grid), dim3(kWave), 0, st, a);
  else if (nch < kWave)
    hipLaunchKernelGGL((t2s_step_fused<DT, 1, false>), dim3(grid), dim3(kWave), 0, st, a);
  else if (nch == 2 * kWave)
    hipLaunchKernelGGL((t2s_step_fused<DT, 2, true>), dim3(grid), dim3(kWave), 0, st, a);
  else
    hipLaunchKernelGGL((t2s_step_fused<DT, 2, false>), dim3(grid), dim3(kWave), 0, st, a);
  return launch_status();
}

bool a16(const void* p) { return !p || aligned16(p); }

}  // namespace

// Device addresses of kRowZeros / kRowOnes on the current device, looked up once per device (with
// that device current) and kept until the process ends. In host code the arrays' names are only
// stand-ins for the symbols: the layer records get these addresses. False when the lookup fails.
__attribute__((visibility("hidden"))) bool step_fill_rows(const float** zeros, const float** ones) {
  static std::mutex mu;
  static const float* z[kMaxDevices] = {};
  static const float* o[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lock(mu);
  if (!z[dev]) {
    void *pz = nullptr, *po = nullptr;
    if (hipGetSymbolAddress(&pz, HIP_SYMBOL(kRowZeros)) != hipSuccess || !pz ||
        hipGetSymbolAddress(&po, HIP_SYMBOL(kRowOnes)) != hipSuccess || !po)
      return false;
    z[dev] = static_cast<const float*>(pz);
    o[dev] = static_cast<const float*>(po);
  }
  *zeros = z[dev];
  *ones = o[dev];
  return true;
}

}  // namespace gsvk

using namespace gsvk;

namespace gsvk {
namespace {

// Validation of a descriptor, then its launch arguments in `a` (GSVK_OK) or the status.
int build_step_args(const gsvk_t2s_step_desc* d, StepArgs& a) {
  if (!d || !d->x || !d->h || !d->attn_out || !d->ff || !d->ffn_out || !d->audio_table ||
      !d->ids || !d->pos || !d->pe)
    return GSVK_E_NULL;
  if (!valid_dtype(d->dtype) || !valid_dtype(d->table_dtype)) return GSVK_E_DTYPE;
  if (d->index_type != GSVK_I64 && d->index_type != GSVK_I32) return GSVK_E_DTYPE;
  if (d->batch == 0 || d->d_model == 0 || d->ffn == 0 || d->layers == 0 || d->vocab == 0 ||
      d->max_pos == 0)
    return GSVK_E_SIZE;
  if (d->layers > static_cast<size_t>(kMaxStepLayers) || d->batch > (1ul << 20) ||
      d->ffn > (1ul << 24) || d->vocab > (1ul << 40) || d->max_pos > (1ul << 40))
    return GSVK_E_SIZE;
  if (!(d->eps >= 0.0) || !std::isfinite(d->eps)) return GSVK_E_ARG;
  const size_t V = d->dtype == GSVK_F32 ? 4 : 8;
  // one wave holds a row: at most 2 chunks per lane (more would spill the prefetch ring); rows of
  // whole 16-byte chunks
  if (d->d_model % V || d->d_model / V > 2 * kWave || d->ffn % V) return GSVK_E_ARG;
  for (size_t l = 0; l < d->layers; ++l)
    if (!d->attn_out[l] || !d->ff[l] || !d->ffn_out[l]) return GSVK_E_NULL;

  const size_t esz = dtype_size(d->dtype), B = d->batch, D = d->d_model, FF = d->ffn;
  const size_t row_b = B * D * esz, ff_b = B * FF * esz, pb = D * 4;
  // alignment: 16-byte rows everywhere (the per-op launches would take their vector paths)
  bool al = a16(d->x) && a16(d->h) && a16(d->audio_table) && a16(d->pe);
  auto at = [](const float* const* arr, size_t l) { return arr ? arr[l] : nullptr; };
  for (size_t l = 0; l < d->layers && al; ++l)
    al = a16(d->attn_out[l]) && a16(d->ff[l]) && a16(d->ffn_out[l]) && a16(at(d->bout, l)) &&
         a16(at(d->n1g, l)) && a16(at(d->n1b, l)) && a16(at(d->b1, l)) && a16(at(d->b2, l)) &&
         a16(at(d->n2g, l)) && a16(at(d->n2b, l));
  if (!al) return GSVK_E_ARG;
  // x and h are written by the chain and read by nothing else; each ff[l] is read and written in
  // place by its own tiles only.
  if (overlaps(d->x, row_b, d->h, row_b)) return GSVK_E_ALIAS;
  const size_t isz = d->index_type == GSVK_I64 ? 8 : 4;
  for (void* out : {d->x, d->h}) {
    if (overlaps(out, row_b, d->audio_table, d->vocab * D * dtype_size(d->table_dtype)) ||
        overlaps(out, row_b, d->ids, B * isz) || overlaps(out, row_b, d->pos, B * 8) ||
        overlaps(out, row_b, d->pe, d->max_pos * D * 4) || overlaps(out, row_b, d->err, d->err ? 4 : 0))
      return GSVK_E_ALIAS;
    for (size_t l = 0; l < d->layers; ++l) {
      if (overlaps(out, row_b, d->attn_out[l], row_b) || overlaps(out, row_b, d->ffn_out[l], row_b) ||
          overlaps(out, row_b, d->ff[l], ff_b))
        return GSVK_E_ALIAS;
      for (const float* p : {at(d->bout, l), at(d->n1g, l), at(d->n1b, l), at(d->b2, l),
                             at(d->n2g, l), at(d->n2b, l)})
        if (overlaps(out, row_b, p, p ? pb : 0)) return GSVK_E_ALIAS;
    }
  }
  // The ReLU tiles write ff[l] while the chain waves read every other input, so ff[l] may overlap
  // nothing but itself.
  for (size_t l = 0; l < d->layers; ++l) {
    const void* ff = d->ff[l];
    if (overlaps(ff, ff_b, d->audio_table, d->vocab * D * dtype_size(d->table_dtype)) ||
        overlaps(ff, ff_b, d->ids, B * isz) || overlaps(ff, ff_b, d->pos, B * 8) ||
        overlaps(ff, ff_b, d->pe, d->max_pos * D * 4) || overlaps(ff, ff_b, d->err, d->err ? 4 : 0))
      return GSVK_E_ALIAS;
    for (size_t m = 0; m < d->layers; ++m) {
      if ((m != l && overlaps(ff, ff_b, d->ff[m], ff_b)) ||
          overlaps(ff, ff_b, d->attn_out[m], row_b) || overlaps(ff, ff_b, d->ffn_out[m], row_b) ||
          overlaps(ff, ff_b, at(d->b1, m), at(d->b1, m) ? FF * 4 : 0))
        return GSVK_E_ALIAS;
      for (const float* p : {at(d->bout, m), at(d->n1g, m), at(d->n1b, m), at(d->b2, m),
                             at(d->n2g, m), at(d->n2b, m)})
        if (overlaps(ff, ff_b, p, p ? pb : 0)) return GSVK_E_ALIAS;
    }
  }

  a = StepArgs{};
  a.table = d->audio_table;
  a.ids = d->ids;
  a.pos = d->pos;
  a.pe = d->pe;
  a.err = d->err;
  a.x = d->x;
  a.h = d->h;
  a.vocab = static_cast<long>(d->vocab);
  a.max_pos = static_cast<long>(d->max_pos);
  a.B = static_cast<long>(B);
  a.D = static_cast<long>(D);
  a.FF = static_cast<long>(FF);
  const long ff_nch = static_cast<long>(FF / V);
  a.relu_col_tiles = static_cast<int>((ff_nch + kWave - 1) / kWave);
  a.relu_waves_per_layer = ((a.B + kReluRows - 1) / kReluRows) * a.relu_col_tiles;
  a.inv_n = 1.0 / static_cast<double>(D);
  a.inv_n_f = static_cast<float>(a.inv_n);
  a.eps = static_cast<float>(d->eps);
  a.alpha = d->alpha;
  a.ids32 = d->index_type == GSVK_I32;
  a.tab_dt = d->table_dtype;
  a.layers = static_cast<int>(d->layers);
  // one-wave workgroups: the launch's work-items (64 per workgroup) must stay under 2^32
  if (static_cast<size_t>(a.B + a.layers * a.relu_waves_per_layer) >= (1ul << 26)) return GSVK_E_SIZE;
  const float *zeros = nullptr, *ones = nullptr;
  if (!step_fill_rows(&zeros, &ones)) return GSVK_E_HIP;
  auto or_fill = [](const float* p, const float* fill) { return p ? p : fill; };
  for (size_t l = 0; l < d->layers; ++l)
    a.L[l] = StepLayer{d->attn_out[l],
                       or_fill(at(d->bout, l), zeros),
                       or_fill(at(d->n1g, l), ones),
                       or_fill(at(d->n1b, l), zeros),
                       d->ff[l],
                       at(d->b1, l),
                       d->ffn_out[l],
                       or_fill(at(d->b2, l), zeros),
                       or_fill(at(d->n2g, l), ones),
                       or_fill(at(d->n2b, l), zeros)};
  return GSVK_OK;
}

// Everything a descriptor's validation and launch arguments depend on: its sizes, types and
// scalars, every pointer of it and of its per-layer arrays, and the current device (the filler
// rows' addresses are per device). False when it cannot be keyed (missing arrays, too many
// layers): the full validation then reports why.
constexpr int kKeyWords = 20 + 10 * kMaxStepLayers;
struct StepKey {
  uint64_t w[kKeyWords];
  int n = 0;
};

bool step_key(const gsvk_t2s_step_desc* d, int dev, StepKey& k) {
  if (!d || !d->attn_out || !d->ff || !d->ffn_out || d->layers == 0 ||
      d->layers > static_cast<size_t>(kMaxStepLayers))
    return false;
  auto u = [](const void* p) { return static_cast<uint64_t>(reinterpret_cast<uintptr_t>(p)); };
  auto at = [](const float* const* arr, size_t l) { return arr ? arr[l] : nullptr; };
  uint64_t eps_bits, alpha_bits = __builtin_bit_cast(uint32_t, d->alpha);
  static_assert(sizeof(d->eps) == 8, "eps is a double");
  __builtin_memcpy(&eps_bits, &d->eps, 8);
  const uint64_t head[20] = {static_cast<uint64_t>(d->dtype), static_cast<uint64_t>(d->table_dtype),
                             static_cast<uint64_t>(d->index_type), d->batch, d->d_model, d->ffn,
                             d->layers, d->vocab, d->max_pos, eps_bits, alpha_bits,
                             u(d->audio_table), u(d->ids), u(d->pos), u(d->pe), u(d->err), u(d->x),
                             u(d->h), static_cast<uint64_t>(dev), 0};
  int n = 0;
  for (uint64_t v : head) k.w[n++] = v;
  for (size_t l = 0; l < d->layers; ++l) {
    const void* const per[10] = {d->attn_out[l], at(d->bout, l), at(d->n1g, l), at(d->n1b, l),
                                 d->ff[l], at(d->b1, l), d->ffn_out[l], at(d->b2, l),
                                 at(d->n2g, l), at(d->n2b, l)};
    for (const void* p : per) k.w[n++] = u(p);
  }
  k.n = n;
  return true;
}

int launch_args(int dtype, const StepArgs& a, hipStream_t st) {
  switch (dtype) {
    case GSVK_F32: return launch_step<GSVK_F32>(a, st);
    case GSVK_F16: return launch_step<GSVK_F16>(a, st);
    default: return launch_step<GSVK_BF16>(a, st);
  }
}

}  // namespace
}  // namespace gsvk

// A decode loop launches the same descriptor every token: validating one of 24 layers checks a few
// thousand pairs of ranges for overlap (microseconds of host time per call), so each host thread
// keeps the launch arguments of the last descriptor it validated and reuses them when the next
// call's descriptor has exactly the same contents on the same device.
extern "C" int gsvk_t2s_step_fused(const gsvk_t2s_step_desc* d, void* stream) {
  thread_local StepKey last_key;
  thread_local StepArgs last_args;
  thread_local int last_dtype = -1;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  StepKey key;
  const bool keyed = step_key(d, dev, key);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (keyed && last_dtype >= 0 && key.n == last_key.n &&
      __builtin_memcmp(key.w, last_key.w, sizeof(uint64_t) * key.n) == 0)
    return launch_args(last_dtype, last_args, st);
  StepArgs a;
  const int rc = build_step_args(d, a);
  if (rc != GSVK_OK) return rc;
  if (keyed) {
    last_key = key;
    last_args = a;
    last_dtype = d->dtype;
  }
  return launch_args(d->dtype, a, st);
}
