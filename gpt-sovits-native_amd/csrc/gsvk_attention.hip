// gsvk_attention.hip — T2S decode attention for B sequences at once: append the new token's k / v
// to each sequence's KV cache and attend the single query over all cached keys, per head.
//
// The scan over the cache is HBM-bound (2 * len * D cache elements per sequence and step), so the
// layout decides the speed. The cache is token-major as the reference keeps it (row k holds all H
// heads: cache[k * D + h * HD + e]), so a wave reads one whole key row per load instruction: lane l
// holds dims 8l .. 8l+7, HD / 8 lanes make one head, D / 8 <= 64 lanes make the row. Per key a lane
// forms its 8-term partial dot, the HD / 8 lanes of a head add theirs with xor shuffles, and every
// lane keeps its head's online-softmax state (running max m, sum l, output o[8]).
//
// Keys are split into C chunks per sequence (grid.x), each chunk over the 4 waves of a workgroup
// (key k0 + w + 4 j for wave w). The wave states are merged in wave order through LDS; with C > 1
// each chunk writes its (m, l, o) to a workspace and a second kernel merges the chunks in chunk
// order and divides by l. Softmax is formed as exp(s - m) against running maxima and rescaled
// (exp(m_old - m_new)), which equals the reference's exp(s - max) / sum up to fp32 rounding.
#include <cmath>

#include "gsvk_common.hpp"

namespace gsvk {
namespace {

constexpr int kAttnWaves = 4;
#ifndef GSVK_ATTN_KPG
#define GSVK_ATTN_KPG 2
#endif
#ifndef GSVK_ATTN_DEPTH
#define GSVK_ATTN_DEPTH 2
#endif
constexpr int kKeysPerGroup = GSVK_ATTN_KPG;  // keys per wave per pipeline step
constexpr int kDepth = GSVK_ATTN_DEPTH;        // groups of loads in flight per wave
constexpr int kMaxChunks = 16;
// A call whose cache rows (K and V) reach this size reads them with the non-temporal hint. Across
// a decode step the layers' caches stream through the 256 MB MALL once each, so at this size per
// layer (24 layers: > 384 MB) nothing read this way is found there again; the hint keeps the MALL for
// the weights and activations that are. Measured on the whole T2S decode step (B = 64, 1024 keys,
// 134 MB per layer): 1198 -> 1122 us.
constexpr size_t kAttnStreamBytes = 16ul << 20;

struct AttnArgs {
  const float* qkv;  // [B, ldq]: q | k | v, fp32
  void* kc;          // [B, max_len, D]
  void* vc;
  const int64_t* pos;
  void* out;         // [B, ldo]
  float4* part;      // [B, C, 3, 64] float4: o[0:4], o[4:8], (m, l, 0, 0)
  int32_t* err;
  long ldq, ldo, max_len, D, HD;
  float scale;
};

// 8 consecutive elements at element index i (two 16-byte stores for fp32, one for 16-bit).
template <int DT>
__device__ __forceinline__ void store8(void* base, size_t i, const float (&v)[8]) {
  if constexpr (DT == GSVK_F32) {
    const float a[4] = {v[0], v[1], v[2], v[3]}, b[4] = {v[4], v[5], v[6], v[7]};
    Store<GSVK_F32>::store<false>(base, i, a);
    Store<GSVK_F32>::store<false>(base, i + 4, b);
  } else {
    Store<DT>::template store<false>(base, i, v);
  }
}

template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == GSVK_F32) return x;
  else if constexpr (DT == GSVK_F16) return h2f(f2h(x));
  else return bf2f(f2bf(x));
}

// Raw cache data of one pipeline step (kKeysPerGroup keys, K and V), converted when used so the
// loads are never waited for early.
template <int DT>
struct KeyGroup {
  static constexpr int W = DT == GSVK_F32 ? 2 : 1;  // 16-byte words per 8 elements
  u32x4 k[kKeysPerGroup][W];
  u32x4 v[kKeysPerGroup][W];
};

template <int DT>
__device__ __forceinline__ void unpack8(const u32x4 (&w)[KeyGroup<DT>::W], float (&f)[8]) {
  if constexpr (DT == GSVK_F32) {
    // Store<F32>::unpack copies the vector lanes out before the bit cast (a bit cast of an
    // ext_vector element directly is miscompiled as element 0).
    float lo[4], hi[4];
    Store<GSVK_F32>::unpack(w[0], lo);
    Store<GSVK_F32>::unpack(w[1], hi);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[i] = lo[i];
      f[4 + i] = hi[i];
    }
  } else {
    Store<DT>::unpack(w[0], f);
  }
}

// Sum over the lpd lanes of a head (lpd a power of two, groups aligned). Head widths of up to 4
// lanes (HD <= 32) use DPP quad permutes; wider heads add xor shuffles.
__device__ __forceinline__ float head_sum(float s, int lpd) {
  if (lpd >= 2)
    s += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, s),
                                                            0xB1, 0xF, 0xF, true));  // [1,0,3,2]
  if (lpd >= 4)
    s += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, s),
                                                            0x4E, 0xF, 0xF, true));  // [2,3,0,1]
  for (int off = 4; off < lpd; off <<= 1) s += __shfl_xor(s, off, kWave);
  return s;
}

// exp(a - b) for a running maximum b; 0 when a is -inf (also when both are -inf). The hardware
// exponential (v_exp_f32 on (a - b) log2 e) is within a few ulp plus |a - b| 2^-24 relative, far
// inside this path's 1e-5 tolerance.
__device__ __forceinline__ float exp_rel(float a, float b) {
  return a == -INFINITY ? 0.f : __expf(a - b);
}

template <int KVT, int OUTT, bool NT>
__global__ __launch_bounds__(kWave * kAttnWaves) void attn_chunk(AttnArgs a) {
  __shared__ float st_m[kAttnWaves][kWave], st_l[kAttnWaves][kWave];
  __shared__ float st_o[kAttnWaves][8][kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const long b = blockIdx.y, c = blockIdx.x, C = gridDim.x;
  const long D = a.D;
  const int lpd = static_cast<int>(a.HD / 8);
  const bool lane_on = 8 * lane < D;
  const size_t col = static_cast<size_t>(lane_on ? 8 * lane : 0);

  const int64_t pos = a.pos[b];
  const bool valid = pos >= 0 && pos < a.max_len;
  const long len = valid ? pos + 1 : 0;
  const long chunk = (len + C - 1) / C;
  const long k0 = min(len, c * chunk), k1 = min(len, k0 + chunk);

  // query (fp32) and the new key / value rounded to the cache type, as the append stores them
  const float* qrow = a.qkv + b * a.ldq;
  float q[8], kn[8], vn[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    q[i] = qrow[col + i];
    kn[i] = round_to<KVT>(qrow[D + col + i]);
    vn[i] = round_to<KVT>(qrow[2 * D + col + i]);
  }
  const size_t seq = static_cast<size_t>(b) * a.max_len * D;
  if (valid && wave == 0 && lane_on && k0 <= pos && pos < k1) {
    // The append: only this chunk covers pos, and it uses kn / vn for that key instead of reading
    // the cache back, so no other workgroup depends on these stores.
    store8<KVT>(a.kc, seq + static_cast<size_t>(pos) * D + col, kn);
    store8<KVT>(a.vc, seq + static_cast<size_t>(pos) * D + col, vn);
  }
  if (!valid && c == 0 && wave == 0 && lane == 0 && a.err) *a.err = 1;

  float m = -INFINITY, l = 0.f, o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = 0.f;

  // This wave's keys: k0 + wave + 4 j. Groups of kKeysPerGroup, kDepth groups of loads in flight.
  const long nk = k1 > k0 + wave ? (k1 - k0 - wave + kAttnWaves - 1) / kAttnWaves : 0;
  const long ng = (nk + kKeysPerGroup - 1) / kKeysPerGroup;
  auto key_of = [&](long g, int u) { return k0 + wave + kAttnWaves * (g * kKeysPerGroup + u); };
  constexpr size_t kEsz = KVT == GSVK_F32 ? 4 : 2;
  auto load = [&](KeyGroup<KVT>& f, long g) {
#pragma unroll
    for (int u = 0; u < kKeysPerGroup; ++u) {
      const size_t byte = (seq + static_cast<size_t>(min(key_of(g, u), k1 - 1)) * D + col) * kEsz;
#pragma unroll
      for (int w = 0; w < KeyGroup<KVT>::W; ++w) {
        f.k[u][w] = ld16<NT>(static_cast<const char*>(a.kc) + byte + 16 * w);
        f.v[u][w] = ld16<NT>(static_cast<const char*>(a.vc) + byte + 16 * w);
      }
    }
  };
  auto step = [&](const KeyGroup<KVT>& f, long g) {
    float s[kKeysPerGroup];
    float vr[kKeysPerGroup][8];
    float mb = -INFINITY;
#pragma unroll
    for (int u = 0; u < kKeysPerGroup; ++u) {
      const long k = key_of(g, u);
      float kr[8];
      unpack8<KVT>(f.k[u], kr);
      unpack8<KVT>(f.v[u], vr[u]);
      if (k == pos) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          kr[i] = kn[i];
          vr[u][i] = vn[i];
        }
      }
      // A padded slot (k >= k1) re-read row k1 - 1, which in the chunk holding pos is the row
      // the append is writing: possibly stale bits, Inf or NaN. Its score is -inf (p = 0), and
      // its values are zeroed too, since 0 * Inf / NaN would poison o.
      if (k >= k1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) vr[u][i] = 0.f;
      }
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) d = __builtin_fmaf(q[i], kr[i], d);
      d = head_sum(d, lpd) * a.scale;
      s[u] = k < k1 ? d : -INFINITY;
      mb = fmaxf(mb, s[u]);
    }
    const float mn = fmaxf(m, mb);
    const float corr = exp_rel(m, mn);
    l *= corr;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] *= corr;
#pragma unroll
    for (int u = 0; u < kKeysPerGroup; ++u) {
      const float p = exp_rel(s[u], mn);
      l += p;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = __builtin_fmaf(p, vr[u][i], o[i]);
    }
    m = mn;
  };
  if (ng > 0) {
    // Group g sits in f[g % kDepth]; its reload (group g + kDepth, clamped: an in-bounds reread
    // past the end) is issued right after it is used, so the loads stay unconditional.
    KeyGroup<KVT> f[kDepth];
#pragma unroll
    for (int s = 0; s < kDepth; ++s) load(f[s], min(static_cast<long>(s), ng - 1));
    for (long g = 0; g < ng; g += kDepth) {
#pragma unroll
      for (int s = 0; s < kDepth; ++s) {
        if (g + s < ng) step(f[s], g + s);
        load(f[s], min(g + s + kDepth, ng - 1));
      }
    }
  }

  // merge the four waves (wave order), then finish or publish the chunk
  st_m[wave][lane] = m;
  st_l[wave][lane] = l;
#pragma unroll
  for (int i = 0; i < 8; ++i) st_o[wave][i][lane] = o[i];
  __syncthreads();
  if (wave != 0) return;
  float M = st_m[0][lane];
#pragma unroll
  for (int w = 1; w < kAttnWaves; ++w) M = fmaxf(M, st_m[w][lane]);
  float L = 0.f, O[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) O[i] = 0.f;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) {
    const float f = exp_rel(st_m[w][lane], M);
    L = __builtin_fmaf(st_l[w][lane], f, L);
#pragma unroll
    for (int i = 0; i < 8; ++i) O[i] = __builtin_fmaf(st_o[w][i][lane], f, O[i]);
  }
  if (C == 1) {
    if (!lane_on) return;
    float y[8];
    const float inv = 1.f / L;  // L = 0 only for an invalid position: NaN row
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = L > 0.f ? O[i] * inv : __builtin_nanf("");
    store8<OUTT>(a.out, static_cast<size_t>(b) * a.ldo + col, y);
    return;
  }
  float4* p = a.part + (static_cast<size_t>(b) * C + c) * 3 * kWave;
  p[lane] = float4{O[0], O[1], O[2], O[3]};
  p[kWave + lane] = float4{O[4], O[5], O[6], O[7]};
  p[2 * kWave + lane] = float4{M, L, 0.f, 0.f};
}

// Merge the C chunk states of one sequence and divide by the softmax sum. One wave per chunk
// loads that chunk's (m, l, o) (all C loads in flight at once); wave 0 merges them in chunk order.
template <int OUTT>
__global__ __launch_bounds__(kWave * kMaxChunks) void attn_merge(AttnArgs a, int C) {
  __shared__ float sm[kMaxChunks][kWave], sl[kMaxChunks][kWave];
  __shared__ float so[kMaxChunks][8][kWave];
  const int lane = threadIdx.x & (kWave - 1), c = threadIdx.x / kWave;
  const long b = blockIdx.x;
  const float4* p = a.part + static_cast<size_t>(b) * C * 3 * kWave;
  if (c < C) {
    const float4 lo = p[(c * 3 + 0) * kWave + lane], hi = p[(c * 3 + 1) * kWave + lane];
    const float4 ml = p[(c * 3 + 2) * kWave + lane];
    sm[c][lane] = ml.x;
    sl[c][lane] = ml.y;
    so[c][0][lane] = lo.x;
    so[c][1][lane] = lo.y;
    so[c][2][lane] = lo.z;
    so[c][3][lane] = lo.w;
    so[c][4][lane] = hi.x;
    so[c][5][lane] = hi.y;
    so[c][6][lane] = hi.z;
    so[c][7][lane] = hi.w;
  }
  __syncthreads();
  if (c != 0 || 8 * lane >= a.D) return;
  float M = -INFINITY;
  for (int k = 0; k < C; ++k) M = fmaxf(M, sm[k][lane]);
  float L = 0.f, O[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) O[i] = 0.f;
  for (int k = 0; k < C; ++k) {
    const float f = exp_rel(sm[k][lane], M);
    L = __builtin_fmaf(sl[k][lane], f, L);
#pragma unroll
    for (int i = 0; i < 8; ++i) O[i] = __builtin_fmaf(so[k][i][lane], f, O[i]);
  }
  float y[8];
  const float inv = 1.f / L;
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = L > 0.f ? O[i] * inv : __builtin_nanf("");
  store8<OUTT>(a.out, static_cast<size_t>(b) * a.ldo + 8 * lane, y);
}

// Key chunks per sequence: one round of at most one workgroup per CU, 4 chunks at B = 64 on 256
// CUs. The workgroups of a launch stream their keys in step, so a partly filled last round costs a
// whole one. Measured on the whole T2S decode step (B = 64, 1024 and 2048 cached keys, non-temporal
// cache reads): 4 chunks ran 2.3% faster than 8 (two full rounds, twice the merge reads) and 5-6%
// faster than 6 (a half-full second round); 9 chunks were slower than 8 and 16 slower again.
// Contexts up to 256 keys take one chunk per 128 keys, and no chunk is shorter than 64 keys.
int chunks_for(size_t batch, size_t len_bound) {
  const long lb = static_cast<long>(len_bound), B = static_cast<long>(batch);
  long c;
  if (lb <= 256) {
    c = (lb + 127) / 128;
  } else {
    c = device_cus() / B;
    c = std::min(c, (lb + 63) / 64);
  }
  return static_cast<int>(std::max(1L, std::min<long>(c, kMaxChunks)));
}

template <int KVT, int OUTT>
void launch_attn(const AttnArgs& a, size_t B, int C, bool nt, hipStream_t st) {
  const dim3 grid(C, static_cast<unsigned>(B));
  if (nt)
    hipLaunchKernelGGL((attn_chunk<KVT, OUTT, true>), grid, dim3(kWave * kAttnWaves), 0, st, a);
  else
    hipLaunchKernelGGL((attn_chunk<KVT, OUTT, false>), grid, dim3(kWave * kAttnWaves), 0, st, a);
  if (C > 1)
    hipLaunchKernelGGL((attn_merge<OUTT>), dim3(static_cast<unsigned>(B)), dim3(kWave * C), 0, st,
                       a, C);
}

template <int KVT>
void launch_out(int outt, const AttnArgs& a, size_t B, int C, bool nt, hipStream_t st) {
  switch (outt) {
    case GSVK_F32: return launch_attn<KVT, GSVK_F32>(a, B, C, nt, st);
    case GSVK_F16: return launch_attn<KVT, GSVK_F16>(a, B, C, nt, st);
    default: return launch_attn<KVT, GSVK_BF16>(a, B, C, nt, st);
  }
}

size_t part_bytes(size_t B, int C) { return C > 1 ? B * C * 3 * kWave * 16 : 0; }

}  // namespace
}  // namespace gsvk

using namespace gsvk;

extern "C" size_t gsvk_decode_attention_workspace_bytes(size_t batch, size_t heads,
                                                        size_t head_dim, size_t len_bound) {
  (void)heads;
  (void)head_dim;
  if (batch == 0) return 0;
  if (len_bound) return part_bytes(batch, chunks_for(batch, len_bound));
  // len_bound 0: the launch then uses max_len, which this query does not see, so size for the
  // most chunks any context takes. Short contexts (<= 256 keys) take one chunk per 128 keys
  // whatever the batch; longer ones at most CUs / batch. With more sequences than half the CUs
  // the short form takes more chunks than the long one (B = 200 on 256 CUs: 2 against 1).
  return std::max(part_bytes(batch, chunks_for(batch, 256)),
                  part_bytes(batch, chunks_for(batch, 1ul << 31)));
}

namespace gsvk {

// The whole call after the workspace decision. need_ws: the caller's workspace must hold the
// chunk states (the no-allocation form); otherwise a missing or short workspace means one chunk.
__attribute__((visibility("hidden"))) int attention_call(
                   int kv_dtype, int out_dtype, const float* qkv, size_t ldq, void* k_cache,
                   void* v_cache, size_t max_len, const int64_t* pos, void* out, size_t ldo,
                   size_t batch, size_t heads, size_t head_dim, size_t len_bound, void* workspace,
                   size_t workspace_bytes, bool need_ws, int32_t* err, void* stream) {
  if (!valid_dtype(kv_dtype) || !valid_dtype(out_dtype)) return GSVK_E_DTYPE;
  if (!qkv || !k_cache || !v_cache || !pos || !out) return GSVK_E_NULL;
  const size_t D = heads * head_dim;
  if (batch == 0 || heads == 0 || head_dim == 0 || max_len == 0 || batch > 65535 ||
      max_len > (1ul << 31))
    return GSVK_E_SIZE;
  // one wave holds a key row: 8 dims per lane, D <= 512; a head spans a power-of-two lane count
  if (D > 512 || head_dim % 8 || (head_dim / 8 & (head_dim / 8 - 1))) return GSVK_E_ARG;
  if (ldq < 3 * D || ldo < D) return GSVK_E_SIZE;
  const size_t esz = dtype_size(kv_dtype), cache_bytes = batch * max_len * D * esz;
  const size_t obytes = span_bytes(batch, D, ldo, dtype_size(out_dtype));
  if (overlaps(k_cache, cache_bytes, v_cache, cache_bytes) ||
      overlaps(k_cache, cache_bytes, qkv, span_bytes(batch, 3 * D, ldq, 4)) ||
      overlaps(v_cache, cache_bytes, qkv, span_bytes(batch, 3 * D, ldq, 4)) ||
      overlaps(out, obytes, qkv, span_bytes(batch, 3 * D, ldq, 4)) ||
      overlaps(out, obytes, k_cache, cache_bytes) || overlaps(out, obytes, v_cache, cache_bytes))
    return GSVK_E_ALIAS;
  if (!aligned16(qkv) || !aligned16(k_cache) || !aligned16(v_cache) || ldq % 4 ||
      (out_dtype == GSVK_F32 ? ldo % 4 : ldo % 8) || !aligned16(out))
    return GSVK_E_ARG;

  int C = chunks_for(batch, len_bound ? len_bound : max_len);
  if (need_ws && part_bytes(batch, C) > workspace_bytes) return GSVK_E_SIZE;
  if (C > 1 && (!workspace || workspace_bytes < part_bytes(batch, C) || !aligned16(workspace)))
    C = 1;  // without the workspace every sequence runs as one chunk
  if (C > 1 && (overlaps(workspace, part_bytes(batch, C), out, obytes) ||
                overlaps(workspace, part_bytes(batch, C), k_cache, cache_bytes) ||
                overlaps(workspace, part_bytes(batch, C), v_cache, cache_bytes)))
    return GSVK_E_ALIAS;
  AttnArgs a{qkv, k_cache, v_cache, pos, out, static_cast<float4*>(workspace), err,
             static_cast<long>(ldq), static_cast<long>(ldo), static_cast<long>(max_len),
             static_cast<long>(D), static_cast<long>(head_dim),
             1.0f / std::sqrt(static_cast<float>(head_dim))};
  hipStream_t st = static_cast<hipStream_t>(stream);
  // cache rows this call reads: K and V of up to len_bound (else max_len) keys per sequence
  const size_t keys = len_bound ? std::min(len_bound, max_len) : max_len;
  const bool nt = 2 * batch * keys * D * esz >= kAttnStreamBytes;
  switch (kv_dtype) {
    case GSVK_F32: launch_out<GSVK_F32>(out_dtype, a, batch, C, nt, st); break;
    case GSVK_F16: launch_out<GSVK_F16>(out_dtype, a, batch, C, nt, st); break;
    default: launch_out<GSVK_BF16>(out_dtype, a, batch, C, nt, st); break;
  }
  return launch_status();
}

}  // namespace gsvk

extern "C" int gsvk_decode_attention(int kv_dtype, int out_dtype, const float* qkv, size_t ldq,
                                     void* k_cache, void* v_cache, size_t max_len,
                                     const int64_t* pos, void* out, size_t ldo, size_t batch,
                                     size_t heads, size_t head_dim, size_t len_bound,
                                     void* workspace, size_t workspace_bytes, int32_t* err,
                                     void* stream) {
  return attention_call(kv_dtype, out_dtype, qkv, ldq, k_cache, v_cache, max_len, pos, out, ldo,
                        batch, heads, head_dim, len_bound, workspace, workspace_bytes, false, err,
                        stream);
}

