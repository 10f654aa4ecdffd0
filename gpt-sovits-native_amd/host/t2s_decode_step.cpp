// t2s_decode_step.cpp — one T2S decode step over B sequences, issued through the C ABI and recorded
// into a HIP graph (one graph launch per step): the epilogue chain alone (gsvk_t2s_step_*) and the
// whole step with its GEMVs and attention (gsvk_t2s_decode_*).
#include <hip/hip_runtime.h>

#include <new>
#include <type_traits>
#include <vector>

#include "gsvk.h"
#include "gsvk_t2s.h"

namespace gsvk {
// csrc/gsvk_step.hip: the device addresses the fused step's launch puts in place of absent
// parameter vectors, looked up once per device.
bool step_fill_rows(const float** zeros, const float** ones);
}  // namespace gsvk

namespace {

bool desc_ok(const gsvk_t2s_step_desc* d) {
  if (!d || !d->x || !d->h || !d->attn_out || !d->ff || !d->ffn_out) return false;
  if (d->batch == 0 || d->d_model == 0 || d->ffn == 0 || d->layers == 0) return false;
  for (size_t l = 0; l < d->layers; ++l)
    if (!d->attn_out[l] || !d->ff[l] || !d->ffn_out[l]) return false;
  return true;
}

int issue(const gsvk_t2s_step_desc* d, void* st) {
  const size_t B = d->batch, D = d->d_model, FF = d->ffn;
  int rc = gsvk_embed_pe(d->dtype, d->table_dtype, d->index_type, d->audio_table, d->vocab, d->ids,
                         d->pos, 0, d->pe, d->max_pos, d->alpha, nullptr, nullptr, d->x, B, D,
                         d->err, st);
  if (rc) return rc;
  auto at = [](const float* const* arr, size_t l) { return arr ? arr[l] : nullptr; };
  for (size_t l = 0; l < d->layers; ++l) {
    rc = gsvk_add_layernorm(d->dtype, d->attn_out[l], at(d->bout, l), d->x, at(d->n1g, l),
                            at(d->n1b, l), d->h, B, D, D, d->eps, st);
    if (rc) return rc;
    rc = gsvk_bias_act(d->dtype, GSVK_ACT_RELU, d->ff[l], at(d->b1, l), d->ff[l], B, FF, FF, 0.f,
                       st);
    if (rc) return rc;
    rc = gsvk_add_layernorm(d->dtype, d->ffn_out[l], at(d->b2, l), d->h, at(d->n2g, l),
                            at(d->n2b, l), d->x, B, D, D, d->eps, st);
    if (rc) return rc;
  }
  return GSVK_OK;
}

bool decode_ok(const gsvk_t2s_decode_desc* d) {
  if (!d || !d->layer || !d->x || !d->h || !d->z || !d->attn || !d->ff || !d->qkv || !d->kv_pos)
    return false;
  if (d->batch == 0 || d->d_model == 0 || d->heads == 0 || d->ffn == 0 || d->layers == 0)
    return false;
  if (d->w_logits && !d->logits) return false;
  for (size_t l = 0; l < d->layers; ++l) {
    const gsvk_t2s_layer& L = d->layer[l];
    if (!L.wqkv || !L.wout || !L.w1 || !L.w2 || !L.k_cache || !L.v_cache) return false;
  }
  return true;
}

size_t storage_bytes(int dt) { return dt == GSVK_F32 ? 4 : 2; }

template <class T>
T* advance(T* p, size_t bytes) {
  using B = typename std::conditional<std::is_const<T>::value, const char, char>::type;
  return p ? reinterpret_cast<T*>(reinterpret_cast<B*>(p) + bytes) : nullptr;
}

// One decode step for the rows [b0, b0 + n) of the batch, launch by launch, in block_decode_impl's
// order. Every launch is row-local (each GEMV row, each sequence's attention and cache rows), so a
// part of the batch runs exactly as the whole would for those rows; ws is the part's slice of the
// attention workspace.
int issue_rows(const gsvk_t2s_decode_desc* d, size_t b0, size_t n, void* ws, size_t ws_bytes,
               void* st) {
  const size_t B = n, D = d->d_model, FF = d->ffn, H = d->heads;
  const int dt = d->dtype;
  const size_t esz = storage_bytes(dt), kesz = storage_bytes(d->kv_dtype);
  const size_t isz = d->index_type == GSVK_I32 ? 4 : 8;
  void* const x = advance(d->x, b0 * D * esz);
  void* const h = advance(d->h, b0 * D * esz);
  void* const z = advance(d->z, b0 * D * esz);
  void* const attn = advance(d->attn, b0 * D * esz);
  void* const ff = advance(d->ff, b0 * FF * esz);
  float* const qkv = d->qkv + b0 * 3 * D;
  float* const logits = d->logits ? d->logits + b0 * d->vocab : nullptr;
  const int64_t* const kv_pos = d->kv_pos + b0;
  const size_t cache_off = b0 * d->max_len * D * kesz;
  int rc = GSVK_OK;
  // without a position array row r takes position r: the part's rows start at b0
  if ((rc = gsvk_embed_pe(dt, d->table_dtype, d->index_type, d->audio_table, d->vocab,
                          advance(d->ids, b0 * isz), d->pos ? d->pos + b0 : nullptr,
                          d->pos ? 0 : static_cast<int64_t>(b0), d->pe, d->max_pos, d->alpha,
                          nullptr, nullptr, x, B, D, d->err, st)))
    return rc;
  // Each post-LN is folded into the GEMV that reads its output (gsvk_gemv_f16w_ln): norm1 into
  // W1, norm2 into the next layer's QKV or, after the last layer, the logits.
  for (size_t l = 0; l < d->layers; ++l) {
    const gsvk_t2s_layer& L = d->layer[l];
    if (l == 0) {
      rc = gsvk_gemv_f16w(dt, 1, x, D, L.wqkv, L.bqkv, GSVK_ACT_NONE, 0.f, nullptr, GSVK_F32,
                          qkv, 3 * D, B, 3 * D, D, st);
    } else {  // x = norm2_{l-1}(z), qkv = W_qkv x + b  (t2s_engine.cpp:1119, 1044-1049)
      const gsvk_t2s_layer& P = d->layer[l - 1];
      rc = gsvk_gemv_f16w_ln(dt, 1, z, D, P.n2g, P.n2b, d->eps, x, D, L.wqkv, L.bqkv,
                             GSVK_ACT_NONE, 0.f, nullptr, GSVK_F32, qkv, 3 * D, B, 3 * D, D, st);
    }
    if (rc) return rc;
    if ((rc = gsvk_decode_attention(d->kv_dtype, dt, qkv, 3 * D,
                                    advance(L.k_cache, cache_off),
                                    advance(L.v_cache, cache_off), d->max_len, kv_pos, attn, D,
                                    B, H, D / H, d->len_bound, ws, ws_bytes, d->err, st)))
      return rc;
    if ((rc = gsvk_gemv_f16w(dt, 1, attn, D, L.wout, L.bout, GSVK_ACT_NONE, 0.f, x, dt, z, D, B, D,
                             D, st)))
      return rc;
    // h = norm1(z), ff = relu(W1 h + b1)  (t2s_engine.cpp:1097, 1105-1112)
    if ((rc = gsvk_gemv_f16w_ln(dt, 1, z, D, L.n1g, L.n1b, d->eps, h, D, L.w1, L.b1,
                                GSVK_ACT_RELU, 0.f, nullptr, dt, ff, FF, B, FF, D, st)))
      return rc;
    if ((rc = gsvk_gemv_f16w(dt, 1, ff, FF, L.w2, L.b2, GSVK_ACT_NONE, 0.f, h, dt, z, D, B, D, FF,
                             st)))
      return rc;
  }
  const gsvk_t2s_layer& last = d->layer[d->layers - 1];
  if (d->w_logits)  // x = norm2(z), logits = W_logits x
    return gsvk_gemv_f16w_ln(dt, 1, z, D, last.n2g, last.n2b, d->eps, x, D, d->w_logits, nullptr,
                             GSVK_ACT_NONE, 0.f, nullptr, GSVK_F32, logits, d->vocab, B, d->vocab,
                             D, st);
  return gsvk_add_layernorm(dt, z, nullptr, nullptr, last.n2g, last.n2b, x, B, D, D, d->eps, st);
}

// The batch in two parts. At decode sizes every launch but the attention scan is bound by latency,
// not bandwidth, so the two parts' launch chains are recorded on two streams of one graph, which
// the runtime issues on two hardware queues and runs side by side. Measured on the whole step
// (B = 64, 24 layers): 1098 -> 1082-1092 us at 1024 cached keys and 1548-1555 -> 1457-1461 us at
// 2048. The gain is small because one part's chain alone takes 916-1049 us: the chain's launch
// latency, not its rows, sets the step time. Batches of fewer than kSplitRows sequences, and
// workspaces too small for both parts' attention states, run as one part.
constexpr size_t kSplitRows = 32;
constexpr size_t kWsAlign = 256;

size_t attn_ws(const gsvk_t2s_decode_desc* d, size_t n) {
  return gsvk_decode_attention_workspace_bytes(n, d->heads, d->d_model / d->heads,
                                               d->len_bound ? d->len_bound : d->max_len);
}

struct Part {
  size_t b0, n;
  void* ws;
  size_t ws_bytes;
};

int parts_of(const gsvk_t2s_decode_desc* d, Part (&p)[2]) {
  const size_t B = d->batch;
  if (d->parts != 1 && B >= kSplitRows && d->workspace) {
    const size_t n0 = B / 2, n1 = B - n0;
    const size_t w0 = (attn_ws(d, n0) + kWsAlign - 1) / kWsAlign * kWsAlign, w1 = attn_ws(d, n1);
    if (d->workspace_bytes >= w0 + w1) {
      p[0] = Part{0, n0, d->workspace, w0};
      p[1] = Part{n0, n1, static_cast<char*>(d->workspace) + w0, w1};
      return 2;
    }
  }
  p[0] = Part{0, B, d->workspace, d->workspace_bytes};
  return 1;
}

// The parts one after another on one stream: the same launches as the graph records, so an eager
// step gives the graph's bits.
int issue_decode(const gsvk_t2s_decode_desc* d, void* st) {
  Part p[2];
  const int np = parts_of(d, p);
  for (int i = 0; i < np; ++i)
    if (int rc = issue_rows(d, p[i].b0, p[i].n, p[i].ws, p[i].ws_bytes, st)) return rc;
  return GSVK_OK;
}

int count_part_launches(const gsvk_t2s_decode_desc* d, const Part& p) {
  const size_t lb = d->len_bound ? d->len_bound : d->max_len;
  const size_t need = gsvk_decode_attention_workspace_bytes(p.n, d->heads, d->d_model / d->heads,
                                                            lb);
  const bool merge = need > 0 && p.ws && p.ws_bytes >= need;
  // gather; per layer QKV (+ norm2 of the layer before), attention (+ merge), out-proj,
  // W1 (+ norm1), W2; then the logits (+ the last norm2) or the last norm2 alone
  return static_cast<int>(1 + d->layers * (merge ? 6 : 5) + 1);
}

int count_decode_launches(const gsvk_t2s_decode_desc* d) {
  Part p[2];
  const int np = parts_of(d, p);
  int n = 0;
  for (int i = 0; i < np; ++i) n += count_part_launches(d, p[i]);
  return n;
}

}  // namespace

struct gsvk_t2s_step {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int launches = 0;
};

extern "C" int gsvk_t2s_step_eager(const gsvk_t2s_step_desc* desc, void* stream) {
  if (!desc_ok(desc)) return GSVK_E_NULL;
  return issue(desc, stream);
}

// Record the launches `issue` makes into a graph on a private stream and instantiate it.
// issue(cap, side, fork) may also launch on `side`, a second stream: fork() (at most once) makes
// everything issued on side from then on depend on what cap has issued so far, and side is joined
// back into cap at the end of the capture (graph branches that run concurrently).
template <class Issue>
int record2(Issue issue, int launches, gsvk_t2s_step** out) {
  hipStream_t cap = nullptr, side = nullptr;
  hipEvent_t fork_ev = nullptr, join_ev = nullptr;
  auto release = [&]() {
    if (fork_ev) (void)hipEventDestroy(fork_ev);
    if (join_ev) (void)hipEventDestroy(join_ev);
    if (side) (void)hipStreamDestroy(side);
    if (cap) (void)hipStreamDestroy(cap);
  };
  if (hipStreamCreateWithFlags(&cap, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&side, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&fork_ev, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&join_ev, hipEventDisableTiming) != hipSuccess) {
    release();
    return GSVK_E_HIP;
  }
  auto* s = new (std::nothrow) gsvk_t2s_step;
  if (!s) {
    release();
    return GSVK_E_HIP;
  }
  int rc = GSVK_OK;
  if (hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    rc = GSVK_E_HIP;
  } else {
    bool forked = false;
    auto fork = [&]() -> int {
      if (forked) return GSVK_OK;
      forked = true;
      return hipEventRecord(fork_ev, cap) == hipSuccess &&
                     hipStreamWaitEvent(side, fork_ev, 0) == hipSuccess
                 ? GSVK_OK
                 : GSVK_E_HIP;
    };
    rc = issue(cap, side, fork);
    // a forked side branch always joins back (also after an error), or the capture cannot end
    if (forked && (hipEventRecord(join_ev, side) != hipSuccess ||
                   hipStreamWaitEvent(cap, join_ev, 0) != hipSuccess) && rc == GSVK_OK)
      rc = GSVK_E_HIP;
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(cap, &g);
    if (rc == GSVK_OK && e != hipSuccess) rc = GSVK_E_HIP;
    s->graph = g;
  }
  if (rc == GSVK_OK && hipGraphInstantiate(&s->exec, s->graph, nullptr, nullptr, 0) != hipSuccess)
    rc = GSVK_E_HIP;
  release();
  if (rc != GSVK_OK) {
    gsvk_t2s_step_destroy(s);
    return rc;
  }
  s->launches = launches;
  *out = s;
  return GSVK_OK;
}

template <class Issue>
int record(Issue issue, int launches, gsvk_t2s_step** out) {
  return record2([&issue](hipStream_t cap, hipStream_t, auto&) { return issue(cap); }, launches,
                 out);
}

// The recorder with concurrent branches (the SoVITS decoder's ResBlocks): issue_fn(ctx, cap, side,
// fork, join) launches on cap and on the nside streams side[0 .. nside - 1]; it uses fork (to be
// recorded on cap) and join[i] (on side[i]) to make the side streams' work depend on cap's and
// cap's on theirs, and must join every side stream back into cap before it returns (also after an
// error), or the capture cannot end.
__attribute__((visibility("hidden"))) int gsvk_record_graph_branches_(
    int (*issue_fn)(const void*, hipStream_t, const hipStream_t*, hipEvent_t, const hipEvent_t*),
    const void* ctx, int nside, int launches, gsvk_t2s_step** out) {
  constexpr int kMaxSide = 4;
  if (!out) return GSVK_E_NULL;
  *out = nullptr;
  if (nside < 1 || nside > kMaxSide) return GSVK_E_ARG;
  hipStream_t cap = nullptr, side[kMaxSide] = {};
  hipEvent_t fork = nullptr, join[kMaxSide] = {};
  auto release = [&]() {
    if (fork) (void)hipEventDestroy(fork);
    for (int i = 0; i < nside; ++i) {
      if (join[i]) (void)hipEventDestroy(join[i]);
      if (side[i]) (void)hipStreamDestroy(side[i]);
    }
    if (cap) (void)hipStreamDestroy(cap);
  };
  bool ok = hipStreamCreateWithFlags(&cap, hipStreamNonBlocking) == hipSuccess &&
            hipEventCreateWithFlags(&fork, hipEventDisableTiming) == hipSuccess;
  for (int i = 0; ok && i < nside; ++i)
    ok = hipStreamCreateWithFlags(&side[i], hipStreamNonBlocking) == hipSuccess &&
         hipEventCreateWithFlags(&join[i], hipEventDisableTiming) == hipSuccess;
  auto* s = ok ? new (std::nothrow) gsvk_t2s_step : nullptr;
  if (!s) {
    release();
    return GSVK_E_HIP;
  }
  int rc = GSVK_OK;
  if (hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    rc = GSVK_E_HIP;
  } else {
    rc = issue_fn(ctx, cap, side, fork, join);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(cap, &g);
    if (rc == GSVK_OK && e != hipSuccess) rc = GSVK_E_HIP;
    s->graph = g;
  }
  if (rc == GSVK_OK && hipGraphInstantiate(&s->exec, s->graph, nullptr, nullptr, 0) != hipSuccess)
    rc = GSVK_E_HIP;
  release();
  if (rc != GSVK_OK) {
    gsvk_t2s_step_destroy(s);
    return rc;
  }
  s->launches = launches;
  *out = s;
  return GSVK_OK;
}

extern "C" int gsvk_t2s_step_create(const gsvk_t2s_step_desc* desc, gsvk_t2s_step** out) {
  if (!out) return GSVK_E_NULL;
  *out = nullptr;
  if (!desc_ok(desc)) return GSVK_E_NULL;
  return record([desc](hipStream_t st) { return issue(desc, st); },
                static_cast<int>(1 + 3 * desc->layers), out);
}

extern "C" int gsvk_t2s_step_create_fused(const gsvk_t2s_step_desc* desc, gsvk_t2s_step** out) {
  if (!out) return GSVK_E_NULL;
  *out = nullptr;
  if (!desc_ok(desc)) return GSVK_E_NULL;
  // the launch's device-address lookup runs here, before the capture, not inside it
  const float *zeros = nullptr, *ones = nullptr;
  if (!gsvk::step_fill_rows(&zeros, &ones)) return GSVK_E_HIP;
  // an unsupported shape fails inside the capture; record() then ends it and keeps no graph
  return record([desc](hipStream_t st) { return gsvk_t2s_step_fused(desc, st); }, 1, out);
}

extern "C" int gsvk_t2s_decode_eager(const gsvk_t2s_decode_desc* desc, void* stream) {
  if (!decode_ok(desc)) return GSVK_E_NULL;
  if (desc->parts != 0 && desc->parts != 1) return GSVK_E_ARG;
  return issue_decode(desc, stream);
}

extern "C" int gsvk_t2s_decode_create(const gsvk_t2s_decode_desc* desc, gsvk_t2s_step** out) {
  if (!out) return GSVK_E_NULL;
  *out = nullptr;
  if (!decode_ok(desc)) return GSVK_E_NULL;
  if (desc->parts != 0 && desc->parts != 1) return GSVK_E_ARG;
  return record2(
      [desc](hipStream_t cap, hipStream_t side, auto& fork) {
        Part p[2];
        const int np = parts_of(desc, p);
        if (np == 1) return issue_rows(desc, 0, p[0].n, p[0].ws, p[0].ws_bytes, cap);
        // (Starting the second half only after the first half's layer-0 attention, so that the
        // halves run half a layer apart, measured the same.)
        int rc = fork();
        if (rc == GSVK_OK) rc = issue_rows(desc, p[0].b0, p[0].n, p[0].ws, p[0].ws_bytes, cap);
        if (rc == GSVK_OK) rc = issue_rows(desc, p[1].b0, p[1].n, p[1].ws, p[1].ws_bytes, side);
        return rc;
      },
      count_decode_launches(desc), out);
}

extern "C" size_t gsvk_t2s_decode_workspace_bytes(size_t batch, size_t heads, size_t head_dim,
                                                  size_t len_bound) {
  if (batch == 0) return 0;
  const size_t whole = gsvk_decode_attention_workspace_bytes(batch, heads, head_dim, len_bound);
  if (batch < kSplitRows) return whole;
  const size_t n0 = batch / 2;
  const size_t w0 = gsvk_decode_attention_workspace_bytes(n0, heads, head_dim, len_bound);
  const size_t parts = (w0 + kWsAlign - 1) / kWsAlign * kWsAlign +
                       gsvk_decode_attention_workspace_bytes(batch - n0, heads, head_dim,
                                                             len_bound);
  return parts > whole ? parts : whole;
}

extern "C" int gsvk_t2s_step_run(gsvk_t2s_step* step, void* stream) {
  if (!step || !step->exec) return GSVK_E_NULL;
  return hipGraphLaunch(step->exec, static_cast<hipStream_t>(stream)) == hipSuccess ? GSVK_OK
                                                                                   : GSVK_E_HIP;
}

extern "C" int gsvk_t2s_step_launches(const gsvk_t2s_step* step) {
  return step ? step->launches : 0;
}

extern "C" void gsvk_t2s_step_destroy(gsvk_t2s_step* step) {
  if (!step) return;
  if (step->exec) (void)hipGraphExecDestroy(step->exec);
  if (step->graph) (void)hipGraphDestroy(step->graph);
  delete step;
}
