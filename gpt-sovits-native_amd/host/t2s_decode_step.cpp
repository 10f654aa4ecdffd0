// t2s_decode_step.cpp — one T2S decode step over B sequences, issued through the C ABI and recorded
// into a HIP graph (one graph launch per step): the epilogue chain alone (gsvk_t2s_step_*) and the
// whole step with its GEMVs and attention (gsvk_t2s_decode_*).
#include <hip/hip_runtime.h>

#include <new>
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

// One decode step, launch by launch, in block_decode_impl's order.
int issue_decode(const gsvk_t2s_decode_desc* d, void* st) {
  const size_t B = d->batch, D = d->d_model, FF = d->ffn, H = d->heads;
  const int dt = d->dtype;
  int rc = gsvk_embed_pe(dt, d->table_dtype, d->index_type, d->audio_table, d->vocab, d->ids,
                         d->pos, 0, d->pe, d->max_pos, d->alpha, nullptr, nullptr, d->x, B, D,
                         d->err, st);
  if (rc) return rc;
  // Each post-LN is folded into the GEMV that reads its output (gsvk_gemv_f16w_ln): norm1 into
  // W1, norm2 into the next layer's QKV or, after the last layer, the logits.
  for (size_t l = 0; l < d->layers; ++l) {
    const gsvk_t2s_layer& L = d->layer[l];
    if (l == 0) {
      rc = gsvk_gemv_f16w(dt, 1, d->x, D, L.wqkv, L.bqkv, GSVK_ACT_NONE, 0.f, nullptr, GSVK_F32,
                          d->qkv, 3 * D, B, 3 * D, D, st);
    } else {  // x = norm2_{l-1}(z), qkv = W_qkv x + b  (t2s_engine.cpp:1119, 1044-1049)
      const gsvk_t2s_layer& P = d->layer[l - 1];
      rc = gsvk_gemv_f16w_ln(dt, 1, d->z, D, P.n2g, P.n2b, d->eps, d->x, D, L.wqkv, L.bqkv,
                             GSVK_ACT_NONE, 0.f, nullptr, GSVK_F32, d->qkv, 3 * D, B, 3 * D, D, st);
    }
    if (rc) return rc;
    if ((rc = gsvk_decode_attention(d->kv_dtype, dt, d->qkv, 3 * D, L.k_cache, L.v_cache,
                                    d->max_len, d->kv_pos, d->attn, D, B, H, D / H, d->len_bound,
                                    d->workspace, d->workspace_bytes, d->err, st)))
      return rc;
    if ((rc = gsvk_gemv_f16w(dt, 1, d->attn, D, L.wout, L.bout, GSVK_ACT_NONE, 0.f, d->x, dt, d->z,
                             D, B, D, D, st)))
      return rc;
    // h = norm1(z), ff = relu(W1 h + b1)  (t2s_engine.cpp:1097, 1105-1112)
    if ((rc = gsvk_gemv_f16w_ln(dt, 1, d->z, D, L.n1g, L.n1b, d->eps, d->h, D, L.w1, L.b1,
                                GSVK_ACT_RELU, 0.f, nullptr, dt, d->ff, FF, B, FF, D, st)))
      return rc;
    if ((rc = gsvk_gemv_f16w(dt, 1, d->ff, FF, L.w2, L.b2, GSVK_ACT_NONE, 0.f, d->h, dt, d->z, D, B,
                             D, FF, st)))
      return rc;
  }
  const gsvk_t2s_layer& last = d->layer[d->layers - 1];
  if (d->w_logits)  // x = norm2(z), logits = W_logits x
    return gsvk_gemv_f16w_ln(dt, 1, d->z, D, last.n2g, last.n2b, d->eps, d->x, D, d->w_logits,
                             nullptr, GSVK_ACT_NONE, 0.f, nullptr, GSVK_F32, d->logits, d->vocab, B,
                             d->vocab, D, st);
  return gsvk_add_layernorm(dt, d->z, nullptr, nullptr, last.n2g, last.n2b, d->x, B, D, D, d->eps,
                            st);
}

int count_decode_launches(const gsvk_t2s_decode_desc* d) {
  const size_t lb = d->len_bound ? d->len_bound : d->max_len;
  const bool merge = gsvk_decode_attention_workspace_bytes(d->batch, d->heads,
                                                           d->d_model / d->heads, lb) > 0 &&
                     d->workspace &&
                     d->workspace_bytes >= gsvk_decode_attention_workspace_bytes(
                                               d->batch, d->heads, d->d_model / d->heads, lb);
  // gather; per layer QKV (+ norm2 of the layer before), attention (+ merge), out-proj,
  // W1 (+ norm1), W2; then the logits (+ the last norm2) or the last norm2 alone
  return static_cast<int>(1 + d->layers * (merge ? 6 : 5) + 1);
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
template <class Issue>
int record(Issue issue, int launches, gsvk_t2s_step** out) {
  hipStream_t cap = nullptr;
  if (hipStreamCreateWithFlags(&cap, hipStreamNonBlocking) != hipSuccess) return GSVK_E_HIP;
  auto* s = new (std::nothrow) gsvk_t2s_step;
  if (!s) {
    (void)hipStreamDestroy(cap);
    return GSVK_E_HIP;
  }
  int rc = GSVK_OK;
  if (hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    rc = GSVK_E_HIP;
  } else {
    rc = issue(cap);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(cap, &g);
    if (rc == GSVK_OK && e != hipSuccess) rc = GSVK_E_HIP;
    s->graph = g;
  }
  if (rc == GSVK_OK && hipGraphInstantiate(&s->exec, s->graph, nullptr, nullptr, 0) != hipSuccess)
    rc = GSVK_E_HIP;
  (void)hipStreamDestroy(cap);
  if (rc != GSVK_OK) {
    gsvk_t2s_step_destroy(s);
    return rc;
  }
  s->launches = launches;
  *out = s;
  return GSVK_OK;
}

// The recorder for other drivers of this library (the SoVITS decoder): issue_fn(ctx, stream)
// makes the launches.
__attribute__((visibility("hidden"))) int gsvk_record_graph_(
    int (*issue_fn)(const void*, hipStream_t), const void* ctx, int launches,
    gsvk_t2s_step** out) {
  if (!out) return GSVK_E_NULL;
  *out = nullptr;
  return record([issue_fn, ctx](hipStream_t st) { return issue_fn(ctx, st); }, launches, out);
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
  return issue_decode(desc, stream);
}

extern "C" int gsvk_t2s_decode_create(const gsvk_t2s_decode_desc* desc, gsvk_t2s_step** out) {
  if (!out) return GSVK_E_NULL;
  *out = nullptr;
  if (!decode_ok(desc)) return GSVK_E_NULL;
  return record(
      [desc](hipStream_t st) { return issue_decode(desc, st); }, count_decode_launches(desc), out);
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
