// t2s_decode_step.cpp — the epilogue chain of one T2S decode step over B sequences, issued through
// the C ABI and recorded into a HIP graph (one graph launch per step instead of 73 API launches).
#include <hip/hip_runtime.h>

#include <new>
#include <vector>

#include "gsvk.h"
#include "gsvk_t2s.h"

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

extern "C" int gsvk_t2s_step_create(const gsvk_t2s_step_desc* desc, gsvk_t2s_step** out) {
  if (!out) return GSVK_E_NULL;
  *out = nullptr;
  if (!desc_ok(desc)) return GSVK_E_NULL;
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
    rc = issue(desc, cap);
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
  s->launches = static_cast<int>(1 + 3 * desc->layers);
  *out = s;
  return GSVK_OK;
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
