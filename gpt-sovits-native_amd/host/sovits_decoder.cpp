// sovits_decoder.cpp — the SoVITS decoder (Generator::forward, src/sovits/dec.hpp:264-345) issued
// through the C ABI as a fixed sequence of fused convolution launches, eager or recorded into a HIP
// graph (gsvk_sovits_decoder_*).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "gsvk.h"
#include "gsvk_sovits.h"

namespace {

constexpr size_t kAlign = 256;  // bytes: alignment of every workspace region

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Workspace layout: the folded bias (c0 floats), then 8 activation slots of `slot` elements of the
// activation dtype each: X (stage input, then the stage output), Y (upsampler output, the first
// residual), TA0..TA2 (each ResBlock's pair middle activation, so the three ResBlocks can run
// side by side) and CUR0..CUR2 (the three branch accumulators). The pairs' LeakyReLU inputs are
// not stored: the first conv of a pair reads lrelu(cur) as it loads (GSVK_CONV_X_LRELU).
enum Slot {
  kX,
  kY,
  kTa0,
  kCur0 = kTa0 + GSVK_SOVITS_RESBLOCKS,
  kSlots = kCur0 + GSVK_SOVITS_RESBLOCKS
};

// ResBlocks 1 and 2 of every stage run on two more streams, concurrent with ResBlock 0 on the main
// one (they share only the upsampler's output, which they read); the branch mean waits for all
// three. In a recorded graph the streams and events are the capture's; eagerly, the side streams
// are the device's own (below) and the events the call's.
constexpr int kSide = GSVK_SOVITS_RESBLOCKS - 1;
struct Branches {
  const hipStream_t* side;  // kSide streams
  hipEvent_t fork;
  const hipEvent_t* join;
};

struct Layout {
  size_t vec_bytes = 0;   // bytes of the folded bias (c0 floats, rounded up)
  size_t slot_bytes = 0;  // bytes of one activation slot
  size_t t_out = 0;       // samples of the output
  size_t bytes = 0;
};

// The shapes a valid descriptor must have (no buffer pointers needed) and the workspace layout.
int shapes(const gsvk_sovits_decoder_desc* d, Layout* lay) {
  if (!d || !d->stage) return GSVK_E_NULL;
  if (d->dtype != GSVK_F32 && d->dtype != GSVK_F16) return GSVK_E_DTYPE;
  if (d->frames == 0 || d->c_z == 0 || d->c0 == 0 || d->pre_k == 0 || d->post_k == 0 ||
      d->n_stages == 0 || d->n_stages > GSVK_SOVITS_MAX_STAGES)
    return GSVK_E_SIZE;
  size_t c = d->c0, T = d->frames, slot = d->c0 * d->frames;
  for (size_t s = 0; s < d->n_stages; ++s) {
    const gsvk_sovits_stage& S = d->stage[s];
    if (S.c_in != c || S.c_out == 0 || S.ups_k == 0 || S.ups_u == 0) return GSVK_E_SIZE;
    for (size_t j = 0; j < GSVK_SOVITS_RESBLOCKS; ++j)
      if (S.res_k[j] == 0) return GSVK_E_SIZE;
    for (size_t m = 0; m < GSVK_SOVITS_PAIRS; ++m)
      if (S.res_dil[m] == 0) return GSVK_E_SIZE;
    if (T > SIZE_MAX / S.ups_u) return GSVK_E_SIZE;
    c = S.c_out;
    T *= S.ups_u;
    if (T > SIZE_MAX / c) return GSVK_E_SIZE;
    if (c * T > slot) slot = c * T;
  }
  const size_t esz = d->dtype == GSVK_F32 ? 4 : 2;
  if (slot > (SIZE_MAX / 2) / esz / kSlots) return GSVK_E_SIZE;
  lay->vec_bytes = round_up(d->c0 * sizeof(float), kAlign);
  lay->slot_bytes = round_up(slot * esz, kAlign);
  lay->t_out = T;
  lay->bytes = lay->vec_bytes + kSlots * lay->slot_bytes;
  return GSVK_OK;
}

// Shapes, every weight and buffer pointer, and the workspace; the convolutions check the rest
// (aliasing, strides) themselves.
int check_workspace(const gsvk_sovits_decoder_desc* d, Layout* lay) {
  const int rc = shapes(d, lay);
  if (rc) return rc;
  if (!d->pre_w || !d->post_w || !d->z || !d->out) return GSVK_E_NULL;
  if (d->g_in && (!d->cond_w || !d->ge)) return GSVK_E_NULL;
  for (size_t s = 0; s < d->n_stages; ++s) {
    const gsvk_sovits_stage& S = d->stage[s];
    if (!S.ups_w) return GSVK_E_NULL;
    for (size_t j = 0; j < GSVK_SOVITS_RESBLOCKS; ++j)
      for (size_t m = 0; m < GSVK_SOVITS_PAIRS; ++m)
        if (!S.w1[j][m] || !S.w2[j][m]) return GSVK_E_NULL;
  }
  if (!d->workspace) return GSVK_E_NULL;
  if (reinterpret_cast<uintptr_t>(d->workspace) % 16 != 0) return GSVK_E_ARG;
  if (d->workspace_bytes < lay->bytes) return GSVK_E_SIZE;
  return GSVK_OK;
}

int count_launches(const gsvk_sovits_decoder_desc* d) {
  // cond with the bias fold (with conditioning), conv_pre, 20 per stage, conv_post
  return (d->g_in ? 1 : 0) + 1 + 20 * static_cast<int>(d->n_stages) + 1;
}

// The launches of one decoder pass in Generator::forward's order.
int issue(const gsvk_sovits_decoder_desc* d, const Layout& lay, void* st, const Branches* br) {
  const int dt = d->dtype, rx = d->round_x;
  const float slope = 0.1f;  // LRELU_SLOPE (dec.hpp:284, 322, 324)
  char* ws = static_cast<char*>(d->workspace);
  float* bias = reinterpret_cast<float*>(ws);
  void* slot[kSlots];
  for (int i = 0; i < kSlots; ++i)
    slot[i] = ws + lay.vec_bytes + static_cast<size_t>(i) * lay.slot_bytes;
  int rc = GSVK_OK;

  // x = lrelu(conv_pre(z) + b_pre + cond(ge)[:, 0], 0.1): the broadcast add of dec.hpp:275-279
  // folded into the bias, the stage-0 leaky_relu_io (dec.hpp:284) into the store. cond is a k = 1
  // convolution of one frame, i.e. a GEMV; b_pre enters as its residual, so one launch leaves
  // bias = (W_cond ge + b_cond) + b_pre in fp32.
  const float* pre_bias = d->pre_b;
  if (d->g_in) {
    if ((rc = gsvk_gemv_f16w(GSVK_F32, rx, d->ge, d->g_in, d->cond_w, d->cond_b, GSVK_ACT_NONE, 0.f,
                             d->pre_b, GSVK_F32, bias, d->c0, 1, d->c0, d->g_in, st)))
      return rc;
    pre_bias = bias;
  }
  size_t T = d->frames;
  if ((rc = gsvk_conv1d(dt, rx, d->z, T, d->pre_w, pre_bias, GSVK_CONV_EPI_LRELU, slope, nullptr,
                        nullptr, 0, slot[kX], T, d->c_z, d->c0, T, d->pre_k, 1, st)))
    return rc;

  for (size_t s = 0; s < d->n_stages; ++s) {
    const gsvk_sovits_stage& S = d->stage[s];
    const size_t C = S.c_out, Tu = T * S.ups_u;
    // y = ups(x)  (dec.hpp:285)
    if ((rc = gsvk_convt1d(dt, rx, slot[kX], T, S.ups_w, S.ups_b, GSVK_CONV_EPI_BIAS, 0.f, nullptr,
                           nullptr, 0, slot[kY], Tu, S.c_in, C, T, S.ups_k, S.ups_u, st)))
      return rc;
    T = Tu;
    if (br) {  // (a failed wait still reaches the joins below)
      if (hipEventRecord(br->fork, static_cast<hipStream_t>(st)) != hipSuccess) return GSVK_E_HIP;
      for (int i = 0; i < kSide; ++i)
        if (hipStreamWaitEvent(br->side[i], br->fork, 0) != hipSuccess) rc = GSVK_E_HIP;
    }
    const void* curs[GSVK_SOVITS_RESBLOCKS];
    for (size_t j = 0; j < GSVK_SOVITS_RESBLOCKS && rc == GSVK_OK; ++j) {
      void* bst = br && j > 0 ? br->side[j - 1] : st;
      void* cur = slot[kCur0 + j];
      void* ta = slot[kTa0 + j];
      curs[j] = cur;
      const void* src = slot[kY];  // cur_j starts as a copy of y (dec.hpp:316): read it in place
      const void* res = slot[kY];
      for (size_t m = 0; m < GSVK_SOVITS_PAIRS; ++m) {
        // t_a = lrelu(convs1[m](lrelu(cur_j)))  (dec.hpp:322-324: leaky_relu_write as the
        // convolution reads its input, leaky_relu_io in its store)
        if ((rc = gsvk_conv1d(dt, rx, src, T, S.w1[j][m], S.b1[j][m],
                              GSVK_CONV_EPI_LRELU | GSVK_CONV_X_LRELU, slope, nullptr, nullptr, 0,
                              ta, T, C, C, T, S.res_k[j], S.res_dil[m], bst)))
          break;
        // cur_j = res + convs2[m](t_a)  (dec.hpp:325-326)
        if ((rc = gsvk_conv1d(dt, rx, ta, T, S.w2[j][m], S.b2[j][m], GSVK_CONV_EPI_RES, slope, cur,
                              res, T, nullptr, T, C, C, T, S.res_k[j], 1, bst)))
          break;
        src = cur;
        res = nullptr;  // in place from the second pair on
      }
    }
    if (br)  // every side stream joins back, also after an error (a capture must end joined)
      for (int i = 0; i < kSide; ++i)
        if ((hipEventRecord(br->join[i], br->side[i]) != hipSuccess ||
             hipStreamWaitEvent(static_cast<hipStream_t>(st), br->join[i], 0) != hipSuccess) &&
            rc == GSVK_OK)
          rc = GSVK_E_HIP;
    if (rc) return rc;
    // x = lrelu(mean_j cur_j): mul_write / add_scaled_inplace (dec.hpp:328-333) with the next
    // stage's leaky_relu_io (dec.hpp:284, 0.1) or the final one (dec.hpp:342, 0.01).
    const float next_slope = s + 1 < d->n_stages ? slope : 0.01f;
    if ((rc = gsvk_resblock_branch_mean(dt, curs, nullptr, GSVK_SOVITS_RESBLOCKS, slot[kX], C * T,
                                        1, next_slope, st)))
      return rc;
  }
  // out = tanh(conv_post(x))  (dec.hpp:343-344; conv_post has no bias)
  return gsvk_conv1d(dt, rx, slot[kX], T, d->post_w, nullptr, GSVK_CONV_EPI_TANH, 0.f, nullptr,
                     nullptr, 0, d->out, T, d->stage[d->n_stages - 1].c_out, 1, T, d->post_k, 1,
                     st);
}

// The eager form's side streams: two per device, created on its first eager call and kept for the
// process (default priority, non-blocking). Calls that overlap on one device share them; each
// call's own events order its launches, so sharing only serializes the calls' side work.
constexpr int kMaxDevices = 64;
int device_side_streams(hipStream_t (&side)[kSide]) {
  static std::mutex mu;
  static hipStream_t streams[kMaxDevices][kSide];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return GSVK_E_HIP;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < kSide; ++i) {
    if (!streams[dev][i] &&
        hipStreamCreateWithFlags(&streams[dev][i], hipStreamNonBlocking) != hipSuccess) {
      streams[dev][i] = nullptr;
      return GSVK_E_HIP;
    }
    side[i] = streams[dev][i];
  }
  return GSVK_OK;
}

}  // namespace

// The graph handle and its recorder live in t2s_decode_step.cpp.
__attribute__((visibility("hidden"))) int gsvk_record_graph_branches_(
    int (*issue_fn)(const void*, hipStream_t, const hipStream_t*, hipEvent_t, const hipEvent_t*),
    const void* ctx, int nside, int launches, gsvk_t2s_step** out);

extern "C" size_t gsvk_sovits_decoder_workspace_bytes(const gsvk_sovits_decoder_desc* desc) {
  Layout lay;
  return shapes(desc, &lay) == GSVK_OK ? lay.bytes : 0;
}

extern "C" int gsvk_sovits_decoder_eager(const gsvk_sovits_decoder_desc* desc, void* stream) {
  Layout lay;
  int rc = check_workspace(desc, &lay);
  if (rc) return rc;
  hipStream_t side[kSide];
  hipEvent_t fork = nullptr, join[kSide] = {};
  rc = device_side_streams(side);
  if (rc == GSVK_OK && hipEventCreateWithFlags(&fork, hipEventDisableTiming) != hipSuccess)
    rc = GSVK_E_HIP;
  for (int i = 0; i < kSide && rc == GSVK_OK; ++i)
    if (hipEventCreateWithFlags(&join[i], hipEventDisableTiming) != hipSuccess) rc = GSVK_E_HIP;
  if (rc == GSVK_OK) {
    const Branches br{side, fork, join};
    rc = issue(desc, lay, stream, &br);
  }
  // (an event destroyed while its record is pending is released once that work completes)
  if (fork) (void)hipEventDestroy(fork);
  for (int i = 0; i < kSide; ++i)
    if (join[i]) (void)hipEventDestroy(join[i]);
  return rc;
}

extern "C" int gsvk_sovits_decoder_create(const gsvk_sovits_decoder_desc* desc,
                                          gsvk_t2s_step** out) {
  if (!out) return GSVK_E_NULL;
  *out = nullptr;
  Layout lay;
  const int rc = check_workspace(desc, &lay);
  if (rc) return rc;
  struct Ctx {
    const gsvk_sovits_decoder_desc* d;
    Layout lay;
  } ctx{desc, lay};
  return gsvk_record_graph_branches_(
      [](const void* c, hipStream_t st, const hipStream_t* side, hipEvent_t fork,
         const hipEvent_t* join) {
        const Ctx* x = static_cast<const Ctx*>(c);
        const Branches br{side, fork, join};
        return issue(x->d, x->lay, st, &br);
      },
      &ctx, GSVK_SOVITS_RESBLOCKS - 1, count_launches(desc), out);
}
