/*
 * gsvk_sovits.h — the SoVITS decoder (Generator::forward, src/sovits/dec.hpp:264-345) on the GPU as
 * one sequence of fused launches over caller-owned device buffers, eager or recorded into a HIP
 * graph. Every convolution is gsvk_conv1d / gsvk_convt1d (include/gsvk.h) with the element-wise
 * passes around it fused into its store:
 *
 *   bias = (W_cond ge + b_cond) + b_pre      cond (dec.hpp:271) as a GEMV of one  1 launch
 *                                            frame (gsvk_gemv_f16w), the broadcast add
 *                                            (dec.hpp:275-279) folded into its output
 *   x    = lrelu(conv_pre(z) + bias, 0.1)    (dec.hpp:268, 275-279, 284)          1 launch
 *   per stage s (dec.hpp:283-336):                                               20 launches
 *     y = ups(x)
 *     per ResBlock j, pair m: t_a = lrelu(convs1[m](lrelu(c))), c = m ? cur_j : y   (X_LRELU input,
 *                             LRELU epilogue); cur_j = c + convs2[m](t_a)           (RES epilogue)
 *     x = lrelu(sum_j cur_j * (1/3), s < last ? 0.1 : 0.01)             (branch mean, dec.hpp:342)
 *   out  = tanh(conv_post(x))                [1, T out]    (dec.hpp:343-344)       1 launch
 *
 * The folded broadcast rounds (W z + b_pre) + cv as W z + (b_pre + cv): within the convolution's
 * tolerance. Convolution weights are the packed forms (gsvk_conv1d_pack / gsvk_convt1d_pack of the
 * .gsv's fp16 [out, in, k] / [in, out, k] tensors); cond's is its fp16 [c0, g_in] matrix as stored
 * (the k = 1 weight, row-major, unpacked); biases fp32. Activations of `dtype` (F32, the reference's,
 * or F16 storage: every stored activation rounded to fp16, arithmetic in fp32); round_x as in
 * gsvk_conv1d (F32 only). ge and the folded bias are fp32 for either dtype.
 */
#ifndef GSVK_SOVITS_H
#define GSVK_SOVITS_H

#include <stddef.h>
#include <stdint.h>

#include "gsvk_t2s.h" /* gsvk_t2s_step: the recorded-graph handle (run / launches / destroy) */

#ifdef __cplusplus
extern "C" {
#endif

#define GSVK_SOVITS_MAX_STAGES 8
#define GSVK_SOVITS_RESBLOCKS 3 /* ResBlock1 per stage (dec.hpp:51-52) */
#define GSVK_SOVITS_PAIRS 3     /* conv pairs per ResBlock1 */

/* One Generator stage: the upsampler ups[i] (c_in -> c_out, kernel ups_k, stride ups_u) and the
 * three ResBlock1 resblocks[i][j] (kernel res_k[j]; convs1 dilations res_dil[m], convs2 dilation 1). */
typedef struct gsvk_sovits_stage {
  size_t c_in, c_out, ups_k, ups_u;
  const uint16_t* ups_w; /* packed transposed weights */
  const float* ups_b;
  size_t res_k[GSVK_SOVITS_RESBLOCKS];
  size_t res_dil[GSVK_SOVITS_PAIRS];
  const uint16_t* w1[GSVK_SOVITS_RESBLOCKS][GSVK_SOVITS_PAIRS]; /* packed convs1 */
  const float* b1[GSVK_SOVITS_RESBLOCKS][GSVK_SOVITS_PAIRS];
  const uint16_t* w2[GSVK_SOVITS_RESBLOCKS][GSVK_SOVITS_PAIRS]; /* packed convs2 */
  const float* b2[GSVK_SOVITS_RESBLOCKS][GSVK_SOVITS_PAIRS];
} gsvk_sovits_stage;

typedef struct gsvk_sovits_decoder_desc {
  int dtype;   /* GSVK_F32 or GSVK_F16 activations */
  int round_x; /* 1: fp32 activations rounded to fp16 in the convolutions (the AMX path) */
  size_t frames, c_z, c0; /* z [c_z, frames] -> conv_pre -> [c0, frames] */
  size_t pre_k;
  const uint16_t* pre_w; /* packed conv_pre */
  const float* pre_b;    /* may be NULL */
  size_t g_in;           /* cond input channels; 0: no conditioning */
  const uint16_t* cond_w; /* cond's fp16 [c0, g_in] weight matrix (not packed) */
  const float* cond_b;
  size_t n_stages;
  const gsvk_sovits_stage* stage;
  size_t post_k;
  const uint16_t* post_w; /* packed conv_post (c_out of the last stage -> 1, no bias) */
  const void* z;  /* [c_z, frames], dtype */
  const void* ge; /* [g_in] fp32 (column 0 of the reference's ge); NULL when g_in == 0 */
  void* out;      /* [frames * prod(ups_u)], dtype */
  void* workspace; /* gsvk_sovits_decoder_workspace_bytes(desc) bytes, 16-byte aligned */
  size_t workspace_bytes;
} gsvk_sovits_decoder_desc;

/* Workspace bytes the decoder needs for the descriptor's shapes (its buffer and weight pointers may
 * still be NULL); 0 on invalid shapes. Host only. */
size_t gsvk_sovits_decoder_workspace_bytes(const gsvk_sovits_decoder_desc* desc);
/* Issue the decoder's launches on `stream` (GSVK_E_NULL / E_SIZE / E_ARG on a bad descriptor).
 * ResBlocks 1 and 2 of each stage run on two streams the library keeps per device, ordered after
 * the work already on `stream` and joined back into it (each stage's branch mean waits for them), so
 * `stream` orders the whole decoder as usual. Those streams are created on the device's first call:
 * a caller recording this call into a graph of its own makes one call outside the capture first
 * (gsvk_sovits_decoder_create records the same launches by itself). */
int gsvk_sovits_decoder_eager(const gsvk_sovits_decoder_desc* desc, void* stream);
/* Record the same launches into a HIP graph; run it with gsvk_t2s_step_run, free it with
 * gsvk_t2s_step_destroy. The graph keeps the descriptor's pointers: the buffers must outlive it. */
int gsvk_sovits_decoder_create(const gsvk_sovits_decoder_desc* desc, gsvk_t2s_step** out);

#ifdef __cplusplus
}
#endif

#endif /* GSVK_SOVITS_H */
