/*
 * gsvk_t2s.h — C ABI of the T2S decode-step epilogue chain (host driver over gsvk.h).
 *
 * One T2S decode step, as T2SEngine runs it for each new token, interleaves GEMVs with the fused
 * epilogues this library provides. This driver issues the epilogue part of one step for B
 * sequences in the reference's order:
 *   x = audio_emb[id] + alpha_audio * pe[pos]                 (t2s_engine.cpp:1866-1869)
 *   for each layer l:                                         (block_decode_impl, 1035-1120)
 *     h  = LN1( (attn_out[l] + bout[l]) + x )                 (1096-1098)
 *     ff[l] = relu( ff[l] + b1[l] )   in place                (1111-1112)
 *     x  = LN2( (ffn_out[l] + b2[l]) + h )                    (1117-1119)
 * attn_out[l], ff[l] and ffn_out[l] stand for the outputs of the out-projection, W1 and W2 GEMVs
 * of layer l (the GEMVs themselves are not part of this library). That is 1 + 3*layers launches
 * (73 for the 24-layer model); gsvk_t2s_step_create records them once into a HIP graph so a step
 * is one graph launch.
 */
#ifndef GSVK_T2S_H
#define GSVK_T2S_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gsvk_t2s_step_desc {
  int dtype;          /* activation storage (gsvk_dtype) of x, h, attn_out, ff, ffn_out        */
  size_t batch;       /* B sequences, one new token each                                        */
  size_t d_model;     /* D (512)                                                                */
  size_t ffn;         /* FF (2048)                                                              */
  size_t layers;      /* 24                                                                     */
  double eps;         /* LayerNorm eps (config ln_eps, 1e-5)                                    */
  /* decode input: embedding gather + alpha * PE */
  const void* audio_table; /* [vocab, D], table_dtype                                           */
  int table_dtype;
  size_t vocab;
  const void* ids;         /* [B] sampled tokens                                                */
  int index_type;          /* gsvk_index_type                                                   */
  const int64_t* pos;      /* [B] positions (P + idx per sequence)                              */
  const float* pe;         /* [max_pos, D] gsvk_pe_table                                         */
  size_t max_pos;
  float alpha;
  int32_t* err;            /* optional device flag for out-of-range ids / positions             */
  /* activations */
  void* x;                 /* [B, D] step input, then each layer's output                       */
  void* h;                 /* [B, D] norm1 output of the current layer                          */
  /* per-layer arrays of `layers` device pointers (the host arrays are copied at create) */
  const void* const* attn_out; /* [B, D]  */
  const float* const* bout;    /* [D]     */
  const float* const* n1g;     /* [D]     */
  const float* const* n1b;     /* [D]     */
  void* const* ff;             /* [B, FF] */
  const float* const* b1;      /* [FF]    */
  const void* const* ffn_out;  /* [B, D]  */
  const float* const* b2;      /* [D]     */
  const float* const* n2g;     /* [D]     */
  const float* const* n2b;     /* [D]     */
} gsvk_t2s_step_desc;

typedef struct gsvk_t2s_step gsvk_t2s_step;

/* Issue the 1 + 3*layers launches of one step directly on `stream` (no graph). */
int gsvk_t2s_step_eager(const gsvk_t2s_step_desc* desc, void* stream);

/* Validate desc, record one step into a HIP graph and instantiate it. */
int gsvk_t2s_step_create(const gsvk_t2s_step_desc* desc, gsvk_t2s_step** out);
/* Launch the recorded step on `stream`. */
int gsvk_t2s_step_run(gsvk_t2s_step* step, void* stream);
/* Number of kernel launches in one step (1 + 3*layers). */
int gsvk_t2s_step_launches(const gsvk_t2s_step* step);
void gsvk_t2s_step_destroy(gsvk_t2s_step* step);

#ifdef __cplusplus
}
#endif

#endif /* GSVK_T2S_H */
