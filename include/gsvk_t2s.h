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

/* The same step as ONE kernel launch (no counterpart in the reference, which runs these loops
 * one row at a time; replaces the 1 + 3*layers launches above). The LayerNorm chain is row-local
 * (row b of layer l+1 reads only row b of layer l), so one wave walks the whole chain of one
 * sequence while the other waves of the launch run the ReLU tiles. Every h and x is stored as the
 * per-op launches store it (the final x and h are the last layer's), every ff[l] is updated in
 * place. The gather and ff[l] are bitwise those of gsvk_t2s_step_eager; each LayerNorm takes its
 * statistics in one pass as gsv::kern::layernorm does (kern.cpp:27-59: sum and sum of squares,
 * a centred second pass only where E[x^2] - mean^2 < 0), where gsvk_add_layernorm takes exact
 * two-pass ones, so h and x agree with the per-op launches within the LayerNorm tolerance per
 * layer, not bit for bit. Deterministic: the same inputs give the same bits on every call.
 * Limits: layers <= 32 (the layer pointers travel in the kernel arguments); d_model a multiple of
 * 8 (4 for f32) and at most 1024 (f16 / bf16) or 512 (f32) elements; ffn a multiple of 8 (4);
 * every pointer 16-byte aligned; x, h, ff[l] overlapping nothing else.
 * GSVK_E_ARG / GSVK_E_SIZE when the shape is outside these limits (use the forms above). */
int gsvk_t2s_step_fused(const gsvk_t2s_step_desc* desc, void* stream);
/* gsvk_t2s_step_fused recorded into a HIP graph (one node); run / launches / destroy as above. */
int gsvk_t2s_step_create_fused(const gsvk_t2s_step_desc* desc, gsvk_t2s_step** out);

/* ------------------------------------------------------------------------------------------------
 * The whole T2S decode step for B sequences: the same epilogue chain with the GEMVs and the
 * attention that feed it, as T2SEngine::generate runs one token (t2s_engine.cpp:1864-1885:
 * x = audio_emb[id] + alpha * PE, block_decode_impl for every layer, predict_layer_fp):
 *   x = embed_pe(ids, pos)                                          (1866-1869)
 *   for each layer l (block_decode_impl, 1035-1120):
 *     qkv  = Wqkv x + bqkv                           fp32           (1044-1049)
 *     attn = attention(qkv, K_l, V_l, kv_pos)        + KV append    (1051-1087)
 *     z    = (Wout attn + bout) + x;   h = LN1(z)                   (1090-1098)
 *     ff   = relu(W1 h + b1)                                        (1105-1112)
 *     z    = (W2 ff + b2) + h;         x = LN2(z)                   (1113-1119)
 *   logits = Wp x                                    fp32, no bias  (predict_layer_fp, 704-707)
 * Activations x, h, z, attn, ff are stored in `dtype`; GEMVs round x to fp16 (gemv_fmlal) and
 * accumulate in fp32; the epilogues add in fp32 before the single rounding to `dtype`.
 * pos[b] is the PE position of the new token (P + idx), kv_pos[b] its cache slot (cur_len); the
 * step attends over kv_pos[b] + 1 keys. Per layer: 4 GEMV launches and the attention (+ 1 chunk
 * merge when len_bound > 256); LN1 runs inside the W1 GEMV and LN2 inside the next layer's QKV GEMV
 * (gsvk_gemv_f16w_ln, within the LayerNorm tolerance of separate launches); plus the embedding
 * and the logits GEMV
 * with the last LN2 (a LayerNorm launch when there are no logits).
 * ------------------------------------------------------------------------------------------------ */
typedef struct gsvk_t2s_layer {
  const uint16_t* wqkv; /* [3D, D] fp16 */
  const float* bqkv;    /* [3D]          */
  const uint16_t* wout; /* [D, D]        */
  const float* bout;    /* [D]           */
  const float* n1g;     /* [D]           */
  const float* n1b;
  const uint16_t* w1;   /* [FF, D]       */
  const float* b1;      /* [FF]          */
  const uint16_t* w2;   /* [D, FF]       */
  const float* b2;      /* [D]           */
  const float* n2g;
  const float* n2b;
  void* k_cache;        /* [B, max_len, D] kv_dtype */
  void* v_cache;
} gsvk_t2s_layer;

typedef struct gsvk_t2s_decode_desc {
  int dtype;            /* activation storage                                      */
  int kv_dtype;         /* cache storage                                           */
  size_t batch, d_model, heads, ffn, layers;
  size_t max_len;       /* cache rows per sequence                                 */
  size_t len_bound;     /* upper bound of kv_pos[b] + 1 (0 = max_len)              */
  double eps;
  const void* audio_table; /* [vocab, D] */
  int table_dtype;
  size_t vocab;
  const void* ids;         /* [B] */
  int index_type;
  const int64_t* pos;      /* [B] PE positions */
  const int64_t* kv_pos;   /* [B] cache slots  */
  const float* pe;         /* [max_pos, D] */
  size_t max_pos;
  float alpha;
  int32_t* err;            /* optional: bad id / position / cache slot */
  const gsvk_t2s_layer* layer; /* [layers], host memory, read by eager / create only */
  const uint16_t* w_logits;    /* [vocab, D] fp16 or NULL */
  float* logits;               /* [B, vocab] */
  /* scratch activations, all [B, ...] in dtype except qkv (fp32) */
  void* x;   /* [B, D]  */
  void* h;   /* [B, D]  */
  void* z;   /* [B, D]  */
  void* attn;/* [B, D]  */
  void* ff;  /* [B, FF] */
  float* qkv;/* [B, 3D] */
  void* workspace;         /* gsvk_t2s_decode_workspace_bytes(batch, heads, D/heads, len)     */
  size_t workspace_bytes;
  int parts;               /* 0: two halves when batch >= 32, else one chain; 1: one chain    */
} gsvk_t2s_decode_desc;

/* With parts 0 a batch of 32 sequences or more runs as two halves, when the workspace holds both
 * halves' attention states (gsvk_t2s_decode_workspace_bytes; otherwise as one chain): every launch
 * is row-local, so each half is the same chain of launches over its rows, and the graph records the
 * two chains on two branches that run concurrently (one half's latency-bound GEMVs overlap the
 * other half's cache scan). An eager step issues the two chains one after the other on `stream`:
 * the same launches, the same bits. */
int gsvk_t2s_decode_eager(const gsvk_t2s_decode_desc* desc, void* stream);
/* Records one step into a HIP graph; run / launches / destroy with the gsvk_t2s_step calls. */
int gsvk_t2s_decode_create(const gsvk_t2s_decode_desc* desc, gsvk_t2s_step** out);
/* Workspace bytes for a step of `batch` sequences (len_bound as in the desc; 0 = any length):
 * the larger of what one chain and the two halves' attention calls need. No counterpart in the
 * reference (its attention keeps no chunk states). */
size_t gsvk_t2s_decode_workspace_bytes(size_t batch, size_t heads, size_t head_dim,
                                       size_t len_bound);

#ifdef __cplusplus
}
#endif

#endif /* GSVK_T2S_H */
