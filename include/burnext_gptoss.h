/*
 * burnext_gptoss.h -- C ABI of the GPT-OSS decoder decode step around the MI355X MoE layer
 * (burnext_moe.h): embedding, per layer RmsNorm + streaming multi-query attention with a rolling
 * KV cache, learned sinks, YaRN RoPE and alternating sliding-window / full layers, then the MoE
 * layer; final RmsNorm, LM head and greedy argmax.  Every kernel is HIP for gfx950.
 *
 * Reference interfaces replaced (paths relative to the ariawisp/burn-extended tree):
 *   burnext_gptoss_create      GptOssConfig::init + set_moe_quant_resident  src/models/gpt_oss.rs:115-189,458-467
 *   burnext_gptoss_decode      AutoregressiveModel::forward_logits (decode branch)
 *                              + greedy argmax                             src/models/gpt_oss.rs:226-252
 *   burnext_gptoss_reset       StreamingMqaCache::reset                     src/attention/streaming_mqa.rs:175-179
 *   burnext_gptoss_cache_load  (new: fills the cache with given rows -- what a prefill leaves)
 *   burnext_gptoss_destroy     drop of GptOssModel
 *
 * Conventions as burnext_moe.h: host pointers read at create only; device pointers otherwise;
 * asynchronous on `stream`, no host synchronisation and no allocation in decode; statuses and
 * burnext_last_error().  The cache position bookkeeping (rows held) is host state advanced at
 * each decode call, as the reference's local_end_index is.
 */
#ifndef BURNEXT_GPTOSS_H
#define BURNEXT_GPTOSS_H

#include "burnext_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Mirrors GptOssConfig (src/models/gpt_oss.rs:18-47) for the decode path. */
typedef struct burnext_gptoss_config {
  uint32_t vocab_size;
  uint32_t d_model;        /* multiple of 4 */
  uint32_t n_layers;
  uint32_t n_heads;
  uint32_t kv_heads;        /* n_heads / kv_heads a power of two <= 16 */
  uint32_t head_dim;       /* multiple of 8, <= 128 */
  uint32_t max_batch;      /* <= 16 */
  uint32_t cache_len;      /* rolling KV cache rows per (layer, batch row); cache_len * n_heads / kv_heads <= 4M */
  uint32_t window_policy;  /* WindowPolicy (src/cache/mod.rs:7-33): 0 Full, 1 Fixed(window),
                              2 EveryOther { window, full_on_even } */
  uint32_t window;
  uint32_t full_on_even;
  uint32_t rope_head_stride; /* 1: head h rotated at start_pos + h, as the reference's RoPE over
                                [B, T, heads, d] does (it takes the head axis as the sequence);
                                0: every head at start_pos */
  uint32_t max_positions;  /* decode positions pos < max_positions (RoPE table rows: max_positions + n_heads) */
  uint32_t kv_bf16;        /* 0: f32 cache rows (the reference's float element); 1: bf16 rows */
  float rms_eps;           /* Burn RmsNorm epsilon (1e-5) */
  float rope_theta;        /* RoPE base */
  float rope_scaling_factor, rope_initial_context, rope_ntk_alpha, rope_ntk_beta; /* init_ntk_yarn */
  float scale_dk;          /* scores divided by sqrt(scale_dk): 1 for pre-scaled q/k (GPT-OSS) */
  uint32_t sink_tokens;    /* GptOssConfig.sink_tokens (src/models/gpt_oss.rs:35,211), < cache_len: the
                              cache keeps the rows of the first sink_tokens positions through eviction
                              (src/attention/cache_ops.rs:64-117), and Window(w) attends over the last
                              sink_tokens + min(w, rows - sink_tokens) cache rows
                              (src/attention/streaming_mqa.rs:332-339); a windowed layer needs at least
                              sink_tokens cache rows (BURNEXT_INVALID_ARG before any launch otherwise) */
  uint32_t experts_bf16;   /* 0: the MoE layers' expert projections take the normalised f32 rows (the
                              reference's element, two bf16 MFMA terms); 1: those rows rounded to bf16
                              once (one term; routing, residuals and norms stay f32).  No counterpart
                              in the reference; results within 2e-2 of it */
} burnext_gptoss_config;

/* Dense weights (host, bf16 bit patterns, row-major [out, in] as Burn Linear's transposed weight;
 * layer tensors stacked along a leading [n_layers] axis). */
typedef struct burnext_gptoss_weights {
  const uint16_t *tok_emb;    /* [V, D] */
  const uint16_t *norm_attn;  /* [L, D] */
  const uint16_t *wq, *bq;    /* [L, nH*dk, D], [L, nH*dk] */
  const uint16_t *wk, *bk;    /* [L, kvH*dk, D], [L, kvH*dk] */
  const uint16_t *wv, *bv;    /* [L, kvH*dk, D], [L, kvH*dk] */
  const uint16_t *wo, *bo;    /* [L, D, nH*dk], [L, D] */
  const uint16_t *sinks;      /* [L, nH] learned sinks (head h = kv head h / groups, group h % groups), nullable */
  const uint16_t *norm_final; /* [D] */
  const uint16_t *lm_head;    /* [V, D] */
} burnext_gptoss_weights;

typedef struct burnext_gptoss *burnext_gptoss_t;

/* Uploads the dense weights (repacked into the decode GEMV's tiled layout), builds the YaRN RoPE
 * table and allocates the KV cache; `moe_layers` [n_layers] are MoE layers created with
 * burnext_moe_layer_create on the same device (d_model must match), not owned by the decoder. */
burnext_status burnext_gptoss_create(const burnext_gptoss_config *cfg, const burnext_gptoss_weights *w,
                                     const burnext_moe_layer_t *moe_layers, int device, burnext_gptoss_t *out);
void burnext_gptoss_destroy(burnext_gptoss_t model);

/* Workspace bytes of a decode step with `batch` rows (non-decreasing in batch). */
burnext_status burnext_gptoss_workspace_size(burnext_gptoss_t model, uint32_t batch, uint64_t *bytes);

/* Empties the cache (no device work). */
burnext_status burnext_gptoss_reset(burnext_gptoss_t model);

/* Replaces the cache contents with `len` rows per (layer, batch row) for positions 0 .. len-1:
 * k, v device f32 [L, batch, len, kvH, dk] (the reference's cache layout, keys already rotated),
 * stored in the cache's element type (kv_bf16).  len <= cache_len. */
burnext_status burnext_gptoss_cache_load(burnext_gptoss_t model, const float *k, const float *v, uint32_t batch,
                                         uint32_t len, void *stream);

/* One decode step: tokens[batch] (device int32) at absolute position `pos`, which must equal the
 * number of positions seen so far.  While the cache holds rows, batch may not exceed the batch
 * rows it holds them for (those of the last cache_load or decode; BURNEXT_INVALID_ARG, reset
 * first).  `window` is the caller's AttnWindow (0 = Full, w > 0 =
 * Window(w)), combined with each layer's policy window as combine_windows does (the smaller).
 * next_tokens[batch] (device int32) = argmax of the logits (lowest index on ties, NaN lowest);
 * logits [batch, V] f32 (device, nullable); hidden [batch, D] f32 (device, nullable): the last
 * layer's output before the final norm. */
burnext_status burnext_gptoss_decode(burnext_gptoss_t model, const int32_t *tokens, uint32_t batch, uint32_t pos,
                                     uint32_t window, int32_t *next_tokens, float *logits, float *hidden,
                                     void *workspace, uint64_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* BURNEXT_GPTOSS_H */
