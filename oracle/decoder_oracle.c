/*
 * decoder_oracle.c -- CPU restatement of burn-extended's GPT-OSS decoder decode step around the
 * MoE layer (the "full decoder decode" benchmark config).
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker of the decoder kernels in
 * burn-extended_amd/csrc/decoder.hip.  Nothing in the product library links, loads or calls it;
 * only tests/, smoke() and bench.py's cpu_baseline leg use it.
 *
 * Reference (ariawisp/burn-extended) functions restated here:
 *   GptOssModel::forward_logits, decode branch ... src/models/gpt_oss.rs:226-252
 *     hidden = tok_emb(last token); per layer l: window = combine_windows(window, policy(l)),
 *     hidden = layer.forward(hidden); logits = lm_head(norm_final(hidden))
 *   GptOssLayer::forward .......................... src/models/gpt_oss.rs:101-113
 *     hidden = hidden + attn(RmsNorm(hidden)); return moe(hidden)  (the MoE adds its own norm and residual)
 *   StreamingMultiQueryAttention::forward_streaming src/attention/streaming_mqa.rs:239-419
 *     q/k/v Linear (with bias); RoPE on q and k; cache append with eviction (roll) when full;
 *     active window; scores = q k^T / sqrt(scale_dk) (scale_dk = 1: pre_scaled_qk); sinks softmax;
 *     context = weights v; output Linear (with bias)
 *   apply_sinks_then_softmax ...................... src/attention/core.rs:34-55
 *     softmax over [scores..., sink] then the sink column dropped
 *   init_ntk_yarn ................................. src/rope/mod.rs:11-52
 *   WindowPolicy::EveryOther / combine_windows .... src/cache/mod.rs:7-44
 *   evict_and_roll_mqa ............................ src/attention/cache_ops.rs:64-117
 *
 * Third-party semantics restated (Burn at rev 0c13f844dc530e36dddff4626f9644746dbe53c6, not
 * vendored; its published algorithm):
 *   RotaryEncoding (burn-core nn/rope_encoding.rs): inv_freq[i] = 1 / theta^(2 i / d) for
 *     i < d / 2 (then the caller's frequency scaling); freq_complex[p][2i], [2i+1] =
 *     (cos(p inv_freq[i]), sin(p inv_freq[i])); apply(x, start) treats dimension D-2 of x as the
 *     sequence and rotates interleaved pairs: y[2i] = x[2i] c - x[2i+1] s, y[2i+1] = x[2i+1] c +
 *     x[2i] s with (c, s) = freq_complex[start + seq index].  The reference applies it to
 *     [B, T, heads, d] (streaming_mqa.rs:262-289), so the sequence index is the head index:
 *     at decode head h of q (and of k) is rotated at position start_pos + h.  head_stride = 1
 *     reproduces that; head_stride = 0 rotates every head at start_pos.
 *   RmsNorm: x / sqrt(mean(x^2) + eps) * gamma.   Linear: y = x W^T + b.
 *
 * Parity pins (tests/test_oracle.py): RoPE tables against closed forms (factor <= 1 is plain
 * RoPE; ramp ends give inv_freq / factor and inv_freq; |rotation| = concentration) and complex
 * multiplication; sinks softmax against closed forms (sink -> -inf is softmax, weight mass
 * 1 - sink share) and float64 brute force; the whole step against an independent float64
 * numpy restatement (tests/test_oracle.py::test_decoder_step_float64), windowed = full within
 * the window, key-order invariance of the cache.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_OK 0
#define ORACLE_INVALID 1

typedef struct {
  int64_t d, f, e, k;
  float alpha, limit, eps;
  int64_t bf16_rows;
} oracle_cfg;

int oracle_moe_forward(const float *x, int64_t n, const oracle_cfg *cfg, const uint8_t *w1b, const uint8_t *w1s,
                       const uint8_t *w2b, const uint8_t *w2s, int ue8_offset, const float *b1, const float *b2,
                       const float *router_w, const float *router_b, const float *gamma, int layout,
                       int apply_rmsnorm, int add_residual, float *y, int32_t *idx_out, float *w_out);

/* YaRN-scaled inverse frequencies (src/rope/mod.rs:11-52 over Burn's
 * init_with_frequency_scaling): inv[i] = theta^(-2i/d), i < d/2; with factor > 1,
 * r = clamp((2i - low) / (high - low), 0, 1) (the closure recovers "i" = -(2d/2) ln(inv)/ln(theta)
 * = 2i), inv = inv / factor * (1 - r) + inv * r, low = d ln(ctx / (beta 2 pi)) / ln(theta),
 * high = d ln(ctx / (alpha 2 pi)) / ln(theta); concentration = 0.1 ln(factor) + 1 multiplies
 * the cos/sin table.  Returns ORACLE_INVALID where the reference asserts. */
int oracle_yarn_inv_freq(int64_t d, double theta, double factor, double ctx, double alpha, double beta, float *inv,
                         float *concentration) {
  if (d < 2 || d % 2) return ORACLE_INVALID;
  const int64_t half = d / 2;
  for (int64_t i = 0; i < half; ++i) inv[i] = (float)(1.0 / pow(theta, (double)(2 * i) / (double)d));
  *concentration = 1.0f;
  if (factor <= 1.0) return ORACLE_OK;
  const double dd = (double)d, lb = log(theta), two_pi = 6.283185307179586476925;
  const double low = dd * log(ctx / (beta * two_pi)) / lb, high = dd * log(ctx / (alpha * two_pi)) / lb;
  if (!(low > 0.0 && high > 0.0 && low < high && high < dd - 1.0)) return ORACLE_INVALID;
  for (int64_t i = 0; i < half; ++i) {
    const double f = (double)inv[i];
    const double irec = -log(f) * dd / lb;  /* = 2 i */
    double r = (irec - low) / (high - low);
    r = r < 0.0 ? 0.0 : (r > 1.0 ? 1.0 : r);
    inv[i] = (float)(f / factor * (1.0 - r) + f * r);
  }
  *concentration = (float)(0.1 * log(factor) + 1.0);
  return ORACLE_OK;
}

/* cos/sin table [npos][d/2][2]: angle = p * inv[i] as one f32 product (the reference builds the
 * table in f32), cos and sin of that angle times the concentration, rounded once to f32. */
void oracle_rope_table(const float *inv, int64_t d, float concentration, int64_t npos, float *table) {
  for (int64_t p = 0; p < npos; ++p)
    for (int64_t i = 0; i < d / 2; ++i) {
      const float a = (float)p * inv[i];
      table[(p * (d / 2) + i) * 2] = (float)(cos((double)a) * concentration);
      table[(p * (d / 2) + i) * 2 + 1] = (float)(sin((double)a) * concentration);
    }
}

/* Rotates heads x[h][d] in place: head h at position pos0 + h * head_stride (see header). */
void oracle_rope_apply(float *x, int64_t heads, int64_t d, int64_t pos0, int64_t head_stride, const float *table) {
  for (int64_t h = 0; h < heads; ++h) {
    const int64_t p = pos0 + h * head_stride;
    float *xr = x + h * d;
    for (int64_t i = 0; i < d / 2; ++i) {
      const float c = table[(p * (d / 2) + i) * 2], s = table[(p * (d / 2) + i) * 2 + 1];
      const float x0 = xr[2 * i], x1 = xr[2 * i + 1];
      xr[2 * i] = x0 * c - x1 * s;
      xr[2 * i + 1] = x1 * c + x0 * s;
    }
  }
}

/* y[b][n] = sum_c x[b][c] w[n][c] (+ bias[n]); c ascending. */
void oracle_linear(const float *x, int64_t nb, int64_t k, const float *w, const float *bias, int64_t n, float *y) {
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < n; ++o)
    for (int64_t b = 0; b < nb; ++b) {
      float s = 0.0f;
      for (int64_t c = 0; c < k; ++c) s += x[b * k + c] * w[o * k + c];
      y[b * n + o] = s + (bias ? bias[o] : 0.0f);
    }
}

/* Burn RmsNorm of nb rows (plain sum of squares). */
static void rmsnorm_rows(const float *x, int64_t nb, int64_t d, const float *gamma, float eps, float *y) {
  for (int64_t b = 0; b < nb; ++b) {
    float ss = 0.0f;
    for (int64_t c = 0; c < d; ++c) ss += x[b * d + c] * x[b * d + c];
    const float r = sqrtf(ss / (float)d + eps);
    for (int64_t c = 0; c < d; ++c) y[b * d + c] = (x[b * d + c] / r) * (gamma ? gamma[c] : 1.0f);
  }
}

/* Attention of one query row per head over nk keys with sinks (src/attention/core.rs:34-55):
 * q [nh][d], keys k[j][kvh][d], values v[j][kvh][d] (j < nk, the rows kk0 .. of a buffer with
 * kv_stride floats per key), head h reads kv head h / (nh / nkv); scores scaled by
 * 1/sqrt(scale_dk); sinks [nh] (nullable: plain softmax).  out [nh][d]. */
void oracle_sink_attention(const float *q, const float *k, const float *v, int64_t nk, int64_t kv_stride, int64_t nh,
                           int64_t nkv, int64_t d, const float *sinks, float scale_dk, float *out) {
  const int64_t groups = nh / nkv;
  double *s = (double *)malloc(sizeof(double) * (size_t)(nk + 1));
  for (int64_t h = 0; h < nh; ++h) {
    const int64_t kh = h / groups;
    const float inv = 1.0f / sqrtf(scale_dk);
    float m = sinks ? sinks[h] : -INFINITY;
    for (int64_t j = 0; j < nk; ++j) {
      float acc = 0.0f;
      for (int64_t c = 0; c < d; ++c) acc += q[h * d + c] * k[j * kv_stride + kh * d + c];
      s[j] = acc * inv;
      if ((float)s[j] > m) m = (float)s[j];
    }
    float z = sinks ? expf(sinks[h] - m) : 0.0f;
    for (int64_t j = 0; j < nk; ++j) {
      s[j] = expf((float)s[j] - m);
      z += (float)s[j];
    }
    for (int64_t c = 0; c < d; ++c) {
      float acc = 0.0f;
      for (int64_t j = 0; j < nk; ++j) acc += (float)s[j] / z * v[j * kv_stride + kh * d + c];
      out[h * d + c] = acc;
    }
  }
  free(s);
}

/* Model dimensions and policies (mirrors GptOssConfig, src/models/gpt_oss.rs:18-47). */
typedef struct {
  int64_t vocab, d_model, n_layers, n_heads, kv_heads, head_dim, batch, cache_len;
  int64_t window_policy;    /* WindowPolicy: 0 Full, 1 Fixed(window), 2 EveryOther{window, full_on_even} */
  int64_t window;
  int64_t full_on_even;     /* EveryOther: 1 = even layers full, odd layers windowed */
  int64_t rope_head_stride; /* 1: reference positions (start_pos + head index), 0: start_pos */
  float rms_eps;
  float scale_dk;           /* 1 with pre-scaled q/k (GPT-OSS) */
  int64_t sink_tokens;      /* StreamingMqaCache::sink_tokens (src/attention/streaming_mqa.rs:143) */
  int64_t experts_bf16;     /* the device option: every MoE layer with cfg.bf16_rows = 1 */
} oracle_dec_cfg;

/* Weights as f32 (the device's bf16 values), per layer l at offset l * (layer size). */
typedef struct {
  const float *tok_emb;     /* [V][D] */
  const float *norm_attn;   /* [L][D] */
  const float *wq, *bq;     /* [L][nH dk][D], [L][nH dk] */
  const float *wk, *bk;     /* [L][kvH dk][D], [L][kvH dk] */
  const float *wv, *bv;
  const float *wo, *bo;     /* [L][D][nH dk], [L][D] */
  const float *sinks;       /* [L][nH] (nullable: no sinks) */
  const float *norm_final;  /* [D] */
  const float *lm_head;     /* [V][D] */
  const float *rope_table;  /* [npos][dk/2][2] */
} oracle_dec_weights;

/* One MoE layer's tensors (oracle_moe_forward arguments). */
typedef struct {
  oracle_cfg cfg;
  const uint8_t *w1b, *w1s, *w2b, *w2s;
  int ue8_offset;
  const float *b1, *b2, *router_w, *router_b, *gamma;
  int layout;
} oracle_moe_layer;

/* One decode step (src/models/gpt_oss.rs:226-252) for batch rows b < B: tokens[b] at absolute
 * position pos, caller_window the caller's AttnWindow (0 = Full, w > 0 = Window(w)).
 * Cache k, v: [L][B][cache_len][kvH][dk] with *cache_used valid rows per layer
 * (the reference's local_end_index; all layers advance together), updated in place with the
 * reference's append / evict-and-roll.  Outputs: logits [B][V] (nullable), hidden_out [B][D]
 * (nullable: the final hidden state before norm_final), next_tok [B] (argmax, lowest index on
 * ties). */
int oracle_decoder_step(const oracle_dec_cfg *c, const oracle_dec_weights *w, const oracle_moe_layer *moe,
                        const int32_t *tokens, int64_t pos, int64_t caller_window, float *cache_k, float *cache_v,
                        int64_t *cache_used, float *logits, float *hidden_out, int32_t *next_tok) {
  const int64_t B = c->batch, D = c->d_model, nH = c->n_heads, kvH = c->kv_heads, dk = c->head_dim;
  const int64_t qd = nH * dk, kd = kvH * dk, cap = c->cache_len, sink = c->sink_tokens;
  if (B <= 0 || nH % kvH || cap <= 0 || sink < 0 || sink > cap) return ORACLE_INVALID;
  float *h = (float *)malloc(sizeof(float) * B * D);
  float *xn = (float *)malloc(sizeof(float) * B * D);
  float *q = (float *)malloc(sizeof(float) * B * qd);
  float *kk = (float *)malloc(sizeof(float) * B * kd);
  float *vv = (float *)malloc(sizeof(float) * B * kd);
  float *ctx = (float *)malloc(sizeof(float) * B * qd);
  float *o = (float *)malloc(sizeof(float) * B * D);
  float *h2 = (float *)malloc(sizeof(float) * B * D);
  for (int64_t b = 0; b < B; ++b) memcpy(h + b * D, w->tok_emb + (int64_t)tokens[b] * D, sizeof(float) * D);
  /* cache append with eviction (streaming_mqa.rs:294-323, cache_ops.rs:64-117), one new row: when
   * the cache is full, num_evicted = 1 and avail = used - sink rows after the sink rows; with
   * avail > 1 the rows [sink, used) roll left by one (row sink + i takes row sink + (i + 1) mod
   * avail; the wrapped row is overwritten next), else (avail <= num_evicted) nothing moves; then
   * local_end = used - 1 + 1 and the new row goes to local_end - 1 */
  int rc = ORACLE_OK;
  int64_t used = *cache_used;
  const int evict = used + 1 > cap;
  const int64_t avail = used > sink ? used - sink : 0;
  const int roll = evict && avail > 1;
  const int64_t nused = evict ? used : used + 1;
  const int64_t row = nused - 1;
  /* the active window of every layer (streaming_mqa.rs:332-339): Full = all nused rows,
   * Window(w) = the last sink + min(w, nused - sink) rows; a windowed layer with fewer than sink
   * rows has no valid window (the reference's shapes disagree there) */
  for (int64_t l = 0; l < c->n_layers && sink > 0; ++l) {
    int64_t lw = 0;
    if (c->window_policy == 1) lw = c->window;
    if (c->window_policy == 2) lw = ((l % 2 == 0) == (c->full_on_even != 0)) ? 0 : c->window;
    if (caller_window > 0) lw = lw == 0 ? caller_window : (caller_window < lw ? caller_window : lw);
    if (lw > 0 && nused < sink) return ORACLE_INVALID;
  }
  for (int64_t l = 0; l < c->n_layers; ++l) {
    rmsnorm_rows(h, B, D, w->norm_attn + l * D, c->rms_eps, xn);
    oracle_linear(xn, B, D, w->wq + l * qd * D, w->bq + l * qd, qd, q);
    oracle_linear(xn, B, D, w->wk + l * kd * D, w->bk + l * kd, kd, kk);
    oracle_linear(xn, B, D, w->wv + l * kd * D, w->bv + l * kd, kd, vv);
    for (int64_t b = 0; b < B; ++b) {
      oracle_rope_apply(q + b * qd, nH, dk, pos, c->rope_head_stride, w->rope_table);
      oracle_rope_apply(kk + b * kd, kvH, dk, pos, c->rope_head_stride, w->rope_table);
    }
    const int64_t lstride = B * cap * kd;
    for (int64_t b = 0; b < B; ++b) {
      float *ck = cache_k + l * lstride + b * cap * kd, *cv = cache_v + l * lstride + b * cap * kd;
      if (roll) {  /* rows sink+1 .. used-1 move to sink .. used-2 (row used-1 is rewritten below) */
        memmove(ck + sink * kd, ck + (sink + 1) * kd, sizeof(float) * (size_t)((avail - 1) * kd));
        memmove(cv + sink * kd, cv + (sink + 1) * kd, sizeof(float) * (size_t)((avail - 1) * kd));
      }
      memcpy(ck + row * kd, kk + b * kd, sizeof(float) * kd);
      memcpy(cv + row * kd, vv + b * kd, sizeof(float) * kd);
    }
    /* window_for(l) (src/cache/mod.rs:15-33) combined with the caller's (combine_windows, 0 = Full);
     * Full = every cached row, Window(w) = the last sink + min(w, rows - sink) rows */
    int64_t lw = 0;
    if (c->window_policy == 1) lw = c->window;
    if (c->window_policy == 2) lw = ((l % 2 == 0) == (c->full_on_even != 0)) ? 0 : c->window;
    if (caller_window > 0) lw = lw == 0 ? caller_window : (caller_window < lw ? caller_window : lw);
    const int64_t active = lw > 0 ? sink + (lw < nused - sink ? lw : nused - sink) : nused;
    const int64_t start = nused - active;
    for (int64_t b = 0; b < B; ++b) {
      const float *ck = cache_k + l * lstride + b * cap * kd + start * kd;
      const float *cv = cache_v + l * lstride + b * cap * kd + start * kd;
      oracle_sink_attention(q + b * qd, ck, cv, active, kd, nH, kvH, dk, w->sinks ? w->sinks + l * nH : NULL,
                            c->scale_dk, ctx + b * qd);
    }
    oracle_linear(ctx, B, qd, w->wo + l * D * qd, w->bo + l * D, D, o);
    for (int64_t i = 0; i < B * D; ++i) h[i] = h[i] + o[i];
    const oracle_moe_layer *m = moe + l;
    oracle_cfg mc = m->cfg;
    mc.bf16_rows = c->experts_bf16 ? 1 : 0;
    rc = oracle_moe_forward(h, B, &mc, m->w1b, m->w1s, m->w2b, m->w2s, m->ue8_offset, m->b1, m->b2,
                                m->router_w, m->router_b, m->gamma, m->layout, 1, 1, h2, NULL, NULL);
    if (rc != ORACLE_OK) break;
    memcpy(h, h2, sizeof(float) * B * D);
  }
  if (rc == ORACLE_OK) {
    *cache_used = nused;
    if (hidden_out) memcpy(hidden_out, h, sizeof(float) * B * D);
    rmsnorm_rows(h, B, D, w->norm_final, c->rms_eps, xn);
    float *lg = logits ? logits : (float *)malloc(sizeof(float) * B * c->vocab);
    oracle_linear(xn, B, D, w->lm_head, NULL, c->vocab, lg);
    /* greedy: largest logit, lowest index on ties, NaN below every number */
    if (next_tok)
      for (int64_t b = 0; b < B; ++b) {
        const float *r = lg + b * c->vocab;
        int64_t best = 0;
        for (int64_t i = 1; i < c->vocab; ++i)
          if ((isnan(r[best]) && !isnan(r[i])) || r[i] > r[best]) best = i;
        next_tok[b] = (int32_t)best;
      }
    if (!logits) free(lg);
  }
  free(h);
  free(xn);
  free(q);
  free(kk);
  free(vv);
  free(ctx);
  free(o);
  free(h2);
  return rc;
}
