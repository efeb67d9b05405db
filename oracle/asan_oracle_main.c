/*
 * asan_oracle_main.c -- AddressSanitizer / UndefinedBehaviorSanitizer driver of the CPU oracle.
 *
 * TEST INFRASTRUCTURE ONLY (built by `make -C oracle asan`, run by tests/test_asan.py): calls every
 * entry point of oracle/moe_oracle.c and oracle/decoder_oracle.c on small and ragged shapes (odd
 * widths, partial scale groups, both gate_up layouts, scale offsets, ties and NaN in top-k, every
 * window policy, cache eviction) so that an out-of-bounds index or an uninitialised read in the
 * oracle fails the sanitizer.  Prints "asan oracle ok" and returns 0 on success.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  int64_t d, f, e, k;
  float alpha, limit, eps;
  int64_t bf16_rows;
} oracle_cfg;
float oracle_round_bf16(float v);

float oracle_fp4_value(int nib);
float oracle_e8m0_scale(int s);
void oracle_dequant_mxfp4_bytes(const uint8_t *blocks, const uint8_t *scales, int64_t rows, int64_t b, float *out);
void oracle_dequant_matrix(const uint8_t *blocks, const uint8_t *scales, int64_t rows, int64_t cols, int64_t bpr,
                           int64_t gpr, int ue8_offset, float *out);
void oracle_rmsnorm(const float *x, int64_t n, int64_t d, const float *gamma, float eps, float *xn);
void oracle_router(const float *xn, int64_t n, int64_t d, const float *w, const float *b, int64_t e, float *out);
void oracle_route_logits(const float *x, int64_t n, int64_t d, const float *gamma, float eps, int apply_rmsnorm,
                         const float *w, const float *b, int64_t e, float *out);
void oracle_topk_softmax(const float *logits, int64_t n, int64_t e, int64_t k, int32_t *idx, float *w);
void oracle_dispatch(const int32_t *idx, int64_t n, int64_t k, int64_t e, int32_t *seg_off, int32_t *perm,
                     int32_t *pos_of);
float oracle_swiglu(float g, float l, float alpha, float limit);
int oracle_moe_forward(const float *x, int64_t n, const oracle_cfg *cfg, const uint8_t *w1b, const uint8_t *w1s,
                       const uint8_t *w2b, const uint8_t *w2s, int ue8_offset, const float *b1, const float *b2,
                       const float *router_w, const float *router_b, const float *gamma, int layout,
                       int apply_rmsnorm, int add_residual, float *y, int32_t *idx_out, float *w_out);
int oracle_moe_forward_reference(const float *x, int64_t n, const oracle_cfg *cfg, const uint8_t *w1b,
                                 const uint8_t *w1s, const uint8_t *w2b, const uint8_t *w2s, int ue8_offset,
                                 const float *b1, const float *b2, const float *router_w, const float *router_b,
                                 const float *gamma, int b2_per_ftile, float *y);
int oracle_yarn_inv_freq(int64_t d, double theta, double factor, double ctx, double alpha, double beta, float *inv,
                         float *concentration);
void oracle_rope_table(const float *inv, int64_t d, float concentration, int64_t npos, float *table);
void oracle_rope_apply(float *x, int64_t heads, int64_t d, int64_t pos0, int64_t head_stride, const float *table);
void oracle_linear(const float *x, int64_t nb, int64_t k, const float *w, const float *bias, int64_t n, float *y);
void oracle_sink_attention(const float *q, const float *k, const float *v, int64_t nk, int64_t kv_stride, int64_t nh,
                           int64_t nkv, int64_t d, const float *sinks, float scale_dk, float *out);

typedef struct {
  int64_t vocab, d_model, n_layers, n_heads, kv_heads, head_dim, batch, cache_len;
  int64_t window_policy, window, full_on_even, rope_head_stride;
  float rms_eps, scale_dk;
  int64_t sink_tokens;
  int64_t experts_bf16;
} oracle_dec_cfg;
typedef struct {
  const float *tok_emb, *norm_attn, *wq, *bq, *wk, *bk, *wv, *bv, *wo, *bo, *sinks, *norm_final, *lm_head,
      *rope_table;
} oracle_dec_weights;
typedef struct {
  oracle_cfg cfg;
  const uint8_t *w1b, *w1s, *w2b, *w2s;
  int ue8_offset;
  const float *b1, *b2, *router_w, *router_b, *gamma;
  int layout;
} oracle_moe_layer;
int oracle_decoder_step(const oracle_dec_cfg *c, const oracle_dec_weights *w, const oracle_moe_layer *moe,
                        const int32_t *tokens, int64_t pos, int64_t caller_window, float *cache_k, float *cache_v,
                        int64_t *cache_used, float *logits, float *hidden_out, int32_t *next_tok);

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return (uint32_t)(rng_state >> 16);
}
static float frand(float s) { return ((float)(rnd() % 20001) / 10000.0f - 1.0f) * s; }
/* exact-size heap buffers: any read or write past the end is a sanitizer error */
static float *fbuf(int64_t n, float s) {
  float *p = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  for (int64_t i = 0; i < n; ++i) p[i] = frand(s);
  return p;
}
static uint8_t *bbuf(int64_t n, int lo, int hi) {
  uint8_t *p = (uint8_t *)malloc((size_t)(n > 0 ? n : 1));
  for (int64_t i = 0; i < n; ++i) p[i] = (uint8_t)(lo + (int)(rnd() % (uint32_t)(hi - lo + 1)));
  return p;
}
static int fails = 0;
static void check(int ok, const char *what) {
  if (!ok) {
    fprintf(stderr, "FAIL %s\n", what);
    ++fails;
  }
}

typedef struct {
  oracle_cfg c;
  uint8_t *w1b, *w1s, *w2b, *w2s;
  float *b1, *b2, *rw, *rb, *g;
} layer_t;

static layer_t make_layer(int64_t D, int64_t F, int64_t E, int64_t K, int ue8) {
  layer_t L;
  L.c.d = D;
  L.c.f = F;
  L.c.e = E;
  L.c.k = K;
  L.c.alpha = 1.702f;
  L.c.limit = 7.0f;
  L.c.eps = 1e-5f;
  L.c.bf16_rows = (D + F) & 1;  /* ragged shapes also take the bf16-row products */
  const int64_t bpr1 = (D + 1) / 2, gpr1 = (D + 31) / 32, bpr2 = (F + 1) / 2, gpr2 = (F + 31) / 32;
  L.w1b = bbuf(E * 2 * F * bpr1, 0, 255);
  L.w1s = bbuf(E * 2 * F * gpr1, 119 + ue8, 123 + ue8);
  L.w2b = bbuf(E * D * bpr2, 0, 255);
  L.w2s = bbuf(E * D * gpr2, 119 + ue8, 123 + ue8);
  L.b1 = fbuf(E * 2 * F, 0.01f);
  L.b2 = fbuf(E * D, 0.01f);
  L.rw = fbuf(E * D, 0.05f);
  L.rb = fbuf(E, 0.1f);
  L.g = fbuf(D, 0.2f);
  for (int64_t i = 0; i < D; ++i) L.g[i] += 1.0f;
  return L;
}
static void free_layer(layer_t *L) {
  free(L->w1b);
  free(L->w1s);
  free(L->w2b);
  free(L->w2s);
  free(L->b1);
  free(L->b2);
  free(L->rw);
  free(L->rb);
  free(L->g);
}

static void moe_cases(void) {
  /* (D, F, E, K, n, ue8): odd widths and partial 32-column scale groups */
  const int64_t cases[][6] = {{64, 64, 4, 2, 5, 0}, {40, 72, 3, 2, 7, 14}, {33, 17, 5, 3, 1, 0}, {96, 48, 8, 8, 3, 14},
                              {31, 31, 2, 4, 2, 0}};
  for (size_t ci = 0; ci < sizeof(cases) / sizeof(cases[0]); ++ci) {
    const int64_t D = cases[ci][0], F = cases[ci][1], E = cases[ci][2], K = cases[ci][3], n = cases[ci][4];
    const int ue8 = (int)cases[ci][5];
    const int64_t Ke = K < E ? K : E;
    layer_t L = make_layer(D, F, E, K, ue8);
    float *x = fbuf(n * D, 1.0f);
    float *y = fbuf(n * D, 0.0f), *y2 = fbuf(n * D, 0.0f);
    int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n * Ke));
    float *w = fbuf(n * Ke, 0.0f);
    for (int layout = 0; layout < 2; ++layout)
      for (int flags = 0; flags < 4; ++flags)
        check(oracle_moe_forward(x, n, &L.c, L.w1b, L.w1s, L.w2b, L.w2s, ue8, L.b1, L.b2, L.rw, L.rb,
                                 (flags & 1) ? L.g : NULL, layout, flags & 1, (flags >> 1) & 1, y, idx, w) == 0,
              "moe_forward");
    check(oracle_moe_forward(x, n, &L.c, L.w1b, L.w1s, L.w2b, L.w2s, ue8, L.b1, L.b2, L.rw, NULL, NULL, 1, 1, 1, y,
                             NULL, NULL) == 0,
          "moe_forward null outputs");
    for (int per = 0; per < 2; ++per)
      check(oracle_moe_forward_reference(x, n, &L.c, L.w1b, L.w1s, L.w2b, L.w2s, ue8, L.b1, L.b2, L.rw, L.rb, L.g, per,
                                         y2) == 0,
            "moe_forward_reference");
    /* pieces */
    float *xn = fbuf(n * D, 0.0f), *lg = fbuf(n * E, 0.0f), *lg2 = fbuf(n * E, 0.0f);
    oracle_rmsnorm(x, n, D, L.g, 1e-5f, xn);
    oracle_rmsnorm(x, n, D, NULL, 1e-5f, xn);
    oracle_router(xn, n, D, L.rw, L.rb, E, lg);
    oracle_router(xn, n, D, L.rw, NULL, E, lg);
    oracle_route_logits(x, n, D, L.g, 1e-5f, 1, L.rw, L.rb, E, lg2);
    oracle_route_logits(x, n, D, NULL, 1e-5f, 0, L.rw, NULL, E, lg2);
    oracle_topk_softmax(lg, n, E, Ke, idx, w);
    int32_t *seg = (int32_t *)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t *perm = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n * Ke));
    int32_t *pos = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n * Ke));
    oracle_dispatch(idx, n, Ke, E, seg, perm, pos);
    check(seg[E] == (int32_t)(n * Ke), "dispatch total");
    float *dq = fbuf(E * 2 * F * D, 0.0f);
    oracle_dequant_matrix(L.w1b, L.w1s, E * 2 * F, D, (D + 1) / 2, (D + 31) / 32, ue8, dq);
    free(dq);
    free(seg);
    free(perm);
    free(pos);
    free(xn);
    free(lg);
    free(lg2);
    free(x);
    free(y);
    free(y2);
    free(idx);
    free(w);
    free_layer(&L);
  }
  /* top-k with ties and NaN; n = 0 */
  float lg[2 * 6] = {1, 1, 1, NAN, 0, 1, NAN, NAN, NAN, NAN, NAN, NAN};
  int32_t idx[2 * 3];
  float w[2 * 3];
  oracle_topk_softmax(lg, 2, 6, 3, idx, w);
  check(idx[0] == 0 && idx[1] == 1 && idx[2] == 2, "topk ties");
  oracle_topk_softmax(lg, 0, 6, 3, idx, w);
  /* dequant helpers */
  uint8_t blocks[3 * 5], scales[3];
  for (int i = 0; i < 15; ++i) blocks[i] = (uint8_t)(i * 37);
  for (int i = 0; i < 3; ++i) scales[i] = (uint8_t)(120 + i * 60);
  float out[3 * 10];
  oracle_dequant_mxfp4_bytes(blocks, scales, 3, 5, out);
  for (int nib = 0; nib < 16; ++nib) (void)oracle_fp4_value(nib);
  for (int s = 0; s < 256; ++s) (void)oracle_e8m0_scale(s);
  check(oracle_swiglu(100.0f, 100.0f, 1.702f, 7.0f) > 0.0f, "swiglu");
}

static void decoder_cases(void) {
  /* (V, D, L, nH, kvH, dk, B, cap, policy, window, full_on_even, stride, caller window, sink tokens) */
  const int64_t cases[][14] = {{37, 40, 3, 4, 2, 16, 2, 5, 2, 3, 1, 1, 0, 0},
                               {29, 64, 2, 8, 1, 8, 3, 4, 1, 2, 0, 0, 3, 1},
                               {50, 32, 2, 2, 2, 32, 1, 6, 0, 1, 0, 1, 0, 2}};
  for (size_t ci = 0; ci < sizeof(cases) / sizeof(cases[0]); ++ci) {
    const int64_t *q = cases[ci];
    oracle_dec_cfg c;
    c.vocab = q[0];
    c.d_model = q[1];
    c.n_layers = q[2];
    c.n_heads = q[3];
    c.kv_heads = q[4];
    c.head_dim = q[5];
    c.batch = q[6];
    c.cache_len = q[7];
    c.window_policy = q[8];
    c.window = q[9];
    c.full_on_even = q[10];
    c.rope_head_stride = q[11];
    c.rms_eps = 1e-5f;
    c.scale_dk = 1.0f;
    c.sink_tokens = q[13];
    c.experts_bf16 = ci & 1;
    const int64_t V = c.vocab, D = c.d_model, L = c.n_layers, qd = c.n_heads * c.head_dim,
                  kd = c.kv_heads * c.head_dim, B = c.batch, steps = c.cache_len + 3;
    const int64_t npos = steps + c.n_heads;
    float *inv = fbuf(c.head_dim / 2, 0.0f), conc = 0.0f;
    const int yrc = oracle_yarn_inv_freq(c.head_dim, 150000.0, ci == 2 ? 1.0 : 32.0, 4096.0, 1.0, 32.0, inv, &conc);
    check(yrc == 0, "yarn");
    float *table = fbuf(npos * c.head_dim, 0.0f);
    oracle_rope_table(inv, c.head_dim, conc, npos, table);
    oracle_dec_weights w;
    float *bufs[14];
    const int64_t sizes[13] = {V * D, L * D, L * qd * D, L * qd, L * kd * D, L * kd, L * kd * D, L * kd, L * D * qd,
                               L * D, L * c.n_heads, D, V * D};
    for (int i = 0; i < 13; ++i) bufs[i] = fbuf(sizes[i], i == 0 ? 1.0f : 0.2f);
    w.tok_emb = bufs[0];
    w.norm_attn = bufs[1];
    w.wq = bufs[2];
    w.bq = bufs[3];
    w.wk = bufs[4];
    w.bk = bufs[5];
    w.wv = bufs[6];
    w.bv = bufs[7];
    w.wo = bufs[8];
    w.bo = bufs[9];
    w.sinks = ci == 1 ? NULL : bufs[10];
    w.norm_final = bufs[11];
    w.lm_head = bufs[12];
    w.rope_table = table;
    layer_t *ml = (layer_t *)malloc(sizeof(layer_t) * (size_t)L);
    oracle_moe_layer *moe = (oracle_moe_layer *)malloc(sizeof(oracle_moe_layer) * (size_t)L);
    for (int64_t l = 0; l < L; ++l) {
      ml[l] = make_layer(D, 24 + 8 * l, 4, 2, 0);
      moe[l].cfg = ml[l].c;
      moe[l].w1b = ml[l].w1b;
      moe[l].w1s = ml[l].w1s;
      moe[l].w2b = ml[l].w2b;
      moe[l].w2s = ml[l].w2s;
      moe[l].ue8_offset = 0;
      moe[l].b1 = ml[l].b1;
      moe[l].b2 = ml[l].b2;
      moe[l].router_w = ml[l].rw;
      moe[l].router_b = ml[l].rb;
      moe[l].gamma = ml[l].g;
      moe[l].layout = (int)(l & 1);
    }
    float *ck = fbuf(L * B * c.cache_len * kd, 0.0f), *cv = fbuf(L * B * c.cache_len * kd, 0.0f);
    float *logits = fbuf(B * V, 0.0f), *hidden = fbuf(B * D, 0.0f);
    int32_t *tok = (int32_t *)malloc(sizeof(int32_t) * (size_t)B), *nxt = (int32_t *)malloc(sizeof(int32_t) * (size_t)B);
    for (int64_t b = 0; b < B; ++b) tok[b] = (int32_t)((b * 7) % V);
    int64_t used = 0;
    for (int64_t pos = 0; pos < steps; ++pos) {
      check(oracle_decoder_step(&c, &w, moe, tok, pos, q[12], ck, cv, &used, pos & 1 ? NULL : logits,
                                pos & 2 ? NULL : hidden, nxt) == 0,
            "decoder_step");
      memcpy(tok, nxt, sizeof(int32_t) * (size_t)B);
    }
    check(used == c.cache_len, "cache rows");
    /* pieces */
    float *xh = fbuf(c.n_heads * c.head_dim, 1.0f);
    oracle_rope_apply(xh, c.n_heads, c.head_dim, 2, c.rope_head_stride, table);
    float *y = fbuf(2 * qd, 0.0f);
    oracle_linear(bufs[0], 2, D, bufs[2], bufs[3], qd, y);
    oracle_linear(bufs[0], 2, D, bufs[2], NULL, qd, y);
    float *att = fbuf(c.n_heads * c.head_dim, 0.0f);
    oracle_sink_attention(xh, ck, cv, c.cache_len, kd, c.n_heads, c.kv_heads, c.head_dim, bufs[10], 1.0f, att);
    oracle_sink_attention(xh, ck, cv, 1, kd, c.n_heads, c.kv_heads, c.head_dim, NULL, 4.0f, att);
    free(att);
    free(y);
    free(xh);
    free(ck);
    free(cv);
    free(logits);
    free(hidden);
    free(tok);
    free(nxt);
    for (int64_t l = 0; l < L; ++l) free_layer(&ml[l]);
    free(ml);
    free(moe);
    for (int i = 0; i < 13; ++i) free(bufs[i]);
    free(table);
    free(inv);
  }
  float inv[8], conc;
  check(oracle_yarn_inv_freq(16, 150000.0, 32.0, 4096.0, 32.0, 1.0, inv, &conc) != 0, "yarn assert");
  check(oracle_yarn_inv_freq(15, 150000.0, 1.0, 4096.0, 1.0, 32.0, inv, &conc) != 0, "yarn odd d");
}

int main(void) {
  moe_cases();
  decoder_cases();
  if (fails) {
    fprintf(stderr, "%d checks failed\n", fails);
    return 1;
  }
  printf("asan oracle ok\n");
  return 0;
}
