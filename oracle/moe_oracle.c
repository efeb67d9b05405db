/*
 * moe_oracle.c -- CPU restatement of burn-extended's GPT-OSS MoE feed-forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP kernels in
 * burn-extended_amd/csrc and the CPU baseline timed by bench.py (cpu_baseline leg).
 * Nothing in the product library links, loads or calls it.  Only tests/, the smoke()
 * check and bench.py's cpu_baseline leg may use it.
 *
 * Reference (ariawisp/burn-extended) functions restated here:
 *   fp4 LUT / dequant ......... src/loader/mxfp4.rs:10-13, :56-79 (exact powi form)
 *   element addressing ........ src/quant/gpu.rs:124-131 (byte = blocks[row*bpr + c/2],
 *                               low nibble for even c; scale = scales[row*gpr + c/32])
 *   RMSNorm + router Linear ... src/moe/mod.rs:109-110 (Burn RmsNorm: x / sqrt(mean(x^2)+eps) * gamma;
 *                               routing applies 1/r after the dot product, see oracle_route_logits)
 *   top-k + softmax ........... src/moe/mod.rs:271-276 (softmax over the k selected logits)
 *   W1 + clamped SwiGLU ....... src/quant/gpu.rs:89-146, src/activation/mod.rs:5-45
 *   W2 + weighted accumulate .. src/quant/gpu.rs:148-192, src/moe/mod.rs:405-411
 *   model.bin scale offset .... src/bin/gptoss_export.rs:529,562 (stored = s + 14 mod 256)
 *
 * Fixed reduction orders.  Routing (RMSNorm sum of squares and router logits) uses the
 * order the GPU route kernel uses, so indices and logits can be compared bit-exactly:
 *   lane partials  p[l] = fmaf(a[c], b[c], p[l]) over c = 512 i + 8 l + j, i ascending, then
 *                  j = 0..7 ascending (lane l owns 8-element chunks; l = 0..63)
 *   butterfly      for off in 32,16,8,4,2,1:  p'[l] = p[l] + p[l ^ off]
 * IEEE addition is commutative, so every lane ends with the same value; lane 0 is used.
 *
 * Parity pins (what checks each function; see tests/test_oracle.py):
 *   oracle_fp4_value / oracle_e8m0_scale / dequant: the reference KATs of
 *     tests/mxfp4_dequant_tests.rs:4-25, exhaustive 16 codes x 256 scale bytes against
 *     numpy.ldexp, and the e2m1 bit-field closed form.
 *   oracle_rmsnorm / oracle_router / oracle_route_logits: float64 brute force (tolerance) and
 *     the lane order restated with exact rational arithmetic in Python (bit-exact).
 *   oracle_topk_softmax: brute-force stable sort by (value desc, index asc); ties and
 *     -inf special cases; sum of weights.
 *   oracle_dispatch: permutation / histogram / stability invariants.
 *   oracle_moe_forward: float64 numpy brute force, the HF transformers GPT-OSS experts
 *     module (third-party implementation of the same layer), zero-weight residual
 *     invariant (tests/moe_basic_tests.rs:31-33), gate/up layout permutation invariance,
 *     hand-computed one-hot closed forms.
 *   oracle_round_bf16: brute-force nearest bf16 value (ties to the even significand) over
 *     random, boundary and tie inputs.
 *   oracle_moe_forward with bf16_rows: the same forward on rows and SwiGLU outputs rounded by
 *     oracle_round_bf16 beforehand (bit-exact), and the default forward within the bf16 bar.
 *   oracle_moe_forward_reference: agrees with oracle_moe_forward (halves layout) where
 *     the reference's b2-per-f-tile quirk is inactive (F <= 256), and differs by exactly
 *     (ceil(F/256)-1) * sum_p w_p*b2 when it is active.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_OK 0
#define ORACLE_INVALID 1

/* e2m1 magnitudes indexed by nibble; index 8 is -0.0 (src/loader/mxfp4.rs:10-13). */
static const float FP4_VALUES[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                     -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

float oracle_fp4_value(int nib) { return FP4_VALUES[nib & 15]; }

/* 2^(s-127) as the reference's (2.0f32).powi(s - 127) produces it (src/loader/mxfp4.rs:58):
 * exact for s in 0..254 (s = 0 gives the subnormal 2^-127); s = 255 overflows to +inf. */
float oracle_e8m0_scale(int s) { return ldexpf(1.0f, (s & 255) - 127); }

/* Reference test helper form: one scale byte per row of `b` packed bytes
 * (src/loader/mxfp4.rs:56-79).  out has rows * 2b floats. */
void oracle_dequant_mxfp4_bytes(const uint8_t *blocks, const uint8_t *scales, int64_t rows, int64_t b,
                                float *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float sc = oracle_e8m0_scale(scales[r]);
    for (int64_t i = 0; i < b; ++i) {
      const uint8_t byte = blocks[r * b + i];
      out[r * 2 * b + 2 * i] = FP4_VALUES[byte & 15] * sc;
      out[r * 2 * b + 2 * i + 1] = FP4_VALUES[byte >> 4] * sc;
    }
  }
}

/* Matrix form used by the kernels: [rows, cols] with bpr bytes and gpr scale groups per row
 * (src/quant/gpu.rs:124-131).  Scale bytes are stored with `ue8_offset` added mod 256
 * (src/bin/gptoss_export.rs:562); the true exponent byte is (stored - ue8_offset) mod 256. */
void oracle_dequant_matrix(const uint8_t *blocks, const uint8_t *scales, int64_t rows, int64_t cols, int64_t bpr,
                           int64_t gpr, int ue8_offset, float *out) {
  float sct[256];
  for (int s = 0; s < 256; ++s) sct[s] = oracle_e8m0_scale(s);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      const uint8_t byte = blocks[r * bpr + (c >> 1)];
      const int nib = (c & 1) ? (byte >> 4) : (byte & 15);
      const int s = ((int)scales[r * gpr + (c >> 5)] - ue8_offset) & 255;
      out[r * cols + c] = FP4_VALUES[nib] * sct[s];
    }
  }
}

/* One 64-lane dot product in the GPU route kernel's order (see header). */
static float lane_dot(const float *a, const float *b, int64_t n) {
  float p[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int64_t c0 = 8 * l; c0 < n; c0 += 512)
      for (int64_t c = c0; c < c0 + 8 && c < n; ++c) acc = fmaf(a[c], b[c], acc);
    p[l] = acc;
  }
  for (int off = 32; off >= 1; off >>= 1) {
    float q[64];
    for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ off];
    memcpy(p, q, sizeof(p));
  }
  return p[0];
}

/* Burn RmsNorm (src/moe/mod.rs:109): xn = (x / sqrt(mean(x^2) + eps)) * gamma.
 * gamma may be NULL (ones, the RmsNormConfig::init value). */
void oracle_rmsnorm(const float *x, int64_t n, int64_t d, const float *gamma, float eps, float *xn) {
  for (int64_t t = 0; t < n; ++t) {
    const float *xr = x + t * d;
    const float ss = lane_dot(xr, xr, d);
    const float ms = ss / (float)d;
    const float r = sqrtf(ms + eps);
    for (int64_t c = 0; c < d; ++c) {
      const float g = gamma ? gamma[c] : 1.0f;
      xn[t * d + c] = (xr[c] / r) * g;
    }
  }
}

/* Router Linear (src/moe/mod.rs:110): logits[t,e] = dot(xn[t], W[e]) + b[e]; W is [E, D]
 * (model.bin orientation, src/loader/modelbin.rs:286-291).  b may be NULL. */
void oracle_router(const float *xn, int64_t n, int64_t d, const float *w, const float *b, int64_t e,
                   float *logits) {
  for (int64_t t = 0; t < n; ++t)
    for (int64_t j = 0; j < e; ++j) {
      const float s = lane_dot(xn + t * d, w + j * d, d);
      logits[t * e + j] = s + (b ? b[j] : 0.0f);
    }
}

/* Routing logits as the GPU router computes them.  With apply_rmsnorm the normalisation is
 * applied after the dot product:
 *   r_t = sqrt(lane_dot(x_t, x_t) / D + eps)          (Burn RmsNorm denominator)
 *   logit[t,e] = lane_dot(x_t, gw_e) / r_t + b[e],    gw_e[c] = gamma[c] * W[e,c] (f32)
 * which equals Linear(RmsNorm(x)) (src/moe/mod.rs:109-110) up to f32 rounding (Burn's own
 * order is unpinned); gamma NULL means ones, and then gw_e = W[e] exactly.  Without
 * apply_rmsnorm: logit[t,e] = lane_dot(x_t, W[e]) + b[e]. */
void oracle_route_logits(const float *x, int64_t n, int64_t d, const float *gamma, float eps, int apply_rmsnorm,
                         const float *w, const float *b, int64_t e, float *logits) {
  float *gw = (float *)malloc(sizeof(float) * (size_t)(d > 0 ? d : 1));
  float *r = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  /* r_t once per token (the same bits every expert's logit would recompute) */
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < n; ++t) r[t] = apply_rmsnorm ? sqrtf(lane_dot(x + t * d, x + t * d, d) / (float)d + eps) : 1.0f;
  for (int64_t j = 0; j < e; ++j) {
    for (int64_t c = 0; c < d; ++c) gw[c] = (apply_rmsnorm && gamma) ? gamma[c] * w[j * d + c] : w[j * d + c];
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < n; ++t) {
      const float u = lane_dot(x + t * d, gw, d);
      const float lgt = apply_rmsnorm ? u / r[t] : u;
      logits[t * e + j] = lgt + (b ? b[j] : 0.0f);
    }
  }
  free(r);
  free(gw);
}

/* Strict total order used for selection: larger value first, NaN below everything,
 * equal values (including -0 == +0) broken by the lower expert index. */
static int beats(float va, int ia, float vb, int ib) {
  const int na = isnan(va), nb = isnan(vb);
  if (na || nb) {
    if (na && nb) return ia < ib;
    return nb;
  }
  if (va > vb) return 1;
  if (va < vb) return 0;
  return ia < ib;
}

/* top-k then softmax over the selected logits (src/moe/mod.rs:271-276):
 *   w_p = exp(v_p - v_0) / sum_q exp(v_q - v_0), sum taken q ascending.
 * k = min(max(k,1), E) as at src/moe/mod.rs:133. */
void oracle_topk_softmax(const float *logits, int64_t n, int64_t e, int64_t k, int32_t *idx, float *w) {
  if (k < 1) k = 1;
  if (k > e) k = e;
  unsigned char *taken = (unsigned char *)malloc((size_t)e);
  float *ex = (float *)malloc(sizeof(float) * (size_t)k);
  for (int64_t t = 0; t < n; ++t) {
    const float *lg = logits + t * e;
    memset(taken, 0, (size_t)e);
    for (int64_t p = 0; p < k; ++p) {
      int bi = -1;
      float bv = 0.0f;
      for (int64_t j = 0; j < e; ++j) {
        if (taken[j]) continue;
        if (bi < 0 || beats(lg[j], (int)j, bv, bi)) {
          bi = (int)j;
          bv = lg[j];
        }
      }
      taken[bi] = 1;
      idx[t * k + p] = bi;
    }
    const float m = lg[idx[t * k]];
    float s = 0.0f;
    for (int64_t p = 0; p < k; ++p) {
      ex[p] = expf(lg[idx[t * k + p]] - m);
      s += ex[p];
    }
    for (int64_t p = 0; p < k; ++p) w[t * k + p] = ex[p] / s;
  }
  free(taken);
  free(ex);
}

/* Dispatch into expert-contiguous segments (no reference counterpart: the reference masks
 * densely per expert, src/moe/mod.rs:279-288).  seg_off[E+1] is the exclusive scan of the
 * histogram; inside a segment entries are ordered by token ascending (stable counting sort of
 * the flat entry id t*k+p).  perm[pos] = t*k+p, pos_of[t*k+p] = pos. */
void oracle_dispatch(const int32_t *idx, int64_t n, int64_t k, int64_t e, int32_t *seg_off, int32_t *perm,
                     int32_t *pos_of) {
  int32_t *cur = (int32_t *)calloc((size_t)e + 1, sizeof(int32_t));
  memset(seg_off, 0, sizeof(int32_t) * (size_t)(e + 1));
  for (int64_t i = 0; i < n * k; ++i) seg_off[idx[i] + 1] += 1;
  for (int64_t j = 0; j < e; ++j) seg_off[j + 1] += seg_off[j];
  for (int64_t j = 0; j < e; ++j) cur[j] = seg_off[j];
  for (int64_t i = 0; i < n * k; ++i) {
    const int32_t pos = cur[idx[i]]++;
    perm[pos] = (int32_t)i;
    pos_of[i] = pos;
  }
  free(cur);
}

/* Clamped GPT-OSS SwiGLU (src/activation/mod.rs:5-12, src/quant/gpu.rs:140-145). */
float oracle_swiglu(float g, float l, float alpha, float limit) {
  const float xg = fminf(g, limit);
  const float xl = fmaxf(-limit, fminf(l, limit));
  const float sig = 1.0f / (1.0f + expf(-alpha * xg));
  return (xg * sig) * (xl + 1.0f);
}

typedef struct {
  int64_t d, f, e, k;
  float alpha, limit, eps;
  int64_t bf16_rows; /* 1: the expert products take the normalised rows and the SwiGLU outputs
                        rounded to bf16 (the device's one-term option; no counterpart in the
                        reference, which multiplies f32 rows) */
} oracle_cfg;

/* Nearest bf16 value of v (ties to the even significand; NaN stays NaN): f32 bits + 0x7FFF + the
 * lowest kept bit, truncated to the top 16 bits. */
float oracle_round_bf16(float v) {
  uint32_t u;
  memcpy(&u, &v, sizeof u);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u)
    u = (u | 0x00400000u) & 0xFFFF0000u;
  else
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  memcpy(&v, &u, sizeof v);
  return v;
}

/* W1 source row that holds the gate (lin = 0) or linear (lin = 1) half of feature f.
 * layout 0 = halves ([0,F) gate, [F,2F) linear: src/quant/gpu.rs:112-113 / src/moe/mod.rs:336-337),
 * layout 1 = interleaved (even gate, odd linear: src/activation/mod.rs:5-12, GPT-OSS checkpoints). */
static int64_t w1_row(int layout, int64_t f, int lin, int64_t F) {
  return layout == 1 ? 2 * f + lin : f + (lin ? F : 0);
}

/* Dequantised element of one expert's matrix (exact; see oracle_dequant_matrix). */
static float SCALE_TABLE[256];
static int scale_table_ready = 0;
static void init_scale_table(void) {
  if (scale_table_ready) return;
  for (int s = 0; s < 256; ++s) SCALE_TABLE[s] = oracle_e8m0_scale(s);
  scale_table_ready = 1;
}
static inline float deq(const uint8_t *blocks, const uint8_t *scales, int64_t row, int64_t c, int64_t bpr,
                        int64_t gpr, int ue8) {
  const uint8_t byte = blocks[row * bpr + (c >> 1)];
  const int nib = (c & 1) ? (byte >> 4) : (byte & 15);
  const int s = ((int)scales[row * gpr + (c >> 5)] - ue8) & 255;
  return FP4_VALUES[nib] * SCALE_TABLE[s];
}

/*
 * The build's layer semantics (what burnext_moe_forward computes), f32 throughout:
 *   xn  = apply_rmsnorm ? RmsNorm(x) : x
 *   top-k / softmax as above
 *   for each (t, p), e = idx[t,p]:
 *     g_f = sum_{c asc} xn[t,c]*W1[e, gate_row(f), c] + b1[e, gate_row(f)]   (mul then add,
 *     l_f likewise on the linear row, as `sum_g += inp * w_g` in src/quant/gpu.rs:135-139)
 *     a_f = swiglu(g_f, l_f)
 *     o_d = sum_{f asc} a_f * W2[e, d, f]
 *     acc_d += (o_d + b2[e,d]) * w[t,p]       (p ascending; b2 added once)
 *   y = (add_residual ? x : 0) + acc
 * Weights are in the on-disk/resident form: W1 [E, 2F, bpr1] bytes + [E, 2F, gpr1] scales,
 * W2 [E, D, bpr2] + [E, D, gpr2]; biases f32 [E, 2F] (same row order as W1) and [E, D].
 * Routing inputs are the RMS-normed activations; idx_out / w_out (nullable) receive routing.
 */
int oracle_moe_forward(const float *x, int64_t n, const oracle_cfg *cfg, const uint8_t *w1b, const uint8_t *w1s,
                       const uint8_t *w2b, const uint8_t *w2s, int ue8_offset, const float *b1, const float *b2,
                       const float *router_w, const float *router_b, const float *gamma, int layout,
                       int apply_rmsnorm, int add_residual, float *y, int32_t *idx_out, float *w_out) {
  const int64_t D = cfg->d, F = cfg->f, E = cfg->e;
  int64_t K = cfg->k;
  if (K < 1) K = 1;
  if (K > E) K = E;
  if (D <= 0 || F <= 0 || E <= 0 || n < 0) return ORACLE_INVALID;
  const int64_t bpr1 = (D + 1) / 2, gpr1 = (D + 31) / 32, bpr2 = (F + 1) / 2, gpr2 = (F + 31) / 32;
  float *xn = (float *)malloc(sizeof(float) * (size_t)(n * D + 1));
  float *lg = (float *)malloc(sizeof(float) * (size_t)(n * E + 1));
  int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n * K + 1));
  float *wt = (float *)malloc(sizeof(float) * (size_t)(n * K + 1));
  /* per-slot expert outputs (o + b2) * w, summed per token in slot order afterwards */
  float *slot = (float *)malloc(sizeof(float) * (size_t)(n * K * D + 1));
  float *W1 = (float *)malloc(sizeof(float) * (size_t)(2 * F * D));
  float *W2 = (float *)malloc(sizeof(float) * (size_t)(D * F));
  float *act = (float *)malloc(sizeof(float) * (size_t)F);
  if (apply_rmsnorm)
    oracle_rmsnorm(x, n, D, gamma, cfg->eps, xn);
  else
    memcpy(xn, x, sizeof(float) * (size_t)(n * D));
  if (cfg->bf16_rows)  /* xn feeds only the expert products: routing reads x */
    for (int64_t i = 0; i < n * D; ++i) xn[i] = oracle_round_bf16(xn[i]);
  oracle_route_logits(x, n, D, gamma, cfg->eps, apply_rmsnorm, router_w, router_b, E, lg);
  oracle_topk_softmax(lg, n, E, K, idx, wt);
  for (int64_t e = 0; e < E; ++e) {
    int used = 0;
    for (int64_t i = 0; i < n * K; ++i) used |= idx[i] == e;
    if (!used) continue;
    /* exact dequantisation of the expert (values identical to deq() element by element) */
    oracle_dequant_matrix(w1b + e * 2 * F * bpr1, w1s + e * 2 * F * gpr1, 2 * F, D, bpr1, gpr1, ue8_offset, W1);
    oracle_dequant_matrix(w2b + e * D * bpr2, w2s + e * D * gpr2, D, F, bpr2, gpr2, ue8_offset, W2);
    for (int64_t i = 0; i < n * K; ++i) {
      if (idx[i] != e) continue;
      const int64_t t = i / K;
      const float *xr = xn + t * D;
#pragma omp parallel for schedule(static)
      for (int64_t f = 0; f < F; ++f) {
        const int64_t rg = w1_row(layout, f, 0, F), rl = w1_row(layout, f, 1, F);
        const float *wg = W1 + rg * D, *wl = W1 + rl * D;
        float sg = 0.0f, sl = 0.0f;
        for (int64_t c = 0; c < D; ++c) {
          const float pg = xr[c] * wg[c];
          const float pl = xr[c] * wl[c];
          sg = sg + pg;
          sl = sl + pl;
        }
        sg = sg + b1[e * 2 * F + rg];
        sl = sl + b1[e * 2 * F + rl];
        const float a = oracle_swiglu(sg, sl, cfg->alpha, cfg->limit);
        act[f] = cfg->bf16_rows ? oracle_round_bf16(a) : a;
      }
      const float wp = wt[i];
      float *so = slot + i * D;
#pragma omp parallel for schedule(static)
      for (int64_t dd = 0; dd < D; ++dd) {
        const float *w2r = W2 + dd * F;
        float s = 0.0f;
        for (int64_t f = 0; f < F; ++f) {
          const float pr = act[f] * w2r[f];
          s = s + pr;
        }
        so[dd] = (s + b2[e * D + dd]) * wp;
      }
    }
  }
  for (int64_t t = 0; t < n; ++t)
    for (int64_t dd = 0; dd < D; ++dd) {
      float acc = 0.0f;
      for (int64_t p = 0; p < K; ++p) acc = acc + slot[(t * K + p) * D + dd];
      y[t * D + dd] = (add_residual ? x[t * D + dd] : 0.0f) + acc;
    }
  if (idx_out) memcpy(idx_out, idx, sizeof(int32_t) * (size_t)(n * K));
  if (w_out) memcpy(w_out, wt, sizeof(float) * (size_t)(n * K));
  free(xn);
  free(lg);
  free(idx);
  free(wt);
  free(slot);
  free(W1);
  free(W2);
  free(act);
  return ORACLE_OK;
}

/*
 * Literal restatement of the reference algorithm MoeGatedSwiGLU::forward_resident
 * (src/moe/mod.rs:129-411 with the kernels of src/quant/gpu.rs:89-192), used as the CPU
 * baseline and to quantify the reference's b2 quirk.  Follows its loop structure:
 *   token tiles of 256 (:263); for each expert e in 0..E used in the tile (:279-288):
 *     f-tiles of 256 (:316-317); K1 over ALL tile tokens (no routing filter,
 *     gpu.rs:120-136) with the halves row pairing row_g = f, row_l = F + f (:336-337) and the
 *     hard-coded alpha 1.702 / limit 7 (gpu.rs:140-141); K2 over tokens with w != 0
 *     (gpu.rs:171) adding (sum + b2) * w for every f-tile (gpu.rs:191: b2 once per f-tile);
 *     acc_tile += ex_tile_sum (:405)
 *   y = x + acc (:411)
 * Scales use the exact 2^(s-127) (not the kernel's exp(.. * ln2)), s = stored - ue8_offset
 * mod 256.  b2_per_ftile = 1 reproduces the reference's b2-per-f-tile quirk; 0 adds b2 in the
 * first f-tile only (bias once, as GPT-OSS defines the layer).  Routing as oracle_moe_forward.  The gate_up layout argument is not taken: the
 * reference kernel always pairs halves.  OpenMP parallelises the (token, f) and (token, d)
 * grids as the reference's launch grids do.
 */
int oracle_moe_forward_reference(const float *x, int64_t n, const oracle_cfg *cfg, const uint8_t *w1b,
                                 const uint8_t *w1s, const uint8_t *w2b, const uint8_t *w2s, int ue8_offset,
                                 const float *b1, const float *b2, const float *router_w, const float *router_b,
                                 const float *gamma, int b2_per_ftile, float *y) {
  const int64_t D = cfg->d, F = cfg->f, E = cfg->e;
  int64_t K = cfg->k;
  if (K < 1) K = 1;
  if (K > E) K = E;
  if (D <= 0 || F <= 0 || E <= 0 || n < 0) return ORACLE_INVALID;
  const int64_t bpr1 = (D + 1) / 2, gpr1 = (D + 31) / 32, bpr2 = (F + 1) / 2, gpr2 = (F + 31) / 32;
  float *xn = (float *)malloc(sizeof(float) * (size_t)(n * D + 1));
  float *lg = (float *)malloc(sizeof(float) * (size_t)(n * E + 1));
  int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n * K + 1));
  float *wt = (float *)malloc(sizeof(float) * (size_t)(n * K + 1));
  init_scale_table();
  oracle_rmsnorm(x, n, D, gamma, cfg->eps, xn);
  oracle_route_logits(x, n, D, gamma, cfg->eps, 1, router_w, router_b, E, lg);
  oracle_topk_softmax(lg, n, E, K, idx, wt);
  const int64_t tile_n = n < 256 ? (n < 1 ? 1 : n) : 256;
  const int64_t tile_f = F < 256 ? F : 256;
  float *act = (float *)malloc(sizeof(float) * (size_t)(tile_n * tile_f));
  float *ex_sum = (float *)malloc(sizeof(float) * (size_t)(tile_n * D));
  float *acc_tile = (float *)malloc(sizeof(float) * (size_t)(tile_n * D));
  float *we = (float *)malloc(sizeof(float) * (size_t)tile_n);
  for (int64_t s0 = 0; s0 < n; s0 += tile_n) {
    const int64_t tn = (n - s0) < tile_n ? (n - s0) : tile_n;
    memset(acc_tile, 0, sizeof(float) * (size_t)(tn * D));
    for (int64_t e = 0; e < E; ++e) {
      float used = 0.0f;
      for (int64_t r = 0; r < tn; ++r) {
        float s = 0.0f;
        for (int64_t p = 0; p < K; ++p) s += (idx[(s0 + r) * K + p] == e) ? wt[(s0 + r) * K + p] : 0.0f;
        we[r] = s;
        used += s;
      }
      if (used == 0.0f) continue;
      const uint8_t *eb1 = w1b + e * 2 * F * bpr1, *es1 = w1s + e * 2 * F * gpr1;
      const uint8_t *eb2 = w2b + e * D * bpr2, *es2 = w2s + e * D * gpr2;
      memset(ex_sum, 0, sizeof(float) * (size_t)(tn * D));
      for (int64_t f0 = 0; f0 < F; f0 += tile_f) {
        const int64_t tf = (F - f0) < tile_f ? (F - f0) : tile_f;
#pragma omp parallel for collapse(2) schedule(static)
        for (int64_t r = 0; r < tn; ++r)
          for (int64_t fr = 0; fr < tf; ++fr) {
            const int64_t rg = f0 + fr, rl = F + f0 + fr;
            float sg = 0.0f, sl = 0.0f;
            for (int64_t c = 0; c < D; ++c) {
              const float xv = xn[(s0 + r) * D + c];
              sg += xv * deq(eb1, es1, rg, c, bpr1, gpr1, ue8_offset);
              sl += xv * deq(eb1, es1, rl, c, bpr1, gpr1, ue8_offset);
            }
            sg += b1[e * 2 * F + rg];
            sl += b1[e * 2 * F + rl];
            act[r * tf + fr] = oracle_swiglu(sg, sl, 1.702f, 7.0f);
          }
#pragma omp parallel for collapse(2) schedule(static)
        for (int64_t r = 0; r < tn; ++r)
          for (int64_t dd = 0; dd < D; ++dd) {
            if (we[r] == 0.0f) continue;
            float s = 0.0f;
            for (int64_t fr = 0; fr < tf; ++fr) s += act[r * tf + fr] * deq(eb2, es2, dd, f0 + fr, bpr2, gpr2, ue8_offset);
            const float bias = (b2_per_ftile || f0 == 0) ? b2[e * D + dd] : 0.0f;
            ex_sum[r * D + dd] = ex_sum[r * D + dd] + (s + bias) * we[r];
          }
      }
      for (int64_t i = 0; i < tn * D; ++i) acc_tile[i] = acc_tile[i] + ex_sum[i];
    }
    for (int64_t r = 0; r < tn; ++r)
      for (int64_t dd = 0; dd < D; ++dd) y[(s0 + r) * D + dd] = x[(s0 + r) * D + dd] + acc_tile[r * D + dd];
  }
  free(act);
  free(ex_sum);
  free(acc_tile);
  free(we);
  free(xn);
  free(lg);
  free(idx);
  free(wt);
  return ORACLE_OK;
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
