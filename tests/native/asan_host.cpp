// asan_host.cpp -- AddressSanitizer / UndefinedBehaviorSanitizer driver of the library's host code.
//
// Built by burn-extended_amd/build.py (build_asan: the library sources with the host half
// instrumented, device code unchanged) and run by tests/test_asan.py.  It drives the public C ABI
// only (include/burnext_moe.h, include/burnext_gptoss.h):
//  - always: every create on small and ragged shapes (odd widths, partial scale groups, both gate_up
//    layouts, f32 / bf16 tensors, scale offsets, with and without gamma / sinks / YaRN), which runs
//    the whole host preparation (MXFP4 repack, bias permutation, gamma folding, dense tiling, RoPE
//    table) before the device is touched, and the argument checks of every entry point;
//  - with a HIP device: the same layers created, workspace sizes for 1..64 tokens, forwards at
//    decode and mid sizes in both activation dtypes, route / dispatch / route_dispatch, the
//    no-allocation forward, dequant, and a decoder decoding past cache eviction.
// Prints "asan host ok" and returns 0 when every status matched.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "burnext_gptoss.h"
#include "burnext_moe.h"

namespace {

uint64_t g_rng = 0x2545F4914F6CDD1Dull;
uint32_t rnd() {
  g_rng ^= g_rng << 13;
  g_rng ^= g_rng >> 7;
  g_rng ^= g_rng << 17;
  return (uint32_t)(g_rng >> 16);
}
float frand(float s) { return ((float)(rnd() % 20001) / 10000.0f - 1.0f) * s; }
uint16_t bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
std::vector<uint8_t> bytes(size_t n, int lo, int hi) {
  std::vector<uint8_t> v(n);
  for (auto &b : v) b = (uint8_t)(lo + (int)(rnd() % (uint32_t)(hi - lo + 1)));
  return v;
}
std::vector<float> floats(size_t n, float s) {
  std::vector<float> v(n);
  for (auto &x : v) x = frand(s);
  return v;
}
std::vector<uint16_t> halves(size_t n, float s, float mean = 0.0f) {
  std::vector<uint16_t> v(n);
  for (auto &x : v) x = bf16(mean + frand(s));
  return v;
}

int g_fail = 0;
void expect(burnext_status got, burnext_status want, const char *what) {
  if (got != want) {
    fprintf(stderr, "FAIL %s: status %d, expected %d (%s)\n", what, (int)got, (int)want, burnext_last_error());
    ++g_fail;
  }
}

struct HostLayer {
  burnext_moe_config cfg{};
  burnext_mxfp4_desc d1{}, d2{};
  std::vector<uint8_t> w1b, w1s, w2b, w2s;
  std::vector<float> b1f, b2f, rwf, rbf, gf;
  std::vector<uint16_t> b1h, b2h, rwh, rbh, gh;
  int ue8 = 0;
};

HostLayer make_layer(uint32_t D, uint32_t F, uint32_t E, uint32_t K, int ue8) {
  HostLayer h;
  h.cfg = {D, F, E, K, 1.702f, 7.0f, 1e-5f, 0};
  h.ue8 = ue8;
  h.d1 = {E, 2ull * F, D, (D + 1ull) / 2, (D + 31ull) / 32, ue8};
  h.d2 = {E, D, F, (F + 1ull) / 2, (F + 31ull) / 32, ue8};
  h.w1b = bytes(E * h.d1.rows * h.d1.bpr, 0, 255);
  h.w1s = bytes(E * h.d1.rows * h.d1.gpr, 119 + ue8, 123 + ue8);
  h.w2b = bytes(E * h.d2.rows * h.d2.bpr, 0, 255);
  h.w2s = bytes(E * h.d2.rows * h.d2.gpr, 119 + ue8, 123 + ue8);
  h.b1f = floats((size_t)E * 2 * F, 0.01f);
  h.b2f = floats((size_t)E * D, 0.01f);
  h.rwf = floats((size_t)E * D, 0.05f);
  h.rbf = floats(E, 0.1f);
  h.gf = floats(D, 0.1f);
  for (auto &g : h.gf) g += 1.0f;
  for (float v : h.b1f) h.b1h.push_back(bf16(v));
  for (float v : h.b2f) h.b2h.push_back(bf16(v));
  for (float v : h.rwf) h.rwh.push_back(bf16(v));
  for (float v : h.rbf) h.rbh.push_back(bf16(v));
  for (float v : h.gf) h.gh.push_back(bf16(v));
  return h;
}

burnext_status create(const HostLayer &h, bool bf16_tensors, bool gamma, burnext_gate_up_layout layout,
                      burnext_moe_layer_t *out) {
  const burnext_dtype dt = bf16_tensors ? BURNEXT_BF16 : BURNEXT_F32;
  const void *b1 = bf16_tensors ? (const void *)h.b1h.data() : (const void *)h.b1f.data();
  const void *b2 = bf16_tensors ? (const void *)h.b2h.data() : (const void *)h.b2f.data();
  const void *rw = bf16_tensors ? (const void *)h.rwh.data() : (const void *)h.rwf.data();
  const void *rb = bf16_tensors ? (const void *)h.rbh.data() : (const void *)h.rbf.data();
  const void *g = !gamma ? nullptr : (bf16_tensors ? (const void *)h.gh.data() : (const void *)h.gf.data());
  return burnext_moe_layer_create(&h.cfg, &h.d1, h.w1b.data(), h.w1s.data(), &h.d2, h.w2b.data(), h.w2s.data(), b1,
                                  b2, dt, rw, rb, dt, g, dt, layout, 0, out);
}

template <typename T>
T *dev_alloc(size_t n) {
  void *p = nullptr;
  if (hipMalloc(&p, n * sizeof(T) + 256) != hipSuccess) return nullptr;
  (void)hipMemset(p, 0, n * sizeof(T) + 256);
  return (T *)p;
}

void moe_on_gpu(burnext_moe_layer_t L, const HostLayer &h) {
  const uint32_t D = h.cfg.d_model, E = h.cfg.num_experts, K = std::min(h.cfg.experts_per_token, E);
  uint64_t prev = 0;
  for (uint64_t n = 1; n <= 64; ++n) {
    uint64_t b = 0;
    expect(burnext_moe_workspace_size(L, n, &b), BURNEXT_OK, "workspace_size");
    if (b < prev) {
      fprintf(stderr, "FAIL workspace_size decreases at n=%llu\n", (unsigned long long)n);
      ++g_fail;
    }
    prev = b;
  }
  const uint64_t nmax = 40;
  uint64_t wsb = 0;
  expect(burnext_moe_workspace_size(L, nmax, &wsb), BURNEXT_OK, "workspace_size 40");
  void *ws = dev_alloc<uint8_t>(wsb);
  float *x = dev_alloc<float>(nmax * D), *y = dev_alloc<float>(nmax * D);
  std::vector<float> hx = floats(nmax * D, 1.0f);
  (void)hipMemcpy(x, hx.data(), hx.size() * 4, hipMemcpyHostToDevice);
  int32_t *idx = dev_alloc<int32_t>(nmax * K), *seg = dev_alloc<int32_t>(E + 1), *perm = dev_alloc<int32_t>(nmax * K);
  float *w = dev_alloc<float>(nmax * K), *lg = dev_alloc<float>(nmax * E);
  for (uint64_t n : {1ull, 3ull, 16ull, 17ull, 40ull}) {
    for (int xb = 0; xb < 2; ++xb) {
      const burnext_dtype dt = xb ? BURNEXT_BF16 : BURNEXT_F32;
      expect(burnext_moe_forward(L, x, dt, y, n, BURNEXT_FORWARD_DEFAULT, ws, wsb, nullptr), BURNEXT_OK, "forward");
      expect(burnext_moe_forward(L, x, dt, y, n, 0, ws, wsb, nullptr), BURNEXT_OK, "forward no flags");
    }
    expect(burnext_moe_route(L, x, BURNEXT_F32, n, BURNEXT_APPLY_RMSNORM, idx, w, lg, ws, wsb, nullptr), BURNEXT_OK,
           "route");
    expect(burnext_moe_dispatch(L, idx, n, seg, perm, ws, wsb, nullptr), BURNEXT_OK, "dispatch");
    expect(burnext_moe_route_dispatch(L, x, BURNEXT_F32, n, BURNEXT_APPLY_RMSNORM, idx, w, seg, perm, ws, wsb,
                                      nullptr),
           BURNEXT_OK, "route_dispatch");
  }
  expect(burnext_moe_forward_noalloc(L, x, BURNEXT_F32, y, 2, BURNEXT_FORWARD_DEFAULT, nullptr), BURNEXT_OK, "noalloc");
  expect(burnext_moe_forward(L, x, BURNEXT_F32, y, nmax, BURNEXT_FORWARD_DEFAULT, ws, wsb - 1, nullptr),
         BURNEXT_WORKSPACE_TOO_SMALL, "small workspace");
  expect(burnext_moe_forward(L, x, BURNEXT_F32, x, 2, BURNEXT_FORWARD_DEFAULT, ws, wsb, nullptr), BURNEXT_INVALID_ARG,
         "aliasing");
  (void)hipDeviceSynchronize();
  for (void *p : {(void *)ws, (void *)x, (void *)y, (void *)idx, (void *)seg, (void *)perm, (void *)w, (void *)lg})
    (void)hipFree(p);
}

void moe_cases(bool gpu) {
  const uint32_t shapes[][5] = {{64, 64, 4, 2, 0}, {40, 72, 3, 2, 14}, {33, 17, 5, 3, 0}, {96, 48, 8, 8, 14}};
  for (const auto &s : shapes) {
    const HostLayer h = make_layer(s[0], s[1], s[2], s[3], (int)s[4]);
    for (int variant = 0; variant < 4; ++variant) {
      burnext_moe_layer_t L = nullptr;
      const burnext_status st = create(h, variant & 1, variant & 2,
                                       (variant & 1) ? BURNEXT_GATE_UP_HALVES : BURNEXT_GATE_UP_INTERLEAVED, &L);
      if (!gpu) {
        expect(st, BURNEXT_INVALID_ARG, "create without a device");
        if (!strstr(burnext_last_error(), "HIP device")) {
          fprintf(stderr, "FAIL create without a device: %s\n", burnext_last_error());
          ++g_fail;
        }
        continue;
      }
      expect(st, BURNEXT_OK, "create");
      if (st == BURNEXT_OK && variant == 0) moe_on_gpu(L, h);
      burnext_moe_layer_destroy(L);
    }
  }
  // argument checks
  HostLayer h = make_layer(64, 64, 4, 2, 0);
  burnext_moe_layer_t L = nullptr;
  expect(burnext_moe_layer_create(&h.cfg, &h.d1, nullptr, h.w1s.data(), &h.d2, h.w2b.data(), h.w2s.data(),
                                  h.b1f.data(), h.b2f.data(), BURNEXT_F32, h.rwf.data(), nullptr, BURNEXT_F32, nullptr,
                                  BURNEXT_F32, BURNEXT_GATE_UP_INTERLEAVED, 0, &L),
         BURNEXT_INVALID_ARG, "null blocks");
  burnext_mxfp4_desc bad = h.d1;
  bad.gpr += 1;
  expect(burnext_moe_layer_create(&h.cfg, &bad, h.w1b.data(), h.w1s.data(), &h.d2, h.w2b.data(), h.w2s.data(),
                                  h.b1f.data(), h.b2f.data(), BURNEXT_F32, h.rwf.data(), nullptr, BURNEXT_F32, nullptr,
                                  BURNEXT_F32, BURNEXT_GATE_UP_INTERLEAVED, 0, &L),
         BURNEXT_INVALID_ARG, "bad descriptor");
  uint64_t b = 0;
  expect(burnext_moe_workspace_size(nullptr, 8, &b), BURNEXT_INVALID_ARG, "null layer");
  expect(burnext_mxfp4_dequant(nullptr, nullptr, nullptr, nullptr, BURNEXT_F32, nullptr), BURNEXT_INVALID_ARG,
         "dequant null");
  if (gpu) {
    const uint64_t rows = 7, cols = 70;
    const burnext_mxfp4_desc d{1, rows, cols, (cols + 1) / 2, (cols + 31) / 32, 14};
    auto hb = bytes(rows * d.bpr, 0, 255), hs = bytes(rows * d.gpr, 0, 255);
    uint8_t *db = dev_alloc<uint8_t>(hb.size()), *ds = dev_alloc<uint8_t>(hs.size());
    float *out = dev_alloc<float>(rows * cols);
    (void)hipMemcpy(db, hb.data(), hb.size(), hipMemcpyHostToDevice);
    (void)hipMemcpy(ds, hs.data(), hs.size(), hipMemcpyHostToDevice);
    expect(burnext_mxfp4_dequant(&d, db, ds, out, BURNEXT_F32, nullptr), BURNEXT_OK, "dequant");
    expect(burnext_mxfp4_dequant(&d, db, ds, out, BURNEXT_BF16, nullptr), BURNEXT_OK, "dequant bf16");
    (void)hipDeviceSynchronize();
    (void)hipFree(db);
    (void)hipFree(ds);
    (void)hipFree(out);
  }
}

void decoder_cases(bool gpu) {
  struct Case {
    uint32_t V, D, L, nH, kvH, dk, B, cap, policy, window, full_on_even, stride, kv_bf16;
    float factor;
    bool sinks;
  };
  const Case cases[] = {{37, 40, 3, 4, 2, 16, 2, 5, 2, 3, 1, 1, 0, 32.0f, true},
                        {29, 64, 2, 8, 1, 8, 3, 70, 1, 2, 0, 0, 1, 1.0f, false},
                        {50, 32, 2, 2, 2, 32, 1, 6, 0, 1, 0, 1, 0, 32.0f, true}};
  for (const Case &k : cases) {
    burnext_gptoss_config c{};
    c.vocab_size = k.V;
    c.d_model = k.D;
    c.n_layers = k.L;
    c.n_heads = k.nH;
    c.kv_heads = k.kvH;
    c.head_dim = k.dk;
    c.max_batch = k.B;
    c.cache_len = k.cap;
    c.window_policy = k.policy;
    c.window = k.window;
    c.full_on_even = k.full_on_even;
    c.rope_head_stride = k.stride;
    c.max_positions = k.cap + 8;
    c.kv_bf16 = k.kv_bf16;
    c.rms_eps = 1e-5f;
    c.rope_theta = 150000.0f;
    c.rope_scaling_factor = k.factor;
    c.rope_initial_context = 4096.0f;
    c.rope_ntk_alpha = 1.0f;
    c.rope_ntk_beta = 32.0f;
    c.scale_dk = 1.0f;
    const uint32_t qd = k.nH * k.dk, kd = k.kvH * k.dk;
    auto emb = halves((size_t)k.V * k.D, 1.0f), na = halves((size_t)k.L * k.D, 0.1f, 1.0f);
    auto wq = halves((size_t)k.L * qd * k.D, 0.1f), bq = halves((size_t)k.L * qd, 0.1f);
    auto wk = halves((size_t)k.L * kd * k.D, 0.1f), bk = halves((size_t)k.L * kd, 0.1f);
    auto wv = halves((size_t)k.L * kd * k.D, 0.1f), bv = halves((size_t)k.L * kd, 0.1f);
    auto wo = halves((size_t)k.L * k.D * qd, 0.1f), bo = halves((size_t)k.L * k.D, 0.1f);
    auto sk = halves((size_t)k.L * k.nH, 0.5f), nf = halves(k.D, 0.1f, 1.0f), lm = halves((size_t)k.V * k.D, 0.1f);
    burnext_gptoss_weights w{emb.data(), na.data(), wq.data(), bq.data(), wk.data(), bk.data(), wv.data(),
                             bv.data(), wo.data(), bo.data(), k.sinks ? sk.data() : nullptr, nf.data(), lm.data()};
    std::vector<HostLayer> hl;
    std::vector<burnext_moe_layer_t> moe(k.L, nullptr);
    for (uint32_t l = 0; l < k.L; ++l) hl.push_back(make_layer(k.D, 24 + 8 * l, 4, 2, 0));
    if (!gpu) {
      // placeholders: create validates them for null, prepares everything on the host and stops
      // at the device check before it reads a handle
      for (uint32_t l = 0; l < k.L; ++l) moe[l] = (burnext_moe_layer_t)(uintptr_t)(0x1000 + l);
      burnext_gptoss_t m = nullptr;
      expect(burnext_gptoss_create(&c, &w, moe.data(), 0, &m), BURNEXT_INVALID_ARG, "decoder create without a device");
      if (!strstr(burnext_last_error(), "HIP device")) {
        fprintf(stderr, "FAIL decoder create without a device: %s\n", burnext_last_error());
        ++g_fail;
      }
      continue;
    }
    for (uint32_t l = 0; l < k.L; ++l) expect(create(hl[l], false, true, BURNEXT_GATE_UP_INTERLEAVED, &moe[l]), BURNEXT_OK, "moe create");
    burnext_gptoss_t m = nullptr;
    expect(burnext_gptoss_create(&c, &w, moe.data(), 0, &m), BURNEXT_OK, "decoder create");
    if (m) {
      uint64_t wsb = 0;
      expect(burnext_gptoss_workspace_size(m, k.B, &wsb), BURNEXT_OK, "decoder workspace");
      void *ws = dev_alloc<uint8_t>(wsb);
      int32_t *tok = dev_alloc<int32_t>(k.B), *nxt = dev_alloc<int32_t>(k.B);
      float *lg = dev_alloc<float>((size_t)k.B * k.V), *hid = dev_alloc<float>((size_t)k.B * k.D);
      const uint32_t pre = k.cap / 2;
      float *kc = dev_alloc<float>((size_t)k.L * k.B * pre * kd), *vc = dev_alloc<float>((size_t)k.L * k.B * pre * kd);
      expect(burnext_gptoss_cache_load(m, kc, vc, k.B, pre, nullptr), BURNEXT_OK, "cache_load");
      for (uint32_t p = pre; p < k.cap + 6; ++p)
        expect(burnext_gptoss_decode(m, tok, k.B, p, p % 3 == 0 ? 2 : 0, nxt, (p & 1) ? lg : nullptr,
                                     (p & 2) ? hid : nullptr, ws, wsb, nullptr),
               BURNEXT_OK, "decode");
      expect(burnext_gptoss_decode(m, tok, k.B, 0, 0, nxt, nullptr, nullptr, ws, wsb, nullptr), BURNEXT_INVALID_ARG,
             "decode wrong pos");
      expect(burnext_gptoss_reset(m), BURNEXT_OK, "reset");
      expect(burnext_gptoss_decode(m, tok, 1, 0, 0, nxt, lg, hid, ws, wsb, nullptr), BURNEXT_OK, "decode after reset");
      (void)hipDeviceSynchronize();
      for (void *p : {ws, (void *)tok, (void *)nxt, (void *)lg, (void *)hid, (void *)kc, (void *)vc}) (void)hipFree(p);
      burnext_gptoss_destroy(m);
    }
    for (auto *L : moe) burnext_moe_layer_destroy(L);
  }
  burnext_gptoss_t m = nullptr;
  expect(burnext_gptoss_create(nullptr, nullptr, nullptr, 0, &m), BURNEXT_INVALID_ARG, "decoder null config");
  expect(burnext_gptoss_decode(nullptr, nullptr, 1, 0, 0, nullptr, nullptr, nullptr, nullptr, 0, nullptr),
         BURNEXT_INVALID_ARG, "decode null model");
}

}  // namespace

int main() {
  int ndev = 0;
  const bool gpu = hipGetDeviceCount(&ndev) == hipSuccess && ndev > 0;
  printf("asan host: %s\n", gpu ? "HIP device present (host code of every entry point)" : "no HIP device (host preparation and argument checks)");
  moe_cases(gpu);
  decoder_cases(gpu);
  if (g_fail) {
    fprintf(stderr, "%d checks failed\n", g_fail);
    return 1;
  }
  printf("asan host ok\n");
  return 0;
}
