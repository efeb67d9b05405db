// layer.hip -- host side of the C ABI (include/burnext_moe.h): layer upload and repack,
// workspace layout, and the launch sequence of one MoE forward on a HIP stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../include/burnext_moe.h"
#include "kernels.hpp"

using namespace burnext;

namespace burnext {
thread_local LaunchTimer *g_launch_timer = nullptr;
}

namespace {

thread_local std::string g_last_error;

burnext_status fail(burnext_status st, const std::string &msg) {
  g_last_error = msg;
  return st;
}

burnext_status ok() {
  g_last_error.clear();
  return BURNEXT_OK;
}

inline uint64_t cdiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }
inline uint64_t align_up(uint64_t a, uint64_t b) { return cdiv(a, b) * b; }

float bf16_to_f32_host(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float read_scalar(const void *p, burnext_dtype dt, size_t i) {
  return dt == BURNEXT_BF16 ? bf16_to_f32_host(((const uint16_t *)p)[i]) : ((const float *)p)[i];
}

// Restores the caller's current device on scope exit.
struct DeviceGuard {
  int prev = -1;
  bool ok = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    ok = hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

// Timed dispatches of the profiling hook (process-wide: the previous dispatch on a stream may
// belong to another layer).  A dispatch queued behind a running kernel can take its begin stamp
// before that kernel ends, so a dispatch's time is the exclusive part of its interval:
// end - max(begin, end of the previous timed dispatch on the same stream).  Pairs read by a
// layer wait in `done` until the next enable finds nothing pending (a pending record may still
// refer to their end events), then return to the device's pool.
struct ProfRec {
  hipEvent_t a, b;      // dispatch begin / end
  hipEvent_t prev_end;  // end event of the previous timed dispatch on the same stream, or null
  const void *layer;
  int kernel, device;
};
struct Profiler {
  std::mutex mu;
  std::vector<ProfRec> pending;
  std::vector<ProfRec> done;
  std::map<int, std::vector<std::pair<hipEvent_t, hipEvent_t>>> pool;  // per device
  std::map<hipStream_t, hipEvent_t> last_end;
};
Profiler &profiler() {
  static Profiler *p = new Profiler;  // never destroyed: its events may outlive every layer
  return *p;
}

}  // namespace

namespace burnext {
// The thread's burnext_last_error() message, shared with the decoder entry points.
burnext_status set_error(burnext_status st, const std::string &msg) { return fail(st, msg); }
}  // namespace burnext

// Tiled MXFP4 layout of one projection (see the expert_gemv comment in kernels.hip).
struct TiledMx {
  uint32_t rows = 0, rows_p = 0, cols = 0, nb = 0, nrt = 0;
  uint64_t blocks_per_expert = 0, scales_per_expert = 0, gscales_per_expert = 0;
  uint8_t *blocks = nullptr, *scales = nullptr;
  // the grouped GEMM's copy of the scales: per group of 4 row tiles and block of 4 K-groups, lane
  // l's 16 bytes hold its scale byte of row tile 4 g + r and K-group 4 j + k at byte 4 r + k (one
  // 16-byte load per wave and 4 K-groups instead of 16 single-dword loads); zero where the row
  // tile or the block does not exist
  uint8_t *gscales = nullptr;
};

struct burnext_moe_layer {
  int device = 0;
  uint32_t D = 0, F = 0, E = 0, K = 0;
  float alpha = 1.702f, limit = 7.0f, eps = 1e-5f;
  bool disabled = false;
  uint32_t Dp = 0, Fp = 0;
  TiledMx w1, w2;
  float *b1 = nullptr;  // [E, w1.rows_p], interleaved (gate, linear) order
  float *b2 = nullptr;  // [E, w2.rows_p] (rows padded to the 16-row tile, zeros)
  void *router_w = nullptr;   // [E, D] as given (routing without RmsNorm)
  bool router_bf16 = false;
  void *router_wg = nullptr;  // [E, D] gamma-folded rows (routing with RmsNorm); may alias router_w
  bool router_wg_bf16 = false;
  float *router_b = nullptr;  // [E]
  float *gamma = nullptr;     // [D]
  int num_cus = 256;
  bool profiling = false;
};

namespace burnext {
// d_model and device of a MoE layer (the decoder checks them against its own at create).
void moe_layer_shape(const burnext_moe_layer *L, uint32_t *d_model, int *device) {
  *d_model = L->D;
  *device = L->device;
}
}  // namespace burnext

namespace {

// W1 internal row r (interleaved: even = gate, odd = linear) -> source row for `layout`.
inline uint32_t w1_src_row(uint32_t r, uint32_t F, burnext_gate_up_layout layout) {
  return layout == BURNEXT_GATE_UP_INTERLEAVED ? r : ((r & 1u) ? F + (r >> 1) : (r >> 1));
}

// Repacks one expert of a [rows, cols] MXFP4 matrix into the tiled layout.  Scale bytes are
// normalised to true e8m0 exponents ((stored - ue8_offset) mod 256, the inverse of the model.bin
// writer's wrapping add, reference src/bin/gptoss_export.rs:562).  Padding rows, columns and
// blocks are zero codes with scale byte 0.
void repack_expert(const uint8_t *src_b, const uint8_t *src_s, uint64_t bpr, uint64_t gpr, int ue8,
                   const TiledMx &t, bool is_w1, uint32_t F, burnext_gate_up_layout layout, uint8_t *dst_b,
                   uint8_t *dst_s) {
  const uint32_t nb = t.nb, nkg = (nb + 3) / 4;
  for (uint32_t rt = 0; rt < t.nrt; ++rt) {
    for (uint32_t kg = 0; kg < nkg; ++kg) {
      const uint32_t nbk = std::min(4u, nb - 4 * kg);
      for (uint32_t q = 0; q < nbk; ++q) {
        for (uint32_t i = 0; i < 16; ++i) {
          const uint32_t row = rt * 16 + i, blk = 4 * kg + q, lane = q * 16 + i;
          uint8_t *db = dst_b + (uint64_t)rt * nb * 256 + (uint64_t)kg * 1024 + (uint64_t)lane * 16;
          uint8_t *ds = dst_s + (uint64_t)rt * nb * 16 + (uint64_t)kg * 64 + lane;
          memset(db, 0, 16);
          *ds = 0;
          if (row >= t.rows) continue;
          const uint32_t sr = is_w1 ? w1_src_row(row, F, layout) : row;
          const uint8_t *rb = src_b + (uint64_t)sr * bpr;
          const uint64_t b0 = (uint64_t)blk * 16;
          for (uint64_t u = 0; u < 16 && b0 + u < bpr; ++u) {
            uint8_t byte = rb[b0 + u];
            const uint64_t c = 2 * (b0 + u);  // column of the low nibble
            if (c + 1 >= t.cols) byte &= 0x0F;
            if (c >= t.cols) byte = 0;
            db[u] = byte;
          }
          *ds = (uint8_t)(((int)src_s[(uint64_t)sr * gpr + blk] - ue8) & 255);
        }
      }
    }
  }
}

// Host half of the upload: geometry of t and the repacked bytes of all E experts (no device call,
// so create can prepare everything before it touches the GPU).
burnext_status repack_tiled(TiledMx &t, uint32_t E, uint32_t rows, uint32_t cols, const uint8_t *blocks,
                            const uint8_t *scales, const burnext_mxfp4_desc &d, bool is_w1, uint32_t F,
                            burnext_gate_up_layout layout, std::vector<uint8_t> &hb, std::vector<uint8_t> &hs,
                            std::vector<uint8_t> &hg) {
  t.rows = rows;
  t.rows_p = (uint32_t)align_up(rows, 16);
  t.cols = cols;
  t.nb = (uint32_t)cdiv(cols, 32);
  t.nrt = t.rows_p / 16;
  t.blocks_per_expert = (uint64_t)t.rows_p * t.nb * 16;
  t.scales_per_expert = (uint64_t)t.rows_p * t.nb;
  const uint32_t nkg = (t.nb + 3u) / 4u, nkq = (nkg + 3u) / 4u, ngr = (t.nrt + 3u) / 4u;
  t.gscales_per_expert = (uint64_t)ngr * nkq * 1024u;
  try {
    hb.resize(t.blocks_per_expert * E);
    hs.resize(t.scales_per_expert * E);
    hg.assign(t.gscales_per_expert * E, 0);
  } catch (const std::bad_alloc &) {
    return fail(BURNEXT_OUT_OF_MEMORY, "host allocation failed while repacking MXFP4 weights");
  }
  const uint64_t src_bpe = (uint64_t)rows * d.bpr, src_spe = (uint64_t)rows * d.gpr;
  const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  const unsigned nthr = std::min<unsigned>(hw, E);
  std::vector<std::thread> pool;
  for (unsigned w = 0; w < nthr; ++w) {
    pool.emplace_back([&, w]() {
      for (uint32_t e = w; e < E; e += nthr)
        repack_expert(blocks + e * src_bpe, scales + e * src_spe, d.bpr, d.gpr, d.ue8_offset, t, is_w1, F, layout,
                      hb.data() + e * t.blocks_per_expert, hs.data() + e * t.scales_per_expert);
    });
  }
  for (auto &th : pool) th.join();
  // the GEMM's scale copy, from the tiled scales (byte kg * 64 + l of row tile rt; lanes whose
  // block 4 kg + l / 16 is beyond nb stay zero)
  for (uint32_t e = 0; e < E; ++e) {
    const uint8_t *se = hs.data() + e * t.scales_per_expert;
    uint8_t *ge = hg.data() + e * t.gscales_per_expert;
    for (uint32_t rt = 0; rt < t.nrt; ++rt)
      for (uint32_t kg = 0; kg < nkg; ++kg)
        for (uint32_t l = 0; l < 64; ++l) {
          if (4u * kg + l / 16u >= t.nb) continue;
          const uint64_t dst = (((uint64_t)(rt / 4u) * nkq + kg / 4u) * 64u + l) * 16u + (rt % 4u) * 4u + kg % 4u;
          ge[dst] = se[(uint64_t)rt * t.nb * 16u + kg * 64u + l];
        }
  }
  return BURNEXT_OK;
}

burnext_status upload_tiled(TiledMx &t, const std::vector<uint8_t> &hb, const std::vector<uint8_t> &hs,
                            const std::vector<uint8_t> &hg) {
  if (hipMalloc(&t.blocks, hb.size()) != hipSuccess || hipMalloc(&t.scales, hs.size()) != hipSuccess ||
      hipMalloc(&t.gscales, hg.size()) != hipSuccess)
    return fail(BURNEXT_OUT_OF_MEMORY, "hipMalloc failed for MXFP4 weights");
  if (hipMemcpy(t.blocks, hb.data(), hb.size(), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(t.scales, hs.data(), hs.size(), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(t.gscales, hg.data(), hg.size(), hipMemcpyHostToDevice) != hipSuccess)
    return fail(BURNEXT_DEVICE_ERROR, "hipMemcpy of MXFP4 weights failed");
  return BURNEXT_OK;
}

template <typename T>
burnext_status upload_vec(T **dst, const std::vector<T> &v) {
  if (hipMalloc((void **)dst, std::max<size_t>(v.size(), 1) * sizeof(T)) != hipSuccess)
    return fail(BURNEXT_OUT_OF_MEMORY, "hipMalloc failed");
  if (!v.empty() && hipMemcpy(*dst, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
    return fail(BURNEXT_DEVICE_ERROR, "hipMemcpy failed");
  return BURNEXT_OK;
}

void free_layer(burnext_moe_layer *L) {
  if (!L) return;
  DeviceGuard g(L->device);
  if (L->router_wg == L->router_w) L->router_wg = nullptr;
  for (void *p : {(void *)L->w1.blocks, (void *)L->w1.scales, (void *)L->w1.gscales, (void *)L->w2.blocks,
                  (void *)L->w2.scales, (void *)L->w2.gscales,
                  (void *)L->b1, (void *)L->b2, L->router_w, L->router_wg, (void *)L->router_b, (void *)L->gamma})
    if (p) (void)hipFree(p);
  {  // its unread timed dispatches: their events stay (later records may refer to them)
    Profiler &P = profiler();
    std::lock_guard<std::mutex> lk(P.mu);
    for (size_t i = 0; i < P.pending.size();)
      if (P.pending[i].layer == L) {
        P.done.push_back(P.pending[i]);
        P.pending.erase(P.pending.begin() + (std::ptrdiff_t)i);
      } else {
        ++i;
      }
  }
  delete L;
}

bool check_desc(const burnext_mxfp4_desc *d, uint64_t E, uint64_t rows, uint64_t cols, const char *name,
                std::string &msg) {
  char buf[256];
  if (d->experts != E || d->rows != rows || d->cols != cols || d->bpr != cdiv(cols, 2) || d->gpr != cdiv(cols, 32) ||
      d->ue8_offset < 0 || d->ue8_offset > 255) {
    snprintf(buf, sizeof(buf),
             "%s descriptor {experts=%llu rows=%llu cols=%llu bpr=%llu gpr=%llu ue8_offset=%d} does not match "
             "expected {experts=%llu rows=%llu cols=%llu bpr=%llu gpr=%llu ue8_offset in [0,255]}",
             name, (unsigned long long)d->experts, (unsigned long long)d->rows, (unsigned long long)d->cols,
             (unsigned long long)d->bpr, (unsigned long long)d->gpr, d->ue8_offset, (unsigned long long)E,
             (unsigned long long)rows, (unsigned long long)cols, (unsigned long long)cdiv(cols, 2),
             (unsigned long long)cdiv(cols, 32));
    msg = buf;
    return false;
  }
  return true;
}

// Expert GEMV launch shape for n tokens: token rows staged per pass and the persistent grid (as
// many workgroups as stay resident: LDS-limited, at most 4 per CU, at least one per possible
// active expert; the kernel splits it among the active experts, gemv_share).
struct GemvCfg {
  uint32_t mt, grid, nrec;
};

bool gate_up_split(const burnext_moe_layer &L, uint64_t n);

GemvCfg gemv_cfg(const burnext_moe_layer &L, uint64_t n, int nt, bool gate_up) {
  const TiledMx &t = gate_up ? L.w1 : L.w2;
  GemvCfg c{};
  const size_t per_tok = gemv_lds_bytes(nt, 1, t.nb);
  // LDS rows reserved for one token pass (a segment with more tokens takes another pass over its
  // expert's weights): 8 at decode sizes and whenever routing leaves at most 4 tokens per expert on
  // average (3 workgroups per CU at D = 2880), else the most that still lets 2 workgroups share a
  // CU (14 at D = 2880), at most 16.  Memory parallelism beats the extra passes (measured, per
  // step: 120B T = 64 478 -> 373 us with 8 instead of 16; 20B T = 64 / 128 / 200 282 / 292 / 410
  // -> 192 / 243 / 335 us with 14 instead of 16).
  const uint64_t max_active = std::min<uint64_t>(L.E, n * L.K);
  c.nrec = (uint32_t)max_active;
  const bool small_segments = n <= 16 || n * L.K <= 4ull * L.E;
  // two-term (f32) activations at decode sizes: 4 rows per pass keep 3 workgroups per CU (8 rows
  // would leave one; segments beyond 4 tokens are rare there and take a second pass)
  uint32_t mt = (nt >= 2 && n <= 16) ? 4 : 8;
  if (!small_segments)
    for (mt = 16; mt > 8 && gemv_total_lds_bytes(nt, mt, t.nb, c.nrec) > 80 * 1024; --mt) {
    }
  mt = (uint32_t)std::min<uint64_t>(mt, n);
  c.mt = (uint32_t)std::min<size_t>(mt, std::max<size_t>(1, (96 * 1024) / per_tok));
  const size_t lds = gemv_launch_lds_bytes(nt, c.mt, t.nb, c.nrec, gate_up && gate_up_split(L, n));
  const uint64_t per_cu = std::max<uint64_t>(1, std::min<uint64_t>(4, (160 * 1024) / std::max<size_t>(lds, 1)));
  c.grid = (uint32_t)std::max<uint64_t>(max_active, std::min<uint64_t>((uint64_t)L.num_cus * per_cu, max_active * t.nrt));
  return c;
}

// Decode-sized batches that touch so few experts that their gate_up row tiles are fewer than 8 per
// CU (2/3 of a tile per wave) split every tile's K range in kGateUpSplit parts, one per wave of a
// workgroup: a wave then streams 6 instead of 23 K-groups at D = 2880 (120B T = 1: 4 experts, 1440
// row tiles for 3072 waves), and the workgroup sums the parts before the SwiGLU.
bool gate_up_split(const burnext_moe_layer &L, uint64_t n) {
  return n <= kSmallRouteMaxTokens && std::min<uint64_t>(L.E, n * L.K) * L.w1.nrt < 8ull * (uint64_t)L.num_cus &&
         (L.w1.nb + 3u) / 4u >= kGateUpSplit;
}

// Workspace carve-up for n tokens (every region 256-byte aligned).
struct WsLayout {
  uint64_t rms, logits, topk_idx, topk_w, meta, exrec, perm, pos_of, xn, act, ypart, dcnt, total;
  uint64_t tile_off, xq[4], aq[4];  // grouped-GEMM path: tile prefix, xq / act rows (hi lo shi slo)
  bool gemm;                        // the grouped-GEMM regions are present
};

// bf16 batches of at least kGemmMinTokens tokens with at least kGemmMinPerExpert routed tokens per
// expert on average run the grouped GEMM; the others, and every f32 batch (the GEMM's two activation
// terms carry about 2^-6 relative precision), run the expert GEMVs.  Measured per step (us, GEMV
// against GEMM, D = F = 2880, k = 4): E = 32: 145 / 147 at 32 tokens, 175 / 144 at 64, 239 / 155 at
// 128, 367 / 163 at 256; E = 128: 366 / 390 at 64, 469 / 439 at 128, 438 / 448 at 200, 455 / 461 at
// 256, 796 / 494 at 512.
constexpr uint64_t kGemmMinTokens = 64;
constexpr uint64_t kGemmMinPerExpert = 4;
inline bool use_gemm_path(const burnext_moe_layer &L, uint64_t n) {
  return n >= kGemmMinTokens && n * L.K >= kGemmMinPerExpert * L.E;
}

// Codes per row of the GEMM's activation rows over K = cols of a tiled projection (whole 128-wide
// K-groups): the hi term's bytes; the lo term takes half as many.
inline uint32_t qrow_bytes(const TiledMx &t) { return ((t.nb + 3u) / 4u) * 128u; }
// Scale bytes per row and term of those rows: one per 32 codes, rows padded to 16 bytes.
inline uint32_t qscale_bytes(const TiledMx &t) { return (uint32_t)align_up(qrow_bytes(t) / 32u, 16); }

// Largest batch m <= min(n, kSmallRouteMaxTokens) that still splits gate_up in K-parts (0: none).
// gate_up_split holds for m = 1 .. some bound, since the touched-expert bound min(E, m k) grows
// with m.
uint64_t max_split_tokens(const burnext_moe_layer &L, uint64_t n) {
  uint64_t ms = 0;
  for (uint64_t m = 1; m <= std::min<uint64_t>(n, kSmallRouteMaxTokens); ++m)
    if (gate_up_split(L, m)) ms = m;
  return ms;
}

// The experts of a decode-sized batch in one launch (moe_fused_kernel, opt-in by
// BURNEXT_FUSED_EXPERTS): batches of at most kSmallRouteMaxTokens tokens with top-k <= 8 whose
// geometry fits, except where the decoder fuses the next RmsNorm into the combine (post_norm).
// Sets g when it applies.
bool use_fused(const burnext_moe_layer &L, uint64_t n, int nt, bool post_norm, FusedGeom &g) {
  if (post_norm || n == 0 || n > kSmallRouteMaxTokens || L.K > 8u) return false;
  return fused_geometry(L.w1.nb, L.w2.nb, L.w2.nrt, L.Dp, (uint32_t)L.num_cus,
                        (uint32_t)std::min<uint64_t>(L.E, n * L.K), L.K, n, nt, g);
}

// Partial slot rows the fused kernel may write for a batch of m tokens (its most slices x m k),
// 0 when it does not apply (the slice cap does not depend on the activation terms).
uint64_t fused_rows(const burnext_moe_layer &L, uint64_t m) {
  FusedGeom g{};
  if (!use_fused(L, m, 1, false, g) && !use_fused(L, m, 2, false, g)) return 0;
  return (uint64_t)g.nsl_cap * m * L.K;
}

// Workspace regions for n tokens.  Every region is sized for the largest need of any batch of
// m <= n tokens, so burnext_moe_workspace_size(n) is non-decreasing in n and one workspace sized
// for the largest batch serves every smaller one: the K-part buffer of decode-sized batches
// (ypart in kDownSplitFew or kDownSplit parts) is larger per token than a bigger batch's
// single-part ypart.
WsLayout ws_layout(const burnext_moe_layer &L, uint64_t n) {
  WsLayout w{};
  uint64_t off = 0;
  auto take = [&](uint64_t bytes) {
    const uint64_t o = off;
    off = align_up(off + std::max<uint64_t>(bytes, 1), 256);
    return o;
  };
  const uint64_t nk = n * L.K;
  const uint64_t ms = max_split_tokens(L, n), ns = std::min<uint64_t>(n, kSmallRouteMaxTokens);
  w.rms = take(n * 4);
  w.logits = take(n * L.E * 4);
  w.topk_idx = take(nk * 4);
  w.topk_w = take(nk * 4);
  w.meta = take((2ull * L.E + 2) * 4);
  w.exrec = take((uint64_t)L.E * kRecWords * 4);
  w.perm = take(nk * 4);
  w.pos_of = take(nk * 4);
  w.gemm = use_gemm_path(L, n);
  w.xn = take(n * L.Dp * 4);  // normalised rows, x dtype (f32 size covers both)
  w.act = take(nk * L.Fp * 4);
  if (w.gemm) {
    w.tile_off = take((L.E + 1ull) * 4);
    const uint64_t kx = qrow_bytes(L.w1), ka = qrow_bytes(L.w2);
    w.xq[0] = take(n * kx);
    w.xq[1] = take(n * kx / 2);  // e2m1 lo codes, two per byte
    w.xq[2] = take(n * qscale_bytes(L.w1));
    w.xq[3] = take(n * qscale_bytes(L.w1));
    w.aq[0] = take(nk * ka);
    w.aq[1] = take(nk * ka / 2);
    w.aq[2] = take(nk * qscale_bytes(L.w2));
    w.aq[3] = take(nk * qscale_bytes(L.w2));
  }
  // decode-sized batches split the down projection's K range in parts (kDownSplitFew when gate_up
  // is split too, else kDownSplit), or (the fused kernel) in feature slices: a partial-sum buffer
  // each, sized for the largest m <= n
  uint64_t frows = 0;
  for (uint64_t m = 1; m <= ns; ++m) frows = std::max(frows, fused_rows(L, m));
  const uint64_t yrows = std::max({nk, ns * L.K * kDownSplit, ms * L.K * kDownSplitFew, frows});
  w.ypart = take(yrows * L.Dp * 4);
  w.dcnt = take(((n + kDispatchChunk - 1) / kDispatchChunk) * (uint64_t)L.E * 4);
  w.total = off;
  return w;
}

struct WsPtrs {
  float *rms;
  float *logits;
  int32_t *topk_idx;
  float *topk_w;
  int32_t *seg_off, *active, *num_active, *perm, *pos_of;
  int32_t *exrec;
  void *xn;
  float *act, *ypart;
  int32_t *tile_off;
  int32_t *dcnt;  // per-chunk expert counts of the multi-workgroup dispatch
  QRows xq, aq;
};

WsPtrs ws_ptrs(const burnext_moe_layer &L, const WsLayout &w, void *base) {
  uint8_t *b = (uint8_t *)base;
  WsPtrs p{};
  p.rms = (float *)(b + w.rms);
  p.logits = (float *)(b + w.logits);
  p.topk_idx = (int32_t *)(b + w.topk_idx);
  p.topk_w = (float *)(b + w.topk_w);
  p.seg_off = (int32_t *)(b + w.meta);
  p.active = p.seg_off + L.E + 1;
  p.num_active = p.active + L.E;
  p.exrec = (int32_t *)(b + w.exrec);
  p.xn = b + w.xn;
  if (w.gemm) {
    p.tile_off = (int32_t *)(b + w.tile_off);
    p.xq = QRows{b + w.xq[0], b + w.xq[1], b + w.xq[2], b + w.xq[3], qrow_bytes(L.w1), qscale_bytes(L.w1)};
    p.aq = QRows{b + w.aq[0], b + w.aq[1], b + w.aq[2], b + w.aq[3], qrow_bytes(L.w2), qscale_bytes(L.w2)};
  }
  p.perm = (int32_t *)(b + w.perm);
  p.pos_of = (int32_t *)(b + w.pos_of);
  p.act = (float *)(b + w.act);
  p.ypart = (float *)(b + w.ypart);
  p.dcnt = (int32_t *)(b + w.dcnt);
  return p;
}

constexpr size_t kLdsBudget = 160 * 1024;

// Router token block: up to 8 tokens whose f32 rows (padded to 512) fit in LDS, halved down to 2
// while the grid (token blocks x expert groups of 4 * epw) has fewer than 512 workgroups: the
// kernel's time is one workgroup's latency chain (stage, norm, dots) until the CUs fill
// (measured 15.7 -> 11.2 us at 64 tokens and 18.7 -> 14.3 us at 200, E = 32, D = 2880).
uint32_t router_tb(const burnext_moe_layer &L, uint64_t n, uint32_t epw) {
  const uint32_t Dpad = (uint32_t)align_up(L.D, 512);
  const uint64_t groups = (L.E + 4u * epw - 1) / (4u * epw);
  uint32_t tb = 8;
  while (tb > 1 && router_lds_bytes(tb, Dpad) > kLdsBudget) tb >>= 1;
  while (tb > 2 && (n + tb - 1) / tb * groups < 512) tb >>= 1;
  return tb;
}

// Set while burnext_moe_forward_noalloc runs: its launches are never timed (timing creates events).
thread_local bool g_untimed = false;

// While profiling is on, binds a HIP event pair to every kernel dispatch launched in its scope
// (hipExtLaunchKernel through the thread's LaunchTimer), recorded under kernel id k: the pair
// carries the dispatch's own begin and end, as rocprofv3's kernel trace does.
struct ProfScope final : LaunchTimer {
  burnext_moe_layer *L;
  hipStream_t s;
  int k;
  LaunchTimer *prev;
  bool on;
  ProfScope(burnext_moe_layer *L_, hipStream_t s_, int k_)
      : L(L_), s(s_), k(k_), prev(g_launch_timer), on(L_->profiling && !g_untimed) {
    if (on) g_launch_timer = this;
  }
  ~ProfScope() override {
    if (on) g_launch_timer = prev;
  }
  bool pair(hipEvent_t &a, hipEvent_t &b) override {
    a = b = nullptr;
    Profiler &P = profiler();
    std::lock_guard<std::mutex> lk(P.mu);
    auto &pool = P.pool[L->device];
    if (!pool.empty()) {  // a pair from an earlier pass: no event creation between launches
      a = pool.back().first;
      b = pool.back().second;
      pool.pop_back();
    } else {
      // timing-only events: no system-scope fence when they complete (that fence's cache
      // write-back and invalidate would be charged to the dispatch and slow the next one)
      if (hipEventCreateWithFlags(&a, hipEventDisableSystemFence) != hipSuccess) return false;
      if (hipEventCreateWithFlags(&b, hipEventDisableSystemFence) != hipSuccess) {
        (void)hipEventDestroy(a);
        a = nullptr;
        return false;
      }
    }
    auto it = P.last_end.find(s);
    P.pending.push_back({a, b, it == P.last_end.end() ? nullptr : it->second, L, k, L->device});
    P.last_end[s] = b;
    return true;
  }
};

enum KernelId {
  kKRouter = 0, kKTopk = 1, kKDispatch = 2, kKGateUp = 3, kKDown = 4, kKCombine = 5, kKExperts = 7  // 6: reserved
};

burnext_status check_launch(hipError_t e, const char *what) {
  if (e != hipSuccess) return fail(BURNEXT_DEVICE_ERROR, std::string(what) + ": " + hipGetErrorString(e));
  return BURNEXT_OK;
}

// Router logits (and r per token when normalising) into the workspace: router_rows_kernel for
// batches of kRouterRowsMinTokens tokens or more whose rows fit its registers, router_kernel else.
burnext_status run_router(burnext_moe_layer *L, const void *x, bool x_bf16, uint64_t n, bool norm, float *rms,
                          float *logits, void *xn, hipStream_t s, const QRows *xq = nullptr, bool xn_bf16 = false) {
  RouterArgs ra{};
  ra.xn = xn;
  ra.xn_bf16 = xn_bf16 ? 1 : 0;
  if (xq) ra.xq = *xq;
  ra.gamma = L->gamma;
  ra.Dp = L->Dp;
  ra.x = x;
  ra.rw = norm ? L->router_wg : L->router_w;
  const bool w_bf16 = norm ? L->router_wg_bf16 : L->router_bf16;
  ra.rb = L->router_b;
  ra.logits = logits;
  ra.rms = rms;
  ra.n = (uint32_t)n;
  ra.D = L->D;
  ra.Dpad = (uint32_t)align_up(L->D, 512);
  ra.E = L->E;
  ra.epw = n <= 64 ? 1 : 2;
  ra.tb = router_tb(*L, n, ra.epw);
  ra.eps = L->eps;
  ra.apply_norm = norm ? 1 : 0;
  const bool vec = L->D % 8 == 0 && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)ra.rw & 15u) == 0;
  const uint32_t lim = 512u * kFrontChunks;
  const bool rows = vec && n >= kRouterRowsMinTokens && L->D <= lim && (!xn || L->Dp <= lim) &&
                    (!xq || !xq->hi || xq->kq <= lim) && !xn_bf16;  // (bf16 rows: router_kernel)
  ProfScope ps(L, s, kKRouter);
  // 4 tokens per wave (32 per workgroup) once that still gives every CU a workgroup: half the LDS
  // reads per token (measured: 120B T = 8192 206 -> 171 us; slower while the grid is short of the CUs)
  const int tpw = n >= 32ull * (uint64_t)L->num_cus ? 4 : 2;
  return check_launch(rows ? launch_router_rows(ra, x_bf16, w_bf16, tpw, s) : launch_router(ra, x_bf16, w_bf16, vec, s),
                      "router kernel launch");
}

burnext_status run_small_route(burnext_moe_layer *L, uint64_t n, const WsPtrs &p, const float *logits,
                               int32_t *topk_idx, float *topk_w, hipStream_t s) {
  SmallRouteArgs a{};
  a.logits = logits;
  a.exrec = p.exrec;
  a.topk_idx = topk_idx;
  a.topk_w = topk_w;
  a.seg_off = p.seg_off;
  a.perm = p.perm;
  a.pos_of = p.pos_of;
  a.active = p.active;
  a.num_active = p.num_active;
  a.n = (uint32_t)n;
  a.E = L->E;
  a.K = L->K;
  ProfScope ps(L, s, kKTopk);
  return check_launch(launch_small_route(a, s), "small-batch routing kernel launch");
}

burnext_status run_topk(burnext_moe_layer *L, uint64_t n, const float *logits, int32_t *idx, float *w, hipStream_t s) {
  TopkArgs ta{};
  ta.logits = logits;
  ta.topk_idx = idx;
  ta.topk_w = w;
  ta.n = (uint32_t)n;
  ta.E = L->E;
  ta.K = L->K;
  ProfScope ps(L, s, kKTopk);
  return check_launch(launch_topk(ta, s), "top-k kernel launch");
}

burnext_status run_dispatch(burnext_moe_layer *L, uint64_t n, const int32_t *idx, int32_t *seg_off, int32_t *perm,
                            int32_t *pos_of, int32_t *active, int32_t *num_active, int32_t *exrec,
                            int32_t *chunk_cnt, hipStream_t s, int32_t *tile_off = nullptr) {
  DispatchArgs da{};
  da.chunk_cnt = chunk_cnt;
  da.tile_off = tile_off;
  da.exrec = exrec;
  da.topk_idx = idx;
  da.seg_off = seg_off;
  da.perm = perm;
  da.pos_of = pos_of;
  da.active = active;
  da.num_active = num_active;
  da.n = (uint32_t)n;
  da.K = L->K;
  da.E = L->E;
  ProfScope ps(L, s, kKDispatch);
  return check_launch(launch_dispatch(da, s), "dispatch kernel launch");
}

// The decode-sized router (one wave per expert and token pair) covers n <= 16 tokens with
// D % 8 == 0, D <= 3072 and 16-byte aligned x and router rows; otherwise router_kernel runs.
bool router_small_ok(const burnext_moe_layer &L, uint64_t n, const void *x, bool norm) {
  const void *rw = norm ? L.router_wg : L.router_w;
  return n >= 1 && n <= kSmallRouteMaxTokens && L.D % 8 == 0 && L.D <= 512u * kFrontChunks &&
         ((uintptr_t)x & 15u) == 0 && ((uintptr_t)rw & 15u) == 0;
}

burnext_status run_router_small(burnext_moe_layer *L, const void *x, bool x_bf16, uint64_t n, bool norm, float *rms,
                                float *logits, void *xn, bool xn_bf16, hipStream_t s) {
  FrontArgs a{};
  a.xn_bf16 = xn_bf16 ? 1 : 0;
  a.x = x;
  a.rw = norm ? L->router_wg : L->router_w;
  const bool w_bf16 = norm ? L->router_wg_bf16 : L->router_bf16;
  a.rb = L->router_b;
  a.gamma = L->gamma;
  a.xn = xn;
  a.logits = logits;
  a.rms = rms;
  a.n = (uint32_t)n;
  a.D = L->D;
  a.Dp = L->Dp;
  a.E = L->E;
  a.eps = L->eps;
  a.apply_norm = norm ? 1 : 0;
  ProfScope ps(L, s, kKRouter);
  return check_launch(launch_router_small(a, x_bf16, w_bf16, s), "router kernel launch");
}

// The layer input formed by the router (internal: a decoder's residual add after its attention
// block): x = resid + (sum_h part_h + bias), written to xout (router_front_kernel).
struct PreAdd {
  const float *part;
  uint64_t part_stride;
  uint32_t nparts;
  const float *bias;
  const float *resid;
  float *xout;
};

bool front_ok(const burnext_moe_layer &L, uint64_t n) {
  return !L.disabled && n >= 1 && n <= kSmallRouteMaxTokens && L.D % 8 == 0 && L.D <= 512u * kFrontChunks &&
         L.Dp <= 512u * kFrontChunks && ((uintptr_t)L.router_wg & 15u) == 0 && ((uintptr_t)L.router_w & 15u) == 0;
}

burnext_status run_router_front(burnext_moe_layer *L, const PreAdd &pa, uint64_t n, bool norm, float *rms,
                                float *logits, void *xn, bool xn_bf16, hipStream_t s) {
  PreFrontArgs a{};
  FrontArgs &f = a.f;
  f.xn_bf16 = xn_bf16 ? 1 : 0;
  f.x = pa.xout;
  f.rw = norm ? L->router_wg : L->router_w;
  const bool w_bf16 = norm ? L->router_wg_bf16 : L->router_bf16;
  f.rb = L->router_b;
  f.gamma = L->gamma;
  f.xn = xn;
  f.logits = logits;
  f.rms = rms;
  f.n = (uint32_t)n;
  f.D = L->D;
  f.Dp = L->Dp;
  f.E = L->E;
  f.eps = L->eps;
  f.apply_norm = norm ? 1 : 0;
  a.part = pa.part;
  a.part_stride = pa.part_stride;
  a.nparts = pa.nparts;
  a.bias = pa.bias;
  a.resid = pa.resid;
  a.xout = pa.xout;
  ProfScope ps(L, s, kKRouter);
  return check_launch(launch_router_front(a, w_bf16, s), "router front launch");
}

// The weighted combine + residual of every path (token-major slot rows in p.ypart).
// An RmsNorm of the layer's output fused into its combine (internal: the decoder's next norm).
struct PostNorm {
  const float *gamma;
  float eps;
  float *out;
};

burnext_status combine(burnext_moe_layer *L, const void *x, void *y, bool xb, uint64_t n, uint32_t flags,
                       const WsPtrs &p, hipStream_t s, uint32_t nparts = 1, bool part_bf16 = false,
                       const PostNorm *pn = nullptr, const FusedGeom *slices = nullptr) {
  CombineArgs c{};
  c.x = x;
  c.y = y;
  c.ypart = p.ypart;
  c.nparts = nparts;
  c.part_bf16 = part_bf16 ? 1 : 0;
  c.part_stride = n * L->K * L->Dp;
  c.topk_w = p.topk_w;
  c.n = (uint32_t)n;
  c.D = L->D;
  c.Dp = L->Dp;
  c.K = L->K;
  c.add_residual = (flags & BURNEXT_ADD_RESIDUAL) ? 1 : 0;
  if (pn) {
    c.ngamma = pn->gamma;
    c.nout = pn->out;
    c.neps = pn->eps;
  }
  if (slices) {  // the fused kernel's slices: their count follows num_active on the device
    c.num_active = p.num_active;
    c.slice_grid = slices->grid;
    c.slice_cap = std::min(L->w2.nb, slices->nsl_cap);
  }
  burnext_status st;
  {
    ProfScope ps(L, s, kKCombine);
    st = slices ? check_launch(launch_combine_slices(c, xb, s), "combine launch")  // the fused kernel's slices
                : check_launch(launch_combine(c, xb, s), "combine launch");
  }
  return st == BURNEXT_OK ? ok() : st;
}

// The fused decode experts (use_fused): one launch over (active expert, slice) items.
burnext_status run_fused(burnext_moe_layer *L, uint64_t n, int nt, bool xb, const FusedGeom &fg, const WsPtrs &p,
                         hipStream_t s) {
  FusedArgs a{};
  a.w1b = L->w1.blocks;
  a.w1s = L->w1.scales;
  a.w2b = L->w2.blocks;
  a.w2s = L->w2.scales;
  a.w1b_es = L->w1.blocks_per_expert;
  a.w1s_es = L->w1.scales_per_expert;
  a.w2b_es = L->w2.blocks_per_expert;
  a.w2s_es = L->w2.scales_per_expert;
  a.b1 = L->b1;
  a.b2 = L->b2;
  a.b1_es = L->w1.rows_p;
  a.b2_es = L->w2.rows_p;
  a.nrt1 = L->w1.nrt;
  a.nb1 = L->w1.nb;
  a.kt1 = L->w1.cols;
  a.nrt2 = L->w2.nrt;
  a.nb2 = L->w2.nb;
  a.D = L->D;
  a.nsl_cap = fg.nsl_cap;
  a.sb_max = fg.sb_max;
  a.mt_max = fg.mt;
  a.num_active = p.num_active;
  a.exrec = p.exrec;
  a.perm = p.perm;
  a.topk = L->K;
  a.xn = p.xn;
  a.out = p.ypart;
  a.out_stride = L->Dp;
  a.slice_stride = n * L->K * L->Dp;
  a.alpha = L->alpha;
  a.limit = L->limit;
  ProfScope ps(L, s, kKExperts);
  return check_launch(launch_fused(a, fg, nt, xb, s), "fused experts launch");
}

// Grouped-GEMM path (use_gemm_path): router (+ the two-term rows of xn), top-k,
// dispatch (+ token-tile prefix), gate_up GEMM (SwiGLU, quantised act rows), down GEMM (slot rows).
burnext_status forward_gemm(burnext_moe_layer *L, const void *x, bool xb, uint64_t n, bool norm, const WsPtrs &p,
                            hipStream_t s) {
  burnext_status st = run_router(L, x, xb, n, norm, p.rms, p.logits, nullptr, s, &p.xq);
  if (st == BURNEXT_OK) st = run_topk(L, n, p.logits, p.topk_idx, p.topk_w, s);
  if (st == BURNEXT_OK)
    st = run_dispatch(L, n, p.topk_idx, p.seg_off, p.perm, p.pos_of, p.active, p.num_active, p.exrec, p.dcnt, s,
                      p.tile_off);
  if (st != BURNEXT_OK) return st;
  const uint64_t nk = n * L->K;
  const uint64_t max_tiles = (nk + kGemmTok - 1) / kGemmTok + std::min<uint64_t>(L->E, nk);
  for (int up = 1; up >= 0; --up) {
    const TiledMx &t = up ? L->w1 : L->w2;
    GemmArgs g{};
    g.wb = t.blocks;
    g.ws = t.gscales;
    g.wb_estride = t.blocks_per_expert;
    g.ws_estride = t.gscales_per_expert;
    g.bias = up ? L->b1 : L->b2;
    g.bias_estride = t.rows_p;
    g.nrt = t.nrt;
    g.nb = t.nb;
    g.kt = t.cols;
    g.out_rows = up ? 2 * L->F : L->D;
    g.nrb = (t.rows_p + kGemmRows - 1) / kGemmRows;
    g.seg_off = p.seg_off;
    g.tile_off = p.tile_off;
    g.perm = p.perm;
    g.E = L->E;
    g.topk = L->K;
    g.b = up ? p.xq : p.aq;
    g.act = p.aq;
    g.act_feats = L->F;
    g.out = (uint16_t *)p.ypart;
    g.out_stride = L->Dp;
    g.alpha = L->alpha;
    g.limit = L->limit;
    const uint64_t grid = align_up((uint64_t)g.nrb * max_tiles, 8);
    if (grid > 0x7fffffffull) return fail(BURNEXT_UNSUPPORTED, "expert GEMM grid too large");
    ProfScope ps(L, s, up ? kKGateUp : kKDown);
    st = check_launch(launch_gemm(g, up != 0, (uint32_t)grid, s), up ? "gate_up GEMM launch" : "down GEMM launch");
    if (st != BURNEXT_OK) return st;
  }
  return BURNEXT_OK;
}

burnext_status check_ws(burnext_moe_layer *L, uint64_t n, void *ws, uint64_t ws_bytes, WsLayout &w) {
  w = ws_layout(*L, n);
  if (!ws) return fail(BURNEXT_INVALID_ARG, "workspace is null");
  if (((uintptr_t)ws & 255u) != 0) return fail(BURNEXT_INVALID_ARG, "workspace must be 256-byte aligned");
  if (ws_bytes < w.total) {
    char buf[160];
    snprintf(buf, sizeof(buf), "workspace of %llu bytes is smaller than the %llu bytes needed for %llu tokens",
             (unsigned long long)ws_bytes, (unsigned long long)w.total, (unsigned long long)n);
    return fail(BURNEXT_WORKSPACE_TOO_SMALL, buf);
  }
  return BURNEXT_OK;
}

constexpr uint64_t kMaxTokens = 1ull << 22;

// Scratch of burnext_moe_forward_noalloc: one fixed device array per GPU (it lives in this file's
// code object, so every device the library runs on holds its own copy until the process ends).
// Host code never passes `scratch` itself to a kernel -- on the host that name is only a stand-in
// for the symbol -- but the device address hipGetSymbolAddress returns for the current device.
constexpr uint64_t kScratchBytes = 16ull << 20;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `device` (which must be current), looked up once per device.
burnext_status scratch_address(int device, void **out);

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
burnext_status scratch_address(int device, void **out) {
  if (device < 0 || device >= kMaxDevices) return fail(BURNEXT_UNSUPPORTED, "device index above 63");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(BURNEXT_DEVICE_ERROR, std::string("hipGetSymbolAddress of the scratch array failed: ") +
                                            hipGetErrorString(e));
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return BURNEXT_OK;
}
}  // namespace

namespace burnext {

bool moe_front_fusable(const burnext_moe_layer *L, uint64_t n, uint32_t nparts);

// burnext_moe_forward; with pn, the RmsNorm of y (pn->gamma, pn->eps into pn->out) runs inside the
// combine where the path allows it (decode-sized GEMV path, f32 rows), and *norm_done says whether
// it did (otherwise the caller normalises y itself).
burnext_status forward_impl(burnext_moe_layer *L, const void *x, burnext_dtype x_dtype, void *y, uint64_t n,
                            uint32_t flags, void *workspace, uint64_t ws_bytes, void *stream, const PostNorm *pn,
                            bool *norm_done, const PreAdd *pa = nullptr, bool experts_bf16 = false) {
  if (norm_done) *norm_done = false;
  if (!L) return fail(BURNEXT_INVALID_ARG, "layer is null");
  if (pa && (x != pa->xout || x_dtype != BURNEXT_F32 || !moe_front_fusable(L, n, pa->nparts)))
    return fail(BURNEXT_INVALID_ARG, "formed input rows need f32 rows, x == xout and a decode-sized batch");
  if (x_dtype != BURNEXT_F32 && x_dtype != BURNEXT_BF16) return fail(BURNEXT_INVALID_ARG, "bad x_dtype");
  if (flags & ~(BURNEXT_APPLY_RMSNORM | BURNEXT_ADD_RESIDUAL | BURNEXT_FUSED_EXPERTS))
    return fail(BURNEXT_INVALID_ARG, "unknown flag bits");
  if (n > kMaxTokens) return fail(BURNEXT_UNSUPPORTED, "n_tokens above 4194304 is not supported");
  if (n == 0) return ok();
  if (!x || !y) return fail(BURNEXT_INVALID_ARG, "x or y is null");
  if (x == y) return fail(BURNEXT_INVALID_ARG, "x and y must not alias");
  const bool xb = x_dtype == BURNEXT_BF16;
  hipStream_t s = (hipStream_t)stream;
  DeviceGuard guard(L->device);
  if (!guard.ok) return fail(BURNEXT_DEVICE_ERROR, "hipSetDevice failed");
  if (L->disabled) {  // identity, src/moe/mod.rs:106-108
    const burnext_status cs =
        check_launch(hipMemcpyAsync(y, x, n * L->D * (xb ? 2 : 4), hipMemcpyDeviceToDevice, s), "identity copy");
    return cs == BURNEXT_OK ? ok() : cs;
  }
  WsLayout w;
  burnext_status st = check_ws(L, n, workspace, ws_bytes, w);
  if (st != BURNEXT_OK) return st;
  const WsPtrs p = ws_ptrs(*L, w, workspace);
  const bool norm = (flags & BURNEXT_APPLY_RMSNORM) != 0;
  if (w.gemm && xb) {
    st = forward_gemm(L, x, xb, n, norm, p, s);
    if (st != BURNEXT_OK) return st;
    return combine(L, x, y, xb, n, flags, p, s, 1, true);  // bf16 slot rows from the down GEMM
  }
  // f32 activations: two bf16 terms (hi + bf16 of the residual, ~2^-17 relative per value); with
  // experts_bf16 the router writes the normalised rows rounded to bf16 once and every expert
  // projection takes one term (the down projection rounds the SwiGLU rows as it stages them)
  const bool small_router = !pa && router_small_ok(*L, n, x, norm);
  const bool xnb = xb || experts_bf16;
  const int nt = xnb ? 1 : 2;
  FusedGeom fg{};
  const bool fused_experts = (flags & BURNEXT_FUSED_EXPERTS) && use_fused(*L, n, nt, pn != nullptr, fg);
  // a single token routes inside the gate_up launch (route_one_token: no routing launch)
  const bool route1 = n == 1 && !fused_experts && L->E <= kMaxExperts && L->K <= kMaxTopK && L->K <= L->E;
  const GemvCfg cfg_up = gemv_cfg(*L, n, nt, true), cfg_dn = gemv_cfg(*L, n, nt, false);
  // down projection of decode-sized batches: every row tile's K range in ksplit fixed parts of
  // whole K-groups (separate work units, so the units are a fraction of a tile each and spread
  // evenly over the waves; measured slower from 64 tokens on)
  const bool up_split = gate_up_split(*L, n);
  // (few touched experts: kDownSplitFew parts, as many as the workspace holds for those batches)
  const uint32_t ksplit = (up_split && (L->w2.nb + 3u) / 4u >= kDownSplitFew) ? kDownSplitFew
                        : (n <= kSmallRouteMaxTokens && (L->w2.nb + 3u) / 4u >= kDownSplit) ? kDownSplit : 1u;
  st = pa             ? run_router_front(L, *pa, n, norm, p.rms, p.logits, p.xn, xnb, s)
       : small_router ? run_router_small(L, x, xb, n, norm, p.rms, p.logits, p.xn, xnb && !xb, s)
                      : run_router(L, x, xb, n, norm, p.rms, p.logits, p.xn, s, nullptr, xnb && !xb);
  if (st == BURNEXT_OK && n <= kSmallRouteMaxTokens) {
    if (!route1) st = run_small_route(L, n, p, p.logits, p.topk_idx, p.topk_w, s);
  } else if (st == BURNEXT_OK) {
    st = run_topk(L, n, p.logits, p.topk_idx, p.topk_w, s);
    if (st == BURNEXT_OK)
      st = run_dispatch(L, n, p.topk_idx, p.seg_off, p.perm, p.pos_of, p.active, p.num_active, p.exrec, p.dcnt, s);
  }
  if (st != BURNEXT_OK) return st;

  if (fused_experts) {
    st = run_fused(L, n, nt, xnb, fg, p, s);
    if (st != BURNEXT_OK) return st;
    return combine(L, x, y, xb, n, flags, p, s, 1, false, nullptr, &fg);
  }

  auto gemv = [&](bool gate_up) -> burnext_status {
    const GemvCfg &cf = gate_up ? cfg_up : cfg_dn;
    const TiledMx &t = gate_up ? L->w1 : L->w2;
    GemvArgs g{};
    g.wb = t.blocks;
    g.ws = t.scales;
    g.wb_estride = t.blocks_per_expert;
    g.ws_estride = t.scales_per_expert;
    g.bias = gate_up ? L->b1 : L->b2;
    g.bias_estride = t.rows_p;  // multiple of 16: 16-byte aligned rows of 4 for the epilogue
    g.nrt = t.nrt;
    g.nb = t.nb;
    g.kt = t.cols;
    g.out_rows = gate_up ? L->F : L->D;
    g.mt_max = cf.mt;
    g.seg_off = p.seg_off;
    g.active = p.active;
    g.num_active = p.num_active;
    g.perm = p.perm;
    g.exrec = p.exrec;
    g.topk = L->K;
    g.brows = gate_up ? p.xn : (const void *)p.act;
    g.out = gate_up ? p.act : p.ypart;
    g.out_stride = gate_up ? L->Fp : L->Dp;
    g.alpha = L->alpha;
    g.limit = L->limit;
    g.nrec = cf.nrec;
    g.num_cus = (uint32_t)L->num_cus;
    g.weighted = n <= kSmallRouteMaxTokens ? 1u : 0u;  // measured: strided shares faster from 64 tokens on
    if (!gate_up && ksplit > 1u) {
      g.ksplit = ksplit;
      g.out_half = n * L->K * L->Dp;
    }
    if (gate_up && up_split) g.ksplit = kGateUpSplit;  // K-parts on the waves of a workgroup, summed there
    if (gate_up && route1) {
      g.route1_lg = p.logits;
      g.route1_E = L->E;
      g.rout = RouteOut{p.topk_idx, p.topk_w, p.seg_off, p.perm, p.pos_of, p.active, p.num_active, p.exrec};
    }
    ProfScope ps(L, s, gate_up ? kKGateUp : kKDown);
    return check_launch(launch_gemv(g, nt, gate_up, xnb, cf.grid, s), gate_up ? "gate_up launch" : "down launch");
  };
  st = gemv(true);
  if (st != BURNEXT_OK) return st;
  // a single token routed in gate_up, down in kDownSplitFew parts and no fused norm: the down
  // projection and the combine in one launch (down_combine1_kernel, the same arithmetic)
  if (route1 && ksplit == kDownSplitFew && !pn && L->K <= kDownComb1MaxK && L->w2.nb * 32u <= kDownComb1MaxKp &&
      (nt == 1 || !xb)) {
    DownComb1Args d{};
    d.wb = L->w2.blocks;
    d.ws = L->w2.scales;
    d.wb_estride = L->w2.blocks_per_expert;
    d.ws_estride = L->w2.scales_per_expert;
    d.bias = L->b2;
    d.bias_estride = L->w2.rows_p;
    d.nrt = L->w2.nrt;
    d.nb = L->w2.nb;
    d.kt = L->w2.cols;
    d.D = L->D;
    d.K = L->K;
    d.act = p.act;
    d.act_stride = L->Fp;
    d.topk_idx = p.topk_idx;
    d.pos_of = p.pos_of;
    d.topk_w = p.topk_w;
    d.x = x;
    d.y = y;
    d.add_residual = (flags & BURNEXT_ADD_RESIDUAL) ? 1u : 0u;
    ProfScope ps(L, s, kKDown);
    st = check_launch(launch_down_combine1(d, nt, xb, s), "down + combine launch");
    return st == BURNEXT_OK ? ok() : st;
  }
  st = gemv(false);
  if (st != BURNEXT_OK) return st;

  // the fused RmsNorm of y: f32 rows of at most 4096 values (combine_norm_kernel)
  const bool fuse = pn && !xb && L->D % 4 == 0 && L->D <= 4096 &&
                    (((uintptr_t)x | (uintptr_t)y | (uintptr_t)pn->out | (uintptr_t)pn->gamma) & 15u) == 0;
  st = combine(L, x, y, xb, n, flags, p, s, ksplit, false, fuse ? pn : nullptr);
  if (st == BURNEXT_OK && norm_done) *norm_done = fuse;
  return st;
}

// The decoder's entry: burnext_moe_forward with the next RmsNorm fused where possible, and with
// the layer input x = resid + (sum_h part_h + bias) formed by the router when part is not null
// (then x must be the f32 rows xout that receive it, and moe_front_fusable must hold).
burnext_status moe_forward_post_norm(burnext_moe_layer *L, const void *x, burnext_dtype x_dtype, void *y, uint64_t n,
                                     uint32_t flags, void *workspace, uint64_t ws_bytes, void *stream,
                                     const float *gamma, float eps, float *xn, bool *norm_done, const float *part,
                                     uint64_t part_stride, uint32_t nparts, const float *bias, const float *resid,
                                     bool experts_bf16) {
  const PostNorm pn{gamma, eps, xn};
  const PreAdd pa{part, part_stride, nparts, bias, resid, (float *)x};
  return forward_impl(L, x, x_dtype, y, n, flags, workspace, ws_bytes, stream, gamma && xn ? &pn : nullptr,
                      norm_done, part ? &pa : nullptr, experts_bf16);
}

// nparts: the K-part partial sums of the output projection the router adds (router_front_kernel
// takes at most kFrontMaxParts of them; more run the separate residual add).
bool moe_front_fusable(const burnext_moe_layer *L, uint64_t n, uint32_t nparts) {
  return L && nparts >= 1u && nparts <= kFrontMaxParts && front_ok(*L, n);
}

}  // namespace burnext

extern "C" {

const char *burnext_last_error(void) { return g_last_error.c_str(); }

burnext_status burnext_moe_layer_create(const burnext_moe_config *cfg, const burnext_mxfp4_desc *w1_desc,
                                        const uint8_t *w1_blocks, const uint8_t *w1_scales,
                                        const burnext_mxfp4_desc *w2_desc, const uint8_t *w2_blocks,
                                        const uint8_t *w2_scales, const void *b1, const void *b2,
                                        burnext_dtype bias_dtype, const void *router_w, const void *router_b,
                                        burnext_dtype router_dtype, const void *norm_gamma, burnext_dtype norm_dtype,
                                        burnext_gate_up_layout gate_up_layout, int device,
                                        burnext_moe_layer_t *out_layer) {
  if (!out_layer) return fail(BURNEXT_INVALID_ARG, "out_layer is null");
  *out_layer = nullptr;
  if (!cfg || !w1_desc || !w2_desc || !w1_blocks || !w1_scales || !w2_blocks || !w2_scales || !b1 || !b2 || !router_w)
    return fail(BURNEXT_INVALID_ARG, "null config, descriptor, weight or bias pointer");
  const uint32_t D = cfg->d_model, F = cfg->ffn_hidden, E = cfg->num_experts;
  if (D == 0 || F == 0 || E == 0) return fail(BURNEXT_INVALID_ARG, "d_model, ffn_hidden and num_experts must be > 0");
  if (E > kMaxExperts) return fail(BURNEXT_UNSUPPORTED, "num_experts above 256 is not supported");
  if (D > 32768 || F > 32768) return fail(BURNEXT_UNSUPPORTED, "d_model and ffn_hidden above 32768 are not supported");
  const uint32_t K = std::min(std::max(cfg->experts_per_token, 1u), E);
  if (K > kMaxTopK) return fail(BURNEXT_UNSUPPORTED, "experts_per_token above 32 is not supported");
  if ((bias_dtype != BURNEXT_F32 && bias_dtype != BURNEXT_BF16) ||
      (router_dtype != BURNEXT_F32 && router_dtype != BURNEXT_BF16) ||
      (norm_dtype != BURNEXT_F32 && norm_dtype != BURNEXT_BF16))
    return fail(BURNEXT_INVALID_ARG, "dtype must be BURNEXT_F32 or BURNEXT_BF16");
  if (gate_up_layout != BURNEXT_GATE_UP_HALVES && gate_up_layout != BURNEXT_GATE_UP_INTERLEAVED)
    return fail(BURNEXT_INVALID_ARG, "gate_up_layout must be HALVES or INTERLEAVED");
  std::string msg;
  if (!check_desc(w1_desc, E, 2ull * F, D, "w1", msg) || !check_desc(w2_desc, E, D, F, "w2", msg))
    return fail(BURNEXT_INVALID_ARG, msg);

  // host preparation (no device call): tiled experts, biases in the internal row order, gamma and
  // the gamma-folded router rows
  TiledMx t1, t2;
  std::vector<uint8_t> hb1t, hs1t, hg1t, hb2t, hs2t, hg2t;
  burnext_status st =
      repack_tiled(t1, E, 2 * F, D, w1_blocks, w1_scales, *w1_desc, true, F, gate_up_layout, hb1t, hs1t, hg1t);
  if (st == BURNEXT_OK)
    st = repack_tiled(t2, E, D, F, w2_blocks, w2_scales, *w2_desc, false, F, gate_up_layout, hb2t, hs2t, hg2t);
  if (st != BURNEXT_OK) return st;
  std::vector<float> hb1((size_t)E * t1.rows_p, 0.0f), hb2((size_t)E * t2.rows_p, 0.0f), hrb(E, 0.0f), hg(D, 1.0f);
  for (uint32_t e = 0; e < E; ++e) {
    for (uint32_t r = 0; r < 2 * F; ++r)
      hb1[(size_t)e * t1.rows_p + r] = read_scalar(b1, bias_dtype, (size_t)e * 2 * F + w1_src_row(r, F, gate_up_layout));
    for (uint32_t d = 0; d < D; ++d) hb2[(size_t)e * t2.rows_p + d] = read_scalar(b2, bias_dtype, (size_t)e * D + d);
    if (router_b) hrb[e] = read_scalar(router_b, router_dtype, e);
  }
  if (norm_gamma)
    for (uint32_t d = 0; d < D; ++d) hg[d] = read_scalar(norm_gamma, norm_dtype, d);
  // RmsNorm routing uses gamma-folded rows gw[e, c] = gamma[c] * w[e, c] (f32); with gamma all ones
  // they equal the given rows, which are then shared.
  bool ones = true;
  for (uint32_t d = 0; d < D; ++d) ones = ones && hg[d] == 1.0f;
  std::vector<float> gw;
  if (!ones) {
    gw.resize((size_t)E * D);
    for (uint32_t e = 0; e < E; ++e)
      for (uint32_t d = 0; d < D; ++d) gw[(size_t)e * D + d] = hg[d] * read_scalar(router_w, router_dtype, (size_t)e * D + d);
  }

  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
    return fail(BURNEXT_INVALID_ARG, "device index out of range (or no HIP device)");

  DeviceGuard guard(device);
  if (!guard.ok) return fail(BURNEXT_DEVICE_ERROR, "hipSetDevice failed");
  {
    static std::once_flag once;
    static hipError_t cfg_err = hipSuccess;
    std::call_once(once, [] {
      cfg_err = configure_kernels();
      if (cfg_err == hipSuccess) cfg_err = configure_gemm_kernels();
      if (cfg_err == hipSuccess) cfg_err = configure_fused_kernels();
    });
    if (cfg_err != hipSuccess) return fail(BURNEXT_DEVICE_ERROR, std::string("kernel configuration failed: ") + hipGetErrorString(cfg_err));
  }

  burnext_moe_layer *L = new (std::nothrow) burnext_moe_layer();
  if (!L) return fail(BURNEXT_OUT_OF_MEMORY, "host allocation failed");
  L->device = device;
  L->D = D;
  L->F = F;
  L->E = E;
  L->K = K;
  L->alpha = cfg->swiglu_alpha;
  L->limit = cfg->swiglu_limit;
  L->eps = cfg->rms_eps;
  L->disabled = cfg->disabled != 0;
  L->Dp = (uint32_t)align_up(D, 32);
  L->Fp = (uint32_t)align_up(F, 32);
  L->w1 = t1;
  L->w2 = t2;

  st = upload_tiled(L->w1, hb1t, hs1t, hg1t);
  if (st == BURNEXT_OK) st = upload_tiled(L->w2, hb2t, hs2t, hg2t);
  // biases (f32 on device), b1 permuted to the interleaved internal row order
  if (st == BURNEXT_OK) st = upload_vec(&L->b1, hb1);
  if (st == BURNEXT_OK) st = upload_vec(&L->b2, hb2);
  if (st == BURNEXT_OK) st = upload_vec(&L->router_b, hrb);
  if (st == BURNEXT_OK) st = upload_vec(&L->gamma, hg);
  if (st == BURNEXT_OK) {
    L->router_bf16 = router_dtype == BURNEXT_BF16;
    const size_t rbytes = (size_t)E * D * (L->router_bf16 ? 2 : 4);
    if (hipMalloc(&L->router_w, rbytes) != hipSuccess)
      st = fail(BURNEXT_OUT_OF_MEMORY, "hipMalloc failed for router weight");
    else if (hipMemcpy(L->router_w, router_w, rbytes, hipMemcpyHostToDevice) != hipSuccess)
      st = fail(BURNEXT_DEVICE_ERROR, "hipMemcpy failed for router weight");
  }
  if (st == BURNEXT_OK) {
    if (ones) {
      L->router_wg = L->router_w;
      L->router_wg_bf16 = L->router_bf16;
    } else {
      float *dgw = nullptr;
      st = upload_vec(&dgw, gw);
      L->router_wg = dgw;
      L->router_wg_bf16 = false;
    }
  }
  if (st == BURNEXT_OK) {
    void *sp = nullptr;
    st = scratch_address(device, &sp);
  }
  if (st == BURNEXT_OK) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
      L->num_cus = cus;
  }
  if (st != BURNEXT_OK) {
    free_layer(L);
    return st;
  }
  *out_layer = L;
  return ok();
}

void burnext_moe_layer_destroy(burnext_moe_layer_t layer) { free_layer(layer); }

burnext_status burnext_moe_workspace_size(burnext_moe_layer_t L, uint64_t n_tokens, uint64_t *bytes) {
  if (!L || !bytes) return fail(BURNEXT_INVALID_ARG, "null layer or output pointer");
  if (n_tokens > kMaxTokens) return fail(BURNEXT_UNSUPPORTED, "n_tokens above 4194304 is not supported");
  *bytes = ws_layout(*L, n_tokens).total;
  return ok();
}

burnext_status burnext_moe_forward(burnext_moe_layer_t L, const void *x, burnext_dtype x_dtype, void *y,
                                   uint64_t n, uint32_t flags, void *workspace, uint64_t ws_bytes, void *stream) {
  return burnext::forward_impl(L, x, x_dtype, y, n, flags, workspace, ws_bytes, stream, nullptr, nullptr);
}

burnext_status burnext_moe_forward_noalloc(burnext_moe_layer_t L, const void *x, burnext_dtype x_dtype, void *y,
                                           uint64_t n, uint32_t flags, void *stream) {
  if (!L) return fail(BURNEXT_INVALID_ARG, "layer is null");
  if (n > kMaxTokens) return fail(BURNEXT_UNSUPPORTED, "n_tokens above 4194304 is not supported");
  const uint64_t need = ws_layout(*L, n).total;
  if (need > kScratchBytes) {
    char buf[200];
    snprintf(buf, sizeof(buf),
             "burnext_moe_forward_noalloc: %llu tokens need %llu bytes of scratch; its fixed scratch holds %llu "
             "(use burnext_moe_forward with a workspace)",
             (unsigned long long)n, (unsigned long long)need, (unsigned long long)kScratchBytes);
    return fail(BURNEXT_UNSUPPORTED, buf);
  }
  void *ws = nullptr;
  {
    DeviceGuard guard(L->device);
    if (!guard.ok) return fail(BURNEXT_DEVICE_ERROR, "hipSetDevice failed");
    const burnext_status st = scratch_address(L->device, &ws);
    if (st != BURNEXT_OK) return st;
  }
  struct Untimed {
    bool prev = g_untimed;
    Untimed() { g_untimed = true; }
    ~Untimed() { g_untimed = prev; }
  } untimed;
  return burnext_moe_forward(L, x, x_dtype, y, n, flags, ws, kScratchBytes, stream);
}

burnext_status burnext_moe_route(burnext_moe_layer_t L, const void *x, burnext_dtype x_dtype, uint64_t n,
                                 uint32_t flags, int32_t *topk_idx, float *topk_w, float *logits, void *workspace,
                                 uint64_t ws_bytes, void *stream) {
  if (!L) return fail(BURNEXT_INVALID_ARG, "layer is null");
  if (x_dtype != BURNEXT_F32 && x_dtype != BURNEXT_BF16) return fail(BURNEXT_INVALID_ARG, "bad x_dtype");
  if (flags & ~(BURNEXT_APPLY_RMSNORM | BURNEXT_ADD_RESIDUAL)) return fail(BURNEXT_INVALID_ARG, "unknown flag bits");
  if (n > kMaxTokens) return fail(BURNEXT_UNSUPPORTED, "n_tokens above 4194304 is not supported");
  if (n == 0) return ok();
  if (!x || !topk_idx || !topk_w) return fail(BURNEXT_INVALID_ARG, "null x / topk_idx / topk_w");
  hipStream_t s = (hipStream_t)stream;
  DeviceGuard guard(L->device);
  if (!guard.ok) return fail(BURNEXT_DEVICE_ERROR, "hipSetDevice failed");
  WsLayout w;
  burnext_status st = check_ws(L, n, workspace, ws_bytes, w);
  if (st != BURNEXT_OK) return st;
  const WsPtrs p = ws_ptrs(*L, w, workspace);
  float *lg = logits ? logits : p.logits;
  const bool xb = x_dtype == BURNEXT_BF16, norm = (flags & BURNEXT_APPLY_RMSNORM) != 0;
  // the forward's routing kernels for this batch size
  st = router_small_ok(*L, n, x, norm) ? run_router_small(L, x, xb, n, norm, p.rms, lg, nullptr, false, s)
                                  : run_router(L, x, xb, n, norm, p.rms, lg, nullptr, s);
  if (st == BURNEXT_OK)
    st = n <= kSmallRouteMaxTokens ? run_small_route(L, n, p, lg, topk_idx, topk_w, s)
                                   : run_topk(L, n, lg, topk_idx, topk_w, s);
  return st == BURNEXT_OK ? ok() : st;
}

burnext_status burnext_moe_dispatch(burnext_moe_layer_t L, const int32_t *topk_idx, uint64_t n, int32_t *seg_offsets,
                                    int32_t *perm, void *workspace, uint64_t ws_bytes, void *stream) {
  if (!L) return fail(BURNEXT_INVALID_ARG, "layer is null");
  if (n > kMaxTokens) return fail(BURNEXT_UNSUPPORTED, "n_tokens above 4194304 is not supported");
  if (!topk_idx || !seg_offsets || !perm) return fail(BURNEXT_INVALID_ARG, "null topk_idx / seg_offsets / perm");
  hipStream_t s = (hipStream_t)stream;
  DeviceGuard guard(L->device);
  if (!guard.ok) return fail(BURNEXT_DEVICE_ERROR, "hipSetDevice failed");
  WsLayout w;
  burnext_status st = check_ws(L, n, workspace, ws_bytes, w);
  if (st != BURNEXT_OK) return st;
  const WsPtrs p = ws_ptrs(*L, w, workspace);
  st = run_dispatch(L, n, topk_idx, seg_offsets, perm, p.pos_of, p.active, p.num_active, p.exrec, p.dcnt, s);
  return st == BURNEXT_OK ? ok() : st;
}

burnext_status burnext_moe_route_dispatch(burnext_moe_layer_t L, const void *x, burnext_dtype x_dtype, uint64_t n,
                                          uint32_t flags, int32_t *topk_idx, float *topk_w, int32_t *seg_offsets,
                                          int32_t *perm, void *workspace, uint64_t ws_bytes, void *stream) {
  if (!L) return fail(BURNEXT_INVALID_ARG, "layer is null");
  if (x_dtype != BURNEXT_F32 && x_dtype != BURNEXT_BF16) return fail(BURNEXT_INVALID_ARG, "bad x_dtype");
  if (flags & ~(BURNEXT_APPLY_RMSNORM | BURNEXT_ADD_RESIDUAL)) return fail(BURNEXT_INVALID_ARG, "unknown flag bits");
  if (n > kMaxTokens) return fail(BURNEXT_UNSUPPORTED, "n_tokens above 4194304 is not supported");
  if (n == 0) return ok();
  if (!x || !topk_idx || !topk_w || !seg_offsets || !perm)
    return fail(BURNEXT_INVALID_ARG, "null x / topk_idx / topk_w / seg_offsets / perm");
  hipStream_t s = (hipStream_t)stream;
  DeviceGuard guard(L->device);
  if (!guard.ok) return fail(BURNEXT_DEVICE_ERROR, "hipSetDevice failed");
  WsLayout w;
  burnext_status st = check_ws(L, n, workspace, ws_bytes, w);
  if (st != BURNEXT_OK) return st;
  WsPtrs p = ws_ptrs(*L, w, workspace);
  // the caller's buffers take the places of the workspace's segment offsets and entry list, so
  // the kernels write them exactly as in a forward of this batch size
  int32_t *active = p.active, *num_active = p.num_active;
  p.seg_off = seg_offsets;
  p.perm = perm;
  const bool xb = x_dtype == BURNEXT_BF16, norm = (flags & BURNEXT_APPLY_RMSNORM) != 0;
  st = router_small_ok(*L, n, x, norm) ? run_router_small(L, x, xb, n, norm, p.rms, p.logits, nullptr, false, s)
                                  : run_router(L, x, xb, n, norm, p.rms, p.logits, nullptr, s);
  if (st == BURNEXT_OK && n <= kSmallRouteMaxTokens) {
    st = run_small_route(L, n, p, p.logits, topk_idx, topk_w, s);
  } else if (st == BURNEXT_OK) {
    st = run_topk(L, n, p.logits, topk_idx, topk_w, s);
    if (st == BURNEXT_OK)
      st = run_dispatch(L, n, topk_idx, seg_offsets, perm, p.pos_of, active, num_active, p.exrec, p.dcnt, s);
  }
  return st == BURNEXT_OK ? ok() : st;
}

burnext_status burnext_mxfp4_dequant(const burnext_mxfp4_desc *desc, const uint8_t *blocks, const uint8_t *scales,
                                     void *out, burnext_dtype out_dtype, void *stream) {
  if (!desc || !blocks || !scales || !out) return fail(BURNEXT_INVALID_ARG, "null descriptor or buffer");
  if (out_dtype != BURNEXT_F32 && out_dtype != BURNEXT_BF16) return fail(BURNEXT_INVALID_ARG, "bad out_dtype");
  if (desc->bpr != cdiv(desc->cols, 2) || desc->gpr != cdiv(desc->cols, 32) || desc->ue8_offset < 0 ||
      desc->ue8_offset > 255)
    return fail(BURNEXT_INVALID_ARG, "descriptor bpr/gpr/ue8_offset inconsistent with cols");
  DequantArgs a{};
  a.blocks = blocks;
  a.scales = scales;
  a.out = out;
  a.rows = desc->experts * desc->rows;
  a.cols = desc->cols;
  a.bpr = desc->bpr;
  a.gpr = desc->gpr;
  a.ue8_offset = desc->ue8_offset;
  a.out_bf16 = out_dtype == BURNEXT_BF16;
  burnext_status st = check_launch(launch_dequant(a, (hipStream_t)stream), "dequant launch");
  return st == BURNEXT_OK ? ok() : st;
}

burnext_status burnext_moe_profile_enable(burnext_moe_layer_t L, int enable) {
  if (!L) return fail(BURNEXT_INVALID_ARG, "layer is null");
  L->profiling = enable != 0;
  if (enable) {
    Profiler &P = profiler();
    std::lock_guard<std::mutex> lk(P.mu);
    if (P.pending.empty()) {  // nothing refers to the read pairs any more: reuse them
      for (auto &r : P.done) P.pool[r.device].push_back({r.a, r.b});
      P.done.clear();
      P.last_end.clear();
    }
  }
  return ok();
}

burnext_status burnext_moe_profile_read(burnext_moe_layer_t L, double *ms_total, uint64_t *launches, int n_kernels) {
  if (!L || !ms_total || !launches || n_kernels < 0) return fail(BURNEXT_INVALID_ARG, "null argument");
  for (int k = 0; k < n_kernels; ++k) {
    ms_total[k] = 0.0;
    launches[k] = 0;
  }
  Profiler &P = profiler();
  std::vector<ProfRec> mine;
  {
    std::lock_guard<std::mutex> lk(P.mu);
    for (size_t i = 0; i < P.pending.size();)
      if (P.pending[i].layer == L) {
        mine.push_back(P.pending[i]);
        P.pending.erase(P.pending.begin() + (std::ptrdiff_t)i);
      } else {
        ++i;
      }
  }
  DeviceGuard guard(L->device);
  burnext_status st = BURNEXT_OK;
  for (auto &r : mine) {
    float ms = 0.0f, gap = 0.0f;
    if (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess)
      st = BURNEXT_DEVICE_ERROR;
    // exclusive part: not before the previous timed dispatch on the stream ended
    if (r.prev_end && hipEventElapsedTime(&gap, r.prev_end, r.b) == hipSuccess && gap >= 0.0f && gap < ms) ms = gap;
    if (r.kernel >= 0 && r.kernel < n_kernels) {
      ms_total[r.kernel] += ms;
      launches[r.kernel] += 1;
    }
  }
  {
    std::lock_guard<std::mutex> lk(P.mu);
    P.done.insert(P.done.end(), mine.begin(), mine.end());
  }
  if (st != BURNEXT_OK) return fail(st, "event synchronisation failed");
  return ok();
}

}  // extern "C"
