// decoder.hip -- GPT-OSS decoder decode step on gfx950 around the MoE layer (include/burnext_gptoss.h).
//
// Per decode step (batch rows b < B, one token each, absolute position pos):
//   embed_kernel        hidden[b] = tok_emb[token[b]]                       (f32 residual stream)
//   per layer l:
//     rmsnorm_kernel    xn = RmsNorm(hidden) with norm_attn[l] (layer 0; see the MoE combine below)
//     dense_gemv_kernel the fused q|k|v projection as K-part partial sums (bf16 weights on
//                       v_mfma_f32_16x16x32_bf16, activations as two bf16 terms)
//     qkv_post_kernel   sum of parts + bias, RoPE on q and k (YaRN table), k and v written into the
//                       rolling cache at slot pos mod cache_len
//     attn_chunk_kernel one query row per head against 256 cached keys per workgroup: chunk
//                       maximum, exp, sums and the weighted value sum (flash-decoding split)
//     attn_combine_kernel  chunks merged with the learned sink in the softmax denominator (a layer
//                       whose window is one chunk merges it in the attention launch itself)
//     dense_gemv_kernel the output projection; o_post_kernel hidden += sum + bias (where the MoE
//                       router cannot: router_front_kernel forms that row itself for decode batches)
//     burnext_moe_forward  the MoE layer (its own RmsNorm and residual) on the HIP MoE kernels;
//                       its combine (combine_norm_kernel) also writes the next layer's xn (after
//                       the last layer: norm_final), so rmsnorm_kernel runs for layer 0 only
//   LM head: lm_stream_kernel (equal runs of the tiled matrix per wave, logits and each
//                       workgroup's best per row) + lm_fix_kernel (the tiles cut between runs) for
//                       batches of at most 8 rows, else dense_gemv_kernel + logits_kernel; then
//                       argmax_kernel
//
// Replaces src/models/gpt_oss.rs:101-113,226-252 and src/attention/streaming_mqa.rs:239-419
// (Burn tensor ops on WGPU).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "../../include/burnext_gptoss.h"
#include "kernels.hpp"
#include "mx_device.hpp"

struct burnext_moe_layer;

namespace burnext {
burnext_status set_error(burnext_status st, const std::string &msg);
void moe_layer_shape(const burnext_moe_layer *L, uint32_t *d_model, int *device);
burnext_status moe_forward_post_norm(burnext_moe_layer *L, const void *x, burnext_dtype x_dtype, void *y, uint64_t n,
                                     uint32_t flags, void *workspace, uint64_t ws_bytes, void *stream,
                                     const float *gamma, float eps, float *xn, bool *norm_done, const float *part,
                                     uint64_t part_stride, uint32_t nparts, const float *bias, const float *resid,
                                     bool experts_bf16);
bool moe_front_fusable(const burnext_moe_layer *L, uint64_t n, uint32_t nparts);
}  // namespace burnext

using namespace burnext;

namespace {

constexpr uint32_t kDenseMaxH = 16;   // K-groups (32 inputs each) per GEMV work unit
constexpr uint32_t kDenseWaves = 8;   // row tiles (one per wave) per GEMV workgroup
constexpr uint32_t kAttnChunk = 256;  // cached keys per attention workgroup
constexpr uint32_t kMaxGroups = 16;   // query heads per kv head
constexpr uint32_t kMaxHeadDim = 128;
constexpr uint32_t kMaxBatch = 16;
constexpr uint32_t kLogitsPerBlock = 1024;
constexpr int32_t kNoIndex = 0x7fffffff;

// ---------------------------------------------------------------------------------------------
// Cache rows: f32 (the reference's element) or bf16.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void kv_store2(float *p, float a, float b) { *(float2 *)p = make_float2(a, b); }
__device__ __forceinline__ void kv_store2(uint16_t *p, float a, float b) {
  *(uint32_t *)p = (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
}
__device__ __forceinline__ void kv_store1(float *p, float a) { *p = a; }
__device__ __forceinline__ void kv_store1(uint16_t *p, float a) { *p = f32_to_bf16_bits(a); }
__device__ __forceinline__ void kv_load4(const float *p, float (&v)[4]) {
  const float4 x = *(const float4 *)p;
  v[0] = x.x;
  v[1] = x.y;
  v[2] = x.z;
  v[3] = x.w;
}
__device__ __forceinline__ void kv_load4(const uint16_t *p, float (&v)[4]) {
  const uint2 r = *(const uint2 *)p;
  v[0] = bf16_bits_to_f32((uint16_t)r.x);
  v[1] = bf16_bits_to_f32((uint16_t)(r.x >> 16));
  v[2] = bf16_bits_to_f32((uint16_t)r.y);
  v[3] = bf16_bits_to_f32((uint16_t)(r.y >> 16));
}
template <typename KV>
__device__ __forceinline__ void kv_load8(const KV *p, float (&v)[8]) {
  float a[4], b[4];
  kv_load4(p, a);
  kv_load4(p + 4, b);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    v[u] = a[u];
    v[4 + u] = b[u];
  }
}

// Maximum over the 64 lanes of a wave, in every lane (every lane active): lane 0's chain, broadcast.
__device__ __forceinline__ float wave_max(float v) {
  float r[1] = {v};
  wave_max_to_lane0_n<1>(r);
  return lane0_broadcast(r[0]);
}

// Cache layouts of one layer (cap_p = cache_len rounded up to 64 rows).
// K: [maxB][kvH][cap_p / 64][dk / 4][64 rows][4]: the 4-wide dimension quads of 64 consecutive
//    slots are contiguous, so the score phase (one lane per key) reads 16 bytes per lane with
//    consecutive lanes on consecutive addresses.
// V: [maxB][kvH][cap_p][dk] row-major (the value phase reads rows with lanes along dk).
__host__ __device__ __forceinline__ size_t k_index(uint32_t b, uint32_t g, uint32_t slot, uint32_t d, uint32_t kvH,
                                                   uint32_t cap_p, uint32_t dk) {
  return ((((size_t)b * kvH + g) * (cap_p / 64u) + slot / 64u) * (dk / 4u) + d / 4u) * 256u + (slot % 64u) * 4u +
         (d % 4u);
}
__host__ __device__ __forceinline__ size_t v_index(uint32_t b, uint32_t g, uint32_t slot, uint32_t d, uint32_t kvH,
                                                   uint32_t cap_p, uint32_t dk) {
  return (((size_t)b * kvH + g) * cap_p + slot) * dk + d;
}

// ---------------------------------------------------------------------------------------------
// Dense decode GEMV.  Weights W [N, K] bf16, repacked at create into tiles of 16 rows x 32
// inputs (1 KiB): tile t, K-group kg at (t * nkg + kg) KiB, lane l = 16 q + i holding
// W[16 t + i][32 kg + 8 q .. +8] -- the A operand of v_mfma_f32_16x16x32_bf16 for one K step.
// Workgroup (x, h): NW waves, row tiles NW x .. NW x + NW - 1, K-groups [h H, (h + 1) H).  Every wave
// first issues all its H weight loads (16 KiB in flight at H = 16); while they are in flight the
// workgroup stages the B token rows of its K range in LDS as two bf16 terms (hi, lo = bf16 of the
// residual; together f32-accurate to ~2^-17).  Lanes of token columns >= B feed zeros to the
// MFMA.  2 MFMAs per K-group.  Output: partial sums out[h][b][n] (no bias).  K % 4 == 0.
// ---------------------------------------------------------------------------------------------
struct DenseArgs {
  const uint8_t *w;
  const float *x;  // [B, K]
  float *out;      // [parts][B][N]
  uint32_t N, K, nkg, ntiles, B, H;
  uint64_t part_stride;
};

template <uint32_t NW>
__global__ __launch_bounds__(NW * 64) void dense_gemv_kernel(DenseArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const uint32_t H = a.H, ldk = H * 32u + 8u;  // +8: consecutive token rows start on other banks
  uint16_t *bs = (uint16_t *)smem;             // [2 terms][16 tokens][ldk]
  const uint32_t h = blockIdx.y, kg0 = h * H, kg1 = min(kg0 + H, a.nkg), nk = kg1 - kg0;
  const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
  const uint32_t tile = blockIdx.x * NW + wv;
  const bool tv = tile < a.ntiles;  // wave-uniform
  const uint32_t tl = tv ? tile : a.ntiles - 1u;
  // activation quads of rows j < B in this K range (at most 16 x 16 x 8 / 256 = 8 per thread),
  // requested before the weights: the in-order load counter then lets the staging wait for
  // them alone
  const uint32_t k0 = kg0 * 32u, kq = nk * 8u;  // quads per row
  constexpr uint32_t kXq = 16u * kDenseMaxH * 8u / (NW * 64u);
  float4 xv[kXq];
#pragma unroll
  for (uint32_t u = 0; u < kXq; ++u) {
    const uint32_t i = threadIdx.x + u * NW * 64u, j = i / kq, qq = i - j * kq, k = k0 + 4u * qq;
    xv[u] = (i < a.B * kq && k < a.K) ? *(const float4 *)(a.x + (size_t)j * a.K + k) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  uint4 wbuf[kDenseMaxH];
  const uint8_t *wt = a.w + ((size_t)tl * a.nkg + kg0) * 1024u + lane * 16u;
#pragma unroll
  for (uint32_t s = 0; s < kDenseMaxH; ++s)  // unconditional (clamped): a static count of loads in flight
    wbuf[s] = load_stream16(wt + (size_t)min(s, nk - 1u) * 1024u);
#pragma unroll
  for (uint32_t u = 0; u < kXq; ++u) {
    const uint32_t i = threadIdx.x + u * NW * 64u, j = i / kq, qq = i - j * kq;
    if (i >= a.B * kq) continue;
    const float vv[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
    uint32_t hi[2], lo[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      uint32_t tp[2];
      split_bf16x2<2>(vv[2 * u], vv[2 * u + 1], tp);
      hi[u] = tp[0];
      lo[u] = tp[1];
    }
    *(uint2 *)(bs + (size_t)j * ldk + 4u * qq) = make_uint2(hi[0], hi[1]);
    *(uint2 *)(bs + (size_t)(16u + j) * ldk + 4u * qq) = make_uint2(lo[0], lo[1]);
  }
  __syncthreads();
  const uint32_t i16 = lane & 15u, q = lane >> 4;
  const bool bok = i16 < a.B;
  const u32x4_t zero = {0u, 0u, 0u, 0u};
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (uint32_t s = 0; s < kDenseMaxH; ++s) {
    if (s < nk) {
      const bf16x8_t A = __builtin_bit_cast(bf16x8_t, wbuf[s]);
#pragma unroll
      for (uint32_t term = 0; term < 2u; ++term) {
        const u32x4_t raw = bok ? *(const u32x4_t *)(bs + (size_t)(term * 16u + i16) * ldk + 32u * s + 8u * q) : zero;
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8_t, raw), acc, 0, 0, 0);
      }
    }
  }
  if (!tv || !bok) return;
  float *o = a.out + (size_t)h * a.part_stride + (size_t)i16 * a.N;
  const uint32_t r0 = tile * 16u + 4u * q;
#pragma unroll
  for (uint32_t r = 0; r < 4u; ++r)
    if (r0 + r < a.N) o[r0 + r] = acc[r];
}

// ---------------------------------------------------------------------------------------------
// q|k|v post-processing: one thread per pair (2 i, 2 i + 1) of one head of one batch row.
// Sum of the K-part partials plus bias; RoPE for q and k: pair i of head hh at position
// pos + hh * head_stride rotated by table[p][i] = (cos, sin) x concentration:
//   y0 = x0 c - x1 s, y1 = x1 c + x0 s   (Burn RotaryEncoding, interleaved pairs)
// q goes to qbuf [B][nH dk] (f32); k and v to the cache at slot (k_index / v_index layouts).
// ---------------------------------------------------------------------------------------------
struct QkvPostArgs {
  const float *part;  // [parts][B][qd + 2 kd]
  uint64_t part_stride;
  uint32_t parts;
  const float *bias;  // [qd + 2 kd]
  const float *rope;  // [npos][dk / 2][2]
  float *qbuf;        // [B][nH * dk]
  void *kc, *vc;      // this layer's cache
  uint32_t B, nH, kvH, dk, cap_p, slot, pos, head_stride;
};

// P > 0: exactly P parts, all of a thread's loads (its P part pairs, bias pair and RoPE pair)
// requested before any is used -- one memory round trip (a loop over a run-time part count waits
// for each part in turn); P = 0: a.parts parts in a loop.
template <typename KV, uint32_t P>
__global__ __launch_bounds__(256) void qkv_post_kernel(QkvPostArgs a) {
  const uint32_t b = blockIdx.y, qd = a.nH * a.dk, kd = a.kvH * a.dk, N = qd + 2u * kd;
  const uint32_t pr = blockIdx.x * blockDim.x + threadIdx.x;
  if (pr >= N / 2u) return;
  const uint32_t o = 2u * pr;
  const uint32_t half = a.dk / 2u;
  const bool rot = o < qd + kd;  // q or k: rotate
  const uint32_t local = o < qd ? o : (rot ? o - qd : o - qd - kd), hh = local / a.dk, i = (local - hh * a.dk) / 2u;
  const uint32_t p = a.pos + hh * a.head_stride;
  float2 cs = make_float2(1.0f, 0.0f);
  float s0 = 0.0f, s1 = 0.0f;
  const float *pp = a.part + (size_t)b * N + o;
  if constexpr (P > 0) {
    float2 pv[P];
#pragma unroll
    for (uint32_t h = 0; h < P; ++h) pv[h] = *(const float2 *)(pp + (size_t)h * a.part_stride);
    const float2 bv = *(const float2 *)(a.bias + o);
    const float2 csl = *(const float2 *)(a.rope + ((size_t)p * half + i) * 2u);  // in the table for v rows too
    if (rot) cs = csl;
#pragma unroll
    for (uint32_t h = 0; h < P; ++h) {
      s0 = s0 + pv[h].x;
      s1 = s1 + pv[h].y;
    }
    s0 = s0 + bv.x;
    s1 = s1 + bv.y;
  } else {
    for (uint32_t h = 0; h < a.parts; ++h) {
      const float2 v = *(const float2 *)(pp + (size_t)h * a.part_stride);
      s0 = s0 + v.x;
      s1 = s1 + v.y;
    }
    s0 = s0 + a.bias[o];
    s1 = s1 + a.bias[o + 1u];
    if (rot) cs = *(const float2 *)(a.rope + ((size_t)p * half + i) * 2u);
  }
  const float x0 = s0, x1 = s1;
  KV *kc = (KV *)a.kc, *vc = (KV *)a.vc;
  if (rot) {
    const float y0 = x0 * cs.x - x1 * cs.y, y1 = x1 * cs.x + x0 * cs.y;
    if (o < qd) {
      *(float2 *)(a.qbuf + (size_t)b * qd + local) = make_float2(y0, y1);
    } else {
      kv_store2(kc + k_index(b, hh, a.slot, local - hh * a.dk, a.kvH, a.cap_p, a.dk), y0, y1);
    }
  } else {
    const uint32_t local = o - qd - kd, hh = local / a.dk;
    kv_store2(vc + v_index(b, hh, a.slot, local - hh * a.dk, a.kvH, a.cap_p, a.dk), x0, x1);
  }
}

template <typename KV>
hipError_t launch_qkv_post(const QkvPostArgs &a, dim3 grid, hipStream_t s) {
  switch (a.parts) {  // the part counts dense_plan gives (1 .. 8 at d_model <= 4096): one round trip
    case 1: return launch_kernel(qkv_post_kernel<KV, 1>, grid, dim3(256), 0, s, a);
    case 2: return launch_kernel(qkv_post_kernel<KV, 2>, grid, dim3(256), 0, s, a);
    case 3: return launch_kernel(qkv_post_kernel<KV, 3>, grid, dim3(256), 0, s, a);
    case 4: return launch_kernel(qkv_post_kernel<KV, 4>, grid, dim3(256), 0, s, a);
    case 5: return launch_kernel(qkv_post_kernel<KV, 5>, grid, dim3(256), 0, s, a);
    case 6: return launch_kernel(qkv_post_kernel<KV, 6>, grid, dim3(256), 0, s, a);
    case 7: return launch_kernel(qkv_post_kernel<KV, 7>, grid, dim3(256), 0, s, a);
    case 8: return launch_kernel(qkv_post_kernel<KV, 8>, grid, dim3(256), 0, s, a);
    default: return launch_kernel(qkv_post_kernel<KV, 0>, grid, dim3(256), 0, s, a);
  }
}

// ---------------------------------------------------------------------------------------------
// Attention, flash-decoding split.  Workgroup (chunk c, kv head g, batch b) covers positions
// keys i = 256 c + t (t < 256, i < nkeys) of the active window (slots by key_slot), for the G
// query heads of kv head g.
//   scores: thread t, s[j] = (q[j] . k[p]) / sqrt(scale_dk) (q broadcast from LDS, k in
//     dimension quads from the tiled K layout)
//   m[j] = chunk maximum (wave maxima, then the 4 waves), e = exp(s - m) (0 outside the window),
//   l[j] = sum of e (wave butterflies, then the 4 waves in order)
//   acc[j][d] = sum of e v: thread (key lane kq = t / 16, dim quad dq = t % 16) takes keys
//     kq, kq + 16, ... in order, the 4 key lanes of a wave are summed by shuffles and the 4 waves
//     in order through LDS
// Output: part[b][g][c][j] = {m, l, acc[dk]}.
// ---------------------------------------------------------------------------------------------
struct AttnArgs {
  const float *q;        // [B][nH * dk]
  const void *kc, *vc;   // this layer's cache
  float *part;           // [B][kvH][nchunk][groups][dk + 2]
  uint32_t nH, kvH, dk, cap_p, nchunk;
  // the active window's keys i < nkeys: the sink rows first (i < nsk: slot sk_lo + i, holding
  // position sk_lo + i), then the recent positions p_lo + (i - nsk) at their ring slots;
  // p_mod = (p_lo - sink) mod ring (the recent keys are at most ring)
  uint32_t nkeys, nsk, sk_lo, p_mod, sink, ring;  // ring = cache_len - sink
  float inv_scale;       // 1 / sqrt(scale_dk)
  // one chunk (attn_chunk64_kernel only): the sink merge in the same launch, ctx written directly
  // (null: the chunk partials go to part for attn_combine_kernel)
  float *ctx;            // [B][nH * dk]
  const float *sinks;    // [nH] or null
};

// Cache slot of key i of the active window.  The cache keeps the first `sink` positions in slots
// 0 .. sink - 1 and every later position p in slot sink + (p - sink) mod (cache_len - sink): the
// rows the reference's evict-and-roll keeps (src/attention/cache_ops.rs:64-117), without moving
// any row (sink = 0: slot p mod cache_len).
__device__ __forceinline__ uint32_t key_slot(const AttnArgs &a, uint32_t i) {
  const uint32_t r = a.p_mod + (i - a.nsk);  // < 2 ring: p_mod < ring, i - nsk < ring
  return i < a.nsk ? a.sk_lo + i : a.sink + (r >= a.ring ? r - a.ring : r);
}

template <typename KV, uint32_t G>
__global__ __launch_bounds__(256) void attn_chunk_kernel(AttnArgs a) {
  __shared__ __align__(16) float q_l[kMaxGroups * kMaxHeadDim];   // 8 KiB
  __shared__ float e_l[kAttnChunk * kMaxGroups];                  // 16 KiB: e[key][j]
  __shared__ float m_l[4 * kMaxGroups], l_l[4 * kMaxGroups];
  __shared__ __align__(16) float acc_l[4 * kMaxGroups * 16 * 4];  // [wave][j][dq][4]: 16 KiB
  const uint32_t c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const uint32_t dk = a.dk, nq = dk / 4u, t = threadIdx.x, lane = t & 63u, w = t >> 6;
  const KV *kc = (const KV *)a.kc, *vc = (const KV *)a.vc;
  for (uint32_t i = t; i < G * dk; i += blockDim.x) q_l[i] = a.q[(size_t)b * a.nH * dk + (size_t)g * G * dk + i];
  __syncthreads();
  const uint32_t i0 = c * kAttnChunk, ki = i0 + t;  // this chunk's first key, this thread's key
  const bool valid = ki < a.nkeys;
  float s[G];
#pragma unroll
  for (uint32_t j = 0; j < G; ++j) s[j] = 0.0f;
  {
    // dimension quads in batches of 8 loads in flight (quads past dk and keys outside the window
    // read a valid slot and are not used)
    const KV *kr = kc + k_index(b, g, valid ? key_slot(a, ki) : 0u, 0u, a.kvH, a.cap_p, dk);
    for (uint32_t q0 = 0; q0 < nq; q0 += 8u) {
      float kv[8][4];
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) kv_load4(kr + (size_t)min(q0 + u, nq - 1u) * 256u, kv[u]);
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) {
        if (q0 + u < nq) {
#pragma unroll
          for (uint32_t j = 0; j < G; ++j) {
            const float4 qa = *(const float4 *)(q_l + j * dk + 4u * (q0 + u));
            s[j] = fmaf(qa.x, kv[u][0], s[j]);
            s[j] = fmaf(qa.y, kv[u][1], s[j]);
            s[j] = fmaf(qa.z, kv[u][2], s[j]);
            s[j] = fmaf(qa.w, kv[u][3], s[j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (uint32_t j = 0; j < G; ++j) {
    s[j] = valid ? s[j] * a.inv_scale : -INFINITY;
    const float mw = wave_max(s[j]);
    if (lane == 0) m_l[w * kMaxGroups + j] = mw;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t j = 0; j < G; ++j) {
    const float m = fmaxf(fmaxf(m_l[j], m_l[kMaxGroups + j]), fmaxf(m_l[2u * kMaxGroups + j], m_l[3u * kMaxGroups + j]));
    const float e = valid ? expf(s[j] - m) : 0.0f;
    e_l[t * G + j] = e;
    const float lw = wave_sum_butterfly(e);
    if (lane == 0) l_l[w * kMaxGroups + j] = lw;
  }
  __syncthreads();
  const uint32_t kq = t >> 4, dq = t & 15u;
  const uint32_t nkeys = min(kAttnChunk, a.nkeys - i0);
  float *out = a.part + (((size_t)b * a.kvH + g) * a.nchunk + c) * (size_t)G * (dk + 2u);
  for (uint32_t dbase = 0; dbase < nq; dbase += 16u) {
    const uint32_t dqq = dbase + dq;
    float acc[G][4];
#pragma unroll
    for (uint32_t j = 0; j < G; ++j) acc[j][0] = acc[j][1] = acc[j][2] = acc[j][3] = 0.0f;
    if (dqq < nq) {
      // keys kq + 16 i in batches of 4 loads in flight (past the chunk: a valid row, weight 0)
      for (uint32_t k0 = kq; k0 < nkeys; k0 += 64u) {
        float v[4][4];
#pragma unroll
        for (uint32_t u = 0; u < 4u; ++u) {
          const uint32_t key = min(k0 + 16u * u, nkeys - 1u);
          kv_load4(vc + v_index(b, g, key_slot(a, i0 + key), 4u * dqq, a.kvH, a.cap_p, dk), v[u]);
        }
#pragma unroll
        for (uint32_t u = 0; u < 4u; ++u) {
          const uint32_t key = k0 + 16u * u;
          if (key < nkeys) {
#pragma unroll
            for (uint32_t j = 0; j < G; ++j) {
              const float e = e_l[key * G + j];
              acc[j][0] = fmaf(e, v[u][0], acc[j][0]);
              acc[j][1] = fmaf(e, v[u][1], acc[j][1]);
              acc[j][2] = fmaf(e, v[u][2], acc[j][2]);
              acc[j][3] = fmaf(e, v[u][3], acc[j][3]);
            }
          }
        }
      }
    }
    // the 4 key lanes of a wave (lane bits 4 and 5)
#pragma unroll
    for (uint32_t j = 0; j < G; ++j) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc[j][u] = acc[j][u] + __shfl_xor(acc[j][u], 16, 64);
        acc[j][u] = acc[j][u] + __shfl_xor(acc[j][u], 32, 64);
      }
    }
    if (dbase != 0) __syncthreads();  // the previous pass has read acc_l
    if (lane < 16u) {
#pragma unroll
      for (uint32_t j = 0; j < G; ++j)
        *(float4 *)(acc_l + ((w * kMaxGroups + j) * 16u + dq) * 4u) = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
    }
    __syncthreads();
    for (uint32_t i = t; i < G * 16u; i += blockDim.x) {
      const uint32_t j = i >> 4, dd = i & 15u;
      if (dbase + dd >= nq) continue;
      float4 r = *(const float4 *)(acc_l + (j * 16u + dd) * 4u);
#pragma unroll
      for (uint32_t w2 = 1; w2 < 4u; ++w2) {
        const float4 v = *(const float4 *)(acc_l + ((w2 * kMaxGroups + j) * 16u + dd) * 4u);
        r = make_float4(r.x + v.x, r.y + v.y, r.z + v.z, r.w + v.w);
      }
      float *dst = out + (size_t)j * (dk + 2u) + 2u + 4u * (dbase + dd);
      dst[0] = r.x;
      dst[1] = r.y;
      dst[2] = r.z;
      dst[3] = r.w;
    }
  }
  if (t < G) {
    out[(size_t)t * (dk + 2u)] =
        fmaxf(fmaxf(m_l[t], m_l[kMaxGroups + t]), fmaxf(m_l[2u * kMaxGroups + t], m_l[3u * kMaxGroups + t]));
    out[(size_t)t * (dk + 2u) + 1u] = (l_l[t] + l_l[kMaxGroups + t]) + (l_l[2u * kMaxGroups + t] + l_l[3u * kMaxGroups + t]);
  }
}

// Raw cache quads (4 values), loaded now and converted at use so that the loads stay in flight.
template <typename KV> struct RawQ;
template <> struct RawQ<float> { float4 v; };
template <> struct RawQ<uint16_t> { uint2 v; };
// cache rows are read once per step: nontemporal loads
__device__ __forceinline__ void raw_load(const float *p, RawQ<float> &r) {
  const f32x4_t v = __builtin_nontemporal_load((const f32x4_t *)p);
  r.v = make_float4(v[0], v[1], v[2], v[3]);
}
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void raw_load(const uint16_t *p, RawQ<uint16_t> &r) {
  const u32x2_t v = __builtin_nontemporal_load((const u32x2_t *)p);
  r.v = make_uint2(v[0], v[1]);
}
__device__ __forceinline__ void raw_vals(const RawQ<float> &r, float (&v)[4]) {
  v[0] = r.v.x;
  v[1] = r.v.y;
  v[2] = r.v.z;
  v[3] = r.v.w;
}
__device__ __forceinline__ void raw_vals(const RawQ<uint16_t> &r, float (&v)[4]) {
  v[0] = bf16_bits_to_f32((uint16_t)r.v.x);
  v[1] = bf16_bits_to_f32((uint16_t)(r.v.x >> 16));
  v[2] = bf16_bits_to_f32((uint16_t)r.v.y);
  v[3] = bf16_bits_to_f32((uint16_t)(r.v.y >> 16));
}

// G consecutive floats of LDS (16-byte aligned for G >= 4, 8-byte for G = 2) in the widest
// accesses that fit.
template <uint32_t G>
__device__ __forceinline__ void lds_store_g(float *p, const float (&v)[G]) {
  if constexpr (G >= 4) {
#pragma unroll
    for (uint32_t j = 0; j < G; j += 4u) *(float4 *)(p + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
  } else if constexpr (G == 2) {
    *(float2 *)p = make_float2(v[0], v[1]);
  } else {
    p[0] = v[0];
  }
}
template <uint32_t G>
__device__ __forceinline__ void lds_load_g(const float *p, float (&v)[G]) {
  if constexpr (G >= 4) {
#pragma unroll
    for (uint32_t j = 0; j < G; j += 4u) {
      const float4 x = *(const float4 *)(p + j);
      v[j] = x.x;
      v[j + 1] = x.y;
      v[j + 2] = x.z;
      v[j + 3] = x.w;
    }
  } else if constexpr (G == 2) {
    const float2 x = *(const float2 *)p;
    v[0] = x.x;
    v[1] = x.y;
  } else {
    v[0] = p[0];
  }
}

// The same chunk as attn_chunk_kernel for head_dim <= 64 and G <= 8: every thread requests its q
// quad and its key's (up to) 16 K quads before waiting for any of them, and the 16 value quads its
// (key lane kq, dim quad dq) slot of the value phase needs as soon as its scores have consumed the
// K quads -- K and V never held at once, so 4 workgroups share a CU (118 VGPRs) and a full
// layer's 2 048 workgroups run in 2 rounds instead of 2.7 at 3 per CU (decoder step 3.505 ->
// 3.489 ms against requesting the value quads with the K quads).  Keys past the window and quads
// past head_dim read a valid slot and are not used.  Same arithmetic order as attn_chunk_kernel.
template <typename KV, uint32_t G>
__global__ __launch_bounds__(256, 4) void attn_chunk64_kernel(AttnArgs a) {
  __shared__ __align__(16) float q_l[G * 64];
  __shared__ __align__(16) float e_l[kAttnChunk * G];
  __shared__ float m_l[4 * G], l_l[4 * G];
  __shared__ __align__(16) float acc_l[4 * G * 16 * 4];  // [wave][j][dq][4]
  const uint32_t c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const uint32_t dk = a.dk, nq = dk / 4u, t = threadIdx.x, lane = t & 63u, w = t >> 6;
  const KV *kc = (const KV *)a.kc, *vc = (const KV *)a.vc;
  const uint32_t i0 = c * kAttnChunk, ki = i0 + t;  // this chunk's first key, this thread's key
  const bool valid = ki < a.nkeys;
  const uint32_t nkeys = min(kAttnChunk, a.nkeys - i0);
  // requests: q quad, K quads, value quads
  const uint32_t nqq = G * nq;  // q quads of this kv head's G query heads (<= 128)
  const float *qsrc = a.q + (size_t)b * a.nH * dk + (size_t)g * G * dk;
  const float4 qv = *(const float4 *)(qsrc + 4u * min(t, nqq - 1u));
  __builtin_amdgcn_sched_barrier(0);  // q first: its wait then leaves the K and V loads in flight
  RawQ<KV> kr[16];
  const KV *kb = kc + k_index(b, g, key_slot(a, valid ? ki : i0), 0u, a.kvH, a.cap_p, dk);
#pragma unroll
  for (uint32_t u = 0; u < 16u; ++u) raw_load(kb + (size_t)min(u, nq - 1u) * 256u, kr[u]);
  const uint32_t kq = t >> 4, dq = t & 15u, dqc = min(dq, nq - 1u);
  if (t < nqq) *(float4 *)(q_l + 4u * t) = qv;
  __syncthreads();
  float s[G];
#pragma unroll
  for (uint32_t j = 0; j < G; ++j) s[j] = 0.0f;
#pragma unroll
  for (uint32_t u = 0; u < 16u; ++u) {
    if (u < nq) {
      float k4[4];
      raw_vals(kr[u], k4);
#pragma unroll
      for (uint32_t j = 0; j < G; ++j) {
        const float4 qa = *(const float4 *)(q_l + j * dk + 4u * u);
        s[j] = fmaf(qa.x, k4[0], s[j]);
        s[j] = fmaf(qa.y, k4[1], s[j]);
        s[j] = fmaf(qa.z, k4[2], s[j]);
        s[j] = fmaf(qa.w, k4[3], s[j]);
      }
    }
  }
  // the value quads, requested once the scores hold what the K quads gave
  __builtin_amdgcn_sched_barrier(0);
  RawQ<KV> vr[16];
#pragma unroll
  for (uint32_t i = 0; i < 16u; ++i) {
    const uint32_t key = min(kq + 16u * i, nkeys - 1u);
    raw_load(vc + v_index(b, g, key_slot(a, i0 + key), 4u * dqc, a.kvH, a.cap_p, dk), vr[i]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // wave maxima and sums of the G heads: lane-0 reductions, the G chains interleaved
  float red[G];
#pragma unroll
  for (uint32_t j = 0; j < G; ++j) {
    s[j] = valid ? s[j] * a.inv_scale : -INFINITY;
    red[j] = s[j];
  }
  wave_max_to_lane0_n<(int)G>(red);
  if (lane == 0) {
#pragma unroll
    for (uint32_t j = 0; j < G; ++j) m_l[w * G + j] = red[j];
  }
  __syncthreads();
  float e[G];
#pragma unroll
  for (uint32_t j = 0; j < G; ++j) {
    const float m = fmaxf(fmaxf(m_l[j], m_l[G + j]), fmaxf(m_l[2u * G + j], m_l[3u * G + j]));
    e[j] = valid ? expf(s[j] - m) : 0.0f;
    red[j] = e[j];
  }
  lds_store_g<G>(e_l + t * G, e);
  wave_sum_to_lane0_n<(int)G>(red);
  if (lane == 0) {
#pragma unroll
    for (uint32_t j = 0; j < G; ++j) l_l[w * G + j] = red[j];
  }
  __syncthreads();
  float acc[G][4];
#pragma unroll
  for (uint32_t j = 0; j < G; ++j) acc[j][0] = acc[j][1] = acc[j][2] = acc[j][3] = 0.0f;
  // no branch: keys past the window have e = 0 and their (clamped) value quads are zeroed, so
  // they add +0; quads past head_dim are never written out
#pragma unroll
  for (uint32_t i = 0; i < 16u; ++i) {
    const uint32_t key = kq + 16u * i;
    float v4[4], ek[G];
    raw_vals(vr[i], v4);
#pragma unroll
    for (int u = 0; u < 4; ++u) v4[u] = key < nkeys ? v4[u] : 0.0f;
    lds_load_g<G>(e_l + key * G, ek);
#pragma unroll
    for (uint32_t j = 0; j < G; ++j) {
      acc[j][0] = fmaf(ek[j], v4[0], acc[j][0]);
      acc[j][1] = fmaf(ek[j], v4[1], acc[j][1]);
      acc[j][2] = fmaf(ek[j], v4[2], acc[j][2]);
      acc[j][3] = fmaf(ek[j], v4[3], acc[j][3]);
    }
  }
  // the 4 key lanes of the wave (lanes dq, dq + 16, dq + 32, dq + 48): lane dq gets
  // (a[dq] + a[dq + 16]) + (a[dq + 32] + a[dq + 48]) by permlane swaps
#pragma unroll
  for (uint32_t j = 0; j < G; ++j) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[j][u]), __float_as_uint(acc[j][u]), false, false);
      acc[j][u] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
  }
#pragma unroll
  for (uint32_t j = 0; j < G; ++j) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[j][u]), __float_as_uint(acc[j][u]), false, false);
      acc[j][u] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
  }
  if (lane < 16u) {
#pragma unroll
    for (uint32_t j = 0; j < G; ++j)
      *(float4 *)(acc_l + ((w * G + j) * 16u + dq) * 4u) = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
  }
  __syncthreads();
  if (a.ctx != nullptr) {
    // the only chunk: attn_combine_kernel's arithmetic for one chunk -- M = max(sink, m),
    // f = exp(m - M), 1 / L = 1 / (l f + exp(sink - M)), ctx = (acc f) (1 / L)
    for (uint32_t i = t; i < G * 16u; i += blockDim.x) {
      const uint32_t j = i >> 4, dd = i & 15u;
      if (dd >= nq) continue;
      float4 r = *(const float4 *)(acc_l + (j * 16u + dd) * 4u);
#pragma unroll
      for (uint32_t w2 = 1; w2 < 4u; ++w2) {
        const float4 v = *(const float4 *)(acc_l + ((w2 * G + j) * 16u + dd) * 4u);
        r = make_float4(r.x + v.x, r.y + v.y, r.z + v.z, r.w + v.w);
      }
      const float m = fmaxf(fmaxf(m_l[j], m_l[G + j]), fmaxf(m_l[2u * G + j], m_l[3u * G + j]));
      const float l = (l_l[j] + l_l[G + j]) + (l_l[2u * G + j] + l_l[3u * G + j]);
      const float sink = a.sinks ? a.sinks[g * G + j] : -INFINITY;
      const float M = fmaxf(sink, m);
      const float f = expf(m - M);
      const float rinv = 1.0f / (__fmul_rn(l, f) + (a.sinks ? expf(sink - M) : 0.0f));
      float *dst = a.ctx + (size_t)b * a.nH * dk + (size_t)(g * G + j) * dk + 4u * dd;
      *(float4 *)dst = make_float4(__fmul_rn(r.x, f) * rinv, __fmul_rn(r.y, f) * rinv, __fmul_rn(r.z, f) * rinv,
                                   __fmul_rn(r.w, f) * rinv);
    }
    return;
  }
  float *out = a.part + (((size_t)b * a.kvH + g) * a.nchunk + c) * (size_t)G * (dk + 2u);
  for (uint32_t i = t; i < G * 16u; i += blockDim.x) {
    const uint32_t j = i >> 4, dd = i & 15u;
    if (dd >= nq) continue;
    float4 r = *(const float4 *)(acc_l + (j * 16u + dd) * 4u);
#pragma unroll
    for (uint32_t w2 = 1; w2 < 4u; ++w2) {
      const float4 v = *(const float4 *)(acc_l + ((w2 * G + j) * 16u + dd) * 4u);
      r = make_float4(r.x + v.x, r.y + v.y, r.z + v.z, r.w + v.w);
    }
    float *dst = out + (size_t)j * (dk + 2u) + 2u + 4u * dd;
    dst[0] = r.x;
    dst[1] = r.y;
    dst[2] = r.z;
    dst[3] = r.w;
  }
  if (t < G) {
    out[(size_t)t * (dk + 2u)] = fmaxf(fmaxf(m_l[t], m_l[G + t]), fmaxf(m_l[2u * G + t], m_l[3u * G + t]));
    out[(size_t)t * (dk + 2u) + 1u] = (l_l[t] + l_l[G + t]) + (l_l[2u * G + t] + l_l[3u * G + t]);
  }
}

// Chunks merged with the sink (src/attention/core.rs:34-55): per head j, M = max(sink, max_c m_c),
// f_c = exp(m_c - M), L = exp(sink - M) + sum_c l_c f_c; ctx[d] = sum_c acc_c[d] f_c / L.
// Workgroup (kv head g, batch b): wave w takes heads w, w + 4, ... with lanes over chunks (wave
// max / butterfly sums, chunks lane-strided in order), f in LDS; then threads over (head, dim
// pair) sum the chunks in order.  Dynamic LDS: (nchunk * groups + groups) floats.
struct CombineAttnArgs {
  const float *part;   // [B][kvH][nchunk][groups][dk + 2]
  const float *sinks;  // [nH] or null
  float *ctx;          // [B][nH * dk]
  uint32_t nH, kvH, dk, nchunk;
};

__global__ __launch_bounds__(256) void attn_combine_kernel(CombineAttnArgs a) {
  extern __shared__ float cl[];  // f[nchunk][groups], then 1/L[groups]
  const uint32_t g = blockIdx.x, b = blockIdx.y, groups = a.nH / a.kvH, dk = a.dk, rec = dk + 2u;
  const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6, nc = a.nchunk;
  const float *base = a.part + ((size_t)b * a.kvH + g) * nc * (size_t)groups * rec;
  float *rinv = cl + (size_t)nc * groups;
  for (uint32_t j = w; j < groups; j += 4u) {
    const float sink = a.sinks ? a.sinks[g * groups + j] : -INFINITY;
    float M = sink;
    for (uint32_t c = lane; c < nc; c += 64u) M = fmaxf(M, base[((size_t)c * groups + j) * rec]);
    M = wave_max(M);
    float L = 0.0f;
    for (uint32_t c = lane; c < nc; c += 64u) {
      const float *pc = base + ((size_t)c * groups + j) * rec;
      const float f = expf(pc[0] - M);
      cl[c * groups + j] = f;
      L = L + pc[1] * f;
    }
    L = wave_sum_butterfly(L);
    if (lane == 0) rinv[j] = 1.0f / (L + (a.sinks ? expf(sink - M) : 0.0f));
  }
  __syncthreads();
  const uint32_t half = dk / 2u;
  for (uint32_t i = t; i < groups * half; i += blockDim.x) {
    const uint32_t j = i / half, d = 2u * (i - j * half);
    float ax = 0.0f, ay = 0.0f;
#pragma unroll 8
    for (uint32_t c = 0; c < nc; ++c) {
      const float f = cl[c * groups + j];
      const float2 v = *(const float2 *)(base + ((size_t)c * groups + j) * rec + 2u + d);
      ax = fmaf(v.x, f, ax);
      ay = fmaf(v.y, f, ay);
    }
    const float r = rinv[j];
    *(float2 *)(a.ctx + (size_t)b * a.nH * dk + (size_t)(g * groups + j) * dk + d) = make_float2(ax * r, ay * r);
  }
}

// hidden[b][n] += sum of the K-part partials + bias (the attention residual).
struct OPostArgs {
  const float *part;
  uint64_t part_stride;
  uint32_t parts, N;
  const float *bias;
  float *hidden;
};
__global__ __launch_bounds__(256) void o_post_kernel(OPostArgs a) {
  const uint32_t b = blockIdx.y, n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= a.N) return;
  float s = 0.0f;
  for (uint32_t h = 0; h < a.parts; ++h) s = s + a.part[(size_t)h * a.part_stride + (size_t)b * a.N + n];
  a.hidden[(size_t)b * a.N + n] = a.hidden[(size_t)b * a.N + n] + (s + a.bias[n]);
}

// y[b] = x[b] / sqrt(mean(x[b]^2) + eps) * gamma (Burn RmsNorm); one workgroup per row, D % 4 == 0.
// Rows of up to 4096 values stay in registers between the two passes.
struct NormArgs {
  const float *x;
  const float *gamma;
  float *y;
  uint32_t D;
  float eps;
};
__global__ __launch_bounds__(256) void rmsnorm_kernel(NormArgs a) {
  __shared__ float red[4];
  constexpr uint32_t kR = 4;
  const uint32_t b = blockIdx.x, t = threadIdx.x, nq = a.D / 4u;
  const float4 *x4 = (const float4 *)(a.x + (size_t)b * a.D);
  float4 v[kR];
  float ss = 0.0f;
#pragma unroll
  for (uint32_t r = 0; r < kR; ++r) {
    const uint32_t i = t + r * 256u;
    v[r] = i < nq ? x4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
#pragma unroll
  for (uint32_t r = 0; r < kR; ++r) {
    ss = fmaf(v[r].x, v[r].x, ss);
    ss = fmaf(v[r].y, v[r].y, ss);
    ss = fmaf(v[r].z, v[r].z, ss);
    ss = fmaf(v[r].w, v[r].w, ss);
  }
  for (uint32_t i = t + kR * 256u; i < nq; i += 256u) {
    const float4 u = x4[i];
    ss = fmaf(u.x, u.x, ss);
    ss = fmaf(u.y, u.y, ss);
    ss = fmaf(u.z, u.z, ss);
    ss = fmaf(u.w, u.w, ss);
  }
  ss = wave_sum_butterfly(ss);
  if ((t & 63u) == 0) red[t >> 6] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float rr = sqrtf(tot / (float)a.D + a.eps);
  const float4 *g4 = (const float4 *)a.gamma;
  float4 *y4 = (float4 *)(a.y + (size_t)b * a.D);
#pragma unroll
  for (uint32_t r = 0; r < kR; ++r) {
    const uint32_t i = t + r * 256u;
    if (i < nq) {
      const float4 gg = g4[i];
      y4[i] = make_float4((v[r].x / rr) * gg.x, (v[r].y / rr) * gg.y, (v[r].z / rr) * gg.z, (v[r].w / rr) * gg.w);
    }
  }
  for (uint32_t i = t + kR * 256u; i < nq; i += 256u) {
    const float4 u = x4[i], gg = g4[i];
    y4[i] = make_float4((u.x / rr) * gg.x, (u.y / rr) * gg.y, (u.z / rr) * gg.z, (u.w / rr) * gg.w);
  }
}

// hidden[b] = tok_emb[token[b]]; a token outside [0, V) reads row 0 (the caller keeps tokens in
// range: the reference's embedding lookup fails on them, which device code cannot report here).
struct EmbedArgs {
  const int32_t *tokens;
  const uint16_t *emb;
  float *hidden;
  uint32_t D, V;
};
__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
  const uint32_t b = blockIdx.y, c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= a.D) return;
  const int32_t tk = a.tokens[b];
  const uint32_t row = (tk >= 0 && (uint32_t)tk < a.V) ? (uint32_t)tk : 0u;
  a.hidden[(size_t)b * a.D + c] = bf16_bits_to_f32(a.emb[(size_t)row * a.D + c]);
}

// LM head: logits[b][v] = sum of the K-part partials (written when requested) and the best entry
// of each block of kLogitsPerBlock vocabulary entries (`beats`: larger value, NaN lowest, lower
// index on ties).
struct LogitsArgs {
  const float *part;
  uint64_t part_stride;
  uint32_t parts, V, nblk;
  float *logits;  // [B][V] or null
  float *bval;    // [B][nblk]
  int32_t *bidx;  // [B][nblk]
};

__device__ __forceinline__ void block_best(float &bv, int32_t &bi, float *rv, int32_t *ri) {
  const uint32_t t = threadIdx.x;
  rv[t] = bv;
  ri[t] = bi;
  __syncthreads();
  for (uint32_t st = 128; st >= 1; st >>= 1) {
    if (t < st && ri[t + st] != kNoIndex && (ri[t] == kNoIndex || beats(rv[t + st], ri[t + st], rv[t], ri[t]))) {
      rv[t] = rv[t + st];
      ri[t] = ri[t + st];
    }
    __syncthreads();
  }
  bv = rv[0];
  bi = ri[0];
}

__global__ __launch_bounds__(256) void logits_kernel(LogitsArgs a) {
  __shared__ float rv[256];
  __shared__ int32_t ri[256];
  const uint32_t b = blockIdx.y, t = threadIdx.x;
  float bv = -INFINITY;
  int32_t bi = kNoIndex;
  for (uint32_t u = 0; u < kLogitsPerBlock / 256u; ++u) {
    const uint32_t v = blockIdx.x * kLogitsPerBlock + u * 256u + t;
    if (v >= a.V) break;
    float s = 0.0f;
    for (uint32_t h = 0; h < a.parts; ++h) s = s + a.part[(size_t)h * a.part_stride + (size_t)b * a.V + v];
    if (a.logits) a.logits[(size_t)b * a.V + v] = s;
    if (bi == kNoIndex || beats(s, (int32_t)v, bv, bi)) {
      bv = s;
      bi = (int32_t)v;
    }
  }
  block_best(bv, bi, rv, ri);
  if (t == 0) {
    a.bval[(size_t)b * a.nblk + blockIdx.x] = bv;
    a.bidx[(size_t)b * a.nblk + blockIdx.x] = bi;
  }
}

struct ArgmaxArgs {
  const float *bval;
  const int32_t *bidx;
  uint32_t nblk;
  int32_t *next;
};
__global__ __launch_bounds__(256) void argmax_kernel(ArgmaxArgs a) {
  __shared__ float rv[256];
  __shared__ int32_t ri[256];
  const uint32_t b = blockIdx.x, t = threadIdx.x;
  float bv = -INFINITY;
  int32_t bi = kNoIndex;
  for (uint32_t i = t; i < a.nblk; i += blockDim.x) {
    const float v = a.bval[(size_t)b * a.nblk + i];
    const int32_t ix = a.bidx[(size_t)b * a.nblk + i];
    if (ix != kNoIndex && (bi == kNoIndex || beats(v, ix, bv, bi))) {
      bv = v;
      bi = ix;
    }
  }
  block_best(bv, bi, rv, ri);
  if (t == 0) a.next[b] = bi;
}

// ---------------------------------------------------------------------------------------------
// LM head for batches of at most kLmMaxB rows: the K-split partials, their sum and the block
// maxima of dense_gemv_kernel + logits_kernel in one streaming pass.  The tiled matrix's K-groups,
// in layout order (tile t, K-group kg at linear index t nkg + kg, (t nkg + kg) KiB), are cut into W
// contiguous equal runs, one per wave of a persistent grid (kLmWaves waves per workgroup, one
// workgroup per CU): wave g streams K-groups [g I / W, (g + 1) I / W) of I = ntiles nkg in one
// register pipeline of kLmSlots K-groups (each slot refilled right after its MFMA), against both
// terms of the batch rows held in LDS for the whole K range (rows 0 .. B-1 the hi terms, B .. 2B-1
// the lo terms, one MFMA per K-group with both in its 16 columns).  A tile the wave covers whole
// ends in its logits (written when requested) and the wave's running best per row (`beats`), which
// the workgroup reduces to one entry per row (slot blockIdx.x); a tile cut by the boundary g between
// two runs (at most one cut per tile: runs are at least nkg long) leaves its head part (wave g - 1)
// and tail part (wave g) in fix[g], which lm_fix_kernel adds; argmax_kernel reduces the entries.
// Dummy refills past a run's end read the batch rows (resident in L2), not weights.
// ---------------------------------------------------------------------------------------------
constexpr uint32_t kLmWaves = 16;
constexpr uint32_t kLmMaxB = 8;
constexpr uint32_t kLmSlots = 6;
constexpr uint32_t kLmMaxK = 4096;
constexpr uint32_t kLmStage = kLmMaxB * kLmMaxK / 8u / (kLmWaves * 64u);  // batch-row chunks (8 floats) per thread

struct LmArgs {
  const uint8_t *w;  // tiled [ntiles][nkg] KiB
  const float *x;    // [B][K]
  float *logits;     // [B][V] or null
  float *fix;        // [W][2][B][16]: head (side 0) and tail (side 1) parts of the tile cut at boundary g
  float *bval;       // [B][nblk]: stream workgroup i's best of row b at b nblk + i, lm_fix_kernel
                     // workgroup x's at b nblk + nblk_s + x
  int32_t *bidx;     // [B][nblk]
  uint64_t iters;    // ntiles * nkg
  uint32_t iq, ir;   // iters = iq W + ir
  uint32_t V, K, nkg, B, W, nblk, nblk_s;
};

// (bv, bi) <- the better of it and lane (lane ^ m)'s (`beats`; kNoIndex for none)
__device__ __forceinline__ void best_xor(float &bv, int32_t &bi, int m) {
  const float ov = __shfl_xor(bv, m, 64);
  const int32_t oi = __shfl_xor(bi, m, 64);
  if (oi != kNoIndex && (bi == kNoIndex || beats(ov, oi, bv, bi))) {
    bv = ov;
    bi = oi;
  }
}

__global__ __launch_bounds__(kLmWaves * 64) void lm_stream_kernel(LmArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t *bs = (uint16_t *)smem;  // [2B][ldk]
  constexpr uint32_t CJ = kLmSlots;
  const uint32_t nkg = a.nkg, Kp = nkg * 32u, ldk = Kp + 8u, B = a.B;
  const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
  const uint32_t gw = blockIdx.x * kLmWaves + wv;
  const uint64_t beg = (uint64_t)gw * a.iters / a.W, end = (uint64_t)(gw + 1u) * a.iters / a.W;
  // the batch rows' chunks first (the staging then waits for them alone: loads complete in order)
  const uint32_t k8 = Kp / 8u, nch = B * k8;
  // (no branch around a load: chunks outside the rows read row 0's first chunk and are zeroed at use)
  float4 xv[kLmStage][2];
#pragma unroll
  for (uint32_t u = 0; u < kLmStage; ++u) {
    const uint32_t id = threadIdx.x + u * kLmWaves * 64u, j = id / k8, k = (id - j * k8) * 8u;
    const bool ok = id < nch && k < a.K;  // K % 8 == 0: a chunk is wholly inside or outside
    const float *p = a.x + (ok ? (size_t)j * a.K + k : 0u);
    xv[u][0] = *(const float4 *)p;
    xv[u][1] = *(const float4 *)(p + 4);
  }
  const uint8_t *wl = a.w + lane * 16u;
  const uint8_t *dummy = (const uint8_t *)a.x + lane * 16u;  // B K 4 >= 1 KiB
  uint4 abuf[CJ];
#pragma unroll
  for (uint32_t j = 0; j < CJ; ++j) abuf[j] = load_stream16(beg + j < end ? wl + (beg + j) * 1024u : dummy);
#pragma unroll
  for (uint32_t u = 0; u < kLmStage; ++u) {
    const uint32_t id = threadIdx.x + u * kLmWaves * 64u, j = id / k8, k = (id - j * k8) * 8u;
    if (id >= nch) continue;
    float v8[8] = {xv[u][0].x, xv[u][0].y, xv[u][0].z, xv[u][0].w, xv[u][1].x, xv[u][1].y, xv[u][1].z, xv[u][1].w};
    if (k >= a.K) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v8[e] = 0.0f;
    }
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      uint32_t tp[2];
      split_bf16x2<2>(v8[2 * p], v8[2 * p + 1], tp);
      hi[p] = tp[0];
      lo[p] = tp[1];
    }
    *(uint4 *)(bs + (size_t)j * ldk + k) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *(uint4 *)(bs + (size_t)(B + j) * ldk + k) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  }
  __syncthreads();

  const uint32_t i16 = lane & 15u, q = lane >> 4;
  const bool bcol = i16 < 2u * B;
  const uint16_t *brow = bs + (size_t)min(i16, 2u * B - 1u) * ldk + 8u * q;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  float bv = -INFINITY;
  int32_t bi = kNoIndex;
  uint32_t tile = (uint32_t)(beg / nkg), kg = (uint32_t)(beg - (uint64_t)tile * nkg), kg_first = kg;
  for (uint64_t base = beg; base < end; base += CJ) {
#pragma unroll
    for (uint32_t j = 0; j < CJ; ++j) {
      const uint64_t cur = base + j;
      const bool live = cur < end;  // wave-uniform
      if (live) {
        const u32x4_t zero = {0u, 0u, 0u, 0u};
        const u32x4_t r = *(const u32x4_t *)(brow + 32u * kg);
        const u32x4_t raw = bcol ? r : zero;
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, abuf[j]), __builtin_bit_cast(bf16x8_t, raw),
                                                      acc, 0, 0, 0);
      }
      // every slot refills, past the run's end with the dummy: a static count of loads in flight
      const uint64_t nx = cur + CJ;
      abuf[j] = load_stream16(nx < end ? wl + nx * 1024u : dummy);
      if (live) {
        if (kg + 1u == nkg || cur + 1u == end) {
          // token j's lo column (j + B) onto its hi column j: lanes i16 < B hold rows 4q .. 4q + 3
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) acc[rr] = acc[rr] + __shfl(acc[rr], (int)(lane + B), 64);
          if (kg_first == 0u && kg + 1u == nkg) {  // whole tile
            if (i16 < B) {
#pragma unroll
              for (uint32_t rr = 0; rr < 4u; ++rr) {
                const uint32_t row = tile * 16u + 4u * q + rr;
                if (row < a.V) {
                  if (a.logits) a.logits[(size_t)i16 * a.V + row] = acc[rr];
                  if (bi == kNoIndex || beats(acc[rr], (int32_t)row, bv, bi)) {
                    bv = acc[rr];
                    bi = (int32_t)row;
                  }
                }
              }
            }
          } else if (i16 < B) {  // head (the run ends inside the tile) or tail (it began inside)
            const uint32_t side = kg_first == 0u ? 0u : 1u, bnd = side == 0u ? gw + 1u : gw;
            *(float4 *)(a.fix + (((size_t)bnd * 2u + side) * B + i16) * 16u + 4u * q) = make_float4(acc[0], acc[1], acc[2], acc[3]);
          }
          acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
        if (++kg == nkg) {
          kg = 0;
          kg_first = 0;
          ++tile;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // the run's best per row (lanes i16, i16 + 16, i16 + 32, i16 + 48 hold row i16's candidates),
  // then the workgroup's over its waves
  __shared__ float wbv[kLmWaves][kLmMaxB];
  __shared__ int32_t wbi[kLmWaves][kLmMaxB];
  best_xor(bv, bi, 16);
  best_xor(bv, bi, 32);
  if (q == 0u && i16 < B) {
    wbv[wv][i16] = bv;
    wbi[wv][i16] = bi;
  }
  __syncthreads();
  if (threadIdx.x < B) {
    float v = -INFINITY;
    int32_t ix = kNoIndex;
    for (uint32_t w = 0; w < kLmWaves; ++w) {
      const int32_t oi = wbi[w][threadIdx.x];
      if (oi != kNoIndex && (ix == kNoIndex || beats(wbv[w][threadIdx.x], oi, v, ix))) {
        v = wbv[w][threadIdx.x];
        ix = oi;
      }
    }
    a.bval[(size_t)threadIdx.x * a.nblk + blockIdx.x] = v;
    a.bidx[(size_t)threadIdx.x * a.nblk + blockIdx.x] = ix;
  }
}

// The tiles cut between two runs: head + tail per row, logits when requested, and each
// workgroup's best per row (slot nblk_s + blockIdx.x; boundary 0 and cuts on tile edges give no
// candidate).  Workgroup (x, j): boundaries g = 256 x + t of batch row j.  The cuts
// g I / W = g q + (g r) / W (I = q W + r) in 32-bit arithmetic.
__global__ __launch_bounds__(256) void lm_fix_kernel(LmArgs a) {
  const uint32_t j = blockIdx.y, t = threadIdx.x, g = blockIdx.x * 256u + t;
  float bv = -INFINITY;
  int32_t bi = kNoIndex;
  if (g > 0u && g < a.W) {
    const uint32_t cut = g * a.iq + (g * a.ir) / a.W;
    const uint32_t tile = cut / a.nkg;
    if (cut != tile * a.nkg) {
      const float *hp = a.fix + (((size_t)g * 2u + 0u) * a.B + j) * 16u;
      const float *tp = a.fix + (((size_t)g * 2u + 1u) * a.B + j) * 16u;
      float h[16], u[16];
#pragma unroll
      for (uint32_t i = 0; i < 16u; i += 4u) {
        *(float4 *)(h + i) = *(const float4 *)(hp + i);
        *(float4 *)(u + i) = *(const float4 *)(tp + i);
      }
#pragma unroll
      for (uint32_t i = 0; i < 16u; ++i) {
        const uint32_t row = tile * 16u + i;
        if (row < a.V) {
          const float v = h[i] + u[i];
          if (a.logits) a.logits[(size_t)j * a.V + row] = v;
          if (bi == kNoIndex || beats(v, (int32_t)row, bv, bi)) {
            bv = v;
            bi = (int32_t)row;
          }
        }
      }
    }
  }
  __shared__ float wbv[4];
  __shared__ int32_t wbi[4];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) best_xor(bv, bi, m);
  if ((t & 63u) == 0u) {
    wbv[t >> 6] = bv;
    wbi[t >> 6] = bi;
  }
  __syncthreads();
  if (t == 0u) {
    float v = -INFINITY;
    int32_t ix = kNoIndex;
    for (uint32_t w = 0; w < 4u; ++w)
      if (wbi[w] != kNoIndex && (ix == kNoIndex || beats(wbv[w], wbi[w], v, ix))) {
        v = wbv[w];
        ix = wbi[w];
      }
    a.bval[(size_t)j * a.nblk + a.nblk_s + blockIdx.x] = v;
    a.bidx[(size_t)j * a.nblk + a.nblk_s + blockIdx.x] = ix;
  }
}

// f32 rows [B][len][kvH][dk] of one layer -> cache slots 0 .. len-1 (k_index or v_index layout).
struct CacheLoadArgs {
  const float *src;
  void *dst;
  uint32_t B, len, kvH, dk, cap_p, is_k;
};
template <typename KV>
__global__ __launch_bounds__(256) void cache_load_kernel(CacheLoadArgs a) {
  const uint64_t n = (uint64_t)a.B * a.len * a.kvH * a.dk;
  KV *dst = (KV *)a.dst;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t d = (uint32_t)(i % a.dk);
    uint64_t r = i / a.dk;
    const uint32_t hh = (uint32_t)(r % a.kvH);
    r /= a.kvH;
    const uint32_t p = (uint32_t)(r % a.len), b = (uint32_t)(r / a.len);
    const size_t o = a.is_k ? k_index(b, hh, p, d, a.kvH, a.cap_p, a.dk) : v_index(b, hh, p, d, a.kvH, a.cap_p, a.dk);
    kv_store1(dst + o, a.src[i]);
  }
}

inline uint64_t cdiv(uint64_t x, uint64_t y) { return (x + y - 1) / y; }
inline uint64_t align_up(uint64_t x, uint64_t y) { return cdiv(x, y) * y; }

float bf16h(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// A dense [N, K] bf16 matrix in the GEMV's tiled layout (dense_gemv_kernel).
struct DenseMat {
  uint8_t *w = nullptr;
  uint32_t N = 0, K = 0, nkg = 0, ntiles = 0, H = 0, parts = 0;
};

// Tiles and K-groups of an [N, K] matrix.
void dense_geometry(DenseMat &m) {
  m.nkg = (uint32_t)cdiv(m.K, 32);
  m.ntiles = (uint32_t)cdiv(m.N, 16);
}

// K-groups per work unit: the largest H <= kDenseMaxH (halving, down to 4) that still gives at
// least 4 waves per CU.  Fewer, longer units won at the 20B shapes (q|k|v 90 K-groups, output
// projection 128): H = 4 / 8 / 16 measured 4.52 / 4.23 / 4.11 ms per 24-layer batch-8 decode step.
void dense_plan(DenseMat &m, int num_cus) {
  dense_geometry(m);
  uint32_t H = kDenseMaxH;
  while (H > 4 && (uint64_t)m.ntiles * cdiv(m.nkg, H) < 4ull * (uint64_t)num_cus) H >>= 1;
  m.H = std::min<uint32_t>(H, m.nkg);
  m.parts = (uint32_t)cdiv(m.nkg, m.H);
}

// Host [N, K] bf16 -> tiled layout (rows beyond N and inputs beyond K are zeros).
std::vector<uint16_t> dense_tile(const uint16_t *src, uint32_t N, uint32_t K, const DenseMat &m) {
  std::vector<uint16_t> out((size_t)m.ntiles * m.nkg * 512, 0);
  for (uint32_t t = 0; t < m.ntiles; ++t)
    for (uint32_t kg = 0; kg < m.nkg; ++kg)
      for (uint32_t l = 0; l < 64; ++l) {
        const uint32_t row = 16 * t + (l & 15), k0 = 32 * kg + 8 * (l >> 4);
        if (row >= N) continue;
        uint16_t *d = out.data() + ((size_t)t * m.nkg + kg) * 512 + l * 8;
        for (uint32_t e = 0; e < 8; ++e)
          if (k0 + e < K) d[e] = src[(size_t)row * K + k0 + e];
      }
  return out;
}

}  // namespace

struct burnext_gptoss {
  int device = 0;
  burnext_gptoss_config cfg{};
  uint32_t qd = 0, kd = 0, groups = 0;
  int num_cus = 256;
  std::vector<burnext_moe_layer_t> moe;
  uint16_t *emb = nullptr;
  DenseMat lm;
  std::vector<DenseMat> qkv, wo;
  float *bqkv = nullptr, *bo = nullptr, *norm_attn = nullptr, *norm_final = nullptr, *sinks = nullptr, *rope = nullptr;
  uint8_t *kc = nullptr, *vc = nullptr;  // per layer: k_index / v_index layouts of the cache element
  size_t kv_elem = 4;
  uint32_t cap_p = 0;        // cache_len rounded up to 64 rows
  uint64_t layer_cache = 0;  // elements per layer
  uint32_t used = 0;         // cache rows held
  uint32_t cache_batch = 0;  // batch rows whose cache holds all `used` rows (0 while used == 0)
  uint64_t pos_next = 0;     // positions seen
  std::vector<void *> allocs;
};

namespace {

struct GWs {
  uint64_t hid, hid2, xn, part, q, ctx, attn, bval, bidx, moe, total;
  uint64_t moe_bytes;
  uint32_t nblk;
};

// The streaming LM head (lm_stream_kernel) serves batches of at most kLmMaxB rows whose d_model
// fits its LDS staging (K <= kLmMaxK, K % 8 == 0, a batch of at least 1 KiB for the dummy refills)
// and vocabularies of at least one row tile per wave of one workgroup (and fewer than 2^32
// K-groups: lm_fix_kernel's 32-bit cuts).
bool lm_stream_ok(const burnext_gptoss &M, uint32_t B) {
  const uint32_t K = M.lm.K;
  return B >= 1u && B <= kLmMaxB && K <= kLmMaxK && K % 8u == 0u && (uint64_t)B * K * 4u >= 1024u &&
         M.lm.ntiles >= kLmWaves && (uint64_t)M.lm.ntiles * M.lm.nkg < (1ull << 32);
}
// Its waves: one workgroup per CU, at most one wave per row tile (so every run spans at least nkg
// K-groups and a tile is cut at most once).
uint32_t lm_waves(const burnext_gptoss &M) {
  return std::min<uint32_t>((uint32_t)M.num_cus, M.lm.ntiles / kLmWaves) * kLmWaves;
}
size_t lm_lds_bytes(uint32_t B, uint32_t nkg) { return 2ull * B * (nkg * 32u + 8u) * 2u; }

GWs gptoss_ws(const burnext_gptoss &M, uint32_t B, uint64_t moe_bytes) {
  GWs w{};
  uint64_t off = 0;
  auto take = [&](uint64_t bytes) {
    const uint64_t o = off;
    off = align_up(off + std::max<uint64_t>(bytes, 1), 256);
    return o;
  };
  const auto &c = M.cfg;
  const bool lm_stream = lm_stream_ok(M, B);
  const uint32_t lw = lm_waves(M);
  // the LM head's partials (K-split path) or its cut tiles' parts (streaming path)
  uint64_t part_elems = lm_stream ? (uint64_t)lw * 2u * B * 16u : (uint64_t)M.lm.parts * B * M.lm.N;
  for (const auto &m : M.qkv) part_elems = std::max<uint64_t>(part_elems, (uint64_t)m.parts * B * m.N);
  for (const auto &m : M.wo) part_elems = std::max<uint64_t>(part_elems, (uint64_t)m.parts * B * m.N);
  const uint64_t max_chunks = cdiv(c.cache_len, kAttnChunk);
  w.nblk = lm_stream ? lw / kLmWaves + (uint32_t)cdiv(lw, 256) : (uint32_t)cdiv(c.vocab_size, kLogitsPerBlock);
  w.hid = take((uint64_t)B * c.d_model * 4);
  w.hid2 = take((uint64_t)B * c.d_model * 4);
  w.xn = take((uint64_t)B * c.d_model * 4);
  w.part = take(part_elems * 4);
  w.q = take((uint64_t)B * M.qd * 4);
  w.ctx = take((uint64_t)B * M.qd * 4);
  w.attn = take((uint64_t)B * c.kv_heads * max_chunks * M.groups * (c.head_dim + 2ull) * 4);
  w.bval = take((uint64_t)B * w.nblk * 4);
  w.bidx = take((uint64_t)B * w.nblk * 4);
  w.moe = take(moe_bytes);
  w.moe_bytes = moe_bytes;
  w.total = off;
  return w;
}

burnext_status hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) return set_error(BURNEXT_DEVICE_ERROR, std::string(what) + ": " + hipGetErrorString(e));
  return BURNEXT_OK;
}

struct DevGuard {
  int prev = -1;
  bool ok = false;
  explicit DevGuard(int d) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    ok = hipSetDevice(d) == hipSuccess;
  }
  ~DevGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

void free_model(burnext_gptoss *M) {
  if (!M) return;
  DevGuard g(M->device);
  for (void *p : M->allocs)
    if (p) (void)hipFree(p);
  delete M;
}

burnext_status dev_alloc(burnext_gptoss *M, void **dst, size_t bytes) {
  if (hipMalloc(dst, std::max<size_t>(bytes, 1)) != hipSuccess) {
    *dst = nullptr;
    return set_error(BURNEXT_OUT_OF_MEMORY, "hipMalloc failed in burnext_gptoss_create");
  }
  M->allocs.push_back(*dst);
  return BURNEXT_OK;
}

template <typename T>
burnext_status upload(burnext_gptoss *M, T **dst, const T *src, size_t n) {
  const burnext_status st = dev_alloc(M, (void **)dst, n * sizeof(T));
  if (st != BURNEXT_OK) return st;
  if (n && hipMemcpy(*dst, src, n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
    return set_error(BURNEXT_DEVICE_ERROR, "hipMemcpy failed in burnext_gptoss_create");
  return BURNEXT_OK;
}

burnext_status dense_gemv(const DenseMat &m, const float *x, uint32_t B, float *out, hipStream_t s) {
  DenseArgs a{};
  a.w = m.w;
  a.x = x;
  a.out = out;
  a.N = m.N;
  a.K = m.K;
  a.nkg = m.nkg;
  a.ntiles = m.ntiles;
  a.B = B;
  a.H = m.H;
  a.part_stride = (uint64_t)B * m.N;
  const size_t lds = 2ull * 16 * (m.H * 32 + 8) * 2;
  return hip_check(launch_kernel(dense_gemv_kernel<kDenseWaves>, dim3((uint32_t)cdiv(m.ntiles, kDenseWaves), m.parts),
                                 dim3(kDenseWaves * 64), lds, s, a),
                   "dense GEMV launch");
}

// the shapes attn_chunk64_kernel serves (the only attention kernel that merges a single chunk itself)
bool attn_direct_ok(uint32_t dk, uint32_t groups) {
  return dk <= 64u && (groups == 1u || groups == 2u || groups == 4u || groups == 8u);
}

template <typename KV>
hipError_t launch_attention_kv(uint32_t groups, dim3 grid, hipStream_t s, const AttnArgs &a) {
  if (a.ctx != nullptr && !attn_direct_ok(a.dk, groups)) return hipErrorInvalidValue;
  if (a.dk <= 64u) {  // a chunk's q and K quads in one memory round trip, its V quads right after the scores
    switch (groups) {
      case 1: return launch_kernel(attn_chunk64_kernel<KV, 1>, grid, dim3(256), 0, s, a);
      case 2: return launch_kernel(attn_chunk64_kernel<KV, 2>, grid, dim3(256), 0, s, a);
      case 4: return launch_kernel(attn_chunk64_kernel<KV, 4>, grid, dim3(256), 0, s, a);
      case 8: return launch_kernel(attn_chunk64_kernel<KV, 8>, grid, dim3(256), 0, s, a);
      default: break;
    }
  }
  switch (groups) {
    case 1: return launch_kernel(attn_chunk_kernel<KV, 1>, grid, dim3(256), 0, s, a);
    case 2: return launch_kernel(attn_chunk_kernel<KV, 2>, grid, dim3(256), 0, s, a);
    case 4: return launch_kernel(attn_chunk_kernel<KV, 4>, grid, dim3(256), 0, s, a);
    case 8: return launch_kernel(attn_chunk_kernel<KV, 8>, grid, dim3(256), 0, s, a);
    case 16: return launch_kernel(attn_chunk_kernel<KV, 16>, grid, dim3(256), 0, s, a);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_attention(bool kv_bf16, uint32_t groups, dim3 grid, hipStream_t s, const AttnArgs &a) {
  return kv_bf16 ? launch_attention_kv<uint16_t>(groups, grid, s, a) : launch_attention_kv<float>(groups, grid, s, a);
}

// YaRN-scaled inverse frequencies and concentration (src/rope/mod.rs:11-52 over Burn's
// RotaryEncoding frequency scaling): inv[i] = theta^(-2 i / d); with factor > 1 the ramp
// r = clamp((2 i - low) / (high - low), 0, 1) blends inv / factor (r = 0) and inv (r = 1),
// low = d ln(ctx / (beta 2 pi)) / ln theta, high = d ln(ctx / (alpha 2 pi)) / ln theta; the
// cos/sin table is multiplied by 0.1 ln(factor) + 1.
bool yarn_frequencies(const burnext_gptoss_config &c, std::vector<double> &inv, double &conc) {
  const uint32_t dk = c.head_dim, half = dk / 2;
  inv.assign(half, 0.0);
  for (uint32_t i = 0; i < half; ++i) inv[i] = (double)(float)(1.0 / std::pow((double)c.rope_theta, (2.0 * i) / dk));
  conc = 1.0;
  if (!(c.rope_scaling_factor > 1.0f)) return true;
  const double dd = dk, lb = std::log((double)c.rope_theta), two_pi = 6.283185307179586476925;
  const double low = dd * std::log(c.rope_initial_context / (c.rope_ntk_beta * two_pi)) / lb;
  const double high = dd * std::log(c.rope_initial_context / (c.rope_ntk_alpha * two_pi)) / lb;
  if (!(low > 0.0 && high > 0.0 && low < high && high < dd - 1.0)) return false;
  for (uint32_t i = 0; i < half; ++i) {
    const double f = inv[i], ir = -std::log(f) * dd / lb;
    const double r = std::min(1.0, std::max(0.0, (ir - low) / (high - low)));
    inv[i] = (double)(float)(f / c.rope_scaling_factor * (1.0 - r) + f * r);
  }
  conc = (double)(float)(0.1 * std::log((double)c.rope_scaling_factor) + 1.0);
  return true;
}

// The layer's attention window, 0 = Full: WindowPolicy::window_for(l) combined with the caller's
// window by combine_windows (src/cache/mod.rs:15-44): Full yields the other, two windows the smaller.
uint32_t layer_window(const burnext_gptoss_config &c, uint32_t l, uint32_t caller) {
  uint32_t pw = 0;
  if (c.window_policy == 1) pw = c.window;
  if (c.window_policy == 2) pw = ((l % 2 == 0) == (c.full_on_even != 0)) ? 0 : c.window;
  if (pw == 0) return caller;
  return caller == 0 ? pw : std::min(pw, caller);
}

burnext_status moe_ws_bytes(const burnext_gptoss *M, uint32_t batch, uint64_t *bytes) {
  uint64_t moe = 0;
  for (auto *m : M->moe) {
    uint64_t b = 0;
    const burnext_status s = burnext_moe_workspace_size(m, batch, &b);
    if (s != BURNEXT_OK) return s;
    moe = std::max(moe, b);
  }
  *bytes = moe;
  return BURNEXT_OK;
}

}  // namespace

extern "C" {

burnext_status burnext_gptoss_create(const burnext_gptoss_config *cfg, const burnext_gptoss_weights *w,
                                     const burnext_moe_layer_t *moe_layers, int device, burnext_gptoss_t *out) {
  if (!out) return set_error(BURNEXT_INVALID_ARG, "out is null");
  *out = nullptr;
  if (!cfg || !w || !moe_layers) return set_error(BURNEXT_INVALID_ARG, "null config, weights or MoE layers");
  const auto &c = *cfg;
  if (!w->tok_emb || !w->norm_attn || !w->wq || !w->bq || !w->wk || !w->bk || !w->wv || !w->bv || !w->wo || !w->bo ||
      !w->norm_final || !w->lm_head)
    return set_error(BURNEXT_INVALID_ARG, "null weight pointer");
  if (!c.vocab_size || !c.d_model || !c.n_layers || !c.n_heads || !c.kv_heads || !c.head_dim || !c.max_batch ||
      !c.cache_len || !c.max_positions)
    return set_error(BURNEXT_INVALID_ARG, "zero dimension in burnext_gptoss_config");
  if (c.n_heads % c.kv_heads || c.n_heads / c.kv_heads > kMaxGroups || ((c.n_heads / c.kv_heads) & (c.n_heads / c.kv_heads - 1)))
    return set_error(BURNEXT_UNSUPPORTED, "n_heads / kv_heads must be a power of two <= 16");
  if (c.head_dim % 8 || c.head_dim > kMaxHeadDim)
    return set_error(BURNEXT_UNSUPPORTED, "head_dim must be a multiple of 8 and at most 128");
  if (c.max_batch > kMaxBatch) return set_error(BURNEXT_UNSUPPORTED, "max_batch above 16 is not supported");
  if (c.d_model % 4) return set_error(BURNEXT_UNSUPPORTED, "d_model must be a multiple of 4");
  if (c.rope_head_stride > 1 || c.kv_bf16 > 1 || c.full_on_even > 1 || c.experts_bf16 > 1)
    return set_error(BURNEXT_INVALID_ARG, "rope_head_stride, kv_bf16, full_on_even and experts_bf16 must be 0 or 1");
  if (c.window_policy > 2) return set_error(BURNEXT_INVALID_ARG, "window_policy must be 0 (Full), 1 (Fixed) or 2 (EveryOther)");
  if (c.window_policy != 0 && c.window == 0) return set_error(BURNEXT_INVALID_ARG, "window must be positive");
  if (c.sink_tokens >= c.cache_len) return set_error(BURNEXT_INVALID_ARG, "sink_tokens must be below cache_len");
  if (c.cache_len > (1u << 30) || c.max_positions > (1u << 30))
    return set_error(BURNEXT_UNSUPPORTED, "cache_len and max_positions above 2^30 are not supported");
  if ((c.n_heads % c.kv_heads) == 0 && (cdiv(c.cache_len, kAttnChunk) + 1) * (c.n_heads / c.kv_heads) > 16384)
    return set_error(BURNEXT_UNSUPPORTED, "cache_len * n_heads / kv_heads above 4M rows (attention combine LDS)");
  if (!(c.scale_dk > 0.0f) || !(c.rms_eps >= 0.0f) || !(c.rope_theta > 1.0f))
    return set_error(BURNEXT_INVALID_ARG, "scale_dk > 0, rope_theta > 1 and rms_eps >= 0 are required");
  std::vector<double> inv;
  double conc = 1.0;
  if (!yarn_frequencies(c, inv, conc))
    return set_error(BURNEXT_INVALID_ARG, "YaRN thresholds out of range (the reference asserts 0 < low < high < d - 1)");
  for (uint32_t l = 0; l < c.n_layers; ++l)
    if (!moe_layers[l]) return set_error(BURNEXT_INVALID_ARG, "null MoE layer handle");

  // host preparation (no device call): tiled projections, f32 biases / norms / sinks, RoPE table
  const uint32_t dk = c.head_dim, half = dk / 2, qd = c.n_heads * dk, kd = c.kv_heads * dk;
  const uint32_t D = c.d_model, L = c.n_layers, V = c.vocab_size, N3 = qd + 2 * kd;
  DenseMat lm;
  std::vector<DenseMat> qkv(L), wo(L);
  std::vector<std::vector<uint16_t>> qkv_t(L), wo_t(L);
  std::vector<uint16_t> lm_t;
  std::vector<float> bq((size_t)L * N3), bo((size_t)L * D), na((size_t)L * D), nf(D), sk, tab;
  try {
    lm.N = V;
    lm.K = D;
    dense_geometry(lm);
    lm_t = dense_tile(w->lm_head, V, D, lm);
    std::vector<uint16_t> fused((size_t)N3 * D);
    for (uint32_t l = 0; l < L; ++l) {
      memcpy(fused.data(), w->wq + (size_t)l * qd * D, (size_t)qd * D * 2);
      memcpy(fused.data() + (size_t)qd * D, w->wk + (size_t)l * kd * D, (size_t)kd * D * 2);
      memcpy(fused.data() + (size_t)(qd + kd) * D, w->wv + (size_t)l * kd * D, (size_t)kd * D * 2);
      qkv[l].N = N3;
      qkv[l].K = D;
      dense_geometry(qkv[l]);
      qkv_t[l] = dense_tile(fused.data(), N3, D, qkv[l]);
      wo[l].N = D;
      wo[l].K = qd;
      dense_geometry(wo[l]);
      wo_t[l] = dense_tile(w->wo + (size_t)l * D * qd, D, qd, wo[l]);
    }
    for (uint32_t l = 0; l < L; ++l) {
      for (uint32_t i = 0; i < qd; ++i) bq[(size_t)l * N3 + i] = bf16h(w->bq[(size_t)l * qd + i]);
      for (uint32_t i = 0; i < kd; ++i) {
        bq[(size_t)l * N3 + qd + i] = bf16h(w->bk[(size_t)l * kd + i]);
        bq[(size_t)l * N3 + qd + kd + i] = bf16h(w->bv[(size_t)l * kd + i]);
      }
      for (uint32_t i = 0; i < D; ++i) {
        bo[(size_t)l * D + i] = bf16h(w->bo[(size_t)l * D + i]);
        na[(size_t)l * D + i] = bf16h(w->norm_attn[(size_t)l * D + i]);
      }
    }
    for (uint32_t i = 0; i < D; ++i) nf[i] = bf16h(w->norm_final[i]);
    if (w->sinks) {
      sk.resize((size_t)L * c.n_heads);
      for (size_t i = 0; i < sk.size(); ++i) sk[i] = bf16h(w->sinks[i]);
    }
    // RoPE table [max_positions + nH][dk/2][2] = (cos, sin) x concentration
    const uint64_t npos = (uint64_t)c.max_positions + c.n_heads;
    tab.resize(npos * half * 2);
    for (uint64_t p = 0; p < npos; ++p)
      for (uint32_t i = 0; i < half; ++i) {
        const float ang = (float)p * (float)inv[i];  // one f32 product, as the reference's f32 table
        tab[(p * half + i) * 2] = (float)(std::cos((double)ang) * conc);
        tab[(p * half + i) * 2 + 1] = (float)(std::sin((double)ang) * conc);
      }
  } catch (const std::bad_alloc &) {
    return set_error(BURNEXT_OUT_OF_MEMORY, "host allocation failed while preparing the decoder weights");
  }

  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
    return set_error(BURNEXT_INVALID_ARG, "device index out of range (or no HIP device)");
  for (uint32_t l = 0; l < c.n_layers; ++l) {
    uint32_t dm = 0;
    int dev = -1;
    moe_layer_shape(moe_layers[l], &dm, &dev);
    if (dm != c.d_model || dev != device)
      return set_error(BURNEXT_INVALID_ARG, "MoE layer d_model or device differs from the decoder's");
  }
  DevGuard guard(device);
  if (!guard.ok) return set_error(BURNEXT_DEVICE_ERROR, "hipSetDevice failed");
  burnext_gptoss *M = new (std::nothrow) burnext_gptoss();
  if (!M) return set_error(BURNEXT_OUT_OF_MEMORY, "host allocation failed");
  M->device = device;
  M->cfg = c;
  M->qd = qd;
  M->kd = kd;
  M->groups = c.n_heads / c.kv_heads;
  M->kv_elem = c.kv_bf16 ? 2 : 4;
  M->cap_p = (uint32_t)align_up(c.cache_len, 64);
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0) M->num_cus = cus;
  if (hipFuncSetAttribute((const void *)lm_stream_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lm_lds_bytes(kLmMaxB, kLmMaxK / 32u)) != hipSuccess) {
    delete M;
    return set_error(BURNEXT_DEVICE_ERROR, "hipFuncSetAttribute (LM head LDS) failed");
  }
  M->moe.assign(moe_layers, moe_layers + c.n_layers);
  burnext_status st = upload(M, &M->emb, w->tok_emb, (size_t)V * D);
  auto up_dense = [&](DenseMat &m, const DenseMat &geom, const std::vector<uint16_t> &t) -> burnext_status {
    m = geom;
    dense_plan(m, M->num_cus);
    uint16_t *p = nullptr;
    const burnext_status s2 = upload(M, &p, t.data(), t.size());
    m.w = (uint8_t *)p;
    return s2;
  };
  if (st == BURNEXT_OK) st = up_dense(M->lm, lm, lm_t);
  M->qkv.resize(L);
  M->wo.resize(L);
  for (uint32_t l = 0; l < L && st == BURNEXT_OK; ++l) {
    st = up_dense(M->qkv[l], qkv[l], qkv_t[l]);
    if (st == BURNEXT_OK) st = up_dense(M->wo[l], wo[l], wo_t[l]);
  }
  if (st == BURNEXT_OK) st = upload(M, &M->bqkv, bq.data(), bq.size());
  if (st == BURNEXT_OK) st = upload(M, &M->bo, bo.data(), bo.size());
  if (st == BURNEXT_OK) st = upload(M, &M->norm_attn, na.data(), na.size());
  if (st == BURNEXT_OK) st = upload(M, &M->norm_final, nf.data(), nf.size());
  if (st == BURNEXT_OK && w->sinks) st = upload(M, &M->sinks, sk.data(), sk.size());
  if (st == BURNEXT_OK) st = upload(M, &M->rope, tab.data(), tab.size());
  if (st == BURNEXT_OK) {  // KV cache
    M->layer_cache = (uint64_t)c.max_batch * c.kv_heads * M->cap_p * dk;
    const size_t bytes = (size_t)L * M->layer_cache * M->kv_elem;
    st = dev_alloc(M, (void **)&M->kc, bytes);
    if (st == BURNEXT_OK) st = dev_alloc(M, (void **)&M->vc, bytes);
    if (st == BURNEXT_OK && (hipMemset(M->kc, 0, bytes) != hipSuccess || hipMemset(M->vc, 0, bytes) != hipSuccess))
      st = set_error(BURNEXT_DEVICE_ERROR, "hipMemset of the KV cache failed");
  }
  if (st != BURNEXT_OK) {
    free_model(M);
    return st;
  }
  *out = M;
  return set_error(BURNEXT_OK, "");
}

void burnext_gptoss_destroy(burnext_gptoss_t M) { free_model(M); }

burnext_status burnext_gptoss_workspace_size(burnext_gptoss_t M, uint32_t batch, uint64_t *bytes) {
  if (!M || !bytes) return set_error(BURNEXT_INVALID_ARG, "null model or output pointer");
  if (batch == 0 || batch > M->cfg.max_batch) return set_error(BURNEXT_INVALID_ARG, "batch must be in [1, max_batch]");
  uint64_t moe = 0;
  const burnext_status s = moe_ws_bytes(M, batch, &moe);
  if (s != BURNEXT_OK) return s;
  *bytes = gptoss_ws(*M, batch, moe).total;
  return set_error(BURNEXT_OK, "");
}

burnext_status burnext_gptoss_reset(burnext_gptoss_t M) {
  if (!M) return set_error(BURNEXT_INVALID_ARG, "null model");
  M->used = 0;
  M->cache_batch = 0;
  M->pos_next = 0;
  return set_error(BURNEXT_OK, "");
}

burnext_status burnext_gptoss_cache_load(burnext_gptoss_t M, const float *k, const float *v, uint32_t batch,
                                         uint32_t len, void *stream) {
  if (!M) return set_error(BURNEXT_INVALID_ARG, "null model");
  if (batch == 0 || batch > M->cfg.max_batch) return set_error(BURNEXT_INVALID_ARG, "batch must be in [1, max_batch]");
  if (len > M->cfg.cache_len) return set_error(BURNEXT_INVALID_ARG, "len exceeds cache_len");
  if (len > 0 && (!k || !v)) return set_error(BURNEXT_INVALID_ARG, "null cache rows");
  DevGuard guard(M->device);
  if (!guard.ok) return set_error(BURNEXT_DEVICE_ERROR, "hipSetDevice failed");
  hipStream_t s = (hipStream_t)stream;
  const uint64_t per_layer = (uint64_t)batch * len * M->cfg.kv_heads * M->cfg.head_dim;
  for (uint32_t l = 0; l < M->cfg.n_layers && len > 0; ++l)
    for (int which = 0; which < 2; ++which) {
      CacheLoadArgs a{};
      a.src = (which ? v : k) + l * per_layer;
      a.dst = (which ? M->vc : M->kc) + l * M->layer_cache * M->kv_elem;
      a.B = batch;
      a.len = len;
      a.kvH = M->cfg.kv_heads;
      a.dk = M->cfg.head_dim;
      a.cap_p = M->cap_p;
      a.is_k = which == 0 ? 1u : 0u;
      const dim3 grid((uint32_t)std::min<uint64_t>(cdiv(per_layer, 256), 8192));
      const hipError_t e = M->cfg.kv_bf16 ? launch_kernel(cache_load_kernel<uint16_t>, grid, dim3(256), 0, s, a)
                                          : launch_kernel(cache_load_kernel<float>, grid, dim3(256), 0, s, a);
      const burnext_status st = hip_check(e, "cache load launch");
      if (st != BURNEXT_OK) return st;
    }
  M->used = len;
  M->cache_batch = len ? batch : 0u;
  M->pos_next = len;
  return set_error(BURNEXT_OK, "");
}

burnext_status burnext_gptoss_decode(burnext_gptoss_t M, const int32_t *tokens, uint32_t B, uint32_t pos,
                                     uint32_t window, int32_t *next_tokens, float *logits, float *hidden,
                                     void *workspace, uint64_t ws_bytes, void *stream) {
  if (!M || !tokens || !next_tokens) return set_error(BURNEXT_INVALID_ARG, "null model, tokens or next_tokens");
  const auto &c = M->cfg;
  if (B == 0 || B > c.max_batch) return set_error(BURNEXT_INVALID_ARG, "batch must be in [1, max_batch]");
  if (M->used > 0 && B > M->cache_batch) {
    // rows >= cache_batch hold no entries for the cached positions (the reference's cache is
    // sized for one batch): decoding them would attend over rows that were never written
    char buf[160];
    snprintf(buf, sizeof(buf), "batch %u exceeds the %u batch rows the cache holds (reset first)", B,
             M->cache_batch);
    return set_error(BURNEXT_INVALID_ARG, buf);
  }
  if (pos != M->pos_next) {
    char buf[160];
    snprintf(buf, sizeof(buf), "pos %u is not the next position (%llu positions seen)", pos,
             (unsigned long long)M->pos_next);
    return set_error(BURNEXT_INVALID_ARG, buf);
  }
  if (pos >= c.max_positions) return set_error(BURNEXT_UNSUPPORTED, "pos >= max_positions (beyond the RoPE table)");
  if (!workspace || ((uintptr_t)workspace & 255u))
    return set_error(BURNEXT_INVALID_ARG, "workspace null or not 256-byte aligned");
  uint64_t moe_bytes = 0;
  burnext_status st = moe_ws_bytes(M, B, &moe_bytes);
  if (st != BURNEXT_OK) return st;
  const GWs w = gptoss_ws(*M, B, moe_bytes);
  if (ws_bytes < w.total)
    return set_error(BURNEXT_WORKSPACE_TOO_SMALL, "workspace smaller than burnext_gptoss_workspace_size");
  DevGuard guard(M->device);
  if (!guard.ok) return set_error(BURNEXT_DEVICE_ERROR, "hipSetDevice failed");
  hipStream_t s = (hipStream_t)stream;
  uint8_t *base = (uint8_t *)workspace;
  float *hid = (float *)(base + w.hid), *hid2 = (float *)(base + w.hid2), *xn = (float *)(base + w.xn);
  float *part = (float *)(base + w.part), *qb = (float *)(base + w.q), *ctx = (float *)(base + w.ctx);
  float *attn = (float *)(base + w.attn), *bval = (float *)(base + w.bval);
  int32_t *bidx = (int32_t *)(base + w.bidx);
  void *moe_ws = base + w.moe;
  const uint32_t D = c.d_model, dk = c.head_dim, cap = c.cache_len, N3 = M->qd + 2 * M->kd;
  // cache rows after this step's append (the reference's local_end_index) and the new row's slot:
  // the first sink positions keep slots 0 .. sink - 1, later positions cycle over the others
  const uint32_t S = c.sink_tokens, ring = cap - S;
  const uint32_t used = (uint32_t)std::min<uint64_t>((uint64_t)M->used + 1, cap);
  const uint32_t slot = pos < S ? pos : S + (pos - S) % ring;
  if (used < S)  // Window(w) spans the last sink + min(w, rows - sink) rows: it needs the sink rows
    for (uint32_t l = 0; l < c.n_layers; ++l)
      if (layer_window(c, l, window) != 0)
        return set_error(BURNEXT_INVALID_ARG, "a windowed layer needs at least sink_tokens cache rows");
  {
    EmbedArgs a{tokens, M->emb, hid, D, c.vocab_size};
    st = hip_check(launch_kernel(embed_kernel, dim3((uint32_t)cdiv(D, 256), B), dim3(256), 0, s, a), "embedding launch");
    if (st != BURNEXT_OK) return st;
  }
  bool normed = false;  // xn already holds the norm the next step needs (fused into the MoE combine)
  for (uint32_t l = 0; l < c.n_layers; ++l) {
    if (!normed) {
      NormArgs na{hid, M->norm_attn + (size_t)l * D, xn, D, c.rms_eps};
      st = hip_check(launch_kernel(rmsnorm_kernel, dim3(B), dim3(256), 0, s, na), "RmsNorm launch");
      if (st != BURNEXT_OK) return st;
    }
    st = dense_gemv(M->qkv[l], xn, B, part, s);
    if (st != BURNEXT_OK) return st;
    QkvPostArgs qa{};
    qa.part = part;
    qa.part_stride = (uint64_t)B * N3;
    qa.parts = M->qkv[l].parts;
    qa.bias = M->bqkv + (size_t)l * N3;
    qa.rope = M->rope;
    qa.qbuf = qb;
    qa.kc = M->kc + l * M->layer_cache * M->kv_elem;
    qa.vc = M->vc + l * M->layer_cache * M->kv_elem;
    qa.B = B;
    qa.nH = c.n_heads;
    qa.kvH = c.kv_heads;
    qa.dk = dk;
    qa.cap_p = M->cap_p;
    qa.slot = slot;
    qa.pos = pos;
    qa.head_stride = c.rope_head_stride;
    const dim3 qgrid((uint32_t)cdiv(N3 / 2, 256), B);
    st = hip_check(c.kv_bf16 ? launch_qkv_post<uint16_t>(qa, qgrid, s) : launch_qkv_post<float>(qa, qgrid, s),
                   "q/k/v post launch");
    if (st != BURNEXT_OK) return st;
    const uint32_t lw = layer_window(c, l, window);  // 0 = Full
    // Full: every row; Window(lw): the last sink + min(lw, rows - sink) rows (used >= S checked)
    const uint32_t active = lw ? S + std::min(lw, used - S) : used;
    AttnArgs aa{};
    aa.q = qb;
    aa.kc = qa.kc;
    aa.vc = qa.vc;
    aa.part = attn;
    aa.nH = c.n_heads;
    aa.kvH = c.kv_heads;
    aa.dk = dk;
    aa.cap_p = M->cap_p;
    // window rows [used - active, used) of the reference's cache order: the sink rows among them
    // (rows < sink hold positions 0 .. sink - 1), then rows >= sink, which hold the latest positions
    const uint32_t wstart = used - active, nsink_rows = std::min(S, used);
    aa.nsk = wstart < nsink_rows ? nsink_rows - wstart : 0u;
    aa.sk_lo = wstart;
    const uint32_t nrec = used - std::max(wstart, S < used ? S : used);
    const uint32_t p_lo = pos + 1 - nrec;  // first recent position (>= S when nrec > 0)
    aa.p_mod = nrec ? (p_lo - S) % ring : 0u;
    aa.nkeys = aa.nsk + nrec;
    aa.sink = S;
    aa.ring = ring;
    aa.nchunk = (uint32_t)cdiv(aa.nkeys, kAttnChunk);
    aa.inv_scale = 1.0f / std::sqrt(c.scale_dk);
    const float *sinks_l = M->sinks ? M->sinks + (size_t)l * c.n_heads : nullptr;
    // a single chunk (windowed layers) merges the sink in the attention launch itself
    const bool direct = aa.nchunk == 1 && attn_direct_ok(dk, M->groups);
    if (direct) {
      aa.ctx = ctx;
      aa.sinks = sinks_l;
    }
    const dim3 agrid(aa.nchunk, c.kv_heads, B);
    st = hip_check(launch_attention(c.kv_bf16 != 0, M->groups, agrid, s, aa), "attention launch");
    if (st != BURNEXT_OK) return st;
    CombineAttnArgs ca{attn, sinks_l, ctx, c.n_heads, c.kv_heads, dk, aa.nchunk};
    if (!direct)
      st = hip_check(launch_kernel(attn_combine_kernel, dim3(c.kv_heads, B), dim3(256),
                                   (size_t)(aa.nchunk + 1) * M->groups * 4, s, ca),
                     "attention combine launch");
    if (st == BURNEXT_OK) st = dense_gemv(M->wo[l], ctx, B, part, s);
    if (st != BURNEXT_OK) return st;
    // the MoE layer; its combine also writes the next norm of the new hidden rows (the next
    // layer's attention norm, after the last layer the final norm) when its path allows
    const float *next_gamma = l + 1 < c.n_layers ? M->norm_attn + (size_t)(l + 1) * D : M->norm_final;
    const float *bo = M->bo + (size_t)l * D;
    if (moe_front_fusable(M->moe[l], B, M->wo[l].parts)) {
      // its router also forms the residual hid2 = hid + (sum of the output projection's parts + bo)
      st = moe_forward_post_norm(M->moe[l], hid2, BURNEXT_F32, hid, B, BURNEXT_FORWARD_DEFAULT, moe_ws, w.moe_bytes,
                                 stream, next_gamma, c.rms_eps, xn, &normed, part, (uint64_t)B * D, M->wo[l].parts,
                                 bo, hid, c.experts_bf16 != 0);
      if (st != BURNEXT_OK) return st;
    } else {
      OPostArgs oa{part, (uint64_t)B * D, M->wo[l].parts, D, bo, hid};
      st = hip_check(launch_kernel(o_post_kernel, dim3((uint32_t)cdiv(D, 256), B), dim3(256), 0, s, oa),
                     "o post launch");
      if (st != BURNEXT_OK) return st;
      st = moe_forward_post_norm(M->moe[l], hid, BURNEXT_F32, hid2, B, BURNEXT_FORWARD_DEFAULT, moe_ws, w.moe_bytes,
                                 stream, next_gamma, c.rms_eps, xn, &normed, nullptr, 0, 0, nullptr, nullptr,
                                 c.experts_bf16 != 0);
      if (st != BURNEXT_OK) return st;
      std::swap(hid, hid2);
    }
  }
  if (hidden) {
    st = hip_check(hipMemcpyAsync(hidden, hid, (size_t)B * D * 4, hipMemcpyDeviceToDevice, s), "hidden copy");
    if (st != BURNEXT_OK) return st;
  }
  if (!normed) {
    NormArgs nf{hid, M->norm_final, xn, D, c.rms_eps};
    st = hip_check(launch_kernel(rmsnorm_kernel, dim3(B), dim3(256), 0, s, nf), "final RmsNorm launch");
    if (st != BURNEXT_OK) return st;
  }
  if (lm_stream_ok(*M, B)) {
    LmArgs la{};
    la.w = M->lm.w;
    la.x = xn;
    la.logits = logits;
    la.fix = part;
    la.bval = bval;
    la.bidx = bidx;
    la.iters = (uint64_t)M->lm.ntiles * M->lm.nkg;
    la.V = c.vocab_size;
    la.K = M->lm.K;
    la.nkg = M->lm.nkg;
    la.B = B;
    la.W = lm_waves(*M);
    la.iq = (uint32_t)(la.iters / la.W);
    la.ir = (uint32_t)(la.iters % la.W);
    la.nblk = w.nblk;
    la.nblk_s = la.W / kLmWaves;
    st = hip_check(launch_kernel(lm_stream_kernel, dim3(la.W / kLmWaves), dim3(kLmWaves * 64), lm_lds_bytes(B, la.nkg), s, la),
                   "LM head launch");
    if (st != BURNEXT_OK) return st;
    st = hip_check(launch_kernel(lm_fix_kernel, dim3((uint32_t)cdiv(la.W, 256), B), dim3(256), 0, s, la), "LM head fix-up launch");
    if (st != BURNEXT_OK) return st;
  } else {
    st = dense_gemv(M->lm, xn, B, part, s);
    if (st != BURNEXT_OK) return st;
    LogitsArgs la{part, (uint64_t)B * c.vocab_size, M->lm.parts, c.vocab_size, w.nblk, logits, bval, bidx};
    st = hip_check(launch_kernel(logits_kernel, dim3(w.nblk, B), dim3(256), 0, s, la), "logits launch");
    if (st != BURNEXT_OK) return st;
  }
  ArgmaxArgs ga{bval, bidx, w.nblk, next_tokens};
  st = hip_check(launch_kernel(argmax_kernel, dim3(B), dim3(256), 0, s, ga), "argmax launch");
  if (st != BURNEXT_OK) return st;
  M->used = used;
  M->cache_batch = B;  // only rows < B received this position's entry
  M->pos_next = (uint64_t)pos + 1;
  return set_error(BURNEXT_OK, "");
}

}  // extern "C"
