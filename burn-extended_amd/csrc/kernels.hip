// kernels.hip -- MI355X (gfx950) kernels of the GPT-OSS MoE feed-forward over MXFP4 experts.
//
// router_kernel     RmsNorm + router logits, parallel over token blocks x expert groups
//                   replaces src/moe/mod.rs:109-110 (Burn RmsNorm / Linear)
// router_rows       the same for prefill batches: one wave per few tokens, rows in registers,
//                   also writes the two-term (MXFP8 hi + MXFP4 lo) rows of the grouped GEMM
// topk_kernel       top-k + softmax over the selected logits, one wave per token
//                   replaces src/moe/mod.rs:271-276 (topk_with_indices, max/exp/sum/div)
// dispatch_kernel   histogram / exclusive scan / stable scatter into expert segments
//                   replaces the per-expert dense masks of src/moe/mod.rs:279-288
// router_small      decode-sized router (n <= 16): one wave per (expert, token pair), also
//                   writes the normalised token rows for the expert GEMV
// small_route       top-k/softmax/dispatch of a decode-sized batch by one workgroup
// expert_gemv       MXFP4 x bf16 projection on MFMA 16x16x32 bf16, e2m1+e8m0 dequantised in
//                   registers; gate_up staging applies the RmsNorm and the epilogue fuses bias +
//                   clamped SwiGLU
//                   replaces w1_swiglu_dense_kernel / w2_scatter_dense_kernel (src/quant/gpu.rs:89-192)
// combine_kernel    y = x + sum_p w_p * (down_p + b2), deterministic slot order
//                   replaces the accumulate + residual of src/moe/mod.rs:405-411
//                   (combine_norm_kernel: the same, then a decoder's next RmsNorm of y)
// dequant_kernel    test hook: exact dequantisation (src/loader/mxfp4.rs:56-79)
#include "kernels.hpp"
#include "mx_device.hpp"

namespace burnext {

__device__ __forceinline__ float load_val(const float *p, size_t i) { return p[i]; }
__device__ __forceinline__ float load_val(const uint16_t *p, size_t i) { return bf16_bits_to_f32(p[i]); }
__device__ __forceinline__ void store_val(float *p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void store_val(uint16_t *p, size_t i, float v) { p[i] = f32_to_bf16_bits(v); }

__device__ __forceinline__ void store8(uint16_t *p, const float (&v)[8]) {
  uint32_t w4[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w4[j] = (uint32_t)f32_to_bf16_bits(v[2 * j]) | ((uint32_t)f32_to_bf16_bits(v[2 * j + 1]) << 16);
  *(uint4 *)p = make_uint4(w4[0], w4[1], w4[2], w4[3]);
}
__device__ __forceinline__ void store8(float *p, const float (&v)[8]) {
  *(float4 *)p = make_float4(v[0], v[1], v[2], v[3]);
  *(float4 *)(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

// ---------------------------------------------------------------------------------------------
// 8-element chunks: raw register form between load and use, and guarded scalar loads.
// ---------------------------------------------------------------------------------------------
template <typename T> struct Chunk8;
template <> struct Chunk8<float> {
  float4 a, b;
};
template <> struct Chunk8<uint16_t> {
  uint4 a;
};
__device__ __forceinline__ void chunk_load(Chunk8<float> &c, const float *p) {
  c.a = *(const float4 *)p;
  c.b = *(const float4 *)(p + 4);
}
__device__ __forceinline__ void chunk_load(Chunk8<uint16_t> &c, const uint16_t *p) { c.a = *(const uint4 *)p; }
__device__ __forceinline__ void chunk_vals(const Chunk8<float> &c, float (&v)[8]) {
  v[0] = c.a.x; v[1] = c.a.y; v[2] = c.a.z; v[3] = c.a.w; v[4] = c.b.x; v[5] = c.b.y; v[6] = c.b.z; v[7] = c.b.w;
}
__device__ __forceinline__ void chunk_vals(const Chunk8<uint16_t> &c, float (&v)[8]) {
  const uint32_t w4[4] = {c.a.x, c.a.y, c.a.z, c.a.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = __uint_as_float(w4[j] << 16);
    v[2 * j + 1] = __uint_as_float(w4[j] & 0xFFFF0000u);
  }
}
template <typename T>
__device__ __forceinline__ void load8_guarded(const T *p, uint32_t nvalid, float (&v)[8]) {
#pragma unroll
  for (uint32_t j = 0; j < 8u; ++j) v[j] = j < nvalid ? load_val(p, j) : 0.0f;
}

// Register chunks held per router row: 6 (3072 columns) for bf16 rows, 3 for f32 rows.
template <typename WT> struct RouteChunks { static constexpr int value = sizeof(WT) == 2 ? 6 : 3; };

// Lane-transposed LDS position of element c of a row: element 512 i + 8 l + j lives at
// 512 i + 64 j + l, so lane l reading its chunk element j hits consecutive addresses across the
// wave (conflict-free) in the fixed reduction order.
__device__ __forceinline__ uint32_t tpos(uint32_t c) { return (c & ~511u) | ((c & 7u) << 6) | ((c & 511u) >> 3); }
__device__ __forceinline__ uint32_t tpos_inv(uint32_t q) { return (q & ~511u) | ((q & 63u) << 3) | ((q >> 6) & 7u); }

// ---------------------------------------------------------------------------------------------
// Router kernel.  Grid (token blocks of tb <= 8, expert groups of 4 * epw); 4 waves.
// Fixed reduction order of every dot product, mirrored by the oracle: lane l owns the
// 8-element chunks c = 512 i + 8 l + j; its partial is fmaf over i ascending then j ascending;
// then the xor butterfly over the 64 lanes.  With apply_norm the normalisation comes after the
// dot product: logit = dot(x, gamma * w) / sqrt(dot(x, x) / D + eps) + b.
//  1. each wave issues the loads of its router rows (registers) before anything else
//  2. the workgroup stages its tokens into LDS (lane-transposed layout)
//  3. dot products for all tokens of the block, butterflies interleaved across tokens
//  4. sums of squares -> r per token (expert group 0 writes r for the expert GEMV staging)
// ---------------------------------------------------------------------------------------------
size_t router_lds_bytes(uint32_t tb, uint32_t Dpad) { return sizeof(float) * ((size_t)tb * Dpad + 8); }

// N butterfly sums at once (wave_sum_butterfly's bits in every lane; every lane active)
template <int N>
__device__ __forceinline__ void wave_sum_butterfly_n(float (&v)[N]) {
  wave_sum_to_lane0_n<N>(v);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = lane0_broadcast(v[i]);
}


template <typename XT, typename WT, bool VEC>
__global__ __launch_bounds__(kRouterThreads) void router_kernel(RouterArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const uint32_t D = a.D, Dpad = a.Dpad, E = a.E;
  float *xs = (float *)smem;
  float *rr = xs + (size_t)a.tb * Dpad;
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t t0 = blockIdx.x * a.tb;
  const uint32_t nh = min(a.tb, a.n - t0);
  const XT *x = (const XT *)a.x;
  const WT *rw = (const WT *)a.rw;
  constexpr int RC = RouteChunks<WT>::value;

  // 1. router rows of this wave: experts eb + w and (epw == 2) eb + 4 + w
  const uint32_t eb = blockIdx.y * 4u * a.epw;
  const uint32_t e0 = eb + w, e1 = eb + 4u + w;
  const bool has0 = e0 < E, has1 = a.epw == 2u && e1 < E;
  Chunk8<WT> r0[RC], r1[RC];
  if (VEC) {
#pragma unroll
    for (int i = 0; i < RC; ++i) {
      const uint32_t c0 = 512u * i + 8u * lane;
      if (has0 && c0 < D) chunk_load(r0[i], rw + (size_t)e0 * D + c0);
      if (has1 && c0 < D) chunk_load(r1[i], rw + (size_t)e1 * D + c0);
    }
  }

  // 2. stage tokens (contiguous [nh, D]); one batch of SU chunk loads per thread in flight
  if (VEC) {
    constexpr int SU = sizeof(XT) == 2 ? 12 : 6;
    const uint32_t nch = nh * D / 8u;
    for (uint32_t base = threadIdx.x; base < nch; base += SU * blockDim.x) {
      Chunk8<XT> c[SU];
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const uint32_t ch = min(base + (uint32_t)u * blockDim.x, nch - 1u);
        chunk_load(c[u], x + (size_t)t0 * D + (size_t)ch * 8u);
      }
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const uint32_t ch = base + (uint32_t)u * blockDim.x;
        if (ch >= nch) continue;
        const uint32_t f0 = ch * 8u, tt = f0 / D, c0 = f0 - tt * D;
        float v[8];
        chunk_vals(c[u], v);
        float *dst = xs + (size_t)tt * Dpad + tpos(c0);
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[64 * j] = v[j];
      }
    }
  } else {
    for (uint32_t f = threadIdx.x; f < nh * D; f += blockDim.x) {
      const uint32_t tt = f / D, c = f - tt * D;
      xs[(size_t)tt * Dpad + tpos(c)] = load_val(x, (size_t)t0 * D + f);
    }
  }
  __syncthreads();

  // 4 (first, all waves): r per token, tokens w and w + 4 of the block
  if (a.apply_norm) {
    float ss[2] = {0.0f, 0.0f};
    for (uint32_t c0 = 8u * lane; c0 < D; c0 += 512u) {
      const uint32_t nv = min(8u, D - c0), q0 = tpos(c0);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (w + 4u * h >= a.tb) continue;
        const float *xq = xs + (size_t)(w + 4u * h) * Dpad + q0;
#pragma unroll
        for (uint32_t j = 0; j < 8u; ++j)
          if (VEC || j < nv) ss[h] = fmaf(xq[64u * j], xq[64u * j], ss[h]);
      }
    }
    wave_sum_butterfly_n<2>(ss);
    if (lane == 0) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t tt = w + 4u * h;
        if (tt < nh) {
          rr[tt] = sqrtf(ss[h] / (float)D + a.eps);
          if (a.rms && blockIdx.y == 0) a.rms[t0 + tt] = rr[tt];
        }
      }
    }
  }

  __syncthreads();  // rr visible
  // normalised rows xn = x * (1/r) * gamma (x without RmsNorm) for the expert GEMV in the x dtype,
  // zero padded to Dp, and (grouped GEMM) their two-term form zero padded to the K-group
  // length.  Every expert group shares the writing (chunk or block i of the token block by group
  // i mod gridDim.y), before the dot products so the stores drain meanwhile.
  auto gamma8 = [&](uint32_t c0, float g[8]) {  // gamma[c0 .. c0 + 8), ones beyond D
    if (VEC && c0 < D) {  // D % 8 == 0: the whole chunk is inside
      const float4 g0 = *(const float4 *)(a.gamma + c0), g1 = *(const float4 *)(a.gamma + c0 + 4);
      g[0] = g0.x; g[1] = g0.y; g[2] = g0.z; g[3] = g0.w; g[4] = g1.x; g[5] = g1.y; g[6] = g1.z; g[7] = g1.w;
    } else {
#pragma unroll
      for (uint32_t j = 0; j < 8u; ++j) g[j] = c0 + j < D ? a.gamma[c0 + j] : 1.0f;
    }
  };
  const uint32_t wstart = threadIdx.x + blockDim.x * blockIdx.y, wstep = blockDim.x * gridDim.y;
  if (a.xn) {
    XT *xn = (XT *)a.xn;
    const uint32_t cpr = a.Dp / 8u;  // Dp is a multiple of 32
    for (uint32_t ch = wstart; ch < nh * cpr; ch += wstep) {
      const uint32_t tt = ch / cpr, c0 = (ch - tt * cpr) * 8u;
      const float ir = a.apply_norm ? 1.0f / rr[tt] : 1.0f;
      float g[8], v[8];
      if (a.apply_norm) gamma8(c0, g);
#pragma unroll
      for (uint32_t j = 0; j < 8u; ++j) {
        const uint32_t c = c0 + j;
        float u = 0.0f;
        if (c < D) {
          u = xs[(size_t)tt * Dpad + tpos(c)];
          if (a.apply_norm) u = (u * ir) * g[j];
        }
        v[j] = u;
      }
      if (a.xn_bf16)
        store8((uint16_t *)a.xn + (size_t)(t0 + tt) * a.Dp + c0, v);
      else
        store8(xn + (size_t)(t0 + tt) * a.Dp + c0, v);
    }
  }
  if (a.xq.hi) {
    // one 32-value block per thread-iteration
    const uint32_t nbk = a.xq.kq >> 5;
    for (uint32_t f = wstart; f < nh * nbk; f += wstep) {
      const uint32_t tt = f / nbk, bk = f - tt * nbk;
      const float ir = a.apply_norm ? 1.0f / rr[tt] : 1.0f;
      float v[32], amax = 0.0f;
#pragma unroll
      for (uint32_t q = 0; q < 4u; ++q) {
        float g[8];
        if (a.apply_norm) gamma8(bk * 32u + 8u * q, g);
#pragma unroll
        for (uint32_t j = 0; j < 8u; ++j) {
          const uint32_t c = bk * 32u + 8u * q + j;
          float u = 0.0f;
          if (c < D) {
            u = xs[(size_t)tt * Dpad + tpos(c)];
            if (a.apply_norm) u = (u * ir) * g[j];
          }
          v[8u * q + j] = u;
          amax = fmaxf(amax, fabsf(u));
        }
      }
      const size_t row = t0 + tt;
      mx84_quantize32(v, amax, a.xq.hi + row * a.xq.kq + bk * 32u, a.xq.lo + row * (a.xq.kq / 2u) + bk * 16u,
                      a.xq.shi + row * a.xq.ss + bk, a.xq.slo + row * a.xq.ss + bk);
    }
  }

  // 3. dot products
  float acc0[8], acc1[8];
#pragma unroll
  for (int tt = 0; tt < 8; ++tt) acc0[tt] = acc1[tt] = 0.0f;
  if (has0) {
    for (uint32_t cg = 0; cg < D; cg += 512u * RC) {
      if (VEC && cg > 0) {
#pragma unroll
        for (int i = 0; i < RC; ++i) {
          const uint32_t c0 = cg + 512u * i + 8u * lane;
          if (c0 < D) chunk_load(r0[i], rw + (size_t)e0 * D + c0);
          if (has1 && c0 < D) chunk_load(r1[i], rw + (size_t)e1 * D + c0);
        }
      }
#pragma unroll
      for (int i = 0; i < RC; ++i) {
        const uint32_t c0 = cg + 512u * i + 8u * lane;
        if (c0 >= D) continue;
        const uint32_t nv = min(8u, D - c0);
        float w0[8], w1[8];
        if (VEC) {
          chunk_vals(r0[i], w0);
          if (has1) chunk_vals(r1[i], w1);
        } else {
          load8_guarded(rw + (size_t)e0 * D + c0, nv, w0);
          if (has1) load8_guarded(rw + (size_t)e1 * D + c0, nv, w1);
        }
        const uint32_t q0 = tpos(c0);
#pragma unroll
        for (uint32_t tt = 0; tt < 8u; ++tt) {
          if (tt >= a.tb) break;
          const float *xq = xs + (size_t)tt * Dpad + q0;  // rows in [nh, tb) hold stale data; unused
#pragma unroll
          for (uint32_t j = 0; j < 8u; ++j) {
            if (VEC || j < nv) {
              const float xv = xq[64u * j];
              acc0[tt] = fmaf(xv, w0[j], acc0[tt]);
              if (has1) acc1[tt] = fmaf(xv, w1[j], acc1[tt]);
            }
          }
        }
      }
    }
    wave_sum_butterfly_n<8>(acc0);
    if (has1) wave_sum_butterfly_n<8>(acc1);
  }
  if (has0 && lane < nh) {
    // lane tt writes token tt's logits (all lanes hold the reduced values)
    float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
    for (uint32_t tt = 0; tt < 8u; ++tt)
      if (lane == tt) {
        v0 = acc0[tt];
        v1 = acc1[tt];
      }
    const uint32_t t = t0 + lane;
    const float r = a.apply_norm ? rr[lane] : 1.0f;
    a.logits[(size_t)t * E + e0] = (a.apply_norm ? v0 / r : v0) + a.rb[e0];
    if (has1) a.logits[(size_t)t * E + e1] = (a.apply_norm ? v1 / r : v1) + a.rb[e1];
  }
}

// ---------------------------------------------------------------------------------------------
// Prefill router (D % 8 == 0, D, Dp and the two-term row length <= 512 * kFrontChunks, 16-byte
// aligned rows).  Workgroup of kRowsThreads: wave w holds tokens T (8 b + w) .. +T in registers
// (f32, T = 2 or 4); the router rows pass through LDS as f32 in stages of kRowsExperts experts (double
// buffered, filled by all threads, one barrier per stage), so each row is converted once per
// workgroup and read by every wave from LDS.  LDS row layout: element 512 i + 8 l + j at
// 512 i + 256 (j / 4) + 4 l + j % 4, so lane l's two float4 of its chunk are conflict-free.
// Same fixed reduction order and formulas as router_kernel (lane l owns chunks c = 512 i + 8 l + j,
// fmaf over i then j, xor butterfly; logit = dot / r + b): the logits, r and the written rows
// equal router_kernel's bit for bit.  The two-term rows come from the registers: a 32-value
// block is the 8-value chunks of lanes 4 b .. 4 b + 3, its maxima taken over those four lanes.
// ---------------------------------------------------------------------------------------------
constexpr int kRowsExperts = 4;    // experts per LDS stage
constexpr uint32_t kRowsSpan = 512u * kFrontChunks;  // f32 LDS row stride
size_t router_rows_lds_bytes() { return sizeof(float) * (2u * kRowsExperts * kRowsSpan + kMaxExperts); }

template <typename XT, typename WT, int T>  // T tokens per wave (2, or 4 for the largest batches)
__global__ __launch_bounds__(kRowsThreads) void router_rows_kernel(RouterArgs a) {
  constexpr int G = kRowsExperts, RC = kFrontChunks;
  constexpr uint32_t FC = (G * kRowsSpan / 8u + kRowsThreads - 1u) / kRowsThreads;  // fill chunks per thread
  extern __shared__ __align__(16) float wls[];  // [2][G][kRowsSpan], then rb [E]
  float *rbl = wls + 2u * G * kRowsSpan;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t t0 = (blockIdx.x * (kRowsThreads / 64u) + (threadIdx.x >> 6)) * (uint32_t)T;
  const bool active = t0 < a.n;  // wave-uniform; inactive waves still fill and meet the barriers
  const uint32_t D = a.D, E = a.E, cpr = D / 8u;  // chunks per router row
  const XT *x = (const XT *)a.x;
  const WT *rw = (const WT *)a.rw;
  const uint32_t nt = active ? min((uint32_t)T, a.n - t0) : 0u;
  const uint32_t nstage = (E + G - 1u) / G;

  // stage fill: chunk f = threadIdx.x + kRowsThreads m of a stage is chunk ch = f % cpr (= 64 i + l)
  // of the stage's expert row k = f / cpr
  uint32_t fk[FC], fsrc[FC], fdst[FC];
#pragma unroll
  for (uint32_t m = 0; m < FC; ++m) {
    const uint32_t f = threadIdx.x + kRowsThreads * m, k = f / cpr, ch = f - k * cpr;
    fk[m] = k;
    fsrc[m] = k * D + ch * 8u;
    fdst[m] = k * kRowsSpan + (ch >> 6) * 512u + (ch & 63u) * 4u;
  }
  Chunk8<WT> fr[FC];
  auto fill_load = [&](uint32_t st) {
#pragma unroll
    for (uint32_t m = 0; m < FC; ++m)
      if (fk[m] < (uint32_t)G && st * G + fk[m] < E) chunk_load(fr[m], rw + (size_t)st * G * D + fsrc[m]);
  };
  auto fill_store = [&](uint32_t st, uint32_t buf) {
#pragma unroll
    for (uint32_t m = 0; m < FC; ++m) {
      if (fk[m] < (uint32_t)G && st * G + fk[m] < E) {
        float v[8];
        chunk_vals(fr[m], v);
        float *d = wls + buf * G * kRowsSpan + fdst[m];
        *(float4 *)d = make_float4(v[0], v[1], v[2], v[3]);
        *(float4 *)(d + 256) = make_float4(v[4], v[5], v[6], v[7]);
      }
    }
  };
  fill_load(0);
  for (uint32_t e = threadIdx.x; e < E; e += kRowsThreads) rbl[e] = a.rb[e];
  // zeros at the chunk positions beyond D of every row (never filled): the dot loop runs over
  // all RC chunks, and fmaf(0, 0, acc) == acc for the +0-started sums
  for (uint32_t f = threadIdx.x; f < 2u * G * (RC * 64u - cpr); f += kRowsThreads) {
    const uint32_t row = f / (RC * 64u - cpr), ch = cpr + (f - row * (RC * 64u - cpr));
    float *d = wls + row * kRowsSpan + (ch >> 6) * 512u + (ch & 63u) * 4u;
    *(float4 *)d = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    *(float4 *)(d + 256) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }

  // this wave's token rows as f32 (zeros beyond D), every chunk requested before any is used: no
  // branch around a load (a branch per chunk made the wave wait for the chunks one by one), so
  // chunks past D or of an inactive wave read a valid chunk and are zeroed
  float xv[T][RC][8];
  {
    Chunk8<XT> cx[T][RC];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < RC; ++i) {
        const uint32_t c0 = min(512u * i + 8u * lane, D - 8u);
        const uint32_t row = min(t0 + min((uint32_t)t, max(nt, 1u) - 1u), a.n - 1u);
        chunk_load(cx[t][i], x + (size_t)row * D + c0);
      }
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < RC; ++i) {
        const bool ok = active && 512u * i + 8u * lane < D;
        chunk_vals(cx[t][i], xv[t][i]);
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[t][i][j] = ok ? xv[t][i][j] : 0.0f;
      }
  }

  // r per token
  float r[T];
#pragma unroll
  for (int t = 0; t < T; ++t) r[t] = 1.0f;
  if (a.apply_norm) {
    float ss[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      ss[t] = 0.0f;
#pragma unroll
      for (int i = 0; i < RC; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) ss[t] = fmaf(xv[t][i][j], xv[t][i][j], ss[t]);
    }
    wave_sum_to_lane0_n<T>(ss);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      r[t] = sqrtf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss[t]), 0)) / (float)D + a.eps);
      if (a.rms && lane == 0 && (uint32_t)t < nt) a.rms[t0 + t] = r[t];
    }
  }

  // normalised rows xn = x * (1/r) * gamma (x without RmsNorm), zero padded to Dp, and their
  // two-term form zero padded to the K-group length; written before the dot products so
  // the stores drain meanwhile
  if (active && (a.xn || a.xq.hi)) {
#pragma unroll
    for (int i = 0; i < RC; ++i) {
      const uint32_t c0 = 512u * i + 8u * lane;
      if (512u * i >= max(a.xn ? a.Dp : 0u, a.xq.hi ? a.xq.kq : 0u)) break;  // wave-uniform
      float g[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) g[j] = 1.0f;
      if (a.apply_norm && c0 < D) {
        const float4 g0 = *(const float4 *)(a.gamma + c0), g1 = *(const float4 *)(a.gamma + c0 + 4);
        g[0] = g0.x; g[1] = g0.y; g[2] = g0.z; g[3] = g0.w; g[4] = g1.x; g[5] = g1.y; g[6] = g1.z; g[7] = g1.w;
      }
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float ir = a.apply_norm ? 1.0f / r[t] : 1.0f;
        float u[8];  // zeros beyond D: xv is zero there and gamma one
#pragma unroll
        for (int j = 0; j < 8; ++j) u[j] = a.apply_norm ? (xv[t][i][j] * ir) * g[j] : xv[t][i][j];
        const size_t row = t0 + (uint32_t)t;
        const bool tv = (uint32_t)t < nt;
        if (a.xn && tv && c0 < a.Dp) store8((XT *)a.xn + row * a.Dp + c0, u);
        if (a.xq.hi && 512u * i < a.xq.kq) {  // wave-uniform
          float amax = 0.0f;
#pragma unroll
          for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(u[j]));
          amax = fmaxf(amax, dpp_mov<0xB1>(amax));  // lanes 4 b .. 4 b + 3 hold block b
          amax = fmaxf(amax, dpp_mov<0x4E>(amax));
          const uint32_t sbh = mx8_scale_byte(amax);
          const float ih = sbh ? mx8_inv_scale(sbh) : 0.0f, sh = e8m0_to_f32(sbh);
          uint32_t ch[4];
          float res[8], rmax = 0.0f;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            ch[k] = f32x2_to_fp8x2(u[2 * k] * ih, u[2 * k + 1] * ih);
            res[2 * k] = u[2 * k] - fp8_to_f32<0>(ch[k]) * sh;
            res[2 * k + 1] = u[2 * k + 1] - fp8_to_f32<1>(ch[k]) * sh;
            rmax = fmaxf(rmax, fmaxf(fabsf(res[2 * k]), fabsf(res[2 * k + 1])));
          }
          rmax = fmaxf(rmax, dpp_mov<0xB1>(rmax));
          rmax = fmaxf(rmax, dpp_mov<0x4E>(rmax));
          const uint32_t sbl = mx4_scale_byte(rmax);
          const float sl = mx4_divisor(sbl);
          if (tv && c0 < a.xq.kq) {
            uint32_t cl = 0u;
            cl = e2m1x2<0>(cl, res[0], res[1], sl);
            cl = e2m1x2<1>(cl, res[2], res[3], sl);
            cl = e2m1x2<2>(cl, res[4], res[5], sl);
            cl = e2m1x2<3>(cl, res[6], res[7], sl);
            *(uint2 *)(a.xq.hi + row * a.xq.kq + c0) = make_uint2(ch[0] | (ch[1] << 16), ch[2] | (ch[3] << 16));
            *(uint32_t *)(a.xq.lo + row * (a.xq.kq / 2u) + c0 / 2u) = cl;
            if ((lane & 3u) == 0u) {
              a.xq.shi[row * a.xq.ss + (c0 >> 5)] = (uint8_t)sbh;
              a.xq.slo[row * a.xq.ss + (c0 >> 5)] = (uint8_t)sbl;
            }
          }
        }
      }
    }
  }

  fill_store(0, 0);
  __syncthreads();

  // dot products, G experts per stage; lane q < G * T finishes (expert st * G + q / T, token q % T)
  for (uint32_t st = 0; st < nstage; ++st) {
    const uint32_t buf = st & 1u;
    if (st + 1u < nstage) fill_load(st + 1u);
    if (active) {
      float acc[G * T];
#pragma unroll
      for (int q = 0; q < G * T; ++q) acc[q] = 0.0f;
#pragma unroll
      for (int k = 0; k < G; ++k) {
        const float *wrow = wls + (buf * G + k) * kRowsSpan + lane * 4u;
#pragma unroll
        for (int i = 0; i < RC; ++i) {
          const float4 w0 = *(const float4 *)(wrow + 512u * i), w1 = *(const float4 *)(wrow + 512u * i + 256u);
          const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
          for (int t = 0; t < T; ++t)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[k * T + t] = fmaf(xv[t][i][j], w[j], acc[k * T + t]);
        }
      }
      wave_sum_to_lane0_n<G * T>(acc);
      float v = 0.0f, rq = r[0];
#pragma unroll
      for (int q = 0; q < G * T; ++q) {
        const float aq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc[q]), 0));
        if (lane == (uint32_t)q) {
          v = aq;
          rq = r[q % T];
        }
      }
      const uint32_t e = st * G + lane / T, t = lane % T;
      if (lane < (uint32_t)(G * T) && e < E && t < nt)
        a.logits[(size_t)(t0 + t) * E + e] = (a.apply_norm ? v / rq : v) + rbl[e];
    }
    if (st + 1u < nstage) {
      fill_store(st + 1u, buf ^ 1u);
      __syncthreads();
    }
  }
}

__device__ __forceinline__ uint32_t readlane_u(uint32_t v, uint32_t k) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)k);
}
template <int CTRL> __device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
// Inclusive prefix sum over the wave's lanes: row_shr 1, 2, 4, 8 inside each row of 16 (lanes
// without a source add 0), then the totals of the rows below (lanes 15, 31, 47).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  v += dpp_u<0x111>(v);  // row_shr:1
  v += dpp_u<0x112>(v);  // row_shr:2
  v += dpp_u<0x114>(v);  // row_shr:4
  v += dpp_u<0x118>(v);  // row_shr:8
  const uint32_t r0 = readlane_u(v, 15), r1 = readlane_u(v, 31), r2 = readlane_u(v, 47);
  const uint32_t row = (threadIdx.x & 63u) >> 4;
  return v + (row == 0u ? 0u : row == 1u ? r0 : row == 2u ? r0 + r1 : r0 + r1 + r2);
}
// The same inside each half-wave of 32 lanes (lanes 0-31 and 32-63 scanned separately).
__device__ __forceinline__ uint32_t half_wave_incl_scan(uint32_t v) {
  v += dpp_u<0x111>(v);
  v += dpp_u<0x112>(v);
  v += dpp_u<0x114>(v);
  v += dpp_u<0x118>(v);
  const uint32_t r0 = readlane_u(v, 15), r2 = readlane_u(v, 47);
  const uint32_t row = (threadIdx.x & 63u) >> 4;
  return v + (row == 1u ? r0 : row == 3u ? r2 : 0u);
}

// Exclusive prefix sums over the experts e < E (E <= 256) of their entry counts c_e, of
// [c_e > 0] and of ceil(c_e / kGemmTok), for thread e (threads 0 .. 255 of a workgroup of at least
// 256): wave scans, then the totals of the waves below from LDS (tot_l: 12 ints).  Called by
// every thread of the workgroup (two barriers); threads from 256 on get zeros.
__device__ void expert_prefix(const int32_t *cnt, uint32_t E, int32_t *tot_l, int32_t &off, int32_t &ra, int32_t &toff) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
  const int32_t c = (tid < E && tid < kMaxExperts) ? cnt[tid] : 0;
  const uint32_t v0 = (uint32_t)c, v1 = c > 0 ? 1u : 0u, v2 = (uint32_t)((c + (int32_t)kGemmTok - 1) / (int32_t)kGemmTok);
  const uint32_t i0 = wave_incl_scan(v0), i1 = wave_incl_scan(v1), i2 = wave_incl_scan(v2);
  if (w < 4u && lane == 63u) {
    tot_l[3u * w] = (int32_t)i0;
    tot_l[3u * w + 1u] = (int32_t)i1;
    tot_l[3u * w + 2u] = (int32_t)i2;
  }
  __syncthreads();
  int32_t b0 = 0, b1 = 0, b2 = 0;
  for (uint32_t w2 = 0; w2 < w && w2 < 4u; ++w2) {
    b0 += tot_l[3u * w2];
    b1 += tot_l[3u * w2 + 1u];
    b2 += tot_l[3u * w2 + 2u];
  }
  off = b0 + (int32_t)(i0 - v0);
  ra = b1 + (int32_t)(i1 - v1);
  toff = b2 + (int32_t)(i2 - v2);
  __syncthreads();  // tot_l free again
}

// (h, l) = the larger of the 64-bit keys (h, l) and (h2, l2), high word first
__device__ __forceinline__ void key_max(uint32_t &h, uint32_t &l, uint32_t h2, uint32_t l2) {
  const bool g = h2 > h || (h2 == h && l2 > l);
  h = g ? h2 : h;
  l = g ? l2 : l;
}
// Maximum of the 64-bit keys (h, l) over the wave, in every lane: quad permutations (lanes
// l ^ 1, l ^ 2), row rotations by 4 and 8 (the row's four quads), then the permlane swaps
// between rows 16 and 32 apart.
__device__ __forceinline__ void wave_max_key(uint32_t &h, uint32_t &l) {
  key_max(h, l, dpp_u<0xB1>(h), dpp_u<0xB1>(l));    // quad_perm [1,0,3,2]
  key_max(h, l, dpp_u<0x4E>(h), dpp_u<0x4E>(l));    // quad_perm [2,3,0,1]
  key_max(h, l, dpp_u<0x124>(h), dpp_u<0x124>(l));  // row_ror:4
  key_max(h, l, dpp_u<0x128>(h), dpp_u<0x128>(l));  // row_ror:8
  {
    const auto ph = __builtin_amdgcn_permlane16_swap(h, h, false, false);
    const auto pl = __builtin_amdgcn_permlane16_swap(l, l, false, false);
    h = ph[0];
    l = pl[0];
    key_max(h, l, ph[1], pl[1]);
  }
  {
    const auto ph = __builtin_amdgcn_permlane32_swap(h, h, false, false);
    const auto pl = __builtin_amdgcn_permlane32_swap(l, l, false, false);
    h = ph[0];
    l = pl[0];
    key_max(h, l, ph[1], pl[1]);
  }
}

// ---------------------------------------------------------------------------------------------
// Top-k and softmax, one wave per token: lane l holds experts l + 64 j (j < J); K rounds of a
// wave-wide maximum of the packed keys topk_key (larger value, NaN lowest, ties to the lower index)
// not yet taken select the experts of ranks 0 .. K-1 in order.  Softmax over the selected logits:
// w_p = exp(v_p - v_0) / sum_q exp(v_q - v_0), the sum taken q = 0..K-1 ascending from 0.
// Same selection and weights as route_small_body.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float softmax_weight(const float *selv, uint32_t K, uint32_t p) {
  const float m = selv[0];
  float s = 0.0f;
  for (uint32_t q = 0; q < K; ++q) s += expf(selv[q] - m);
  return expf(selv[p] - m) / s;
}

template <int J>  // E <= 64 J
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(TopkArgs a) {
  __shared__ float selv_l[kTopkThreads / 64u][kMaxTopK];
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t t = blockIdx.x * (blockDim.x >> 6) + w;
  if (t >= a.n) return;  // wave-uniform, and no workgroup barrier follows
  const uint32_t E = a.E, K = a.K;
  float v[J];
  uint32_t kh[J], kl[J], rank[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t e = lane + 64u * j;
    v[j] = e < E ? a.logits[(size_t)t * E + e] : 0.0f;
    const uint64_t key = topk_key(v[j], e);
    kh[j] = (uint32_t)(key >> 32);
    kl[j] = (uint32_t)key;
    rank[j] = ~0u;
  }
  for (uint32_t r = 0; r < K; ++r) {
    uint32_t bh = 0u, bl = 0u;  // below every real key (the low word ~index is never 0)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const bool cand = lane + 64u * j < E && rank[j] == ~0u;
      if (cand && (kh[j] > bh || (kh[j] == bh && kl[j] > bl))) {
        bh = kh[j];
        bl = kl[j];
      }
    }
    wave_max_key(bh, bl);
#pragma unroll
    for (int j = 0; j < J; ++j)
      if (lane + 64u * j < E && kh[j] == bh && kl[j] == bl) rank[j] = r;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t e = lane + 64u * j;
    if (e < E && rank[j] < K) {
      selv_l[w][rank[j]] = v[j];
      a.topk_idx[(size_t)t * K + rank[j]] = (int32_t)e;
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's selv_l writes complete (lgkmcnt(0) only)
  __builtin_amdgcn_wave_barrier();
  for (uint32_t p = lane; p < K; p += 64u) a.topk_w[(size_t)t * K + p] = softmax_weight(selv_l[w], K, p);
}


// ---------------------------------------------------------------------------------------------
// Dispatch by one workgroup (any batch size).  Stable counting sort of the flat entries t*K+p by
// expert: the rank of (t, e) inside expert e's segment is the number of earlier tokens that chose
// e, computed per chunk of blockDim.x tokens from a per-expert token bitmap (order-independent
// atomicOr) and popcount prefixes, so the result does not depend on thread timing.
// LDS: cnt[E], base[E], bm[E * words], wpre[E * words] (words = blockDim.x / 32).
// ---------------------------------------------------------------------------------------------
__device__ void block_dispatch(const int32_t *idx, uint32_t n, uint32_t K, uint32_t E, int32_t *seg_off,
                               int32_t *perm, int32_t *pos_of, int32_t *active, int32_t *num_active,
                               int32_t *exrec, int32_t *tile_off, int32_t *lds) {
  const uint32_t tid = threadIdx.x, nth = blockDim.x, words = nth >> 5;  // 32 words: nth = 1024
  int32_t *cnt = lds, *base = lds + E;
  uint32_t *bm = (uint32_t *)(lds + 2 * E);
  int32_t *wpre = lds + 2 * E + E * words;
  int32_t *aidx = wpre + E * words;  // active slot of each expert
  int32_t *segs = aidx + E;          // segment start of each expert
  int32_t *tot_l = segs + E + 1;     // [12] wave totals of expert_prefix
  for (uint32_t e = tid; e < E; e += nth) cnt[e] = 0;
  __syncthreads();
  for (uint32_t i = tid; i < n * K; i += nth) {
    const int32_t e = idx[i];
    if (e >= 0 && (uint32_t)e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // exclusive scans and active list (expert e by thread e)
  int32_t off, ra, toff;
  expert_prefix(cnt, E, tot_l, off, ra, toff);
  if (tid < E) {
    const uint32_t e = tid;
    if (tile_off) tile_off[e] = toff;
    seg_off[e] = off;
    base[e] = off;
    segs[e] = off;
    aidx[e] = ra;
    if (cnt[e] > 0) {
      active[ra] = (int32_t)e;
      exrec[ra * kRecWords + 0] = (int32_t)e;
      exrec[ra * kRecWords + 1] = off;
      exrec[ra * kRecWords + 2] = cnt[e];
    }
    if (e + 1 == E) {
      seg_off[E] = off + cnt[e];
      if (tile_off) tile_off[E] = toff + (cnt[e] + (int32_t)kGemmTok - 1) / (int32_t)kGemmTok;
      const int32_t na = ra + (cnt[e] > 0);
      *num_active = na;
      lds[4 * E + 2 * E * words] = na;
      for (uint32_t e3 = (uint32_t)na; e3 < E; ++e3) active[e3] = -1;
    }
  }
  __syncthreads();
  for (uint32_t c0 = 0; c0 < n; c0 += nth) {
    for (uint32_t i = tid; i < E * words; i += nth) bm[i] = 0u;
    __syncthreads();
    const uint32_t t = c0 + tid;
    const uint32_t wi = tid >> 5, bit = tid & 31u;
    if (t < n) {
      for (uint32_t p = 0; p < K; ++p) {
        const int32_t e = idx[t * K + p];
        if (e >= 0 && (uint32_t)e < E) atomicOr(&bm[e * words + wi], 1u << bit);
      }
    }
    __syncthreads();
    // popcount prefixes over each expert's 32 bitmap words: word i by lane i mod 64 of a
    // half-wave scan (every wave runs the same number of rounds)
    for (uint32_t i0 = 0; i0 < E * words; i0 += nth) {
      const uint32_t i = i0 + tid;
      const uint32_t v = i < E * words ? (uint32_t)__popc(bm[i]) : 0u;
      const uint32_t incl = half_wave_incl_scan(v);
      if (i < E * words) wpre[i] = (int32_t)(incl - v);
    }
    __syncthreads();
    if (t < n) {
      for (uint32_t p = 0; p < K; ++p) {
        const int32_t e = idx[t * K + p];
        if (e < 0 || (uint32_t)e >= E) continue;
        const int32_t r = wpre[e * words + wi] + __popc(bm[e * words + wi] & ((1u << bit) - 1u));
        const int32_t pos = base[e] + r;
        perm[pos] = (int32_t)(t * K + p);
        pos_of[t * K + p] = pos;
        const int32_t j = pos - segs[e];  // entry index inside the expert's segment
        if (j < (int32_t)kRecTokens) {
          exrec[aidx[e] * kRecWords + 4 + j] = (int32_t)t;
          exrec[aidx[e] * kRecWords + 4 + kRecTokens + j] = (int32_t)(t * K + p);
        }
      }
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += nth) base[e] += wpre[e * words + words - 1] + __popc(bm[e * words + words - 1]);
    __syncthreads();
  }
}

size_t dispatch_lds_bytes(uint32_t E, uint32_t threads) {
  return sizeof(int32_t) * ((size_t)E * (4 + 2 * (threads / 32)) + 16);
}

// Dispatch of a large batch in two launches over chunks of kDispatchChunk tokens (workgroup c owns
// tokens [c * kDispatchChunk, +kDispatchChunk), thread = token).  dispatch_count_kernel: the
// per-expert entry counts of each chunk (LDS atomics: order-independent).  dispatch_wide_kernel:
// totals and earlier-chunk counts from those; an entry's segment position is seg_off[e] + (entries
// of e in earlier chunks) + (rank among this chunk's tokens choosing e, from a per-expert token
// bitmap).  Its workgroup 0 writes the segment offsets, token-tile prefix, active list and
// records.  Results equal block_dispatch's.
__global__ __launch_bounds__(kDispatchChunk) void dispatch_count_kernel(DispatchArgs a) {
  __shared__ int32_t cnt[kMaxExperts];
  const uint32_t tid = threadIdx.x, E = a.E, K = a.K;
  for (uint32_t e = tid; e < E; e += kDispatchChunk) cnt[e] = 0;
  __syncthreads();
  const uint32_t t = blockIdx.x * kDispatchChunk + tid;
  if (t < a.n) {
    if (K <= 8u) {  // the token's K indices requested together (a loop waits for each in turn)
      int32_t ev[8];
#pragma unroll
      for (uint32_t p = 0; p < 8u; ++p) ev[p] = a.topk_idx[(size_t)t * K + min(p, K - 1u)];
#pragma unroll
      for (uint32_t p = 0; p < 8u; ++p)
        if (p < K && ev[p] >= 0 && (uint32_t)ev[p] < E) atomicAdd(&cnt[ev[p]], 1);
    } else {
      for (uint32_t p = 0; p < K; ++p) {
        const int32_t e = a.topk_idx[(size_t)t * K + p];
        if (e >= 0 && (uint32_t)e < E) atomicAdd(&cnt[e], 1);
      }
    }
  }
  __syncthreads();
  for (uint32_t e = tid; e < E; e += kDispatchChunk) a.chunk_cnt[(size_t)blockIdx.x * E + e] = cnt[e];
}

__global__ __launch_bounds__(kDispatchChunk) void dispatch_wide_kernel(DispatchArgs a) {
  constexpr uint32_t W = kDispatchChunk / 32u;  // bitmap words per expert
  static_assert(kDispatchChunk >= kMaxExperts, "expert_prefix: thread e handles expert e");
  __shared__ int32_t call[kMaxExperts], cbef[kMaxExperts], segs[kMaxExperts], aidx[kMaxExperts], base[kMaxExperts];
  __shared__ uint32_t bm[kMaxExperts * W];
  __shared__ int32_t tot_l[12];
  const uint32_t tid = threadIdx.x, c = blockIdx.x, E = a.E, K = a.K, n = a.n;
  const uint32_t t = c * kDispatchChunk + tid;
  const uint32_t nchunk = gridDim.x;
  for (uint32_t e = tid; e < E; e += kDispatchChunk) call[e] = cbef[e] = 0;
  for (uint32_t i = tid; i < E * W; i += kDispatchChunk) bm[i] = 0u;
  __syncthreads();
  // every chunk's counts, all loads issued together: totals and earlier-chunk sums (LDS integer
  // atomics, order-independent)
  // (8 per thread at a time, clamped past the end: a plain loop waited for each load in turn)
  const uint32_t ncnt = nchunk * E;
  for (uint32_t i0 = tid; i0 < ncnt; i0 += 8u * kDispatchChunk) {
    int32_t v[8];
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) v[u] = a.chunk_cnt[min(i0 + u * kDispatchChunk, ncnt - 1u)];
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      const uint32_t i = i0 + u * kDispatchChunk;
      if (i < ncnt && v[u] != 0) {
        const uint32_t c2 = i / E, e = i - c2 * E;
        atomicAdd(&call[e], v[u]);
        if (c2 < c) atomicAdd(&cbef[e], v[u]);
      }
    }
  }
  __syncthreads();
  if (t < n) {
    if (K <= 8u) {  // the token's K indices requested together
      int32_t ev[8];
#pragma unroll
      for (uint32_t p = 0; p < 8u; ++p) ev[p] = a.topk_idx[(size_t)t * K + min(p, K - 1u)];
#pragma unroll
      for (uint32_t p = 0; p < 8u; ++p)
        if (p < K && ev[p] >= 0 && (uint32_t)ev[p] < E) atomicOr(&bm[ev[p] * W + (tid >> 5)], 1u << (tid & 31u));
    } else {
      for (uint32_t p = 0; p < K; ++p) {
        const int32_t e = a.topk_idx[(size_t)t * K + p];
        if (e >= 0 && (uint32_t)e < E) atomicOr(&bm[e * W + (tid >> 5)], 1u << (tid & 31u));
      }
    }
  }
  __syncthreads();
  // exclusive scans over experts (expert e by thread e)
  int32_t off, ra, toff;
  expert_prefix(call, E, tot_l, off, ra, toff);
  if (tid < E) {
    const uint32_t e = tid;
    segs[e] = off;
    aidx[e] = ra;
    base[e] = off + cbef[e];
    if (c == 0) {
      if (a.tile_off) a.tile_off[e] = toff;
      a.seg_off[e] = off;
      if (call[e] > 0) {
        a.active[ra] = (int32_t)e;
        a.exrec[ra * kRecWords + 0] = (int32_t)e;
        a.exrec[ra * kRecWords + 1] = off;
        a.exrec[ra * kRecWords + 2] = call[e];
      }
      if (e + 1 == E) {
        a.seg_off[E] = off + call[e];
        if (a.tile_off) a.tile_off[E] = toff + (call[e] + (int32_t)kGemmTok - 1) / (int32_t)kGemmTok;
        const int32_t na = ra + (call[e] > 0);
        *a.num_active = na;
        for (uint32_t e3 = (uint32_t)na; e3 < E; ++e3) a.active[e3] = -1;
      }
    }
  }
  __syncthreads();
  if (t >= n) return;
  const uint32_t wi = tid >> 5, bit = tid & 31u;
  for (uint32_t p = 0; p < K; ++p) {
    const int32_t e = a.topk_idx[(size_t)t * K + p];
    if (e < 0 || (uint32_t)e >= E) continue;
    int32_t r = __popc(bm[e * W + wi] & ((1u << bit) - 1u));
    for (uint32_t w2 = 0; w2 < wi; ++w2) r += __popc(bm[e * W + w2]);
    const int32_t pos = base[e] + r;
    const int32_t slot = (int32_t)(t * K + p);
    a.perm[pos] = slot;
    a.pos_of[slot] = pos;
    const int32_t j = pos - segs[e];
    if (j < (int32_t)kRecTokens) {
      a.exrec[aidx[e] * kRecWords + 4 + j] = (int32_t)t;
      a.exrec[aidx[e] * kRecWords + 4 + kRecTokens + j] = slot;
    }
  }
}

__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(DispatchArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  block_dispatch(a.topk_idx, a.n, a.K, a.E, a.seg_off, a.perm, a.pos_of, a.active, a.num_active, a.exrec,
                 a.tile_off, (int32_t *)smem);
}

// ---------------------------------------------------------------------------------------------
// Routing of a decode-sized batch (T <= 16, E <= 256) by one workgroup of T waves.
//  phase 1 (wave t = token t): lane l holds experts l + 64 j (j < J); K rounds of a wave-wide
//    maximum of the packed keys (topk_key, the `beats` order) not yet taken select the experts
//    of ranks 0 .. K-1; softmax over the selected logits (q ascending) by lanes p < K.
//  phase 2 (every wave): per-expert counts and exclusive scans (DPP prefix sums); wave 0 writes
//    the active list and records, wave t token t's segment positions (earlier tokens first).
// Results equal topk_kernel + block_dispatch.
// ---------------------------------------------------------------------------------------------

template <int J>
__device__ void route_small_dispatch(uint32_t T, uint32_t E, uint32_t K, const RouteOut &o,
                                     int8_t (*rank_l)[kSmallRouteMaxTokens], int32_t *na_l);

// Routing of T <= 16 tokens over E <= 64 * J experts from logits lg[t * E + e] (global or LDS) by
// a workgroup of at least T waves.  Every wave of the workgroup must call it (it has a barrier).
template <int J>
__device__ void route_small_body(const float *lg, uint32_t T, uint32_t E, uint32_t K, const RouteOut &o,
                                 int8_t (*rank_l)[kSmallRouteMaxTokens], float (*selv_l)[kMaxTopK],
                                 int32_t *na_l) {
  const uint32_t lane = threadIdx.x & 63u, t = threadIdx.x >> 6;
  if (t < T) {
    float v[J];
    uint64_t key[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t e = lane + 64u * j;
      v[j] = e < E ? lg[(size_t)t * E + e] : 0.0f;
      key[j] = topk_key(v[j], e);
    }
    // K rounds of a wave-wide maximum over the keys not yet taken: round r finds the expert of
    // rank r (keys are unique, so exactly one lane holds it); the rest keep rank ~0u
    uint32_t rank[J], kh[J], kl[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      rank[j] = ~0u;
      kh[j] = (uint32_t)(key[j] >> 32);
      kl[j] = (uint32_t)key[j];
    }
    for (uint32_t r = 0; r < K; ++r) {
      uint32_t bh = 0u, bl = 0u;  // below every real key (the low word ~index is never 0)
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const bool cand = lane + 64u * j < E && rank[j] == ~0u;
        if (cand && (kh[j] > bh || (kh[j] == bh && kl[j] > bl))) {
          bh = kh[j];
          bl = kl[j];
        }
      }
      wave_max_key(bh, bl);
#pragma unroll
      for (int j = 0; j < J; ++j)
        if (lane + 64u * j < E && kh[j] == bh && kl[j] == bl) rank[j] = r;
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t e = lane + 64u * j;
      if (e >= E) continue;
      const bool sel = rank[j] < K;
      rank_l[e][t] = sel ? (int8_t)rank[j] : (int8_t)-1;
      if (sel) {
        selv_l[t][rank[j]] = v[j];
        o.topk_idx[(size_t)t * K + rank[j]] = (int32_t)e;
      }
    }
    // this wave's selv_l writes complete (lgkmcnt(0) only: the global stores stay in flight)
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    for (uint32_t p = lane; p < K; p += 64u) o.topk_w[(size_t)t * K + p] = softmax_weight(selv_l[t], K, p);
  }
  __syncthreads();
  route_small_dispatch<J>(T, E, K, o, rank_l, na_l);
}

// Rank of token t in the 16 rank bytes rk (4 dwords) of one expert: -1 = not chosen.
__device__ __forceinline__ int rank_byte(const uint32_t (&rk)[4], uint32_t t) {
  return (int)(int8_t)(uint8_t)(rk[t >> 2] >> (8u * (t & 3u)));
}

// Dispatch part of route_small_body, run by every wave: each computes the per-expert counts and
// scans (lane e reads the ranks of expert e in all tokens with one 16-byte LDS read,
// rank_l[e][t]); wave 0 writes the per-expert outputs (segment offsets, active list, record
// headers), wave t < T the segment entries of token t (its position inside expert e's segment is
// the number of earlier tokens that chose e).
template <int J>
__device__ void route_small_dispatch(uint32_t T, uint32_t E, uint32_t K, const RouteOut &o,
                                     int8_t (*rank_l)[kSmallRouteMaxTokens], int32_t *na_l) {
  static_assert(kSmallRouteMaxTokens == 16, "one 16-byte read per expert");
  const uint32_t lane = threadIdx.x & 63u, t = threadIdx.x >> 6;
  int cnt[J];
  uint32_t rk[J][4];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t e = lane + 64u * j;
    const uint4 v = e < E ? *(const uint4 *)rank_l[e] : make_uint4(~0u, ~0u, ~0u, ~0u);
    rk[j][0] = v.x;
    rk[j][1] = v.y;
    rk[j][2] = v.z;
    rk[j][3] = v.w;
    int c = 0;
#pragma unroll
    for (uint32_t t2 = 0; t2 < kSmallRouteMaxTokens; ++t2) c += (t2 < T && rank_byte(rk[j], t2) >= 0) ? 1 : 0;
    cnt[j] = c;
  }
  // exclusive scans over the experts (token counts and experts with tokens), chunk by chunk
  int off[J], ra[J];
  int total = 0, nact = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t c = (uint32_t)cnt[j], nz = c > 0u ? 1u : 0u;
    const uint32_t ic = wave_incl_scan(c), inz = wave_incl_scan(nz);
    off[j] = total + (int)(ic - c);
    ra[j] = nact + (int)(inz - nz);
    total += (int)readlane_u(ic, 63);
    nact += (int)readlane_u(inz, 63);
  }
  // seg_off, active[0..nact) from the experts with tokens, active[nact..E) = -1 (disjoint writes)
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t e = lane + 64u * j;
    if (t != 0 || e >= E) continue;
    o.seg_off[e] = off[j];
    if (cnt[j] > 0) {
      o.active[ra[j]] = (int32_t)e;
      int32_t *rec = o.exrec + ra[j] * kRecWords;
      rec[0] = (int32_t)e;
      rec[1] = off[j];
      rec[2] = cnt[j];
    }
    if ((int)e >= nact) o.active[e] = -1;
  }
  if (t == 0 && lane == 0) {
    o.seg_off[E] = total;
    *o.num_active = nact;
    *na_l = nact;
  }
  if (t >= T) return;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t e = lane + 64u * j;
    if (e >= E) continue;
    const int r = rank_byte(rk[j], t);
    if (r < 0) continue;
    int seen = 0;  // earlier tokens that chose e
#pragma unroll
    for (uint32_t t2 = 0; t2 < kSmallRouteMaxTokens; ++t2) seen += (t2 < t && rank_byte(rk[j], t2) >= 0) ? 1 : 0;
    const int pos = off[j] + seen;
    const int32_t slot = (int32_t)(t * K + (uint32_t)r);
    o.perm[pos] = slot;
    o.pos_of[slot] = pos;
    if (seen < (int)kRecTokens) {
      o.exrec[ra[j] * kRecWords + 4 + seen] = (int32_t)t;
      o.exrec[ra[j] * kRecWords + 4 + kRecTokens + seen] = slot;
    }
  }
}

template <int J>
__global__ __launch_bounds__(1024) void small_route_kernel(SmallRouteArgs a) {
  __shared__ __align__(16) int8_t rank_l[kMaxExperts][kSmallRouteMaxTokens];
  __shared__ float selv_l[kSmallRouteMaxTokens][kMaxTopK];
  __shared__ int32_t na_l;
  const RouteOut o{a.topk_idx, a.topk_w, a.seg_off, a.perm, a.pos_of, a.active, a.num_active, a.exrec};
  route_small_body<J>(a.logits, a.n, a.E, a.K, o, rank_l, selv_l, &na_l);
}

// ---------------------------------------------------------------------------------------------
// Decode router (n <= 16 tokens, D % 8 == 0, D <= 512 * kFrontChunks, 16-byte aligned rows):
// workgroup e = expert e, wave w = tokens 2w and 2w + 1.  Every lane issues all of its loads
// at once (router row chunks and both tokens' chunks, and the gamma chunks it normalises), then
// computes the two dot products and sums of squares in the fixed lane order (lane l owns chunks
// c = 512 i + 8 l + j, fmaf over i then j, xor butterfly) -- no LDS, no barrier.
// logit = dot / r + b with r = sqrt(sum(x^2) / D + eps) (r = 1 without RmsNorm).  Workgroup 0
// writes r; the normalised rows xn_t = x_t * (1/r_t) * gamma (x_t without RmsNorm) in the x
// dtype (bf16 with xn_bf16), zero padded to Dp, for the expert GEMV are written chunk by chunk, chunk i (columns
// 512 i ..) by workgroup i mod E, so no workgroup carries all of them.  Results equal
// router_kernel bit for bit.
// ---------------------------------------------------------------------------------------------
template <typename XT, typename WT>
__global__ __launch_bounds__(512) void router_small_kernel(FrontArgs a) {
  constexpr int RC = kFrontChunks;
  const uint32_t D = a.D, E = a.E, n = a.n;
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t e = blockIdx.x;
  const uint32_t t0 = 2u * w, t1 = min(2u * w + 1u, n - 1u);
  const bool has1 = 2u * w + 1u < n;
  const XT *x = (const XT *)a.x;
  const WT *rw = (const WT *)a.rw + (size_t)e * D;
  const bool xn_wg = blockIdx.x == 0 && a.xn;
  // xn chunk i is written by workgroup i mod E
  auto own = [&](int i) { return a.xn != nullptr && (uint32_t)i % E == e; };

  Chunk8<WT> wc[RC];
  Chunk8<XT> xc0[RC], xc1[RC];
  Chunk8<float> gc[RC];
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    const uint32_t c0 = min(512u * i + 8u * lane, D - 8u);  // clamped: lanes past D reload a valid chunk
    chunk_load(wc[i], rw + c0);
    chunk_load(xc0[i], x + (size_t)t0 * D + c0);
    chunk_load(xc1[i], x + (size_t)t1 * D + c0);
    if (own(i) && a.apply_norm) chunk_load(gc[i], a.gamma + c0);
  }
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // dot t0, dot t1, sumsq t0, sumsq t1
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    if (512u * i + 8u * lane >= D) continue;
    float wv[8], x0[8], x1[8];
    chunk_vals(wc[i], wv);
    chunk_vals(xc0[i], x0);
    chunk_vals(xc1[i], x1);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc[0] = fmaf(x0[j], wv[j], acc[0]);
      acc[1] = fmaf(x1[j], wv[j], acc[1]);
      acc[2] = fmaf(x0[j], x0[j], acc[2]);
      acc[3] = fmaf(x1[j], x1[j], acc[3]);
    }
  }
  wave_sum_butterfly_n<4>(acc);
  const float r0 = a.apply_norm ? sqrtf(acc[2] / (float)D + a.eps) : 1.0f;
  const float r1 = a.apply_norm ? sqrtf(acc[3] / (float)D + a.eps) : 1.0f;
  if (lane == 0) {
    a.logits[(size_t)t0 * E + e] = (a.apply_norm ? acc[0] / r0 : acc[0]) + a.rb[e];
    if (has1) a.logits[(size_t)t1 * E + e] = (a.apply_norm ? acc[1] / r1 : acc[1]) + a.rb[e];
    if (blockIdx.x == 0 && a.rms) {
      a.rms[t0] = r0;
      if (has1) a.rms[t1] = r1;
    }
  }
  if (!a.xn) return;
  const float ir0 = 1.0f / r0, ir1 = 1.0f / r1;
  auto put = [&](uint32_t t, uint32_t c0, const float (&v)[8]) {
    if (a.xn_bf16)
      store8((uint16_t *)a.xn + (size_t)t * a.Dp + c0, v);
    else
      store8((XT *)a.xn + (size_t)t * a.Dp + c0, v);
  };
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    const uint32_t c0 = 512u * i + 8u * lane;
    if (!own(i) || c0 >= a.Dp) continue;  // Dp is a multiple of 32, D of 8: a chunk is all data or all padding
    float x0[8], x1[8], g[8];
    if (c0 < D) {
      chunk_vals(xc0[i], x0);
      chunk_vals(xc1[i], x1);
      if (a.apply_norm) {
        chunk_vals(gc[i], g);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          x0[j] = (x0[j] * ir0) * g[j];
          x1[j] = (x1[j] * ir1) * g[j];
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) x0[j] = x1[j] = 0.0f;
    }
    put(t0, c0, x0);
    if (has1) put(t1, c0, x1);
  }
  // rows beyond RC chunks of padding (Dp > 512 * RC cannot happen: Dp <= D + 31 <= 512 * RC + 31)
  for (uint32_t c0 = 512u * RC + 8u * lane; xn_wg && c0 < a.Dp; c0 += 512u) {
    const float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    put(t0, c0, z);
    if (has1) put(t1, c0, z);
  }
}

// ---------------------------------------------------------------------------------------------
// Decode router with its input rows formed first (a decoder's residual after the attention
// block): workgroup (t, g) of 8 waves serves token t and experts 8 g .. 8 g + 7, one per wave.
//   1. every wave requests its expert's router row chunks; the workgroup then forms the row
//      x = resid + (sum_h part_h + bias) (parts in order from 0, the arithmetic of a separate
//      residual-add kernel), chunk c (8 values) by thread c, into LDS; workgroup c mod G writes
//      chunk c to xout;
//   2. wave w forms the logit of expert 8 g + w exactly as router_small_kernel does for (e, t):
//      lane l owns chunks 512 i + 8 l + j, fmaf over i then j for the dot and the sum of squares,
//      xor butterfly, logit = dot / r + b with r = sqrt(sum / D + eps);
//   3. xn_t = x (1/r) gamma (zero padded to Dp; f32, or bf16 with xn_bf16) chunk by chunk, chunk
//      c by workgroup c mod G.
// Logits, r and xn take router_small_kernel's arithmetic on x = xout.  f32 rows, n <= 16,
// D % 8 == 0, D <= 512 * kFrontChunks, nparts <= kFrontMaxParts, 16-byte aligned rows.
// ---------------------------------------------------------------------------------------------
template <typename WT>
__global__ __launch_bounds__(512) void router_front_kernel(PreFrontArgs a) {
  constexpr int RC = kFrontChunks;
  __shared__ __align__(16) float xs[512u * RC];
  const FrontArgs &f = a.f;
  const uint32_t D = f.D, E = f.E, t = blockIdx.x, g = blockIdx.y, G = gridDim.y;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
  const uint32_t e = 8u * g + w;
  const bool ev = e < E;  // wave-uniform
  const WT *rw = (const WT *)f.rw + (size_t)min(e, E - 1u) * D;
  Chunk8<WT> wc[RC];
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    const uint32_t c0 = min(512u * i + 8u * lane, D - 8u);  // clamped: lanes past D reload a valid chunk
    chunk_load(wc[i], rw + c0);
  }
  // this thread's xn chunk (written in step 3) and its gamma values, requested early
  const uint32_t nc = D / 8u, c = tid;
  const bool own = c < f.Dp / 8u && c % G == g && f.xn != nullptr;
  Chunk8<float> gc;
  if (own && f.apply_norm && c < nc) chunk_load(gc, f.gamma + 8u * c);
  // 1. the row
  if (c < nc) {
    const size_t o = (size_t)t * D + 8u * c;
    float sv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    Chunk8<float> rc, bc;  // requested with the parts: one round trip
    chunk_load(rc, a.resid + o);
    chunk_load(bc, a.bias + 8u * c);
    for (uint32_t h0 = 0; h0 < a.nparts; h0 += 8u) {
      Chunk8<float> pc[8];
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) chunk_load(pc[u], a.part + (size_t)min(h0 + u, a.nparts - 1u) * a.part_stride + o);
      // every part's add is unconditional (+0 for the clamped reloads past nparts: sv starts at +0
      // and is never -0, so sv + 0 == sv): a conditional add let the compiler sink each load into
      // its branch and wait for the parts one at a time
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) {
        float pv[8];
        chunk_vals(pc[u], pv);
        const bool use = h0 + u < a.nparts;
#pragma unroll
        for (int j = 0; j < 8; ++j) sv[j] = sv[j] + (use ? pv[j] : 0.0f);
      }
    }
    float rv[8], bv[8], xv[8];
    chunk_vals(rc, rv);
    chunk_vals(bc, bv);
#pragma unroll
    for (int j = 0; j < 8; ++j) xv[j] = rv[j] + (sv[j] + bv[j]);
    *(float4 *)(xs + 8u * c) = make_float4(xv[0], xv[1], xv[2], xv[3]);
    *(float4 *)(xs + 8u * c + 4u) = make_float4(xv[4], xv[5], xv[6], xv[7]);
    if (c % G == g) store8(a.xout + o, xv);
  }
  __syncthreads();
  // 2. logit of expert e (every wave forms r: step 3 needs it)
  float acc[2] = {0.0f, 0.0f};  // dot, sum of squares
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    const uint32_t c0 = 512u * i + 8u * lane;
    if (c0 >= D) continue;
    float wv[8], x0[8];
    chunk_vals(wc[i], wv);
    const float4 lo = *(const float4 *)(xs + c0), hi = *(const float4 *)(xs + c0 + 4u);
    x0[0] = lo.x; x0[1] = lo.y; x0[2] = lo.z; x0[3] = lo.w; x0[4] = hi.x; x0[5] = hi.y; x0[6] = hi.z; x0[7] = hi.w;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc[0] = fmaf(x0[j], wv[j], acc[0]);
      acc[1] = fmaf(x0[j], x0[j], acc[1]);
    }
  }
  wave_sum_butterfly_n<2>(acc);
  const float r = f.apply_norm ? sqrtf(acc[1] / (float)D + f.eps) : 1.0f;
  if (lane == 0u && ev) f.logits[(size_t)t * E + e] = (f.apply_norm ? acc[0] / r : acc[0]) + f.rb[e];
  if (tid == 0u && g == 0u && f.rms) f.rms[t] = r;
  // 3. normalised row chunk c
  if (own) {
    float u[8];
    if (c < nc) {
      const float4 lo = *(const float4 *)(xs + 8u * c), hi = *(const float4 *)(xs + 8u * c + 4u);
      u[0] = lo.x; u[1] = lo.y; u[2] = lo.z; u[3] = lo.w; u[4] = hi.x; u[5] = hi.y; u[6] = hi.z; u[7] = hi.w;
      if (f.apply_norm) {
        const float ir = 1.0f / r;
        float gv[8];
        chunk_vals(gc, gv);
#pragma unroll
        for (int j = 0; j < 8; ++j) u[j] = (u[j] * ir) * gv[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) u[j] = 0.0f;
    }
    if (f.xn_bf16)
      store8((uint16_t *)f.xn + (size_t)t * f.Dp + 8u * c, u);
    else
      store8((float *)f.xn + (size_t)t * f.Dp + 8u * c, u);
  }
}

// Routing of one token (E <= kMaxExperts experts, K <= min(E, kMaxTopK)) inside a workgroup of at
// least K threads: wave 0 takes the top K by K wave-wide maxima of the packed keys (topk_key and
// wave_max_key, route_small_body's selection and order); then thread r < K places the expert of
// rank r at its active slot, the number of selected experts with a lower index (the dispatch's
// expert order, one token each), and writes that slot's record into lrec (LDS, [K][kRecWords]:
// expert, segment offset = slot, 1 token, token 0, slot r).  With wout (workgroup 0 of the launch)
// it also writes the routing outputs o: indices and softmax weights in rank order, segment offsets,
// active list, entry list and records.  Returns K.  Every thread of the workgroup must call it.
__device__ __forceinline__ uint32_t route_one_token(const float *lg, uint32_t E, uint32_t K, const RouteOut &o,
                                                    bool wout, int32_t *lrec) {
  __shared__ int32_t sel_l[kMaxTopK];
  __shared__ float selv_l[kMaxTopK];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  if (tid < 64u) {
    constexpr int J = (int)(kMaxExperts / 64u);
    float v[J];
    uint32_t kh[J], kl[J];
    bool taken[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t e = lane + 64u * (uint32_t)j;
      v[j] = e < E ? lg[e] : 0.0f;
      const uint64_t key = topk_key(v[j], e);
      kh[j] = (uint32_t)(key >> 32);
      kl[j] = (uint32_t)key;
      taken[j] = e >= E;
    }
    for (uint32_t r = 0; r < K; ++r) {
      uint32_t bh = 0u, bl = 0u;  // below every real key (the low word ~index is never 0)
#pragma unroll
      for (int j = 0; j < J; ++j)
        if (!taken[j] && (kh[j] > bh || (kh[j] == bh && kl[j] > bl))) {
          bh = kh[j];
          bl = kl[j];
        }
      wave_max_key(bh, bl);
#pragma unroll
      for (int j = 0; j < J; ++j)
        if (!taken[j] && kh[j] == bh && kl[j] == bl) {  // the one lane and chunk holding rank r
          taken[j] = true;
          sel_l[r] = (int32_t)(lane + 64u * (uint32_t)j);
          selv_l[r] = v[j];
        }
    }
  }
  __syncthreads();
  if (tid < K) {
    const int32_t e = sel_l[tid];
    int32_t pos = 0;
    for (uint32_t u = 0; u < K; ++u) pos += sel_l[u] < e ? 1 : 0;
    int32_t *rec = lrec + pos * (int32_t)kRecWords;
    rec[0] = e;
    rec[1] = pos;
    rec[2] = 1;
    rec[4] = 0;
    rec[4 + kRecTokens] = (int32_t)tid;
    if (wout) {
      o.topk_idx[tid] = e;
      o.topk_w[tid] = softmax_weight(selv_l, K, tid);
      o.active[pos] = e;
      o.perm[pos] = (int32_t)tid;
      o.pos_of[tid] = pos;
      int32_t *g = o.exrec + pos * (int32_t)kRecWords;
      g[0] = e;
      g[1] = pos;
      g[2] = 1;
      g[4] = 0;
      g[4 + kRecTokens] = (int32_t)tid;
    }
  }
  if (wout) {  // segment offsets: the selected experts below e; inactive slots
    for (uint32_t e = tid; e <= E; e += blockDim.x) {
      int32_t c = 0;
      for (uint32_t u = 0; u < K; ++u) c += (uint32_t)sel_l[u] < e ? 1 : 0;
      o.seg_off[e] = c;
      if (e >= K && e < E) o.active[e] = -1;
    }
    if (tid == 0) *o.num_active = (int32_t)K;
  }
  __syncthreads();
  return K;
}

// ---------------------------------------------------------------------------------------------
// Expert projection on MFMA.  Tiled MXFP4 layout of one expert (written by the layer upload):
//   row tile rt (16 rows) occupies nb*256 bytes; inside it K-group kg (4 blocks of 32 columns)
//   occupies 1024 bytes (tail group: 256 per block) where lane l = q*16 + i holds the 16 bytes
//   of row 16*rt + i, block 4*kg + q -- one coalesced 128-bit load per lane per K-group.
//   Scales: rt*nb*16 + kg*64 + l, one e8m0 byte per lane.
// MFMA v_mfma_f32_16x16x32_bf16, four steps s per K-group: lane (i, q) supplies A = 8 weights
// (dword s of its 16 bytes, dequantised exactly by v_cvt_scalef32_pk_bf16_fp4 with its block's
// scale) and B = the same 8 K positions of token j = lane & 15 from LDS.  The K positions of a
// step differ per lane group but are identical between A and B, so the product sums every
// (row, token, k) exactly once.  Output: lane holds C[rows 4q..4q+3][token j].
// f32 activations are split into NT bf16 terms: NT MFMAs per step, or (NT = 2 and at most 8 rows
// per token pass) one MFMA whose columns hold both terms -- column c reads B row c, term 1 of token
// j sits at row mt_max + j -- and the two columns of a token are summed once per tile.
// ---------------------------------------------------------------------------------------------

// a / b for a < 2^20 and b <= 2^12 given rb = 1.0f / b: the rounding error of (a + 0.5) * rb
// (< 2^-22 relative) is far below the distance 0.5 / b of (a + 0.5) / b from an integer.
__device__ __forceinline__ uint32_t div_small(uint32_t a, float rb) {
  return (uint32_t)(((float)a + 0.5f) * rb);
}


// Share of workgroup g of a grid of G among na active experts of nunits work units each: active
// slot ai = g mod na, as its p-th workgroup (p = g / na), owns the contiguous units
// [lo, lo + cnt).  The shares of a slot's workgroups are weighted by dispatch round r =
// min(g / num_cus, 3) (kRoundWeight, per projection): workgroups are placed on the CUs round by round, and the
// later ones share their CU with older ones that the memory system serves first.  32-bit
// arithmetic: nunits * (round-0 weight) * G < 2^32 (checked at launch).  Returns false when the
// workgroup has no units.
template <bool GATE_UP>
__device__ __forceinline__ bool gemv_share(uint32_t g, uint32_t G, uint32_t na, uint32_t nunits, uint32_t num_cus,
                                           uint32_t &ai, uint32_t &lo, uint32_t &cnt) {
  constexpr const uint32_t *wr = kRoundWeight[GATE_UP ? 0 : 1];
  if (na == 0u || na > G) return false;
  ai = g % na;
  const uint32_t p = g / na, nw = (G - 1u - ai) / na + 1u;  // part index, workgroups of slot ai
  uint32_t b[4];  // parts p' >= b[k] are in round >= k (p' * na + ai >= k * num_cus)
#pragma unroll
  for (uint32_t k = 1; k < 4; ++k) {
    const uint32_t kc = k * num_cus;
    b[k] = kc <= ai ? 0u : (kc - ai + na - 1u) / na;
  }
  auto wsum = [&](uint32_t x) {  // weights of parts 0 .. x-1
    int32_t w = (int32_t)(wr[0] * x);
#pragma unroll
    for (uint32_t k = 1; k < 4; ++k)
      if (x > b[k]) w += ((int32_t)wr[k] - (int32_t)wr[k - 1]) * (int32_t)(x - b[k]);
    return (uint32_t)w;
  };
  const uint32_t wt = wsum(nw);
  lo = nunits * wsum(p) / wt;
  cnt = nunits * wsum(p + 1u) / wt - lo;
  return cnt > 0u;
}

// Work split.  Grid of G workgroups (as many as stay resident); workgroup g owns the units
// gemv_share gives it (decode-sized batches) or a strided share (units part + wpe * i of slot
// g / wpe, larger batches), wave w every 4th of them from its w-th.  A unit is a row tile or (down with
// ksplit) one of ksplit fixed K-parts of a row tile (unit u: part u / nrt of row tile u mod nrt).
// gate_up in kGateUpSplit K-parts: the workgroup's units are row tiles and wave w takes K-part w of
// every one of them; at each tile's end the parts meet in LDS (one barrier), wave 0 sums them in
// part order (b1 in part 0) and writes the SwiGLU rows.
// Every workgroup stages its expert's B operand once per token pass (a pass = up to mt_max of the
// expert's routed tokens; one pass at decode sizes).  A workgroup learns num_active, its expert,
// segment and first tokens from one round trip (num_active plus the record table).
// Memory pipeline: waves stream their tiles in steps of kGemvKgPerWave K-groups held in one
// register buffer; each K-group slot is refilled with the next step's K-group (also across tile
// boundaries) right after its MFMAs, so kGemvKgPerWave - 1 K-groups stay in flight.  Everything
// a step consumes besides the weights (bias, B from LDS) is requested before that step's
// refills: loads complete in order, so waiting for those never waits for the prefetch.
// At start-up the B operand's staging loads are issued before the first weight loads for the same
// reason.  No branch surrounds a weight load.
template <int NT, bool GATE_UP, typename XT, int SPLIT, bool PK>
__global__ __launch_bounds__(kGemvThreads) __attribute__((amdgpu_waves_per_eu(3))) void expert_gemv_kernel(GemvArgs a) {
  static_assert(!PK || NT == 2, "packed columns hold two terms");
  static_assert(SPLIT >= 1 && (GATE_UP ? (SPLIT == 1 || SPLIT == (int)kGateUpSplit) : (SPLIT <= (int)kDownSplit || SPLIT == (int)kDownSplitFew)),
                "K-parts of the units");
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr uint32_t CJ = kGemvKgPerWave;
  const uint32_t Kp = a.nb * 32u, ldk = Kp + 8u;
  const uint32_t mtm = a.mt_max;
  uint16_t *bs = (uint16_t *)smem;
  int32_t *rec_l = (int32_t *)(smem + gemv_stage_bytes(NT, mtm, a.nb, a.nrec));  // [kRecWords]
  int32_t *tok_l = rec_l + kRecWords;                                             // [mtm]
  const uint32_t nrt = a.nrt;
  // work units: row tiles, or (down with ksplit) row tile u mod nrt, K-groups of part u / nrt
  constexpr uint32_t nsplit = (uint32_t)SPLIT;  // a.ksplit, fixed at compile time
  constexpr bool kInWg = GATE_UP && SPLIT > 1;    // K-parts of a row tile on the 4 waves of a workgroup
  static_assert(!kInWg || SPLIT == 4, "one K-part per wave");
  const uint32_t nunits = kInWg ? nrt : nrt * nsplit;
  // one round trip: num_active and the record table (the table is staged through the B area), or
  // (single-token gate_up) the token's logits, routed here into the same table
  uint32_t na;
  if (GATE_UP && a.route1_lg != nullptr) {
    const RouteOut ro = a.rout;
    na = route_one_token(a.route1_lg, a.route1_E, a.topk, ro, blockIdx.x == 0, (int32_t *)smem);
  } else {
    na = (uint32_t)*a.num_active;
    const uint4 *src = (const uint4 *)a.exrec;
    uint4 *dst = (uint4 *)smem;
    const uint32_t nv = a.nrec * (kRecWords / 4u);
    for (uint32_t i = threadIdx.x; i < nv; i += blockDim.x) dst[i] = src[i];
  }
  // this workgroup's units: lo + us * i, i < ntw (workgroup-uniform return when it has none)
  uint32_t ai = 0, lo = 0, ntw = 0, us = 1;
  if (a.weighted) {
    if (!gemv_share<GATE_UP>(blockIdx.x, gridDim.x, na, nunits, a.num_cus, ai, lo, ntw)) return;
  } else {
    // strided: workgroup g = ai * wpe + part owns units part, part + wpe, ... of slot ai, so an
    // expert's workgroups sweep its weights together (few pages hot at a time)
    if (na == 0u) return;
    const uint32_t wpe = max(1u, min(gridDim.x / na, nunits));
    ai = blockIdx.x / wpe;
    if (ai >= na) return;
    lo = blockIdx.x - ai * wpe;
    us = wpe;
    ntw = (nunits - lo + wpe - 1u) / wpe;
  }
  __syncthreads();
  const int32_t *rec0 = (const int32_t *)smem + ai * kRecWords;  // valid until the first staging
  if (threadIdx.x < kRecWords) rec_l[threadIdx.x] = rec0[threadIdx.x];
  const int e = rec0[0];
  const int seg0 = rec0[1];
  const int M = rec0[2];
  const uint32_t npass = (uint32_t)M <= mtm ? 1u : ((uint32_t)M + mtm - 1u) / mtm;

  const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
  const uint32_t i16 = lane & 15u, q = lane >> 4;
  const uint32_t nkg = (a.nb + 3u) >> 2;
  const uint32_t tail = a.nb - 4u * (nkg - 1u);
  const uint32_t H = (nkg + nsplit - 1u) / nsplit;  // K-groups per unit
  const uint32_t nst = (H + CJ - 1u) / CJ;           // steps per unit
  const uint8_t *wexp = a.wb + (size_t)e * a.wb_estride;
  const uint8_t *sexp = a.ws + (size_t)e * a.ws_estride;
  auto unit_h = [&](uint32_t u) { return nsplit == 1u ? 0u : (nsplit == 2u ? (u >= nrt ? 1u : 0u) : u / nrt); };
  auto unit_rt = [&](uint32_t u) { return u - unit_h(u) * nrt; };

  // K-group of slot j of step st; lanes outside the tile load the tile's first 16 bytes instead
  // (valid memory) and are neutralised at use (scale 1.0, zero B): no branch surrounds a load, so
  // partial vmcnt waits keep later loads in flight.
  auto kg_of = [&](uint32_t h, uint32_t st, uint32_t j) { return h * H + CJ * st + j; };
  auto lane_ok = [&](uint32_t h, uint32_t kg) {
    return kg < min(h * H + H, nkg) && q < (kg + 1u == nkg ? tail : 4u);
  };
  auto load_step = [&](uint32_t u, uint32_t st, uint4(&av)[CJ], uint32_t(&sv)[CJ]) {
    const uint32_t rt = unit_rt(u), h = unit_h(u);
    const uint8_t *wt = wexp + (size_t)rt * a.nb * 256u;
    const uint8_t *stp = sexp + (size_t)rt * a.nb * 16u;
#pragma unroll
    for (uint32_t j = 0; j < CJ; ++j) {
      const uint32_t kg = kg_of(h, st, j);
      const bool ok = lane_ok(h, kg);
      av[j] = load_stream16(wt + (ok ? kg * 1024u + lane * 16u : 0u));
      // the dword holding this lane's scale byte (byte lane & 3), kept raw until use: a byte load
      // would be re-extended at the loop back-edge, which waits for the prefetch to land
      sv[j] = *(const uint32_t *)(stp + (ok ? kg * 64u + (lane & ~3u) : 0u));
    }
  };
  const uint32_t sshift = 8u * (lane & 3u);
  // the dummy refills' offset into the expert's bias rows (rows_p >= 16 floats: in bounds)
  const uint32_t dummy_off = min(lane * 16u, a.bias_estride * 4u - 16u);

  // Staging of the B operand for token pass `pass_`: mt rows x Kp, NT bf16 terms, zero beyond the
  // true K.  Rows: gate_up the routed tokens' xn rows, down the segment's act rows (both
  // [*, Kp] in XT).  `first_loads` runs once, after the first batch's global loads are issued.
  uint32_t mt = 0, m0 = 0;
  const float rk8n = 1.0f / (float)(Kp >> 3);
  auto stage = [&](uint32_t pass_, auto &&first_loads) {
    m0 = pass_ * mtm;
    mt = min(mtm, (uint32_t)M - m0);
    if (threadIdx.x < mt) {
      // token t (gate_up) or slot t * topk + p (down) of segment entry jj: from the record for
      // the first kRecTokens entries (pass 0 reads the table copy in LDS, later passes rec_l),
      // else from the global segment list
      const uint32_t jj = m0 + threadIdx.x;
      const int32_t *rec = pass_ == 0 ? rec0 : rec_l;
      int32_t v;
      if (jj < kRecTokens) {
        v = rec[4 + (GATE_UP ? 0u : kRecTokens) + jj];
      } else {
        const int32_t slot = a.perm[seg0 + (int)jj];
        v = GATE_UP ? slot / (int32_t)a.topk : slot;
      }
      tok_l[threadIdx.x] = v;
    }
    __syncthreads();
    constexpr int SB = NT == 1 ? 3 : 2;
    const XT *src = (const XT *)a.brows;
    const uint32_t k8n = Kp >> 3, nitm = mt * k8n;
    bool first = true;
    for (uint32_t base = threadIdx.x; base < nitm; base += SB * blockDim.x) {
      Chunk8<XT> cx[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const uint32_t id = min(base + (uint32_t)u * blockDim.x, nitm - 1u);
        const uint32_t j = div_small(id, rk8n), kb = (id - j * k8n) * 8u;
        const size_t row = GATE_UP ? (size_t)tok_l[j] : (size_t)(seg0 + (int)(m0 + j));
        chunk_load(cx[u], src + row * Kp + kb);
      }
      if (first) first_loads();
      first = false;
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const uint32_t id = base + (uint32_t)u * blockDim.x;
        if (id >= nitm) continue;
        const uint32_t j = div_small(id, rk8n), kb = (id - j * k8n) * 8u;
        float v8[8];
        chunk_vals(cx[u], v8);
#pragma unroll
        for (int v = 0; v < 8; ++v) v8[v] = kb + (uint32_t)v < a.kt ? v8[v] : 0.0f;
        uint32_t pk[NT][4];
#pragma unroll
        for (int v = 0; v < 8; v += 2) {
          uint32_t tp[NT];
          split_bf16x2<NT>(v8[v], v8[v + 1], tp);
#pragma unroll
          for (int term = 0; term < NT; ++term) pk[term][v >> 1] = tp[term];
        }
#pragma unroll
        for (int term = 0; term < NT; ++term)
          *(uint4 *)(bs + ((size_t)term * mtm + j) * ldk + kb) = make_uint4(pk[term][0], pk[term][1], pk[term][2], pk[term][3]);
      }
    }
    if (first) first_loads();
    __syncthreads();
  };

  // this wave's units: lo + us * i for i = wv, wv + 4, ... < ntw (first unit clamped into the
  // expert for the start-up loads of a wave without units); in-workgroup K-parts: K-part wv of
  // row tiles lo + us * i, i < ntw (unit index rt + wv * nrt)
  const uint32_t my_first = kInWg ? lo + wv * nrt : lo + us * wv, tstride = kInWg ? us : 4u * us;
  const uint32_t my_tiles = kInWg ? ntw : (wv < ntw ? (ntw - wv + 3u) / 4u : 0u);
  const uint32_t first_c = kInWg ? my_first : min(my_first, nunits - 1u);
  float *red = (float *)(smem + gemv_red_offset(NT, mtm, a.nb, a.nrec));  // kInWg: [2][4][64][4]
  uint32_t parity = 0;
  const uint32_t total = my_tiles * nst;  // steps of this wave per token pass
  uint32_t ti = 0, st = 0, g = 0;         // tile ordinal, step in tile, step count
  uint4 abuf[CJ];
  uint32_t sbuf[CJ];
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};

  // One step: the CJ K-groups of the current step, each slot refilled with the same slot of the
  // next step as soon as its MFMAs have consumed it (so CJ - 1 K-groups stay in flight from one
  // register buffer); at the end of a tile, the epilogue.  Returns false when the wave's steps
  // are done.
  // PK: both activation terms in the columns of one MFMA (launched with 2 mt_max <= 16; columns
  // 2 mt_max .. 15 unused)
  auto do_step = [&]() -> bool {
    if (g >= total) return false;
    const uint32_t u = my_first + tstride * ti, rt = unit_rt(u), h = unit_h(u);
    // the bias of this lane's 4 epilogue rows, requested before this step's refills
    const f32x4_t bias4 = *(const f32x4_t *)(a.bias + (size_t)e * a.bias_estride + rt * 16u + 4u * q);
    // next step: next step of this tile, step 0 of the next tile, or (last step of the pass) a
    // dummy refill that keeps the load count static: 1 KiB of the expert's bias rows, which the
    // epilogues read, so these loads hit L2 (the weights stream with nontemporal loads)
    const bool more_st = st + 1u < nst;
    const bool more_t = ti + 1u < my_tiles;
    const bool last = !more_st && !more_t;
    const uint32_t nu = more_st ? u : (more_t ? u + tstride : u);
    const uint32_t nrt_ = unit_rt(nu), nh = unit_h(nu);
    const uint32_t nst_ = more_st ? st + 1u : (more_t ? 0u : st);
    const uint8_t *nwt = last ? (const uint8_t *)(a.bias + (size_t)e * a.bias_estride) : wexp + (size_t)nrt_ * a.nb * 256u;
    const uint8_t *nsp = sexp + (size_t)nrt_ * a.nb * 16u;
    const bool bval = i16 < mt;
    // B row of this lane's column: token i16, or (packed) term i16 / mt_max of token i16 % mt_max
    const uint32_t pcol = i16 < mtm ? i16 : i16 - mtm;
    const bool bcol = PK ? (i16 < 2u * mtm && pcol < mt) : bval;
    const uint16_t *brow = bs + (size_t)(PK ? min(i16, 2u * mtm - 1u) : min(i16, mtm - 1u)) * ldk;  // zeroed at use
    // few-expert batches (gate_up in K-parts: one or two tokens per expert) read B only in the lanes
    // of present tokens, an exec-masked read (120B T = 1 gate_up 17.7 -> 14.3 us); with more tokens
    // per expert the branches cost more than the skipped reads (20B T = 8 gate_up 37.8 -> 39.2 us)
    constexpr bool kMaskB = GATE_UP && SPLIT == (int)kGateUpSplit;
#pragma unroll
    for (uint32_t j = 0; j < CJ; ++j) {
      const uint32_t kg = kg_of(h, st, j);
      const bool ok = lane_ok(h, kg);
      const bool bok = bcol && ok;
      const float sc = ok ? e8m0_to_f32((sbuf[j] >> sshift) & 0xFFu) : 1.0f;
      const uint32_t kb = ok ? 32u * (4u * kg + q) : 0u;
      const uint32_t wd[4] = {abuf[j].x, abuf[j].y, abuf[j].z, abuf[j].w};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8_t A = fp4x8_to_bf16x8(wd[s], sc);
#pragma unroll
        for (int term = 0; term < (PK ? 1 : NT); ++term) {
          const uint16_t *bp = brow + (size_t)term * mtm * ldk + kb + 8u * s;
          u32x4_t raw = {0u, 0u, 0u, 0u};
          if constexpr (kMaskB) {
            if (bok) raw = *(const u32x4_t *)bp;  // lanes of absent tokens skip the LDS read
          } else {
            const u32x4_t r = *(const u32x4_t *)bp;
            raw = bok ? r : raw;
          }
          const bf16x8_t B = __builtin_bit_cast(bf16x8_t, raw);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, acc, 0, 0, 0);
        }
      }
      // refill slot j with the next step's K-group j
      {
        const uint32_t nkg_ = kg_of(nh, nst_, j);
        const bool nok = lane_ok(nh, nkg_);
        abuf[j] = load_stream16(nwt + (last ? dummy_off : (nok ? nkg_ * 1024u + lane * 16u : 0u)));
        sbuf[j] = *(const uint32_t *)(nsp + (nok ? nkg_ * 64u + (lane & ~3u) : 0u));
      }
      // keep each K-group's LDS reads, MFMAs and refill together (bounds the live registers)
      __builtin_amdgcn_sched_barrier(0);
    }
    ++g;
    if (++st < nst) return true;
    st = 0;
    if constexpr (PK) {  // token j's term-1 column (j + mt_max) onto its term-0 column
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = acc[r] + __shfl(acc[r], (int)(lane + mtm), 64);
    }
    // epilogue: lane holds rows 4q..4q+3 of tile rt for token column i16
    if constexpr (kInWg) {
      // every wave (a workgroup's waves walk the same tiles): part h's rows, b1 in part 0
      const f32x4_t b4 = h ? f32x4_t{0.0f, 0.0f, 0.0f, 0.0f} : bias4;
      float *rp = red + (size_t)parity * (4u * 64u * 4u);
      *(float4 *)(rp + (wv * 64u + lane) * 4u) = make_float4(acc[0] + b4[0], acc[1] + b4[1], acc[2] + b4[2], acc[3] + b4[3]);
      __syncthreads();
      if (wv == 0u && bval) {
        float v[4];
#pragma unroll
        for (uint32_t r = 0; r < 4u; ++r) v[r] = 0.0f;
#pragma unroll
        for (uint32_t hh = 0; hh < 4u; ++hh) {
          const float4 pp = *(const float4 *)(rp + (hh * 64u + lane) * 4u);
          v[0] = v[0] + pp.x;
          v[1] = v[1] + pp.y;
          v[2] = v[2] + pp.z;
          v[3] = v[3] + pp.w;
        }
        const int pos = seg0 + (int)(m0 + i16);
        const uint32_t f0 = (rt * 16u + 4u * q) >> 1;
        const float o0 = swiglu_clamp_f(v[0], v[1], a.alpha, a.limit);
        const float o1 = swiglu_clamp_f(v[2], v[3], a.alpha, a.limit);
        float *o = a.out + (size_t)pos * a.out_stride + f0;
        if (f0 + 1u < a.out_rows) {
          *(float2 *)o = make_float2(o0, o1);
        } else if (f0 < a.out_rows) {
          o[0] = o0;
        }
      }
      parity ^= 1u;  // the next tile's parts go to the other half (wave 0 may still read this one)
    } else if (bval) {
      const uint32_t r0 = rt * 16u + 4u * q;
      if constexpr (GATE_UP) {
        const int pos = seg0 + (int)(m0 + i16);
        const uint32_t f0 = r0 >> 1;
        const float o0 = swiglu_clamp_f(acc[0] + bias4[0], acc[1] + bias4[1], a.alpha, a.limit);
        const float o1 = swiglu_clamp_f(acc[2] + bias4[2], acc[3] + bias4[3], a.alpha, a.limit);
        float *o = a.out + (size_t)pos * a.out_stride + f0;
        if (f0 + 1u < a.out_rows) {
          *(float2 *)o = make_float2(o0, o1);
        } else if (f0 < a.out_rows) {
          o[0] = o0;
        }
      } else {
        // token-major slot row t * topk + p, expert bias b2 added once (K-part 0)
        float *o = a.out + h * a.out_half + (size_t)tok_l[i16] * a.out_stride + r0;
        const f32x4_t b4 = h ? f32x4_t{0.0f, 0.0f, 0.0f, 0.0f} : bias4;
        if (r0 + 3u < a.out_rows) {
          *(float4 *)o = make_float4(acc[0] + b4[0], acc[1] + b4[1], acc[2] + b4[2], acc[3] + b4[3]);
        } else {
          for (uint32_t r = 0; r < 4u; ++r)
            if (r0 + r < a.out_rows) o[r] = acc[r] + b4[r];
        }
      }
    }
    acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    return ++ti < my_tiles;
  };
  for (uint32_t pass = 0; pass < npass; ++pass) {
    // every wave (also one without tiles) reaches the staging barriers of every pass
    if (pass > 0) __syncthreads();  // all waves done with the previous pass's B
    stage(pass, [&] { load_step(first_c, 0u, abuf, sbuf); });
    ti = 0;
    st = 0;
    g = 0;
    while (do_step()) {
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Down projection + combine of a single-token batch (top-k K <= 4, the down K range in
// kDownSplitFew parts): workgroup r (one per 16-row tile of the D outputs) of 16 waves; wave w
// takes slot p = w / 4 (expert topk_idx[p], SwiGLU row pos_of[p]) and K-part h = w % 4 of tile r --
// the down GEMV's work unit, with its operand layout, K order, NT-term B rows (both terms in the
// columns of one MFMA) and bias in part 0 -- and leaves its 16 rows in LDS; threads 0..15 then
// add them as combine_kernel does (parts in order, slots ascending, acc + part sum x w_p, then
// x + acc): the same bits as the two launches, one launch fewer.  Waves of slots >= K take no
// unit.  The B rows are requested before the weights (loads complete in order).
// ---------------------------------------------------------------------------------------------
size_t down_combine1_lds_bytes(int nt, uint32_t nb) {
  return (size_t)kDownComb1MaxK * (size_t)nt * (nb * 32u + 8u) * 2u + kDownComb1MaxK * kDownSplitFew * 16u * 4u;
}

template <int NT, typename XT>
__global__ __launch_bounds__(1024) void down_combine1_kernel(DownComb1Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr uint32_t CJ = kGemvKgPerWave;
  const uint32_t Kp = a.nb * 32u, ldk = Kp + 8u, K = a.K;
  uint16_t *bs = (uint16_t *)smem;  // [slot][term][ldk]
  float *red = (float *)(smem + (size_t)kDownComb1MaxK * NT * ldk * 2u);  // [slot][part][16]
  const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
  const uint32_t p = wv >> 2, h = wv & 3u, rt = blockIdx.x;
  const bool live = p < K;  // wave-uniform
  const uint32_t i16 = lane & 15u, q = lane >> 4;
  const uint32_t nkg = (a.nb + 3u) >> 2, tail = a.nb - 4u * (nkg - 1u);
  const uint32_t H = (nkg + kDownSplitFew - 1u) / kDownSplitFew;  // the down GEMV's parts
  const uint32_t kg0 = min(h * H, nkg), kg1 = min(kg0 + H, nkg);
  // B staging: chunk c = thread + 1024 u of slot c / k8n, inputs 8 (c % k8n) ..
  const uint32_t k8n = Kp >> 3, nitm = K * k8n;
  constexpr uint32_t SB = (kDownComb1MaxK * kDownComb1MaxKp / 8u + 1023u) / 1024u;  // chunks per thread
  int32_t pos[SB];
#pragma unroll
  for (uint32_t u = 0; u < SB; ++u) {
    const uint32_t id = min(threadIdx.x + u * 1024u, nitm - 1u);
    pos[u] = a.pos_of[id / k8n];
  }
  const int32_t e = a.topk_idx[live ? p : 0u];
  Chunk8<float> cx[SB];
#pragma unroll
  for (uint32_t u = 0; u < SB; ++u) {
    const uint32_t id = min(threadIdx.x + u * 1024u, nitm - 1u), j = id / k8n, kb = (id - j * k8n) * 8u;
    chunk_load(cx[u], a.act + (size_t)pos[u] * a.act_stride + kb);
  }
  const uint8_t *wt = a.wb + (size_t)e * a.wb_estride + (size_t)rt * a.nb * 256u;
  const uint8_t *stp = a.ws + (size_t)e * a.ws_estride + (size_t)rt * a.nb * 16u;
  auto lane_ok = [&](uint32_t kg) { return kg < kg1 && q < (kg + 1u == nkg ? tail : 4u); };
  uint4 abuf[CJ];
  uint32_t sbuf[CJ];
#pragma unroll
  for (uint32_t j = 0; j < CJ; ++j) {
    const uint32_t kg = kg0 + j;
    const bool ok = lane_ok(kg);
    abuf[j] = load_stream16(wt + (ok ? kg * 1024u + lane * 16u : 0u));
    sbuf[j] = *(const uint32_t *)(stp + (ok ? kg * 64u + (lane & ~3u) : 0u));
  }
#pragma unroll
  for (uint32_t u = 0; u < SB; ++u) {
    const uint32_t id = threadIdx.x + u * 1024u;
    if (id >= nitm) continue;
    const uint32_t j = id / k8n, kb = (id - j * k8n) * 8u;
    float v8[8];
    chunk_vals(cx[u], v8);
#pragma unroll
    for (int v = 0; v < 8; ++v) v8[v] = kb + (uint32_t)v < a.kt ? v8[v] : 0.0f;
    uint32_t pk[NT][4];
#pragma unroll
    for (int v = 0; v < 8; v += 2) {
      uint32_t tp[NT];
      split_bf16x2<NT>(v8[v], v8[v + 1], tp);
#pragma unroll
      for (int term = 0; term < NT; ++term) pk[term][v >> 1] = tp[term];
    }
#pragma unroll
    for (int term = 0; term < NT; ++term)
      *(uint4 *)(bs + ((size_t)j * NT + term) * ldk + kb) = make_uint4(pk[term][0], pk[term][1], pk[term][2], pk[term][3]);
  }
  __syncthreads();
  if (live) {
    // B column i16: term i16 of this slot's row (columns >= NT zero)
    const bool bcol = i16 < (uint32_t)NT;
    const uint16_t *brow = bs + ((size_t)p * NT + min(i16, (uint32_t)NT - 1u)) * ldk;
    const uint32_t sshift = 8u * (lane & 3u);
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t s0 = kg0; s0 < kg1; s0 += CJ) {
#pragma unroll
      for (uint32_t j = 0; j < CJ; ++j) {
        const uint32_t kg = s0 + j;
        const bool ok = lane_ok(kg);
        const bool bok = bcol && ok;
        const float sc = ok ? e8m0_to_f32((sbuf[j] >> sshift) & 0xFFu) : 1.0f;
        const uint32_t kb = ok ? 32u * (4u * kg + q) : 0u;
        const uint32_t wd[4] = {abuf[j].x, abuf[j].y, abuf[j].z, abuf[j].w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bf16x8_t A = fp4x8_to_bf16x8(wd[s], sc);
          const u32x4_t r = *(const u32x4_t *)(brow + kb + 8u * s);
          const u32x4_t zero = {0u, 0u, 0u, 0u};
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8_t, bok ? r : zero), acc, 0, 0, 0);
        }
        // next step's K-group j (a part longer than CJ K-groups; else the tile's first block again)
        const uint32_t nkg_ = kg + CJ;
        const bool nok = lane_ok(nkg_);
        abuf[j] = load_stream16(wt + (nok ? nkg_ * 1024u + lane * 16u : 0u));
        sbuf[j] = *(const uint32_t *)(stp + (nok ? nkg_ * 64u + (lane & ~3u) : 0u));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (NT == 2) {  // the lo term's column 1 onto column 0
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = acc[r] + __shfl(acc[r], (int)(lane + 1u), 64);
    }
    if (i16 == 0u) {
      const uint32_t r0 = rt * 16u + 4u * q;
      const f32x4_t b4 = h ? f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}
                           : *(const f32x4_t *)(a.bias + (size_t)e * a.bias_estride + r0);
      *(float4 *)(red + (p * kDownSplitFew + h) * 16u + 4u * q) =
          make_float4(acc[0] + b4[0], acc[1] + b4[1], acc[2] + b4[2], acc[3] + b4[3]);
    }
  }
  __syncthreads();
  if (threadIdx.x < 16u) {
    const uint32_t row = rt * 16u + threadIdx.x;
    if (row < a.D) {
      float acc = 0.0f;
      for (uint32_t pp = 0; pp < K; ++pp) {
        const float *rp = red + pp * kDownSplitFew * 16u + threadIdx.x;
        float v = rp[0];
#pragma unroll
        for (uint32_t hh = 1; hh < kDownSplitFew; ++hh) v = v + rp[hh * 16u];
        acc = acc + v * a.topk_w[pp];
      }
      const XT *x = (const XT *)a.x;
      XT *y = (XT *)a.y;
      float xv = 0.0f;
      if (a.add_residual) {
        if constexpr (sizeof(XT) == 2) xv = bf16_bits_to_f32(x[row]);
        else xv = x[row];
      }
      if constexpr (sizeof(XT) == 2) {
        y[row] = f32_to_bf16_bits(xv + acc);
      } else {
        y[row] = xv + acc;
      }
    }
  }
}

hipError_t launch_down_combine1(const DownComb1Args &a, int nt, bool x_bf16, hipStream_t s) {
  if (a.K == 0u || a.K > kDownComb1MaxK || a.nb * 32u > kDownComb1MaxKp || a.D == 0u || a.nrt * 16u < a.D)
    return hipErrorInvalidValue;
  const size_t lds = down_combine1_lds_bytes(nt, a.nb);
  const dim3 grid((a.D + 15u) / 16u), block(1024);
  if (nt == 1) {
    return x_bf16 ? launch_kernel(down_combine1_kernel<1, uint16_t>, grid, block, lds, s, a)
                  : launch_kernel(down_combine1_kernel<1, float>, grid, block, lds, s, a);
  }
  if (nt == 2 && !x_bf16) return launch_kernel(down_combine1_kernel<2, float>, grid, block, lds, s, a);
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------------------
// Combine: y[t, d] = (add_residual ? x[t, d] : 0) + sum_{p asc} yslot[t*K + p, d] * w_p, where the
// down projection already wrote yslot = down_p + b2[e_p] token-major (f32, in NP K-parts, or bf16
// when PB).  Every load of a thread is independent of the others (one memory round trip); four
// outputs per thread.
// ---------------------------------------------------------------------------------------------
template <typename XT, int NP, bool PB>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
  static_assert(!PB || NP == 1, "bf16 slot rows come in one part");
  const uint32_t t = blockIdx.y;
  const uint32_t d0 = (blockIdx.x * blockDim.x + threadIdx.x) * 4u;
  if (d0 >= a.D) return;
  const uint32_t nv = min(4u, a.D - d0);
  const XT *x = (const XT *)a.x;
  // four whole values (D % 4 == 0, 16-byte aligned x and y): one 8- or 16-byte access for x and y
  const bool vec = nv == 4u && (a.D & 3u) == 0u && (((uintptr_t)a.x | (uintptr_t)a.y) & 15u) == 0u;
  float xv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (a.add_residual && vec) {
    const XT *xp = x + (size_t)t * a.D + d0;
    if constexpr (sizeof(XT) == 2) {
      const uint2 r = *(const uint2 *)xp;
      xv[0] = bf16_bits_to_f32((uint16_t)r.x);
      xv[1] = bf16_bits_to_f32((uint16_t)(r.x >> 16));
      xv[2] = bf16_bits_to_f32((uint16_t)r.y);
      xv[3] = bf16_bits_to_f32((uint16_t)(r.y >> 16));
    } else {
      const float4 r = *(const float4 *)xp;
      xv[0] = r.x;
      xv[1] = r.y;
      xv[2] = r.z;
      xv[3] = r.w;
    }
  } else if (a.add_residual) {
#pragma unroll
    for (uint32_t j = 0; j < 4u; ++j) xv[j] = j < nv ? load_val(x, (size_t)t * a.D + d0 + j) : 0.0f;
  }
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t p0 = 0; p0 < a.K; p0 += 8u) {
    float wv[8];
    float4 yv[8], yh[NP > 1 ? NP - 1 : 1][8];
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      const uint32_t p = min(p0 + u, a.K - 1u);
      wv[u] = a.topk_w[(size_t)t * a.K + p];
      const size_t row = ((size_t)t * a.K + p) * a.Dp + d0;  // Dp % 4 == 0, d0 < Dp
      if constexpr (PB) {
        const uint2 r = *(const uint2 *)((const uint16_t *)a.ypart + row);
        yv[u] = make_float4(bf16_bits_to_f32((uint16_t)r.x), bf16_bits_to_f32((uint16_t)(r.x >> 16)),
                            bf16_bits_to_f32((uint16_t)r.y), bf16_bits_to_f32((uint16_t)(r.y >> 16)));
      } else {
        yv[u] = *(const float4 *)((const float *)a.ypart + row);
      }
#pragma unroll
      for (int h = 1; h < NP; ++h) yh[h - 1][u] = *(const float4 *)((const float *)a.ypart + h * a.part_stride + row);
    }
#pragma unroll
    for (int h = 1; h < NP; ++h)
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u)
        yv[u] = make_float4(yv[u].x + yh[h - 1][u].x, yv[u].y + yh[h - 1][u].y, yv[u].z + yh[h - 1][u].z, yv[u].w + yh[h - 1][u].w);
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      if (p0 + u >= a.K) break;
      acc[0] = acc[0] + yv[u].x * wv[u];
      acc[1] = acc[1] + yv[u].y * wv[u];
      acc[2] = acc[2] + yv[u].z * wv[u];
      acc[3] = acc[3] + yv[u].w * wv[u];
    }
  }
  XT *y = (XT *)a.y;
  if (vec) {
    XT *yp = y + (size_t)t * a.D + d0;
    if constexpr (sizeof(XT) == 2) {
      *(uint2 *)yp = make_uint2((uint32_t)f32_to_bf16_bits(xv[0] + acc[0]) | ((uint32_t)f32_to_bf16_bits(xv[1] + acc[1]) << 16),
                                (uint32_t)f32_to_bf16_bits(xv[2] + acc[2]) | ((uint32_t)f32_to_bf16_bits(xv[3] + acc[3]) << 16));
    } else {
      *(float4 *)yp = make_float4(xv[0] + acc[0], xv[1] + acc[1], xv[2] + acc[2], xv[3] + acc[3]);
    }
  } else {
    for (uint32_t j = 0; j < nv; ++j) store_val(y, (size_t)t * a.D + d0 + j, xv[j] + acc[j]);
  }
}

// ---------------------------------------------------------------------------------------------
// Combine followed by the RmsNorm of its output (a decoder's next norm, one launch instead of
// two): f32 x, y and nout, f32 slot rows in NP K-parts, D % 4 == 0, D <= 4096, 16-byte aligned
// rows.  One workgroup of 256 threads per token row; thread i computes output quads q = i + 256 r
// with combine_kernel's arithmetic (parts summed in order, slots p ascending), keeps them in
// registers and normalises the row: sum of squares over r then x, y, z, w (zeros past the row),
// wave butterfly, (w0 + w1) + (w2 + w3); nout = (y / sqrt(sum / D + eps)) * gamma.  The quads of
// all slots of a pass (4 slots, 2 with 4 K-parts) are requested together: one memory round trip
// per pass.
// ---------------------------------------------------------------------------------------------
template <int NP>
__global__ __launch_bounds__(256) void combine_norm_kernel(CombineArgs a) {
  constexpr uint32_t kR = 4, kP = NP >= 4 ? 2 : 4;  // slots per pass (register budget)
  __shared__ float red[4];
  const uint32_t t = blockIdx.x, tid = threadIdx.x, nq = a.D / 4u;
  const float4 *x4 = (const float4 *)((const float *)a.x + (size_t)t * a.D);
  const float4 *g4 = (const float4 *)a.ngamma;
  const float *yp = (const float *)a.ypart;
  float4 xv[kR], gv[kR];
#pragma unroll
  for (uint32_t r = 0; r < kR; ++r) {
    const uint32_t q = min(tid + 256u * r, nq - 1u);  // clamped: quads past the row reload a valid one
    xv[r] = a.add_residual ? x4[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    gv[r] = g4[q];
  }
  float acc[kR][4];
#pragma unroll
  for (uint32_t r = 0; r < kR; ++r) acc[r][0] = acc[r][1] = acc[r][2] = acc[r][3] = 0.0f;
  for (uint32_t p0 = 0; p0 < a.K; p0 += kP) {
    float wv[kP];
    float4 yv[kR][kP], yh[NP > 1 ? NP - 1 : 1][kR][kP];
#pragma unroll
    for (uint32_t u = 0; u < kP; ++u) {
      const uint32_t p = min(p0 + u, a.K - 1u);
      wv[u] = a.topk_w[(size_t)t * a.K + p];
#pragma unroll
      for (uint32_t r = 0; r < kR; ++r) {
        const size_t row = ((size_t)t * a.K + p) * a.Dp + 4u * min(tid + 256u * r, nq - 1u);
        yv[r][u] = *(const float4 *)(yp + row);
#pragma unroll
        for (int h = 1; h < NP; ++h) yh[h - 1][r][u] = *(const float4 *)(yp + h * a.part_stride + row);
      }
    }
    // every request of the pass is out before the sums consume any (the scheduler otherwise
    // interleaves them slot by slot, one memory round trip per slot)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int h = 1; h < NP; ++h)
#pragma unroll
      for (uint32_t r = 0; r < kR; ++r)
#pragma unroll
        for (uint32_t u = 0; u < kP; ++u)
          yv[r][u] = make_float4(yv[r][u].x + yh[h - 1][r][u].x, yv[r][u].y + yh[h - 1][r][u].y,
                                 yv[r][u].z + yh[h - 1][r][u].z, yv[r][u].w + yh[h - 1][r][u].w);
#pragma unroll
    for (uint32_t u = 0; u < kP; ++u) {
      if (p0 + u >= a.K) break;
#pragma unroll
      for (uint32_t r = 0; r < kR; ++r) {
        acc[r][0] = acc[r][0] + yv[r][u].x * wv[u];
        acc[r][1] = acc[r][1] + yv[r][u].y * wv[u];
        acc[r][2] = acc[r][2] + yv[r][u].z * wv[u];
        acc[r][3] = acc[r][3] + yv[r][u].w * wv[u];
      }
    }
  }
  float4 *y4 = (float4 *)((float *)a.y + (size_t)t * a.D);
  float4 v[kR];
  float ss = 0.0f;
#pragma unroll
  for (uint32_t r = 0; r < kR; ++r) {
    const uint32_t q = tid + 256u * r;
    v[r] = q < nq ? make_float4(xv[r].x + acc[r][0], xv[r].y + acc[r][1], xv[r].z + acc[r][2], xv[r].w + acc[r][3])
                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (q < nq) y4[q] = v[r];
  }
#pragma unroll
  for (uint32_t r = 0; r < kR; ++r) {
    ss = fmaf(v[r].x, v[r].x, ss);
    ss = fmaf(v[r].y, v[r].y, ss);
    ss = fmaf(v[r].z, v[r].z, ss);
    ss = fmaf(v[r].w, v[r].w, ss);
  }
  ss = wave_sum_butterfly(ss);
  if ((tid & 63u) == 0u) red[tid >> 6] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float rr = sqrtf(tot / (float)a.D + a.neps);
  float4 *n4 = (float4 *)(a.nout + (size_t)t * a.D);
#pragma unroll
  for (uint32_t r = 0; r < kR; ++r) {
    const uint32_t q = tid + 256u * r;
    if (q < nq)
      n4[q] = make_float4((v[r].x / rr) * gv[r].x, (v[r].y / rr) * gv[r].y, (v[r].z / rr) * gv[r].z,
                          (v[r].w / rr) * gv[r].w);
  }
}

// ---------------------------------------------------------------------------------------------
// Dequant hook: one thread per packed byte.  f32 output uses the bit-built LUT value times the
// bit-built 2^(s-127); bf16 output uses the same v_cvt_scalef32_pk_bf16_fp4 conversion as the
// expert projections, so the exhaustive test of this hook covers their dequantisation.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dequant_kernel(DequantArgs a) {
  const uint64_t total = a.rows * a.bpr;
  for (uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total;
       id += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t r = id / a.bpr, b = id % a.bpr;
    const uint64_t c = 2u * b;
    const uint32_t byte = a.blocks[id];
    const uint32_t s = ((uint32_t)a.scales[r * a.gpr + (c >> 5)] - (uint32_t)a.ue8_offset) & 255u;
    const float sc = e8m0_to_f32(s);
    if (a.out_bf16) {
      const uint32_t v = fp4x2_to_bf16x2_bits<0>(byte, sc);
      uint16_t *o = (uint16_t *)a.out + r * a.cols + c;
      o[0] = (uint16_t)(v & 0xFFFFu);
      if (c + 1 < a.cols) o[1] = (uint16_t)(v >> 16);
    } else {
      float *o = (float *)a.out + r * a.cols + c;
      o[0] = fp4_to_f32(byte & 15u) * sc;
      if (c + 1 < a.cols) o[1] = fp4_to_f32(byte >> 4) * sc;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------------
hipError_t configure_kernels() {
  const int big = 160 * 1024;
  hipError_t err = hipSuccess;
// (the dynamic limit is what the CU's LDS leaves beside the kernel's static LDS)
#define BX_ATTR(f)                                                                                                  \
  do {                                                                                                               \
    hipFuncAttributes fa_{};                                                                                         \
    hipError_t e_ = hipFuncGetAttributes(&fa_, (const void *)(f));                                                   \
    if (e_ == hipSuccess)                                                                                            \
      e_ = hipFuncSetAttribute((const void *)(f), hipFuncAttributeMaxDynamicSharedMemorySize,                        \
                               big - (int)fa_.sharedSizeBytes);                                                      \
    if (e_ != hipSuccess && err == hipSuccess) err = e_;                                                             \
  } while (0)
  BX_ATTR((down_combine1_kernel<1, uint16_t>));
  BX_ATTR((down_combine1_kernel<1, float>));
  BX_ATTR((down_combine1_kernel<2, float>));
  BX_ATTR((router_kernel<float, float, true>));
  BX_ATTR((router_kernel<float, uint16_t, true>));
  BX_ATTR((router_kernel<uint16_t, float, true>));
  BX_ATTR((router_kernel<uint16_t, uint16_t, true>));
  BX_ATTR((router_kernel<float, float, false>));
  BX_ATTR((router_kernel<float, uint16_t, false>));
  BX_ATTR((router_kernel<uint16_t, float, false>));
  BX_ATTR((router_kernel<uint16_t, uint16_t, false>));
  BX_ATTR((router_rows_kernel<float, float, 2>));
  BX_ATTR((router_rows_kernel<float, float, 4>));
  BX_ATTR((router_rows_kernel<float, uint16_t, 2>));
  BX_ATTR((router_rows_kernel<float, uint16_t, 4>));
  BX_ATTR((router_rows_kernel<uint16_t, float, 2>));
  BX_ATTR((router_rows_kernel<uint16_t, float, 4>));
  BX_ATTR((router_rows_kernel<uint16_t, uint16_t, 2>));
  BX_ATTR((router_rows_kernel<uint16_t, uint16_t, 4>));
  BX_ATTR(dispatch_kernel);
  BX_ATTR((expert_gemv_kernel<1, true, uint16_t, 1, false>));
  BX_ATTR((expert_gemv_kernel<1, true, float, 1, false>));
  BX_ATTR((expert_gemv_kernel<1, true, uint16_t, kGateUpSplit, false>));
  BX_ATTR((expert_gemv_kernel<1, true, float, kGateUpSplit, false>));
  BX_ATTR((expert_gemv_kernel<1, false, float, 1, false>));
  BX_ATTR((expert_gemv_kernel<1, false, float, kDownSplit, false>));
  BX_ATTR((expert_gemv_kernel<1, false, float, kDownSplitFew, false>));
  BX_ATTR((expert_gemv_kernel<2, true, uint16_t, 1, false>));
  BX_ATTR((expert_gemv_kernel<2, true, float, 1, false>));
  BX_ATTR((expert_gemv_kernel<2, true, uint16_t, kGateUpSplit, false>));
  BX_ATTR((expert_gemv_kernel<2, true, float, kGateUpSplit, false>));
  BX_ATTR((expert_gemv_kernel<2, false, float, 1, false>));
  BX_ATTR((expert_gemv_kernel<2, false, float, kDownSplit, false>));
  BX_ATTR((expert_gemv_kernel<2, false, float, kDownSplitFew, false>));
  BX_ATTR((expert_gemv_kernel<2, true, uint16_t, 1, true>));
  BX_ATTR((expert_gemv_kernel<2, true, float, 1, true>));
  BX_ATTR((expert_gemv_kernel<2, true, uint16_t, kGateUpSplit, true>));
  BX_ATTR((expert_gemv_kernel<2, true, float, kGateUpSplit, true>));
  BX_ATTR((expert_gemv_kernel<2, false, float, 1, true>));
  BX_ATTR((expert_gemv_kernel<2, false, float, kDownSplit, true>));
  BX_ATTR((expert_gemv_kernel<2, false, float, kDownSplitFew, true>));
#undef BX_ATTR
  return err;
}

template <typename XT, typename WT>
static void router_launch(const RouterArgs &a, bool vec, dim3 grid, size_t lds, hipStream_t s) {
  if (vec)
    (void)launch_kernel(router_kernel<XT, WT, true>, grid, dim3(kRouterThreads), lds, s, a);
  else
    (void)launch_kernel(router_kernel<XT, WT, false>, grid, dim3(kRouterThreads), lds, s, a);
}

template <typename XT, typename WT>
static void rows_launch(const RouterArgs &a, int tokens_per_wave, dim3 grid, dim3 block, size_t lds, hipStream_t s) {
  if (tokens_per_wave == 4)
    (void)launch_kernel(router_rows_kernel<XT, WT, 4>, grid, block, lds, s, a);
  else
    (void)launch_kernel(router_rows_kernel<XT, WT, 2>, grid, block, lds, s, a);
}

hipError_t launch_router_rows(const RouterArgs &a, bool x_bf16, bool w_bf16, int tokens_per_wave, hipStream_t s) {
  if (tokens_per_wave != 2 && tokens_per_wave != 4) return hipErrorInvalidValue;
  if (a.D % 8u != 0 || a.D > kRowsSpan || (a.xn && a.Dp > kRowsSpan) || (a.xq.hi && a.xq.kq > kRowsSpan))
    return hipErrorInvalidValue;
  const uint32_t tpb = (uint32_t)tokens_per_wave * (kRowsThreads / 64u);
  const dim3 grid((a.n + tpb - 1) / tpb), block(kRowsThreads);
  const size_t lds = router_rows_lds_bytes();
  if (x_bf16 && w_bf16)
    rows_launch<uint16_t, uint16_t>(a, tokens_per_wave, grid, block, lds, s);
  else if (x_bf16)
    rows_launch<uint16_t, float>(a, tokens_per_wave, grid, block, lds, s);
  else if (w_bf16)
    rows_launch<float, uint16_t>(a, tokens_per_wave, grid, block, lds, s);
  else
    rows_launch<float, float>(a, tokens_per_wave, grid, block, lds, s);
  return hipGetLastError();
}

hipError_t launch_router(const RouterArgs &a, bool x_bf16, bool w_bf16, bool vec, hipStream_t s) {
  const dim3 grid((a.n + a.tb - 1) / a.tb, (a.E + 4 * a.epw - 1) / (4 * a.epw));
  const size_t lds = router_lds_bytes(a.tb, a.Dpad);
  if (x_bf16) {
    if (w_bf16)
      router_launch<uint16_t, uint16_t>(a, vec, grid, lds, s);
    else
      router_launch<uint16_t, float>(a, vec, grid, lds, s);
  } else {
    if (w_bf16)
      router_launch<float, uint16_t>(a, vec, grid, lds, s);
    else
      router_launch<float, float>(a, vec, grid, lds, s);
  }
  return hipGetLastError();
}

hipError_t launch_small_route(const SmallRouteArgs &a, hipStream_t s) {
  if (a.n == 0 || a.n > kSmallRouteMaxTokens || a.E > kMaxExperts || a.K > kMaxTopK) return hipErrorInvalidValue;
  // at least 8 waves: the work-map writes spread over the whole workgroup
  const dim3 block(64 * max(a.n, 8u));
  if (a.E <= 64)
    (void)launch_kernel(small_route_kernel<1>, dim3(1), block, 0, s, a);
  else if (a.E <= 128)
    (void)launch_kernel(small_route_kernel<2>, dim3(1), block, 0, s, a);
  else
    (void)launch_kernel(small_route_kernel<4>, dim3(1), block, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_router_front(const PreFrontArgs &a, bool w_bf16, hipStream_t s) {
  const FrontArgs &f = a.f;
  if (f.n == 0 || f.n > kSmallRouteMaxTokens || f.D % 8u != 0 || f.D > 512u * kFrontChunks || f.Dp > 512u * kFrontChunks ||
      f.Dp % 8u != 0 || f.E == 0 || f.E > kMaxExperts || !f.logits || f.x != a.xout || a.nparts == 0 ||
      a.nparts > kFrontMaxParts || !a.part || !a.bias || !a.resid || !a.xout ||
      (((uintptr_t)a.part | (uintptr_t)a.bias | (uintptr_t)a.resid | (uintptr_t)a.xout | (uintptr_t)f.rw |
        (uintptr_t)f.gamma | (uintptr_t)f.xn) & 15u) || (a.part_stride & 3u))
    return hipErrorInvalidValue;
  const dim3 g(f.n, (f.E + 7u) / 8u), b(512);
  if (w_bf16)
    (void)launch_kernel(router_front_kernel<uint16_t>, g, b, 0, s, a);
  else
    (void)launch_kernel(router_front_kernel<float>, g, b, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_router_small(const FrontArgs &a, bool x_bf16, bool w_bf16, hipStream_t s) {
  if (a.n == 0 || a.n > kSmallRouteMaxTokens || a.D % 8u != 0 || a.D > 512u * kFrontChunks || !a.logits)
    return hipErrorInvalidValue;
  const dim3 g(a.E), b(64 * ((a.n + 1) / 2));
  if (x_bf16 && w_bf16)
    (void)launch_kernel(router_small_kernel<uint16_t, uint16_t>, g, b, 0, s, a);
  else if (x_bf16)
    (void)launch_kernel(router_small_kernel<uint16_t, float>, g, b, 0, s, a);
  else if (w_bf16)
    (void)launch_kernel(router_small_kernel<float, uint16_t>, g, b, 0, s, a);
  else
    (void)launch_kernel(router_small_kernel<float, float>, g, b, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_topk(const TopkArgs &a, hipStream_t s) {
  if (a.E == 0 || a.E > kMaxExperts || a.K == 0 || a.K > kMaxTopK || a.K > a.E) return hipErrorInvalidValue;
  const uint32_t wpb = kTopkThreads / 64;
  const dim3 grid((a.n + wpb - 1) / wpb), block(kTopkThreads);
  if (a.E <= 64)
    (void)launch_kernel(topk_kernel<1>, grid, block, 0, s, a);
  else if (a.E <= 128)
    (void)launch_kernel(topk_kernel<2>, grid, block, 0, s, a);
  else
    (void)launch_kernel(topk_kernel<4>, grid, block, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_dispatch(const DispatchArgs &a, hipStream_t s) {
  if (a.n >= kDispatchWideMinTokens) {
    if (!a.chunk_cnt) return hipErrorInvalidValue;
    const dim3 grid((a.n + kDispatchChunk - 1) / kDispatchChunk), block(kDispatchChunk);
    (void)launch_kernel(dispatch_count_kernel, grid, block, 0, s, a);
    (void)launch_kernel(dispatch_wide_kernel, grid, block, 0, s, a);
  } else {
    (void)launch_kernel(dispatch_kernel, dim3(1), dim3(kDispatchThreads), dispatch_lds_bytes(a.E, kDispatchThreads), s, a);
  }
  return hipGetLastError();
}

template <int NT, bool PK>
static void launch_gemv_t(const GemvArgs &a, bool gate_up, bool x_bf16, dim3 g, size_t lds, hipStream_t s) {
  const dim3 block(kGemvThreads);
  const bool split = !gate_up && a.ksplit > 1u;
  const bool usplit = gate_up && a.ksplit > 1u;
  if (split && a.ksplit == kDownSplitFew)
    (void)launch_kernel(expert_gemv_kernel<NT, false, float, kDownSplitFew, PK>, g, block, lds, s, a);
  else if (split)
    (void)launch_kernel(expert_gemv_kernel<NT, false, float, kDownSplit, PK>, g, block, lds, s, a);
  else if (!gate_up)
    (void)launch_kernel(expert_gemv_kernel<NT, false, float, 1, PK>, g, block, lds, s, a);
  else if (usplit && x_bf16)
    (void)launch_kernel(expert_gemv_kernel<NT, true, uint16_t, kGateUpSplit, PK>, g, block, lds, s, a);
  else if (usplit)
    (void)launch_kernel(expert_gemv_kernel<NT, true, float, kGateUpSplit, PK>, g, block, lds, s, a);
  else if (x_bf16)
    (void)launch_kernel(expert_gemv_kernel<NT, true, uint16_t, 1, PK>, g, block, lds, s, a);
  else
    (void)launch_kernel(expert_gemv_kernel<NT, true, float, 1, PK>, g, block, lds, s, a);
}

hipError_t launch_gemv(const GemvArgs &a, int nt, bool gate_up, bool x_bf16, uint32_t grid, hipStream_t s) {
  const uint64_t nunits = (uint64_t)a.nrt * (a.ksplit > 1u ? a.ksplit : 1u);
  if (grid == 0 || nunits * std::max(kRoundWeight[0][0], kRoundWeight[1][0]) * grid >= (1ull << 32)) return hipErrorInvalidValue;
  const dim3 g(grid);
  if (a.route1_lg && (!gate_up || a.route1_E > kMaxExperts || a.topk > kMaxTopK || a.topk > a.route1_E ||
                      a.nrec < a.topk || a.topk > kGemvThreads))
    return hipErrorInvalidValue;
  const size_t lds = gemv_launch_lds_bytes(nt, a.mt_max, a.nb, a.nrec, gate_up && a.ksplit > 1u);
  if (!gate_up && a.ksplit > 1u && a.ksplit != kDownSplit && a.ksplit != kDownSplitFew) return hipErrorInvalidValue;
  if (gate_up && a.ksplit > 1u && a.ksplit != kGateUpSplit) return hipErrorInvalidValue;
  if (nt == 1)
    launch_gemv_t<1, false>(a, gate_up, x_bf16, g, lds, s);
  else if (nt == 2 && 2u * a.mt_max <= 16u)  // both terms in one MFMA's columns
    launch_gemv_t<2, true>(a, gate_up, x_bf16, g, lds, s);
  else if (nt == 2)
    launch_gemv_t<2, false>(a, gate_up, x_bf16, g, lds, s);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// Combine of the grouped-GEMM path (bf16 x, y and slot rows, D % 8 == 0, 16-byte aligned x and
// y): eight outputs per thread, 16-byte loads and stores; the same per-element arithmetic and
// order as combine_kernel.
__device__ __forceinline__ void bf16x8_to_f32(const uint4 r, float (&v)[8]) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[2 * k] = bf16_bits_to_f32((uint16_t)w[k]);
    v[2 * k + 1] = bf16_bits_to_f32((uint16_t)(w[k] >> 16));
  }
}
__global__ __launch_bounds__(256) void combine_rows8_kernel(CombineArgs a) {
  const uint32_t t = blockIdx.y;
  const uint32_t d0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8u;
  if (d0 >= a.D) return;
  float xv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (a.add_residual) bf16x8_to_f32(*(const uint4 *)((const uint16_t *)a.x + (size_t)t * a.D + d0), xv);
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t p0 = 0; p0 < a.K; p0 += 8u) {
    float wv[8];
    uint4 yr[8];
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      const uint32_t p = min(p0 + u, a.K - 1u);
      wv[u] = a.topk_w[(size_t)t * a.K + p];
      yr[u] = load_stream16((const uint16_t *)a.ypart + ((size_t)t * a.K + p) * a.Dp + d0);  // Dp % 32 == 0; read once
    }
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      if (p0 + u >= a.K) break;
      float yv[8];
      bf16x8_to_f32(yr[u], yv);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = acc[j] + yv[j] * wv[u];
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    o[k] = (uint32_t)f32_to_bf16_bits(xv[2 * k] + acc[2 * k]) | ((uint32_t)f32_to_bf16_bits(xv[2 * k + 1] + acc[2 * k + 1]) << 16);
  *(uint4 *)((uint16_t *)a.y + (size_t)t * a.D + d0) = make_uint4(o[0], o[1], o[2], o[3]);
}

hipError_t launch_combine(const CombineArgs &a, bool x_bf16, hipStream_t s) {
  const dim3 grid((a.D + 1023) / 1024, a.n), block(256);
  if (a.nparts != 1u && a.nparts != kDownSplit && a.nparts != kDownSplitFew) return hipErrorInvalidValue;
  if (a.part_bf16 && a.nparts != 1u) return hipErrorInvalidValue;
  if (a.nout) {
    if (x_bf16 || a.part_bf16 || !a.ngamma || a.D == 0u || a.D % 4u != 0u || a.D > 4096u || a.Dp % 4u != 0u ||
        (((uintptr_t)a.x | (uintptr_t)a.y | (uintptr_t)a.nout | (uintptr_t)a.ngamma | (uintptr_t)a.ypart) & 15u))
      return hipErrorInvalidValue;
    if (a.nparts == 1u)
      (void)launch_kernel(combine_norm_kernel<1>, dim3(a.n), dim3(256), 0, s, a);
    else if (a.nparts == kDownSplit)
      (void)launch_kernel(combine_norm_kernel<kDownSplit>, dim3(a.n), dim3(256), 0, s, a);
    else
      (void)launch_kernel(combine_norm_kernel<kDownSplitFew>, dim3(a.n), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  if (a.part_bf16 && x_bf16 && a.D % 8u == 0u && (((uintptr_t)a.x | (uintptr_t)a.y) & 15u) == 0u) {
    (void)launch_kernel(combine_rows8_kernel, dim3((a.D + 2047u) / 2048u, a.n), dim3(256), 0, s, a);
  } else if (a.part_bf16) {
    if (x_bf16)
      (void)launch_kernel(combine_kernel<uint16_t, 1, true>, grid, block, 0, s, a);
    else
      (void)launch_kernel(combine_kernel<float, 1, true>, grid, block, 0, s, a);
  } else if (a.nparts == 1u) {
    if (x_bf16)
      (void)launch_kernel(combine_kernel<uint16_t, 1, false>, grid, block, 0, s, a);
    else
      (void)launch_kernel(combine_kernel<float, 1, false>, grid, block, 0, s, a);
  } else if (a.nparts == kDownSplitFew) {
    if (x_bf16)
      (void)launch_kernel(combine_kernel<uint16_t, kDownSplitFew, false>, grid, block, 0, s, a);
    else
      (void)launch_kernel(combine_kernel<float, kDownSplitFew, false>, grid, block, 0, s, a);
  } else {
    if (x_bf16)
      (void)launch_kernel(combine_kernel<uint16_t, kDownSplit, false>, grid, block, 0, s, a);
    else
      (void)launch_kernel(combine_kernel<float, kDownSplit, false>, grid, block, 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_dequant(const DequantArgs &a, hipStream_t s) {
  const uint64_t total = a.rows * a.bpr;
  uint64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks == 0) return hipSuccess;
  (void)launch_kernel(dequant_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace burnext
