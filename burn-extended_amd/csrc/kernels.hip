// kernels.hip -- MI355X (gfx950) kernels of the GPT-OSS MoE feed-forward over MXFP4 experts.
//
// route_kernel      RmsNorm + router logits + top-k/softmax (+ dispatch for one-workgroup batches)
//                   replaces src/moe/mod.rs:109-110,271-276 (Burn RmsNorm/Linear/topk ops)
// dispatch_kernel   histogram / exclusive scan / stable scatter into expert segments
//                   replaces the per-expert dense masks of src/moe/mod.rs:279-288
// expert_gemv       MXFP4 x bf16 projection on MFMA 16x16x32 bf16, e2m1+e8m0 dequantised in
//                   registers; gate_up epilogue fuses bias + clamped SwiGLU
//                   replaces w1_swiglu_dense_kernel / w2_scatter_dense_kernel (src/quant/gpu.rs:89-192)
// combine_kernel    y = x + sum_p w_p * (down_p + b2), deterministic slot order
//                   replaces the accumulate + residual of src/moe/mod.rs:405-411
// dequant_kernel    test hook: exact dequantisation (src/loader/mxfp4.rs:56-79)
#include "kernels.hpp"
#include "mx_device.hpp"

namespace burnext {

__device__ __forceinline__ float load_val(const float *p, size_t i) { return p[i]; }
__device__ __forceinline__ float load_val(const uint16_t *p, size_t i) { return bf16_bits_to_f32(p[i]); }
__device__ __forceinline__ void store_val(float *p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void store_val(uint16_t *p, size_t i, float v) { p[i] = f32_to_bf16_bits(v); }

// ---------------------------------------------------------------------------------------------
// Dispatch by one workgroup.  Stable counting sort of the flat entries t*K+p by expert: the rank
// of (t, e) inside expert e's segment is the number of earlier tokens that chose e, computed per
// chunk of blockDim.x tokens from a per-expert token bitmap (order-independent atomicOr) and
// popcount prefixes, so the result does not depend on thread timing.
// LDS: cnt[E], base[E], bm[E * words], wpre[E * words] (words = blockDim.x / 32).
// ---------------------------------------------------------------------------------------------
__device__ void block_dispatch(const int32_t *idx, uint32_t n, uint32_t K, uint32_t E, int32_t *seg_off,
                               int32_t *perm, int32_t *pos_of, int32_t *active, int32_t *num_active,
                               int32_t *lds) {
  const uint32_t tid = threadIdx.x, nth = blockDim.x, words = nth >> 5;
  int32_t *cnt = lds, *base = lds + E;
  uint32_t *bm = (uint32_t *)(lds + 2 * E);
  int32_t *wpre = lds + 2 * E + E * words;
  for (uint32_t e = tid; e < E; e += nth) cnt[e] = 0;
  __syncthreads();
  for (uint32_t i = tid; i < n * K; i += nth) {
    const int32_t e = idx[i];
    if (e >= 0 && (uint32_t)e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int32_t run = 0, na = 0;
    for (uint32_t e = 0; e < E; ++e) {
      seg_off[e] = run;
      base[e] = run;
      if (cnt[e] > 0) active[na++] = (int32_t)e;
      run += cnt[e];
    }
    seg_off[E] = run;
    for (uint32_t e = (uint32_t)na; e < E; ++e) active[e] = -1;
    *num_active = na;
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
    for (uint32_t i = tid; i < E * words; i += nth) {
      const uint32_t e = i / words, w = i % words;
      int32_t s = 0;
      for (uint32_t w2 = 0; w2 < w; ++w2) s += __popc(bm[e * words + w2]);
      wpre[i] = s;
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
      }
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += nth) base[e] += wpre[e * words + words - 1] + __popc(bm[e * words + words - 1]);
    __syncthreads();
  }
}

size_t dispatch_lds_bytes(uint32_t E, uint32_t threads) { return sizeof(int32_t) * (size_t)E * (2 + 2 * (threads / 32)); }

size_t route_lds_bytes(uint32_t tpb, uint32_t D, uint32_t E, uint32_t K, uint32_t threads) {
  size_t b = sizeof(float) * (size_t)tpb * D + sizeof(float) * (size_t)tpb * E + 2 * sizeof(int32_t) * (size_t)tpb * K;
  return b + dispatch_lds_bytes(E, threads);
}

// ---------------------------------------------------------------------------------------------
// Route kernel: one workgroup of 8 waves per block of tpb (<= 8) tokens.
//  phase 0  wave w loads token w, optional RmsNorm (sum of squares in the fixed lane/butterfly
//           order), keeps xn in LDS and writes its bf16 terms for the expert GEMVs
//  phase 1  logits: wave w computes experts w, w+8, ... for all tokens of the block; per logit
//           lane partials fmaf over c = lane + 64 i, then the butterfly, then + bias
//  phase 2  top-k: wave w selects token w's experts by repeated wave arg-max under `beats`
//           (ties -> lower index), softmax over the selected logits (lane 0, ascending order)
//  phase 3  (fuse_dispatch) the same workgroup builds the expert segments
// ---------------------------------------------------------------------------------------------
template <typename XT, typename WT>
__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const uint32_t tpb = a.tpb, D = a.D, E = a.E, K = a.K;
  float *xs = (float *)smem;
  float *lg = xs + (size_t)tpb * D;
  int32_t *sel = (int32_t *)(lg + (size_t)tpb * E);
  float *selv = (float *)(sel + (size_t)tpb * K);
  int32_t *dlds = (int32_t *)(selv + (size_t)tpb * K);

  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const uint32_t t0 = blockIdx.x * tpb;
  const uint32_t nh = min(tpb, a.n - t0);
  const XT *x = (const XT *)a.x;

  // phase 0
  if (w < nh) {
    const uint32_t t = t0 + w;
    float *xr = xs + (size_t)w * D;
    float p = 0.0f;
    for (uint32_t c = lane; c < D; c += 64) {
      const float v = load_val(x, (size_t)t * D + c);
      xr[c] = v;
      p = fmaf(v, v, p);
    }
    if (a.apply_norm) {
      p = wave_sum_butterfly(p);
      const float ms = p / (float)D;
      const float r = sqrtf(ms + a.eps);
      for (uint32_t c = lane; c < D; c += 64) xr[c] = (xr[c] / r) * a.gamma[c];
    }
    if (a.xn_terms) {
      uint16_t *dst = a.xn_terms + (size_t)t * a.nt * a.Dp;
      for (uint32_t c = lane; c < a.Dp; c += 64) {
        float v = c < D ? xr[c] : 0.0f;
        for (uint32_t i = 0; i < a.nt; ++i) {
          const uint16_t b = f32_to_bf16_bits(v);
          dst[(size_t)i * a.Dp + c] = b;
          v = v - bf16_bits_to_f32(b);
        }
      }
    }
  }
  __syncthreads();

  // phase 1
  const WT *rw = (const WT *)a.rw;
  for (uint32_t e = w; e < E; e += nwaves) {
    float acc[8];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) acc[tt] = 0.0f;
    const WT *wr = rw + (size_t)e * D;
    for (uint32_t c = lane; c < D; c += 64) {
      const float wv = load_val(wr, c);
#pragma unroll
      for (uint32_t tt = 0; tt < 8; ++tt)
        if (tt < nh) acc[tt] = fmaf(xs[(size_t)tt * D + c], wv, acc[tt]);
    }
#pragma unroll
    for (uint32_t tt = 0; tt < 8; ++tt) {
      if (tt < nh) {
        const float s = wave_sum_butterfly(acc[tt]);
        if (lane == 0) lg[tt * E + e] = s + a.rb[e];
      }
    }
  }
  __syncthreads();

  // phase 2
  if (w < nh) {
    const uint32_t t = t0 + w;
    const float *lr = lg + (size_t)w * E;
    float v[4];
    bool tk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t e = lane + 64u * j;
      v[j] = e < E ? lr[e] : 0.0f;
      tk[j] = e >= E;
    }
    for (uint32_t p = 0; p < K; ++p) {
      float bv = 0.0f;
      int bi = -1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = (int)(lane + 64u * j);
        if (!tk[j] && (bi < 0 || beats(v[j], e, bv, bi))) {
          bv = v[j];
          bi = e;
        }
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (oi >= 0 && (bi < 0 || beats(ov, oi, bv, bi))) {
          bv = ov;
          bi = oi;
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (bi == (int)(lane + 64u * j)) tk[j] = true;
      if (lane == 0) {
        sel[w * K + p] = bi;
        selv[w * K + p] = bv;
      }
    }
    if (lane == 0) {
      const float m = selv[w * K];
      float s = 0.0f;
      for (uint32_t p = 0; p < K; ++p) s += expf(selv[w * K + p] - m);
      for (uint32_t p = 0; p < K; ++p) {
        a.topk_idx[(size_t)t * K + p] = sel[w * K + p];
        a.topk_w[(size_t)t * K + p] = expf(selv[w * K + p] - m) / s;
      }
    }
    if (a.logits)
      for (uint32_t e = lane; e < E; e += 64) a.logits[(size_t)t * E + e] = lr[e];
  }

  // phase 3
  if (a.fuse_dispatch) {
    __syncthreads();
    block_dispatch(sel, a.n, K, E, a.seg_off, a.perm, a.pos_of, a.active, a.num_active, dlds);
  }
}

__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(DispatchArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  block_dispatch(a.topk_idx, a.n, a.K, a.E, a.seg_off, a.perm, a.pos_of, a.active, a.num_active,
                 (int32_t *)smem);
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
// f32 activations are split into NT bf16 terms (NT MFMAs per step).
// ---------------------------------------------------------------------------------------------
size_t gemv_lds_bytes(int nt, uint32_t mt_max, uint32_t nb) {
  return sizeof(uint16_t) * (size_t)nt * mt_max * (32u * nb + 8u);
}

__device__ __forceinline__ float swiglu_clamp(float g, float l, float alpha, float limit) {
  const float xg = fminf(g, limit);
  const float xl = fmaxf(-limit, fminf(l, limit));
  const float sig = 1.0f / (1.0f + expf(-alpha * xg));
  return (xg * sig) * (xl + 1.0f);
}

template <int NT, bool GATE_UP>
__global__ __launch_bounds__(kGemvThreads) void expert_gemv_kernel(GemvArgs a) {
  const int ai = (int)blockIdx.y;
  if (ai >= *a.num_active) return;
  const uint32_t rt_begin = blockIdx.x * a.tiles_per_wg;
  if (rt_begin >= a.nrt) return;
  const int e = a.active[ai];
  const int seg0 = a.seg_off[e];
  const int M = a.seg_off[e + 1] - seg0;

  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t *bs = (uint16_t *)smem;
  const uint32_t Kp = a.nb * 32u, ldk = Kp + 8u;
  const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
  const uint32_t i16 = lane & 15u, q = lane >> 4;
  const uint8_t *wexp = a.wb + (size_t)e * a.wb_estride;
  const uint8_t *sexp = a.ws + (size_t)e * a.ws_estride;
  const uint32_t nkg = (a.nb + 3u) >> 2;
  const uint32_t tail = a.nb - 4u * (nkg - 1u);
  const uint32_t mtm = a.mt_max;

  for (int m0 = 0; m0 < M; m0 += (int)mtm) {
    const uint32_t mt = (uint32_t)min((int)mtm, M - m0);
    __syncthreads();
    // stage B: mt tokens x Kp, NT bf16 terms, zero beyond the true K
    const uint32_t k8n = Kp >> 3;
    for (uint32_t id = threadIdx.x; id < mt * k8n; id += blockDim.x) {
      const uint32_t j = id / k8n, kb = (id % k8n) * 8u;
      if constexpr (GATE_UP) {
        const uint32_t tok = (uint32_t)a.perm[seg0 + m0 + (int)j] / a.topk;
#pragma unroll
        for (int term = 0; term < NT; ++term) {
          uint4 v = *(const uint4 *)(a.bterms + ((size_t)tok * NT + term) * Kp + kb);
          if (kb + 8u > a.kt) {
            uint16_t *h = (uint16_t *)&v;
            for (uint32_t u = 0; u < 8u; ++u)
              if (kb + u >= a.kt) h[u] = 0;
          }
          *(uint4 *)(bs + ((size_t)term * mtm + j) * ldk + kb) = v;
        }
      } else {
        const float *src = a.bf32 + (size_t)(seg0 + m0 + (int)j) * Kp + kb;
        const float4 lo = *(const float4 *)src, hi = *(const float4 *)(src + 4);
        const float vals[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        uint32_t pk[NT][4];
#pragma unroll
        for (int u = 0; u < 8; u += 2) {
          uint16_t t0[NT], t1[NT];
          split_bf16<NT>(kb + (uint32_t)u < a.kt ? vals[u] : 0.0f, t0);
          split_bf16<NT>(kb + (uint32_t)u + 1u < a.kt ? vals[u + 1] : 0.0f, t1);
#pragma unroll
          for (int term = 0; term < NT; ++term) pk[term][u >> 1] = (uint32_t)t0[term] | ((uint32_t)t1[term] << 16);
        }
#pragma unroll
        for (int term = 0; term < NT; ++term)
          *(uint4 *)(bs + ((size_t)term * mtm + j) * ldk + kb) = make_uint4(pk[term][0], pk[term][1], pk[term][2], pk[term][3]);
      }
    }
    __syncthreads();

    const bool bval = i16 < mt;
    const uint16_t *brow = bs + (size_t)i16 * ldk;
    for (uint32_t rt = rt_begin + wv; rt < min(rt_begin + a.tiles_per_wg, a.nrt); rt += 4u) {
      const uint8_t *wt = wexp + (size_t)rt * a.nb * 256u;
      const uint8_t *st = sexp + (size_t)rt * a.nb * 16u;
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      uint4 acur[4];
      uint32_t scur[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t kg = (uint32_t)u;
        const bool ok = kg < nkg && q < (kg + 1u == nkg ? tail : 4u);
        acur[u] = ok ? *(const uint4 *)(wt + kg * 1024u + lane * 16u) : make_uint4(0u, 0u, 0u, 0u);
        scur[u] = ok ? (uint32_t)st[kg * 64u + lane] : 0u;
      }
      for (uint32_t c0 = 0; c0 < nkg; c0 += 4u) {
        uint4 anx[4];
        uint32_t snx[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t kg = c0 + 4u + (uint32_t)u;
          const bool ok = kg < nkg && q < (kg + 1u == nkg ? tail : 4u);
          anx[u] = ok ? *(const uint4 *)(wt + kg * 1024u + lane * 16u) : make_uint4(0u, 0u, 0u, 0u);
          snx[u] = ok ? (uint32_t)st[kg * 64u + lane] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t kg = c0 + (uint32_t)u;
          if (kg >= nkg) break;
          const bool ok = q < (kg + 1u == nkg ? tail : 4u);
          const bool bok = bval && ok;
          const float sc = e8m0_to_f32(scur[u]);
          const uint32_t kb = 32u * (4u * kg + q);
          const uint32_t wd[4] = {acur[u].x, acur[u].y, acur[u].z, acur[u].w};
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const bf16x8_t A = fp4x8_to_bf16x8(wd[s], sc);
#pragma unroll
            for (int term = 0; term < NT; ++term) {
              bf16x8_t B = {};
              if (bok) B = *(const bf16x8_t *)(brow + (size_t)term * mtm * ldk + kb + 8u * s);
              acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, acc, 0, 0, 0);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          acur[u] = anx[u];
          scur[u] = snx[u];
        }
      }
      // epilogue: lane holds rows 4q..4q+3 of tile rt for token column i16
      if (bval) {
        const int pos = seg0 + m0 + (int)i16;
        const uint32_t r0 = rt * 16u + 4u * q;
        if constexpr (GATE_UP) {
          const float *bb = a.bias + (size_t)e * a.bias_estride + r0;
          const uint32_t f0 = r0 >> 1;
          const float o0 = swiglu_clamp(acc[0] + bb[0], acc[1] + bb[1], a.alpha, a.limit);
          const float o1 = swiglu_clamp(acc[2] + bb[2], acc[3] + bb[3], a.alpha, a.limit);
          float *o = a.out + (size_t)pos * a.out_stride + f0;
          if (f0 + 1u < a.out_rows) {
            *(float2 *)o = make_float2(o0, o1);
          } else if (f0 < a.out_rows) {
            o[0] = o0;
          }
        } else {
          float *o = a.out + (size_t)pos * a.out_stride + r0;
          if (r0 + 3u < a.out_rows) {
            *(float4 *)o = make_float4(acc[0], acc[1], acc[2], acc[3]);
          } else {
            for (uint32_t r = 0; r < 4u; ++r)
              if (r0 + r < a.out_rows) o[r] = acc[r];
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Combine: y[t, d] = (add_residual ? x[t, d] : 0) + sum_{p asc} (ypart[pos(t,p), d] + b2[e_p, d]) * w_p
// ---------------------------------------------------------------------------------------------
template <typename XT>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
  const uint32_t t = blockIdx.y;
  const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= a.D) return;
  float acc = 0.0f;
  for (uint32_t p = 0; p < a.K; ++p) {
    const int32_t e = a.topk_idx[(size_t)t * a.K + p];
    if (e < 0 || (uint32_t)e >= a.E) continue;
    const float w = a.topk_w[(size_t)t * a.K + p];
    const int32_t pos = a.pos_of[(size_t)t * a.K + p];
    acc = acc + (a.ypart[(size_t)pos * a.Dp + d] + a.b2[(size_t)e * a.D + d]) * w;
  }
  const XT *x = (const XT *)a.x;
  const float r = (a.add_residual ? load_val(x, (size_t)t * a.D + d) : 0.0f) + acc;
  store_val((XT *)a.y, (size_t)t * a.D + d, r);
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
#define BX_ATTR(f)                                                                                                  \
  do {                                                                                                               \
    hipError_t e_ = hipFuncSetAttribute((const void *)(f), hipFuncAttributeMaxDynamicSharedMemorySize, big);       \
    if (e_ != hipSuccess && err == hipSuccess) err = e_;                                                             \
  } while (0)
  BX_ATTR((route_kernel<float, float>));
  BX_ATTR((route_kernel<float, uint16_t>));
  BX_ATTR((route_kernel<uint16_t, float>));
  BX_ATTR((route_kernel<uint16_t, uint16_t>));
  BX_ATTR(dispatch_kernel);
  BX_ATTR((expert_gemv_kernel<1, true>));
  BX_ATTR((expert_gemv_kernel<1, false>));
  BX_ATTR((expert_gemv_kernel<3, true>));
  BX_ATTR((expert_gemv_kernel<3, false>));
#undef BX_ATTR
  return err;
}

hipError_t launch_route(const RouteArgs &a, bool x_bf16, bool w_bf16, hipStream_t s) {
  const dim3 grid((a.n + a.tpb - 1) / a.tpb), block(kRouteThreads);
  const size_t lds = route_lds_bytes(a.tpb, a.D, a.E, a.K, kRouteThreads);
  if (x_bf16) {
    if (w_bf16)
      route_kernel<uint16_t, uint16_t><<<grid, block, lds, s>>>(a);
    else
      route_kernel<uint16_t, float><<<grid, block, lds, s>>>(a);
  } else {
    if (w_bf16)
      route_kernel<float, uint16_t><<<grid, block, lds, s>>>(a);
    else
      route_kernel<float, float><<<grid, block, lds, s>>>(a);
  }
  return hipGetLastError();
}

hipError_t launch_dispatch(const DispatchArgs &a, hipStream_t s) {
  dispatch_kernel<<<dim3(1), dim3(kDispatchThreads), dispatch_lds_bytes(a.E, kDispatchThreads), s>>>(a);
  return hipGetLastError();
}

hipError_t launch_gemv(const GemvArgs &a, int nt, bool gate_up, uint32_t grid_x, uint32_t grid_y, hipStream_t s) {
  const dim3 grid(grid_x, grid_y), block(kGemvThreads);
  const size_t lds = gemv_lds_bytes(nt, a.mt_max, a.nb);
  if (nt == 1) {
    if (gate_up)
      expert_gemv_kernel<1, true><<<grid, block, lds, s>>>(a);
    else
      expert_gemv_kernel<1, false><<<grid, block, lds, s>>>(a);
  } else if (nt == 3) {
    if (gate_up)
      expert_gemv_kernel<3, true><<<grid, block, lds, s>>>(a);
    else
      expert_gemv_kernel<3, false><<<grid, block, lds, s>>>(a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_combine(const CombineArgs &a, bool x_bf16, hipStream_t s) {
  const dim3 grid((a.D + 255) / 256, a.n), block(256);
  if (x_bf16)
    combine_kernel<uint16_t><<<grid, block, 0, s>>>(a);
  else
    combine_kernel<float><<<grid, block, 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_dequant(const DequantArgs &a, hipStream_t s) {
  const uint64_t total = a.rows * a.bpr;
  uint64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks == 0) return hipSuccess;
  dequant_kernel<<<dim3((uint32_t)blocks), dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace burnext
