// gemm.hip -- grouped expert GEMM of prefill-sized batches on gfx950's block-scaled MFMA.
//
// replaces w1_swiglu_dense_kernel / w2_scatter_dense_kernel (src/quant/gpu.rs:89-192) for
// batches whose expert segments hold many tokens (the reference runs them per 256-token tile
// and per used expert, src/moe/mod.rs:262-404).
//
// v_mfma_scale_f32_16x16x128_f8f6f4 with A = MXFP4 weights (cbsz 4) and B = MXFP8 activations
// (blgp 0), e8m0 block scales applied by the matrix core:
//   A: lane l = 16 g + i holds row i, K [32 g, 32 g + 32) as 16 bytes (low nibble first) -- one
//      K-group of the tiled weight layout, read straight from HBM -- and that block's scale.
//   B: lane l = 16 g + j holds column (token) j, K [16 g, 16 g + 16) in bytes 0-15 and
//      K [64 + 16 g, 64 + 16 g + 16) in bytes 16-31; its scale operand is the scale of
//      K [32 g, 32 g + 32) of column j.
//   C: lane l = 16 q + j holds rows 4 q .. 4 q + 3 of column j.
// Activations are two MXFP8 terms (hi + lo), so each product is two MFMAs into one accumulator.
#include "kernels.hpp"
#include "mx_device.hpp"

namespace burnext {

typedef int32_t i32x8_t __attribute__((ext_vector_type(8)));

namespace {
// One K-group of the B tile in LDS, chunk-major: [term 2][16-byte chunk 8][token 128], so the 16
// lanes reading one chunk of 16 consecutive tokens read 256 contiguous bytes; then the scale
// dwords [term 2][token 128] (byte g = scale of K [32 g, 32 g + 32)).
constexpr uint32_t kBufBytes = 2u * 8u * kGemmTok * 16u;
constexpr uint32_t kScBytes = 2u * kGemmTok * 4u;
typedef __attribute__((address_space(3))) void lds_void;
}  // namespace

size_t gemm_lds_bytes() { return 2 * ((size_t)kBufBytes + kScBytes) + 2 * kGemmTok * 4 + 64; }

// Work item of workgroup b: blockIdx is remapped so that the workgroups of one XCD (b mod 8)
// take a contiguous run of items, then item = token tile gt * nrb + row block rb (rb fastest):
// the workgroups sharing a token tile's B run together on one XCD.  Each workgroup computes
// kGemmRows weight rows (8 row tiles) x kGemmTok tokens with 4 waves of 64 x 64 (wave wr, wc:
// rows 64 wr.., tokens 64 wc..; 4 x 4 MFMA tiles).  Per K-group the B tile (two terms) is staged
// into LDS by direct-to-LDS loads (double buffered, one barrier per K-group) while each wave
// loads its own A K-group (4 row tiles, 16 bytes per lane each) one K-group ahead.
template <bool GATE_UP>
__global__ __launch_bounds__(256, 2) void expert_gemm_kernel(GemmArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  int32_t *rows_l = (int32_t *)(smem + 2 * (kBufBytes + kScBytes));  // [kGemmTok] B row, -1 = none
  int32_t *slot_l = rows_l + kGemmTok;                                // [kGemmTok] down: slot
  int32_t *info_l = slot_l + kGemmTok;                                // [0] expert [1] tile of it

  const uint32_t G = gridDim.x, b = blockIdx.x;
  const uint32_t it = (b & 7u) * (G >> 3) + (b >> 3);  // G is a multiple of 8
  const uint32_t gt = it / a.nrb, rb = it - gt * a.nrb;
  if (threadIdx.x == 0) info_l[0] = -1;
  __syncthreads();
  for (uint32_t e = threadIdx.x; e < a.E; e += blockDim.x) {
    const uint32_t lo = (uint32_t)a.tile_off[e], hi = (uint32_t)a.tile_off[e + 1];
    if (gt >= lo && gt < hi) {
      info_l[0] = (int32_t)e;
      info_l[1] = (int32_t)(gt - lo);
    }
  }
  __syncthreads();
  const int e = info_l[0];
  if (e < 0) return;  // workgroup-uniform: beyond the realised token tiles
  const int seg0 = a.seg_off[e];
  const uint32_t M = (uint32_t)(a.seg_off[e + 1] - seg0);
  const uint32_t m0 = (uint32_t)info_l[1] * kGemmTok;
  const uint32_t ntok = min(kGemmTok, M - m0);
  for (uint32_t i = threadIdx.x; i < kGemmTok; i += blockDim.x) {
    int32_t row = -1, slot = -1;
    if (i < ntok) {
      const int32_t pos = seg0 + (int32_t)(m0 + i);
      slot = a.perm[pos];
      row = GATE_UP ? slot / (int32_t)a.topk : pos;
    }
    rows_l[i] = row;
    slot_l[i] = slot;
  }
  __syncthreads();

  const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
  const uint32_t wr = wv >> 1, wc = wv & 1u;
  const uint32_t i16 = lane & 15u, q = lane >> 4;
  const uint32_t nkg = (a.nb + 3u) >> 2, tail = a.nb - 4u * (nkg - 1u);
  const uint32_t kq = a.b.kq, sq = kq >> 5;  // code bytes and scale bytes per B row
  const uint8_t *wexp = a.wb + (size_t)e * a.wb_estride;
  const uint8_t *sexp = a.ws + (size_t)e * a.ws_estride;

  // ---- B staging by direct-to-LDS loads (no registers): per K-group 32 wave instructions of
  // 64 x 16 bytes (wave w: instructions w, w + 4, ..: chunk plane (term, chunk) = i / 2, tokens
  // 64 (i % 2) + lane) and 4 of 64 x 4 scale bytes (wave w: term w / 2, tokens 64 (w % 2) + lane).
  // Token columns beyond the tile read the tile's first row; their results are never stored.
  // row offsets of tokens lane and 64 + lane; wave w's scale instruction: term w / 2, half w % 2
  const int32_t r0l = rows_l[lane], r1l = rows_l[64u + lane];
  const size_t row0 = (size_t)(r0l >= 0 ? r0l : rows_l[0]), row1 = (size_t)(r1l >= 0 ? r1l : rows_l[0]);
  const uint8_t *ssrc = ((wv >> 1) ? a.b.slo : a.b.shi) + ((wv & 1u) ? row1 : row0) * sq;
  auto stage = [&](uint32_t kg, uint32_t p) {
    uint8_t *bd = smem + p * kBufBytes;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t i = wv + 4u * (uint32_t)k;
      const uint32_t plane = i >> 1, half = i & 1u, term = plane >> 3, chunk = plane & 7u;
      const uint8_t *src = (term ? a.b.lo : a.b.hi) + (half ? row1 : row0) * kq;
      __builtin_amdgcn_global_load_lds((const void *)(src + kg * 128u + chunk * 16u),
                                       (lds_void *)(bd + (plane * kGemmTok + half * 64u) * 16u), 16, 0, 0);
    }
    __builtin_amdgcn_global_load_lds((const void *)(ssrc + kg * 4u),
                                     (lds_void *)(smem + 2 * kBufBytes + p * kScBytes +
                                                  ((wv >> 1) * kGemmTok + (wv & 1u) * 64u) * 4u),
                                     4, 0, 0);
  };

  // ---- A: this wave's 4 row tiles of K-group kg (lanes outside the tile's blocks read the
  // tile's first 16 bytes and are neutralised: zero codes, scale 1)
  uint32_t rtile[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) rtile[rt] = min(rb * 8u + wr * 4u + (uint32_t)rt, a.nrt - 1u);
  auto lane_ok = [&](uint32_t kg) { return kg < nkg && q < (kg + 1u == nkg ? tail : 4u); };
  uint4 aw[4];
  uint32_t as[4];
  auto load_a = [&](uint32_t kg, uint4(&w)[4], uint32_t(&s)[4]) {
    const bool ok = lane_ok(kg);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      w[rt] = *(const uint4 *)(wexp + (size_t)rtile[rt] * a.nb * 256u + (ok ? kg * 1024u + lane * 16u : 0u));
      s[rt] = *(const uint32_t *)(sexp + (size_t)rtile[rt] * a.nb * 16u + (ok ? kg * 64u + (lane & ~3u) : 0u));
    }
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc[rt][tt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  stage(0, 0);
  load_a(0, aw, as);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's direct-to-LDS loads have landed
  __syncthreads();
  const uint32_t ash = 8u * (lane & 3u);
  for (uint32_t kg = 0; kg < nkg; ++kg) {
    const uint32_t p = kg & 1u;
    const uint32_t kn = min(kg + 1u, nkg - 1u);  // last iteration: reloads (unused), no branch
    stage(kn, p ^ 1u);  // the other buffer: every wave left it at the previous barrier
    uint4 awn[4];
    uint32_t asn[4];
    load_a(kn, awn, asn);
    const bool ok = lane_ok(kg);
    i32x8_t A[4];
    int32_t sa[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const uint4 w4 = ok ? aw[rt] : make_uint4(0u, 0u, 0u, 0u);
      A[rt] = i32x8_t{(int32_t)w4.x, (int32_t)w4.y, (int32_t)w4.z, (int32_t)w4.w, 0, 0, 0, 0};
      sa[rt] = ok ? (int32_t)((as[rt] >> ash) & 0xFFu) : 127;
    }
    const uint8_t *bd = smem + p * kBufBytes;
    const uint8_t *bsc = smem + 2 * kBufBytes + p * kScBytes;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const uint32_t tok = wc * 64u + (uint32_t)tt * 16u + i16;
      // lane group q: chunks q and 4 + q (K [16 q, +16) and [64 + 16 q, +16)) of both terms
      const uint8_t *r = bd + (q * kGemmTok + tok) * 16u;
      const uint4 h0 = *(const uint4 *)r, h1 = *(const uint4 *)(r + 4u * kGemmTok * 16u);
      const uint4 l0 = *(const uint4 *)(r + 8u * kGemmTok * 16u), l1 = *(const uint4 *)(r + 12u * kGemmTok * 16u);
      const i32x8_t Bh = {(int32_t)h0.x, (int32_t)h0.y, (int32_t)h0.z, (int32_t)h0.w,
                          (int32_t)h1.x, (int32_t)h1.y, (int32_t)h1.z, (int32_t)h1.w};
      const i32x8_t Bl = {(int32_t)l0.x, (int32_t)l0.y, (int32_t)l0.z, (int32_t)l0.w,
                          (int32_t)l1.x, (int32_t)l1.y, (int32_t)l1.z, (int32_t)l1.w};
      const int32_t sbh = bsc[tok * 4u + q], sbl = bsc[(kGemmTok + tok) * 4u + q];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        acc[rt][tt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[rt], Bh, acc[rt][tt], 4, 0, 0, sa[rt], 0, sbh);
        acc[rt][tt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[rt], Bl, acc[rt][tt], 4, 0, 0, sa[rt], 0, sbl);
      }
      // one token tile's B fragments live at a time
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      aw[rt] = awn[rt];
      as[rt] = asn[rt];
    }
    __builtin_amdgcn_s_waitcnt(0);  // K-group kn's direct-to-LDS loads have landed
    __syncthreads();
  }

  // ---- epilogue
  if constexpr (GATE_UP) {
    // wave wr owns features rb*64 + wr*32 .. +32: one MX block per token.  Lane (q, j) holds
    // features 8 rt + 2 q + {0, 1} (interleaved gate/linear row pairs) of its token columns.
    const uint32_t fb = rb * 64u + wr * 32u;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const uint32_t tok = wc * 64u + (uint32_t)tt * 16u + i16;
      float o[8];
      float amax = 0.0f;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const uint32_t r0 = rb * 128u + wr * 64u + (uint32_t)rt * 16u + 4u * q;  // W1 row
        const bool rv = rb * 8u + wr * 4u + (uint32_t)rt < a.nrt;
        const f32x4_t bb = *(const f32x4_t *)(a.bias + (size_t)e * a.bias_estride + min(r0, a.bias_estride - 4u));
        const uint32_t f0 = fb + (uint32_t)rt * 8u + 2u * q;
        float v0 = swiglu_clamp_f(acc[rt][tt][0] + bb[0], acc[rt][tt][1] + bb[1], a.alpha, a.limit);
        float v1 = swiglu_clamp_f(acc[rt][tt][2] + bb[2], acc[rt][tt][3] + bb[3], a.alpha, a.limit);
        v0 = (rv && f0 < a.act_feats) ? v0 : 0.0f;
        v1 = (rv && f0 + 1u < a.act_feats) ? v1 : 0.0f;
        o[2 * rt] = v0;
        o[2 * rt + 1] = v1;
        amax = fmaxf(amax, fmaxf(fabsf(v0), fabsf(v1)));
      }
      amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
      amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
      const uint32_t sbh = mx8_scale_byte(amax);
      const float ih = sbh ? mx8_inv_scale(sbh) : 0.0f, sh = e8m0_to_f32(sbh);
      uint32_t ch[4];
      float res[8], rmax = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        ch[k] = f32x2_to_fp8x2(o[2 * k] * ih, o[2 * k + 1] * ih);
        res[2 * k] = o[2 * k] - fp8_to_f32<0>(ch[k]) * sh;
        res[2 * k + 1] = o[2 * k + 1] - fp8_to_f32<1>(ch[k]) * sh;
        rmax = fmaxf(rmax, fmaxf(fabsf(res[2 * k]), fabsf(res[2 * k + 1])));
      }
      rmax = fmaxf(rmax, __shfl_xor(rmax, 16, 64));
      rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
      const uint32_t sbl = mx8_scale_byte(rmax);
      const float il = sbl ? mx8_inv_scale(sbl) : 0.0f;
      if (tok < ntok) {
        const size_t row = (size_t)(seg0 + (int32_t)(m0 + tok));
        uint8_t *dh = a.act.hi + row * a.act.kq + fb + 2u * q;
        uint8_t *dl = a.act.lo + row * a.act.kq + fb + 2u * q;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          *(uint16_t *)(dh + 8u * k) = (uint16_t)ch[k];
          *(uint16_t *)(dl + 8u * k) = (uint16_t)f32x2_to_fp8x2(res[2 * k] * il, res[2 * k + 1] * il);
        }
        if (q == 0) {
          a.act.shi[row * (a.act.kq >> 5) + (fb >> 5)] = (uint8_t)sbh;
          a.act.slo[row * (a.act.kq >> 5) + (fb >> 5)] = (uint8_t)sbl;
        }
      }
    }
    // zero the K padding of the act rows beyond the last row block's features
    if (rb + 1u == a.nrb) {
      const uint32_t f_end = a.nrb * 64u, padb = a.act.kq - f_end;  // multiple of 32
      for (uint32_t i = threadIdx.x; i < ntok * padb; i += blockDim.x) {
        const uint32_t tk = i / padb, c = i - tk * padb;
        const size_t row = (size_t)(seg0 + (int32_t)(m0 + tk));
        a.act.hi[row * a.act.kq + f_end + c] = 0;
        a.act.lo[row * a.act.kq + f_end + c] = 0;
        if ((c & 31u) == 0u) {
          a.act.shi[row * (a.act.kq >> 5) + ((f_end + c) >> 5)] = 0;
          a.act.slo[row * (a.act.kq >> 5) + ((f_end + c) >> 5)] = 0;
        }
      }
    }
  } else {
    // token-major slot rows t * topk + p, expert bias b2 added once
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const uint32_t tok = wc * 64u + (uint32_t)tt * 16u + i16;
      if (tok >= ntok) continue;
      float *orow = a.out + (size_t)slot_l[tok] * a.out_stride;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        if (rb * 8u + wr * 4u + (uint32_t)rt >= a.nrt) continue;
        const uint32_t r0 = rb * 128u + wr * 64u + (uint32_t)rt * 16u + 4u * q;
        const f32x4_t bb = *(const f32x4_t *)(a.bias + (size_t)e * a.bias_estride + r0);
        if (r0 + 3u < a.out_rows) {
          *(float4 *)(orow + r0) = make_float4(acc[rt][tt][0] + bb[0], acc[rt][tt][1] + bb[1],
                                               acc[rt][tt][2] + bb[2], acc[rt][tt][3] + bb[3]);
        } else {
          for (uint32_t r = 0; r < 4u; ++r)
            if (r0 + r < a.out_rows) orow[r0 + r] = acc[rt][tt][r] + bb[r];
        }
      }
    }
  }
}

hipError_t configure_gemm_kernels() {
  const int lds = (int)gemm_lds_bytes();
  hipError_t e1 = hipFuncSetAttribute((const void *)expert_gemm_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  hipError_t e2 = hipFuncSetAttribute((const void *)expert_gemm_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  return e1 != hipSuccess ? e1 : e2;
}

hipError_t launch_gemm(const GemmArgs &a, bool gate_up, uint32_t grid, hipStream_t s) {
  if (grid == 0 || (grid & 7u) != 0 || a.nrb == 0 || a.b.kq % 128u != 0) return hipErrorInvalidValue;
  if (gate_up)
    expert_gemm_kernel<true><<<dim3(grid), dim3(256), gemm_lds_bytes(), s>>>(a);
  else
    expert_gemm_kernel<false><<<dim3(grid), dim3(256), gemm_lds_bytes(), s>>>(a);
  return hipGetLastError();
}

}  // namespace burnext
