// fused.hip -- the experts of a decode-sized MoE batch in one launch (gfx950), and the combine over
// its slices.  Replaces, for batches of at most 16 tokens, the gate_up and down expert GEMVs of
// kernels.hip (reference w1_swiglu_dense_kernel / w2_scatter_dense_kernel, src/quant/gpu.rs:89-192)
// with one launch: each workgroup streams the weights of one (expert, feature slice) item, and no
// workgroup waits for another, so the batch pays one launch-to-first-weights start-up instead of
// two.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "kernels.hpp"
#include "mx_device.hpp"

namespace burnext {
namespace {

// s_waitcnt lgkmcnt(0) only (vmcnt and expcnt left at their maxima)
constexpr int kLgkm0 = 0xF | (7 << 4) | (3 << 14);

// Workgroup barrier for data in LDS: the wave's LDS accesses are complete before it arrives; its
// global loads (the weight prefetch) stay in flight -- __syncthreads() would wait for them too.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kLgkm0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// a / b for a < 2^20 and b <= 2^12 given rb = 1.0f / b (exact: see div_small in kernels.hip)
__device__ __forceinline__ uint32_t fdiv_small(uint32_t a, float rb) { return (uint32_t)(((float)a + 0.5f) * rb); }

constexpr uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }

// 8 consecutive activations (f32 or bf16 bits), loaded raw and converted at use.
template <typename T> struct Raw8;
template <> struct Raw8<float> { float4 a, b; };
template <> struct Raw8<uint16_t> { uint4 a; };
__device__ __forceinline__ void raw_load8(Raw8<float> &c, const float *p) {
  c.a = *(const float4 *)p;
  c.b = *(const float4 *)(p + 4);
}
__device__ __forceinline__ void raw_load8(Raw8<uint16_t> &c, const uint16_t *p) { c.a = *(const uint4 *)p; }
__device__ __forceinline__ void raw_vals8(const Raw8<float> &c, float (&v)[8]) {
  v[0] = c.a.x, v[1] = c.a.y, v[2] = c.a.z, v[3] = c.a.w, v[4] = c.b.x, v[5] = c.b.y, v[6] = c.b.z, v[7] = c.b.w;
}
__device__ __forceinline__ void raw_vals8(const Raw8<uint16_t> &c, float (&v)[8]) {
  const uint32_t w[4] = {c.a.x, c.a.y, c.a.z, c.a.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_bits_to_f32((uint16_t)w[i]);
    v[2 * i + 1] = bf16_bits_to_f32((uint16_t)(w[i] >> 16));
  }
}
__device__ __forceinline__ float ld_val(const float *p, size_t i) { return p[i]; }
__device__ __forceinline__ float ld_val(const uint16_t *p, size_t i) { return bf16_bits_to_f32(p[i]); }
__device__ __forceinline__ void st_val(float *p, size_t i, float v) { p[i] = v; }
__device__ __forceinline__ void st_val(uint16_t *p, size_t i, float v) { p[i] = f32_to_bf16_bits(v); }

// LDS carve-up of moe_fused_kernel (byte offsets, 16-byte aligned regions): the staged token rows
// of a pass (NT bf16 terms), the SwiGLU rows of up to 16 tokens (NT terms, zero where unused), the
// K-part pre-activations of a pass, the slice's b1 rows, b2 (slice 0), record and token lists,
// the phase-1 unit counter.
struct FusedLds {
  uint32_t bs, act, pre, b1, b2, rec, slot, tok, cnt, total;
};
__host__ __device__ inline FusedLds fused_lds(int nt, uint32_t sb_max, uint32_t mt, uint32_t nb1, uint32_t Dp2) {
  FusedLds l{};
  const uint32_t ldk = 32u * nb1 + 8u, af = 32u * sb_max + 8u;
  l.bs = 0;
  l.act = align16((uint32_t)nt * mt * ldk * 2u);
  l.pre = align16(l.act + (uint32_t)nt * 16u * af * 2u);
  // K-parts (ks1 > 1) only for slices of fewer than kFusedWaves W1 row tiles: ks1 * tiles <= waves
  l.b1 = align16(l.pre + mt * 16u * kFusedWaves * 4u);
  l.b2 = align16(l.b1 + 64u * sb_max * 4u);
  l.rec = align16(l.b2 + Dp2 * 4u);
  l.slot = l.rec + kRecWords * 4u;
  l.tok = l.slot + 16u * 4u;
  l.cnt = l.tok + 16u * 4u;
  l.total = align16(l.cnt + 4u);
  return l;
}

// Slices per expert for na active experts on a grid of G workgroups (also combine_slices_kernel).
__device__ __forceinline__ uint32_t fused_slices(uint32_t G, uint32_t na, uint32_t cap) {
  return max(1u, min(G / max(na, 1u), cap));
}

// ---------------------------------------------------------------------------------------------
// moe_fused_kernel.  Workgroup g (of G, one per CU) takes items g, g + G, ... of na * nsl, item =
// (active-expert slot ai, slice s); slice s = W2 K blocks [b_lo, b_hi) = SwiGLU features
// [32 b_lo, 32 b_hi) = W1 interleaved rows [64 b_lo, 64 b_hi) = W1 row tiles [4 b_lo, 4 b_hi).
//   phase 1 (per token pass of mt_max tokens): units = (W1 row tile of the slice, K-part h < ks1
//     of its K-groups; ks1 > 1 only for slices of fewer W1 row tiles than waves), numbered over
//     the passes: wave w takes unit w, then the next free one from a workgroup counter in LDS
//     (waves that stream slower take fewer), in steps of kFusedKgPerStep K-groups; lane (j, q) of
//     a unit's MFMA output holds rows 4q..4q+3 of the tile for token j = two (gate, linear)
//     pairs.  With ks1 = 1 the unit's epilogue adds b1 and writes the clamped SwiGLU of both
//     features to LDS (NT bf16 terms: the rounding the separate down GEMV applies to its f32
//     input); with ks1 > 1 it writes the raw pre-activations, which the workgroup sums in part
//     order at the pass barrier.
//   phase 2: units = W2 row tiles (all D rows) over the slice's K-groups, every token of the
//     expert at once (the SwiGLU rows of up to 16 tokens are in LDS).  Epilogue: the partial
//     output rows of the expert's slots, with b2 in slice 0.
// Lanes whose block lies outside a unit (the K tail, blocks outside the slice) load a valid
// address and are neutralised by a zero scale: A = 0, and their B reads take the start of their
// own LDS row (finite values; B rows past the pass's tokens only feed output columns not stored).
// Memory pipeline (as expert_gemv_kernel): kFusedKgPerStep register slots per wave, each
// refilled right after its MFMAs with the same slot of the next step -- generated one step ahead
// across units, passes and the two phases (past the end: dummy loads of the expert's bias rows,
// which keep the count of loads static) -- so the next pass's or phase 2's first weights are in
// flight while the wave waits at a pass barrier.  All bookkeeping is wave-uniform (scalar) and
// the rare paths (epilogues, barriers, staging) sit outside the unrolled slots, which keeps the
// kernel's code small: a version with them inlined in every slot ran at half the bandwidth.
// ---------------------------------------------------------------------------------------------
template <int NT, typename XT>
__global__ __launch_bounds__(kFusedWaves * 64) __attribute__((amdgpu_waves_per_eu(4))) void moe_fused_kernel(FusedArgs a) {
  constexpr uint32_t CJ = kFusedKgPerStep;
  constexpr uint32_t W = kFusedWaves;
  constexpr uint32_t NTH = W * 64u;
  extern __shared__ __align__(16) unsigned char smem[];
  const uint32_t mtm = a.mt_max;
  const uint32_t Dp2 = a.nrt2 * 16u;
  const FusedLds ly = fused_lds(NT, a.sb_max, mtm, a.nb1, Dp2);
  const uint32_t Kp1 = a.nb1 * 32u, ldk = Kp1 + 8u;
  const uint32_t AF = 32u * a.sb_max + 8u;
  uint16_t *bs = (uint16_t *)(smem + ly.bs);
  uint16_t *act = (uint16_t *)(smem + ly.act);
  float *pre = (float *)(smem + ly.pre);
  float *b1l = (float *)(smem + ly.b1);
  float *b2l = (float *)(smem + ly.b2);
  int32_t *rec_l = (int32_t *)(smem + ly.rec);
  int32_t *slot_l = (int32_t *)(smem + ly.slot);
  int32_t *tok_l = (int32_t *)(smem + ly.tok);
  uint32_t *ucnt = (uint32_t *)(smem + ly.cnt);

  const uint32_t lane = threadIdx.x & 63u, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t i16 = lane & 15u, q = lane >> 4;
  const uint32_t sshift = 8u * (lane & 3u);
  const uint32_t G = gridDim.x;
  const uint32_t na = __builtin_amdgcn_readfirstlane((uint32_t)*a.num_active);
  const uint32_t nsl = fused_slices(G, na, min(a.nb2, a.nsl_cap));
  const uint32_t items = na * nsl;
  const uint32_t nkg1 = (a.nb1 + 3u) >> 2, tail1 = a.nb1 - 4u * (nkg1 - 1u);
  const uint32_t T1 = a.nb1 * 256u, S1 = a.nb1 * 16u, T2 = a.nb2 * 256u, S2 = a.nb2 * 16u;
  // per-lane parts of the B operand's LDS byte offsets; a neutralised lane (zero scale) reads the
  // first 32 values of its own row instead, which are finite (0 x NaN would poison its column)
  const uint32_t bs_row = 2u * min(i16, mtm - 1u) * ldk, bs_lane = bs_row + 64u * q;
  const uint32_t act_row = 2u * i16 * AF, act_lane = act_row + 64u * q;
  const uint32_t bs_tstride = mtm * ldk * 2u, act_tstride = 16u * AF * 2u;

  for (uint32_t it = blockIdx.x; it < items; it += G) {
    const uint32_t ai = it / nsl, s = it - ai * nsl;
    if (threadIdx.x < kRecWords) rec_l[threadIdx.x] = a.exrec[(size_t)ai * kRecWords + threadIdx.x];
    if (threadIdx.x == 0) *ucnt = 0u;
    __syncthreads();
    const int e = __builtin_amdgcn_readfirstlane(rec_l[0]), seg0 = __builtin_amdgcn_readfirstlane(rec_l[1]);
    // segment size: at most the batch's tokens (<= 16), clamped so the lists stay in bounds
    const uint32_t M = min((uint32_t)__builtin_amdgcn_readfirstlane(rec_l[2]), 16u);
    if (threadIdx.x < M) {
      // segment entry j: slot t * topk + p from the record (first kRecTokens) or the segment list
      const uint32_t jj = threadIdx.x;
      const int32_t slot = jj < kRecTokens ? rec_l[4 + kRecTokens + jj] : a.perm[seg0 + (int)jj];
      slot_l[jj] = slot;
      tok_l[jj] = slot / (int32_t)a.topk;
    }
    // slice geometry (wave-uniform)
    const uint32_t b_lo = s * a.nb2 / nsl, b_hi = (s + 1u) * a.nb2 / nsl;
    const uint32_t rt0 = 4u * b_lo;
    const uint32_t nt1 = min(4u * (b_hi - b_lo), a.nrt1 - rt0);  // W1 row tiles of the slice
    uint32_t ks1 = nt1 >= W ? 1u : min(W / nt1, nkg1);
    const uint32_t H1 = (nkg1 + ks1 - 1u) / ks1;
    ks1 = (nkg1 + H1 - 1u) / H1;  // no empty K-part
    const uint32_t nu1 = nt1 * ks1;
    const uint32_t PR = 16u * nt1;  // pre-activation row stride
    const uint32_t kg2_lo = b_lo >> 2, kpr = ((b_hi - 1u) >> 2) + 1u - kg2_lo;  // W2 K-groups of the slice
    const uint32_t npass = (M + mtm - 1u) / mtm;
    const uint32_t NU = npass * nu1;  // phase-1 units over all passes, pass-major
    const uint8_t *w1e = a.w1b + (size_t)e * a.w1b_es, *s1e = a.w1s + (size_t)e * a.w1s_es;
    const uint8_t *w2e = a.w2b + (size_t)e * a.w2b_es, *s2e = a.w2s + (size_t)e * a.w2s_es;
    const uint8_t *dummy = (const uint8_t *)(a.b1 + (size_t)e * a.b1_es) + min(lane * 16u, a.b1_es * 4u - 16u);
    // this wave's phase-2 W2 row tiles [r_lo, r_hi) (balanced split)
    const uint32_t r_lo = wv * a.nrt2 / W, r_hi = (wv + 1u) * a.nrt2 / W;

    // Refill generator, one step ahead of the consumer.  Mode 0: a phase-1 step (K-groups
    // kg0 .. kg0 + CJ - 1 of unit g; those at or past kend are padding); mode 1: phase-2 slots
    // (row tile u, K-group kg2_lo + kk); mode 2: past the end (dummy loads).  g is the unit of
    // the step the generator loads next (NU and above once in mode 1 or 2).
    struct Gen {
      uint32_t mode, g, u, kg0, kend, kk;
      const uint8_t *wb, *sp;
    } gen{};
    auto gen_unit1 = [&](uint32_t g) {
      const uint32_t u = g % nu1, h = u / nt1;
      gen.g = g;
      gen.kg0 = h * H1;
      gen.kend = min(nkg1, gen.kg0 + H1);
      gen.wb = w1e + (size_t)(rt0 + (u - h * nt1)) * T1;
      gen.sp = s1e + (size_t)(rt0 + (u - h * nt1)) * S1;
    };
    auto gen_phase2 = [&]() {
      gen.g = NU;
      gen.mode = r_lo < r_hi ? 1u : 2u;
      gen.u = r_lo;
      gen.kk = 0u;
      gen.wb = w2e + (size_t)r_lo * T2;
      gen.sp = s2e + (size_t)r_lo * S2;
    };
    if (wv < NU) {
      gen.mode = 0u;
      gen_unit1(wv);
    } else {
      gen_phase2();
    }
    // the load of slot j of the generator's step (mode 1 advances per slot)
    auto gen_slot = [&](uint32_t j, uint4 &av, uint32_t &sv) {
      const uint8_t *wp = dummy, *sp = s1e;
      if (gen.mode == 0u) {
        const uint32_t kg = gen.kg0 + j;
        const bool ok = kg < gen.kend && (kg + 1u < nkg1 || q < tail1);
        wp = gen.wb + (ok ? kg * 1024u + lane * 16u : 0u);
        sp = gen.sp + (ok ? kg * 64u + (lane & ~3u) : 0u);
      } else if (gen.mode == 1u) {
        const uint32_t kg = kg2_lo + gen.kk, blk = 4u * kg + q;
        const bool ok = blk >= b_lo && blk < b_hi;
        wp = gen.wb + kg * 1024u + (ok ? lane * 16u : 0u);
        sp = gen.sp + kg * 64u + (ok ? (lane & ~3u) : 0u);
        if (++gen.kk == kpr) {
          gen.kk = 0u;
          gen.wb += T2;
          gen.sp += S2;
          if (++gen.u == r_hi) gen.mode = 2u;
        }
      }
      av = load_stream16(wp);
      sv = *(const uint32_t *)sp;  // the dword holding this lane's scale byte (byte lane & 3)
    };
    // after the CJ slots of a step: a mode-0 generator moves to its next step
    auto gen_step = [&]() {
      if (gen.mode != 0u) return;
      gen.kg0 += CJ;
      if (gen.kg0 < gen.kend) return;
      uint32_t v = 0u;
      if (lane == 0u) v = atomicAdd(ucnt, 1u);
      const uint32_t g = W + __builtin_amdgcn_readfirstlane(v);
      if (g < NU) {
        gen_unit1(g);
      } else {
        gen_phase2();
      }
    };

    // zero the SwiGLU rows (tokens past the expert's and features past F must read as 0)
    for (uint32_t i = threadIdx.x; i < (uint32_t)NT * 16u * AF / 2u; i += NTH) ((uint32_t *)act)[i] = 0u;
    __syncthreads();  // tok_l / slot_l written

    uint4 abuf[CJ];
    uint32_t sbuf[CJ];
    // staging of pass p's token rows (NT bf16 terms, zero beyond the true K); with `first` the
    // generator's first step is loaded after the first batch of rows
    auto stage = [&](uint32_t p, bool first) {
      constexpr int SBT = NT == 1 ? 3 : 2;
      const XT *src = (const XT *)a.xn;
      const uint32_t m0 = p * mtm, mt = min(mtm, M - m0);
      const uint32_t k8n = Kp1 >> 3, nitm = mt * k8n;
      const float rk8n = 1.0f / (float)k8n;
      for (uint32_t base = threadIdx.x; base < nitm; base += SBT * NTH) {
        Raw8<XT> cx[SBT];
#pragma unroll
        for (int u = 0; u < SBT; ++u) {
          const uint32_t id = min(base + (uint32_t)u * NTH, nitm - 1u);
          const uint32_t j = fdiv_small(id, rk8n), kb = (id - j * k8n) * 8u;
          raw_load8(cx[u], src + (size_t)tok_l[m0 + j] * Kp1 + kb);
        }
        if (first) {
#pragma unroll
          for (uint32_t j = 0; j < CJ; ++j) gen_slot(j, abuf[j], sbuf[j]);
          gen_step();
        }
        first = false;
#pragma unroll
        for (int u = 0; u < SBT; ++u) {
          const uint32_t id = base + (uint32_t)u * NTH;
          if (id >= nitm) continue;
          const uint32_t j = fdiv_small(id, rk8n), kb = (id - j * k8n) * 8u;
          float v8[8];
          raw_vals8(cx[u], v8);
#pragma unroll
          for (int v = 0; v < 8; ++v) v8[v] = kb + (uint32_t)v < a.kt1 ? v8[v] : 0.0f;
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
      if (first) {
#pragma unroll
        for (uint32_t j = 0; j < CJ; ++j) gen_slot(j, abuf[j], sbuf[j]);
        gen_step();
      }
    };
    {
      // the slice's b1 rows and (slice 0) b2: requested with the first token rows and weights,
      // stored after them (one round trip); rows past kFusedBiasRegs * NTH are copied after
      const float *b1e = a.b1 + (size_t)e * a.b1_es + rt0 * 16u;
      const float *b2e = a.b2 + (size_t)e * a.b2_es;
      const uint32_t n1 = nt1 * 16u, nb = n1 + (s == 0u ? Dp2 : 0u);
      auto bsrc = [&](uint32_t i) { return i < n1 ? b1e + i : b2e + (i - n1); };
      auto bdst = [&](uint32_t i) { return i < n1 ? b1l + i : b2l + (i - n1); };
      float bv[kFusedBiasRegs];
#pragma unroll
      for (uint32_t r = 0; r < kFusedBiasRegs; ++r) {
        const uint32_t i = threadIdx.x + r * NTH;
        bv[r] = i < nb ? *bsrc(i) : 0.0f;
      }
      stage(0u, true);
#pragma unroll
      for (uint32_t r = 0; r < kFusedBiasRegs; ++r) {
        const uint32_t i = threadIdx.x + r * NTH;
        if (i < nb) *bdst(i) = bv[r];
      }
      for (uint32_t i = threadIdx.x + kFusedBiasRegs * NTH; i < nb; i += NTH) *bdst(i) = *bsrc(i);
    }
    __syncthreads();

    // one K-group slot: A = the slot's 32 e2m1 codes per lane at scale sc (0: neutralised lane),
    // B from LDS at byte offset boff (+ term stride)
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    auto mfma_slot = [&](uint32_t j, float sc, const unsigned char *bb, uint32_t boff, uint32_t tstride) {
      const uint32_t wd[4] = {abuf[j].x, abuf[j].y, abuf[j].z, abuf[j].w};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const bf16x8_t A = fp4x8_to_bf16x8(wd[st], sc);
#pragma unroll
        for (int term = 0; term < NT; ++term) {
          const u32x4_t r = *(const u32x4_t *)(bb + boff + term * tstride + 16u * st);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8_t, r), acc, 0, 0, 0);
        }
      }
    };

    // ---- phase 1: passes of up to mtm tokens, units in steps of CJ K-groups
    uint32_t cg = wv;  // the consumer's unit (as numbered by the generator)
    for (uint32_t p = 0; p < npass; ++p) {
      const uint32_t m0 = p * mtm, mt = min(mtm, M - m0);
      while (cg < (p + 1u) * nu1) {
        const uint32_t u = cg - p * nu1, h = u / nt1, rt = rt0 + (u - h * nt1);
        uint32_t nxt = cg;
        const uint32_t ks = h * H1, ke = min(nkg1, ks + H1);
        for (uint32_t k0 = ks; k0 < ke; k0 += CJ) {
#pragma unroll
          for (uint32_t j = 0; j < CJ; ++j) {
            const uint32_t kg = k0 + j;
            if (kg < ke) {
              const bool ok = kg + 1u < nkg1 || q < tail1;
              const float sc = ok ? e8m0_to_f32((sbuf[j] >> sshift) & 0xFFu) : 0.0f;
              mfma_slot(j, sc, (const unsigned char *)bs, ok ? bs_lane + kg * 256u : bs_row, bs_tstride);
            }
            gen_slot(j, abuf[j], sbuf[j]);
            // keep each K-group's LDS reads, MFMAs and refill together (bounds the live registers)
            __builtin_amdgcn_sched_barrier(0);
          }
          nxt = gen.g;  // the unit of the step just requested: the consumer's next after this unit
          gen_step();
        }
        // the unit's epilogue: lane (i16, q) holds rows 4q..4q+3 of the tile for token m0 + i16
        const uint32_t r0 = 16u * (rt - rt0) + 4u * q;  // row of the slice's W1 rows
        if (i16 < mt) {
          if (ks1 == 1u) {
            const float o0 = swiglu_clamp_f(acc[0] + b1l[r0], acc[1] + b1l[r0 + 1u], a.alpha, a.limit);
            const float o1 = swiglu_clamp_f(acc[2] + b1l[r0 + 2u], acc[3] + b1l[r0 + 3u], a.alpha, a.limit);
            uint32_t tp[NT];
            split_bf16x2<NT>(o0, o1, tp);
#pragma unroll
            for (int term = 0; term < NT; ++term)
              *(uint32_t *)(act + ((size_t)term * 16u + m0 + i16) * AF + (r0 >> 1)) = tp[term];
          } else {
            const bool hb = h == 0u;  // b1 in part 0
            *(float4 *)(pre + ((size_t)h * mtm + i16) * PR + r0) =
                make_float4(acc[0] + (hb ? b1l[r0] : 0.0f), acc[1] + (hb ? b1l[r0 + 1u] : 0.0f),
                            acc[2] + (hb ? b1l[r0 + 2u] : 0.0f), acc[3] + (hb ? b1l[r0 + 3u] : 0.0f));
          }
        }
        acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        cg = nxt;
      }
      // pass barrier (every wave): the pass's SwiGLU rows (K-parts summed in part order) complete;
      // then the next pass's token rows are staged
      lds_barrier();
      if (ks1 > 1u) {
        const uint32_t nf = nt1 * 8u;
        for (uint32_t i = threadIdx.x; i < mt * nf; i += NTH) {
          const uint32_t j = i / nf, f = i - j * nf;
          float g = pre[(size_t)j * PR + 2u * f], l = pre[(size_t)j * PR + 2u * f + 1u];
          for (uint32_t hh = 1; hh < ks1; ++hh) {
            g = g + pre[((size_t)hh * mtm + j) * PR + 2u * f];
            l = l + pre[((size_t)hh * mtm + j) * PR + 2u * f + 1u];
          }
          uint16_t t[NT];
          split_bf16<NT>(swiglu_clamp_f(g, l, a.alpha, a.limit), t);
#pragma unroll
          for (int term = 0; term < NT; ++term) act[((size_t)term * 16u + m0 + j) * AF + f] = t[term];
        }
        lds_barrier();
      }
      if (p + 1u < npass) {
        stage(p + 1u, false);
        __syncthreads();
      }
    }

    // ---- phase 2: this wave's W2 row tiles over the slice's K-groups, all tokens
    const uint32_t n2 = (r_hi - r_lo) * kpr;
    uint32_t crt = r_lo, ckk = 0;
    for (uint32_t g0 = 0; g0 < n2; g0 += CJ) {
#pragma unroll
      for (uint32_t j = 0; j < CJ; ++j) {
        if (g0 + j < n2) {
          const uint32_t kg = kg2_lo + ckk, blk = 4u * kg + q;
          const bool ok = blk >= b_lo && blk < b_hi;
          const float sc = ok ? e8m0_to_f32((sbuf[j] >> sshift) & 0xFFu) : 0.0f;
          mfma_slot(j, sc, (const unsigned char *)act, ok ? act_lane + (4u * kg - b_lo) * 64u : act_row, act_tstride);
          if (++ckk == kpr) {  // the row tile's epilogue: partial rows of the expert's slots
            const uint32_t r0 = 16u * crt + 4u * q;
            if (i16 < M && r0 < a.D) {
              float *o = a.out + (size_t)s * a.slice_stride + (size_t)slot_l[i16] * a.out_stride + r0;
              const bool bz = s == 0u;  // b2 once, with slice 0
              const float v0 = acc[0] + (bz ? b2l[r0] : 0.0f), v1 = acc[1] + (bz ? b2l[r0 + 1u] : 0.0f);
              const float v2 = acc[2] + (bz ? b2l[r0 + 2u] : 0.0f), v3 = acc[3] + (bz ? b2l[r0 + 3u] : 0.0f);
              if (r0 + 3u < a.D) {
                *(float4 *)o = make_float4(v0, v1, v2, v3);
              } else {
                o[0] = v0;
                if (r0 + 1u < a.D) o[1] = v1;
                if (r0 + 2u < a.D) o[2] = v2;
              }
            }
            acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            ckk = 0u;
            ++crt;
          }
        }
        gen_slot(j, abuf[j], sbuf[j]);
        __builtin_amdgcn_sched_barrier(0);
      }
      gen_step();
    }
    __syncthreads();  // the LDS areas are free for the next item
  }
}

// ---------------------------------------------------------------------------------------------
// combine_slices_kernel: y[t, d] = (add_residual ? x[t, d] : 0) + sum_{p asc} w_p * v_p[d] with
// v_p = the slot row t * K + p summed over the fused kernel's slices in order (slice 0 first, b2
// included there).  Thread (quad c of the row, slot p) requests its slices' quads together (in
// batches of 16); the G = K rounded up to a power of two lanes of a quad then meet in lane p = 0
// by shuffles, in p order.
// ---------------------------------------------------------------------------------------------
template <typename XT, int G>
__global__ __launch_bounds__(256) void combine_slices_kernel(CombineArgs a) {
  const uint32_t t = blockIdx.y;
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t c = gid / G, p = gid % G;
  const uint32_t d0 = c * 4u;
  const uint32_t pp = min(p, a.K - 1u);
  const bool live = d0 < a.D;
  const uint32_t dd = live ? d0 : 0u;
  const uint32_t nparts = fused_slices(a.slice_grid, (uint32_t)*a.num_active, a.slice_cap);
  const float *base = (const float *)a.ypart + ((size_t)t * a.K + pp) * a.Dp + dd;
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (uint32_t s0 = 0; s0 < nparts; s0 += 16u) {
    float4 r[16];
#pragma unroll
    for (uint32_t u = 0; u < 16u; ++u) r[u] = *(const float4 *)(base + (size_t)min(s0 + u, nparts - 1u) * a.part_stride);
#pragma unroll
    for (uint32_t u = 0; u < 16u; ++u) {
      if (s0 + u >= nparts) break;
      if (s0 + u == 0u) {
        v = r[0];
      } else {
        v = make_float4(v.x + r[u].x, v.y + r[u].y, v.z + r[u].z, v.w + r[u].w);
      }
    }
  }
  const float w = p < a.K ? a.topk_w[(size_t)t * a.K + p] : 0.0f;
  // lane p of the quad group: its weighted slot row; lane 0 sums them in p order
  const float4 wv = make_float4(v.x * w, v.y * w, v.z * w, v.w * w);
  const uint32_t lane0 = (threadIdx.x & 63u) & ~(uint32_t)(G - 1);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int k = 0; k < G; ++k) {
    const float4 o = make_float4(__shfl(wv.x, (int)lane0 + k, 64), __shfl(wv.y, (int)lane0 + k, 64),
                                 __shfl(wv.z, (int)lane0 + k, 64), __shfl(wv.w, (int)lane0 + k, 64));
    if ((uint32_t)k < a.K) acc = make_float4(acc.x + o.x, acc.y + o.y, acc.z + o.z, acc.w + o.w);
  }
  if (p != 0u || !live) return;
  const uint32_t nv = min(4u, a.D - d0);
  const float av[4] = {acc.x, acc.y, acc.z, acc.w};
  const XT *x = (const XT *)a.x;
  XT *y = (XT *)a.y;
  for (uint32_t j = 0; j < nv; ++j) {
    const size_t i = (size_t)t * a.D + d0 + j;
    const float xv = a.add_residual ? ld_val(x, i) : 0.0f;
    st_val(y, i, xv + av[j]);
  }
}

}  // namespace

// Launch geometry of the fused kernel for a batch of n tokens (decode sizes): one workgroup per
// CU; the partial slot rows of all slices within kFusedPartBytes (nsl_cap); LDS for the widest
// slice the device can choose (the fewest slices: at max_active active experts).
bool fused_geometry(uint32_t nb1, uint32_t nb2, uint32_t nrt2, uint32_t Dp, uint32_t num_cus, uint32_t max_active,
                    uint32_t topk, uint64_t n, int nt, FusedGeom &g) {
  if (n == 0 || n > kSmallRouteMaxTokens || (nt != 1 && nt != 2) || nb1 == 0 || nb2 == 0 || nrt2 == 0 ||
      max_active == 0 || num_cus == 0 || topk == 0)
    return false;
  g.grid = num_cus;
  const uint64_t row_bytes = n * topk * (uint64_t)Dp * 4u;
  g.nsl_cap = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(nb2, kFusedPartBytes / row_bytes));
  const uint32_t nsl_min = std::max(1u, std::min(num_cus / max_active, g.nsl_cap));
  g.sb_max = (nb2 + nsl_min - 1u) / nsl_min;
  g.mt = (uint32_t)std::min<uint64_t>(n, 8u);
  g.lds = fused_lds(nt, g.sb_max, g.mt, nb1, nrt2 * 16u).total;
  return g.lds <= 160u * 1024u;
}

hipError_t launch_fused(const FusedArgs &a, const FusedGeom &g, int nt, bool x_bf16, hipStream_t s) {
  if (g.grid == 0 || a.mt_max != g.mt || a.mt_max == 0 || a.mt_max > 8u || a.sb_max != g.sb_max ||
      a.nsl_cap != g.nsl_cap || a.D == 0 || a.D > a.nrt2 * 16u || a.b1_es < 4u)
    return hipErrorInvalidValue;
  const dim3 grid(g.grid), block(kFusedWaves * 64u);
  if (nt == 1)
    (void)(x_bf16 ? launch_kernel(moe_fused_kernel<1, uint16_t>, grid, block, g.lds, s, a)
                  : launch_kernel(moe_fused_kernel<1, float>, grid, block, g.lds, s, a));
  else if (nt == 2)
    (void)(x_bf16 ? launch_kernel(moe_fused_kernel<2, uint16_t>, grid, block, g.lds, s, a)
                  : launch_kernel(moe_fused_kernel<2, float>, grid, block, g.lds, s, a));
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_combine_slices(const CombineArgs &a, bool x_bf16, hipStream_t s) {
  if (a.K == 0 || a.K > 8u || a.D == 0 || !a.num_active || a.slice_grid == 0 || a.slice_cap == 0) return hipErrorInvalidValue;
  const uint32_t G = a.K <= 1u ? 1u : a.K <= 2u ? 2u : a.K <= 4u ? 4u : 8u;
  const uint64_t threads = (uint64_t)((a.D + 3u) / 4u) * G;
  const dim3 grid((uint32_t)((threads + 255u) / 256u), a.n), block(256);
#define BX_CS(G_) \
  (x_bf16 ? launch_kernel(combine_slices_kernel<uint16_t, G_>, grid, block, 0, s, a) \
          : launch_kernel(combine_slices_kernel<float, G_>, grid, block, 0, s, a))
  if (G == 1u) (void)BX_CS(1);
  else if (G == 2u) (void)BX_CS(2);
  else if (G == 4u) (void)BX_CS(4);
  else (void)BX_CS(8);
#undef BX_CS
  return hipGetLastError();
}

hipError_t configure_fused_kernels() {
  const int big = 160 * 1024;
  hipError_t err = hipSuccess;
  auto set = [&](const void *f) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, big);
    if (e != hipSuccess && err == hipSuccess) err = e;
  };
  set((const void *)moe_fused_kernel<1, uint16_t>);
  set((const void *)moe_fused_kernel<1, float>);
  set((const void *)moe_fused_kernel<2, uint16_t>);
  set((const void *)moe_fused_kernel<2, float>);
  return err;
}

}  // namespace burnext
