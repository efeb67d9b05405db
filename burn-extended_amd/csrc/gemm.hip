// gemm.hip -- grouped expert GEMM of prefill-sized batches on gfx950's block-scaled MFMA.
//
// replaces w1_swiglu_dense_kernel / w2_scatter_dense_kernel (src/quant/gpu.rs:89-192) for
// batches whose expert segments hold many tokens (the reference runs them per 256-token tile
// and per used expert, src/moe/mod.rs:262-404).
//
// v_mfma_scale_f32_16x16x128_f8f6f4 with A = MXFP4 weights (cbsz 4) and B = activations as an
// MXFP8 hi term (blgp 0) and an MXFP4 lo term (blgp 4), e8m0 block scales applied by the matrix
// core:
//   A: lane l = 16 g + i holds row i, K [32 g, 32 g + 32) as 16 bytes (low nibble first) -- one
//      K-group of the tiled weight layout, loaded straight into registers -- and that block's
//      scale.
//   B hi (fp8): lane l = 16 g + j holds column (token) j, K [16 g, 16 g + 16) in bytes 0-15 and
//      K [64 + 16 g, 64 + 16 g + 16) in bytes 16-31; B lo (fp4): lane l holds K [32 g, 32 g + 32)
//      of column j as 16 bytes, as A does; each term's scale operand is its scale of
//      K [32 g, 32 g + 32) of column j.
//   C: lane l = 16 q + j holds rows 4 q .. 4 q + 3 of column j.
// Activations are two terms (hi + lo), so each product is two MFMAs into one accumulator.
#include <type_traits>

#include "kernels.hpp"
#include "mx_device.hpp"

namespace burnext {

typedef int32_t i32x8_t __attribute__((ext_vector_type(8)));
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

namespace {
// One pipeline stage (one 128-wide K-group of the activations; the weights bypass LDS) in LDS:
//   B hi codes [token 64][slot 8] x 16 bytes, chunk c of token t in slot c ^ ((t >> 1) & 7):
//     a fill instruction reads 8 whole 128-byte rows (coalesced) and the 16 lanes reading one
//     chunk of 16 consecutive tokens hit 16 distinct 16-byte bank groups;
//   B lo codes [token 64][slot 4] x 16 bytes (64-byte fp4 rows), chunk c of token t in slot
//     c ^ ((t >> 2) & 2): a fill instruction reads 16 whole rows, and the operand reads are free
//     of bank conflicts (slot c ^ ((t >> 2) & 3) measured 2-way conflicted on gfx950).
// The B scales come in blocks of 4 K-groups, outside the stage ring: two slots (double buffer)
// of [term 2][token 64][16 bytes] (byte 4 k + g = scale of K [32 g, 32 g + 32) of K-group 4 j + k
// of block j).  One 16-byte fill instruction per wave and block (32 tokens of one term, the
// upper 32 lanes masked) replaces four gathers of 4-byte pieces: the gathers' per-row cost in the
// address and data paths took 35 of gate_up's 412 us at C3.
constexpr uint32_t kRowTiles = kGemmRows / 16u;
constexpr uint32_t kBHi = 8u * kGemmTok * 16u;
constexpr uint32_t kBData = kBHi + 4u * kGemmTok * 16u;
constexpr uint32_t kStage = kBData;
constexpr uint32_t kStages = 5;
constexpr uint32_t kScaleSlot = 2u * kGemmTok * 16u;
constexpr uint32_t kScaleRing = 2u * kScaleSlot;
constexpr uint32_t kWaves = 4;
static_assert(kGemmTok == 64, "four waves of 64 x 64 tiles cover 256 rows x 64 tokens");
typedef __attribute__((address_space(3))) void lds_void;
// s_waitcnt with vmcnt(n) only (expcnt and lgkmcnt left at their maxima), n < 64
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
// s_waitcnt lgkmcnt(0) only (vmcnt and expcnt left at their maxima)
constexpr int kLgkmcnt0 = 0xF | (7 << 4) | (3 << 14);

// Clamped SwiGLU with the hardware exp2 and reciprocal (about 1 ulp each): the epilogue feeds it
// straight into the two-term quantisation (2^-6-level), so the precise expf and division
// of swiglu_clamp_f would only cost VALU time there.
__device__ __forceinline__ float swiglu_clamp_fast(float g, float l, float alpha, float limit) {
  const float xg = fminf(g, limit);
  const float xl = fmaxf(-limit, fminf(l, limit));
  const float sig = __builtin_amdgcn_rcpf(1.0f + __expf(-alpha * xg));
  return (xg * sig) * (xl + 1.0f);
}

// Maximum over lanes l, l ^ 16, l ^ 32 and l ^ 48 (the four lane groups q of a token column), by
// the permlane swaps between rows 16 and 32 lanes apart.
__device__ __forceinline__ float max_lanes_16_32(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const auto p2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p2[0]), __uint_as_float(p2[1]));
}

// Barrier of the stage ring.  Each wave has already waited (vmcnt) for its own direct-to-LDS
// loads of the stage the others read next; its LDS reads are complete (lgkmcnt(0)) before it
// arrives, so a slot refilled after the barrier has no pending readers.  Loads of later stages
// stay in flight: __syncthreads() would wait for every outstanding load (its fence covers the
// direct-to-LDS writes).  The empty asm statements keep the compiler from moving memory
// accesses across.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kLgkmcnt0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
}  // namespace

size_t gemm_lds_bytes() { return (size_t)kStages * kStage + kScaleRing + 2 * kGemmTok * 4 + 64 + 2 * (kMaxExperts + 1) * 4; }

// Work item of workgroup b: blockIdx is remapped so that the workgroups of one XCD (b mod 8)
// take a contiguous run of Q = ceil(N / 8) of the N realised items (N = nrb * token tiles, read
// from tile_off[E]; the grid is sized for the most tiles routing can produce, and sizing the runs
// by the grid left the last XCD a small remainder while the other seven did all the work).  Items
// go in groups of 8 token tiles: row block rb of the group's tiles, tiles fastest, so the ~64
// workgroups an XCD runs at once share about 8 row blocks of weights and 8 tiles of activations
// in its L2 (gate_up HBM reads 2.1 -> 1.0 GB per launch at C3 against row blocks fastest).
// A workgroup (4 waves; two workgroups per CU, whose K-loops drift apart, so one's LDS reads
// and waits overlap the other's MFMAs) computes kGemmRows weight rows (16 row tiles) x kGemmTok
// tokens; wave w computes rows 64 w .. 64 w + 63 (4 x 4 MFMA tiles of 16 x 16, two terms each).
// Weights go straight from the tiled layout into registers, two K-groups ahead (two register
// sets), their scales from the GEMM scale copy (one 16-byte load per wave and 4 K-groups, the byte
// picked by the MFMA's op_sel; the K-loop is unrolled by 4 for it); activations stream through a 5-stage LDS ring filled by direct-to-LDS loads four
// K-groups ahead (3 instructions per wave per stage, and one per 4 K-groups for the scales);
// one barrier per K-group.
template <bool GATE_UP>
__global__ __launch_bounds__(256, 2) void expert_gemm_kernel(GemmArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint8_t *scl = smem + kStages * kStage;                      // B scale blocks [slot 2]
  int32_t *rows_l = (int32_t *)(scl + kScaleRing);              // [kGemmTok] B row, -1 = none
  int32_t *slot_l = rows_l + kGemmTok;                     // [kGemmTok] down: slot
  int32_t *info_l = slot_l + kGemmTok;                     // [0] expert [1] tile of it
  int32_t *toff_l = info_l + 16;                           // [E + 1] tile_off
  int32_t *soff_l = toff_l + kMaxExperts + 1;              // [E + 1] seg_off

  // one round trip for both prefixes (E + 1 <= 257 entries each), then the item and its expert
  // from LDS
  for (uint32_t t = threadIdx.x; t <= a.E; t += blockDim.x) {
    toff_l[t] = a.tile_off[t];
    soff_l[t] = a.seg_off[t];
  }
  if (threadIdx.x == 0) info_l[0] = -1;
  __syncthreads();
  const uint32_t b = blockIdx.x;
  const uint32_t NT = (uint32_t)toff_l[a.E];
  const uint32_t N = a.nrb * NT, Q = (N + 7u) / 8u;  // 8 * Q <= gridDim.x
  const uint32_t it = (b & 7u) * Q + (b >> 3);
  if ((b >> 3) >= Q || it >= N) return;  // workgroup-uniform: no item
  // items in groups of 8 token tiles: row block rb of the group's tiles, tiles fastest
  const uint32_t grp = it / (8u * a.nrb), r = it - grp * 8u * a.nrb;
  const uint32_t gsz = min(8u, NT - grp * 8u);
  const uint32_t rb = r / gsz, gt = grp * 8u + (r - rb * gsz);
  for (uint32_t e = threadIdx.x; e < a.E; e += blockDim.x) {
    const uint32_t lo = (uint32_t)toff_l[e], hi = (uint32_t)toff_l[e + 1];
    if (gt >= lo && gt < hi) {
      info_l[0] = (int32_t)e;
      info_l[1] = (int32_t)(gt - lo);
    }
  }
  __syncthreads();
  const int e = info_l[0];
  if (e < 0) return;  // workgroup-uniform: beyond the realised token tiles
  const int seg0 = soff_l[e];
  const uint32_t M = (uint32_t)(soff_l[e + 1] - seg0);
  const uint32_t m0 = (uint32_t)info_l[1] * kGemmTok;
  const uint32_t ntok = min(kGemmTok, M - m0);
  // B rows: gate_up reads token rows (slot / topk of the segment entries, one more round trip);
  // down reads the segment's own rows, and its output slots are needed only by the epilogue, so
  // their load is waited for after the K-loop
  static_assert(kGemmTok <= 256, "one segment entry per thread");
  // every thread loads (clamped index: no branch around the load); entries >= ntok are dropped
  const int32_t slot_own = a.perm[seg0 + (int32_t)min(m0 + threadIdx.x, M - 1u)];
  if (threadIdx.x < kGemmTok) {
    const uint32_t i = threadIdx.x;
    if (GATE_UP)
      rows_l[i] = i < ntok ? slot_own / (int32_t)a.topk : -1;
    else
      rows_l[i] = i < ntok ? seg0 + (int32_t)(m0 + i) : -1;
  }
  ring_barrier();  // rows_l written (LDS); down's slot load stays in flight

  const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
  const uint32_t wr = wv;  // this wave's 64-row quarter of the workgroup's rows
  const uint32_t i16 = lane & 15u, q = lane >> 4;
  const uint32_t nkg = (a.nb + 3u) >> 2, tail = a.nb - 4u * (nkg - 1u);
  const uint32_t kq = a.b.kq, ss = a.b.ss;  // code bytes and scale bytes per B row
  const uint8_t *wexp = a.wb + (size_t)e * a.wb_estride;
  const uint8_t *sexp = a.ws + (size_t)e * a.ws_estride;
  auto lane_ok = [&](uint32_t kg) { return kg < nkg && q < (kg + 1u == nkg ? tail : 4u); };

  // ---- stage fill by direct-to-LDS loads.  Token columns beyond the tile read the tile's first
  // row and row tiles beyond the expert its last one; their results are never stored.
  // B hi codes: instruction m (< 2) of wave wv fills tokens 8 (wv + 4 m) + lane / 8; this lane's
  // two tokens and its swizzled chunk.  B lo codes: wave wv's one instruction fills tokens
  // 16 wv + lane / 4, chunk lane & 3 into slot (lane & 3) ^ ((token >> 2) & 2).  On gfx950 the
  // operand reads of this layout are conflict free, while slot (lane & 3) ^ ((token >> 2) & 3),
  // free under a plain 64-bank model, measured 2-way conflicted (LDS bank-conflict counters over
  // all 256 XOR maps of token bits into the slot: only token bits 2-3 matter, and bit 3 alone
  // into slot bit 1 is one of the conflict-free maps).
  const uint32_t tk0 = 8u * wv + (lane >> 3), tk1 = tk0 + 32u;
  const int32_t rk0 = rows_l[tk0], rk1 = rows_l[tk1];
  const size_t browk0 = (size_t)(rk0 >= 0 ? rk0 : rows_l[0]) * kq, browk1 = (size_t)(rk1 >= 0 ? rk1 : rows_l[0]) * kq;
  const uint32_t bchunk = ((lane & 7u) ^ ((tk0 >> 1) & 7u)) * 16u;  // tk1 has the same swizzle
  const uint32_t tkl = 16u * wv + (lane >> 2);
  const int32_t rkl = rows_l[tkl];
  const size_t browl = (size_t)(rkl >= 0 ? rkl : rows_l[0]) * (kq / 2u);
  const uint32_t lchunk = ((lane & 3u) ^ ((tkl >> 2) & 2u)) * 16u;
  // B scale blocks: term wv / 2, token 32 (wv % 2) + lane (lanes < 32)
  const int32_t rsl = rows_l[32u * (wv & 1u) + (lane & 31u)];
  const size_t rows = (size_t)(rsl >= 0 ? rsl : rows_l[0]);
  // this wave's 4 row tiles (clamped to the expert's last) and their group in the GEMM's scale
  // copy (clamped to the last group: rows beyond the expert are never stored)
  const uint8_t *arow[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const uint32_t t = min(rb * kRowTiles + wr * 4u + (uint32_t)rt, a.nrt - 1u);
    arow[rt] = wexp + (size_t)t * a.nb * 256u + lane * 16u;
  }
  const uint32_t nkq = (nkg + 3u) >> 2, ngr = (a.nrt + 3u) >> 2;
  const uint8_t *srow = sexp + (size_t)min(rb * (kRowTiles / 4u) + wr, ngr - 1u) * nkq * 1024u + lane * 16u;
  auto stage = [&](uint32_t kg, uint32_t p) {
    uint8_t *st = smem + p * kStage;
#pragma unroll
    for (int m = 0; m < 2; ++m) {  // B hi codes: token group wv + 4 m
      const uint32_t tg = wv + 4u * (uint32_t)m;
      const uint8_t *src = a.b.hi + (m ? browk1 : browk0) + kg * 128u + bchunk;
      __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(st + tg * 64u * 16u), 16, 0, 0);
    }
    {  // B lo codes: tokens 16 wv .. 16 wv + 15
      const uint8_t *src = a.b.lo + browl + kg * 64u + lchunk;
      __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(st + kBHi + wv * 1024u), 16, 0, 0);
    }
  };
  // B scale block j (K-groups 4 j .. 4 j + 3) into slot p: 16 bytes per token and term
  auto stage_scales = [&](uint32_t j, uint32_t p) {
    const uint8_t *src = (wv >= 2u ? a.b.slo : a.b.shi) + rows * ss + j * 16u;
    if (lane < 32u)
      __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(scl + p * kScaleSlot + wv * 512u), 16, 0, 0);
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc[rt][tt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // MFMA operands: the A operands (row tiles) of a K-group, and the B operands of one token tile.
  // The A scales of 4 K-groups come in one 16-byte load (dword rt: byte k = K-group 4 j + k of row
  // tile rt); the MFMA picks byte k by the scale operand's op_sel.
  struct AFrag {
    i32x4_t A[4];
  };
  struct BFrag {
    i32x8_t Bh, Bl;
    int32_t sbh, sbl;
  };
  const i32x4_t z4 = {0, 0, 0, 0};
  // A straight from the tiled weights into registers.  Lanes outside the last K-group's blocks read
  // the row tile's first block (finite fp4 codes; their scale byte in the copy is 0): the B rows
  // are zero beyond K (codes 0 in the K padding of xq and act), so their products add zeros.
  auto load_a = [&](uint32_t kg, AFrag &f) {
    const uint32_t off = lane_ok(kg) ? kg * 1024u : 0u;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) f.A[rt] = *(const i32x4_t *)(arow[rt] + off);
    __builtin_amdgcn_sched_barrier(0);  // the wait counts below assume this issue order
  };
  // A scales of K-groups 4 j .. 4 j + 3 (lanes beyond the blocks read scale byte 0)
  auto load_as = [&](uint32_t j, i32x4_t &s4) {
    s4 = *(const i32x4_t *)(srow + j * 1024u);
    __builtin_amdgcn_sched_barrier(0);
  };

  // st: the K-group's stage; sc: its scale block slot plus 4 (K-group mod 4)
  auto read_b = [&](const uint8_t *st, const uint8_t *sc, int tt, BFrag &f) {
    const uint32_t tok = (uint32_t)tt * 16u + i16;
    // lane group q: hi chunks q and 4 + q (K [16 q, +16) and [64 + 16 q, +16)); lo chunk q
    // (K [32 q, +32))
    const uint32_t sw = (tok >> 1) & 7u;
    const uint8_t *r = st + tok * 128u;
    const uint32_t s1 = (q ^ sw) * 16u, s2 = ((4u + q) ^ sw) * 16u;
    const i32x4_t h0 = *(const i32x4_t *)(r + s1), h1 = *(const i32x4_t *)(r + s2);
    const i32x4_t l0 = *(const i32x4_t *)(st + kBHi + tok * 64u + (q ^ ((tok >> 2) & 2u)) * 16u);
    f.Bh = __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7);
    f.Bl = __builtin_shufflevector(l0, z4, 0, 1, 2, 3, 4, 5, 6, 7);
    f.sbh = sc[tok * 16u + q];
    f.sbl = sc[kGemmTok * 16u + tok * 16u + q];
  };
  // KP: the K-group's position in its scale block, the op_sel byte of the A scale dwords
  auto mma = [&](const AFrag &fa, const i32x4_t &sa, const BFrag &fb, int tt, auto KP) {
    constexpr int kp = (int)decltype(KP)::value;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const i32x8_t A8 = __builtin_shufflevector(fa.A[rt], z4, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[rt][tt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A8, fb.Bh, acc[rt][tt], 4, 0, kp, sa[rt], 0, fb.sbh);
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const i32x8_t A8 = __builtin_shufflevector(fa.A[rt], z4, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[rt][tt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A8, fb.Bl, acc[rt][tt], 4, 4, kp, sa[rt], 0, fb.sbl);
    }
  };

  // the epilogue's bias rows (4 row tiles of this wave), requested before the first stage so that
  // they have long arrived when the K-loop ends (loads complete in order: the first stage wait
  // covers them)
  f32x4_t bias4[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const uint32_t r0 = rb * kGemmRows + wr * 64u + (uint32_t)rt * 16u + 4u * q;
    bias4[rt] = *(const f32x4_t *)(a.bias + (size_t)e * a.bias_estride + min(r0, a.bias_estride - 4u));
  }
  // B stages of K-groups 0..3 and scale block 0, then A of K-group 0, A scale block 0 and A of
  // K-group 1 (loads complete in order).  The compiler must not reorder these groups: the
  // s_waitcnt counts below assume this issue order.
#pragma unroll
  for (uint32_t j = 0; j < kStages - 1u; ++j) stage(min(j, nkg - 1u), j);
  stage_scales(0, 0);
  __builtin_amdgcn_sched_barrier(0);
  AFrag ar0, ar1;
  i32x4_t sa_cur, sa_nxt;  // A scales of the current block, and of the next (loaded at position 2)
  load_a(0, ar0);
  load_as(0, sa_cur);
  load_a(min(1u, nkg - 1u), ar1);
  __builtin_amdgcn_s_waitcnt(vmcnt_only(4));  // A(0), its scales and every B stage before them landed
  ring_barrier();
  // K-group kg at position P = kg mod 4 of its scale block (a compile-time constant: the block
  // loads, one per 4 K-groups, change the wait count)
  auto iter = [&](uint32_t kg, AFrag &ar, auto P) {
    constexpr uint32_t kP = decltype(P)::value;
    stage(min(kg + kStages - 1u, nkg - 1u), (kg + kStages - 1u) % kStages);  // the slot every wave left
    // the next scale block into the slot of the previous one (every wave is past its last K-group)
    if constexpr (kP == 0u) stage_scales(min((kg >> 2) + 1u, (nkg - 1u) >> 2), ((kg >> 2) + 1u) & 1u);
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t *st = smem + (kg % kStages) * kStage;
    const uint8_t *sc = scl + ((kg >> 2) & 1u) * kScaleSlot + kP * 4u;
    BFrag b0, b1;
    // the operand reads and MFMAs at raised wave priority, so that the other workgroup's waves on
    // the SIMD issue their loads around them (C3 gate_up 402 -> 397 us, down 217.6 -> 216.0 us)
    __builtin_amdgcn_s_setprio(1);
    read_b(st, sc, 0, b0);
    read_b(st, sc, 1, b1);
    mma(ar, sa_cur, b0, 0, P);
    read_b(st, sc, 2, b0);
    mma(ar, sa_cur, b1, 1, P);
    read_b(st, sc, 3, b1);
    mma(ar, sa_cur, b0, 2, P);
    mma(ar, sa_cur, b1, 3, P);
    // schedule: tile 0's operand reads, then each next tile's reads one by one between the MFMAs
    // of the tile before it (gate_up 474 -> 468 us at C3 against the compiler's own order)
    __builtin_amdgcn_sched_group_barrier(0x100, 5, 0);  // 0x100: LDS reads, 0x008: MFMAs
#pragma unroll
    for (int t = 0; t < 3; ++t) {
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    __builtin_amdgcn_s_setprio(0);
    load_a(min(kg + 2u, nkg - 1u), ar);
    // at position 2, the next block's A scales (needed from K-group kg + 2 on)
    if constexpr (kP == 2u) load_as(min((kg >> 2) + 1u, nkq - 1u), sa_nxt);
    // issued after A(kg + 1): B(kg + 4), at position 0 a B scale block, A(kg + 2) and at position 2
    // the A scale block (3 [+ 1] + 4 [+ 1]); B(kg + 1) and kg + 1's B scale block went out before
    // A(kg + 1).  At position 3 the A scale block issued after A(kg + 1) is waited for too (3 + 4).
    __builtin_amdgcn_s_waitcnt(vmcnt_only(kP == 0u || kP == 2u ? 8 : 7));
    if constexpr (kP == 3u) sa_cur = sa_nxt;
    ring_barrier();
  };
  using P0 = std::integral_constant<uint32_t, 0>;
  using P1 = std::integral_constant<uint32_t, 1>;
  using P2 = std::integral_constant<uint32_t, 2>;
  using P3 = std::integral_constant<uint32_t, 3>;
  uint32_t kg = 0;
  for (; kg + 3u < nkg; kg += 4u) {
    iter(kg, ar0, P0{});
    iter(kg + 1u, ar1, P1{});
    iter(kg + 2u, ar0, P2{});
    iter(kg + 3u, ar1, P3{});
  }
  if (kg < nkg) iter(kg, ar0, P0{});
  if (kg + 1u < nkg) iter(kg + 1u, ar1, P1{});
  if (kg + 2u < nkg) iter(kg + 2u, ar0, P2{});
  __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // the trailing reloads have landed
  if (!GATE_UP) {
    if (threadIdx.x < kGemmTok) slot_l[threadIdx.x] = threadIdx.x < ntok ? slot_own : -1;
    __syncthreads();
  }

  // ---- epilogue: results are staged in LDS (the stage ring is free once every wave's last
  // direct-to-LDS loads have landed) and leave as whole 16-byte row segments: scattered 1-, 2- and
  // 8-byte stores write each line piecewise
  ring_barrier();
  uint8_t *ep = smem;
  if constexpr (GATE_UP) {
    // wave wr owns features rb*128 + wr*32 .. +32: one MX block per token.  Lane (q, j) holds
    // features 8 rt + 2 q + {0, 1} (interleaved gate/linear row pairs) of its token columns.
    // LDS: hi codes [token 64][128], lo codes [token 64][64], scale bytes [term 2][token 64][4].
    constexpr uint32_t kHs = 144u, kLs = 80u;  // padded LDS row strides: few bank conflicts for the per-lane writes
    uint8_t *hi_l = ep, *lo_l = ep + kGemmTok * kHs, *sc_l = ep + kGemmTok * (kHs + kLs);
    const uint32_t fb = rb * (kGemmRows / 2u) + wr * 32u;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const uint32_t tok = (uint32_t)tt * 16u + i16;
      float o[8];
      float amax = 0.0f;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const bool rv = rb * kRowTiles + wr * 4u + (uint32_t)rt < a.nrt;
        const f32x4_t bb = bias4[rt];
        const uint32_t f0 = fb + (uint32_t)rt * 8u + 2u * q;
        float v0 = swiglu_clamp_fast(acc[rt][tt][0] + bb[0], acc[rt][tt][1] + bb[1], a.alpha, a.limit);
        float v1 = swiglu_clamp_fast(acc[rt][tt][2] + bb[2], acc[rt][tt][3] + bb[3], a.alpha, a.limit);
        v0 = (rv && f0 < a.act_feats) ? v0 : 0.0f;
        v1 = (rv && f0 + 1u < a.act_feats) ? v1 : 0.0f;
        o[2 * rt] = v0;
        o[2 * rt + 1] = v1;
        amax = fmaxf(amax, fmaxf(fabsf(v0), fabsf(v1)));
      }
      amax = max_lanes_16_32(amax);
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
      rmax = max_lanes_16_32(rmax);
      const uint32_t sbl = mx4_scale_byte(rmax);
      const float sl = mx4_divisor(sbl);
      // lo: features 8 k + 2 q and 8 k + 2 q + 1 of the block are one byte of e2m1 codes
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        *(uint16_t *)(hi_l + tok * kHs + wr * 32u + 8u * k + 2u * q) = (uint16_t)ch[k];
        lo_l[tok * kLs + wr * 16u + 4u * k + q] = (uint8_t)e2m1x2<0>(0u, res[2 * k], res[2 * k + 1], sl);
      }
      if (q == 0) {
        sc_l[tok * 4u + wr] = (uint8_t)sbh;
        sc_l[(kGemmTok + tok) * 4u + wr] = (uint8_t)sbl;
      }
    }
    __syncthreads();
    // rows seg0 + m0 + tok (consecutive): hi 128 bytes, lo 64 bytes and 4 + 4 scale bytes each
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (uint32_t m = 0; m < 2u; ++m) {
      const uint32_t c = t + 256u * m, tok = c >> 3, part = c & 7u;
      if (tok < ntok) {
        const size_t row = (size_t)(seg0 + (int32_t)(m0 + tok));
        *(uint4 *)(a.act.hi + row * a.act.kq + rb * 128u + 16u * part) = *(const uint4 *)(hi_l + tok * kHs + 16u * part);
      }
    }
    {
      const uint32_t tok = t >> 2, part = t & 3u;
      if (tok < ntok) {
        const size_t row = (size_t)(seg0 + (int32_t)(m0 + tok));
        *(uint4 *)(a.act.lo + row * (a.act.kq / 2u) + rb * 64u + 16u * part) = *(const uint4 *)(lo_l + tok * kLs + 16u * part);
      }
    }
    if (t < 2u * kGemmTok) {
      const uint32_t term = t / kGemmTok, tok = t - term * kGemmTok;
      if (tok < ntok) {
        const size_t row = (size_t)(seg0 + (int32_t)(m0 + tok));
        *(uint32_t *)((term ? a.act.slo : a.act.shi) + row * a.act.ss + rb * 4u) = *(const uint32_t *)(sc_l + (term * kGemmTok + tok) * 4u);
      }
    }
    // zero the K padding of the act rows beyond the last row block's features
    if (rb + 1u == a.nrb) {
      const uint32_t f_end = a.nrb * (kGemmRows / 2u), padb = a.act.kq - f_end;  // multiple of 32
      for (uint32_t i = threadIdx.x; i < ntok * padb; i += blockDim.x) {
        const uint32_t tk = i / padb, c = i - tk * padb;
        const size_t row = (size_t)(seg0 + (int32_t)(m0 + tk));
        a.act.hi[row * a.act.kq + f_end + c] = 0;
        if ((c & 1u) == 0u) a.act.lo[row * (a.act.kq / 2u) + (f_end + c) / 2u] = 0;
        if ((c & 31u) == 0u) {
          a.act.shi[row * a.act.ss + ((f_end + c) >> 5)] = 0;
          a.act.slo[row * a.act.ss + ((f_end + c) >> 5)] = 0;
        }
      }
    }
  } else {
    // token-major slot rows t * topk + p in bf16 (the layer output is bf16 on this path), expert
    // bias b2 added once.  LDS: [token 64][256 rows] bf16.
    constexpr uint32_t kOs = 264u;  // padded row stride (elements)
    uint16_t *o_l = (uint16_t *)ep;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const uint32_t tok = (uint32_t)tt * 16u + i16;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const uint32_t rl = wr * 64u + (uint32_t)rt * 16u + 4u * q;  // row within the block
        const f32x4_t bb = bias4[rt];
        uint16_t o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = f32_to_bf16_bits(acc[rt][tt][r] + bb[r]);
        *(uint2 *)(o_l + tok * kOs + rl) = make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
      }
    }
    __syncthreads();
    // 64 tokens x 32 chunks of 8 rows
    for (uint32_t c = threadIdx.x; c < kGemmTok * 32u; c += blockDim.x) {
      const uint32_t tok = c >> 5, part = c & 31u;
      if (tok >= ntok) continue;
      const uint32_t r0 = rb * kGemmRows + 8u * part;
      if (r0 >= a.out_rows) continue;
      uint16_t *orow = a.out + (size_t)slot_l[tok] * a.out_stride;
      const uint16_t *src = o_l + tok * kOs + 8u * part;
      if (r0 + 7u < a.out_rows) {
        *(uint4 *)(orow + r0) = *(const uint4 *)src;
      } else {
        for (uint32_t r = 0; r < 8u; ++r)
          if (r0 + r < a.out_rows) orow[r0 + r] = src[r];
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
  // B scale rows hold whole 16-byte blocks of 4 K-groups (ss >= kq / 32, a multiple of 16)
  if (grid == 0 || (grid & 7u) != 0 || a.nrb == 0 || a.b.kq % 128u != 0 || a.b.ss % 16u != 0 || a.b.ss * 32u < a.b.kq)
    return hipErrorInvalidValue;
  if (gate_up && (a.act.kq % 128u != 0 || a.act.ss * 32u < a.act.kq)) return hipErrorInvalidValue;
  if (gate_up)
    (void)launch_kernel(expert_gemm_kernel<true>, dim3(grid), dim3(64 * kWaves), gemm_lds_bytes(), s, a);
  else
    (void)launch_kernel(expert_gemm_kernel<false>, dim3(grid), dim3(64 * kWaves), gemm_lds_bytes(), s, a);
  return hipGetLastError();
}

}  // namespace burnext
