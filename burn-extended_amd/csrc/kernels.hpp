// kernels.hpp -- argument blocks and host-side launchers of the MoE kernels (gfx950).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace burnext {

// Per-launch timing.  While a LaunchTimer is installed on the calling thread (the layer's
// profiling scope), every launcher below binds a fresh HIP event pair to each kernel dispatch
// through hipExtLaunchKernel: the events then carry that dispatch's own begin and end timestamps
// (the kernel's execution time, the figure rocprofv3's kernel trace reports), not the stream
// positions around it.  Without a timer the launch is a plain hipLaunchKernel.
struct LaunchTimer {
  virtual bool pair(hipEvent_t &start, hipEvent_t &stop) = 0;  // false: launch untimed
  virtual ~LaunchTimer() = default;
};
extern thread_local LaunchTimer *g_launch_timer;

template <typename A>
inline hipError_t launch_kernel(void (*k)(A), dim3 grid, dim3 block, size_t lds, hipStream_t s, const A &a) {
  A arg = a;
  void *args[] = {(void *)&arg};
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (g_launch_timer && g_launch_timer->pair(e0, e1))
    return hipExtLaunchKernel((const void *)k, grid, block, args, lds, s, e0, e1, 0);
  return hipLaunchKernel((const void *)k, grid, block, args, lds, s);
}

// The grouped GEMM's activation rows (see mx_device.hpp): kq codes per row, K padded to whole
// 128-wide K-groups with zero codes and zero scale bytes, natural K order -- the hi term as MXFP8
// (kq bytes per row), the lo term as MXFP4 (kq / 2 bytes per row, two codes per byte); kq / 32
// scale bytes per row and term, in rows of ss = kq / 32 rounded up to 16 bytes (the GEMM stages
// the scales of 4 K-groups of a row with one 16-byte load; the bytes past kq / 32 are not used).
struct QRows {
  uint8_t *hi, *lo;    // [rows, kq], [rows, kq / 2]
  uint8_t *shi, *slo;  // [rows, ss]
  uint32_t kq, ss;
};

// Router logits for a block of tokens x a group of experts.  With apply_norm the rows are the
// gamma-folded router weights and logit = dot(x, gw) / r + b, r = sqrt(mean(x^2) + eps); the
// workgroups of expert group 0 also write r per token for the expert GEMV staging.
struct RouterArgs {
  const void *x;
  const void *rw;     // router weight [E, D] (f32 or bf16 bits), gamma-folded when apply_norm
  const float *rb;    // router bias [E]
  float *logits;      // [n, E]
  float *rms;         // [n] (written when apply_norm), nullable
  void *xn;           // [n, Dp] normalised rows in the x dtype (bf16 with xn_bf16; expert group 0
                      // writes), nullable
  QRows xq;           // the same rows in the GEMM's two-term form (expert group 0 writes when xq.hi)
  const float *gamma; // [D]
  uint32_t n, D, Dpad, Dp, E, tb, epw;
  float eps;
  int apply_norm;
  int xn_bf16;        // xn rows rounded to bf16 (nearest even) whatever the x dtype (router_kernel)
};

// Top-k + softmax per token (one wave per token) from logits [n, E].
struct TopkArgs {
  const float *logits;
  int32_t *topk_idx;
  float *topk_w;
  uint32_t n, E, K;
};

// Per-active-expert record written by the routing kernels: [0] expert, [1] segment offset,
// [2] segment size M, [3] unused, [4 + j] token t and [4 + kRecTokens + j] slot t*K + p of the
// j-th segment entry, for j < min(M, kRecTokens).
constexpr uint32_t kRecWords = 32;
constexpr uint32_t kRecTokens = 14;

// Output pointers of the small-batch routing (top-k, softmax, dispatch, records).
struct RouteOut {
  int32_t *topk_idx;
  float *topk_w;
  int32_t *seg_off, *perm, *pos_of, *active, *num_active;
  int32_t *exrec;
};

struct DispatchArgs {
  const int32_t *topk_idx;
  int32_t *seg_off, *perm, *pos_of, *active, *num_active;
  int32_t *exrec;     // [E, kRecWords]
  int32_t *tile_off;  // [E + 1] prefix of ceil(M_e / kGemmTok), or null
  int32_t *chunk_cnt; // [ceil(n / kDispatchChunk), E] scratch of the multi-workgroup dispatch
  uint32_t n, K, E;
};

// One expert projection over the tiled MXFP4 layout (see the expert_gemv comment in kernels.hip).
// Persistent-style: gridDim.x workgroups split the flattened (active expert, row tile) items.
struct GemvArgs {
  const uint8_t *wb;      // tiled e2m1 blocks, expert stride wb_estride bytes
  const uint8_t *ws;      // tiled e8m0 scales, expert stride ws_estride bytes
  uint64_t wb_estride, ws_estride;
  const float *bias;      // [E, rows_p] (zero padded): gate_up b1 (interleaved order), down b2
  uint32_t bias_estride;
  uint32_t nrt;           // 16-row tiles per expert
  uint32_t nb;            // 32-wide K blocks (K padded = 32 * nb)
  uint32_t kt;            // true K
  uint32_t out_rows;      // gate_up: F output features; down: D
  uint32_t mt_max;        // tokens staged per pass (<= 16)
  const int32_t *seg_off, *active, *num_active, *perm;
  const int32_t *exrec;   // [E, kRecWords] per-active-expert records
  uint32_t nrec;          // records loaded: min(E, n * topk), every slot that can be active
  uint32_t num_cus;       // CUs of the device (dispatch rounds of the grid, see gemv_share)
  uint32_t weighted;      // 1: gemv_share's contiguous round-weighted shares; 0: strided shares
  uint32_t topk;
  // B operand rows: gate_up xn [n, Kp] (x dtype), down act [n*k, Kp] f32 (segment order)
  const void *brows;
  float *out;             // gate_up: act [n*k, Fp] (segment order); down: token-major slots [n*k, Dp]
  uint32_t out_stride;
  float alpha, limit;
  // every row tile's K range split into ksplit (0 or 1: none) fixed parts.  down: separate work
  // units, part h's partial sums go to out + h * out_half (bias in part 0), the combine adds the
  // parts; gate_up (kGateUpSplit parts): wave h of a workgroup takes part h of each of its row
  // tiles, the workgroup sums the parts in order (bias in part 0) and writes the SwiGLU rows
  uint32_t ksplit;
  uint64_t out_half;
  // gate_up of a single-token batch with its routing in the launch (route1_lg: the token's
  // route1_E logits, topk = K <= kMaxTopK): every workgroup selects the top K itself and lays out
  // the K records (one token each, experts in index order) in LDS; workgroup 0 also writes rout
  // for the down projection and the combine.  seg_off, active, num_active, perm and exrec above
  // are then unused by this launch.
  const float *route1_lg;
  uint32_t route1_E;
  RouteOut rout;
};

// Single-token batches (top-k <= kDownComb1MaxK) whose down projection takes kDownSplitFew K-parts:
// the down GEMV and the combine in one launch (down_combine1_kernel).  Weights, biases and geometry
// as GemvArgs (down); act the gate_up launch's SwiGLU rows [pos][act_stride] f32 (position
// pos_of[p] for slot p); y[d] = x[d] (add_residual, else 0) + sum over slots p (ascending) of
// w_p * (sum of the 4 parts).  K inputs (F padded to 32) at most kDownComb1MaxKp.
constexpr uint32_t kDownComb1MaxK = 4;
constexpr uint32_t kDownComb1MaxKp = 4096;
struct DownComb1Args {
  const uint8_t *wb, *ws;
  uint64_t wb_estride, ws_estride;
  const float *bias;  // b2 [E, rows_p]
  uint32_t bias_estride, nrt, nb, kt, D, K;
  const float *act;
  uint32_t act_stride;
  const int32_t *topk_idx, *pos_of;
  const float *topk_w;
  const void *x;  // [D] x dtype (token 0)
  void *y;        // [D] x dtype
  uint32_t add_residual;
};
hipError_t launch_down_combine1(const DownComb1Args &a, int nt, bool x_bf16, hipStream_t s);
size_t down_combine1_lds_bytes(int nt, uint32_t nb);

// Routing of a decode-sized batch (n <= kSmallRouteMaxTokens) by one workgroup: top-k, softmax,
// dispatch, all outputs to global.
struct SmallRouteArgs {
  const float *logits;
  int32_t *topk_idx;
  float *topk_w;
  int32_t *seg_off, *perm, *pos_of, *active, *num_active;
  int32_t *exrec;    // [E, kRecWords]
  uint32_t n, E, K;
};

// Decode-sized router (router_small_kernel, n <= kSmallRouteMaxTokens, D % 8 == 0, aligned rows):
// logits, r and the normalised rows xn for the gate_up GEMV.
struct FrontArgs {
  const void *x;
  const void *rw;      // router weight [E, D], gamma-folded when apply_norm
  const float *rb;     // [E]
  const float *gamma;  // [D]
  void *xn;            // [n, Dp] x dtype (bf16 with xn_bf16), or null
  float *logits;       // [n, E]
  float *rms;          // [n] or null
  uint32_t n, D, Dp, E;
  float eps;
  int apply_norm;
  int xn_bf16;         // xn rows rounded to bf16 (nearest even) whatever the x dtype
};
constexpr int kFrontChunks = 6;  // router_small_kernel: D <= 512 * kFrontChunks

// The decode router with the input rows formed first (router_front_kernel, f32 rows): a decoder's
// attention residual x = resid + (sum_h part_h + bias) of the output projection's K-part partials
// [nparts][n][D] is written to xout and routed as router_small_kernel routes f.x = xout.
struct PreFrontArgs {
  FrontArgs f;
  const float *part;
  uint64_t part_stride;
  uint32_t nparts;
  const float *bias;   // [D]
  const float *resid;  // [n, D]
  float *xout;         // [n, D]
};
constexpr uint32_t kFrontMaxParts = 16;

// Grouped expert GEMM for prefill-sized batches (expert_gemm_kernel): every active expert's
// segment is cut into tiles of kGemmTok routed tokens; a workgroup computes kGemmRows weight
// rows x one token tile with the block-scaled MFMA (MXFP4 weights x MXFP8 hi + MXFP4 lo activations).
constexpr uint32_t kGemmTok = 64;
constexpr uint32_t kGemmRows = 256;
struct GemmArgs {
  const uint8_t *wb, *ws;  // tiled MXFP4 codes (as GemvArgs); scales in the GEMM's copy (groups of
                           // 4 row tiles x blocks of 4 K-groups, 16 bytes per lane)
  uint64_t wb_estride, ws_estride;
  const float *bias;       // [E, rows_p]
  uint32_t bias_estride;
  uint32_t nrt, nb, kt, out_rows;
  uint32_t nrb;            // kGemmRows-row blocks per expert
  const int32_t *seg_off;  // [E + 1]
  const int32_t *tile_off; // [E + 1] exclusive prefix of ceil(M_e / kGemmTok)
  const int32_t *perm;     // segment entries t * topk + p
  uint32_t E, topk;
  QRows b;                 // B rows: gate_up xq (token rows), down act (segment rows)
  QRows act;               // gate_up output: SwiGLU rows in segment order, quantised
  uint32_t act_feats;      // gate_up: F (features written; [F, act.kq) zero-filled)
  uint16_t *out;           // down: token-major slot rows [n*k, out_stride] bf16
  uint32_t out_stride;
  float alpha, limit;
};

// The experts of a decode-sized batch in one launch (moe_fused_kernel): one workgroup per
// (active expert, feature slice) item, at most one item per CU.  The slice count per expert is
// set on the device from the number of active experts na: nsl = clamp(G / na, 1, min(nb2,
// nsl_cap)) for a grid of G workgroups, slice s = the 32-feature blocks [s nb2 / nsl,
// (s + 1) nb2 / nsl).  Phase 1 computes the slice's SwiGLU features for the expert's tokens (its
// interleaved W1 rows over all of D, bias, clamped SwiGLU; token passes of mt_max rows) into
// LDS; phase 2 multiplies W2's matching K range (every output row) with them and writes, per
// slot, the partial output row of slice s (b2 with slice 0).  No workgroup waits for another
// (split-K over F); combine_slices_kernel adds the slices in order.
struct FusedArgs {
  const uint8_t *w1b, *w1s, *w2b, *w2s;  // tiled MXFP4 codes and scales (as GemvArgs)
  uint64_t w1b_es, w1s_es, w2b_es, w2s_es;
  const float *b1, *b2;  // [E, w1 rows_p] interleaved order, [E, w2 rows_p]
  uint32_t b1_es, b2_es;
  uint32_t nrt1, nb1;    // W1 row tiles (2F rows), K blocks of 32 (D)
  uint32_t kt1;          // true K of W1 (D)
  uint32_t nrt2, nb2;    // W2 row tiles (D rows), K blocks (F)
  uint32_t D;            // output rows
  uint32_t nsl_cap;      // most slices per expert (the partial-row buffer's size)
  uint32_t sb_max;       // widest slice in blocks the LDS is sized for
  uint32_t mt_max;       // tokens per phase-1 pass
  const int32_t *num_active, *exrec, *perm;
  uint32_t topk;
  const void *xn;        // B rows of phase 1: [n, 32 * nb1] x dtype (normalised tokens)
  float *out;            // partial slot rows [nsl][n * topk][out_stride]
  uint64_t slice_stride; // elements between slices
  uint32_t out_stride;
  float alpha, limit;
};
constexpr uint32_t kFusedKgPerStep = 6;   // K-groups per wave per step of the fused kernel
constexpr uint32_t kFusedWaves = 16;      // waves per workgroup (one workgroup per CU)
constexpr uint64_t kFusedPartBytes = 8ull << 20;  // budget of the partial slot rows
constexpr uint32_t kFusedBiasRegs = 4;     // bias values per thread held in registers over the staging

struct CombineArgs {
  const void *x;
  void *y;
  const void *ypart;   // token-major slot rows [n*K, Dp], expert bias included: f32, or bf16 (part_bf16)
  uint32_t nparts;     // K-parts of ypart (1 = complete rows), parts part_stride elements apart,
  uint64_t part_stride;  // summed in order before the weighting
  int part_bf16;       // bf16 slot rows (the grouped GEMM's down output; nparts 1)
  const float *topk_w;
  uint32_t n, D, Dp, K;
  int add_residual;
  // optional RmsNorm of the result (combine_norm_kernel; f32 x and y, unsplit or K-part f32 slot
  // rows): nout[t] = y[t] / sqrt(mean(y[t]^2) + neps) * ngamma, when nout is not null
  const float *ngamma;
  float *nout;
  float neps;
  // combine_slices_kernel: the fused kernel's slice count, from num_active as that kernel sets it
  // (nparts = clamp(slice_grid / na, 1, slice_cap))
  const int32_t *num_active;
  uint32_t slice_grid, slice_cap;
};

struct DequantArgs {
  const uint8_t *blocks, *scales;
  void *out;
  uint64_t rows, cols, bpr, gpr;
  int ue8_offset;
  int out_bf16;
};

size_t router_lds_bytes(uint32_t tb, uint32_t Dpad);
size_t dispatch_lds_bytes(uint32_t E, uint32_t threads);
__host__ __device__ inline size_t gemv_lds_bytes(int nt, uint32_t mt_max, uint32_t nb) {
  return sizeof(uint16_t) * (size_t)nt * mt_max * (32u * nb + 8u);
}
// B staging (which first holds the record table), the chosen record and the per-token row index.
__host__ __device__ inline size_t gemv_stage_bytes(int nt, uint32_t mt_max, uint32_t nb, uint32_t nrec) {
  const size_t b = gemv_lds_bytes(nt, mt_max, nb), t = 4u * (size_t)nrec * 32u;
  return b > t ? b : t;
}
__host__ __device__ inline size_t gemv_total_lds_bytes(int nt, uint32_t mt_max, uint32_t nb, uint32_t nrec) {
  return gemv_stage_bytes(nt, mt_max, nb, nrec) + 4u * 32u + 4u * (size_t)mt_max + 16u;
}
// gate_up in K-parts (kGateUpSplit waves of a workgroup per row tile): the parts' tile results
// meet in LDS after the other regions, [tile parity][wave][lane] x 4 floats
constexpr size_t kGemvRedBytes = 2u * 4u * 64u * 16u;
__host__ __device__ inline size_t gemv_red_offset(int nt, uint32_t mt_max, uint32_t nb, uint32_t nrec) {
  return (gemv_total_lds_bytes(nt, mt_max, nb, nrec) + 15u) & ~(size_t)15u;
}
__host__ __device__ inline size_t gemv_launch_lds_bytes(int nt, uint32_t mt_max, uint32_t nb, uint32_t nrec, bool red) {
  return red ? gemv_red_offset(nt, mt_max, nb, nrec) + kGemvRedBytes : gemv_total_lds_bytes(nt, mt_max, nb, nrec);
}
constexpr uint32_t kGemvKgPerWave = 6;  // K-groups per wave per step (6 KiB of weights in flight)

constexpr uint32_t kRouterThreads = 256;
// router_rows_kernel from this batch size on: its time is one workgroup's pass over all E router
// rows (37 us at E = 32, 104 us at E = 128, D = 2880) while router_kernel's grows with n * E;
// measured crossover between 1000 and 1200 tokens for both E
constexpr uint32_t kRouterRowsMinTokens = 1152;
constexpr uint32_t kRowsThreads = 512;
constexpr uint32_t kTopkThreads = 512;
constexpr uint32_t kDispatchThreads = 1024;
constexpr uint32_t kDispatchChunk = 256;           // dispatch_wide_kernel: tokens per workgroup
constexpr uint32_t kDispatchWideMinTokens = 1024;  // dispatch_wide_kernel from this batch size on
constexpr uint32_t kGemvThreads = 256;
// relative shares of the expert GEMV workgroups of dispatch rounds 0..3 (see gemv_share), gate_up
// and down (measured: flatter weights for down, where the K-halves already even out the waves)
constexpr uint32_t kRoundWeight[2][4] = {{20, 10, 4, 2}, {20, 16, 11, 8}};
constexpr uint32_t kDownSplit = 2;  // K-parts per down row tile of the expert GEMV (decode-sized batches; 3, 4 and 6 measured slower)
// K-parts per gate_up row tile when a batch touches so few experts that whole row tiles leave most
// waves idle (one part per wave of a workgroup, summed in LDS before the SwiGLU epilogue)
constexpr uint32_t kGateUpSplit = 4;
constexpr uint32_t kDownSplitFew = 4;  // K-parts per down row tile for the same batches
constexpr uint32_t kMaxTopK = 32;
constexpr uint32_t kMaxExperts = 256;
constexpr uint32_t kSmallRouteMaxTokens = 16;  // decode-sized batches: one-workgroup routing kernel

hipError_t launch_router(const RouterArgs &a, bool x_bf16, bool w_bf16, bool vec, hipStream_t s);
// router_rows_kernel: D % 8 == 0 and D, Dp (with xn) and xq.kq (with xq) <= 512 * kFrontChunks,
// 16-byte aligned x and router rows; 2 or 4 tokens per wave (16 or 32 per workgroup)
hipError_t launch_router_rows(const RouterArgs &a, bool x_bf16, bool w_bf16, int tokens_per_wave, hipStream_t s);
hipError_t launch_small_route(const SmallRouteArgs &a, hipStream_t s);
hipError_t launch_router_small(const FrontArgs &a, bool x_bf16, bool w_bf16, hipStream_t s);
hipError_t launch_router_front(const PreFrontArgs &a, bool w_bf16, hipStream_t s);
hipError_t launch_topk(const TopkArgs &a, hipStream_t s);
hipError_t launch_dispatch(const DispatchArgs &a, hipStream_t s);
hipError_t launch_gemv(const GemvArgs &a, int nt, bool gate_up, bool x_bf16, uint32_t grid, hipStream_t s);
hipError_t launch_combine(const CombineArgs &a, bool x_bf16, hipStream_t s);
// Fused decode experts: launch geometry chosen by the host (fused_geometry in fused.hip) from the
// batch size and the most experts it can activate (max_active); the slicing itself is set on the
// device from the realised count.
struct FusedGeom {
  uint32_t grid;     // workgroups (the CUs)
  uint32_t nsl_cap;  // most slices per expert
  uint32_t sb_max;   // widest slice in 32-feature blocks
  uint32_t mt;       // tokens per phase-1 pass
  size_t lds;
};
bool fused_geometry(uint32_t nb1, uint32_t nb2, uint32_t nrt2, uint32_t Dp, uint32_t num_cus, uint32_t max_active,
                    uint32_t topk, uint64_t n, int nt, FusedGeom &g);
hipError_t launch_fused(const FusedArgs &a, const FusedGeom &g, int nt, bool x_bf16, hipStream_t s);
// combine over the slices of the fused kernel: y = x + sum_p w_p * (sum_s part[s][t k + p]),
// parts part_stride apart, their count as the fused kernel set it (CombineArgs.num_active)
hipError_t launch_combine_slices(const CombineArgs &a, bool x_bf16, hipStream_t s);
hipError_t configure_fused_kernels();
hipError_t launch_gemm(const GemmArgs &a, bool gate_up, uint32_t grid, hipStream_t s);
hipError_t configure_gemm_kernels();
size_t gemm_lds_bytes();
hipError_t launch_dequant(const DequantArgs &a, hipStream_t s);
hipError_t configure_kernels();

}  // namespace burnext
