// kernels.hpp -- argument blocks and host-side launchers of the MoE kernels (gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace burnext {

// Route: optional RmsNorm, router logits, top-k + softmax, bf16 activation terms for the
// expert GEMVs, and (single-workgroup batches) the dispatch into expert segments.
struct RouteArgs {
  const void *x;
  const void *rw;  // router weight [E, D] (f32 or bf16 bits)
  const float *rb; // router bias [E]
  const float *gamma;
  uint16_t *xn_terms; // [n, nt, Dp] bf16 bits, nullable
  float *logits;      // [n, E], nullable
  int32_t *topk_idx;  // [n, K]
  float *topk_w;      // [n, K]
  int32_t *seg_off, *perm, *pos_of, *active, *num_active; // fused dispatch outputs
  uint32_t n, D, Dp, E, K, tpb, nt;
  float eps;
  int apply_norm;
  int fuse_dispatch;
};

struct DispatchArgs {
  const int32_t *topk_idx;
  int32_t *seg_off, *perm, *pos_of, *active, *num_active;
  uint32_t n, K, E;
};

// One expert projection over the tiled MXFP4 layout (see layer.hip, "tiled layout").
struct GemvArgs {
  const uint8_t *wb;      // tiled e2m1 blocks, expert stride wb_estride bytes
  const uint8_t *ws;      // tiled e8m0 scales, expert stride ws_estride bytes
  uint64_t wb_estride, ws_estride;
  const float *bias;      // gate_up: b1 [E, rows_p] (interleaved order); unused for down
  uint32_t bias_estride;
  uint32_t nrt;           // 16-row tiles per expert
  uint32_t nb;            // 32-wide K blocks (K padded = 32 * nb)
  uint32_t kt;            // true K
  uint32_t out_rows;      // gate_up: F output features; down: D
  uint32_t tiles_per_wg;  // row tiles per workgroup (multiple of the 4 waves)
  uint32_t mt_max;        // tokens staged per pass (<= 16)
  const int32_t *seg_off, *active, *num_active, *perm;
  uint32_t topk;
  const uint16_t *bterms; // gate_up B operand: xn terms [n, NT, Kp]
  const float *bf32;      // down B operand: act [n*k, Kp] f32
  float *out;             // gate_up: act [n*k, Fp]; down: ypart [n*k, Dp]
  uint32_t out_stride;
  float alpha, limit;
};

struct CombineArgs {
  const void *x;
  void *y;
  const float *ypart;
  const float *b2;
  const int32_t *topk_idx;
  const float *topk_w;
  const int32_t *pos_of;
  uint32_t n, D, Dp, E, K;
  int add_residual;
};

struct DequantArgs {
  const uint8_t *blocks, *scales;
  void *out;
  uint64_t rows, cols, bpr, gpr;
  int ue8_offset;
  int out_bf16;
};

// LDS bytes the route kernel needs for a given token block.
size_t route_lds_bytes(uint32_t tpb, uint32_t D, uint32_t E, uint32_t K, uint32_t threads);
size_t dispatch_lds_bytes(uint32_t E, uint32_t threads);
size_t gemv_lds_bytes(int nt, uint32_t mt_max, uint32_t nb);

constexpr uint32_t kRouteThreads = 512;
constexpr uint32_t kDispatchThreads = 1024;
constexpr uint32_t kGemvThreads = 256;
constexpr uint32_t kMaxTopK = 32;
constexpr uint32_t kMaxExperts = 256;

hipError_t launch_route(const RouteArgs &a, bool x_bf16, bool w_bf16, hipStream_t s);
hipError_t launch_dispatch(const DispatchArgs &a, hipStream_t s);
hipError_t launch_gemv(const GemvArgs &a, int nt, bool gate_up, uint32_t grid_x, uint32_t grid_y, hipStream_t s);
hipError_t launch_combine(const CombineArgs &a, bool x_bf16, hipStream_t s);
hipError_t launch_dequant(const DequantArgs &a, hipStream_t s);
hipError_t configure_kernels();

}  // namespace burnext
