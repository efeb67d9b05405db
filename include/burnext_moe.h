/*
 * burnext_moe.h -- C ABI of the MI355X (gfx950) GPT-OSS MoE feed-forward with MXFP4 experts.
 *
 * Drop-in boundary for burn-extended's MoE hot path.  Each entry point names the reference
 * interface it replaces (paths relative to the ariawisp/burn-extended tree):
 *
 *   burnext_moe_layer_create   MoeQuantLayerResident::new            src/quant/gpu.rs:30-54
 *                              + MoeGatedSwiGLU::set_resident         src/moe/mod.rs:95-97
 *                              + the module's norm/gate/bias params   src/moe/mod.rs:35-57
 *   burnext_moe_forward        MoeGatedSwiGLU::forward                src/moe/mod.rs:99-115
 *                              (forward_resident                      src/moe/mod.rs:122-412)
 *   burnext_moe_workspace_size (new: the reference allocates per call, src/moe/mod.rs:262,326)
 *   burnext_moe_forward_noalloc (no counterpart: the forward for callers that cannot allocate)
 *   burnext_moe_route          gate Linear + topk_with_indices + softmax  src/moe/mod.rs:110,271-276
 *   burnext_moe_dispatch       per-expert routing masks               src/moe/mod.rs:279-288
 *   burnext_moe_route_dispatch top-k + softmax + routing masks, as the forward runs them
 *                                                                     src/moe/mod.rs:271-288
 *   burnext_mxfp4_dequant      dequant_mxfp4_bytes                    src/loader/mxfp4.rs:56-79
 *   burnext_moe_layer_destroy  drop of Arc<MoeQuantLayerResident>     src/moe/mod.rs:56
 *   burnext_last_error         (new: the reference panics, src/moe/mod.rs:111-113)
 *
 * Conventions
 *  - Host pointers are read during burnext_moe_layer_create only; the caller keeps ownership and
 *    no host copy is retained (the reference keeps one, src/quant/gpu.rs:19-21,50-51).
 *  - All other data pointers are DEVICE pointers on the layer's device.  `stream` is a
 *    hipStream_t (NULL = default stream).  Calls are asynchronous on that stream, never
 *    synchronise the host, never allocate, and are safe to capture in a HIP graph.
 *  - A workspace is caller-provided device memory of at least burnext_moe_workspace_size()
 *    bytes, 256-byte aligned.  Concurrent calls on one layer need distinct workspaces.
 *  - No C++ exception or abort crosses this boundary: failures return a status and set a
 *    thread-local message readable with burnext_last_error().
 */
#ifndef BURNEXT_MOE_H
#define BURNEXT_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum burnext_status {
  BURNEXT_OK = 0,
  BURNEXT_INVALID_ARG = 1,        /* null pointer, descriptor/shape mismatch, bad enum */
  BURNEXT_UNSUPPORTED = 2,        /* shape outside what the kernels are built for */
  BURNEXT_OUT_OF_MEMORY = 3,      /* device allocation failed in layer_create */
  BURNEXT_DEVICE_ERROR = 4,       /* a HIP runtime call or kernel launch failed */
  BURNEXT_WORKSPACE_TOO_SMALL = 5 /* ws_bytes < burnext_moe_workspace_size() */
} burnext_status;

typedef enum burnext_dtype { BURNEXT_F32 = 0, BURNEXT_BF16 = 1 } burnext_dtype;

/* Row order of the fused gate_up (W1) matrix and its bias.
 * HALVES: rows [0,F) are the gate, rows [F,2F) the linear half -- the pairing the reference
 *         kernel uses (src/quant/gpu.rs:112-113, src/moe/mod.rs:336-337).
 * INTERLEAVED: even row 2f = gate, odd row 2f+1 = linear -- GPT-OSS checkpoints and the crate's
 *         swiglu_clamp (src/activation/mod.rs:5-12). */
typedef enum burnext_gate_up_layout { BURNEXT_GATE_UP_HALVES = 0, BURNEXT_GATE_UP_INTERLEAVED = 1 } burnext_gate_up_layout;

/* Mirrors QuantLinearMxFp4Desc (src/quant/mod.rs:3-11).  Blocks are [experts, rows, bpr] bytes
 * (two e2m1 codes per byte, low nibble = even column), scales [experts, rows, gpr] e8m0 bytes
 * stored as (exponent + ue8_offset) mod 256: ue8_offset = 0 for safetensors, 14 for model.bin
 * (src/loader/modelbin.rs:452-453, src/bin/gptoss_export.rs:529). */
typedef struct burnext_mxfp4_desc {
  uint64_t experts;
  uint64_t rows;
  uint64_t cols;
  uint64_t bpr; /* must equal ceil(cols / 2)  */
  uint64_t gpr; /* must equal ceil(cols / 32) */
  int32_t ue8_offset;
} burnext_mxfp4_desc;

/* Mirrors MoeConfig (src/moe/mod.rs:22-33); rms_eps is Burn's RmsNorm epsilon (default 1e-5). */
typedef struct burnext_moe_config {
  uint32_t d_model;
  uint32_t ffn_hidden;
  uint32_t num_experts;
  uint32_t experts_per_token; /* clamped to [1, num_experts] as src/moe/mod.rs:133 */
  float swiglu_alpha;
  float swiglu_limit;
  float rms_eps;
  int32_t disabled; /* non-zero: forward is the identity (src/moe/mod.rs:106-108) */
} burnext_moe_config;

typedef struct burnext_moe_layer *burnext_moe_layer_t;

/* forward / route flags */
#define BURNEXT_APPLY_RMSNORM 1u /* route on RmsNorm(x) (src/moe/mod.rs:109) */
#define BURNEXT_ADD_RESIDUAL 2u  /* y = x + MoE(...) (src/moe/mod.rs:411)   */
#define BURNEXT_FORWARD_DEFAULT (BURNEXT_APPLY_RMSNORM | BURNEXT_ADD_RESIDUAL)
/* Forward only, opt-in, no counterpart in the reference: batches of at most 16 tokens with
 * top-k <= 8 run gate_up, SwiGLU and down in one launch split over feature slices (each
 * workgroup one slice of one active expert), then a combine that sums the slices in order.  Same
 * results to the forward's tolerance; on MI355X it measured slower than the default two expert
 * GEMVs at every decode shape tried, so the default path does not take it. */
#define BURNEXT_FUSED_EXPERTS 4u

/* Uploads one layer to `device` and repacks W1/W2 into the kernels' tiled layout.
 * Host inputs: w1 [E, 2F, ...] per w1_desc, w2 [E, D, ...] per w2_desc, b1 [E, 2F] (same row
 * order as w1), b2 [E, D], both of bias_dtype; router_w [E, D] and router_b [E] (nullable = 0)
 * of router_dtype; norm_gamma [D] of norm_dtype (nullable = ones). */
burnext_status burnext_moe_layer_create(const burnext_moe_config *cfg, const burnext_mxfp4_desc *w1_desc,
                                        const uint8_t *w1_blocks, const uint8_t *w1_scales,
                                        const burnext_mxfp4_desc *w2_desc, const uint8_t *w2_blocks,
                                        const uint8_t *w2_scales, const void *b1, const void *b2,
                                        burnext_dtype bias_dtype, const void *router_w, const void *router_b,
                                        burnext_dtype router_dtype, const void *norm_gamma, burnext_dtype norm_dtype,
                                        burnext_gate_up_layout gate_up_layout, int device,
                                        burnext_moe_layer_t *out_layer);

void burnext_moe_layer_destroy(burnext_moe_layer_t layer);

/* Workspace bytes needed by forward/route/dispatch for any batch of up to n_tokens tokens: the
 * size is non-decreasing in n_tokens, so one workspace sized for the largest batch serves every
 * smaller one. */
burnext_status burnext_moe_workspace_size(burnext_moe_layer_t layer, uint64_t n_tokens, uint64_t *bytes);

/* y[n, D] = flags-selected MoE forward of x[n, D]; x and y share x_dtype and may not alias. */
burnext_status burnext_moe_forward(burnext_moe_layer_t layer, const void *x, burnext_dtype x_dtype, void *y,
                                   uint64_t n_tokens, uint32_t flags, void *workspace, uint64_t ws_bytes,
                                   void *stream);

/* No counterpart in the reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): burnext_moe_forward
 * with the library's own fixed scratch in place of a caller workspace.  The scratch is one 16 MiB
 * device array per GPU, held from the first layer created on that GPU until the process ends;
 * a batch whose burnext_moe_workspace_size exceeds 16 MiB (above 128 tokens at the GPT-OSS
 * shapes) returns BURNEXT_UNSUPPORTED.  The call allocates nothing (no hipMalloc, no events: the
 * profiling hook does not time it).  Every call on one GPU shares that GPU's scratch, which keeps
 * the last call's contents: calls that overlap on one GPU (other streams or threads) race. */
burnext_status burnext_moe_forward_noalloc(burnext_moe_layer_t layer, const void *x, burnext_dtype x_dtype, void *y,
                                           uint64_t n_tokens, uint32_t flags, void *stream);

/* Routing only: topk_idx[n, k] (int32, descending logit, ties to the lower expert index),
 * topk_w[n, k] (softmax over the selected logits); logits[n, E] optional (nullable).
 * flags: BURNEXT_APPLY_RMSNORM selects routing on RmsNorm(x). */
burnext_status burnext_moe_route(burnext_moe_layer_t layer, const void *x, burnext_dtype x_dtype,
                                 uint64_t n_tokens, uint32_t flags, int32_t *topk_idx, float *topk_w,
                                 float *logits, void *workspace, uint64_t ws_bytes, void *stream);

/* Expert-contiguous dispatch of topk_idx[n, k] (distinct experts per token, each in [0, E)):
 * seg_offsets[E+1] = exclusive scan of the expert histogram; perm[n*k] lists flat entry ids
 * t*k+p grouped by expert, tokens ascending inside a group. */
burnext_status burnext_moe_dispatch(burnext_moe_layer_t layer, const int32_t *topk_idx, uint64_t n_tokens,
                                    int32_t *seg_offsets, int32_t *perm, void *workspace, uint64_t ws_bytes,
                                    void *stream);

/* Routing and dispatch exactly as burnext_moe_forward runs them for a batch of n_tokens
 * (src/moe/mod.rs:110,271-288): for n <= 16 the one-workgroup kernel that fuses top-k, softmax and
 * the expert-contiguous dispatch; above, the top-k kernel then the dispatch kernels.  Outputs as
 * burnext_moe_route (topk_idx, topk_w) and burnext_moe_dispatch (seg_offsets[E+1], perm[n*k]). */
burnext_status burnext_moe_route_dispatch(burnext_moe_layer_t layer, const void *x, burnext_dtype x_dtype,
                                          uint64_t n_tokens, uint32_t flags, int32_t *topk_idx, float *topk_w,
                                          int32_t *seg_offsets, int32_t *perm, void *workspace, uint64_t ws_bytes,
                                          void *stream);

/* Dequantises a [desc.experts * desc.rows, desc.cols] MXFP4 matrix to f32 (exact
 * LUT[code] * 2^(s-127), s = stored - ue8_offset mod 256) or bf16 (same values; e2m1 times a
 * power of two is exact in bf16).  blocks/scales/out are device pointers. */
burnext_status burnext_mxfp4_dequant(const burnext_mxfp4_desc *desc, const uint8_t *blocks, const uint8_t *scales,
                                     void *out, burnext_dtype out_dtype, void *stream);

/* Per-kernel timing hook (a HIP event pair bound to each kernel dispatch of forward through
 * hipExtLaunchKernel: the kernel's own begin and end timestamps; timing-only events without the
 * system-scope fence).  A dispatch's time is the exclusive part of its interval, from
 * max(begin, end of the previous timed dispatch on the same stream) to its end: a dispatch queued
 * behind a running kernel can be stamped as begun before that kernel ends.
 * enable != 0 starts recording; read returns, per kernel id, accumulated milliseconds and
 * launch counts since the last read (it synchronises on the recorded events) and resets.  Event
 * pairs are pooled per process: an enable call made when every layer's records have been read
 * returns them to the pool, so a later recorded pass creates no events between its launches.
 * Kernel ids: 0 router, 1 top-k, 2 dispatch, 3 gate_up (with its SwiGLU), 4 down, 5 combine,
 * 6 reserved (records nothing), 7 the fused experts of BURNEXT_FUSED_EXPERTS (gate_up, SwiGLU and
 * down as one kernel; ids 3 and 4 then record nothing).  Batches of at most 16 tokens run top-k
 * and dispatch as one kernel, recorded under id 1; id 2 then records nothing.  A single-token
 * forward routes inside its gate_up launch (id 3); ids 1 and 2 then record nothing, and where its
 * down projection runs with the combine in one launch (top-k <= 4, no fused norm) that launch is
 * recorded under id 4 and id 5 records nothing. */
#define BURNEXT_NUM_KERNELS 8
burnext_status burnext_moe_profile_enable(burnext_moe_layer_t layer, int enable);
burnext_status burnext_moe_profile_read(burnext_moe_layer_t layer, double *ms_total, uint64_t *launches,
                                        int n_kernels);

/* Message of the last failing call on this thread ("" if none). */
const char *burnext_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* BURNEXT_MOE_H */
