/*
 * glm53_moe.h -- C ABI of libglm53moe.so, the MI355X (gfx950) routed-MoE
 * library for livglm's GLM-5.3-Flash MoE layer.
 *
 * Conventions (every entry point):
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *     All work is enqueued on it; no entry point synchronises, allocates device
 *     memory or frees it.  The caller owns every buffer.
 *   - Pointers are device pointers to row-major arrays.  bf16 values travel as
 *     uint16_t bit patterns.  Expert banks hold the reference checkpoint's
 *     tensors (weight_packed / weight_scale, expert_source.py:189-229),
 *     stacked over experts: gate/up packed [E][I][d/2] u8, gate/up scales
 *     [E][I][d/32] u8, down packed [E][d][I/2] u8, down scales [E][d][I/32]
 *     u8.  The scales keep the checkpoint's row-major layout; each expert's
 *     packed codes are in the BANK LAYOUT: a matrix of `rows` x K codes with
 *     rows % 16 == 0 and K % 128 == 0 (every geometry the MFMA kernels take)
 *     is tile-major -- the 16-row x 128-code block (t, c) is 1 KB at byte
 *     (t K/128 + c) 1024, its 16-byte piece r + 16 q holding row 16 t + r,
 *     codes 128 c + 32 q .. + 31 -- and any other matrix stays row-major.
 *     glm_mxfp4_tile and glm_bank_scatter write it from checkpoint bytes.
 *   - Return value: GLM_OK (0) or a negative GLM_ERR_* code; the message is
 *     available from glm_last_error() on the calling thread.  No C++ exception
 *     crosses the ABI.
 *   - Calls are re-entrant; concurrent calls on different streams must use
 *     different output and workspace buffers.
 */
#ifndef GLM53_MOE_H
#define GLM53_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GLM_ABI_VERSION 2

#define GLM_OK 0
#define GLM_ERR_INVALID_ARGUMENT (-1) /* null pointer, negative size, bad enum */
#define GLM_ERR_UNSUPPORTED_SHAPE (-2) /* shape outside what the kernels accept */
#define GLM_ERR_HIP (-3)               /* a HIP runtime call failed */
#define GLM_ERR_WORKSPACE (-4)         /* workspace too small */

/* Weight storage formats (layers.py:38-70 quantization_mode). */
#define GLM_FMT_BF16 0  /* bf16 [out][in] */
#define GLM_FMT_MXFP8 1 /* E4M3FN codes [out][in] u8 + E8M0 scales [out][in/32] */
#define GLM_FMT_MXFP4 2 /* packed E2M1 [out][in/2] u8 + E8M0 scales [out][in/32] */

/* Shared-exponent rules for glm_mx_quantize (the rule of mx.quantize is not
 * published; see layers.py:89-94). */
#define GLM_MX_RULE_NEAREST 0 /* e = round(log2(amax / elem_max)), saturating elements */
#define GLM_MX_RULE_OCP 1     /* e = floor(log2(amax)) - emax_elem (OCP MX v1.0) */

/* Version of this header's ABI; bump on any signature change. */
int glm_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *glm_last_error(void);

/*
 * Router.  Replaces TopKRouter.__call__ (src/glm53flash/moe.py:36-63).
 * x bf16 [T][d]; weight f32 [E][d]; bias f32 [E].
 * logits f32 [T][E] = f32(x) @ weight^T; scores = sigmoid(logits);
 * choice = scores + bias; group top-2-sum mask keeps `topk_group` of
 * `n_group` groups; indices u32 [T][k] = the k best choices in ASCENDING order
 * (best expert last, moe.py:33-34,58; ties rank the larger index higher);
 * weights f32 [T][k] = scores[indices], normalised by (sum + 1e-20) when
 * norm_topk_prob, times routed_scaling_factor.  logits is a required output.
 * Limits: E <= 1024, E % n_group == 0, E / n_group >= 2, 1 <= k <= min(E, 64),
 * d % 4 == 0; every buffer 16-byte aligned (all entry points require this).
 */
int glm_router_topk(void *stream, const uint16_t *x, int T, int d, const float *weight,
                    const float *bias, int E, int top_k, int n_group, int topk_group,
                    int norm_topk_prob, float routed_scaling_factor, float *logits,
                    float *weights, uint32_t *indices);

/*
 * Token-to-expert dispatch: histogram, exclusive prefix sum, stable permute.
 * Replaces the host-side route materialisation of
 * _expert_ssd_route_cache_plan / ExpertSSD.__call__ dedupe+remap
 * (native_expert_ssd.py:475-525, expert_ssd.py:159-169).
 * indices u32 [T*k] (row-major (t, j) pairs, P = T*k).
 * counts [E]; offsets [E+1] (exclusive scan of counts); perm [P] (sorted
 * position -> pair t*k+j, each expert's pairs ascending); inv [P] (pair ->
 * sorted position); pair_token [P] (sorted position -> token t); active [E]
 * (ids of experts with count > 0, ascending, then -1); num_active [1];
 * work [E][4] (per active slot u: {expert, offsets[expert], count, 0}; slots
 * u >= num_active hold {-1, 0, 0, 0}); status [1] (0, or 1 if an index >= E
 * was seen -- such pairs are dropped, inv = -1, and the sorted positions past
 * offsets[E] hold -1 in perm and pair_token).  Up to 4096 pairs one
 * workgroup sorts them; beyond, two chunk-parallel launches over 1024-pair
 * chunks: each chunk ranks its pairs per expert and counts them, then each
 * chunk sums the counts of the chunks before it and places its pairs
 * (pair_token holds the chunk counts until it is filled last; the result is
 * the same).
 * Limits: E <= 448 (one workgroup's LDS holds the per-expert bitmaps).
 */
int glm_moe_dispatch(void *stream, const uint32_t *indices, int T, int top_k, int E,
                     int32_t *counts, int32_t *offsets, int32_t *perm, int32_t *inv,
                     int32_t *pair_token, int32_t *active, int32_t *num_active, int32_t *work,
                     int32_t *status);

/*
 * Routed gate/up projections + limited SwiGLU.  Replaces
 * mx._expert_ssd_mxfp4_pair_qmv + limited_swiglu (native_expert_ssd.py:696-706,
 * expert_ssd.py:103-107), and gather_qmm for T > 1 (native_expert_ssd.py:726-741).
 * x bf16 [T][d]; h bf16 [T*k][I] in SORTED (dispatch) order:
 * h[pos] = swiglu(bf16(x[pair_token[pos]] . Wg[e]^T), bf16(x . Wu[e]^T)) for
 * the rows pos of each work slot (glm_moe_dispatch).
 * Limits: d % 32 == 0, I % 16 == 0.
 */
int glm_expert_gate_up(void *stream, const uint16_t *x, int T, int d, int I, int E, int top_k,
                       const uint8_t *gate_packed, const uint8_t *gate_scales,
                       const uint8_t *up_packed, const uint8_t *up_scales,
                       const int32_t *pair_token, const int32_t *work, float swiglu_limit,
                       uint16_t *h);

/*
 * Few-token selection + routed gate/up, token-major (no dispatch).  For each
 * pair (t, j): token t's experts are chosen from its router logits exactly as
 * glm_router_topk chooses them (TopKRouter.__call__, moe.py:36-63), and
 * h[t*k + j] = limited SwiGLU of expert indices[t][j]'s gate/up projections
 * of x[t] (native_expert_ssd.py:696-706, expert_ssd.py:103-107).
 * logits f32 [T][E] (as glm_router_topk writes them); weights f32 [T][k] and
 * indices u32 [T][k] are written as glm_router_topk writes them; h bf16
 * [T*k][I] in pair order.
 * Limits: T <= 4, k <= 8, E <= 448, d / 512 in {2, 4, 6, 8},
 * I / 128 in {1, 2, 4, 6, 8, 16}, plus the router's limits.
 */
int glm_route_gate_up(void *stream, const float *logits, const float *bias, int T, int E,
                      int top_k, int n_group, int topk_group, int norm_topk_prob,
                      float routed_scaling_factor, const uint16_t *x, int d, int I,
                      const uint8_t *gate_packed, const uint8_t *gate_scales,
                      const uint8_t *up_packed, const uint8_t *up_scales, float swiglu_limit,
                      float *weights, uint32_t *indices, uint16_t *h);

/*
 * Routed down projection.  Replaces mx._expert_ssd_mxfp4_masked_qmv
 * (native_expert_ssd.py:707-717) and gather_qmm(down) (native_expert_ssd.py:743).
 * h bf16 [T*k][I] (sorted order); y bf16 [T*k][d] (sorted order).
 * Limits: I % 32 == 0, d % 16 == 0.
 */
int glm_expert_down(void *stream, const uint16_t *h, int T, int top_k, int I, int d, int E,
                    const uint8_t *down_packed, const uint8_t *down_scales, const int32_t *work,
                    uint16_t *y);

/*
 * Row tiles of the grouped GEMMs below, from a dispatch work list: every
 * active slot u (work[u] = {expert, first sorted position, rows, 0}) gives
 * nt = ceil(rows / 160) tiles {expert, first position, tile rows, 0}, in slot
 * order: the slot's 16-row blocks B = ceil(rows / 16) are dealt out evenly,
 * tile i starting at row 16 floor(i B / nt) of the slot, so every tile has at
 * most 160 rows and all but the slot's last a multiple of 16.  tiles int4
 * [max_tiles] with max_tiles >= ceil(T*k / 160) + E; num_tiles [1].  No
 * reference counterpart: it feeds the prefill GEMMs below, which take tiles
 * of at most 160 rows.
 */
int glm_moe_tiles(void *stream, const int32_t *work, int E, int32_t *tiles, int32_t *num_tiles);

/*
 * Exact two-term FP8 split of bf16 activations for the block-scaled MFMA
 * GEMMs below.  For every 32-element group of a row:
 *   x = hi * 2^(shi - 127) + lo * 2^(slo - 127),
 * hi, lo E4M3FN codes (hi rounded to nearest-even, lo the rounded residual),
 * shi, slo E8M0, each the smallest scale that keeps its group within 448.
 * A bf16 element has 8 significant bits and each code holds 4, so elements
 * within ~14 binades of their group's maximum are reproduced exactly; smaller
 * ones err by < 2^-22 of that maximum.
 * split: one buffer of glm_act_split_bytes(rows, K) bytes holding hi
 * [rows][K], lo [rows][K], shi [rows][K/32], slo [rows][K/32], each 256-byte
 * aligned.  No reference counterpart: it is the activation operand format of
 * the grouped GEMMs.  Limits: K % 32 == 0.
 */
size_t glm_act_split_bytes(int rows, int K);
int glm_act_split_fp8(void *stream, const uint16_t *x, int rows, int K, void *split);

/*
 * Activation formats of the grouped GEMMs (act_format).  Every form is
 * block-scaled over 32-element groups with E8M0 scales, each term's scale the
 * smallest power of two that keeps the group within the element maximum:
 *   GLM_ACT_FP8X2  the exact two-term E4M3FN split above; two MFMAs per
 *                  block at the FP8 rate;
 *   GLM_ACT_FP6X2  two E2M3 terms (hi, then the rounded exact residual):
 *                  ~3e-4 relative error on Gaussian rows; two MFMAs at the
 *                  FP6 rate (twice FP8's);
 *   GLM_ACT_FP4    one E2M1 term: ~12 % relative error; one MFMA at the FP4
 *                  rate;
 *   GLM_ACT_FP8FP6 hi E4M3FN + lo E2M3 of the exact residual: exact for
 *                  elements at most two binades below their group maximum's,
 *                  error at most max / 840 (~3e-4 relative on Gaussian rows,
 *                  as FP6X2); the hi MFMA at the FP8 rate, the lo at FP6's.
 * Split layout (glm_act_split_bytes_fmt(rows, K, fmt) bytes, regions 256-byte
 * aligned): hi codes, lo codes, hi scales [rows][K/32], lo scales (FP4: codes,
 * scales).  Code rows: FP8X2 [K] one byte per element; FP4 [K/2], two codes
 * per byte, low nibble first; FP6X2 (both terms) and FP8FP6 (the lo term; hi
 * as FP8X2) [K] in 128-byte chunks per 128 elements,
 * group g's 32 codes packed 6 bits each, low bits first, bytes 0..15 at 16 g
 * and bytes 16..23 at 64 + 16 g (the rest zero).
 * No reference counterpart (the reference multiplies bf16 activations): the
 * lower-precision forms are speed/accuracy variants of the grouped GEMMs.
 * Limits: K % 32 == 0 (FP6X2, FP8FP6: K % 128 == 0); glm_act_split_bytes_fmt returns
 * 0 outside them.
 */
#define GLM_ACT_FP8X2 0
#define GLM_ACT_FP6X2 1
#define GLM_ACT_FP4 2
#define GLM_ACT_FP8FP6 3
size_t glm_act_split_bytes_fmt(int rows, int K, int act_format);
int glm_act_split(void *stream, const uint16_t *x, int rows, int K, int act_format, void *split);

/*
 * Prefill routed gate/up as grouped GEMMs over the row tiles of
 * glm_moe_tiles, on the block-scaled MFMA: MXFP4 weights as stored, the
 * activations as their FP8 split.  Replaces gather_qmm(gate/up) +
 * limited_swiglu over all (t, j) pairs (native_expert_ssd.py:726-741,
 * expert_ssd.py:103-107,185-186).
 * x_split: glm_act_split_fp8 of x bf16 [T][d].  h bf16 [T*k][I] in sorted
 * order, token rows through pair_token (as glm_expert_gate_up).
 * tiles int32 [max_tiles][4] {expert, first sorted row, rows, 0} as
 * glm_moe_tiles writes them; the device-side *num_tiles is clamped to
 * max_tiles and tiles with rows <= 0 or a negative expert or row are skipped,
 * but expert ids must lie in the bank and rows inside h (the library is not
 * given E or T*k here and cannot check them).
 * Limits: d % 512 == 0, I % 256 == 0.
 */
int glm_expert_gate_up_grouped(void *stream, const void *x_split, int T, int d, int I,
                               const uint8_t *gate_packed, const uint8_t *gate_scales,
                               const uint8_t *up_packed, const uint8_t *up_scales,
                               const int32_t *pair_token, const int32_t *tiles,
                               const int32_t *num_tiles, int max_tiles, float swiglu_limit,
                               uint16_t *h);

/*
 * Prefill routed down projection as grouped GEMMs (native_expert_ssd.py:743).
 * h_split: glm_act_split_fp8 of h bf16 [P = T*k][I] (sorted order).
 * y bf16 [P][d] in sorted order.  Limits: d % 512 == 0, I % 256 == 0.
 */
int glm_expert_down_grouped(void *stream, const void *h_split, int P, int I, int d,
                            const uint8_t *down_packed, const uint8_t *down_scales,
                            const int32_t *tiles, const int32_t *num_tiles, int max_tiles,
                            uint16_t *y);

/*
 * glm_expert_gate_up_grouped / glm_expert_down_grouped with the activations
 * split in act_format (glm_act_split of x, of h).  GLM_ACT_FP8X2 is exactly
 * the entry points above.  No reference counterpart: format variants of the
 * same products (native_expert_ssd.py:726-743).
 */
int glm_expert_gate_up_grouped_fmt(void *stream, int act_format, const void *x_split, int T,
                                   int d, int I, const uint8_t *gate_packed,
                                   const uint8_t *gate_scales, const uint8_t *up_packed,
                                   const uint8_t *up_scales, const int32_t *pair_token,
                                   const int32_t *tiles, const int32_t *num_tiles, int max_tiles,
                                   float swiglu_limit, uint16_t *h);
int glm_expert_down_grouped_fmt(void *stream, int act_format, const void *h_split, int P, int I,
                                int d, const uint8_t *down_packed, const uint8_t *down_scales,
                                const int32_t *tiles, const int32_t *num_tiles, int max_tiles,
                                uint16_t *y);

/*
 * Weighted combine + shared add (moe.py:198-201):
 * out[t] = sum_{j=0..k-1} f32(y[inv[t*k+j]]) * weights[t*k+j]  (sequential j)
 *          + f32(shared[t])    (shared may be NULL).
 * out is f32 [T][d].
 */
int glm_moe_combine(void *stream, const uint16_t *y, const int32_t *inv, const float *weights,
                    const uint16_t *shared, int T, int top_k, int d, float *out);

/*
 * Dense linear y = bf16(x @ deq(W)^T), f32 accumulate.  Replaces
 * DeferredLinear.__call__ (layers.py:38-70): bf16 (`x @ weight.T`),
 * mx.quantized_matmul(mode="mxfp8"/"mxfp4", group_size=32).
 * x bf16 [T][in]; weight per `fmt`; scales NULL for bf16; y bf16 [T][out].
 * Limits: in % 32 == 0, out % 16 == 0.
 */
int glm_linear(void *stream, const uint16_t *x, int T, int in_dims, const void *weight,
               const uint8_t *scales, int fmt, int out_dims, uint16_t *y);

/*
 * glm_linear on an f32 input: every x value is rounded to bf16 (RNE) as it
 * is read, so the result equals glm_linear of the bf16 cast of x -- the cast
 * the decoder applies to its f32 residual before the native path
 * (native_expert_ssd.py:655-658), fused into the linear.
 * x f32 [T][in].  Limits: T <= 4, in % 32 == 0, out % 8 == 0.
 */
int glm_linear_f32(void *stream, const float *x, int T, int in_dims, const void *weight,
                   const uint8_t *scales, int fmt, int out_dims, uint16_t *y);

/*
 * RMSNorm of f32 rows followed by the MXFP8 resident linear: RMSNorm
 * (layers.py:119-131; unweighted when norm_weight is NULL, layers.py:134-140),
 * x * (1 / sqrt(mean(x^2) + eps)) * w, rounded to bf16, then
 * DeferredLinear.__call__ (layers.py:56-70) on it -- the decoder's norm in
 * front of a resident projection, fused so that the normalised row is never
 * written out.  Equal to glm_rms_norm (bf16 output) + glm_linear up to the
 * order of the f32 sum of squares.
 * x f32 [T][in]; norm_weight f32 [in] or NULL; weight/scales MXFP8
 * (GLM_FMT_MXFP8 only); y bf16 [T][out].
 * Limits: T <= 4, in % 256 == 0, out % 8 == 0.
 */
int glm_rms_norm_linear(void *stream, const float *x, int T, int in_dims,
                        const float *norm_weight, float eps, const void *weight,
                        const uint8_t *scales, int fmt, int out_dims, uint16_t *y);

/*
 * Dense SwiGLU MLP (the shared expert).  Replaces DenseMLP.__call__
 * (layers.py:160-171): out = down(limited_swiglu(gate(x), up(x))).
 * All three weights share `fmt`.  h is caller scratch bf16 [T][I].
 */
int glm_dense_mlp(void *stream, const uint16_t *x, int T, int d, int I, int fmt,
                  const void *gate_w, const uint8_t *gate_s, const void *up_w,
                  const uint8_t *up_s, const void *down_w, const uint8_t *down_s,
                  float swiglu_limit, uint16_t *h, uint16_t *out);

/*
 * Group-32 MX quantisation of a bf16 matrix.  Replaces
 * mx.quantize(group_size=32, bits=8|4, mode="mxfp8"|"mxfp4") in
 * DeferredLinear.quantize_to_mxfp (layers.py:72-99).
 * w bf16 [rows][cols]; fmt GLM_FMT_MXFP8 (codes [rows][cols]) or
 * GLM_FMT_MXFP4 (codes [rows][cols/2]); scales [rows][cols/32].
 * Elements round to nearest-even and saturate at the format maximum.
 */
int glm_mx_quantize(void *stream, const uint16_t *w, int rows, int cols, int fmt, int rule,
                    uint8_t *codes, uint8_t *scales);

/*
 * Group-32 MX dequantisation to f32 (the exact decode every MX kernel applies
 * in registers; gather_qmm / quantized_matmul read the same values).
 */
int glm_mx_dequantize(void *stream, const uint8_t *codes, const uint8_t *scales, int rows,
                      int cols, int fmt, float *out);

/* limited_swiglu on bf16 arrays (expert_ssd.py:103-107), bf16 intermediates. */
int glm_limited_swiglu(void *stream, const uint16_t *gate, const uint16_t *up, int64_t n,
                       float limit, uint16_t *out);

/*
 * Workspace needed by glm_moe_forward for these sizes (bytes).
 */
size_t glm_moe_workspace_bytes(int T, int d, int E, int top_k, int I, int I_shared);

/*
 * Zero-fills a workspace with a plain kernel (no memset node, so it may be
 * captured in a graph).  glm_moe_forward does not need it; it is provided so
 * callers can give a workspace a defined initial state.  Calls that overlap
 * on one workspace race.
 */
int glm_moe_workspace_init(void *stream, void *workspace, size_t workspace_bytes);

/*
 * One whole routed-MoE layer on a bf16 [T][d] input.  Replaces
 * ExpertSSDMoE.__call__ / _call_impl (moe.py:96-201) with an HBM-resident
 * expert bank: router -> dispatch -> gate/up+SwiGLU -> down -> shared expert
 * -> weighted combine, all on `stream` with no host synchronisation.  Up to
 * four tokens (top_k <= 8) it is three kernels: router logits (+ bf16 shared
 * gate/up), top-k selection + routed gate/up (+ shared down), routed down +
 * weighted combine.  Up to 64 tokens (T*k <= 512) it is the decode path:
 * router logits, selection, dispatch (+ shared down), routed gate/up, routed
 * down, combine.  Beyond that the dispatch and the grouped MFMA GEMMs.
 * shared_in (may be NULL): the shared expert's bf16 output [T][d] computed by
 * the caller -- e.g. with glm_dense_mlp on a second stream, overlapping the
 * routing -- in which case the shared weights are not read.
 * out f32 [T][d].  Optional outputs (may be NULL): weights f32 [T][k],
 * indices u32 [T][k].  The shared expert is skipped when shared_gate is NULL.
 * Shared-expert weights use `shared_fmt` (GLM_FMT_BF16: scale pointers NULL;
 * GLM_FMT_MXFP8/MXFP4: the resident MX layout): gate/up [I_shared][d],
 * down [d][I_shared].
 * Limits: E <= 448, d % 32 == 0, I % 32 == 0.
 */
int glm_moe_forward(void *stream, const uint16_t *x, int T, int d, const float *router_weight,
                    const float *router_bias, int E, int top_k, int n_group, int topk_group,
                    int norm_topk_prob, float routed_scaling_factor, int I,
                    const uint8_t *gate_packed, const uint8_t *gate_scales,
                    const uint8_t *up_packed, const uint8_t *up_scales,
                    const uint8_t *down_packed, const uint8_t *down_scales, int I_shared,
                    int shared_fmt, const void *shared_gate, const uint8_t *shared_gate_scales,
                    const void *shared_up, const uint8_t *shared_up_scales,
                    const void *shared_down, const uint8_t *shared_down_scales,
                    const uint16_t *shared_in, float swiglu_limit, void *workspace,
                    size_t workspace_bytes, float *out, float *weights_out,
                    uint32_t *indices_out);


/* Size of the device array behind glm_moe_forward_noalloc (per device). */
#define GLM_NOALLOC_SCRATCH_BYTES (64u << 20)

/*
 * glm_moe_forward without a workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  No counterpart in the reference.
 * The layer's workspace is a file-scope device array of
 * GLM_NOALLOC_SCRATCH_BYTES inside the library: every device that loads the
 * library holds its own copy until the process ends, and its address is
 * looked up once per device, on the first call with that device current
 * (that call may itself be made under HIP graph capture; replays of a
 * captured call equal glm_moe_forward's result).
 * Sizes whose workspace (glm_moe_workspace_bytes) exceeds the array are
 * rejected with GLM_ERR_WORKSPACE before any device work; decode sizes fit
 * (T = 64 at d 2048, E 128, k 8, I 768, I_shared 768 needs 8.7 MiB; T = 64 at
 * d 4096, E 288, I 2048 needs 33.4 MiB), 4096-token prefill does not.
 * `stream` must belong to the current device.  Nothing in the array needs to
 * start at zero; each call leaves its contents there.  All calls on one
 * device share the array, so calls that overlap on a device race: issue them
 * on one stream (or order them).  Allocates and frees nothing.  Arguments and
 * results otherwise as glm_moe_forward.
 */
int glm_moe_forward_noalloc(void *stream, const uint16_t *x, int T, int d,
                            const float *router_weight, const float *router_bias, int E,
                            int top_k, int n_group, int topk_group, int norm_topk_prob,
                            float routed_scaling_factor, int I, const uint8_t *gate_packed,
                            const uint8_t *gate_scales, const uint8_t *up_packed,
                            const uint8_t *up_scales, const uint8_t *down_packed,
                            const uint8_t *down_scales, int I_shared, int shared_fmt,
                            const void *shared_gate, const uint8_t *shared_gate_scales,
                            const void *shared_up, const uint8_t *shared_up_scales,
                            const void *shared_down, const uint8_t *shared_down_scales,
                            const uint16_t *shared_in, float swiglu_limit, float *out,
                            float *weights_out, uint32_t *indices_out);

/*
 * glm_moe_forward with the routed experts' E8M0 scales kept ScaleX Mode-B
 * coded in HBM (docs/scalex-mode-b.md:24-33; the reference's ScaleX QMV,
 * native_expert_ssd.py:653-694): scalex_rows + e * scalex_stride holds expert
 * e's Mode-B row (encode_mode_b_row, scale_codec.py:150-154: the Mode-A
 * record of its gate | down | up scale bytes and the u16 tile directory) with
 * the directory in front: the (raw + 511) / 512 + 1 u16 entries zero-padded
 * to a multiple of 16 bytes, then the record (24-byte header, primary codes,
 * exception positions and values).  The few-token kernels decode the scale rows of their
 * tiles into LDS while the weights stream (the reference decodes 512-scale
 * tiles into threadgroup memory inside its QMV); the outputs are
 * bit-identical to glm_moe_forward on the decoded scales.  The gate/up/down
 * scale pointers of glm_moe_forward are replaced by scalex_rows/stride; the
 * other arguments are the same.  Limits: the few-token path (T <= 4,
 * top_k <= 8, d / 512 in {2, 4, 6, 8}, I / 128 in {1, 2, 4, 6, 8, 16});
 * rows 256-byte aligned, stride a positive multiple of 256.  The rows must be
 * valid Mode-B rows (the host codec validates them; the kernels trust the
 * header, the directory and the exception order).
 */
int glm_moe_forward_scalex(void *stream, const uint16_t *x, int T, int d,
                           const float *router_weight, const float *router_bias, int E, int top_k,
                           int n_group, int topk_group, int norm_topk_prob,
                           float routed_scaling_factor, int I, const uint8_t *gate_packed,
                           const uint8_t *up_packed, const uint8_t *down_packed,
                           const uint8_t *scalex_rows, int64_t scalex_stride, int I_shared,
                           int shared_fmt, const void *shared_gate,
                           const uint8_t *shared_gate_scales, const void *shared_up,
                           const uint8_t *shared_up_scales, const void *shared_down,
                           const uint8_t *shared_down_scales, const uint16_t *shared_in,
                           float swiglu_limit, void *workspace, size_t workspace_bytes, float *out,
                           float *weights_out, uint32_t *indices_out);

/* ------------------------------------------------------------ decoder FFN site */

/* glm_hc_pre / glm_hc_post flag: the streams are bf16 in the model (passed
 * here as their exact f32 values); the reference's rounding points of that
 * dtype apply (collapsed rounded to bf16; in hyper_residual post, comb and the
 * mixing sum rounded to bf16, mhc.py:46,57-59). */
#define GLM_HC_BF16_STREAMS 1

/*
 * Workspace bytes of glm_hc_pre (per-slice partial sums of the hyper-connection
 * GEMV); 0 for invalid sizes.
 */
size_t glm_hc_workspace_bytes(int T, int hc, int d);

/*
 * The FFN-site hyper-connection of a decoder layer, HyperConnection.__call__
 * (mhc.py:23-48; the layer's ffn_hc, model.py:59,134), with the
 * post-attention RMSNorm (model.py:57,135; layers.py:119-131) fused:
 *   flat = rms_norm(streams[t] flattened, eps = rms_eps)   (unweighted)
 *   mixed = flat @ fn^T, split into pre/post/comb parts of hc, hc, hc*hc
 *   pre  = sigmoid(mixed_pre * scale[0] + base_pre) + hc_eps
 *   post = 2 sigmoid(mixed_post * scale[1] + base_post)             -> post [T][hc]
 *   comb = softmax_rows(mixed_comb * scale[2] + base_comb) + hc_eps, then a
 *          column normalisation and sinkhorn_iters - 1 (row, column) rounds,
 *          each x / (sum + hc_eps)                                  -> comb [T][hc][hc]
 *   collapsed = sum_i pre[i] streams[t][i]                          -> collapsed [T][d] (may be NULL)
 *   normed = bf16(rms_norm(collapsed) * norm_weight)               -> normed [T][d] (may be NULL;
 *            norm_weight f32 [d] or NULL for an unweighted norm, eps = norm_eps)
 * streams f32 [T][hc][d]; fn f32 [2 hc + hc^2][hc d]; base f32 [2 hc + hc^2];
 * scale f32 [3].  The reference routes the two-row case of the GEMV to
 * mx._expert_ssd_two_row_gemv (mhc.py:28-32).  Limits: hc <= 8, d % 4 == 0,
 * d <= 8192.
 */
int glm_hc_pre(void *stream, const float *streams, int T, int hc, int d, const float *fn,
               const float *base, const float *scale, int sinkhorn_iters, float rms_eps,
               float hc_eps, const float *norm_weight, float norm_eps, int flags, void *workspace,
               size_t workspace_bytes, float *post, float *comb, float *collapsed,
               uint16_t *normed);

/*
 * hyper_residual (mhc.py:51-60):
 *   out[t][j] = post[t][j] * y[t] + sum_i comb[t][i][j] * residual[t][i]
 * residual f32 [T][hc][d], y f32 [T][d] (the MoE layer's output), post f32
 * [T][hc], comb f32 [T][hc][hc] -> out f32 [T][hc][d].  flags: GLM_HC_BF16_STREAMS
 * when the residual streams are bf16 in the model (residual passed as f32).
 */
int glm_hc_post(void *stream, const float *residual, int T, int hc, int d, const float *y,
                const float *post, const float *comb, int flags, float *out);

/*
 * glm_moe_forward followed by the FFN site's hyper_residual (model.py:136,
 * mhc.py:51-60) on its output:
 *   hc_out[t][j] = post[t][j] * out[t] + sum_i comb[t][i][j] * residual[t][i]
 * residual f32 [T][hc][d] (the streams the site started from), post f32
 * [T][hc] and comb f32 [T][hc][hc] from glm_hc_pre; hc_out f32 [T][hc][d];
 * flags as glm_hc_post.  `out` is written too.  On the few-token path the
 * update runs inside the layer's last kernel (one launch less than
 * glm_moe_forward + glm_hc_post); otherwise it is a separate launch.  Same
 * limits as glm_moe_forward, hc <= 8.
 */
int glm_moe_forward_hc(void *stream, const uint16_t *x, int T, int d, const float *router_weight,
                       const float *router_bias, int E, int top_k, int n_group, int topk_group,
                       int norm_topk_prob, float routed_scaling_factor, int I,
                       const uint8_t *gate_packed, const uint8_t *gate_scales,
                       const uint8_t *up_packed, const uint8_t *up_scales,
                       const uint8_t *down_packed, const uint8_t *down_scales, int I_shared,
                       int shared_fmt, const void *shared_gate, const uint8_t *shared_gate_scales,
                       const void *shared_up, const uint8_t *shared_up_scales,
                       const void *shared_down, const uint8_t *shared_down_scales,
                       const uint16_t *shared_in, float swiglu_limit, void *workspace,
                       size_t workspace_bytes, float *out, float *weights_out,
                       uint32_t *indices_out, const float *residual, int hc, const float *post,
                       const float *comb, int flags, float *hc_out);

/*
 * RMSNorm (layers.py:119-131) and UnweightedRMSNorm (layers.py:134-140) of
 * f32 rows: out = x * (1 / sqrt(mean(x^2) + eps)) * weight (weight f32 [d] or
 * NULL); written as f32 (out) and/or rounded to bf16 (out_bf16).  d % 4 == 0.
 */
int glm_rms_norm(void *stream, const float *x, int T, int d, const float *weight, float eps,
                 float *out, uint16_t *out_bf16);

/* ------------------------------------------------------------ expert bank loading */

/* glm_file_read_ranges flag: drop the file's page-cache pages of the ranges
 * after reading them (the intent of the reference's no_file_cache option,
 * native_expert_ssd.py:102,337). */
#define GLM_READ_DROP_CACHE 1

/*
 * Reads n byte ranges of one file into host memory: dst[i] receives bytes
 * [offset[i], offset[i] + length[i]).  `threads` worker threads (1..256) pread
 * pieces of at most 2 MiB.  Replaces the file side of the reference's direct
 * expert reader, mx._open_expert_safetensors_direct (native_expert_ssd.py:
 * 320-339) + mx._expert_ssd_direct_load_into (native_expert_ssd.py:379-385).
 * Host-only: no GPU call.  Fails (GLM_ERR_INVALID_ARGUMENT) on an unreadable
 * file, a range past its end or a short read.
 */
int glm_file_read_ranges(const char *path, int n, const int64_t *offset, const int64_t *length,
                         void *const *dst, int threads, int flags);

/*
 * Moves n segments out of a device staging buffer on `stream`: segments is a
 * HOST table int64 [n][4] of {source offset in staging, destination device
 * address, bytes, tile_k}; tile_k > 0 marks a whole row-major MXFP4 matrix of
 * tile_k codes a row (bytes = rows * tile_k / 2, rows % 16 == 0, tile_k % 128
 * == 0, a 16-byte aligned destination) that lands in the bank layout,
 * tile_k == 0 a plain copy.  The table is validated against staging_bytes and copied to
 * device_table (device memory of at least 32 n bytes, owned by the caller and
 * kept until the stream has run the copy).  Replaces the device side of
 * mx._expert_ssd_direct_load_into (native_expert_ssd.py:379-385), which wrote
 * one expert's six tensors into its slot (allocate_slots,
 * native_expert_ssd.py:352-363); here one launch fills many experts' slots.
 */
int glm_bank_scatter(void *stream, const uint8_t *staging, int64_t staging_bytes,
                     const int64_t *segments, int n, int64_t *device_table);

/*
 * Checkpoint MXFP4 codes -> the bank layout: `count` consecutive row-major
 * matrices of rows x K codes (rows * K / 2 bytes each, K % 32 == 0) at src
 * are written to dst, tile-major when rows % 16 == 0 and K % 128 == 0 (src
 * and dst 16-byte aligned), else copied unchanged.  src and dst must not
 * overlap.  No counterpart in the reference, whose MLX kernels read the
 * checkpoint rows (native_expert_ssd.py:653-694): the tiles let one wave load
 * of the expert kernels read 1 KB of contiguous memory.
 */
int glm_mxfp4_tile(void *stream, const uint8_t *src, uint8_t *dst, int64_t count, int rows,
                   int K);

/* 1 when the bank stores a rows x K MXFP4 matrix tile-major, else 0. */
int glm_mxfp4_is_tiled(int rows, int K);

/*
 * Decodes n ScaleX Mode-A scale records (scale_codec.py:35-91,151-201) that
 * sit in a device staging buffer into raw E8M0 bytes.  records is a HOST
 * table int64 [n][13]: staging offset, encoded bytes, raw bytes, codec (0 raw,
 * 1 one bit, 2 two bits), palette (4 bytes, little-endian), primary bytes,
 * exception count, then (destination, bytes) for the gate, down and up scale
 * tensors of the expert, which receive the raw bytes in that order.  The
 * table is checked (lengths consistent with the codec, destinations covering
 * the raw bytes, records inside staging_bytes) and copied to device_table
 * (device memory of at least 104 n bytes, kept until the stream has run the
 * copy).  Exception positions must be ascending (the caller checks them; an
 * unordered list decodes wrongly but stays in bounds).  Replaces the per-call
 * Mode-B decode of the reference's ScaleX kernels (native_expert_ssd.py:
 * 653-694, docs/scalex-mode-b.md:29-33) for banks that keep plain scales:
 * the loader decodes once, when the layer is loaded into HBM.  Banks that keep
 * the Mode-B rows are decoded inside the few-token kernels on every call
 * instead (glm_moe_forward_scalex).
 */
int glm_scalex_decode(void *stream, const uint8_t *staging, int64_t staging_bytes,
                      const int64_t *records, int n, int64_t *device_table);

#ifdef __cplusplus
}
#endif

#endif /* GLM53_MOE_H */
