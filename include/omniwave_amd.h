/*
 * omniwave_amd — C ABI of the MI355X (gfx950) BiGEMM backend.
 *
 * Plain pointers and sizes only.  Every device pointer is caller-owned memory on the current
 * HIP device; the library never allocates or frees caller memory.  Launches are asynchronous
 * on the `stream` argument (a hipStream_t passed as void*; NULL = the null stream).  Every
 * entry point returns OW_OK (0) or an error code; ow_last_error() returns the message of the
 * calling thread's most recent failure.
 *
 * The upstream reference (QuackPhuc/omniwave) is pure Python; the interfaces each entry point
 * replaces are cited as reference file:line.
 */
#ifndef OMNIWAVE_AMD_H
#define OMNIWAVE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define OW_OK 0
#define OW_ERR_INVALID 1     /* bad argument (null pointer, negative size, inconsistent shape) */
#define OW_ERR_UNSUPPORTED 2 /* shape/dtype outside the kernel envelope */
#define OW_ERR_HIP 3         /* HIP runtime error (message names the call) */

/* Route kinds: the `route` strings of omniweave/models/routing.py:152-159. */
#define OW_ROUTE_LOCAL 0
#define OW_ROUTE_SHIFTED 1
#define OW_ROUTE_RADIX 2

/* Element types. */
#define OW_DTYPE_F32 0
#define OW_DTYPE_BF16 1
#define OW_DTYPE_F16 2

/* Fusion flags of ow_bigemm_fwd. */
#define OW_FUSE_NORM 1     /* x is raw; apply the block's RMSNorm (omniweave/models/block.py:83-85) */
#define OW_FUSE_RESIDUAL 2 /* write x + delta instead of delta (omniweave/models/block.py:108) */
#define OW_FUSE_FP8 4      /* fp8-e4m3 channel side with ow_pack_weights_fp8 weights (needs OW_FUSE_NORM) */

/*
 * Route plan descriptor: the arguments of build_route_plan
 * (omniweave/models/routing.py:128-137) plus the window/shift constants that
 * _local_token_order / _shifted_token_order hard-code (routing.py:57,71-72).
 */
typedef struct OwPlan {
  int32_t height;
  int32_t width;
  int32_t channels;
  int32_t spatial_tile; /* g */
  int32_t channel_tile; /* d */
  int32_t route;        /* OW_ROUTE_* */
  int32_t radix_level;
  int32_t window;       /* 4 in the reference */
  int32_t shift;        /* 2 in the reference */
} OwPlan;

/* Library version (major*10000 + minor*100 + patch). */
int ow_version(void);

/* Message of the calling thread's last failed call ("" if none). */
const char* ow_last_error(void);

/*
 * Q_s = ceil(H*W / g) token groups and Q_c = ceil(C / d) channel groups of a plan
 * (the shapes of RoutePlan.token_indices / channel_indices, routing.py:25-26).
 */
int ow_plan_dims(const OwPlan* plan, int32_t* q_s, int32_t* q_c);

/*
 * Host-side route tables.  Replaces build_route_plan (omniweave/models/routing.py:128-179):
 * writes token_index[Q_s*g] (pad = H*W) and channel_index[Q_c*d] (pad = C), identical to
 * RoutePlan.token_indices / channel_indices flattened row-major.  The masks are
 * (index < H*W) and (index < C).
 */
int ow_route_build(const OwPlan* plan, int32_t* token_index, int32_t* channel_index);

/*
 * Output-row table for a block whose output feeds space_to_depth(factor) (omniweave/models/
 * backbone.py:14-27,183-186): out_rows[i] = the row, within its image, that token
 * token_index[i] occupies in space_to_depth(out, factor) viewed as [H*W, C] rows (pad = H*W).
 * Pass it to ow_bigemm_fwd_rows to write the block output directly in that layout.
 */
int ow_route_s2d_rows(const OwPlan* plan, int32_t factor, const int32_t* token_index, int32_t* out_rows);

/*
 * Size in bytes of the packed weight buffer for q_c channel groups, channel tile d,
 * expanded tile rd and compute dtype (OW_DTYPE_BF16 / OW_DTYPE_F16 / OW_DTYPE_F32).
 */
size_t ow_packed_weight_bytes(int32_t q_c, int32_t d, int32_t rd, int32_t compute_dtype);

/*
 * Pack the block's BiGEMM weights into the MFMA operand order the forward kernel reads.
 * Replaces the per-call weight pre-cast of the accelerated backend
 * (omniweave/ops/triton.py:221-230).  a_u/a_v/a_o: [g,g]; b_u/b_v: [q_c,d,rd];
 * b_o: [q_c,rd,d]; all contiguous, element type weight_dtype (any OW_DTYPE_*).
 *
 * Folded into the packed values (then rounded to compute_dtype, nearest-even):
 *   B_u rows x -log2(e), B_v rows x -ln(2)   (SiLU evaluated as U'V'/(1 + 2^U'));
 *   B_u / B_v row c of group q x norm_weight[channel_index[q*d + c]] when norm_weight is
 *   non-NULL (the block's RMSNorm weight);
 *   B_o column c of group q x gamma[channel_index[q*d + c]] when gamma is non-NULL (the
 *   LayerScale, [C] fp32; omniweave/ops/reference.py:168-171 scales delta by it).
 * With channel_index given, rows / columns of pad channels are packed as 0.  A buffer packed
 * with norm_weight must be used with OW_FUSE_NORM, one packed without it without
 * OW_FUSE_NORM.  channel_index: device table of ow_route_build (required when norm_weight or
 * gamma is non-NULL).  `packed` must hold ow_packed_weight_bytes(...).
 */
int ow_pack_weights(const void* a_u, const void* a_v, const void* a_o,
                    const void* b_u, const void* b_v, const void* b_o,
                    int32_t weight_dtype, const float* norm_weight, const float* gamma,
                    const int32_t* channel_index, int32_t channels,
                    int32_t g, int32_t q_c, int32_t d, int32_t rd,
                    int32_t compute_dtype, void* packed, void* stream);

/*
 * fp8 inference variant (no counterpart in the reference, which has no fp8 path): the
 * channel-side product V' = P B_v'' runs on the K = 64 e4m3 MFMA with fp32 accumulation; the
 * token side, U' = P B_u'', the gate, Z B_o and A_o W stay in the activation dtype (each
 * e4m3-quantised operand adds ~2.6% rel-L2 to delta; quantising U' as well would put delta
 * past 5e-2 of fp32).  Per-tensor scales: B_v'' by its absmax over all channel groups; P_v by
 * the static bound ||A_v||_inf sqrt(C) that the RMSNorm'd rows obey (hence OW_FUSE_NORM), its
 * multiplier folded into the token operand; V''s dequantisation folded into the packed B_o.
 * Packed layout: the token-side head (act_dtype), 16 scale floats, then per (q, 32-row chunk)
 * in 1 KB units the act_dtype B_u'' fragments, the fp8 B_v'' K64 fragments (2 KB each) and the
 * act_dtype B_o fragments, padded to a multiple of 4 units.  Arguments as ow_pack_weights;
 * `packed` holds ow_packed_weight_bytes_fp8(q_c, d, rd) bytes.
 */
size_t ow_packed_weight_bytes_fp8(int32_t q_c, int32_t d, int32_t rd);
int ow_pack_weights_fp8(const void* a_u, const void* a_v, const void* a_o,
                        const void* b_u, const void* b_v, const void* b_o,
                        int32_t weight_dtype, const float* norm_weight, const float* gamma,
                        const int32_t* channel_index, int32_t channels,
                        int32_t g, int32_t q_c, int32_t d, int32_t rd,
                        int32_t act_dtype, void* packed, void* stream);

/*
 * RMSNorm row scales: scale[i] = rsqrt(mean_c(x[i, c]^2) + eps) for rows x [rows, channels],
 * with the reference's rounding points (mean in fp32, then var, var + eps and rsqrt each
 * rounded to `dtype`; omniweave/models/block.py:83-84).  Replaces the variance/rsqrt part of
 * OmniWeaveBlock.forward's RMSNorm.
 */
int ow_rms_scale(const void* x, float* scale, int64_t rows, int32_t channels, float eps,
                 int32_t dtype, void* stream);

/*
 * Workspace bytes ow_bigemm_fwd may need: batch*H*W fp32 row scales with OW_FUSE_NORM, else 0.
 * Only launches whose RMSNorm statistics come from a separate pass use it (fp32 activations,
 * element access for ragged / unaligned rows, or a channel count the in-kernel statistics do
 * not cover); for the others `workspace` may be NULL and workspace_bytes 0.
 */
size_t ow_fwd_workspace_bytes(const OwPlan* plan, int32_t batch, int32_t flags);

/*
 * Fused BiGEMM forward.  Replaces bigemm(..., backend) (omniweave/ops/bigemm.py:24-73) and,
 * with flags, the RMSNorm -> bigemm -> residual sequence of OmniWeaveBlock.forward
 * (omniweave/models/block.py:80-108, eval mode).
 *
 *   x, out        [batch, H*W, C] NHWC, element type `dtype` (out may not alias x;
 *                 both may be NULL when batch == 0, which launches nothing)
 *   eps           RMSNorm epsilon (1e-6 in the reference), used with OW_FUSE_NORM
 *   packed        ow_pack_weights output for this (q_c, d, rd, dtype) with the block's
 *                 LayerScale gamma folded in, packed with the RMSNorm weight exactly when
 *                 flags has OW_FUSE_NORM
 *   packed_bytes  size of `packed`; must equal ow_packed_weight_bytes(q_c, d, rd, dtype)
 *   token_index   device copy of ow_route_build's token table [Q_s*g]
 *   channel_index device copy of ow_route_build's channel table [Q_c*d]
 *   workspace     ow_fwd_workspace_bytes(plan, batch, flags) bytes of device memory when the
 *                 launch needs it (see ow_fwd_workspace_bytes), else may be NULL
 *
 * For every tile (b, q_s, q_c): T = rows token_index[q_s,:] x columns channel_index[q_c,:]
 * of x (pads read as zero; RMSNorm-scaled with OW_FUSE_NORM), delta = A_o (SiLU(A_u T B_u) *
 * (A_v T B_v)) B_o scaled per column by gamma; valid rows/columns are written back to their
 * NHWC positions (omniweave/ops/reference.py:120-173).  With OW_FUSE_NORM the row scales
 * come from the same read of x when d = 64, rd = 128 and C = q_c * 64 with q_c <= 4 (and
 * x, out 16-byte aligned); otherwise they are computed first (ow_rms_scale into the
 * workspace), on the same stream.  Envelope: g = 16, d in {64,128}, rd in {128,256}, dtype
 * in {bf16, f16}.
 */
int ow_bigemm_fwd(const void* x, void* out, float eps,
                  const void* packed, size_t packed_bytes,
                  const int32_t* token_index, const int32_t* channel_index,
                  const OwPlan* plan, int32_t batch, int32_t rd, int32_t dtype,
                  int32_t flags, void* workspace, size_t workspace_bytes, void* stream);

/*
 * ow_bigemm_fwd with the output rows permuted: token slot i (token_index[i] of image b) is
 * written to row b*H*W + out_rows[i] of out instead of row b*H*W + token_index[i]; the input
 * rows, residual and RMSNorm are unchanged.  out_rows (device, [Q_s*g], pad = H*W) must map
 * the valid slots one-to-one onto [0, H*W), e.g. ow_route_s2d_rows, so that the block and the
 * space_to_depth after it (omniweave/models/backbone.py:183-186) are one pass over HBM.
 * bf16 / f16 activations only.
 */
int ow_bigemm_fwd_rows(const void* x, void* out, float eps,
                       const void* packed, size_t packed_bytes,
                       const int32_t* token_index, const int32_t* channel_index, const int32_t* out_rows,
                       const OwPlan* plan, int32_t batch, int32_t rd, int32_t dtype,
                       int32_t flags, void* workspace, size_t workspace_bytes, void* stream);

/*
 * ow_bigemm_fwd / ow_bigemm_fwd_rows (out_rows may be NULL) for consecutive blocks of a stage
 * (omniweave/models/backbone.py:75-80, each block's RMSNorm at omniweave/models/block.py:83-84
 * reading the previous block's output).  With stats_out non-NULL ([batch*H*W, Q_c] floats)
 * the launch may also write, per output row and channel group, the sum of squares of the
 * stored values of the group's columns; *stats_written (host) says whether it did (bf16 /
 * f16, contiguous channel groups, the streamed d = 128 kernel, out_rows NULL).  Passing those
 * sums to the next block as stats_in (stats_in_parts = that block's predecessor's Q_c) gives
 * it its RMSNorm statistics without reading whole rows; the result equals ow_bigemm_fwd's up
 * to the summation order of the mean of squares.  Needs OW_FUSE_NORM with stats_in; bf16 /
 * f16 activations only.  stats_in and stats_out must not overlap (the launch reads one while
 * other workgroups write the other; overlapping ranges are rejected with OW_ERR_INVALID).
 */
int ow_bigemm_fwd_chain(const void* x, void* out, float eps,
                        const void* packed, size_t packed_bytes,
                        const int32_t* token_index, const int32_t* channel_index, const int32_t* out_rows,
                        const OwPlan* plan, int32_t batch, int32_t rd, int32_t dtype, int32_t flags,
                        const float* stats_in, int32_t stats_in_parts, float* stats_out,
                        int32_t* stats_written, void* workspace, size_t workspace_bytes, void* stream);

/*
 * ow_bigemm_fwd (drop_scale NULL) or ow_bigemm_fwd_drop for training, also handing the RMSNorm
 * row scales r = 1 / sqrt(mean_c x^2 + eps) that the launch applied to the backward (the
 * reference's autograd keeps its normalised activations, omniweave/models/block.py:83-108, and
 * ow_bwd_rmsnorm / ow_bwd_fused_routed need r): where the launch forms every row's scale in one
 * place -- the statistics pass, or the d = 64 16-token kernel -- it writes them to row_scale
 * ([batch * H * W] fp32, device) and sets *scales_written to 1; otherwise *scales_written is 0
 * and the caller forms them with ow_rms_scale.  Needs OW_FUSE_NORM for any scales to be written.
 */
int ow_bigemm_fwd_scales(const void* x, void* out, float eps, const void* packed, size_t packed_bytes,
                         const int32_t* token_index, const int32_t* channel_index, const OwPlan* plan,
                         int32_t batch, int32_t rd, int32_t dtype, int32_t flags, const float* drop_scale,
                         float* row_scale, int32_t* scales_written, void* workspace, size_t workspace_bytes,
                         void* stream);

/*
 * ow_bigemm_fwd for training with per-sample drop-path (stochastic depth,
 * omniweave/models/block.py:99-107): drop_scale [batch] (fp32, device) multiplies each image's
 * rounded delta before the residual, out = round(x + round(round(delta) * drop_scale[b])) (or
 * round(round(delta) * drop_scale[b]) without OW_FUSE_RESIDUAL; fp32 activations: one fp32
 * product).  drop_scale[b] = keep_mask[b] * (1 / keep_probability) reproduces the reference's
 * delta * keep_mask / keep_probability, whose division by a scalar PyTorch evaluates on the
 * GPU as a product with the fp32 reciprocal.  Other arguments as ow_bigemm_fwd.
 */
int ow_bigemm_fwd_drop(const void* x, void* out, float eps,
                       const void* packed, size_t packed_bytes,
                       const int32_t* token_index, const int32_t* channel_index,
                       const OwPlan* plan, int32_t batch, int32_t rd, int32_t dtype,
                       int32_t flags, const float* drop_scale, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * ow_bigemm_fwd without a workspace argument.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops with
 * a fixed footprint, harnesses that forbid hipMalloc).  The RMSNorm row scales that
 * ow_bigemm_fwd keeps in its workspace (see ow_fwd_workspace_bytes) go to a scratch array in
 * the library's device memory instead: 1,048,576 fp32 rows (4 MiB), held on each GPU the
 * library runs on until the process ends.  A launch that would need more rows (batch * H * W)
 * is rejected with OW_ERR_UNSUPPORTED before any device work.  The call allocates nothing; the
 * first call on a device looks up the array's address there (hipGetSymbolAddress).  All calls
 * on one GPU share its array, so calls that overlap on one GPU (concurrent streams, threads)
 * race; calls ordered on one stream do not.  Results equal ow_bigemm_fwd's bit for bit.
 */
int ow_bigemm_fwd_noalloc(const void* x, void* out, float eps,
                          const void* packed, size_t packed_bytes,
                          const int32_t* token_index, const int32_t* channel_index,
                          const OwPlan* plan, int32_t batch, int32_t rd, int32_t dtype,
                          int32_t flags, void* stream);

/*
 * Backbone stem as one gather-GEMM (omniweave/models/backbone.py:121,173-176): image
 * [batch, 3, height, width] (NCHW) -> space_to_depth(4) -> x W^T with weight [n_out, 48]
 * (nn.Linear(48, n_out, bias=False), input order (row offset, column offset, channel)) ->
 * out [batch, height/4, width/4, n_out] (NHWC).  fp32 accumulation, one rounding to dtype
 * (OW_DTYPE_BF16 or OW_DTYPE_F16; image, weight and out share it).  height, width divisible
 * by 4; n_out in {32, 64, 96, 128, 192, 256}; image 8-byte, out 16-byte aligned.
 */
int ow_stem_fwd(const void* image, const void* weight, void* out, int32_t batch, int32_t height,
                int32_t width, int32_t n_out, int32_t dtype, void* stream);

/*
 * Backward building blocks.  Replace the fp32 autograd recompute of the accelerated backend
 * (omniweave/ops/triton.py:256-292); the plain channel-side GEMMs between them are the
 * caller's (batched hipBLASLt).  Notation: slots = batch * Q_s * 16 token slots per channel
 * group (pad slots included), tensors [Q_c][slots][d] are slot-major, compute dtype `dtype`
 * (OW_DTYPE_BF16, OW_DTYPE_F16, or OW_DTYPE_F32 for fp32 activations: fp32 tiles and plain
 * fp32 kernels; the alignment and multiple-of-8 conditions below are for the 16-bit types).
 */

/* out[b][i] = x[b][i] * scale[b] rounded to dtype, for b < batch and i < per_sample: the
 * gradient of the delta branch under drop-path (the autograd of delta * keep_mask /
 * keep_probability, omniweave/models/block.py:99-107, with scale = keep_mask / keep_probability
 * as in ow_bigemm_fwd_drop).  out may alias x. */
int ow_scale_samples(const void* x, const float* scale, void* out, int32_t batch, int64_t per_sample,
                     int32_t dtype, void* stream);

/* Folded weights as plain matrices: B_u'' = -log2(e) w B_u and B_v'' = -ln(2) w B_v
 * ([q_c][d][rd] and transposed [q_c][rd][d]), B_o'' = B_o diag(gamma) ([q_c][rd][d] and
 * transposed [q_c][d][rd]); w = norm_weight (NULL: 1), pad channels 0. */
int ow_fold_weights(const void* b_u, const void* b_v, const void* b_o, int32_t weight_dtype,
                    const float* norm_weight, const float* gamma, const int32_t* channel_index,
                    int32_t channels, int32_t q_c, int32_t d, int32_t rd, int32_t compute_dtype,
                    void* bu, void* bu_t, void* bv, void* bv_t, void* bo, void* bo_t, void* stream);

/* Routed tiles of x * r (r = rscale per row, NULL: 1) and of dy into [Q_c][slots][d]
 * (pack_tiles, omniweave/ops/reference.py:16-64, for both tensors; pads 0).  d % 8 == 0;
 * xt, dyt 16-byte aligned. */
int ow_bwd_gather(const void* x, const void* dy, const float* rscale, const int32_t* token_index,
                  const int32_t* channel_index, const OwPlan* plan, int32_t batch, int32_t dtype,
                  void* xt, void* dyt, void* stream);

/* SiLU-gate backward over n folded values: z = u v s, du = dz v s (1 - ln2 u (1 - s)),
 * dv = dz u s with s = 1 / (1 + 2^u) (SiLU(U) V and its gradient, reference.py:159).
 * n % 8 == 0; all six buffers 16-byte aligned. */
int ow_bwd_gate(const void* u, const void* v, const void* dz, void* z, void* du, void* dv, int64_t n,
                int32_t dtype, void* stream);

/* [Q_c][slots][d] tiles -> g [batch * H * W, C] (dtype) at their routed positions
 * (unpack_tiles, reference.py:67-117; pads dropped).  Every element of g is written (the
 * routes are permutations), so g needs no clearing.  d % 8 == 0; dxt 16-byte aligned. */
int ow_bwd_scatter(const void* dxt, const int32_t* token_index, const int32_t* channel_index,
                   const OwPlan* plan, int32_t batch, int32_t dtype, void* g, void* stream);

/* Token mixing of 16-row tiles (the A_{u,v,o} products of reference.py:155-162 and their
 * transposes): out_tile = m1 in1_tile (+ m2 in2_tile when in2 is non-NULL); m1, m2 [16][16]
 * fp32 row-major on the device; in/out [n_tiles][16][d], d in {64, 128}. */
int ow_tile_mix(const void* in1, const float* m1, const void* in2, const float* m2, void* out,
                int64_t n_tiles, int32_t d, int32_t dtype, void* stream);

/* Gradient of a token matrix: partial[i][j][w] = (sum over the tiles of wave w of
 * in1_tile in2_tile^T)[i][j] (fp32, [16][16][n_waves], w < n_waves, tiles assigned
 * round-robin); the caller sums over w (a fixed order, so the result is deterministic). */
int ow_tile_outer(const void* in1, const void* in2, float* partial, int32_t n_waves, int64_t n_tiles,
                  int32_t d, int32_t dtype, void* stream);

/* Per row: dx = (residual ? dout : 0) + r g - x r^3 / C sum_c(g x) with rscale, or + g
 * without it (the RMSNorm and residual of omniweave/models/block.py:83-108). */
int ow_bwd_rmsnorm(const void* x, const void* g, const float* rscale, const void* dout, void* dx,
                   int64_t rows, int32_t channels, int32_t residual, int32_t dtype, void* stream);

/* Packed weights of the fused backward (d 64 or 128, rd 128 or 256): per channel group and
 * 32-row chunk, the folded B_u'', B_v'', B_o'' as the forward's and transposed 32x32x16 MFMA
 * operands (3 d / 16 + 6 d / 32 fragments of 1 KB: 24 at d = 64, 48 at d = 128);
 * ow_bwd_packed_bytes gives the size. */
size_t ow_bwd_packed_bytes(int32_t q_c, int32_t d, int32_t rd);
int ow_pack_bwd_weights(const void* b_u, const void* b_v, const void* b_o, int32_t weight_dtype,
                        const float* norm_weight, const float* gamma, const int32_t* channel_index,
                        int32_t channels, int32_t q_c, int32_t d, int32_t rd, int32_t compute_dtype,
                        void* packed, void* stream);

/* The d = 64 backward in one kernel (replaces ow_tile_mix x4, ow_tile_outer x3 and the
 * channel-side GEMMs; the reference's fp32 autograd recompute, omniweave/ops/triton.py:256-292):
 * from the routed tiles X' and dY ([q_c][slots][64], ow_bwd_gather) and the fp32 [16][16] token
 * matrices, per 32-slot pair: P_u = A_u X', P_v = A_v X', dW' = A_o^T dY (stored to pu, pv, dw,
 * [q_c][slots][64] elements, each row in the pair-operand channel order: element 16 k + 8 h + j
 * is channel 16 k + 8 (j / 4) + 4 h + j % 4, as ow_bwd_param_reduce64 reads them), U'^T, V'^T,
 * dZ^T and the gate backward per 32-row chunk, W' = Z B_o'', dP_u = dU' B_u''^T, dP_v = dV' B_v''^T,
 * dX' = A_u^T dP_u + A_v^T dP_v (stored to dxt), and the token-matrix gradients dA_u = sum
 * dP_u X'^T, dA_v = sum dP_v X'^T, dA_o = sum dY W'^T as per-workgroup fp32 partials
 * partial[w][3][256] (w < n_partial = ow_bwd_fused_partials(slots, q_c, rd); element 16 t + k),
 * which the caller sums over w.  slots % 32 == 0, bf16 / f16. */
int64_t ow_bwd_fused_partials(int64_t slots, int32_t q_c, int32_t rd);
int ow_bwd_fused(const void* xt, const void* dyt, const float* a_u, const float* a_v, const float* a_o,
                 const void* packed, size_t packed_bytes, void* pu, void* pv, void* dw, void* dxt, float* partial,
                 int64_t n_partial, int64_t slots, int32_t q_c, int32_t d, int32_t rd, int32_t dtype, void* stream);

/* The d = 128 backward's token side and first channel-side products in one kernel (replaces
 * ow_tile_mix x3, the U'/V'/dZ GEMMs and ow_bwd_gate of the composed backward; the reference's
 * fp32 autograd recompute, omniweave/ops/triton.py:256-292): from the routed tiles X' and dY
 * ([q_c][slots][128], ow_bwd_gather) and the fp32 [16][16] token matrices, per 32-slot pair
 * P_u = A_u X', P_v = A_v X', dW' = A_o^T dY (stored to pu, pv, dw, [q_c][slots][128]) and per
 * 32-row chunk of the expanded dimension U'^T, V'^T, dZ^T and the gate backward, stored as z,
 * du, dv ([q_c][slots][rd]).  packed from ow_pack_bwd_weights with d = 128; slots % 16 == 0,
 * bf16 / f16, every buffer 16-byte aligned and below 2 GiB. */
int ow_bwd_channel(const void* xt, const void* dyt, const float* a_u, const float* a_v, const float* a_o,
                   const void* packed, size_t packed_bytes, void* pu, void* pv, void* dw, void* z, void* du,
                   void* dv, int64_t slots, int32_t q_c, int32_t d, int32_t rd, int32_t dtype, void* stream);

/* The rest of the d = 128 backward's channel side in one kernel (replaces the W'/dP GEMMs,
 * ow_tile_outer x3 and the dX' ow_tile_mix): from z, du, dv of ow_bwd_channel and the tiles X',
 * dY, per 32-slot pair dP_u = dU' B_u''^T, dP_v = dV' B_v''^T, dX' = A_u^T dP_u + A_v^T dP_v
 * (stored to dxt, [q_c][slots][128]), W' = Z B_o'' and the token-matrix gradients dA_u = sum
 * dP_u X'^T, dA_v = sum dP_v X'^T, dA_o = sum dY W'^T as per-workgroup fp32 partials
 * partial[w][3][256] (w < n_partial = ow_bwd_channel_partials(slots, q_c); element 16 t + k),
 * which the caller sums over w.  Shapes and alignment as ow_bwd_channel. */
int64_t ow_bwd_channel_partials(int64_t slots, int32_t q_c);
int ow_bwd_channel2(const void* xt, const void* dyt, const void* z, const void* du, const void* dv,
                    const float* a_u, const float* a_v, const void* packed, size_t packed_bytes, void* dxt,
                    float* partial, int64_t n_partial, int64_t slots, int32_t q_c, int32_t d, int32_t rd,
                    int32_t dtype, void* stream);

/* ow_bwd_channel and ow_bwd_channel2 with the routing folded in (replace ow_bwd_gather before
 * them and ow_bwd_scatter after them), for plans whose channel order is the identity (radix
 * level 0 or one channel group) and C = q_c * 128.  Slot (image b, token group s, row t) of
 * group q is row b * H * W + token_index[16 s + t] of x, dy ([batch * H * W][C]) at columns
 * 128 q ..; pad slots read as zero.  ow_bwd_channel_routed folds the RMSNorm scales (rscale
 * [batch * H * W], NULL without the norm) into the token matrices (P_u = A_u diag(r) x);
 * ow_bwd_channel2_routed forms X' = x r rounded to the compute dtype (as ow_bwd_gather) for the
 * token-matrix gradients and writes dX' to g[b * H * W + token_index[16 s + t]][128 q ..]
 * (every element of g [batch * H * W][C] once) instead of dxt.  slots = batch * q_s * 16; the
 * other arguments as in ow_bwd_channel / ow_bwd_channel2; x, dy, g 16-byte aligned and below
 * 2 GiB. */
int ow_bwd_channel_routed(const void* x, const void* dy, const float* rscale, const int32_t* token_index,
                          const OwPlan* plan, int32_t batch, const float* a_u, const float* a_v, const float* a_o,
                          const void* packed, size_t packed_bytes, void* pu, void* pv, void* dw, void* z, void* du,
                          void* dv, int32_t rd, int32_t dtype, void* stream);
int ow_bwd_channel2_routed(const void* x, const void* dy, const float* rscale, const void* z, const void* du,
                           const void* dv, const float* a_u, const float* a_v, const void* packed, size_t packed_bytes,
                           const int32_t* token_index, const OwPlan* plan, int32_t batch, void* g, float* partial,
                           int64_t n_partial, int32_t rd, int32_t dtype, void* stream);

/* Parameter-gradient reduction of the d = 64 backward (replaces the slot-reduction GEMMs over
 * the intermediates, omniweave/ops/triton.py:256-292 through autograd): from pu, pv, dw
 * ([q_c][slots][64], as ow_bwd_fused / ow_bwd_fused_routed write them) and the packed weights of
 * the same call (ow_pack_bwd_weights), U' = P_u B_u'', V' = P_v B_v'', dZ = dW' B_o''^T and the
 * gate backward (Z, dU', dV') are recomputed per 32-slot pair and the sums over slot ranges of
 * dB_u'' = P_u^T dU', dB_v'' = P_v^T dV' (each [64][rd]) and dB_o'' = Z^T dW' ([rd][64]) per
 * channel group are formed, fp32.  partial holds n_partial =
 * ow_bwd_param_reduce64_partials(slots, q_c, rd) rows of 3 * 64 * rd floats (a multiple of q_c):
 * R = n_partial / q_c ranges, each a [3][q_c][64 * rd] block (product, group), so the gradients
 * are the sum of the R blocks (ow_sum_rows with rows R, cols 3 * q_c * 64 * rd).
 * slots % 32 == 0, rd in {128, 256}, bf16 / f16. */
int64_t ow_bwd_param_reduce64_partials(int64_t slots, int32_t q_c, int32_t rd);
int ow_bwd_param_reduce64(const void* pu, const void* pv, const void* dw, const void* packed, size_t packed_bytes,
                          float* partial, int64_t n_partial, int64_t slots, int32_t q_c, int32_t rd, int32_t dtype,
                          void* stream);

/* The same reduction for d = 128, from the slot-major intermediates of ow_bwd_channel /
 * ow_bwd_channel_routed (pu, pv, dw [q_c][slots][128]; z, du, dv [q_c][slots][rd], rows in slot
 * order): partial holds n_partial = ow_bwd_param_reduce128_partials(slots, q_c, rd) rows of
 * 3 * 128 * rd floats, R = n_partial / q_c blocks [3][q_c][128 * rd] whose sum (ow_sum_rows) is
 * dB_u'', dB_v'' ([128][rd] per group) and dB_o'' ([rd][128]).  slots % 16 == 0, rd in
 * {128, 256}, bf16 / f16; each intermediate below 2 GiB. */
int64_t ow_bwd_param_reduce128_partials(int64_t slots, int32_t q_c, int32_t rd);
int ow_bwd_param_reduce128(const void* pu, const void* pv, const void* dw, const void* z, const void* du,
                           const void* dv, float* partial, int64_t n_partial, int64_t slots, int32_t q_c, int32_t rd,
                           int32_t dtype, void* stream);

/* out[c] = sum over r < rows of partial[r * cols + c], fp32, in a fixed order for given rows
 * and cols (run to run identical): the sums of the per-workgroup partials above and of the
 * token-matrix partials of ow_bwd_fused / ow_bwd_channel2 (the reference's autograd sums them
 * inside its GEMMs, omniweave/ops/triton.py:256-292).  cols % 4 == 0, both pointers 16-byte
 * aligned, rows >= 1. */
int ow_sum_rows(const float* partial, int64_t rows, int64_t cols, float* out, void* stream);

/* ow_bwd_fused with the routing folded in, for plans whose channel order is the identity
 * (radix level 0 or one channel group) and C = q_c * 64 (replaces ow_bwd_gather and
 * ow_bwd_scatter around it as well): X' = x r and dY rows are read from x, dy ([rows][C],
 * rscale as in ow_bwd_gather, NULL without the RMSNorm) through the token table, and dX' is
 * written to g ([rows][C], every element once) for ow_bwd_rmsnorm.  The other outputs as in
 * ow_bwd_fused (slots = batch * q_s * 16). */
int ow_bwd_fused_routed(const void* x, const void* dy, const float* rscale, const int32_t* token_index,
                        const OwPlan* plan, int32_t batch, const float* a_u, const float* a_v, const float* a_o,
                        const void* packed, size_t packed_bytes, void* pu, void* pv, void* dw, void* g,
                        float* partial, int64_t n_partial, int32_t rd, int32_t dtype, void* stream);

/* Parameter gradients from the folded ones (dbu, dbv [q_c][d][rd], dbo [q_c][rd][d], fp32):
 * g_bu, g_bv, g_bo (fp32, parameter shapes), g_gamma [C] and, with norm_weight, g_norm_weight
 * [C] (each channel written once). */
int ow_bwd_params(const void* b_u, const void* b_v, const void* b_o, int32_t weight_dtype,
                  const float* norm_weight, const float* gamma, const int32_t* channel_index,
                  int32_t channels, int32_t q_c, int32_t d, int32_t rd, const float* dbu,
                  const float* dbv, const float* dbo, float* g_bu, float* g_bv, float* g_bo,
                  float* g_gamma, float* g_norm_weight, void* stream);

/* The backward's small parameters (norm weight, gamma, A_u, A_v, A_o; the reference's autograd
 * takes them in fp32, omniweave/ops/triton.py:256-292) converted into one fp32 buffer in one
 * launch: source k (dtype[k] in OW_DTYPE_*, count[k] values) goes to dst at the sum of the
 * counts before it.  1 <= n <= 8. */
int ow_small_to_f32(const void* const* src, const int32_t* dtype, const int64_t* count, int32_t n, float* dst,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OMNIWAVE_AMD_H */
