/*
 * msda.h — C ABI of the MI355X (gfx950) multi-scale deformable-attention library.
 *
 * The library computes RF-DETR-JAX's deformable-attention core: bilinear, zero-padded sampling of
 * a multi-level value map at per-query sample positions, weighted by per-sample attention weights
 * and summed over levels x points; and the three gradients of that map (value, sampling
 * locations, attention weights).
 *
 * Reference interface replaced (paths are into the RF-DETR-JAX source tree):
 *   msda_fwd  <- ms_deform_attn_core_rows(value, spatial_shapes, sampling_locations,
 *                attention_weights, sampler)            src/rfdetr_jax/models/ops.py:208-292
 *                (the per-level sampler _sample_rows,   ops.py:64-134, and the point-weighted
 *                einsum,                                ops.py:289)
 *   msda_bwd  <- the VJP of the same function, which the reference obtains by JAX autodiff of
 *                ops.py:64-134 + ops.py:289, and which its fused TPU sampler implements by hand
 *                in _sample_bwd / _backward_kernel      src/rfdetr_jax/models/deform_pallas.py:97-120,157-175
 *
 * Layouts (all row-major, contiguous):
 *   value                 [batch * n_heads, len_value, head_dim]    value_dtype   (ops.py:218)
 *   sampling_locations    [batch, len_query, n_heads, n_levels, n_points, 2]  f32, (x, y) in [0,1]
 *   attention_weights     [batch, len_query, n_heads, n_levels * n_points]    f32, level-major
 *   output                [batch, len_query, n_heads * head_dim]    output_dtype  (ops.py:229)
 *   spatial_shapes        host int32 [n_levels][2] = (H_l, W_l)
 *   level_start_index     host int32 [n_levels] = prefix sums of H_l * W_l (may be NULL)
 *   len_value             sum over levels of H_l * W_l
 *
 * Semantics: torch grid_sample(mode="bilinear", padding_mode="zeros", align_corners=False) on the
 * normalised grid 2*loc-1, exactly as ops.py:83-134 and ops.py:270 state it. Sample coordinates
 * are computed in f32 without fused multiply-adds so floor() decisions match the reference.
 *
 * Calls are enqueue-only on `stream` (a hipStream_t, passed as void*; NULL = default stream):
 * no allocation, no host synchronisation, no global mutable state beyond one-time per-device
 * initialisation. All buffers, including the backward's scratch workspace, are owned by the
 * caller. Inputs are read-only; every output element is written by the call (grad_value needs no
 * zero-initialisation).
 *
 * Return values: MSDA_OK (0) or a negative MSDA_ERR_* code; msda_last_error() then returns a
 * message for the calling thread. Argument validation happens before any HIP call.
 */
#ifndef MSDA_H_
#define MSDA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum msda_dtype {
  MSDA_DTYPE_F32 = 0,
  MSDA_DTYPE_BF16 = 1
};

enum msda_status {
  MSDA_OK = 0,
  MSDA_ERR_INVALID_ARGUMENT = -1, /* shapes, pointers or level table inconsistent */
  MSDA_ERR_UNSUPPORTED = -2,      /* valid but outside what the kernels handle (dtype, head_dim) */
  MSDA_ERR_LAUNCH = -3,           /* a kernel launch failed */
  MSDA_ERR_DEVICE = -4            /* a HIP runtime query failed */
};

/*
 * The reference's sampler names (ms_deform_attn_core_rows's `sampler`, ops.py:208-241), for
 * msda_fwd_sampler / msda_bwd_sampler. MSDA_SAMPLER_HIP is this library's own: f32 interpolation
 * throughout, what msda_fwd / msda_bwd compute.
 */
enum msda_sampler {
  MSDA_SAMPLER_HIP = 0,
  MSDA_SAMPLER_GATHER = 1,     /* ops.py:64-134 _sample_rows */
  MSDA_SAMPLER_GATHER_F32 = 2, /* ops.py:137-144 _sample_rows_f32 */
  MSDA_SAMPLER_MATMUL = 3,     /* ops.py:147-186 _sample_rows_matmul */
  MSDA_SAMPLER_AUTO = 4,       /* per level: matmul when H * W <= 4096, else gather (ops.py:42, :277-279) */
  MSDA_SAMPLER_PALLAS = 5      /* deform_pallas.py:193-228 sample_weighted */
};

/* Maximum number of feature levels per call. */
#define MSDA_MAX_LEVELS 16

/* Library version string, e.g. "msda-gfx950 0.1.0". */
const char* msda_version(void);

/* Message describing the last failed call on the calling thread ("" if none). */
const char* msda_last_error(void);

/*
 * Process-wide override of a launch-tuning knob (an MSDA_* name, e.g. "MSDA_BWD_BANDS"); value
 * NULL removes the override. Knobs otherwise come from the environment, read once per name at its
 * first use. They choose launch shapes: results stay within the documented tolerances. The knobs
 * that select the opt-in sorted-gather backward (MSDA_BWD_GATHER*) or force banded backward plans
 * (MSDA_BWD_FORCE_BANDS) change msda_bwd_workspace_size's answer: query it after setting them.
 * Not to be called while another thread launches.
 * No counterpart in the reference; for benchmarks and tests that compare launch variants.
 * Returns MSDA_OK, or MSDA_ERR_INVALID_ARGUMENT for a name that does not start with "MSDA_".
 */
int msda_set_tuning(const char* name, const char* value);

/*
 * Forward: output = sum_{l,p} A[b,q,h,l*P+p] * bilinear(value[b*H+h], level l, loc[b,q,h,l,p]).
 * Replaces ms_deform_attn_core_rows (src/rfdetr_jax/models/ops.py:208-292) and its "pallas"
 * branch (ops.py:243-263 -> deform_pallas.py:193-228 sample_weighted), interpolating in f32
 * throughout; msda_fwd_sampler adds a named sampler's rounding points.
 * output_dtype is the dtype of result_type(value, attention_weights) in the reference (ops.py:260),
 * i.e. MSDA_DTYPE_F32 whenever the weights are f32; MSDA_DTYPE_BF16 is accepted for callers that
 * keep bf16 weights.
 */
int msda_fwd(const void* value, int value_dtype,
             const float* sampling_locations, const float* attention_weights,
             void* output, int output_dtype,
             int batch, int n_heads, int head_dim, int len_query,
             int n_levels, int n_points,
             const int32_t* spatial_shapes, const int32_t* level_start_index,
             int64_t len_value, void* stream);

/*
 * msda_fwd computing what the named reference sampler computes (`sampler`: enum msda_sampler),
 * the `sampler` argument of ms_deform_attn_core_rows (ops.py:208-292). They differ in where a bf16
 * value map is rounded and in how the Pallas kernel forms pixel coordinates; with an f32 value
 * map gather, gather-f32, matmul and auto are the f32 interpolation of msda_fwd.
 *   GATHER      bf16 value: the fractions, 1 - fraction, the four corner-weight products, each
 *               value * weight product and the four-corner sum rounded to bf16 (ops.py:88-91,
 *               :123, :134; the sum taken in f32).
 *   GATHER_F32  bf16 value: f32 interpolation, the sample rounded to bf16 (ops.py:137-144).
 *   MATMUL      bf16 value: the axis kernels 1 - f and f rounded to bf16, their products rounded
 *               to bf16 (ops.py:170-184), the contraction with the values in f32 and rounded to
 *               bf16 (ops.py:186).
 *   AUTO        per level, MATMUL when H * W <= 4096, else GATHER (ops.py:42, :277-279).
 *   PALLAS      pixel coordinates loc * size - 0.5 (deform_pallas.py:223-224) instead of
 *               ((2 loc - 1 + 1) size - 1) / 2 (ops.py:83-84, :270); f32 interpolation.
 * Each sample's weighted sum over levels and points is formed in f32 (ops.py:289). Returns
 * MSDA_ERR_INVALID_ARGUMENT for an unknown sampler code; otherwise as msda_fwd.
 */
int msda_fwd_sampler(const void* value, int value_dtype,
                     const float* sampling_locations, const float* attention_weights,
                     void* output, int output_dtype, int sampler,
                     int batch, int n_heads, int head_dim, int len_query,
                     int n_levels, int n_points,
                     const int32_t* spatial_shapes, const int32_t* level_start_index,
                     int64_t len_value, void* stream);

/*
 * Device workspace msda_bwd needs for this shape, in bytes, or a negative MSDA_ERR_* code: the f32
 * partial grad_value sums of the query blocks when the backward splits each (slice, level)'s
 * queries over several workgroups (n_blocks * batch * n_heads * len_value * head_dim * 4 bytes),
 * else 0. It depends on the shape, the device and the MSDA_* tuning knobs in force (read from the
 * environment once, or set by msda_set_tuning); with no knob set, on the shape and the device
 * only. The reference has no counterpart: JAX autodiff materialises its own intermediates
 * (ops.py:120-134); an XLA FFI handler asks ffi::ScratchAllocator for this many bytes.
 */
int64_t msda_bwd_workspace_size(int batch, int n_heads, int head_dim, int len_query,
                                int n_levels, int n_points,
                                const int32_t* spatial_shapes, const int32_t* level_start_index,
                                int64_t len_value);

/*
 * Backward (vector-Jacobian product of msda_fwd with cotangent grad_output):
 *   grad_value              [batch*n_heads, len_value, head_dim]  value_dtype (accumulated in f32,
 *                           rounded once; deform_pallas.py:175 casts the same way)
 *   grad_sampling_locations [batch, len_query, n_heads, n_levels, n_points, 2] f32
 *   grad_attention_weights  [batch, len_query, n_heads, n_levels*n_points]     f32
 * Replaces the JAX autodiff VJP of ops.py:64-134/289 and deform_pallas.py:157-175 (_sample_bwd).
 * Any of the three gradient pointers may be NULL to skip that gradient. grad_output has
 * grad_output_dtype (the forward's output dtype). grad_value is accumulated in LDS in f64 (a * w of
 * two f32 values is exact in f64, its product with g is rounded to f64's 53 bits); a workgroup owns
 * a (slice, level band) and writes its
 * rows once, rounded to value_dtype, or, when a level's queries are split over several
 * workgroups, writes f32 partial rows into the workspace that a second kernel adds in block order.
 * workspace must hold msda_bwd_workspace_size() bytes (16-byte aligned); it may be NULL when that
 * size is 0 or grad_value is NULL.
 * Limits (MSDA_ERR_UNSUPPORTED beyond them): levels of at most 32000 rows and columns,
 * len_query * n_heads * head_dim < 2^30 and len_query * n_heads * n_levels * n_points < 2^24, and
 * one image row of every level (its f64 accumulator, two staged value rows and a point list of at
 * least one query) within the LDS: about 158 columns at head_dim 64 and 318 at head_dim 32 in f32.
 */
int msda_bwd(const void* value, int value_dtype,
             const float* sampling_locations, const float* attention_weights,
             const void* grad_output, int grad_output_dtype,
             void* grad_value, float* grad_sampling_locations, float* grad_attention_weights,
             int batch, int n_heads, int head_dim, int len_query,
             int n_levels, int n_points,
             const int32_t* spatial_shapes, const int32_t* level_start_index,
             int64_t len_value, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * msda_bwd for the gradient of msda_fwd_sampler: the VJP of the f32 interpolation at the pixel
 * coordinates the named sampler forms (PALLAS: loc * size - 0.5, deform_pallas.py:157-175; the
 * others those of ops.py:83-84), so the floor decisions are the forward's. The bf16 rounding points
 * of GATHER, GATHER_F32 and MATMUL are forward-only: their VJP through the bf16 casts rounds the
 * cotangents and scatter-adds them in bf16 in an order XLA chooses, which no fixed-order kernel
 * reproduces; the gradients here are the f32 ones, within the bf16 tolerance of the reference's.
 * Workspace as msda_bwd_workspace_size(); arguments and results otherwise as msda_bwd.
 */
int msda_bwd_sampler(const void* value, int value_dtype,
                     const float* sampling_locations, const float* attention_weights,
                     const void* grad_output, int grad_output_dtype,
                     void* grad_value, float* grad_sampling_locations, float* grad_attention_weights,
                     int sampler,
                     int batch, int n_heads, int head_dim, int len_query,
                     int n_levels, int n_points,
                     const int32_t* spatial_shapes, const int32_t* level_start_index,
                     int64_t len_value, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * msda_bwd without a workspace argument and without any device allocation, for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The partial sums go to a file-scope device array of
 * 16 MiB that the library holds on every GPU it runs on until the process ends; a shape whose
 * msda_bwd_workspace_size() exceeds it returns MSDA_ERR_UNSUPPORTED. Every call on one GPU uses
 * that GPU's array: calls that overlap on one GPU (different streams, or threads) race. Nothing in
 * the array needs clearing (every partial element is written before it is read). Arguments and
 * results otherwise as msda_bwd.
 */
int msda_bwd_noalloc(const void* value, int value_dtype,
                     const float* sampling_locations, const float* attention_weights,
                     const void* grad_output, int grad_output_dtype,
                     void* grad_value, float* grad_sampling_locations, float* grad_attention_weights,
                     int batch, int n_heads, int head_dim, int len_query,
                     int n_levels, int n_points,
                     const int32_t* spatial_shapes, const int32_t* level_start_index,
                     int64_t len_value, void* stream);

/*
 * The MSDeformAttn prologue fused into the kernels. These entry points take what the module's
 * projections produce and form the core's inputs inside the kernels, so sampling locations and
 * attention weights never exist in memory:
 *   sampling_locations = reference_points + sampling_offsets / (W_l, H_l)        (ref_dim == 2)
 *                      = ref[..., :2] + sampling_offsets / n_points * ref[..., 2:] * 0.5
 *                                                                                 (ref_dim == 4)
 *   attention_weights  = softmax(attention_logits) over the n_levels * n_points axis, in f32.
 * Replaces the body of MSDeformAttn.__call__ from the offsets to the core call,
 * src/rfdetr_jax/models/ops.py:388-410 (locations :388-399 with precise_divide :46-62, softmax
 * :403-404, core :408-410), and its JAX autodiff VJP.
 * Layouts:
 *   reference_points  [batch, len_query, n_levels, ref_dim]                     f32 (ref_dim 2 or 4)
 *   sampling_offsets  [batch, len_query, n_heads, n_levels, n_points, 2]         f32
 *   attention_logits  [batch, len_query, n_heads, n_levels * n_points]           f32
 * Other arguments as msda_fwd; reference_points must be aligned to 4 * ref_dim bytes.
 */
int msda_fused_fwd(const void* value, int value_dtype,
                   const float* reference_points, int ref_dim,
                   const float* sampling_offsets, const float* attention_logits,
                   void* output, int output_dtype,
                   int batch, int n_heads, int head_dim, int len_query,
                   int n_levels, int n_points,
                   const int32_t* spatial_shapes, const int32_t* level_start_index,
                   int64_t len_value, void* stream);

/*
 * Workspace of msda_fused_bwd, in bytes, or a negative MSDA_ERR_* code: msda_bwd's record bins
 * plus per-head-group partial sums of the reference-point gradient (up to
 * batch * len_query * n_heads * n_levels * ref_dim floats), summed by a small second kernel.
 */
int64_t msda_fused_bwd_workspace_size(int batch, int n_heads, int head_dim, int len_query,
                                      int n_levels, int n_points, int ref_dim,
                                      const int32_t* spatial_shapes, const int32_t* level_start_index,
                                      int64_t len_value);

/*
 * Backward of msda_fused_fwd:
 *   grad_value              [batch*n_heads, len_value, head_dim]   value_dtype
 *   grad_sampling_offsets   [batch, len_query, n_heads, n_levels, n_points, 2]  f32
 *   grad_attention_logits   [batch, len_query, n_heads, n_levels*n_points]      f32
 *   grad_reference_points   [batch, len_query, n_levels, ref_dim]               f32
 * Any gradient pointer may be NULL to skip it. The workspace (16-byte aligned, at least
 * msda_fused_bwd_workspace_size() bytes) is needed when grad_value or grad_reference_points is
 * requested. Limits as msda_bwd.
 */
int msda_fused_bwd(const void* value, int value_dtype,
                   const float* reference_points, int ref_dim,
                   const float* sampling_offsets, const float* attention_logits,
                   const void* grad_output, int grad_output_dtype,
                   void* grad_value, float* grad_sampling_offsets, float* grad_attention_logits,
                   float* grad_reference_points,
                   int batch, int n_heads, int head_dim, int len_query,
                   int n_levels, int n_points,
                   const int32_t* spatial_shapes, const int32_t* level_start_index,
                   int64_t len_value, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Grid sampling of channels-first feature maps: bilinear_grid_sample and point_sample of the
 * segmentation head. Replaces
 *   bilinear_grid_sample(inputs, grid, padding_mode)   src/rfdetr_jax/models/ops.py:189-205
 *     (the sampler _sample_rows with padding_mode,    ops.py:64-134)
 *   point_sample(inputs, point_coords, mode)           src/rfdetr_jax/models/heads/segmentation.py:146-170
 *     (nearest sampling, _nearest_grid_sample,         segmentation.py:173-186)
 * and their JAX autodiff VJPs.
 * Layouts (row-major, contiguous):
 *   input        [n, channels, height, width]   dtype (MSDA_DTYPE_F32 or MSDA_DTYPE_BF16)
 *   grid         [n, n_points, 2] f32 (x, y): grid coordinates in [-1, 1] (MSDA_GRID_COORDS,
 *                bilinear_grid_sample; n_points = Hg * Wg) or point_sample's points in [0, 1]
 *                (MSDA_GRID_UNIT_POINTS; the kernel forms grid = 2 p - 1, segmentation.py:166)
 *   output       [n, channels, n_points]        dtype
 * Semantics: torch grid_sample(align_corners=False) as ops.py:64-134 writes it; zero padding masks
 * out-of-bounds corners, border padding clips them (the unmasked weights replicate the edge);
 * nearest sampling rounds half to even and clips, with border padding only.
 */
enum msda_grid_kind { MSDA_GRID_COORDS = 0, MSDA_GRID_UNIT_POINTS = 1 };
enum msda_padding { MSDA_PADDING_ZEROS = 0, MSDA_PADDING_BORDER = 1 };
enum msda_sample_mode { MSDA_SAMPLE_BILINEAR = 0, MSDA_SAMPLE_NEAREST = 1 };

int msda_grid_sample_fwd(const void* input, int dtype, const float* grid, int grid_kind,
                         void* output, int n, int channels, int height, int width, int n_points,
                         int padding_mode, int sample_mode, void* stream);

/*
 * Backward of msda_grid_sample_fwd for cotangent grad_output [n, channels, n_points] (dtype):
 *   grad_input [n, channels, height, width] dtype (accumulated in f32, fully written: no
 *              zero-fill needed), and grad_grid [n, n_points, 2] f32 (the gradient of the grid
 *              coordinates or of the unit points, per grid_kind; zero for nearest sampling).
 * Either output may be NULL. Widths above 16384 are MSDA_ERR_UNSUPPORTED for grad_input.
 */
int msda_grid_sample_bwd(const void* input, int dtype, const float* grid, int grid_kind,
                         const void* grad_output, void* grad_input, float* grad_grid,
                         int n, int channels, int height, int width, int n_points,
                         int padding_mode, int sample_mode, void* stream);

/*
 * MSDeformAttn's value projection with its epilogue fused in: one MFMA product writes
 *   value[(b * n_heads + h) * len_in + s][d] = padded[b, s] ? 0 : (input[b, s, :] . W[h * head_dim + d, :] + bias[h * head_dim + d])
 * Replaces value_proj (Linear, src/rfdetr_jax/models/layers.py:258-280: x @ W^T + b in the input
 * dtype), the padding mask (ops.py:377-379) and the head split (ops.py:405-407) of
 * MSDeformAttn.__call__, so the [B, S, C] projection and its transpose never exist in memory.
 * Layouts:
 *   input         [batch, len_in, in_features]           dtype (MSDA_DTYPE_F32 or MSDA_DTYPE_BF16)
 *   weight        [n_heads * head_dim, in_features] f32  (torch Linear layout; rounded to bf16 when
 *                                                        the input is bf16, as weight.astype(x.dtype))
 *   bias          [n_heads * head_dim] f32 or NULL
 *   padding_mask  [batch, len_in] uint8 (non-zero = padded) or NULL
 *   value         [batch * n_heads, len_in, head_dim]    dtype (the core's value layout)
 */
int msda_value_proj_fwd(const void* input, int dtype, const float* weight, const float* bias,
                        const uint8_t* padding_mask, void* value,
                        int batch, int len_in, int in_features, int n_heads, int head_dim, void* stream);

/* Workspace of msda_value_proj_bwd in bytes (a function of the shape only), or a negative code. */
int64_t msda_value_proj_bwd_workspace_size(int batch, int len_in, int in_features, int n_heads, int head_dim);

/*
 * Backward of msda_value_proj_fwd for cotangent grad_value [batch * n_heads, len_in, head_dim]:
 *   grad_input  [batch, len_in, in_features] dtype, grad_weight [n_heads * head_dim, in_features]
 *   f32, grad_bias [n_heads * head_dim] f32; padded rows contribute nothing. Any of the three may be
 * NULL. The workspace (16-byte aligned) holds grad_weight's split partial sums and is needed when
 * grad_weight or grad_bias is requested; they are added in a fixed order (deterministic).
 */
int msda_value_proj_bwd(const void* input, int dtype, const float* weight, const uint8_t* padding_mask,
                        const void* grad_value, void* grad_input, float* grad_weight, float* grad_bias,
                        int batch, int len_in, int in_features, int n_heads, int head_dim,
                        void* workspace, int64_t workspace_bytes, void* stream);

/* ---- Decoder self-attention -----------------------------------------------------------------
 * scaled_dot_product_attention (src/rfdetr_jax/models/layers.py:54-99, the XLA path) as used by
 * MultiheadAttention (layers.py:491-548) in the decoder's grouped self-attention
 * (src/rfdetr_jax/models/transformer.py:200-210): per slice z and head h,
 *   out = softmax(q k^T / sqrt(D), blocked positions -> finfo(float32).min) v
 * over len queries and len keys of head_dim = D channels (32 or 64). The slices are
 * z = g * batch + b for b < batch, g < groups, the order of _split_groups (transformer.py:350-354):
 * with groups > 1 the caller passes the unsplit [batch, groups * len, C] rows and the kernels read
 * group g of image b in place. Every tensor is addressed as
 *   base + b * s_b + g * s_g + h * s_h + row * s_row + channel
 * with the four element strides given per tensor in `strides` (in that order; each a multiple of 4,
 * base pointers aligned to 4 elements). Examples: [Z, H, L, D] contiguous (the reference
 * function's layout): (H L D, 0, L D, D) with groups = 1; the decoder's [B, G P, C] rows with
 * C = H D: (G P C, P C, D, C).
 *
 * mask: [len, len] bytes (non-zero blocks a key for a query: torch's boolean convention,
 * layers.py:69, :93-94) or NULL. dtype: MSDA_DTYPE_F32 or MSDA_DTYPE_BF16 for every tensor;
 * arithmetic is f32 (v_mfma_f32_32x32x2_f32), softmax in f32.
 * stats: [batch * groups * heads * len][4] f32, 16-byte aligned, z-major (z = g * batch + b), then
 * head, then query: the forward writes entries 0 and 1 (a reference score m, between 8 below and
 * 64 above the row maximum, and log2 of the softmax denominator taken relative to m, in units of
 * log2(e) q.k / sqrt(D)); the backward reads them and uses entry 2 for rowsum(grad_out * out).
 * Dropout on the attention weights (layers.py:537-544, active only with dropout > 0 in training)
 * is msda_attention_fwd_dropout's. len is at most 65536, each row stride s_row below 2^24 elements
 * and len * s_row below 2^31 (row offsets within a (slice, head) are formed in 32 bits).
 */
int msda_attention_fwd(const void* q, const void* k, const void* v, int dtype, void* out, float* stats,
                       int batch, int groups, int heads, int len, int head_dim,
                       const int64_t* strides /* [4 tensors: q, k, v, out][4] */, const uint8_t* mask, void* stream);

/*
 * Backward of msda_attention_fwd for the cotangent grad_out: grad_q, grad_k, grad_v (each may be
 * NULL to skip it; same layouts and dtype rules). out and stats are the forward's (stats entry 2
 * is overwritten). With head_dim 32, no mask, len <= 320 and grad_q plus grad_k or grad_v
 * requested, one kernel forms all gradients (the tuning knob MSDA_ATTN_FUSED=0 selects the
 * two-kernel path instead; the two agree within f32 summation order).
 * strides: [8 tensors: q, k, v, out, grad_out, grad_q, grad_k, grad_v][4].
 */
int msda_attention_bwd(const void* q, const void* k, const void* v, const void* out, float* stats,
                       const void* grad_out, int dtype, void* grad_q, void* grad_k, void* grad_v,
                       int batch, int groups, int heads, int len, int head_dim,
                       const int64_t* strides, const uint8_t* mask, void* stream);

/*
 * msda_attention_fwd with dropout on the softmax weights, as MultiheadAttention applies it in
 * training (layers.py:537-544: weights = nn.Dropout(rate)(softmax(scores)), then weights @ v):
 *   out = (softmax(...) * keep / (1 - rate)) v.
 * keep(z, h, q, k) is a function of (seed, z * heads + h, q, k) alone: each kernel that needs it
 * regenerates it, so the backward of the same call (same seed and rate) drops the same weights and
 * nothing is stored. A weight is kept with probability 1 - round(rate * 65536) / 65536. The
 * reference draws its mask from JAX's threefry stream (flax nn.Dropout): the distribution is the
 * same, the particular mask is not. rate in [0, 1) (MSDA_ERR_INVALID_ARGUMENT otherwise); rate 0
 * computes what msda_attention_fwd computes. stats as msda_attention_fwd's (the softmax of every
 * weight, before dropout). Dropout runs in the chunked kernels (neither the staged bf16 forward nor
 * the fused backward).
 * No counterpart in the reference's C interface (its dropout is a JAX op around the product); for
 * callers that train with attention dropout.
 */
int msda_attention_fwd_dropout(const void* q, const void* k, const void* v, int dtype, void* out, float* stats,
                               int batch, int groups, int heads, int len, int head_dim,
                               const int64_t* strides, const uint8_t* mask, float rate, uint64_t seed, void* stream);

/*
 * Backward of msda_attention_fwd_dropout (same rate and seed as the forward call):
 *   dV = (P * keep / (1 - rate))^T dO,  dP = (dO V^T) * keep / (1 - rate),
 *   dS = P (dP - rowsum(dO * out)),     dQ = dS K / sqrt(D),  dK = dS^T Q / sqrt(D).
 * Arguments otherwise as msda_attention_bwd (always the two-kernel path).
 */
int msda_attention_bwd_dropout(const void* q, const void* k, const void* v, const void* out, float* stats,
                               const void* grad_out, int dtype, void* grad_q, void* grad_k, void* grad_v,
                               int batch, int groups, int heads, int len, int head_dim,
                               const int64_t* strides, const uint8_t* mask, float rate, uint64_t seed, void* stream);

/*
 * The keep decisions of msda_attention_fwd_dropout for (rate, seed): keep[z * heads + h][q][k] = 1
 * where weight (q, k) is kept, else 0 ([batch * groups * heads][len][len] bytes, z = g * batch + b).
 * For tests and for callers that need the mask itself; no counterpart in the reference.
 */
int msda_attention_dropout_keep(int batch, int groups, int heads, int len, float rate, uint64_t seed,
                                uint8_t* keep, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSDA_H_ */
