/*
 * akas_fp8.h -- C ABI of the MI355X (gfx950) block-scaled FP8 matrix-product
 * path: FP8 activation quantizer, 128x128 block-scaled linear, expert routing,
 * permutation, tile maps and packing, grouped expert GEMMs (gate_up with fused
 * SwiGLU re-quantization, down) and the weighted top-k combine.
 *
 * One entry point per operator kind of the reference's graph API.  Each
 * comment cites the reference interface it replaces (paths relative to the
 * reference repository root).
 *
 * Conventions (all entry points):
 *   - every pointer is a device pointer on the current HIP device, except
 *     where noted; dims are passed by value;
 *   - `stream` is a hipStream_t (0 = the legacy default stream);
 *   - calls are asynchronous and stream-ordered: no allocation, no host
 *     synchronization and no host reads of device data happen inside a call,
 *     so every call can be captured in a HIP graph;
 *   - geometry, null pointers and dtype codes are validated on the host before
 *     any launch; the return value is AKAS_OK or a negative AKAS_ERR_* code;
 *   - distinct streams may call concurrently; calls sharing a workspace must
 *     be stream-ordered.
 *
 * Layouts (row-major, last index fastest):
 *   activation codes  u8  [rows, k]         scales f32 [rows, k/128]
 *   weight codes      u8  [(E,) n, k]       scales f32|bf16 [(E,) ceil(n/128), k/128]
 *   routes            i32 [E, r]  value row*top + rank, padding -1
 *   tile maps         i32 [layouts, (r*top+3)/4 + E]
 */
#ifndef AKAS_FP8_H
#define AKAS_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The library is built with hidden visibility; only these entry points are
   exported. */
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* element dtype codes */
#define AKAS_DTYPE_F32 0
#define AKAS_DTYPE_F16 1
#define AKAS_DTYPE_BF16 2

/* status codes */
#define AKAS_OK 0
#define AKAS_ERR_GEOMETRY -1 /* invalid shape / tile geometry (reference ValueError) */
#define AKAS_ERR_NULL -2     /* required pointer is null */
#define AKAS_ERR_DTYPE -3    /* unsupported dtype code */
#define AKAS_ERR_LAUNCH -4   /* HIP launch failed */
#define AKAS_ERR_WORKSPACE -5 /* workspace missing or too small */
#define AKAS_ERR_SCRATCH -6   /* problem larger than the library's static scratch */

/* Bytes of the static device scratch of akas_fp8_linear_noalloc (per GPU). */
#define AKAS_NOALLOC_SCRATCH_BYTES (64u << 20)

/* Library version (major*10000 + minor*100 + patch). */
int akas_version(void);

/* Static text for a status code. */
const char* akas_status_string(int status);

/* Number of entry points declared in this header and exported by the library. */
int akas_abi_count(void);

/* ------------------------------------------------------------------------ */
/* FP8 activation quantizer                                                  */
/* ------------------------------------------------------------------------ */

/*
 * quantize(r, k[, top, input_dtype]): x -> out, scales.
 * Replaces src/akas/quantization/activations/fp8/cuda.py:10-56 (kind
 * "quantize", OutputABI (1, 2) at definition.py:43-48).
 * rows = r * (top or 1); x is f32/f16/bf16 [rows, k]; k % 128 == 0.
 * scales[g] = max(max|x_g|, 1e-12) / 448; out = e4m3(x / scale), bit-exact.
 */
int akas_quantize(const void* x, int x_dtype, uint8_t* out, float* scales,
                  int64_t rows, int64_t k, void* stream);

/*
 * rms_quantize: x, w -> [y,] codes, scales.  RMSNorm fused with the
 * activation quantizer.  It has no single reference counterpart: it fuses
 * the reference's kind "rms" (src/akas/ops/normalization/definition.py:10-31,
 * equation normalization/validation.py:31-52) with the kind "quantize" that
 * consumes its output (activations/fp8/cuda.py:10-56).
 *   y = round_y(x * (1 / sqrt(sum(x^2)/cols + eps)) * w'), w' = w (or 1 + w
 *   when zero_centered); y [rows, cols] in y_dtype is written when y != NULL;
 *   codes [rows, cols] / scales [rows, cols/128] are quantize(y) of exactly
 *   those rounded values, bit for bit.
 * x f32/f16/bf16, w f32/bf16 [cols]; cols % 128 == 0 and cols <= 8192; eps
 * finite and >= 0; x, w, y 16-byte aligned, codes 8-byte aligned (else
 * AKAS_ERR_GEOMETRY).
 */
int akas_rms_quantize(const void* x, int x_dtype, const void* w, int w_dtype, float eps,
                      int zero_centered, void* y, int y_dtype, uint8_t* codes, float* scales,
                      int64_t rows, int64_t cols, void* stream);

/*
 * dequantize_fp8: codes, scales -> out (f32/f16/bf16) = decode(code) * scale.
 * Replaces src/akas/quantization/activations/fp8/kernel.py dequantize
 * (kind "dequantize_fp8", definition.py:43-46, 61-70).
 */
int akas_dequantize_fp8(const uint8_t* codes, const float* scales, void* out, int out_dtype,
                        int64_t rows, int64_t k, void* stream);

/*
 * Block-quantize f32 weights [batch, n, k] to e4m3 codes and 128x128 block
 * scales max(max|block|, 1e-12)/448 (rounded to bf16 first when
 * scale_dtype == AKAS_DTYPE_BF16).  Device equivalent of the host weight
 * preparation src/akas/quantization/weights/fp8/kernel.py:34-59 with the
 * storage layout of weights/fp8/definition.py:12-27.
 */
int akas_quantize_weight_blocks(const float* w, uint8_t* codes, void* scales, int scale_dtype,
                                int64_t batch, int64_t n, int64_t k, void* stream);

/* ------------------------------------------------------------------------ */
/* Dense block-scaled FP8 linear                                             */
/* ------------------------------------------------------------------------ */

/*
 * Workspace bytes needed by akas_fp8_linear for (r, k, o): activation codes
 * and scales (plus split-K partials for small-r launches).  Host-only.
 */
size_t akas_fp8_linear_workspace_size(int64_t r, int64_t k, int64_t o);

/*
 * fp8_linear(r, k, o[, input_dtype]): x, w, scales -> out.
 * Replaces src/akas/ops/linear/cuda.py:642-646 (fp8_inline, _mma with inline
 * quantization :102-501) and the r<=8 GEMV native_fp8 (:757-828); kind
 * registered at src/akas/ops/linear/definition.py:1890-1914.
 * x f32/f16/bf16 [r, k]; w u8 [o, k]; w_scales f32|bf16 [ceil(o/128), k/128];
 * out f32/f16/bf16 [r, o] = quantize(x) . dequant(w)^T, f32 accumulation.
 * k % 128 == 0 and o % 16 == 0.  The workspace (at least
 * akas_fp8_linear_workspace_size(r, k, o) bytes) needs no initialization:
 * its prior contents never reach the output.  Calls that share a workspace
 * must be ordered on one stream.
 */
int akas_fp8_linear(const void* x, int x_dtype, const uint8_t* w, const void* w_scales,
                    int scale_dtype, void* out, int out_dtype, void* workspace,
                    size_t workspace_bytes, int64_t r, int64_t k, int64_t o, void* stream);

/*
 * fp8_linear without allocation and without a workspace argument.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * akas_fp8_linear (bit for bit); the workspace is a static device array of
 * AKAS_NOALLOC_SCRATCH_BYTES held by every GPU the library runs on until the
 * process ends.  Returns AKAS_ERR_SCRATCH when
 * akas_fp8_linear_workspace_size(r, k, o) exceeds it.  The call never calls
 * hipMalloc or hipFree.  All calls on one GPU share its array: calls that
 * overlap in time on one GPU (two streams, or two host threads) race;
 * calls ordered on one stream do not.
 */
int akas_fp8_linear_noalloc(const void* x, int x_dtype, const uint8_t* w, const void* w_scales,
                            int scale_dtype, void* out, int out_dtype, int64_t r, int64_t k,
                            int64_t o, void* stream);

/*
 * projection_partial(r, k, o, partitions): prequantized x, w, scales,
 * activation_scales -> out.
 * Replaces src/akas/ops/linear/cuda.py:649-653 (fp8_prequantized) and
 * :452-483; kind at src/akas/ops/linear/definition.py:1304-1321.
 * partitions == 1: out [r, o] in out_dtype.  partitions > 1: out f32
 * [r, partitions, o] with partition p summing k-blocks
 * [p*k/(128*partitions), (p+1)*k/(128*partitions)).
 */
int akas_projection_partial(const uint8_t* x, const float* activation_scales, const uint8_t* w,
                            const void* w_scales, int scale_dtype, void* out, int out_dtype,
                            int64_t r, int64_t k, int64_t o, int partitions, void* stream);

/*
 * projection_merge(r, o, partitions) / expert_merge(r, top, o, partitions):
 * partial f32 [rows, partitions, o] -> out [rows, o] (serial f32 sum).
 * Replaces src/akas/ops/linear/cuda.py:1369-1402 (kinds projection_merge,
 * src/akas/ops/linear/definition.py:1322-1328, and expert_merge,
 * src/akas/ops/moe/definition.py:2409-2420).  rows = r * (top or 1).
 */
int akas_projection_merge(const float* partial, void* out, int out_dtype, int64_t rows, int64_t o,
                          int partitions, void* stream);

/* ------------------------------------------------------------------------ */
/* Routing                                                                   */
/* ------------------------------------------------------------------------ */

/*
 * biased_router(r, experts, top, scale, normalize): logits, bias -> ids, weights.
 * Replaces src/akas/ops/moe/kernel.py:154-203 (kind at
 * src/akas/ops/moe/definition.py:1946-1971).  Selects on
 * sigmoid(l) + b (ties -> lowest index); weights = sigmoid(l_sel) * scale /
 * (sum + 1e-6) when normalize, else sigmoid(l_sel) * scale.
 * experts <= 1024, top <= experts.
 */
int akas_biased_router(const float* logits, const float* bias, int32_t* ids, float* weights,
                       int64_t r, int experts, int top, float scale, int normalize, void* stream);

/*
 * biased_softmax_router(r, experts, top, scale): logits, bias -> ids, weights.
 * Replaces src/akas/ops/moe/kernel.py:444-499 (definition.py:2475-2490).
 * Selects on logits + bias (ties -> lowest index); weights = scale *
 * softmax over the selected unbiased logits.
 */
int akas_biased_softmax_router(const float* logits, const float* bias, int32_t* ids,
                               float* weights, int64_t r, int experts, int top, float scale,
                               void* stream);

/*
 * router(r, experts, top): logits -> ids, weights (the block-fp8 decode
 * variant's router kind).
 * Replaces src/akas/ops/moe/cuda.py:2011-2050 (registered as "router" at
 * src/akas/ops/moe/definition.py:1651-1657, :1836-1842).  The f32 logits are
 * rounded to bf16 before selection (ties -> lowest index); weights = softmax
 * over the selected rounded logits, relative to the first (largest) one.
 */
int akas_router(const float* logits, int32_t* ids, float* weights, int64_t r, int experts,
                int top, void* stream);

/*
 * The MoE block's router and its activation quantizer in one launch, for
 * blocks whose router takes the 16-lanes-per-row form (experts <= 64,
 * top <= 8).  No counterpart in the reference: it fuses two of its kinds,
 * biased_router / biased_softmax_router (softmax != 0) over logits and bias
 * (src/akas/ops/moe/kernel.py:154-203, :444-499) and quantize over x [r, k]
 * (src/akas/quantization/activations/fp8/cuda.py:10-56), which share no
 * data.  ids, weights, codes and scales are bit-identical to the two
 * separate entry points' outputs.
 */
int akas_router_quantize(const float* logits, const float* bias, int32_t* ids, float* weights,
                         int64_t r, int experts, int top, float scale, int softmax, int normalize,
                         const void* x, int x_dtype, uint8_t* codes, float* scales, int64_t k,
                         void* stream);

/*
 * moe_groups(r, top): ids -> experts, routes (the block-fp8 decode variant's
 * route tables).  Replaces src/akas/ops/moe/cuda.py:1978-2008.  For each
 * (row, rank) group g of ids [r, top]: experts[g] = ids[g] when no earlier
 * group (in row, rank order) holds that expert, else -1; routes [r*top, r]:
 * for an owning group, routes[g, b] = the last rank at which row b selected
 * the expert, or -1; all -1 for other groups.  Bit-exact.
 */
int akas_moe_groups(const int32_t* ids, int32_t* experts, int32_t* routes, int64_t r, int top,
                    void* stream);

/*
 * quantized_routes(r, experts, top): ids, active -> counts, routes.
 * Replaces src/akas/ops/moe/kernel.py:121-151 and the parallel variant
 * src/akas/ops/moe/cuda.py:2187-2322.  Stable (row, rank) order, bit-exact;
 * routes [experts, r] padded with -1.  Requires each row's ids to hold an
 * expert at most once (true of top-k ids), so counts[e] <= r.
 */
int akas_quantized_routes(const int32_t* ids, const int32_t* active, int32_t* counts,
                          int32_t* routes, int64_t r, int experts, int top, void* stream);

/*
 * expert_tile_map(r, experts, top[, max_block_m]): counts -> tile_experts, tile_rows.
 * Replaces src/akas/ops/moe/kernel.py:79-118 (parallel cuda.py:2095-2175).
 * Shape [layouts, (r*top+3)/4 + experts] with layouts = log2(max_block_m) - 1
 * (row tiles 4, 8, ..., max_block_m); padding (-1, 0).
 */
int akas_expert_tile_map(const int32_t* counts, int32_t* tile_experts, int32_t* tile_rows,
                         int64_t r, int experts, int top, int max_block_m, void* stream);

/*
 * expert_pack(r, top, experts, k, max_block_m[, routed_input]):
 * x, activation_scales, counts, routes, tile_experts, tile_offsets ->
 * packed, packed_scales, expert_offsets.
 * Replaces src/akas/ops/moe/cuda.py:2423-2502 (kind at
 * src/akas/ops/moe/definition.py:2491-2501).  packed [cap*A, k] with
 * cap = tile_capacity(r, top, experts, A), A = max_block_m; padding codes 0,
 * scales 1; expert_offsets written for non-empty experts only.
 */
int akas_expert_pack(const uint8_t* x, const float* activation_scales, const int32_t* counts,
                     const int32_t* routes, const int32_t* tile_experts,
                     const int32_t* tile_offsets, uint8_t* packed, float* packed_scales,
                     int32_t* expert_offsets, int64_t r, int top, int experts, int64_t k,
                     int max_block_m, int routed_input, void* stream);

/* ------------------------------------------------------------------------ */
/* Grouped expert GEMMs                                                      */
/* ------------------------------------------------------------------------ */

/*
 * expert_partial(r, top, experts, o, k, routed_input, partitions, tile_map
 * [, max_block_m, output_dtype, packed_input]):
 * x, activation_scales, w, scales, counts, routes, tile_experts, tile_offsets
 * [, expert_offsets] -> out.
 * Replaces src/akas/ops/moe/cuda.py:541-1354 (_bucketed, mapped registration
 * src/akas/ops/moe/definition.py:2326-2366).
 *   x: codes [r, k] (or [r, top, k] if routed_input; or packed [cap*A, k]
 *      when packed_input) with 1x128 activation scales;
 *   w: [experts, o, k] codes, scales [experts, ceil(o/128), k/128];
 *   out: [r, top, o] in out_dtype (partitions == 1) or f32
 *        [r, top, partitions, o]; only routed (row, rank) entries are written.
 * The tile map is validated for shape; work items are derived on the device
 * from counts (identical to the map's layout by construction).
 * o % 128 == 0, k % 128 == 0.
 */
int akas_expert_partial(const uint8_t* x, const float* activation_scales, const uint8_t* w,
                        const void* w_scales, int scale_dtype, const int32_t* counts,
                        const int32_t* routes, const int32_t* tile_experts,
                        const int32_t* tile_offsets, const int32_t* expert_offsets, void* out,
                        int out_dtype, int64_t r, int top, int experts, int64_t o, int64_t k,
                        int routed_input, int partitions, int max_block_m, int packed_input,
                        void* stream);

/*
 * expert_combine(r, top, experts, o, k, routed_input[, max_block_m,
 * contribution_dtype, packed_input]): x, activation_scales, w, scales,
 * counts, routes[, expert_offsets], ids, weights[, active] -> contributions,
 * out.
 * The down projection with routed_combine folded into its epilogue: the
 * expert_partial product scattered to (row, rank) (src/akas/ops/moe/
 * cuda.py:541-1354, the scatter at :956-966) followed by routed_combine
 * (src/akas/ops/moe/kernel.py:206-267) in one launch, bit-identical to
 * expert_partial(partitions = 1, contribution_dtype) -> routed_combine.
 *   contributions: [r, top, o] in contribution_dtype (f32/f16/bf16), written
 *     for every routed (row, rank) as expert_partial writes them;
 *   out: f32 [r, o]; out[b, c] = fma-fold over the live ranks of row b in
 *     rank order of contributions[b, rank, c] * weights[b, rank] (starting
 *     from 0); rows with active == 0 (active may be null: every row active)
 *     or with no live rank are zero.  A rank is live when
 *     0 <= ids[b, rank] < experts -- exactly the ranks quantized_routes
 *     routes, so counts/routes must be quantized_routes(ids, active).
 *   arrivals: int32 [r, o / 128]; zero before the first call, and every call
 *     leaves it zero.  Calls that share one arrivals buffer must not
 *     overlap (use one buffer per stream).
 * contributions and out 16-byte aligned; o % 128 == 0, k % 128 == 0.
 * The workgroup whose stored tile completes a row's live ranks for a column
 * block folds that row's block; no workgroup waits for another.
 */
int akas_expert_combine(const uint8_t* x, const float* activation_scales, const uint8_t* w,
                        const void* w_scales, int scale_dtype, const int32_t* counts,
                        const int32_t* routes, const int32_t* expert_offsets, const int32_t* ids,
                        const float* weights, const int32_t* active, void* contributions,
                        int contribution_dtype, float* out, int32_t* arrivals, int64_t r,
                        int top, int experts, int64_t o, int64_t k, int routed_input,
                        int max_block_m, int packed_input, void* stream);

/*
 * fp8_experts(r, experts, top, o, k, routed_input): x, w, scales, experts,
 * routes -> out (the block-fp8 decode variant's expert products).
 * Replaces src/akas/ops/moe/cuda.py:439-531.  x f32/f16/bf16 [r, k] (or
 * [r, top, k] when routed_input) is quantized per 1x128 group; for every
 * group g with experts[g] = e >= 0 and row b with rank = routes[g, b] >= 0,
 * out[b, rank, :] = x_row . dequant(w[e])^T with x_row = x[b] (x[b, rank]
 * when routed), f32 accumulation; other entries of out are left untouched.
 * The group tables are moe_groups'.  o % 128 == 0 and k % 128 == 0; the
 * caller's workspace holds at least akas_fp8_experts_workspace_size() bytes.
 */
size_t akas_fp8_experts_workspace_size(int64_t r, int top, int experts, int64_t k,
                                       int routed_input);
int akas_fp8_experts(const void* x, int x_dtype, const uint8_t* w, const void* w_scales,
                     int scale_dtype, const int32_t* group_experts, const int32_t* group_routes,
                     void* out, int out_dtype, void* workspace, size_t workspace_bytes, int64_t r,
                     int top, int experts, int64_t o, int64_t k, int routed_input, void* stream);

/*
 * fp8_expert_swiglu(r, top, experts, o, k[, product_dtype, activation_dtype,
 * max_block_m, packed_input, packed_output]):
 * x, activation_scales, w, scales, w2, scales2, counts, routes, tile_experts,
 * tile_offsets[, expert_offsets] -> out, output_scales.
 * Replaces the paired _bucketed epilogue src/akas/ops/moe/cuda.py:823-946
 * (kind at src/akas/ops/moe/definition.py:2367-2406, 1861-1863).
 * g = x.w^T, u = x.w2^T (f32), rounded to product_dtype; a = silu(g)*u
 * rounded to activation_dtype; per 128 columns s = max(max|a|,1e-12)/448 and
 * out = e4m3(a/s).  out u8 [r, top, o] (or packed [cap*A, o]), output_scales
 * f32 [r, top, o/128] (or [cap*A, o/128]).  Bit-identical to expert_partial
 * x2 -> swiglu_experts -> quantize with the same dtypes.
 */
int akas_fp8_expert_swiglu(const uint8_t* x, const float* activation_scales, const uint8_t* w,
                           const void* w_scales, const uint8_t* w2, const void* w2_scales,
                           int scale_dtype, const int32_t* counts, const int32_t* routes,
                           const int32_t* tile_experts, const int32_t* tile_offsets,
                           const int32_t* expert_offsets, uint8_t* out, float* output_scales,
                           int64_t r, int top, int experts, int64_t o, int64_t k,
                           int product_dtype, int activation_dtype, int max_block_m,
                           int packed_input, int packed_output, void* stream);

/*
 * quantized_routes followed by fp8_expert_swiglu (unpacked rows) in one
 * launch: ids, active, x, activation_scales, w, scales, w2, scales2 ->
 * counts, routes, out, output_scales.  No counterpart in the reference, which
 * runs the two kinds one after the other (src/akas/ops/moe/kernel.py:121-151,
 * src/akas/ops/moe/cuda.py:823-946); for callers that run both on a decode
 * batch.  counts [experts] and routes [experts, r] are bit-identical to
 * akas_quantized_routes' (the down projection and the combine read them),
 * out u8 [r, top, o] and output_scales f32 [r, top, o/128] to
 * akas_fp8_expert_swiglu's over those tables.  active [r] may be null
 * (every row active).  One launch when experts <= 512, top <= 64, 1 <= r*top <= 4096 and
 * r*top / experts <= 48 (every workgroup scans ids itself); otherwise the two
 * kinds' launches.
 */
int akas_routed_fp8_expert_swiglu(const int32_t* ids, const int32_t* active, int32_t* counts,
                                  int32_t* routes, const uint8_t* x,
                                  const float* activation_scales, const uint8_t* w,
                                  const void* w_scales, const uint8_t* w2, const void* w2_scales,
                                  int scale_dtype, uint8_t* out, float* output_scales, int64_t r,
                                  int top, int experts, int64_t o, int64_t k, int product_dtype,
                                  int activation_dtype, void* stream);

/*
 * expert_swiglu(r, top, experts, o, k[, product_dtype, activation_dtype,
 * output_dtype, max_block_m, packed_input, packed_output]), the FP8 paired
 * form: x, activation_scales, w, scales, w2, scales2, counts, routes,
 * tile_experts, tile_offsets[, expert_offsets] -> out.
 * Replaces src/akas/ops/moe/cuda.py:1531-1534 (fp8_paired_swiglu, kind
 * registered at src/akas/ops/moe/definition.py:2138-2188, OutputABI (-1,)).
 * fp8_expert_swiglu without the re-quantization: g, u rounded to
 * product_dtype, a = silu(g)*u rounded to activation_dtype, stored in
 * out_dtype: out [r, top, o] (or packed [cap*A, o]).  Bit-identical to
 * expert_partial x2 -> swiglu_experts with the same dtypes.
 */
int akas_expert_swiglu(const uint8_t* x, const float* activation_scales, const uint8_t* w,
                       const void* w_scales, const uint8_t* w2, const void* w2_scales,
                       int scale_dtype, const int32_t* counts, const int32_t* routes,
                       const int32_t* tile_experts, const int32_t* tile_offsets,
                       const int32_t* expert_offsets, void* out, int out_dtype, int64_t r, int top,
                       int experts, int64_t o, int64_t k, int product_dtype,
                       int activation_dtype, int max_block_m, int packed_input, int packed_output,
                       void* stream);

/*
 * expert_pair_partial(r, top, experts, o, k, partitions[, max_block_m]):
 * x, activation_scales, w, scales, w2, scales2, counts, routes, tile_experts,
 * tile_offsets -> gate, up.
 * Replaces src/akas/ops/moe/cuda.py:1537-1542 (paired_partial, kind
 * registered at src/akas/ops/moe/definition.py:2423-2462, OutputABI (-2, -1)
 * ("gate", "up")); the partitions policy of fp8_expert_swiglu
 * (definition.py:796-948) feeds its outputs to swiglu_experts.
 * gate, up f32 [r, top, partitions, o]: the expert_partial products of w and
 * of w2 over k-partition p (k-blocks [p*k/(128*partitions), ...)), each
 * bit-identical to expert_partial on that weight; only routed entries are
 * written.  x codes [r, k] (not routed), o % 128 == 0,
 * (k / 128) % partitions == 0.
 */
int akas_expert_pair_partial(const uint8_t* x, const float* activation_scales, const uint8_t* w,
                             const void* w_scales, const uint8_t* w2, const void* w2_scales,
                             int scale_dtype, const int32_t* counts, const int32_t* routes,
                             const int32_t* tile_experts, const int32_t* tile_offsets,
                             float* gate, float* up, int64_t r, int top, int experts, int64_t o,
                             int64_t k, int partitions, int max_block_m, void* stream);

/*
 * swiglu_experts(r, top, c, expert_rows, input_dtype, output_dtype
 * [, round_inputs, round_dtype, partitions]): g, u -> out.
 * Replaces src/akas/ops/activation/kernel.py:28-88.  g, u
 * [r, top, (partitions,) c] in input_dtype; partitions are summed in f32
 * first; round_inputs rounds g and u to round_dtype; out [r, top, c] =
 * g / (1 + exp(-g)) * u stored in output_dtype.
 */
int akas_swiglu_experts(const void* g, const void* u, int input_dtype, void* out,
                        int output_dtype, int64_t r, int top, int64_t c, int partitions,
                        int round_inputs, int round_dtype, void* stream);

/*
 * moe_combine(r, top, c): experts, weights, shared, gate -> out.
 * Replaces src/akas/ops/moe/cuda.py:392-422 (decode_moe_combine, the
 * Qwen3.5 block-fp8 MoE combine with a sigmoid-gated shared expert; test
 * equation moe/validation.py:506-515):
 *   out[b, col] = sum_rank bf16(experts[b, rank, col]) * weights[b, rank]
 *                 + bf16(shared[b, col]) / (1 + exp(-bf16(gate[b])))
 * in f32, ranks in order.  experts [r, top, c], shared [r, c], gate [r]
 * (f32/f16/bf16 each), weights f32 [r, top], out f32 [r, c]; c % 8 == 0;
 * experts and out 16-byte aligned.
 */
int akas_moe_combine(const void* experts, int input_dtype, const float* weights,
                     const void* shared, int shared_dtype, const void* gate, int gate_dtype,
                     float* out, int64_t r, int top, int64_t c, void* stream);

/*
 * routed_combine(r, top, c[, input_dtype]): experts, weights, active -> out.
 * Replaces src/akas/ops/moe/kernel.py:206-267.  out f32 [r, c] =
 * sum over rank (serial order) of experts[r, rank, c] * weights[r, rank];
 * rows with active == 0 are zero.
 */
int akas_routed_combine(const void* experts, int input_dtype, const float* weights,
                        const int32_t* active, float* out, int64_t r, int top, int64_t c,
                        void* stream);

/*
 * The shared-expert MoE block (Qwen3.5 block-fp8) in one call:
 * x f32/f16/bf16 [r, h], router logits f32 [r, experts] and the shared
 * expert's gate logit shared_gate f32/f16/bf16 [r] -> out f32 [r, h].
 * No counterpart in the reference, whose program composes the block from
 * kinds (src/akas/ops/moe/definition.py:293-418): decode_router
 * (cuda.py:2011-2050), quantize, the routed experts' gate/up, SwiGLU, FP8
 * re-quantization and down products (f32 products and activations), the
 * shared expert's FP8 gate/up -> SwiGLU -> FP8 down as dense linears, and
 * moe_combine (cuda.py:392-422).  For callers that run the whole block: the
 * shared expert (sw1/sw3 [f, h], sw2 [h, f], scales as the bank's) is
 * computed as expert `experts` of the routed launches, at rank top of every
 * row, the router shares a launch with the quantizer of x and, for decode
 * batches, the route scan runs inside the gate/up launch: four launches and
 * no dense launches beside them.
 * Bank w1/w3 [experts, f, h], w2 [experts, h, f], 128x128 block scales of
 * scale_dtype (f32 or bf16) for all six weights.  Contributions are kept in
 * bf16, which moe_combine rounds them to.  h % 128 == 0, f % 128 == 0,
 * experts + 1 <= 1024, top <= 32; workspace (16-byte aligned) of at least
 * akas_shared_expert_moe_workspace_size() bytes; out 16-byte aligned.
 */
size_t akas_shared_expert_moe_workspace_size(int64_t r, int experts, int top, int64_t h,
                                             int64_t f);
int akas_shared_expert_moe(const void* x, int x_dtype, const float* logits,
                           const void* shared_gate, int gate_dtype, const uint8_t* w1,
                           const void* s1, const uint8_t* w3, const void* s3, const uint8_t* w2,
                           const void* s2, const uint8_t* sw1, const void* ss1,
                           const uint8_t* sw3, const void* ss3, const uint8_t* sw2,
                           const void* ss2, int scale_dtype, float* out, void* workspace,
                           size_t workspace_bytes, int64_t r, int experts, int top, int64_t h,
                           int64_t f, void* stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* AKAS_FP8_H */
