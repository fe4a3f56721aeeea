// Launches shared between the MoE sources: the routing side (moe_route.hip)
// run by the entry points of the grouped expert kernels (moe_gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace akas {

// decode_router (bf16-rounded logits, softmax over the top-k: ids and
// weights [r, top]) and quantize of x [r, k] (x_dtype f32/f16/bf16) in one
// launch: the same ids, weights, codes and scales as the two.  Returns an
// AKAS status.
int launch_decode_router_quantize(const float* logits, int32_t* ids, float* weights, int64_t r,
                                  int experts, int top, const void* x, int x_dtype,
                                  uint8_t* codes, float* scales, int64_t k, hipStream_t s);

// quantized_routes: counts [experts] and routes [experts, r] from ids
// [r, top] and active [r] (null: every row active).
void launch_quantized_routes(const int32_t* ids, const int32_t* active, int32_t* counts,
                             int32_t* routes, int64_t r, int experts, int top, hipStream_t s);

// quantized_routes over ids [r, top] for experts + 1 experts, every row
// active: a route names the entry row * (top + 1) + rank, and expert
// `experts` routes every row at rank top.  counts [experts + 1], routes
// [experts + 1, r].
void launch_routes_with_shared(const int32_t* ids, int32_t* counts, int32_t* routes, int64_t r,
                               int experts, int top, hipStream_t s);

// moe_combine over bf16 contributions [r, top + 1, c] whose rank top is the
// shared expert: out f32 [r, c] = the weighted ranks 0 .. top-1 (weights
// [r, top]) plus rank top under the sigmoid of gate [r].  c % 8 == 0,
// 16-byte aligned contributions and out.
void launch_shared_rank_combine(const uint16_t* contributions, const float* weights,
                                const void* gate, int gate_dtype, float* out, int64_t r, int top,
                                int64_t c, hipStream_t s);

}  // namespace akas
