// Exhaustive check of a device helper against IEEE float32 arithmetic, for
// the tests (built into libakas_probe.so, not part of the path's C ABI).
//
// group_scale -- make_group_scale (common.h) forms a 1x128 group's scale
//   s = max(amax, 1e-12) / 448 and its reciprocal r = 1 / s without a
//   division sequence.  For every float32 amax in [1e-12, FLT_MAX] (every
//   value the group maximum can take at or above the floor; every scale in
//   [2^-49, 2^120] is reached) it compares s with the correctly rounded
//   quotient, r with the correctly rounded reciprocal of that s, and the
//   correction term c with s; amax = +inf must give s = inf, r = c = 0.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../common.h"

#define PROBE_API extern "C" __attribute__((visibility("default")))

namespace {

constexpr uint32_t kScaleLo = 0x2B8CBCCCu;  // 1e-12f
constexpr uint32_t kScaleHi = 0x7F7FFFFFu;  // FLT_MAX

// out[0]: mismatching inputs; out[1..8]: the first few of them (bit patterns).
__global__ __launch_bounds__(256) void group_scale_check_kernel(unsigned long long* __restrict__ out) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t b = kScaleLo + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b <= kScaleHi + 1ull;
       b += stride) {
    const bool inf = b == kScaleHi + 1ull;  // 0x7F800000
    const float a = __uint_as_float((uint32_t)b);
    const akas::GroupScale g = akas::make_group_scale(a);
    bool ok;
    if (inf) {
      ok = g.s == __builtin_inff() && __float_as_uint(g.r) == 0u && __float_as_uint(g.c) == 0u;
    } else {
      const float s = __fdiv_rn(a, 448.0f);
      ok = __float_as_uint(g.s) == __float_as_uint(s) &&
           __float_as_uint(g.r) == __float_as_uint(__fdiv_rn(1.0f, s)) &&
           __float_as_uint(g.c) == __float_as_uint(s);
    }
    if (!ok) {
      const unsigned long long k = atomicAdd(&out[0], 1ull);
      if (k < 8) out[1 + k] = b;
    }
  }
}

}  // namespace

// out: 9 device words, zeroed by the caller.  Returns 0 once launched.
PROBE_API int akas_probe_group_scale_check(unsigned long long* out, void* stream) {
  if (!out) return -1;
  group_scale_check_kernel<<<8192, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(out);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
