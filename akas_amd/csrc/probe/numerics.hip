// Exhaustive checks of device helpers against the arithmetic they stand
// for, for the tests (built into libakas_probe.so, not part of the path's C
// ABI).
//
// group_scale -- make_group_scale (common.h) forms a 1x128 group's scale
//   s = max(amax, 1e-12) / 448 and its reciprocal r = 1 / s without a
//   division sequence.  For every float32 amax in [1e-12, FLT_MAX] (every
//   value the group maximum can take at or above the floor; every scale in
//   [2^-49, 2^120] is reached) it compares s with the correctly rounded
//   quotient, r with the correctly rounded reciprocal of that s, and the
//   correction term c with s; amax = +inf must give s = inf, r = c = 0.
// e4m3_pack  -- the hardware pack v_cvt_pk_fp8_f32 (cvt_e4m3x2), which the
//   quantizers use on quotients clamped to 448, against e4m3_encode, the
//   integer restatement of the reference encoder
//   (src/akas/quantization/_shared/e4m3.py:16-29), for every float32 with
//   |v| < 464, both signs, zeros and subnormals included.
// bf16_pack  -- v_cvt_pk_bf16_f32 (f32x2_to_bf16x2) against the reference's
//   integer round to nearest even, (bits + 0x7FFF + lsb) >> 16
//   (src/akas/quantization/_shared/rounding.py:43-54), for every non-NaN
//   float32 pattern.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../common.h"

#define PROBE_API extern "C" __attribute__((visibility("default")))

namespace {

constexpr uint32_t kScaleLo = 0x2B8CBCCCu;  // 1e-12f
constexpr uint32_t kScaleHi = 0x7F7FFFFFu;  // FLT_MAX

// out[0]: mismatching inputs; out[1..8]: the first few of them (bit patterns).
__device__ void note_mismatch(unsigned long long* out, uint64_t b) {
  const unsigned long long k = atomicAdd(&out[0], 1ull);
  if (k < 8) out[1 + k] = b;
}

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
    if (!ok) note_mismatch(out, b);
  }
}

// Patterns 0 .. 0x43E7FFFF (|v| < 464) with either sign bit.
__global__ __launch_bounds__(256) void e4m3_pack_check_kernel(unsigned long long* __restrict__ out) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < 2ull * 0x43E80000ull; i += stride) {
    const uint32_t b = (uint32_t)(i >> 1) | ((uint32_t)(i & 1) << 31);
    const float v = __uint_as_float(b);
    const uint32_t hw = akas::cvt_e4m3x2<false>(v, v, 0u) & 0xFFu;
    if (hw != akas::e4m3_encode(v)) note_mismatch(out, b);
  }
}

__global__ __launch_bounds__(256) void bf16_pack_check_kernel(unsigned long long* __restrict__ out) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < (1ull << 32); b += stride) {
    const uint32_t u = (uint32_t)b;
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) continue;  // NaN
    const float v = __uint_as_float(u);
    const uint32_t want = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    const uint32_t got = akas::f32x2_to_bf16x2(v, v);
    if ((got & 0xFFFFu) != want || (got >> 16) != want) note_mismatch(out, b);
  }
}

}  // namespace

// out: 9 device words, zeroed by the caller.  Returns 0 once launched.
PROBE_API int akas_probe_e4m3_pack_check(unsigned long long* out, void* stream) {
  if (!out) return -1;
  e4m3_pack_check_kernel<<<8192, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(out);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// out: 9 device words, zeroed by the caller.  Returns 0 once launched.
PROBE_API int akas_probe_bf16_pack_check(unsigned long long* out, void* stream) {
  if (!out) return -1;
  bf16_pack_check_kernel<<<8192, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(out);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// out: 9 device words, zeroed by the caller.  Returns 0 once launched.
PROBE_API int akas_probe_group_scale_check(unsigned long long* out, void* stream) {
  if (!out) return -1;
  group_scale_check_kernel<<<8192, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(out);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
