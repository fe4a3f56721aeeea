// Roofline ceilings of the GPU, measured by two probe kernels.  Benchmark
// infrastructure built into its own library (libakas_probe.so), not part of
// the path's C ABI:
//   stream_read -- every 16-byte chunk of a buffer read once, eight loads in
//                  flight per thread, folded into one word per thread that is
//                  stored only if it matches a sentinel (so the loads stay but
//                  nothing is written);
//   mfma        -- back-to-back FP8 MFMAs (16x16x128, OCP e4m3 operands in
//                  registers) on four independent accumulators per wave.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define PROBE_API extern "C" __attribute__((visibility("default")))

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;
constexpr uint32_t kSentinel = 0x9E3779B9u;

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src,
                                                              size_t chunks,
                                                              uint32_t* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * kThreads;
  size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
  uint32_t fold = 0;
  for (; i + (kUnroll - 1) * stride < chunks; i += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = src[i + u * stride];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) fold ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < chunks; i += stride) {
    const u32x4 v = src[i];
    fold ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (fold == kSentinel) sink[(size_t)blockIdx.x * kThreads + threadIdx.x] = fold;
}

constexpr int kChains = 4;

__global__ __launch_bounds__(kThreads) void mfma_kernel(uint32_t* __restrict__ sink, int iters) {
  const int lane = threadIdx.x & 63;
  v8i a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = 0x38383838 ^ (lane * 0x01010101 & 0x07070707);  // finite e4m3 codes
    b[e] = 0x30303030 ^ (e * 0x01010101);
  }
  v4f acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c)
      acc[c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[c], 0, 0, 0, 127, 0, 127);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  if (__float_as_uint(s) == kSentinel) sink[(size_t)blockIdx.x * kThreads + threadIdx.x] = 1u;
}

}  // namespace

// Reads `bytes` (a multiple of 16) from src with `blocks` workgroups of 256
// threads; sink holds blocks * 256 words (written only on a sentinel match).
PROBE_API int akas_probe_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks,
                                     void* stream) {
  if (!src || !sink || bytes % 16 || blocks < 1) return -1;
  stream_read_kernel<<<blocks, kThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const u32x4*>(src), bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// blocks workgroups of four waves, each wave issuing iters * 4 MFMAs of
// 16 x 16 x 128 (65,536 flops each); sink as above.
PROBE_API int akas_probe_mfma(uint32_t* sink, int iters, int blocks, void* stream) {
  if (!sink || iters < 1 || blocks < 1) return -1;
  mfma_kernel<<<blocks, kThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(sink, iters);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

PROBE_API double akas_probe_mfma_flops(int iters, int blocks) {
  return (double)blocks * (kThreads / 64) * iters * kChains * 16.0 * 16.0 * 128.0 * 2.0;
}
