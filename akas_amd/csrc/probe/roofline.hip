// Roofline ceilings of the GPU, measured by two probe kernels.  Benchmark
// infrastructure built into its own library (libakas_probe.so), not part of
// the path's C ABI:
//   stream_read -- every 16-byte chunk of a buffer read once, eight loads in
//                  flight per thread, folded into one word per thread that is
//                  stored only if it matches a sentinel (so the loads stay but
//                  nothing is written);
//   mfma        -- back-to-back FP8 MFMAs (16x16x128, OCP e4m3 operands in
//                  registers) on four independent accumulators per wave;
//   load_mix    -- the loads of the decode split GEMM (16 < M <= 256,
//                  K = 2048) without its products, its LDS staging or its
//                  stores: the same workgroups, waves, tile order, load
//                  instructions, issue order and prefetch depth.
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

// The split GEMM's workgroup decomposition (16 < M <= 256, K = 2048): tiles
// of BM = 16*MT*MH rows x 48 columns, m-tiles of one column block adjacent
// after the XCD remap (workgroup i runs on XCD i % 8, and each XCD takes a
// contiguous range of tiles).  Wave (kq, mh) covers k-quarter kq (k-blocks
// 4kq .. 4kq+3) for rows mh*16*MT .. +16*MT-1.  Its loads:
//   weights: the wave's share of the quarter's 48-row slice, two rows of 512
//            contiguous bytes per 16-byte-per-lane load (BN/2/MH loads);
//   activations: AF = 1, fragment-major 16-row tiles (one 2 KB block per
//            tile and k-block), two 1 KB loads per tile and k-block; AF = 0,
//            row-major codes, four lanes per row, two 16-byte loads each
//            (64 bytes apart) per tile and k-block; PF k-blocks up front and
//            each slot refilled once it is taken;
// AFIRST issues the activations ahead of the weights.  Every word is folded
// into one register per lane.
constexpr int kMixK = 2048, kMixKb = kMixK / 128, kMixBn = 48;
// The GEMM's LDS (four quarters of a 48-row x 512-byte weight slice), held
// unused, so that one workgroup runs per CU as the GEMM's do.
constexpr size_t kMixLds = 4 * kMixBn * 512;

__device__ __forceinline__ int mix_remap(int hw_id, int total) {
  const int per = total / 8;
  if (per == 0 || hw_id >= per * 8) return hw_id;
  return (hw_id % 8) * per + hw_id / 8;
}

__device__ __forceinline__ uint32_t fold4(const u32x4& v) { return v[0] ^ v[1] ^ v[2] ^ v[3]; }

template <int MT, int MH, int PF, int AFIRST, int AF>
__global__ __launch_bounds__(256 * MH) void load_mix_kernel(const uint8_t* __restrict__ w,
                                                            const uint8_t* __restrict__ a, int M,
                                                            int N, uint32_t* __restrict__ sink) {
  constexpr int KBW = 4, WLOADS = kMixBn / 2 / MH, BM = 16 * MT * MH;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = wave % 4, mh = wave / 4;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = N / kMixBn;
  const int id = mix_remap(blockIdx.x, tiles_m * tiles_n);
  const int tm = id % tiles_m, tn = id / tiles_m;
  const int m0 = tm * BM + mh * 16 * MT, n0 = tn * kMixBn, kb0 = kq * KBW;
  const int last_tile = (M - 1) >> 4;
  const uint8_t* wsrc = w + (size_t)(n0 + mh * (kMixBn / MH) + (lane >> 5)) * kMixK +
                        (size_t)kb0 * 128 + 16 * (lane & 31);
  u32x4 wl[WLOADS];
  u32x4 ar[PF][MT][2];
  auto load_a = [&](int i, int s, u32x4 (&f)[2]) {
    if constexpr (AF) {
      const size_t t = ((size_t)(min((m0 >> 4) + i, last_tile) * kMixKb + kb0 + s) << 11) + 16 * lane;
      f[0] = *reinterpret_cast<const u32x4*>(a + t);
      f[1] = *reinterpret_cast<const u32x4*>(a + t + 1024);
    } else {
      const int row = min(m0 + 16 * i + (lane >> 2), M - 1);
      const size_t t = (size_t)row * kMixK + (size_t)(kb0 + s) * 128 + 16 * (lane & 3);
      f[0] = *reinterpret_cast<const u32x4*>(a + t);
      f[1] = *reinterpret_cast<const u32x4*>(a + t + 64);
    }
  };
  auto issue_w = [&]() {
#pragma unroll
    for (int q = 0; q < WLOADS; ++q) wl[q] = *reinterpret_cast<const u32x4*>(wsrc + (size_t)(2 * q) * kMixK);
  };
  auto issue_a = [&]() {
#pragma unroll
    for (int s = 0; s < PF; ++s)
#pragma unroll
      for (int i = 0; i < MT; ++i) load_a(i, s, ar[s][i]);
  };
  if constexpr (AFIRST) {
    issue_a();
    __builtin_amdgcn_sched_barrier(0);
    issue_w();
  } else {
    issue_w();
    __builtin_amdgcn_sched_barrier(0);
    issue_a();
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t fold = 0;
#pragma unroll
  for (int q = 0; q < WLOADS; ++q) fold ^= fold4(wl[q]);
#pragma unroll
  for (int s = 0; s < KBW; ++s) {
    const int slot = s % PF;
#pragma unroll
    for (int i = 0; i < MT; ++i) fold ^= fold4(ar[slot][i][0]) ^ fold4(ar[slot][i][1]);
    if (s + PF < KBW) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < MT; ++i) load_a(i, s + PF, ar[slot][i]);
    }
  }
  if (fold == kSentinel) sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = fold;
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

template <int AF>
static int launch_load_mix(const uint8_t* wp, const uint8_t* ap, int M, int N, uint32_t* sink,
                           hipStream_t s) {
  const int tiles_n = N / kMixBn;
  int blocks;
  if (M <= 32) {
    blocks = tiles_n * ((M + 15) / 16);
    load_mix_kernel<1, 1, 4, 1, AF><<<blocks, 256, kMixLds, s>>>(wp, ap, M, N, sink);
  } else if (M <= 64) {
    blocks = tiles_n * ((M + 31) / 32);
    load_mix_kernel<2, 1, 4, 1, AF><<<blocks, 256, kMixLds, s>>>(wp, ap, M, N, sink);
  } else if (M <= 128) {
    blocks = tiles_n * ((M + 63) / 64);
    load_mix_kernel<2, 2, 2, 0, AF><<<blocks, 512, kMixLds, s>>>(wp, ap, M, N, sink);
  } else {
    blocks = tiles_n * ((M + 127) / 128);
    load_mix_kernel<4, 2, 2, 0, AF><<<blocks, 512, kMixLds, s>>>(wp, ap, M, N, sink);
  }
  return blocks;
}

// The split GEMM's loads for M rows (16 < M <= 256) against an N x 2048
// weight matrix w (N a multiple of 48) and activations a: fragment-major
// (af = 1, ((M + 15) / 16) * 16 * 2048 bytes) or row-major (af = 0, M * 2048
// bytes); sink holds 512 words per workgroup.  The workgroup count is
// returned through *blocks_out.
PROBE_API int akas_probe_load_mix(const void* w, const void* a, int M, int N, int af,
                                  uint32_t* sink, int* blocks_out, void* stream) {
  if (!w || !a || !sink || M <= 16 || M > 256 || N < kMixBn || N % kMixBn) return -1;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint8_t* wp = reinterpret_cast<const uint8_t*>(w);
  const uint8_t* ap = reinterpret_cast<const uint8_t*>(a);
  const int blocks = af ? launch_load_mix<1>(wp, ap, M, N, sink, s) : launch_load_mix<0>(wp, ap, M, N, sink, s);
  if (blocks_out) *blocks_out = blocks;
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

PROBE_API double akas_probe_mfma_flops(int iters, int blocks) {
  return (double)blocks * (kThreads / 64) * iters * kChains * 16.0 * 16.0 * 128.0 * 2.0;
}
