// FP8 activation quantizer (1 x 128 groups), activation dequantizer and the
// 128 x 128 weight block quantizer for gfx950.
//
// Activation quantize is HBM-bound: 16 lanes own one 128-value group, each
// lane streams 8 contiguous values (one 16-byte load for bf16/f16, two for
// f32), the group maximum is a 16-lane butterfly, and each lane stores its 8
// codes as one 8-byte word.  Division by the group scale is the exact
// correctly rounded quotient (common.h), so codes match the reference's IEEE
// division bit for bit.
#include "quant_group.h"

namespace akas {

// One 128-group per 16 lanes; grid-stride over all groups.
// (src/akas/quantization/activations/fp8/cuda.py:10-56, warp form :80-141)
//
// FRAG selects the fragment-major code layout that the decode GEMM reads:
// the codes of rows 16t..16t+15, k-block b form one 2 KB tile at
// (t * KB + b) * 2048, in which MFMA lane l = r + 16g (row r) finds chunks g
// and 4+g of its row (16 bytes each) at 16l and 1024 + 16l, so one
// contiguous 1 KB load per half delivers a whole operand fragment.  Groups
// are then taken tile by tile (16 rows of one k-block per 256 threads), so
// a block writes one whole tile; the padding rows of the last tile are
// skipped.
template <int DT, bool FRAG>
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ x,
                                                       uint8_t* __restrict__ out,
                                                       float* __restrict__ scales,
                                                       int64_t groups, int kb_per_row, int64_t rows) {
  const int lane16 = threadIdx.x & 15;
  const int64_t first = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4;
  const int64_t stride = ((int64_t)gridDim.x * blockDim.x) >> 4;
  for (int64_t g = first; g < groups; g += stride) {
    int64_t gi = g, at;                         // gi: the group in row-major order
    if constexpr (FRAG) {
      const int64_t t = g >> 4;                 // tile (16-row block, k-block)
      const int64_t kb = t % kb_per_row, rb = t / kb_per_row;
      const int r = (int)(g & 15), c = lane16 >> 1;
      const int64_t row = rb * 16 + r;
      if (row >= rows) continue;                // uniform across the group's 16 lanes
      gi = row * kb_per_row + kb;
      at = ((rb * kb_per_row + kb) << 11) + ((c >> 2) << 10) + ((r + 16 * (c & 3)) << 4) + 8 * (lane16 & 1);
    }
    const int64_t base = gi * kBlock + lane16 * 8;
    if constexpr (!FRAG) at = base;
    float v[8], s;
    load8<DT>(x, base, v);
    const uint2 codes = quantize8(v, s);
    *reinterpret_cast<uint2*>(out + at) = codes;
    if (lane16 == 0) scales[gi] = s;
  }
}

__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t* __restrict__ codes,
                                                         const float* __restrict__ scales,
                                                         void* __restrict__ out, int out_dtype,
                                                         int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float v = e4m3_decode(codes[i]) * scales[i / kBlock];
    store_elem(out, i, v, out_dtype);
  }
}

// One workgroup per 128 x 128 weight block: block max, scale, codes.
__global__ __launch_bounds__(256) void weight_block_kernel(const float* __restrict__ w,
                                                           uint8_t* __restrict__ codes,
                                                           void* __restrict__ scales,
                                                           int scale_dtype, int64_t n,
                                                           int64_t k) {
  __shared__ float red[4];
  const int64_t nb = (n + kBlock - 1) / kBlock, kb = k / kBlock;
  const int64_t blk = blockIdx.x;
  const int64_t b = blk / (nb * kb), rem = blk % (nb * kb);
  const int64_t bn = rem / kb, bk = rem % kb;
  const float* src = w + b * n * k;
  uint8_t* dst = codes + b * n * k;
  const int t = threadIdx.x;
  float m = 0.f;
  for (int e = t; e < kBlock * kBlock; e += 256) {
    int64_t row = bn * kBlock + e / kBlock, col = bk * kBlock + e % kBlock;
    if (row < n) m = __builtin_fmaxf(m, __builtin_fabsf(src[row * k + col]));
  }
  m = wave_max(m);
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  m = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
  float s = __fdiv_rn(__builtin_fmaxf(m, 1e-12f), 448.0f);
  if (scale_dtype == AKAS_DTYPE_BF16) s = round_bf16(s);
  for (int e = t; e < kBlock * kBlock; e += 256) {
    int64_t row = bn * kBlock + e / kBlock, col = bk * kBlock + e % kBlock;
    if (row < n) {
      float v = src[row * k + col];
      dst[row * k + col] = (uint8_t)e4m3_encode(__fdiv_rn(v, s));
    }
  }
  if (t == 0) {
    int64_t si = b * nb * kb + bn * kb + bk;
    if (scale_dtype == AKAS_DTYPE_F32)
      reinterpret_cast<float*>(scales)[si] = s;
    else
      reinterpret_cast<uint16_t*>(scales)[si] = (uint16_t)f32_to_bf16_bits(s);
  }
}

static inline bool float_dtype(int d) {
  return d == AKAS_DTYPE_F32 || d == AKAS_DTYPE_F16 || d == AKAS_DTYPE_BF16;
}

}  // namespace akas


using namespace akas;

namespace akas {

template <bool FRAG>
static void launch_quantize_t(const void* x, int x_dtype, uint8_t* out, float* scales,
                              int64_t groups, int kb_per_row, int64_t rows, hipStream_t s) {
  const int64_t want = (groups + 15) / 16;  // 16 groups per 256-thread block
  const int grid = (int)(want < 8192 ? want : 8192);
  switch (x_dtype) {
    case AKAS_DTYPE_F32:
      quantize_kernel<AKAS_DTYPE_F32, FRAG><<<grid, 256, 0, s>>>(x, out, scales, groups, kb_per_row, rows);
      break;
    case AKAS_DTYPE_F16:
      quantize_kernel<AKAS_DTYPE_F16, FRAG><<<grid, 256, 0, s>>>(x, out, scales, groups, kb_per_row, rows);
      break;
    default:
      quantize_kernel<AKAS_DTYPE_BF16, FRAG><<<grid, 256, 0, s>>>(x, out, scales, groups, kb_per_row, rows);
  }
}

int launch_quantize(const void* x, int x_dtype, uint8_t* out, float* scales, int64_t rows,
                    int64_t k, bool fragment_major, hipStream_t s) {
  const int kb = (int)(k / kBlock);
  if (fragment_major)  // whole 16-row tiles, padding rows skipped
    launch_quantize_t<true>(x, x_dtype, out, scales, ((rows + 15) / 16) * 16 * kb, kb, rows, s);
  else
    launch_quantize_t<false>(x, x_dtype, out, scales, rows * kb, kb, rows, s);
  return hipGetLastError() == hipSuccess ? AKAS_OK : AKAS_ERR_LAUNCH;
}

}  // namespace akas

extern "C" int akas_quantize(const void* x, int x_dtype, uint8_t* out, float* scales,
                             int64_t rows, int64_t k, void* stream) {
  if (rows < 0 || k <= 0 || k % kBlock) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(x_dtype)) return AKAS_ERR_DTYPE;
  if (rows == 0) return AKAS_OK;
  if (!x || !out || !scales) return AKAS_ERR_NULL;
  return launch_quantize(x, x_dtype, out, scales, rows, k, false, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int akas_dequantize_fp8(const uint8_t* codes, const float* scales, void* out,
                                   int out_dtype, int64_t rows, int64_t k, void* stream) {
  if (rows < 0 || k <= 0 || k % kBlock) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(out_dtype)) return AKAS_ERR_DTYPE;
  if (rows == 0) return AKAS_OK;
  if (!codes || !scales || !out) return AKAS_ERR_NULL;
  const int64_t n = rows * k;
  const int64_t want = (n + 255) / 256;
  const int grid = (int)(want < 16384 ? want : 16384);
  dequantize_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(codes, scales, out,
                                                                             out_dtype, n);
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}

extern "C" int akas_quantize_weight_blocks(const float* w, uint8_t* codes, void* scales,
                                           int scale_dtype, int64_t batch, int64_t n, int64_t k,
                                           void* stream) {
  if (batch < 0 || n < 0 || k <= 0 || k % kBlock) return AKAS_ERR_GEOMETRY;
  if (scale_dtype != AKAS_DTYPE_F32 && scale_dtype != AKAS_DTYPE_BF16) return AKAS_ERR_DTYPE;
  if (batch == 0 || n == 0) return AKAS_OK;
  if (!w || !codes || !scales) return AKAS_ERR_NULL;
  const int64_t blocks = batch * ((n + kBlock - 1) / kBlock) * (k / kBlock);
  if (blocks > 0x7FFFFFFF) return AKAS_ERR_GEOMETRY;
  weight_block_kernel<<<(int)blocks, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      w, codes, scales, scale_dtype, n, k);
  AKAS_CHECK_LAUNCH();
  return AKAS_OK;
}
