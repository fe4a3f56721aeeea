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

constexpr int64_t kRmsQuantizeMaxCols = 8192;  // four waves of at most 2048 columns

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

// RMSNorm fused with the 1x128 quantizer (the producer step before the
// quantizer in the LFM2 programs: kinds "rms" then "quantize").
//   y = round_YT( (x * (1 / sqrt(sum(x^2) / cols + eps))) * w' ),
//   w' = w, or 1 + w when zero_centered
// (src/akas/ops/normalization/definition.py:10-31, equation of
// normalization/validation.py:31-52), written when y != nullptr, and the
// codes/scales of exactly those rounded values (quantize8, the quantizer's
// own group code).
//
// WPR waves per row (1 up to 2048 columns, 4 beyond): wave q of a row owns
// columns [q*span, q*span + span) with span a multiple of 128 and at most
// 2048, and lane l holds, for chunk j, the 8 values at span offset
// 512j + 8l .. +7, so 16 lanes own one 128-group as in the quantizer.  The
// sum of squares is accumulated per lane in chunk order, reduced by a fixed
// xor butterfly within the wave (every lane ends with the same total) and,
// for WPR = 4, summed over the waves in wave order through LDS.
template <int DT, int WT, int YT, int WPR>
__global__ __launch_bounds__(256) void rms_quantize_kernel(const void* __restrict__ x,
                                                           const void* __restrict__ w, float eps,
                                                           int zero_centered, void* __restrict__ y,
                                                           uint8_t* __restrict__ codes,
                                                           float* __restrict__ scales,
                                                           int64_t rows, int cols, int span) {
  constexpr int NJ = 4;  // 4 x 512 = 2048 columns per wave at most
  constexpr int ROWS_PER_BLOCK = 4 / WPR;
  __shared__ float part[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = wave % WPR;
  const int c0 = q * span, c1 = min(c0 + span, cols);
  const int groups = cols / kBlock;
  // every thread of a block runs the same number of iterations (WPR = 4
  // synchronizes inside the loop)
  for (int64_t r0 = (int64_t)blockIdx.x * ROWS_PER_BLOCK; r0 < rows; r0 += (int64_t)gridDim.x * ROWS_PER_BLOCK) {
    const int64_t row = r0 + wave / WPR;
    const bool live = row < rows;
    const int64_t rbase = (live ? row : r0) * cols;
    // All of the row's chunks are requested before the first is used (a
    // load under its chunk's condition waited for the one before).
    Raw8 raw[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = c0 + 512 * j + 8 * lane;
      raw[j] = load8_raw<DT>(x, rbase + (col < c1 ? col : c0));
    }
    float v[NJ][8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = c0 + 512 * j + 8 * lane;
      if (live && col < c1) {
        unpack8<DT>(raw[j], v[j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[j][e], v[j][e], ss);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[j][e] = 0.f;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if constexpr (WPR > 1) {
      if (lane == 0) part[wave] = ss;
      __syncthreads();
      ss = part[0];
#pragma unroll
      for (int k = 1; k < WPR; ++k) ss += part[k];
      __syncthreads();  // the next row's partials overwrite part[]
    }
    if (!live) continue;
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)cols) + eps));
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = c0 + 512 * j + 8 * lane;
      // all 16 lanes of a group are on the same side of c1 (multiples of 128)
      if (c0 + 512 * j + 8 * (lane & ~15) >= c1) continue;
      float wv[8];
      load8<WT>(w, col, wv);
      float qv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float we = zero_centered ? 1.0f + wv[e] : wv[e];
        qv[e] = round_t<YT>((v[j][e] * inv) * we);
      }
      if (y != nullptr) {
        if constexpr (YT == AKAS_DTYPE_F32) {
          float4* dst = reinterpret_cast<float4*>(reinterpret_cast<float*>(y) + rbase + col);
          dst[0] = float4{qv[0], qv[1], qv[2], qv[3]};
          dst[1] = float4{qv[4], qv[5], qv[6], qv[7]};
        } else {
          uint4 pk;
          uint32_t* u = reinterpret_cast<uint32_t*>(&pk);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            u[i] = YT == AKAS_DTYPE_BF16 ? f32x2_to_bf16x2(qv[2 * i], qv[2 * i + 1])
                                         : f32x2_to_f16x2(qv[2 * i], qv[2 * i + 1]);
          *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(y) + rbase + col) = pk;
        }
      }
      float sc;
      const uint2 c8 = quantize8(qv, sc);
      *reinterpret_cast<uint2*>(codes + rbase + col) = c8;
      if ((lane & 15) == 0) scales[row * groups + col / kBlock] = sc;
    }
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

template <int DT, int WT, int YT>
static int launch_rms_quantize_t(const void* x, const void* w, float eps, int zero_centered, void* y,
                                 uint8_t* codes, float* scales, int64_t rows, int cols, hipStream_t s) {
  if (cols <= 2048) {  // one wave per row, four rows per 256-thread block
    const int64_t want = (rows + 3) / 4;
    const int grid = (int)(want < 16384 ? want : 16384);
    rms_quantize_kernel<DT, WT, YT, 1><<<grid, 256, 0, s>>>(x, w, eps, zero_centered, y, codes, scales,
                                                            rows, cols, cols);
  } else {  // four waves per row, spans of whole 128-groups
    const int span = (((cols + 3) / 4 + kBlock - 1) / kBlock) * kBlock;
    const int grid = (int)(rows < 16384 ? rows : 16384);
    rms_quantize_kernel<DT, WT, YT, 4><<<grid, 256, 0, s>>>(x, w, eps, zero_centered, y, codes, scales,
                                                            rows, cols, span);
  }
  return hipGetLastError() == hipSuccess ? AKAS_OK : AKAS_ERR_LAUNCH;
}

static int launch_rms_quantize(const void* x, int x_dtype, const void* w, int w_dtype, float eps,
                               int zero_centered, void* y, int y_dtype, uint8_t* codes, float* scales,
                               int64_t rows, int cols, hipStream_t s) {
  auto by_w = [&](auto XD, auto YD) {
    constexpr int X = decltype(XD)::value, Y = decltype(YD)::value;
    return w_dtype == AKAS_DTYPE_F32
               ? launch_rms_quantize_t<X, AKAS_DTYPE_F32, Y>(x, w, eps, zero_centered, y, codes, scales, rows, cols, s)
               : launch_rms_quantize_t<X, AKAS_DTYPE_BF16, Y>(x, w, eps, zero_centered, y, codes, scales, rows, cols, s);
  };
  auto by_y = [&](auto XD) {
    switch (y_dtype) {
      case AKAS_DTYPE_F32: return by_w(XD, DtypeTag<AKAS_DTYPE_F32>{});
      case AKAS_DTYPE_F16: return by_w(XD, DtypeTag<AKAS_DTYPE_F16>{});
      default: return by_w(XD, DtypeTag<AKAS_DTYPE_BF16>{});
    }
  };
  switch (x_dtype) {
    case AKAS_DTYPE_F32: return by_y(DtypeTag<AKAS_DTYPE_F32>{});
    case AKAS_DTYPE_F16: return by_y(DtypeTag<AKAS_DTYPE_F16>{});
    default: return by_y(DtypeTag<AKAS_DTYPE_BF16>{});
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

extern "C" int akas_rms_quantize(const void* x, int x_dtype, const void* w, int w_dtype, float eps,
                                 int zero_centered, void* y, int y_dtype, uint8_t* codes,
                                 float* scales, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0 || cols % kBlock || cols > kRmsQuantizeMaxCols) return AKAS_ERR_GEOMETRY;
  if (!float_dtype(x_dtype) || !float_dtype(y_dtype)) return AKAS_ERR_DTYPE;
  if (w_dtype != AKAS_DTYPE_F32 && w_dtype != AKAS_DTYPE_BF16) return AKAS_ERR_DTYPE;
  if (!(eps >= 0.f) || !(eps < __builtin_huge_valf())) return AKAS_ERR_GEOMETRY;
  if (rows == 0) return AKAS_OK;
  if (!x || !w || !codes || !scales) return AKAS_ERR_NULL;
  // 16-byte loads and stores of 8-value chunks, 8-byte code stores
  const auto misaligned = [](const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a != 0; };
  if (misaligned(x, 16) || misaligned(w, 16) || (y && misaligned(y, 16)) || misaligned(codes, 8) ||
      misaligned(scales, 4))
    return AKAS_ERR_GEOMETRY;
  return launch_rms_quantize(x, x_dtype, w, w_dtype, eps, zero_centered ? 1 : 0, y, y_dtype, codes,
                             scales, rows, (int)cols, reinterpret_cast<hipStream_t>(stream));
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
