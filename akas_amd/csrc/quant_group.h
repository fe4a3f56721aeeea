// One 1x128 activation group quantized by 16 consecutive lanes (8 values
// each): shared by the standalone quantizer and the GEMMs that quantize
// their activation slab while staging it, so both produce the same codes.
// (src/akas/quantization/activations/fp8/cuda.py:10-56, warp form :80-141)
#pragma once

#include "common.h"

namespace akas {

// 8 contiguous values of a float buffer of dtype DT, widened to f32.
template <int DT>
AKAS_DEV void load8(const void* x, int64_t base, float v[8]) {
  if constexpr (DT == AKAS_DTYPE_F32) {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + base);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    uint4 w = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + base);
    uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == AKAS_DTYPE_BF16) {
        v[2 * i] = __uint_as_float(u[i] << 16);
        v[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
      } else {
        v[2 * i] = f16_bits_to_f32(u[i] & 0xFFFFu);
        v[2 * i + 1] = f16_bits_to_f32(u[i] >> 16);
      }
    }
  }
}

// The same 8 values as raw bits, widened later by unpack8: a kernel can put
// these loads in flight ahead of others and convert once they arrive.
struct Raw8 {
  u32x4 lo, hi;  // hi: second half of an f32 octet (unused for 16-bit dtypes)
};

template <int DT>
AKAS_DEV Raw8 load8_raw(const void* x, int64_t base) {
  Raw8 r;
  if constexpr (DT == AKAS_DTYPE_F32) {
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(x) + base);
    r.lo = p[0];
    r.hi = p[1];
  } else {
    r.lo = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(x) + base);
    r.hi = u32x4{0u, 0u, 0u, 0u};
  }
  return r;
}

template <int DT>
AKAS_DEV void unpack8(const Raw8& r, float v[8]) {
  if constexpr (DT == AKAS_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = __uint_as_float(r.lo[i]);
      v[4 + i] = __uint_as_float(r.hi[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == AKAS_DTYPE_BF16) {
        v[2 * i] = __uint_as_float(r.lo[i] << 16);
        v[2 * i + 1] = __uint_as_float(r.lo[i] & 0xFFFF0000u);
      } else {
        v[2 * i] = f16_bits_to_f32(r.lo[i] & 0xFFFFu);
        v[2 * i + 1] = f16_bits_to_f32(r.lo[i] >> 16);
      }
    }
  }
}

// Codes of this lane's 8 values (low word = values 0..3) and the group scale
// max(max|x|, 1e-12) / 448, the maximum taken over the 16 lanes of the group
// (lanes 16*i .. 16*i+15 of the wave, all active).
//
// The 16-lane maximum is four DPP row operations (quad swaps, then the
// half-row and row mirrors), which stay in the VALU instead of going
// through the LDS crossbar as lane shuffles do.  The lane maxima are
// non-negative and never a quiet NaN (the lane's own maximum skips one), so
// the unsigned maximum of their bit patterns is their float maximum; it
// folds each DPP move into a v_max_u32_dpp.
template <int CTRL>
AKAS_DEV float dpp_max(float m) {
  const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, __float_as_int(m), CTRL, 0xF, 0xF, true);
  const uint32_t b = __float_as_uint(m);
  return __uint_as_float(b > o ? b : o);
}

AKAS_DEV float row16_max(float m) {
  m = dpp_max<0xB1>(m);   // quad_perm [1,0,3,2]: lane ^ 1
  m = dpp_max<0x4E>(m);   // quad_perm [2,3,0,1]: lane ^ 2
  m = dpp_max<0x141>(m);  // row_half_mirror: lane i <- 7 - i within 8 lanes
  return dpp_max<0x140>(m);  // row_mirror: lane i <- 15 - i within 16 lanes
}

AKAS_DEV uint2 quantize8(const float v[8], float& scale) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = __builtin_fmaxf(m, __builtin_fabsf(v[i]));
  m = row16_max(m);
  const GroupScale gs = make_group_scale(m);
  scale = gs.s;
  return make_uint2(e4m3_encode4_scaled(v[0], v[1], v[2], v[3], gs),
                    e4m3_encode4_scaled(v[4], v[5], v[6], v[7], gs));
}

// Activation quantizer launch (quantize.hip): row-major codes [rows, k], or
// the fragment-major tiles of the decode GEMM when fragment_major is set
// (rows rounded up to 16; the padding rows of the last tile are not written).
int launch_quantize(const void* x, int x_dtype, uint8_t* out, float* scales, int64_t rows,
                    int64_t k, bool fragment_major, hipStream_t s);

}  // namespace akas
