// Shared device helpers for the gfx950 block-scaled FP8 path.
//
// OCP e4m3 codec, exact float32 quotient, bf16/f16 rounding, dtype-generic
// loads/stores, the FP8 MFMA wrapper and its fragment layout, and launch
// helpers.  Everything here is written for CDNA4 (gfx950) wave64.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/akas_fp8.h"

#define AKAS_DEV __device__ __forceinline__

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
// 16-byte staging word as a native vector (HIP's uint4 is a struct with a
// union, which keeps arrays of it out of registers).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

namespace akas {

constexpr int kBlock = 128;  // quantization group / weight block edge
constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// e4m3 codec
// ---------------------------------------------------------------------------

// Magnitude code of a non-negative float32, nearest-even, saturating at 126
// (448).  Normals round the f32 pattern at mantissa bit 20 and rebias by
// 960 = 120 << 3; magnitudes below 2^-6 are rint(|v| * 512).
// (src/akas/quantization/_shared/e4m3.py:16-29)
AKAS_DEV uint32_t e4m3_magnitude_code(float mag) {
  uint32_t bits = __float_as_uint(mag) & 0x7FFFFFFFu;
  uint32_t rounded = bits + 0x7FFFFu + ((bits >> 20) & 1u);
  int normal = (int)(rounded >> 20) - 960;
  int sub = (int)__builtin_rintf(mag * 512.0f);
  int code = mag < 0.015625f ? sub : normal;
  code = code < 0 ? 0 : (code > 126 ? 126 : code);
  return (uint32_t)code;
}

// Full encoder: sign of v's bit pattern ORed into the magnitude code.
AKAS_DEV uint32_t e4m3_encode(float v) {
  return e4m3_magnitude_code(__builtin_fabsf(v)) | ((__float_as_uint(v) >> 24) & 128u);
}

// e4m3 byte -> float32 (exact). (src/akas/quantization/_shared/e4m3.py:4-13)
AKAS_DEV float e4m3_decode(uint32_t b) {
  uint32_t e = (b >> 3) & 15u, f = b & 7u;
  uint32_t mag_bits = e ? (((e + 120u) << 23) | (f << 20)) : 0u;
  float mag = e ? __uint_as_float(mag_bits) : (float)f * (1.0f / 512.0f);
  return (b & 128u) ? -mag : mag;
}

// ---------------------------------------------------------------------------
// exact float32 division by a per-group scale
// ---------------------------------------------------------------------------
//
// The reference divides every element by its group scale with IEEE float32
// division.  With r = RN(1/s) (one correctly rounded division per group),
// q0 = RN(x*r), e = x - q0*s (exact through fma) and q = RN(q0 + e*r) is the
// correctly rounded quotient RN(x/s) for finite, non-underflowing operands
// (Markstein's correction theorem; Muller et al., Handbook of Floating-Point
// Arithmetic, ch. 4).  Zero keeps x's sign because callers take the sign bit
// from x, never from q.  A group holding +-inf has s = inf and r = 0; the
// correction then runs with 0 in place of s, so every finite x gives
// q = 0 = RN(x / inf) (with s itself, 0 * inf would make it NaN), and an
// infinite x gives NaN, as inf / inf does.
struct GroupScale {
  float s;  // the group scale max(max|x|, 1e-12) / 448
  float r;  // RN(1 / s)
  float c;  // s in the correction step: s when finite, else 0
};

// Both divisions without a division sequence:
//   s = RN(a / 448) by the same correction, with RN(1/448) as a constant;
//   r = RN(1 / s) by one Newton step from v_rcp_f32, e = 1 - s*y0 (exact
//   through fma), r = RN(y0 + e*y0).
// Each equals IEEE float32 division for every input it can receive (every
// float32 a in [1e-12, FLT_MAX], whose scales cover [2^-49, 2^120]),
// compared exhaustively on gfx950 by the numerics probe (probe/numerics.hip).
// An infinite maximum gives s = inf and r = c = 0, as the divisions do.
AKAS_DEV GroupScale make_group_scale(float amax) {
#pragma clang fp contract(off)
  constexpr float kInv448 = 0x1.24924ap-9f;  // RN(1/448)
  const float a = __builtin_fmaxf(amax, 1e-12f);
  const bool finite = a < __builtin_inff();
  const float q0 = a * kInv448;
  const float s = __builtin_fmaf(__builtin_fmaf(-q0, 448.0f, a), kInv448, q0);
  const float y0 = __builtin_amdgcn_rcpf(s);
  const float r = __builtin_fmaf(__builtin_fmaf(-s, y0, 1.0f), y0, y0);
  GroupScale g;
  g.s = finite ? s : a;
  g.r = finite ? r : 0.0f;
  g.c = finite ? s : 0.0f;
  return g;
}

AKAS_DEV float exact_quotient_magnitude(float ax, const GroupScale& g) {
  float q0 = ax * g.r;
  float e = __builtin_fmaf(-q0, g.c, ax);
  return __builtin_fmaf(e, g.r, q0);
}

// enc(RN(x / s)) with the sign taken from x (matches -0.0 / s = -0.0).
AKAS_DEV uint32_t e4m3_encode_scaled(float x, const GroupScale& g) {
  float q = exact_quotient_magnitude(__builtin_fabsf(x), g);
  return e4m3_magnitude_code(q) | ((__float_as_uint(x) >> 24) & 128u);
}

// Signed quotient RN(x / s), clamped to 448 in magnitude.  |x| <= max|group|
// bounds it by 448 * (1 + 2^-24) anyway; the clamp maps nothing to a new code
// (all of (448, 464) encodes to 448).
AKAS_DEV float scaled_quotient(float x, const GroupScale& g) {
  const float q = __builtin_fminf(exact_quotient_magnitude(__builtin_fabsf(x), g), 448.0f);
  return __builtin_copysignf(q, x);
}

// Hardware OCP-e4m3 conversion of two values into the low (HI=false) or high
// (HI=true) 16 bits of `old`.  For |v| < 464 it is bit-identical to the
// reference encoder (src/akas/quantization/_shared/e4m3.py:16-29), ties,
// subnormals and signed zero included -- compared over every float32
// pattern in that range on gfx950 by the numerics probe (probe/numerics.hip);
// above 464 it would produce NaN, which scaled_quotient() rules out.
template <bool HI>
AKAS_DEV uint32_t cvt_e4m3x2(float a, float b, uint32_t old) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, HI);
}

// Four scaled values -> four codes in one word (byte i = value i).
AKAS_DEV uint32_t e4m3_encode4_scaled(float x0, float x1, float x2, float x3,
                                      const GroupScale& g) {
  const uint32_t w = cvt_e4m3x2<false>(scaled_quotient(x0, g), scaled_quotient(x1, g), 0u);
  return cvt_e4m3x2<true>(scaled_quotient(x2, g), scaled_quotient(x3, g), w);
}

// ---------------------------------------------------------------------------
// bf16 / f16 conversions (round to nearest even, finite inputs)
// ---------------------------------------------------------------------------

AKAS_DEV float bf16_bits_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

// Round to nearest even (src/akas/quantization/_shared/rounding.py:43-54,
// the integer form (bits + 0x7FFF + lsb) >> 16).  gfx950's v_cvt_pk_bf16_f32
// gives the same bits as that integer form for every non-NaN f32 pattern,
// denormals included (compared over all 2^32 patterns on the GPU by the
// numerics probe, probe/numerics.hip), and
// costs one instruction per two values.
AKAS_DEV uint32_t f32_to_bf16_bits(float v) {
  const __bf16 h = (__bf16)v;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// Two values packed low/high with one v_cvt_pk_bf16_f32 (round to nearest
// even, as the scalar conversion; converting the halves one at a time costs
// two conversions, a shift and an or).
AKAS_DEV uint32_t f32x2_to_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

AKAS_DEV float round_bf16(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

AKAS_DEV float f16_bits_to_f32(uint32_t h) {
  _Float16 x;
  uint16_t b = (uint16_t)h;
  __builtin_memcpy(&x, &b, 2);
  return (float)x;
}

// The empty asm pins v as a finished float32: without it the compiler may
// fold the multiply that produced v into a mixed-precision v_mad_mix /
// v_fma_mix with an f16 result, rounding once instead of f32-then-f16 as the
// reference (and every other kernel here) does.
AKAS_DEV uint32_t f32_to_f16_bits(float v) {
  asm volatile("" : "+v"(v));
  _Float16 x = (_Float16)v;  // v_cvt_f16_f32: round to nearest even
  uint16_t b;
  __builtin_memcpy(&b, &x, 2);
  return b;
}

AKAS_DEV float round_f16(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }

// Two values packed low/high with one v_cvt_pk_f16_f32 (round to nearest
// even), each first fixed in a register as f32_to_f16_bits does.
AKAS_DEV uint32_t f32x2_to_f16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  asm volatile("" : "+v"(lo), "+v"(hi));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, f16x2));
}

AKAS_DEV float round_to(float v, int dtype) {
  return dtype == AKAS_DTYPE_BF16 ? round_bf16(v) : (dtype == AKAS_DTYPE_F16 ? round_f16(v) : v);
}

// Compile-time-dtype rounding for unrolled epilogues: a runtime dtype inside
// an unrolled loop costs a scalar branch per element.
template <int DT>
AKAS_DEV float round_t(float v) {
  if constexpr (DT == AKAS_DTYPE_BF16)
    return round_bf16(v);
  else if constexpr (DT == AKAS_DTYPE_F16)
    return round_f16(v);
  else
    return v;
}

template <int D>
struct DtypeTag {
  static constexpr int value = D;
};

// f(DtypeTag<d>{}) with the (wave-uniform) runtime dtype d made compile-time.
template <class F>
AKAS_DEV void with_dtype(int d, F&& f) {
  if (d == AKAS_DTYPE_BF16)
    f(DtypeTag<AKAS_DTYPE_BF16>{});
  else if (d == AKAS_DTYPE_F16)
    f(DtypeTag<AKAS_DTYPE_F16>{});
  else
    f(DtypeTag<AKAS_DTYPE_F32>{});
}

// Element load of a float-like buffer (f32 / f16 / bf16).
AKAS_DEV float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == AKAS_DTYPE_F32) return ((const float*)p)[i];
  uint32_t h = ((const uint16_t*)p)[i];
  return dtype == AKAS_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

AKAS_DEV void store_elem(void* p, int64_t i, float v, int dtype) {
  if (dtype == AKAS_DTYPE_F32) {
    ((float*)p)[i] = v;
  } else {
    ((uint16_t*)p)[i] = (uint16_t)(dtype == AKAS_DTYPE_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
  }
}

// Block-scale element (f32 or bf16 storage).
AKAS_DEV float load_scale(const void* p, int64_t i, int scale_dtype) {
  return scale_dtype == AKAS_DTYPE_F32 ? ((const float*)p)[i]
                                       : bf16_bits_to_f32(((const uint16_t*)p)[i]);
}

// Compile-time-dtype form for hot loops: a runtime dtype branch around a
// global load makes the compiler drain every outstanding load at the join.
template <int SDT>
AKAS_DEV float load_scale_t(const void* p, int64_t i) {
  if constexpr (SDT == AKAS_DTYPE_F32)
    return reinterpret_cast<const float*>(p)[i];
  else
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

// ---------------------------------------------------------------------------
// Correctly rounded float32 exp, and the router's sigmoid built on it
// ---------------------------------------------------------------------------
//
// exp_rn(x) = RN32(e^x), the float32 nearest to the exact exponential, for
// every float32 x whose result is a normal float32 or overflows (x >=
// -87.33); below that the result is within one subnormal step.
//
// Fast path: e^x in double (the device library's exp, within 1 ulp of
// double), rounded once to float32.  That rounding can only go wrong when
// e^x lies within about 1 double ulp of a float32 rounding midpoint, so any
// result whose low 29 fraction bits (the bits below float32 precision) lie
// within 16 units of the midpoint pattern 2^28 takes the slow path: e^x in
// double-double arithmetic (about 100 bits), rounded to float32 from both
// words.  An exhaustive scan of all float32 inputs finds about fifty such
// inputs in the range a sigmoid needs; the closest lies 1.27 double ulps
// from a midpoint.
namespace dd {
// Double-double arithmetic: value = hi + lo, |lo| <= ulp(hi) / 2.  The
// error-free transformations need every operation rounded on its own, so
// each function turns contraction off for its body.
struct Dd {
  double hi, lo;
};
AKAS_DEV Dd quick_two_sum(double a, double b) {
#pragma clang fp contract(off)
  const double s = a + b;
  return {s, b - (s - a)};
}
AKAS_DEV Dd two_sum(double a, double b) {
#pragma clang fp contract(off)
  const double s = a + b, bb = s - a;
  return {s, (a - (s - bb)) + (b - bb)};
}
AKAS_DEV Dd add(const Dd& a, const Dd& b) {
#pragma clang fp contract(off)
  const Dd s = two_sum(a.hi, b.hi), t = two_sum(a.lo, b.lo);
  const Dd u = quick_two_sum(s.hi, s.lo + t.hi);
  return quick_two_sum(u.hi, u.lo + t.lo);
}
AKAS_DEV Dd mul(const Dd& a, const Dd& b) {
#pragma clang fp contract(off)
  const double p = a.hi * b.hi;
  const double e = __builtin_fma(a.hi, b.hi, -p);
  return quick_two_sum(p, e + (a.hi * b.lo + a.lo * b.hi));
}
// a / n for a small positive integer n: the remainder of the leading
// quotient is exact through one FMA.
AKAS_DEV Dd div_int(const Dd& a, double n) {
#pragma clang fp contract(off)
  const double q = a.hi / n;
  const double rem = __builtin_fma(-q, n, a.hi);
  return quick_two_sum(q, (rem + a.lo) / n);
}
// e^x for |x| <= 104: x = k ln2 + r with |r| <= ln2/2, ln2 split as
// kLn2Hi (trailing zero bits, so k * kLn2Hi is exact and x - k * kLn2Hi is
// exact by Sterbenz's lemma) + kLn2Lo; e^r by its Taylor series to degree
// 20 in nested form 1 + r(1 + r/2(1 + r/3(...))) (truncation below 2^-90
// relative); then the exact scaling by 2^k.
AKAS_DEV Dd exp_dd(double x) {
#pragma clang fp contract(off)
  constexpr double kLn2Hi = 6.93147180369123816490e-01;  // 0x3FE62E42FEE00000
  constexpr double kLn2Lo = 1.90821492927058770002e-10;  // ln2 - kLn2Hi
  constexpr double kInvLn2 = 1.44269504088896338700e+00;
  const double k = __builtin_rint(x * kInvLn2);
  const double rhi = __builtin_fma(-k, kLn2Hi, x);  // exact
  const double p = k * kLn2Lo;
  const Dd r = add(Dd{rhi, 0.0}, Dd{-p, -__builtin_fma(k, kLn2Lo, -p)});
  Dd t{1.0, 0.0};
  for (int i = 20; i >= 1; --i) t = add(Dd{1.0, 0.0}, div_int(mul(r, t), (double)i));
  return {__builtin_ldexp(t.hi, (int)k), __builtin_ldexp(t.lo, (int)k)};
}
}  // namespace dd

// Distance, in units of the last double bit, of a positive double from the
// float32 rounding midpoint of its binade (normal float32 range).
AKAS_DEV int64_t midpoint_distance(double v) {
  const int64_t low = (int64_t)(__double_as_longlong(v) & ((1ll << 29) - 1));
  const int64_t d = low - (1ll << 28);
  return d < 0 ? -d : d;
}

AKAS_DEV float exp_rn(float x) {
  const double e = exp((double)x);
  if (midpoint_distance(e) > 16) return (float)e;
  const dd::Dd y = dd::exp_dd((double)x);
  // hi is the double nearest to hi + lo; only when hi is itself a float32
  // midpoint does lo decide the direction (lo == 0: ties to even).
  if (midpoint_distance(y.hi) != 0 || y.lo == 0.0) return (float)y.hi;
  const long long b = __double_as_longlong(y.hi);
  return (float)__longlong_as_double(y.lo > 0.0 ? b + 1 : b - 1);
}

// The sigmoid router's score term 1 / (1 + e^-l) in float32 with a
// correctly rounded exponential and IEEE addition and division: the
// reference kernel's float32 expression (src/akas/ops/moe/kernel.py:171,
// :189-190) with every step rounded once.
AKAS_DEV float router_sigmoid(float l) { return __fdiv_rn(1.0f, 1.0f + exp_rn(-l)); }

// ---------------------------------------------------------------------------
// SwiGLU element: g / (1 + exp(-g)) * u in float32
// (src/akas/ops/activation/kernel.py:83-88).  One definition shared by the
// fused and the separate kernels so their results are bit-identical.
// ---------------------------------------------------------------------------
//
// exp(-g) = 2^t with t = -g * log2(e) formed as a rounded head t0 plus the
// tail recovered by FMA (Cody-Waite style argument splitting, log2(e) held as
// a float head + float tail), so the argument carries ~1 ulp of error even
// for large |g|; 2^t0 comes from v_exp_f32 and the tail is applied as
// 2^t0 * (1 + tail * ln 2) (a product, not an FMA, so an overflowed 2^t0
// stays +inf instead of inf - inf).  1 / (1 + e) uses v_rcp_f32.  The result is
// within a few float ulp of g / (1 + exp(-g)) * u -- well inside the
// reference's 2e-6 relative code band -- at about a tenth of the cost of
// expf plus a correctly rounded division.
AKAS_DEV float swiglu_elem(float g, float u) {
  // Every fused multiply-add below is explicit: automatic contraction would
  // depend on the surrounding code and could round the fused and the
  // separate kernels differently.
#pragma clang fp contract(off)
  constexpr float kLog2eHi = 1.44269502162933349609375f;   // float(log2 e)
  constexpr float kLog2eLo = 1.925963033500011079e-8f;     // log2 e - kLog2eHi
  constexpr float kLn2 = 0.693147180559945309f;
  const float x = -g;
  const float t0 = x * kLog2eHi;
  const float tail = __builtin_fmaf(x, kLog2eLo, __builtin_fmaf(x, kLog2eHi, -t0));
  const float p = __builtin_amdgcn_exp2f(t0);
  const float e = p * (1.0f + tail * kLn2);  // stays +inf when 2^t0 overflows
  const float sig = __builtin_amdgcn_rcpf(1.0f + e);
  return g * sig * u;
}

// ---------------------------------------------------------------------------
// FP8 MFMA: D(16x16, f32) = A(16x128, e4m3) * B(128x16, e4m3)
// ---------------------------------------------------------------------------
//
// Fragment layout used throughout (wave64):
//   A operand: lane l holds 32 bytes of row (l % 16), k-group g = l / 16,
//              bytes k = 32*g .. 32*g+31 of the 128-deep block.
//   B operand: lane l holds the same 32 k-bytes of column (l % 16).
//   D:         lane l, element i holds row 4*(l/16) + i, column l % 16.
// The instruction sums matching (lane group, byte) positions of A and B, so
// any consistent assignment of k to (g, byte) gives the same product.  The
// row/column assignment of D is verified on the device by the exact-product
// tests with distinct per-row and per-block scales in tests/test_gpu_linear.py
// (a misplaced row or column lands on a different scale and fails them).
// The scaled MFMA with unit E8M0 scales (127) is the plain FP8 product;
// format code 0 selects OCP e4m3 for both operands.
AKAS_DEV v4f mfma_e4m3(const v8i& a, const v8i& b) {
  v4f z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127, 0, 127);
}

AKAS_DEV v4f mfma_e4m3_acc(const v8i& a, const v8i& b, const v4f& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// ---------------------------------------------------------------------------
// wave reductions
// ---------------------------------------------------------------------------
AKAS_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

AKAS_DEV int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Inclusive prefix sum across the 64 lanes.
AKAS_DEV int wave_inclusive_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

// ---------------------------------------------------------------------------
// launch helpers
// ---------------------------------------------------------------------------

// gfx950 dispatches consecutive workgroups round-robin over its 8 XCDs, each
// with a private L2.  Remap the hardware id so that consecutive logical tiles
// land on the same XCD (and share its L2) while every XCD gets an equal share.
AKAS_DEV int xcd_remap(int hw_id, int total) {
  constexpr int kXcd = 8;
  int per = total / kXcd;
  if (per == 0 || hw_id >= per * kXcd) return hw_id;
  return (hw_id % kXcd) * per + hw_id / kXcd;
}

}  // namespace akas

// Host-side status helpers.
#define AKAS_CHECK_LAUNCH()                              \
  do {                                                   \
    if (hipGetLastError() != hipSuccess) return AKAS_ERR_LAUNCH; \
  } while (0)
