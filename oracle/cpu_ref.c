/*
 * CPU restatement of the reference's block-scaled FP8 equations, in C.
 *
 * TEST INFRASTRUCTURE AND CPU BASELINE ONLY (see oracle/__init__.py): used by
 * tests/ as a checker and by bench.py's cpu_baseline leg as the timed CPU
 * path.  The product (akas_amd) never links it.
 *
 * Follows:
 *   e4m3 encode/decode   src/akas/quantization/_shared/e4m3.py:4-29
 *   quantize             src/akas/quantization/activations/fp8/validation.py:27-36
 *   fp8 linear           src/akas/ops/linear/validation.py:206-230 (f32 here)
 *   MoE layer            tests/support/native_fp8_reference.py:116-144 with the
 *                        softmax router of src/akas/ops/moe/kernel.py:444-499
 * Accumulation is float32 (the timed baseline); weights decode through a
 * 256-entry table.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static float g_lut[256];
static int g_lut_ready = 0;

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* e4m3.py:4-13 */
float ref_decode_e4m3(uint8_t b) {
  int e = (b >> 3) & 15, f = b & 7;
  float mag = e == 0 ? (float)f / 512.0f : (1.0f + (float)f / 8.0f) * ldexpf(1.0f, e - 7);
  return (b & 128) ? -mag : mag;
}

/* e4m3.py:16-29 */
uint8_t ref_encode_e4m3(float v) {
  uint32_t bits = f2u(v);
  float mag = fabsf(v);
  uint32_t rounded = (bits & 0x7FFFFFFFu) + 0x7FFFFu + ((bits >> 20) & 1u);
  int64_t normal = (int64_t)(rounded >> 20) - 960;
  int64_t sub = (int64_t)rintf(mag * 512.0f);
  int64_t code = mag < 0.015625f ? sub : normal;
  if (code < 0) code = 0;
  if (code > 126) code = 126;
  return (uint8_t)code | (uint8_t)((bits >> 24) & 128u);
}

static void lut_init(void) {
  if (g_lut_ready) return;
  for (int i = 0; i < 256; ++i) g_lut[i] = ref_decode_e4m3((uint8_t)i);
  g_lut_ready = 1;
}

static float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

static uint16_t f32_to_bf16(float v) {
  uint32_t b = f2u(v);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

/* activations/fp8/validation.py:27-36 -- one 128-group */
static void quantize_group(const float* x, uint8_t* codes, float* scale) {
  float m = 0.0f;
  for (int j = 0; j < 128; ++j) m = fmaxf(m, fabsf(x[j]));
  float s = fmaxf(m, 1e-12f) / 448.0f;
  for (int j = 0; j < 128; ++j) codes[j] = ref_encode_e4m3(x[j] / s);
  *scale = s;
}

/* bf16 x [rows, k] -> codes, scales */
int ref_quantize_bf16(const uint16_t* x, uint8_t* codes, float* scales, int64_t rows, int64_t k,
                      int threads) {
  if (k % 128) return -1;
  int64_t groups = rows * (k / 128);
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t g = 0; g < groups; ++g) {
    float v[128];
    for (int j = 0; j < 128; ++j) v[j] = bf16_to_f32(x[g * 128 + j]);
    quantize_group(v, codes + g * 128, scales + g);
  }
  return 0;
}

/*
 * fp8 linear on bf16 activations: quantize x per 1x128 group, decode codes
 * and weights, y[m, n] = sum_k xdeq[m, k] * wdeq[n, k] (f32), stored bf16
 * (out_bf16 != 0) or f32.  ws: f32 [ceil(o/128), k/128].
 */
int ref_fp8_linear_bf16(const uint16_t* x, const uint8_t* w, const float* ws, void* out,
                        int out_bf16, int64_t r, int64_t k, int64_t o, int threads) {
  if (k % 128) return -1;
  lut_init();
  const int64_t kb = k / 128;
  float* xd = (float*)malloc(sizeof(float) * r * k);
  uint8_t* codes = (uint8_t*)malloc(r * k);
  float* sc = (float*)malloc(sizeof(float) * r * kb);
  if (!xd || !codes || !sc) return -2;
  ref_quantize_bf16(x, codes, sc, r, k, threads);
  for (int64_t i = 0; i < r * k; ++i) xd[i] = g_lut[codes[i]] * sc[i / 128];
#pragma omp parallel num_threads(threads)
  {
    float* wd = (float*)malloc(sizeof(float) * k);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < o; ++n) {
      const uint8_t* wr = w + n * k;
      const float* srow = ws + (n / 128) * kb;
      for (int64_t j = 0; j < k; ++j) wd[j] = g_lut[wr[j]] * srow[j / 128];
      for (int64_t m = 0; m < r; ++m) {
        const float* xr = xd + m * k;
        float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
        for (int64_t j = 0; j < k; ++j) acc += xr[j] * wd[j];
        if (out_bf16)
          ((uint16_t*)out)[m * o + n] = f32_to_bf16(acc);
        else
          ((float*)out)[m * o + n] = acc;
      }
    }
    free(wd);
  }
  free(xd);
  free(codes);
  free(sc);
  return 0;
}

/* decoded expert weight rows [n0, n1) of one expert: wd[(n - n0) * k + j] */
static void decode_rows(const uint8_t* w, const float* ws, int64_t n0, int64_t n1, int64_t k,
                        float* wd) {
  const int64_t kb = k / 128;
  for (int64_t n = n0; n < n1; ++n)
    for (int64_t j = 0; j < k; ++j)
      wd[(n - n0) * k + j] = g_lut[w[n * k + j]] * ws[(n / 128) * kb + j / 128];
}

/*
 * One routed MoE layer (softmax top-k router, bias 0):
 *   x bf16 [T, H], logits f32 [T, E], w1/w3 [E, F, H], w2 [E, H, F] codes,
 *   s1/s3 f32 [E, F/128, H/128], s2 f32 [E, H/128, F/128] -> out f32 [T, H].
 * Experts are processed in parallel over output columns.
 */
int ref_moe_layer_bf16(const uint16_t* x, const float* logits, const uint8_t* w1, const float* s1,
                       const uint8_t* w3, const float* s3, const uint8_t* w2, const float* s2,
                       float* out, int64_t T, int64_t H, int64_t F, int E, int top,
                       int threads) {
  if (H % 128 || F % 128 || top > 32) return -1;
  lut_init();
  int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * T * top);
  float* prob = (float*)malloc(sizeof(float) * T * top);
  float* xd = (float*)malloc(sizeof(float) * T * H);
  uint8_t* qc = (uint8_t*)malloc(T * H);
  float* qs = (float*)malloc(sizeof(float) * T * (H / 128));
  float* contrib = (float*)calloc((size_t)T * top * H, sizeof(float));
  float* act = (float*)malloc(sizeof(float) * T * top * F);
  if (!ids || !prob || !xd || !qc || !qs || !contrib || !act) return -2;
  /* router: select on logits (bias 0), lowest index on ties; softmax over the
   * selected logits (kernel.py:444-499) */
  for (int64_t t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    float chosen[32];
    unsigned char used[1024] = {0};
    for (int rank = 0; rank < top; ++rank) {
      int best = -1;
      for (int e = 0; e < E; ++e)
        if (!used[e] && (best < 0 || l[e] > l[best])) best = e;
      used[best] = 1;
      ids[t * top + rank] = best;
      chosen[rank] = l[best];
    }
    float peak = chosen[0];
    for (int i = 1; i < top; ++i) peak = fmaxf(peak, chosen[i]);
    float total = 0.0f;
    for (int i = 0; i < top; ++i) total += expf(chosen[i] - peak);
    for (int i = 0; i < top; ++i) prob[t * top + i] = expf(chosen[i] - peak) / total;
  }
  ref_quantize_bf16(x, qc, qs, T, H, threads);
  for (int64_t i = 0; i < T * H; ++i) xd[i] = g_lut[qc[i]] * qs[i / 128];
  /* gate/up + SwiGLU + activation re-quantization, per expert */
  for (int e = 0; e < E; ++e) {
    int64_t n_rows = 0;
    for (int64_t i = 0; i < T * top; ++i) n_rows += ids[i] == e;
    if (!n_rows) continue;
    int64_t* pairs = (int64_t*)malloc(sizeof(int64_t) * n_rows);
    int64_t c = 0;
    for (int64_t i = 0; i < T * top; ++i)
      if (ids[i] == e) pairs[c++] = i;
    const uint8_t* g_w = w1 + (int64_t)e * F * H;
    const uint8_t* u_w = w3 + (int64_t)e * F * H;
    const float* g_s = s1 + (int64_t)e * (F / 128) * (H / 128);
    const float* u_s = s3 + (int64_t)e * (F / 128) * (H / 128);
#pragma omp parallel num_threads(threads)
    {
      float* gd = (float*)malloc(sizeof(float) * 128 * H);
      float* ud = (float*)malloc(sizeof(float) * 128 * H);
#pragma omp for schedule(static)
      for (int64_t fb = 0; fb < F / 128; ++fb) {
        decode_rows(g_w, g_s, fb * 128, fb * 128 + 128, H, gd);
        decode_rows(u_w, u_s, fb * 128, fb * 128 + 128, H, ud);
        for (int64_t p = 0; p < n_rows; ++p) {
          const float* xr = xd + (pairs[p] / top) * H;
          float a[128];
          for (int j = 0; j < 128; ++j) {
            float ga = 0.0f, ua = 0.0f;
#pragma omp simd reduction(+ : ga, ua)
            for (int64_t h = 0; h < H; ++h) {
              ga += xr[h] * gd[j * H + h];
              ua += xr[h] * ud[j * H + h];
            }
            a[j] = ga / (1.0f + expf(-ga)) * ua;
          }
          uint8_t q[128];
          float s;
          quantize_group(a, q, &s);
          float* dst = act + pairs[p] * F + fb * 128;
          for (int j = 0; j < 128; ++j) dst[j] = g_lut[q[j]] * s;
        }
      }
      free(gd);
      free(ud);
    }
    /* down projection */
    const uint8_t* d_w = w2 + (int64_t)e * H * F;
    const float* d_s = s2 + (int64_t)e * (H / 128) * (F / 128);
#pragma omp parallel num_threads(threads)
    {
      float* dd = (float*)malloc(sizeof(float) * 128 * F);
#pragma omp for schedule(static)
      for (int64_t hb = 0; hb < H / 128; ++hb) {
        decode_rows(d_w, d_s, hb * 128, hb * 128 + 128, F, dd);
        for (int64_t p = 0; p < n_rows; ++p) {
          const float* ar = act + pairs[p] * F;
          for (int j = 0; j < 128; ++j) {
            float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
            for (int64_t f = 0; f < F; ++f) acc += ar[f] * dd[j * F + f];
            contrib[pairs[p] * H + hb * 128 + j] = acc;
          }
        }
      }
      free(dd);
    }
    free(pairs);
  }
  /* weighted combine in rank order (kernel.py:248-265) */
  for (int64_t t = 0; t < T; ++t)
    for (int64_t h = 0; h < H; ++h) {
      float acc = 0.0f;
      for (int rank = 0; rank < top; ++rank)
        acc += contrib[(t * top + rank) * H + h] * prob[t * top + rank];
      out[t * H + h] = acc;
    }
  free(ids);
  free(prob);
  free(xd);
  free(qc);
  free(qs);
  free(contrib);
  free(act);
  return 0;
}

/*
 * Check of the device quotient technique (test infrastructure): for n seeded
 * (x, group max) pairs, compare enc(RN(x/s)) with the device formulation
 * r = RN(1/s), q0 = RN(x*r), e = fma(-q0, c, x), q = fma(e, r, q0) with
 * c = s, or 0 where s is inf (a group holding inf, where x / s = 0 for every
 * finite x); libm fmaf is correctly rounded.  Returns the number of code
 * mismatches; also counts quotient mismatches into *quotient_mismatch.
 */
static uint64_t splitmix(uint64_t* s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

int64_t ref_check_exact_quotient(int64_t n, uint64_t seed, int64_t* quotient_mismatch) {
  int64_t bad = 0, qbad = 0;
  uint64_t st = seed;
  for (int64_t i = 0; i < n; ++i) {
    uint64_t a = splitmix(&st), b = splitmix(&st);
    /* bf16-grid group max in a wide exponent range; x bf16 with |x| <= amax */
    uint32_t mb = (uint32_t)((a & 0xFFFF) | 0x3000) << 16;
    mb = (mb & 0x807FFFFFu) | ((uint32_t)(90 + (a >> 16) % 70) << 23);
    float amax = fabsf(u2f(mb));
    float frac = (float)((b >> 11) & 0xFFFFFF) / 16777216.0f;
    float x = (float)(((b >> 40) & 1) ? -1 : 1) * amax * frac;
    x = bf16_to_f32(f32_to_bf16(x));
    if (fabsf(x) > amax) x = copysignf(amax, x);
    /* one sample in 64 as a finite x in a group whose maximum is inf */
    if (((a >> 58) & 63) == 0) amax = INFINITY;
    float s = fmaxf(amax, 1e-12f) / 448.0f;
    float r = 1.0f / s;
    float c = isinf(s) ? 0.0f : s;
    float ax = fabsf(x);
    float q0 = ax * r;
    float e = fmaf(-q0, c, ax);
    float q = fmaf(e, r, q0);
    float exact = ax / s;
    if (q != exact) ++qbad;
    uint8_t c1 = ref_encode_e4m3(x / s);
    uint8_t c2 = ref_encode_e4m3(q) | (uint8_t)((f2u(x) >> 24) & 128u);
    if (c1 != c2) ++bad;
  }
  if (quotient_mismatch) *quotient_mismatch = qbad;
  return bad;
}
