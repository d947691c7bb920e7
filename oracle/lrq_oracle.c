/*
 * lrq_oracle.c -- CPU restatement of the weight-quantization path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this file.  It is the checker that tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg compare the HIP kernels against.
 *
 * What it restates (all citations are into the Lumen-RL reference tree):
 *
 *   lrqo_fp8_block_quant   WeightQuantizer.quantize_tensor,
 *                          lumenrl/quantization/weight_quantizer.py:40-77, in the
 *                          op order of :59-71 (amax -> /448 -> clamp(tiny) ->
 *                          optional pow2 -> x/s -> float8_e4m3fn), applied to
 *                          1xB row blocks (the reference) or to 2-D tiles
 *                          (128x128, same op order).
 *   lrqo_fp8_block_quant_f64  the same on a float64 tensor, every op in
 *                          float64 (:59-71), then the float32 step of :68.
 *   lrqo_pow2_*            _round_scale_pow2, weight_quantizer.py:24-27.
 *   lrqo_fp8_block_dequant WeightQuantizer.dequantize_tensor, :79-89, and the
 *                          bf16 cast of dequantize_state_dict, :133.
 *   lrqo_mx_quant          MXFP8 / MXFP4 (OCP Microscaling v1.0): not present in
 *                          the reference tree (delegated to absent aiter/vLLM
 *                          code, examples/DAPO/atom_aiter_shim/sitecustomize.py:28-32);
 *                          this is the spec's closed form with the conventions
 *                          documented at lrqo_mx_quant.
 *
 * The reference computes with torch on x86 CPUs.  The IEEE-754 results are
 * restated with plain C float arithmetic (gcc, no -ffast-math, no FMA
 * contraction, denormals on).  Where torch's x86 kernels make a choice IEEE
 * leaves open (NaN payloads and signs, NaN in bf16/fp16 casts) the choice is
 * written out explicitly below, as observed from torch 2.10 on x86 (AVX2 and
 * AVX512 kernels agree):
 *   - amax over a block containing any NaN returns the canonical NaN
 *     0x7FC00000 whatever the payloads.
 *   - a division with a NaN operand returns that operand, quieted (first
 *     operand wins when both are NaN); inf/inf and 0/0 return the x86 default
 *     NaN 0xFFC00000 (negative).
 *   - float -> bfloat16 maps every NaN to 0xFFFF, else rounds to nearest even.
 *   - float -> float16 keeps sign and the top payload bits of a NaN, quieted.
 *   - float -> float8_e4m3fn rounds to nearest even, does not saturate: a
 *     magnitude that rounds above 448, inf and NaN all give 0x7F | sign.
 *   - float8_e4m3fn 0x7F / 0xFF decode to 0x7FF00000 / 0xFFF00000.
 * Two torch results depend on whether an element falls in the vectorized body
 * or the scalar tail of torch's loop: bf16 arithmetic on NaN (0xFFFF vs 0x7FC0)
 * and torch.pow(2, NaN) (all-ones vs 0x7FC00000).  The oracle pins the
 * vectorized body, which is what all but the last few blocks of a tensor get.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { LRQO_BF16 = 0, LRQO_F16 = 1, LRQO_F32 = 2 };
enum { LRQO_ARITH_F32 = 0, LRQO_ARITH_NATIVE = 1 };

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline int is_nan_bits(uint32_t u) { return (u & 0x7FFFFFFFu) > 0x7F800000u; }

/* ------------------------------------------------------------------ */
/* 16-bit float formats                                                */
/* ------------------------------------------------------------------ */

float lrqo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* torch x86 vectorized float->bfloat16: NaN -> 0xFFFF, else RNE. */
uint16_t lrqo_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if (is_nan_bits(u)) return 0xFFFFu;
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

float lrqo_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13));
  if (e == 0) {  /* subnormal or zero: m * 2^-24, exact in float */
    float v = (float)m * 0x1p-24f;
    return u2f(f2u(v) | sign);
  }
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* IEEE float -> binary16, round to nearest even, subnormals kept. */
uint16_t lrqo_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
  if (a == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
  float af = u2f(a);
  if (af < 0x1p-14f) {
    /* subnormal range: integer number of 2^-24 units, RNE */
    float t = af * 0x1p24f; /* exact scaling */
    float n = nearbyintf(t);
    return (uint16_t)(sign | (uint16_t)n); /* n == 1024 becomes min normal */
  }
  int32_t e = (int32_t)(a >> 23) - 127; /* >= -14 */
  uint32_t mant = a & 0x7FFFFFu;
  uint32_t keep = mant >> 13, rem = mant & 0x1FFFu;
  uint32_t code = ((uint32_t)(e + 15) << 10) | keep;
  if (rem > 0x1000u || (rem == 0x1000u && (keep & 1u))) code += 1u;
  if (code >= 0x7C00u) code = 0x7C00u; /* overflow to inf */
  return (uint16_t)(sign | code);
}

/* ------------------------------------------------------------------ */
/* 8-bit and 4-bit element formats                                     */
/* ------------------------------------------------------------------ */

/* float8_e4m3fn: bias 7, 3 mantissa bits, no inf, 0x7F/0xFF = NaN, max 448.
 * Round to nearest even, non-saturating. */
uint8_t lrqo_f32_to_e4m3(float f) {
  uint32_t u = f2u(f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7FFFFFFFu;
  if (a >= 0x7F800000u) return (uint8_t)(sign | 0x7Fu); /* inf, NaN */
  float af = u2f(a);
  if (af < 0x1p-6f) {
    /* e4m3 subnormals are multiples of 2^-9 */
    float n = nearbyintf(af * 512.0f); /* exact scaling, RNE */
    return (uint8_t)(sign | (uint8_t)n); /* n == 8 is the min normal 0x08 */
  }
  int32_t e = (int32_t)(a >> 23) - 127; /* >= -6 */
  if (e > 8) return (uint8_t)(sign | 0x7Fu);
  uint32_t mant = a & 0x7FFFFFu;
  uint32_t keep = mant >> 20, rem = mant & 0xFFFFFu;
  uint32_t code = ((uint32_t)(e + 7) << 3) | keep;
  if (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) code += 1u;
  if (code > 0x7Eu) code = 0x7Fu; /* rounds to 480 or above: NaN */
  return (uint8_t)(sign | code);
}

float lrqo_e4m3_to_f32(uint8_t c) {
  uint32_t sign = (uint32_t)(c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xFu, m = c & 7u;
  if (e == 0xF && m == 7) return u2f(sign | 0x7FF00000u);
  if (e == 0) return u2f(f2u((float)m * 0x1p-9f) | sign);
  return u2f(sign | ((e + 120u) << 23) | (m << 20));
}

/* E2M1: bias 1, 1 mantissa bit, magnitudes {0,.5,1,1.5,2,3,4,6}.
 * Round to nearest even, saturate at 6.  Returns the 4-bit code. */
uint8_t lrqo_f32_to_e2m1(float f) {
  uint32_t u = f2u(f);
  uint8_t sign = (uint8_t)((u >> 28) & 0x8u);
  uint32_t a = u & 0x7FFFFFFFu;
  if (a >= 0x7F800000u) return (uint8_t)(sign | 0x7u); /* not reached on the MX path */
  float af = u2f(a);
  if (af < 1.0f) {
    float n = nearbyintf(af * 2.0f); /* multiples of 0.5, RNE; 2 -> 1.0 */
    return (uint8_t)(sign | (uint8_t)n);
  }
  int32_t e = (int32_t)(a >> 23) - 127; /* >= 0 */
  if (e > 2) return (uint8_t)(sign | 0x7u);
  uint32_t mant = a & 0x7FFFFFu;
  uint32_t keep = mant >> 22, rem = mant & 0x3FFFFFu;
  uint32_t code = ((uint32_t)(e + 1) << 1) | keep;
  if (rem > 0x200000u || (rem == 0x200000u && (keep & 1u))) code += 1u;
  if (code > 7u) code = 7u;
  return (uint8_t)(sign | code);
}

float lrqo_e2m1_to_f32(uint8_t c) {
  static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  float v = mag[c & 7u];
  return (c & 8u) ? -v : v;
}

/* ------------------------------------------------------------------ */
/* x86 division as torch sees it                                       */
/* ------------------------------------------------------------------ */

static inline float quiet(float a) { return u2f(f2u(a) | 0x00400000u); }

float lrqo_x86_div(float a, float b) {
  if (isnan(a)) return quiet(a);
  if (isnan(b)) return quiet(b);
  if ((isinf(a) && isinf(b)) || (a == 0.0f && b == 0.0f)) return u2f(0xFFC00000u);
  return a / b;
}

/* ------------------------------------------------------------------ */
/* _round_scale_pow2 (weight_quantizer.py:24-27)                        */
/* ------------------------------------------------------------------ */
/* torch.pow(2, torch.round(torch.log2(s))) for fp32 s >= FLT_MIN.  torch's
 * fp32 log2 on x86 agrees with the correctly rounded log2 at every rounding
 * cut (checked exhaustively against torch in tests/), and torch.round is
 * round-half-even, so the closed form is 2^roundeven(RN_f32(log2 s)).
 * RN_f32(log2 s) is obtained from the double log2 rounded to float. */
float lrqo_pow2_f32(float s) {
  if (isnan(s)) return s;
  if (isinf(s)) return s;
  float l = (float)log2((double)s);
  float r = nearbyintf(l);
  return ldexpf(1.0f, (int)r); /* 2^128 overflows to inf, as torch.pow does */
}

/* bf16 scale: log2 computed in float then rounded to bf16, round, pow. */
uint16_t lrqo_pow2_bf16(uint16_t s) {
  float sf = lrqo_bf16_to_f32(s);
  if (isnan(sf) || isinf(sf)) return s;
  float l = lrqo_bf16_to_f32(lrqo_f32_to_bf16((float)log2((double)sf)));
  float r = nearbyintf(l);
  return lrqo_f32_to_bf16(ldexpf(1.0f, (int)r));
}

uint16_t lrqo_pow2_f16(uint16_t s) {
  float sf = lrqo_f16_to_f32(s);
  if (isnan(sf) || isinf(sf)) return s;
  float l = lrqo_f16_to_f32(lrqo_f32_to_f16((float)log2((double)sf)));
  float r = nearbyintf(l);
  return lrqo_f32_to_f16(ldexpf(1.0f, (int)r));
}

/* ------------------------------------------------------------------ */
/* FP8 blockwise quantization                                           */
/* ------------------------------------------------------------------ */

static inline float load_in(const void* in, int dtype, int64_t idx) {
  switch (dtype) {
    case LRQO_BF16: return lrqo_bf16_to_f32(((const uint16_t*)in)[idx]);
    case LRQO_F16: return lrqo_f16_to_f32(((const uint16_t*)in)[idx]);
    default: return ((const float*)in)[idx];
  }
}

/* Round a float result of the reference's arithmetic to the compute dtype. */
static inline float round_to(int cdt, float v) {
  if (cdt == LRQO_BF16) return lrqo_bf16_to_f32(lrqo_f32_to_bf16(v));
  if (cdt == LRQO_F16) return lrqo_f16_to_f32(lrqo_f32_to_f16(v));
  return v;
}

/* Per-block scale in the compute dtype, as a float value.
 * amax_bits: max of (float bits & 0x7FFFFFFF) over the block. */
static float block_scale(int cdt, uint32_t amax_bits, int pow2) {
  float amax;
  if (amax_bits > 0x7F800000u) {
    /* canonical NaN from amax, in the compute dtype's own encoding */
    amax = u2f(0x7FC00000u);
  } else {
    amax = u2f(amax_bits);
  }
  /* amax / fp8_max  (weight_quantizer.py:61-62), in the compute dtype */
  float s = round_to(cdt, lrqo_x86_div(amax, 448.0f));
  /* clamp(min=finfo(dtype).tiny)  (:63); NaN propagates */
  float tiny = (cdt == LRQO_F16) ? 0x1p-14f : FLT_MIN;
  if (!isnan(s) && s < tiny) s = tiny;
  if (pow2 && isnan(s)) {
    /* torch.pow(2, NaN) in its vectorized x86 loop returns all-ones bits
     * (0xFFFFFFFF / 0xFFFF); its scalar tail loop returns the canonical NaN.
     * The vectorized result is the one pinned here. */
    if (cdt == LRQO_BF16) s = lrqo_bf16_to_f32(0xFFFFu);
    else if (cdt == LRQO_F16) s = lrqo_f16_to_f32(0xFFFFu);
    else s = u2f(0xFFFFFFFFu);
  } else if (pow2) {
    if (cdt == LRQO_BF16) s = lrqo_bf16_to_f32(lrqo_pow2_bf16(lrqo_f32_to_bf16(s)));
    else if (cdt == LRQO_F16) s = lrqo_f16_to_f32(lrqo_pow2_f16(lrqo_f32_to_f16(s)));
    else s = lrqo_pow2_f32(s);
  }
  return s;
}

static inline uint8_t elem_code(int cdt, float x, float s) {
  /* (blocks / expanded) in the compute dtype, .to(float32), .to(e4m3fn)  (:67-71) */
  float q = round_to(cdt, lrqo_x86_div(x, s));
  return lrqo_f32_to_e4m3(q);
}

/*
 * in      : [batch][rows][ld] elements of in_dtype (row r of matrix b at
 *           b*bstride + r*ld); only the first `cols` of each row are read.
 * codes   : [batch][rows][cols] e4m3 bytes.
 * scales  : [batch][ceil(rows/blk_r)][ceil(cols/blk_c)], float32 when the
 *           compute dtype is float32, else 16-bit words of the compute dtype.
 * arith   : LRQO_ARITH_F32 (float32 arithmetic: the reference after the
 *           .to(float32) of quantize_state_dict :109) or LRQO_ARITH_NATIVE
 *           (arithmetic in the input dtype: quantize_tensor called directly on
 *           a bf16/fp16 tensor).
 * Blocks at the right/bottom edge may be partial (amax over the valid part).
 */
int lrqo_fp8_block_quant(const void* in, int in_dtype, int arith, int64_t batch,
                         int64_t rows, int64_t cols, int64_t ld, int64_t bstride,
                         int64_t blk_r, int64_t blk_c, int pow2, uint8_t* codes,
                         void* scales, int nthreads) {
  if (blk_r < 1 || blk_c < 1 || batch < 0 || rows < 0 || cols < 0) return 1;
  int cdt = (arith == LRQO_ARITH_NATIVE) ? in_dtype : LRQO_F32;
  int64_t tr = (rows + blk_r - 1) / blk_r, tc = (cols + blk_c - 1) / blk_c;
  int64_t ntiles = batch * tr * tc;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 16)
#endif
  for (int64_t t = 0; t < ntiles; ++t) {
    int64_t b = t / (tr * tc), rem = t % (tr * tc);
    int64_t r0 = (rem / tc) * blk_r, c0 = (rem % tc) * blk_c;
    int64_t r1 = r0 + blk_r < rows ? r0 + blk_r : rows;
    int64_t c1 = c0 + blk_c < cols ? c0 + blk_c : cols;
    uint32_t amax_bits = 0;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t c = c0; c < c1; ++c) {
        uint32_t a = f2u(load_in(in, in_dtype, b * bstride + r * ld + c)) & 0x7FFFFFFFu;
        if (a > amax_bits) amax_bits = a;
      }
    float s = block_scale(cdt, amax_bits, pow2);
    if (cdt == LRQO_F32) ((float*)scales)[t] = s;
    else if (cdt == LRQO_BF16) ((uint16_t*)scales)[t] = lrqo_f32_to_bf16(s);
    else ((uint16_t*)scales)[t] = lrqo_f32_to_f16(s);
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t c = c0; c < c1; ++c) {
        float x = load_in(in, in_dtype, b * bstride + r * ld + c);
        codes[(b * rows + r) * cols + c] = elem_code(cdt, x, s);
      }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* float64 arithmetic: quantize_tensor on a float64 tensor             */
/* ------------------------------------------------------------------ */
/* weight_quantizer.py:59-71 evaluated in float64, the dtype of the tensor:
 * amax (a NaN anywhere gives the canonical 0x7FF8000000000000), amax / 448.0,
 * clamp(min=finfo(float64).tiny = 2^-1022), optional pow2, x / s in float64,
 * then the explicit .to(float32) of :68 (round to nearest even: a double
 * rounding, f64 quotient -> f32 -> e4m3) and .to(float8_e4m3fn) of :71.
 * torch's x86 NaN choices are the float32 ones (observed with torch 2.10):
 * a division with a NaN operand returns that operand quieted (x's own
 * first), inf/inf is the default NaN 0xFFF8000000000000 (negative), a float64
 * NaN converts to a float32 NaN of the same sign, and torch.pow(2, NaN)
 * returns all-ones bits in the vectorized loop body (pinned here). */
static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

double lrqo_x86_div_f64(double a, double b) {
  if (isnan(a)) return u2d(d2u(a) | 0x0008000000000000ull);
  if (isnan(b)) return u2d(d2u(b) | 0x0008000000000000ull);
  if ((isinf(a) && isinf(b)) || (a == 0.0 && b == 0.0)) return u2d(0xFFF8000000000000ull);
  return a / b;
}

/* _round_scale_pow2 (weight_quantizer.py:24-27) on a float64 scale >= 2^-1022:
 * 2^roundeven(log2 s).  The double log2 here gives the same rounding cut as
 * torch's float64 log2 on every exponent (checked against torch in tests/). */
double lrqo_pow2_f64(double s) {
  if (isnan(s) || isinf(s)) return s;
  double r = nearbyint(log2(s));
  return ldexp(1.0, (int)r); /* 2^1024 overflows to inf, as torch.pow does */
}

int lrqo_fp8_block_quant_f64(const double* in, int64_t batch, int64_t rows, int64_t cols,
                             int64_t ld, int64_t bstride, int64_t blk_r, int64_t blk_c,
                             int pow2, uint8_t* codes, double* scales, int nthreads) {
  if (blk_r < 1 || blk_c < 1 || batch < 0 || rows < 0 || cols < 0) return 1;
  int64_t tr = (rows + blk_r - 1) / blk_r, tc = (cols + blk_c - 1) / blk_c;
  int64_t ntiles = batch * tr * tc;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 16)
#endif
  for (int64_t t = 0; t < ntiles; ++t) {
    int64_t b = t / (tr * tc), rem = t % (tr * tc);
    int64_t r0 = (rem / tc) * blk_r, c0 = (rem % tc) * blk_c;
    int64_t r1 = r0 + blk_r < rows ? r0 + blk_r : rows;
    int64_t c1 = c0 + blk_c < cols ? c0 + blk_c : cols;
    uint64_t amax_bits = 0;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t c = c0; c < c1; ++c) {
        uint64_t a = d2u(in[b * bstride + r * ld + c]) & 0x7FFFFFFFFFFFFFFFull;
        if (a > amax_bits) amax_bits = a;
      }
    double amax = amax_bits > 0x7FF0000000000000ull ? u2d(0x7FF8000000000000ull) : u2d(amax_bits);
    double s = lrqo_x86_div_f64(amax, 448.0);
    if (!isnan(s) && s < DBL_MIN) s = DBL_MIN;
    if (pow2) s = isnan(s) ? u2d(0xFFFFFFFFFFFFFFFFull) : lrqo_pow2_f64(s);
    scales[t] = s;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t c = c0; c < c1; ++c) {
        double x = in[b * bstride + r * ld + c];
        float q = (float)lrqo_x86_div_f64(x, s); /* RNE; a NaN keeps its sign */
        codes[(b * rows + r) * cols + c] = lrqo_f32_to_e4m3(q);
      }
  }
  return 0;
}

void lrqo_pow2_f64_n(const double* in, double* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = lrqo_pow2_f64(in[i]);
}

/* dequantize_tensor (:79-89): fp32(code) * fp32(scale) per block; optional
 * bf16 output (dequantize_state_dict :133).  scale_dtype: LRQO_F32 or
 * LRQO_BF16 (the sidecar of quantize_state_dict :111) or LRQO_F16.
 * out_dtype: LRQO_F32 or LRQO_BF16. */
int lrqo_fp8_block_dequant(const uint8_t* codes, const void* scales, int scale_dtype,
                           int64_t batch, int64_t rows, int64_t cols, int64_t blk_r,
                           int64_t blk_c, void* out, int out_dtype, int nthreads) {
  if (blk_r < 1 || blk_c < 1) return 1;
  int64_t tr = (rows + blk_r - 1) / blk_r, tc = (cols + blk_c - 1) / blk_c;
  int64_t n = batch * rows;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t br = 0; br < n; ++br) {
    int64_t b = br / rows, r = br % rows;
    for (int64_t c = 0; c < cols; ++c) {
      int64_t si = (b * tr + r / blk_r) * tc + c / blk_c;
      float s = load_in(scales, scale_dtype, si);
      float v = lrqo_e4m3_to_f32(codes[br * cols + c]);
      /* torch's vectorized x86 product: a NaN scale wins (quieted), then a
       * NaN code's own NaN; 0 * inf is the default NaN 0xFFC00000. */
      float o;
      if (isnan(s)) o = quiet(s);
      else if (isnan(v)) o = v;
      else if ((v == 0.0f && isinf(s)) || (isinf(v) && s == 0.0f)) o = u2f(0xFFC00000u);
      else o = v * s;
      if (out_dtype == LRQO_BF16) ((uint16_t*)out)[br * cols + c] = lrqo_f32_to_bf16(o);
      else ((float*)out)[br * cols + c] = o;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* MXFP8 / MXFP4 (OCP Microscaling Formats v1.0)                        */
/* ------------------------------------------------------------------ */
/*
 * Per contiguous group of 32 elements along the last dim:
 *   amax      = max |x| (exact);
 *   E8M0      = clamp(floor(log2 amax) - emax_elem + 127, 0, 254), taken from
 *               the float exponent field (emax_elem = 8 for E4M3, 2 for E2M1);
 *               an all-zero or subnormal-amax group clamps to 0 (2^-127);
 *   element   = x * 2^(127 - E8M0) (a power-of-two scaling), then
 *               E4M3: clamp to +-448, round to nearest even;
 *               E2M1: round to nearest even on {0,.5,1,1.5,2,3,4,6}, clamp +-6.
 *   A group whose amax is inf or NaN gets E8M0 = 0xFF (NaN).  Its elements:
 *               E4M3: NaN/inf -> 0x7F|sign, finite -> +-0 (0x00/0x80);
 *               E2M1: every element -> +-0 (0x0/0x8); the NaN scale decodes
 *               the whole group to NaN.
 *   Zero signs are kept (-0 -> 0x80 / 0x8).
 * codes : fmt 8 -> [rows][cols] bytes; fmt 4 -> [rows][cols/2] bytes, element
 *         2i in the low nibble, 2i+1 in the high nibble.
 * scales: [rows][cols/32] E8M0 bytes.
 */
int lrqo_mx_quant(const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t ld,
                  int fmt, uint8_t* codes, uint8_t* scales, int nthreads) {
  if (cols % 32 != 0 || (fmt != 8 && fmt != 4)) return 1;
  int64_t ng = cols / 32;
  int emax = (fmt == 8) ? 8 : 2;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < ng; ++g) {
      float x[32];
      uint32_t amax_bits = 0;
      for (int i = 0; i < 32; ++i) {
        x[i] = load_in(in, in_dtype, r * ld + g * 32 + i);
        uint32_t a = f2u(x[i]) & 0x7FFFFFFFu;
        if (a > amax_bits) amax_bits = a;
      }
      uint8_t* cp = codes + (fmt == 8 ? r * cols + g * 32 : r * (cols / 2) + g * 16);
      if (amax_bits >= 0x7F800000u) {
        scales[r * ng + g] = 0xFFu;
        for (int i = 0; i < 32; ++i) {
          uint32_t u = f2u(x[i]);
          if (fmt == 8) {
            uint8_t sgn = (uint8_t)((u >> 24) & 0x80u);
            cp[i] = ((u & 0x7FFFFFFFu) >= 0x7F800000u) ? (uint8_t)(sgn | 0x7Fu) : sgn;
          } else {
            uint8_t nib = (uint8_t)((u >> 28) & 0x8u);
            if (i & 1) cp[i / 2] |= (uint8_t)(nib << 4);
            else cp[i / 2] = nib;
          }
        }
        continue;
      }
      int32_t e = (int32_t)(amax_bits >> 23) - emax;
      if (e < 0) e = 0;
      scales[r * ng + g] = (uint8_t)e;
      for (int i = 0; i < 32; ++i) {
        float v = ldexpf(x[i], 127 - e);
        if (fmt == 8) {
          if (v > 448.0f) v = 448.0f;
          if (v < -448.0f) v = -448.0f;
          cp[i] = lrqo_f32_to_e4m3(v);
        } else {
          uint8_t nib = lrqo_f32_to_e2m1(v);
          if (i & 1) cp[i / 2] |= (uint8_t)(nib << 4);
          else cp[i / 2] = nib;
        }
      }
    }
  }
  return 0;
}

/* Activation fake-quant of _FP8W8A8Linear.forward
 * (lumenrl/quantization/fp8_rollout.py:53-72): x -> float32, per 1xB block
 * s = clamp(amax/448, tiny) [pow2], x_dq = float32(x/s) * s -- no e4m3 rounding.
 * In x * s (torch's vectorized x86 product) a NaN scale wins, then a NaN x;
 * 0 * inf is the default NaN 0xFFC00000. */
static inline float x86_mul_scale_first(float q, float s) {
  if (isnan(s)) return quiet(s);
  if (isnan(q)) return quiet(q);
  if ((q == 0.0f && isinf(s)) || (isinf(q) && s == 0.0f)) return u2f(0xFFC00000u);
  return q * s;
}

int lrqo_act_qdq(const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t blk, int pow2,
                 float* out, int nthreads) {
  if (blk < 1 || cols % blk != 0) return 1;
  int64_t nb = rows * (cols / blk);
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t b = 0; b < nb; ++b) {
    int64_t base = b * blk;
    uint32_t amax_bits = 0;
    for (int64_t i = 0; i < blk; ++i) {
      uint32_t a = f2u(load_in(in, in_dtype, base + i)) & 0x7FFFFFFFu;
      if (a > amax_bits) amax_bits = a;
    }
    float s = block_scale(LRQO_F32, amax_bits, pow2);
    for (int64_t i = 0; i < blk; ++i) {
      float x = load_in(in, in_dtype, base + i);
      out[base + i] = x86_mul_scale_first(lrqo_x86_div(x, s), s);
    }
  }
  return 0;
}

/* Per-tensor FP8 scale of FP8KVCacheQuantizer.recalibrate_scales
 * (lumenrl/quantization/fp8_kv_cache.py:52-54): w.to(float32).abs().max(),
 * clamp(min=FLT_MIN), then / 448 (division AFTER the clamp, so an all-zero
 * tensor gives the subnormal FLT_MIN/448).  A NaN anywhere gives the canonical
 * quiet NaN 0x7FC00000: torch's multi-threaded CPU reduction over more than
 * 32768 elements, the regime of every q/k/v projection (a single-threaded or
 * smaller reduction gives all-ones instead).  Returns the scale's bit pattern;
 * `in` is `n` contiguous elements. */
uint32_t lrqo_tensor_scale(const void* in, int in_dtype, int64_t n) {
  uint32_t amax_bits = 0;
  for (int64_t i = 0; i < n; ++i) {
    uint32_t a = f2u(load_in(in, in_dtype, i)) & 0x7FFFFFFFu;
    if (a > amax_bits) amax_bits = a;
  }
  if (amax_bits > 0x7F800000u) return 0x7FC00000u;
  float amax = u2f(amax_bits);
  if (amax < 0x1p-126f) amax = 0x1p-126f;
  return f2u(amax / 448.0f);
}

/* Bulk element converters, for exhaustive checks against torch. */
void lrqo_f32_to_e4m3_n(const float* in, uint8_t* out, int64_t n) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t i = 0; i < n; ++i) out[i] = lrqo_f32_to_e4m3(in[i]);
}

void lrqo_f32_to_e4m3_bits_range(uint32_t start, int64_t n, uint8_t* out) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t i = 0; i < n; ++i) out[i] = lrqo_f32_to_e4m3(u2f(start + (uint32_t)i));
}

void lrqo_f32_to_bf16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = lrqo_f32_to_bf16(in[i]);
}

void lrqo_f32_to_f16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = lrqo_f32_to_f16(in[i]);
}

void lrqo_f32_to_e2m1_n(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = lrqo_f32_to_e2m1(in[i]);
}

void lrqo_pow2_f32_n(const float* in, float* out, int64_t n) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t i = 0; i < n; ++i) out[i] = lrqo_pow2_f32(in[i]);
}
