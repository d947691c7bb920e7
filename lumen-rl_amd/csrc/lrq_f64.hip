// FP8 E4M3 blockwise quantization of float64 tensors in float64 arithmetic.
//
// WeightQuantizer.quantize_tensor on a float64 tensor
// (lumenrl/quantization/weight_quantizer.py:40-77) evaluates every op in the
// tensor's dtype: amax, amax / 448 (:61-62), clamp(min = 2^-1022) (:63), the
// optional pow2 rounding (:64-65) and x / s (:67).  The quotient is then
// rounded to float32 (:68) before the e4m3 cast (:71): a double rounding
// (f64 -> f32 -> e4m3) that this kernel keeps.  Scales are written as float64.
//
// One wave per block (any block shape), four blocks per 256-thread
// work-group, no LDS and no barrier.  Lanes walk each block row with 8-byte
// loads, so a 1x128 block is one contiguous 1 KiB read per wave; the encode
// pass re-reads the block, which the first pass has just brought into L2.
// A rare input (float64 weights), so the path favours exactness over speed:
// IEEE float64 division per element and the software e4m3 encoder.
#include "lrq_device.hpp"
#include "lrq_internal.hpp"

namespace lrq {

namespace {

__device__ __forceinline__ double u2d(uint64_t u) { return __longlong_as_double((long long)u); }
__device__ __forceinline__ uint64_t d2u(double d) { return (uint64_t)__double_as_longlong(d); }

constexpr uint64_t kAbs64 = 0x7FFFFFFFFFFFFFFFull;
constexpr uint64_t kInf64 = 0x7FF0000000000000ull;
constexpr uint64_t kNaN64 = 0x7FF8000000000000ull;  // torch's amax of a block holding a NaN

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, off, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), off, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    v = v > o ? v : o;
  }
  return v;
}

// 2^round(log2 s) for a normal float64 s, as torch.log2 / round / pow give it
// on float64 (weight_quantizer.py:24-27): the rounding cut of each exponent is
// tabulated in lrq_pow2_tables.h.
__device__ __forceinline__ double pow2_f64(double s) {
  const uint64_t b = d2u(s), e = b >> 52, m = b & 0xFFFFFFFFFFFFFull;
  const uint64_t up = m >= kPow2CutF64[e - 1] ? 1u : 0u;
  return u2d((e + up) << 52);  // e + up == 2047 gives +inf, as torch.pow(2, 1024.)
}

// e4m3 byte of x / s for one element (x86 torch semantics; see block_scale's kinds).
__device__ __forceinline__ uint32_t code_f64(double x, double s, int kind) {
  const uint64_t ux = d2u(x);
  const uint32_t sx = (uint32_t)(ux >> 56) & 0x80u;
  const bool xnan = (ux & kAbs64) > kInf64, xinf = (ux & kAbs64) == kInf64;
  if (kind == kScaleNaN) return 0x7Fu | (xnan ? sx : ((uint32_t)(d2u(s) >> 56) & 0x80u));
  if (kind == kScaleInf) {
    if (xnan) return 0x7Fu | sx;  // x / inf keeps x's NaN
    if (xinf) return 0xFFu;       // inf / inf: the default NaN, negative
    return sx;                    // finite / inf = +-0
  }
  return sw_e4m3((float)(x / s));  // IEEE float64 quotient, RNE to float32, RNE to e4m3
}

}  // namespace

__global__ __launch_bounds__(256) void k_f64(Desc single, const Desc* __restrict__ descs,
                                             const uint32_t* __restrict__ map, int pow2,
                                             int blk_r, int blk_c) {
  Desc d;
  int64_t u;
  pick_desc<kXcdRunStream>(single, descs, map, d, u);
  const int lane = threadIdx.x & 63;
  const int64_t per = d.units_r * d.units_c;
  const int64_t blk = 4 * u + (threadIdx.x >> 6);
  if (blk >= d.batch * per) return;  // the tensor's last work-group may hold fewer blocks
  const int64_t b = blk / per;
  const int64_t rem = blk - b * per;
  const int64_t tr = rem / d.units_c, tc = rem - tr * d.units_c;
  const int64_t r0 = tr * blk_r, c0 = tc * blk_c;
  const int64_t nr = r0 + blk_r <= d.rows ? blk_r : d.rows - r0;
  const int64_t nc = c0 + blk_c <= d.cols ? blk_c : d.cols - c0;
  const double* in = static_cast<const double*>(d.in) + b * d.bstride + r0 * d.ld + c0;
  uint8_t* codes = d.codes + (b * d.rows + r0) * d.cols + c0;

  uint64_t a = 0;
  for (int64_t r = 0; r < nr; ++r)
    for (int64_t c = lane; c < nc; c += 64) {
      const uint64_t v = (uint64_t)gld<long long>(in + r * d.ld + c) & kAbs64;
      a = v > a ? v : a;
    }
  a = wave_max_u64(a);  // every lane holds the block amax

  double s;
  int kind;
  if (a > kInf64) {
    // amax -> canonical NaN; /448 and clamp keep it.  torch.pow(2, NaN)
    // returns all-ones bits in its vectorized x86 loop.
    s = u2d(pow2 ? ~0ull : kNaN64);
    kind = kScaleNaN;
  } else if (a == kInf64) {
    s = u2d(kInf64);
    kind = kScaleInf;
  } else {
    s = u2d(a) / 448.0;                                    // IEEE float64 division
    s = s < 0x1p-1022 ? 0x1p-1022 : s;                     // clamp(min=finfo(float64).tiny)
    if (pow2) s = pow2_f64(s);
    kind = d2u(s) == kInf64 ? kScaleInf : kScaleExact;     // pow2 overflow: every x/inf is +-0
  }
  if (lane == 0) gst<double>(static_cast<double*>(d.scales) + blk, s);

  for (int64_t r = 0; r < nr; ++r)
    for (int64_t c = lane; c < nc; c += 64) {
      const double x = __longlong_as_double(gld<long long>(in + r * d.ld + c));
      gst<uint8_t>(codes + r * d.cols + c, (uint8_t)code_f64(x, s, kind));
    }
}

hipError_t launch_f64(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                      const uint32_t* map, int64_t units, hipStream_t stream) {
  hipLaunchKernelGGL(k_f64, dim3((unsigned)units), dim3(256), 0, stream, single, descs, map, cfg.pow2,
                     cfg.blk_r, cfg.blk_c);
  return hipGetLastError();
}

}  // namespace lrq
