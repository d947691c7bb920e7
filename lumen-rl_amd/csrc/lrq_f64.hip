// FP8 E4M3 blockwise quantization of float64 tensors in float64 arithmetic.
//
// WeightQuantizer.quantize_tensor on a float64 tensor
// (lumenrl/quantization/weight_quantizer.py:40-77) evaluates every op in the
// tensor's dtype: amax, amax / 448 (:61-62), clamp(min = 2^-1022) (:63), the
// optional pow2 rounding (:64-65) and x / s (:67).  The quotient is then
// rounded to float32 (:68) before the e4m3 cast (:71): a double rounding
// (f64 -> f32 -> e4m3) that this kernel keeps.  Scales are written as float64.
//
// k_row_f64 takes dense 1xB blocks (B = 32...512, the reference's layout) with
// 16-byte loads.  Its quotients of finite blocks use one correctly rounded 1/s
// per block and Markstein's correction per element (the IEEE division near
// underflow) and the hardware e4m3 encoder.  k_f64 takes every other shape,
// one wave per block (any block shape), four blocks per 256-thread work-group,
// re-reading the block from L2 for the encode, with the IEEE float64 division
// and the software encoder.
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

// Max over aligned groups of LPB lanes (LPB = 2..64) of 64-bit values.
template <int LPB>
__device__ __forceinline__ uint64_t group_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 1; off < LPB; off <<= 1) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, off, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), off, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    v = v > o ? v : o;
  }
  return v;
}

// The block scale of weight_quantizer.py:60-65 in float64 from the block's
// max |x| bit pattern, and its kind (kScaleExact / kScaleInf / kScaleNaN).
__device__ __forceinline__ void block_scale_f64(uint64_t a, bool pow2, double& s, int& kind) {
  if (a > kInf64) {
    // amax -> canonical NaN; /448 and clamp keep it.  torch.pow(2, NaN)
    // returns all-ones bits in its vectorized x86 loop.
    s = u2d(pow2 ? ~0ull : kNaN64);
    kind = kScaleNaN;
  } else if (a == kInf64) {
    s = u2d(kInf64);
    kind = kScaleInf;
  } else {
    s = u2d(a) / 448.0;                                 // IEEE float64 division
    s = s < 0x1p-1022 ? 0x1p-1022 : s;                  // clamp(min=finfo(float64).tiny)
    if (pow2) s = pow2_f64(s);
    kind = d2u(s) == kInf64 ? kScaleInf : kScaleExact;  // pow2 overflow: every x/inf is +-0
  }
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
  block_scale_f64(a, pow2 != 0, s, kind);
  if (lane == 0) gst<double>(static_cast<double*>(d.scales) + blk, s);

  for (int64_t r = 0; r < nr; ++r)
    for (int64_t c = lane; c < nc; c += 64) {
      const double x = __longlong_as_double(gld<long long>(in + r * d.ld + c));
      gst<uint8_t>(codes + r * d.cols + c, (uint8_t)code_f64(x, s, kind));
    }
}

// 1xB row blocks (B = 32...512) of a dense float64 tensor.  Wave instruction i
// reads 128 consecutive doubles (1 KiB; 16 bytes = 2 doubles per lane), so a
// block spans B/2 lanes of one instruction (B < 128) or B/128 instructions of
// all 64 lanes (B >= 128).  Each wave runs kF64RowInstr instructions; code
// stores are 2 bytes per lane (128 contiguous bytes per wave instruction).
template <int B>
__global__ __launch_bounds__(256) void k_row_f64(Desc single, const Desc* __restrict__ descs,
                                                 const uint32_t* __restrict__ map, int pow2) {
  constexpr int IPB = B >= 128 ? B / 128 : 1;  // instructions per block
  constexpr int LPB = B >= 128 ? 64 : B / 2;   // lanes per block
  constexpr int NI = kF64RowInstr;
  static_assert(NI % IPB == 0, "a wave holds whole blocks");
  Desc d;
  int64_t u;
  pick_desc<kXcdRunRow>(single, descs, map, d, u);
  const int lane = threadIdx.x & 63;
  const int64_t n = d.rows * d.cols;
  const int64_t e0 = (u * 4 + (threadIdx.x >> 6)) * (NI * 128) + 2 * lane;  // first element, instruction 0
  const double* in = static_cast<const double*>(d.in);
  uint64_t x[NI][2];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t e = e0 + i * 128;
    x[i][0] = x[i][1] = 0;
    if (e < n) {
      const v4u v = load_nt(in + e);
      x[i][0] = ((uint64_t)v.y << 32) | v.x;
      x[i][1] = ((uint64_t)v.w << 32) | v.z;
    }
  }
#pragma unroll
  for (int i = 0; i < NI; i += IPB) {
    const int64_t eb = e0 + i * 128;  // this lane's first element of the block's first instruction
    if (eb - 2 * lane >= n) break;     // wave-uniform: past the tensor's end (blocks are whole)
    uint64_t a = 0;
#pragma unroll
    for (int j = i; j < i + IPB; ++j) {
      const uint64_t a0 = x[j][0] & kAbs64, a1 = x[j][1] & kAbs64;
      a = a0 > a ? a0 : a;
      a = a1 > a ? a1 : a;
    }
    a = group_max_u64<LPB>(a);
    double s;
    int kind;
    block_scale_f64(a, pow2 != 0, s, kind);
    // Finite blocks use Markstein's correction of q0 = x * y with y = RN(1/s):
    // q0 is within an ulp of x/s, the residual x - q0 s is then exact, and
    // RN(q0 + residual * y) = RN(x/s).  The residual's last bit is about 2^-104
    // |x|, so it is exact while |x| >= 2^-968; elements below that, or with a
    // quotient below 2^-900, take the IEEE division.
    const bool fast = kind == kScaleExact;
    const double y = fast ? 1.0 / s : 0.0;
    const int64_t blk = eb / B;
    if (lane % LPB == 0 && eb < n) gst<double>(static_cast<double*>(d.scales) + blk, s);
#pragma unroll
    for (int j = i; j < i + IPB; ++j) {
      const int64_t e = e0 + j * 128;
      if (e >= n) continue;
      uint32_t c;
      if (fast) {
        float q[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const double xv = u2d(x[j][k]);
          const double q0 = xv * y;
          double qv;
          if ((__builtin_fabs(xv) >= 0x1p-968 && __builtin_fabs(q0) >= 0x1p-900) || xv == 0.0) {
            const double t = __builtin_fma(q0, s, -xv);
            qv = __builtin_fma(-t, y, q0);  // -(q0 s - x): x = -0 keeps its sign
          } else {
            qv = xv / s;  // a quotient near underflow: the IEEE division
          }
          q[k] = (float)qv;
        }
        c = cvt_e4m3x2<false>(q[0], q[1], 0u) & 0xFFFFu;  // finite |q| <= 448 sqrt 2: the hardware encoder
      } else {
        c = code_f64(u2d(x[j][0]), s, kind) | (code_f64(u2d(x[j][1]), s, kind) << 8);
      }
      gst_nt<uint16_t>(d.codes + e, (uint16_t)c);
    }
  }
}

hipError_t launch_f64(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                      const uint32_t* map, int64_t units, hipStream_t stream) {
  const dim3 grid((unsigned)units), block(256);
  if (cfg.kernel == kKernF64Row) {
    switch (cfg.blk_c) {
      case 32: hipLaunchKernelGGL(k_row_f64<32>, grid, block, 0, stream, single, descs, map, cfg.pow2); break;
      case 64: hipLaunchKernelGGL(k_row_f64<64>, grid, block, 0, stream, single, descs, map, cfg.pow2); break;
      case 128: hipLaunchKernelGGL(k_row_f64<128>, grid, block, 0, stream, single, descs, map, cfg.pow2); break;
      case 256: hipLaunchKernelGGL(k_row_f64<256>, grid, block, 0, stream, single, descs, map, cfg.pow2); break;
      case 512: hipLaunchKernelGGL(k_row_f64<512>, grid, block, 0, stream, single, descs, map, cfg.pow2); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  hipLaunchKernelGGL(k_f64, grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.blk_r, cfg.blk_c);
  return hipGetLastError();
}

}  // namespace lrq
