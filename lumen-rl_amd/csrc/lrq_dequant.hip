// FP8 E4M3 block dequantization and device diagnostics.
//
// Dequant restates WeightQuantizer.dequantize_tensor
// (lumenrl/quantization/weight_quantizer.py:79-89): fp32(code) * fp32(scale)
// per block, and optionally the bf16 cast of dequantize_state_dict (:133).
// NaN results follow torch's vectorized x86 product: a NaN scale propagates
// quieted (also over a NaN code); else a NaN code's 0x7FF00000|sign; 0 * inf is
// the default NaN 0xFFC00000; bf16 output maps every NaN to 0xFFFF.
#include "lrq_device.hpp"
#include "lrq_internal.hpp"

namespace lrq {

__device__ __forceinline__ float e4m3_decode(uint32_t c) {
  const uint32_t s = (c & 0x80u) << 24, e = (c >> 3) & 0xFu, m = c & 7u;
  float v = e ? u2f(((e + 120u) << 23) | (m << 20)) : (float)m * 0x1p-9f;
  if (e == 0xFu && m == 7u) v = u2f(0x7FF00000u);
  return u2f(f2u(v) | s);
}

__device__ __forceinline__ float x86_mul(float v, float s) {
  const uint32_t av = f2u(v) & 0x7FFFFFFFu, as = f2u(s) & 0x7FFFFFFFu;
  if (as > 0x7F800000u) return u2f(f2u(s) | 0x00400000u);
  if (av > 0x7F800000u) return v;
  if ((av == 0u && as == 0x7F800000u) || (as == 0u && av == 0x7F800000u)) return u2f(0xFFC00000u);
  return v * s;
}

template <int SDT, int ODT>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ codes,
                                                 const void* __restrict__ scales, int64_t batch,
                                                 int64_t rows, int64_t cols, int blk_r, int blk_c,
                                                 void* __restrict__ out) {
  const int64_t tr = (rows + blk_r - 1) / blk_r, tc = (cols + blk_c - 1) / blk_c;
  const int64_t n = batch * rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t br = i / cols, c = i - br * cols;
    const int64_t b = br / rows, r = br - b * rows;
    const int64_t si = (b * tr + r / blk_r) * tc + c / blk_c;
    float s;
    if constexpr (SDT == kF32) s = static_cast<const float*>(scales)[si];
    else if constexpr (SDT == kBF16) s = u2f((uint32_t)static_cast<const uint16_t*>(scales)[si] << 16);
    else s = f16_to_f32(static_cast<const uint16_t*>(scales)[si]);
    const float o = x86_mul(e4m3_decode(codes[i]), s);
    if constexpr (ODT == kF32) static_cast<float*>(out)[i] = o;
    else static_cast<uint16_t*>(out)[i] = (uint16_t)bf16_bits(o);
  }
}

hipError_t launch_dequant(const uint8_t* codes, const void* scales, int scale_dtype,
                          int64_t batch, int64_t rows, int64_t cols, int blk_r, int blk_c,
                          void* out, int out_dtype, hipStream_t stream) {
  const int64_t n = batch * rows * cols;
  int64_t g = (n + 255) / 256;
  if (g > 65536 * 4) g = 65536 * 4;
  if (g < 1) g = 1;
  const dim3 grid((unsigned)g), block(256);
#define LRQ_DQ(S, O) hipLaunchKernelGGL((k_dequant<S, O>), grid, block, 0, stream, codes, scales, batch, rows, cols, blk_r, blk_c, out)
  if (out_dtype == kF32) {
    if (scale_dtype == kF32) LRQ_DQ(kF32, kF32);
    else if (scale_dtype == kBF16) LRQ_DQ(kBF16, kF32);
    else LRQ_DQ(kF16, kF32);
  } else {
    if (scale_dtype == kF32) LRQ_DQ(kF32, kBF16);
    else if (scale_dtype == kBF16) LRQ_DQ(kBF16, kBF16);
    else LRQ_DQ(kF16, kBF16);
  }
#undef LRQ_DQ
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// diagnostics: the element encoders on raw inputs, for exhaustive checks
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_diag_e4m3_bits(uint32_t start, int64_t n, uint8_t* out) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  const uint32_t b = start + (uint32_t)i;
  // n is a multiple of 4 (checked by the host): 4 encodes -> one dword
  const uint32_t w = cvt_e4m3x4(u2f(b), u2f(b + 1u), u2f(b + 2u), u2f(b + 3u));
  *reinterpret_cast<uint32_t*>(out + i) = w;
}

hipError_t launch_diag_e4m3_bits(uint32_t start, int64_t n, uint8_t* out, hipStream_t stream) {
  const int64_t g = (n / 4 + 255) / 256;
  hipLaunchKernelGGL(k_diag_e4m3_bits, dim3((unsigned)g), dim3(256), 0, stream, start, n, out);
  return hipGetLastError();
}

}  // namespace lrq
