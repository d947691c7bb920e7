// Unscaled cast to float8_e4m3fn: torch's `tensor.to(torch.float8_e4m3fn)`,
// the FP8 path of DynamicWeightLoader
// (lumenrl/engine/inference/weight_loader.py:19-43), over a whole state dict
// in one grouped launch.
//
// Element rule (torch on x86): widen to float32 (exact for bf16/fp16), round
// to nearest even onto e4m3fn; |x| that rounds past 448, +-inf and NaN give
// NaN = 0x7F | sign.  gfx950's v_cvt_pk_fp8_f32 matches it on every non-NaN
// float32 (checked exhaustively); on NaN it writes 0xFF whatever the sign, so a
// chunk holding a NaN takes the software encoder.
//
// A work-group converts one unit of kCastUnit elements of one tensor: 16
// elements per lane in 16-byte nontemporal loads, lane-interleaved so every
// wave instruction reads one contiguous span and writes whole code lines.
// The 16-byte loads take any element-aligned input; tensors whose codes are
// not aligned to one chunk of codes (8 bytes for 16-bit inputs, 4 for
// float32) take an element-wise walk of the same unit; the last n % (elements per load) of a
// tensor are converted element-wise by the unit that holds them.
#include <string.h>

#include "lrq.h"
#include "lrq_device.hpp"
#include "lrq_internal.hpp"

namespace lrq {

template <int DT>
__device__ __forceinline__ float cast_elem(const void* base, int64_t i) {
  if constexpr (DT == kF32) return gld<float>(static_cast<const float*>(base) + i);
  else if constexpr (DT == kBF16) return u2f((uint32_t)gld<uint16_t>(static_cast<const uint16_t*>(base) + i) << 16);
  else return f16_to_f32(gld<uint16_t>(static_cast<const uint16_t*>(base) + i));
}

// Four floats -> four e4m3fn bytes (element 0 in the low byte), torch's rule.
__device__ __forceinline__ uint32_t cast4(float a, float b, float c, float d) {
  const bool nan = (a != a) | (b != b) | (c != c) | (d != d);
  if (__builtin_expect(nan, 0))
    return sw_e4m3(a) | (sw_e4m3(b) << 8) | (sw_e4m3(c) << 16) | (sw_e4m3(d) << 24);
  return cvt_e4m3x4(a, b, c, d);
}

template <int DT>
__global__ __launch_bounds__(256) void k_cast_e4m3(Desc single, const Desc* __restrict__ descs,
                                                   const uint32_t* __restrict__ map) {
  constexpr int EPL = DT == kF32 ? 4 : 8;   // elements per 16-byte load
  constexpr int NL = kCastLaneElems / EPL;  // loads per lane
  Desc d;
  int64_t u;
  pick_desc<kXcdRunStream>(single, descs, map, d, u);
  const int64_t n = d.cols;
  const int64_t base = u * kCastUnit;
  const int tid = threadIdx.x;
  uint8_t* out = d.codes;
  if (d.units_c) {  // aligned: chunk j of lane tid starts at base + (256 j + tid) EPL
    v4u v[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int64_t e = base + (int64_t)(256 * j + tid) * EPL;
      v[j] = e + EPL <= n ? load_nt(static_cast<const char*>(d.in) + e * (DT == kF32 ? 4 : 2))
                          : v4u{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int64_t e = base + (int64_t)(256 * j + tid) * EPL;
      if (e + EPL > n) continue;
      if constexpr (DT == kF32) {
        store_nt(out + e, cast4(u2f(v[j].x), u2f(v[j].y), u2f(v[j].z), u2f(v[j].w)));
      } else {
        const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        float f[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if constexpr (DT == kBF16) {
            f[2 * k] = bf16_lo(w[k]);
            f[2 * k + 1] = bf16_hi(w[k]);
          } else {
            f[2 * k] = f16_to_f32(w[k] & 0xFFFFu);
            f[2 * k + 1] = f16_to_f32(w[k] >> 16);
          }
        }
        store_nt(out + e, v2u{cast4(f[0], f[1], f[2], f[3]), cast4(f[4], f[5], f[6], f[7])});
      }
    }
    const int64_t nfull = n - n % EPL;  // tail: fewer than EPL elements
    if (nfull < n && nfull >= base && nfull < base + kCastUnit && tid < n - nfull) {
      const float x = cast_elem<DT>(d.in, nfull + tid);
      gst<uint8_t>(out + nfull + tid, (uint8_t)(x != x ? sw_e4m3(x) : (cvt_e4m3x2<false>(x, 0.0f, 0u) & 0xFFu)));
    }
  } else {  // misaligned: element-wise walk of the unit
    const int64_t end = base + kCastUnit < n ? base + kCastUnit : n;
    for (int64_t i = base + tid; i < end; i += 256) {
      const float x = cast_elem<DT>(d.in, i);
      gst<uint8_t>(out + i, (uint8_t)(x != x ? sw_e4m3(x) : (cvt_e4m3x2<false>(x, 0.0f, 0u) & 0xFFu)));
    }
  }
}

hipError_t launch_cast(int dtype, const Desc& single, const Desc* descs, const uint32_t* map,
                       int64_t units, hipStream_t stream) {
  const dim3 grid((unsigned)units), block(256);
  switch (dtype) {
    case kBF16: hipLaunchKernelGGL(k_cast_e4m3<kBF16>, grid, block, 0, stream, single, descs, map); break;
    case kF16: hipLaunchKernelGGL(k_cast_e4m3<kF16>, grid, block, 0, stream, single, descs, map); break;
    case kF32: hipLaunchKernelGGL(k_cast_e4m3<kF32>, grid, block, 0, stream, single, descs, map); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace lrq
