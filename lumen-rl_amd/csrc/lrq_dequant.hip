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

template <int SDT>
__device__ __forceinline__ float load_scale(const void* scales, int64_t i) {
  if constexpr (SDT == kF32) return gld<float>(static_cast<const float*>(scales) + i);
  else if constexpr (SDT == kBF16) return u2f((uint32_t)gld<uint16_t>(static_cast<const uint16_t*>(scales) + i) << 16);
  else return f16_to_f32(gld<uint16_t>(static_cast<const uint16_t*>(scales) + i));
}

// Scale index of element (b, r, c) of a [batch, rows, cols] tensor.
__device__ __forceinline__ int64_t scale_index(const Desc& d, int64_t e, int blk_r, int blk_c) {
  const int64_t br = e / d.cols, c = e - br * d.cols;
  const int64_t b = br / d.rows, r = br - b * d.rows;
  return (b * d.units_r + r / blk_r) * d.units_c + c / blk_c;
}

// Generic: one element per thread, any shape and alignment.
template <int SDT, int ODT>
__global__ __launch_bounds__(256) void k_dequant_generic(Desc single, const Desc* __restrict__ descs,
                                                         const uint32_t* __restrict__ map, int blk_r,
                                                         int blk_c) {
  Desc d;
  int64_t u;
  pick_desc<kXcdRunStream>(single, descs, map, d, u);
  const int64_t i = u * 256 + threadIdx.x;
  if (i >= d.nblocks) return;
  const uint8_t* codes = static_cast<const uint8_t*>(d.in);
  const float o = x86_mul(e4m3_decode(gld<uint8_t>(codes + i)), load_scale<SDT>(d.scales, scale_index(d, i, blk_r, blk_c)));
  if constexpr (ODT == kF32) gst<float>(reinterpret_cast<float*>(d.codes) + i, o);
  else gst<uint16_t>(reinterpret_cast<uint16_t*>(d.codes) + i, (uint16_t)bf16_bits(o));
}

// Vectorized: a lane-chunk is CPC codes (8 for bf16 output, 4 for fp32) whose
// output is exactly one 16-byte store, so every wave load and store
// instruction covers one contiguous span (512 B / 256 B of codes, 1 KiB out);
// kDequantChunks chunks per lane, all loaded before the first store (codes at
// any byte alignment).  A chunk lies inside one block (blk_c and cols
// multiples of CPC), so its scale is uniform: when the scale is finite
// and non-zero and no code is NaN the chunk takes the hardware path
// (v_cvt_pk_f32_fp8 -> multiply -> v_cvt_pk_bf16_f32); anything else takes the
// explicit x86 rules.  ROWS1: 1xB blocks over dense rows (scale = element / blk_c).
__device__ __forceinline__ bool word_has_nan_code(uint32_t w) {
  // byte c has (c & 0x7F) == 0x7F  <=>  adding 1 to its low 7 bits carries into bit 7
  return (((w & 0x7F7F7F7Fu) + 0x01010101u) & 0x80808080u) != 0u;
}

template <int SDT, int ODT, bool ROWS1, int CPC>
__global__ __launch_bounds__(256) void k_dequant(Desc single, const Desc* __restrict__ descs,
                                                 const uint32_t* __restrict__ map, int blk_r, int blk_c) {
  // CPC codes per lane-chunk: 8 (bf16 out, one 16-byte store) or 4 (float32
  // out, one 16-byte store; bf16 out for widths 8 does not divide, 8 bytes)
  constexpr int NW = CPC / 4;                // code words per chunk
  constexpr int NCH = kDequantChunks;        // chunks per lane
  Desc d;
  int64_t u;
  pick_desc<kXcdRunStream>(single, descs, map, d, u);
  const int tid = threadIdx.x;
  const uint8_t* codes = static_cast<const uint8_t*>(d.in);
  uint32_t cw[NCH][NW];
  float sc[NCH];
  bool ok[NCH];
  int64_t at[NCH];  // chunks past the end re-read the last one: no branch around loads
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t ch = u * (256 * NCH) + j * 256 + tid;
    ok[j] = ch < d.nblocks;
    at[j] = ok[j] ? ch : d.nblocks - 1;
  }
#pragma unroll
  for (int j = 0; j < NCH; ++j) {  // every code load first, then the scales
    if constexpr (NW == 2) {
      const v2u v = load_nt8(codes + at[j] * CPC);
      cw[j][0] = v.x;
      cw[j][1] = v.y;
    } else {
      cw[j][0] = load_nt4(codes + at[j] * CPC);
    }
  }
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t si = ROWS1 ? (at[j] * CPC) / blk_c : scale_index(d, at[j] * CPC, blk_r, blk_c);
    sc[j] = load_scale<SDT>(d.scales, si);
  }
  v4u val[NCH];  // every chunk decoded before the first store (bf16 x 4: .x, .y)
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const float s = sc[j];
    const uint32_t as = f2u(s) & 0x7FFFFFFFu;
    bool nan_code = false;
#pragma unroll
    for (int q = 0; q < NW; ++q) nan_code |= word_has_nan_code(cw[j][q]);
    float o[CPC];
    const bool fast = as < 0x7F800000u && as != 0u && !nan_code;
    if (fast) {
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        const f32x2 lo = e4m3x2_to_f32<false>(cw[j][q]), hi = e4m3x2_to_f32<true>(cw[j][q]);
        o[4 * q + 0] = lo.x * s;
        o[4 * q + 1] = lo.y * s;
        o[4 * q + 2] = hi.x * s;
        o[4 * q + 3] = hi.y * s;
      }
    } else {
#pragma unroll
      for (int k = 0; k < CPC; ++k) o[k] = x86_mul(e4m3_decode((cw[j][k >> 2] >> (8 * (k & 3))) & 0xFFu), s);
    }
    if constexpr (ODT == kBF16) {
      uint32_t w[CPC / 2];
#pragma unroll
      for (int k = 0; k < CPC / 2; ++k)
        w[k] = fast ? bf16x2_bits(o[2 * k], o[2 * k + 1]) : bf16_bits(o[2 * k]) | (bf16_bits(o[2 * k + 1]) << 16);
      if constexpr (CPC == 8) val[j] = {w[0], w[1], w[2], w[3]};
      else val[j] = {w[0], w[1], 0u, 0u};
    } else {
      val[j] = {f2u(o[0]), f2u(o[1]), f2u(o[2]), f2u(o[3])};
    }
  }
  uint8_t* out = static_cast<uint8_t*>(d.codes);
  constexpr int OB = CPC * (ODT == kBF16 ? 2 : 4);  // output bytes per chunk: 16, or 8 (bf16 x 4)
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    if (!ok[j]) continue;
    if constexpr (OB == 16) gst_nt<v4u>(out + at[j] * OB, val[j]);
    else store_nt(out + at[j] * OB, v2u{val[j].x, val[j].y});
  }
}

template <int SDT, int ODT>
static hipError_t launch_dq(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                            const uint32_t* map, int64_t units, hipStream_t stream) {
  const dim3 grid((unsigned)units), block(256);
  const bool rows1 = cfg.blk_r == 1 && (map != nullptr ? cfg.rows_dense : (single.cols % cfg.blk_c == 0));
  constexpr int C0 = ODT == kBF16 ? 8 : 4;  // the chunk of full 16-byte stores
  if (cfg.kernel == kKernDequant && cfg.chunk == C0 && rows1)
    hipLaunchKernelGGL((k_dequant<SDT, ODT, true, C0>), grid, block, 0, stream, single, descs, map, cfg.blk_r, cfg.blk_c);
  else if (cfg.kernel == kKernDequant && cfg.chunk == C0)
    hipLaunchKernelGGL((k_dequant<SDT, ODT, false, C0>), grid, block, 0, stream, single, descs, map, cfg.blk_r, cfg.blk_c);
  else if (ODT == kBF16 && cfg.kernel == kKernDequant && rows1)
    hipLaunchKernelGGL((k_dequant<SDT, ODT, true, 4>), grid, block, 0, stream, single, descs, map, cfg.blk_r, cfg.blk_c);
  else if (ODT == kBF16 && cfg.kernel == kKernDequant)
    hipLaunchKernelGGL((k_dequant<SDT, ODT, false, 4>), grid, block, 0, stream, single, descs, map, cfg.blk_r, cfg.blk_c);
  else
    hipLaunchKernelGGL((k_dequant_generic<SDT, ODT>), grid, block, 0, stream, single, descs, map, cfg.blk_r, cfg.blk_c);
  return hipGetLastError();
}

hipError_t launch_dequant(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                          const uint32_t* map, int64_t units, hipStream_t stream) {
  const bool f32 = cfg.out_dtype == kF32;
  switch (cfg.in_dtype) {
    case kF32: return f32 ? launch_dq<kF32, kF32>(cfg, single, descs, map, units, stream)
                          : launch_dq<kF32, kBF16>(cfg, single, descs, map, units, stream);
    case kBF16: return f32 ? launch_dq<kBF16, kF32>(cfg, single, descs, map, units, stream)
                           : launch_dq<kBF16, kBF16>(cfg, single, descs, map, units, stream);
    case kF16: return f32 ? launch_dq<kF16, kF32>(cfg, single, descs, map, units, stream)
                          : launch_dq<kF16, kBF16>(cfg, single, descs, map, units, stream);
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// MX dequantization (OCP MX v1.0): element * 2^(E-127) per 1x32 group, E8M0
// 0xFF = NaN, in float32 as torch evaluates codes.float() * scales.float()
// (float8_e8m0fnu: E = 0 is the subnormal 2^-127, 0xFF the signalling NaN
// 0x7F800001).  Vectorized x86 body, code first: a NaN e4m3 code keeps its
// 0x7FF00000 | sign; otherwise a NaN scale propagates quieted.  Every other
// product is exact -- four significant bits times a power of two, 2^-136 at
// the smallest -- except 448 * 2^127 and above, which overflow to inf.
// A lane-chunk is CPC elements (8 for bf16 output, 4 for fp32) whose output is
// one 16-byte store; cols % 32 == 0 puts every chunk inside one group.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  return e == 0xFFu ? u2f(0x7F800001u) : e == 0u ? u2f(0x00400000u) : u2f(e << 23);
}

__device__ __forceinline__ float mx_mul(float v, float s) {
  if ((f2u(v) & 0x7FFFFFFFu) > 0x7F800000u) return v;
  if ((f2u(s) & 0x7FFFFFFFu) > 0x7F800000u) return u2f(f2u(s) | 0x00400000u);
  return v * s;
}

// E2M1 nibble -> float: {0, 0.5, 1, 1.5, 2, 3, 4, 6} with the sign bit.
__device__ __forceinline__ float e2m1_decode(uint32_t n) {
  const uint32_t e = (n >> 1) & 3u, m = n & 1u;
  const uint32_t b = e ? ((126u + e) << 23) | (m << 22) : (m ? 0x3F000000u : 0u);
  return u2f(b | ((n & 8u) << 28));
}

template <int FMT, int ODT>
__global__ __launch_bounds__(256) void k_mx_dequant(Desc single, const Desc* __restrict__ descs,
                                                    const uint32_t* __restrict__ map) {
  constexpr int CPC = ODT == kBF16 ? 8 : 4;      // elements per lane-chunk
  constexpr int CB = FMT == 8 ? CPC : CPC / 2;   // code bytes per lane-chunk
  constexpr int NCH = kDequantChunks;
  Desc d;
  int64_t u;
  pick_desc<kXcdRunStream>(single, descs, map, d, u);
  const int tid = threadIdx.x;
  const uint8_t* codes = static_cast<const uint8_t*>(d.in);
  const uint8_t* sc = static_cast<const uint8_t*>(d.scales);
  uint32_t cw[NCH][2];
  uint32_t ex[NCH];
  bool ok[NCH];
  int64_t at[NCH];  // chunks past the end re-read the last one: no branch around loads
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t ch = u * (256 * NCH) + j * 256 + tid;
    ok[j] = ch < d.nblocks;
    at[j] = ok[j] ? ch : d.nblocks - 1;
  }
#pragma unroll
  for (int j = 0; j < NCH; ++j) {  // every code load first, then the scale bytes
    const uint8_t* p = codes + at[j] * CB;
    if constexpr (CB == 8) {
      const v2u v = load_nt8(p);
      cw[j][0] = v.x;
      cw[j][1] = v.y;
    } else if constexpr (CB == 4) {
      cw[j][0] = load_nt4(p);
    } else {
      cw[j][0] = load_nt2(p);
    }
  }
#pragma unroll
  for (int j = 0; j < NCH; ++j) ex[j] = gld<uint8_t>(sc + ((at[j] * CPC) >> 5));
  v4u val[NCH];  // every chunk decoded before the first store
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const float s = e8m0_to_f32(ex[j]);
    float o[CPC];
    bool fast = ex[j] != 0xFFu;
    if constexpr (FMT == 8) {
#pragma unroll
      for (int q = 0; q < CPC / 4; ++q) fast = fast && !word_has_nan_code(cw[j][q]);
      if (fast) {
#pragma unroll
        for (int q = 0; q < CPC / 4; ++q) {
          const f32x2 lo = e4m3x2_to_f32<false>(cw[j][q]), hi = e4m3x2_to_f32<true>(cw[j][q]);
          o[4 * q + 0] = lo.x * s;
          o[4 * q + 1] = lo.y * s;
          o[4 * q + 2] = hi.x * s;
          o[4 * q + 3] = hi.y * s;
        }
      } else {
#pragma unroll
        for (int k = 0; k < CPC; ++k) o[k] = mx_mul(e4m3_decode((cw[j][k >> 2] >> (8 * (k & 3))) & 0xFFu), s);
      }
    } else {
#pragma unroll
      for (int k = 0; k < CPC; ++k) {
        const float v = e2m1_decode((cw[j][0] >> (4 * k)) & 0xFu);  // element 2i: low nibble
        o[k] = fast ? v * s : mx_mul(v, s);
      }
    }
    if constexpr (ODT == kBF16) {
      uint32_t w[CPC / 2];
#pragma unroll
      for (int k = 0; k < CPC / 2; ++k)
        w[k] = fast ? bf16x2_bits(o[2 * k], o[2 * k + 1]) : bf16_bits(o[2 * k]) | (bf16_bits(o[2 * k + 1]) << 16);
      if constexpr (CPC == 8) val[j] = {w[0], w[1], w[2], w[3]};
      else val[j] = {w[0], w[1], 0u, 0u};
    } else {
      val[j] = {f2u(o[0]), f2u(o[1]), f2u(o[2]), f2u(o[3])};
    }
  }
  uint8_t* out = static_cast<uint8_t*>(d.codes);
  constexpr int OB = CPC * (ODT == kBF16 ? 2 : 4);  // output bytes per chunk: 16, or 8 (bf16 x 4)
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    if (!ok[j]) continue;
    if constexpr (OB == 16) gst_nt<v4u>(out + at[j] * OB, val[j]);
    else store_nt(out + at[j] * OB, v2u{val[j].x, val[j].y});
  }
}

hipError_t launch_mx_dequant(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                             const uint32_t* map, int64_t units, hipStream_t stream) {
  const dim3 grid((unsigned)units), block(256);
  const bool f32 = cfg.out_dtype == kF32;
  if (cfg.mx_fmt == 8) {
    if (f32) hipLaunchKernelGGL((k_mx_dequant<8, kF32>), grid, block, 0, stream, single, descs, map);
    else hipLaunchKernelGGL((k_mx_dequant<8, kBF16>), grid, block, 0, stream, single, descs, map);
  } else if (cfg.mx_fmt == 4) {
    if (f32) hipLaunchKernelGGL((k_mx_dequant<4, kF32>), grid, block, 0, stream, single, descs, map);
    else hipLaunchKernelGGL((k_mx_dequant<4, kBF16>), grid, block, 0, stream, single, descs, map);
  } else {
    return hipErrorInvalidValue;
  }
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

__global__ __launch_bounds__(256) void k_diag_bf16_bits(uint32_t start, int64_t n, uint16_t* out) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 2;
  if (i >= n) return;
  const uint32_t b = start + (uint32_t)i;
  *reinterpret_cast<uint32_t*>(out + i) = bf16x2_bits(u2f(b), u2f(b + 1u));
}

hipError_t launch_diag_bf16_bits(uint32_t start, int64_t n, uint16_t* out, hipStream_t stream) {
  const int64_t g = (n / 2 + 255) / 256;
  hipLaunchKernelGGL(k_diag_bf16_bits, dim3((unsigned)g), dim3(256), 0, stream, start, n, out);
  return hipGetLastError();
}

hipError_t launch_diag_e4m3_bits(uint32_t start, int64_t n, uint8_t* out, hipStream_t stream) {
  const int64_t g = (n / 4 + 255) / 256;
  hipLaunchKernelGGL(k_diag_e4m3_bits, dim3((unsigned)g), dim3(256), 0, stream, start, n, out);
  return hipGetLastError();
}

}  // namespace lrq
