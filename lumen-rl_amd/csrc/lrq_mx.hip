// MXFP8 / MXFP4 quantization kernels (OCP Microscaling v1.0), gfx950 wave64.
//
// No counterpart kernel exists in the reference tree: LumenRL hands MX weights
// to vLLM/ATOM/aiter (`quantization: mxfp4`,
// examples/Qwen3_8B_SDDD_MI350_vLLM/configs/opd_qwen3_8b.yaml:43;
// aiter quant_mxfp8, examples/DAPO/atom_aiter_shim/sitecustomize.py:31-32).
// Per 1x32 group along the last dim: E8M0 = clamp(floor(log2 amax) - emax +
// 127, 0, 254) (0xFF for inf/NaN groups); elements x * 2^(127-E8M0) rounded to
// nearest even, saturating (E4M3 +-448, E2M1 +-6).  E2M1 uses gfx950's scaled
// FP4 pack-convert; E4M3 scales, clamps and uses the FP8 pack-convert.
//
// k_mx (bf16/f16): a quad of lanes per group (8 elements per lane); wave w of
// work-group u takes groups 64*kMxLoads*u + 16*kMxLoads*w + 16j + (lane>>2),
// j < kMxLoads, so each load instruction of a wave reads 16 whole groups =
// 1 KiB contiguous.  k_mx_f32: 8 lanes per group, the same 1 KiB per load.
#include "lrq_device.hpp"
#include "lrq_internal.hpp"

namespace lrq {

// 8 bf16/f16 elements (16 bytes) -> w[0..3]
__device__ __forceinline__ void mx_load8(const void* base, int64_t off, uint32_t (&w)[4]) {
  const v4u a = load_nt(static_cast<const uint16_t*>(base) + off);
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
}

template <int DT, int N>
__device__ __forceinline__ float mx_elem(const uint32_t (&w)[N], int i) {
  if constexpr (DT == kF32) return u2f(w[i]);
  else if constexpr (DT == kBF16) return (i & 1) ? bf16_hi(w[i >> 1]) : bf16_lo(w[i >> 1]);
  else return f16_to_f32((i & 1) ? (w[i >> 1] >> 16) : (w[i >> 1] & 0xFFFFu));
}

// amax of 8 bf16/f16 elements, as float32 bits
template <int DT>
__device__ __forceinline__ uint32_t mx_amax8(const uint32_t (&w)[4]) {
  u16x2 m = u16x2{0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) m = amax_bf16x2(m, w[i]);
  const uint32_t a = m.x > m.y ? m.x : m.y;
  if constexpr (DT == kBF16) return a << 16;
  return f2u(f16_to_f32(a));
}

// E (4 or 8) elements of a group -> E4M3 bytes (E) or E2M1 nibbles (E, in the
// low E/2 bytes of r.x).
template <int DT, int FMT, int E = 8, int N>
__device__ __forceinline__ v2u mx_encode(const uint32_t (&w)[N], uint32_t e8m0) {
  v2u r;
  if (e8m0 != 0xFFu) {
    if constexpr (FMT == 8) {
      const float mult = mx_mult(e8m0);
      float v[8];
#pragma unroll
      for (int i = 0; i < E; ++i) v[i] = __builtin_amdgcn_fmed3f(mx_elem<DT>(w, i) * mult, -448.0f, 448.0f);
      r.x = cvt_e4m3x4(v[0], v[1], v[2], v[3]);
      r.y = 0u;
      if constexpr (E == 8) r.y = cvt_e4m3x4(v[4], v[5], v[6], v[7]);
    } else {
      uint32_t n = mx_fp4x2<0>(0u, mx_elem<DT>(w, 0), mx_elem<DT>(w, 1), e8m0);
      n = mx_fp4x2<1>(n, mx_elem<DT>(w, 2), mx_elem<DT>(w, 3), e8m0);
      if constexpr (E == 8) {
        n = mx_fp4x2<2>(n, mx_elem<DT>(w, 4), mx_elem<DT>(w, 5), e8m0);
        n = mx_fp4x2<3>(n, mx_elem<DT>(w, 6), mx_elem<DT>(w, 7), e8m0);
      }
      r.x = n;
      r.y = 0u;
    }
  } else {
    // inf/NaN group: E4M3 NaN|sign for inf/NaN elements, +-0 otherwise;
    // E2M1 has no NaN: +-0 for every element.
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const uint32_t u = f2u(mx_elem<DT>(w, i));
      uint32_t c;
      if constexpr (FMT == 8) {
        c = ((u >> 24) & 0x80u) | ((u & 0x7FFFFFFFu) >= 0x7F800000u ? 0x7Fu : 0u);
        if (i < 4) lo |= c << (8 * i);
        else hi |= c << (8 * (i - 4));
      } else {
        c = (u >> 28) & 0x8u;
        lo |= c << (4 * i);
      }
    }
    r.x = lo;
    r.y = hi;
  }
  return r;
}

template <int DT, int FMT>
__global__ __launch_bounds__(256) void k_mx(Desc single, const Desc* __restrict__ descs,
                                            const uint32_t* __restrict__ map) {
  constexpr int kEmax = FMT == 8 ? 8 : 2;
  Desc d;
  int64_t u;
  pick_desc<kXcdRunMx>(single, descs, map, d, u);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int p = lane & 3;
  const int64_t g0 = u * (64 * kMxLoads) + (tid >> 6) * (16 * kMxLoads) + (lane >> 2);

  uint32_t w[kMxLoads][4];
  bool ok[kMxLoads];
#pragma unroll
  for (int j = 0; j < kMxLoads; ++j) {
    const int64_t g = g0 + 16 * j;
    ok[j] = g < d.nblocks;
    if (ok[j]) {
      int64_t off;
      if (d.ld == d.cols) {
        off = g * 32 + p * 8;
      } else {
        const int64_t row = g / d.bpr;
        off = row * d.ld + (g - row * d.bpr) * 32 + p * 8;
      }
      mx_load8(d.in, off, w[j]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[j][i] = 0u;
    }
  }

#pragma unroll
  for (int j = 0; j < kMxLoads; ++j) {
    // quads are either wholly in range or wholly out: the DPP stays in-quad
    const uint32_t a = quad_max(mx_amax8<DT>(w[j]));
    const uint32_t e = mx_e8m0<kEmax>(a);
    if (!ok[j]) continue;
    const int64_t g = g0 + 16 * j;
    const v2u c = mx_encode<DT, FMT>(w[j], e);
    if constexpr (FMT == 8) {
      store_nt(d.codes + g * 32 + p * 8, c);
    } else {
      store_nt(d.codes + g * 16 + p * 4, (uint32_t)c.x);
    }
    if (p == 0) gst<uint8_t>(static_cast<uint8_t*>(d.scales) + g, (uint8_t)e);
  }
}

// Float32 input: 8 lanes per group and 4 elements per lane, so each lane makes
// one 16-byte load per group and each wave load instruction reads 8 whole
// groups = 1 KiB contiguous (k_mx's 8 elements per lane would take two loads
// at a 32-byte lane stride).  A work-group covers the same 64 * kMxLoads groups
// as k_mx: wave w takes groups 64*kMxLoads*u + 16*kMxLoads*w + 8j + (lane>>3).
// Lanes past the last group load the last group (in bounds) and store nothing.
template <int FMT>
__global__ __launch_bounds__(256) void k_mx_f32(Desc single, const Desc* __restrict__ descs,
                                                const uint32_t* __restrict__ map) {
  constexpr int kEmax = FMT == 8 ? 8 : 2;
  constexpr int J = 2 * kMxLoads;
  Desc d;
  int64_t u;
  pick_desc<kXcdRunMx>(single, descs, map, d, u);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int p = lane & 7;
  const int64_t g0 = u * (64 * kMxLoads) + (tid >> 6) * (16 * kMxLoads) + (lane >> 3);
  const float* in = static_cast<const float*>(d.in);

  uint32_t w[J][4];
  bool ok[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t g = g0 + 8 * j;
    ok[j] = g < d.nblocks;
    const int64_t gc = ok[j] ? g : d.nblocks - 1;
    int64_t off;
    if (d.ld == d.cols) {
      off = gc * 32 + p * 4;
    } else {
      const int64_t row = gc / d.bpr;
      off = row * d.ld + (gc - row * d.bpr) * 32 + p * 4;
    }
    const v4u a = load_nt(in + off);
    w[j][0] = a.x; w[j][1] = a.y; w[j][2] = a.z; w[j][3] = a.w;
  }
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int j = 0; j < J; ++j) {
    uint32_t a = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t m = w[j][i] & 0x7FFFFFFFu;
      a = m > a ? m : a;
    }
    // the 8 lanes of a group share g: wholly in range or wholly out
    const uint32_t e = mx_e8m0<kEmax>(group_max<8>(a));
    if (!ok[j]) continue;
    const int64_t g = g0 + 8 * j;
    const v2u c = mx_encode<kF32, FMT, 4>(w[j], e);
    if constexpr (FMT == 8) {
      store_nt(d.codes + g * 32 + p * 4, (uint32_t)c.x);
    } else {
      gst_nt<uint16_t>(d.codes + g * 16 + p * 2, (uint16_t)c.x);
    }
    if (p == 0) gst<uint8_t>(static_cast<uint8_t*>(d.scales) + g, (uint8_t)e);
  }
}

// Generic: one thread per group, scalar loads, any stride/alignment.
template <int DT, int FMT>
__global__ __launch_bounds__(256) void k_mx_generic(Desc single, const Desc* __restrict__ descs,
                                                    const uint32_t* __restrict__ map) {
  constexpr int kEmax = FMT == 8 ? 8 : 2;
  Desc d;
  int64_t u;
  pick_desc<kXcdRunStream>(single, descs, map, d, u);
  const int64_t g = u * 256 + threadIdx.x;
  if (g >= d.nblocks) return;
  const int64_t row = g / d.bpr;
  const int64_t base = row * d.ld + (g - row * d.bpr) * 32;
  float x[32];
  uint32_t a = 0u;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    if constexpr (DT == kF32) x[i] = gld<float>(static_cast<const float*>(d.in) + base + i);
    else if constexpr (DT == kBF16) x[i] = u2f((uint32_t)gld<uint16_t>(static_cast<const uint16_t*>(d.in) + base + i) << 16);
    else x[i] = f16_to_f32(gld<uint16_t>(static_cast<const uint16_t*>(d.in) + base + i));
    const uint32_t m = f2u(x[i]) & 0x7FFFFFFFu;
    a = m > a ? m : a;
  }
  const uint32_t e = mx_e8m0<kEmax>(a);
  gst<uint8_t>(static_cast<uint8_t*>(d.scales) + g, (uint8_t)e);
  const float mult = e != 0xFFu ? mx_mult(e) : 0.0f;
  if constexpr (FMT == 8) {
    uint8_t* out = d.codes + g * 32;
    for (int i = 0; i < 32; ++i) {
      const uint32_t ux = f2u(x[i]);
      uint32_t c;
      if (e == 0xFFu) c = ((ux >> 24) & 0x80u) | ((ux & 0x7FFFFFFFu) >= 0x7F800000u ? 0x7Fu : 0u);
      else c = sw_e4m3(__builtin_amdgcn_fmed3f(x[i] * mult, -448.0f, 448.0f));
      gst<uint8_t>(out + i, (uint8_t)c);
    }
  } else {
    uint8_t* out = d.codes + g * 16;
    for (int i = 0; i < 32; i += 2) {
      uint32_t lo, hi;
      if (e == 0xFFu) {
        lo = (f2u(x[i]) >> 28) & 0x8u;
        hi = (f2u(x[i + 1]) >> 28) & 0x8u;
      } else {
        lo = e2m1_code(x[i] * mult);
        hi = e2m1_code(x[i + 1] * mult);
      }
      gst<uint8_t>(out + i / 2, (uint8_t)(lo | (hi << 4)));
    }
  }
}

// Diagnostic: the element path of k_mx on raw inputs; pair k = elements
// (2k, 2k+1) shares E8M0 byte e8m0[k]; one output byte (code or nibble) per element.
template <int FMT>
__global__ __launch_bounds__(256) void k_diag_mx(const float* __restrict__ in,
                                                 const uint8_t* __restrict__ e8m0, int64_t npairs,
                                                 uint8_t* __restrict__ out) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= npairs) return;
  uint32_t w[8];
  w[0] = f2u(in[2 * k]);
  w[1] = f2u(in[2 * k + 1]);
#pragma unroll
  for (int i = 2; i < 8; ++i) w[i] = 0u;
  const v2u c = mx_encode<kF32, FMT>(w, e8m0[k]);
  if constexpr (FMT == 8) {
    out[2 * k] = (uint8_t)(c.x & 0xFFu);
    out[2 * k + 1] = (uint8_t)((c.x >> 8) & 0xFFu);
  } else {
    out[2 * k] = (uint8_t)(c.x & 0xFu);
    out[2 * k + 1] = (uint8_t)((c.x >> 4) & 0xFu);
  }
}

hipError_t launch_diag_mx(int fmt, const float* in, const uint8_t* e8m0, int64_t n, uint8_t* out,
                          hipStream_t stream) {
  const int64_t npairs = n / 2;
  const dim3 grid((unsigned)((npairs + 255) / 256)), block(256);
  if (fmt == 8) hipLaunchKernelGGL((k_diag_mx<8>), grid, block, 0, stream, in, e8m0, npairs, out);
  else hipLaunchKernelGGL((k_diag_mx<4>), grid, block, 0, stream, in, e8m0, npairs, out);
  return hipGetLastError();
}

template <int DT>
static hipError_t launch_mx_typed(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                                  const uint32_t* map, int64_t units, hipStream_t stream) {
  const dim3 grid((unsigned)units), block(256);
  const bool gen = cfg.kernel == kKernGenericMx;
  if (cfg.mx_fmt == 8) {
    if (gen) hipLaunchKernelGGL((k_mx_generic<DT, 8>), grid, block, 0, stream, single, descs, map);
    else if constexpr (DT == kF32) hipLaunchKernelGGL((k_mx_f32<8>), grid, block, 0, stream, single, descs, map);
    else hipLaunchKernelGGL((k_mx<DT, 8>), grid, block, 0, stream, single, descs, map);
  } else {
    if (gen) hipLaunchKernelGGL((k_mx_generic<DT, 4>), grid, block, 0, stream, single, descs, map);
    else if constexpr (DT == kF32) hipLaunchKernelGGL((k_mx_f32<4>), grid, block, 0, stream, single, descs, map);
    else hipLaunchKernelGGL((k_mx<DT, 4>), grid, block, 0, stream, single, descs, map);
  }
  return hipGetLastError();
}

hipError_t launch_mx(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                     const uint32_t* map, int64_t units, hipStream_t stream) {
  switch (cfg.in_dtype) {
    case kBF16: return launch_mx_typed<kBF16>(cfg, single, descs, map, units, stream);
    case kF16: return launch_mx_typed<kF16>(cfg, single, descs, map, units, stream);
    case kF32: return launch_mx_typed<kF32>(cfg, single, descs, map, units, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace lrq
