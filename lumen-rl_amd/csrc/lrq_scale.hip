// Per-tensor FP8 scale of the KV-cache quantizer
// (lumenrl/quantization/fp8_kv_cache.py:52-54): for each tensor
//   scale = max(|w|.max(), FLT_MIN) / 448     (clamp before the division),
// NaN anywhere -> 0x7FC00000 (torch's multi-threaded x86 reduction).
//
// Two launches over a grouped table:
//   k_amax          every work-group streams one 8 KiB unit of one tensor with
//                   kAmaxLoads (two) 16-byte nontemporal loads per lane, all
//                   issued before the reduction, and writes the unit's max |x| bit pattern to
//                   workspace[global unit];
//   k_tensor_scale  one 1024-thread work-group per tensor reduces its units'
//                   partials (16-byte loads) and writes the float32 scale.
// No atomics and no zero-initialised memory: every partial is written before
// it is read, and the result does not depend on scheduling.
#include <string.h>

#include <mutex>

#include "lrq.h"
#include "lrq_device.hpp"
#include "lrq_internal.hpp"

// The partial-maximum workspace of lrq_tensor_scale_grouped_static, for callers
// that cannot allocate device memory.  Every device the library runs on holds
// its own copy for the life of the process.  Host code never passes `scratch`
// itself to a kernel (on the host it is only a stand-in for the symbol): it
// looks up the device address once per device (static_workspace) and passes
// that.
static __device__ __align__(256) uint32_t scratch[LRQ_STATIC_WORKSPACE_BYTES / 4];

namespace lrq {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint32_t* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device
}  // namespace

hipError_t static_workspace(int dev, uint32_t** out) {
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // with `dev` current
    if (cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = static_cast<uint32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}


// Elements per unit of the vector kernel (256 lanes x kAmaxLoads x 16 bytes).
int64_t amax_unit_elems(int dtype, bool vec) {
  return vec ? 256 * kAmaxLoads * (16 / (dtype == kF32 ? 4 : 2)) : 256 * 32;
}

// Element e of a tensor's [batch, rows, cols] sequence -> input offset.
__device__ __forceinline__ int64_t amax_offset(const Desc& d, int64_t e) {
  const int64_t per = d.rows * d.cols;
  const int64_t b = e / per;
  const int64_t r = (e - b * per) / d.cols;
  return b * d.bstride + r * d.ld + (e - b * per - r * d.cols);
}

// |x| bit pattern of one 16-bit element widened to float32 order (bf16 and
// f16 |x| patterns are ordered like their values; NaN patterns sort above inf).
template <int DT>
__device__ __forceinline__ uint32_t abs16_to_f32_bits(uint32_t h) {
  if constexpr (DT == kBF16) return h << 16;
  else return f2u(f16_to_f32(h));
}

__device__ __forceinline__ uint32_t block_reduce_max(uint32_t v, uint32_t* lds) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) lds[w] = v;
  __syncthreads();
  uint32_t r = lds[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) r = lds[i] > r ? lds[i] : r;
  return r;
}

// Max |x| bit pattern (float32 order) over this lane's part of unit u.
// VEC: 16-byte loads (element-aligned input, any row pitch, cols a multiple of
// the 16-byte element count); DENSE: the tensor is one contiguous run.
// Otherwise the lane walks single elements.
template <int DT, bool VEC, bool DENSE>
__device__ __forceinline__ uint32_t lane_amax(const Desc& d, int64_t u) {
  const int64_t n = d.batch * d.rows * d.cols;
  if constexpr (VEC) {
    constexpr int EPL = DT == kF32 ? 4 : 8;  // elements per 16-byte load
    constexpr int ES = DT == kF32 ? 4 : 2;
    const int64_t e0 = u * (256 * kAmaxLoads * EPL) + EPL * (int64_t)threadIdx.x;
    v4u v[kAmaxLoads];
#pragma unroll
    for (int j = 0; j < kAmaxLoads; ++j) {
      const int64_t e = e0 + (int64_t)256 * EPL * j;
      v[j] = v4u{0u, 0u, 0u, 0u};
      if (e < n) v[j] = load_nt(static_cast<const char*>(d.in) + (DENSE ? e : amax_offset(d, e)) * ES);
    }
    if constexpr (DT == kF32) {
      uint32_t a = 0u;
#pragma unroll
      for (int j = 0; j < kAmaxLoads; ++j) {
        const uint32_t w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t t = w4[i] & 0x7FFFFFFFu;
          a = t > a ? t : a;
        }
      }
      return a;
    } else {
      u16x2 a = u16x2{0, 0};
#pragma unroll
      for (int j = 0; j < kAmaxLoads; ++j) {
        a = amax_bf16x2(a, v[j].x);
        a = amax_bf16x2(a, v[j].y);
        a = amax_bf16x2(a, v[j].z);
        a = amax_bf16x2(a, v[j].w);
      }
      return abs16_to_f32_bits<DT>(a.x > a.y ? a.x : a.y);
    }
  } else {
    const int64_t e0 = u * (256 * 32) + threadIdx.x;
    uint32_t a = 0u;
    for (int j = 0; j < 32; ++j) {
      const int64_t e = e0 + 256 * j;
      if (e >= n) break;
      const int64_t off = DENSE ? e : amax_offset(d, e);
      uint32_t t;
      if constexpr (DT == kF32) t = gld<uint32_t>(static_cast<const uint32_t*>(d.in) + off) & 0x7FFFFFFFu;
      else t = abs16_to_f32_bits<DT>(gld<uint16_t>(static_cast<const uint16_t*>(d.in) + off) & 0x7FFFu);
      a = t > a ? t : a;
    }
    return a;
  }
}

// Grouped: the table's map names each work-group's tensor; a tensor's
// units_c / units_r flag 16-byte loads / a contiguous layout (uniform per
// work-group, so the branch below is a scalar one).
template <int DT>
__global__ __launch_bounds__(256) void k_amax(Desc single, const Desc* __restrict__ descs,
                                              const uint32_t* __restrict__ map, uint32_t* __restrict__ partial) {
  __shared__ uint32_t lds[4];
  Desc d;
  int64_t u;
  pick_desc<kXcdRunStream>(single, descs, map, d, u);
  uint32_t m;
  if (d.units_c) m = d.units_r ? lane_amax<DT, true, true>(d, u) : lane_amax<DT, true, false>(d, u);
  else m = d.units_r ? lane_amax<DT, false, true>(d, u) : lane_amax<DT, false, false>(d, u);
  m = block_reduce_max(m, lds);
  if (threadIdx.x == 0) partial[d.unit0 + u] = m;
}

// One 1024-thread work-group per tensor: max over the tensor's partials, then
// the scale.  The partials between the first and last 16-byte boundary of the
// tensor's slice are read 4 at a time, kScaleLoads loads in flight per thread
// (a 2 GiB tensor has 262144 partials: 8 rounds instead of 1024 with one
// 4-byte load per thread and round); the at most 3 before and 3 after are read
// singly.
constexpr int kScaleLoads = 8;
__global__ __launch_bounds__(kScaleThreads) void k_tensor_scale(const Desc* __restrict__ descs,
                                                                const uint32_t* __restrict__ partial) {
  __shared__ uint32_t lds[kScaleThreads / 64];
  const Desc d = descs[blockIdx.x];
  const uint32_t* p = partial + d.unit0;
  const int64_t n = d.units;
  const int tid = threadIdx.x;
  int64_t head = (int64_t)((16u - ((uintptr_t)p & 15u)) & 15u) / 4;  // partials before a 16-byte boundary
  head = head < n ? head : n;
  uint32_t a = tid < head ? p[tid] : 0u;
  const v4u* q = reinterpret_cast<const v4u*>(p + head);
  const int64_t nv = (n - head) / 4;  // 16-byte groups
  for (int64_t i = tid; i < nv; i += (int64_t)kScaleThreads * kScaleLoads) {
    v4u v[kScaleLoads];
#pragma unroll
    for (int k = 0; k < kScaleLoads; ++k) {
      const int64_t j = i + (int64_t)kScaleThreads * k;
      v[k] = j < nv ? q[j] : v4u{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int k = 0; k < kScaleLoads; ++k) {
      const uint32_t m01 = v[k].x > v[k].y ? v[k].x : v[k].y, m23 = v[k].z > v[k].w ? v[k].z : v[k].w;
      const uint32_t m = m01 > m23 ? m01 : m23;
      a = m > a ? m : a;
    }
  }
  const int64_t t0 = head + 4 * nv;  // the last n - t0 (< 4) partials
  if (tid < n - t0) a = p[t0 + tid] > a ? p[t0 + tid] : a;
  a = wave_max(a);
  if ((tid & 63) == 0) lds[tid >> 6] = a;
  __syncthreads();
  a = lds[0];
#pragma unroll
  for (int w = 1; w < kScaleThreads / 64; ++w) a = lds[w] > a ? lds[w] : a;
  if (tid == 0) {
    float s;
    if (a > 0x7F800000u) {
      s = u2f(0x7FC00000u);
    } else {
      float amax = u2f(a);
      amax = amax < 0x1p-126f ? 0x1p-126f : amax;
      s = amax / 448.0f;  // IEEE division (correctly rounded, subnormal results kept)
    }
    gst<float>(d.scales, s);
  }
}

hipError_t launch_tensor_scale(const LaunchCfg& cfg, const Desc* descs, const uint32_t* map, int64_t n,
                               int64_t units, uint32_t* partial, hipStream_t stream) {
  Desc none;
  memset(&none, 0, sizeof(none));
  const dim3 grid((unsigned)units), block(256);
  switch (cfg.in_dtype) {
    case kBF16: hipLaunchKernelGGL(k_amax<kBF16>, grid, block, 0, stream, none, descs, map, partial); break;
    case kF16: hipLaunchKernelGGL(k_amax<kF16>, grid, block, 0, stream, none, descs, map, partial); break;
    case kF32: hipLaunchKernelGGL(k_amax<kF32>, grid, block, 0, stream, none, descs, map, partial); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_tensor_scale, dim3((unsigned)n), dim3(kScaleThreads), 0, stream, descs, partial);
  return hipGetLastError();
}

}  // namespace lrq
