// Activation fake-quant of the FP8 W8A8 rollout linear
// (lumenrl/quantization/fp8_rollout.py:53-72): per 1xB block of each token row,
// s = clamp(amax/448, FLT_MIN) [pow2], x_dq = float32(x/s) * s.  The reference
// emulates FP8 activations without rounding them to e4m3, so x_dq is what the
// GEMM consumes; results match torch on x86 bit for bit (IEEE division per
// element, x86 NaN/inf rules on blocks whose scale is not finite).
//
// Kernels by block width B: k_act_qdq8 (16-bit input, B = 32..512 powers of
// two) and k_act_qdq (float32, B = 32..256), then for other widths k_act_pad
// (whole 16-byte chunks, up to 32 per block), k_act_wide (up to 512) and
// k_act_generic (any B).
#include "lrq.h"
#include "lrq_device.hpp"
#include "lrq_internal.hpp"

namespace lrq {

// torch's vectorized x86 product x * s: a NaN scale wins (quieted), then a
// NaN x; 0 * inf is the default NaN.
__device__ __forceinline__ float x86_mul_scale_first(float q, float s) {
  const uint32_t aq = f2u(q) & 0x7FFFFFFFu, as = f2u(s) & 0x7FFFFFFFu;
  if (as > 0x7F800000u) return u2f(f2u(s) | 0x00400000u);
  if (aq > 0x7F800000u) return u2f(f2u(q) | 0x00400000u);
  if ((aq == 0u && as == 0x7F800000u) || (as == 0u && aq == 0x7F800000u)) return u2f(0xFFC00000u);
  return q * s;
}
__device__ __forceinline__ float x86_div(float x, float s) {
  const uint32_t ax = f2u(x) & 0x7FFFFFFFu, as = f2u(s) & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return u2f(f2u(x) | 0x00400000u);
  if (as > 0x7F800000u) return u2f(f2u(s) | 0x00400000u);
  if ((ax == 0x7F800000u && as == 0x7F800000u) || (ax == 0u && as == 0u)) return u2f(0xFFC00000u);
  return x / s;
}

// 4 float32 elements (one 16-byte load; 4-byte alignment suffices)
__device__ __forceinline__ void load4(const void* base, int64_t off, float (&x)[4]) {
  const v4u v = load_nt(static_cast<const float*>(base) + off);
  x[0] = u2f(v.x); x[1] = u2f(v.y); x[2] = u2f(v.z); x[3] = u2f(v.w);
}

// Shared by both kernels: the [rows, cols] matrix is walked as its row-major
// element sequence e = row * cols + col (the output is dense), a 1xB block is
// B/EPL consecutive lanes holding EPL consecutive elements each, and
// cols % B == 0 keeps every block inside one row and one wave span.

__device__ __forceinline__ int64_t act_offset(int64_t e, int64_t cols, int64_t ld, bool dense) {
  if (dense) return e;
  const int64_t row = e / cols;
  return row * ld + (e - row * cols);
}

// x_dq for one lane's elements, given the block's |x| maximum bit pattern.
template <int N>
__device__ __forceinline__ void act_block(const float (&x)[N], uint32_t amax, int pow2, uint32_t (&o)[N]) {
  const BlockScale bs = block_scale<kF32>(amax, pow2 != 0);
  if (bs.kind <= kScaleExact) {
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = f2u((x[i] / bs.s) * bs.s);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = f2u(x86_mul_scale_first(x86_div(x[i], bs.s), bs.s));
  }
}

// x_dq of one element, given its block's scale (act_block's per-element step).
__device__ __forceinline__ uint32_t act_elem(float x, const BlockScale& bs) {
  if (bs.kind <= kScaleExact) return f2u((x / bs.s) * bs.s);
  return f2u(x86_mul_scale_first(x86_div(x, bs.s), bs.s));
}

template <int N>
__device__ __forceinline__ uint32_t abs_max(const float (&x)[N]) {
  uint32_t a = 0u;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint32_t m = f2u(x[i]) & 0x7FFFFFFFu;
    a = m > a ? m : a;
  }
  return a;
}

// 16-bit inputs, 8 elements per lane: one 16-byte load per lane (a wave reads
// 1 KiB), 2048 elements per work-group.  Lane t of a wave holds elements
// 8t..8t+7 of the wave's 512-element span; the float32 results are exchanged
// across the wave so that store h of lane t writes elements 256h + 4t .. +3
// (owned by lane 32h + t/2, half t&1): each store instruction writes 1 KiB
// of whole cache lines.
template <int DT, int LPB, bool DENSE>
__global__ __launch_bounds__(256) void k_act_qdq8(const uint16_t* __restrict__ in, int64_t rows, int64_t cols,
                                                  int64_t ld, float* __restrict__ out, int pow2) {
  const int64_t n = rows * cols;
  const int lane = threadIdx.x & 63;
  const int64_t span = xcd_unit<kXcdRunStream>(blockIdx.x, gridDim.x) * 2048 + (threadIdx.x >> 6) * 512;
  const int64_t e = span + 8 * lane;
  v4u v = {0u, 0u, 0u, 0u};
  if (e < n) v = load_nt(in + act_offset(e, cols, ld, DENSE));
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float x[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (DT == kBF16) {
      x[2 * i] = bf16_lo(w[i]);
      x[2 * i + 1] = bf16_hi(w[i]);
    } else {
      x[2 * i] = f16_to_f32(w[i] & 0xFFFFu);
      x[2 * i + 1] = f16_to_f32(w[i] >> 16);
    }
  }
  const uint32_t a = group_max<LPB>(abs_max(x));  // a group is all in or all out of range
  uint32_t o[8];
  act_block(x, a, pow2, o);
  const bool odd = lane & 1;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int src = 32 * h + (lane >> 1);
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (uint32_t)__shfl((int)o[i], src, 64);
      const uint32_t hi = (uint32_t)__shfl((int)o[4 + i], src, 64);
      r[i] = odd ? hi : lo;
    }
    const int64_t eo = span + 256 * h + 4 * lane;
    if (eo < n) __builtin_nontemporal_store(v4u{r[0], r[1], r[2], r[3]}, reinterpret_cast<v4u*>(out + eo));
  }
}

// Float32 input, 4 elements per lane, NCH 1024-element chunks per
// work-group: in chunk j lane t holds elements 1024j + 4t .. +3, so each wave
// load reads one contiguous span and each store writes 1 KiB.  All NCH loads
// are issued before the first reduction.
template <int LPB, int NCH, bool DENSE>
__global__ __launch_bounds__(256) void k_act_qdq(const void* __restrict__ in, int64_t rows, int64_t cols,
                                                 int64_t ld, float* __restrict__ out, int pow2) {
  const int64_t n = rows * cols;
  const int64_t base = xcd_unit<kXcdRunStream>(blockIdx.x, gridDim.x) * (1024 * NCH) + 4 * (int64_t)threadIdx.x;
  float x[NCH][4];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t e = base + 1024 * j;
    x[j][0] = x[j][1] = x[j][2] = x[j][3] = 0.0f;
    if (e < n) load4(in, act_offset(e, cols, ld, DENSE), x[j]);
  }
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t e = base + 1024 * j;
    const uint32_t a = group_max<LPB>(abs_max(x[j]));
    if (e >= n) continue;
    uint32_t o[4];
    act_block(x[j], a, pow2, o);
    __builtin_nontemporal_store(v4u{o[0], o[1], o[2], o[3]}, reinterpret_cast<v4u*>(out + e));
  }
}

// Any other block width B (cols % B == 0; the vector kernels take 32, 64,
// 128, 256 and, for 16-bit input, 512): one wave per block, four per
// work-group.  The wave walks the
// block's elements 64 at a time twice, for the amax and then for x_dq (the
// second pass reads from L2); each pass's loads and float32 stores are
// coalesced across the wave.
template <int DT, bool DENSE>
__global__ __launch_bounds__(256) void k_act_generic(const void* __restrict__ in, int64_t rows, int64_t cols,
                                                     int64_t ld, int64_t blk, float* __restrict__ out, int pow2) {
  const int64_t nb = rows * (cols / blk);
  const int64_t bi = xcd_unit<kXcdRunStream>(blockIdx.x, gridDim.x) * 4 + (threadIdx.x >> 6);
  if (bi >= nb) return;  // the whole wave: this kernel has no barrier
  const int lane = threadIdx.x & 63;
  const int64_t e0 = bi * blk;  // the block's first element of the dense sequence
  auto load = [&](int64_t i) -> float {
    const int64_t off = act_offset(e0 + i, cols, ld, DENSE);
    if constexpr (DT == kF32) return gld<float>(static_cast<const float*>(in) + off);
    else if constexpr (DT == kBF16) return u2f((uint32_t)gld<uint16_t>(static_cast<const uint16_t*>(in) + off) << 16);
    else return f16_to_f32(gld<uint16_t>(static_cast<const uint16_t*>(in) + off));
  };
  uint32_t a = 0u;
  for (int64_t i = lane; i < blk; i += 64) {
    const uint32_t m = f2u(load(i)) & 0x7FFFFFFFu;
    a = m > a ? m : a;
  }
  a = __builtin_amdgcn_readfirstlane(wave_max(a));
  const BlockScale bs = block_scale<kF32>(a, pow2 != 0);
  for (int64_t i = lane; i < blk; i += 64) gst_nt<float>(out + e0 + i, u2f(act_elem(load(i), bs)));
}

// Widths that are a multiple of one 16-byte chunk (8 elements of 16-bit
// input, 4 of float32) up to 512 chunks: one wave per block, four per
// work-group, lane l holding chunks l + 64 k (k < NCH) in registers, so the
// block is read once.  Lanes past the block's chunks re-load its first chunk
// and drop out of the amax.  The float32 results go out as 16-byte stores, each
// store instruction writing whole lines (16-bit input: results exchanged
// across the wave as in k_act_qdq8).
template <int DT, int NCH, bool DENSE>
__global__ __launch_bounds__(256) void k_act_wide(const void* __restrict__ in, int64_t rows, int64_t cols,
                                                  int64_t ld, int64_t blk, float* __restrict__ out, int pow2) {
  constexpr int EPL = DT == kF32 ? 4 : 8;  // elements per 16-byte chunk
  const int64_t nb = rows * (cols / blk);
  const int64_t bi = xcd_unit<kXcdRunStream>(blockIdx.x, gridDim.x) * 4 + (threadIdx.x >> 6);
  if (bi >= nb) return;  // the whole wave: this kernel has no barrier
  const int lane = threadIdx.x & 63;
  const int g = (int)(blk / EPL);  // chunks per block
  const int64_t e0 = bi * blk;
  const char* src = static_cast<const char*>(in);
  v4u v[NCH];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
    v[k] = load_nt(src + act_offset(e0 + (int64_t)(c < g ? c : 0) * EPL, cols, ld, DENSE) * (DT == kF32 ? 4 : 2));
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t a = 0u;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    if (lane + 64 * k >= g) continue;
    const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t m;
      if constexpr (DT == kF32) {
        m = w[i] & 0x7FFFFFFFu;
      } else {
        const uint32_t lo = DT == kBF16 ? f2u(bf16_lo(w[i])) : f2u(f16_to_f32(w[i] & 0xFFFFu));
        const uint32_t hi = DT == kBF16 ? f2u(bf16_hi(w[i])) : f2u(f16_to_f32(w[i] >> 16));
        const uint32_t ml = lo & 0x7FFFFFFFu, mh = hi & 0x7FFFFFFFu;
        m = ml > mh ? ml : mh;
      }
      a = m > a ? m : a;
    }
  }
  a = __builtin_amdgcn_readfirstlane(wave_max(a));
  const BlockScale bs = block_scale<kF32>(a, pow2 != 0);
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    if (64 * k >= g) break;  // wave-uniform: every lane takes part in the shuffles below
    const int c = lane + 64 * k;
    const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
    if constexpr (DT == kF32) {
      if (c < g) {
        const v4u o = {act_elem(u2f(w[0]), bs), act_elem(u2f(w[1]), bs), act_elem(u2f(w[2]), bs),
                       act_elem(u2f(w[3]), bs)};
        __builtin_nontemporal_store(o, reinterpret_cast<v4u*>(out + e0 + (int64_t)c * EPL));
      }
    } else {
      uint32_t o[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = DT == kBF16 ? bf16_lo(w[i]) : f16_to_f32(w[i] & 0xFFFFu);
        const float hi = DT == kBF16 ? bf16_hi(w[i]) : f16_to_f32(w[i] >> 16);
        o[2 * i] = act_elem(lo, bs);
        o[2 * i + 1] = act_elem(hi, bs);
      }
      // as k_act_qdq8: store h of lane t writes elements 256 h + 4 t .. + 3 of
      // slot k's 512-element span (lane 32 h + t/2's chunk, half t & 1), so
      // each store instruction writes whole lines
      const bool odd = lane & 1;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int src = 32 * h + (lane >> 1);
        uint32_t r[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t lo = (uint32_t)__shfl((int)o[i], src, 64);
          const uint32_t hi = (uint32_t)__shfl((int)o[4 + i], src, 64);
          r[i] = odd ? hi : lo;
        }
        if (src + 64 * k < g)
          __builtin_nontemporal_store(v4u{r[0], r[1], r[2], r[3]},
                                      reinterpret_cast<v4u*>(out + e0 + 512 * k + 256 * h + 4 * lane));
      }
    }
  }
}

// Narrow widths of whole 16-byte chunks (g <= 32 of them): a block's chunks
// sit on an aligned group of L = nextpow2(g) lanes (4 at least), so a wave
// instruction holds 64/L blocks; each lane runs kActPadInstr instructions,
// each on the wave's next 64/L blocks.  Lanes past g re-load their block's
// first chunk and drop out of the amax; every lane of a group computes the
// group's scale.
constexpr int kActPadInstr = 4;
template <int DT, int L, bool DENSE>
__global__ __launch_bounds__(256) void k_act_pad(const void* __restrict__ in, int64_t rows, int64_t cols,
                                                 int64_t ld, int64_t blk, float* __restrict__ out, int pow2) {
  constexpr int EPL = DT == kF32 ? 4 : 8;  // elements per 16-byte chunk
  constexpr int BPI = 64 / L;              // blocks per wave instruction
  const int64_t nb = rows * (cols / blk);
  const int lane = threadIdx.x & 63;
  const int g = (int)(blk / EPL);
  const int c = lane % L;
  const int64_t b0 = (xcd_unit<kXcdRunStream>(blockIdx.x, gridDim.x) * 4 + (threadIdx.x >> 6)) *
                         (kActPadInstr * BPI) + lane / L;
  const char* src = static_cast<const char*>(in);
  v4u v[kActPadInstr];
#pragma unroll
  for (int i = 0; i < kActPadInstr; ++i) {
    const int64_t b = b0 + i * BPI;
    const int64_t bb = b < nb ? b : nb - 1;
    v[i] = load_nt(src + act_offset(bb * blk + (int64_t)(c < g ? c : 0) * EPL, cols, ld, DENSE) *
                             (DT == kF32 ? 4 : 2));
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kActPadInstr; ++i) {
    const int64_t b = b0 + i * BPI;
    const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
    float x[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == kF32) {
        x[j] = u2f(w[j]);
      } else {
        x[2 * j] = DT == kBF16 ? bf16_lo(w[j]) : f16_to_f32(w[j] & 0xFFFFu);
        x[2 * j + 1] = DT == kBF16 ? bf16_hi(w[j]) : f16_to_f32(w[j] >> 16);
      }
    }
    uint32_t a = 0u;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const uint32_t m = f2u(x[j]) & 0x7FFFFFFFu;
      a = m > a ? m : a;
    }
    a = group_max<L>(c < g ? a : 0u);  // the whole group is in or out of range
    const BlockScale bs = block_scale<kF32>(a, pow2 != 0);
    if (c < g && b < nb) {
      float* dst = out + b * blk + (int64_t)c * EPL;
      uint32_t o[8];
#pragma unroll
      for (int j = 0; j < EPL; ++j) o[j] = act_elem(x[j], bs);
      __builtin_nontemporal_store(v4u{o[0], o[1], o[2], o[3]}, reinterpret_cast<v4u*>(dst));
      if constexpr (EPL == 8)
        __builtin_nontemporal_store(v4u{o[4], o[5], o[6], o[7]}, reinterpret_cast<v4u*>(dst + 4));
    }
  }
}

// k_act_pad's lanes per block for a width (0: not a whole number of 16-byte
// chunks, or more than 32 of them).
int act_pad_lanes(int dtype, int64_t blk) {
  const int epl = dtype == kF32 ? 4 : 8;
  if (blk % epl || blk / epl > 32) return 0;
  int l = 4;
  while (l < blk / epl) l *= 2;
  return l;
}

// k_act_wide's chunk slots per lane for a block width (0: not a whole number
// of 16-byte chunks, or wider than 512 chunks).
int act_wide_slots(int dtype, int64_t blk) {
  const int epl = dtype == kF32 ? 4 : 8;
  if (blk % epl) return 0;
  const int64_t g = blk / epl;
  return g <= 64 ? 1 : g <= 128 ? 2 : g <= 256 ? 4 : g <= 512 ? 8 : 0;
}

constexpr int kActChunks = 2;

// Blocks of 32, 64, 128 or 256 elements (16-bit input: also 512) take the
// vector kernels: 16-bit input the 8-per-lane one (any element alignment and
// row pitch: its 16-byte loads take 2-byte-aligned addresses), float32 the
// 4-per-lane one.  Other widths of whole 16-byte chunks take k_act_pad (up to
// 32 chunks, several blocks per wave instruction) or k_act_wide (up to 512,
// one block per wave); the rest k_act_generic (one block per wave).
bool act_vector_block(int dtype, int64_t blk) {
  return blk == 32 || blk == 64 || blk == 128 || blk == 256 || (blk == 512 && dtype != kF32);
}

int64_t act_grid(int dtype, int64_t rows, int64_t cols, int64_t blk) {
  if (!act_vector_block(dtype, blk)) {
    const int64_t nb = rows * (cols / blk);
    const int l = act_pad_lanes(dtype, blk);
    const int64_t per_wg = l ? 4 * kActPadInstr * (64 / l) : 4;
    return (nb + per_wg - 1) / per_wg;
  }
  const int64_t per_wg = dtype != kF32 ? 2048 : 1024 * kActChunks;
  return (rows * cols + per_wg - 1) / per_wg;
}

template <int DT, bool DENSE>
static hipError_t launch_act_typed(const void* in, int64_t rows, int64_t cols, int64_t ld, int64_t blk,
                                   float* out, int pow2, hipStream_t stream) {
  const dim3 grid((unsigned)act_grid(DT, rows, cols, blk)), block(256);
  const uint16_t* in16 = static_cast<const uint16_t*>(in);
  if (!act_vector_block(DT, blk) && act_pad_lanes(DT, blk)) {
    switch (act_pad_lanes(DT, blk)) {
      case 4: hipLaunchKernelGGL((k_act_pad<DT, 4, DENSE>), grid, block, 0, stream, in, rows, cols, ld, blk, out, pow2); break;
      case 8: hipLaunchKernelGGL((k_act_pad<DT, 8, DENSE>), grid, block, 0, stream, in, rows, cols, ld, blk, out, pow2); break;
      case 16: hipLaunchKernelGGL((k_act_pad<DT, 16, DENSE>), grid, block, 0, stream, in, rows, cols, ld, blk, out, pow2); break;
      default: hipLaunchKernelGGL((k_act_pad<DT, 32, DENSE>), grid, block, 0, stream, in, rows, cols, ld, blk, out, pow2); break;
    }
  } else if (!act_vector_block(DT, blk)) {
    switch (act_wide_slots(DT, blk)) {
      case 1: hipLaunchKernelGGL((k_act_wide<DT, 1, DENSE>), grid, block, 0, stream, in, rows, cols, ld, blk, out, pow2); break;
      case 2: hipLaunchKernelGGL((k_act_wide<DT, 2, DENSE>), grid, block, 0, stream, in, rows, cols, ld, blk, out, pow2); break;
      case 4: hipLaunchKernelGGL((k_act_wide<DT, 4, DENSE>), grid, block, 0, stream, in, rows, cols, ld, blk, out, pow2); break;
      case 8: hipLaunchKernelGGL((k_act_wide<DT, 8, DENSE>), grid, block, 0, stream, in, rows, cols, ld, blk, out, pow2); break;
      default: hipLaunchKernelGGL((k_act_generic<DT, DENSE>), grid, block, 0, stream, in, rows, cols, ld, blk, out, pow2); break;
    }
  } else if constexpr (DT != kF32) {
    switch (blk) {
      case 32: hipLaunchKernelGGL((k_act_qdq8<DT, 4, DENSE>), grid, block, 0, stream, in16, rows, cols, ld, out, pow2); break;
      case 64: hipLaunchKernelGGL((k_act_qdq8<DT, 8, DENSE>), grid, block, 0, stream, in16, rows, cols, ld, out, pow2); break;
      case 128: hipLaunchKernelGGL((k_act_qdq8<DT, 16, DENSE>), grid, block, 0, stream, in16, rows, cols, ld, out, pow2); break;
      case 256: hipLaunchKernelGGL((k_act_qdq8<DT, 32, DENSE>), grid, block, 0, stream, in16, rows, cols, ld, out, pow2); break;
      case 512: hipLaunchKernelGGL((k_act_qdq8<DT, 64, DENSE>), grid, block, 0, stream, in16, rows, cols, ld, out, pow2); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (blk) {
      case 32: hipLaunchKernelGGL((k_act_qdq<8, kActChunks, DENSE>), grid, block, 0, stream, in, rows, cols, ld, out, pow2); break;
      case 64: hipLaunchKernelGGL((k_act_qdq<16, kActChunks, DENSE>), grid, block, 0, stream, in, rows, cols, ld, out, pow2); break;
      case 128: hipLaunchKernelGGL((k_act_qdq<32, kActChunks, DENSE>), grid, block, 0, stream, in, rows, cols, ld, out, pow2); break;
      case 256: hipLaunchKernelGGL((k_act_qdq<64, kActChunks, DENSE>), grid, block, 0, stream, in, rows, cols, ld, out, pow2); break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

hipError_t launch_act(const void* in, int dtype, int64_t rows, int64_t cols, int64_t ld, int64_t blk,
                      float* out, int pow2, hipStream_t stream) {
  const bool dense = rows == 1 || ld == cols;
  switch (dtype) {
    case kBF16:
      return dense ? launch_act_typed<kBF16, true>(in, rows, cols, ld, blk, out, pow2, stream)
                   : launch_act_typed<kBF16, false>(in, rows, cols, ld, blk, out, pow2, stream);
    case kF16:
      return dense ? launch_act_typed<kF16, true>(in, rows, cols, ld, blk, out, pow2, stream)
                   : launch_act_typed<kF16, false>(in, rows, cols, ld, blk, out, pow2, stream);
    case kF32:
      return dense ? launch_act_typed<kF32, true>(in, rows, cols, ld, blk, out, pow2, stream)
                   : launch_act_typed<kF32, false>(in, rows, cols, ld, blk, out, pow2, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace lrq
