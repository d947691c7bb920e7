// Device-side numerics shared by every quantization kernel (gfx950 only).
//
// The FP8 block rules restate WeightQuantizer.quantize_tensor
// (lumenrl/quantization/weight_quantizer.py:59-71) as torch evaluates it on an
// x86 CPU; the MX rules are the OCP Microscaling v1.0 closed form.  Every
// function here is exercised bit-for-bit against the CPU oracle by the tests.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lrq_pow2_tables.h"

namespace lrq {

enum : int { kBF16 = 0, kF16 = 1, kF32 = 2, kF64 = 3 };

// ---------------------------------------------------------------------------
// bit helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// Two bf16 packed in one dword -> float (exact).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return u2f(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return u2f(w & 0xFFFF0000u); }

// float -> bf16 bits as torch's x86 kernels round: NaN -> 0xFFFF, else RNE.
__device__ __forceinline__ uint32_t bf16_bits(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFu;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_round(float f) { return u2f(bf16_bits(f) << 16); }
// bf16_round for a value known not to be NaN (RNE; inf and overflow to inf as IEEE)
__device__ __forceinline__ float bf16_round_finite(float f) {
  const uint32_t u = f2u(f);
  return u2f((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
}

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}
// float -> binary16 bits, RNE, subnormals kept; NaN keeps sign and top payload.
__device__ __forceinline__ uint32_t f16_bits(float f) {
  uint32_t u = f2u(f);
  uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7E00u | ((a >> 13) & 0x3FFu);
  return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f);  // IEEE RNE, keeps subnormals
}
__device__ __forceinline__ float f16_round(float f) { return f16_to_f32(f16_bits(f)); }
// f16_round for a value known not to be NaN: IEEE RNE to binary16 and back
__device__ __forceinline__ float f16_round_finite(float f) { return (float)(_Float16)f; }

// ---------------------------------------------------------------------------
// element encoders
// ---------------------------------------------------------------------------
// Two floats -> two float8_e4m3fn bytes (RNE) in the low (HI=false) or high
// (HI=true) half of `old`.  gfx950's v_cvt_pk_fp8_f32 is the OCP e4m3 encoder,
// round-to-nearest-even; over every float32 bit pattern it matches torch's
// float8_e4m3fn cast except on NaN inputs (0xFF for any NaN sign).  Only
// finite |v| <= 448 is ever fed to it; inf/NaN blocks use special_code().
template <bool HI>
__device__ __forceinline__ uint32_t cvt_e4m3x2(float a, float b, uint32_t old) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, HI);
}

// Four floats -> four e4m3 bytes (element 0 in the low byte).
__device__ __forceinline__ uint32_t cvt_e4m3x4(float a, float b, float c, float d) {
  uint32_t w = cvt_e4m3x2<false>(a, b, 0u);
  return cvt_e4m3x2<true>(c, d, w);
}

// Software float8_e4m3fn encoder, RNE, non-saturating (overflow, inf, NaN ->
// 0x7F|sign).  Used only for tiles holding inf/NaN, where torch's x86 NaN
// rules decide the bytes.
__device__ __forceinline__ uint32_t sw_e4m3(float f) {
  uint32_t u = f2u(f);
  uint32_t sign = (u >> 24) & 0x80u, a = u & 0x7FFFFFFFu;
  if (a >= 0x7F800000u) return sign | 0x7Fu;
  float af = u2f(a);
  if (af < 0x1p-6f) return sign | (uint32_t)__builtin_rintf(af * 512.0f);
  int e = (int)(a >> 23) - 127;
  if (e > 8) return sign | 0x7Fu;
  uint32_t keep = (a >> 20) & 7u, rem = a & 0xFFFFFu;
  uint32_t code = ((uint32_t)(e + 7) << 3) | keep;
  code += (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) ? 1u : 0u;
  return sign | (code > 0x7Eu ? 0x7Fu : code);
}

// E2M1 nibble of a finite float: RNE onto {0,.5,1,1.5,2,3,4,6}, saturating.
// Software form, kept for the generic (unaligned) MX kernel.
__device__ __forceinline__ uint32_t e2m1_code(float v) {
  uint32_t u = f2u(v);
  uint32_t sign = (u >> 28) & 0x8u, a = u & 0x7FFFFFFFu;
  float af = u2f(a);
  // |v| < 1: multiples of 0.5 -- adding 2^22 (ulp 0.5) rounds to nearest even.
  uint32_t sub = f2u(af + 4194304.0f) - 0x4A800000u;
  // |v| >= 1: keep one mantissa bit with RNE; exponent rebased so 1.0 -> 2.
  uint32_t nrm = (a - 0x3F000000u + 0x1FFFFFu + ((a >> 22) & 1u)) >> 22;
  nrm = nrm > 7u ? 7u : nrm;
  return sign | (af < 1.0f ? sub : nrm);
}

// Two finite elements of an MXFP4 group with E8M0 exponent e -> two E2M1
// nibbles (first in the low nibble) written into byte SEL of `old`.
// gfx950's v_cvt_scalef32_pk_fp4_f32 divides by 2^(e-127) -- the scale
// operand's exponent field is read as the E8M0 byte -- then rounds to nearest
// even and saturates at +-6; it matches the OCP rule (x * 2^(127-e) through
// e2m1_code) on every finite bf16 x and every e (checked exhaustively).
template <int SEL>
__device__ __forceinline__ uint32_t mx_fp4x2(uint32_t old, float a, float b, uint32_t e8m0) {
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(old, a, b, u2f(e8m0 << 23), SEL);
}

// e4m3fn byte pair (low or high 16 bits of `w`) -> two floats, via gfx950's
// v_cvt_pk_f32_fp8.  Exact for every non-NaN code; callers route NaN codes
// (0x7F/0xFF) through e4m3 rules of their own.
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <bool HI>
__device__ __forceinline__ f32x2 e4m3x2_to_f32(uint32_t w) {
  return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, HI);
}

// Two floats -> two bf16 (first in the low half), round to nearest even, via
// v_cvt_pk_bf16_f32.  Matches bf16_bits() on every non-NaN float32 (checked
// exhaustively); NaN inputs must take bf16_bits() (torch writes 0xFFFF).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_bits(float a, float b) {
  const bf16x2 h = __builtin_convertvector((f32x2){a, b}, bf16x2);
  return __builtin_bit_cast(uint32_t, h);
}

// ---------------------------------------------------------------------------
// FP8 block scale (weight_quantizer.py:60-65)
// ---------------------------------------------------------------------------
enum : int { kScaleFast = 0, kScaleExact = 1, kScaleInf = 2, kScaleNaN = 3 };

struct BlockScale {
  float s;   // the scale, as a float value of the compute dtype
  float y;   // correctly rounded 1/s (kScaleFast)
  int kind;
};

// 2^round(log2 s) for a normal positive float32 s (torch.log2/round/pow).
__device__ __forceinline__ float pow2_f32(float s) {
  uint32_t b = f2u(s), e = b >> 23, m = b & 0x7FFFFFu;
  uint32_t up = m >= kPow2CutF32[e - 1] ? 1u : 0u;
  return u2f((e + up) << 23);  // e + up == 255 gives +inf, as torch.pow(2, 128.)
}
__device__ __forceinline__ float pow2_bf16(float s) {  // s is a normal bf16 value
  uint32_t b = f2u(s), e = b >> 23, m = (b >> 16) & 0x7Fu;
  uint32_t up = m >= kPow2CutBF16[e - 1] ? 1u : 0u;
  return u2f((e + up) << 23);
}
__device__ __forceinline__ float pow2_f16(float s) {  // s is a normal f16 value
  uint32_t h = f16_bits(s), e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  uint32_t up = m >= kPow2CutF16[e - 1] ? 1u : 0u;
  return f16_to_f32((e + up) << 10);  // e + up == 31 gives +inf
}

// amax_bits = max over the block of (float32 bits & 0x7FFFFFFF).
// CDT = compute dtype (kF32 for float32 arithmetic, else the input dtype).
template <int CDT>
__device__ __forceinline__ BlockScale block_scale(uint32_t amax_bits, bool pow2) {
  BlockScale r;
  r.y = 0.0f;
  if (amax_bits > 0x7F800000u) {
    // amax -> canonical NaN; /448 keeps it; a bf16 result rounds to 0xFFFF.
    // torch.pow(2, NaN) (pow2 scales) returns all-ones bits in torch's
    // vectorized x86 loop.
    if (pow2) r.s = CDT == kF32 ? u2f(0xFFFFFFFFu) : (CDT == kBF16 ? u2f(0xFFFF0000u) : f16_to_f32(0xFFFFu));
    else r.s = CDT == kBF16 ? u2f(0xFFFF0000u) : u2f(0x7FC00000u);
    r.kind = kScaleNaN;
    return r;
  }
  if (amax_bits == 0x7F800000u) {
    r.s = u2f(0x7F800000u);
    r.kind = kScaleInf;
    return r;
  }
  float amax = u2f(amax_bits);
  float s = amax / 448.0f;  // IEEE division, correctly rounded
  if (CDT == kBF16) s = bf16_round(s);
  if (CDT == kF16) s = f16_round(s);
  const float tiny = CDT == kF16 ? 0x1p-14f : 0x1p-126f;
  s = s < tiny ? tiny : s;
  if (pow2) s = CDT == kF32 ? pow2_f32(s) : (CDT == kBF16 ? pow2_bf16(s) : pow2_f16(s));
  r.s = s;
  if (s == u2f(0x7F800000u)) {  // pow2 overflow: every finite x/inf is +-0
    r.kind = kScaleInf;
    return r;
  }
  r.y = 1.0f / s;  // IEEE division, correctly rounded
  // Blocks whose amax is below 2^-80 may hold subnormal x whose Markstein
  // residual underflows; they take the exact division (never real weights).
  r.kind = amax < 0x1p-80f ? kScaleExact : kScaleFast;
  return r;
}

// q = x / s as float32 arithmetic rounds it, for finite-scale blocks.
// kScaleFast: Markstein's correction of x*y with y = RN(1/s): with y correctly
// rounded and the residual exact, RN(q0 + (x - q0*s)*y) = RN(x/s).  The
// residual is formed as -(q0*s - x) so that x = -0 keeps its sign.
// x and s are finite here, so the quotient is never NaN.
template <int CDT>
__device__ __forceinline__ float block_quot(float x, const BlockScale& b) {
  if (CDT == kBF16) {
    // bf16 arithmetic: RN_bf16(RN_f32(x/s)); x*y lands on the same bf16 value
    // for every bf16 x and every bf16 s (checked exhaustively).
    return bf16_round_finite(b.kind == kScaleFast ? x * b.y : x / b.s);
  }
  float q;
  if (b.kind == kScaleFast) {
    const float q0 = x * b.y;
    const float t = __builtin_fmaf(q0, b.s, -x);
    q = __builtin_fmaf(-t, b.y, q0);
  } else {
    q = x / b.s;
  }
  // fp16 arithmetic: RN_f16(RN_f32(x/s)); every nonzero fp16 x has |x| >= 2^-24,
  // so the residual never underflows (checked exhaustively over fp16 pairs)
  return CDT == kF16 ? f16_round_finite(q) : q;
}

// e4m3 byte of x in a block whose scale is inf or NaN (torch on x86):
//   x / NaN  -> NaN of the scale, or x itself if x is NaN;
//   x / inf  -> +-0 for finite x; inf/inf -> default NaN 0xFFC00000 (negative).
// In bf16/fp16 arithmetic the quotient is rounded to the dtype first
// (bf16: every NaN -> 0xFFFF; fp16: NaN keeps its sign).
template <int CDT>
__device__ __forceinline__ uint32_t special_code(float x, const BlockScale& b) {
  uint32_t ux = f2u(x), ax = ux & 0x7FFFFFFFu, sx = (ux >> 24) & 0x80u;
  bool xnan = ax > 0x7F800000u, xinf = ax == 0x7F800000u;
  if (b.kind == kScaleNaN) {
    if (CDT == kBF16) return 0xFFu;
    return 0x7Fu | (xnan ? sx : ((f2u(b.s) >> 24) & 0x80u));
  }
  // inf scale
  if (xnan) return CDT == kBF16 ? 0xFFu : (0x7Fu | sx);
  if (xinf) return 0xFFu;
  return sx;
}

// ---------------------------------------------------------------------------
// MX scale (OCP MX v1.0): E8M0 = clamp(floor(log2 amax) - emax + 127, 0, 254),
// 0xFF for inf/NaN groups.
// ---------------------------------------------------------------------------
template <int EMAX>
__device__ __forceinline__ uint32_t mx_e8m0(uint32_t amax_bits) {
  if (amax_bits >= 0x7F800000u) return 0xFFu;
  int e = (int)(amax_bits >> 23) - EMAX;
  return e < 0 ? 0u : (uint32_t)e;
}
// 2^(127 - E) as a float (E <= 246 for E4M3, <= 252 for E2M1: always normal).
__device__ __forceinline__ float mx_mult(uint32_t e8m0) { return u2f((254u - e8m0) << 23); }

// ---------------------------------------------------------------------------
// streaming memory access and XCD-aware work order
// ---------------------------------------------------------------------------
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// Every tensor is device memory, but the kernels take their pointers from
// descriptors, so the compiler sees generic pointers and would emit flat_*
// accesses, which also count against the LDS counter.  These helpers access
// memory through the global address space (global_* instructions).
#define LRQ_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ T gld(const void* p) {
  return *(const LRQ_GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ void gst(void* p, T v) {
  *(LRQ_GLOBAL T*)p = v;
}
// Weights are read once and codes written once: non-temporal accesses keep
// them from displacing anything in L2/MALL (measured +5% HBM throughput).
template <class T>
__device__ __forceinline__ T gld_nt(const void* p) {
  return __builtin_nontemporal_load((const LRQ_GLOBAL T*)p);
}
template <class T>
__device__ __forceinline__ void gst_nt(void* p, T v) {
  __builtin_nontemporal_store(v, (LRQ_GLOBAL T*)p);
}
// Input loads take element-aligned addresses (2 bytes suffice): under the HSA
// ABI the hardware runs in unaligned-access mode (LLVM enables
// unaligned-access-mode for amdhsa targets), so a 16-byte load from a 2-byte
// aligned address is still one global_load_dwordx4, split by the memory
// pipeline where it crosses a cache line.  Aligned addresses compile to the
// same instruction as a 16-byte-aligned type would.
typedef unsigned int v4u_in __attribute__((ext_vector_type(4), aligned(2)));
__device__ __forceinline__ v4u load_nt(const void* p) {
  return __builtin_nontemporal_load((const LRQ_GLOBAL v4u_in*)p);
}
// Code loads of the dequant kernels take any byte alignment, likewise.
typedef unsigned int v2u_in __attribute__((ext_vector_type(2), aligned(1)));
typedef uint32_t u32_in __attribute__((aligned(1)));
typedef uint16_t u16_in __attribute__((aligned(1)));
__device__ __forceinline__ v2u load_nt8(const void* p) { return __builtin_nontemporal_load((const LRQ_GLOBAL v2u_in*)p); }
__device__ __forceinline__ uint32_t load_nt4(const void* p) {
  return __builtin_nontemporal_load((const LRQ_GLOBAL u32_in*)p);
}
__device__ __forceinline__ uint16_t load_nt2(const void* p) {
  return __builtin_nontemporal_load((const LRQ_GLOBAL u16_in*)p);
}
// Code stores take any byte alignment, in the same unaligned-access mode: the
// row kernels write blocks whose width is not a multiple of 8 at odd offsets.
typedef unsigned int v2u_out __attribute__((ext_vector_type(2), aligned(1)));
typedef unsigned int u32_out __attribute__((aligned(1)));
__device__ __forceinline__ void store_nt(void* p, v2u v) {
  __builtin_nontemporal_store(v, (LRQ_GLOBAL v2u_out*)p);
}
__device__ __forceinline__ void store_nt(void* p, uint32_t v) {
  __builtin_nontemporal_store(v, (LRQ_GLOBAL u32_out*)p);
}
typedef uint16_t u16_out __attribute__((aligned(1)));
__device__ __forceinline__ void store_nt2(void* p, uint16_t v) {
  __builtin_nontemporal_store(v, (LRQ_GLOBAL u16_out*)p);
}

// MI355X dispatches work-group i to XCD i % 8.  Work units adjacent in memory
// (the tiles of a 128-row band, consecutive row blocks) are given to one XCD in
// runs of RUN, so each XCD streams contiguous hundreds of KiB instead of every
// eighth unit.  A bijection on [0, n); the tail past the last whole run group
// keeps the identity order.  The best RUN depends on the kernel's unit size
// (per-kernel constants in lrq_internal.hpp).
template <int64_t RUN>
__device__ __forceinline__ int64_t xcd_unit(int64_t i, int64_t n) {
  constexpr int64_t chunk = 8 * RUN;
  if (i >= (n / chunk) * chunk) return i;
  const int64_t r = i % chunk;
  return (i - r) + (r % 8) * RUN + r / 8;
}

// ---------------------------------------------------------------------------
// small reductions
// ---------------------------------------------------------------------------
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Running max of |bf16| bit patterns over a dword holding two bf16 values.
__device__ __forceinline__ u16x2 amax_bf16x2(u16x2 m, uint32_t w) {
  return __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w & 0x7FFF7FFFu));
}

// Max over the 4 lanes of a quad (DPP quad_perm, no LDS).
__device__ __forceinline__ uint32_t quad_max(uint32_t v) {
  uint32_t o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);  // [1,0,3,2]
  v = v > o ? v : o;
  o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);  // [2,3,0,1]
  return v > o ? v : o;
}

// Max over aligned groups of LPB lanes (LPB = 2..64): DPP within 16 lanes,
// shuffles beyond.
template <int LPB>
__device__ __forceinline__ uint32_t group_max(uint32_t v) {
  uint32_t o;
  if constexpr (LPB >= 2) { o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false); v = v > o ? v : o; }
  if constexpr (LPB >= 4) { o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false); v = v > o ? v : o; }
  // row_half_mirror: lane i <- lane 7-i within its 8-lane half (joins the two
  // quads of an 8-lane group); row_mirror: lane i <- lane 15-i (joins halves)
  if constexpr (LPB >= 8) { o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false); v = v > o ? v : o; }
  if constexpr (LPB >= 16) { o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false); v = v > o ? v : o; }
  if constexpr (LPB >= 32) { o = (uint32_t)__shfl_xor((int)v, 16, 64); v = v > o ? v : o; }
  if constexpr (LPB >= 64) { o = (uint32_t)__shfl_xor((int)v, 32, 64); v = v > o ? v : o; }
  return v;
}

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
    v = v > o ? v : o;
  }
  return v;
}

}  // namespace lrq
