// FP8 E4M3 blockwise quantization of float64 tensors in float64 arithmetic.
//
// WeightQuantizer.quantize_tensor on a float64 tensor
// (lumenrl/quantization/weight_quantizer.py:40-77) evaluates every op in the
// tensor's dtype: amax, amax / 448 (:61-62), clamp(min = 2^-1022) (:63), the
// optional pow2 rounding (:64-65) and x / s (:67).  The quotient is then
// rounded to float32 (:68) before the e4m3 cast (:71): a double rounding
// (f64 -> f32 -> e4m3) that this kernel keeps.  Scales are written as float64.
//
// k_row_f64 takes 1xB blocks (B = 32...2048, powers of two, the reference's
// layout), k_row_pad_f64 narrower widths (5 <= B < 128) on padded lane groups,
// k_row_wide_f64 the other 1xB widths up to 16384, and k_tile_f64 128x128 tiles,
// all with 16-byte loads.  Their quotients of finite blocks use one correctly
// rounded 1/s per block and Markstein's correction per element (the IEEE
// division in blocks with tiny scales) and the hardware e4m3 encoder.  k_f64
// takes every other shape, one wave per block (any block shape), four blocks
// per 256-thread work-group, re-reading the block from L2 for the encode, with
// the IEEE float64 division and the software encoder.
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

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int off) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, off, 64);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), off, 64);
  return ((uint64_t)hi << 32) | lo;
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}

// Max over aligned groups of LPB lanes (LPB = 2..64) of 64-bit values: DPP
// within 16 lanes (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror), shuffles beyond.
template <int LPB>
__device__ __forceinline__ uint64_t group_max_u64(uint64_t v) {
  if constexpr (LPB >= 2) v = umax64(v, dpp_u64<0xB1>(v));
  if constexpr (LPB >= 4) v = umax64(v, dpp_u64<0x4E>(v));
  if constexpr (LPB >= 8) v = umax64(v, dpp_u64<0x141>(v));
  if constexpr (LPB >= 16) v = umax64(v, dpp_u64<0x140>(v));
  if constexpr (LPB >= 32) v = umax64(v, shfl_xor_u64(v, 16));
  if constexpr (LPB >= 64) v = umax64(v, shfl_xor_u64(v, 32));
  return v;
}

// Maxima of V per-lane values (V = 1, 2, 4, 8) over aligned groups of G lanes
// (G = 16, 32, 64): halving exchanges across lanes G/2, G/4, ... apart leave
// each lane one value, then a G / V lane group reduction.  Lane l returns the
// maximum of value (l % G) / (G / V) over its group.
template <int V, int G>
__device__ __forceinline__ uint64_t split_max(const uint64_t (&p)[V], int lane) {
  static_assert((V == 1 || V == 2 || V == 4 || V == 8) && V <= G, "1, 2, 4 or 8 values");
  uint64_t c[V];
#pragma unroll
  for (int k = 0; k < V; ++k) c[k] = p[k];
#pragma unroll
  for (int nv = V, off = G / 2; nv > 1; nv /= 2, off /= 2) {
    const bool up = lane & off;  // this lane keeps the upper half of its values
#pragma unroll
    for (int k = 0; k < nv / 2; ++k) {
      const uint64_t keep = up ? c[nv / 2 + k] : c[k], send = up ? c[k] : c[nv / 2 + k];
      c[k] = umax64(keep, shfl_xor_u64(send, off));
    }
  }
  return group_max_u64<G / V>(c[0]);
}

__device__ __forceinline__ double shfl_f64(double v, int src) {
  const uint64_t u = d2u(v);
  const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)u, src, 64);
  const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(u >> 32), src, 64);
  return u2d(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const uint64_t u = d2u(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
  return u2d(((uint64_t)hi << 32) | lo);
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

// Blocks whose quotients may take Markstein's correction (see code2_f64).
__device__ __forceinline__ bool fast_block(double s, int kind) {
  return kind == kScaleExact && s >= 0x1p-900;
}

// e4m3 codes of two elements (first in the low byte) of a block with scale s,
// y = RN(1/s).  In a fast block the quotient is q0 = x y corrected once:
// q = RN(q0 - (q0 s - x) y), Markstein's step, which gives RN(x / s) when the
// residual q0 s - x is exact.  It is exact for |x| >= 2^-968 with a quotient
// of at least 2^-900; with s >= 2^-900 every element whose quotient reaches
// 2^-12 meets both bounds (|x| >= 2^-912).  A smaller quotient is within a
// few ulps of x/s either way, so it stays below 2^-11 through the float32
// rounding and encodes to +-0: the sign is x's (s > 0), set explicitly.
// Other blocks take the IEEE division and the software encoder.
__device__ __forceinline__ uint32_t code2_f64(uint64_t a, uint64_t b, double s, double y, int kind,
                                              bool fast) {
  if (!fast) return code_f64(u2d(a), s, kind) | (code_f64(u2d(b), s, kind) << 8);
  const uint64_t xs[2] = {a, b};
  float q[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const double x = u2d(xs[k]);
    const double q0 = x * y;
    const double t = __builtin_fma(q0, s, -x);
    const float qf = (float)__builtin_fma(-t, y, q0);
    q[k] = u2f((f2u(qf) & 0x7FFFFFFFu) | ((uint32_t)(xs[k] >> 32) & 0x80000000u));
  }
  return cvt_e4m3x2<false>(q[0], q[1], 0u) & 0xFFFFu;  // finite |q| <= 448 sqrt 2
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

// 1xB row blocks (B = 32...2048, powers of two) of a float64 tensor.  Wave instruction i
// reads 128 consecutive doubles of the row-major element sequence (1 KiB when
// the rows are dense; 16 bytes = 2 doubles per lane, never split by a row end
// since cols is even), so a block spans B/2 lanes of one instruction (B < 128)
// or B/128 instructions of all 64 lanes (B >= 128).  PITCHED: rows ld apart,
// element e read at e + (e / cols) (ld - cols).  Each wave runs kF64RowInstr
// instructions (B/128 for 1x1024 and 1x2048); code stores are 2 bytes per
// lane (128 contiguous bytes per wave instruction).
// For B >= 128 a wave holds NI / (B/128) whole blocks: each lane computes the
// scale of one of them (split_max) and the scales reach the whole wave by
// readlane, so the quotient loop runs on wave-uniform s and 1/s.
template <int B, bool PITCHED>
__global__ __launch_bounds__(256) void k_row_f64(Desc single, const Desc* __restrict__ descs,
                                                 const uint32_t* __restrict__ map, int pow2) {
  constexpr int IPB = B >= 128 ? B / 128 : 1;  // instructions per block
  constexpr int LPB = B >= 128 ? 64 : B / 2;   // lanes per block
  constexpr int NI = f64_row_instr(B);
  static_assert(NI % IPB == 0, "a wave holds whole blocks");
  Desc d;
  int64_t u;
  pick_desc<kXcdRunRow>(single, descs, map, d, u);
  const int lane = threadIdx.x & 63;
  const int64_t n = d.rows * d.cols;
  const int64_t w0 = (u * 4 + (threadIdx.x >> 6)) * (NI * 128);  // the wave's first element
  const int64_t e0 = w0 + 2 * lane;                                // this lane's, instruction 0
  const double* in = static_cast<const double*>(d.in);
  // Every lane loads (a lane past the end re-reads the last two elements and
  // drops them), so the loads issue back to back with no branch between.
  // The scheduling barrier keeps the selects that read the first load from
  // being hoisted above the later loads (which would wait on it).
  v4u raw[NI];
  bool ok[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t e = e0 + i * 128;
    ok[i] = e < n;  // n is a multiple of B >= 32: e < n covers e + 1
    const int64_t ee = ok[i] ? e : n - 2;
    raw[i] = load_nt(in + (PITCHED ? ee + (ee / d.cols) * (d.ld - d.cols) : ee));
  }
  __builtin_amdgcn_sched_barrier(0);
  uint64_t x[NI][2];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    x[i][0] = ok[i] ? ((uint64_t)raw[i].y << 32) | raw[i].x : 0;
    x[i][1] = ok[i] ? ((uint64_t)raw[i].w << 32) | raw[i].z : 0;
  }
  if constexpr (B >= 128) {
    constexpr int V = NI / IPB;   // blocks per wave
    constexpr int G = 64 / V;     // lanes holding one block's scale
    uint64_t p[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      p[v] = 0;
#pragma unroll
      for (int j = v * IPB; j < (v + 1) * IPB; ++j)
        p[v] = umax64(p[v], umax64(x[j][0] & kAbs64, x[j][1] & kAbs64));
    }
    double s;
    int kind;
    block_scale_f64(split_max<V, 64>(p, lane), pow2 != 0, s, kind);
    const double y = 1.0 / s;  // correctly rounded
    const int64_t mine = w0 + (lane / G) * B;  // first element of this lane's block
    if (lane % G == 0 && mine < n) gst<double>(static_cast<double*>(d.scales) + mine / B, s);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      if (w0 + v * B >= n) break;  // wave-uniform: blocks are whole
      const double sv = readlane_f64(s, v * G), yv = readlane_f64(y, v * G);
      const int kv = __builtin_amdgcn_readlane(kind, v * G);
      const bool fast = fast_block(sv, kv);
#pragma unroll
      for (int j = v * IPB; j < (v + 1) * IPB; ++j)
        gst_nt<uint16_t>(d.codes + e0 + j * 128,
                         (uint16_t)code2_f64(x[j][0], x[j][1], sv, yv, kv, fast));
    }
  } else {
    // A block spans LPB lanes of one instruction: the NI partials of each
    // LPB-lane group split so that each lane computes one scale (block
    // (lane % LPB) / Q of its group's instructions), which the group's other
    // lanes fetch by shuffle.
    constexpr int Q = LPB / NI;  // lanes holding one block's scale
    uint64_t p[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) p[i] = umax64(x[i][0] & kAbs64, x[i][1] & kAbs64);
    double s;
    int kind;
    block_scale_f64(split_max<NI, LPB>(p, lane), pow2 != 0, s, kind);
    const double y = 1.0 / s;  // correctly rounded
    const int64_t mine = w0 + ((lane % LPB) / Q) * 128 + (lane / LPB) * B;  // this lane's block
    if (lane % Q == 0 && mine < n) gst<double>(static_cast<double*>(d.scales) + mine / B, s);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      if (w0 + i * 128 >= n) break;  // wave-uniform: past the tensor's end
      const int src = (lane / LPB) * LPB + i * Q;
      const double si = shfl_f64(s, src), yi = shfl_f64(y, src);
      const int ki = __shfl(kind, src, 64);
      const int64_t e = e0 + i * 128;  // this lane's elements of instruction i
      if (e < n)
        gst_nt<uint16_t>(d.codes + e, (uint16_t)code2_f64(x[i][0], x[i][1], si, yi, ki, fast_block(si, ki)));
    }
  }
}

// One 128x128 float64 tile held by 512 threads: thread t holds 16-byte chunk
// t % 64 of rows t / 64 + 8 i (i < 16), so each wave instruction reads one whole
// 1 KiB tile row.  FULL tiles load and store unconditionally; an edge tile's
// lanes outside the matrix re-read its first two elements and drop them, so
// the loads still issue back to back.
template <bool FULL>
__device__ __forceinline__ void tile_f64(const Desc& d, int64_t u, int64_t b, int64_t r0, int64_t col,
                                         int pow2, uint64_t* red) {
  constexpr int NL = 16, RS = 8;
  const double* in = static_cast<const double*>(d.in) + b * d.bstride;
  uint8_t* codes = d.codes + b * d.rows * d.cols;
  const int lane = threadIdx.x & 63;
  v4u v[NL];
  if constexpr (FULL) {
    const double* p = in + r0 * d.ld + col;
#pragma unroll
    for (int i = 0; i < NL; ++i) v[i] = load_nt(p + (int64_t)(RS * i) * d.ld);
  } else {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const bool ok = col < d.cols && r0 + RS * i < d.rows;
      v[i] = load_nt(in + (ok ? (r0 + RS * i) * d.ld + col : 0));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NL; ++i)
      if (!(col < d.cols && r0 + RS * i < d.rows)) v[i] = v4u{0u, 0u, 0u, 0u};
  }
  uint64_t a = 0;
#pragma unroll
  for (int i = 0; i < NL; ++i)
    a = umax64(a, umax64((((uint64_t)v[i].y << 32) | v[i].x) & kAbs64,
                         (((uint64_t)v[i].w << 32) | v[i].z) & kAbs64));
  a = group_max_u64<64>(a);
  if (lane == 0) red[threadIdx.x >> 6] = a;
  __syncthreads();
  a = red[0];
#pragma unroll
  for (int w = 1; w < 8; ++w) a = umax64(a, red[w]);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  double s;
  int kind;
  block_scale_f64(((uint64_t)hi << 32) | lo, pow2 != 0, s, kind);
  if (threadIdx.x == 0) gst<double>(static_cast<double*>(d.scales) + u, s);
  const bool fast = fast_block(s, kind);
  const double y = fast ? 1.0 / s : 0.0;
  uint8_t* q = codes + r0 * d.cols + col;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const uint32_t c = code2_f64(((uint64_t)v[i].y << 32) | v[i].x, ((uint64_t)v[i].w << 32) | v[i].z,
                                 s, y, kind, fast);
    if (FULL || (col < d.cols && r0 + RS * i < d.rows)) gst_nt<uint16_t>(q + (int64_t)(RS * i) * d.cols, (uint16_t)c);
  }
}

// 128x128 tiles of a float64 tensor (the vLLM/ATOM tile layout, in float64
// arithmetic): one 512-thread work-group per tile; the tile stays in VGPRs,
// one LDS step joins the eight waves' maxima, and s, 1/s are tile-uniform.
__global__ __launch_bounds__(512) void k_tile_f64(Desc single, const Desc* __restrict__ descs,
                                                  const uint32_t* __restrict__ map, int pow2) {
  __shared__ uint64_t red[8];
  Desc d;
  int64_t u;
  pick_desc<kXcdRunTileF64>(single, descs, map, d, u);
  const int64_t per = d.units_r * d.units_c;
  const int64_t b = u / per;
  const int64_t rem = u - b * per;
  const int64_t tr = rem / d.units_c, tc = rem - tr * d.units_c;
  const int64_t r0 = tr * 128 + (threadIdx.x >> 6);
  const int64_t col = tc * 128 + 2 * (threadIdx.x & 63);  // cols is even: col < cols covers col + 1
  if (tr * 128 + 128 <= d.rows && tc * 128 + 128 <= d.cols) tile_f64<true>(d, u, b, r0, col, pow2, red);
  else tile_f64<false>(d, u, b, r0, col, pow2, red);
}

// 1xB blocks of a float64 tensor for the widths neither k_row_f64 nor
// k_row_pad_f64 takes (128 < B <= 16384 but the powers of two to 2048, and
// B = 2..4): ceil(B/2) chunks of 2 doubles (16
// bytes), the last starting at B - 2 when B is odd (it overlaps its
// neighbour: the amax ignores the repeat, and both lanes write the same
// codes).  As k_row_wide: W waves per block (1 up to B = 1024, 4 up to 4096,
// then a 512- or 1024-thread work-group of 8 or 16 waves up to 16384), lane l
// of wave w holding chunks 64 w + l + 64 W k for k < K = ceil(g / 64W) <= 8;
// with W = 1 a wave takes P consecutive blocks.  Lanes past a block's end,
// and slots past K, re-load its first chunk and drop out of the amax, so the
// loads issue without branches.  Quotients as in k_row_f64 (Markstein's step in
// fast blocks, IEEE division otherwise).
template <int W, int P>
__global__ __launch_bounds__(W > 4 ? 64 * W : 256) void k_row_wide_f64(Desc single, const Desc* __restrict__ descs,
                                                                       const uint32_t* __restrict__ map, int pow2,
                                                                       int bw) {
  static_assert(W == 1 || P == 1, "blocks of several waves: one block per wave group");
  constexpr int WAVES = W > 4 ? W : 4;  // waves per work-group
  constexpr int KP = 8 / P;  // chunk slots per block
  __shared__ uint64_t red[WAVES];
  Desc d;
  int64_t u;
  pick_desc<kXcdRunRow>(single, descs, map, d, u);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = (bw + 1) / 2;  // chunks per block
  const int K = (g + 64 * W - 1) / (64 * W);
  const int64_t blk0 = (u * (WAVES / W) + wave / W) * P;
  const int c0 = 64 * (wave % W) + lane;
  const double* in = static_cast<const double*>(d.in);

  bool live[P];
  int64_t gb[P];
  v4u raw[P][KP];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    live[p] = blk0 + p < d.nblocks;  // the same for the W waves of a block
    gb[p] = live[p] ? blk0 + p : d.nblocks - 1;
    const int64_t row = gb[p] / d.bpr;
    const int64_t base = row * d.ld + (gb[p] - row * d.bpr) * bw;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
      // every slot loads (past the block's chunks: its first chunk again, an
      // L2 hit), so the loads carry no branches and issue back to back
      const int c = c0 + 64 * W * k;
      const bool ok = k < K && c < g;
      raw[p][k] = load_nt(in + base + (ok ? (2 * c > bw - 2 ? bw - 2 : 2 * c) : 0));
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  uint64_t am[P];  // block maxima, wave-uniform
#pragma unroll
  for (int p = 0; p < P; ++p) {
    uint64_t a = 0;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
      const bool ok = k < K && c0 + 64 * W * k < g;
      const uint64_t m = umax64((((uint64_t)raw[p][k].y << 32) | raw[p][k].x) & kAbs64,
                                (((uint64_t)raw[p][k].w << 32) | raw[p][k].z) & kAbs64);
      a = umax64(a, ok ? m : 0);
    }
    a = group_max_u64<64>(a);
    if constexpr (W > 1) {
      if (lane == 0) red[wave] = a;
      __syncthreads();
      const int w0 = wave & ~(W - 1);
#pragma unroll
      for (int w = 0; w < W; ++w) a = umax64(a, red[w0 + w]);
    }
    am[p] = a;
  }
  // one pass of the float64 scale math for all P blocks: lane p computes block
  // p's scale and 1/s, which readlane hands to the whole wave
  uint64_t mine = am[0];
#pragma unroll
  for (int p = 1; p < P; ++p) mine = (lane % P) == p ? am[p] : mine;
  double s_l;
  int kind_l;
  block_scale_f64(mine, pow2 != 0, s_l, kind_l);
  const double y_l = 1.0 / s_l;  // correctly rounded
#pragma unroll
  for (int p = 0; p < P; ++p) {
    if (!live[p]) continue;
    const double s = readlane_f64(s_l, p), y = readlane_f64(y_l, p);
    const int kind = __builtin_amdgcn_readlane(kind_l, p);
    const bool fast = fast_block(s, kind);
    if (c0 == 0) gst<double>(static_cast<double*>(d.scales) + gb[p], s);
#pragma unroll
    for (int k = 0; k < KP; ++k) {
      const int c = c0 + 64 * W * k;
      if (k < K && c < g) {
        const int64_t off = 2 * c > bw - 2 ? bw - 2 : 2 * c;
        const uint64_t x0 = ((uint64_t)raw[p][k].y << 32) | raw[p][k].x;
        const uint64_t x1 = ((uint64_t)raw[p][k].w << 32) | raw[p][k].z;
        store_nt2(d.codes + gb[p] * bw + off, (uint16_t)code2_f64(x0, x1, s, y, kind, fast));
      }
      // one chunk's quotients at a time: interleaving all of them would take
      // four times the registers (occupancy 2)
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// 1xB blocks of a float64 tensor, 5 <= B < 128 (other than 32 and 64, which
// k_row_f64 takes): a block's g = ceil(B/2) chunks of 2 doubles sit on an
// aligned group of L = nextpow2(g) lanes (the last chunk starting at B - 2 when
// B is odd), so a wave instruction holds 64/L blocks and a lane runs
// kF64RowInstr instructions, each on the next 64/L blocks.  Lanes past g
// re-load their block's first chunk and drop out of the amax, so the loads
// issue without branches.  split_max leaves each lane the maximum of one of
// its group's blocks; the group's other lanes fetch that scale by shuffle.
// Quotients as in k_row_f64.
template <int L>
__global__ __launch_bounds__(256) void k_row_pad_f64(Desc single, const Desc* __restrict__ descs,
                                                     const uint32_t* __restrict__ map, int pow2, int bw) {
  constexpr int NI = kF64RowInstr;  // instructions per lane
  constexpr int BPI = 64 / L;       // blocks per wave instruction
  constexpr int Q = L / NI;         // lanes holding one block's scale
  static_assert(L >= NI && L <= 64, "a lane group holds one scale per instruction");
  Desc d;
  int64_t u;
  pick_desc<kXcdRunRow>(single, descs, map, d, u);
  const int lane = threadIdx.x & 63;
  const int g = (bw + 1) / 2;  // chunks per block
  const int c = lane % L;      // this lane's chunk of its block
  const int off = c < g ? (2 * c > bw - 2 ? bw - 2 : 2 * c) : 0;
  const int64_t b0 = (u * 4 + (threadIdx.x >> 6)) * (NI * BPI) + lane / L;  // block, instruction 0
  const double* in = static_cast<const double*>(d.in);
  v4u raw[NI];
  bool ok[NI];
  int64_t blk[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t b = b0 + i * BPI;
    ok[i] = c < g && b < d.nblocks;
    blk[i] = b < d.nblocks ? b : d.nblocks - 1;
    int64_t base;
    if (d.ld == d.cols) {
      base = blk[i] * bw;
    } else {
      const int64_t row = blk[i] / d.bpr;
      base = row * d.ld + (blk[i] - row * d.bpr) * bw;
    }
    raw[i] = load_nt(in + base + off);
  }
  __builtin_amdgcn_sched_barrier(0);
  uint64_t p[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const uint64_t m = umax64((((uint64_t)raw[i].y << 32) | raw[i].x) & kAbs64,
                              (((uint64_t)raw[i].w << 32) | raw[i].z) & kAbs64);
    p[i] = ok[i] ? m : 0;
  }
  double s;
  int kind;
  block_scale_f64(split_max<NI, L>(p, lane), pow2 != 0, s, kind);  // block of instruction c / Q
  const double y = 1.0 / s;  // correctly rounded
  const int64_t mine = b0 + (c / Q) * BPI;
  if (c % Q == 0 && mine < d.nblocks) gst<double>(static_cast<double*>(d.scales) + mine, s);
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int src = (lane / L) * L + i * Q;
    const double si = shfl_f64(s, src), yi = shfl_f64(y, src);
    const int ki = __shfl(kind, src, 64);
    if (ok[i]) {
      const uint64_t x0 = ((uint64_t)raw[i].y << 32) | raw[i].x;
      const uint64_t x1 = ((uint64_t)raw[i].w << 32) | raw[i].z;
      store_nt2(d.codes + blk[i] * bw + off, (uint16_t)code2_f64(x0, x1, si, yi, ki, fast_block(si, ki)));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

hipError_t launch_f64(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                      const uint32_t* map, int64_t units, hipStream_t stream) {
  const dim3 grid((unsigned)units), block(256);
  if (cfg.kernel == kKernF64Row) {
    if (cfg.pitched) {
      switch (cfg.blk_c) {
        case 32: hipLaunchKernelGGL((k_row_f64<32, true>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 64: hipLaunchKernelGGL((k_row_f64<64, true>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 128: hipLaunchKernelGGL((k_row_f64<128, true>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 256: hipLaunchKernelGGL((k_row_f64<256, true>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 512: hipLaunchKernelGGL((k_row_f64<512, true>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 1024: hipLaunchKernelGGL((k_row_f64<1024, true>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 2048: hipLaunchKernelGGL((k_row_f64<2048, true>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        default: return hipErrorInvalidValue;
      }
    } else {
      switch (cfg.blk_c) {
        case 32: hipLaunchKernelGGL((k_row_f64<32, false>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 64: hipLaunchKernelGGL((k_row_f64<64, false>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 128: hipLaunchKernelGGL((k_row_f64<128, false>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 256: hipLaunchKernelGGL((k_row_f64<256, false>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 512: hipLaunchKernelGGL((k_row_f64<512, false>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 1024: hipLaunchKernelGGL((k_row_f64<1024, false>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        case 2048: hipLaunchKernelGGL((k_row_f64<2048, false>), grid, block, 0, stream, single, descs, map, cfg.pow2); break;
        default: return hipErrorInvalidValue;
      }
    }
    return hipGetLastError();
  }
  if (cfg.kernel == kKernF64Wide) {
    const int bw = cfg.blk_c;
    switch (f64_pad_lanes(cfg.blk_c)) {
      case 4: hipLaunchKernelGGL((k_row_pad_f64<4>), grid, block, 0, stream, single, descs, map, cfg.pow2, bw); return hipGetLastError();
      case 8: hipLaunchKernelGGL((k_row_pad_f64<8>), grid, block, 0, stream, single, descs, map, cfg.pow2, bw); return hipGetLastError();
      case 16: hipLaunchKernelGGL((k_row_pad_f64<16>), grid, block, 0, stream, single, descs, map, cfg.pow2, bw); return hipGetLastError();
      case 32: hipLaunchKernelGGL((k_row_pad_f64<32>), grid, block, 0, stream, single, descs, map, cfg.pow2, bw); return hipGetLastError();
      case 64: hipLaunchKernelGGL((k_row_pad_f64<64>), grid, block, 0, stream, single, descs, map, cfg.pow2, bw); return hipGetLastError();
      default: break;
    }
    switch (f64_wide_blocks_per_wave(cfg.blk_c)) {
      case 4: hipLaunchKernelGGL((k_row_wide_f64<1, 4>), grid, block, 0, stream, single, descs, map, cfg.pow2, bw); break;
      case 2: hipLaunchKernelGGL((k_row_wide_f64<1, 2>), grid, block, 0, stream, single, descs, map, cfg.pow2, bw); break;
      case 1: hipLaunchKernelGGL((k_row_wide_f64<1, 1>), grid, block, 0, stream, single, descs, map, cfg.pow2, bw); break;
      default: {  // one block of W = threads / 64 waves
        const dim3 wg(wg_threads(kKernF64Wide, kF64, cfg.blk_c));
        if (wg.x == 256)
          hipLaunchKernelGGL((k_row_wide_f64<4, 1>), grid, wg, 0, stream, single, descs, map, cfg.pow2, bw);
        else if (wg.x == 512)
          hipLaunchKernelGGL((k_row_wide_f64<8, 1>), grid, wg, 0, stream, single, descs, map, cfg.pow2, bw);
        else
          hipLaunchKernelGGL((k_row_wide_f64<16, 1>), grid, wg, 0, stream, single, descs, map, cfg.pow2, bw);
        break;
      }
    }
    return hipGetLastError();
  }
  if (cfg.kernel == kKernF64Tile) {
    hipLaunchKernelGGL(k_tile_f64, grid, dim3(512), 0, stream, single, descs, map, cfg.pow2);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(k_f64, grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.blk_r, cfg.blk_c);
  return hipGetLastError();
}

}  // namespace lrq
