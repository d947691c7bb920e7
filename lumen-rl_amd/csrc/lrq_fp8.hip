// FP8 E4M3 blockwise quantization kernels (gfx950, wave64).
//
// Restates WeightQuantizer.quantize_tensor
// (lumenrl/quantization/weight_quantizer.py:40-77): per block amax -> /448 ->
// clamp(tiny) -> [pow2] -> x/s -> float8_e4m3fn, in one HBM pass (bf16 in,
// e4m3 + scale out).  Five kernels:
//   k_tile128  : 128x128 tiles (the vLLM/ATOM `weight_scale_inv` layout), one
//                512-thread work-group per tile, the tile held in VGPRs;
//                tiles handed to XCDs in runs of 4 or 8 by row pitch
//                (pick_desc_tile).
//   k_row      : 1xB row blocks (the reference's own layout), ceil(B/8)
//                consecutive lanes per block (padded to a power of two) so
//                every wave instruction is one contiguous span; one scale
//                computation per lane, shared by shuffles.
//   k_row_f32  : the same for float32 input, one 16-byte load per 4 elements.
//   k_row_wide : 1xB row blocks wider than 512 (but 1024 and 2048) up to
//                65536, 1 to 16 waves per block, the block held in VGPRs.
//   k_generic  : any block shape, stride or alignment (one work-group per
//                block, scalar loads); the fallback for odd inputs.
// All of them share lrq_device.hpp's block_scale / block_quot / special_code.
#include "lrq_device.hpp"
#include "lrq_internal.hpp"

namespace lrq {

// 8 consecutive input elements.
template <int DT>
struct Chunk {
  static constexpr int kWords = DT == kF32 ? 8 : 4;
  uint32_t w[kWords];
};

template <int DT>
__device__ __forceinline__ void load_chunk(Chunk<DT>& c, const void* base, int64_t off) {
  if constexpr (DT == kF32) {
    const float* p = static_cast<const float*>(base) + off;
    const v4u a = load_nt(p), b = load_nt(p + 4);
    c.w[0] = a.x; c.w[1] = a.y; c.w[2] = a.z; c.w[3] = a.w;
    c.w[4] = b.x; c.w[5] = b.y; c.w[6] = b.z; c.w[7] = b.w;
  } else {
    const v4u a = load_nt(static_cast<const uint16_t*>(base) + off);
    c.w[0] = a.x; c.w[1] = a.y; c.w[2] = a.z; c.w[3] = a.w;
  }
}

template <int DT>
__device__ __forceinline__ void zero_chunk(Chunk<DT>& c) {
#pragma unroll
  for (int i = 0; i < Chunk<DT>::kWords; ++i) c.w[i] = 0u;
}

template <int DT>
__device__ __forceinline__ float elem(const Chunk<DT>& c, int i) {
  if constexpr (DT == kF32) return u2f(c.w[i]);
  else if constexpr (DT == kBF16) return (i & 1) ? bf16_hi(c.w[i >> 1]) : bf16_lo(c.w[i >> 1]);
  else return f16_to_f32((i & 1) ? (c.w[i >> 1] >> 16) : (c.w[i >> 1] & 0xFFFFu));
}

// Running amax: 16-bit inputs keep packed u16 maxima of |bits|, float32 keeps
// the max of |bits|.  Magnitude bit patterns order like the values, with NaN
// above inf, so integer max is an exact, NaN-detecting amax.
template <int DT>
struct Amax {
  u16x2 m16;
  uint32_t m32;
  __device__ __forceinline__ void init() { m16 = u16x2{0, 0}; m32 = 0u; }
  __device__ __forceinline__ void add(const Chunk<DT>& c) {
    if constexpr (DT == kF32) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t a = c.w[i] & 0x7FFFFFFFu;
        m32 = a > m32 ? a : m32;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) m16 = amax_bf16x2(m16, c.w[i]);
    }
  }
  // float32 bits of the amax (non-negative)
  __device__ __forceinline__ uint32_t bits() const {
    if constexpr (DT == kF32) return m32;
    uint32_t a = m16.x > m16.y ? m16.x : m16.y;
    if constexpr (DT == kBF16) return a << 16;
    return f2u(f16_to_f32(a));
  }
};

// 8 elements -> 8 e4m3 bytes (element 0 lowest).
template <int DT, int CDT>
__device__ __forceinline__ v2u encode_chunk(const Chunk<DT>& c, const BlockScale& b) {
  v2u r;
  if (b.kind == kScaleFast) {
    float q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = block_quot<CDT>(elem<DT>(c, i), b);
    r.x = cvt_e4m3x4(q[0], q[1], q[2], q[3]);
    r.y = cvt_e4m3x4(q[4], q[5], q[6], q[7]);
  } else if (b.kind == kScaleExact) {
    float q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = block_quot<CDT>(elem<DT>(c, i), b);
    r.x = cvt_e4m3x4(q[0], q[1], q[2], q[3]);
    r.y = cvt_e4m3x4(q[4], q[5], q[6], q[7]);
  } else {
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo |= special_code<CDT>(elem<DT>(c, i), b) << (8 * i);
      hi |= special_code<CDT>(elem<DT>(c, i + 4), b) << (8 * i);
    }
    r.x = lo;
    r.y = hi;
  }
  return r;
}

template <int CDT>
__device__ __forceinline__ void store_scale(void* scales, int64_t idx, float s, int scale_bf16) {
  if (CDT == kF32 && !scale_bf16) {
    gst<float>(static_cast<float*>(scales) + idx, s);
  } else {
    uint32_t h = (CDT == kF16) ? f16_bits(s) : bf16_bits(s);
    gst<uint16_t>(static_cast<uint16_t*>(scales) + idx, (uint16_t)h);
  }
}

// ---------------------------------------------------------------------------
// 128x128 tiles, T = kTileThreads threads per tile.  Thread t owns column
// chunk (t & 15) of rows (t >> 4) + (T/16) i: each load instruction of a wave
// reads 4 full 256-byte rows.  T = 512 (4 loads per thread) beats 256 (8
// loads) by 1-4% on large launches and by 5% on a single 4096^2 weight; 1024
// (2 loads) loses 15% to its 16-wave reduction.
// ---------------------------------------------------------------------------
template <int DT, int CDT, int T>
__global__ __launch_bounds__(T) void k_tile128(Desc single, const Desc* __restrict__ descs,
                                               const uint32_t* __restrict__ map, int pow2,
                                               int scale_bf16) {
  constexpr int NL = 2048 / T;  // 16-byte chunks per thread
  constexpr int RS = T / 16;    // rows between a thread's chunks
  __shared__ uint32_t red[T / 64];
  Desc d;
  int64_t u;
  pick_desc_tile(single, descs, map, d, u);

  const int64_t per = d.units_r * d.units_c;
  const int64_t b = u / per;
  const int64_t rem = u - b * per;
  const int64_t tr = rem / d.units_c;
  const int64_t tc = rem - tr * d.units_c;
  const int64_t r0 = tr * 128, c0 = tc * 128;
  const int tid = threadIdx.x;
  const int64_t col = c0 + (tid & 15) * 8;
  const int rr = tid >> 4;
  const int64_t in_base = b * d.bstride + (r0 + rr) * d.ld + col;
  const int64_t out_base = (b * d.rows + r0 + rr) * d.cols + col;
  const bool full = (r0 + 128 <= d.rows) && (c0 + 128 <= d.cols);
  const bool col_ok = col < d.cols;

  Chunk<DT> ch[NL];
  if (full) {
#pragma unroll
    for (int i = 0; i < NL; ++i) load_chunk<DT>(ch[i], d.in, in_base + (int64_t)(RS * i) * d.ld);
  } else {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if (col_ok && r0 + rr + RS * i < d.rows) load_chunk<DT>(ch[i], d.in, in_base + (int64_t)(RS * i) * d.ld);
      else zero_chunk<DT>(ch[i]);
    }
  }

  Amax<DT> am;
  am.init();
#pragma unroll
  for (int i = 0; i < NL; ++i) am.add(ch[i]);
  uint32_t a = group_max<64>(am.bits());  // DPP within rows of 16, two shuffles across
  if ((tid & 63) == 0) red[tid >> 6] = a;
  __syncthreads();
  a = red[0];
#pragma unroll
  for (int w = 1; w < T / 64; ++w) a = red[w] > a ? red[w] : a;
  a = __builtin_amdgcn_readfirstlane(a);  // tile-uniform: scalar scale math

  const BlockScale bs = block_scale<CDT>(a, pow2 != 0);
  if (tid == 0) store_scale<CDT>(d.scales, u, bs.s, scale_bf16);

#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const v2u q = encode_chunk<DT, CDT>(ch[i], bs);
    if (full || (col_ok && r0 + rr + RS * i < d.rows))
      store_nt(d.codes + out_base + (int64_t)(RS * i) * d.cols, q);
  }
}

// ---------------------------------------------------------------------------
// 1xB row blocks (B = 8*LPB, LPB = 1..64 lanes per block).  The 64 lanes of a
// wave cover 64 consecutive 8-element chunks, so each load instruction reads
// one contiguous span (1 KiB of bf16) and each store writes whole 128-byte
// code lines; lane c of a block holds chunk c of it.  Instruction j of wave w
// covers blocks (NJ w + j) * (64 / LPB) + lane / LPB of the work-group, with
// NJ = kRowBlocks blocks per lane.
// The block amax is reduced over its LPB lanes (DPP within 16 lanes, shuffles
// beyond).  Each lane then computes the scale of ONE of its NJ blocks and
// the NJ scales are exchanged by shuffles, so the IEEE divisions cost one
// pair per lane instead of NJ.  Rows are folded over the batch by the host.
// LPB = 1 or 2 (1x8, 1x16) gives every lane its own blocks' scales.
// PAD takes the other widths B = 9..512: a block is g = ceil(B/8) chunks in the
// LPB-lane group of the next power of two (2 at least), whose last LPB - g
// lanes idle, so the same DPP reductions apply (padding beat a segmented
// reduction over exactly g lanes in 16 of 18 width x dtype cases).  When 8
// does not divide B the last chunk starts at B - 8, overlapping its
// neighbour: the amax is unchanged by the repeat, and both lanes write the
// same codes to the shared bytes.  IPB = 2 or 4 takes 1x1024 and 1x2048
// blocks, each spanning IPB of a wave's instructions.
// ---------------------------------------------------------------------------
template <int DT, int CDT, int LPB, bool PAD = false, int IPB = 1>
__global__ __launch_bounds__(256) void k_row(Desc single, const Desc* __restrict__ descs,
                                             const uint32_t* __restrict__ map, int pow2,
                                             int scale_bf16, int bw = 0) {
  // PAD: blocks of bw elements, g = ceil(bw/8) <= LPB chunks, in LPB-lane
  // groups whose last LPB - g lanes idle.  IPB > 1: blocks of 512 IPB elements
  // spanning IPB consecutive wave instructions of all 64 lanes (1x1024, 1x2048).
  static_assert(IPB == 1 || (LPB == 64 && !PAD && kRowBlocks % IPB == 0), "whole blocks per wave");
  const int B = PAD ? bw : 8 * LPB * IPB;  // elements per block
  const int G = PAD ? (bw + 7) / 8 : LPB;  // lanes holding a chunk of the block
  constexpr int BPI = 64 / LPB;       // blocks per wave instruction
  constexpr int NJ = kRowBlocks;      // wave instructions (chunks per lane)
  constexpr int NB = NJ / IPB;        // blocks per lane
  Desc d;
  int64_t u;
  pick_desc<kXcdRunRow>(single, descs, map, d, u);
  const int tid = threadIdx.x, lane = tid & 63;
  const int c = lane & (LPB - 1);     // chunk of the block held by this lane
  const int64_t wb = u * (4 * NB * BPI) + (tid >> 6) * (NB * BPI) + lane / LPB;  // block at j = 0

  Chunk<DT> ch[NJ];
  bool ok[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t gb = wb + (j / IPB) * BPI;
    const int64_t part = (j % IPB) * 512 + (PAD && c * 8 > B - 8 ? B - 8 : c * 8);  // element of the block
    ok[j] = (!PAD || c < G) && gb < d.nblocks;
    if (ok[j]) {
      int64_t off;
      if (d.ld == d.cols) {
        off = gb * B + part;
      } else {
        const int64_t row = gb / d.bpr;
        off = row * d.ld + (gb - row * d.bpr) * B + part;
      }
      load_chunk<DT>(ch[j], d.in, off);
    } else {
      zero_chunk<DT>(ch[j]);
    }
  }
  uint32_t am[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    Amax<DT> a;
    a.init();
#pragma unroll
    for (int j = k * IPB; j < (k + 1) * IPB; ++j) a.add(ch[j]);
    am[k] = group_max<LPB>(a.bits());  // every lane takes part: groups never straddle
  }
  BlockScale bs[NB];
  if constexpr (LPB < NB) {
    // 1x8 / 1x16: fewer lanes per block than blocks per lane; each lane
    // computes its own NB scales
#pragma unroll
    for (int k = 0; k < NB; ++k) bs[k] = block_scale<CDT>(am[k], pow2 != 0);
  } else {
    // lane c computes the scale of block k = c % NB of its group; gather all NB
    uint32_t mine = am[0];
#pragma unroll
    for (int k = 1; k < NB; ++k) mine = (c % NB) == k ? am[k] : mine;
    const BlockScale own = block_scale<CDT>(mine, pow2 != 0);
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int src = (lane & ~(LPB - 1)) | k;  // idle PAD lanes hold the group max too
      bs[k].s = __shfl(own.s, src, 64);
      bs[k].y = __shfl(own.y, src, 64);
      bs[k].kind = __shfl(own.kind, src, 64);
    }
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (!ok[j]) continue;
    const int64_t gb = wb + (j / IPB) * BPI;
    if (c == 0 && j % IPB == 0) store_scale<CDT>(d.scales, gb, bs[j / IPB].s, scale_bf16);
    const int64_t part = (j % IPB) * 512 + (PAD && c * 8 > B - 8 ? B - 8 : c * 8);
    store_nt(d.codes + gb * B + part, encode_chunk<DT, CDT>(ch[j], bs[j / IPB]));
  }
}

// ---------------------------------------------------------------------------
// 1xB row blocks of float32 input (B = 8...1024): a lane's chunk is one
// 16-byte load of 4 floats, so each wave instruction reads 1 KiB contiguous
// (k_row's 8-element chunks of float32 take two loads at a 32-byte stride,
// each instruction covering a 2 KiB span at half density).  A block spans
// LPB = B/4 lanes of one instruction (B <= 256) or all 64 lanes of IPB
// instructions (B = 512, 1024); NJ = kRowBlocks instructions per wave, one
// scale computation per lane as in k_row.
// ---------------------------------------------------------------------------
template <int LPB, int IPB>
__global__ __launch_bounds__(256) void k_row_f32(Desc single, const Desc* __restrict__ descs,
                                                 const uint32_t* __restrict__ map, int pow2,
                                                 int scale_bf16) {
  static_assert(IPB == 1 || LPB == 64, "multi-instruction blocks span the whole wave");
  constexpr int NJ = kRowBlocks;      // wave instructions (chunks per lane)
  static_assert(NJ % IPB == 0, "whole blocks per wave");
  constexpr int B = 4 * LPB * IPB;    // elements per block
  constexpr int BPI = 64 / LPB;       // blocks per wave instruction
  constexpr int NB = NJ / IPB;        // blocks per lane
  Desc d;
  int64_t u;
  pick_desc<kXcdRunRow>(single, descs, map, d, u);
  const int tid = threadIdx.x, lane = tid & 63;
  const int c = lane & (LPB - 1);     // chunk of the block held by this lane
  const int64_t wb = u * (4 * NB * BPI) + (tid >> 6) * (NB * BPI) + lane / LPB;  // block at j = 0
  const float* in = static_cast<const float*>(d.in);

  v4u v[NJ];
  bool ok[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t gb = wb + (j / IPB) * BPI;
    const int64_t part = (j % IPB) * 256 + c * 4;  // element of the block
    ok[j] = gb < d.nblocks;
    if (ok[j]) {
      int64_t off;
      if (d.ld == d.cols) {
        off = gb * B + part;
      } else {
        const int64_t row = gb / d.bpr;
        off = row * d.ld + (gb - row * d.bpr) * B + part;
      }
      v[j] = load_nt(in + off);
    } else {
      v[j] = v4u{0u, 0u, 0u, 0u};
    }
  }
  uint32_t am[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    uint32_t a = 0u;
#pragma unroll
    for (int j = k * IPB; j < (k + 1) * IPB; ++j) {
      const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t m = w[i] & 0x7FFFFFFFu;
        a = m > a ? m : a;
      }
    }
    am[k] = group_max<LPB>(a);
  }
  BlockScale bs[NB];
  if constexpr (LPB < NB) {
    // 1x8: two lanes per block, each lane computes its own NB scales
#pragma unroll
    for (int k = 0; k < NB; ++k) bs[k] = block_scale<kF32>(am[k], pow2 != 0);
  } else {
    uint32_t mine = am[0];
#pragma unroll
    for (int k = 1; k < NB; ++k) mine = (c % NB) == k ? am[k] : mine;
    const BlockScale own = block_scale<kF32>(mine, pow2 != 0);
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int src = (lane & ~(LPB - 1)) | k;
      bs[k].s = __shfl(own.s, src, 64);
      bs[k].y = __shfl(own.y, src, 64);
      bs[k].kind = __shfl(own.kind, src, 64);
    }
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (!ok[j]) continue;
    const int64_t gb = wb + (j / IPB) * BPI;
    const BlockScale& b = bs[j / IPB];
    const float x[4] = {u2f(v[j].x), u2f(v[j].y), u2f(v[j].z), u2f(v[j].w)};
    uint32_t code;
    if (b.kind <= kScaleExact) {
      code = cvt_e4m3x4(block_quot<kF32>(x[0], b), block_quot<kF32>(x[1], b),
                        block_quot<kF32>(x[2], b), block_quot<kF32>(x[3], b));
    } else {
      code = special_code<kF32>(x[0], b) | (special_code<kF32>(x[1], b) << 8) |
             (special_code<kF32>(x[2], b) << 16) | (special_code<kF32>(x[3], b) << 24);
    }
    if (c == 0 && j % IPB == 0) store_scale<kF32>(d.scales, gb, b.s, scale_bf16);
    store_nt(d.codes + gb * B + (j % IPB) * 256 + c * 4, code);
  }
}

// ---------------------------------------------------------------------------
// Wide 1xB row blocks, 512 < B <= 65536 (other than 1024 and 2048, which
// k_row takes), in g = ceil(B/8) chunks: a block belongs to W waves of the
// work-group (W = 1, 2 or 4 of a 256-thread work-group; 8 or 16 waves, the
// whole work-group, past B = 16384), whose lane l of wave w holds chunks
// c = 64 w + l + 64 W k for k < K = ceil(g / 64W).  When 8 does not divide B
// the last chunk starts at B - 8, overlapping its neighbour (the amax ignores
// the repeat; both lanes write the same codes).  A lane has NC chunk slots
// (4 or 8); with W = 1 a wave takes P = NC/KP consecutive blocks of
// KP = nextpow2(K) slots each, so it keeps about NC loads in flight per lane
// whatever the width.  Every wave
// instruction of a block reads 1 KiB contiguous (of bf16), except the last
// when 64 W does not divide g: its lanes past the end, and every slot past K,
// re-load chunk 0 of their block (in bounds, an L2 hit) and drop out of the
// amax, so no branch separates the loads.  The W waves' maxima meet in LDS;
// the scale math then runs once per block.
// ---------------------------------------------------------------------------
template <int DT, int CDT, int W, int P, int NC>
__global__ __launch_bounds__(W > 4 ? 64 * W : 256) void k_row_wide(Desc single, const Desc* __restrict__ descs,
                                                                   const uint32_t* __restrict__ map, int pow2,
                                                                   int scale_bf16, int bw) {
  static_assert(W == 1 || P == 1, "blocks of several waves: one block per wave group");
  constexpr int WAVES = W > 4 ? W : 4;  // waves per work-group
  const int g = (bw + 7) / 8;  // chunks per block
  constexpr int KP = NC / P;  // chunk slots per block
  __shared__ uint32_t red[WAVES];
  Desc d;
  int64_t u;
  pick_desc<kXcdRunRow>(single, descs, map, d, u);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = (g + 64 * W - 1) / (64 * W);  // <= KP
  const int64_t blk0 = (u * (WAVES / W) + wave / W) * P;
  const int64_t B = bw;
  const int c0 = 64 * (wave % W) + lane;

  bool live[P];
  int64_t gb[P];
  Chunk<DT> ch[P][KP];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    live[p] = blk0 + p < d.nblocks;  // the same for the W waves of a block
    gb[p] = live[p] ? blk0 + p : d.nblocks - 1;
    int64_t base;
    if (d.ld == d.cols) {
      base = gb[p] * B;
    } else {
      const int64_t row = gb[p] / d.bpr;
      base = row * d.ld + (gb[p] - row * d.bpr) * B;
    }
#pragma unroll
    for (int k = 0; k < KP; ++k) {
      // every slot loads (past the block's chunks: its first chunk again, an L2
      // hit), so no branch separates the loads (1x640: 56 -> 67 %)
      const int c = c0 + 64 * W * k;
      const bool ok = k < K && c < g;
      load_chunk<DT>(ch[p][k], d.in, base + (ok ? (8 * c > bw - 8 ? bw - 8 : 8 * c) : 0));
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  BlockScale bs[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    Amax<DT> am;
    am.init();
#pragma unroll
    for (int k = 0; k < KP; ++k) {
      if (k < K && c0 + 64 * W * k < g) am.add(ch[p][k]);
    }
    uint32_t a = group_max<64>(am.bits());
    if constexpr (W > 1) {
      if (lane == 0) red[wave] = a;
      __syncthreads();
      const int w0 = wave & ~(W - 1);
#pragma unroll
      for (int w = 0; w < W; ++w) a = red[w0 + w] > a ? red[w0 + w] : a;
    }
    a = __builtin_amdgcn_readfirstlane(a);  // block-uniform: scalar scale math
    bs[p] = block_scale<CDT>(a, pow2 != 0);
  }
#pragma unroll
  for (int p = 0; p < P; ++p) {
    if (!live[p]) continue;
    if (c0 == 0) store_scale<CDT>(d.scales, gb[p], bs[p].s, scale_bf16);
#pragma unroll
    for (int k = 0; k < KP; ++k) {
      const int c = c0 + 64 * W * k;
      if (k < K && c < g)
        store_nt(d.codes + gb[p] * B + (8 * c > bw - 8 ? bw - 8 : 8 * c), encode_chunk<DT, CDT>(ch[p][k], bs[p]));
    }
  }
}

// ---------------------------------------------------------------------------
// Generic: one work-group per block of any shape; scalar loads; edge blocks
// partial.  Unit u = (b, tile row, tile col) row-major = the scale index.
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float load_elem(const void* base, int64_t off) {
  if constexpr (DT == kF32) return gld<float>(static_cast<const float*>(base) + off);
  else if constexpr (DT == kBF16) return u2f((uint32_t)gld<uint16_t>(static_cast<const uint16_t*>(base) + off) << 16);
  else return f16_to_f32(gld<uint16_t>(static_cast<const uint16_t*>(base) + off));
}

template <int DT, int CDT>
__global__ __launch_bounds__(256) void k_generic(Desc single, const Desc* __restrict__ descs,
                                                 const uint32_t* __restrict__ map, int pow2,
                                                 int scale_bf16, int blk_r, int blk_c) {
  __shared__ uint32_t red[4];
  Desc d;
  int64_t u;
  pick_desc<kXcdRunStream>(single, descs, map, d, u);
  const int64_t per = d.units_r * d.units_c;
  const int64_t b = u / per;
  const int64_t rem = u - b * per;
  const int64_t tr = rem / d.units_c;
  const int64_t tc = rem - tr * d.units_c;
  const int64_t r0 = tr * blk_r, c0 = tc * blk_c;
  const int64_t nr = (r0 + blk_r <= d.rows ? blk_r : d.rows - r0);
  const int64_t nc = (c0 + blk_c <= d.cols ? blk_c : d.cols - c0);
  const int64_t n = nr * nc;
  const int tid = threadIdx.x;

  uint32_t a = 0u;
  for (int64_t i = tid; i < n; i += 256) {
    const int64_t r = r0 + i / nc, c = c0 + i % nc;
    const uint32_t v = f2u(load_elem<DT>(d.in, b * d.bstride + r * d.ld + c)) & 0x7FFFFFFFu;
    a = v > a ? v : a;
  }
  a = wave_max(a);
  if ((tid & 63) == 0) red[tid >> 6] = a;
  __syncthreads();
  a = red[0];
  a = red[1] > a ? red[1] : a;
  a = red[2] > a ? red[2] : a;
  a = red[3] > a ? red[3] : a;

  const BlockScale bs = block_scale<CDT>(a, pow2 != 0);
  if (tid == 0) store_scale<CDT>(d.scales, u, bs.s, scale_bf16);
  for (int64_t i = tid; i < n; i += 256) {
    const int64_t r = r0 + i / nc, c = c0 + i % nc;
    const float x = load_elem<DT>(d.in, b * d.bstride + r * d.ld + c);
    const uint32_t code =
        bs.kind <= kScaleExact ? sw_e4m3(block_quot<CDT>(x, bs)) : special_code<CDT>(x, bs);
    gst<uint8_t>(d.codes + (b * d.rows + r) * d.cols + c, (uint8_t)code);
  }
}

// ---------------------------------------------------------------------------
// host-side dispatch
// ---------------------------------------------------------------------------
template <int DT, int CDT>
static hipError_t launch_fp8_typed(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                                   const uint32_t* map, int64_t units, hipStream_t stream) {
  const dim3 grid((unsigned)units), block(256);
  switch (cfg.kernel) {
    case kKernTile128:
      hipLaunchKernelGGL((k_tile128<DT, CDT, kTileThreads>), grid, dim3(kTileThreads), 0, stream, single, descs,
                         map, cfg.pow2, cfg.scale_bf16);
      break;
    case kKernRowQuad:
      switch (cfg.blk_c) {
        case 32: hipLaunchKernelGGL((k_row<DT, CDT, 4>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
        case 64: hipLaunchKernelGGL((k_row<DT, CDT, 8>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
        case 128: hipLaunchKernelGGL((k_row<DT, CDT, 16>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
        case 256: hipLaunchKernelGGL((k_row<DT, CDT, 32>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
        case 512: hipLaunchKernelGGL((k_row<DT, CDT, 64>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
        case 1024: hipLaunchKernelGGL((k_row<DT, CDT, 64, false, 2>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
        case 2048: hipLaunchKernelGGL((k_row<DT, CDT, 64, false, 4>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
        default: return hipErrorInvalidValue;
      }
      break;
    case kKernRowF32:
      if constexpr (DT == kF32) {
        switch (cfg.blk_c) {
          case 8: hipLaunchKernelGGL((k_row_f32<2, 1>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
          case 16: hipLaunchKernelGGL((k_row_f32<4, 1>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
          case 32: hipLaunchKernelGGL((k_row_f32<8, 1>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
          case 64: hipLaunchKernelGGL((k_row_f32<16, 1>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
          case 128: hipLaunchKernelGGL((k_row_f32<32, 1>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
          case 256: hipLaunchKernelGGL((k_row_f32<64, 1>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
          case 512: hipLaunchKernelGGL((k_row_f32<64, 2>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
          case 1024: hipLaunchKernelGGL((k_row_f32<64, 4>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16); break;
          default: return hipErrorInvalidValue;
        }
        break;
      }
      return hipErrorInvalidValue;
    case kKernRowG: {
      // widths 8..512 other than 32..512 powers of two: g = ceil(bw/8) chunks
      // in the next power of two of lanes (1x8 and 1x16 unpadded)
      const int bw = (int)cfg.blk_c, g = (bw + 7) / 8;
      if (bw == 8)
        hipLaunchKernelGGL((k_row<DT, CDT, 1>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16, bw);
      else if (bw == 16)
        hipLaunchKernelGGL((k_row<DT, CDT, 2>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16, bw);
      else if (g <= 2)
        hipLaunchKernelGGL((k_row<DT, CDT, 2, true>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16, bw);
      else if (g <= 4)
        hipLaunchKernelGGL((k_row<DT, CDT, 4, true>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16, bw);
      else if (g <= 8)
        hipLaunchKernelGGL((k_row<DT, CDT, 8, true>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16, bw);
      else if (g <= 16)
        hipLaunchKernelGGL((k_row<DT, CDT, 16, true>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16, bw);
      else if (g <= 32)
        hipLaunchKernelGGL((k_row<DT, CDT, 32, true>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16, bw);
      else
        hipLaunchKernelGGL((k_row<DT, CDT, 64, true>), grid, block, 0, stream, single, descs, map, cfg.pow2, cfg.scale_bf16, bw);
      break;
    }
    case kKernRowWide: {
      const int g = (int)cfg.blk_c;  // the block width
      const WideShape ws = wide_shape(DT, cfg.blk_c);
#define LRQ_WIDE(W, P, NC)                                                                         \
  hipLaunchKernelGGL((k_row_wide<DT, CDT, W, P, NC>), grid, dim3(wg_threads(kKernRowWide, DT, cfg.blk_c)), 0, stream, single, \
                     descs, map, cfg.pow2, cfg.scale_bf16, g)
      if (ws.nc == kWideChunks) {
        if (ws.w == 16) LRQ_WIDE(16, 1, kWideChunks);
        else if (ws.w == 8) LRQ_WIDE(8, 1, kWideChunks);
        else if (ws.w == 4) LRQ_WIDE(4, 1, kWideChunks);
        else LRQ_WIDE(1, 1, kWideChunks);
      } else {
        if (ws.w == 4) LRQ_WIDE(4, 1, 4);
        else if (ws.w == 2) LRQ_WIDE(2, 1, 4);
        else if (ws.p == 2) LRQ_WIDE(1, 2, 4);
        else LRQ_WIDE(1, 1, 4);
      }
#undef LRQ_WIDE
      break;
    }
    case kKernGenericFp8:
      hipLaunchKernelGGL((k_generic<DT, CDT>), grid, block, 0, stream, single, descs, map,
                         cfg.pow2, cfg.scale_bf16, cfg.blk_r, cfg.blk_c);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_fp8(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                      const uint32_t* map, int64_t units, hipStream_t stream) {
  if (cfg.arith == 0) {
    switch (cfg.in_dtype) {
      case kBF16: return launch_fp8_typed<kBF16, kF32>(cfg, single, descs, map, units, stream);
      case kF16: return launch_fp8_typed<kF16, kF32>(cfg, single, descs, map, units, stream);
      case kF32: return launch_fp8_typed<kF32, kF32>(cfg, single, descs, map, units, stream);
    }
  } else {
    switch (cfg.in_dtype) {
      case kBF16: return launch_fp8_typed<kBF16, kBF16>(cfg, single, descs, map, units, stream);
      case kF16: return launch_fp8_typed<kF16, kF16>(cfg, single, descs, map, units, stream);
      case kF32: return launch_fp8_typed<kF32, kF32>(cfg, single, descs, map, units, stream);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace lrq
