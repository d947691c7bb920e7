// Internal launch interface shared by the kernel files and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lrq_device.hpp"

namespace lrq {

// One tensor of a launch: `batch` matrices of [rows, cols], input row stride
// `ld` and matrix stride `bstride` (elements); codes and scales are dense.
// For a grouped launch `unit0` is the first work-group of this tensor.
struct Desc {
  const void* in;
  uint8_t* codes;
  void* scales;
  int64_t batch, rows, cols, ld, bstride;
  int64_t unit0;
  int64_t units;     // work-groups of this tensor
  int64_t units_c;   // tile kernel: tiles per row band; amax: 1 = 16-byte loads
  int64_t units_r;   // tile kernel: tile rows per matrix; amax: 1 = contiguous
  int64_t nblocks;   // row/MX kernels: number of blocks/groups
  int64_t bpr;       // row/MX kernels: blocks (groups) per row; k_tile128: log2 of its XCD run
};
static_assert(sizeof(Desc) == 112, "Desc layout is part of the grouped table format");

enum Kernel : int {
  kKernTile128 = 0,   // 128x128 FP8 tiles, one work-group per tile
  kKernRowQuad = 1,   // 1xB FP8 blocks, B/8 consecutive lanes per block
  kKernGenericFp8 = 2,
  kKernMx = 3,        // MXFP8 / MXFP4, one quad per 32-group
  kKernGenericMx = 4,
  kKernDequant = 5,        // FP8 dequant, 16 codes per lane-chunk
  kKernGenericDequant = 6, // FP8 dequant, one element per thread
  kKernAmax = 7,           // per-tensor max |x| partials + scale (two launches)
  kKernCopy = 8,           // grouped byte copy (bucket pass-through tensors)
  kKernCast = 9,           // grouped unscaled cast to float8_e4m3fn
  kKernMxDequant = 10,     // MXFP8 / MXFP4 dequant, 8 (bf16 out) or 4 (fp32) elements per lane-chunk
  kKernF64 = 11,           // FP8 blocks of a float64 tensor in float64 arithmetic, one wave per block
  kKernF64Row = 12,        // 1xB float64 blocks (B = 32..2048, powers of two), 16-byte loads
  kKernF64Tile = 13,       // 128x128 float64 tiles, one 512-thread work-group per tile
  kKernRowWide = 16,       // 1xB FP8 blocks, 512 < B <= 65536 but 1024/2048: k_row_wide
  kKernF64Wide = 17,       // 1xB float64 blocks k_row_f64 does not take, 2 <= B <= 16384:
                           // k_row_pad_f64 (5 <= B < 128), else k_row_wide_f64
  kKernRowF32 = 15,        // 1xB FP8 blocks of float32 input (B = 8..1024, a power of two), one 16-byte load per lane chunk
  kKernRowG = 14,          // 1xB FP8 blocks, B = 8..512 but 32..512 powers of two: k_row with
                           // 1- or 2-lane groups (1x8, 1x16), else g = ceil(B/8) lanes of each
                           // next-power-of-two group (2 at least) active
};

// Work per lane of the streaming kernels, shared by the kernels and the
// work-group planner (values chosen by sweeps on an MI355X).
constexpr int64_t kCopyUnit = 4096;  // k_copy: bytes per work-group (one 16 B load per lane)
constexpr int kDequantChunks = 2;    // k_dequant: 16-byte output chunks per lane (2 beat 1, 4 and 8)
constexpr int kMxLoads = 2;          // k_mx: 32-element groups per quad of lanes (2 beat 1, 3 and 4)
constexpr int kWideChunks = 8;       // k_row_wide: 8-element chunks per lane (at most)
constexpr int64_t kWideMax = 16 * 64 * 8 * kWideChunks;  // k_row_wide: widest block (16 waves)
// k_row_wide's launch shape for a 1xB block (512 < B <= 65536) of g =
// ceil(B/8) chunks: the block takes C = nextpow2(ceil(g/64)) 64-lane steps of
// chunk slots, as NC slots per lane on W = C/NC waves (at least one; 8 or 16
// waves make a 512- or 1024-thread work-group of one block), and a wave holds
// P = NC/C blocks (at least one).  Every slot past a block's chunks re-loads
// its first chunk.  NC = 4 (43-57 VGPRs) unless the sweeps on an MI355X
// favoured 8 (65-97 VGPRs): blocks past C = 16, blocks of exactly
// 512 chunks (one wave, every slot used: 1x4096 by 1-2 %) and 16-bit blocks
// of more than 768 chunks (4 waves of 4 slots, all used: 1x7168 and 1x8192 by
// 1.5-2 %).  4 slots instead of 8 gained up to 9 % elsewhere (1x4104), float32
// up to 8.7 % (1x5120).
struct WideShape {
  int nc, w, p;  // chunk slots per lane, waves per block, blocks per wave
};
constexpr WideShape wide_shape(int dtype, int64_t blk_c) {
  const int64_t g = (blk_c + 7) / 8;
  int c = 1;
  while (64 * c < g) c *= 2;
  if (c > 16 || g == 64 * 8 || (dtype != kF32 && g > 64 * 12)) return {kWideChunks, c > 32 ? c / 8 : c > 8 ? 4 : 1, 1};
  return {4, c > 4 ? c / 4 : 1, c < 4 ? 4 / c : 1};
}
constexpr int kTileThreads = 512;    // k_tile128: threads per 128x128 tile (512 beat 256 and 1024)
constexpr int kRowBlocks = 4;        // k_row: wave instructions per lane, one 1xB block each up to B = 512, sharing
                                     // one scale computation (4: 2 is 7% slower with bf16 scales, 3 slower with both)
// XCD run length (xcd_unit) per kernel, in work units; sweeps over 8..128.
// k_tile128 takes a run per tensor (Desc::bpr, the log2 of it, from the
// input's row pitch: tile_run_log2).  Rows of a multiple of 8 KiB take runs of
// 4 tiles, so the 8 XCDs share every 32-tile group (one 8 KiB row span of a
// K = 4096 band) and XCD x always reads its own 1 KiB column slice of it
// (address bits 10-12 == x for 8 KiB-aligned rows).  Against runs of 32 (whole
// K = 4096 bands per XCD): C2 80.1-80.9 % of 8 TB/s from 77.6-79.2 %, its 36
// down_proj (K = 12288) 81 % from 77-78 %, single 2 GiB weights 81.4-82 % at
// K = 4096 and 12288; runs of 2, 6, 8 and 16 lose 5-10 points on C2.  Other
// pitches take runs of 8: the 48 Qwen3-30B-A3B expert layers (4 KiB gate_up
// rows, 1.5 KiB down rows; one launch per layer) 82.5-82.8 % against
// 81.8-82.3 % with runs of 4, interleaved in one process (runs of 16, 32 or
// one tile row for the down rows: within 0.3 points of 8).
constexpr int kTileRunLog2Wide = 2;    // rows of a multiple of 8 KiB: runs of 4
constexpr int kTileRunLog2Narrow = 3;  // any other row pitch: runs of 8
constexpr int tile_run_log2(int64_t pitch_bytes) {
  return pitch_bytes % 8192 == 0 ? kTileRunLog2Wide : kTileRunLog2Narrow;
}
constexpr int64_t kXcdRunTileF64 = 32;  // k_tile_f64: 32 tiles (128 KiB each)
constexpr int64_t kXcdRunRow = 16;     // k_row: 256 KiB of bf16 (32 loses 2%)
constexpr int64_t kXcdRunMx = 64;      // k_mx: 512 KiB of bf16 (32 loses 2.5%, 128 ties)
// dequant, act, amax, copy, cast, generic kernels: runs of 4, 8 and 16 lose
// 2-10 points on dequantize, cast, activation and tensor-scale launches; 64 ties.
constexpr int64_t kXcdRunStream = 32;
constexpr int kCastLaneElems = 16;   // k_cast_e4m3: elements per lane
constexpr int64_t kCastUnit = 256 * kCastLaneElems;  // k_cast_e4m3: elements per work-group
constexpr int kAmaxLoads = 2;        // k_amax: 16-byte loads per lane (2 beat 1, 3, 4 and 8)
constexpr int kScaleThreads = 1024;  // k_tensor_scale: one work-group per tensor
// k_row_f64: 1 KiB wave instructions per wave (128 doubles each); 4 beats 8 by
// 8-10% on 1x128 blocks.  1x1024 and 1x2048 blocks take one block per wave.
constexpr int kF64RowInstr = 4;
constexpr int f64_row_instr(int64_t blk_c) { return blk_c > 128 * kF64RowInstr ? (int)(blk_c / 128) : kF64RowInstr; }
// k_row_wide_f64's blocks per wave for a 1xB float64 block: 4, 2 or 1 when its
// ceil(B/2) 16-byte chunks take at most 2, 4 or 8 of a wave's 64-lane steps,
// 0 when it takes 4, 8 or 16 waves (B > 1024: up to 4096, 8192, 16384).
constexpr int f64_wide_blocks_per_wave(int64_t blk_c) {
  return blk_c <= 256 ? 4 : blk_c <= 512 ? 2 : blk_c <= 1024 ? 1 : 0;
}
// Narrower float64 blocks (5 <= B < 128) take k_row_pad_f64 instead: the
// lanes of a block's aligned group, L = nextpow2(ceil(B/2)) (4..64), or 0 for
// widths outside that range.
constexpr int f64_pad_lanes(int64_t blk_c) {
  if (blk_c < 5 || blk_c >= 128) return 0;
  int l = 4;
  while (2 * l < blk_c) l *= 2;
  return l;
}

// Threads per work-group of `kernel` for 1xB blocks of width blk_c: 512 for
// the tile kernels, 64 W for k_row_wide's 8- and 16-wave blocks, 512 or 1024
// for k_row_wide_f64's blocks past 4096, else 256.  The launch code uses the
// same rule, and the C ABI sizes its 32-bit thread-count guard by it.
constexpr int wg_threads(int kernel, int in_dtype, int64_t blk_c) {
  if (kernel == kKernTile128 || kernel == kKernF64Tile) return kTileThreads;
  if (kernel == kKernRowWide) {
    const WideShape ws = wide_shape(in_dtype, blk_c);
    return ws.w > 4 ? 64 * ws.w : 256;
  }
  if (kernel == kKernF64Wide && f64_pad_lanes(blk_c) == 0 && f64_wide_blocks_per_wave(blk_c) == 0)
    return blk_c <= 4096 ? 256 : blk_c <= 8192 ? 512 : 1024;
  return 256;
}

// Descriptor and local work unit of this work-group: the single-tensor
// descriptor (kernel argument) or, for a grouped launch, the one the device
// map names for the work-group index remapped into XCD runs of RUN units
// (xcd_unit).
template <int64_t RUN>
__device__ __forceinline__ void pick_desc(const Desc& single, const Desc* descs,
                                          const uint32_t* map, Desc& d, int64_t& u) {
  const int64_t wg = xcd_unit<RUN>(blockIdx.x, gridDim.x);
  if (map != nullptr) {
    const uint32_t t = map[wg];
    d = descs[t];
    u = wg - d.unit0;
  } else {
    d = single;
    u = wg;
  }
}

// The 128x128 tile kernel's descriptor and local tile: xcd_unit over the
// tensor's own tiles with its run of 2^Desc::bpr (shifts and masks only).  A
// grouped tensor may start at any work-group; 8 consecutive work-groups still
// visit each XCD once, so each run of 2^bpr tiles lands on one XCD.
__device__ __forceinline__ void pick_desc_tile(const Desc& single, const Desc* descs,
                                               const uint32_t* map, Desc& d, int64_t& u) {
  const uint32_t wg = blockIdx.x;
  uint32_t i;
  if (map != nullptr) {
    d = descs[map[wg]];
    i = wg - (uint32_t)d.unit0;
  } else {
    d = single;
    i = wg;
  }
  const uint32_t lg = (uint32_t)d.bpr, chunk = 8u << lg;
  if (i < ((uint32_t)d.units & ~(chunk - 1u))) {
    const uint32_t r = i & (chunk - 1u);
    i = (i - r) + ((r & 7u) << lg) + (r >> 3);
  }
  u = i;
}

// Launch parameters common to every tensor of one launch.
struct LaunchCfg {
  int kernel;     // Kernel
  int in_dtype;   // kBF16 / kF16 / kF32 (kF64: FP8 blocks in float64 arithmetic only)
  int arith;      // 0: float32 arithmetic, 1: input dtype's arithmetic
  int pow2;       // pow2 scale rounding
  int blk_r, blk_c;
  int mx_fmt;     // 8 or 4
  int scale_bf16; // FP8 kernels: write the float32 scales rounded to bf16
  int out_dtype;  // dequant: kF32 or kBF16 (in_dtype is then the scale dtype)
  int rows_dense; // dequant, 1xB: every tensor has cols % blk_c == 0
  int pitched;    // float64 rows: some tensor's row pitch exceeds its width
  int chunk;      // FP8 dequant: codes per lane-chunk (8: bf16 out, 4: float32 out or narrow blocks)
};

// Work-groups a tensor needs under `cfg` (filled into d.units and the unit
// geometry fields).  Returns false if the kernel cannot take the tensor.
bool plan_units(const LaunchCfg& cfg, Desc& d);

// Enqueue one launch over `n` descriptors.  Single tensor: descs_dev == null
// and `single` is passed by value.  Grouped: descs_dev/map_dev are device
// arrays (map_dev[wg] = descriptor index) and total_units work-groups run.
hipError_t launch(const LaunchCfg& cfg, const Desc& single, const Desc* descs_dev,
                  const uint32_t* map_dev, int64_t total_units, hipStream_t stream);
hipError_t launch_fp8(const LaunchCfg&, const Desc&, const Desc*, const uint32_t*, int64_t, hipStream_t);
hipError_t launch_mx(const LaunchCfg&, const Desc&, const Desc*, const uint32_t*, int64_t, hipStream_t);
hipError_t launch_dequant(const LaunchCfg&, const Desc&, const Desc*, const uint32_t*, int64_t, hipStream_t);
hipError_t launch_f64(const LaunchCfg&, const Desc&, const Desc*, const uint32_t*, int64_t, hipStream_t);

// Per-tensor scales: k_amax over `units` work-groups writing partial[unit],
// then one work-group per tensor (n) reducing them into the tensor's scale.
int64_t amax_unit_elems(int dtype, bool vec);
hipError_t launch_tensor_scale(const LaunchCfg& cfg, const Desc* descs, const uint32_t* map, int64_t n,
                               int64_t units, uint32_t* partial, hipStream_t stream);

// Device address of the library-owned tensor-scale workspace
// (LRQ_STATIC_WORKSPACE_BYTES) on device `dev`, looked up once per device.
hipError_t static_workspace(int dev, uint32_t** out);

// Grouped byte copy over `units` work-groups.
hipError_t launch_copy(const Desc* descs, const uint32_t* map, int64_t units, hipStream_t stream);
hipError_t launch_mx_dequant(const LaunchCfg& cfg, const Desc& single, const Desc* descs,
                             const uint32_t* map, int64_t units, hipStream_t stream);
hipError_t launch_cast(int dtype, const Desc& single, const Desc* descs, const uint32_t* map,
                       int64_t units, hipStream_t stream);

// Activation fake-quant.
int64_t act_grid(int dtype, int64_t rows, int64_t cols, int64_t blk);
hipError_t launch_act(const void* in, int dtype, int64_t rows, int64_t cols, int64_t ld, int64_t blk,
                      float* out, int pow2, hipStream_t stream);

// Diagnostics: element encoders applied to raw inputs.
hipError_t launch_diag_e4m3_bits(uint32_t start, int64_t n, uint8_t* out, hipStream_t stream);
hipError_t launch_diag_bf16_bits(uint32_t start, int64_t n, uint16_t* out, hipStream_t stream);
hipError_t launch_diag_mx(int fmt, const float* in, const uint8_t* e8m0, int64_t n, uint8_t* out,
                          hipStream_t stream);

}  // namespace lrq
