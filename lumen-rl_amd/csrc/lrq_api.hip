// C ABI of liblrq (include/lrq.h): argument checks, kernel choice, grouped
// tables, error reporting.  No device memory is allocated here.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "lrq.h"
#include "lrq_device.hpp"
#include "lrq_internal.hpp"

using lrq::Desc;
using lrq::LaunchCfg;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return 0;
  return fail((int)e, "%s: %s", what, hipGetErrorString(e));
}

int64_t esize(int dt) { return dt == lrq::kF64 ? 8 : dt == lrq::kF32 ? 4 : 2; }
bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
bool valid_dtype(int dt) { return dt == lrq::kBF16 || dt == lrq::kF16 || dt == lrq::kF32; }
bool pow2_block(int64_t b) { return b == 32 || b == 64 || b == 128 || b == 256 || b == 512; }
// widths k_row takes with whole lane groups: 4..64 lanes, or 2 / 4 wave instructions
bool row_block(int64_t b) { return pow2_block(b) || b == 1024 || b == 2048; }

constexpr uint32_t kMagic = 0x4C525154u;  // "LRQT"
constexpr uint32_t kTableVersion = 5u;  // 5: k_tile128 descriptors carry their XCD run
// HIP takes a launch's thread count (work-groups x threads per work-group) as
// a 32-bit value.  kMaxGrid is the limit for 256-thread work-groups;
// max_units() gives it for the work-group size of the launch `cfg` selects.
constexpr int64_t kMaxGrid = 0xFFFFFFFFll / 256;
int64_t max_units(const LaunchCfg& cfg) {
  return 0xFFFFFFFFll / lrq::wg_threads(cfg.kernel, cfg.in_dtype, cfg.blk_c);
}

// Table layout, host and device alike: [header | n descriptors | map].  The
// host table ends at map_off (`bytes`); the device table adds the uint32
// work-group -> tensor map (4 bytes per work-group, `dev_bytes` in all), which
// the device writes itself (lrq_group_build_map) instead of uploading it.
struct GroupHeader {
  uint32_t magic, version;
  LaunchCfg cfg;
  int64_t n, units, desc_off, map_off, bytes, dev_bytes;
};

int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// Largest element offset the kernels' 64-bit index arithmetic is allowed to
// reach (2^48 elements, far beyond any device's memory): extents whose
// products pass it are rejected before they can wrap.
constexpr int64_t kMaxElems = int64_t(1) << 48;

bool span_ok(int64_t batch, int64_t rows, int64_t cols, int64_t ld, int64_t bstride) {
  int64_t a, b, c;
  if (batch < 0 || rows < 0 || cols < 0 || ld < 0 || bstride < 0) return false;
  if (batch > kMaxElems || rows > kMaxElems || cols > kMaxElems || ld > kMaxElems || bstride > kMaxElems)
    return false;
  if (__builtin_mul_overflow(batch, rows, &a) || __builtin_mul_overflow(a, cols, &b) || b > kMaxElems)
    return false;  // elements
  if (__builtin_mul_overflow(rows, ld, &a) || a > kMaxElems) return false;  // one matrix's extent
  if (batch > 1 && (__builtin_mul_overflow(batch - 1, bstride, &c) || c > kMaxElems - a)) return false;
  return true;
}

// Fill a Desc from a tensor and check its shape.
int make_desc(const lrq_tensor& t, Desc& d, bool need_codes = true, bool need_scales = true) {
  if (t.batch < 0 || t.rows < 0 || t.cols < 0) return fail(LRQ_ERR_ARG, "negative extent");
  if (!span_ok(t.batch, t.rows, t.cols, t.ld < t.cols ? t.cols : t.ld, t.batch > 1 ? t.batch_stride : 0))
    return fail(LRQ_ERR_ARG, "extents exceed 2^48 elements");
  if (t.batch == 0 || t.rows == 0 || t.cols == 0) {
    memset(&d, 0, sizeof(d));
    d.batch = t.batch; d.rows = t.rows; d.cols = t.cols;
    return 0;
  }
  if (t.ld < t.cols) return fail(LRQ_ERR_ARG, "ld (%lld) < cols (%lld)", (long long)t.ld, (long long)t.cols);
  if (t.batch > 1 && t.batch_stride < (t.rows - 1) * t.ld + t.cols)
    return fail(LRQ_ERR_ARG, "batch_stride (%lld) overlaps matrices", (long long)t.batch_stride);
  if (!t.in || (need_codes && !t.codes) || (need_scales && !t.scales)) return fail(LRQ_ERR_ARG, "null pointer");
  memset(&d, 0, sizeof(d));
  d.in = t.in;
  d.codes = static_cast<uint8_t*>(t.codes);
  d.scales = t.scales;
  d.batch = t.batch; d.rows = t.rows; d.cols = t.cols; d.ld = t.ld;
  d.bstride = t.batch > 1 ? t.batch_stride : t.rows * t.ld;
  return 0;
}

// Fold the batch into rows when matrices are evenly spaced (1-D kernels).
bool fold_batch(Desc& d) {
  if (d.batch == 1) return true;
  if (d.bstride != d.rows * d.ld) return false;
  d.rows *= d.batch;
  d.batch = 1;
  d.bstride = d.rows * d.ld;
  return true;
}

int fp8_kernel_for(const Desc& d, int in_dtype, int64_t blk_r, int64_t blk_c) {
  if (in_dtype == lrq::kF64) {
    const bool row = blk_r == 1 && row_block(blk_c) && d.cols % blk_c == 0 &&
                     (d.batch == 1 || d.bstride == d.rows * d.ld) && aligned(d.in, 8) &&
                     aligned(d.codes, 2) && aligned(d.scales, 8);
    if (row) return lrq::kKernF64Row;
    // other widths 2..16384 (2-double chunks, the last overlapped when B is odd)
    const bool wide = blk_r == 1 && blk_c >= 2 && blk_c <= 16384 && d.cols % blk_c == 0 &&
                      (d.batch == 1 || d.bstride == d.rows * d.ld) && aligned(d.in, 8) && aligned(d.scales, 8);
    if (wide) return lrq::kKernF64Wide;
    const bool tile = blk_r == 128 && blk_c == 128 && aligned(d.in, 8) && d.cols % 2 == 0 &&
                      aligned(d.codes, 2) && aligned(d.scales, 8);
    return tile ? lrq::kKernF64Tile : lrq::kKernF64;
  }
  const int64_t es = esize(in_dtype);
  // input loads take element-aligned addresses (any row pitch); the tile
  // kernel's chunks of 8 elements stay inside a row, and 1xB blocks hold
  // ceil(B/8) chunks whose last one may overlap its neighbour
  const bool vec_row = aligned(d.in, (uintptr_t)es) && aligned(d.codes, 8) &&
                       (d.batch == 1 || d.bstride == d.rows * d.ld);
  const bool vec = aligned(d.in, (uintptr_t)es) && aligned(d.codes, 8) && d.cols % 8 == 0;
  if (blk_r == 128 && blk_c == 128 && vec) return lrq::kKernTile128;
  if (in_dtype == lrq::kF32 && blk_r == 1 && (pow2_block(blk_c) || blk_c == 8 || blk_c == 16 || blk_c == 1024) &&
      d.cols % blk_c == 0 && vec && aligned(d.codes, 4) && (d.batch == 1 || d.bstride == d.rows * d.ld))
    return lrq::kKernRowF32;  // float32 input: 4-float chunks, 1 KiB per wave instruction
  if (blk_r == 1 && row_block(blk_c) && d.cols % blk_c == 0 && vec &&
      (d.batch == 1 || d.bstride == d.rows * d.ld))
    return lrq::kKernRowQuad;
  // other widths 8..512: 1- and 2-lane groups (1x8, 1x16), padded lane groups
  // of ceil(B/8) chunks beyond
  if (blk_r == 1 && blk_c >= 8 && blk_c <= 512 && d.cols % blk_c == 0 && vec_row)
    return lrq::kKernRowG;
  // wider blocks: one wave per block up to 4096, up to 16 waves up to 65536
  if (blk_r == 1 && blk_c > 512 && blk_c <= lrq::kWideMax && d.cols % blk_c == 0 && vec_row)
    return lrq::kKernRowWide;
  return lrq::kKernGenericFp8;
}

// codes (d.in) at any alignment; the output (d.codes) takes 16-byte stores, and
// each lane-chunk of cpc codes must lie inside one block and one row
int dequant_kernel_for(const Desc& d, int64_t blk_c, int64_t cpc) {
  const bool vec = aligned(d.codes, 16) && d.cols % cpc == 0 && blk_c % cpc == 0;
  return vec ? lrq::kKernDequant : lrq::kKernGenericDequant;
}

int mx_kernel_for(const Desc& d, int in_dtype, int fmt) {
  const int64_t es = esize(in_dtype);
  const bool vec = aligned(d.in, (uintptr_t)es) && (d.batch == 1 || d.bstride == d.rows * d.ld) &&
                   aligned(d.codes, fmt == 8 ? 8 : 4);
  return vec ? lrq::kKernMx : lrq::kKernGenericMx;
}

}  // namespace

namespace lrq {

bool plan_units(const LaunchCfg& cfg, Desc& d) {
  if (d.batch == 0 || d.rows == 0 || d.cols == 0) {
    d.units = 0;
    return true;
  }
  switch (cfg.kernel) {
    case kKernTile128:
    case kKernF64Tile:
    case kKernGenericFp8:
      d.units_r = (d.rows + cfg.blk_r - 1) / cfg.blk_r;
      d.units_c = (d.cols + cfg.blk_c - 1) / cfg.blk_c;
      d.units = d.batch * d.units_r * d.units_c;
      if (cfg.kernel == kKernTile128) d.bpr = tile_run_log2(d.ld * esize(cfg.in_dtype));
      return true;
    case kKernF64Row: {  // 4 waves x f64_row_instr instructions of 128 doubles
      if (!fold_batch(d)) return false;
      const int64_t per_wg = 4 * f64_row_instr(cfg.blk_c) * 128;
      d.units = (d.batch * d.rows * d.cols + per_wg - 1) / per_wg;
      return true;
    }
    case kKernF64Wide: {  // 4 waves of 64/L blocks per instruction (B < 128), of P blocks
                          // each (B <= 1024), or one block of 4 waves
      if (!fold_batch(d)) return false;
      d.bpr = d.cols / cfg.blk_c;
      d.nblocks = d.rows * d.bpr;
      const int L = f64_pad_lanes(cfg.blk_c);
      const int P = f64_wide_blocks_per_wave(cfg.blk_c);
      const int64_t per_wg = L > 0 ? 4 * kF64RowInstr * (64 / L) : P > 0 ? 4 * P : 1;
      d.units = (d.nblocks + per_wg - 1) / per_wg;
      return true;
    }
    case kKernF64:  // one wave per block, four per work-group
      d.units_r = (d.rows + cfg.blk_r - 1) / cfg.blk_r;
      d.units_c = (d.cols + cfg.blk_c - 1) / cfg.blk_c;
      d.nblocks = d.batch * d.units_r * d.units_c;
      d.units = (d.nblocks + 3) / 4;
      return true;
    case kKernRowQuad: {
      if (!fold_batch(d)) return false;
      d.bpr = d.cols / cfg.blk_c;
      d.nblocks = d.rows * d.bpr;
      // 4 waves x kRowBlocks instructions of 512 elements
      const int64_t per_wg = cfg.blk_c <= 512 ? 4 * kRowBlocks * (512 / cfg.blk_c)
                                              : 4 * kRowBlocks / (cfg.blk_c / 512);
      d.units = (d.nblocks + per_wg - 1) / per_wg;
      return true;
    }
    case kKernRowF32: {  // 4 waves x kRowBlocks instructions of 256 floats
      if (!fold_batch(d)) return false;
      d.bpr = d.cols / cfg.blk_c;
      d.nblocks = d.rows * d.bpr;
      const int64_t per_wg = cfg.blk_c <= 256 ? 4 * kRowBlocks * (256 / cfg.blk_c)
                                              : 4 * kRowBlocks / (cfg.blk_c / 256);
      d.units = (d.nblocks + per_wg - 1) / per_wg;
      return true;
    }
    case kKernRowWide: {  // 4 waves of P blocks each, 2 blocks of 2 waves, or one block of 4-16 waves
      if (!fold_batch(d)) return false;
      d.bpr = d.cols / cfg.blk_c;
      d.nblocks = d.rows * d.bpr;
      const WideShape ws = wide_shape(cfg.in_dtype, cfg.blk_c);
      const int64_t per_wg = ws.w >= 4 ? 1 : 4 / ws.w * ws.p;
      d.units = (d.nblocks + per_wg - 1) / per_wg;
      return true;
    }
    case kKernRowG: {
      if (!fold_batch(d)) return false;
      d.bpr = d.cols / cfg.blk_c;
      d.nblocks = d.rows * d.bpr;
      int64_t lanes = 1;  // a block's lane group: the next power of two of ceil(blk_c / 8)
      while (lanes < (cfg.blk_c + 7) / 8) lanes *= 2;
      const int64_t per_wg = 4 * kRowBlocks * (64 / lanes);
      d.units = (d.nblocks + per_wg - 1) / per_wg;
      return true;
    }
    case kKernDequant:
    case kKernGenericDequant:
      d.units_r = (d.rows + cfg.blk_r - 1) / cfg.blk_r;
      d.units_c = (d.cols + cfg.blk_c - 1) / cfg.blk_c;
      if (cfg.kernel == kKernDequant) {
        const int64_t cpc = cfg.chunk;  // codes per lane-chunk
        d.nblocks = d.batch * d.rows * d.cols / cpc;
        d.units = (d.nblocks + 256 * kDequantChunks - 1) / (256 * kDequantChunks);
      } else {
        d.nblocks = d.batch * d.rows * d.cols;
        d.units = (d.nblocks + 255) / 256;
      }
      return true;
    case kKernMx:
    case kKernGenericMx:
      if (!fold_batch(d)) {
        // generic MX walks rows through `ld` only; a ragged batch stride is
        // handled by the caller (one launch per matrix)
        return false;
      }
      d.bpr = d.cols / 32;
      d.nblocks = d.rows * d.bpr;
      if (cfg.kernel == kKernMx) d.units = (d.nblocks + 64 * kMxLoads - 1) / (64 * kMxLoads);
      else d.units = (d.nblocks + 255) / 256;
      return true;
  }
  return false;
}

hipError_t launch(const LaunchCfg& cfg, const Desc& single, const Desc* descs_dev,
                  const uint32_t* map_dev, int64_t total_units, hipStream_t stream) {
  if (cfg.kernel == kKernMxDequant)
    return launch_mx_dequant(cfg, single, descs_dev, map_dev, total_units, stream);
  if (cfg.kernel == kKernMx || cfg.kernel == kKernGenericMx)
    return launch_mx(cfg, single, descs_dev, map_dev, total_units, stream);
  if (cfg.kernel == kKernDequant || cfg.kernel == kKernGenericDequant)
    return launch_dequant(cfg, single, descs_dev, map_dev, total_units, stream);
  if (cfg.kernel == kKernF64 || cfg.kernel == kKernF64Row || cfg.kernel == kKernF64Tile ||
      cfg.kernel == kKernF64Wide)
    return launch_f64(cfg, single, descs_dev, map_dev, total_units, stream);
  return launch_fp8(cfg, single, descs_dev, map_dev, total_units, stream);
}

}  // namespace lrq

namespace {

int run_single(const LaunchCfg& cfg, Desc& d, hipStream_t stream) {
  if (!lrq::plan_units(cfg, d))
    return fail(LRQ_ERR_ARG, "batch stride must equal rows*ld for this format");
  if (d.units == 0) return 0;
  if (d.units > max_units(cfg)) return fail(LRQ_ERR_ARG, "tensor too large for one launch");
  d.unit0 = 0;
  return check_hip(lrq::launch(cfg, d, nullptr, nullptr, d.units, stream), "kernel launch");
}

int mx_quant(int fmt, const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t ld,
             uint8_t* codes, uint8_t* scales, hipStream_t stream) {
  g_err.clear();
  if (!valid_dtype(in_dtype)) return fail(LRQ_ERR_ARG, "bad input dtype %d", in_dtype);
  if (cols % 32 != 0) return fail(LRQ_ERR_ARG, "cols (%lld) must be a multiple of 32", (long long)cols);
  int64_t mstride;
  if (__builtin_mul_overflow(rows, ld, &mstride)) return fail(LRQ_ERR_ARG, "extents exceed 2^48 elements");
  lrq_tensor t{in, codes, scales, 1, rows, cols, ld, mstride};
  Desc d;
  if (int rc = make_desc(t, d)) return rc;
  LaunchCfg cfg{};
  cfg.in_dtype = in_dtype;
  cfg.mx_fmt = fmt;
  cfg.kernel = mx_kernel_for(d, in_dtype, fmt);
  return run_single(cfg, d, stream);
}

// Host table bytes; *map_off is also where the device table's map starts.
int64_t table_layout(int64_t n, int64_t* desc_off, int64_t* map_off) {
  const int64_t h = align_up((int64_t)sizeof(GroupHeader), 256);
  *desc_off = h;
  *map_off = align_up(h + n * (int64_t)sizeof(Desc), 256);
  return *map_off;
}

// Work-group -> tensor map, one thread per work-group: tensors own consecutive
// ranges [unit0, unit0 + units) in table order (checked by lrq_group_pack), so
// the owner of w is the LAST tensor with unit0 <= w; an empty tensor shares
// its unit0 with a later one and is never picked.
__global__ __launch_bounds__(256) void k_build_map(const Desc* __restrict__ descs, int64_t n,
                                                   int64_t units, uint32_t* __restrict__ map) {
  const int64_t w = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (w >= units) return;
  int64_t lo = 0, hi = n;  // descs[lo].unit0 <= w, and every t >= hi has unit0 > w
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) / 2;
    if (lrq::gld<int64_t>(&descs[mid].unit0) <= w) lo = mid;
    else hi = mid;
  }
  lrq::gst<uint32_t>(map + w, (uint32_t)lo);
}

// Build the launch configuration and descriptors for a group; `ds` may be null
// (sizing only).  Returns 0 or an error; *units_out = total work-groups.
int plan_group(int fmt, const lrq_tensor* ts, int64_t n, int in_dtype, int64_t blk_r,
               int64_t blk_c, unsigned flags, LaunchCfg* cfg_out, Desc* ds, int64_t* units_out,
               bool limit = true) {
  if (n < 0 || (n > 0 && !ts)) return fail(LRQ_ERR_ARG, "bad tensor list");
  if (n > 0xFFFFFFFFll) return fail(LRQ_ERR_ARG, "more than 2^32 tensors in one table");  // uint32 map
  if (in_dtype == lrq::kF64) {
    // float64 input: quantize_tensor on a float64 tensor, float64 arithmetic only
    if (fmt != LRQ_FMT_FP8_BLOCK)
      return fail(LRQ_ERR_ARG, "float64 input is accepted by the FP8 block format only");
    if (!(flags & LRQ_FLAG_NATIVE_ARITH))
      return fail(LRQ_ERR_ARG, "float64 input is quantized in float64 arithmetic: pass LRQ_FLAG_NATIVE_ARITH");
  } else if (!valid_dtype(in_dtype)) {
    return fail(LRQ_ERR_ARG, "bad input dtype %d", in_dtype);
  }
  LaunchCfg cfg{};
  cfg.in_dtype = in_dtype;
  if (fmt == LRQ_FMT_FP8_BLOCK) {
    if (blk_r < 1 || blk_c < 1 || blk_r > (1 << 20) || blk_c > (1 << 20))
      return fail(LRQ_ERR_ARG, "bad block %lldx%lld", (long long)blk_r, (long long)blk_c);
    cfg.blk_r = (int)blk_r;
    cfg.blk_c = (int)blk_c;
    cfg.pow2 = (flags & LRQ_FLAG_POW2_SCALE) ? 1 : 0;
    cfg.arith = (flags & LRQ_FLAG_NATIVE_ARITH) && in_dtype != lrq::kF32 ? 1 : 0;
    cfg.scale_bf16 = (flags & LRQ_FLAG_SCALE_BF16) && !cfg.arith ? 1 : 0;
  } else if (fmt == LRQ_FMT_MXFP8 || fmt == LRQ_FMT_MXFP4) {
    cfg.mx_fmt = fmt == LRQ_FMT_MXFP8 ? 8 : 4;
  } else if (fmt == LRQ_FMT_FP8_DEQUANT) {
    if (blk_r < 1 || blk_c < 1 || blk_r > (1 << 20) || blk_c > (1 << 20))
      return fail(LRQ_ERR_ARG, "bad block %lldx%lld", (long long)blk_r, (long long)blk_c);
    cfg.blk_r = (int)blk_r;
    cfg.blk_c = (int)blk_c;
    cfg.out_dtype = (flags & LRQ_FLAG_OUT_BF16) ? lrq::kBF16 : lrq::kF32;
    // a lane-chunk lies inside one block and one row: 8 codes (one 16-byte
    // bf16 store) when every width allows, else 4 (16-byte float32 or 8-byte
    // bf16 stores)
    cfg.chunk = cfg.out_dtype == lrq::kBF16 && blk_c % 8 == 0 ? 8 : 4;
    for (int64_t i = 0; i < n; ++i)
      if (ts[i].cols % cfg.chunk != 0) cfg.chunk = 4;
  } else if (fmt == LRQ_FMT_TENSOR_SCALE) {
    cfg.kernel = lrq::kKernAmax;
  } else if (fmt == LRQ_FMT_COPY) {
    cfg.kernel = lrq::kKernCopy;
  } else if (fmt == LRQ_FMT_CAST_E4M3) {
    cfg.kernel = lrq::kKernCast;
  } else if (fmt == LRQ_FMT_MXFP8_DEQUANT || fmt == LRQ_FMT_MXFP4_DEQUANT) {
    cfg.kernel = lrq::kKernMxDequant;
    cfg.mx_fmt = fmt == LRQ_FMT_MXFP8_DEQUANT ? 8 : 4;
    cfg.out_dtype = (flags & LRQ_FLAG_OUT_BF16) ? lrq::kBF16 : lrq::kF32;
  } else {
    return fail(LRQ_ERR_ARG, "bad format %d", fmt);
  }
  int kernel = -1;
  int64_t units = 0;
  for (int64_t i = 0; i < n; ++i) {
    Desc d;
    if (int rc = make_desc(ts[i], d, fmt != LRQ_FMT_TENSOR_SCALE,
                           fmt != LRQ_FMT_COPY && fmt != LRQ_FMT_CAST_E4M3))
      return fail(rc, "tensor %lld: %s", (long long)i, g_err.c_str());
    if (cfg.kernel == lrq::kKernMxDequant) {
      if (d.batch == 0 || d.rows == 0 || d.cols == 0) {
        d.unit0 = units;
        d.units = 0;
        if (ds) ds[i] = d;
        continue;
      }
      if (d.ld != d.cols || d.bstride != d.rows * d.cols)
        return fail(LRQ_ERR_ARG, "tensor %lld: MX dequant needs dense codes (ld == cols)", (long long)i);
      if (d.cols % 32 != 0) return fail(LRQ_ERR_ARG, "tensor %lld: cols %% 32 != 0", (long long)i);
      const int64_t cpc = cfg.out_dtype == lrq::kBF16 ? 8 : 4;  // elements per lane-chunk
      if (!aligned(d.codes, 16))  // the codes may sit at any byte alignment
        return fail(LRQ_ERR_ALIGN, "tensor %lld: MX dequant needs a 16-byte aligned output", (long long)i);
      d.nblocks = d.batch * d.rows * d.cols / cpc;
      d.units = (d.nblocks + 256 * lrq::kDequantChunks - 1) / (256 * lrq::kDequantChunks);
      d.unit0 = units;
      units += d.units;
      if (ds) ds[i] = d;
      continue;
    }
    if (fmt == LRQ_FMT_CAST_E4M3) {
      if (d.batch > 1 || d.rows > 1 || (d.cols > 0 && d.ld != d.cols))
        return fail(LRQ_ERR_ARG, "tensor %lld: a cast entry is one contiguous run (batch = rows = 1)", (long long)i);
      const int64_t es = esize(in_dtype);
      d.units_c = aligned(d.in, (uintptr_t)es) && aligned(d.codes, es == 4 ? 4 : 8) ? 1 : 0;
      d.units = (d.cols + lrq::kCastUnit - 1) / lrq::kCastUnit;
      d.unit0 = units;
      units += d.units;
      if (ds) ds[i] = d;
      continue;
    }
    if (fmt == LRQ_FMT_COPY) {
      if (d.batch > 1 || d.rows > 1 || (d.cols > 0 && d.ld != d.cols))
        return fail(LRQ_ERR_ARG, "tensor %lld: a copy entry is one run of bytes (batch = rows = 1)", (long long)i);
      if (d.cols > 0 && (!aligned(d.in, 16) || !aligned(d.codes, 16)))
        return fail(LRQ_ERR_ALIGN, "tensor %lld: copy source and destination must be 16-byte aligned", (long long)i);
      d.units = (d.cols + lrq::kCopyUnit - 1) / lrq::kCopyUnit;
      d.unit0 = units;
      units += d.units;
      if (ds) ds[i] = d;
      continue;
    }
    if (fmt == LRQ_FMT_TENSOR_SCALE) {
      if (d.batch == 0 || d.rows == 0 || d.cols == 0)
        return fail(LRQ_ERR_ARG, "tensor %lld is empty: a max over no elements is undefined", (long long)i);
      if (!aligned(d.scales, 4)) return fail(LRQ_ERR_ALIGN, "tensor %lld: scale not 4-byte aligned", (long long)i);
      const int64_t es = esize(in_dtype);
      const bool vec = aligned(d.in, (uintptr_t)es) && d.cols % (16 / es) == 0;
      const bool dense = d.ld == d.cols && (d.batch == 1 || d.bstride == d.rows * d.cols);
      d.units_c = vec ? 1 : 0;
      d.units_r = dense ? 1 : 0;
      const int64_t per = lrq::amax_unit_elems(in_dtype, vec);
      d.units = (d.batch * d.rows * d.cols + per - 1) / per;
      d.unit0 = units;
      units += d.units;
      if (ds) ds[i] = d;
      continue;
    }
    if (d.batch == 0 || d.rows == 0 || d.cols == 0) {
      if (ds) { ds[i] = d; ds[i].unit0 = units; ds[i].units = 0; }
      continue;
    }
    int k;
    if (fmt == LRQ_FMT_FP8_BLOCK) {
      if (in_dtype == lrq::kF64 && (!aligned(d.in, 8) || (d.scales && !aligned(d.scales, 8))))
        return fail(LRQ_ERR_ALIGN, "tensor %lld: float64 input and scales must be 8-byte aligned", (long long)i);
      k = fp8_kernel_for(d, in_dtype, blk_r, blk_c);
    } else if (fmt == LRQ_FMT_FP8_DEQUANT) {
      if (d.ld != d.cols || d.bstride != d.rows * d.cols)
        return fail(LRQ_ERR_ARG, "tensor %lld: dequant needs dense codes (ld == cols)", (long long)i);
      k = dequant_kernel_for(d, blk_c, cfg.chunk);
    } else {
      if (d.cols % 32 != 0) return fail(LRQ_ERR_ARG, "tensor %lld: cols %% 32 != 0", (long long)i);
      k = mx_kernel_for(d, in_dtype, cfg.mx_fmt);
    }
    if (kernel < 0) kernel = k;
    if (k != kernel)
      return fail(LRQ_ERR_ARG, "tensor %lld needs a different kernel than tensor 0 "
                  "(alignment/shape); group it separately", (long long)i);
    cfg.kernel = k;
    if (!lrq::plan_units(cfg, d))
      return fail(LRQ_ERR_ARG, "tensor %lld: batch stride must equal rows*ld", (long long)i);
    d.unit0 = units;
    units += d.units;
    if (ds) ds[i] = d;
  }
  if (kernel < 0 && fmt != LRQ_FMT_TENSOR_SCALE && fmt != LRQ_FMT_COPY &&
      fmt != LRQ_FMT_CAST_E4M3 && cfg.kernel != lrq::kKernMxDequant)  // only empty tensors
    cfg.kernel = fmt == LRQ_FMT_FP8_BLOCK     ? lrq::kKernGenericFp8
                 : fmt == LRQ_FMT_FP8_DEQUANT ? lrq::kKernGenericDequant
                                              : lrq::kKernGenericMx;
  if (cfg.kernel == lrq::kKernF64Row) {
    cfg.pitched = 0;
    for (int64_t i = 0; i < n; ++i)
      if (ts[i].rows > 1 && ts[i].ld != ts[i].cols) cfg.pitched = 1;
  }
  if (fmt == LRQ_FMT_FP8_DEQUANT) {
    cfg.rows_dense = 1;
    for (int64_t i = 0; i < n; ++i)
      if (ts[i].cols % blk_c != 0) cfg.rows_dense = 0;
  }
  if (limit && units > max_units(cfg)) return fail(LRQ_ERR_ARG, "group too large for one launch");
  *cfg_out = cfg;
  *units_out = units;
  return 0;
}

}  // namespace

extern "C" {

int lrq_fp8_block_quant(const void* in, int in_dtype, int64_t batch, int64_t rows, int64_t cols,
                        int64_t ld, int64_t batch_stride, int64_t blk_r, int64_t blk_c,
                        uint8_t* codes, void* scales, unsigned flags, lrq_stream_t stream) {
  g_err.clear();
  lrq_tensor t{in, codes, scales, batch, rows, cols, ld, batch_stride};
  LaunchCfg cfg;
  Desc d;
  int64_t units;
  if (int rc = plan_group(LRQ_FMT_FP8_BLOCK, &t, 1, in_dtype, blk_r, blk_c, flags, &cfg, &d, &units,
                          /*limit=*/false))
    return rc;
  if (units == 0) return 0;
  if (units > max_units(cfg)) {
    // More work-groups than one launch takes (small blocks on the one-block-per-
    // work-group generic kernel): one launch per matrix, then per band of rows
    // (whole block rows), each re-planned on its own.
    const int64_t es = esize(in_dtype);
    const int64_t ses = in_dtype == lrq::kF64 ? 8
                        : (flags & LRQ_FLAG_NATIVE_ARITH) && in_dtype != lrq::kF32 ? 2
                        : (flags & LRQ_FLAG_SCALE_BF16) ? 2 : 4;
    const int64_t srows = (rows + blk_r - 1) / blk_r, scols = (cols + blk_c - 1) / blk_c;
    auto* in8 = static_cast<const uint8_t*>(in);
    auto* sc8 = static_cast<uint8_t*>(scales);
    if (batch > 1) {
      for (int64_t b = 0; b < batch; ++b)
        if (int rc = lrq_fp8_block_quant(in8 + b * batch_stride * es, in_dtype, 1, rows, cols, ld, rows * ld,
                                         blk_r, blk_c, codes + b * rows * cols, sc8 + b * srows * scols * ses,
                                         flags, stream))
          return rc;
      return 0;
    }
    const int64_t parts = units / max_units(cfg) + 2;
    const int64_t band = (srows + parts - 1) / parts * blk_r;  // rows per launch
    if (band >= rows) return fail(LRQ_ERR_ARG, "one row of blocks exceeds a launch");
    for (int64_t r0 = 0; r0 < rows; r0 += band) {
      const int64_t nr = rows - r0 < band ? rows - r0 : band;
      if (int rc = lrq_fp8_block_quant(in8 + r0 * ld * es, in_dtype, 1, nr, cols, ld, nr * ld, blk_r, blk_c,
                                       codes + r0 * cols, sc8 + (r0 / blk_r) * scols * ses, flags, stream))
        return rc;
    }
    return 0;
  }
  d.unit0 = 0;
  return check_hip(lrq::launch(cfg, d, nullptr, nullptr, units, (hipStream_t)stream), "kernel launch");
}

int lrq_fp8_block_dequant(const uint8_t* codes, const void* scales, int scale_dtype,
                          int64_t batch, int64_t rows, int64_t cols, int64_t blk_r,
                          int64_t blk_c, void* out, int out_dtype, lrq_stream_t stream) {
  g_err.clear();
  if (out_dtype != lrq::kF32 && out_dtype != lrq::kBF16) return fail(LRQ_ERR_ARG, "bad out dtype %d", out_dtype);
  int64_t mstride;
  if (__builtin_mul_overflow(rows, cols, &mstride)) return fail(LRQ_ERR_ARG, "extents exceed 2^48 elements");
  lrq_tensor t{codes, out, const_cast<void*>(scales), batch, rows, cols, cols, mstride};
  LaunchCfg cfg;
  Desc d;
  int64_t units;
  const unsigned flags = out_dtype == lrq::kBF16 ? LRQ_FLAG_OUT_BF16 : 0u;
  if (int rc = plan_group(LRQ_FMT_FP8_DEQUANT, &t, 1, scale_dtype, blk_r, blk_c, flags, &cfg, &d, &units))
    return rc;
  if (units == 0) return 0;
  d.unit0 = 0;
  return check_hip(lrq::launch(cfg, d, nullptr, nullptr, units, (hipStream_t)stream), "kernel launch");
}

int lrq_mxfp8_quant(const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t ld,
                    uint8_t* codes, uint8_t* scales, lrq_stream_t stream) {
  return mx_quant(8, in, in_dtype, rows, cols, ld, codes, scales, (hipStream_t)stream);
}

int lrq_mxfp4_quant(const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t ld,
                    uint8_t* codes, uint8_t* scales, lrq_stream_t stream) {
  return mx_quant(4, in, in_dtype, rows, cols, ld, codes, scales, (hipStream_t)stream);
}

int lrq_act_qdq(const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t ld, int64_t blk,
                unsigned flags, float* out, lrq_stream_t stream) {
  g_err.clear();
  if (!valid_dtype(in_dtype)) return fail(LRQ_ERR_ARG, "bad input dtype %d", in_dtype);
  if (blk < 1) return fail(LRQ_ERR_ARG, "activation block must be positive, got %lld", (long long)blk);
  if (rows < 0 || cols < 0 || cols % blk != 0)
    return fail(LRQ_ERR_ARG, "cols (%lld) must be a multiple of the block", (long long)cols);
  if (!span_ok(1, rows, cols, ld < cols ? cols : ld, 0)) return fail(LRQ_ERR_ARG, "extents exceed 2^48 elements");
  if (rows == 0 || cols == 0) return 0;
  if (ld < cols) return fail(LRQ_ERR_ARG, "ld < cols");
  if (!in || !out) return fail(LRQ_ERR_ARG, "null pointer");
  const int64_t es = esize(in_dtype);
  if (!aligned(in, (uintptr_t)es) || !aligned(out, 16))
    return fail(LRQ_ERR_ALIGN, "activation input must be element-aligned, out 16-byte aligned");
  if (lrq::act_grid(in_dtype, rows, cols, blk) > kMaxGrid) return fail(LRQ_ERR_ARG, "tensor too large for one launch");
  return check_hip(lrq::launch_act(in, in_dtype, rows, cols, ld, blk, out,
                                   (flags & LRQ_FLAG_POW2_SCALE) ? 1 : 0, (hipStream_t)stream),
                   "kernel launch");
}

int lrq_cast_e4m3(const void* in, int in_dtype, int64_t n, uint8_t* out, lrq_stream_t stream) {
  g_err.clear();
  lrq_tensor t{in, out, nullptr, 1, 1, n, n, n};
  LaunchCfg cfg;
  Desc d;
  int64_t units;
  if (n < 0) return fail(LRQ_ERR_ARG, "negative element count");
  if (int rc = plan_group(LRQ_FMT_CAST_E4M3, &t, 1, in_dtype, 1, 1, 0, &cfg, &d, &units)) return rc;
  if (units == 0) return 0;
  d.unit0 = 0;
  return check_hip(lrq::launch_cast(in_dtype, d, nullptr, nullptr, units, (hipStream_t)stream),
                   "kernel launch");
}

int lrq_mx_dequant(int fmt, const uint8_t* codes, const uint8_t* scales, int64_t rows,
                   int64_t cols, void* out, int out_dtype, lrq_stream_t stream) {
  g_err.clear();
  if (fmt != LRQ_FMT_MXFP8 && fmt != LRQ_FMT_MXFP4) return fail(LRQ_ERR_ARG, "bad MX format %d", fmt);
  if (out_dtype != lrq::kF32 && out_dtype != lrq::kBF16) return fail(LRQ_ERR_ARG, "bad out dtype %d", out_dtype);
  int64_t mstride;
  if (__builtin_mul_overflow(rows, cols, &mstride)) return fail(LRQ_ERR_ARG, "extents exceed 2^48 elements");
  lrq_tensor t{codes, out, const_cast<uint8_t*>(scales), 1, rows, cols, cols, mstride};
  LaunchCfg cfg;
  Desc d;
  int64_t units;
  const int gfmt = fmt == LRQ_FMT_MXFP8 ? LRQ_FMT_MXFP8_DEQUANT : LRQ_FMT_MXFP4_DEQUANT;
  const unsigned flags = out_dtype == lrq::kBF16 ? LRQ_FLAG_OUT_BF16 : 0u;
  if (int rc = plan_group(gfmt, &t, 1, lrq::kBF16, 1, 32, flags, &cfg, &d, &units)) return rc;
  if (units == 0) return 0;
  d.unit0 = 0;
  return check_hip(lrq::launch(cfg, d, nullptr, nullptr, units, (hipStream_t)stream), "kernel launch");
}

int64_t lrq_group_table_bytes(int fmt, const lrq_tensor* tensors, int64_t n, int in_dtype,
                              int64_t blk_r, int64_t blk_c, unsigned flags) {
  g_err.clear();
  LaunchCfg cfg;
  int64_t units;
  if (int rc = plan_group(fmt, tensors, n, in_dtype, blk_r, blk_c, flags, &cfg, nullptr, &units))
    return rc;
  int64_t a, b;
  return table_layout(n, &a, &b);
}

int lrq_group_pack(int fmt, const lrq_tensor* tensors, int64_t n, int in_dtype, int64_t blk_r,
                   int64_t blk_c, unsigned flags, void* host_table, int64_t capacity) {
  g_err.clear();
  if (!host_table) return fail(LRQ_ERR_ARG, "null table");
  LaunchCfg cfg;
  int64_t units;
  if (int rc = plan_group(fmt, tensors, n, in_dtype, blk_r, blk_c, flags, &cfg, nullptr, &units))
    return rc;
  GroupHeader h{};
  const int64_t bytes = table_layout(n, &h.desc_off, &h.map_off);
  if (capacity < bytes)
    return fail(LRQ_ERR_CAPACITY, "table needs %lld bytes, have %lld", (long long)bytes, (long long)capacity);
  char* base = static_cast<char*>(host_table);
  memset(base, 0, (size_t)bytes);
  Desc* ds = reinterpret_cast<Desc*>(base + h.desc_off);
  if (int rc = plan_group(fmt, tensors, n, in_dtype, blk_r, blk_c, flags, &cfg, ds, &units)) return rc;
  for (int64_t i = 0, next = 0; i < n; next += ds[i].units, ++i)  // the order k_build_map relies on
    if (ds[i].unit0 != next || ds[i].units < 0)
      return fail(LRQ_ERR_TABLE, "tensor %lld: work-groups out of table order", (long long)i);
  h.magic = kMagic;
  h.version = kTableVersion;
  h.cfg = cfg;
  h.n = n;
  h.units = units;
  h.bytes = bytes;
  h.dev_bytes = h.map_off + units * 4;
  memcpy(base, &h, sizeof(h));
  return 0;
}

int64_t lrq_group_device_bytes(const void* host_table) {
  g_err.clear();
  if (!host_table) return fail(LRQ_ERR_ARG, "null table");
  GroupHeader h;
  memcpy(&h, host_table, sizeof(h));
  if (h.magic != kMagic || h.version != kTableVersion) return fail(LRQ_ERR_TABLE, "not an lrq table");
  return h.dev_bytes;
}

int lrq_group_build_map(const void* host_table, void* device_table, lrq_stream_t stream) {
  g_err.clear();
  if (!host_table || !device_table) return fail(LRQ_ERR_ARG, "null table");
  GroupHeader h;
  memcpy(&h, host_table, sizeof(h));
  if (h.magic != kMagic || h.version != kTableVersion) return fail(LRQ_ERR_TABLE, "not an lrq table");
  if (!aligned(device_table, 256)) return fail(LRQ_ERR_ALIGN, "device table must be 256-byte aligned");
  if (h.cfg.kernel == lrq::kKernAmax) {
    // Set-up of a tensor-scale table: look up the static workspace's device
    // address now, so lrq_tensor_scale_grouped_static makes no symbol lookup
    // (a runtime call that is not a stream operation) when a caller captures it.
    // Best effort: the caller-workspace entry point does not need it, and the
    // static one repeats the lookup, and reports its failure, if this one failed.
    int d = -1;
    uint32_t* ws = nullptr;
    if ((stream ? hipStreamGetDevice((hipStream_t)stream, &d) : hipGetDevice(&d)) != hipSuccess ||
        lrq::static_workspace(d, &ws) != hipSuccess)
      (void)hipGetLastError();
  }
  if (h.units == 0) return 0;
  char* dev = static_cast<char*>(device_table);
  const int64_t grid = (h.units + 255) / 256;
  hipLaunchKernelGGL(k_build_map, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const Desc*>(dev + h.desc_off), h.n, h.units,
                     reinterpret_cast<uint32_t*>(dev + h.map_off));
  return check_hip(hipGetLastError(), "kernel launch");
}

int lrq_quant_grouped(const void* host_table, const void* device_table, lrq_stream_t stream) {
  g_err.clear();
  if (!host_table || !device_table) return fail(LRQ_ERR_ARG, "null table");
  GroupHeader h;
  memcpy(&h, host_table, sizeof(h));
  if (h.magic != kMagic || h.version != kTableVersion) return fail(LRQ_ERR_TABLE, "not an lrq table");
  if (h.units == 0) return 0;
  if (h.cfg.kernel == lrq::kKernAmax)
    return fail(LRQ_ERR_ARG, "a tensor-scale table needs a workspace: call lrq_tensor_scale_grouped");
  const char* dev = static_cast<const char*>(device_table);
  const Desc* descs = reinterpret_cast<const Desc*>(dev + h.desc_off);
  const uint32_t* map = reinterpret_cast<const uint32_t*>(dev + h.map_off);
  if (h.cfg.kernel == lrq::kKernCopy)
    return check_hip(lrq::launch_copy(descs, map, h.units, (hipStream_t)stream), "kernel launch");
  Desc dummy;
  memset(&dummy, 0, sizeof(dummy));
  if (h.cfg.kernel == lrq::kKernCast)
    return check_hip(lrq::launch_cast(h.cfg.in_dtype, dummy, descs, map, h.units, (hipStream_t)stream),
                     "kernel launch");
  return check_hip(lrq::launch(h.cfg, dummy, descs, map, h.units, (hipStream_t)stream), "kernel launch");
}

int64_t lrq_group_workspace_bytes(const void* host_table) {
  g_err.clear();
  if (!host_table) return fail(LRQ_ERR_ARG, "null table");
  GroupHeader h;
  memcpy(&h, host_table, sizeof(h));
  if (h.magic != kMagic || h.version != kTableVersion) return fail(LRQ_ERR_TABLE, "not an lrq table");
  return h.cfg.kernel == lrq::kKernAmax ? h.units * 4 : 0;
}

int lrq_tensor_scale_grouped(const void* host_table, const void* device_table, void* workspace,
                             int64_t workspace_bytes, lrq_stream_t stream) {
  g_err.clear();
  if (!host_table || !device_table) return fail(LRQ_ERR_ARG, "null table");
  GroupHeader h;
  memcpy(&h, host_table, sizeof(h));
  if (h.magic != kMagic || h.version != kTableVersion) return fail(LRQ_ERR_TABLE, "not an lrq table");
  if (h.cfg.kernel != lrq::kKernAmax) return fail(LRQ_ERR_ARG, "not a tensor-scale table");
  if (h.n == 0) return 0;
  if (!workspace || !aligned(workspace, 4)) return fail(LRQ_ERR_ARG, "workspace must be 4-byte aligned device memory");
  if (workspace_bytes < h.units * 4)
    return fail(LRQ_ERR_CAPACITY, "workspace needs %lld bytes, have %lld", (long long)(h.units * 4),
                (long long)workspace_bytes);
  if (h.n > 0xFFFFFFFFll / lrq::kScaleThreads)  // the finishing launch: a work-group per tensor
    return fail(LRQ_ERR_ARG, "too many tensors for one launch");
  const char* dev = static_cast<const char*>(device_table);
  const Desc* descs = reinterpret_cast<const Desc*>(dev + h.desc_off);
  const uint32_t* map = reinterpret_cast<const uint32_t*>(dev + h.map_off);
  return check_hip(lrq::launch_tensor_scale(h.cfg, descs, map, h.n, h.units, static_cast<uint32_t*>(workspace),
                                            (hipStream_t)stream),
                   "kernel launch");
}

int lrq_tensor_scale_grouped_static(const void* host_table, const void* device_table,
                                    lrq_stream_t stream) {
  g_err.clear();
  if (!host_table || !device_table) return fail(LRQ_ERR_ARG, "null table");
  GroupHeader h;
  memcpy(&h, host_table, sizeof(h));
  if (h.magic != kMagic || h.version != kTableVersion) return fail(LRQ_ERR_TABLE, "not an lrq table");
  if (h.cfg.kernel != lrq::kKernAmax) return fail(LRQ_ERR_ARG, "not a tensor-scale table");
  if (h.n == 0) return 0;
  if (h.units > (int64_t)(LRQ_STATIC_WORKSPACE_BYTES / 4))
    return fail(LRQ_ERR_CAPACITY, "table needs %lld bytes of workspace, the static workspace holds %lld",
                (long long)(h.units * 4), (long long)LRQ_STATIC_WORKSPACE_BYTES);
  if (h.n > 0xFFFFFFFFll / lrq::kScaleThreads)  // the finishing launch: a work-group per tensor
    return fail(LRQ_ERR_ARG, "too many tensors for one launch");
  int dev = -1;
  if (int rc = check_hip(stream ? hipStreamGetDevice((hipStream_t)stream, &dev) : hipGetDevice(&dev),
                         "device of the stream"))
    return rc;
  uint32_t* ws = nullptr;
  if (int rc = check_hip(lrq::static_workspace(dev, &ws), "static workspace address")) return rc;
  const char* dt = static_cast<const char*>(device_table);
  const Desc* descs = reinterpret_cast<const Desc*>(dt + h.desc_off);
  const uint32_t* map = reinterpret_cast<const uint32_t*>(dt + h.map_off);
  return check_hip(lrq::launch_tensor_scale(h.cfg, descs, map, h.n, h.units, ws, (hipStream_t)stream),
                   "kernel launch");
}

int64_t lrq_group_units(const void* host_table) {
  g_err.clear();
  if (!host_table) return fail(LRQ_ERR_ARG, "null table");
  GroupHeader h;
  memcpy(&h, host_table, sizeof(h));
  if (h.magic != kMagic || h.version != kTableVersion) return fail(LRQ_ERR_TABLE, "not an lrq table");
  return h.units;
}

int lrq_group_kernel(const void* host_table) {
  g_err.clear();
  if (!host_table) return fail(LRQ_ERR_ARG, "null table");
  GroupHeader h;
  memcpy(&h, host_table, sizeof(h));
  if (h.magic != kMagic || h.version != kTableVersion) return fail(LRQ_ERR_TABLE, "not an lrq table");
  return h.cfg.kernel;
}

const char* lrq_version(void) { return "lrq 0.1.0 gfx950"; }
const char* lrq_last_error(void) { return g_err.c_str(); }

int lrq_diag_e4m3_bits(uint32_t start, int64_t n, uint8_t* out, lrq_stream_t stream) {
  g_err.clear();
  if (n <= 0 || n % 4 != 0 || !out || !aligned(out, 4)) return fail(LRQ_ERR_ARG, "bad diag args");
  if ((n / 4 + 255) / 256 > kMaxGrid) return fail(LRQ_ERR_ARG, "n too large");
  return check_hip(lrq::launch_diag_e4m3_bits(start, n, out, (hipStream_t)stream), "kernel launch");
}

int lrq_diag_bf16_bits(uint32_t start, int64_t n, uint16_t* out, lrq_stream_t stream) {
  g_err.clear();
  if (n <= 0 || n % 2 != 0 || !out || !aligned(out, 4)) return fail(LRQ_ERR_ARG, "bad diag args");
  if ((n / 2 + 255) / 256 > kMaxGrid) return fail(LRQ_ERR_ARG, "n too large");
  return check_hip(lrq::launch_diag_bf16_bits(start, n, out, (hipStream_t)stream), "kernel launch");
}

int lrq_diag_mx_encode(int fmt, const float* in, const uint8_t* e8m0, uint8_t* out, int64_t n,
                       lrq_stream_t stream) {
  g_err.clear();
  if ((fmt != LRQ_FMT_MXFP8 && fmt != LRQ_FMT_MXFP4) || n <= 0 || n % 2 != 0 || !in || !e8m0 || !out)
    return fail(LRQ_ERR_ARG, "bad diag args");
  if ((n / 2 + 255) / 256 > kMaxGrid) return fail(LRQ_ERR_ARG, "n too large");
  return check_hip(lrq::launch_diag_mx(fmt == LRQ_FMT_MXFP8 ? 8 : 4, in, e8m0, n, out,
                                       (hipStream_t)stream), "kernel launch");
}

}  // extern "C"
