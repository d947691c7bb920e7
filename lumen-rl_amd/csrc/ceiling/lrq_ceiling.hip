// Copy-only kernels with the access patterns of the quantization kernels: the
// measured bandwidth ceilings that bench.py (--mode ceiling) sets beside the
// kernels they bound, on the same input and the same device.  No arithmetic
// beyond an XOR that keeps the loads live; the same nontemporal loads and
// stores, work-group geometry and XCD-run order as the kernel each mirrors:
//
//   k_ceil_tile<T>  : k_tile128 (128x128 tiles of bf16, T threads per tile, thread
//                     t holding 16-byte chunk t % 16 of rows t / 16 + (T/16) i),
//                     8 bytes written per chunk, runs of kXcdRunTile tiles
//   k_ceil_stream   : k_row (4 waves x kRowBlocks wave instructions of 512 bf16,
//                     1 KiB contiguous each; or 8 instructions), 8 bytes written
//                     per chunk
//   k_ceil_widen    : k_dequant's 1:2 bytes (kDequantChunks chunks per lane,
//                     8 bytes read and 16 written per chunk)
//   k_ceil_fill     : write-only, the store side of k_dequant (kDequantChunks
//                     16-byte stores per lane)
//   k_ceil_read     : read-only, the load side of k_amax (kAmaxLoads 16-byte
//                     loads per lane, one 4-byte partial per work-group)
//
// Every entry point takes `lds_bytes`, an LDS reservation per work-group that
// caps how many work-groups a CU holds (160 KiB of LDS per CU; 0: no cap): a
// bare copy at full residency can fall below a kernel that does more work per
// load, so the ceiling of a pattern is its best copy over a few caps.
//
// Measurement infrastructure only: this library is not part of the C ABI of
// include/lrq.h and the quantization path never loads it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lrq_internal.hpp"

namespace lrq {
namespace {

__device__ __forceinline__ v2u fold(v4u v) { return v2u{v.x ^ v.y, v.z ^ v.w}; }

template <int T>
__global__ __launch_bounds__(T) void k_ceil_tile(const uint16_t* __restrict__ in, uint8_t* __restrict__ out,
                                                 int64_t tiles_c, int64_t cols) {
  constexpr int NL = 2048 / T;  // 16-byte chunks per thread
  constexpr int RS = T / 16;    // rows between a thread's chunks
  const int64_t u = xcd_unit<kXcdRunTile>(blockIdx.x, gridDim.x);
  const int64_t tr = u / tiles_c, tc = u - tr * tiles_c;
  const int tid = threadIdx.x;
  const int64_t base = (tr * 128 + (tid >> 4)) * cols + tc * 128 + (tid & 15) * 8;
  v4u v[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) v[i] = load_nt(in + base + (int64_t)(RS * i) * cols);
#pragma unroll
  for (int i = 0; i < NL; ++i) store_nt(out + base + (int64_t)(RS * i) * cols, fold(v[i]));
}

template <int NL>
__global__ __launch_bounds__(256) void k_ceil_stream(const uint16_t* __restrict__ in, uint8_t* __restrict__ out) {
  const int64_t u = xcd_unit<kXcdRunRow>(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t e0 = (u * 4 + wave) * (NL * 512) + lane * 8;
  v4u v[NL];
#pragma unroll
  for (int j = 0; j < NL; ++j) v[j] = load_nt(in + e0 + j * 512);
#pragma unroll
  for (int j = 0; j < NL; ++j) store_nt(out + e0 + j * 512, fold(v[j]));
}

__global__ __launch_bounds__(256) void k_ceil_widen(const uint8_t* __restrict__ in, uint8_t* __restrict__ out) {
  const int64_t u = xcd_unit<kXcdRunStream>(blockIdx.x, gridDim.x);
  v2u v[kDequantChunks];
#pragma unroll
  for (int j = 0; j < kDequantChunks; ++j) v[j] = load_nt8(in + (u * (256 * kDequantChunks) + j * 256 + threadIdx.x) * 8);
#pragma unroll
  for (int j = 0; j < kDequantChunks; ++j) {
    const v4u w = {v[j].x, v[j].x ^ v[j].y, v[j].y, ~v[j].x};
    gst_nt<v4u>(out + (u * (256 * kDequantChunks) + j * 256 + threadIdx.x) * 16, w);
  }
}

__global__ __launch_bounds__(256) void k_ceil_fill(uint8_t* __restrict__ out) {
  const int64_t u = xcd_unit<kXcdRunStream>(blockIdx.x, gridDim.x);
  const int64_t b0 = u * (256 * 16 * kDequantChunks) + threadIdx.x * 16;
  const v4u v = {(uint32_t)u, (uint32_t)threadIdx.x, 0x3C003C00u, 0x3C003C00u};
#pragma unroll
  for (int j = 0; j < kDequantChunks; ++j) gst_nt<v4u>(out + b0 + j * 256 * 16, v);
}

__global__ __launch_bounds__(256) void k_ceil_read(const uint8_t* __restrict__ in, uint32_t* __restrict__ partials) {
  const int64_t u = xcd_unit<kXcdRunStream>(blockIdx.x, gridDim.x);
  const int64_t b0 = u * (256 * 16 * kAmaxLoads) + threadIdx.x * 16;
  v4u v[kAmaxLoads];
#pragma unroll
  for (int j = 0; j < kAmaxLoads; ++j) v[j] = load_nt(in + b0 + j * 256 * 16);
  uint32_t a = 0;
#pragma unroll
  for (int j = 0; j < kAmaxLoads; ++j) a ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  a = group_max<64>(a);
  __shared__ uint32_t red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
  __syncthreads();
  if (threadIdx.x == 0) partials[u] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

}  // namespace
}  // namespace lrq

using namespace lrq;

// 128x128 tiles of a dense bf16 [rows, cols] matrix (rows and cols multiples of
// 128) into a dense [rows, cols] byte matrix; threads = 256, 512 or 1024.
extern "C" int lrqc_tile(const void* in, void* out, int64_t rows, int64_t cols, int threads, int lds_bytes,
                         hipStream_t stream) {
  if (rows <= 0 || cols <= 0 || rows % 128 || cols % 128 || lds_bytes < 0 || lds_bytes > 65536)
    return hipErrorInvalidValue;
  const int64_t tiles_c = cols / 128, tiles = rows / 128 * tiles_c;
  if (tiles > 0x7FFFFFFF) return hipErrorInvalidValue;
  const dim3 grid((unsigned)tiles);
  const auto* x = static_cast<const uint16_t*>(in);
  auto* y = static_cast<uint8_t*>(out);
  switch (threads) {
    case 256: hipLaunchKernelGGL(k_ceil_tile<256>, grid, dim3(256), lds_bytes, stream, x, y, tiles_c, cols); break;
    case 512: hipLaunchKernelGGL(k_ceil_tile<512>, grid, dim3(512), lds_bytes, stream, x, y, tiles_c, cols); break;
    case 1024: hipLaunchKernelGGL(k_ceil_tile<1024>, grid, dim3(1024), lds_bytes, stream, x, y, tiles_c, cols); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// `elems` contiguous bf16 (a multiple of 2048 * loads) into `elems` bytes,
// loads = 4 (k_row's kRowBlocks) or 8 wave instructions per lane.
extern "C" int lrqc_stream(const void* in, void* out, int64_t elems, int loads, int lds_bytes, hipStream_t stream) {
  if ((loads != 4 && loads != 8) || lds_bytes < 0 || lds_bytes > 65536) return hipErrorInvalidValue;
  const int64_t per_wg = 4 * 512 * (int64_t)loads;
  if (elems <= 0 || elems % per_wg || elems / per_wg > 0x7FFFFFFF) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(elems / per_wg));
  const auto* x = static_cast<const uint16_t*>(in);
  auto* y = static_cast<uint8_t*>(out);
  if (loads == 4) hipLaunchKernelGGL(k_ceil_stream<4>, grid, dim3(256), lds_bytes, stream, x, y);
  else hipLaunchKernelGGL(k_ceil_stream<8>, grid, dim3(256), lds_bytes, stream, x, y);
  return hipGetLastError();
}

// `chunks` 8-byte chunks (a multiple of 256 * kDequantChunks) into as many
// 16-byte chunks: k_dequant's 1:2 pattern (8 codes in, 8 bf16 out per chunk).
extern "C" int lrqc_widen(const void* in, void* out, int64_t chunks, int lds_bytes, hipStream_t stream) {
  constexpr int64_t per_wg = 256 * kDequantChunks;
  if (chunks <= 0 || chunks % per_wg || chunks / per_wg > 0x7FFFFFFF || lds_bytes < 0 || lds_bytes > 65536)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ceil_widen, dim3((unsigned)(chunks / per_wg)), dim3(256), lds_bytes, stream,
                     static_cast<const uint8_t*>(in), static_cast<uint8_t*>(out));
  return hipGetLastError();
}

// Writes `bytes` (a multiple of 4096 * kDequantChunks).
extern "C" int lrqc_fill(void* out, int64_t bytes, int lds_bytes, hipStream_t stream) {
  constexpr int64_t per_wg = 256 * 16 * kDequantChunks;
  if (bytes <= 0 || bytes % per_wg || bytes / per_wg > 0x7FFFFFFF || lds_bytes < 0 || lds_bytes > 65536)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ceil_fill, dim3((unsigned)(bytes / per_wg)), dim3(256), lds_bytes, stream,
                     static_cast<uint8_t*>(out));
  return hipGetLastError();
}

// Reads `bytes` (a multiple of 4096 * kAmaxLoads); writes one uint32 per
// work-group to `partials` (lrqc_read_partials(bytes) of them).
extern "C" int64_t lrqc_read_partials(int64_t bytes) { return bytes / (256 * 16 * kAmaxLoads); }

extern "C" int lrqc_read(const void* in, int64_t bytes, uint32_t* partials, int lds_bytes, hipStream_t stream) {
  constexpr int64_t per_wg = 256 * 16 * kAmaxLoads;
  if (bytes <= 0 || bytes % per_wg || bytes / per_wg > 0x7FFFFFFF || lds_bytes < 0 || lds_bytes > 65536)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ceil_read, dim3((unsigned)(bytes / per_wg)), dim3(256), lds_bytes, stream,
                     static_cast<const uint8_t*>(in), partials);
  return hipGetLastError();
}
