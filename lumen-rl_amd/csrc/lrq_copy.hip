// Grouped byte copy: the pass-through tensors of a weight-transfer bucket
// (norms, embeddings, lm_head: lumenrl/engine/inference/bucketed_weight_transfer.py:137-165
// copies every tensor into the bucket) moved by ONE launch next to the grouped
// quantize, instead of one copy per tensor.
//
// A work-group moves one 4 KiB unit of one tensor: one 16-byte nontemporal
// load and store per lane, each wave instruction covering 1 KiB contiguous
// (4 KiB units measured 3% faster than 8 KiB and 4% faster than 16 KiB).  Source and destination are 16-byte aligned (checked by
// the packer); the last n % 16 bytes of a tensor are copied bytewise by the
// unit that holds them.
#include <string.h>

#include "lrq.h"
#include "lrq_device.hpp"
#include "lrq_internal.hpp"

namespace lrq {

__global__ __launch_bounds__(256) void k_copy(Desc single, const Desc* __restrict__ descs,
                                              const uint32_t* __restrict__ map) {
  Desc d;
  int64_t u;
  pick_desc<kXcdRunStream>(single, descs, map, d, u);
  const int64_t n = d.cols;  // bytes
  const char* src = static_cast<const char*>(d.in);
  char* dst = reinterpret_cast<char*>(d.codes);
  const int64_t base = u * kCopyUnit;
  const int tid = threadIdx.x;
  constexpr int kLoads = (int)(kCopyUnit / 4096);  // 16-byte loads per lane
  v4u v[kLoads];
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const int64_t off = base + (int64_t)(256 * j + tid) * 16;
    v[j] = off + 16 <= n ? load_nt(src + off) : v4u{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const int64_t off = base + (int64_t)(256 * j + tid) * 16;
    if (off + 16 <= n) gst_nt<v4u>(dst + off, v[j]);
  }
  const int64_t n16 = n & ~int64_t(15);
  if (n16 < n && n16 >= base && n16 < base + kCopyUnit && tid < n - n16) gst<char>(dst + n16 + tid, gld<char>(src + n16 + tid));
}

hipError_t launch_copy(const Desc* descs, const uint32_t* map, int64_t units, hipStream_t stream) {
  Desc none;
  memset(&none, 0, sizeof(none));
  hipLaunchKernelGGL(k_copy, dim3((unsigned)units), dim3(256), 0, stream, none, descs, map);
  return hipGetLastError();
}

}  // namespace lrq
