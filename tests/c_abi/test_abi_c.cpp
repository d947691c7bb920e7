// A C/C++ caller of liblrq with no torch: device buffers from hipMalloc, the
// grouped table packed on the host and uploaded by hand, every result compared
// byte for byte with the CPU oracle (oracle/lrq_oracle.c, test infrastructure).
// Prints one line per check and "c-abi ok" at the end; exits non-zero on the
// first mismatch or error.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "lrq.h"

extern "C" {
int lrqo_fp8_block_quant(const void* in, int in_dtype, int arith, int64_t batch, int64_t rows,
                         int64_t cols, int64_t ld, int64_t bstride, int64_t blk_r, int64_t blk_c,
                         int pow2, uint8_t* codes, void* scales, int nthreads);
int lrqo_mx_quant(const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t ld, int fmt,
                  uint8_t* codes, uint8_t* scales, int nthreads);
int lrqo_act_qdq(const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t blk, int pow2,
                 float* out, int nthreads);
uint32_t lrqo_tensor_scale(const void* in, int in_dtype, int64_t n);
int lrqo_fp8_block_quant_f64(const double* in, int64_t batch, int64_t rows, int64_t cols,
                             int64_t ld, int64_t bstride, int64_t blk_r, int64_t blk_c,
                             int pow2, uint8_t* codes, double* scales, int nthreads);
void lrqo_f32_to_e4m3_n(const float* in, uint8_t* out, int64_t n);
}

#define HIP(x)                                                                  \
  do {                                                                          \
    hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                     \
      fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      exit(2);                                                                  \
    }                                                                           \
  } while (0)
#define LRQ(x)                                                                  \
  do {                                                                          \
    int r_ = (x);                                                               \
    if (r_ != 0) {                                                              \
      fprintf(stderr, "lrq error %d at line %d: %s\n", r_, __LINE__, lrq_last_error()); \
      exit(3);                                                                  \
    }                                                                           \
  } while (0)

static void expect(bool ok, const char* what) {
  printf("%-44s %s\n", what, ok ? "ok" : "MISMATCH");
  fflush(stdout);
  if (!ok) exit(1);
}

// Seeded bf16 weights: N(0, 0.02^2)-like values with a few outliers and one
// all-zero 128x128 tile.
static std::vector<uint16_t> make_weights(int64_t rows, int64_t cols, uint32_t seed) {
  std::vector<uint16_t> w((size_t)(rows * cols));
  uint32_t s = seed;
  for (size_t i = 0; i < w.size(); ++i) {
    float acc = 0.0f;
    for (int k = 0; k < 4; ++k) {
      s = s * 1664525u + 1013904223u;
      acc += (float)(s >> 8) / 16777216.0f - 0.5f;
    }
    float f = acc * 0.035f;
    if ((s & 1023u) == 7u) f *= 80.0f;
    uint32_t b;
    memcpy(&b, &f, 4);
    w[i] = (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
  }
  for (int64_t r = 0; r < 128 && r < rows; ++r)
    for (int64_t c = 0; c < 128 && c < cols; ++c) w[(size_t)(r * cols + c)] = 0;
  return w;
}

int main() {
  int ndev = 0;
  HIP(hipGetDeviceCount(&ndev));
  if (ndev < 1) {
    fprintf(stderr, "no HIP device\n");
    return 4;
  }
  printf("%s\n", lrq_version());
  hipStream_t st;
  HIP(hipStreamCreate(&st));

  // two weights of one layer: [512, 1024] and [256, 3072]
  const int64_t R[2] = {512, 256}, C[2] = {1024, 3072};
  std::vector<uint16_t> hw[2] = {make_weights(R[0], C[0], 1u), make_weights(R[1], C[1], 2u)};
  void* dw[2];
  uint8_t* dcodes[2];
  float* dscales[2];
  for (int i = 0; i < 2; ++i) {
    HIP(hipMalloc(&dw[i], hw[i].size() * 2));
    HIP(hipMemcpy(dw[i], hw[i].data(), hw[i].size() * 2, hipMemcpyHostToDevice));
    HIP(hipMalloc(&dcodes[i], (size_t)(R[i] * C[i])));
    HIP(hipMalloc(&dscales[i], (size_t)(R[i] * C[i] / 128) * 4));
  }

  // 1. single tensor, 128x128 tiles and 1x128 rows
  for (int blk_r : {128, 1}) {
    const int64_t ns = (R[0] / blk_r) * (C[0] / 128);
    LRQ(lrq_fp8_block_quant(dw[0], LRQ_DTYPE_BF16, 1, R[0], C[0], C[0], R[0] * C[0], blk_r, 128,
                            dcodes[0], dscales[0], 0, (lrq_stream_t)st));
    HIP(hipStreamSynchronize(st));
    std::vector<uint8_t> got((size_t)(R[0] * C[0])), want(got.size());
    std::vector<float> gs((size_t)ns), ws(gs.size());
    HIP(hipMemcpy(got.data(), dcodes[0], got.size(), hipMemcpyDeviceToHost));
    HIP(hipMemcpy(gs.data(), dscales[0], gs.size() * 4, hipMemcpyDeviceToHost));
    lrqo_fp8_block_quant(hw[0].data(), LRQ_DTYPE_BF16, 0, 1, R[0], C[0], C[0], R[0] * C[0], blk_r, 128,
                         0, want.data(), ws.data(), 0);
    expect(got == want && memcmp(gs.data(), ws.data(), gs.size() * 4) == 0,
           blk_r == 128 ? "lrq_fp8_block_quant 128x128" : "lrq_fp8_block_quant 1x128");
  }

  // 1b. a view one element into weight 1 (2-byte aligned rows, pitch 3072),
  // 255 x 2304, in 1x128 and 1x36 blocks (36: the last 8-element chunk of each
  // block overlaps its neighbour)
  {
    const int64_t vr = 255, vc = 2304, vld = C[1];
    const uint16_t* dv = static_cast<const uint16_t*>(dw[1]) + 1;
    std::vector<uint16_t> hv((size_t)(vr * vc));
    for (int64_t r = 0; r < vr; ++r)
      memcpy(&hv[(size_t)(r * vc)], &hw[1][(size_t)(1 + r * vld)], (size_t)vc * 2);
    float* dvs;  // scales of the narrowest blocks: vr * vc / 36 floats
    HIP(hipMalloc(&dvs, (size_t)(vr * (vc / 36)) * 4));
    for (int64_t bc : {128, 36}) {
      const int64_t ns = vr * (vc / bc);
      LRQ(lrq_fp8_block_quant(dv, LRQ_DTYPE_BF16, 1, vr, vc, vld, vr * vld, 1, bc, dcodes[1], dvs, 0,
                              (lrq_stream_t)st));
      HIP(hipStreamSynchronize(st));
      std::vector<uint8_t> got((size_t)(vr * vc)), want(got.size());
      std::vector<float> gs((size_t)ns), ws(gs.size());
      HIP(hipMemcpy(got.data(), dcodes[1], got.size(), hipMemcpyDeviceToHost));
      HIP(hipMemcpy(gs.data(), dvs, gs.size() * 4, hipMemcpyDeviceToHost));
      lrqo_fp8_block_quant(hv.data(), LRQ_DTYPE_BF16, 0, 1, vr, vc, vc, vr * vc, 1, bc, 0, want.data(), ws.data(), 0);
      expect(got == want && memcmp(gs.data(), ws.data(), gs.size() * 4) == 0,
             bc == 128 ? "lrq_fp8_block_quant 1x128, offset view" : "lrq_fp8_block_quant 1x36, offset view");
    }
    HIP(hipFree(dvs));
  }

  // 2. grouped: both tensors in one launch through a hand-uploaded table
  lrq_tensor ts[2];
  for (int i = 0; i < 2; ++i) {
    ts[i].in = dw[i];
    ts[i].codes = dcodes[i];
    ts[i].scales = dscales[i];
    ts[i].batch = 1;
    ts[i].rows = R[i];
    ts[i].cols = C[i];
    ts[i].ld = C[i];
    ts[i].batch_stride = R[i] * C[i];
  }
  const int64_t bytes = lrq_group_table_bytes(LRQ_FMT_FP8_BLOCK, ts, 2, LRQ_DTYPE_BF16, 128, 128, 0);
  if (bytes <= 0) LRQ((int)bytes);
  std::vector<uint8_t> host_table((size_t)bytes);
  LRQ(lrq_group_pack(LRQ_FMT_FP8_BLOCK, ts, 2, LRQ_DTYPE_BF16, 128, 128, 0, host_table.data(), bytes));
  void* dev_table;
  const int64_t dev_bytes = lrq_group_device_bytes(host_table.data());
  if (dev_bytes < bytes) LRQ((int)dev_bytes);
  HIP(hipMalloc(&dev_table, (size_t)dev_bytes));
  HIP(hipMemcpy(dev_table, host_table.data(), (size_t)bytes, hipMemcpyHostToDevice));
  LRQ(lrq_group_build_map(host_table.data(), dev_table, (lrq_stream_t)st));
  for (int i = 0; i < 2; ++i) HIP(hipMemset(dcodes[i], 0xAB, (size_t)(R[i] * C[i])));
  LRQ(lrq_quant_grouped(host_table.data(), dev_table, (lrq_stream_t)st));
  HIP(hipStreamSynchronize(st));
  bool same = lrq_group_units(host_table.data()) == (R[0] / 128) * (C[0] / 128) + (R[1] / 128) * (C[1] / 128);
  same = same && lrq_group_kernel(host_table.data()) >= 0 && lrq_group_kernel(nullptr) == LRQ_ERR_ARG;
  for (int i = 0; i < 2; ++i) {
    const int64_t ns = (R[i] / 128) * (C[i] / 128);
    std::vector<uint8_t> got((size_t)(R[i] * C[i])), want(got.size());
    std::vector<float> gs((size_t)ns), ws(gs.size());
    HIP(hipMemcpy(got.data(), dcodes[i], got.size(), hipMemcpyDeviceToHost));
    HIP(hipMemcpy(gs.data(), dscales[i], gs.size() * 4, hipMemcpyDeviceToHost));
    lrqo_fp8_block_quant(hw[i].data(), LRQ_DTYPE_BF16, 0, 1, R[i], C[i], C[i], R[i] * C[i], 128, 128, 0,
                         want.data(), ws.data(), 0);
    same = same && got == want && memcmp(gs.data(), ws.data(), gs.size() * 4) == 0;
  }
  expect(same, "lrq_group_pack + lrq_quant_grouped (2 tensors)");

  // 3. MXFP8 / MXFP4 of tensor 1
  for (int fmt : {8, 4}) {
    const int64_t cb = fmt == 8 ? R[1] * C[1] : R[1] * C[1] / 2;
    uint8_t* dsc;
    HIP(hipMalloc(&dsc, (size_t)(R[1] * C[1] / 32)));
    if (fmt == 8) LRQ(lrq_mxfp8_quant(dw[1], LRQ_DTYPE_BF16, R[1], C[1], C[1], dcodes[1], dsc, (lrq_stream_t)st));
    else LRQ(lrq_mxfp4_quant(dw[1], LRQ_DTYPE_BF16, R[1], C[1], C[1], dcodes[1], dsc, (lrq_stream_t)st));
    HIP(hipStreamSynchronize(st));
    std::vector<uint8_t> got((size_t)cb), want(got.size()), gs((size_t)(R[1] * C[1] / 32)), ws(gs.size());
    HIP(hipMemcpy(got.data(), dcodes[1], got.size(), hipMemcpyDeviceToHost));
    HIP(hipMemcpy(gs.data(), dsc, gs.size(), hipMemcpyDeviceToHost));
    lrqo_mx_quant(hw[1].data(), LRQ_DTYPE_BF16, R[1], C[1], C[1], fmt, want.data(), ws.data(), 0);
    expect(got == want && gs == ws, fmt == 8 ? "lrq_mxfp8_quant" : "lrq_mxfp4_quant");
    HIP(hipFree(dsc));
  }

  // 4. activation fake-quant of tensor 0 viewed as 512 tokens x 1024
  {
    float* dout;
    HIP(hipMalloc(&dout, (size_t)(R[0] * C[0]) * 4));
    LRQ(lrq_act_qdq(dw[0], LRQ_DTYPE_BF16, R[0], C[0], C[0], 128, 0, dout, (lrq_stream_t)st));
    HIP(hipStreamSynchronize(st));
    std::vector<float> got((size_t)(R[0] * C[0])), want(got.size());
    HIP(hipMemcpy(got.data(), dout, got.size() * 4, hipMemcpyDeviceToHost));
    lrqo_act_qdq(hw[0].data(), LRQ_DTYPE_BF16, R[0], C[0], 128, 0, want.data(), 0);
    expect(memcmp(got.data(), want.data(), got.size() * 4) == 0, "lrq_act_qdq");
    HIP(hipFree(dout));
  }

  // 5. per-tensor scales of both tensors with a caller workspace
  {
    float* dsc;
    HIP(hipMalloc(&dsc, 2 * sizeof(float)));
    lrq_tensor tt[2] = {ts[0], ts[1]};
    tt[0].codes = tt[1].codes = nullptr;
    tt[0].scales = dsc;
    tt[1].scales = dsc + 1;
    const int64_t tb = lrq_group_table_bytes(LRQ_FMT_TENSOR_SCALE, tt, 2, LRQ_DTYPE_BF16, 1, 1, 0);
    if (tb <= 0) LRQ((int)tb);
    std::vector<uint8_t> ht((size_t)tb);
    LRQ(lrq_group_pack(LRQ_FMT_TENSOR_SCALE, tt, 2, LRQ_DTYPE_BF16, 1, 1, 0, ht.data(), tb));
    void* dt;
    HIP(hipMalloc(&dt, (size_t)lrq_group_device_bytes(ht.data())));
    HIP(hipMemcpy(dt, ht.data(), (size_t)tb, hipMemcpyHostToDevice));
    LRQ(lrq_group_build_map(ht.data(), dt, (lrq_stream_t)st));
    const int64_t wsb = lrq_group_workspace_bytes(ht.data());
    void* dws;
    HIP(hipMalloc(&dws, (size_t)wsb));
    LRQ(lrq_tensor_scale_grouped(ht.data(), dt, dws, wsb, (lrq_stream_t)st));
    HIP(hipStreamSynchronize(st));
    uint32_t got[2];
    HIP(hipMemcpy(got, dsc, sizeof(got), hipMemcpyDeviceToHost));
    const bool ok = got[0] == lrqo_tensor_scale(hw[0].data(), LRQ_DTYPE_BF16, R[0] * C[0]) &&
                    got[1] == lrqo_tensor_scale(hw[1].data(), LRQ_DTYPE_BF16, R[1] * C[1]);
    expect(ok, "lrq_tensor_scale_grouped");
    // the same tables through the entry point that allocates nothing: the library's
    // static workspace instead of dws, twice (the second call reuses its contents)
    for (int rep = 0; rep < 2; ++rep) {
      HIP(hipMemset(dsc, 0xFF, 2 * sizeof(float)));
      LRQ(lrq_tensor_scale_grouped_static(ht.data(), dt, (lrq_stream_t)st));
      HIP(hipStreamSynchronize(st));
      uint32_t got2[2];
      HIP(hipMemcpy(got2, dsc, sizeof(got2), hipMemcpyDeviceToHost));
      expect(got2[0] == got[0] && got2[1] == got[1], "lrq_tensor_scale_grouped_static");
    }
    HIP(hipFree(dws));
    HIP(hipFree(dt));
    HIP(hipFree(dsc));
  }

  // 5b. float64 input in float64 arithmetic (quantize_tensor on a float64 tensor):
  //     tensor 0's values scaled off the bf16 grid, 1x128 blocks, float64 scales
  {
    const int64_t n = R[0] * C[0];
    std::vector<double> hx((size_t)n);
    for (int64_t i = 0; i < n; ++i) {
      uint32_t b = (uint32_t)hw[0][(size_t)i] << 16;
      float f;
      memcpy(&f, &b, 4);
      hx[(size_t)i] = (double)f * (1.0 + 1e-9 * (double)(i % 7));
    }
    for (int pow2 = 0; pow2 < 2; ++pow2) {
      double* dx;
      uint8_t* dq;
      double* ds;
      const int64_t ns = R[0] * (C[0] / 128);
      HIP(hipMalloc(&dx, (size_t)n * 8));
      HIP(hipMalloc(&dq, (size_t)n));
      HIP(hipMalloc(&ds, (size_t)ns * 8));
      HIP(hipMemcpy(dx, hx.data(), (size_t)n * 8, hipMemcpyHostToDevice));
      const unsigned flags = LRQ_FLAG_NATIVE_ARITH | (pow2 ? LRQ_FLAG_POW2_SCALE : 0u);
      LRQ(lrq_fp8_block_quant(dx, LRQ_DTYPE_F64, 1, R[0], C[0], C[0], R[0] * C[0], 1, 128, dq, ds, flags,
                              (lrq_stream_t)st));
      HIP(hipStreamSynchronize(st));
      std::vector<uint8_t> gq((size_t)n), wq((size_t)n);
      std::vector<double> gs((size_t)ns), wsc((size_t)ns);
      HIP(hipMemcpy(gq.data(), dq, (size_t)n, hipMemcpyDeviceToHost));
      HIP(hipMemcpy(gs.data(), ds, (size_t)ns * 8, hipMemcpyDeviceToHost));
      lrqo_fp8_block_quant_f64(hx.data(), 1, R[0], C[0], C[0], R[0] * C[0], 1, 128, pow2, wq.data(),
                               wsc.data(), 0);
      expect(memcmp(gq.data(), wq.data(), (size_t)n) == 0 && memcmp(gs.data(), wsc.data(), (size_t)ns * 8) == 0,
             pow2 ? "lrq_fp8_block_quant float64, pow2" : "lrq_fp8_block_quant float64");
      HIP(hipFree(ds));
      HIP(hipFree(dq));
      HIP(hipFree(dx));
    }
  }

  // 6. unscaled e4m3 cast of tensor 1 (x 300, so values pass 448 -> NaN) and of an
  //    odd-length, 2-byte-offset slice of it (element-wise path and tail)
  {
    const int64_t n = R[1] * C[1];
    std::vector<uint16_t> hx((size_t)n);
    std::vector<float> fx((size_t)n);
    for (int64_t i = 0; i < n; ++i) {
      uint32_t b = (uint32_t)hw[1][(size_t)i] << 16;
      float f;
      memcpy(&f, &b, 4);
      f *= 300.0f;
      memcpy(&b, &f, 4);
      hx[(size_t)i] = (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
      b = (uint32_t)hx[(size_t)i] << 16;
      memcpy(&fx[(size_t)i], &b, 4);
    }
    void* dx;
    uint8_t* dq;
    HIP(hipMalloc(&dx, (size_t)n * 2));
    HIP(hipMalloc(&dq, (size_t)n));
    HIP(hipMemcpy(dx, hx.data(), (size_t)n * 2, hipMemcpyHostToDevice));
    std::vector<uint8_t> want((size_t)n), got((size_t)n);
    lrqo_f32_to_e4m3_n(fx.data(), want.data(), n);
    LRQ(lrq_cast_e4m3(dx, LRQ_DTYPE_BF16, n, dq, (lrq_stream_t)st));
    HIP(hipStreamSynchronize(st));
    HIP(hipMemcpy(got.data(), dq, (size_t)n, hipMemcpyDeviceToHost));
    expect(memcmp(got.data(), want.data(), (size_t)n) == 0, "lrq_cast_e4m3 (vector path)");
    const int64_t m = n - 1001;
    LRQ(lrq_cast_e4m3(static_cast<uint16_t*>(dx) + 1, LRQ_DTYPE_BF16, m, dq, (lrq_stream_t)st));
    HIP(hipStreamSynchronize(st));
    HIP(hipMemcpy(got.data(), dq, (size_t)m, hipMemcpyDeviceToHost));
    expect(memcmp(got.data(), want.data() + 1, (size_t)m) == 0, "lrq_cast_e4m3 (offset, odd length)");
    HIP(hipFree(dq));
    HIP(hipFree(dx));
  }

  // 7. MXFP8 dequant of tensor 1's codes back to fp32: exact products, so the
  //    reference value is the decoded code times 2^(E-127) computed on the host
  {
    const int64_t n = R[1] * C[1], g = n / 32;
    uint8_t *dq8, *ds8;
    float* dout;
    HIP(hipMalloc(&dq8, (size_t)n));
    HIP(hipMalloc(&ds8, (size_t)g));
    HIP(hipMalloc(&dout, (size_t)n * 4));
    LRQ(lrq_mxfp8_quant(dw[1], LRQ_DTYPE_BF16, R[1], C[1], C[1], dq8, ds8, (lrq_stream_t)st));
    LRQ(lrq_mx_dequant(LRQ_FMT_MXFP8, dq8, ds8, R[1], C[1], dout, LRQ_DTYPE_F32, (lrq_stream_t)st));
    HIP(hipStreamSynchronize(st));
    std::vector<uint8_t> q((size_t)n), sc((size_t)g);
    std::vector<float> got((size_t)n);
    HIP(hipMemcpy(q.data(), dq8, (size_t)n, hipMemcpyDeviceToHost));
    HIP(hipMemcpy(sc.data(), ds8, (size_t)g, hipMemcpyDeviceToHost));
    HIP(hipMemcpy(got.data(), dout, (size_t)n * 4, hipMemcpyDeviceToHost));
    bool ok = true;
    for (int64_t i = 0; i < n && ok; ++i) {
      const uint32_t c = q[(size_t)i], e = (c >> 3) & 15u, m = c & 7u, E = sc[(size_t)(i / 32)];
      if ((c & 0x7Fu) == 0x7Fu || E == 0xFFu) continue;  // NaN rules are covered by the Python tests
      const double v = (e ? (1.0 + m / 8.0) * ldexp(1.0, (int)e - 7) : m * ldexp(1.0, -9)) * ((c & 0x80u) ? -1 : 1);
      ok = got[(size_t)i] == (float)ldexp(v, (int)E - 127);
    }
    expect(ok, "lrq_mxfp8_quant + lrq_mx_dequant (fp32)");
    HIP(hipFree(dout));
    HIP(hipFree(ds8));
    HIP(hipFree(dq8));
  }

  // 8. argument errors come back as codes with a message, not as faults
  {
    const int rc = lrq_fp8_block_quant(dw[0], LRQ_DTYPE_BF16, 1, R[0], C[0], C[0] - 1, R[0] * C[0], 128, 128,
                                       dcodes[0], dscales[0], 0, (lrq_stream_t)st);
    expect(rc == LRQ_ERR_ARG && strlen(lrq_last_error()) > 0, "ld < cols rejected with LRQ_ERR_ARG");
  }

  HIP(hipFree(dev_table));
  for (int i = 0; i < 2; ++i) {
    HIP(hipFree(dw[i]));
    HIP(hipFree(dcodes[i]));
    HIP(hipFree(dscales[i]));
  }
  HIP(hipStreamDestroy(st));
  printf("c-abi ok\n");
  return 0;
}
