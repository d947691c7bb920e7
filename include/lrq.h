/*
 * lrq.h -- C ABI of the MI355X (gfx950) weight-quantization library
 * (liblrq.so): bf16/fp16/fp32 weights -> blockwise FP8 E4M3, MXFP8, MXFP4.
 *
 * The reference (Lumen-RL) is pure Python and has no FFI; each entry point
 * below states which reference interface it replaces.  A caller binds these
 * with ctypes (the shipped Python package does), cffi or plain C.
 *
 * Conventions
 *   - Every pointer argument named in/codes/scales/out is DEVICE memory the
 *     caller allocated (torch does, in the Python package).  The library never
 *     allocates or frees device memory (its one static device array is part of
 *     the loaded code object).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and
 *     is stream-ordered; no entry point synchronizes the device.
 *   - Return 0 on success, LRQ_ERR_* (< 0) for a rejected argument, or a
 *     positive hipError_t if the HIP runtime failed.  lrq_last_error() gives
 *     the message of the last failure on the calling thread.
 *   - Element counts and strides are in elements of the input dtype.
 *   - Layouts: codes are dense row-major [batch, rows, cols] (e4m3 bytes) or
 *     [rows, cols/2] (e2m1, element 2i in the low nibble of byte i).
 *   - Entry points are re-entrant.  The library keeps no device state other
 *     than the static workspace of lrq_tensor_scale_grouped_static.
 */
#ifndef LRQ_H_
#define LRQ_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* lrq_stream_t; /* == hipStream_t */

/* input / scale dtypes */
#define LRQ_DTYPE_BF16 0
#define LRQ_DTYPE_F16 1
#define LRQ_DTYPE_F32 2
#define LRQ_DTYPE_F64 3 /* FP8 block quantization only (lrq_fp8_block_quant and LRQ_FMT_FP8_BLOCK
                           tables), with LRQ_FLAG_NATIVE_ARITH: float64 arithmetic and
                           float64 scales, as quantize_tensor on a float64 tensor
                           (weight_quantizer.py:59-71, the quotient rounded to float32 at
                           :68 before the e4m3 cast) */

/* flags */
#define LRQ_FLAG_POW2_SCALE 1u   /* FP8Config.use_weight_pow2_scale (fp8_config.py:22) */
#define LRQ_FLAG_NATIVE_ARITH 2u /* arithmetic in the input dtype (quantize_tensor on a
                                    bf16/fp16 tensor) instead of float32 */
#define LRQ_FLAG_SCALE_BF16 4u   /* write float32-arithmetic scales rounded to bf16, the
                                    `_fp8_scales` sidecar of quantize_state_dict
                                    (weight_quantizer.py:111) */
#define LRQ_FLAG_OUT_BF16 8u     /* grouped dequant: bf16 output (dequantize_state_dict) */

/* formats (grouped launches) */
#define LRQ_FMT_FP8_BLOCK 0
#define LRQ_FMT_MXFP8 1
#define LRQ_FMT_MXFP4 2
#define LRQ_FMT_FP8_DEQUANT 3 /* grouped dequant: lrq_tensor.in = codes, .codes = output,
                                 in_dtype = scale dtype, LRQ_FLAG_OUT_BF16 = bf16 output */
#define LRQ_FMT_TENSOR_SCALE 4 /* per-tensor FP8 scale (lrq_tensor_scale_grouped):
                                  lrq_tensor.in = weight, .scales = one float32 out,
                                  .codes unused (may be NULL) */
#define LRQ_FMT_COPY 5 /* grouped byte copy through lrq_quant_grouped: lrq_tensor.in =
                          source, .codes = destination (both 16-byte aligned), .cols =
                          bytes, batch = rows = 1, .ld = .cols, .scales unused (may be
                          NULL); in_dtype must be a valid dtype and is otherwise ignored.
                          The pass-through tensors of a weight-transfer bucket in one
                          launch (bucketed_weight_transfer.py:137-165 copies each) */
#define LRQ_FMT_MXFP8_DEQUANT 7 /* grouped MX dequant through lrq_quant_grouped (see
                                   lrq_mx_dequant): lrq_tensor.in = codes, .codes =
                                   output, .scales = E8M0 bytes; dense [batch, rows,
                                   cols] with cols % 32 == 0; LRQ_FLAG_OUT_BF16 = bf16
                                   output; in_dtype must be a valid dtype, else unused */
#define LRQ_FMT_MXFP4_DEQUANT 8
#define LRQ_FMT_CAST_E4M3 6 /* grouped unscaled cast through lrq_quant_grouped (see
                               lrq_cast_e4m3): lrq_tensor.in = source (in_dtype),
                               .codes = e4m3fn output, .cols = elements, batch = rows
                               = 1, .ld = .cols, .scales unused (may be NULL) */

/* errors */
#define LRQ_ERR_ARG (-1)      /* invalid argument (shape, dtype, block size, null) */
#define LRQ_ERR_ALIGN (-2)    /* pointer/stride alignment a format requires */
#define LRQ_ERR_CAPACITY (-3) /* caller buffer too small */
#define LRQ_ERR_TABLE (-4)    /* grouped table corrupt or from another version */

/*
 * Blockwise FP8 E4M3 quantization with one scale per blk_r x blk_c block.
 * Replaces WeightQuantizer.quantize_tensor
 * (lumenrl/quantization/weight_quantizer.py:40-77) -- blk_r = 1,
 * blk_c = block_size -- and the 128x128 `weight_scale_inv` tiling that vLLM /
 * ATOM per-block FP8 loaders consume (blk_r = blk_c = 128;
 * lumenrl/engine/inference/vllm_fp8_utils.py:104-118).
 *   in      : batch matrices [rows, cols]; row r of matrix b at
 *             in + b*batch_stride + r*ld (elements of in_dtype).
 *   codes   : [batch, rows, cols] e4m3fn bytes.
 *   scales  : [batch, ceil(rows/blk_r), ceil(cols/blk_c)]: float32, or values of
 *             the input dtype with LRQ_FLAG_NATIVE_ARITH (16-bit words, or float64
 *             for LRQ_DTYPE_F64), or bf16 with LRQ_FLAG_SCALE_BF16.  Edge blocks
 *             may be partial.
 * in needs element alignment only (any ld): with codes aligned to 8 bytes and
 * cols % 8 == 0, 128x128 tiles and 1xB blocks of 8 <= B <= 65536 run on the
 * vector kernels; other shapes and alignments on the generic kernel.
 * Bit-exact with the reference evaluated by torch on x86, including NaN, inf,
 * all-zero and subnormal blocks.
 */
int lrq_fp8_block_quant(const void* in, int in_dtype, int64_t batch, int64_t rows,
                        int64_t cols, int64_t ld, int64_t batch_stride, int64_t blk_r,
                        int64_t blk_c, uint8_t* codes, void* scales, unsigned flags,
                        lrq_stream_t stream);

/*
 * Inverse: out = fp32(code) * fp32(scale) per block.  Replaces
 * WeightQuantizer.dequantize_tensor (weight_quantizer.py:79-89); out_dtype
 * LRQ_DTYPE_BF16 adds the `.to(torch.bfloat16)` of dequantize_state_dict
 * (:133).  scale_dtype: LRQ_DTYPE_F32 / _BF16 / _F16.  out_dtype: _F32 / _BF16.
 */
int lrq_fp8_block_dequant(const uint8_t* codes, const void* scales, int scale_dtype,
                          int64_t batch, int64_t rows, int64_t cols, int64_t blk_r,
                          int64_t blk_c, void* out, int out_dtype, lrq_stream_t stream);

/*
 * MXFP8: E4M3 codes [rows, cols] plus one E8M0 byte per 1x32 group along cols
 * (scales [rows, cols/32]).  MXFP4: E2M1 codes [rows, cols/2] and the same
 * scales.  cols must be a multiple of 32.  No reference function (the
 * reference delegates MX to absent aiter/vLLM code:
 * examples/DAPO/atom_aiter_shim/sitecustomize.py:31-32,
 * examples/Qwen3_8B_SDDD_MI350_vLLM/configs/opd_qwen3_8b.yaml:43); the rules
 * are OCP MX v1.0 with round-to-nearest-even and saturation.  in needs element
 * alignment only (any ld); codes aligned to 8 bytes (MXFP8) or 4 (MXFP4) take
 * the vector kernel, others the generic one.
 */
int lrq_mxfp8_quant(const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t ld,
                    uint8_t* codes, uint8_t* scales, lrq_stream_t stream);
int lrq_mxfp4_quant(const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t ld,
                    uint8_t* codes, uint8_t* scales, lrq_stream_t stream);

/*
 * Activation fake-quant of the FP8 W8A8 rollout linear: per 1 x blk block of
 * each row (a token's hidden vector), s = clamp(amax/448, FLT_MIN), optional
 * pow2 (LRQ_FLAG_POW2_SCALE = FP8Config.use_activation_pow2_scale), and
 * out = float32(x / s) * s.  Replaces the activation ops of
 * _FP8W8A8Linear.forward (lumenrl/quantization/fp8_rollout.py:53-72).
 *   in  : [rows, cols] in_dtype, element-aligned, any row stride ld;
 *   out : [rows, cols] float32, dense, 16-byte aligned;  blk any width that
 *         divides cols (32, 64, 128, 256 and, for 16-bit input, 512 on the
 *         vector kernels, others on kernels of one wave per block).
 */
int lrq_act_qdq(const void* in, int in_dtype, int64_t rows, int64_t cols, int64_t ld, int64_t blk,
                unsigned flags, float* out, lrq_stream_t stream);

/*
 * Unscaled cast of n contiguous elements to float8_e4m3fn, as torch's
 * `tensor.to(torch.float8_e4m3fn)`: round to nearest even, |x| rounding past
 * 448, +-inf and NaN -> NaN (0x7F | sign).  Replaces the FP8 path of
 * DynamicWeightLoader (lumenrl/engine/inference/weight_loader.py:19-43,
 * `_maybe_fp8_quantize_tensor`); a whole state dict goes through one grouped
 * launch with LRQ_FMT_CAST_E4M3.  Any alignment; codes aligned to 8 bytes (4
 * for float32 input) take the vector path, whose 16-byte loads take any
 * element-aligned input.
 */
int lrq_cast_e4m3(const void* in, int in_dtype, int64_t n, uint8_t* out, lrq_stream_t stream);

/*
 * MX dequantization, the inverse of lrq_mxfp8_quant / lrq_mxfp4_quant:
 * out = element * 2^(E-127) per 1x32 group (OCP MX v1.0), evaluated as torch's
 * codes.float() * scales.view(float8_e8m0fnu).float() on x86 (E8M0 0xFF is
 * NaN and propagates; a NaN e4m3 code keeps its sign), then out_dtype
 * (LRQ_DTYPE_F32, or LRQ_DTYPE_BF16 rounded to nearest even).  No reference
 * function (the reference hands MX weights to absent vLLM/aiter loaders:
 * examples/Qwen3_8B_SDDD_MI350_vLLM/configs/opd_qwen3_8b.yaml:43); the
 * receiving side's view of what the quantizer sent.
 *   fmt   : LRQ_FMT_MXFP8 (codes [rows, cols]) or LRQ_FMT_MXFP4 (codes
 *           [rows, cols/2], element 2i in the low nibble);
 *   scales: [rows, cols/32] E8M0;  out: dense [rows, cols], 16-byte aligned;
 *   codes aligned to one lane-chunk of codes (MXFP8: 8 bytes for bf16 output,
 *   4 for fp32; MXFP4: 4 and 2).
 */
int lrq_mx_dequant(int fmt, const uint8_t* codes, const uint8_t* scales, int64_t rows,
                   int64_t cols, void* out, int out_dtype, lrq_stream_t stream);

/*
 * Grouped launch: many tensors (a layer, a whole weight set, or MoE expert
 * stacks) quantized by ONE kernel launch.  Replaces the per-tensor Python loop
 * of WeightQuantizer.quantize_state_dict (weight_quantizer.py:91-115) and the
 * per-expert loaders (lumenrl/engine/inference/vllm_moe_weight_sync.py:232-283).
 *
 * 1. lrq_group_table_bytes() sizes the host table for `n` tensors (a header
 *    and one 112-byte descriptor per tensor).
 * 2. lrq_group_pack() validates the tensors and writes the table into a HOST
 *    buffer.
 * 3. The caller allocates lrq_group_device_bytes(host_table) bytes of device
 *    memory (256-byte aligned), copies the host table verbatim to its start,
 *    and calls lrq_group_build_map() on the same stream, which writes the
 *    work-group -> tensor map behind it (4 bytes per work-group) on the device.
 *    Once per table: it stays valid while the tensors' storage does.
 * 4. lrq_quant_grouped() takes both copies: the host copy supplies the launch
 *    geometry, the device copy is what the kernel reads.
 * All tensors of a table share fmt, in_dtype, block shape and flags, and must
 * all qualify for the same kernel (the pack fails otherwise).
 * With fmt LRQ_FMT_FP8_DEQUANT the same tables drive the grouped inverse:
 * WeightQuantizer.dequantize_state_dict (weight_quantizer.py:117-134), one launch per table.
 */
typedef struct lrq_tensor {
  const void* in;       /* device input */
  void* codes;          /* device codes */
  void* scales;         /* device scales */
  int64_t batch;        /* matrices (MoE experts); >= 1 */
  int64_t rows, cols;   /* per matrix */
  int64_t ld;           /* input row stride (elements) */
  int64_t batch_stride; /* input matrix stride (elements) */
} lrq_tensor;

int64_t lrq_group_table_bytes(int fmt, const lrq_tensor* tensors, int64_t n, int in_dtype,
                              int64_t blk_r, int64_t blk_c, unsigned flags);
int lrq_group_pack(int fmt, const lrq_tensor* tensors, int64_t n, int in_dtype, int64_t blk_r,
                   int64_t blk_c, unsigned flags, void* host_table, int64_t capacity);
/* device table size: the host table plus 4 bytes per work-group */
int64_t lrq_group_device_bytes(const void* host_table);
/* writes the map of a device table whose first lrq_group_table_bytes() bytes
 * hold the uploaded host table (stream-ordered before this call) */
int lrq_group_build_map(const void* host_table, void* device_table, lrq_stream_t stream);
int lrq_quant_grouped(const void* host_table, const void* device_table, lrq_stream_t stream);
/* work-groups of a packed table's launch (for bandwidth accounting) */
int64_t lrq_group_units(const void* host_table);
/* kernel a packed table launches, as an opaque id >= 0: a list split into
 * several tables (consecutive tensors per launch) takes one kernel exactly when
 * every table reports the same id, as lrq_group_pack() requires of one table */
int lrq_group_kernel(const void* host_table);
/*
 * Per-tensor FP8 scales of the KV-cache quantizer, for a table packed with
 * fmt LRQ_FMT_TENSOR_SCALE (blk_r, blk_c and flags are ignored):
 *   scale = max(|w|.max(), FLT_MIN) / 448  per tensor (float32),
 * the clamp applied BEFORE the division as in
 * FP8KVCacheQuantizer.recalibrate_scales (lumenrl/quantization/fp8_kv_cache.py:52-54),
 * which this replaces for all q/k/v projections in two launches.  A tensor
 * holding a NaN gets 0x7FC00000 (torch's multi-threaded x86 reduction);
 * empty tensors are rejected (torch's max() raises for them).
 * `workspace` is device memory of at least lrq_group_workspace_bytes(table)
 * bytes (4 per work-group) that the launch overwrites; launches sharing one
 * workspace must be stream-ordered.  lrq_group_workspace_bytes() is 0 for
 * every other format.
 */
int64_t lrq_group_workspace_bytes(const void* host_table);
int lrq_tensor_scale_grouped(const void* host_table, const void* device_table, void* workspace,
                             int64_t workspace_bytes, lrq_stream_t stream);

/*
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): lrq_tensor_scale_grouped with the partial-maximum
 * workspace taken from a library-owned static device array of
 * LRQ_STATIC_WORKSPACE_BYTES per device instead of a caller buffer.  Same
 * tables, same results, and no allocation of any kind.
 *   - A table needing more than LRQ_STATIC_WORKSPACE_BYTES of workspace
 *     (lrq_group_workspace_bytes(), 4 bytes per 8 KiB of weights: 4 MiB
 *     covers at least 8 GiB of weights) is rejected with LRQ_ERR_CAPACITY
 *     before any device work.
 *   - Every call on one device shares that device's array.  Calls ordered on
 *     one stream are safe (every partial is written before it is read); calls
 *     that overlap on one device (different streams, or threads without
 *     ordering) race and may return wrong scales.
 *   - The array's address is looked up once per device, when
 *     lrq_group_build_map() sets up a tensor-scale table there (or on the
 *     first call on a device no such table was set up on).  A call captured
 *     into a HIP graph after that set-up makes no runtime call beyond
 *     hipStreamGetDevice and its two kernel launches.
 */
#define LRQ_STATIC_WORKSPACE_BYTES (4u << 20)
int lrq_tensor_scale_grouped_static(const void* host_table, const void* device_table,
                                    lrq_stream_t stream);

/* Library version string ("lrq <semver> gfx950"). */
const char* lrq_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char* lrq_last_error(void);

/*
 * Diagnostics (no reference counterpart): the device element encoders applied
 * to raw inputs, so tests can compare them with the CPU oracle exhaustively.
 *   lrq_diag_e4m3_bits: out[i] = e4m3(float with bit pattern start + i), via
 *     the hardware pack-convert the FP8 kernels use; n a multiple of 4.
 *   lrq_diag_bf16_bits: out[i] = bf16 (bit pattern) of the float with bit pattern
 *     start + i, via the hardware pack-convert the dequant kernel uses; n even.
 *   lrq_diag_mx_encode: the MXFP8 (fmt LRQ_FMT_MXFP8) or MXFP4 (LRQ_FMT_MXFP4)
 *     element path of the MX kernel: elements 2k and 2k+1 of `in` encoded
 *     under E8M0 byte e8m0[k]; out[i] = E4M3 byte or E2M1 nibble of in[i];
 *     n even.
 */
int lrq_diag_e4m3_bits(uint32_t start, int64_t n, uint8_t* out, lrq_stream_t stream);
int lrq_diag_bf16_bits(uint32_t start, int64_t n, uint16_t* out, lrq_stream_t stream);
int lrq_diag_mx_encode(int fmt, const float* in, const uint8_t* e8m0, uint8_t* out, int64_t n,
                       lrq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LRQ_H_ */
