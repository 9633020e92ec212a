/* C ABI of the MI355X quantized-linear library (libgsq.so).
 *
 * Plain pointers and sizes only; no framework types cross this boundary. All device
 * pointers belong to the caller and must live on the device that is current when the
 * call is made. Work is enqueued on `stream` (a hipStream_t; NULL = default stream) and
 * nothing synchronizes with the host. Functions return 0 on success and a nonzero
 * GSQ_E_* code otherwise; gsq_last_error() then describes the failure (per thread).
 *
 * Quant type ids are GGML's (mlx_gsq/gguf/parser.py:26-31): Q2_K 10, Q4_K 12, Q6_K 14,
 * IQ2_XXS 16, IQ2_XS 17, IQ3_XXS 18, IQ1_S 19, IQ3_S 21, IQ2_S 22, IQ4_XS 23, IQ1_M 29.
 * Packed weights are the untouched GGUF superblocks of an N x K matrix, row-major:
 * N * (K/256) blocks of gsq_block_bytes(type) bytes (qmv.py:539-543).
 * Activation/output dtype codes: GSQ_F32 0, GSQ_F16 1, GSQ_BF16 2.
 */
#ifndef GSQ_H
#define GSQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GSQ_OK 0
#define GSQ_E_VALUE 1       /* bad shape/size/alignment (the reference raises ValueError) */
#define GSQ_E_UNSUPPORTED 2 /* unknown quant type (NotImplementedError) */
#define GSQ_E_TABLES 3      /* codebook of a grid type not set on this device */
#define GSQ_E_HIP 4         /* HIP runtime error */
#define GSQ_E_TYPE 5        /* bad dtype code (TypeError) */

#define GSQ_F32 0
#define GSQ_F16 1
#define GSQ_BF16 2
#define GSQ_IDS_I32 0       /* embedding id dtype codes */
#define GSQ_IDS_I64 1

/* Library ABI version. */
int gsq_version(void);

/* Bytes per 256-weight superblock, or -1 for an unsupported type.
 * Replaces QUANT_BLOCK_SIZES lookups (mlx_gsq/gguf/parser.py:35-42). */
int gsq_block_bytes(int qtype_id);

/* Upload a codebook for a grid type (IQ1_S, IQ1_M, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS,
 * IQ3_S) and the 128-entry ksigns table to the current device. `grid` is a host array
 * of entries x coords float32 values; every value must be exact in fp16.
 * Replaces the table buffers the reference hands its kernels
 * (iq_lookup_decode.py:46-53 `_tables`, iq3_s_decode.py:56-61 `_grid`). */
int gsq_set_tables(int qtype_id, const float* grid, int64_t entries, int64_t coords,
                   const uint8_t* ksigns, int64_t n_ksigns);

/* Prepare the current device and `stream` (a hipStream_t; NULL = default stream) for calls
 * that must neither allocate nor copy synchronously, such as calls under HIP graph capture:
 * builds the fixed tables of the non-grid types and the QMM workspace of `stream`. Without
 * it the first call on a device or stream does that work itself, which fails with
 * GSQ_E_VALUE while the stream is capturing. Codebooks still come from gsq_set_tables. No
 * counterpart in the reference (MLX compiles and caches its kernels lazily, qmv.py:66). */
int gsq_prepare(void* stream);

/* 1 if the current device holds the tables `qtype_id` needs, else 0. */
int gsq_tables_ready(int qtype_id);

/* Dequantize `nblocks` superblocks to float32 (nblocks * 256 values, 16-byte aligned).
 * Bit-exact with the CPU dequantizer. Replaces registry.decode
 * (mlx_gsq/runtime/kernels/registry.py:28-32) and the decode kernels behind it. */
int gsq_dequant(int qtype_id, const void* packed, int64_t nblocks, float* out, void* stream);

/* y[M, N] = x[M, K] * W[N, K]^T with the fused-dequant matrix-vector kernel (decode path,
 * small M). Replaces quantized_matvec (mlx_gsq/runtime/kernels/qmv.py:537-576). */
int gsq_qmv(int qtype_id, const void* packed, const void* x, int x_dtype, void* y, int y_dtype,
            int64_t M, int64_t N, int64_t K, void* stream);

/* Same product with the tiled MFMA kernel (prefill, large M). Replaces quantized_matmul
 * (mlx_gsq/runtime/kernels/qmm.py:559-594). Workgroups that share an output tile exchange
 * fp32 partials through a workspace the library keeps per (device, stream) and allocates on
 * the first call on that stream (or in gsq_prepare): calls on one stream run in order and
 * share it, calls on different streams may overlap and never share one. */
int gsq_qmm(int qtype_id, const void* packed, const void* x, int x_dtype, void* y, int y_dtype,
            int64_t M, int64_t N, int64_t K, void* stream);

/* gsq_qmm without any allocation, for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. Split-tile partials and arrival counters live in a fixed device array of
 * 32 MiB + 4 KiB that each device holds until the process ends (tile heights are lowered until
 * the partials of one workgroup per CU fit; a device with more than 256 CUs is refused with
 * GSQ_E_VALUE). Every call on a device shares that array, so calls that overlap on one device
 * (several streams, concurrent graph nodes) race and give wrong results: serialize them. Fixed
 * tables must exist first (gsq_prepare, gsq_set_tables); a call that would need to build one
 * returns GSQ_E_VALUE instead. Results match gsq_qmm within the QMM tolerance (bit for bit
 * where both pick the same tile plan, as for M <= 64). */
int gsq_qmm_noalloc(int qtype_id, const void* packed, const void* x, int x_dtype, void* y, int y_dtype,
                    int64_t M, int64_t N, int64_t K, void* stream);

/* Packed embedding gather: out[t, :] = dequantized row ids[t] of a (vocab, dims) packed table,
 * rounded to out_dtype (GSQ_F32 / GSQ_F16 / GSQ_BF16, round-to-nearest-even from the exact
 * float32 value); ids are int32 (GSQ_IDS_I32) or int64 (GSQ_IDS_I64), n_ids of them; dims a
 * multiple of 256; out 16-byte aligned, n_ids * dims values. Ids outside [0, vocab) give rows
 * of zeros. Replaces iq2_s_embedding (mlx_gsq/runtime/kernels/embedding.py:30-36), which is
 * IQ2_S only; this entry point takes any of the 11 types. */
int gsq_embedding(int qtype_id, const void* packed, const void* ids, int ids_dtype, int64_t n_ids,
                  int64_t vocab, int64_t dims, void* out, int out_dtype, void* stream);

/* Message of the last failed call on this thread ("" if none). */
const char* gsq_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* GSQ_H */
