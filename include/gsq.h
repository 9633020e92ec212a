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
 * of entries x coords float32 values; every value must be exact in fp16. `ksigns` must be
 * the published table (entry i = i with bit 7 set to the parity of i), else GSQ_E_VALUE.
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

/* y[M, N] = x[M, K] * W[N, K]^T with the fused-dequant matrix-vector kernels (decode path,
 * small M): 1-2 rows (and fp32 / bf16 x) on the vector kernel, 3-8 fp16 rows (2 on matrices of
 * 2^26+ weights with K <= 8192) on the quad-row kernel (matrix-core products of four weight rows
 * at a time), more rows in launches of 8.
 * Replaces quantized_matvec (mlx_gsq/runtime/kernels/qmv.py:537-576). x at any address aligned
 * to its element size: one that is not 16-byte aligned is first copied into the stream's QMM
 * workspace (see gsq_qmm; made on that first call). */
int gsq_qmv(int qtype_id, const void* packed, const void* x, int x_dtype, void* y, int y_dtype,
            int64_t M, int64_t N, int64_t K, void* stream);

/* y0[1, N0] = x * W0^T and y1[1, N1] = x * W1^T for one fp16 activation row x[K] and two packed
 * matrices of any two types (q|k and v of an attention layer) in one launch, the CUs shared in
 * proportion to the two products' expected times (bytes x a per-type measured time per byte).
 * No counterpart in the reference, whose model applies each projection on its own
 * (mlx_gsq/models/qwen35.py); for GSQGroupedLinear. Results as two gsq_qmv calls give them,
 * within the QMV tolerance (a product alone may run another launch plan). Products the shared
 * kernel does not take (plans that do not decode items in pairs: Q6_K, IQ3_S at K = 5120, rows
 * of other than 20 superblocks; matrices or rows not 4-byte aligned; x not 16-byte aligned) run
 * as those two calls. y0, y1 and x must not overlap (GSQ_E_VALUE). */
int gsq_qmv_group2(int qtype_id0, const void* packed0, int64_t N0, void* y0, int qtype_id1, const void* packed1,
                   int64_t N1, void* y1, const void* x, int y_dtype, int64_t K, void* stream);

/* One fp16 activation row that the QMV kernel forms itself before the product (a decode
 * step's norm or MLP activation fused into the projection that consumes it; no counterpart in
 * the reference, whose model runs them as separate mlx operations in
 * mlx_gsq/models/qwen35.py). y[1, N] = row * W[N, K]^T with
 *   GSQ_PRE_ADD_RMSNORM: s = round(x + pre_a) (pre_a may be NULL: s = x), written to res_out
 *     when not NULL; row = round(s / sqrt(mean(s^2) + eps)
 *     * pre_w), as gsq_add_rms_norm computes it;
 *   GSQ_PRE_SWIGLU: x holds [gate | up] (2K values); row = round(silu(gate) * up), as
 *     gsq_swiglu computes it (pre_a, pre_w, eps, res_out unused).
 * The row is written to x_out when not NULL. The first workgroup writes res_out and x_out while
 * the others still read x, pre_a and pre_w, so an output that overlaps any of them (or the other
 * output) is refused with GSQ_E_VALUE. All vectors fp16, 16-byte aligned; K a multiple
 * of 8 up to 32768. With conv_rows > 0 (fp16 y), output rows r < conv_rows also run a
 * depthwise causal convolution (the GatedDeltaNet's, of the qkv rows of its input projection):
 * state conv_state [conv_kernel - 1, conv_rows] fp16 shifted in place with the new input
 * round(y[r]), weights conv_w [conv_rows, conv_kernel] fp16, conv_out[r] = silu(sum) in float32,
 * as gsq_gdn_step's convolution computes it (pass its conv_state as NULL afterwards). */
#define GSQ_PRE_ADD_RMSNORM 1
#define GSQ_PRE_SWIGLU 2
int gsq_qmv_pre(int qtype_id, const void* packed, int pre_op, const void* x, const void* pre_a, const void* pre_w,
                float eps, void* res_out, void* x_out, void* y, int y_dtype, int64_t N, int64_t K, void* conv_state,
                const void* conv_w, int64_t conv_rows, int64_t conv_kernel, float* conv_out, void* stream);

/* Same product with the tiled MFMA kernel (prefill, large M). Replaces quantized_matmul
 * (mlx_gsq/runtime/kernels/qmm.py:559-594). Workgroups that share an output tile exchange
 * fp32 partials through a workspace the library keeps per (device, stream) and allocates on
 * the first call on that stream (or in gsq_prepare): calls on one stream run in order and
 * share it, calls on different streams may overlap and never share one. A workspace is 2 slots
 * of 256 x 256 floats per CU plus counters (128 MB on a 256-CU device), held until the process
 * ends, for at most 64 streams per device; the call that makes it synchronizes the device once.
 * A graph captured from stream S uses S's workspace: its replays must not overlap other QMM
 * work on S or replays of other graphs captured from S. */
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

/* ---- the decode step around the projections (Qwen3.5-hybrid) ----
 * Element-wise work of one decoder step fused into single launches. The reference runs it as
 * mlx / mlx-lm operations inside mlx_gsq/models/qwen35.py (RMSNorm, SwiGLU MLP, the patched
 * GatedDeltaNet :48-111); no entry point of its own corresponds. Tensors are row-major in one
 * dtype (GSQ_F32 / GSQ_F16 / GSQ_BF16), math in float32, results rounded once. */

/* Per row of `dim` values (a multiple of 8, at most 8192; all pointers 16-byte aligned): if
 * delta is not NULL, x = round(x + delta) (written back); then y = round(x / sqrt(mean(x^2) +
 * eps) * w). Replaces the residual add and RMSNorm of a layer. */
int gsq_add_rms_norm(void* x, const void* delta, const void* w, void* y, int64_t rows, int64_t dim, float eps,
                     int dtype, void* stream);

/* out[r, i] = round(silu(gu[r, i]) * gu[r, n + i]) for rows of 2n values (gate then up).
 * Replaces the SwiGLU of the MLP. */
int gsq_swiglu(const void* gate_up, void* out, int64_t rows, int64_t n, int dtype, void* stream);

/* One GatedDeltaNet token for `batch` rows (replaces the conv / gated_delta_update / gated
 * norm part of qwen35.py:58-108 for one token, and the in_proj_a / in_proj_b projections):
 * per row, the depthwise causal convolution (kernel conv_kernel, state conv_state [batch,
 * conv_kernel-1, conv_dim] shifted in place, weights conv_w [conv_dim, conv_kernel]) and SiLU
 * of the new qkv row (conv_dim = 2 * key_heads * head_k_dim + value_heads * head_v_dim), into
 * `work` (batch x conv_dim float32, scratch); q and k RMS-normalized per head (eps 1e-6) times
 * head_k_dim^-1 and ^-1/2; value head h reads q/k head h % key_heads (GGUF order); a and b =
 * x . w_ab rows h and value_heads + h (w_ab [2 value_heads, hidden]), rounded to the dtype;
 * beta = sigmoid(b), decay = exp(ssm_a * softplus(a + dt_bias)); the float32 state rec_state
 * [batch, value_heads, head_k_dim, head_v_dim] updated in place (S = decay S; S += k (beta (v -
 * S^T k))^T) and o = S^T q; out = round(o / rms(o) * norm_w * silu(z)) with eps over each
 * head's head_v_dim values. Strides are in elements between batch rows. head_k_dim a multiple
 * of 4 up to 128, head_v_dim 64..256 in steps of 64, conv_kernel 2..8. conv_state NULL: the
 * convolution has run already (gsq_qmv_pre's epilogue) and `work` holds its outputs; qkv and
 * conv_w are then not read. */
int gsq_gdn_step(const void* qkv, int64_t qkv_stride, const void* z, int64_t z_stride, const void* x,
                 int64_t x_stride, const void* w_ab, int64_t hidden, void* conv_state, const void* conv_w,
                 const float* ssm_a, const float* dt_bias, float* rec_state, const void* norm_w, void* out,
                 int64_t out_stride, float* work, int64_t batch, int64_t key_heads, int64_t value_heads,
                 int64_t head_k_dim, int64_t head_v_dim, int64_t conv_kernel, float eps, int dtype, void* stream);

/* gsq_gdn_step over a sequence (prefill): `seq` tokens of each of `batch` rows, rows b * seq + t
 * of qkv, z, ab and out (row strides in elements); ab holds the a and b projections of each
 * token (2 * value_heads values: a then b, rounded to the dtype, e.g. one GEMM of the layer input
 * with w_ab). Same arithmetic per token as gsq_gdn_step; the recurrent state stays in registers
 * from the first token to the last and the convolution state ends at the sequence's last
 * conv_kernel - 1 inputs. work: batch * seq * conv_dim floats. */
int gsq_gdn_seq(const void* qkv, int64_t qkv_stride, const void* z, int64_t z_stride, const void* ab,
                int64_t ab_stride, void* conv_state, const void* conv_w, const float* ssm_a, const float* dt_bias,
                float* rec_state, const void* norm_w, void* out, int64_t out_stride, float* work, int64_t batch,
                int64_t seq, int64_t key_heads, int64_t value_heads, int64_t head_k_dim, int64_t head_v_dim,
                int64_t conv_kernel, float eps, int dtype, void* stream);

/* One new token of gated grouped-query attention for `batch` rows (replaces the attention of a
 * full-attention layer at decode, qwen35.py's mlx-lm attention): per query head h (kv head
 * h / (heads / kv_heads)), q = round(rms_norm(q) * q_norm_w) from the q half of qg's head
 * block [q | gate] and k likewise from k with k_norm_w (eps), both rotated on their first
 * rotary_dim dims (rotate-half, angle pos * inv_freq[i]) and rounded; k and v written at *pos
 * into k_cache / v_cache [batch, kv_heads, max_len, head_dim]; softmax over positions 0..*pos of
 * q . K / sqrt(head_dim); out = round(sum p V * sigmoid(gate)). *pos is read on the device;
 * when it is outside 0..max_len-1 (a graph replayed past the cache's end) the kernels write NaN
 * to out and nothing to the caches. head_dim a multiple of 4 up to 256. Strides in elements. With work NULL one
 * workgroup per (row, head) covers every position (max_len at most 32768); otherwise the
 * positions are split into ceil(max_len / chunk) chunks (chunk a multiple of 64 up to 1024,
 * max_len up to 2^20), one workgroup each, whose partial softmax sums meet in work (batch *
 * heads * ceil(max_len / chunk) * (head_dim + 2) floats) and are combined by a second kernel:
 * for long contexts. */
int gsq_attn_decode(const void* qg, int64_t qg_stride, const void* k, int64_t k_stride, const void* v,
                    int64_t v_stride, const void* q_norm_w, const void* k_norm_w, const double* inv_freq,
                    void* k_cache, void* v_cache, const int64_t* pos, void* out, int64_t out_stride, int64_t batch,
                    int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t rotary_dim, int64_t max_len,
                    float eps, float* work, int64_t chunk, int dtype, void* stream);

/* Message of the last failed call on this thread ("" if none). */
const char* gsq_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* GSQ_H */
