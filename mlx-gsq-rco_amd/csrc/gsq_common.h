// Common definitions for the gfx950 quantized-linear kernels.
//
// Superblock layouts and decode formulas follow the reference decoders
// (mlx_gsq/runtime/kernels/k_decode.py:18-80, iq_lookup_decode.py:6-39,
// iq3_s_decode.py:16-40). Every supported format packs 256 weights per superblock.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gsq {

enum QType : int {
  Q2_K = 10, Q4_K = 12, Q6_K = 14, IQ2_XXS = 16, IQ2_XS = 17, IQ3_XXS = 18,
  IQ1_S = 19, IQ3_S = 21, IQ2_S = 22, IQ4_XS = 23, IQ1_M = 29,
};

template <int T> struct BlockBytes;
template <> struct BlockBytes<Q2_K> { static constexpr int v = 84; };
template <> struct BlockBytes<Q4_K> { static constexpr int v = 144; };
template <> struct BlockBytes<Q6_K> { static constexpr int v = 210; };
template <> struct BlockBytes<IQ2_XXS> { static constexpr int v = 66; };
template <> struct BlockBytes<IQ2_XS> { static constexpr int v = 74; };
template <> struct BlockBytes<IQ3_XXS> { static constexpr int v = 98; };
template <> struct BlockBytes<IQ1_S> { static constexpr int v = 50; };
template <> struct BlockBytes<IQ3_S> { static constexpr int v = 110; };
template <> struct BlockBytes<IQ2_S> { static constexpr int v = 82; };
template <> struct BlockBytes<IQ4_XS> { static constexpr int v = 136; };
template <> struct BlockBytes<IQ1_M> { static constexpr int v = 56; };

inline int block_bytes_of(int t) {
  switch (t) {
    case Q2_K: return 84; case Q4_K: return 144; case Q6_K: return 210;
    case IQ2_XXS: return 66; case IQ2_XS: return 74; case IQ3_XXS: return 98;
    case IQ1_S: return 50; case IQ3_S: return 110; case IQ2_S: return 82;
    case IQ4_XS: return 136; case IQ1_M: return 56;
    default: return 0;
  }
}

// Codebook geometry of the grid types (entries, coordinates); 0 for the others.
inline void grid_shape_of(int t, int* entries, int* coords) {
  *entries = 0; *coords = 0;
  switch (t) {
    case IQ1_S: case IQ1_M: *entries = 2048; *coords = 8; break;
    case IQ2_XXS: *entries = 256; *coords = 8; break;
    case IQ2_XS: *entries = 512; *coords = 8; break;
    case IQ2_S: *entries = 1024; *coords = 8; break;
    case IQ3_XXS: *entries = 256; *coords = 4; break;
    case IQ3_S: *entries = 512; *coords = 4; break;
    default: break;
  }
}

// Device-resident tables for one type, built by gsq_set_tables.
struct DevTables {
  const uint16_t* grid16;   // fp16 codebook, entries x coords (grid types)
  const uint8_t* ksigns;    // [128]
  const uint8_t* qmv_tbl;   // the QMV kernel's LDS table image of this type (see gsq_qmv.hip)
  const uint8_t* qmm_tbl;   // the QMM kernels' LDS table image of this type
};

// Launch-plan parameters of the QMV kernel: waves per workgroup, target in-flight weight
// bytes per CU, workgroups per CU, the most rows for which a single fp16 activation row of
// at most 3 slices goes one slice per wave, the waves per workgroup of that plan, and the
// most ring items a wave issues per main-loop step, whether the activations may be staged in
// LDS (else every wave reads its slices from global memory), and whether 2.5-slice rows may be
// decoded two items at a time.
// Fused activation prologue of a one-row fp16 QMV (gsq_qmv_pre): the kernel forms its input
// row itself before the product.
//   QMV_PRE_ADD_NORM: row = x (+ a), rounded to fp16, written to res (when given); input =
//     round(row / rms(row) * w), written to out (when given). eps: the norm's epsilon.
//   QMV_PRE_SWIGLU: x = [gate | up] (2K values); input = round(silu(gate) * up), written to out
//     (when given).
enum { QMV_PRE_NONE = 0, QMV_PRE_ADD_NORM = 1, QMV_PRE_SWIGLU = 2 };
struct QmvPre {
  int op = QMV_PRE_NONE;
  const void* a = nullptr;
  const void* w = nullptr;
  void* res = nullptr;
  void* out = nullptr;
  float eps = 0.f;
  // convolution epilogue (conv_rows > 0): output rows r < conv_rows are the channels of a
  // depthwise causal convolution of kernel conv_k with state conv_state [conv_k - 1, conv_rows]
  // (fp16, shifted in place) and weights conv_w [conv_rows, conv_k] (fp16); conv_out[r] =
  // silu(convolution) in fp32. The row's fp16 output is the convolution's new input.
  void* conv_state = nullptr;
  const void* conv_w = nullptr;
  float* conv_out = nullptr;
  int conv_rows = 0, conv_k = 0;
};

struct QmvTuning {
  int waves;
  int inflight_bytes;
  int wg_per_cu;
  int gl1_rows;
  int gl1_waves;
  int fill;
  int x_lds;
  int pair;
};

// Launch-plan overrides of the QMM kernels: activation tile height in 16-row blocks (0 = by
// M), the fewest K columns (256 wide) per workgroup (0 = default) and waves per workgroup for
// tiles of 128 or 256 rows (4, or 0 = 8); the small-batch kernel's largest M (0 = 16, -1 =
// never used), waves (4, 8 or 16; 0 = 16 on products of at least 2^26 weights, else 8), 16-row
// blocks per wave (2 or 4 with 4 or 8 waves; 0 = 1) and fewest columns per workgroup (0 = 1).
struct QmmTuning {
  int mf;
  int min_cols;
  int waves;
  int small_max_m;
  int small_waves;
  int small_nb;
  int small_min_cols;
  int order;  // tiled kernel's tile order: 2 = activation tile fastest, else weight tile fastest
};

// Arguments of one GatedDeltaNet token step (gsq_gdn_step; kernels in gsq_model.hip).
struct GdnArgs {
  const void* qkv;  // [B] rows of conv_dim (row stride qkv_stride elements)
  const void* z;    // [B] rows of Hv*dv (row stride z_stride)
  const void* x;    // [B] rows of the layer input, hidden values (row stride x_stride)
  const void* w_ab; // [2 Hv, hidden]: the a rows, then the b rows
  void* conv;       // [B, K-1, conv_dim] convolution state (activation dtype)
  const void* conv_w;  // [conv_dim, K]
  const float* ssm_a;  // [Hv] = -exp(A_log)
  const float* dt_bias;  // [Hv]
  float* rec;          // [B, Hv, dk, dv] recurrent state
  const void* norm_w;  // [dv]
  void* out;           // [B] rows of Hv*dv (row stride out_stride)
  float* work;         // [B, conv_dim] convolution outputs (after SiLU); [B * S, conv_dim] for a sequence
  int64_t qkv_stride, z_stride, x_stride, out_stride;
  int B, Hk, Hv, dk, dv, K, hidden;
  // a sequence of S tokens per batch row (the prefill kernels): rows b * S + t of qkv, z, out
  // and of ab, the a and b projections (2 Hv values per row, activation dtype, row stride
  // ab_stride), computed beforehand
  int S = 1;
  const void* ab = nullptr;
  int64_t ab_stride = 0;
  float eps;
};

// Arguments of one single-token gated attention (gsq_attn_decode; kernel in gsq_model.hip).
struct AttnArgs {
  const void* qg;   // [B] rows of H * 2hd: per head q then gate (row stride qg_stride)
  const void* k;    // [B] rows of Hkv * hd (row stride k_stride)
  const void* v;    // [B] rows of Hkv * hd (row stride v_stride)
  const void* q_norm_w;  // [hd]
  const void* k_norm_w;  // [hd]
  const double* inv_freq;  // [rd / 2]
  void* kc;         // [B, Hkv, L, hd]
  void* vc;         // [B, Hkv, L, hd]
  const int64_t* pos;  // position of the new token (device)
  void* out;        // [B] rows of H * hd (row stride out_stride)
  int64_t qg_stride, k_stride, v_stride, out_stride;
  int B, H, Hkv, hd, rd, L;
  float eps;
  // positions split into chunks of `chunk` (nsplit = ceil(L / chunk)) when work is not null:
  // per (row, head, chunk) the partial softmax max, sum and hd weighted V sums, then combined
  float* work = nullptr;
  int chunk = 0, nsplit = 0;
};

// QMM workspace: fp32 partial tiles of workgroups that share an output tile (2 slots per
// workgroup, each sized to the launch plan's tile) and one arrival counter per workgroup, kept
// at zero between launches. `part_bytes` bounds 2 * groups * slot bytes; `max_groups` bounds the
// workgroups (counters). One workspace is never used by two launches that may overlap.
struct QmmWorkspace {
  float* part;
  int* cnt;
  int max_groups;
  long long part_bytes;
};

// Non-linear IQ4_XS values (k_decode.py:77).
__device__ __constant__ static const int8_t kIQ4Values[16] = {
    -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// float32 -> bfloat16 bits, round to nearest even; a NaN stays a (quiet) NaN of the same sign
// (adding the rounding bias to a NaN whose high mantissa bits are all ones would carry into
// the sign and give -0 or +0).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float v) {
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (b >> 16) | 0x0040u;
  b += 0x7FFFu + ((b >> 16) & 1u);
  return b >> 16;
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// ---- byte access helpers -----------------------------------------------------------
// Global memory: byte loads (the dequant instrument does not need wide loads).
__device__ __forceinline__ uint32_t gb(const uint8_t* p, int i) { return p[i]; }
__device__ __forceinline__ uint32_t gu16(const uint8_t* p, int i) { return (uint32_t)p[i] | ((uint32_t)p[i + 1] << 8); }
__device__ __forceinline__ uint32_t gu32(const uint8_t* p, int i) {
  return (uint32_t)p[i] | ((uint32_t)p[i + 1] << 8) | ((uint32_t)p[i + 2] << 16) | ((uint32_t)p[i + 3] << 24);
}

// LDS: N consecutive 32-bit words starting at an even byte offset (superblocks are only
// 2-byte aligned). A4 = the offset is known to be a multiple of 4: plain dword loads.
// Otherwise N+1 aligned dwords are read and funnel-shifted into place: gfx950 LDS does serve
// ds_read_b32/b64/b128 at 2-byte aligned addresses, but such reads stall the LDS pipeline
// (SQ_LDS_UNALIGNED_STALL), which costs more than one v_alignbyte per word.
template <int N, bool A4 = false>
__device__ __forceinline__ void lds_words(const uint8_t* base, uint32_t off, uint32_t (&w)[N]) {
  if constexpr (A4) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(base + off);
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = p[i];
  } else {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(base + (off & ~3u));
    const uint32_t sh = off & 3u;
    uint32_t a[N + 1];
#pragma unroll
    for (int i = 0; i <= N; ++i) a[i] = p[i];
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = __builtin_amdgcn_alignbyte(a[i + 1], a[i], sh);
  }
}
template <bool A4 = false>
__device__ __forceinline__ uint32_t lds_w32(const uint8_t* base, uint32_t off) {
  uint32_t w[1];
  lds_words<1, A4>(base, off, w);
  return w[0];
}
__device__ __forceinline__ uint32_t lds_u16(const uint8_t* base, uint32_t off) {
  return *reinterpret_cast<const uint16_t*>(base + off);
}
__device__ __forceinline__ uint32_t lds_u8(const uint8_t* base, uint32_t off) { return base[off]; }

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t width) {
  return __builtin_amdgcn_ubfe(v, off, width);
}

// ---- LDS DMA -------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Cooperative DMA of a 16-byte aligned buffer of `bytes` (a multiple of 16) by all waves of
// the workgroup; returns the instructions this wave issued.
__device__ __forceinline__ int dma_copy(const void* src, int bytes, uint8_t* dst, int wave, int nw, int lane) {
  const int ngran = bytes >> 4, per_wave = 64;
  int issued = 0;
  for (int c0 = wave * per_wave; c0 < ngran; c0 += nw * per_wave) {
    const int c = c0 + lane;
    if (c < ngran)
      __builtin_amdgcn_global_load_lds(static_cast<const uint8_t*>(src) + (size_t)c * 16,
                                       (lds_ptr_t)(dst + c0 * 16), 16, 0, 0);
    ++issued;
  }
  return issued;
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt bits 3:0 and
// 15:14); n above 63 waits for vmcnt(63), and a smaller immediate only waits longer.
__device__ __forceinline__ void wait_vmcnt(int n) {
#define GSQ_VMW(k) case k: __builtin_amdgcn_s_waitcnt(0x0F70 | ((k) & 15) | (((k) >> 4) << 14)); break;
#define GSQ_VMW8(k) GSQ_VMW(k) GSQ_VMW(k + 1) GSQ_VMW(k + 2) GSQ_VMW(k + 3) GSQ_VMW(k + 4) GSQ_VMW(k + 5) \
  GSQ_VMW(k + 6) GSQ_VMW(k + 7)
  switch (n < 0 ? 0 : n) {
    GSQ_VMW8(0) GSQ_VMW8(8) GSQ_VMW8(16) GSQ_VMW8(24) GSQ_VMW8(32) GSQ_VMW8(40) GSQ_VMW8(48) GSQ_VMW8(56)
    default: __builtin_amdgcn_s_waitcnt(0x0F70 | 15 | (3 << 14)); break;
  }
#undef GSQ_VMW8
#undef GSQ_VMW
}

}  // namespace gsq
