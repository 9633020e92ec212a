// Packed embedding row gather: out[t, :] = dequant(row ids[t] of the packed table), rounded to
// the output dtype. Counterpart of the reference's IQ2_S embedding lookup
// (mlx_gsq/runtime/kernels/embedding.py:9-36), which runs its per-element IQ2_S decoder on the
// gathered row (iq_lookup_decode.py:18-22) and stores bfloat16 or half.
//
// One thread per 32-weight group of one output row: the group decodes exactly in float32 (the
// dequant kernel's decoder, so values are bit-identical to the CPU dequantizer) and becomes 32
// values of the output dtype with round-to-nearest-even. The gather reads
// dims / 256 superblocks per token and writes dims output values: HBM-bound, write-dominated.
// Ids outside [0, vocab) give rows of zeros.
#include "gsq_decode.h"

namespace gsq {

enum { EMB_F32 = 0, EMB_F16 = 1, EMB_BF16 = 2 };

// Output bytes of one 32-weight group are contiguous, and so are the groups of consecutive
// threads (element offset = 32 x thread index, across token rows), so a wave's 64 groups are
// one contiguous span of 64 x 32 values. Each lane stages its group's bytes in LDS and then
// stores 16-byte pieces of the span such that every store instruction of the wave writes 1 KB
// of consecutive memory (a lane's own group would put 64 lanes 64 or 128 bytes apart).
// Lane slots are padded by 16 bytes so that the 16-byte LDS writes of 16 lanes hit distinct
// banks.
template <int OB>  // output bytes per group: 64 (fp16 / bf16) or 128 (fp32)
struct EmbStage {
  static constexpr int kSlot = OB + 16;
  static constexpr int kWave = 64 * kSlot;
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// NT: streaming (nontemporal) stores, for outputs of many rows that no later work of the kernel
// reads (4096 ids: 15.5 -> 13.8 us); a few rows (a decode step's token) keep plain stores, whose
// lines stay in L2 for the kernel that reads them next. A compile-time choice: a runtime branch
// between the two stores is merged into one plain store by the compiler.
template <int T, int OB, bool NT>
__device__ __forceinline__ void embedding_body(const uint8_t* __restrict__ packed, const void* __restrict__ ids,
                                               int ids64, int64_t n_ids, int64_t vocab, int64_t dims,
                                               uint8_t* __restrict__ out, int odt, const DevTables& t,
                                               uint8_t* stage) {
  using S = EmbStage<OB>;
  const int lane = threadIdx.x & 63;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t gpr = dims >> 5;  // groups per row
  const int64_t total = n_ids * gpr;
  const bool live = gid < total;
  const int64_t tok = live ? gid / gpr : 0;
  const int64_t gr = gid - tok * gpr;
  const int64_t id = !live ? -1
                           : (ids64 ? static_cast<const int64_t*>(ids)[tok]
                                    : (int64_t) static_cast<const int32_t*>(ids)[tok]);
  float v[32];
  if (id >= 0 && id < vocab) {
    dq_group<T>(packed + (id * (dims >> 8) + (gr >> 3)) * BlockBytes<T>::v, (int)(gr & 7), t, v);
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = 0.f;
  }
  uint4* mine = reinterpret_cast<uint4*>(stage + lane * S::kSlot);
  if constexpr (OB == 128) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      mine[i] = make_uint4(__builtin_bit_cast(uint32_t, v[4 * i]), __builtin_bit_cast(uint32_t, v[4 * i + 1]),
                           __builtin_bit_cast(uint32_t, v[4 * i + 2]), __builtin_bit_cast(uint32_t, v[4 * i + 3]));
  } else {
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t lo, hi;
      if (odt == EMB_F16) {
        lo = __builtin_bit_cast(uint16_t, (_Float16)v[2 * i]);
        hi = __builtin_bit_cast(uint16_t, (_Float16)v[2 * i + 1]);
      } else {
        lo = f32_to_bf16_bits(v[2 * i]);
        hi = f32_to_bf16_bits(v[2 * i + 1]);
      }
      w[i] = lo | (hi << 16);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) mine[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  }
  __syncthreads();
  // store i of the wave: bytes [1024 i + 16 lane, +16) of its span, i.e. piece (lane % P) of the
  // group of lane 64 i / P... (P = OB / 16 pieces per group)
  constexpr int P = OB / 16;
  const int64_t wave0 = gid - lane;  // the wave's first group
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int src = (1024 / OB) * i + lane / P;  // lane whose group holds this piece
    if (wave0 + src < total) {
      const uint4 val = *reinterpret_cast<const uint4*>(stage + src * S::kSlot + 16 * (lane % P));
      uint4* dst = reinterpret_cast<uint4*>(out + (wave0 + src) * OB + 16 * (lane % P));
      if constexpr (NT) __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, val), reinterpret_cast<u32x4_t*>(dst));
      else *dst = val;
    }
  }
}

constexpr int64_t kEmbStreamRows = 64;  // rows from which the output is stored nontemporally

template <int T, bool NT>
__global__ void __launch_bounds__(256) embedding_kernel(const uint8_t* __restrict__ packed, const void* __restrict__ ids,
                                                        int ids64, int64_t n_ids, int64_t vocab, int64_t dims,
                                                        void* __restrict__ out, int odt, DevTables t) {
  __shared__ __attribute__((aligned(16))) uint8_t stage[4 * EmbStage<128>::kWave];
  uint8_t* ws = stage + (threadIdx.x >> 6) * (odt == EMB_F32 ? EmbStage<128>::kWave : EmbStage<64>::kWave);
  if (odt == EMB_F32)
    embedding_body<T, 128, NT>(packed, ids, ids64, n_ids, vocab, dims, static_cast<uint8_t*>(out), odt, t, ws);
  else
    embedding_body<T, 64, NT>(packed, ids, ids64, n_ids, vocab, dims, static_cast<uint8_t*>(out), odt, t, ws);
}

template <int T>
static hipError_t launch_embedding_t(const uint8_t* packed, const void* ids, int ids64, int64_t n_ids, int64_t vocab,
                                     int64_t dims, void* out, int odt, const DevTables& t, hipStream_t s) {
  const int64_t threads = n_ids * (dims >> 5);
  const int64_t grid = (threads + 255) / 256;
  if (n_ids >= kEmbStreamRows)
    hipLaunchKernelGGL((embedding_kernel<T, true>), dim3((unsigned)grid), dim3(256), 0, s, packed, ids, ids64, n_ids,
                       vocab, dims, out, odt, t);
  else
    hipLaunchKernelGGL((embedding_kernel<T, false>), dim3((unsigned)grid), dim3(256), 0, s, packed, ids, ids64, n_ids,
                       vocab, dims, out, odt, t);
  return hipGetLastError();
}

hipError_t launch_embedding(int qt, const uint8_t* packed, const void* ids, int ids64, int64_t n_ids, int64_t vocab,
                            int64_t dims, void* out, int odt, const DevTables& t, hipStream_t s) {
  switch (qt) {
    case Q2_K: return launch_embedding_t<Q2_K>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    case Q4_K: return launch_embedding_t<Q4_K>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    case Q6_K: return launch_embedding_t<Q6_K>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    case IQ4_XS: return launch_embedding_t<IQ4_XS>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    case IQ3_S: return launch_embedding_t<IQ3_S>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    case IQ3_XXS: return launch_embedding_t<IQ3_XXS>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    case IQ2_XXS: return launch_embedding_t<IQ2_XXS>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    case IQ2_XS: return launch_embedding_t<IQ2_XS>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    case IQ2_S: return launch_embedding_t<IQ2_S>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    case IQ1_S: return launch_embedding_t<IQ1_S>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    case IQ1_M: return launch_embedding_t<IQ1_M>(packed, ids, ids64, n_ids, vocab, dims, out, odt, t, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gsq
