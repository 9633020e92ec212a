// Packed embedding row gather: out[t, :] = dequant(row ids[t] of the packed table), rounded to
// the output dtype. Counterpart of the reference's IQ2_S embedding lookup
// (mlx_gsq/runtime/kernels/embedding.py:9-36), which runs its per-element IQ2_S decoder on the
// gathered row (iq_lookup_decode.py:18-22) and stores bfloat16 or half.
//
// One thread per 32-weight group of one output row: the group decodes exactly in float32 (the
// dequant kernel's decoder, so values are bit-identical to the CPU dequantizer) and is stored
// as 32 values of the output dtype with round-to-nearest-even. The gather reads
// dims / 256 superblocks per token and writes dims output values: HBM-bound, write-dominated.
// Ids outside [0, vocab) give rows of zeros.
#include "gsq_decode.h"

namespace gsq {

enum { EMB_F32 = 0, EMB_F16 = 1, EMB_BF16 = 2 };

template <int T>
__global__ void __launch_bounds__(256) embedding_kernel(const uint8_t* __restrict__ packed, const void* __restrict__ ids,
                                                        int ids64, int64_t n_ids, int64_t vocab, int64_t dims,
                                                        void* __restrict__ out, int odt, DevTables t) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t gpr = dims >> 5;  // groups per row
  const int64_t tok = gid / gpr;
  if (tok >= n_ids) return;
  const int64_t gr = gid - tok * gpr;
  const int64_t id = ids64 ? static_cast<const int64_t*>(ids)[tok] : (int64_t) static_cast<const int32_t*>(ids)[tok];
  float v[32];
  if (id >= 0 && id < vocab) {
    dq_group<T>(packed + (id * (dims >> 8) + (gr >> 3)) * BlockBytes<T>::v, (int)(gr & 7), t, v);
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = 0.f;
  }
  const int64_t o = tok * dims + gr * 32;
  if (odt == EMB_F32) {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(out) + o);
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
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
    uint4* p = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + o);
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  }
}

template <int T>
static hipError_t launch_embedding_t(const uint8_t* packed, const void* ids, int ids64, int64_t n_ids, int64_t vocab,
                                     int64_t dims, void* out, int odt, const DevTables& t, hipStream_t s) {
  const int64_t threads = n_ids * (dims >> 5);
  const int64_t grid = (threads + 255) / 256;
  hipLaunchKernelGGL(embedding_kernel<T>, dim3((unsigned)grid), dim3(256), 0, s, packed, ids, ids64, n_ids, vocab,
                     dims, out, odt, t);
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
