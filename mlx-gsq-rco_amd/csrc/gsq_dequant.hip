// Bit-exact dequantization: packed superblocks -> float32, one thread per 32-weight group.
//
// This is the parity instrument of the path (the reference's decode kernels
// k_decode.py:17-105, iq_lookup_decode.py:5-62, iq3_s_decode.py:7-79 play the same role,
// checked bit-exactly against gguf-py in tests/test_metal_decoders.py:9-23).
// Every value is computed in float32 with the reference's formula; all products are exact
// in float32, and Q2_K/Q4_K round once in their final subtraction, so the result is
// identical to the CPU dequantizer regardless of evaluation order or FMA contraction.
#include "gsq_decode.h"

namespace gsq {

template <int T>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* __restrict__ packed, int64_t nblocks,
                                                      float* __restrict__ out, DevTables t) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t blk = gid >> 3;
  if (blk >= nblocks) return;
  const int g = (int)(gid & 7);
  float v[32];
  dq_group<T>(packed + blk * BlockBytes<T>::v, g, t, v);
  float4* o4 = reinterpret_cast<float4*>(out + blk * 256 + g * 32);
#pragma unroll
  for (int i = 0; i < 8; ++i) o4[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

template <int T>
static hipError_t launch_dequant_t(const uint8_t* packed, int64_t nblocks, float* out, const DevTables& t,
                                   hipStream_t s) {
  const int64_t threads = nblocks * 8;
  const int64_t grid = (threads + 255) / 256;
  hipLaunchKernelGGL(dequant_kernel<T>, dim3((unsigned)grid), dim3(256), 0, s, packed, nblocks, out, t);
  return hipGetLastError();
}

hipError_t launch_dequant(int qt, const uint8_t* packed, int64_t nblocks, float* out, const DevTables& t,
                          hipStream_t s) {
  switch (qt) {
    case Q2_K: return launch_dequant_t<Q2_K>(packed, nblocks, out, t, s);
    case Q4_K: return launch_dequant_t<Q4_K>(packed, nblocks, out, t, s);
    case Q6_K: return launch_dequant_t<Q6_K>(packed, nblocks, out, t, s);
    case IQ4_XS: return launch_dequant_t<IQ4_XS>(packed, nblocks, out, t, s);
    case IQ3_S: return launch_dequant_t<IQ3_S>(packed, nblocks, out, t, s);
    case IQ3_XXS: return launch_dequant_t<IQ3_XXS>(packed, nblocks, out, t, s);
    case IQ2_XXS: return launch_dequant_t<IQ2_XXS>(packed, nblocks, out, t, s);
    case IQ2_XS: return launch_dequant_t<IQ2_XS>(packed, nblocks, out, t, s);
    case IQ2_S: return launch_dequant_t<IQ2_S>(packed, nblocks, out, t, s);
    case IQ1_S: return launch_dequant_t<IQ1_S>(packed, nblocks, out, t, s);
    case IQ1_M: return launch_dequant_t<IQ1_M>(packed, nblocks, out, t, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gsq
