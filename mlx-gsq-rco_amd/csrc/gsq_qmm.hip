// Tiled quantized matrix-matrix product (QMM) for prefill: y[M,N] = x[M,K] * W[N,K]^T.
//
// Counterpart of the reference's tiled decode-once kernel
// (mlx_gsq/runtime/kernels/qmm.py:252-325, dispatched by quantized_matmul qmm.py:559-594):
// each weight tile is decoded once into an fp16 LDS tile (the reference also stores its
// decoded tile as half, qmm.py:181) and reused by every activation row of the workgroup's
// M tile; products accumulate in fp32.
//
// gfx950 schedule: a 256-thread workgroup computes a BM x BN = 64 x 64 output tile over
// K steps of 64 (two 32-weight groups per weight row). Per step, half of the threads
// decode the 64 rows x 2 groups of weights (exact fp32 -> fp16, round to nearest even),
// the other half stage the activation tile as fp16; then each wave multiplies a 32 x 32
// sub-tile with v_mfma_f32_16x16x32_f16.
#include "gsq_decode.h"

namespace gsq {

enum { QDT_F32 = 0, QDT_F16 = 1, QDT_BF16 = 2 };

constexpr int kBM = 64, kBN = 64, kKS = 64, kLdsStride = kKS + 8;  // halves per LDS row

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

struct QmmArgs {
  const uint8_t* packed;
  const void* x;
  void* y;
  int64_t M, N;
  int K, x_dtype, y_dtype;
  DevTables tb;
};

__device__ __forceinline__ float qmm_load_x(const void* x, int dt, int64_t i) {
  if (dt == QDT_F16) return (float)reinterpret_cast<const _Float16*>(x)[i];
  if (dt == QDT_BF16) return __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t*>(x)[i] << 16);
  return reinterpret_cast<const float*>(x)[i];
}

__device__ __forceinline__ void qmm_store_y(void* y, int dt, int64_t i, float v) {
  if (dt == QDT_F16) reinterpret_cast<_Float16*>(y)[i] = (_Float16)v;
  else if (dt == QDT_BF16) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    b += 0x7FFFu + ((b >> 16) & 1u);
    reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)(b >> 16);
  } else reinterpret_cast<float*>(y)[i] = v;
}

template <int T>
__global__ void __launch_bounds__(256) qmm_kernel(QmmArgs a) {
  constexpr int BB = BlockBytes<T>::v;
  __shared__ __attribute__((aligned(16))) _Float16 wt[kBN * kLdsStride];
  __shared__ __attribute__((aligned(16))) _Float16 xt[kBM * kLdsStride];
  const int tid = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * kBN;
  const int64_t m0 = (int64_t)blockIdx.y * kBM;
  const int nb = a.K / 256;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;

  float4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < a.K; k0 += kKS) {
    if (tid < 128) {
      // decode one 32-weight group: row r of the tile, group kg of this K step
      const int r = tid >> 1, kg = tid & 1;
      const int64_t n = n0 + r;
      _Float16* dst = wt + r * kLdsStride + 32 * kg;
      if (n < a.N) {
        const int gidx = (k0 >> 5) + kg;
        const uint8_t* blk = a.packed + (n * nb + (gidx >> 3)) * BB;
        float v[32];
        dq_group<T>(blk, gidx & 7, a.tb, v);
#pragma unroll
        for (int i = 0; i < 32; ++i) dst[i] = (_Float16)v[i];
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) dst[i] = (_Float16)0.f;
      }
    } else {
      const int t = tid - 128, r = t >> 1, half = t & 1;
      const int64_t m = m0 + r;
      _Float16* dst = xt + r * kLdsStride + 32 * half;
      if (m < a.M) {
        const int64_t base = m * a.K + k0 + 32 * half;
#pragma unroll
        for (int i = 0; i < 32; ++i) dst[i] = (_Float16)qmm_load_x(a.x, a.x_dtype, base + i);
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) dst[i] = (_Float16)0.f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kKS; kk += 32) {
      half8_t af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const half8_t*>(xt + (wm * 32 + i * 16 + (lane & 15)) * kLdsStride + kk + 8 * (lane >> 4));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const half8_t*>(wt + (wn * 32 + j * 16 + (lane & 15)) * kLdsStride + kk + 8 * (lane >> 4));
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  // C layout: lane holds rows 4*(lane/16)+e (e=0..3) of column lane%16 of each 16x16 tile
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + wn * 32 + j * 16 + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + e;
        if (m < a.M && n < a.N) qmm_store_y(a.y, a.y_dtype, m * a.N + n, acc[i][j][e]);
      }
    }
}

template <int T>
static hipError_t launch_qmm_t(const QmmArgs& a, hipStream_t s) {
  dim3 grid((unsigned)((a.N + kBN - 1) / kBN), (unsigned)((a.M + kBM - 1) / kBM));
  hipLaunchKernelGGL(qmm_kernel<T>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_qmm(int qt, const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M, int64_t N,
                      int K, const DevTables& tb, hipStream_t s) {
  QmmArgs a;
  a.packed = packed; a.x = x; a.y = y; a.M = M; a.N = N; a.K = K; a.x_dtype = xdt; a.y_dtype = ydt; a.tb = tb;
  switch (qt) {
    case Q2_K: return launch_qmm_t<Q2_K>(a, s);
    case Q4_K: return launch_qmm_t<Q4_K>(a, s);
    case Q6_K: return launch_qmm_t<Q6_K>(a, s);
    case IQ4_XS: return launch_qmm_t<IQ4_XS>(a, s);
    case IQ3_S: return launch_qmm_t<IQ3_S>(a, s);
    case IQ3_XXS: return launch_qmm_t<IQ3_XXS>(a, s);
    case IQ2_XXS: return launch_qmm_t<IQ2_XXS>(a, s);
    case IQ2_XS: return launch_qmm_t<IQ2_XS>(a, s);
    case IQ2_S: return launch_qmm_t<IQ2_S>(a, s);
    case IQ1_S: return launch_qmm_t<IQ1_S>(a, s);
    case IQ1_M: return launch_qmm_t<IQ1_M>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gsq
