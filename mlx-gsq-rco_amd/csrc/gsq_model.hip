// Fused element-wise work of the Qwen3.5-hybrid decode step around the packed projections:
// residual add + RMSNorm, SwiGLU, and one GatedDeltaNet token step.
//
// The reference runs these as mlx / mlx-lm operations (mlx_gsq/models/qwen35.py:48-111 and the
// mlx-lm layers it patches: RMSNorm, SwiGLU MLP, gated_delta_update). Each kernel computes what
// the torch formulation in mlx_gsq_amd/models/qwen35.py computes, in fp32 with the same
// roundings to the activation dtype, in one launch instead of tens: at M = 1 the step is made of
// thousands of tiny operations and their launch cost, not their arithmetic, bounds it.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gsq_common.h"

namespace gsq {

enum { MD_F32 = 0, MD_F16 = 1, MD_BF16 = 2 };

template <int DT> struct Elem;
template <> struct Elem<MD_F32> {
  using T = float;
  __device__ static float ld(const T* p) { return *p; }
  __device__ static T mk(float v) { return v; }
};
template <> struct Elem<MD_F16> {
  using T = _Float16;
  __device__ static float ld(const T* p) { return (float)*p; }
  __device__ static T mk(float v) { return (_Float16)v; }
};
template <> struct Elem<MD_BF16> {
  using T = uint16_t;
  __device__ static float ld(const T* p) { return __builtin_bit_cast(float, (uint32_t)*p << 16); }
  __device__ static T mk(float v) { return (uint16_t)f32_to_bf16_bits(v); }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Workgroup barrier that waits for this wave's LDS operations only: global loads issued before
// it stay in flight. The kernels here exchange data between threads through LDS only.
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// sum of v over the block (blockDim.x a multiple of 64, at most 1024); every thread gets it
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_sum(v);
  lds_sync();  // red may still be read by a previous call
  if (lane == 0) red[wave] = v;
  lds_sync();
  float s = 0.f;
  for (int i = 0; i < nw; ++i) s += red[i];
  return s;
}

// four sums at once (one pair of barriers)
__device__ __forceinline__ float4 block_sum4(float4 v, float4* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = make_float4(wave_sum(v.x), wave_sum(v.y), wave_sum(v.z), wave_sum(v.w));
  lds_sync();
  if (lane == 0) red[wave] = v;
  lds_sync();
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int i = 0; i < nw; ++i) {
    const float4 r = red[i];
    s.x += r.x; s.y += r.y; s.z += r.z; s.w += r.w;
  }
  return s;
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }

// ---- residual add + RMSNorm ------------------------------------------------------------
// Row r: if delta, x[r] = round(x[r] + delta[r]) (written back); y[r] = round(x[r] / rms * w).
// One workgroup per row; every thread loads its (up to kNormChunks) 8-element chunks before the
// first use and keeps them in registers, so a row costs one round trip to memory, not one per
// element.
constexpr int kNormThreads = 256, kNormChunks = 4;  // rows of up to 8192 values

template <int DT>
struct Vec8 {  // 8 consecutive elements of a row, as float
  float v[8];
  __device__ void load(const typename Elem<DT>::T* p) {
    if constexpr (DT == MD_F32) {
      const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      const uint4 q = *reinterpret_cast<const uint4*>(p);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const typename Elem<DT>::T lo = __builtin_bit_cast(typename Elem<DT>::T, (uint16_t)(w[i] & 0xFFFFu));
        const typename Elem<DT>::T hi = __builtin_bit_cast(typename Elem<DT>::T, (uint16_t)(w[i] >> 16));
        v[2 * i] = Elem<DT>::ld(&lo);
        v[2 * i + 1] = Elem<DT>::ld(&hi);
      }
    }
  }
  __device__ void store(typename Elem<DT>::T* p) const {
    if constexpr (DT == MD_F32) {
      reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const typename Elem<DT>::T lo = Elem<DT>::mk(v[2 * i]), hi = Elem<DT>::mk(v[2 * i + 1]);
        w[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
      }
      *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
};

template <int DT>
__global__ void __launch_bounds__(kNormThreads) add_rms_norm_kernel(typename Elem<DT>::T* x,
                                                                    const typename Elem<DT>::T* delta,
                                                                    const typename Elem<DT>::T* w,
                                                                    typename Elem<DT>::T* y, int dim, float eps) {
  using T = typename Elem<DT>::T;
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  T* xr = x + row * dim;
  T* yr = y + row * dim;
  const T* dr = delta ? delta + row * dim : nullptr;
  Vec8<DT> xv[kNormChunks], wv[kNormChunks];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int i = 8 * (c * kNormThreads + (int)threadIdx.x);
    if (i < dim) {
      xv[c].load(xr + i);
      wv[c].load(w + i);
    }
  }
  if (dr) {
    Vec8<DT> dv[kNormChunks];
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
      const int i = 8 * (c * kNormThreads + (int)threadIdx.x);
      if (i < dim) dv[c].load(dr + i);
    }
#pragma unroll
    for (int c = 0; c < kNormChunks; ++c) {
      const int i = 8 * (c * kNormThreads + (int)threadIdx.x);
      if (i < dim) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {  // the sum rounded to the activation dtype, as stored
          const T s = Elem<DT>::mk(xv[c].v[e] + dv[c].v[e]);
          xv[c].v[e] = Elem<DT>::ld(&s);
        }
        xv[c].store(xr + i);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int i = 8 * (c * kNormThreads + (int)threadIdx.x);
    if (i < dim) {
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += xv[c].v[e] * xv[c].v[e];
    }
  }
  const float rinv = 1.f / sqrtf(block_sum(ss, red) / (float)dim + eps);
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int i = 8 * (c * kNormThreads + (int)threadIdx.x);
    if (i < dim) {
      Vec8<DT> o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o.v[e] = xv[c].v[e] * rinv * wv[c].v[e];
      o.store(yr + i);
    }
  }
}

// ---- SwiGLU -----------------------------------------------------------------------------
// out[r, i] = round(silu(gu[r, i]) * gu[r, n + i]) for rows of 2n (gate then up).
template <int DT>
__global__ void __launch_bounds__(256) swiglu_kernel(const typename Elem<DT>::T* gu, typename Elem<DT>::T* out,
                                                     int64_t rows, int n) {
  using E = Elem<DT>;
  const int64_t total = rows * n;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / n, i = t - r * n;
    const typename E::T* g = gu + r * 2 * n;
    out[t] = E::mk(silu_f(E::ld(g + i)) * E::ld(g + n + i));
  }
}

// ---- GatedDeltaNet token step -----------------------------------------------------------
constexpr int kGdnMaxDk = 128;  // largest key head dim
constexpr int kGdnMaxK = 8;     // largest convolution kernel
constexpr int kGdnRowGroups = 4;  // threads per state column, each with dk / 4 rows

// Causal depthwise convolution + SiLU of every channel of the new qkv row, one thread per
// (batch row, channel): the channel's window [K-1 cached inputs, the new one] and the shift of
// its cached inputs. Outputs in fp32 to `work`.
template <int DT>
__global__ void __launch_bounds__(256) gdn_conv_kernel(GdnArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  const int conv_dim = 2 * a.Hk * a.dk + a.Hv * a.dv, K = a.K;
  const int c = blockIdx.x * 256 + threadIdx.x, bb = blockIdx.y;
  if (c >= conv_dim) return;
  T* cst = static_cast<T*>(a.conv) + (int64_t)bb * (K - 1) * conv_dim + c;
  const T* cw = static_cast<const T*>(a.conv_w) + (int64_t)c * K;
  float in[kGdnMaxK];  // static indices only: the window stays in registers
#pragma unroll
  for (int t = 0; t < kGdnMaxK; ++t)
    in[t] = t < K - 1 ? E::ld(cst + (int64_t)t * conv_dim)
                      : (t == K - 1 ? E::ld(static_cast<const T*>(a.qkv) + (int64_t)bb * a.qkv_stride + c) : 0.f);
  float acc = in[0] * E::ld(cw);
#pragma unroll
  for (int t = 1; t < kGdnMaxK; ++t)
    if (t < K) acc = acc + in[t] * E::ld(cw + t);
#pragma unroll
  for (int t = 0; t + 1 < kGdnMaxK; ++t)
    if (t < K - 1) cst[(int64_t)t * conv_dim] = E::mk(in[t + 1]);
  a.work[(int64_t)bb * conv_dim + c] = silu_f(acc);
}

// The recurrence of value head h (reads q/k head h % Hk) for one batch row: a and b from the
// layer input (rounded to the activation dtype, as a projection's output is), q and k
// RMS-normalized per head, then with kGdnRowGroups x dv threads, thread (g, j) holding rows
// [g dk/4, (g+1) dk/4) of state column j in registers: S = decay S; kv = S^T k; S += k (beta
// (v - kv))^T; o = S^T q (partial sums over the row groups combined in LDS); then the gated
// RMSNorm over the head's dv columns. Every global load is issued at the start and the barriers
// wait on LDS only, so the kernel costs about one memory round trip plus its reductions.
template <int DT>
__global__ void __launch_bounds__(1024) gdn_rec_kernel(GdnArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  constexpr int R = kGdnRowGroups, MAXR = kGdnMaxDk / R, V = 2;
  __shared__ float sq[kGdnMaxDk], sk[kGdnMaxDk], part[R][256], red[16];
  __shared__ float4 red4[16];
  const int h = blockIdx.x, bb = blockIdx.y, tid = threadIdx.x, nt = blockDim.x;
  const int dk = a.dk, dv = a.dv, Hk = a.Hk, Hv = a.Hv, kh = h % Hk;
  const int key_dim = Hk * dk, conv_dim = 2 * key_dim + Hv * dv;
  const int g = tid / dv, j = tid - g * dv, rows = dk / R;
  const float* co = a.work + (int64_t)bb * conv_dim;
  // the state column (rows past the thread's last one re-read that row and are not used)
  float* S = a.rec + ((int64_t)bb * Hv + h) * dk * dv + (int64_t)g * rows * dv + j;
  float col[MAXR];
#pragma unroll
  for (int i = 0; i < MAXR; ++i) col[i] = S[(int64_t)min(i, rows - 1) * dv];
  const float v = co[2 * key_dim + h * dv + j];
  const int qi = min(tid, dk - 1);
  const float qr = co[kh * dk + qi], kr = co[key_dim + kh * dk + qi];
  const float zv = E::ld(static_cast<const T*>(a.z) + (int64_t)bb * a.z_stride + h * dv + j);
  const float nw = E::ld(static_cast<const T*>(a.norm_w) + j);
  const float dtb = a.dt_bias[h], sa = a.ssm_a[h];
  // a and b of this head: dot products of the layer input with two rows of w_ab
  const T* xr = static_cast<const T*>(a.x) + (int64_t)bb * a.x_stride;
  const T* wa = static_cast<const T*>(a.w_ab) + (int64_t)h * a.hidden;
  const T* wb = static_cast<const T*>(a.w_ab) + (int64_t)(Hv + h) * a.hidden;
  float pa = 0.f, pb = 0.f;
  if ((a.hidden & 7) == 0 && ((reinterpret_cast<uintptr_t>(xr) | reinterpret_cast<uintptr_t>(wa) |
                               reinterpret_cast<uintptr_t>(wb)) & 15) == 0) {
    Vec8<DT> xv[V], av[V], bv[V];  // 8 values per load, at clamped (in-bounds) offsets
#pragma unroll
    for (int c = 0; c < V; ++c) {
      const int i = min(8 * (c * nt + tid), a.hidden - 8);
      xv[c].load(xr + i);
      av[c].load(wa + i);
      bv[c].load(wb + i);
    }
#pragma unroll
    for (int c = 0; c < V; ++c) {
      const float on = 8 * (c * nt + tid) < a.hidden ? 1.f : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pa += on * xv[c].v[e] * av[c].v[e];
        pb += on * xv[c].v[e] * bv[c].v[e];
      }
    }
    for (int i = 8 * (V * nt + tid); i < a.hidden; i += 8 * nt)  // rows wider than 8 V nt
      for (int e = 0; e < 8; ++e) {
        const float x = E::ld(xr + i + e);
        pa += x * E::ld(wa + i + e);
        pb += x * E::ld(wb + i + e);
      }
  } else {
    for (int i = tid; i < a.hidden; i += nt) {
      const float x = E::ld(xr + i);
      pa += x * E::ld(wa + i);
      pb += x * E::ld(wb + i);
    }
  }
  const float4 r = block_sum4(make_float4(pa, pb, tid < dk ? qr * qr : 0.f, tid < dk ? kr * kr : 0.f), red4);
  // q and k of key head kh, RMS-normalized (eps 1e-6) and scaled by dk^-1 and dk^-1/2
  if (tid < dk) {
    sq[tid] = qr * (1.f / sqrtf(r.z / (float)dk + 1e-6f)) * (1.f / (float)dk);
    sk[tid] = kr * (1.f / sqrtf(r.w / (float)dk + 1e-6f)) * (1.f / sqrtf((float)dk));
  }
  // beta and decay (every thread holds the same sums and computes them alike)
  const T ra = E::mk(r.x), rb = E::mk(r.y);  // the projections' outputs are stored rounded
  const float av_ = E::ld(&ra) + dtb, bv_ = E::ld(&rb);
  const float sp = av_ > 20.f ? av_ : log1pf(expf(av_));  // softplus (torch's threshold 20)
  const float beta = 1.f / (1.f + expf(-bv_));
  const float decay = expf(sa * sp);
  lds_sync();
  const float* kg = sk + g * rows;
  const float* qg = sq + g * rows;
  float kv = 0.f;
#pragma unroll
  for (int i = 0; i < MAXR; ++i) {
    const float s = col[i] * decay;
    col[i] = s;
    kv += (i < rows ? s : 0.f) * kg[min(i, rows - 1)];
  }
  part[g][j] = kv;
  lds_sync();
  kv = 0.f;
  for (int q = 0; q < R; ++q) kv += part[q][j];
  const float delta = (v - kv) * beta;
  float o = 0.f;
#pragma unroll
  for (int i = 0; i < MAXR; ++i) {
    const float s = col[i] + kg[min(i, rows - 1)] * delta;
    col[i] = s;
    o += (i < rows ? s : 0.f) * qg[min(i, rows - 1)];
  }
#pragma unroll
  for (int i = 0; i < MAXR; ++i)
    if (i < rows) S[(int64_t)i * dv] = col[i];
  lds_sync();  // every thread has read part[][j] for kv
  part[g][j] = o;
  lds_sync();
  o = 0.f;
  for (int q = 0; q < R; ++q) o += part[q][j];
  // gated RMSNorm over the dv columns (every row group holds the same o; group 0's sum is used)
  const float ss = block_sum(g == 0 ? o * o : 0.f, red);
  if (g == 0) {
    const float rn = 1.f / sqrtf(ss / (float)dv + a.eps);
    static_cast<T*>(a.out)[(int64_t)bb * a.out_stride + h * dv + j] = E::mk(o * rn * nw * silu_f(zv));
  }
}

// ---- GatedDeltaNet over a sequence (prefill) ----------------------------------------------
// The convolution of every (token, channel) at once (thread per channel, grid over tokens and
// batch rows): the window of token t is the inputs t-K+1 .. t, from the state for those before
// the sequence. The state is left alone here and advanced by gdn_rec_seq_kernel afterwards.
template <int DT>
__global__ void __launch_bounds__(256) gdn_conv_seq_kernel(GdnArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  const int conv_dim = 2 * a.Hk * a.dk + a.Hv * a.dv, K = a.K, S = a.S;
  const int c = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y, bb = blockIdx.z;
  if (c >= conv_dim) return;
  const T* cst = static_cast<const T*>(a.conv) + (int64_t)bb * (K - 1) * conv_dim + c;
  const T* q = static_cast<const T*>(a.qkv) + (int64_t)bb * S * a.qkv_stride + c;
  const T* cw = static_cast<const T*>(a.conv_w) + (int64_t)c * K;
  float in[kGdnMaxK];
#pragma unroll
  for (int i = 0; i < kGdnMaxK; ++i) {
    const int u = t - (K - 1) + i;  // input position (negative: from the state)
    in[i] = i < K ? (u < 0 ? E::ld(cst + (int64_t)(K - 1 + u) * conv_dim) : E::ld(q + (int64_t)u * a.qkv_stride)) : 0.f;
  }
  float acc = in[0] * E::ld(cw);
#pragma unroll
  for (int i = 1; i < kGdnMaxK; ++i)
    if (i < K) acc = acc + in[i] * E::ld(cw + i);
  a.work[((int64_t)bb * S + t) * conv_dim + c] = silu_f(acc);
}

// The recurrence of value head h over the S tokens of batch row b, the state column held in
// registers from the first token to the last; per token as gdn_rec_kernel (a and b read from
// `ab` instead of being projected here). Also advances the convolution state of the head's
// channels (v channels, and the q/k channels of key head h when h < Hk) to the last K-1 inputs.
template <int DT>
__global__ void __launch_bounds__(1024) gdn_rec_seq_kernel(GdnArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  constexpr int R = kGdnRowGroups, MAXR = kGdnMaxDk / R;
  __shared__ float sq[kGdnMaxDk], sk[kGdnMaxDk], part[R][256], red[16];
  __shared__ float4 red4[16];
  const int h = blockIdx.x, bb = blockIdx.y, tid = threadIdx.x, nt = blockDim.x;
  const int dk = a.dk, dv = a.dv, Hk = a.Hk, Hv = a.Hv, kh = h % Hk, S = a.S, K = a.K;
  const int key_dim = Hk * dk, conv_dim = 2 * key_dim + Hv * dv;
  const int g = tid / dv, j = tid - g * dv, rows = dk / R;
  float* Sp = a.rec + ((int64_t)bb * Hv + h) * dk * dv + (int64_t)g * rows * dv + j;
  float col[MAXR];
#pragma unroll
  for (int i = 0; i < MAXR; ++i) col[i] = Sp[(int64_t)min(i, rows - 1) * dv];
  const float nw = E::ld(static_cast<const T*>(a.norm_w) + j);
  const float dtb = a.dt_bias[h], sa = a.ssm_a[h];
  const int qi = min(tid, dk - 1);
  const float* kg = sk + g * rows;
  const float* qg = sq + g * rows;
  for (int t = 0; t < S; ++t) {
    const int64_t row = (int64_t)bb * S + t;
    const float* co = a.work + row * conv_dim;
    const float v = co[2 * key_dim + h * dv + j];
    const float qr = co[kh * dk + qi], kr = co[key_dim + kh * dk + qi];
    const float zv = E::ld(static_cast<const T*>(a.z) + row * a.z_stride + h * dv + j);
    const T* abr = static_cast<const T*>(a.ab) + row * a.ab_stride;
    const float av = E::ld(abr + h) + dtb, bv = E::ld(abr + Hv + h);
    const float4 r = block_sum4(make_float4(0.f, 0.f, tid < dk ? qr * qr : 0.f, tid < dk ? kr * kr : 0.f), red4);
    if (tid < dk) {
      sq[tid] = qr * (1.f / sqrtf(r.z / (float)dk + 1e-6f)) * (1.f / (float)dk);
      sk[tid] = kr * (1.f / sqrtf(r.w / (float)dk + 1e-6f)) * (1.f / sqrtf((float)dk));
    }
    const float sp = av > 20.f ? av : log1pf(expf(av));
    const float beta = 1.f / (1.f + expf(-bv));
    const float decay = expf(sa * sp);
    lds_sync();
    float kv = 0.f;
#pragma unroll
    for (int i = 0; i < MAXR; ++i) {
      const float s = col[i] * decay;
      col[i] = s;
      kv += (i < rows ? s : 0.f) * kg[min(i, rows - 1)];
    }
    part[g][j] = kv;
    lds_sync();
    kv = 0.f;
    for (int q = 0; q < R; ++q) kv += part[q][j];
    const float delta = (v - kv) * beta;
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < MAXR; ++i) {
      const float s = col[i] + kg[min(i, rows - 1)] * delta;
      col[i] = s;
      o += (i < rows ? s : 0.f) * qg[min(i, rows - 1)];
    }
    lds_sync();  // every thread has read part[][j] for kv, and sq / sk for this token
    part[g][j] = o;
    lds_sync();
    o = 0.f;
    for (int q = 0; q < R; ++q) o += part[q][j];
    const float ss = block_sum(g == 0 ? o * o : 0.f, red);
    if (g == 0) {
      const float rn = 1.f / sqrtf(ss / (float)dv + a.eps);
      static_cast<T*>(a.out)[row * a.out_stride + h * dv + j] = E::mk(o * rn * nw * silu_f(zv));
    }
  }
#pragma unroll
  for (int i = 0; i < MAXR; ++i)
    if (i < rows) Sp[(int64_t)i * dv] = col[i];
  // the convolution state: the last K-1 inputs (from the sequence, or shifted from the state
  // when the sequence is shorter), in ascending slots so an in-place shift reads before it writes
  const int nch = dv + (h < Hk ? 2 * dk : 0);
  T* cst = static_cast<T*>(a.conv) + (int64_t)bb * (K - 1) * conv_dim;
  const T* qs = static_cast<const T*>(a.qkv) + (int64_t)bb * S * a.qkv_stride;
  for (int idx = tid; idx < nch; idx += nt) {
    const int c = idx < dv ? 2 * key_dim + h * dv + idx : (idx < dv + dk ? h * dk + idx - dv : key_dim + h * dk + idx - dv - dk);
    for (int i = 0; i < K - 1; ++i) {
      const int u = S - (K - 1) + i;
      cst[(int64_t)i * conv_dim + c] = u < 0 ? cst[(int64_t)(K - 1 + u) * conv_dim + c] : qs[(int64_t)u * a.qkv_stride + c];
    }
  }
}

hipError_t launch_gdn_seq(int dt, const GdnArgs& a, hipStream_t s) {
  const int conv_dim = 2 * a.Hk * a.dk + a.Hv * a.dv;
  const dim3 cgrid((unsigned)((conv_dim + 255) / 256), (unsigned)a.S, (unsigned)a.B), rgrid((unsigned)a.Hv, (unsigned)a.B);
  const dim3 rblock((unsigned)(kGdnRowGroups * a.dv));
  if (dt == MD_F16) {
    hipLaunchKernelGGL(gdn_conv_seq_kernel<MD_F16>, cgrid, dim3(256), 0, s, a);
    hipLaunchKernelGGL(gdn_rec_seq_kernel<MD_F16>, rgrid, rblock, 0, s, a);
  } else if (dt == MD_BF16) {
    hipLaunchKernelGGL(gdn_conv_seq_kernel<MD_BF16>, cgrid, dim3(256), 0, s, a);
    hipLaunchKernelGGL(gdn_rec_seq_kernel<MD_BF16>, rgrid, rblock, 0, s, a);
  } else {
    hipLaunchKernelGGL(gdn_conv_seq_kernel<MD_F32>, cgrid, dim3(256), 0, s, a);
    hipLaunchKernelGGL(gdn_rec_seq_kernel<MD_F32>, rgrid, rblock, 0, s, a);
  }
  return hipGetLastError();
}

// ---- gated attention, one new token -------------------------------------------------------
// Workgroup (query head h, batch row b), 256 threads, kv head h / rep. In order, as the torch
// formulation rounds: q = round(rms_norm(q) * w_q), k likewise with w_k, both rotated on their
// first rd dims (rotate-half, angle pos * inv_freq[i], computed in double) and rounded; the
// kv head's first query head writes k and v at position pos of the caches (other workgroups use
// the copies they computed, so no workgroup reads a cache slot another may still be writing);
// scores q . K[j] / sqrt(hd) for j <= pos, softmax, o = sum_j p_j V[j], out = round(o *
// sigmoid(gate)).

template <int DT>
__device__ __forceinline__ void attn_norm_rope(const typename Elem<DT>::T* src, const typename Elem<DT>::T* w,
                                               const AttnArgs& a, int p, float* dst, float* red) {
  using E = Elem<DT>;
  using T = typename E::T;
  const int t = threadIdx.x, hd = a.hd, rd = a.rd;
  const float x = t < hd ? E::ld(src + t) : 0.f;
  const float rinv = 1.f / sqrtf(block_sum(x * x, red) / (float)hd + a.eps);
  float n = 0.f;
  if (t < hd) {
    const T r = E::mk(x * rinv * E::ld(w + t));
    n = E::ld(&r);
    dst[t] = n;
  }
  __syncthreads();
  if (t < rd) {
    const int hr = rd / 2, i = t < hr ? t : t - hr;
    const double ang = (double)p * a.inv_freq[i];
    const float c = (float)cos(ang), s = (float)sin(ang);
    const float other = t < hr ? -dst[t + hr] : dst[t - hr];
    const T r = E::mk(n * c + other * s);
    n = E::ld(&r);
  }
  __syncthreads();
  if (t < hd) dst[t] = n;
  __syncthreads();
}

// Two block sums at once (one pair of LDS barriers); red holds at least 16 floats.
__device__ __forceinline__ float2 block_sum2(float a, float b, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  a = wave_sum(a);
  b = wave_sum(b);
  lds_sync();
  if (lane == 0) { red[wave] = a; red[8 + wave] = b; }
  lds_sync();
  float sa = 0.f, sb = 0.f;
  for (int i = 0; i < nw; ++i) { sa += red[i]; sb += red[8 + i]; }
  return make_float2(sa, sb);
}

// Single-token gated attention, one workgroup per (query head, batch row). Every global load
// of the step is issued at the start: q, its gate, the new k and v, both norm weights, the
// rotary frequency, the first pass of cached K rows (a quarter row per thread, positions
// 0..63) and the first 8 cached V rows; the barriers wait on LDS only, so a short context costs
// one memory round trip. The arithmetic (norms, rotary, scores, softmax, V sums) is the same
// as, and in the same order as, the separate steps it replaces.
// A position outside the cache (pos < 0 or pos >= L, e.g. a graph replayed past the cache's
// end) would write K / V rows outside the head's cache slab and scores past the LDS: the
// attention kernels then write NaN rows to out and touch nothing else. Uniform per workgroup.
template <typename T, typename E>
__device__ __forceinline__ bool attn_pos_invalid(const AttnArgs& a, int h, int bb, int t) {
  const int64_t p = a.pos[0];
  if (p >= 0 && p < a.L) return false;
  if (t < a.hd) static_cast<T*>(a.out)[(int64_t)bb * a.out_stride + (int64_t)h * a.hd + t] = E::mk(__builtin_nanf(""));
  return true;
}

template <int DT>
__global__ void __launch_bounds__(256) attn_decode_kernel(AttnArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  extern __shared__ float sc[];  // scores of positions 0..pos
  __shared__ float sq[256], sk[256], red[16];
  const int h = blockIdx.x, bb = blockIdx.y, t = threadIdx.x;
  const int hd = a.hd, rd = a.rd, rep = a.H / a.Hkv, kvh = h / rep;
  if (attn_pos_invalid<T, E>(a, h, bb, t)) return;  // uniform: before any cache, LDS or barrier
  const int p = (int)a.pos[0];
  const T* qg = static_cast<const T*>(a.qg) + (int64_t)bb * a.qg_stride + (int64_t)h * 2 * hd;
  const T* kn = static_cast<const T*>(a.k) + (int64_t)bb * a.k_stride + (int64_t)kvh * hd;
  const T* vn = static_cast<const T*>(a.v) + (int64_t)bb * a.v_stride + (int64_t)kvh * hd;
  const int64_t base = ((int64_t)bb * a.Hkv + kvh) * a.L * hd;
  const T* K = static_cast<const T*>(a.kc) + base;
  const T* V = static_cast<const T*>(a.vc) + base;
  const bool th = t < hd;
  const float xq = th ? E::ld(qg + t) : 0.f, gate = th ? E::ld(qg + hd + t) : 0.f;
  const float xk = th ? E::ld(kn + t) : 0.f, xv = th ? E::ld(vn + t) : 0.f;
  const float wq = th ? E::ld(static_cast<const T*>(a.q_norm_w) + t) : 0.f;
  const float wk = th ? E::ld(static_cast<const T*>(a.k_norm_w) + t) : 0.f;
  const int hr = rd / 2;
  const double fr = t < rd ? a.inv_freq[t < hr ? t : t - hr] : 0.0;
  // scores: 64 positions per pass, four threads per position (a quarter of hd each); with hd a
  // multiple of 32 and an aligned cache, a thread's quarter row is read as 8-value chunks, all
  // issued before the first use (the first pass's here)
  const int quarter = hd / 4, pi = t >> 2, qd = t & 3, nchunk = quarter >> 3, d0 = qd * quarter;
  const bool vec = (hd & 31) == 0 && (reinterpret_cast<uintptr_t>(K) & 15) == 0;
  Vec8<DT> kv[8];  // quarter <= 64: at most 8 chunks (later ones re-read the last)
  const bool k_early = vec && pi < p;  // position pi of the first pass, a cached one
  if (k_early) {
#pragma unroll
    for (int c = 0; c < 8; ++c) kv[c].load(K + (int64_t)pi * hd + d0 + 8 * min(c, nchunk - 1));
  }
  float v8[8];  // V rows 0..7 of this thread's column, when the first block of 8 is whole
  const bool v_early = th && p >= 8;
  if (v_early) {
#pragma unroll
    for (int u = 0; u < 8; ++u) v8[u] = E::ld(V + (int64_t)u * hd + t);
  }
  // q and k: RMS norm (one pair of barriers for both sums), then the partial rotary
  const float2 ss = block_sum2(xq * xq, xk * xk, red);
  const float rq = 1.f / sqrtf(ss.x / (float)hd + a.eps), rk = 1.f / sqrtf(ss.y / (float)hd + a.eps);
  float nq = 0.f, nk = 0.f;
  if (th) {
    const T q1 = E::mk(xq * rq * wq), k1 = E::mk(xk * rk * wk);
    nq = E::ld(&q1);
    nk = E::ld(&k1);
    sq[t] = nq;
    sk[t] = nk;
  }
  lds_sync();
  if (t < rd) {
    const double ang = (double)p * fr;
    const float c = (float)cos(ang), s = (float)sin(ang);
    const float oq = t < hr ? -sq[t + hr] : sq[t - hr], ok = t < hr ? -sk[t + hr] : sk[t - hr];
    const T q2 = E::mk(nq * c + oq * s), k2 = E::mk(nk * c + ok * s);
    nq = E::ld(&q2);
    nk = E::ld(&k2);
  }
  lds_sync();
  if (th) {
    sq[t] = nq;
    sk[t] = nk;
  }
  if (h % rep == 0 && th) {
    static_cast<T*>(a.kc)[base + (int64_t)p * hd + t] = E::mk(nk);
    static_cast<T*>(a.vc)[base + (int64_t)p * hd + t] = E::mk(xv);
  }
  lds_sync();
  const float scale = 1.f / sqrtf((float)hd);
  float mx = -INFINITY;
  for (int j0 = 0; j0 <= p; j0 += 64) {
    const int j = j0 + pi;
    float part = 0.f;
    if (j <= p) {
      if (j == p) {
        for (int d = 0; d < quarter; ++d) part += sq[d0 + d] * sk[d0 + d];
      } else if (vec) {
        if (j0 > 0 || !k_early) {
          const T* kr = K + (int64_t)j * hd + d0;
#pragma unroll
          for (int c = 0; c < 8; ++c) kv[c].load(kr + 8 * min(c, nchunk - 1));
        }
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (c < nchunk) {
#pragma unroll
            for (int e = 0; e < 8; ++e) part += sq[d0 + 8 * c + e] * kv[c].v[e];
          }
      } else {
        const T* kr = K + (int64_t)j * hd + d0;
        for (int d = 0; d < quarter; ++d) part += sq[d0 + d] * E::ld(kr + d);
      }
    }
    part += __shfl_xor(part, 1, 64);
    part += __shfl_xor(part, 2, 64);
    if (j <= p && qd == 0) {
      sc[j] = part * scale;
      mx = fmaxf(mx, part * scale);
    }
  }
  // softmax over positions 0..pos
  {
    float m = mx;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    lds_sync();
    if ((t & 63) == 0) red[t >> 6] = m;
    lds_sync();
    m = -INFINITY;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) m = fmaxf(m, red[i]);
    float sum = 0.f;
    for (int j = t; j <= p; j += blockDim.x) {
      const float e = expf(sc[j] - m);
      sc[j] = e;
      sum += e;
    }
    sum = block_sum(sum, red);
    const float inv = 1.f / sum;
    for (int j = t; j <= p; j += blockDim.x) sc[j] *= inv;
    lds_sync();
  }
  if (th) {
    float o = 0.f;
    int j = 0;
    if (v_early) {
#pragma unroll
      for (int u = 0; u < 8; ++u) o += sc[u] * v8[u];
      j = 8;
    }
    for (; j + 8 <= p; j += 8) {  // 8 positions' loads in flight at a time, summed in order
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = E::ld(V + (int64_t)(j + u) * hd + t);
#pragma unroll
      for (int u = 0; u < 8; ++u) o += sc[j + u] * v[u];
    }
    for (; j < p; ++j) o += sc[j] * E::ld(V + (int64_t)j * hd + t);
    o += sc[p] * xv;
    static_cast<T*>(a.out)[(int64_t)bb * a.out_stride + (int64_t)h * hd + t] = E::mk(o * (1.f / (1.f + expf(-gate))));
  }
}

// ---- gated attention over position chunks (long contexts) --------------------------------
// Workgroup (query head h, batch row b, chunk c) covers positions [c chunk, (c + 1) chunk) up to
// pos: q (and, in the chunk holding pos, the new k and v, which its KV head's first query head
// also writes to the caches) as in attn_decode_kernel, the chunk's scores, their max m_c, the
// sum l_c of exp(score - m_c) and o_c = sum exp(score - m_c) V, written to work; chunks past
// pos write m_c = -inf. attn_combine_kernel then forms softmax-weighted V from the chunks,
// o = sum_c exp(m_c - m) o_c / sum_c exp(m_c - m) l_c with m the largest m_c, and the gate.
constexpr int kAttnChunkMax = 1024;

template <int DT>
__global__ void __launch_bounds__(256) attn_chunk_kernel(AttnArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  __shared__ float sq[256], sk[256], sv[256], red[16], sc[kAttnChunkMax];
  const int h = blockIdx.x, bb = blockIdx.y, c = blockIdx.z, t = threadIdx.x;
  const int hd = a.hd, rep = a.H / a.Hkv, kvh = h / rep;
  if (a.pos[0] < 0 || a.pos[0] >= a.L) return;  // the combine kernel writes NaN rows
  const int p = (int)a.pos[0];
  const int j0 = c * a.chunk;
  float* part = a.work + (((int64_t)bb * a.H + h) * a.nsplit + c) * (hd + 2);
  if (j0 > p) {  // a chunk past the new token: contributes nothing
    if (t == 0) { part[0] = -INFINITY; part[1] = 0.f; }
    if (t < hd) part[2 + t] = 0.f;
    return;
  }
  const int j1 = min(j0 + a.chunk, p + 1);  // positions [j0, j1)
  const bool has_new = p < j0 + a.chunk;    // the chunk holds the new token (uniform)
  const T* qg = static_cast<const T*>(a.qg) + (int64_t)bb * a.qg_stride + (int64_t)h * 2 * hd;
  attn_norm_rope<DT>(qg, static_cast<const T*>(a.q_norm_w), a, p, sq, red);
  const int64_t base = ((int64_t)bb * a.Hkv + kvh) * a.L * hd;
  const T* K = static_cast<const T*>(a.kc) + base;
  const T* V = static_cast<const T*>(a.vc) + base;
  if (has_new) {
    attn_norm_rope<DT>(static_cast<const T*>(a.k) + (int64_t)bb * a.k_stride + (int64_t)kvh * hd,
                       static_cast<const T*>(a.k_norm_w), a, p, sk, red);
    const T* vr = static_cast<const T*>(a.v) + (int64_t)bb * a.v_stride + (int64_t)kvh * hd;
    if (t < hd) sv[t] = E::ld(vr + t);
    if (h % rep == 0 && t < hd) {
      static_cast<T*>(a.kc)[base + (int64_t)p * hd + t] = E::mk(sk[t]);
      static_cast<T*>(a.vc)[base + (int64_t)p * hd + t] = E::mk(sv[t]);
    }
  }
  __syncthreads();
  const float scale = 1.f / sqrtf((float)hd);
  const int quarter = hd / 4, pi = t >> 2, qd = t & 3, nchunk = quarter >> 3;
  const bool vec = (hd & 31) == 0 && (reinterpret_cast<uintptr_t>(K) & 15) == 0;
  float mx = -INFINITY;
  for (int jb = j0; jb < j1; jb += 64) {
    const int j = jb + pi;
    float part_s = 0.f;
    if (j < j1) {
      const int d0 = qd * quarter;
      if (j == p) {
        for (int d = 0; d < quarter; ++d) part_s += sq[d0 + d] * sk[d0 + d];
      } else if (vec) {
        const T* kr = K + (int64_t)j * hd + d0;
        Vec8<DT> kv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) kv[u].load(kr + 8 * min(u, nchunk - 1));
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (u < nchunk) {
#pragma unroll
            for (int e = 0; e < 8; ++e) part_s += sq[d0 + 8 * u + e] * kv[u].v[e];
          }
      } else {
        const T* kr = K + (int64_t)j * hd + d0;
        for (int d = 0; d < quarter; ++d) part_s += sq[d0 + d] * E::ld(kr + d);
      }
    }
    part_s += __shfl_xor(part_s, 1, 64);
    part_s += __shfl_xor(part_s, 2, 64);
    if (j < j1 && qd == 0) {
      sc[j - j0] = part_s * scale;
      mx = fmaxf(mx, part_s * scale);
    }
  }
  float m = mx;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  __syncthreads();
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  m = -INFINITY;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) m = fmaxf(m, red[i]);
  float sum = 0.f;
  for (int j = t; j < j1 - j0; j += blockDim.x) {
    const float e = expf(sc[j] - m);
    sc[j] = e;
    sum += e;
  }
  sum = block_sum(sum, red);
  __syncthreads();
  if (t < hd) {
    float o = 0.f;
    const int jn = has_new ? p : j1;  // cached positions; the new one comes from sv
    int j = j0;
    for (; j + 8 <= jn; j += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = E::ld(V + (int64_t)(j + u) * hd + t);
#pragma unroll
      for (int u = 0; u < 8; ++u) o += sc[j - j0 + u] * v[u];
    }
    for (; j < jn; ++j) o += sc[j - j0] * E::ld(V + (int64_t)j * hd + t);
    if (has_new) o += sc[p - j0] * sv[t];
    part[2 + t] = o;
  }
  if (t == 0) { part[0] = m; part[1] = sum; }
}

template <int DT>
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  const int h = blockIdx.x, bb = blockIdx.y, t = threadIdx.x, hd = a.hd;
  if (attn_pos_invalid<T, E>(a, h, bb, t)) return;
  if (t >= hd) return;
  const float* part = a.work + ((int64_t)bb * a.H + h) * a.nsplit * (hd + 2);
  float m = -INFINITY;
  for (int c = 0; c < a.nsplit; ++c) m = fmaxf(m, part[(int64_t)c * (hd + 2)]);
  float l = 0.f, o = 0.f;
  for (int c = 0; c < a.nsplit; ++c) {
    const float* pc = part + (int64_t)c * (hd + 2);
    const float w = expf(pc[0] - m);  // 0 for chunks past the new token
    l += w * pc[1];
    o += w * pc[2 + t];
  }
  const T* qg = static_cast<const T*>(a.qg) + (int64_t)bb * a.qg_stride + (int64_t)h * 2 * hd;
  const float gate = E::ld(qg + hd + t);
  static_cast<T*>(a.out)[(int64_t)bb * a.out_stride + (int64_t)h * hd + t] =
      E::mk(o / l * (1.f / (1.f + expf(-gate))));
}

constexpr int kAttnMaxPositions = 32768;  // scores of up to this many positions stay in LDS

template <int DT>
static hipError_t attn_lds_attr() {
  static bool done = false;
  if (!done) {
    hipError_t e = hipFuncSetAttribute((const void*)attn_decode_kernel<DT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       kAttnMaxPositions * (int)sizeof(float));
    if (e != hipSuccess) return e;
    done = true;
  }
  return hipSuccess;
}

hipError_t launch_attn_decode(int dt, const AttnArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)a.H, (unsigned)a.B);
  if (a.work) {
    if (a.chunk < 64 || a.chunk > kAttnChunkMax || a.nsplit < 1 || (int64_t)a.nsplit * a.chunk < a.L)
      return hipErrorInvalidValue;
    const dim3 cgrid((unsigned)a.H, (unsigned)a.B, (unsigned)a.nsplit);
    if (dt == MD_F16) {
      hipLaunchKernelGGL(attn_chunk_kernel<MD_F16>, cgrid, dim3(256), 0, s, a);
      hipLaunchKernelGGL(attn_combine_kernel<MD_F16>, grid, dim3(256), 0, s, a);
    } else if (dt == MD_BF16) {
      hipLaunchKernelGGL(attn_chunk_kernel<MD_BF16>, cgrid, dim3(256), 0, s, a);
      hipLaunchKernelGGL(attn_combine_kernel<MD_BF16>, grid, dim3(256), 0, s, a);
    } else {
      hipLaunchKernelGGL(attn_chunk_kernel<MD_F32>, cgrid, dim3(256), 0, s, a);
      hipLaunchKernelGGL(attn_combine_kernel<MD_F32>, grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
  }
  const size_t lds = (size_t)a.L * sizeof(float);
  if (a.L > kAttnMaxPositions) return hipErrorInvalidValue;
  hipError_t e = dt == MD_F16 ? attn_lds_attr<MD_F16>() : (dt == MD_BF16 ? attn_lds_attr<MD_BF16>() : attn_lds_attr<MD_F32>());
  if (e != hipSuccess) return e;
  if (dt == MD_F16) hipLaunchKernelGGL(attn_decode_kernel<MD_F16>, grid, dim3(256), lds, s, a);
  else if (dt == MD_BF16) hipLaunchKernelGGL(attn_decode_kernel<MD_BF16>, grid, dim3(256), lds, s, a);
  else hipLaunchKernelGGL(attn_decode_kernel<MD_F32>, grid, dim3(256), lds, s, a);
  return hipGetLastError();
}

hipError_t launch_add_rms_norm(int dt, void* x, const void* delta, const void* w, void* y, int64_t rows, int dim,
                               float eps, hipStream_t s) {
  const dim3 grid((unsigned)rows), block(kNormThreads);
  if (dt == MD_F16)
    hipLaunchKernelGGL(add_rms_norm_kernel<MD_F16>, grid, block, 0, s, static_cast<_Float16*>(x),
                       static_cast<const _Float16*>(delta), static_cast<const _Float16*>(w), static_cast<_Float16*>(y),
                       dim, eps);
  else if (dt == MD_BF16)
    hipLaunchKernelGGL(add_rms_norm_kernel<MD_BF16>, grid, block, 0, s, static_cast<uint16_t*>(x),
                       static_cast<const uint16_t*>(delta), static_cast<const uint16_t*>(w), static_cast<uint16_t*>(y),
                       dim, eps);
  else
    hipLaunchKernelGGL(add_rms_norm_kernel<MD_F32>, grid, block, 0, s, static_cast<float*>(x),
                       static_cast<const float*>(delta), static_cast<const float*>(w), static_cast<float*>(y), dim, eps);
  return hipGetLastError();
}

hipError_t launch_swiglu(int dt, const void* gu, void* out, int64_t rows, int n, hipStream_t s) {
  const int64_t total = rows * n;
  const unsigned blocks = (unsigned)(total / 256 + 1 < 8192 ? total / 256 + 1 : 8192);
  if (dt == MD_F16)
    hipLaunchKernelGGL(swiglu_kernel<MD_F16>, dim3(blocks), dim3(256), 0, s, static_cast<const _Float16*>(gu),
                       static_cast<_Float16*>(out), rows, n);
  else if (dt == MD_BF16)
    hipLaunchKernelGGL(swiglu_kernel<MD_BF16>, dim3(blocks), dim3(256), 0, s, static_cast<const uint16_t*>(gu),
                       static_cast<uint16_t*>(out), rows, n);
  else
    hipLaunchKernelGGL(swiglu_kernel<MD_F32>, dim3(blocks), dim3(256), 0, s, static_cast<const float*>(gu),
                       static_cast<float*>(out), rows, n);
  return hipGetLastError();
}

hipError_t launch_gdn_step(int dt, const GdnArgs& a, hipStream_t s) {
  const int conv_dim = 2 * a.Hk * a.dk + a.Hv * a.dv;
  const dim3 cgrid((unsigned)((conv_dim + 255) / 256), (unsigned)a.B), rgrid((unsigned)a.Hv, (unsigned)a.B);
  const dim3 rblock((unsigned)(kGdnRowGroups * a.dv));
  // without a convolution state, `work` already holds the convolution outputs
  const bool conv = a.conv != nullptr;
  if (dt == MD_F16) {
    if (conv) hipLaunchKernelGGL(gdn_conv_kernel<MD_F16>, cgrid, dim3(256), 0, s, a);
    hipLaunchKernelGGL(gdn_rec_kernel<MD_F16>, rgrid, rblock, 0, s, a);
  } else if (dt == MD_BF16) {
    if (conv) hipLaunchKernelGGL(gdn_conv_kernel<MD_BF16>, cgrid, dim3(256), 0, s, a);
    hipLaunchKernelGGL(gdn_rec_kernel<MD_BF16>, rgrid, rblock, 0, s, a);
  } else {
    if (conv) hipLaunchKernelGGL(gdn_conv_kernel<MD_F32>, cgrid, dim3(256), 0, s, a);
    hipLaunchKernelGGL(gdn_rec_kernel<MD_F32>, rgrid, rblock, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace gsq
