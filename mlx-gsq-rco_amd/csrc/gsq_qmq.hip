// Quad-row QMV (QMQ): y[M, N] = x[M, K] W^T for 2 <= M <= 8 fp16 activation rows, with the
// products on the matrix cores (v_mfma_f32_4x4x4_16b_f16) and the vector kernel's decoders.
//
// Counterpart of the reference's multi-row packed-dot kernels (mlx_gsq/runtime/kernels/
// qmv.py:76-528, whose kernels take every activation row of the batch, dispatched by
// quantized_matvec qmv.py:537-576) for the small batches that quantized_matvec keeps on the
// vector path.
//
// * Quad layout: a wave's 64 lanes are 16 blocks of 4; lane 4b + r decodes weight row r of a
//   quad of consecutive rows at group b of a "quad slice" (2 superblocks = 16 groups of 32
//   weights per row). The four lanes of a block decode the same K positions of four rows, so one
//   4x4x4 MFMA per 4 weights multiplies them with the same 4 positions of 4 activation rows (one
//   quad; 2 quads for M > 4): a lane's group is decoded once, as in the vector kernel, and the
//   per-row activation products that would take M v_dot2 per weight pair take M / 4 MFMAs per 4
//   weights.
// * A wave owns GL consecutive quad slices (a K range) and keeps the activations of its
//   groups (its lane's activation row of every quad) in registers, read from one copy of the M
//   rows that the workgroup stages in LDS when it fits (else from memory); the W waves of a row slot
//   cover K; each wave streams its K range of consecutive row quads (one item per quad: four
//   row pieces of 2 GL superblocks) through a private LDS ring with direct-to-LDS DMA and exact
//   vmcnt waits, with no barrier in the main loop, like the vector kernel.
// * Per item, each lane's sums (4 NQ activation rows of its weight row) are reduced over the
//   four blocks of each 16-lane row (DPP) into LDS; the workgroup sums the four row parts of
//   its W partials per output at the end and writes its rows.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "gsq_common.h"
#include "gsq_qmv_decode.h"

namespace gsq {

// Activations of group u (elements 32u .. 32u + 31) for the lane's activation rows 4t + r,
// clamped to row M - 1 (their results are not stored), in the type's pairing; the partial sums
// of all four rows of each quad come from the quad's other lanes (DPP broadcasts).
template <int T, int NQ>
__device__ __forceinline__ void qmq_load_x(XQuad<NQ, Qmv<T>::kSums>& xr, int u, const uint16_t* x, int ld, int M,
                                           int r) {
  constexpr int NS = Qmv<T>::kSums;
  using P = Qmv<T>;
  float own[NQ][NS > 0 ? NS : 1];
#pragma unroll
  for (int t = 0; t < NQ; ++t) {
    const int m = min(4 * t + r, M - 1);
    const uint4* p = reinterpret_cast<const uint4*>(x + (int64_t)m * ld + 32 * u);
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = p[k];
    uint32_t w[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      w[4 * k] = v[k].x; w[4 * k + 1] = v[k].y; w[4 * k + 2] = v[k].z; w[4 * k + 3] = v[k].w;
    }
    if constexpr (NS > 0) {
      constexpr uint32_t kOnes = 0x3C003C00u;  // fp16 (1, 1)
      float s8[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float sm = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) sm = dot2(w[4 * i + j], kOnes, sm);
        s8[i] = sm;
      }
      if constexpr (NS == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) own[t][i] = s8[i];
      } else if constexpr (NS == 2) {
        own[t][0] = s8[0] + s8[1];
        own[t][1] = s8[2] + s8[3];
      } else {
        own[t][0] = (s8[0] + s8[1]) + (s8[2] + s8[3]);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if constexpr (P::kPair == PAIR_NAT) {
        xr.h[t][i] = w[i];
      } else {
        int e0, e1;
        pair_idx<P::kPair>(i, e0, e1);
        xr.h[t][i] = half_pair(w, e0, e1);
      }
    }
  }
  if constexpr (NS > 0) {
    // row 4t + i's sums are lane 4b + i's: quad_perm [i, i, i, i]
#pragma unroll
    for (int t = 0; t < NQ; ++t)
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int v = __builtin_bit_cast(int, own[t][s]);
        xr.s8[4 * t + 0][s] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x00, 0xF, 0xF, false));
        xr.s8[4 * t + 1][s] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0x55, 0xF, 0xF, false));
        xr.s8[4 * t + 2][s] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0xAA, 0xF, 0xF, false));
        xr.s8[4 * t + 3][s] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, v, 0xFF, 0xF, 0xF, false));
      }
  }
}

// Sum of the four blocks of each 16-lane row at the lane's position r = lane % 4 (DPP row
// shifts): lanes 12 + r of each row then hold their row's part; the four rows' parts are summed
// with the workgroup's W partials at the end.
__device__ __forceinline__ float qmq_row_sum(float v) {
  v += dpp_f<0x114, 0xF>(v);  // row_shr:4
  v += dpp_f<0x118, 0xF>(v);  // row_shr:8
  return v;
}

// DMA of item t's four row pieces into the ring buffer dst: granule c of the buffer is granule
// c % G of row c / G's piece (rows past the quad's fourth, and granules past a piece's last one,
// reload that piece's last granule, so the instruction count stays fixed). Row pieces start at
// their 16-byte granule: the decoders add the piece's offset within it.
__device__ __forceinline__ void qmq_dma_item(const QmvArgs& a, int64_t row4, uintptr_t col0, int piece_bytes,
                                             uint8_t* dst, int lane) {
  const int G = a.gran;
  for (int j = 0; j < a.cdma; ++j) {
    const int c = j * 64 + lane;
    const int rr = min(c / G, 3), cg = c - rr * G;
    const int64_t row = min(row4 + rr, a.N - 1);
    const uintptr_t start = reinterpret_cast<uintptr_t>(a.packed) + (uintptr_t)(row * a.row_bytes) + col0;
    const uintptr_t A0 = start & ~(uintptr_t)15;
    const int ngran = (int)((start + (uintptr_t)piece_bytes + 15 - A0) >> 4);
    const uintptr_t src = A0 + (uintptr_t)(cg < ngran ? cg : ngran - 1) * 16;
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src), (lds_ptr_t)(dst + j * 1024), 16, 0, 0);
  }
}

// AL: alignment of the rows. 0: any (2-byte aligned); 1: rows start 4-byte aligned, so each
// lane's offset within its piece keeps the same low bits from item to item (the funnel shifts
// of its word reads are item-invariant); 2: superblocks 4-byte aligned too (plain word reads).
// The same DMA from offsets computed once: with rows starting 4-byte aligned, the rows of
// consecutive items of a wave (4 x slots rows apart) sit at the same offsets within their
// 16-byte granules, so each lane's source is the item's first row piece plus an item-invariant
// offset (rel, for the first kPreJ instructions). Only for items whose four rows exist.
constexpr int kPreJ = 4;
__device__ __forceinline__ void qmq_dma_rel(const QmvArgs& a, int64_t row4, uintptr_t col0, int piece_bytes,
                                            int (&rel)[kPreJ], int lane) {
  const int G = a.gran;
  const uintptr_t base = reinterpret_cast<uintptr_t>(a.packed) + (uintptr_t)(row4 * a.row_bytes) + col0;
#pragma unroll
  for (int j = 0; j < kPreJ; ++j) {
    const int c = j * 64 + lane;
    const int rr = min(c / G, 3), cg = c - rr * G;
    const uintptr_t start = base + (uintptr_t)rr * (uintptr_t)a.row_bytes;
    const uintptr_t A0 = start & ~(uintptr_t)15;
    const int ngran = (int)((start + (uintptr_t)piece_bytes + 15 - A0) >> 4);
    rel[j] = (int)((intptr_t)(A0 + (uintptr_t)(cg < ngran ? cg : ngran - 1) * 16) - (intptr_t)base);
  }
}
__device__ __forceinline__ void qmq_dma_fast(const QmvArgs& a, int64_t row4, uintptr_t col0, const int (&rel)[kPreJ],
                                             uint8_t* dst) {
  const uintptr_t base = reinterpret_cast<uintptr_t>(a.packed) + (uintptr_t)(row4 * a.row_bytes) + col0;
#pragma unroll
  for (int j = 0; j < kPreJ; ++j)
    if (j < a.cdma)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(base + (intptr_t)rel[j]),
                                       (lds_ptr_t)(dst + j * 1024), 16, 0, 0);
}

// Threads per workgroup: up to 16 waves for the one-quad variants of one or two slices per wave
// (at most 128 registers), else 12.
constexpr int qmq_max_threads(int nq, int gl) { return nq == 1 && gl <= 2 ? 1024 : 768; }

template <int T, int NQ, int GL, int AL>
__global__ void __launch_bounds__(qmq_max_threads(NQ, GL)) qmq_kernel(QmvArgs a) {
  using P = Qmv<T>;
  constexpr int BB = BlockBytes<T>::v, MR = 4 * NQ, NS = P::kSums;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* tbl = QmvTblLds<P::kLds>::get();
  uint8_t* dyn = smem - a.tbl_bytes;
  const int tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* red = reinterpret_cast<float*>(dyn + a.red_off);  // [rows_per_wg][MR][W][4]
  uint8_t* ring = dyn + a.ring_off + wave * a.nb * a.sbuf;

  const int64_t r0 = (int64_t)blockIdx.x * a.rows_per_wg;
  const int64_t r1 = min(a.N, r0 + (int64_t)a.rows_per_wg);
  const int nquads = (int)((r1 - r0 + 3) >> 2);
  // row slot (quads slot, slot + slots, ...) and K range (quad slices sl0 .. sl0 + nq - 1)
  const int slot = wave / a.W, ws = wave - slot * a.W;
  const bool live = slot < a.slots && slot < nquads;
  const int sl0 = ws * GL;
  const int nq = live ? max(0, min(GL, a.nslices - sl0)) : 0;
  const int nbk = min(2 * GL, a.nblk - 2 * sl0);  // superblocks per row piece
  const int piece = nbk * BB;
  const int nitems = nq > 0 ? (nquads - slot + a.slots - 1) / a.slots : 0;
  const uintptr_t col0 = (uintptr_t)sl0 * 2 * BB;
  const int r = lane & 3, blk = lane >> 2;

  // item t's DMA: the precomputed offsets while all four rows exist (rows 4-byte aligned and
  // at most kPreJ instructions per item), else the per-lane computation with clamped rows
  const bool pre = AL >= 1 && a.cdma <= kPreJ;
  int rel[kPreJ];
  if (pre) qmq_dma_rel(a, r0 + 4 * slot, col0, piece, rel, lane);
  auto issue = [&](int t, uint8_t* dst) {
    const int64_t row4 = r0 + 4 * (slot + (int64_t)t * a.slots);
    if (pre && row4 + 3 < a.N) qmq_dma_fast(a, row4, col0, rel, dst);
    else qmq_dma_item(a, row4, col0, piece, dst, lane);
  };
  int issued = 0;
  if (nitems > 0) {
    issue(0, ring);
    issued = 1;
  }
  if constexpr (P::kLds > 0) dma_copy(a.tb.qmv_tbl, P::kLds, tbl, wave, nw, lane);
  // activations staged in LDS once per workgroup (x_lds): rows of K + 8 fp16 (16 bytes of pad,
  // so that the four rows a 16-lane read covers fall into distinct banks); the row slots then
  // share one copy instead of each loading its own from L2
  const uint16_t* xs = reinterpret_cast<const uint16_t*>(dyn + a.x_off);
  if (a.x_lds)
    for (int m = 0; m < a.M; ++m)
      dma_copy(static_cast<const uint16_t*>(a.x) + (int64_t)m * a.K, 2 * a.K, dyn + a.x_off + m * (2 * a.K + 16), wave,
               nw, lane);

  // the lane's activations of each slice (group blk of slice sl0 + q), from LDS or from memory
  XQuad<NQ, NS> xr[GL];
  if (a.x_lds) {
    wait_vmcnt(0);    // this wave's first item and its shares of the table and activations
    __syncthreads();  // ... and every other wave's shares
#pragma unroll
    for (int q = 0; q < GL; ++q) {
      const int u = (sl0 + q) * 16 + blk;
      const bool act = q < nq && u < (a.K >> 5);
      qmq_load_x<T, NQ>(xr[q], act ? u : 0, xs, a.K + 8, a.M, r);
    }
  } else {
#pragma unroll
    for (int q = 0; q < GL; ++q) {
      const int u = (sl0 + q) * 16 + blk;
      const bool act = q < nq && u < (a.K >> 5);
      qmq_load_x<T, NQ>(xr[q], act ? u : 0, static_cast<const uint16_t*>(a.x), a.K, a.M, r);
    }
    wait_vmcnt(0);    // this wave's first item and its share of the table have landed
    __syncthreads();  // ... and every other wave's share of the table
  }

  for (int t = 0; t < nitems; ++t) {
    if (nitems > 2) set_progress_prio(t);
    wait_vmcnt((issued - 1 - t) * a.cdma);  // item t has landed (vmcnt is in order)
    const int lim = min(nitems, t + a.nb);
#pragma unroll 1
    for (int k = 0; k < a.fill && issued < lim; ++k, ++issued)
      issue(issued, ring + (issued % a.nb) * a.sbuf);
    const int64_t row4 = r0 + 4 * (slot + (int64_t)t * a.slots);
    const int64_t row = min(row4 + r, a.N - 1);
    const uint32_t delta =
        (uint32_t)((reinterpret_cast<uintptr_t>(a.packed) + (uintptr_t)(row * a.row_bytes) + col0) & 15u);
    const uint8_t* b = ring + (t % a.nb) * a.sbuf;
    const uint32_t e = (uint32_t)(r * a.gran * 16) + (AL >= 1 ? (delta & ~3u) : delta);
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    if (nbk == 2 * nq) {
      // every slice of this wave holds two superblocks: every lane's group exists
#pragma unroll
      for (int q = 0; q < GL; ++q)
        if (q < nq)
          P::template dot<MR, false, AL == 2>(b, e + (uint32_t)((2 * q + (blk >> 3)) * BB), blk & 7, tbl, xr[q], acc);
    } else {
#pragma unroll
      for (int q = 0; q < GL; ++q) {
        if (q < nq) {
          const int sb = 2 * q + (blk >> 3);  // superblock of the lane's group within the piece
          const bool ok = sb < nbk;
          float part[MR];
#pragma unroll
          for (int m = 0; m < MR; ++m) part[m] = 0.f;
          P::template dot<MR, false, AL == 2>(b, e + (uint32_t)((ok ? sb : 0) * BB), blk & 7, tbl, xr[q], part);
#pragma unroll
          for (int m = 0; m < MR; ++m) acc[m] += ok ? part[m] : 0.f;
        }
      }
    }
    const int rl = (int)(row4 - r0) + r;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float v = qmq_row_sum(acc[m]);
      // sums stay in LDS until the end (a global store would count against vmcnt)
      if ((lane & 15) >= 12) red[((rl * MR + m) * a.W + ws) * 4 + (lane >> 4)] = v;
    }
  }
  __syncthreads();
  const int nout = (int)(r1 - r0) * MR;
  for (int o = tid; o < nout; o += blockDim.x) {
    float v = 0.f;
    for (int w = 0; w < 4 * a.W; ++w) v += red[o * 4 * a.W + w];
    const int rl = o / MR, m = o - rl * MR;
    if (m < a.M) store_y(a.y, a.y_dtype, (int64_t)m * a.N + r0 + rl, v);
  }
}

// ---- host side --------------------------------------------------------------------------
extern QmvTuning g_qmv_tuning;
int qmv_lds_table_bytes_of(int qt);

template <int T, int NQ, int GL, int AL>
static hipError_t launch_qmq_t(const QmvArgs& a, int grid, int threads, size_t lds, hipStream_t s) {
  auto k = qmq_kernel<T, NQ, GL, AL>;
  // a build that spills registers (some types' eight-row variants) is not run: the vector
  // kernel takes those products
  static const bool spills = [&] {
    hipFuncAttributes fa;
    return hipFuncGetAttributes(&fa, (const void*)k) != hipSuccess || fa.localSizeBytes > 0;
  }();
  if (spills) return hipErrorNotSupported;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       160 * 1024 - Qmv<T>::kLds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(k, dim3(grid), dim3(threads), lds, s, a);
  return hipGetLastError();
}

// rows 4-byte aligned: plain word reads where superblocks are a multiple of 4 bytes, else
// item-invariant funnel shifts
template <int T, int NQ, int GL>
static hipError_t launch_qmq_a4(const QmvArgs& a, bool a4, int grid, int threads, size_t lds, hipStream_t s) {
  if (a4) return launch_qmq_t<T, NQ, GL, BlockBytes<T>::v % 4 == 0 ? 2 : 1>(a, grid, threads, lds, s);
  return launch_qmq_t<T, NQ, GL, 0>(a, grid, threads, lds, s);
}

template <int T>
static hipError_t launch_qmq_type(const QmvArgs& a, int nq, int gl, bool a4, int grid, int threads, size_t lds,
                                  hipStream_t s) {
  if (nq == 1) {
    switch (gl) {
      case 1: return launch_qmq_a4<T, 1, 1>(a, a4, grid, threads, lds, s);
      case 2: return launch_qmq_a4<T, 1, 2>(a, a4, grid, threads, lds, s);
      case 3: return launch_qmq_a4<T, 1, 3>(a, a4, grid, threads, lds, s);
      case 5: return launch_qmq_a4<T, 1, 5>(a, a4, grid, threads, lds, s);
      default: return hipErrorInvalidValue;
    }
  }
  switch (gl) {
    case 1: return launch_qmq_a4<T, 2, 1>(a, a4, grid, threads, lds, s);
    case 2: return launch_qmq_a4<T, 2, 2>(a, a4, grid, threads, lds, s);
    case 3: return launch_qmq_a4<T, 2, 3>(a, a4, grid, threads, lds, s);
    default: return hipErrorInvalidValue;
  }
}

// Launch plan: one workgroup per CU, each owning a multiple of 4 consecutive rows; quad slices
// of 2 superblocks, GL per wave (2, or the fewest that let W = ceil(slices / GL) waves cover K
// within 16 waves: 3 on K = 17408), as many row slots of W waves as the variant's thread limit
// allows (16 waves for one quad and at most 2 slices per wave, else 12) and the rows keep busy,
// a ring as deep as LDS allows (at most 8 items). Returns hipErrorNotSupported for shapes or
// builds it does not take (the caller then runs the vector kernel). Measured on the 27B layer
// products (GSQ_QMQ_GL / GSQ_QMQ_WAVES override the slices and waves): 3 slices per wave were
// 2-7% slower than 2 on K = 5120 except 17408 x 5120, 5 up to 20% slower on K = 17408.
hipError_t launch_qmq(int qt, const uint8_t* packed, const void* x, void* y, int ydt, int M, int64_t N, int K,
                      const DevTables& tb, int num_cus, hipStream_t s) {
  if (M < 2 || M > 8 || (K & 255) || K < 256) return hipErrorNotSupported;
  QmvArgs a;
  std::memset(&a, 0, sizeof(a));
  a.packed = packed; a.x = x; a.y = y; a.N = N; a.K = K; a.M = M; a.x_dtype = DT_F16; a.y_dtype = ydt; a.tb = tb;
  a.qtype = qt;
  const int nq = M <= 4 ? 1 : 2;
  const int bb = block_bytes_of(qt);
  if (bb <= 0) return hipErrorInvalidValue;
  a.nblk = K / 256;
  a.row_bytes = a.nblk * bb;
  a.nslices = (a.nblk + 1) / 2;
  static const int env_gl = [] {
    const char* v = std::getenv("GSQ_QMQ_GL");
    return v ? std::atoi(v) : 0;
  }();
  static const int env_waves = [] {
    const char* v = std::getenv("GSQ_QMQ_WAVES");
    return v ? std::atoi(v) : 0;
  }();
  const int max_gl = nq == 1 ? 5 : 3;
  const int kWaves = env_waves > 0 && env_waves <= 16 ? env_waves : 16;
  int gl = env_gl > 0 ? std::min(env_gl, max_gl) : 2;
  if (gl == 4) gl = 5;
  while (gl < max_gl && (a.nslices + gl - 1) / gl > kWaves) gl = gl == 3 ? 5 : gl + 1;
  if (gl > a.nslices) gl = a.nslices;
  a.W = (a.nslices + gl - 1) / gl;
  const int max_waves = std::min(kWaves, qmq_max_threads(nq, gl) / 64);
  if (a.W > max_waves) return hipErrorNotSupported;
  a.slots = max_waves / a.W;
  int grid = num_cus;
  const int64_t quads = (N + 3) / 4;
  if (quads < grid) grid = (int)quads;
  const int64_t qpw = (quads + grid - 1) / grid;
  if (qpw * 4 > (1 << 20)) return hipErrorNotSupported;
  a.rows_per_wg = (int)(4 * qpw);
  grid = (int)((N + a.rows_per_wg - 1) / a.rows_per_wg);
  // at least ~2.5 row quads per slot: with fewer, the extra waves' start-up costs more than they
  // gain (5120 x 5120: 12 waves 5% faster than 15; 17408 x 5120: 15 waves 13% faster than 12)
  const int slot_cap = (int)std::max<int64_t>(1, (2 * qpw + 4) / 5);
  if (a.slots > slot_cap) a.slots = slot_cap;
  const int nw = a.slots * a.W;
  // row pieces: 2 GL superblocks (+15 bytes of granule alignment, +4 of decoder over-read)
  const int piece = std::min(2 * gl, a.nblk) * bb;
  a.gran = (piece + 19 + 15) / 16;
  a.cdma = (4 * a.gran + 63) / 64;
  a.sbuf = a.cdma * 1024;
  a.tbl_bytes = (qmv_lds_table_bytes_of(qt) + 15) & ~15;
  if (a.tbl_bytes > 0 && !tb.qmv_tbl) return hipErrorInvalidValue;
  a.red_off = a.tbl_bytes;
  const int red_bytes = (a.rows_per_wg * 4 * nq * a.W * 16 + 15) & ~15;
  const int lds_cap = 160 * 1024;
  // the activations in LDS (rows of 2K + 16 bytes) when a ring of two items per wave still fits
  static const int env_xlds = [] {
    const char* v = std::getenv("GSQ_QMQ_XLDS");
    return v ? std::atoi(v) : 1;
  }();
  a.x_off = a.red_off + red_bytes;
  const int x_region = M * (2 * K + 16);
  a.x_lds = env_xlds > 0 && a.x_off + x_region + 2 * nw * a.sbuf <= lds_cap ? 1 : 0;
  a.ring_off = a.x_off + (a.x_lds ? x_region : 0);
  int nb = (lds_cap - a.ring_off) / (nw * a.sbuf);
  if (nb > 8) nb = 8;
  while (nb > 2 && (nb - 2) * a.cdma > 31) --nb;  // exact vmcnt waits go up to 31
  if (nb < 2) return hipErrorNotSupported;
  a.nb = nb;
  a.fill = g_qmv_tuning.fill < 1 ? 1 : g_qmv_tuning.fill;
  const bool a4 = ((reinterpret_cast<uintptr_t>(packed) | (uintptr_t)a.row_bytes) & 3) == 0;
  const size_t lds = (size_t)a.ring_off + (size_t)nw * nb * a.sbuf - (size_t)a.tbl_bytes;  // dynamic part
  const int threads = nw * 64;
  switch (qt) {
    case Q2_K: return launch_qmq_type<Q2_K>(a, nq, gl, a4, grid, threads, lds, s);
    case Q4_K: return launch_qmq_type<Q4_K>(a, nq, gl, a4, grid, threads, lds, s);
    case Q6_K: return launch_qmq_type<Q6_K>(a, nq, gl, a4, grid, threads, lds, s);
    case IQ4_XS: return launch_qmq_type<IQ4_XS>(a, nq, gl, a4, grid, threads, lds, s);
    case IQ3_S: return launch_qmq_type<IQ3_S>(a, nq, gl, a4, grid, threads, lds, s);
    case IQ3_XXS: return launch_qmq_type<IQ3_XXS>(a, nq, gl, a4, grid, threads, lds, s);
    case IQ2_XXS: return launch_qmq_type<IQ2_XXS>(a, nq, gl, a4, grid, threads, lds, s);
    case IQ2_XS: return launch_qmq_type<IQ2_XS>(a, nq, gl, a4, grid, threads, lds, s);
    case IQ2_S: return launch_qmq_type<IQ2_S>(a, nq, gl, a4, grid, threads, lds, s);
    case IQ1_S: return launch_qmq_type<IQ1_S>(a, nq, gl, a4, grid, threads, lds, s);
    case IQ1_M: return launch_qmq_type<IQ1_M>(a, nq, gl, a4, grid, threads, lds, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gsq
