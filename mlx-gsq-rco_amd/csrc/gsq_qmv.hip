// Fused dequant + matrix-vector product (QMV): the vector kernel for up to 4 activation rows per
// launch (gsq_qmv sends batches of 3-8 fp16 rows to the quad-row kernel in gsq_qmq.hip instead),
// the per-type table images, the fused activation prologue and the two-product launch. The
// per-type decoders are in gsq_qmv_decode.h.
//
// Counterpart of the reference's per-type packed-dot kernels
// (mlx_gsq/runtime/kernels/qmv.py:76-528, dispatched by quantized_matvec qmv.py:537-576).
// Layout and arithmetic follow the decoder formulas; the schedule is gfx950-specific:
//
// * A "slice" is 8 consecutive superblocks (64 groups of 32 weights) of one row; lane l of a
//   wave decodes group l of a slice (block l/8, group l%8).
// * A wave owns up to GL consecutive slices of every row it processes (a K range, at most
//   GL*8 superblocks) and keeps their activations in registers as fp16 pairs, permuted to
//   match the type's decode pairing, with the partial sums the offset terms need. Rows with
//   more slices are split across W waves (a row slot); each wave reduces its 64 lanes with
//   DPP into LDS, and the workgroup writes its rows (summing W > 1 partials) once at the end.
// * Every wave streams its K range of consecutive rows (one "item" per row) through a
//   private LDS ring with direct-to-LDS DMA loads (global_load_lds_dwordx4), nb-1 items in
//   flight, and waits only on its own vmcnt: the main loop has no workgroup barriers, so
//   waves never wait for each other. Every item issues the same number of DMA instructions,
//   so the wait count is plain arithmetic.
// * A workgroup owns a contiguous range of rows; each row slot owns a contiguous sub-range, so
//   every wave reads long sequential spans of the packed matrix.
// * The decode turns packed bits into fp16 pairs with masks (K-quant codes as normal fp16
//   numbers: 2- and 4-bit codes in the top mantissa bits of 1.0, 6-bit codes as integers under
//   1024's exponent), byte lookups (IQ4_XS) or LDS-resident codebook entries with sign masks
//   (IQ types) and accumulates with v_dot2_f32_f16 in fp32. Per-group scales are applied once
//   per group.
// * Prologue: the type's LDS table and the activations are fetched once per workgroup (DMA),
//   behind the first weight slices of every wave.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "gsq_common.h"
#include "gsq_qmv_decode.h"

namespace gsq {

// Register weight of a variant = activation rows x slices per wave, doubled for
// split-precision (fp32/bf16) activations, which keep two fp16 parts per value. Workgroups
// shrink as the weight grows so that no variant spills: weight <= 2: 16 waves, 3 to 6: 12 waves
// (two rows of three slices fit 168 registers: 129-145 used, and 12 waves make the 17408-row
// and 17408-wide two-row products 4-32% faster than 8), 7 and more: 8 waves (16 waves of
// weight 3 measured no faster than 12).
constexpr int qmv_weight(int mr, int gl, bool xs) { return mr * gl * (xs ? 2 : 1); }
constexpr int qmv_max_threads(int w) { return w >= 7 ? 512 : (w >= 3 ? 768 : 1024); }
constexpr int kMaxRing = 16;

template <int T, int MR, bool XS>
__device__ __forceinline__ void qmv_load_x1(XReg<MR, XS, Qmv<T>::kSums>& xr, bool act, int u, const void* x, int dt,
                                            int K, int M) {
  constexpr int NS = Qmv<T>::kSums;
  using P = Qmv<T>;
  if constexpr (!XS) {
    // fp16 activations (the only input of the !XS variants): the pairs are byte permutes of
    // the loaded words and the partial sums v_dot2 against (1, 1), with no conversions
    // Lanes without a group here (act false) and rows past M load group 0 / row M - 1: their
    // decodes are discarded (the callers select 0 for them, and rows past M are not stored), so
    // no zero fill is needed.
    (void)dt;
    (void)act;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      uint32_t w[16];
      {
        const int mm = m < M ? m : M - 1;
        const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + (int64_t)mm * K + 32 * u);
        uint4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = p[k];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          w[4 * k] = v[k].x; w[4 * k + 1] = v[k].y; w[4 * k + 2] = v[k].z; w[4 * k + 3] = v[k].w;
        }
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
          for (int i = 0; i < 4; ++i) xr.s8[m][i] = s8[i];
        } else if constexpr (NS == 2) {
          xr.s8[m][0] = s8[0] + s8[1];
          xr.s8[m][1] = s8[2] + s8[3];
        } else {
          xr.s8[m][0] = (s8[0] + s8[1]) + (s8[2] + s8[3]);
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if constexpr (P::kPair == PAIR_NAT) {
          xr.h[m][i] = w[i];  // pairs (2i, 2i + 1) are the loaded words
        } else {
          int e0, e1;
          pair_idx<P::kPair>(i, e0, e1);
          xr.h[m][i] = half_pair(w, e0, e1);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float xv[32];
    load_x32(x, dt, (int64_t)m * K + 32 * u, act && m < M, xv);
    if constexpr (NS > 0) {
      float s8[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float sm = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c) sm += xv[8 * i + c];
        s8[i] = sm;
      }
      if constexpr (NS == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) xr.s8[m][i] = s8[i];
      } else if constexpr (NS == 2) {
        xr.s8[m][0] = s8[0] + s8[1];
        xr.s8[m][1] = s8[2] + s8[3];
      } else {
        xr.s8[m][0] = (s8[0] + s8[1]) + (s8[2] + s8[3]);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int e0, e1;
      pair_idx<P::kPair>(i, e0, e1);
      const _Float16 h0 = (_Float16)xv[e0], h1 = (_Float16)xv[e1];
      xr.h[m][i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
      if constexpr (XS) xr.l[m][i] = pack_h2(xv[e0] - (float)h0, xv[e1] - (float)h1);
    }
  }
}

// ---- fused activation prologue (one fp16 row, activations staged in LDS) ----------------
__device__ __forceinline__ void h8_unpack(const uint4 q, float (&f)[8]) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = h2f(w[i] & 0xFFFFu);
    f[2 * i + 1] = h2f(w[i] >> 16);
  }
}
__device__ __forceinline__ uint4 h8_pack(const float (&f)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack_h2(f[2 * i], f[2 * i + 1]);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Forms the kernel's input row in the LDS activation stage xst (K fp16 values), after the
// prologue barrier, with the same arithmetic and roundings as the separate add + RMSNorm and
// SwiGLU kernels; workgroup 0 also writes the row(s) the caller asked for. Chunk c of 8
// values belongs to the same thread in every pass, so passes need no barrier between them
// except the norm's sum. Ends with a barrier: every wave then reads its activations.
__device__ __forceinline__ void qmv_pre(const QmvArgs& a, uint8_t* xst, float* red, int tid, int nt) {
  const int nch = a.K >> 3;
  uint4* xs = reinterpret_cast<uint4*>(xst);
  const bool w0 = blockIdx.x == 0;
  if (a.pre.op == QMV_PRE_SWIGLU) {
    const uint4* gu = static_cast<const uint4*>(a.pre.a);  // gate (K values), then up (K)
    for (int c = tid; c < nch; c += nt) {
      float g[8], u[8], o[8];
      h8_unpack(gu[c], g);
      h8_unpack(gu[nch + c], u);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = g[e] / (1.f + expf(-g[e])) * u[e];
      const uint4 r = h8_pack(o);
      xs[c] = r;
      if (w0 && a.pre.out) static_cast<uint4*>(a.pre.out)[c] = r;
    }
  } else {
    const uint4* d = static_cast<const uint4*>(a.pre.a);
    const uint4* w = static_cast<const uint4*>(a.pre.w);
    const uint4 w_first = tid < nch ? w[tid] : make_uint4(0u, 0u, 0u, 0u);  // in flight during the sum
    float ss = 0.f;
    for (int c = tid; c < nch; c += nt) {
      float v[8];
      h8_unpack(xs[c], v);
      if (d) {
        float dv[8];
        h8_unpack(d[c], dv);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)(_Float16)(v[e] + dv[e]);  // stored rounded
        xs[c] = h8_pack(v);
      }
      if (w0 && a.pre.res) static_cast<uint4*>(a.pre.res)[c] = h8_pack(v);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < (nt >> 6); ++i) tot += red[i];
    const float rinv = 1.f / sqrtf(tot / (float)a.K + a.pre.eps);
    for (int c = tid; c < nch; c += nt) {
      float v[8], wv[8], o[8];
      h8_unpack(xs[c], v);
      h8_unpack(c == tid ? w_first : w[c], wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[e] * rinv * wv[e];
      const uint4 r = h8_pack(o);
      xs[c] = r;
      if (w0 && a.pre.out) static_cast<uint4*>(a.pre.out)[c] = r;
    }
  }
  __syncthreads();
}

// Convolution inputs of the workgroup's rows (kernel 4, the model's), fetched in the prologue
// into LDS (16 bytes per row: the 3 cached inputs and the 4 weights, fp16) so that the epilogue
// does not wait for memory; through LDS, not registers, which the main loop needs.
__device__ __forceinline__ void qmv_conv_prefetch(const QmvArgs& a, int64_t r, uint4& v) {
  const QmvPre& p = a.pre;
  const uint16_t* st = static_cast<const uint16_t*>(p.conv_state) + r;
  const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.conv_w) + r * 4);
  v = make_uint4((uint32_t)st[0] | ((uint32_t)st[p.conv_rows] << 16), st[2 * (int64_t)p.conv_rows], w.x, w.y);
}

// Convolution epilogue of output row r (QmvPre conv_*), after its fp16 output y was formed: the
// arithmetic of the separate GatedDeltaNet convolution kernel, for one channel. cp: the row's
// prefetched inputs, or null.
__device__ __forceinline__ void qmv_post_conv(const QmvArgs& a, int64_t r, float y, const uint4* cp) {
  const QmvPre& p = a.pre;
  const int C = p.conv_rows, K = p.conv_k;
  _Float16* st = static_cast<_Float16*>(p.conv_state) + r;
  const _Float16* w = static_cast<const _Float16*>(p.conv_w) + r * K;
  float in[8], wf[8];  // the window: K - 1 cached inputs, then the new one (static indices only)
  if (cp) {
    const uint4 c = *cp;
    in[0] = h2f(c.x & 0xFFFFu); in[1] = h2f(c.x >> 16); in[2] = h2f(c.y); in[3] = (float)(_Float16)y;
    wf[0] = h2f(c.z & 0xFFFFu); wf[1] = h2f(c.z >> 16); wf[2] = h2f(c.w & 0xFFFFu); wf[3] = h2f(c.w >> 16);
#pragma unroll
    for (int t = 4; t < 8; ++t) in[t] = wf[t] = 0.f;
  } else {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      in[t] = t < K - 1 ? (float)st[(int64_t)t * C] : (t == K - 1 ? (float)(_Float16)y : 0.f);
      wf[t] = t < K ? (float)w[t] : 0.f;
    }
  }
  float acc = in[0] * wf[0];
#pragma unroll
  for (int t = 1; t < 8; ++t)
    if (t < K) acc = acc + in[t] * wf[t];
#pragma unroll
  for (int t = 0; t + 1 < 8; ++t)
    if (t < K - 1) st[(int64_t)t * C] = (_Float16)in[t + 1];
  p.conv_out[r] = acc / (1.f + expf(-acc));
}

// PR (one fp16 activation row, K = 5120: 20 superblocks = 2.5 slices per row, one wave per
// row): the wave's items are decoded two at a time as five full slices instead of 2 x 3 with
// half of every third slice idle: slices 0 and 1 of items t and t + 1, then one slice whose
// lanes 0-31 take item t's last 4 superblocks and lanes 32-63 item t + 1's. Both rows use the
// same activations, so that slice's activations are those of groups 128 + lane % 32. Items
// stay one row each in the ring (separate buffers).
// PRE: the variant with the fused activation prologue and convolution epilogue (QmvPre; one
// fp16 row), a separate instantiation so that the plain kernels carry none of its code.
// AL: alignment of the packed rows in the ring. 0: any (2-byte aligned); 1: every item starts
// 4-byte aligned (packed and row bytes multiples of 4), so an item's offset within its 16-byte
// granule goes into the wave-uniform buffer base and each lane's offsets within the item (and
// the funnel shifts of its word reads) stay the same from item to item, computed once; 2: also
// every superblock starts 4-byte aligned (block bytes a multiple of 4): plain word reads.
// The kernel body for workgroup `bid` of the product `a`. The type's LDS table is static LDS at
// address 0 (a constant the table reads fold into their address arithmetic), or with DT the
// start of dynamic LDS (kernels over products of several types); either way the layout offsets
// of `a` count from the table's start. Both are derived from the LDS arrays here, so that every
// access through them is known to be an LDS access.
template <int T, int MR, bool XS, int GL, int AL, bool PR, bool PRE, bool DT = false>
__device__ __forceinline__ void qmv_body(const QmvArgs& a, int bid) {
  static_assert(!PRE || (MR == 1 && !XS), "the fused prologue takes one fp16 row");
  using P = Qmv<T>;
  constexpr int BB = BlockBytes<T>::v;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* tbl;
  uint8_t* dyn;
  if constexpr (DT) {
    tbl = smem;
    dyn = smem;
  } else {
    tbl = QmvTblLds<P::kLds>::get();
    dyn = smem - a.tbl_bytes;
  }
  // the wave index as a wave-uniform (scalar) value: everything derived from it (row slot,
  // item count, DMA wait counts, loop bounds) then stays in scalar registers and branches
  const int tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint8_t* xst = dyn + a.x_off;
  float* red = reinterpret_cast<float*>(dyn + a.red_off);   // [rows_per_wg][MR][W]
  uint8_t* ring = dyn + a.ring_off + wave * a.nb * a.sbuf;  // this wave's ring

  const int64_t r0 = (int64_t)bid * a.rows_per_wg;
  const int64_t r1 = min(a.N, r0 + (int64_t)a.rows_per_wg);
  // row slot of this wave and its K range (slices sl0 .. sl0 + nq - 1). Slot s takes rows
  // r0 + s, r0 + s + slots, ...: at any time the waves of a workgroup read neighbouring rows,
  // one contiguous span of the packed matrix.
  const int slot = wave / a.W, ws = wave - slot * a.W;
  const int nrow_items = (int)(r1 - r0);
  const bool live = slot < a.slots && slot < nrow_items;
  const int sl0 = ws * GL;
  const int nq = live ? max(0, min(GL, a.nslices - sl0)) : 0;
  const int nbk = min(8 * GL, a.nblk - sl0 * 8);             // superblocks per item (per row)
  const int item_bytes = nbk * BB;
  const int nitems = nq > 0 ? (nrow_items - slot + a.slots - 1) / a.slots : 0;
  // item t = K range of row r0 + slot + t * slots
  const int64_t row0 = r0 + slot;
  const uintptr_t base = reinterpret_cast<uintptr_t>(a.packed) + (uintptr_t)(row0 * a.row_bytes + (int64_t)sl0 * 8 * BB);
  const uintptr_t stride = (uintptr_t)a.row_bytes * (uintptr_t)a.slots;

  // ---- prologue: this wave's first item, then the table and the activations (once per
  // workgroup); the ring fills up gradually (below). A wave that queued its whole ring at once
  // would stall in DMA issue (the CU's memory queue is full at kernel start) before its first
  // item's decode, and would put the first items of the waves behind it back. The first item
  // goes ahead of the table and activation copies, which would otherwise delay it in that queue
  // (1024x5120 products 0.1 us faster in the graph step, ~0.5 us in back-to-back launches).
  int issued = 0;  // items issued so far (wave-uniform)
  if (nitems > 0) {
    dma_item(base, item_bytes, a.cdma, ring, lane);
    issued = 1;
  }
  if constexpr (P::kLds > 0) dma_copy(a.tb.qmv_tbl, P::kLds, tbl, wave, nw, lane);
  if (a.x_lds && !(PRE && a.pre.op == QMV_PRE_SWIGLU)) dma_copy(a.x, a.x_bytes, xst, wave, nw, lane);
  // a convolution epilogue's inputs of row r0 + tid (into LDS after the wait below)
  uint4 cpv;
  const bool cpf = PRE && a.conv_lds && tid < (int)(r1 - r0) && r0 + tid < a.pre.conv_rows;
  if (cpf) qmv_conv_prefetch(a, r0 + tid, cpv);
  wait_vmcnt(0);  // this wave's first item and its share of the table and activations have landed
  if (cpf) reinterpret_cast<uint4*>(dyn + a.conv_off)[tid] = cpv;
  __syncthreads();              // ... and every other wave's share
  if constexpr (PRE) {
    if (a.pre.op != QMV_PRE_NONE) qmv_pre(a, xst, red, tid, blockDim.x);
  }

  XReg<MR, XS, P::kSums> xr[GL];
#pragma unroll
  for (int q = 0; q < GL; ++q) {
    const int u = (PR && q == 2) ? 128 + (lane & 31) : (sl0 + q) * 64 + lane;
    const bool act = q < nq && u < (a.K >> 5);
    if (a.x_lds) qmv_load_x1<T, MR, XS>(xr[q], act, act ? u : 0, xst, a.x_dtype, a.K, a.M);
    else qmv_load_x1<T, MR, XS>(xr[q], act, act ? u : 0, a.x, a.x_dtype, a.K, a.M);
  }

  if constexpr (PR) {
    // ---- main loop, items in pairs: up to nb - 2 items in flight while a pair is decoded ----
    for (int t = 0; t < nitems; t += 2) {
      if (nitems > 2) set_progress_prio(t >> 1);
      const int np = min(2, nitems - t);
      // top the ring up to item t + nb - 1 (the buffers of items < t are consumed), at most
      // 2 fill items per pair, then wait until items t and t + 1 have landed
      const int lim = min(nitems, t + a.nb);
#pragma unroll 1
      for (int k = 0; k < 2 * a.fill && issued < lim; ++k, ++issued)
        dma_item(base + (uintptr_t)issued * stride, item_bytes, a.cdma, ring + (issued % a.nb) * a.sbuf, lane);
      wait_vmcnt((issued - t - np) * a.cdma);
      const uint32_t dA = (uint32_t)((base + (uintptr_t)t * stride) & 15u);
      const uint32_t dB = np == 2 ? (uint32_t)((base + (uintptr_t)(t + 1) * stride) & 15u) : dA;
      // AL > 0: the item offsets go into the (uniform) bases, the lane offsets are item-invariant
      const uint8_t* bA = ring + (t % a.nb) * a.sbuf + (AL ? dA : 0u);
      const uint8_t* bB = np == 2 ? ring + ((t + 1) % a.nb) * a.sbuf + (AL ? dB : 0u) : bA;
      const uint32_t eA = AL ? 0u : dA, eB = AL ? 0u : dB;
      float accA[MR], accB[MR], pt[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) { accA[m] = 0.f; accB[m] = 0.f; pt[m] = 0.f; }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t o = (uint32_t)((q * 8 + (lane >> 3)) * BB);
        P::template dot<MR, XS, AL == 2>(bA, eA + o, lane & 7, tbl, xr[q], accA);
        if (np == 2) P::template dot<MR, XS, AL == 2>(bB, eB + o, lane & 7, tbl, xr[q], accB);
      }
      const bool rowA = lane < 32;
      P::template dot<MR, XS, AL == 2>(rowA ? bA : bB, (rowA ? eA : eB) + (uint32_t)((16 + ((lane & 31) >> 3)) * BB),
                                       lane & 7, tbl, xr[2], pt);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        accA[m] += rowA ? pt[m] : 0.f;
        accB[m] += rowA ? 0.f : pt[m];
      }
      const int rl = (int)(row0 + (int64_t)t * a.slots - r0);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float vA = wave_sum_to_lane63(accA[m]);
        const float vB = wave_sum_to_lane63(accB[m]);
        if (lane == 63) {
          red[rl * MR + m] = vA;
          if (np == 2) red[(rl + a.slots) * MR + m] = vB;
        }
      }
    }
  } else {
  // ---- main loop: one item per row, up to nb-1 items in flight ----
  int buf = 0;
  for (int t = 0; t < nitems; ++t) {
    if (nitems > 2) set_progress_prio(t);
    wait_vmcnt((issued - 1 - t) * a.cdma);  // item t has landed (vmcnt is in order)
    // top the ring up to item t + nb - 1, at most two items per step (one in steady state);
    // item i goes to buffer i % nb, whose previous item (i - nb < t) has been consumed
    const int lim = min(nitems, t + a.nb);
#pragma unroll 1
    for (int k = 0; k < a.fill && issued < lim; ++k, ++issued)
      dma_item(base + (uintptr_t)issued * stride, item_bytes, a.cdma, ring + (issued % a.nb) * a.sbuf, lane);
    const int64_t row = row0 + (int64_t)t * a.slots;
    const uint32_t delta = (uint32_t)((base + (uintptr_t)t * stride) & 15u);
    const uint8_t* b = ring + buf * a.sbuf + (AL ? delta : 0u);  // AL > 0: see the paired loop
    const uint32_t e = AL ? 0u : delta;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int q = 0; q < GL; ++q) {
      if (q < nq) {
        // lane -> group (block lane/8, group lane%8) of slice sl0 + q
        const int blk = q * 8 + (lane >> 3);
        const bool ok = blk < nbk;
        float part[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) part[m] = 0.f;
        P::template dot<MR, XS, AL == 2>(b, e + (uint32_t)((ok ? blk : 0) * BB), lane & 7, tbl, xr[q], part);
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] += ok ? part[m] : 0.f;
      }
    }
    if (++buf == a.nb) buf = 0;
    const int rl = (int)(row - r0);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float v = wave_sum_to_lane63(acc[m]);
      // row sums stay in LDS until the end: a global store here would count against vmcnt
      // behind the ring's DMA and make the next item's wait also wait for the store
      if (lane == 63) red[(rl * MR + m) * a.W + ws] = v;
    }
  }
  }
  {
    __syncthreads();
    const int nout = (int)(r1 - r0) * MR;
    for (int o = tid; o < nout; o += blockDim.x) {
      float v = 0.f;
      for (int w = 0; w < a.W; ++w) v += red[o * a.W + w];
      const int rl = o / MR, m = o - rl * MR;
      if (m < a.M) store_y(a.y, a.y_dtype, (int64_t)m * a.N + r0 + rl, v);
      if constexpr (PRE) {
        if (r0 + rl < a.pre.conv_rows)
          qmv_post_conv(a, r0 + rl, v,  // row rl was prefetched by thread rl
                        a.conv_lds && rl < (int)blockDim.x ? reinterpret_cast<const uint4*>(dyn + a.conv_off) + rl
                                                           : nullptr);
      }
    }
  }
}

template <int T, int MR, bool XS, int GL, int AL, bool PR = false, bool PRE = false>
__global__ void __launch_bounds__(qmv_max_threads(qmv_weight(MR, GL, XS))) qmv_kernel(QmvArgs a) {
  qmv_body<T, MR, XS, GL, AL, PR, PRE>(a, blockIdx.x);
}

template <int T, int MR, bool XS, int GL, int AL, bool PR = false, bool PRE = false>
static hipError_t launch_qmv_t(const QmvArgs& a, int grid, int threads, size_t lds, hipStream_t s) {
  auto k = qmv_kernel<T, MR, XS, GL, AL, PR, PRE>;
  // 0: not set up; 1: ready; 2: an AL = 1 build that spills registers (its item-invariant lane
  // offsets stay live across the loop), replaced by the AL = 0 build of the same variant
  static int state = 0;
  if (!state) {
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       160 * 1024 - Qmv<T>::kLds);
    if (e != hipSuccess) return e;
    state = 1;
    if constexpr (AL == 1) {
      hipFuncAttributes fa;
      e = hipFuncGetAttributes(&fa, (const void*)k);
      if (e != hipSuccess) return e;
      if (fa.localSizeBytes > 0) state = 2;
    }
  }
  if constexpr (AL == 1) {
    if (state == 2) return launch_qmv_t<T, MR, XS, GL, 0, PR, PRE>(a, grid, threads, lds, s);
  }
  hipLaunchKernelGGL(k, dim3(grid), dim3(threads), lds, s, a);
  return hipGetLastError();
}

template <int T>
static int qmv_tbl_bytes() { return Qmv<T>::kTbl; }
template <int T>
static int qmv_lds_tbl_bytes() { return Qmv<T>::kLds; }

// Slices per wave of each variant: activation registers per lane stay near 60 (fp16, one
// activation row: 3 slices x 20) to keep 16 waves per CU resident.
static int qmv_gl(int mr, bool xs) {
  if (mr == 1) return xs ? 1 : 3;
  if (mr == 2) return 1;
  return 1;
}

template <int T, int AL>
static hipError_t launch_qmv_variant(const QmvArgs& a, int mr, bool xs, int gl, int grid, int threads, size_t lds,
                                     hipStream_t s) {
  if (a.pre.op != QMV_PRE_NONE || a.pre.conv_rows > 0) {  // one fp16 row (checked by the plan)
    if (gl == 1) return launch_qmv_t<T, 1, false, 1, AL, false, true>(a, grid, threads, lds, s);
    if (a.pair) return launch_qmv_t<T, 1, false, 3, AL, true, true>(a, grid, threads, lds, s);
    return launch_qmv_t<T, 1, false, 3, AL, false, true>(a, grid, threads, lds, s);
  }
  if (mr == 1 && !xs && gl == 1) return launch_qmv_t<T, 1, false, 1, AL>(a, grid, threads, lds, s);
  if (mr == 1 && !xs && a.pair) return launch_qmv_t<T, 1, false, 3, AL, true>(a, grid, threads, lds, s);
  if (mr == 1) return xs ? launch_qmv_t<T, 1, true, 1, AL>(a, grid, threads, lds, s) : launch_qmv_t<T, 1, false, 3, AL>(a, grid, threads, lds, s);
  if (mr == 2) {
    if (xs) return launch_qmv_t<T, 2, true, 1, AL>(a, grid, threads, lds, s);
    return gl == 3 ? launch_qmv_t<T, 2, false, 3, AL>(a, grid, threads, lds, s)
                   : launch_qmv_t<T, 2, false, 1, AL>(a, grid, threads, lds, s);
  }
  if (mr == 4 && !xs) return launch_qmv_t<T, 4, false, 1, AL>(a, grid, threads, lds, s);
  return hipErrorInvalidValue;
}

// Alignment variant (qmv_kernel AL): types whose superblock size is a multiple of 4 read their
// fields with plain dword loads when the packed matrix is 4-byte aligned (every superblock then
// is); the rest funnel-shift, with item-invariant shifts when the packed matrix and its rows
// are 4-byte aligned (an even number of superblocks per row), else per item.
template <int T>
static hipError_t launch_qmv_type(const QmvArgs& a, int mr, bool xs, int gl, int grid, int threads, size_t lds,
                                  hipStream_t s) {
  const bool rows4 = (reinterpret_cast<uintptr_t>(a.packed) & 3) == 0 && (a.row_bytes & 3) == 0;
  if constexpr (BlockBytes<T>::v % 4 == 0) {
    if ((reinterpret_cast<uintptr_t>(a.packed) & 3) == 0)
      return launch_qmv_variant<T, 2>(a, mr, xs, gl, grid, threads, lds, s);
  } else {
    if (rows4) return launch_qmv_variant<T, 1>(a, mr, xs, gl, grid, threads, lds, s);
  }
  return launch_qmv_variant<T, 0>(a, mr, xs, gl, grid, threads, lds, s);
}

int qmv_table_bytes(int qt) {
  switch (qt) {
    case Q2_K: return qmv_tbl_bytes<Q2_K>(); case Q4_K: return qmv_tbl_bytes<Q4_K>();
    case Q6_K: return qmv_tbl_bytes<Q6_K>(); case IQ4_XS: return qmv_tbl_bytes<IQ4_XS>();
    case IQ3_S: return qmv_tbl_bytes<IQ3_S>(); case IQ3_XXS: return qmv_tbl_bytes<IQ3_XXS>();
    case IQ2_XXS: return qmv_tbl_bytes<IQ2_XXS>(); case IQ2_XS: return qmv_tbl_bytes<IQ2_XS>();
    case IQ2_S: return qmv_tbl_bytes<IQ2_S>(); case IQ1_S: return qmv_tbl_bytes<IQ1_S>();
    case IQ1_M: return qmv_tbl_bytes<IQ1_M>();
    default: return -1;
  }
}

// Bytes of the table image the QMV kernel copies into LDS (a prefix of the image).
static int qmv_lds_table_bytes(int qt) {
  switch (qt) {
    case Q2_K: return qmv_lds_tbl_bytes<Q2_K>(); case Q4_K: return qmv_lds_tbl_bytes<Q4_K>();
    case Q6_K: return qmv_lds_tbl_bytes<Q6_K>(); case IQ4_XS: return qmv_lds_tbl_bytes<IQ4_XS>();
    case IQ3_S: return qmv_lds_tbl_bytes<IQ3_S>(); case IQ3_XXS: return qmv_lds_tbl_bytes<IQ3_XXS>();
    case IQ2_XXS: return qmv_lds_tbl_bytes<IQ2_XXS>(); case IQ2_XS: return qmv_lds_tbl_bytes<IQ2_XS>();
    case IQ2_S: return qmv_lds_tbl_bytes<IQ2_S>(); case IQ1_S: return qmv_lds_tbl_bytes<IQ1_S>();
    case IQ1_M: return qmv_lds_tbl_bytes<IQ1_M>();
    default: return -1;
  }
}

int qmv_lds_table_bytes_of(int qt) { return qmv_lds_table_bytes(qt); }

// Sign XOR mask for elements 2i (bit 15) and 2i+1 (bit 31) of sign byte s.
static uint32_t sign_mask_pair_host(uint32_t s, int i) {
  return (((s >> (2 * i)) & 1u) << 15) | (((s >> (2 * i + 1)) & 1u) << 31);
}

static int grid_image_bytes(int qt) {
  switch (qt) {
    case IQ1_S: case IQ1_M: return 2048 * 8 * 2;
    case IQ2_XXS: return 256 * 8 * 2;
    case IQ2_XS: return 512 * 8 * 2;
    case IQ2_S: return 1024 * 8 * 2;
    case IQ3_XXS: return 256 * 4 * 2;
    case IQ3_S: return 512 * 4 * 2;
    default: return 0;
  }
}

// fp16 bits of v if it is exact in fp16, else -1
static int32_t exact_h(float v) {
  const _Float16 h = (_Float16)v;
  return (float)h == v ? (int32_t)__builtin_bit_cast(uint16_t, h) : -1;
}

// Signed half-entry table (Qmv<IQ3_S / IQ3_XXS / IQ2_XXS>): for every entry e, group of four
// values hf (halves of an 8-value entry) and sign nibble nb, the four values with bit c of nb
// flipping the sign of value c, at fp16 index ((e * halves + hf) * 16 + nb) * 4.
static void build_signed_table(const uint16_t* grid16, int entries, int coords, uint16_t* out) {
  const int halves = coords / 4;
  for (int e = 0; e < entries; ++e)
    for (int hf = 0; hf < halves; ++hf)
      for (int nb = 0; nb < 16; ++nb)
        for (int c = 0; c < 4; ++c)
          out[((e * halves + hf) * 16 + nb) * 4 + c] =
              (uint16_t)(grid16[e * coords + 4 * hf + c] ^ (((nb >> c) & 1) ? 0x8000u : 0u));
}

// The exact LDS table image of type qt for the QMV kernel (qmv_table_bytes(qt) bytes; its first
// kLds bytes are copied into LDS): the IQ4_XS value pairs; the signed half-entry tables of IQ3_S,
// IQ3_XXS and IQ2_XXS; IQ1_M's codebook with both deltas added; the fp16 codebook of IQ1_S,
// IQ2_S and IQ2_XS, the last followed by its 16 nibble sign masks. Returns 1 when built, 0 for
// a type without a table, -1 when a value of the image is not exact in fp16.
int build_qmv_table(int qt, const uint16_t* grid16, const uint8_t* ksigns, std::vector<uint8_t>& out) {
  (void)ksigns;
  const int bytes = qmv_table_bytes(qt);
  if (bytes <= 0) return 0;
  out.assign((size_t)bytes, 0);
  uint32_t* w = reinterpret_cast<uint32_t*>(out.data());
  uint16_t* h = reinterpret_cast<uint16_t*>(out.data());
  switch (qt) {
    case IQ4_XS: {
      static const int8_t kv[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
      for (int i = 0; i < 256; ++i) {
        const _Float16 lo = (_Float16)(float)kv[i & 15], hi = (_Float16)(float)kv[i >> 4];
        w[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
      }
      return 1;
    }
    case IQ3_S: build_signed_table(grid16, 512, 4, h); return 1;
    case IQ3_XXS: build_signed_table(grid16, 256, 4, h); return 1;
    case IQ2_XXS: build_signed_table(grid16, 256, 8, h); return 1;
    case IQ1_M:
      for (int i = 0; i < 2 * 2048 * 8; ++i) {
        const float g = (float)__builtin_bit_cast(_Float16, grid16[i & (2048 * 8 - 1)]);
        const int32_t v = exact_h(g + (i < 2048 * 8 ? 0.125f : -0.125f));
        if (v < 0) return -1;
        h[i] = (uint16_t)v;
      }
      return 1;
    case IQ2_XS: {
      const int gb = grid_image_bytes(qt);
      std::memcpy(out.data(), grid16, (size_t)gb);
      uint32_t* m = reinterpret_cast<uint32_t*>(out.data() + gb);
      for (int i = 0; i < 16 * 2; ++i) m[i] = sign_mask_pair_host((uint32_t)(i >> 1), i & 1);
      return 1;
    }
    case IQ1_S: case IQ2_S:
      std::memcpy(out.data(), grid16, (size_t)grid_image_bytes(qt));
      return 1;
    default: return 0;
  }
}

// Byte size of the QMM kernels' table image of a type (their decoders' layout): the fp16
// codebook followed by 16 nibble sign masks (IQ2_S, IQ3_S, IQ3_XXS), and for IQ2_XXS / IQ2_XS
// the 128 ksigns masks of four words after those; for IQ1_S / IQ1_M the codebook with both
// deltas added (as IQ1_M's QMV image: entry i is grid[i % 2048] + (i < 2048 ? 0.125 : -0.125)).
int qmm_table_bytes(int qt) {
  switch (qt) {
    case IQ1_S: case IQ1_M: return 2 * 2048 * 8 * 2;
    case IQ2_XXS: return 256 * 8 * 2 + 16 * 8 + 128 * 16;
    case IQ2_XS: return 512 * 8 * 2 + 16 * 8 + 128 * 16;
    case IQ2_S: return 1024 * 8 * 2 + 16 * 8;
    case IQ3_XXS: return 256 * 4 * 2 + 16 * 8;
    case IQ3_S: return 512 * 4 * 2 + 16 * 8;
    default: return 0;
  }
}

// The QMM kernels' table image (qmm_table_bytes(qt) bytes); returns 1 when built, 0 for a type
// without one.
int build_qmm_table(int qt, const uint16_t* grid16, const uint8_t* ksigns, std::vector<uint8_t>& out) {
  const int bytes = qmm_table_bytes(qt);
  if (bytes <= 0) return 0;
  if (qt == IQ1_S || qt == IQ1_M) return build_qmv_table(IQ1_M, grid16, ksigns, out);  // the delta table
  out.assign((size_t)bytes, 0);
  const int gb = grid_image_bytes(qt);
  std::memcpy(out.data(), grid16, (size_t)gb);
  uint32_t* m = reinterpret_cast<uint32_t*>(out.data() + gb);
  for (int i = 0; i < 16 * 2; ++i) m[i] = sign_mask_pair_host((uint32_t)(i >> 1), i & 1);  // 16 nibble masks
  if (qt == IQ2_XXS || qt == IQ2_XS)  // then 128 ksigns masks of 4 dwords
    for (int i = 0; i < 128 * 4; ++i) m[32 + i] = sign_mask_pair_host(ksigns[i >> 2], i & 3);
  return 1;
}

static constexpr int kLdsBytes = 160 * 1024;

// Launch-plan parameters: waves per workgroup, in-flight bytes per CU the ring depth aims
// for, workgroups per CU.
// GSQ_QMV_TUNING="waves,inflight_kib,wg_per_cu,gl1_rows,gl1_waves,fill,x_lds,pair" overrides the defaults (read once, at library
// load), for measuring launch plans without a rebuild.
static QmvTuning qmv_tuning_from_env() {
  QmvTuning t = {12, 96 * 1024, 1, 5120, 15, 1, 1, 1};
  if (const char* s = std::getenv("GSQ_QMV_TUNING")) {
    // a prefix of the fields may be given; the rest keep their defaults
    int v[8] = {t.waves, t.inflight_bytes / 1024, t.wg_per_cu, t.gl1_rows, t.gl1_waves, t.fill, t.x_lds, t.pair};
    std::sscanf(s, "%d,%d,%d,%d,%d,%d,%d,%d", &v[0], &v[1], &v[2], &v[3], &v[4], &v[5], &v[6], &v[7]);
    t = {v[0], v[1] * 1024, v[2], v[3], v[4], v[5], v[6], v[7]};
  }
  return t;
}
QmvTuning g_qmv_tuning = qmv_tuning_from_env();

// Activation rows per launch: up to 4 for fp16 activations, 2 for fp32/bf16.
static int qmv_rows_per_launch(int xdt) { return xdt == DT_F16 ? 4 : 2; }

// Launch plan for up to 4 activation rows: one workgroup of nw waves per CU, each owning about
// N / #CU consecutive rows; W waves per row (ceil(slices / GL)), nw / W row slots.
// A plan computed without a launch (launch_qmv_rows with `plan`): the arguments, the slices per
// wave and the launch shape, with the table counted in the dynamic LDS size (the kernel over two
// products keeps both tables there).
struct QmvPlan {
  QmvArgs a;
  int gl, grid, threads;
  size_t lds;
};

static hipError_t launch_qmv_rows(int qt, const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int mr,
                                  int M, int64_t N, int K, const DevTables& tb, int num_cus, hipStream_t s,
                                  const QmvPre& pre = QmvPre(), QmvPlan* plan = nullptr) {
  QmvArgs a;
  a.packed = packed; a.x = x; a.y = y; a.N = N; a.K = K; a.M = M; a.x_dtype = xdt; a.y_dtype = ydt; a.tb = tb;
  a.qtype = qt;
  a.pre = pre;
  const bool has_pre = pre.op != QMV_PRE_NONE;
  if (has_pre && (M != 1 || xdt != DT_F16 || (K & 7))) return hipErrorInvalidValue;
  if (pre.conv_rows > 0 && (M != 1 || xdt != DT_F16 || ydt != DT_F16 || pre.conv_rows > N || pre.conv_k < 2 ||
                            pre.conv_k > 8))
    return hipErrorInvalidValue;
  const int bb = block_bytes_of(qt);
  a.nblk = K / 256;
  a.row_bytes = a.nblk * bb;
  a.nslices = (a.nblk + 7) / 8;
  const bool xs = xdt != DT_F16;
  int gl = qmv_gl(mr, xs);
  // one fp16 row of at most 3 slices and few rows: one slice per wave (3 waves per row). IQ1_S,
  // IQ2_XXS and IQ2_XS keep the paired three-slice plan down to 4097 rows: on 5120x5120 it is
  // 8-10% / 5% / 3% faster for them (the one-slice plan leaves half of every third slice
  // idle), while IQ4_XS and Q6_K (never paired) are 5-17% slower with it and the rest even
  const int gl1_rows = (qt == IQ1_S || qt == IQ2_XXS || qt == IQ2_XS) ? std::min(g_qmv_tuning.gl1_rows, 4096)
                                                                       : g_qmv_tuning.gl1_rows;
  const bool gl1 = !plan && mr == 1 && !xs && a.nslices <= 3 && N <= gl1_rows;
  if (gl1) gl = 1;
  // two fp16 rows: three slices per wave once a workgroup has at least 8 rows (17408 x 5120:
  // 13% faster than one slice per wave, 5120 x 17408 13%, 5120 x 5120 2-4%; with 4 rows per
  // workgroup, as on 1024 x 5120, three waves per row keep more waves busy and are 12% faster)
  if (mr == 2 && !xs && N >= 8ll * num_cus && (a.nslices + 2) / 3 <= qmv_max_threads(qmv_weight(2, 3, false)) / 64)
    gl = 3;
  a.W = (a.nslices + gl - 1) / gl;
  const int wpc = g_qmv_tuning.wg_per_cu < 1 ? 1 : g_qmv_tuning.wg_per_cu;
  const int max_waves = qmv_max_threads(qmv_weight(mr, gl, xs)) / 64;
  a.tbl_bytes = (qmv_lds_table_bytes(qt) + 15) & ~15;
  if (a.tbl_bytes > 0 && !tb.qmv_tbl) return hipErrorInvalidValue;
  const int lds_cap = kLdsBytes / wpc;
  a.x_bytes = M * K * (xdt == DT_F32 ? 4 : 2);
  // waves: as many as the variant allows (a multiple of W) unless the tuning asks for fewer
  int nw = gl1 ? g_qmv_tuning.gl1_waves : g_qmv_tuning.waves;
  if (nw < 1) nw = 1;
  if (nw > max_waves) nw = max_waves;
  if (a.W > max_waves) return hipErrorInvalidValue;
  if (nw < a.W) nw = a.W;
  a.slots = nw / a.W;
  nw = a.slots * a.W;
  int grid = num_cus * wpc;
  if (N < grid) grid = (int)N;
  a.rows_per_wg = (int)((N + grid - 1) / grid);
  grid = (int)((N + a.rows_per_wg - 1) / a.rows_per_wg);
  // item: GL slices of a row (+15 bytes of granule alignment, +4 of decoder over-read)
  const int item_bytes = (a.nblk < 8 * gl ? a.nblk : 8 * gl) * bb;
  a.cdma = (item_bytes + 19 + 1023) / 1024;
  a.sbuf = a.cdma * 1024;
  // row sums; the fused prologue also sums per wave there (16 floats)
  int red_bytes = (a.rows_per_wg * mr * a.W * 4 + 15) & ~15;
  if (has_pre && red_bytes < 64) red_bytes = 64;
  // two rows with one wave per row and fewer than two items per wave slot: a ring under three
  // items deep (even with the activations outside LDS) costs more than the extra waves gain, so
  // 8 waves (IQ3_S and Q6_K on 5120 x 5120 are 10-21% slower with 12; the 17408-row and
  // 17408-wide products 4-32% faster with 12 than with 8)
  if (mr == 2 && a.W == 1 && nw > 8 && a.rows_per_wg < 2 * nw &&
      (lds_cap - a.tbl_bytes - red_bytes) / (nw * a.sbuf) < 3) {
    nw = 8;
    a.slots = nw;
  }
  // activations go to LDS only if the ring keeps at least 3 items per wave (always with a
  // fused prologue, which forms them there)
  a.x_lds = (has_pre || (g_qmv_tuning.x_lds && a.tbl_bytes + a.x_bytes + red_bytes + nw * 3 * a.sbuf <= lds_cap))
                ? 1 : 0;
  a.x_off = a.tbl_bytes;
  a.red_off = a.x_off + (a.x_lds ? a.x_bytes : 0);
  // kernel-4 convolution epilogue: every row of a workgroup is one thread's to prefetch
  a.conv_lds = (pre.conv_rows > 0 && pre.conv_k == 4) ? 1 : 0;
  a.conv_off = a.red_off + red_bytes;
  a.ring_off = a.conv_off + (a.conv_lds ? a.rows_per_wg * 16 : 0);
  int nb = (lds_cap - a.ring_off) / (nw * a.sbuf);
  // large items: fewer waves rather than a ring of one buffer
  while (nb < 2 && nw > a.W) {
    nw -= a.W;
    a.slots = nw / a.W;
    nb = (lds_cap - a.ring_off) / (nw * a.sbuf);
  }
  // in-flight target per CU: nw * (nb - 1) items
  const int want = 1 + (g_qmv_tuning.inflight_bytes * wpc / (item_bytes > 0 ? item_bytes : 1) + nw - 1) / nw;
  if (nb > want) nb = want;
  if (nb > kMaxRing) nb = kMaxRing;
  while (nb > 2 && (nb - 2) * a.cdma > 31) --nb;  // exact vmcnt waits go up to 31
  if (nb < 2) return hipErrorInvalidValue;
  a.nb = nb;
  a.fill = g_qmv_tuning.fill < 1 ? 1 : g_qmv_tuning.fill;
  // items decoded in pairs (qmv_kernel PR): one fp16 row of 20 superblocks per wave and at least
  // three ring buffers (a pair being decoded and one in flight); every type but Q6_K, whose
  // ring is two buffers deep at 12 waves (measured on 17408x5120: IQ1_S/IQ1_M/IQ2_S/Q2_K 4-7%,
  // IQ2_XS 4%, IQ2_XXS 3%, IQ3_XXS/Q4_K/IQ3_S/IQ4_XS 1-2% faster than unpaired)
  const bool pair_type = qt != Q6_K;
  a.pair = (g_qmv_tuning.pair && pair_type && mr == 1 && !xs && gl == 3 && a.W == 1 && a.nblk == 20 && nb >= 3) ? 1 : 0;
  const int threads = nw * 64;
  const size_t lds_all = (size_t)a.ring_off + (size_t)nw * nb * a.sbuf;
  if (lds_all > (size_t)lds_cap) return hipErrorInvalidValue;
  if (plan) {
    plan->a = a;
    plan->gl = gl;
    plan->grid = grid;
    plan->threads = threads;
    plan->lds = lds_all;
    return hipSuccess;
  }
  const size_t lds = lds_all - (size_t)a.tbl_bytes;  // dynamic part: the table is static LDS
  switch (qt) {
    case Q2_K: return launch_qmv_type<Q2_K>(a, mr, xs, gl, grid, threads, lds, s);
    case Q4_K: return launch_qmv_type<Q4_K>(a, mr, xs, gl, grid, threads, lds, s);
    case Q6_K: return launch_qmv_type<Q6_K>(a, mr, xs, gl, grid, threads, lds, s);
    case IQ4_XS: return launch_qmv_type<IQ4_XS>(a, mr, xs, gl, grid, threads, lds, s);
    case IQ3_S: return launch_qmv_type<IQ3_S>(a, mr, xs, gl, grid, threads, lds, s);
    case IQ3_XXS: return launch_qmv_type<IQ3_XXS>(a, mr, xs, gl, grid, threads, lds, s);
    case IQ2_XXS: return launch_qmv_type<IQ2_XXS>(a, mr, xs, gl, grid, threads, lds, s);
    case IQ2_XS: return launch_qmv_type<IQ2_XS>(a, mr, xs, gl, grid, threads, lds, s);
    case IQ2_S: return launch_qmv_type<IQ2_S>(a, mr, xs, gl, grid, threads, lds, s);
    case IQ1_S: return launch_qmv_type<IQ1_S>(a, mr, xs, gl, grid, threads, lds, s);
    case IQ1_M: return launch_qmv_type<IQ1_M>(a, mr, xs, gl, grid, threads, lds, s);
    default: return hipErrorInvalidValue;
  }
}

// ---- two products of one activation row in one launch -----------------------------------
// Workgroups [0, g0) compute product a0, the rest product a1, each with the body of its own
// type (a switch on the type id; every type but Q6_K, which is never decoded in item pairs)
// and its own launch plan; both tables sit at the start of dynamic LDS. The alignment variant
// per type is fixed (plain word reads for superblocks of a multiple of 4 bytes, else
// item-invariant funnel shifts; IQ3_S, whose build with those spills registers, per item), so
// the launcher requires 4-byte aligned packed matrices and rows.
template <int T>
constexpr int qmv_group_al() { return BlockBytes<T>::v % 4 == 0 ? 2 : (T == IQ3_S ? 0 : 1); }

__device__ __forceinline__ void qmv_group_part(const QmvArgs& a, int bid) {
#define GSQ_QMV_GROUP_CASE(T) \
  case T: qmv_body<T, 1, false, 3, qmv_group_al<T>(), true, false, true>(a, bid); break;
  switch (a.qtype) {
    GSQ_QMV_GROUP_CASE(Q2_K) GSQ_QMV_GROUP_CASE(Q4_K) GSQ_QMV_GROUP_CASE(IQ4_XS) GSQ_QMV_GROUP_CASE(IQ3_S)
    GSQ_QMV_GROUP_CASE(IQ3_XXS) GSQ_QMV_GROUP_CASE(IQ2_XXS) GSQ_QMV_GROUP_CASE(IQ2_XS) GSQ_QMV_GROUP_CASE(IQ2_S)
    GSQ_QMV_GROUP_CASE(IQ1_S) GSQ_QMV_GROUP_CASE(IQ1_M)
    default: break;
  }
#undef GSQ_QMV_GROUP_CASE
}

__global__ void __launch_bounds__(qmv_max_threads(qmv_weight(1, 3, false))) qmv_group_kernel(QmvArgs a0, QmvArgs a1,
                                                                                             int g0) {
  if ((int)blockIdx.x < g0) qmv_group_part(a0, (int)blockIdx.x);
  else qmv_group_part(a1, (int)blockIdx.x - g0);
}

// y0 = x W0^T and y1 = x W1^T for one fp16 activation row in one launch, the CUs shared in
// proportion to the two products' expected times. hipErrorNotSupported when the two plans do not fit this
// kernel (the caller then launches the products one by one).
hipError_t launch_qmv_group2(int qt0, const uint8_t* p0, int64_t N0, void* y0, const DevTables& tb0, int qt1,
                             const uint8_t* p1, int64_t N1, void* y1, const DevTables& tb1, const void* x, int ydt,
                             int K, int num_cus, hipStream_t s) {
  if (qt0 == Q6_K || qt1 == Q6_K || num_cus < 2) return hipErrorNotSupported;
  const int64_t rb0 = (int64_t)(K / 256) * block_bytes_of(qt0), rb1 = (int64_t)(K / 256) * block_bytes_of(qt1);
  if (((reinterpret_cast<uintptr_t>(p0) | reinterpret_cast<uintptr_t>(p1)) & 3) || (rb0 & 3) || (rb1 & 3))
    return hipErrorNotSupported;
  // the CUs go in proportion to each product's expected time alone: its bytes times the type's
  // measured time per byte (us per MB on the 17408x5120 products; the decode, not the stream,
  // sets it for most types). 10% faster than a share by bytes on IQ1_M + IQ4_XS, 1.4% on
  // IQ2_XS + IQ4_XS.
  auto us_per_mb = [](int qt) {
    switch (qt) {
      case IQ1_M: return 0.58; case IQ1_S: return 0.60; case IQ2_XXS: return 0.55; case IQ2_XS: return 0.52;
      case IQ2_S: return 0.48; case IQ3_XXS: return 0.38; case IQ3_S: return 0.42; case IQ4_XS: return 0.35;
      case Q2_K: return 0.44; case Q4_K: return 0.33; default: return 0.27;
    }
  };
  const double b0 = (double)N0 * (double)rb0 * us_per_mb(qt0), b1 = (double)N1 * (double)rb1 * us_per_mb(qt1);
  int c0 = (int)(num_cus * b0 / (b0 + b1) + 0.5);
  c0 = c0 < 1 ? 1 : (c0 > num_cus - 1 ? num_cus - 1 : c0);
  // a share of few CUs for many rows can leave a plan without room (its row sums outgrow LDS):
  // the products then go one by one, each on all CUs
  QmvPlan q0, q1;
  if (launch_qmv_rows(qt0, p0, x, DT_F16, y0, ydt, 1, 1, N0, K, tb0, c0, s, QmvPre(), &q0) != hipSuccess ||
      launch_qmv_rows(qt1, p1, x, DT_F16, y1, ydt, 1, 1, N1, K, tb1, num_cus - c0, s, QmvPre(), &q1) != hipSuccess)
    return hipErrorNotSupported;
  if (q0.gl != 3 || q1.gl != 3 || !q0.a.pair || !q1.a.pair || q0.threads != q1.threads) return hipErrorNotSupported;
  hipError_t e;
  static bool attr_set = false;
  if (!attr_set) {
    e = hipFuncSetAttribute((const void*)qmv_group_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const size_t lds = q0.lds > q1.lds ? q0.lds : q1.lds;
  hipLaunchKernelGGL(qmv_group_kernel, dim3(q0.grid + q1.grid), dim3(q0.threads), lds, s, q0.a, q1.a, q0.grid);
  return hipGetLastError();
}

// Copy of `bytes` (a multiple of 16) from a 2-byte aligned src to a 16-byte aligned dst: the
// QMV kernels read activations in 16-byte pieces, so an x that is not 16-byte aligned goes
// through this copy first. One thread per 16 bytes, read as eight 2-byte pieces.
__global__ void __launch_bounds__(256) stage_copy_kernel(const uint16_t* __restrict__ src, uint4* __restrict__ dst,
                                                         int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n16) return;
  const uint16_t* p = src + 8 * i;
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = (uint32_t)p[2 * j] | ((uint32_t)p[2 * j + 1] << 16);
  dst[i] = make_uint4(w[0], w[1], w[2], w[3]);
}

hipError_t launch_stage_copy(const void* src, void* dst, int64_t bytes, hipStream_t s) {
  const int64_t n16 = bytes / 16;
  if (n16 <= 0) return hipSuccess;
  hipLaunchKernelGGL(stage_copy_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, s,
                     static_cast<const uint16_t*>(src), static_cast<uint4*>(dst), n16);
  return hipGetLastError();
}

// y[M, N] = x[M, K] W^T: activation rows go out in launches of up to 4 (2 for fp32/bf16).
// One fp16 activation row formed by a fused prologue (QmvPre) from x and the prologue's inputs.
hipError_t launch_qmv_pre(int qt, const uint8_t* packed, const void* x, void* y, int ydt, int64_t N, int K,
                          const QmvPre& pre, const DevTables& tb, int num_cus, hipStream_t s) {
  return launch_qmv_rows(qt, packed, x, DT_F16, y, ydt, 1, 1, N, K, tb, num_cus, s, pre);
}

hipError_t launch_qmq(int qt, const uint8_t* packed, const void* x, void* y, int ydt, int M, int64_t N, int K,
                      const DevTables& tb, int num_cus, hipStream_t s);

// GSQ_QMV_QUAD=0 keeps batches of 3-8 fp16 rows on the vector kernel (for measurements)
static const bool g_qmv_quad = [] {
  const char* v = std::getenv("GSQ_QMV_QUAD");
  return !(v && v[0] == '0');
}();

hipError_t launch_qmv(int qt, const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M, int64_t N,
                      int K, const DevTables& tb, int num_cus, hipStream_t s) {
  const size_t xe = xdt == DT_F32 ? 4 : 2, ye = ydt == DT_F32 ? 4 : 2;
  // fp16 rows in launches of up to 8 on the quad-row kernel (matrix-core products) while at
  // least 3 are left and it takes the shape, or 2 on matrices of 2^26+ weights with K <= 8192,
  // whose activations it stages in LDS (IQ2_S 17408x5120 at 2 rows: 15.2 us against 17.4 on the
  // vector kernel); other 1-2 row launches stay on the vector kernel, as fast or faster there
  // (5120x17408 at 2 rows: 19.6 against 20.0). GSQ_QMQ_TWO=0 keeps 2 rows on the vector kernel.
  int64_t r0 = 0;
  if (g_qmv_quad && xdt == DT_F16) {
    static const int env_min2 = [] {
      const char* v = std::getenv("GSQ_QMQ_TWO");
      return v ? std::atoi(v) : 1;
    }();
    const int min_rows = env_min2 > 0 && N * (int64_t)K >= (1ll << 26) && K <= 8192 ? 2 : 3;
    for (; M - r0 >= min_rows; r0 += 8) {
      const int mrow = (int)(M - r0 < 8 ? M - r0 : 8);
      const hipError_t e = launch_qmq(qt, packed, static_cast<const char*>(x) + r0 * K * xe, static_cast<char*>(y) +
                                      r0 * N * ye, ydt, mrow, N, K, tb, num_cus, s);
      if (e == hipErrorNotSupported) break;
      if (e != hipSuccess) return e;
    }
  }
  // rows per launch: the widest variant whose waves per row (one per GL slices) fit a workgroup
  int chunk = qmv_rows_per_launch(xdt);
  const bool xs = xdt != DT_F16;
  const int nslices = (K / 256 + 7) / 8;
  auto fits = [&](int mr) {
    const int gl = qmv_gl(mr, xs);
    return (nslices + gl - 1) / gl <= qmv_max_threads(qmv_weight(mr, gl, xs)) / 64;
  };
  while (chunk > 1 && !fits(chunk)) chunk /= 2;
  for (int64_t r = r0; r < M; r += chunk) {
    const int mrow = (int)((M - r) < chunk ? (M - r) : chunk);
    const int mr = mrow <= 1 ? 1 : (mrow <= 2 ? 2 : 4);
    const void* xr = static_cast<const char*>(x) + r * K * xe;
    void* yr = static_cast<char*>(y) + r * N * ye;
    hipError_t e = launch_qmv_rows(qt, packed, xr, xdt, yr, ydt, mr, mrow, N, K, tb, num_cus, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace gsq
