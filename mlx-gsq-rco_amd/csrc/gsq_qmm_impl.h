// Tiled quantized matrix-matrix product (QMM) for prefill: y[M,N] = x[M,K] * W[N,K]^T.
//
// Counterpart of the reference's tiled decode-once kernel
// (mlx_gsq/runtime/kernels/qmm.py:252-325, dispatched by quantized_matmul qmm.py:559-594):
// every weight is decoded once per activation tile into fp16 (the reference's decoded tile is
// half, qmm.py:181), activations are staged as fp16 (qmm.py:150-165) and products accumulate
// in fp32.
//
// gfx950 kernel (fp16 activations), one 256-thread workgroup per CU:
//  * output tile = BM activation rows x 256 weight rows; wave w owns weight rows
//    [64w, 64w + 64) and all BM rows, so its weights are private to it: the wave decodes them
//    straight into v_mfma_f32_16x16x32_f16 B operands (lane l: row l%16 of a 16-row block,
//    weights 8(l/16)..+7 of the 32-weight group) and they never pass through LDS as fp16.
//  * the wave's 64 superblocks of the current 256-wide K column sit in a private
//    two-column LDS ring, filled by global_load_lds DMA one column ahead; each row has a
//    16-byte aligned slot holding the granules that cover its (2-byte aligned) superblock.
//  * activations: a ring of `lx` K32 stages of BM x 32 fp16 shared by the four waves, filled
//    by DMA lx-1 stages ahead into a layout whose 16-byte octets are XOR-swizzled per row
//    (octet o of row m at position o ^ ((m >> 2) & 3)) so that the ds_read_b128 A-operand
//    reads of a wave are free of bank conflicts.
//  * all DMA waits are exact s_waitcnt vmcnt counts derived from the fixed issue order; one
//    s_barrier per K32 stage (per pair of stages on rings of four or more stages) guards the
//    shared activation ring.
//  * stream-K work split: the (tile, K column) iterations are divided evenly over as many
//    workgroups as there are CUs, so shapes whose tile count is not a multiple of the CU count
//    (17408 = 17 * 1024 rows) still fill the chip. A tile split between workgroups is
//    finished by the last one to arrive (per-tile arrival counter), which sums the fp32
//    partials in a fixed order (deterministic) and writes y; the workgroup holding a tile's
//    first columns keeps its own piece in registers when it finds the others already in.
//  * tiles are numbered weight tile fastest and workgroups renumbered so that consecutive work
//    (one activation tile, neighbouring weight tiles and K ranges) lands on one XCD and shares
//    its L2.
// fp32 / bf16 activations use the generic kernel below.
#pragma once
#include <cstdlib>
#include <type_traits>
#include <utility>

#include "gsq_decode.h"
#include "gsq_qmm_decode.h"

namespace gsq {

enum { QDT_F32 = 0, QDT_F16 = 1, QDT_BF16 = 2 };

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// Final outputs are not read again by the kernel, so fp32 ones are written as streaming
// (nontemporal) stores; the split-K partials, which the fix-up reads back, keep plain stores.
__device__ __forceinline__ void qmm_store_y(void* y, int dt, int64_t i, float v) {
  if (dt == QDT_F16) reinterpret_cast<_Float16*>(y)[i] = (_Float16)v;
  else if (dt == QDT_BF16) reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)f32_to_bf16_bits(v);
  else __builtin_nontemporal_store(v, reinterpret_cast<float*>(y) + i);
}

// ---- MFMA kernel ----------------------------------------------------------------------
constexpr int kQBN = 256;                   // weight rows per tile
constexpr int kQLds = 160 * 1024;

// WV waves per workgroup (4: one per SIMD, or 8: two per SIMD), each owning kQBN / WV weight
// rows of the tile.
template <int T, int WV>
struct QmmGeo {
  static constexpr int kBB = BlockBytes<T>::v;
  static constexpr int kRows = kQBN / WV;  // weight rows per wave
  static constexpr int kNB = kRows / 16;   // 16-row B blocks per wave
  // granules per row slot: enough for a superblock at any 2-byte offset (up to 14) within its
  // first granule, rounded up to an odd count so that the sixteen rows a wave reads at once
  // fall into distinct LDS bank groups (except Q6_K with 8 waves, whose rings would otherwise
  // leave no room for two activation stages of 256 rows)
  static constexpr int kNeed = (kBB + 14 + 15) / 16;
  static constexpr int kGran = (T == Q6_K && WV == 8) ? kNeed : (kNeed | 1);
  static constexpr int kSlot = kGran * 16;
  static constexpr int kGW = (kRows * kGran + 63) / 64;  // DMA instructions per column per wave
  static constexpr int kCol = kGW * 1024;                // one column of the wave's ring
  static constexpr int kRing = 2 * kCol;                 // per wave: two columns
};

// Byte size of a type's LDS table image (fp16 codebook followed by the 16 nibble sign masks,
// and for IQ2_XXS / IQ2_XS the 128 ksigns masks of four words that their decoders read; for
// IQ1_S / IQ1_M the codebook with each delta added; built by build_qmm_table in gsq_qmv.hip);
// checked against the host-built image at launch.
template <int T>
constexpr int qmm_tbl_bytes() {
  return T == IQ1_S || T == IQ1_M ? 2 * 2048 * 8 * 2
       : T == IQ2_XXS            ? 256 * 8 * 2 + 16 * 8 + 128 * 16
       : T == IQ2_XS             ? 512 * 8 * 2 + 16 * 8 + 128 * 16
       : T == IQ2_S              ? 1024 * 8 * 2 + 16 * 8
       : T == IQ3_XXS            ? 256 * 4 * 2 + 16 * 8
       : T == IQ3_S              ? 512 * 4 * 2 + 16 * 8
                                 : 0;
}

// LDS plan of (type, activation tile height MF x 16 rows, waves): table image, activation ring
// of kLx K32 stages (as deep as the LDS left over allows, up to 8), the waves' weight rings and
// a small broadcast slot.
template <int T, int MF, int WV>
struct QmmPlan {
  static constexpr int kTbl = qmm_tbl_bytes<T>();
  static constexpr int kW = WV * QmmGeo<T, WV>::kRing;
  static constexpr int kLx0 = (kQLds - kTbl - kW - 32) / (16 * MF * 64);
  static constexpr int kLx = kLx0 > 8 ? 8 : kLx0;
  static constexpr int kXOff = kTbl;
  static constexpr int kWOff = kXOff + kLx * 16 * MF * 64;
  static constexpr int kBcOff = kWOff + kW;
  static constexpr int kLds = kBcOff + 32;
  static constexpr bool kValid = kLx >= 2 && MF >= WV;  // every wave issues activation DMA
};

// The DMA schedule of one wave (per K32 stage q of Q): the table copy, then column 0 and
// activation stages 0 .. P-1; each stage issues the next activation stage (NX instructions,
// while it exists) and, at a column start, the next column (GW instructions). With one barrier
// per stage (BP false), P = LX - 1 and stage q issues activation stage q + LX - 1; it needs the
// column of stage q + 1 and activation stage q + 1 when the A operands are read one stage
// ahead (PF), else activation stage q. With one barrier per pair of stages (BP: rings of four
// or more stages), P = LX - 2 and the pair (q, q + 1), q even, issues activation stages
// q + LX - 2 and q + LX - 1 after its barrier, into the slots of stages q - 2 and q - 1, which
// every wave has finished; it needs activation stages q and q + 1 and the columns of stages
// q + 1 and q + 2. qmm_wait_n is the number of this wave's instructions that may still be in
// flight at a wait (vmcnt is in order).
constexpr int qmm_pro_x(int Q, int LX, bool BP) {
  const int p = BP ? LX - 2 : LX - 1;
  return p < Q ? p : Q;
}
constexpr int qmm_issued_before(int q, int Q, int LX, int NX, int GW, bool BP) {
  const int P = qmm_pro_x(Q, LX, BP);
  int x = 0;
  if (BP) x = (q + LX - 2 < Q ? q + LX - 2 : Q) - P;
  else x = q < Q - LX + 1 ? q : Q - LX + 1;
  const int cols = (q + 7) / 8 < Q / 8 - 1 ? (q + 7) / 8 : Q / 8 - 1;
  return GW + NX * P + NX * (x > 0 ? x : 0) + GW * cols;
}
constexpr int qmm_end_x(int k, int Q, int LX, int NX, int GW, bool BP) {
  const int P = qmm_pro_x(Q, LX, BP);
  if (k < P) return GW + NX * (k + 1);
  if (!BP) return qmm_issued_before(k - LX + 1, Q, LX, NX, GW, false) + NX;
  const int qp = 2 * ((k - LX + 2) >> 1);  // the pair that issues stage k
  return qmm_issued_before(qp, Q, LX, NX, GW, true) + NX * (k - (qp + LX - 2) + 1);
}
constexpr int qmm_end_w(int c, int Q, int LX, int NX, int GW, bool BP) {
  if (c == 0) return GW;
  const int qp = 8 * (c - 1);  // the stage (pair) that issues column c, after its activations
  const int nx = BP ? (qp + LX - 2 < Q ? 1 : 0) + (qp + LX - 1 < Q ? 1 : 0) : (qp + LX - 1 < Q ? 1 : 0);
  return qmm_issued_before(qp, Q, LX, NX, GW, BP) + NX * nx + GW;
}
constexpr int qmm_wait_n(int q, int Q, int LX, int NX, int GW, bool BP, bool PF) {
  int need = 0, wc = -1;
  if (BP) {
    need = qmm_end_x(q + 1, Q, LX, NX, GW, true);
    wc = (q + 2 < Q ? q + 2 : q + 1) >> 3;
  } else {
    need = qmm_end_x(PF && q + 1 < Q ? q + 1 : q, Q, LX, NX, GW, false);
    wc = q + 1 < Q ? (q + 1) >> 3 : -1;
  }
  if (wc >= 0) {
    const int ew = qmm_end_w(wc, Q, LX, NX, GW, BP);
    need = need > ew ? need : ew;
  }
  return qmm_issued_before(q, Q, LX, NX, GW, BP) - need;
}
// Every count the schedule produces (column counts 1..40 cover the start, steady state and
// end of any range), distinct, in descending order.
struct QmmWaitSet {
  int v[64];
  int n;
};
template <int LX, int NX, int GW, bool BP, bool PF>
constexpr QmmWaitSet qmm_wait_set() {
  QmmWaitSet w{};
  w.n = 0;
  for (int cols = 1; cols <= 40; ++cols)
    for (int q = 0; q < 8 * cols; q += BP ? 2 : 1) {
      int c = qmm_wait_n(q, 8 * cols, LX, NX, GW, BP, PF);
      if (c > 63) c = 63;
      bool seen = false;
      for (int i = 0; i < w.n; ++i) seen = seen || w.v[i] == c;
      if (!seen && w.n < 64) w.v[w.n++] = c;
    }
  for (int i = 0; i < w.n; ++i)
    for (int j = i + 1; j < w.n; ++j)
      if (w.v[j] > w.v[i]) {
        const int t = w.v[i];
        w.v[i] = w.v[j];
        w.v[j] = t;
      }
  return w;
}
template <int N>
__device__ __forceinline__ void wait_vm_imm() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
// s_waitcnt vmcnt(c) for the largest schedule count c <= n: a short chain of compile-time
// immediates, largest (steady-state) counts first
template <int LX, int NX, int GW, bool BP, bool PF, int K = 0>
__device__ __forceinline__ void qmm_wait(int n) {
  constexpr QmmWaitSet W = qmm_wait_set<LX, NX, GW, BP, PF>();
  if constexpr (K >= W.n) {
    wait_vm_imm<0>();
  } else {
    constexpr int c = W.v[K];
    if (n >= c) wait_vm_imm<c>();
    else qmm_wait<LX, NX, GW, BP, PF, K + 1>(n);
  }
}

struct QmmMfmaArgs {
  const uint8_t* packed;
  const _Float16* x;
  void* y;
  int M, N, K;
  int y_dtype;
  int nblk;              // superblocks per row (K / 256)
  long long row_bytes;
  int mt;                // activation tiles
  int nt;                // weight tiles (kQBN rows)
  int nfast;             // tile t = (activation tile t / nt, weight tile t % nt), else (t % mt, t / mt)
  int units;             // tiles * nblk
  int G;                 // workgroups
  int xcd_remap;         // G is a multiple of 8
  const uint8_t* tbl;    // the type's table image (codebook + sign masks), or null
  int tbl_bytes;         // multiple of 16
  float* part;           // 2 * G partial slots of slot_floats
  int slot_floats;       // floats per partial slot: MF * NB * 64 * WV * 4 (BM x 256)
  long long part_bytes;  // capacity of `part`
  int* cnt;              // per-tile arrival counters, indexed by the tile's first workgroup
};

// Partial tiles travel between workgroups (possibly on different XCDs, whose L2 caches are
// not coherent with each other) as whole 16-byte buffer stores written through to the
// device-coherent level (sc1) and buffer loads that bypass the caches (sc0 sc1): no L2
// write-back or invalidate of unrelated data, and full cache lines per wave instruction.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// A slot holds one workgroup's partial tile: `slot_floats` floats (the plan's tile size).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t qmm_slot_rsrc(float* part, int slot, int slot_floats) {
  return __builtin_amdgcn_make_buffer_rsrc(part + (size_t)slot * (size_t)slot_floats, 0, slot_floats * 4, 0x00020000);
}
__device__ __forceinline__ void qmm_st_coherent(__amdgpu_buffer_rsrc_t r, int off, float4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, off, 0, 16 /* sc1 */);
}
__device__ __forceinline__ float4_t qmm_ld_coherent(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 17 /* sc0 sc1 */));
}

// workgroup whose range holds column u: ranges are [floor(w*units/G), floor((w+1)*units/G))
__device__ __forceinline__ int qmm_owner(int u, int units, int G) {
  return (int)(((long long)(u + 1) * G + units - 1) / units) - 1;
}
__device__ __forceinline__ int qmm_first_col(int w, int units, int G) {
  return (int)((long long)w * units / G);
}

// A loop over 0 .. N - 1 unrolled at compile time (each index a constant): code over the
// accumulator arrays whose unrolled size exceeds the loop unroller's limits (MF x NB = 64 float4
// with 4 waves) would otherwise index them at run time, which moves the whole array to scratch
// memory (a scratch load and store around every MFMA).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int MF, int NB>
__device__ __forceinline__ void qmm_store_tile(void* y, int ydt, int M, int N, const float4_t (&acc)[MF][NB], int m0,
                                               int n0, int lane) {
  static_for<MF>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = n0 + 16 * j + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * i + 4 * (lane >> 4) + e;
        if (m < M && n < N) qmm_store_y(y, ydt, (int64_t)m * N + n, acc[i][j][e]);
      }
    }
  });
}

// One 16-row block of a wave's output (v[j][e]: row m + 4 (lane / 16) + e, column
// n0 + 16 j + lane % 16) written as whole row pieces: the wave transposes it through its own
// LDS area `st` (16 rows of 16 NB floats, row stride 16 NB + 4) and every lane stores 8
// consecutive fp32 outputs of one row with two 16-byte stores, so each row piece of 64 NB bytes
// is written whole (the accumulator layout alone gives four rows of 64 bytes per store
// instruction). The LDS operations of one wave complete in order, so the reads see the writes.
template <int NB>
__device__ __forceinline__ void qmm_store_rows_f32(float* y, int M, int N, const float4_t (&v)[NB], int m, int n0,
                                                   int lane, float* st) {
  constexpr int W = 16 * NB, S = W + 4, LPR = W / 8, RPP = 64 / LPR;
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) st[(4 * (lane >> 4) + e) * S + 16 * j + (lane & 15)] = v[j][e];
#pragma unroll
  for (int r0 = 0; r0 < 16; r0 += RPP) {
    const int r = r0 + lane / LPR, c = 8 * (lane % LPR);
    if (r < 16) {
      const float4_t a = *reinterpret_cast<const float4_t*>(st + r * S + c);
      const float4_t b = *reinterpret_cast<const float4_t*>(st + r * S + c + 4);
      const int mm = m + r, nn = n0 + c;
      if (mm < M) {
        float* yp = y + (int64_t)mm * N + nn;
        if (nn + 8 <= N) {
          __builtin_nontemporal_store(a, reinterpret_cast<float4_t*>(yp));
          __builtin_nontemporal_store(b, reinterpret_cast<float4_t*>(yp + 4));
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            if (nn + k < N) yp[k] = a[k];
            if (nn + 4 + k < N) yp[4 + k] = b[k];
          }
        }
      }
    }
  }
}

// Issues the activation stages of one workgroup in order: stage q (ring slot b) of tile t,
// column c; row[i] = this lane's source row (clamped to the matrix) and octet for DMA
// instruction i, laid out for the XOR-swizzled ring (octet o of row m at o ^ ((m >> 2) & 3)).
template <int NX, int BM, int LX>
struct QmmXIter {
  const _Float16* x;
  int M, K, mt, nt, nfast, nblk;
  int q, t, c, b;
  const _Float16* row[NX];
  __device__ __forceinline__ void rows(int wave, int lane) {
    const int m0 = (nfast ? t / nt : t % mt) * BM;
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int s = (wave * NX + i) * 64 + lane;
      const int m = s >> 2;
      const int o = (s & 3) ^ ((m >> 2) & 3);
      row[i] = x + (long long)min(m0 + m, M - 1) * K + 8 * o;
    }
  }
  __device__ __forceinline__ void init(const _Float16* x_, int M_, int K_, int mt_, int nt_, int nfast_, int nblk_, int ub,
                                       int wave, int lane) {
    x = x_;
    M = M_;
    K = K_;
    mt = mt_;
    nt = nt_;
    nfast = nfast_;
    nblk = nblk_;
    q = 0;
    b = 0;
    t = ub / nblk;
    c = ub - t * nblk;
    rows(wave, lane);
  }
  __device__ __forceinline__ void issue(uint8_t* xring, int wave, int lane) {
    const int kk = c * 256 + (q & 7) * 32;
    uint8_t* buf = xring + b * (BM * 64) + wave * NX * 1024;
#pragma unroll
    for (int i = 0; i < NX; ++i)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(row[i] + kk), (lds_ptr_t)(buf + i * 1024), 16, 0, 0);
    ++q;
    if (++b == LX) b = 0;
    if ((q & 7) == 0 && ++c == nblk) {
      c = 0;
      ++t;
      rows(wave, lane);
    }
  }
};

// The type's table image in static LDS (LDS address 0).
template <int B>
struct QmmTblLds {
  __device__ __forceinline__ static uint8_t* get() {
    __shared__ __attribute__((aligned(16))) uint8_t t[B];
    return t;
  }
};
template <>
struct QmmTblLds<0> {
  __device__ __forceinline__ static uint8_t* get() { return nullptr; }
};

template <int T, int MF, bool A4, int WV>
__global__ void __launch_bounds__(64 * WV, 1) qmm_mfma_kernel(QmmMfmaArgs args) {
  // the arguments as plain values (no reference to the argument block escapes, so it is never
  // copied to scratch memory, whose loads would wait on the DMA counter)
  const uint8_t* const packed = args.packed;
  const _Float16* const xg = args.x;
  void* const yg = args.y;
  const int M = args.M, N = args.N, K = args.K, ydt = args.y_dtype, nblk = args.nblk, mt = args.mt;
  const int nt = args.nt, nfast = args.nfast;
  auto tile_m = [&](int t) { return nfast ? t / nt : t % mt; };
  auto tile_n = [&](int t) { return nfast ? t % nt : t / mt; };
  const int units = args.units, G = args.G, xcd = args.xcd_remap, tbl_bytes = args.tbl_bytes;
  const long long row_bytes = args.row_bytes;
  const uint8_t* const tblg = args.tbl;
  float* const part = args.part;
  const int slot_floats = args.slot_floats;
  int* const cnt = args.cnt;
  using Geo = QmmGeo<T, WV>;
  constexpr int BB = Geo::kBB, GW = Geo::kGW, GR = Geo::kGran, S = Geo::kSlot;
  constexpr int RW = Geo::kRows, NB = Geo::kNB, TH = 64 * WV;
  constexpr int BM = 16 * MF, NX = MF / WV;  // NX: activation DMA instructions per wave per stage
  using Plan = QmmPlan<T, MF, WV>;
  constexpr int LX = Plan::kLx;
  static_assert(Plan::kValid, "activation ring needs two stages");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int bid = blockIdx.x;
  const int w = xcd ? (bid & 7) * (G >> 3) + (bid >> 3) : bid;
  const int ub = qmm_first_col(w, units, G), ue = qmm_first_col(w + 1, units, G);
  const int ncols = ue - ub;  // >= 1: G <= units
  const int Q = 8 * ncols;    // K32 stages of this workgroup
  constexpr int lx = LX;
  // the table image is static LDS at address 0 (its reads fold the base into their address
  // arithmetic); the plan's other offsets count from the table's start, where dynamic LDS
  // begins after the table
  uint8_t* dyn = lds - Plan::kTbl;
  uint8_t* xring = dyn + Plan::kXOff;
  uint8_t* wring = dyn + Plan::kWOff + wave * Geo::kRing;
  uint8_t* tbl = QmmTblLds<Plan::kTbl>::get();

  // the type's table image first in this wave's DMA order: the first wait covers it
  if (tbl_bytes) dma_copy(tblg, tbl_bytes, tbl, wave, WV, lane);

  // activation stages are issued in order by an iterator
  QmmXIter<NX, BM, LX> xi;
  xi.init(xg, M, K, mt, nt, nfast, nblk, ub, wave, lane);
  // weight column cl (local index): the wave's RW superblocks, granule e of the column at
  // byte 16e (row e / GR, granule e % GR of that row); granules past a row's last one reload
  // its last granule, and lanes past the last row (whole instructions) reload the last row's,
  // so every lane stays active and the count stays fixed
  auto issue_w = [&](int cl) {
    const int u = ub + cl;
    const int tile = u / nblk, c = u - tile * nblk;
    const int n0 = tile_n(tile) * kQBN + wave * RW;
    uint8_t* buf = wring + (cl & 1) * Geo::kCol;
#pragma unroll
    for (int i = 0; i < GW; ++i) {
      const int e = i * 64 + lane;
      const int r = min(e / GR, RW - 1), qg = e - (e / GR) * GR;
      const int n = min(n0 + r, N - 1);
      const uintptr_t p = reinterpret_cast<uintptr_t>(packed) + (uintptr_t)((long long)n * row_bytes) +
                          (uintptr_t)c * BB;
      const uintptr_t a0 = p & ~(uintptr_t)15;
      const int ng = (int)((p + BB + 15 - a0) >> 4);
      const uintptr_t src = a0 + (uintptr_t)(qg < ng ? qg : ng - 1) * 16;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src), (lds_ptr_t)(buf + i * 1024), 16, 0, 0);
    }
  };

  // A operands one stage ahead when the ring has a stage to spare: stage q reads stage q + 1's
  // activations while its MFMAs run on the operands read during stage q - 1
  constexpr bool PF = LX >= 3 && WV == 4;
  // one barrier per pair of stages when the ring has four or more stages (the DMA schedule
  // above; the waves drift apart by up to a stage between barriers)
  constexpr bool BP = !PF && LX >= 4;
  const int P = qmm_pro_x(Q, lx, BP);

  // B operands of stage q: the four 16-row blocks of the wave's weight rows, group q % 8 of
  // column q / 8; dl = the low address bits of the lane's four superblocks in that column
  auto decode = [&](int q, const uint32_t (&dl)[NB], half8_t (&bf)[NB]) {
    const uint8_t* wb = wring + ((q >> 3) & 1) * Geo::kCol;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      uint32_t o[4];
      QmmDec<T, A4>::run(wb + (16 * j + (lane & 15)) * S, dl[j], tbl, q & 7, lane >> 4, o);
      bf[j] = __builtin_bit_cast(half8_t, o);
    }
  };
  auto col_delta = [&](int q, uint32_t (&dl)[NB]) {
    const int u = ub + (q >> 3);
    const int tl = u / nblk, c = u - tl * nblk;
    const int n0 = tile_n(tl) * kQBN + wave * RW;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = min(n0 + 16 * j + (lane & 15), N - 1);
      dl[j] = (uint32_t)((reinterpret_cast<uintptr_t>(packed) + (uintptr_t)((long long)n * row_bytes) +
                          (uintptr_t)c * BB) & 15u);
    }
  };
  // A operands of a stage: MF 16-row blocks (row l % 16, octet l / 16, swizzled)
  const int xoff = (lane & 15) * 64 + (((lane >> 4) ^ ((lane >> 2) & 3)) << 4);
  auto load_a = [&](int slot, half8_t (&af)[MF]) {
    const uint32_t* xb = reinterpret_cast<const uint32_t*>(xring + slot * (BM * 64) + xoff);
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      const uint32_t* p = xb + i * 256;
      const uint32_t aw[4] = {p[0], p[1], p[2], p[3]};
      af[i] = __builtin_bit_cast(half8_t, aw);
    }
  };
  int* bc = reinterpret_cast<int*>(dyn + Plan::kBcOff);
  // the per-wave transpose areas of the final row stores, over the rings
  constexpr int kSt = 16 * (16 * NB + 4);  // floats per wave
  static_assert(WV * kSt * 4 <= Plan::kBcOff - Plan::kXOff, "row-store areas exceed the rings");
  float* const st = reinterpret_cast<float*>(xring) + wave * kSt;
  const bool yrows = ydt == QDT_F32 && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(yg) & 15) == 0;

  // prologue: table, column 0 and the first activation stages in flight; stage 0's weights
  issue_w(0);
  for (int q = 0; q < P; ++q) xi.issue(xring, wave, lane);
  qmm_wait<LX, NX, GW, BP, PF>(NX * (P - 1));  // table, column 0 and stage 0 (this wave's share)
  __syncthreads();
  uint32_t dl[NB];
  col_delta(0, dl);
  half8_t bcur[NB];
  decode(0, dl, bcur);
  half8_t acur[MF], anext[MF], bnext[NB];
  if constexpr (PF) load_a(0, acur);
  int rb = PF ? 1 : 0;  // ring slot of the next activations read

  // one segment = this workgroup's columns of one tile; stage q multiplies its activations
  // with weights decoded during stage q - 1 and decodes the weights of stage q + 1
  for (int q0 = 0; q0 < Q;) {
    const int u0 = ub + (q0 >> 3);
    const int tile = u0 / nblk;
    const int q1 = q0 + 8 * (min(ue, (tile + 1) * nblk) - u0);
    const int m0 = tile_m(tile) * BM, n0 = tile_n(tile) * kQBN + wave * RW;
    float4_t acc[MF][NB];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f};

    // stage q: the operands (ua, ub_) were read and decoded during stage q - 1; this stage reads
    // and decodes those of stage q + 1 into (na, nb). Two stages per iteration with the roles
    // of the register sets swapped, so no operand is copied between stages.
    auto stage = [&](int q, const half8_t (&ua)[MF], const half8_t (&ub_)[NB], half8_t (&na)[MF],
                     half8_t (&nb)[NB]) __attribute__((always_inline)) {
      const int cl = q >> 3;
      if (!BP || (q & 1) == 0) {
        // the activations read until the next wait and the columns decoded until then have
        // landed (this wave's DMAs)
        qmm_wait<LX, NX, GW, BP, PF>(qmm_wait_n(q, Q, lx, NX, GW, BP, PF));
        // every wave's DMAs of those stages are in; every wave is done with the slots of the
        // stages before them
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if constexpr (BP) {
          if (q + lx - 2 < Q) xi.issue(xring, wave, lane);
          if (q + lx - 1 < Q) xi.issue(xring, wave, lane);
        } else {
          if (q + lx - 1 < Q) xi.issue(xring, wave, lane);
        }
        if ((q & 7) == 0 && cl + 1 < ncols) issue_w(cl + 1);
      }
      // weights of stage q + 1 (after the last stage they come from stale, in-bounds LDS and
      // are not used): unconditional, in one scheduling region with the MFMAs
      if (((q + 1) & 7) == 0) col_delta(q + 1, dl);
      decode(q + 1, dl, nb);
      // LDS reads stay in this order: the decode's table reads are waited for without waiting
      // for the activation reads issued after them (LDS completes in order)
      __builtin_amdgcn_sched_barrier(0x1 | 0x2 | 0x4 | 0x8);
      // a wave issuing its MFMAs takes issue priority over the SIMD's other wave, which is
      // still decoding: the matrix pipe gets its next instruction as soon as it can take one
      // (2-4% faster at M = 512 and 2048)
      __builtin_amdgcn_s_setprio(1);
      // stage q + 1's activations (after the last stage: stale, in-bounds LDS, not used), or
      // stage q's without the lookahead
      load_a(rb, na);
      if (++rb == lx) rb = 0;
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(PF ? ua[i] : na[i], ub_[j], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);  // stages stay apart: two sets of operands at most
      __builtin_amdgcn_s_setprio(0);
    };
    // a segment is whole columns: its stage count is a multiple of 8
    for (int q = q0; q < q1; q += 2) {
      stage(q, acur, bcur, anext, bnext);
      stage(q + 1, anext, bnext, acur, bcur);
    }

    // end of this workgroup's part of `tile`
    const int wf = qmm_owner(tile * nblk, units, G);
    const int wl = qmm_owner(tile * nblk + nblk - 1, units, G);
    // after the workgroup's last stage the rings hold nothing that is still needed: fp32 rows
    // of the tile are then written whole through a per-wave LDS transpose
    const bool end_lds = yrows && q1 == Q;
    // direct: this workgroup's accumulators hold the whole tile (its only piece, or the other
    // pieces' partials added in place below)
    constexpr int CH = 8;  // output blocks per batch of partial loads
    bool direct = wf == wl;
    bool last = false;
    if (!direct) {
      // slot 2w: the tile this workgroup starts in; slot 2w + 1: the tile it ends in
      const int slot = 2 * w + (q0 == 0 ? 0 : 1);
      // the workgroup holding the tile's first columns (its range's last work, so often the
      // last to arrive) looks at the arrival count first: if every other piece is in, it stores
      // no partial and adds the others' partials to its accumulators in place, in workgroup
      // order from +0, the same sums as the memory path below (it also takes this path when
      // its own increment shows it last)
      const bool own = w == wf;
      if (tid == 0) bc[0] = own ? __hip_atomic_load(&cnt[wf], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -1;
      __syncthreads();
      last = bc[0] == wl - wf;
      if (!last) {
        const __amdgpu_buffer_rsrc_t ps = qmm_slot_rsrc(part, slot, slot_floats);
        // every store has completed (device-coherent) before the arrival count is incremented;
        // 16-row blocks wholly past M (padding rows of the last activation tile) are not stored
#pragma unroll
        for (int i = 0; i < MF; ++i)
          if (m0 + 16 * i < M) {
#pragma unroll
            for (int j = 0; j < NB; ++j) qmm_st_coherent(ps, ((i * NB + j) * TH + tid) * 16, acc[i][j]);
          }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) bc[1] = __hip_atomic_fetch_add(&cnt[wf], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        last = bc[1] == wl - wf;
      }
      if (last && own) {
#pragma unroll
        for (int i = 0; i < MF; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j) acc[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f} + acc[i][j];
        for (int v = wf + 1; v <= wl; ++v) {
          const int vs = 2 * v + (tile == qmm_first_col(v, units, G) / nblk ? 0 : 1);
          const __amdgpu_buffer_rsrc_t pv = qmm_slot_rsrc(part, vs, slot_floats);
#pragma unroll
          for (int ij0 = 0; ij0 < MF * NB; ij0 += CH) {
            if (m0 + 16 * (ij0 / NB) < M) {
              float4_t ld[CH];
#pragma unroll
              for (int t = 0; t < CH; ++t) ld[t] = qmm_ld_coherent(pv, ((ij0 + t) * TH + tid) * 16);
#pragma unroll
              for (int t = 0; t < CH; ++t) acc[(ij0 + t) / NB][(ij0 + t) % NB] += ld[t];
            }
          }
        }
        if (tid == 0) __hip_atomic_store(&cnt[wf], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        direct = true;
      }
    }
    if (direct) {
      if (end_lds) {
        __syncthreads();  // every wave is done with the rings
        static_for<MF>([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          if (m0 + 16 * i < M) qmm_store_rows_f32<NB>(static_cast<float*>(yg), M, N, acc[i], m0 + 16 * i, n0, lane, st);
        });
      } else {
        qmm_store_tile<MF, NB>(yg, ydt, M, N, acc, m0, n0, lane);
      }
    } else {
      if (last) {  // sum the partials in workgroup order
        const int mb = m0 + 4 * (lane >> 4), nb = n0 + (lane & 15);
#pragma unroll 1
        for (int ij0 = 0; ij0 < MF * NB; ij0 += CH) {
          // batches that start past M hold only padding rows, whose partials were not stored
          if (m0 + 16 * (ij0 / NB) >= M) break;
          float4_t sum[CH];
#pragma unroll
          for (int t = 0; t < CH; ++t) sum[t] = (float4_t){0.f, 0.f, 0.f, 0.f};
          for (int v = wf; v <= wl; ++v) {
            const int vs = 2 * v + (tile == qmm_first_col(v, units, G) / nblk ? 0 : 1);
            const __amdgpu_buffer_rsrc_t pv = qmm_slot_rsrc(part, vs, slot_floats);
            float4_t ld[CH];
#pragma unroll
            for (int t = 0; t < CH; ++t) ld[t] = qmm_ld_coherent(pv, ((ij0 + t) * TH + tid) * 16);
#pragma unroll
            for (int t = 0; t < CH; ++t) sum[t] += ld[t];
          }
          if (end_lds) {
#pragma unroll
            for (int a = 0; a < CH / NB; ++a) {
              const int i = ij0 / NB + a;
              float4_t v[NB];
#pragma unroll
              for (int j = 0; j < NB; ++j) v[j] = sum[a * NB + j];
              if (m0 + 16 * i < M) qmm_store_rows_f32<NB>(static_cast<float*>(yg), M, N, v, m0 + 16 * i, n0, lane, st);
            }
          } else {
#pragma unroll
            for (int t = 0; t < CH; ++t) {
              const int ij = ij0 + t;
              const int n = nb + 16 * (ij % NB);
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int m = mb + 16 * (ij / NB) + e;
                if (m < M && n < N) qmm_store_y(yg, ydt, (int64_t)m * N + n, sum[t][e]);
              }
            }
          }
        }
        if (tid == 0) __hip_atomic_store(&cnt[wf], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
    }
    q0 = q1;
  }
}

// ---- generic kernel (fp32 / bf16 activations) ------------------------------------------
// 64 x 64 output tile per 256 threads over K steps of 64: half of the threads decode 64 rows x
// two groups of weights (exact fp32 -> fp16), the other half stage the activations as fp16
// (qmm.py:160-165 converts fp32 activations to half the same way); each wave multiplies a
// 32 x 32 sub-tile with v_mfma_f32_16x16x32_f16.
constexpr int kGBM = 64, kGBN = 64, kGKS = 64, kGStride = kGKS + 8;

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

template <int T>
__global__ void __launch_bounds__(256) qmm_generic_kernel(QmmArgs a) {
  constexpr int BB = BlockBytes<T>::v;
  __shared__ __attribute__((aligned(16))) _Float16 wt[kGBN * kGStride];
  __shared__ __attribute__((aligned(16))) _Float16 xt[kGBM * kGStride];
  const int tid = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * kGBN;
  const int64_t m0 = (int64_t)blockIdx.y * kGBM;
  const int nb = a.K / 256;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;

  float4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < a.K; k0 += kGKS) {
    if (tid < 128) {
      const int r = tid >> 1, kg = tid & 1;
      const int64_t n = n0 + r;
      _Float16* dst = wt + r * kGStride + 32 * kg;
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
      _Float16* dst = xt + r * kGStride + 32 * half;
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
    for (int kk = 0; kk < kGKS; kk += 32) {
      half8_t af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const half8_t*>(xt + (wm * 32 + i * 16 + (lane & 15)) * kGStride + kk + 8 * (lane >> 4));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const half8_t*>(wt + (wn * 32 + j * 16 + (lane & 15)) * kGStride + kk + 8 * (lane >> 4));
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

}  // namespace gsq

#include "gsq_qmm_small.h"

namespace gsq {

// ---- host side --------------------------------------------------------------------------
extern QmmTuning g_qmm_tuning;

int qmm_table_bytes(int qt);  // the QMM kernels' LDS table image of a type (gsq_qmv.hip)
static bool qmm_grid_type(int qt) {
  return qt == IQ1_S || qt == IQ1_M || qt == IQ2_XXS || qt == IQ2_XS || qt == IQ2_S || qt == IQ3_XXS || qt == IQ3_S;
}

// Floats of one partial slot of the tiled kernel: every lane of the WV waves stores MF x NB
// float4 accumulators (a BM x 256 tile).
template <int T, int MF, int WV>
constexpr int qmm_slot_floats() { return MF * QmmGeo<T, WV>::kNB * 64 * WV * 4; }

template <int T, int MF, bool A4, int WV>
static hipError_t launch_mfma_t(QmmMfmaArgs a, hipStream_t s) {
  if constexpr (!QmmPlan<T, MF, WV>::kValid) {
    return hipErrorInvalidValue;
  } else {
    a.slot_floats = qmm_slot_floats<T, MF, WV>();
    if (2ll * a.G * a.slot_floats * 4 > a.part_bytes) return hipErrorInvalidValue;
    auto k = qmm_mfma_kernel<T, MF, A4, WV>;
    static bool attr_set = false;
    if (!attr_set) {
      hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         kQLds - QmmPlan<T, MF, WV>::kTbl);
      if (e != hipSuccess) return e;
      attr_set = true;
    }
    constexpr size_t lds = QmmPlan<T, MF, WV>::kLds - QmmPlan<T, MF, WV>::kTbl;  // dynamic part
    hipLaunchKernelGGL(k, dim3(a.G), dim3(64 * WV), lds, s, a);
    return hipGetLastError();
  }
}

template <int T, int MF, int WV>
static hipError_t launch_mfma_a4(const QmmMfmaArgs& a, bool a4, hipStream_t s) {
  if constexpr (BlockBytes<T>::v % 4 == 0) {
    if (a4) return launch_mfma_t<T, MF, true, WV>(a, s);
  }
  return launch_mfma_t<T, MF, false, WV>(a, s);
}
// 8 waves where the tile allows it (and the tuning does not ask for 4), else 4
template <int T, int MF>
static hipError_t launch_mfma_mf(const QmmMfmaArgs& a, bool a4, bool w8, hipStream_t s) {
  if constexpr (QmmPlan<T, MF, 8>::kValid) {
    if (w8) return launch_mfma_a4<T, MF, 8>(a, a4, s);
  }
  return launch_mfma_a4<T, MF, 4>(a, a4, s);
}

// Plan and launch the MFMA kernel for type T: activation tile height (MF 16-row blocks) from M
// (64 rows up to 64, 128 up to 128, else 256), then the stream-K grid:
// one workgroup per CU, at most one per (tile, K column) unit.
// Bytes of one partial slot of the plan launch_mfma_mf<T, mf> picks (8 waves where valid).
template <int T>
static long long qmm_slot_bytes(int mf, bool w8) {
  auto pick = [&](auto mfc) -> long long {
    constexpr int MF = decltype(mfc)::value;
    if constexpr (QmmPlan<T, MF, 8>::kValid) {
      if (w8) return 4ll * qmm_slot_floats<T, MF, 8>();
    }
    return 4ll * qmm_slot_floats<T, MF, 4>();
  };
  if (mf == 4) return pick(std::integral_constant<int, 4>{});
  if (mf == 8) return pick(std::integral_constant<int, 8>{});
  return pick(std::integral_constant<int, 16>{});
}

template <int T>
static hipError_t launch_mfma(QmmMfmaArgs& a, int num_cus, const QmmWorkspace& ws, hipStream_t s) {
  if (a.tbl_bytes != qmm_tbl_bytes<T>()) return hipErrorInvalidValue;
  int mf = g_qmm_tuning.mf;
  if (mf == 0) mf = a.M <= 64 ? 4 : (a.M <= 128 ? 8 : 16);
  if (mf != 4 && mf != 8 && mf != 16) return hipErrorInvalidValue;
  const bool a4 = (reinterpret_cast<uintptr_t>(a.packed) & 3) == 0;
  const bool w8 = g_qmm_tuning.waves != 4;
  // at least min_cols columns per workgroup: fewer workgroups share each tile when the
  // problem is small, which bounds the partial-tile traffic
  const int min_cols = g_qmm_tuning.min_cols > 0 ? g_qmm_tuning.min_cols : 2;
  for (;;) {
    const int bm = 16 * mf;
    a.mt = (a.M + bm - 1) / bm;
    a.nt = (int)((a.N + kQBN - 1) / kQBN);
    // weight tile fastest: the workgroups of one XCD (consecutive units) share an activation
    // tile in its L2 (3-6% faster at M = 2048 than activation tile fastest)
    a.nfast = g_qmm_tuning.order == 2 ? 0 : 1;
    const long long units = (long long)a.mt * a.nt * a.nblk;
    if (units >= (1ll << 31)) return hipErrorInvalidValue;
    a.units = (int)units;
    const int gmax = (a.units + min_cols - 1) / min_cols;
    a.G = num_cus < gmax ? num_cus : gmax;
    if (a.G > ws.max_groups) a.G = ws.max_groups;
    // a workspace too small for this tile height's partials at this grid: lower tiles
    if (2ll * a.G * qmm_slot_bytes<T>(mf, w8) <= ws.part_bytes) break;
    if (mf == 4) return hipErrorInvalidValue;
    mf /= 2;
  }
  a.xcd_remap = (a.G % 8 == 0) ? 1 : 0;
  a.part = ws.part;
  a.part_bytes = ws.part_bytes;
  a.cnt = ws.cnt;
  switch (mf) {
    case 4: return launch_mfma_mf<T, 4>(a, a4, w8, s);
    case 8: return launch_mfma_mf<T, 8>(a, a4, w8, s);
    default: return launch_mfma_mf<T, 16>(a, a4, w8, s);
  }
}

// Lane layout of the small-batch kernel's decode: whole groups per lane (HX) for every type but
// Q6_K and Q2_K, whose fragment decoders share few field reads between a group's octets (at
// M = 4 and 16 on 17408 / 8192 / 4096-row products: the codebook types 1-17% faster, IQ4_XS
// 2-8%, Q4_K 1-7%, Q2_K -1 to +3%, Q6_K 8-16% slower). GSQ_QMS_HX=0 / 1 sets it for every type
// (read once, for measurements).
template <int T>
constexpr bool qms_group_layout() { return T != Q6_K && T != Q2_K; }

template <int T, int WV, int NB>
static hipError_t launch_qms_a4(const QmsArgs& a, bool a4, hipStream_t s) {
  static const int env_hx = [] {
    const char* v = std::getenv("GSQ_QMS_HX");
    return v ? std::atoi(v) : -1;
  }();
  const bool hx = env_hx < 0 ? qms_group_layout<T>() : env_hx > 0;
  if constexpr (BlockBytes<T>::v % 4 == 0) {
    if (a4) return hx ? launch_qms_t<T, true, WV, NB, true>(a, s) : launch_qms_t<T, true, WV, NB, false>(a, s);
  }
  return hx ? launch_qms_t<T, false, WV, NB, true>(a, s) : launch_qms_t<T, false, WV, NB, false>(a, s);
}

// Plan and launch the small-batch kernel for type T (M <= 16): row groups of WV * 16 * NB
// rows (8 waves of 16 rows unless the tuning asks otherwise), units divided over at most one
// workgroup per CU, at least min_cols columns each.
template <int T>
static hipError_t launch_qms(QmsArgs& a, int num_cus, const QmmWorkspace& ws, hipStream_t s) {
  if (a.tbl_bytes != qmm_tbl_bytes<T>()) return hipErrorInvalidValue;
  // 16 waves of 16 rows on products of at least 2^26 weights (the 17408-row and 17408-wide 27B
  // projections: 4-10% faster than 8 waves, whose two waves per SIMD leave the decode's LDS and
  // MFMA latency exposed; the smaller products, with fewer row groups per CU, are faster with 8)
  const bool big = (long long)a.N * a.K >= (1ll << 26) && QmsPlan<T, 16, 1>::kValid;
  const int wv = g_qmm_tuning.small_waves == 4 ? 4
               : g_qmm_tuning.small_waves == 16 ? 16
               : g_qmm_tuning.small_waves == 8 ? 8 : (big ? 16 : 8);
  const int nb = g_qmm_tuning.small_nb == 2 ? 2 : (g_qmm_tuning.small_nb == 4 ? 4 : 1);
  const int rg = wv * 16 * nb;
  const long long units = (((long long)a.N + rg - 1) / rg) * a.nblk;
  if (units >= (1ll << 31)) return hipErrorInvalidValue;
  a.units = (int)units;
  const int min_cols = g_qmm_tuning.small_min_cols > 0 ? g_qmm_tuning.small_min_cols : 1;
  const int gmax = (a.units + min_cols - 1) / min_cols;
  a.G = num_cus < gmax ? num_cus : gmax;
  if (a.G > ws.max_groups) a.G = ws.max_groups;
  // the partials of G workgroups must fit the workspace (slot: NB * 64 * WV float4)
  while (a.G > 1 && 2ll * a.G * (nb * 64 * wv * 16) > ws.part_bytes) --a.G;
  a.xcd_remap = (a.G % 8 == 0) ? 1 : 0;
  a.part = ws.part;
  a.part_bytes = ws.part_bytes;
  a.cnt = ws.cnt;
  const bool a4 = (reinterpret_cast<uintptr_t>(a.packed) & 3) == 0;
  if (wv == 16) return launch_qms_a4<T, 16, 1>(a, a4, s);
  if (wv == 8)
    return nb == 4 ? launch_qms_a4<T, 8, 4>(a, a4, s) : nb == 2 ? launch_qms_a4<T, 8, 2>(a, a4, s)
                                                                 : launch_qms_a4<T, 8, 1>(a, a4, s);
  return nb == 4 ? launch_qms_a4<T, 4, 4>(a, a4, s) : nb == 2 ? launch_qms_a4<T, 4, 2>(a, a4, s)
                                                               : launch_qms_a4<T, 4, 1>(a, a4, s);
}

template <int T>
static hipError_t launch_generic_t(const QmmArgs& a, hipStream_t s) {
  dim3 grid((unsigned)((a.N + kGBN - 1) / kGBN), (unsigned)((a.M + kGBM - 1) / kGBM));
  hipLaunchKernelGGL(qmm_generic_kernel<T>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int T>
static hipError_t launch_qmm_type(const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int64_t M,
                                  int64_t N, int K, const DevTables& tb, int num_cus, const QmmWorkspace& ws,
                                  hipStream_t s) {
  const int small_max = g_qmm_tuning.small_max_m == 0 ? 16 : g_qmm_tuning.small_max_m;
  const bool x16 = (reinterpret_cast<uintptr_t>(x) & 15) == 0;  // the MFMA kernels read 16-byte pieces
  if (xdt == QDT_F16 && x16 && ws.part && M >= 1 && M <= small_max && M <= 16 && N < (1ll << 31)) {
    QmsArgs a{};
    a.packed = packed;
    a.x = static_cast<const _Float16*>(x);
    a.y = y;
    a.M = (int)M;
    a.N = (int)N;
    a.K = K;
    a.y_dtype = ydt;
    a.nblk = K / 256;
    a.row_bytes = (long long)a.nblk * BlockBytes<T>::v;
    if (qmm_grid_type(T)) {
      if (!tb.qmm_tbl) return hipErrorInvalidValue;
      a.tbl = tb.qmm_tbl;
      a.tbl_bytes = qmm_table_bytes(T);
    }
    return launch_qms<T>(a, num_cus, ws, s);
  }
  if (xdt == QDT_F16 && x16 && ws.part && M < (1ll << 31) && N < (1ll << 31)) {
    QmmMfmaArgs a{};
    a.packed = packed;
    a.x = static_cast<const _Float16*>(x);
    a.y = y;
    a.M = (int)M;
    a.N = (int)N;
    a.K = K;
    a.y_dtype = ydt;
    a.nblk = K / 256;
    a.row_bytes = (long long)a.nblk * BlockBytes<T>::v;
    if (qmm_grid_type(T)) {
      if (!tb.qmm_tbl) return hipErrorInvalidValue;
      a.tbl = tb.qmm_tbl;
      a.tbl_bytes = qmm_table_bytes(T);
    }
    return launch_mfma<T>(a, num_cus, ws, s);
  }
  QmmArgs a;
  a.packed = packed; a.x = x; a.y = y; a.M = M; a.N = N; a.K = K; a.x_dtype = xdt; a.y_dtype = ydt; a.tb = tb;
  return launch_generic_t<T>(a, s);
}

}  // namespace gsq
