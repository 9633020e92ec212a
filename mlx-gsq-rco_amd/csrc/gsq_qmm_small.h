// Small-batch quantized matrix product: y[M,N] = x[M,K] * W[N,K]^T for 1 <= M <= 16 fp16
// activation rows (the decode-batch range between the matrix-vector and the tiled kernel).
//
// Same products as the reference's quantized_matvec for small batches
// (mlx_gsq/runtime/kernels/qmv.py:537-576, which loops its vector kernel over the rows) and
// quantized_matmul (qmm.py:559-594): weights rounded to fp16 as in the tiled kernel's decoded
// tile (qmm.py:181), fp32 accumulation.
//
// The whole batch fits one 16-row MFMA operand, so the weights are decoded once per product
// and the cost is the weight stream plus its decode, nearly independent of M:
//  * work unit = (row group of WV * 16 * NB weight rows, one 256-wide K column); units are
//    divided evenly over one workgroup per CU (stream-K), rows of a group split over the waves
//    (16 * NB each, decoded straight into v_mfma_f32_16x16x32_f16 B operands);
//  * per column, the workgroup stages the 16 x 256 fp16 activation slice in LDS (each wave
//    DMAs 8 / WV of its eight 1 KB rows pairs, octet o of row m at position o ^ m so the A
//    reads of 16 rows hit distinct banks) and each wave DMAs its rows' superblocks into a
//    private ring slot; the rings are D columns deep and filled D - 1 columns ahead, with
//    exact vmcnt waits and one barrier per column (not per 32-wide stage);
//  * A operand: row m = lane % 16 of the staged slice (rows past M repeat row M - 1 and
//    their outputs are dropped); output lane l holds rows 4(l/16)..+3 of weight row l % 16;
//  * B operands, two lane layouts (HX): lane group q = lane / 16 either decodes octet q of each
//    of the superblock's 8 groups (one MFMA per group, its k-slots one group), or whole groups
//    q and q + 4 (HX, QmsGroup: a group's field reads and scale arithmetic serve its 32 weights
//    instead of 8; one MFMA per octet takes four groups, lane group q's k-slots being octets of
//    its own groups in A and B alike, with the groups' sub-scales inside the fp16 values and the
//    superblock's d on the MFMA sum);
//  * a row group split between workgroups is finished by the last to arrive, which sums
//    the fp32 partials in workgroup order (deterministic), as in the tiled kernel.
#pragma once

namespace gsq {

template <int T, int WV, int NB>
struct QmsGeo {
  static constexpr int kBB = BlockBytes<T>::v;
  static constexpr int kRows = 16 * NB;     // weight rows per wave
  static constexpr int kRG = WV * kRows;    // weight rows per row group
  static constexpr int kNeed = (kBB + 14 + 15) / 16;
  static constexpr int kGran = kNeed | 1;   // odd: the 16 rows read at once use distinct banks
  static constexpr int kSlot = kGran * 16;
  static constexpr int kGW = (kRows * kGran + 63) / 64;  // weight DMA instructions per column
  static constexpr int kWCol = kGW * 1024;
  // activation DMA instructions per column per wave (with 16 waves, waves 0-7 issue one each)
  static constexpr int kXI = WV >= 8 ? 1 : 8 / WV;
  static constexpr int kE = kGW + kXI;      // DMA instructions per column of a wave that stages activations
};

constexpr int kQmsX = 16 * 256 * 2;  // one column of activations (16 rows x 256 fp16)

template <int T, int WV, int NB>
struct QmsPlan {
  using G = QmsGeo<T, WV, NB>;
  static constexpr int kTbl = qmm_tbl_bytes<T>();
  static constexpr int kPer = kQmsX + WV * G::kWCol;  // LDS per ring column
  static constexpr int kD0 = (kQLds - kTbl - 32) / kPer;
  static constexpr int kD = kD0 > 6 ? 6 : kD0;
  static constexpr int kXOff = kTbl;
  static constexpr int kWOff = kXOff + kD * kQmsX;
  static constexpr int kBcOff = kWOff + kD * WV * G::kWCol;
  static constexpr int kLds = kBcOff + 32;
  static constexpr bool kValid = kD >= 2 && (WV == 4 || WV == 8 || WV == 16) && (kD - 2) * G::kE <= 63;
};

struct QmsArgs {
  const uint8_t* packed;
  const _Float16* x;
  void* y;
  int M, N, K;
  int y_dtype;
  int nblk;            // superblocks per row (K / 256)
  long long row_bytes;
  int units;           // row groups * nblk
  int G;               // workgroups
  int xcd_remap;       // G is a multiple of 8
  const uint8_t* tbl;  // the type's table image, or null
  int tbl_bytes;
  float* part;         // 2 * G partial slots of slot_floats
  int slot_floats;     // floats per partial slot: NB * 64 * WV * 4
  long long part_bytes;  // capacity of `part`
  int* cnt;            // arrival counters, indexed by a group's first workgroup
};

// one workgroup per CU (LDS-bound): WV / 4 waves per SIMD, which the register allocation and
// the scheduler may assume (latency hiding by independent work within the wave)
template <int T, bool A4, int WV, int NB, bool HX>
__global__ void __launch_bounds__(64 * WV, 1) __attribute__((amdgpu_waves_per_eu(WV / 4, WV / 4)))
qms_kernel(QmsArgs args) {
  const uint8_t* const packed = args.packed;
  const _Float16* const xg = args.x;
  void* const yg = args.y;
  const int M = args.M, N = args.N, K = args.K, ydt = args.y_dtype, nblk = args.nblk;
  const int units = args.units, G = args.G, xcd = args.xcd_remap, tbl_bytes = args.tbl_bytes;
  const long long row_bytes = args.row_bytes;
  const uint8_t* const tblg = args.tbl;
  float* const part = args.part;
  const int slot_floats = args.slot_floats;
  int* const cnt = args.cnt;
  using Geo = QmsGeo<T, WV, NB>;
  using Plan = QmsPlan<T, WV, NB>;
  constexpr int BB = Geo::kBB, GW = Geo::kGW, GR = Geo::kGran, S = Geo::kSlot, RW = Geo::kRows;
  constexpr int XI = Geo::kXI, D = Plan::kD, TH = 64 * WV;
  static_assert(Plan::kValid, "ring needs two columns");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bid = blockIdx.x;
  const int w = xcd ? (bid & 7) * (G >> 3) + (bid >> 3) : bid;
  const int ub = qmm_first_col(w, units, G), ue = qmm_first_col(w + 1, units, G);
  const int ncols = ue - ub;  // >= 1: G <= units
  uint8_t* dyn = lds - Plan::kTbl;
  uint8_t* xring = dyn + Plan::kXOff;
  uint8_t* wring = dyn + Plan::kWOff + wave * (D * Geo::kWCol);
  uint8_t* tbl = QmmTblLds<Plan::kTbl>::get();

  if (tbl_bytes) dma_copy(tblg, tbl_bytes, tbl, wave, WV, lane);

  // activation DMA sources of this lane: instruction i of this wave fills 1 KB (rows 2j, 2j+1)
  // of a column slot; lane -> row m, slot position p, source octet p ^ m
  const bool xw = wave < 8;  // this wave stages activations (every wave unless there are 16)
  const int E = Geo::kGW + (xw ? XI : 0);  // its DMA instructions per column
  const _Float16* xsrc[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int j = wave * XI + i;
    const int m = 2 * j + (lane >> 5), p = lane & 31;
    xsrc[i] = xg + (long long)min(m, M - 1) * K + 8 * (p ^ m);
  }
  auto issue = [&](int cl) {
    const int u = ub + cl;
    const int grp = u / nblk, c = u - grp * nblk;
    const int slot = cl % D;
    uint8_t* xb = xring + slot * kQmsX + wave * XI * 1024;
    if (xw) {
#pragma unroll
      for (int i = 0; i < XI; ++i)
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(xsrc[i] + c * 256), (lds_ptr_t)(xb + i * 1024), 16, 0, 0);
    }
    const int n0 = grp * Geo::kRG + wave * RW;
    uint8_t* wb = wring + slot * Geo::kWCol;
#pragma unroll
    for (int i = 0; i < GW; ++i) {
      const int e = i * 64 + lane;
      const int r = min(e / GR, RW - 1), qg = e - (e / GR) * GR;
      const int n = min(n0 + r, N - 1);
      const uintptr_t p = reinterpret_cast<uintptr_t>(packed) + (uintptr_t)((long long)n * row_bytes) + (uintptr_t)c * BB;
      const uintptr_t a0 = p & ~(uintptr_t)15;
      const int ng = (int)((p + BB + 15 - a0) >> 4);
      const uintptr_t src = a0 + (uintptr_t)(qg < ng ? qg : ng - 1) * 16;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src), (lds_ptr_t)(wb + i * 1024), 16, 0, 0);
    }
  };
  int* bc = reinterpret_cast<int*>(dyn + Plan::kBcOff);

  // prologue: columns 0 .. D-2 in flight
  const int pre = min(D - 1, ncols);
  for (int cl = 0; cl < pre; ++cl) issue(cl);

  // A operand offset of this lane in a column slot: row m = lane % 16, octet 4g + lane / 16
  const int am = lane & 15, aq = lane >> 4;
  float4_t acc[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) acc[j] = (float4_t){0.f, 0.f, 0.f, 0.f};

  for (int cl = 0; cl < ncols; ++cl) {
    // this wave's DMAs of column cl have landed (columns after it may still be in flight)
    wait_vmcnt((min(cl + D - 2, ncols - 1) - cl) * E);
    // every wave's share of column cl is in; every wave is done with column cl - 1's slot
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (cl + D - 1 < ncols) issue(cl + D - 1);
    const int u = ub + cl;
    const int grp = u / nblk, c = u - grp * nblk;
    const int n0 = grp * Geo::kRG + wave * RW;
    const int slot = cl % D;
    const uint8_t* xb = xring + slot * kQmsX + am * 512;
    const uint8_t* wb = wring + slot * Geo::kWCol;
    uint32_t dl[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = min(n0 + 16 * j + am, N - 1);
      dl[j] = (uint32_t)((reinterpret_cast<uintptr_t>(packed) + (uintptr_t)((long long)n * row_bytes) +
                          (uintptr_t)c * BB) & 15u);
    }
    if constexpr (HX) {
      // group layout: lane group aq decodes whole groups aq and aq + 4 of its row (the field
      // reads serve 32 weights); the MFMA's k-slots of lane group aq are octets of those groups
      // in A and B alike, so one MFMA takes four groups of a superblock
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        half8_t af[4];
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          const uint32_t* ap = reinterpret_cast<const uint32_t*>(xb + (((4 * (aq + 4 * h) + f) ^ am) << 4));
          const uint32_t aw[4] = {ap[0], ap[1], ap[2], ap[3]};
          af[f] = __builtin_bit_cast(half8_t, aw);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const uint8_t* rb = wb + (16 * j + am) * S;
          uint32_t o[4][4];
          if constexpr (QmsGroup<T, A4>::kOn) {
            const float d = QmsGroup<T, A4>::run(rb, dl[j], tbl, aq + 4 * h, o);
            float4_t t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int f = 0; f < 4; ++f)
              t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[f], __builtin_bit_cast(half8_t, o[f]), t, 0, 0, 0);
            acc[j] += d * t;
          } else {
#pragma unroll
            for (int f = 0; f < 4; ++f) QmmDec<T, A4>::run(rb, dl[j], tbl, aq + 4 * h, f, o[f]);
#pragma unroll
            for (int f = 0; f < 4; ++f)
              acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[f], __builtin_bit_cast(half8_t, o[f]), acc[j], 0, 0, 0);
          }
        }
      }
    } else {
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const uint32_t* ap = reinterpret_cast<const uint32_t*>(xb + (((4 * g + aq) ^ am) << 4));
      const uint32_t aw[4] = {ap[0], ap[1], ap[2], ap[3]};
      const half8_t af = __builtin_bit_cast(half8_t, aw);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        uint32_t o[4];
        if constexpr (QmsRaw<T, A4>::kOn) {
          // raw values into a fresh accumulator, scaled once per group
          const float sc = QmsRaw<T, A4>::run(wb + (16 * j + am) * S, dl[j], tbl, g, aq, o);
          const float4_t t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, __builtin_bit_cast(half8_t, o),
                                                                    (float4_t){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          acc[j] += sc * t;
        } else {
          QmmDec<T, A4>::run(wb + (16 * j + am) * S, dl[j], tbl, g, aq, o);
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, __builtin_bit_cast(half8_t, o), acc[j], 0, 0, 0);
        }
      }
    }
    }

    if (c != nblk - 1 && cl != ncols - 1) continue;
    // end of this workgroup's part of row group grp
    const int wf = qmm_owner(grp * nblk, units, G);
    const int wl = qmm_owner(grp * nblk + nblk - 1, units, G);
    const int mb = 4 * aq;
    if (wf == wl) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int n = n0 + 16 * j + am;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (mb + e < M && n < N) qmm_store_y(yg, ydt, (int64_t)(mb + e) * N + n, acc[j][e]);
      }
    } else {
      const int slotp = 2 * w + (grp == ub / nblk ? 0 : 1);  // first group of this workgroup: slot 2w
      const __amdgpu_buffer_rsrc_t ps = qmm_slot_rsrc(part, slotp, slot_floats);
#pragma unroll
      for (int j = 0; j < NB; ++j) qmm_st_coherent(ps, (j * TH + tid) * 16, acc[j]);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) bc[0] = __hip_atomic_fetch_add(&cnt[wf], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      if (bc[0] == wl - wf) {  // last to arrive: sum the partials in workgroup order
        float4_t sum[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) sum[j] = (float4_t){0.f, 0.f, 0.f, 0.f};
        // workgroups after wf start inside this group (their slot 2v); wf may have started in
        // an earlier one. Four workgroups' loads in flight at a time, summed in order.
        const int s0 = 2 * wf + (qmm_first_col(wf, units, G) / nblk == grp ? 0 : 1);
        int v = wf;
        for (; v + 3 <= wl; v += 4) {
          float4_t ld[4][NB];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const __amdgpu_buffer_rsrc_t pv = qmm_slot_rsrc(part, v + t == wf ? s0 : 2 * (v + t), slot_floats);
#pragma unroll
            for (int j = 0; j < NB; ++j) ld[t][j] = qmm_ld_coherent(pv, (j * TH + tid) * 16);
          }
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int j = 0; j < NB; ++j) sum[j] += ld[t][j];
        }
        for (; v <= wl; ++v) {
          const __amdgpu_buffer_rsrc_t pv = qmm_slot_rsrc(part, v == wf ? s0 : 2 * v, slot_floats);
#pragma unroll
          for (int j = 0; j < NB; ++j) sum[j] += qmm_ld_coherent(pv, (j * TH + tid) * 16);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int n = n0 + 16 * j + am;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (mb + e < M && n < N) qmm_store_y(yg, ydt, (int64_t)(mb + e) * N + n, sum[j][e]);
        }
        if (tid == 0) __hip_atomic_store(&cnt[wf], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = (float4_t){0.f, 0.f, 0.f, 0.f};
  }
}

template <int T, bool A4, int WV, int NB, bool HX>
static hipError_t launch_qms_t(QmsArgs a, hipStream_t s) {
  if constexpr (!QmsPlan<T, WV, NB>::kValid) {
    return hipErrorInvalidValue;
  } else {
    a.slot_floats = NB * 64 * WV * 4;  // every lane stores NB float4 accumulators
    if (2ll * a.G * a.slot_floats * 4 > a.part_bytes) return hipErrorInvalidValue;
    auto k = qms_kernel<T, A4, WV, NB, HX>;
    static bool attr_set = false;
    if (!attr_set) {
      hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         kQLds - QmsPlan<T, WV, NB>::kTbl);
      if (e != hipSuccess) return e;
      attr_set = true;
    }
    constexpr size_t lds = QmsPlan<T, WV, NB>::kLds - QmsPlan<T, WV, NB>::kTbl;
    hipLaunchKernelGGL(k, dim3(a.G), dim3(64 * WV), lds, s, a);
    return hipGetLastError();
  }
}

}  // namespace gsq
