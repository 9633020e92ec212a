// Fused dequant + matrix-vector product (QMV) for M <= 4 activation rows.
//
// Counterpart of the reference's per-type packed-dot kernels
// (mlx_gsq/runtime/kernels/qmv.py:76-528, dispatched by quantized_matvec qmv.py:537-576).
// Layout and arithmetic follow the decoder formulas; the schedule is gfx950-specific:
//
// * A workgroup owns a contiguous range of whole weight rows, i.e. one contiguous byte range
//   of the packed matrix, and streams it through LDS with direct-to-LDS DMA loads
//   (global_load_lds_dwordx4), J rows per step, double buffered. Streams of whole rows keep
//   HBM accesses long and sequential.
// * Lane u of the workgroup owns 32-weight group u of every row (K/32 lanes). Its 32
//   activations stay in registers for the whole kernel as fp16 pairs, permuted to match
//   the type's decode pairing, with per-8 sums for the offset terms.
// * The decode turns packed bits into fp16 pairs with magic-number ORs (K-quants), byte
//   lookups (IQ4_XS) or LDS-resident codebook entries with sign masks (IQ types) and
//   accumulates with v_dot2_f32_f16 in fp32. Per-group scales are applied once per group.
// * Per step, lane partials are reduced through LDS and written as y.
#include "gsq_common.h"

namespace gsq {

struct QmvArgs {
  const uint8_t* packed;
  const void* x;
  void* y;
  int64_t N;
  int64_t total_bytes;
  int K, M, x_dtype, y_dtype;
  int rows_per_wg, J, row_bytes, buf_bytes, tbl_bytes;
  DevTables tb;
};

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };
constexpr int kJMax = 8;
constexpr int kQmvMaxThreads = 576;  // K <= 18432

// ---- activation pairing ------------------------------------------------------------
enum Pairing { PAIR_NAT = 0, PAIR_K = 1, PAIR_16 = 2 };

template <int PR>
__device__ __forceinline__ void pair_idx(int i, int& a, int& b) {
  if (PR == PAIR_NAT) { a = 2 * i; b = 2 * i + 1; }
  else if (PR == PAIR_K) { int k = i >> 1; a = 4 * k + (i & 1); b = a + 2; }
  else { a = i; b = i + 16; }
}

template <int MR, bool XS>
struct XReg {
  uint32_t h[MR][16];
  uint32_t l[MR][XS ? 16 : 1];
  float s8[MR][4];  // sums of elements 8i..8i+7
};

template <int MR, bool XS>
__device__ __forceinline__ void dacc(uint32_t w, const XReg<MR, XS>& x, int i, float (&acc)[MR]) {
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    acc[m] = dot2(w, x.h[m][i], acc[m]);
    if constexpr (XS) acc[m] = dot2(w, x.l[m][i], acc[m]);
  }
}

// (C + q, C + q') as an fp16 pair -> (q, q') exactly (one v_pk_add_f16). The magic-number
// decode yields fp16 values 1024 + code; removing the offset before the dot keeps the fp32
// sums free of cancellation.
template <int C>
__device__ __forceinline__ uint32_t sub_magic(uint32_t v) {
  const half2_t r = __builtin_bit_cast(half2_t, v) - (half2_t){(_Float16)(float)C, (_Float16)(float)C};
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint32_t sub_magic1024(uint32_t v) { return sub_magic<1024>(v); }

// ---- per-type decode + dot -----------------------------------------------------------
template <int T> struct Qmv;

template <> struct Qmv<Q4_K> {
  static constexpr int kPair = PAIR_K;
  static constexpr int kTbl = 0;
  __device__ static void load_tables(uint8_t*, const DevTables&, int, int) {}
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t*, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    uint32_t h[4];
    lds_words<4>(buf, off, h);
    const float d = h2f(h[0] & 0xFFFFu), dmin = h2f(h[0] >> 16);
    const uint32_t j8 = 8u * (g & 3);
    const uint32_t A = bfe(h[1], j8, 8), B = bfe(h[2], j8, 8), C = bfe(h[3], j8, 8);
    uint32_t sc, mn;
    if (g < 4) { sc = A & 63u; mn = B & 63u; }
    else { sc = (C & 15u) | ((A >> 6) << 4); mn = (C >> 4) | ((B >> 6) << 4); }
    uint32_t q[8];
    lds_words<8>(buf, off + 16 + 32 * (g >> 1), q);
    const uint32_t sh = 4u * (g & 1);
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      uint32_t v = q[k] >> sh;
      dacc<MR, XS>(sub_magic1024((v & 0x000F000Fu) | 0x64006400u), x, 2 * k, acc);
      dacc<MR, XS>(sub_magic1024(((v >> 8) & 0x000F000Fu) | 0x64006400u), x, 2 * k + 1, acc);
    }
    const float s = d * (float)sc;
    const float o = -(dmin * (float)mn);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float xs = (x.s8[m][0] + x.s8[m][1]) + (x.s8[m][2] + x.s8[m][3]);
      out[m] += s * acc[m] + o * xs;
    }
  }
};

template <> struct Qmv<Q2_K> {
  static constexpr int kPair = PAIR_K;
  static constexpr int kTbl = 0;
  __device__ static void load_tables(uint8_t*, const DevTables&, int, int) {}
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t*, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    const uint32_t sm = lds_u16(buf, off + 2 * g);
    const uint32_t dd = lds_w32(buf, off + 80);
    const float d = h2f(dd & 0xFFFFu), dmin = h2f(dd >> 16);
    uint32_t q[8];
    lds_words<8>(buf, off + 16 + 32 * (g >> 2), q);
    const uint32_t sh = 2u * (g & 3);
    float a0[MR], a1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) { a0[m] = 0.f; a1[m] = 0.f; }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      // 2-bit values are small next to the 1024 magic offset: remove it exactly in fp16
      // before the dot so the fp32 sums carry no cancellation.
      uint32_t v = q[k] >> sh;
      const uint32_t A = sub_magic1024((v & 0x00030003u) | 0x64006400u);
      const uint32_t B = sub_magic1024(((v >> 8) & 0x00030003u) | 0x64006400u);
      if (k < 4) { dacc<MR, XS>(A, x, 2 * k, a0); dacc<MR, XS>(B, x, 2 * k + 1, a0); }
      else { dacc<MR, XS>(A, x, 2 * k, a1); dacc<MR, XS>(B, x, 2 * k + 1, a1); }
    }
    const float s0 = d * (float)(sm & 15u), s1 = d * (float)((sm >> 8) & 15u);
    const float o0 = -(dmin * (float)((sm >> 4) & 15u));
    const float o1 = -(dmin * (float)((sm >> 12) & 15u));
#pragma unroll
    for (int m = 0; m < MR; ++m)
      out[m] += s0 * a0[m] + s1 * a1[m] + o0 * (x.s8[m][0] + x.s8[m][1]) + o1 * (x.s8[m][2] + x.s8[m][3]);
  }
};

template <> struct Qmv<Q6_K> {
  static constexpr int kPair = PAIR_K;
  static constexpr int kTbl = 0;
  __device__ static void load_tables(uint8_t*, const DevTables&, int, int) {}
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t*, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    const int chunk = g >> 2, plane = g & 3;
    uint32_t ql[8], qh[8];
    lds_words<8>(buf, off + 64 * chunk + 32 * (plane & 1), ql);
    lds_words<8>(buf, off + 128 + 32 * chunk, qh);
    const uint32_t sc2 = lds_u16(buf, off + 192 + 2 * g);
    const float d = h2f(lds_u16(buf, off + 208));
    const uint32_t ls = 4u * (plane >> 1), hs = 2u * plane;
    float a0[MR], a1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) { a0[m] = 0.f; a1[m] = 0.f; }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t L = ql[k] >> ls, H = qh[k] >> hs;
      const uint32_t A = sub_magic<1056>((L & 0x000F000Fu) | ((H & 0x00030003u) << 4) | 0x64006400u);
      const uint32_t B = sub_magic<1056>(((L >> 8) & 0x000F000Fu) | (((H >> 8) & 0x00030003u) << 4) | 0x64006400u);
      if (k < 4) { dacc<MR, XS>(A, x, 2 * k, a0); dacc<MR, XS>(B, x, 2 * k + 1, a0); }
      else { dacc<MR, XS>(A, x, 2 * k, a1); dacc<MR, XS>(B, x, 2 * k + 1, a1); }
    }
    const float s0 = d * (float)(int)(int8_t)(sc2 & 0xFFu), s1 = d * (float)(int)(int8_t)(sc2 >> 8);
#pragma unroll
    for (int m = 0; m < MR; ++m)
      out[m] += s0 * a0[m] + s1 * a1[m];
  }
};

template <> struct Qmv<IQ4_XS> {
  static constexpr int kPair = PAIR_16;
  static constexpr int kTbl = 1024;  // 256 fp16 pairs (kvalues[lo nibble], kvalues[hi nibble])
  __device__ static void load_tables(uint8_t* tbl, const DevTables&, int tid, int nthr) {
    uint32_t* t = reinterpret_cast<uint32_t*>(tbl);
    for (int i = tid; i < 256; i += nthr)
      t[i] = pack_h2((float)kIQ4Values[i & 15], (float)kIQ4Values[i >> 4]);
  }
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    const uint32_t hd = lds_w32(buf, off);
    const float d = h2f(hd & 0xFFFFu);
    const uint32_t low = (lds_u8(buf, off + 4 + (g >> 1)) >> (4 * (g & 1))) & 15u;
    const uint32_t high = ((hd >> 16) >> (2 * g)) & 3u;
    const int scale = (int)(low | (high << 4)) - 32;
    uint32_t q[4];
    lds_words<4>(buf, off + 8 + 16 * g, q);
    const uint32_t* t = reinterpret_cast<const uint32_t*>(tbl);
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dacc<MR, XS>(t[(q[k] >> (8 * i)) & 255u], x, 4 * k + i, acc);
    }
    const float s = d * (float)scale;
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += s * acc[m];
  }
};

// Sign masks: for sign byte s, dword i flips the fp16 signs of elements 2i (bit 15) and
// 2i+1 (bit 31).
__device__ __forceinline__ uint32_t sign_mask_pair(uint32_t s, int i) {
  return (((s >> (2 * i)) & 1u) << 15) | (((s >> (2 * i + 1)) & 1u) << 31);
}

template <int ENTRIES, int COORDS>
__device__ __forceinline__ void copy_grid(uint8_t* tbl, const DevTables& tb, int tid, int nthr) {
  const uint4* src = reinterpret_cast<const uint4*>(tb.grid16);
  uint4* dst = reinterpret_cast<uint4*>(tbl);
  constexpr int n = ENTRIES * COORDS * 2 / 16;
  for (int i = tid; i < n; i += nthr) dst[i] = src[i];
}

// 128 x 16 B sign masks of the ksigns table, after a grid of GRIDB bytes.
__device__ __forceinline__ void build_ks_masks(uint8_t* dst, const DevTables& tb, int tid, int nthr) {
  uint32_t* t = reinterpret_cast<uint32_t*>(dst);
  for (int i = tid; i < 128 * 4; i += nthr) t[i] = sign_mask_pair(tb.ksigns[i >> 2], i & 3);
}

template <> struct Qmv<IQ3_S> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kGridB = 512 * 4 * 2;
  static constexpr int kTbl = kGridB + 16 * 8;  // grid + 16 nibble sign masks
  __device__ static void load_tables(uint8_t* tbl, const DevTables& tb, int tid, int nthr) {
    copy_grid<512, 4>(tbl, tb, tid, nthr);
    uint32_t* t = reinterpret_cast<uint32_t*>(tbl + kGridB);
    for (int i = tid; i < 32; i += nthr) t[i] = sign_mask_pair(i >> 1, i & 1);
  }
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    const float d = h2f(lds_u16(buf, off));
    const uint32_t snib = (lds_u8(buf, off + 106 + (g >> 1)) >> (4 * (g & 1))) & 15u;
    const float db = d * (float)(1u + 2u * snib);
    uint32_t q[2];
    lds_words<2>(buf, off + 2 + 8 * g, q);
    const uint32_t qh = lds_u8(buf, off + 66 + g);
    const uint32_t sg = lds_w32(buf, off + 74 + 4 * g);
    const uint2* grid = reinterpret_cast<const uint2*>(tbl);
    const uint2* sm = reinterpret_cast<const uint2*>(tbl + kGridB);
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t idx = ((q[e >> 2] >> (8 * (e & 3))) & 255u) | (((qh >> e) & 1u) << 8);
      uint2 G = grid[idx];
      const uint2 M = sm[(sg >> (4 * e)) & 15u];
      dacc<MR, XS>(G.x ^ M.x, x, 2 * e, acc);
      dacc<MR, XS>(G.y ^ M.y, x, 2 * e + 1, acc);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += db * acc[m];
  }
};

template <> struct Qmv<IQ3_XXS> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kGridB = 256 * 4 * 2;
  static constexpr int kTbl = kGridB + 128 * 16;
  __device__ static void load_tables(uint8_t* tbl, const DevTables& tb, int tid, int nthr) {
    copy_grid<256, 4>(tbl, tb, tid, nthr);
    build_ks_masks(tbl + kGridB, tb, tid, nthr);
  }
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    const float dh = h2f(lds_u16(buf, off));
    uint32_t q[2];
    lds_words<2>(buf, off + 2 + 8 * g, q);
    const uint32_t u = lds_w32(buf, off + 66 + 4 * g);
    const float d = dh * (0.5f + (float)(u >> 28)) * 0.5f;
    const uint2* grid = reinterpret_cast<const uint2*>(tbl);
    const uint4* km = reinterpret_cast<const uint4*>(tbl + kGridB);
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint4 M = km[(u >> (7 * l)) & 127u];
      const uint2 G0 = grid[(q[l >> 1] >> (16 * (l & 1))) & 255u];
      const uint2 G1 = grid[(q[l >> 1] >> (16 * (l & 1) + 8)) & 255u];
      dacc<MR, XS>(G0.x ^ M.x, x, 4 * l, acc);
      dacc<MR, XS>(G0.y ^ M.y, x, 4 * l + 1, acc);
      dacc<MR, XS>(G1.x ^ M.z, x, 4 * l + 2, acc);
      dacc<MR, XS>(G1.y ^ M.w, x, 4 * l + 3, acc);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += d * acc[m];
  }
};

template <> struct Qmv<IQ2_XXS> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kGridB = 256 * 8 * 2;
  static constexpr int kTbl = kGridB + 128 * 16;
  __device__ static void load_tables(uint8_t* tbl, const DevTables& tb, int tid, int nthr) {
    copy_grid<256, 8>(tbl, tb, tid, nthr);
    build_ks_masks(tbl + kGridB, tb, tid, nthr);
  }
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    const float dh = h2f(lds_u16(buf, off));
    uint32_t q[2];
    lds_words<2>(buf, off + 2 + 8 * g, q);
    const uint32_t u = q[1];
    const float d = dh * (0.5f + (float)(u >> 28)) * 0.25f;
    const uint4* grid = reinterpret_cast<const uint4*>(tbl);
    const uint4* km = reinterpret_cast<const uint4*>(tbl + kGridB);
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint4 M = km[(u >> (7 * l)) & 127u];
      const uint4 G = grid[(q[0] >> (8 * l)) & 255u];
      dacc<MR, XS>(G.x ^ M.x, x, 4 * l, acc);
      dacc<MR, XS>(G.y ^ M.y, x, 4 * l + 1, acc);
      dacc<MR, XS>(G.z ^ M.z, x, 4 * l + 2, acc);
      dacc<MR, XS>(G.w ^ M.w, x, 4 * l + 3, acc);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += d * acc[m];
  }
};

template <> struct Qmv<IQ2_XS> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kGridB = 512 * 8 * 2;
  static constexpr int kTbl = kGridB + 128 * 16;
  __device__ static void load_tables(uint8_t* tbl, const DevTables& tb, int tid, int nthr) {
    copy_grid<512, 8>(tbl, tb, tid, nthr);
    build_ks_masks(tbl + kGridB, tb, tid, nthr);
  }
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    const float dh = h2f(lds_u16(buf, off));
    uint32_t q[2];
    lds_words<2>(buf, off + 2 + 8 * g, q);
    const uint32_t sb = lds_u8(buf, off + 66 + g);
    const uint4* grid = reinterpret_cast<const uint4*>(tbl);
    const uint4* km = reinterpret_cast<const uint4*>(tbl + kGridB);
    float a0[MR], a1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) { a0[m] = 0.f; a1[m] = 0.f; }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t v = (q[l >> 1] >> (16 * (l & 1))) & 0xFFFFu;
      const uint4 M = km[(v >> 9) & 127u];
      const uint4 G = grid[v & 511u];
      if (l < 2) {
        dacc<MR, XS>(G.x ^ M.x, x, 4 * l, a0); dacc<MR, XS>(G.y ^ M.y, x, 4 * l + 1, a0);
        dacc<MR, XS>(G.z ^ M.z, x, 4 * l + 2, a0); dacc<MR, XS>(G.w ^ M.w, x, 4 * l + 3, a0);
      } else {
        dacc<MR, XS>(G.x ^ M.x, x, 4 * l, a1); dacc<MR, XS>(G.y ^ M.y, x, 4 * l + 1, a1);
        dacc<MR, XS>(G.z ^ M.z, x, 4 * l + 2, a1); dacc<MR, XS>(G.w ^ M.w, x, 4 * l + 3, a1);
      }
    }
    const float d0 = dh * (0.5f + (float)(sb & 15u)) * 0.25f, d1 = dh * (0.5f + (float)(sb >> 4)) * 0.25f;
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += d0 * a0[m] + d1 * a1[m];
  }
};

template <> struct Qmv<IQ2_S> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kGridB = 1024 * 8 * 2;
  static constexpr int kTbl = kGridB + 256 * 16;
  __device__ static void load_tables(uint8_t* tbl, const DevTables& tb, int tid, int nthr) {
    copy_grid<1024, 8>(tbl, tb, tid, nthr);
    uint32_t* t = reinterpret_cast<uint32_t*>(tbl + kGridB);
    for (int i = tid; i < 256 * 4; i += nthr) t[i] = sign_mask_pair(i >> 2, i & 3);
  }
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    const float dh = h2f(lds_u16(buf, off));
    const uint32_t qs = lds_w32(buf, off + 2 + 4 * g);
    const uint32_t sg = lds_w32(buf, off + 34 + 4 * g);
    const uint32_t qh = lds_u8(buf, off + 66 + g);
    const uint32_t sb = lds_u8(buf, off + 74 + g);
    const uint4* grid = reinterpret_cast<const uint4*>(tbl);
    const uint4* bm = reinterpret_cast<const uint4*>(tbl + kGridB);
    float a0[MR], a1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) { a0[m] = 0.f; a1[m] = 0.f; }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t idx = ((qs >> (8 * l)) & 255u) | (((qh >> (2 * l)) & 3u) << 8);
      const uint4 G = grid[idx];
      const uint4 M = bm[(sg >> (8 * l)) & 255u];
      if (l < 2) {
        dacc<MR, XS>(G.x ^ M.x, x, 4 * l, a0); dacc<MR, XS>(G.y ^ M.y, x, 4 * l + 1, a0);
        dacc<MR, XS>(G.z ^ M.z, x, 4 * l + 2, a0); dacc<MR, XS>(G.w ^ M.w, x, 4 * l + 3, a0);
      } else {
        dacc<MR, XS>(G.x ^ M.x, x, 4 * l, a1); dacc<MR, XS>(G.y ^ M.y, x, 4 * l + 1, a1);
        dacc<MR, XS>(G.z ^ M.z, x, 4 * l + 2, a1); dacc<MR, XS>(G.w ^ M.w, x, 4 * l + 3, a1);
      }
    }
    const float d0 = dh * (0.5f + (float)(sb & 15u)) * 0.25f, d1 = dh * (0.5f + (float)(sb >> 4)) * 0.25f;
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += d0 * a0[m] + d1 * a1[m];
  }
};

template <> struct Qmv<IQ1_S> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kTbl = 2048 * 8 * 2;
  __device__ static void load_tables(uint8_t* tbl, const DevTables& tb, int tid, int nthr) {
    copy_grid<2048, 8>(tbl, tb, tid, nthr);
  }
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    const float dh = h2f(lds_u16(buf, off));
    const uint32_t qs = lds_w32(buf, off + 2 + 4 * g);
    const uint32_t h = lds_u16(buf, off + 34 + 2 * g);
    const float d = dh * (float)(2u * ((h >> 12) & 7u) + 1u);
    const float delta = (h & 0x8000u) ? -0.125f : 0.125f;
    const uint4* grid = reinterpret_cast<const uint4*>(tbl);
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint4 G = grid[((qs >> (8 * l)) & 255u) | (((h >> (3 * l)) & 7u) << 8)];
      dacc<MR, XS>(G.x, x, 4 * l, acc); dacc<MR, XS>(G.y, x, 4 * l + 1, acc);
      dacc<MR, XS>(G.z, x, 4 * l + 2, acc); dacc<MR, XS>(G.w, x, 4 * l + 3, acc);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float xs = (x.s8[m][0] + x.s8[m][1]) + (x.s8[m][2] + x.s8[m][3]);
      out[m] += d * (acc[m] + delta * xs);
    }
  }
};

template <> struct Qmv<IQ1_M> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kTbl = 2048 * 8 * 2;
  __device__ static void load_tables(uint8_t* tbl, const DevTables& tb, int tid, int nthr) {
    copy_grid<2048, 8>(tbl, tb, tid, nthr);
  }
  template <int MR, bool XS>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const XReg<MR, XS>& x,
                             float (&out)[MR]) {
    const uint32_t qs = lds_w32(buf, off + 4 * g);
    const uint32_t qh = lds_u16(buf, off + 32 + 2 * g);
    uint32_t w[2];
    lds_words<2>(buf, off + 48, w);
    const uint32_t w0 = w[0] & 0xFFFFu, w1 = w[0] >> 16, w2 = w[1] & 0xFFFFu, w3 = w[1] >> 16;
    const uint32_t dbits = ((w0 & 61440u) >> 12) | ((w1 & 61440u) >> 8) | ((w2 & 61440u) >> 4) | (w3 & 61440u);
    const float d = h2f(dbits);
    const uint32_t ww = (g >> 1) == 0 ? w0 : ((g >> 1) == 1 ? w1 : ((g >> 1) == 2 ? w2 : w3));
    const uint32_t sh0 = 3u * ((2 * g) & 3);
    const float d0 = d * (float)(2u * ((ww >> sh0) & 7u) + 1u);
    const float d1 = d * (float)(2u * ((ww >> (sh0 + 3)) & 7u) + 1u);
    const uint4* grid = reinterpret_cast<const uint4*>(tbl);
    float a[4][MR];
#pragma unroll
    for (int l = 0; l < 4; ++l)
#pragma unroll
      for (int m = 0; m < MR; ++m) a[l][m] = 0.f;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t hn = (qh >> (4 * l)) & 15u;
      const uint4 G = grid[((qs >> (8 * l)) & 255u) | ((hn & 7u) << 8)];
      dacc<MR, XS>(G.x, x, 4 * l, a[l]); dacc<MR, XS>(G.y, x, 4 * l + 1, a[l]);
      dacc<MR, XS>(G.z, x, 4 * l + 2, a[l]); dacc<MR, XS>(G.w, x, 4 * l + 3, a[l]);
      const float delta = (hn & 8u) ? -0.125f : 0.125f;
#pragma unroll
      for (int m = 0; m < MR; ++m) a[l][m] += delta * x.s8[m][l];
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += d0 * (a[0][m] + a[1][m]) + d1 * (a[2][m] + a[3][m]);
  }
};

// ---- staging: bytes [start, end) of the packed matrix -> LDS ---------------------------
// LDS byte i of dst holds global byte (A0 + i), A0 = (packed + start) rounded down to 16.
// Interior 16-byte chunks go through the LDS DMA path; chunks that straddle either end of
// the packed allocation are copied byte by byte so nothing outside it is read.
__device__ __forceinline__ void stage_rows(const uint8_t* packed, int64_t total, int64_t start, int64_t end,
                                           uint8_t* dst, int tid, int nthr) {
  const uintptr_t lo = reinterpret_cast<uintptr_t>(packed), hi = lo + (uintptr_t)total;
  const uintptr_t A0 = (lo + (uintptr_t)start) & ~(uintptr_t)15;
  const uintptr_t A1 = (lo + (uintptr_t)end + 15) & ~(uintptr_t)15;
  const int nchunks = (int)((A1 - A0) >> 4);
  const int wave = tid >> 6, lane = tid & 63, nw = nthr >> 6;
  for (int c0 = wave * 64; c0 < nchunks; c0 += nw * 64) {
    const int c = c0 + lane;
    const uintptr_t ca = A0 + (uintptr_t)c * 16;
    if (c < nchunks) {
      if (ca >= lo && ca + 16 <= hi) {
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(ca),
                                         (__attribute__((address_space(3))) void*)(dst + c0 * 16), 16, 0, 0);
      } else {
        for (int k = 0; k < 16; ++k)
          if (ca + k >= lo && ca + k < hi) dst[c * 16 + k] = *reinterpret_cast<const uint8_t*>(ca + k);
      }
    }
  }
}

__device__ __forceinline__ float load_x(const void* x, int dt, int64_t i) {
  if (dt == DT_F16) return (float)reinterpret_cast<const _Float16*>(x)[i];
  if (dt == DT_BF16) {
    uint32_t b = reinterpret_cast<const uint16_t*>(x)[i];
    return __builtin_bit_cast(float, b << 16);
  }
  return reinterpret_cast<const float*>(x)[i];
}

__device__ __forceinline__ void store_y(void* y, int dt, int64_t i, float v) {
  if (dt == DT_F16) reinterpret_cast<_Float16*>(y)[i] = (_Float16)v;
  else if (dt == DT_BF16) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    b += 0x7FFFu + ((b >> 16) & 1u);  // round to nearest even
    reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)(b >> 16);
  } else reinterpret_cast<float*>(y)[i] = v;
}

template <int T, int MR, bool XS>
__global__ void __launch_bounds__(576) qmv_kernel(QmvArgs a) {
  using P = Qmv<T>;
  constexpr int BB = BlockBytes<T>::v;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, nthr = blockDim.x;
  uint8_t* tbl = smem;
  uint8_t* bufs = smem + a.tbl_bytes;
  float* red = reinterpret_cast<float*>(bufs + 2 * a.buf_bytes);  // [kJMax*MR][nthr]

  const int64_t r0 = (int64_t)blockIdx.x * a.rows_per_wg;
  const int64_t r1 = min(a.N, r0 + (int64_t)a.rows_per_wg);
  if (r0 >= r1) return;
  if (r0 < r1) stage_rows(a.packed, a.total_bytes, r0 * a.row_bytes, min(r1, r0 + a.J) * a.row_bytes, bufs, tid, nthr);
  P::load_tables(tbl, a.tb, tid, nthr);

  const int U = a.K >> 5;
  const bool active = tid < U;
  const int u = active ? tid : 0;
  const int b = u >> 3, g = u & 7;

  XReg<MR, XS> xr;
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float xv[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) xv[i] = (active && m < a.M) ? load_x(a.x, a.x_dtype, (int64_t)m * a.K + 32 * u + i) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c) s += xv[8 * i + c];
      xr.s8[m][i] = s;
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

  int bi = 0;
  for (int64_t rs = r0; rs < r1; rs += a.J) {
    const int64_t re = min(r1, rs + (int64_t)a.J);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (re < r1) stage_rows(a.packed, a.total_bytes, re * a.row_bytes, min(r1, re + a.J) * a.row_bytes,
                            bufs + (bi ^ 1) * a.buf_bytes, tid, nthr);
    const uint8_t* buf = bufs + bi * a.buf_bytes;
    const uint32_t delta = (uint32_t)((reinterpret_cast<uintptr_t>(a.packed) + (uintptr_t)(rs * a.row_bytes)) & 15u);
    const int nj = (int)(re - rs);
    float acc[kJMax][MR];
#pragma unroll
    for (int j = 0; j < kJMax; ++j)
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[j][m] = 0.f;
    if (active) {
#pragma unroll
      for (int j = 0; j < kJMax; ++j)
        if (j < nj) P::template dot<MR, XS>(buf, delta + (uint32_t)(j * a.row_bytes + b * BB), g, tbl, xr, acc[j]);
    }
#pragma unroll
    for (int j = 0; j < kJMax; ++j)
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (j < nj) red[(j * MR + m) * nthr + tid] = acc[j][m];
    __syncthreads();
    // one wave per output (row j, activation row m)
    const int wave = tid >> 6, lane = tid & 63, nw = nthr >> 6;
    for (int o = wave; o < nj * MR; o += nw) {
      float s = 0.f;
      for (int i = lane; i < nthr; i += 64) s += red[o * nthr + i];
#pragma unroll
      for (int w = 32; w >= 1; w >>= 1) s += __shfl_xor(s, w, 64);
      const int j = o / MR, m = o % MR;
      if (lane == 0 && m < a.M) store_y(a.y, a.y_dtype, (int64_t)m * a.N + rs + j, s);
    }
    bi ^= 1;
  }
}

template <int T, int MR, bool XS>
static hipError_t launch_qmv_t(const QmvArgs& a, int grid, int threads, size_t lds, hipStream_t s) {
  auto k = qmv_kernel<T, MR, XS>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(k, dim3(grid), dim3(threads), lds, s, a);
  return hipGetLastError();
}

template <int T>
static int qmv_tbl_bytes() { return Qmv<T>::kTbl; }

template <int T>
static hipError_t launch_qmv_type(const QmvArgs& a, int mr, bool xs, int grid, int threads, size_t lds,
                                  hipStream_t s) {
  if (mr == 1) return xs ? launch_qmv_t<T, 1, true>(a, grid, threads, lds, s) : launch_qmv_t<T, 1, false>(a, grid, threads, lds, s);
  if (mr == 2) return xs ? launch_qmv_t<T, 2, true>(a, grid, threads, lds, s) : launch_qmv_t<T, 2, false>(a, grid, threads, lds, s);
  if (xs) return hipErrorInvalidValue;  // split-precision activations run at most 2 rows per launch
  return launch_qmv_t<T, 4, false>(a, grid, threads, lds, s);
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

// Launch plan: one workgroup of K/32 lanes (rounded up to whole waves) per CU, each
// owning N/#CU consecutive rows, J rows per double-buffered step.
hipError_t launch_qmv(int qt, const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int M, int64_t N,
                      int K, const DevTables& tb, int num_cus, hipStream_t s) {
  QmvArgs a;
  a.packed = packed; a.x = x; a.y = y; a.N = N; a.K = K; a.M = M; a.x_dtype = xdt; a.y_dtype = ydt; a.tb = tb;
  const int bb = block_bytes_of(qt);
  a.row_bytes = (K / 256) * bb;
  a.total_bytes = N * (int64_t)a.row_bytes;
  a.tbl_bytes = (qmv_table_bytes(qt) + 15) & ~15;
  const int U = K / 32;
  const int threads = ((U + 63) / 64) * 64;
  if (threads > kQmvMaxThreads) return hipErrorInvalidValue;
  const int mr = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
  if (xdt != DT_F16 && mr > 2) return hipErrorInvalidValue;
  const int jmax = kJMax;
  const int red_bytes = jmax * mr * threads * 4;
  const int budget = 160 * 1024 - a.tbl_bytes - red_bytes - 256;
  int J = (budget / 2 - 48) / a.row_bytes;
  if (J > jmax) J = jmax;
  if (J < 1) return hipErrorInvalidValue;
  a.J = J;
  a.buf_bytes = ((J * a.row_bytes + 48) + 15) & ~15;
  int grid = num_cus;
  if (N < grid) grid = (int)N;
  a.rows_per_wg = (int)((N + grid - 1) / grid);
  grid = (int)((N + a.rows_per_wg - 1) / a.rows_per_wg);
  const size_t lds = (size_t)a.tbl_bytes + 2 * (size_t)a.buf_bytes + (size_t)red_bytes;
  const bool xs = xdt != DT_F16;
  switch (qt) {
    case Q2_K: return launch_qmv_type<Q2_K>(a, mr, xs, grid, threads, lds, s);
    case Q4_K: return launch_qmv_type<Q4_K>(a, mr, xs, grid, threads, lds, s);
    case Q6_K: return launch_qmv_type<Q6_K>(a, mr, xs, grid, threads, lds, s);
    case IQ4_XS: return launch_qmv_type<IQ4_XS>(a, mr, xs, grid, threads, lds, s);
    case IQ3_S: return launch_qmv_type<IQ3_S>(a, mr, xs, grid, threads, lds, s);
    case IQ3_XXS: return launch_qmv_type<IQ3_XXS>(a, mr, xs, grid, threads, lds, s);
    case IQ2_XXS: return launch_qmv_type<IQ2_XXS>(a, mr, xs, grid, threads, lds, s);
    case IQ2_XS: return launch_qmv_type<IQ2_XS>(a, mr, xs, grid, threads, lds, s);
    case IQ2_S: return launch_qmv_type<IQ2_S>(a, mr, xs, grid, threads, lds, s);
    case IQ1_S: return launch_qmv_type<IQ1_S>(a, mr, xs, grid, threads, lds, s);
    case IQ1_M: return launch_qmv_type<IQ1_M>(a, mr, xs, grid, threads, lds, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gsq
