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
  int rows_per_wg, J, row_bytes, buf_bytes, tbl_bytes, red_bytes;
  int slots, lanes_per_slot, red_tpr;
  DevTables tb;
};

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

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

// Small unsigned codes q (< 1024) placed in the low bits of an fp16 lane are the subnormal
// values q * 2^-24, so a masked code pair is directly a v_dot2_f32_f16 operand: the fp16 x
// fp16 products are exact in fp32 and the group scale absorbs the 2^24.
constexpr float kSub = 16777216.f;  // 2^24

// Split-precision activations (XS: fp32/bf16 split into fp16 hi + lo) have subnormal lo
// parts, and subnormal x subnormal products lose bits in v_dot2, so those variants encode
// codes as exact normal fp16 integers instead: (1024 + q) with the 1024 removed by one
// v_pk_add_f16.
template <bool XS>
__device__ __forceinline__ uint32_t enc_codes(uint32_t codes) {
  if constexpr (XS) {
    const half2_t r = __builtin_bit_cast(half2_t, codes | 0x64006400u) - (half2_t){(_Float16)1024.f, (_Float16)1024.f};
    return __builtin_bit_cast(uint32_t, r);
  } else {
    return codes;
  }
}
template <bool XS>
__device__ __forceinline__ constexpr float enc_scale() { return XS ? 1.f : kSub; }

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
      const uint32_t v = q[k] >> sh;
      dacc<MR, XS>(enc_codes<XS>(v & 0x000F000Fu), x, 2 * k, acc);
      dacc<MR, XS>(enc_codes<XS>((v >> 8) & 0x000F000Fu), x, 2 * k + 1, acc);
    }
    const float s = d * (float)sc * enc_scale<XS>();
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
      const uint32_t v = q[k] >> sh;
      const uint32_t A = enc_codes<XS>(v & 0x00030003u);
      const uint32_t B = enc_codes<XS>((v >> 8) & 0x00030003u);
      if (k < 4) { dacc<MR, XS>(A, x, 2 * k, a0); dacc<MR, XS>(B, x, 2 * k + 1, a0); }
      else { dacc<MR, XS>(A, x, 2 * k, a1); dacc<MR, XS>(B, x, 2 * k + 1, a1); }
    }
    const float s0 = d * (float)(sm & 15u) * enc_scale<XS>(), s1 = d * (float)((sm >> 8) & 15u) * enc_scale<XS>();
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
      const uint32_t A = enc_codes<XS>((L & 0x000F000Fu) | ((H & 0x00030003u) << 4));
      const uint32_t B = enc_codes<XS>(((L >> 8) & 0x000F000Fu) | (((H >> 8) & 0x00030003u) << 4));
      if (k < 4) { dacc<MR, XS>(A, x, 2 * k, a0); dacc<MR, XS>(B, x, 2 * k + 1, a0); }
      else { dacc<MR, XS>(A, x, 2 * k, a1); dacc<MR, XS>(B, x, 2 * k + 1, a1); }
    }
    const float s0 = d * (float)(int)(int8_t)(sc2 & 0xFFu), s1 = d * (float)(int)(int8_t)(sc2 >> 8);
#pragma unroll
    for (int m = 0; m < MR; ++m)
      out[m] += s0 * (enc_scale<XS>() * a0[m] - 32.f * (x.s8[m][0] + x.s8[m][1])) +
                s1 * (enc_scale<XS>() * a1[m] - 32.f * (x.s8[m][2] + x.s8[m][3]));
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
// Interior 16-byte chunks go through the LDS DMA path (global_load_lds_dwordx4). Chunks that
// straddle either end of the packed allocation are copied byte by byte, so nothing outside
// it is read. Returns the number of DMA instructions this wave issued (wave-uniform), which
// the consumer uses for an exact vmcnt wait.
__device__ __forceinline__ int stage_rows(const uint8_t* packed, int64_t total, int64_t start, int64_t end,
                                          uint8_t* dst, int tid, int nthr) {
  const uintptr_t lo = reinterpret_cast<uintptr_t>(packed), hi = lo + (uintptr_t)total;
  const uintptr_t A0 = (lo + (uintptr_t)start) & ~(uintptr_t)15;
  const uintptr_t A1 = (lo + (uintptr_t)end + 15) & ~(uintptr_t)15;
  const int nchunks = (int)((A1 - A0) >> 4);
  const int wave = tid >> 6, lane = tid & 63, nw = nthr >> 6;
  int issued = 0;
  for (int c0 = wave * 64; c0 < nchunks; c0 += nw * 64) {
    const int c = c0 + lane;
    const uintptr_t ca = A0 + (uintptr_t)c * 16;
    const bool valid = c < nchunks;
    const bool dma = valid && ca >= lo && ca + 16 <= hi;
    if (__builtin_amdgcn_ballot_w64(dma) != 0) ++issued;
    if (dma) {
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(ca),
                                       (__attribute__((address_space(3))) void*)(dst + c0 * 16), 16, 0, 0);
    } else if (valid) {
      for (int k = 0; k < 16; ++k)
        if (ca + k >= lo && ca + k < hi) dst[c * 16 + k] = *reinterpret_cast<const uint8_t*>(ca + k);
    }
  }
  return __builtin_amdgcn_readfirstlane(issued);
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding); n is clamped to 63,
// and a smaller immediate only waits longer.
__device__ __forceinline__ void wait_vmcnt(int n) {
#define GSQ_VMW(k) case k: __builtin_amdgcn_s_waitcnt(0x0F70 | ((k) & 15) | (((k) >> 4) << 14)); break;
  switch (n < 0 ? 0 : n) {
    GSQ_VMW(0) GSQ_VMW(1) GSQ_VMW(2) GSQ_VMW(3) GSQ_VMW(4) GSQ_VMW(5) GSQ_VMW(6) GSQ_VMW(7)
    GSQ_VMW(8) GSQ_VMW(9) GSQ_VMW(10) GSQ_VMW(11) GSQ_VMW(12) GSQ_VMW(13) GSQ_VMW(14) GSQ_VMW(15)
    default: __builtin_amdgcn_s_waitcnt(0x0F70 | 15); break;
  }
#undef GSQ_VMW
}

__device__ __forceinline__ float load_x(const void* x, int dt, int64_t i) {
  if (dt == DT_F16) return (float)reinterpret_cast<const _Float16*>(x)[i];
  if (dt == DT_BF16) {
    uint32_t b = reinterpret_cast<const uint16_t*>(x)[i];
    return __builtin_bit_cast(float, b << 16);
  }
  return reinterpret_cast<const float*>(x)[i];
}

// 32 consecutive activations starting at element i0 (64-byte aligned) -> float, with
// 16-byte vector loads all in flight before the first use; zeros when !valid.
__device__ __forceinline__ void load_x32(const void* x, int dt, int64_t i0, bool valid, float (&xv)[32]) {
  if (!valid) {
#pragma unroll
    for (int i = 0; i < 32; ++i) xv[i] = 0.f;
    return;
  }
  if (dt == DT_F32) {
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(x) + i0);
    uint4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = p[k];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      xv[4 * k] = __builtin_bit_cast(float, v[k].x); xv[4 * k + 1] = __builtin_bit_cast(float, v[k].y);
      xv[4 * k + 2] = __builtin_bit_cast(float, v[k].z); xv[4 * k + 3] = __builtin_bit_cast(float, v[k].w);
    }
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + i0);
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = p[k];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (dt == DT_F16) {
          xv[8 * k + 2 * j] = h2f(w[j] & 0xFFFFu);
          xv[8 * k + 2 * j + 1] = h2f(w[j] >> 16);
        } else {
          xv[8 * k + 2 * j] = __builtin_bit_cast(float, w[j] << 16);
          xv[8 * k + 2 * j + 1] = __builtin_bit_cast(float, w[j] & 0xFFFF0000u);
        }
      }
    }
  }
}

__device__ __forceinline__ void store_y(void* y, int dt, int64_t i, float v) {
  if (dt == DT_F16) reinterpret_cast<_Float16*>(y)[i] = (_Float16)v;
  else if (dt == DT_BF16) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    b += 0x7FFFu + ((b >> 16) & 1u);  // round to nearest even
    reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)(b >> 16);
  } else reinterpret_cast<float*>(y)[i] = v;
}

// Sum over the 64 lanes of a wave with DPP row operations; the total lands in lane 63.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xF, false));
}

__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v += dpp_f<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141, 0xF>(v);  // row_half_mirror
  v += dpp_f<0x140, 0xF>(v);  // row_mirror: every lane holds its row (16 lanes) total
  v += dpp_f<0x142, 0xA>(v);  // row_bcast15 into rows 1 and 3
  v += dpp_f<0x143, 0xC>(v);  // row_bcast31 into rows 2 and 3
  return v;
}

// Register-heavy variants (4 activation rows, or 2 rows x 2 groups) run at most 512 threads.
template <int W> struct QmvBounds { static constexpr int v = W >= 4 ? 512 : 1024; };

template <int T, int MR, bool XS, int GL>
__global__ void __launch_bounds__(QmvBounds<MR * GL>::v) qmv_kernel(QmvArgs a) {
  using P = Qmv<T>;
  constexpr int BB = BlockBytes<T>::v;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, nthr = blockDim.x;
  uint8_t* tbl = smem;
  float* red = reinterpret_cast<float*>(smem + a.tbl_bytes);  // [rows_per_wg][MR][Ua]
  uint8_t* ring = smem + a.tbl_bytes + a.red_bytes;            // 3 x buf_bytes

  const int64_t r0 = (int64_t)blockIdx.x * a.rows_per_wg;
  const int64_t r1 = min(a.N, r0 + (int64_t)a.rows_per_wg);
  if (r0 >= r1) return;
  const int nsteps = (int)((r1 - r0 + a.J - 1) / a.J);
  auto step_rows = [&](int s, int64_t& rs, int64_t& re) {
    rs = r0 + (int64_t)s * a.J;
    re = min(r1, rs + (int64_t)a.J);
  };
  // DMA instructions this wave issued for the next step (kept in scalars: a runtime-indexed
  // array would live in scratch, and scratch reads wait for every outstanding DMA)
  int cnt_next = 0;
  {
    int64_t rs, re;
    step_rows(0, rs, re);
    stage_rows(a.packed, a.total_bytes, rs * a.row_bytes, re * a.row_bytes, ring, tid, nthr);
    if (nsteps > 1) {
      step_rows(1, rs, re);
      cnt_next = stage_rows(a.packed, a.total_bytes, rs * a.row_bytes, re * a.row_bytes, ring + a.buf_bytes, tid, nthr);
    }
  }
  P::load_tables(tbl, a.tb, tid, nthr);

  const int Ls = a.lanes_per_slot;
  const int slot = min(tid / Ls, a.slots), ls = tid - min(tid / Ls, a.slots) * Ls;
  const int U = a.K >> 5;
  const int Ua = (U + GL - 1) / GL;  // lanes of a slot that hold partials
  XReg<MR, XS> xr[GL];
  int gb[GL], gg[GL];
  bool act[GL];
#pragma unroll
  for (int q = 0; q < GL; ++q) {
    const int u = ls * GL + q;
    act[q] = slot < a.slots && u < U;
    const int uu = act[q] ? u : 0;
    gb[q] = uu >> 3;
    gg[q] = uu & 7;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float xv[32];
      load_x32(a.x, a.x_dtype, (int64_t)m * a.K + 32 * uu, act[q] && m < a.M, xv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c) s += xv[8 * i + c];
        xr[q].s8[m][i] = s;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        int e0, e1;
        pair_idx<P::kPair>(i, e0, e1);
        const _Float16 h0 = (_Float16)xv[e0], h1 = (_Float16)xv[e1];
        xr[q].h[m][i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        if constexpr (XS) xr[q].l[m][i] = pack_h2(xv[e0] - (float)h0, xv[e1] - (float)h1);
      }
    }
  }
  const bool any_act = act[0];

  for (int s = 0; s < nsteps; ++s) {
    wait_vmcnt(s + 1 < nsteps ? cnt_next : 0);
    __syncthreads();
    int cnt_after = 0;
    if (s + 2 < nsteps) {
      int64_t rs2, re2;
      step_rows(s + 2, rs2, re2);
      cnt_after = stage_rows(a.packed, a.total_bytes, rs2 * a.row_bytes, re2 * a.row_bytes,
                             ring + ((s + 2) % 3) * a.buf_bytes, tid, nthr);
    }
    cnt_next = cnt_after;
    int64_t rs, re;
    step_rows(s, rs, re);
    const uint8_t* buf = ring + (s % 3) * a.buf_bytes;
    const uint32_t delta = (uint32_t)((reinterpret_cast<uintptr_t>(a.packed) + (uintptr_t)(rs * a.row_bytes)) & 15u);
    const int nj = (int)(re - rs);
    if (any_act) {
      for (int j = slot; j < nj; j += a.slots) {
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
        for (int q = 0; q < GL; ++q)
          if (act[q]) P::template dot<MR, XS>(buf, delta + (uint32_t)(j * a.row_bytes + gb[q] * BB), gg[q], tbl, xr[q], acc);
        const int rl = (int)(rs - r0) + j;
#pragma unroll
        for (int m = 0; m < MR; ++m) red[(rl * MR + m) * Ua + ls] = acc[m];
      }
    }
  }
  __syncthreads();
  // final reduction: TPR consecutive threads per (row, activation row); each sums a
  // contiguous run of partials, then the run sums are combined with DPP inside 16-lane rows.
  const int nout = (int)(r1 - r0) * MR;
  const int TPR = a.red_tpr;
  const int per = ((Ua + TPR - 1) / TPR + 3) & ~3;
  for (int o0 = 0; o0 < nout; o0 += nthr / TPR) {
    const int o = o0 + tid / TPR, p = tid % TPR;
    float v = 0.f;
    if (o < nout) {
      const float4* rp = reinterpret_cast<const float4*>(red + (size_t)o * Ua);
      const int i0 = p * per, i1 = min(Ua, i0 + per);  // multiples of 4
      float4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int i = i0 >> 2; i < (i1 >> 2); ++i) {
        const float4 t = rp[i];
        s4.x += t.x; s4.y += t.y; s4.z += t.z; s4.w += t.w;
      }
      v = (s4.x + s4.y) + (s4.z + s4.w);
    }
    if (TPR >= 2) v += dpp_f<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    if (TPR >= 4) v += dpp_f<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    if (TPR >= 8) v += dpp_f<0x141, 0xF>(v);  // row_half_mirror
    if (TPR >= 16) v += dpp_f<0x140, 0xF>(v); // row_mirror
    if (o < nout && p == 0) {
      const int rl = o / MR, m = o - rl * MR;
      if (m < a.M) store_y(a.y, a.y_dtype, (int64_t)m * a.N + r0 + rl, v);
    }
  }
}

template <int T, int MR, bool XS, int GL>
static hipError_t launch_qmv_t(const QmvArgs& a, int grid, int threads, size_t lds, hipStream_t s) {
  auto k = qmv_kernel<T, MR, XS, GL>;
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

template <int T, int GL>
static hipError_t launch_qmv_gl(const QmvArgs& a, int mr, bool xs, int grid, int threads, size_t lds,
                                hipStream_t s) {
  if (mr == 1) return xs ? launch_qmv_t<T, 1, true, GL>(a, grid, threads, lds, s) : launch_qmv_t<T, 1, false, GL>(a, grid, threads, lds, s);
  if (mr == 2) return xs ? launch_qmv_t<T, 2, true, GL>(a, grid, threads, lds, s) : launch_qmv_t<T, 2, false, GL>(a, grid, threads, lds, s);
  // 4 activation rows only with fp16 activations and one group per lane (register budget)
  if (xs || GL != 1) return hipErrorInvalidValue;
  return launch_qmv_t<T, 4, false, 1>(a, grid, threads, lds, s);
}

template <int T>
static hipError_t launch_qmv_type(const QmvArgs& a, int gl, int mr, bool xs, int grid, int threads, size_t lds,
                                  hipStream_t s) {
  return gl == 1 ? launch_qmv_gl<T, 1>(a, mr, xs, grid, threads, lds, s)
                 : launch_qmv_gl<T, 2>(a, mr, xs, grid, threads, lds, s);
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

// Launch plan. One workgroup per CU, each owning ceil(N / #CU) consecutive rows (one
// contiguous byte range). A workgroup has `slots` row slots of `lanes_per_slot` lanes;
// lane l of a slot owns GL consecutive 32-weight groups of every row the slot processes.
// Rows stream through a 3-deep LDS ring, J rows per step.
hipError_t launch_qmv(int qt, const uint8_t* packed, const void* x, int xdt, void* y, int ydt, int M, int64_t N,
                      int K, const DevTables& tb, int num_cus, hipStream_t s) {
  QmvArgs a;
  a.packed = packed; a.x = x; a.y = y; a.N = N; a.K = K; a.M = M; a.x_dtype = xdt; a.y_dtype = ydt; a.tb = tb;
  const int bb = block_bytes_of(qt);
  a.row_bytes = (K / 256) * bb;
  a.total_bytes = N * (int64_t)a.row_bytes;
  a.tbl_bytes = (qmv_table_bytes(qt) + 15) & ~15;
  const int U = K / 32;
  const int gl = U > 320 ? 2 : 1;
  const int Ls = (U + gl - 1) / gl;  // lanes per row slot; slots need not align to waves
  const int mr = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
  const int max_threads = mr * gl >= 4 ? 512 : 1024;
  if (Ls > max_threads) return hipErrorInvalidValue;
  int slots = max_threads / Ls;
  if (slots > 16) slots = 16;
  const int threads = (slots * Ls + 63) / 64 * 64;
  if ((xdt != DT_F16 || gl != 1) && mr > 2) return hipErrorInvalidValue;
  int grid = num_cus;
  if (N < grid) grid = (int)N;
  a.rows_per_wg = (int)((N + grid - 1) / grid);
  const int Ua = (U + gl - 1) / gl;
  // the per-row partials must fit in LDS next to the tables and a ring of >= 2-row steps
  const int ring_min = 3 * (2 * a.row_bytes + 64);
  int max_rows = (160 * 1024 - a.tbl_bytes - ring_min - 64) / (mr * Ua * 4);
  if (max_rows < 1) max_rows = 1;
  if (a.rows_per_wg > max_rows) a.rows_per_wg = max_rows;
  grid = (int)((N + a.rows_per_wg - 1) / a.rows_per_wg);
  a.red_bytes = ((a.rows_per_wg * mr * Ua * 4) + 15) & ~15;
  a.red_tpr = Ua >= 256 ? 16 : (Ua >= 64 ? 8 : 4);
  const int budget = 160 * 1024 - a.tbl_bytes - a.red_bytes - 64;
  int J = (budget / 3 - 48) / a.row_bytes;
  if (J > a.rows_per_wg) J = a.rows_per_wg;
  if (J > 2 * slots) J = 2 * slots;
  if (J < 1) return hipErrorInvalidValue;
  a.J = J;
  a.buf_bytes = ((J * a.row_bytes + 48) + 15) & ~15;
  a.slots = slots;
  a.lanes_per_slot = Ls;
  const size_t lds = (size_t)a.tbl_bytes + (size_t)a.red_bytes + 3 * (size_t)a.buf_bytes;
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  const bool xs = xdt != DT_F16;
  switch (qt) {
    case Q2_K: return launch_qmv_type<Q2_K>(a, gl, mr, xs, grid, threads, lds, s);
    case Q4_K: return launch_qmv_type<Q4_K>(a, gl, mr, xs, grid, threads, lds, s);
    case Q6_K: return launch_qmv_type<Q6_K>(a, gl, mr, xs, grid, threads, lds, s);
    case IQ4_XS: return launch_qmv_type<IQ4_XS>(a, gl, mr, xs, grid, threads, lds, s);
    case IQ3_S: return launch_qmv_type<IQ3_S>(a, gl, mr, xs, grid, threads, lds, s);
    case IQ3_XXS: return launch_qmv_type<IQ3_XXS>(a, gl, mr, xs, grid, threads, lds, s);
    case IQ2_XXS: return launch_qmv_type<IQ2_XXS>(a, gl, mr, xs, grid, threads, lds, s);
    case IQ2_XS: return launch_qmv_type<IQ2_XS>(a, gl, mr, xs, grid, threads, lds, s);
    case IQ2_S: return launch_qmv_type<IQ2_S>(a, gl, mr, xs, grid, threads, lds, s);
    case IQ1_S: return launch_qmv_type<IQ1_S>(a, gl, mr, xs, grid, threads, lds, s);
    case IQ1_M: return launch_qmv_type<IQ1_M>(a, gl, mr, xs, grid, threads, lds, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gsq
