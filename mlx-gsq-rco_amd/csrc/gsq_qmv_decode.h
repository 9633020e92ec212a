// The QMV kernels' shared pieces: launch arguments, activation registers, the per-type
// decoders (decode of one 32-weight group into fp16 pairs, accumulated with v_dot2_f32_f16 or,
// through the XQuad overload of dacc, with 4x4x4 MFMAs), the ring DMA and the wave reductions.
// Included by gsq_qmv.hip (the vector kernels) and gsq_qmq.hip (the quad-row kernels).
#pragma once
#include "gsq_common.h"

namespace gsq {

struct QmvArgs {
  const uint8_t* packed;
  const void* x;
  void* y;
  int64_t N;
  int K, M, x_dtype, y_dtype;
  int row_bytes;    // packed bytes per row
  int nblk;         // superblocks per row (K / 256)
  int nslices;      // slices per row, ceil(nblk / 8)
  int W;            // waves per row slot (the row's slices split GL per wave)
  int slots;        // row slots per workgroup
  int rows_per_wg;
  int nb;           // ring depth per wave (items)
  int sbuf;         // bytes per ring buffer (cdma KB)
  int cdma;         // DMA instructions per item
  int fill;         // most ring items issued per main-loop step (per item pair: 2 x fill)
  int pair;         // items decoded in pairs (the PR variant of qmv_kernel)
  int qtype;        // the type id (read by the kernel over two products of any types)
  int tbl_bytes, x_off, x_bytes, x_lds, red_off, ring_off;  // LDS layout
  int conv_lds, conv_off;  // prefetched convolution inputs (16 bytes per row of the workgroup)
  int gran;         // quad-row kernel: 16-byte granules per row of an item buffer
  DevTables tb;
  QmvPre pre;       // fused activation prologue (one fp16 row)
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

// Activations of one 32-weight group for MR activation rows: 16 fp16 pairs (hi parts), the
// lo parts for split-precision inputs, and NS partial sums the type's offset terms need
// (NS=1: all 32, NS=2: the two halves of 16, NS=4: the four runs of 8).
template <int MR, bool XS, int NS>
struct XReg {
  uint32_t h[MR][16];
  uint32_t l[MR][XS ? 16 : 1];
  float s8[MR][NS > 0 ? NS : 1];
};

template <int MR, bool XS, int NS>
__device__ __forceinline__ void dacc(uint32_t w, const XReg<MR, XS, NS>& x, int i, float (&acc)[MR]) {
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    acc[m] = dot2(w, x.h[m][i], acc[m]);
    if constexpr (XS) acc[m] = dot2(w, x.l[m][i], acc[m]);
  }
}

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Activations of one 32-weight group in the layout of v_mfma_f32_4x4x4_16b_f16 (16 blocks of 4
// lanes; lane 4b + r supplies row r of block b's 4 x 4 A operand and column r of its B operand,
// and receives column r of its result): lane 4b + r decodes weight row r of a row quad at the
// group of block b and holds h[t] = the 16 fp16 pairs of activation row 4t + r at that group, in
// the type's pairing, with s8 = the group's partial sums of all 4 NQ activation rows (the
// decoders' offset terms). pend holds the first weight pair of the MFMA being formed.
template <int NQ, int NS>
struct XQuad {
  uint32_t h[NQ][16];
  float s8[4 * NQ][NS > 0 ? NS : 1];
  mutable uint32_t pend;
};

// The decoders hand over their weight pairs in order, pairs 2j and 2j + 1 consecutively into
// the same accumulators; each second pair completes the four weights of one MFMA per
// activation quad t, whose result column gives lane 4b + r the products of weight row r with
// activation rows 4t .. 4t + 3 in acc[4t .. 4t + 3].
template <int MR, bool XS, int NQ, int NS>
__device__ __forceinline__ void dacc(uint32_t w, const XQuad<NQ, NS>& x, int i, float (&acc)[MR]) {
  static_assert(MR == 4 * NQ && !XS, "four activation rows per quad, fp16 activations");
  if ((i & 1) == 0) {
    x.pend = w;
    return;
  }
  const uint32_t bw[2] = {x.pend, w};
  const half4_t b = __builtin_bit_cast(half4_t, bw);
#pragma unroll
  for (int t = 0; t < NQ; ++t) {
    const uint32_t aw[2] = {x.h[t][i - 1], x.h[t][i]};
    f32x4_t d = {acc[4 * t], acc[4 * t + 1], acc[4 * t + 2], acc[4 * t + 3]};
    d = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, aw), b, d, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[4 * t + e] = d[e];
  }
}

// Q6_K's 6-bit codes, each under 1024's exponent byte (a byte permute puts 0x64 above each code
// byte), become exact normal fp16 integers for v_dot2_f32_f16 by one exact v_pk_add_f16 that
// removes the 1024. The bare code bits would be the fp16 subnormals q * 2^-24, but
// v_dot2_f32_f16 does not form products of subnormal operands exactly on gfx950 (measured:
// relative errors up to ~5e-5 per product, far more once accumulated), while every product of
// normal fp16 values is exact in fp32.
__device__ __forceinline__ uint32_t unbias_codes(uint32_t biased) {
  const half2_t r = __builtin_bit_cast(half2_t, biased) - (half2_t){(_Float16)1024.f, (_Float16)1024.f};
  return __builtin_bit_cast(uint32_t, r);
}

typedef unsigned short ushort2_t __attribute__((ext_vector_type(2)));

// Views of an LDS table of 8- or 16-byte entries read as scalar words (the compiler merges
// them into ds_read_b64/b128). Vector-typed LDS loads would make the compiler drain every
// in-flight LDS DMA before each table read.
struct LdsV2 {
  const uint8_t* p;
  __device__ __forceinline__ uint2 operator[](uint32_t i) const {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p + 8 * i);
    return make_uint2(q[0], q[1]);
  }
};
struct LdsV4 {
  const uint8_t* p;
  __device__ __forceinline__ uint4 operator[](uint32_t i) const {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p + 16 * i);
    return make_uint4(q[0], q[1], q[2], q[3]);
  }
};

// Sign bits applied with bit operations: bit k of a group's 32 sign bits flips weight k. The fp16
// pair of weights 2w, 2w+1 takes its sign bits (15 and 31) from bits 2w and 2w+1: two packed
// 16-bit halves [bits 0-15 | bits 1-16] and [bits 16-31 | bits 17-31] of the sign word, shifted
// left by 15 - 2(w mod 8) per half, put those bits at 15 and 31; v_bfi then replaces the sign
// bits of the codebook pair (codebook values are positive, so this equals the XOR of a mask).
struct SignBits {
  uint32_t z[2];
  __device__ __forceinline__ explicit SignBits(uint32_t s) {
    const uint32_t t = s >> 1;
    z[0] = __builtin_amdgcn_perm(t, s, 0x05040100u);
    z[1] = __builtin_amdgcn_perm(t, s, 0x07060302u);
  }
  template <int W>
  __device__ __forceinline__ uint32_t apply(uint32_t g) const {
    constexpr unsigned short sh = 15 - 2 * (W & 7);
    const uint32_t m = __builtin_bit_cast(uint32_t, __builtin_bit_cast(ushort2_t, z[W >> 3]) << (ushort2_t){sh, sh});
    return (m & 0x80008000u) | (g & 0x7FFF7FFFu);
  }
};

// ---- per-type decode + dot -----------------------------------------------------------
// Qmv<T>::kTbl is the size of the type's table image, an exact byte image prepared on the host
// (build_qmv_table in gsq_qmv.hip); its first kLds bytes are copied into LDS with DMA at kernel start.
// Codebooks are fp16; sign tables hold XOR masks that flip the fp16 sign bits of a pair of
// codebook values.
template <int T> struct Qmv;

// K-quant codes of at most 4 bits go into the top mantissa bits of fp16 1.0: a 4-bit code q at
// mantissa bits 6-9 is 1 + q/16, a 2-bit code at bits 8-9 is 1 + q/4. Each is a normal fp16
// number, so every product with an fp16 activation is exact in v_dot2_f32_f16 (which does not
// form products of subnormal operands exactly on gfx950), and placing a code pair costs one
// shift and one and-or, with no subtraction. The 1 is removed per group through the activation
// sums: sum x (1 + q/16) = S + sum x q / 16, where S and sum x q / 16 are of the same size
// (about one bit cancels, against ten for codes below an exponent of 1024).
template <> struct Qmv<Q4_K> {
  static constexpr int kPair = PAIR_K;
  static constexpr int kSums = 1;
  static constexpr int kTbl = 0;
  static constexpr int kLds = kTbl;  // bytes of it the QMV decoder keeps in LDS
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t*, const X& x,
                             float (&out)[MR]) {
    uint32_t h[4];
    lds_words<4, A4>(buf, off, h);  // d, dmin, 12 scale bytes (k_decode.py:38-46)
    const float d = h2f(h[0] & 0xFFFFu), dmin = h2f(h[0] >> 16);
    const uint32_t j8 = 8u * (g & 3);
    const uint32_t A = bfe(h[1], j8, 8), B = bfe(h[2], j8, 8), C = bfe(h[3], j8, 8);
    const bool lo = g < 4;
    const uint32_t sc = lo ? (A & 63u) : ((C & 15u) | ((A >> 6) << 4));
    const uint32_t mn = lo ? (B & 63u) : ((C >> 4) | ((B >> 6) << 4));
    uint32_t q[8];
    lds_words<8, A4>(buf, off + 16 + 32 * (g >> 1), q);
    // the group's nibble of bytes 0, 2 (pair 2k) and bytes 1, 3 (pair 2k + 1) of word k moved to
    // bits 6-9 of each half: even groups use the low nibbles, odd groups the high ones
    const bool odd = g & 1;
    const uint32_t sa = odd ? 2u : 6u, sb = odd ? 6u : 2u;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      dacc<MR, XS>(((q[k] << sa) & 0x03C003C0u) | 0x3C003C00u, x, 2 * k, acc);
      dacc<MR, XS>(((q[k] >> sb) & 0x03C003C0u) | 0x3C003C00u, x, 2 * k + 1, acc);
    }
    // d sc sum x q - dmin mn S = 16 d sc acc - (16 d sc + dmin mn) S
    const float s = 16.f * d * (float)sc;
    const float o = -(s + dmin * (float)mn);
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += s * acc[m] + o * x.s8[m][0];
  }
};

template <> struct Qmv<Q2_K> {
  static constexpr int kPair = PAIR_K;
  static constexpr int kSums = 2;
  static constexpr int kTbl = 0;
  static constexpr int kLds = kTbl;  // bytes of it the QMV decoder keeps in LDS
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t*, const X& x,
                             float (&out)[MR]) {
    const uint32_t sm = lds_u16(buf, off + 2 * g);
    const uint32_t dd = lds_w32<A4>(buf, off + 80);
    const float d = h2f(dd & 0xFFFFu), dmin = h2f(dd >> 16);
    uint32_t q[8];
    lds_words<8, A4>(buf, off + 16 + 32 * (g >> 2), q);
    // the group's 2-bit field of bytes 0, 2 and of bytes 1, 3 moved to bits 8-9 of each half
    const uint32_t sh = 2u * (g & 3), sa = 8u - sh;
    float a0[MR], a1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) { a0[m] = 0.f; a1[m] = 0.f; }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t A = ((q[k] << sa) & 0x03000300u) | 0x3C003C00u;
      const uint32_t B = ((q[k] >> sh) & 0x03000300u) | 0x3C003C00u;
      if (k < 4) { dacc<MR, XS>(A, x, 2 * k, a0); dacc<MR, XS>(B, x, 2 * k + 1, a0); }
      else { dacc<MR, XS>(A, x, 2 * k, a1); dacc<MR, XS>(B, x, 2 * k + 1, a1); }
    }
    // per half h: d sc_h sum x q - dmin mn_h S_h = 4 d sc_h acc_h - (4 d sc_h + dmin mn_h) S_h
    const float s0 = 4.f * d * (float)(sm & 15u), s1 = 4.f * d * (float)((sm >> 8) & 15u);
    const float o0 = -(s0 + dmin * (float)((sm >> 4) & 15u));
    const float o1 = -(s1 + dmin * (float)((sm >> 12) & 15u));
#pragma unroll
    for (int m = 0; m < MR; ++m)
      out[m] += s0 * a0[m] + s1 * a1[m] + o0 * x.s8[m][0] + o1 * x.s8[m][1];
  }
};

template <> struct Qmv<Q6_K> {
  static constexpr int kPair = PAIR_K;
  static constexpr int kSums = 2;
  static constexpr int kTbl = 0;
  static constexpr int kLds = kTbl;  // bytes of it the QMV decoder keeps in LDS
  // Group g = plane g % 4 of 128-weight chunk g / 4: weight e takes nibble plane / 2 of ql byte
  // 64 chunk + 32 (plane % 2) + e and bits 2 plane of qh byte 128 + 32 chunk + e (k_decode.py:
  // 51-64). Each word of 4 weights is one funnel shift out of the ql stream (nibble to bits
  // 0-3 of every byte) and one out of the qh stream (2 bits to bits 4-5), which also absorbs
  // the superblock's 2-byte alignment; the 6-bit codes then assemble bytewise and two byte
  // permutes spread them into the fp16 code pairs (elements 0, 2 and 1, 3), with the exponent
  // byte of 1024 above each code.
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t*, const X& x,
                             float (&out)[MR]) {
    const int chunk = g >> 2, plane = g & 3;
    const uint32_t lbit = 8u * (off + 64 * chunk + 32 * (plane & 1)) + 4u * (plane >> 1);
    const uint32_t hbit = 8u * (off + 128 + 32 * chunk) + 2u * plane - 4u;  // bits 2 plane -> 4
    const uint32_t* pl = reinterpret_cast<const uint32_t*>(buf + ((lbit >> 5) << 2));
    const uint32_t* ph = reinterpret_cast<const uint32_t*>(buf + ((hbit >> 5) << 2));
    const uint32_t nl = lbit & 31u, nh = hbit & 31u;
    uint32_t wl[9], wh[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) { wl[i] = pl[i]; wh[i] = ph[i]; }
    const uint32_t sc2 = lds_u16(buf, off + 192 + 2 * g);
    const float d = h2f(lds_u16(buf, off + 208));
    float a0[MR], a1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) { a0[m] = 0.f; a1[m] = 0.f; }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t L = __builtin_amdgcn_alignbit(wl[k + 1], wl[k], nl);
      const uint32_t H = __builtin_amdgcn_alignbit(wh[k + 1], wh[k], nh);
      const uint32_t C = (L & 0x0F0F0F0Fu) | (H & 0x30303030u);
      // code bytes 0, 2 (A) and 1, 3 (B) under 1024's exponent byte 0x64, then 1024 removed
      const uint32_t A = unbias_codes(__builtin_amdgcn_perm(0x64646464u, C, 0x04020400u));
      const uint32_t B = unbias_codes(__builtin_amdgcn_perm(0x64646464u, C, 0x04030401u));
      if (k < 4) { dacc<MR, XS>(A, x, 2 * k, a0); dacc<MR, XS>(B, x, 2 * k + 1, a0); }
      else { dacc<MR, XS>(A, x, 2 * k, a1); dacc<MR, XS>(B, x, 2 * k + 1, a1); }
    }
    const float s0 = d * (float)(int)(int8_t)(sc2 & 0xFFu), s1 = d * (float)(int)(int8_t)(sc2 >> 8);
#pragma unroll
    for (int m = 0; m < MR; ++m)
      out[m] += s0 * (a0[m] - 32.f * x.s8[m][0]) + s1 * (a1[m] - 32.f * x.s8[m][1]);
  }
};

template <> struct Qmv<IQ4_XS> {
  static constexpr int kPair = PAIR_16;
  static constexpr int kSums = 0;
  static constexpr int kTbl = 1024;  // 256 fp16 pairs (kvalues[lo nibble], kvalues[hi nibble])
  static constexpr int kLds = kTbl;  // bytes of it the QMV decoder keeps in LDS
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const X& x,
                             float (&out)[MR]) {
    const uint32_t hd = lds_w32<A4>(buf, off);
    const float d = h2f(hd & 0xFFFFu);
    const uint32_t low = (lds_u8(buf, off + 4 + (g >> 1)) >> (4 * (g & 1))) & 15u;
    const uint32_t high = ((hd >> 16) >> (2 * g)) & 3u;
    const int scale = (int)(low | (high << 4)) - 32;
    uint32_t q[4];
    lds_words<4, A4>(buf, off + 8 + 16 * g, q);
    const uint32_t* t = reinterpret_cast<const uint32_t*>(tbl);
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    uint32_t v[16];  // all sixteen value-pair reads of the group in flight before the first use
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) v[4 * k + i] = t[bfe(q[k], 8 * i, 8)];
#pragma unroll
    for (int j = 0; j < 16; ++j) dacc<MR, XS>(v[j], x, j, acc);
    const float s = d * (float)scale;
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += s * acc[m];
  }
};

// Signed half-entry tables (IQ3_S, IQ3_XXS, IQ2_XXS): four codebook values with the signs of
// one sign nibble applied, for every (entry, nibble) pair, 8 bytes each: a lookup by (entry,
// nibble) yields the signed fp16 pairs directly, with no sign-mask reads and no XORs (each 8
// weights cost two 8-byte reads, the bytes of the unsigned entry). Entry-major: byte offset
// (entry << 7 | nibble << 3) for 4-value entries, (entry << 8 | half << 7 | nibble << 3) for
// 8-value entries, half 0 holding values 0-3.
struct LdsV2Off {
  const uint8_t* p;
  __device__ __forceinline__ uint2 at(uint32_t byte_off) const {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p + byte_off);
    return make_uint2(q[0], q[1]);
  }
};

// Sign byte of a ksigns field from the table's closed form (entry i = i with bit 7 the parity
// of i; the library rejects any other table): k7 | popcount(k7) << 7. Bits 8-9 of the result
// hold the rest of the popcount, which the callers mask off.
__device__ __forceinline__ uint32_t ksign_byte(uint32_t k7) {
  return k7 | (__builtin_amdgcn_ubfe(__builtin_popcount(k7), 0, 3) << 7);
}

template <> struct Qmv<IQ3_S> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kSums = 0;
  // signed table: 512 entries x 16 sign nibbles x 4 fp16 values
  static constexpr int kTbl = 512 * 16 * 8;
  static constexpr int kLds = kTbl;  // bytes of it the QMV decoder keeps in LDS
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const X& x,
                             float (&out)[MR]) {
    const float d = h2f(lds_u16(buf, off));
    const uint32_t snib = (lds_u8(buf, off + 106 + (g >> 1)) >> (4 * (g & 1))) & 15u;
    const float db = d * (float)(1u + 2u * snib);
    uint32_t q[2];
    lds_words<2, A4>(buf, off + 2 + 8 * g, q);
    const uint32_t qh = lds_u8(buf, off + 66 + g);
    const uint32_t sg = lds_w32<A4>(buf, off + 74 + 4 * g);
    const LdsV2Off t{tbl};
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    uint2 Gs[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {  // all table reads of the group in flight before the first use
      // entry (qs byte | qh bit e << 8) << 7 | sign nibble e << 3 (iq3_s_decode.py:25-33)
      const uint32_t hi = ((qh << (15 - e)) & 0x8000u) | (bfe(q[e >> 2], 8 * (e & 3), 8) << 7);
      const uint32_t nb = e == 0 ? (sg << 3) & 0x78u : (sg >> (4 * e - 3)) & 0x78u;
      Gs[e] = t.at(hi | nb);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dacc<MR, XS>(Gs[e].x, x, 2 * e, acc);
      dacc<MR, XS>(Gs[e].y, x, 2 * e + 1, acc);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += db * acc[m];
  }
};

template <> struct Qmv<IQ3_XXS> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kSums = 0;
  // signed table: 256 entries x 16 sign nibbles x 4 fp16 values
  static constexpr int kTbl = 256 * 16 * 8;
  static constexpr int kLds = kTbl;  // bytes of it the QMV decoder keeps in LDS
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const X& x,
                             float (&out)[MR]) {
    const float dh = h2f(lds_u16(buf, off));
    uint32_t q[2];
    lds_words<2, A4>(buf, off + 2 + 8 * g, q);
    const uint32_t u = lds_w32<A4>(buf, off + 66 + 4 * g);
    const float d = dh * (0.5f + (float)(u >> 28)) * 0.5f;
    const LdsV2Off t{tbl};
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    uint2 G0[4], G1[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) {  // all table reads of the group in flight before the first use
      const uint32_t s8 = ksign_byte(bfe(u, 7 * l, 7));
      G0[l] = t.at((bfe(q[l >> 1], 16 * (l & 1), 8) << 7) | ((s8 << 3) & 0x78u));
      G1[l] = t.at((bfe(q[l >> 1], 16 * (l & 1) + 8, 8) << 7) | ((s8 >> 1) & 0x78u));
    }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      dacc<MR, XS>(G0[l].x, x, 4 * l, acc);
      dacc<MR, XS>(G0[l].y, x, 4 * l + 1, acc);
      dacc<MR, XS>(G1[l].x, x, 4 * l + 2, acc);
      dacc<MR, XS>(G1[l].y, x, 4 * l + 3, acc);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += d * acc[m];
  }
};

template <> struct Qmv<IQ2_XXS> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kSums = 0;
  // signed table: 256 entries x 2 halves x 16 sign nibbles x 4 fp16 values
  static constexpr int kTbl = 256 * 2 * 16 * 8;
  static constexpr int kLds = kTbl;  // bytes of it the QMV decoder keeps in LDS
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const X& x,
                             float (&out)[MR]) {
    const float dh = h2f(lds_u16(buf, off));
    uint32_t q[2];
    lds_words<2, A4>(buf, off + 2 + 8 * g, q);
    const uint32_t u = q[1];
    const float d = dh * (0.5f + (float)(u >> 28)) * 0.25f;
    const LdsV2Off t{tbl};
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    uint2 G0[4], G1[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) {  // all table reads of the group in flight before the first use
      const uint32_t s8 = ksign_byte(bfe(u, 7 * l, 7));
      const uint32_t eb = bfe(q[0], 8 * l, 8) << 8;
      G0[l] = t.at(eb | ((s8 << 3) & 0x78u));
      G1[l] = t.at((eb | 128u) | ((s8 >> 1) & 0x78u));
    }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      dacc<MR, XS>(G0[l].x, x, 4 * l, acc);
      dacc<MR, XS>(G0[l].y, x, 4 * l + 1, acc);
      dacc<MR, XS>(G1[l].x, x, 4 * l + 2, acc);
      dacc<MR, XS>(G1[l].y, x, 4 * l + 3, acc);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += d * acc[m];
  }
};

// Sign masks of one ksigns field (8 weights, 4 words) for IQ2_XS: the sign byte from the
// table's closed form (two instructions), and its two nibbles index the 16 nibble masks of two
// words each, a 128-byte table whose reads never conflict (16-byte masks read at random from a
// 2 KB table put the LDS ~40% of the time in bank conflicts). IQ2_XS's 512-entry codebook is too
// large for a signed half-entry table (128 KB).
__device__ __forceinline__ uint4 ksigns_masks(const uint8_t* nib, uint32_t k7) {
  const uint32_t s8 = k7 | ((__builtin_popcount(k7) & 1u) << 7);
  const LdsV2 nm{nib};
  const uint2 lo = nm[s8 & 15u], hi = nm[s8 >> 4];
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

template <> struct Qmv<IQ2_XS> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kSums = 0;
  static constexpr int kGridB = 512 * 8 * 2;
  static constexpr int kTbl = kGridB + 16 * 8;  // grid, then 16 nibble sign masks
  static constexpr int kLds = kTbl;             // bytes of it the QMV decoder keeps in LDS
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const X& x,
                             float (&out)[MR]) {
    const float dh = h2f(lds_u16(buf, off));
    uint32_t q[2];
    lds_words<2, A4>(buf, off + 2 + 8 * g, q);
    const uint32_t sb = lds_u8(buf, off + 66 + g);
    const LdsV4 grid{tbl};
    float a0[MR], a1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) { a0[m] = 0.f; a1[m] = 0.f; }
    uint4 Ms[4], Gs[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) {  // all table reads of the group in flight before the first use
      Ms[l] = ksigns_masks(tbl + kGridB, bfe(q[l >> 1], 16 * (l & 1) + 9, 7));
      Gs[l] = grid[bfe(q[l >> 1], 16 * (l & 1), 9)];
    }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint4 M = Ms[l], G = Gs[l];
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
  static constexpr int kSums = 0;
  static constexpr int kGridB = 1024 * 8 * 2;
  // image: the grid; QMV applies the signs with bit operations (SignBits: a third fewer LDS
  // reads per group, 0-2% faster than nibble masks)
  static constexpr int kTbl = kGridB;
  static constexpr int kLds = kGridB;
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const X& x,
                             float (&out)[MR]) {
    const float dh = h2f(lds_u16(buf, off));
    const uint32_t qs = lds_w32<A4>(buf, off + 2 + 4 * g);
    const uint32_t sg = lds_w32<A4>(buf, off + 34 + 4 * g);
    const uint32_t qh = lds_u8(buf, off + 66 + g);
    const uint32_t sb = lds_u8(buf, off + 74 + g);
    const LdsV4 grid{tbl};
    float a0[MR], a1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) { a0[m] = 0.f; a1[m] = 0.f; }
    uint4 Gs[4];
#pragma unroll
    for (int l = 0; l < 4; ++l)  // all table reads of the group in flight before the first use
      Gs[l] = grid[bfe(qs, 8 * l, 8) | (bfe(qh, 2 * l, 2) << 8)];
    const SignBits sbits(sg);
    dacc<MR, XS>(sbits.apply<0>(Gs[0].x), x, 0, a0);   dacc<MR, XS>(sbits.apply<1>(Gs[0].y), x, 1, a0);
    dacc<MR, XS>(sbits.apply<2>(Gs[0].z), x, 2, a0);   dacc<MR, XS>(sbits.apply<3>(Gs[0].w), x, 3, a0);
    dacc<MR, XS>(sbits.apply<4>(Gs[1].x), x, 4, a0);   dacc<MR, XS>(sbits.apply<5>(Gs[1].y), x, 5, a0);
    dacc<MR, XS>(sbits.apply<6>(Gs[1].z), x, 6, a0);   dacc<MR, XS>(sbits.apply<7>(Gs[1].w), x, 7, a0);
    dacc<MR, XS>(sbits.apply<8>(Gs[2].x), x, 8, a1);   dacc<MR, XS>(sbits.apply<9>(Gs[2].y), x, 9, a1);
    dacc<MR, XS>(sbits.apply<10>(Gs[2].z), x, 10, a1); dacc<MR, XS>(sbits.apply<11>(Gs[2].w), x, 11, a1);
    dacc<MR, XS>(sbits.apply<12>(Gs[3].x), x, 12, a1); dacc<MR, XS>(sbits.apply<13>(Gs[3].y), x, 13, a1);
    dacc<MR, XS>(sbits.apply<14>(Gs[3].z), x, 14, a1); dacc<MR, XS>(sbits.apply<15>(Gs[3].w), x, 15, a1);
    const float d0 = dh * (0.5f + (float)(sb & 15u)) * 0.25f, d1 = dh * (0.5f + (float)(sb >> 4)) * 0.25f;
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += d0 * a0[m] + d1 * a1[m];
  }
};

template <> struct Qmv<IQ1_S> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kSums = 1;
  static constexpr int kTbl = 2048 * 8 * 2;
  static constexpr int kLds = kTbl;  // bytes of it the QMV decoder keeps in LDS
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const X& x,
                             float (&out)[MR]) {
    const float dh = h2f(lds_u16(buf, off));
    const uint32_t qs = lds_w32<A4>(buf, off + 2 + 4 * g);
    const uint32_t h = lds_u16(buf, off + 34 + 2 * g);
    const float d = dh * (float)(2u * ((h >> 12) & 7u) + 1u);
    const float delta = (h & 0x8000u) ? -0.125f : 0.125f;
    const LdsV4 grid{tbl};
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    uint4 Gs[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) Gs[l] = grid[bfe(qs, 8 * l, 8) | (bfe(h, 3 * l, 3) << 8)];
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint4 G = Gs[l];
      dacc<MR, XS>(G.x, x, 4 * l, acc); dacc<MR, XS>(G.y, x, 4 * l + 1, acc);
      dacc<MR, XS>(G.z, x, 4 * l + 2, acc); dacc<MR, XS>(G.w, x, 4 * l + 3, acc);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float xs = x.s8[m][0];
      out[m] += d * (acc[m] + delta * xs);
    }
  }
};

// IQ1_M's image holds every codebook entry twice, with its delta added (iq_lookup_decode.py:
// 31-37: w = d (2 s + 1) (grid + delta), delta = -0.125 when bit 3 of the entry's qh nibble is
// set, else +0.125): entry (nibble << 8 | qs byte) is grid[qs | (nibble & 7) << 8] + delta, so
// the whole 4-bit nibble indexes it and the group needs no per-entry delta term (values
// +-0.125 / 0.875 / 1.125 for the published codebook, exact in fp16; the library refuses a
// codebook for which grid +- 0.125 is not exact).
template <> struct Qmv<IQ1_M> {
  static constexpr int kPair = PAIR_NAT;
  static constexpr int kSums = 0;
  static constexpr int kTbl = 2 * 2048 * 8 * 2;
  static constexpr int kLds = kTbl;  // bytes of it the QMV decoder keeps in LDS
  template <int MR, bool XS, bool A4, class X>
  __device__ static void dot(const uint8_t* buf, uint32_t off, int g, const uint8_t* tbl, const X& x,
                             float (&out)[MR]) {
    const uint32_t qs = lds_w32<A4>(buf, off + 4 * g);
    const uint32_t qh = lds_u16(buf, off + 32 + 2 * g);
    uint32_t w[2];
    lds_words<2, A4>(buf, off + 48, w);
    // d: the top nibbles of the four scale words (iq_lookup_decode.py:34-35)
    const uint32_t dbits = ((w[0] >> 12) & 0xFu) | ((w[0] >> 24) & 0xF0u) | ((w[1] >> 4) & 0xF00u) |
                           ((w[1] >> 16) & 0xF000u);
    const float d = h2f(dbits);
    const uint32_t ww = lds_u16(buf, off + 48 + 2 * (g >> 1));  // this group's scale word
    const uint32_t sh0 = 6u * (g & 1);
    const float d0 = d * (float)(2u * ((ww >> sh0) & 7u) + 1u);
    const float d1 = d * (float)(2u * ((ww >> (sh0 + 3)) & 7u) + 1u);
    const LdsV4 grid{tbl};
    float a0[MR], a1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) { a0[m] = 0.f; a1[m] = 0.f; }
    uint4 Gs[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) Gs[l] = grid[bfe(qs, 8 * l, 8) | (bfe(qh, 4 * l, 4) << 8)];
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint4 G = Gs[l];
      if (l < 2) {
        dacc<MR, XS>(G.x, x, 4 * l, a0); dacc<MR, XS>(G.y, x, 4 * l + 1, a0);
        dacc<MR, XS>(G.z, x, 4 * l + 2, a0); dacc<MR, XS>(G.w, x, 4 * l + 3, a0);
      } else {
        dacc<MR, XS>(G.x, x, 4 * l, a1); dacc<MR, XS>(G.y, x, 4 * l + 1, a1);
        dacc<MR, XS>(G.z, x, 4 * l + 2, a1); dacc<MR, XS>(G.w, x, 4 * l + 3, a1);
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] += d0 * a0[m] + d1 * a1[m];
  }
};

// ---- staging ------------------------------------------------------------------------
// DMA of the whole 16-byte granules covering [start, start + bytes) into LDS at dst with
// exactly n wave instructions (lane i of instruction j writes dst + (64 j + i) * 16, so dst
// must hold n KB). Lanes past the last granule reload the first one into their own slot,
// which keeps the instruction count fixed. A granule that holds any byte of a tensor lies in
// the same memory page as that byte, so the granules at an unaligned start or end of the
// packed matrix are read whole; their bytes outside the matrix are never used.
__device__ __forceinline__ void dma_item(uintptr_t start, int bytes, int n, uint8_t* dst, int lane) {
  const uintptr_t A0 = start & ~(uintptr_t)15;
  const int ngran = (int)((start + (uintptr_t)bytes + 15 - A0) >> 4);
  for (int j = 0; j < n; ++j) {
    const int c = j * 64 + lane;
    const uintptr_t src = A0 + (uintptr_t)(c < ngran ? c : 0) * 16;
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src),
                                     (__attribute__((address_space(3))) void*)(dst + j * 1024), 16, 0, 0);
  }
}


// Issue priority of this wave by progress: 3 - min(steps done, 3). A SIMD's arbiter issues
// from the highest-priority wave, the oldest among equals; left at one priority, the three
// waves of a SIMD finish one after the other (oldest first) and the last runs its final
// items alone, with nothing to cover its LDS and memory latency. Lowering the priority of
// the waves that are ahead keeps the three in step to the end (1-11% faster on the 27B
// shapes; the 1024-row products, one or two items per wave, skip it).
__device__ __forceinline__ void set_progress_prio(int steps_done) {
  if (steps_done <= 0) __builtin_amdgcn_s_setprio(3);
  else if (steps_done == 1) __builtin_amdgcn_s_setprio(2);
  else if (steps_done == 2) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
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
  else if (dt == DT_BF16) reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)f32_to_bf16_bits(v);
  else reinterpret_cast<float*>(y)[i] = v;
}

// Full-wave sum with DPP row operations; the total lands in lane 63.
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

// fp16 x[e0] (low half) and x[e1] (high half) out of the 16 words holding x[0..31], by one
// byte permute (v_perm_b32 selector bytes 0-3 pick the second source, 4-7 the first).
__device__ __forceinline__ uint32_t half_pair(const uint32_t (&w)[16], int e0, int e1) {
  const uint32_t b0 = 2u * (uint32_t)(e0 & 1), b2 = 4u + 2u * (uint32_t)(e1 & 1);
  const uint32_t sel = b0 | ((b0 + 1u) << 8) | (b2 << 16) | ((b2 + 1u) << 24);
  return __builtin_amdgcn_perm(w[e1 >> 1], w[e0 >> 1], sel);
}

// The type's table image in static LDS (at LDS address 0, a constant the table reads fold into
// their address arithmetic); the rest of the layout is dynamic LDS behind it.
template <int B>
struct QmvTblLds {
  __device__ __forceinline__ static uint8_t* get() {
    __shared__ __attribute__((aligned(16))) uint8_t t[B];
    return t;
  }
};
template <>
struct QmvTblLds<0> {
  __device__ __forceinline__ static uint8_t* get() { return nullptr; }
};

}  // namespace gsq
