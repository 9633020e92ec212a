// fp16 decode of one MFMA B-operand fragment slice: eight consecutive weights (octet
// kq = 0..3 of group g = 0..7) of one superblock held in LDS, as four fp16 pairs.
//
// Each weight is the reference decoder's value (mlx_gsq/runtime/kernels/k_decode.py:18-80,
// iq_lookup_decode.py:6-39, iq3_s_decode.py:16-40) rounded to fp16 (the reference QMM's
// decoded tile is half, qmm.py:181). One v_fma_mix per weight forms scale * code + offset
// exactly and rounds it once to fp16 (round to nearest even):
//  * K-quant and IQ4_XS codes enter as fp16 subnormals (bits = the code, value code * 2^-24)
//    against a scale multiplied by 2^24, so the product is the exact integer multiple;
//  * codebook types read the fp16 codebook entries directly and flip signs with XOR masks
//    of fp16 pairs, from the same LDS table image as the QMV kernel.
// For Q6_K, IQ4_XS and every product of the real codebooks the float32 value is exact, so
// this is the reference's fp16 tile bit for bit; where the reference's float32 expression
// rounds (Q2_K / Q4_K's d*sc*q - dmin*m, products with arbitrary codebook values) the
// single rounding can differ from its float32-then-fp16 double rounding by one fp16 ulp when
// the float32 value falls on an fp16 tie.
//
// The superblock sits at byte `sd` (2-byte aligned; A4: 4-byte aligned) of its 16-byte aligned
// LDS row slot `sb`: word reads take the aligned slot address and funnel-shift by sd's low bits
// (LDS reads at 2-byte aligned addresses are served, but stall). `tbl` points at the type's
// table image: fp16 codebook (entries x coords) followed by its sign masks.
#pragma once
#include "gsq_common.h"

namespace gsq {

// fp16 pair {fma(a, h.lo, c), fma(a, h.hi, c)} with h an fp16 pair and a, c float: each result
// is computed exactly and rounded once (v_fma_mixlo_f16 / v_fma_mixhi_f16). Its result must
// pass through a compiler-visible VALU instruction (the codebook decoders' sign XOR) before an
// MFMA reads it: the compiler inserts no wait states after asm (codes8 carries its own).
// (the host pass never runs this device-only function; the VGPR asm constraints exist only in
// the device compilation)
__device__ __forceinline__ uint32_t mix2(float a, uint32_t h, float c) {
  uint32_t r = 0;
#if defined(__HIP_DEVICE_COMPILE__)
  asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(h), "v"(c));
  asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(r) : "v"(a), "v"(h), "v"(c));
#endif
  return r;
}

// bytes 0,1 (lo) or 2,3 (hi) of q as the two halves of a word (fp16 subnormal codes)
__device__ __forceinline__ uint32_t spread_lo(uint32_t q) { return __builtin_amdgcn_perm(0u, q, 0x0c010c00u); }
__device__ __forceinline__ uint32_t spread_hi(uint32_t q) { return __builtin_amdgcn_perm(0u, q, 0x0c030c02u); }

constexpr float kCode = 16777216.f;  // 2^24: an fp16 subnormal with bits q has value q * 2^-24

// eight byte codes (two words) -> fp16 of a * code + c (a24 = a * 2^24), as the four fp16
// pairs of an MFMA B operand. The results go straight into v_mfma, which may read a VGPR only
// two wait states after a VALU wrote it; the compiler cannot see that an asm statement is a
// VALU write, so the eight conversions are one asm block that ends with those two wait states
// (s_nop 1), and the outputs are early-clobber (written while inputs are still being read).
__device__ __forceinline__ void codes8(const uint32_t (&q)[2], float a24, float c, uint32_t (&o)[4]) {
  const uint32_t h0 = spread_lo(q[0]), h1 = spread_hi(q[0]), h2 = spread_lo(q[1]), h3 = spread_hi(q[1]);
#if defined(__HIP_DEVICE_COMPILE__)
  asm("v_fma_mixlo_f16 %0, %4, %5, %6 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixlo_f16 %1, %4, %7, %6 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixlo_f16 %2, %4, %8, %6 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixlo_f16 %3, %4, %9, %6 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %0, %4, %5, %6 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %1, %4, %7, %6 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %2, %4, %8, %6 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %3, %4, %9, %6 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "s_nop 1"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3])
      : "v"(a24), "v"(h0), "v"(c), "v"(h1), "v"(h2), "v"(h3));
#else
  o[0] = h0; o[1] = h1; o[2] = h2; o[3] = h3; (void)a24; (void)c;
#endif
}

// four fp16 pairs h -> {fma(a, h.lo, c), fma(a, h.hi, c)} as one asm block ending in the two
// wait states an MFMA needs after a VALU write (for results that reach an MFMA directly, with
// no compiler-visible instruction in between); outputs early-clobber, as in codes8.
__device__ __forceinline__ void mix8(float a, const uint32_t (&h)[4], float c, uint32_t (&o)[4]) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm("v_fma_mixlo_f16 %0, %4, %5, %6 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixlo_f16 %1, %4, %7, %6 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixlo_f16 %2, %4, %8, %6 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixlo_f16 %3, %4, %9, %6 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %0, %4, %5, %6 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %1, %4, %7, %6 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %2, %4, %8, %6 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %3, %4, %9, %6 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "s_nop 1"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3])
      : "v"(a), "v"(h[0]), "v"(c), "v"(h[1]), "v"(h[2]), "v"(h[3]));
#else
  o[0] = h[0]; o[1] = h[1]; o[2] = h[2]; o[3] = h[3]; (void)a; (void)c;
#endif
}

__device__ __forceinline__ const uint32_t* tbl_words(const uint8_t* tbl, uint32_t byte_off) {
  return reinterpret_cast<const uint32_t*>(tbl + byte_off);
}

template <int T, bool A4>
struct QmmDec;

// Q2_K (k_decode.py:18-30): w = d*(sm&15)*q - dmin*(sm>>4)
template <bool A4>
struct QmmDec<Q2_K, A4> {
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t*, int g, int kq, uint32_t (&o)[4]) {
    uint32_t q[2];
    lds_words<2, A4>(sb, sd + 16 + (g >> 2) * 32 + 8 * kq, q);
    const int sh = 2 * (g & 3);
    q[0] = (q[0] >> sh) & 0x03030303u;
    q[1] = (q[1] >> sh) & 0x03030303u;
    const uint32_t dd = lds_w32<A4>(sb, sd + 80);
    const uint32_t sm = lds_u8(sb, sd + 2 * g + (kq >> 1));
    const float a = h2f(dd & 0xFFFFu) * (float)(sm & 15u);
    const float b = h2f(dd >> 16) * (float)(sm >> 4);
    codes8(q, a * kCode, -b, o);
  }
};

// Q4_K (k_decode.py:31-50): w = d*sc*q - dmin*mn with 6-bit scales/mins
template <bool A4>
struct QmmDec<Q4_K, A4> {
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t*, int g, int kq, uint32_t (&o)[4]) {
    uint32_t q[2];
    lds_words<2, A4>(sb, sd + 16 + (g >> 1) * 32 + 8 * kq, q);
    const int sh = 4 * (g & 1);
    q[0] = (q[0] >> sh) & 0x0F0F0F0Fu;
    q[1] = (q[1] >> sh) & 0x0F0F0F0Fu;
    uint32_t s[3];
    lds_words<3, A4>(sb, sd + 4, s);
    const uint32_t dd = lds_w32<A4>(sb, sd + 0);
    uint32_t sc, mn;
    const int gg = g & 3;
    if (g < 4) {
      sc = bfe(s[0], 8 * gg, 6);
      mn = bfe(s[1], 8 * gg, 6);
    } else {
      const uint32_t lo = bfe(s[2], 8 * gg, 8);
      sc = (lo & 15u) | (bfe(s[0], 8 * gg + 6, 2) << 4);
      mn = (lo >> 4) | (bfe(s[1], 8 * gg + 6, 2) << 4);
    }
    const float a = h2f(dd & 0xFFFFu) * (float)sc;
    const float b = h2f(dd >> 16) * (float)mn;
    codes8(q, a * kCode, -b, o);
  }
};

// Q6_K (k_decode.py:51-65): w = d*scale*(q - 32), q = low nibble | 2 high bits << 4
template <bool A4>
struct QmmDec<Q6_K, A4> {
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t*, int g, int kq, uint32_t (&o)[4]) {
    const int h = g >> 2, pl = g & 3;
    uint32_t ql[2], qh[2];
    lds_words<2, A4>(sb, sd + h * 64 + (pl & 1) * 32 + 8 * kq, ql);
    lds_words<2, A4>(sb, sd + 128 + h * 32 + 8 * kq, qh);
    const int shl = 4 * (pl >> 1), shh = 2 * pl;
    uint32_t q[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) q[i] = ((ql[i] >> shl) & 0x0F0F0F0Fu) | (((qh[i] >> shh) & 0x03030303u) << 4);
    const int sc = (int)(int8_t)lds_u8(sb, sd + 192 + 2 * g + (kq >> 1));
    const float a = h2f(lds_u16(sb, sd + 208)) * (float)sc;
    codes8(q, a * kCode, -32.f * a, o);
  }
};

// IQ4_XS (k_decode.py:66-80): w = d*scale*kvalues[q]; kvalues + 128 looked up as bytes
template <bool A4>
struct QmmDec<IQ4_XS, A4> {
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t*, int g, int kq, uint32_t (&o)[4]) {
    uint32_t q[2];
    lds_words<2, A4>(sb, sd + 8 + 16 * g + 8 * (kq & 1), q);
    const int sh = 4 * (kq >> 1);
    const uint32_t dw = lds_w32<A4>(sb, sd + 0);
    const uint32_t low = (lds_u8(sb, sd + 4 + g / 2) >> (4 * (g & 1))) & 15u;
    const uint32_t high = ((dw >> 16) >> (2 * g)) & 3u;
    const float a = h2f(dw & 0xFFFFu) * (float)((int)(low | (high << 4)) - 32);
    // kvalues + 128 = {1,24,45,63,79,93,106,118,129,141,153,166,181,197,217,241}
    constexpr uint32_t T0 = 0x3F2D1801u, T1 = 0x766A5D4Fu, T2 = 0xA6998D81u, T3 = 0xF1D9C5B5u;
    uint32_t u[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t c = (q[i] >> sh) & 0x0F0F0F0Fu;
      const uint32_t sel = c & 0x07070707u;
      const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel);
      const uint32_t hi = __builtin_amdgcn_perm(T3, T2, sel);
      const uint32_t m = ((c >> 3) & 0x01010101u) * 0xFFu;
      u[i] = (hi & m) | (lo & ~m);
    }
    codes8(u, a * kCode, -128.f * a, o);
  }
};

// IQ3_S (iq3_s_decode.py:16-40): w = +-d*(1+2*s)*grid[gi][c], 9-bit grid index; sign masks
// per nibble (two words) after the codebook
template <bool A4>
struct QmmDec<IQ3_S, A4> {
  static constexpr uint32_t kGridB = 512 * 4 * 2;
  static constexpr uint32_t kMaskB = kGridB;
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const float d = h2f(lds_u16(sb, sd + 0));
    const uint32_t sbyte = lds_u8(sb, sd + 106 + (g >> 1));
    const float db = d * (float)(1u + 2u * ((sbyte >> (4 * (g & 1))) & 15u));
    const uint32_t qh = lds_u8(sb, sd + 66 + g);
    const uint32_t qq = lds_u16(sb, sd + 2 + 8 * g + 2 * kq);
    const uint32_t i0 = (qq & 0xFFu) | ((qh << (8 - 2 * kq)) & 256u);
    const uint32_t i1 = (qq >> 8) | ((qh << (7 - 2 * kq)) & 256u);
    const uint32_t signs = lds_u8(sb, sd + 74 + 4 * g + kq);
    const uint32_t* e0 = tbl_words(tbl, i0 * 8);
    const uint32_t* e1 = tbl_words(tbl, i1 * 8);
    // nibble masks (16 entries: few distinct LDS addresses per read, unlike the 256 byte masks)
    const uint32_t* m0 = tbl_words(tbl, kMaskB + (signs & 15u) * 8);
    const uint32_t* m1 = tbl_words(tbl, kMaskB + (signs >> 4) * 8);
    o[0] = mix2(db, e0[0], 0.f) ^ m0[0];
    o[1] = mix2(db, e0[1], 0.f) ^ m0[1];
    o[2] = mix2(db, e1[0], 0.f) ^ m1[0];
    o[3] = mix2(db, e1[1], 0.f) ^ m1[1];
  }
};

// one 8-wide codebook entry times d, with four sign-mask pairs (HM) or none; the entry and
// mask words are read before any is used
template <bool HM>
__device__ __forceinline__ void grid8(const uint8_t* tbl, uint32_t qi, float d, float c, const uint32_t* m,
                                      uint32_t (&o)[4]) {
  const uint32_t* e = tbl_words(tbl, qi * 16);
  uint32_t ev[4], mv[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 4; ++i) ev[i] = e[i];
  if constexpr (HM) {
#pragma unroll
    for (int i = 0; i < 4; ++i) mv[i] = m[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = mix2(d, ev[i], c) ^ mv[i];  // the XOR is the visible VALU write
  } else {
    mix8(d, ev, c, o);  // no sign masks: the asm block carries the MFMA wait states itself
  }
}

// Sign masks of one ksigns field (8 weights, 4 words): the sign byte from the ksigns table's
// closed form (entry i = i with bit 7 the parity of i; the library accepts no other table),
// the masks of its two nibbles from the 16-entry nibble-mask table after the codebook, whose
// reads never conflict. Used by IQ3_XXS (11-21% faster than 16-byte masks read from a 2 KB
// table, M = 4..512); IQ2_XXS and IQ2_XS read those 16-byte masks, which follow the nibble
// table in their images (the nibble form was 1-6% slower for them here).
__device__ __forceinline__ void ksigns_masks(const uint8_t* tbl, uint32_t mask_off, uint32_t k7, uint32_t (&m)[4]) {
  const uint32_t s8 = k7 | ((__builtin_popcount(k7) & 1u) << 7);
  const uint32_t* lo = tbl_words(tbl, mask_off + (s8 & 15u) * 8);
  const uint32_t* hi = tbl_words(tbl, mask_off + (s8 >> 4) * 8);
  m[0] = lo[0]; m[1] = lo[1]; m[2] = hi[0]; m[3] = hi[1];
}

// IQ3_XXS (iq_lookup_decode.py:7-12): w = +-d*(0.5+s)*0.5*grid[qi][c], ksigns masks
template <bool A4>
struct QmmDec<IQ3_XXS, A4> {
  static constexpr uint32_t kGridB = 256 * 4 * 2;
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const uint32_t u = lds_w32<A4>(sb, sd + 66 + 4 * g);
    const float d = h2f(lds_u16(sb, sd + 0)) * (0.5f + (float)(u >> 28)) * 0.5f;
    uint32_t m[4];
    ksigns_masks(tbl, kGridB, (u >> (7 * kq)) & 127u, m);
    const uint32_t qq = lds_u16(sb, sd + 2 + 8 * g + 2 * kq);
    const uint32_t* e0 = tbl_words(tbl, (qq & 0xFFu) * 8);
    const uint32_t* e1 = tbl_words(tbl, (qq >> 8) * 8);
    o[0] = mix2(d, e0[0], 0.f) ^ m[0];
    o[1] = mix2(d, e0[1], 0.f) ^ m[1];
    o[2] = mix2(d, e1[0], 0.f) ^ m[2];
    o[3] = mix2(d, e1[1], 0.f) ^ m[3];
  }
};

// IQ2_XXS (iq_lookup_decode.py:23-26)
template <bool A4>
struct QmmDec<IQ2_XXS, A4> {
  static constexpr uint32_t kGridB = 256 * 8 * 2;
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const uint32_t u = lds_w32<A4>(sb, sd + 2 + 8 * g + 4);
    const float d = h2f(lds_u16(sb, sd + 0)) * (0.5f + (float)(u >> 28)) * 0.25f;
    grid8<true>(tbl, lds_u8(sb, sd + 2 + 8 * g + kq), d, 0.f, tbl_words(tbl, kGridB + 16 * 8 + ((u >> (7 * kq)) & 127u) * 16), o);
  }
};

// IQ2_XS (iq_lookup_decode.py:13-17)
template <bool A4>
struct QmmDec<IQ2_XS, A4> {
  static constexpr uint32_t kGridB = 512 * 8 * 2;
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const uint32_t q = lds_u16(sb, sd + 2 + 2 * (4 * g + kq));
    const uint32_t sc = (lds_u8(sb, sd + 66 + g) >> (4 * (kq >> 1))) & 15u;
    const float d = h2f(lds_u16(sb, sd + 0)) * (0.5f + (float)sc) * 0.25f;
    grid8<true>(tbl, q & 511u, d, 0.f, tbl_words(tbl, kGridB + 16 * 8 + (q >> 9) * 16), o);
  }
};

// IQ2_S (iq_lookup_decode.py:18-22): sign masks per nibble (two words) after the codebook
template <bool A4>
struct QmmDec<IQ2_S, A4> {
  static constexpr uint32_t kGridB = 1024 * 8 * 2;
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const int oo = 4 * g + kq;
    const uint32_t hi = (lds_u8(sb, sd + 66 + g) >> (2 * kq)) & 3u;
    const uint32_t qi = lds_u8(sb, sd + 2 + oo) | (hi << 8);
    const uint32_t sc = (lds_u8(sb, sd + 74 + g) >> (4 * (kq >> 1))) & 15u;
    const float d = h2f(lds_u16(sb, sd + 0)) * (0.5f + (float)sc) * 0.25f;
    const uint32_t sg = lds_u8(sb, sd + 34 + oo);
    const uint32_t* e = tbl_words(tbl, qi * 16);
    const uint32_t* m0 = tbl_words(tbl, kGridB + (sg & 15u) * 8);
    const uint32_t* m1 = tbl_words(tbl, kGridB + (sg >> 4) * 8);
    const uint32_t ev[4] = {e[0], e[1], e[2], e[3]};
    const uint32_t mv[4] = {m0[0], m0[1], m1[0], m1[1]};
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = mix2(d, ev[i], 0.f) ^ mv[i];
  }
};

// IQ1_S (iq_lookup_decode.py:27-30): w = d*(2*s+1)*(grid[qi][c] + delta); the table holds
// grid + delta (entry qi | 2048 for delta = -0.125, the sign bit 15 of qh)
template <bool A4>
struct QmmDec<IQ1_S, A4> {
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const uint32_t h = lds_u16(sb, sd + 34 + 2 * g);
    const float d = h2f(lds_u16(sb, sd + 0)) * (float)(2u * ((h >> 12) & 7u) + 1u);
    const uint32_t qi = lds_u8(sb, sd + 2 + 4 * g + kq) | (((h >> (3 * kq)) & 7u) << 8) | ((h >> 15) << 11);
    grid8<false>(tbl, qi, d, 0.f, nullptr, o);
  }
};

// IQ1_M (iq_lookup_decode.py:31-37): w = d*(2*sc+1)*(grid[qi][c] + delta), d from the four
// scale words' top nibbles; the table holds grid + delta, indexed by the whole qh nibble (bit 3
// = delta's sign)
template <bool A4>
struct QmmDec<IQ1_M, A4> {
  __device__ __forceinline__ static void run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    uint32_t w[2];
    lds_words<2, A4>(sb, sd + 48, w);
    const uint32_t w0 = w[0] & 0xFFFFu, w1 = w[0] >> 16, w2 = w[1] & 0xFFFFu, w3 = w[1] >> 16;
    const uint32_t dbits = ((w0 & 61440u) >> 12) | ((w1 & 61440u) >> 8) | ((w2 & 61440u) >> 4) | (w3 & 61440u);
    const int oo = 4 * g + kq;
    const uint32_t hn = (lds_u8(sb, sd + 32 + oo / 2) >> (4 * (oo & 1))) & 15u;
    const uint32_t qi = lds_u8(sb, sd + oo) | (hn << 8);
    const int sci = 2 * g + (kq >> 1);
    const uint32_t ww = (sci >> 2) == 0 ? w0 : ((sci >> 2) == 1 ? w1 : ((sci >> 2) == 2 ? w2 : w3));
    const uint32_t sc = (ww >> (3 * (sci & 3))) & 7u;
    const float d = h2f(dbits) * (float)(2u * sc + 1u);
    grid8<false>(tbl, qi, d, 0.f, nullptr, o);
  }
};

// ---- raw fragments for the small-batch kernel ----------------------------------------------
// QmsRaw<T>::run gives the eight weights of octet kq of group g without the group's common
// float scale: codebook values with their signs applied (a sign flip is exact) and, for the
// types whose sub-scale changes every 16 weights (IQ2_XS, IQ2_S, IQ1_M), multiplied by that
// sub-scale in fp16 (v_pk_mul_f16: (0.5 + sc) * grid for the IQ2 value sets {8, 25, 43, 62},
// (2 sc + 1) * (grid +- 0.125) for IQ1, at most 11 significant bits, so exact); it returns the
// float scale s of the group, whose weights are s times these values. The small-batch kernel
// multiplies the raw values into a fresh accumulator and adds s times it to the output
// accumulator: four FMAs per fragment, against one v_fma_mix per weight when every weight is
// scaled and rounded to fp16 (QmmDec), and every product is formed from the exact weight.
template <int T, bool A4>
struct QmsRaw {
  static constexpr bool kOn = false;
};

__device__ __forceinline__ uint32_t pk_mul_h(uint32_t v, _Float16 f) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, v) * (half2_t){f, f});
}

template <bool A4>
struct QmsRaw<IQ3_S, A4> {
  static constexpr bool kOn = true;
  static constexpr uint32_t kMaskB = 512 * 4 * 2;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const float d = h2f(lds_u16(sb, sd + 0));
    const uint32_t sbyte = lds_u8(sb, sd + 106 + (g >> 1));
    const float db = d * (float)(1u + 2u * ((sbyte >> (4 * (g & 1))) & 15u));
    const uint32_t qh = lds_u8(sb, sd + 66 + g);
    const uint32_t qq = lds_u16(sb, sd + 2 + 8 * g + 2 * kq);
    const uint32_t i0 = (qq & 0xFFu) | ((qh << (8 - 2 * kq)) & 256u);
    const uint32_t i1 = (qq >> 8) | ((qh << (7 - 2 * kq)) & 256u);
    const uint32_t signs = lds_u8(sb, sd + 74 + 4 * g + kq);
    const uint32_t* e0 = tbl_words(tbl, i0 * 8);
    const uint32_t* e1 = tbl_words(tbl, i1 * 8);
    const uint32_t* m0 = tbl_words(tbl, kMaskB + (signs & 15u) * 8);
    const uint32_t* m1 = tbl_words(tbl, kMaskB + (signs >> 4) * 8);
    o[0] = e0[0] ^ m0[0];
    o[1] = e0[1] ^ m0[1];
    o[2] = e1[0] ^ m1[0];
    o[3] = e1[1] ^ m1[1];
    return db;
  }
};

template <bool A4>
struct QmsRaw<IQ3_XXS, A4> {
  static constexpr bool kOn = true;
  static constexpr uint32_t kGridB = 256 * 4 * 2;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const uint32_t u = lds_w32<A4>(sb, sd + 66 + 4 * g);
    const float d = h2f(lds_u16(sb, sd + 0)) * (0.5f + (float)(u >> 28)) * 0.5f;
    uint32_t m[4];
    ksigns_masks(tbl, kGridB, (u >> (7 * kq)) & 127u, m);
    const uint32_t qq = lds_u16(sb, sd + 2 + 8 * g + 2 * kq);
    const uint32_t* e0 = tbl_words(tbl, (qq & 0xFFu) * 8);
    const uint32_t* e1 = tbl_words(tbl, (qq >> 8) * 8);
    o[0] = e0[0] ^ m[0];
    o[1] = e0[1] ^ m[1];
    o[2] = e1[0] ^ m[2];
    o[3] = e1[1] ^ m[3];
    return d;
  }
};

template <bool A4>
struct QmsRaw<IQ2_XXS, A4> {
  static constexpr bool kOn = true;
  static constexpr uint32_t kGridB = 256 * 8 * 2;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const uint32_t u = lds_w32<A4>(sb, sd + 2 + 8 * g + 4);
    const float d = h2f(lds_u16(sb, sd + 0)) * (0.5f + (float)(u >> 28)) * 0.25f;
    const uint32_t* e = tbl_words(tbl, lds_u8(sb, sd + 2 + 8 * g + kq) * 16);
    const uint32_t* m = tbl_words(tbl, kGridB + 16 * 8 + ((u >> (7 * kq)) & 127u) * 16);
    uint32_t ev[4], mv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) { ev[i] = e[i]; mv[i] = m[i]; }
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = ev[i] ^ mv[i];
    return d;
  }
};

template <bool A4>
struct QmsRaw<IQ2_XS, A4> {
  static constexpr bool kOn = true;
  static constexpr uint32_t kGridB = 512 * 8 * 2;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const uint32_t q = lds_u16(sb, sd + 2 + 2 * (4 * g + kq));
    const uint32_t sc = (lds_u8(sb, sd + 66 + g) >> (4 * (kq >> 1))) & 15u;
    const _Float16 f = (_Float16)(0.5f + (float)sc);
    const uint32_t* e = tbl_words(tbl, (q & 511u) * 16);
    const uint32_t* m = tbl_words(tbl, kGridB + 16 * 8 + (q >> 9) * 16);
    uint32_t ev[4], mv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) { ev[i] = e[i]; mv[i] = m[i]; }
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pk_mul_h(ev[i], f) ^ mv[i];
    return h2f(lds_u16(sb, sd + 0)) * 0.25f;
  }
};

template <bool A4>
struct QmsRaw<IQ2_S, A4> {
  static constexpr bool kOn = true;
  static constexpr uint32_t kGridB = 1024 * 8 * 2;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const int oo = 4 * g + kq;
    const uint32_t hi = (lds_u8(sb, sd + 66 + g) >> (2 * kq)) & 3u;
    const uint32_t qi = lds_u8(sb, sd + 2 + oo) | (hi << 8);
    const uint32_t sc = (lds_u8(sb, sd + 74 + g) >> (4 * (kq >> 1))) & 15u;
    const _Float16 f = (_Float16)(0.5f + (float)sc);
    const uint32_t sg = lds_u8(sb, sd + 34 + oo);
    const uint32_t* e = tbl_words(tbl, qi * 16);
    const uint32_t* m0 = tbl_words(tbl, kGridB + (sg & 15u) * 8);
    const uint32_t* m1 = tbl_words(tbl, kGridB + (sg >> 4) * 8);
    const uint32_t ev[4] = {e[0], e[1], e[2], e[3]};
    const uint32_t mv[4] = {m0[0], m0[1], m1[0], m1[1]};
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pk_mul_h(ev[i], f) ^ mv[i];
    return h2f(lds_u16(sb, sd + 0)) * 0.25f;
  }
};

template <bool A4>
struct QmsRaw<IQ1_S, A4> {
  static constexpr bool kOn = true;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    const uint32_t h = lds_u16(sb, sd + 34 + 2 * g);
    const uint32_t qi = lds_u8(sb, sd + 2 + 4 * g + kq) | (((h >> (3 * kq)) & 7u) << 8) | ((h >> 15) << 11);
    const uint32_t* e = tbl_words(tbl, qi * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = e[i];
    return h2f(lds_u16(sb, sd + 0)) * (float)(2u * ((h >> 12) & 7u) + 1u);
  }
};

template <bool A4>
struct QmsRaw<IQ1_M, A4> {
  static constexpr bool kOn = true;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g, int kq, uint32_t (&o)[4]) {
    uint32_t w[2];
    lds_words<2, A4>(sb, sd + 48, w);
    const uint32_t dbits = ((w[0] >> 12) & 0xFu) | ((w[0] >> 24) & 0xF0u) | ((w[1] >> 4) & 0xF00u) |
                           ((w[1] >> 16) & 0xF000u);
    const int oo = 4 * g + kq;
    const uint32_t hn = (lds_u8(sb, sd + 32 + oo / 2) >> (4 * (oo & 1))) & 15u;
    const uint32_t qi = lds_u8(sb, sd + oo) | (hn << 8);
    const int sci = 2 * g + (kq >> 1);
    const uint32_t sc = (lds_u16(sb, sd + 48 + 2 * (sci >> 2)) >> (3 * (sci & 3))) & 7u;
    const _Float16 f = (_Float16)(float)(2u * sc + 1u);
    const uint32_t* e = tbl_words(tbl, qi * 16);
    uint32_t ev[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ev[i] = e[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pk_mul_h(ev[i], f);
    return h2f(dbits);
  }
};

// ---- whole-group fragments for the small-batch kernel's group layout --------------------------
// QmsGroup<T>::run gives the four fragments (octets kq = 0..3) of group g: for the codebook
// types the signed codebook values times the group's or 16-weight sub-scale in fp16, (2 s + 1) x
// value or (0.5 + s) x value, exact in fp16 for the published value sets (at most 11 significant
// bits), and returns the superblock's float scale d (times a power of two): all groups of a
// superblock share it, so one MFMA may take four groups' fragments and the scale goes onto the
// sum. The group's field words are read first, then every codebook and sign-mask read of its 32
// weights, then the arithmetic, so that the reads are in flight together.
template <int T, bool A4>
struct QmsGroup {
  static constexpr bool kOn = false;
};

template <bool A4>
struct QmsGroup<IQ2_S, A4> {
  static constexpr bool kOn = true;
  static constexpr uint32_t kGridB = 1024 * 8 * 2;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g,
                                              uint32_t (&o)[4][4]) {
    const uint32_t qs4 = lds_w32<A4>(sb, sd + 2 + 4 * g);
    const uint32_t sg4 = lds_w32<A4>(sb, sd + 34 + 4 * g);
    const uint32_t qh = lds_u8(sb, sd + 66 + g);
    const uint32_t scb = lds_u8(sb, sd + 74 + g);
    uint4 e[4];
    uint2 m0[4], m1[4];
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      const uint32_t qi = bfe(qs4, 8 * kq, 8) | (bfe(qh, 2 * kq, 2) << 8);
      const uint32_t s = bfe(sg4, 8 * kq, 8);
      e[kq] = *reinterpret_cast<const uint4*>(tbl + qi * 16);
      m0[kq] = *reinterpret_cast<const uint2*>(tbl + kGridB + (s & 15u) * 8);
      m1[kq] = *reinterpret_cast<const uint2*>(tbl + kGridB + (s >> 4) * 8);
    }
    const _Float16 f0 = (_Float16)(0.5f + (float)(scb & 15u)), f1 = (_Float16)(0.5f + (float)(scb >> 4));
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      const _Float16 f = kq < 2 ? f0 : f1;
      o[kq][0] = pk_mul_h(e[kq].x, f) ^ m0[kq].x;
      o[kq][1] = pk_mul_h(e[kq].y, f) ^ m0[kq].y;
      o[kq][2] = pk_mul_h(e[kq].z, f) ^ m1[kq].x;
      o[kq][3] = pk_mul_h(e[kq].w, f) ^ m1[kq].y;
    }
    return h2f(lds_u16(sb, sd)) * 0.25f;
  }
};

template <bool A4>
struct QmsGroup<IQ2_XS, A4> {
  static constexpr bool kOn = true;
  static constexpr uint32_t kGridB = 512 * 8 * 2;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g,
                                              uint32_t (&o)[4][4]) {
    uint32_t qw[2];
    lds_words<2, A4>(sb, sd + 2 + 8 * g, qw);
    const uint32_t scb = lds_u8(sb, sd + 66 + g);
    uint4 e[4], m[4];
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      const uint32_t q = bfe(qw[kq >> 1], 16 * (kq & 1), 16);
      e[kq] = *reinterpret_cast<const uint4*>(tbl + (q & 511u) * 16);
      m[kq] = *reinterpret_cast<const uint4*>(tbl + kGridB + 16 * 8 + (q >> 9) * 16);
    }
    const _Float16 f0 = (_Float16)(0.5f + (float)(scb & 15u)), f1 = (_Float16)(0.5f + (float)(scb >> 4));
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      const _Float16 f = kq < 2 ? f0 : f1;
      o[kq][0] = pk_mul_h(e[kq].x, f) ^ m[kq].x;
      o[kq][1] = pk_mul_h(e[kq].y, f) ^ m[kq].y;
      o[kq][2] = pk_mul_h(e[kq].z, f) ^ m[kq].z;
      o[kq][3] = pk_mul_h(e[kq].w, f) ^ m[kq].w;
    }
    return h2f(lds_u16(sb, sd)) * 0.25f;
  }
};

template <bool A4>
struct QmsGroup<IQ2_XXS, A4> {
  static constexpr bool kOn = true;
  static constexpr uint32_t kGridB = 256 * 8 * 2;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g,
                                              uint32_t (&o)[4][4]) {
    uint32_t w[2];  // four codebook indices, then four 7-bit sign indices and the 4-bit scale
    lds_words<2, A4>(sb, sd + 2 + 8 * g, w);
    uint4 e[4], m[4];
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      e[kq] = *reinterpret_cast<const uint4*>(tbl + bfe(w[0], 8 * kq, 8) * 16);
      m[kq] = *reinterpret_cast<const uint4*>(tbl + kGridB + 16 * 8 + bfe(w[1], 7 * kq, 7) * 16);
    }
    const _Float16 f = (_Float16)(float)(2u * (w[1] >> 28) + 1u);  // (0.5 + s) / 4 = (2 s + 1) / 8
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      o[kq][0] = pk_mul_h(e[kq].x, f) ^ m[kq].x;
      o[kq][1] = pk_mul_h(e[kq].y, f) ^ m[kq].y;
      o[kq][2] = pk_mul_h(e[kq].z, f) ^ m[kq].z;
      o[kq][3] = pk_mul_h(e[kq].w, f) ^ m[kq].w;
    }
    return h2f(lds_u16(sb, sd)) * 0.125f;
  }
};

template <bool A4>
struct QmsGroup<IQ3_XXS, A4> {
  static constexpr bool kOn = true;
  static constexpr uint32_t kGridB = 256 * 4 * 2;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g,
                                              uint32_t (&o)[4][4]) {
    uint32_t qw[2];  // eight codebook indices (one per 4 weights)
    lds_words<2, A4>(sb, sd + 2 + 8 * g, qw);
    const uint32_t u = lds_w32<A4>(sb, sd + 66 + 4 * g);
    uint2 e[8];
    uint32_t m[4][4];
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      e[2 * kq] = *reinterpret_cast<const uint2*>(tbl + bfe(qw[kq >> 1], 16 * (kq & 1), 8) * 8);
      e[2 * kq + 1] = *reinterpret_cast<const uint2*>(tbl + bfe(qw[kq >> 1], 16 * (kq & 1) + 8, 8) * 8);
      ksigns_masks(tbl, kGridB, (u >> (7 * kq)) & 127u, m[kq]);
    }
    const _Float16 f = (_Float16)(float)(2u * (u >> 28) + 1u);  // (0.5 + s) / 2 = (2 s + 1) / 4
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      o[kq][0] = pk_mul_h(e[2 * kq].x, f) ^ m[kq][0];
      o[kq][1] = pk_mul_h(e[2 * kq].y, f) ^ m[kq][1];
      o[kq][2] = pk_mul_h(e[2 * kq + 1].x, f) ^ m[kq][2];
      o[kq][3] = pk_mul_h(e[2 * kq + 1].y, f) ^ m[kq][3];
    }
    return h2f(lds_u16(sb, sd)) * 0.25f;
  }
};

template <bool A4>
struct QmsGroup<IQ3_S, A4> {
  static constexpr bool kOn = true;
  static constexpr uint32_t kMaskB = 512 * 4 * 2;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g,
                                              uint32_t (&o)[4][4]) {
    uint32_t qw[2];  // eight low index bytes (one per 4 weights)
    lds_words<2, A4>(sb, sd + 2 + 8 * g, qw);
    const uint32_t qh = lds_u8(sb, sd + 66 + g);
    const uint32_t sg4 = lds_w32<A4>(sb, sd + 74 + 4 * g);
    const uint32_t scb = lds_u8(sb, sd + 106 + (g >> 1));
    uint2 e[8], m[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // codebook entry i: weights 4 i .. 4 i + 3, sign nibble i
      const uint32_t qi = bfe(qw[i >> 2], 8 * (i & 3), 8) | (bfe(qh, i, 1) << 8);
      e[i] = *reinterpret_cast<const uint2*>(tbl + qi * 8);
      m[i] = *reinterpret_cast<const uint2*>(tbl + kMaskB + bfe(sg4, 4 * i, 4) * 8);
    }
    const _Float16 f = (_Float16)(float)(1u + 2u * ((scb >> (4 * (g & 1))) & 15u));
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      o[kq][0] = pk_mul_h(e[2 * kq].x, f) ^ m[2 * kq].x;
      o[kq][1] = pk_mul_h(e[2 * kq].y, f) ^ m[2 * kq].y;
      o[kq][2] = pk_mul_h(e[2 * kq + 1].x, f) ^ m[2 * kq + 1].x;
      o[kq][3] = pk_mul_h(e[2 * kq + 1].y, f) ^ m[2 * kq + 1].y;
    }
    return h2f(lds_u16(sb, sd));
  }
};

template <bool A4>
struct QmsGroup<IQ1_S, A4> {
  static constexpr bool kOn = true;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g,
                                              uint32_t (&o)[4][4]) {
    const uint32_t qs4 = lds_w32<A4>(sb, sd + 2 + 4 * g);
    const uint32_t h = lds_u16(sb, sd + 34 + 2 * g);
    uint4 e[4];
#pragma unroll
    for (int kq = 0; kq < 4; ++kq)  // the table holds entry + delta; entry qi | 2048 for delta -0.125
      e[kq] = *reinterpret_cast<const uint4*>(
          tbl + (bfe(qs4, 8 * kq, 8) | (bfe(h, 3 * kq, 3) << 8) | ((h >> 15) << 11)) * 16);
    const _Float16 f = (_Float16)(float)(2u * ((h >> 12) & 7u) + 1u);
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      o[kq][0] = pk_mul_h(e[kq].x, f);
      o[kq][1] = pk_mul_h(e[kq].y, f);
      o[kq][2] = pk_mul_h(e[kq].z, f);
      o[kq][3] = pk_mul_h(e[kq].w, f);
    }
    return h2f(lds_u16(sb, sd));
  }
};

// IQ1_M: the raw fragments (their 16-weight sub-scales already inside, d common to the superblock)
template <bool A4>
struct QmsGroup<IQ1_M, A4> {
  static constexpr bool kOn = true;
  __device__ __forceinline__ static float run(const uint8_t* sb, uint32_t sd, const uint8_t* tbl, int g,
                                              uint32_t (&o)[4][4]) {
    float d = 0.f;
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) d = QmsRaw<IQ1_M, A4>::run(sb, sd, tbl, g, kq, o[kq]);
    return d;
  }
};

}  // namespace gsq
