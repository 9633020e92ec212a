// Exact per-group dequantization (32 weights of one superblock group -> float32).
//
// Each specialization restates the reference formula for its format
// (mlx_gsq/runtime/kernels/k_decode.py:18-80, iq_lookup_decode.py:6-39,
// iq3_s_decode.py:16-40). All products are exact in float32; Q2_K/Q4_K round once in the
// final subtraction, so results are bit-identical to the CPU dequantizer.
#pragma once
#include "gsq_common.h"

namespace gsq {

template <int T>
__device__ __forceinline__ void dq_group(const uint8_t* b, int g, const DevTables& t, float* o);

template <>
__device__ __forceinline__ void dq_group<Q2_K>(const uint8_t* b, int g, const DevTables&, float* o) {
  const float d = h2f(gu16(b, 80)), dmin = h2f(gu16(b, 82));
  const int chunk = g >> 2, plane = g & 3;
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    uint32_t q = (gb(b, 16 + chunk * 32 + p) >> (2 * plane)) & 3u;
    uint32_t sm = gb(b, 2 * g + (p >> 4));
    o[p] = d * (float)(sm & 15u) * (float)q - dmin * (float)(sm >> 4);
  }
}

template <>
__device__ __forceinline__ void dq_group<Q4_K>(const uint8_t* b, int g, const DevTables&, float* o) {
  const uint8_t* s = b + 4;
  uint32_t sc, mn;
  if (g < 4) {
    sc = s[g] & 63u; mn = s[4 + g] & 63u;
  } else {
    int gg = g - 4;
    sc = (s[8 + gg] & 15u) | ((s[gg] >> 2) & 48u);
    mn = (s[8 + gg] >> 4) | ((s[4 + gg] >> 2) & 48u);
  }
  const float d = h2f(gu16(b, 0)), dmin = h2f(gu16(b, 2));
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    uint32_t q = (gb(b, 16 + (g >> 1) * 32 + p) >> (4 * (g & 1))) & 15u;
    o[p] = d * (float)sc * (float)q - dmin * (float)mn;
  }
}

template <>
__device__ __forceinline__ void dq_group<Q6_K>(const uint8_t* b, int g, const DevTables&, float* o) {
  const float d = h2f(gu16(b, 208));
  const int chunk = g >> 2, plane = g & 3;
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    int in_chunk = plane * 32 + p;
    uint32_t ql = (gb(b, chunk * 64 + (in_chunk & 63)) >> (4 * (in_chunk >> 6))) & 15u;
    uint32_t qh = (gb(b, 128 + chunk * 32 + p) >> (2 * plane)) & 3u;
    int q = (int)(ql | (qh << 4)) - 32;
    int scale = (int)(int8_t)b[192 + 2 * g + (p >> 4)];
    o[p] = d * (float)scale * (float)q;
  }
}

template <>
__device__ __forceinline__ void dq_group<IQ4_XS>(const uint8_t* b, int g, const DevTables&, float* o) {
  uint32_t scales_h = gu16(b, 2);
  uint32_t low = (gb(b, 4 + g / 2) >> (4 * (g & 1))) & 15u;
  uint32_t high = (scales_h >> (2 * g)) & 3u;
  int scale = (int)(low | (high << 4)) - 32;
  const float d = h2f(gu16(b, 0));
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    uint32_t q = (gb(b, 8 + g * 16 + (p & 15)) >> (4 * (p >> 4))) & 15u;
    o[p] = d * (float)scale * (float)kIQ4Values[q];
  }
}

template <>
__device__ __forceinline__ void dq_group<IQ3_S>(const uint8_t* b, int g, const DevTables& t, float* o) {
  const float d = h2f(gu16(b, 0));
  uint32_t sbyte = gb(b, 106 + (g >> 1));
  uint32_t snib = (g & 1) ? (sbyte >> 4) : (sbyte & 15u);
  const float db = d * (float)(1u + 2u * snib);
  uint32_t qh = gb(b, 66 + g);
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    int l = p >> 3, c = p & 7;
    uint32_t gi = (c < 4) ? (gb(b, 2 + g * 8 + l * 2) | ((qh << (8 - 2 * l)) & 256u))
                          : (gb(b, 2 + g * 8 + l * 2 + 1) | ((qh << (7 - 2 * l)) & 256u));
    float mag = h2f(t.grid16[gi * 4 + (c & 3)]);
    bool neg = (gb(b, 74 + g * 4 + l) >> c) & 1u;
    o[p] = neg ? -db * mag : db * mag;
  }
}

template <>
__device__ __forceinline__ void dq_group<IQ3_XXS>(const uint8_t* b, int g, const DevTables& t, float* o) {
  uint32_t u = gu32(b, 66 + g * 4);
  const float d = h2f(gu16(b, 0)) * (0.5f + (float)(u >> 28)) * 0.5f;
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    int l = p >> 3, c = p & 7;
    bool neg = (t.ksigns[(u >> (7 * l)) & 127u] >> c) & 1u;
    uint32_t qi = gb(b, 2 + g * 8 + l * 2 + (c >= 4 ? 1 : 0));
    float v = h2f(t.grid16[qi * 4 + (c & 3)]);
    o[p] = neg ? -d * v : d * v;
  }
}

template <>
__device__ __forceinline__ void dq_group<IQ2_XXS>(const uint8_t* b, int g, const DevTables& t, float* o) {
  const uint8_t* q = b + 2 + g * 8;
  uint32_t u = gu32(q, 4);
  const float d = h2f(gu16(b, 0)) * (0.5f + (float)(u >> 28)) * 0.25f;
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    int l = p >> 3, c = p & 7;
    bool neg = (t.ksigns[(u >> (7 * l)) & 127u] >> c) & 1u;
    float v = h2f(t.grid16[(uint32_t)q[l] * 8 + c]);
    o[p] = neg ? -d * v : d * v;
  }
}

template <>
__device__ __forceinline__ void dq_group<IQ2_XS>(const uint8_t* b, int g, const DevTables& t, float* o) {
  const float dh = h2f(gu16(b, 0));
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    int e = g * 32 + p, gg = e >> 4, pp = e & 15, sub = pp >> 3, c = pp & 7, oo = gg * 2 + sub;
    uint32_t q = gu16(b, 2 + oo * 2);
    uint32_t sc = (gb(b, 66 + gg / 2) >> (4 * (gg & 1))) & 15u;
    float d = dh * (0.5f + (float)sc) * 0.25f;
    bool neg = (t.ksigns[(q >> 9) & 127u] >> c) & 1u;
    float v = h2f(t.grid16[(q & 511u) * 8 + c]);
    o[p] = neg ? -d * v : d * v;
  }
}

template <>
__device__ __forceinline__ void dq_group<IQ2_S>(const uint8_t* b, int g, const DevTables& t, float* o) {
  const float dh = h2f(gu16(b, 0));
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    int e = g * 32 + p, gg = e >> 4, pp = e & 15, sub = pp >> 3, c = pp & 7, oo = gg * 2 + sub;
    uint32_t hi = (gb(b, 66 + oo / 4) >> (2 * (oo & 3))) & 3u;
    uint32_t qi = gb(b, 2 + oo) | (hi << 8);
    uint32_t sc = (gb(b, 74 + gg / 2) >> (4 * (gg & 1))) & 15u;
    float d = dh * (0.5f + (float)sc) * 0.25f;
    bool neg = (gb(b, 34 + oo) >> c) & 1u;
    float v = h2f(t.grid16[qi * 8 + c]);
    o[p] = neg ? -d * v : d * v;
  }
}

template <>
__device__ __forceinline__ void dq_group<IQ1_S>(const uint8_t* b, int g, const DevTables& t, float* o) {
  uint32_t h = gu16(b, 34 + g * 2);
  const float d = h2f(gu16(b, 0)) * (float)(2u * ((h >> 12) & 7u) + 1u);
  const float delta = (h & 32768u) ? -0.125f : 0.125f;
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    int l = p >> 3, c = p & 7;
    uint32_t qi = gb(b, 2 + g * 4 + l) | (((h >> (3 * l)) & 7u) << 8);
    o[p] = d * (h2f(t.grid16[qi * 8 + c]) + delta);
  }
}

template <>
__device__ __forceinline__ void dq_group<IQ1_M>(const uint8_t* b, int g, const DevTables& t, float* o) {
  uint32_t w0 = gu16(b, 48), w1 = gu16(b, 50), w2 = gu16(b, 52), w3 = gu16(b, 54);
  uint32_t dbits = ((w0 & 61440u) >> 12) | ((w1 & 61440u) >> 8) | ((w2 & 61440u) >> 4) | (w3 & 61440u);
  const float d = h2f(dbits);
#pragma unroll
  for (int p = 0; p < 32; ++p) {
    int sg = p >> 4, r = p & 15, sub = r >> 3, c = r & 7, oo = g * 4 + sg * 2 + sub;
    uint32_t hn = (gb(b, 32 + oo / 2) >> (4 * (oo & 1))) & 15u;
    uint32_t qi = gb(b, oo) | ((hn & 7u) << 8);
    float delta = (hn & 8u) ? -0.125f : 0.125f;
    int sci = g * 2 + sg, wi = sci >> 2, sh = 3 * (sci & 3);
    uint32_t ww = wi == 0 ? w0 : (wi == 1 ? w1 : (wi == 2 ? w2 : w3));
    uint32_t sc = (ww >> sh) & 7u;
    o[p] = d * (float)(2u * sc + 1u) * (h2f(t.grid16[qi * 8 + c]) + delta);
  }
}

}  // namespace gsq
