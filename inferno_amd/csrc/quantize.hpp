// Synthetic data: counter-based normal generator and a simple GGUF block
// quantiser, usable on host and device.
//
// The reference has no quantiser. This one is our own min/max method (per
// sub-block range -> integer scale relative to a per-super-block f16 scale,
// then nearest-integer codes); it only has to produce valid blocks, since
// every consumer (GPU kernels and the CPU oracle) decodes the same bytes.
// Byte layouts follow crates/gguf/src/lib.rs:1226-1499 and the block
// builders of its tests (:2535-2610).
#pragma once
#include "common.hpp"

namespace inferno {

HD uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

// Element i of the standard-normal stream `seed` (Box-Muller on a pair).
HD float synth_normal(uint64_t seed, uint64_t i) {
  uint64_t key = splitmix64(seed * 0x2545f4914f6cdd1dull + 0x632be59bd9b4e019ull);
  uint64_t pair = i >> 1;
  uint64_t a = splitmix64(key ^ (2 * pair));
  uint64_t b = splitmix64(key ^ (2 * pair + 1));
  float u1 = float((a >> 40) + 1) * (1.0f / 16777216.0f);  // (0, 1]
  float u2 = float(b >> 40) * (1.0f / 16777216.0f);        // [0, 1)
  float r = sqrtf(-2.0f * logf(u1));
  float th = 6.283185307179586f * u2;
  return (i & 1) ? r * sinf(th) : r * cosf(th);
}

HD float qround(float v) { return __builtin_rintf(v); }
HD int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
HD float f16r(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }
HD void store_le16(uint8_t* p, uint16_t v) {
  p[0] = uint8_t(v);
  p[1] = uint8_t(v >> 8);
}

// Q2_K: [scales 16 | qs 64 | d | dmin]; group g (16 values) = scale byte g;
// value v = 128h + 32p + 16s + i lives in qs[32h + 16s + i] bits 2p.
HD void quantize_q2_k(const float* x, uint8_t* b) {
  float scale[16], mins[16], max_scale = 0.f, max_min = 0.f;
  for (int g = 0; g < 16; ++g) {
    float mn = 0.f, mx = -3.0e38f;
    for (int i = 0; i < 16; ++i) {
      mn = fminf(mn, x[16 * g + i]);
      mx = fmaxf(mx, x[16 * g + i]);
    }
    scale[g] = (mx - mn) / 3.f;
    mins[g] = -mn;
    max_scale = fmaxf(max_scale, scale[g]);
    max_min = fmaxf(max_min, mins[g]);
  }
  float d = f16r(max_scale / 15.f), dmin = f16r(max_min / 15.f);
  for (int i = 0; i < 84; ++i) b[i] = 0;
  for (int g = 0; g < 16; ++g) {
    int sc = d > 0.f ? clampi(int(qround(scale[g] / d)), 0, 15) : 0;
    int m = dmin > 0.f ? clampi(int(qround(mins[g] / dmin)), 0, 15) : 0;
    b[g] = uint8_t(sc | (m << 4));
    float step = d * float(sc), off = dmin * float(m);
    int h = g / 8, p = (g / 2) & 3, s = g & 1;
    for (int i = 0; i < 16; ++i) {
      int q = step > 0.f ? clampi(int(qround((x[16 * g + i] + off) / step)), 0, 3) : 0;
      b[16 + 32 * h + 16 * s + i] |= uint8_t(q << (2 * p));
    }
  }
  store_le16(b + 80, f32_to_f16_bits(d));
  store_le16(b + 82, f32_to_f16_bits(dmin));
}

// Q3_K: [hmask 32 | qs 64 | scales 12 | d]; signed 6-bit group scales,
// codes q in [-4, 3] stored as q+4 (low 2 bits in qs, bit 2 in hmask).
HD void quantize_q3_k(const float* x, uint8_t* b) {
  float scale[16], amax = 0.f;
  for (int g = 0; g < 16; ++g) {
    float xm = 0.f;
    for (int i = 0; i < 16; ++i)
      if (fabsf(x[16 * g + i]) > fabsf(xm)) xm = x[16 * g + i];
    scale[g] = xm / -4.f;
    amax = fmaxf(amax, fabsf(scale[g]));
  }
  float d = f16r(amax / 31.f);
  for (int i = 0; i < 110; ++i) b[i] = 0;
  uint8_t* hm = b;
  uint8_t* qs = b + 32;
  uint8_t* sc = b + 96;
  for (int g = 0; g < 16; ++g) {
    int s = d > 0.f ? clampi(int(qround(scale[g] / d)), -32, 31) : 0;
    int S = s + 32;
    if (g < 8) sc[g] |= uint8_t(S & 15);
    else sc[g - 8] |= uint8_t((S & 15) << 4);
    sc[8 + g % 4] |= uint8_t(((S >> 4) & 3) << (2 * (g / 4)));
    float step = d * float(s);
    for (int i = 0; i < 16; ++i) {
      int q = step != 0.f ? clampi(int(qround(x[16 * g + i] / step)), -4, 3) : 0;
      int qq = q + 4;
      qs[32 * (g / 8) + 16 * (g & 1) + i] |= uint8_t((qq & 3) << (2 * ((g / 2) & 3)));
      if (qq & 4) hm[16 * (g & 1) + i] |= uint8_t(1u << (g / 2));
    }
  }
  store_le16(b + 108, f32_to_f16_bits(d));
}

// Q4_K: [d | dmin | scales 12 | qs 128]; eight 32-value groups with 6-bit
// (scale, min); value 32g+i = nibble (g&1) of qs[32(g/2) + i].
HD void quantize_q4_k(const float* x, uint8_t* b) {
  float scale[8], mins[8], max_scale = 0.f, max_min = 0.f;
  for (int g = 0; g < 8; ++g) {
    float mn = 0.f, mx = -3.0e38f;
    for (int i = 0; i < 32; ++i) {
      mn = fminf(mn, x[32 * g + i]);
      mx = fmaxf(mx, x[32 * g + i]);
    }
    scale[g] = (mx - mn) / 15.f;
    mins[g] = -mn;
    max_scale = fmaxf(max_scale, scale[g]);
    max_min = fmaxf(max_min, mins[g]);
  }
  float d = f16r(max_scale / 63.f), dmin = f16r(max_min / 63.f);
  for (int i = 0; i < 144; ++i) b[i] = 0;
  uint8_t* s = b + 4;
  uint8_t* qs = b + 16;
  for (int g = 0; g < 8; ++g) {
    int sc = d > 0.f ? clampi(int(qround(scale[g] / d)), 0, 63) : 0;
    int m = dmin > 0.f ? clampi(int(qround(mins[g] / dmin)), 0, 63) : 0;
    if (g < 4) {
      s[g] |= uint8_t(sc);
      s[g + 4] |= uint8_t(m);
    } else {
      s[g + 4] |= uint8_t((sc & 15) | ((m & 15) << 4));
      s[g - 4] |= uint8_t((sc >> 4) << 6);
      s[g] |= uint8_t((m >> 4) << 6);
    }
    float step = d * float(sc), off = dmin * float(m);
    for (int i = 0; i < 32; ++i) {
      int q = step > 0.f ? clampi(int(qround((x[32 * g + i] + off) / step)), 0, 15) : 0;
      qs[32 * (g / 2) + i] |= uint8_t(q << (4 * (g & 1)));
    }
  }
  store_le16(b, f32_to_f16_bits(d));
  store_le16(b + 2, f32_to_f16_bits(dmin));
}

// Q6_K: [ql 128 | qh 64 | int8 scales 16 | d]; codes q in [-32, 31] as q+32.
HD void quantize_q6_k(const float* x, uint8_t* b) {
  float scale[16], amax = 0.f;
  for (int g = 0; g < 16; ++g) {
    float xm = 0.f;
    for (int i = 0; i < 16; ++i)
      if (fabsf(x[16 * g + i]) > fabsf(xm)) xm = x[16 * g + i];
    scale[g] = xm / -32.f;
    amax = fmaxf(amax, fabsf(scale[g]));
  }
  float d = f16r(amax / 127.f);
  for (int i = 0; i < 210; ++i) b[i] = 0;
  uint8_t* ql = b;
  uint8_t* qh = b + 128;
  for (int g = 0; g < 16; ++g) {
    int s = d > 0.f ? clampi(int(qround(scale[g] / d)), -128, 127) : 0;
    b[192 + g] = uint8_t(int8_t(s));
    float step = d * float(s);
    for (int j = 0; j < 16; ++j) {
      int v = 16 * g + j;
      int half = v / 128, quarter = (v % 128) / 32, i = v % 32;
      int q = step != 0.f ? clampi(int(qround(x[v] / step)), -32, 31) : 0;
      int qq = q + 32;
      int li = 64 * half + (quarter & 1) * 32 + i;
      ql[li] |= uint8_t((qq & 15) << (quarter >= 2 ? 4 : 0));
      qh[32 * half + i] |= uint8_t((qq >> 4) << (2 * quarter));
    }
  }
  store_le16(b + 208, f32_to_f16_bits(d));
}

// Q8_0: [d | int8 x32].
HD void quantize_q8_0(const float* x, uint8_t* b) {
  float amax = 0.f;
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
  float d = f16r(amax / 127.f);
  store_le16(b, f32_to_f16_bits(d));
  for (int i = 0; i < 32; ++i) {
    int q = d > 0.f ? clampi(int(qround(x[i] / d)), -127, 127) : 0;
    b[2 + i] = uint8_t(int8_t(q));
  }
}

HD void quantize_block(int quant, const float* x, uint8_t* b) {
  switch (quant) {
    case INFERNO_Q2_K: quantize_q2_k(x, b); break;
    case INFERNO_Q3_K: quantize_q3_k(x, b); break;
    case INFERNO_Q4_K: quantize_q4_k(x, b); break;
    case INFERNO_Q6_K: quantize_q6_k(x, b); break;
    case INFERNO_Q8_0: quantize_q8_0(x, b); break;
  }
}

}  // namespace inferno
