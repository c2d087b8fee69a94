// Decode GEMVs of the routed Q2_K / Q3_K / Q4_K experts for one token on the
// matrix cores (v_mfma_f32_16x16x32_f16), activations staged as f16 runs.
//
// Both expert GEMVs (gate/up against x, down against h) share one block dot:
// a 16-row tile of one super-block column (256 values) is one set of MFMA
// tiles C[m][n] = sum_k A[m][k] B[k][n] with
//   B (weights, row n = lane & 15): a quant field masked in place inside a
//     16-bit half is an exact f16 subnormal q 2^(b - 24) (b = the field's bit
//     offset), so two fields come out of one v_and_b32;
//   A (activations): row m is the 16-value run m of the column (one group of
//     Q2_K/Q3_K, half a group of Q4_K), holding the run's values only in the
//     K slots that carry that run's fields, zeros elsewhere (block diagonal);
//     each run's dot product lands in its own row of C;
//   the run's f16 values are x * s_run * 2^-shift(run), with s_run a power of
//     two per run (max |x| of the run in [2^14, 2^15)) and shift the field
//     offset that format puts the run at, so C = s_run 2^-24 sum x q for
//     every run whatever its field offset; the run factors 2^48 / s_run and
//     the run sums of x are staged beside the values.
// Group scales and minimums enter after the MFMA, per C row.
//
// Staged run row (words), K values: [pairs K/2][run sums K/16][run factors
// K/16]; run r holds 8 words, word j = values (base, base + 2) with base =
// 4 (j >> 1) + (j & 1), the order in which masked fields pair up.
//
// Reference semantics: dequantize_q2_k_block / q3_k / q4_k
// (crates/gguf/src/lib.rs:1226-1405); gate/up with SwiGLU and the routing
// weight folded into h, down summed over the ranks
// (crates/backend/src/metal/kernels/gguf_moe_kernels.metal:340-565,
// laguna_xs_kernels.metal:1578-1715). Accumulation is fp32; the order differs
// from the reference's (the parity bound is the layer tolerance).
#pragma once
#include "decode.hpp"
#include "decode_mfma.hpp"

namespace inferno {
namespace runs_decode {

using mfma_decode::as_h2;
using mfma_decode::floatx4;
using mfma_decode::half8;
using mfma_decode::u32x4;
using mfma_decode::lds_words_a2;
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32_a2 __attribute__((aligned(2)));

constexpr int kWaves = 16;
constexpr int kThreads = 64 * kWaves;
constexpr float kTwoM24 = 1.0f / 16777216.0f;
// Expert id of the shared expert when it runs as the token's assignment k
// (DecodeArgs::shared_slot): its gate/up/down rows come from sgate/sup/sdown.
constexpr uint32_t kSharedId = 0xffffffffu;

__host__ __device__ constexpr int run_words(int K) { return K / 2 + K / 8; }

// ------------------------------------------------------------- formats

template <int Q>
struct RF;

__device__ __forceinline__ half8 load_a(const uint32_t* p) {
  return __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ floatx4 mfma(half8 a, uint4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// Q2_K [scales 16 | qs 64 | d | dmin]. Run = group g (16 values) = 8 h + 2 p
// + s: field plane p of qs bytes 32 h + 16 s + i. MFMA (pp, hf): B lane group
// q = 2 h + s takes qs bytes 16 q + 8 hf + {0, 2, 1, 3, 4, 6, 5, 7} at plane
// pp; run m is live in lane group 2 (m >> 3) + (m & 1), MFMAs pp = (m >> 1) & 3.
template <>
struct RF<INFERNO_Q2_K> {
  static constexpr int kBytes = 84;
  typedef mfma_decode::half2v half2v_t;
  __host__ __device__ static int run_shift(int r) { return 2 * ((r >> 1) & 3); }
  template <int NA>
  __device__ static void dot(const uint8_t* blk, const uint32_t* const (&cols)[NA],
                             const uint32_t* zero, int n, int q, floatx4 (&C)[NA]) {
    const bool act = q == 2 * (n >> 3) + (n & 1);
    const int pm = (n >> 1) & 3;
    const u32x4_a2 qs = *reinterpret_cast<const u32x4_a2*>(blk + 16 + 16 * q);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint32_t w0 = hf ? qs.z : qs.x, w1 = hf ? qs.w : qs.y;
      const uint32_t o0 = w0 >> 8, o1 = w1 >> 8;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const uint32_t M = 0x00030003u << (2 * pp);
        const uint4 bv = make_uint4(w0 & M, o0 & M, w1 & M, o1 & M);
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          const uint32_t* src = (act && pp == pm) ? cols[a] + n * 8 + 4 * hf : zero;
          C[a] = mfma(load_a(src), bv, C[a]);
        }
      }
    }
  }
  // sum over this lane's C rows (runs 4 q + j) of the group dots, the run sums
  // and factors at sums[4 q + j], kk[4 q + j]
  __device__ static float epilogue(const uint8_t* blk, floatx4 C, float4 sums, float4 kk,
                                   int q) {
    const uint32_t scw = *reinterpret_cast<const u32_a2*>(blk + 4 * q);
    const half2v_t dm = as_h2(*reinterpret_cast<const u32_a2*>(blk + 80));
    const float c[4] = {C[0], C[1], C[2], C[3]};
    const float s[4] = {sums.x, sums.y, sums.z, sums.w};
    const float f[4] = {kk.x, kk.y, kk.z, kk.w};
    float S = 0.f, Mn = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t b = (scw >> (8 * j)) & 0xffu;
      S = fmaf(float(b & 15u), c[j] * f[j], S);
      Mn = fmaf(float(b >> 4), s[j], Mn);
    }
    return (float)dm.x * (S * kTwoM24) - (float)dm.y * Mn;
  }
};

// Q3_K [hmask 32 | qs 64 | scales 12 | d]: the low two bits sit where Q2_K's
// do (qs at byte 32), the high bit of value i of group g = 8 h + 2 p + s in
// hmask byte 16 s + i, bit 4 h + p. Masked at bit 2 pp + 2 of the same half
// it joins the low field: q3 4^pp = (low + 4 hbit) 4^pp, one MFMA per
// (pp, hf) as for Q2_K. Value = gs (q3 - 4), gs = d (s6 - 32).
template <>
struct RF<INFERNO_Q3_K> {
  static constexpr int kBytes = 110;
  typedef mfma_decode::half2v half2v_t;
  __host__ __device__ static int run_shift(int r) { return 2 * ((r >> 1) & 3); }
  template <int NA>
  __device__ static void dot(const uint8_t* blk, const uint32_t* const (&cols)[NA],
                             const uint32_t* zero, int n, int q, floatx4 (&C)[NA]) {
    const bool act = q == 2 * (n >> 3) + (n & 1);
    const int pm = (n >> 1) & 3;
    uint32_t qs[4], hm[4];
    lds_words_a2(blk + 32 + 16 * q, qs);
    lds_words_a2(blk + 16 * (q & 1), hm);
    // lane group q = 2 h + s needs bit 4 h + pp of each hmask byte: shifted
    // down by 4 h once, bit pp of every byte is that bit
    const int hsh = 4 * (q >> 1);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint32_t w0 = qs[2 * hf], w1 = qs[2 * hf + 1];
      const uint32_t x0 = hm[2 * hf] >> hsh, x1 = hm[2 * hf + 1] >> hsh;
      const uint32_t o0 = w0 >> 8, o1 = w1 >> 8;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const uint32_t M = 0x00030003u << (2 * pp);
        const uint32_t MH = 0x00040004u << (2 * pp);
        // bytes 0, 2: bit pp to bit 2 pp + 2; bytes 1, 3: bit 8 + pp to 2 pp + 2
        const uint4 bv = make_uint4((w0 & M) | ((x0 << (pp + 2)) & MH),
                                    (o0 & M) | ((x0 >> (6 - pp)) & MH),
                                    (w1 & M) | ((x1 << (pp + 2)) & MH),
                                    (o1 & M) | ((x1 >> (6 - pp)) & MH));
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          const uint32_t* src = (act && pp == pm) ? cols[a] + n * 8 + 4 * hf : zero;
          C[a] = mfma(load_a(src), bv, C[a]);
        }
      }
    }
  }
  __device__ static float epilogue(const uint8_t* blk, floatx4 C, float4 sums, float4 kk,
                                   int q) {
    // groups 4 q + j: low nibble of scales[(4 q + j) % 8] (high nibble for
    // q >= 2), high two bits of scales[8 + j] at bit 2 q
    uint32_t lw[1], hw[1];
    lds_words_a2(blk + 96 + 4 * (q & 1), lw);
    lds_words_a2(blk + 104, hw);
    const uint32_t lo = lw[0], hi = hw[0];
    const uint32_t s6 = ((lo >> (4 * (q >> 1))) & 0x0f0f0f0fu) | (((hi >> (2 * q)) & 0x03030303u) << 4);
    const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk + 108));
    const float c[4] = {C[0], C[1], C[2], C[3]};
    const float s[4] = {sums.x, sums.y, sums.z, sums.w};
    const float f[4] = {kk.x, kk.y, kk.z, kk.w};
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float gs = float(int((s6 >> (8 * j)) & 0xffu) - 32);
      acc = fmaf(gs, fmaf(c[j] * f[j], kTwoM24, -4.0f * s[j]), acc);
    }
    return d * acc;
  }
};

// Q4_K [d | dmin | scales 12 | qs 128]: group g (32 values) = runs 2 g, 2 g +
// 1; qs chunk c (bytes 32 c ..) holds groups 2 c (low nibbles) and 2 c + 1
// (high nibbles). MFMA (jj, nib): lane group q takes chunk q bytes 8 jj +
// {0, 2, 1, 3, 4, 6, 5, 7}, nibble nib (a field at bit 4 nib of the byte).
// Run m = 2 g + half is live in lane group m >> 2, MFMAs nib = (m >> 1) & 1,
// jj = 2 (m & 1) + {0, 1} (its 16 values are chunk bytes 16 (m & 1) ..).
template <>
struct RF<INFERNO_Q4_K> {
  static constexpr int kBytes = 144;
  typedef mfma_decode::half2v half2v_t;
  __host__ __device__ static int run_shift(int r) { return 4 * ((r >> 1) & 1); }
  template <int NA>
  __device__ static void dot(const uint8_t* blk, const uint32_t* const (&cols)[NA],
                             const uint32_t* zero, int n, int q, floatx4 (&C)[NA]) {
    const bool act = q == (n >> 2);
    const int nm = (n >> 1) & 1, hm = n & 1;
    const u32x4_a2 c0 = *reinterpret_cast<const u32x4_a2*>(blk + 16 + 32 * q);
    const u32x4_a2 c1 = *reinterpret_cast<const u32x4_a2*>(blk + 32 + 32 * q);
    const uint32_t w[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const uint32_t w0 = w[2 * jj], w1 = w[2 * jj + 1];
      const uint32_t o0 = w0 >> 8, o1 = w1 >> 8;
#pragma unroll
      for (int nib = 0; nib < 2; ++nib) {
        const uint32_t M = nib ? 0x00f000f0u : 0x000f000fu;
        const uint4 bv = make_uint4(w0 & M, o0 & M, w1 & M, o1 & M);
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          const uint32_t* src =
              (act && nib == nm && (jj >> 1) == hm) ? cols[a] + n * 8 + 4 * (jj & 1) : zero;
          C[a] = mfma(load_a(src), bv, C[a]);
        }
      }
    }
  }
  __device__ static float epilogue(const uint8_t* blk, floatx4 C, float4 sums, float4 kk,
                                   int q) {
    // runs 4 q + j: groups 2 q (j < 2) and 2 q + 1 (j >= 2); 6-bit scale and
    // min of group g (crates/gguf/src/lib.rs:1407-1416), from the 12 scale
    // bytes read as three dwords
    const uint32_t w0 = *reinterpret_cast<const u32_a2*>(blk + 4);
    const uint32_t w1 = *reinterpret_cast<const u32_a2*>(blk + 8);
    const uint32_t w2 = *reinterpret_cast<const u32_a2*>(blk + 12);
    auto sb = [&](int i) -> uint32_t {
      const uint32_t w = i < 4 ? w0 : (i < 8 ? w1 : w2);
      return (w >> (8 * (i & 3))) & 0xffu;
    };
    float sc[2], mn[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int g = 2 * q + k;
      uint32_t s, m;
      if (g < 4) {
        s = sb(g) & 63u;
        m = sb(g + 4) & 63u;
      } else {
        s = (sb(g + 4) & 15u) | ((sb(g - 4) >> 6) << 4);
        m = (sb(g + 4) >> 4) | ((sb(g) >> 6) << 4);
      }
      sc[k] = float(s);
      mn[k] = float(m);
    }
    const half2v_t dm = as_h2(*reinterpret_cast<const u32_a2*>(blk));
    const float S0 = fmaf(C[0], kk.x, C[1] * kk.y), S1 = fmaf(C[2], kk.z, C[3] * kk.w);
    const float D = fmaf(sc[0], S0, sc[1] * S1) * kTwoM24;
    const float Mn = fmaf(mn[0], sums.x + sums.y, mn[1] * (sums.z + sums.w));
    return (float)dm.x * D - (float)dm.y * Mn;
  }
};

// Q6_K [ql 128 | qh 64 | scales 16 (int8) | d] (crates/gguf/src/lib.rs:
// 1418-1470): value j = 128 h + 32 u + l (half h, quarter u, l < 32) is
// q6 = (ql[64 h + 32 (u & 1) + l] >> 4 (u >> 1)) & 15 | ((qh[32 h + l] >> 2 u)
// & 3) << 4, value = d sc[8 h + 2 u + l / 16] (q6 - 32): run r (16 values) =
// 8 h + 2 u + s has scale byte r. MFMA (h, u): lane group q = 2 s + hf takes
// ql bytes 64 h + 32 (u & 1) + 8 q .. + 7 and qh bytes 32 h + 8 q .. + 7, the
// six bits assembled inside each 16-bit half at bit 4 (u >> 1) (the nibble
// where it lies, qh's two bits above it): an exact f16 subnormal q6 2^(4 (u
// >> 1) - 24). Run m is live in lane groups q with q >> 1 == (m & 1), half
// hf = q & 1 of its values, in MFMA (m >> 3, (m >> 1) & 3).
template <>
struct RF<INFERNO_Q6_K> {
  static constexpr int kBytes = 210;
  typedef mfma_decode::half2v half2v_t;
  __host__ __device__ static int run_shift(int r) { return 4 * ((r >> 2) & 1); }
  template <int NA>
  __device__ static void dot(const uint8_t* blk, const uint32_t* const (&cols)[NA],
                             const uint32_t* zero, int n, int q, floatx4 (&C)[NA]) {
    const bool act_q = (q >> 1) == (n & 1);
    const int mh = n >> 3, mu = (n >> 1) & 3;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t l0[2], l1[2], hw[2];
      lds_words_a2(blk + 64 * h + 8 * q, l0);
      lds_words_a2(blk + 64 * h + 32 + 8 * q, l1);
      lds_words_a2(blk + 128 + 32 * h + 8 * q, hw);
      const uint2 hq = make_uint2(hw[0], hw[1]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t w0 = (u & 1) ? l1[0] : l0[0], w1 = (u & 1) ? l1[1] : l0[1];
        const int nb = 4 * (u >> 1);  // the field's bit offset
        const uint32_t M = 0x000f000fu << nb, MH = 0x00300030u << nb;
        // qh bits 2 u, 2 u + 1 of each byte moved to bits nb + 4, nb + 5
        auto hb = [&](uint32_t x) {
          const int sh = nb + 4 - 2 * u;
          return (sh >= 0 ? (x << sh) : (x >> -sh)) & MH;
        };
        const uint4 bv = make_uint4((w0 & M) | hb(hq.x), ((w0 >> 8) & M) | hb(hq.x >> 8),
                                    (w1 & M) | hb(hq.y), ((w1 >> 8) & M) | hb(hq.y >> 8));
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          const uint32_t* src = (act_q && mh == h && mu == u) ? cols[a] + n * 8 + 4 * (q & 1) : zero;
          C[a] = mfma(load_a(src), bv, C[a]);
        }
      }
    }
  }
  __device__ static float epilogue(const uint8_t* blk, floatx4 C, float4 sums, float4 kk,
                                   int q) {
    // runs 4 q + j: int8 scales at bytes 192 + 4 q + j
    uint32_t sws[1];
    lds_words_a2(blk + 192 + 4 * q, sws);
    const uint32_t sw = sws[0];
    const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk + 208));
    const float c[4] = {C[0], C[1], C[2], C[3]};
    const float s[4] = {sums.x, sums.y, sums.z, sums.w};
    const float f[4] = {kk.x, kk.y, kk.z, kk.w};
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float sc = float(int8_t((sw >> (8 * j)) & 0xffu));
      acc = fmaf(sc, fmaf(c[j] * f[j], kTwoM24, -32.0f * s[j]), acc);
    }
    return d * acc;
  }
};

// Bit offset at which format `quant` keeps the fields of run r (r < 16) of a
// super-block column: the scale the runs of h are staged with for the down
// kernel of that format.
__device__ __forceinline__ int run_shift_of(int quant, int r) {
  switch (quant) {
    case INFERNO_Q4_K: return RF<INFERNO_Q4_K>::run_shift(r);
    case INFERNO_Q6_K: return RF<INFERNO_Q6_K>::run_shift(r);
    default: return RF<INFERNO_Q2_K>::run_shift(r);  // Q2_K, Q3_K
  }
}

// ------------------------------------------------------------- staging

// Words per staged x row: one f16 term (bf16 tokens), or two (fp32 tokens:
// the hi pairs, run sums and factors as above, then the lo pairs K/2).
__host__ __device__ constexpr int xrun_words(int K, bool split) {
  return run_words(K) + (split ? K / 2 : 0);
}
// Word offset of the lo pairs in a split row.
__host__ __device__ constexpr int xrun_lo(int K) { return run_words(K); }
// The lo term carries (v - hi) 2^11, so the products of one run add up as
// C_hi + 2^-11 C_lo: about 22 significant bits of each fp32 value.
constexpr float kLoScale = 2048.0f, kLoInv = 1.0f / 2048.0f;

// Stages one 16-value run held one value per lane by a 16-lane group (lane i
// of the group holds value i; all 16 call it) into the run row layout above,
// values scaled by s_run 2^-shift; SPLIT also writes the lo term.
template <bool SPLIT = false>
__device__ __forceinline__ void stage_run16(float v, uint32_t* row, int K, int run, int shift) {
  const int lane = threadIdx.x & 63, i = lane & 15;
  float m = fabsf(v), sum = v;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    m = fmaxf(m, __shfl_xor(m, o, 16));
    sum += __shfl_xor(sum, o, 16);
  }
  float s = 1.0f;  // zero or non-finite runs keep scale 1
  if (m > 0.f && m < 3.0e38f) {
    int e;
    frexpf(m, &e);
    s = ldexpf(1.0f, 15 - e);
  }
  const float vs = v * (s * ldexpf(1.0f, -shift));
  const _Float16 hv = (_Float16)vs;
  const uint32_t hb = __builtin_bit_cast(uint16_t, hv);
  const int j = i & 7, base = 4 * (j >> 1) + (j & 1);
  const uint32_t h0 = __shfl(hb, base, 16), h1 = __shfl(hb, base + 2, 16);
  if (i < 8) row[run * 8 + j] = h0 | (h1 << 16);
  if constexpr (SPLIT) {
    // vs - hv is exact in fp32 (hv is vs rounded), and below half an f16
    // step of hv, so 2^11 times it stays in range
    const _Float16 lv = (_Float16)((vs - (float)hv) * kLoScale);
    const uint32_t lb = __builtin_bit_cast(uint16_t, lv);
    const uint32_t l0 = __shfl(lb, base, 16), l1 = __shfl(lb, base + 2, 16);
    if (i < 8) row[xrun_lo(K) + run * 8 + j] = l0 | (l1 << 16);
  }
  if (i == 0) {
    float* sums = reinterpret_cast<float*>(row + K / 2);
    sums[run] = sum;
    sums[K / 16 + run] = 16777216.0f * 16777216.0f / s;
  }
}

// LDS pitch of a tile row of rb bytes: rows of an even number of 16-byte
// chunks get 16 bytes of padding (an odd pitch in 16-byte units puts the 16
// rows a lane group reads on distinct banks); others stay packed (a tile is
// then one contiguous run of chunks).
__host__ __device__ constexpr int row_pitch(int rb) { return rb % 32 == 0 ? rb + 16 : rb; }
// Stores 16-byte chunk i of a tile of rows of rb bytes at pitch row_pitch(rb).
__device__ __forceinline__ void store_tile_chunk(uint8_t* tl, int rb, int i, const u32x4& v) {
  if (rb % 32 == 0) {
    const int cr = rb / 16, row = i / cr;
    *reinterpret_cast<u32x4*>(tl + row * (rb + 16) + (i - row * cr) * 16) = v;
  } else {
    *reinterpret_cast<u32x4*>(tl + 16 * i) = v;
  }
}

// ------------------------------------------------------------- gate/up

// Persistent over 16-row tiles t = blockIdx.x + j gridDim.x of the active
// slots (gate and up rows of one expert, 2 x 16 x NB x kBytes contiguous
// bytes, loaded into registers, stored to LDS, the next tile's loads in
// flight while this one is computed). x is the token's staged run row (bf16
// tokens: exact in f16 with the run scale), copied to LDS once. Units (matrix, column) are spread
// over the wavefronts; the gate and up sums meet in LDS in wavefront order.
// h = silu(gate) * up * w goes out as a staged run row for the down kernel.
template <int Q, int NB>
struct GateUpShape {
  static constexpr int H = NB * kKBlock;
  static constexpr int rb = NB * RF<Q>::kBytes;
  static constexpr int Sx = run_words(H);
  static constexpr int chunks = 2 * 16 * rb / 16;  // per tile
  static constexpr int PER = (chunks + kThreads - 1) / kThreads;
};

template <int Q, int NB>
__host__ __device__ constexpr size_t gate_up_runs_lds() {
  using S = GateUpShape<Q, NB>;
  return size_t(S::Sx + 4) * 4 + size_t(2 * 16) * row_pitch(S::rb) + size_t(kWaves * 2 * 16) * 4 +
         size_t(3 * kMaxExperts) * 4;
}

template <int Q, int NB>
__global__ void __launch_bounds__(kThreads) gate_up_runs_kernel(DecodeArgs p, int ntiles) {
  using S = GateUpShape<Q, NB>;
  extern __shared__ uint32_t smem[];
  constexpr int rb = S::rb, PER = S::PER, Sx = S::Sx, H = S::H;
  const int I = p.I;
  uint32_t* xs = smem;
  uint32_t* zero = smem + Sx;
  constexpr int RS = row_pitch(rb);
  uint8_t* tl = reinterpret_cast<uint8_t*>(zero + 4);                     // [2][16 rows at pitch RS]
  float* part = reinterpret_cast<float*>(tl + 2 * 16 * RS);              // [wave][2][16]
  uint32_t* slot_e = reinterpret_cast<uint32_t*>(part + kWaves * 2 * 16);
  uint32_t* slot_a = slot_e + kMaxExperts;
  float* slot_w = reinterpret_cast<float*>(slot_a + kMaxExperts);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, q = lane >> 4;
  const int tiles_i = I / kRows;
  u32x4 v[PER];
  auto fetch = [&](int t, uint32_t expert) {
    const size_t off = size_t(expert) * p.gate_stride + size_t(t % tiles_i) * 16 * size_t(rb);
    const u32x4* g4 = reinterpret_cast<const u32x4*>(p.gate + off);
    const u32x4* u4 = reinterpret_cast<const u32x4*>(p.up + off);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      int i = j * kThreads + tid;
      i = i < S::chunks ? i : S::chunks - 1;  // clamped; the extra chunks are not stored
      v[j] = mfma_decode::ld_tile(i < S::chunks / 2 ? g4 + i : u4 + (i - S::chunks / 2));
    }
  };
  int t = blockIdx.x;
  if (t < ntiles) fetch(t, p.slots[t / tiles_i].x);
  for (int i = tid; i < Sx / 4; i += kThreads)
    reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(p.stage_xr)[i];
  if (tid < 4) zero[tid] = 0;
  for (int j = tid; j < p.max_slots; j += kThreads) {
    const uint4 sl = p.slots[j];
    slot_e[j] = sl.x;
    slot_a[j] = sl.w;
    slot_w[j] = p.weights[sl.w];
  }
  const float* sums = reinterpret_cast<const float*>(xs + H / 2);
  const float* kks = sums + H / 16;
  for (; t < ntiles; t += gridDim.x) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = j * kThreads + tid;
      if (i < S::chunks) store_tile_chunk(tl, rb, i, v[j]);
    }
    __syncthreads();
    if (t + int(gridDim.x) < ntiles) fetch(t + gridDim.x, slot_e[(t + gridDim.x) / tiles_i]);
    const int slot = t / tiles_i, tile = t - slot * tiles_i;
    float acc[2] = {0.f, 0.f};
    for (int u = wave; u < 2 * NB; u += kWaves) {
      const int mat = u & 1, c = u >> 1;
      const uint8_t* blk = tl + (mat * 16 + n) * RS + c * RF<Q>::kBytes;
      const float4 xsum = *reinterpret_cast<const float4*>(sums + c * 16 + 4 * q);
      const float4 kk = *reinterpret_cast<const float4*>(kks + c * 16 + 4 * q);
      const uint32_t* const cols[1] = {xs + c * 128};
      floatx4 C[1] = {{0.f, 0.f, 0.f, 0.f}};
      RF<Q>::template dot<1>(blk, cols, zero, n, q, C);
      const float r = RF<Q>::epilogue(blk, C[0], xsum, kk, q);
      acc[0] += mat == 0 ? r : 0.f;
      acc[1] += mat == 1 ? r : 0.f;
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      float r = acc[m];
      r += __shfl_xor(r, 16, kWave);
      r += __shfl_xor(r, 32, kWave);
      if (q == 0) part[(wave * 2 + m) * 16 + n] = r;
    }
    __syncthreads();
    // lanes 0..15 sum gate rows, 16..31 up rows, over the wavefronts in
    // order; the next tile's LDS writes start only after a barrier these
    // lanes also reach
    if (tid < 32) {
      float r = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) r += part[(w * 2 + (tid >> 4)) * 16 + (tid & 15)];
      const float u = __shfl_down(r, 16, kWave);
      const uint32_t a = slot_a[slot];  // the slot's (single) assignment
      const float h = silu(r) * u * slot_w[slot];
      if (tid < 16)
        stage_run16(h, p.stage_h + size_t(a) * run_words(I), I, tile,
                    run_shift_of(p.h_quant, tile & 15));
    }
  }
}

// ------------------------------------------------------------------ down

// Output tile = TR rows of H over all k ranks (rank r's down rows [TR t,
// TR t + TR) of expert e_r, TR * NB * kBytes contiguous bytes each); block
// (rank, column) = one block dot against h_r (staged run rows written by the
// gate/up kernel). Lanes n >= TR read row TR - 1 again and are not written.
// out = (residual + shared down) + routed, wavefronts summed in order:
// deterministic, no float atomics.
template <int Q, int NB, int TR>
struct DownShape {
  static constexpr int K = NB * kKBlock;  // the expert intermediate I
  static constexpr int rb = NB * RF<Q>::kBytes;
  static constexpr int Sh = run_words(K);
  static_assert(TR * rb % 16 == 0, "a rank tile must be whole 16-byte chunks");
};

// k: the ranks the kernel sums (the routed k, plus the shared expert when
// it runs as rank k)
template <int Q, int NB, int TR>
__host__ __device__ constexpr size_t down_runs_lds(int k) {
  using S = DownShape<Q, NB, TR>;
  return size_t(k * S::Sh + 4) * 4 + size_t(k * TR) * S::rb + size_t(kWaves * 16) * 4 +
         size_t(kMaxTopK + 1) * 4;
}

template <int Q, int NB, int TR>
__host__ __device__ constexpr int down_runs_per(int k) {
  return (k * TR * NB * RF<Q>::kBytes / 16 + kThreads - 1) / kThreads;
}

template <int Q, int NB, int TR, int PER>
__global__ void __launch_bounds__(kThreads) down_runs_kernel(DecodeArgs p, int ntiles) {
  using S = DownShape<Q, NB, TR>;
  extern __shared__ uint32_t smem[];
  constexpr int K = S::K, rb = S::rb, Sh = S::Sh;
  constexpr int cr = TR * rb / 16;  // 16-byte chunks per rank tile
  const int k = p.k + p.shared_slot;  // ranks summed: rank p.k is the shared expert
  uint32_t* hs = smem;                                     // [k][Sh]
  uint32_t* zero = hs + k * Sh;
  uint8_t* tl = reinterpret_cast<uint8_t*>(zero + 4);     // [k][TR rows of rb], contiguous
  float* part = reinterpret_cast<float*>(tl + k * TR * rb);  // [wave][16]
  uint32_t* rank_e = reinterpret_cast<uint32_t*>(part + kWaves * 16);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, q = lane >> 4;
  const int nr = n < TR ? n : TR - 1;
  if (tid < p.k) rank_e[tid] = p.ids[tid];
  if (tid == p.k && p.shared_slot) rank_e[tid] = kSharedId;
  u32x4 v[PER];
  auto fetch = [&](int t) {
    const int nv = k * cr;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      int i = j * kThreads + tid;
      i = i < nv ? i : nv - 1;  // clamped; the extra chunks are not stored
      const int r = i / cr, w = i - r * cr;
      const uint32_t e = rank_e[r];
      const uint8_t* base = e == kSharedId ? p.sdown : p.down + size_t(e) * p.down_stride;
      const u32x4* src = reinterpret_cast<const u32x4*>(base + size_t(t) * TR * rb);
      v[j] = mfma_decode::ld_tile(src + w);
    }
  };
  int t = blockIdx.x;
  __syncthreads();
  if (t < ntiles) fetch(t);
  for (int i = tid; i < k * Sh / 4; i += kThreads)
    reinterpret_cast<uint4*>(hs)[i] = reinterpret_cast<const uint4*>(p.stage_h)[i];
  if (tid < 4) zero[tid] = 0;
  const int nblk = k * NB;
  for (; t < ntiles; t += gridDim.x) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = j * kThreads + tid;
      if (i < k * cr) *reinterpret_cast<u32x4*>(tl + 16 * i) = v[j];
    }
    __syncthreads();
    if (t + int(gridDim.x) < ntiles) fetch(t + gridDim.x);
    // the output rows' residual and shared down, fetched now so that the
    // epilogue below does not wait for them
    float base = 0.f;
    if (tid < TR) {
      const size_t o = size_t(t) * TR + tid;
      base = (p.residual ? p.residual[o] : 0.f) + (p.ys ? p.ys[o] : 0.f);
    }
    float acc = 0.f;
    for (int b = wave; b < nblk; b += kWaves) {
      const int r = b / NB, c = b - r * NB;
      const uint32_t* hr = hs + r * Sh;
      const float* sums = reinterpret_cast<const float*>(hr + K / 2);
      const float4 hsum = *reinterpret_cast<const float4*>(sums + c * 16 + 4 * q);
      const float4 kk = *reinterpret_cast<const float4*>(sums + K / 16 + c * 16 + 4 * q);
      const uint8_t* blk = tl + (r * TR + nr) * rb + c * RF<Q>::kBytes;
      const uint32_t* const cols[1] = {hr + c * 128};
      floatx4 C[1] = {{0.f, 0.f, 0.f, 0.f}};
      RF<Q>::template dot<1>(blk, cols, zero, n, q, C);
      acc += RF<Q>::epilogue(blk, C[0], hsum, kk, q);
    }
    acc += __shfl_xor(acc, 16, kWave);
    acc += __shfl_xor(acc, 32, kWave);
    if (q == 0) part[wave * 16 + n] = acc;
    __syncthreads();
    if (tid < TR) {
      float y = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) y += part[w * 16 + tid];
      p.out[size_t(t) * TR + tid] = base + y;
    }
  }
}

// ------------------------------------------------- several tokens (T > 1)
//
// Below the prefill threshold with T > 1 the layer's assignments are grouped
// by expert (the select launch's slots: expert, assignment range); each
// expert tile is computed once for all of the expert's tokens. Workgroup b
// takes tiles b, b + G, ... of the (slot, tile) list (G = grid size), so the
// tiles in flight at any time are neighbours in HBM. With a tile's weights
// the kernel prefetches, into registers, the staged rows (x for gate/up, h
// for down) of the first NT tokens of the tile's slot; a slot with more
// tokens runs its further chunks of NT with a synchronous load from L2.
// Every token takes the same block dot (RF<Q>::dot against that token's run
// row); fp32 tokens add the lo term's MFMAs (NA = 2).

// Assignment c of slot sl (its first one is kept in the descriptor).
__device__ __forceinline__ uint32_t slot_assignment(const DecodeArgs& p, const uint4& sl, uint32_t c) {
  return c == sl.y ? sl.w : p.sorted[c];
}

// Copies the staged rows (words each) of nt entries into LDS rows of the
// same width; `src(i)` gives entry i's row.
template <int WV = kWaves, typename Src>
__device__ __forceinline__ void load_rows(uint32_t* dst, int words, int nt, Src src) {
  const int w4 = words / 4;
  for (int i = threadIdx.x; i < nt * w4; i += (64 * WV)) {
    const int e = i / w4, o = i - e * w4;
    reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src(e))[o];
  }
}

// Register prefetch of the first NT entries' staged rows (W4 16-byte words
// each) of a slot: entry e = i / W4 of flat index i = x (64 * WV) + tid.
template <int NT, int W4, int WV = kWaves>
struct RowPrefetch {
  static constexpr int XP = (NT * W4 + (64 * WV) - 1) / (64 * WV);
  u32x4 v[XP];
  uint32_t a[XP];  // the entry's assignment (kept where i % W4 == 0)
  // `row(a)` is assignment a's staged row
  template <typename Row>
  __device__ __forceinline__ void load(const DecodeArgs& p, const uint4& sl, int nt, Row row) {
#pragma unroll
    for (int x = 0; x < XP; ++x) {
      const int i = x * (64 * WV) + int(threadIdx.x);
      if (i < nt * W4) {
        const int e = i / W4;
        a[x] = slot_assignment(p, sl, sl.y + uint32_t(e));
        v[x] = reinterpret_cast<const u32x4*>(row(a[x]))[i - e * W4];
      }
    }
  }
  __device__ __forceinline__ void store(uint32_t* dst, uint32_t* tok_a, int nt) const {
#pragma unroll
    for (int x = 0; x < XP; ++x) {
      const int i = x * (64 * WV) + int(threadIdx.x);
      if (i < nt * W4) {
        reinterpret_cast<u32x4*>(dst)[i] = v[x];
        if (i % W4 == 0) tok_a[i / W4] = a[x];
      }
    }
  }
};

template <int Q, int NB, bool SPLIT, int NT, int WV = kWaves>
struct MultiGateUpShape {
  static constexpr int H = NB * kKBlock;
  static constexpr int rb = NB * RF<Q>::kBytes;
  static constexpr int Sx = xrun_words(H, SPLIT);
  static constexpr int chunks = 2 * 16 * rb / 16;
  static constexpr int PER = (chunks + (64 * WV) - 1) / (64 * WV);
};

// LDS of the selecting variant's additions: topk1_wave's scratch and the
// slot table (expert, assignment, routing weight per slot)
constexpr size_t kSelMultiLds = 8 + sizeof(Top1Lds) + size_t(3 * (kMaxTopK + 1)) * 4;

template <int Q, int NB, bool SPLIT, int NT, bool SEL = false, int WV = kWaves>
__host__ __device__ constexpr size_t gate_up_multi_lds() {
  using S = MultiGateUpShape<Q, NB, SPLIT, NT, WV>;
  return size_t(NT) * S::Sx * 4 + 16 + size_t(2 * 16) * row_pitch(S::rb) +
         size_t(WV * NT * 16) * 4 + size_t(2 * NT) * 4 + (SEL ? kSelMultiLds : 0);
}

// SEL (one token, no shared expert in this launch's epilogue): the kernel
// selects itself, as gate_up_fp4_kernel's prologue does (wavefront 15 of
// every workgroup: the route launch's logit partials, topk1_wave) into an
// LDS slot table (slot j = the j-th smallest selected id, its one
// assignment = its rank, its routing weight), and workgroup 0 writes the
// ids, weights and dispatch for the down launch: no select launch.
template <int Q, int NB, bool SPLIT, int NT, bool SEL = false, int WV = kWaves>
__global__ void __launch_bounds__(64 * WV) gate_up_runs_multi_kernel(DecodeArgs p) {
  using S = MultiGateUpShape<Q, NB, SPLIT, NT, WV>;
  constexpr int NA = SPLIT ? 2 : 1;
  extern __shared__ uint32_t smem[];
  constexpr int rb = S::rb, PER = S::PER, Sx = S::Sx, H = S::H, RS = row_pitch(rb);
  const int I = p.I, k = p.k;
  uint32_t* xs = smem;                                              // [NT][Sx]
  uint32_t* zero = xs + NT * Sx;
  uint8_t* tl = reinterpret_cast<uint8_t*>(zero + 4);               // [2][16 rows at pitch RS]
  float* part = reinterpret_cast<float*>(tl + 2 * 16 * RS);         // [wave][NT][16]
  uint32_t* tok_ab = reinterpret_cast<uint32_t*>(part + WV * NT * 16);  // [2][NT]
  // SEL: topk1_wave's scratch (8-byte aligned: every region above is a
  // whole number of 8-byte words) and the slot table
  Top1Lds* tk = reinterpret_cast<Top1Lds*>(tok_ab + 2 * NT);
  // (kMaxTopK + 1 entries: the shared expert as slot k)
  uint32_t* sel_e = reinterpret_cast<uint32_t*>(tk + 1);
  uint32_t* sel_a = sel_e + kMaxTopK + 1;
  float* sel_w = reinterpret_cast<float*>(sel_a + kMaxTopK + 1);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, q = lane >> 4;
  const int tiles_i = I / kRows;
  int ntiles;
  if constexpr (SEL) {
    if (wave == WV - 1) {
      __builtin_amdgcn_s_setprio(3);
      float lg[4], bs[4];
      load_logits1(p, lg, bs);
      topk1_wave_narrow(lg, bs, p.E, k, p.score_fn, p.norm, p.scale, tk);
      if (lane < k) {  // slot j = j-th smallest id, assignment = its rank
        const uint32_t rank = tk->rank[lane];
        sel_e[lane] = tk->id[lane];
        sel_a[lane] = rank;
        sel_w[lane] = tk->w[rank];
      }
      if (lane == 0 && p.shared_slot) {  // the shared expert: assignment k, weight 1
        sel_e[k] = kSharedId;
        sel_a[k] = uint32_t(k);
        sel_w[k] = 1.0f;
      }
      __builtin_amdgcn_s_setprio(0);
      if (blockIdx.x == 0) select1_write(p, tk);
    }
    __syncthreads();
    ntiles = (k + p.shared_slot) * tiles_i;  // one token: every slot is a distinct expert
  } else {
    ntiles = int(p.active[0]) * tiles_i;
  }
  // slot j's descriptor {expert, first, end, first assignment} and the
  // routing weight of assignment a (of slot j)
  auto slot_of = [&](int j) -> uint4 {
    if constexpr (SEL) return make_uint4(sel_e[j], uint32_t(j), uint32_t(j + 1), sel_a[j]);
    else return p.slots[j];
  };
  auto weight_of = [&](int j, uint32_t a) -> float {
    if constexpr (SEL) return sel_w[j];
    else return p.weights[a];
  };
  int t = blockIdx.x;
  if (t >= ntiles) return;  // uniform per workgroup
  u32x4 v[PER];
  RowPrefetch<NT, Sx / 4, WV> xr;
  // token of assignment a (the shared expert's assignments T k + t follow
  // the routed ones)
  const uint32_t Tk = uint32_t(p.T) * uint32_t(k);
  auto row_of = [&](uint32_t a) {
    return p.stage_xr + size_t(a < Tk ? a / uint32_t(k) : a - Tk) * Sx;
  };
  auto fetch = [&](int tt) {
    const uint4 s2 = slot_of(tt / tiles_i);
    const size_t off = size_t(tt % tiles_i) * 16 * size_t(rb);
    const bool sh = s2.x == kSharedId;
    const u32x4* g4 =
        reinterpret_cast<const u32x4*>((sh ? p.sgate : p.gate + size_t(s2.x) * p.gate_stride) + off);
    const u32x4* u4 =
        reinterpret_cast<const u32x4*>((sh ? p.sup : p.up + size_t(s2.x) * p.gate_stride) + off);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      int i = j * (64 * WV) + tid;
      i = i < S::chunks ? i : S::chunks - 1;  // clamped; the extra chunks are not stored
      v[j] = mfma_decode::ld_tile(i < S::chunks / 2 ? g4 + i : u4 + (i - S::chunks / 2));
    }
    xr.load(p, s2, min(NT, int(s2.z - s2.y)), row_of);
  };
  fetch(t);
  if (tid < 4) zero[tid] = 0;
  // SEL: the down launch's workgroup of this index (on the same XCD) starts
  // with its tile blockIdx.x. Under this workgroup's last tile, its tile
  // registers v (free from then on) load the k (+ shared) ranks' rows of
  // that down tile, as far as kWarmPer chunks per thread reach; the data is
  // not used, the loads leave the rows in this XCD's L2. Ordinary loads the
  // compiler counts: nothing waits for them until the sink at the end.
  constexpr int kWarmPer = SEL ? (PER < 4 ? PER : 4) : 0;
  auto warm_down = [&]() {
    if (!p.dpf_rows || int(blockIdx.x) >= p.H / p.dpf_rows) return;  // uniform
    const size_t tb = size_t(p.dpf_rows) * size_t(p.dpf_row_bytes);
    const int cr = int(tb / 16), nc = (k + p.shared_slot) * cr;
#pragma unroll
    for (int j = 0; j < kWarmPer; ++j) {
      const int i = min(j * (64 * WV) + tid, nc - 1), r = i / cr, w = i - r * cr;
      const uint32_t e = sel_e[r];
      const uint8_t* base = e == kSharedId ? p.sdown : p.down + size_t(e) * p.down_stride;
      v[j] = reinterpret_cast<const u32x4*>(base + size_t(blockIdx.x) * tb)[w];
    }
  };
  const int mat = wave & 1;  // units (mat, c) = wave + 16 j: the matrix is the wave's parity
  for (int it = 0; t < ntiles; t += gridDim.x, ++it) {
    const int slot = t / tiles_i, tile = t - slot * tiles_i;
    const uint4 sl = slot_of(slot);
    // the assignments of the chunk in LDS; two buffers, so this store does
    // not race the previous tile's h staging (which reads the other one)
    uint32_t* tok_a = tok_ab + (it & 1) * NT;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = j * (64 * WV) + tid;
      if (i < S::chunks) store_tile_chunk(tl, rb, i, v[j]);
    }
    xr.store(xs, tok_a, min(NT, int(sl.z - sl.y)));
    __syncthreads();
    if (t + int(gridDim.x) < ntiles) fetch(t + gridDim.x);
    else if constexpr (kWarmPer > 0) warm_down();  // the last tile of this workgroup
    for (int c0 = int(sl.y); c0 < int(sl.z); c0 += NT) {
      const int nt = min(NT, int(sl.z) - c0);
      if (c0 != int(sl.y)) {  // a later chunk of a slot with more than NT tokens
        __syncthreads();      // the previous chunk's readers of tok_a / part / xs are done
        if (tid < nt) tok_a[tid] = slot_assignment(p, sl, uint32_t(c0 + tid));
        __syncthreads();
        load_rows<WV>(xs, Sx, nt, [&](int e) { return row_of(tok_a[e]); });
        __syncthreads();
      }
      // one token at a time (the tile's blocks are read from LDS again per
      // token; a register array over the tokens would spill)
      for (int ti = 0; ti < nt; ++ti) {
        const uint32_t* row = xs + ti * Sx;
        const float* sums = reinterpret_cast<const float*>(row + H / 2);
        float acc = 0.f;
        for (int c = wave >> 1; c < NB; c += WV / 2) {
          const uint8_t* blk = tl + (mat * 16 + n) * RS + c * RF<Q>::kBytes;
          const float4 xsum = *reinterpret_cast<const float4*>(sums + c * 16 + 4 * q);
          const float4 kk = *reinterpret_cast<const float4*>(sums + H / 16 + c * 16 + 4 * q);
          uint32_t const* cols[NA];
          cols[0] = row + c * 128;
          if constexpr (SPLIT) cols[NA - 1] = row + xrun_lo(H) + c * 128;
          floatx4 C[NA];
#pragma unroll
          for (int a = 0; a < NA; ++a) C[a] = floatx4{0.f, 0.f, 0.f, 0.f};
          RF<Q>::template dot<NA>(blk, cols, zero, n, q, C);
          floatx4 Ce = C[0];
          if constexpr (SPLIT) {
#pragma unroll
            for (int i = 0; i < 4; ++i) Ce[i] = fmaf(C[NA - 1][i], kLoInv, Ce[i]);
          }
          acc += RF<Q>::epilogue(blk, Ce, xsum, kk, q);
        }
        acc += __shfl_xor(acc, 16, kWave);
        acc += __shfl_xor(acc, 32, kWave);
        if (q == 0) part[(wave * NT + ti) * 16 + n] = acc;
      }
      __syncthreads();
      // a 16-lane group per token: gate rows from the even wavefronts, up
      // rows from the odd ones, in wavefront order
      if (tid < 16 * nt) {
        const int ti = tid >> 4, row = tid & 15;
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int w = 0; w < WV; w += 2) {
          g += part[(w * NT + ti) * 16 + row];
          u += part[((w + 1) * NT + ti) * 16 + row];
        }
        const uint32_t a = tok_a[ti];
        const float h = silu(g) * u * weight_of(slot, a);
        stage_run16(h, p.stage_h + size_t(a) * run_words(I), I, tile,
                    run_shift_of(p.h_quant, tile & 15));
      }
      // the next writes of part and xs come after a barrier these lanes reach
    }
  }
  if constexpr (kWarmPer > 0) {  // sink of the warm-up loads: the kernel ends after them
#pragma unroll
    for (int j = 0; j < kWarmPer; ++j) asm volatile("" : : "v"(v[j]));
  }
}

// Down for T > 1: tile = (slot, 16 RG rows of H); unit (row group g, column
// c) = one block dot per token of the slot against its h row; the column
// partials meet in LDS and are summed in column order into y[a] (fp32 rows per
// assignment, combined over the ranks by the combine launch).
template <int Q, int NB, int RG, int NT>
struct MultiDownShape {
  static constexpr int K = NB * kKBlock;  // the expert intermediate I
  static constexpr int rb = NB * RF<Q>::kBytes;
  static constexpr int Sh = run_words(K);
  static constexpr int rows = 16 * RG;
  static constexpr int chunks = rows * rb / 16;
  static constexpr int PER = (chunks + kThreads - 1) / kThreads;
  static_assert(rows * rb % 16 == 0, "a down tile must be whole 16-byte chunks");
};

template <int Q, int NB, int RG, int NT>
__host__ __device__ constexpr size_t down_multi_lds() {
  using S = MultiDownShape<Q, NB, RG, NT>;
  return size_t(NT) * S::Sh * 4 + 16 + size_t(S::rows) * row_pitch(S::rb) +
         size_t(RG * NB * NT * 16) * 4 + size_t(2 * NT) * 4;
}

template <int Q, int NB, int RG, int NT>
__global__ void __launch_bounds__(kThreads) down_runs_multi_kernel(DecodeArgs p) {
  using S = MultiDownShape<Q, NB, RG, NT>;
  extern __shared__ uint32_t smem[];
  constexpr int K = S::K, rb = S::rb, Sh = S::Sh, PER = S::PER, RS = row_pitch(rb);
  const int H = p.H;
  uint32_t* hs = smem;                                              // [NT][Sh]
  uint32_t* zero = hs + NT * Sh;
  uint8_t* tl = reinterpret_cast<uint8_t*>(zero + 4);               // [rows at pitch RS]
  float* part = reinterpret_cast<float*>(tl + S::rows * RS);        // [RG * NB][NT][16]
  uint32_t* tok_ab = reinterpret_cast<uint32_t*>(part + RG * NB * NT * 16);  // [2][NT]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, q = lane >> 4;
  const int tiles_h = H / S::rows;
  const int ntiles = int(p.active[0]) * tiles_h;
  int t = blockIdx.x;
  if (t >= ntiles) return;  // uniform per workgroup
  u32x4 v[PER];
  RowPrefetch<NT, Sh / 4> hr_pf;
  auto row_of = [&](uint32_t a) { return p.stage_h + size_t(a) * Sh; };
  auto fetch = [&](int tt) {
    const uint4 s2 = p.slots[tt / tiles_h];
    const u32x4* src = reinterpret_cast<const u32x4*>(
        p.down + size_t(s2.x) * p.down_stride + size_t(tt % tiles_h) * S::rows * size_t(rb));
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      int i = j * kThreads + tid;
      i = i < S::chunks ? i : S::chunks - 1;  // clamped; the extra chunks are not stored
      v[j] = mfma_decode::ld_tile(src + i);
    }
    hr_pf.load(p, s2, min(NT, int(s2.z - s2.y)), row_of);
  };
  fetch(t);
  if (tid < 4) zero[tid] = 0;
  for (int it = 0; t < ntiles; t += gridDim.x, ++it) {
    const int slot = t / tiles_h, rt = t - slot * tiles_h;
    const uint4 sl = p.slots[slot];
    uint32_t* tok_a = tok_ab + (it & 1) * NT;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = j * kThreads + tid;
      if (i < S::chunks) store_tile_chunk(tl, rb, i, v[j]);
    }
    hr_pf.store(hs, tok_a, min(NT, int(sl.z - sl.y)));
    __syncthreads();
    if (t + int(gridDim.x) < ntiles) fetch(t + gridDim.x);
    for (int c0 = int(sl.y); c0 < int(sl.z); c0 += NT) {
      const int nt = min(NT, int(sl.z) - c0);
      if (c0 != int(sl.y)) {  // a later chunk of a slot with more than NT tokens
        __syncthreads();      // the previous chunk's readers of tok_a / part / hs are done
        if (tid < nt) tok_a[tid] = slot_assignment(p, sl, uint32_t(c0 + tid));
        __syncthreads();
        load_rows(hs, Sh, nt, [&](int e) { return row_of(tok_a[e]); });
        __syncthreads();
      }
      for (int u = wave; u < RG * NB; u += kWaves) {
        const int g = u / NB, c = u - g * NB;
        const uint8_t* blk = tl + (g * 16 + n) * RS + c * RF<Q>::kBytes;
        for (int ti = 0; ti < nt; ++ti) {
          const uint32_t* hr = hs + ti * Sh;
          const float* sums = reinterpret_cast<const float*>(hr + K / 2);
          const float4 hsum = *reinterpret_cast<const float4*>(sums + c * 16 + 4 * q);
          const float4 kk = *reinterpret_cast<const float4*>(sums + K / 16 + c * 16 + 4 * q);
          const uint32_t* const cols[1] = {hr + c * 128};
          floatx4 C[1] = {{0.f, 0.f, 0.f, 0.f}};
          RF<Q>::template dot<1>(blk, cols, zero, n, q, C);
          float r = RF<Q>::epilogue(blk, C[0], hsum, kk, q);
          r += __shfl_xor(r, 16, kWave);
          r += __shfl_xor(r, 32, kWave);
          if (q == 0) part[(u * NT + ti) * 16 + n] = r;
        }
      }
      __syncthreads();
      for (int i = tid; i < RG * nt * 16; i += kThreads) {
        const int g = i / (nt * 16), ti = (i >> 4) % nt, row = i & 15;
        float y = 0.f;
#pragma unroll
        for (int c = 0; c < NB; ++c) y += part[((g * NB + c) * NT + ti) * 16 + row];
        p.y[size_t(tok_a[ti]) * H + size_t(rt) * S::rows + g * 16 + row] = y;
      }
      // the next writes of part and hs come after a barrier these threads reach
    }
  }
}

}  // namespace runs_decode
}  // namespace inferno
