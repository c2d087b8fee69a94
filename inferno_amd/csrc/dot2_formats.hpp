// Packed-f16 dequant-dot building blocks shared by the GEMV kernels.
//
// A 2- or 4-bit field masked in place out of a 32-bit word, two bytes apart
// (bits b and 16+b), IS a pair of f16 subnormals q*2^(b-24). One v_and_b32
// turns four quant bytes' fields into such a pair, and v_dot2_f32_f16
// multiplies it with a pair of f16 activations and adds to an fp32
// accumulator exactly (the products are exact in fp32). The field position
// and the 2^24 go into the per-group scale, the K-quant minimum into a
// per-run activation sum: ~1.5 VALU ops per weight for Q2_K.
//
// Staged activations (per row of K values, all in 32-bit words):
//   [hi pairs K/2][lo pairs K/2, fp32 inputs only][run sums K/16][run inv scales K/16]
// Every 16-value run is scaled by its own power of two so that its max|x|
// lands in [2^14, 2^15): no f16 overflow, bf16 inputs stay exact. Pairs are
// stored in the (i, i+2) order the masked fields come in. For fp32 inputs a
// second pair array holds the rounding residual x 2^12, so the product keeps
// about 22 significant bits. Run sums are of the unscaled values.
#pragma once
#include "gemv_common.hpp"

namespace inferno {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t q, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, q), __builtin_bit_cast(f16x2, x), acc,
                                false);
}

constexpr float kTwo24 = 16777216.0f;
constexpr int kRows = 16;      // rows per workgroup

// Byte `idx` (0..15, runtime) of the 16 bytes held in w0..w3, without
// indexing a register array (which would force it into scratch).
__device__ __forceinline__ uint32_t byte16(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                           int idx) {
  const uint32_t w = idx < 8 ? (idx < 4 ? w0 : w1) : (idx < 12 ? w2 : w3);
  return (w >> (8 * (idx & 3))) & 0xffu;
}

constexpr float kLo = 1.0f / 4096.0f;  // residual pairs are stored x 2^12

// Staged row (words): [hi pairs K/2][lo pairs K/2 if split][run sums K/16][run invs K/16]
__host__ __device__ constexpr int staged_stride(int K, bool split) {
  return K / 2 * (split ? 2 : 1) + K / 8;
}

// One 16-value run: eight field words against eight activation pairs.
__device__ __forceinline__ float dot8(const uint32_t f[8], uint4 a, uint4 b) {
  float t = 0.f;
  t = dot2(f[0], a.x, t);
  t = dot2(f[1], a.y, t);
  t = dot2(f[2], a.z, t);
  t = dot2(f[3], a.w, t);
  t = dot2(f[4], b.x, t);
  t = dot2(f[5], b.y, t);
  t = dot2(f[6], b.z, t);
  t = dot2(f[7], b.w, t);
  return t;
}

// Activation view of one staged row for one super-block column.
template <bool SPLIT>
struct XRow {
  const uint32_t* hi;   // pairs of this column (128 words)
  const uint32_t* lo;   // residual pairs of this column
  const float* sums;    // 16 run sums of this column (unscaled)
  const float* invs;    // 16 run inverse scales of this column
  // sum over the run of field * x, in unscaled activation units
  __device__ __forceinline__ float run(const uint32_t f[8], int r) const {
    const uint4 a = *reinterpret_cast<const uint4*>(hi + 8 * r);
    const uint4 b = *reinterpret_cast<const uint4*>(hi + 8 * r + 4);
    float t = dot8(f, a, b);
    if constexpr (SPLIT) {
      const uint4 c = *reinterpret_cast<const uint4*>(lo + 8 * r);
      const uint4 d = *reinterpret_cast<const uint4*>(lo + 8 * r + 4);
      t = fmaf(dot8(f, c, d), kLo, t);
    }
    return t * invs[r];
  }
};

// View of staged row `row` (stride staged_stride(K, SPLIT)) at super-block column `col`.
template <bool SPLIT>
__device__ __forceinline__ XRow<SPLIT> xrow_at(const uint32_t* row, int K, int col) {
  const float* sums = reinterpret_cast<const float*>(row + K / 2 * (SPLIT ? 2 : 1));
  return XRow<SPLIT>{row + col * 128, row + K / 2 + col * 128, sums + col * 16,
                     sums + K / 16 + col * 16};
}

// Stages one 16-value run (v in natural order) of a row: writes 8 hi pair
// words, 8 lo pair words when SPLIT, the run sum and the inverse scale.
template <bool SPLIT>
__device__ __forceinline__ void stage_run(const float v[16], uint32_t* row, int K, int run) {
  float m = 0.f, sum = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    m = fmaxf(m, fabsf(v[i]));
    sum += v[i];
  }
  float scale = 1.0f;  // zero or non-finite runs keep scale 1
  if (m > 0.f && m < 3.0e38f) {
    int e;
    frexpf(m, &e);  // m = f * 2^e, f in [0.5, 1)
    scale = ldexpf(1.0f, 15 - e);
  }
  uint32_t* hi = row + run * 8;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int base = 4 * (j >> 1) + (j & 1);
    const float a = v[base] * scale, b = v[base + 2] * scale;
    const _Float16 ah = (_Float16)a, bh = (_Float16)b;
    hi[j] = uint32_t(__builtin_bit_cast(uint16_t, ah)) |
            (uint32_t(__builtin_bit_cast(uint16_t, bh)) << 16);
    if constexpr (SPLIT) {
      const _Float16 al = (_Float16)((a - float(ah)) * 4096.0f);
      const _Float16 bl = (_Float16)((b - float(bh)) * 4096.0f);
      row[K / 2 + run * 8 + j] = uint32_t(__builtin_bit_cast(uint16_t, al)) |
                                 (uint32_t(__builtin_bit_cast(uint16_t, bl)) << 16);
    }
  }
  float* sums = reinterpret_cast<float*>(row + K / 2 * (SPLIT ? 2 : 1));
  sums[run] = sum;
  sums[K / 16 + run] = 1.0f / scale;
}

// ---------------------------------------------------------------- formats
// Each format: kBytes per super-block, kDw = dwords a sub-lane loads per
// super-block, kU = super-blocks batched per wavefront, load(), and dot()
// returning the block's contribution in scaled-activation units.

template <int Q>
struct Fmt;

// Q2_K [scales 16 | qs 64 | d | dmin]; sub = 2h + s; runs 8h + 2p + s.
template <>
struct Fmt<INFERNO_Q2_K> {
  static constexpr int kBytes = 84;
  static constexpr int kDw = 7;
  static constexpr int kU = 2;
  __device__ static void load(const uint8_t* b, int sub, uint32_t r[kDw]) {
    const int h = sub >> 1, s = sub & 1;
    const uint4 q = ld_u4(b + 16 + 32 * h + 16 * s);
    const uint2 sc = ld_u2(b + 8 * h);
    r[0] = q.x; r[1] = q.y; r[2] = q.z; r[3] = q.w;
    r[4] = sc.x; r[5] = sc.y;
    r[6] = ld_u1(b + 80);
  }
  template <bool SPLIT>
  __device__ static float dot(const uint32_t r[kDw], int sub, const XRow<SPLIT>& x) {
    const int h = sub >> 1, s = sub & 1;
    // scale bytes of p = 0..3 sit at bytes s, 2+s of r[4] and of r[5]
    const uint32_t scb = __builtin_amdgcn_perm(r[5], r[4], s ? 0x07050301u : 0x06040200u);
    uint32_t odd[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) odd[j] = r[j] >> 8;
    float acc_s = 0.f, acc_m = 0.f;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int run = 8 * h + 2 * p + s;
      const uint32_t m = 0x00030003u << (2 * p);
      const uint32_t f[8] = {r[0] & m, odd[0] & m, r[1] & m, odd[1] & m,
                             r[2] & m, odd[2] & m, r[3] & m, odd[3] & m};
      const float t = x.run(f, run);
      const uint32_t byte = (scb >> (8 * p)) & 0xffu;
      acc_s = fmaf(float(byte & 15u) * (kTwo24 / float(1 << (2 * p))), t, acc_s);
      acc_m = fmaf(float(byte >> 4), x.sums[run], acc_m);
    }
    const float d = f16_bits_to_f32_fast(uint16_t(r[6]));
    const float dmin = f16_bits_to_f32_fast(uint16_t(r[6] >> 16));
    return d * acc_s - dmin * acc_m;
  }
};

// Q3_K [hmask 32 | qs 64 | scales 12 | d]; sub = 2n + half; runs g = 8n + 2j + half.
template <>
struct Fmt<INFERNO_Q3_K> {
  static constexpr int kBytes = 110;
  static constexpr int kDw = 12;
  static constexpr int kU = 1;
  __device__ static void load(const uint8_t* b, int sub, uint32_t r[kDw]) {
    const int n = sub >> 1, half = sub & 1;
    const uint4 q = ld_u4(b + 32 + 32 * n + 16 * half);
    const uint4 hm = ld_u4(b + 16 * half);
    const uint4 sc = ld_u4(b + 94);  // bytes 94..109: [qs tail 2 | scales 12 | d 2]
    r[0] = q.x; r[1] = q.y; r[2] = q.z; r[3] = q.w;
    r[4] = hm.x; r[5] = hm.y; r[6] = hm.z; r[7] = hm.w;
    r[8] = sc.x; r[9] = sc.y; r[10] = sc.z; r[11] = sc.w;
  }
  template <bool SPLIT>
  __device__ static float dot(const uint32_t r[kDw], int sub, const XRow<SPLIT>& x) {
    const int n = sub >> 1, half = sub & 1;
    auto scale_byte = [&](int i) -> uint32_t { return byte16(r[8], r[9], r[10], r[11], 2 + i); };
    uint32_t qo[4], ho[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qo[j] = r[j] >> 8;
      ho[j] = r[4 + j] >> 8;
    }
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int g = 8 * n + 2 * j + half;
      const uint32_t mq = 0x00030003u << (2 * j);
      const uint32_t mh = 0x00010001u << (4 * n + j);
      const uint32_t fq[8] = {r[0] & mq, qo[0] & mq, r[1] & mq, qo[1] & mq,
                              r[2] & mq, qo[2] & mq, r[3] & mq, qo[3] & mq};
      const uint32_t fh[8] = {r[4] & mh, ho[0] & mh, r[5] & mh, ho[1] & mh,
                              r[6] & mh, ho[2] & mh, r[7] & mh, ho[3] & mh};
      const float tq = x.run(fq, g);
      const float th = x.run(fh, g);
      // 6-bit signed group scale (crates/gguf/src/lib.rs:1317-1334)
      const uint32_t lo = g < 8 ? (scale_byte(g % 8) & 15u) : (scale_byte(g % 8) >> 4);
      const uint32_t hi = (scale_byte(8 + g % 4) >> (2 * (g / 4))) & 3u;
      const float gs = float(int(lo | (hi << 4)) - 32);
      // value = gs * (q + 4*hbit - 4)
      const float sq = kTwo24 / float(1 << (2 * j));
      const float sh = 4.0f * kTwo24 / float(1 << (4 * n + j));
      acc = fmaf(gs, sq * tq + sh * th - 4.0f * x.sums[g], acc);
    }
    return f16_bits_to_f32_fast(uint16_t(r[11] >> 16)) * acc;
  }
};

// Q4_K [d | dmin | scales 12 | qs 128]; sub = c owns qs[32c, 32c+32):
// groups 2c (low nibbles, runs 4c, 4c+1) and 2c+1 (high nibbles, runs 4c+2, 4c+3).
template <>
struct Fmt<INFERNO_Q4_K> {
  static constexpr int kBytes = 144;
  static constexpr int kDw = 12;
  static constexpr int kU = 1;
  __device__ static void load(const uint8_t* b, int sub, uint32_t r[kDw]) {
    const uint4 q0 = ld_u4(b + 16 + 32 * sub);
    const uint4 q1 = ld_u4(b + 32 + 32 * sub);
    const uint4 hd = ld_u4(b);
    r[0] = q0.x; r[1] = q0.y; r[2] = q0.z; r[3] = q0.w;
    r[4] = q1.x; r[5] = q1.y; r[6] = q1.z; r[7] = q1.w;
    r[8] = hd.x; r[9] = hd.y; r[10] = hd.z; r[11] = hd.w;
  }
  template <bool SPLIT>
  __device__ static float dot(const uint32_t r[kDw], int sub, const XRow<SPLIT>& x) {
    // scales[i], i in 0..11, at block byte 4 + i
    auto sbyte = [&](int i) -> uint32_t { return byte16(r[8], r[9], r[10], r[11], 4 + i); };
    float dsum = 0.f, msum = 0.f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int g = 2 * sub + k;
      uint32_t sc, m;
      if (g < 4) {
        sc = sbyte(g) & 63u;
        m = sbyte(g + 4) & 63u;
      } else {
        sc = (sbyte(g + 4) & 15u) | ((sbyte(g - 4) >> 6) << 4);
        m = (sbyte(g + 4) >> 4) | ((sbyte(g) >> 6) << 4);
      }
      const uint32_t mask = k == 0 ? 0x000f000fu : 0x00f000f0u;
      float t = 0.f;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const uint32_t* w = r + 4 * half;
        const uint32_t f[8] = {w[0] & mask, (w[0] >> 8) & mask, w[1] & mask, (w[1] >> 8) & mask,
                               w[2] & mask, (w[2] >> 8) & mask, w[3] & mask, (w[3] >> 8) & mask};
        t += x.run(f, 4 * sub + 2 * k + half);
      }
      dsum = fmaf(float(sc) * (k == 0 ? kTwo24 : kTwo24 / 16.0f), t, dsum);
      msum = fmaf(float(m), x.sums[4 * sub + 2 * k] + x.sums[4 * sub + 2 * k + 1], msum);
    }
    const float d = f16_bits_to_f32_fast(uint16_t(r[8]));
    const float dmin = f16_bits_to_f32_fast(uint16_t(r[8] >> 16));
    return d * dsum - dmin * msum;
  }
};

// Q8_0 super-block = eight 34-byte blocks [d | int8 x32]; sub owns blocks
// 2 sub and 2 sub + 1 (runs 4 sub .. 4 sub + 3). int8 codes enter as the
// offset-binary bytes q ^ 0x80 = q + 128; the 128 * sum(x) comes back out
// through the run sums.
template <>
struct Fmt<INFERNO_Q8_0> {
  static constexpr int kBytes = 272;
  static constexpr int kDw = 17;
  static constexpr int kU = 1;
  __device__ static void load(const uint8_t* b, int sub, uint32_t r[kDw]) {
    const uint8_t* p = b + 68 * sub;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = ld_u4(p + 16 * i);
      r[4 * i] = v.x; r[4 * i + 1] = v.y; r[4 * i + 2] = v.z; r[4 * i + 3] = v.w;
    }
    r[16] = ld_u1(p + 64);
  }
  template <bool SPLIT>
  __device__ static float dot(const uint32_t r[kDw], int sub, const XRow<SPLIT>& x) {
    // block 0: d = bytes 0-1, codes bytes 2..33; block 1: d = bytes 34-35, codes 36..67
    uint32_t q[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = __builtin_amdgcn_alignbyte(r[j + 1], r[j], 2) ^ 0x80808080u;
#pragma unroll
    for (int j = 0; j < 8; ++j) q[8 + j] = r[9 + j] ^ 0x80808080u;
    const uint32_t m = 0x00ff00ffu;
    float acc = 0.f;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      float t = 0.f;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const uint32_t* w = q + 8 * blk + 4 * half;
        const uint32_t f[8] = {w[0] & m, (w[0] >> 8) & m, w[1] & m, (w[1] >> 8) & m,
                               w[2] & m, (w[2] >> 8) & m, w[3] & m, (w[3] >> 8) & m};
        t += x.run(f, 4 * sub + 2 * blk + half);
      }
      const float d = f16_bits_to_f32_fast(blk == 0 ? uint16_t(r[0]) : uint16_t(r[8] >> 16));
      const float xs = x.sums[4 * sub + 2 * blk] + x.sums[4 * sub + 2 * blk + 1];
      acc = fmaf(d, kTwo24 * t - 128.0f * xs, acc);
    }
    return acc;
  }
};


// Waves per SIMD the single-activation kernels are compiled for: four (128
// VGPRs) where the format fits without spilling in the streaming loop,
// three (168 VGPRs) for Q3_K and for split (fp32) activations.
template <int Q, bool SPLIT>
struct Occupancy {
  static constexpr int value = (Q == INFERNO_Q3_K || SPLIT) ? 3 : 4;
};

// ------------------------------------------------------------ tile compute

// LDS floats TileDot needs for its partial sums (two matrices, `waves` wavefronts).
__host__ __device__ constexpr int tile_part_floats(int nt, int waves = 4) {
  return waves * kRows * nt * 2;
}

// One 16-row tile of one (or two: gate and up) expert matrices against NT
// staged activation rows held in LDS (`xs`, row stride S words). Lane =
// row slot * 4 + sub; the WAVES wavefronts split the super-block columns
// and meet in LDS. `row0`/`row1` point at this lane's row of each matrix.
// A wavefront loads KU columns per batch (default: the format's batch, one
// column for split activations); the first batch can be issued (prefetch)
// before the activations are in LDS, so the two memory latencies overlap.
// With WAVES * KU >= the column count every quant load of the tile is in
// flight at once.
template <int Q, int NMAT, int NT, bool SPLIT, int WAVES = 4, int KU = 0>
struct TileDot {
  using F = Fmt<Q>;
  static constexpr int kU = KU > 0 ? KU : (SPLIT ? 1 : F::kU);
  const uint8_t* row0;
  const uint8_t* row1;
  int K, bpr, wave, sub;
  uint32_t raw[NMAT][kU][F::kDw];
  float acc[NMAT][NT];

  __device__ __forceinline__ TileDot(const uint8_t* r0, const uint8_t* r1, int K_)
      : row0(r0), row1(r1), K(K_), bpr(K_ / kKBlock) {
    const int tid = threadIdx.x;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    sub = tid & 3;
  }
  __device__ __forceinline__ void load(int cb) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int col = cb + WAVES * u;
      if (col < bpr) {
        F::load(row0 + size_t(col) * F::kBytes, sub, raw[0][u]);
        if constexpr (NMAT == 2) F::load(row1 + size_t(col) * F::kBytes, sub, raw[1][u]);
      }
    }
  }
  // Issues the first batch of this wavefront's quant loads.
  __device__ __forceinline__ void prefetch() { load(wave); }
  // Dot products against the NT (nt live) staged rows; prefetch() must have
  // been called since the last run(). Ends with a barrier; afterwards
  // res[(m * kRows + slot) * NT + t] holds matrix m, row slot, activation t.
  __device__ __forceinline__ void run(const uint32_t* xs, int S, int nt, float* part, float* res) {
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[m][t] = 0.f;
    for (int cb = wave; cb < bpr; cb += WAVES * kU) {
      if (cb != wave) load(cb);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int col = cb + WAVES * u;
        if (col < bpr) {
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            if (t < nt) {
              const XRow<SPLIT> xv = xrow_at<SPLIT>(xs + t * S, K, col);
#pragma unroll
              for (int m = 0; m < NMAT; ++m) acc[m][t] += F::dot(raw[m][u], sub, xv);
            }
          }
        }
      }
    }
    const int tid = threadIdx.x, slot = (tid & 63) >> 2;
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float v = acc[m][t];
        v += __shfl_xor(v, 1, kWave);
        v += __shfl_xor(v, 2, kWave);
        if (sub == 0) part[((m * WAVES + wave) * kRows + slot) * NT + t] = v;
      }
    __syncthreads();
    if (tid < NMAT * kRows * NT) {
      const int m = tid / (kRows * NT), rest = tid % (kRows * NT);
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) v += part[(m * WAVES + w) * kRows * NT + rest];
      res[tid] = v;
    }
    __syncthreads();
  }
};

// Copies n 16-byte words from global memory into LDS with every thread of
// a THREADS-thread workgroup, DEPTH loads in flight per thread (loads clamped
// to the last word, stores guarded, so the batch stays in registers).
template <int DEPTH = 4, int THREADS = 256>
__device__ __forceinline__ void copy_to_lds(uint4* to, const uint4* from, int n) {
  const int tid = threadIdx.x;
  for (int base = 0; base < n; base += THREADS * DEPTH) {
    uint4 v[DEPTH];
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) v[j] = from[min(base + j * THREADS + tid, n - 1)];
#pragma unroll
    for (int j = 0; j < DEPTH; ++j)
      if (base + j * THREADS + tid < n) to[base + j * THREADS + tid] = v[j];
  }
}

// Copies `nt` staged rows (S words each, S a multiple of 4) into LDS; src(t)
// gives the row pointer.
template <int THREADS = 256, typename SrcFn>
__device__ __forceinline__ void copy_rows_to_lds(uint32_t* xs, int S, int nt, SrcFn src) {
  for (int t = 0; t < nt; ++t)
    copy_to_lds<4, THREADS>(reinterpret_cast<uint4*>(xs + t * S),
                            reinterpret_cast<const uint4*>(src(t)), S / 4);
}

// Stages one 16-value run held one value per lane by lanes 0..15 of a
// wavefront (lane i holds value i); the other lanes pass through. Same
// layout as stage_run<true>; the run sum is a fixed-order tree.
__device__ __forceinline__ void stage_run_lanes(float v, uint32_t* row, int K, int run) {
  const int lane = threadIdx.x & 63;
  float m = fabsf(v), sum = v;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    m = fmaxf(m, __shfl_xor(m, o, 16));
    sum += __shfl_xor(sum, o, 16);
  }
  float scale = 1.0f;  // zero or non-finite runs keep scale 1
  if (m > 0.f && m < 3.0e38f) {
    int e;
    frexpf(m, &e);
    scale = ldexpf(1.0f, 15 - e);
  }
  const float a = v * scale;
  const _Float16 ah = (_Float16)a;
  const _Float16 al = (_Float16)((a - float(ah)) * 4096.0f);
  const uint32_t hb = __builtin_bit_cast(uint16_t, ah), lb = __builtin_bit_cast(uint16_t, al);
  // pair word j holds values (base, base + 2), base = 4 (j >> 1) + (j & 1)
  const int j = lane & 7;
  const int base = 4 * (j >> 1) + (j & 1);
  const uint32_t h0 = __shfl(hb, base, 16), h1 = __shfl(hb, base + 2, 16);
  const uint32_t l0 = __shfl(lb, base, 16), l1 = __shfl(lb, base + 2, 16);
  if (lane < 8)
    row[run * 8 + j] = h0 | (h1 << 16);
  else if (lane < 16)
    row[K / 2 + run * 8 + j] = l0 | (l1 << 16);
  if (lane == 0) {
    float* sums = reinterpret_cast<float*>(row + K);
    sums[run] = sum;
    sums[K / 16 + run] = 1.0f / scale;
  }
}

// gate/up epilogue shared by the separate and the fused kernels, run by the
// first 16 lanes of wave 0 (lane s owns row s of the tile): h = silu(g) * u * w
// for activation t, written in fp32 (h_f32, may be null) and as one staged
// run (h_staged row, may be null).
__device__ __forceinline__ void swiglu_tile_out(const float* res, int NT, int t, float w,
                                                float* h_f32, uint32_t* h_staged, int I,
                                                int tile) {
  const int s = threadIdx.x & 15;
  const float g = res[s * NT + t], u = res[(kRows + s) * NT + t];
  const float v = silu(g) * u * w;
  if (h_f32) h_f32[tile * kRows + s] = v;
  if (h_staged) stage_run_lanes(v, h_staged, I, tile);
}

}  // namespace inferno
