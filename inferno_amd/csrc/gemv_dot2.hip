// Decode dequant-GEMV for K-quant experts (Q2_K, Q3_K, Q4_K) on packed-f16
// dot products.
//
// Idea: a 2- or 4-bit field masked in place out of a 32-bit word, two bytes
// apart (bits b and 16+b), IS a pair of f16 subnormals q*2^(b-24). One
// v_and_b32 turns four quant bytes' fields into such a pair, and
// v_dot2_f32_f16 multiplies it with a pair of f16 activations and adds to
// an fp32 accumulator, exactly (the products are exact in fp32). The field
// position and the 2^24 go into the per-group scale, the K-quant minimum
// into a per-run activation sum. That is ~1.5 VALU ops per weight, against
// a budget of ~1.6 at the HBM roofline for Q2_K.
//
// Activations are staged once per call (stage_rows_kernel) into a global
// buffer that every workgroup copies into LDS: scaled by a per-row power of
// two so that max|x| lands in [2^14, 2^15) (no f16 overflow, bf16 inputs
// stay exact), stored as f16 pairs in the (i, i+2) order the masked fields
// come in, plus fp32 sums of every 16-value run. fp32 inputs get a second
// f16 pair array holding the rounding residual (x 2^12), and a second dot2
// per field, so the product keeps ~22 significant bits.
//
// Work item: 16 rows of one expert (gate and up together for the SwiGLU
// stage). Lane = row slot * 4 + sub; a sub-lane owns 64 values of a
// super-block. The four wavefronts split the row's super-blocks
// (interleaved) and meet in LDS for the final sum, so each wavefront issues
// all its loads before the first dot product.
//
// Semantics follow crates/backend/src/metal/kernels/gguf_moe_kernels.metal:
// 340-565 (gate/up SwiGLU with the routing weight folded, down per
// assignment) and laguna_xs_kernels.metal:1578-1642 (Q4_K).
#include "gemv_common.hpp"

namespace inferno {
namespace {

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

// Staged row (dwords): [hi pairs K/2][lo pairs K/2 if split][run sums K/16][inv, pad 3]
__host__ __device__ constexpr int staged_stride(int K, bool split) {
  return K / 2 * (split ? 2 : 1) + K / 16 + 4;
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
  const float* sums;    // 16 run sums of this column
  __device__ __forceinline__ float run(const uint32_t f[8], int r) const {
    const uint4 a = *reinterpret_cast<const uint4*>(hi + 8 * r);
    const uint4 b = *reinterpret_cast<const uint4*>(hi + 8 * r + 4);
    float t = dot8(f, a, b);
    if constexpr (SPLIT) {
      const uint4 c = *reinterpret_cast<const uint4*>(lo + 8 * r);
      const uint4 d = *reinterpret_cast<const uint4*>(lo + 8 * r + 4);
      t = fmaf(dot8(f, c, d), kLo, t);
    }
    return t;
  }
};

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

// ------------------------------------------------------------ staging

// One workgroup per activation row: row max -> power-of-two scale -> f16
// pairs (and residual pairs when SPLIT) + run sums, written in the staged
// layout.
template <typename XT, bool SPLIT>
__global__ void __launch_bounds__(256)
    stage_rows_kernel(const XT* __restrict__ x, int K, uint32_t* __restrict__ staged) {
  __shared__ float red[4];
  __shared__ float sc_sh;
  const int tid = threadIdx.x;
  const XT* row = x + size_t(blockIdx.x) * K;
  uint32_t* dst = staged + size_t(blockIdx.x) * staged_stride(K, SPLIT);
  float m = 0.f;
  for (int i = tid; i < K; i += 256) m = fmaxf(m, fabsf(to_f32(row[i])));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) {
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float scale = 1.0f;  // zero or non-finite rows keep scale 1
    if (mx > 0.f && mx < 3.0e38f) {
      int e;
      frexpf(mx, &e);  // mx = f * 2^e, f in [0.5, 1)
      scale = ldexpf(1.0f, 15 - e);
    }
    sc_sh = scale;
    float* tail = reinterpret_cast<float*>(dst + K / 2 * (SPLIT ? 2 : 1) + K / 16);
    tail[0] = 1.0f / scale;
    tail[1] = tail[2] = tail[3] = 0.f;
  }
  __syncthreads();
  const float scale = sc_sh;
  float* sums = reinterpret_cast<float*>(dst + K / 2 * (SPLIT ? 2 : 1));
  // one run (16 values = 8 pairs) per thread iteration
  for (int run = tid; run < K / 16; run += 256) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int base = run * 16 + 4 * (j >> 1) + (j & 1);
      const float a = to_f32(row[base]) * scale, b = to_f32(row[base + 2]) * scale;
      const _Float16 ah = (_Float16)a, bh = (_Float16)b;
      dst[run * 8 + j] = uint32_t(__builtin_bit_cast(uint16_t, ah)) |
                         (uint32_t(__builtin_bit_cast(uint16_t, bh)) << 16);
      if constexpr (SPLIT) {
        const _Float16 al = (_Float16)((a - float(ah)) * 4096.0f);
        const _Float16 bl = (_Float16)((b - float(bh)) * 4096.0f);
        dst[K / 2 + run * 8 + j] = uint32_t(__builtin_bit_cast(uint16_t, al)) |
                                   (uint32_t(__builtin_bit_cast(uint16_t, bl)) << 16);
      }
      s += a + b;
    }
    sums[run] = s;
  }
}

// ------------------------------------------------------------- kernel

template <int Q, int MODE, int NT, bool SPLIT>
__device__ __forceinline__ void dot2_body(const GemvArgs& p, const uint32_t* __restrict__ staged) {
  using F = Fmt<Q>;
  constexpr bool kGateUp = MODE == kGateUpRouted || MODE == kGateUpDense;
  constexpr bool kRouted = MODE == kGateUpRouted || MODE == kDownRouted;
  constexpr int kMats = kGateUp ? 2 : 1;
  extern __shared__ uint32_t smem[];
  const int K = p.K;
  const int S = staged_stride(K, SPLIT);
  uint32_t* xs = smem;                                             // NT * S
  float* part = reinterpret_cast<float*>(smem + NT * S);          // 4 waves * 16 rows * NT * 2

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int slot = lane >> 2, sub = lane & 3;
  const int row = blockIdx.x * kRows + slot;
  const int rowc = row < p.rows ? row : p.rows - 1;

  uint32_t e = 0, lo = 0, hi = uint32_t(p.n_tokens);
  if constexpr (kRouted) {
    if (blockIdx.y >= p.active[0]) return;
    e = p.active[1 + blockIdx.y];
    lo = p.offsets[e];
    hi = p.offsets[e + 1];
  }
  const int bpr = K / kKBlock;
  const size_t row_bytes = size_t(bpr) * F::kBytes;
  const uint8_t* base0 = p.w0 + size_t(e) * p.expert_stride + size_t(rowc) * row_bytes;
  const uint8_t* base1 =
      kGateUp ? p.w1 + size_t(e) * p.expert_stride + size_t(rowc) * row_bytes : nullptr;

  for (uint32_t c0 = lo; c0 < hi; c0 += NT) {
    const int nt = int(min(uint32_t(NT), hi - c0));
    // copy the staged activation rows of this chunk into LDS (16-byte moves)
    for (int t = 0; t < nt; ++t) {
      uint32_t src = c0 + uint32_t(t);
      if constexpr (MODE == kGateUpRouted) src = p.sorted[src] / uint32_t(p.k);
      else if constexpr (MODE == kDownRouted) src = p.sorted[src];
      const uint4* from = reinterpret_cast<const uint4*>(staged + size_t(src) * S);
      uint4* to = reinterpret_cast<uint4*>(xs + t * S);
      for (int i = tid; i < S / 4; i += 256) to[i] = from[i];
    }
    __syncthreads();

    float acc[kMats][NT];
#pragma unroll
    for (int m = 0; m < kMats; ++m)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[m][t] = 0.f;

    for (int cb = wave; cb < bpr; cb += 4 * F::kU) {
      uint32_t raw[kMats][F::kU][F::kDw];
#pragma unroll
      for (int u = 0; u < F::kU; ++u) {
        const int col = cb + 4 * u;
        if (col < bpr) {
          F::load(base0 + size_t(col) * F::kBytes, sub, raw[0][u]);
          if constexpr (kGateUp) F::load(base1 + size_t(col) * F::kBytes, sub, raw[1][u]);
        }
      }
#pragma unroll
      for (int u = 0; u < F::kU; ++u) {
        const int col = cb + 4 * u;
        if (col < bpr) {
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            if (t < nt) {
              const uint32_t* xr = xs + t * S;
              const XRow<SPLIT> xv{xr + col * 128, xr + K / 2 + col * 128,
                                   reinterpret_cast<const float*>(xr + K / 2 * (SPLIT ? 2 : 1)) +
                                       col * 16};
#pragma unroll
              for (int m = 0; m < kMats; ++m) acc[m][t] += F::dot(raw[m][u], sub, xv);
            }
          }
        }
      }
    }
    // reduce: 4 sub-lanes, then 4 wavefronts through LDS
#pragma unroll
    for (int m = 0; m < kMats; ++m)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float v = acc[m][t];
        v += __shfl_xor(v, 1, kWave);
        v += __shfl_xor(v, 2, kWave);
        if (sub == 0) part[((wave * kRows + slot) * NT + t) * 2 + m] = v;
      }
    __syncthreads();
    if (tid < kRows * NT) {
      const int s = tid / NT, t = tid % NT;
      const int r = blockIdx.x * kRows + s;
      if (t < nt && r < p.rows) {
        float v[2] = {0.f, 0.f};
#pragma unroll
        for (int m = 0; m < kMats; ++m)
#pragma unroll
          for (int w = 0; w < 4; ++w) v[m] += part[((w * kRows + s) * NT + t) * 2 + m];
        const float inv = reinterpret_cast<const float*>(xs + t * S + S - 4)[0];
        const float g = v[0] * inv;
        if constexpr (MODE == kGateUpRouted) {
          const uint32_t a = p.sorted[c0 + t];
          p.out[size_t(a) * p.rows + r] = silu(g) * (v[1] * inv) * p.route_w[a];
        } else if constexpr (MODE == kGateUpDense) {
          p.out[size_t(c0 + t) * p.rows + r] = silu(g) * (v[1] * inv);
        } else if constexpr (MODE == kDownRouted) {
          p.out[size_t(p.sorted[c0 + t]) * p.rows + r] = g;
        } else {
          const size_t o = size_t(c0 + t) * p.rows + r;
          float ra = 0.f;
          if (p.yk) {
            for (int rk = 0; rk < p.k; ++rk) ra += p.yk[(size_t(c0 + t) * p.k + rk) * p.rows + r];
          } else if (p.res_a) {
            ra = p.res_a[o];
          }
          p.out[o] = ra + (p.res_b ? p.res_b[o] : 0.f) + g;
        }
      }
    }
    __syncthreads();
  }
}

// Single-token groups (decode) are held to 128 VGPRs so four workgroups fit
// per CU and a T=1 grid runs in one round; multi-token groups trade
// occupancy for accumulators.
template <int Q, int MODE, bool SPLIT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8)))
    dot2_kernel_1(GemvArgs p, const uint32_t* __restrict__ staged) {
  dot2_body<Q, MODE, 1, SPLIT>(p, staged);
}

template <int Q, int MODE, int NT, bool SPLIT>
__global__ void __launch_bounds__(256) dot2_kernel_n(GemvArgs p,
                                                     const uint32_t* __restrict__ staged) {
  dot2_body<Q, MODE, NT, SPLIT>(p, staged);
}

template <int Q, int MODE, int NT, bool SPLIT>
int launch_nt(hipStream_t s, const GemvArgs& a, const uint32_t* staged, int n_slots) {
  dim3 grid(unsigned((a.rows + kRows - 1) / kRows), unsigned(n_slots));
  const size_t lds = (size_t(NT) * staged_stride(a.K, SPLIT) + size_t(4) * kRows * NT * 2) * 4;
  if (lds > 160 * 1024) {
    set_error("activation row too long for the LDS staging buffer");
    return INFERNO_ERR_INVALID;
  }
  if constexpr (NT == 1)
    dot2_kernel_1<Q, MODE, SPLIT><<<grid, 256, lds, s>>>(a, staged);
  else
    dot2_kernel_n<Q, MODE, NT, SPLIT><<<grid, 256, lds, s>>>(a, staged);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int Q, int MODE, bool SPLIT>
int launch_q(hipStream_t s, const GemvArgs& a, const uint32_t* staged, int n_slots, int nt) {
  if (nt <= 1) return launch_nt<Q, MODE, 1, SPLIT>(s, a, staged, n_slots);
  if (nt == 2) return launch_nt<Q, MODE, 2, SPLIT>(s, a, staged, n_slots);
  return launch_nt<Q, MODE, 4, SPLIT>(s, a, staged, n_slots);
}

template <int MODE, bool SPLIT>
int launch_fmt(hipStream_t s, int quant, const GemvArgs& a, const uint32_t* staged, int n_slots,
               int nt) {
  switch (quant) {
    case INFERNO_Q2_K: return launch_q<INFERNO_Q2_K, MODE, SPLIT>(s, a, staged, n_slots, nt);
    case INFERNO_Q3_K: return launch_q<INFERNO_Q3_K, MODE, SPLIT>(s, a, staged, n_slots, nt);
    case INFERNO_Q4_K: return launch_q<INFERNO_Q4_K, MODE, SPLIT>(s, a, staged, n_slots, nt);
    case INFERNO_Q8_0: return launch_q<INFERNO_Q8_0, MODE, SPLIT>(s, a, staged, n_slots, nt);
  }
  set_error("quant kind has no packed-f16 GEMV");
  return INFERNO_ERR_INVALID;
}

}  // namespace

bool dot2_supported(int quant) {
  return quant == INFERNO_Q2_K || quant == INFERNO_Q3_K || quant == INFERNO_Q4_K ||
         quant == INFERNO_Q8_0;
}

size_t staged_bytes(size_t rows, size_t K, int x_dtype) {
  return rows * size_t(staged_stride(int(K), x_dtype == INFERNO_F32)) * 4;
}

int launch_stage(hipStream_t s, const void* x, int x_dtype, size_t rows, size_t K,
                 uint32_t* staged) {
  if (rows == 0) return INFERNO_OK;
  if (x_dtype == INFERNO_BF16)
    stage_rows_kernel<uint16_t, false><<<unsigned(rows), 256, 0, s>>>(
        static_cast<const uint16_t*>(x), int(K), staged);
  else
    stage_rows_kernel<float, true><<<unsigned(rows), 256, 0, s>>>(static_cast<const float*>(x),
                                                                  int(K), staged);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int MODE>
int launch_dot2(hipStream_t s, int quant, const GemvArgs& a, const uint32_t* staged, int x_dtype,
                int n_slots, int nt) {
  if (x_dtype == INFERNO_F32) return launch_fmt<MODE, true>(s, quant, a, staged, n_slots, nt);
  return launch_fmt<MODE, false>(s, quant, a, staged, n_slots, nt);
}

template int launch_dot2<kGateUpRouted>(hipStream_t, int, const GemvArgs&, const uint32_t*, int,
                                        int, int);
template int launch_dot2<kGateUpDense>(hipStream_t, int, const GemvArgs&, const uint32_t*, int,
                                       int, int);
template int launch_dot2<kDownRouted>(hipStream_t, int, const GemvArgs&, const uint32_t*, int,
                                      int, int);
template int launch_dot2<kDownDense>(hipStream_t, int, const GemvArgs&, const uint32_t*, int,
                                     int, int);

}  // namespace inferno
