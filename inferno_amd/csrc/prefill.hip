// Prefill MoE experts as grouped dequant-GEMMs on the gfx950 matrix cores.
//
// For every active expert e with n_e assignments (dispatch groups), gate/up:
//   h[a, :] = silu(x[t_a] G_e^T) * (x[t_a] U_e^T) * w_a      (f16 rows of h)
// then down: y[a, :] = h[a, :] D_e^T (fp32 rows per assignment), summed over
// ranks in rank order by the combine. Semantics follow the reference's
// prefill kernels (crates/backend/src/metal/kernels/gguf_moe_prefill_kernels.metal:
// 256-508 gate/up with the routing weight folded, :510-691 down, :693-714
// combine), which also run the expert products on f16 operands with fp32
// accumulation.
//
// Work item: 128 weight rows (gate and up rows together for the SwiGLU pass)
// x TM dispatch rows (TM = 128, or 32 for an expert's small remainder). Each
// wavefront owns 32 weight rows and all TM tokens, issuing
// v_mfma_f32_32x32x16_f16 with the weights as the A operand and the tokens
// as B. Every lane dequantises its own A fragments (8 values of one row per
// 16-deep k step) straight from the GGUF bytes: a quant field masked in place
// out of a 32-bit word, at bits p and 16 + p, is a pair of exact f16
// subnormals q * 2^(p-24), and one v_fma_mix per value (f16 field, fp32
// scale * 2^(24-p), fp32 offset) yields the value rounded once to f16. The
// mask takes bytes 0 and 2 (then 1 and 3) of a word, so within every group of
// eight k the operands run in the order 0 2 1 3 4 6 5 7; the f16 activations
// (x16, h16) are stored in that same order, which leaves the sum unchanged.
// The token tile (TM x 64 f16) is double buffered in LDS. Tiles come from a
// per-expert list built on the device from the dispatch, so nothing waits on
// the host.
#include "prefill.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "gemv_common.hpp"
#include "routing_dev.hpp"

namespace inferno {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2), aligned(8)));

constexpr int kUnit = 256;       // values per K unit (super-block / eight Q8_0 blocks)
constexpr int kTileN = 128;      // weight rows per workgroup
constexpr int kLdsPitch = 72;    // halfs per LDS token row (64 + 8 pad: conflict-free reads)
constexpr size_t kGemmCUs = 256;  // MI355X CUs (fixed, so a shape takes the same kernel on any device)

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }
__device__ __forceinline__ uint32_t as_u32(half2v v) { return __builtin_bit_cast(uint32_t, v); }

// v(f) = f * mult + off for both f16 subnormal fields of a masked word, in f16.
__device__ __forceinline__ uint32_t fma_pair(uint32_t fields, float mult, float off) {
  const half2v f = as_h2(fields);
  const half2v r = {(_Float16)__builtin_fmaf((float)f[0], mult, off),
                    (_Float16)__builtin_fmaf((float)f[1], mult, off)};
  return as_u32(r);
}

// Eight values from bytes 0..7 of (w0, w1) with the field under `mask` (the
// same mask in both 16-bit halves, at bit position p): value = field * mult +
// off, mult already holding the 2^(24 - p). Output order 0 2 1 3 4 6 5 7.
__device__ __forceinline__ half8 dequant8(uint32_t w0, uint32_t w1, uint32_t mask, float mult,
                                          float off) {
  const uint32_t a = fma_pair(w0 & mask, mult, off);
  const uint32_t b = fma_pair((w0 >> 8) & mask, mult, off);
  const uint32_t c = fma_pair(w1 & mask, mult, off);
  const uint32_t d = fma_pair((w1 >> 8) & mask, mult, off);
  return __builtin_bit_cast(half8, make_uint4(a, b, c, d));
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// f16 half `hi` of w, exactly widened, times m plus c in fp32 (v_fma_mix_f32).
__device__ __forceinline__ float mix_mul(uint32_t w, int hi, float m, float c) {
  const half2v h = as_h2(w);
  return __builtin_fmaf((float)h[hi], m, c);
}

// ------------------------------------------------------------- A fragments
// A lane (row i, k half kg) dequantises, for 64-value chunk QC of a K unit
// and k step s = 0..3, the values 64 QC + 16 s + 8 kg .. +8 of its row.
// load() fetches everything the four k steps of one chunk need; get()
// returns the eight f16 values of step s (order 0 2 1 3 4 6 5 7).

template <int Q>
struct Frag;

// Q2_K [scales 16 | qs 64 | d | dmin]: value j = 128 h + 32 p + l uses
// q = (qs[32 h + l] >> 2 p) & 3 and scale byte 16-group j / 16
// (crates/gguf/src/lib.rs:1226-1293).
template <>
struct Frag<INFERNO_Q2_K> {
  static constexpr int kBytes = 84, kRaw = 6;
  __device__ static void load(const uint8_t* b, int qc, int kg, uint32_t r[kRaw]) {
    const int h = qc >> 1;
    const uint2 a = ld_u2(b + 16 + 32 * h + 8 * kg);
    const uint2 c = ld_u2(b + 32 + 32 * h + 8 * kg);
    r[0] = a.x; r[1] = a.y; r[2] = c.x; r[3] = c.y;
    r[4] = ld_u1(b + 4 * qc);  // scale bytes of groups 4 qc .. 4 qc + 3
    r[5] = ld_u1(b + 80);      // d | dmin
  }
  // Group scale and min nibbles enter masked in place as f16 subnormals
  // (n * 2^-24, byte s of r[4] in half s / 2 of the word shifted by 8 (s & 1))
  // and one v_fma_mix_f32 each scales them by d * 2^(48 - 2p) and
  // -dmin * 2^24: mult = sc d 2^(24 - 2p) and off = -m dmin, each rounded
  // once as d * float(sc) is.
  template <int QC>
  __device__ static half8 get(const uint32_t r[kRaw], int s) {
    const int p = 2 * (QC & 1) + (s >> 1);
    const uint32_t sw = (s & 1) ? (r[4] >> 8) : r[4];
    const float d = f16_bits_to_f32_fast(uint16_t(r[5]));
    const float dmin = f16_bits_to_f32_fast(uint16_t(r[5] >> 16));
    const float mult = mix_mul(sw & 0x000f000fu, s >> 1, __builtin_amdgcn_ldexpf(d, 48 - 2 * p), 0.0f);
    const float off = mix_mul((sw >> 4) & 0x000f000fu, s >> 1, __builtin_amdgcn_ldexpf(-dmin, 24), 0.0f);
    return dequant8((s & 1) ? r[2] : r[0], (s & 1) ? r[3] : r[1], 0x00030003u << (2 * p), mult,
                    off);
  }
};

// Q3_K [hmask 32 | qs 64 | scales 12 | d]: value j = 128 n + 32 jj + l uses
// q = (qs[32 n + l] >> 2 jj) & 3, high bit hmask[l] bit (4 n + jj), 6-bit
// signed group scale; value = d (s6 - 32) (q + 4 hbit - 4)
// (crates/gguf/src/lib.rs:1295-1367).
template <>
struct Frag<INFERNO_Q3_K> {
  static constexpr int kBytes = 110, kRaw = 11;
  __device__ static void load(const uint8_t* b, int qc, int kg, uint32_t r[kRaw]) {
    const int n = qc >> 1;
    const uint2 qa = ld_u2(b + 32 + 32 * n + 8 * kg);
    const uint2 qb = ld_u2(b + 48 + 32 * n + 8 * kg);
    const uint2 ha = ld_u2(b + 8 * kg);
    const uint2 hb = ld_u2(b + 16 + 8 * kg);
    r[0] = qa.x; r[1] = qa.y; r[2] = qb.x; r[3] = qb.y;
    r[4] = ha.x; r[5] = ha.y; r[6] = hb.x; r[7] = hb.y;
    r[8] = ld_u1(b + 96 + 4 * (qc & 1));  // low-nibble bytes of groups (4 qc + s) % 8
    r[9] = ld_u1(b + 104);                // high-bit bytes
    r[10] = *reinterpret_cast<const uint16_t*>(b + 108);  // d
  }
  template <int QC>
  __device__ static half8 get(const uint32_t r[kRaw], int s) {
    const int n = QC >> 1, jj = 2 * (QC & 1) + (s >> 1);
    const int hshift = 4 * n + jj;
    // q + 4 hbit as a 3-bit field at the bottom of every byte: bits 0-1
    // from the shifted qs word, bit 2 (and higher bits, which the dequant
    // mask drops) from the hmask word shifted to put bit hshift at bit 2:
    // one bit-field insert (v_bfi_b32) per word
    auto field3 = [&](uint32_t q, uint32_t h) {
      const uint32_t qs = q >> (2 * jj);
      const uint32_t hs = hshift >= 2 ? (h >> (hshift - 2)) : (h << (2 - hshift));
      return (qs & 0x03030303u) | (hs & ~0x03030303u);
    };
    const uint32_t w0 = field3((s & 1) ? r[2] : r[0], (s & 1) ? r[6] : r[4]) & 0x07070707u;
    const uint32_t w1 = field3((s & 1) ? r[3] : r[1], (s & 1) ? r[7] : r[5]) & 0x07070707u;
    // the group's 6-bit scale (byte s of this chunk's four) and dl = d (s6 -
    // 32) in f16, as the reference's half dequantisation forms it (the fp32
    // product of two f16 values is exact, so one rounding)
    const uint32_t lo = QC < 2 ? (r[8] & 0x0f0f0f0fu) : ((r[8] >> 4) & 0x0f0f0f0fu);
    const uint32_t s6 = lo | (((r[9] >> (2 * QC)) & 0x03030303u) << 4);
    const int sc = int((s6 >> (8 * ((s & 1) + 2 * (s >> 1)))) & 0xffu);
    const float d = f16_bits_to_f32_fast(uint16_t(r[10]));
    const _Float16 dlh = (_Float16)(d * float(sc - 32));
    const half2v dl2 = {dlh, dlh};
    const half2v m4 = {(_Float16)-1028.0f, (_Float16)-1028.0f};
    // q + 4 hbit (0..7) in the low mantissa byte under the f16 exponent of
    // 1024 (byte 0x64 above it, one v_perm per pair): 1024 + u, exactly;
    // minus 1028 is u - 4 exactly, times dl rounds once. Pairs (bytes 0, 2)
    // and (1, 3): value order 0 2 1 3 4 6 5 7.
    auto pair = [&](uint32_t w, uint32_t sel) {
      const half2v f = as_h2(__builtin_amdgcn_perm(0x64646464u, w, sel));
      return as_u32((f + m4) * dl2);
    };
    return __builtin_bit_cast(half8, make_uint4(pair(w0, 0x04020400u), pair(w0, 0x04030401u),
                                                pair(w1, 0x04020400u), pair(w1, 0x04030401u)));
  }
};

// Q4_K [d | dmin | scales 12 | qs 128]: value j = 64 c + 32 hh + l uses
// q = (qs[32 c + l] >> 4 hh) & 15 and the 6-bit (sc, m) of group 2 c + hh
// (crates/gguf/src/lib.rs:1369-1416).
template <>
struct Frag<INFERNO_Q4_K> {
  static constexpr int kBytes = 144, kRaw = 8;
  __device__ static void load(const uint8_t* b, int qc, int kg, uint32_t r[kRaw]) {
    const uint2 a = ld_u2(b + 16 + 32 * qc + 8 * kg);
    const uint2 c = ld_u2(b + 32 + 32 * qc + 8 * kg);
    r[0] = a.x; r[1] = a.y; r[2] = c.x; r[3] = c.y;
    r[4] = ld_u1(b + 4); r[5] = ld_u1(b + 8); r[6] = ld_u1(b + 12);  // scales
    r[7] = ld_u1(b);  // d | dmin
  }
  template <int QC>
  __device__ static half8 get(const uint32_t r[kRaw], int s) {
    const int hh = s >> 1, g = 2 * QC + hh;
    auto sb = [&](int i) -> uint32_t {
      const uint32_t w = i < 4 ? r[4] : (i < 8 ? r[5] : r[6]);
      return byte_of(w, i & 3);
    };
    uint32_t sc, m;
    if (g < 4) {
      sc = sb(g) & 63u;
      m = sb(g + 4) & 63u;
    } else {
      sc = (sb(g + 4) & 15u) | ((sb(g - 4) >> 6) << 4);
      m = (sb(g + 4) >> 4) | ((sb(g) >> 6) << 4);
    }
    const float d = f16_bits_to_f32_fast(uint16_t(r[7]));
    const float dmin = f16_bits_to_f32_fast(uint16_t(r[7] >> 16));
    const float mult = __builtin_amdgcn_ldexpf(d * float(sc), 24 - 4 * hh);
    return dequant8((s & 1) ? r[2] : r[0], (s & 1) ? r[3] : r[1], 0x000f000fu << (4 * hh), mult,
                    -(dmin * float(m)));
  }
};

// Q6_K [ql 128 | qh 64 | scales 16 (int8) | d]: value j = 128 h + 32 u + l
// uses q6 = (ql[64 h + 32 (u & 1) + l] >> 4 (u >> 1)) & 15 | ((qh[32 h + l]
// >> 2 u) & 3) << 4 and value = d sc[8 h + 2 u + l / 16] (q6 - 32)
// (crates/gguf/src/lib.rs:1418-1470). Chunk qc = 2 h + (u >> 1): step s has
// u = 2 (qc & 1) + (s >> 1) and l = 16 (s & 1) + 8 kg + i. The six bits are
// assembled per byte, then one v_fma_mix per value: q6 * (d sc) - 32 d sc,
// rounded once as the reference's fp32 (d sc) (q6 - 32) is, then to f16.
template <>
struct Frag<INFERNO_Q6_K> {
  static constexpr int kBytes = 210, kRaw = 14;
  __device__ static void load(const uint8_t* b, int qc, int kg, uint32_t r[kRaw]) {
    const int h = qc >> 1;
#pragma unroll
    for (int s = 0; s < 4; ++s) {  // ql bytes 64 h + 32 (s >> 1) + 16 (s & 1) + 8 kg
      const uint2 v = ld_u2(b + 64 * h + 16 * s + 8 * kg);
      r[2 * s] = v.x;
      r[2 * s + 1] = v.y;
    }
    const uint2 q0 = ld_u2(b + 128 + 32 * h + 8 * kg);
    const uint2 q1 = ld_u2(b + 128 + 32 * h + 16 + 8 * kg);
    r[8] = q0.x; r[9] = q0.y; r[10] = q1.x; r[11] = q1.y;
    r[12] = ld_u1(b + 192 + 8 * h + 4 * (qc & 1));  // scales 8 h + 2 u + {0, 1}
    r[13] = *reinterpret_cast<const uint16_t*>(b + 208);  // d
  }
  template <int QC>
  __device__ static half8 get(const uint32_t r[kRaw], int s) {
    const int u = 2 * (QC & 1) + (s >> 1), nib = QC & 1;
    auto six = [&](uint32_t w, uint32_t x) {
      return ((w >> (4 * nib)) & 0x0f0f0f0fu) | (((x >> (2 * u)) & 0x03030303u) << 4);
    };
    const uint32_t w0 = six(r[2 * s], r[8 + 2 * (s & 1)]);
    const uint32_t w1 = six(r[2 * s + 1], r[9 + 2 * (s & 1)]);
    const float d = f16_bits_to_f32_fast(uint16_t(r[13]));
    const float dsc = d * float(int8_t(byte_of(r[12], 2 * (s >> 1) + (s & 1))));
    return dequant8(w0, w1, 0x003f003fu, __builtin_amdgcn_ldexpf(dsc, 24), -32.0f * dsc);
  }
};

// Q8_0: a K unit is eight 34-byte blocks [d | int8 x32]; value = d * q
// (crates/gguf/src/lib.rs:1472-1499). Codes enter as q ^ 0x80 = q + 128.
template <>
struct Frag<INFERNO_Q8_0> {
  static constexpr int kBytes = 272, kRaw = 10;
  __device__ static void load(const uint8_t* b, int qc, int kg, uint32_t r[kRaw]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int blk = 2 * qc + (s >> 1);
      const uint2 v = ld_u2(b + 34 * blk + 2 + 16 * (s & 1) + 8 * kg);
      r[2 * s] = v.x;
      r[2 * s + 1] = v.y;
    }
    r[8] = *reinterpret_cast<const uint16_t*>(b + 68 * qc);
    r[9] = *reinterpret_cast<const uint16_t*>(b + 68 * qc + 34);
  }
  template <int QC>
  __device__ static half8 get(const uint32_t r[kRaw], int s) {
    const float d = f16_bits_to_f32_fast(uint16_t((s >> 1) ? r[9] : r[8]));
    return dequant8(r[2 * s] ^ 0x80808080u, r[2 * s + 1] ^ 0x80808080u, 0x00ff00ffu,
                    __builtin_amdgcn_ldexpf(d, 24), -128.0f * d);
  }
};

// ------------------------------------------------------------------ GEMM

struct GemmArgs {
  const uint8_t* w0;       // gate (or the down / single matrix)
  const uint8_t* w1;       // up, null for one matrix
  size_t stride;           // bytes per expert matrix
  const uint16_t* xin;     // f16 input rows (k order 0 2 1 3 4 6 5 7), K halfs each
  uint32_t in_div;         // input row = (sorted[c] or c) / in_div
  const uint32_t* sorted;  // dispatch order, null = dense (identity)
  const float* route_w;    // routing weight per assignment, null = 1
  const uint4* tiles;      // {expert, c0, c1, 0}; null = dense tiles of TM rows
  const uint32_t* n_tiles;
  uint32_t rows;           // dense: number of rows
  int N, K;                // output rows per matrix, reduction length
  uint16_t* h_out;         // two matrices: f16 SwiGLU rows [*, N] (k order as xin)
  float* y_out;            // one matrix: fp32 rows [*, N]
};

template <int TM>
constexpr size_t gemm_lds_bytes() {
  return size_t(2) * TM * kLdsPitch * 2;
}

// Two waves per SIMD: the accumulators fit beside the operands in 256
// registers, and a second workgroup per CU hides the load latency.
template <int TM>
struct GemmOcc {
  static constexpr int value = 2;
};

template <int Q, int NMAT, int TM>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(GemmOcc<TM>::value, 8)))
    gemm_kernel(GemmArgs p) {
  using F = Frag<Q>;
  constexpr int NB = TM / 32;  // 32-token blocks
  extern __shared__ __attribute__((aligned(16))) uint16_t xs_raw[];
  auto xs = [&](int buf, int row) { return xs_raw + (size_t(buf) * TM + row) * kLdsPitch; };
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, kg = lane >> 5;
  uint32_t e = 0, c0, c1;
  if (p.tiles) {
    if (blockIdx.y >= *p.n_tiles) return;
    const uint4 t = p.tiles[blockIdx.y];
    e = t.x;
    c0 = t.y;
    c1 = t.z;
  } else {
    c0 = blockIdx.y * TM;
    c1 = min(c0 + uint32_t(TM), p.rows);
  }
  const int n0 = blockIdx.x * kTileN;
  const int K = p.K;
  const size_t row_bytes = size_t(K / kUnit) * F::kBytes;
  const size_t roff = size_t(e) * p.stride + size_t(n0 + 32 * wave + i) * row_bytes;
  const uint8_t* w0 = p.w0 + roff;
  const uint8_t* w1 = NMAT == 2 ? p.w1 + roff : nullptr;

  // token rows this thread stages: piece pc (8 halfs) of rows (tid >> 3) + 32 j
  const int pc = tid & 7;
  const uint16_t* src[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const uint32_t c = c0 + uint32_t((tid >> 3) + 32 * j);
    src[j] = nullptr;
    if (c < c1) {
      const uint32_t a = p.sorted ? p.sorted[c] : c;
      src[j] = p.xin + size_t(a / p.in_div) * K + 8 * pc;
    }
  }
  uint4 xv[NB];
  auto load_x = [&](int st) {
#pragma unroll
    for (int j = 0; j < NB; ++j)
      xv[j] = src[j] ? *reinterpret_cast<const uint4*>(src[j] + 64 * st) : make_uint4(0, 0, 0, 0);
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int j = 0; j < NB; ++j)
      *reinterpret_cast<uint4*>(xs(buf, (tid >> 3) + 32 * j) + 8 * pc) = xv[j];
  };

  floatx16 acc0[NB], acc1[NB];
#pragma unroll
  for (int tb = 0; tb < NB; ++tb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      acc0[tb][v] = 0.f;
      acc1[tb][v] = 0.f;
    }
  }
  // PD + 1 register sets for the quant bytes: chunk g (= 4 kb + qc) uses
  // set qc % (PD + 1), and the loads of chunk g + PD are in flight while it
  // is computed. PD = 3 keeps ~3x the bytes in flight; the two formats with
  // the most raw words per chunk would spill at 128 tokens and keep PD = 1.
  constexpr int PD = (NMAT == 2 && TM == 128 && (Q == INFERNO_Q3_K || Q == INFERNO_Q8_0)) ? 1 : 3;
  constexpr int NS = PD + 1;
  uint32_t ra[NS][F::kRaw], rb[NS][F::kRaw];
  const int nkb = K / kUnit;
  const int nch = 4 * nkb;
  load_x(0);
#pragma unroll
  for (int g = 0; g < PD; ++g) {
    if (g < nch) {
      F::load(w0 + size_t(g / 4) * F::kBytes, g & 3, kg, ra[g % NS]);
      if constexpr (NMAT == 2) F::load(w1 + size_t(g / 4) * F::kBytes, g & 3, kg, rb[g % NS]);
    }
  }
  store_x(0);
  __syncthreads();

  auto step = [&](auto qc_c, int kb) __attribute__((always_inline)) {
    constexpr int QC = decltype(qc_c)::value;
    constexpr int buf = QC & 1;
    constexpr int PQ = (QC + PD) & 3;          // chunk of chunk g + PD within its block
    constexpr int PS = (QC + PD) % NS;         // its register set
    constexpr int CS = QC % NS;                // this chunk's register set
    const int st = 4 * kb + QC;
    const bool more = st + 1 < nch;
    if (more) load_x(st + 1);
    if (st + PD < nch) {
      const size_t boff = size_t(kb + (QC + PD) / 4) * F::kBytes;
      F::load(w0 + boff, PQ, kg, ra[PS]);
      if constexpr (NMAT == 2) F::load(w1 + boff, PQ, kg, rb[PS]);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const half8 a0 = F::template get<QC>(ra[CS], s);
      half8 a1;
      if constexpr (NMAT == 2) a1 = F::template get<QC>(rb[CS], s);
#pragma unroll
      for (int tb = 0; tb < NB; ++tb) {
        const half8 b = *reinterpret_cast<const half8*>(xs(buf, tb * 32 + i) + 16 * s + 8 * kg);
        acc0[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b, acc0[tb], 0, 0, 0);
        if constexpr (NMAT == 2)
          acc1[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b, acc1[tb], 0, 0, 0);
      }
    }
    if (more) store_x(buf ^ 1);
    __syncthreads();
  };
  for (int kb = 0; kb < nkb; ++kb) {
    step(std::integral_constant<int, 0>{}, kb);
    step(std::integral_constant<int, 1>{}, kb);
    step(std::integral_constant<int, 2>{}, kb);
    step(std::integral_constant<int, 3>{}, kb);
  }

  // accumulator element v of lane (i, kg): weight row 8 (v / 4) + 4 kg + v % 4
  // of this wavefront's 32, token column i of the 32-token block
#pragma unroll
  for (int tb = 0; tb < NB; ++tb) {
    const uint32_t c = c0 + uint32_t(tb * 32 + i);
    if (c >= c1) continue;
    const uint32_t a = p.sorted ? p.sorted[c] : c;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int r0 = n0 + 32 * wave + 8 * g4 + 4 * kg;
      if constexpr (NMAT == 2) {
        const float wa = p.route_w ? p.route_w[a] : 1.0f;
        float h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          h[r] = silu(acc0[tb][4 * g4 + r]) * acc1[tb][4 * g4 + r] * wa;
        // rows r0 .. r0 + 3 stored in the k order 0 2 1 3 of the next GEMM
        const half2v lo = {(_Float16)h[0], (_Float16)h[2]};
        const half2v hi = {(_Float16)h[1], (_Float16)h[3]};
        *reinterpret_cast<uint2*>(p.h_out + size_t(a) * p.N + r0) = make_uint2(as_u32(lo), as_u32(hi));
      } else {
        *reinterpret_cast<float4*>(p.y_out + size_t(a) * p.N + r0) =
            make_float4(acc0[tb][4 * g4], acc0[tb][4 * g4 + 1], acc0[tb][4 * g4 + 2],
                        acc0[tb][4 * g4 + 3]);
      }
    }
  }
}

// ------------------------------------------------- LDS-staged weight GEMM
// The same product for the K-quant formats whose super-block fits LDS twice
// over at 512 rows (Q2_K, Q3_K), with two changes measured to matter more
// than the dequantisation: (1) weights are fetched with contiguous dword
// loads, each wavefront instruction covering whole super-blocks of two or
// three rows, a quarter of the next K unit per 64-deep step, and stored to LDS, where every lane reads
// its fragment; loading fragments straight from their rows touches 32 rows
// per instruction and cost more than the token traffic; (2) a workgroup of
// eight wavefronts covers 256 rows of each matrix, so each token tile
// (TM x 64 f16 from LDS) feeds twice the rows of the four-wavefront kernel
// (WAVES = 8; WAVES = 4 keeps two workgroups per CU).

template <int Q>
struct Stage;
// Q2_K: 84 bytes = 21 words per row, rows 21 words apart in LDS (an odd
// pitch: 32-bit fragment reads of 32 rows spread over the banks); three rows
// per wavefront load instruction.
template <>
struct Stage<INFERNO_Q2_K> {
  static constexpr int kWords = 21, kPitch = 21;
  using Chunk = uint32_t;
  __device__ static Chunk load(const uint8_t* b) { return ld_u1(b); }
  __device__ static void put(uint32_t* row, int j, Chunk v) { row[j] = v; }
  __device__ static int offset(int j) { return 4 * j; }
  __device__ static void frag(const uint32_t* row, int qc, int kg, uint32_t r[6]) {
    const int h = qc >> 1;
    const uint32_t* a = row + 4 + 8 * h + 2 * kg;
    r[0] = a[0]; r[1] = a[1]; r[2] = a[4]; r[3] = a[5];
    r[4] = row[qc];
    r[5] = row[20];
  }
};
// Q3_K: 110 bytes per row; word 27 is the dword at byte 106 (d in its high
// half), so no load passes the super-block. The staged words are the loaded
// ones as they are: nothing uses a loaded value before its LDS store, so the
// loads stay in flight through the step's MFMAs.
template <>
struct Stage<INFERNO_Q3_K> {
  static constexpr int kWords = 28, kPitch = 28;
  using Chunk = uint32_t;
  __device__ static Chunk load(const uint8_t* b) { return ld_u1(b); }
  __device__ static void put(uint32_t* row, int j, Chunk v) { row[j] = v; }
  __device__ static int offset(int j) { return j == 27 ? 106 : 4 * j; }
  __device__ static void frag(const uint32_t* row, int qc, int kg, uint32_t r[11]) {
    const int n = qc >> 1;
    const u32x2a qa = *reinterpret_cast<const u32x2a*>(row + 8 + 8 * n + 2 * kg);
    const u32x2a qb = *reinterpret_cast<const u32x2a*>(row + 12 + 8 * n + 2 * kg);
    const u32x2a ha = *reinterpret_cast<const u32x2a*>(row + 2 * kg);
    const u32x2a hb = *reinterpret_cast<const u32x2a*>(row + 4 + 2 * kg);
    r[0] = qa.x; r[1] = qa.y; r[2] = qb.x; r[3] = qb.y;
    r[4] = ha.x; r[5] = ha.y; r[6] = hb.x; r[7] = hb.y;
    r[8] = row[24 + (qc & 1)];
    r[9] = row[26];
    r[10] = row[27] >> 16;
  }
};
// Q4_K: 144 bytes per row, fetched as nine 16-byte chunks (seven rows per
// wavefront load instruction) and stored as dwords at an odd pitch of 37
// words; Frag<Q4_K>'s words read back from LDS.
template <>
struct Stage<INFERNO_Q4_K> {
  static constexpr int kWords = 9, kPitch = 37;
  using Chunk = uint4;
  __device__ static int offset(int j) { return 16 * j; }
  __device__ static Chunk load(const uint8_t* b) { return ld_u4(b); }
  __device__ static void put(uint32_t* row, int j, Chunk v) {
    row[4 * j] = v.x; row[4 * j + 1] = v.y; row[4 * j + 2] = v.z; row[4 * j + 3] = v.w;
  }
  __device__ static void frag(const uint32_t* row, int qc, int kg, uint32_t r[8]) {
    const uint32_t* a = row + 4 + 8 * qc + 2 * kg;  // qs bytes 16 + 32 qc + 8 kg
    r[0] = a[0]; r[1] = a[1]; r[2] = a[4]; r[3] = a[5];
    r[4] = row[1]; r[5] = row[2]; r[6] = row[3];  // scales
    r[7] = row[0];                                // d | dmin
  }
};

// Q6_K: 210 bytes per row, fetched as thirteen 16-byte chunks (bytes
// 0..207) and a fourteenth, bytes 194..209, of which only the last dword
// (d in its high half) is kept, so no load passes the super-block; stored as
// 53 dwords per row (an odd pitch); Frag<Q6_K>'s words read back from LDS.
template <>
struct Stage<INFERNO_Q6_K> {
  static constexpr int kWords = 14, kPitch = 53;
  using Chunk = uint4;
  __device__ static int offset(int j) { return j == 13 ? 194 : 16 * j; }
  __device__ static Chunk load(const uint8_t* b) { return ld_u4(b); }
  __device__ static void put(uint32_t* row, int j, Chunk v) {
    if (j == 13) {
      row[52] = v.w;
      return;
    }
    row[4 * j] = v.x; row[4 * j + 1] = v.y; row[4 * j + 2] = v.z; row[4 * j + 3] = v.w;
  }
  __device__ static void frag(const uint32_t* row, int qc, int kg, uint32_t r[14]) {
    const int h = qc >> 1;
#pragma unroll
    for (int s = 0; s < 4; ++s) {  // ql bytes 64 h + 16 s + 8 kg
      r[2 * s] = row[16 * h + 4 * s + 2 * kg];
      r[2 * s + 1] = row[16 * h + 4 * s + 2 * kg + 1];
    }
    r[8] = row[32 + 8 * h + 2 * kg];  // qh bytes 128 + 32 h + 8 kg
    r[9] = row[33 + 8 * h + 2 * kg];
    r[10] = row[36 + 8 * h + 2 * kg];  // qh bytes 144 + 32 h + 8 kg
    r[11] = row[37 + 8 * h + 2 * kg];
    r[12] = row[48 + 2 * h + (qc & 1)];  // scales 8 h + 4 (qc & 1) ..
    r[13] = row[52] >> 16;               // d
  }
};

// Q8_0: a K unit is 272 bytes (eight 34-byte blocks), fetched as 17
// 16-byte chunks per row (three rows per wavefront load instruction) and
// stored as dwords at an odd pitch of 69 words. The int8 codes of the even
// blocks start 2 bytes past a word boundary and are realigned from three
// words; those of the odd blocks are word aligned.
template <>
struct Stage<INFERNO_Q8_0> {
  static constexpr int kWords = 17, kPitch = 69;
  using Chunk = uint4;
  __device__ static int offset(int j) { return 16 * j; }
  __device__ static Chunk load(const uint8_t* b) { return ld_u4(b); }
  __device__ static void put(uint32_t* row, int j, Chunk v) {
    row[4 * j] = v.x; row[4 * j + 1] = v.y; row[4 * j + 2] = v.z; row[4 * j + 3] = v.w;
  }
  __device__ static void frag(const uint32_t* row, int qc, int kg, uint32_t r[10]) {
    // block 2 qc: codes at byte 68 qc + 2 + 16 s + 8 kg (s = 0, 1)
    const uint32_t* ev = row + 17 * qc + 2 * kg;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t w0 = ev[4 * s], w1 = ev[4 * s + 1], w2 = ev[4 * s + 2];
      r[2 * s] = __builtin_amdgcn_alignbyte(w1, w0, 2);
      r[2 * s + 1] = __builtin_amdgcn_alignbyte(w2, w1, 2);
    }
    // block 2 qc + 1: codes at byte 68 qc + 36 + 16 s + 8 kg
    const uint32_t* od = row + 17 * qc + 9 + 2 * kg;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      r[4 + 2 * s] = od[4 * s];
      r[5 + 2 * s] = od[4 * s + 1];
    }
    r[8] = row[17 * qc] & 0xffffu;  // d of block 2 qc (bytes 0..1)
    r[9] = row[17 * qc + 8] >> 16;  // d of block 2 qc + 1 (bytes 34..35)
  }
};

// Halfs per LDS token row of a buffer of XG 64-deep steps (+ 8 pad).
constexpr int x_pitch(int XG) { return 64 * (XG > 1 ? XG : 1) + 8; }

template <int Q, int NMAT, int TM, int WR, int SB = 0, int XU = 0>
constexpr size_t gemm2_lds_bytes() {
  return size_t(2) * TM * x_pitch(XU) * 2 +
         size_t(SB ? 1 : 2) * 32 * WR * NMAT * Stage<Q>::kPitch * 4;
}

// WR x WT wavefronts: wavefront (wr, wt) computes weight rows 32 wr .. + 32
// of each matrix for token blocks wt NBW .. + NBW (NBW = TM / 32 / WT);
// WT = 2 halves the accumulators per wavefront (each row group's fragments
// are then dequantised by two wavefronts). OCC = waves per SIMD. SB = 1:
// one weight buffer in LDS; the next K unit is held in registers (all four
// quarters) and stored after an extra barrier at the end of the unit, so the
// workgroup needs half the LDS and more of them fit on a CU (measured on the
// Q3_K down over 32 tokens: four waves per SIMD, 0.61 vs 0.84 ms).
// SPL = 1 (gate/up only): each wavefront computes one matrix (wavefronts
// 0..WR-1 gate, WR..2WR-1 up), halving its fragment and accumulator
// registers; after the K loop the up wavefronts pass their sums to the gate
// wavefronts through the (then free) LDS for the SwiGLU.
// XU = XG in {2, 4}: the token tile of XG 64-deep steps (TM x 64 XG f16) is
// double buffered instead of each step's, loaded into registers at the
// group's first step and stored into the other buffer at its last, so a K
// unit takes 4 / XG barriers (XG = 4 with SB = 1: two, around the next
// unit's weight stores) instead of four or five, and the wavefronts drift
// apart between them (one's dequantisation beside another's MFMA).
template <int Q, int NMAT, int TM, int PF, int WR, int WT, int OCC, int SB = 0, int SPL = 0,
          int XU = 0>
__global__ void __launch_bounds__(64 * (SPL ? 2 * WR : WR * WT))
    __attribute__((amdgpu_waves_per_eu(OCC, OCC))) gemm2_kernel(GemmArgs p) {
  using F = Frag<Q>;
  using S = Stage<Q>;
  static_assert(!SPL || (NMAT == 2 && WT == 1), "matrix split: gate/up, no token split");
  static_assert(!SPL || size_t(WR) * (TM / 32) * 16 * 64 * 4 <= gemm2_lds_bytes<Q, NMAT, TM, WR, SB, XU>(),
                "the up sums passed through LDS fit in the workgroup's LDS");
  static_assert(XU == 0 || XU == 2 || XU == 4, "token buffers of 1, 2 or 4 steps");
  static_assert(!(SB && XU == 2), "the single weight buffer takes whole-unit token buffers");
  constexpr int XG = XU ? XU : 1;   // 64-deep steps per token buffer
  constexpr int XPitch = x_pitch(XU);
  constexpr int XPR = 8 * XG;  // 16-byte token pieces per row of a buffer
  constexpr int WAVES = SPL ? 2 * WR : WR * WT;
  constexpr int NB = TM / 32;
  static_assert(NB % WT == 0, "token blocks split evenly over WT");
  constexpr int NBW = NB / WT;          // token blocks per wavefront
  constexpr int NT = 64 * WAVES;        // threads
  constexpr int TN = 32 * WR;           // weight rows per matrix
  constexpr int R = TN * NMAT;          // staged weight rows
  static_assert(R % WAVES == 0, "staged rows split evenly over wavefronts");
  constexpr int RW = R / WAVES;         // rows staged by one wavefront
  constexpr int RPI = 64 / S::kWords;   // rows per load instruction
  constexpr int NI = (RW + RPI - 1) / RPI;
  constexpr int XP = (TM * XPR + NT - 1) / NT;  // 16-byte token pieces per thread
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* xs_base = smem;
  uint32_t* ws_base = reinterpret_cast<uint32_t*>(smem + 2 * TM * XPitch);
  auto xs = [&](int buf, int row) { return xs_base + (size_t(buf) * TM + row) * XPitch; };
  auto wsr = [&](int buf, int rr) { return ws_base + (size_t(SB ? 0 : buf) * R + rr) * S::kPitch; };
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, kg = lane >> 5;
  const int wr = wave % WR, wt = SPL ? 0 : wave / WR;
  const int mw = SPL ? wave / WR : 0;  // this wavefront's matrix (SPL)
  uint32_t e = 0, c0, c1;
  if (p.tiles) {
    if (blockIdx.y >= *p.n_tiles) return;
    const uint4 t = p.tiles[blockIdx.y];
    e = t.x;
    c0 = t.y;
    c1 = t.z;
  } else {
    c0 = blockIdx.y * TM;
    c1 = min(c0 + uint32_t(TM), p.rows);
  }
  if (c1 <= c0) return;  // uniform: no rows (the epilogue's clamped reads need one)
  const int n0 = blockIdx.x * TN;
  const int K = p.K;
  const size_t row_bytes = size_t(K / kUnit) * F::kBytes;

  // weight staging: lane covers word j of row (lane / kWords) of each
  // instruction's RPI rows; wavefront rows [wave RW, wave RW + RW) of the
  // R staged rows (matrix (wave RW) / 256)
  const int lrow = lane / S::kWords, j = lane - lrow * S::kWords;
  const int woff = S::offset(j);
  const bool wlane = lrow < RPI;
  const int rr0 = wave * RW;
  const uint8_t* wm = (NMAT == 2 && rr0 >= TN) ? p.w1 : p.w0;
  const uint8_t* wsrc = wm + size_t(e) * p.stride + size_t(n0 + rr0 % TN + lrow) * row_bytes + woff;
  // the next K unit is fetched in NP parts of NQ load instructions: PF = 1,
  // a quarter per 64-deep step, stored at the end of that step; PF = 2,
  // halves at steps 0 and 1, each stored two steps later (more registers,
  // twice the latency covered)
  constexpr int NP = (PF == 1 || SB) ? 4 : 2;
  constexpr int NQ = (NI + NP - 1) / NP;
  typename S::Chunk wv[SB ? 4 : PF][NQ];
  auto gload_w = [&](int kb, int part, int slot) {
    const uint8_t* b = wsrc + size_t(kb) * F::kBytes;
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int q = part * NQ + u;
      if (q < NI && wlane && q * RPI + lrow < RW) wv[slot][u] = S::load(b + size_t(q * RPI) * row_bytes);
    }
  };
  auto store_w = [&](int buf, int part, int slot) {
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int q = part * NQ + u;
      if (q < NI && wlane && q * RPI + lrow < RW) S::put(wsr(buf, rr0 + q * RPI + lrow), j, wv[slot][u]);
    }
  };

  // token staging: piece c = tid + NT q -> row c / XPR, 8 halfs at 8 (c % XPR)
  const uint16_t* src[XP];
#pragma unroll
  for (int q = 0; q < XP; ++q) {
    const int c = tid + NT * q, row = c / XPR;
    const uint32_t cc = c0 + uint32_t(row);
    src[q] = nullptr;
    if (row < TM && cc < c1) {
      const uint32_t a = p.sorted ? p.sorted[cc] : cc;
      src[q] = p.xin + size_t(a / p.in_div) * K + 8 * (c % XPR);
    }
  }
  // token pieces of step t (XU: of step group t) sit in register slot
  // t % PF (XU: slot 0) until stored
  constexpr int XS = XU ? 1 : PF;
  uint4 xv[XS][XP];
  auto load_x = [&](int st, int slot) {
#pragma unroll
    for (int q = 0; q < XP; ++q)
      xv[slot][q] = src[q] ? *reinterpret_cast<const uint4*>(src[q] + 64 * XG * st)
                           : make_uint4(0, 0, 0, 0);
  };
  auto store_x = [&](int buf, int slot) {
#pragma unroll
    for (int q = 0; q < XP; ++q) {
      const int c = tid + NT * q;
      if (XP * NT == TM * XPR || c < TM * XPR)
        *reinterpret_cast<uint4*>(xs(buf, c / XPR) + 8 * (c % XPR)) = xv[slot][q];
    }
  };

  floatx16 acc0[NBW], acc1[NBW];
#pragma unroll
  for (int tb = 0; tb < NBW; ++tb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      acc0[tb][v] = 0.f;
      acc1[tb][v] = 0.f;
    }
  }
  const int nkb = K / kUnit;
  const int nch = 4 * nkb;
#pragma unroll
  for (int part = 0; part < NP; ++part) {
    gload_w(0, part, 0);
    store_w(0, part, 0);
  }
  load_x(0, 0);
  store_x(0, 0);
  if (!XU && PF == 2 && 1 < nch) load_x(1, 1 % PF);
  __syncthreads();

  auto step = [&](auto qc_c, int kb) __attribute__((always_inline)) {
    constexpr int QC = decltype(qc_c)::value;
    const int st = 4 * kb + QC;
    const int grp = st / XG;  // token group (XU) of this step
    const int buf = grp & 1;
    const bool more = st + 1 < nch;
    // x of step st + PF into slot (st + PF) % PF (XU: of the next step group
    // at this group's first step); weights of unit kb + 1
    if constexpr (XU) {
      if (QC % XG == 0 && (grp + 1) * XG < nch) load_x(grp + 1, 0);
    } else if (st + PF < nch) {
      load_x(st + PF, QC % PF);
    }
    if (kb + 1 < nkb) {
      if constexpr (SB) gload_w(kb + 1, QC, QC);
      else if constexpr (PF == 1) gload_w(kb + 1, QC, 0);
      else if constexpr (QC < 2) gload_w(kb + 1, QC, QC);
    }
    uint32_t ra[F::kRaw], rb[F::kRaw];
    if constexpr (SPL) {
      S::frag(wsr(kb & 1, mw * TN + 32 * wr + i), QC, kg, ra);
    } else {
      S::frag(wsr(kb & 1, 32 * wr + i), QC, kg, ra);
      if constexpr (NMAT == 2) S::frag(wsr(kb & 1, TN + 32 * wr + i), QC, kg, rb);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const half8 a0 = F::template get<QC>(ra, s);
      half8 a1;
      if constexpr (NMAT == 2 && !SPL) a1 = F::template get<QC>(rb, s);
#pragma unroll
      for (int tb = 0; tb < NBW; ++tb) {
        const half8 b = *reinterpret_cast<const half8*>(xs(buf, (wt * NBW + tb) * 32 + i) +
                                                        64 * (QC % XG) + 16 * s + 8 * kg);
        acc0[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b, acc0[tb], 0, 0, 0);
        if constexpr (NMAT == 2 && !SPL)
          acc1[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b, acc1[tb], 0, 0, 0);
      }
    }
    if constexpr (XU) {
      // the next group's tokens into the other buffer (free since the last
      // group's end barrier); SB: one barrier pair per unit around the next
      // unit's weights (every wavefront done with this unit's); else the
      // next unit's weights go, a quarter per step, into the other weight
      // buffer (read by no one during this unit) and a barrier ends each
      // token group
      if (QC % XG == XG - 1 && (grp + 1) * XG < nch) store_x(buf ^ 1, 0);
      if constexpr (SB) {
        if (QC == 3 && kb + 1 < nkb) {
          __syncthreads();
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) store_w(0, qq, qq);
          __syncthreads();
        }
      } else {
        if (kb + 1 < nkb) {
          if constexpr (PF == 1) store_w((kb + 1) & 1, QC, 0);
          else if constexpr (QC >= 2) store_w((kb + 1) & 1, QC - 2, QC - 2);
        }
        if (QC % XG == XG - 1) __syncthreads();
      }
      return;
    }
    if (more) store_x(buf ^ 1, (QC + 1) % PF);
    if constexpr (SB) {
      if (QC == 3 && kb + 1 < nkb) {
        __syncthreads();  // every wavefront is done with this unit's weights
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) store_w(0, qq, qq);
      }
    } else if (kb + 1 < nkb) {
      if constexpr (PF == 1) store_w((kb + 1) & 1, QC, 0);
      else if constexpr (QC >= 2) store_w((kb + 1) & 1, QC - 2, QC - 2);
    }
    __syncthreads();
  };
  for (int kb = 0; kb < nkb; ++kb) {
    step(std::integral_constant<int, 0>{}, kb);
    step(std::integral_constant<int, 1>{}, kb);
    step(std::integral_constant<int, 2>{}, kb);
    step(std::integral_constant<int, 3>{}, kb);
  }

  // accumulator element v of lane (i, kg): weight row 8 (v / 4) + 4 kg + v % 4
  // of this wavefront's 32, token column i of the 32-token block. The
  // assignment of each of the lane's token columns is loaded here, for every
  // token block at once and from a clamped index (a load under the bound
  // check would be waited for at the check's join), so it is in flight
  // through the exchange below; the routing weights follow in one round trip.
  uint32_t asg[NBW];
#pragma unroll
  for (int tb = 0; tb < NBW; ++tb) {
    const uint32_t c = min(c0 + uint32_t((wt * NBW + tb) * 32 + i), c1 - 1);
    asg[tb] = p.sorted ? p.sorted[c] : c;
  }
  if constexpr (SPL) {
    // the up wavefronts' sums to the gate wavefronts, through the LDS of
    // the token and weight buffers (no wavefront reads them after this
    // barrier)
    float* xch = reinterpret_cast<float*>(smem);  // [WR][NBW][16][64]
    __syncthreads();
    if (mw == 1) {
#pragma unroll
      for (int tb = 0; tb < NBW; ++tb)
#pragma unroll
        for (int v = 0; v < 16; ++v) xch[((wr * NBW + tb) * 16 + v) * 64 + lane] = acc0[tb][v];
    }
    __syncthreads();
    if (mw == 1) return;
#pragma unroll
    for (int tb = 0; tb < NBW; ++tb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc1[tb][v] = xch[((wr * NBW + tb) * 16 + v) * 64 + lane];
  }
  float wts[NBW];
#pragma unroll
  for (int tb = 0; tb < NBW; ++tb) wts[tb] = (NMAT == 2 && p.route_w) ? p.route_w[asg[tb]] : 1.0f;
#pragma unroll
  for (int tb = 0; tb < NBW; ++tb) {
    const uint32_t c = c0 + uint32_t((wt * NBW + tb) * 32 + i);
    if (c >= c1) continue;
    const uint32_t a = asg[tb];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int r0 = n0 + 32 * wr + 8 * g4 + 4 * kg;
      if constexpr (NMAT == 2) {
        const float wa = wts[tb];
        float h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          h[r] = silu(acc0[tb][4 * g4 + r]) * acc1[tb][4 * g4 + r] * wa;
        const half2v lo = {(_Float16)h[0], (_Float16)h[2]};
        const half2v hi = {(_Float16)h[1], (_Float16)h[3]};
        *reinterpret_cast<uint2*>(p.h_out + size_t(a) * p.N + r0) = make_uint2(as_u32(lo), as_u32(hi));
      } else {
        *reinterpret_cast<float4*>(p.y_out + size_t(a) * p.N + r0) =
            make_float4(acc0[tb][4 * g4], acc0[tb][4 * g4 + 1], acc0[tb][4 * g4 + 2],
                        acc0[tb][4 * g4 + 3]);
      }
    }
  }
}

// ------------------------------------------------------------- planning

// The tile lists themselves are written by the dispatch launch
// (dispatch_scan with a PlanOut, routing_dev.hpp).

// Upper bounds of the tile lists (grid heights): a 128-row tile covers at
// least 65 rows, the 64- and 32-row lists hold at most one tile per expert.
size_t bound128(size_t A, size_t E) { return A / 65 + 1; }
size_t bound_small(size_t A, size_t E) { return std::min(E, A) + 1; }

// ----------------------------------------------------------- conversions

// x -> f16 with the k order 0 2 1 3 4 6 5 7 inside every group of eight.
template <typename XT>
__global__ void __launch_bounds__(256)
    to_f16_kernel(const XT* __restrict__ x, size_t n8, uint4* __restrict__ out) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n8) return;
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = to_f32(x[8 * i + j]);
  const half2v a = {(_Float16)v[0], (_Float16)v[2]}, b = {(_Float16)v[1], (_Float16)v[3]};
  const half2v c = {(_Float16)v[4], (_Float16)v[6]}, d = {(_Float16)v[5], (_Float16)v[7]};
  out[i] = make_uint4(as_u32(a), as_u32(b), as_u32(c), as_u32(d));
}

// out = (residual + ys) + y ranks 0..k-1 of the token, in that order; one
// float4 per thread. The k rank rows are loaded at once (KMAX slots, the
// indices clamped to k - 1 and the extra slots not added), so a wavefront
// has all of its loads in flight instead of one rank at a time; they are
// read once, as nontemporal loads (c5: 216 -> 181 us for 905 MB).
typedef float fx4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load_nt(const float4* p) {
  const fx4 q = __builtin_nontemporal_load(reinterpret_cast<const fx4*>(p));
  return make_float4(q[0], q[1], q[2], q[3]);
}

template <int KMAX>
__global__ void __launch_bounds__(256)
    combine_kernel(const float* __restrict__ y, const float* __restrict__ ys,
                   const float* __restrict__ residual, int k, uint32_t H4, uint32_t n4,
                   float4* __restrict__ out) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= n4) return;
  const uint32_t t = i / H4, c4 = i - t * H4;
  const float4* y4 = reinterpret_cast<const float4*>(y);
  float4 u[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) u[r] = load_nt(y4 + (size_t(t) * k + min(r, k - 1)) * H4 + c4);
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (residual) v = reinterpret_cast<const float4*>(residual)[i];
  if (ys) {
    const float4 s = reinterpret_cast<const float4*>(ys)[i];
    v.x += s.x; v.y += s.y; v.z += s.z; v.w += s.w;
  }
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    if (r < k) {
      v.x += u[r].x; v.y += u[r].y; v.z += u[r].z; v.w += u[r].w;
    }
  }
  out[i] = v;
}

// ------------------------------------------------------------- launchers

// INFERNO_PREFILL_GEMM2=0 keeps the four-wavefront kernel for every format.
bool gemm2_enabled() {
  return !switch_off("INFERNO_PREFILL_GEMM2");
}

// Token tiles of whole K units in the 32-token staged GEMMs
// (INFERNO_PREFILL_XU=0: per 64-deep step).
bool unit_tokens() { return !switch_off("INFERNO_PREFILL_XU"); }

template <int Q, int NMAT, int TM>
int launch_gemm(hipStream_t s, const GemmArgs& a, unsigned grid_y) {
  if (grid_y == 0) return INFERNO_OK;
  // Q2_K (c5) on more, smaller workgroups with one LDS weight buffer, so
  // that three or four waves share each SIMD: the 128-token down on staged
  // weights (four wavefronts, 48 KB of LDS, three workgroups per CU; the
  // fragment-load kernel runs two waves per SIMD): 1125 -> 1066 us; the
  // 64-token gate/up as one matrix per wavefront on 64-row tiles (four
  // wavefronts, four workgroups per CU): 468 -> 438 us; c5 layer 5.28 ->
  // 5.22 ms (three A/B pairs); the 64-token down with one LDS weight buffer
  // at four waves per SIMD: 300 -> 221 us, layer 4.93 -> 4.84 ms.
  // INFERNO_PREFILL_Q2_SMALL_WG=0: the kernels below.
  if constexpr (Q == INFERNO_Q2_K && (TM == 128 || TM == 64) && (NMAT == 1 || TM == 64)) {
    if (a.N % 128 == 0 && gemm2_enabled() && !switch_off("INFERNO_PREFILL_Q2_SMALL_WG")) {
      if constexpr (NMAT == 1 && TM == 128) {
        const dim3 g2(unsigned(a.N / 128), grid_y);
        gemm2_kernel<Q, 1, TM, 1, 4, 1, 3, 1, 0><<<g2, 256, gemm2_lds_bytes<Q, 1, TM, 4, 1>(), s>>>(a);
      } else if constexpr (NMAT == 1) {
        const dim3 g2(unsigned(a.N / 128), grid_y);
        gemm2_kernel<Q, 1, TM, 1, 4, 1, 4, 1, 0><<<g2, 256, gemm2_lds_bytes<Q, 1, TM, 4, 1>(), s>>>(a);
      } else {
        const dim3 g2(unsigned(a.N / 64), grid_y);
        gemm2_kernel<Q, 2, TM, 1, 2, 1, 4, 1, 1><<<g2, 256, gemm2_lds_bytes<Q, 2, TM, 2, 1>(), s>>>(a);
      }
      INF_LAUNCHED();
      return INFERNO_OK;
    }
  }
  // staged weights where measured faster: 32- and 64-token tiles, the Q3_K
  // down, the Q2_K gate/up over 128 tokens and the Q8_0 shared expert (the
  // Q3_K 128-token gate/up and the Q2_K 128-token down stay on the fragment
  // loads). Q3_K prefetches two steps ahead.
  constexpr bool kStaged =
      ((Q == INFERNO_Q2_K || Q == INFERNO_Q3_K) &&
       (TM <= 64 || (NMAT == 1 && Q == INFERNO_Q3_K) || (NMAT == 2 && Q == INFERNO_Q2_K))) ||
      (Q == INFERNO_Q8_0 && (TM == 32 || TM == 128)) ||
      (Q == INFERNO_Q4_K && TM == 32) || (Q == INFERNO_Q6_K && NMAT == 1 && TM == 32);
  if constexpr (kStaged) {
    // INFERNO_PREFILL_Q4_STAGED=0: Q4_K and Q6_K on the fragment-load kernel
    if (a.N % 128 == 0 && gemm2_enabled() &&
        ((Q != INFERNO_Q4_K && Q != INFERNO_Q6_K) || !switch_off("INFERNO_PREFILL_Q4_STAGED"))) {
      const dim3 grid(unsigned(a.N / 128), grid_y);
      if constexpr (Q == INFERNO_Q8_0 && TM == 128) {
        // Q8_0 (272-byte K units): one weight buffer; gate/up with one
        // matrix per wavefront
        if constexpr (NMAT == 2)
          gemm2_kernel<Q, 2, TM, 1, 4, 1, 2, 1, 1>
              <<<grid, 512, gemm2_lds_bytes<Q, 2, TM, 4, 1>(), s>>>(a);
        else
          gemm2_kernel<Q, 1, TM, 1, 4, 1, 2, 1>
              <<<grid, 256, gemm2_lds_bytes<Q, 1, TM, 4, 1>(), s>>>(a);
      } else if constexpr (NMAT == 1 && TM == 32) {
        // down over few tokens: one weight buffer, four waves per SIMD (at
        // 64 tokens the 128-register budget spills)
        // (token tiles per K unit as in the gate/up below measured slower
        // here: c3 down 0.69 against 0.60 ms)
        gemm2_kernel<Q, 1, TM, 2, 4, 1, 4, 1>
            <<<grid, 256, gemm2_lds_bytes<Q, 1, TM, 4, 1>(), s>>>(a);
      } else if constexpr (NMAT == 2 && TM == 32) {
        // gate/up over few tokens: one matrix per wavefront (eight), one
        // weight buffer, four waves per SIMD; token tiles per K unit
        // (INFERNO_PREFILL_XU=0: per 64-deep step; Q8_0 keeps them per step,
        // its unit tiles would spill). Fewer than two workgroups per CU of
        // 128-row tiles (few experts, narrow I: c1, the XS layer): 64-row
        // tiles on four wavefronts, twice the workgroups, so that more of
        // the weights are in flight per CU
        // (not Q3_K: its 64-row instance spills 18 registers)
        if constexpr (Q == INFERNO_Q2_K || Q == INFERNO_Q4_K) {
          if (unit_tokens() && size_t(a.N / 128) * grid_y < 2 * kGemmCUs &&
              !switch_off("INFERNO_PREFILL_NARROW32")) {
            const dim3 g2(unsigned(a.N / 64), grid_y);
            gemm2_kernel<Q, 2, TM, 1, 2, 1, 4, 1, 1, 4>
                <<<g2, 256, gemm2_lds_bytes<Q, 2, TM, 2, 1, 4>(), s>>>(a);
            INF_LAUNCHED();
            return INFERNO_OK;
          }
        }
        if (Q != INFERNO_Q8_0 && unit_tokens())
          gemm2_kernel<Q, 2, TM, 1, 4, 1, 4, 1, 1, Q != INFERNO_Q8_0 ? 4 : 0>
              <<<grid, 512, gemm2_lds_bytes<Q, 2, TM, 4, 1, Q != INFERNO_Q8_0 ? 4 : 0>(), s>>>(a);
        else
          gemm2_kernel<Q, 2, TM, 1, 4, 1, 4, 1, 1>
              <<<grid, 512, gemm2_lds_bytes<Q, 2, TM, 4, 1>(), s>>>(a);
      } else if constexpr (NMAT == 2 && TM == 128) {
        // Q2_K gate/up over 128 tokens: one matrix per wavefront (64
        // accumulators each), compiled for three waves per SIMD (lab, dense
        // tiles: 1.81 vs 2.13 ms for the fragment-load kernel; c5 layer:
        // 5.21 vs 5.29 ms)
        // INFERNO_PREFILL_XU2=1: token tiles of two steps, one barrier per
        // two steps, compiled for two waves per SIMD (one 8-wave workgroup
        // per CU either way)
        // Default: 64 rows per matrix on four wavefronts (one matrix each) with
        // one LDS weight buffer, three workgroups per CU, so that three waves
        // share each SIMD (the 128-row eight-wavefront tile fits one
        // workgroup per CU: two waves per SIMD): c5 gate/up 1.98 -> 1.85 ms.
        // INFERNO_PREFILL_G128_WIDE=1: the 128-row tile.
        if (!switch_on("INFERNO_PREFILL_G128_WIDE") && !switch_on("INFERNO_PREFILL_XU2")) {
          const dim3 g2(unsigned(a.N / 64), grid_y);
          gemm2_kernel<Q, 2, TM, 1, 2, 1, 3, 1, 1>
              <<<g2, 256, gemm2_lds_bytes<Q, 2, TM, 2, 1>(), s>>>(a);
        } else if (switch_on("INFERNO_PREFILL_XU2"))
          gemm2_kernel<Q, 2, TM, 1, 4, 1, 2, 0, 1, 2>
              <<<grid, 512, gemm2_lds_bytes<Q, 2, TM, 4, 0, 2>(), s>>>(a);
        else
          gemm2_kernel<Q, 2, TM, 1, 4, 1, 3, 0, 1>
              <<<grid, 512, gemm2_lds_bytes<Q, 2, TM, 4, 0>(), s>>>(a);
      } else {
        constexpr int PF = Q == INFERNO_Q3_K ? 2 : 1;
        gemm2_kernel<Q, NMAT, TM, PF, 4, 1, 2><<<grid, 256, gemm2_lds_bytes<Q, NMAT, TM, 4>(), s>>>(a);
      }
      INF_LAUNCHED();
      return INFERNO_OK;
    }
  }
  const dim3 grid(unsigned(a.N / kTileN), grid_y);
  gemm_kernel<Q, NMAT, TM><<<grid, 256, gemm_lds_bytes<TM>(), s>>>(a);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int NMAT, int TM>
int launch_gemm_q(hipStream_t s, int quant, const GemmArgs& a, unsigned grid_y) {
  switch (quant) {
    case INFERNO_Q2_K: return launch_gemm<INFERNO_Q2_K, NMAT, TM>(s, a, grid_y);
    case INFERNO_Q3_K: return launch_gemm<INFERNO_Q3_K, NMAT, TM>(s, a, grid_y);
    case INFERNO_Q4_K: return launch_gemm<INFERNO_Q4_K, NMAT, TM>(s, a, grid_y);
    case INFERNO_Q8_0: return launch_gemm<INFERNO_Q8_0, NMAT, TM>(s, a, grid_y);
    case INFERNO_Q6_K:  // a down format only
      if constexpr (NMAT == 1) return launch_gemm<INFERNO_Q6_K, 1, TM>(s, a, grid_y);
      break;
  }
  set_error("quant kind has no MFMA prefill GEMM");
  return INFERNO_ERR_INVALID;
}

struct PlanView {
  uint4* l128;
  uint4* l64;
  uint4* l32;
  uint32_t* counts;
  size_t n128, n64, n32;
};

PlanView plan_view(uint32_t* plan, size_t A, size_t E) {
  PlanView v;
  v.n128 = bound128(A, E);
  v.n64 = bound_small(A, E);
  v.n32 = bound_small(A, E);
  v.l128 = reinterpret_cast<uint4*>(plan);
  v.l64 = v.l128 + v.n128;
  v.l32 = v.l64 + v.n64;
  v.counts = reinterpret_cast<uint32_t*>(v.l32 + v.n32);
  return v;
}

// The three tile-list launches of one GEMM.
// A list no expert can fill (max_rows rows at most: no 128-row tile below
// 65 rows, no 64-row tile below 33) is not launched; its grid of workgroups
// that find no tile would still take a few microseconds.
template <int NMAT>
int launch_tiled(hipStream_t s, int quant, GemmArgs a, const PlanView& v, size_t max_rows) {
  int st;
  a.tiles = v.l128;
  a.n_tiles = v.counts;
  if (max_rows > 64 && (st = launch_gemm_q<NMAT, 128>(s, quant, a, unsigned(v.n128)))) return st;
  a.tiles = v.l64;
  a.n_tiles = v.counts + 1;
  if (max_rows > 32 && (st = launch_gemm_q<NMAT, 64>(s, quant, a, unsigned(v.n64)))) return st;
  a.tiles = v.l32;
  a.n_tiles = v.counts + 2;
  return launch_gemm_q<NMAT, 32>(s, quant, a, unsigned(v.n32));
}

// Dense Q8_0 GEMM over a small batch with 32 weight rows per workgroup (one
// wavefront per matrix): the 128-row tiles of a 1536-row shared expert over
// 32 tokens make only 12 workgroups, and one CU takes in roughly 17 GB/s.
template <int NMAT>
int launch_dense_narrow(hipStream_t s, const GemmArgs& a, unsigned grid_y) {
  const dim3 grid(unsigned(a.N / 32), grid_y);
  if constexpr (NMAT == 2)
    gemm2_kernel<INFERNO_Q8_0, 2, 32, 1, 1, 1, 2, 1, 1>
        <<<grid, 128, gemm2_lds_bytes<INFERNO_Q8_0, 2, 32, 1, 1>(), s>>>(a);
  else
    gemm2_kernel<INFERNO_Q8_0, 1, 32, 2, 1, 1, 2, 1>
        <<<grid, 64, gemm2_lds_bytes<INFERNO_Q8_0, 1, 32, 1, 1>(), s>>>(a);
  INF_LAUNCHED();
  return INFERNO_OK;
}

// Dense GEMMs: tiles of TM rows over all T rows; TM from T so that small
// batches still spread over the chip (Q8_0 below 128 workgroups of 128-row
// tiles: 32-row tiles).
template <int NMAT>
int launch_dense(hipStream_t s, int quant, GemmArgs a, size_t T) {
  if (T >= 2048) return launch_gemm_q<NMAT, 128>(s, quant, a, unsigned((T + 127) / 128));
  const unsigned gy = unsigned((T + 31) / 32);
  if (quant == INFERNO_Q8_0 && a.N % 32 == 0 && size_t(a.N / 128) * gy < 128 && gemm2_enabled() &&
      !switch_off("INFERNO_PREFILL_NARROW"))
    return launch_dense_narrow<NMAT>(s, a, gy);
  return launch_gemm_q<NMAT, 32>(s, quant, a, gy);
}

}  // namespace

bool prefill_supported(int quant) {
  return quant == INFERNO_Q2_K || quant == INFERNO_Q3_K || quant == INFERNO_Q4_K ||
         quant == INFERNO_Q8_0;
}

bool prefill_routed_supported(int quant, int down_quant, size_t H, size_t I, size_t E) {
  auto routed = [](int q) {
    return q == INFERNO_Q2_K || q == INFERNO_Q3_K || q == INFERNO_Q4_K;
  };
  return routed(quant) && (routed(down_quant) || down_quant == INFERNO_Q6_K) &&
         H % kUnit == 0 && I % kUnit == 0 && E <= 256;
}

bool prefill_dense_supported(int quant, int down_quant, size_t H, size_t Is) {
  return prefill_supported(quant) && quant != INFERNO_Q6_K &&
         (prefill_supported(down_quant) || down_quant == INFERNO_Q6_K) && H % kUnit == 0 &&
         Is % kUnit == 0 && H % kTileN == 0 && Is % kTileN == 0;
}

PlanOut prefill_plan_out(uint32_t* plan, size_t A, size_t E) {
  const PlanView v = plan_view(plan, A, E);
  return PlanOut{v.l128, v.l64, v.l32, v.counts};
}

size_t prefill_plan_words(size_t A, size_t E) {
  return 4 * (bound128(A, E) + 2 * bound_small(A, E)) + 4;
}

int launch_to_f16(hipStream_t s, const void* x, int x_dtype, size_t rows, size_t K,
                  uint16_t* out) {
  const size_t n8 = rows * K / 8;
  if (n8 == 0) return INFERNO_OK;
  const unsigned grid = unsigned((n8 + 255) / 256);
  if (x_dtype == INFERNO_BF16)
    to_f16_kernel<uint16_t><<<grid, 256, 0, s>>>(static_cast<const uint16_t*>(x), n8,
                                                 reinterpret_cast<uint4*>(out));
  else
    to_f16_kernel<float><<<grid, 256, 0, s>>>(static_cast<const float*>(x), n8,
                                              reinterpret_cast<uint4*>(out));
  INF_LAUNCHED();
  return INFERNO_OK;
}

int launch_prefill_gate_up(hipStream_t s, const PrefillRouted& p) {
  const size_t A = p.T * p.k;
  if (A == 0) return INFERNO_OK;
  if (!prefill_routed_supported(p.quant, p.down_quant, p.H, p.I, p.E)) {
    set_error("MFMA prefill path does not cover this layer");
    return INFERNO_ERR_INVALID;
  }
  const PlanView v = plan_view(p.plan, A, p.E);
  GemmArgs g{};
  g.w0 = static_cast<const uint8_t*>(p.gate);
  g.w1 = static_cast<const uint8_t*>(p.up);
  g.stride = p.I * (p.H / kUnit) * size_t(block_bytes(p.quant));
  g.xin = p.x16;
  g.in_div = uint32_t(p.k);
  g.sorted = p.sorted;
  g.route_w = p.weights;
  g.N = int(p.I);
  g.K = int(p.H);
  g.h_out = p.h16;
  return launch_tiled<2>(s, p.quant, g, v, p.max_rows ? p.max_rows : A);
}

int launch_prefill_down(hipStream_t s, const PrefillRouted& p) {
  const size_t A = p.T * p.k;
  if (A == 0) return INFERNO_OK;
  const PlanView v = plan_view(p.plan, A, p.E);
  GemmArgs d{};
  d.w0 = static_cast<const uint8_t*>(p.down);
  d.stride = p.H * (p.I / kUnit) * size_t(block_bytes(p.down_quant));
  d.xin = p.h16;
  d.in_div = 1;
  d.sorted = p.sorted;
  d.N = int(p.H);
  d.K = int(p.I);
  d.y_out = p.y;
  return launch_tiled<1>(s, p.down_quant, d, v, p.max_rows ? p.max_rows : A);
}

int launch_prefill_dense(hipStream_t s, int quant, int down_quant, const void* gate,
                         const void* up, const void* down, const uint16_t* x16, size_t T,
                         size_t H, size_t Is, uint16_t* h16, float* ys, void* blas_ws,
                         void* lib_ws) {
  if (T == 0) return INFERNO_OK;
  if (H % kUnit || Is % kUnit) {
    set_error("MFMA prefill path needs 256-multiple dimensions");
    return INFERNO_ERR_INVALID;
  }
  if (blas_ws != nullptr && lib_ws != nullptr && dense_blas_takes(quant, down_quant, T, H, Is))
    return launch_dense_blas(s, gate, up, down, x16, T, H, Is, ys, blas_ws, lib_ws);
  GemmArgs g{};
  g.w0 = static_cast<const uint8_t*>(gate);
  g.w1 = static_cast<const uint8_t*>(up);
  g.xin = x16;
  g.in_div = 1;
  g.rows = uint32_t(T);
  g.N = int(Is);
  g.K = int(H);
  g.h_out = h16;
  int st;
  if ((st = launch_dense<2>(s, quant, g, T))) return st;
  GemmArgs d{};
  d.w0 = static_cast<const uint8_t*>(down);
  d.xin = h16;
  d.in_div = 1;
  d.rows = uint32_t(T);
  d.N = int(H);
  d.K = int(Is);
  d.y_out = ys;
  return launch_dense<1>(s, down_quant, d, T);
}

int launch_prefill_combine(hipStream_t s, const float* y, const float* ys, const float* residual,
                           size_t T, size_t k, size_t H, float* out) {
  const size_t n4 = T * H / 4;
  if (n4 == 0) return INFERNO_OK;
  if (H % 4 || n4 > 0xffffffffu || k == 0 || k > size_t(kMaxTopK)) {
    set_error("prefill combine: H must be a multiple of 4, T * H / 4 < 2^32, 1 <= k <= 16");
    return INFERNO_ERR_INVALID;
  }
  float4* o = reinterpret_cast<float4*>(out);
  const unsigned grid = unsigned((n4 + 255) / 256);
  const uint32_t H4 = uint32_t(H / 4), N4 = uint32_t(n4);
  if (k > 8)
    combine_kernel<16><<<grid, 256, 0, s>>>(y, ys, residual, int(k), H4, N4, o);
  else
    combine_kernel<8><<<grid, 256, 0, s>>>(y, ys, residual, int(k), H4, N4, o);
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace inferno
