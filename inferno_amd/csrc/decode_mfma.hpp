// Decode GEMVs of the routed Q2_K experts for one token on the matrix
// cores, with every 16-row tile read from HBM as one contiguous range and
// staged in LDS.
//
// gate/up (v_mfma_scale_f32_16x16x128_f8f6f4, fp8 x fp4): the dot product
// of a 16-row tile over one super-block column is one MFMA tile C[m][n] =
// sum_k A[m][k] B[k][n] in two K halves (the bit planes 0, 2 and 1, 3):
//   B (weights): lane (row n, lane group kq) holds the 16 qs bytes
//     qs[16 kq .. 16 kq + 15] of its row's block. A 2-bit field in the low
//     two bits of a nibble is the fp4 (e2m1) value q / 2, so one v_and_b32
//     with 0x33333333 yields eight operand values (planes 0 and 2; after a
//     shift by 2, planes 1 and 3).
//   A (activations): x is two e4m3 terms (E8M0 scales 2^e1 and 2^(e1 - 4)).
//     In the MFMA of planes u, u + 2, row r of A is term r >> 3 of one of
//     the 8 groups (scale bytes m = 8h + 2p + s) whose fields those planes
//     hold, x only in the K positions of that group, so each (group, term)
//     16-value dot product lands in its own row of C; the row's scale
//     operand (one per lane, lane l for row l % 16, measured) is its term's.
//   Operand K layout (gfx950, measured): A lane group qa holds k = 16 qa + t
//     in bytes t < 16 and k = 64 + 16 qa + t in bytes 16 + t; B lane group q
//     holds k = 32 q + nibble.
//   C: lane (kq, n) holds term kq >> 1 of four groups of row n, all among
//     groups 8 (kq & 1) .. + 7 (scale dwords 2 (kq & 1), + 1); the offset
//     terms (minimum) enter once, on the term-0 lanes. The group scale and minimum
//     enter with v_fma_mix: the 4-bit scale and min nibbles masked in place
//     are f16 subnormals, so no byte-to-float conversion is needed.
//
// down (v_mfma_f32_16x16x32_f16): the same block-diagonal A with f16 h (a
// masked 2-bit field at bits 2p and 16 + 2p is a pair of exact f16
// subnormals q 2^(2p - 24)), per-run scales of h.
//
// Reference semantics: dequantize_q2_k_block (crates/gguf/src/lib.rs:
// 1226-1293): value = (d * (sc & 15)) * q - dmin * (sc >> 4); gate/up with
// SwiGLU and the routing weight folded into h (gguf_moe_kernels.metal:
// 340-455). Accumulation is fp32; the sum order differs from the reference's
// (the parity bound is the layer tolerance, rel-L2 2e-3).
//
// A workgroup (16 wavefronts) is persistent over tiles t = blockIdx.x + j *
// gridDim.x: it writes tile t (held in registers) to LDS, issues the loads of
// tile t + gridDim.x into the same registers, and computes tile t from LDS.
// No workgroup waits on another.
#pragma once
#include "decode.hpp"
#include "decode_select.hpp"
#include "dot2_formats.hpp"

namespace inferno {
namespace mfma_decode {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));

// A 16-byte chunk of a routed weight tile, which a decode launch reads once
// per call: a nontemporal load (c2 -0.5, c4 -1, c1 -0.7 us per step; the
// same hint on the packed-f16 GEMV loads, whose 16-byte reads straddle
// blocks and lines, cost c2 +4 and c4 +11 us)
__device__ __forceinline__ u32x4 ld_tile(const u32x4* p) { return __builtin_nontemporal_load(p); }

// Global -> LDS copy of n 16-byte words by NT threads in two steps, so that
// a kernel can issue other loads between them: load() puts every word of
// this thread (at most MAXIT) in flight at once (a load-store loop waits for
// each load in turn), store() writes them; words past MAXIT * NT are copied
// by a plain loop in store().
template <int NT, int MAXIT>
struct LdsCopy {
  uint4 t[MAXIT];
  __device__ __forceinline__ void load(const uint4* src, int n) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < MAXIT; ++i) t[i] = src[min(i * NT + tid, n - 1)];
  }
  __device__ __forceinline__ void store(uint4* dst, const uint4* src, int n) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < MAXIT; ++i)
      if (i * NT + tid < n) dst[i * NT + tid] = t[i];
    for (int j = MAXIT * NT + tid; j < n; j += NT) dst[j] = src[j];
  }
};
typedef uint32_t u32_a2 __attribute__((aligned(2)));
typedef int v8i __attribute__((ext_vector_type(8)));

// N words at an LDS address that is only 2-byte aligned (Q3_K and Q6_K
// blocks, 110 and 210 bytes, start at 2 mod 4 every other block): N + 1
// aligned word reads and N byte-aligns. The word at p - (p & 3) + 4 N may lie
// past the block (never past the LDS allocation: a later block, row or
// region follows); its bytes are shifted out.
template <int N>
__device__ __forceinline__ void lds_words_a2(const uint8_t* p, uint32_t (&out)[N]) {
  const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(p)) & 3u;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(p - sh);
  uint32_t d[N + 1];
#pragma unroll
  for (int i = 0; i <= N; ++i) d[i] = w[i];
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
}


constexpr int kWaves = 16;
constexpr int kThreads = 64 * kWaves;
constexpr int kQ2Bytes = 84;
constexpr int kRowPad = 16;    // LDS row padding (bytes): rows start on distinct banks

// ---------------------------------------------------------- x staging
//
// The gate/up kernel multiplies fp4 weights (below) by fp8 activations:
// x = 2^e1 * (t1 + t2 / 16), t1 = e4m3(x 2^-e1), t2 = e4m3(16 (x 2^-e1 - t1)),
// with one e1 per 256-value column putting its max|x| in [128, 256). Two
// e4m3 terms carry a bf16 value exactly (8 significant bits) unless it lies
// below ~max|x| 2^-17 of its column. Staged row (words), per token:
//   [column images K/256 x 256][run sums K/16][column exponents K/256], padded to 4.
// A column image is [term 2][group m 16][half 2] x 16 bytes laid out for the
// A operand of v_mfma_scale_f32_16x16x128_f8f6f4 (see gate_up_fp4_kernel):
// byte t of (m, half) holds value i = 4 j + b of group m, j = 2 half + t / 8,
// b = (t % 8) / 2, when t % 2 == p(m) >> 1, and 0 otherwise.

__host__ __device__ constexpr int stage_words(int K) { return (K + K / 16 + K / 256 + 3) & ~3; }

// e4m3 (OCP, bias 7, max 448) of a float, round to nearest even; |f| here
// stays below 256, so no saturation case arises.
__device__ __forceinline__ uint32_t to_e4m3(float f) {
  const uint32_t sign = f < 0.f ? 0x80u : 0u;
  const float a = fabsf(f);
  if (!(a >= 0.0009765625f)) return sign;  // below half the smallest subnormal (2^-9); NaN -> 0
  int e;
  frexpf(a, &e);  // a = f 2^e, f in [0.5, 1): a = 1.m 2^(e-1)
  int E = e - 1;
  if (E < -6) return sign | uint32_t(rintf(a * 512.f));  // subnormal: units of 2^-9 (8 = 0x08)
  float mant = rintf(ldexpf(a, 3 - E));  // in [8, 16]
  if (mant >= 16.f) {
    mant = 8.f;
    E += 1;
  }
  if (E > 8) return sign | 0x7eu;
  return sign | (uint32_t(E + 7) << 3) | (uint32_t(mant) - 8u);
}
__device__ __forceinline__ float from_e4m3(uint32_t b) {
  const float s = (b & 0x80u) ? -1.f : 1.f;
  const uint32_t E = (b >> 3) & 15u, M = b & 7u;
  if (E == 0) return s * float(M) * (1.f / 512.f);
  return s * ldexpf(1.f + float(M) * 0.125f, int(E) - 7);
}

// Stages super-block column `col` of one bf16 row into `row` (the layout
// above); one full wavefront, lane l holding values 4l .. 4l + 3 (group
// m = l / 4, quarter u = l % 4 of it).
__device__ __forceinline__ void stage_column(const uint16_t* x, uint32_t* row, int K, int col) {
  const int lane = threadIdx.x & 63;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = bf16_bits_to_f32(x[col * kKBlock + 4 * lane + i]);
  float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  int e1 = 0;  // zero or non-finite columns keep exponent 0
  if (mx > 0.f && mx < 3.0e38f) {
    int e;
    frexpf(mx, &e);
    e1 = e - 8;
  }
  const int m = lane >> 2, u = lane & 3, e = (m >> 2) & 1;
  uint32_t w[2][2] = {{0u, 0u}, {0u, 0u}};  // [term][word]: bytes 2b + e of this quarter
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float a = ldexpf(v[b], -e1);
    const uint32_t b1 = to_e4m3(a);
    const uint32_t b2 = to_e4m3((a - from_e4m3(b1)) * 16.f);
    const int sh = 16 * (b & 1) + 8 * e;
    w[0][b >> 1] |= b1 << sh;
    w[1][b >> 1] |= b2 << sh;
  }
  uint32_t* img = row + col * 256 + m * 8 + (u >> 1) * 4 + (u & 1) * 2;
#pragma unroll
  for (int tm = 0; tm < 2; ++tm) {
    img[tm * 128] = w[tm][0];
    img[tm * 128 + 1] = w[tm][1];
  }
  float sum = (v[0] + v[1]) + (v[2] + v[3]);
  sum += __shfl_xor(sum, 1, kWave);
  sum += __shfl_xor(sum, 2, kWave);
  float* sums = reinterpret_cast<float*>(row + K);
  if (u == 0) sums[col * 16 + m] = sum;
  if (lane == 0) reinterpret_cast<int*>(row + K + K / 16)[col] = e1;
}

// Stages one 16-value run held one value per lane by lanes 0..15 (lane i
// holds value i; only those lanes call it) into a K-wide row of the MFMA
// layout with a per-run scale: [pairs K/2][run sums K/16][run factors
// K/16], factor = 2^48 / s_run. The gate/up kernel writes h this way (one
// 16-row tile is one run of h); the down kernel reads it.
__device__ __forceinline__ void stage_run_lanes_mfma(float v, uint32_t* row, int K, int run) {
  const int lane = threadIdx.x & 63;
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
  const int p = ((run & 15) >> 1) & 3;  // bit plane of this run's group
  const _Float16 hv = (_Float16)(v * (s * ldexpf(1.0f, -2 * p)));
  const uint32_t hb = __builtin_bit_cast(uint16_t, hv);
  // pair word j holds values (base, base + 2), base = 4 (j >> 1) + (j & 1)
  const int j = lane & 7;
  const int base = 4 * (j >> 1) + (j & 1);
  const uint32_t h0 = __shfl(hb, base, 16), h1 = __shfl(hb, base + 2, 16);
  if (lane < 8) row[run * 8 + j] = h0 | (h1 << 16);
  if (lane == 0) {
    float* sums = reinterpret_cast<float*>(row + K / 2);
    sums[run] = sum;
    sums[K / 16 + run] = 16777216.0f * 16777216.0f / s;
  }
}

// Words per row of that layout.
__host__ __device__ constexpr int run_stage_words(int K) { return K / 2 + K / 8; }

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

// Loads tile t's gate and up rows (16 contiguous rows each) into registers,
// one 16-byte chunk per thread and step.
template <int PER>
__device__ __forceinline__ void fetch_tile(u32x4 (&v)[PER], const DecodeArgs& p, int tiles_i,
                                           int rb, int t, uint32_t expert) {
  const int nv = rb;  // 16-byte chunks per matrix (16 rows of rb bytes)
  const size_t off = size_t(expert) * p.gate_stride + size_t(t % tiles_i) * 16 * size_t(rb);
  const u32x4* g4 = reinterpret_cast<const u32x4*>(p.gate + off);
  const u32x4* u4 = reinterpret_cast<const u32x4*>(p.up + off);
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    int i = j * kThreads + tid;
    i = i < 2 * nv ? i : 2 * nv - 1;  // clamped; the extra chunks are not stored
    v[j] = ld_tile(i < nv ? g4 + i : u4 + (i - nv));
  }
}

// Block bytes of the formats the fp8 x fp4 gate/up takes.
__host__ __device__ constexpr int fp4_block_bytes(int Q) { return Q == INFERNO_Q3_K ? 110 : kQ2Bytes; }

// Chunks per thread of a layer with NB super-block columns.
__host__ __device__ constexpr int chunks_per_thread(int NB, int bytes = kQ2Bytes) {
  return (2 * NB * bytes + kThreads - 1) / kThreads;
}

// LDS layout of gate_up_fp4_kernel, in bytes from the start of its dynamic
// LDS; the kernel takes its region pointers from here and the launcher its
// allocation (end), so a host-side check of this function is a check of the
// kernel's layout. Regions, and when they are live:
//   xs      staged x (stage_words(H) words): prologue copy .. last tile;
//   zero    16 zero bytes (A operand of inactive lanes): whole kernel;
//   tl      the routed tile, gate and up, 32 rows of rb + kRowPad bytes: loop;
//   part    per-wavefront row sums [wave][matrix][16] floats: loop;
//   slot_e/slot_a/slot_w  per-slot expert, assignment, weight: whole kernel;
//   tk      Top1Lds of the selection (SEL): prologue;
//   sdpart  shared-down parts [wave][8] floats (SEL): prologue .. first tile;
//   hsd     the shared expert's staged h, staged_stride(Is, false) words
//           (SEL with the shared down): prologue;
//   sdl     per-wavefront shared-down rows, kSdMaxOctets * kSdWpo areas of
//           SharedDownSlice::kWaveLds bytes, written by the LDS DMA of their
//           own wavefront (SEL with the shared down): prologue.
struct Fp4Lds {
  int xs, zero, tl, part, slot_e, slot_a, slot_w, tk, sdpart, hsd, sdl, sdl_bytes, end;
};
__host__ __device__ constexpr int align_up(int v, int a) { return (v + a - 1) / a * a; }
__host__ __device__ constexpr Fp4Lds fp4_lds_layout(int H, int quant, bool sel, int Is_sd) {
  Fp4Lds L{};
  const int rb = H / kKBlock * fp4_block_bytes(quant);
  L.xs = 0;
  L.zero = L.xs + stage_words(H) * 4;
  L.tl = L.zero + 16;
  L.part = L.tl + 2 * 16 * (rb + kRowPad);
  L.slot_e = L.part + kWaves * 2 * 16 * 4;
  L.slot_a = L.slot_e + kMaxExperts * 4;
  L.slot_w = L.slot_a + kMaxExperts * 4;
  L.tk = align_up(L.slot_w + kMaxExperts * 4, 8);  // Top1Lds holds 64-bit keys
  L.sdpart = L.tk + (sel ? int(sizeof(Top1Lds)) : 0);
  L.hsd = L.sdpart + (sel ? kWaves * 8 * 4 : 0);
  L.sdl = align_up(L.hsd + (sel ? staged_stride(Is_sd, false) * 4 : 0), 16);
  L.sdl_bytes = (sel && Is_sd) ? kSdMaxOctets * kSdWpo * SharedDownSlice::kWaveLds : 0;
  L.end = L.sdl + L.sdl_bytes;
  return L;
}

// NB = H / 256 super-block columns (rows must be whole 16-byte chunks: NB a
// multiple of 4 for Q2_K, of 8 for Q3_K); compile-time so that the chunk ->
// (matrix, row, column) split and the LDS addressing use constant divisors
// and strides.
//
// Q3_K [hmask 32 | qs 64 | scales 12 | d] has Q2_K's low two bits in qs at
// byte 32 and the high bit of value i of group g = 8 h + 2 p + s in hmask
// byte 16 s + i, bit 4 h + p: lane group q = 2 h + s moves bit 4 h + p of
// hmask byte i into the low bit of the nibble that holds plane p of qs byte
// i, a second fp4 B (value hbit / 2) whose MFMAs take the A scale + 2 (x 4),
// so C = sum x (low + 4 hbit) / 2 = sum x q3 / 2; value = gs (q3 - 4).
//
// SEL (one token): the launch also does the select launch's work, so the
// layer takes three launches. Every workgroup selects the token's experts
// itself (wavefront 15: the route launch's logit partials, topk1_wave) into
// its slot table, and workgroup 0 writes the ids, weights and dispatch for
// the down launch; meanwhile the other wavefronts form the shared expert's
// h from the route launch's partials and load the shared down rows of this
// workgroup's 8-row octets (octet o = blockIdx.x + w gridDim.x for wavefront
// w), whose dot products run while the first routed tile's loads are in
// flight. The selection is the select launch's (same function), so the
// result does not depend on which launch ran it.
// SP: the selection's router slots per lane (SEL; 4 covers 256 experts, 2
// covers 128 with half the ballots per search step).
template <int Q, int NB, bool SEL, int SP = 4>
__global__ void __launch_bounds__(kThreads) gate_up_fp4_kernel(DecodeArgs p, int ntiles) {
  extern __shared__ uint32_t smem[];
  constexpr int kB = fp4_block_bytes(Q);
  constexpr int H = NB * kKBlock, PER = chunks_per_thread(NB, kB);
  constexpr int rb = NB * kB, RS = rb + kRowPad, nv = rb;
  static_assert(rb % 16 == 0, "rows must be whole 16-byte chunks");
  constexpr int Sm = stage_words(H);
  const int I = p.I;
  // shared down in this launch (SEL with a shared expert and its ys rows)
  const int is_sd = (SEL && p.Is && p.ys) ? p.Is : 0;
  constexpr Fp4Lds L = fp4_lds_layout(H, Q, SEL, 0);  // sdl: the only offset is_sd moves
  uint8_t* lds = reinterpret_cast<uint8_t*>(smem);
  uint32_t* xs = reinterpret_cast<uint32_t*>(lds + L.xs);
  uint32_t* zero = reinterpret_cast<uint32_t*>(lds + L.zero);
  uint8_t* tl = lds + L.tl;
  float* part = reinterpret_cast<float*>(lds + L.part);  // [wave][matrix][16]
  uint32_t* slot_e = reinterpret_cast<uint32_t*>(lds + L.slot_e);  // [max_slots]
  uint32_t* slot_a = reinterpret_cast<uint32_t*>(lds + L.slot_a);
  float* slot_w = reinterpret_cast<float*>(lds + L.slot_w);
  Top1Lds* tk = reinterpret_cast<Top1Lds*>(lds + L.tk);
  float* sdpart = reinterpret_cast<float*>(lds + L.sdpart);  // [wave][8] shared down parts (SEL)
  uint32_t* hsd = reinterpret_cast<uint32_t*>(lds + L.hsd);  // shared h (SEL)
  // shared down rows (SEL)
  uint32_t* sdl = reinterpret_cast<uint32_t*>(lds + fp4_lds_layout(H, Q, SEL, is_sd).sdl);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, q = lane >> 4;
  const int tiles_i = I / kRows;
  u32x4 v[PER];
  int t = blockIdx.x;
  // SEL: this workgroup's shared down rows [sd_row0, sd_row0 + sd_rows)
  int sd_rows = 0, sd_row0 = 0;
  if constexpr (SEL) {
    constexpr int kSelWave = kWaves - 1;
    const bool sdown = p.Is && p.ys;  // else the shared down runs in the down launch
    if (sdown) {
      const int G = int(gridDim.x), rw = 8 * ((p.H / 8 + G - 1) / G);
      sd_row0 = int(blockIdx.x) * rw;
      sd_rows = max(0, min(rw, p.H - sd_row0));
    }
    if (wave == kSelWave) {
      // the selection: the longest chain of the prologue, so nothing else,
      // and first in issue on its SIMD
      __builtin_amdgcn_s_setprio(3);
      float lg[4], bs[4];
      load_logits1(p, lg, bs);
      topk1_wave_p<SP>(lg, bs, p.E, p.k, p.score_fn, p.norm, p.scale, tk);
      if (lane < p.k) {  // slot j = j-th smallest id, assignment = its rank
        const uint32_t rank = tk->rank[lane];
        slot_e[lane] = tk->id[lane];
        slot_a[lane] = rank;
        slot_w[lane] = tk->w[rank];
      }
      __builtin_amdgcn_s_setprio(0);
      if (blockIdx.x == 0) select1_write(p, tk);
    } else {
      constexpr int kT = kSelWave * kWave;  // threads of the other wavefronts
      if (sd_rows) form_shared_h<kT>(p, hsd, tid);
      for (int i = tid; i < Sm / 4; i += kT)
        reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(p.stage_xm)[i];
      if (tid < 4) zero[tid] = 0;
      // the shared down rows this wavefront dots, copied to LDS while the
      // selection runs (HBM is idle until the first routed tile is known)
      if (wave < (sd_rows / 8) * kSdWpo)
        SharedDownSlice::fetch_lds(p, sdl + wave * (SharedDownSlice::kWaveLds / 4), wave, sd_row0);
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wavefront's copies are in LDS
    }
    __syncthreads();
    if (t < ntiles) fetch_tile<PER>(v, p, tiles_i, rb, t, slot_e[t / tiles_i]);
    // the shared down, while the first routed tile's loads are in flight;
    // its parts are summed into ys after the next barrier
    if (wave < (sd_rows / 8) * kSdWpo)
      SharedDownSlice::dot_lds(p, sdl + wave * (SharedDownSlice::kWaveLds / 4), hsd, wave, sdpart);
  } else {
    if (t < ntiles) fetch_tile<PER>(v, p, tiles_i, rb, t, p.slots[t / tiles_i].x);
    for (int i = tid; i < Sm / 4; i += kThreads)
      reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(p.stage_xm)[i];
    if (tid < 4) zero[tid] = 0;
    // per-slot expert, assignment and routing weight, read once
    for (int j = tid; j < p.max_slots; j += kThreads) {
      const uint4 sl = p.slots[j];
      slot_e[j] = sl.x;
      slot_a[j] = sl.w;
      slot_w[j] = p.weights[sl.w];
    }
  }
  // the shared expert's gate/up partial sums (split over K in the route
  // launch) -> SwiGLU -> staged h rows for down8_kernel, one 16-row tile per
  // workgroup (with the MFMA down the select launch forms them itself)
  if (p.Is && !p.h_mfma && tid < 16) {
    for (int st = blockIdx.x; st < p.Is / kRows; st += gridDim.x) {
      float g = 0.f, u = 0.f;
      for (int k = 0; k < p.shared_parts; ++k) {
        g += p.shared_gu[(size_t(k) * 2) * p.Is + st * kRows + tid];
        u += p.shared_gu[(size_t(k) * 2 + 1) * p.Is + st * kRows + tid];
      }
      stage_run_lanes(silu(g) * u, p.stage_hs, p.Is, st);
    }
  }
  // A operand (fp8 x) of MFMA u (planes u, u + 2): row r holds term r >> 3
  // of group g(j, u), j = r & 7 (g = 8 (j >> 2) + 4 ((j >> 1) & 1) + 2 u +
  // (j & 1)), in the two lanes whose K range covers B's lane group
  // 2 (g >> 3) + (g & 1): kq >> 1 == j & 1, in operand bytes 16..31 for
  // g >= 8; every other lane reads zeros. The row's E8M0 scale (one per
  // lane, for row n) is that of its term, so both terms of a group land in
  // C already scaled and the final sum over lane groups adds them.
  const bool act = (q >> 1) == (n & 1);
  const int hi16 = (n >> 2) & 1, tmA = n >> 3;
  const int gA = 8 * ((n >> 2) & 1) + 4 * ((n >> 1) & 1) + (n & 1);  // g(j, 0); + 2 u
  // C: lane (kq, n) holds rows 4 kq + i of weight row n: term kq >> 1 of
  // groups 8 (kq & 1) + 4 (i >> 1) + 2 u + (i & 1); the offset terms (min,
  // Q3_K's -4) enter once, on the term-0 lanes
  const int hq = q & 1;
  const bool term0 = q < 2;
  const float* sums = reinterpret_cast<const float*>(xs + H);
  const int* e1s = reinterpret_cast<const int*>(xs + H + H / 16);
  // SEL: the down launch's workgroup of this index (on the same XCD) starts
  // with its tile blockIdx.x. When this workgroup has no next routed tile to
  // fetch, its tile registers v (free from then on) load the k selected
  // experts' rows of that down tile, as far as kWarmPer chunks per thread reach;
  // the data is not used, the loads leave the rows in this XCD's L2. They
  // are ordinary loads the compiler counts: nothing waits for them until
  // the sink after the loop (no LDS is written).
  // 64 KB per workgroup at most; none for the widest Q3_K rows, whose
  // registers are all taken by the tile loop (the sink would spill)
  constexpr int kWarmPer = (Q == INFERNO_Q3_K && NB > 16) ? 0 : PER < 4 ? PER : 4;
  bool warmed = false;
  auto warm_down = [&]() {
    warmed = true;
    if (!p.dpf_rows || int(blockIdx.x) >= p.H / p.dpf_rows) return;  // uniform
    const size_t rbd = size_t(p.dpf_row_bytes);
    const int cr = int(size_t(p.dpf_rows) * rbd / 16), nc = p.k * cr;
#pragma unroll
    for (int j = 0; j < kWarmPer; ++j) {
      const int i = min(j * kThreads + tid, nc - 1), r = i / cr, w = i - r * cr;
      v[j] = reinterpret_cast<const u32x4*>(p.down + size_t(slot_e[r]) * p.down_stride +
                                            size_t(blockIdx.x) * p.dpf_rows * rbd)[w];
    }
  };
  for (; t < ntiles; t += gridDim.x) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = j * kThreads + tid;
      if (i < 2 * nv) {
        const int mat = i >= nv, rem = i - mat * nv, row = rem / (rb / 16), c16 = rem - row * (rb / 16);
        *reinterpret_cast<u32x4*>(tl + (mat * 16 + row) * RS + c16 * 16) = v[j];
      }
    }
    __syncthreads();
    if (t + int(gridDim.x) < ntiles)
      fetch_tile<PER>(v, p, tiles_i, rb, t + gridDim.x, slot_e[(t + gridDim.x) / tiles_i]);
    if constexpr (SEL) {  // once: the shared down parts (written before this barrier)
      if (sd_rows && tid < sd_rows) SharedDownSlice::store(p, sdpart, tid, sd_row0);
      sd_rows = 0;
      if (kWarmPer && t + int(gridDim.x) >= ntiles) warm_down();
    }
    const int slot = t / tiles_i, tile = t - slot * tiles_i;
    float acc[2] = {0.f, 0.f};
    for (int c = wave; c < NB; c += kWaves) {
      v8i A[2];  // [u]
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t* img = xs + c * 256 + (gA + 2 * u) * 8 + (q & 1) * 4 + tmA * 128;
        const uint32_t* lo = (act && !hi16) ? img : zero;
        const uint32_t* hi = (act && hi16) ? img : zero;
        const uint4 a0 = *reinterpret_cast<const uint4*>(lo);
        const uint4 a1 = *reinterpret_cast<const uint4*>(hi);
        A[u] = v8i{int(a0.x), int(a0.y), int(a0.z), int(a0.w),
                   int(a1.x), int(a1.y), int(a1.z), int(a1.w)};
      }
      // x sums of this lane's groups 8 hq + 0..7
      const float4 xa = *reinterpret_cast<const float4*>(sums + c * 16 + 8 * hq);
      const float4 xb = *reinterpret_cast<const float4*>(sums + c * 16 + 8 * hq + 4);
      const int sa = 127 + e1s[c] - 4 * tmA;  // E8M0 scale of this lane's A row's term
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const uint8_t* blk = tl + (m * 16 + n) * RS + c * kB;
        // B (fp4 weights): a 2-bit field in the low bits of a nibble is the
        // e2m1 value q / 2; planes 0 (low nibble) and 2 (high nibble) in
        // MFMA 0, planes 1 and 3 in MFMA 1
        const uint32_t F = 0x33333333u;
        floatx4 C0 = {0.f, 0.f, 0.f, 0.f}, C1 = C0;
        if constexpr (Q == INFERNO_Q3_K) {
          uint32_t qw[4], hw[4];
          lds_words_a2(blk + 32 + 16 * q, qw);
          lds_words_a2(blk + 16 * (q & 1), hw);
          const u32x4 qs = {qw[0], qw[1], qw[2], qw[3]}, hm = {hw[0], hw[1], hw[2], hw[3]};
          const v8i B0 = v8i{int(qs.x & F), int(qs.y & F), int(qs.z & F), int(qs.w & F), 0, 0, 0, 0};
          const v8i B1 = v8i{int((qs.x >> 2) & F), int((qs.y >> 2) & F), int((qs.z >> 2) & F),
                             int((qs.w >> 2) & F), 0, 0, 0, 0};
          // high bits: bit 4 h + p of each hmask byte to bit 0 of the nibble
          // holding plane p (p = 0, 2 for MFMA 0; 1, 3 for MFMA 1)
          const int hsh = 4 * (q >> 1);
          const uint32_t x0 = hm.x >> hsh, x1 = hm.y >> hsh, x2 = hm.z >> hsh, x3 = hm.w >> hsh;
          const uint32_t L = 0x01010101u, U = 0x10101010u;
          const v8i H0 = v8i{int((x0 & L) | ((x0 << 2) & U)), int((x1 & L) | ((x1 << 2) & U)),
                             int((x2 & L) | ((x2 << 2) & U)), int((x3 & L) | ((x3 << 2) & U)),
                             0, 0, 0, 0};
          const v8i H1 = v8i{int(((x0 >> 1) & L) | ((x0 << 1) & U)),
                             int(((x1 >> 1) & L) | ((x1 << 1) & U)),
                             int(((x2 >> 1) & L) | ((x2 << 1) & U)),
                             int(((x3 >> 1) & L) | ((x3 << 1) & U)), 0, 0, 0, 0};
          C0 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[0], B0, C0, 0, 4, 0, sa, 0, 127);
          C1 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[1], B1, C1, 0, 4, 0, sa, 0, 127);
          C0 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[0], H0, C0, 0, 4, 0, sa + 2, 0, 127);
          C1 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[1], H1, C1, 0, 4, 0, sa + 2, 0, 127);
          // group 8 hq + k: 6-bit scale = nibble hq of scales[k] | bits
          // 2 (2 hq + k / 4) .. + 1 of scales[8 + k % 4] at bit 4
          uint32_t sc[3];
          lds_words_a2(blk + 96, sc);
          const uint32_t l0 = sc[0], l1 = sc[1], hb = sc[2];
          const uint32_t s6a = ((l0 >> (4 * hq)) & 0x0f0f0f0fu) | (((hb >> (4 * hq)) & 0x03030303u) << 4);
          const uint32_t s6b = ((l1 >> (4 * hq)) & 0x0f0f0f0fu) | (((hb >> (4 * hq + 2)) & 0x03030303u) << 4);
          const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk + 108));
          // C_u[i] is group k = 4 (i >> 1) + 2 u + (i & 1): bytes 2 u + (i & 1)
          // of s6a (i < 2) or s6b
          const float xsv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
          const float off = term0 ? -4.0f : 0.f;
          float tt = 0.f;
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int k = 4 * (i >> 1) + 2 * u + (i & 1);
              const uint32_t sw = (i < 2) ? s6a : s6b;
              const float gs = float(int((sw >> (8 * (2 * u + (i & 1)))) & 0xffu) - 32);
              const float cv = u ? C1[i] : C0[i];
              tt = fmaf(gs, fmaf(2.0f, cv, off * xsv[k]), tt);
            }
          acc[m] = fmaf(d, tt, acc[m]);
          continue;
        }
        const u32x4_a4 qs = *reinterpret_cast<const u32x4_a4*>(blk + 16 + 16 * q);
        const uint32_t sw0 = *reinterpret_cast<const uint32_t*>(blk + 8 * hq);
        const uint32_t sw1 = *reinterpret_cast<const uint32_t*>(blk + 8 * hq + 4);
        const uint32_t dmw = *reinterpret_cast<const uint32_t*>(blk + 80);
        const v8i B0 = v8i{int(qs.x & F), int(qs.y & F), int(qs.z & F), int(qs.w & F), 0, 0, 0, 0};
        const v8i B1 = v8i{int((qs.x >> 2) & F), int((qs.y >> 2) & F), int((qs.z >> 2) & F),
                           int((qs.w >> 2) & F), 0, 0, 0, 0};
        C0 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[0], B0, C0, 0, 4, 0, sa, 0, 127);
        C1 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[1], B1, C1, 0, 4, 0, sa, 0, 127);
        // scale nibbles and min nibbles of groups 8 hq + k as f16 subnormal
        // pairs: bytes (0, 2) and (1, 3) of scale dwords 2 hq (k < 4) and
        // 2 hq + 1; C_u[i] is group k = 4 (i >> 1) + 2 u + (i & 1)
        const uint32_t sh0 = sw0 >> 8, sh1 = sw1 >> 8;
        const half2v a02 = as_h2(sw0 & 0x000f000fu), a13 = as_h2(sh0 & 0x000f000fu);
        const half2v b02 = as_h2(sw1 & 0x000f000fu), b13 = as_h2(sh1 & 0x000f000fu);
        const half2v ma02 = as_h2(sw0 & 0x00f000f0u), ma13 = as_h2(sh0 & 0x00f000f0u);
        const half2v mb02 = as_h2(sw1 & 0x00f000f0u), mb13 = as_h2(sh1 & 0x00f000f0u);
        const half2v dm = as_h2(dmw);
        float S = fmaf((float)a02.x, C0[0], 0.f);
        S = fmaf((float)a13.x, C0[1], S);
        S = fmaf((float)b02.x, C0[2], S);
        S = fmaf((float)b13.x, C0[3], S);
        S = fmaf((float)a02.y, C1[0], S);
        S = fmaf((float)a13.y, C1[1], S);
        S = fmaf((float)b02.y, C1[2], S);
        S = fmaf((float)b13.y, C1[3], S);
        float Mn = fmaf((float)ma02.x, xa.x, 0.f);
        Mn = fmaf((float)ma13.x, xa.y, Mn);
        Mn = fmaf((float)ma02.y, xa.z, Mn);
        Mn = fmaf((float)ma13.y, xa.w, Mn);
        Mn = fmaf((float)mb02.x, xb.x, Mn);
        Mn = fmaf((float)mb13.x, xb.y, Mn);
        Mn = fmaf((float)mb02.y, xb.z, Mn);
        Mn = fmaf((float)mb13.y, xb.w, Mn);
        // value = d * sc * q - dmin * m: C holds sum (q / 2) x, S carries
        // 2^-24 (the scale nibble), Mn 2^-20 (the min nibble)
        acc[m] = fmaf((float)dm.x * 33554432.0f, S, acc[m]);
        acc[m] = fmaf(term0 ? -(float)dm.y * 1048576.0f : 0.f, Mn, acc[m]);
      }
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      float r = acc[m];
      r += __shfl_xor(r, 16, kWave);
      r += __shfl_xor(r, 32, kWave);
      if (q == 0) part[(wave * 2 + m) * 16 + n] = r;
    }
    __syncthreads();
    // lanes 0..15 sum gate rows, lanes 16..31 up rows, over the wavefronts
    // in order; no barrier follows: the next tile's LDS writes only start
    // the next compute phase after a barrier this wavefront also reaches
    if (tid < 32) {
      float r = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) r += part[(w * 2 + (tid >> 4)) * 16 + (tid & 15)];
      const float u = __shfl_down(r, 16, kWave);
      if (tid < 16) {
        const uint32_t a = slot_a[slot];  // the slot's (single) assignment
        const float h = silu(r) * u * slot_w[slot];
        if (p.h_mfma)  // the MFMA down kernel reads h
          stage_run_lanes_mfma(h, p.stage_h + size_t(a) * run_stage_words(I), I, tile);
        else
          stage_run_lanes(h, p.stage_h + size_t(a) * staged_stride(I, true), I, tile);
      }
    }
  }
  if constexpr (SEL) {
    if (kWarmPer && !warmed) warm_down();
    // a workgroup without routed tiles sums its shared down parts here
    if (sd_rows) {
      __syncthreads();
      if (tid < sd_rows) SharedDownSlice::store(p, sdpart, tid, sd_row0);
    }
    // sink of the warm-up loads: they stay, and the kernel ends after them
#pragma unroll
    for (int j = 0; j < kWarmPer; ++j) asm volatile("" : : "v"(v[j]));
  }
}

// ------------------------------------------------------------------ down
//
// Routed down for one token on the matrix cores: output tile = 16 rows of
// H, all k ranks (the k selected experts' down rows [16t, 16t + 16), each
// 16 * NB * 84 contiguous bytes, streamed into LDS as in gate/up). A block
// (rank r, super-block column c) is one MFMA tile against h_r, whose rows
// the gate/up kernel staged with a per-run scale (stage_run_lanes_mfma);
// each wavefront takes the blocks b = wave + 16 j and keeps per-row sums.
// out = (residual + shared down) + routed, with the wavefronts' sums added
// in order: deterministic, no float atomics. The shared down (ys) was
// computed by the select launch.

constexpr int kMaxDownRanks = 8;

__host__ __device__ constexpr int down_chunks_per_thread(int NB, int k, int TR) {
  return (k * TR * NB * kQ2Bytes / 16 + kThreads - 1) / kThreads;
}

template <int NB, int TR, int PER>
__device__ __forceinline__ void fetch_down_tile(u32x4 (&v)[PER], const DecodeArgs& p, int k,
                                                const uint32_t* rank_e, int t) {
  constexpr int rb = NB * kQ2Bytes;   // bytes per row
  constexpr int cr = TR * rb / 16;    // chunks per rank tile (TR rows)
  const int tid = threadIdx.x, nv = k * cr;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    int i = j * kThreads + tid;
    i = i < nv ? i : nv - 1;  // clamped; the extra chunks are not stored
    const int r = i / cr, w = i - r * cr;
    const u32x4* src = reinterpret_cast<const u32x4*>(p.down + size_t(rank_e[r]) * p.down_stride +
                                                      size_t(t) * TR * rb);
    v[j] = ld_tile(src + w);
  }
}

// TR output rows per tile: 16, or 12 so that H = 6144 makes 512 tiles, two
// per workgroup on a 256-CU part (16-row tiles leave half the CUs a second
// round); MFMA columns n >= TR read stale LDS rows and are not written.
template <int NB, int TR, int PER>
__global__ void __launch_bounds__(kThreads) down_q2k_kernel(DecodeArgs p, int ntiles) {
  extern __shared__ uint32_t smem[];
  constexpr int K = NB * kKBlock;  // the expert intermediate I
  constexpr int rb = NB * kQ2Bytes, RS = rb + kRowPad, Sh = run_stage_words(K);
  constexpr int cr = TR * rb / 16;
  const int k = p.k;
  uint32_t* hs = smem;                             // [k][Sh]
  uint32_t* zero = hs + kMaxDownRanks * Sh;
  uint8_t* tl = reinterpret_cast<uint8_t*>(zero + 4);  // [k][16 rows][RS]
  float* part = reinterpret_cast<float*>(tl + kMaxDownRanks * 16 * RS);  // [wave][16]
  uint32_t* rank_e = reinterpret_cast<uint32_t*>(part + kWaves * 16);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, q = lane >> 4;
  if (tid < k) rank_e[tid] = p.ids[tid];
  u32x4 v[PER];
  int t = blockIdx.x;
  __syncthreads();
  // the staged h rows and the first tile in flight together
  LdsCopy<kThreads, (kMaxDownRanks * Sh / 4 + kThreads - 1) / kThreads> hcp;
  const uint4* hsrc = reinterpret_cast<const uint4*>(p.stage_h);
  hcp.load(hsrc, k * Sh / 4);
  if (t < ntiles) fetch_down_tile<NB, TR, PER>(v, p, k, rank_e, t);
  hcp.store(reinterpret_cast<uint4*>(hs), hsrc, k * Sh / 4);
  if (tid < 4) zero[tid] = 0;
  const bool act = q == 2 * (n >> 3) + (n & 1);
  const int pm = (n >> 1) & 3;
  const int nblk = k * NB;
  for (; t < ntiles; t += gridDim.x) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = j * kThreads + tid;
      if (i < k * cr) {
        const int r = i / cr, w = i - r * cr, row = w / (rb / 16), c16 = w - row * (rb / 16);
        *reinterpret_cast<u32x4*>(tl + (r * 16 + row) * RS + c16 * 16) = v[j];
      }
    }
    __syncthreads();
    if (t + int(gridDim.x) < ntiles) fetch_down_tile<NB, TR, PER>(v, p, k, rank_e, t + gridDim.x);
    float acc = 0.f;
    for (int b = wave; b < nblk; b += kWaves) {
      const int r = b / NB, c = b - r * NB;
      const uint32_t* hr = hs + r * Sh;
      half8 A[4][2];
#pragma unroll
      for (int pp = 0; pp < 4; ++pp)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const uint32_t* src = (act && pp == pm) ? hr + c * 128 + n * 8 + 4 * hf : zero;
          A[pp][hf] = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(src));
        }
      const float* sums = reinterpret_cast<const float*>(hr + K / 2);
      const float4 xsum = *reinterpret_cast<const float4*>(sums + c * 16 + 4 * q);
      const float4 kk = *reinterpret_cast<const float4*>(sums + K / 16 + c * 16 + 4 * q);
      const uint8_t* blk = tl + (r * 16 + n) * RS + c * kQ2Bytes;
      const u32x4_a4 qs = *reinterpret_cast<const u32x4_a4*>(blk + 16 + 16 * q);
      const uint32_t scw = *reinterpret_cast<const uint32_t*>(blk + 4 * q);
      const uint32_t dmw = *reinterpret_cast<const uint32_t*>(blk + 80);
      floatx4 C = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const uint32_t w0 = hf ? qs.z : qs.x, w1 = hf ? qs.w : qs.y;
        const uint32_t o0 = w0 >> 8, o1 = w1 >> 8;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const uint32_t M = 0x00030003u << (2 * pp);
          const uint4 bv = make_uint4(w0 & M, o0 & M, w1 & M, o1 & M);
          C = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[pp][hf], __builtin_bit_cast(half8, bv), C,
                                                     0, 0, 0);
        }
      }
      const uint32_t sh = scw >> 8;
      const half2v s02 = as_h2(scw & 0x000f000fu), s13 = as_h2(sh & 0x000f000fu);
      const half2v m02 = as_h2(scw & 0x00f000f0u), m13 = as_h2(sh & 0x00f000f0u);
      const half2v dm = as_h2(dmw);
      // per-run scales: group i of this lane is run 4q + i of column c
      float S = fmaf((float)s02.x, C[0] * kk.x, 0.f);
      S = fmaf((float)s13.x, C[1] * kk.y, S);
      S = fmaf((float)s02.y, C[2] * kk.z, S);
      S = fmaf((float)s13.y, C[3] * kk.w, S);
      float Mn = fmaf((float)m02.x, xsum.x, 0.f);
      Mn = fmaf((float)m13.x, xsum.y, Mn);
      Mn = fmaf((float)m02.y, xsum.z, Mn);
      Mn = fmaf((float)m13.y, xsum.w, Mn);
      acc = fmaf((float)dm.x, S, acc);
      acc = fmaf(-(float)dm.y * 1048576.0f, Mn, acc);
    }
    acc += __shfl_xor(acc, 16, kWave);
    acc += __shfl_xor(acc, 32, kWave);
    if (q == 0) part[wave * 16 + n] = acc;
    __syncthreads();
    // no barrier follows (as in gate/up): part is rewritten only after the
    // next tile's first barrier, which these lanes also reach
    if (tid < TR) {
      float y = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) y += part[w * 16 + tid];
      const size_t o = size_t(t) * TR + tid;
      const float base = (p.residual ? p.residual[o] : 0.f) + (p.ys ? p.ys[o] : 0.f);
      p.out[o] = base + y;
    }
  }
}

inline bool down_covers(int I, int k) {
  const int NB = I / kKBlock;
  return I % kKBlock == 0 && NB == 8 && k >= 1 && k <= kMaxDownRanks;
}

inline size_t down_lds_bytes(int I) {
  const int rb = I / kKBlock * kQ2Bytes;
  return size_t(kMaxDownRanks * run_stage_words(I) + 4) * 4 +
         size_t(kMaxDownRanks * 16) * (rb + kRowPad) + size_t(kWaves * 16) * 4 +
         size_t(kMaxDownRanks) * 4;
}

// True when the kernel has an instance for a layer of width H: NB = H / 256
// in {4, 8, ..., 28} (whole 16-byte chunks per row, at most five chunks per
// thread: six spill).
inline bool covers_width(int H) {
  const int NB = H / kKBlock;
  return H % kKBlock == 0 && NB % 4 == 0 && NB >= 4 && NB <= 28;
}

// sel: the selecting launch; Is_sd: the shared expert's width when its down
// runs in that launch, else 0
inline size_t lds_bytes(int H, int quant = INFERNO_Q2_K, bool sel = false, int Is_sd = 0) {
  return size_t(fp4_lds_layout(H, quant, sel, Is_sd).end);
}

}  // namespace mfma_decode
}  // namespace inferno
