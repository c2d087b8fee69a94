// Router: fp32 logits projection and exact top-k gating.
//
// Top-k follows crates/model/src/moe_router.rs:835-940: selection value
// (sigmoid score + bias, or logit + bias for softmax), ordered by
// f32::total_cmp descending with the lower expert id winning ties; weights
// are the unbiased scores in rank order, renormalised by their rank-order
// sum, times the routed scaling factor. One wavefront per token; every lane
// holds up to four candidates and each round is a DPP wavefront max of the
// order-preserving key, then of ~expert id among the lanes holding that key
// (routing_dev.hpp).
#include <cstdlib>

#include "routing_dev.hpp"

namespace inferno {
namespace {

template <typename T>
__device__ __forceinline__ float load_x(const T* p, size_t i);
template <>
__device__ __forceinline__ float load_x<float>(const float* p, size_t i) {
  return p[i];
}
template <>
__device__ __forceinline__ float load_x<uint16_t>(const uint16_t* p, size_t i) {
  return bf16_bits_to_f32(p[i]);
}


// Few tokens, H not a multiple of 32 (else the matrix-core kernels): one
// wavefront per expert row; the row is read once with 16-byte loads and
// dotted with every token (T <= 16).
template <typename XT>
__global__ void __launch_bounds__(256)
    logits_small_kernel(const XT* __restrict__ x, const float* __restrict__ w, int T, int H,
                        int E, float* __restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= E) return;
  float acc[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t] = 0.f;
  const float* row = w + size_t(e) * H;
  for (int h0 = lane * 4; h0 < H; h0 += 256) {
    float4 wv = *reinterpret_cast<const float4*>(row + h0);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      if (t < T) {
        const size_t base = size_t(t) * H + h0;
        acc[t] += wv.x * load_x(x, base) + wv.y * load_x(x, base + 1) +
                  wv.z * load_x(x, base + 2) + wv.w * load_x(x, base + 3);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    if (t < T) {
      float s = wave_sum(acc[t]);
      if (lane == 0) logits[size_t(t) * E + e] = s;
    }
  }
}

// Many tokens: 64x64 output tile per 256-thread block, K staged through LDS,
// 4x4 outputs per thread.
template <typename XT>
__global__ void __launch_bounds__(256)
    logits_tiled_kernel(const XT* __restrict__ x, const float* __restrict__ w, int T, int H,
                        int E, float* __restrict__ logits) {
  constexpr int TM = 64, TN = 64, TK = 32;
  __shared__ float xs[TK][TM + 4];
  __shared__ float ws[TK][TN + 4];
  const int tid = threadIdx.x;
  const int m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
  const int tm = (tid / 16) * 4, tn = (tid % 16) * 4;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < H; k0 += TK) {
    for (int i = tid; i < TM * TK; i += 256) {
      int r = i / TK, c = i % TK;
      int gm = m0 + r, gk = k0 + c;
      xs[c][r] = (gm < T && gk < H) ? load_x(x, size_t(gm) * H + gk) : 0.f;
      int gn = n0 + r;
      ws[c][r] = (gn < E && gk < H) ? w[size_t(gn) * H + gk] : 0.f;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < TK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = xs[kk][tm + i];
        b[i] = ws[kk][tn + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int gm = m0 + tm + i, gn = n0 + tn + j;
      if (gm < T && gn < E) logits[size_t(gm) * E + gn] = acc[i][j];
    }
}

// Many tokens on the fp32 matrix cores (v_mfma_f32_16x16x4_f32: fp32 products
// and sums, so the logits keep fp32 accuracy). A wavefront computes 16
// experts x 16*NTB tokens; a workgroup of four covers 64 experts. Per 32-deep
// K block, lane (row r = lane % 16, group g = lane / 16) holds
// w[e0 + r][k0 + 8 g .. +8] and the same eight k of each of its NTB token
// rows; MFMA step j multiplies element j of every group (k = k0 + 8 g + j).
typedef float float4v __attribute__((ext_vector_type(4)));

template <typename XT>
__device__ __forceinline__ void load8(const XT* p, bool ok, float v[8]);
template <>
__device__ __forceinline__ void load8<float>(const float* p, bool ok, float v[8]) {
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
  if (ok) {
    a = *reinterpret_cast<const float4*>(p);
    b = *reinterpret_cast<const float4*>(p + 4);
  }
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, bool ok, float v[8]) {
  uint4 q = make_uint4(0, 0, 0, 0);
  if (ok) q = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __builtin_bit_cast(float, w[i] << 16);
    v[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
  }
}

template <typename XT, int NTB>
__global__ void __launch_bounds__(256)
    logits_mfma_kernel(const XT* __restrict__ x, const float* __restrict__ w, int T, int H, int E,
                       float* __restrict__ logits, uint16_t* __restrict__ x16 = nullptr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int e0 = blockIdx.x * 64 + wave * 16, t0 = blockIdx.y * (16 * NTB);
  const bool ev = e0 + r < E;
  const float* wrow = w + size_t(ev ? e0 + r : 0) * H + 8 * g;
  const XT* xrow[NTB];
  bool tv[NTB];
#pragma unroll
  for (int b = 0; b < NTB; ++b) {
    const int t = t0 + 16 * b + r;
    tv[b] = t < T;
    xrow[b] = x + size_t(tv[b] ? t : 0) * H + 8 * g;
  }
  float4v acc[NTB][2];
#pragma unroll
  for (int b = 0; b < NTB; ++b)
#pragma unroll
    for (int h = 0; h < 2; ++h) acc[b][h] = float4v{0.f, 0.f, 0.f, 0.f};
  // blockIdx.z: K chunk of H / gridDim.z (whole 32-deep blocks), partial
  // logits to logits + z T E (summed in chunk order by the top-k kernel)
  const int kc = H / int(gridDim.z), kbeg = int(blockIdx.z) * kc;
  logits += size_t(blockIdx.z) * size_t(T) * E;
  for (int k0 = kbeg; k0 < kbeg + kc; k0 += 32) {
    float a[8];
    load8<float>(wrow + k0, ev, a);
#pragma unroll
    for (int b = 0; b < NTB; ++b) {
      float v[8];
      load8<XT>(xrow[b] + k0, tv[b], v);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[b][j & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], v[j], acc[b][j & 1], 0, 0, 0);
      // x16: the f16 copy of x for the grouped GEMMs (to_f16_kernel's k
      // order 0 2 1 3 4 6 5 7), written by the first expert group's first
      // wavefront, which reads every token row of the tile over its chunk
      if (x16 != nullptr && blockIdx.x == 0 && wave == 0 && tv[b]) {
        auto pair = [](float lo, float hi) {
          return uint32_t(__builtin_bit_cast(uint16_t, (_Float16)lo)) |
                 (uint32_t(__builtin_bit_cast(uint16_t, (_Float16)hi)) << 16);
        };
        *reinterpret_cast<uint4*>(x16 + size_t(t0 + 16 * b + r) * H + k0 + 8 * g) =
            make_uint4(pair(v[0], v[2]), pair(v[1], v[3]), pair(v[4], v[6]), pair(v[5], v[7]));
      }
    }
  }
  // lane holds C[4 g + q][r]: expert e0 + 4 g + q, token t0 + 16 b + r
#pragma unroll
  for (int b = 0; b < NTB; ++b) {
    const int t = t0 + 16 * b + r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = e0 + 4 * g + q;
      if (t < T && e < E) logits[size_t(t) * E + e] = acc[b][0][q] + acc[b][1][q];
    }
  }
}

// Many bf16 tokens on the bf16 matrix cores without losing fp32 accuracy:
// every fp32 router weight is the exact sum of three bf16 terms (truncate,
// subtract, truncate the remainder, subtract: the last remainder has at most
// eight significant bits), a bf16 x bf16 product is exact in fp32, so
// x . w = sum of three bf16 MFMA dots accumulated in fp32. Per 32-deep K
// block lane (row r = lane % 16, group
// g = lane / 16) holds w[e][k0 + 8 g .. + 8] and the same eight k of each
// token row: v_mfma_f32_16x16x32_bf16 pairs the operands slot by slot.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void split3(const float4& a, const float4& b, u32x4v t[3]) {
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t h[3][8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v[j]);
    const uint32_t u1 = u & 0xffff0000u;
    const float r1 = v[j] - __builtin_bit_cast(float, u1);
    const uint32_t u2 = __builtin_bit_cast(uint32_t, r1) & 0xffff0000u;
    const float r2 = r1 - __builtin_bit_cast(float, u2);
    h[0][j] = u1;
    h[1][j] = u2;
    h[2][j] = __builtin_bit_cast(uint32_t, r2);
  }
#pragma unroll
  for (int m = 0; m < 3; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      t[m][i] = __builtin_amdgcn_perm(h[m][2 * i + 1], h[m][2 * i], 0x07060302u);
}

// A workgroup of 4 * KS wavefronts covers 64 experts x 16 * NTB tokens;
// wavefront (s, q) takes experts e0 + 16 q and the 32-deep K blocks s,
// s + KS, ...; the KS partial tiles are summed through LDS in split order
// (fixed, so the logits do not depend on scheduling). Operands are loaded
// straight in MFMA layout, two register sets in flight. (Staging 64-deep K
// slices through LDS with whole-line loads measured no faster: the kernel is
// bound by bytes moved into each CU, about 17 GB/s per CU, not by the access
// pattern.) Rows past E or T read row 0 and are never stored: MFMA output
// rows and columns are independent, so the loads need no masks.
// blockIdx.z splits K into gridDim.z chunks of whole 32-deep blocks (every
// chunk a multiple of 2 KS of them): chunk z writes its partial logits to
// logits + z T E, summed in chunk order by the top-k kernel; a small batch
// then spreads over enough workgroups to draw on every CU.
// x16 (non-null only for KS = 1): the f16 copy of x for the grouped GEMMs
// (to_f16_kernel's values and k order 0 2 1 3 4 6 5 7), written by the first
// expert group's first wavefront from the token rows it loads over its chunk.
template <int NTB, int KS>
__global__ void __launch_bounds__(256 * KS)
    logits_bf16x3_kernel(const uint16_t* __restrict__ x, const float* __restrict__ w, int T,
                         int H, int E, float* __restrict__ logits,
                         uint16_t* __restrict__ x16 = nullptr) {
  __shared__ float4v part[KS > 1 ? KS - 1 : 1][4][NTB][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = wave & 3, s = wave >> 2;
  const int r = lane & 15, g = lane >> 4;
  const int e0 = blockIdx.x * 64 + q * 16, t0 = blockIdx.y * (16 * NTB);
  const float* wrow = w + size_t(e0 + r < E ? e0 + r : 0) * H + 8 * g;
  const uint16_t* xrow[NTB];
#pragma unroll
  for (int b = 0; b < NTB; ++b) {
    const int t = t0 + 16 * b + r;
    xrow[b] = x + size_t(t < T ? t : 0) * H + 8 * g;
  }
  float4v acc[NTB];
#pragma unroll
  for (int b = 0; b < NTB; ++b) acc[b] = float4v{0.f, 0.f, 0.f, 0.f};
  const int nkz = H / 32 / int(gridDim.z);  // blocks in this chunk
  const int kz0 = int(blockIdx.z) * nkz;
  const int nkb = kz0 + nkz;
  logits += size_t(blockIdx.z) * size_t(T) * E;
  struct Buf {
    float4 wa, wb;
    u32x4v xv[NTB];
  };
  // out-of-range prefetches re-read the last block (harmless, never used)
  auto load = [&](int kb, Buf& u) {
    const int k0 = (kb < nkb ? kb : nkb - 1) * 32;
    u.wa = *reinterpret_cast<const float4*>(wrow + k0);
    u.wb = *reinterpret_cast<const float4*>(wrow + k0 + 4);
#pragma unroll
    for (int b = 0; b < NTB; ++b) u.xv[b] = *reinterpret_cast<const u32x4v*>(xrow[b] + k0);
  };
  auto compute = [&](const Buf& u) {
    u32x4v wt[3];
    split3(u.wa, u.wb, wt);
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int b = 0; b < NTB; ++b)
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wt[m]),
                                                         __builtin_bit_cast(bf16x8, u.xv[b]),
                                                         acc[b], 0, 0, 0);
  };
  const bool w16 = KS == 1 && x16 != nullptr && blockIdx.x == 0 && wave == 0;  // uniform
  auto store16 = [&](const Buf& u, int kb) {
#pragma unroll
    for (int b = 0; b < NTB; ++b) {
      const int t = t0 + 16 * b + r;
      if (t >= T) continue;
      auto f16 = [](uint32_t bf) {  // bf16 bits -> fp32 -> f16 (round to nearest even)
        return uint32_t(__builtin_bit_cast(uint16_t, (_Float16)__builtin_bit_cast(float, bf)));
      };
      uint32_t h[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h[2 * i] = f16(u.xv[b][i] << 16);
        h[2 * i + 1] = f16(u.xv[b][i] & 0xffff0000u);
      }
      *reinterpret_cast<uint4*>(x16 + size_t(t) * H + kb * 32 + 8 * g) =
          make_uint4(h[0] | (h[2] << 16), h[1] | (h[3] << 16), h[4] | (h[6] << 16),
                     h[5] | (h[7] << 16));
    }
  };
  // the host launches this kernel only when 2 * KS divides the chunk's blocks
  Buf u0, u1;
  load(kz0 + s, u0);
  load(kz0 + s + KS, u1);
  for (int kb = kz0 + s; kb < nkb; kb += 2 * KS) {
    compute(u0);
    if (w16) store16(u0, kb);
    load(kb + 2 * KS, u0);
    compute(u1);
    if (w16) store16(u1, kb + KS);
    load(kb + 3 * KS, u1);
  }
  if constexpr (KS > 1) {
    if (s > 0)
#pragma unroll
      for (int b = 0; b < NTB; ++b) part[s - 1][q][b][lane] = acc[b];
    __syncthreads();
    if (s > 0) return;
#pragma unroll
    for (int j = 0; j < KS - 1; ++j)
#pragma unroll
      for (int b = 0; b < NTB; ++b) acc[b] += part[j][q][b][lane];
  }
  // lane holds C[4 g + i][r]: expert e0 + 4 g + i, token t0 + 16 b + r
#pragma unroll
  for (int b = 0; b < NTB; ++b) {
    const int t = t0 + 16 * b + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + 4 * g + i;
      if (t < T && e < E) logits[size_t(t) * E + e] = acc[b][i];
    }
  }
}

// One wavefront per token.
__global__ void __launch_bounds__(256)
    topk_kernel(const float* __restrict__ logits, const float* __restrict__ bias, int T, int E,
                int k, int score_fn, int norm, float scale, uint32_t* __restrict__ ids,
                float* __restrict__ weights, uint32_t* __restrict__ token_idx) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  uint32_t sel[kMaxTopK];
  topk_row_wave(logits + size_t(t) * E, bias, E, k, score_fn, norm, scale, t, ids, weights,
                token_idx, sel);
}

// K-chunk partial logits [parts][T][E] (parts <= kMaxRouterParts): one token
// per workgroup; thread e sums expert e's partials in chunk order (all loads
// issued together) into an LDS row, then wavefront 0 selects.
constexpr int kMaxRouterParts = 16;
__global__ void __launch_bounds__(256)
    topk_parts_kernel(const float* __restrict__ parts_in, const float* __restrict__ bias, int T,
                      int E, int k, int score_fn, int norm, float scale, uint32_t* __restrict__ ids,
                      float* __restrict__ weights, uint32_t* __restrict__ token_idx, int parts) {
  __shared__ float row[kMaxExperts];
  const int t = blockIdx.x, e = threadIdx.x;
  if (e < E) {
    const float* src = parts_in + size_t(t) * E + e;
    const size_t stride = size_t(T) * E;
    float v[kMaxRouterParts];
#pragma unroll
    for (int z = 0; z < kMaxRouterParts; ++z)  // clamped: all loads go out together
      v[z] = src[size_t(min(z, parts - 1)) * stride];
    float sum = 0.f;
#pragma unroll
    for (int z = 0; z < kMaxRouterParts; ++z)
      if (z < parts) sum += v[z];
    row[e] = sum;
  }
  __syncthreads();
  if (threadIdx.x >= 64) return;
  uint32_t sel[kMaxTopK];
  topk_row_wave(row, bias, E, k, score_fn, norm, scale, t, ids, weights, token_idx, sel);
}

}  // namespace

// INFERNO_ROUTER_BF16X3=0 keeps the fp32 matrix-core logits for bf16 tokens.
static bool bf16x3_enabled() {
  return !switch_off("INFERNO_ROUTER_BF16X3");
}

// K chunks for the router logits of a T-token batch (bf16 tokens on the
// bf16x3 kernel, fp32 tokens on the fp32 MFMA kernel): 1 when the
// batch alone gives the kernel enough workgroups; else the most (a power of
// two, up to kMaxRouterParts) that keeps at most kRouterSplitGroups
// workgroups of the one-group kernel and a whole number of 32-deep block
// pairs per chunk.
constexpr size_t kRouterSplitGroups = 256;
int router_logit_parts_max(size_t T, size_t H, size_t E) {
  if (H % 256) return 1;
  const size_t base = ((E + 63) / 64) * ((T + 15) / 16);
  if (base * 2 > kRouterSplitGroups) return 1;
  int z = 1;
  while (z < kMaxRouterParts && base * size_t(2 * z) <= kRouterSplitGroups && (H / 32) % size_t(4 * z) == 0) z *= 2;
  return z;
}
bool router_writes_x16(size_t T, size_t H, size_t E, int x_dtype, int parts) {
  (void)T; (void)E;
  return parts > 1 && H % 32 == 0;
}

int router_logit_parts(size_t T, size_t H, size_t E, int x_dtype) {
  if (x_dtype == INFERNO_BF16 && !bf16x3_enabled()) return 1;
  return router_logit_parts_max(T, H, E);
}

int launch_router_logit_parts(hipStream_t s, const void* x, int x_dtype, const float* w, size_t T,
                              size_t H, size_t E, float* parts_out, int parts, uint16_t* x16) {
  if (x16 != nullptr && !router_writes_x16(T, H, E, x_dtype, parts)) {
    set_error("router logits: this launch does not write the f16 copy of x");
    return INFERNO_ERR_INVALID;
  }
  if (parts <= 1) return launch_router_logits(s, x, x_dtype, w, T, H, E, parts_out);
  if (T == 0 || E == 0) return INFERNO_OK;
  const dim3 grid(unsigned((E + 63) / 64), unsigned((T + 15) / 16), unsigned(parts));
  if (x_dtype == INFERNO_BF16)
    logits_bf16x3_kernel<1, 1><<<grid, 256, 0, s>>>(static_cast<const uint16_t*>(x), w, int(T),
                                                    int(H), int(E), parts_out, x16);
  else  // fp32 tokens on the fp32 matrix cores, K split the same way
    logits_mfma_kernel<float, 1><<<grid, 256, 0, s>>>(static_cast<const float*>(x), w, int(T),
                                                      int(H), int(E), parts_out, x16);
  INF_LAUNCHED();
  return INFERNO_OK;
}

int launch_router_logits(hipStream_t s, const void* x, int x_dtype, const float* w, size_t T,
                         size_t H, size_t E, float* logits) {
  if (T == 0 || E == 0) return INFERNO_OK;
  if (T <= 16 && H % 32) {
    dim3 grid(unsigned((E + 3) / 4));
    if (x_dtype == INFERNO_BF16)
      logits_small_kernel<uint16_t><<<grid, 256, 0, s>>>(static_cast<const uint16_t*>(x), w,
                                                         int(T), int(H), int(E), logits);
    else
      logits_small_kernel<float><<<grid, 256, 0, s>>>(static_cast<const float*>(x), w, int(T),
                                                      int(H), int(E), logits);
  } else if (H % 32 == 0) {
    // fp32 MFMA: 64-token wavefront tiles for large batches (router rows
    // reused four times per load), 16-token tiles otherwise (more tiles)
    const bool wide = T >= 2048;
    const unsigned tt = wide ? 64u : 16u;
    dim3 grid(unsigned((E + 63) / 64), unsigned((T + tt - 1) / tt));
    if (x_dtype == INFERNO_BF16 && H % 256 == 0 && bf16x3_enabled()) {
      // 64-token tiles, K split in two, for large batches; 16-token tiles,
      // K split in four, otherwise (more waves for fewer tiles)
      if (wide)
        logits_bf16x3_kernel<4, 2><<<grid, 512, 0, s>>>(static_cast<const uint16_t*>(x), w,
                                                        int(T), int(H), int(E), logits);
      else
        logits_bf16x3_kernel<1, 4><<<grid, 1024, 0, s>>>(static_cast<const uint16_t*>(x), w,
                                                         int(T), int(H), int(E), logits);
    } else if (x_dtype == INFERNO_BF16) {
      if (wide)
        logits_mfma_kernel<uint16_t, 4><<<grid, 256, 0, s>>>(static_cast<const uint16_t*>(x), w,
                                                             int(T), int(H), int(E), logits);
      else
        logits_mfma_kernel<uint16_t, 1><<<grid, 256, 0, s>>>(static_cast<const uint16_t*>(x), w,
                                                             int(T), int(H), int(E), logits);
    } else {
      if (wide)
        logits_mfma_kernel<float, 4><<<grid, 256, 0, s>>>(static_cast<const float*>(x), w, int(T),
                                                          int(H), int(E), logits);
      else
        logits_mfma_kernel<float, 1><<<grid, 256, 0, s>>>(static_cast<const float*>(x), w, int(T),
                                                          int(H), int(E), logits);
    }
  } else {
    dim3 grid(unsigned((E + 63) / 64), unsigned((T + 63) / 64));
    if (x_dtype == INFERNO_BF16)
      logits_tiled_kernel<uint16_t><<<grid, 256, 0, s>>>(static_cast<const uint16_t*>(x), w,
                                                         int(T), int(H), int(E), logits);
    else
      logits_tiled_kernel<float><<<grid, 256, 0, s>>>(static_cast<const float*>(x), w, int(T),
                                                      int(H), int(E), logits);
  }
  INF_LAUNCHED();
  return INFERNO_OK;
}

int launch_router_topk(hipStream_t s, const float* logits, const float* bias, size_t T, size_t E,
                       size_t k, int score_fn, int norm, float scale, uint32_t* ids,
                       float* weights, uint32_t* token_idx, int parts) {
  if (T == 0) return INFERNO_OK;
  if (parts > 1)
    topk_parts_kernel<<<unsigned(T), 256, 0, s>>>(logits, bias, int(T), int(E), int(k), score_fn,
                                                   norm, scale, ids, weights, token_idx, parts);
  else
    topk_kernel<<<unsigned((T + 3) / 4), 256, 0, s>>>(logits, bias, int(T), int(E), int(k),
                                                      score_fn, norm, scale, ids, weights,
                                                      token_idx);
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace inferno
