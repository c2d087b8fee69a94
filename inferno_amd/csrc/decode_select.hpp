// One-token selection and Q8_0 shared-expert down, shared by the decode
// select launch and the fp8 x fp4 gate/up launch that absorbs it.
//
// With one token the dispatch is the k selected ids sorted ascending, one
// assignment each (crates/moe/src/routing.rs:27-85 with T = 1), and the
// shared expert's down (crates/backend/src/backend.rs:1682,
// laguna_q8_0_matvec_add2_device) only needs the shared gate/up partial sums
// of the route launch, so both can run in any launch after it. No workgroup
// waits on another: every workgroup that needs the selection computes it.
#pragma once
#include "decode.hpp"
#include "dot2_formats.hpp"
#include "routing_dev.hpp"

namespace inferno {

// Lanes of one full wavefront write, from topk1_wave's result, the ids and
// weights (rank order), then the dispatch and the slot descriptors (slot j =
// the j-th smallest id, assignment = its rank).
__device__ __forceinline__ void select1_write(const DecodeArgs& p, const Top1Lds* tk) {
  const int lane = threadIdx.x & 63;
  const int E = p.E, k = p.k;
  if (lane < k) {
    p.ids[lane] = tk->rid[lane];
    p.weights[lane] = tk->w[lane];
    const uint32_t id = tk->id[lane], rank = tk->rank[lane];
    p.sorted[lane] = rank;  // assignment index t*k + r with t = 0
    p.active[1 + lane] = id;
    p.slots[lane] = make_uint4(id, uint32_t(lane), uint32_t(lane) + 1u, rank);
  }
  if (lane == 0) p.active[0] = uint32_t(k);
  // offsets[e] = number of ids below e
  uint32_t ids[kMaxTopK];
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) ids[j] = j < k ? tk->id[j] : 0xffffffffu;
  for (int e = lane; e <= E; e += 64) {
    uint32_t below = 0;
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) below += ids[j] < uint32_t(e) ? 1u : 0u;
    p.offsets[e] = below;
  }
}

// The token's logits from the route launch's chunk partials (summed in chunk
// order, as sum_partials) and the bias, lane holding experts lane + 64 j; all
// loads are issued before the sums, unconditionally (indices clamped, values
// past the ends replaced by zero afterwards): a load under a branch makes the
// join wait for its data. One full wavefront.
__device__ __forceinline__ void load_logits1(const DecodeArgs& p, float (&lg)[4], float (&bs)[4]) {
  const int lane = threadIdx.x & 63;
  const int E = p.E, nc = p.n_chunks;
  const float* bp = p.bias ? p.bias : p.partials;  // uniform
  float bv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bv[j] = bp[min(lane + 64 * j, E - 1)];
  for (int c0 = 0; c0 < nc; c0 += 8) {
    float v[4][8];  // 32 loads in flight
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int c = 0; c < 8; ++c)
        v[j][c] = p.partials[size_t(min(c0 + c, nc - 1)) * E + min(lane + 64 * j, E - 1)];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool live = lane + 64 * j < E;
      float s = c0 == 0 ? 0.f : lg[j];
#pragma unroll
      for (int c = 0; c < 8; ++c)  // zeros past the last chunk, as sum_partials
        s += (live && c0 + c < nc) ? v[j][c] : 0.f;
      lg[j] = s;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) bs[j] = (p.bias && lane + 64 * j < E) ? bv[j] : 0.f;
}

// h = silu(sum of gate partials) * (sum of up partials) of the shared expert,
// staged as a packed-f16 row (xss, Is values). One lane forms the float4 at
// position v4 (values 4 v4 .. + 3, parts added in order 0, 1, ... as the
// gate/up kernels do); a lane quad holds one 16-value run, which gives the
// run's maximum, its sum in value order (as stage_run forms it) and the hi
// pair words 2 (v4 & 3), + 1, which take only this lane's values. Every lane
// of the wavefront must take part (quad shuffles).
constexpr int kMaxSharedParts = 8;
struct SharedHQuad {
  float4 gv[kMaxSharedParts], uv[kMaxSharedParts];
  // unconditional loads (part and position clamped; stage() drops the
  // extra parts): a load under a branch makes the join wait for its data
  __device__ __forceinline__ void load(const DecodeArgs& p, int v4, bool live) {
    const int Is = p.Is, v = live ? v4 : 0;
#pragma unroll
    for (int k = 0; k < kMaxSharedParts; ++k) {
      const size_t kk = size_t(min(k, p.shared_parts - 1));
      gv[k] = reinterpret_cast<const float4*>(p.shared_gu + (kk * 2) * Is)[v];
      uv[k] = reinterpret_cast<const float4*>(p.shared_gu + (kk * 2 + 1) * Is)[v];
    }
  }
  __device__ __forceinline__ void stage(const DecodeArgs& p, uint32_t* xss, int v4, bool live) {
    const int lane = threadIdx.x & 63;
    const int Is = p.Is, parts = p.shared_parts;
    float4 gs = make_float4(0.f, 0.f, 0.f, 0.f), us = gs;
#pragma unroll
    for (int k = 0; k < kMaxSharedParts; ++k)
      if (live && k < parts) {
        gs.x += gv[k].x; gs.y += gv[k].y; gs.z += gv[k].z; gs.w += gv[k].w;
        us.x += uv[k].x; us.y += uv[k].y; us.z += uv[k].z; us.w += uv[k].w;
      }
    const float h0 = silu(gs.x) * us.x, h1 = silu(gs.y) * us.y;
    const float h2 = silu(gs.z) * us.z, h3 = silu(gs.w) * us.w;
    float m = fmaxf(fmaxf(fabsf(h0), fabsf(h1)), fmaxf(fabsf(h2), fabsf(h3)));
    m = fmaxf(m, __shfl_xor(m, 1, kWave));
    m = fmaxf(m, __shfl_xor(m, 2, kWave));
    const int q0 = lane & ~3;
    float sum = 0.f;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) sum = __shfl((((sum + h0) + h1) + h2) + h3, q0 + qq, kWave);
    float scale = 1.0f;  // zero or non-finite runs keep scale 1
    if (m > 0.f && m < 3.0e38f) {
      int e;
      frexpf(m, &e);
      scale = ldexpf(1.0f, 15 - e);
    }
    auto pack = [](float a, float b) {
      const _Float16 ah = (_Float16)a, bh = (_Float16)b;
      return uint32_t(__builtin_bit_cast(uint16_t, ah)) | (uint32_t(__builtin_bit_cast(uint16_t, bh)) << 16);
    };
    if (!live) return;
    const int run = v4 >> 2, qi = v4 & 3;
    *reinterpret_cast<uint2*>(xss + run * 8 + 2 * qi) =
        make_uint2(pack(h0 * scale, h2 * scale), pack(h1 * scale, h3 * scale));
    if (qi == 0) {
      float* sums = reinterpret_cast<float*>(xss + Is / 2);
      sums[run] = sum;
      sums[Is / 16 + run] = 1.0f / scale;
    }
  }
};

// The whole shared h by NT threads (thread index tid, whole wavefronts);
// all of a thread's loads are issued before its sums. Is / 4 must be a
// multiple of 64.
template <int NT>
__device__ __forceinline__ void form_shared_h(const DecodeArgs& p, uint32_t* xss, int tid) {
  // float4 positions per thread in flight (each holds every part's loads)
  constexpr int kIt = (NT >= 1024 || kMaxSharedParts > 4) ? 1 : 2;
  const int n4 = p.Is / 4;
  for (int v0 = tid; v0 < n4; v0 += NT * kIt) {
    SharedHQuad hq[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) hq[it].load(p, v0 + NT * it, v0 + NT * it < n4);
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      if (v0 + NT * it >= n4) break;  // uniform per wavefront: n4 is a multiple of 64
      hq[it].stage(p, xss, v0 + NT * it, true);
    }
  }
}

// Shared down of a workgroup's rows in the gate/up launch: rows [row0, row0
// + nrows) (whole 8-row octets, at most three), staged in LDS as they lie in
// the file (rows of Is / 32 Q8_0 blocks). kSdWpo wavefronts per octet:
// wavefront w takes octet j = w / kSdWpo and lane (row r = (lane >> 2) & 7,
// sub = lane & 3, cp = lane >> 5) the 256-value unit q = cp + 2 (w %
// kSdWpo) of its row (two Q8_0 blocks of it, sub). dot() reduces the unit
// against the staged h (xss) over sub and cp within the wavefront into
// part[w][r]; store() (after a barrier) adds an octet's kSdWpo parts in
// order into ys. One unit per lane: Is <= 512 kSdWpo.
constexpr int kSdWpo = 4;
constexpr int kSdMaxOctets = 3;
struct SharedDownSlice {
  using FS = Fmt<INFERNO_Q8_0>;
  __device__ __forceinline__ static size_t row_bytes(int Is) { return size_t(Is / 32) * 34; }
  __device__ __forceinline__ static void dot(const DecodeArgs& p, const uint32_t* rows,
                                             const uint32_t* xss, int w, float* part) {
    const int lane = threadIdx.x & 63;
    const int r = (lane >> 2) & 7, sub = lane & 3, cp = lane >> 5;
    const int Is = p.Is, ubs = Is / kKBlock, q = cp + 2 * (w % kSdWpo);
    float acc = 0.f;
    if (q < ubs) {
      // the lane's 68 bytes, dword aligned (rows and units are multiples of 4 bytes)
      const uint32_t* src = rows + (size_t((w / kSdWpo) * 8 + r) * row_bytes(Is) +
                                    size_t(q) * FS::kBytes + size_t(sub) * 68) / 4;
      uint32_t raw[FS::kDw];
#pragma unroll
      for (int i = 0; i < FS::kDw; ++i) raw[i] = src[i];
      acc = FS::dot(raw, sub, xrow_at<false>(xss, Is, q));
    }
    acc += __shfl_xor(acc, 1, kWave);
    acc += __shfl_xor(acc, 2, kWave);
    acc += __shfl_xor(acc, 32, kWave);
    if ((lane & 35) == 0) part[w * 8 + r] = acc;
  }
  // The same dot with the wavefront's own rows in LDS, copied there by
  // fetch_lds: row r of the octet at r * nu units (nu = units(w, Is)).
  __device__ __forceinline__ static int units(int w, int Is) {
    return max(0, min(2, Is / kKBlock - 2 * (w % kSdWpo)));
  }
  __device__ __forceinline__ static void dot_lds(const DecodeArgs& p, const uint32_t* wrows,
                                                 const uint32_t* xss, int w, float* part) {
    const int lane = threadIdx.x & 63;
    const int r = (lane >> 2) & 7, sub = lane & 3, cp = lane >> 5;
    const int Is = p.Is, nu = units(w, Is), q = cp + 2 * (w % kSdWpo);
    float acc = 0.f;
    if (cp < nu) {
      const uint32_t* src = wrows + (size_t(r * nu + cp) * FS::kBytes + size_t(sub) * 68) / 4;
      uint32_t raw[FS::kDw];
#pragma unroll
      for (int i = 0; i < FS::kDw; ++i) raw[i] = src[i];
      acc = FS::dot(raw, sub, xrow_at<false>(xss, Is, q));
    }
    acc += __shfl_xor(acc, 1, kWave);
    acc += __shfl_xor(acc, 2, kWave);
    acc += __shfl_xor(acc, 32, kWave);
    if ((lane & 35) == 0) part[w * 8 + r] = acc;
  }
  // LDS bytes per wavefront for fetch_lds: 8 rows x 2 units
  static constexpr int kWaveLds = 8 * 2 * FS::kBytes;
  // Wavefront w's rows of its octet (its units only) into wrows by the LDS
  // DMA (64 consecutive 16-byte chunks per copy, counted in vmcnt; the
  // caller waits). The last copy ends at the last chunk (it starts inside
  // the previous one: those chunks are written twice with the same bytes).
  __device__ __forceinline__ static void fetch_lds(const DecodeArgs& p, uint32_t* wrows, int w,
                                                   int row0) {
    const int lane = threadIdx.x & 63, Is = p.Is, nu = units(w, Is);
    if (nu == 0) return;  // uniform
    const int cpr = nu * (FS::kBytes / 16), nch = 8 * cpr;  // 16-byte chunks
    const uint8_t* base = p.sdown + size_t(row0 + (w / kSdWpo) * 8) * row_bytes(Is) +
                          size_t(2 * (w % kSdWpo)) * FS::kBytes;
    static_assert(8 * (FS::kBytes / 16) >= kWave, "one copy fits a one-unit octet");
    for (int b0 = 0; b0 < nch; b0 += kWave) {
      const int b = min(b0, nch - kWave), c = b + lane, r = c / cpr, cc = c - r * cpr;
      const uint8_t* src = base + size_t(r) * row_bytes(Is) + size_t(cc) * 16;
      __builtin_amdgcn_global_load_lds(
          (__attribute__((address_space(1))) const void*)src,
          (__attribute__((address_space(3))) void*)(reinterpret_cast<uint8_t*>(wrows) + b * 16), 16,
          0, 0);
    }
  }
  // thread i < nrows: row row0 + i
  __device__ __forceinline__ static void store(const DecodeArgs& p, const float* part, int i,
                                               int row0) {
    const int j = i >> 3, r = i & 7;
    float y = 0.f;
#pragma unroll
    for (int wi = 0; wi < kSdWpo; ++wi) y += part[(j * kSdWpo + wi) * 8 + r];
    p.ys[size_t(row0 + i)] = y;
  }
};

}  // namespace inferno
