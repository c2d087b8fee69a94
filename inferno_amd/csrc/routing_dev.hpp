// Device-side routing helpers shared by the router kernels and the fused
// decode path: exact top-k per token on one wavefront
// (crates/model/src/moe_router.rs:835-940 semantics) and the deterministic
// single-workgroup dispatch.
#pragma once
#include "kernels.hpp"

namespace inferno {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// Order-preserving map of the f32 total order (f32::total_cmp) onto u32.
__device__ __forceinline__ uint32_t total_order_key(float f) {
  uint32_t b = f32_to_bits(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// Wavefront max of a u32 with DPP row moves and four readlanes; every lane
// of the wavefront must be active. Returns the (uniform) maximum.
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0xB1, 0xF, 0xF, false)));   // quad [1,0,3,2]
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x4E, 0xF, 0xF, false)));   // quad [2,3,0,1]
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x141, 0xF, 0xF, false)));  // half mirror
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x140, 0xF, 0xF, false)));  // row mirror
  const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return max(max(a, b), max(c, d));
}

// Exact top-k of one token's logits by one full wavefront (lane holds
// experts lane, lane+64, lane+128, lane+192). `row` may live in global
// memory or LDS. The order is (selection key desc by the f32 total order,
// id asc); the k-th best is found by a bit-serial search with ballot counts
// and the selected k are ranked against each other. Lanes 0..k-1 store the
// results at their ranks; every lane also gets the selected ids in rank
// order in `sel_id` (wave-uniform).
// PER: candidates per lane (E <= 64 PER).
template <int PER>
__device__ __forceinline__ void topk_row_wave_p(const float* row, const float* __restrict__ bias,
                                                int E, int k, int score_fn, int norm, float scale,
                                                int t, uint32_t* __restrict__ ids,
                                                float* __restrict__ weights,
                                                uint32_t* __restrict__ token_idx,
                                                uint32_t (&sel_id)[kMaxTopK]) {
  static_assert(PER >= 1 && PER * kWave <= kMaxExperts, "candidates per lane");
  const int lane = threadIdx.x & 63;
  float lg[PER], score[PER];
  uint32_t key[PER];
  bool live[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + j * kWave;
    lg[j] = e < E ? row[e] : -INFINITY;
  }
  float lmax = 0.f, denom_all = 0.f;
  if (score_fn == INFERNO_SCORE_SOFTMAX) {
    float m = lg[0];
#pragma unroll
    for (int j = 1; j < PER; ++j) m = fmaxf(m, lg[j]);
    lmax = wave_max(m);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + j * kWave;
    float s, sel;
    if (score_fn == INFERNO_SCORE_SIGMOID) {
      s = 1.0f / (1.0f + expf(-lg[j]));
      sel = s;
    } else {
      s = e < E ? expf(lg[j] - lmax) : 0.f;
      sel = lg[j];
    }
    score[j] = s;
    const float bv = bias != nullptr ? bias[min(e, E - 1)] : 0.0f;  // clamped, unconditional
    const float corrected = sel + (e < E ? bv : 0.0f);
    key[j] = total_order_key(corrected);
    live[j] = e < E;
  }
  if (score_fn == INFERNO_SCORE_SOFTMAX && !norm) {
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < PER; ++j) part += score[j];
    denom_all = wave_sum(part);
  }
  // Selection without k dependent rounds. Every candidate gets a distinct
  // 41-bit rank key: live bit 40 | selection key << 8 | (255 - id), so a
  // larger value is a better (key desc, id asc) candidate. A bit-serial
  // search finds the k-th largest value: for each bit from the top, keep it
  // set if at least k candidates are at or above the prefix so far (ballot
  // counts). The candidates at or above it are exactly the top k.
  uint64_t rk[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t e = uint32_t(lane + j * kWave);
    rk[j] = live[j] ? ((uint64_t(1) << 40) | (uint64_t(key[j]) << 8) | uint64_t(255u - (e & 255u)))
                    : 0;
  }
  uint64_t kth = uint64_t(1) << 40;  // at least k candidates are live (k <= E)
  for (int bit = 39; bit >= 0; --bit) {
    const uint64_t cand = kth | (uint64_t(1) << bit);
    uint32_t cnt = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) cnt += uint32_t(__popcll(__ballot(rk[j] >= cand)));
    if (cnt >= uint32_t(k)) {
      kth = cand;
      if (cnt == uint32_t(k)) break;  // exactly the k winners are at or above kth
    }
  }
  // the selected candidates, gathered in lane order into lanes 0..k-1
  // (source lanes are wavefront-uniform: readlane, no LDS round trips)
  auto rd32 = [](uint32_t v, int src) {
    return uint32_t(__builtin_amdgcn_readlane(int(v), src));
  };
  uint64_t my_rk = 0;
  uint32_t my_id = 0xffffffffu;
  float my_score = 0.f;
  {
    int n = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      uint64_t m = __ballot(rk[j] >= kth);
      while (m) {
        const int src = __builtin_ctzll(m);
        m &= m - 1;
        const uint64_t r = (uint64_t(rd32(uint32_t(rk[j] >> 32), src)) << 32) |
                           rd32(uint32_t(rk[j]), src);
        const float sc = __uint_as_float(rd32(__float_as_uint(score[j]), src));
        if (lane == n) {
          my_rk = r;
          my_id = uint32_t(src + j * kWave);
          my_score = sc;
        }
        ++n;
      }
    }
  }
  // rank of each selected candidate among the k (0 = best)
  uint32_t rank = 0;
  for (int i = 0; i < k; ++i) {
    const uint64_t o = (uint64_t(rd32(uint32_t(my_rk >> 32), i)) << 32) | rd32(uint32_t(my_rk), i);
    rank += o > my_rk ? 1u : 0u;
  }
  const bool mine = lane < k;
  // rank order: ids for the callers, scores summed in rank order
  float sum = 0.f;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    sel_id[r] = 0xffffffffu;
    if (r < k) {
      const uint64_t at = __ballot(mine && rank == uint32_t(r));
      const int src = __builtin_ctzll(at);
      sel_id[r] = rd32(my_id, src);
      if (norm) sum += __uint_as_float(rd32(__float_as_uint(my_score), src));
    }
  }
  if (!norm && score_fn == INFERNO_SCORE_SOFTMAX) sum = denom_all;
  const bool divide = (norm || score_fn == INFERNO_SCORE_SOFTMAX) && sum > 0.f && isfinite(sum);
  if (mine) {
    float wv = my_score;
    if (divide) wv /= sum;
    const size_t a = size_t(t) * k + rank;
    ids[a] = my_id;
    weights[a] = wv * scale;
    if (token_idx) token_idx[a] = uint32_t(t);
  }
}

// One candidate per lane for routers of at most 64 experts (one ballot per
// search step instead of four), else four.
__device__ __forceinline__ void topk_row_wave(const float* row, const float* __restrict__ bias,
                                              int E, int k, int score_fn, int norm, float scale,
                                              int t, uint32_t* __restrict__ ids,
                                              float* __restrict__ weights,
                                              uint32_t* __restrict__ token_idx,
                                              uint32_t (&sel_id)[kMaxTopK]) {
  if (E <= kWave)
    topk_row_wave_p<1>(row, bias, E, k, score_fn, norm, scale, t, ids, weights, token_idx, sel_id);
  else
    topk_row_wave_p<kMaxExperts / kWave>(row, bias, E, k, score_fn, norm, scale, t, ids, weights,
                                         token_idx, sel_id);
}


// LDS scratch of topk1_wave.
struct Top1Lds {
  uint64_t rk[kMaxTopK];    // selected rank keys, ascending expert id
  uint32_t id[kMaxTopK];    // selected ids, ascending
  float sc[kMaxTopK];       // their scores
  uint32_t rank[kMaxTopK];  // rank of id-ordered entry j
  uint32_t rid[kMaxTopK];   // ids in rank order
  float w[kMaxTopK];        // routing weights in rank order
};

// Exact top-k of one token by one full wavefront, the semantics of
// topk_row_wave with a shorter dependency chain: lane holds the logits of
// experts lane + 64 j in lg[j] (anything for e >= E). The k-th largest
// selection key K is found bit by bit on 32-bit compares; every key above
// K wins, and of the keys equal to K the lowest ids fill the remaining
// places. The k winners are
// compacted into LDS in expert-id order with ballot prefix counts, and each
// winner's rank comes from comparing it with the k compacted (key, id)
// pairs. On return (after a wave barrier) s holds the winners in id order
// with their ranks, and ids and weights in rank order; weights are
// renormalised by the rank-order sum of the scores (as topk_row_wave).
// PER: the slots lg[j], j < PER, that can hold an expert (E <= 64 PER).
template <int PER>
__device__ __forceinline__ void topk1_wave_p(const float (&lgin)[4], const float (&bs)[4], int E,
                                             int k, int score_fn, int norm, float scale,
                                             Top1Lds* __restrict__ s) {
  static_assert(PER >= 1 && PER * kWave <= kMaxExperts, "slots per lane");
  const int lane = threadIdx.x & 63;
  float score[PER];
  uint32_t key[PER];
  bool live[PER];
  float lmax = 0.f;
  if (score_fn == INFERNO_SCORE_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) m = fmaxf(m, lane + j * kWave < E ? lgin[j] : -INFINITY);
    lmax = wave_max(m);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + j * kWave;
    live[j] = e < E;
    const float l = live[j] ? lgin[j] : -INFINITY;
    float sv, sel;
    if (score_fn == INFERNO_SCORE_SIGMOID) {
      sv = 1.0f / (1.0f + expf(-l));
      sel = sv;
    } else {
      sv = live[j] ? expf(l - lmax) : 0.f;
      sel = l;
    }
    score[j] = sv;
    // dead candidates get key 0, the lowest; they also have the highest ids,
    // so a live key of 0 still goes first
    key[j] = live[j] ? total_order_key(sel + bs[j]) : 0u;
  }
  float denom_all = 0.f;
  if (score_fn == INFERNO_SCORE_SOFTMAX && !norm) {
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < PER; ++j) part += score[j];
    denom_all = wave_sum(part);
  }
  // K: the largest value with at least k keys at or above it, one bit per
  // step from the top (four ballot counts each; measured faster than two
  // bits per step, whose extra compares each cost a VALU -> SGPR round trip)
  // The search stops as soon as exactly k keys are at or above the prefix
  // found so far: those k are the winners whatever the remaining bits of K
  // (with distinct-ish keys that is after ~log2(E) + a few steps, not 32);
  // kth is then a lower bound of K that no loser reaches, which the winner
  // rule below handles as it does K itself.
  uint32_t kth = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t c = kth | (1u << b);
    uint32_t n = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) n += uint32_t(__popcll(__ballot(key[j] >= c)));
    if (n >= uint32_t(k)) {
      kth = c;
      if (n == uint32_t(k)) break;  // uniform
    }
  }
  // winners: keys above K, then the lowest ids among keys equal to K
  uint32_t above = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) above += uint32_t(__popcll(__ballot(key[j] > kth)));
  uint32_t rem = uint32_t(k) - above;
  bool win[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const bool eq = key[j] == kth;
    const uint64_t em = __ballot(eq);
    const uint32_t before = __builtin_amdgcn_mbcnt_hi(uint32_t(em >> 32),
                                                      __builtin_amdgcn_mbcnt_lo(uint32_t(em), 0u));
    win[j] = key[j] > kth || (eq && before < rem);
    const uint32_t ne = uint32_t(__popcll(em));
    rem = rem > ne ? rem - ne : 0u;
  }
  // compact the k winners in expert-id order (j major, then lane); rank key
  // (key << 8 | 255 - id): larger is better
  uint32_t base = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint64_t m = __ballot(win[j]);
    if (win[j]) {
      const uint32_t e = uint32_t(lane + j * kWave);
      const uint32_t pos = base + uint32_t(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32),
                                                  __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u)));
      s->rk[pos] = (uint64_t(key[j]) << 8) | uint64_t(255u - (e & 255u));
      s->id[pos] = e;
      s->sc[pos] = score[j];
    }
    base += uint32_t(__popcll(m));
  }
  __builtin_amdgcn_wave_barrier();  // LDS is in order within a wavefront
  uint32_t my_rank = 0;
  if (lane < k) {
    const uint64_t mine = s->rk[lane];
    for (int i = 0; i < k; ++i) my_rank += s->rk[i] > mine ? 1u : 0u;
    s->rank[lane] = my_rank;
    s->rid[my_rank] = s->id[lane];
    s->w[my_rank] = s->sc[lane];
  }
  __builtin_amdgcn_wave_barrier();
  float sum = 0.f;
  if (norm)
    for (int r = 0; r < k; ++r) sum += s->w[r];  // rank order, every lane
  if (!norm && score_fn == INFERNO_SCORE_SOFTMAX) sum = denom_all;
  const bool divide = (norm || score_fn == INFERNO_SCORE_SOFTMAX) && sum > 0.f && isfinite(sum);
  if (lane < k) {
    float wv = s->w[lane];
    if (divide) wv /= sum;
    s->w[lane] = wv * scale;
  }
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ void topk1_wave(const float (&lgin)[4], const float (&bs)[4], int E,
                                           int k, int score_fn, int norm, float scale,
                                           Top1Lds* __restrict__ s) {
  topk1_wave_p<kMaxExperts / kWave>(lgin, bs, E, k, score_fn, norm, scale, s);
}

// The same with one slot per lane when the router has at most 64 experts
// (one ballot per search step instead of four: c1 20.0 -> 19.0 us per
// token). Only the run kernels' prologue takes it: in the fp8 x fp4
// gate/up kernel the second instantiation cost c2 +1.2 us.
__device__ __forceinline__ void topk1_wave_narrow(const float (&lgin)[4], const float (&bs)[4],
                                                  int E, int k, int score_fn, int norm,
                                                  float scale, Top1Lds* __restrict__ s) {
  if (E <= kWave)
    topk1_wave_p<1>(lgin, bs, E, k, score_fn, norm, scale, s);
  else
    topk1_wave_p<kMaxExperts / kWave>(lgin, bs, E, k, score_fn, norm, scale, s);
}

constexpr int kDispatchThreads = 1024;
constexpr int kDispatchWaves = kDispatchThreads / kWave;


// Lanes of this wavefront holding the same expert as this lane (ok lanes
// only): one ballot per expert-id bit.
__device__ __forceinline__ uint64_t expert_match(uint32_t e, bool ok, int nbits) {
  uint64_t match = __ballot(ok);
  for (int bit = 0; bit < nbits; ++bit) {
    const uint64_t b = __ballot(ok && ((e >> bit) & 1u));
    match &= ((e >> bit) & 1u) ? b : ~b;
  }
  return match;
}

__device__ __forceinline__ int expert_bits(int E) {
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  return nbits;
}

// Tiles of one expert with n rows: full 128-row tiles, then the remainder r
// as one 128-row (r > 64), 64-row (r > 32) or 32-row tile. The
// dequantisation cost of a tile does not depend on its row count, the MFMA
// cost does: small remainders take the cheaper narrow tiles.
struct TileCounts {
  uint32_t t128, t64, t32;
};
__device__ __forceinline__ TileCounts tile_counts(uint32_t n) {
  const uint32_t r = n % 128;
  TileCounts t{n / 128, 0, 0};
  if (r > 64) t.t128 += 1;
  else if (r > 32) t.t64 = 1;
  else if (r > 0) t.t32 = 1;
  return t;
}

// Exclusive scan of count[0..E) on wavefront 0 (each lane owns four
// consecutive experts, E <= 256) into cursor[]; when `write`, also the
// expert offsets (offsets[E] = total) and the compacted active list
// (active[0] = number of experts with assignments), and with plan.l128 set
// the tile lists (experts in id order, tile counts scanned the same way).
__device__ __forceinline__ void dispatch_scan(const uint32_t* count, int E, uint32_t* cursor,
                                              bool write, uint32_t* __restrict__ offsets,
                                              uint32_t* __restrict__ active,
                                              PlanOut plan = PlanOut{}) {
  const int lane = threadIdx.x & 63;
  uint32_t c4[4], f4[4], cs = 0, fs = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * lane + j;
    c4[j] = e < E ? count[e] : 0u;
    f4[j] = c4[j] > 0 ? 1u : 0u;
    cs += c4[j];
    fs += f4[j];
  }
  uint32_t ci = cs, fi = fs;  // inclusive wave scans
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t cu = __shfl_up(ci, o, kWave), fu = __shfl_up(fi, o, kWave);
    if (lane >= o) {
      ci += cu;
      fi += fu;
    }
  }
  uint32_t cex = ci - cs, fex = fi - fs;
  const uint32_t c_first = cex;  // offset of this lane's first expert
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * lane + j;
    if (e < E) {
      cursor[e] = cex;
      if (write) {
        offsets[e] = cex;
        if (c4[j] > 0) active[1 + fex] = uint32_t(e);
      }
    }
    cex += c4[j];
    fex += f4[j];
  }
  if (write && lane == 63) {
    offsets[E] = ci;
    active[0] = fi;
  }
  if (!write || plan.l128 == nullptr) return;  // uniform
  TileCounts t4[4];
  uint32_t s128 = 0, s64 = 0, s32 = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    t4[j] = tile_counts(c4[j]);  // zero for e >= E (c4 is zero there)
    s128 += t4[j].t128;
    s64 += t4[j].t64;
    s32 += t4[j].t32;
  }
  uint32_t i128 = s128, i64 = s64, i32 = s32;  // inclusive wave scans
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t a = __shfl_up(i128, o, kWave), b = __shfl_up(i64, o, kWave),
                   c = __shfl_up(i32, o, kWave);
    if (lane >= o) {
      i128 += a;
      i64 += b;
      i32 += c;
    }
  }
  uint32_t o128 = i128 - s128, o64 = i64 - s64, o32 = i32 - s32, lo = c_first;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t e = uint32_t(4 * lane + j), hi = lo + c4[j];
    for (uint32_t q = 0; q < t4[j].t128; ++q)
      plan.l128[o128 + q] = make_uint4(e, lo + 128 * q, min(hi, lo + 128 * (q + 1)), 0);
    if (t4[j].t64) plan.l64[o64] = make_uint4(e, lo + 128 * t4[j].t128, hi, 0);
    if (t4[j].t32) plan.l32[o32] = make_uint4(e, lo + 128 * t4[j].t128, hi, 0);
    o128 += t4[j].t128;
    o64 += t4[j].t64;
    o32 += t4[j].t32;
    lo = hi;
  }
  if (lane == 63) {
    plan.counts[0] = i128;
    plan.counts[1] = i64;
    plan.counts[2] = i32;
  }
}

// Stable scatter of assignments [a_begin, a_end) (a_begin a multiple of
// 1024) to sorted[cursor[e]++]: inside a wavefront the rank among earlier
// lanes with the same expert comes from the match mask; wavefront counts per
// expert are prefix-summed across the 16 wavefronts through LDS. 1024-thread
// workgroup; ends with a barrier.
__device__ __forceinline__ void dispatch_scatter(const uint32_t* ids, int a_begin, int a_end, int E,
                                                 uint32_t* cursor, uint32_t* wcount,
                                                 uint32_t* __restrict__ sorted) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nbits = expert_bits(E);
  for (int base = a_begin; base < a_end; base += kDispatchThreads) {
    const int a = base + tid;
    const bool valid = a < a_end;
    const uint32_t e = valid ? ids[a] : 0xffffffffu;
    const bool ok = valid && e < uint32_t(E);
    const uint64_t match = expert_match(e, ok, nbits);
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const uint32_t rank = uint32_t(__popcll(match & lt));
    const bool leader = ok && (match & lt) == 0ull;
    // per-wave per-expert counts, written by each match group's first lane
    for (int i = tid; i < kDispatchWaves * E; i += kDispatchThreads) wcount[i] = 0u;
    __syncthreads();
    if (leader) wcount[wave * E + int(e)] = uint32_t(__popcll(match));
    __syncthreads();
    if (ok) {
      uint32_t before = 0;
      for (int w = 0; w < wave; ++w) before += wcount[w * E + int(e)];
      sorted[cursor[e] + before + rank] = uint32_t(a);
    }
    __syncthreads();
    for (int ex = tid; ex < E; ex += kDispatchThreads) {
      uint32_t tot = 0;
      for (int w = 0; w < kDispatchWaves; ++w) tot += wcount[w * E + ex];
      cursor[ex] += tot;
    }
    __syncthreads();
  }
}

// Body of the dispatch: must run on a 1024-thread workgroup; `ids` may
// live in global memory or LDS.
__device__ __forceinline__ void dispatch_block(const uint32_t* ids, int A, int E,
                                               uint32_t* __restrict__ offsets,
                                               uint32_t* __restrict__ sorted,
                                               uint32_t* __restrict__ active,
                                               PlanOut plan = PlanOut{}) {
  __shared__ uint32_t count[kMaxExperts];
  __shared__ uint32_t cursor[kMaxExperts];
  __shared__ uint32_t wcount[kDispatchWaves * kMaxExperts];  // [wave][expert], row stride E
  const int tid = threadIdx.x, wave = tid >> 6;
  for (int e = tid; e < E; e += kDispatchThreads) count[e] = 0;
  __syncthreads();
  for (int a = tid; a < A; a += kDispatchThreads) {
    uint32_t e = ids[a];
    if (e < uint32_t(E)) atomicAdd(&count[e], 1u);
  }
  __syncthreads();
  if (wave == 0) dispatch_scan(count, E, cursor, true, offsets, active, plan);
  __syncthreads();
  dispatch_scatter(ids, 0, A, E, cursor, wcount, sorted);
}


}  // namespace inferno
