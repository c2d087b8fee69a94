// CPU oracle — test infrastructure only (see oracle.h for the scope rule and
// the reference citations). Compiled with -ffp-contract=off so every fp32
// expression rounds exactly as written, like the reference's Rust.
#include "oracle.h"

#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

constexpr size_t kKBlock = 256;

// Splits [0, n) over up to `threads` workers; runs fn(begin, end) on each.
template <typename Fn>
void parallel_for(size_t n, int threads, Fn fn) {
  if (threads <= 1 || n < 2) {
    fn(size_t(0), n);
    return;
  }
  size_t workers = std::min<size_t>(size_t(threads), n);
  std::vector<std::thread> pool;
  pool.reserve(workers);
  for (size_t w = 0; w < workers; ++w) {
    size_t b = n * w / workers, e = n * (w + 1) / workers;
    pool.emplace_back([=] { fn(b, e); });
  }
  for (auto& t : pool) t.join();
}

inline uint16_t le16(const uint8_t* p) { return uint16_t(p[0]) | (uint16_t(p[1]) << 8); }

// Q2_K: crates/gguf/src/lib.rs:1226-1293.
// Layout [scales 16 | qs 64 | d f16 | dmin f16]; value = (d*(sc&15))*q - dmin*(sc>>4).
int dq_q2_k(const uint8_t* b, float* out) {
  const uint8_t* scales = b;
  const uint8_t* qs = b + 16;
  float d = oracle_f16_to_f32(le16(b + 80));
  float mn = oracle_f16_to_f32(le16(b + 82));
  if (!std::isfinite(d) || !std::isfinite(mn)) return -2;
  int si = 0, qo = 0, oo = 0;
  while (oo < 256) {
    int shift = 0;
    for (int p = 0; p < 4; ++p) {
      for (int half = 0; half < 2; ++half) {
        uint8_t sm = scales[si++];
        float scale = d * float(sm & 0x0f);
        float min_off = mn * float(sm >> 4);
        for (int i = 0; i < 16; ++i)
          out[oo + i] = scale * float((qs[qo + 16 * half + i] >> shift) & 3) - min_off;
        oo += 16;
      }
      shift += 2;
    }
    qo += 32;
  }
  return 0;
}

// Q3_K: crates/gguf/src/lib.rs:1295-1367.
// Layout [hmask 32 | qs 64 | scales 12 | d f16].
int dq_q3_k(const uint8_t* b, float* out) {
  const uint8_t* hm = b;
  const uint8_t* qs = b + 32;
  const uint8_t* sc = b + 96;
  float d = oracle_f16_to_f32(le16(b + 108));
  if (!std::isfinite(d)) return -2;
  for (int g = 0; g < 16; ++g) {
    int qoff = 32 * (g / 8) + 16 * (g & 1);
    int hoff = 16 * (g & 1);
    uint8_t hbit = uint8_t(1u << (g / 2));
    static const uint16_t low_masks[4] = {0x03, 0x0c, 0x30, 0xc0};
    uint16_t lmask = low_masks[g / 4];
    uint16_t nmask = g < 8 ? 0x0f : 0xf0;
    uint16_t slow = sc[g % 8], shigh = sc[8 + g % 4];
    uint16_t packed = ((g / 4) & 1) ? uint16_t((slow & nmask) | ((shigh & lmask) << 2))
                                    : uint16_t((slow & nmask) | ((shigh & lmask) << 4));
    float gs = g < 8 ? d * (float(packed) - 32.0f) : d * (float(packed) / 16.0f - 32.0f);
    float neg = 4.0f * gs;
    int lane = (g / 2) & 3;
    int shift = 2 * lane;
    uint8_t qmask = uint8_t(3u << shift);
    float qscale = 1.0f / float(1u << shift);
    for (int i = 0; i < 16; ++i) {
      float low = float(qs[qoff + i] & qmask) * qscale;
      float sub = (hm[hoff + i] & hbit) == 0 ? neg : 0.0f;
      out[16 * g + i] = gs * low - sub;
    }
  }
  return 0;
}

// crates/gguf/src/lib.rs:1407-1416
inline void q4_scale_min(int g, const uint8_t* s, uint8_t* sc, uint8_t* m) {
  if (g < 4) {
    *sc = s[g] & 0x3f;
    *m = s[g + 4] & 0x3f;
  } else {
    *sc = uint8_t((s[g + 4] & 0x0f) | ((s[g - 4] >> 6) << 4));
    *m = uint8_t((s[g + 4] >> 4) | ((s[g] >> 6) << 4));
  }
}

// Q4_K: crates/gguf/src/lib.rs:1369-1405.
// Layout [d f16 | dmin f16 | scales 12 | qs 128]; value = (d*sc)*q - dmin*m.
int dq_q4_k(const uint8_t* b, float* out) {
  float d = oracle_f16_to_f32(le16(b));
  float dmin = oracle_f16_to_f32(le16(b + 2));
  if (!std::isfinite(d) || !std::isfinite(dmin)) return -2;
  const uint8_t* s = b + 4;
  const uint8_t* qs = b + 16;
  for (int g = 0; g < 8; ++g) {
    uint8_t sc, m;
    q4_scale_min(g, s, &sc, &m);
    int qoff = (g / 2) * 32, shift = (g & 1) * 4;
    for (int i = 0; i < 32; ++i) {
      uint8_t q = (qs[qoff + i] >> shift) & 0x0f;
      out[g * 32 + i] = d * float(sc) * float(q) - dmin * float(m);
    }
  }
  return 0;
}

// Q6_K: crates/gguf/src/lib.rs:1418-1470.
// Layout [ql 128 | qh 64 | scales int8 16 | d f16]; value = (d*sc)*(q-32).
int dq_q6_k(const uint8_t* b, float* out) {
  const uint8_t* ql = b;
  const uint8_t* qh = b + 128;
  const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192);
  float d = oracle_f16_to_f32(le16(b + 208));
  if (!std::isfinite(d)) return -2;
  for (int half = 0; half < 2; ++half) {
    for (int i = 0; i < 32; ++i) {
      int sl = i / 16;
      uint8_t l0 = ql[64 * half + i] & 0x0f, l1 = ql[64 * half + 32 + i] & 0x0f;
      uint8_t l2 = ql[64 * half + i] >> 4, l3 = ql[64 * half + 32 + i] >> 4;
      uint8_t h = qh[32 * half + i];
      uint8_t q[4] = {uint8_t(l0 | ((h & 3) << 4)), uint8_t(l1 | (((h >> 2) & 3) << 4)),
                      uint8_t(l2 | (((h >> 4) & 3) << 4)), uint8_t(l3 | (((h >> 6) & 3) << 4))};
      for (int quarter = 0; quarter < 4; ++quarter) {
        float s = float(sc[8 * half + sl + 2 * quarter]);
        out[128 * half + 32 * quarter + i] = d * s * (float(q[quarter]) - 32.0f);
      }
    }
  }
  return 0;
}

// Q8_0: crates/gguf/src/lib.rs:1472-1499. Layout [d f16 | int8 x32]; value = d*q.
int dq_q8_0(const uint8_t* b, float* out) {
  float d = oracle_f16_to_f32(le16(b));
  if (!std::isfinite(d)) return -2;
  for (int i = 0; i < 32; ++i) out[i] = d * float(int8_t(b[2 + i]));
  return 0;
}

int dq_block(int quant, const uint8_t* b, float* out) {
  switch (quant) {
    case ORC_Q2_K: return dq_q2_k(b, out);
    case ORC_Q3_K: return dq_q3_k(b, out);
    case ORC_Q4_K: return dq_q4_k(b, out);
    case ORC_Q6_K: return dq_q6_k(b, out);
    case ORC_Q8_0: return dq_q8_0(b, out);
  }
  return -1;
}

// One quantised row against x: per-block fp32 dot in value order, block dots
// summed sequentially (the shape of cpu_q2_matrix_vector,
// crates/backend/src/metal/gguf_moe.rs:756-799).
int row_dot(int quant, const uint8_t* row, size_t cols, const float* x, float* result) {
  const size_t bv = size_t(oracle_block_values(quant));
  const size_t bb = size_t(oracle_block_bytes(quant));
  float vals[256];
  float sum = 0.0f;
  for (size_t b = 0; b < cols / bv; ++b) {
    int st = dq_block(quant, row + b * bb, vals);
    if (st) return st;
    float bd = 0.0f;
    for (size_t v = 0; v < bv; ++v) bd += x[b * bv + v] * vals[v];
    sum += bd;
  }
  *result = sum;
  return 0;
}

// Dequantises one row (cols values) into out; the values row_dot uses.
int dq_row(int quant, const uint8_t* row, size_t cols, float* out) {
  const size_t bv = size_t(oracle_block_values(quant));
  const size_t bb = size_t(oracle_block_bytes(quant));
  for (size_t b = 0; b < cols / bv; ++b) {
    int st = dq_block(quant, row + b * bb, out + b * bv);
    if (st) return st;
  }
  return 0;
}

// row_dot over an already dequantised row: the same per-block then
// sequential summation order, so the same fp32 result.
float dot_dequantized(const float* vals, size_t cols, size_t bv, const float* x) {
  float sum = 0.0f;
  for (size_t b = 0; b < cols / bv; ++b) {
    float bd = 0.0f;
    for (size_t v = 0; v < bv; ++v) bd += x[b * bv + v] * vals[b * bv + v];
    sum += bd;
  }
  return sum;
}

// Activation rows interleaved eight at a time, [group][column][8] (lanes
// past the last row zero), so that one dequantised weight row is dotted with
// eight rows as eight independent summation chains that advance as a vector.
struct Panel {
  size_t n = 0, cols = 0;
  std::vector<float> data;
  template <typename RowAt>
  void build(size_t rows, size_t c, RowAt row_at) {
    n = rows;
    cols = c;
    data.assign(((rows + 7) / 8) * c * 8, 0.0f);
    for (size_t r = 0; r < rows; ++r) {
      const float* src = row_at(r);
      float* dst = data.data() + (r / 8) * c * 8 + (r % 8);
      for (size_t v = 0; v < c; ++v) dst[v * 8] = src[v];
    }
  }
};

// out[w * n + r] = dot_dequantized(row w of vals, row r of the panel) for
// nw dequantised weight rows (stride cols) and every panel row: each lane
// keeps dot_dequantized's order (per-block sums, then blocks in order); the
// eight lanes are one vector of independent fp32 operations (no
// contraction), two groups in flight for latency. Panel groups are the outer
// loop so they stay in cache across the rows.
typedef float F8 __attribute__((vector_size(32)));

inline F8 load8(const float* p) {
  F8 v;
  std::memcpy(&v, p, sizeof(v));
  return v;
}

__attribute__((target_clones("avx2", "default")))
void dot_panel(const float* vals, size_t nw, size_t bv, const Panel& p, float* out) {
  const size_t groups = (p.n + 7) / 8;
  for (size_t g = 0; g < groups; g += 2) {
    const bool two = g + 1 < groups;
    const float* x0 = p.data.data() + g * p.cols * 8;
    const float* x1 = two ? x0 + p.cols * 8 : x0;
    for (size_t w = 0; w < nw; ++w) {
      const float* wr = vals + w * p.cols;
      F8 s0 = {}, s1 = {};
      for (size_t b = 0; b < p.cols; b += bv) {
        F8 d0 = {}, d1 = {};
        for (size_t v = b; v < b + bv; ++v) {
          const float wv = wr[v];
          d0 += load8(x0 + v * 8) * wv;
          d1 += load8(x1 + v * 8) * wv;
        }
        s0 += d0;
        s1 += d1;
      }
      for (size_t j = 0; j < 8 && g * 8 + j < p.n; ++j) out[w * p.n + g * 8 + j] = s0[j];
      if (two)
        for (size_t j = 0; j < 8 && (g + 1) * 8 + j < p.n; ++j)
          out[w * p.n + (g + 1) * 8 + j] = s1[j];
    }
  }
}

inline float silu(float g) { return g / (1.0f + std::exp(-g)); }

// total_cmp ordering of crates/model/src/moe_router.rs:930-936: the float's
// bits mapped to an order-preserving integer.
inline int32_t total_key(float f) {
  int32_t b;
  std::memcpy(&b, &f, 4);
  return b ^ int32_t(uint32_t(b >> 31) >> 1);
}

struct Candidate {
  uint32_t id;
  float corrected;
  float score;
};

// crates/model/src/moe_router.rs:930-936
inline bool better(const Candidate& l, const Candidate& r) {
  int32_t a = total_key(l.corrected), b = total_key(r.corrected);
  if (a != b) return a > b;
  return l.id < r.id;
}

// crates/model/src/moe_router.rs:909-928
void insert_candidate(std::vector<Candidate>& top, size_t k, const Candidate& c) {
  if (k == 0) return;
  size_t at = top.size();
  for (size_t i = 0; i < top.size(); ++i)
    if (better(c, top[i])) {
      at = i;
      break;
    }
  if (at < k) {
    top.insert(top.begin() + long(at), c);
    if (top.size() > k) top.pop_back();
  }
}

}  // namespace

extern "C" {

// crates/gguf/src/lib.rs:1501-1528
float oracle_f16_to_f32(uint16_t bits) {
  uint32_t sign = uint32_t(bits & 0x8000) << 16;
  uint32_t exponent = (bits >> 10) & 0x1f;
  uint32_t fraction = bits & 0x03ff;
  uint32_t out;
  if (exponent == 0) {
    if (fraction == 0) {
      out = sign;
    } else {
      uint32_t mant = fraction;
      int32_t e = -14;
      while ((mant & 0x0400) == 0) {
        mant <<= 1;
        e -= 1;
      }
      mant &= 0x03ff;
      out = sign | (uint32_t(e + 127) << 23) | (mant << 13);
    }
  } else if (exponent == 0x1f) {
    out = sign | 0x7f800000u | (fraction << 13);
  } else {
    out = sign | ((exponent + 112) << 23) | (fraction << 13);
  }
  float f;
  std::memcpy(&f, &out, 4);
  return f;
}

// crates/gguf/src/lib.rs:21-27
int oracle_block_bytes(int quant) {
  switch (quant) {
    case ORC_Q2_K: return 84;
    case ORC_Q3_K: return 110;
    case ORC_Q4_K: return 144;
    case ORC_Q6_K: return 210;
    case ORC_Q8_0: return 34;
  }
  return -1;
}

int oracle_block_values(int quant) {
  if (quant == ORC_Q8_0) return 32;
  if (oracle_block_bytes(quant) < 0) return -1;
  return int(kKBlock);
}

int oracle_dequantize(int quant, const uint8_t* blocks, size_t n_blocks, float* out) {
  const int bb = oracle_block_bytes(quant), bv = oracle_block_values(quant);
  if (bb < 0) return -1;
  for (size_t i = 0; i < n_blocks; ++i) {
    int st = dq_block(quant, blocks + i * size_t(bb), out + i * size_t(bv));
    if (st) return st;
  }
  return 0;
}

int oracle_linear(const float* x, const float* w, size_t rows, size_t in_f, size_t out_f,
                  float* out, int threads) {
  parallel_for(rows * out_f, threads, [&](size_t b, size_t e) {
    for (size_t idx = b; idx < e; ++idx) {
      size_t r = idx / out_f, o = idx % out_f;
      float s = 0.0f;
      for (size_t h = 0; h < in_f; ++h) s += x[r * in_f + h] * w[o * in_f + h];
      out[idx] = s;
    }
  });
  return 0;
}

// Sigmoid: crates/model/src/moe_router.rs:835-900 (select_topk_row).
// Softmax: closed form described in oracle.h.
int oracle_router_topk(const float* logits, const float* bias, size_t T, size_t E, size_t k,
                       int score_fn, int norm, float scale, uint32_t* ids, float* weights) {
  if (E == 0 || k == 0 || k > E) return -1;
  if (score_fn != ORC_SCORE_SIGMOID && score_fn != ORC_SCORE_SOFTMAX) return -1;
  std::vector<Candidate> top;
  std::vector<float> p(E);
  for (size_t t = 0; t < T; ++t) {
    const float* row = logits + t * E;
    top.clear();
    float lmax = -INFINITY;
    if (score_fn == ORC_SCORE_SOFTMAX) {
      for (size_t e = 0; e < E; ++e) lmax = std::fmax(lmax, row[e]);
      for (size_t e = 0; e < E; ++e) p[e] = std::exp(row[e] - lmax);
    }
    for (size_t e = 0; e < E; ++e) {
      float score = score_fn == ORC_SCORE_SIGMOID ? 1.0f / (1.0f + std::exp(-row[e])) : p[e];
      float sel = score_fn == ORC_SCORE_SIGMOID ? score : row[e];
      float corrected = sel + (bias ? bias[e] : 0.0f);
      insert_candidate(top, k, Candidate{uint32_t(e), corrected, score});
    }
    float w[64];
    for (size_t r = 0; r < k; ++r) {
      w[r] = top[r].score;
      if (!std::isfinite(w[r]) || w[r] < 0.0f) return -3;
    }
    if (norm) {
      float sum = 0.0f;
      for (size_t r = 0; r < k; ++r) sum += w[r];
      if (!std::isfinite(sum) || sum <= 0.0f) return -3;
      for (size_t r = 0; r < k; ++r) w[r] /= sum;
    } else if (score_fn == ORC_SCORE_SOFTMAX) {
      float sum = 0.0f;
      for (size_t e = 0; e < E; ++e) sum += p[e];
      for (size_t r = 0; r < k; ++r) w[r] /= sum;
    }
    for (size_t r = 0; r < k; ++r) {
      ids[t * k + r] = top[r].id;
      weights[t * k + r] = w[r] * scale;
    }
  }
  return 0;
}

// crates/moe/src/routing.rs:27-85 — expert-major, token order then rank order.
int oracle_dispatch(const uint32_t* ids, size_t T, size_t k, size_t E, uint32_t* offsets,
                    uint32_t* sorted) {
  if (E == 0) return -1;
  std::vector<uint32_t> count(E + 1, 0);
  for (size_t a = 0; a < T * k; ++a) {
    if (ids[a] >= E) return -1;
    count[ids[a]]++;
  }
  offsets[0] = 0;
  for (size_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + count[e];
  std::vector<uint32_t> cursor(offsets, offsets + E);
  for (size_t a = 0; a < T * k; ++a) sorted[cursor[ids[a]]++] = uint32_t(a);
  return 0;
}

int oracle_qmatvec(int quant, const uint8_t* w, size_t rows, size_t cols, const float* x,
                   float* y) {
  const int bv = oracle_block_values(quant), bb = oracle_block_bytes(quant);
  if (bv < 0 || cols % size_t(bv)) return -1;
  const size_t row_bytes = cols / size_t(bv) * size_t(bb);
  for (size_t r = 0; r < rows; ++r) {
    int st = row_dot(quant, w + r * row_bytes, cols, x, &y[r]);
    if (st) return st;
  }
  return 0;
}

int oracle_moe_routed(int quant, int down_quant, const uint8_t* gate, const uint8_t* up,
                      const uint8_t* down, const float* x, size_t T, size_t H, size_t I,
                      size_t E, size_t k, const uint32_t* ids, const float* weights, float* y,
                      int threads) {
  const int gbb = oracle_block_bytes(quant), dbb = oracle_block_bytes(down_quant);
  if (gbb < 0 || dbb < 0 || H % kKBlock || I % kKBlock) return -1;
  for (size_t a = 0; a < T * k; ++a)
    if (ids[a] >= E) return -1;
  const size_t grow = H / kKBlock * size_t(gbb), drow = I / kKBlock * size_t(dbb);
  const size_t gbv = size_t(oracle_block_values(quant)), dbv = size_t(oracle_block_values(down_quant));
  const size_t A = T * k;
  // assignments of each expert (any order: every (assignment, row) value is
  // computed on its own); each expert row is dequantised once and dotted with
  // the activations of all the expert's assignments
  std::vector<std::vector<uint32_t>> of(E);
  for (size_t a = 0; a < A; ++a) of[ids[a]].push_back(uint32_t(a));
  std::vector<uint32_t> used;
  for (size_t e = 0; e < E; ++e)
    if (!of[e].empty()) used.push_back(uint32_t(e));
  std::vector<float> h(A * I);
  constexpr size_t kRowsPerItem = 16;
  const size_t gate_items = (I + kRowsPerItem - 1) / kRowsPerItem;
  std::vector<int> status(std::max<size_t>(used.size() * gate_items, H), 0);
  // gate/up + SwiGLU * routing weight: gguf_moe_kernels.metal:340-400
  parallel_for(used.size() * gate_items, threads, [&](size_t b, size_t e) {
    std::vector<float> gv(kRowsPerItem * H), uv(kRowsPerItem * H), gs(kRowsPerItem * A),
        us(kRowsPerItem * A);
    Panel xp;
    size_t panel_ex = size_t(-1);
    for (size_t item = b; item < e; ++item) {
      const size_t ex = used[item / gate_items];
      const std::vector<uint32_t>& as = of[ex];
      if (ex != panel_ex) {
        xp.build(as.size(), H, [&](size_t j) { return x + (as[j] / k) * H; });
        panel_ex = ex;
      }
      const size_t i0 = (item % gate_items) * kRowsPerItem;
      const size_t nr = std::min(I, i0 + kRowsPerItem) - i0;
      int st = 0;
      for (size_t r = 0; r < nr && !st; ++r) {
        st = dq_row(quant, gate + (ex * I + i0 + r) * grow, H, gv.data() + r * H);
        if (!st) st = dq_row(quant, up + (ex * I + i0 + r) * grow, H, uv.data() + r * H);
      }
      if (st) {
        status[item] = st;
        continue;
      }
      dot_panel(gv.data(), nr, gbv, xp, gs.data());
      dot_panel(uv.data(), nr, gbv, xp, us.data());
      const size_t n = as.size();
      for (size_t r = 0; r < nr; ++r)
        for (size_t j = 0; j < n; ++j)
          h[size_t(as[j]) * I + i0 + r] = silu(gs[r * n + j]) * us[r * n + j] * weights[as[j]];
    }
  });
  for (size_t i = 0; i < status.size(); ++i)
    if (status[i]) return status[i];
  // down, summed over ranks in rank order: gguf_moe_kernels.metal:457-510
  const size_t down_items = (H + kRowsPerItem - 1) / kRowsPerItem;
  std::vector<Panel> hps(E);
  parallel_for(used.size(), threads, [&](size_t b, size_t e) {
    for (size_t u = b; u < e; ++u) {
      const std::vector<uint32_t>& as = of[used[u]];
      hps[used[u]].build(as.size(), I, [&](size_t j) { return h.data() + size_t(as[j]) * I; });
    }
  });
  parallel_for(down_items, threads, [&](size_t b, size_t e) {
    std::vector<float> dv(kRowsPerItem * I), v(kRowsPerItem * A), r(kRowsPerItem * A);
    for (size_t item = b; item < e; ++item) {
      const size_t o0 = item * kRowsPerItem, nr = std::min(H, o0 + kRowsPerItem) - o0;
      for (uint32_t ex : used) {
        const std::vector<uint32_t>& as = of[ex];
        int st = 0;
        for (size_t q = 0; q < nr && !st; ++q)
          st = dq_row(down_quant, down + (ex * H + o0 + q) * drow, I, dv.data() + q * I);
        if (st) {
          status[item] = st;
          break;
        }
        dot_panel(dv.data(), nr, dbv, hps[ex], r.data());
        const size_t n = as.size();
        for (size_t q = 0; q < nr; ++q)
          for (size_t j = 0; j < n; ++j) v[q * A + as[j]] = r[q * n + j];
      }
      if (status[item]) continue;
      for (size_t q = 0; q < nr; ++q)
        for (size_t t = 0; t < T; ++t) {
          float acc = 0.0f;
          for (size_t rk = 0; rk < k; ++rk) acc += v[q * A + t * k + rk];
          y[t * H + o0 + q] = acc;
        }
    }
  });
  for (size_t i = 0; i < status.size(); ++i)
    if (status[i]) return status[i];
  return 0;
}

int oracle_shared_ffn(int quant, int down_quant, const uint8_t* gate, const uint8_t* up,
                      const uint8_t* down, const float* x, size_t T, size_t H, size_t Is,
                      const float* routed, const float* residual, float* out, int threads) {
  const int gbv = oracle_block_values(quant), dbv = oracle_block_values(down_quant);
  if (gbv < 0 || dbv < 0 || H % size_t(gbv) || Is % size_t(dbv)) return -1;
  const size_t grow = H / size_t(gbv) * size_t(oracle_block_bytes(quant));
  const size_t drow = Is / size_t(dbv) * size_t(oracle_block_bytes(down_quant));
  std::vector<float> hs(T * Is);
  std::vector<int> status(std::max(Is, H), 0);
  // q2_kernels.metal:2133-2235 (Q8_0 gate/up SwiGLU, no routing weight;
  // Laguna XS: Q4_K gate/up, laguna_xs_kernels.metal:1922-1926); each
  // weight row dequantised once and dotted with every token
  Panel xp;
  xp.build(T, H, [&](size_t t) { return x + t * H; });
  parallel_for(Is, threads, [&](size_t b, size_t e) {
    std::vector<float> gv(H), uv(H), gs(T), us(T);
    for (size_t i = b; i < e; ++i) {
      int st = dq_row(quant, gate + i * grow, H, gv.data());
      if (!st) st = dq_row(quant, up + i * grow, H, uv.data());
      if (st) {
        status[i] = st;
        continue;
      }
      dot_panel(gv.data(), 1, size_t(gbv), xp, gs.data());
      dot_panel(uv.data(), 1, size_t(gbv), xp, us.data());
      for (size_t t = 0; t < T; ++t) hs[t * Is + i] = silu(gs[t]) * us[t];
    }
  });
  for (size_t i = 0; i < Is; ++i)
    if (status[i]) return status[i];
  // q2_kernels.metal:2066-2131: residual_a + residual_b + value
  Panel hp;
  hp.build(T, Is, [&](size_t t) { return hs.data() + t * Is; });
  parallel_for(H, threads, [&](size_t b, size_t e) {
    std::vector<float> dv(Is), r(T);
    for (size_t o = b; o < e; ++o) {
      int st = dq_row(down_quant, down + o * drow, Is, dv.data());
      if (st) {
        status[o] = st;
        continue;
      }
      dot_panel(dv.data(), 1, size_t(dbv), hp, r.data());
      for (size_t t = 0; t < T; ++t) {
        const size_t idx = t * H + o;
        float ra = routed ? routed[idx] : 0.0f, rb = residual ? residual[idx] : 0.0f;
        out[idx] = ra + rb + r[t];
      }
    }
  });
  for (size_t i = 0; i < H; ++i)
    if (status[i]) return status[i];
  return 0;
}

int oracle_shared_q8_0(const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                       const float* x, size_t T, size_t H, size_t Is, const float* routed,
                       const float* residual, float* out, int threads) {
  return oracle_shared_ffn(ORC_Q8_0, ORC_Q8_0, gate, up, down, x, T, H, Is, routed, residual, out,
                           threads);
}

// crates/backend/src/backend.rs:10298-10352 (expert-major assignment order)
int oracle_weighted_index_add_combine(const float* acc, const uint32_t* token_idx,
                                      const float* expert_out, const float* expert_w,
                                      size_t T, size_t H, size_t A, float* out) {
  std::memcpy(out, acc, T * H * sizeof(float));
  for (size_t a = 0; a < A; ++a) {
    if (token_idx[a] >= T) return -1;
    for (size_t h = 0; h < H; ++h)
      out[token_idx[a] * H + h] += expert_out[a * H + h] * expert_w[a];
  }
  return 0;
}

// crates/backend/src/backend.rs:10211-10257
int oracle_rms_norm(const float* x, const float* w, size_t rows, size_t H, float eps,
                    float* out) {
  for (size_t r = 0; r < rows; ++r) {
    const float* row = x + r * H;
    float ss = 0.0f;
    for (size_t i = 0; i < H; ++i) {
      float sq = row[i] * row[i];
      if (!std::isfinite(sq)) return -3;
      ss += sq;
    }
    float mean = ss / float(H);
    float scale = std::sqrt(mean + eps);
    if (!std::isfinite(scale) || scale <= 0.0f) return -3;
    for (size_t i = 0; i < H; ++i) out[r * H + i] = row[i] / scale * w[i];
  }
  return 0;
}

}  // extern "C"
