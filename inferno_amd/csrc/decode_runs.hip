// Launchers of the f16-run matrix-core decode kernels (decode_runs.hpp):
// instances per format, super-block columns and register batch.
#include <cstdlib>

#include "decode.hpp"
#include "decode_runs.hpp"

namespace inferno {
namespace {

using namespace runs_decode;

constexpr size_t kLdsMax = 160 * 1024;

int cus_now() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) !=
                       hipSuccess)
    cus[dev] = 0;
  return cus[dev];
}

// Raises a kernel's dynamic LDS limit once per process.
template <typename K>
int allow_lds(K kern, bool& done) {
  if (!done) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, int(kLdsMax)) != hipSuccess) {
      set_error("runs decode kernel: cannot raise its LDS limit");
      return INFERNO_ERR_DEVICE;
    }
    done = true;
  }
  return INFERNO_OK;
}

template <int Q, int NB>
int gate_up_nb(hipStream_t s, const DecodeArgs& a) {
  static bool attr = false;
  auto* kern = gate_up_runs_kernel<Q, NB>;
  if (int st = allow_lds(kern, attr)) return st;
  const int ntiles = a.max_slots * (a.I / kRows);
  const unsigned grid = unsigned(std::min(ntiles, cus_now()));
  kern<<<grid, kThreads, gate_up_runs_lds<Q, NB>(), s>>>(a, ntiles);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int Q>
int gate_up_q(hipStream_t s, const DecodeArgs& a) {
  switch (a.H / kKBlock) {
    case 4: return gate_up_nb<Q, 4>(s, a);
    case 8: return gate_up_nb<Q, 8>(s, a);
    case 12: return gate_up_nb<Q, 12>(s, a);
    case 16: return gate_up_nb<Q, 16>(s, a);
    default: return gate_up_nb<Q, 24>(s, a);
  }
}

template <int Q>
size_t gate_up_lds_q(int NB) {
  switch (NB) {
    case 4: return gate_up_runs_lds<Q, 4>();
    case 8: return gate_up_runs_lds<Q, 8>();
    case 12: return gate_up_runs_lds<Q, 12>();
    case 16: return gate_up_runs_lds<Q, 16>();
    case 24: return gate_up_runs_lds<Q, 24>();
    default: return ~size_t(0);
  }
}

// Output rows per down tile: 16, or 8 when the k ranks' 16-row tiles and h
// rows do not fit the LDS (or a thread would hold more than 8 chunks).
template <int Q, int NB, int TR>
bool down_tr_fits(int k) {
  return down_runs_per<Q, NB, TR>(k) <= 8 && down_runs_lds<Q, NB, TR>(k) <= kLdsMax;
}

template <int Q, int NB, int TR, int PER>
int down_per(hipStream_t s, const DecodeArgs& a) {
  static bool attr = false;
  auto* kern = down_runs_kernel<Q, NB, TR, PER>;
  if (int st = allow_lds(kern, attr)) return st;
  const int ntiles = a.H / TR;
  const unsigned grid = unsigned(std::min(ntiles, cus_now()));
  kern<<<grid, kThreads, down_runs_lds<Q, NB, TR>(a.k + a.shared_slot), s>>>(a, ntiles);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int Q, int NB, int TR>
int down_tr(hipStream_t s, const DecodeArgs& a) {
  const int per = down_runs_per<Q, NB, TR>(a.k + a.shared_slot);
  if (per <= 2) return down_per<Q, NB, TR, 2>(s, a);
  if (per <= 4) return down_per<Q, NB, TR, 4>(s, a);
  if (per <= 6) return down_per<Q, NB, TR, 6>(s, a);
  return down_per<Q, NB, TR, 8>(s, a);
}

// 16-row tiles when they fit and give every CU a tile (H / 16 >= CUs),
// else 8-row tiles (H = 2048: 128 tiles of 16 rows would leave half of a
// 256-CU part idle)
template <int Q, int NB>
int pick_tr(int k, int H) {
  const bool fits16 = down_tr_fits<Q, NB, 16>(k), fits8 = down_tr_fits<Q, NB, 8>(k);
  if (fits16 && (!fits8 || H / 16 >= cus_now())) return 16;
  return 8;
}

template <int Q, int NB>
int down_nb(hipStream_t s, const DecodeArgs& a) {
  if (pick_tr<Q, NB>(a.k + a.shared_slot, a.H) == 16) return down_tr<Q, NB, 16>(s, a);
  return down_tr<Q, NB, 8>(s, a);
}

template <int Q>
int down_q(hipStream_t s, const DecodeArgs& a) {
  switch (a.I / kKBlock) {
    case 2: return down_nb<Q, 2>(s, a);
    case 3: return down_nb<Q, 3>(s, a);
    case 4: return down_nb<Q, 4>(s, a);
    case 6: return down_nb<Q, 6>(s, a);
    default: return down_nb<Q, 8>(s, a);
  }
}

template <int Q, int NB>
bool down_nb_fits(int k) {
  return down_tr_fits<Q, NB, 16>(k) || down_tr_fits<Q, NB, 8>(k);
}

template <int Q>
bool down_fits(int NB, int k) {
  switch (NB) {
    case 2: return down_nb_fits<Q, 2>(k);
    case 3: return down_nb_fits<Q, 3>(k);
    case 4: return down_nb_fits<Q, 4>(k);
    case 6: return down_nb_fits<Q, 6>(k);
    case 8: return down_nb_fits<Q, 8>(k);
    default: return false;
  }
}

}  // namespace

size_t decode_runs_stage_words(size_t H) { return size_t(xrun_words(int(H), true)); }

bool runs_gate_up_covers(int quant, int H, int x_dtype) {
  if (H % kKBlock || x_dtype != INFERNO_BF16) return false;
  const int NB = H / kKBlock;
  size_t lds;
  switch (quant) {
    case INFERNO_Q2_K: lds = gate_up_lds_q<INFERNO_Q2_K>(NB); break;
    case INFERNO_Q3_K: lds = gate_up_lds_q<INFERNO_Q3_K>(NB); break;
    case INFERNO_Q4_K: lds = gate_up_lds_q<INFERNO_Q4_K>(NB); break;
    default: return false;
  }
  return lds <= kLdsMax && cus_now() > 0;
}

bool runs_down_covers(int quant, int H, int I, int k) {
  // k: ranks summed, up to kMaxTopK routed ones plus the shared expert
  if (I % kKBlock || H % 16 || k < 1 || k > kMaxTopK + 1) return false;
  const int NB = I / kKBlock;
  switch (quant) {
    case INFERNO_Q2_K: return down_fits<INFERNO_Q2_K>(NB, k);
    case INFERNO_Q3_K: return down_fits<INFERNO_Q3_K>(NB, k);
    case INFERNO_Q4_K: return down_fits<INFERNO_Q4_K>(NB, k);
    case INFERNO_Q6_K: return down_fits<INFERNO_Q6_K>(NB, k);
    default: return false;
  }
}

int launch_gate_up_runs(hipStream_t s, const DecodeArgs& a, int quant) {
  switch (quant) {
    case INFERNO_Q2_K: return gate_up_q<INFERNO_Q2_K>(s, a);
    case INFERNO_Q3_K: return gate_up_q<INFERNO_Q3_K>(s, a);
    default: return gate_up_q<INFERNO_Q4_K>(s, a);
  }
}

int runs_down_tile_rows(int quant, int H, int I, int k) {
  auto pick = [&](auto q_c) {
    constexpr int Q = decltype(q_c)::value;
    switch (I / kKBlock) {
      case 2: return pick_tr<Q, 2>(k, H);
      case 3: return pick_tr<Q, 3>(k, H);
      case 4: return pick_tr<Q, 4>(k, H);
      case 6: return pick_tr<Q, 6>(k, H);
      default: return pick_tr<Q, 8>(k, H);
    }
  };
  switch (quant) {
    case INFERNO_Q2_K: return pick(std::integral_constant<int, INFERNO_Q2_K>{});
    case INFERNO_Q3_K: return pick(std::integral_constant<int, INFERNO_Q3_K>{});
    case INFERNO_Q6_K: return pick(std::integral_constant<int, INFERNO_Q6_K>{});
    default: return pick(std::integral_constant<int, INFERNO_Q4_K>{});
  }
}

int runs_down_row_bytes(int quant, int I) {
  const int NB = I / kKBlock;
  switch (quant) {
    case INFERNO_Q2_K: return NB * RF<INFERNO_Q2_K>::kBytes;
    case INFERNO_Q3_K: return NB * RF<INFERNO_Q3_K>::kBytes;
    case INFERNO_Q6_K: return NB * RF<INFERNO_Q6_K>::kBytes;
    default: return NB * RF<INFERNO_Q4_K>::kBytes;
  }
}

int launch_down_runs(hipStream_t s, const DecodeArgs& a, int quant) {
  switch (quant) {
    case INFERNO_Q2_K: return down_q<INFERNO_Q2_K>(s, a);
    case INFERNO_Q3_K: return down_q<INFERNO_Q3_K>(s, a);
    case INFERNO_Q6_K: return down_q<INFERNO_Q6_K>(s, a);
    default: return down_q<INFERNO_Q4_K>(s, a);
  }
}

// ------------------------------------------------- several tokens (T > 1)

namespace {

// Tokens per LDS pass of the gate/up: the most (8, 4 or 2) whose staged rows
// fit beside the tile.
template <int Q, int NB, bool SPLIT>
constexpr int multi_nt() {
  return gate_up_multi_lds<Q, NB, SPLIT, 8>() <= kLdsMax   ? 8
         : gate_up_multi_lds<Q, NB, SPLIT, 4>() <= kLdsMax ? 4
                                                           : 2;
}

// Down row groups per tile: 128, 64, 32 or 16 rows, the most whose weights
// stay within 56 KB (H is a multiple of 256, so every choice divides it).
template <int Q, int NB>
constexpr int multi_rg() {
  constexpr int rb = NB * RF<Q>::kBytes;
  return 128 * rb <= 56 * 1024 ? 8 : 64 * rb <= 56 * 1024 ? 4 : 32 * rb <= 56 * 1024 ? 2 : 1;
}
constexpr int kDownNT = 8;

// SEL: one token, the selection in the launch (one token per LDS pass)
template <int Q, int NB, bool SPLIT, bool SEL>
int gate_up_multi_nb(hipStream_t s, const DecodeArgs& a) {
  constexpr int NT = SEL ? 1 : multi_nt<Q, NB, SPLIT>();
  // upper bound: active slots <= max_slots (plus the shared slot)
  const int ntiles = (a.max_slots + a.shared_slot) * (a.I / kRows);
  if constexpr (SEL) {
    // one token: workgroups of WV wavefronts, several per CU (all of a
    // layer's tiles in flight at once); INFERNO_DECODE_SEL_WAVES = 16, 8
    // (default) or 4
    const char* wv = std::getenv("INFERNO_DECODE_SEL_WAVES");
    const int waves = wv ? std::atoi(wv) : 8;
    auto launch_wv = [&](auto wv_c) -> int {
      constexpr int WV = decltype(wv_c)::value;
      static bool attr_wv = false;
      auto* kw = gate_up_runs_multi_kernel<Q, NB, SPLIT, NT, SEL, WV>;
      if (int st = allow_lds(kw, attr_wv)) return st;
      constexpr size_t lds = gate_up_multi_lds<Q, NB, SPLIT, NT, SEL, WV>();
      const int per_cu = std::min(int(16 / WV), int(kLdsMax / lds));
      const unsigned grid = unsigned(std::min(ntiles, per_cu * cus_now()));
      kw<<<grid, 64 * WV, lds, s>>>(a);
      INF_LAUNCHED();
      return INFERNO_OK;
    };
    if (waves == 8) return launch_wv(std::integral_constant<int, 8>{});
    if (waves == 4) return launch_wv(std::integral_constant<int, 4>{});
  }
  static bool attr = false;
  auto* kern = gate_up_runs_multi_kernel<Q, NB, SPLIT, NT, SEL>;
  if (int st = allow_lds(kern, attr)) return st;
  const unsigned grid = unsigned(std::min(ntiles, cus_now()));
  kern<<<grid, kThreads, gate_up_multi_lds<Q, NB, SPLIT, NT, SEL>(), s>>>(a);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int Q, bool SPLIT, bool SEL>
int gate_up_multi_q(hipStream_t s, const DecodeArgs& a) {
  switch (a.H / kKBlock) {
    case 4: return gate_up_multi_nb<Q, 4, SPLIT, SEL>(s, a);
    case 8: return gate_up_multi_nb<Q, 8, SPLIT, SEL>(s, a);
    case 12: return gate_up_multi_nb<Q, 12, SPLIT, SEL>(s, a);
    case 16: return gate_up_multi_nb<Q, 16, SPLIT, SEL>(s, a);
    default: return gate_up_multi_nb<Q, 24, SPLIT, SEL>(s, a);
  }
}

template <int Q, bool SPLIT>
size_t gate_up_multi_lds_q(int NB) {
  switch (NB) {
    case 4: return gate_up_multi_lds<Q, 4, SPLIT, multi_nt<Q, 4, SPLIT>()>();
    case 8: return gate_up_multi_lds<Q, 8, SPLIT, multi_nt<Q, 8, SPLIT>()>();
    case 12: return gate_up_multi_lds<Q, 12, SPLIT, multi_nt<Q, 12, SPLIT>()>();
    case 16: return gate_up_multi_lds<Q, 16, SPLIT, multi_nt<Q, 16, SPLIT>()>();
    case 24: return gate_up_multi_lds<Q, 24, SPLIT, multi_nt<Q, 24, SPLIT>()>();
    default: return ~size_t(0);
  }
}

template <int Q, int NB>
int down_multi_nb(hipStream_t s, const DecodeArgs& a) {
  constexpr int RG = multi_rg<Q, NB>();
  static bool attr = false;
  auto* kern = down_runs_multi_kernel<Q, NB, RG, kDownNT>;
  if (int st = allow_lds(kern, attr)) return st;
  const int ntiles = a.max_slots * (a.H / (16 * RG));
  const unsigned grid = unsigned(std::min(ntiles, cus_now()));
  kern<<<grid, kThreads, down_multi_lds<Q, NB, RG, kDownNT>(), s>>>(a);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int Q>
int down_multi_q(hipStream_t s, const DecodeArgs& a) {
  switch (a.I / kKBlock) {
    case 3: return down_multi_nb<Q, 3>(s, a);
    case 4: return down_multi_nb<Q, 4>(s, a);
    case 6: return down_multi_nb<Q, 6>(s, a);
    default: return down_multi_nb<Q, 8>(s, a);
  }
}

template <int Q>
size_t down_multi_lds_q(int NB) {
  switch (NB) {
    case 3: return down_multi_lds<Q, 3, multi_rg<Q, 3>(), kDownNT>();
    case 4: return down_multi_lds<Q, 4, multi_rg<Q, 4>(), kDownNT>();
    case 6: return down_multi_lds<Q, 6, multi_rg<Q, 6>(), kDownNT>();
    case 8: return down_multi_lds<Q, 8, multi_rg<Q, 8>(), kDownNT>();
    default: return ~size_t(0);
  }
}

template <int Q>
bool multi_covers_q(int H, int I, bool split) {
  const int NB = H / kKBlock, NBI = I / kKBlock;
  const size_t gu = split ? gate_up_multi_lds_q<Q, true>(NB) : gate_up_multi_lds_q<Q, false>(NB);
  return gu <= kLdsMax && down_multi_lds_q<Q>(NBI) <= kLdsMax;
}

}  // namespace

bool runs_multi_covers(int quant, int H, int I, int x_dtype) {
  if (H % kKBlock || I % kKBlock || H % 128 || cus_now() <= 0) return false;
  if (x_dtype != INFERNO_BF16 && x_dtype != INFERNO_F32) return false;
  const bool split = x_dtype == INFERNO_F32;
  switch (quant) {
    case INFERNO_Q2_K: return multi_covers_q<INFERNO_Q2_K>(H, I, split);
    case INFERNO_Q3_K: return multi_covers_q<INFERNO_Q3_K>(H, I, split);
    case INFERNO_Q4_K: return multi_covers_q<INFERNO_Q4_K>(H, I, split);
    default: return false;
  }
}

template <bool SEL>
int gate_up_multi_sel(hipStream_t s, const DecodeArgs& a, int quant) {
  const bool split = a.x_dtype == INFERNO_F32;
  switch (quant) {
    case INFERNO_Q2_K:
      return split ? gate_up_multi_q<INFERNO_Q2_K, true, SEL>(s, a) : gate_up_multi_q<INFERNO_Q2_K, false, SEL>(s, a);
    case INFERNO_Q3_K:
      return split ? gate_up_multi_q<INFERNO_Q3_K, true, SEL>(s, a) : gate_up_multi_q<INFERNO_Q3_K, false, SEL>(s, a);
    default:
      return split ? gate_up_multi_q<INFERNO_Q4_K, true, SEL>(s, a) : gate_up_multi_q<INFERNO_Q4_K, false, SEL>(s, a);
  }
}

int launch_gate_up_runs_multi(hipStream_t s, const DecodeArgs& a, int quant, bool sel) {
  return sel ? gate_up_multi_sel<true>(s, a, quant) : gate_up_multi_sel<false>(s, a, quant);
}

// The selecting variant's LDS fits (one token per pass).
bool runs_multi_sel_covers(int quant, int H, int x_dtype) {
  const bool split = x_dtype == INFERNO_F32;
  const int NB = H / kKBlock;
  auto lds = [&](auto q_c) -> size_t {
    constexpr int Q = decltype(q_c)::value;
    switch (NB) {
      case 4: return split ? gate_up_multi_lds<Q, 4, true, 1, true>() : gate_up_multi_lds<Q, 4, false, 1, true>();
      case 8: return split ? gate_up_multi_lds<Q, 8, true, 1, true>() : gate_up_multi_lds<Q, 8, false, 1, true>();
      case 12: return split ? gate_up_multi_lds<Q, 12, true, 1, true>() : gate_up_multi_lds<Q, 12, false, 1, true>();
      case 16: return split ? gate_up_multi_lds<Q, 16, true, 1, true>() : gate_up_multi_lds<Q, 16, false, 1, true>();
      case 24: return split ? gate_up_multi_lds<Q, 24, true, 1, true>() : gate_up_multi_lds<Q, 24, false, 1, true>();
      default: return ~size_t(0);
    }
  };
  switch (quant) {
    case INFERNO_Q2_K: return lds(std::integral_constant<int, INFERNO_Q2_K>{}) <= kLdsMax;
    case INFERNO_Q3_K: return lds(std::integral_constant<int, INFERNO_Q3_K>{}) <= kLdsMax;
    case INFERNO_Q4_K: return lds(std::integral_constant<int, INFERNO_Q4_K>{}) <= kLdsMax;
    default: return false;
  }
}


int launch_down_runs_multi(hipStream_t s, const DecodeArgs& a, int quant) {
  switch (quant) {
    case INFERNO_Q2_K: return down_multi_q<INFERNO_Q2_K>(s, a);
    case INFERNO_Q3_K: return down_multi_q<INFERNO_Q3_K>(s, a);
    default: return down_multi_q<INFERNO_Q4_K>(s, a);
  }
}

}  // namespace inferno
