// Launchers of the f16-run matrix-core decode kernels (decode_runs.hpp):
// instances per format, super-block columns and register batch.
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
  kern<<<grid, kThreads, down_runs_lds<Q, NB, TR>(a.k), s>>>(a, ntiles);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int Q, int NB, int TR>
int down_tr(hipStream_t s, const DecodeArgs& a) {
  const int per = down_runs_per<Q, NB, TR>(a.k);
  if (per <= 2) return down_per<Q, NB, TR, 2>(s, a);
  if (per <= 4) return down_per<Q, NB, TR, 4>(s, a);
  if (per <= 6) return down_per<Q, NB, TR, 6>(s, a);
  return down_per<Q, NB, TR, 8>(s, a);
}

template <int Q, int NB>
int down_nb(hipStream_t s, const DecodeArgs& a) {
  if (down_tr_fits<Q, NB, 16>(a.k)) return down_tr<Q, NB, 16>(s, a);
  return down_tr<Q, NB, 8>(s, a);
}

template <int Q>
int down_q(hipStream_t s, const DecodeArgs& a) {
  switch (a.I / kKBlock) {
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
    case 3: return down_nb_fits<Q, 3>(k);
    case 4: return down_nb_fits<Q, 4>(k);
    case 6: return down_nb_fits<Q, 6>(k);
    case 8: return down_nb_fits<Q, 8>(k);
    default: return false;
  }
}

}  // namespace

size_t decode_runs_stage_words(size_t H) { return size_t(run_words(int(H))); }

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
  if (I % kKBlock || H % 16 || k < 1 || k > kMaxTopK) return false;
  const int NB = I / kKBlock;
  switch (quant) {
    case INFERNO_Q2_K: return down_fits<INFERNO_Q2_K>(NB, k);
    case INFERNO_Q3_K: return down_fits<INFERNO_Q3_K>(NB, k);
    case INFERNO_Q4_K: return down_fits<INFERNO_Q4_K>(NB, k);
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

int launch_down_runs(hipStream_t s, const DecodeArgs& a, int quant) {
  switch (quant) {
    case INFERNO_Q2_K: return down_q<INFERNO_Q2_K>(s, a);
    case INFERNO_Q3_K: return down_q<INFERNO_Q3_K>(s, a);
    default: return down_q<INFERNO_Q4_K>(s, a);
  }
}

}  // namespace inferno
