// extern "C" entry points: argument validation (mirroring the reference's
// Err paths, e.g. crates/backend/src/metal/gguf_moe.rs:84-121 and
// crates/backend/src/metal/moe.rs:582-623), workspace carving and kernel
// sequencing. No function allocates device memory or synchronises.
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "decode.hpp"
#include "prefill.hpp"
#include "timing.hpp"
#include "gemv_common.hpp"
#include "quantize.hpp"

namespace inferno {

thread_local std::string g_last_error;
void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

namespace {

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

size_t align_up(size_t v) { return (v + 255) & ~size_t(255); }

// Carves aligned sub-buffers out of a caller workspace.
struct Carver {
  char* base;
  size_t used = 0;
  template <typename T>
  T* take(size_t count) {
    T* p = reinterpret_cast<T*>(base ? base + used : nullptr);
    used += align_up(count * sizeof(T));
    return p;
  }
};

bool is_routed_quant(int q) {
  return q == INFERNO_Q2_K || q == INFERNO_Q3_K || q == INFERNO_Q4_K;
}
bool is_down_quant(int q) { return is_routed_quant(q) || q == INFERNO_Q6_K; }

// Bytes of one expert matrix of `rows` rows over `cols` values.
size_t matrix_bytes(int quant, size_t rows, size_t cols) {
  return rows * (cols / size_t(block_values(quant))) * size_t(block_bytes(quant));
}

int check_len(const char* label, size_t got, size_t experts, size_t stride) {
  if (got != experts * stride) {
    set_error(std::string("GGUF ") + label + " expert payload must contain " +
              std::to_string(experts * stride) + " bytes, got " + std::to_string(got));
    return INFERNO_ERR_SIZE;
  }
  return INFERNO_OK;
}

struct MoeScratch {
  uint32_t* offsets;
  uint32_t* sorted;
  uint32_t* active;
  float* h;
  float* y;
  uint32_t* stage_x;  // staged activations of x (sized for fp32 input); f16 x on the MFMA path
  uint32_t* stage_h;  // staged activations of h
  uint32_t* plan;     // MFMA path: expert tile lists
};

// Staged activation rows, sized for the fp32 (split) layout, the larger one.
size_t stage_words(size_t rows, size_t K) {
  return gemv_stage_bytes(INFERNO_Q2_K, rows, K, INFERNO_F32) / 4;
}

MoeScratch carve_moe(Carver& c, size_t T, size_t k, size_t E, size_t H, size_t I) {
  MoeScratch m;
  m.offsets = c.take<uint32_t>(E + 1);
  m.sorted = c.take<uint32_t>(T * k);
  m.active = c.take<uint32_t>(E + 1);
  m.h = c.take<float>(T * k * I);
  m.y = c.take<float>(T * k * H);
  m.stage_x = c.take<uint32_t>(stage_words(T, H));
  // (one row more: the shared expert's h when it runs as assignment k)
  m.stage_h = c.take<uint32_t>(stage_words(T * k + 1, I));
  m.plan = c.take<uint32_t>(prefill_plan_words(T * k, E));
  return m;
}

int validate_moe(int quant, int down_quant, size_t gate_bytes, size_t up_bytes,
                 size_t down_bytes, size_t T, size_t k, size_t E, size_t H, size_t I) {
  INF_CHECK_ARG(is_routed_quant(quant), "routed gate/up experts must be Q2_K, Q3_K or Q4_K");
  INF_CHECK_ARG(is_down_quant(down_quant), "routed down experts must be Q2_K, Q3_K, Q4_K or Q6_K");
  if (T == 0 || k == 0 || k > E) {
    set_error("GGUF MoE routing dimensions are invalid: tokens=" + std::to_string(T) +
              ", top_k=" + std::to_string(k) + ", experts=" + std::to_string(E));
    return INFERNO_ERR_INVALID;
  }
  INF_CHECK_ARG(E <= size_t(kMaxExperts), "at most 256 experts are supported");
  INF_CHECK_ARG(k <= size_t(kMaxTopK), "top_k must be at most 16");
  if (H % kKBlock || I % kKBlock || H == 0 || I == 0) {
    set_error("GGUF MoE dimensions must use 256-wide quant blocks, got in=" + std::to_string(H) +
              ", intermediate=" + std::to_string(I));
    return INFERNO_ERR_INVALID;
  }
  INF_CHECK_ARG(T * k < (size_t(1) << 31), "too many assignments");
  int st;
  if ((st = check_len("gate", gate_bytes, E, matrix_bytes(quant, I, H)))) return st;
  if ((st = check_len("up", up_bytes, E, matrix_bytes(quant, I, H)))) return st;
  if ((st = check_len("down", down_bytes, E, matrix_bytes(down_quant, H, I)))) return st;
  return INFERNO_OK;
}

// Routed part shared by inferno_gguf_moe and the layer: dispatch, gate/up,
// down. Leaves per-assignment down rows (already routing-weighted) in m.y.
// Many assignments take the MFMA grouped GEMM; few take the packed-f16 GEMV.
// Is: the layer's shared expert width (0: none); with one, the decode
// launches keep more assignments (they run the shared expert inside them).
bool use_mfma(int quant, int down_quant, size_t T, size_t k, size_t E, size_t H, size_t I,
              size_t Is = 0) {
  const size_t from = Is ? kPrefillMinAssignmentsShared : kPrefillMinAssignments;
  return T * k >= env_size("INFERNO_PREFILL_MIN_ASSIGNMENTS", from) &&
         prefill_routed_supported(quant, down_quant, H, I, E);
}

// `x16`: x already converted to f16 (MFMA path), or null. `distinct_ids`:
// every token's k ids are distinct (the layer's own top-k), so one expert
// takes at most T rows (caller ids may repeat an expert within a token).
int run_routed(hipStream_t s, int quant, int down_quant, const void* gate, const void* up,
               const void* down, const void* x, int x_dtype, const uint32_t* ids,
               const float* w, size_t T, size_t k, size_t E, size_t H, size_t I,
               const MoeScratch& m, bool x_staged, bool mfma, const uint16_t* x16 = nullptr,
               bool distinct_ids = false) {
  int st;
  // on the MFMA path the dispatch also writes the GEMM's tile lists
  const PlanOut plan = mfma ? prefill_plan_out(m.plan, T * k, E) : PlanOut{};
  if ((st = launch_dispatch(s, ids, T, k, E, m.offsets, m.sorted, m.active, mfma ? &plan : nullptr)))
    return st;
  if (mfma) {
    if (!x16) {
      uint16_t* conv = reinterpret_cast<uint16_t*>(m.stage_x);
      if ((st = launch_to_f16(s, x, x_dtype, T, H, conv))) return st;
      x16 = conv;
    }
    PrefillRouted p{quant, down_quant, gate, up, down, x16, m.offsets, m.sorted, m.active, w,
                    T, k, E, H, I, reinterpret_cast<uint16_t*>(m.h), m.y, m.plan,
                    distinct_ids ? T : 0};
    if ((st = timed(s, kTimerGateUp, "prefill: grouped gate/up GEMMs (gemm_kernel / gemm2_kernel, MFMA)",
                    [&] { return launch_prefill_gate_up(s, p); })))
      return st;
    return timed(s, kTimerDown, "prefill: grouped down GEMMs (gemm_kernel / gemm2_kernel, MFMA)",
                 [&] { return launch_prefill_down(s, p); });
  }
  // gate/up writes h already staged for the down pass (when the down kind has a
  // packed-f16 kernel; Q6_K reads the fp32 h)
  const bool h_staged = dot2_supported(down_quant);
  if ((st = timed(s, kTimerGateUp, "stage: routed gate/up GEMV", [&] {
         return launch_gemv_gate_up_routed(s, quant, gate, up, x, x_dtype, m.stage_x, x_staged,
                                           m.offsets, m.sorted, m.active, w, T, k, E, H, I, m.h,
                                           h_staged ? m.stage_h : nullptr);
       })))
    return st;
  return timed(s, kTimerDown, "stage: routed down GEMV", [&] {
    return launch_gemv_down_routed(s, down_quant, down, m.h, m.stage_h, h_staged, m.offsets,
                                   m.sorted, m.active, T, k, E, H, I, m.y);
  });
}

// The reference returns Ok(None) ("unsupported here, the caller may fall
// back") when no native device backs the backend (backend.rs:6688-6692 and
// the non-Metal branches); the counterpart here is INFERNO_UNSUPPORTED when
// the process sees no HIP device. Argument errors are reported before this
// check, as the reference validates before it looks for the device.
int require_device() {
  static const int count = [] {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess ? n : 0;
  }();
  if (count > 0) return INFERNO_OK;
  set_error("no HIP device is available (unsupported here; the caller may fall back)");
  return INFERNO_UNSUPPORTED;
}

int need_ws(void* ws, size_t have, size_t need) {
  if (need > 0 && (ws == nullptr || have < need)) {
    set_error("workspace too small: need " + std::to_string(need) + " bytes");
    return INFERNO_ERR_SIZE;
  }
  return INFERNO_OK;
}

}  // namespace
}  // namespace inferno

using namespace inferno;

extern "C" {

const char* inferno_last_error(void) { return g_last_error.c_str(); }

int inferno_block_bytes(int quant) { return block_bytes(quant); }
int inferno_block_values(int quant) { return block_values(quant); }

int inferno_kernel_timing_enable(int enable) {
  clear_error();
  kernel_timing_enable(enable != 0);
  return INFERNO_OK;
}

int inferno_kernel_timing_read(int which, double* total_ms, uint64_t* launches) {
  clear_error();
  INF_CHECK_ARG(total_ms && launches, "null output pointer");
  INF_CHECK_ARG(kernel_timing_read(which, total_ms, launches), "unknown timer");
  return INFERNO_OK;
}

int inferno_kernel_timing_label(int which, char* buf, size_t len) {
  clear_error();
  INF_CHECK_ARG(which >= 0 && which < kNumTimers, "unknown timer");
  INF_CHECK_ARG(buf && len > 0, "null buffer");
  const char* l = kernel_timing_label(which);
  size_t n = 0;
  while (l[n] && n + 1 < len) {
    buf[n] = l[n];
    ++n;
  }
  buf[n] = '\0';
  return INFERNO_OK;
}

int inferno_stream_synchronize(void* stream) {
  clear_error();
  INF_HIP(hipStreamSynchronize(as_stream(stream)));
  return INFERNO_OK;
}

int inferno_gguf_dequantize(void* stream, int quant, const void* blocks, size_t n_blocks,
                            float* out) {
  clear_error();
  INF_CHECK_ARG(block_bytes(quant) > 0, "unknown quant kind");
  INF_CHECK_ARG(n_blocks == 0 || (blocks && out), "null pointer");
  if (int st_ = require_device()) return st_;
  return launch_dequant(as_stream(stream), quant, blocks, n_blocks, out);
}

int inferno_router_logits(void* stream, const void* x, int x_dtype, const float* w_router,
                          size_t T, size_t H, size_t E, float* logits) {
  clear_error();
  INF_CHECK_ARG(x_dtype == INFERNO_F32 || x_dtype == INFERNO_BF16, "x dtype must be F32 or BF16");
  INF_CHECK_ARG(H > 0 && H % 4 == 0, "hidden size must be a positive multiple of 4");
  INF_CHECK_ARG(E > 0, "expert count must be positive");
  INF_CHECK_ARG(T == 0 || (x && w_router && logits), "null pointer");
  if (int st_ = require_device()) return st_;
  return launch_router_logits(as_stream(stream), x, x_dtype, w_router, T, H, E, logits);
}

int inferno_moe_router_topk(void* stream, const float* logits, const float* bias, size_t T,
                            size_t E, size_t k, int score_fn, int norm_topk_prob,
                            float routed_scaling_factor, uint32_t* expert_ids,
                            float* expert_weights, uint32_t* token_indices) {
  clear_error();
  INF_CHECK_ARG(T > 0 && E > 0, "MoE router top-k requires non-zero token_count and expert_count");
  if (k == 0 || k > size_t(kMaxTopK)) {
    set_error("MoE router top-k supports 1..=16 selected experts, got " + std::to_string(k));
    return INFERNO_ERR_INVALID;
  }
  if (k > E) {
    set_error("MoE router top-k " + std::to_string(k) + " exceeds expert_count " +
              std::to_string(E));
    return INFERNO_ERR_INVALID;
  }
  if (E > size_t(kMaxExperts)) {
    set_error("MoE router top-k supports at most 256 experts, got " + std::to_string(E));
    return INFERNO_ERR_INVALID;
  }
  INF_CHECK_ARG(score_fn == INFERNO_SCORE_SIGMOID || score_fn == INFERNO_SCORE_SOFTMAX,
                "score_fn must be SIGMOID or SOFTMAX");
  INF_CHECK_ARG(std::isfinite(routed_scaling_factor), "MoE router routed scaling factor must be finite");
  INF_CHECK_ARG(logits && expert_ids && expert_weights, "null pointer");
  if (int st_ = require_device()) return st_;
  return launch_router_topk(as_stream(stream), logits, bias, T, E, k, score_fn, norm_topk_prob,
                            routed_scaling_factor, expert_ids, expert_weights, token_indices);
}

int inferno_moe_dispatch(void* stream, const uint32_t* expert_ids, size_t T, size_t k, size_t E,
                         uint32_t* offsets, uint32_t* sorted, uint32_t* active) {
  clear_error();
  INF_CHECK_ARG(E > 0 && E <= size_t(kMaxExperts), "expert_count must be in 1..=256");
  INF_CHECK_ARG(T * k < (size_t(1) << 31), "too many assignments");
  INF_CHECK_ARG(offsets && active && (T * k == 0 || (expert_ids && sorted)), "null pointer");
  if (int st_ = require_device()) return st_;
  return launch_dispatch(as_stream(stream), expert_ids, T, k, E, offsets, sorted, active);
}

size_t inferno_gguf_moe_workspace_bytes(size_t T, size_t k, size_t E, size_t H, size_t I) {
  Carver c{nullptr};
  carve_moe(c, T, k, E, H, I);
  return c.used;
}

int inferno_gguf_moe(void* stream, int quant, int down_quant, const void* gate,
                     size_t gate_bytes, const void* up, size_t up_bytes, const void* down,
                     size_t down_bytes, const void* x, int x_dtype, const uint32_t* expert_ids,
                     const float* expert_weights, size_t T, size_t k, size_t E, size_t H,
                     size_t I, float* out, void* workspace, size_t workspace_bytes) {
  clear_error();
  int st = validate_moe(quant, down_quant, gate_bytes, up_bytes, down_bytes, T, k, E, H, I);
  if (st) return st;
  INF_CHECK_ARG(x_dtype == INFERNO_F32 || x_dtype == INFERNO_BF16, "x dtype must be F32 or BF16");
  INF_CHECK_ARG(gate && up && down && x && expert_ids && expert_weights && out && workspace,
                "null pointer");
  size_t need = inferno_gguf_moe_workspace_bytes(T, k, E, H, I);
  if (workspace_bytes < need) {
    set_error("workspace too small: need " + std::to_string(need) + " bytes");
    return INFERNO_ERR_SIZE;
  }
  if (int st_ = require_device()) return st_;
  Carver c{static_cast<char*>(workspace)};
  MoeScratch m = carve_moe(c, T, k, E, H, I);
  hipStream_t s = as_stream(stream);
  if ((st = run_routed(s, quant, down_quant, gate, up, down, x, x_dtype, expert_ids,
                       expert_weights, T, k, E, H, I, m, false,
                       use_mfma(quant, down_quant, T, k, E, H, I))))
    return st;
  return launch_topk_combine(s, nullptr, nullptr, m.y, nullptr, T, H, k, out);
}

size_t inferno_gemv_workspace_bytes(size_t rows, size_t K) {
  return gemv_stage_bytes(INFERNO_Q2_K, rows, K, INFERNO_F32);
}

int inferno_moe_expert_gate_up_swiglu(void* stream, int quant, const void* gate,
                                      size_t gate_bytes, const void* up, size_t up_bytes,
                                      const void* x, int x_dtype, const uint32_t* offsets,
                                      const uint32_t* sorted, const uint32_t* active,
                                      const float* expert_weights, size_t T, size_t k, size_t E,
                                      size_t H, size_t I, float* h, void* workspace,
                                      size_t workspace_bytes) {
  clear_error();
  int st = validate_moe(quant, quant, gate_bytes, up_bytes, E * matrix_bytes(quant, H, I), T, k,
                        E, H, I);
  if (st) return st;
  INF_CHECK_ARG(x_dtype == INFERNO_F32 || x_dtype == INFERNO_BF16, "x dtype must be F32 or BF16");
  INF_CHECK_ARG(gate && up && x && offsets && sorted && active && expert_weights && h,
                "null pointer");
  if ((st = need_ws(workspace, workspace_bytes, gemv_stage_bytes(quant, T, H, x_dtype)))) return st;
  if (int st_ = require_device()) return st_;
  return launch_gemv_gate_up_routed(as_stream(stream), quant, gate, up, x, x_dtype,
                                    static_cast<uint32_t*>(workspace), false, offsets, sorted,
                                    active, expert_weights, T, k, E, H, I, h, nullptr);
}

int inferno_moe_expert_down(void* stream, int down_quant, const void* down, size_t down_bytes,
                            const float* h, const uint32_t* offsets, const uint32_t* sorted,
                            const uint32_t* active, size_t T, size_t k, size_t E, size_t H,
                            size_t I, float* y, void* workspace, size_t workspace_bytes) {
  clear_error();
  int st = validate_moe(INFERNO_Q2_K, down_quant, E * matrix_bytes(INFERNO_Q2_K, I, H),
                        E * matrix_bytes(INFERNO_Q2_K, I, H), down_bytes, T, k, E, H, I);
  if (st) return st;
  INF_CHECK_ARG(down && h && offsets && sorted && active && y, "null pointer");
  if ((st = need_ws(workspace, workspace_bytes,
                    gemv_stage_bytes(down_quant, T * k, I, INFERNO_F32))))
    return st;
  if (int st_ = require_device()) return st_;
  return launch_gemv_down_routed(as_stream(stream), down_quant, down, h,
                                 static_cast<uint32_t*>(workspace), false, offsets, sorted, active,
                                 T, k, E, H, I, y);
}

int inferno_q8_0_gate_up_swiglu(void* stream, const void* gate, size_t gate_bytes, const void* up,
                                size_t up_bytes, const void* x, int x_dtype, size_t T, size_t H,
                                size_t Is, float* out, void* workspace, size_t workspace_bytes) {
  clear_error();
  INF_CHECK_ARG(H % kKBlock == 0 && Is > 0 && H > 0, "Q8_0 in_features must be a multiple of 256");
  INF_CHECK_ARG(x_dtype == INFERNO_F32 || x_dtype == INFERNO_BF16, "x dtype must be F32 or BF16");
  int st;
  if ((st = check_len("shared gate", gate_bytes, 1, matrix_bytes(INFERNO_Q8_0, Is, H)))) return st;
  if ((st = check_len("shared up", up_bytes, 1, matrix_bytes(INFERNO_Q8_0, Is, H)))) return st;
  if (T == 0) return INFERNO_OK;
  INF_CHECK_ARG(gate && up && x && out, "null pointer");
  if ((st = need_ws(workspace, workspace_bytes, gemv_stage_bytes(INFERNO_Q8_0, T, H, x_dtype))))
    return st;
  if (int st_ = require_device()) return st_;
  return launch_gemv_gate_up_dense(as_stream(stream), INFERNO_Q8_0, gate, up, x, x_dtype,
                                   static_cast<uint32_t*>(workspace), false, T, H, Is, out,
                                   nullptr);
}

int inferno_q8_0_matvec_add2(void* stream, const void* w, size_t w_bytes, const float* input,
                             const float* residual_a, const float* residual_b, size_t T,
                             size_t In, size_t O, float* out, void* workspace,
                             size_t workspace_bytes) {
  clear_error();
  INF_CHECK_ARG(In % kKBlock == 0 && In > 0 && O > 0, "Q8_0 in_features must be a multiple of 256");
  int st;
  if ((st = check_len("shared down", w_bytes, 1, matrix_bytes(INFERNO_Q8_0, O, In)))) return st;
  if (T == 0) return INFERNO_OK;
  INF_CHECK_ARG(w && input && out, "null pointer");
  if ((st = need_ws(workspace, workspace_bytes, gemv_stage_bytes(INFERNO_Q8_0, T, In, INFERNO_F32))))
    return st;
  if (int st_ = require_device()) return st_;
  return launch_gemv_down_dense(as_stream(stream), INFERNO_Q8_0, w, input,
                                static_cast<uint32_t*>(workspace), false, nullptr, 0, residual_a,
                                residual_b, T, In, O, out);
}

int inferno_moe_topk_combine_residual(void* stream, const float* shared, const float* residual,
                                      const float* expert_outputs, const float* expert_weights,
                                      size_t T, size_t H, size_t k, float* out) {
  clear_error();
  INF_CHECK_ARG(k > 0 && H > 0, "top_k and hidden size must be positive");
  INF_CHECK_ARG(T == 0 || (expert_outputs && expert_weights && out), "null pointer");
  if (int st_ = require_device()) return st_;
  return launch_topk_combine(as_stream(stream), shared, residual, expert_outputs, expert_weights,
                             T, H, k, out);
}

int inferno_moe_weighted_index_add_combine(void* stream, const float* acc,
                                           const uint32_t* token_indices,
                                           const float* expert_outputs,
                                           const float* expert_weights, size_t T, size_t H,
                                           size_t A, float* out) {
  clear_error();
  INF_CHECK_ARG(T == 0 || (acc && out), "null pointer");
  INF_CHECK_ARG(A == 0 || (token_indices && expert_outputs && expert_weights), "null pointer");
  if (int st_ = require_device()) return st_;
  return launch_index_add_combine(as_stream(stream), acc, token_indices, expert_outputs,
                                  expert_weights, T, H, A, out);
}

int inferno_moe_gather_tokens(void* stream, const float* x, const uint32_t* token_indices,
                              size_t T, size_t H, size_t A, float* out) {
  clear_error();
  INF_CHECK_ARG(A == 0 || (x && token_indices && out), "null pointer");
  if (int st_ = require_device()) return st_;
  return launch_gather(as_stream(stream), x, token_indices, T, H, A, out);
}

int inferno_rms_norm(void* stream, const float* x, const float* w, size_t rows, size_t H,
                     float eps, float* out) {
  clear_error();
  INF_CHECK_ARG(H > 0 && eps >= 0.f, "rms_norm needs a positive width and eps >= 0");
  INF_CHECK_ARG(rows == 0 || (x && w && out), "null pointer");
  if (int st_ = require_device()) return st_;
  return launch_rms_norm(as_stream(stream), x, w, rows, H, eps, out, INFERNO_F32);
}

size_t inferno_rms_norm_router_topk_workspace_bytes(size_t T) {
  return (T * sizeof(uint32_t) + 255) / 256 * 256;
}

int inferno_rms_norm_router_topk(void* stream, const float* x, const float* norm_weight, float eps,
                                 const float* router, const float* bias, size_t T, size_t H,
                                 size_t E, size_t k, int score_fn, int norm_topk_prob,
                                 float routed_scaling_factor, int act_dtype, void* normed_out,
                                 float* logits_out, uint32_t* expert_ids, float* expert_weights,
                                 void* workspace, size_t workspace_bytes) {
  clear_error();
  INF_CHECK_ARG(eps >= 0.f, "eps must be >= 0");
  INF_CHECK_ARG(act_dtype == INFERNO_F32 || act_dtype == INFERNO_BF16,
                "act dtype must be F32 or BF16");
  INF_CHECK_ARG(score_fn == INFERNO_SCORE_SIGMOID || score_fn == INFERNO_SCORE_SOFTMAX,
                "score_fn must be SIGMOID or SOFTMAX");
  if (T == 0) return INFERNO_OK;
  INF_CHECK_ARG(x && norm_weight && router && logits_out, "null pointer");
  const bool topk = expert_ids != nullptr;
  if (topk) {
    INF_CHECK_ARG(expert_weights && workspace, "null pointer");
    if (workspace_bytes < inferno_rms_norm_router_topk_workspace_bytes(T)) {
      set_error("workspace too small: need " +
                std::to_string(inferno_rms_norm_router_topk_workspace_bytes(T)) + " bytes");
      return INFERNO_ERR_SIZE;
    }
  }
  if (!norm_router_supported(T, H, E, topk ? k : 0)) {
    set_error("fused norm+router needs H a multiple of 64 up to 8192, E <= 256, k <= min(E, 16)");
    return INFERNO_UNSUPPORTED;
  }
  if (int st_ = require_device()) return st_;
  return launch_norm_router(as_stream(stream), x, norm_weight, eps, router, bias, T, H, E, k,
                            score_fn, norm_topk_prob, routed_scaling_factor, act_dtype, normed_out,
                            logits_out, static_cast<uint32_t*>(workspace),
                            topk ? expert_ids : nullptr, expert_weights);
}

// ------------------------------------------------------------- layer

namespace {
struct LayerScratch {
  float* logits;
  uint32_t* ids;
  float* weights;
  float* hs;
  uint32_t* stage_hs;
  MoeScratch moe;
  // fused decode path
  float* partials;
  float* ys;
  uint4* slots;
  uint32_t* stage_xm;
  uint32_t* stage_xr;
  float* shared_gu;
  void* blas;     // the Q8_0 shared expert on library GEMMs (large batches), or null
  void* rblas;    // the router's bf16 terms for the library GEMMs (large batches), or null
  void* blas_lib; // the library's workspace when either runs, or null
};
// lib: the library GEMMs (hipBLASLt) may run (their regions are carved);
// the no-alloc entry point passes false: the library allocates on its own.
LayerScratch carve_layer(Carver& c, const inferno_moe_layer* L, size_t T, bool lib = true) {
  LayerScratch s;
  // router logits, or their K-chunk partials for a small bf16 batch
  s.logits = c.take<float>(T * L->experts *
                           size_t(router_logit_parts_max(T, L->hidden, L->experts)));
  s.ids = c.take<uint32_t>(T * L->top_k);
  s.weights = c.take<float>(T * L->top_k);
  s.hs = c.take<float>(T * (L->shared_intermediate ? L->shared_intermediate : 1));
  s.stage_hs = c.take<uint32_t>(L->shared_intermediate ? stage_words(T, L->shared_intermediate) : 1);
  s.moe = carve_moe(c, T, L->top_k, L->experts, L->hidden, L->intermediate);
  s.partials = c.take<float>(size_t(L->hidden / decode_chunk(L->hidden)) * T * L->experts);
  s.ys = c.take<float>(T * L->hidden);
  s.slots = c.take<uint4>(L->experts);
  s.stage_xm = c.take<uint32_t>(T * decode_mfma_stage_words(L->hidden));
  s.stage_xr = c.take<uint32_t>(T * decode_runs_stage_words(L->hidden));
  s.shared_gu = c.take<float>(L->shared_intermediate
                                  ? decode_shared_partial_floats(L->hidden, L->shared_intermediate)
                                  : 1);
  const int sq = L->shared_quant ? L->shared_quant : INFERNO_Q8_0;
  const int sdq = L->shared_down_quant ? L->shared_down_quant : INFERNO_Q8_0;
  // (only batches that can take the grouped GEMMs: a decode call carries no
  // f16 copy of the shared expert)
  const bool blas = lib && L->shared_intermediate && T * L->top_k >= kPrefillMinAssignments &&
                    dense_blas_fits(sq, sdq, T, L->hidden, L->shared_intermediate);
  s.blas = blas ? static_cast<void*>(c.take<unsigned char>(
                      dense_blas_workspace_bytes(T, L->hidden, L->shared_intermediate)))
                : nullptr;
  const bool rblas = lib && router_blas_fits(T, L->hidden, L->experts);
  s.rblas = rblas ? static_cast<void*>(c.take<unsigned char>(
                        router_blas_workspace_bytes(T, L->hidden, L->experts)))
                  : nullptr;
  s.blas_lib = (blas || rblas) ? static_cast<void*>(c.take<unsigned char>(
                                     blas_lib_workspace_bytes()))
                               : nullptr;
  return s;
}
}  // namespace

namespace {
size_t layer_workspace_bytes(const inferno_moe_layer* layer, size_t T, bool lib) {
  if (!layer) return 0;
  Carver c{nullptr};
  carve_layer(c, layer, T, lib);
  return c.used;
}
}  // namespace

size_t inferno_moe_layer_workspace_bytes(const inferno_moe_layer* layer, size_t T) {
  return layer_workspace_bytes(layer, T, true);
}

namespace {
int layer_forward(void* stream, const inferno_moe_layer* L, const void* x, int x_dtype,
                  const float* residual, size_t T, float* out, uint32_t* expert_ids_out,
                  float* expert_weights_out, void* workspace, size_t workspace_bytes,
                  const float* logits_ready, bool lib = true);
}  // namespace

int inferno_moe_layer_forward(void* stream, const inferno_moe_layer* L, const void* x,
                              int x_dtype, const float* residual, size_t T, float* out,
                              uint32_t* expert_ids_out, float* expert_weights_out,
                              void* workspace, size_t workspace_bytes) {
  return layer_forward(stream, L, x, x_dtype, residual, T, out, expert_ids_out,
                       expert_weights_out, workspace, workspace_bytes, nullptr);
}

namespace {
// True when one token's shared expert runs as assignment k of the run
// decode kernels: a shared expert with the routed formats and width (the
// Laguna XS layer).
bool layer_shared_slot(const inferno_moe_layer* L, size_t T, int x_dtype) {
  const size_t Is = L->shared_intermediate;
  const int sq = L->shared_quant ? L->shared_quant : INFERNO_Q8_0;
  const int sdq = L->shared_down_quant ? L->shared_down_quant : INFERNO_Q8_0;
  return Is != 0 && Is == L->intermediate && sq == L->quant && sdq == L->down_quant &&
         decode_shared_slot_supported(T, L->top_k, L->experts, L->hidden, L->intermediate,
                                      x_dtype, L->quant, L->down_quant);
}

// True when the layer forward takes the fused decode launches for T tokens.
bool layer_takes_decode(const inferno_moe_layer* L, size_t T, int x_dtype) {
  const size_t Is = L->shared_intermediate;
  const int sq = L->shared_quant ? L->shared_quant : INFERNO_Q8_0;
  const int sdq = L->shared_down_quant ? L->shared_down_quant : INFERNO_Q8_0;
  const bool shared_q8 = Is == 0 || (sq == INFERNO_Q8_0 && sdq == INFERNO_Q8_0);
  if (layer_shared_slot(L, T, x_dtype)) return true;
  return decode_supported(T, L->top_k, L->experts, L->hidden, L->intermediate, Is, x_dtype,
                          L->quant, L->down_quant) &&
         shared_q8 &&
         (T == 1 || !use_mfma(L->quant, L->down_quant, T, L->top_k, L->experts, L->hidden,
                              L->intermediate, Is));
}

// logits_ready: the tokens' router logits [T, E], already formed (the
// stack's fused RMSNorm -> router launch); only the decode path takes them
int layer_forward(void* stream, const inferno_moe_layer* L, const void* x, int x_dtype,
                  const float* residual, size_t T, float* out, uint32_t* expert_ids_out,
                  float* expert_weights_out, void* workspace, size_t workspace_bytes,
                  const float* logits_ready, bool lib) {
  clear_error();
  INF_CHECK_ARG(L != nullptr, "null layer");
  const size_t H = L->hidden, E = L->experts, I = L->intermediate, k = L->top_k;
  int st = validate_moe(L->quant, L->down_quant, L->gate_bytes, L->up_bytes, L->down_bytes, T, k,
                        E, H, I);
  if (st) return st;
  INF_CHECK_ARG(x_dtype == INFERNO_F32 || x_dtype == INFERNO_BF16, "x dtype must be F32 or BF16");
  INF_CHECK_ARG(L->score_fn == INFERNO_SCORE_SIGMOID || L->score_fn == INFERNO_SCORE_SOFTMAX,
                "score_fn must be SIGMOID or SOFTMAX");
  INF_CHECK_ARG(std::isfinite(L->routed_scaling_factor), "routed scaling factor must be finite");
  INF_CHECK_ARG(L->router && L->gate && L->up && L->down && x && out && workspace, "null pointer");
  const size_t Is = L->shared_intermediate;
  const int sq = L->shared_quant ? L->shared_quant : INFERNO_Q8_0;
  const int sdq = L->shared_down_quant ? L->shared_down_quant : INFERNO_Q8_0;
  if (Is) {
    INF_CHECK_ARG(L->shared_gate && L->shared_up && L->shared_down, "null shared expert pointer");
    INF_CHECK_ARG(sq == INFERNO_Q8_0 || is_routed_quant(sq),
                  "shared gate/up must be Q8_0, Q2_K, Q3_K or Q4_K");
    INF_CHECK_ARG(sdq == INFERNO_Q8_0 || is_down_quant(sdq),
                  "shared down must be Q8_0, Q2_K, Q3_K, Q4_K or Q6_K");
    INF_CHECK_ARG(Is % kKBlock == 0, "shared intermediate must be a multiple of 256");
    if ((st = check_len("shared gate", L->shared_gate_bytes, 1, matrix_bytes(sq, Is, H))))
      return st;
    if ((st = check_len("shared up", L->shared_up_bytes, 1, matrix_bytes(sq, Is, H))))
      return st;
    if ((st = check_len("shared down", L->shared_down_bytes, 1, matrix_bytes(sdq, H, Is))))
      return st;
  }
  // the fused decode launches and the dense MFMA shared GEMMs take a Q8_0
  // shared expert (the GLM and Laguna S layers); other formats (Laguna XS:
  // Q4_K gate/up, Q4_K or Q6_K down) run the shared expert on the GEMV kernels
  const bool shared_q8 = Is == 0 || (sq == INFERNO_Q8_0 && sdq == INFERNO_Q8_0);
  size_t need = layer_workspace_bytes(L, T, lib);
  if (workspace_bytes < need) {
    set_error("workspace too small: need " + std::to_string(need) + " bytes");
    return INFERNO_ERR_SIZE;
  }
  if (int st_ = require_device()) return st_;
  Carver c{static_cast<char*>(workspace)};
  LayerScratch w = carve_layer(c, L, T, lib);
  hipStream_t s = as_stream(stream);
  uint32_t* ids = expert_ids_out ? expert_ids_out : w.ids;
  float* wts = expert_weights_out ? expert_weights_out : w.weights;
  // the fused decode path below the grouped GEMM's assignment threshold
  // (use_mfma; and for one token); from there the grouped MFMA GEMM reads
  // each expert's weights once for all its tokens
  const bool decode = layer_takes_decode(L, T, x_dtype);
  if (logits_ready && !decode) {
    set_error("precomputed logits need the decode path");
    return INFERNO_ERR_INVALID;
  }
  if (decode) {
    DecodeArgs d{};
    d.T = int(T); d.H = int(H); d.E = int(E); d.I = int(I); d.k = int(k); d.Is = int(Is);
    d.score_fn = L->score_fn; d.norm = L->norm_topk_prob; d.scale = L->routed_scaling_factor;
    d.x = x; d.x_dtype = x_dtype; d.router = L->router; d.bias = L->router_bias;
    d.gate = static_cast<const uint8_t*>(L->gate);
    d.up = static_cast<const uint8_t*>(L->up);
    d.down = static_cast<const uint8_t*>(L->down);
    d.gate_stride = matrix_bytes(L->quant, I, H);
    d.down_stride = matrix_bytes(L->down_quant, H, I);
    d.sgate = static_cast<const uint8_t*>(L->shared_gate);
    d.sup = static_cast<const uint8_t*>(L->shared_up);
    d.sdown = static_cast<const uint8_t*>(L->shared_down);
    d.residual = residual; d.out = out; d.ids = ids; d.weights = wts;
    d.partials = w.partials; d.stage_x = w.moe.stage_x; d.offsets = w.moe.offsets;
    d.sorted = w.moe.sorted; d.active = w.moe.active; d.stage_h = w.moe.stage_h;
    d.stage_hs = w.stage_hs; d.slots = w.slots; d.stage_xm = w.stage_xm;
    d.stage_xr = w.stage_xr;
    d.shared_gu = w.shared_gu;
    d.ys = w.ys;
    d.y = w.moe.y;
    d.logits_ready = logits_ready;
    d.shared_slot = layer_shared_slot(L, T, x_dtype) ? 1 : 0;
    d.h_quant = L->down_quant;
    return launch_decode_layer(s, d, L->quant);
  }
  // bf16 tokens of a large batch: the logits as one library GEMM over the
  // router's three bf16 terms
  const bool router_blas = w.rblas != nullptr && w.blas_lib != nullptr &&
                           router_blas_takes(T, H, E, x_dtype);
  const int parts = router_blas ? 1 : router_logit_parts(T, H, E, x_dtype);
  const bool mfma_path = use_mfma(L->quant, L->down_quant, T, k, E, H, I, Is);
  // the shared expert on the dense MFMA GEMMs when its formats have them
  // (Q8_0; the Laguna XS Q4_K gate/up with Q4_K or Q6_K down), else on the
  // GEMV kernels
  const bool shared_gemm = Is && prefill_dense_supported(sq, sdq, H, Is);
  // x in f16 for the grouped GEMMs (moe.stage_x, which a shared expert on
  // the GEMVs stages into first); fp32 tokens over K chunks get it from the
  // logits launch (INFERNO_ROUTER_X16=0: its own launch)
  uint16_t* x16 = reinterpret_cast<uint16_t*>(w.moe.stage_x);
  const bool x16_by_router = mfma_path && !(Is && !shared_gemm) &&
                             router_writes_x16(T, H, E, x_dtype, parts) &&
                             !switch_off("INFERNO_ROUTER_X16");
  if (router_blas) {
    if ((st = launch_router_blas(s, static_cast<const uint16_t*>(x), L->router, T, H, E,
                                 w.logits, w.rblas, w.blas_lib)))
      return st;
  } else if ((st = launch_router_logit_parts(s, x, x_dtype, L->router, T, H, E, w.logits, parts,
                                             x16_by_router ? x16 : nullptr))) {
    return st;
  }
  if ((st = launch_router_topk(s, w.logits, L->router_bias, T, E, k, L->score_fn,
                               L->norm_topk_prob, L->routed_scaling_factor, ids, wts, nullptr,
                               parts)))
    return st;
  // shared expert on the GEMV kernels: gate/up from x staged in moe.stage_x
  // (h staged for the down when its format has a packed-f16 kernel), down
  // with the routed rows and the residual folded in
  const bool sdq_staged = dot2_supported(sdq);
  auto shared_gate_up_gemv = [&](bool staged_ready) {
    return launch_gemv_gate_up_dense(s, sq, L->shared_gate, L->shared_up, x, x_dtype,
                                     w.moe.stage_x, staged_ready, T, H, Is, w.hs,
                                     sdq_staged ? w.stage_hs : nullptr);
  };
  auto shared_down_gemv = [&] {
    return launch_gemv_down_dense(s, sdq, L->shared_down, w.hs, sdq_staged ? w.stage_hs : nullptr,
                                  sdq_staged, w.moe.y, k, nullptr, residual, T, Is, H, out);
  };
  if (mfma_path) {
    // a shared expert on the GEMVs runs its gate/up first, while moe.stage_x
    // still holds its staging (the f16 copy of x reuses it)
    if (Is && !shared_gemm && (st = shared_gate_up_gemv(false))) return st;
    // x in f16 once for the routed and the shared expert GEMMs
    if (!x16_by_router && (st = launch_to_f16(s, x, x_dtype, T, H, x16))) return st;
    if ((st = run_routed(s, L->quant, L->down_quant, L->gate, L->up, L->down, x, x_dtype, ids,
                         wts, T, k, E, H, I, w.moe, false, true, x16, true)))
      return st;
    if (Is && !shared_gemm) return shared_down_gemv();
    if (shared_gemm &&
        (st = launch_prefill_dense(s, sq, sdq, L->shared_gate, L->shared_up, L->shared_down, x16,
                                   T, H, Is, reinterpret_cast<uint16_t*>(w.hs), w.ys, w.blas,
                                   w.blas_lib)))
      return st;
    return launch_prefill_combine(s, w.moe.y, Is ? w.ys : nullptr, residual, T, k, H, out);
  }
  // x is staged once for the routed and the shared gate/up
  if ((st = launch_stage(s, x, x_dtype, T, H, w.moe.stage_x))) return st;
  if ((st = run_routed(s, L->quant, L->down_quant, L->gate, L->up, L->down, x, x_dtype, ids, wts,
                       T, k, E, H, I, w.moe, true, mfma_path)))
    return st;
  if (Is) {
    if ((st = shared_gate_up_gemv(true))) return st;
    return shared_down_gemv();
  }
  return launch_topk_combine(s, nullptr, residual, w.moe.y, nullptr, T, H, k, out);
}
}  // namespace

// ------------------------------------------------- layer, no allocation

namespace {
// Device-resident scratch for inferno_moe_layer_forward_noalloc: one copy per
// GPU (each device's code object holds its own), kept until the process ends.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of the current device's `scratch` (host code may not use
// the array's name as an address); looked up once per device.
int scratch_ptr(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("no-alloc layer: cannot query the current device");
    return INFERNO_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error(std::string("no-alloc layer: hipGetSymbolAddress(scratch) failed: ") +
                hipGetErrorString(e));
      return INFERNO_ERR_DEVICE;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return INFERNO_OK;
}
}  // namespace

size_t inferno_moe_layer_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

int inferno_moe_layer_forward_noalloc(void* stream, const inferno_moe_layer* L, const void* x,
                                      int x_dtype, const float* residual, size_t T, float* out,
                                      uint32_t* expert_ids_out, float* expert_weights_out) {
  clear_error();
  INF_CHECK_ARG(L != nullptr, "null layer");
  // no library GEMMs here (hipBLASLt allocates): the shared expert and the
  // router stay on the grouped kernels
  const size_t need = layer_workspace_bytes(L, T, false);
  if (need > kNoAllocScratchBytes) {
    set_error("no-alloc layer: these shapes need " + std::to_string(need) +
              " bytes of scratch, above the fixed maximum of " +
              std::to_string(kNoAllocScratchBytes) + " (use inferno_moe_layer_forward with a "
              "caller workspace)");
    return INFERNO_ERR_SIZE;
  }
  if (int st_ = require_device()) return st_;
  void* ws = nullptr;
  int st = scratch_ptr(&ws);
  if (st) return st;
  return layer_forward(stream, L, x, x_dtype, residual, T, out, expert_ids_out,
                       expert_weights_out, ws, kNoAllocScratchBytes, nullptr, false);
}

// ------------------------------------------------------------- stack

namespace {
struct StackScratch {
  void* normed;      // [T, H] activations of the current layer (fp32 or bf16)
  float* logits;     // [T, E] router logits of the fused RMSNorm -> router launch
  float* stream[2];  // [T, H] residual stream between layers (ping-pong)
  void* layer_ws;    // the layers' own workspace (the largest one)
  size_t layer_ws_bytes;
};
StackScratch carve_stack(Carver& c, const inferno_moe_layer* layers, size_t n, size_t T) {
  StackScratch s;
  const size_t H = n ? layers[0].hidden : 0;
  s.normed = c.take<float>(T * H);
  size_t E = 0;
  for (size_t l = 0; l < n; ++l) E = std::max(E, layers[l].experts);
  s.logits = c.take<float>(T * E);
  // layer l (but the last) writes stream[l & 1]
  s.stream[0] = c.take<float>(n > 1 ? T * H : 0);
  s.stream[1] = c.take<float>(n > 2 ? T * H : 0);
  size_t most = 0;
  for (size_t l = 0; l < n; ++l) most = std::max(most, inferno_moe_layer_workspace_bytes(&layers[l], T));
  s.layer_ws = c.take<char>(most);
  s.layer_ws_bytes = most;
  return s;
}
}  // namespace

size_t inferno_moe_stack_workspace_bytes(const inferno_moe_layer* layers, size_t n_layers,
                                         size_t T) {
  if (!layers || n_layers == 0) return 0;
  Carver c{nullptr};
  carve_stack(c, layers, n_layers, T);
  return c.used;
}

int inferno_moe_stack_forward(void* stream, const inferno_moe_layer* layers, size_t n_layers,
                              const float* const* norm_weights, float eps, int act_dtype,
                              const float* hidden, size_t T, float* out,
                              uint32_t* expert_ids_out, void* workspace, size_t workspace_bytes) {
  clear_error();
  INF_CHECK_ARG(layers != nullptr && norm_weights != nullptr && n_layers > 0, "empty layer stack");
  INF_CHECK_ARG(act_dtype == INFERNO_F32 || act_dtype == INFERNO_BF16,
                "activation dtype must be F32 or BF16");
  INF_CHECK_ARG(eps >= 0.f && std::isfinite(eps), "rms_norm eps must be finite and >= 0");
  INF_CHECK_ARG(hidden && out && workspace && T > 0, "null pointer or no tokens");
  INF_CHECK_ARG(hidden != out, "the stack output must not alias its input");
  const size_t H = layers[0].hidden;
  for (size_t l = 0; l < n_layers; ++l) {
    INF_CHECK_ARG(layers[l].hidden == H, "every layer of a stack must have the same hidden size");
    INF_CHECK_ARG(norm_weights[l] != nullptr, "null RMSNorm weight");
  }
  const size_t need = inferno_moe_stack_workspace_bytes(layers, n_layers, T);
  if (workspace_bytes < need) {
    set_error("workspace too small: need " + std::to_string(need) + " bytes");
    return INFERNO_ERR_SIZE;
  }
  if (int st_ = require_device()) return st_;
  Carver c{static_cast<char*>(workspace)};
  StackScratch w = carve_stack(c, layers, n_layers, T);
  hipStream_t s = as_stream(stream);
  const float* r = hidden;
  size_t id_off = 0;
  for (size_t l = 0; l < n_layers; ++l) {
    float* next = l + 1 == n_layers ? out : w.stream[l & 1];
    // INFERNO_STACK_FUSED_ROUTER=1: for decode layers, RMSNorm and the
    // router logits in one launch (the layer's route launch then only stages
    // x and runs the shared gate/up). Off by default: measured slower on the
    // c4 stack (189.9-190.1 against 184.4-185.8 us per step), since every
    // workgroup of that launch forms the normalised row before its logits
    const inferno_moe_layer* L = &layers[l];
    const bool fused = switch_on("INFERNO_STACK_FUSED_ROUTER") &&
                       layer_takes_decode(L, T, act_dtype) &&
                       norm_router_supported(T, H, L->experts, 0);
    int st = fused ? launch_norm_router(s, r, norm_weights[l], eps, L->router, nullptr, T, H,
                                        L->experts, 0, 0, 0, 1.f, act_dtype, w.normed, w.logits,
                                        nullptr, nullptr, nullptr)
                   : launch_rms_norm(s, r, norm_weights[l], T, H, eps, w.normed, act_dtype);
    if (st) return st;
    st = layer_forward(stream, L, w.normed, act_dtype, r, T, next,
                       expert_ids_out ? expert_ids_out + id_off : nullptr, nullptr, w.layer_ws,
                       w.layer_ws_bytes, fused ? w.logits : nullptr);
    if (st) {
      set_error("layer " + std::to_string(l) + ": " + g_last_error);
      return st;
    }
    id_off += T * layers[l].top_k;
    r = next;
  }
  return INFERNO_OK;
}

// ------------------------------------------------------ synthetic data

int inferno_synth_normal(void* stream, uint64_t seed, float stddev, size_t n, int dtype,
                         void* out) {
  clear_error();
  INF_CHECK_ARG(dtype == INFERNO_F32 || dtype == INFERNO_BF16, "dtype must be F32 or BF16");
  INF_CHECK_ARG(n == 0 || out, "null pointer");
  if (int st_ = require_device()) return st_;
  return launch_synth_normal(as_stream(stream), seed, stddev, n, dtype, out);
}

int inferno_synth_normal_host(uint64_t seed, float stddev, size_t n, float* out) {
  clear_error();
  INF_CHECK_ARG(n == 0 || out, "null pointer");
  for (size_t i = 0; i < n; ++i) out[i] = stddev * synth_normal(seed, i);
  return INFERNO_OK;
}

int inferno_quantize_rows_host(int quant, const float* x, size_t rows, size_t cols, void* out) {
  clear_error();
  INF_CHECK_ARG(block_bytes(quant) > 0, "unknown quant kind");
  const size_t bv = size_t(block_values(quant)), bb = size_t(block_bytes(quant));
  INF_CHECK_ARG(cols % bv == 0, "cols must be a multiple of the block size");
  auto* o = static_cast<uint8_t*>(out);
  for (size_t r = 0; r < rows; ++r)
    for (size_t b = 0; b < cols / bv; ++b)
      quantize_block(quant, x + r * cols + b * bv, o + (r * (cols / bv) + b) * bb);
  return INFERNO_OK;
}

int inferno_synth_quantized(void* stream, int quant, uint64_t seed, float stddev, size_t rows,
                            size_t cols, void* out) {
  clear_error();
  INF_CHECK_ARG(block_bytes(quant) > 0, "unknown quant kind");
  INF_CHECK_ARG(cols % size_t(block_values(quant)) == 0, "cols must be a multiple of the block size");
  if (int st_ = require_device()) return st_;
  return launch_synth_quantized(as_stream(stream), quant, seed, stddev, rows, cols, out);
}

int inferno_synth_quantized_host(int quant, uint64_t seed, float stddev, size_t rows, size_t cols,
                                 void* out) {
  clear_error();
  INF_CHECK_ARG(block_bytes(quant) > 0, "unknown quant kind");
  const size_t bv = size_t(block_values(quant)), bb = size_t(block_bytes(quant));
  INF_CHECK_ARG(cols % bv == 0, "cols must be a multiple of the block size");
  auto* o = static_cast<uint8_t*>(out);
  float x[256];
  for (size_t r = 0; r < rows; ++r)
    for (size_t b = 0; b < cols / bv; ++b) {
      for (size_t v = 0; v < bv; ++v) x[v] = stddev * synth_normal(seed, r * cols + b * bv + v);
      quantize_block(quant, x, o + (r * (cols / bv) + b) * bb);
    }
  return INFERNO_OK;
}

}  // extern "C"
