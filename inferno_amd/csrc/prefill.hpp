// Prefill (many tokens per expert): grouped dequant-GEMM on MFMA (prefill.hip).
#pragma once
#include "common.hpp"

namespace inferno {

// Weight kinds the MFMA GEMM dequantises (routed Q2_K/Q3_K/Q4_K, Q8_0 dense).
bool prefill_supported(int quant);
// True when the routed layer (gate/up kind, down kind, shapes) has the MFMA path.
bool prefill_routed_supported(int quant, int down_quant, size_t H, size_t I, size_t E);
// Assignments from which the routed layer takes the MFMA path (measured
// crossovers against the several-token decode kernels, with the shared
// expert of the MFMA path on the library GEMMs; INFERNO_PREFILL_MIN_ASSIGNMENTS
// overrides both). Without a shared expert (c1): 32 assignments 55.7 against
// 63.2 us on the decode kernels, 48 70.9 against 67.2, 64 82.5 against
// 71.5. With one (c2, c4): 48-56 decode (c2 T = 6 0.262 against 0.313 ms),
// 64 even (c2 T = 8 0.335 against 0.338), 70 and up MFMA (c4 T = 7 1.030
// against 1.015, T = 8 1.151 against 1.050, c2 T = 10 0.408 against 0.378).
constexpr size_t kPrefillMinAssignments = 48;
constexpr size_t kPrefillMinAssignmentsShared = 66;

// 32-bit words of the routed planner's scratch (tile lists and counts).
size_t prefill_plan_words(size_t A, size_t E);
// The tile lists inside that scratch, for the dispatch launch to fill
// (launch_dispatch with a plan) before launch_prefill_gate_up reads them.
PlanOut prefill_plan_out(uint32_t* plan, size_t A, size_t E);

// x [rows, K] (bf16 or fp32) -> f16 [rows, K], round to nearest even.
int launch_to_f16(hipStream_t s, const void* x, int x_dtype, size_t rows, size_t K, uint16_t* out);

struct PrefillRouted {
  int quant, down_quant;
  const void *gate, *up, *down;  // packed experts [E][rows][blocks]
  const uint16_t* x16;           // [T, H] f16
  const uint32_t* offsets;       // [E+1] from the dispatch
  const uint32_t* sorted;        // [A]
  const uint32_t* active;        // [E+1]
  const float* weights;          // [A] routing weights (folded into h)
  size_t T, k, E, H, I;
  uint16_t* h16;                 // [A, I] SwiGLU intermediate, f16
  float* y;                      // [A, H] per-assignment down rows
  uint32_t* plan;                // prefill_plan_words(A, E)
  // most rows one expert can take: T when every token's ids are distinct
  // (the layer's own top-k), 0 when unknown (caller ids: up to A)
  size_t max_rows;
};

// Routed gate/up (+SwiGLU, routing weight) over the dispatch groups: plans
// the expert tiles, then the GEMM; writes h16.
int launch_prefill_gate_up(hipStream_t s, const PrefillRouted& p);
// Routed down over the same tiles (after launch_prefill_gate_up): writes y.
int launch_prefill_down(hipStream_t s, const PrefillRouted& p);

// True when a dense (shared) expert of these formats and widths has the
// MFMA GEMMs (gate/up Q2_K/Q3_K/Q4_K/Q8_0, down also Q6_K).
bool prefill_dense_supported(int quant, int down_quant, size_t H, size_t Is);
// Dense expert over all T rows (gate/up format quant, down down_quant):
// h16 = silu(x G^T) * (x U^T); ys = h16 D^T.
// The Q8_0 shared expert of a batch of T tokens on library GEMMs (f16
// weights expanded per call, fp32 accumulation): taken by
// launch_prefill_dense when it is given a workspace of
// dense_blas_workspace_bytes and dense_blas_takes holds.
// dense_blas_fits: the shapes the path covers (the workspace is sized by it);
// dense_blas_takes: those, unless switched off.
bool dense_blas_fits(int quant, int down_quant, size_t T, size_t H, size_t Is);
bool dense_blas_takes(int quant, int down_quant, size_t T, size_t H, size_t Is);
size_t dense_blas_workspace_bytes(size_t T, size_t H, size_t Is);
int launch_dense_blas(hipStream_t s, const void* gate, const void* up, const void* down,
                      const uint16_t* x16, size_t T, size_t H, size_t Is, float* ys, void* ws,
                      void* lib_ws);
// The library's own workspace, shared by the calls of one stream.
size_t blas_lib_workspace_bytes();
// Router logits of T bf16 tokens as three bf16 library GEMMs over the exact
// three-term split of the fp32 router (fp32 accumulation): logits [T][E].
bool router_blas_fits(size_t T, size_t H, size_t E);
bool router_blas_takes(size_t T, size_t H, size_t E, int x_dtype);
size_t router_blas_workspace_bytes(size_t T, size_t H, size_t E);
int launch_router_blas(hipStream_t s, const uint16_t* x, const float* w, size_t T, size_t H,
                       size_t E, float* logits, void* terms_ws, void* lib_ws);
int launch_prefill_dense(hipStream_t s, int quant, int down_quant, const void* gate,
                         const void* up, const void* down, const uint16_t* x16, size_t T,
                         size_t H, size_t Is, uint16_t* h16, float* ys,
                         void* blas_ws = nullptr, void* lib_ws = nullptr);

// out = (residual + ys) + sum over ranks of y[t*k + r] (rank order); residual,
// ys may be null.
int launch_prefill_combine(hipStream_t s, const float* y, const float* ys, const float* residual,
                           size_t T, size_t k, size_t H, float* out);

}  // namespace inferno
