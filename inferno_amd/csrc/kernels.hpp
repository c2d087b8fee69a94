// Internal launcher declarations shared by the kernel files and the C ABI.
#pragma once
#include <algorithm>

#include "common.hpp"

namespace inferno {

int launch_dequant(hipStream_t s, int quant, const void* blocks, size_t n_blocks, float* out);
int launch_synth_normal(hipStream_t s, uint64_t seed, float stddev, size_t n, int dtype,
                        void* out);
int launch_synth_quantized(hipStream_t s, int quant, uint64_t seed, float stddev, size_t rows,
                           size_t cols, void* out);

int launch_router_logits(hipStream_t s, const void* x, int x_dtype, const float* w, size_t T,
                         size_t H, size_t E, float* logits);
int launch_router_topk(hipStream_t s, const float* logits, const float* bias, size_t T, size_t E,
                       size_t k, int score_fn, int norm, float scale, uint32_t* ids,
                       float* weights, uint32_t* token_idx, int parts = 1);
// Router logits of bf16 tokens split over K chunks for small batches (more
// workgroups): router_logit_parts() chunks of partials [parts][T][E], summed
// by launch_router_topk(..., parts); router_logit_parts_max() bounds it for
// any token type and switch setting (workspace sizing).
int router_logit_parts(size_t T, size_t H, size_t E, int x_dtype);
int router_logit_parts_max(size_t T, size_t H, size_t E);
// True when the K-chunk logits launch of fp32 tokens (parts > 1) can also
// write x in f16 (the grouped GEMMs' copy, as launch_to_f16 writes it).
bool router_writes_x16(size_t T, size_t H, size_t E, int x_dtype, int parts);
int launch_router_logit_parts(hipStream_t s, const void* x, int x_dtype, const float* w, size_t T,
                              size_t H, size_t E, float* parts_out, int parts,
                              uint16_t* x16 = nullptr);

// plan: also write the grouped GEMM's tile lists (routing_dev.hpp PlanOut)
int launch_dispatch(hipStream_t s, const uint32_t* ids, size_t T, size_t k, size_t E,
                    uint32_t* offsets, uint32_t* sorted, uint32_t* active,
                    const PlanOut* plan = nullptr);

// GEMV stages. Packed-f16 formats (Q2_K, Q3_K, Q4_K, Q8_0) stage their
// activation rows into `stage` (gemv_stage_bytes bytes) first; with
// staged_ready the rows are already there (the layer stages x once for the
// routed and the shared gate/up).
size_t gemv_stage_bytes(int quant, size_t rows, size_t K, int x_dtype);
int launch_gemv_gate_up_routed(hipStream_t s, int quant, const void* gate, const void* up,
                               const void* x, int x_dtype, uint32_t* stage, bool staged_ready,
                               const uint32_t* offsets, const uint32_t* sorted,
                               const uint32_t* active, const float* route_w, size_t T, size_t k,
                               size_t E, size_t H, size_t I, float* h_out,
                               uint32_t* h_staged_out);
int launch_gemv_down_routed(hipStream_t s, int quant, const void* down, const float* h,
                            uint32_t* stage, bool staged_ready, const uint32_t* offsets,
                            const uint32_t* sorted, const uint32_t* active, size_t T, size_t k,
                            size_t E, size_t H, size_t I, float* y_out);
int launch_gemv_gate_up_dense(hipStream_t s, int quant, const void* gate, const void* up,
                              const void* x, int x_dtype, uint32_t* stage, bool staged_ready,
                              size_t T, size_t H, size_t I, float* out, uint32_t* out_staged);
int launch_gemv_down_dense(hipStream_t s, int quant, const void* w, const float* input,
                           uint32_t* stage, bool staged_ready, const float* yk, size_t k,
                           const float* res_a, const float* res_b, size_t T, size_t In, size_t O,
                           float* out);

int launch_topk_combine(hipStream_t s, const float* shared, const float* residual,
                        const float* expert_outputs, const float* expert_weights, size_t T,
                        size_t H, size_t k, float* out);
int launch_index_add_combine(hipStream_t s, const float* acc, const uint32_t* token_idx,
                             const float* expert_outputs, const float* expert_weights, size_t T,
                             size_t H, size_t A, float* out);
int launch_gather(hipStream_t s, const float* x, const uint32_t* token_idx, size_t T, size_t H,
                  size_t A, float* out);
// out is fp32 or bf16 (out_dtype INFERNO_F32 / INFERNO_BF16)
int launch_rms_norm(hipStream_t s, const float* x, const float* w, size_t rows, size_t H,
                    float eps, void* out, int out_dtype = INFERNO_F32);

// RMSNorm -> router logits (-> top-k when ids is not null) in one launch
// (norm_router.hip); tickets: T words, zero on entry, left zero.
bool norm_router_supported(size_t T, size_t H, size_t E, size_t k);
int launch_norm_router(hipStream_t s, const float* x, const float* norm_w, float eps,
                       const float* router, const float* bias, size_t T, size_t H, size_t E,
                       size_t k, int score_fn, int norm, float scale, int act_dtype, void* normed,
                       float* logits, uint32_t* tickets, uint32_t* ids, float* weights);

}  // namespace inferno
