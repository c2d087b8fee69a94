/*
 * CPU oracle for the routed MoE layer — TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path (inferno_amd/)
 * never links or calls it.
 *
 * It restates, in scalar C++ with fp32 arithmetic and -ffp-contract=off, the
 * semantics of the reference (nektarlabs/inferno, Rust + Metal):
 *   - f16 -> f32 bit conversion           crates/gguf/src/lib.rs:1501-1528
 *   - Q2_K / Q3_K / Q4_K / Q6_K / Q8_0     crates/gguf/src/lib.rs:1226-1499
 *     block dequantisation, same evaluation order
 *   - sigmoid + correction-bias top-k      crates/model/src/moe_router.rs:835-940
 *     with (score desc, id asc) total_cmp ordering, rank-order renorm, x scale
 *   - stable expert-major dispatch         crates/moe/src/routing.rs:27-85
 *   - gate/up SwiGLU with the routing      crates/backend/src/metal/kernels/
 *     weight folded into the intermediate    gguf_moe_kernels.metal:340-400
 *   - down projection summed over ranks    gguf_moe_kernels.metal:457-510
 *   - Q8_0 shared expert + two residuals   q2_kernels.metal:2066-2235
 *   - weighted index-add combine           crates/backend/src/backend.rs:10298-10352
 *   - RMSNorm                              crates/backend/src/backend.rs:10211-10257
 * Softmax scoring has no compute path in the reference (the config validator
 * accepts it, crates/config/src/validation.rs:112-116); it is defined here by
 * closed form: select by (logit + bias) desc / id asc, weight = exp(l - lmax)
 * normalised over the selected experts (norm) or over all experts (no norm).
 *
 * Parity pins (tests/test_oracle.py): the reference's dequant known-answer
 * tests, its router tie-break and dispatch-order tests, its combine KAT,
 * exhaustive f16 conversion against numpy, and fp64 brute force on small
 * matrices. The quantizer is NOT part of the oracle (no reference
 * counterpart exists); the oracle only ever consumes bytes.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* quant kinds: same numbering as include/inferno_moe.h */
enum { ORC_Q2_K = 10, ORC_Q3_K = 11, ORC_Q4_K = 12, ORC_Q6_K = 14, ORC_Q8_0 = 8 };
enum { ORC_SCORE_SIGMOID = 0, ORC_SCORE_SOFTMAX = 1 };

/* All functions return 0 on success, negative on invalid input. */
float oracle_f16_to_f32(uint16_t bits);
int oracle_block_bytes(int quant);
int oracle_block_values(int quant);
int oracle_dequantize(int quant, const uint8_t* blocks, size_t n_blocks, float* out);

/* logits[t,e] = sum_h x[t,h] * w[e,h], sequential fp32 over h */
int oracle_linear(const float* x, const float* w, size_t rows, size_t in_f, size_t out_f,
                  float* out, int threads);

int oracle_router_topk(const float* logits, const float* bias /*nullable*/, size_t T, size_t E,
                       size_t k, int score_fn, int norm, float scale, uint32_t* ids,
                       float* weights);

/* offsets[E+1]; sorted[A] = assignment indices (t*k + r) grouped by expert,
 * tokens ascending then rank ascending inside each expert. */
int oracle_dispatch(const uint32_t* ids, size_t T, size_t k, size_t E, uint32_t* offsets,
                    uint32_t* sorted);

/* Quantised matrix-vector: y[r] = sum_b dot(dequant(row r block b), x[b*256..]).
 * Per-row fp32 sequential sum over blocks of the block dot (fp32 sequential
 * over the block's values). */
int oracle_qmatvec(int quant, const uint8_t* w, size_t rows, size_t cols, const float* x,
                   float* y);

/* Routed experts: y[t,o] = sum_{r<k} W_down[e_{t,r}] . h_{t,r} with
 * h_{t,r}[i] = silu(g) * u * w_{t,r} (Laguna folding).
 * gate/up: E*I rows of H values; down: E*H rows of I values. */
int oracle_moe_routed(int quant, int down_quant, const uint8_t* gate, const uint8_t* up,
                      const uint8_t* down, const float* x, size_t T, size_t H, size_t I,
                      size_t E, size_t k, const uint32_t* ids, const float* weights,
                      float* y, int threads);

/* Q8_0 shared expert: out[t,o] = routed[t,o] + residual[t,o] + W_d . (silu(W_g x) * (W_u x)).
 * routed/residual nullable (treated as zero). */
// Shared expert of any gate/up and down format (Q8_0 for GLM / Laguna S;
// Laguna XS: Q4_K gate/up, Q4_K or Q6_K down): out = routed + residual +
// W_down (silu(W_gate x) * (W_up x)); routed / residual may be NULL.
int oracle_shared_ffn(int quant, int down_quant, const uint8_t* gate, const uint8_t* up,
                      const uint8_t* down, const float* x, size_t T, size_t H, size_t Is,
                      const float* routed, const float* residual, float* out, int threads);
int oracle_shared_q8_0(const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                       const float* x, size_t T, size_t H, size_t Is, const float* routed,
                       const float* residual, float* out, int threads);

int oracle_weighted_index_add_combine(const float* acc, const uint32_t* token_idx,
                                      const float* expert_out, const float* expert_w,
                                      size_t T, size_t H, size_t A, float* out);

int oracle_rms_norm(const float* x, const float* w, size_t rows, size_t H, float eps,
                    float* out);

#ifdef __cplusplus
}
#endif
