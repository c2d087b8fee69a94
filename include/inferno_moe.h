/*
 * inferno_moe.h — C ABI of the MI355X (gfx950) routed Mixture-of-Experts layer.
 *
 * Drop-in boundary for the routed-expert forward of nektarlabs/inferno. The
 * reference exposes it as methods of the Rust `trait Backend`
 * (crates/backend/src/backend.rs:711); each entry point below names the trait
 * method (file:line) it replaces. A Rust `Backend` implementation binds these
 * symbols through `extern "C"` declarations.
 *
 * Conventions
 *  - Every pointer argument that names a tensor is a DEVICE pointer owned by
 *    the caller, except where a function is marked _host.
 *  - `stream` is a hipStream_t (NULL = the default stream). All work is
 *    stream-ordered; no function synchronises the stream except
 *    inferno_stream_synchronize.
 *  - Return value: INFERNO_OK (0), INFERNO_UNSUPPORTED (1, the reference's
 *    `Ok(None)`: the caller may fall back; returned by every entry point that
 *    launches work when the process sees no HIP device, after argument
 *    validation, as backend.rs:6688-6692 returns Ok(None) without a native
 *    device) or a negative error (the reference's `Err(Error::Backend{..})`),
 *    with a message retrievable via inferno_last_error() on the calling
 *    thread. Nothing throws across the ABI.
 *  - Quantised expert tensors are the exact GGUF byte layouts: a 3-D tensor
 *    [E][rows][cols/256] of super-blocks (Q8_0: [E][rows][cols/32] blocks),
 *    expert stride = rows * (cols/values_per_block) * block_bytes. Byte lengths
 *    are validated like crates/backend/src/metal/gguf_moe.rs:241-266.
 */
#ifndef INFERNO_MOE_H
#define INFERNO_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum inferno_status {
  INFERNO_OK = 0,
  INFERNO_UNSUPPORTED = 1,
  INFERNO_ERR_INVALID = -1, /* shape / argument error */
  INFERNO_ERR_SIZE = -2,    /* byte length or workspace too small */
  INFERNO_ERR_DEVICE = -3   /* HIP runtime error */
};

/* Quantisation kinds use the ggml type ids (crates/gguf/src/lib.rs GgmlType). */
enum inferno_quant {
  INFERNO_Q8_0 = 8,
  INFERNO_Q2_K = 10,
  INFERNO_Q3_K = 11,
  INFERNO_Q4_K = 12,
  INFERNO_Q6_K = 14
};

enum inferno_dtype { INFERNO_F32 = 0, INFERNO_BF16 = 1 };

enum inferno_score_fn { INFERNO_SCORE_SIGMOID = 0, INFERNO_SCORE_SOFTMAX = 1 };

/* Last error message of the calling thread ("" if none). */
const char* inferno_last_error(void);

/* Bytes per block / values per block of a quant kind; -1 if unknown.
 * Replaces GgufQuantBlockKind::block_byte_len / values_per_block
 * (crates/gguf/src/lib.rs:1199-1215). Host-only, no GPU needed. */
int inferno_block_bytes(int quant);
int inferno_block_values(int quant);

/* Waits for `stream`. */
int inferno_stream_synchronize(void* stream);

/* ---------------------------------------------------------------- dequant */

/* out[n_blocks * values_per_block] = bit-exact fp32 dequantisation of GGUF
 * blocks. Replaces GgufQuantBlockKind::decode_block
 * (crates/gguf/src/lib.rs:1212-1221, formulas :1226-1499). Non-finite block
 * scales are not rejected on the device: they propagate into the output. */
int inferno_gguf_dequantize(void* stream, int quant, const void* blocks, size_t n_blocks,
                            float* out);

/* ----------------------------------------------------------------- router */

/* logits[T,E] = x[T,H] . w_router[E,H]^T in fp32 (x is f32 or bf16).
 * Replaces the router projection `backend.linear_f32_device(flat_input,
 * prepared.router)` (crates/model/src/laguna/gguf_model.rs:742-748). */
int inferno_router_logits(void* stream, const void* x, int x_dtype, const float* w_router,
                          size_t T, size_t H, size_t E, float* logits);

/* Exact top-k over router logits, one wavefront per token.
 *  sigmoid: score = 1/(1+exp(-l)); selection on score + bias[e];
 *  softmax: score = exp(l - max_l); selection on l + bias[e];
 *  ties on the selection value go to the lower expert id (total order of
 *  f32::total_cmp); weights = unbiased scores in rank order, divided by their
 *  rank-order sum when norm_topk_prob (softmax without norm: by the sum over
 *  all experts), then multiplied by routed_scaling_factor.
 * Outputs are token-major [T*k]: expert_ids, expert_weights, token_indices
 * (token_indices may be NULL). bias may be NULL. E <= 256, k <= 16.
 * Replaces Backend::moe_router_topk_resident_device (backend.rs:2151) and
 * moe_router_topk_device (backend.rs:2140); semantics of
 * crates/model/src/moe_router.rs:835-940 and moe_kernels.metal:115-208. */
int inferno_moe_router_topk(void* stream, const float* logits, const float* bias, size_t T,
                            size_t E, size_t k, int score_fn, int norm_topk_prob,
                            float routed_scaling_factor, uint32_t* expert_ids,
                            float* expert_weights, uint32_t* token_indices);

/* --------------------------------------------------------------- dispatch */

/* Deterministic token->expert dispatch: histogram, exclusive scan, stable
 * scatter. offsets[E+1]; sorted[T*k] = assignment indices (t*k + r) grouped
 * by expert, tokens ascending then rank ascending inside an expert;
 * active[0] = number of experts with at least one assignment, active[1..]
 * = those expert ids ascending (active has E+1 entries).
 * Replaces crates/moe/src/routing.rs:27-85 (build_dispatch_plan) and the
 * atomic, order-nondeterministic laguna_prefill_build_expert_map_kernel
 * (gguf_moe_prefill_kernels.metal:172-254). */
int inferno_moe_dispatch(void* stream, const uint32_t* expert_ids, size_t T, size_t k,
                         size_t E, uint32_t* offsets, uint32_t* sorted, uint32_t* active);

/* --------------------------------------------------------- routed experts */

/* Workspace bytes inferno_gguf_moe needs for these shapes. */
size_t inferno_gguf_moe_workspace_bytes(size_t T, size_t k, size_t E, size_t H, size_t I);

/* Routed-expert forward: out[T,H] = sum_{r<k} W_down[e_{t,r}] .
 * (silu(W_gate[e] x_t) * (W_up[e] x_t) * w_{t,r}), the rank sum in fixed
 * rank order (deterministic, no float atomics).
 * quant: gate/up kind (Q2_K, Q3_K, Q4_K); down_quant: Q2_K, Q3_K, Q4_K, Q6_K.
 * gate/up: E*I rows of H values; down: E*H rows of I values. H and I must be
 * multiples of 256. expert_ids/expert_weights: [T*k] token-major routing from
 * inferno_moe_router_topk. x: [T,H] f32 or bf16.
 * Replaces Backend::laguna_gguf_moe_device (backend.rs:1722, Q2_K/Q3_K) and
 * laguna_xs_gguf_moe_device (backend.rs:1738, Q4_K with Q4_K/Q6_K down). */
int inferno_gguf_moe(void* stream, int quant, int down_quant, const void* gate,
                     size_t gate_bytes, const void* up, size_t up_bytes, const void* down,
                     size_t down_bytes, const void* x, int x_dtype,
                     const uint32_t* expert_ids, const float* expert_weights, size_t T,
                     size_t k, size_t E, size_t H, size_t I, float* out, void* workspace,
                     size_t workspace_bytes);

/* Workspace bytes of a GEMV entry point that reads `rows` activation rows of
 * length K (it stages them as packed f16 pairs before streaming weights):
 * gate/up: rows = T, K = H; down: rows = T*k, K = I; Q8_0 shared gate/up:
 * rows = T, K = H; Q8_0 matvec: rows = T, K = In. */
size_t inferno_gemv_workspace_bytes(size_t rows, size_t K);

/* Stage-level entry points over a dispatch (inferno_moe_dispatch outputs).
 * gate/up: h[a, i] = silu(W_gate[e_a] x_t) * (W_up[e_a] x_t) * w_a for every
 * assignment a = t*k + r, h is [T*k, I] fp32. Replaces
 * Backend::q2_k_multi_expert_gate_up_swiglu_device (backend.rs:1696) for all
 * K-quant kinds. */
int inferno_moe_expert_gate_up_swiglu(void* stream, int quant, const void* gate,
                                      size_t gate_bytes, const void* up, size_t up_bytes,
                                      const void* x, int x_dtype, const uint32_t* offsets,
                                      const uint32_t* sorted, const uint32_t* active,
                                      const float* expert_weights, size_t T, size_t k, size_t E,
                                      size_t H, size_t I, float* h, void* workspace,
                                      size_t workspace_bytes);

/* down: y[a, o] = W_down[e_a] . h[a] for every assignment, y is [T*k, H].
 * Replaces Backend::q2_k_multi_expert_matvec_device (backend.rs:1711). */
int inferno_moe_expert_down(void* stream, int down_quant, const void* down, size_t down_bytes,
                            const float* h, const uint32_t* offsets, const uint32_t* sorted,
                            const uint32_t* active, size_t T, size_t k, size_t E, size_t H,
                            size_t I, float* y, void* workspace, size_t workspace_bytes);

/* --------------------------------------------------------- shared expert */

/* out[T,Is] = silu(W_g x) * (W_u x), Q8_0 weights [Is rows of H].
 * Replaces Backend::q8_0_gate_up_swiglu_device (backend.rs:1578). */
int inferno_q8_0_gate_up_swiglu(void* stream, const void* gate, size_t gate_bytes,
                                const void* up, size_t up_bytes, const void* x, int x_dtype,
                                size_t T, size_t H, size_t Is, float* out, void* workspace,
                                size_t workspace_bytes);

/* out[T,O] = residual_a + residual_b + W . input, Q8_0 W [O rows of In].
 * residual_a / residual_b may be NULL (zero).
 * Replaces Backend::laguna_q8_0_matvec_add2_device (backend.rs:1682). */
int inferno_q8_0_matvec_add2(void* stream, const void* w, size_t w_bytes, const float* input,
                             const float* residual_a, const float* residual_b, size_t T,
                             size_t In, size_t O, float* out, void* workspace,
                             size_t workspace_bytes);

/* --------------------------------------------------------------- combine */

/* out[T,H] = shared + residual + sum_{r<k} expert_outputs[t*k+r] * w[t*k+r],
 * rank order. shared/residual may be NULL.
 * Replaces Backend::moe_topk_combine_residual_device (backend.rs:2130). */
int inferno_moe_topk_combine_residual(void* stream, const float* shared, const float* residual,
                                      const float* expert_outputs, const float* expert_weights,
                                      size_t T, size_t H, size_t k, float* out);

/* out[T,H] = acc + sum over assignments a with token_indices[a]==t of
 * expert_outputs[a] * w[a], in assignment order (no atomics).
 * Replaces Backend::moe_weighted_index_add_combine(_device)
 * (backend.rs:899, :2120). */
int inferno_moe_weighted_index_add_combine(void* stream, const float* acc,
                                           const uint32_t* token_indices,
                                           const float* expert_outputs,
                                           const float* expert_weights, size_t T, size_t H,
                                           size_t A, float* out);

/* out[A,H] = x[token_indices[a]] (rows with an out-of-range index are zero).
 * Replaces Backend::moe_gather_tokens / moe_gather_rows_device
 * (backend.rs:891, :2106). */
int inferno_moe_gather_tokens(void* stream, const float* x, const uint32_t* token_indices,
                              size_t T, size_t H, size_t A, float* out);

/* out = x / sqrt(mean(x^2) + eps) * w, per row.
 * Replaces Backend::rms_norm (reference_rms_norm_f32, backend.rs:10211). */
int inferno_rms_norm(void* stream, const float* x, const float* w, size_t rows, size_t H,
                     float eps, float* out);

/* Workspace bytes of inferno_rms_norm_router_topk with the top-k (T ticket
 * words, 256-byte aligned). The workspace must be zero-filled before its
 * first use; every call leaves it zero again. */
size_t inferno_rms_norm_router_topk_workspace_bytes(size_t T);

/* RMSNorm -> router logits -> exact top-k of T decode tokens in one launch:
 *   normed[t] = x[t] / sqrt(mean(x[t]^2) + eps) * norm_weight, rounded to
 *     act_dtype (F32 or BF16; bit-identical to inferno_rms_norm's values);
 *   logits_out[t, e] = normed[t] . router[e] (fp32 router [E,H]);
 *   with expert_ids != NULL, the top-k of inferno_moe_router_topk over those
 *   logits into expert_ids / expert_weights [T*k] (bias may be NULL).
 * normed_out may be NULL. H a multiple of 64 up to 8192, E <= 256, k <= 16.
 * Without the top-k the workspace may be NULL. Calls sharing a workspace
 * must not overlap (they share its tickets).
 * Replaces Backend::laguna_xs_rms_norm_router_device (backend.rs:1162;
 * laguna_xs_rms_norm_router_decode_f32_kernel, laguna_xs_kernels.metal:
 * 1274-1365) followed by the decode top-k (laguna_xs_router_top8_decode_f32_kernel,
 * laguna_xs_kernels.metal:1077-1165; Backend::moe_router_topk_resident_device,
 * backend.rs:2151). */
int inferno_rms_norm_router_topk(void* stream, const float* x, const float* norm_weight, float eps,
                                 const float* router, const float* bias, size_t T, size_t H,
                                 size_t E, size_t k, int score_fn, int norm_topk_prob,
                                 float routed_scaling_factor, int act_dtype, void* normed_out,
                                 float* logits_out, uint32_t* expert_ids, float* expert_weights,
                                 void* workspace, size_t workspace_bytes);

/* --------------------------------------------------------- whole layer */

/* One MoE FFN layer as the reference model calls it
 * (crates/model/src/laguna/gguf_model.rs:731-860): router logits -> top-k ->
 * routed experts -> Q8_0 shared expert -> + residual. */
typedef struct inferno_moe_layer {
  size_t hidden;            /* H */
  size_t experts;           /* E */
  size_t intermediate;      /* I (routed) */
  size_t top_k;             /* k */
  int quant;                /* routed gate/up kind */
  int down_quant;           /* routed down kind */
  int score_fn;             /* INFERNO_SCORE_* */
  int norm_topk_prob;       /* renormalise selected weights */
  float routed_scaling_factor;
  const float* router;      /* [E,H] fp32 */
  const float* router_bias; /* [E] or NULL */
  const void* gate;         /* routed packed experts */
  const void* up;
  const void* down;
  size_t gate_bytes, up_bytes, down_bytes;
  size_t shared_intermediate; /* Is; 0 = no shared expert */
  const void* shared_gate;    /* [Is rows of H], shared_quant */
  const void* shared_up;
  const void* shared_down;    /* [H rows of Is], shared_down_quant */
  size_t shared_gate_bytes, shared_up_bytes, shared_down_bytes;
  /* Shared expert formats; 0 = Q8_0 (GLM, Laguna S). Laguna XS: Q4_K gate/up
   * with Q4_K or Q6_K down (crates/model/src/laguna/gguf_model.rs:829-849,
   * laguna_xs_gguf_moe_shared_device backend.rs:1754). */
  int shared_quant;           /* Q8_0, Q2_K, Q3_K or Q4_K */
  int shared_down_quant;      /* Q8_0, Q2_K, Q3_K, Q4_K or Q6_K */
} inferno_moe_layer;

size_t inferno_moe_layer_workspace_bytes(const inferno_moe_layer* layer, size_t T);

/* out[T,H] = residual + routed(x) + shared(x); residual may be NULL.
 * expert_ids_out / expert_weights_out ([T*k], may be NULL) receive the
 * routing for inspection. */
int inferno_moe_layer_forward(void* stream, const inferno_moe_layer* layer, const void* x,
                              int x_dtype, const float* residual, size_t T, float* out,
                              uint32_t* expert_ids_out, float* expert_weights_out,
                              void* workspace, size_t workspace_bytes);

/* inferno_moe_layer_forward without a workspace argument and without any
 * device allocation. No counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Its scratch is a fixed device array of
 * inferno_moe_layer_noalloc_max_bytes() bytes (32 MiB) per GPU, held until
 * the process ends; shapes whose workspace exceeds it return INFERNO_ERR_SIZE
 * (decode up to T = 32 fits the c2 and c4 shapes). It runs no library GEMM
 * (hipBLASLt allocates): the shared expert and the router logits stay on the
 * grouped kernels, so its outputs can differ in the last bits from
 * inferno_moe_layer_forward's on batches where that call takes them (bitwise
 * equal with INFERNO_SHARED_BLAS=0 up to 511 tokens).
 * Every call on one GPU uses that GPU's one array: calls that overlap on a GPU
 * (several streams or threads) race and must be serialised by the caller.
 * Nothing in the scratch needs to start at zero; it keeps the last call's
 * contents. */
size_t inferno_moe_layer_noalloc_max_bytes(void);
int inferno_moe_layer_forward_noalloc(void* stream, const inferno_moe_layer* layer,
                                      const void* x, int x_dtype, const float* residual,
                                      size_t T, float* out, uint32_t* expert_ids_out,
                                      float* expert_weights_out);

/* ---------------------------------------------------------- layer stack */

/* n_layers consecutive MoE layers on one residual stream, as the reference
 * decoder runs its MoE blocks (crates/model/src/laguna/gguf_model.rs:612-657,
 * attention left out): for each layer l,
 *   a_l     = rms_norm(r_l, norm_weights[l], eps)   (backend.rs:10211-10257),
 *             rounded to act_dtype (BF16: nearest even; F32: as is);
 *   r_{l+1} = r_l + routed_l(a_l) + shared_l(a_l)   (inferno_moe_layer_forward,
 *             residual = r_l).
 * hidden = r_0, fp32 [T,H]; out = r_n, fp32 [T,H] (must not alias hidden).
 * norm_weights is a HOST array of n_layers device pointers to fp32 [H].
 * expert_ids_out (may be NULL) receives each layer's routing, layer after
 * layer: [T*k_0] then [T*k_1] ... Every layer must have the same hidden size. */
size_t inferno_moe_stack_workspace_bytes(const inferno_moe_layer* layers, size_t n_layers,
                                         size_t T);
int inferno_moe_stack_forward(void* stream, const inferno_moe_layer* layers, size_t n_layers,
                              const float* const* norm_weights, float eps, int act_dtype,
                              const float* hidden, size_t T, float* out,
                              uint32_t* expert_ids_out, void* workspace, size_t workspace_bytes);

/* ------------------------------------------------------- kernel timing */

/* Measurement hook with no counterpart in the reference (benchmarks only).
 * While enabled, the routed gate/up launch and the routed down launch of
 * inferno_moe_layer_forward / inferno_gguf_moe (fused decode kernels or the
 * stage path) are bracketed with HIP events on the caller's stream, recorded
 * without waiting; inferno_kernel_timing_read waits for a timer's recorded
 * events and sums their elapsed times. The events cost a little per launch:
 * leave timing off outside measurement. */
enum {
  INFERNO_TIMER_GATE_UP = 0,
  INFERNO_TIMER_DOWN = 1,
  INFERNO_TIMER_ROUTE = 2,  /* fused decode: router partials (+ shared gate/up) */
  INFERNO_TIMER_SELECT = 3  /* fused decode: top-k + dispatch */
};
int inferno_kernel_timing_enable(int enable);
/* Waits for the timer's recorded launches, returns their summed
 * milliseconds and count, and resets the timer. */
int inferno_kernel_timing_read(int which, double* total_ms, uint64_t* launches);
/* Copies (NUL-terminated, truncated to len) the label of the last launch a
 * timer measured: "<kind>: <kernel> (<what it streams>)", kind one of
 * mfma, tiles, ring, route, route+shared, select, down8, prefill, stage. */
int inferno_kernel_timing_label(int which, char* buf, size_t len);

/* -------------------------------------------------------- synthetic data */

/* Seeded synthetic inputs (splitmix64 + Box-Muller, counter based, so any
 * element can be generated independently): out[i] = stddev * N(0,1)_i for
 * element i of stream `seed`. *_host run on the CPU and need no GPU. */
int inferno_synth_normal(void* stream, uint64_t seed, float stddev, size_t n, int dtype,
                         void* out);
int inferno_synth_normal_host(uint64_t seed, float stddev, size_t n, float* out);

/* Quantise rows of fp32 values into GGUF blocks (own simple min/max method,
 * not the ggml search; any valid block is acceptable because every consumer
 * decodes the same bytes). */
int inferno_quantize_rows_host(int quant, const float* x, size_t rows, size_t cols, void* out);

/* Generates stddev*N(0,1) weights for `rows` x `cols` (element index
 * row*cols+col of stream `seed`) and quantises them on the device. */
int inferno_synth_quantized(void* stream, int quant, uint64_t seed, float stddev, size_t rows,
                            size_t cols, void* out);
int inferno_synth_quantized_host(int quant, uint64_t seed, float stddev, size_t rows,
                                 size_t cols, void* out);

#ifdef __cplusplus
}
#endif
#endif /* INFERNO_MOE_H */
