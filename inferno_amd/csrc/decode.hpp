// Fused decode path of one MoE layer (decode.hip).
#pragma once
#include <type_traits>

#include "kernels.hpp"

namespace inferno {

struct DecodeArgs {
  int T, H, E, I, k, Is;
  int score_fn, norm;
  float scale;
  const void* x;
  int x_dtype;
  const float* router;  // [E, H] fp32
  const float* bias;    // [E] or null
  const uint8_t* gate;  // routed packed experts
  const uint8_t* up;
  const uint8_t* down;
  size_t gate_stride;   // bytes per expert (gate, up)
  size_t down_stride;   // bytes per expert (down)
  const uint8_t* sgate; // Q8_0 shared expert (null when Is == 0)
  const uint8_t* sup;
  const uint8_t* sdown;
  const float* residual;  // [T, H] or null
  float* out;             // [T, H]
  uint32_t* ids;          // [T*k]
  float* weights;         // [T*k]
  // workspace
  float* partials;        // [n_chunks, T, E]
  uint32_t* stage_x;      // [T, staged_stride(H, x fp32)]
  uint32_t* offsets;      // [E+1]
  uint32_t* sorted;       // [T*k]
  uint32_t* active;       // [E+1]
  uint4* slots;           // [E] per active slot: expert, lo, hi, first assignment
  uint32_t* stage_h;      // [T*k, staged_stride(I, true)]
  uint32_t* stage_hs;     // [T, staged_stride(Is, true)]
  uint32_t* stage_xm;     // [T, decode_mfma_stage_words(H)]: x staged for the MFMA gate/up
  uint32_t* stage_xr;     // [T, decode_runs_stage_words(H)]: x as f16 runs (runs gate/up)
  int xr_quant;           // format whose field offsets the x runs are staged for
  int h_quant;            // format whose field offsets the h runs are staged for (the down's)
  int shared_slot;        // 1: the shared expert (Is == I, the routed formats) is the
                          // token's assignment k, weight 1 (one token, run kernels)
  float* shared_gu;       // [shared_parts][2][Is]: shared gate/up partial sums (MFMA path, T = 1)
  int shared_parts;       // K parts of the shared gate/up in the route launch
  float* ys;              // [T, H]: shared down output (MFMA down path)
  float* y;               // [T*k, H]: down rows per assignment (several-token run kernels)
  int h_mfma;             // gate/up writes h in the MFMA down layout
  // the down launch's first tile per workgroup index (rows, bytes per row;
  // 0: none): the selecting gate/up launch warms its XCD's L2 with it
  int dpf_rows, dpf_row_bytes;
  // the tokens' router logits [T, E] when a previous launch already formed
  // them (the stack's fused RMSNorm -> router launch); the route launch then
  // only stages x and runs the shared gate/up parts
  const float* logits_ready;
  // filled by launch_decode_layer
  int chunk, n_chunks, max_slots, routed_tiles;
};

// True when the fused path covers the layer (token count, format and LDS fit).
bool decode_supported(size_t T, size_t k, size_t E, size_t H, size_t I, size_t Is, int x_dtype,
                      int quant, int down_quant);
int decode_chunk(size_t H);
// True when one token of a layer whose shared expert has the routed formats
// (gate/up quant, down down_quant) and width I runs the shared expert as
// assignment k of the run kernels (DecodeArgs::shared_slot).
bool decode_shared_slot_supported(size_t T, size_t k, size_t E, size_t H, size_t I, int x_dtype,
                                  int quant, int down_quant);
// Words per token of the activation staging used by the MFMA gate/up kernel.
size_t decode_mfma_stage_words(size_t H);
// Words per token of the f16-run staging of x (fp32 tokens: split layout).
size_t decode_runs_stage_words(size_t H);
// Floats of the shared gate/up partial-sum buffer (T = 1 MFMA path).
size_t decode_shared_partial_floats(size_t H, size_t Is);
int launch_decode_layer(hipStream_t s, const DecodeArgs& a, int quant);

// f16-run matrix-core decode kernels (decode_runs.hip): whether they cover a
// shape, and their launchers (one token; gate/up writes h as run rows).
bool runs_gate_up_covers(int quant, int H, int x_dtype);
bool runs_down_covers(int quant, int H, int I, int k);
int launch_gate_up_runs(hipStream_t s, const DecodeArgs& a, int quant);
int launch_down_runs(hipStream_t s, const DecodeArgs& a, int quant);
// Rows per tile and bytes per row of the run down kernel for this layer.
int runs_down_tile_rows(int quant, int H, int I, int k);
int runs_down_row_bytes(int quant, int I);
// The same kernels for T > 1 tokens (no shared expert): gate/up per expert
// tile for all of the expert's tokens, down rows per assignment into a.y.
bool runs_multi_covers(int quant, int H, int I, int x_dtype);
// sel: one token, the selection inside the launch (no select launch before)
int launch_gate_up_runs_multi(hipStream_t s, const DecodeArgs& a, int quant, bool sel = false);
bool runs_multi_sel_covers(int quant, int H, int x_dtype);
int launch_down_runs_multi(hipStream_t s, const DecodeArgs& a, int quant);


}  // namespace inferno
