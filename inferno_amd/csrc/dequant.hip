// Bit-exact GGUF block dequantisation on the device, plus the synthetic
// normal / quantised-weight generators.
//
// The dequant expressions repeat the evaluation order of
// crates/gguf/src/lib.rs:1226-1499 with floating-point contraction disabled,
// so every output is bit-identical to the reference's CPU decode.
#include "kernels.hpp"
#include "quantize.hpp"

namespace inferno {
namespace {

#pragma clang fp contract(off)

// One thread per output value.
__device__ float dq_q2_k(const uint8_t* b, int v) {
  int h = v >> 7, p = (v >> 5) & 3, s = (v >> 4) & 1, i = v & 15;
  uint8_t sm = b[8 * h + 2 * p + s];
  float d = f16_bits_to_f32(load_le16(b + 80));
  float mn = f16_bits_to_f32(load_le16(b + 82));
  float scale = d * float(sm & 0x0f);
  float min_off = mn * float(sm >> 4);
  uint8_t q = (b[16 + 32 * h + 16 * s + i] >> (2 * p)) & 3;
  return scale * float(q) - min_off;
}

__device__ float dq_q3_k(const uint8_t* b, int v) {
  int g = v >> 4, i = v & 15;
  const uint8_t* sc = b + 96;
  float d = f16_bits_to_f32(load_le16(b + 108));
  uint32_t lmask = 3u << (2 * (g / 4));
  uint32_t nmask = g < 8 ? 0x0fu : 0xf0u;
  uint32_t slow = sc[g % 8], shigh = sc[8 + g % 4];
  uint32_t packed = ((g / 4) & 1) ? ((slow & nmask) | ((shigh & lmask) << 2))
                                  : ((slow & nmask) | ((shigh & lmask) << 4));
  float gs = g < 8 ? d * (float(packed) - 32.0f) : d * (float(packed) / 16.0f - 32.0f);
  float neg = 4.0f * gs;
  int shift = 2 * ((g / 2) & 3);
  float low = float(b[32 + 32 * (g / 8) + 16 * (g & 1) + i] & (3u << shift)) *
              (1.0f / float(1u << shift));
  float sub = (b[16 * (g & 1) + i] & (1u << (g / 2))) == 0 ? neg : 0.0f;
  return gs * low - sub;
}

__device__ float dq_q4_k(const uint8_t* b, int v) {
  int g = v >> 5, i = v & 31;
  const uint8_t* s = b + 4;
  float d = f16_bits_to_f32(load_le16(b));
  float dmin = f16_bits_to_f32(load_le16(b + 2));
  uint32_t sc, m;
  if (g < 4) {
    sc = s[g] & 0x3fu;
    m = s[g + 4] & 0x3fu;
  } else {
    sc = (s[g + 4] & 0x0fu) | ((s[g - 4] >> 6) << 4);
    m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
  }
  uint32_t q = (b[16 + 32 * (g / 2) + i] >> (4 * (g & 1))) & 0x0fu;
  return d * float(sc) * float(q) - dmin * float(m);
}

__device__ float dq_q6_k(const uint8_t* b, int v) {
  int half = v >> 7, quarter = (v >> 5) & 3, i = v & 31;
  float d = f16_bits_to_f32(load_le16(b + 208));
  uint32_t l = b[64 * half + 32 * (quarter & 1) + i];
  l = quarter >= 2 ? (l >> 4) : (l & 15u);
  uint32_t h = (b[128 + 32 * half + i] >> (2 * quarter)) & 3u;
  uint32_t q = l | (h << 4);
  float s = float(int8_t(b[192 + 8 * half + i / 16 + 2 * quarter]));
  return d * s * (float(q) - 32.0f);
}

__device__ float dq_q8_0(const uint8_t* b, int v) {
  float d = f16_bits_to_f32(load_le16(b));
  return d * float(int8_t(b[2 + v]));
}

template <int Q>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* __restrict__ blocks,
                                                      size_t n_values, float* __restrict__ out) {
  constexpr int BV = Q == INFERNO_Q8_0 ? 32 : 256;
  constexpr int BB = Q == INFERNO_Q2_K   ? 84
                     : Q == INFERNO_Q3_K ? 110
                     : Q == INFERNO_Q4_K ? 144
                     : Q == INFERNO_Q6_K ? 210
                                         : 34;
  size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= n_values) return;
  const uint8_t* b = blocks + (idx / BV) * BB;
  int v = int(idx % BV);
  float r;
  if constexpr (Q == INFERNO_Q2_K) r = dq_q2_k(b, v);
  else if constexpr (Q == INFERNO_Q3_K) r = dq_q3_k(b, v);
  else if constexpr (Q == INFERNO_Q4_K) r = dq_q4_k(b, v);
  else if constexpr (Q == INFERNO_Q6_K) r = dq_q6_k(b, v);
  else r = dq_q8_0(b, v);
  out[idx] = r;
}

#pragma clang fp contract(on)

__global__ void __launch_bounds__(256)
    synth_normal_kernel(uint64_t seed, float stddev, size_t n, int dtype, void* out) {
  size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v = stddev * synth_normal(seed, i);
  if (dtype == INFERNO_BF16)
    static_cast<uint16_t*>(out)[i] = f32_to_bf16_bits(v);
  else
    static_cast<float*>(out)[i] = v;
}

// One thread per block: generate its values, quantise, write the bytes.
__global__ void __launch_bounds__(128)
    synth_quant_kernel(int quant, uint64_t seed, float stddev, size_t rows, size_t cols,
                       uint8_t* __restrict__ out) {
  const int bv = block_values(quant), bb = block_bytes(quant);
  const size_t bpr = cols / size_t(bv);
  size_t blk = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (blk >= rows * bpr) return;
  size_t row = blk / bpr, col0 = (blk % bpr) * size_t(bv);
  float x[256];
  for (int v = 0; v < bv; ++v) x[v] = stddev * synth_normal(seed, row * cols + col0 + size_t(v));
  uint8_t tmp[210];
  quantize_block(quant, x, tmp);
  uint8_t* dst = out + blk * size_t(bb);
  for (int i = 0; i < bb; ++i) dst[i] = tmp[i];
}

}  // namespace

int launch_dequant(hipStream_t s, int quant, const void* blocks, size_t n_blocks, float* out) {
  size_t n = n_blocks * size_t(block_values(quant));
  if (n == 0) return INFERNO_OK;
  dim3 grid(unsigned((n + 255) / 256));
  auto b = static_cast<const uint8_t*>(blocks);
  switch (quant) {
    case INFERNO_Q2_K: dequant_kernel<INFERNO_Q2_K><<<grid, 256, 0, s>>>(b, n, out); break;
    case INFERNO_Q3_K: dequant_kernel<INFERNO_Q3_K><<<grid, 256, 0, s>>>(b, n, out); break;
    case INFERNO_Q4_K: dequant_kernel<INFERNO_Q4_K><<<grid, 256, 0, s>>>(b, n, out); break;
    case INFERNO_Q6_K: dequant_kernel<INFERNO_Q6_K><<<grid, 256, 0, s>>>(b, n, out); break;
    case INFERNO_Q8_0: dequant_kernel<INFERNO_Q8_0><<<grid, 256, 0, s>>>(b, n, out); break;
    default: set_error("unknown quant kind"); return INFERNO_ERR_INVALID;
  }
  INF_LAUNCHED();
  return INFERNO_OK;
}

int launch_synth_normal(hipStream_t s, uint64_t seed, float stddev, size_t n, int dtype,
                        void* out) {
  if (n == 0) return INFERNO_OK;
  synth_normal_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(seed, stddev, n, dtype, out);
  INF_LAUNCHED();
  return INFERNO_OK;
}

int launch_synth_quantized(hipStream_t s, int quant, uint64_t seed, float stddev, size_t rows,
                           size_t cols, void* out) {
  size_t nblk = rows * (cols / size_t(block_values(quant)));
  if (nblk == 0) return INFERNO_OK;
  synth_quant_kernel<<<unsigned((nblk + 127) / 128), 128, 0, s>>>(
      quant, seed, stddev, rows, cols, static_cast<uint8_t*>(out));
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace inferno
