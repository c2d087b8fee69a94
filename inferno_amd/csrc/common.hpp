// Shared host/device definitions: GGUF block geometry, f16/bf16 bit helpers,
// wavefront reductions, error plumbing for the C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <string>

#include "inferno_moe.h"

#define HD __host__ __device__ __forceinline__

namespace inferno {

// True when the environment variable `name` starts with '0' (a kernel-variant
// switch turned off). Read on every call, so a process can change it between
// calls; it costs one environment scan per launch decision.
inline bool switch_off(const char* name) {
  const char* v = std::getenv(name);
  return v && v[0] == '0';
}

// True when the environment variable `name` starts with '1' (an off-by-
// default variant switched on).
inline bool switch_on(const char* name) {
  const char* v = std::getenv(name);
  return v && v[0] == '1';
}

// The environment variable `name` as a non-negative integer, or `dflt` when
// it is unset or not a number (a tuning threshold; read on every call).
inline size_t env_size(const char* name, size_t dflt) {
  const char* v = std::getenv(name);
  if (!v || *v < '0' || *v > '9') return dflt;
  return size_t(std::strtoull(v, nullptr, 10));
}

// The grouped GEMM's tile lists, written by the dispatch launch when `l128`
// is set (the prefill path): per-expert tiles {expert, first row, end row,
// 0} in expert order, split by row count, and the three list lengths.
struct PlanOut {
  uint4* l128;
  uint4* l64;
  uint4* l32;
  uint32_t* counts;  // [3]: lengths of l128, l64, l32
};

constexpr int kWave = 64;        // CDNA wavefront width
constexpr int kKBlock = 256;     // K-quant super-block values
constexpr int kQ8Block = 32;     // Q8_0 block values
constexpr int kMaxExperts = 256; // router wave holds 4 candidates per lane
constexpr int kMaxTopK = 16;     // crates/backend/src/metal/kernels/moe_kernels.metal:131

// GGUF block sizes: crates/gguf/src/lib.rs:21-27.
HD int block_bytes(int quant) {
  switch (quant) {
    case INFERNO_Q2_K: return 84;
    case INFERNO_Q3_K: return 110;
    case INFERNO_Q4_K: return 144;
    case INFERNO_Q6_K: return 210;
    case INFERNO_Q8_0: return 34;
  }
  return -1;
}
HD int block_values(int quant) {
  if (quant == INFERNO_Q8_0) return kQ8Block;
  return block_bytes(quant) < 0 ? -1 : kKBlock;
}
// Bytes of one 256-value "super-block" (Q8_0: eight 34-byte blocks).
HD int super_bytes(int quant) { return quant == INFERNO_Q8_0 ? 8 * 34 : block_bytes(quant); }

HD float bits_to_f32(uint32_t b) { return __builtin_bit_cast(float, b); }
HD uint32_t f32_to_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

// IEEE half -> float by bit manipulation (subnormals, inf, NaN payloads kept),
// the arithmetic of crates/gguf/src/lib.rs:1501-1528 written independently.
HD float f16_bits_to_f32(uint16_t h) {
  uint32_t sign = uint32_t(h & 0x8000u) << 16;
  uint32_t ex = (h >> 10) & 0x1fu;
  uint32_t fr = h & 0x3ffu;
  if (ex == 0x1fu) return bits_to_f32(sign | 0x7f800000u | (fr << 13));
  if (ex != 0) return bits_to_f32(sign | ((ex + 112u) << 23) | (fr << 13));
  if (fr == 0) return bits_to_f32(sign);
  // subnormal: value = fr * 2^-24, exact in f32
  int msb = 31 - __builtin_clz(fr);  // value = 1.m * 2^(msb - 24)
  uint32_t e = uint32_t(msb - 24 + 127);
  uint32_t mant = (fr << (23 - msb)) & 0x7fffffu;
  return bits_to_f32(sign | (e << 23) | mant);
}

// float -> f16 bits, round to nearest even (compiler conversion).
HD uint16_t f32_to_f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

HD float bf16_bits_to_f32(uint16_t b) { return bits_to_f32(uint32_t(b) << 16); }
HD uint16_t f32_to_bf16_bits(float f) {  // round to nearest even; NaN kept quiet
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

HD uint16_t load_le16(const uint8_t* p) { return uint16_t(p[0] | (uint16_t(p[1]) << 8)); }

// --------------------------------------------------------------- errors
void set_error(const std::string& msg);
void clear_error();

}  // namespace inferno

#define INF_CHECK_ARG(cond, msg)                 \
  do {                                           \
    if (!(cond)) {                               \
      ::inferno::set_error(std::string(msg));    \
      return INFERNO_ERR_INVALID;                \
    }                                            \
  } while (0)

#define INF_HIP(call)                                                                 \
  do {                                                                                \
    hipError_t e_ = (call);                                                           \
    if (e_ != hipSuccess) {                                                           \
      ::inferno::set_error(std::string(#call) + ": " + hipGetErrorString(e_));        \
      return INFERNO_ERR_DEVICE;                                                      \
    }                                                                                 \
  } while (0)

// After a kernel launch: report launch errors without synchronising.
#define INF_LAUNCHED()                                                               \
  do {                                                                               \
    hipError_t e_ = hipGetLastError();                                               \
    if (e_ != hipSuccess) {                                                          \
      ::inferno::set_error(std::string("kernel launch: ") + hipGetErrorString(e_));  \
      return INFERNO_ERR_DEVICE;                                                     \
    }                                                                                \
  } while (0)
