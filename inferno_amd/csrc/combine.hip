// Data movement and combine kernels. Every output element is written by one
// thread that sums its contributions in a fixed order — no float atomics, so
// results are bitwise reproducible run to run.
#include <type_traits>

#include "kernels.hpp"
#include "norm_dev.hpp"

namespace inferno {
namespace {

// shared + residual + sum_r y[t*k+r] * w[t*k+r] in rank order
// (crates/backend/src/metal/kernels/moe_kernels.metal:210-238).
__global__ void __launch_bounds__(256)
    topk_combine_kernel(const float* __restrict__ shared, const float* __restrict__ residual,
                        const float* __restrict__ y, const float* __restrict__ w, size_t T,
                        size_t H, int k, float* __restrict__ out) {
  size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= T * H) return;
  size_t t = i / H, h = i % H;
  float v = (shared ? shared[i] : 0.f) + (residual ? residual[i] : 0.f);
  for (int r = 0; r < k; ++r) {
    size_t a = t * size_t(k) + size_t(r);
    v += y[a * H + h] * (w ? w[a] : 1.0f);
  }
  out[i] = v;
}

// The same sum, four columns per thread (H a multiple of 4, 16-byte aligned
// rows), the k rank rows (and weights) loaded at once: KMAX slots, indices
// clamped to k - 1, the extra slots not added.
__device__ __forceinline__ void add_scaled(float4& v, const float4& u, float s) {
  v.x += u.x * s; v.y += u.y * s; v.z += u.z * s; v.w += u.w * s;
}

typedef float fx4 __attribute__((ext_vector_type(4)));

template <int KMAX>
__global__ void __launch_bounds__(256)
    topk_combine4_kernel(const float* __restrict__ shared, const float* __restrict__ residual,
                         const float* __restrict__ y, const float* __restrict__ w, uint32_t H4,
                         uint32_t n4, int k, float* __restrict__ out) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= n4) return;
  const uint32_t t = i / H4, c4 = i - t * H4;
  const float4* y4 = reinterpret_cast<const float4*>(y);
  float4 u[KMAX];
  float ws[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    const size_t a = size_t(t) * k + min(r, k - 1);
    const fx4 q = __builtin_nontemporal_load(reinterpret_cast<const fx4*>(y4 + a * H4 + c4));
    u[r] = make_float4(q[0], q[1], q[2], q[3]);  // read once: nontemporal
    ws[r] = w ? w[a] : 1.0f;
  }
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  const float4 sh = shared ? reinterpret_cast<const float4*>(shared)[i] : z;
  const float4 rs = residual ? reinterpret_cast<const float4*>(residual)[i] : z;
  float4 v = make_float4(sh.x + rs.x, sh.y + rs.y, sh.z + rs.z, sh.w + rs.w);
#pragma unroll
  for (int r = 0; r < KMAX; ++r)
    if (r < k) add_scaled(v, u[r], ws[r]);
  reinterpret_cast<float4*>(out)[i] = v;
}

// acc + contributions of every assignment of token t, in assignment order
// (crates/backend/src/backend.rs:10298-10352; moe_kernels.metal:53-81).
__global__ void __launch_bounds__(256)
    index_add_combine_kernel(const float* __restrict__ acc, const uint32_t* __restrict__ tok,
                             const float* __restrict__ y, const float* __restrict__ w, size_t T,
                             size_t H, size_t A, float* __restrict__ out) {
  size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= T * H) return;
  size_t t = i / H, h = i % H;
  float v = acc[i];
  for (size_t a = 0; a < A; ++a)
    if (tok[a] == t) v += y[a * H + h] * w[a];
  out[i] = v;
}

// moe_kernels.metal:5-28
__global__ void __launch_bounds__(256)
    gather_kernel(const float* __restrict__ x, const uint32_t* __restrict__ tok, size_t T,
                  size_t H, size_t A, float* __restrict__ out) {
  size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= A * H) return;
  size_t a = i / H, h = i % H;
  uint32_t t = tok[a];
  out[i] = t < T ? x[size_t(t) * H + h] : 0.f;
}

// One 1024-thread workgroup per row (rms_norm_row, norm_dev.hpp). The
// output is fp32 or bf16 (round to nearest even), the activation type a
// following layer consumes.
template <typename OutT>
__device__ __forceinline__ void store_norm(OutT* out, size_t i, float v) {
  if constexpr (std::is_same<OutT, float>::value)
    out[i] = v;
  else
    out[i] = f32_to_bf16_bits(v);
}

template <typename OutT>
__global__ void __launch_bounds__(kNormThreads)
    rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ w, size_t H, float eps,
                    OutT* __restrict__ out) {
  __shared__ float part[kNormThreads / 64 + 1];
  OutT* orow = out + size_t(blockIdx.x) * H;
  rms_norm_row(x + size_t(blockIdx.x) * H, w, H, eps, part,
               [&](size_t i, float v) { store_norm(orow, i, v); });
}

unsigned blocks_for(size_t n) { return unsigned((n + 255) / 256); }

}  // namespace

int launch_topk_combine(hipStream_t s, const float* shared, const float* residual,
                        const float* y, const float* w, size_t T, size_t H, size_t k,
                        float* out) {
  if (T * H == 0) return INFERNO_OK;
  auto a16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  const size_t n4 = T * H / 4;
  if (H % 4 == 0 && n4 <= 0xffffffffu && k >= 1 && k <= size_t(kMaxTopK) && a16(y) && a16(out) &&
      a16(shared) && a16(residual)) {
    const unsigned grid = unsigned((n4 + 255) / 256);
    if (k <= 8)
      topk_combine4_kernel<8><<<grid, 256, 0, s>>>(shared, residual, y, w, uint32_t(H / 4),
                                                   uint32_t(n4), int(k), out);
    else
      topk_combine4_kernel<16><<<grid, 256, 0, s>>>(shared, residual, y, w, uint32_t(H / 4),
                                                    uint32_t(n4), int(k), out);
    INF_LAUNCHED();
    return INFERNO_OK;
  }
  topk_combine_kernel<<<blocks_for(T * H), 256, 0, s>>>(shared, residual, y, w, T, H, int(k),
                                                        out);
  INF_LAUNCHED();
  return INFERNO_OK;
}

int launch_index_add_combine(hipStream_t s, const float* acc, const uint32_t* tok,
                             const float* y, const float* w, size_t T, size_t H, size_t A,
                             float* out) {
  if (T * H == 0) return INFERNO_OK;
  index_add_combine_kernel<<<blocks_for(T * H), 256, 0, s>>>(acc, tok, y, w, T, H, A, out);
  INF_LAUNCHED();
  return INFERNO_OK;
}

int launch_gather(hipStream_t s, const float* x, const uint32_t* tok, size_t T, size_t H,
                  size_t A, float* out) {
  if (A * H == 0) return INFERNO_OK;
  gather_kernel<<<blocks_for(A * H), 256, 0, s>>>(x, tok, T, H, A, out);
  INF_LAUNCHED();
  return INFERNO_OK;
}

int launch_rms_norm(hipStream_t s, const float* x, const float* w, size_t rows, size_t H,
                    float eps, void* out, int out_dtype) {
  if (rows == 0) return INFERNO_OK;
  if (out_dtype == INFERNO_BF16)
    rms_norm_kernel<uint16_t><<<unsigned(rows), kNormThreads, 0, s>>>(x, w, H, eps,
                                                                      static_cast<uint16_t*>(out));
  else
    rms_norm_kernel<float><<<unsigned(rows), kNormThreads, 0, s>>>(x, w, H, eps,
                                                                   static_cast<float*>(out));
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace inferno
