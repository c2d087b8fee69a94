// The Q8_0 shared expert of a large prefill batch, and the router logits of
// a large bf16 batch, as library GEMMs (hipBLASLt).
//
// Reference: the shared expert of the prefill layer (crates/model/src/
// laguna/gguf_model.rs:802-823; q8_0 gate/up SwiGLU and matvec-add kernels,
// q2_kernels.metal:2066-2133): shared = W_d (silu(W_g x) * (W_u x)).
//
// Over many tokens it is a plain dense GEMM, so it runs as one: the Q8_0
// blocks are expanded to f16 (round(d * q), the value the MFMA kernels'
// in-register dequantisation forms), hipBLASLt multiplies with fp32
// accumulation and fp32 output, a small kernel forms h = silu(g) * u in f16
// (one rounding, as the grouped kernels' epilogue), and a second GEMM gives
// the shared rows ys in fp32. The gate/up weights are expanded in the k
// order of the f16 token copy (0 2 1 3 4 6 5 7 inside every eight, the
// grouped kernels' operand order), the down weights and h in plain order.
//
// Work per call: the expansion reads the 34-byte blocks once and writes
// 2 bytes per weight; the GEMMs are the library's (its algorithm picked by
// its heuristic once per shape and kept). The router logits (reference:
// the router linear, gguf_model.rs:742-748) take the fp32 router split
// exactly into three bf16 terms, one bf16 GEMM over the three terms' rows
// (fp32 accumulation) and an ordered sum of the three per expert.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "gemv_common.hpp"
#include "prefill.hpp"

namespace inferno {
namespace {

// Tokens from which the shared expert takes the library GEMMs (below it the
// grouped kernels' dense path): every prefill batch. Measured against the
// dense path: c2 T = 12 0.462 -> 0.401 ms, c2 T = 16 0.511 -> 0.445, c4
// T = 12 1.389 -> 1.236, T = 32 1.830 -> 1.650, T = 64 1.888 -> 1.733 (the
// dense path's 32-row tiles gave a 1536-row shared expert 48 workgroups).
constexpr size_t kBlasMinTokens = 1;
constexpr size_t kBlasWsBytes = size_t(32) << 20;  // the library's own workspace
// Tokens from which bf16 router logits take the library GEMM (c3's 512:
// 1.777-1.779 against 1.785-1.795 ms on the K-chunk kernel).
constexpr size_t kRouterBlasMinTokens = 512;

// Q8_0 [d f16 | 32 int8] blocks -> f16 rows. A 256-thread workgroup takes
// 64 consecutive 272-byte units (eight blocks, 256 values; 16-byte aligned)
// of one matrix: the units are read into LDS with contiguous 16-byte loads,
// all issued before the first LDS store (a load-store loop waited for each
// load in turn: c4 T = 32 29 us per layer), then every output chunk of eight
// values (one uint4) is formed from LDS by one thread, so that the stores are
// contiguous too. permute: k order 0 2 1 3 4 6 5 7 inside every eight. The
// three matrices (gate, up: permuted; down: plain) in one launch.
struct ExpandArgs {
  const uint8_t* src[3];
  uint16_t* dst[3];
  size_t groups[3];  // kExpandUnits-unit groups of each matrix (the last may be partial)
  size_t units[3];   // 256-value units of each matrix
  int permute[3];
};
constexpr int kExpandThreads = 256;
constexpr int kExpandUnits = 64;
constexpr int kUnitBytes = 272;
constexpr int kExpandLoads = (kExpandUnits * kUnitBytes / 16 + kExpandThreads - 1) / kExpandThreads;
__global__ void __launch_bounds__(kExpandThreads) q8_0_to_f16_kernel(ExpandArgs a) {
  __shared__ uint4 lds[kExpandUnits * kUnitBytes / 16];
  size_t g = blockIdx.x;
  int m = 0;
  while (m < 3 && g >= a.groups[m]) g -= a.groups[m++];
  if (m == 3) return;  // uniform
  const int tid = threadIdx.x;
  const size_t u0 = g * kExpandUnits;
  const int nu = int(min(size_t(kExpandUnits), a.units[m] - u0));
  const uint4* s4 = reinterpret_cast<const uint4*>(a.src[m] + u0 * kUnitBytes);
  const int n16 = nu * kUnitBytes / 16;
  uint4 v[kExpandLoads];
#pragma unroll
  for (int i = 0; i < kExpandLoads; ++i) v[i] = s4[min(i * kExpandThreads + tid, n16 - 1)];
#pragma unroll
  for (int i = 0; i < kExpandLoads; ++i)
    if (i * kExpandThreads + tid < n16) lds[i * kExpandThreads + tid] = v[i];
  __syncthreads();
  const uint8_t* lb = reinterpret_cast<const uint8_t*>(lds);
  const bool perm = a.permute[m] != 0;
  uint4* o4 = reinterpret_cast<uint4*>(a.dst[m] + u0 * 256);
  const int nchunks = nu * 32;  // uint4 chunks of eight values
  for (int c = tid; c < nchunks; c += kExpandThreads) {
    const int u = c >> 5, w = c & 31, blk = w >> 2, q8 = w & 3;
    const uint8_t* bp = lb + u * kUnitBytes + 34 * blk;
    const float d = f16_bits_to_f32(uint16_t(bp[0] | (bp[1] << 8)));
    uint32_t hv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q)
      hv[q] = __builtin_bit_cast(uint16_t, (_Float16)(d * float(int8_t(bp[2 + 8 * q8 + q]))));
    const int p1 = perm ? 2 : 1, p2 = perm ? 1 : 2, p5 = perm ? 6 : 5, p6 = perm ? 5 : 6;
    o4[c] = make_uint4(hv[0] | (hv[p1] << 16), hv[p2] | (hv[3] << 16), hv[4] | (hv[p5] << 16),
                       hv[p6] | (hv[7] << 16));
  }
}

// The router's fp32 weights as three bf16 terms (terms + m E H, m = 0, 1,
// 2): truncate, subtract, truncate, subtract, truncate; the last remainder
// has at most eight significant bits, so w = t0 + t1 + t2 exactly, and a
// bf16 x bf16 product is exact in fp32: the three terms' bf16 products
// accumulated in fp32 give fp32-accurate logits (the split of the router logits kernel's
// bf16x3 path, done once per call here).
__global__ void __launch_bounds__(256)
    split3_kernel(const float* __restrict__ w, size_t n8, size_t n, uint16_t* __restrict__ terms) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n8) return;
  const float4 a = reinterpret_cast<const float4*>(w)[2 * i];
  const float4 b = reinterpret_cast<const float4*>(w)[2 * i + 1];
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t h[3][4];
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    uint32_t t[3][2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t u = __builtin_bit_cast(uint32_t, v[j + q]);
      const uint32_t u1 = u & 0xffff0000u;
      const float r1 = v[j + q] - __builtin_bit_cast(float, u1);
      const uint32_t u2 = __builtin_bit_cast(uint32_t, r1) & 0xffff0000u;
      const float r2 = r1 - __builtin_bit_cast(float, u2);
      t[0][q] = u1 >> 16;
      t[1][q] = u2 >> 16;
      t[2][q] = __builtin_bit_cast(uint32_t, r2) >> 16;
    }
#pragma unroll
    for (int m = 0; m < 3; ++m) h[m][j / 2] = t[m][0] | (t[m][1] << 16);
  }
#pragma unroll
  for (int m = 0; m < 3; ++m)
    reinterpret_cast<uint4*>(terms + size_t(m) * n)[i] = make_uint4(h[m][0], h[m][1], h[m][2], h[m][3]);
}

// h[t][i] = silu(gu[t][i]) * gu[t][Is + i] in f16 (plain order), from the
// gate/up GEMM's fp32 rows [T][2 Is].
__global__ void __launch_bounds__(256)
    swiglu_f16_kernel(const float* __restrict__ gu, size_t T, size_t Is,
                      uint16_t* __restrict__ h) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= T * Is) return;
  const size_t t = i / Is, c = i - t * Is;
  const float g = gu[t * 2 * Is + c], u = gu[t * 2 * Is + Is + c];
  h[i] = __builtin_bit_cast(uint16_t, (_Float16)(silu(g) * u));
}

constexpr int kMaxBlasDevices = 64;
std::mutex g_blas_mu;
hipblasLtHandle_t g_blas[kMaxBlasDevices] = {};
std::map<std::tuple<int, int, int, int, int, int>, hipblasLtMatmulHeuristicResult_t> g_algo;

int blas_error(const char* what, int status) {
  set_error(std::string("hipBLASLt ") + what + " failed (status " + std::to_string(status) + ")");
  return INFERNO_ERR_DEVICE;
}

// D[n][m] (row-major, fp32) = X[n][k] (row-major f16) . W[m][k]^T (row-major
// f16): column-major D^T = op(W)^T-view x X-view with op(A) = T.
int blas_gemm(hipStream_t s, const uint16_t* W, const uint16_t* X, float* D, int m, int n, int k,
              void* ws, hipDataType in_type = HIP_R_16F, float beta = 0.0f) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxBlasDevices) {
    set_error("hipBLASLt: cannot query the current device");
    return INFERNO_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lock(g_blas_mu);
  if (!g_blas[dev]) {
    const hipblasStatus_t st = hipblasLtCreate(&g_blas[dev]);
    if (st != HIPBLAS_STATUS_SUCCESS) return blas_error("create", int(st));
  }
  hipblasLtHandle_t h = g_blas[dev];
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  int rc = INFERNO_OK;
  hipblasStatus_t st;
  const hipblasOperation_t tA = HIPBLAS_OP_T, tB = HIPBLAS_OP_N;
  const float alpha = 1.0f;
  auto fail = [&](const char* what) {
    rc = blas_error(what, int(st));
    return rc;
  };
  do {
    if ((st = hipblasLtMatmulDescCreate(&op, HIPBLAS_COMPUTE_32F, HIP_R_32F)) != HIPBLAS_STATUS_SUCCESS) {
      fail("matmul descriptor");
      break;
    }
    hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSA, &tA, sizeof(tA));
    hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSB, &tB, sizeof(tB));
    if ((st = hipblasLtMatrixLayoutCreate(&la, in_type, k, m, k)) != HIPBLAS_STATUS_SUCCESS ||
        (st = hipblasLtMatrixLayoutCreate(&lb, in_type, k, n, k)) != HIPBLAS_STATUS_SUCCESS ||
        (st = hipblasLtMatrixLayoutCreate(&lc, HIP_R_32F, m, n, m)) != HIPBLAS_STATUS_SUCCESS) {
      fail("matrix layout");
      break;
    }
    const auto key = std::make_tuple(dev, m, n, k, int(in_type), beta != 0.0f ? 1 : 0);
    auto it = g_algo.find(key);
    if (it == g_algo.end()) {
      hipblasLtMatmulPreference_t pref = nullptr;
      if ((st = hipblasLtMatmulPreferenceCreate(&pref)) != HIPBLAS_STATUS_SUCCESS) {
        fail("preference");
        break;
      }
      const uint64_t wsb = kBlasWsBytes;
      hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                            sizeof(wsb));
      hipblasLtMatmulHeuristicResult_t res{};
      int found = 0;
      st = hipblasLtMatmulAlgoGetHeuristic(h, op, la, lb, lc, lc, pref, 1, &res, &found);
      hipblasLtMatmulPreferenceDestroy(pref);
      if (st != HIPBLAS_STATUS_SUCCESS || found < 1) {
        if (st == HIPBLAS_STATUS_SUCCESS) st = HIPBLAS_STATUS_NOT_SUPPORTED;
        fail("heuristic");
        break;
      }
      it = g_algo.emplace(key, res).first;
    }
    if ((st = hipblasLtMatmul(h, op, &alpha, W, la, X, lb, &beta, D, lc, D, lc, &it->second.algo,
                              ws, kBlasWsBytes, s)) != HIPBLAS_STATUS_SUCCESS) {
      fail("matmul");
      break;
    }
  } while (false);
  if (lc) hipblasLtMatrixLayoutDestroy(lc);
  if (lb) hipblasLtMatrixLayoutDestroy(lb);
  if (la) hipblasLtMatrixLayoutDestroy(la);
  if (op) hipblasLtMatmulDescDestroy(op);
  return rc;
}

// Carved regions of the workspace, 256-byte aligned.
struct BlasWs {
  uint16_t* wgu;  // [2 Is][H] f16 (gate rows, then up rows), k order permuted
  uint16_t* wd;   // [H][Is] f16
  float* gu;      // [T][2 Is] fp32
  uint16_t* h;    // [T][Is] f16
  size_t end;
};
BlasWs carve(void* base, size_t T, size_t H, size_t Is) {
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  BlasWs w{};
  char* p = static_cast<char*>(base);
  size_t o = 0;
  w.wgu = reinterpret_cast<uint16_t*>(p + o); o += al(2 * Is * H * 2);
  w.wd = reinterpret_cast<uint16_t*>(p + o);  o += al(H * Is * 2);
  w.gu = reinterpret_cast<float*>(p + o);     o += al(T * 2 * Is * 4);
  w.h = reinterpret_cast<uint16_t*>(p + o);   o += al(T * Is * 2);
  w.end = o;
  return w;
}

int launch_expand(hipStream_t s, const void* gate, const void* up, const void* down, size_t H,
                  size_t Is, uint16_t* wgu, uint16_t* wd) {
  ExpandArgs a{};
  a.src[0] = static_cast<const uint8_t*>(gate);
  a.src[1] = static_cast<const uint8_t*>(up);
  a.src[2] = static_cast<const uint8_t*>(down);
  a.dst[0] = wgu;
  a.dst[1] = wgu + Is * H;
  a.dst[2] = wd;
  const size_t units = Is * H / 256;  // H, Is multiples of 256
  for (int m = 0; m < 3; ++m) {
    a.units[m] = units;
    a.groups[m] = (units + kExpandUnits - 1) / kExpandUnits;
    a.permute[m] = m < 2 ? 1 : 0;
  }
  q8_0_to_f16_kernel<<<unsigned(3 * a.groups[0]), kExpandThreads, 0, s>>>(a);
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace

bool dense_blas_fits(int quant, int down_quant, size_t T, size_t H, size_t Is) {
  return quant == INFERNO_Q8_0 && down_quant == INFERNO_Q8_0 && Is > 0 && T >= kBlasMinTokens &&
         H % 256 == 0 && Is % 256 == 0 && T < (size_t(1) << 30) && 2 * Is < (size_t(1) << 30) &&
         H < (size_t(1) << 30);
}

// INFERNO_SHARED_BLAS=0: the grouped kernels' dense path at every T.
bool dense_blas_takes(int quant, int down_quant, size_t T, size_t H, size_t Is) {
  return dense_blas_fits(quant, down_quant, T, H, Is) && !switch_off("INFERNO_SHARED_BLAS");
}

size_t dense_blas_workspace_bytes(size_t T, size_t H, size_t Is) {
  return carve(nullptr, T, H, Is).end + 256;
}

int launch_dense_blas(hipStream_t s, const void* gate, const void* up, const void* down,
                      const uint16_t* x16, size_t T, size_t H, size_t Is, float* ys, void* ws,
                      void* lib_ws) {
  const BlasWs w = carve(reinterpret_cast<void*>((reinterpret_cast<uintptr_t>(ws) + 255) /
                                                 256 * 256), T, H, Is);
  int st;
  if ((st = launch_expand(s, gate, up, down, H, Is, w.wgu, w.wd))) return st;
  if ((st = blas_gemm(s, w.wgu, x16, w.gu, int(2 * Is), int(T), int(H), lib_ws))) return st;
  const size_t n = T * Is;
  swiglu_f16_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(w.gu, T, Is, w.h);
  INF_LAUNCHED();
  return blas_gemm(s, w.wd, w.h, ys, int(H), int(T), int(Is), lib_ws);
}

size_t blas_lib_workspace_bytes() { return kBlasWsBytes; }

// ------------------------------------------------------------ router

bool router_blas_fits(size_t T, size_t H, size_t E) {
  return T >= kRouterBlasMinTokens && H % 8 == 0 && H < (size_t(1) << 30) && E >= 1 &&
         E <= 256 && T < (size_t(1) << 30);
}

bool router_blas_takes(size_t T, size_t H, size_t E, int x_dtype) {
  return x_dtype == INFERNO_BF16 && router_blas_fits(T, H, E) &&
         !switch_off("INFERNO_ROUTER_BLAS") && !switch_off("INFERNO_ROUTER_BF16X3");
}

namespace {
// The three terms' logits of T tokens [T][3E] (term-major within a token)
// are added as (t0 + t1) + t2 per expert: the order of the three
// accumulating GEMMs (beta 1) this single GEMM replaces.
__global__ void __launch_bounds__(256)
    sum3_kernel(const float* __restrict__ d3, size_t T, uint32_t E, float* __restrict__ logits) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= T * E) return;
  const size_t t = i / E, e = i - t * E;
  const float* r = d3 + t * 3 * E + e;
  logits[i] = (r[0] + r[E]) + r[2 * E];
}
}  // namespace

size_t router_blas_workspace_bytes(size_t T, size_t H, size_t E) {
  return (3 * E * H * 2 + 255) / 256 * 256 + (T * 3 * E * 4 + 255) / 256 * 256 + 256;
}

int launch_router_blas(hipStream_t s, const uint16_t* x, const float* w, size_t T, size_t H,
                       size_t E, float* logits, void* terms_ws, void* lib_ws) {
  uint16_t* terms = reinterpret_cast<uint16_t*>((reinterpret_cast<uintptr_t>(terms_ws) + 255) /
                                                256 * 256);
  float* d3 = reinterpret_cast<float*>(terms + (3 * E * H + 127) / 128 * 128);
  const size_t n8 = E * H / 8;
  split3_kernel<<<unsigned((n8 + 255) / 256), 256, 0, s>>>(w, n8, E * H, terms);
  INF_LAUNCHED();
  // the three terms [3][E][H] are one [3E][H] operand: one GEMM of 3E
  // columns fills the chip better than three of E (c5: 256 columns made
  // 256 tiles of 64 x 64, one workgroup per CU)
  if (int st = blas_gemm(s, terms, x, d3, int(3 * E), int(T), int(H), lib_ws, HIP_R_16BF, 0.0f))
    return st;
  sum3_kernel<<<unsigned((T * E + 255) / 256), 256, 0, s>>>(d3, T, uint32_t(E), logits);
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace inferno
