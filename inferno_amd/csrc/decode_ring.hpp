// Decode gate/up for one token with the selected experts' quant bytes
// streamed HBM -> LDS by direct-to-LDS copies (global_load_lds_dwordx4).
//
// A workgroup is persistent and runs a list of jobs; a job is one 16-row
// gate/up tile, either of a routed slot (the slot's Q2_K expert) or of the
// Q8_0 shared expert. A job is a sequence of items: one matrix's 16 rows
// over a range of super-block columns, at most 16 KB (Q2_K: 8 columns, each
// lane two rows of one column; Q8_0: 3 columns, each lane one row). Items
// land in a ring of kDepth LDS slots: wavefronts 0..2 copy item n + kDepth - 1
// (every lane one 16-byte chunk, gathered over the 16 rows) while all four
// wavefronts compute item n. The quant bytes never pass through VGPRs, so the
// bytes in flight per CU are bounded by LDS instead of registers, and the
// copies of the next items overlap the dot products of this one.
//
// Every LDS read of the compute phase is an inline ds_read: the compiler
// treats a direct-to-LDS copy as a pending write of unknown LDS addresses
// and would otherwise wait for all outstanding copies (vmcnt(0)) before each
// LDS read, which serialises copy and compute. Completion of an item's copies
// is tracked explicitly instead: each copying wavefront issues exactly PW
// copy instructions per item, waits with s_waitcnt vmcnt(PW * newer items),
// and a workgroup barrier publishes the item. Wavefront 3 issues no copies;
// it writes the job outputs (global stores count on vmcnt too, so keeping
// them out of the copying wavefronts keeps those counts exact).
//
// Per unit (row, super-block column, sub-lane) the dot products are those of
// Fmt<Q>::dot in dot2_formats.hpp: same fields, same scale and minimum
// algebra, same staged activation layout. (Values are taken out of the asm
// vector outputs with element accesses and __uint_as_float:
// __builtin_bit_cast of a vector element compiled to a read of element 0.)
#pragma once
#include "decode.hpp"
#include "dot2_formats.hpp"

namespace inferno {
namespace ring {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kSlotBytes = 16384;              // one item
constexpr int kDepth = 4;                      // ring slots
constexpr int kDmaWaves = 3;                   // wavefronts that copy
constexpr int kPartFloats = 2 * 4 * kRows;     // [matrix][wavefront][row]

// A batch of LDS reads is one asm statement ending in s_waitcnt lgkmcnt(0),
// with early-clobber outputs: the registers are written asynchronously, so
// no output may share a register with an address still to be read, and the
// compiler must not move or copy an output before the data has landed. The
// LDS/scalar-memory counter holds at most 15 outstanding operations: a batch
// first drains whatever the compiler left in flight (a scalar load, say), and
// a batch longer than 15 reads waits (lgkmcnt(N)) before its 16th.

// LDS byte offset of a shared-memory pointer (the low 32 bits of the
// generic address are the offset inside the LDS aperture).
__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>(p));
}

// An LDS write the compiler does not see, completed before returning (a
// barrier does not wait for outstanding LDS writes, and the compiler adds no
// wait for a write it does not know about).
__device__ __forceinline__ void wr1(uint32_t a, float v) {
  asm volatile("ds_write_b32 %0, %1\n s_waitcnt lgkmcnt(0)" : : "v"(a), "v"(v) : "memory");
}

// s_waitcnt immediate (gfx9): vmcnt bits [3:0] and [15:14], expcnt 7, lgkmcnt 15
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

__device__ __forceinline__ uint4 v4(u32x4 a) { return make_uint4(a.x, a.y, a.z, a.w); }

__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  return v;
}

// Staged activation row in LDS: [hi pairs K/2][run sums K/16][run inv scales K/16],
// the hi pairs with the four 16-word blocks of every 64-word half-column h of
// column c stored at block b ^ x_swizzle(c, h): lanes reading different
// columns / halves of one block index then hit different LDS banks.
__device__ __forceinline__ int x_swizzle(int col, int h) { return (2 * (col & 1) + h) & 3; }

struct XLds {
  uint32_t hi, sums, invs;  // byte offsets
};

// ------------------------------------------------------------- formats


// Q2_K [scales 16 | qs 64 | d | dmin]; sub = 2h + s; runs 8h + 2p + s.
// One (row, sub) unit of a super-block column from its quant words (qs
// words q, scale words sc0/sc1, d|dmin word dd) and the column's staged
// activations for the unit's four runs.
__device__ __forceinline__ float q2k_unit(const uint32_t (&r)[4], uint32_t sc0, uint32_t sc1,
                                          uint32_t dd, int s, const uint4 (&xs)[8],
                                          const float (&sums)[4], const float (&invs)[4]) {
  // scale bytes of p = 0..3 sit at bytes s, 2+s of the two scale words
  const uint32_t scb = __builtin_amdgcn_perm(sc1, sc0, s ? 0x07050301u : 0x06040200u);
  uint32_t odd[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) odd[j] = r[j] >> 8;
  float acc_s = 0.f, acc_m = 0.f;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t m = 0x00030003u << (2 * p);
    const uint32_t f[8] = {r[0] & m, odd[0] & m, r[1] & m, odd[1] & m,
                           r[2] & m, odd[2] & m, r[3] & m, odd[3] & m};
    const float t = dot8(f, xs[2 * p], xs[2 * p + 1]) * invs[p];
    const uint32_t byte = (scb >> (8 * p)) & 0xffu;
    acc_s = fmaf(float(byte & 15u) * (kTwo24 / float(1 << (2 * p))), t, acc_s);
    acc_m = fmaf(float(byte >> 4), sums[p], acc_m);
  }
  const float d = f16_bits_to_f32_fast(uint16_t(dd));
  const float dmin = f16_bits_to_f32_fast(uint16_t(dd >> 16));
  return d * acc_s - dmin * acc_m;
}

template <int Q>
struct RingFmt;

// Routed Q2_K items are 16 rows x 8 columns (672-byte row segments); a lane
// computes rows r and r + 8 of one (column, sub) against one read of the
// column's activations, halving the activation traffic per weight (rows
// r = 0..7 start on eight different LDS banks).
template <>
struct RingFmt<INFERNO_Q2_K> {
  static constexpr int kBytes = 84;
  static constexpr int kCols = 8;
  static constexpr uint32_t kSeg = kCols * kBytes;  // row segment bytes
  // blk: LDS byte address of row r's block in this column
  __device__ static void dot2(uint32_t blk, int sub, const XLds& x, int col, float& o0,
                              float& o1) {
    const int h = sub >> 1, s = sub & 1;
    const uint32_t qa = blk + 16 + 32 * h + 16 * s;
    const uint32_t qb = qa + 8 * kSeg;
    const uint32_t sa = blk + 8 * h, sb = sa + 8 * kSeg;
    const uint32_t da = blk + 80, db = da + 8 * kSeg;
    const int g = x_swizzle(col, h);
    const uint32_t xh = x.hi + 4 * (col * 128 + 64 * h + 8 * s);
    const uint32_t x0a = xh + 64 * (0 ^ g), x1a = xh + 64 * (1 ^ g);
    const uint32_t x2a = xh + 64 * (2 ^ g), x3a = xh + 64 * (3 ^ g);
    const uint32_t ra = 4 * (col * 16 + 8 * h + s);
    u32x2 qa01, qa23, qb01, qb23, sca, scb, s02, s46, i02, i46;
    uint32_t dda, ddb;
    u32x4 x0, x1, x2, x3, x4, x5, x6, x7;
    asm volatile(
        "s_waitcnt lgkmcnt(0)\n"
        "ds_read2_b32 %0, %20 offset0:0 offset1:1\n"
        "ds_read2_b32 %1, %20 offset0:2 offset1:3\n"
        "ds_read2_b32 %2, %21 offset0:0 offset1:1\n"
        "ds_read2_b32 %3, %21 offset0:2 offset1:3\n"
        "ds_read2_b32 %4, %22 offset0:0 offset1:1\n"
        "ds_read2_b32 %5, %23 offset0:0 offset1:1\n"
        "ds_read_b32 %6, %24\n"
        "ds_read_b32 %7, %25\n"
        "ds_read_b128 %8, %26 offset:0\n"
        "ds_read_b128 %9, %26 offset:16\n"
        "ds_read_b128 %10, %27 offset:0\n"
        "ds_read_b128 %11, %27 offset:16\n"
        "ds_read_b128 %12, %28 offset:0\n"
        "ds_read_b128 %13, %28 offset:16\n"
        "s_waitcnt lgkmcnt(8)\n"
        "ds_read_b128 %14, %29 offset:0\n"
        "ds_read_b128 %15, %29 offset:16\n"
        "ds_read2_b32 %16, %30 offset0:0 offset1:2\n"
        "ds_read2_b32 %17, %30 offset0:4 offset1:6\n"
        "ds_read2_b32 %18, %31 offset0:0 offset1:2\n"
        "ds_read2_b32 %19, %31 offset0:4 offset1:6\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(qa01), "=&v"(qa23), "=&v"(qb01), "=&v"(qb23), "=&v"(sca), "=&v"(scb),
          "=&v"(dda), "=&v"(ddb), "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3), "=&v"(x4),
          "=&v"(x5), "=&v"(x6), "=&v"(x7), "=&v"(s02), "=&v"(s46), "=&v"(i02), "=&v"(i46)
        : "v"(qa), "v"(qb), "v"(sa), "v"(sb), "v"(da), "v"(db), "v"(x0a), "v"(x1a), "v"(x2a),
          "v"(x3a), "v"(x.sums + ra), "v"(x.invs + ra));
    const uint4 xs[8] = {v4(x0), v4(x1), v4(x2), v4(x3), v4(x4), v4(x5), v4(x6), v4(x7)};
    const float sums[4] = {__uint_as_float(s02.x), __uint_as_float(s02.y),
                           __uint_as_float(s46.x), __uint_as_float(s46.y)};
    const float invs[4] = {__uint_as_float(i02.x), __uint_as_float(i02.y),
                           __uint_as_float(i46.x), __uint_as_float(i46.y)};
    const uint32_t ra4[4] = {qa01.x, qa01.y, qa23.x, qa23.y};
    const uint32_t rb4[4] = {qb01.x, qb01.y, qb23.x, qb23.y};
    o0 = q2k_unit(ra4, sca.x, sca.y, dda, s, xs, sums, invs);
    o1 = q2k_unit(rb4, scb.x, scb.y, ddb, s, xs, sums, invs);
  }
};

// Q8_0 super-block = eight 34-byte blocks [d | int8 x32]; sub owns blocks
// 2 sub and 2 sub + 1 (68 bytes at 68 sub, runs 4 sub .. 4 sub + 3).
template <>
struct RingFmt<INFERNO_Q8_0> {
  static constexpr int kBytes = 272;
  __device__ static float dot(uint32_t blk, int sub, const XLds& x, int col) {
    const uint32_t a = blk + 68 * sub;
    // runs 4 sub .. 4 sub + 3 = blocks b0 = 2 (sub & 1) and b0 + 1 of half h
    const int h = sub >> 1, g = x_swizzle(col, h), b0 = 2 * (sub & 1);
    const uint32_t xh = x.hi + 4 * (col * 128 + 64 * h);
    const uint32_t xa = xh + 64 * (b0 ^ g), xb = xh + 64 * ((b0 + 1) ^ g);
    const uint32_t ra = 4 * (col * 16 + 4 * sub);
    u32x2 w0, w1, w2, w3, w4, w5, w6, w7, s01, s23, i01, i23;
    uint32_t w8;
    u32x4 x0, x1, x2, x3, x4, x5, x6, x7;
    asm volatile(
        "s_waitcnt lgkmcnt(0)\n"
        "ds_read2_b32 %0, %21 offset0:0 offset1:1\n"
        "ds_read2_b32 %1, %21 offset0:2 offset1:3\n"
        "ds_read2_b32 %2, %21 offset0:4 offset1:5\n"
        "ds_read2_b32 %3, %21 offset0:6 offset1:7\n"
        "ds_read2_b32 %4, %21 offset0:8 offset1:9\n"
        "ds_read2_b32 %5, %21 offset0:10 offset1:11\n"
        "ds_read2_b32 %6, %21 offset0:12 offset1:13\n"
        "ds_read2_b32 %7, %21 offset0:14 offset1:15\n"
        "ds_read_b32 %8, %21 offset:64\n"
        "ds_read_b128 %9, %22 offset:0\n"
        "ds_read_b128 %10, %22 offset:16\n"
        "ds_read_b128 %11, %22 offset:32\n"
        "ds_read_b128 %12, %22 offset:48\n"
        "ds_read_b128 %13, %23 offset:0\n"
        "ds_read_b128 %14, %23 offset:16\n"
        "s_waitcnt lgkmcnt(9)\n"
        "ds_read_b128 %15, %23 offset:32\n"
        "ds_read_b128 %16, %23 offset:48\n"
        "ds_read2_b32 %17, %24 offset0:0 offset1:1\n"
        "ds_read2_b32 %18, %24 offset0:2 offset1:3\n"
        "ds_read2_b32 %19, %25 offset0:0 offset1:1\n"
        "ds_read2_b32 %20, %25 offset0:2 offset1:3\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(w0), "=&v"(w1), "=&v"(w2), "=&v"(w3), "=&v"(w4), "=&v"(w5), "=&v"(w6),
          "=&v"(w7), "=&v"(w8), "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3), "=&v"(x4),
          "=&v"(x5), "=&v"(x6), "=&v"(x7), "=&v"(s01), "=&v"(s23), "=&v"(i01), "=&v"(i23)
        : "v"(a), "v"(xa), "v"(xb), "v"(x.sums + ra), "v"(x.invs + ra));
    const uint32_t r[17] = {w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y, w4.x,
                            w4.y, w5.x, w5.y, w6.x, w6.y, w7.x, w7.y, w8};
    const uint4 xs[8] = {v4(x0), v4(x1), v4(x2), v4(x3), v4(x4), v4(x5), v4(x6), v4(x7)};
    const float sums[4] = {__uint_as_float(s01.x), __uint_as_float(s01.y),
                           __uint_as_float(s23.x), __uint_as_float(s23.y)};
    const float invs[4] = {__uint_as_float(i01.x), __uint_as_float(i01.y),
                           __uint_as_float(i23.x), __uint_as_float(i23.y)};
    // block 0: d = bytes 0-1, codes bytes 2..33; block 1: d = bytes 34-35, codes 36..67
    uint32_t q[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = __builtin_amdgcn_alignbyte(r[j + 1], r[j], 2) ^ 0x80808080u;
#pragma unroll
    for (int j = 0; j < 8; ++j) q[8 + j] = r[9 + j] ^ 0x80808080u;
    const uint32_t m = 0x00ff00ffu;
    float acc = 0.f;
#pragma unroll
    for (int blk2 = 0; blk2 < 2; ++blk2) {
      float t = 0.f;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const uint32_t* w = q + 8 * blk2 + 4 * half;
        const uint32_t f[8] = {w[0] & m, (w[0] >> 8) & m, w[1] & m, (w[1] >> 8) & m,
                               w[2] & m, (w[2] >> 8) & m, w[3] & m, (w[3] >> 8) & m};
        const int rr = 2 * blk2 + half;
        t += dot8(f, xs[2 * rr], xs[2 * rr + 1]) * invs[rr];
      }
      const float d = f16_bits_to_f32_fast(blk2 == 0 ? uint16_t(r[0]) : uint16_t(r[8] >> 16));
      const float xsum = sums[2 * blk2] + sums[2 * blk2 + 1];
      acc = fmaf(d, kTwo24 * t - 128.0f * xsum, acc);
    }
    return acc;
  }
};

// ------------------------------------------------------------- planning

// Item shape of one format: columns per item (the last item of a row may
// hold fewer), items per matrix row, 16-byte chunks per row segment, and
// 1 KB copy pieces per item.
struct RingShape {
  int cols, last_cols, nkr;
  int cpr, cpr_last;
  int pieces, pieces_last;
};

struct RingPlan {
  RingShape routed, shared;
  int tiles_i;         // 16-row tiles of a routed matrix
  int S, R;            // shared and routed jobs
  int x_pieces;        // 1 KB copies of the staged activation row
  uint32_t x_bytes;    // staged activation bytes
};

inline void ring_pieces(RingShape& s) {
  s.pieces = (kRows * s.cpr * 16 + 1023) / 1024;
  s.pieces_last = (kRows * s.cpr_last * 16 + 1023) / 1024;
}

// Shared (Q8_0) items: as many columns as fit 16 rows in a slot with 16-byte
// aligned row segments, evened out over the row.
inline bool ring_shape_q8(int nsb, RingShape& s) {
  constexpr int bytes = 272;
  int mx = kSlotBytes / (kRows * bytes);
  while (mx > 0 && (mx * bytes) % 16) --mx;
  if (mx <= 0) return false;
  const int nkr = (nsb + mx - 1) / mx;
  int cols = (nsb + nkr - 1) / nkr;
  while ((cols * bytes) % 16) ++cols;
  if (cols > mx) cols = mx;
  s.cols = cols;
  s.nkr = (nsb + cols - 1) / cols;
  s.last_cols = nsb - (s.nkr - 1) * cols;
  if ((s.last_cols * bytes) % 16) return false;
  s.cpr = cols * bytes / 16;
  s.cpr_last = s.last_cols * bytes / 16;
  ring_pieces(s);
  return true;
}

// Routed Q2_K items: 8 columns each, so the row needs a multiple of 8 super-blocks.
inline bool ring_shape_q2k(int nsb, RingShape& s) {
  constexpr int cols = RingFmt<INFERNO_Q2_K>::kCols;
  if (nsb % cols) return false;
  s.cols = s.last_cols = cols;
  s.nkr = nsb / cols;
  s.cpr = s.cpr_last = cols * RingFmt<INFERNO_Q2_K>::kBytes / 16;
  ring_pieces(s);
  return true;
}

// ------------------------------------------------------------- the kernel

// Routed Q2_K gate/up with the Q8_0 shared expert, one token. PW = copy
// instructions per copying wavefront per item (ceil(max pieces / 3)).
template <int PW>
__global__ void __launch_bounds__(256, 2) gate_up_ring_kernel(DecodeArgs p, RingPlan pl) {
  using FR = RingFmt<INFERNO_Q2_K>;
  using FS = RingFmt<INFERNO_Q8_0>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, g = blockIdx.x;
  const int H = p.H;
  const int nsb_h = H / kKBlock;

  // this workgroup's jobs: workgroups [0, S) take one shared tile each, the
  // others the routed tiles round robin
  const bool shared_wg = g < pl.S;
  int njobs, job0 = 0, jstep = 1;
  if (shared_wg) {
    njobs = 1;
    job0 = g;
  } else {
    const int gr = g - pl.S, Gr = G - pl.S;
    njobs = gr < pl.R ? (pl.R - gr + Gr - 1) / Gr : 0;
    job0 = gr;
    jstep = Gr;
  }
  if (njobs == 0) return;
  const RingShape& sh = shared_wg ? pl.shared : pl.routed;
  const int ipj = 2 * sh.nkr;  // items per job
  const int nitems = njobs * ipj;
  const int kbytes = shared_wg ? FS::kBytes : FR::kBytes;
  const size_t rb = size_t(nsb_h) * kbytes;

  const uint32_t x_off = lds_off(lds);
  const uint32_t part_off = x_off + uint32_t(pl.x_pieces) * 1024;
  uint8_t* ring = lds + pl.x_pieces * 1024 + kPartFloats * 4;
  const uint32_t ring_off = lds_off(ring);
  const XLds xl{x_off, x_off + uint32_t(H / 2) * 4, x_off + uint32_t(H / 2 + H / 16) * 4};

  // this lane's copy offsets, the same for every item of a shape: piece i of
  // wavefront w is min(w + 3 i, pieces - 1); its lane chunk (clamped to the
  // item) sits at row c / cpr, byte 16 (c % cpr) of the row segment
  uint32_t off_full[PW], off_last[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    {
      const int piece = min(wave + kDmaWaves * i, sh.pieces - 1);
      const int c = min(piece * 64 + lane, kRows * sh.cpr - 1);
      off_full[i] = uint32_t(c / sh.cpr) * uint32_t(rb) + uint32_t(c % sh.cpr) * 16;
    }
    {
      const int piece = min(wave + kDmaWaves * i, sh.pieces_last - 1);
      const int c = min(piece * 64 + lane, kRows * sh.cpr_last - 1);
      off_last[i] = uint32_t(c / sh.cpr_last) * uint32_t(rb) + uint32_t(c % sh.cpr_last) * 16;
    }
  }

  // slot descriptors of the routed slots (lane j holds slot j), loaded once:
  // a vector load waited for later would wait for every copy issued after it
  uint32_t slot_e = 0, slot_a = 0;
  struct Item {
    const uint8_t* base;  // row 0, first column of the item
    int cols, col0, mat;
    bool lastc, last;     // last column range of its matrix / last item of its job
  };
  auto item = [&](int ord) -> Item {
    const int ji = ord / ipj, ii = ord - ji * ipj;
    const int job = job0 + ji * jstep;
    const int mat = ii / sh.nkr, kr = ii - mat * sh.nkr;
    Item d;
    d.mat = mat;
    d.last = ii == ipj - 1;
    d.lastc = kr == sh.nkr - 1;
    d.col0 = kr * sh.cols;
    d.cols = d.lastc ? sh.last_cols : sh.cols;
    const uint8_t* m;
    if (shared_wg) {
      m = (mat ? p.sup : p.sgate) + size_t(job) * kRows * rb;
    } else {
      const int j = job / pl.tiles_i, tile = job - j * pl.tiles_i;
      const uint32_t e = __builtin_amdgcn_readlane(slot_e, j);
      m = (mat ? p.up : p.gate) + size_t(e) * p.gate_stride + size_t(tile) * kRows * rb;
    }
    d.base = m + size_t(d.col0) * kbytes;
    return d;
  };
  // copy item `ord` into ring slot ord % kDepth
  auto issue = [&](int ord) {
    const Item d = item(ord);
    uint8_t* slot = ring + (ord % kDepth) * kSlotBytes;
    const int np = d.lastc ? sh.pieces_last : sh.pieces;
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int piece = min(wave + kDmaWaves * i, np - 1);
      const uint8_t* src = d.base + (d.lastc ? off_last[i] : off_full[i]);
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)(slot + piece * 1024), 16, 0, 0);
    }
  };

  const bool copier = wave < kDmaWaves;
  if (copier) {
    // staged activation row (x_pieces KB, repeated last chunk past its end)
    const int xchunks = int(pl.x_bytes / 16);
    const int xpw = (pl.x_pieces + kDmaWaves - 1) / kDmaWaves;
    for (int i = 0; i < xpw; ++i) {
      const int piece = min(wave + kDmaWaves * i, pl.x_pieces - 1);
      int c = min(piece * 64 + lane, xchunks - 1);
      if (c < H / 8) {  // hi pairs: 32 chunks per column, 16 per half, 4 per block
        const int col = c >> 5, h = (c >> 4) & 1, b = (c >> 2) & 3;
        c = (c & ~12) | ((b ^ x_swizzle(col, h)) << 2);
      }
      __builtin_amdgcn_global_load_lds(
          (const void*)(reinterpret_cast<const uint8_t*>(p.stage_x) + size_t(c) * 16),
          (lds_ptr_t)(lds + piece * 1024), 16, 0, 0);
    }
  }
  if (!shared_wg) {
    if (lane < p.k) {
      const uint4 sl = p.slots[lane];
      slot_e = sl.x;
      slot_a = sl.w;
    }
    wait_vm<0>();  // the activation copy is in flight alongside this round trip
  }
  if (copier) {
#pragma unroll
    for (int o = 0; o < kDepth - 1; ++o)
      if (o < nitems) issue(o);
  }

  // routed lanes: sub = lane & 3, column 2 wave + ((lane >> 2) & 1), rows
  // lane >> 3 and + 8; shared lanes: sub = lane & 3, row lane >> 2,
  // columns wave, wave + 4, ...
  const int sub = lane & 3;
  const int rrow = lane >> 3, rcol = 2 * wave + ((lane >> 2) & 1);
  const int srow = lane >> 2;
  float acc[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
  int job_ord = 0;
  for (int n = 0; n < nitems; ++n) {
    if (copier) {
      const int newer = min(nitems - 1 - n, kDepth - 2);
      if (newer >= 2) wait_vm<2 * PW>();
      else if (newer == 1) wait_vm<PW>();
      else wait_vm<0>();
    }
    __builtin_amdgcn_s_barrier();
    if (copier && n + kDepth - 1 < nitems) issue(n + kDepth - 1);
    const Item d = item(n);
    const uint32_t slot = ring_off + uint32_t((n % kDepth) * kSlotBytes);
    float a0 = 0.f, a1 = 0.f;
    if (shared_wg) {
      const uint32_t seg = uint32_t(d.cols * FS::kBytes);
      for (int c = wave; c < d.cols; c += 4)
        a0 += FS::dot(slot + uint32_t(srow) * seg + uint32_t(c * FS::kBytes), sub, xl, d.col0 + c);
    } else {
      FR::dot2(slot + uint32_t(rrow) * FR::kSeg + uint32_t(rcol * FR::kBytes), sub, xl,
               d.col0 + rcol, a0, a1);
    }
    acc[d.mat][0] += a0;
    acc[d.mat][1] += a1;
    if (d.last) {
      // sum the sub-lanes (and for routed lanes the two columns), then the
      // wavefronts in LDS
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        if (shared_wg) {
          const float v = quad_sum(acc[m][0]);
          if (sub == 0) wr1(part_off + uint32_t(((m * 4 + wave) * kRows + srow) * 4), v);
        } else {
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            float v = quad_sum(acc[m][r]);
            v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v),
                                                                    0x141, 0xF, 0xF, false));
            if ((lane & 7) == 0) wr1(part_off + uint32_t(((m * 4 + wave) * kRows + rrow + 8 * r) * 4), v);
          }
        }
        acc[m][0] = acc[m][1] = 0.f;
      }
      __builtin_amdgcn_s_barrier();
      if (wave == 3) {
        const int s = lane & 15;
        const uint32_t pa = part_off + uint32_t(s * 4);
        float gsum, usum;
        {
          uint32_t g0, g1, g2, g3, u0, u1, u2, u3;
          asm volatile(
              "s_waitcnt lgkmcnt(0)\n"
              "ds_read_b32 %0, %8 offset:0\n"
              "ds_read_b32 %1, %8 offset:64\n"
              "ds_read_b32 %2, %8 offset:128\n"
              "ds_read_b32 %3, %8 offset:192\n"
              "ds_read_b32 %4, %8 offset:256\n"
              "ds_read_b32 %5, %8 offset:320\n"
              "ds_read_b32 %6, %8 offset:384\n"
              "ds_read_b32 %7, %8 offset:448\n"
              "s_waitcnt lgkmcnt(0)"
              : "=&v"(g0), "=&v"(g1), "=&v"(g2), "=&v"(g3), "=&v"(u0), "=&v"(u1), "=&v"(u2),
                "=&v"(u3)
              : "v"(pa));
          gsum = ((__uint_as_float(g0) + __uint_as_float(g1)) + __uint_as_float(g2)) +
                 __uint_as_float(g3);
          usum = ((__uint_as_float(u0) + __uint_as_float(u1)) + __uint_as_float(u2)) +
                 __uint_as_float(u3);
        }
        const int job = job0 + job_ord * jstep;
        if (shared_wg) {
          const float v = silu(gsum) * usum;
          stage_run_lanes(v, p.stage_hs, p.Is, job);
        } else {
          const int j = job / pl.tiles_i, tile = job - j * pl.tiles_i;
          const uint32_t asg = __builtin_amdgcn_readlane(slot_a, j);  // the slot's assignment
          const float v = silu(gsum) * usum * p.weights[asg];
          stage_run_lanes(v, p.stage_h + size_t(asg) * staged_stride(p.I, true), p.I, tile);
        }
      }
      ++job_ord;
    }
  }
}

}  // namespace ring
}  // namespace inferno
