// Host-side check of the LDS layout of the one-token fp8 x fp4 gate/up
// kernel (gate_up_fp4_kernel, decode_mfma.hpp), for every shape it is
// instantiated for (Q2_K with 4..28 super-block columns, Q3_K with 8, 16,
// 24), with and without the selection (SEL) and with every shared-expert
// width whose down runs in that launch.
//
// The byte ranges each phase of the kernel writes are replayed on the host
// from the kernel's own index formulas, against the layout function the
// kernel takes its region pointers from (fp4_lds_layout). Checked:
//   - every write lands inside its region, and every region inside the
//     allocation the launcher requests (lds_bytes);
//   - regions are pairwise disjoint (all of them: the kernel's lifetimes
//     overlap for most pairs);
//   - alignment of the vector accesses (16 bytes for uint4 / LDS DMA, 8 for
//     Top1Lds);
//   - each wavefront's LDS-DMA rows (SharedDownSlice::fetch_lds) stay inside
//     its own area, so no wavefront's copies reach rows another one dots;
//   - every output row of the shared down (ys) is owned by exactly one
//     (workgroup, thread) for the grid the launcher uses;
// Not replayed here, as it holds by construction: after the selection
// barrier the kernel writes LDS only to tl, part and sdpart (the down
// warm-up loads registers, not LDS), so the DMA-written sdl rows and the
// staged hsd row are never rewritten while the shared down reads them.
// Prints one line per checked shape and "OK <n>" at the end; exits non-zero
// on the first failure. Built and run by tests/test_lds_layout.py (CPU).
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "decode_mfma.hpp"

using namespace inferno;
using namespace inferno::mfma_decode;

namespace {

struct Region {
  const char* name;
  int lo, hi;  // [lo, hi) bytes
};

int fails = 0;
#define CHECK(c, ...)                        \
  do {                                       \
    if (!(c)) {                              \
      std::fprintf(stderr, "FAIL: " __VA_ARGS__); \
      std::fprintf(stderr, "\n");            \
      ++fails;                               \
      return false;                          \
    }                                        \
  } while (0)

bool inside(const Region& r, int lo, int hi) { return lo >= r.lo && hi <= r.hi; }

bool check_shape(int quant, int NB, bool sel, int Is_sd, int cus) {
  const int H = NB * kKBlock;
  const Fp4Lds L = fp4_lds_layout(H, quant, sel, Is_sd);
  const int alloc = int(lds_bytes(H, quant, sel, Is_sd));
  const int kB = fp4_block_bytes(quant), rb = NB * kB, RS = rb + kRowPad;
  const int Sm = stage_words(H);
  std::vector<Region> R = {
      {"xs", L.xs, L.zero},          {"zero", L.zero, L.tl},         {"tl", L.tl, L.part},
      {"part", L.part, L.slot_e},    {"slot_e", L.slot_e, L.slot_a}, {"slot_a", L.slot_a, L.slot_w},
      {"slot_w", L.slot_w, L.slot_w + kMaxExperts * 4},
  };
  if (sel) {
    R.push_back({"tk", L.tk, L.sdpart});
    R.push_back({"sdpart", L.sdpart, L.hsd});
    if (Is_sd) {
      R.push_back({"hsd", L.hsd, L.hsd + staged_stride(Is_sd, false) * 4});
      R.push_back({"sdl", L.sdl, L.sdl + L.sdl_bytes});
    }
  }
  CHECK(alloc == L.end, "alloc %d != layout end %d", alloc, L.end);
  for (const Region& r : R) {
    CHECK(r.lo >= 0 && r.lo <= r.hi && r.hi <= alloc, "%s [%d,%d) outside [0,%d)", r.name, r.lo,
          r.hi, alloc);
  }
  for (size_t i = 0; i < R.size(); ++i)
    for (size_t j = i + 1; j < R.size(); ++j)
      CHECK(R[i].hi <= R[j].lo || R[j].hi <= R[i].lo, "%s [%d,%d) overlaps %s [%d,%d)", R[i].name,
            R[i].lo, R[i].hi, R[j].name, R[j].lo, R[j].hi);
  auto reg = [&](const char* n) -> const Region& {
    for (const Region& r : R)
      if (std::string(r.name) == n) return r;
    std::fprintf(stderr, "no region %s\n", n);
    std::exit(2);
  };
  CHECK(L.xs % 16 == 0 && L.zero % 16 == 0 && L.tl % 16 == 0 && RS % 16 == 0 && L.part % 16 == 0,
        "vector alignment");
  CHECK(L.tk % 8 == 0, "Top1Lds alignment");
  // prologue: staged x copy (Sm / 4 uint4), zero (4 words)
  CHECK(inside(reg("xs"), L.xs, L.xs + (Sm / 4) * 16), "xs copy");
  CHECK(Sm % 4 == 0, "xs copy covers Sm words");
  CHECK(inside(reg("zero"), L.zero, L.zero + 16), "zero");
  // loop: tl stores of chunk i < 2 nv (nv = rb 16-byte chunks per matrix:
  // 16 rows of rb bytes), held PER per thread
  {
    const int nv = rb, PER = chunks_per_thread(NB, kB);
    CHECK(2 * nv <= PER * kThreads, "a thread holds at most PER chunks of the tile");
    int mx = 0;
    for (int i = 0; i < 2 * nv; ++i) {
      const int mat = i >= nv, rem = i - mat * nv, row = rem / (rb / 16), c16 = rem - row * (rb / 16);
      CHECK(row < 16 && c16 < rb / 16, "tile chunk %d maps to row %d", i, row);
      mx = std::max(mx, L.tl + (mat * 16 + row) * RS + c16 * 16 + 16);
    }
    CHECK(inside(reg("tl"), L.tl, mx), "tl stores end at %d past %d", mx, reg("tl").hi);
  }
  // loop: part[(wave * 2 + m) * 16 + n]
  CHECK(inside(reg("part"), L.part, L.part + ((kWaves - 1) * 2 + 1) * 16 * 4 + 16 * 4), "part");
  if (!sel) return true;
  CHECK(inside(reg("tk"), L.tk, L.tk + int(sizeof(Top1Lds))), "tk");
  CHECK(inside(reg("sdpart"), L.sdpart, L.sdpart + kWaves * 8 * 4), "sdpart");
  if (!Is_sd) return true;
  // the launcher's grid and the rows a workgroup takes (sel_in_gate_up)
  const int tiles = 8 * (2048 / kRows);  // any ntiles >= cus gives grid = cus
  const int G = std::min(tiles, cus);
  const int rw = 8 * ((H / 8 + G - 1) / G);
  if (rw > 8 * kSdMaxOctets) return true;  // the launcher keeps the select launch
  // hsd: form_shared_h writes uint2 at words run * 8 + 2 qi (run < Is / 16),
  // and the sums at Is / 2 + run, Is / 2 + Is / 16 + run
  CHECK(L.hsd % 8 == 0, "hsd alignment");
  CHECK(inside(reg("hsd"), L.hsd, L.hsd + (Is_sd / 2) * 4), "hsd pairs");
  CHECK(inside(reg("hsd"), L.hsd, L.hsd + (Is_sd / 2 + Is_sd / 8) * 4), "hsd sums");
  // sdl: wavefront w < octets * kSdWpo copies chunks [b, b + 64) of its area
  CHECK(L.sdl % 16 == 0, "sdl alignment");
  for (int b0 = 0; b0 < G; ++b0) {
    const int row0 = b0 * rw, rows = std::max(0, std::min(rw, H - row0));
    const int waves = (rows / 8) * kSdWpo;
    CHECK(waves <= kSdMaxOctets * kSdWpo && waves <= kWaves - 1,
          "shared-down wavefronts %d must leave the selection wavefront alone", waves);
    for (int w = 0; w < waves; ++w) {
      const int nu = std::max(0, std::min(2, Is_sd / kKBlock - 2 * (w % kSdWpo)));
      if (!nu) continue;
      const int cpr = nu * (SharedDownSlice::FS::kBytes / 16), nch = 8 * cpr;
      const int area = L.sdl + w * SharedDownSlice::kWaveLds;
      for (int c0 = 0; c0 < nch; c0 += kWave) {
        const int b = std::min(c0, nch - kWave);
        CHECK(b >= 0, "a copy of 64 chunks fits the octet (nch %d)", nch);
        const int lo = area + b * 16, hi = area + (b + kWave) * 16;
        CHECK(lo >= area && hi <= area + SharedDownSlice::kWaveLds,
              "wavefront %d copy [%d,%d) leaves its area", w, lo, hi);
        CHECK(inside(reg("sdl"), lo, hi), "sdl copy");
      }
      // dot_lds reads row r at (r * nu + cp) * 272 + sub * 68, 68 bytes
      for (int r = 0; r < 8; ++r)
        for (int cp = 0; cp < nu; ++cp)
          for (int sub = 0; sub < 4; ++sub) {
            const int lo = area + (r * nu + cp) * SharedDownSlice::FS::kBytes + sub * 68;
            CHECK(lo + 68 <= area + nch * 16, "dot_lds reads past the copied rows");
          }
    }
  }
  // ys rows: row0 + i for i < rows, one owner each
  std::vector<int> own(H, 0);
  for (int b0 = 0; b0 < G; ++b0) {
    const int row0 = b0 * rw, rows = std::max(0, std::min(rw, H - row0));
    for (int i = 0; i < rows; ++i) own[row0 + i]++;
  }
  for (int r = 0; r < H; ++r) CHECK(own[r] == 1, "ys row %d written %d times", r, own[r]);
  return true;
}

}  // namespace

int main(int argc, char** argv) {
  const int cus = argc > 1 ? std::atoi(argv[1]) : 256;
  int n = 0;
  struct S {
    int q, nb;
  };
  std::vector<S> shapes;
  for (int nb = 4; nb <= 28; nb += 4) shapes.push_back({INFERNO_Q2_K, nb});
  for (int nb : {8, 16, 24}) shapes.push_back({INFERNO_Q3_K, nb});
  for (const S& s : shapes)
    for (int sel = 0; sel < 2; ++sel)
      for (int Is = 0; Is <= 2 * kKBlock * kSdWpo; Is += kKBlock) {
        if (!sel && Is) continue;
        if (size_t(fp4_lds_layout(s.nb * kKBlock, s.q, sel, Is).end) > 160 * 1024) continue;
        if (!check_shape(s.q, s.nb, sel, Is, cus)) {
          std::fprintf(stderr, "shape q=%d NB=%d sel=%d Is=%d\n", s.q, s.nb, sel, Is);
          return 1;
        }
        std::printf("q=%d NB=%d sel=%d Is=%d end=%d\n", s.q, s.nb, sel, Is,
                    fp4_lds_layout(s.nb * kKBlock, s.q, sel, Is).end);
        ++n;
      }
  std::printf("OK %d\n", n);
  return fails ? 1 : 0;
}
