// Host-side fuzz of the library's planning and argument checks, built with
// AddressSanitizer and UndefinedBehaviorSanitizer on the host code only
// (tests/sanitize/build_fuzz.py).  It never launches a
// kernel and never dereferences an operand pointer: it calls the C ABI's
// host-only entry points (tile configuration, workspace size, ragged-round
// cut, block -> tile map) on seeded random problems, shapes from 0 to 2^24
// per dimension, strides from 0 to past the row, 2-byte to 256-byte aligned
// fake addresses (half the problems in clean layouts: 16-byte rows, aligned
// bases, as the fast kernels take them) and every forced tile, and the
// launching entry points with
// arguments they must reject before any launch.  The sanitizers report any
// out-of-bounds access, overflow or other undefined behaviour on these paths;
// the checks below assert the documented results.  Exit status 0: no
// mismatch (a sanitizer report aborts with a non-zero status).
//
//   usage: host_plan_fuzz [iterations]     (no GPU needed)

#include <cinttypes>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "f16acc.h"

namespace {

uint64_t g_state = 0x9e3779b97f4a7c15ull;
uint64_t next_u64() {  // splitmix64
  uint64_t z = (g_state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
int64_t uniform(int64_t lo, int64_t hi) { return lo + (int64_t)(next_u64() % (uint64_t)(hi - lo + 1)); }

// An extent: mostly model-like sizes, sometimes 0, 1, odd or very large.
int64_t extent() {
  switch (uniform(0, 9)) {
    case 0: return uniform(0, 2);
    case 1: return uniform(1, 64);
    case 2: return uniform(1, 600);
    case 3: return 64 * uniform(1, 160);
    case 4: return 256 * uniform(1, 64);
    case 5: return uniform(1, 20000);
    case 6: return 8 * uniform(1, 20000);
    case 7: return uniform(1, 1 << 24);
    case 8: return 151936;
    default: return 128 * uniform(1, 128) + uniform(-1, 1);
  }
}

// A stride for a dimension whose other dimension is `row` elements long.
int64_t stride(int64_t row) {
  switch (uniform(0, 6)) {
    case 0: return 0;                              // broadcast
    case 1: return 1;
    case 2: return row;                            // contiguous
    case 3: return row + uniform(1, 64);           // padded
    case 4: return 8 * ((row + 7) / 8);            // 16-byte rows
    case 5: return uniform(1, row > 8 ? row : 8);  // overlapping window
    default: return uniform(1, 1 << 20);
  }
}

const void* fake_ptr() {  // never dereferenced: only its alignment matters
  static const uintptr_t aligns[] = {2, 4, 8, 16, 256};
  return (const void*)(uintptr_t)(0x10000000ull + aligns[uniform(0, 4)] * uniform(1, 1000));
}

int g_fail = 0;
// coverage: the table's picks per tile, per family, workspace kinds, cuts
long g_pick[F16ACC_NUM_TILES], g_family[3], g_ws_none, g_ws_header, g_ws_split, g_cut_rows, g_cut_cols,
    g_unsupported;
void check(bool ok, const char* what, int64_t M, int64_t N, int64_t K) {
  if (ok) return;
  ++g_fail;
  if (g_fail <= 20) std::printf("MISMATCH %s at M=%" PRId64 " N=%" PRId64 " K=%" PRId64 "\n", what, M, N, K);
}

constexpr int kTileBm[F16ACC_NUM_TILES] = {256, 256, 128, 128, 128, 64, 128, 64, 256};
constexpr int kTileBn[F16ACC_NUM_TILES] = {256, 128, 256, 128, 128, 64, 96, 32, 288};

void fuzz_one() {
  const bool clean = uniform(0, 1);
  int64_t M = extent(), N = extent(), K = extent();
  if (clean) {  // 16-byte rows in either b layout
    K = 8 * ((K + 7) / 8);
    N = 8 * ((N + 7) / 8);
  }
  const bool kc = uniform(0, 1);
  const int64_t sam = clean ? K : stride(K), sak = clean || uniform(0, 3) ? 1 : stride(M);
  const int64_t sbk = kc ? 1 : clean ? N : stride(N), sbn = kc ? (clean ? K : stride(K)) : 1;
  const void* a = clean ? (const void*)(uintptr_t)0x10000000ull : fake_ptr();
  const void* b = clean ? (const void*)(uintptr_t)0x20000000ull : fake_ptr();

  for (int forced = -2; forced <= F16ACC_NUM_TILES; ++forced) {
    int tile = -1, bm = 0, bn = 0, fam = -1, thr = 0;
    int64_t tm = -1, tn = -1;
    const int rc = f16acc_tile_config(M, N, K, sam, sak, sbk, sbn, a, b, forced, &tile, &bm, &bn, &tm, &tn, &fam, &thr);
    if (forced < -1 || forced >= F16ACC_NUM_TILES) {
      check(rc == F16ACC_E_ARG, "tile_config accepts a bad tile id", M, N, K);
      continue;
    }
    check(rc == 0 || rc == F16ACC_E_UNSUPPORTED, "tile_config return code", M, N, K);
    if (rc != 0) {
      ++g_unsupported;
      continue;
    }
    if (forced == -1 && tile >= 0 && tile < F16ACC_NUM_TILES && fam >= 0 && fam < 3) {
      ++g_pick[tile];
      ++g_family[fam];
    }
    check(tile >= 0 && tile < F16ACC_NUM_TILES, "tile id out of range", M, N, K);
    if (tile < 0 || tile >= F16ACC_NUM_TILES) continue;
    check(bm == kTileBm[tile] && bn == kTileBn[tile], "tile shape", M, N, K);
    check(tm == (M + bm - 1) / bm && tn == (N + bn - 1) / bn, "tile grid", M, N, K);
    check(fam >= F16ACC_FAMILY_FAST && fam <= F16ACC_FAMILY_REG, "family", M, N, K);
    check(thr == 256 || thr == 512, "threads", M, N, K);
    // every output pointer may be NULL
    check(f16acc_tile_config(M, N, K, sam, sak, sbk, sbn, a, b, forced, nullptr, nullptr, nullptr, nullptr, nullptr,
                             nullptr, nullptr) == 0,
          "tile_config with NULL outputs", M, N, K);
  }

  size_t bytes = 12345;
  const int wrc = f16acc_workspace_size(M, N, K, sam, sak, sbk, sbn, a, b, &bytes);
  check(wrc == 0 || wrc == F16ACC_E_UNSUPPORTED, "workspace_size return code", M, N, K);
  if (wrc == 0) {
    check(bytes == 0 || bytes >= F16ACC_WS_HEADER, "workspace smaller than its header", M, N, K);
    ++(bytes == 0 ? g_ws_none : bytes == F16ACC_WS_HEADER ? g_ws_header : g_ws_split);
  }

  int64_t nsplit = 0;
  const int trc = f16acc_tail_split(M, N, K, sam, sak, sbk, sbn, a, b, &nsplit);
  check(trc == 0 || trc == F16ACC_E_UNSUPPORTED, "tail_split return code", M, N, K);
  if (trc == 0) {
    check((nsplit >= 0 && nsplit < (N > 0 ? N : 1)) || (nsplit < 0 && -nsplit < M), "tail cut", M, N, K);
    g_cut_cols += nsplit > 0;
    g_cut_rows += nsplit < 0;
  }

  // arguments the launching entry points reject before any launch
  uint8_t flags[4];
  char out[16];
  const int64_t bad[][3] = {{-1, N, K}, {M, -1, K}, {M, N, -1}};
  for (const auto& d : bad) {
    check(f16acc_gemm(a, b, out, flags, d[0], d[1], d[2], sam, sak, sbk, sbn, N, 1, F16ACC_OUT_F16, 1, nullptr) ==
              F16ACC_E_ARG,
          "gemm accepts a negative extent", M, N, K);
    check(f16acc_gemm_ws(a, b, nullptr, out, flags, d[0], d[1], d[2], sam, sak, sbk, sbn, N, 1, F16ACC_OUT_F32, 1,
                         nullptr, out, sizeof(out)) == F16ACC_E_ARG,
          "gemm_ws accepts a negative extent", M, N, K);
  }
  if (M > 0 && N > 0) {
    check(f16acc_gemm(a, b, nullptr, flags, M, N, K, sam, sak, sbk, sbn, N, 1, F16ACC_OUT_F16, 1, nullptr) ==
              F16ACC_E_ARG,
          "gemm accepts a NULL c", M, N, K);
    check(f16acc_gemm(a, b, out, flags, M, N, K, sam, sak, sbk, sbn, N, 1, 7, 1, nullptr) == F16ACC_E_ARG,
          "gemm accepts a bad out_dtype", M, N, K);
    check(f16acc_gemm(a, b, out, flags, M, N, K, sam, sak, sbk, sbn, N, 1, F16ACC_OUT_F16, 2, nullptr) == F16ACC_E_ARG,
          "gemm accepts a bad chunked flag", M, N, K);
    check(f16acc_gemm_tile(a, b, out, flags, M, N, K, sam, sak, sbk, sbn, N, 1, F16ACC_OUT_F16, 1, nullptr,
                           F16ACC_NUM_TILES) == F16ACC_E_ARG,
          "gemm_tile accepts a bad tile id", M, N, K);
    if (K > 0)
      check(f16acc_gemm(nullptr, b, out, flags, M, N, K, sam, sak, sbk, sbn, N, 1, F16ACC_OUT_F16, 1, nullptr) ==
                F16ACC_E_ARG,
            "gemm accepts a NULL a", M, N, K);
  }
  // zero-size outputs return at once, whatever the pointers
  check(f16acc_gemm(nullptr, nullptr, nullptr, nullptr, 0, N, K, 0, 0, 0, 0, 0, 0, F16ACC_OUT_F16, 1, nullptr) == 0,
        "gemm with M = 0", M, N, K);
  check(f16acc_gemm(nullptr, nullptr, nullptr, nullptr, M, 0, K, 0, 0, 0, 0, 0, 0, F16ACC_OUT_F16, 1, nullptr) == 0,
        "gemm with N = 0", M, N, K);
}

// The block -> tile map is a bijection on every grid up to 40 x 40, and
// rejects blocks outside the grid.
void block_map() {
  for (int64_t tm = 1; tm <= 40; ++tm)
    for (int64_t tn = 1; tn <= 40; ++tn) {
      std::vector<char> seen((size_t)(tm * tn), 0);
      for (int64_t blk = 0; blk < tm * tn; ++blk) {
        int64_t i = -1, j = -1;
        if (f16acc_block_tile(blk, tm, tn, &i, &j) != 0 || i < 0 || i >= tm || j < 0 || j >= tn ||
            seen[(size_t)(i * tn + j)]++) {
          check(false, "block_tile is not a bijection", tm, tn, blk);
          return;
        }
      }
      int64_t i, j;
      check(f16acc_block_tile(tm * tn, tm, tn, &i, &j) == F16ACC_E_ARG, "block_tile past the grid", tm, tn, 0);
      check(f16acc_block_tile(-1, tm, tn, &i, &j) == F16ACC_E_ARG, "block_tile below the grid", tm, tn, 0);
    }
}

}  // namespace

int main(int argc, char** argv) {
  const long iters = argc > 1 ? std::atol(argv[1]) : 3000;
  check(f16acc_abi_version() > 0, "abi version", 0, 0, 0);
  for (int code = -6; code <= 2; ++code) check(f16acc_strerror(code) != nullptr, "strerror", code, 0, 0);
  block_map();
  for (long it = 0; it < iters; ++it) fuzz_one();
  std::printf("table picks by tile:");
  for (int t = 0; t < F16ACC_NUM_TILES; ++t) std::printf(" %ld", g_pick[t]);
  std::printf("\nfamilies fast/generic/reg: %ld %ld %ld; unsupported: %ld\n", g_family[0], g_family[1], g_family[2],
              g_unsupported);
  std::printf("workspace none/header/split: %ld %ld %ld; ragged-round cuts by columns/rows: %ld %ld\n", g_ws_none,
              g_ws_header, g_ws_split, g_cut_cols, g_cut_rows);
  std::printf("host_plan_fuzz: %ld problems, %d mismatches\n", iters, g_fail);
  return g_fail ? 1 : 0;
}
