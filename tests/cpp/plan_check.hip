// Host-only check of the GEMV grid plans (nve_amd/csrc/w4_launch.h).  Persistent: for
// every wave of the grid, replays the kernel's tile walk (w4_persistent.h) and checks
// that every pointer it would load from belongs to a real matrix, that no wave has
// more tiles than its LDS result slots, and that every row tile is computed exactly
// once.  Runs on the CPU; makes no HIP runtime call.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../nve_amd/csrc/w4_launch.h"

static int failures = 0;
#define CHECK(c, ...)                   \
  do {                                  \
    if (!(c)) {                         \
      ++failures;                       \
      if (failures < 20) {              \
        std::printf("FAIL: " __VA_ARGS__); \
        std::printf("\n");              \
      }                                 \
    }                                   \
  } while (0)

static void check(const int* ns, int nseg, int K, int occ, int depth) {
  static uint8_t fake_nib[3][16];
  static float fake_sc[3][4];
  W4Segs s{};
  s.nseg = nseg;
  for (int i = 0; i < nseg; ++i) {
    s.nib[i] = fake_nib[i];
    s.sc[i] = fake_sc[i];
    s.out[i] = fake_sc[i];
    s.n[i] = ns[i];
  }
  const W4Tiling t = choose_persistent_tiling(K, depth);
  const int grid = plan_persistent(s, t.R, 4 * 256 * occ);
  if (grid <= 0) return;  // the launcher falls back to the one-shot kernel
  std::vector<std::vector<int>> seen(nseg);
  for (int i = 0; i < nseg; ++i) seen[i].assign((ns[i] + t.R - 1) / t.R, 0);
  for (int w = 0; w < grid * 4; ++w) {
    const W4Wave wv = resolve_wave(s, w);
    int sg = -1;
    for (int i = 0; i < nseg; ++i)
      if (wv.nib == s.nib[i]) sg = i;
    CHECK(sg >= 0, "wave %d of K=%d maps to no matrix", w, K);
    if (sg < 0) continue;
    const int T = wv.tiles, W = wv.stride, t0 = wv.t0;
    const int first = t0 < T ? t0 : 0;  // the unconditional first prefetch
    CHECK(first >= 0 && first < (int)seen[sg].size(), "first tile %d out of range", first);
    if (t0 >= T) continue;
    CHECK(W >= 1, "stride %d", W);
    const int want = (T - t0 + W - 1) / W;
    CHECK(want <= kPersistentMaxTilesPerWave, "wave %d has %d tiles", w, want);
    const int cnt = want < kPersistentMaxTilesPerWave ? want : kPersistentMaxTilesPerWave;
    for (int i = 0; i < cnt; ++i) {
      const int tile = t0 + i * W;
      CHECK(tile < T, "tile %d >= %d", tile, T);
      if (tile < T) seen[sg][tile]++;
      const int tn = t0 + (i + 1) * W;
      const int pre = i + 1 < cnt ? tn : 0;
      CHECK(pre >= 0 && pre < T, "prefetch tile %d out of range", pre);
      const int row_last = tile * t.R + t.R - 1;
      (void)row_last;  // rows past n are clamped to n-1 by the kernel
    }
  }
  for (int i = 0; i < nseg; ++i)
    for (size_t j = 0; j < seen[i].size(); ++j)
      CHECK(seen[i][j] == 1, "K=%d seg %d tile %zu computed %d times", K, i, j, seen[i][j]);
}

// One-shot tiling (choose_w4_tiling): the (R, NJ) it returns is a compiled case, the
// grid covers every row, the rows-per-wave reduction never leaves the grid less
// balanced than the rule it replaced, and the 8B gate gets the balanced 1792-workgroup
// grid.
static bool compiled_case(const W4Tiling& t) {
#define NVE_CASE(RR, JJ, MM) if (t.R == RR && t.NJ == JJ && t.multi == MM) return true;
  NVE_W4_TILING_CASES(NVE_CASE)
#undef NVE_CASE
  return false;
}

static void check_oneshot(const int* ns, int nseg, int K) {
  W4Segs s{};
  s.nseg = nseg;
  long rows = 0;
  for (int i = 0; i < nseg; ++i) {
    s.n[i] = ns[i];
    rows += ns[i];
  }
  const W4Tiling t = choose_w4_tiling(s, K);
  CHECK(compiled_case(t), "K=%d rows=%ld: tiling R=%d NJ=%d not compiled", K, rows, t.R, t.NJ);
  finalize_segments(s, t.R);
  for (int i = 0; i < nseg; ++i) {
    const int wgs = (i + 1 < nseg ? s.wg_begin[i + 1] : s.wg_total) - s.wg_begin[i];
    CHECK((long)wgs * 4 * t.R >= ns[i], "K=%d seg %d: %d workgroups of %d rows miss rows of %d", K, i, wgs,
          4 * t.R, ns[i]);
  }
  // against doubling R (the rows per wave the balance step may have halved)
  if (t.R < 8) {
    long w2 = 0;
    for (int i = 0; i < nseg; ++i) w2 += (ns[i] + 8L * t.R - 1) / (8L * t.R);
    const double mine = w4_grid_imbalance(s.wg_total), doubled = w4_grid_imbalance(w2);
    CHECK(mine <= 1.05 || mine <= doubled || w2 < 512, "K=%d rows=%ld: imbalance %.3f worse than %.3f", K, rows,
          mine, doubled);
  }
}

int main() {
  {
    const int gate = 14336;
    W4Segs s{};
    s.nseg = 1;
    s.n[0] = gate;
    const W4Tiling t = choose_w4_tiling(s, 4096);
    finalize_segments(s, t.R);
    CHECK(t.R == 2 && s.wg_total == 1792, "8B gate: R=%d, %d workgroups", t.R, s.wg_total);
  }
  const int Ks[] = {32, 64, 96, 2048, 3072, 4096, 8192, 14336, 16384};
  const int Ns[] = {1, 2, 3, 5, 37, 512, 1000, 1024, 3072, 4096, 8192, 14336, 128256, 151936};
  const int Kos[] = {32, 64, 96, 2048, 3072, 4096, 8192, 14336, 16384, 16416, 32768};
  for (int K : Kos) {
    for (int n : Ns) check_oneshot(&n, 1, K);
    const int qkv[3] = {3072, 1024, 1024}, odd[3] = {5, 4000, 37}, gu[2] = {14336, 14336};
    check_oneshot(qkv, 3, K);
    check_oneshot(odd, 3, K);
    check_oneshot(gu, 2, K);
  }
  for (int K : Ks)
    for (int depth = 4; depth <= 8; depth += 4)
      for (int occ = 1; occ <= 8; occ *= 2) {
        for (int n : Ns) check(&n, 1, K, occ, depth);
        const int qkv[3] = {3072, 1024, 1024}, odd[3] = {5, 4000, 37}, big[3] = {14336, 14336, 1};
        check(qkv, 3, K, occ, depth);
        check(odd, 3, K, occ, depth);
        check(big, 3, K, occ, depth);
        const int gu[2] = {14336, 14336};
        check(gu, 2, K, occ, depth);
      }
  std::printf("%s (%d failures)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
