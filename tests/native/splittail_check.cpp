// Host-side check of version 9's tail schedule and version 11's split of
// under-filled grids (vk_splittail.hpp): simulates every workgroup of a
// launch for many tile counts, k-depths and CU counts -- for the plan sk_plan
// (or sk_plan_fill) chooses and, for sk_plan, every other admissible piece
// count -- and checks that the pieces cover each (tile, k-iteration) exactly
// once and that the pieces of a split tile agree on where they meet.
// Prints "ok <cases> <split plans>" or the first violation; exit status 1 on a
// violation.
#include "vk_splittail.hpp"

#include <cstdio>
#include <set>
#include <vector>

using namespace vk;

static int fail(const char* what, int tm, int tn, int I, int C, const SkPlan& p) {
  std::printf("FAIL %s: tiles %dx%d, I %d, C %d, plan dp %d units %d pieces %d chunks %d\n", what, tm, tn, I, C,
              p.dp, p.units, p.pieces, p.chunks);
  return 1;
}

static int check_plan(int tiles_m, int tiles_n, int I, int C, const SkPlan& p, int extra = kSkLastExtra) {
  const int T = tiles_m * tiles_n;
  const int grid = p.dp + p.units;
  std::vector<int> cover((size_t)T * I, 0);
  std::set<std::pair<int, int>> tiles_seen;
  std::vector<SkWork> work(grid);
  for (int bid = 0; bid < grid; bid++) {
    const SkWork w = sk_work(bid, T, I, p, extra);
    work[bid] = w;
    if (w.cid < 0 || w.cid >= T || w.kb < 0 || w.ke > I || w.kb >= w.ke) return fail("work range", tiles_m, tiles_n, I, C, p);
    for (int k = w.kb; k < w.ke; k++) cover[(size_t)w.cid * I + k]++;
    int tm, tn;
    raster_tile(w.cid, tiles_m, tiles_n, tm, tn);
    if (tm < 0 || tm >= tiles_m || tn < 0 || tn >= tiles_n) return fail("raster out of range", tiles_m, tiles_n, I, C, p);
    tiles_seen.insert({tm, tn});
    if (bid < p.dp) {
      if (w.np != 1 || w.kb != 0 || w.ke != I) return fail("whole tile split", tiles_m, tiles_n, I, C, p);
      continue;
    }
    if (w.np != p.pieces || w.p < 0 || w.p >= w.np) return fail("piece index", tiles_m, tiles_n, I, C, p);
    if (w.ke - w.kb < (I - extra) / p.pieces || w.ke - w.kb < 1)
      return fail("piece shorter than (I - extra) / pieces", tiles_m, tiles_n, I, C, p);
    if (w.p == w.np - 1 && w.ke - w.kb < (I - extra) / p.pieces + extra)
      return fail("last piece without its extra iterations", tiles_m, tiles_n, I, C, p);
    if ((size_t)(w.tile + 1) * kSkWaves > kSkCounterBytes / sizeof(unsigned)) return fail("counter out of range", tiles_m, tiles_n, I, C, p);
    if (sk_unit_of(p, T, w.tile, w.p) != bid - p.dp) return fail("unit_of(own piece) != self", tiles_m, tiles_n, I, C, p);
    if (p.chunks == 8) {
      const int x = bid % 8;  // the XCD this workgroup is dealt to
      if (w.cid / (T / 8) != x) return fail("tile off its XCD share", tiles_m, tiles_n, I, C, p);
    }
  }
  for (int v : cover)
    if (v != 1) return fail("iteration not covered exactly once", tiles_m, tiles_n, I, C, p);
  if ((int)tiles_seen.size() != T) return fail("raster not a bijection", tiles_m, tiles_n, I, C, p);
  // The meeting points: piece q of every split tile is where each piece looks.
  std::set<int> tiles_split, cids_split;
  for (int bid = p.dp; bid < grid; bid++) {
    const SkWork& w = work[bid];
    tiles_split.insert(w.tile);
    cids_split.insert(w.cid);
    for (int q = 0; q < w.np; q++) {
      const int u = sk_unit_of(p, T, w.tile, q);
      if (u < 0 || u >= p.units) return fail("partner unit out of range", tiles_m, tiles_n, I, C, p);
      const SkWork& o = work[p.dp + u];
      if (o.tile != w.tile || o.cid != w.cid || o.p != q) return fail("partner is not piece q of this tile", tiles_m, tiles_n, I, C, p);
      if (q + 1 < w.np && o.ke != work[p.dp + sk_unit_of(p, T, w.tile, q + 1)].kb)
        return fail("pieces not contiguous in k order", tiles_m, tiles_n, I, C, p);
    }
  }
  if (tiles_split.size() != cids_split.size()) return fail("tail tile numbering not one-to-one", tiles_m, tiles_n, I, C, p);
  return 0;
}

// xcd_remap is a bijection of [0, total) whose image of the workgroups of
// XCD x (bid % 8 == x) is one contiguous range, the ranges in XCD order.
static int check_remap() {
  for (int total = 1; total <= 4200; total++) {
    std::vector<int> lo(8, total), hi(8, -1), cnt(8, 0), seen(total, 0);
    for (int b = 0; b < total; b++) {
      const int c = xcd_remap(b, total), x = b % 8;
      if (c < 0 || c >= total || seen[c]++) {
        std::printf("FAIL xcd_remap not a bijection: total %d\n", total);
        return 1;
      }
      lo[x] = c < lo[x] ? c : lo[x];
      hi[x] = c > hi[x] ? c : hi[x];
      cnt[x]++;
    }
    int next = 0;
    for (int x = 0; x < 8; x++) {
      if (cnt[x] == 0) continue;
      if (lo[x] != next || hi[x] - lo[x] + 1 != cnt[x]) {
        std::printf("FAIL xcd_remap share of XCD %d not contiguous: total %d\n", x, total);
        return 1;
      }
      next = hi[x] + 1;
    }
  }
  return 0;
}

int main() {
  if (check_remap()) return 1;
  long long cases = 0, split_plans = 0, forced = 0;
  const int Is[] = {1, 4, 8, 15, 16, 17, 31, 32, 43, 64, 65, 100, 128, 172, 256};
  const int Cs[] = {256, 240, 304, 80, 64, 8, 1};
  for (int tiles_m = 1; tiles_m <= 24; tiles_m++)
    for (int tiles_n = 1; tiles_n <= 48; tiles_n += (tiles_n < 16 ? 1 : 5))
      for (int I : Is)
        for (int C : Cs) {
          const int T = tiles_m * tiles_n;
          const SkPlan p = sk_plan(T, I, C);
          const int Cc = C < kSkMaxUnits ? C : kSkMaxUnits;
          if (p.units == 0) {
            if (p.dp != T || p.pieces != 1) return fail("whole plan", tiles_m, tiles_n, I, C, p);
          } else {
            split_plans++;
            const int r = T - p.dp;
            if (p.dp % Cc || p.dp != T / Cc * Cc || p.units != p.pieces * r || p.units > Cc || p.units % p.chunks ||
                p.pieces < 2 || p.pieces > kSkMaxPieces || I / p.pieces < kSkMinIters)
              return fail("plan shape", tiles_m, tiles_n, I, C, p);
          }
          if (check_plan(tiles_m, tiles_n, I, C, p)) return 1;
          cases++;
          // every other admissible piece count, as a plan of its own
          if (T % Cc == 0) continue;
          const int dp = T / Cc * Cc, r = T - dp;
          const int chunks = (T % 8 == 0) ? 8 : 1;
          if (chunks == 8 && dp % 8) continue;
          for (int s = 2; s <= kSkMaxPieces && s * r <= Cc && I / s >= kSkMinIters; s++) {
            if (check_plan(tiles_m, tiles_n, I, C, SkPlan{dp, s * r, s, chunks})) return 1;
            forced++;
          }
        }
  // Version 11's split of under-filled grids.
  long long fill_plans = 0;
  for (int tiles_m = 1; tiles_m <= 24; tiles_m++)
    for (int tiles_n = 1; tiles_n <= 48; tiles_n += (tiles_n < 16 ? 1 : 5))
      for (int I : Is)
        for (int C : Cs) {
          const int T = tiles_m * tiles_n;
          const SkPlan p = sk_plan_fill(T, I, C);
          const int Cc = C < kSkMaxUnits ? C : kSkMaxUnits;
          if (p.units == 0) {
            if (p.dp != T || p.pieces != 1) return fail("fill: whole plan", tiles_m, tiles_n, I, C, p);
            if (2 * T <= Cc && Cc / T >= 2 && I / kFillMinIters >= 2) return fail("fill: split missed", tiles_m, tiles_n, I, C, p);
            continue;
          }
          fill_plans++;
          if (p.dp != 0 || p.units != p.pieces * T || p.units > Cc || p.pieces < 2 || p.pieces > kFillMaxPieces ||
              I / p.pieces < kFillMinIters || p.chunks != (T % 8 == 0 ? 8 : 1))
            return fail("fill: plan shape", tiles_m, tiles_n, I, C, p);
          if (check_plan(tiles_m, tiles_n, I, C, p, kFillLastExtra)) return 1;
          cases++;
        }
  if (fill_plans == 0) {
    std::printf("FAIL no fill plan split anything\n");
    return 1;
  }
  // Plans the GPU tests rely on (256 CUs).
  struct Want { int T, I, dp, units, pieces, chunks; } wants[] = {
      {16 * 43, 64, 688, 0, 1, 1},    // 4096 x 11008 x 4096: 176 of 256 busy, left whole
      {8 * 8, 64, 0, 256, 4, 8},      // 2048 x 2048 x 4096
      {16 * 17, 64, 256, 64, 4, 8},   // 4096 x 4352 x 4096: 16 tail tiles
      {16 * 16, 64, 256, 0, 1, 1},    // 4096^3: one full wave
  };
  for (const Want& w : wants) {
    const SkPlan p = sk_plan(w.T, w.I, 256);
    if (p.dp != w.dp || p.units != w.units || p.pieces != w.pieces || p.chunks != w.chunks) {
      std::printf("FAIL plan for T %d I %d: dp %d units %d pieces %d chunks %d\n", w.T, w.I, p.dp, p.units, p.pieces,
                  p.chunks);
      return 1;
    }
  }
  struct WantFill { int T, I, units, pieces, chunks; } fills[] = {
      {4 * 32, 32, 256, 2, 8},  // 512 x 4096 x 4096
      {8 * 8, 32, 256, 4, 8},   // 1000 x 1000 x 4000
      {1 * 16, 18, 32, 2, 8},   // 128 x 2048 x 2304
      {3 * 5, 64, 120, 8, 1},   // 384 x 640 x 8192
      {2 * 3, 16, 12, 2, 1},    // 200 x 296 x 2000
      {8 * 8, 8, 0, 1, 1},      // 1000^3: 8 k-tiles, left whole
      {16 * 16, 32, 0, 1, 1},   // 2048 x 2048 x 4096: one full wave
  };
  for (const WantFill& w : fills) {
    const SkPlan p = sk_plan_fill(w.T, w.I, 256);
    if (p.units != w.units || p.pieces != w.pieces || (p.units && p.chunks != w.chunks)) {
      std::printf("FAIL fill plan for T %d I %d: units %d pieces %d chunks %d\n", w.T, w.I, p.units, p.pieces, p.chunks);
      return 1;
    }
  }
  std::printf("ok %lld cases, %lld split plans, %lld forced piece counts, %lld fill plans\n", cases, split_plans,
              forced, fill_plans);
  return 0;
}
