// vk_splittail.hpp -- the tail schedule of the 256x256-tile fp16 GEMM
// (version 9) and the split of under-filled 128x128-tile grids (version 11):
// which workgroup computes which k-range of which tile, and where the pieces
// of a split tile meet.  Host and device code share these
// functions, so the launch, the kernel and the schedule's own tests agree.
//
// With T tiles of I k-tile iterations each on C compute units (one workgroup
// per CU), the first dp = floor(T / C) * C tiles run whole, one per workgroup,
// in xcd_remap order.  The r = T - dp tail tiles would leave C - r CUs idle in
// the last wave; instead each is cut into s equal k-slices (s pieces, s * r <=
// C) computed by s workgroups at once, and the pieces are summed.
//
// Why equal, aligned slices rather than stream-K's equal shares of the
// flattened k-space (the reference's matmul_f16_v9_streamk.cu): measured on
// MI355X (4096 x 11008 x 4096, 176 tail tiles over 256 units of 44
// iterations), stream-K's units run at scattered k offsets, so the tiles of
// one XCD stop sharing A and B panels in its L2 and each k-iteration took
// 2.2-2.5 us instead of 1.5 us, and a piece hand-off costs 5-8 us (a 256 KB
// fp32 partial per workgroup out, and the last arrival reads the others back).
// With aligned slices, units on neighbouring tiles work on the same k-range
// at the same time, as whole tiles do, and every unit has exactly one piece.
//
// When T is divisible by 8 the whole tiles are the first dp / 8 raster
// positions of each XCD's share (xcd_remap) and the tail is the rest of each
// share: unit u runs on XCD u % 8 (dp is a multiple of 8) and takes the
// pieces of that XCD's r / 8 tail tiles ("chunks" = 8); otherwise there is one
// chunk: the whole tiles are positions [0, dp), dealt to the XCDs by
// xcd_remap over dp, and the tail the positions after them.
#pragma once

#include "vk_tile.hpp"

#include <cstdint>

namespace vk {

constexpr int kSkMaxUnits = 256;  // split-tail workgroups per launch, at most
constexpr int kSkMinIters = 8;    // k-tile iterations per piece, at least
constexpr int kSkMaxPieces = 8;   // pieces per tile, at most
constexpr int kSkWaves = 8;       // counters per tile (one per wave)

struct SkPlan {
  int dp;      // whole tiles: workgroups 0 .. dp-1
  int units;   // split-tail workgroups dp .. dp+units-1 (0: none)
  int pieces;  // k-slices per tail tile (units = pieces * tail tiles)
  int chunks;  // 8: units and tail tiles dealt per XCD; 1: one range
};

// First k-tile iteration of piece p of s.  The last piece gets kSkLastExtra
// more iterations than the others: they finish first and write their
// partials while it computes, so that when it finishes it usually finds them
// all in memory (the counter already at s - 1) and skips writing its own.
constexpr int kSkLastExtra = 3;
__host__ __device__ inline int sk_piece_begin(int p, int I, int s, int extra = kSkLastExtra) {
  return (int)((int64_t)p * (I - extra) / s);
}

// Cost model of the tail, in thousandths of a k-tile iteration of a full
// wave (~1.5 us on MI355X), fitted to per-workgroup timelines of version 9
// and to version 7 tails (s_memrealtime stamps):
//  * a k-iteration takes u(b) = 0.63 + 0.30 b, b = the fraction of CUs busy:
//    the part is power-limited, so a part-empty wave clocks higher (one CU in
//    sixteen busy: ~1.0 us per iteration; all: ~1.5 us);
//  * a split tile's hand-off adds ~6 iterations for two pieces (~10 us: the
//    first pieces write their 256 KB partials, the last reads them back, 8
//    loads per lane in flight) and ~2 more per further piece (the slowest
//    hand-off measured 9.6, 13.4, 19 and 17-22 us for 2, 4, 7 and 8 pieces).
__host__ __device__ inline int64_t sk_iter_cost(int64_t busy, int64_t C) { return 630 + 300 * busy / C; }

__host__ __device__ inline int64_t sk_whole_cost(int64_t r, int64_t I, int64_t C) { return sk_iter_cost(r, C) * I; }

__host__ __device__ inline int64_t sk_split_cost(int64_t r, int64_t I, int64_t C, int64_t s) {
  const int64_t last = (I - kSkLastExtra + s - 1) / s + kSkLastExtra;  // the longest piece
  return sk_iter_cost(s * r, C) * last + 1000 * (6 + 2 * (s - 2));
}

// The schedule for T tiles of I iterations on C compute units: the cheapest
// s in [2, kSkMaxPieces] with s * r <= C and I / s >= kSkMinIters, used when
// its modelled cost is at most 4/5 of the whole-tile tail's.
__host__ __device__ inline SkPlan sk_plan(int64_t T, int64_t I, int num_cus) {
  const SkPlan whole{(int)T, 0, 1, 1};
  const int64_t C = num_cus < kSkMaxUnits ? num_cus : kSkMaxUnits;
  if (C <= 0 || T % C == 0) return whole;
  const int64_t dp = T / C * C, r = T - dp;
  const int chunks = (T % 8 == 0) ? 8 : 1;  // as xcd_remap
  if (chunks == 8 && dp % 8 != 0) return whole;
  int64_t best = 0, best_cost = 0;
  for (int64_t s = 2; s <= kSkMaxPieces && s * r <= C && I / s >= kSkMinIters; s++) {
    const int64_t c = sk_split_cost(r, I, C, s);
    if (best == 0 || c < best_cost) {
      best = s;
      best_cost = c;
    }
  }
  if (best == 0 || 5 * best_cost > 4 * sk_whole_cost(r, I, C)) return whole;
  return SkPlan{(int)dp, (int)(best * r), (int)best, chunks};
}

// Version 11 (128x128 tiles) splits whole grids that fill at most half of the
// CUs: T tiles of I k-tiles on C CUs with 2T <= C, every tile cut into
// s = min(8, C / T, I / 8) pieces (no whole tiles: dp = 0), the last piece
// kFillLastExtra k-tiles longer.  With T % 8 == 0 each XCD takes the pieces
// of its own share of the raster.  A piece of fewer than 8 k-tiles (~1 us
// each) does not repay the hand-off, measured on MI355X at 3-6 us (a piece's
// partial published in 1.4-3.2 us, the last arrival's reads 1.2-4.5 us):
// 1000^3 (8 k-tiles) took 12.8 us in 2 pieces against 9.8 whole.
constexpr int kFillMinIters = 8;
constexpr int kFillMaxPieces = 8;
constexpr int kFillLastExtra = 1;
// min_iters: the fewest k-tiles per piece (the fp32 kernel's k-tiles take
// ~1.7 us each, so it splits down to 2).
__host__ __device__ inline SkPlan sk_plan_fill(int64_t T, int64_t I, int num_cus, int min_iters = kFillMinIters) {
  const SkPlan whole{(int)T, 0, 1, 1};
  const int64_t C = num_cus < kSkMaxUnits ? num_cus : kSkMaxUnits;
  if (C <= 0 || T <= 0 || 2 * T > C || min_iters < 1) return whole;
  int64_t s = C / T;
  if (s > kFillMaxPieces) s = kFillMaxPieces;
  if (s > I / min_iters) s = I / min_iters;
  if (s < 2) return whole;
  return SkPlan{0, (int)(s * T), (int)s, T % 8 == 0 ? 8 : 1};
}

// The work of one workgroup: k-tile iterations [kb, ke) of the tile at raster
// position cid, which is piece p of np.  For a split tile, `tile` numbers it
// among the tail tiles (for its counters) and the pieces of tile t are the
// units unit_of(t, 0 .. np-1).
struct SkWork {
  int cid;
  int kb, ke;
  int np, p;
  int tile;  // tail tile index (split tiles only)
};

// Workgroup of piece q of tail tile `tile` (x = tile / rc is its chunk).
__host__ __device__ inline int sk_unit_of(const SkPlan& pl, int T, int tile, int q) {
  const int rc = (T - pl.dp) / pl.chunks;
  const int x = tile / rc, sl = tile - x * rc;
  return x + pl.chunks * (sl * pl.pieces + q);
}

__host__ __device__ inline SkWork sk_work(int bid, int T, int I, const SkPlan& pl, int extra = kSkLastExtra) {
  SkWork w{};
  if (bid < pl.dp) {
    // whole tiles: raster positions [0, dp) (with 8 chunks: the first dp / 8
    // of each XCD's share of [0, T))
    w.cid = xcd_remap(bid, pl.chunks == 8 ? T : pl.dp);
    w.kb = 0;
    w.ke = I;
    w.np = 1;
    w.p = 0;
    w.tile = 0;
    return w;
  }
  const int u = bid - pl.dp;
  const int rc = (T - pl.dp) / pl.chunks;
  const int x = u % pl.chunks, lu = u / pl.chunks;
  const int sl = lu / pl.pieces;
  w.p = lu - sl * pl.pieces;
  w.np = pl.pieces;
  w.tile = x * rc + sl;
  w.cid = (pl.chunks == 8 ? x * (T >> 3) + (pl.dp >> 3) : pl.dp) + sl;
  w.kb = sk_piece_begin(w.p, I, pl.pieces, extra);
  w.ke = w.p + 1 < pl.pieces ? sk_piece_begin(w.p + 1, I, pl.pieces, extra) : I;
  return w;
}

// Counter words (all zero between calls): kSkWaves per tail tile.
constexpr size_t kSkCounterBytes = (size_t)kSkMaxUnits * kSkWaves * sizeof(unsigned);

}  // namespace vk
