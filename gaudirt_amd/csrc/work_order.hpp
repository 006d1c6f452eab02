// Order in which the workgroups of one XCD take the work items of its share.
// Plain constexpr integer code: the device compiler treats it as host and
// device code, and the CPU tests compile it with g++.
#pragma once

#include <cstdint>

namespace gk {

// Division by a runtime divisor 1 <= d <= 2^31 as a multiply and a shift, for
// dividends 0 <= x < 2^31: with s = ceil(log2 d), mul = floor(2^(31+s) / d) + 1
// (below 2^32) and shift = 31 + s, x / d == (x * mul) >> shift, because
// x * mul / 2^(31+s) exceeds x / d by less than 2^-s <= 1/d. The host computes
// the pair once per launch; a kernel then divides in two or three
// instructions instead of the ~25 of a general 32-bit division.
struct DivMagic {
  uint32_t mul, shift;
};

constexpr DivMagic div_magic(uint32_t d) {
  uint32_t s = 0;
  while (s < 32 && (uint64_t(1) << s) < d) ++s;
  return DivMagic{uint32_t((uint64_t(1) << (31 + s)) / d + 1), 31 + s};
}

constexpr uint32_t fast_div(uint32_t x, DivMagic m) { return uint32_t((uint64_t(x) * m.mul) >> m.shift); }


// The j-th item (0 <= j < cnt) of an XCD whose share is the items
// [lo, lo + cnt) of a launch ordered (kv head, sequence, row tile), row tiles
// fastest, `tiles` row tiles per sequence. The share is taken by row tile,
// highest first, and within one row tile in ascending item order. In a
// causal chunk a higher row tile sees more keys, and a workgroup that starts
// later takes the XCD's first CU to fall free, so the light tiles fill in
// behind the heavy ones (longest processing time first): with two rounds of
// workgroups per CU the heaviest tile is paired with the lightest instead of
// with another heavy one.
template <class DivTiles>
constexpr int heavy_first_item(int lo, int cnt, int tiles, int j, DivTiles div_tiles) {
  // u = tiles - 1 - tile ranks the tiles heaviest first. Tile t occurs `full`
  // times in the share, once more when (t - lo) mod tiles < rem: for u in
  // [a0, b0) and in [a1, tiles). 32-bit arithmetic (the kernel runs this on
  // the scalar unit, where 64-bit division costs hundreds of instructions):
  // with lo + cnt <= 2^30 every value stays below 2^31; a1 is capped at n,
  // which leaves below() unchanged for the ranks u < n it is asked about.
  const int n = tiles, full = div_tiles(cnt), rem = cnt - full * n, r0 = lo - div_tiles(lo) * n;
  const int b0 = n - r0;
  const int a0 = b0 - rem > 0 ? b0 - rem : 0;
  const int x = n - r0 - rem;  // a1 = max(x + n, b0), capped at n
  const int a1 = x >= 0 ? n : (x + n > b0 ? x + n : b0);
  // Items of the share whose rank is below u (at most cnt).
  auto below = [&](int u) {
    int e0 = u - a0, e1 = u - a1;
    e0 = e0 < 0 ? 0 : (e0 > b0 - a0 ? b0 - a0 : e0);
    e1 = e1 < 0 ? 0 : e1;
    return full * u + e0 + e1;
  };
  // Largest rank u with below(u) <= j; its tile holds item j.
  int lo_u = 0, hi_u = n - 1;
  while (lo_u < hi_u) {
    const int mid = (lo_u + hi_u + 1) / 2;
    if (below(mid) <= j) lo_u = mid;
    else hi_u = mid - 1;
  }
  const int tile = n - 1 - lo_u, k = j - below(lo_u);
  const int t = tile - r0 + n;  // in [1, 2n)
  return lo + (t >= n ? t - n : t) + k * n;
}

constexpr int heavy_first_item(int lo, int cnt, int tiles, int j) {
  return heavy_first_item(lo, cnt, tiles, j, [tiles](int x) { return x / tiles; });
}

// First visible key of a row of `ctx` keys under a sliding window (0 = none).
constexpr int visible_left(int ctx, int window) { return (window > 0 && ctx > window) ? ctx - window : 0; }

// Tiles of one row in the balanced decode schedule: tile k holds the keys
// [k ts, (k + 1) ts), and the row owns the tiles that hold its visible keys
// [visible_left(ctx, window), ctx); an empty row owns one fully masked tile.
// Without a window that is ceil(ctx / ts) <= ctx / ts + 1 tiles; a window can
// start mid-tile, which adds at most one: never above ctx / ts + 2.
constexpr int stream_row_tile_count(int ctx, int window, int ts) {
  const int c = ctx > 0 ? ctx : 0;
  return c > 0 ? (c + ts - 1) / ts - visible_left(c, window) / ts : 1;
}

// Fixed cost of a work unit in the balanced schedule, in tiles: a unit of n
// tiles takes n + kStreamUnitCost positions of the schedule's numbering (the
// cost first, then its tiles), so that a workgroup whose share crosses many
// short units (each one a finish with its stores, and a new query) is given
// fewer tiles. 0 numbers the tiles alone.
#ifndef GK_STREAM_UNIT_COST
#define GK_STREAM_UNIT_COST 2
#endif
constexpr int kStreamUnitCost = GK_STREAM_UNIT_COST;

// Where a workgroup starts whose share begins `off` positions into a row's
// units (`weight` = tiles + cost positions each): unit h, tile j, after
// passing over `skip` positions of that unit's cost.
struct StreamStart {
  int h, j, skip;
};
constexpr StreamStart stream_start(uint32_t off, uint32_t weight, int cost) {
  const int h = (int)(off / weight);
  const int jw = (int)(off - (uint32_t)h * weight);
  return jw < cost ? StreamStart{h, 0, cost - jw} : StreamStart{h, jw - cost, 0};
}

// The balanced schedule numbers the positions of a whole batch (units *
// (tiles + cost) of each row) in 32 bits, and its kernel splits them over
// `wgs` workgroups with (total + wgs - 1) / wgs, and a workgroup's cursor
// steps up to the cost past the last position: total + wgs + cost must stay
// below 2^31. With every row_context <= max_context a row has at most
// max_context / ts + 2 tiles, so the host runs the schedule only when this
// holds.
constexpr int64_t stream_position_limit(int64_t wgs) { return (int64_t(1) << 31) - wgs - kStreamUnitCost; }
constexpr bool stream_tiles_fit(int64_t units, int64_t max_context, int ts, int64_t wgs) {
  return units >= 0 && max_context >= 0 && wgs >= 1 &&
         units * (max_context / ts + 2 + kStreamUnitCost) < stream_position_limit(wgs);
}

}  // namespace gk
