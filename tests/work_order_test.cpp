// CPU checks of gaudirt_amd/csrc/work_order.hpp: gk::heavy_first_item, the
// prefill kernel's order of work items inside one XCD's share (for every
// share of many launch shapes: a permutation of the share, row tiles
// non-increasing, ascending items within one row tile); gk::fast_div; the
// balanced decode schedule's tile counts, 2^31 gate and split with per-unit
// fixed cost (gk::stream_start). Prints OK on success.
#include <algorithm>
#include <cstdio>
#include <vector>

#include "work_order.hpp"

namespace {

int failures = 0;

void check_share(int lo, int cnt, int tiles) {
  std::vector<char> seen(cnt, 0);
  int prev_tile = tiles, prev_item = -1;
  for (int j = 0; j < cnt; ++j) {
    const int item = gk::heavy_first_item(lo, cnt, tiles, j);
    const gk::DivMagic magic = gk::div_magic(uint32_t(tiles));
    if (gk::heavy_first_item(lo, cnt, tiles, j, [magic](int x) { return int(gk::fast_div(uint32_t(x), magic)); }) !=
        item) {
      if (failures++ < 10) std::printf("lo=%d cnt=%d tiles=%d j=%d: the fast_div form differs\n", lo, cnt, tiles, j);
      return;
    }
    if (item < lo || item >= lo + cnt || seen[item - lo]) {
      if (failures++ < 10) std::printf("lo=%d cnt=%d tiles=%d j=%d: item %d out of share or repeated\n", lo, cnt, tiles, j, item);
      return;
    }
    seen[item - lo] = 1;
    const int tile = item % tiles;
    if (tile > prev_tile || (tile == prev_tile && item <= prev_item)) {
      if (failures++ < 10) std::printf("lo=%d cnt=%d tiles=%d j=%d: item %d (tile %d) after item %d (tile %d)\n", lo,
                                       cnt, tiles, j, item, tile, prev_item, prev_tile);
      return;
    }
    prev_tile = tile;
    prev_item = item;
  }
}

// The shares of a launch of `items` workgroups over 8 XCDs, as the kernel cuts them.
void check_launch(int items, int tiles) {
  const int per = items / 8, extra = items % 8;
  for (int x = 0; x < 8; ++x) {
    const int lo = x * per + (x < extra ? x : extra), cnt = per + (x < extra ? 1 : 0);
    if (cnt > 0) check_share(lo, cnt, tiles);
  }
}

// gk::fast_div against the division it replaces: every divisor up to 4096 and
// divisors around each power of two, with the dividends where an error would
// show first (multiples of d and their neighbours, the top of the range) and
// pseudo-random ones.
void check_fast_div() {
  std::vector<uint32_t> divisors;
  for (uint32_t d = 1; d <= 4096; ++d) divisors.push_back(d);
  for (int b = 12; b <= 31; ++b)
    for (int64_t k = -3; k <= 3; ++k) {
      const int64_t d = (int64_t(1) << b) + k;
      if (d >= 1 && d <= (int64_t(1) << 31)) divisors.push_back(uint32_t(d));
    }
  uint64_t state = 0x9e3779b97f4a7c15ull;
  auto next = [&]() {
    state ^= state << 13, state ^= state >> 7, state ^= state << 17;
    return uint32_t(state) & 0x7fffffffu;
  };
  for (uint32_t d : divisors) {
    const gk::DivMagic m = gk::div_magic(d);
    std::vector<uint32_t> xs = {0u, 1u, d - 1, d, d + 1, 0x7fffffffu, 0x7ffffffeu};
    const uint32_t top = 0x7fffffffu / d;
    for (uint32_t q : {1u, 2u, 3u, top / 2, top - 1, top})
      if (q >= 1 && uint64_t(q) * d <= 0x7fffffffu) {
        xs.push_back(q * d - 1);
        xs.push_back(q * d);
        if (uint64_t(q) * d + 1 <= 0x7fffffffu) xs.push_back(q * d + 1);
      }
    for (int i = 0; i < 64; ++i) xs.push_back(next());
    for (uint32_t x : xs)
      if (x <= 0x7fffffffu && gk::fast_div(x, m) != x / d) {
        if (failures++ < 10) std::printf("fast_div(%u, d=%u) = %u, want %u\n", x, d, gk::fast_div(x, m), x / d);
        return;
      }
  }
}

// The balanced decode schedule's tile count per row against a brute-force
// count of the tiles holding visible keys, and the host gate
// (stream_tiles_fit) against the kernel's own overflow test: whenever the
// gate passes, a batch of rows at max_context, under any window, numbers its
// tiles with total + wgs below 2^31.
void check_stream_gate() {
  for (int ts : {16, 32}) {
    for (int window : {0, 1, 2, 15, 16, 17, 31, 32, 33, 100, 513, 4096}) {
      for (int ctx = 0; ctx <= 1200; ++ctx) {
        const int left = gk::visible_left(ctx, window);
        int brute = 0;
        for (int tile = 0; tile * ts < ctx; ++tile)
          if ((tile + 1) * ts > left) ++brute;
        if (brute == 0) brute = 1;  // an empty row owns one masked tile
        const int count = gk::stream_row_tile_count(ctx, window, ts);
        if (count != brute || count > ctx / ts + 2) {
          if (failures++ < 10)
            std::printf("ts=%d window=%d ctx=%d: count %d, brute force %d\n", ts, window, ctx, count, brute);
          return;
        }
      }
    }
  }
  const int64_t limit = int64_t(1) << 31;
  for (int ts : {16, 32}) {
    for (int64_t wgs : {int64_t(1), int64_t(256), int64_t(1024), int64_t(4096)}) {
      for (int64_t units : {int64_t(1), int64_t(7), int64_t(1023), int64_t(65535), int64_t(65535) * 8 * 4}) {
        // The largest per-row position bound n = max_context / ts + 2 + cost the gate admits.
        const int64_t n_max = (gk::stream_position_limit(wgs) - 1) / units;
        const int64_t fixed = 2 + gk::kStreamUnitCost;  // n = max_context / ts + fixed
        if (n_max < fixed) continue;
        const int64_t mc_fit = (n_max - fixed) * ts + ts - 1, mc_over = (n_max - fixed + 1) * ts;
        if (!gk::stream_tiles_fit(units, mc_fit, ts, wgs) || gk::stream_tiles_fit(units, mc_over, ts, wgs)) {
          if (failures++ < 10)
            std::printf("ts=%d wgs=%lld units=%lld: gate boundary not at max_context %lld / %lld\n", ts,
                        (long long)wgs, (long long)units, (long long)mc_fit, (long long)mc_over);
          return;
        }
        if (mc_fit > 0x7fffffff) continue;  // row_context is int32
        // Every row at mc_fit under the windows that maximise its tiles.
        for (int window : {0, ts - 1, ts + 1, 2 * ts - 1, (int)std::min<int64_t>(mc_fit, 0x7fffffff)}) {
          const int64_t total = units * (gk::stream_row_tile_count((int)mc_fit, window, ts) + gk::kStreamUnitCost);
          // The kernel's own test, and room for its cursor's last step past the end.
          if (total >= gk::stream_position_limit(wgs) || total + wgs + gk::kStreamUnitCost >= limit) {
            if (failures++ < 10)
              std::printf("ts=%d wgs=%lld units=%lld window=%d: gate passed but total %lld reaches the limit\n", ts,
                          (long long)wgs, (long long)units, window, (long long)total);
            return;
          }
        }
      }
    }
  }
  // Degenerate inputs never pass.
  if (gk::stream_tiles_fit(-1, 100, 32, 1024) || gk::stream_tiles_fit(1, -1, 32, 1024) ||
      gk::stream_tiles_fit(1, 100, 32, 0)) {
    if (failures++ < 10) std::printf("stream_tiles_fit accepted a negative or empty size\n");
  }
}

// The balanced decode schedule as the kernel walks it: rows of `units_per_row`
// units with tiles[row] tiles each, every unit preceded by `cost` positions of
// fixed cost, the numbering split over `wgs` workgroups. Checks that every
// tile of every unit is visited exactly once and in order, that a workgroup
// starting inside a unit's cost starts at its first tile, and that the
// partial slots the workgroups write for a split unit are the ones the merge
// reads for it (first part 2 wf + (g0 == wf per ? 0 : 1), then 2 w for each
// later workgroup w, wf = g0 / per, g0 the position of the unit's first tile).
void check_stream_schedule(const std::vector<int>& tiles, int units_per_row, int wgs, int cost) {
  const int rows = (int)tiles.size(), U = units_per_row, units = rows * U;
  std::vector<int64_t> start(units + 1, 0);  // position of each unit's cost
  for (int u = 0; u < units; ++u) start[u + 1] = start[u] + tiles[u / U] + cost;
  const int64_t total = start[units];
  const int64_t per = (total + wgs - 1) / wgs;
  std::vector<int> visited(units, 0), first_wg(units, -1), last_wg(units, -1);
  std::vector<std::vector<int>> slots(units);
  auto fail = [&](const char* what, int w, int u) {
    if (failures++ < 10)
      std::printf("schedule rows=%d U=%d wgs=%d cost=%d: %s (workgroup %d, unit %d)\n", rows, U, wgs, cost, what, w, u);
  };
  for (int w = 0; w < wgs; ++w) {
    const int64_t g_begin = w * per, g_end = std::min(g_begin + per, total);
    if (g_begin >= g_end) continue;
    int row = 0;
    while ((int64_t)(row + 1) * U <= units && start[(row + 1) * U] <= g_begin) ++row;
    const gk::StreamStart st =
        gk::stream_start(uint32_t(g_begin - start[row * U]), uint32_t(tiles[row] + cost), cost);
    int h = st.h, j = st.j;
    int64_t g = g_begin + st.skip;
    if (st.h >= U || (st.skip > 0 && st.j != 0)) return fail("start outside the row", w, row * U);
    while (g < g_end) {
      const int u = row * U + h, count = tiles[row];
      if (g != start[u] + cost + j) return fail("position does not match the tile", w, u);
      if (visited[u] != j) return fail("tile visited out of order or twice", w, u);
      ++visited[u];
      if (j == 0) first_wg[u] = w;
      if (j == count - 1) last_wg[u] = w;
      const bool seg_end = j == count - 1 || g == g_end - 1;
      if (seg_end) {
        const int64_t g0 = g - j;
        const bool whole = g0 >= g_begin && g0 + count <= g_end;
        if (!whole) slots[u].push_back(2 * w + (g0 <= g_begin ? 0 : 1));
      }
      ++g;
      if (++j == count) {
        j = 0;
        g += cost;
        if (++h == U) h = 0, ++row;
        if (row >= rows) break;
      }
    }
  }
  for (int u = 0; u < units; ++u) {
    if (visited[u] != tiles[u / U]) return fail("unit not fully visited", -1, u);
    const int64_t g0 = start[u] + cost;
    const int wf = (int)(g0 / per);
    if (first_wg[u] != wf) return fail("first tile not in workgroup g0 / per", first_wg[u], u);
    if (first_wg[u] == last_wg[u]) {
      if (!slots[u].empty()) return fail("whole unit left a partial", first_wg[u], u);
      continue;
    }
    const int first_slot = 2 * wf + (g0 == wf * per ? 0 : 1);
    const int nparts = last_wg[u] - wf + 1;
    if ((int)slots[u].size() != nparts) return fail("partial count differs from the span", wf, u);
    for (int k = 0; k < nparts; ++k)
      if (slots[u][k] != (k == 0 ? first_slot : 2 * (wf + k))) return fail("partial slot differs from the merge's", wf + k, u);
  }
}

void check_stream_schedules() {
  uint64_t state = 0x243f6a8885a308d3ull;
  auto next = [&](int n) {
    state ^= state << 13, state ^= state >> 7, state ^= state << 17;
    return int(state % uint64_t(n));
  };
  for (int cost = 0; cost <= 3; ++cost) {
    for (int trial = 0; trial < 400; ++trial) {
      const int rows = 1 + next(40), U = 1 + next(8), wgs = 1 + next(96);
      std::vector<int> tiles(rows);
      for (int& t : tiles) t = 1 + (next(4) == 0 ? next(200) : next(6));
      check_stream_schedule(tiles, U, wgs, cost);
    }
    // C2-, C3- and C5-like shapes at 1024 workgroups.
    for (int shape = 0; shape < 3; ++shape) {
      const int rows = shape == 0 ? 64 : shape == 1 ? 256 : 32;
      std::vector<int> tiles(rows);
      for (int& t : tiles) t = shape == 0 ? 16 + next(113) : shape == 1 ? 4 + next(61) : 32 + next(993);
      check_stream_schedule(tiles, 8, 1024, cost);
    }
  }
}

}  // namespace

int main() {
  check_fast_div();
  check_stream_gate();
  check_stream_schedules();
  // C4: 8 sequences x 8 kv heads x 8 row tiles.
  check_launch(512, 8);
  // Every small shape, every alignment of a share against the row tiles.
  for (int tiles = 1; tiles <= 40; ++tiles)
    for (int lo = 0; lo < 2 * tiles + 3; ++lo)
      for (int cnt = 1; cnt <= 3 * tiles + 5; ++cnt) check_share(lo, cnt, tiles);
  for (int tiles = 1; tiles <= 64; ++tiles)
    for (int groups = 1; groups <= 40; ++groups) check_launch(tiles * groups, tiles);
  // Long chunks: many row tiles, shares cut across sequences.
  check_launch(1024 * 7 * 3, 1024);
  check_share(123457, 98765, 4099);
  check_share((1 << 30) - 5000, 4999, 1 << 29);
  // The 2^30-item limit with row tiles as large as the launch (32-bit bounds; UBSan checks overflow).
  check_share(0, 5000, 1 << 30);
  check_share((1 << 30) - 3000, 3000, (1 << 30) - 1);
  check_share((1 << 30) - 4097, 4097, 4096);
  if (failures) {
    std::printf("%d failures\n", failures);
    return 1;
  }
  // The C4 order of XCD 0: tiles 7..0, eight sequences each.
  for (int j = 0; j < 64; ++j) {
    const int item = gk::heavy_first_item(0, 64, 8, j);
    if (item % 8 != 7 - j / 8 || item / 8 != j % 8) {
      std::printf("C4 share: j=%d item %d\n", j, item);
      return 1;
    }
  }
  std::printf("OK\n");
  return 0;
}
