// CPU check of gk::heavy_first_item (gaudirt_amd/csrc/work_order.hpp), the
// prefill kernel's order of work items inside one XCD's share. For every
// share of many launch shapes it checks what the order must be: a
// permutation of the share, row tiles non-increasing, ascending items within
// one row tile. Prints OK on success.
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

}  // namespace

int main() {
  check_fast_div();
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
