// Order in which the workgroups of one XCD take the work items of its share.
// Plain constexpr integer code: the device compiler treats it as host and
// device code, and the CPU tests compile it with g++.
#pragma once

namespace gk {

// The j-th item (0 <= j < cnt) of an XCD whose share is the items
// [lo, lo + cnt) of a launch ordered (kv head, sequence, row tile), row tiles
// fastest, `tiles` row tiles per sequence. The share is taken by row tile,
// highest first, and within one row tile in ascending item order. In a
// causal chunk a higher row tile sees more keys, and a workgroup that starts
// later takes the XCD's first CU to fall free, so the light tiles fill in
// behind the heavy ones (longest processing time first): with two rounds of
// workgroups per CU the heaviest tile is paired with the lightest instead of
// with another heavy one.
constexpr int heavy_first_item(int lo, int cnt, int tiles, int j) {
  // u = tiles - 1 - tile ranks the tiles heaviest first. Tile t occurs `full`
  // times in the share, once more when (t - lo) mod tiles < rem: for u in
  // [a0, b0) and in [a1, tiles).
  const long long n = tiles, full = cnt / tiles, rem = cnt % tiles, r0 = lo % tiles;
  const long long b0 = n - r0;
  const long long a0 = b0 - rem > 0 ? b0 - rem : 0;
  const long long a1 = 2 * n - r0 - rem > b0 ? 2 * n - r0 - rem : b0;
  // Items of the share whose rank is below u.
  auto below = [&](long long u) {
    long long e0 = u - a0, e1 = u - a1;
    e0 = e0 < 0 ? 0 : (e0 > b0 - a0 ? b0 - a0 : e0);
    e1 = e1 < 0 ? 0 : e1;
    return full * u + e0 + e1;
  };
  // Largest rank u with below(u) <= j; its tile holds item j.
  long long lo_u = 0, hi_u = n - 1;
  while (lo_u < hi_u) {
    const long long mid = (lo_u + hi_u + 1) / 2;
    if (below(mid) <= j) lo_u = mid;
    else hi_u = mid - 1;
  }
  const long long tile = n - 1 - lo_u, k = j - below(lo_u);
  return (int)(lo + (tile - r0 + n) % n + k * n);
}

}  // namespace gk
