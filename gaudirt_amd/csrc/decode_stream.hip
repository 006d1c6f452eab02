// Balanced paged decode for gfx950 ("stream" schedule).
//
// The grid holds exactly as many one-wave workgroups as the GPU keeps resident.
// All key tiles of the batch form one sequence: work units (row, kv head, head
// group) in row-major order, each unit's tiles in key order, each unit
// preceded by kStreamUnitCost positions that stand for its fixed cost (the
// finish of a unit: its stores, which hold up the next tile wait, and a new
// query). Workgroup w takes the contiguous range [w * per, (w + 1) * per) of
// those positions, so every workgroup streams about the same number of K/V
// bytes however skewed the context lengths are, a few tiles fewer for each
// unit it crosses, and its two-stage LDS pipeline runs without a break from
// its first tile to its last: crossing into the next unit only swaps the
// query (prefetched into LDS with that unit's first tile) and the softmax
// state.
//
// A unit whose tiles all fall in one workgroup is finalised there (bf16
// output). A unit that spans workgroups w_first .. w_last leaves one partial
// (unnormalised fp32 output, max and sum in log2 units) per workgroup, and the
// merge kernel combines them with the log-sum-exp rule. Each workgroup has at
// most two partial units (the one it starts in and the one it ends in), so the
// partials live in 2 * wgs fixed slots: slot 2w for the segment that begins at
// the workgroup's first tile, 2w + 1 for one that begins later.
//
// Tiles are TS-key ranges at absolute key positions (tile k = keys [k TS,
// (k + 1) TS)), so with block_size >= TS every tile lies in one pool block and
// needs one block-table entry, fetched with a scalar load one tile ahead;
// shorter blocks take one entry per 16-byte load or, below one load's keys,
// one per key (the MODE template argument). Keys outside a row's visible
// range [left, ctx) are masked. Inside a unit the
// tiles are visited rotated by kv_head * count / kv_heads: the kv heads of a
// row then stream different blocks at any moment, instead of the same block
// offset in regions a power-of-two apart, which concentrates the reads on a
// subset of the HBM channels.
//
// The per-tile arithmetic is the partitioned MFMA kernel's (paged_decode.hip):
// S^T = K . Q^T with v_mfma_f32_16x16x32_bf16, online softmax, P rounded
// to bf16, P . V from a transposed LDS read, both tiles loaded HBM -> LDS with
// 16-byte buffer loads (global_load_lds_dwordx4).
#include "decode_common.hpp"
#include "work_order.hpp"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace gk {
namespace {

typedef __attribute__((address_space(3))) char lds_char_t;
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));


struct StreamArgs {
  DecodeArgs d;
  int32_t units_per_row;  // kv_heads * head_groups
  int32_t wgs;            // workgroups of the grid
  DivMagic wgs_div, head_groups_div, kv_heads_div;  // division by wgs, head_groups, kv_heads (work_order.hpp)
  float* unit_span;       // per unit: {first partial slot, last workgroup} as int32 bits
};

// A row's tiles: visible keys [left, ctx) occupy tiles first .. first + count - 1.
// An empty row still owns one (fully masked) tile, so every unit is finalised.
struct RowTiles {
  int first, count, left, ctx;
};

template <int TS>
__device__ __forceinline__ RowTiles row_tiles(int ctx, int window) {
  RowTiles r;
  r.ctx = ctx > 0 ? ctx : 0;
  r.left = visible_left(r.ctx, window);
  r.first = r.left / TS;
  r.count = stream_row_tile_count(r.ctx, window, TS);
  return r;
}


// Inclusive prefix sum over the wave's 64 lanes with DPP lane shifts (no LDS
// round trips): row_shr 1, 2, 4, 8 scan each 16-lane row (a source outside
// the row reads 0), then row_bcast:15 adds row 0's total into row 1 and row
// 2's into row 3, and row_bcast:31 adds the total of rows 0-1 into rows 2-3.
__device__ __forceinline__ int wave_inclusive_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);   // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);   // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1 and 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2 and 3
  return x;
}

__device__ __forceinline__ int wave_sum(int x) { return __builtin_amdgcn_readlane(wave_inclusive_scan(x), 63); }

// Position in the tile sequence, with the row data it needs (wave-uniform).
struct Cursor {
  int row, h, j;            // unit (row, h = kv head * head_groups + head group), tile j of the unit
  int kvh, rot;             // the unit's kv head; rotation of its tile order
  RowTiles rt;
  int req, qrow;            // block-table row, query/output row
  int g;                    // index in the tile sequence (below 2^31: the host routes larger batches elsewhere)
  int next_ctx, next_req, next_qrow;  // row + 1, fetched ahead
};

// What consuming one tile needs (wave-uniform). The tile's keys fall into NR
// runs of TS / NR keys, each inside one pool block: one run when blocks hold
// at least TS keys, one run per 16-byte load of the tile when they hold at
// least one load's keys (kKeyBlocks keeps no runs here: its per-key entries go
// straight to the loads).
template <int NR>
struct TileDesc {
  int tb;                   // first key of the tile
  int left, ctx;            // visible keys of the row
  int row, h, j, qrow;      // the unit (its kv head is h / head_groups) and the tile's place in it
  int g;
  uint32_t row0[NR];        // byte offset of run i's first key in its kv head's K (and V) region
  int flags;                // kTileFirst / kTileLast: first / last tile of the unit in this
                            // workgroup; kUnitLast: the unit's last tile
};
constexpr int kTileFirst = 1, kTileLast = 2, kUnitLast = 4;

// Block-table entries of one tile's runs.
template <int NR>
struct TileEntries {
  int e[NR];
  int keyed;  // per-key entries packed into one VGPR, lane k = key k (kKeyBlocks)
};

// How a tile's slots are found (the MODE template argument):
//  kTileBlocks  blocks of >= TS keys: one block-table entry per tile;
//  kLoadBlocks  blocks of >= 64 / CPR keys (one 16-byte load per lane): one
//               entry per load instruction;
//  kKeyBlocks   shorter blocks, down to the token-granular map (block 1): one
//               entry per key, each lane picking its key's among the load's.
// All entries are scalar loads issued one tile ahead.
constexpr int kTileBlocks = 0, kLoadBlocks = 1, kKeyBlocks = 2;

// Per-tile arithmetic (the ARITH template argument):
//  kArithMfma  S^T = K . Q^T and P . V on 16 x 16 MFMA tiles whose 16 columns
//              are a unit's query heads (every GQA group; 1-3 heads leave
//              padding columns);
//  kArithDot   groups of 1-3 heads, head_dim 64/128: wave-level v_dot2_f32_bf16
//              with fp32 accumulation. Q.K: each lane holds one key of the
//              tile and half of its dims (lanes l and l + 32 the two halves),
//              the halves added across the 32-lane swap. P.V: each lane owns
//              D / 64 output dims and reads them for four keys at a time with
//              the transposed LDS read; the probabilities of two keys at a
//              time reach every lane as one scalar (a packed bf16 pair).
// The shipping build runs the MFMA form at every group: under the balanced
// schedule the dot form measured slower at groups 1, 2 and 3 (same box, C2's
// batch at 8 / 16 / 24 query heads: 102.0 / 102.5 / 102.9 us against 107.9 /
// 113.0 / 120.0 us). GK_STREAM_DOT=1 builds the dot form for units of 1-3
// heads (head_dim 64/128).
#ifndef GK_STREAM_DOT
#define GK_STREAM_DOT 0
#endif
constexpr int kArithMfma = 0, kArithDot = 1;
constexpr int kDotMaxHeads = 3;

template <int D, bool SOFTCAP, int MODE, int ARITH>
__device__ __forceinline__ void decode_stream_body(StreamArgs sa) {
  using S = MfmaShape<D>;
  constexpr int TS = S::TS;
  constexpr bool DOT = ARITH == kArithDot;
  static_assert(!DOT || TS == 32, "the dot form pairs each key with two lanes (head_dim 64/128)");
  constexpr int DNC = D / 16;  // dot form: 16-byte chunks of a key row per lane (half the row)
  constexpr int DOD = D / 64;  // dot form: output dims per lane
  constexpr int NR = MODE == kTileBlocks ? 1 : MODE == kLoadBlocks ? S::LOADS : TS;  // key runs of a tile
  constexpr int KPR = TS / NR;  // keys of one run
  [[maybe_unused]] constexpr int KPL = 64 / S::CPR;  // keys of one load instruction
  // kKeyBlocks hands its per-key entries straight from the prefetch to the
  // loads (a descriptor holding TS offsets would live in scratch memory).
  using TileDesc = gk::TileDesc<MODE == kKeyBlocks ? 1 : NR>;
  constexpr int QBYTES = 16 * D * 2;  // one unit's query heads (up to 16)
  // Two K/V stages, each tile its own LDS object so that the compiler tells
  // reads of one from the direct loads in flight into another, and the two
  // query buffers (one object: a query read waits for the newest query load,
  // which is never younger than the tile it comes with).
  __shared__ __attribute__((aligned(16))) char kt0[S::TILE];
  __shared__ __attribute__((aligned(16))) char vt0[S::TILE];
  __shared__ __attribute__((aligned(16))) char kt1[S::TILE];
  __shared__ __attribute__((aligned(16))) char vt1[S::TILE];
  __shared__ __attribute__((aligned(16))) char qs[2][QBYTES];

  const DecodeArgs& a = sa.d;
  const int lane = threadIdx.x;
  const int q = lane >> 4, c16 = lane & 15;
  const int U = sa.units_per_row;
  const int w = blockIdx.x;

  // ---- Schedule ---------------------------------------------------------
  // Row window: lane l holds row wb + l's context, block-table row and output row.
  int wb = 0, wctx = 0, wreq = 0, wmap = 0;
  auto load_window = [&](int base) {
    wb = base;
    const int r = base + lane;
    wctx = 0;
    wreq = r;
    wmap = r;
    if (r < a.rows) {
      wctx = a.row_context[r];
      if (a.row_request) wreq = a.row_request[r];
      if (a.row_map) wmap = a.row_map[r];
    }
  };
  // The contexts of the first kPre windows are loaded together (one memory
  // round trip, not one per window); rows beyond them are read per window.
  constexpr int kPre = 8;
  int pctx[kPre];
#pragma unroll
  for (int k = 0; k < kPre; ++k) {
    const int r = 64 * k + lane;
    pctx[k] = r < a.rows ? a.row_context[r] : 0;
  }
  load_window(0);
  int lane_tiles = 0;
#pragma unroll
  for (int k = 0; k < kPre; ++k)
    if (64 * k + lane < a.rows) lane_tiles += row_tiles<TS>(pctx[k], a.window).count + kStreamUnitCost;
  int64_t total = wave_sum(lane_tiles);
  for (int base = 64 * kPre; base < a.rows; base += 64) {
    const int r = base + lane;
    total += wave_sum(r < a.rows ? row_tiles<TS>(a.row_context[r], a.window).count + kStreamUnitCost : 0);
  }
  total *= U;
  // The positions are numbered in 32 bits from here on (fewer scalar
  // registers in the tile loop): the host sends only batches whose positions,
  // with row_context <= max_context, stay below the limit (stream_tiles_fit). A
  // caller whose row_context exceeds its max_context can still get here; then
  // every output row becomes NaN and every span record is marked unwritten,
  // so the merge leaves those rows alone instead of combining stale partials.
  if (total >= stream_position_limit(sa.wgs)) {
    for (int r = w; r < a.rows; r += sa.wgs) {
      const int orow = a.row_map ? a.row_map[r] : r;
      uint16_t* dst = a.out + (int64_t)orow * a.out_stride;
      for (int e = lane; e < a.q_heads * D; e += 64) dst[e] = 0x7fc0;
      for (int u = lane; u < U; u += 64) {
        sa.unit_span[((int64_t)r * U + u) * 2] = __int_as_float(-1);
        sa.unit_span[((int64_t)r * U + u) * 2 + 1] = __int_as_float(-1);
      }
    }
    return;
  }
  const int per = (int)fast_div((uint32_t)(total + sa.wgs - 1), sa.wgs_div);
  const int g_begin = w * per;
  const int g_end = min(g_begin + per, (int)total);
  if (g_begin >= g_end) return;

  // The row holding position g_begin, and the position of its first unit.
  int row = 0;
  int row_base = 0;
  int pre = 0;
  bool found = false;
#pragma unroll
  for (int k = 0; k < kPre; ++k) {
    if (found || 64 * k >= a.rows) continue;
    const int r = 64 * k + lane;
    const int n = r < a.rows ? row_tiles<TS>(pctx[k], a.window).count + kStreamUnitCost : 0;
    const int incl = wave_inclusive_scan(n);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(r < a.rows && (pre + incl) * U > g_begin);
    if (hit) {
      const int f = __builtin_ctzll(hit);
      row = 64 * k + f;
      row_base = (pre + __builtin_amdgcn_readlane(incl - n, f)) * U;
      found = true;
    } else {
      pre += __builtin_amdgcn_readlane(incl, 63);
    }
  }
  for (int base = 64 * kPre; !found && base < a.rows; base += 64) {
    load_window(base);
    const int r = base + lane;
    const int n = r < a.rows ? row_tiles<TS>(wctx, a.window).count + kStreamUnitCost : 0;
    const int incl = wave_inclusive_scan(n);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(r < a.rows && (pre + incl) * U > g_begin);
    if (hit) {
      const int f = __builtin_ctzll(hit);
      row = base + f;
      row_base = (pre + __builtin_amdgcn_readlane(incl - n, f)) * U;
      found = true;
    } else {
      pre += __builtin_amdgcn_readlane(incl, 63);
    }
  }
  if (!found) return;  // unreachable: g_begin < total
  if ((row & ~63) != wb) load_window(row & ~63);

  // A new unit's kv head and the rotation of its tile order.
  auto enter_unit = [&](Cursor& c) {
    c.kvh = (int)fast_div((uint32_t)c.h, sa.head_groups_div);
    const int64_t spread = (int64_t)c.kvh * c.rt.count;
    c.rot = spread < (int64_t(1) << 31) ? (int)fast_div((uint32_t)spread, sa.kv_heads_div)
                                         : (int)(spread / a.kv_heads);
  };
  Cursor cur;
  {
    const int l = row - wb;
    cur.row = row;
    cur.rt = row_tiles<TS>(__builtin_amdgcn_readlane(wctx, l), a.window);
    cur.req = __builtin_amdgcn_readlane(wreq, l);
    cur.qrow = __builtin_amdgcn_readlane(wmap, l);
    // A share that starts inside a unit's fixed cost starts at its first tile.
    const StreamStart st = stream_start((uint32_t)(g_begin - row_base), (uint32_t)(cur.rt.count + kStreamUnitCost),
                                        kStreamUnitCost);
    cur.h = st.h;
    cur.j = st.j;
    cur.g = g_begin + st.skip;
    enter_unit(cur);
    cur.next_ctx = cur.next_req = cur.next_qrow = 0;
    if (row + 1 < a.rows) {
      cur.next_ctx = scalar_load(a.row_context, row + 1);
      cur.next_req = a.row_request ? scalar_load(a.row_request, row + 1) : row + 1;
      cur.next_qrow = a.row_map ? scalar_load(a.row_map, row + 1) : row + 1;
    }
  }
  if (cur.g >= g_end) return;  // the share holds only a unit's fixed cost
  auto advance = [&](Cursor& c) {
    ++c.g;
    if (++c.j < c.rt.count) return;
    c.j = 0;
    c.g += kStreamUnitCost;
    if (++c.h < U) {
      enter_unit(c);
      return;
    }
    c.h = 0;
    ++c.row;
    c.rt = row_tiles<TS>(c.next_ctx, a.window);
    c.req = c.next_req;
    c.qrow = c.next_qrow;
    if (c.row + 1 < a.rows) {
      c.next_ctx = scalar_load(a.row_context, c.row + 1);
      c.next_req = a.row_request ? scalar_load(a.row_request, c.row + 1) : c.row + 1;
      c.next_qrow = a.row_map ? scalar_load(a.row_map, c.row + 1) : c.row + 1;
    }
    enter_unit(c);
  };
  const int shift = a.block_shift;
  const int block_mask = (1 << shift) - 1;
  // First key of the cursor's tile (rotated order inside the unit).
  auto tile_key = [&](const Cursor& c) {
    int p = c.j + c.rot;
    if (p >= c.rt.count) p -= c.rt.count;
    return (c.rt.first + p) * TS;
  };
  // Block-table entries of the cursor's tile (scalar loads, issued ahead of use).
  // A run wholly outside the visible keys takes the entry of the nearest
  // visible key instead, so that only blocks the row owns are read; its keys
  // are masked. An empty row's masked tile reads no table entry.
  auto table_entry = [&](const Cursor& c) {
    TileEntries<NR> r;
    const int tb = tile_key(c);
    const int64_t bt_row = (int64_t)c.req * a.bt_stride;
    if constexpr (MODE == kKeyBlocks) {
      if (shift == 0 && tb >= c.rt.left && tb + TS <= c.rt.ctx) {
        // Token-granular map, every key of the tile visible: TS consecutive
        // entries, all in range (wide scalar loads).
#pragma unroll
        for (int i = 0; i < NR; ++i) r.e[i] = scalar_load(a.block_tables, bt_row + tb + i);
        return r;
      }
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      int key = tb + i * KPR;
      if constexpr (MODE != kTileBlocks) key = min(max(key, c.rt.left), c.rt.ctx - 1);
      r.e[i] = c.rt.ctx > 0 ? scalar_load(a.block_tables, bt_row + (key >> shift)) : 0;
    }
    return r;
  };
  auto kv_head_of = [&](const TileDesc& t) { return (int)fast_div((uint32_t)t.h, sa.head_groups_div); };
  auto describe = [&](const Cursor& c, const TileEntries<NR>& en) {
    constexpr int NROW = MODE == kKeyBlocks ? 1 : NR;
    TileDesc t;
    t.tb = tile_key(c);
    t.left = c.rt.left;
    t.ctx = c.rt.ctx;
    t.row = c.row;
    t.h = c.h;
    t.j = c.j;
    t.qrow = c.qrow;
    t.g = c.g;
#pragma unroll
    for (int i = 0; i < NROW; ++i)
      t.row0[i] = (((uint32_t)en.e[i] << shift) | (uint32_t)((t.tb + i * KPR) & block_mask)) * (uint32_t)(2 * D);
    t.flags = (c.j == 0 || c.g == g_begin ? kTileFirst : 0) |
              (c.j == c.rt.count - 1 || c.g == g_end - 1 ? kTileLast : 0) | (c.j == c.rt.count - 1 ? kUnitLast : 0);
    return t;
  };

  // ---- Loads -------------------------------------------------------------
  const uint32_t region = (uint32_t)(a.slots * D * 2);
  // K and V tiles -> LDS: load i, lane l fills piece s = 64 i + l, i.e. key
  // s / CPR, stored chunk s % CPR, which holds the key's chunk (s % CPR) ^ swz.
  // Byte offset of the row of key tt of the tile (this lane's key of load i).
  // kKeyBlocks: lane k of `keyed` holds key k's entry (written lane by lane
  // from the scalar entries); each lane fetches its own key's with a permute.
  auto row_of = [&](const TileDesc& t, int keyed, int i, int tt) -> uint32_t {
    if constexpr (MODE == kTileBlocks) return t.row0[0] + tt * (2 * D);
    if constexpr (MODE == kLoadBlocks) return t.row0[i] + (tt - i * KPR) * (2 * D);
    const int e = __builtin_amdgcn_ds_bpermute(tt << 2, keyed);
    return (((uint32_t)e << shift) | (uint32_t)((t.tb + tt) & block_mask)) * (uint32_t)(2 * D);
  };
  // kKeyBlocks: pack the prefetched scalar entries into one VGPR (lane k =
  // key k), so that one register instead of TS carries them to the loads.
  auto pack = [&](TileEntries<NR>& en) {
    if constexpr (MODE == kKeyBlocks) {
      int keyed = 0;
#pragma unroll
      for (int k = 0; k < TS; ++k) asm("v_writelane_b32 %0, %1, %2" : "=v"(keyed) : "s"(en.e[k]), "i"(k), "0"(keyed));
      en.keyed = keyed;
    }
  };
  auto issue_tile = [&](const TileDesc& t, const TileEntries<NR>& en, char* kt, char* vt) {
    const int keyed = en.keyed;
    const uint16_t* kbase = a.pool + (int64_t)kv_head_of(t) * a.slots * D;
    const uint16_t* vbase = kbase + (int64_t)a.kv_heads * a.slots * D;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, region, kBufferDword3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, region, kBufferDword3);
    const uint32_t kl = lds_addr(kt), vl = lds_addr(vt);
#pragma unroll
    for (int i = 0; i < S::LOADS; ++i) {
      const int s = i * 64 + lane, tt = s / S::CPR, pc = s % S::CPR;
      lds_dma16_once(kl + i * 1024, krs, row_of(t, keyed, i, tt) + ((pc ^ swz(tt, D / 8)) << 4));
    }
#pragma unroll
    for (int i = 0; i < S::LOADS; ++i) {
      const int s = i * 64 + lane, tt = s / S::CPR, pc = s % S::CPR;
      lds_dma16_once(vl + i * 1024, vrs, row_of(t, keyed, i, tt) + ((pc ^ swz(tt, D / 8)) << 4));
    }
  };
  // The unit's query heads -> LDS ([head][D], row-major). The resource covers
  // the valid heads only, so the rest of the buffer reads as zero.
  auto issue_query = [&](const TileDesc& t, char* qsb) {
    const int kvh = kv_head_of(t), hg = t.h - kvh * a.head_groups;
    const int hv = min(16, a.group - hg * 16);
    const uint16_t* qp = a.query + (int64_t)t.qrow * a.q_stride + (int64_t)(kvh * a.group + hg * 16) * D;
    const uint32_t bytes = (uint32_t)(hv * D * 2);
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc((void*)qp, (short)0, bytes, kBufferDword3);
    const uint32_t ql = lds_addr(qsb);
#pragma unroll
    for (int i = 0; i < QBYTES / 1024; ++i)
      if (i * 1024 < (int)bytes) lds_dma16(ql + i * 1024, qrs, i * 1024 + lane * 16);
  };

  // ---- Attention state -----------------------------------------------------
  bf16x8_t qb[S::NC];
  f32x4_t o[S::NO];
  float m_run = -INFINITY, l_run = 0.f;
  // Dot form: per head (uniform) running max, threshold and base; per lane
  // the partial sum of its key's probabilities and its output dims.
  u32x4_t qd[kDotMaxHeads][DOT ? DNC : 1];
  float od[kDotMaxHeads][DOT ? DOD : 1];
  float dm_run[kDotMaxHeads], dm_thr[kDotMaxHeads], dm_base[kDotMaxHeads], dl[kDotMaxHeads];
  // Without softcap: (m_run + kDecodeRescaleSlack) / scale, the raw-score
  // threshold of a re-base; and the base of the probabilities (m_run, or 0
  // before the first maximum). Both change only at a re-base.
  float m_thr = -INFINITY, m_base = 0.f;
  const float inv_scale = 1.f / a.score_scale;

  // Maximum and sum over the 32 keys of a tile in the dot form (lanes l and
  // l + 32 hold the same key): a 16-lane butterfly, then the two 16-lane rows
  // of each half combined; every lane receives the result.
  auto key32_max = [&](float x) {
    x = max2(x, dpp<kDppQuadXor1>(x));
    x = max2(x, dpp<kDppQuadXor2>(x));
    x = max2(x, dpp<kDppRowHalfMirror>(x));
    x = max2(x, dpp<kDppRowMirror>(x));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return max2(__uint_as_float(r[0]), __uint_as_float(r[1]));
  };
  auto key32_sum = [&](float x) {
    x = group_sum<16>(x);
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  };
  // Finished segments are not stored right away. The pipeline's waits count
  // every vector memory operation older than the newest tile (vmcnt), so a
  // store issued among the tile loads holds up the next wait until it is
  // acknowledged, which under full read load takes about a tile's time. Up to
  // two segments wait in registers instead and go out when the workgroup's
  // pipeline has drained (or when a third one needs the room). With D = 256
  // the registers are not there: segments are stored at once.
  constexpr int kMaxPend = D <= 128 ? 2 : 0;
  // Indices and flags in 32-bit words, not pointers (fewer scalar registers
  // held across the tile loop); addresses are formed when storing.
  struct Pending {
    f32x4_t v[S::NO];   // output rows already divided by l (output) or the raw partial
    float m, l;         // partial: running max / sum of head c16 (lanes q == 0)
    int dst;            // output row (bf16 output) or partial slot
    int kind;           // valid heads | 32 for a bf16 output | head 0 << 6 (output)
    int span;           // unit_span element of the record to write (-1: none)
    int span0, span1;
  };
  Pending pend0, pend1;
  int npend = 0;
  auto flush = [&](const Pending& e) {
    const int hv = e.kind & 31;
    const bool out = (e.kind & 32) != 0;
    const int head0 = e.kind >> 6;
    const int64_t part = (int64_t)e.dst * a.heads_per_group;  // partial slot's first head
    if constexpr (DOT) {
      // Lane (g = lane / 16, i = lane % 16) holds dims DOD * 16 g + 16 j + i
      // of every head (v[h][j]).
#pragma unroll
      for (int h = 0; h < kDotMaxHeads; ++h) {
        if (h >= hv) continue;
#pragma unroll
        for (int j = 0; j < DOD; ++j) {
          const int dim = DOD * 16 * (lane >> 4) + 16 * j + (lane & 15);
          if (out) a.out[(int64_t)e.dst * a.out_stride + (int64_t)(head0 + h) * D + dim] = (uint16_t)bf16_bits(e.v[h][j]);
          else a.part_o[(part + h) * D + dim] = e.v[h][j];
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int h = 4 * q + r;
        if (h >= hv) continue;
        if (out) {
          uint16_t* dst = a.out + (int64_t)e.dst * a.out_stride + (int64_t)(head0 + h) * D + c16;
#pragma unroll
          for (int c = 0; c < S::NO; ++c) dst[16 * c] = (uint16_t)bf16_bits(e.v[c][r]);
        } else {
          float* dst = a.part_o + (part + h) * D + c16;
#pragma unroll
          for (int c = 0; c < S::NO; ++c) dst[16 * c] = e.v[c][r];
        }
      }
    }
    if (!out && q == 0 && c16 < hv) {
      float* ml = a.part_ml + (part + c16) * 2;
      ml[0] = e.m;
      ml[1] = e.l;
    }
    if (e.span >= 0 && lane == 0) {
      sa.unit_span[e.span] = __int_as_float(e.span0);
      sa.unit_span[e.span + 1] = __int_as_float(e.span1);
    }
  };

  auto finalize = [&](const TileDesc& t) {
    float lrow[4];
    float lt[kDotMaxHeads];
    if constexpr (DOT) {
#pragma unroll
      for (int h = 0; h < kDotMaxHeads; ++h) lt[h] = key32_sum(dl[h]);
    } else {
      l_run = col4_sum(l_run);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        lrow[r] = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * q + r) << 2, __float_as_int(l_run)));
    }
    const int kvh = kv_head_of(t), hg = t.h - kvh * a.head_groups;
    const int hv = min(16, a.group - hg * 16);
    const int head0 = kvh * a.group + hg * 16;
    const int g0 = t.g - t.j;  // the unit's first tile
    if (kMaxPend == 2 && npend == 2) {
      flush(pend0);
      pend0 = pend1;
      npend = 1;
    }
    Pending e;
    const bool whole = g0 >= g_begin && g0 + row_tiles<TS>(t.ctx, a.window).count <= g_end;
    if constexpr (DOT) {
      // Lane h (< hv) carries head h's max and sum.
      e.m = lane == 0 ? dm_run[0] : lane == 1 ? dm_run[1] : dm_run[2];
      e.l = lane == 0 ? lt[0] : lane == 1 ? lt[1] : lt[2];
#pragma unroll
      for (int h = 0; h < kDotMaxHeads; ++h) {
        const float inv = whole ? (lt[h] > 0.f ? 1.f / lt[h] : 0.f) : 1.f;
#pragma unroll
        for (int j = 0; j < DOD; ++j) e.v[h][j] = od[h][j] * inv;
      }
    } else {
      e.m = m_run;
      e.l = l_run;
    }
    if (whole) {
      e.kind = hv | 32 | (head0 << 6);
      e.dst = t.qrow;
      if constexpr (!DOT) {
        float inv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) inv[r] = lrow[r] > 0.f ? 1.f / lrow[r] : 0.f;
#pragma unroll
        for (int c = 0; c < S::NO; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r) e.v[c][r] = o[c][r] * inv[r];
      }
    } else {
      e.kind = hv;
      e.dst = 2 * w + (g0 <= g_begin ? 0 : 1);  // partial slot
      if constexpr (!DOT) {
#pragma unroll
        for (int c = 0; c < S::NO; ++c) e.v[c] = o[c];
      }
    }
    e.span = -1;
    e.span0 = e.span1 = 0;
    if (t.flags & kUnitLast) {
      // This workgroup holds the unit's last tile: record where its partials are.
      const int wf = (int)((uint32_t)g0 / (uint32_t)per);
      e.span = (t.row * U + t.h) * 2;
      e.span0 = (int)(2 * wf + (g0 == wf * per ? 0 : 1));
      e.span1 = w;
    }
    if constexpr (kMaxPend == 0) {
      flush(e);
    } else {
      if (npend == 0) pend0 = e;
      else pend1 = e;
      ++npend;
    }
  };

  // Attend one tile from one stage (its loads, and its unit's query, have landed).
  auto read_query = [&](const TileDesc& t, const char* qsb) {
    const int hg = t.h - kv_head_of(t) * a.head_groups;
    const int hv = min(16, a.group - hg * 16);
    if constexpr (DOT) {
      // Head h's half (lane / 32) of the dims, as DNC 16-byte chunks.
      const int half = lane >> 5;
#pragma unroll
      for (int h = 0; h < kDotMaxHeads; ++h)
#pragma unroll
        for (int i = 0; i < DNC; ++i)
          qd[h][i] = h < hv ? *reinterpret_cast<const u32x4_t*>(qsb + h * (2 * D) + (half * DNC + i) * 16)
                            : u32x4_t{0u, 0u, 0u, 0u};
    } else {
#pragma unroll
      for (int c = 0; c < S::NC; ++c) {
        bf16x8_t v = *reinterpret_cast<const bf16x8_t*>(qsb + c16 * (2 * D) + (4 * c + q) * 16);
        qb[c] = c16 < hv ? v : bf16x8_t{};
      }
    }
  };
  // Masked keys of a tile hold arbitrary pool data: zero their V rows so that
  // a zero probability cannot meet a non-finite value.
  auto zero_masked_v = [&](const TileDesc& t, char* vt) {
    if (t.tb < t.left || t.tb + TS > t.ctx) {
#pragma unroll
      for (int i = 0; i < S::LOADS; ++i) {
        const int s = i * 64 + lane;
        const int key = t.tb + s / S::CPR;
        if (key < t.left || key >= t.ctx) *reinterpret_cast<uint4*>(vt + s * 16) = make_uint4(0, 0, 0, 0);
      }
    }
  };
  // Dot form of one tile: Q.K per key, online softmax per head, P.V per dim.
  auto dot_tile = [&](const TileDesc& t, const char* kt, char* vt) {
    const int kvh = kv_head_of(t), hg = t.h - kvh * a.head_groups;
    const int hv = min(16, a.group - hg * 16);
    const int key = lane & 31, half = lane >> 5;
    u32x4_t kc[DNC];
#pragma unroll
    for (int i = 0; i < DNC; ++i)
      kc[i] = *reinterpret_cast<const u32x4_t*>(kt + key * (2 * D) + (((half * DNC + i) ^ swz(key, D / 8)) << 4));
    float sd[kDotMaxHeads];
#pragma unroll
    for (int h = 0; h < kDotMaxHeads; ++h) {
      sd[h] = -INFINITY;
      if (h >= hv) continue;  // uniform
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int i = 0; i < DNC; ++i) {
        a0 = dot2(qd[h][i][0], kc[i][0], a0);
        a1 = dot2(qd[h][i][1], kc[i][1], a1);
        a0 = dot2(qd[h][i][2], kc[i][2], a0);
        a1 = dot2(qd[h][i][3], kc[i][3], a1);
      }
      const float part = a0 + a1;
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(part), __float_as_uint(part), false, false);
      float sv = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      if constexpr (SOFTCAP) sv = a.softcap_log2 * soft_tanh(sv * a.score_scale);
      const int k = t.tb + key;
      sd[h] = (SOFTCAP || !(t.tb >= t.left && t.tb + TS <= t.ctx)) ? ((k >= t.left && k < t.ctx) ? sv : -INFINITY)
                                                                    : sv;
    }
    // Re-base each head whose tile maximum passes its threshold.
    float mx[kDotMaxHeads];
    bool any = false;
#pragma unroll
    for (int h = 0; h < kDotMaxHeads; ++h) {
      mx[h] = h < hv ? key32_max(sd[h]) : -INFINITY;
      any = any || mx[h] > (SOFTCAP ? dm_run[h] + kDecodeRescaleSlack : dm_thr[h]);
    }
    if (__builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
      for (int h = 0; h < kDotMaxHeads; ++h) {
        if (!(mx[h] > (SOFTCAP ? dm_run[h] + kDecodeRescaleSlack : dm_thr[h]))) continue;  // uniform
        const float m_new = fmaxf(dm_run[h], SOFTCAP ? mx[h] : mx[h] * a.score_scale);
        const float alpha = dm_run[h] == -INFINITY ? 0.f : fast_exp2(dm_run[h] - m_new);
        dl[h] *= alpha;
#pragma unroll
        for (int j = 0; j < DOD; ++j) od[h][j] *= alpha;
        dm_run[h] = m_new;
        dm_thr[h] = (m_new + kDecodeRescaleSlack) * inv_scale;
        dm_base[h] = m_new == -INFINITY ? 0.f : m_new;
      }
    }
    // Probabilities (fp32 into the sums, bf16 into P.V), packed by key pairs:
    // lane 2k of each half holds keys (2k, 2k + 1) of every head.
    uint32_t pp[kDotMaxHeads];
#pragma unroll
    for (int h = 0; h < kDotMaxHeads; ++h) {
      const float p = SOFTCAP ? fast_exp2(sd[h] - dm_base[h]) : fast_exp2(__builtin_fmaf(sd[h], a.score_scale, -dm_base[h]));
      dl[h] += h < hv ? p : 0.f;
      const uint32_t b = bf16_bits(p);
      const uint32_t nb = __float_as_uint(dpp<kDppQuadXor1>(__uint_as_float(b)));
      pp[h] = b | (nb << 16);
    }
    zero_masked_v(t, vt);
    // P.V: the 16-lane group g = lane / 16 reads, for key quad kq, the 4 x 16
    // block of keys 4 kq .. + 3 and dims 32 g + 16 j .. + 15 (D = 128;
    // 16 g .. + 15 at D = 64) transposed: lane i of the group receives dim
    // d_j = block start + i for the four keys.
    const int grp = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int kq = 0; kq < TS / 4; ++kq) {
      const int tk = 4 * kq + (i16 >> 2);
#pragma unroll
      for (int j = 0; j < DOD; ++j) {
        const int c0 = DOD * 16 * grp + 16 * j;  // first dim of the block
        const int lc = c0 / 8 + ((i16 & 3) >> 1);
        const bf16x4_t v = lds_read_tr4(vt + tk * (2 * D) + ((lc ^ swz(tk, D / 8)) << 4) + ((i16 & 1) << 3));
        const auto vw = __builtin_bit_cast(u32x2_t, v);
#pragma unroll
        for (int h = 0; h < kDotMaxHeads; ++h) {
          if (h >= hv) continue;  // uniform
          const uint32_t p01 = __builtin_amdgcn_readlane(pp[h], 4 * kq);
          const uint32_t p23 = __builtin_amdgcn_readlane(pp[h], 4 * kq + 2);
          od[h][j] = dot2(vw[1], p23, dot2(vw[0], p01, od[h][j]));
        }
      }
    }
  };
  auto consume = [&](const TileDesc& t, const char* kt, char* vt, int qpar_t) {
    if (t.flags & kTileFirst) {
      read_query(t, qs[qpar_t]);
      if constexpr (DOT) {
#pragma unroll
        for (int h = 0; h < kDotMaxHeads; ++h) {
#pragma unroll
          for (int j = 0; j < DOD; ++j) od[h][j] = 0.f;
          dm_run[h] = -INFINITY;
          dm_thr[h] = -INFINITY;
          dm_base[h] = 0.f;
          dl[h] = 0.f;
        }
      } else {
#pragma unroll
        for (int c = 0; c < S::NO; ++c) o[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        m_run = -INFINITY;
        l_run = 0.f;
        m_thr = -INFINITY;
        m_base = 0.f;
      }
    }
    if constexpr (DOT) {
      dot_tile(t, kt, vt);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (t.flags & kTileLast) finalize(t);
      return;
    }

    // K tile -> registers as the A operand of S^T: lane (q, c16), group h holds
    // key 16h + c16, logical chunk 4c + q.
    bf16x8_t kr[S::TG][S::NC];
#pragma unroll
    for (int h = 0; h < S::TG; ++h) {
      const int tt = 16 * h + c16;
#pragma unroll
      for (int c = 0; c < S::NC; ++c)
        kr[h][c] = *reinterpret_cast<const bf16x8_t*>(kt + tt * (2 * D) + (((4 * c + q) ^ swz(tt, D / 8)) << 4));
    }
    f32x4_t sc[S::TG];
#pragma unroll
    for (int h = 0; h < S::TG; ++h) {
      sc[h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < S::NC; ++c) sc[h] = mfma32(kr[h][c], qb[c], sc[h]);
    }

    // Mask, and the row maximum over this lane's scores. Without softcap the
    // scores stay raw: a tile whose keys are all visible needs no per-element
    // mask, the maximum is compared with (m_run + kDecodeRescaleSlack) / scale
    // (kept with m_run), and the scale folds into the exponent below.
    const bool inside = !SOFTCAP && t.tb >= t.left && t.tb + TS <= t.ctx;  // wave-uniform
    if (!inside) {
#pragma unroll
      for (int h = 0; h < S::TG; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float s = sc[h][r];
          if constexpr (SOFTCAP) s = a.softcap_log2 * soft_tanh(s * a.score_scale);
          const int key = t.tb + 16 * h + 4 * q + r;
          sc[h][r] = (key >= t.left && key < t.ctx) ? s : -INFINITY;
        }
    }
    float mx;
    {
      float v[4 * S::TG];
#pragma unroll
      for (int i = 0; i < 4 * S::TG; ++i) v[i] = sc[i >> 2][i & 3];
      mx = col4_max(tree_max(v));
    }
    if (__builtin_amdgcn_ballot_w64(mx > (SOFTCAP ? m_run + kDecodeRescaleSlack : m_thr))) {
      const float m_new = fmaxf(m_run, SOFTCAP ? mx : mx * a.score_scale);
      const float alpha = m_run == -INFINITY ? 0.f : fast_exp2(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
      m_thr = (m_new + kDecodeRescaleSlack) * inv_scale;
      m_base = m_new == -INFINITY ? 0.f : m_new;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float f = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * q + r) << 2, __float_as_int(alpha)));
#pragma unroll
        for (int c = 0; c < S::NO; ++c) o[c][r] *= f;
      }
    }
#pragma unroll
    for (int h = 0; h < S::TG; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = SOFTCAP ? fast_exp2(sc[h][r] - m_base) : fast_exp2(__builtin_fmaf(sc[h][r], a.score_scale, -m_base));
        sc[h][r] = p;
        l_run += p;
      }

    zero_masked_v(t, vt);

    if constexpr (TS == 32) {
      bf16x8_t pa;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pa[r] = (__bf16)sc[0][r];
        pa[4 + r] = (__bf16)sc[1][r];
      }
#pragma unroll
      for (int c = 0; c < S::NO; ++c) {
        const int lc = 2 * c + ((c16 & 3) >> 1);
        const int t0 = 4 * q + (c16 >> 2), t1 = t0 + 16;
        const char* p0 = vt + t0 * (2 * D) + ((lc ^ swz(t0, D / 8)) << 4) + ((c16 & 1) << 3);
        const char* p1 = vt + t1 * (2 * D) + ((lc ^ swz(t1, D / 8)) << 4) + ((c16 & 1) << 3);
        const bf16x4_t v0 = lds_read_tr4(p0);
        const bf16x4_t v1 = lds_read_tr4(p1);
        const bf16x8_t vb = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
        o[c] = mfma32(pa, vb, o[c]);
      }
    } else {
      bf16x4_t pa;
#pragma unroll
      for (int r = 0; r < 4; ++r) pa[r] = (__bf16)sc[0][r];
#pragma unroll
      for (int c = 0; c < S::NO; ++c) {
        const int lc = 2 * c + ((c16 & 3) >> 1);
        const int t0 = 4 * q + (c16 >> 2);
        const char* p0 = vt + t0 * (2 * D) + ((lc ^ swz(t0, D / 8)) << 4) + ((c16 & 1) << 3);
        o[c] = mfma16(pa, lds_read_tr4(p0), o[c]);
      }
    }
    // The stage is refilled next: every LDS read of it must have returned.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (t.flags & kTileLast) finalize(t);
  };

  // ---- Pipeline ------------------------------------------------------------
  // Stage 0 / stage 1 alternate; the query buffer alternates per unit. The
  // share ends at the position g_end: `ahead` says whether the cursor, one
  // tile past the last issued one, is still inside it.
  int qpar = 0;
  TileEntries<NR> first_entry = table_entry(cur);
  pack(first_entry);
  TileDesc d0 = describe(cur, first_entry), d1;
  int qp0 = 0, qp1 = 0;                // query buffer of the tile in stage 0 / 1
  if (d0.flags & kTileFirst) issue_query(d0, qs[0]);
  issue_tile(d0, first_entry, kt0, vt0);
  advance(cur);
  bool ahead = cur.g < g_end;
  TileEntries<NR> next_entry = {};
  if (ahead) {
    next_entry = table_entry(cur);
    pack(next_entry);
  }
  while (true) {
    bool more = ahead;
    if (more) {
      d1 = describe(cur, next_entry);
      if (d1.flags & kTileFirst) {
        qpar ^= 1;
        issue_query(d1, qs[qpar]);
      }
      qp1 = qpar;
      issue_tile(d1, next_entry, kt1, vt1);
      advance(cur);
      ahead = cur.g < g_end;
      if (ahead) next_entry = table_entry(cur);
      wait_vmem<2 * S::LOADS>();
      pack(next_entry);  // its scalar loads landed during the wait
    } else {
      wait_vmem<0>();
    }
    consume(d0, kt0, vt0, qp0);
    if (!more) break;

    more = ahead;
    if (more) {
      d0 = describe(cur, next_entry);
      if (d0.flags & kTileFirst) {
        qpar ^= 1;
        issue_query(d0, qs[qpar]);
      }
      qp0 = qpar;
      issue_tile(d0, next_entry, kt0, vt0);
      advance(cur);
      ahead = cur.g < g_end;
      if (ahead) next_entry = table_entry(cur);
      wait_vmem<2 * S::LOADS>();
      pack(next_entry);  // its scalar loads landed during the wait
    } else {
      wait_vmem<0>();
    }
    consume(d1, kt1, vt1, qp1);
    if (!more) break;
  }
  // Every tile has been consumed: store the segments still held.
  if (kMaxPend > 0 && npend >= 1) flush(pend0);
  if (kMaxPend > 0 && npend == 2) flush(pend1);
}

template <int D, bool SOFTCAP, int MODE>
__global__ __launch_bounds__(64, 1) void decode_stream_kernel(StreamArgs sa) {
  decode_stream_body<D, SOFTCAP, MODE, kArithMfma>(sa);
}
template <int D, bool SOFTCAP, int MODE>
__global__ __launch_bounds__(64, 1) void decode_stream_dot_kernel(StreamArgs sa) {
  decode_stream_body<D, SOFTCAP, MODE, kArithDot>(sa);
}

// ---------------------------------------------------------------------------
// Merge of the units that span workgroups
// ---------------------------------------------------------------------------
struct StreamMergeArgs {
  const float* part_o;
  const float* part_ml;
  const float* unit_span;
  const int32_t* row_map;
  int32_t group, head_groups, heads_per_group, units_per_row, wgs;
  uint16_t* out;
  int64_t out_stride;
};

// One wave per (row, query head).
template <int D>
__global__ __launch_bounds__(64) void stream_merge_kernel(StreamMergeArgs m) {
  constexpr int PER_LANE = D / 64;
  const int lane = threadIdx.x;
  const int head = blockIdx.x, row = blockIdx.y;
  const int kvh = head / m.group, within = head - kvh * m.group;
  const int hg = within / 16, hh = within - hg * 16;
  const int64_t unit = (int64_t)row * m.units_per_row + kvh * m.head_groups + hg;
  const int first_slot = __float_as_int(m.unit_span[unit * 2]);
  const int w_last = __float_as_int(m.unit_span[unit * 2 + 1]);
  const int w_first = first_slot >> 1;
  if (w_first >= w_last) return;            // finalised by its only workgroup
  if (first_slot < 0 || w_last >= m.wgs) return;  // not a span this call wrote
  const int nslots = w_last - w_first + 1;
  auto slot_of_part = [&](int k) { return k == 0 ? first_slot : 2 * (w_first + k); };
  // One pass with a running max; the partials of BATCH slots are loaded
  // together, one memory round trip per batch: batches of four for units of
  // up to four parts, of sixteen for longer units (long contexts spread one
  // unit over many workgroups).
  float mm = -INFINITY, ll = 0.f;
  float acc[PER_LANE];
#pragma unroll
  for (int e = 0; e < PER_LANE; ++e) acc[e] = 0.f;
  auto merge_parts = [&](auto batch) {
    constexpr int BATCH = decltype(batch)::value;
    for (int k0 = 0; k0 < nslots; k0 += BATCH) {
      float mp[BATCH], lp[BATCH], op[BATCH][PER_LANE];
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int64_t pi = (int64_t)slot_of_part(min(k0 + u, nslots - 1)) * m.heads_per_group + hh;
        mp[u] = m.part_ml[pi * 2];
        lp[u] = m.part_ml[pi * 2 + 1];
#pragma unroll
        for (int e = 0; e < PER_LANE; ++e) op[u][e] = m.part_o[pi * D + lane + 64 * e];
      }
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        // Slots past the unit's last (clamped duplicates) weigh zero.
        const float mu = k0 + u < nslots ? mp[u] : -INFINITY;
        const float mn = fmaxf(mm, mu);
        const float fa = mm == -INFINITY ? 0.f : fast_exp2(mm - mn);
        const float fb = mu == -INFINITY ? 0.f : fast_exp2(mu - mn);
        ll = ll * fa + lp[u] * fb;
#pragma unroll
        for (int e = 0; e < PER_LANE; ++e) acc[e] = acc[e] * fa + op[u][e] * fb;
        mm = mn;
      }
    }
  };
  if (nslots <= 4) merge_parts(std::integral_constant<int, 4>{});
  else merge_parts(std::integral_constant<int, 16>{});
  const float inv = ll > 0.f ? 1.f / ll : 0.f;
  const int orow = m.row_map ? m.row_map[row] : row;
  uint16_t* dst = m.out + (int64_t)orow * m.out_stride + (int64_t)head * D;
#pragma unroll
  for (int e = 0; e < PER_LANE; ++e) dst[lane + 64 * e] = (uint16_t)bf16_bits(acc[e] * inv);
}

template <int D, bool SOFTCAP, int MODE>
int resident_per_cu() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_stream_kernel<D, SOFTCAP, MODE>, 64, 0) !=
          hipSuccess ||
      n <= 0)
    n = 1;
  return n;
}

template <int D, int MODE>
int resident_per_cu(bool softcap) {
  return softcap ? resident_per_cu<D, true, MODE>() : resident_per_cu<D, false, MODE>();
}

template <int D>
int resident_per_cu(bool softcap, int mode) {
  if (mode == kKeyBlocks) return resident_per_cu<D, kKeyBlocks>(softcap);
  if (mode == kLoadBlocks) return resident_per_cu<D, kLoadBlocks>(softcap);
  return resident_per_cu<D, kTileBlocks>(softcap);
}

template <int D, int MODE>
void launch_stream_mode(const StreamArgs& sa, bool softcap, dim3 grid, hipStream_t stream) {
#if GK_STREAM_DOT
  if constexpr (D <= 128) {
    if (sa.d.heads_per_group <= kDotMaxHeads) {
      if (softcap) decode_stream_dot_kernel<D, true, MODE><<<grid, 64, 0, stream>>>(sa);
      else decode_stream_dot_kernel<D, false, MODE><<<grid, 64, 0, stream>>>(sa);
      return;
    }
  }
#endif
  if (softcap) decode_stream_kernel<D, true, MODE><<<grid, 64, 0, stream>>>(sa);
  else decode_stream_kernel<D, false, MODE><<<grid, 64, 0, stream>>>(sa);
}

template <int D>
void launch_stream_kernel(const StreamArgs& sa, bool softcap, int mode, dim3 grid, hipStream_t stream) {
  if (mode == kKeyBlocks) launch_stream_mode<D, kKeyBlocks>(sa, softcap, grid, stream);
  else if (mode == kLoadBlocks) launch_stream_mode<D, kLoadBlocks>(sa, softcap, grid, stream);
  else launch_stream_mode<D, kTileBlocks>(sa, softcap, grid, stream);
}

// Slot lookup of a block size (the kernel's MODE).
int block_mode(int head_dim, int block_size) {
  const int ts = head_dim == 256 ? 16 : 32, keys_per_load = 64 / (head_dim / 8);
  return block_size >= ts ? kTileBlocks : block_size >= keys_per_load ? kLoadBlocks : kKeyBlocks;
}

}  // namespace

int device_cus();

// Workgroups of the balanced grid: the CUs times the workgroups one CU keeps
// resident (LDS-bound), queried once per device and kernel variant.
int stream_decode_wgs(int head_dim, bool softcap, int block_size) {
  static std::mutex mu;
  static int cached[64][3][2][3] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  const int di = head_dim == 64 ? 0 : (head_dim == 128 ? 1 : 2);
  const int mode = block_mode(head_dim, block_size);
  std::lock_guard<std::mutex> lock(mu);
  int& slot = cached[dev][di][softcap ? 1 : 0][mode];
  if (!slot) {
    int per_cu = 1;
    switch (head_dim) {
      case 64: per_cu = resident_per_cu<64>(softcap, mode); break;
      case 128: per_cu = resident_per_cu<128>(softcap, mode); break;
      default: per_cu = resident_per_cu<256>(softcap, mode); break;
    }
    slot = device_cus() * per_cu;
  }
  return slot;
}

size_t stream_decode_workspace_bytes(int head_dim, int heads_per_group, int64_t units, int wgs) {
  const size_t parts = (size_t)2 * wgs * heads_per_group;
  const size_t o_bytes = (parts * head_dim * sizeof(float) + 255) & ~size_t{255};
  const size_t ml_bytes = (parts * 2 * sizeof(float) + 255) & ~size_t{255};
  return o_bytes + ml_bytes + (size_t)units * 2 * sizeof(float);
}

int launch_stream_decode(const DecodeArgs& a, bool softcap, int head_dim, int wgs, void* workspace,
                         hipStream_t stream) {
  StreamArgs sa{};
  sa.d = a;
  sa.units_per_row = a.kv_heads * a.head_groups;
  sa.wgs = wgs;
  sa.wgs_div = div_magic((uint32_t)wgs);
  sa.head_groups_div = div_magic((uint32_t)a.head_groups);
  sa.kv_heads_div = div_magic((uint32_t)a.kv_heads);
  const size_t parts = (size_t)2 * wgs * a.heads_per_group;
  const size_t o_bytes = (parts * head_dim * sizeof(float) + 255) & ~size_t{255};
  const size_t ml_bytes = (parts * 2 * sizeof(float) + 255) & ~size_t{255};
  sa.d.part_o = static_cast<float*>(workspace);
  sa.d.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + o_bytes);
  sa.unit_span = reinterpret_cast<float*>(static_cast<char*>(workspace) + o_bytes + ml_bytes);

  const dim3 grid(wgs);
  const int mode = block_mode(head_dim, 1 << a.block_shift);
  switch (head_dim) {
    case 64: launch_stream_kernel<64>(sa, softcap, mode, grid, stream); break;
    case 128: launch_stream_kernel<128>(sa, softcap, mode, grid, stream); break;
    default: launch_stream_kernel<256>(sa, softcap, mode, grid, stream); break;
  }
  if (int rc = hip_status(hipGetLastError(), "gk_paged_decode stream launch")) return rc;

  StreamMergeArgs m{};
  m.part_o = sa.d.part_o;
  m.part_ml = sa.d.part_ml;
  m.unit_span = sa.unit_span;
  m.row_map = a.row_map;
  m.group = a.group;
  m.head_groups = a.head_groups;
  m.heads_per_group = a.heads_per_group;
  m.units_per_row = sa.units_per_row;
  m.wgs = wgs;
  m.out = a.out;
  m.out_stride = a.out_stride;
  const dim3 mgrid(a.q_heads, a.rows);
  switch (head_dim) {
    case 64: stream_merge_kernel<64><<<mgrid, 64, 0, stream>>>(m); break;
    case 128: stream_merge_kernel<128><<<mgrid, 64, 0, stream>>>(m); break;
    default: stream_merge_kernel<256><<<mgrid, 64, 0, stream>>>(m); break;
  }
  return hip_status(hipGetLastError(), "gk_paged_decode stream merge launch");
}

}  // namespace gk
