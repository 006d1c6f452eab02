// Chunked / prefix-shared paged prefill attention for gfx950 (bf16 MFMA).
//
// A sequence contributes a chunk of consecutive query rows at positions
// prefix .. prefix + rows - 1; row i attends keys [left_i, prefix + i] of its
// request (causal; left_i = prefix + i - window + 1 with a sliding window).
// The chunk's own K/V rows are already in the pool (the store runs first), so
// every key is read through the block table.
//
// Work decomposition. A workgroup of eight waves owns one (sequence, kv head,
// tile of rows). The GQA group is folded into the tile: its 256 "query rows"
// (128 at head_dim 256) are (row, head) pairs, so one K/V tile serves every
// head of the group. Each wave computes 32 query rows (two 16-column MFMA
// tiles; one, 16 rows, at head_dim 256) against the keys of a step (64 at
// head_dim 128, 32 at head_dim 64 and 256):
//   S^T[key][qrow] = K . Q^T      v_mfma_f32_16x16x32_bf16, K from LDS
//   O[qrow][dim]  += P . V        P straight from S^T's registers, V read
//                                 transposed from LDS (ds_read_b64_tr_b16)
// A step's K and V tiles are shared by the eight waves through LDS: 16-byte
// buffer->LDS loads issued by the whole workgroup, XOR-swizzled by token,
// double-buffered so the next tile streams in while the current one is used.
// Online softmax runs in log2 units with a lazily re-based running maximum.
//
// Numerics versus the reference (the tile chain of
// src/bridge/paged_attention_tiles.cpp:57-195): fp32 scores times scale,
// probabilities rounded to bf16 before P.V (relative to the running maximum),
// fp32 accumulation, one normalisation at the end by the sum of those bf16
// probabilities, bf16 output.
#include "gk_mfma.hpp"
#include "work_order.hpp"

#include <algorithm>
#include <type_traits>

namespace gk {
namespace {

// Waves per workgroup (each owns 16 * kNT query rows). Eight, one workgroup
// per CU (two waves per SIMD): each K/V tile is loaded into LDS once for 256
// query rows instead of twice for two 128-row workgroups (C4, 64-key steps,
// same box: 180.0 -> 174.1 us with four -> eight waves; 168.8 us together with
// the early V reads below).
constexpr int kPrefillWaves = 8;
// 16-column query tiles per wave. Two at head_dim 64 and 128: three fit in 256
// VGPRs only without the early V reads, and four spill; both also quantise
// C4's rows badly (48- or 64-row tiles of 512-row chunks leave a partial round
// of workgroups). One at head_dim 256, whose output accumulators alone take 64
// VGPRs per tile: with two, every head_dim 256 instance spills 536-588 bytes
// per lane; four waves of two tiles (one wave per SIMD, accumulators in AGPRs,
// no spills) measured 163.6-164.7 -> 227.4-227.5 us on C4's shapes at head_dim
// 256: the second wave of a SIMD matters more than halving the operand reads.
constexpr int kNT = 2;
constexpr int kQrowsPerWave = 16 * kNT;
template <int D>
constexpr int prefill_nt() { return D > 128 ? 1 : kNT; }
// Query rows per workgroup at head dimension d.
constexpr int prefill_qrows(int d) { return kPrefillWaves * 16 * (d > 128 ? 1 : kNT); }
// Keys per step: 64 at head_dim 128 (half the per-step barriers, cross-lane
// maxima, re-base checks and load setup of 32-key steps: C4 178.1 -> 166.8
// us); 32 at head_dim 64, whose 64-key form needs 130 VGPRs and so would drop
// from four waves per SIMD to three, and at head_dim 256, where a 64-key K
// and V tile pair takes 64 KiB of LDS per stage.
template <int D>
constexpr int prefill_keys() { return D == 128 ? 64 : 32; }
// K/V pipeline depth. Two: three and four stages measured the same on C4 (the
// kernel is bound by its instruction stream, not by load latency).
constexpr int kStages = 2;
constexpr float kLazyRescale = 8.f;
// XCDs of an MI355X: consecutive workgroups of a launch go to consecutive XCDs.
constexpr int kXcds = 8;

struct PrefillArgs {
  const uint16_t* query;
  int64_t q_stride;
  const uint16_t* pool;
  int64_t slots;
  const int32_t* block_tables;
  int64_t bt_stride;
  int32_t block_shift;
  const int32_t* seq_request;
  const int32_t* seq_first_row;
  const int32_t* seq_rows;
  const int32_t* seq_prefix;
  int32_t q_heads, kv_heads, group, rows_per_tile;
  int32_t tiles, seqs;  // row tiles per sequence; sequences
  float score_scale;   // scale * log2(e), or scale / softcap when capping
  float softcap_log2;  // softcap * log2(e) when capping
  int32_t window;
  uint16_t* out;
  int64_t out_stride;
  DivMagic tiles_div, seqs_div, group_div;  // division by tiles, seqs and group (work_order.hpp)
};

template <int D>
struct PrefillShape {
  static constexpr int NC = D / 32;                 // 32-dim k chunks of Q.K
  static constexpr int CPR = D / 8;                 // 16-byte chunks per head row
  static constexpr int NO = D / 16;                 // 16-dim output chunks
  static constexpr int TILE = prefill_keys<D>() * D * 2;  // bytes of one K or V tile
  static constexpr int NI = TILE / 1024;            // 1 KiB load instructions per tile
};

// How a step's slots are found (the MODE template argument):
//  kStepBlocks  blocks of at least a step's keys: one scalar block-table entry per step;
//  kLoadBlocks  blocks of >= 64 / (D / 8) keys (one load instruction's): one
//               scalar entry per load instruction;
//  kKeyBlocks   shorter blocks, down to the token-granular map (block 1): each
//               lane reads its own key's entry with a vector load.
constexpr int kStepBlocks = 0, kLoadBlocks = 1, kKeyBlocks = 2;

// Head_dim 128 step order. 0: every wave runs Q.K(i), softmax(i), P.V(i)
// after the step's barrier, so the two waves of a SIMD reach their MFMA and
// VALU phases together. 1 (build variant): the waves of the second half
// (waves 4-7, the second wave of each SIMD) run Q.K(i), P.V(i - 1),
// softmax(i), the same operations on the accumulators in the same order but
// half a step later, so one wave's softmax can run under the other's MFMAs.
// V tiles of three steps are then live (three V stages, two K stages).
#ifndef GK_PREFILL_LAG
#define GK_PREFILL_LAG 0
#endif
// Head_dim 128 software pipeline (build variant, no softcap): iteration i
// runs Q.K(i) interleaved with the probabilities of step i - 1, then
// P.V(i - 1) interleaved with the row maxima of step i, so each wave's own
// instruction stream alternates MFMAs with independent VALU work. V lags K by
// one step in LDS (the same two K and two V stages).
#ifndef GK_PREFILL_PIPE
#define GK_PREFILL_PIPE 0
#endif
#ifndef GK_PREFILL_PIPE_ORDER
#define GK_PREFILL_PIPE_ORDER 1
#endif

template <int D, bool SOFTCAP, int MODE>
__global__ __launch_bounds__(kPrefillWaves * 64, 1) void prefill_kernel(PrefillArgs a) {
  using S = PrefillShape<D>;
  // This head dimension's query tiles per wave (in place of the namespace's).
  constexpr int kNT = prefill_nt<D>(), kQrowsPerWave = 16 * kNT;
  constexpr int kKeys = prefill_keys<D>();
  static_assert(kKeys == 32 || kKeys == 64, "a step is one or two 32-key halves");
  constexpr int kKG = kKeys / 16;  // 16-key groups per step (Q.K tiles)
  constexpr int kKH = kKeys / 32;  // 32-key halves per step (P.V k chunks)
  // Load instructions per wave per K (or V) tile; wave w issues instructions w, w + waves, ...
  constexpr int LPW = (S::NI + kPrefillWaves - 1) / kPrefillWaves;
  constexpr int NE = MODE == kStepBlocks ? 1 : LPW;  // block-table entries per wave (per lane) per step
  constexpr int KPL = kKeys / S::NI;                 // keys of one load instruction
  constexpr bool CLAMPED = MODE != kStepBlocks;      // entries of keys outside [key_begin, key_end) clamped
  static_assert(MODE != kKeyBlocks || kStages == 2, "per-lane entries rely on the step's full drain");
  // kStages K/V stages. The direct loads are asm statements the compiler does
  // not track, so one array serves every stage; reads are ordered by the
  // explicit vmcnt wait and the barrier of each step.
  // A region of its own (after the stages) holds, after the step loop, each
  // wave's output rows in bf16 (rows padded by 16 bytes so that the four
  // q-groups' rows of a write fall on different banks), read back as 16-byte
  // pieces for the global stores. Being separate from the stages, a wave
  // starts its output as soon as its own last step ends, with no barrier
  // (132 KiB at head_dim 128, one workgroup per CU either way).
  constexpr bool kLag = GK_PREFILL_LAG && D == 128 && !SOFTCAP;  // softcap: no registers to spare
  constexpr bool kPipe = GK_PREFILL_PIPE && D == 128 && !SOFTCAP && !kLag;
  constexpr int kOutRowBytes = 2 * D + 16;
  constexpr int kKvBytes = (kLag ? 5 : kStages * 2) * S::TILE,
                kOutBytes = kPrefillWaves * kQrowsPerWave * kOutRowBytes;
  __shared__ __attribute__((aligned(16))) char lds[kKvBytes + kOutBytes];
  auto kv = reinterpret_cast<char(*)[2][S::TILE]>(lds);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (LDS bases of the direct loads)
  const int q = lane >> 4, c16 = lane & 15;
  // Work item (row tile, sequence, kv head), row tiles fastest, kv heads
  // slowest. Workgroup b runs on XCD b % 8, so b is mapped to items with each
  // XCD taking one contiguous eighth of that order: the workgroups sharing a
  // kv head's K/V (every row tile of every sequence, which share the prefix)
  // run under one L2 instead of fetching it into all eight. Inside its share
  // an XCD takes the row tiles highest first (heavy_first_item).
  //
  // The prologue is a chain of scalar loads: the arguments, the sequence's
  // fields, its first block-table entry, then the first K/V tile. Each link is
  // a memory round trip, so every argument is materialised in one batch at the
  // top and the four sequence fields are loaded together ahead of the
  // early-exit test (the compiler would otherwise fetch the sequence pointers
  // after the work-item arithmetic and the fields one by one: six round trips
  // before the first K/V load instead of three).
  asm volatile("" ::"s"(a.seq_rows), "s"(a.seq_prefix), "s"(a.seq_first_row), "s"(a.seq_request),
               "s"(a.block_tables), "s"(a.query), "s"(a.pool), "s"(a.out), "s"(a.tiles), "s"(a.seqs),
               "s"(a.rows_per_tile), "s"(a.group), "s"(a.bt_stride), "s"(a.block_shift), "s"(a.window),
               "s"(a.q_stride), "s"(a.slots), "s"(a.kv_heads), "s"(gridDim.x), "s"(a.tiles_div.mul),
               "s"(a.tiles_div.shift), "s"(a.seqs_div.mul), "s"(a.seqs_div.shift), "s"(a.group_div.mul),
               "s"(a.group_div.shift));
  const int nitems = gridDim.x, xcd = blockIdx.x % kXcds, per_xcd = nitems / kXcds, extra = nitems % kXcds;
  // Divisions by runtime values go through the host's multiply-shift pairs.
  const auto div_tiles = [&](int x) { return (int)fast_div((uint32_t)x, a.tiles_div); };
  const auto div_group = [&](int x) { return (int)fast_div((uint32_t)x, a.group_div); };
  const int item = heavy_first_item(xcd * per_xcd + min(xcd, extra), per_xcd + (xcd < extra), a.tiles,
                                    (int)blockIdx.x / kXcds, div_tiles);
  const int item_seq = div_tiles(item), tile = item - item_seq * a.tiles;
  const int kvh = (int)fast_div((uint32_t)item_seq, a.seqs_div), seq = item_seq - kvh * a.seqs;
  const int rows = a.seq_rows[seq], prefix = a.seq_prefix[seq], seq_first = a.seq_first_row[seq];
  const int request = a.seq_request[seq];
  asm volatile("" ::"s"(rows), "s"(prefix), "s"(seq_first), "s"(request));
  const int r0 = tile * a.rows_per_tile;
  if (r0 >= rows) return;
  const int nr = min(a.rows_per_tile, rows - r0);
  const int first_row = seq_first + r0;
  const int32_t* __restrict__ bt = a.block_tables + (int64_t)request * a.bt_stride;
  const int g = a.group;
  const int pos_lo = prefix + r0, pos_hi = prefix + r0 + nr - 1;
  const int key_end = pos_hi + 1;
  const int key_begin = a.window > 0 ? max(0, pos_lo - a.window + 1) : 0;
  const int kb0 = key_begin & ~(kKeys - 1);
  const int nsteps = (key_end - kb0 + kKeys - 1) / kKeys;

  // This lane's query rows (one per 16-column tile): qrow = (row, head).
  int qpos[kNT], qleft[kNT];
  bool qvalid[kNT];
  bf16x8_t qb[kNT][S::NC];
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt) {
    const int qr = wave * kQrowsPerWave + nt * 16 + c16;
    const int row = div_group(qr), head = qr - row * g;
    qvalid[nt] = row < nr;
    qpos[nt] = qvalid[nt] ? pos_lo + row : -1;
    qleft[nt] = a.window > 0 ? qpos[nt] - a.window + 1 : 0;
    const uint16_t* src = a.query + (int64_t)(first_row + row) * a.q_stride + (int64_t)(kvh * g + head) * D;
#pragma unroll
    for (int c = 0; c < S::NC; ++c) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (qvalid[nt]) v = load16(src + (4 * c + q) * 8);
      qb[nt][c] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  // Smallest query position and largest window start over this wave's valid rows.
  const int wave_pos_min = pos_lo + div_group(wave * kQrowsPerWave);
  const int wave_left_max =
      a.window > 0 ? pos_lo + min(nr - 1, div_group(wave * kQrowsPerWave + kQrowsPerWave - 1)) - a.window + 1 : 0;

  // At d 128 the row sums of the bf16 probabilities run on one more MFMA per
  // half step against an all-ones operand, in the output layout (rows 4q + r).
  // At d 64 the registers would drop the kernel from four waves per SIMD to
  // three, which costs more than it saves: each lane sums its query row on the
  // VALU (component 0 of l_run).
  constexpr bool kMfmaSum = D >= 128;
  // Step loop (below): at d 64 two groups of waves alternate between MFMA and
  // softmax phases (C4 shapes: 113.7 -> 104.8 us); at d 128 the same order
  // measured 158.9 -> 181.0 us, with or without the phase offset, so d 128
  // keeps one barrier per step with every wave in Q.K -> softmax -> P.V order.
  constexpr bool kPingPong = D < 128;
  f32x4_t o[kNT][S::NO];
  float m_run[kNT];
  // Without softcap the re-base check compares the raw score maximum with
  // (m_run + kLazyRescale) / scale, kept per tile and updated at each re-base:
  // the step's maximum is scaled only when a re-base is due.
  float m_thr[kNT];
  const float inv_scale = 1.f / a.score_scale;
  // The base the probabilities are formed against: m_run, or 0 while the row
  // has no maximum yet (kept with m_run, so a step does not select it).
  float m_base[kNT];
  f32x4_t l_run[kNT];
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt) {
#pragma unroll
    for (int c = 0; c < S::NO; ++c) o[nt][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    m_run[nt] = -INFINITY;
    m_thr[nt] = -INFINITY;
    m_base[nt] = 0.f;
    l_run[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  const uint16_t* kbase = a.pool + (int64_t)kvh * a.slots * D;
  const uint16_t* vbase = kbase + (int64_t)a.kv_heads * a.slots * D;
  const uint32_t region = (uint32_t)(a.slots * D * 2);
  // The unrolled d 128 loop passes the resources to the direct-load asm as
  // words made uniform with readfirstlane (the compiler keeps the opaque
  // resource in VGPRs there); d 64 keeps the builtin resource (1.8% faster).
  auto make_rsrc = [&](const uint16_t* base) {
    if constexpr (D < 128) return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, region, kBufferDword3);
    else return buffer_words(base, region);
  };
  using Rsrc = decltype(make_rsrc(kbase));
  const Rsrc krs = make_rsrc(kbase), vrs = make_rsrc(vbase);
  const int shift = a.block_shift, bmask = (1 << shift) - 1;

  // Block-table entries of the step at key tb (scalar loads, or per-lane
  // vector loads for kKeyBlocks, fetched a step ahead: the loop's wait before
  // its closing barrier covers them). With CLAMPED a key outside
  // [key_begin, key_end) takes the entry of the nearest such key.
  struct Entries {
    int e[NE];
  };
  auto entry_of = [&](int tb) __attribute__((always_inline)) {
    Entries en;
#pragma unroll
    for (int k = 0; k < NE; ++k) {
      int key = tb;
      if constexpr (MODE == kLoadBlocks) key += (wave + k * kPrefillWaves) * KPL;
      if constexpr (MODE == kKeyBlocks) key += (wave + k * kPrefillWaves) * KPL + lane / S::CPR;
      if constexpr (CLAMPED) key = min(max(key, key_begin), key_end - 1);
      if constexpr (MODE == kKeyBlocks) en.e[k] = bt[key >> shift];
      else en.e[k] = scalar_load(bt, key >> shift);
    }
    return en;
  };
  // Byte offsets of this wave's direct loads for the step at tb, the same for
  // its K and its V tile. Steps are kKeys-aligned. Piece p = 64 ins + lane of
  // load instruction ins (wave ins % waves): token p / CPR, stored chunk
  // p % CPR holding the token's chunk (p % CPR) ^ swz(token, D / 8). A token
  // outside [key_begin, key_end) reads the row of the nearest token inside:
  // every row read is a stored token, so the masked keys' V rows are finite
  // and their zero probabilities contribute exactly zero (no zeroing pass).
  // The clamped token stays in the block of the entry used for it: blocks of
  // kKeys or more hold the whole step, shorter blocks whole load instructions
  // or (kKeyBlocks) the lane's own token, and clamping is monotone.
  struct Offsets {
    uint32_t v[LPW];
  };
  auto offsets_of = [&](int tb, const Entries& en) __attribute__((always_inline)) {
    Offsets of{};
    // One block holds the whole step: the clamped key's offset in the step
    // stays in [0, kKeys) (the first step starts at or below key_begin, the
    // last holds key_end - 1), so the slot is a scalar base plus that offset.
    const int lo = key_begin - tb, hi = key_end - 1 - tb;
    const uint32_t step_slot = ((uint32_t)en.e[0] << shift) + (uint32_t)(tb & bmask);
#pragma unroll
    for (int k = 0; k < LPW; ++k) {
      const int ins = wave + k * kPrefillWaves;
      if (S::NI % kPrefillWaves != 0 && ins >= S::NI) break;  // wave-uniform
      const int p = ins * 64 + lane, tt = p / S::CPR, pc = p % S::CPR;
      uint32_t slot;
      if constexpr (MODE == kStepBlocks) {
        slot = step_slot + (uint32_t)min(max(tt, lo), hi);
      } else {
        const int key = min(max(tb + tt, key_begin), key_end - 1);
        slot = (uint32_t)((en.e[k] << shift) | (key & bmask));
      }
      of.v[k] = slot * (2 * D) + ((pc ^ swz(tt, D / 8)) << 4);
    }
    return of;
  };
  auto issue = [&](const Offsets& of, Rsrc rs, char* tile) __attribute__((always_inline)) {
    // Per-lane entries are vector loads of the previous step, already complete
    // (the loop waits for every load before its closing barrier); say so to
    // the compiler.
    if constexpr (MODE == kKeyBlocks) wait_vmem_visible();
    const uint32_t base = lds_addr(tile);
#pragma unroll
    for (int k = 0; k < LPW; ++k) {
      const int ins = wave + k * kPrefillWaves;
      if (S::NI % kPrefillWaves != 0 && ins >= S::NI) break;  // wave-uniform
      if constexpr (D < 128) lds_dma16(base + ins * 1024, rs, of.v[k]);
      else lds_dma16_w(base + ins * 1024, rs, of.v[k]);
    }
  };

  // Scores of the current step and probabilities of the previous one.
  f32x4_t sc[kKG][kNT];
  bf16x8_t pa[kKH][kNT];

  // S^T = K.Q^T into sc: lane (q, c16) gets qrow c16 (+16 nt), keys tb + 16h + 4q + r.
  auto scores = [&](const char* kt) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < kKG; ++h) {
      const int tt = 16 * h + c16;
      bf16x8_t kr[S::NC];
#pragma unroll
      for (int c = 0; c < S::NC; ++c)
        kr[c] = *reinterpret_cast<const bf16x8_t*>(kt + tt * (2 * D) + (((4 * c + q) ^ swz(tt, D / 8)) << 4));
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        sc[h][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < S::NC; ++c) sc[h][nt] = mfma32(kr[c], qb[nt][c], sc[h][nt]);
      }
    }
  };

  // V operand c of P . V for the 32-key half hh of the V tile vt: keys
  // 32hh + 4q + (c16 >> 2) and 32hh + 16 + 4q + (c16 >> 2), dims
  // 16c + 4 (c16 & 3), read transposed.
  auto read_v = [&](const char* vt, int hh, int c) __attribute__((always_inline)) {
    const int lc = 2 * c + ((c16 & 3) >> 1);
    const int t0 = 32 * hh + 4 * q + (c16 >> 2), t1 = t0 + 16;
    const bf16x4_t v0 = lds_read_tr4(vt + t0 * (2 * D) + ((lc ^ swz(t0, D / 8)) << 4) + ((c16 & 1) << 3));
    const bf16x4_t v1 = lds_read_tr4(vt + t1 * (2 * D) + ((lc ^ swz(t1, D / 8)) << 4) + ((c16 & 1) << 3));
    return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  // O[qrow][dim] += P . V with pa and the V tile vt, and the row sums. The
  // first half's operands come from vfirst when the caller read them earlier.
  auto accumulate = [&](const char* vt, const bf16x8_t* vfirst, int nfirst = S::NO) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < S::NO; ++c) {
#pragma unroll
      for (int hh = 0; hh < kKH; ++hh) {
        const bf16x8_t v = (hh == 0 && vfirst && c < nfirst) ? vfirst[c] : read_v(vt, hh, c);
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) o[nt][c] = mfma32(pa[hh][nt], v, o[nt][c]);
      }
    }
    if constexpr (kMfmaSum) {
      const bf16x8_t ones = {(__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f,
                             (__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f};
#pragma unroll
      for (int hh = 0; hh < kKH; ++hh)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) l_run[nt] = mfma32(pa[hh][nt], ones, l_run[nt]);
    }
  };

  // Online softmax of the step at tb: mask sc, form pa, re-base o and l_run.
  // A step whose keys every valid query row of this wave sees (below the
  // causal diagonal, inside the window) needs no per-element mask. Without
  // softcap the scale folds into the exponent: masked scores become -inf in
  // place (the same registers on both paths), the row maximum is taken on raw
  // scores (scale > 0), and p = exp2(fma(s, scale, -max)).
  auto softmax = [&](int tb) __attribute__((always_inline)) {
    const bool full = !SOFTCAP && tb + kKeys - 1 <= wave_pos_min && tb >= wave_left_max;
    // Mask, and each tile's row maximum over this lane's 4 kKG scores.
    float mx[kNT];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      if constexpr (SOFTCAP) {
#pragma unroll
        for (int h = 0; h < kKG; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = tb + 16 * h + 4 * q + r;
            const float sv = a.softcap_log2 * soft_tanh(sc[h][nt][r] * a.score_scale);
            sc[h][nt][r] = (key <= qpos[nt] && key >= qleft[nt]) ? sv : -INFINITY;
          }
      } else if (!full) {
#pragma unroll
        for (int h = 0; h < kKG; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = tb + 16 * h + 4 * q + r;
            sc[h][nt][r] = (key <= qpos[nt] && key >= qleft[nt]) ? sc[h][nt][r] : -INFINITY;
          }
      }
      float t[4 * kKG];
#pragma unroll
      for (int i = 0; i < 4 * kKG; ++i) t[i] = sc[i >> 2][nt][i & 3];
      mx[nt] = tree_max(t);  // log2 units with softcap, raw scores without
    }
    // The probabilities of both tiles are formed right away against the
    // running maxima, before the cross-lane reduction of the steps' maxima,
    // which only decides afterwards whether a (rare) re-base is due; that
    // recomputes them against the new maximum. Same values as re-basing
    // first. Empty asm uses keep them above the re-base branch, which the
    // compiler would otherwise sink them into, behind the reduction (C4 shapes
    // at head_dim 64: 107.2 -> 105.4 us). One branch serves both tiles, so the
    // common path of a step is one basic block (head_dim 128: 156.3 ->
    // 154.9 us against a branch per tile).
    auto probabilities = [&](int nt, float base) __attribute__((always_inline)) {
      float ps[4 * kKG];
#pragma unroll
      for (int i = 0; i < 4 * kKG; ++i) {
        if constexpr (SOFTCAP) ps[i] = fast_exp2(sc[i >> 2][nt][i & 3] - base);
        else ps[i] = fast_exp2(__builtin_fmaf(sc[i >> 2][nt][i & 3], a.score_scale, -base));
      }
#pragma unroll
      for (int i = 0; i < 4 * kKG; ++i) pa[i >> 3][nt][i & 7] = (__bf16)ps[i];
      if constexpr (!kMfmaSum) {
        float l = 0.f;
#pragma unroll
        for (int i = 0; i < 4 * kKG; ++i) l += ps[i];
        return l;
      }
      return 0.f;
    };
    float lsum[kNT];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      lsum[nt] = probabilities(nt, m_base[nt]);
#pragma unroll
      for (int hh = 0; hh < kKH; ++hh) {
        const auto w = __builtin_bit_cast(u32x4_t, pa[hh][nt]);
        asm volatile("" ::"v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]));
      }
    }
#pragma unroll
    for (int nt = 0; nt + 1 < kNT; nt += 2) col4_max2(mx[nt], mx[nt + 1]);
    if constexpr (kNT % 2) mx[kNT - 1] = col4_max(mx[kNT - 1]);
    bool any = false;
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) any = any || (mx[nt] > (SOFTCAP ? m_run[nt] + kLazyRescale : m_thr[nt]));
    if (__builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        if (!__builtin_amdgcn_ballot_w64(mx[nt] > (SOFTCAP ? m_run[nt] + kLazyRescale : m_thr[nt]))) continue;
        const float m_new = fmaxf(m_run[nt], SOFTCAP ? mx[nt] : mx[nt] * a.score_scale);
        const float alpha = m_run[nt] == -INFINITY ? 0.f : fast_exp2(m_run[nt] - m_new);
        m_run[nt] = m_new;
        m_thr[nt] = (m_new + kLazyRescale) * inv_scale;
        m_base[nt] = m_new == -INFINITY ? 0.f : m_new;
        if constexpr (!kMfmaSum) l_run[nt][0] *= alpha;
        // o rows are qrows 4q + r; qrow h's factor lives in lanes with c16 == h.
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float f = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * q + r) << 2, __float_as_int(alpha)));
#pragma unroll
          for (int c = 0; c < S::NO; ++c) o[nt][c][r] *= f;
          if constexpr (kMfmaSum) l_run[nt][r] *= f;
        }
        lsum[nt] = probabilities(nt, m_base[nt]);
      }
    }
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
      if constexpr (!kMfmaSum) l_run[nt][0] += lsum[nt];
  };

  static_assert(kStages == 2, "K and V alternate between two stages");
  if constexpr (kLag) {
    // K stages at lds + s TILE (s = step % 2), V stages after them
    // (step % 3). One barrier per step, as below: after it every wave's loads
    // of step i have landed and every wave has finished with K(i - 1) and
    // V(i - 2), whose stages take step i + 1's loads. The second half's
    // P.V(i - 1) reads V(i - 1), which stays until the barrier of step i + 1.
    const bool lead = wave < kPrefillWaves / 2;
    char* const vstages = lds + 2 * S::TILE;
    Entries e_next{};
    {
      const Offsets first = offsets_of(kb0, entry_of(kb0));
      issue(first, krs, lds);
      issue(first, vrs, vstages);
    }
    if (1 < nsteps) e_next = entry_of(kb0 + kKeys);
    int vs = 0;  // V stage of the current step
    // One loop per half (a single loop with both orders keeps both orders'
    // registers live); LEAD selects the order at compile time.
    auto body = [&](int step, auto stage, auto lead_t) __attribute__((always_inline)) {
      constexpr int cur = decltype(stage)::value, next = cur ^ 1;
      constexpr bool LEAD = decltype(lead_t)::value;
      const int tb = kb0 + step * kKeys;
      const int vnext = vs == 2 ? 0 : vs + 1, vprev = vs == 0 ? 2 : vs - 1;
      wait_vmem<0>();
      __syncthreads();
      wait_vmem_visible();
      if (step + 1 < nsteps) {
        const Offsets of = offsets_of(tb + kKeys, e_next);
        issue(of, krs, lds + next * S::TILE);
        issue(of, vrs, vstages + vnext * S::TILE);
        if (step + 2 < nsteps) e_next = entry_of(tb + 2 * kKeys);
      }
      scores(lds + cur * S::TILE);
      if constexpr (LEAD) {
        const char* vt = vstages + vs * S::TILE;
        bf16x8_t vfirst[S::NO];
#pragma unroll
        for (int c = 0; c < S::NO; ++c) vfirst[c] = read_v(vt, 0, c);
        softmax(tb);
        accumulate(vt, vfirst);
      } else {
        if (step > 0) accumulate(vstages + vprev * S::TILE, nullptr);
        softmax(tb);
      }
      vs = vnext;
    };
    auto run = [&](auto lead_t) __attribute__((always_inline)) {
      int step = 0;
      for (; step + 1 < nsteps; step += 2) {
        body(step, std::integral_constant<int, 0>{}, lead_t);
        body(step + 1, std::integral_constant<int, 1>{}, lead_t);
      }
      if (step < nsteps) body(step, std::integral_constant<int, 0>{}, lead_t);
    };
    if (lead) {
      run(std::true_type{});
    } else {
      run(std::false_type{});
      // P.V of the last step (its V stage is never refilled).
      accumulate(vstages + (vs == 0 ? 2 : vs - 1) * S::TILE, nullptr);
    }
  } else if constexpr (kPipe) {
    // Iteration i (0 <= i <= nsteps), after the step's barrier:
    //   loads  K(i + 1) -> K stage (i + 1) % 2 and V(i) -> V stage i % 2 (both
    //          last read in iteration i - 1);
    //   A      S(i) = K(i) . Q^T, interleaved with P(i - 1) = exp2(S(i - 1)
    //          scale - base) (independent instructions of one wave);
    //   mask   S(i), on steps that cross the diagonal or the window;
    //   B      O += P(i - 1) . V(i - 1), interleaved with the row maxima of S(i);
    //   re-base (rare) after B, so P(i - 1) keeps the base it was formed
    //          against and P(i) is formed against the new one.
    // The same operations on o and l_run in the same order as the loop below.
    f32x4_t sp[2][kKG][kNT];
    Offsets off_v = offsets_of(kb0, entry_of(kb0));  // offsets of the step whose V is issued next
    issue(off_v, krs, kv[0][0]);
    Entries e_next{};
    if (1 < nsteps) e_next = entry_of(kb0 + kKeys);

    auto qk = [&](const char* kt, f32x4_t(&dst)[kKG][kNT]) __attribute__((always_inline)) {
#pragma unroll
      for (int h = 0; h < kKG; ++h) {
        const int tt = 16 * h + c16;
        bf16x8_t kr[S::NC];
#pragma unroll
        for (int c = 0; c < S::NC; ++c)
          kr[c] = *reinterpret_cast<const bf16x8_t*>(kt + tt * (2 * D) + (((4 * c + q) ^ swz(tt, D / 8)) << 4));
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
          dst[h][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < S::NC; ++c) dst[h][nt] = mfma32(kr[c], qb[nt][c], dst[h][nt]);
        }
      }
    };
    auto probs = [&](const f32x4_t(&src)[kKG][kNT]) __attribute__((always_inline)) {
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
        for (int i = 0; i < 4 * kKG; ++i)
          pa[i >> 3][nt][i & 7] = (__bf16)fast_exp2(__builtin_fmaf(src[i >> 2][nt][i & 3], a.score_scale, -m_base[nt]));
    };
    auto mask = [&](int tb, f32x4_t(&s)[kKG][kNT]) __attribute__((always_inline)) {
      const bool full = tb + kKeys - 1 <= wave_pos_min && tb >= wave_left_max;
      if (!full) {
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
          for (int h = 0; h < kKG; ++h)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int key = tb + 16 * h + 4 * q + r;
              s[h][nt][r] = (key <= qpos[nt] && key >= qleft[nt]) ? s[h][nt][r] : -INFINITY;
            }
      }
    };
    auto row_max = [&](const f32x4_t(&s)[kKG][kNT], float(&mx)[kNT]) __attribute__((always_inline)) {
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        float t[4 * kKG];
#pragma unroll
        for (int i = 0; i < 4 * kKG; ++i) t[i] = s[i >> 2][nt][i & 3];
        mx[nt] = tree_max(t);
      }
      static_assert(kNT == 2, "one pair of tiles");
      col4_max2(mx[0], mx[1]);
    };
    auto rebase = [&](const float(&mx)[kNT]) __attribute__((always_inline)) {
      bool any = false;
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) any = any || mx[nt] > m_thr[nt];
      if (!__builtin_amdgcn_ballot_w64(any)) return;
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        if (!__builtin_amdgcn_ballot_w64(mx[nt] > m_thr[nt])) continue;
        const float m_new = fmaxf(m_run[nt], mx[nt] * a.score_scale);
        const float alpha = m_run[nt] == -INFINITY ? 0.f : fast_exp2(m_run[nt] - m_new);
        m_run[nt] = m_new;
        m_thr[nt] = (m_new + kLazyRescale) * inv_scale;
        m_base[nt] = m_new == -INFINITY ? 0.f : m_new;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float f = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * q + r) << 2, __float_as_int(alpha)));
#pragma unroll
          for (int c = 0; c < S::NO; ++c) o[nt][c][r] *= f;
          l_run[nt][r] *= f;
        }
      }
    };
    // Barrier and loads of iteration i.
    auto top = [&](int i, auto stage) __attribute__((always_inline)) {
      constexpr int cur = decltype(stage)::value, next = cur ^ 1;
      const int tb = kb0 + i * kKeys;
      wait_vmem<0>();
      __syncthreads();
      wait_vmem_visible();  // as in the loop below
      if (i + 1 < nsteps) {
        const Offsets of = offsets_of(tb + kKeys, e_next);
        issue(of, krs, kv[next][0]);
        issue(off_v, vrs, kv[cur][1]);
        off_v = of;
        if (i + 2 < nsteps) e_next = entry_of(tb + 2 * kKeys);
      } else if (i < nsteps) {
        issue(off_v, vrs, kv[cur][1]);
      }
    };
    // Instruction order of the two phases: one MFMA, then independent VALU
    // work, with each group's LDS operand reads issued a group ahead.
    auto order_a = [&]() __attribute__((always_inline)) {
#if GK_PREFILL_PIPE_ORDER
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int h = 0; h < kKG; ++h) {
#pragma unroll
        for (int k = 0; k < 2 * kNT; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x402, 3, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x402, 2, 0);
        }
        if (h + 2 < kKG) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      }
#endif
    };
    auto order_b = [&]() __attribute__((always_inline)) {
#if GK_PREFILL_PIPE_ORDER
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);
#pragma unroll
      for (int c = 0; c < S::NO; ++c) {
#pragma unroll
        for (int k = 0; k < 2 * kNT; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
          __builtin_amdgcn_sched_group_barrier(0x402, 1, 1);
        }
        if (c + 2 < S::NO) __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kNT * kKH, 1);
#endif
    };
    // Empty asm uses of the probabilities at the end of phase A: the compiler
    // would otherwise sink their computation to P.V, past the mask branch.
    auto anchor_pa = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int hh = 0; hh < kKH; ++hh)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
          const auto w = __builtin_bit_cast(u32x4_t, pa[hh][nt]);
          asm volatile("" ::"v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]));
        }
    };
    auto steady = [&](int i, auto stage) __attribute__((always_inline)) {
      constexpr int cur = decltype(stage)::value, prev = cur ^ 1;
      top(i, stage);
      qk(kv[cur][0], sp[cur]);
      probs(sp[prev]);
      order_a();
      anchor_pa();
      mask(kb0 + i * kKeys, sp[cur]);
      float mx[kNT];
      row_max(sp[cur], mx);
      accumulate(kv[prev][1], nullptr);
      order_b();
      rebase(mx);
    };
    auto last = [&](int i, auto stage) __attribute__((always_inline)) {
      constexpr int prev = decltype(stage)::value ^ 1;
      top(i, stage);
      probs(sp[prev]);
      accumulate(kv[prev][1], nullptr);
    };
    using Zero = std::integral_constant<int, 0>;
    using One = std::integral_constant<int, 1>;
    {
      top(0, Zero{});
      qk(kv[0][0], sp[0]);
      mask(kb0, sp[0]);
      float mx[kNT];
      row_max(sp[0], mx);
      rebase(mx);
    }
    int i = 1;
    for (; i + 1 < nsteps; i += 2) {
      steady(i, One{});
      steady(i + 1, Zero{});
    }
    if (i < nsteps) {
      steady(i, One{});
      last(i + 1, Zero{});
    } else {
      last(i, One{});
    }
  } else if constexpr (!kPingPong) {
    // One barrier per step: before it each wave waits for its own loads of
    // the current stage; after it every wave's loads of the stage have landed
    // and every wave has finished the previous step, whose stage is refilled
    // with the next step. The first half's V operands are read before the
    // softmax, their LDS latency behind its arithmetic.
    Entries e_next{};
    {
      const Offsets first = offsets_of(kb0, entry_of(kb0));
      issue(first, krs, kv[0][0]);
      issue(first, vrs, kv[0][1]);
    }
    if (1 < nsteps) e_next = entry_of(kb0 + kKeys);
    // The loop is unrolled over the two stages, so that every LDS address of a
    // step is a per-lane offset plus an immediate (stage, 16-key group, half):
    // ~44 fewer VALU instructions per wave and step (C4: 148.6 -> 138.0 us).
    // The lambdas are forced inline (with three call sites the compiler made
    // the softmax a real call with a stack frame) and the buffer resources go
    // to the direct-load asm as scalar words (make_rsrc).
    auto body = [&](int step, auto stage) __attribute__((always_inline)) {
      constexpr int cur = decltype(stage)::value, next = cur ^ 1;
      const int tb = kb0 + step * kKeys;
      wait_vmem<0>();
      __syncthreads();
      // Every load of this wave has landed; tell the compiler. Its wait-count
      // model does not see the asm direct loads or waits, so it still counts
      // the query loads before the loop (and, with per-lane entries, the entry
      // loads) as outstanding, and would put an s_waitcnt vmcnt(0) before
      // their first use in the step: after this step's direct loads, which it
      // would then wait for (C4: 185.2 -> 183.9 us).
      wait_vmem_visible();
      if (step + 1 < nsteps) {
        const Offsets of = offsets_of(tb + kKeys, e_next);
        issue(of, krs, kv[next][0]);
        issue(of, vrs, kv[next][1]);
        if (step + 2 < nsteps) e_next = entry_of(tb + 2 * kKeys);
      }
      scores(kv[cur][0]);
      if constexpr (D <= 128) {
        bf16x8_t vfirst[S::NO];
#pragma unroll
        for (int c = 0; c < S::NO; ++c) vfirst[c] = read_v(kv[cur][1], 0, c);
        softmax(tb);
        accumulate(kv[cur][1], vfirst);
      } else {
        // head_dim 256: half the V operands are read early (32 VGPRs; C4's
        // shapes at head_dim 256, same box: none 162.7-164.2 us, a quarter
        // 160.5-162.8, half 158.2-158.7, all 164.9-166.0).
        constexpr int NF = S::NO / 2;
        bf16x8_t vfirst[NF];
#pragma unroll
        for (int c = 0; c < NF; ++c) vfirst[c] = read_v(kv[cur][1], 0, c);
        softmax(tb);
        accumulate(kv[cur][1], vfirst, NF);
      }
    };
    int step = 0;
    for (; step + 1 < nsteps; step += 2) {
      body(step, std::integral_constant<int, 0>{});
      body(step + 1, std::integral_constant<int, 1>{});
    }
    if (step < nsteps) body(step, std::integral_constant<int, 0>{});
  } else {
    // Two groups of waves, one wave of each on every SIMD (waves w and w + 4
    // share a SIMD), take turns between the matrix cores and the vector ALU.
    // A wave's work per step is an MFMA phase M(i) (scores of step i, then
    // P.V of step i - 1) and a VALU phase S(i) (the softmax of step i), run as
    // M(0) S(0) M(1) S(1) ... M(n) with a barrier after each phase. The
    // second group passes one barrier before its first phase and the first
    // group one after its last, so the second runs every phase one barrier
    // interval later: between two barriers one wave of each SIMD is in an
    // MFMA phase while the other is in a softmax phase.
    //
    // LDS: a wave's iteration i reads K(i) (stage i % 2) and V(i - 1) (stage
    // (i - 1) % 2). At its start each wave issues its share of the direct
    // loads of K(i + 1) and V(i), into the stages that both groups last read
    // in iteration i - 1, and waits for them before the barrier that ends
    // interval 2i + 1 (the first group's second barrier of the iteration, the
    // second group's first), after which the first group reads them.
    const bool lead = wave < kPrefillWaves / 2;
    Entries e_next = entry_of(kb0);
    Offsets off_v = offsets_of(kb0, e_next);  // offsets of the step whose V is issued next
    issue(off_v, krs, kv[0][0]);
    if (1 < nsteps) e_next = entry_of(kb0 + kKeys);
    wait_vmem<0>();
    __syncthreads();
    wait_vmem_visible();  // as in the other loop: the query (and entry) loads have landed
    if (!lead) __syncthreads();
    for (int i = 0; i <= nsteps; ++i) {
      const int tb = kb0 + i * kKeys;
      if (i + 1 < nsteps) {
        const Offsets off_k = offsets_of(tb + kKeys, e_next);
        issue(off_k, krs, kv[(i + 1) & 1][0]);
        issue(off_v, vrs, kv[i & 1][1]);
        off_v = off_k;
        if (i + 2 < nsteps) e_next = entry_of(tb + 2 * kKeys);
      } else if (i + 1 == nsteps) {
        issue(off_v, vrs, kv[i & 1][1]);
      }
      if (i < nsteps) scores(kv[i & 1][0]);
      if (i > 0) accumulate(kv[(i - 1) & 1][1], nullptr);
      if (!lead) wait_vmem<0>();
      __syncthreads();
      if (i < nsteps) softmax(tb);
      if (lead) wait_vmem<0>();
      __syncthreads();
      wait_vmem_visible();
    }
    if (lead) __syncthreads();
  }

  // Normalise into bf16 rows in LDS: o row 4q + r of tile nt, its sum in
  // l_run[nt][r] (MFMA sums) or in lane c16 == 4q + r after the cross-row sum
  // (VALU sums). Then each wave stores its own rows as 16-byte pieces: the
  // wave's LDS operations complete in order, so it reads back what it wrote.
  // (Stored straight from the MFMA layout, a lane's values are 2-byte
  // elements 32 bytes apart: 64 narrow stores per lane.)
  char* rows_lds = lds + kKvBytes + wave * kQrowsPerWave * kOutRowBytes;
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt) {
    float l = 0.f;
    if constexpr (!kMfmaSum) l = col4_sum(l_run[nt][0]);
    // The hardware reciprocal (within one fp32 ulp, far below the bf16
    // rounding that follows) instead of a full division; every row sum is at
    // least 1 (the row's maximum contributes at least 1).
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float lr = kMfmaSum ? l_run[nt][r]
                                : __int_as_float(__builtin_amdgcn_ds_bpermute((4 * q + r) << 2, __float_as_int(l)));
      const float inv = lr > 0.f ? __builtin_amdgcn_rcpf(lr) : 0.f;
      __bf16* dst = reinterpret_cast<__bf16*>(rows_lds + (nt * 16 + 4 * q + r) * kOutRowBytes) + c16;
#pragma unroll
      for (int c = 0; c < S::NO; ++c) dst[16 * c] = (__bf16)(o[nt][c][r] * inv);
    }
  }
  constexpr int kPieces = kQrowsPerWave * D / 8;  // 16-byte pieces of the wave's rows
  static_assert(kPieces % 64 == 0, "whole pieces per lane");
#pragma unroll
  for (int i = 0; i < kPieces / 64; ++i) {
    const int piece = i * 64 + lane, ql = piece / (D / 8), part = piece % (D / 8);
    const int qr = wave * kQrowsPerWave + ql;
    const int row = div_group(qr), head = qr - row * g;
    const uint4 v = *reinterpret_cast<const uint4*>(rows_lds + ql * kOutRowBytes + part * 16);
    if (row < nr)
      *reinterpret_cast<uint4*>(a.out + (int64_t)(first_row + row) * a.out_stride + (int64_t)(kvh * g + head) * D +
                                part * 8) = v;
  }
}

// ---------------------------------------------------------------------------
// head_dim 128 on 32 x 32 tiles (v_mfma_f32_32x32x16_bf16)
// ---------------------------------------------------------------------------
// An opt-in build variant (GK_PREFILL_MFMA32=1), not the shipping form: on C4
// it ran 147.5 us against 135.5 us for prefill_kernel (same box). Its
// counters show less of every instruction class but 52% more wave-cycles
// waiting: with one 32-row tile per wave each K operand read feeds a single
// 32-cycle MFMA, and at ~250 VGPRs (two waves per SIMD) the compiler cannot
// keep reads in flight ahead of their MFMAs. The same work item, pipeline
// and numerics as prefill_kernel, with each wave's 32 query rows as one
// 32-column tile:
//   S^T[key][qrow] = K . Q^T      per 32-key group, 8 MFMAs over 16-dim chunks
//   O^T[dim][qrow] += V^T . P^T   per 32-dim block, 4 MFMAs over 16-key chunks
// Output lane l holds column l % 32 of both products: all 32 scores of one
// step and all 64 accumulator values of the lane's query row (half the keys
// and dims; lane l + 32 holds the rest of the same row). The probabilities are
// the B operand of P.V straight from the score registers, re-basing scales a
// lane's own registers, and a row's maximum and sum combine the two halves
// with one 32-lane swap. Against 16 x 16 tiles: half the MFMA issues per step,
// no cross-lane moves of the re-base factors, and the row sums on the VALU
// (v_dot2 of the bf16 probabilities with ones) instead of four MFMAs.
//
// Lane layouts of v_mfma_f32_32x32x16_bf16 (checked on the GPU with an
// in-bounds probe): A row l % 32 and B column l % 32 hold k slots
// 8 (l / 32) .. + 7; D register r of lane l is row 8 (r / 4) + 4 (l / 32) +
// r % 4, column l % 32.
//
// LDS token swizzle swz32 (16-byte chunk c of token t stored at c ^ swz32(t)):
//  - K operand reads (ds_read_b128, 32 lanes at a time over 128 banks, two
//    256-byte rows per bank row): the 32 tokens of a key group read one
//    logical chunk, so swz32 must be a bijection of bits 1-4 of t for each t0;
//  - V^T reads (ds_read_b64_tr_b16, 32 lanes over 64 banks): 4 consecutive
//    tokens (aligned) x an aligned group of 4 chunks, so bits 2-3 of swz32 must
//    be a bijection of (t0, t1).
// swz32 = t1 << 3 | (t0 ^ t2) << 2 | t3 << 1 | t4 meets both.
__device__ __forceinline__ int swz32(int t) {
  return ((t & 2) << 2) | (((t ^ (t >> 2)) & 1) << 2) | ((t & 8) >> 2) | ((t >> 4) & 1);
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16_t mfma32x32(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

template <bool SOFTCAP, int MODE>
__global__ __launch_bounds__(kPrefillWaves * 64, 1) void prefill32_kernel(PrefillArgs a) {
  constexpr int D = 128;
  using S = PrefillShape<D>;
  constexpr int kKeys = 64;        // keys per step: two 32-key groups
  constexpr int NC = D / 16;       // 16-dim k chunks of Q.K
  constexpr int NB = D / 32;       // 32-dim blocks of P.V
  constexpr int KC = kKeys / 16;   // 16-key k chunks of P.V
  static_assert(S::TILE == kKeys * D * 2, "tile of a 64-key step");
  constexpr int LPW = (S::NI + kPrefillWaves - 1) / kPrefillWaves;
  constexpr int NE = MODE == kStepBlocks ? 1 : LPW;
  constexpr int KPL = kKeys / S::NI;
  constexpr bool CLAMPED = MODE != kStepBlocks;
  constexpr int kOutRowBytes = 2 * D + 16;
  constexpr int kKvBytes = 2 * 2 * S::TILE, kOutBytes = kPrefillWaves * kQrowsPerWave * kOutRowBytes;
  static_assert(kQrowsPerWave == 32, "one 32-column tile per wave");
  __shared__ __attribute__((aligned(16))) char lds[kKvBytes + kOutBytes];
  auto kv = reinterpret_cast<char(*)[2][S::TILE]>(lds);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hf = lane >> 5, col = lane & 31;  // half (k slots / output rows) and column of the 32 x 32 tiles
  // Work item and prologue: as prefill_kernel.
  asm volatile("" ::"s"(a.seq_rows), "s"(a.seq_prefix), "s"(a.seq_first_row), "s"(a.seq_request),
               "s"(a.block_tables), "s"(a.query), "s"(a.pool), "s"(a.out), "s"(a.tiles), "s"(a.seqs),
               "s"(a.rows_per_tile), "s"(a.group), "s"(a.bt_stride), "s"(a.block_shift), "s"(a.window),
               "s"(a.q_stride), "s"(a.slots), "s"(a.kv_heads), "s"(gridDim.x), "s"(a.tiles_div.mul),
               "s"(a.tiles_div.shift), "s"(a.seqs_div.mul), "s"(a.seqs_div.shift), "s"(a.group_div.mul),
               "s"(a.group_div.shift));
  const int nitems = gridDim.x, xcd = blockIdx.x % kXcds, per_xcd = nitems / kXcds, extra = nitems % kXcds;
  const auto div_tiles = [&](int x) { return (int)fast_div((uint32_t)x, a.tiles_div); };
  const auto div_group = [&](int x) { return (int)fast_div((uint32_t)x, a.group_div); };
  const int item = heavy_first_item(xcd * per_xcd + min(xcd, extra), per_xcd + (xcd < extra), a.tiles,
                                    (int)blockIdx.x / kXcds, div_tiles);
  const int item_seq = div_tiles(item), tile = item - item_seq * a.tiles;
  const int kvh = (int)fast_div((uint32_t)item_seq, a.seqs_div), seq = item_seq - kvh * a.seqs;
  const int rows = a.seq_rows[seq], prefix = a.seq_prefix[seq], seq_first = a.seq_first_row[seq];
  const int request = a.seq_request[seq];
  asm volatile("" ::"s"(rows), "s"(prefix), "s"(seq_first), "s"(request));
  const int r0 = tile * a.rows_per_tile;
  if (r0 >= rows) return;
  const int nr = min(a.rows_per_tile, rows - r0);
  const int first_row = seq_first + r0;
  const int32_t* __restrict__ bt = a.block_tables + (int64_t)request * a.bt_stride;
  const int g = a.group;
  const int pos_lo = prefix + r0, pos_hi = prefix + r0 + nr - 1;
  const int key_end = pos_hi + 1;
  const int key_begin = a.window > 0 ? max(0, pos_lo - a.window + 1) : 0;
  const int kb0 = key_begin & ~(kKeys - 1);
  const int nsteps = (key_end - kb0 + kKeys - 1) / kKeys;

  // This lane's query row qrow = (row, head), column `col` of the wave's tile.
  const int qr = wave * kQrowsPerWave + col;
  const int qrow_row = div_group(qr), qrow_head = qr - qrow_row * g;
  const bool qvalid = qrow_row < nr;
  const int qpos = qvalid ? pos_lo + qrow_row : -1;
  const int qleft = a.window > 0 ? qpos - a.window + 1 : 0;
  // Q^T as the B operand of S^T = K . Q^T: k chunk c holds dims 16 c + 8 hf .. + 7.
  bf16x8_t qb[NC];
  {
    const uint16_t* src =
        a.query + (int64_t)(first_row + qrow_row) * a.q_stride + (int64_t)(kvh * g + qrow_head) * D + 8 * hf;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (qvalid) v = load16(src + 16 * c);
      qb[c] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  const int wave_pos_min = pos_lo + div_group(wave * kQrowsPerWave);
  const int wave_left_max =
      a.window > 0 ? pos_lo + min(nr - 1, div_group(wave * kQrowsPerWave + kQrowsPerWave - 1)) - a.window + 1 : 0;

  f32x16_t o[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) o[b] = f32x16_t{};
  // Running maximum (log2 units), its re-base threshold on raw scores, the
  // probability base (m_run, or 0 before the first maximum) and this lane's
  // share of the row sum (its half of the keys).
  float m_run = -INFINITY, m_thr = -INFINITY, m_base = 0.f, l_run = 0.f;
  const float inv_scale = 1.f / a.score_scale;

  const uint16_t* kbase = a.pool + (int64_t)kvh * a.slots * D;
  const uint16_t* vbase = kbase + (int64_t)a.kv_heads * a.slots * D;
  const uint32_t region = (uint32_t)(a.slots * D * 2);
  const u32x4_t krs = buffer_words(kbase, region), vrs = buffer_words(vbase, region);
  const int shift = a.block_shift, bmask = (1 << shift) - 1;

  struct Entries {
    int e[NE];
  };
  auto entry_of = [&](int tb) __attribute__((always_inline)) {
    Entries en;
#pragma unroll
    for (int k = 0; k < NE; ++k) {
      int key = tb;
      if constexpr (MODE == kLoadBlocks) key += (wave + k * kPrefillWaves) * KPL;
      if constexpr (MODE == kKeyBlocks) key += (wave + k * kPrefillWaves) * KPL + lane / S::CPR;
      if constexpr (CLAMPED) key = min(max(key, key_begin), key_end - 1);
      if constexpr (MODE == kKeyBlocks) en.e[k] = bt[key >> shift];
      else en.e[k] = scalar_load(bt, key >> shift);
    }
    return en;
  };
  // Direct-load offsets as in prefill_kernel, with the swz32 token swizzle.
  struct Offsets {
    uint32_t v[LPW];
  };
  auto offsets_of = [&](int tb, const Entries& en) __attribute__((always_inline)) {
    Offsets of{};
    const int lo = key_begin - tb, hi = key_end - 1 - tb;
    const uint32_t step_slot = ((uint32_t)en.e[0] << shift) + (uint32_t)(tb & bmask);
#pragma unroll
    for (int k = 0; k < LPW; ++k) {
      const int ins = wave + k * kPrefillWaves;
      if (S::NI % kPrefillWaves != 0 && ins >= S::NI) break;
      const int p = ins * 64 + lane, tt = p / S::CPR, pc = p % S::CPR;
      uint32_t slot;
      if constexpr (MODE == kStepBlocks) {
        slot = step_slot + (uint32_t)min(max(tt, lo), hi);
      } else {
        const int key = min(max(tb + tt, key_begin), key_end - 1);
        slot = (uint32_t)((en.e[k] << shift) | (key & bmask));
      }
      of.v[k] = slot * (2 * D) + ((pc ^ swz32(tt)) << 4);
    }
    return of;
  };
  auto issue = [&](const Offsets& of, u32x4_t rs, char* t) __attribute__((always_inline)) {
    if constexpr (MODE == kKeyBlocks) wait_vmem_visible();
    const uint32_t base = lds_addr(t);
#pragma unroll
    for (int k = 0; k < LPW; ++k) {
      const int ins = wave + k * kPrefillWaves;
      if (S::NI % kPrefillWaves != 0 && ins >= S::NI) break;
      lds_dma16_w(base + ins * 1024, rs, of.v[k]);
    }
  };

  f32x16_t sc[2];        // scores of the step's two key groups
  bf16x8_t pa[KC];       // probabilities: B operand of k chunk kc (keys 16 kc .. + 15)

  // S^T = K . Q^T: group kg's scores in sc[kg]; lane (hf, col) reads token
  // 32 kg + col, logical chunk 2 c + hf.
#ifndef GK_PREFILL32_AHEAD
#define GK_PREFILL32_AHEAD 0
#endif
  // With GK_PREFILL32_AHEAD = n > 0 the two key groups' chains alternate and
  // each chunk's K operands are read n chunks ahead, fenced with full
  // scheduling barriers so the scheduler cannot move the reads back next to
  // their MFMAs (the wait-count pass then waits only for the older chunk).
  auto scores = [&](const char* kt) __attribute__((always_inline)) {
    if constexpr (GK_PREFILL32_AHEAD == 0) {
#pragma unroll
      for (int kg = 0; kg < 2; ++kg) {
        sc[kg] = f32x16_t{};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const bf16x8_t kr = *reinterpret_cast<const bf16x8_t*>(kt + (32 * kg + col) * (2 * D) +
                                                                (((2 * c + hf) ^ swz32(col)) << 4));
          sc[kg] = mfma32x32(kr, qb[c], sc[kg]);
        }
      }
    } else {
      constexpr int A = GK_PREFILL32_AHEAD;
      auto kread = [&](int kg, int c) __attribute__((always_inline)) {
        return *reinterpret_cast<const bf16x8_t*>(kt + (32 * kg + col) * (2 * D) + (((2 * c + hf) ^ swz32(col)) << 4));
      };
      bf16x8_t kr[A + 1][2];
#pragma unroll
      for (int c = 0; c < A; ++c) {
        kr[c][0] = kread(0, c);
        kr[c][1] = kread(1, c);
      }
      sc[0] = sc[1] = f32x16_t{};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (c + A < NC) {
          kr[(c + A) % (A + 1)][0] = kread(0, c + A);
          kr[(c + A) % (A + 1)][1] = kread(1, c + A);
        }
        __builtin_amdgcn_sched_barrier(0);
        sc[0] = mfma32x32(kr[c % (A + 1)][0], qb[c], sc[0]);
        sc[1] = mfma32x32(kr[c % (A + 1)][1], qb[c], sc[1]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // V^T operand of k chunk kc, dim block b: lane (hf, col) gets dim 32 b + col
  // at keys 16 kc + 4 hf + (0..3) and 16 kc + 8 + 4 hf + (0..3); each 16-lane
  // group reads 4 consecutive keys x 16 dims transposed.
  auto read_v = [&](const char* vt, int kc, int b) __attribute__((always_inline)) {
    const int i = lane & 15, gb = (lane >> 4) & 1;
    const int lc = 4 * b + 2 * gb + ((i & 3) >> 1);
    const int t0 = 16 * kc + 4 * hf + (i >> 2), t1 = t0 + 8;
    const bf16x4_t v0 = lds_read_tr4(vt + t0 * (2 * D) + ((lc ^ swz32(t0)) << 4) + ((i & 1) << 3));
    const bf16x4_t v1 = lds_read_tr4(vt + t1 * (2 * D) + ((lc ^ swz32(t1)) << 4) + ((i & 1) << 3));
    return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  // P.V; with GK_PREFILL32_AHEAD > 0 the next k chunk's V operands are read
  // before this chunk's MFMAs, fenced the same way.
  auto accumulate = [&](const char* vt, const bf16x8_t* vfirst) __attribute__((always_inline)) {
    if constexpr (GK_PREFILL32_AHEAD == 0) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const bf16x8_t v = (kc == 0 && vfirst) ? vfirst[b] : read_v(vt, kc, b);
          o[b] = mfma32x32(v, pa[kc], o[b]);
        }
    } else {
      bf16x8_t vv[2][NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) vv[0][b] = vfirst[b];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        if (kc + 1 < KC)
#pragma unroll
          for (int b = 0; b < NB; ++b) vv[(kc + 1) & 1][b] = read_v(vt, kc + 1, b);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < NB; ++b) o[b] = mfma32x32(vv[kc & 1][b], pa[kc], o[b]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // Online softmax of the step at tb. Score register r of group kg is key
  // tb + 32 kg + 8 (r / 4) + 4 hf + r % 4 of this lane's query row.
  auto softmax = [&](int tb) __attribute__((always_inline)) {
    const bool full = !SOFTCAP && tb + kKeys - 1 <= wave_pos_min && tb >= wave_left_max;
    if constexpr (SOFTCAP) {
#pragma unroll
      for (int kg = 0; kg < 2; ++kg)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = tb + 32 * kg + 8 * (r >> 2) + 4 * hf + (r & 3);
          const float sv = a.softcap_log2 * soft_tanh(sc[kg][r] * a.score_scale);
          sc[kg][r] = (key <= qpos && key >= qleft) ? sv : -INFINITY;
        }
    } else if (!full) {
#pragma unroll
      for (int kg = 0; kg < 2; ++kg)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = tb + 32 * kg + 8 * (r >> 2) + 4 * hf + (r & 3);
          sc[kg][r] = (key <= qpos && key >= qleft) ? sc[kg][r] : -INFINITY;
        }
    }
    float t[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) t[i] = sc[i >> 4][i & 15];
    float mx = tree_max(t);
    // Probabilities against the current base right away (as prefill_kernel);
    // the cross-half maximum only decides afterwards whether to re-base.
    auto probabilities = [&](float base) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        float ps;
        if constexpr (SOFTCAP) ps = fast_exp2(sc[i >> 4][i & 15] - base);
        else ps = fast_exp2(__builtin_fmaf(sc[i >> 4][i & 15], a.score_scale, -base));
        pa[i >> 3][i & 7] = (__bf16)ps;
      }
    };
    probabilities(m_base);
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const auto w = __builtin_bit_cast(u32x4_t, pa[kc]);
      asm volatile("" ::"v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]));
    }
    {
      const auto h2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = max2(__uint_as_float(h2[0]), __uint_as_float(h2[1]));
    }
    if (__builtin_amdgcn_ballot_w64(mx > (SOFTCAP ? m_run + kLazyRescale : m_thr))) {
      if (mx > (SOFTCAP ? m_run + kLazyRescale : m_thr)) {
        const float m_new = fmaxf(m_run, SOFTCAP ? mx : mx * a.score_scale);
        const float alpha = m_run == -INFINITY ? 0.f : fast_exp2(m_run - m_new);
        m_run = m_new;
        m_thr = (m_new + kLazyRescale) * inv_scale;
        m_base = m_new == -INFINITY ? 0.f : m_new;
        l_run *= alpha;
#pragma unroll
        for (int b = 0; b < NB; ++b) o[b] *= alpha;
      }
      probabilities(m_base);
    }
    // This lane's share of the row sum: the bf16 probabilities, in pairs.
    const bf16x2_t ones = {(__bf16)1.f, (__bf16)1.f};
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bf16x2_t pair = {pa[kc][2 * u], pa[kc][2 * u + 1]};
        l_run = __builtin_amdgcn_fdot2_f32_bf16(pair, ones, l_run, false);
      }
  };

  {
    Entries e_next{};
    {
      const Offsets first = offsets_of(kb0, entry_of(kb0));
      issue(first, krs, kv[0][0]);
      issue(first, vrs, kv[0][1]);
    }
    if (1 < nsteps) e_next = entry_of(kb0 + kKeys);
    auto body = [&](int step, auto stage) __attribute__((always_inline)) {
      constexpr int cur = decltype(stage)::value, next = cur ^ 1;
      const int tb = kb0 + step * kKeys;
      wait_vmem<0>();
      __syncthreads();
      wait_vmem_visible();
      if (step + 1 < nsteps) {
        const Offsets of = offsets_of(tb + kKeys, e_next);
        issue(of, krs, kv[next][0]);
        issue(of, vrs, kv[next][1]);
        if (step + 2 < nsteps) e_next = entry_of(tb + 2 * kKeys);
      }
      scores(kv[cur][0]);
      bf16x8_t vfirst[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) vfirst[b] = read_v(kv[cur][1], 0, b);
      softmax(tb);
      accumulate(kv[cur][1], vfirst);
    };
    int step = 0;
    for (; step + 1 < nsteps; step += 2) {
      body(step, std::integral_constant<int, 0>{});
      body(step + 1, std::integral_constant<int, 1>{});
    }
    if (step < nsteps) body(step, std::integral_constant<int, 0>{});
  }

  // Normalise: the row sum is this lane's share plus lane (col + 32)'s; the
  // lane's dims 32 b + 8 u + 4 hf + (0..3) go to its row in LDS as 8-byte
  // pieces, then each wave stores its rows as 16-byte pieces.
  {
    const auto h2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    const float l = __uint_as_float(h2[0]) + __uint_as_float(h2[1]);
    const float inv = l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f;
    char* row_lds = lds + kKvBytes + (wave * kQrowsPerWave + col) * kOutRowBytes;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        bf16x4_t w;
#pragma unroll
        for (int v = 0; v < 4; ++v) w[v] = (__bf16)(o[b][4 * u + v] * inv);
        *reinterpret_cast<bf16x4_t*>(row_lds + (32 * b + 8 * u + 4 * hf) * 2) = w;
      }
  }
  char* rows_lds = lds + kKvBytes + wave * kQrowsPerWave * kOutRowBytes;
  constexpr int kPieces = kQrowsPerWave * D / 8;
#pragma unroll
  for (int i = 0; i < kPieces / 64; ++i) {
    const int piece = i * 64 + lane, ql = piece / (D / 8), part = piece % (D / 8);
    const int qrr = wave * kQrowsPerWave + ql;
    const int row = div_group(qrr), head = qrr - row * g;
    const uint4 v = *reinterpret_cast<const uint4*>(rows_lds + ql * kOutRowBytes + part * 16);
    if (row < nr)
      *reinterpret_cast<uint4*>(a.out + (int64_t)(first_row + row) * a.out_stride + (int64_t)(kvh * g + head) * D +
                                part * 8) = v;
  }
}

// Head_dim 128 on 16 x 16 tiles with prefill_kernel (0, shipping) or on 32 x 32
// tiles with prefill32_kernel (1, a build variant kept for its measurement).
#ifndef GK_PREFILL_MFMA32
#define GK_PREFILL_MFMA32 0
#endif

template <int D, int MODE>
void launch_mode(const PrefillArgs& a, bool softcap, dim3 grid, hipStream_t stream) {
  if constexpr (D == 128 && GK_PREFILL_MFMA32) {
    if (softcap) prefill32_kernel<true, MODE><<<grid, kPrefillWaves * 64, 0, stream>>>(a);
    else prefill32_kernel<false, MODE><<<grid, kPrefillWaves * 64, 0, stream>>>(a);
  } else {
    if (softcap) prefill_kernel<D, true, MODE><<<grid, kPrefillWaves * 64, 0, stream>>>(a);
    else prefill_kernel<D, false, MODE><<<grid, kPrefillWaves * 64, 0, stream>>>(a);
  }
}

template <int D>
void launch(const PrefillArgs& a, bool softcap, int block_size, dim3 grid, hipStream_t stream) {
  constexpr int keys = prefill_keys<D>();
  if (block_size >= keys) launch_mode<D, kStepBlocks>(a, softcap, grid, stream);
  else if (block_size >= keys / PrefillShape<D>::NI) launch_mode<D, kLoadBlocks>(a, softcap, grid, stream);
  else launch_mode<D, kKeyBlocks>(a, softcap, grid, stream);
}

}  // namespace

int paged_prefill(const gk_prefill_params* p, hipStream_t stream) {
  if (!p) return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_prefill: null parameters");
  if (p->struct_size != sizeof(gk_prefill_params))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_prefill: struct_size does not match this library's gk_prefill_params");
  if (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256)
    return fail(GK_ERR_UNSUPPORTED, "gk_paged_prefill: head dimension must be 64, 128 or 256");
  if (p->q_heads <= 0 || p->kv_heads <= 0 || p->q_heads % p->kv_heads || p->q_heads / p->kv_heads > 128)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_prefill: invalid head geometry (GQA group at most 128)");
  if (!is_pow2(p->block_size) || p->block_size > (1 << 20))
    return fail(GK_ERR_UNSUPPORTED, "gk_paged_prefill: block_size must be a power of two of at most 2^20");
  if (p->seqs < 0 || p->seqs > 65535 || p->max_rows < 0 || p->slots <= 0)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_prefill: sequence count, rows or slots out of range");
  if (p->slots > (int64_t)(UINT32_MAX / 2) / p->head_dim)
    return fail(GK_ERR_UNSUPPORTED, "gk_paged_prefill: one kv head's K or V region must stay below 4 GiB");
  if (!(p->scale > 0.f) || !(p->scale < INFINITY) || !(p->softcap >= 0.f) || !(p->softcap < INFINITY))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_prefill: invalid scale or softcap");
  if (p->seqs == 0 || p->max_rows == 0) return GK_OK;
  if (!p->query || !p->pool || !p->block_tables || !p->seq_request || !p->seq_first_row || !p->seq_rows ||
      !p->seq_prefix || !p->out)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_prefill: null pointer");
  const auto misaligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) != 0; };
  if (misaligned(p->query) || misaligned(p->pool) || misaligned(p->out) || (p->q_row_stride & 7) ||
      (p->out_row_stride & 7) || p->q_row_stride < (int64_t)p->q_heads * p->head_dim ||
      p->out_row_stride < (int64_t)p->q_heads * p->head_dim)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_prefill: query/pool/out must be 16-byte aligned with full rows");
  PrefillArgs a{};
  a.query = static_cast<const uint16_t*>(p->query);
  a.q_stride = p->q_row_stride;
  a.pool = static_cast<const uint16_t*>(p->pool);
  a.slots = p->slots;
  a.block_tables = p->block_tables;
  a.bt_stride = p->bt_stride;
  a.block_shift = log2_int(p->block_size);
  a.seq_request = p->seq_request;
  a.seq_first_row = p->seq_first_row;
  a.seq_rows = p->seq_rows;
  a.seq_prefix = p->seq_prefix;
  a.q_heads = p->q_heads;
  a.kv_heads = p->kv_heads;
  a.group = p->q_heads / p->kv_heads;
  a.rows_per_tile = prefill_qrows(p->head_dim) / a.group;
  a.tiles = (p->max_rows + a.rows_per_tile - 1) / a.rows_per_tile;
  a.seqs = p->seqs;
  const bool softcap = p->softcap > 0.f;
  a.score_scale = softcap ? p->scale / p->softcap : p->scale * kLog2e;
  a.softcap_log2 = p->softcap * kLog2e;
  a.window = p->sliding_window > 0 ? p->sliding_window : 0;
  a.out = static_cast<uint16_t*>(p->out);
  a.out_stride = p->out_row_stride;
  a.tiles_div = div_magic((uint32_t)a.tiles);
  a.seqs_div = div_magic((uint32_t)a.seqs);
  a.group_div = div_magic((uint32_t)a.group);
  const int64_t items = (int64_t)a.tiles * p->kv_heads * p->seqs;
  if (items > (int64_t)1 << 30) return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_prefill: too many rows");
  const dim3 grid((unsigned)items);
  if (p->head_dim == 64) launch<64>(a, softcap, p->block_size, grid, stream);
  else if (p->head_dim == 128) launch<128>(a, softcap, p->block_size, grid, stream);
  else launch<256>(a, softcap, p->block_size, grid, stream);
  return hip_status(hipGetLastError(), "gk_paged_prefill launch");
}

}  // namespace gk

extern "C" int gk_paged_prefill(const gk_prefill_params* params, hipStream_t stream) {
  gk::clear_error();
  return gk::paged_prefill(params, stream);
}
