// Paged decode attention for gfx950: split-K partitions + log-sum-exp merge.
//
// Work decomposition. A work item is one (query row, kv head, head group,
// partition of `partition` keys). The query heads that share a kv head are
// computed together, so each K/V byte is read from HBM once per group. The
// partition's block-table entries are staged in LDS first, so no K/V load ever
// waits on another load (a block-table lookup is an LDS read).
//
// These kernels run when the caller fixes the partition (a row's output then
// depends on that row alone) or when a batch exceeds the balanced schedule's
// 32-bit numbering; otherwise decode_stream.hip's balanced schedule runs. Two
// kernels compute a partition:
//
//  * decode_mfma_kernel (GQA group >= 4, head_dim 64/128/256): one wave per
//    work item. The group's query heads are the 16 rows of bf16 MFMA tiles.
//    Scores are computed transposed, S^T[token][head] = K . Q^T with
//    v_mfma_f32_16x16x32_bf16, which leaves each lane holding one head's
//    scores for 8 tokens: exactly the A operand of the P.V MFMA, so
//    probabilities never move between lanes. K and V tiles go HBM -> LDS with
//    16-byte buffer->LDS loads (two stages), rows stored with their 16-byte
//    chunks XOR-swizzled by token; K is read back with ds_read_b128 as the A
//    operand of S^T, V transposed with ds_read_b64_tr_b16 as the B operand
//    [token][dim] of P.V.
//
//  * decode_dot_kernel (groups 1..3, where a 16-row MFMA tile would be mostly
//    padding, which the partitioned grid's short items would pay for): a
//    workgroup of four waves per work item. Q.K and P.V run as
//    wave-level bf16 dot2 (v_dot2_f32_bf16) with fp32 accumulation. A head row
//    of D bf16 is split over LPT = D/16 lanes; one load instruction covers
//    TPW = 64/LPT consecutive tokens, so every cache line fetched is used in
//    full. The waves' partial states are merged through LDS.
//
// Partial results (unnormalised fp32 output and (max, sum) in log2 units) go to
// the workspace; a second kernel merges the partitions of each row with the
// log-sum-exp rule. A row with a single partition is finalised in place.
//
// Numerics versus the reference (src/bridge/paged_attention.cpp:99-122 and the
// tile chain of src/bridge/paged_attention_tiles.cpp:157-188): scores are fp32
// q.k times scale; probabilities are rounded to bf16 before P.V as in the
// reference, but relative to a running rather than the final max, and
// normalised once at the end; sums use the unrounded fp32 probabilities.
#include "decode_common.hpp"

#include <algorithm>
#include <mutex>

namespace gk {
namespace {

constexpr int kWaves = 4;
// Waves per SIMD the MFMA kernel is compiled for: 3 at head_dim 64 (92
// registers). At head_dim 128 and 256 its LDS (two K and two V stages, 32 KiB
// at head_dim 128) keeps at most five workgroups on a CU, so a target of 3
// would only bound the registers: head_dim 128 needs 216 (184 VGPRs and 32
// AGPRs), missed that target and ran at 2 anyway, and compiled for 2 it
// measured C5 at 2048-key partitions 240.2-240.6 -> 236.3-236.4 us (C2
// 111.6-111.7 -> 111.2-111.6).
#ifndef GK_MFMA_WAVES_PER_SIMD
#define GK_MFMA_WAVES_PER_SIMD 3
#endif
template <int D>
constexpr int mfma_waves_per_simd() { return D >= 128 ? 2 : GK_MFMA_WAVES_PER_SIMD; }


__device__ __forceinline__ uint32_t word(const uint4& v, int e) {
  return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}


// Partition bounds shared by both kernels: keys [t_begin, t_end) of the row.
struct PartitionRange {
  int t_begin, t_end, nparts;
};

__device__ __forceinline__ PartitionRange partition_range(const DecodeArgs& a, int ctx, int part) {
  const int left = visible_left(ctx, a.window);
  const int span = ctx > left ? ctx - left : 0;
  PartitionRange r;
  r.nparts = (span + a.partition - 1) / a.partition;
  r.t_begin = left + part * a.partition;
  r.t_end = min(r.t_begin + a.partition, ctx);
  return r;
}

// Stage the block-table entries covering keys [t_begin, t_end) in LDS:
// s_bt[i] = block id of block (t_begin >> shift) + i. Ends with a barrier.
__device__ __forceinline__ int stage_block_ids(const DecodeArgs& a, const int32_t* __restrict__ bt, int t_begin,
                                               int t_end, int32_t* s_bt) {
  const int b0 = t_begin >> a.block_shift;
  const int nblk = t_end > t_begin ? ((t_end - 1) >> a.block_shift) - b0 + 1 : 0;
  for (int i = threadIdx.x; i < nblk; i += blockDim.x) s_bt[i] = bt[b0 + i];
  __syncthreads();
  return b0;
}

// ---------------------------------------------------------------------------
// MFMA kernel
// ---------------------------------------------------------------------------

// One wave per workgroup; the workgroup owns (partition blockIdx.x, kv head /
// head group blockIdx.y, query row blockIdx.z). Waves never synchronise with
// each other: partitions are uniform in size, so the GPU stays evenly loaded
// however skewed the context lengths are, and the log-sum-exp merge combines
// a row's partitions afterwards.
template <int D, bool SOFTCAP>
__global__ __launch_bounds__(64, mfma_waves_per_simd<D>()) void decode_mfma_kernel(DecodeArgs a) {
  using S = MfmaShape<D>;
  // Two stages of K and V tiles (separate objects, so the compiler can tell a
  // stage's reads from the other stage's loads in flight).
  __shared__ __attribute__((aligned(16))) char kt0[S::TILE];
  __shared__ __attribute__((aligned(16))) char vt0[S::TILE];
  __shared__ __attribute__((aligned(16))) char kt1[S::TILE];
  __shared__ __attribute__((aligned(16))) char vt1[S::TILE];
  extern __shared__ int32_t s_bt[];

  const int lane = threadIdx.x;
  const int q = lane >> 4, c16 = lane & 15;
  const int row = blockIdx.z;
  const int qrow = a.row_map ? a.row_map[row] : row;  // query/output row of this work row
  const int kvh = blockIdx.y / a.head_groups, hg = blockIdx.y % a.head_groups;
  const int ctx = a.row_context[row];
  const PartitionRange pr = partition_range(a, ctx, blockIdx.x);
  if ((int)blockIdx.x >= (pr.nparts > 1 ? pr.nparts : 1)) return;
  const int request = a.row_request ? a.row_request[row] : row;
  const int32_t* __restrict__ bt = a.block_tables + (int64_t)request * a.bt_stride;
  const int b0 = stage_block_ids(a, bt, pr.t_begin, pr.t_end, s_bt);
  const int shift = a.block_shift;

  // Valid heads of this workgroup: rows [0, hv) of the 16-row tiles.
  const int hv = min(16, a.group - hg * 16);
  const int head0 = kvh * a.group + hg * 16;

  // Q^T as the B operand of S^T = K.Q^T: lane (q, c16) holds head c16's dims of
  // chunk (4 * c + q) for k chunk c.
  bf16x8_t qb[S::NC];
#pragma unroll
  for (int c = 0; c < S::NC; ++c) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (c16 < hv) v = load16(a.query + (int64_t)qrow * a.q_stride + (int64_t)(head0 + c16) * D + (4 * c + q) * 8);
    qb[c] = __builtin_bit_cast(bf16x8_t, v);
  }

  f32x4_t o[S::NO];
#pragma unroll
  for (int c = 0; c < S::NO; ++c) o[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  // One buffer resource per (kv head, K or V) region of the pool: loads take
  // 32-bit byte offsets (slot * 2D + chunk), and the range check of the
  // resource turns any offset past the region into a zero read.
  const uint16_t* kbase = a.pool + (int64_t)kvh * a.slots * D;
  const uint16_t* vbase = kbase + (int64_t)a.kv_heads * a.slots * D;
  const uint32_t region = (uint32_t)(a.slots * D * 2);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, region, kBufferDword3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, region, kBufferDword3);
  const int t_last = pr.t_end - 1;
  const int block_mask = (1 << shift) - 1;

  // Issue the direct loads of the step at key tb into one stage.
  auto issue = [&](int tb, char* kt, char* vt) {
    // K and V tiles -> LDS with 16-byte direct loads (global_load_lds_dwordx4):
    // load i, lane l fills piece s = 64 i + l of the tile, i.e. token s / CPR,
    // stored chunk s % CPR, which holds the token's chunk (s % CPR) ^ swz(token, D / 8).
    // One load instruction thus covers whole 128-byte lines of four keys. When
    // the whole step lies in one pool block (block_size >= TS, the common case)
    // its slots are consecutive and one lookup serves every key; otherwise each
    // key is looked up, and keys past the partition read its last key (mapped,
    // so in bounds): their scores are masked and their V rows zeroed.
    if ((tb & block_mask) + S::TS <= block_mask + 1) {
      const uint32_t row0 = (uint32_t)slot_of(s_bt, b0, shift, tb) * (2 * D);
      // Load i, lane l: piece s = 64 i + l (token s / CPR, stored chunk s % CPR).
      // The K tile is issued first, then the V tile: each a contiguous burst.
#pragma unroll
      for (int i = 0; i < S::LOADS; ++i) {
        const int s = i * 64 + lane, tt = s / S::CPR, pc = s % S::CPR;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_t*)(kt + i * 1024), 16,
                                                 row0 + tt * (2 * D) + ((pc ^ swz(tt, D / 8)) << 4), 0, 0,
                                                 kKvLoadPolicyBits);
      }
#pragma unroll
      for (int i = 0; i < S::LOADS; ++i) {
        const int s = i * 64 + lane, tt = s / S::CPR, pc = s % S::CPR;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_t*)(vt + i * 1024), 16,
                                                 row0 + tt * (2 * D) + ((pc ^ swz(tt, D / 8)) << 4), 0, 0,
                                                 kKvLoadPolicyBits);
      }
    } else {
#pragma unroll
      for (int i = 0; i < S::LOADS; ++i) {
        const int s = i * 64 + lane, tt = s / S::CPR, pc = s % S::CPR;
        const uint32_t row = (uint32_t)slot_of(s_bt, b0, shift, min(tb + tt, t_last)) * (2 * D);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_t*)(kt + i * 1024), 16, row + ((pc ^ swz(tt, D / 8)) << 4),
                                                 0, 0, kKvLoadPolicyBits);
      }
#pragma unroll
      for (int i = 0; i < S::LOADS; ++i) {
        const int s = i * 64 + lane, tt = s / S::CPR, pc = s % S::CPR;
        const uint32_t row = (uint32_t)slot_of(s_bt, b0, shift, min(tb + tt, t_last)) * (2 * D);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_t*)(vt + i * 1024), 16, row + ((pc ^ swz(tt, D / 8)) << 4),
                                                 0, 0, kKvLoadPolicyBits);
      }
    }
  };

  // Attend the step at key tb from one stage (its loads have landed).
  auto consume = [&](int tb, const char* kt, char* vt) {
    // K tile -> registers as the A operand of S^T: lane (q, c16), group h holds
    // token 16h + c16, logical chunk 4c + q.
    bf16x8_t kr[S::TG][S::NC];
#pragma unroll
    for (int h = 0; h < S::TG; ++h) {
      const int tt = 16 * h + c16;
#pragma unroll
      for (int c = 0; c < S::NC; ++c)
        kr[h][c] = *reinterpret_cast<const bf16x8_t*>(kt + tt * (2 * D) + (((4 * c + q) ^ swz(tt, D / 8)) << 4));
    }

    // S^T = K.Q^T: lane (q, c16) gets head c16, tokens tb + 16h + 4q + r.
    f32x4_t sc[S::TG];
#pragma unroll
    for (int h = 0; h < S::TG; ++h) {
      sc[h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < S::NC; ++c) sc[h] = mfma32(kr[h][c], qb[c], sc[h]);
    }

    float mx = -INFINITY;
#pragma unroll
    for (int h = 0; h < S::TG; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float s;
        if constexpr (SOFTCAP) s = a.softcap_log2 * soft_tanh(sc[h][r] * a.score_scale);
        else s = sc[h][r] * a.score_scale;
        s = (tb + 16 * h + 4 * q + r < pr.t_end) ? s : -INFINITY;
        sc[h][r] = s;
        mx = fmaxf(mx, s);
      }
    mx = col4_max(mx);
    if (__builtin_amdgcn_ballot_w64(mx > m_run + kDecodeRescaleSlack)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = m_run == -INFINITY ? 0.f : fast_exp2(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
      // o rows are heads 4q + r; head h's factor lives in lanes with c16 == h.
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float f = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * q + r) << 2, __float_as_int(alpha)));
#pragma unroll
        for (int c = 0; c < S::NO; ++c) o[c][r] *= f;
      }
    }
    const float base = m_run == -INFINITY ? 0.f : m_run;
#pragma unroll
    for (int h = 0; h < S::TG; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = fast_exp2(sc[h][r] - base);
        sc[h][r] = p;
        l_run += p;
      }

    // Rows of keys past the partition hold arbitrary pool data: zero them so
    // that a zero probability cannot meet a non-finite value.
    if (tb + S::TS > pr.t_end) {
#pragma unroll
      for (int i = 0; i < S::LOADS; ++i) {
        const int s = i * 64 + lane;
        if (tb + s / S::CPR >= pr.t_end) *reinterpret_cast<uint4*>(vt + s * 16) = make_uint4(0, 0, 0, 0);
      }
    }

    // O[head][dim] += P . V
    if constexpr (S::TS == 32) {
      bf16x8_t pa;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pa[r] = (__bf16)sc[0][r];
        pa[4 + r] = (__bf16)sc[1][r];
      }
#pragma unroll
      for (int c = 0; c < S::NO; ++c) {
        // tokens 4q + (c16 >> 2) and 16 + 4q + (c16 >> 2); dims 16c + 4 (c16 & 3)
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
        const bf16x4_t v0 = lds_read_tr4(p0);
        o[c] = mfma16(pa, v0, o[c]);
      }
    }
    // The next step's direct loads overwrite both tiles: every read of them
    // must have returned first.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };

  // Two-stage pipeline: the next step's loads are in flight while the wave
  // attends the current step; only the current stage's loads are waited for.
  int tb = pr.t_begin;
  issue(tb, kt0, vt0);
  while (true) {
    const int t1 = tb + S::TS;
    if (t1 < pr.t_end) {
      issue(t1, kt1, vt1);
      wait_vmem<2 * S::LOADS>();
    } else {
      wait_vmem<0>();
    }
    consume(tb, kt0, vt0);
    if (t1 >= pr.t_end) break;
    const int t2 = t1 + S::TS;
    if (t2 < pr.t_end) {
      issue(t2, kt0, vt0);
      wait_vmem<2 * S::LOADS>();
    } else {
      wait_vmem<0>();
    }
    consume(t1, kt1, vt1);
    if (t2 >= pr.t_end) break;
    tb = t2;
  }

  // Per-head sums over the four lane groups; m_run is already uniform per head.
  l_run = col4_sum(l_run);
  // o rows are heads 4q + r: fetch each row's sum from lane c16 == 4q + r.
  float lrow[4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
    lrow[r] = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * q + r) << 2, __float_as_int(l_run)));

  if (pr.nparts <= 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * q + r;
      if (h >= hv) continue;
      const float inv = lrow[r] > 0.f ? 1.f / lrow[r] : 0.f;
      uint16_t* dst = a.out + (int64_t)qrow * a.out_stride + (int64_t)(head0 + h) * D + c16;
#pragma unroll
      for (int c = 0; c < S::NO; ++c) dst[16 * c] = (uint16_t)bf16_bits(o[c][r] * inv);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * q + r;
      if (h >= hv) continue;
      const int64_t pi = ((int64_t)row * a.q_heads + head0 + h) * a.max_parts + blockIdx.x;
      float* dst = a.part_o + pi * D + c16;
#pragma unroll
      for (int c = 0; c < S::NO; ++c) dst[16 * c] = o[c][r];
    }
    if (q == 0 && c16 < hv) {
      const int64_t pi = ((int64_t)row * a.q_heads + head0 + c16) * a.max_parts + blockIdx.x;
      a.part_ml[pi * 2] = m_run;
      a.part_ml[pi * 2 + 1] = l_run;
    }
  }
}

// ---------------------------------------------------------------------------
// dot2 kernel (small groups)
// ---------------------------------------------------------------------------
template <int D, int G, bool SOFTCAP>
__global__ __launch_bounds__(kWaves * 64) void decode_dot_kernel(DecodeArgs a) {
  constexpr int LPT = D / 16;                      // lanes per token
  constexpr int TPW = 64 / LPT;                    // tokens per wave step
  constexpr int U = (D == 256) ? 4 : 32 / TPW;     // steps per iteration (even)
  constexpr int TOK_IT = TPW * U;                  // tokens per wave iteration
  static_assert(U % 2 == 0, "tokens are paired for dot2");

  __shared__ float s_o[kWaves][G][D];
  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];
  extern __shared__ int32_t s_bt[];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = lane / LPT, j = lane % LPT;
  const int row = blockIdx.z;
  const int qrow = a.row_map ? a.row_map[row] : row;  // query/output row of this work row
  const int kvh = blockIdx.y / a.head_groups, hg = blockIdx.y % a.head_groups;
  const int ctx = a.row_context[row];
  const PartitionRange pr = partition_range(a, ctx, blockIdx.x);
  if ((int)blockIdx.x >= (pr.nparts > 1 ? pr.nparts : 1)) return;
  const int request = a.row_request ? a.row_request[row] : row;
  const int32_t* __restrict__ bt = a.block_tables + (int64_t)request * a.bt_stride;
  const int b0 = stage_block_ids(a, bt, pr.t_begin, pr.t_end, s_bt);
  const int shift = a.block_shift;

  const int c0 = j * 8, c1 = D / 2 + j * 8;
  const int head0 = kvh * a.group + hg * G;

  uint32_t qa[G][4], qb[G][4];
#pragma unroll
  for (int gh = 0; gh < G; ++gh) {
    uint4 x = make_uint4(0, 0, 0, 0), y = make_uint4(0, 0, 0, 0);
    if (hg * G + gh < a.group) {
      const uint16_t* q = a.query + (int64_t)qrow * a.q_stride + (int64_t)(head0 + gh) * D;
      x = load16(q + c0);
      y = load16(q + c1);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qa[gh][e] = word(x, e);
      qb[gh][e] = word(y, e);
    }
  }

  float m[G], l[G], o[G][16];
#pragma unroll
  for (int gh = 0; gh < G; ++gh) {
    m[gh] = -INFINITY;
    l[gh] = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) o[gh][e] = 0.f;
  }

  const uint16_t* __restrict__ kbase = a.pool + (int64_t)kvh * a.slots * D;
  const int64_t vhalf = (int64_t)a.kv_heads * a.slots * D;

  for (int tb = pr.t_begin + wave * TOK_IT; tb < pr.t_end; tb += kWaves * TOK_IT) {
    uint4 ka[U], kb[U], va[U], vb[U];
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = tb + u * TPW + grp;
      valid[u] = t < pr.t_end;
      // Keys past the partition read its last key (mapped, in bounds); masked below.
      const int slot = slot_of(s_bt, b0, shift, min(t, pr.t_end - 1));
      const uint16_t* kp = kbase + (int64_t)slot * D;
      ka[u] = load16_once(kp + c0);
      kb[u] = load16_once(kp + c1);
      va[u] = load16_once(kp + vhalf + c0);
      vb[u] = load16_once(kp + vhalf + c1);
    }

    float p[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int gh = 0; gh < G; ++gh) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc = dot2(qa[gh][e], word(ka[u], e), acc);
          acc = dot2(qb[gh][e], word(kb[u], e), acc);
        }
        acc = group_sum<LPT>(acc);
        float s;
        if constexpr (SOFTCAP) s = a.softcap_log2 * soft_tanh(acc * a.score_scale);
        else s = acc * a.score_scale;
        p[u][gh] = valid[u] ? s : -INFINITY;
      }
    }

    bool rescale = false;
    float alpha[G];
#pragma unroll
    for (int gh = 0; gh < G; ++gh) {
      float mx = m[gh];
#pragma unroll
      for (int u = 0; u < U; ++u) mx = fmaxf(mx, p[u][gh]);
      const float origin = (mx == -INFINITY) ? 0.f : mx;
      alpha[gh] = fast_exp2(m[gh] - origin);
      float sum = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        p[u][gh] = fast_exp2(p[u][gh] - origin);
        sum += p[u][gh];
      }
      l[gh] = l[gh] * alpha[gh] + sum;
      m[gh] = mx;
      rescale |= alpha[gh] != 1.f;
    }
    if (__builtin_amdgcn_ballot_w64(rescale)) {
#pragma unroll
      for (int gh = 0; gh < G; ++gh)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[gh][e] *= alpha[gh];
    }
    if (tb + TOK_IT > pr.t_end) {
      // Tail: masked tokens read slot 0, whose contents are arbitrary; zero them
      // so that a zero probability cannot meet a non-finite value.
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (!valid[u]) {
          va[u] = make_uint4(0, 0, 0, 0);
          vb[u] = make_uint4(0, 0, 0, 0);
        }
    }

#pragma unroll
    for (int u = 0; u < U; u += 2) {
      uint32_t pp[G];
#pragma unroll
      for (int gh = 0; gh < G; ++gh) pp[gh] = pack_bf16x2(p[u][gh], p[u + 1][gh]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t x0 = word(va[u], e), x1 = word(va[u + 1], e);
        const uint32_t y0 = word(vb[u], e), y1 = word(vb[u + 1], e);
        const uint32_t xlo = (x0 & 0xffffu) | (x1 << 16), xhi = (x0 >> 16) | (x1 & 0xffff0000u);
        const uint32_t ylo = (y0 & 0xffffu) | (y1 << 16), yhi = (y0 >> 16) | (y1 & 0xffff0000u);
#pragma unroll
        for (int gh = 0; gh < G; ++gh) {
          o[gh][2 * e] = dot2(pp[gh], xlo, o[gh][2 * e]);
          o[gh][2 * e + 1] = dot2(pp[gh], xhi, o[gh][2 * e + 1]);
          o[gh][8 + 2 * e] = dot2(pp[gh], ylo, o[gh][8 + 2 * e]);
          o[gh][8 + 2 * e + 1] = dot2(pp[gh], yhi, o[gh][8 + 2 * e + 1]);
        }
      }
    }
  }

  // Merge the TPW token groups of the wave: rescale to the wave max, then sum.
#pragma unroll
  for (int gh = 0; gh < G; ++gh) {
    float mw = m[gh];
#pragma unroll
    for (int mask = LPT; mask < 64; mask <<= 1) mw = fmaxf(mw, shfl_xor(mw, mask));
    const float sc = (m[gh] == -INFINITY) ? 0.f : fast_exp2(m[gh] - mw);
    float lw = l[gh] * sc;
#pragma unroll
    for (int mask = LPT; mask < 64; mask <<= 1) lw += shfl_xor(lw, mask);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float v = o[gh][e] * sc;
#pragma unroll
      for (int mask = LPT; mask < 64; mask <<= 1) v += shfl_xor(v, mask);
      o[gh][e] = v;
    }
    m[gh] = mw;
    l[gh] = lw;
  }
  if (grp == 0) {
#pragma unroll
    for (int gh = 0; gh < G; ++gh)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s_o[wave][gh][c0 + e] = o[gh][e];
        s_o[wave][gh][c1 + e] = o[gh][8 + e];
      }
  }
  if (lane == 0) {
#pragma unroll
    for (int gh = 0; gh < G; ++gh) {
      s_m[wave][gh] = m[gh];
      s_l[wave][gh] = l[gh];
    }
  }
  __syncthreads();

  const bool single = pr.nparts <= 1;
  for (int idx = threadIdx.x; idx < G * D; idx += kWaves * 64) {
    const int gh = idx / D, d = idx % D;
    if (hg * G + gh >= a.group) continue;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, s_m[w][gh]);
    float acc = 0.f, ll = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float sc = (s_m[w][gh] == -INFINITY) ? 0.f : fast_exp2(s_m[w][gh] - mm);
      acc += sc * s_o[w][gh][d];
      ll += sc * s_l[w][gh];
    }
    const int qh = head0 + gh;
    if (single) {
      a.out[(int64_t)qrow * a.out_stride + (int64_t)qh * D + d] = (uint16_t)bf16_bits(ll > 0.f ? acc / ll : 0.f);
    } else {
      const int64_t pi = ((int64_t)row * a.q_heads + qh) * a.max_parts + blockIdx.x;
      a.part_o[pi * D + d] = acc;
      if (d == 0) {
        a.part_ml[pi * 2] = mm;
        a.part_ml[pi * 2 + 1] = ll;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Split-K merge
// ---------------------------------------------------------------------------
struct MergeArgs {
  const float* part_o;
  const float* part_ml;
  const int32_t* part_count;   // explicit counts, or
  const int32_t* row_context;  // derive counts from contexts when part_count is null
  const int32_t* row_map;      // output row of each work row (null = identity)
  int32_t window, partition;
  int32_t rows, heads, max_parts;
  uint16_t* out;
  int64_t out_stride;
};

// One wave per (row, head): log-sum-exp merge of the row's partitions.
template <int D>
__global__ __launch_bounds__(64) void split_k_merge_kernel(MergeArgs a) {
  constexpr int PER_LANE = D / 64;
  const int lane = threadIdx.x;
  const int head = blockIdx.x, row = blockIdx.y;
  int nparts;
  if (a.part_count) {
    nparts = a.part_count[row];
  } else {
    const int ctx = a.row_context[row];
    const int left = visible_left(ctx, a.window);
    const int span = ctx > left ? ctx - left : 0;
    nparts = (span + a.partition - 1) / a.partition;
    if (nparts <= 1) return;  // finalised by the partition kernel
  }
  nparts = min(nparts, a.max_parts);
  const int64_t base = ((int64_t)row * a.heads + head) * a.max_parts;
  float mm = -INFINITY;
  for (int p = 0; p < nparts; ++p) mm = fmaxf(mm, a.part_ml[(base + p) * 2]);
  float acc[PER_LANE];
#pragma unroll
  for (int k = 0; k < PER_LANE; ++k) acc[k] = 0.f;
  float ll = 0.f;
  for (int p = 0; p < nparts; ++p) {
    const float mp = a.part_ml[(base + p) * 2];
    const float sc = (mp == -INFINITY) ? 0.f : fast_exp2(mp - mm);
    ll += sc * a.part_ml[(base + p) * 2 + 1];
#pragma unroll
    for (int k = 0; k < PER_LANE; ++k) acc[k] += sc * a.part_o[(base + p) * D + lane + 64 * k];
  }
  const float inv = ll > 0.f ? 1.f / ll : 0.f;
  const int orow = a.row_map ? a.row_map[row] : row;
  uint16_t* dst = a.out + (int64_t)orow * a.out_stride + (int64_t)head * D;
#pragma unroll
  for (int k = 0; k < PER_LANE; ++k) dst[lane + 64 * k] = (uint16_t)bf16_bits(acc[k] * inv);
}

template <int D>
void launch_merge(const MergeArgs& m, hipStream_t stream) {
  split_k_merge_kernel<D><<<dim3(m.heads, m.rows), 64, 0, stream>>>(m);
}

void launch_merge_dispatch(int head_dim, const MergeArgs& m, hipStream_t stream) {
  switch (head_dim) {
    case 64: launch_merge<64>(m, stream); break;
    case 128: launch_merge<128>(m, stream); break;
    default: launch_merge<256>(m, stream); break;
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
template <int D, int G>
void launch_dot(const DecodeArgs& a, bool softcap, dim3 grid, size_t lds, hipStream_t stream) {
  if (softcap) decode_dot_kernel<D, G, true><<<grid, kWaves * 64, lds, stream>>>(a);
  else decode_dot_kernel<D, G, false><<<grid, kWaves * 64, lds, stream>>>(a);
}

template <int D>
void launch_dot_g(int g, const DecodeArgs& a, bool softcap, dim3 grid, size_t lds, hipStream_t stream) {
  switch (g) {
    case 1: launch_dot<D, 1>(a, softcap, grid, lds, stream); break;
    case 2: launch_dot<D, 2>(a, softcap, grid, lds, stream); break;
    default: launch_dot<D, 3>(a, softcap, grid, lds, stream); break;
  }
}

template <int D>
void launch_mfma(const DecodeArgs& a, bool softcap, dim3 grid, size_t lds, hipStream_t stream) {
  if (softcap) decode_mfma_kernel<D, true><<<grid, 64, lds, stream>>>(a);
  else decode_mfma_kernel<D, false><<<grid, 64, lds, stream>>>(a);
}

// Query heads one workgroup computes for a kv head: the whole group up to 16
// (MFMA rows) when the group is >= 4, else the group itself (dot2 path).
bool use_mfma(int group) { return group >= 4; }
int heads_per_workgroup(int group) { return use_mfma(group) ? std::min(group, 16) : group; }

int validate(const gk_decode_params* p) {
  if (!p) return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: null parameters");
  if (p->struct_size != sizeof(gk_decode_params))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: struct_size does not match this library's gk_decode_params");
  if (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256)
    return fail(GK_ERR_UNSUPPORTED, "gk_paged_decode: head dimension must be 64, 128 or 256");
  if (p->q_heads <= 0 || p->kv_heads <= 0 || p->q_heads % p->kv_heads || p->q_heads > 1024)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: invalid head geometry");
  if (p->rows < 0 || p->rows > 65535 || p->slots <= 0 || p->max_context < 0)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: rows, slots or max_context out of range");
  if (!is_pow2(p->block_size) || p->block_size > (1 << 20))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: block_size must be a power of two");
  if (p->partition_tokens < 0 || (p->partition_tokens % 32) || p->partition_tokens > 8192)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: partition_tokens must be a multiple of 32, at most 8192");
  if (!(p->scale > 0.f) || !(p->scale < INFINITY) || !(p->softcap >= 0.f) || !(p->softcap < INFINITY))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: invalid scale or softcap");
  if (p->rows == 0) return GK_OK;
  if (!p->query || !p->pool || !p->block_tables || !p->row_context || !p->out)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: null pointer");
  const auto misaligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) != 0; };
  if (p->slots > (int64_t)(UINT32_MAX / 2) / p->head_dim)
    return fail(GK_ERR_UNSUPPORTED, "gk_paged_decode: one kv head's K or V region must stay below 4 GiB");
  if (misaligned(p->query) || misaligned(p->pool) || (p->q_row_stride & 7) ||
      p->q_row_stride < (int64_t)p->q_heads * p->head_dim || p->out_row_stride < (int64_t)p->q_heads * p->head_dim)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: query/pool must be 16-byte aligned with full rows");
  return GK_OK;
}

}  // namespace

// Compute units of the current device (cached per device; 256 on MI355X).
int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// Split-K partition (keys per work item). MFMA path: one wave per item, its
// two K/V stages in LDS; a CU holds kLdsBytes / stage bytes of them.
//  - Work units (row, kv head, head group) at least fill the resident waves:
//    one item per unit (no merge), the partition covering max_context.
//  - Otherwise 2048-key items while one round of them (at the expected mean
//    length max_context / 2) fits the resident waves, else 1024.
// dot2 path: halve a 2048-key partition until the items fill the GPU.
// The balanced schedule (decode_stream.hip) serves every GQA group and block
// size whenever the caller leaves the partition to the library (at groups 1-3
// most of its 16 MFMA head columns are padding, which costs nothing against
// the K/V stream); an explicit partition takes the partitioned kernels.
// The balanced schedule numbers the batch's tiles in 32 bits: it runs when
// every row's tiles (at most max_context / TS + 2 with a window's offset)
// times the units, plus the grid's workgroups, stay below 2^31 (the kernel's
// own test, stream_tiles_fit); larger batches take the partitioned kernel.
bool use_stream(const gk_decode_params* p) {
  const int group = p->q_heads / p->kv_heads;
  if (p->partition_tokens != 0) return false;
  const int hpw = heads_per_workgroup(group);
  const int64_t units = (int64_t)p->rows * p->kv_heads * ((group + hpw - 1) / hpw);
  const int ts = p->head_dim == 256 ? 16 : 32;
  return stream_tiles_fit(units, p->max_context, ts,
                          stream_decode_wgs(p->head_dim, p->softcap > 0.f, p->block_size));
}

int32_t decode_partition(const gk_decode_params* p) {
  if (p->partition_tokens > 0) return p->partition_tokens;
  if (use_stream(p)) return 0;
  const int group = p->q_heads / p->kv_heads;
  const int hpw = heads_per_workgroup(group);
  const int64_t units = (int64_t)p->rows * p->kv_heads * ((group + hpw - 1) / hpw);
  const int64_t mean_context = std::max<int64_t>(1, p->max_context / 2);
  if (use_mfma(group)) {
    constexpr int64_t kLdsBytes = 160 * 1024;
    const int64_t stage_bytes = 2LL * 2 * (p->head_dim == 256 ? 16 : 32) * p->head_dim * 2;
    const int64_t resident = (int64_t)device_cus() * std::max<int64_t>(1, kLdsBytes / stage_bytes);
    if (units >= resident) {
      int32_t part = 1024;
      while (part < p->max_context && part < 8192) part *= 2;
      return part;
    }
    return units * ((mean_context + 2047) / 2048) <= resident ? 2048 : 1024;
  }
  int32_t part = 2048;
  while (part > 128 && units * ((mean_context + part - 1) / part) < 2048) part /= 2;
  return part;
}

int32_t decode_max_parts(const gk_decode_params* p) {
  const int32_t part = decode_partition(p);
  if (part == 0) return 1;
  return std::max<int32_t>(1, (p->max_context + part - 1) / part);
}

int64_t stream_units(const gk_decode_params* p) {
  const int group = p->q_heads / p->kv_heads;
  const int hpw = heads_per_workgroup(group);
  return (int64_t)p->rows * p->kv_heads * ((group + hpw - 1) / hpw);
}

size_t decode_workspace_bytes(const gk_decode_params* p) {
  if (p->rows > 0 && use_stream(p))
    return stream_decode_workspace_bytes(p->head_dim, heads_per_workgroup(p->q_heads / p->kv_heads), stream_units(p),
                                         stream_decode_wgs(p->head_dim, p->softcap > 0.f, p->block_size));
  const int32_t parts = decode_max_parts(p);
  if (parts <= 1 || p->rows == 0) return 0;
  const size_t n = (size_t)p->rows * p->q_heads * parts;
  const size_t o_bytes = (n * p->head_dim * sizeof(float) + 255) & ~size_t{255};
  return o_bytes + n * 2 * sizeof(float);
}

int paged_decode(const gk_decode_params* p, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (int rc = validate(p)) return rc;
  if (p->rows == 0) return GK_OK;
  if (p->new_key) {
    if (!p->new_value || !p->slot_mapping)
      return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: fused store needs new_value and slot_mapping");
    if (int rc = launch_kv_store(p->new_key, p->new_value, p->new_kv_row_stride, p->new_kv_row_stride,
                                 p->slot_mapping, p->rows, const_cast<void*>(p->pool), p->slots, p->kv_heads,
                                 p->head_dim, stream))
      return rc;
  }
  const int32_t part = decode_partition(p);
  const int32_t max_parts = decode_max_parts(p);
  const size_t need = decode_workspace_bytes(p);
  if (need > workspace_bytes || (need && !workspace))
    return fail(GK_ERR_WORKSPACE, "gk_paged_decode: workspace too small (" + std::to_string(need) + " bytes needed)");
  const int group = p->q_heads / p->kv_heads;
  const int hpw = heads_per_workgroup(group);
  DecodeArgs a{};
  a.query = static_cast<const uint16_t*>(p->query);
  a.q_stride = p->q_row_stride;
  a.pool = static_cast<const uint16_t*>(p->pool);
  a.slots = p->slots;
  a.block_tables = p->block_tables;
  a.bt_stride = p->bt_stride;
  a.block_shift = log2_int(p->block_size);
  a.row_request = p->row_request;
  a.row_context = p->row_context;
  a.row_map = p->row_map;
  a.rows = p->rows;
  a.q_heads = p->q_heads;
  a.kv_heads = p->kv_heads;
  a.group = group;
  a.heads_per_group = hpw;
  a.head_groups = (group + hpw - 1) / hpw;
  const bool softcap = p->softcap > 0.f;
  a.score_scale = softcap ? p->scale / p->softcap : p->scale * kLog2e;
  a.softcap_log2 = p->softcap * kLog2e;
  a.window = p->sliding_window > 0 ? p->sliding_window : 0;
  a.partition = part;
  a.max_parts = max_parts;
  a.out = static_cast<uint16_t*>(p->out);
  a.out_stride = p->out_row_stride;
  if (use_stream(p))
    return launch_stream_decode(a, softcap, p->head_dim, stream_decode_wgs(p->head_dim, softcap, p->block_size), workspace,
                                stream);
  if (need) {
    const size_t n = (size_t)p->rows * p->q_heads * max_parts;
    const size_t o_bytes = (n * p->head_dim * sizeof(float) + 255) & ~size_t{255};
    a.part_o = static_cast<float*>(workspace);
    a.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + o_bytes);
  }
  // Block-table entries one partition can span (its start need not be block aligned).
  const size_t bt_lds = sizeof(int32_t) * (size_t)(((part - 1) >> a.block_shift) + 2);
  const dim3 grid(max_parts, p->kv_heads * a.head_groups, p->rows);
  if (use_mfma(group)) {
    switch (p->head_dim) {
      case 64: launch_mfma<64>(a, softcap, grid, bt_lds, stream); break;
      case 128: launch_mfma<128>(a, softcap, grid, bt_lds, stream); break;
      default: launch_mfma<256>(a, softcap, grid, bt_lds, stream); break;
    }
  } else {
    switch (p->head_dim) {
      case 64: launch_dot_g<64>(hpw, a, softcap, grid, bt_lds, stream); break;
      case 128: launch_dot_g<128>(hpw, a, softcap, grid, bt_lds, stream); break;
      default: launch_dot_g<256>(hpw, a, softcap, grid, bt_lds, stream); break;
    }
  }
  if (int rc = hip_status(hipGetLastError(), "gk_paged_decode partition launch")) return rc;
  if (max_parts > 1) {
    MergeArgs m{};
    m.part_o = a.part_o;
    m.part_ml = a.part_ml;
    m.row_context = p->row_context;
    m.row_map = p->row_map;
    m.window = a.window;
    m.partition = part;
    m.rows = p->rows;
    m.heads = p->q_heads;
    m.max_parts = max_parts;
    m.out = a.out;
    m.out_stride = p->out_row_stride;
    launch_merge_dispatch(p->head_dim, m, stream);
    if (int rc = hip_status(hipGetLastError(), "gk_paged_decode merge launch")) return rc;
  }
  return GK_OK;
}

int split_k_merge(const float* partial_out, const float* partial_ml, const int32_t* part_count, int32_t rows,
                  int32_t heads, int32_t max_parts, int32_t head_dim, void* out, int64_t out_row_stride,
                  hipStream_t stream) {
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(GK_ERR_UNSUPPORTED, "gk_split_k_merge: head dimension must be 64, 128 or 256");
  if (rows < 0 || rows > 65535 || heads <= 0 || heads > 65535 || max_parts <= 0 ||
      out_row_stride < (int64_t)heads * head_dim)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_split_k_merge: invalid sizes");
  if (rows == 0) return GK_OK;
  if (!partial_out || !partial_ml || !part_count || !out)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_split_k_merge: null pointer");
  MergeArgs m{};
  m.part_o = partial_out;
  m.part_ml = partial_ml;
  m.part_count = part_count;
  m.rows = rows;
  m.heads = heads;
  m.max_parts = max_parts;
  m.out = static_cast<uint16_t*>(out);
  m.out_stride = out_row_stride;
  launch_merge_dispatch(head_dim, m, stream);
  return hip_status(hipGetLastError(), "gk_split_k_merge launch");
}

// ---------------------------------------------------------------------------
// Allocation-free decode: the split-K workspace in a static device array
// ---------------------------------------------------------------------------
namespace {

// Every GPU the library runs on holds this array until the process ends. Each
// device has its own copy at its own address, looked up once per device with
// hipGetSymbolAddress; host code uses only that address, never the name.
static __device__ __align__(256) unsigned char scratch[GK_DECODE_SCRATCH_BYTES];

std::mutex scratch_mutex;
void* scratch_address[64] = {};

// Address of `scratch` on the current device (which must be the stream's).
int scratch_on_device(hipStream_t stream, void** out) {
  int dev = 0;
  if (int rc = hip_status(hipGetDevice(&dev), "gk_paged_decode_scratch: hipGetDevice")) return rc;
  hipDevice_t stream_dev = dev;
  if (int rc = hip_status(hipStreamGetDevice(stream, &stream_dev), "gk_paged_decode_scratch: hipStreamGetDevice"))
    return rc;
  if (stream_dev != dev)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode_scratch: the stream belongs to another device than the current one");
  if (dev < 0 || dev >= 64) return fail(GK_ERR_UNSUPPORTED, "gk_paged_decode_scratch: device index above 63");
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_address[dev]) {
    void* address = nullptr;
    if (int rc = hip_status(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)),
                            "gk_paged_decode_scratch: hipGetSymbolAddress"))
      return rc;
    scratch_address[dev] = address;
  }
  *out = scratch_address[dev];
  return GK_OK;
}

}  // namespace

// Nothing in the workspace has to start at zero: every partial and every span
// record the merge reads is written by the same call's decode kernel first.
int paged_decode_scratch(const gk_decode_params* p, hipStream_t stream) {
  if (int rc = validate(p)) return rc;
  if (p->rows == 0) return GK_OK;
  const size_t need = decode_workspace_bytes(p);
  if (need > GK_DECODE_SCRATCH_BYTES)
    return fail(GK_ERR_WORKSPACE, "gk_paged_decode_scratch: these parameters need " + std::to_string(need) +
                                      " bytes of workspace, more than the " + std::to_string(GK_DECODE_SCRATCH_BYTES) +
                                      "-byte static scratch; call gk_paged_decode with a workspace instead");
  void* workspace = nullptr;
  if (need)
    if (int rc = scratch_on_device(stream, &workspace)) return rc;
  return paged_decode(p, workspace, need, stream);
}

}  // namespace gk

extern "C" size_t gk_paged_decode_workspace_bytes(const gk_decode_params* params) {
  return params && params->struct_size == sizeof(gk_decode_params) ? gk::decode_workspace_bytes(params) : 0;
}

extern "C" int32_t gk_paged_decode_partition_tokens(const gk_decode_params* params) {
  return params && params->struct_size == sizeof(gk_decode_params) ? gk::decode_partition(params) : 0;
}

extern "C" int gk_paged_decode(const gk_decode_params* params, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
  gk::clear_error();
  return gk::paged_decode(params, workspace, workspace_bytes, stream);
}

extern "C" int gk_split_k_merge(const float* partial_out, const float* partial_ml, const int32_t* part_count,
                                int32_t rows, int32_t heads, int32_t max_parts, int32_t head_dim, void* out,
                                int64_t out_row_stride, hipStream_t stream) {
  gk::clear_error();
  return gk::split_k_merge(partial_out, partial_ml, part_count, rows, heads, max_parts, head_dim, out,
                           out_row_stride, stream);
}

extern "C" int gk_paged_decode_scratch(const gk_decode_params* params, hipStream_t stream) {
  gk::clear_error();
  return gk::paged_decode_scratch(params, stream);
}
