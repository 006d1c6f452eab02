// Paged decode attention for gfx950: split-K partitions + log-sum-exp merge.
//
// Work decomposition. One workgroup of NW waves owns one (query row, kv head,
// head group, partition of `partition` keys). The G query heads that share a
// kv head are computed together, so each K/V byte is read from HBM once per
// group. Decode has no dense contraction to feed MFMA (M = G <= 8 rows), so
// Q.K and P.V run as wave-level bf16 dot2 (v_dot2_f32_bf16) with fp32
// accumulation.
//
// Lane layout. A head row of D bf16 (2*D bytes) is split over LPT = D/16 lanes;
// lane j of a token group owns d in [8j, 8j+8) and [D/2 + 8j, D/2 + 8j + 8).
// One load instruction therefore covers TPW = 64/LPT consecutive tokens times a
// contiguous half row (128 B for D = 128): every cache line fetched is used in
// full. Q.K partial sums are reduced over the LPT lanes with DPP; the token
// group keeps its own running max/sum/output (online softmax), P.V needs no
// cross-lane traffic, and the groups, then the waves, are merged once at the
// end (registers, then LDS).
//
// Partial results (unnormalised fp32 output and (max, sum) in log2 units) go to
// the workspace; a second kernel merges the partitions of each row with the
// log-sum-exp rule. A row with a single partition is finalised in place.
//
// Numerics versus the reference (src/bridge/paged_attention.cpp:99-122 and the
// tile chain of src/bridge/paged_attention_tiles.cpp:189-219): scores are fp32
// q.k times scale; probabilities are rounded to bf16 before P.V as in the
// reference, but relative to a running rather than the final max, and
// normalised once at the end; sums use the unrounded fp32 probabilities.
#include "gk_common.hpp"

#include <algorithm>

namespace gk {
namespace {

constexpr int kWaves = 4;

struct DecodeArgs {
  const uint16_t* query;
  int64_t q_stride;
  const uint16_t* pool;
  int64_t slots;
  const int32_t* block_tables;
  int64_t bt_stride;
  int32_t block_shift;
  const int32_t* row_request;
  const int32_t* row_context;
  int32_t rows, q_heads, kv_heads, group, head_groups;
  float score_scale;  // scale * log2(e), or scale / softcap when capping
  float softcap_log2; // softcap * log2(e) when capping
  int32_t window, partition, max_parts;
  uint16_t* out;
  int64_t out_stride;
  float* part_o;
  float* part_ml;
};

__device__ __forceinline__ uint4 load16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

__device__ __forceinline__ uint32_t word(const uint4& v, int e) {
  return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}

// tanh via exp2: tanh(x) = 1 - 2 / (2^(2x log2 e) + 1); saturates cleanly at +-1.
__device__ __forceinline__ float soft_tanh(float x) {
  const float e = fast_exp2(2.f * kLog2e * x);
  return 1.f - 2.f / (e + 1.f);
}

__device__ __forceinline__ int visible_left(int ctx, int window) {
  return (window > 0 && ctx > window) ? ctx - window : 0;
}

template <int D, int G, bool SOFTCAP>
__global__ __launch_bounds__(kWaves * 64) void decode_partition_kernel(DecodeArgs a) {
  constexpr int LPT = D / 16;                      // lanes per token
  constexpr int TPW = 64 / LPT;                    // tokens per wave step
  constexpr int U = (D == 256) ? 4 : 32 / TPW;     // steps per iteration (even)
  constexpr int TOK_IT = TPW * U;                  // tokens per wave iteration
  static_assert(U % 2 == 0, "tokens are paired for dot2");

  __shared__ float s_o[kWaves][G][D];
  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = lane / LPT, j = lane % LPT;
  const int row = blockIdx.z;
  const int kvh = blockIdx.y / a.head_groups, hg = blockIdx.y % a.head_groups;
  const int ctx = a.row_context[row];
  const int left = visible_left(ctx, a.window);
  const int span = ctx > left ? ctx - left : 0;
  const int nparts = (span + a.partition - 1) / a.partition;
  const int part = blockIdx.x;
  if (part >= (nparts > 1 ? nparts : 1)) return;
  const int t_begin = left + part * a.partition;
  const int t_end = min(t_begin + a.partition, ctx);

  const int request = a.row_request ? a.row_request[row] : row;
  const int32_t* __restrict__ bt = a.block_tables + (int64_t)request * a.bt_stride;
  const int c0 = j * 8, c1 = D / 2 + j * 8;
  const int head0 = kvh * a.group + hg * G;

  uint32_t qa[G][4], qb[G][4];
#pragma unroll
  for (int gh = 0; gh < G; ++gh) {
    uint4 x = make_uint4(0, 0, 0, 0), y = make_uint4(0, 0, 0, 0);
    if (hg * G + gh < a.group) {
      const uint16_t* q = a.query + (int64_t)row * a.q_stride + (int64_t)(head0 + gh) * D;
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
  const int bmask = (1 << a.block_shift) - 1;

  for (int tb = t_begin + wave * TOK_IT; tb < t_end; tb += kWaves * TOK_IT) {
    uint4 ka[U], kb[U], va[U], vb[U];
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = tb + u * TPW + grp;
      valid[u] = t < t_end;
      int slot = 0;
      if (valid[u]) slot = (bt[t >> a.block_shift] << a.block_shift) | (t & bmask);
      const uint16_t* kp = kbase + (int64_t)slot * D;
      ka[u] = load16(kp + c0);
      kb[u] = load16(kp + c1);
      va[u] = load16(kp + vhalf + c0);
      vb[u] = load16(kp + vhalf + c1);
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
    if (tb + TOK_IT > t_end) {
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

  const bool single = nparts <= 1;
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
      a.out[(int64_t)row * a.out_stride + (int64_t)qh * D + d] = (uint16_t)bf16_bits(ll > 0.f ? acc / ll : 0.f);
    } else {
      const int64_t pi = ((int64_t)row * a.q_heads + qh) * a.max_parts + part;
      a.part_o[pi * D + d] = acc;
      if (d == 0) {
        a.part_ml[pi * 2] = mm;
        a.part_ml[pi * 2 + 1] = ll;
      }
    }
  }
}

struct MergeArgs {
  const float* part_o;
  const float* part_ml;
  const int32_t* part_count;   // explicit counts, or
  const int32_t* row_context;  // derive counts from contexts when part_count is null
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
  uint16_t* dst = a.out + (int64_t)row * a.out_stride + (int64_t)head * D;
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

template <int D, int G>
void launch_partition(const DecodeArgs& a, bool softcap, dim3 grid, hipStream_t stream) {
  if (softcap) decode_partition_kernel<D, G, true><<<grid, kWaves * 64, 0, stream>>>(a);
  else decode_partition_kernel<D, G, false><<<grid, kWaves * 64, 0, stream>>>(a);
}

template <int D>
void launch_partition_g(int g, const DecodeArgs& a, bool softcap, dim3 grid, hipStream_t stream) {
  switch (g) {
    case 1: launch_partition<D, 1>(a, softcap, grid, stream); break;
    case 2: launch_partition<D, 2>(a, softcap, grid, stream); break;
    case 4: launch_partition<D, 4>(a, softcap, grid, stream); break;
    default: launch_partition<D, 8>(a, softcap, grid, stream); break;
  }
}

int group_tile(int group) { return group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : 8; }

int validate(const gk_decode_params* p) {
  if (!p) return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: null parameters");
  if (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256)
    return fail(GK_ERR_UNSUPPORTED, "gk_paged_decode: head dimension must be 64, 128 or 256");
  if (p->q_heads <= 0 || p->kv_heads <= 0 || p->q_heads % p->kv_heads || p->q_heads > 1024)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: invalid head geometry");
  if (p->rows < 0 || p->rows > 65535 || p->slots <= 0 || p->max_context < 0)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: rows, slots or max_context out of range");
  if (!is_pow2(p->block_size) || p->block_size > (1 << 20))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: block_size must be a power of two");
  if (p->partition_tokens < 0 || (p->partition_tokens % 32))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: partition_tokens must be a multiple of 32");
  if (!(p->scale > 0.f) || !(p->scale < INFINITY) || !(p->softcap >= 0.f) || !(p->softcap < INFINITY))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: invalid scale or softcap");
  if (p->rows == 0) return GK_OK;
  if (!p->query || !p->pool || !p->block_tables || !p->row_context || !p->out)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: null pointer");
  const auto misaligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) != 0; };
  if (misaligned(p->query) || misaligned(p->pool) || (p->q_row_stride & 7) ||
      p->q_row_stride < (int64_t)p->q_heads * p->head_dim || p->out_row_stride < (int64_t)p->q_heads * p->head_dim)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_decode: query/pool must be 16-byte aligned with full rows");
  return GK_OK;
}

}  // namespace

int32_t decode_partition(const gk_decode_params* p) {
  if (p->partition_tokens > 0) return p->partition_tokens;
  const int group = p->q_heads / p->kv_heads;
  const int64_t units = (int64_t)p->rows * p->kv_heads * ((group + group_tile(group) - 1) / group_tile(group));
  const int64_t mean_context = std::max<int64_t>(1, p->max_context / 2);
  int32_t part = 2048;
  while (part > 128 && units * ((mean_context + part - 1) / part) < 2048) part /= 2;
  return part;
}

int32_t decode_max_parts(const gk_decode_params* p) {
  const int32_t part = decode_partition(p);
  return std::max<int32_t>(1, (p->max_context + part - 1) / part);
}

size_t decode_workspace_bytes(const gk_decode_params* p) {
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
  const int g = group_tile(group);
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
  a.rows = p->rows;
  a.q_heads = p->q_heads;
  a.kv_heads = p->kv_heads;
  a.group = group;
  a.head_groups = (group + g - 1) / g;
  const bool softcap = p->softcap > 0.f;
  a.score_scale = softcap ? p->scale / p->softcap : p->scale * kLog2e;
  a.softcap_log2 = p->softcap * kLog2e;
  a.window = p->sliding_window > 0 ? p->sliding_window : 0;
  a.partition = part;
  a.max_parts = max_parts;
  a.out = static_cast<uint16_t*>(p->out);
  a.out_stride = p->out_row_stride;
  if (need) {
    const size_t n = (size_t)p->rows * p->q_heads * max_parts;
    const size_t o_bytes = (n * p->head_dim * sizeof(float) + 255) & ~size_t{255};
    a.part_o = static_cast<float*>(workspace);
    a.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + o_bytes);
  }
  const dim3 grid(max_parts, p->kv_heads * a.head_groups, p->rows);
  switch (p->head_dim) {
    case 64: launch_partition_g<64>(g, a, softcap, grid, stream); break;
    case 128: launch_partition_g<128>(g, a, softcap, grid, stream); break;
    default: launch_partition_g<256>(g, a, softcap, grid, stream); break;
  }
  if (int rc = hip_status(hipGetLastError(), "gk_paged_decode partition launch")) return rc;
  if (max_parts > 1) {
    MergeArgs m{};
    m.part_o = a.part_o;
    m.part_ml = a.part_ml;
    m.row_context = p->row_context;
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

}  // namespace gk

extern "C" size_t gk_paged_decode_workspace_bytes(const gk_decode_params* params) {
  return params ? gk::decode_workspace_bytes(params) : 0;
}

extern "C" int32_t gk_paged_decode_partition_tokens(const gk_decode_params* params) {
  return params ? gk::decode_partition(params) : 0;
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
