// Device-side paged metadata for gfx950: validation and normalisation of
// device-resident scheduler inputs, block tables derived from a request map,
// and the page allocator of the pool's write side.
//
//  gk_metadata_normalize   device half of PagedMetadata.from_device,
//                          from_device_with_tokens, _from_scheduler and
//                          _from_scheduler_fused (src/bridge/paged_metadata.cpp:176-430)
//  gk_block_tables         block table of a page-aligned request map
//  gk_paged_alloc_slots    _C._allocate_paged_slots
//  gk_paged_release_slots  _C._release_paged_slots
//                          (src/bridge/paged_slot_allocator.cpp:91-190)
//
// All of it is integer work of a few hundred KiB at most; one thread per row,
// per visible prefix position or per token, with no shared tiles.
#include "gk_common.hpp"

#include <algorithm>
#include <climits>
#include <cstring>

namespace gk {
namespace {

constexpr int kThreads = 256;
constexpr int kPageCandidates = 10;  // page sizes 2 .. 1024 (flag bit k: 2 << k)

__device__ __forceinline__ int64_t load_index(const void* p, int is64, int64_t i) {
  return is64 ? static_cast<const int64_t*>(p)[i] : static_cast<const int32_t*>(p)[i];
}

__device__ __forceinline__ uint32_t slot_hash(int32_t slot, uint32_t mask) {
  return (static_cast<uint32_t>(slot) * 2654435761u) & mask;
}

// Load that bypasses the CU's L1, for words other waves of the same grid
// updated with atomics (which complete in L2).
__device__ __forceinline__ int32_t coherent_load(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Largest index s in [0, n) with offsets[s * stride] <= e (offsets
// non-decreasing, offsets[0] <= e).
template <typename T>
__device__ __forceinline__ int last_at_or_below(const T* offsets, int stride, int n, int64_t e) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offsets[(int64_t)mid * stride] <= e) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

struct NormArgs {
  const void* locations;
  const void* batch_requests;
  const void* positions;
  const void* token_ids;
  int32_t loc64, req64, pos64, tok64;
  const int32_t* mapping;
  const int32_t* row_seq;
  const int32_t* seq_prefix;
  const int32_t* seq_first_row;
  const int64_t* seq_visible;  // [batch] first visible element of each sequence
  int64_t visible_total;
  int32_t rows, padded_rows, batch, requests, context, vocabulary;
  int64_t slots;
  int32_t* out_locations;
  int32_t* out_requests;
  int32_t* out_positions;
  int32_t* out_tokens;
  int32_t* status;
  int32_t* token_status;
  int32_t* page_flags;
  int32_t* table_keys;  // [mask + 1] output slot, -1 = empty
  int32_t* table_rows;  // [mask + 1] smallest row writing that slot
  int32_t* seq_bits;    // [batch] bit 0: missing prefix slot, bit 1: aliased prefix slot
  uint32_t table_mask;
};

__global__ __launch_bounds__(kThreads) void fill_kernel(int32_t* p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) p[i] = v;
}

// Host-staged words carried in the launch's own kernel arguments: the
// kernel stores them at `device`, and inputs that point into that range are
// read from the argument copy (the grid is writing the memory they name).
template <bool kStaged>
struct Staged {};
template <>
struct Staged<true> {
  int32_t* device;
  int32_t count;
  int32_t row_seq, seq_prefix, seq_first_row, positions;  // word offsets into `words`, or -1
  int32_t words[GK_METADATA_INLINE_WORDS];
};

template <bool kStaged>
__device__ __forceinline__ int32_t staged_word(const Staged<kStaged>& s, int off, const int32_t* p, int64_t i) {
  if constexpr (kStaged) {
    if (off >= 0) return s.words[off + i];
  }
  return p[i];
}

template <bool kStaged>
__device__ __forceinline__ int64_t staged_index(const Staged<kStaged>& s, int off, const void* p, int is64,
                                                int64_t i) {
  if constexpr (kStaged) {
    if (off >= 0) {
      if (!is64) return s.words[off + i];
      const uint32_t lo = static_cast<uint32_t>(s.words[off + 2 * i]);
      return static_cast<int64_t>(static_cast<uint64_t>(static_cast<uint32_t>(s.words[off + 2 * i + 1])) << 32 | lo);
    }
  }
  return load_index(p, is64, i);
}

// Pass 1, one thread per padded row: int32 rows (zeros past `rows`), range
// codes 1/2, mapping agreement 3, expected position 5, token range; rows with
// no code claim their output slot in the hash table.
template <bool kStaged>
__global__ __launch_bounds__(kThreads) void normalize_rows_kernel(NormArgs a, Staged<kStaged> st) {
  int row_seq_off = -1, prefix_off = -1, first_off = -1, positions_off = -1;
  if constexpr (kStaged) {
    for (int j = blockIdx.x * kThreads + threadIdx.x; j < st.count; j += gridDim.x * kThreads)
      st.device[j] = st.words[j];
    row_seq_off = st.row_seq;
    prefix_off = st.seq_prefix;
    first_off = st.seq_first_row;
    positions_off = st.positions;
  }
  for (int i = blockIdx.x * kThreads + threadIdx.x; i < a.padded_rows; i += gridDim.x * kThreads) {
    if (i >= a.rows) {
      a.out_locations[i] = 0;
      a.out_requests[i] = 0;
      a.out_positions[i] = 0;
      if (a.token_ids) a.out_tokens[i] = 0;
      if (a.status) a.status[i] = 0;
      if (a.token_status) a.token_status[i] = 0;
      continue;
    }
    const int seq = staged_word(st, row_seq_off, a.row_seq, i);
    const int64_t loc = load_index(a.locations, a.loc64, i);
    const int64_t pos = staged_index(st, positions_off, a.positions, a.pos64, i);
    const int64_t req = load_index(a.batch_requests, a.req64, seq);
    a.out_locations[i] = static_cast<int32_t>(loc);
    a.out_positions[i] = static_cast<int32_t>(pos);
    a.out_requests[i] = static_cast<int32_t>(req);
    if (a.token_ids) {
      const int64_t tok = load_index(a.token_ids, a.tok64, i);
      a.out_tokens[i] = static_cast<int32_t>(tok);
      if (a.token_status) a.token_status[i] = (tok < 0 || tok >= a.vocabulary) ? 1 : 0;
    }
    if (!a.status) continue;
    int code = 0;
    if (loc < 0 || loc >= a.slots || pos < 0 || pos >= a.context) code = 1;
    else if (req < 0 || req >= a.requests) code = 2;
    if (a.mapping) {
      if (code == 0 && a.mapping[req * a.context + pos] != static_cast<int32_t>(loc)) code = 3;
      if (code == 0 && pos != (int64_t)staged_word(st, prefix_off, a.seq_prefix, seq) +
                                   (i - staged_word(st, first_off, a.seq_first_row, seq)))
        code = 5;
      if (code == 0) {
        const int32_t key = static_cast<int32_t>(loc);
        uint32_t h = slot_hash(key, a.table_mask);
        while (true) {
          const int32_t prev = atomicCAS(a.table_keys + h, -1, key);
          if (prev == -1 || prev == key) break;
          h = (h + 1) & a.table_mask;
        }
        atomicMin(a.table_rows + h, i);
      }
    }
    a.status[i] = code;
  }
}

// Row owning output slot `slot` (smallest row writing it), or -1.
__device__ __forceinline__ int owner_of(const NormArgs& a, int32_t slot) {
  uint32_t h = slot_hash(slot, a.table_mask);
  for (uint32_t n = 0; n <= a.table_mask; ++n) {
    const int32_t key = a.table_keys[h];
    if (key == -1) return -1;
    if (key == slot) return a.table_rows[h];
    h = (h + 1) & a.table_mask;
  }
  return -1;
}

// Pass 2, one thread per visible (sequence, position t < prefix + length):
// the request's prefix has a slot at t (else bit 0) that is no other
// (request, position)'s output slot (else bit 1); page-size alignment flags.
__global__ __launch_bounds__(kThreads) void prefix_kernel(NormArgs a) {
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < a.visible_total;
       e += (int64_t)gridDim.x * kThreads) {
    const int s = last_at_or_below(a.seq_visible, 1, a.batch, e);
    const int t = static_cast<int>(e - a.seq_visible[s]);
    const int64_t req = load_index(a.batch_requests, a.req64, s);
    if (req < 0 || req >= a.requests) continue;  // code 2 on the sequence's rows
    const int32_t* map = a.mapping + req * a.context;
    const int32_t slot = map[t];
    if (a.status) {
      int bits = 0;
      if (slot < 0) {
        bits = 1;
      } else {
        const int o = owner_of(a, slot);
        if (o >= 0 && (a.out_requests[o] != static_cast<int32_t>(req) || a.out_positions[o] != t)) bits = 2;
      }
      if (bits) atomicOr(a.seq_bits + s, bits);
    }
    if (a.page_flags) {
      int bad = 0;
#pragma unroll
      for (int k = 0; k < kPageCandidates; ++k) {
        const int page = 2 << k;
        const int32_t first_slot = map[t & ~(page - 1)];
        if (slot < 0 || first_slot < 0 || (first_slot & (page - 1)) != 0 || slot != first_slot + (t & (page - 1)))
          bad |= 1 << k;
      }
      if (bad) atomicOr(a.page_flags, bad);
    }
  }
}

// Pass 3, one thread per row: a later row writing an earlier row's slot gets
// code 4; the first row of a sequence whose prefix failed gets 6 (missing)
// or else 7 (aliased). A row keeps the first code it was given.
__global__ __launch_bounds__(kThreads) void finish_rows_kernel(NormArgs a) {
  for (int i = blockIdx.x * kThreads + threadIdx.x; i < a.rows; i += gridDim.x * kThreads) {
    if (a.status[i] != 0) continue;
    int code = 0;
    if (owner_of(a, a.out_locations[i]) != i) code = 4;
    const int s = a.row_seq[i];
    if (code == 0 && a.seq_first_row[s] == i) {
      const int bits = a.seq_bits[s];
      code = (bits & 1) ? 6 : (bits & 2) ? 7 : 0;
    }
    if (code) a.status[i] = code;
  }
}

__global__ __launch_bounds__(kThreads) void block_tables_kernel(const int32_t* mapping, int32_t requests,
                                                               int32_t context, int32_t page, int32_t* tables,
                                                               int32_t pages) {
  const int64_t n = (int64_t)requests * pages;
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < n; e += (int64_t)gridDim.x * kThreads) {
    const int64_t r = e / pages, k = e % pages;
    const int64_t t = k * page;
    int32_t v = -1;
    if (t < context) {
      const int32_t slot = mapping[r * context + t];
      v = slot >= 0 ? slot / page : -1;
    }
    tables[e] = v;
  }
}

int grid_for(int64_t n) { return (int)std::min<int64_t>(std::max<int64_t>((n + kThreads - 1) / kThreads, 1), 4096); }

uint32_t table_capacity(int32_t rows) {
  uint32_t cap = 64;
  while (cap < 2u * static_cast<uint32_t>(rows)) cap <<= 1;
  return cap;
}

// ---------------------------------------------------------------------------
// Page allocator
// ---------------------------------------------------------------------------
// One thread per new token. seq_meta[4 s .. 4 s + 3] = {prefix, length, first
// output index, first free page}: the first min(length, (-prefix) mod P)
// tokens continue the page ending at last_slots[s], the rest take pages
// free_pages[first free page + j / P] in order.
__global__ __launch_bounds__(kThreads) void alloc_slots_kernel(const int64_t* last_slots, const int64_t* free_pages,
                                                              const int64_t* meta, int32_t batch, int64_t page,
                                                              int64_t total, int64_t* out) {
  for (int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x; e < total; e += (int64_t)gridDim.x * kThreads) {
    const int s = last_at_or_below(meta + 2, 4, batch, e);
    const int64_t prefix = meta[4 * s], length = meta[4 * s + 1];
    const int64_t j = e - meta[4 * s + 2];
    const int64_t existing = std::min<int64_t>(length, (page - prefix % page) % page);
    if (j < existing) {
      out[e] = last_slots[s] + 1 + j;
    } else {
      const int64_t i = j - existing;
      out[e] = free_pages[meta[4 * s + 3] + i / page] * page + i % page;
    }
  }
}

// Released slots -> their pages, first occurrences in input order, in one
// workgroup. first[p] = smallest input index releasing page p; pages 1 ..
// max_pages are the pool's (page 0 is reserved). count[0] = number of
// distinct pages, or -1 when a slot lies outside the pool.
constexpr int kReleaseThreads = 1024;

__global__ __launch_bounds__(kReleaseThreads) void release_slots_kernel(const int64_t* slots, int64_t n,
                                                                       int64_t page, int64_t max_pages,
                                                                       int32_t* first, int64_t* out_pages,
                                                                       int32_t* count) {
  __shared__ int32_t s_scan[kReleaseThreads];
  __shared__ int32_t s_bad;
  const int tid = threadIdx.x;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  for (int64_t i = tid; i < n; i += kReleaseThreads) {
    const int64_t s = slots[i];
    const int64_t p = s >= 0 ? s / page : -1;
    if (p < 1 || p > max_pages) atomicOr(&s_bad, 1);
    else atomicMin(first + p, static_cast<int32_t>(i));
  }
  __syncthreads();
  if (s_bad) {
    if (tid == 0) count[0] = -1;
    return;
  }
  int32_t base = 0;
  for (int64_t c0 = 0; c0 < n; c0 += kReleaseThreads) {
    const int64_t i = c0 + tid;
    int64_t p = 0;
    int flag = 0;
    if (i < n) {
      p = slots[i] / page;
      flag = coherent_load(first + p) == static_cast<int32_t>(i);
    }
    s_scan[tid] = flag;
    __syncthreads();
    for (int d = 1; d < kReleaseThreads; d <<= 1) {
      const int v = tid >= d ? s_scan[tid - d] : 0;
      __syncthreads();
      s_scan[tid] += v;
      __syncthreads();
    }
    if (flag) out_pages[base + s_scan[tid] - 1] = p;
    base += s_scan[kReleaseThreads - 1];
    __syncthreads();
  }
  if (tid == 0) count[0] = base;
}

}  // namespace
}  // namespace gk

using gk::fail;

extern "C" size_t gk_metadata_workspace_bytes(int32_t rows, int32_t batch) {
  if (rows <= 0 || batch <= 0) return 0;
  const size_t cap = gk::table_capacity(rows);
  return (cap * 2 + static_cast<size_t>(batch)) * sizeof(int32_t);
}

extern "C" int gk_metadata_normalize(const gk_metadata_params* p, void* workspace, size_t workspace_bytes,
                                     hipStream_t stream) {
  gk::clear_error();
  if (!p) return fail(GK_ERR_INVALID_ARGUMENT, "gk_metadata_normalize: null parameters");
  if (p->struct_size != sizeof(gk_metadata_params))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_metadata_normalize: struct_size does not match this library");
  if (p->rows <= 0 || p->rows > (1 << 24) || p->padded_rows < p->rows || p->padded_rows > (1 << 25) ||
      p->batch <= 0 || p->batch > p->rows || p->requests <= 0 || p->context <= 0 || p->slots <= 0 ||
      p->slots > INT32_MAX || (int64_t)p->requests * p->context > INT32_MAX || p->vocabulary < 0 ||
      p->visible_total < 0 || (p->token_ids && p->vocabulary <= 0))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_metadata_normalize: dimensions outside supported range");
  const bool checks = p->mapping && p->status;
  if (!p->locations || !p->batch_requests || !p->positions || !p->row_seq || !p->seq_prefix ||
      !p->seq_first_row || !p->out_locations || !p->out_requests || !p->out_positions ||
      (p->token_ids && !p->out_tokens) || (p->page_flags && !p->mapping) ||
      ((checks || p->page_flags) && p->visible_total > 0 && !p->seq_visible))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_metadata_normalize: null pointer");
  // Staged words: where each input that points into them starts, as a word
  // offset; an input only partly inside, or an input the kernel does not
  // redirect (or an output) inside, is refused.
  gk::Staged<true> st{};
  if (p->staged_words || p->staged_device || p->staged_count) {
    if (!p->staged_words || !p->staged_device || p->staged_count <= 0 ||
        p->staged_count > GK_METADATA_INLINE_WORDS)
      return fail(GK_ERR_INVALID_ARGUMENT, "gk_metadata_normalize: staged words need a host pointer, a device "
                                           "pointer and 1 to " + std::to_string(GK_METADATA_INLINE_WORDS) + " words");
    const uintptr_t lo = reinterpret_cast<uintptr_t>(p->staged_device);
    const uintptr_t hi = lo + static_cast<uintptr_t>(p->staged_count) * sizeof(int32_t);
    const auto inside = [&](const void* q) {
      const uintptr_t a = reinterpret_cast<uintptr_t>(q);
      return q && a >= lo && a < hi;
    };
    bool bad = false;
    const auto offset = [&](const void* q, int64_t words) -> int32_t {
      if (!inside(q)) return -1;
      const uintptr_t a = reinterpret_cast<uintptr_t>(q);
      if ((a - lo) % sizeof(int32_t) || a + static_cast<uintptr_t>(words) * sizeof(int32_t) > hi) bad = true;
      return static_cast<int32_t>((a - lo) / sizeof(int32_t));
    };
    st.device = p->staged_device;
    st.count = p->staged_count;
    st.row_seq = offset(p->row_seq, p->rows);
    st.seq_prefix = offset(p->seq_prefix, p->batch);
    st.seq_first_row = offset(p->seq_first_row, p->batch);
    st.positions = offset(p->positions, static_cast<int64_t>(p->rows) * (p->positions_int64 ? 2 : 1));
    for (const void* q : {p->locations, p->batch_requests, p->token_ids, static_cast<const void*>(p->mapping),
                          static_cast<const void*>(p->out_locations), static_cast<const void*>(p->out_requests),
                          static_cast<const void*>(p->out_positions), static_cast<const void*>(p->out_tokens),
                          static_cast<const void*>(p->status), static_cast<const void*>(p->token_status),
                          static_cast<const void*>(p->page_flags)})
      bad = bad || inside(q);
    if (bad)
      return fail(GK_ERR_INVALID_ARGUMENT,
                  "gk_metadata_normalize: an input or output overlaps the staged words in an unsupported way");
    std::memcpy(st.words, p->staged_words, static_cast<size_t>(p->staged_count) * sizeof(int32_t));
  }
  const size_t need = checks ? gk_metadata_workspace_bytes(p->rows, p->batch) : 0;
  if (checks && (workspace_bytes < need || !workspace))
    return fail(GK_ERR_WORKSPACE, "gk_metadata_normalize: workspace too small (" + std::to_string(need) + " bytes)");
  gk::NormArgs a{};
  a.locations = p->locations;
  a.batch_requests = p->batch_requests;
  a.positions = p->positions;
  a.token_ids = p->token_ids;
  a.loc64 = p->locations_int64;
  a.req64 = p->requests_int64;
  a.pos64 = p->positions_int64;
  a.tok64 = p->tokens_int64;
  a.mapping = checks ? p->mapping : nullptr;
  a.row_seq = p->row_seq;
  a.seq_prefix = p->seq_prefix;
  a.seq_first_row = p->seq_first_row;
  a.seq_visible = p->seq_visible;
  a.visible_total = p->visible_total;
  a.rows = p->rows;
  a.padded_rows = p->padded_rows;
  a.batch = p->batch;
  a.requests = p->requests;
  a.context = p->context;
  a.vocabulary = p->vocabulary;
  a.slots = p->slots;
  a.out_locations = p->out_locations;
  a.out_requests = p->out_requests;
  a.out_positions = p->out_positions;
  a.out_tokens = p->out_tokens;
  a.status = p->status;
  a.token_status = p->token_ids ? p->token_status : nullptr;
  a.page_flags = p->page_flags;
  if (checks) {
    const uint32_t cap = gk::table_capacity(p->rows);
    a.table_keys = static_cast<int32_t*>(workspace);
    a.table_rows = a.table_keys + cap;
    a.seq_bits = a.table_rows + cap;
    a.table_mask = cap - 1;
    gk::fill_kernel<<<gk::grid_for(cap), gk::kThreads, 0, stream>>>(a.table_keys, cap, -1);
    gk::fill_kernel<<<gk::grid_for(cap), gk::kThreads, 0, stream>>>(a.table_rows, cap, INT_MAX);
    gk::fill_kernel<<<gk::grid_for(p->batch), gk::kThreads, 0, stream>>>(a.seq_bits, p->batch, 0);
  }
  if (p->page_flags) gk::fill_kernel<<<1, gk::kThreads, 0, stream>>>(p->page_flags, 1, 0);
  if (st.count)
    gk::normalize_rows_kernel<true><<<gk::grid_for(p->padded_rows), gk::kThreads, 0, stream>>>(a, st);
  else
    gk::normalize_rows_kernel<false><<<gk::grid_for(p->padded_rows), gk::kThreads, 0, stream>>>(a, {});
  if ((checks || p->page_flags) && p->visible_total > 0) {
    gk::NormArgs b = a;
    b.mapping = p->mapping;
    gk::prefix_kernel<<<gk::grid_for(p->visible_total), gk::kThreads, 0, stream>>>(b);
  }
  if (checks) gk::finish_rows_kernel<<<gk::grid_for(p->rows), gk::kThreads, 0, stream>>>(a);
  return gk::hip_status(hipGetLastError(), "gk_metadata_normalize launch");
}

extern "C" int gk_block_tables(const int32_t* mapping, int32_t requests, int32_t context, int32_t page_size,
                               int32_t* tables, int32_t pages, hipStream_t stream) {
  gk::clear_error();
  if (requests <= 0 || context <= 0 || pages <= 0 || !gk::is_pow2(page_size) || page_size > 1024 ||
      (int64_t)requests * context > INT32_MAX || (int64_t)requests * pages > INT32_MAX)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_block_tables: invalid geometry");
  if (!mapping || !tables) return fail(GK_ERR_INVALID_ARGUMENT, "gk_block_tables: null pointer");
  gk::block_tables_kernel<<<gk::grid_for((int64_t)requests * pages), gk::kThreads, 0, stream>>>(
      mapping, requests, context, page_size, tables, pages);
  return gk::hip_status(hipGetLastError(), "gk_block_tables launch");
}

extern "C" int gk_paged_alloc_slots(const int64_t* last_slots, const int64_t* free_pages, const int64_t* seq_meta,
                                    int32_t batch, int64_t page_size, int64_t total, int64_t* out_slots,
                                    hipStream_t stream) {
  gk::clear_error();
  if (batch <= 0 || page_size < 1 || page_size > INT32_MAX || total <= 0 || total > ((int64_t)1 << 30))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_alloc_slots: invalid geometry");
  if (!last_slots || !free_pages || !seq_meta || !out_slots)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_alloc_slots: null pointer");
  gk::alloc_slots_kernel<<<gk::grid_for(total), gk::kThreads, 0, stream>>>(last_slots, free_pages, seq_meta, batch,
                                                                           page_size, total, out_slots);
  return gk::hip_status(hipGetLastError(), "gk_paged_alloc_slots launch");
}

extern "C" size_t gk_paged_release_workspace_bytes(int64_t max_pages) {
  return max_pages > 0 && max_pages <= INT32_MAX ? (size_t)(max_pages + 1) * sizeof(int32_t) : 0;
}

extern "C" int gk_paged_release_slots(const int64_t* slots, int64_t n, int64_t page_size, int64_t max_pages,
                                      void* workspace, size_t workspace_bytes, int64_t* out_pages,
                                      int32_t* out_count, hipStream_t stream) {
  gk::clear_error();
  if (n <= 0 || n > ((int64_t)1 << 30) || page_size < 1 || page_size > INT32_MAX || max_pages <= 0 ||
      max_pages > INT32_MAX)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_release_slots: invalid release geometry");
  if (!slots || !out_pages || !out_count) return fail(GK_ERR_INVALID_ARGUMENT, "gk_paged_release_slots: null pointer");
  if (workspace_bytes < gk_paged_release_workspace_bytes(max_pages) || !workspace)
    return fail(GK_ERR_WORKSPACE, "gk_paged_release_slots: workspace too small");
  int32_t* first = static_cast<int32_t*>(workspace);
  gk::fill_kernel<<<gk::grid_for(max_pages + 1), gk::kThreads, 0, stream>>>(first, max_pages + 1, INT32_MAX);
  gk::release_slots_kernel<<<1, gk::kReleaseThreads, 0, stream>>>(slots, n, page_size, max_pages, first, out_pages,
                                                                   out_count);
  return gk::hip_status(hipGetLastError(), "gk_paged_release_slots launch");
}
