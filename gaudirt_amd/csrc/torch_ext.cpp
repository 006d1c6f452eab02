// PyTorch-ROCm binding of the paged-attention path: the reference's operator
// API for it (TORCH_LIBRARY gaudirt, src/bridge/generic_private_use1.cpp:430-489),
// with every device step going through the C ABI of libgaudirt_amd.so.
//
//   torch.classes.gaudirt.PagedMetadata   slot mapping, block tables, lengths
//   torch.ops.gaudirt.paged_attn          KV store + attention over the pool
//   torch.ops.gaudirt._paged_attn_validated
//   torch.ops.gaudirt._advance_decode_lengths
//   gaudirt_amd._C._allocate_paged_kv     head-major pool on the block allocator
//   gaudirt_amd._C._allocate_paged_slots / _release_paged_slots   page allocator
//
// Errors are TORCH_CHECK failures (RuntimeError in Python) raised before any
// KV byte is written, with the message fragments the reference's tests match.
#include <ATen/ATen.h>
#include <c10/core/Storage.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/custom_class.h>
#include <torch/extension.h>
#include <torch/library.h>

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <bit>
#include <cmath>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <numeric>
#include <unordered_map>
#include <utility>
#include <vector>

#include "gaudirt_amd.h"

namespace gaudirt_amd {
namespace {

void check_gk(int rc, const char* what) {
  TORCH_CHECK(rc == GK_OK, what, ": ", gk_last_error());
}

// Split-K partition of the decode rows of paged_attn. 0 (the default) leaves
// it to the library: the balanced schedule, whose split points depend on the
// whole batch, so a row's last bits can change with the rows around it. A
// fixed partition of that many keys (the partitioned kernel) makes every
// decode row's output a function of that row alone, bit for bit: the
// reference's single-row replay equals the batched row
// (tests/paged_attention_smoke.py:145-150).
std::atomic<int32_t> g_decode_partition{0};

hipStream_t current_stream() { return c10::hip::getCurrentHIPStream().stream(); }

int current_device() {
  int dev = 0;
  TORCH_CHECK(hipGetDevice(&dev) == hipSuccess, "GaudiRT: no current HIP device");
  return dev;
}

at::TensorOptions device_int32() {
  return at::TensorOptions().device(at::Device(at::kCUDA, current_device())).dtype(at::kInt);
}

// Host words -> a device int32 tensor of `total` words (the first
// words.size() filled) on the current stream through pinned staging: the
// host does not wait for queued device work, and torch's host allocator
// keeps the staging block until the copy has run.
at::Tensor upload_words(const int32_t* words, int64_t count, int64_t total) {
  auto device = at::empty({total}, device_int32());
  if (count > 0) {
    auto host = at::empty({count}, at::TensorOptions().dtype(at::kInt).pinned_memory(true));
    std::memcpy(host.data_ptr<int32_t>(), words, count * sizeof(int32_t));
    device.narrow(0, 0, count).copy_(host, /*non_blocking=*/true);
  }
  return device;
}
at::Tensor upload_words(const std::vector<int32_t>& words, int64_t total) {
  return upload_words(words.data(), static_cast<int64_t>(words.size()), total);
}

// Allocator whose resize leaves new elements uninitialised, for host copies
// that are written in full right after (zero-filling a 1 MB request map first
// cost about as much as copying it).
template <class T>
struct UninitAllocator : std::allocator<T> {
  template <class U>
  struct rebind {
    using other = UninitAllocator<U>;
  };
  UninitAllocator() = default;
  template <class U>
  UninitAllocator(const UninitAllocator<U>&) noexcept {}
  template <class U>
  void construct(U* p) noexcept {
    ::new (static_cast<void*>(p)) U;
  }
  template <class U, class... A>
  void construct(U* p, A&&... a) {
    ::new (static_cast<void*>(p)) U(std::forward<A>(a)...);
  }
};
using HostWords = std::vector<int32_t, UninitAllocator<int32_t>>;

// Word offset of the next 256-byte aligned section of a packed int32 buffer.
int64_t reserve_words(int64_t& cursor, int64_t count) {
  const int64_t start = cursor;
  cursor += (count + 63) / 64 * 64;
  return start;
}

// ---------------------------------------------------------------------------
// Stream-ordered block allocator behind the KV pools (one per device).
// ---------------------------------------------------------------------------
std::mutex g_alloc_mutex;
std::array<gk_allocator*, 64> g_allocators{};

gk_allocator* device_allocator(int device) {
  TORCH_CHECK(device >= 0 && device < 64, "GaudiRT: invalid device index ", device);
  std::lock_guard<std::mutex> lock(g_alloc_mutex);
  if (!g_allocators[device]) {
    size_t free_bytes = 0, total_bytes = 0;
    c10::hip::HIPGuard guard(device);
    TORCH_CHECK(hipMemGetInfo(&free_bytes, &total_bytes) == hipSuccess, "GaudiRT: hipMemGetInfo failed");
    gk_allocator* a = nullptr;
    check_gk(gk_allocator_create(device, total_bytes, 256ull << 20, &a), "GaudiRT: KV allocator");
    g_allocators[device] = a;
  }
  return g_allocators[device];
}

struct PoolBlock {
  gk_allocator* allocator;
  void* base;
};

void free_pool_block(void* ctx) {
  auto* block = static_cast<PoolBlock*>(ctx);
  (void)gk_allocator_free(block->allocator, block->base);
  delete block;
}

// If `tensor` lives in a pool from the block allocator, record `stream` as a
// user so the block is fenced before any reuse on another stream.
void record_pool_stream(const at::Tensor& tensor, hipStream_t stream) {
  const auto& dp = tensor.storage().data_ptr();
  if (dp.get_deleter() != &free_pool_block) return;
  auto* block = static_cast<PoolBlock*>(dp.get_context());
  check_gk(gk_allocator_record_stream(block->allocator, block->base, stream), "GaudiRT: KV pool record_stream");
}

// allocate_paged_kv (src/bridge/paged_kv_pool.cpp:15-41): zeroed bf16
// [layers, 2, kv_heads, slots, head_dim]; layer l's key pool view is
// pool[l, 0].transpose(0, 1) -> [slots, kv_heads, head_dim], its value pool
// pool[l, 1].transpose(0, 1). The reference's 131072-slot descriptor cap is a
// Synapse artefact and is not kept; one head's K (or V) region must stay below
// 4 GiB (32-bit buffer offsets).
at::Tensor allocate_paged_kv(int64_t layers, int64_t slots, int64_t heads, int64_t head_dim) {
  TORCH_CHECK(layers > 0 && layers <= 4096 && slots > 0 && heads > 0 && heads <= 256 &&
                  (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
                  slots <= static_cast<int64_t>(std::numeric_limits<uint32_t>::max() / 2) / head_dim,
              "GaudiRT: unsupported head-major KV pool geometry");
  const uint64_t layer_bytes = 2ull * heads * slots * head_dim * sizeof(uint16_t);
  TORCH_CHECK(layer_bytes <= std::numeric_limits<uint64_t>::max() / static_cast<uint64_t>(layers),
              "GaudiRT: KV pool size overflow");
  const uint64_t bytes = layer_bytes * layers;
  const int device = current_device();
  gk_allocator* allocator = device_allocator(device);
  const hipStream_t stream = current_stream();
  void* base = nullptr;
  check_gk(gk_allocator_alloc(allocator, bytes, stream, &base), "GaudiRT: KV pool allocation");
  auto* block = new PoolBlock{allocator, base};
  c10::DataPtr data(base, block, &free_pool_block, at::Device(at::kCUDA, device));
  c10::Storage storage(c10::Storage::use_byte_size_t(), bytes, std::move(data), nullptr, false);
  auto pool = at::empty({0}, at::TensorOptions().device(at::kCUDA, device).dtype(at::kBFloat16));
  pool.set_(storage, 0, {layers, 2, heads, slots, head_dim},
            {2 * heads * slots * head_dim, heads * slots * head_dim, slots * head_dim, head_dim, 1});
  TORCH_CHECK(hipMemsetAsync(base, 0, bytes, stream) == hipSuccess, "GaudiRT: failed to initialize KV pool");
  return pool;
}

pybind11::dict allocator_stats(int64_t device) {
  gk_allocator_stats s{};
  check_gk(gk_allocator_get_stats(device_allocator(static_cast<int>(device)), &s), "GaudiRT: allocator stats");
  pybind11::dict d;
  d["allocated_bytes"] = s.allocated_bytes;
  d["peak_bytes"] = s.peak_bytes;
  d["reserved_bytes"] = s.reserved_bytes;
  d["largest_free_block"] = s.largest_free_block;
  d["slabs"] = s.slabs;
  d["events_created"] = s.events_created;
  return d;
}

// ---------------------------------------------------------------------------
// Attention plan: a device int32 tensor [row_request | row_context | block
// tables] whose DataPtr context owns the host-side schedule, so launches need
// no device-to-host read (the reference keeps its AttentionPlan the same way,
// src/bridge/attention_plan.cpp:31-34,132-140).
// ---------------------------------------------------------------------------
struct PlanInfo {
  int64_t rows = 0, query_heads = 0, kv_heads = 0, head_dim = 0, slots = 0;
  int64_t block_size = 1, bt_stride = 0, requests = 0, sliding_window = -1;
  int device = 0;
  hipStream_t stream = nullptr;
  at::Tensor storage;  // the plan's own device buffer
  int64_t block_table_offset = 0;
  // Read in place instead of from `storage` when defined: the token-granular
  // request map as the block tables (page 1), and the metadata's own row
  // requests when every row is a decode row in batch order.
  // requests, visible keys and the identity row map when every row is a
  // decode row in batch order (a serving decode step needs no plan upload).
  at::Tensor block_tables_ref, row_request_ref, row_context_ref;
  const int32_t* block_tables(const int32_t* words) const {
    return block_tables_ref.defined() ? block_tables_ref.data_ptr<int32_t>() : words + block_table_offset;
  }
  const int32_t* row_request(const int32_t* words) const {
    return row_request_ref.defined() ? row_request_ref.data_ptr<int32_t>() : words + row_request_offset;
  }
  const int32_t* row_context(const int32_t* words) const {
    return row_context_ref.defined() ? row_context_ref.data_ptr<int32_t>() : words + row_context_offset;
  }
  const int32_t* row_map(const int32_t* words) const {
    return row_context_ref.defined() ? nullptr : words + row_map_offset;
  }
  // Rows attended one by one (gk_paged_decode): request, visible keys and the
  // batch row of each.
  int64_t decode_rows = 0, decode_max_context = 0;
  int64_t row_request_offset = 0, row_context_offset = 0, row_map_offset = 0;
  // Runs of consecutive positions attended as MFMA tiles (gk_paged_prefill).
  int64_t prefill_seqs = 0, prefill_max_rows = 0;
  int64_t seq_request_offset = 0, seq_first_row_offset = 0, seq_rows_offset = 0, seq_prefix_offset = 0;
};

// Runs of at least this many consecutive positions go to the prefill kernel.
constexpr int64_t kPrefillMinRows = 8;

void release_plan(void* ctx) { delete static_cast<PlanInfo*>(ctx); }

at::Tensor make_plan_tensor(std::unique_ptr<PlanInfo> info) {
  const auto& buffer = info->storage;
  const auto nbytes = buffer.nbytes();
  const auto numel = buffer.numel();
  void* data = buffer.data_ptr();
  const auto device = buffer.device();
  c10::DataPtr dp(data, info.release(), &release_plan, device);
  c10::Storage storage(c10::Storage::use_byte_size_t(), nbytes, std::move(dp), nullptr, false);
  auto plan = at::empty({0}, at::TensorOptions().device(device).dtype(at::kInt));
  plan.set_(storage, 0, {numel}, {1});
  return plan;
}

const PlanInfo& plan_data(const at::Tensor& tensor) {
  TORCH_CHECK(tensor.is_cuda() && tensor.device().index() == current_device(),
              "GaudiRT attention: expected a device metadata plan");
  const auto& dp = tensor.storage().data_ptr();
  TORCH_CHECK(dp.get_deleter() == &release_plan && tensor.data_ptr() == dp.get(),
              "GaudiRT attention: invalid or expired metadata plan");
  return *static_cast<const PlanInfo*>(dp.get_context());
}

// ---------------------------------------------------------------------------
// PagedMetadata (src/bridge/paged_metadata.hpp:17-109). Host constructor
// src/bridge/paged_metadata.cpp:82-174; device constructors (from_device,
// from_device_with_tokens, _from_scheduler, _from_scheduler_fused)
// src/bridge/paged_metadata.cpp:176-430.
// ---------------------------------------------------------------------------
class PagedMetadata : public torch::CustomClassHolder {
 public:
  static constexpr int64_t kMaxRows = 8192;

  PagedMetadata(const at::Tensor& locations, const at::Tensor& requests, const at::Tensor& positions,
                const at::Tensor& mapping, int64_t slots) {
    for (const auto& tensor : {locations, requests, positions, mapping})
      TORCH_CHECK(tensor.device().is_cpu() && tensor.is_contiguous() &&
                      (tensor.scalar_type() == at::kInt || tensor.scalar_type() == at::kLong),
                  "GaudiRT: paged metadata must be contiguous CPU int32 or int64");
    TORCH_CHECK(locations.dim() == 1 && requests.dim() == 1 && positions.dim() == 1 && mapping.dim() == 2 &&
                    locations.size(0) == requests.size(0) && locations.size(0) == positions.size(0),
                "GaudiRT: invalid paged metadata ranks or row counts");
    const int64_t m = locations.size(0), request_count = mapping.size(0), context = mapping.size(1);
    TORCH_CHECK(m > 0 && m <= kMaxRows && slots > 0 && slots <= std::numeric_limits<int32_t>::max() &&
                    request_count > 0 && request_count <= std::numeric_limits<int32_t>::max() && context > 0 &&
                    context <= std::numeric_limits<int32_t>::max() &&
                    mapping.numel() <= std::numeric_limits<int32_t>::max(),
                "GaudiRT: paged metadata dimensions outside supported range");
    // The reference checks the whole request map first, then each row (the
    // first failing row reports its first failing check), then every visible
    // prefix in (request, position) order; the first failure of that order is
    // the one reported. Here the row checks read the map from the caller's
    // tensor, and one pass per request row copies and range-checks the row
    // and, while it is in cache, walks the request's visible prefix; faults
    // are recorded and raised in the reference's order after the pass.
    const int64_t map_n = mapping.numel();
    const bool map32 = mapping.scalar_type() == at::kInt;
    const auto map_at = [&](int64_t i) -> int64_t {
      return map32 ? mapping.data_ptr<int32_t>()[i] : mapping.data_ptr<int64_t>()[i];
    };
    const auto loc = locations.to(at::kLong), req = requests.to(at::kLong), pos = positions.to(at::kLong);
    const int64_t* loc_p = loc.data_ptr<int64_t>();
    const int64_t* req_p = req.data_ptr<int64_t>();
    const int64_t* pos_p = pos.data_ptr<int64_t>();
    enum RowFault : int { kRowOk = 0, kRowRange, kRowMismatch, kRowDuplicate };
    std::vector<int> fault(m, kRowOk);
    for (int64_t i = 0; i < m; ++i) {
      if (loc_p[i] < 0 || loc_p[i] >= slots || req_p[i] < 0 || req_p[i] >= request_count || pos_p[i] < 0 ||
          pos_p[i] >= context)
        fault[i] = kRowRange;
      else if (map_at(req_p[i] * context + pos_p[i]) != loc_p[i])
        fault[i] = kRowMismatch;
    }
    // Output slots sorted with their row: a slot's rows after its first are
    // duplicates, and the sorted list answers "which rows write slots in
    // [a, b)" below.
    std::vector<int64_t> by_slot(m);
    std::iota(by_slot.begin(), by_slot.end(), int64_t{0});
    std::sort(by_slot.begin(), by_slot.end(),
              [&](int64_t a, int64_t b) { return loc_p[a] != loc_p[b] ? loc_p[a] < loc_p[b] : a < b; });
    for (int64_t k = 1; k < m; ++k)
      if (loc_p[by_slot[k]] == loc_p[by_slot[k - 1]] && fault[by_slot[k]] == kRowOk) fault[by_slot[k]] = kRowDuplicate;
    const auto bad_row = std::find_if(fault.begin(), fault.end(), [](int f) { return f != kRowOk; });
    const bool rows_ok = bad_row == fault.end();
    if (rows_ok) {
      locations_h_.assign(loc_p, loc_p + m);
      requests_h_.assign(req_p, req_p + m);
      positions_h_.assign(pos_p, pos_p + m);
      max_position_.assign(request_count, -1);
      for (int64_t i = 0; i < m; ++i)
        max_position_[requests_h_[i]] = std::max(max_position_[requests_h_[i]], positions_h_[i]);
    }
    // Every request's visible prefix (positions up to its last row) must have
    // slots, none of them the output slot of another (request, position). The
    // prefix is walked as runs of consecutive slots (slot - position constant,
    // compared eight positions at a time); a run's slot range is looked up
    // among the written slots only when a 2^16-bit filter of them (slot mod
    // 2^16) has a bit in it. The same walk finds the page size of the map: the
    // largest power of two P <= 1024 such that each visible token t sits at
    // map[t - t % P] + t % P with map[t - t % P] a multiple of P. That holds
    // exactly when every run start (t = 0, or map[t] != map[t - 1] + 1) has
    // both t and map[t] divisible by P, so P is the lowest set bit of the OR
    // of those values.
    std::vector<uint64_t> written(1024, 0);
    for (int64_t i = 0; i < m; ++i) written[(loc_p[i] >> 6) & 1023] |= uint64_t{1} << (loc_p[i] & 63);
    const auto filter_hit = [&](int32_t first_slot, int64_t count) {
      uint32_t bit = static_cast<uint32_t>(first_slot) & 65535u;
      int64_t left = std::min<int64_t>(count, 65536);
      while (left > 0) {
        const uint32_t off = bit & 63u;
        const int64_t take = std::min<int64_t>(left, 64 - off);
        const uint64_t mask = (take == 64 ? ~uint64_t{0} : (uint64_t{1} << take) - 1) << off;
        if (written[bit >> 6] & mask) return true;
        left -= take;
        bit = (bit + static_cast<uint32_t>(take)) & 65535u;
      }
      return false;
    };
    enum PrefixFault : int { kPrefixOk = 0, kPrefixMissing, kPrefixAlias };
    int prefix_fault = kPrefixOk;
    uint32_t breaks = 0;
    const auto walk_prefix = [&](int64_t request) {
      const int32_t* row_map = mapping_h_.data() + request * context;
      const int32_t last = max_position_[request];
      int32_t p = 0;
      while (p <= last) {
        const int32_t s0 = row_map[p];
        if (s0 < 0) {
          prefix_fault = kPrefixMissing;
          return;
        }
        breaks |= static_cast<uint32_t>(p) | static_cast<uint32_t>(s0);
        const int32_t shift = s0 - p;  // slot - position along the run (slots are below 2^31 - 1)
        int32_t q = p + 1;
        while (int64_t{q} + 8 <= int64_t{last} + 1) {
          bool broken = false;
          for (int k = 0; k < 8; ++k) broken |= row_map[q + k] - (q + k) != shift;
          if (broken) break;
          q += 8;
        }
        while (q <= last && row_map[q] - q == shift) ++q;
        // Positions [p, q) hold slots [s0, s0 + q - p); their writers, in slot
        // (and so position) order, must be this request at that position.
        if (filter_hit(s0, q - p)) {
          auto it = std::lower_bound(by_slot.begin(), by_slot.end(), s0,
                                     [&](int64_t row, int32_t s) { return loc_p[row] < s; });
          for (; it != by_slot.end() && loc_p[*it] < static_cast<int64_t>(s0) + (q - p); ++it) {
            const int64_t position = p + (loc_p[*it] - s0);
            if (requests_h_[*it] != request || positions_h_[*it] != position) {
              prefix_fault = kPrefixAlias;
              return;
            }
          }
        }
        p = q;
      }
    };
    mapping_h_.resize(map_n);
    const uint32_t slot_limit = static_cast<uint32_t>(slots);
    uint32_t out_of_range = 0;
    for (int64_t request = 0; request < request_count; ++request) {
      int32_t* dst = mapping_h_.data() + request * context;
      if (map32) {
        // -1 <= slot < slots as one unsigned comparison (slots <= INT32_MAX).
        const int32_t* src = mapping.data_ptr<int32_t>() + request * context;
        for (int64_t t = 0; t < context; ++t) {
          const int32_t slot = src[t];
          dst[t] = slot;
          out_of_range |= static_cast<uint32_t>(static_cast<uint32_t>(slot) + 1u > slot_limit);
        }
      } else {
        const int64_t* src = mapping.data_ptr<int64_t>() + request * context;
        for (int64_t t = 0; t < context; ++t) {
          const int64_t slot = src[t];
          dst[t] = static_cast<int32_t>(slot);
          out_of_range |= static_cast<uint32_t>(slot < -1 || slot >= slots);
        }
      }
      if (rows_ok && !out_of_range && prefix_fault == kPrefixOk && max_position_[request] >= 0) walk_prefix(request);
    }
    TORCH_CHECK(!out_of_range, "GaudiRT: request-to-token slot is out of range");
    if (!rows_ok) {
      TORCH_CHECK(*bad_row != kRowRange, "GaudiRT: paged metadata index is out of range");
      TORCH_CHECK(*bad_row != kRowMismatch, "GaudiRT: output slot does not match request-to-token mapping");
      TORCH_CHECK(false, "GaudiRT: duplicate output KV slot");
    }
    TORCH_CHECK(prefix_fault != kPrefixMissing, "GaudiRT: missing KV slot in a visible prefix");
    TORCH_CHECK(prefix_fault != kPrefixAlias, "GaudiRT: output KV slot aliases another visible prefix position");
    // Runs of consecutive positions of one request, from their boundaries.
    std::vector<int32_t> run_starts;
    for (int64_t i = 0; i < m; ++i)
      if (i == 0 || requests_h_[i] != requests_h_[i - 1] || positions_h_[i] != positions_h_[i - 1] + 1)
        run_starts.push_back(static_cast<int32_t>(i));
    run_starts.push_back(static_cast<int32_t>(m));
    for (size_t k = 0; k + 1 < run_starts.size(); ++k)
      sequences_.push_back({run_starts[k], run_starts[k + 1] - run_starts[k], positions_h_[run_starts[k]]});
    page_ = 1024;
    while (page_ > 1 && (breaks & static_cast<uint32_t>(page_ - 1))) page_ >>= 1;
    rows_ = m;
    slots_ = slots;
    request_count_ = request_count;
    context_ = context;
    // One device buffer: header | locations | requests | positions. The request
    // map goes to the device only when something reads it there (the
    // token-granular plan or request_mapping()).
    int64_t cursor = 0;
    const auto header_offset = reserve_words(cursor, 1);
    const auto locations_offset = reserve_words(cursor, m);
    const auto requests_offset = reserve_words(cursor, m);
    const auto positions_offset = reserve_words(cursor, m);
    const auto row_context_offset = reserve_words(cursor, m);
    std::vector<int32_t> words(cursor, 0);
    words[header_offset] = static_cast<int32_t>(m);
    std::copy(locations_h_.begin(), locations_h_.end(), words.begin() + locations_offset);
    std::copy(requests_h_.begin(), requests_h_.end(), words.begin() + requests_offset);
    std::copy(positions_h_.begin(), positions_h_.end(), words.begin() + positions_offset);
    for (int64_t i = 0; i < m; ++i) words[row_context_offset + i] = positions_h_[i] + 1;
    storage_ = upload_words(words, cursor);
    header_ = storage_.narrow(0, header_offset, 1);
    locations_ = storage_.narrow(0, locations_offset, m);
    requests_ = storage_.narrow(0, requests_offset, m);
    positions_ = storage_.narrow(0, positions_offset, m);
    row_context_ = storage_.narrow(0, row_context_offset, m);
  }

  // Device constructor. Sequence s covers the next lengths[s] rows at
  // positions prefixes[s] + i of request batch_requests[s]. Unless
  // scheduler_owned, the rows are validated on the device and the host waits
  // for the per-row codes; scheduler-owned inputs are only normalised, with
  // no host wait.
  PagedMetadata(const at::Tensor& locations, const at::Tensor& batch_requests, const at::Tensor& positions,
                const at::Tensor& mapping, const std::vector<int64_t>& prefixes, const std::vector<int64_t>& lengths,
                int64_t slots, const at::Tensor& token_ids, int64_t vocabulary, bool scheduler_owned,
                bool fuse_scheduler_plan) {
    TORCH_CHECK(!fuse_scheduler_plan || scheduler_owned,
                "GaudiRT device metadata: fused plan requires scheduler-owned inputs");
    const int device = current_device();
    const auto on_device = [device](const at::Tensor& t) { return t.is_cuda() && t.device().index() == device; };
    const auto index_type = [](const at::Tensor& t) {
      return t.scalar_type() == at::kInt || t.scalar_type() == at::kLong;
    };
    for (const auto& tensor : {locations, batch_requests})
      TORCH_CHECK(on_device(tensor) && tensor.dim() == 1 && index_type(tensor),
                  "GaudiRT device metadata: expected gaudirt int32 or int64 vectors");
    const bool positions_on_cpu = fuse_scheduler_plan && positions.device().is_cpu();
    TORCH_CHECK(positions.dim() == 1 &&
                    ((positions_on_cpu && positions.scalar_type() == at::kLong && positions.is_contiguous()) ||
                     (on_device(positions) && index_type(positions))),
                "GaudiRT device metadata: invalid position input");
    TORCH_CHECK(on_device(mapping) && mapping.scalar_type() == at::kInt && mapping.dim() == 2 && mapping.is_contiguous(),
                "GaudiRT device metadata: expected a contiguous gaudirt int32 request map");
    const int64_t m = locations.numel(), batch = batch_requests.numel();
    const int64_t request_count = mapping.size(0), context = mapping.size(1);
    const bool has_tokens = token_ids.defined();
    TORCH_CHECK((has_tokens && on_device(token_ids) && token_ids.dim() == 1 && token_ids.numel() == m &&
                 index_type(token_ids) && vocabulary > 0 && vocabulary <= std::numeric_limits<int32_t>::max()) ||
                    (!has_tokens && vocabulary == 0),
                "GaudiRT device metadata: invalid token ID inputs or vocabulary");
    TORCH_CHECK(m > 0 && m <= kMaxRows && positions.numel() == m && batch > 0 && batch <= m &&
                    static_cast<int64_t>(prefixes.size()) == batch && static_cast<int64_t>(lengths.size()) == batch &&
                    slots > 0 && slots <= std::numeric_limits<int32_t>::max() && request_count > 0 &&
                    request_count <= std::numeric_limits<int32_t>::max() && context > 0 &&
                    context <= std::numeric_limits<int32_t>::max() &&
                    mapping.numel() <= std::numeric_limits<int32_t>::max(),
                "GaudiRT device metadata: dimensions outside supported range");
    const int64_t bucket = static_cast<int64_t>(std::bit_ceil(static_cast<uint64_t>(m)));
    // Sequence s owns rows [seq_first[s], seq_first[s] + lengths[s]) at positions
    // prefixes[s] + i; seq_visible[s] counts the visible keys of the earlier
    // sequences. Each sequence is checked as its rows are laid out, so the
    // first bad one is reported.
    std::vector<int32_t> seq_first(batch + 1, 0), seq_prefix(batch), last(batch), row_seq(m);
    std::vector<int64_t> seq_visible(batch + 1, 0);
    positions_h_.assign(m, 0);
    for (int64_t s = 0; s < batch; ++s) {
      const int64_t prefix = prefixes[s], length = lengths[s], row0 = seq_first[s];
      TORCH_CHECK(prefix >= 0 && prefix < context && length > 0 && length <= context - prefix && length <= m - row0,
                  "GaudiRT device metadata: invalid sequence lengths");
      seq_first[s + 1] = static_cast<int32_t>(row0 + length);
      seq_visible[s + 1] = seq_visible[s] + prefix + length;
      seq_prefix[s] = static_cast<int32_t>(prefix);
      last[s] = seq_first[s + 1] - 1;
      std::fill(row_seq.begin() + row0, row_seq.begin() + row0 + length, static_cast<int32_t>(s));
      std::iota(positions_h_.begin() + row0, positions_h_.begin() + row0 + length, static_cast<int32_t>(prefix));
      sequences_.push_back({static_cast<int32_t>(row0), static_cast<int32_t>(length), static_cast<int32_t>(prefix)});
    }
    TORCH_CHECK(seq_first[batch] == m, "GaudiRT device metadata: sequence lengths do not cover token rows");
    if (positions_on_cpu)
      TORCH_CHECK(std::equal(positions_h_.begin(), positions_h_.end(), positions.data_ptr<int64_t>()),
                  "GaudiRT device metadata: host position does not match scheduler lengths");
    const int64_t visible = seq_visible[batch];
    seq_first.pop_back();
    seq_visible.pop_back();
    // One buffer: host-staged words first (one copy), then the device outputs.
    int64_t words = 0;
    const auto header_offset = reserve_words(words, 1);
    const auto last_offset = reserve_words(words, batch);
    const auto row_seq_offset = reserve_words(words, m);
    const auto prefix_offset = reserve_words(words, batch);
    const auto first_offset = reserve_words(words, batch);
    const auto visible_offset = reserve_words(words, 2 * batch);
    const auto row_context_offset = reserve_words(words, m);
    const auto model_offset = positions_on_cpu ? reserve_words(words, 2 * m) : 0;
    const auto staged_words = words;
    const auto locations_offset = reserve_words(words, bucket);
    const auto requests_offset = reserve_words(words, bucket);
    const auto positions_offset = reserve_words(words, bucket);
    const auto tokens_offset = has_tokens ? reserve_words(words, bucket) : 0;
    // Codes, token codes and page flags are adjacent: one read-back.
    const auto status_offset = scheduler_owned ? 0 : reserve_words(words, 2 * bucket + 1);
    std::vector<int32_t> host(staged_words, 0);
    host[header_offset] = static_cast<int32_t>(m);
    for (int64_t i = 0; i < m; ++i) host[row_context_offset + i] = positions_h_[i] + 1;
    std::copy(last.begin(), last.end(), host.begin() + last_offset);
    std::copy(row_seq.begin(), row_seq.end(), host.begin() + row_seq_offset);
    std::copy(seq_prefix.begin(), seq_prefix.end(), host.begin() + prefix_offset);
    std::copy(seq_first.begin(), seq_first.end(), host.begin() + first_offset);
    std::memcpy(host.data() + visible_offset, seq_visible.data(), batch * sizeof(int64_t));
    if (positions_on_cpu) std::memcpy(host.data() + model_offset, positions.data_ptr<int64_t>(), m * sizeof(int64_t));
    // Up to GK_METADATA_INLINE_WORDS staged words travel in the normalisation
    // launch's arguments (no upload); more go through pinned staging.
    const bool inline_staged = staged_words <= GK_METADATA_INLINE_WORDS;
    storage_ = inline_staged ? at::empty({words}, device_int32()) : upload_words(host, words);
    int32_t* base = storage_.data_ptr<int32_t>();
    header_ = storage_.narrow(0, header_offset, 1);
    last_token_indices_ = storage_.narrow(0, last_offset, batch);
    locations_ = storage_.narrow(0, locations_offset, m);
    requests_ = storage_.narrow(0, requests_offset, m);
    positions_ = storage_.narrow(0, positions_offset, m);
    row_context_ = storage_.narrow(0, row_context_offset, m);
    if (has_tokens) token_ids_ = storage_.narrow(0, tokens_offset, m);
    if (positions_on_cpu)
      model_positions_ = storage_.narrow(0, model_offset, 2 * m).view(at::kLong);
    else if (fuse_scheduler_plan)
      model_positions_ = positions;
    mapping_ = mapping;
    rows_ = m;
    slots_ = slots;
    request_count_ = request_count;
    context_ = context;
    vocabulary_ = vocabulary;

    // Strided inputs are packed first (the kernels read dense vectors).
    const auto dense = [](const at::Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); };
    const auto loc = dense(locations), req = dense(batch_requests);
    const auto pos = positions_on_cpu ? model_positions_ : dense(positions);
    const auto tok = has_tokens ? dense(token_ids) : at::Tensor();
    gk_metadata_params p{};
    p.struct_size = sizeof(p);
    p.locations = loc.data_ptr();
    p.locations_int64 = loc.scalar_type() == at::kLong;
    p.batch_requests = req.data_ptr();
    p.requests_int64 = req.scalar_type() == at::kLong;
    p.positions = pos.data_ptr();
    p.positions_int64 = pos.scalar_type() == at::kLong;
    p.token_ids = has_tokens ? tok.data_ptr() : nullptr;
    p.tokens_int64 = has_tokens && tok.scalar_type() == at::kLong;
    p.row_seq = base + row_seq_offset;
    p.seq_prefix = base + prefix_offset;
    p.seq_first_row = base + first_offset;
    p.seq_visible = reinterpret_cast<const int64_t*>(base + visible_offset);
    p.visible_total = visible;
    p.rows = static_cast<int32_t>(m);
    p.padded_rows = static_cast<int32_t>(bucket);
    p.batch = static_cast<int32_t>(batch);
    p.requests = static_cast<int32_t>(request_count);
    p.context = static_cast<int32_t>(context);
    p.vocabulary = static_cast<int32_t>(vocabulary);
    p.slots = slots;
    p.out_locations = base + locations_offset;
    p.out_requests = base + requests_offset;
    p.out_positions = base + positions_offset;
    p.out_tokens = has_tokens ? base + tokens_offset : nullptr;
    if (inline_staged) {
      p.staged_words = host.data();
      p.staged_device = base;
      p.staged_count = static_cast<int32_t>(staged_words);
    }
    at::Tensor workspace;
    if (!scheduler_owned) {
      p.mapping = mapping.data_ptr<int32_t>();
      p.status = base + status_offset;
      p.token_status = base + status_offset + bucket;
      p.page_flags = base + status_offset + 2 * bucket;
      const size_t need = gk_metadata_workspace_bytes(p.rows, p.batch);
      workspace = at::empty({static_cast<int64_t>(need)}, mapping.options().dtype(at::kByte));
      check_gk(gk_metadata_normalize(&p, workspace.data_ptr(), need, current_stream()), "GaudiRT device metadata");
      // The reference's checked constructor also waits here for the codes.
      const auto flags = storage_.narrow(0, status_offset, 2 * bucket + 1).cpu();
      const int32_t* codes = flags.data_ptr<int32_t>();
      for (int64_t row = 0; row < m; ++row)
        TORCH_CHECK(codes[row] == 0, "GaudiRT device metadata: invalid scheduler metadata at row ", row, ", code ",
                    codes[row]);
      if (has_tokens)
        for (int64_t row = 0; row < m; ++row)
          TORCH_CHECK(codes[bucket + row] == 0, "GaudiRT device metadata: token ID outside vocabulary at row ", row);
      page_ = 1;
      for (int k = 9; k >= 0; --k)
        if (!(codes[2 * bucket] & (1 << k))) {
          page_ = int64_t{2} << k;
          break;
        }
    } else {
      check_gk(gk_metadata_normalize(&p, nullptr, 0, current_stream()), "GaudiRT device metadata");
      page_ = 1;  // no host wait: the plan reads the token-granular map
    }
  }

  static c10::intrusive_ptr<PagedMetadata> from_device(const at::Tensor& locations, const at::Tensor& batch_requests,
                                                       const at::Tensor& positions, const at::Tensor& mapping,
                                                       std::vector<int64_t> prefixes, std::vector<int64_t> lengths,
                                                       int64_t slots) {
    return c10::make_intrusive<PagedMetadata>(locations, batch_requests, positions, mapping, prefixes, lengths, slots,
                                              at::Tensor(), 0, false, false);
  }
  static c10::intrusive_ptr<PagedMetadata> from_device_with_tokens(
      const at::Tensor& locations, const at::Tensor& batch_requests, const at::Tensor& positions,
      const at::Tensor& mapping, std::vector<int64_t> prefixes, std::vector<int64_t> lengths, int64_t slots,
      const at::Tensor& token_ids, int64_t vocabulary) {
    return c10::make_intrusive<PagedMetadata>(locations, batch_requests, positions, mapping, prefixes, lengths, slots,
                                              token_ids, vocabulary, false, false);
  }
  // Scheduler inputs were checked at request entry; slots and request maps
  // come from the scheduler's own pools.
  static c10::intrusive_ptr<PagedMetadata> from_scheduler(const at::Tensor& locations, const at::Tensor& batch_requests,
                                                          const at::Tensor& positions, const at::Tensor& mapping,
                                                          std::vector<int64_t> prefixes, std::vector<int64_t> lengths,
                                                          int64_t slots, const c10::optional<at::Tensor>& token_ids,
                                                          int64_t vocabulary) {
    return c10::make_intrusive<PagedMetadata>(locations, batch_requests, positions, mapping, prefixes, lengths, slots,
                                              token_ids.value_or(at::Tensor()), vocabulary, true, false);
  }
  static c10::intrusive_ptr<PagedMetadata> from_scheduler_fused(
      const at::Tensor& locations, const at::Tensor& batch_requests, const at::Tensor& positions,
      const at::Tensor& mapping, std::vector<int64_t> prefixes, std::vector<int64_t> lengths, int64_t slots,
      const c10::optional<at::Tensor>& token_ids, int64_t vocabulary, int64_t query_heads, int64_t kv_heads,
      int64_t head_dim) {
    auto metadata = c10::make_intrusive<PagedMetadata>(locations, batch_requests, positions, mapping, prefixes, lengths,
                                                       slots, token_ids.value_or(at::Tensor()), vocabulary, true, true);
    metadata->attention_plan(query_heads, kv_heads, head_dim);
    return metadata;
  }

  int64_t rows() const { return rows_; }
  int64_t slots() const { return slots_; }
  int64_t context() const { return context_; }
  at::Tensor rotary_positions() const { return positions_; }
  at::Tensor rotary_header() const { return header_; }
  at::Tensor row_locations() const { return locations_; }
  at::Tensor row_requests() const { return requests_; }
  at::Tensor request_mapping() { return device_mapping(); }
  at::Tensor model_positions() const {
    TORCH_CHECK(model_positions_.defined(), "GaudiRT: model positions require fused scheduler metadata");
    return model_positions_;
  }
  at::Tensor last_token_indices() const {
    TORCH_CHECK(last_token_indices_.defined(), "GaudiRT: last-token indices require batched metadata");
    return last_token_indices_;
  }
  at::Tensor token_ids() const {
    TORCH_CHECK(token_ids_.defined(), "GaudiRT: token IDs were not validated in this metadata");
    return token_ids_;
  }
  int64_t vocabulary() const { return vocabulary_; }
  std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, int64_t>
  forward_tensors(int64_t query_heads, int64_t kv_heads, int64_t head_dim) {
    return {token_ids(), last_token_indices(), rotary_positions(), rotary_header(), row_locations(),
            row_requests(), attention_plan(query_heads, kv_heads, head_dim), context_};
  }

  at::Tensor attention_plan(int64_t query_heads, int64_t kv_heads, int64_t head_dim) {
    return attention_plan_for(query_heads, kv_heads, head_dim, -1);
  }

  // attention_plan_for (src/bridge/attention_plan.cpp:146-172 for the checks).
  at::Tensor attention_plan_for(int64_t query_heads, int64_t kv_heads, int64_t head_dim, int64_t sliding_window) {
    TORCH_CHECK(sliding_window == -1 || (sliding_window > 0 && sliding_window <= std::numeric_limits<int32_t>::max()),
                "GaudiRT attention: invalid sliding window size");
    const int64_t window = sliding_window > 0 ? sliding_window : -1;
    auto cached = plans_.find(window);
    if (cached != plans_.end()) {
      const auto& plan = plan_data(cached->second);
      TORCH_CHECK(plan.query_heads == query_heads && plan.kv_heads == kv_heads && plan.head_dim == head_dim,
                  "GaudiRT attention: metadata already bound to different head geometry");
      return cached->second;
    }
    TORCH_CHECK(query_heads > 0 && query_heads <= 1024 && kv_heads > 0 && kv_heads <= 256 &&
                    query_heads % kv_heads == 0 && (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
                    slots_ > 0 && slots_ <= static_cast<int64_t>(std::numeric_limits<uint32_t>::max() / 2) / head_dim,
                "GaudiRT attention: unsupported head or request-map geometry");
    auto info = std::make_unique<PlanInfo>();
    info->rows = rows_;
    info->query_heads = query_heads;
    info->kv_heads = kv_heads;
    info->head_dim = head_dim;
    info->slots = slots_;
    info->requests = request_count_;
    info->sliding_window = window;
    info->device = current_device();
    info->stream = current_stream();
    // Block tables: the largest power-of-two page P (<= 1024) for which every
    // visible token t of every request sits at mapping[r, t - t % P] + t % P
    // with a P-aligned page start; P = 1 keeps the token-granular map.
    const bool host_map = !mapping_h_.empty();
    const int64_t page = page_;
    const int64_t max_pages = std::max<int64_t>(1, (context_ + page - 1) / page);
    // Split the rows: runs of >= kPrefillMinRows consecutive positions become
    // prefill sequences (MFMA tiles of rows x heads) when the prefill kernel
    // supports the geometry; every other row is a decode row. The requests of
    // device-built metadata are filled in on the device below.
    // The prefill kernel takes any page size, the token-granular map included.
    const bool prefill_ok = query_heads / kv_heads <= 128;
    std::vector<int32_t> dec_request, dec_context, dec_map, seq_request, seq_first, seq_rows, seq_prefix;
    for (const auto& run : sequences_) {
      if (prefill_ok && run.length >= kPrefillMinRows) {
        seq_request.push_back(host_map ? requests_h_[run.row] : 0);
        seq_first.push_back(run.row);
        seq_rows.push_back(run.length);
        seq_prefix.push_back(run.prefix);
        info->prefill_max_rows = std::max<int64_t>(info->prefill_max_rows, run.length);
        continue;
      }
      for (int32_t i = run.row; i < run.row + run.length; ++i) {
        dec_request.push_back(host_map ? requests_h_[i] : 0);
        dec_context.push_back(positions_h_[i] + 1);
        dec_map.push_back(i);
        info->decode_max_context = std::max<int64_t>(info->decode_max_context, positions_h_[i] + 1);
      }
    }
    std::vector<int32_t> words;
    const auto append = [&](const std::vector<int32_t>& v) {
      while (words.size() % 4) words.push_back(0);  // 16-byte aligned sections
      const auto offset = static_cast<int64_t>(words.size());
      words.insert(words.end(), v.begin(), v.end());
      return offset;
    };
    info->decode_rows = static_cast<int64_t>(dec_map.size());
    // Every row a decode row, in batch order (a serving decode step): the
    // decode kernel reads the metadata's row requests directly.
    bool all_decode = info->decode_rows == rows_;
    for (int64_t i = 0; all_decode && i < info->decode_rows; ++i) all_decode = dec_map[i] == i;
    if (all_decode) {
      info->row_request_ref = requests_;
      info->row_context_ref = row_context_;
      dec_request.clear();
      dec_context.clear();
      dec_map.clear();
    }
    info->row_request_offset = append(dec_request);
    info->row_context_offset = append(dec_context);
    info->row_map_offset = append(dec_map);
    info->prefill_seqs = static_cast<int64_t>(seq_rows.size());
    info->seq_request_offset = append(seq_request);
    info->seq_first_row_offset = append(seq_first);
    info->seq_rows_offset = append(seq_rows);
    info->seq_prefix_offset = append(seq_prefix);
    // Page 1: the request map itself is the block table, read in place.
    std::vector<int32_t> tables;
    if (page == 1) {
      info->block_tables_ref = device_mapping();
    } else if (host_map) {
      tables.assign(request_count_ * max_pages, -1);
      for (int64_t r = 0; r < request_count_; ++r)
        for (int64_t t = 0; t <= max_position_[r]; t += page)
          tables[r * max_pages + t / page] = mapping_h_[r * context_ + t] / static_cast<int32_t>(page);
    }
    info->block_table_offset = append(tables);
    const int64_t total = host_map || page == 1 ? static_cast<int64_t>(words.size())
                                                : info->block_table_offset + request_count_ * max_pages;
    info->block_size = page;
    info->bt_stride = max_pages;
    // A plan whose sections are all read in place (a decode step over the
    // token-granular map) keeps the metadata's row contexts as its storage:
    // no allocation and no copy.
    info->storage = total == 0 && all_decode ? row_context_ : upload_words(words, total);
    if (!host_map) {
      auto& storage = info->storage;
      const auto section = [&](int64_t offset, int64_t count) { return storage.narrow(0, offset, count); };
      if (info->decode_rows && !all_decode)
        section(info->row_request_offset, info->decode_rows)
            .copy_(requests_.index_select(0, section(info->row_map_offset, info->decode_rows)));
      if (info->prefill_seqs)
        section(info->seq_request_offset, info->prefill_seqs)
            .copy_(requests_.index_select(0, section(info->seq_first_row_offset, info->prefill_seqs)));
      if (page != 1)
        check_gk(gk_block_tables(mapping_.data_ptr<int32_t>(), static_cast<int32_t>(request_count_),
                                 static_cast<int32_t>(context_), static_cast<int32_t>(page),
                                 storage.data_ptr<int32_t>() + info->block_table_offset,
                                 static_cast<int32_t>(max_pages), info->stream),
                 "GaudiRT attention: block tables");
    }
    auto plan = make_plan_tensor(std::move(info));
    plans_.emplace(window, plan);
    return plan;
  }

 private:
  struct Sequence {
    int32_t row, length, prefix;
  };

  // The request map on the device: the device constructors' own input, or
  // (host constructor) the host copy, uploaded on the current stream on first use.
  const at::Tensor& device_mapping() {
    if (!mapping_.defined())
      mapping_ = upload_words(mapping_h_.data(), static_cast<int64_t>(mapping_h_.size()), request_count_ * context_)
                     .view({request_count_, context_});
    return mapping_;
  }

  int64_t rows_ = 0, slots_ = 0, request_count_ = 0, context_ = 0, vocabulary_ = 0, page_ = 1;
  // Host copies (host constructor only; device metadata keeps positions_h_).
  std::vector<int32_t> locations_h_, requests_h_, positions_h_, max_position_;
  HostWords mapping_h_;  // the request map as constructed (host constructor only)
  std::vector<Sequence> sequences_;
  // row_context_: visible keys of each row (its position + 1), the decode
  // kernel's row_context when every row is a decode row.
  at::Tensor storage_, locations_, requests_, positions_, row_context_, mapping_, header_, token_ids_,
      last_token_indices_,
      model_positions_;
  std::unordered_map<int64_t, at::Tensor> plans_;
};

// Output storage of pow2(rows) rows rounded to 256 bytes, shaped [rows, width]
// (bucket_output, src/bridge/generic_private_use1.cpp:207-219).
at::Tensor bucket_output(const at::Tensor& like, int64_t rows, int64_t width) {
  const uint64_t bucket = std::bit_ceil(static_cast<uint64_t>(rows));
  const uint64_t bytes = (bucket * width * sizeof(uint16_t) + 255) & ~uint64_t{255};
  auto output = at::empty({static_cast<int64_t>(bytes / sizeof(uint16_t))}, like.options().dtype(at::kBFloat16));
  output.unsafeGetTensorImpl()->set_sizes_contiguous({rows, width});
  return output;
}

// Rows of a 2-D bf16 matrix as the kernels take them: 16-byte aligned, row
// stride a multiple of 8 elements, unit column stride; else a packed copy in
// fresh storage (contiguous() would hand back a contiguous view whose start is
// not 16-byte aligned unchanged).
at::Tensor kernel_rows(const at::Tensor& t) {
  const bool ok = t.stride(1) == 1 && t.stride(0) % 8 == 0 && t.stride(0) >= t.size(1) &&
                  (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15) == 0;
  return ok ? t : t.clone(at::MemoryFormat::Contiguous);
}

// paged_attn_validated / paged_attn_internal (src/bridge/paged_attention.cpp:164-347):
// store the rows' K/V into the pool, then attend every row over its request's
// visible keys.
// Rotary embedding fused into the KV store of an attention call: the cos/sin
// cache, the rows' positions and the rotation geometry.
struct RotarySpec {
  at::Tensor cache;      // bf16 [cache_rows, rotary_dim], contiguous
  at::Tensor positions;  // int32 [rows], device
  int64_t rotary_dim;
  bool neox;
};

at::Tensor paged_attn_impl(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                           const at::Tensor& key_pool, const at::Tensor& value_pool, const at::Tensor& locations,
                           const at::Tensor& plan_tensor, int64_t head_dim, double scale, double softcap,
                           int64_t sliding_window, const RotarySpec* rotary) {
  const auto& plan = plan_data(plan_tensor);
  const hipStream_t stream = current_stream();
  const float scale_f = static_cast<float>(scale), softcap_f = static_cast<float>(softcap);
  TORCH_CHECK(plan.stream == stream && std::isfinite(scale) && std::isfinite(scale_f) && scale_f > 0 &&
                  std::isfinite(softcap) && std::isfinite(softcap_f) && softcap_f >= 0.0f &&
                  (sliding_window == -1 || (sliding_window > 0 && sliding_window <= std::numeric_limits<int32_t>::max())) &&
                  head_dim == plan.head_dim,
              "GaudiRT attention: invalid scale, stream, or head dimension");
  TORCH_CHECK(plan.sliding_window <= 0 || plan.sliding_window == sliding_window,
              "GaudiRT attention: plan sliding_window mismatch");
  const int device = current_device();
  for (const auto& input : {query, key, value})
    TORCH_CHECK(input.is_cuda() && input.device().index() == device && input.scalar_type() == at::kBFloat16 &&
                    input.dim() == 2 && input.size(0) == plan.rows,
                "GaudiRT attention: Q/K/V must be BF16 device matrices with matching rows");
  TORCH_CHECK(query.size(1) == plan.query_heads * head_dim && key.size(1) == plan.kv_heads * head_dim &&
                  value.size(1) == key.size(1) && locations.dim() == 1 && locations.numel() == plan.rows &&
                  locations.scalar_type() == at::kInt && locations.is_cuda(),
              "GaudiRT attention: Q/K/V or slot dimensions do not match metadata");
  for (const auto& pool : {key_pool, value_pool})
    TORCH_CHECK(pool.is_cuda() && pool.device().index() == device && pool.scalar_type() == at::kBFloat16 &&
                    pool.dim() == 3 && pool.size(0) == plan.slots && pool.size(1) == plan.kv_heads &&
                    pool.size(2) == head_dim && pool.stride(0) == head_dim && pool.stride(1) == plan.slots * head_dim &&
                    pool.stride(2) == 1,
                "GaudiRT attention: head-major combined KV pool is required");
  const auto pool_address = reinterpret_cast<uintptr_t>(key_pool.data_ptr());
  const auto value_address = reinterpret_cast<uintptr_t>(value_pool.data_ptr());
  const uint64_t value_offset = static_cast<uint64_t>(plan.slots) * plan.kv_heads * head_dim * sizeof(uint16_t);
  const auto& pool_storage = key_pool.storage();
  const auto storage_base = reinterpret_cast<uintptr_t>(pool_storage.data());
  TORCH_CHECK(pool_storage.unsafeGetStorageImpl() == value_pool.storage().unsafeGetStorageImpl() &&
                  value_address == pool_address + value_offset && pool_address >= storage_base &&
                  pool_address % 256 == 0 &&
                  pool_address - storage_base + 2 * value_offset <= pool_storage.nbytes(),
              "GaudiRT attention: KV pool descriptor is not backed by combined storage");
  record_pool_stream(key_pool, stream);

  auto q = kernel_rows(query);
  const auto k = kernel_rows(key), v = kernel_rows(value);
  auto output = bucket_output(query, plan.rows, query.size(1));
  void* pool = key_pool.data_ptr();
  // KV store first, on the same stream: rows of one sequence attend each
  // other's new keys.
  if (!rotary) {
    check_gk(gk_kv_store(k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0), locations.data_ptr<int32_t>(),
                         static_cast<int32_t>(plan.rows), pool, plan.slots, static_cast<int32_t>(plan.kv_heads),
                         static_cast<int32_t>(head_dim), stream),
             "GaudiRT attention: KV store");
  } else {
    // Rotated keys go straight into the pool; the rotated queries feed the attention.
    auto q_rot = at::empty({plan.rows, query.size(1)}, query.options());
    gk_rotary_params r{};
    r.struct_size = sizeof(r);
    r.query = q.data_ptr();
    r.q_row_stride = q.stride(0);
    r.q_width = q.size(1);
    r.key = k.data_ptr();
    r.k_row_stride = k.stride(0);
    r.k_width = k.size(1);
    r.positions = rotary->positions.data_ptr();
    r.positions_int64 = 0;
    r.cos_sin = rotary->cache.data_ptr();
    r.cache_rows = rotary->cache.size(0);
    r.rows = static_cast<int32_t>(plan.rows);
    r.head_dim = static_cast<int32_t>(head_dim);
    r.rotary_dim = static_cast<int32_t>(rotary->rotary_dim);
    r.is_neox = rotary->neox ? 1 : 0;
    r.q_out = q_rot.data_ptr();
    r.q_out_row_stride = q_rot.stride(0);
    r.value = v.data_ptr();
    r.v_row_stride = v.stride(0);
    r.slot_mapping = locations.data_ptr<int32_t>();
    r.pool = pool;
    r.slots = plan.slots;
    r.kv_heads = static_cast<int32_t>(plan.kv_heads);
    check_gk(gk_rotary_kv_store(&r, stream), "GaudiRT attention: rotary KV store");
    q = q_rot;
  }
  const int32_t* words = plan.storage.data_ptr<int32_t>();
  const int32_t sw = sliding_window > 0 ? static_cast<int32_t>(sliding_window) : -1;
  if (plan.prefill_seqs) {
    gk_prefill_params f{};
    f.struct_size = sizeof(f);
    f.query = q.data_ptr();
    f.q_row_stride = q.stride(0);
    f.pool = pool;
    f.slots = plan.slots;
    f.block_tables = plan.block_tables(words);
    f.bt_stride = plan.bt_stride;
    f.block_size = static_cast<int32_t>(plan.block_size);
    f.seq_request = words + plan.seq_request_offset;
    f.seq_first_row = words + plan.seq_first_row_offset;
    f.seq_rows = words + plan.seq_rows_offset;
    f.seq_prefix = words + plan.seq_prefix_offset;
    f.seqs = static_cast<int32_t>(plan.prefill_seqs);
    f.max_rows = static_cast<int32_t>(plan.prefill_max_rows);
    f.q_heads = static_cast<int32_t>(plan.query_heads);
    f.kv_heads = static_cast<int32_t>(plan.kv_heads);
    f.head_dim = static_cast<int32_t>(head_dim);
    f.scale = scale_f;
    f.softcap = softcap_f;
    f.sliding_window = sw;
    f.out = output.data_ptr();
    f.out_row_stride = output.stride(0);
    check_gk(gk_paged_prefill(&f, stream), "GaudiRT attention (prefill)");
  }
  if (plan.decode_rows) {
    gk_decode_params p{};
    p.struct_size = sizeof(p);
    p.query = q.data_ptr();
    p.q_row_stride = q.stride(0);
    p.pool = pool;
    p.slots = plan.slots;
    p.block_tables = plan.block_tables(words);
    p.bt_stride = plan.bt_stride;
    p.block_size = static_cast<int32_t>(plan.block_size);
    p.row_request = plan.row_request(words);
    p.row_context = plan.row_context(words);
    p.row_map = plan.row_map(words);
    p.rows = static_cast<int32_t>(plan.decode_rows);
    p.q_heads = static_cast<int32_t>(plan.query_heads);
    p.kv_heads = static_cast<int32_t>(plan.kv_heads);
    p.head_dim = static_cast<int32_t>(head_dim);
    p.scale = scale_f;
    p.softcap = softcap_f;
    p.sliding_window = sw;
    p.max_context = static_cast<int32_t>(plan.decode_max_context);
    p.partition_tokens = g_decode_partition.load(std::memory_order_relaxed);
    p.out = output.data_ptr();
    p.out_row_stride = output.stride(0);
    const size_t need = gk_paged_decode_workspace_bytes(&p);
    at::Tensor workspace;
    if (need) workspace = at::empty({static_cast<int64_t>(need)}, query.options().dtype(at::kByte));
    check_gk(gk_paged_decode(&p, need ? workspace.data_ptr() : nullptr, need, stream), "GaudiRT attention");
  }
  return output;
}

// _paged_attn_validated (src/bridge/paged_attention.cpp:172-347).
at::Tensor paged_attn_validated(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                                const at::Tensor& key_pool, const at::Tensor& value_pool, const at::Tensor& locations,
                                const at::Tensor& requests, const at::Tensor& positions, const at::Tensor& plan_tensor,
                                const at::Tensor& header, int64_t head_dim, double scale, double softcap,
                                int64_t sliding_window) {
  (void)requests;
  (void)positions;
  (void)header;
  return paged_attn_impl(query, key, value, key_pool, value_pool, locations, plan_tensor, head_dim, scale, softcap,
                         sliding_window, nullptr);
}

// paged_attn (src/bridge/generic_private_use1.cpp:277-293).
at::Tensor paged_attn(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                      const at::Tensor& key_pool, const at::Tensor& value_pool,
                      const c10::intrusive_ptr<PagedMetadata>& metadata, int64_t head_dim, double scale, double softcap,
                      int64_t sliding_window) {
  TORCH_CHECK(metadata, "GaudiRT paged attention: metadata is required");
  TORCH_CHECK(query.dim() == 2 && key_pool.dim() == 3 && (head_dim == 64 || head_dim == 128 || head_dim == 256),
              "GaudiRT paged attention: invalid tensor ranks or head dimension");
  const auto q_heads = query.size(1) / head_dim;
  const auto kv_heads = key_pool.size(1);
  auto plan = sliding_window > 0 ? metadata->attention_plan_for(q_heads, kv_heads, head_dim, sliding_window)
                                 : metadata->attention_plan(q_heads, kv_heads, head_dim);
  return paged_attn_validated(query, key, value, key_pool, value_pool, metadata->row_locations(),
                              metadata->row_requests(), metadata->rotary_positions(), plan, metadata->rotary_header(),
                              head_dim, scale, softcap, sliding_window);
}

// ---------------------------------------------------------------------------
// Rotary position embedding
// ---------------------------------------------------------------------------

// Row limit of the bucketed rotary outputs (src/bridge/bucket_program.hpp:20).
constexpr int64_t kMaxBucketRows = 8192;

// A bf16 matrix as the rotary kernel takes it: unit column stride, any row stride.
at::Tensor rotary_rows(const at::Tensor& t) { return t.stride(1) == 1 ? t : t.contiguous(); }

void launch_rotary(const at::Tensor& query, const at::Tensor& key, const at::Tensor& cache,
                   const at::Tensor& positions, int64_t head_dim, int64_t rotary_dim, bool is_neox,
                   const at::Tensor& q_out, const at::Tensor& k_out) {
  const auto q = rotary_rows(query), k = rotary_rows(key);
  gk_rotary_params p{};
  p.struct_size = sizeof(p);
  p.query = q.data_ptr();
  p.q_row_stride = q.stride(0);
  p.q_width = q.size(1);
  p.key = k.data_ptr();
  p.k_row_stride = k.stride(0);
  p.k_width = k.size(1);
  p.positions = positions.data_ptr();
  p.positions_int64 = positions.scalar_type() == at::kLong ? 1 : 0;
  p.cos_sin = cache.data_ptr();
  p.cache_rows = cache.size(0);
  p.rows = static_cast<int32_t>(q.size(0));
  p.head_dim = static_cast<int32_t>(head_dim);
  p.rotary_dim = static_cast<int32_t>(rotary_dim);
  p.is_neox = is_neox ? 1 : 0;
  p.q_out = q_out.data_ptr();
  p.q_out_row_stride = q_out.stride(0);
  p.k_out = k_out.data_ptr();
  p.k_out_row_stride = k_out.stride(0);
  check_gk(gk_rotary_embedding(&p, current_stream()), "GaudiRT rotary");
}

// Checks of src/bridge/generic_private_use1.cpp:330-353 (messages kept: the
// reference's tests match "cache" and "rotary dimension").
void check_rotary_inputs(const at::Tensor& query, const at::Tensor& key, const at::Tensor& cache, int64_t context,
                         int64_t head_dim, int64_t rotary_dim) {
  TORCH_CHECK(head_dim > 0 && head_dim <= std::numeric_limits<int32_t>::max() && rotary_dim > 0 &&
                  rotary_dim <= head_dim && rotary_dim % 2 == 0,
              "GaudiRT rotary: invalid head or rotary dimension");
  const int device = current_device();
  for (const auto& tensor : {query, key, cache})
    TORCH_CHECK(tensor.is_cuda() && tensor.device().index() == device && tensor.scalar_type() == at::kBFloat16,
                "GaudiRT rotary: expected BF16 device tensors");
  TORCH_CHECK(query.dim() == 2 && key.dim() == 2 && query.size(0) > 0 && query.size(0) <= kMaxBucketRows &&
                  key.size(0) == query.size(0) && query.size(1) > 0 && key.size(1) > 0 &&
                  query.size(1) <= std::numeric_limits<int32_t>::max() &&
                  key.size(1) <= std::numeric_limits<int32_t>::max() && query.size(1) % head_dim == 0 &&
                  key.size(1) % head_dim == 0,
              "GaudiRT rotary: invalid query or key geometry");
  TORCH_CHECK(cache.dim() == 2 && context > 0 && cache.size(0) >= context &&
                  cache.size(0) <= std::numeric_limits<int32_t>::max() && cache.size(1) == rotary_dim,
              "GaudiRT rotary: cache does not cover validated positions");
}

// _rotary_embedding_validated (src/bridge/generic_private_use1.cpp:327-405):
// positions come from validated metadata (every position < context <= cache rows).
std::tuple<at::Tensor, at::Tensor> rotary_embedding_validated(const at::Tensor& query, const at::Tensor& key,
                                                              const at::Tensor& cache, const at::Tensor& positions,
                                                              const at::Tensor& header, int64_t context,
                                                              int64_t head_dim, int64_t rotary_dim, bool is_neox) {
  check_rotary_inputs(query, key, cache, context, head_dim, rotary_dim);
  const auto rows = query.size(0);
  TORCH_CHECK(positions.device() == query.device() && positions.scalar_type() == at::kInt && positions.dim() == 1 &&
                  positions.size(0) == rows && positions.is_contiguous() && header.device() == query.device() &&
                  header.scalar_type() == at::kInt && header.dim() == 1 && header.size(0) == 1 &&
                  header.is_contiguous(),
              "GaudiRT rotary: invalid validated metadata tensors");
  const auto table = cache.contiguous();
  auto q_out = bucket_output(query, rows, query.size(1));
  auto k_out = bucket_output(key, rows, key.size(1));
  launch_rotary(query, key, table, positions, head_dim, rotary_dim, is_neox, q_out, k_out);
  return {q_out, k_out};
}

// rotary_embedding (src/bridge/generic_private_use1.cpp:407-415).
std::tuple<at::Tensor, at::Tensor> rotary_embedding(const at::Tensor& query, const at::Tensor& key,
                                                    const at::Tensor& cache,
                                                    const c10::intrusive_ptr<PagedMetadata>& metadata,
                                                    int64_t head_dim, int64_t rotary_dim, bool is_neox) {
  TORCH_CHECK(metadata, "GaudiRT rotary: metadata is required");
  return rotary_embedding_validated(query, key, cache, metadata->rotary_positions(), metadata->rotary_header(),
                                    metadata->context(), head_dim, rotary_dim, is_neox);
}

// rotary_embedding_positions (src/bridge/eager_ops.cpp:1243-1300): positions
// given directly (int32 or int64), 2-D or 3-D rows, outputs of the input shape.
// A position outside the cache reads the nearest cache row.
std::tuple<at::Tensor, at::Tensor> rotary_embedding_positions(const at::Tensor& query, const at::Tensor& key,
                                                              const at::Tensor& cache, const at::Tensor& positions,
                                                              int64_t head_dim, int64_t rotary_dim, bool is_neox) {
  TORCH_CHECK(head_dim > 0 && head_dim <= std::numeric_limits<int32_t>::max() && rotary_dim > 0 &&
                  rotary_dim <= head_dim && rotary_dim % 2 == 0,
              "GaudiRT: rotary_embedding_positions invalid head_size or rotary_dim");
  TORCH_CHECK(query.is_cuda() && key.device() == query.device() && cache.device() == query.device() &&
                  positions.device() == query.device(),
              "GaudiRT: rotary_embedding_positions requires same-device GPU tensors");
  TORCH_CHECK(query.scalar_type() == at::kBFloat16 && key.scalar_type() == at::kBFloat16 &&
                  cache.scalar_type() == at::kBFloat16 &&
                  (positions.scalar_type() == at::kInt || positions.scalar_type() == at::kLong),
              "GaudiRT: rotary_embedding_positions expects BF16 query/key/cache and Int32/Int64 positions");
  TORCH_CHECK((query.dim() == 2 || query.dim() == 3) && key.dim() == query.dim() && key.size(0) == query.size(0) &&
                  cache.dim() == 2 && cache.size(1) == rotary_dim && cache.size(0) > 0 && positions.dim() == 1 &&
                  positions.size(0) == query.size(0),
              "GaudiRT: rotary_embedding_positions shape mismatch");
  if (!query.numel()) return {at::empty(query.sizes(), query.options()), at::empty(key.sizes(), key.options())};
  const auto rows = query.size(0);
  const auto q2 = query.reshape({rows, -1}), k2 = key.reshape({rows, -1});
  TORCH_CHECK(q2.size(1) % head_dim == 0 && k2.size(1) % head_dim == 0 && q2.size(1) / head_dim <= 65535 &&
                  k2.size(1) / head_dim <= 65535 && rows <= std::numeric_limits<int32_t>::max(),
              "GaudiRT: rotary_embedding_positions shape mismatch");
  auto q_out = at::empty(query.sizes(), query.options());
  auto k_out = at::empty(key.sizes(), key.options());
  launch_rotary(q2, k2, cache.contiguous(), positions.contiguous(), head_dim, rotary_dim, is_neox,
                q_out.view({rows, -1}), k_out.view({rows, -1}));
  return {q_out, k_out};
}

// rotary_paged_attn: the rotary embedding of a layer fused into the KV store of
// its paged attention. Equals paged_attn(q', k', value, ...) with
// (q', k') = rotary_embedding(query, key, cache, metadata, ...), bit for bit,
// but the rotated keys go from registers into the pool instead of through an
// intermediate tensor. No counterpart in the reference: there the rotary
// recipe and the attention store are separate launches
// (src/bridge/generic_private_use1.cpp:327-405, src/bridge/paged_attention.cpp:66-76).
at::Tensor rotary_paged_attn(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                             const at::Tensor& key_pool, const at::Tensor& value_pool, const at::Tensor& cache,
                             const c10::intrusive_ptr<PagedMetadata>& metadata, int64_t head_dim, int64_t rotary_dim,
                             bool is_neox, double scale, double softcap, int64_t sliding_window) {
  TORCH_CHECK(metadata, "GaudiRT paged attention: metadata is required");
  TORCH_CHECK(query.dim() == 2 && key_pool.dim() == 3 && (head_dim == 64 || head_dim == 128 || head_dim == 256),
              "GaudiRT paged attention: invalid tensor ranks or head dimension");
  check_rotary_inputs(query, key, cache, metadata->context(), head_dim, rotary_dim);
  const auto q_heads = query.size(1) / head_dim;
  const auto kv_heads = key_pool.size(1);
  auto plan = sliding_window > 0 ? metadata->attention_plan_for(q_heads, kv_heads, head_dim, sliding_window)
                                 : metadata->attention_plan(q_heads, kv_heads, head_dim);
  const RotarySpec spec{cache.contiguous(), metadata->rotary_positions(), rotary_dim, is_neox};
  return paged_attn_impl(query, key, value, key_pool, value_pool, metadata->row_locations(), plan, head_dim, scale,
                         softcap, sliding_window, &spec);
}

// advance_decode_lengths (src/bridge/eager_scheduler.cpp:50-82).
std::tuple<at::Tensor, at::Tensor> advance_decode_lengths(const at::Tensor& seq_lens, const at::Tensor& orig_seq_lens) {
  TORCH_CHECK(seq_lens.is_cuda() && orig_seq_lens.device() == seq_lens.device() &&
                  seq_lens.scalar_type() == at::kLong && orig_seq_lens.scalar_type() == at::kInt &&
                  seq_lens.dim() == 1 && orig_seq_lens.sizes() == seq_lens.sizes() &&
                  seq_lens.numel() <= std::numeric_limits<int>::max() && seq_lens.is_contiguous() &&
                  orig_seq_lens.is_contiguous(),
              "GaudiRT decode lengths: expected matching contiguous int64 and int32 vectors");
  auto next = at::empty_like(seq_lens), orig_next = at::empty_like(orig_seq_lens);
  if (!seq_lens.numel()) return {next, orig_next};
  TORCH_CHECK(seq_lens.numel() <= (1LL << 30), "GaudiRT decode lengths: count exceeds supported range");
  check_gk(gk_advance_decode_lengths(seq_lens.data_ptr<int64_t>(), orig_seq_lens.data_ptr<int32_t>(), seq_lens.numel(),
                                     next.data_ptr<int64_t>(), orig_next.data_ptr<int32_t>(), current_stream()),
           "GaudiRT decode lengths");
  return {next, orig_next};
}

// ---------------------------------------------------------------------------
// Paged slot allocator (src/bridge/paged_slot_allocator.cpp:91-190).
// ---------------------------------------------------------------------------
void require_indices(const at::Tensor& tensor) {
  TORCH_CHECK(tensor.is_cuda() && tensor.device().index() == current_device() && tensor.scalar_type() == at::kLong &&
                  tensor.dim() == 1 && tensor.is_contiguous(),
              "GaudiRT paged allocator: expected contiguous device int64 indices");
}

// New slots for the next lengths[s] tokens of each sequence: the tail of the
// page holding last_slots[s] first, then whole pages from free_pages in order.
// Returns (slots [sum(lengths)] int64, pages taken from free_pages).
std::tuple<at::Tensor, int64_t> allocate_paged_slots(const at::Tensor& last_slots, const at::Tensor& free_pages,
                                                     const std::vector<int64_t>& prefixes,
                                                     const std::vector<int64_t>& lengths, int64_t page_size) {
  require_indices(last_slots);
  require_indices(free_pages);
  TORCH_CHECK(page_size >= 1 && page_size <= std::numeric_limits<int32_t>::max() && !prefixes.empty() &&
                  prefixes.size() <= (size_t{1} << 30) && prefixes.size() == lengths.size() &&
                  last_slots.numel() == static_cast<int64_t>(prefixes.size()),
              "GaudiRT paged allocator: unsupported page size or request count");
  const int64_t batch = static_cast<int64_t>(prefixes.size());
  std::vector<int64_t> meta(4 * batch);
  int64_t total = 0, pages = 0;
  for (int64_t s = 0; s < batch; ++s) {
    const int64_t prefix = prefixes[s], length = lengths[s];
    TORCH_CHECK(prefix >= 0 && length >= 0 && prefix + length <= std::numeric_limits<int32_t>::max(),
                "GaudiRT paged allocator: invalid request lengths");
    meta[4 * s] = prefix;
    meta[4 * s + 1] = length;
    meta[4 * s + 2] = total;
    meta[4 * s + 3] = pages;
    total += length;
    pages += (prefix + length + page_size - 1) / page_size - (prefix + page_size - 1) / page_size;
  }
  TORCH_CHECK(total > 0 && total <= (int64_t{1} << 30) && pages <= (int64_t{1} << 30) && pages <= free_pages.numel(),
              "GaudiRT paged allocator: invalid token count or insufficient free pages");
  if (page_size == 1) return {free_pages.narrow(0, 0, total).clone(), total};
  std::vector<int32_t> words(meta.size() * 2);
  std::memcpy(words.data(), meta.data(), meta.size() * sizeof(int64_t));
  const auto device_meta = upload_words(words, static_cast<int64_t>(words.size()));
  auto slots = at::empty({total}, last_slots.options());
  check_gk(gk_paged_alloc_slots(last_slots.data_ptr<int64_t>(), free_pages.data_ptr<int64_t>(),
                                reinterpret_cast<const int64_t*>(device_meta.data_ptr<int32_t>()),
                                static_cast<int32_t>(batch), page_size, total, slots.data_ptr<int64_t>(),
                                current_stream()),
           "GaudiRT paged allocator");
  return {slots, pages};
}

// Distinct pages of the released slots in order of first occurrence. Waits
// for the count, as the reference does.
at::Tensor release_paged_slots(const at::Tensor& slots, int64_t page_size, int64_t max_pages) {
  require_indices(slots);
  TORCH_CHECK(page_size >= 1 && page_size <= std::numeric_limits<int32_t>::max() && max_pages > 0 &&
                  max_pages <= std::numeric_limits<int32_t>::max() && slots.numel() > 0 &&
                  slots.numel() <= (int64_t{1} << 30),
              "GaudiRT paged allocator: invalid release geometry");
  const size_t need = gk_paged_release_workspace_bytes(max_pages);
  auto workspace = at::empty({static_cast<int64_t>(need)}, slots.options().dtype(at::kByte));
  auto pages = at::empty_like(slots);
  auto count = at::empty({1}, slots.options().dtype(at::kInt));
  check_gk(gk_paged_release_slots(slots.data_ptr<int64_t>(), slots.numel(), page_size, max_pages,
                                  workspace.data_ptr(), need, pages.data_ptr<int64_t>(), count.data_ptr<int32_t>(),
                                  current_stream()),
           "GaudiRT paged allocator");
  const int32_t released = count.cpu().data_ptr<int32_t>()[0];
  TORCH_CHECK(released > 0 && released <= slots.numel(),
              "GaudiRT paged allocator: released slot is outside the KV pool");
  return pages.narrow(0, 0, released);
}

}  // namespace
}  // namespace gaudirt_amd

TORCH_LIBRARY(gaudirt, m) {
  using gaudirt_amd::PagedMetadata;
  m.class_<PagedMetadata>("PagedMetadata")
      .def(torch::init<at::Tensor, at::Tensor, at::Tensor, at::Tensor, int64_t>())
      .def_static("from_device", &PagedMetadata::from_device)
      .def_static("from_device_with_tokens", &PagedMetadata::from_device_with_tokens)
      .def_static("_from_scheduler", &PagedMetadata::from_scheduler)
      .def_static("_from_scheduler_fused", &PagedMetadata::from_scheduler_fused)
      .def("rows", &PagedMetadata::rows)
      .def("slots", &PagedMetadata::slots)
      .def("context", &PagedMetadata::context)
      .def("forward_tensors", &PagedMetadata::forward_tensors)
      .def("rotary_positions", &PagedMetadata::rotary_positions)
      .def("model_positions", &PagedMetadata::model_positions)
      .def("rotary_header", &PagedMetadata::rotary_header)
      .def("row_locations", &PagedMetadata::row_locations)
      .def("row_requests", &PagedMetadata::row_requests)
      .def("request_mapping", &PagedMetadata::request_mapping)
      .def("attention_plan", &PagedMetadata::attention_plan)
      .def("attention_plan_for", &PagedMetadata::attention_plan_for)
      .def("last_token_indices", &PagedMetadata::last_token_indices)
      .def("token_ids", &PagedMetadata::token_ids)
      .def("vocabulary", &PagedMetadata::vocabulary);
  m.def("paged_attn(Tensor query, Tensor key, Tensor value, Tensor(a!) key_pool, Tensor(b!) value_pool, "
        "__torch__.torch.classes.gaudirt.PagedMetadata metadata, int head_dim, float scale, "
        "float softcap=0.0, int sliding_window=-1) -> Tensor");
  m.def("_paged_attn_validated(Tensor query, Tensor key, Tensor value, Tensor(a!) key_pool, Tensor(b!) value_pool, "
        "Tensor locations, Tensor requests, Tensor positions, Tensor mapping, Tensor header, "
        "int head_dim, float scale, float softcap=0.0, int sliding_window=-1) -> Tensor");
  m.def("_advance_decode_lengths(Tensor seq_lens, Tensor orig_seq_lens) -> (Tensor, Tensor)");
  m.def("rotary_embedding(Tensor query, Tensor key, Tensor cache, "
        "__torch__.torch.classes.gaudirt.PagedMetadata metadata, int head_dim, int rotary_dim, bool is_neox) "
        "-> (Tensor, Tensor)");
  m.def("rotary_embedding_positions(Tensor query, Tensor key, Tensor cache, Tensor positions, "
        "int head_dim, int rotary_dim, bool is_neox) -> (Tensor, Tensor)");
  m.def("_rotary_embedding_validated(Tensor query, Tensor key, Tensor cache, Tensor positions, "
        "Tensor header, int context, int head_dim, int rotary_dim, bool is_neox) -> (Tensor, Tensor)");
  m.def("rotary_paged_attn(Tensor query, Tensor key, Tensor value, Tensor(a!) key_pool, Tensor(b!) value_pool, "
        "Tensor cache, __torch__.torch.classes.gaudirt.PagedMetadata metadata, int head_dim, int rotary_dim, "
        "bool is_neox, float scale, float softcap=0.0, int sliding_window=-1) -> Tensor");
}

TORCH_LIBRARY_IMPL(gaudirt, CUDA, m) {
  m.impl("paged_attn", TORCH_FN(gaudirt_amd::paged_attn));
  m.impl("_paged_attn_validated", TORCH_FN(gaudirt_amd::paged_attn_validated));
  m.impl("_advance_decode_lengths", TORCH_FN(gaudirt_amd::advance_decode_lengths));
  m.impl("rotary_embedding", TORCH_FN(gaudirt_amd::rotary_embedding));
  m.impl("rotary_embedding_positions", TORCH_FN(gaudirt_amd::rotary_embedding_positions));
  m.impl("_rotary_embedding_validated", TORCH_FN(gaudirt_amd::rotary_embedding_validated));
  m.impl("rotary_paged_attn", TORCH_FN(gaudirt_amd::rotary_paged_attn));
}

namespace gaudirt_amd {
void set_decode_partition(int64_t tokens) {
  TORCH_CHECK(tokens >= 0 && tokens <= 8192 && tokens % 32 == 0,
              "GaudiRT: the decode partition must be 0 (library choice) or a multiple of 32 keys up to 8192");
  g_decode_partition.store(static_cast<int32_t>(tokens), std::memory_order_relaxed);
}
int64_t decode_partition() { return g_decode_partition.load(std::memory_order_relaxed); }
}  // namespace gaudirt_amd

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("_set_decode_partition", &gaudirt_amd::set_decode_partition,
        "split-K partition of paged_attn's decode rows (0: library choice; > 0: fixed, batch-invariant)");
  m.def("_decode_partition", &gaudirt_amd::decode_partition);
  m.def("_allocate_paged_kv", &gaudirt_amd::allocate_paged_kv, "zeroed head-major bf16 KV pool");
  m.def("_allocate_paged_slots", &gaudirt_amd::allocate_paged_slots, "page-granular KV slots for new tokens");
  m.def("_release_paged_slots", &gaudirt_amd::release_paged_slots, "distinct pages of released KV slots");
  m.def("_kv_allocator_stats", &gaudirt_amd::allocator_stats, pybind11::arg("device") = 0);
  m.def("_paged_attn_kv_tile", [](int64_t) { return 512; });
  m.def("version", []() { return std::string(gk_version()); });
}
