// Stream-ordered block allocator for the KV pool and attention workspaces.
//
// Contract of runtime::BlockCachingAllocator in the reference
// (include/gaudirt/runtime/block_caching_allocator.hpp:19-70,
// src/block_caching_allocator.cpp:120-293), on HIP:
//   - HBM comes from hipMalloc slabs (up to a byte budget) carved into
//     256-byte aligned blocks; allocation is best fit, frees merge neighbours.
//   - Every stream that used a block is recorded (the allocating stream
//     implicitly, others through record_stream). After free, the block keeps
//     those streams as pending producers; a later allocation on stream S makes
//     S wait on an event recorded on each other producer. There is no host
//     synchronisation on the allocation path.
//   - Events come from a pool and are reused as soon as the wait is enqueued,
//     so steady state creates no events.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "gk_common.hpp"

struct gk_allocator {
  static constexpr uint64_t kAlignment = 256;

  struct Block {
    uint64_t bytes = 0;
    bool allocated = false;
    int slab = 0;
    std::vector<hipStream_t> streams;  // users while allocated
    std::vector<hipStream_t> pending;  // producers to fence before reuse
  };

  int device = 0;
  uint64_t budget = 0, slab_bytes = 0;
  uint64_t reserved = 0, allocated = 0, peak = 0, events_created = 0;
  std::map<uintptr_t, Block> blocks;
  std::set<std::pair<uint64_t, uintptr_t>> free_by_size;
  std::vector<std::pair<uintptr_t, uint64_t>> slabs;  // base, bytes (base 0 = released)
  std::vector<hipEvent_t> idle_events;
  std::mutex mutex;
};

namespace {

using Allocator = gk_allocator;

struct DeviceGuard {
  int previous = -1;
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&previous) != hipSuccess) previous = -1;
    if (previous != device) (void)hipSetDevice(device);
  }
  ~DeviceGuard() {
    if (previous >= 0) (void)hipSetDevice(previous);
  }
};

void add_unique(std::vector<hipStream_t>& to, const std::vector<hipStream_t>& from) {
  for (auto s : from)
    if (std::find(to.begin(), to.end(), s) == to.end()) to.push_back(s);
}

int fence(Allocator& a, hipStream_t producer, hipStream_t consumer) {
  hipEvent_t event;
  if (!a.idle_events.empty()) {
    event = a.idle_events.back();
    a.idle_events.pop_back();
  } else {
    if (int rc = gk::hip_status(hipEventCreateWithFlags(&event, hipEventDisableTiming), "allocator event create"))
      return rc;
    ++a.events_created;
  }
  int rc = gk::hip_status(hipEventRecord(event, producer), "allocator event record");
  if (!rc) rc = gk::hip_status(hipStreamWaitEvent(consumer, event, 0), "allocator stream wait");
  a.idle_events.push_back(event);
  return rc;
}

void insert_free(Allocator& a, uintptr_t address, const Allocator::Block& block) {
  a.free_by_size.insert({block.bytes, address});
}
void erase_free(Allocator& a, uintptr_t address, const Allocator::Block& block) {
  a.free_by_size.erase({block.bytes, address});
}

int add_slab(Allocator& a, uint64_t size) {
  uint64_t bytes = std::max(size, a.slab_bytes);
  if (a.reserved + bytes > a.budget) bytes = size;  // fall back to an exact-size slab
  if (a.reserved + bytes > a.budget)
    return gk::fail(GK_ERR_OUT_OF_MEMORY, "gk_allocator: budget of " + std::to_string(a.budget) +
                                              " bytes exhausted (" + std::to_string(a.reserved) + " reserved)");
  void* base = nullptr;
  {
    DeviceGuard guard(a.device);
    const hipError_t err = hipMalloc(&base, bytes);
    if (err != hipSuccess) {
      (void)hipGetLastError();
      return gk::fail(GK_ERR_OUT_OF_MEMORY, std::string("gk_allocator: hipMalloc failed: ") + hipGetErrorString(err));
    }
  }
  const int slab = static_cast<int>(a.slabs.size());
  a.slabs.push_back({reinterpret_cast<uintptr_t>(base), bytes});
  a.reserved += bytes;
  Allocator::Block block;
  block.bytes = bytes;
  block.slab = slab;
  const uintptr_t address = reinterpret_cast<uintptr_t>(base);
  a.blocks.emplace(address, block);
  insert_free(a, address, block);
  return GK_OK;
}

}  // namespace

extern "C" int gk_allocator_create(int32_t device, uint64_t budget_bytes, uint64_t slab_bytes, gk_allocator** out) {
  gk::clear_error();
  if (!out || budget_bytes == 0) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_create: invalid arguments");
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count)
    return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_create: invalid device");
  auto* a = new Allocator();
  a->device = device;
  a->budget = budget_bytes;
  a->slab_bytes = std::max<uint64_t>(Allocator::kAlignment,
                                     (slab_bytes + Allocator::kAlignment - 1) & ~(Allocator::kAlignment - 1));
  *out = a;
  return GK_OK;
}

extern "C" int gk_allocator_destroy(gk_allocator* a) {
  gk::clear_error();
  if (!a) return GK_OK;
  {
    DeviceGuard guard(a->device);
    (void)hipDeviceSynchronize();
    for (auto& [base, bytes] : a->slabs)
      if (base) (void)hipFree(reinterpret_cast<void*>(base));
    for (auto e : a->idle_events) (void)hipEventDestroy(e);
  }
  delete a;
  return GK_OK;
}

extern "C" int gk_allocator_alloc(gk_allocator* a, uint64_t bytes, hipStream_t stream, void** out) {
  gk::clear_error();
  if (!a || !out) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_alloc: null argument");
  const uint64_t size = std::max<uint64_t>(Allocator::kAlignment,
                                           (bytes + Allocator::kAlignment - 1) & ~(Allocator::kAlignment - 1));
  std::lock_guard<std::mutex> lock(a->mutex);
  auto it = a->free_by_size.lower_bound({size, 0});
  if (it == a->free_by_size.end()) {
    if (int rc = add_slab(*a, size)) return rc;
    it = a->free_by_size.lower_bound({size, 0});
  }
  const uintptr_t address = it->second;
  auto& block = a->blocks.at(address);
  erase_free(*a, address, block);
  for (auto producer : block.pending)
    if (producer != stream)
      if (int rc = fence(*a, producer, stream)) {
        insert_free(*a, address, block);
        return rc;
      }
  if (block.bytes > size) {
    Allocator::Block rest;
    rest.bytes = block.bytes - size;
    rest.slab = block.slab;
    rest.pending = block.pending;
    a->blocks.emplace(address + size, rest);
    insert_free(*a, address + size, rest);
    block.bytes = size;
  }
  block.allocated = true;
  block.pending.clear();
  block.streams = {stream};
  a->allocated += size;
  a->peak = std::max(a->peak, a->allocated);
  *out = reinterpret_cast<void*>(address);
  return GK_OK;
}

extern "C" int gk_allocator_record_stream(gk_allocator* a, void* ptr, hipStream_t stream) {
  gk::clear_error();
  if (!a || !ptr) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_record_stream: null argument");
  std::lock_guard<std::mutex> lock(a->mutex);
  const uintptr_t address = reinterpret_cast<uintptr_t>(ptr);
  auto it = a->blocks.upper_bound(address);
  if (it == a->blocks.begin()) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator: unknown live allocation");
  --it;
  if (!it->second.allocated || address - it->first >= it->second.bytes)
    return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator: unknown live allocation");
  add_unique(it->second.streams, {stream});
  return GK_OK;
}

extern "C" int gk_allocator_free(gk_allocator* a, void* ptr) {
  gk::clear_error();
  if (!a || !ptr) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_free: null argument");
  std::lock_guard<std::mutex> lock(a->mutex);
  auto it = a->blocks.find(reinterpret_cast<uintptr_t>(ptr));
  if (it == a->blocks.end() || !it->second.allocated)
    return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator: unknown or freed allocation");
  a->allocated -= it->second.bytes;
  it->second.allocated = false;
  it->second.pending.swap(it->second.streams);
  it->second.streams.clear();
  // merge with free neighbours of the same slab
  auto next = std::next(it);
  if (next != a->blocks.end() && !next->second.allocated && next->second.slab == it->second.slab &&
      it->first + it->second.bytes == next->first) {
    erase_free(*a, next->first, next->second);
    it->second.bytes += next->second.bytes;
    add_unique(it->second.pending, next->second.pending);
    a->blocks.erase(next);
  }
  if (it != a->blocks.begin()) {
    auto prev = std::prev(it);
    if (!prev->second.allocated && prev->second.slab == it->second.slab &&
        prev->first + prev->second.bytes == it->first) {
      erase_free(*a, prev->first, prev->second);
      prev->second.bytes += it->second.bytes;
      add_unique(prev->second.pending, it->second.pending);
      a->blocks.erase(it);
      it = prev;
    }
  }
  insert_free(*a, it->first, it->second);
  return GK_OK;
}

extern "C" int gk_allocator_empty_cache(gk_allocator* a) {
  gk::clear_error();
  if (!a) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_empty_cache: null allocator");
  std::lock_guard<std::mutex> lock(a->mutex);
  DeviceGuard guard(a->device);
  for (auto& [address, block] : a->blocks) {
    (void)address;
    if (block.allocated) continue;
    for (auto s : block.pending)
      if (int rc = gk::hip_status(hipStreamSynchronize(s), "gk_allocator_empty_cache synchronize")) return rc;
    block.pending.clear();
  }
  for (size_t slab = 0; slab < a->slabs.size(); ++slab) {
    auto& [base, bytes] = a->slabs[slab];
    if (!base) continue;
    auto it = a->blocks.find(base);
    if (it == a->blocks.end() || it->second.allocated || it->second.bytes != bytes) continue;
    erase_free(*a, it->first, it->second);
    a->blocks.erase(it);
    if (int rc = gk::hip_status(hipFree(reinterpret_cast<void*>(base)), "gk_allocator_empty_cache hipFree")) return rc;
    a->reserved -= bytes;
    base = 0;
    bytes = 0;
  }
  return GK_OK;
}

extern "C" int gk_allocator_get_stats(gk_allocator* a, gk_allocator_stats* stats) {
  gk::clear_error();
  if (!a || !stats) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_get_stats: null argument");
  std::lock_guard<std::mutex> lock(a->mutex);
  stats->allocated_bytes = a->allocated;
  stats->peak_bytes = a->peak;
  stats->reserved_bytes = a->reserved;
  stats->largest_free_block = a->free_by_size.empty() ? 0 : a->free_by_size.rbegin()->first;
  uint64_t live = 0;
  for (auto& [base, bytes] : a->slabs) live += base ? 1 : 0;
  stats->slabs = live;
  stats->events_created = a->events_created;
  return GK_OK;
}
