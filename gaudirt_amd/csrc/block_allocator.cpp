// C ABI of the stream-ordered block allocator (gk_allocator_*): the
// bookkeeping of block_allocator_core.cpp on the HIP runtime of one device.
#include <hip/hip_runtime.h>

#include <memory>
#include <string>

#include "block_allocator.hpp"
#include "gk_common.hpp"

namespace {

// Makes `device` current for the lifetime of the guard.
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

// AllocatorRuntime on HIP: slabs from hipMalloc, fences from timing-free events.
class HipRuntime final : public gk::AllocatorRuntime {
 public:
  explicit HipRuntime(int device) : device_(device) {}

  int malloc(uint64_t bytes, void** out, std::string& error) override {
    DeviceGuard guard(device_);
    return check(hipMalloc(out, bytes), "hipMalloc", error, GK_ERR_OUT_OF_MEMORY);
  }
  int free(void* ptr, std::string& error) override {
    DeviceGuard guard(device_);
    return check(hipFree(ptr), "hipFree", error);
  }
  int event_create(gk::EventHandle* out, std::string& error) override {
    DeviceGuard guard(device_);
    hipEvent_t event = nullptr;
    const int rc = check(hipEventCreateWithFlags(&event, hipEventDisableTiming), "hipEventCreateWithFlags", error);
    *out = event;
    return rc;
  }
  int event_destroy(gk::EventHandle event, std::string& error) override {
    return check(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy", error);
  }
  int event_record(gk::EventHandle event, gk::StreamHandle stream, std::string& error) override {
    return check(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)), "hipEventRecord",
                 error);
  }
  int stream_wait_event(gk::StreamHandle stream, gk::EventHandle event, std::string& error) override {
    return check(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(event), 0),
                 "hipStreamWaitEvent", error);
  }
  int stream_synchronize(gk::StreamHandle stream, std::string& error) override {
    return check(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize", error);
  }
  int device_synchronize(std::string& error) override {
    DeviceGuard guard(device_);
    return check(hipDeviceSynchronize(), "hipDeviceSynchronize", error);
  }

 private:
  static int check(hipError_t err, const char* what, std::string& error, int code = GK_ERR_HIP) {
    if (err == hipSuccess) return GK_OK;
    (void)hipGetLastError();
    error = std::string(what) + ": " + hipGetErrorString(err);
    return code;
  }
  int device_;
};

}  // namespace

// The opaque handle of the C ABI: the runtime binding and the bookkeeping on it.
struct gk_allocator {
  explicit gk_allocator(int device, uint64_t budget, uint64_t slab)
      : runtime(device), pool(runtime, budget, slab) {}
  HipRuntime runtime;
  gk::BlockAllocator pool;
};

namespace {
int result(gk_allocator* a, int rc) { return rc ? gk::fail(rc, a->pool.error()) : GK_OK; }
}  // namespace

extern "C" int gk_allocator_create(int32_t device, uint64_t budget_bytes, uint64_t slab_bytes, gk_allocator** out) {
  gk::clear_error();
  if (!out || budget_bytes == 0) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_create: invalid arguments");
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count)
    return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_create: invalid device");
  *out = new gk_allocator(device, budget_bytes, slab_bytes);
  return GK_OK;
}

extern "C" int gk_allocator_destroy(gk_allocator* a) {
  gk::clear_error();
  delete a;
  return GK_OK;
}

extern "C" int gk_allocator_alloc(gk_allocator* a, uint64_t bytes, hipStream_t stream, void** out) {
  gk::clear_error();
  if (!a) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_alloc: null allocator");
  return result(a, a->pool.allocate(bytes, stream, out));
}

extern "C" int gk_allocator_record_stream(gk_allocator* a, void* ptr, hipStream_t stream) {
  gk::clear_error();
  if (!a) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_record_stream: null allocator");
  return result(a, a->pool.record_stream(ptr, stream));
}

extern "C" int gk_allocator_free(gk_allocator* a, void* ptr) {
  gk::clear_error();
  if (!a) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_free: null allocator");
  return result(a, a->pool.release(ptr));
}

extern "C" int gk_allocator_empty_cache(gk_allocator* a) {
  gk::clear_error();
  if (!a) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_empty_cache: null allocator");
  return result(a, a->pool.empty_cache());
}

extern "C" int gk_allocator_get_stats(gk_allocator* a, gk_allocator_stats* stats) {
  gk::clear_error();
  if (!a || !stats) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_allocator_get_stats: null argument");
  const gk::AllocatorStats s = a->pool.stats();
  stats->allocated_bytes = s.allocated_bytes;
  stats->peak_bytes = s.peak_bytes;
  stats->reserved_bytes = s.reserved_bytes;
  stats->largest_free_block = s.largest_free_block;
  stats->slabs = s.slabs;
  stats->events_created = s.events_created;
  return GK_OK;
}
