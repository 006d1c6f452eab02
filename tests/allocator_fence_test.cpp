// CPU unit test of the block allocator's stream-ordering contract, built with
// g++ against a recording mock of the device runtime (no GPU): the cases of
// the reference's tests/block_allocator_fences_unit_test.cpp restated for this
// allocator. Every fence must be a record on the producer followed by a wait
// on the consumer; an event is never recorded again before the wait on its
// previous record; same-stream reuse needs no fence; producers survive splits
// and merges; steady state creates no events. Prints "OK" and exits 0.
#include <cassert>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <random>
#include <string>
#include <vector>

#include "block_allocator.hpp"

namespace {

#define CHECK(cond)                                                        \
  do {                                                                     \
    if (!(cond)) {                                                         \
      std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
      std::exit(1);                                                        \
    }                                                                      \
  } while (0)

gk::StreamHandle stream(unsigned id) { return reinterpret_cast<gk::StreamHandle>(uintptr_t{id}); }

struct MockEvent {
  gk::StreamHandle recorded_on = nullptr;
  uint64_t ordinal = 0;   // which record on that stream
  bool awaiting_wait = false;
};

// A fence as the consumer saw it: the producer stream and record ordinal of the waited event.
struct Wait {
  gk::StreamHandle consumer, producer;
  uint64_t ordinal;
};

class MockRuntime final : public gk::AllocatorRuntime {
 public:
  int malloc(uint64_t bytes, void** out, std::string&) override {
    next_base_ += 1 << 20;  // slabs far apart, never adjacent
    *out = reinterpret_cast<void*>(next_base_);
    slabs_[next_base_] = bytes;
    return 0;
  }
  int free(void* ptr, std::string&) override {
    CHECK(slabs_.erase(reinterpret_cast<uintptr_t>(ptr)) == 1);
    return 0;
  }
  int event_create(gk::EventHandle* out, std::string&) override {
    *out = new MockEvent;
    ++created;
    ++live_events;
    return 0;
  }
  int event_destroy(gk::EventHandle event, std::string&) override {
    delete static_cast<MockEvent*>(event);
    --live_events;
    return 0;
  }
  int event_record(gk::EventHandle event, gk::StreamHandle s, std::string&) override {
    auto& e = *static_cast<MockEvent*>(event);
    CHECK(!e.awaiting_wait);  // recorded again before its previous record was waited on
    e = {s, ++records[s], true};
    return 0;
  }
  int stream_wait_event(gk::StreamHandle s, gk::EventHandle event, std::string&) override {
    auto& e = *static_cast<MockEvent*>(event);
    CHECK(e.awaiting_wait);  // a wait must follow a record
    waits.push_back({s, e.recorded_on, e.ordinal});
    e.awaiting_wait = false;
    return 0;
  }
  int stream_synchronize(gk::StreamHandle s, std::string&) override {
    synchronized.push_back(s);
    return 0;
  }
  int device_synchronize(std::string&) override { return 0; }

  void reset_log() {
    records.clear();
    waits.clear();
    synchronized.clear();
  }
  size_t slabs() const { return slabs_.size(); }

  uint64_t created = 0;
  int64_t live_events = 0;
  std::map<gk::StreamHandle, uint64_t> records;
  std::vector<Wait> waits;
  std::vector<gk::StreamHandle> synchronized;

 private:
  uintptr_t next_base_ = 0;
  std::map<uintptr_t, uint64_t> slabs_;
};

void* alloc(gk::BlockAllocator& pool, uint64_t bytes, unsigned s) {
  void* p = nullptr;
  CHECK(pool.allocate(bytes, stream(s), &p) == 0 && p);
  CHECK(reinterpret_cast<uintptr_t>(p) % gk::BlockAllocator::kAlignment == 0);
  return p;
}

void release(gk::BlockAllocator& pool, void* p) { CHECK(pool.release(p) == 0); }

}  // namespace

int main() {
  {  // Same-stream reuse: FIFO order on the stream suffices, no event at all.
    MockRuntime rt;
    {
      gk::BlockAllocator pool(rt, 1 << 16, 4096);
      for (int i = 0; i < 1000; ++i) release(pool, alloc(pool, 256, 1));
      CHECK(rt.created == 0 && rt.records.empty() && rt.waits.empty());
      CHECK(pool.stats().slabs == 1 && pool.stats().allocated_bytes == 0 && pool.stats().peak_bytes == 256);
    }
    CHECK(rt.live_events == 0 && rt.slabs() == 0);
  }
  for (bool reverse : {false, true}) {  // Neighbours merge and keep their producer.
    MockRuntime rt;
    gk::BlockAllocator pool(rt, 1 << 16, 4096);
    void* left = alloc(pool, 256, 1);
    void* right = alloc(pool, 256, 1);
    release(pool, reverse ? right : left);
    release(pool, reverse ? left : right);
    void* merged = alloc(pool, 512, 2);
    CHECK(merged == left);
    CHECK(rt.waits.size() == 1 && rt.waits[0].consumer == stream(2) && rt.waits[0].producer == stream(1));
    CHECK(rt.waits[0].ordinal == 1 && rt.records[stream(1)] == 1);
    release(pool, merged);
  }
  {  // Best fit over separated free blocks; each reuse on a new stream fences the producer.
    MockRuntime rt;
    gk::BlockAllocator pool(rt, 1 << 16, 4096);
    void* a = alloc(pool, 256, 1);
    void* gap = alloc(pool, 256, 1);
    void* b = alloc(pool, 256, 1);
    void* guard = alloc(pool, 256, 1);
    release(pool, a);
    release(pool, b);
    void* first = alloc(pool, 256, 2);
    CHECK(first == a && rt.waits.size() == 1 && rt.waits[0].ordinal == 1);
    void* second = alloc(pool, 256, 3);
    CHECK(second == b && rt.waits.size() == 2 && rt.waits[1].ordinal == 2);
    CHECK(rt.waits[0].producer == stream(1) && rt.waits[1].producer == stream(1));
    CHECK(rt.waits[0].consumer == stream(2) && rt.waits[1].consumer == stream(3));
    CHECK(rt.created == 1);  // the one event went back to the pool after its wait
    for (void* p : {gap, first, second, guard}) release(pool, p);
  }
  {  // record_stream adds producers; reuse fences every producer but the consumer.
    MockRuntime rt;
    gk::BlockAllocator pool(rt, 1 << 16, 4096);
    void* p = alloc(pool, 256, 1);
    CHECK(pool.record_stream(static_cast<char*>(p) + 100, stream(2)) == 0);  // interior pointers name the block
    release(pool, p);
    p = alloc(pool, 256, 1);
    CHECK(rt.waits.size() == 1 && rt.waits[0].producer == stream(2) && rt.waits[0].consumer == stream(1));
    CHECK(pool.record_stream(p, stream(2)) == 0);
    release(pool, p);
    rt.reset_log();
    p = alloc(pool, 256, 3);
    CHECK(rt.waits.size() == 2);
    CHECK(rt.waits[0].producer == stream(1) && rt.waits[1].producer == stream(2));
    CHECK(rt.waits[0].consumer == stream(3) && rt.waits[1].consumer == stream(3));
    release(pool, p);
    CHECK(pool.record_stream(p, stream(2)) != 0);          // no longer live
    CHECK(pool.release(p) != 0);                           // double free
    CHECK(pool.release(static_cast<char*>(p) + 256) != 0); // not a block start
  }
  {  // A split keeps the producers on the free tail.
    MockRuntime rt;
    gk::BlockAllocator pool(rt, 1 << 16, 4096);
    release(pool, alloc(pool, 1024, 1));
    void* head = alloc(pool, 256, 2);
    CHECK(rt.waits.size() == 1 && rt.waits[0].producer == stream(1));
    void* tail = alloc(pool, 256, 3);
    CHECK(tail == static_cast<char*>(head) + 256);
    CHECK(rt.waits.size() == 2 && rt.waits[1].producer == stream(1) && rt.waits[1].consumer == stream(3));
    release(pool, head);
    release(pool, tail);
  }
  {  // empty_cache waits for pending producers, then returns whole free slabs.
    MockRuntime rt;
    gk::BlockAllocator pool(rt, 1 << 16, 4096);
    void* keep = alloc(pool, 4096, 1);   // slab 1, fully live
    void* p = alloc(pool, 4096, 2);      // slab 2
    release(pool, p);
    CHECK(pool.empty_cache() == 0);
    CHECK(rt.synchronized.size() == 1 && rt.synchronized[0] == stream(2));
    CHECK(pool.stats().slabs == 1 && pool.stats().reserved_bytes == 4096 && rt.slabs() == 1);
    CHECK(rt.created == 0 && rt.records.empty());
    release(pool, keep);
  }
  {  // Budget: an exact-size slab when the default one does not fit, then out of memory.
    MockRuntime rt;
    gk::BlockAllocator pool(rt, 6144, 4096);
    void* a = alloc(pool, 4096, 1);
    void* b = alloc(pool, 2048, 1);
    void* c = nullptr;
    CHECK(pool.allocate(256, stream(1), &c) == gk::BlockAllocator::kOutOfMemory && !c);
    CHECK(pool.error().find("budget") != std::string::npos);
    release(pool, a);
    release(pool, b);
  }
  {  // Steady state across two streams: events come from the pool, none is created.
    MockRuntime rt;
    gk::BlockAllocator pool(rt, 1 << 20, 1 << 16);
    auto cycle = [&](int i) {
      void* p = alloc(pool, 256 * (1 + i % 7), i % 2 ? 1 : 2);
      CHECK(pool.record_stream(p, stream(i % 2 ? 2 : 1)) == 0);
      void* q = alloc(pool, 4096, 1);
      release(pool, p);
      release(pool, q);
    };
    for (int i = 0; i < 10; ++i) cycle(i);
    const uint64_t warm = rt.created;
    CHECK(warm >= 1 && warm <= 2);
    const size_t waits_before = rt.waits.size();
    for (int i = 10; i < 1010; ++i) cycle(i);
    CHECK(rt.created == warm);
    CHECK(rt.waits.size() > waits_before);  // the cycles did fence
    CHECK(pool.stats().allocated_bytes == 0);
  }
  {  // tests/block_allocator_device_test.cpp:27-58: 256-byte blocks and their
     // accounting, a neighbour merge, the whole slab coalescing back after a
     // random allocate/free stress, and peak accounting (one stream: no fence).
    MockRuntime rt;
    constexpr uint64_t slab = 4 << 20;
    gk::BlockAllocator pool(rt, slab, slab);
    void* a = alloc(pool, 1, 1);
    void* b = alloc(pool, 257, 1);
    void* c = alloc(pool, 9, 1);
    CHECK(pool.stats().allocated_bytes == 1024);
    release(pool, b);
    release(pool, a);
    void* merged = alloc(pool, 768, 1);
    CHECK(merged == a);
    release(pool, merged);
    release(pool, c);
    void* entire = alloc(pool, slab, 1);
    CHECK(entire == a);
    release(pool, entire);
    std::mt19937 rng(12345);
    std::vector<void*> live;
    for (int i = 0; i < 2000; ++i) {
      if (!live.empty() && rng() % 2) {
        const size_t index = rng() % live.size();
        release(pool, live[index]);
        live.erase(live.begin() + static_cast<std::ptrdiff_t>(index));
      } else {
        live.push_back(alloc(pool, 1 + rng() % 2048, 1));
      }
    }
    for (void* p : live) release(pool, p);
    entire = alloc(pool, slab, 1);
    CHECK(entire == a);
    release(pool, entire);
    CHECK(pool.stats().allocated_bytes == 0 && pool.stats().peak_bytes == slab && pool.stats().slabs == 1);
    CHECK(rt.created == 0 && rt.waits.empty());
  }
  std::printf("OK\n");
  return 0;
}
