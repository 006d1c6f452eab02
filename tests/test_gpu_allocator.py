"""GPU tests of the stream-ordered block allocator through the C ABI (gk_allocator_*).

The reference pins the contract of its BlockCachingAllocator in
tests/block_allocator_fences_unit_test.cpp:25-71 (CPU, mocked events; here
tests/test_allocator_fences.py). On the GPU: a block freed while its producer
stream still has queued writes, and reallocated on another stream, is only
touched there after those writes (the consumer waits on an event, the host
never synchronises); and a thousand alloc / record_stream / free cycles over
two streams create no new events once warm.
"""

import ctypes

import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch

    from gaudirt_amd import capi

    assert torch.cuda.is_available()
    return torch, capi, capi.load()


def stats(capi, lib, a):
    s = capi.AllocatorStats()
    capi.check(lib.gk_allocator_get_stats(a, ctypes.byref(s)))
    return s


def test_cross_stream_reuse_orders_after_the_producer(env):
    torch, capi, lib = env
    a = ctypes.c_void_p()
    capi.check(lib.gk_allocator_create(0, 4 << 30, 1 << 30, ctypes.byref(a)))
    n = 1 << 26  # 64 M int64 = 512 MiB per buffer
    seq_a = torch.full((n,), 1000, dtype=torch.int64, device="cuda")
    seq_b = torch.full((n,), 2000, dtype=torch.int64, device="cuda")
    orig = torch.zeros(n, dtype=torch.int32, device="cuda")
    orig_next = torch.empty_like(orig)
    check = torch.empty(n, dtype=torch.int64, device="cuda")
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()  # default priority
    torch.cuda.synchronize()
    h1, h2 = ctypes.c_void_p(s1.cuda_stream), ctypes.c_void_p(s2.cuda_stream)
    p = ctypes.c_void_p()
    capi.check(lib.gk_allocator_alloc(a, n * 8, h1, ctypes.byref(p)))

    def advance(src, dst, stream):
        capi.check(lib.gk_advance_decode_lengths(src, ctypes.c_void_p(orig.data_ptr()), n, dst,
                                                 ctypes.c_void_p(orig_next.data_ptr()), stream))

    # The producer: ~10 ms of writes of 1001 into the block, queued on s1.
    for _ in range(40):
        advance(ctypes.c_void_p(seq_a.data_ptr()), p, h1)
    print("producer queued on s1; freeing and reallocating on s2 without a host wait", flush=True)
    capi.check(lib.gk_allocator_free(a, p))
    q = ctypes.c_void_p()
    capi.check(lib.gk_allocator_alloc(a, n * 8, h2, ctypes.byref(q)))
    assert q.value == p.value, "best fit should hand the same block back"
    advance(ctypes.c_void_p(seq_b.data_ptr()), q, h2)                 # block = 2001, after the fence
    advance(q, ctypes.c_void_p(check.data_ptr()), h2)                 # check = block + 1
    torch.cuda.synchronize()
    assert bool((check == 2002).all()), "the consumer stream touched the block before the producer finished"
    s = stats(capi, lib, a)
    assert s.events_created == 1 and s.allocated_bytes == n * 8
    capi.check(lib.gk_allocator_free(a, q))
    capi.check(lib.gk_allocator_destroy(a))


def test_two_stream_cycles_create_no_events_when_warm(env):
    torch, capi, lib = env
    a = ctypes.c_void_p()
    capi.check(lib.gk_allocator_create(0, 1 << 30, 64 << 20, ctypes.byref(a)))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    handles = [ctypes.c_void_p(s1.cuda_stream), ctypes.c_void_p(s2.cuda_stream)]
    n = 4096
    seq = torch.arange(n, dtype=torch.int64, device="cuda")
    orig = torch.zeros(n, dtype=torch.int32, device="cuda")
    orig_next = torch.empty_like(orig)
    torch.cuda.synchronize()

    def cycle(i):
        mine, other = handles[i % 2], handles[1 - i % 2]
        p = ctypes.c_void_p()
        capi.check(lib.gk_allocator_alloc(a, 8 * n + 256 * (i % 5), mine, ctypes.byref(p)))
        capi.check(lib.gk_advance_decode_lengths(ctypes.c_void_p(seq.data_ptr()), ctypes.c_void_p(orig.data_ptr()), n,
                                                 p, ctypes.c_void_p(orig_next.data_ptr()), mine))
        capi.check(lib.gk_allocator_record_stream(a, p, other))
        capi.check(lib.gk_allocator_free(a, p))

    for i in range(10):
        cycle(i)
    warm = stats(capi, lib, a).events_created
    assert 1 <= warm <= 2, warm
    for i in range(10, 1010):
        cycle(i)
    torch.cuda.synchronize()
    s = stats(capi, lib, a)
    print(f"events created: {warm} warm, {s.events_created} after 1000 more cycles; slabs {s.slabs}", flush=True)
    assert s.events_created == warm and s.allocated_bytes == 0 and s.slabs == 1
    capi.check(lib.gk_allocator_empty_cache(a))
    assert stats(capi, lib, a).reserved_bytes == 0
    capi.check(lib.gk_allocator_destroy(a))
