"""GPU tests of the stream-ordered block allocator through the C ABI (gk_allocator_*).

The reference pins the contract of its BlockCachingAllocator in
tests/block_allocator_fences_unit_test.cpp:25-71 (CPU, mocked events; here
tests/test_allocator_fences.py). On the GPU: a block freed while its producer
stream still has queued writes, and reallocated on another stream, is only
touched there after those writes (the consumer waits on an event, the host
never synchronises); a thousand alloc / record_stream / free cycles over
two streams create no new events once warm; blocks written by two streams
merge and serve a third (tests/block_allocator_device_test.cpp:114-135); and
three streams passing one block round reuse their events
(tests/allocator_event_reuse_device_test.cpp:22-69).
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


def test_cross_stream_coalescing_rounds(env):
    """tests/block_allocator_device_test.cpp:114-135: 128 rounds of two adjacent
    blocks written by two producer streams (the second alternating between two
    streams, and queued behind a longer write so that it is still running),
    freed in alternating order, merged and handed out whole to a third stream,
    whose reads must see both producers' writes."""
    torch, capi, lib = env
    a = ctypes.c_void_p()
    capi.check(lib.gk_allocator_create(0, 1 << 30, 64 << 20, ctypes.byref(a)))
    s, h2d, d2h = torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()  # default priority
    hs, hh, hd = (ctypes.c_void_p(x.cuda_stream) for x in (s, h2d, d2h))
    n = 8192  # 64 KiB of int64 per block
    src = torch.arange(n, dtype=torch.int64, device="cuda") + 12345
    orig = torch.zeros(2 * n, dtype=torch.int32, device="cuda")
    orig_next = [torch.empty_like(orig) for _ in range(3)]
    big = 1 << 23
    big_src = torch.zeros(big, dtype=torch.int64, device="cuda")
    big_dst = [torch.empty_like(big_src) for _ in range(2)]
    big_orig = torch.zeros(big, dtype=torch.int32, device="cuda")
    big_orig_next = [torch.empty_like(big_orig) for _ in range(2)]
    check = torch.empty(2 * n, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()

    def advance(seq, dst, count, scratch, stream):
        capi.check(lib.gk_advance_decode_lengths(seq, ctypes.c_void_p(orig.data_ptr()), count, dst,
                                                 ctypes.c_void_p(scratch.data_ptr()), stream))

    for it in range(128):
        left, right = ctypes.c_void_p(), ctypes.c_void_p()
        capi.check(lib.gk_allocator_alloc(a, 8 * n, hs, ctypes.byref(left)))
        capi.check(lib.gk_allocator_alloc(a, 8 * n, hs, ctypes.byref(right)))
        assert right.value == left.value + 8 * n, "blocks of one round are not adjacent"
        second, k = (hd, 1) if it % 2 else (hh, 0)
        advance(ctypes.c_void_p(src.data_ptr()), left, n, orig_next[0], hh)
        capi.check(lib.gk_advance_decode_lengths(ctypes.c_void_p(big_src.data_ptr()),
                                                 ctypes.c_void_p(big_orig.data_ptr()), big,
                                                 ctypes.c_void_p(big_dst[k].data_ptr()),
                                                 ctypes.c_void_p(big_orig_next[k].data_ptr()), second))
        advance(ctypes.c_void_p(src.data_ptr()), right, n, orig_next[1], second)
        capi.check(lib.gk_allocator_record_stream(a, left, hh))
        capi.check(lib.gk_allocator_record_stream(a, right, second))
        for p in ((right, left) if it % 2 else (left, right)):
            capi.check(lib.gk_allocator_free(a, p))
        combined = ctypes.c_void_p()
        capi.check(lib.gk_allocator_alloc(a, 16 * n, hs, ctypes.byref(combined)))
        assert combined.value == left.value, "the two blocks did not merge"
        advance(combined, ctypes.c_void_p(check.data_ptr()), 2 * n, orig_next[2], hs)  # check = block + 1
        torch.cuda.synchronize()
        assert bool((check[:n] == src + 2).all()) and bool((check[n:] == src + 2).all()), f"round {it}"
        capi.check(lib.gk_allocator_free(a, combined))
    st = stats(capi, lib, a)
    print(f"events created {st.events_created}, slabs {st.slabs}", flush=True)
    assert st.allocated_bytes == 0 and st.slabs == 1 and st.events_created <= 4
    capi.check(lib.gk_allocator_destroy(a))


def test_three_stream_event_reuse_keeps_data_ordered(env):
    """tests/allocator_event_reuse_device_test.cpp:22-69: 512 steps, each
    writing a 256-byte block on one of three streams, freeing it, taking the
    same block back on the next stream and copying it out there, with no host
    wait; once the three streams are primed no event is created, and every
    copy saw its own step's write."""
    torch, capi, lib = env
    a = ctypes.c_void_p()
    capi.check(lib.gk_allocator_create(0, 1 << 30, 64 << 20, ctypes.byref(a)))
    streams = [torch.cuda.Stream() for _ in range(3)]  # default priority
    handles = [ctypes.c_void_p(x.cuda_stream) for x in streams]
    steps, words = 512, 32  # 256 bytes of int64 per step
    idx = torch.arange(steps * words, dtype=torch.int64).reshape(steps, words)
    host_in = (idx // words * 37 + idx % words * 19) & 255
    inp = host_in.cuda()
    out = torch.full_like(inp, -1)
    orig = torch.zeros(words, dtype=torch.int32, device="cuda")
    orig_next = [torch.empty_like(orig) for _ in streams]
    torch.cuda.synchronize()

    def advance(src, dst, k):
        capi.check(lib.gk_advance_decode_lengths(src, ctypes.c_void_p(orig.data_ptr()), words, dst,
                                                 ctypes.c_void_p(orig_next[k].data_ptr()), handles[k]))

    def step(i):
        prod, cons = i % 3, (i + 1) % 3
        target = ctypes.c_void_p()
        capi.check(lib.gk_allocator_alloc(a, 8 * words, handles[prod], ctypes.byref(target)))
        advance(ctypes.c_void_p(inp[i].data_ptr()), target, prod)          # block = input + 1
        capi.check(lib.gk_allocator_free(a, target))
        reused = ctypes.c_void_p()
        capi.check(lib.gk_allocator_alloc(a, 8 * words, handles[cons], ctypes.byref(reused)))
        assert reused.value == target.value, f"step {i}: allocation not reused"
        advance(reused, ctypes.c_void_p(out[i].data_ptr()), cons)          # out = block + 1
        capi.check(lib.gk_allocator_free(a, reused))

    for i in range(3):
        step(i)
    warm = stats(capi, lib, a).events_created
    for i in range(3, steps):
        step(i)
    torch.cuda.synchronize()
    st = stats(capi, lib, a)
    print(f"events created: {warm} after priming, {st.events_created} after {steps} steps", flush=True)
    assert st.events_created == warm and 1 <= warm <= 3
    assert torch.equal(out.cpu(), host_in + 2), "a consumer read its block before the producer's write"
    assert st.allocated_bytes == 0
    capi.check(lib.gk_allocator_destroy(a))
