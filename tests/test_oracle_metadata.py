"""Pin the oracle's device-metadata validation and paged slot allocator.

Known answers come from the reference's own tests: the rejection cases of
tests/paged_device_metadata_smoke.py:109-125 on that test's data, and the
expected slots and pages of tests/paged_slots_device_smoke.py,
tests/paged_attention_generalized_smoke.py:146-158 and
tests/dynamic_eager_ops_smoke.py:383-418, evaluated here as literal lists.
The accept/reject decision is also checked against a set-based brute force of
the host constructor's rules (src/bridge/paged_metadata.cpp:82-138) on random
corruptions. The host constructor's reported failure (host_metadata_error) is
pinned by the reference's tests/paged_metadata_smoke.py cases, by the order
its loops impose, and against the device codes on random layouts.
"""

import numpy as np
import pytest

from oracle import oracle as orc

# tests/paged_device_metadata_smoke.py:17-46 ("small" geometry).
REQUESTS, CONTEXT = 8, 1024
SLOTS = REQUESTS * CONTEXT + 1
REQUEST_ORDER = [7, 2, 5, 1, 6, 0, 4, 3]


def smoke_data(rows):
    """The reference smoke test's valid layout for `rows` token rows."""
    mapping = np.arange(1, SLOTS, dtype=np.int32).reshape(REQUESTS, CONTEXT)
    batch = min(rows, REQUESTS)
    requests = np.array(REQUEST_ORDER[:batch], dtype=np.int64)
    lengths = [rows // batch + int(i < rows % batch) for i in range(batch)]
    prefixes = [2 + i for i in range(batch)]
    row_requests = np.repeat(requests, lengths)
    positions = np.concatenate([np.arange(p, p + n, dtype=np.int64) for p, n in zip(prefixes, lengths)])
    locations = mapping[row_requests, positions].astype(np.int64)
    return locations, requests, positions, mapping, prefixes, lengths


def first_error(codes):
    bad = [(i, c) for i, c in enumerate(codes) if c]
    return bad[0] if bad else None


@pytest.mark.parametrize("rows", [1, 7, 33, 137, 1025, 4096])
def test_reference_layouts_are_valid(rows):
    locations, requests, positions, mapping, prefixes, lengths = smoke_data(rows)
    assert first_error(orc.metadata_codes(locations, requests, positions, mapping, prefixes, lengths, SLOTS)) is None


def test_reference_rejection_codes():
    locations, requests, positions, mapping, prefixes, lengths = smoke_data(7)

    def code(loc=locations, req=requests, pos=positions, mp=mapping, pre=prefixes, lens=lengths):
        return first_error(orc.metadata_codes(loc, req, pos, mp, pre, lens, SLOTS))

    big = 1 << 32
    assert code(loc=locations + np.eye(7, dtype=np.int64)[0] * big) == (0, 1)
    assert code(req=requests + np.eye(7, dtype=np.int64)[0] * big) == (0, 2)
    assert code(pos=positions + np.eye(7, dtype=np.int64)[0] * big) == (0, 1)
    assert code(loc=locations + np.eye(7, dtype=np.int64)[0]) == (0, 3)
    bad = mapping.copy()
    bad[requests[0], 0] = -1
    assert code(mp=bad) == (0, 6)
    bad = mapping.copy()
    bad[requests[1], 0] = locations[0]
    assert code(mp=bad) == (1, 7)
    dup_req, dup_pos = np.array([0, 0]), np.array([2, 2])
    dup_loc = mapping[dup_req, dup_pos].astype(np.int64)
    assert first_error(orc.metadata_codes(dup_loc, dup_req, dup_pos, mapping, [2, 2], [1, 1], SLOTS)) == (1, 4)


def host_constructor_accepts(locations, batch_requests, positions, mapping, prefixes, lengths, slots):
    """Set-based restatement of the host constructor's decision plus the
    device layout (position = prefix + offset)."""
    request_count, context = mapping.shape
    row_requests = np.repeat(np.asarray(batch_requests), lengths)
    expected = np.concatenate([np.arange(p, p + n) for p, n in zip(prefixes, lengths)])
    if not np.array_equal(np.asarray(positions), expected):
        return False
    targets = {}
    for loc, req, pos in zip(locations, row_requests, positions):
        if not (0 <= loc < slots and 0 <= req < request_count and 0 <= pos < context):
            return False
        if mapping[req, pos] != loc or loc in targets:
            return False
        targets[int(loc)] = (int(req), int(pos))
    for req in set(int(r) for r in row_requests):
        last = max(int(p) for r, p in zip(row_requests, positions) if r == req)
        for t in range(last + 1):
            slot = int(mapping[req, t])
            if slot < 0 or targets.get(slot, (req, t)) != (req, t):
                return False
    return True


def test_accept_reject_matches_brute_force():
    rng = np.random.default_rng(42)
    outcomes = set()
    for trial in range(400):
        requests_n, context, slots = 4, 24, 200
        mapping = rng.permutation(slots)[: requests_n * context].reshape(requests_n, context).astype(np.int32)
        batch = int(rng.integers(1, 4))
        batch_requests = rng.permutation(requests_n)[:batch].astype(np.int64)
        prefixes = [int(rng.integers(0, 12)) for _ in range(batch)]
        lengths = [int(rng.integers(1, 6)) for _ in range(batch)]
        kind = trial % 8
        if kind == 6:  # the first sequence twice: its rows write the same slots again
            batch_requests = np.concatenate([batch_requests[:1], batch_requests])
            prefixes, lengths = prefixes[:1] + prefixes, lengths[:1] + lengths
        row_req = np.repeat(batch_requests, lengths)
        positions = np.concatenate([np.arange(p, p + n) for p, n in zip(prefixes, lengths)]).astype(np.int64)
        locations = mapping[row_req, positions].astype(np.int64)
        r = int(rng.integers(0, len(locations)))
        if kind == 1:
            locations[r] = mapping[row_req[r], (positions[r] + 1) % context]
        elif kind == 2:
            mapping[batch_requests[0], int(rng.integers(0, prefixes[0] + 1))] = -1
        elif kind == 3:
            other = (batch_requests[0] + 1) % requests_n
            mapping[other, 0] = locations[r]
        elif kind == 4:  # position off the sequence layout, location consistent with it
            positions[r] += 1
            locations[r] = mapping[row_req[r], positions[r]]
        elif kind == 5:
            locations[r] = slots + int(rng.integers(0, 3))
        elif kind == 7:
            batch_requests[0] = requests_n
        codes = orc.metadata_codes(locations, batch_requests, positions, mapping, prefixes, lengths, slots)
        accept = host_constructor_accepts(locations, batch_requests, positions, mapping, prefixes, lengths, slots)
        assert (first_error(codes) is None) == accept, (trial, codes)
        outcomes.update(set(codes))
    assert outcomes == {0, 1, 2, 3, 4, 5, 6, 7}, outcomes


def reference_smoke_metadata(rows):
    """tests/paged_metadata_smoke.py:14-19 of the reference (192 slots)."""
    mapping = np.arange(192, dtype=np.int32).reshape(3, 64)
    requests = np.arange(rows, dtype=np.int64) % 3
    positions = np.arange(rows, dtype=np.int64) // 3 + 2
    return mapping[requests, positions].astype(np.int64), requests, positions, mapping


def test_host_metadata_error_reference_smoke():
    """Known answers: the host constructor cases of the reference's
    tests/paged_metadata_smoke.py:33-50, on that test's data."""
    for rows in (1, 3, 17, 137):
        assert orc.host_metadata_error(*reference_smoke_metadata(rows), 192) is None
    locations, requests, positions, mapping = reference_smoke_metadata(7)
    duplicate, dup_requests, dup_positions = locations.copy(), requests.copy(), positions.copy()
    duplicate[1], dup_requests[1], dup_positions[1] = duplicate[0], requests[0], positions[0]
    assert orc.host_metadata_error(duplicate, dup_requests, dup_positions, mapping, 192) == "duplicate output KV slot"
    invalid = locations.copy()
    invalid[0] = 192
    assert "out of range" in orc.host_metadata_error(invalid, requests, positions, mapping, 192)
    missing = mapping.copy()
    missing[0, 0] = -1
    assert "missing KV slot" in orc.host_metadata_error(locations, requests, positions, missing, 192)
    alias = mapping.copy()
    alias[1, 0] = locations[0]
    assert "aliases another visible prefix" in orc.host_metadata_error(locations, requests, positions, alias, 192)
    mismatch = mapping.copy()
    mismatch[requests[0], positions[0]] = 191
    assert "does not match" in orc.host_metadata_error(locations, requests, positions, mismatch, 192)


def test_host_metadata_error_order():
    """The first failure in the reference's order is the one reported: the map
    range before any row, rows in order (range, agreement, repeat), then
    prefixes request by request and position by position."""
    locations, requests, positions, mapping = reference_smoke_metadata(7)
    err = lambda loc=locations, req=requests, pos=positions, mp=mapping: orc.host_metadata_error(  # noqa: E731
        loc, req, pos, mp, 192)
    beyond = mapping.copy()
    beyond[2, 63] = 192  # outside every prefix
    bad_loc = locations.copy()
    bad_loc[3] = 5
    assert err(mp=beyond, loc=bad_loc) == "request-to-token slot is out of range"
    assert err(loc=bad_loc) == "output slot does not match request-to-token mapping"
    hole = mapping.copy()
    hole[0, 0] = -1
    assert err(loc=bad_loc, mp=hole) == "output slot does not match request-to-token mapping"
    # request 0 aliases at position 1, request 1 misses position 0: request 0 first
    both = mapping.copy()
    both[0, 1] = locations[1]
    both[1, 0] = -1
    assert err(mp=both) == "output KV slot aliases another visible prefix position"
    # within one request the earlier position wins
    both = mapping.copy()
    both[1, 0] = -1
    both[1, 1] = locations[0]
    assert err(mp=both) == "missing KV slot in a visible prefix"
    # a row's own output slot at its own position is not an alias
    assert err() is None


def test_host_metadata_error_agrees_with_device_codes():
    """On sequence layouts (no position off the layout, code 5), the host
    constructor accepts exactly the rows the device validation gives no code."""
    rng = np.random.default_rng(43)
    seen = set()
    for trial in range(300):
        requests_n, context, slots = 4, 24, 200
        mapping = rng.permutation(slots)[: requests_n * context].reshape(requests_n, context).astype(np.int32)
        batch = int(rng.integers(1, 4))
        batch_requests = rng.permutation(requests_n)[:batch].astype(np.int64)
        prefixes = [int(rng.integers(0, 12)) for _ in range(batch)]
        lengths = [int(rng.integers(1, 6)) for _ in range(batch)]
        row_req = np.repeat(batch_requests, lengths)
        positions = np.concatenate([np.arange(p, p + n) for p, n in zip(prefixes, lengths)]).astype(np.int64)
        locations = mapping[row_req, positions].astype(np.int64)
        r = int(rng.integers(0, len(locations)))
        kind = trial % 5
        if kind == 1:
            locations[r] = mapping[row_req[r], (positions[r] + 1) % context]
        elif kind == 2:
            mapping[batch_requests[0], int(rng.integers(0, prefixes[0] + 1))] = -1
        elif kind == 3:
            mapping[(batch_requests[0] + 1) % requests_n, 0] = locations[r]
        elif kind == 4:
            locations[r] = slots + int(rng.integers(0, 3))
        codes = orc.metadata_codes(locations, batch_requests, positions, mapping, prefixes, lengths, slots)
        error = orc.host_metadata_error(locations, row_req, positions, mapping, slots)
        assert (error is None) == (first_error(codes) is None), (trial, codes, error)
        seen.add(error)
    assert len(seen) >= 4, seen


def test_page_flags_closed_forms():
    ident = np.arange(4 * 2048, dtype=np.int32).reshape(4, 2048)
    assert orc.largest_page(orc.page_flags(ident, [0, 3], [100, 0], [50, 2048])) == 1024
    assert orc.page_flags(ident + 1, [1], [0], [3]) == (1 << 10) - 1
    rng = np.random.default_rng(3)
    for page in (2, 16, 32, 128, 512):
        blocks = rng.permutation(64)[:8] * 2 + 1  # odd block ids: no larger page lines up
        mapping = (blocks[:, None] * page + np.arange(page)).reshape(1, -1).astype(np.int32)
        flags = orc.page_flags(mapping, [0], [0], [mapping.shape[1]])
        assert orc.largest_page(flags) == page, (page, bin(flags))
    # A hole in the visible range (slot -1) fails every page size; beyond it nothing is checked.
    hole = ident.copy()
    hole[0, 10] = -1
    assert orc.page_flags(hole, [0], [0], [11]) == (1 << 10) - 1
    assert orc.largest_page(orc.page_flags(hole, [0], [0], [10])) == 1024


# tests/paged_slots_device_smoke.py, evaluated.
SMOKE_SLOTS = {
    16: list(range(208, 224)) + [112, 113, 114] + list(range(1303, 1312)) + list(range(368, 373)) +
        list(range(656, 672)) + list(range(192, 196)) + [1343] + list(range(528, 544)) + list(range(880, 896)) +
        list(range(976, 992)) + list(range(240, 256)) + [288],
    64: list(range(832, 851)) + list(range(5191, 5205)) + list(range(448, 468)) + [5375] +
        list(range(1472, 1536)) + [2624],
}
SMOKE_USED = {16: 10, 64: 4}


@pytest.mark.parametrize("page", [16, 64])
def test_allocator_reference_smoke(page):
    prefixes, lengths = [0, 7, page, 2 * page - 1], [19, 14, 20, 66]
    previous = [-1, 81 * page + 6, 82 * page + page - 1, 83 * page + page - 2]
    pages = [13, 7, 23, 41, 12, 33, 55, 61, 15, 18, 19, 20, 21, 22, 24, 25]
    slots, used = orc.allocate_paged_slots(previous, pages, prefixes, lengths, page)
    assert slots == SMOKE_SLOTS[page] and used == SMOKE_USED[page]
    released = [13 * page + 7, 7 * page, 13 * page, 23 * page + page - 1, 7 * page + 3]
    assert orc.release_paged_slots(released, page, 512) == [13, 7, 23]
    for invalid in (0, 513 * page, 1 << 40):
        with pytest.raises(ValueError, match="outside the KV pool"):
            orc.release_paged_slots([invalid], page, 512)


def test_allocator_generalized_and_dynamic_cases():
    # tests/paged_attention_generalized_smoke.py:146-158 at P = 8 and P = 1.
    slots, used = orc.allocate_paged_slots([-1, 802, 1607], list(range(10, 80)), [0, 3, 8], [5, 7, 10], 8)
    assert slots == [80, 81, 82, 83, 84, 803, 804, 805, 806, 807, 88, 89] + list(range(96, 104)) + [104, 105]
    assert used == 4
    slots, used = orc.allocate_paged_slots([-1, 100, 200], list(range(10, 80)), [0, 3, 1], [5, 7, 3], 1)
    assert slots == list(range(10, 25)) and used == 15
    assert orc.release_paged_slots([9000 * 8, 9000 * 8 + 7, 12000 * 8], 8, 16384) == [9000, 12000]
    # tests/dynamic_eager_ops_smoke.py:383-405: a sequence with no previous slot
    # (last = -1) still continues from it inside its first partial page.
    slots, used = orc.allocate_paged_slots([-1, -1], list(range(100, 112)), [0, 3], [5, 7], 16)
    assert slots == [1600, 1601, 1602, 1603, 1604, 0, 1, 2, 3, 4, 5, 6] and used == 1


def test_allocator_invariants():
    rng = np.random.default_rng(9)
    for page in (2, 16, 128):
        batch = 6
        prefixes = [int(x) for x in rng.integers(0, 3 * page, batch)]
        lengths = [int(x) for x in rng.integers(0, 4 * page, batch)]
        held = rng.permutation(np.arange(1, 500))[:batch]
        last = [int(h) * page + (p - 1) % page if p % page else -1 for h, p in zip(held, prefixes)]
        free = [int(x) for x in rng.permutation(np.arange(500, 900))]
        slots, used = orc.allocate_paged_slots(last, free, prefixes, lengths, page)
        assert len(slots) == sum(lengths) and len(set(slots)) == len(slots)
        positions = [p + i for p, n in zip(prefixes, lengths) for i in range(n)]
        assert all(s % page == t % page for s, t in zip(slots, positions))
        new_pages = orc.release_paged_slots([s for s in slots if s // page >= 500], page, 1000)
        assert new_pages == free[:used]
