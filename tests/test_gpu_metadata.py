"""GPU parity of the device-side metadata builder/validator and the paged slot allocator.

Follows the reference's device smokes: tests/paged_device_metadata_smoke.py
(SGLang-shaped device page maps, rows 1..4096, int32 positions, strided
inputs, rejection codes 1/2/1/3/6/7/4 and "sequence lengths"),
tests/token_metadata_smoke.py, tests/scheduler_metadata_async_smoke.py
(scheduler metadata equals the checked metadata and does not wait for queued
device work), tests/scheduler_metadata_fused_smoke.py (host positions, the
fused plan), tests/paged_slots_device_smoke.py and the allocator cases of
tests/paged_attention_generalized_smoke.py. Status codes, page flags and the
normalised rows are compared with the CPU oracle bit for bit through the C ABI;
attention through device-built metadata equals attention through the host
constructor's metadata bit for bit, and the oracle within max-abs 2e-2 /
mean-abs 2e-3.
"""

import ctypes
import math

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3

# tests/paged_device_metadata_smoke.py:17-46 ("small" geometry).
REQUESTS, CONTEXT = 8, 1024
SLOTS = REQUESTS * CONTEXT + 1
REQUEST_ORDER = [7, 2, 5, 1, 6, 0, 4, 3]


@pytest.fixture(scope="module")
def torch_ext():
    import torch

    import gaudirt_amd

    assert torch.cuda.is_available()
    gaudirt_amd.load_extension()
    return torch


def smoke_data(torch, rows):
    mapping = torch.arange(1, SLOTS, dtype=torch.int32).reshape(REQUESTS, CONTEXT)
    batch = min(rows, REQUESTS)
    requests = torch.tensor(REQUEST_ORDER[:batch], dtype=torch.int64)
    lengths = [rows // batch + int(i < rows % batch) for i in range(batch)]
    prefixes = [2 + i for i in range(batch)]
    row_requests = torch.repeat_interleave(requests, torch.tensor(lengths))
    positions = torch.cat([torch.arange(p, p + n, dtype=torch.int64) for p, n in zip(prefixes, lengths)])
    locations = mapping[row_requests, positions].to(torch.int64)
    return locations, requests, positions, mapping, prefixes, lengths, row_requests


def to_device(torch, source, sliced=False):
    """A device copy of `source`; a stride-2 view of a wider buffer when sliced."""
    if not sliced:
        return source.cuda()
    storage = torch.empty(source.numel() * 2, dtype=source.dtype, device="cuda")
    view = storage[::2]
    view.copy_(source)
    return view


def prepare(torch, locations, requests, positions, mapping, prefixes, lengths, sliced=False):
    inputs = [to_device(torch, t, sliced) for t in (locations, requests, positions)]
    return torch.classes.gaudirt.PagedMetadata.from_device(*inputs, mapping.cuda(), prefixes, lengths, SLOTS), inputs


# ---------------------------------------------------------------------------
# C ABI: every row's code, the page flags and the normalised rows
# ---------------------------------------------------------------------------

def normalize(torch, locations, batch_requests, positions, mapping, prefixes, lengths, slots, tokens=None,
              vocabulary=0, validate=True, staged=False):
    """Runs gk_metadata_normalize. With `staged`, row_seq, seq_prefix,
    seq_first_row, seq_visible (and positions, where they fit) are passed as
    staged words: the launch stores them itself into a device buffer that the
    input pointers name, and result["staged"] holds that buffer afterwards."""
    from gaudirt_amd import capi

    lib = capi.load()
    rows, batch = len(locations), len(prefixes)
    padded = 1 << (rows - 1).bit_length()
    row_seq = np.repeat(np.arange(batch, dtype=np.int32), lengths)
    first = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int32)
    visible = np.array(prefixes, dtype=np.int64) + np.array(lengths, dtype=np.int64)
    seq_visible = np.concatenate([[0], np.cumsum(visible)[:-1]]).astype(np.int64)
    dev = {name: torch.from_numpy(np.ascontiguousarray(a)).cuda() for name, a in (
        ("loc", locations), ("req", batch_requests), ("pos", positions), ("map", mapping), ("row_seq", row_seq),
        ("prefix", np.array(prefixes, dtype=np.int32)), ("first", first), ("visible", seq_visible))}
    if tokens is not None:
        dev["tok"] = torch.from_numpy(np.ascontiguousarray(tokens)).cuda()
    out = {name: torch.full((padded,), -7, dtype=torch.int32, device="cuda")
           for name in ("loc", "req", "pos", "tok", "status", "token_status")}
    flags = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    p = capi.MetadataParams()
    p.locations, p.batch_requests, p.positions = (dev[n].data_ptr() for n in ("loc", "req", "pos"))
    p.locations_int64 = int(dev["loc"].dtype == torch.int64)
    p.requests_int64 = int(dev["req"].dtype == torch.int64)
    p.positions_int64 = int(dev["pos"].dtype == torch.int64)
    if tokens is not None:
        p.token_ids = dev["tok"].data_ptr()
        p.tokens_int64 = int(dev["tok"].dtype == torch.int64)
        p.out_tokens = out["tok"].data_ptr()
        p.token_status = out["token_status"].data_ptr()
    p.mapping = dev["map"].data_ptr() if validate else None
    p.row_seq, p.seq_prefix, p.seq_first_row, p.seq_visible = (
        dev[n].data_ptr() for n in ("row_seq", "prefix", "first", "visible"))
    p.visible_total = int(visible.sum())
    p.rows, p.padded_rows, p.batch = rows, padded, batch
    p.requests, p.context = mapping.shape
    p.vocabulary, p.slots = vocabulary, slots
    p.out_locations, p.out_requests, p.out_positions = (out[n].data_ptr() for n in ("loc", "req", "pos"))
    if validate:
        p.status = out["status"].data_ptr()
        p.page_flags = flags.data_ptr()
    if staged:
        sections = [("row_seq", row_seq), ("prefix", np.array(prefixes, dtype=np.int32)), ("first", first),
                    ("visible", seq_visible)]
        if np.asarray(positions).nbytes // 4 + sum(a.nbytes // 4 for _, a in sections) <= capi.GK_METADATA_INLINE_WORDS:
            sections.append(("pos", np.ascontiguousarray(positions)))
        host = np.concatenate([a.view(np.int32) for _, a in sections]).astype(np.int32)
        assert host.size <= capi.GK_METADATA_INLINE_WORDS
        staged_dev = torch.full((host.size,), -9, dtype=torch.int32, device="cuda")
        offset = 0
        for name, a in sections:
            pointer = staged_dev.data_ptr() + 4 * offset
            if name == "pos":
                p.positions = pointer
            else:
                setattr(p, {"row_seq": "row_seq", "prefix": "seq_prefix", "first": "seq_first_row",
                            "visible": "seq_visible"}[name], pointer)
            offset += a.nbytes // 4
        p.staged_words = host.ctypes.data
        p.staged_device = staged_dev.data_ptr()
        p.staged_count = host.size
    need = lib.gk_metadata_workspace_bytes(rows, batch)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    capi.check(lib.gk_metadata_normalize(ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), need,
                                         capi.current_stream()))
    torch.cuda.synchronize()
    result = {n: t.cpu().numpy() for n, t in out.items()}
    result["flags"] = int(flags.item())
    if staged:
        result["staged"] = staged_dev.cpu().numpy()
        assert np.array_equal(result["staged"], host)
        result["staged_positions"] = sections[-1][0] == "pos"
    return result


def random_problem(rng, kind, requests_n=16, context=512, slots=9000, page=None, max_batch=12):
    if page:
        blocks = rng.permutation(slots // page)[: requests_n * context // page]
        mapping = (blocks[:, None] * page + np.arange(page)).reshape(requests_n, context).astype(np.int32)
    else:
        mapping = rng.permutation(slots)[: requests_n * context].reshape(requests_n, context).astype(np.int32)
    batch = int(rng.integers(1, max_batch))
    batch_requests = rng.permutation(requests_n)[:batch].astype(np.int64)
    prefixes = [int(x) for x in rng.integers(0, 300, batch)]
    lengths = [int(x) for x in rng.integers(1, 40, batch)]
    if kind == 6:
        batch_requests = np.concatenate([batch_requests[:1], batch_requests])
        prefixes, lengths = prefixes[:1] + prefixes, lengths[:1] + lengths
    row_req = np.repeat(batch_requests, lengths)
    positions = np.concatenate([np.arange(p, p + n) for p, n in zip(prefixes, lengths)]).astype(np.int64)
    locations = mapping[row_req, positions].astype(np.int64)
    r = int(rng.integers(0, len(locations)))
    if kind == 1:
        locations[r] = mapping[row_req[r], (positions[r] + 1) % context]
    elif kind == 2:
        mapping[batch_requests[-1], int(rng.integers(0, prefixes[-1] + 1))] = -1
    elif kind == 3:
        other = [q for q in range(requests_n) if q != row_req[r]][0]
        mapping[other, 0] = locations[r]
    elif kind == 4:
        positions[r] += 1
        locations[r] = mapping[row_req[r], positions[r]]
    elif kind == 5:
        locations[r] = [slots, -1, 1 << 33][r % 3]
    elif kind == 7:
        batch_requests[-1] = [requests_n, -1, 1 << 32][r % 3]
    return locations, batch_requests, positions, mapping, prefixes, lengths, slots


@pytest.mark.parametrize("kind", range(8))
def test_status_codes_match_oracle(torch_ext, kind):
    torch = torch_ext
    rng = np.random.default_rng(100 + kind)
    for trial in range(6):
        page = [None, 16, 64][trial % 3]
        loc, req, pos, mapping, prefixes, lengths, slots = random_problem(rng, kind, page=page)
        if trial % 2:  # int32 inputs where they fit
            loc, pos = loc.astype(np.int32) if np.abs(loc).max() < 2**31 else loc, pos.astype(np.int32)
        got = normalize(torch, loc, req, pos, mapping, prefixes, lengths, slots)
        rows = len(loc)
        want = orc.metadata_codes(loc, req, pos, mapping, prefixes, lengths, slots)
        print("kind", kind, "trial", trial, "rows", rows, "codes", sorted(set(want)), flush=True)
        assert list(got["status"][:rows]) == want
        assert (got["status"][rows:] == 0).all()
        assert got["flags"] == orc.page_flags(mapping, req, prefixes, lengths)
        assert np.array_equal(got["loc"][:rows], np.asarray(loc).astype(np.int64).astype(np.int32))
        assert np.array_equal(got["pos"][:rows], np.asarray(pos).astype(np.int64).astype(np.int32))
        assert np.array_equal(got["req"][:rows], np.repeat(req, lengths).astype(np.int32))
        for name in ("loc", "req", "pos"):
            assert (got[name][rows:] == 0).all()


@pytest.mark.parametrize("kind", range(8))
def test_staged_words_match_device_inputs(torch_ext, kind):
    """Staged words carried in the launch (row_seq, seq_prefix, seq_first_row,
    seq_visible and, where they fit, positions) give the same codes, flags and
    rows as the same words read from device memory, and land in the device
    buffer their pointers name."""
    torch = torch_ext
    rng = np.random.default_rng(900 + kind)
    redirected = 0
    for trial in range(4):
        page = [None, 16][trial % 2]
        loc, req, pos, mapping, prefixes, lengths, slots = random_problem(rng, kind, page=page,
                                                                          max_batch=[12, 3][trial % 2])
        if trial >= 2:
            loc, pos = loc.astype(np.int32) if np.abs(loc).max() < 2**31 else loc, pos.astype(np.int32)
        tokens = rng.integers(0, 32000, len(loc)).astype(np.int64)
        plain = normalize(torch, loc, req, pos, mapping, prefixes, lengths, slots, tokens=tokens, vocabulary=32000)
        staged = normalize(torch, loc, req, pos, mapping, prefixes, lengths, slots, tokens=tokens,
                           vocabulary=32000, staged=True)
        print("kind", kind, "trial", trial, "rows", len(loc), "positions staged", staged["staged_positions"],
              flush=True)
        redirected += staged["staged_positions"]
        for name in ("loc", "req", "pos", "tok", "status", "token_status", "flags"):
            assert np.array_equal(plain[name], staged[name]), name
        want = orc.metadata_codes(loc, req, pos, mapping, prefixes, lengths, slots)
        assert list(staged["status"][:len(loc)]) == want
        unchecked = normalize(torch, loc, req, pos, mapping, prefixes, lengths, slots, validate=False, staged=True)
        for name in ("loc", "req", "pos"):
            assert np.array_equal(plain[name], unchecked[name]), name
    assert redirected > 0


def test_tokens_and_unchecked_normalisation(torch_ext):
    torch = torch_ext
    rng = np.random.default_rng(5)
    loc, req, pos, mapping, prefixes, lengths, slots = random_problem(rng, 0)
    rows = len(loc)
    tokens = rng.integers(0, 32000, rows).astype(np.int64)
    tokens[[0, rows - 1]] = [32000, -1]
    got = normalize(torch, loc, req, pos, mapping, prefixes, lengths, slots, tokens=tokens, vocabulary=32000)
    assert np.array_equal(got["tok"][:rows], tokens.astype(np.int32)) and (got["tok"][rows:] == 0).all()
    assert list(got["token_status"][:rows]) == [int(t < 0 or t >= 32000) for t in tokens]
    # Scheduler-owned: no mapping, no codes; the rows are still normalised.
    got = normalize(torch, loc, req, pos, mapping, prefixes, lengths, slots, validate=False)
    assert (got["status"] == -7).all() and got["flags"] == -7
    assert np.array_equal(got["loc"][:rows], loc.astype(np.int32))


def test_block_tables_kernel(torch_ext):
    torch = torch_ext
    from gaudirt_amd import capi

    rng = np.random.default_rng(8)
    page, requests_n, context = 64, 5, 1000
    pages = -(-context // page)
    blocks = rng.permutation(400)[: requests_n * pages]
    mapping = (blocks.reshape(requests_n, pages)[:, :, None] * page + np.arange(page)).reshape(requests_n, -1)
    mapping = mapping[:, :context].astype(np.int32)
    mapping[2, 640:] = -1
    d_map = torch.from_numpy(mapping).cuda()
    tables = torch.full((requests_n, pages), -7, dtype=torch.int32, device="cuda")
    capi.check(capi.load().gk_block_tables(ctypes.c_void_p(d_map.data_ptr()), requests_n, context, page,
                                           ctypes.c_void_p(tables.data_ptr()), pages, capi.current_stream()))
    want = blocks.reshape(requests_n, pages).astype(np.int32)
    want[2, 10:] = -1
    assert np.array_equal(tables.cpu().numpy(), want)


# ---------------------------------------------------------------------------
# torch API: PagedMetadata.from_device and friends
# ---------------------------------------------------------------------------

def attend(torch, meta, pool_base, q, k, v, heads, kv_heads, dim, scale):
    import gaudirt_amd

    pool = gaudirt_amd.allocate_paged_kv(1, SLOTS, kv_heads, dim)
    key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, 0)
    key_pool.copy_(pool_base[0])
    value_pool.copy_(pool_base[1])
    out = torch.ops.gaudirt.paged_attn.default(q, k, v, key_pool, value_pool, meta, dim, scale)
    torch.cuda.synchronize()
    return out, key_pool, value_pool


@pytest.mark.parametrize("rows", [1, 7, 33, 137, 1025, 4096])
def test_from_device_reference_layouts(torch_ext, rows):
    torch = torch_ext
    locations, requests, positions, mapping, prefixes, lengths, row_requests = smoke_data(torch, rows)
    if rows in (33, 1025):
        positions = positions.to(torch.int32)
    meta, keep = prepare(torch, locations, requests, positions, mapping, prefixes, lengths, sliced=rows == 137)
    assert meta.rows() == rows and meta.slots() == SLOTS and meta.context() == CONTEXT
    expected_last = torch.cumsum(torch.tensor(lengths, dtype=torch.int32), dim=0) - 1
    assert meta.last_token_indices().dtype == torch.int32
    assert torch.equal(meta.last_token_indices().cpu(), expected_last)
    assert torch.equal(meta.row_locations().cpu(), locations.to(torch.int32))
    assert torch.equal(meta.row_requests().cpu(), row_requests.to(torch.int32))
    assert torch.equal(meta.rotary_positions().cpu(), positions.to(torch.int32))
    assert meta.rotary_header().cpu().tolist() == [rows]
    if rows == 4096:
        return
    heads, kv_heads, dim = 8, 2, 128
    scale = float(np.float32(1.0 / math.sqrt(dim)))
    gen = torch.Generator().manual_seed(8017 + rows)
    q, k, v = (torch.randn(rows, w, generator=gen).to(torch.bfloat16).cuda()
               for w in (heads * dim, kv_heads * dim, kv_heads * dim))
    base = [torch.randn(SLOTS, kv_heads, dim, generator=gen).to(torch.bfloat16).cuda() for _ in range(2)]
    host_meta = torch.classes.gaudirt.PagedMetadata(locations, row_requests, positions.to(torch.int64), mapping,
                                                    SLOTS)
    got, key_pool, value_pool = attend(torch, meta, base, q, k, v, heads, kv_heads, dim, scale)
    want, _, _ = attend(torch, host_meta, base, q, k, v, heads, kv_heads, dim, scale)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    if rows in (7, 137):
        bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)  # noqa: E731
        pool = np.stack([bits(key_pool.transpose(0, 1)), bits(value_pool.transpose(0, 1))])
        problem = orc.Problem(bits(q), pool, row_requests.numpy(), positions.to(torch.int64).numpy(),
                              mapping.numpy(), heads, kv_heads, dim, scale)
        print(rows, orc.check_tolerance(bits(got), orc.direct_bf16_pv(problem), MAX_ABS, MEAN_ABS), flush=True)
    del keep


@pytest.mark.parametrize("case,code", [("location_high", 1), ("request_high", 2), ("position_high", 1),
                                       ("location_shift", 3), ("missing", 6), ("alias", 7), ("duplicate", 4)])
def test_from_device_rejections(torch_ext, case, code):
    torch = torch_ext
    locations, requests, positions, mapping, prefixes, lengths, _ = smoke_data(torch, 7)
    if case == "location_high":
        locations = locations.clone()
        locations[0] += 1 << 32
    elif case == "request_high":
        requests = requests.clone()
        requests[0] += 1 << 32
    elif case == "position_high":
        positions = positions.clone()
        positions[0] += 1 << 32
    elif case == "location_shift":
        locations = locations.clone()
        locations[0] += 1
    elif case == "missing":
        mapping = mapping.clone()
        mapping[requests[0], 0] = -1
    elif case == "alias":
        mapping = mapping.clone()
        mapping[requests[1], 0] = locations[0]
    elif case == "duplicate":
        requests, positions = torch.tensor([0, 0]), torch.tensor([2, 2])
        locations = mapping[requests, positions].to(torch.int64)
        prefixes, lengths = [2, 2], [1, 1]
    with pytest.raises(RuntimeError, match=f"code {code}"):
        prepare(torch, locations, requests, positions, mapping, prefixes, lengths)


def test_from_device_host_checks(torch_ext):
    torch = torch_ext
    locations, requests, positions, mapping, prefixes, lengths, _ = smoke_data(torch, 7)
    with pytest.raises(RuntimeError, match="sequence lengths"):
        prepare(torch, locations, requests, positions, mapping, prefixes, [lengths[0] + 1] + lengths[1:])
    with pytest.raises(RuntimeError, match="int32 or int64 vectors"):
        prepare(torch, locations.float(), requests, positions, mapping, prefixes, lengths)
    with pytest.raises(RuntimeError, match="int32 request map"):
        torch.classes.gaudirt.PagedMetadata.from_device(locations.cuda(), requests.cuda(), positions.cuda(),
                                                        mapping.long().cuda(), prefixes, lengths, SLOTS)


def test_tokens_validated(torch_ext):
    torch = torch_ext
    locations, requests, positions, mapping, prefixes, lengths, _ = smoke_data(torch, 33)
    tokens = (torch.arange(33, dtype=torch.int64) * 73) % 32000
    args = [locations.cuda(), requests.cuda(), positions.cuda(), mapping.cuda(), prefixes, lengths, SLOTS]
    meta = torch.classes.gaudirt.PagedMetadata.from_device_with_tokens(*args, tokens.cuda(), 32000)
    assert torch.equal(meta.token_ids().cpu(), tokens.to(torch.int32)) and meta.vocabulary() == 32000
    bad = tokens.clone()
    bad[5] = 32000
    with pytest.raises(RuntimeError, match="token ID outside vocabulary at row 5"):
        torch.classes.gaudirt.PagedMetadata.from_device_with_tokens(*args, bad.cuda(), 32000)
    with pytest.raises(RuntimeError, match="token ID inputs or vocabulary"):
        torch.classes.gaudirt.PagedMetadata.from_device_with_tokens(*args, tokens.cuda(), 0)


def scheduler_args(torch, rows, sliced=False):
    locations, requests, positions, mapping, prefixes, lengths, _ = smoke_data(torch, rows)
    inputs = [to_device(torch, t, sliced) for t in (locations, requests, positions)] + [mapping.cuda()]
    tokens = (torch.arange(rows, dtype=torch.int64) * 73) % 32000
    return (*inputs, prefixes, lengths, SLOTS, to_device(torch, tokens, sliced), 32000), tokens


@pytest.mark.parametrize("rows", [1, 7, 33, 137, 1025])
def test_scheduler_metadata_matches_checked(torch_ext, rows):
    torch = torch_ext
    args, tokens = scheduler_args(torch, rows, sliced=rows == 137)
    checked = torch.classes.gaudirt.PagedMetadata.from_device_with_tokens(*args)
    scheduler = torch.classes.gaudirt.PagedMetadata._from_scheduler(*args)
    parts = scheduler.forward_tensors(4, 2, 128)
    for part, name in zip(parts[:6], ("token_ids", "last_token_indices", "rotary_positions", "rotary_header",
                                      "row_locations", "row_requests")):
        assert torch.equal(part.cpu(), getattr(scheduler, name)().cpu()), (rows, name)
    assert parts[6].data_ptr() == scheduler.attention_plan(4, 2, 128).data_ptr()
    assert parts[7] == scheduler.context()
    for name in ("row_locations", "row_requests", "rotary_positions", "last_token_indices", "token_ids"):
        assert torch.equal(getattr(checked, name)().cpu(), getattr(scheduler, name)().cpu()), (rows, name)
    token_view = scheduler.token_ids()
    bucket = 1 << (rows - 1).bit_length()
    padded = token_view.as_strided((bucket,), (1,), token_view.storage_offset()).cpu()
    assert torch.equal(padded[:rows], tokens.int()) and torch.count_nonzero(padded[rows:]) == 0


def test_scheduler_metadata_does_not_wait(torch_ext):
    torch = torch_ext
    args, _ = scheduler_args(torch, 7)
    metadata = torch.classes.gaudirt.PagedMetadata._from_scheduler(*args)
    torch.cuda.synchronize()
    source = torch.empty(64 * 1024**2, dtype=torch.uint8, device="cuda")
    target = torch.empty_like(source)
    for _ in range(256):
        target.copy_(source, non_blocking=True)
    queued = torch.cuda.Event()
    queued.record()
    assert not queued.query(), "device work completed before the asynchronous check"
    following = torch.classes.gaudirt.PagedMetadata._from_scheduler(*args)
    assert not queued.query(), "scheduler metadata waited for earlier device work"
    queued.synchronize()
    assert torch.equal(following.token_ids().cpu(), metadata.token_ids().cpu())


def test_fused_scheduler_metadata(torch_ext):
    torch = torch_ext
    for rows in (1, 3, 17):
        context, slots = 64, 2048
        prefixes = [3 + i for i in range(rows)]
        mapping = torch.zeros((rows, context), dtype=torch.int32)
        for row, prefix in enumerate(prefixes):
            mapping[row, :prefix + 1] = torch.arange(row * context, row * context + prefix + 1)
        locations = torch.tensor([row * context + p for row, p in enumerate(prefixes)], dtype=torch.int64)
        requests = torch.arange(rows, dtype=torch.int64)
        positions = torch.tensor(prefixes, dtype=torch.int64)
        tokens = torch.arange(rows, dtype=torch.int64) + 17
        loc, req, pos, mp, tok = (t.cuda() for t in (locations, requests, positions, mapping, tokens))
        lengths = [1] * rows
        old = torch.classes.gaudirt.PagedMetadata._from_scheduler(loc, req, pos, mp, prefixes, lengths, slots, tok,
                                                                  32000)
        old_plan = old.attention_plan(4, 2, 128)
        fused = torch.classes.gaudirt.PagedMetadata._from_scheduler_fused(loc, req, positions, mp, prefixes, lengths,
                                                                          slots, tok, 32000, 4, 2, 128)
        for name in ("row_locations", "row_requests", "rotary_positions", "rotary_header", "last_token_indices",
                     "token_ids"):
            assert torch.equal(getattr(old, name)().cpu(), getattr(fused, name)().cpu()), (rows, name)
        assert torch.equal(fused.model_positions().cpu(), positions)
        assert torch.equal(old_plan.cpu(), fused.attention_plan(4, 2, 128).cpu())
        with pytest.raises(RuntimeError, match="different head geometry"):
            fused.attention_plan(8, 2, 128)
        with pytest.raises(RuntimeError, match="host position does not match"):
            torch.classes.gaudirt.PagedMetadata._from_scheduler_fused(loc, req, positions + 1, mp, prefixes, lengths,
                                                                      slots, tok, 32000, 4, 2, 128)
    # Plans made on two streams are distinct objects.
    positions = torch.tensor([7], dtype=torch.int64)
    mapping = torch.arange(64, dtype=torch.int32).reshape(1, 64).cuda()
    locations, requests, tokens = (torch.tensor([v], dtype=torch.int64).cuda() for v in (7, 0, 17))
    pending = []
    for stream in (torch.cuda.Stream(), torch.cuda.Stream()):
        with torch.cuda.stream(stream):
            pending.append(torch.classes.gaudirt.PagedMetadata._from_scheduler_fused(
                locations, requests, positions, mapping, [7], [1], 2048, tokens, 32000, 4, 2, 128))
    assert pending[0].attention_plan(4, 2, 128).data_ptr() != pending[1].attention_plan(4, 2, 128).data_ptr()
    torch.cuda.synchronize()
    for metadata in pending:
        assert torch.equal(metadata.model_positions().cpu(), positions)


@pytest.mark.parametrize("page", [4, 16, 32, 128])
def test_page_aligned_device_metadata(torch_ext, page):
    """Device-detected pages: block tables built on the device, prefill runs
    whose requests are gathered on the device; output equal to the host
    constructor's, and to the oracle. The scheduler-owned variant of the same
    inputs (token-granular map) agrees within tolerance."""
    torch = torch_ext
    import gaudirt_amd

    rng = np.random.default_rng(page)
    heads, kv_heads, dim, requests_n, context = 16, 4, 128, 6, 1024
    slots = 96 * 1024
    scale = float(np.float32(1.0 / math.sqrt(dim)))
    blocks = rng.permutation(slots // page - 1)[: requests_n * context // page] + 1
    mapping = (blocks.reshape(requests_n, -1)[:, :, None] * page + np.arange(page)).reshape(requests_n, context)
    mapping = mapping.astype(np.int32)
    batch_requests = np.array([4, 1, 5, 0], dtype=np.int64)
    prefixes, lengths = [300, 0, 777, 1000], [90, 64, 1, 1]
    for r, p, n in zip(batch_requests, prefixes, lengths):
        mapping[r, p + n:] = -1
    for r in set(range(requests_n)) - set(batch_requests.tolist()):
        mapping[r, :] = -1
    row_req = np.repeat(batch_requests, lengths)
    positions = np.concatenate([np.arange(p, p + n) for p, n in zip(prefixes, lengths)]).astype(np.int64)
    locations = mapping[row_req, positions].astype(np.int64)
    rows = len(locations)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    args = [t(locations).cuda(), t(batch_requests).cuda(), t(positions).cuda(), t(mapping).cuda(), prefixes, lengths,
            slots]
    device_meta = torch.classes.gaudirt.PagedMetadata.from_device(*args)
    host_meta = torch.classes.gaudirt.PagedMetadata(t(locations), t(row_req), t(positions), t(mapping), slots)
    sched_meta = torch.classes.gaudirt.PagedMetadata._from_scheduler(*args, None, 0)
    assert orc.largest_page(orc.page_flags(mapping, batch_requests, prefixes, lengths)) == page
    gen = torch.Generator().manual_seed(page)
    q, k, v = (torch.randn(rows, w, generator=gen).to(torch.bfloat16).cuda()
               for w in (heads * dim, kv_heads * dim, kv_heads * dim))
    base = [torch.randn(slots, kv_heads, dim, generator=gen).to(torch.bfloat16).cuda() for _ in range(2)]
    outs = []
    for meta in (device_meta, host_meta, sched_meta):
        pool = gaudirt_amd.allocate_paged_kv(1, slots, kv_heads, dim)
        key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, 0)
        key_pool.copy_(base[0])
        value_pool.copy_(base[1])
        outs.append(torch.ops.gaudirt.paged_attn.default(q, k, v, key_pool, value_pool, meta, dim, scale))
        torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.equal(device_meta.attention_plan(heads, kv_heads, dim).cpu(),
                       host_meta.attention_plan(heads, kv_heads, dim).cpu())
    bits = lambda x: x.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)  # noqa: E731
    pool = np.stack([bits(key_pool.transpose(0, 1)), bits(value_pool.transpose(0, 1))])
    problem = orc.Problem(bits(q), pool, row_req, positions, mapping, heads, kv_heads, dim, scale)
    ref = orc.direct_bf16_pv(problem)
    for out in (outs[0], outs[2]):
        print(page, orc.check_tolerance(bits(out), ref, MAX_ABS, MEAN_ABS), flush=True)


def _irregular_map(rng, requests_n, context, slots, page, kind):
    """A request map built from `page`-slot blocks, then (kind) left alone,
    broken in the middle of one page of one request (a continuation elsewhere,
    aligned only to page / 2), or with one request's blocks shifted by one slot.
    Every request sees all `context` positions."""
    # Even block indices only, so a block shifted by one slot never meets another request's block.
    blocks = 2 * rng.permutation(slots // page // 2 - 2)[: requests_n * context // page] + 2
    mapping = (blocks.reshape(requests_n, -1)[:, :, None] * page + np.arange(page)).reshape(requests_n, context)
    r = int(rng.integers(requests_n))
    if kind == "split" and page >= 2:
        k = int(rng.integers(context // page))
        t0 = k * page + page // 2
        fresh = (slots // page - 1) * page  # the last page's slots, unused by the blocks above
        mapping[r, t0:(k + 1) * page] = fresh + np.arange(page - page // 2)
    elif kind == "shift":
        mapping[r] += 1
    return mapping.astype(np.int32)


@pytest.mark.parametrize("page", [1, 2, 8, 64, 256])
@pytest.mark.parametrize("kind", ["aligned", "split", "shift"])
def test_host_page_detection_matches_device(torch_ext, page, kind):
    """The host constructor finds a map's page size from its breaks in one
    pass; the checked device constructor finds it from per-page flags (pinned
    by the oracle). On aligned, mid-page-broken and shifted maps both must pick
    the same page: their plans (block tables included) and outputs are equal bit
    for bit."""
    torch = torch_ext
    import gaudirt_amd

    rng = np.random.default_rng(page * 7 + len(kind))
    heads, kv_heads, dim, requests_n, context = 16, 4, 128, 5, 512
    slots = 64 * 1024
    scale = float(np.float32(1.0 / math.sqrt(dim)))
    mapping = _irregular_map(rng, requests_n, context, slots, page, kind)
    batch_requests = np.arange(requests_n, dtype=np.int64)
    prefixes, lengths = [context - 1] * requests_n, [1] * requests_n
    expected = orc.largest_page(orc.page_flags(mapping, batch_requests, prefixes, lengths))
    if kind == "aligned":
        assert expected == min(page, 1024)
    if kind == "split" and page >= 4:
        assert expected == page // 2
    if kind == "shift":
        assert expected == 1
    positions = np.array(prefixes, dtype=np.int64)
    locations = mapping[batch_requests, positions].astype(np.int64)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    device_meta = torch.classes.gaudirt.PagedMetadata.from_device(
        t(locations).cuda(), t(batch_requests).cuda(), t(positions).cuda(), t(mapping).cuda(), prefixes, lengths,
        slots)
    host_meta = torch.classes.gaudirt.PagedMetadata(t(locations), t(batch_requests), t(positions), t(mapping), slots)
    assert torch.equal(device_meta.attention_plan(heads, kv_heads, dim).cpu(),
                       host_meta.attention_plan(heads, kv_heads, dim).cpu()), (page, kind, expected)
    gen = torch.Generator().manual_seed(page)
    q, k, v = (torch.randn(requests_n, w, generator=gen).to(torch.bfloat16).cuda()
               for w in (heads * dim, kv_heads * dim, kv_heads * dim))
    outs = []
    for meta in (device_meta, host_meta):
        pool = gaudirt_amd.allocate_paged_kv(1, slots, kv_heads, dim)
        key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, 0)
        key_pool.copy_(torch.ones(slots, kv_heads, dim, dtype=torch.bfloat16, device="cuda"))
        value_pool.copy_(torch.arange(slots, device="cuda").to(torch.bfloat16)[:, None, None].expand(slots, kv_heads,
                                                                                                     dim))
        outs.append(torch.ops.gaudirt.paged_attn.default(q, k, v, key_pool, value_pool, meta, dim, scale))
        torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), (page, kind)
    assert torch.isfinite(outs[0].float()).all()


# ---------------------------------------------------------------------------
# _C._allocate_paged_slots / _C._release_paged_slots
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("page", [16, 64])
def test_slot_allocator_reference_smoke(torch_ext, page):
    torch = torch_ext
    import gaudirt_amd

    ext = gaudirt_amd.load_extension()
    prefixes, lengths = [0, 7, page, 2 * page - 1], [19, 14, 20, 66]
    previous = [-1, 81 * page + 6, 82 * page + page - 1, 83 * page + page - 2]
    pages = [13, 7, 23, 41, 12, 33, 55, 61, 15, 18, 19, 20, 21, 22, 24, 25]
    slots, used = ext._allocate_paged_slots(torch.tensor(previous).cuda(), torch.tensor(pages).cuda(), prefixes,
                                            lengths, page)
    want, want_used = orc.allocate_paged_slots(previous, pages, prefixes, lengths, page)
    assert used == want_used and slots.cpu().tolist() == want and slots.dtype == torch.int64
    released = [13 * page + 7, 7 * page, 13 * page, 23 * page + page - 1, 7 * page + 3]
    assert ext._release_paged_slots(torch.tensor(released).cuda(), page, 512).cpu().tolist() == [13, 7, 23]
    for invalid in (0, 513 * page, 1 << 40):
        with pytest.raises(RuntimeError, match="outside the KV pool"):
            ext._release_paged_slots(torch.tensor([invalid]).cuda(), page, 512)


@pytest.mark.parametrize("page", [1, 8, 16, 32, 64, 128])
def test_slot_allocator_generalized(torch_ext, page):
    torch = torch_ext
    import gaudirt_amd

    ext = gaudirt_amd.load_extension()
    prefixes, lengths = [0, 3, page], [5, 7, page + 2]
    prev = [-1, 100 * page + (2 % page), 200 * page + (page - 1)]
    pages = list(range(10, 80))
    slots, used = ext._allocate_paged_slots(torch.tensor(prev).cuda(), torch.tensor(pages).cuda(), prefixes, lengths,
                                            page)
    want, want_used = orc.allocate_paged_slots(prev, pages, prefixes, lengths, page)
    assert used == want_used and slots.cpu().tolist() == want
    released = [9000 * page, 9000 * page + (page - 1), 12000 * page]
    assert ext._release_paged_slots(torch.tensor(released).cuda(), page, 16384).cpu().tolist() == [9000, 12000]
    assert ext._release_paged_slots(torch.tensor([16384 * page]).cuda(), page, 16384).cpu().tolist() == [16384]


def test_slot_allocator_random_against_oracle(torch_ext):
    torch = torch_ext
    import gaudirt_amd

    ext = gaudirt_amd.load_extension()
    rng = np.random.default_rng(77)
    for page in (2, 16, 128, 256):
        batch = 300
        prefixes = [int(x) for x in rng.integers(0, 4 * page, batch)]
        lengths = [int(x) for x in rng.integers(0, 3 * page, batch)]
        lengths[0] = max(lengths[0], 1)
        last = [int(x) for x in rng.integers(page, 100000 * page, batch)]  # pages 1 .. 100000
        free = [int(x) for x in rng.permutation(200000)[:100000] + 1]
        slots, used = ext._allocate_paged_slots(torch.tensor(last).cuda(), torch.tensor(free).cuda(), prefixes,
                                                lengths, page)
        want, want_used = orc.allocate_paged_slots(last, free, prefixes, lengths, page)
        assert used == want_used and slots.cpu().tolist() == want, page
        release = np.concatenate([np.array(want), rng.integers(page, 200000 * page, 5000)])
        rng.shuffle(release)
        got = ext._release_paged_slots(torch.from_numpy(release).cuda(), page, 200000)
        assert got.cpu().tolist() == orc.release_paged_slots(release, page, 200000), page
    with pytest.raises(RuntimeError, match="insufficient free pages"):
        ext._allocate_paged_slots(torch.tensor([-1]).cuda(), torch.tensor([5]).cuda(), [0], [33], 16)
    with pytest.raises(RuntimeError, match="invalid request lengths"):
        ext._allocate_paged_slots(torch.tensor([-1]).cuda(), torch.tensor([5]).cuda(), [-1], [3], 16)


def test_metadata_of_every_constructor_on_two_streams(torch_ext):
    """tests/paged_metadata_event_reuse_smoke.py and
    tests/paged_staging_event_lifetime_smoke.py of the reference: metadata from
    the host constructor, _from_scheduler, from_device_with_tokens and
    _from_scheduler_fused, built on two streams in turn for 24 rounds and all
    kept alive, then released in reverse order and built again. Every object
    keeps its own rows, positions and tokens, and attention through it on its
    stream is bit-identical across constructors and within the gate of the
    oracle. (The reference also counts its runtime's events; here the torch
    caching allocators own device and pinned staging memory.)"""
    import gaudirt_amd

    torch = torch_ext
    mapping = torch.arange(1, 129, dtype=torch.int32).reshape(2, 64)
    d_mapping = mapping.cuda()
    slots, heads, kv_heads, dim = 129, 4, 2, 128
    scale = float(np.float32(1.0 / math.sqrt(dim)))
    gen = torch.Generator().manual_seed(4404)
    pool = gaudirt_amd.allocate_paged_kv(1, slots, kv_heads, dim)
    key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, 0)
    key_pool.copy_(torch.randn(slots, kv_heads, dim, generator=gen).to(torch.bfloat16))
    value_pool.copy_(torch.randn(slots, kv_heads, dim, generator=gen).to(torch.bfloat16))
    cases = []
    for request, prefix in ((0, 5), (1, 12)):
        positions = torch.arange(prefix, prefix + 3, dtype=torch.int64)
        requests = torch.full((3,), request, dtype=torch.int64)
        locations = mapping[requests, positions].long()
        tokens = torch.tensor([11, 12, 13], dtype=torch.int64) + 100 * request
        query = torch.randn(3, heads * dim, generator=gen).to(torch.bfloat16)
        cases.append(dict(request=request, prefix=prefix, positions=positions, requests=requests,
                          locations=locations, tokens=tokens, query=query.cuda(),
                          device=[t.cuda() for t in (locations, torch.tensor([request]), positions, tokens)]))

    def construct(case, mode):
        loc, breq, pos, tok = case["device"]
        if mode == "host":
            return torch.classes.gaudirt.PagedMetadata(case["locations"], case["requests"], case["positions"],
                                                       mapping, slots)
        if mode == "scheduler":
            return torch.classes.gaudirt.PagedMetadata._from_scheduler(loc, breq, pos, d_mapping, [case["prefix"]],
                                                                       [3], slots, tok, 32000)
        if mode == "checked":
            return torch.classes.gaudirt.PagedMetadata.from_device_with_tokens(
                loc, breq, pos, d_mapping, [case["prefix"]], [3], slots, tok, 32000)
        return torch.classes.gaudirt.PagedMetadata._from_scheduler_fused(
            loc, breq, case["positions"], d_mapping, [case["prefix"]], [3], slots, tok, 32000, heads, kv_heads, dim)

    modes = ("host", "scheduler", "checked", "fused")
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    # The attention step stores each row's own K/V (the pool's values at its
    # slots), so every step leaves the pool as it was.
    kv = [(key_pool[c["locations"].cuda()].reshape(3, -1).clone(),
           value_pool[c["locations"].cuda()].reshape(3, -1).clone()) for c in cases]
    torch.cuda.synchronize()

    def build(rounds):
        pending = []
        for it in range(rounds):
            index = it % 2
            with torch.cuda.stream(streams[index]):
                for mode in modes:
                    meta = construct(cases[index], mode)
                    out = torch.ops.gaudirt.paged_attn.default(cases[index]["query"], kv[index][0], kv[index][1],
                                                               key_pool, value_pool, meta, dim, scale)
                    pending.append((index, mode, meta, out))
        return pending

    def verify(pending):
        torch.cuda.synchronize()
        first = {}
        for index, mode, meta, out in pending:
            case = cases[index]
            assert meta.row_locations().cpu().tolist() == case["locations"].tolist(), (index, mode)
            assert meta.rotary_positions().cpu().tolist() == case["positions"].tolist(), (index, mode)
            if mode != "host":  # device constructors only (batched metadata)
                assert meta.last_token_indices().cpu().tolist() == [2], (index, mode)
                assert meta.token_ids().cpu().tolist() == case["tokens"].tolist(), (index, mode)
            got = bits(out)
            if index not in first:
                first[index] = got
                problem = orc.Problem(bits(case["query"]), np.stack([bits(key_pool.transpose(0, 1)),
                                                                     bits(value_pool.transpose(0, 1))]),
                                      case["requests"].numpy(), case["positions"].numpy(), mapping.numpy(),
                                      heads, kv_heads, dim, scale)
                orc.check_flat_gate(got, orc.direct_bf16_pv(problem))
            assert np.array_equal(got, first[index]), (index, mode)

    def bits(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    pending = build(24)
    verify(pending)
    while pending:
        pending.pop()
    pending = build(16)
    verify(pending)


@pytest.mark.parametrize("slots,context,requests_n", [(7, 6, 1), (129, 64, 2), (1 << 20, 4096, 64)])
def test_scheduler_metadata_at_any_capacity(torch_ext, slots, context, requests_n):
    """tests/scheduler_metadata_capacity_cache_smoke.py of the reference:
    scheduler metadata over a mostly-zero request map of any slot, context and
    request capacity keeps the caller's device map itself (no copy), reports
    its rows, tokens and last-token index, and takes locations at the top of
    the slot range through the same map updated in place. (The reference also
    checks that its compiled recipe does not depend on the capacities.)"""
    torch = torch_ext
    mapping = torch.zeros((requests_n, context), dtype=torch.int32)
    mapping[0, :6] = torch.arange(1, 7, dtype=torch.int32)
    locations = torch.tensor([4, 5, 6], dtype=torch.int64)
    request = torch.tensor([0], dtype=torch.int64)
    positions = torch.tensor([3, 4, 5], dtype=torch.int64)
    tokens = torch.tensor([21, 22, 23], dtype=torch.int64)
    mapping_device = mapping.cuda()
    device = [value.cuda() for value in (locations, request, positions, tokens)]
    metadata = torch.classes.gaudirt.PagedMetadata._from_scheduler(
        device[0], device[1], device[2], mapping_device, [3], [3], slots, device[3], 32000)
    actual = [metadata.row_locations().cpu(), metadata.row_requests().cpu(), metadata.rotary_positions().cpu(),
              metadata.token_ids().cpu(), metadata.last_token_indices().cpu()]
    expected = [locations.int(), torch.zeros(3, dtype=torch.int32), positions.int(), tokens.int(),
                torch.tensor([2], dtype=torch.int32)]
    assert all(torch.equal(a, b) for a, b in zip(actual, expected))
    assert metadata.slots() == slots and metadata.context() == context
    assert metadata.request_mapping().data_ptr() == mapping_device.data_ptr()
    high_locations = torch.arange(slots - 3, slots, dtype=torch.int64)
    mapping_device[0, 3:6].copy_(high_locations.int())
    high = torch.classes.gaudirt.PagedMetadata._from_scheduler(
        high_locations.cuda(), device[1], device[2], mapping_device, [3], [3], slots, device[3], 32000)
    assert torch.equal(high.row_locations().cpu(), high_locations.int())
    # and attention through it reads the top slots (store, then decode rows 3..5 over keys 0..5)
    import gaudirt_amd

    heads, kv_heads, dim = 4, 2, 64
    gen = torch.Generator().manual_seed(slots % 1000)
    pool = gaudirt_amd.allocate_paged_kv(1, slots, kv_heads, dim)
    key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, 0)
    key_pool.copy_(torch.randn(slots, kv_heads, dim, generator=gen).to(torch.bfloat16))
    value_pool.copy_(torch.randn(slots, kv_heads, dim, generator=gen).to(torch.bfloat16))
    q = torch.randn(3, heads * dim, generator=gen).to(torch.bfloat16)
    k = torch.randn(3, kv_heads * dim, generator=gen).to(torch.bfloat16)
    v = torch.randn(3, kv_heads * dim, generator=gen).to(torch.bfloat16)
    scale = float(np.float32(1.0 / math.sqrt(dim)))
    out = torch.ops.gaudirt.paged_attn.default(q.cuda(), k.cuda(), v.cuda(), key_pool, value_pool, high, dim, scale)
    torch.cuda.synchronize()
    bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)  # noqa: E731
    pool_bits = np.stack([bits(key_pool.transpose(0, 1)), bits(value_pool.transpose(0, 1))])
    assert np.array_equal(pool_bits[0][:, slots - 3:], bits(k.reshape(3, kv_heads, dim).transpose(0, 1)))
    problem = orc.Problem(bits(q), pool_bits, np.zeros(3, dtype=np.int64), positions.numpy(),
                          mapping_device.cpu().numpy(), heads, kv_heads, dim, scale)
    orc.check_flat_gate(bits(out), orc.direct_bf16_pv(problem))
