"""CPU checks of the torch boundary: exact schemas, PagedMetadata validation
messages (raised before any device work), fake kernels, and the KV-tile query.

Message fragments follow the reference's host constructor
(src/bridge/paged_metadata.cpp:82-140) and the tests that match them
(tests/paged_metadata_smoke.py:38-54 of the reference).
"""

import numpy as np
import pytest
import torch

import gaudirt_amd

SCHEMAS = {
    "paged_attn": "gaudirt::paged_attn(Tensor query, Tensor key, Tensor value, Tensor(a!) key_pool, "
                  "Tensor(b!) value_pool, __torch__.torch.classes.gaudirt.PagedMetadata metadata, int head_dim, "
                  "float scale, float softcap=0.0, int sliding_window=-1) -> Tensor",
    "_paged_attn_validated": "gaudirt::_paged_attn_validated(Tensor query, Tensor key, Tensor value, "
                             "Tensor(a!) key_pool, Tensor(b!) value_pool, Tensor locations, Tensor requests, "
                             "Tensor positions, Tensor mapping, Tensor header, int head_dim, float scale, "
                             "float softcap=0.0, int sliding_window=-1) -> Tensor",
    "_advance_decode_lengths": "gaudirt::_advance_decode_lengths(Tensor seq_lens, Tensor orig_seq_lens) "
                               "-> (Tensor, Tensor)",
    # src/bridge/generic_private_use1.cpp:464-470
    "rotary_embedding": "gaudirt::rotary_embedding(Tensor query, Tensor key, Tensor cache, "
                        "__torch__.torch.classes.gaudirt.PagedMetadata metadata, int head_dim, int rotary_dim, "
                        "bool is_neox) -> (Tensor, Tensor)",
    "rotary_embedding_positions": "gaudirt::rotary_embedding_positions(Tensor query, Tensor key, Tensor cache, "
                                  "Tensor positions, int head_dim, int rotary_dim, bool is_neox) "
                                  "-> (Tensor, Tensor)",
    "_rotary_embedding_validated": "gaudirt::_rotary_embedding_validated(Tensor query, Tensor key, Tensor cache, "
                                   "Tensor positions, Tensor header, int context, int head_dim, int rotary_dim, "
                                   "bool is_neox) -> (Tensor, Tensor)",
}


@pytest.fixture(scope="module", autouse=True)
def ext():
    return gaudirt_amd.load_extension()


@pytest.mark.parametrize("name", sorted(SCHEMAS))
def test_schema_strings(name):
    # Registered from the reference's exact strings; compared after parsing, as
    # torch prints defaults in its own normal form (0.0 -> 0.).
    assert getattr(torch.ops.gaudirt, name).default._schema == torch._C.parse_schema(SCHEMAS[name])


def test_paged_metadata_methods_exist():
    # TorchScript resolves every method of the class with its signature; a
    # missing or mistyped method fails compilation.
    @torch.jit.script
    def uses_all(m: torch.classes.gaudirt.PagedMetadata, w: int):
        sizes = m.rows() + m.slots() + m.context() + m.vocabulary()
        rows = (m.rotary_positions(), m.rotary_header(), m.row_locations(), m.row_requests(),
                m.request_mapping(), m.model_positions(), m.last_token_indices(), m.token_ids())
        plans = (m.attention_plan(32, 8, 128), m.attention_plan_for(32, 8, 128, w))
        return sizes, rows, plans, m.forward_tensors(32, 8, 128)

    assert uses_all is not None


def _meta(locations, requests, positions, mapping, slots):
    return torch.classes.gaudirt.PagedMetadata(locations, requests, positions, mapping, slots)


def _base():
    mapping = torch.arange(16, dtype=torch.int32).reshape(2, 8)
    requests = torch.tensor([0, 1], dtype=torch.int64)
    positions = torch.tensor([2, 3], dtype=torch.int64)
    locations = mapping[requests, positions].to(torch.int64)
    return locations, requests, positions, mapping


@pytest.mark.parametrize("case,fragment", [
    ("float", "contiguous CPU int32 or int64"),
    ("rank", "invalid paged metadata ranks"),
    ("rows", "dimensions outside supported range"),
    ("map_range", "request-to-token slot is out of range"),
    ("index", "index is out of range"),
    ("mismatch", "does not match"),
    ("duplicate", "duplicate output KV slot"),
    ("missing", "missing KV slot"),
    ("alias", "aliases another visible prefix"),
])
def test_metadata_rejections(case, fragment):
    locations, requests, positions, mapping = _base()
    slots = 16
    if case == "float":
        locations = locations.float()
    elif case == "rank":
        requests = requests[:1]
    elif case == "rows":
        locations = torch.zeros(8193, dtype=torch.int64)
        requests = torch.zeros(8193, dtype=torch.int64)
        positions = torch.zeros(8193, dtype=torch.int64)
    elif case == "map_range":
        mapping = mapping.clone()
        mapping[0, 7] = 16
    elif case == "index":
        positions = positions.clone()
        positions[1] = 8
    elif case == "mismatch":
        locations = locations.clone()
        locations[0] = 5
    elif case == "duplicate":
        mapping = mapping.clone()
        mapping[1, 3] = int(mapping[0, 2])
        locations = torch.tensor([2, 2], dtype=torch.int64)
    elif case == "missing":
        mapping = mapping.clone()
        mapping[0, 1] = -1
    elif case == "alias":
        # request 1's visible prefix contains the slot request 0 is writing
        mapping = mapping.clone()
        mapping[1, 0] = int(mapping[0, 2])
    with pytest.raises(RuntimeError, match=fragment):
        _meta(locations, requests, positions, mapping, slots)


def _host_outcome(locations, requests, positions, mapping, slots):
    """None when the host constructor's validation passes (it then goes on to
    the device, which this container does not have), else the error text."""
    try:
        torch.classes.gaudirt.PagedMetadata(locations, requests, positions, mapping, slots)
    except RuntimeError as error:
        text = str(error)
        return None if "no current HIP device" in text else text
    return None


def _paged_problem(rng, page):
    requests_n = int(rng.integers(1, 7))
    context = int(rng.integers(16, 300))
    pages = -(-context // page)
    blocks = rng.permutation(requests_n * pages + 8)[: requests_n * pages].reshape(requests_n, pages)
    slots = (requests_n * pages + 8) * page
    t = np.arange(context)
    visible = rng.integers(1, context + 1, requests_n)
    mapping = np.where(t[None, :] < visible[:, None], blocks[:, t // page] * page + t % page, -1)
    chosen = rng.permutation(requests_n)[: int(rng.integers(1, requests_n + 1))]
    rows = []
    for request in chosen:
        length = int(rng.integers(1, min(6, int(visible[request])) + 1))
        first = int(rng.integers(0, int(visible[request]) - length + 1))
        rows += [(int(request), first + k) for k in range(length)]
    order = rng.permutation(len(rows))
    requests = np.array([rows[i][0] for i in order], dtype=np.int64)
    positions = np.array([rows[i][1] for i in order], dtype=np.int64)
    locations = mapping[requests, positions].astype(np.int64)
    return locations, requests, positions, mapping.astype(np.int32), slots


def _plant(rng, kind, problem):
    locations, requests, positions, mapping, slots = problem
    locations, requests, positions, mapping = locations.copy(), requests.copy(), positions.copy(), mapping.copy()
    last = {int(r): int(positions[requests == r].max()) for r in np.unique(requests)}
    i = int(rng.integers(0, len(locations)))
    victim = int(rng.choice(list(last)))
    if kind == "missing":
        mapping[victim, int(rng.integers(0, last[victim] + 1))] = -1
    elif kind == "alias":  # a written slot anywhere in some visible prefix
        mapping[victim, int(rng.integers(0, last[victim] + 1))] = locations[i]
    elif kind == "alias_run":  # a whole page holding a written slot, inside a run
        page = int(rng.choice([4, 8, 16]))
        start = int(rng.integers(0, last[victim] + 1)) // page * page
        block = int(locations[i]) // page * page
        end = min(start + page, mapping.shape[1])
        mapping[victim, start:end] = block + np.arange(end - start)
    elif kind == "map_range":
        mapping[int(rng.integers(0, mapping.shape[0])), int(rng.integers(0, mapping.shape[1]))] = \
            [slots, -2, slots + 7][int(rng.integers(0, 3))]
    elif kind == "mismatch":
        locations[i] = (locations[i] + 1) % slots
    elif kind == "duplicate":
        j = int(rng.integers(0, len(locations)))
        locations, requests, positions = (np.append(a, a[j]) for a in (locations, requests, positions))
    elif kind == "index":
        positions[i] = mapping.shape[1]
    return locations, requests, positions, mapping, slots


def test_host_constructor_matches_oracle():
    """The host constructor reports what the reference's constructor would
    (oracle.host_metadata_error: same failure, same order) on random paged and
    token-granular maps, with one or two planted faults: missing and aliased
    prefix slots (also inside a run of consecutive slots), out-of-range map
    entries, rows off the map, repeated rows and out-of-range indices."""
    from oracle import oracle as orc

    rng = np.random.default_rng(2024)
    kinds = ["none", "missing", "alias", "alias_run", "map_range", "mismatch", "duplicate", "index"]
    seen = set()
    for trial in range(480):
        page = [1, 4, 8, 16, 64][trial % 5]
        problem = _paged_problem(rng, page)
        planted = [kinds[(trial // 5) % len(kinds)]]
        if trial % 3 == 0:
            planted.append(kinds[int(rng.integers(1, len(kinds)))])
        for kind in planted:
            if kind != "none":
                problem = _plant(rng, kind, problem)
        locations, requests, positions, mapping, slots = problem
        want = orc.host_metadata_error(locations, requests, positions, mapping, slots)
        as_tensor = lambda a, dtype: torch.from_numpy(np.ascontiguousarray(a.astype(dtype)))  # noqa: E731
        map_dtype = np.int64 if trial % 4 == 1 else np.int32
        got = _host_outcome(as_tensor(locations, np.int64), as_tensor(requests, np.int64),
                            as_tensor(positions, np.int32 if trial % 2 else np.int64), as_tensor(mapping, map_dtype),
                            slots)
        if want is None:
            assert got is None, (trial, planted, got)
        else:
            assert got is not None and want in got, (trial, planted, want, got)
        seen.add(want)
    assert len(seen) == 7, seen


def test_fake_kernels_on_meta_tensors():
    q = torch.empty(5, 8 * 64, device="meta", dtype=torch.bfloat16)
    k = torch.empty(5, 2 * 64, device="meta", dtype=torch.bfloat16)
    pool = torch.empty(32, 2, 64, device="meta", dtype=torch.bfloat16)
    idx = torch.empty(5, device="meta", dtype=torch.int32)
    out = torch.ops.gaudirt._paged_attn_validated(q, k, k, pool, pool, idx, idx, idx, idx, idx, 64, 0.125)
    assert out.shape == q.shape and out.device.type == "meta"
    seq = torch.empty(7, device="meta", dtype=torch.int64)
    orig = torch.empty(7, device="meta", dtype=torch.int32)
    a, b = torch.ops.gaudirt._advance_decode_lengths(seq, orig)
    assert a.shape == seq.shape and b.dtype == torch.int32


def test_kv_tile_and_version(ext):
    assert gaudirt_amd.paged_attn_kv_tile(1) == 512
    assert ext.version().startswith("gaudirt_amd")


def test_device_constructors_have_the_reference_signatures():
    # TorchScript compiles the calls against the registered schemas, with the
    # argument lists the reference's tests use
    # (tests/paged_device_metadata_smoke.py:59-61, tests/scheduler_metadata_async_smoke.py:30-31,
    # tests/scheduler_metadata_fused_smoke.py:36-46).
    @torch.jit.script
    def construct(l: torch.Tensor, r: torch.Tensor, p: torch.Tensor, m: torch.Tensor, t: torch.Tensor):
        a = torch.classes.gaudirt.PagedMetadata.from_device(l, r, p, m, [2], [1], 16)
        b = torch.classes.gaudirt.PagedMetadata.from_device_with_tokens(l, r, p, m, [2], [1], 16, t, 32000)
        c = torch.classes.gaudirt.PagedMetadata._from_scheduler(l, r, p, m, [2], [1], 16, None, 0)
        d = torch.classes.gaudirt.PagedMetadata._from_scheduler_fused(l, r, p, m, [2], [1], 16, t, 32000, 4, 2, 128)
        return a, b, c, d

    assert construct is not None


def test_device_constructors_reject_host_tensors():
    # Host tensors (or a box without a GPU) are refused before any device work.
    locations, requests, positions, mapping = _base()
    with pytest.raises(RuntimeError, match="GaudiRT"):
        torch.classes.gaudirt.PagedMetadata.from_device(locations, requests, positions, mapping, [2, 3], [1, 1], 16)


def test_slot_allocator_rejects_host_tensors(ext):
    last = torch.tensor([-1], dtype=torch.int64)
    with pytest.raises(RuntimeError, match="GaudiRT"):
        ext._allocate_paged_slots(last, torch.arange(4), [0], [3], 16)
    with pytest.raises(RuntimeError, match="GaudiRT"):
        ext._release_paged_slots(last, 16, 512)


def test_rotary_fake_kernels_trace():
    # torch.compile traces the rotary ops (and the fused attention) through the
    # registered fake kernels; no device work happens under FakeTensorMode.
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(5, 4 * 128, dtype=torch.bfloat16)
        k = torch.empty(5, 2 * 128, dtype=torch.bfloat16)
        cache = torch.empty(64, 128, dtype=torch.bfloat16)
        pos = torch.empty(5, dtype=torch.int32)
        qo, ko = torch.ops.gaudirt.rotary_embedding_positions(q, k, cache, pos, 128, 128, True)
        assert qo.shape == q.shape and ko.shape == k.shape and qo.dtype == torch.bfloat16
        qo, ko = torch.ops.gaudirt._rotary_embedding_validated(q, k, cache, pos, torch.empty(1, dtype=torch.int32),
                                                               64, 128, 128, False)
        assert qo.shape == q.shape and ko.shape == k.shape


def test_rotary_paged_attn_schema():
    # The fused op (no reference counterpart) takes paged_attn's arguments plus the rotary ones.
    schema = str(torch.ops.gaudirt.rotary_paged_attn.default._schema)
    assert "Tensor(a!) key_pool" in schema and "Tensor cache" in schema and "int rotary_dim" in schema
