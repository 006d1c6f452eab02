"""CPU oracle for the paged-attention path — TEST INFRASTRUCTURE ONLY.

Python side of the plain-C restatement in ``oracle.c`` (loaded through ctypes)
plus the two pieces of reference host logic the checks need: the tiling policy
that decides which reference numerics a row gets, and the reference's error
gate. Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this module, and only as the checker.

Parity status (how each oracle function is pinned; see tests/test_oracle.py):

- ``bf16_from_f32``: torch's CPU ``.to(torch.bfloat16)`` (an independent RNE
  implementation) on random, tie, NaN and overflow inputs.
Vectors of the reference's own CPU references (tests/golden/reference_vectors.npz,
written by tests/golden/make_reference_vectors.py from tests/paged_attention_reference.py,
tests/paged_attention_reference_test.py and tests/fp64_reference.py; checked by
tests/test_golden.py) pin ``direct_bf16_pv``, ``tiled_bf16_pv``, ``direct_tiled`` and
``bf16_from_f64`` bit for bit on the reference test's inputs, the C1 case and 2,224
roundings; on d 64 chunked-prefill cases (a 300-token prefix; the reference's 3840 + 263
multi-tile shape) a few outputs differ where torch's fp32 exp or summation order rounds a
probability or a sum differently (max abs 9.8e-4, mean abs at most 6e-7).

- ``bf16_from_f64``: the known answer of tests/decoder_cpu_reference_test.py:66-68
  (1 + 2^-8 + 2^-32 -> 1 + 2^-7), exact rational rounding with ``fractions`` on
  random normals, subnormals and ties, the overflow boundary, and rejection of
  non-finite input.
- ``kv_store``: brute-force per-slot audit (every targeted slot holds its row,
  every other byte keeps its sentinel, rows >= valid_rows are never written),
  as in tests/fixed_kv_descriptor_device_test.cpp:146-197.
- ``tile_indices``: the expected index table of tests/attention_plan_smoke.py:32-40.
- ``direct_bf16_pv`` / ``tiled_bf16_pv`` / ``direct_tiled``: the invariant of
  tests/paged_attention_reference_test.py:48-50 on the reference test's own
  seeded inputs (torch.manual_seed(771)), closed forms (one key -> the value row;
  equal scores -> the mean), the fp64 gate, and single-tile reduction
  (tiled with one tile == direct up to one bf16 ulp).
- ``fp64_attention``: closed forms and a brute-force numpy float64 softmax.
- ``guid_attention``: closed forms, the fp64 gate, and the single-tile path
  agreeing with direct_bf16_pv.
- ``isolated_errors``: the known answers of
  tests/paged_attention_reference_test.py:52-59.
- ``check_tolerance`` / ``bf16_ulp``: known answers (one ulp allowed only where
  it exceeds 2e-2) and the seeded case where the fp64 answer itself is one ulp
  from direct_bf16_pv. ``check_flat_gate``: known answers (2e-2 passes, the
  next bf16 step above it fails, also where one ulp exceeds 2e-2; NaN fails;
  the mean bound).
- ``metadata_codes``: the rejection cases of
  tests/paged_device_metadata_smoke.py:109-125 (codes 1, 2, 1, 3, 6, 7, 4 on the
  reference test's own data), acceptance of every valid layout the smoke test
  builds, and agreement of "all codes zero" with a set-based brute force of the
  host constructor's accept/reject decision on random corruptions. Code 5
  (position != prefix + offset) has no reference test vector: parity unpinned
  beyond the brute force.
- ``host_metadata_error``: the host constructor cases of the reference's
  tests/paged_metadata_smoke.py:33-50 on that test's data, the precedence its
  loops impose (map range, then rows, then prefixes by request and position),
  and agreement with ``metadata_codes`` on random sequence layouts
  (tests/test_oracle_metadata.py).
- ``page_flags`` / ``largest_page``: closed forms (identity map -> 1024, a map
  shifted by one slot -> 1, permuted pages of P -> P) and brute force over
  random block tables.
- ``rotary_bf16``: closed forms (cos 1 / sin 0 is the identity, a quarter turn
  maps (a, b) to (-b, a), a half turn negates), a brute force over tiny inputs
  with Python complex products (exact in binary64, so rounding once to fp32 and
  once to bf16 gives the fp32 reference's bits) for both pair layouts, and the
  relative-L2 gate of tests/rotary_runtime_smoke.py:51-60 against the fp64
  form on the reference test's shapes. ``rotary_f64`` is the fp64 form
  (tests/rotary_runtime_smoke.py:34-48 with fp64=True).
- ``allocate_paged_slots`` / ``release_paged_slots``: the expected values of
  tests/paged_slots_device_smoke.py (evaluated literally for P = 16 and 64),
  of tests/paged_attention_generalized_smoke.py:146-158 and
  tests/dynamic_eager_ops_smoke.py:383-418, the rejected releases (page 0,
  page max_pages + 1, 2^40), and invariants (slots distinct, slot % P ==
  position % P, pages drawn in free-list order).
"""

import ctypes
import os
import pathlib

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"


def build():
    """Compile liboracle.so with the committed Makefile."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def _load():
    if not _LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(_LIB_PATH))
    lib.orc_bf16_from_f32.restype = ctypes.c_uint16
    lib.orc_bf16_from_f32.argtypes = [ctypes.c_float]
    lib.orc_bf16_to_f32.restype = ctypes.c_float
    lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _ptr(array, ctype):
    return array.ctypes.data_as(ctypes.POINTER(ctype))


class AttentionArgs(ctypes.Structure):
    _fields_ = [
        ("query", ctypes.c_void_p), ("q_stride", ctypes.c_int64),
        ("key_pool", ctypes.c_void_p), ("value_pool", ctypes.c_void_p),
        ("slot_stride", ctypes.c_int64), ("head_stride", ctypes.c_int64),
        ("requests", ctypes.c_void_p), ("positions", ctypes.c_void_p),
        ("mapping", ctypes.c_void_p), ("context", ctypes.c_int64), ("rows", ctypes.c_int64),
        ("heads", ctypes.c_int32), ("kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_float), ("softcap", ctypes.c_float), ("sliding_window", ctypes.c_int32),
        ("threads", ctypes.c_int32),
    ]


# ---------------------------------------------------------------------------
# Scalar conversions
# ---------------------------------------------------------------------------

def bf16_from_f32(values):
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(values.shape, dtype=np.uint16)
    lib().orc_bf16_from_f32_array(_ptr(values, ctypes.c_float), _ptr(out, ctypes.c_uint16),
                                  ctypes.c_int64(values.size))
    return out


def bf16_to_f32(bits):
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def bf16_from_f64(values):
    """Direct binary64 -> bf16 RNE (tests/fp64_reference.py:7-29). Raises on non-finite input."""
    values = np.ascontiguousarray(values, dtype=np.float64)
    out = np.empty(values.shape, dtype=np.uint16)
    status = lib().orc_bf16_from_f64_array(_ptr(values, ctypes.c_double), _ptr(out, ctypes.c_uint16),
                                           ctypes.c_int64(values.size))
    if status != 0:
        raise ValueError("nonfinite FP64 reference")
    return out


# ---------------------------------------------------------------------------
# KV store and indexing
# ---------------------------------------------------------------------------

def kv_store(key, value, locations, valid_rows, pool, slots, kv_heads, head_dim):
    """Head-major KV store into ``pool`` (uint16 [2, Hkv, S, d] or flat), in place.

    ``key``/``value`` are uint16 [rows, Hkv * d] (row stride may exceed the width).
    """
    assert key.dtype == np.uint16 and value.dtype == np.uint16 and pool.dtype == np.uint16
    assert key.strides == value.strides and key.strides[1] == 2
    assert pool.flags["C_CONTIGUOUS"]
    locations = np.ascontiguousarray(locations, dtype=np.int32)
    row_stride = key.strides[0] // 2
    lib().orc_kv_store(ctypes.c_void_p(key.ctypes.data), ctypes.c_void_p(value.ctypes.data),
                       ctypes.c_int64(row_stride), _ptr(locations, ctypes.c_int32),
                       ctypes.c_int32(valid_rows), _ptr(pool, ctypes.c_uint16),
                       ctypes.c_int64(slots), ctypes.c_int32(kv_heads), ctypes.c_int32(head_dim))
    return pool


def tile_indices(mapping, requests, work, context):
    mapping = np.ascontiguousarray(mapping, dtype=np.int32)
    requests = np.ascontiguousarray(requests, dtype=np.int32)
    work = np.ascontiguousarray(work, dtype=np.int32).reshape(-1, 4)
    out = np.empty((work.shape[0], 64), dtype=np.int32)
    lib().orc_tile_indices(_ptr(mapping, ctypes.c_int32), _ptr(requests, ctypes.c_int32),
                           _ptr(work, ctypes.c_int32), ctypes.c_int64(work.shape[0]),
                           ctypes.c_int32(context), _ptr(out, ctypes.c_int32))
    return out


def mapping_from_block_table(block_table, block_size, context):
    block_table = np.ascontiguousarray(block_table, dtype=np.int32)
    requests, max_blocks = block_table.shape
    mapping = np.empty((requests, context), dtype=np.int32)
    lib().orc_mapping_from_block_table(_ptr(block_table, ctypes.c_int32), ctypes.c_int64(requests),
                                       ctypes.c_int64(max_blocks), ctypes.c_int32(block_size),
                                       ctypes.c_int64(context), _ptr(mapping, ctypes.c_int32))
    return mapping


# ---------------------------------------------------------------------------
# Attention references
# ---------------------------------------------------------------------------

class Problem:
    """One paged-attention problem in the reference's row form.

    query: uint16 [rows, heads * d]; pool: uint16 head-major [2, Hkv, S, d];
    requests/positions: int64 [rows]; mapping: int32 [requests, context].
    """

    def __init__(self, query, pool, requests, positions, mapping, heads, kv_heads, head_dim, scale,
                 softcap=0.0, sliding_window=-1):
        self.query = np.ascontiguousarray(query, dtype=np.uint16)
        self.pool = np.ascontiguousarray(pool, dtype=np.uint16)
        self.requests = np.ascontiguousarray(requests, dtype=np.int64)
        self.positions = np.ascontiguousarray(positions, dtype=np.int64)
        self.mapping = np.ascontiguousarray(mapping, dtype=np.int32)
        self.heads, self.kv_heads, self.head_dim = int(heads), int(kv_heads), int(head_dim)
        self.scale = float(np.float32(scale))
        self.softcap = float(softcap)
        self.sliding_window = int(sliding_window)
        self.slots = self.pool.size // (2 * self.kv_heads * self.head_dim)
        assert self.query.shape[1] >= self.heads * self.head_dim

    def args(self, threads):
        half = self.kv_heads * self.slots * self.head_dim
        base = self.pool.ctypes.data
        return AttentionArgs(
            self.query.ctypes.data, self.query.shape[1], base, base + 2 * half,
            self.head_dim, self.slots * self.head_dim,
            self.requests.ctypes.data, self.positions.ctypes.data, self.mapping.ctypes.data,
            self.mapping.shape[1], self.query.shape[0], self.heads, self.kv_heads, self.head_dim,
            self.scale, self.softcap, self.sliding_window, threads)

    def _out16(self):
        return np.zeros((self.query.shape[0], self.heads * self.head_dim), dtype=np.uint16)


def host_threads():
    """Threads for the attention references: every CPU this process may run on
    (its affinity mask), bounded by OMP_NUM_THREADS when the host sets it to
    the process's CPU share."""
    try:
        cpus = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        cpus = os.cpu_count() or 1
    limit = os.environ.get("OMP_NUM_THREADS", "")
    if limit.isdigit() and int(limit) > 0:
        cpus = min(cpus, int(limit))
    return max(1, cpus)


def _threads(threads):
    return host_threads() if threads is None else threads


def _check(status):
    if status != 0:
        raise RuntimeError(f"oracle attention failed with status {status}")


def direct_bf16_pv(p, threads=None):
    out = p._out16()
    args = p.args(_threads(threads))
    _check(lib().orc_direct_bf16_pv(ctypes.byref(args), _ptr(out, ctypes.c_uint16)))
    return out


def tiled_bf16_pv(p, kv_tile, threads=None):
    out = p._out16()
    args = p.args(_threads(threads))
    _check(lib().orc_tiled_bf16_pv(ctypes.byref(args), ctypes.c_int32(kv_tile), _ptr(out, ctypes.c_uint16)))
    return out


def direct_tiled(p, kv_tile, threads=None):
    out = p._out16()
    args = p.args(_threads(threads))
    _check(lib().orc_direct_tiled(ctypes.byref(args), ctypes.c_int32(kv_tile), _ptr(out, ctypes.c_uint16)))
    return out


def fp64_attention(p, threads=None):
    out = np.zeros((p.query.shape[0], p.heads * p.head_dim), dtype=np.float64)
    args = p.args(_threads(threads))
    _check(lib().orc_fp64_attention(ctypes.byref(args), _ptr(out, ctypes.c_double)))
    return out


def fp64_bf16(p, threads=None):
    """fp64 attention rounded once to bf16 (the reference's ``direct_bf16``), as float64."""
    return bf16_to_f32(bf16_from_f64(fp64_attention(p, threads))).astype(np.float64)


def fp32_softmax_attention(p, threads=None):
    out = p._out16()
    args = p.args(_threads(threads))
    _check(lib().orc_fp32_softmax_attention(ctypes.byref(args), _ptr(out, ctypes.c_uint16)))
    return out


def guid_attention(p, tiles_per_row, kv_tile=512, threads=None):
    out = p._out16()
    tiles = np.ascontiguousarray(tiles_per_row, dtype=np.int32)
    args = p.args(_threads(threads))
    _check(lib().orc_guid_attention(ctypes.byref(args), _ptr(tiles, ctypes.c_int32), ctypes.c_int32(kv_tile),
                                    _ptr(out, ctypes.c_uint16)))
    return out


def reference_tiles_per_row(sequences, query_heads, kv_heads, head_dim, total_rows):
    """Number of 512-key tiles the reference runs for each row's query block.

    Restates the tiling policy of src/bridge/attention_plan.cpp:184-262 without
    a sliding window: ``sequences`` is a list of (first_row, length, prefix).
    A value of 1 means the single fused (direct softmax) launch.
    """
    out = np.zeros(total_rows, dtype=np.int32)
    for first_row, length, prefix in sequences:
        done = 0
        while done < length:
            remaining = length - done
            full_visible = prefix + done + remaining
            decode = remaining == 1
            end = full_visible
            count = min(remaining, 256)
            q_bucket = 1 << (count - 1).bit_length()
            if decode and 512 < end <= 8192:
                direct_kv = (end + 511) & ~511
            else:
                direct_kv = max(128, 1 << (end - 1).bit_length())
            fused_bytes = direct_kv * (4 * kv_heads * head_dim + 10 * query_heads)
            single_decode = decode and (end <= 4096 or (end <= 8192 and fused_bytes <= 40 * 1024 * 1024))
            short_prefill = end <= 512 and q_bucket * direct_kv * query_heads <= 4 * 1024 * 1024
            if not single_decode and not short_prefill:
                row_cap = 512 if length >= 2048 else 256
                max_rows = min(row_cap, (16 * 1024 * 1024) // (512 * query_heads))
                max_rows = 1 << (max_rows.bit_length() - 1)
                count = min(remaining, max_rows)
            visible = prefix + done + count
            kv_bucket = direct_kv if (single_decode or short_prefill) else 512
            tiles = (visible + kv_bucket - 1) // kv_bucket
            out[first_row + done:first_row + done + count] = tiles
            done += count
    return out


def isolated_errors(actual, fp64, tiled, tiled_gate=5e-3):
    """Relative-L2 gate of tests/paged_attention_reference.py:60-69 (numpy restatement).

    ``tiled_gate`` is 5e-3 in that file; the reference's device tests use 1e-3
    (tests/fused_paged_decode_device_test.cpp:458).
    """
    actual, fp64, tiled = (np.asarray(v, dtype=np.float64) for v in (actual, fp64, tiled))
    assert actual.shape == fp64.shape == tiled.shape and actual.ndim >= 2
    assert all(np.isfinite(v).all() for v in (actual, fp64, tiled))
    actual, fp64, tiled = (v.reshape(v.shape[0], -1) for v in (actual, fp64, tiled))
    error64 = (np.linalg.norm(actual - fp64, axis=-1) /
               np.maximum(np.linalg.norm(fp64, axis=-1), 1e-30)).max()
    error_tiled = (np.linalg.norm(actual - tiled, axis=-1) /
                   np.maximum(np.linalg.norm(tiled, axis=-1), 1e-30)).max()
    assert error64 <= 1e-2 and error_tiled <= tiled_gate, (error64, error_tiled)
    return float(error64), float(error_tiled)


def tolerance_errors(actual_bits, reference_bits):
    """(max_abs, mean_abs) between two bf16 bit arrays, compared as float64."""
    a = bf16_to_f32(actual_bits).astype(np.float64)
    b = bf16_to_f32(reference_bits).astype(np.float64)
    diff = np.abs(a - b)
    return float(diff.max()), float(diff.mean())


def bf16_ulp(values):
    """Spacing of bf16 numbers at each value: 2^(floor(log2|x|) - 7) (2^-133 at zero)."""
    x = np.abs(np.asarray(values, dtype=np.float64))
    exponent = np.floor(np.log2(np.where(x > 0, x, 1.0)))
    return np.where(x > 0, np.exp2(np.maximum(exponent, -126) - 7), 2.0 ** -133)


def check_tolerance(actual_bits, reference_bits, max_abs=2e-2, mean_abs=2e-3):
    """The bf16 output gate: every element within max(max_abs, one bf16 ulp of the
    reference value) and the mean absolute error within mean_abs.

    The ulp allowance only matters for |reference| >= 4, where one bf16 ulp
    (0.03125) exceeds 2e-2: there even the fp64 result rounded once to bf16
    differs from direct_bf16_pv by one ulp (pinned in tests/test_oracle.py), so
    a flat 2e-2 bound would reject the exact answer. Returns (max_abs, mean_abs).
    """
    a = bf16_to_f32(actual_bits).astype(np.float64)
    b = bf16_to_f32(reference_bits).astype(np.float64)
    diff = np.abs(a - b)
    bound = np.maximum(max_abs, bf16_ulp(b))
    worst = int(np.argmax(diff - bound))
    assert (diff <= bound).all(), (
        f"element {worst}: actual {a.flat[worst]} reference {b.flat[worst]} |diff| {diff.flat[worst]} "
        f"> bound {bound.flat[worst]}")
    assert diff.mean() <= mean_abs, (float(diff.mean()), mean_abs)
    return float(diff.max()), float(diff.mean())


def check_flat_gate(actual_bits, reference_bits, max_abs=2e-2, mean_abs=2e-3):
    """The benchmark's parity gate taken literally: every element within a flat
    max_abs of the reference (no ulp allowance) and the mean absolute error within
    mean_abs. Used on the benchmark configurations C1-C5, whose outputs stay
    below |4| where one bf16 ulp exceeds 2e-2. Returns (max_abs, mean_abs)."""
    a = bf16_to_f32(actual_bits).astype(np.float64)
    b = bf16_to_f32(reference_bits).astype(np.float64)
    diff = np.abs(a - b)
    worst = int(np.argmax(diff))
    assert np.isfinite(diff).all() and diff.max() <= max_abs, (
        f"element {worst}: actual {a.flat[worst]} reference {b.flat[worst]} |diff| {diff.flat[worst]} > {max_abs}")
    assert diff.mean() <= mean_abs, (float(diff.mean()), mean_abs)
    return float(diff.max()), float(diff.mean())


def ulp_allowance_count(actual_bits, reference_bits, max_abs=2e-2):
    """Elements within one bf16 ulp of the reference but farther than the flat max_abs:
    those that pass check_tolerance only through its ulp allowance."""
    a = bf16_to_f32(actual_bits).astype(np.float64)
    b = bf16_to_f32(reference_bits).astype(np.float64)
    diff = np.abs(a - b)
    return int(((diff > max_abs) & (diff <= bf16_ulp(b))).sum())


# ---------------------------------------------------------------------------
# Device metadata validation and the paged slot allocator (integer host logic,
# small cases: pure Python).
# ---------------------------------------------------------------------------

def _ints(values):
    return [int(v) for v in np.asarray(values).reshape(-1)]


def metadata_codes(locations, batch_requests, positions, mapping, prefixes, lengths, slots):
    """Per-row status codes of PagedMetadata's checked device constructor.

    Follows the checks of the reference's host constructor
    (src/bridge/paged_metadata.cpp:82-138) applied per row of the device layout
    of :176-232 (sequence s owns the next lengths[s] rows at positions
    prefixes[s] + i of request batch_requests[s]), with the codes the
    reference's device validation reports (tests/paged_device_metadata_smoke.py:109-125):
    1 location or position out of range, 2 request out of range, 3 mapping
    disagrees, 5 position != prefix + offset, 4 an earlier row writes the same
    slot, 6 / 7 (on a sequence's first row) a missing / aliased prefix slot.
    A row keeps the first code in that order.
    """
    locations, positions = _ints(locations), _ints(positions)
    batch_requests, prefixes, lengths = _ints(batch_requests), _ints(prefixes), _ints(lengths)
    mapping = np.asarray(mapping)
    request_count, context = mapping.shape
    row_seq, first = [], []
    for s, length in enumerate(lengths):
        first.append(len(row_seq))
        row_seq += [s] * length
    rows = len(locations)
    assert len(row_seq) == rows == len(positions)
    codes = [0] * rows
    owner = {}
    for i in range(rows):
        s = row_seq[i]
        loc, pos, req = locations[i], positions[i], batch_requests[s]
        if not (0 <= loc < slots and 0 <= pos < context):
            codes[i] = 1
        elif not 0 <= req < request_count:
            codes[i] = 2
        elif int(mapping[req, pos]) != loc:
            codes[i] = 3
        elif pos != prefixes[s] + i - first[s]:
            codes[i] = 5
        else:
            owner.setdefault(loc, i)
    for i in range(rows):
        if codes[i] == 0 and owner[locations[i]] != i:
            codes[i] = 4
    for s, req in enumerate(batch_requests):
        if not 0 <= req < request_count:
            continue
        missing = aliased = False
        for t in range(prefixes[s] + lengths[s]):
            slot = int(mapping[req, t])
            if slot < 0:
                missing = True
                continue
            o = owner.get(slot)
            if o is not None and (batch_requests[row_seq[o]], positions[o]) != (req, t):
                aliased = True
        i = first[s]
        if codes[i] == 0 and (missing or aliased):
            codes[i] = 6 if missing else 7
    return codes


def host_metadata_error(locations, requests, positions, mapping, slots):
    """The failure the reference's host PagedMetadata constructor reports
    (src/bridge/paged_metadata.cpp:82-139), as its message fragment, or None.

    Checks in the reference's order, the first failing one reported: every
    request-map entry in [-1, slots) (:103-107); then row by row (:110-130)
    location, request and position in range, mapping[request, position] ==
    location, and no earlier row with the same location; then request by
    request, every position up to the request's last row (:131-139) has a
    slot (>= 0) that no other (request, position) row writes. Dimensions are
    assumed valid (:91-94)."""
    mapping = np.asarray(mapping)
    request_count, context = mapping.shape
    locations, requests, positions = _ints(locations), _ints(requests), _ints(positions)
    if any(not -1 <= int(v) < slots for v in mapping.reshape(-1)):
        return "request-to-token slot is out of range"
    targets = {}
    last = [-1] * request_count
    for loc, req, pos in zip(locations, requests, positions):
        if not (0 <= loc < slots and 0 <= req < request_count and 0 <= pos < context):
            return "paged metadata index is out of range"
        if int(mapping[req, pos]) != loc:
            return "output slot does not match request-to-token mapping"
        if loc in targets:
            return "duplicate output KV slot"
        targets[loc] = (req, pos)
        last[req] = max(last[req], pos)
    for req in range(request_count):
        for t in range(last[req] + 1):
            slot = int(mapping[req, t])
            if slot < 0:
                return "missing KV slot in a visible prefix"
            if targets.get(slot, (req, t)) != (req, t):
                return "output KV slot aliases another visible prefix position"
    return None


def page_flags(mapping, batch_requests, prefixes, lengths):
    """Bit k set iff some visible token t < prefix + length of some sequence is
    not at mapping[r, t & ~(P-1)] + (t & (P-1)) with a P-aligned page start,
    for P = 2 << k (k < 10). The largest P with a clear bit is the page size
    the attention plan can use for block tables (P = 1 when every bit is set)."""
    mapping = np.asarray(mapping)
    flags = 0
    for req, prefix, length in zip(_ints(batch_requests), _ints(prefixes), _ints(lengths)):
        if not 0 <= req < mapping.shape[0]:
            continue
        row = [int(v) for v in mapping[req]]
        for k in range(10):
            page = 2 << k
            for t in range(prefix + length):
                start = row[t - t % page]
                if row[t] < 0 or start < 0 or start % page or row[t] != start + t % page:
                    flags |= 1 << k
                    break
    return flags


def largest_page(flags):
    for k in range(9, -1, -1):
        if not flags & (1 << k):
            return 2 << k
    return 1


def allocate_paged_slots(last_slots, free_pages, prefixes, lengths, page_size):
    """New KV slots for the next lengths[s] tokens of each sequence
    (src/bridge/paged_slot_allocator.cpp:91-140): the first
    min(length, (-prefix) mod P) continue after last_slots[s] in the page the
    sequence already holds, the rest fill whole pages taken from free_pages in
    order. Returns (slots, pages used)."""
    free_pages = _ints(free_pages)
    out, used = [], 0
    for last, prefix, length in zip(_ints(last_slots), _ints(prefixes), _ints(lengths)):
        existing = min(length, (-prefix) % page_size)
        out += [last + 1 + i for i in range(existing)]
        for i in range(length - existing):
            out.append(free_pages[used + i // page_size] * page_size + i % page_size)
        used += -(-(length - existing) // page_size)
    return out, used


def release_paged_slots(slots, page_size, max_pages):
    """Distinct pages slot // P of the released slots in order of first
    occurrence (src/bridge/paged_slot_allocator.cpp:142-190). Pages 1 ..
    max_pages belong to the pool (page 0 is reserved); any other page raises
    ValueError, as the reference rejects it ("outside the KV pool")."""
    pages, seen = [], set()
    for slot in _ints(slots):
        page = slot // page_size if slot >= 0 else -1
        if not 1 <= page <= max_pages:
            raise ValueError("released slot is outside the KV pool")
        if page not in seen:
            seen.add(page)
            pages.append(page)
    return pages


# ---------------------------------------------------------------------------
# Rotary position embedding (tests/rotary_runtime_smoke.py:34-48)
# ---------------------------------------------------------------------------

def _rotary_split(x, rotary_dim, neox):
    half = rotary_dim // 2
    rot = x[..., :rotary_dim]
    return (rot[..., :half], rot[..., half:]) if neox else (rot[..., 0::2], rot[..., 1::2])


def _rotary_join(out, first, second, rotary_dim, neox):
    half = rotary_dim // 2
    if neox:
        out[..., :half] = first
        out[..., half:rotary_dim] = second
    else:
        out[..., 0:rotary_dim:2] = first
        out[..., 1:rotary_dim:2] = second
    return out


def rotary_bf16(x_bits, cos_sin_bits, positions, head_dim, rotary_dim, neox):
    """Rotated bf16 rows (uint16 [rows, width]) as the reference's fp32 form computes
    them: per head, pairs (a, b) -> (bf16(a cos - b sin), bf16(b cos + a sin)) in
    float32 with cos/sin from row ``positions[r]`` of the [cache_rows, rotary_dim]
    table (cos | sin); elements past rotary_dim are unchanged."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows = x_bits.shape[0]
    x = bf16_to_f32(x_bits).reshape(rows, -1, head_dim)
    table = bf16_to_f32(cos_sin_bits)[np.asarray(positions, dtype=np.int64)]
    half = rotary_dim // 2
    cos, sin = table[:, None, :half], table[:, None, half:rotary_dim]
    a, b = _rotary_split(x, rotary_dim, neox)
    first = bf16_from_f32((a * cos - b * sin).astype(np.float32))
    second = bf16_from_f32((b * cos + a * sin).astype(np.float32))
    out = x_bits.reshape(rows, -1, head_dim).copy()
    return _rotary_join(out, first, second, rotary_dim, neox).reshape(x_bits.shape)


def rotary_f64(x_bits, cos_sin_bits, positions, head_dim, rotary_dim, neox):
    """fp64 form: the same pairs computed in binary64 and rounded once to bf16,
    returned as float64 values (tests/rotary_runtime_smoke.py:34-48, fp64=True)."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows = x_bits.shape[0]
    x = bf16_to_f32(x_bits).astype(np.float64).reshape(rows, -1, head_dim)
    table = bf16_to_f32(cos_sin_bits).astype(np.float64)[np.asarray(positions, dtype=np.int64)]
    half = rotary_dim // 2
    cos, sin = table[:, None, :half], table[:, None, half:rotary_dim]
    a, b = _rotary_split(x, rotary_dim, neox)
    first = bf16_to_f32(bf16_from_f64(a * cos - b * sin)).astype(np.float64)
    second = bf16_to_f32(bf16_from_f64(b * cos + a * sin)).astype(np.float64)
    out = x.copy()
    return _rotary_join(out, first, second, rotary_dim, neox).reshape(rows, -1)


def rotary_gate(actual_bits, x_bits, cos_sin_bits, positions, head_dim, rotary_dim, neox):
    """The reference test's acceptance (tests/rotary_runtime_smoke.py:51-60): per-row
    relative L2 error against the fp64 form <= max(3e-3, 2 * floor) and <= 1e-2,
    floor = the fp32 form's own error. Returns (error, floor)."""
    ref64 = rotary_f64(x_bits, cos_sin_bits, positions, head_dim, rotary_dim, neox)
    ref32 = bf16_to_f32(rotary_bf16(x_bits, cos_sin_bits, positions, head_dim, rotary_dim, neox)).astype(np.float64)
    actual = bf16_to_f32(np.asarray(actual_bits, dtype=np.uint16)).astype(np.float64).reshape(ref64.shape)
    assert np.isfinite(actual).all() and np.isfinite(ref64).all()
    denom = np.maximum(np.linalg.norm(ref64, axis=-1), 1e-30)
    error = float((np.linalg.norm(actual - ref64, axis=-1) / denom).max())
    floor = float((np.linalg.norm(ref32 - ref64, axis=-1) / denom).max())
    assert error <= max(3e-3, 2 * floor) and error <= 1e-2, (error, floor)
    return error, floor
