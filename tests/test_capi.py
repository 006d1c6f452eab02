"""CPU checks of the C ABI library: it loads, exports exactly what include/gaudirt_amd.h
declares, leaves no symbol unresolved, and rejects bad arguments before any GPU work."""

import ctypes
import pathlib
import re
import subprocess

import pytest

from gaudirt_amd import capi

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "gaudirt_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(gk_\w+)\s*\(", text, flags=re.M))
    return names


@pytest.fixture(scope="module")
def lib():
    if not capi.LIB_PATH.exists():
        pytest.fail(f"{capi.LIB_PATH} is not built: run `python -m gaudirt_amd.build`")
    return capi.load()


def test_header_declarations_are_exported(lib):
    names = declared_functions()
    assert "gk_paged_decode" in names and "gk_kv_store" in names
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # The Python binding lists the same set.
    assert set(capi.EXPORTED) == names, set(capi.EXPORTED) ^ names


def test_no_unresolved_symbols():
    # A kernel whose host stub was not instantiated shows up as an undefined
    # symbol only when the library is loaded on a GPU box; catch it here.
    out = subprocess.run(["nm", "-D", "--undefined-only", str(capi.LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    unresolved = [line.split()[-1] for line in out.splitlines()
                  if line.split() and line.split()[0] == "U" and "@" not in line.split()[-1]]
    assert not unresolved, unresolved


def test_version_and_error_convention(lib):
    assert lib.gk_version().decode().startswith("gaudirt_amd")
    rc = lib.gk_paged_decode(None, None, 0, None)
    assert rc == capi.GK_ERR_INVALID_ARGUMENT
    assert "null parameters" in lib.gk_last_error().decode()


def test_decode_validation_rejects_before_launch(lib):
    p = capi.DecodeParams()
    p.rows, p.q_heads, p.kv_heads, p.head_dim = 4, 8, 2, 96
    p.block_size, p.slots, p.scale = 128, 8192, 0.1
    assert lib.gk_paged_decode(ctypes.byref(p), None, 0, None) == capi.GK_ERR_UNSUPPORTED
    assert "head dimension" in lib.gk_last_error().decode()
    p.head_dim, p.block_size = 128, 96
    assert lib.gk_paged_decode(ctypes.byref(p), None, 0, None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "power of two" in lib.gk_last_error().decode()
    p.block_size, p.q_heads = 128, 7
    assert lib.gk_paged_decode(ctypes.byref(p), None, 0, None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "head geometry" in lib.gk_last_error().decode()


def test_kv_store_validation(lib):
    rc = lib.gk_kv_store(None, None, 128, 128, None, 4, None, 64, 1, 100, None)
    assert rc == capi.GK_ERR_INVALID_ARGUMENT and "geometry" in lib.gk_last_error().decode()
    assert lib.gk_kv_store(None, None, 128, 128, None, 0, None, 64, 1, 128, None) == capi.GK_OK


def test_struct_size_guard_rejects_mismatched_callers(lib):
    # A caller compiled against another layout of gk_decode_params is rejected
    # before any field past struct_size is read.
    p = capi.DecodeParams()
    p.rows, p.q_heads, p.kv_heads, p.head_dim, p.block_size, p.slots, p.scale = 1, 8, 2, 128, 128, 8192, 0.1
    p.struct_size = ctypes.sizeof(p) - 8
    assert lib.gk_paged_decode(ctypes.byref(p), None, 0, None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "struct_size" in lib.gk_last_error().decode()
    assert lib.gk_paged_decode_workspace_bytes(ctypes.byref(p)) == 0
    q = capi.PrefillParams()
    q.struct_size = 8
    assert lib.gk_paged_prefill(ctypes.byref(q), None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "struct_size" in lib.gk_last_error().decode()


def test_prefill_alignment_validation(lib):
    # query, pool and out must be 16-byte aligned with row strides in whole
    # 16-byte pieces (the kernel writes its output rows as 16-byte stores);
    # checked on the host before anything is launched.
    q = capi.PrefillParams()
    q.q_heads, q.kv_heads, q.head_dim, q.block_size, q.slots, q.scale = 8, 2, 128, 128, 8192, 0.1
    q.seqs, q.max_rows, q.bt_stride = 1, 4, 8
    for name in ("query", "pool", "block_tables", "seq_request", "seq_first_row", "seq_rows", "seq_prefix", "out"):
        setattr(q, name, 256)
    q.q_row_stride = q.out_row_stride = 8 * 128
    for field, value in (("out", 258), ("out_row_stride", 8 * 128 + 4), ("query", 264), ("q_row_stride", 8 * 128 + 2)):
        saved = getattr(q, field)
        setattr(q, field, value)
        assert lib.gk_paged_prefill(ctypes.byref(q), None) == capi.GK_ERR_INVALID_ARGUMENT, field
        assert "16-byte aligned" in lib.gk_last_error().decode(), field
        setattr(q, field, saved)


def test_metadata_and_allocator_validation(lib):
    p = capi.MetadataParams()
    p.struct_size = 16
    assert lib.gk_metadata_normalize(ctypes.byref(p), None, 0, None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "struct_size" in lib.gk_last_error().decode()
    p = capi.MetadataParams()
    p.rows, p.padded_rows, p.batch, p.requests, p.context, p.slots = 4, 4, 5, 2, 64, 128
    assert lib.gk_metadata_normalize(ctypes.byref(p), None, 0, None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "dimensions" in lib.gk_last_error().decode()  # batch > rows
    p.batch = 2
    assert lib.gk_metadata_normalize(ctypes.byref(p), None, 0, None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "null pointer" in lib.gk_last_error().decode()
    # Validation needs the duplicate-slot table: 2 x pow2(>= 2 rows, >= 64) + batch words.
    assert lib.gk_metadata_workspace_bytes(4, 2) == (64 * 2 + 2) * 4
    assert lib.gk_metadata_workspace_bytes(100, 3) == (256 * 2 + 3) * 4
    assert lib.gk_block_tables(None, 2, 64, 48, None, 2, None) == capi.GK_ERR_INVALID_ARGUMENT
    assert lib.gk_paged_alloc_slots(None, None, None, 1, 0, 4, None, None) == capi.GK_ERR_INVALID_ARGUMENT
    assert lib.gk_paged_release_workspace_bytes(512) == 513 * 4
    rc = lib.gk_paged_release_slots(None, 4, 16, 0, None, 0, None, None, None)
    assert rc == capi.GK_ERR_INVALID_ARGUMENT and "release geometry" in lib.gk_last_error().decode()
    rc = lib.gk_paged_release_slots(ctypes.c_void_p(16), 4, 16, 512, ctypes.c_void_p(16), 8, ctypes.c_void_p(16),
                                    ctypes.c_void_p(16), None)
    assert rc == capi.GK_ERR_WORKSPACE


def test_stream_unit_cost_matches_the_header():
    source = (ROOT / "gaudirt_amd" / "csrc" / "work_order.hpp").read_text()
    assert re.search(r"#define GK_STREAM_UNIT_COST (\d+)", source).group(1) == str(capi.STREAM_UNIT_COST)


def test_metadata_staged_words_validation(lib):
    """Staged-word arguments are refused before any launch: missing pointers,
    more than GK_METADATA_INLINE_WORDS words, an input only partly inside the
    staged range, an unredirected input or an output inside it."""
    header = (ROOT / "include" / "gaudirt_amd.h").read_text()
    assert f"#define GK_METADATA_INLINE_WORDS {capi.GK_METADATA_INLINE_WORDS}" in header
    host = (ctypes.c_int32 * capi.GK_METADATA_INLINE_WORDS)()
    staged = 1 << 40  # device addresses are never dereferenced on the host
    p = capi.MetadataParams()
    p.rows, p.padded_rows, p.batch, p.requests, p.context, p.slots = 4, 4, 2, 2, 64, 128
    names = ("locations", "batch_requests", "positions", "row_seq", "seq_prefix", "seq_first_row",
             "out_locations", "out_requests", "out_positions")
    for i, name in enumerate(names):
        setattr(p, name, (1 << 36) + 4096 * i)

    def refused(match):
        assert lib.gk_metadata_normalize(ctypes.byref(p), None, 0, None) == capi.GK_ERR_INVALID_ARGUMENT
        assert match in lib.gk_last_error().decode()

    p.staged_words, p.staged_device, p.staged_count = ctypes.addressof(host), staged, 0
    refused("staged words need")
    p.staged_count = capi.GK_METADATA_INLINE_WORDS + 1
    refused("staged words need")
    p.staged_count, p.staged_words = 64, None
    refused("staged words need")
    p.staged_words = ctypes.addressof(host)
    p.row_seq = staged + 4 * 62  # 4 rows from word 62 of 64
    refused("overlaps the staged words")
    p.row_seq = staged + 2  # not word aligned
    refused("overlaps the staged words")
    p.row_seq = staged
    p.locations = staged + 64
    refused("overlaps the staged words")
    p.locations = 1 << 36
    p.out_positions = staged + 4 * 63
    refused("overlaps the staged words")


def test_rotary_validation(lib):
    p = capi.RotaryParams()
    p.struct_size = 24
    assert lib.gk_rotary_embedding(ctypes.byref(p), None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "struct_size" in lib.gk_last_error().decode()
    p = capi.RotaryParams()
    p.rows, p.head_dim, p.rotary_dim, p.q_width, p.k_width, p.cache_rows = 4, 128, 127, 1024, 256, 64
    assert lib.gk_rotary_embedding(ctypes.byref(p), None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "rotary dimension" in lib.gk_last_error().decode()
    p.rotary_dim, p.k_width = 128, 200
    assert lib.gk_rotary_embedding(ctypes.byref(p), None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "geometry" in lib.gk_last_error().decode()
    p.k_width = 256
    assert lib.gk_rotary_embedding(ctypes.byref(p), None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "null pointer" in lib.gk_last_error().decode()
    p.rows = 0
    assert lib.gk_rotary_embedding(ctypes.byref(p), None) == capi.GK_OK
    # The fused store checks the pool geometry before anything is launched.
    p.rows = 4
    for name in ("query", "key", "positions", "cos_sin", "q_out", "value", "slot_mapping", "pool"):
        setattr(p, name, 16)
    p.q_row_stride, p.k_row_stride, p.q_out_row_stride, p.v_row_stride = 1024, 256, 1024, 256
    p.slots, p.kv_heads = 128, 1
    assert lib.gk_rotary_kv_store(ctypes.byref(p), None) == capi.GK_ERR_INVALID_ARGUMENT
    assert "pool geometry" in lib.gk_last_error().decode()  # k_width != kv_heads * head_dim
