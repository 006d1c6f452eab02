"""ctypes binding of the C ABI in include/gaudirt_amd.h.

This is the thin Python view of ``libgaudirt_amd.so`` that the GPU tests and the
benchmark call through: device buffers are torch tensors on ``cuda``, passed by
pointer together with the current HIP stream. Loading fails loudly when the
library has not been built; there is no other implementation behind it.
"""

import ctypes
import os
import pathlib

PACKAGE = pathlib.Path(__file__).resolve().parent
# GAUDIRT_AMD_LIB selects another build of the same library (e.g. a tuning variant).
LIB_PATH = pathlib.Path(os.environ.get("GAUDIRT_AMD_LIB", PACKAGE / "libgaudirt_amd.so"))

GK_OK = 0
GK_ERR_INVALID_ARGUMENT = 1
GK_ERR_UNSUPPORTED = 2
GK_ERR_HIP = 3
GK_ERR_OUT_OF_MEMORY = 4
GK_ERR_WORKSPACE = 5
GK_DECODE_SCRATCH_BYTES = 32 << 20
GK_METADATA_INLINE_WORDS = 768
# Fixed cost per work unit of the balanced decode schedule, in tiles
# (GK_STREAM_UNIT_COST of gaudirt_amd/csrc/work_order.hpp); it enters the
# schedule's 2^31 gate.
STREAM_UNIT_COST = 2

# Every function include/gaudirt_amd.h declares.
EXPORTED = [
    "gk_last_error", "gk_version", "gk_kv_store", "gk_paged_decode_workspace_bytes",
    "gk_paged_decode_partition_tokens", "gk_paged_decode", "gk_paged_decode_scratch", "gk_paged_prefill",
    "gk_split_k_merge",
    "gk_attn_tile_indices", "gk_advance_decode_lengths",
    "gk_metadata_workspace_bytes", "gk_metadata_normalize", "gk_block_tables",
    "gk_paged_alloc_slots", "gk_paged_release_workspace_bytes", "gk_paged_release_slots",
    "gk_allocator_create", "gk_allocator_destroy", "gk_allocator_alloc", "gk_allocator_record_stream",
    "gk_allocator_free", "gk_allocator_empty_cache", "gk_allocator_get_stats",
    "gk_rotary_embedding", "gk_rotary_kv_store",
]

c_void_p = ctypes.c_void_p
c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float


class _Sized(ctypes.Structure):
    """Parameter struct whose leading struct_size field is filled in on construction."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self.struct_size = ctypes.sizeof(self)


class DecodeParams(_Sized):
    _fields_ = [
        ("struct_size", ctypes.c_size_t),
        ("query", c_void_p), ("q_row_stride", c_i64),
        ("pool", c_void_p), ("slots", c_i64),
        ("block_tables", c_void_p), ("bt_stride", c_i64), ("block_size", c_i32),
        ("row_request", c_void_p), ("row_context", c_void_p), ("rows", c_i32),
        ("q_heads", c_i32), ("kv_heads", c_i32), ("head_dim", c_i32),
        ("scale", c_f32), ("softcap", c_f32), ("sliding_window", c_i32),
        ("max_context", c_i32), ("partition_tokens", c_i32),
        ("out", c_void_p), ("out_row_stride", c_i64),
        ("new_key", c_void_p), ("new_value", c_void_p), ("new_kv_row_stride", c_i64),
        ("slot_mapping", c_void_p), ("row_map", c_void_p),
    ]


class PrefillParams(_Sized):
    _fields_ = [
        ("struct_size", ctypes.c_size_t),
        ("query", c_void_p), ("q_row_stride", c_i64),
        ("pool", c_void_p), ("slots", c_i64),
        ("block_tables", c_void_p), ("bt_stride", c_i64), ("block_size", c_i32),
        ("seq_request", c_void_p), ("seq_first_row", c_void_p), ("seq_rows", c_void_p), ("seq_prefix", c_void_p),
        ("seqs", c_i32), ("max_rows", c_i32),
        ("q_heads", c_i32), ("kv_heads", c_i32), ("head_dim", c_i32),
        ("scale", c_f32), ("softcap", c_f32), ("sliding_window", c_i32),
        ("out", c_void_p), ("out_row_stride", c_i64),
    ]


class RotaryParams(_Sized):
    _fields_ = [
        ("struct_size", ctypes.c_size_t),
        ("query", c_void_p), ("q_row_stride", c_i64), ("q_width", c_i64),
        ("key", c_void_p), ("k_row_stride", c_i64), ("k_width", c_i64),
        ("positions", c_void_p), ("positions_int64", c_i32),
        ("cos_sin", c_void_p), ("cache_rows", c_i64),
        ("rows", c_i32), ("head_dim", c_i32), ("rotary_dim", c_i32), ("is_neox", c_i32),
        ("q_out", c_void_p), ("q_out_row_stride", c_i64),
        ("k_out", c_void_p), ("k_out_row_stride", c_i64),
        ("value", c_void_p), ("v_row_stride", c_i64),
        ("slot_mapping", c_void_p), ("pool", c_void_p), ("slots", c_i64), ("kv_heads", c_i32),
    ]


class MetadataParams(_Sized):
    _fields_ = [
        ("struct_size", ctypes.c_size_t),
        ("locations", c_void_p), ("batch_requests", c_void_p), ("positions", c_void_p), ("token_ids", c_void_p),
        ("locations_int64", c_i32), ("requests_int64", c_i32), ("positions_int64", c_i32), ("tokens_int64", c_i32),
        ("mapping", c_void_p),
        ("row_seq", c_void_p), ("seq_prefix", c_void_p), ("seq_first_row", c_void_p), ("seq_visible", c_void_p),
        ("visible_total", c_i64),
        ("rows", c_i32), ("padded_rows", c_i32), ("batch", c_i32), ("requests", c_i32), ("context", c_i32),
        ("vocabulary", c_i32),
        ("slots", c_i64),
        ("out_locations", c_void_p), ("out_requests", c_void_p), ("out_positions", c_void_p),
        ("out_tokens", c_void_p), ("status", c_void_p), ("token_status", c_void_p), ("page_flags", c_void_p),
        ("staged_words", c_void_p), ("staged_device", c_void_p), ("staged_count", c_i32),
    ]


class AllocatorStats(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint64) for name in (
        "allocated_bytes", "peak_bytes", "reserved_bytes", "largest_free_block", "slabs", "events_created")]


class GkError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"gaudirt_amd error {code}: {message}")
        self.code = code


_lib = None


def load():
    """Load libgaudirt_amd.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: run `python -m gaudirt_amd.build` first")
    # PyTorch-ROCm ships its own HIP runtime. Loading it first makes the library
    # bind to that same runtime; loaded the other way round, the process holds
    # two runtimes and launches on PyTorch's streams fail ("no ROCm-capable
    # device is detected").
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.gk_last_error.restype = ctypes.c_char_p
    lib.gk_version.restype = ctypes.c_char_p
    lib.gk_paged_decode_workspace_bytes.restype = ctypes.c_size_t
    lib.gk_paged_decode_workspace_bytes.argtypes = [ctypes.POINTER(DecodeParams)]
    lib.gk_paged_decode_partition_tokens.restype = c_i32
    lib.gk_paged_decode_partition_tokens.argtypes = [ctypes.POINTER(DecodeParams)]
    lib.gk_paged_decode.argtypes = [ctypes.POINTER(DecodeParams), c_void_p, ctypes.c_size_t, c_void_p]
    lib.gk_paged_decode_scratch.argtypes = [ctypes.POINTER(DecodeParams), c_void_p]
    lib.gk_paged_prefill.argtypes = [ctypes.POINTER(PrefillParams), c_void_p]
    lib.gk_kv_store.argtypes = [c_void_p, c_void_p, c_i64, c_i64, c_void_p, c_i32, c_void_p, c_i64, c_i32, c_i32,
                                c_void_p]
    lib.gk_split_k_merge.argtypes = [c_void_p, c_void_p, c_void_p, c_i32, c_i32, c_i32, c_i32, c_void_p, c_i64,
                                     c_void_p]
    lib.gk_attn_tile_indices.argtypes = [c_void_p, c_void_p, c_void_p, c_i32, c_i32, c_void_p, c_void_p]
    lib.gk_advance_decode_lengths.argtypes = [c_void_p, c_void_p, c_i64, c_void_p, c_void_p, c_void_p]
    lib.gk_metadata_workspace_bytes.restype = ctypes.c_size_t
    lib.gk_metadata_workspace_bytes.argtypes = [c_i32, c_i32]
    lib.gk_metadata_normalize.argtypes = [ctypes.POINTER(MetadataParams), c_void_p, ctypes.c_size_t, c_void_p]
    lib.gk_block_tables.argtypes = [c_void_p, c_i32, c_i32, c_i32, c_void_p, c_i32, c_void_p]
    lib.gk_paged_alloc_slots.argtypes = [c_void_p, c_void_p, c_void_p, c_i32, c_i64, c_i64, c_void_p, c_void_p]
    lib.gk_paged_release_workspace_bytes.restype = ctypes.c_size_t
    lib.gk_paged_release_workspace_bytes.argtypes = [c_i64]
    lib.gk_paged_release_slots.argtypes = [c_void_p, c_i64, c_i64, c_i64, c_void_p, ctypes.c_size_t, c_void_p,
                                           c_void_p, c_void_p]
    lib.gk_allocator_create.argtypes = [c_i32, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(c_void_p)]
    lib.gk_allocator_destroy.argtypes = [c_void_p]
    lib.gk_allocator_alloc.argtypes = [c_void_p, ctypes.c_uint64, c_void_p, ctypes.POINTER(c_void_p)]
    lib.gk_allocator_record_stream.argtypes = [c_void_p, c_void_p, c_void_p]
    lib.gk_allocator_free.argtypes = [c_void_p, c_void_p]
    lib.gk_allocator_empty_cache.argtypes = [c_void_p]
    lib.gk_allocator_get_stats.argtypes = [c_void_p, ctypes.POINTER(AllocatorStats)]
    lib.gk_rotary_embedding.argtypes = [ctypes.POINTER(RotaryParams), c_void_p]
    lib.gk_rotary_kv_store.argtypes = [ctypes.POINTER(RotaryParams), c_void_p]
    _lib = lib
    return lib


def check(code):
    if code != GK_OK:
        raise GkError(code, load().gk_last_error().decode())
    return code


def ptr(tensor):
    """Device pointer of a tensor (None for None)."""
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def current_stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
