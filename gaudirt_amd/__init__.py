"""MI355X-native paged-attention path of GaudiRT (gfx950 HIP kernels behind a C ABI).

Python view of the path, mirroring the reference's ``gaudirt`` operator API
for it (python/gaudirt/__init__.py, src/bridge/generic_private_use1.cpp:430-540):

- ``torch.ops.gaudirt.paged_attn`` / ``_paged_attn_validated`` /
  ``_advance_decode_lengths``, the rotary ops ``rotary_embedding`` /
  ``rotary_embedding_positions`` / ``_rotary_embedding_validated``, and
  ``torch.classes.gaudirt.PagedMetadata`` are registered by the HIP extension
  ``gaudirt_amd._C``, together with ``rotary_paged_attn`` (rotary embedding
  fused into the attention's KV store; no counterpart in the reference);
- ``allocate_paged_kv(layers, slots, kv_heads, head_dim)`` returns a zeroed
  head-major bf16 pool ``[layers, 2, kv_heads, slots, head_dim]`` from the
  stream-ordered block allocator, and ``kv_pool_views(pool, layer)`` its
  ``(key_pool, value_pool)`` views ``[slots, kv_heads, head_dim]``.

- ``set_batch_invariant_decode(enabled, partition_tokens=2048)``: decode rows
  of ``paged_attn`` on fixed split-K partitions, so each row's output is a
  function of that row alone, bit for bit (the reference's single-row replay,
  tests/paged_attention_smoke.py:145-150); off by default, where the balanced
  schedule's split points depend on the whole batch. The environment variable
  ``GAUDIRT_AMD_BATCH_INVARIANT_DECODE`` (``1``, or a partition in keys) turns
  it on when the extension loads.

The extension is loaded on first use of any of these names (or by
``load_extension()``); a missing build raises ImportError. There is no other
implementation behind them.
"""

import os
import pathlib

_PACKAGE = pathlib.Path(__file__).resolve().parent
_ext = None

__all__ = ["load_extension", "PagedMetadata", "paged_attn", "allocate_paged_kv", "kv_pool_views",
           "advance_decode_lengths", "kv_allocator_stats", "paged_attn_kv_tile", "set_batch_invariant_decode",
           "batch_invariant_decode"]

# Keys per split-K partition of the batch-invariant decode mode.
BATCH_INVARIANT_PARTITION = 2048


def load_extension():
    """Import the HIP extension (registers torch.ops.gaudirt.* and the PagedMetadata class)."""
    global _ext
    if _ext is not None:
        return _ext
    import torch

    try:
        from . import _C  # noqa: F401
    except ImportError as exc:
        raise ImportError(
            "gaudirt_amd: the HIP extension _C is not built or cannot load; run `python -m gaudirt_amd.build` "
            f"({exc})") from exc
    from . import _C as ext
    _register_fakes(torch)
    _ext = ext
    env = os.environ.get("GAUDIRT_AMD_BATCH_INVARIANT_DECODE", "").strip()
    if env and env != "0":
        set_batch_invariant_decode(True, BATCH_INVARIANT_PARTITION if env == "1" else int(env))
    return ext


def set_batch_invariant_decode(enabled=True, partition_tokens=BATCH_INVARIANT_PARTITION):
    """Decode rows of paged_attn on fixed partitions of `partition_tokens` keys (a
    multiple of 32 up to 8192): every row's output then depends on that row alone.
    Off: the library's balanced schedule (the default; faster on skewed batches)."""
    load_extension()._set_decode_partition(int(partition_tokens) if enabled else 0)


def batch_invariant_decode():
    """The fixed decode partition in keys, or 0 when the library chooses."""
    return load_extension()._decode_partition()


def _register_fakes(torch):
    """Meta kernels for torch.compile tracing (python/gaudirt/__init__.py:136-153)."""

    @torch.library.register_fake("gaudirt::paged_attn")
    def _fake_paged_attn(query, key, value, key_pool, value_pool, metadata, head_dim, scale, softcap=0.0,
                         sliding_window=-1):
        torch._check(key.shape[0] == query.shape[0])
        torch._check(value.shape[0] == query.shape[0])
        return torch.empty_like(query, memory_format=torch.contiguous_format)

    @torch.library.register_fake("gaudirt::_paged_attn_validated")
    def _fake_paged_attn_validated(query, key, value, key_pool, value_pool, locations, requests, positions,
                                   mapping, header, head_dim, scale, softcap=0.0, sliding_window=-1):
        torch._check(key.shape[0] == query.shape[0])
        torch._check(value.shape[0] == query.shape[0])
        torch._check(locations.shape[0] == query.shape[0])
        torch._check(requests.shape[0] == query.shape[0])
        torch._check(positions.shape[0] == query.shape[0])
        return torch.empty_like(query, memory_format=torch.contiguous_format)

    @torch.library.register_fake("gaudirt::_advance_decode_lengths")
    def _fake_advance_decode_lengths(seq_lens, orig_seq_lens):
        return torch.empty_like(seq_lens), torch.empty_like(orig_seq_lens)

    @torch.library.register_fake("gaudirt::rotary_embedding")
    def _fake_rotary_embedding(query, key, cache, metadata, head_dim, rotary_dim, is_neox):
        torch._check(key.shape[0] == query.shape[0])
        return (torch.empty_like(query, memory_format=torch.contiguous_format),
                torch.empty_like(key, memory_format=torch.contiguous_format))

    @torch.library.register_fake("gaudirt::rotary_embedding_positions")
    def _fake_rotary_embedding_positions(query, key, cache, positions, head_dim, rotary_dim, is_neox):
        torch._check(key.shape[0] == query.shape[0])
        torch._check(positions.shape[0] == query.shape[0])
        return (torch.empty_like(query, memory_format=torch.contiguous_format),
                torch.empty_like(key, memory_format=torch.contiguous_format))

    @torch.library.register_fake("gaudirt::_rotary_embedding_validated")
    def _fake_rotary_embedding_validated(query, key, cache, positions, header, context, head_dim, rotary_dim,
                                         is_neox):
        torch._check(key.shape[0] == query.shape[0])
        torch._check(positions.shape[0] == query.shape[0])
        return (torch.empty_like(query, memory_format=torch.contiguous_format),
                torch.empty_like(key, memory_format=torch.contiguous_format))

    @torch.library.register_fake("gaudirt::rotary_paged_attn")
    def _fake_rotary_paged_attn(query, key, value, key_pool, value_pool, cache, metadata, head_dim, rotary_dim,
                                is_neox, scale, softcap=0.0, sliding_window=-1):
        torch._check(key.shape[0] == query.shape[0])
        torch._check(value.shape[0] == query.shape[0])
        return torch.empty_like(query, memory_format=torch.contiguous_format)


def allocate_paged_kv(layers, slots, kv_heads, head_dim):
    return load_extension()._allocate_paged_kv(layers, slots, kv_heads, head_dim)


def kv_pool_views(pool, layer):
    """(key_pool, value_pool) of one layer: [slots, kv_heads, head_dim] views of the combined storage."""
    return pool[layer, 0].transpose(0, 1), pool[layer, 1].transpose(0, 1)


def kv_allocator_stats(device=0):
    return load_extension()._kv_allocator_stats(device)


def paged_attn_kv_tile(rows):
    return load_extension()._paged_attn_kv_tile(rows)


def __getattr__(name):
    if name in ("PagedMetadata", "paged_attn", "advance_decode_lengths"):
        load_extension()
        import torch

        return {
            "PagedMetadata": lambda: torch.classes.gaudirt.PagedMetadata,
            "paged_attn": lambda: torch.ops.gaudirt.paged_attn,
            "advance_decode_lengths": lambda: torch.ops.gaudirt._advance_decode_lengths,
        }[name]()
    raise AttributeError(f"module 'gaudirt_amd' has no attribute {name!r}")
