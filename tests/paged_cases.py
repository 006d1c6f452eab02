"""Seeded synthetic problems for the paged-attention tests and the benchmark.

A case is the reference's decode/prefill setup in block-table form: a bf16
head-major pool [2, Hkv, S, d], query rows, per-sequence block tables and
lengths. Small cases are generated with numpy on the host; full-size cases are
generated on the GPU with a seeded torch generator and copied back only where
the oracle needs them.
"""

import math

import numpy as np

from oracle import oracle as orc
from gaudirt_amd.workloads import permuted_block_tables  # noqa: F401  (re-exported)


def bf16_normal(rng, shape):
    return orc.bf16_from_f32(rng.standard_normal(shape, dtype=np.float32))


class DecodeCase:
    """Host-side description of a decode problem (numpy arrays; bf16 as uint16)."""

    def __init__(self, query, pool, block_tables, lens, heads, kv_heads, head_dim, block_size, scale=None,
                 softcap=0.0, window=-1):
        self.query = query              # uint16 [B, Hq*d]
        self.pool = pool                # uint16 [2, Hkv, S, d]
        self.block_tables = block_tables  # int32 [B, max_blocks]
        self.lens = lens                # int32 [B] visible keys
        self.heads, self.kv_heads, self.head_dim = heads, kv_heads, head_dim
        self.block_size = block_size
        self.scale = float(np.float32(scale if scale is not None else 1 / math.sqrt(head_dim)))
        self.softcap, self.window = softcap, window

    @property
    def batch(self):
        return self.query.shape[0]

    @property
    def slots(self):
        return self.pool.shape[2]

    def oracle_problem(self):
        context = int(self.lens.max())
        mapping = orc.mapping_from_block_table(self.block_tables, self.block_size, context)
        return orc.Problem(self.query, self.pool, np.arange(self.batch), self.lens.astype(np.int64) - 1, mapping,
                           self.heads, self.kv_heads, self.head_dim, self.scale, self.softcap, self.window)

    def kv_bytes(self):
        """Algorithmic KV bytes one decode step reads (every visible key and value row once per kv head)."""
        return int(self.lens.astype(np.int64).sum()) * self.kv_heads * self.head_dim * 2 * 2


def decode_case(seed, batch, heads, kv_heads, head_dim, block_size, num_blocks, lens):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int32)
    pool = bf16_normal(rng, (2, kv_heads, num_blocks * block_size, head_dim))
    query = bf16_normal(rng, (batch, heads * head_dim))
    tables = permuted_block_tables(rng, lens, block_size, num_blocks)
    return DecodeCase(query, pool, tables, lens, heads, kv_heads, head_dim, block_size)


def c1_case(seed=20261201):
    """Workload C1: batch 4, 8 q / 2 kv heads, d 128, block 128, ctx U[1,512], 64-block pool."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, 513, 4)
    return decode_case(seed + 1, 4, 8, 2, 128, 128, 64, lens)


def host_case(device_case):
    """Oracle view of a workloads.DeviceDecodeCase (copies its pool and queries back)."""
    query, pool = device_case.host_arrays()
    return DecodeCase(query, pool, device_case.tables, device_case.lens, device_case.heads,
                      device_case.kv_heads, device_case.head_dim, device_case.block_size, device_case.scale)


class PrefillCase:
    """Host-side chunked-prefill problem: sequences with a cached prefix plus a chunk of query rows.

    Rows are concatenated per sequence; every key of every chunk (prefix and
    chunk rows) is already in the pool, as after the store. Block tables map
    token t of request r to slot bt[r, t // block] * block + t % block.
    """

    def __init__(self, seed, heads, kv_heads, head_dim, block_size, prefixes, chunks, num_blocks=None,
                 shared_prefix_blocks=0, softcap=0.0, window=-1):
        rng = np.random.default_rng(seed)
        self.heads, self.kv_heads, self.head_dim, self.block_size = heads, kv_heads, head_dim, block_size
        self.prefixes = np.asarray(prefixes, dtype=np.int32)
        self.chunks = np.asarray(chunks, dtype=np.int32)
        lens = self.prefixes + self.chunks
        seqs = len(lens)
        need = (lens + block_size - 1) // block_size
        own = need - shared_prefix_blocks
        if num_blocks is None:
            num_blocks = shared_prefix_blocks + int(own.sum())
        ids = rng.permutation(num_blocks).astype(np.int32)
        shared, cursor = ids[:shared_prefix_blocks], shared_prefix_blocks
        self.block_tables = np.full((seqs, int(need.max())), -1, dtype=np.int32)
        for s in range(seqs):
            self.block_tables[s, :shared_prefix_blocks] = shared
            self.block_tables[s, shared_prefix_blocks:need[s]] = ids[cursor:cursor + own[s]]
            cursor += own[s]
        self.pool = bf16_normal(rng, (2, kv_heads, num_blocks * block_size, head_dim))
        self.first_rows = np.concatenate([[0], np.cumsum(self.chunks)[:-1]]).astype(np.int32)
        self.rows = int(self.chunks.sum())
        self.query = bf16_normal(rng, (self.rows, heads * head_dim))
        self.scale = float(np.float32(1 / math.sqrt(head_dim)))
        self.softcap, self.window = softcap, window
        self.requests = np.repeat(np.arange(seqs), self.chunks).astype(np.int64)
        self.positions = np.concatenate([p + np.arange(c) for p, c in zip(self.prefixes, self.chunks)]).astype(np.int64)

    @property
    def slots(self):
        return self.pool.shape[2]

    def oracle_problem(self, rows=None):
        context = int((self.prefixes + self.chunks).max())
        mapping = orc.mapping_from_block_table(self.block_tables, self.block_size, context)
        sel = np.arange(self.rows) if rows is None else np.asarray(rows)
        return orc.Problem(self.query[sel], self.pool, self.requests[sel], self.positions[sel], mapping,
                           self.heads, self.kv_heads, self.head_dim, self.scale, self.softcap, self.window)
