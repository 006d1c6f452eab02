"""Seeded synthetic workloads of the benchmark configurations.

The benchmark workloads C1-C5 in block-table form: a bf16 head-major pool
[2, Hkv, S, d] filled with N(0, 1), query rows, seeded non-overlapping block
tables and seeded lengths. Generated on the GPU with a seeded torch generator.
"""

import math

import numpy as np


def permuted_block_tables(rng, lens, block_size, num_blocks, sets=1):
    """Seeded non-overlapping block ids: table[b, j] holds tokens [j*blk, (j+1)*blk) of sequence b.

    With sets > 1, returns a list of `sets` tables over disjoint blocks of the same
    pool (same lengths), so that consecutive benchmark steps read different memory.
    """
    need = [(int(n) + block_size - 1) // block_size for n in lens]
    total = sum(need)
    assert total * sets <= num_blocks, (total, sets, num_blocks)
    ids = rng.permutation(num_blocks)[:total * sets].astype(np.int32)
    max_blocks = max(need)
    tables = []
    cursor = 0
    for _ in range(sets):
        table = np.full((len(lens), max_blocks), -1, dtype=np.int32)
        for b, n in enumerate(need):
            table[b, :n] = ids[cursor:cursor + n]
            cursor += n
        tables.append(table)
    return tables[0] if sets == 1 else tables


def repage_tables(table, lens, block_size, page_size):
    """The same tokens as `table` (blocks of `block_size` tokens), as a table of
    pages of `page_size` tokens (a power of two dividing block_size): entry k of
    row b is the page holding token k * page_size, -1 past the row's length."""
    assert 0 < page_size <= block_size and block_size % page_size == 0
    pages = [(int(n) + page_size - 1) // page_size for n in lens]
    out = np.full((len(lens), max(pages)), -1, dtype=np.int32)
    for b, n in enumerate(pages):
        t = np.arange(n, dtype=np.int64) * page_size
        out[b, :n] = (table[b, t // block_size].astype(np.int64) * block_size + t % block_size) // page_size
    return out


# ---------------------------------------------------------------------------
# Full-size configurations (generated on the GPU; need torch + a device)
# ---------------------------------------------------------------------------

CONFIGS = {
    # name: (batch, heads, kv_heads, head_dim, block, pool_blocks, length sampler)
    "c2": (64, 32, 8, 128, 128, 4096, lambda rng, b: rng.integers(512, 4097, b)),
    "c3": (256, 32, 8, 128, 128, None, lambda rng, b: rng.integers(128, 2049, b)),
    "c5": (32, 64, 8, 128, 128, 8192,
           lambda rng, b: np.rint(np.exp(rng.uniform(math.log(1024), math.log(32768), b))).astype(np.int64)),
    # C2's batch, lengths, pool and KV bytes at GQA group 2 (16 q / 8 kv heads),
    # where most of the decode MFMA tile's 16 head columns are padding.
    "c2g2": (64, 16, 8, 128, 128, 4096, lambda rng, b: rng.integers(512, 4097, b)),
    # ... and at group 1 (8 q / 8 kv heads, multi-head attention).
    "c2g1": (64, 8, 8, 128, 128, 4096, lambda rng, b: rng.integers(512, 4097, b)),
    # ... and at group 3 (24 q / 8 kv heads), the largest group below a dense MFMA tile.
    "c2g3": (64, 24, 8, 128, 128, 4096, lambda rng, b: rng.integers(512, 4097, b)),
}


class DeviceDecodeCase:
    """A decode problem whose pool and queries live on the GPU (torch tensors)."""

    def __init__(self, name, seed=1234, device="cuda", table_sets=1):
        import torch

        batch, heads, kv_heads, d, block, pool_blocks, sampler = CONFIGS[name]
        rng = np.random.default_rng(seed)
        lens = np.asarray(sampler(rng, batch), dtype=np.int32)
        self.name = name
        self.store = name == "c3"
        # c3 attends len + 1 keys: the new token sits at position len.
        self.lens = lens + 1 if self.store else lens
        need = (self.lens.astype(np.int64) + block - 1) // block
        if pool_blocks is None:
            pool_blocks = int(need.sum()) * table_sets
        self.batch, self.heads, self.kv_heads, self.head_dim, self.block_size = batch, heads, kv_heads, d, block
        self.scale = float(np.float32(1 / math.sqrt(d)))
        tables = permuted_block_tables(rng, self.lens, block, pool_blocks, sets=table_sets)
        self.table_sets = tables if table_sets > 1 else [tables]
        self.tables = self.table_sets[0]
        self.slots = pool_blocks * block
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        self.pool = torch.empty((2, kv_heads, self.slots, d), dtype=torch.bfloat16, device=device)
        for kind in range(2):
            for h in range(kv_heads):
                self.pool[kind, h].normal_(generator=gen)
        self.query = torch.randn((batch, heads * d), generator=gen, device=device).to(torch.bfloat16)
        self.d_table_sets = [torch.from_numpy(t).to(device) for t in self.table_sets]
        self.d_tables = self.d_table_sets[0]
        self.d_lens = torch.from_numpy(self.lens).to(device)
        if self.store:
            pos = lens.astype(np.int64)
            self.slot_mappings = [(t[np.arange(batch), pos // block].astype(np.int64) * block + pos % block)
                                  for t in self.table_sets]
            self.slot_mapping = self.slot_mappings[0]
            self.d_slot_mappings = [torch.from_numpy(m.astype(np.int32)).to(device) for m in self.slot_mappings]
            self.d_slot_mapping = self.d_slot_mappings[0]
            self.new_key = torch.randn((batch, kv_heads * d), generator=gen, device=device).to(torch.bfloat16)
            self.new_value = torch.randn((batch, kv_heads * d), generator=gen, device=device).to(torch.bfloat16)
        self.out = torch.empty((batch, heads * d), dtype=torch.bfloat16, device=device)

    def kv_bytes(self):
        return int(self.lens.astype(np.int64).sum()) * self.kv_heads * self.head_dim * 2 * 2

    def step_bytes(self, page_size=None):
        """Algorithmic HBM bytes of one step: K/V rows read, Q read, O written, tables and lengths,
        plus the store's read and write of the new rows when the case stores. `page_size`: the
        table's page (default the case's block size)."""
        page = page_size or self.block_size
        b = self.kv_bytes()
        b += 2 * self.batch * self.heads * self.head_dim * 2
        b += int(((self.lens.astype(np.int64) + page - 1) // page).sum()) * 4 + 4 * self.batch
        if self.store:
            b += 2 * 2 * self.batch * self.kv_heads * self.head_dim * 2 + 4 * self.batch
        return b

    def host_arrays(self):
        """(query, pool) copied back as uint16 bf16 bits, after any store has run."""
        import torch

        pool = self.pool.view(torch.int16).cpu().numpy().view(np.uint16)
        query = self.query.view(torch.int16).cpu().numpy().view(np.uint16)
        return query, pool


class DevicePrefillCase:
    """Workload C4 on the GPU: prefix-shared chunked prefill.

    `seqs` sequences share a `prefix`-token prefix through identical block ids
    (the first prefix/block blocks of every table), each adds `chunk` causal
    query rows with blocks of its own. The pool already holds every key (as
    after the store), filled with bf16 N(0, 1).
    """

    def __init__(self, seqs=8, prefix=2048, chunk=512, heads=32, kv_heads=8, head_dim=128, block=128, seed=1234,
                 device="cuda"):
        import torch

        rng = np.random.default_rng(seed)
        self.seqs, self.prefix, self.chunk = seqs, prefix, chunk
        self.heads, self.kv_heads, self.head_dim, self.block_size = heads, kv_heads, head_dim, block
        shared = prefix // block
        own = (prefix + chunk + block - 1) // block - shared
        num_blocks = shared + seqs * own
        ids = rng.permutation(num_blocks).astype(np.int32)
        tables = np.empty((seqs, shared + own), dtype=np.int32)
        tables[:, :shared] = ids[:shared]
        for s in range(seqs):
            tables[s, shared:] = ids[shared + s * own:shared + (s + 1) * own]
        self.tables = tables
        self.slots = num_blocks * block
        self.rows = seqs * chunk
        self.scale = float(np.float32(1 / math.sqrt(head_dim)))
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        self.pool = torch.empty((2, kv_heads, self.slots, head_dim), dtype=torch.bfloat16, device=device)
        for kind in range(2):
            for h in range(kv_heads):
                self.pool[kind, h].normal_(generator=gen)
        self.query = torch.randn((self.rows, heads * head_dim), generator=gen, device=device).to(torch.bfloat16)
        self.out = torch.empty_like(self.query)
        i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(device)
        self.d_tables = i32(tables)
        self.seq_request = i32(np.arange(seqs))
        self.seq_first_row = i32(np.arange(seqs) * chunk)
        self.seq_rows = i32(np.full(seqs, chunk))
        self.seq_prefix = i32(np.full(seqs, prefix))

    def flops(self):
        """Causal-exact FLOPs: every visible (query, key) pair costs 4 d (Q.K and P.V)."""
        pairs = sum(self.prefix + i + 1 for i in range(self.chunk))
        return 4 * self.head_dim * self.heads * self.seqs * pairs
