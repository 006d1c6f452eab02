"""The compiled-path entry torch.ops.gaudirt._paged_attn_validated on the GPU.

The reference's compiled caller hands the attention its inputs as plain
tensors: the rows' slots, requests and positions, the plan tensor in the
`mapping` position and the header (src/bridge/segmented_runner.cpp:377-395,
596-601; python/gaudirt/partitioner.py:274-295 takes 12-14 positional
arguments), from PagedMetadata.forward_tensors
(tests/scheduler_metadata_async_smoke.py:36-44) or the metadata accessors
(tests/paged_tensor_metadata_smoke.py:31-35). Here that entry runs on real
kernels and must equal paged_attn bit for bit (output and KV pool), eagerly
and under torch.compile with the aot_eager backend (AOTAutograd
functionalization, no Inductor and no Triton).
"""

import math

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

HEADS, KV_HEADS, DIM = 32, 8, 128


@pytest.fixture(scope="module")
def torch_ext():
    import torch

    import gaudirt_amd

    assert torch.cuda.is_available()
    gaudirt_amd.load_extension()
    return torch


def bits(torch, t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def mixed_batch(torch, seed=11):
    """Host inputs of a serving step: chunked-prefill runs (prefill kernel) and
    single decode rows (decode kernel), 64-token pages."""
    rng = np.random.default_rng(seed)
    block = 64
    prefix = [0, 300, 77, 1000, 5]
    chunk = [24, 1, 1, 40, 1]
    lens = [p + c for p, c in zip(prefix, chunk)]
    blocks = [(n + block - 1) // block for n in lens]
    ids = rng.permutation(sum(blocks) + 3)
    context = max(lens)
    mapping = np.full((len(lens), context), -1, dtype=np.int32)
    cursor = 0
    for r, n in enumerate(lens):
        for t in range(n):
            mapping[r, t] = ids[cursor + t // block] * block + t % block
        cursor += blocks[r]
    slots = (sum(blocks) + 3) * block
    req = np.concatenate([np.full(c, r) for r, c in enumerate(chunk)]).astype(np.int64)
    pos = np.concatenate([p + np.arange(c) for p, c in zip(prefix, chunk)]).astype(np.int64)
    loc = mapping[req, pos].astype(np.int64)
    gen = torch.Generator().manual_seed(seed)
    rows = len(req)
    q = torch.randn(rows, HEADS * DIM, generator=gen).to(torch.bfloat16)
    k = torch.randn(rows, KV_HEADS * DIM, generator=gen).to(torch.bfloat16)
    v = torch.randn(rows, KV_HEADS * DIM, generator=gen).to(torch.bfloat16)
    base = torch.randn(2, KV_HEADS, slots, DIM, generator=gen).to(torch.bfloat16)
    return dict(mapping=mapping, slots=slots, req=req, pos=pos, loc=loc, prefix=prefix, chunk=chunk, q=q, k=k, v=v,
                base=base)


def pool_from(torch, base):
    import gaudirt_amd

    pool = gaudirt_amd.allocate_paged_kv(1, base.shape[2], KV_HEADS, DIM)
    pool[0].copy_(base.cuda())
    return pool


def eager_reference(torch, data, meta):
    """paged_attn on a fresh pool: (output bits, pool bits)."""
    import gaudirt_amd

    pool = pool_from(torch, data["base"])
    kp, vp = gaudirt_amd.kv_pool_views(pool, 0)
    scale = float(np.float32(1 / math.sqrt(DIM)))
    out = torch.ops.gaudirt.paged_attn.default(data["q"].cuda(), data["k"].cuda(), data["v"].cuda(), kp, vp, meta,
                                               DIM, scale)
    torch.cuda.synchronize()
    return bits(torch, out), bits(torch, pool)


def test_validated_entry_with_plan_tensor(torch_ext):
    import gaudirt_amd

    torch = torch_ext
    data = mixed_batch(torch)
    meta = torch.classes.gaudirt.PagedMetadata(torch.from_numpy(data["loc"]), torch.from_numpy(data["req"]),
                                               torch.from_numpy(data["pos"]), torch.from_numpy(data["mapping"]),
                                               data["slots"])
    want_out, want_pool = eager_reference(torch, data, meta)
    pool = pool_from(torch, data["base"])
    kp, vp = gaudirt_amd.kv_pool_views(pool, 0)
    scale = float(np.float32(1 / math.sqrt(DIM)))
    out = torch.ops.gaudirt._paged_attn_validated.default(
        data["q"].cuda(), data["k"].cuda(), data["v"].cuda(), kp, vp, meta.row_locations(), meta.row_requests(),
        meta.rotary_positions(), meta.attention_plan(HEADS, KV_HEADS, DIM), meta.rotary_header(), DIM, scale)
    torch.cuda.synchronize()
    assert np.array_equal(bits(torch, out), want_out)
    assert np.array_equal(bits(torch, pool), want_pool)
    # and the result is the reference's within the output gate
    problem = orc.Problem(bits(torch, data["q"]), want_pool[0], data["req"], data["pos"], data["mapping"], HEADS,
                          KV_HEADS, DIM, scale)
    print("validated entry", orc.check_tolerance(want_out, orc.direct_bf16_pv(problem)), flush=True)


def device_metadata(torch, data):
    """from_device_with_tokens metadata of the batch (device inputs, token IDs)."""
    batch = len(data["chunk"])
    tokens = torch.arange(len(data["req"]), dtype=torch.int64).cuda() * 7 % 1000
    return torch.classes.gaudirt.PagedMetadata.from_device_with_tokens(
        torch.from_numpy(data["loc"]).cuda(), torch.arange(batch, dtype=torch.int64).cuda(),
        torch.from_numpy(data["pos"]).cuda(), torch.from_numpy(data["mapping"]).cuda(), list(data["prefix"]),
        list(data["chunk"]), data["slots"], tokens, 1000)


def test_validated_entry_with_forward_tensors(torch_ext):
    import gaudirt_amd

    torch = torch_ext
    data = mixed_batch(torch, seed=12)
    meta = device_metadata(torch, data)
    want_out, want_pool = eager_reference(torch, data, meta)
    tokens, last, positions, header, locations, requests, plan, context = meta.forward_tensors(HEADS, KV_HEADS, DIM)
    assert context == meta.context() and plan.data_ptr() == meta.attention_plan(HEADS, KV_HEADS, DIM).data_ptr()
    pool = pool_from(torch, data["base"])
    kp, vp = gaudirt_amd.kv_pool_views(pool, 0)
    scale = float(np.float32(1 / math.sqrt(DIM)))
    out = torch.ops.gaudirt._paged_attn_validated.default(data["q"].cuda(), data["k"].cuda(), data["v"].cuda(), kp,
                                                          vp, locations, requests, positions, plan, header, DIM, scale)
    torch.cuda.synchronize()
    assert np.array_equal(bits(torch, out), want_out)
    assert np.array_equal(bits(torch, pool), want_pool)
    del tokens, last


def test_validated_entry_under_torch_compile(torch_ext):
    """torch.compile(backend="aot_eager") of a layer's attention call: AOTAutograd
    functionalizes the in-place KV store (clones the pool's one base, runs the
    op on views of the clone, copies back). Output and pool equal eager, on the
    first (compiling) call and on a second call with new inputs."""
    import gaudirt_amd

    torch = torch_ext
    scale = float(np.float32(1 / math.sqrt(DIM)))

    def layer(q, k, v, pool, locations, requests, positions, plan, header):
        key_pool, value_pool = pool[0, 0].transpose(0, 1), pool[0, 1].transpose(0, 1)
        return torch.ops.gaudirt._paged_attn_validated(q, k, v, key_pool, value_pool, locations, requests, positions,
                                                       plan, header, DIM, scale)

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    for seed in (13, 14):
        data = mixed_batch(torch, seed=seed)
        meta = torch.classes.gaudirt.PagedMetadata(torch.from_numpy(data["loc"]), torch.from_numpy(data["req"]),
                                                   torch.from_numpy(data["pos"]), torch.from_numpy(data["mapping"]),
                                                   data["slots"])
        want_out, want_pool = eager_reference(torch, data, meta)
        pool = pool_from(torch, data["base"])
        out = compiled(data["q"].cuda(), data["k"].cuda(), data["v"].cuda(), pool, meta.row_locations(),
                       meta.row_requests(), meta.rotary_positions(), meta.attention_plan(HEADS, KV_HEADS, DIM),
                       meta.rotary_header())
        torch.cuda.synchronize()
        assert np.array_equal(bits(torch, out), want_out), seed
        assert np.array_equal(bits(torch, pool), want_pool), seed
        print("compiled call", seed, "equals eager", flush=True)
    del gaudirt_amd


def test_dispatch_smoke_tensors_outlive_their_metadata(torch_ext):
    """tests/paged_attention_dispatch_smoke.py: single decode rows at positions
    18, 254, 255, 511 and 18 again (56 q / 8 kv heads, head_dim 128, one request
    whose token t sits at slot t + 1 of a 1026-slot pool), each through
    _paged_attn_validated after the PagedMetadata object that produced the
    tensors has been deleted and collected: the slots, requests, positions,
    plan and header keep their storage, and every step matches the oracle on
    the pool as stored. The smoke hands the request map where the plan goes;
    the reference's plan check (src/bridge/attention_plan.cpp:132-140) rejects
    such a tensor, and so does this op, with the same message and before any KV
    write."""
    import gc

    import gaudirt_amd

    torch = torch_ext
    heads, kv_heads, dim, context = 56, 8, 128, 1024
    slots = context + 2
    gen = torch.Generator().manual_seed(1907)
    mapping = torch.arange(1, context + 1, dtype=torch.int32).view(1, context)
    pool = gaudirt_amd.allocate_paged_kv(1, slots, kv_heads, dim)
    key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, 0)
    query = torch.randn((1, heads * dim), generator=gen).to(torch.bfloat16).cuda()
    key = torch.randn((1, kv_heads * dim), generator=gen).to(torch.bfloat16).cuda()
    value = torch.randn((1, kv_heads * dim), generator=gen).to(torch.bfloat16).cuda()
    scale = float(np.float32(1 / math.sqrt(dim)))
    op = torch.ops.gaudirt._paged_attn_validated.default
    for position in (18, 254, 255, 511, 18):
        meta = torch.classes.gaudirt.PagedMetadata(torch.tensor([position + 1]), torch.tensor([0]),
                                                   torch.tensor([position]), mapping, slots)
        locations, requests, positions = meta.row_locations(), meta.row_requests(), meta.rotary_positions()
        plan, header = meta.attention_plan(heads, kv_heads, dim), meta.rotary_header()
        request_map = meta.request_mapping()
        del meta
        gc.collect()
        before = bits(torch, pool)
        with pytest.raises(RuntimeError, match="invalid or expired metadata plan"):
            op(query, key, value, key_pool, value_pool, locations, requests, positions, request_map, header, dim,
               scale)
        torch.cuda.synchronize()
        assert np.array_equal(bits(torch, pool), before)
        out = op(query, key, value, key_pool, value_pool, locations, requests, positions, plan, header, dim, scale)
        torch.cuda.synchronize()
        stored = bits(torch, pool)[0]
        problem = orc.Problem(bits(torch, query), stored, np.array([0]), np.array([position]), mapping.numpy(), heads,
                              kv_heads, dim, scale)
        max_abs, mean_abs = orc.check_flat_gate(bits(torch, out), orc.direct_bf16_pv(problem))
        print("position", position, f"max_abs={max_abs:.3e} mean_abs={mean_abs:.3e}", flush=True)
