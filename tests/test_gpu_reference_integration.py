"""GPU ports of the reference's integration smokes of the op path.

- tests/paged_fused_integration_smoke.py: one decode row at prefix 143 and a
  137-row causal prefill from position 0, int32 metadata, the request map
  arange(context) % (slots - 1) + 1, over the geometries its environment
  selects (4/2, 56/8 heads at head_dim 128; 4/2 at 64), and 16/8 heads at
  head_dim 256;
- tests/paged_tiled_integration_smoke.py: 7- and 137-row chunks on a 512-token
  prefix with the new keys as an unaligned column view, for 1 and 256 requests
  sharing the map;
- tests/paged_attention_no_fallback_smoke.py: the three shapes that reference
  rejects (3 rows on a 32-token context; one row at 4095 of 4096 and at 4607
  of 4608, 56/8 heads) run here and match the oracle.

Each case audits the whole KV pool bit for bit against the oracle's store and
gates the output against direct_bf16_pv (max-abs 2e-2, mean-abs 2e-3) and the
reference's relative-L2 gates (isolated_errors against the fp64 truth and
tiled_bf16_pv). The smokes' recipe-cache counters have no counterpart here.
"""

import math

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_ext():
    import torch

    import gaudirt_amd

    assert torch.cuda.is_available()
    gaudirt_amd.load_extension()
    return torch


def bits(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def run(torch, heads, kv_heads, dim, slots, mapping, requests, positions, seed, base_seed, unaligned_key=False):
    import gaudirt_amd

    rows = len(positions)
    gen = torch.Generator().manual_seed(seed)
    query = torch.randn(rows, heads * dim, generator=gen).to(torch.bfloat16)
    key = torch.randn(rows, kv_heads * dim, generator=gen).to(torch.bfloat16)
    value = torch.randn(rows, kv_heads * dim, generator=gen).to(torch.bfloat16)
    key_base = torch.randn(slots, kv_heads, dim, generator=torch.Generator().manual_seed(base_seed)).to(torch.bfloat16)
    value_base = torch.randn(slots, kv_heads, dim,
                             generator=torch.Generator().manual_seed(base_seed + 1)).to(torch.bfloat16)
    locations = mapping[requests.long(), positions.long()].contiguous()
    meta = torch.classes.gaudirt.PagedMetadata(locations, requests, positions, mapping, slots)
    pool = gaudirt_amd.allocate_paged_kv(1, slots, kv_heads, dim)
    key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, 0)
    key_pool.copy_(key_base.cuda())
    value_pool.copy_(value_base.cuda())
    if unaligned_key:
        storage = torch.empty((rows, kv_heads * dim + 1), dtype=torch.bfloat16, device="cuda")
        k = storage[:, 1:]
        k.copy_(key)
    else:
        k = key.cuda()
    scale = float(np.float32(1 / math.sqrt(dim)))
    out = torch.ops.gaudirt.paged_attn.default(query.cuda(), k, value.cuda(), key_pool, value_pool, meta, dim, scale)
    torch.cuda.synchronize()
    expected = np.stack([bits(key_base), bits(value_base)]).transpose(0, 2, 1, 3).copy()  # [2, Hkv, S, d]
    orc.kv_store(bits(key), bits(value), locations.numpy(), rows, expected, slots, kv_heads, dim)
    actual_pool = np.stack([bits(key_pool.transpose(0, 1)), bits(value_pool.transpose(0, 1))])
    assert np.array_equal(actual_pool, expected), "KV pool differs from the oracle store"
    problem = orc.Problem(bits(query), expected, requests.numpy().astype(np.int64),
                          positions.numpy().astype(np.int64), mapping.numpy(), heads, kv_heads, dim, scale)
    actual = bits(out)
    assert np.isfinite(orc.bf16_to_f32(actual)).all()
    max_abs, mean_abs = orc.check_flat_gate(actual, orc.direct_bf16_pv(problem))
    tiled = orc.tiled_bf16_pv(problem, 512)
    errors = orc.isolated_errors(orc.bf16_to_f32(actual), orc.fp64_bf16(problem), orc.bf16_to_f32(tiled))
    return max_abs, mean_abs, errors


# The smoke's geometries, plus head_dim 256 (16 q / 8 kv heads), which the
# reference also accepts and whose 137-row chunk runs the head_dim 256 MFMA
# prefill through the op.
@pytest.mark.parametrize("heads,kv_heads,dim", [(4, 2, 128), (56, 8, 128), (4, 2, 64), (16, 8, 256)])
@pytest.mark.parametrize("case,rows,prefix", [("decode", 1, 143), ("prefill", 137, 0)])
def test_fused_integration(torch_ext, heads, kv_heads, dim, case, rows, prefix):
    torch = torch_ext
    slots, context = 512, 256
    mapping = (torch.arange(context, dtype=torch.int32) % (slots - 1) + 1).reshape(1, -1)
    positions = torch.arange(prefix, prefix + rows, dtype=torch.int32)
    requests = torch.zeros(rows, dtype=torch.int32)
    result = run(torch, heads, kv_heads, dim, slots, mapping, requests, positions, 900 + rows, 512)
    print(case, heads, kv_heads, dim, "max/mean abs, relative l2", result, flush=True)


@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (56, 8)])
@pytest.mark.parametrize("request_count", [1, 256])
@pytest.mark.parametrize("rows", [7, 137])
def test_tiled_integration(torch_ext, heads, kv_heads, request_count, rows):
    torch = torch_ext
    slots, context, prefix, dim = 2048, 1024, 512, 128
    mapping = (torch.arange(context, dtype=torch.int32) % (slots - 1) + 1).reshape(1, -1).repeat(request_count, 1)
    positions = torch.arange(prefix, prefix + rows, dtype=torch.int32)
    requests = torch.zeros(rows, dtype=torch.int32)
    result = run(torch, heads, kv_heads, dim, slots, mapping, requests, positions, 3000 + rows, 520,
                 unaligned_key=True)
    print("tiled extend", rows, "requests", request_count, "max/mean abs, relative l2", result, flush=True)


@pytest.mark.parametrize("rows,context,positions", [(3, 32, [0, 1, 2]), (1, 4096, [4095]), (1, 4608, [4607])])
def test_shapes_the_reference_rejects_run_here(torch_ext, rows, context, positions):
    torch = torch_ext
    slots = context + 1
    mapping = torch.arange(1, slots, dtype=torch.int32).reshape(1, context)
    requests = torch.zeros(rows, dtype=torch.int64)
    result = run(torch, 56, 8, 128, slots, mapping, requests, torch.tensor(positions, dtype=torch.int64),
                 77 + context, 600)
    print("rows", rows, "context", context, "max/mean abs, relative l2", result, flush=True)
