"""128 chained decode steps against the CPU oracle, with a full KV-pool audit per step.

Follows tests/paged_attention_128_state_smoke.py:18-60 (56 q / 8 kv heads,
head_dim 128, N(0, 0.125) data, a cached prefix of 0 or 512 tokens, 128 steps
of store-then-attend, every step against the references and the pool against
the expected store) with four requests of staggered lengths decoding together.
The step state lives on the device as a serving loop keeps it: each step's
positions are the sequence lengths that _advance_decode_lengths produced in
the previous step, the slots are looked up from the device request map, and
the metadata is scheduler-owned (PagedMetadata._from_scheduler, no host
wait). Checked per step: the pool bit for bit against the oracle's store, the
output within max-abs 2e-2 / mean-abs 2e-3 of direct_bf16_pv and the
relative-L2 gates against fp64 and tiled_bf16_pv, and the advanced lengths.
"""

import math

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

HEADS, KV_HEADS, DIM, STEPS, REQUESTS = 56, 8, 128, 128, 4


@pytest.fixture(scope="module")
def torch_ext():
    import torch

    import gaudirt_amd

    assert torch.cuda.is_available()
    gaudirt_amd.load_extension()
    return torch


def bits(torch, t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.timeout(300)
@pytest.mark.parametrize("prefix", [0, 512])
def test_128_chained_decode_steps(torch_ext, prefix):
    import gaudirt_amd

    torch = torch_ext
    rng = np.random.default_rng(8721 + prefix)
    starts = np.array([prefix + 13 * r for r in range(REQUESTS)], dtype=np.int64)  # cached tokens per request
    context = int(starts.max()) + STEPS
    # Request r's token t at slot 1 + r * context + t (slot 0 stays unused, as in the reference test).
    slots = 1 + REQUESTS * context
    mapping = (1 + np.arange(REQUESTS * context, dtype=np.int32)).reshape(REQUESTS, context)

    def small(shape):
        return orc.bf16_from_f32((0.125 * rng.standard_normal(shape)).astype(np.float32))

    expected = np.zeros((2, KV_HEADS, slots, DIM), dtype=np.uint16)
    for r in range(REQUESTS):
        cached = mapping[r, :starts[r]]
        expected[:, :, cached, :] = small((2, KV_HEADS, len(cached), DIM))
    queries = small((STEPS, REQUESTS, HEADS * DIM))
    keys = small((STEPS, REQUESTS, KV_HEADS * DIM))
    values = small((STEPS, REQUESTS, KV_HEADS * DIM))

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()

    pool = gaudirt_amd.allocate_paged_kv(1, slots, KV_HEADS, DIM)
    pool[0].copy_(dev(expected))
    key_pool, value_pool = gaudirt_amd.kv_pool_views(pool, 0)
    mapping_dev = torch.from_numpy(mapping).cuda()
    requests_dev = torch.arange(REQUESTS, dtype=torch.int64).cuda()
    seq_lens = torch.from_numpy(starts).cuda()                      # int64: next position per request
    orig_lens = torch.from_numpy(starts.astype(np.int32)).cuda()    # int32 twin
    scale = float(np.float32(1 / math.sqrt(DIM)))
    worst = [0.0, 0.0, 0.0, 0.0]
    for step in range(STEPS):
        positions = seq_lens
        locations = mapping_dev[requests_dev, positions]
        host_positions = (starts + step).tolist()
        meta = torch.classes.gaudirt.PagedMetadata._from_scheduler(locations, requests_dev, positions, mapping_dev,
                                                                    host_positions, [1] * REQUESTS, slots, None, 0)
        out = torch.ops.gaudirt.paged_attn.default(dev(queries[step]), dev(keys[step]), dev(values[step]), key_pool,
                                                   value_pool, meta, DIM, scale)
        seq_lens, orig_lens = torch.ops.gaudirt._advance_decode_lengths(seq_lens, orig_lens)
        torch.cuda.synchronize()
        pos = starts + step
        orc.kv_store(keys[step], values[step], mapping[np.arange(REQUESTS), pos].astype(np.int64), REQUESTS, expected,
                     slots, KV_HEADS, DIM)
        assert np.array_equal(bits(torch, pool[0]), expected), f"KV pool differs from the oracle after step {step}"
        assert seq_lens.cpu().tolist() == (pos + 1).tolist() and orig_lens.cpu().tolist() == (pos + 1).tolist()
        problem = orc.Problem(queries[step], expected, np.arange(REQUESTS), pos, mapping, HEADS, KV_HEADS, DIM, scale)
        actual = bits(torch, out)
        assert np.isfinite(orc.bf16_to_f32(actual)).all()
        max_abs, mean_abs = orc.check_tolerance(actual, orc.direct_bf16_pv(problem), 2e-2, 2e-3)
        e64, etiled = orc.isolated_errors(orc.bf16_to_f32(actual), orc.fp64_bf16(problem),
                                          orc.bf16_to_f32(orc.tiled_bf16_pv(problem, 512)))
        worst = [max(a, b) for a, b in zip(worst, (max_abs, mean_abs, e64, etiled))]
    print(f"128 chained steps, prefix {prefix}: worst max_abs={worst[0]:.3e} mean_abs={worst[1]:.3e} "
          f"fp64_rel_l2={worst[2]:.3e} tiled_rel_l2={worst[3]:.3e}; pool bit-exact after every step", flush=True)
