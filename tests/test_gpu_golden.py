"""The GPU path against vectors of the reference's own CPU references.

The C1 decode case and the d 64 prefill case of tests/golden/reference_vectors.npz
run through the C ABI (gk_paged_decode, gk_paged_prefill) and are compared with
the reference's direct_bf16_pv and tiled_bf16_pv outputs
(tests/paged_attention_reference.py:6-59) under the parity gate taken
literally: bf16 outputs within a flat max-abs 2e-2 and mean-abs 2e-3.
"""

import numpy as np
import pytest

from oracle import oracle as orc
from tests import paged_cases as cases
from tests.test_golden import GOLDEN, golden_long_case, golden_long_decode_case, golden_prefill_case

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as g:
        return {k: g[k] for k in g.files}


@pytest.fixture(scope="module")
def runner():
    import torch
    assert torch.cuda.is_available()
    from tests import gk_runner
    return gk_runner


def gate(name, actual, ref):
    assert np.isfinite(orc.bf16_to_f32(actual)).all()
    max_abs, mean_abs = orc.check_flat_gate(actual, ref, MAX_ABS, MEAN_ABS)
    print(f"{name}: max_abs={max_abs:.3e} mean_abs={mean_abs:.3e}", flush=True)


@pytest.mark.parametrize("partition", [0, 64])
def test_c1_decode_against_reference_vectors(runner, golden, partition):
    actual = runner.run_case(cases.c1_case(), partition=partition)
    for name in ("c1_direct", "c1_tiled_512", "c1_tiled_64"):
        gate(f"partition {partition} vs {name}", actual, golden[name])


def test_prefill_against_reference_vectors(runner, golden):
    actual = runner.run_prefill_case(golden_prefill_case())
    for name in ("prefill_direct", "prefill_tiled_512", "prefill_tiled_64"):
        gate(f"vs {name}", actual, golden[name])


def test_long_prefill_against_reference_vectors(runner, golden):
    actual = runner.run_prefill_case(golden_long_case())[golden["long_rows"]]
    for name in ("long_direct", "long_tiled_512"):
        gate(f"vs {name}", actual, golden[name])


@pytest.mark.parametrize("partition", [0, 2048])
def test_long_decode_against_reference_vectors(runner, golden, partition):
    actual = runner.run_case(golden_long_decode_case(), partition=partition)
    for name in ("decode_long_direct", "decode_long_tiled_512"):
        gate(f"partition {partition} vs {name}", actual, golden[name])
