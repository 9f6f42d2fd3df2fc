"""bench.py's continuity line with the reference bench, on the CPU: the inputs
of examples/iq2_matmul_bench.rs:251-273 for every format, and the nearest-rank
percentile of its summarize() (examples/iq2_matmul_bench.rs:238-250)."""

import importlib.util
import math
import os

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_workloads_under_test",
                                                  os.path.join(REPO, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
@pytest.mark.parametrize("dims", [(1, 4096, 4096), (2, 7, 320), (3, 300, 1001)])
def test_reference_bench_inputs(inputs, oracle, variant, dims):
    m, n, k = dims
    x, wb, ws = inputs.reference_bench_case_variant(variant, m, n, k)
    nb = n * -(-k // 256)
    # the block sizes come from the oracle's own format tables here, not from
    # the table the helper uses
    bpb, spb = oracle.bytes_per_block(variant), oracle.scales_per_block(variant)
    assert wb.shape == (nb * bpb,) and ws.shape == (nb * spb,) and x.shape == (m, k)
    want_wb = oracle.lcg_fill(nb * bpb, 0xA11CE5ED ^ n)
    want_wb[-1] = 0x5A
    assert np.array_equal(wb, want_wb)
    # every block's d is f16 1.0 (bytes 00 3c); the other scale bytes are the LCG's
    sv = ws.reshape(nb, spb)
    assert (sv[:, 0] == 0x00).all() and (sv[:, 1] == 0x3C).all()
    lcg = oracle.lcg_fill(nb * spb, 0xC0FFEE12 ^ k).reshape(nb, spb)
    assert np.array_equal(sv[:, 2:], lcg[:, 2:])
    # the crate's deterministic activations: ((17 i mod 41) - 20) / 13
    i = np.arange(m * k)
    assert np.array_equal(x.reshape(-1), (((17 * i) % 41) - 20.0).astype(np.float32) / 13)


def test_iq2xxs_bench_inputs_match_the_one_format_helper(inputs):
    a = inputs.reference_bench_case_variant(0, 2, 96, 768)
    b = inputs.reference_bench_case(2, 96, 768)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


def test_nearest_rank_percentile(bench):
    vals = sorted([5.0, 1.0, 4.0, 2.0, 3.0])
    # rank ceil(p n), 1-based: p50 of 5 values is the 3rd, p95 the 5th
    assert bench.nearest_rank(vals, 0.50) == 3.0
    assert bench.nearest_rank(vals, 0.95) == 5.0
    twenty = [float(v) for v in range(1, 21)]
    assert bench.nearest_rank(twenty, 0.95) == 19.0  # ceil(19.0) = 19
    assert bench.nearest_rank(twenty, 0.50) == 10.0
    assert bench.nearest_rank([7.0], 0.95) == 7.0
    for n in (1, 2, 10, 20, 21):
        v = list(range(n))
        assert bench.nearest_rank(v, 0.95) == v[max(1, math.ceil(0.95 * n)) - 1]
