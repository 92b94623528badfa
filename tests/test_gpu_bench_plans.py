"""The plans bench.py measures, checked: the config-1 projection set (bench.make_projection_set,
the bench's seeds) as bench.make_replica builds it -- one 144-segment K=896 plan and one
24-segment K=4864 plan writing 168 matrices' rows into one output -- against the oracle's
restatement of linearQ4 (quant.ts:95-111) for every matrix, at the BASELINE GEMV bar (1e-3
relative with a 1e-5 x rms floor). The reference checks its decode kernel the same way,
one shape at a time (matmul_q4.test.ts:198-214)."""

import os

import numpy as np
import pytest

import bench
import oracle
from conftest import assert_close, gemv_tolerance

pytestmark = pytest.mark.gpu


def test_bench_projection_plans_match_oracle(device):
    mats = bench.make_projection_set()
    assert len(mats) == bench.LAYERS * len(bench.PROJECTIONS)
    rows_total = sum(q.rows for _, q in mats)
    out = device.buffer(rows_total * 4)
    device.zero(out, rows_total * 4)
    rng = np.random.default_rng(7)
    x896 = rng.standard_normal(bench.HIDDEN, dtype=np.float32)
    x4864 = rng.standard_normal(bench.INTER, dtype=np.float32)
    bx896, bx4864 = device.upload(x896), device.upload(x4864)
    rep = bench.make_replica(device, mats, out)
    try:
        p896, p4864 = rep["plans"]
        p896.launch(bx896)
        p4864.launch(bx4864)
        got = device.read_array(out, np.float32, rows_total)
        threads = max(1, min(16, len(os.sched_getaffinity(0))))
        off = 0
        for i, (name, q) in enumerate(mats):
            x = x896 if q.cols == bench.HIDDEN else x4864
            oq = oracle.QuantizedMatrix(q.rows, q.cols, q.block_size, 4, oracle.ENC_SIGNED, q.packed, q.scales, None)
            want = oracle.gemv_threads(x, oq, None, threads)
            assert_close(got[off:off + q.rows], want, *gemv_tolerance(want),
                         label=f"layer {i // len(bench.PROJECTIONS)} {name} ({q.rows}x{q.cols})")
            off += q.rows
        assert off == rows_total
    finally:
        for p in rep["plans"]:
            p.destroy()
        for b in rep["bufs"] + [out, bx896, bx4864]:
            b.release()
