"""Decode GEMV, LM head and argmax on the GPU against the CPU oracle, through the C ABI.

Cases follow the reference's own kernel tests (test/kernels/matmul_q4.test.ts:198-231,
forward_ops.test.ts:397-446) and the BASELINE configs 0-2.
"""

import functools
import json
import os

import numpy as np
import pytest

import oracle
from conftest import FP32_TOLERANCE, assert_close, gemv_tolerance
from enargeia_amd import kernels as K

pytestmark = pytest.mark.gpu


def _upload_quant(device, q):
    bufs = [device.upload(q.packed), device.upload(q.scales)]
    bufs.append(device.upload(q.zeros) if q.zeros is not None else None)
    return bufs


def run_decode(device, x, q, bias, out_len=None, out_offset=0):
    spec = K.with_format(K.MATMUL_Q4_DECODE, q.bits, q.encoding)
    kern = K.ComputeKernel(device, spec)
    n_out = out_len if out_len is not None else q.rows + out_offset
    bx = device.upload(x)
    bp, bs, bz = _upload_quant(device, q)
    bb = device.upload(bias if bias is not None else np.zeros(max(1, q.rows), np.float32))
    bo = device.buffer(n_out * 4)
    device.zero(bo, n_out * 4)
    u = kern.uniform()
    u.write(K.matmul_q4_dims(1, q.rows, q.cols, bias is not None, q.block_size, q.rows, out_offset))
    kern.encode(kern.bind_group([bx, bp, bs, bz, bb, bo, u]), K.matmul_q4_decode_workgroups(q.rows))
    y = device.read_array(bo, np.float32, n_out)
    for b in (bx, bp, bs, bz, bb, bo):
        if b is not None:
            b.release()
    return y


@pytest.mark.parametrize("n", [896, 128, 4864])
def test_decode_matches_reference_single_row(device, n):
    # matmul_q4.test.ts:198-214: k=896, seeds 41/42/43, reference asymmetric block-64 format.
    k = 896
    x = oracle.random_floats(k, 41)
    q = oracle.quantize_q4_ref(oracle.random_floats(n * k, 42), n, k)
    bias = oracle.random_floats(n, 43)
    got = run_decode(device, x, q, bias)
    assert_close(got, oracle.linear_q(x, q, bias, 1), *FP32_TOLERANCE, label=f"q4 decode n={n}")


def test_decode_matches_javascript_golden(device):
    with open(os.path.join(os.path.dirname(__file__), "golden", "js_vectors.json")) as f:
        case = next(c for c in json.load(f)["linear"] if c["name"] == "decode_n128_k896")
    n, k = case["n"], case["k"]
    x = oracle.random_floats(k, case["x_seed"])
    q = oracle.quantize_q4_ref(oracle.random_floats(n * k, case["w_seed"]), n, k)
    got = run_decode(device, x, q, oracle.random_floats(n, case["bias_seed"]))
    expect = np.array(case["out"], dtype=np.uint32).view(np.float32)
    assert_close(got, expect, *FP32_TOLERANCE, label="decode vs JS")


@functools.lru_cache(maxsize=None)
def sym_weights(n, k, seed, group=32, bits=4):
    w = oracle.normal_floats(n * k, seed, 0.02)
    return oracle.quantize_sym(w, n, k, bits, group)


# BASELINE config 0 and the config-1 projection shapes (symmetric int4, group 32).
@pytest.mark.parametrize("n,k", [(896, 896), (128, 896), (4864, 896), (896, 4864)])
def test_decode_baseline_projection_shapes(device, n, k):
    x = oracle.normal_floats(k, 0x5EED ^ 1, 1.0)
    q = sym_weights(n, k, 0x5EED ^ (n * 7 + k))
    got = run_decode(device, x, q, None)
    expect = oracle.linear_q(x, q, None, 1)
    assert_close(got, expect, *gemv_tolerance(expect), label=f"sym int4 {n}x{k}")


def test_decode_long_reduction_reference_format(device):
    n, k = 256, 4864
    x = oracle.random_floats(k, 5)
    q = oracle.quantize_q4_ref(oracle.random_floats(n * k, 6), n, k)
    got = run_decode(device, x, q, None)
    assert_close(got, oracle.linear_q(x, q, None, 1), *FP32_TOLERANCE, label="q4 decode k=4864")


def test_decode_writes_at_out_offset_and_skips_bias(device):
    # matmul_q4.test.ts:181-195, through the decode kernel (outOffset; index 0 untouched).
    k = 64
    q = oracle.quantize_q4_ref(np.full(2 * k, 0.5, np.float32), 2, k)
    got = run_decode(device, np.ones(k, np.float32), q, None, out_len=6, out_offset=4)
    assert got[0] == 0 and got[1] == 0
    assert abs(got[4] - 32) < 1e-3 and abs(got[5] - 32) < 1e-3


@pytest.mark.parametrize("n,k,bs", [(5, 64, 64), (3, 40, 8), (7, 96, 32), (33, 192, 64)])
def test_decode_ragged_and_unchunked_shapes(device, n, k, bs):
    # Shapes the 16-byte-chunk kernel does not take go through the per-element path.
    x = oracle.random_floats(k, 31)
    q = oracle.quantize_q4_ref(oracle.random_floats(n * k, 32), n, k, bs)
    got = run_decode(device, x, q, None)
    assert_close(got, oracle.linear_q(x, q, None, 1), *FP32_TOLERANCE, label=f"ragged {n}x{k}/{bs}")


def test_decode_int8_offset_format(device):
    n, k = 512, 896
    x = oracle.random_floats(k, 9)
    q = oracle.quantize_blocks_n(oracle.random_floats(n * k, 10), n, k, 8)
    got = run_decode(device, x, q, None)
    assert_close(got, oracle.linear_q(x, q, None, 1), *FP32_TOLERANCE, label="int8 decode")


def test_decode_is_deterministic(device):
    # test/helpers/determinism.ts: repeated runs into separate buffers compare bitwise.
    n, k = 4864, 896
    x = oracle.normal_floats(k, 3, 1.0)
    q = sym_weights(n, k, 77)
    first = run_decode(device, x, q, None)
    for _ in range(5):
        assert np.array_equal(run_decode(device, x, q, None).view(np.uint32), first.view(np.uint32))


def test_decode_rejects_bad_dims(device):
    kern = K.ComputeKernel(device, K.MATMUL_Q4_DECODE)
    bufs = [device.buffer(4096) for _ in range(6)]
    u = kern.uniform()
    u.write(K.matmul_q4_dims(1, 8, 100, False, 64))  # 100 is not a multiple of 64
    with pytest.raises(K.EgError, match="not a multiple of 64"):
        kern.encode(kern.bind_group([*bufs, u]), (8, 1, 1))
    for b in bufs:
        b.release()


# ---- LM head --------------------------------------------------------------------------------


@functools.lru_cache(maxsize=None)
def lm_head_config2():
    vocab, hidden = 151936, 896
    table = oracle.normal_floats(vocab * hidden, 0x5EED ^ 0x100, 0.02)
    q = oracle.quantize_sym(table, vocab, hidden, 8, hidden)
    del table
    h = oracle.normal_floats(hidden, 0x5EED ^ 0x101, 1.0)
    logits = oracle.linear_q(h, q, None, 1)
    return q, h, logits


def _run_head(device, q, h, fused, out_offset=0):
    bh = device.upload(h)
    bp, bs, bz = _upload_quant(device, q)
    n = q.rows
    bo = device.buffer((n + out_offset) * 4)
    device.zero(bo, (n + out_offset) * 4)
    dims = K.embedding_dims(1, q.cols, 0, n, q.block_size, n, out_offset)
    res = None
    if fused:
        br = device.buffer(8)
        K.lm_head_argmax(device, bh, bp, bs, bz, bo, br, dims, q.bits, q.encoding)
        res = device.read_array(br, np.uint32, 2)
        br.release()
    else:
        spec = K.embedding_head_spec("q8" if q.bits == 8 else "q4", q.encoding)
        kern = K.ComputeKernel(device, spec)
        u = kern.uniform()
        u.write(dims)
        kern.encode(kern.bind_group([bh, bp, bs, bz, bo, u]), K.embedding_head_workgroups(n))
    logits = device.read_array(bo, np.float32, n + out_offset)
    for b in (bh, bp, bs, bz, bo):
        if b is not None:
            b.release()
    return logits, res


def test_lm_head_q8_config2_logits_and_fused_argmax(device):
    q, h, expect = lm_head_config2()
    logits, _ = _run_head(device, q, h, fused=False)
    assert_close(logits, expect, *gemv_tolerance(expect), label="lm_head_q8 config 2")
    fused_logits, res = _run_head(device, q, h, fused=True)
    assert np.array_equal(fused_logits.view(np.uint32), logits.view(np.uint32))
    top2 = np.sort(expect)[-2:]
    # Bit-exact argmax index whenever the top-2 gap is beyond the GEMV tolerance.
    assert top2[1] - top2[0] > 1e-3 * abs(top2[1])
    assert res[0] == oracle.argmax(expect)
    assert res[0] == oracle.argmax(logits)
    assert res[1] == logits[res[0]].view(np.uint32)


@pytest.mark.parametrize("r1,r2", [(37, 39000), (20000, 20001), (5, 38000)])
def test_lm_head_fused_argmax_across_workgroups_and_calls(device, r1, r2):
    # The fused argmax leaves one (value, index) partial per workgroup, which a finalize launch
    # reduces in a fixed order: consecutive calls on one context each reduce every workgroup's
    # partial, and two equal maxima in rows far apart (different workgroups) resolve to the lower
    # index, as the reference's argmax does (test/reference/ops.ts:237-244: the first maximum kept).
    rows, hidden = 40000, 896
    h = oracle.normal_floats(hidden, 0x5EED ^ r1, 1.0)
    t = oracle.normal_floats(rows * hidden, 0x5EED ^ r2, 0.02).reshape(rows, hidden).copy()
    t[r1] = t[r2] = 0.05 * np.sign(h)  # the same codes and scale: bit-identical logits, the largest
    q = oracle.quantize_sym(t.ravel(), rows, hidden, 8, hidden)
    for _ in range(2):
        logits, res = _run_head(device, q, h, fused=True)
        assert logits[r1].view(np.uint32) == logits[r2].view(np.uint32)
        assert res[0] == min(r1, r2) == int(np.argmax(logits))
        assert res[1] == logits[res[0]].view(np.uint32)


def test_lm_head_q8_reference_format_with_offset(device):
    rows, hidden = 4096, 896
    q = oracle.quantize_blocks_n(oracle.random_floats(rows * hidden, 61), rows, hidden, 8)
    h = oracle.random_floats(hidden, 62)
    logits, res = _run_head(device, q, h, fused=True, out_offset=1000)
    expect = oracle.linear_q(h, q, None, 1)
    assert np.all(logits[:1000] == 0)
    assert_close(logits[1000:], expect, *FP32_TOLERANCE, label="lm_head_q8 reference format")
    assert res[0] == 1000 + oracle.argmax(expect)


def test_lm_head_q4(device):
    rows, hidden = 3000, 896
    q = oracle.quantize_q4_ref(oracle.random_floats(rows * hidden, 71), rows, hidden)
    h = oracle.random_floats(hidden, 72)
    logits, _ = _run_head(device, q, h, fused=False)
    assert_close(logits, oracle.linear_q(h, q, None, 1), *FP32_TOLERANCE, label="lm_head_q4")


# ---- argmax ---------------------------------------------------------------------------------


def _run_argmax(device, logits, count, offset):
    kern = K.ComputeKernel(device, K.ARGMAX)
    bl = device.upload(logits)
    bo = device.buffer(16)
    u = kern.uniform()
    u.write(K.argmax_dims(count, offset))
    kern.encode(kern.bind_group([bl, bo, u]), K.ARGMAX_WORKGROUPS)
    out = device.read_array(bo, np.uint32, 2)
    bl.release()
    bo.release()
    return out


def test_argmax_full_vocabulary(device):
    # forward_ops.test.ts:397-421
    logits = oracle.random_floats(151936, 101)
    logits[123456] = 99
    out = _run_argmax(device, logits, 151936, 0)
    assert out[0] == oracle.argmax_wgsl(logits) == 123456
    assert out[1] == np.float32(99).view(np.uint32)


def test_argmax_ties_to_lowest_index(device):
    # forward_ops.test.ts:423-446
    logits = np.full(2048, -1, np.float32)
    logits[100] = 5
    logits[900] = 5
    assert _run_argmax(device, logits, 2048, 0)[0] == 100


def test_argmax_offset_selects_a_row(device):
    logits = oracle.random_floats(3 * 5000, 5)
    out = _run_argmax(device, logits, 5000, 10000)
    assert out[0] == oracle.argmax_wgsl(logits[10000:15000])


# ---- batched plans --------------------------------------------------------------------------


def test_batched_plan_matches_per_matrix(device):
    # q | k | v of one layer plus a gate matrix: four matrices, one input, one launch.
    k = 896
    x = oracle.normal_floats(k, 12, 1.0)
    mats = [sym_weights(n, k, 900 + i) for i, n in enumerate((896, 128, 128, 4864))]
    bias = oracle.normal_floats(128, 13, 0.02)
    bx = device.upload(x)
    keep, segs, outs = [], [], []
    for i, q in enumerate(mats):
        bp, bs, _ = _upload_quant(device, q)
        bb = device.upload(bias) if i == 1 else None
        bo = device.buffer((q.rows + 3) * 4)
        device.zero(bo, (q.rows + 3) * 4)
        keep += [bp, bs, bo] + ([bb] if bb else [])
        segs.append((bp, bs, None, bb, bo, q.rows, 3))
        outs.append(bo)
    plan = K.GemvPlan(device, k, 32, segs)
    plan.launch(bx)
    for i, q in enumerate(mats):
        got = device.read_array(outs[i], np.float32, q.rows + 3)
        assert np.all(got[:3] == 0)
        expect = oracle.linear_q(x, q, bias if i == 1 else None, 1)
        assert_close(got[3:], expect, *gemv_tolerance(expect), label=f"segment {i}")
    plan.destroy()
    for b in keep + [bx]:
        b.release()


@pytest.mark.parametrize("k", [896, 4864])
def test_batched_plan_many_segments(device, k):
    """A plan of more than four matrices keeps its table in device memory with an index of the
    segment of every pass; each wave looks its first segment up there and walks on through the
    table: segments of 8 to 1024 rows, so a wave's range spans one to several segments and the
    smallest fall inside a single workgroup; biases and outOffsets on some. Every segment
    against the oracle."""
    rows = (8, 16, 24, 136, 8, 512, 64, 8, 32, 1024, 16, 40) if k == 896 else (8, 16, 8, 96, 24, 8, 40, 8)
    x = oracle.normal_floats(k, 1500 + k, 1.0)
    mats = [sym_weights(n, k, 1510 + i) for i, n in enumerate(rows)]
    bx = device.upload(x)
    keep, segs, outs, biases = [bx], [], [], []
    for i, q in enumerate(mats):
        bp, bs, _ = _upload_quant(device, q)
        bias = oracle.normal_floats(q.rows, 1530 + i, 0.02) if i % 3 == 1 else None
        bb = device.upload(bias) if bias is not None else None
        off = 5 if i % 4 == 2 else 0
        bo = device.buffer((q.rows + off) * 4)
        device.zero(bo, (q.rows + off) * 4)
        keep += [bp, bs, bo] + ([bb] if bb else [])
        segs.append((bp, bs, None, bb, bo, q.rows, off))
        outs.append((bo, off))
        biases.append(bias)
    plan = K.GemvPlan(device, k, 32, segs)
    for _ in range(2):  # twice: the table and index are reused as they are
        plan.launch(bx)
        for i, q in enumerate(mats):
            bo, off = outs[i]
            got = device.read_array(bo, np.float32, q.rows + off)
            assert np.all(got[:off] == 0)
            expect = oracle.linear_q(x, q, biases[i], 1)
            assert_close(got[off:], expect, *gemv_tolerance(expect), label=f"k={k} segment {i} ({q.rows} rows)")
    plan.destroy()
    for b in keep:
        b.release()


def test_batched_plan_rejects_bad_tables(device):
    q = sym_weights(896, 896, 5)
    bp, bs, _ = _upload_quant(device, q)
    bo = device.buffer(896 * 4)
    with pytest.raises(K.EgError, match="not a positive multiple of 8"):
        K.GemvPlan(device, 896, 32, [(bp, bs, None, None, bo, 12, 0)])
    with pytest.raises(K.EgError, match="missing a stream"):
        K.GemvPlan(device, 896, 32, [(bp, bs, None, None, bo, 896, 0)], encoding=K.ENC_OFFSET_ZEROS)
    for b in (bp, bs, bo):
        b.release()


# ---- every instantiated pipeline depth ------------------------------------------------------

# (EG_GEMV_SHAPE "team,chunks per lane,rows per lane,depth", bits, K): each entry is a kernel
# the library instantiates; the override makes a fresh context use it for every launch.
DEPTH_CASES = [("32,1,2,3", 4, 896), ("32,1,2,4", 4, 896), ("64,1,4,3", 4, 896), ("64,3,1,3", 4, 4864),
               ("64,3,1,4", 4, 4864), ("64,1,4,3", 8, 896), ("32,1,2,2", 4, 896), ("64,3,2,2", 4, 4864)]


@pytest.mark.parametrize("shape,bits,k", DEPTH_CASES)
def test_pipeline_depths_match_oracle(shape, bits, k):
    """A batched plan over segments of unequal length (so waves start mid-segment and cross
    segment ends with counts that are not multiples of the depth), a plain launch and the fused
    argmax, each under one forced (team, slots, rows, depth) shape."""
    print(f"shape {shape} bits {bits} k {k}", flush=True)
    x = oracle.normal_floats(k, 1300 + k, 1.0)
    rows = (1024, 136, 512, 64)
    mats = [sym_weights(n, k, 1400 + i, 32 if bits == 4 else k, bits) for i, n in enumerate(rows)]
    bias = oracle.normal_floats(136, 1399, 0.02)
    old = os.environ.get("EG_GEMV_SHAPE")
    os.environ["EG_GEMV_SHAPE"] = shape
    try:
        dev = K.Device(0)
    finally:
        if old is None:
            os.environ.pop("EG_GEMV_SHAPE")
        else:
            os.environ["EG_GEMV_SHAPE"] = old
    try:
        bx = dev.upload(x)
        keep, segs, outs = [bx], [], []
        for i, q in enumerate(mats):
            bp, bs = dev.upload(q.packed), dev.upload(q.scales)
            bb = dev.upload(bias) if i == 1 else None
            bo = dev.buffer(q.rows * 4)
            dev.zero(bo, q.rows * 4)
            keep += [bp, bs, bo] + ([bb] if bb else [])
            segs.append((bp, bs, None, bb, bo, q.rows, 0))
            outs.append(bo)
        plan = K.GemvPlan(dev, k, q.block_size, segs, bits=bits)
        plan.launch(bx)
        for i, q in enumerate(mats):
            got = dev.read_array(outs[i], np.float32, q.rows)
            expect = oracle.linear_q(x, q, bias if i == 1 else None, 1)
            assert_close(got, expect, *gemv_tolerance(expect), label=f"{shape} segment {i}")
        plan.destroy()
        # one matrix, plain launch and fused argmax (the LM head entry)
        q = mats[0]
        expect = oracle.linear_q(x, q, None, 1)
        logits, res = _run_head(dev, q, x, fused=True)
        assert_close(logits, expect, *gemv_tolerance(expect), label=f"{shape} single")
        assert res[0] == oracle.argmax(logits)
        for b in keep:
            b.release()
    finally:
        dev.close()
