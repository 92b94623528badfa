"""Long rows (more than 64 16-byte chunks: K > 2048 int4 or K > 1024 int8) on the GPU against the
CPU oracle, through the C ABI.

Such rows take a full-wave team with 2-4 chunk slots per lane, the last slot only partly
filled, and x held in registers per slot. The cases aim at what that can get wrong: odd row
counts (the last tile shifted back), a single row pair, the shortest (65 chunks) and longest
(256 chunks) rows, both encodings at 4 and 8 bits, bias and outOffset, batched plans whose
segments start mid-wave, the fused argmax and the fused input stages (the RMSNorm stage's
second, looped pass past 2048 inputs included).
"""

import ctypes

import numpy as np
import pytest

import oracle
from conftest import FP32_TOLERANCE, assert_close, gemv_tolerance
from enargeia_amd import _lib
from enargeia_amd import kernels as K
from enargeia_amd.model import INPUT_RMSNORM, INPUT_SILU_MUL, GemvInput
from test_gpu_gemv import run_decode, sym_weights

pytestmark = pytest.mark.gpu


def _quant(n, k, bits, fmt, seed):
    if fmt == "sym":
        return sym_weights(n, k, seed, 32 if bits == 4 else k, bits)
    w = oracle.random_floats(n * k, seed)
    return oracle.quantize_q4_ref(w, n, k) if bits == 4 else oracle.quantize_blocks_n(w, n, k, 8)


# (rows, K, bits, format): 152 chunks (the down projection: 3 slots per lane) with 3, 2 and 896
# rows; 66 chunks (2 slots, the second nearly empty), 256 chunks (4 full slots), int8 rows of 128
# chunks in both encodings.
LONG_CASES = [(3, 4864, 4, "sym"), (2, 4864, 4, "sym"), (896, 4864, 4, "sym"), (5, 2112, 4, "ref"),
              (7, 8192, 4, "sym"), (9, 2048, 8, "sym"), (11, 2048, 8, "ref"), (130, 4864, 4, "ref")]


@pytest.mark.parametrize("n,k,bits,fmt", LONG_CASES)
def test_long_rows_plain(device, n, k, bits, fmt):
    print(f"long rows {n}x{k} int{bits} {fmt}", flush=True)
    x = oracle.normal_floats(k, 2000 + k, 1.0)
    q = _quant(n, k, bits, fmt, 2100 + n)
    bias = oracle.normal_floats(n, 2200 + n, 0.02) if n % 2 else None
    off = 3 if n % 2 else 0
    got = run_decode(device, x, q, bias, out_offset=off)
    expect = oracle.linear_q(x, q, bias, 1)
    assert np.all(got[:off] == 0), "rows before outOffset written"
    tol = FP32_TOLERANCE if fmt == "ref" else gemv_tolerance(expect)
    assert_close(got[off:], expect, *tol, label=f"long {n}x{k} int{bits} {fmt}")


def test_long_rows_fused_argmax(device):
    n, k = 4099, 2048
    x = oracle.normal_floats(k, 2301, 1.0)
    q = sym_weights(n, k, 2302, k, 8)
    bx, bp, bs = device.upload(x), device.upload(q.packed), device.upload(q.scales)
    bl, br = device.buffer(n * 4), device.buffer(8)
    K.lm_head_argmax(device, bx, bp, bs, None, bl, br, K.embedding_dims(1, k, 0, n, k, n, 0), 8, K.ENC_SIGNED)
    logits = device.read_array(bl, np.float32, n)
    expect = oracle.linear_q(x, q, None, 1)
    assert_close(logits, expect, *gemv_tolerance(expect), label="long-row logits")
    order = np.argsort(expect)
    assert expect[order[-1]] - expect[order[-2]] > 1e-4 * np.abs(expect).max()
    assert int(device.read_array(br, np.uint32, 2)[0]) == int(order[-1])


def test_long_rows_batched_plan(device):
    """Segments of 8, 16, 896 and 24 rows (not multiples of a wave's share of the tiles), one
    with a bias, one written at an offset."""
    k = 4864
    x = oracle.normal_floats(k, 2401, 1.0)
    rows = (8, 16, 896, 24)
    mats = [sym_weights(r, k, 2410 + i) for i, r in enumerate(rows)]
    bias = oracle.normal_floats(16, 2420, 0.02)
    bx = device.upload(x)
    keep, segs, outs = [bx], [], []
    for i, q in enumerate(mats):
        bp, bs = device.upload(q.packed), device.upload(q.scales)
        bb = device.upload(bias) if i == 1 else None
        off = 5 if i == 3 else 0
        bo = device.buffer((q.rows + off) * 4)
        device.zero(bo, (q.rows + off) * 4)
        keep += [bp, bs, bo] + ([bb] if bb else [])
        segs.append((bp, bs, None, bb, bo, q.rows, off))
        outs.append((bo, off))
    plan = K.GemvPlan(device, k, 32, segs)
    plan.launch(bx)
    for i, q in enumerate(mats):
        bo, off = outs[i]
        got = device.read_array(bo, np.float32, q.rows + off)
        expect = oracle.linear_q(x, q, bias if i == 1 else None, 1)
        assert np.all(got[:off] == 0)
        assert_close(got[off:], expect, *gemv_tolerance(expect), label=f"long plan segment {i}")
    plan.destroy()
    for b in keep:
        b.release()


def _launch_input(device, plan, inp):
    _lib.check(_lib.load().eg_gemv_plan_launch_input(device.ctx, plan.handle, ctypes.byref(inp)), device.ctx)


def test_long_rows_rmsnorm_input(device):
    k, n = 2560, 64  # a hidden width past 2048: long rows with the norm fused
    q = sym_weights(n, k, 2501)
    x = oracle.normal_floats(k, 2502, 3.0)
    w = (1.0 + oracle.normal_floats(k, 2503, 0.1)).astype(np.float32)
    out = device.buffer(n * 4)
    plan = K.GemvPlan(device, k, 32, [(device.upload(q.packed), device.upload(q.scales), None, None, out, n, 0)])
    xb, wb = device.upload(x), device.upload(w)
    _launch_input(device, plan, GemvInput(INPUT_RMSNORM, xb.ptr, wb.ptr, 1e-6))
    got = device.read_array(out, np.float32, n)
    x64 = x.astype(np.float64)
    xn = (x64 / np.sqrt(np.mean(x64 ** 2) + 1e-6) * w).astype(np.float32)
    expect = oracle.linear_q(xn, q, None, 1)
    assert_close(got, expect, *gemv_tolerance(expect), label="long-row rmsnorm input")


def test_long_rows_silu_input_ragged_plan(device):
    k = 4864
    g = oracle.normal_floats(k, 2601, 2.0)
    u = oracle.normal_floats(k, 2602, 1.0)
    mats = [sym_weights(r, k, 2610 + i) for i, r in enumerate((24, 40))]
    outs = [device.buffer(q.rows * 4) for q in mats]
    plan = K.GemvPlan(device, k, 32, [(device.upload(q.packed), device.upload(q.scales), None, None, o, q.rows, 0)
                                      for q, o in zip(mats, outs)])
    gb, ub = device.upload(g), device.upload(u)
    _launch_input(device, plan, GemvInput(INPUT_SILU_MUL, gb.ptr, ub.ptr, 0.0))
    g64 = g.astype(np.float64)
    xs = (g64 / (1 + np.exp(-g64)) * u).astype(np.float32)
    for q, o in zip(mats, outs):
        expect = oracle.linear_q(xs, q, None, 1)
        assert_close(device.read_array(o, np.float32, q.rows), expect, 1e-5 * np.sqrt(np.mean(expect ** 2)), 1e-3,
                     label=f"long-row silu input {q.rows} rows")


def test_long_rows_deterministic(device):
    n, k = 896, 4864
    x = oracle.normal_floats(k, 2801, 1.0)
    q = sym_weights(n, k, 2802)
    first = run_decode(device, x, q, None)
    for _ in range(3):
        assert np.array_equal(run_decode(device, x, q, None).view(np.uint32), first.view(np.uint32))
