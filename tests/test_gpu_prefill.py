"""The bf16-MFMA prefill GEMM (eg_matmul_q4_prefill) against the oracle.

Two bars: against the oracle's bf16 model (bf16 x, bf16 dequantized W, exact products, float64
sums) the MFMA's f32 accumulation must agree to 1e-4; against the fp32 reference
(linearQ4, quant.ts:95-111) it must be within BASELINE's 2e-2 (per element |a - e| <=
2e-2 * (|e| + rms(e))). Shapes follow test/kernels/matmul_q4.test.ts:149-196 and config 3.
"""

import functools

import numpy as np
import pytest

import oracle
from conftest import assert_close
from enargeia_amd import kernels as K

pytestmark = pytest.mark.gpu


def prefill_tol(expect):
    rms = float(np.sqrt(np.mean(np.asarray(expect, np.float64) ** 2)))
    return 2e-2 * rms, 2e-2


def model_tol(expect):
    rms = float(np.sqrt(np.mean(np.asarray(expect, np.float64) ** 2)))
    return 1e-4 * rms, 1e-4


def run_prefill(device, x, q, bias, m, out_len=None, out_stride=None, out_offset=0):
    kern = K.ComputeKernel(device, K.with_format(K.MATMUL_Q4_PREFILL, q.bits, q.encoding))
    stride = q.rows if out_stride is None else out_stride
    n_out = out_len if out_len is not None else (m - 1) * stride + q.rows + out_offset
    bufs = [device.upload(x), device.upload(q.packed), device.upload(q.scales),
            device.upload(q.zeros) if q.zeros is not None else None,
            device.upload(bias if bias is not None else np.zeros(q.rows, np.float32))]
    bo = device.buffer(n_out * 4)
    device.zero(bo, n_out * 4)
    u = kern.uniform()
    u.write(K.matmul_q4_dims(m, q.rows, q.cols, bias is not None, q.block_size, stride, out_offset))
    kern.encode(kern.bind_group([*bufs, bo, u]), K.matmul_q4_prefill_workgroups(m, q.rows))
    y = device.read_array(bo, np.float32, n_out)
    for b in bufs + [bo]:
        if b is not None:
            b.release()
    return y


@pytest.mark.parametrize("m,n,k", [(15, 896, 896), (15, 128, 896), (4, 4864, 896), (64, 32, 64)])
def test_prefill_reference_shapes(device, m, n, k):
    # matmul_q4.test.ts:149-160, seeds 11/12/13, reference asymmetric block-64 weights + bias.
    x = oracle.random_floats(m * k, 11)
    q = oracle.quantize_q4_ref(oracle.random_floats(n * k, 12), n, k)
    bias = oracle.random_floats(n, 13)
    got = run_prefill(device, x, q, bias, m)
    model = oracle.linear_q_bf16(x, q, bias, m)
    assert_close(got, model, *model_tol(model), label=f"bf16 model {m}x{n}x{k}")
    fp32 = oracle.linear_q(x, q, bias, m)
    assert_close(got, fp32, *prefill_tol(fp32), label=f"fp32 reference {m}x{n}x{k}")


def test_prefill_ragged_tile(device):
    # matmul_q4.test.ts:173-179: shapes that do not fill the 64x64 tile.
    x = oracle.random_floats(3 * 64, 31)
    q = oracle.quantize_q4_ref(oracle.random_floats(5 * 64, 32), 5, 64)
    got = run_prefill(device, x, q, None, 3)
    assert_close(got, oracle.linear_q_bf16(x, q, None, 3), *model_tol(oracle.linear_q(x, q, None, 3)),
                 label="ragged 3x5x64")


def test_prefill_out_offset_and_stride(device):
    # matmul_q4.test.ts:181-195 (x = 1, W = 0.5 is exact in bf16: 32 at offset 4 and 5).
    k = 64
    q = oracle.quantize_q4_ref(np.full(2 * k, 0.5, np.float32), 2, k)
    got = run_prefill(device, np.ones(k, np.float32), q, None, 1, out_len=6, out_stride=6, out_offset=4)
    assert got[0] == 0 and got[1] == 0
    assert got[4] == 32 and got[5] == 32


def test_prefill_agrees_with_decode_at_m1(device):
    # matmul_q4.test.ts:216-230: the two kernels are independent statements of the same math.
    from test_gpu_gemv import run_decode
    n, k = 256, 192
    x = oracle.random_floats(k, 51)
    q = oracle.quantize_q4_ref(oracle.random_floats(n * k, 52), n, k)
    dec = run_decode(device, x, q, None)
    pre = run_prefill(device, x, q, None, 1)
    assert_close(pre, dec, *prefill_tol(dec), label="prefill vs decode")


@functools.lru_cache(maxsize=None)
def config3(m, n, k, seed):
    x = oracle.normal_floats(m * k, seed, 1.0)
    q = oracle.quantize_sym(oracle.normal_floats(n * k, seed + 1, 0.02), n, k, 4, 32)
    return x, q


@pytest.mark.parametrize("m", [256, 128])
@pytest.mark.parametrize("n,k", [(4864, 896), (896, 4864)])
def test_prefill_config3(device, m, n, k):
    # X [m x k] ~ N(0,1) through gate/up (896->4864) and down (4864->896).
    x, q = config3(m, n, k, 0x5EED ^ (n + k))
    got = run_prefill(device, x, q, None, m)
    model = oracle.linear_q_bf16_fast(x, q, None, m)
    assert_close(got, model, *model_tol(model), label=f"config 3 bf16 model {m}x{n}x{k}")
    fp32 = oracle.linear_q_fast(x, q, None, m)
    assert_close(got, fp32, *prefill_tol(fp32), label=f"config 3 fp32 {m}x{n}x{k}")


@pytest.mark.parametrize("bits,k,bs", [(4, 40, 8), (8, 128, 64), (4, 96, 32), (4, 96, 48)])
def test_prefill_element_staging_path(device, bits, k, bs):
    m, n = 7, 24
    x = oracle.random_floats(m * k, 61)
    if bits == 4:
        q = oracle.quantize_q4_ref(oracle.random_floats(n * k, 62), n, k, bs)
    else:
        q = oracle.quantize_blocks_n(oracle.random_floats(n * k, 62), n, k, 8, bs)
    got = run_prefill(device, x, q, None, m)
    assert_close(got, oracle.linear_q_bf16(x, q, None, m), *model_tol(oracle.linear_q(x, q, None, m)),
                 label=f"element path bits={bits} k={k}")


@pytest.mark.parametrize("bs", [64, 128])
def test_prefill_symmetric_long_blocks(device, bs):
    # Symmetric int4 with quant blocks of 64 and 128 codes: the staged path finds a code's block
    # by shift, and a 128-code block spans two 64-deep staging steps.
    m, n, k = 33, 96, 640
    x = oracle.normal_floats(m * k, 71, 1.0)
    q = oracle.quantize_sym(oracle.normal_floats(n * k, 72, 0.02), n, k, 4, bs)
    got = run_prefill(device, x, q, None, m)
    model = oracle.linear_q_bf16(x, q, None, m)
    assert_close(got, model, *model_tol(model), label=f"symmetric block {bs} bf16 model")
    fp32 = oracle.linear_q(x, q, None, m)
    assert_close(got, fp32, *prefill_tol(fp32), label=f"symmetric block {bs} fp32")


def test_prefill_deterministic(device):
    x, q = config3(128, 4864, 896, 99)
    a = run_prefill(device, x, q, None, 128)
    b = run_prefill(device, x, q, None, 128)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def run_swiglu(device, x, gate, up, m):
    """eg_matmul_q4_prefill_swiglu through the C ABI: SiLU(x . gate) * (x . up), [m][n]."""
    import ctypes
    from enargeia_amd import _lib
    n, k = gate.rows, gate.cols
    opt = lambda a: device.upload(a) if a is not None else None
    bufs = [device.upload(x), device.upload(gate.packed), device.upload(gate.scales), opt(gate.zeros),
            device.upload(up.packed), device.upload(up.scales), opt(up.zeros)]
    out, scratch = device.buffer(m * n * 4), device.buffer(m * 2 * n * 4)
    d = K.MatmulDims.from_buffer_copy(K.matmul_q4_dims(m, n, k, False, gate.block_size, n, 0))
    vp = lambda b: ctypes.c_void_p(b.ptr if b is not None else None)
    try:
        _lib.check(_lib.load().eg_matmul_q4_prefill_swiglu(device.ctx, *[vp(b) for b in bufs], vp(out), vp(scratch),
                                                            ctypes.byref(d), gate.encoding, gate.bits), device.ctx)
        return device.read_array(out, np.float32, m * n)
    finally:
        for b in bufs + [out, scratch]:
            if b is not None:
                b.release()


@pytest.fixture(scope="module")
def unpaired():
    """A second context whose SwiGLU operator always takes the two-launch form."""
    import os
    os.environ["EG_PREFILL_PAIR"] = "0"
    try:
        dev = K.Device(0)
    finally:
        del os.environ["EG_PREFILL_PAIR"]
    yield dev
    dev.close()


@pytest.mark.parametrize("m,n,k,sym", [(256, 4864, 896, True), (200, 1000, 896, False), (3, 100, 64, True),
                                       (70, 4864, 4864, True)])
def test_prefill_swiglu_pair(device, unpaired, m, n, k, sym):
    # The prompt MLP's gate / up / silu_mul (graph.ts:484-497) as one operator: gate and up rows
    # side by side in paired tiles, SiLU(g) * u in the epilogue. Each projection's f32 sums are
    # the plain GEMM's to the bit (same staging, MFMA order and group split at these shapes), so
    # the result equals the two-launch form (gate | up into the scratch rows, then
    # silu_mul_rows) bit for bit, and SiLU·up of two eg_matmul_q4_prefill outputs computed on the
    # host up to the exponential's and the division's last bits (numpy's float32 exp against the
    # device's expf: 6 ulp measured at most). K = 4864 takes the two-launch form on both.
    x = oracle.random_floats(m * k, 41)
    if sym:
        gate = oracle.quantize_sym(oracle.normal_floats(n * k, 42, 0.05), n, k, 4, 32)
        up = oracle.quantize_sym(oracle.normal_floats(n * k, 43, 0.05), n, k, 4, 32)
    else:
        gate = oracle.quantize_q4_ref(oracle.random_floats(n * k, 42), n, k)
        up = oracle.quantize_q4_ref(oracle.random_floats(n * k, 43), n, k)
    got = run_swiglu(device, x, gate, up, m).reshape(m, n)
    two = run_swiglu(unpaired, x, gate, up, m).reshape(m, n)
    np.testing.assert_array_equal(got.view(np.uint32), two.view(np.uint32))
    g = run_prefill(device, x, gate, None, m).reshape(m, n)
    u = run_prefill(device, x, up, None, m).reshape(m, n)
    want = g / (np.float32(1) + np.exp(-g)) * u
    np.testing.assert_array_max_ulp(got, want.astype(np.float32), maxulp=16)
    # and the fp32 reference: each projection's bar (|a - e| <= 2e-2 (|e| + rms(e))) carried
    # through SiLU(g) * u to first order: |d| <= |SiLU'(g) u| bar_g + |SiLU(g)| bar_u
    gf = oracle.linear_q_fast(x, gate, None, m).reshape(m, n).astype(np.float64)
    uf = oracle.linear_q_fast(x, up, None, m).reshape(m, n).astype(np.float64)
    sig = 1 / (1 + np.exp(-gf))
    ref = gf * sig * uf
    bar = lambda e: 2e-2 * (np.abs(e) + np.sqrt(np.mean(e ** 2)))
    bound = np.abs(sig * (1 + gf * (1 - sig)) * uf) * bar(gf) + np.abs(gf * sig) * bar(uf)
    excess = np.abs(got - ref) / bound
    assert excess.max() <= 1.0, f"swiglu {m}x{n}x{k}: {excess.max() * 100:.1f}% of the carried bar"


@pytest.mark.parametrize("m,n,k", [(512, 896, 896), (1024, 896, 4864), (1024, 1152, 896)])
def test_prefill_row_tiles_per_xcd(device, m, n, k):
    # A multiple of 8 row tiles and a column-tile count that is not: the launch maps whole row
    # tiles to each XCD (workgroup L of the grid runs tile (L / 8 % columns, L % 8 + 8 * (L / 8 /
    # columns))), every tile exactly once - against the bf16 model like any other shape. The
    # K = 4864 case splits K and keeps the grid's own order.
    x, q = config3(m, n, k, 0x5EED ^ (m + n + k))
    got = run_prefill(device, x, q, None, m)
    model = oracle.linear_q_bf16_fast(x, q, None, m)
    assert_close(got, model, *model_tol(model), label=f"xcd rows {m}x{n}x{k}")


def test_prefill_swiglu_rejects_bad_dims(device):
    import ctypes
    from enargeia_amd import _lib
    lib = _lib.load()
    buf = device.buffer(4096)
    p = ctypes.c_void_p(buf.ptr)
    try:
        for dims, what in ((K.matmul_q4_dims(4, 64, 64, True, 32, 64, 0), "bias"),
                           (K.matmul_q4_dims(4, 64, 64, False, 32, 96, 0), "stride"),
                           (K.matmul_q4_dims(4, 62, 64, False, 32, 62, 0), "n % 4")):
            d = K.MatmulDims.from_buffer_copy(dims)
            st = lib.eg_matmul_q4_prefill_swiglu(device.ctx, p, p, p, None, p, p, None, p, p, ctypes.byref(d),
                                                 K.ENC_SIGNED, 4)
            assert st != 0, what
    finally:
        buf.release()
