"""The LM head and the row gather over an f16 or f32 tied table - the reference's 'f16' and 'f32'
embedding dtypes (embedding_variants.ts:26-74, 93-180: the table read as it is, halves through
unpack2x16float) - against the oracle's float64 statement (oracle.decode.dense_head and
dense_values, pinned in tests/test_decode_oracle.py by known half bit patterns, one-hot rows
and the int8 head over the same integers).

Bars: logits within the reference's FP32_TOLERANCE (1e-4 absolute + 1e-4 relative,
test/kernels/matmul_q4.test.ts) of the float64 sums; the fused argmax index equal to the
argmax of the launch's own logits always, and to the oracle's wherever its top-2 gap exceeds
the bar; gathered rows bit-exact (the conversion from f16 is exact).
"""

import ctypes

import numpy as np
import pytest

from conftest import assert_close
from enargeia_amd import _lib
from enargeia_amd import kernels as K
from enargeia_amd.model import INPUT_RMSNORM, GemvInput
from enargeia_amd.quant import dense_table
from oracle.decode import dense_head, dense_values

pytestmark = pytest.mark.gpu

TOL = (1e-4, 1e-4)  # absolute, relative
BITS = {"f16": 16, "f32": 32}


def _vp(p):
    return ctypes.c_void_p(p)


def head(device, x, t, out_offset=0, table_offset=0, fused=True):
    """eg_lm_head and eg_lm_head_argmax over table t; the table placed `table_offset` bytes into
    its buffer (16-byte alignment lost for an offset of 4). Returns (logits, argmax result)."""
    n, k = t.rows, t.cols
    lib = _lib.load()
    raw = np.concatenate([np.zeros(table_offset // 4, np.uint32), t.packed])
    bt, bx = device.upload(raw), device.upload(np.ascontiguousarray(x, np.float32))
    bo, bo2 = device.buffer((n + out_offset) * 4), device.buffer((n + out_offset) * 4)
    br = device.buffer(8)
    d = K.EmbeddingDims.from_buffer_copy(K.embedding_dims(1, k, 0, n, k, n, out_offset))
    try:
        _lib.check(lib.eg_lm_head(device.ctx, _vp(bx.ptr), _vp(bt.ptr + table_offset), None, None, _vp(bo.ptr),
                                  ctypes.byref(d), K.ENC_SIGNED, t.bits), device.ctx)
        res = None
        if fused:
            _lib.check(lib.eg_lm_head_argmax(device.ctx, _vp(bx.ptr), _vp(bt.ptr + table_offset), None, None,
                                             _vp(bo2.ptr), _vp(br.ptr), ctypes.byref(d), K.ENC_SIGNED, t.bits),
                       device.ctx)
            res = device.read_array(br, np.uint32, 2)
            # the fused launch stores the same logits
            np.testing.assert_array_equal(device.read_array(bo2, np.float32, n + out_offset)[out_offset:],
                                          device.read_array(bo, np.float32, n + out_offset)[out_offset:])
        return device.read_array(bo, np.float32, n + out_offset)[out_offset:], res
    finally:
        for b in (bt, bx, bo, bo2, br):
            b.release()


def check_head(got, res, want, label, out_offset=0):
    scale = float(np.abs(want).max())
    assert_close(got, want, TOL[0], TOL[1], label=label)
    if res is not None:
        assert res[0] == out_offset + int(np.argmax(got)), f"{label}: fused argmax {res[0]} vs its logits"
        assert res[1] == got[res[0] - out_offset].view(np.uint32)
        order = np.argsort(want)
        if want[order[-1]] - want[order[-2]] > 2 * (TOL[0] + TOL[1] * scale):
            assert res[0] - out_offset == int(order[-1]), f"{label}: argmax {res[0]} vs oracle {order[-1]}"


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_config2_shape_dense_head(device, dtype):
    # BASELINE config 2's head shape (151,936 x 896) as an f16 (272 MB) or f32 (545 MB) table
    print(f"dense head {dtype} 151936 x 896", flush=True)
    rng = np.random.default_rng(20 + BITS[dtype])
    n, k = 151936, 896
    t = dense_table((rng.standard_normal(n * k, dtype=np.float32) * np.float32(0.02)), n, k, BITS[dtype])
    x = rng.standard_normal(k).astype(np.float32)
    got, res = head(device, x, t)
    check_head(got, res, dense_head(x, t), f"config-2 shape {dtype}")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("n,k,table_offset,out_offset", [(1000, 100, 0, 7), (777, 896, 4, 0), (3, 64, 0, 0),
                                                         (4099, 258, 0, 1)])
def test_ragged_and_unaligned_tables(device, dtype, n, k, table_offset, out_offset):
    """Rows that are not whole 16-byte vectors (k 100, 258 in f16; 258 in f32) and a table that
    is not 16-byte aligned take the element path; outOffset; 3 rows (fewer than a workgroup's
    waves)."""
    rng = np.random.default_rng(n + k)
    if BITS[dtype] == 16 and (n * k) % 2:
        pytest.skip("an f16 table holds an even element count")
    t = dense_table(rng.standard_normal(n * k, dtype=np.float32), n, k, BITS[dtype])
    x = rng.standard_normal(k).astype(np.float32)
    got, res = head(device, x, t, out_offset=out_offset, table_offset=table_offset)
    check_head(got, res, dense_head(x, t), f"{dtype} n={n} k={k} offset={table_offset}", out_offset)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_fused_rmsnorm_input(device, dtype):
    """The decoder's head: the final RMSNorm folded into the launch (eg_lm_head_argmax_input,
    EG_INPUT_RMSNORM) against the oracle's rmsnorm then the dense head."""
    import oracle
    rng = np.random.default_rng(5 + BITS[dtype])
    n, k, eps = 5000, 896, 1e-6
    t = dense_table(rng.standard_normal(n * k, dtype=np.float32) * np.float32(0.05), n, k, BITS[dtype])
    h = rng.standard_normal(k).astype(np.float32) * np.float32(3.0)
    w = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    bt, bh, bw = device.upload(t.packed), device.upload(h), device.upload(w)
    bo, br = device.buffer(n * 4), device.buffer(8)
    inp = GemvInput(INPUT_RMSNORM, bh.ptr, bw.ptr, eps)
    d = K.EmbeddingDims.from_buffer_copy(K.embedding_dims(1, k, 0, n, k, n, 0))
    try:
        _lib.check(_lib.load().eg_lm_head_argmax_input(device.ctx, ctypes.byref(inp), _vp(bt.ptr), None, None,
                                                       _vp(bo.ptr), _vp(br.ptr), ctypes.byref(d), K.ENC_SIGNED,
                                                       BITS[dtype]), device.ctx)
        got, res = device.read_array(bo, np.float32, n), device.read_array(br, np.uint32, 2)
    finally:
        for b in (bt, bh, bw, bo, br):
            b.release()
    want = dense_head(oracle.rmsnorm(h, w, 1, k, eps), t)
    check_head(got, res, want, f"rmsnorm + {dtype} head")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_gather_rows_bit_exact(device, dtype):
    """embed_gather_f16 / _f32 (embedding_variants.ts:93-133): the id's row as it is; an id
    outside [row_begin, row_begin + row_count) leaves out untouched."""
    rng = np.random.default_rng(9)
    n, k = 300, 96
    t = dense_table(rng.standard_normal(n * k, dtype=np.float32), n, k, BITS[dtype])
    rows = dense_values(t)
    bt, bo, btok = device.upload(t.packed), device.buffer(k * 4), device.buffer(4)
    lib = _lib.load()
    try:
        for tok, begin, want in ((17, 0, rows[17]), (299, 0, rows[299]), (150, 100, rows[150]),
                                 (50, 100, None)):
            device.write(bo, np.full(k, -7.0, np.float32))
            device.write(btok, np.array([tok], np.uint32))
            d = K.EmbeddingDims.from_buffer_copy(K.embedding_dims(1, k, begin, n - begin, k, 0, 0))
            pk = _vp(bt.ptr + begin * k * BITS[dtype] // 8)
            _lib.check(lib.eg_embed_gather(device.ctx, _vp(btok.ptr), pk, None, None, _vp(bo.ptr), ctypes.byref(d),
                                           K.ENC_SIGNED, BITS[dtype]), device.ctx)
            got = device.read_array(bo, np.float32, k)
            np.testing.assert_array_equal(got, np.full(k, -7.0, np.float32) if want is None else want)
    finally:
        for b in (bt, bo, btok):
            b.release()


def test_dense_head_argument_errors(device):
    lib = _lib.load()
    buf = device.buffer(1 << 20)
    vp = _vp(buf.ptr)
    try:
        big = K.EmbeddingDims.from_buffer_copy(K.embedding_dims(1, 16400, 0, 4, 16400, 4, 0))
        assert lib.eg_lm_head(device.ctx, vp, vp, None, None, vp, ctypes.byref(big), K.ENC_SIGNED, 16) == \
            _lib.EG_ERR_RANGE
        assert b"16384" in lib.eg_last_error(device.ctx)
        d = K.EmbeddingDims.from_buffer_copy(K.embedding_dims(1, 64, 0, 4, 64, 4, 0))
        # the projections take codes only; bits 24 is no format
        md = K.MatmulDims.from_buffer_copy(K.matmul_q4_dims(1, 4, 64, False, 64, 4, 0))
        assert lib.eg_matmul_q4_decode(device.ctx, vp, vp, vp, None, None, vp, ctypes.byref(md), K.ENC_SIGNED,
                                       16) == _lib.EG_ERR_INVALID
        assert lib.eg_lm_head(device.ctx, vp, vp, vp, None, vp, ctypes.byref(d), K.ENC_SIGNED, 24) == \
            _lib.EG_ERR_INVALID
        assert lib.eg_embed_gather(device.ctx, vp, vp, None, None, vp, ctypes.byref(d), K.ENC_SIGNED, 24) == \
            _lib.EG_ERR_INVALID
        zero = K.EmbeddingDims.from_buffer_copy(K.embedding_dims(1, 64, 0, 0, 64, 0, 0))
        assert lib.eg_lm_head_argmax(device.ctx, vp, vp, None, None, vp, vp, ctypes.byref(zero), K.ENC_SIGNED,
                                     32) == _lib.EG_ERR_INVALID
    finally:
        buf.release()


@pytest.mark.parametrize("bits", [8, 16])
def test_gather_many_ids(device, bits):
    """The reference's gather over dims.seq ids (embedding_variants.ts:113-123: one row per id,
    out[s * hidden + i]), ids of another part of a split table leaving their rows untouched."""
    from enargeia_amd.quant import quantize_sym
    from oracle.decode import dequant_row
    rng = np.random.default_rng(31 + bits)
    n, k = 500, 128
    vals = rng.standard_normal(n * k, dtype=np.float32)
    t = dense_table(vals, n, k, 16) if bits == 16 else quantize_sym(vals, n, k, 8, 32)
    ids = np.array([3, 499, 250, 1000, 0, 250], np.uint32)  # 1000: another part's id
    seq = ids.size
    bt = device.upload(t.packed)
    bs = device.upload(t.scales) if bits == 8 else None
    bo, bid = device.upload(np.full(seq * k, -7.0, np.float32)), device.upload(ids)
    d = K.EmbeddingDims.from_buffer_copy(K.embedding_dims(seq, k, 0, n, k if bits == 16 else 32, 0, 0))
    try:
        _lib.check(_lib.load().eg_embed_gather(device.ctx, _vp(bid.ptr), _vp(bt.ptr), _vp(bs.ptr) if bs else None,
                                               None, _vp(bo.ptr), ctypes.byref(d), K.ENC_SIGNED, bits), device.ctx)
        got = device.read_array(bo, np.float32, seq * k).reshape(seq, k)
    finally:
        for b in (bt, bs, bo, bid):
            if b is not None:
                b.release()
    for s_, i in enumerate(ids):
        want = np.full(k, -7.0, np.float32) if i >= n else dequant_row(t, int(i))
        np.testing.assert_array_equal(got[s_], want, err_msg=f"row {s_} (id {i})")


@pytest.mark.parametrize("dtype", ["q8", "f16"])
def test_gather_through_the_kernel_interface(device, dtype):
    """embeddingGatherSpec(dtype) through ComputeKernel (kernel.ts:20-112), as a reference caller
    binds it: [ids, packed, scales, zeros, out, dims] and embeddingGatherWorkgroups' grid."""
    from enargeia_amd.quant import quantize_sym
    from oracle.decode import dequant_row
    rng = np.random.default_rng(41)
    n, k = 256, 64
    vals = rng.standard_normal(n * k, dtype=np.float32)
    t = dense_table(vals, n, k, 16) if dtype == "f16" else quantize_sym(vals, n, k, 8, k)
    ids = np.array([7, 255, 0, 128], np.uint32)
    kern = K.ComputeKernel(device, K.embedding_gather_spec(dtype, K.ENC_SIGNED))
    bufs = [device.upload(ids), device.upload(t.packed), device.upload(t.scales) if t.scales.size else None, None,
            device.buffer(ids.size * k * 4)]
    try:
        u = kern.uniform()
        u.write(K.embedding_dims(ids.size, k, 0, n, t.block_size, 0, 0))
        kern.encode(kern.bind_group(bufs + [u]), (1, ids.size, 1))
        got = device.read_array(bufs[4], np.float32, ids.size * k).reshape(ids.size, k)
    finally:
        for b in bufs:
            if b is not None:
                b.release()
    for s_, i in enumerate(ids):
        np.testing.assert_array_equal(got[s_], dequant_row(t, int(i)))
