"""eg_lm_head_argmax_noalloc, the entry point that allocates nothing: through the C ABI, its
logits and greedy result must equal eg_lm_head_argmax's bit for bit (same kernels; only the
partials' buffer differs), on two calls in a row, the second over a smaller table, so a stale
partial of the first call cannot leak into the second. Sizes beyond its fixed scratch are
refused before anything runs."""

import ctypes

import numpy as np
import pytest

from enargeia_amd import _lib
from enargeia_amd import kernels as K
from enargeia_amd.quant import normal, quantize_asym, quantize_sym

pytestmark = pytest.mark.gpu


def call(device, fn, x, q, out, result, dims, bits, encoding):
    d = K.EmbeddingDims.from_buffer_copy(dims)
    vp = ctypes.c_void_p
    z = vp(q[2].ptr) if q[2] is not None else None
    _lib.check(fn(device.ctx, vp(x.ptr), vp(q[0].ptr), vp(q[1].ptr), z, vp(out.ptr), vp(result.ptr),
                  ctypes.byref(d), encoding, bits), device.ctx)


def head(device, rows, hidden, seed, fmt):
    w = normal(rows * hidden, seed, 0.02)
    if fmt == "sym":
        t = quantize_sym(w, rows, hidden, 8, hidden)
        return (device.upload(t.packed), device.upload(t.scales), None), K.ENC_SIGNED, hidden
    t = quantize_asym(w, rows, hidden, 8, 64)
    return (device.upload(t.packed), device.upload(t.scales), device.upload(t.zeros)), K.ENC_OFFSET_ZEROS, 64


@pytest.mark.parametrize("fmt", ["sym", "reference"])
def test_noalloc_head_equals_allocating_head(device, fmt):
    lib = _lib.load()
    hidden = 896
    x = device.upload(normal(hidden, 7, 1.0).astype(np.float32))
    for rows, seed in ((151936, 0x5EED ^ 0x1000), (4099, 31)):  # config 2, then a smaller ragged table
        q, enc, block = head(device, rows, hidden, seed, fmt)
        dims = K.embedding_dims(1, hidden, 0, rows, block, rows, 0)
        outs = [device.buffer(rows * 4) for _ in range(2)]
        results = [device.buffer(8) for _ in range(2)]
        for b in outs:
            device.zero(b, rows * 4)
        call(device, lib.eg_lm_head_argmax, x, q, outs[0], results[0], dims, 8, enc)
        call(device, lib.eg_lm_head_argmax_noalloc, x, q, outs[1], results[1], dims, 8, enc)
        logits = [device.read_array(b, np.float32, rows) for b in outs]
        res = [device.read_array(b, np.uint32, 2) for b in results]
        np.testing.assert_array_equal(logits[1], logits[0])
        np.testing.assert_array_equal(res[1], res[0])
        assert int(res[1][0]) == int(np.argmax(logits[1]))  # ties to the lowest index, as np.argmax
        for b in outs + results + [b for b in q if b is not None]:
            b.release()
    x.release()


def test_noalloc_head_rejects_bad_arguments(device):
    lib = _lib.load()
    d = K.EmbeddingDims.from_buffer_copy(K.embedding_dims(1, 896, 0, 16, 896, 16, 0))
    buf = device.buffer(1 << 16)
    vp = ctypes.c_void_p(buf.ptr)
    st = lib.eg_lm_head_argmax_noalloc(device.ctx, vp, vp, vp, None, vp, None, ctypes.byref(d), K.ENC_SIGNED, 8)
    assert st == _lib.EG_ERR_INVALID and b"result is NULL" in lib.eg_last_error(device.ctx)
    st = lib.eg_lm_head_argmax_noalloc(device.ctx, vp, vp, vp, None, vp, vp, ctypes.byref(d), K.ENC_SIGNED, 5)
    assert st == _lib.EG_ERR_INVALID
    buf.release()
