"""Chunked-prefill attention (eg_attention_prefill) against the CPU oracle's restatement of the
reference's prefill (RoPE, f16 cache writes, attn_scores -> softmax -> attn_apply;
cache_variants.ts:81-145, graph.ts:411-459).

Bars: q_rope and the appended cache rows bit-exact (the same double-precision RoPE and f16
rounding); the attention output within 1e-2 relative with an absolute floor of 1e-2 x the
output's RMS, because the matrix cores multiply f16 operands (q and the softmax weights are
rounded to f16, |error| ~ 2^-11 relative each) where the reference multiplies in f32.
"""

import ctypes

import numpy as np
import pytest

from conftest import assert_close
from enargeia_amd import _lib
from oracle.decode import f16_array, prefill_attention

pytestmark = pytest.mark.gpu

H, KV, D, CTX, THETA = 14, 2, 64, 2048, 1.0e6


class PrefillDims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("queries", "keys", "query_begin", "heads", "kv_heads", "head_dim",
                                               "max_context")] + [("theta", ctypes.c_float)]


def run(device, q, k, v, kc16, vc16, begin, dims=None):
    n = q.shape[0]
    bq, bk, bv = device.upload(q), device.upload(k), device.upload(v)
    bkc, bvc = device.upload(kc16), device.upload(vc16)
    bqr, bo = device.buffer(q.nbytes), device.buffer(q.nbytes)
    d = dims or PrefillDims(n, begin + n, begin, H, KV, D, CTX, THETA)
    vp = ctypes.c_void_p
    try:
        _lib.check(_lib.load().eg_attention_prefill(device.ctx, vp(bq.ptr), vp(bk.ptr), vp(bv.ptr), vp(bkc.ptr),
                                                    vp(bvc.ptr), vp(bqr.ptr), vp(bo.ptr), ctypes.byref(d)),
                   device.ctx)
        return (device.read_array(bqr, np.float32, q.size).reshape(q.shape),
                device.read_array(bo, np.float32, q.size).reshape(q.shape),
                device.read_array(bkc, np.uint16, kc16.size).reshape(kc16.shape),
                device.read_array(bvc, np.uint16, vc16.size).reshape(vc16.shape))
    finally:
        for b in (bq, bk, bv, bkc, bvc, bqr, bo):
            b.release()


# (1000, 256) and (1792, 256) split their keys over grid.z (the (query block, head) grid alone
# would leave most CUs idle): 5 and 8 splits of 256 keys, rows whose causal limit ends before a
# split's first key (an empty split for that row) included; (1900, 148) splits into 7; a whole
# 1024- or 2048-token prompt splits so that no workgroup walks more than 8 key tiles (2 and 4
# splits, most of the early query blocks' later splits empty).
@pytest.mark.parametrize("begin,n", [(0, 256), (0, 128), (300, 77), (1900, 148), (5, 1), (63, 64), (1000, 256),
                                     (1792, 256), (0, 1024), (0, 2048)])
def test_prefill_attention_matches_oracle(device, begin, n):
    print(f"prefill attention begin {begin} queries {n}", flush=True)
    rng = np.random.default_rng(1000 + begin + n)
    q = rng.standard_normal((n, H * D), dtype=np.float32)
    k = rng.standard_normal((n, KV * D), dtype=np.float32)
    v = rng.standard_normal((n, KV * D), dtype=np.float32)
    # earlier positions already cached (f16 values), later ones garbage the mask must ignore
    kc = f16_array(rng.standard_normal((CTX, KV, D), dtype=np.float32))
    vc = f16_array(rng.standard_normal((CTX, KV, D), dtype=np.float32))
    kc16, vc16 = kc.astype(np.float16).view(np.uint16), vc.astype(np.float16).view(np.uint16)
    got_qr, got, got_kc, got_vc = run(device, q, k, v, kc16, vc16, begin)
    want_qr, want = prefill_attention(q, k, v, kc, vc, begin, H, KV, D, THETA)
    # The rotation runs in double precision on both sides; the GPU's and the host's double cos /
    # sin may differ in their last bit, which flips the f32 rounding of a rare element by one
    # ulp (1 of 1.8 M at 2048 positions): bit-exact otherwise.
    np.testing.assert_array_max_ulp(got_qr, want_qr, maxulp=1)
    assert np.count_nonzero(got_qr != want_qr) <= max(1, got_qr.size // 100000)
    np.testing.assert_array_equal(got_kc, kc.astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(got_vc, vc.astype(np.float16).view(np.uint16))
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got.ravel(), want.ravel(), 1e-2 * rms, 1e-2, label=f"prefill attention begin {begin} n {n}")


def test_prefill_attention_rejects_bad_dims(device):
    q = np.zeros((4, H * D), np.float32)
    k = np.zeros((4, KV * D), np.float32)
    c = np.zeros((CTX, KV, D), np.uint16)
    with pytest.raises(_lib.EgError, match="head_dim 128 is not supported"):
        run(device, q, k, k, c, c, 0, PrefillDims(4, 4, 0, H, KV, 128, CTX, THETA))
    with pytest.raises(_lib.EgError, match="keys 5 != query_begin 0 \\+ queries 4"):
        run(device, q, k, k, c, c, 0, PrefillDims(4, 5, 0, H, KV, D, CTX, THETA))
    with pytest.raises(_lib.EgRangeError, match="exceed the cache's 2048"):
        run(device, q, k, k, c, c, 2046, PrefillDims(4, 2050, 2046, H, KV, D, CTX, THETA))
    with pytest.raises(_lib.EgError, match="not a multiple of kv_heads"):
        run(device, q, k, k, c, c, 0, PrefillDims(4, 4, 0, 13, KV, D, CTX, THETA))
