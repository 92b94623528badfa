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


def run(device, q, k, v, kc16, vc16, begin, dims=None, heads=H, kv_heads=KV):
    """eg_attention_prefill over f16 caches (uint16 arrays), or eg_attention_prefill_f32 where the
    caches given are float32 arrays."""
    n = q.shape[0]
    f32 = kc16.dtype == np.float32
    bq, bk, bv = device.upload(q), device.upload(k), device.upload(v)
    bkc, bvc = device.upload(kc16), device.upload(vc16)
    bqr, bo = device.buffer(q.nbytes), device.buffer(q.nbytes)
    d = dims or PrefillDims(n, begin + n, begin, heads, kv_heads, D, CTX, THETA)
    vp = ctypes.c_void_p
    fn = _lib.load().eg_attention_prefill_f32 if f32 else _lib.load().eg_attention_prefill
    try:
        _lib.check(fn(device.ctx, vp(bq.ptr), vp(bk.ptr), vp(bv.ptr), vp(bkc.ptr), vp(bvc.ptr), vp(bqr.ptr),
                      vp(bo.ptr), ctypes.byref(d)), device.ctx)
        return (device.read_array(bqr, np.float32, q.size).reshape(q.shape),
                device.read_array(bo, np.float32, q.size).reshape(q.shape),
                device.read_array(bkc, kc16.dtype, kc16.size).reshape(kc16.shape),
                device.read_array(bvc, vc16.dtype, vc16.size).reshape(vc16.shape))
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


# the f32 cache variant: tiles of 256 keys; a chunk inside the first tile, one crossing several
# tiles after cached rows, one ending at the context's end; 7 and 8 query heads per kv head
@pytest.mark.parametrize("begin,n,heads,kv_heads", [(0, 64, H, KV), (300, 77, H, KV), (1900, 148, H, KV),
                                                     (5, 1, H, KV), (0, 300, 16, 2), (511, 130, 8, 4)])
def test_prefill_attention_f32_cache_matches_oracle(device, begin, n, heads, kv_heads):
    """eg_attention_prefill_f32: q_rope as the f16 variant's; the appended rows RoPE(k) (one ulp
    for the double-precision angle) and v exactly, f32; the output over the exact rows within
    the decode attention's f32 bar (1e-5 x rms + 2e-5 relative: f32 FMAs and one exp per score
    against float64)."""
    print(f"prefill attention f32 begin {begin} queries {n} heads {heads}/{kv_heads}", flush=True)
    rng = np.random.default_rng(2000 + begin + n)
    q = rng.standard_normal((n, heads * D), dtype=np.float32)
    k = rng.standard_normal((n, kv_heads * D), dtype=np.float32)
    v = rng.standard_normal((n, kv_heads * D), dtype=np.float32)
    kc = rng.standard_normal((CTX, kv_heads, D), dtype=np.float32)
    vc = rng.standard_normal((CTX, kv_heads, D), dtype=np.float32)
    got_qr, got, got_kc, got_vc = run(device, q, k, v, kc.copy(), vc.copy(), begin, heads=heads, kv_heads=kv_heads)
    want_qr, want = prefill_attention(q, k, v, kc, vc, begin, heads, kv_heads, D, THETA, cache="f32")
    np.testing.assert_array_max_ulp(got_qr, want_qr, maxulp=1)
    np.testing.assert_array_max_ulp(got_kc, kc, maxulp=1)
    np.testing.assert_array_equal(got_vc, vc)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got.ravel(), want.ravel(), 1e-5 * rms, 2e-5, label=f"f32 prefill attention begin {begin} n {n}")


def test_prefill_attention_f32_rejects_wide_groups(device):
    q = np.zeros((2, 18 * D), np.float32)
    k = np.zeros((2, 2 * D), np.float32)
    c = np.zeros((CTX, 2, D), np.float32)
    with pytest.raises(_lib.EgError, match="9 query heads per kv head"):
        run(device, q, k, k, c, c, 0, heads=18, kv_heads=2)


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
