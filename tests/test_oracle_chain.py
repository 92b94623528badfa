"""Pins oracle/chain.py, the prompt chain with the matrix-core path's roundings.

* Structure: with the operand roundings off, the chain over a prompt equals OracleDecoder
  stepping the same prompt one position at a time (itself pinned by tests/test_decode_oracle.py):
  logits of the last row and every cache row. A wrong RoPE position, a causal mask off by one, a
  dropped residual or a mis-wired projection breaks it.
* Operand roundings: the chain's projection with bf16 operands against eo_linear_q_bf16, the C
  statement of the bf16 GEMM model (itself pinned by tests/test_oracle.py); a one-key attention
  returns the value row exactly whatever the f16 rounding (its single weight is exp(0) = 1); and
  the rounded chain differs from the unrounded one by a bf16-sized amount, not zero and not more.
"""

import numpy as np
import pytest

import oracle
from oracle.chain import _attention, _linear, _Weights, prefill_chain
from oracle.decode import OracleDecoder, f16_array


@pytest.fixture(scope="module", params=["sym", "reference"])
def tiny(request):
    from enargeia_amd.model import ModelConfig, synthetic_model
    cfg = ModelConfig(layers=2, hidden=128, heads=4, kv_heads=2, head_dim=32, intermediate=256, vocab=512,
                      max_context=200, group=64 if request.param == "reference" else 32)
    return synthetic_model(cfg, fmt=request.param)


def caches(cfg, seed, filled):
    rng = np.random.default_rng(seed)
    shape = (cfg.layers, cfg.max_context, cfg.kv_heads, cfg.head_dim)
    k = np.zeros(shape, np.float32)
    v = np.zeros(shape, np.float32)
    k[:, :filled] = f16_array(rng.standard_normal((cfg.layers, filled, cfg.kv_heads, cfg.head_dim)))
    v[:, :filled] = f16_array(rng.standard_normal((cfg.layers, filled, cfg.kv_heads, cfg.head_dim)))
    return k, v


@pytest.mark.parametrize("begin,n,chunk,cus", [(0, 9, 256, 256), (5, 7, 256, 256), (0, 1, 256, 256),
                                             (3, 17, 5, 256), (0, 150, 256, 256), (40, 150, 256, 2)])
def test_unrounded_chain_equals_the_stepped_decoder(tiny, begin, n, chunk, cus):
    """Also in chunks of 5 rows, over several key tiles (150 keys) and split into key ranges (a
    2-CU device splits at 8 tiles and more: 190 keys here, 3 tiles, so no split; 150 queries
    over 4 heads leaves 2 CUs busy)."""
    c = tiny.cfg
    prompt = [int(t) for t in oracle.random_ids(n, 40 + n, c.vocab)]
    k, v = caches(c, begin + 1, begin)
    ora = OracleDecoder(tiny, max_context=c.max_context)
    ora.k[:], ora.v[:] = k, v
    for i, t in enumerate(prompt):
        want = ora.step(t, begin + i)
    got = prefill_chain(tiny, prompt, begin, k, v, rounding="none", chunk=chunk, cu_count=cus)
    scale = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    # the stepped decoder scales the scores by 1/sqrt(D) in float64, the chain scales q in f32
    # as the device does: differences in the last f32 bits, ~1e-5 x rms after two layers
    assert np.abs(got - want).max() <= 1e-4 * scale
    # cache rows: f16 values of the same f32 keys and values (a one-ulp f16 difference where the
    # f32 projections differ in their last bits)
    rows = slice(begin, begin + n)
    for mine, theirs in ((k, ora.k), (v, ora.v)):
        np.testing.assert_allclose(mine[:, rows], theirs[:, rows], rtol=2e-3, atol=1e-5)
        np.testing.assert_array_equal(mine[:, :begin], theirs[:, :begin])


def test_chain_projection_is_the_c_bf16_gemm(tiny):
    L = tiny.layers[0]
    x = oracle.normal_floats(3 * tiny.cfg.hidden, 5).reshape(3, -1)
    for name in ("q", "gate"):
        q = L.mats[name]
        bias = L.biases.get(name)
        got = _linear(x, q, bias, _Weights("device"), oracle.bf16_round_array)
        m = oracle.QuantizedMatrix(q.rows, q.cols, q.block_size, q.bits, q.encoding, q.packed, q.scales, q.zeros)
        want = oracle.linear_q_bf16(x, m, bias, 3).reshape(3, -1)
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)


def test_one_key_attention_returns_the_value_row():
    rng = np.random.default_rng(3)
    heads, kv_heads, d = 4, 2, 32
    k = f16_array(rng.standard_normal((8, kv_heads, d)))
    v = f16_array(rng.standard_normal((8, kv_heads, d)))
    q = f16_array(rng.standard_normal((1, heads * d)))
    out = _attention(q, k, v, 0, heads, kv_heads, d, f16_array).reshape(heads, d)
    for h in range(heads):
        np.testing.assert_array_equal(out[h], v[0, h // 2])


def test_rounded_chain_differs_by_a_bf16_amount(tiny):
    c = tiny.cfg
    prompt = [int(t) for t in oracle.random_ids(9, 77, c.vocab)]
    k0, v0 = caches(c, 1, 0)
    k1, v1 = caches(c, 1, 0)
    a = prefill_chain(tiny, prompt, 0, k0, v0, rounding="none").astype(np.float64)
    b = prefill_chain(tiny, prompt, 0, k1, v1, rounding="device").astype(np.float64)
    rel = np.abs(a - b).max() / np.sqrt(np.mean(a * a))
    assert 1e-5 < rel < 5e-2, rel


def test_split_attention_equals_the_unsplit_one():
    """The key-split walk and merge against one walk over all keys (no rounding: equal to f64
    summation order), at a split the device makes: 2 query rows at position 1000 of 14 heads
    take 16 tiles in 4 splits."""
    from oracle.chain import attention_splits
    rng = np.random.default_rng(5)
    heads, kv_heads, d, begin, n = 14, 2, 64, 1000, 2
    assert attention_splits(n, begin + n, heads) == 4
    k = f16_array(rng.standard_normal((begin + n, kv_heads, d)))
    v = f16_array(rng.standard_normal((begin + n, kv_heads, d)))
    q = (rng.standard_normal((n, heads * d)) / 8).astype(np.float32)
    split = _attention(q, k, v, begin, heads, kv_heads, d, lambda a: np.asarray(a, np.float32))
    whole = _attention(q, k, v, begin, heads, kv_heads, d, lambda a: np.asarray(a, np.float32), cu_count=1)
    np.testing.assert_allclose(split, whole, rtol=1e-5, atol=1e-6)
    from oracle.decode import attention
    for i in range(n):
        ref = attention(q[i] * 8, k[:begin + i + 1], v[:begin + i + 1], heads, kv_heads, d)
        np.testing.assert_allclose(split[i], ref, rtol=1e-4, atol=1e-5)
