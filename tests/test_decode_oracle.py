"""Pins the decode-step oracle's own pieces on the CPU: the attention row against closed forms,
the f16 cache rounding, SiLU*mul, and one whole small step against a direct float64
composition of the same operators."""

import numpy as np
import pytest

import oracle
from oracle.decode import OracleDecoder, attention, f16_array, silu_mul


def test_single_position_returns_its_value_row():
    rng = np.random.default_rng(1)
    q = rng.standard_normal(14 * 64).astype(np.float32)
    k = rng.standard_normal((1, 2, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 64)).astype(np.float32)
    out = attention(q, k, v, 14, 2, 64).reshape(14, 64)
    for h in range(14):
        np.testing.assert_array_equal(out[h], v[0, h // 7])


def test_equal_keys_average_the_values():
    rng = np.random.default_rng(2)
    q = rng.standard_normal(4 * 64).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, 1, 64)).astype(np.float32), 9, axis=0)
    v = rng.standard_normal((9, 1, 64)).astype(np.float32)
    out = attention(q, k, v, 4, 1, 64).reshape(4, 64)
    np.testing.assert_allclose(out, np.broadcast_to(v[:, 0].mean(axis=0), (4, 64)), rtol=1e-6, atol=1e-7)


def test_dominant_score_selects_its_row_and_heads_group_contiguously():
    # query head h reads kv head h // (heads / kv_heads): heads 0..6 -> 0, 7..13 -> 1
    head_dim, n = 64, 5
    k = np.zeros((n, 2, head_dim), np.float32)
    v = np.arange(n * 2 * head_dim, dtype=np.float32).reshape(n, 2, head_dim)
    k[3, 0, 0] = 1.0  # kv head 0 matches position 3
    k[1, 1, 1] = 1.0  # kv head 1 matches position 1
    q = np.zeros((14, head_dim), np.float32)
    q[:7, 0] = 1000.0
    q[7:, 1] = 1000.0
    out = attention(q.reshape(-1), k, v, 14, 2, head_dim).reshape(14, head_dim)
    for h in range(7):
        np.testing.assert_allclose(out[h], v[3, 0], rtol=1e-6)
    for h in range(7, 14):
        np.testing.assert_allclose(out[h], v[1, 1], rtol=1e-6)


def test_f16_rounding_is_round_to_nearest_even():
    # 1 + 2^-11 is halfway between 1 and 1 + 2^-10: ties to even gives 1
    assert f16_array(np.array([1 + 2.0 ** -11], np.float32))[0] == 1.0
    assert f16_array(np.array([1 + 3 * 2.0 ** -11], np.float32))[0] == 1 + 2.0 ** -9
    assert f16_array(np.array([65520.0], np.float32))[0] == np.inf


def test_silu_mul_closed_forms():
    g = np.array([0.0, 1.0, -1.0, 20.0], np.float32)
    u = np.array([3.0, 1.0, 2.0, 0.5], np.float32)
    out = silu_mul(g, u)
    assert out[0] == 0.0
    np.testing.assert_allclose(out[1], 1.0 / (1.0 + np.exp(-1.0)), rtol=1e-7)
    np.testing.assert_allclose(out[2], 2.0 * -1.0 / (1.0 + np.exp(1.0)), rtol=1e-7)
    np.testing.assert_allclose(out[3], 0.5 * 20.0, rtol=1e-7)  # silu(x) -> x for large x


@pytest.fixture(scope="module", params=["sym", "reference"])
def tiny_model(request):
    """Both weight formats: the BASELINE ones and the reference quantizer's (asymmetric codes with
    zero-points, non-unit norm weights)."""
    from enargeia_amd.model import ModelConfig, synthetic_model
    cfg = ModelConfig(layers=2, hidden=128, heads=4, kv_heads=2, head_dim=32, intermediate=256, vocab=512,
                      max_context=16, group=64 if request.param == "reference" else 32)
    return synthetic_model(cfg, fmt=request.param)


@pytest.mark.parametrize("fmt", ["sym8_row", "sym4_g32", "asym8_g64", "asym4_g64"])
def test_dequant_row_matches_the_c_dequantizer(fmt):
    """oracle.decode.dequant_row (the embedding gather's row) against oracle.dequantize, the C
    restatement of dequantElement (quant.ts:86-93), for every table format."""
    from enargeia_amd.quant import normal, quantize_asym, quantize_sym
    from oracle.decode import dequant_row
    rows, cols = 24, 192
    w = normal(rows * cols, 91, 0.02)
    q = {"sym8_row": lambda: quantize_sym(w, rows, cols, 8, cols), "sym4_g32": lambda: quantize_sym(w, rows, cols, 4, 32),
         "asym8_g64": lambda: quantize_asym(w, rows, cols, 8, 64),
         "asym4_g64": lambda: quantize_asym(w, rows, cols, 4, 64)}[fmt]()
    full = oracle.dequantize(oracle.QuantizedMatrix(q.rows, q.cols, q.block_size, q.bits, q.encoding, q.packed,
                                                    q.scales, q.zeros))
    for r in (0, 5, rows - 1):
        np.testing.assert_array_equal(dequant_row(q, r), full[r].astype(np.float32))


def test_oracle_step_matches_a_direct_float64_composition(tiny_model):
    """The step against a from-scratch float64 restatement over the dequantized weights: catches
    a wrong operator order, a dropped residual or a mis-wired projection."""
    m = tiny_model
    c = m.cfg
    dec = OracleDecoder(m, cache="f32")
    tokens = [3, 77, 500, 3]

    def deq(q):
        return oracle.dequantize(oracle.QuantizedMatrix(q.rows, q.cols, q.block_size, q.bits, q.encoding,
                                                        q.packed, q.scales, q.zeros)).astype(np.float64)

    W = [{n: deq(q) for n, q in L.mats.items()} for L in m.layers]
    E = deq(m.embedding)
    ks = [[] for _ in range(c.layers)]
    vs = [[] for _ in range(c.layers)]

    def norm(x, w):
        return x / np.sqrt(np.mean(x * x) + c.rms_eps) * w

    def rot(x, heads, pos):
        x = x.reshape(heads, c.head_dim).copy()
        half = c.head_dim // 2
        i = np.arange(half)
        ang = pos / c.rope_theta ** (2 * i / c.head_dim)
        a, b = x[:, :half].copy(), x[:, half:].copy()
        x[:, :half] = a * np.cos(ang) - b * np.sin(ang)
        x[:, half:] = b * np.cos(ang) + a * np.sin(ang)
        return x

    for pos, tok in enumerate(tokens):
        got = dec.step(tok, pos)
        h = E[tok].copy()
        for li, L in enumerate(m.layers):
            xn = norm(h, L.input_norm)
            q = rot(W[li]["q"] @ xn + L.biases["q"], c.heads, pos)
            k = rot(W[li]["k"] @ xn + L.biases["k"], c.kv_heads, pos)
            v = (W[li]["v"] @ xn + L.biases["v"]).reshape(c.kv_heads, c.head_dim)
            ks[li].append(k)
            vs[li].append(v)
            K, V = np.array(ks[li]), np.array(vs[li])
            att = np.empty((c.heads, c.head_dim))
            for hh in range(c.heads):
                kv = hh // (c.heads // c.kv_heads)
                s = K[:, kv] @ q[hh] / np.sqrt(c.head_dim)
                w = np.exp(s - s.max())
                att[hh] = (w / w.sum()) @ V[:, kv]
            h = h + W[li]["o"] @ att.reshape(-1)
            xn = norm(h, L.post_attention_norm)
            g, u = W[li]["gate"] @ xn, W[li]["up"] @ xn
            h = h + W[li]["down"] @ (g / (1 + np.exp(-g)) * u)
        want = E @ norm(h, m.final_norm)
        np.testing.assert_allclose(got, want, rtol=2e-4, atol=2e-5 * np.sqrt(np.mean(want ** 2)))


def test_prefill_attention_closed_forms_and_causality():
    """The oracle's chunked prefill: the first query of an empty cache sees only its own key, so
    its output is its own value row (f16-rounded) for every head of the group; perturbing a later
    row of the chunk changes no earlier output (the causal mask); q_rope is RoPE(q) / sqrt(D)."""
    from oracle.decode import prefill_attention
    H, KV, D, n = 4, 2, 16, 6
    rng = np.random.default_rng(5)
    q = rng.standard_normal((n, H * D), dtype=np.float32)
    k = rng.standard_normal((n, KV * D), dtype=np.float32)
    v = rng.standard_normal((n, KV * D), dtype=np.float32)
    kc = np.zeros((16, KV, D), np.float32)
    vc = np.zeros((16, KV, D), np.float32)
    qr, out = prefill_attention(q, k, v, kc, vc, 0, H, KV, D, 1e4)
    v0 = f16_array(v[0]).reshape(KV, D)
    for h in range(H):
        np.testing.assert_allclose(out[0].reshape(H, D)[h], v0[h // (H // KV)], rtol=0, atol=1e-6)
    np.testing.assert_array_equal(qr[0], (oracle.rope(q[0], 1, H, D, 1e4, 0) * np.float32(0.25)).astype(np.float32))
    k2, v2 = k.copy(), v.copy()
    k2[4] += 3.0
    v2[4] -= 2.0
    _, out2 = prefill_attention(q, k2, v2, np.zeros_like(kc), np.zeros_like(vc), 0, H, KV, D, 1e4)
    np.testing.assert_array_equal(out2[:4], out[:4])
    assert not np.array_equal(out2[4:], out[4:])


def test_prefill_attention_zero_queries_average_the_visible_rows():
    """With q = 0 every score is 0, so query i of a chunk starting at `begin` returns the plain
    mean of the value rows [0, begin + i] of its kv head (cached rows included): a mask that is
    off by one, or a head mapped to the wrong kv head, changes the mean."""
    from oracle.decode import prefill_attention
    H, KV, D, n, begin = 6, 3, 8, 5, 7
    rng = np.random.default_rng(11)
    q = np.zeros((n, H * D), np.float32)
    k = rng.standard_normal((n, KV * D), dtype=np.float32)
    v = rng.standard_normal((n, KV * D), dtype=np.float32)
    kc = f16_array(rng.standard_normal((32, KV, D), dtype=np.float32))
    vc = f16_array(rng.standard_normal((32, KV, D), dtype=np.float32))
    visible = vc.copy()
    visible[begin:begin + n] = f16_array(v).reshape(n, KV, D)
    _, out = prefill_attention(q, k, v, kc, vc, begin, H, KV, D, 1e4)
    for i in range(n):
        mean = visible[:begin + i + 1].astype(np.float64).mean(axis=0)
        for h in range(H):
            np.testing.assert_allclose(out[i].reshape(H, D)[h], mean[h // (H // KV)], rtol=1e-6, atol=1e-7)


def test_prefill_attention_f32_cache_keeps_the_rows_exact():
    """cache="f32" (the reference's f32 cache variant): the appended rows are RoPE(k) and v
    themselves, not f16-rounded, so the first query of an empty cache returns its own value row
    exactly and zero queries return the plain mean of the exact rows (values chosen so that f16
    rounding would move them: an f32 cache that rounds fails both)."""
    from oracle.decode import prefill_attention
    H, KV, D, n, begin = 4, 2, 16, 5, 3
    rng = np.random.default_rng(21)
    q = rng.standard_normal((n, H * D), dtype=np.float32)
    k = rng.standard_normal((n, KV * D), dtype=np.float32)
    v = rng.standard_normal((n, KV * D), dtype=np.float32)
    assert np.any(f16_array(v) != v)
    kc = np.zeros((16, KV, D), np.float32)
    vc = np.zeros((16, KV, D), np.float32)
    _, out = prefill_attention(q, k, v, kc, vc, 0, H, KV, D, 1e4, cache="f32")
    np.testing.assert_array_equal(vc[:n], v.reshape(n, KV, D))
    for i in range(n):
        np.testing.assert_array_equal(kc[i], oracle.rope(k[i], 1, KV, D, 1e4, i).reshape(KV, D))
    for h in range(H):
        np.testing.assert_allclose(out[0].reshape(H, D)[h], v.reshape(n, KV, D)[0, h // (H // KV)], rtol=1e-7, atol=0)
    q0 = np.zeros_like(q)
    kc = rng.standard_normal((16, KV, D), dtype=np.float32)
    vc = rng.standard_normal((16, KV, D), dtype=np.float32)
    visible = vc.copy()
    visible[begin:begin + n] = v.reshape(n, KV, D)
    _, out = prefill_attention(q0, k, v, kc, vc, begin, H, KV, D, 1e4, cache="f32")
    for i in range(n):
        mean = visible[:begin + i + 1].astype(np.float64).mean(axis=0)
        for h in range(H):
            np.testing.assert_allclose(out[i].reshape(H, D)[h], mean[h // (H // KV)], rtol=1e-6, atol=1e-7)


def test_dense_table_packing_known_halves():
    """The f16 table's words (embedding_variants.ts:66-70, unpack2x16float): element 2j in the
    low half. IEEE binary16 bits: 1.0 = 0x3C00, 2.0 = 0x4000, -0.5 = 0xB800, 65504 = 0x7BFF; an
    f32 table keeps each float's own bits."""
    from enargeia_amd.quant import dense_table
    from oracle.decode import dense_values
    v = np.array([1.0, 2.0, -0.5, 65504.0], np.float32)
    t16 = dense_table(v, 1, 4, 16)
    assert t16.packed.tolist() == [0x40003C00, 0x7BFFB800]
    np.testing.assert_array_equal(dense_values(t16)[0], v)
    t32 = dense_table(v, 2, 2, 32)
    assert t32.packed.tolist() == [0x3F800000, 0x40000000, 0xBF000000, 0x477FE000]
    np.testing.assert_array_equal(dense_values(t32), v.reshape(2, 2))


def test_dense_head_closed_forms_and_the_int8_head():
    """lm_head_f16 / lm_head_f32 in the oracle: one-hot rows select x's elements; a table of
    small integers (exact in f16) gives the int8 head's logits over the same integers (scale 1:
    every row's absmax is 127) from the C restatement of linearQ4's loop (quant.ts:95-111);
    dequant_row of a dense table is its row (the gather)."""
    from enargeia_amd.quant import dense_table
    from oracle.decode import dense_head, dense_values, dequant_row
    rng = np.random.default_rng(3)
    k = 64
    x = rng.standard_normal(k).astype(np.float32)
    onehot = np.zeros((8, k), np.float32)
    picks = [(5 * r + 3) % k for r in range(8)]
    onehot[np.arange(8), picks] = 1.0
    for bits in (16, 32):
        np.testing.assert_array_equal(dense_head(x, dense_table(onehot, 8, k, bits)), x[picks])
    ints = rng.integers(-127, 128, size=(16, k)).astype(np.float32)
    ints[:, 0] = 127.0
    q8 = oracle.quantize_sym(ints.reshape(-1), 16, k, 8, k)
    want = oracle.linear_q(x, q8, None, 1)
    got = dense_head(x, dense_table(ints, 16, k, 16))
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)
    t = dense_table(rng.standard_normal((4, k)).astype(np.float32), 4, k, 16)
    for r in range(4):
        np.testing.assert_array_equal(dequant_row(t, r), dense_values(t)[r])
