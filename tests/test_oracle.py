"""Pins the CPU oracle (oracle/eg_oracle.c) before anything is compared against it.

Each check is something other than the oracle's own formula retyped: a real JS engine's output
(tests/golden/js_vectors.json), a known answer taken from the reference's tests, a closed form,
a brute force, or numpy/torch. CPU only.
"""

import json
import math
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def js():
    with open(os.path.join(GOLDEN, "js_vectors.json")) as f:
        return json.load(f)


# ---- RNG ---------------------------------------------------------------------------------


def test_mulberry32_matches_javascript(js):
    for seed, seq in js["mulberry32"].items():
        np.testing.assert_array_equal(oracle.mulberry32_sequence(int(seed), 16), np.array(seq))


def test_random_floats_match_float32array_rounding(js):
    for seed, bits in js["random_floats"].items():
        got = oracle.random_floats(32, int(seed)).view(np.uint32)
        np.testing.assert_array_equal(got, np.array(bits, dtype=np.uint32))


def test_random_floats_range():
    v = oracle.random_floats(100000, 3)
    assert v.min() >= -0.5 and v.max() < 0.5
    assert abs(float(v.mean())) < 0.01


def test_normal_floats_moments():
    v = oracle.normal_floats(200000, 7, sigma=0.02).astype(np.float64)
    assert abs(v.mean()) < 3 * 0.02 / math.sqrt(v.size)
    assert abs(v.std() / 0.02 - 1.0) < 0.01


# ---- reference int4 quantizer (quant.ts:24-74) ------------------------------------------


def test_quantizer_matches_javascript(js):
    for case in js["quantize"]:
        values = np.array(case["values"], dtype=np.uint32).view(np.float32)
        q = oracle.quantize_q4_ref(values, case["rows"], case["cols"], case["blockSize"])
        np.testing.assert_array_equal(q.packed, np.array(case["packed"], dtype=np.uint32), case["name"])
        np.testing.assert_array_equal(q.scales.view(np.uint32), np.array(case["scales"], dtype=np.uint32))
        np.testing.assert_array_equal(q.zeros, np.array(case["zeros"], dtype=np.uint32))


def test_constant_block_recovered_exactly():
    # matmul_q4.test.ts:97-102
    q = oracle.quantize_q4_ref(np.full(64, 0.375, np.float32), 1, 64)
    back = oracle.dequantize(q)
    assert np.all(np.abs(back - 0.375) < 5e-7)


def test_block_endpoints_recovered_exactly():
    # matmul_q4.test.ts:104-113
    values = oracle.random_floats(64, 5)
    values[3] = -1.25
    values[40] = 2.5
    back = oracle.dequantize(oracle.quantize_q4_ref(values, 1, 64))
    assert abs(back[0, 3] + 1.25) < 5e-6
    assert abs(back[0, 40] - 2.5) < 5e-6


def test_error_within_half_step():
    # matmul_q4.test.ts:115-126
    values = oracle.random_floats(64 * 20, 6)
    q = oracle.quantize_q4_ref(values, 20, 64)
    back = oracle.dequantize(q).reshape(-1)
    step = np.repeat(q.scales.astype(np.float64), 64)
    assert np.all(np.abs(back - values) <= step / 2 + 1e-6)


def test_blocks_beat_per_tensor():
    # matmul_q4.test.ts:128-146
    values = oracle.random_floats(128, 7) * np.float32(0.01)
    values[0] = 100
    blocked = oracle.dequantize(oracle.quantize_q4_ref(values, 2, 64, 64)).reshape(-1)
    per_tensor = oracle.dequantize(oracle.quantize_q4_ref(values, 1, 128, 128)).reshape(-1)
    rms = lambda a: math.sqrt(float(np.mean((a[64:] - values[64:]) ** 2)))
    assert rms(blocked) < rms(per_tensor) / 10


def test_halfway_codes_round_up_like_math_round():
    # values 0..15 at scale 1: 2.5 -> 3, 0.5 -> 1 (half up), unlike numpy's ties-to-even.
    v = np.zeros(64, np.float32)
    v[1] = 15
    v[2] = 2.5
    v[3] = 0.5
    q = oracle.quantize_q4_ref(v, 1, 64)
    assert q.scales[0] == 1.0
    codes = [(q.packed[0] >> (4 * i)) & 0xF for i in range(4)]
    assert codes == [0, 15, 3, 1]


# ---- quantize.py restatement (int4 / int8, float32 + rint) ------------------------------


@pytest.mark.parametrize("bits", [4, 8])
def test_blocks_n_endpoints_and_error(bits):
    levels = (1 << bits) - 1
    values = oracle.random_floats(64 * 32, 17)
    q = oracle.quantize_blocks_n(values, 32, 64, bits)
    per = 32 // bits
    codes = ((q.packed[:, None] >> (np.arange(per, dtype=np.uint32) * bits)) & levels).reshape(32, 64)
    v = values.reshape(32, 64)
    assert np.all(codes[np.arange(32), v.argmin(axis=1)] == 0)
    assert np.all(codes[np.arange(32), v.argmax(axis=1)] == levels) or bits == 4  # zero rounding may shift max
    back = oracle.dequantize(q)
    assert np.all(np.abs(back - v) <= q.scales[:, None].astype(np.float64) / 2 * (1 + 1e-5) + 1e-7)


def test_blocks_n_ties_to_even():
    v = np.zeros(64, np.float32)
    v[1] = 15
    v[2] = 2.5
    v[3] = 0.5
    q = oracle.quantize_blocks_n(v, 1, 64, 4)
    codes = [(q.packed[0] >> (4 * i)) & 0xF for i in range(4)]
    assert codes == [0, 15, 2, 0]


def test_blocks_n_degenerate_blocks():
    # DECISIONS.md:522-530: constant block c -> scale |c|/levels; all-zero block -> scale 1.
    v = np.concatenate([np.full(64, 0.375, np.float32), np.zeros(64, np.float32),
                        np.full(64, -2.0, np.float32)])
    q = oracle.quantize_blocks_n(v, 3, 64, 8)
    assert q.scales[0] == np.float32(np.float32(0.375) / np.float32(255))
    assert q.scales[1] == 1.0
    back = oracle.dequantize(q)
    assert np.allclose(back[0], 0.375, atol=1e-6)
    assert np.all(back[1] == 0)
    assert np.allclose(back[2], -2.0, atol=1e-5)


# ---- BASELINE symmetric formats ----------------------------------------------------------


def test_sym_int4_absmax_maps_to_seven():
    v = oracle.normal_floats(32 * 8, 3, 0.02)
    q = oracle.quantize_sym(v, 8, 32, 4, 32)
    assert np.all(q.scales == (np.abs(v.reshape(8, 32)).max(axis=1) / np.float32(7)).astype(np.float32))
    back = oracle.dequantize(q)
    vv = v.reshape(8, 32)
    i = np.abs(vv).argmax(axis=1)
    assert np.all(np.abs(back[np.arange(8), i]) == q.scales.astype(np.float64) * 7)
    assert np.all(np.abs(back - vv) <= q.scales[:, None].astype(np.float64) / 2 * (1 + 1e-6))


def test_sym_int4_packing_low_nibble_first():
    # group of 32 with absmax 7 at scale 1: codes -7..7 written as two's complement nibbles.
    v = np.array([(i % 15) - 7 for i in range(32)], np.float32)
    q = oracle.quantize_sym(v, 1, 32, 4, 32)
    assert q.scales[0] == 1.0
    b = q.packed.view(np.uint8)
    for j in range(16):
        assert b[j] & 0xF == int(v[2 * j]) & 0xF
        assert b[j] >> 4 == int(v[2 * j + 1]) & 0xF


def test_sym_zero_group_and_int8_rows():
    v = np.zeros(64, np.float32)
    q = oracle.quantize_sym(v, 1, 64, 4, 32)
    assert np.all(q.scales == 1.0) and np.all(q.packed == 0)
    rows = oracle.normal_floats(4 * 896, 9, 0.02).reshape(4, 896)
    q8 = oracle.quantize_sym(rows, 4, 896, 8, 896)
    assert np.all(q8.scales == (np.abs(rows).max(axis=1) / np.float32(127)).astype(np.float32))
    back = oracle.dequantize(q8)
    assert np.all(np.abs(back - rows) <= q8.scales[:, None].astype(np.float64) / 2 * (1 + 1e-6))


# ---- dequant brute force ------------------------------------------------------------------


def test_dequant_all_nibbles_and_zeros():
    from oracle import QuantizedMatrix
    for zero in range(16):
        packed = np.array([0x76543210, 0xFEDCBA98], np.uint32)
        q = QuantizedMatrix(1, 16, 16, 4, oracle.ENC_OFFSET_ZEROS, packed, np.array([0.5], np.float32),
                            np.array([zero], np.uint32))
        for col in range(16):
            assert oracle.dequant_element(q, 0, col) == (col - zero) * 0.5
    qs = QuantizedMatrix(1, 16, 16, 4, oracle.ENC_SIGNED, np.array([0x76543210, 0xFEDCBA98], np.uint32),
                         np.array([0.5], np.float32), None)
    for col in range(16):
        assert oracle.dequant_element(qs, 0, col) == (col if col < 8 else col - 16) * 0.5


def test_dequant_all_int8_codes():
    from oracle import QuantizedMatrix
    codes = np.arange(256, dtype=np.uint32)
    packed = (codes.reshape(64, 4) << (np.arange(4, dtype=np.uint32) * 8)).sum(axis=1).astype(np.uint32)
    for zero in (0, 77, 128, 255):
        q = QuantizedMatrix(1, 256, 256, 8, oracle.ENC_OFFSET_ZEROS, packed, np.array([0.25], np.float32),
                            np.array([zero], np.uint32))
        assert np.array_equal(oracle.dequantize(q)[0], (codes.astype(np.float64) - zero) * 0.25)
        assert oracle.dequant_element(q, 0, 200) == (200 - zero) * 0.25
    qs = QuantizedMatrix(1, 256, 256, 8, oracle.ENC_SIGNED, packed, np.array([0.25], np.float32), None)
    signed = np.where(codes >= 128, codes.astype(np.int64) - 256, codes)
    assert np.array_equal(oracle.dequantize(qs)[0], signed * 0.25)


# ---- GEMV ---------------------------------------------------------------------------------


def test_linear_matches_javascript(js):
    for case in js["linear"]:
        m, n, k = case["m"], case["n"], case["k"]
        x = oracle.random_floats(m * k, case["x_seed"])
        q = oracle.quantize_q4_ref(oracle.random_floats(n * k, case["w_seed"]), n, k, 64)
        bias = None if case["bias_seed"] is None else oracle.random_floats(n, case["bias_seed"])
        y = oracle.linear_q(x, q, bias, m)
        np.testing.assert_array_equal(y.view(np.uint32), np.array(case["out"], dtype=np.uint32), case["name"])


def test_linear_writes_at_out_offset():
    # matmul_q4.test.ts:181-195
    k = 64
    q = oracle.quantize_q4_ref(np.full(2 * k, 0.5, np.float32), 2, k)
    out = np.zeros(6, np.float32)
    oracle.linear_q(np.ones(k, np.float32), q, None, 1, out=out, out_stride=6, out_offset=4)
    assert out[0] == 0
    assert abs(out[4] - 32) < 1e-3 and abs(out[5] - 32) < 1e-3


def test_linear_agrees_with_float64_matmul_and_is_linear():
    n, k = 48, 256
    x = oracle.random_floats(3 * k, 2)
    q = oracle.quantize_sym(oracle.normal_floats(n * k, 4, 0.02), n, k, 4, 32)
    y = oracle.linear_q(x, q, None, 3)
    ref = (x.astype(np.float64).reshape(3, k) @ oracle.dequantize(q).T).astype(np.float32).reshape(-1)
    np.testing.assert_allclose(y, ref, rtol=2e-7, atol=1e-9)
    y2 = oracle.linear_q(x * np.float32(2), q, None, 3)
    np.testing.assert_array_equal(y2, y * np.float32(2))
    np.testing.assert_array_equal(oracle.linear_q_fast(x, q, None, 3), y)


def test_bf16_and_f16_rounding_match_library_conversions():
    torch = pytest.importorskip("torch")
    v = np.concatenate([oracle.normal_floats(4096, 5, 3.0), np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9,
                                                                       -2.5, 65504.0, 1e-6], np.float32)])
    bf = torch.from_numpy(v).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(np.array([oracle.bf16_round(float(a)) for a in v], np.float32), bf)
    assert np.array_equal(oracle.bf16_round_array(v), bf)
    f16 = v.astype(np.float16).astype(np.float32)
    assert np.array_equal(np.array([oracle.f16_round(float(a)) for a in v], np.float32), f16)


def test_bf16_model_equals_exact_model_on_bf16_inputs():
    # x on the bf16 grid and weights whose dequantized values are bf16-exact -> no rounding.
    n, k = 16, 64
    x = oracle.bf16_round_array(oracle.random_floats(2 * k, 8))
    v = np.array([((i * 7) % 15) - 7 for i in range(n * k)], np.float32) * np.float32(0.125)
    q = oracle.quantize_sym(v, n, k, 4, 32)
    a = oracle.linear_q_bf16(x, q, None, 2)
    b = oracle.linear_q(x, q, None, 2)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(oracle.linear_q_bf16_fast(x, q, None, 2), a)


# ---- argmax -------------------------------------------------------------------------------


def test_argmax_full_vocabulary_known_answer():
    # forward_ops.test.ts:397-421
    logits = oracle.random_floats(151936, 101)
    logits[123456] = 99
    assert oracle.argmax(logits) == 123456
    assert oracle.argmax_wgsl(logits) == 123456


def test_argmax_ties_to_lowest_index():
    # forward_ops.test.ts:423-446
    logits = np.full(2048, -1, np.float32)
    logits[100] = 5
    logits[900] = 5
    assert oracle.argmax(logits) == 100
    assert oracle.argmax_wgsl(logits) == 100


def test_argmax_matches_numpy():
    for seed in range(5):
        v = oracle.random_floats(10007, 200 + seed)
        assert oracle.argmax(v) == int(np.argmax(v)) == oracle.argmax_wgsl(v)


# ---- sampler (properties only: the reference has no CPU sampler) -------------------------


def _logits(seed, vocab=4096, scale=3.0):
    return oracle.normal_floats(vocab, seed, scale)


def test_sample_greedy_is_argmax():
    for seed in range(4):
        l = _logits(seed)
        tok, info, _ = oracle.sample(l, np.zeros(0, np.uint32), 0.0, 1.0, 1.0, 0.5)
        assert tok == int(np.argmax(l)) and info.greedy == 1
    l = np.full(1000, -3, np.float32)
    l[10] = l[700] = 2.0
    assert oracle.sample(l, np.zeros(0, np.uint32), 0.0, 0.9, 1.0, 0.3)[0] == 10


def test_sample_low_temperature_is_greedy():
    # session.test.ts:292-309: T=0.01, topP=1 picks the argmax
    for seed in range(4):
        l = _logits(10 + seed)
        l[int(np.argmax(l))] += 1.0  # a top-2 gap of >= 1 is 100 temperatures: a point mass
        for r in (1e-6, 0.37, 0.999):
            assert oracle.sample(l, np.zeros(0, np.uint32), 0.01, 1.0, 1.0, r)[0] == int(np.argmax(l))


def test_sample_zero_draw_takes_first_kept_id():
    # sample.wgsl:277 and :309-321: target = random * kept is 0 when random is 0, and the first
    # kept id in ascending order already satisfies running >= 0.
    l = _logits(3)
    assert oracle.sample(l, np.zeros(0, np.uint32), 0.01, 1.0, 1.0, 0.0)[0] == 0


def test_penalty_is_a_set_with_sign_rule():
    l = _logits(21, 2000)
    history = np.array([5, 17, 5, 1999, 17, 3000, 0], np.uint32)  # repeats and an id >= vocab
    _, _, penalized = oracle.sample(l, history, 0.0, 1.0, 1.3, 0.5)
    expect = l.copy()
    for i in sorted(set(int(h) for h in history)):
        if i < l.size:
            expect[i] = expect[i] / np.float32(1.3) if expect[i] > 0 else expect[i] * np.float32(1.3)
    np.testing.assert_array_equal(penalized, expect)


def _float64_nucleus(l, temperature, top_p):
    """Independent float64 statement of the nucleus: exact masses, the same 32-step f32 mids."""
    s = l.astype(np.float64) / temperature
    p = np.exp(s - s.max())
    p = p / p.sum()
    lo, hi = np.float32(0), np.float32(1)
    for _ in range(32):
        mid = np.float32((lo + hi) * np.float32(0.5))
        mass = p[p >= mid].sum()
        if mass < top_p:
            hi = mid
        else:
            lo = mid
    return p, float(lo)


def test_sample_nucleus_and_draw_against_float64():
    checked = 0
    for seed in range(12):
        l = _logits(40 + seed, 3000, 2.0)
        r = oracle.Mulberry32Stream(seed)()
        tok, info, _ = oracle.sample(l, np.zeros(0, np.uint32), 0.7, 0.9, 1.0, r)
        assert info.kept >= 0.9 - 1e-5
        p, thr = _float64_nucleus(l, 0.7, 0.9)
        if info.bisect_margin < 1e-5 or info.threshold_gap < 1e-5:
            continue  # a decision within rounding of its boundary: not comparable
        kept = p >= thr
        assert kept.sum() == info.kept_count
        assert p[tok] >= thr
        target = r * p[kept].sum()
        cum = np.cumsum(np.where(kept, p, 0.0))
        expect = int(np.searchsorted(cum, target, side="left"))
        if info.draw_margin > 1e-5:
            assert tok == expect
            checked += 1
    assert checked >= 8


def test_sample_agrees_with_float64_statement_on_flat_logits():
    # BASELINE config-2-like flat logits: the f32 oracle and exact float64 masses pick the same
    # token whenever the oracle's margins clear its own rounding (~5e-7 relative).
    import cases
    l = oracle.normal_floats(cases.VOCAB, 77, 0.6)
    hist = oracle.random_ids(512, 3, cases.VOCAB)
    rng = oracle.Mulberry32Stream(0x5EED)
    compared = 0
    for _ in range(8):
        r = rng()
        tok, info, _ = oracle.sample(l, hist, 0.7, 0.9, 1.1, r)
        ex, bm, dm = cases.exact_sample(l, hist, 0.7, 0.9, 1.1, r)
        if info.bisect_margin > 2e-6 and info.draw_margin > 2e-6:
            assert tok == ex
            compared += 1
    assert compared >= 3


def test_sample_seeded_reproducible_and_varies():
    l = _logits(77, 3000, 1.0)
    h = np.zeros(0, np.uint32)
    a = [oracle.sample(l, h, 0.9, 0.9, 1.0, oracle.Mulberry32Stream(1)())[0] for _ in range(2)]
    assert a[0] == a[1]
    draws = {oracle.sample(l, h, 0.9, 0.9, 1.0, u)[0] for u in np.linspace(0.05, 0.95, 10)}
    assert len(draws) > 5


def test_sample_top_p_one_keeps_everything():
    l = _logits(5, 1000, 1.0)
    _, info, _ = oracle.sample(l, np.zeros(0, np.uint32), 0.7, 1.0, 1.0, 0.5)
    assert info.threshold == 0.0 and info.kept_count == 1000


# ---- decode-step ops ----------------------------------------------------------------------


def test_rmsnorm_uses_mean_of_squares():
    x = np.array([2.0, 2.0, 2.0, 2.0], np.float32)
    w = np.array([1.0, 0.5, 2.0, -1.0], np.float32)
    y = oracle.rmsnorm(x, w, 1, 4, 1e-6)
    np.testing.assert_allclose(y, w * (2.0 / math.sqrt(4.0 + 1e-6)), rtol=1e-7)


def test_rope_half_rotation():
    head_dim, theta = 64, 1e6
    x = oracle.random_floats(2 * head_dim, 3)
    assert np.array_equal(oracle.rope(x, 1, 2, head_dim, theta, 0), x)  # position 0 unrotated
    e = np.zeros(head_dim, np.float32)
    e[5] = 1.0
    y = oracle.rope(e, 1, 1, head_dim, theta, 100)
    f = 1.0 / theta ** (10 / head_dim)
    assert abs(y[5] - math.cos(100 * f)) < 1e-6 and abs(y[5 + 32] - math.sin(100 * f)) < 1e-6
    assert np.count_nonzero(y) == 2
    z = oracle.rope(x, 1, 2, head_dim, theta, 1234)
    assert abs(np.linalg.norm(z) - np.linalg.norm(x)) < 1e-5
