"""The decode step on the GPU against the CPU oracle: the fused attention (RoPE, f16 cache append,
split-K partials, combine), the GEMV input stages (RMSNorm, SiLU*up, attention combine), and
the whole decoder (reference-shaped model) step by step, eager and as a replayed hipGraph.

Tolerances: attention output and input stages within 1e-5 x rms + 2e-5 relative (f32 vs the
oracle's float64, one exp per score); decoder logits within 2e-3 x rms(logits) absolute (24
layers of f32 GEMVs over the same int4 weights, f16 cache rows that may round one ulp apart),
and greedy tokens identical wherever the oracle's top-2 gap exceeds 1e-2 x rms(logits)."""

import ctypes

import numpy as np
import pytest

from conftest import assert_close
from enargeia_amd import _lib
from enargeia_amd import kernels as K
from enargeia_amd.model import (INPUT_ATTENTION, INPUT_RMSNORM, INPUT_SILU_MUL, INPUT_VECTOR, Decoder, DeviceModel,
                                GemvInput, ModelConfig, attention_dims, synthetic_model)
from enargeia_amd.quant import normal, quantize_asym, quantize_sym
from oracle import rope as oracle_rope
from oracle.decode import OracleDecoder, attention, f16_array

pytestmark = pytest.mark.gpu

ATT_TOL = (1e-5, 2e-5)  # x rms, relative


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def lib():
    return _lib.load()


# ---- fused attention ---------------------------------------------------------------------------


def run_attention(device, cfg, pos, seed=0, chunk=128, cache="f16"):
    """q/k/v and a cache whose rows [0, pos) are random (f16, or f32 for cache="f32", through
    eg_attention_decode_f32); returns (out, k_cache, v_cache, inputs)."""
    rng = np.random.default_rng(seed)
    H, KV, D, T = cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.max_context
    q = rng.standard_normal(H * D).astype(np.float32)
    k = rng.standard_normal(KV * D).astype(np.float32)
    v = rng.standard_normal(KV * D).astype(np.float32)
    ct = np.float16 if cache == "f16" else np.float32
    kc = np.zeros((T, KV, D), ct)
    vc = np.zeros((T, KV, D), ct)
    kc[:pos] = rng.standard_normal((pos, KV, D)).astype(ct)
    vc[:pos] = rng.standard_normal((pos, KV, D)).astype(ct)
    raw = (lambda a: a.view(np.uint16)) if cache == "f16" else (lambda a: a)
    dims = attention_dims(cfg, chunk)
    bufs = dict(q=device.upload(q), k=device.upload(k), v=device.upload(v), kc=device.upload(raw(kc)),
                vc=device.upload(raw(vc)), pos=device.upload(np.array([pos], np.uint32)),
                part=device.buffer(KV * (T // chunk) * (H // KV) * (D + 2) * 4), out=device.buffer(H * D * 4),
                fused=device.buffer(H * D * 4), counter=device.upload(np.zeros(1, np.uint32)))
    vp = ctypes.c_void_p
    fn = lib().eg_attention_decode if cache == "f16" else lib().eg_attention_decode_f32
    _lib.check(fn(device.ctx, vp(bufs["pos"].ptr), vp(bufs["q"].ptr), vp(bufs["k"].ptr), vp(bufs["v"].ptr),
                  vp(bufs["kc"].ptr), vp(bufs["vc"].ptr), vp(bufs["part"].ptr), vp(bufs["counter"].ptr),
                  vp(bufs["fused"].ptr), ctypes.byref(dims)), device.ctx)
    _lib.check(lib().eg_attention_combine(device.ctx, vp(bufs["part"].ptr), vp(bufs["out"].ptr), ctypes.byref(dims)),
               device.ctx)
    out = device.read_array(bufs["out"], np.float32, H * D)
    # the last workgroup's combine equals the standalone combine bit for bit, and leaves the
    # counter at 0 for the next launch
    np.testing.assert_array_equal(device.read_array(bufs["fused"], np.float32, H * D), out)
    assert device.read_array(bufs["counter"], np.uint32, 1)[0] == 0
    if cache == "f16":
        kc_after = device.read_array(bufs["kc"], np.uint16, T * KV * D).view(np.float16).reshape(T, KV, D)
        vc_after = device.read_array(bufs["vc"], np.uint16, T * KV * D).view(np.float16).reshape(T, KV, D)
    else:
        kc_after = device.read_array(bufs["kc"], np.float32, T * KV * D).reshape(T, KV, D)
        vc_after = device.read_array(bufs["vc"], np.float32, T * KV * D).reshape(T, KV, D)
    for b in bufs.values():
        b.release()
    return out, kc_after, vc_after, (q, k, v, kc, vc)


@pytest.mark.parametrize("chunk", [64, 128])
@pytest.mark.parametrize("pos", [0, 1, 5, 63, 64, 127, 128, 129, 1000, 2047])
def test_attention_decode_matches_oracle(device, pos, chunk):
    cfg = ModelConfig()
    out, kc, vc, (q, k, v, kc0, vc0) = run_attention(device, cfg, pos, seed=pos, chunk=chunk)
    H, KV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    qr = oracle_rope(q, 1, H, D, cfg.rope_theta, pos)
    kr = f16_array(oracle_rope(k, 1, KV, D, cfg.rope_theta, pos)).reshape(KV, D)
    vr = f16_array(v).reshape(KV, D)
    # the appended rows (rotated key, value), f16; RoPE's double-precision angle may differ from
    # the host's libm in the last bit, so allow one f16 ulp on the key
    np.testing.assert_array_equal(vc[pos].astype(np.float32), vr)
    np.testing.assert_allclose(kc[pos].astype(np.float32), kr, rtol=2 ** -10, atol=2 ** -24)
    # earlier rows untouched, later rows untouched
    np.testing.assert_array_equal(kc[:pos], kc0[:pos])
    np.testing.assert_array_equal(vc[pos + 1:], vc0[pos + 1:])
    K_all = np.concatenate([kc0[:pos].astype(np.float32), kr[None]], axis=0)
    V_all = np.concatenate([vc0[:pos].astype(np.float32), vr[None]], axis=0)
    want = attention(qr, K_all, V_all, H, KV, D)
    assert_close(out, want, ATT_TOL[0] * rms(want), ATT_TOL[1], label=f"attention pos={pos} chunk={chunk}")


@pytest.mark.parametrize("chunk", [64, 128])
@pytest.mark.parametrize("pos", [0, 1, 63, 64, 128, 129, 1000, 2047])
def test_attention_decode_f32_cache_matches_oracle(device, pos, chunk):
    """The f32 cache variant: the appended value row is v itself and the key row RoPE(k) (one f32
    ulp for the double-precision angle), not their f16 roundings; the output over the exact f32
    rows at the same bar."""
    cfg = ModelConfig()
    out, kc, vc, (q, k, v, kc0, vc0) = run_attention(device, cfg, pos, seed=pos + 7, chunk=chunk, cache="f32")
    H, KV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    qr = oracle_rope(q, 1, H, D, cfg.rope_theta, pos)
    kr = oracle_rope(k, 1, KV, D, cfg.rope_theta, pos).reshape(KV, D)
    np.testing.assert_array_equal(vc[pos], v.reshape(KV, D))
    np.testing.assert_array_max_ulp(kc[pos], kr, maxulp=1)
    assert np.any(f16_array(v) != v)  # an f16 rounding of the row would have shown
    np.testing.assert_array_equal(kc[:pos], kc0[:pos])
    np.testing.assert_array_equal(vc[pos + 1:], vc0[pos + 1:])
    K_all = np.concatenate([kc0[:pos], kr[None]], axis=0)
    V_all = np.concatenate([vc0[:pos], v.reshape(KV, D)[None]], axis=0)
    want = attention(qr, K_all, V_all, H, KV, D)
    assert_close(out, want, ATT_TOL[0] * rms(want), ATT_TOL[1], label=f"f32 attention pos={pos} chunk={chunk}")


def test_attention_rejects_unsupported_shapes(device):
    dims = attention_dims(ModelConfig())
    dims.head_dim = 80
    buf = device.buffer(1 << 16)
    vp = ctypes.c_void_p(buf.ptr)
    st = lib().eg_attention_decode(device.ctx, vp, vp, vp, vp, vp, vp, vp, None, None, ctypes.byref(dims))
    assert st == _lib.EG_ERR_INVALID and b"head_dim" in lib().eg_last_error(device.ctx)
    buf.release()


# ---- GEMV input stages ------------------------------------------------------------------------


def plan_for(device, q, out, bias=None):
    return K.GemvPlan(device, q.cols, q.block_size, [(device.upload(q.packed), device.upload(q.scales), None, bias,
                                                      out, q.rows, 0)])


def launch_input(device, plan, inp):
    _lib.check(lib().eg_gemv_plan_launch_input(device.ctx, plan.handle, ctypes.byref(inp)), device.ctx)


def reference_gemv(q, x):
    import oracle
    return oracle.gemv_threads(x, q, None, 4)


def test_rmsnorm_input_stage(device):
    k, n = 896, 4864
    q = quantize_sym(normal(n * k, 41, 0.02), n, k, 4, 32)
    x = normal(k, 42, 3.0).astype(np.float32)
    w = (1.0 + normal(k, 43, 0.1)).astype(np.float32)
    out = device.buffer(n * 4)
    plan = plan_for(device, q, out)
    xb, wb = device.upload(x), device.upload(w)
    launch_input(device, plan, GemvInput(INPUT_RMSNORM, xb.ptr, wb.ptr, 1e-6))
    got = device.read_array(out, np.float32, n)
    xn = (x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w).astype(np.float32)
    want = reference_gemv(q, xn)
    assert_close(got, want, 1e-5 * rms(want), 1e-3, label="rmsnorm input")


def test_silu_mul_input_stage(device):
    k, n = 4864, 896
    q = quantize_sym(normal(n * k, 51, 0.02), n, k, 4, 32)
    g = normal(k, 52, 2.0).astype(np.float32)
    u = normal(k, 53, 1.0).astype(np.float32)
    out = device.buffer(n * 4)
    plan = plan_for(device, q, out)
    gb, ub = device.upload(g), device.upload(u)
    launch_input(device, plan, GemvInput(INPUT_SILU_MUL, gb.ptr, ub.ptr, 0.0))
    got = device.read_array(out, np.float32, n)
    g64 = g.astype(np.float64)
    want = reference_gemv(q, (g64 / (1 + np.exp(-g64)) * u).astype(np.float32))
    assert_close(got, want, 1e-5 * rms(want), 1e-3, label="silu*up input")


@pytest.mark.parametrize("chunk,max_context,pos", [(64, 2048, 700), (128, 2048, 700), (128, 2048, 2047),
                                                   (128, 512, 300), (128, 256, 130)])
def test_attention_input_stage_equals_combine(device, chunk, max_context, pos):
    """The o projection's input stage must combine the partials exactly as eg_attention_combine:
    32 chunks (the looped statistics), 16 and 4 chunks (the batched ones, chunks % 4 == 0 and
    <= 16), 2 chunks (looped)."""
    cfg = ModelConfig(max_context=max_context)
    rng = np.random.default_rng(7)
    H, KV, D, T = cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.max_context
    dims = attention_dims(cfg, chunk)
    kc = rng.standard_normal((T, KV, D)).astype(np.float16).view(np.uint16)
    bufs = [device.upload(a) for a in (rng.standard_normal(H * D).astype(np.float32),
                                        rng.standard_normal(KV * D).astype(np.float32),
                                        rng.standard_normal(KV * D).astype(np.float32), kc, kc.copy(),
                                        np.array([pos], np.uint32))]
    part = device.buffer(KV * (T // chunk) * (H // KV) * (D + 2) * 4)
    comb = device.buffer(H * D * 4)
    vp = ctypes.c_void_p
    q, k, v, kcb, vcb, pb = bufs
    _lib.check(lib().eg_attention_decode(device.ctx, vp(pb.ptr), vp(q.ptr), vp(k.ptr), vp(v.ptr), vp(kcb.ptr),
                                         vp(vcb.ptr), vp(part.ptr), None, None, ctypes.byref(dims)), device.ctx)
    _lib.check(lib().eg_attention_combine(device.ctx, vp(part.ptr), vp(comb.ptr), ctypes.byref(dims)), device.ctx)
    wq = quantize_sym(normal(H * D * H * D, 61, 0.02), H * D, H * D, 4, 32)
    out_a, out_b = device.buffer(H * D * 4), device.buffer(H * D * 4)
    plan_a, plan_b = plan_for(device, wq, out_a), plan_for(device, wq, out_b)
    launch_input(device, plan_a, GemvInput(INPUT_ATTENTION, part.ptr, None, 0.0, dims))
    plan_b.launch(comb)
    np.testing.assert_array_equal(device.read_array(out_a, np.float32, H * D),
                                  device.read_array(out_b, np.float32, H * D))


# ---- the decoder -------------------------------------------------------------------------------

SMALL = ModelConfig(layers=2, max_context=256)


@pytest.fixture(scope="module")
def small_model():
    return synthetic_model(SMALL)


def prompt_ids(n, vocab, seed=0x5EED):
    import oracle
    return [int(t) for t in oracle.random_ids(n, seed, vocab)]


def check_step(got_logits, want_logits, got_token, label):
    scale = rms(want_logits)
    err = np.abs(got_logits.astype(np.float64) - want_logits)
    assert err.max() <= 2e-3 * scale, f"{label}: logits max error {err.max():.3e} vs rms {scale:.3e}"
    order = np.argsort(want_logits)
    gap = float(want_logits[order[-1]] - want_logits[order[-2]])
    if gap > 1e-2 * scale:
        assert got_token == int(order[-1]), f"{label}: token {got_token} vs oracle {int(order[-1])} (gap {gap:.3e})"
    return gap


def test_decoder_matches_oracle_prompt_then_greedy(device, small_model):
    m = small_model
    dm = DeviceModel(device, m)
    dec = Decoder(dm)
    ora = OracleDecoder(m, max_context=SMALL.max_context)
    prompt = prompt_ids(32, SMALL.vocab)
    checked = 0
    try:
        for pos, tok in enumerate(prompt):
            dec.reset(pos, tok)
            got_token = dec.step()
            want = ora.step(tok, pos)
            check_step(dec.logits(), want, got_token, f"prompt pos {pos}")
            checked += 1
        tok = got_token
        for pos in range(len(prompt), len(prompt) + 16):
            assert dec.position() == pos
            got_token = dec.step()  # the device feeds its own argmax back
            want = ora.step(tok, pos)  # the oracle follows the device's tokens
            check_step(dec.logits(), want, got_token, f"greedy pos {pos}")
            tok = got_token
            checked += 1
    finally:
        dec.close()
        dm.release()
    assert checked == 48


@pytest.mark.parametrize("max_context,prime", [(512, 120), (2048, 1016)])
def test_decoder_long_context_crosses_chunks(device, max_context, prime):
    """The decoder over a primed cache (random f16 rows [0, prime), the same on both sides),
    stepping across a 128-position chunk boundary: 4 chunks at 512 and 16 at 2048 take the
    o projection's batched combine statistics; logits and greedy tokens against the oracle at
    the decoder bar, every step."""
    cfg = ModelConfig(layers=2, max_context=max_context)
    m = synthetic_model(cfg)
    dm = DeviceModel(device, m)
    dec = Decoder(dm)
    ora = OracleDecoder(m, max_context=max_context)
    rng = np.random.default_rng(max_context)
    shape = (cfg.layers, max_context, cfg.kv_heads, cfg.head_dim)
    kf = rng.standard_normal(shape, dtype=np.float32).astype(np.float16)
    vf = rng.standard_normal(shape, dtype=np.float32).astype(np.float16)
    ora.k[:] = kf.astype(np.float32)
    ora.v[:] = vf.astype(np.float32)
    try:
        device.write(dec.buffers.k_cache, kf.view(np.uint16))
        device.write(dec.buffers.v_cache, vf.view(np.uint16))
        device.sync()
        tok = prompt_ids(1, cfg.vocab, max_context)[0]
        dec.reset(prime, tok)
        for pos in range(prime, prime + 16):
            got_token = dec.step()
            check_step(dec.logits(), ora.step(tok, pos), got_token, f"context {max_context} pos {pos}")
            tok = got_token
        assert dec.position() == prime + 16
    finally:
        dec.close()
        dm.release()


def test_decoder_f32_cache_matches_oracle(device, small_model):
    """A decoder created with an f32 KV cache (eg_decoder_create_cache, SessionOptions.cacheDType
    'f32') against the oracle's f32 cache: the prompt stepped position by position, then greedy
    steps, at the decoder bar; the cache holds the steps' rows unrounded (not f16 values) and
    equal to the oracle's within f32 sums' error."""
    m = small_model
    dm = DeviceModel(device, m)
    dec = Decoder(dm, cache="f32")
    ora = OracleDecoder(m, max_context=SMALL.max_context, cache="f32")
    prompt = prompt_ids(24, SMALL.vocab, 0x51)
    try:
        for pos, tok in enumerate(prompt):
            dec.reset(pos, tok)
            got_token = dec.step()
            check_step(dec.logits(), ora.step(tok, pos), got_token, f"f32 cache prompt pos {pos}")
        tok = got_token
        for pos in range(len(prompt), len(prompt) + 12):
            got_token = dec.step()
            check_step(dec.logits(), ora.step(tok, pos), got_token, f"f32 cache greedy pos {pos}")
            tok = got_token
        n = len(prompt) + 12
        L, T, KV, D = SMALL.layers, SMALL.max_context, SMALL.kv_heads, SMALL.head_dim
        for name, ref in (("k", ora.k), ("v", ora.v)):
            buf = dec.buffers.k_cache if name == "k" else dec.buffers.v_cache
            c = device.read_array(buf, np.float32, L * T * KV * D).reshape(L, T, KV, D)
            assert np.count_nonzero(c[:, :n] != f16_array(c[:, :n])) > c[:, :n].size // 2, f"{name}: f16 values"
            np.testing.assert_allclose(c[:, :n], ref[:, :n], rtol=1e-3, atol=1e-4 * np.abs(ref[:, :n]).max())
    finally:
        dec.close()
        dm.release()


def test_decoder_f32_cache_long_context_and_graph(device):
    """An f32 cache primed with random f32 rows [0, 1016) of a 2048 context (16 chunks of the
    split attention), stepping across a chunk boundary against the oracle over the same rows; the
    same steps replayed from a captured graph give the same tokens and logits bit for bit."""
    cfg = ModelConfig(layers=2, max_context=2048)
    m = synthetic_model(cfg)
    dm = DeviceModel(device, m)
    eager, graph = Decoder(dm, cache="f32"), Decoder(dm, cache="f32")
    ora = OracleDecoder(m, max_context=cfg.max_context, cache="f32")
    rng = np.random.default_rng(99)
    shape = (cfg.layers, cfg.max_context, cfg.kv_heads, cfg.head_dim)
    kf = rng.standard_normal(shape, dtype=np.float32)
    vf = rng.standard_normal(shape, dtype=np.float32)
    ora.k[:], ora.v[:] = kf, vf
    prime = 1016
    try:
        for d in (eager, graph):
            device.write(d.buffers.k_cache, kf)
            device.write(d.buffers.v_cache, vf)
        device.sync()
        tok = prompt_ids(1, cfg.vocab, 77)[0]
        eager.reset(prime, tok)
        graph.reset(prime, tok)
        graph.capture()
        for pos in range(prime, prime + 16):
            a, b = eager.step(), graph.step()
            assert a == b, f"pos {pos}: eager {a} graph {b}"
            np.testing.assert_array_equal(eager.logits(), graph.logits())
            check_step(eager.logits(), ora.step(tok, pos), a, f"f32 cache context 2048 pos {pos}")
            tok = a
    finally:
        eager.close()
        graph.close()
        dm.release()


def test_decoder_rejects_unknown_cache_dtype(device, small_model):
    dm = DeviceModel(device, small_model)
    h = ctypes.c_void_p()
    try:
        st = lib().eg_decoder_create_cache(device.ctx, ctypes.byref(dm.desc), 2, ctypes.byref(h))
        assert st == _lib.EG_ERR_INVALID and b"cache dtype 2" in lib().eg_last_error(device.ctx)
        assert not h.value
    finally:
        dm.release()


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_decoder_dense_table_matches_oracle(device, dtype):
    """A tied table stored as it is (--embed-dtype f16 / f32; embedding_variants.ts:26-74): the
    prompt's rows gathered by the prompt chain, each step's next row by the step tail, the head
    with the final norm and the greedy argmax over the table. The prompt through
    eg_decoder_prefill against the oracle stepped position by position (the chain's bf16
    projections: the reference-arithmetic bars of tests/test_gpu_prefill_chain.py), then greedy
    steps at the decoder bar; a captured graph replays the same tokens and logits; sampled steps
    (the head's logits, then the sampler) give ids in range."""
    cfg = ModelConfig(layers=2, max_context=256, vocab=32768)
    m = synthetic_model(cfg, embed_dtype=dtype)
    dm = DeviceModel(device, m)
    dec, graph = Decoder(dm), Decoder(dm)
    ora = OracleDecoder(m, max_context=cfg.max_context)
    prompt = prompt_ids(20, cfg.vocab, 0xD7)
    try:
        tok = dec.prefill(0, prompt)
        for pos, t in enumerate(prompt):
            want = ora.step(t, pos)
        err = np.abs(dec.logits().astype(np.float64) - want).max() / rms(want)
        assert err <= 0.1, f"{dtype} table: prompt logits {err:.3e} x rms from the oracle"
        order = np.argsort(want)
        if want[order[-1]] - want[order[-2]] > 0.2 * rms(want):
            assert tok == int(order[-1])
        # the prompt again through the decode step, position by position (both sides rewrite
        # their cache rows at decode precision), then greedy steps, at the decoder bar
        for pos, t in enumerate(prompt):
            dec.reset(pos, t)
            got_token = dec.step()
            check_step(dec.logits(), ora.step(t, pos), got_token, f"{dtype} table prompt pos {pos}")
        tok = got_token
        for pos in range(len(prompt), len(prompt) + 8):
            got_token = dec.step()
            check_step(dec.logits(), ora.step(tok, pos), got_token, f"{dtype} table greedy pos {pos}")
            tok = got_token
        dec.reset(0, prompt[0])
        graph.reset(0, prompt[0])
        graph.capture()
        for s_ in range(6):
            a, b = dec.step(), graph.step()
            assert a == b, f"{dtype} table step {s_}: eager {a} graph {b}"
            np.testing.assert_array_equal(dec.logits(), graph.logits())
        dec.set_sampling(0.7, 0.9, 1.1)
        for _ in range(4):
            assert 0 <= dec.step() < cfg.vocab
    finally:
        dec.close()
        graph.close()
        dm.release()


def test_decoder_graph_replay_equals_eager(device, small_model):
    dm = DeviceModel(device, small_model)
    eager, graph = Decoder(dm), Decoder(dm)
    try:
        eager.reset(0, 17)
        graph.reset(0, 17)
        graph.capture()
        for step in range(8):
            a, b = eager.step(), graph.step()
            assert a == b, f"step {step}: eager {a} graph {b}"
            np.testing.assert_array_equal(eager.logits(), graph.logits())
        assert graph.position() == 8
    finally:
        eager.close()
        graph.close()
        dm.release()


def test_decoder_full_model_first_steps(device):
    cfg = ModelConfig(max_context=256)
    m = synthetic_model(cfg)
    dm = DeviceModel(device, m)
    dec = Decoder(dm)
    ora = OracleDecoder(m, max_context=cfg.max_context)
    try:
        for pos, tok in enumerate(prompt_ids(4, cfg.vocab, 0x1234)):
            dec.reset(pos, tok)
            got_token = dec.step()
            check_step(dec.logits(), ora.step(tok, pos), got_token, f"24-layer pos {pos}")
    finally:
        dec.close()
        dm.release()


def test_decoder_rejects_bad_reset(device, small_model):
    dm = DeviceModel(device, small_model)
    dec = Decoder(dm)
    try:
        with pytest.raises(_lib.EgRangeError):
            dec.reset(SMALL.max_context, 0)
        with pytest.raises(_lib.EgError):
            dec.reset(0, SMALL.vocab)
    finally:
        dec.close()
        dm.release()


def test_decoder_refuses_calls_inside_a_capture(device, small_model):
    """A step or reset while the context captures would record launches that do not run and
    desynchronise the host's position: both are refused before anything is enqueued."""
    dm = DeviceModel(device, small_model)
    dec = Decoder(dm)
    try:
        dec.reset(3, 17)
        device.capture_begin()
        try:
            with pytest.raises(_lib.EgError) as e:
                dec.step(read_token=False)
            assert e.value.status == _lib.EG_ERR_STATE
            with pytest.raises(_lib.EgError) as e:
                dec.reset(0, 1)
            assert e.value.status == _lib.EG_ERR_STATE
        finally:
            device.capture_end().destroy()
        assert dec.position() == 3
        dec.step()
        assert dec.position() == 4
    finally:
        dec.close()
        dm.release()


def swiglu_plan(device, gate, up, out):
    """eg_gemv_swiglu_plan_create over (gate, up), writing silu(gate . x) * (up . x) to out."""
    table = (K.GemvSegment * 2)()
    keep = []
    for i, q in enumerate((gate, up)):
        bp, bs = device.upload(q.packed), device.upload(q.scales)
        bz = device.upload(q.zeros) if q.zeros is not None else None
        keep += [b for b in (bp, bs, bz) if b is not None]
        table[i] = K.GemvSegment(bp.ptr, bs.ptr, bz.ptr if bz else None, None, out.ptr if i == 0 else None,
                                 q.rows, 0)
    h = ctypes.c_void_p()
    _lib.check(lib().eg_gemv_swiglu_plan_create(device.ctx, gate.cols, gate.block_size, gate.encoding, gate.bits,
                                                table, ctypes.byref(h)), device.ctx)
    return h, keep


@pytest.mark.parametrize("k,n,fmt", [(896, 4864, "sym"), (2048, 512, "sym"), (896, 1024, "offset")])
def test_swiglu_pair_matches_gate_up_plan(device, k, n, fmt):
    """The gate|up pair stores silu(g) * u per row: g and u are the bits a two-matrix plan
    produces (same lane layout and sums), the product the expression of the SiLU input stage;
    checked against the plan's own g and u to a few ulps and against the oracle at the GEMV bar.
    K = 896 takes 32-lane teams, K = 2048 full-wave teams; the reference's offset format too."""
    if fmt == "sym":
        gate = quantize_sym(normal(n * k, 61 + k, 0.02), n, k, 4, 32)
        up = quantize_sym(normal(n * k, 62 + k, 0.02), n, k, 4, 32)
    else:
        gate = quantize_asym(normal(n * k, 63, 0.02), n, k, 4, 64)
        up = quantize_asym(normal(n * k, 64, 0.02), n, k, 4, 64)
    x = normal(k, 65, 2.0).astype(np.float32)
    w = (1.0 + normal(k, 66, 0.1)).astype(np.float32)
    xb, wb = device.upload(x), device.upload(w)
    pair_out, both = device.buffer(n * 4), device.buffer(2 * n * 4)
    h, keep = swiglu_plan(device, gate, up, pair_out)
    inp = GemvInput(INPUT_RMSNORM, xb.ptr, wb.ptr, 1e-6)
    _lib.check(lib().eg_gemv_plan_launch_input(device.ctx, h, ctypes.byref(inp)), device.ctx)
    got = device.read_array(pair_out, np.float32, n)
    segs = []
    for i, q in enumerate((gate, up)):
        bz = device.upload(q.zeros) if q.zeros is not None else None
        segs.append((device.upload(q.packed), device.upload(q.scales), bz, None, both, n, i * n))
    plan = K.GemvPlan(device, k, gate.block_size, segs, encoding=gate.encoding)
    launch_input(device, plan, inp)
    gu = device.read_array(both, np.float32, 2 * n)
    g, u = gu[:n].astype(np.float64), gu[n:].astype(np.float64)
    assert_close(got, g / (1 + np.exp(-g)) * u, 0.0, 4e-7, label="pair vs plan g, u")
    xn = (x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w).astype(np.float32)
    g_ref, u_ref = reference_gemv(gate, xn).astype(np.float64), reference_gemv(up, xn).astype(np.float64)
    want = g_ref / (1 + np.exp(-g_ref)) * u_ref
    assert_close(got, want, 1e-5 * rms(want), 2e-3, label="pair vs oracle")
    _lib.check(lib().eg_gemv_plan_destroy(device.ctx, h), device.ctx)
    plan.destroy()


def test_swiglu_pair_rejects_bad_pairs(device):
    k = 896
    gate = quantize_sym(normal(512 * k, 71, 0.02), 512, k, 4, 32)
    up = quantize_sym(normal(256 * k, 72, 0.02), 256, k, 4, 32)
    out = device.buffer(512 * 4)
    with pytest.raises(K.EgError, match="gate has 512 rows, up 256"):
        swiglu_plan(device, gate, up, out)
    h, _ = swiglu_plan(device, gate, gate, out)
    x = device.upload(normal(k, 73, 1.0).astype(np.float32))
    inp = GemvInput(INPUT_VECTOR, x.ptr, None, 0.0)
    st = lib().eg_gemv_plan_launch_input(device.ctx, h, ctypes.byref(inp))
    assert st == _lib.EG_ERR_INVALID and b"RMSNORM" in lib().eg_last_error(device.ctx)
    _lib.check(lib().eg_gemv_plan_destroy(device.ctx, h), device.ctx)


def test_decode_advance_appends_history_until_capacity(device):
    # eg_decode_advance (Session.decodeStep's bookkeeping, session.ts:347-375): the position
    # moves on every call; the token joins the history while it has room, then the history
    # stays as it is; without a history only the position moves.
    vp = ctypes.c_void_p
    pos = device.upload(np.array([5], np.uint32))
    hist = device.upload(np.array([1, 2, 3, 0], np.uint32))
    hlen = device.upload(np.array([3], np.uint32))
    tok = device.upload(np.array([42], np.uint32))
    try:
        for _ in range(2):
            _lib.check(lib().eg_decode_advance(device.ctx, vp(pos.ptr), vp(hist.ptr), vp(hlen.ptr), vp(tok.ptr), 4),
                       device.ctx)
        assert device.read_array(pos, np.uint32, 1).tolist() == [7]
        assert device.read_array(hist, np.uint32, 4).tolist() == [1, 2, 3, 42]
        assert device.read_array(hlen, np.uint32, 1).tolist() == [4]
        _lib.check(lib().eg_decode_advance(device.ctx, vp(pos.ptr), None, None, vp(tok.ptr), 0), device.ctx)
        assert device.read_array(pos, np.uint32, 1).tolist() == [8]
        st = lib().eg_decode_advance(device.ctx, vp(pos.ptr), vp(hist.ptr), None, vp(tok.ptr), 4)
        assert st == _lib.EG_ERR_INVALID and b"go together" in lib().eg_last_error(device.ctx)
    finally:
        for b in (pos, hist, hlen, tok):
            b.release()
