"""Sampled decoding inside the decoder and its hipGraph (DecodeGraph's sample step,
graph_decode.ts:382-385, driven as Session.generate drives it, session.ts:347-375, 416-495): the
prompt's last position and then sampled steps whose draw (mulberry32, session.ts:75-83),
history (the prompt plus every produced token, :349-350) and sampling parameters all live on the
device.

Checked every step, against the CPU oracle:
  * the draw the step used equals the oracle's mulberry32 stream from seed 0x5eed, bit for bit;
  * the logits (penalized in place) equal oracle.sample's penalized OracleDecoder logits within
    2e-3 x rms (the decoder bar of test_gpu_decode.py);
  * the token equals oracle.sample (sample.wgsl:143-332) applied to the GPU's own logits wherever
    that sampler's decisions are 2e-6 clear of a boundary (the sampler bar of
    test_gpu_sample.py), and equals oracle.sample on OracleDecoder's logits wherever the decisions
    are clear by 4 x max|logit error| / T (a logit error d moves every p by at most a factor
    e^(2d/T), so masses by at most ~2d/T);
  * the history on the device is the prompt plus every token, in order.
The prompt enters through greedy decode steps (the f32 GEMV path, so the cache rows match the
oracle's at the decoder bar; eg_decoder_prefill's bf16 matrix-core chain has its own tests in
test_gpu_prefill_chain.py), then the session's state is set as runPrefill leaves it (history =
prompt, a fresh draw source) and the last prompt position takes the first draw.
The oracle follows the device's tokens, so one near-boundary draw does not end the comparison.
Random-init logits are nearly flat (rms ~0.6 over 151,936 ids): at T 0.7 every id holds ~1e-5
of the mass, so the end-to-end check rarely clears its margin there and a second run at T 0.1
(a peaked distribution) carries it.
Graph replay is bit-identical to eager steps; GREEDY steps advance the draw state once each
(state = seed + n * 0x6D2B79F5, mulberry32's increment), and a penalty with T = 0 takes the
sampler's greedy path over penalized logits."""

import numpy as np
import pytest

import oracle
from enargeia_amd import _lib
from enargeia_amd.model import Decoder, DeviceModel, ModelConfig, synthetic_model
from enargeia_amd.session import RangeError, Session
from enargeia_amd import kernels as K
from oracle.decode import OracleDecoder

pytestmark = pytest.mark.gpu

SMALL = ModelConfig(layers=2, max_context=256)
LOGIT_TOL = 2e-3
SAMPLER_EPS = 2e-6
T, TOP_P, PENALTY = 0.7, 0.9, 1.1  # the reference's live default (ui/engine.ts:261)


@pytest.fixture(scope="module")
def small_model():
    return synthetic_model(SMALL)


def prompt_ids(n, vocab, seed=0x5EED):
    return [int(t) for t in oracle.random_ids(n, seed, vocab)]


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


class Checker:
    def __init__(self, dec, ora, temperature):
        self.dec, self.ora, self.t = dec, ora, temperature
        self.draws = oracle.Mulberry32Stream(0x5EED)
        self.sampler_compared = self.e2e_compared = 0

    def check(self, token, want_logits, history, label):
        r = np.float32(self.draws())
        sp = self.dec.sample_params()
        assert sp["random"].view(np.uint32) == r.view(np.uint32), f"{label}: draw {sp['random']} vs {r}"
        assert sp["history_length"] == len(history) + 1, f"{label}: history length {sp['history_length']}"
        got = self.dec.logits()  # penalized in place by the sample step
        ref_tok, ref_info, ref_pen = oracle.sample(want_logits, np.array(history, np.uint32), self.t, TOP_P,
                                                   PENALTY, r)
        err = float(np.abs(got.astype(np.float64) - ref_pen).max())
        assert err <= LOGIT_TOL * rms(ref_pen), f"{label}: logits max error {err:.3e}"
        # the sampler on the GPU's own (already penalized) logits
        tok, info, _ = oracle.sample(got, np.zeros(0, np.uint32), self.t, TOP_P, 1.0, r)
        if info.bisect_margin > SAMPLER_EPS and info.draw_margin > SAMPLER_EPS:
            assert token == tok, f"{label}: gpu {token} vs oracle sampler on gpu logits {tok}"
            self.sampler_compared += 1
        eps = 4 * err / self.t
        if ref_info.bisect_margin > eps and ref_info.draw_margin > eps:
            assert token == ref_tok, f"{label}: gpu {token} vs oracle {ref_tok} (margins clear by {eps:.2e})"
            self.e2e_compared += 1


# The minimum counts keep the test from passing vacuously: every step whose decisions clear the
# margins must give the same token, and at least this share of the steps must clear them. At
# T 0.7 the random-init logits are nearly flat, so the share clearing the sampler's margins
# depends on the trajectory (16 of 41 steps with one kernel revision, at least 17 with another
# whose logits differ by rounding): 80 steps and a floor of a quarter hold it clear of chance.
@pytest.mark.parametrize("temperature,min_sampler,min_e2e", [(T, 0.25, 0.0), (0.1, 0.8, 0.6)])
@pytest.mark.parametrize("graph", [False, True], ids=["eager", "graph"])
def test_sampled_decode_matches_oracle(device, small_model, graph, temperature, min_sampler, min_e2e):
    dm = DeviceModel(device, small_model)
    dec = Decoder(dm)
    ora = OracleDecoder(small_model, max_context=SMALL.max_context)
    try:
        prompt = prompt_ids(16, SMALL.vocab)
        for pos, t in enumerate(prompt[:-1]):  # the prompt's cache rows, greedy f32 steps
            dec.reset(pos, t)
            dec.step(read_token=False)
        dec.set_sampling(temperature, TOP_P, PENALTY)
        dec.seed(0x5EED)
        dec.set_history(prompt)
        if graph:
            dec.capture()
        c = Checker(dec, ora, temperature)
        dec.reset(len(prompt) - 1, prompt[-1])
        token = dec.step()
        for pos, t in enumerate(prompt):
            want = ora.step(t, pos)
        history = list(prompt)
        c.check(token, want, history, "first token")
        history.append(token)
        steps = 80
        for s in range(steps):
            pos = len(prompt) + s
            new = dec.step()
            want = ora.step(token, pos)
            c.check(new, want, history, f"step {s} (pos {pos})")
            history.append(new)
            token = new
        assert dec.history().tolist() == history
        assert dec.position() == len(prompt) + steps
        print(f"T {temperature}: {c.sampler_compared} of {steps + 1} steps compared with the sampler on the GPU's "
              f"logits, {c.e2e_compared} end to end")
        assert c.sampler_compared >= min_sampler * (steps + 1), f"only {c.sampler_compared} steps clear of the sampler's boundaries"
        assert c.e2e_compared >= min_e2e * (steps + 1), f"only {c.e2e_compared} steps clear end to end"
    finally:
        dec.close()
        dm.release()


def test_sampled_graph_replay_equals_eager(device, small_model):
    dm = DeviceModel(device, small_model)
    eager, graph = Decoder(dm), Decoder(dm)
    try:
        prompt = prompt_ids(8, SMALL.vocab, 77)
        for d in (eager, graph):
            d.set_sampling(T, TOP_P, PENALTY)
            d.seed(1234)
        graph.capture()
        a, b = eager.prefill(0, prompt), graph.prefill(0, prompt)
        assert a == b
        for step in range(24):
            a, b = eager.step(), graph.step()
            assert a == b, f"step {step}: eager {a} graph {b}"
            np.testing.assert_array_equal(eager.logits(), graph.logits())
        assert eager.rng_state() == graph.rng_state() == (1234 + 25 * 0x6D2B79F5) % 2 ** 32
        np.testing.assert_array_equal(eager.history(), graph.history())
    finally:
        eager.close()
        graph.close()
        dm.release()


def test_greedy_steps_draw_once(device, small_model):
    """Every step (greedy included, session.ts:351) advances the draw state by one mulberry32
    increment; the prompt's positions draw nothing but the last (sampleFromPrefill); the
    history is the prompt, then every produced token."""
    dm = DeviceModel(device, small_model)
    a = Decoder(dm)
    try:
        prompt = prompt_ids(12, SMALL.vocab, 5)
        a.seed(99)
        tok_a = a.prefill(0, prompt)
        assert a.rng_state() == (99 + 0x6D2B79F5) % 2 ** 32  # only the sampled position drew
        produced = [tok_a] + [a.step() for _ in range(5)]
        assert a.rng_state() == (99 + 6 * 0x6D2B79F5) % 2 ** 32
        assert a.history().tolist() == prompt + produced
        assert a.position() == len(prompt) + 5
    finally:
        a.close()
        dm.release()


def test_penalty_without_temperature_is_argmax_of_penalized_logits(device, small_model):
    dm = DeviceModel(device, small_model)
    dec = Decoder(dm)
    ora = OracleDecoder(small_model, max_context=SMALL.max_context)
    try:
        prompt = prompt_ids(6, SMALL.vocab, 9)
        for pos, t in enumerate(prompt[:-1]):
            dec.reset(pos, t)
            dec.step(read_token=False)
        dec.set_sampling(0.0, 1.0, 1.5)
        dec.set_history(prompt)
        dec.reset(len(prompt) - 1, prompt[-1])
        tok = dec.step()
        for pos, t in enumerate(prompt):
            want = ora.step(t, pos)
        history = list(prompt)
        for s in range(6):
            got = dec.logits()
            ref_tok, _, ref_pen = oracle.sample(want, np.array(history, np.uint32), 0.0, 1.0, 1.5, 0.5)
            assert float(np.abs(got.astype(np.float64) - ref_pen).max()) <= LOGIT_TOL * rms(ref_pen)
            assert tok == int(np.argmax(got))  # the greedy path of the sampler, ties to the lowest id
            order = np.argsort(ref_pen)
            if ref_pen[order[-1]] - ref_pen[order[-2]] > 1e-2 * rms(ref_pen):
                assert tok == ref_tok
            history.append(tok)
            want = ora.step(tok, len(prompt) + s)
            tok = dec.step()
    finally:
        dec.close()
        dm.release()


def test_session_generate_and_prompt_range(device, small_model):
    """Session.generate: first token from the prompt, then max_tokens - 1 steps or a stop token;
    a prompt past the remaining context is a RangeError with the reference's message."""
    dm = DeviceModel(device, small_model)
    dec = Decoder(dm)
    try:
        s = Session(dec, K.SamplingParams(T, TOP_P, PENALTY), seed=0x5EED)
        prompt = prompt_ids(10, SMALL.vocab, 3)
        r = s.generate(prompt, 12)
        assert len(r.tokens) == 12 and s.filled == 10 + 11
        assert dec.history().tolist() == prompt + r.tokens
        assert r.timing.ttft_seconds > 0 and len(r.timing.inter_token_seconds) == 11
        # the same seed and parameters on a fresh session reproduce the tokens (session.test.ts:260-290)
        dec2 = Decoder(dm)
        s2 = Session(dec2, K.SamplingParams(T, TOP_P, PENALTY), seed=0x5EED)
        assert s2.generate(prompt, 12).tokens == r.tokens
        s3 = Session(Decoder(dm), K.SamplingParams(T, TOP_P, PENALTY), seed=0x5EED + 1)
        assert s3.generate(prompt, 12).tokens != r.tokens
        stop = r.tokens[3]
        s4 = Session(Decoder(dm), K.SamplingParams(T, TOP_P, PENALTY), seed=0x5EED)
        assert s4.generate(prompt, 12, stop_tokens=[stop]).tokens == r.tokens[:r.tokens.index(stop) + 1]
        with pytest.raises(RangeError, match="exceeds the remaining context"):
            s.generate(list(range(SMALL.max_context)), 4)
        with pytest.raises(_lib.EgRangeError, match="exceeds the remaining context"):
            dec.prefill(SMALL.max_context - 2, prompt)
        for x in (dec2, s3.decoder, s4.decoder):
            x.close()
    finally:
        dec.close()
        dm.release()


def _spin(device, on):
    lib = _lib.load()
    _lib.check(lib.eg_test_sample_spin(device.ctx, 1 if on else 0, 0), device.ctx)


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "graph"])
def test_sampler_give_up_is_an_error_and_the_next_step_redoes_it(device, small_model, graph):
    """A sampled step whose sampler gives up (forced from the host: every bounded wait gives up at
    its first poll, and every kernel still exits) is EG_ERR_DEVICE at its readback and moves
    nothing: the position, the history, the draw state and the next step's input stay as they
    were, so the next step redoes it and produces exactly the token a decoder that never failed
    produces. Device-chained (no readback), the failure is reported by the next readback and the
    state is again that of a decoder that never failed."""
    dm = DeviceModel(device, small_model)
    dec, ref = Decoder(dm), Decoder(dm)
    try:
        prompt = prompt_ids(10, SMALL.vocab, 41)
        for d in (dec, ref):
            d.set_sampling(T, TOP_P, PENALTY)
            d.seed(0x5EED)
            if graph:
                d.capture()
        assert dec.prefill(0, prompt) == ref.prefill(0, prompt)
        want = [ref.step() for _ in range(4)]
        got = [dec.step()]
        # a step that gives up, with its readback
        pos, hist, rng = dec.position(), dec.history().tolist(), dec.rng_state()
        _spin(device, True)
        try:
            with pytest.raises(_lib.EgError, match="1 step\\(s\\) gave up"):
                dec.step()
        finally:
            _spin(device, False)
        assert (dec.position(), dec.history().tolist(), dec.rng_state()) == (pos, hist, rng)
        got.append(dec.step())
        # device-chained: the failure surfaces at the next readback, whose step succeeded
        _spin(device, True)
        try:
            dec.step(read_token=False)
        finally:
            _spin(device, False)
        assert (dec.position(), dec.rng_state()) == (pos + 1, ref_rng_after(0x5EED, 3))  # prefill + 2 steps
        with pytest.raises(_lib.EgError, match="1 step\\(s\\) gave up"):
            dec.step()
        got.append(int(dec.history()[-1]))
        got.append(dec.step())
        assert got == want
        np.testing.assert_array_equal(dec.history(), ref.history())
        np.testing.assert_array_equal(dec.logits(), ref.logits())
        assert dec.position() == ref.position() == len(prompt) + 4
        assert dec.rng_state() == ref.rng_state()
    finally:
        dec.close()
        ref.close()
        dm.release()


def ref_rng_after(seed, draws):
    return (seed + draws * 0x6D2B79F5) % 2 ** 32


def test_prefill_give_up_leaves_the_last_prompt_position(device, small_model):
    """A prompt whose sampled first token gives up is an error; the decoder is left at the
    prompt's last position with the prompt as its history and no draw taken, and the next step
    recomputes that position as a decode step and samples it with the first draw."""
    dm = DeviceModel(device, small_model)
    dec = Decoder(dm)
    try:
        prompt = prompt_ids(9, SMALL.vocab, 43)
        dec.set_sampling(0.1, TOP_P, PENALTY)
        dec.seed(0x5EED)
        _spin(device, True)
        try:
            with pytest.raises(_lib.EgError, match="1 step\\(s\\) gave up"):
                dec.prefill(0, prompt)
        finally:
            _spin(device, False)
        assert dec.position() == len(prompt) - 1
        assert dec.history().tolist() == prompt
        assert dec.rng_state() == 0x5EED
        tok = dec.step()
        assert dec.position() == len(prompt)
        assert dec.history().tolist() == prompt + [tok]
        assert dec.rng_state() == ref_rng_after(0x5EED, 1)
        # the token is the sampler's on the logits of that recomputed position, with the first draw
        r = np.float32(oracle.Mulberry32Stream(0x5EED)())
        ref_tok, info, _ = oracle.sample(dec.logits(), np.zeros(0, np.uint32), 0.1, TOP_P, 1.0, r)
        if info.bisect_margin > SAMPLER_EPS and info.draw_margin > SAMPLER_EPS:
            assert tok == ref_tok
    finally:
        dec.close()
        dm.release()
