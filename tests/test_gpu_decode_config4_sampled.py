"""Sampled decoding at BASELINE config 4's full size: the 24-layer Qwen2.5-0.5B-shaped decoder,
f16 cache primed to 1888 positions, the 32-token prompt, then the session's sampled decoding at
T 0.1 / top-p 0.9 / repetition penalty 1.1 from seed 0x5eed (the first draw at the prompt's last
position, sampleFromPrefill; one more per decodeStep, session.ts:347-375, 472-495), against the
CPU oracle's run of the same workload (tests/golden/config4_sampled.npz, written by
tests/golden/gen_config4_sampled.py).

Checked at every one of the 33 sampled steps, eager and as a replayed hipGraph:
  * the draw the step used equals the oracle's mulberry32 draw, bit for bit;
  * the penalized logits at the oracle's 64 largest ids equal the oracle's within 2e-3 x rms
    (the decoder bar of test_gpu_decode.py);
  * the token equals oracle.sample (sample.wgsl:143-332) applied to the GPU's own penalized
    logits wherever that sampler's decisions are 2e-6 clear of a boundary (the sampler bar of
    test_gpu_sample.py): the full-size sampler inside the full-size step;
  * the token equals the oracle's end to end wherever the oracle's sampler decisions are clear of
    their boundaries by 4 x the step's largest logit error there / T (a logit error d moves every
    p by at most a factor e^(2d/T), so the masses by at most ~2d/T; ids outside the 64 hold
    under 1e-9 of the mass at T 0.1). At T 0.1 the random-init model spreads the top-p 0.9
    nucleus over tens of ids, so the mass at the nucleus boundary is within ~1e-3 of topP at
    most steps, and this check clears only where the logits agree to ~1e-5.
Where the tokens differ at a step not clear of its boundaries, the run continues on the oracle's
token and history, so later steps stay comparable."""

import os

import numpy as np
import pytest

import oracle
from enargeia_amd.model import QWEN25_05B, Decoder, DeviceModel, cache_fill, config4_workload, synthetic_model

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config4_sampled.npz")
LOGIT_TOL = 2e-3   # x rms(penalized logits), absolute
SAMPLER_EPS = 2e-6
# end-to-end comparisons clear at 28 of the 33 steps on MI355X (eager and graph); the floor leaves
# room for rounding differences between kernel revisions
MIN_E2E = 0.75


@pytest.fixture(scope="module")
def golden():
    with np.load(FIXTURE, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="module")
def run_setup(device, golden):
    cfg = QWEN25_05B
    w = config4_workload(cfg)
    assert w.prime == int(golden["prime"]) and list(w.prompt) == [int(t) for t in golden["prompt"]]
    kf, vf = cache_fill(cfg, int(golden["fill_seed"]))
    dm = DeviceModel(device, synthetic_model(cfg))
    yield cfg, w, dm, kf, vf
    dm.release()


def run_sampled(device, golden, cfg, w, dm, kf, vf, graph: bool):
    """(steps compared with the sampler on the GPU's logits, steps compared end to end, steps
    continued on the oracle's token) of one run."""
    dec = Decoder(dm)
    T = float(golden["temperature"])
    try:
        device.write(dec.buffers.k_cache, kf.view(np.uint16))
        device.write(dec.buffers.v_cache, vf.view(np.uint16))
        device.sync()
        n_prompt = len(w.prompt)
        for s in range(n_prompt - 1):  # the prompt's cache rows, greedy steps
            dec.reset(w.prime + s, w.prompt[s])
            dec.step(read_token=False)
        dec.set_sampling(T, float(golden["top_p"]), float(golden["penalty"]))
        dec.seed(int(golden["seed"]))
        history = [int(t) for t in w.prompt]
        dec.set_history(history)
        if graph:
            dec.capture()
        dec.reset(w.prime + n_prompt - 1, w.prompt[-1])
        sampler = compared = forced = 0
        top_p = float(golden["top_p"])
        for i, pos in enumerate(golden["positions"]):
            assert dec.position() == pos
            tok = dec.step()
            sp = dec.sample_params()
            assert sp["random"].view(np.uint32) == golden["draws"][i].view(np.uint32), f"step {i}: draw"
            got = dec.logits()  # penalized in place by the sample step
            ids = golden["top_ids"][i]
            err = float(np.abs(got[ids].astype(np.float64) - golden["top_values"][i]).max())
            assert err <= LOGIT_TOL * float(golden["rms"][i]), f"step {i} (pos {pos}): logits off by {err:.3e}"
            mine, info, _ = oracle.sample(got, np.zeros(0, np.uint32), T, top_p, 1.0, float(golden["draws"][i]))
            if info.bisect_margin > SAMPLER_EPS and info.draw_margin > SAMPLER_EPS:
                assert tok == mine, f"step {i} (pos {pos}): token {tok} vs the oracle's sampler on the GPU logits {mine}"
                sampler += 1
            want = int(golden["tokens"][i])
            eps = 4 * err / T
            if golden["bisect_margin"][i] > eps and golden["draw_margin"][i] > eps:
                assert tok == want, f"step {i} (pos {pos}): token {tok} vs oracle {want} (margins clear by {eps:.2e})"
                compared += 1
            history.append(want)
            if tok != want:  # a step inside the boundaries: continue on the oracle's token
                dec.reset(int(pos) + 1, want)
                dec.set_history(history)
                forced += 1
        assert dec.history().tolist() == history
        return sampler, compared, forced
    finally:
        dec.close()


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "graph"])
def test_config4_sampled_decode_matches_oracle(device, golden, run_setup, graph):
    cfg, w, dm, kf, vf = run_setup
    sampler, compared, forced = run_sampled(device, golden, cfg, w, dm, kf, vf, graph)
    steps = len(golden["positions"])
    print(f"config 4 sampled ({'graph' if graph else 'eager'}): {sampler} of {steps} steps compared with the "
          f"sampler on the GPU's logits, {compared} end to end, {forced} continued on the oracle's token")
    assert sampler >= 0.8 * steps
    assert compared >= MIN_E2E * steps
