"""The decode step's layers as ONE persistent launch (eg_layers.hip: the 24 layers' q|k|v, attention,
o, gate|up and down phases in order, workgroups waiting on arrival counters instead of launch
boundaries; a second context created with EG_DECODE_PERSISTENT=1) against the same steps run as
one launch per op (the default context). The phases run the per-op launches' own device code
over virtual grids, so the results must agree to the bit: logits and tokens at every step, greedy
and sampled, eager and replayed from a captured graph, on the 2-layer model and on BASELINE
config 4 at 2048 context. A persistent wait forced to give up (the wait-limit test hook) fails
its step, which changes nothing; the next step redoes it."""

import os

import numpy as np
import pytest

import oracle
from enargeia_amd import _lib
from enargeia_amd import kernels as K
from enargeia_amd.model import (QWEN25_05B, Decoder, DeviceModel, ModelConfig, cache_fill, config4_workload,
                                synthetic_model)

pytestmark = pytest.mark.gpu

SMALL = ModelConfig(layers=2, max_context=256)


@pytest.fixture(scope="module")
def persistent_device():
    os.environ["EG_DECODE_PERSISTENT"] = "1"
    try:
        dev = K.Device(0)
    finally:
        del os.environ["EG_DECODE_PERSISTENT"]
    yield dev
    dev.close()


def launches_per_step(device, dec):
    """Launches one captured step takes (eg_decoder_launches), after capturing it."""
    dec.capture()
    return dec.launches()


def run(device, model, cfg, prompt, steps, sampling, graph, fill=None, start=0):
    dm = DeviceModel(device, model)
    dec = Decoder(dm)
    try:
        if fill is not None:
            device.write(dec.buffers.k_cache, fill[0].view(np.uint16))
            device.write(dec.buffers.v_cache, fill[1].view(np.uint16))
            device.sync()
        if sampling:
            dec.set_sampling(*sampling)
            dec.seed(0x5EED)
        n = launches_per_step(device, dec) if graph else None
        for i, t in enumerate(prompt):
            dec.reset(start + i, t)
            tok = dec.step()
        toks, logits = [tok], [dec.logits().copy()]
        for _ in range(steps):
            toks.append(dec.step())
            logits.append(dec.logits().copy())
        return toks, logits, n, dec.history().tolist(), dec.rng_state()
    finally:
        dec.close()
        dm.release()


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "graph"])
@pytest.mark.parametrize("sampling", [None, (0.7, 0.9, 1.1)], ids=["greedy", "sampled"])
def test_persistent_layers_match_per_op_launches(persistent_device, device, graph, sampling):
    model = synthetic_model(SMALL)
    prompt = [int(t) for t in oracle.random_ids(12, 31, SMALL.vocab)]
    a = run(persistent_device, model, SMALL, prompt, 24, sampling, graph)
    b = run(device, model, SMALL, prompt, 24, sampling, graph)
    if graph:
        extra = 1 if sampling else 0  # the sampler's launch
        assert a[2] == 3 + extra, f"persistent step: {a[2]} launches"
        assert b[2] == 5 * SMALL.layers + 2 + extra, f"per-op step: {b[2]} launches"
    assert a[0] == b[0]
    for s, (x, y) in enumerate(zip(a[1], b[1])):
        np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32), err_msg=f"step {s}")
    assert a[3] == b[3] and a[4] == b[4]


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "graph"])
def test_persistent_layers_config4_bit_exact(persistent_device, device, graph):
    """Config 4 at full size: 24 layers, the cache primed to 1888 positions, the 32-token prompt, 24
    greedy steps; every step's logits to the bit."""
    cfg = QWEN25_05B
    w = config4_workload(cfg)
    model = synthetic_model(cfg)
    fill = cache_fill(cfg, w.fill_seed)
    prompt = list(w.prompt)
    a = run(persistent_device, model, cfg, prompt, 24, None, graph, fill, w.prime)
    b = run(device, model, cfg, prompt, 24, None, graph, fill, w.prime)
    if graph:
        assert a[2] == 3 and b[2] == 5 * cfg.layers + 2
    assert a[0] == b[0]
    for s, (x, y) in enumerate(zip(a[1], b[1])):
        np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32), err_msg=f"step {s}")


def test_persistent_wait_give_up_fails_the_step_and_the_next_redoes_it(persistent_device):
    device = persistent_device
    """The persistent layers' waits forced to give up at their first poll: the step's layers run to
    the end without waiting, the step tail counts the failure and moves nothing, the readback
    reports it; with the default limit restored the next step redoes the step and matches a decoder
    that never failed, logits to the bit."""
    lib = _lib.load()
    model = synthetic_model(SMALL)
    dm = DeviceModel(device, model)
    dec, ref = Decoder(dm), Decoder(dm)
    try:
        prompt = [int(t) for t in oracle.random_ids(8, 33, SMALL.vocab)]
        for d in (dec, ref):
            for i, t in enumerate(prompt):
                d.reset(i, t)
                tok = d.step()
        want = [ref.step() for _ in range(3)]
        pos, hist = dec.position(), dec.history().tolist()
        _lib.check(lib.eg_test_sample_spin(device.ctx, 1, 0), device.ctx)
        try:
            with pytest.raises(_lib.EgError, match="1 step\\(s\\) gave up"):
                dec.step()
        finally:
            _lib.check(lib.eg_test_sample_spin(device.ctx, 0, 0), device.ctx)
        assert dec.position() == pos and dec.history().tolist() == hist
        got = [dec.step() for _ in range(3)]
        assert got == want
        np.testing.assert_array_equal(dec.logits().view(np.uint32), ref.logits().view(np.uint32))
    finally:
        dec.close()
        ref.close()
        dm.release()


def test_production_build_records_no_launch_stamps(device):
    """The product library carries no stamp code (it slows every kernel even switched off): its
    eg_test_launch_stamps refuses a buffer with EG_ERR_STATE, naming the profiling build."""
    lib = _lib.load()
    buf = device.buffer(8192 * 16)
    try:
        with pytest.raises(_lib.EgError, match="profiling build"):
            _lib.check(lib.eg_test_launch_stamps(device.ctx, K._vp(buf.ptr), 1, None), device.ctx)
        _lib.check(lib.eg_test_launch_stamps(device.ctx, None, 0, None), device.ctx)  # off: accepted
    finally:
        buf.release()
