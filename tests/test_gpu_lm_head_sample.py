"""The int8 LM head and the sampler as one sampled token (eg_lm_head_sample) against the
reference's two ops on the same inputs - lm_head_q8, then sample (graph_decode.ts:363-385),
here the head binding then eg_sample, which test_gpu_sample.py holds to the oracle.

The fused head applies the repetition penalty itself and hands the sampler per-workgroup
(max of l/T, index, float64 sum of exp(l/T - max)) partials: its penalized logits must equal
eg_sample's in place bit for bit, and its token must equal eg_sample's draw for draw (the
float64 normaliser is summed in other groups; its f32 rounding is the same here). Ragged
vocabularies make the head's last tile overlap the one before it, with history ids in the
overlap.
"""

import numpy as np
import pytest

import oracle
from cases import config2_history, lm_head_config2
from enargeia_amd import kernels as K

pytestmark = pytest.mark.gpu


class Head:
    def __init__(self, device, q, h):
        self.device = device
        self.q = q
        n = q.rows
        self.bufs = [device.upload(h), device.upload(q.packed), device.upload(q.scales),
                     device.upload(q.zeros) if q.zeros is not None else None]
        self.dims = K.embedding_dims(1, q.cols, 0, n, q.block_size, n, 0)
        self.logits = device.buffer(n * 4)
        self.history = device.buffer(8192 * 4)
        self.token = device.buffer(16)
        self.sampler = K.ComputeKernel(device, K.SAMPLE)
        self.head = K.ComputeKernel(device, K.embedding_head_spec("q8", q.encoding))

    def _history(self, hist):
        h = np.ascontiguousarray(hist, np.uint32)
        if h.size:
            self.device.write(self.history, h)
        return h.size

    def fused(self, hist, params, random):
        n = self._history(hist)
        bh, bp, bs, bz = self.bufs
        K.lm_head_sample(self.device, bh, bp, bs, bz, self.logits, self.history, self.token, self.dims,
                         K.sample_dims(self.q.rows, n, params, random), self.q.bits, self.q.encoding)
        return self._read()

    def separate(self, hist, params, random):
        n = self._history(hist)
        u = self.head.uniform()
        u.write(self.dims)
        self.head.encode(self.head.bind_group(self.bufs + [self.logits, u]), K.embedding_head_workgroups(self.q.rows))
        su = self.sampler.uniform()
        su.write(K.sample_dims(self.q.rows, n, params, random))
        self.sampler.encode(self.sampler.bind_group([self.logits, self.history, self.token, su]), K.SAMPLE_WORKGROUPS)
        return self._read()

    def _read(self):
        tok = int(self.device.read_array(self.token, np.uint32, 1)[0])
        return tok, self.device.read_array(self.logits, np.float32, self.q.rows)

    def close(self):
        for b in self.bufs + [self.logits, self.history, self.token]:
            if b is not None:
                b.release()


def _agree(head, hist, params, draws, label):
    for r in draws:
        ft, fl = head.fused(hist, params, r)
        st, sl = head.separate(hist, params, r)
        assert np.array_equal(fl.view(np.uint32), sl.view(np.uint32)), f"{label}: penalized logits differ"
        assert ft == st, f"{label}: random {r}: fused {ft} separate {st}"
        assert 0 <= ft < head.q.rows


@pytest.fixture(scope="module")
def config2_head(device):
    q, h, _ = lm_head_config2()
    head = Head(device, q, h)
    yield head
    head.close()


@pytest.mark.parametrize("params", [K.SamplingParams(0.7, 0.9, 1.1), K.SamplingParams(1.0, 0.95, 1.0),
                                    K.SamplingParams(0.7, 1.0, 1.1), K.SamplingParams(0.0, 1.0, 1.1),
                                    K.SamplingParams(0.3, 0.5, 1.3)])
def test_config2_fused_equals_head_then_sample(config2_head, params):
    # BASELINE config 2 (151,936 x 896 int8 head) over its 512-id history; greedy with a penalty too
    rng = oracle.Mulberry32Stream(0x5EED)
    _agree(config2_head, config2_history(), params, [rng() for _ in range(8)], f"config 2 {params}")


def test_config2_fused_without_history(config2_head):
    rng = oracle.Mulberry32Stream(7)
    _agree(config2_head, np.zeros(0, np.uint32), K.SamplingParams(0.7, 0.9, 1.1), [rng() for _ in range(4)],
           "no history")


@pytest.mark.parametrize("vocab", [1025, 70001])
def test_ragged_vocab_with_history_in_the_last_tiles(device, vocab):
    hidden = 128
    q = oracle.quantize_sym(oracle.normal_floats(vocab * hidden, vocab, 0.05), vocab, hidden, 8, hidden)
    h = oracle.normal_floats(hidden, vocab + 1, 1.0)
    hist = np.concatenate([np.arange(vocab - 6, vocab, dtype=np.uint32), oracle.random_ids(300, vocab, vocab),
                           np.array([vocab, vocab + 5, 0], np.uint32)])  # ids past the vocabulary are ignored
    head = Head(device, q, h)
    try:
        rng = oracle.Mulberry32Stream(vocab)
        for params in (K.SamplingParams(0.8, 0.95, 1.2), K.SamplingParams(0.0, 1.0, 1.3)):
            _agree(head, hist, params, [rng() for _ in range(4)], f"vocab {vocab} {params}")
    finally:
        head.close()


def test_rejects_bad_arguments(device):
    # Checked on the host before anything is launched: an int4 head, a sample vocabulary that is
    # not the head's rows, an output offset, a history length with no history.
    import ctypes
    from enargeia_amd import _lib
    lib = _lib.load()
    buf = device.buffer(1 << 20)
    vp = ctypes.c_void_p(buf.ptr)
    dims = K.EmbeddingDims.from_buffer_copy(K.embedding_dims(1, 896, 0, 1024, 896, 1024, 0))
    shifted = K.EmbeddingDims.from_buffer_copy(K.embedding_dims(1, 896, 0, 1024, 896, 1024, 8))
    params = K.SamplingParams(0.7, 0.9, 1.1)

    def call(d, sample, bits=8, history=vp):
        sd = K.SampleDims.from_buffer_copy(sample)
        return lib.eg_lm_head_sample(device.ctx, vp, vp, vp, None, vp, history, vp, ctypes.byref(d), K.ENC_SIGNED,
                                     bits, ctypes.byref(sd))

    try:
        assert call(dims, K.sample_dims(1024, 0, params, 0.5), bits=4) == _lib.EG_ERR_INVALID
        assert call(dims, K.sample_dims(1000, 0, params, 0.5)) == _lib.EG_ERR_INVALID
        assert b"must equal the head's rows" in lib.eg_last_error(device.ctx)
        assert call(shifted, K.sample_dims(1024, 0, params, 0.5)) == _lib.EG_ERR_INVALID
        assert call(dims, K.sample_dims(1024, 5, params, 0.5), history=None) == _lib.EG_ERR_INVALID
        assert b"no history buffer" in lib.eg_last_error(device.ctx)
    finally:
        buf.release()
