"""A Qwen2.5-0.5B-shaped model on the device, and the decode-step driver over the C ABI.

Reference: the model and runtime layers (src/model/weights.ts WeightStore, graph_decode.ts
DecodeGraph, src/runtime/session.ts decodeStep). ``synthetic_model`` builds the BASELINE config-4
weights (random N(0, 0.02), norm weights 1, q/k/v biases N(0, 0.02); projections symmetric int4
with an f32 scale per 32, the tied embedding int8 per row) with fixed seeds, ``DeviceModel``
uploads them in the reference layout, and ``Decoder`` drives eg_decoder_* (one greedy step per
call, the token and the position kept on the device).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import ENC_SIGNED, check
from .kernels import Device
from .quant import QuantTensor, dense_table, normal, quantize_asym, quantize_sym


@dataclass(frozen=True)
class ModelConfig:
    """ModelShape (test/reference/ops.ts:17-27) plus the cache length and formats."""

    layers: int = 24
    hidden: int = 896
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    intermediate: int = 4864
    vocab: int = 151936
    max_context: int = 2048
    rms_eps: float = 1e-6
    rope_theta: float = 1e6
    group: int = 32   # int4 scale group along K
    bits: int = 4


QWEN25_05B = ModelConfig()

# (name, rows, cols) of one layer's projections, in decode order (graph_decode.ts:276-353)
def projection_shapes(cfg: ModelConfig):
    kv = cfg.kv_heads * cfg.head_dim
    return [("q", cfg.hidden, cfg.hidden), ("k", kv, cfg.hidden), ("v", kv, cfg.hidden),
            ("o", cfg.hidden, cfg.hidden), ("gate", cfg.intermediate, cfg.hidden),
            ("up", cfg.intermediate, cfg.hidden), ("down", cfg.hidden, cfg.intermediate)]


@dataclass
class HostLayer:
    mats: dict            # name -> QuantTensor
    biases: dict          # "q" / "k" / "v" -> f32 array
    input_norm: np.ndarray
    post_attention_norm: np.ndarray


@dataclass
class HostModel:
    cfg: ModelConfig
    layers: list
    embedding: QuantTensor  # int8 per row, [vocab][hidden]
    final_norm: np.ndarray


def seed_for(layer: int, slot: int, base: int = 0x5EED) -> int:
    """The fixed per-tensor seed: base ^ (layer * 16 + slot)."""
    return base ^ (layer * 16 + slot)


def synthetic_model(cfg: ModelConfig = QWEN25_05B, base: int = 0x5EED, fmt: str = "sym",
                    embed_dtype: str = "q8") -> HostModel:
    """Random-init weights of the model's shape. fmt "sym": the BASELINE formats (int4 with an
    f32 scale per cfg.group weights, int8 per-row table, norms 1). fmt "reference": the
    reference quantizer's formats (asymmetric int4 / int8 in blocks of cfg.group with zero-points,
    quantize.py:74-103, --embed-dtype q8) and norm weights drawn around 1. embed_dtype "f16" or
    "f32" stores the tied table as it is (--embed-dtype f16 / f32) instead of int8."""
    layers = []
    ref = fmt == "reference"
    for layer in range(cfg.layers):
        mats = {}
        for slot, (name, rows, cols) in enumerate(projection_shapes(cfg)):
            w = normal(rows * cols, seed_for(layer, slot, base), 0.02)
            mats[name] = quantize_asym(w, rows, cols, cfg.bits, cfg.group) if ref else \
                quantize_sym(w, rows, cols, cfg.bits, cfg.group)
        biases = {name: normal(rows, seed_for(layer, 8 + slot, base), 0.02).astype(np.float32)
                  for slot, (name, rows, _) in enumerate(projection_shapes(cfg)[:3])}
        if ref:
            n1 = (1.0 + normal(cfg.hidden, seed_for(layer, 12, base), 0.1)).astype(np.float32)
            n2 = (1.0 + normal(cfg.hidden, seed_for(layer, 13, base), 0.1)).astype(np.float32)
        else:
            n1 = np.ones(cfg.hidden, np.float32)
            n2 = n1.copy()
        layers.append(HostLayer(mats, biases, n1, n2))
    table = normal(cfg.vocab * cfg.hidden, base ^ 0x1000, 0.02)
    if embed_dtype in ("f16", "f32"):
        embedding = dense_table(table, cfg.vocab, cfg.hidden, 16 if embed_dtype == "f16" else 32)
    else:
        embedding = quantize_asym(table, cfg.vocab, cfg.hidden, 8, cfg.group) if ref else \
            quantize_sym(table, cfg.vocab, cfg.hidden, 8, cfg.hidden)
    final = (1.0 + normal(cfg.hidden, base ^ 0x2000, 0.1)).astype(np.float32) if ref else np.ones(cfg.hidden, np.float32)
    return HostModel(cfg, layers, embedding, final)


# ---- BASELINE config 4's decode run ------------------------------------------------------------


@dataclass(frozen=True)
class DecodeWorkload:
    """The config-4 decode run, following the reference's prime-then-decode method
    (test/parity/decode.test.ts:97-118): cache rows [0, prime) hold random f16 keys and values,
    the prompt enters at positions [prime, prime + len(prompt)), and `steps` greedy steps follow,
    so the last step runs at position max_context - 1."""

    prime: int
    prompt: tuple
    steps: int
    fill_seed: int


def config4_workload(cfg: ModelConfig = QWEN25_05B, prompt_len: int = 32, steps: int = 128,
                     seed: int = 0x5EED ^ 0x4000, fill_seed: int = 11) -> DecodeWorkload:
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab, prompt_len)
    return DecodeWorkload(cfg.max_context - prompt_len - steps, tuple(int(t) for t in prompt), steps, fill_seed)


def cache_fill(cfg: ModelConfig, seed: int):
    """Random f16 cache contents [layers][max_context][kv_heads][head_dim] for keys, then values
    (one generator, keys drawn first)."""
    rng = np.random.default_rng(seed)
    shape = (cfg.layers, cfg.max_context, cfg.kv_heads, cfg.head_dim)
    n = int(np.prod(shape))
    k = rng.standard_normal(n, dtype=np.float32).astype(np.float16).reshape(shape)
    v = rng.standard_normal(n, dtype=np.float32).astype(np.float16).reshape(shape)
    return k, v


# ---- the C structs --------------------------------------------------------------------------


class QuantMatrix(ctypes.Structure):
    _fields_ = [("packed", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("zeros", ctypes.c_void_p)]


class LayerDesc(ctypes.Structure):
    _fields_ = [(n, QuantMatrix) for n in ("q", "k", "v", "o", "gate", "up", "down")] + [
        (n, ctypes.c_void_p) for n in ("q_bias", "k_bias", "v_bias", "input_norm", "post_attention_norm")]


class ModelDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("layers", "hidden", "heads", "kv_heads", "head_dim", "intermediate", "vocab", "max_context")] + [
        ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("encoding", ctypes.c_int),
        ("bits", ctypes.c_int), ("block_size", ctypes.c_uint32), ("embedding", QuantMatrix),
        ("embed_encoding", ctypes.c_int), ("embed_bits", ctypes.c_int), ("embed_block_size", ctypes.c_uint32),
        ("final_norm", ctypes.c_void_p), ("layer", ctypes.POINTER(LayerDesc))]


class AttentionDims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("heads", "kv_heads", "head_dim", "max_context", "chunk")] + [
        ("theta", ctypes.c_float), ("pad0", ctypes.c_uint32), ("pad1", ctypes.c_uint32)]


class GemvInput(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("x", ctypes.c_void_p), ("x2", ctypes.c_void_p), ("eps", ctypes.c_float),
                ("attention", AttentionDims)]


class DecoderBuffers(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("k_cache", "v_cache", "logits", "hidden", "token", "position",
                                               "history", "sample_params", "rng")]


class SamplingParamsC(ctypes.Structure):
    """eg_sampling_params = SamplingParams (sample.ts:24-31)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("repetition_penalty", ctypes.c_float)]


INPUT_VECTOR, INPUT_RMSNORM, INPUT_SILU_MUL, INPUT_ATTENTION = 0, 1, 2, 3


def attention_dims(cfg: ModelConfig, chunk: int = 128) -> AttentionDims:
    return AttentionDims(cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.max_context, chunk, cfg.rope_theta, 0, 0)


class DeviceModel:
    """The host model's tensors uploaded once (WeightStore.upload, weights.ts:377-419)."""

    def __init__(self, device: Device, host: HostModel):
        self.device = device
        self.cfg = host.cfg
        self.buffers = []

        def up(a):
            b = device.upload(a)
            self.buffers.append(b)
            return b.ptr

        def mat(q: QuantTensor) -> QuantMatrix:
            scales = up(q.scales) if q.scales.size else None  # an f16 / f32 table has none
            return QuantMatrix(up(q.packed), scales, None if q.zeros is None else up(q.zeros))

        self.layer_descs = (LayerDesc * self.cfg.layers)()
        for i, L in enumerate(host.layers):
            d = self.layer_descs[i]
            for name in ("q", "k", "v", "o", "gate", "up", "down"):
                setattr(d, name, mat(L.mats[name]))
            d.q_bias, d.k_bias, d.v_bias = (up(L.biases[n]) for n in ("q", "k", "v"))
            d.input_norm = up(L.input_norm)
            d.post_attention_norm = up(L.post_attention_norm)
        c = self.cfg
        self.desc = ModelDesc(c.layers, c.hidden, c.heads, c.kv_heads, c.head_dim, c.intermediate, c.vocab,
                              c.max_context, c.rms_eps, c.rope_theta, ENC_SIGNED, c.bits, c.group,
                              mat(host.embedding), host.embedding.encoding, host.embedding.bits,
                              host.embedding.block_size, up(host.final_norm),
                              ctypes.cast(self.layer_descs, ctypes.POINTER(LayerDesc)))

    def release(self) -> None:
        for b in self.buffers:
            b.release()
        self.buffers = []


CACHE_DTYPES = {"f16": 0, "f32": 1}  # EG_CACHE_F16, EG_CACHE_F32 (SessionOptions.cacheDType)


class Decoder:
    """eg_decoder: decode steps with the token, the position, the sampler's parameters, its
    history and the draw state on the device (greedy until set_sampling says otherwise).
    cache: the KV cache dtype, "f16" (the default) or "f32"."""

    def __init__(self, model: DeviceModel, cache: str = "f16"):
        self.model = model
        self.device = model.device
        self.cache = cache
        lib = _lib.load()
        h = ctypes.c_void_p()
        check(lib.eg_decoder_create_cache(self.device.ctx, ctypes.byref(model.desc), CACHE_DTYPES[cache],
                                          ctypes.byref(h)), self.device.ctx)
        self.handle = h
        bufs = DecoderBuffers()
        check(lib.eg_decoder_buffers_get(h, ctypes.byref(bufs)), self.device.ctx)
        self.buffers = bufs

    def reset(self, position: int, token: int) -> None:
        check(_lib.load().eg_decoder_reset(self.handle, position, token), self.device.ctx)

    def step(self, read_token: bool = True) -> int | None:
        out = ctypes.c_uint32()
        check(_lib.load().eg_decoder_step(self.handle, ctypes.byref(out) if read_token else None), self.device.ctx)
        return out.value if read_token else None

    def capture(self) -> None:
        check(_lib.load().eg_decoder_capture(self.handle), self.device.ctx)

    def set_sampling(self, temperature: float, top_p: float = 1.0, repetition_penalty: float = 1.0) -> None:
        p = SamplingParamsC(temperature, top_p, repetition_penalty)
        check(_lib.load().eg_decoder_set_sampling(self.handle, ctypes.byref(p)), self.device.ctx)

    def seed(self, seed: int) -> None:
        check(_lib.load().eg_decoder_seed(self.handle, ctypes.c_uint32(seed)), self.device.ctx)

    def set_history(self, ids) -> None:
        a = np.ascontiguousarray(ids, np.uint32)
        check(_lib.load().eg_decoder_set_history(self.handle, a.ctypes.data_as(ctypes.c_void_p), a.size),
              self.device.ctx)

    def prefill(self, position: int, prompt, read_token: bool = True) -> int | None:
        """The prompt at [position, position + len) and its first token (runPrefill +
        sampleFromPrefill)."""
        a = np.ascontiguousarray(prompt, np.uint32)
        out = ctypes.c_uint32()
        check(_lib.load().eg_decoder_prefill(self.handle, position, a.ctypes.data_as(ctypes.c_void_p), a.size,
                                             ctypes.byref(out) if read_token else None), self.device.ctx)
        return out.value if read_token else None

    def set_prefill_chunk(self, rows: int) -> None:
        check(_lib.load().eg_decoder_set_prefill_chunk(self.handle, rows), self.device.ctx)

    def history(self) -> np.ndarray:
        n = int(self.sample_params()["history_length"])
        return self.device.read_array(self.buffers.history, np.uint32, n) if n else np.zeros(0, np.uint32)

    def sample_params(self) -> dict:
        raw = self.device.read_array(self.buffers.sample_params, np.uint32, 8)
        f = raw.view(np.float32)
        return {"vocab": int(raw[0]), "history_length": int(raw[1]), "temperature": float(f[2]),
                "top_p": float(f[3]), "repetition_penalty": float(f[4]), "random": f[5]}

    def rng_state(self) -> int:
        return int(self.device.read_array(self.buffers.rng, np.uint32, 1)[0])

    def logits(self) -> np.ndarray:
        return self.device.read_array(self.buffers.logits, np.float32, self.model.cfg.vocab)

    def launches(self) -> int:
        """Launches one step of the current mode enqueues (eg_decoder_launches)."""
        n = ctypes.c_uint32()
        check(_lib.load().eg_decoder_launches(self.handle, ctypes.byref(n)), self.device.ctx)
        return n.value

    def position(self) -> int:
        return int(self.device.read_array(self.buffers.position, np.uint32, 1)[0])

    def close(self) -> None:
        if self.handle:
            _lib.load().eg_decoder_destroy(self.handle)
            self.handle = None
