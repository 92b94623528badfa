"""The `.enargeia` container from Python: write one (the layout of tools/quantize.py:190-260),
open it through the C++ parser (eg_container_*, enargeia.ts:1-50, 112-240), upload its blob in
one piece and drive the decoder from it (WeightStore.loadQuantized, weights.ts:299-471).

Parsing needs no GPU: ``Container(path)`` works on a host without one (errors come back as
``EgError`` with the reference's EnargeiaError text). ``Container.load(device, config)``
uploads the blob and returns a model the decoder accepts.
"""

from __future__ import annotations

import ctypes
import json
import struct
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import EgError, check
from .model import LayerDesc, ModelConfig, ModelDesc
from .quant import QuantTensor

MAGIC = b"ENARGEIA"
VERSION = 1
BLOCK = 64
ALIGN = 256

DTYPE_Q4, DTYPE_Q8, DTYPE_F32, DTYPE_F16 = 0, 1, 2, 3
DTYPE_NAMES = {DTYPE_Q4: "Q4", DTYPE_Q8: "Q8", DTYPE_F32: "F32", DTYPE_F16: "F16"}
MAX_DIMS = 8


class TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int), ("bits", ctypes.c_int),
                ("ndim", ctypes.c_uint32), ("block_size", ctypes.c_uint32), ("blocks_per_row", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * MAX_DIMS), ("total_blocks", ctypes.c_uint64),
                ("packed", ctypes.c_uint64 * 2), ("scales", ctypes.c_uint64 * 2), ("zeros", ctypes.c_uint64 * 2),
                ("data", ctypes.c_uint64 * 2)]


class ContainerHeader(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("block_size", ctypes.c_uint32), ("tensor_count", ctypes.c_uint32),
                ("pad0", ctypes.c_uint32), ("header_length", ctypes.c_uint64), ("data_offset", ctypes.c_uint64),
                ("blob_bytes", ctypes.c_uint64), ("file_size", ctypes.c_uint64), ("quantization", ctypes.c_char_p)]


class ModelConfigC(ctypes.Structure):
    _fields_ = [("head_dim", ctypes.c_uint32), ("max_context", ctypes.c_uint32), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float)]


# ---- writing ----------------------------------------------------------------------------------


def write_enargeia(path: str, tensors, block_size: int = BLOCK,
                   quantization: str = "asymmetric-int4-blockwise", generator: str = "enargeia_amd") -> dict:
    """Writes `tensors` (name -> QuantTensor in the offset format, or a float32 / float16 array)
    in the given order: each range 256-byte aligned in the blob, the header compact JSON, then
    zeros to the next 256-byte boundary. Returns the header dict."""
    entries = {}
    blob = bytearray()

    def place(payload: bytes) -> list:
        """Appends payload at the next multiple of ALIGN (zero-filled gap): its [begin, end)."""
        blob.extend(bytes(-len(blob) % ALIGN))
        start = len(blob)
        blob.extend(payload)
        return [start, len(blob)]

    for name, t in tensors.items() if isinstance(tensors, dict) else tensors:
        if isinstance(t, QuantTensor):
            if t.zeros is None:
                raise ValueError(f"{name}: the container stores the offset format (codes, scales, zeros)")
            entries[name] = {"dtype": "Q4" if t.bits == 4 else "Q8", "shape": [t.rows, t.cols],
                             "blockSize": t.block_size,
                             "offsets": {"packed": place(np.ascontiguousarray(t.packed, np.uint32).tobytes()),
                                         "scales": place(np.ascontiguousarray(t.scales, np.float32).tobytes()),
                                         "zeros": place(np.ascontiguousarray(t.zeros, np.uint32).tobytes())}}
        else:
            a = np.asarray(t)
            dt = "F16" if a.dtype == np.float16 else "F32"
            a = np.ascontiguousarray(a, np.float16 if dt == "F16" else np.float32)
            entries[name] = {"dtype": dt, "shape": list(a.shape), "offsets": {"data": place(a.tobytes())}}
    header = {"generator": generator, "blockSize": block_size, "quantization": quantization, "tensors": entries}
    raw = json.dumps(header, separators=(",", ":")).encode("utf-8")
    write_raw(path, raw, bytes(blob))
    return header


# Qwen2 checkpoint names (weights.ts:47 for the embedding; the safetensors names the
# reference's graph reads, graph_decode.ts:246-385).
PROJECTION_NAMES = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
                    "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}


def qwen2_tensors(host) -> dict:
    """A HostModel (enargeia_amd.model) as checkpoint-named tensors, in the sorted-name order
    tools/quantize.py writes them."""
    e = host.embedding
    # an f16 / f32 table (bits 16 / 32) is written as the F16 / F32 tensor it is: the packed
    # words hold its elements in order (element 2j in the low half of an f16 pair)
    table = e if e.bits not in (16, 32) else \
        e.packed.view(np.float16 if e.bits == 16 else np.float32).reshape(e.rows, e.cols)
    out = {"model.embed_tokens.weight": table, "model.norm.weight": host.final_norm}
    for i, L in enumerate(host.layers):
        p = f"model.layers.{i}."
        for short, long in PROJECTION_NAMES.items():
            out[p + long + ".weight"] = L.mats[short]
        for short in ("q", "k", "v"):
            out[p + PROJECTION_NAMES[short] + ".bias"] = L.biases[short]
        out[p + "input_layernorm.weight"] = L.input_norm
        out[p + "post_attention_layernorm.weight"] = L.post_attention_norm
    return dict(sorted(out.items()))


def write_raw(path: str, header_json: bytes, blob: bytes, version: int = VERSION, magic: bytes = MAGIC) -> None:
    """The byte layout itself: magic, version, header length, header, zeros to 256, blob."""
    prefix = len(magic) + 8 + len(header_json)
    with open(path, "wb") as f:
        f.write(magic)
        f.write(struct.pack("<I", version))
        f.write(struct.pack("<I", len(header_json)))
        f.write(header_json)
        f.write(b"\0" * ((-prefix) % ALIGN))
        f.write(blob)


# ---- reading ----------------------------------------------------------------------------------


@dataclass
class Tensor:
    name: str
    dtype: str
    bits: int
    shape: tuple
    block_size: int
    blocks_per_row: int
    total_blocks: int
    packed: tuple
    scales: tuple
    zeros: tuple
    data: tuple


class LoadedModel:
    """A container's blob on the device plus the decoder description that points into it."""

    def __init__(self, device, blob: int, desc: ModelDesc, layers, cfg: ModelConfig):
        self.device = device
        self.blob = blob
        self.desc = desc
        self.layer_descs = layers
        self.cfg = cfg

    def release(self) -> None:
        if self.blob:
            check(_lib.load().eg_buf_free(self.device.ctx, ctypes.c_void_p(self.blob)), self.device.ctx)
            self.blob = 0


class Container:
    """An open container (eg_container_open). ``ctx`` is optional: parsing needs no device."""

    def __init__(self, path: str, device=None):
        self.path = path
        self.device = device
        ctx = device.ctx if device is not None else None
        h = ctypes.c_void_p()
        check(_lib.load().eg_container_open(ctx, path.encode(), ctypes.byref(h)), ctx)
        self.handle = h

    def close(self) -> None:
        if self.handle:
            _lib.load().eg_container_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def header(self) -> dict:
        h = ContainerHeader()
        check(_lib.load().eg_container_header_get(self.handle, ctypes.byref(h)), None)
        return {"version": h.version, "blockSize": h.block_size, "tensorCount": h.tensor_count,
                "headerLength": h.header_length, "dataOffset": h.data_offset, "blobBytes": h.blob_bytes,
                "fileSize": h.file_size, "quantization": h.quantization.decode()}

    @staticmethod
    def _tensor(info: TensorInfo) -> Tensor:
        return Tensor(info.name.decode(), DTYPE_NAMES[info.dtype], info.bits, tuple(info.shape[:info.ndim]),
                      info.block_size, info.blocks_per_row, info.total_blocks, tuple(info.packed),
                      tuple(info.scales), tuple(info.zeros), tuple(info.data))

    def tensors(self) -> list:
        out = []
        for i in range(self.header()["tensorCount"]):
            info = TensorInfo()
            check(_lib.load().eg_container_tensor(self.handle, i, ctypes.byref(info)), None)
            out.append(self._tensor(info))
        return out

    def find(self, name: str) -> Tensor:
        info = TensorInfo()
        check(_lib.load().eg_container_find(self.handle, name.encode(), ctypes.byref(info)), None)
        return self._tensor(info)

    def upload(self, device) -> int:
        """The blob in one device allocation (eg_buf_free it, or use ``load``)."""
        blob = ctypes.c_void_p()
        check(_lib.load().eg_container_upload(device.ctx, self.handle, ctypes.byref(blob)), device.ctx)
        return blob.value

    def describe(self, blob: int, head_dim: int = 64, max_context: int = 2048, rms_eps: float = 1e-6,
                 rope_theta: float = 1e6, device=None):
        """eg_container_model_desc: the decoder description of the Qwen2 model in this container,
        every tensor pointer = blob + its range's begin. Pure arithmetic on the header, so `blob`
        may be any address when only the description is inspected."""
        lib = _lib.load()
        ctx = device.ctx if device is not None else None
        cfg_c = ModelConfigC(head_dim, max_context, rms_eps, rope_theta)
        layers = sum(1 for t in self.tensors() if t.name.endswith(".self_attn.q_proj.weight"))
        layer_descs = (LayerDesc * max(1, layers))()
        desc = ModelDesc()
        check(lib.eg_container_model_desc(ctx, self.handle, ctypes.c_void_p(blob), ctypes.byref(cfg_c),
                                          ctypes.byref(desc), layer_descs, len(layer_descs)), ctx)
        cfg = ModelConfig(layers=desc.layers, hidden=desc.hidden, heads=desc.heads, kv_heads=desc.kv_heads,
                          head_dim=desc.head_dim, intermediate=desc.intermediate, vocab=desc.vocab,
                          max_context=desc.max_context, rms_eps=desc.rms_eps, rope_theta=desc.rope_theta,
                          group=desc.block_size, bits=desc.bits)
        return desc, layer_descs, cfg

    def load(self, device, head_dim: int = 64, max_context: int = 2048, rms_eps: float = 1e-6,
             rope_theta: float = 1e6) -> LoadedModel:
        """Uploads the blob and describes the Qwen2 model in it for eg_decoder_create."""
        blob = self.upload(device)
        try:
            desc, layer_descs, cfg = self.describe(blob, head_dim, max_context, rms_eps, rope_theta, device)
        except EgError:
            _lib.load().eg_buf_free(device.ctx, ctypes.c_void_p(blob))
            raise
        return LoadedModel(device, blob, desc, layer_descs, cfg)
