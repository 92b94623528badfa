"""Host mirror of the reference's kernel-op interface for the ops on this path.

Reference: ``src/kernels/kernel.ts`` (KernelSpec :20-28, ComputeKernel :36-112, coverage
:115-124) and the op modules whose specs and uniform builders are restated here:
``matmul_q4.ts`` (:21-90), ``embedding_variants.ts`` (:135-236), ``argmax.ts`` (:8-18) and
``sample.ts`` (:16-52). Names, binding orders, uniform byte layouts and error behaviour follow
the reference; ``encode`` routes on ``spec.name`` to the C ABI instead of recording a WebGPU
dispatch (the WGSL ``code`` string does not exist here).

Buffers are ``Buffer`` objects from ``Device.buffer`` (or anything with an integer ``ptr``) and
may be bound with a byte offset through ``Binding``, as a ``GPUBufferBinding`` can.
"""

from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import ENC_OFFSET_ZEROS, ENC_SIGNED, EgError, EgRangeError, check

MAX_WORKGROUPS_PER_DIMENSION = 65535  # matmul_q4.ts:48, embedding_variants.ts:205


# ---- buffers and device ---------------------------------------------------------------------


class Buffer:
    """A device allocation owned by a Device (BufferPool.acquire / release)."""

    def __init__(self, device: "Device", ptr: int, size: int, label: str = ""):
        self.device = device
        self.ptr = ptr
        self.size = size
        self.label = label

    def release(self) -> None:
        if self.ptr:
            check(_lib.load().eg_buf_free(self.device.ctx, ctypes.c_void_p(self.ptr)), self.device.ctx)
            self.ptr = 0


@dataclass
class Binding:
    """GPUBufferBinding: a buffer plus a byte offset (and optional size)."""

    buffer: object
    offset: int = 0
    size: int | None = None

    @property
    def ptr(self) -> int:
        return _ptr(self.buffer) + self.offset


def _ptr(ref) -> int:
    if ref is None:
        return 0
    if isinstance(ref, int):
        return ref
    if hasattr(ref, "ptr"):
        return int(ref.ptr)
    if hasattr(ref, "data_ptr"):
        return int(ref.data_ptr())
    raise TypeError(f"cannot bind {type(ref).__name__}")


class Device:
    """One HIP device and stream (initGPU, src/gpu/device.ts:116)."""

    def __init__(self, index: int = 0, stream: int | None = None):
        lib = _lib.load()
        ctx = ctypes.c_void_p()
        st = lib.eg_create(index, ctypes.byref(ctx))
        if st != 0:
            raise EgError(st, lib.eg_last_error(None).decode())
        self.ctx = ctx
        self.index = index
        if stream is not None:
            check(lib.eg_set_stream(ctx, ctypes.c_void_p(stream)), ctx)

    @property
    def stream(self) -> int:
        s = ctypes.c_void_p()
        check(_lib.load().eg_get_stream(self.ctx, ctypes.byref(s)), self.ctx)
        return s.value or 0

    def buffer(self, nbytes: int, label: str = "") -> Buffer:
        p = ctypes.c_void_p()
        check(_lib.load().eg_buf_alloc(self.ctx, max(4, int(nbytes)), ctypes.byref(p)), self.ctx)
        return Buffer(self, p.value, max(4, int(nbytes)), label)

    def upload(self, array: np.ndarray, label: str = "") -> Buffer:
        a = np.ascontiguousarray(array)
        buf = self.buffer(a.nbytes, label)
        self.write(buf, a)
        self.sync()  # pageable source: keep it alive until the copy finished
        return buf

    def write(self, ref, array: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(array)
        check(_lib.load().eg_buf_write(self.ctx, ctypes.c_void_p(_ptr(ref)), offset,
                                       a.ctypes.data_as(ctypes.c_void_p), a.nbytes), self.ctx)

    def read(self, ref, nbytes: int, offset: int = 0) -> bytes:
        out = ctypes.create_string_buffer(nbytes)
        check(_lib.load().eg_buf_read(self.ctx, ctypes.c_void_p(_ptr(ref)), offset, out, nbytes), self.ctx)
        return out.raw

    def read_array(self, ref, dtype, count: int, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        return np.frombuffer(self.read(ref, dt.itemsize * count, offset), dtype=dt).copy()

    def zero(self, ref, nbytes: int, offset: int = 0) -> None:
        check(_lib.load().eg_buf_zero(self.ctx, ctypes.c_void_p(_ptr(ref)), offset, nbytes), self.ctx)

    def sync(self) -> None:
        check(_lib.load().eg_sync(self.ctx), self.ctx)

    def close(self) -> None:
        if self.ctx:
            _lib.load().eg_destroy(self.ctx)
            self.ctx = None

    # graph capture (one hipGraph per recorded step list)
    def capture_begin(self) -> None:
        check(_lib.load().eg_graph_begin(self.ctx), self.ctx)

    def capture_end(self) -> "Graph":
        g = ctypes.c_void_p()
        check(_lib.load().eg_graph_end(self.ctx, ctypes.byref(g)), self.ctx)
        return Graph(self, g)


class Graph:
    def __init__(self, device: Device, handle: ctypes.c_void_p):
        self.device = device
        self.handle = handle

    def launch(self) -> None:
        check(_lib.load().eg_graph_launch(self.device.ctx, self.handle), self.device.ctx)

    def destroy(self) -> None:
        if self.handle:
            _lib.load().eg_graph_destroy(self.handle)
            self.handle = None


# ---- KernelSpec / ComputeKernel --------------------------------------------------------------


@dataclass(frozen=True)
class KernelSpec:
    """kernel.ts:20-28. ``bindings`` in order: inputs, then outputs, then the uniform.
    ``bits``/``encoding`` select the code width and zero-point convention of the weight streams
    (the reference's q4 ops are bits=4, offset encoding; lm_head_q8 is bits=8, offset)."""

    name: str
    bindings: tuple
    workgroup_size: tuple
    uniform_bytes: int
    bits: int = 4
    encoding: int = ENC_OFFSET_ZEROS


class Uniform:
    """The host image of a uniform buffer; write() replaces queue.writeBuffer on it."""

    def __init__(self, nbytes: int):
        self.data = bytearray(nbytes)

    def write(self, payload: bytes, offset: int = 0) -> None:
        self.data[offset: offset + len(payload)] = payload


class BindGroup:
    def __init__(self, kernel: "ComputeKernel", resources: Sequence):
        self.kernel = kernel
        self.resources = list(resources)


class ComputeKernel:
    """kernel.ts:36-112 for the ops of this path, executed through the C ABI."""

    def __init__(self, device: Device, spec: KernelSpec):
        if spec.name not in _DISPATCH:
            raise EgError(_lib.EG_ERR_INVALID, f"{spec.name}: not an op of this library")
        self.device = device
        self.spec = spec

    def bind_group(self, resources: Sequence) -> BindGroup:
        if len(resources) != len(self.spec.bindings):
            raise EgError(_lib.EG_ERR_INVALID,
                          f"{self.spec.name}: expected {len(self.spec.bindings)} bindings, got {len(resources)}")
        return BindGroup(self, resources)

    def uniform(self) -> Uniform:
        return Uniform(self.spec.uniform_bytes)

    def encode(self, bind_group: BindGroup, workgroups: Sequence[int]) -> None:
        # kernel.ts:97-107: a grid over the per-dimension limit is a named RangeError, not a
        # silently dropped dispatch.
        for axis, count in enumerate(workgroups):
            if count > MAX_WORKGROUPS_PER_DIMENSION:
                raise EgRangeError(_lib.EG_ERR_RANGE,
                                   f"{self.spec.name}: {count} workgroups on axis {axis} exceeds the "
                                   f"device limit of {MAX_WORKGROUPS_PER_DIMENSION}")
        res = bind_group.resources
        uniform = res[-1]
        raw = bytes(uniform.data if isinstance(uniform, Uniform) else uniform)
        if len(raw) < self.spec.uniform_bytes:
            raise EgError(_lib.EG_ERR_INVALID, f"{self.spec.name}: uniform of {len(raw)} bytes, "
                                               f"expected {self.spec.uniform_bytes}")
        _DISPATCH[self.spec.name](self, [_ptr(r) for r in res[:-1]], raw[: self.spec.uniform_bytes])


def coverage(spec: KernelSpec, counts: Sequence[int]) -> tuple:
    """kernel.ts:115-124"""
    return tuple(max(1, -(-int(c) // int(w))) for c, w in zip(counts, spec.workgroup_size))


# ---- op specs and uniform builders ------------------------------------------------------------

_Q4_BINDINGS = ("read", "read", "read", "read", "read", "read_write", "uniform")

MATMUL_Q4_DECODE = KernelSpec("matmul_q4_decode", _Q4_BINDINGS, (64, 1, 1), 48)      # matmul_q4.ts:32-38
MATMUL_Q4_PREFILL = KernelSpec("matmul_q4_prefill", _Q4_BINDINGS, (16, 16, 1), 48)    # matmul_q4.ts:23-29
ARGMAX = KernelSpec("argmax", ("read", "read_write", "uniform"), (256, 1, 1), 16)     # argmax.ts:8-14
SAMPLE = KernelSpec("sample", ("read_write", "read", "read_write", "uniform"), (256, 1, 1), 32)  # sample.ts:16-22

_EMBED_BINDINGS = ("read", "read", "read", "read", "read_write", "uniform")


def embedding_head_spec(dtype: str, encoding: int = ENC_OFFSET_ZEROS) -> KernelSpec:
    """embeddingHeadSpec (embedding_variants.ts:195-203): q4 and q8 codes, or an f16 / f32 table
    (bits 16 / 32; scales and zeros unused)."""
    bits = {"q4": 4, "q8": 8, "f16": 16, "f32": 32}.get(dtype)
    if bits is None:
        raise EgError(_lib.EG_ERR_INVALID, f"lm_head_{dtype}: the dtypes are q4, q8, f16 and f32")
    return KernelSpec(f"lm_head_{dtype}", _EMBED_BINDINGS, (64, 1, 1), 48, bits, encoding)


def with_format(spec: KernelSpec, bits: int, encoding: int) -> KernelSpec:
    """The same op over another code width / zero-point convention (the BASELINE formats)."""
    return KernelSpec(spec.name, spec.bindings, spec.workgroup_size, spec.uniform_bytes, bits, encoding)


def _u32s(values) -> bytes:
    # Uint32Array conversion (ToUint32): truncate toward zero, wrap modulo 2^32.
    return struct.pack(f"<{len(values)}I", *[int(v) & 0xFFFFFFFF for v in values])


def decode_grid_width(n: int) -> int:
    """matmul_q4.ts:67-69"""
    return min(n, MAX_WORKGROUPS_PER_DIMENSION)


def matmul_q4_dims(m: int, n: int, k: int, use_bias: bool, block_size: int, out_stride: int | None = None,
                   out_offset: int = 0) -> bytes:
    """matmulQ4Dims, matmul_q4.ts:50-64"""
    stride = n if out_stride is None else out_stride
    return _u32s([m, n, k, 1 if use_bias else 0, block_size, int(k / block_size), stride, out_offset,
                  decode_grid_width(n), 0, 0, 0])


def matmul_q4_decode_workgroups(n: int) -> tuple:
    """matmul_q4.ts:87-90"""
    width = decode_grid_width(n)
    return (width, -(-n // width), 1)


def matmul_q4_prefill_workgroups(m: int, n: int) -> tuple:
    """matmul_q4.ts:72-78 (64 x 32 output tile)"""
    return (max(1, -(-n // 32)), max(1, -(-m // 64)), 1)


def embedding_dims(seq: int, hidden: int, row_begin: int, row_count: int, block_size: int,
                   out_stride: int = 0, out_offset: int = 0) -> bytes:
    """embeddingDims, embedding_variants.ts:207-221"""
    return _u32s([seq, hidden, row_begin, row_count, block_size, int(hidden / block_size), out_stride,
                  out_offset, min(max(row_count, 1), MAX_WORKGROUPS_PER_DIMENSION), 0, 0, 0])


def embedding_head_workgroups(rows: int) -> tuple:
    """embedding_variants.ts:233-236"""
    width = min(rows, MAX_WORKGROUPS_PER_DIMENSION)
    return (width, -(-rows // width), 1)


def argmax_dims(count: int, offset: int) -> bytes:
    """argmax.ts:16-18"""
    return _u32s([count, offset, 0, 0])


ARGMAX_WORKGROUPS = (1, 1, 1)
SAMPLE_WORKGROUPS = (1, 1, 1)


@dataclass(frozen=True)
class SamplingParams:
    """sample.ts:24-31"""

    temperature: float
    top_p: float
    repetition_penalty: float


GREEDY = SamplingParams(0.0, 1.0, 1.0)  # sample.ts:33


def sample_dims(vocab: int, history_length: int, params: SamplingParams, random: float) -> bytes:
    """sampleDims, sample.ts:35-50"""
    return _u32s([vocab, history_length]) + struct.pack(
        "<4f", params.temperature, params.top_p, params.repetition_penalty, random) + bytes(8)


# ---- dispatch through the C ABI -------------------------------------------------------------


class MatmulDims(ctypes.Structure):
    _fields_ = [(f, ctypes.c_uint32) for f in
                ("m", "n", "k", "use_bias", "block_size", "blocks_per_row", "out_stride", "out_offset",
                 "grid_width", "pad0", "pad1", "pad2")]


class EmbeddingDims(ctypes.Structure):
    _fields_ = [(f, ctypes.c_uint32) for f in
                ("seq", "hidden", "row_begin", "row_count", "block_size", "blocks_per_row", "out_stride",
                 "out_offset", "grid_width", "pad0", "pad1", "pad2")]


class ArgmaxDims(ctypes.Structure):
    _fields_ = [(f, ctypes.c_uint32) for f in ("count", "offset", "pad0", "pad1")]


class SampleDims(ctypes.Structure):
    _fields_ = [("vocab", ctypes.c_uint32), ("history_length", ctypes.c_uint32),
                ("temperature", ctypes.c_float), ("top_p", ctypes.c_float),
                ("repetition_penalty", ctypes.c_float), ("random", ctypes.c_float),
                ("pad0", ctypes.c_uint32), ("pad1", ctypes.c_uint32)]


def _vp(p: int) -> ctypes.c_void_p:
    return ctypes.c_void_p(p or None)


def embedding_gather_spec(dtype: str, encoding: int = ENC_OFFSET_ZEROS) -> KernelSpec:
    """embeddingGatherSpec (embedding_variants.ts:186-193): binding 0 holds the `seq` ids."""
    h = embedding_head_spec(dtype, encoding)
    return KernelSpec(f"embed_gather_{dtype}", h.bindings, h.workgroup_size, h.uniform_bytes, h.bits, h.encoding)


def _gather(k: ComputeKernel, p: list, raw: bytes) -> None:
    d = EmbeddingDims.from_buffer_copy(raw)
    ctx = k.device.ctx
    ids, packed, scales, zeros, out = p
    check(_lib.load().eg_embed_gather(ctx, _vp(ids), _vp(packed), _vp(scales), _vp(zeros), _vp(out), ctypes.byref(d),
                                      k.spec.encoding, k.spec.bits), ctx)


def _matmul(k: ComputeKernel, p: list, raw: bytes, fn: str) -> None:
    d = MatmulDims.from_buffer_copy(raw)
    ctx = k.device.ctx
    x, packed, scales, zeros, bias, out = p
    check(getattr(_lib.load(), fn)(ctx, _vp(x), _vp(packed), _vp(scales), _vp(zeros), _vp(bias), _vp(out),
                                   ctypes.byref(d), k.spec.encoding, k.spec.bits), ctx)


def _lm_head(k: ComputeKernel, p: list, raw: bytes) -> None:
    d = EmbeddingDims.from_buffer_copy(raw)
    ctx = k.device.ctx
    x, packed, scales, zeros, out = p
    check(_lib.load().eg_lm_head(ctx, _vp(x), _vp(packed), _vp(scales), _vp(zeros), _vp(out), ctypes.byref(d),
                                 k.spec.encoding, k.spec.bits), ctx)


def _argmax(k: ComputeKernel, p: list, raw: bytes) -> None:
    d = ArgmaxDims.from_buffer_copy(raw)
    ctx = k.device.ctx
    check(_lib.load().eg_argmax(ctx, _vp(p[0]), _vp(p[1]), ctypes.byref(d)), ctx)


def _sample(k: ComputeKernel, p: list, raw: bytes) -> None:
    d = SampleDims.from_buffer_copy(raw)
    ctx = k.device.ctx
    check(_lib.load().eg_sample(ctx, _vp(p[0]), _vp(p[1]), _vp(p[2]), ctypes.byref(d)), ctx)


_DISPATCH = {
    "matmul_q4_decode": lambda k, p, r: _matmul(k, p, r, "eg_matmul_q4_decode"),
    "matmul_q4_prefill": lambda k, p, r: _matmul(k, p, r, "eg_matmul_q4_prefill"),
    "lm_head_q4": _lm_head,
    "lm_head_q8": _lm_head,
    "lm_head_f16": _lm_head,
    "lm_head_f32": _lm_head,
    "embed_gather_q4": _gather,
    "embed_gather_q8": _gather,
    "embed_gather_f16": _gather,
    "embed_gather_f32": _gather,
    "argmax": _argmax,
    "sample": _sample,
}


class GemvSegment(ctypes.Structure):
    _fields_ = [("packed", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("zeros", ctypes.c_void_p),
                ("bias", ctypes.c_void_p), ("out", ctypes.c_void_p), ("rows", ctypes.c_uint32),
                ("out_offset", ctypes.c_uint32)]


class GemvPlan:
    """Several decode GEMVs sharing one input and K, launched together (eg_gemv_plan_*).
    ``segments`` are (packed, scales, zeros, bias, out, rows, out_offset) tuples of buffers."""

    def __init__(self, device: Device, k: int, block_size: int, segments, bits: int = 4,
                 encoding: int = ENC_SIGNED):
        self.device = device
        table = (GemvSegment * len(segments))()
        for i, (packed, scales, zeros, bias, out, rows, out_offset) in enumerate(segments):
            table[i] = GemvSegment(_ptr(packed) or None, _ptr(scales) or None, _ptr(zeros) or None,
                                   _ptr(bias) or None, _ptr(out) or None, rows, out_offset)
        h = ctypes.c_void_p()
        check(_lib.load().eg_gemv_plan_create(device.ctx, k, block_size, encoding, bits, table, len(segments),
                                              ctypes.byref(h)), device.ctx)
        self.handle = h

    def launch(self, x) -> None:
        check(_lib.load().eg_gemv_plan_launch(self.device.ctx, self.handle, _vp(_ptr(x))), self.device.ctx)

    def destroy(self) -> None:
        if self.handle:
            check(_lib.load().eg_gemv_plan_destroy(self.device.ctx, self.handle), self.device.ctx)
            self.handle = None


def lm_head_argmax(device: Device, x, packed, scales, zeros, out, result, dims: bytes, bits: int = 8,
                   encoding: int = ENC_OFFSET_ZEROS) -> None:
    """The fused LM head + greedy argmax (no reference op; see include/enargeia_hip.h)."""
    d = EmbeddingDims.from_buffer_copy(dims)
    check(_lib.load().eg_lm_head_argmax(device.ctx, _vp(_ptr(x)), _vp(_ptr(packed)), _vp(_ptr(scales)),
                                        _vp(_ptr(zeros)), _vp(_ptr(out)), _vp(_ptr(result)), ctypes.byref(d),
                                        encoding, bits), device.ctx)


def lm_head_sample(device: Device, x, packed, scales, zeros, logits, history, token, dims: bytes,
                   sample: bytes, bits: int = 8, encoding: int = ENC_OFFSET_ZEROS) -> None:
    """The int8 LM head and the sampler as one sampled token (no reference op; the reference runs
    lm_head_q8 then sample, graph_decode.ts:363-385; see include/enargeia_hip.h). `dims` are the
    head's embedding dims, `sample` the sample dims (sample_dims); token[0] gets the id and
    `logits` the penalized logits, as eg_sample leaves them."""
    d = EmbeddingDims.from_buffer_copy(dims)
    sd = SampleDims.from_buffer_copy(sample)
    check(_lib.load().eg_lm_head_sample(device.ctx, _vp(_ptr(x)), _vp(_ptr(packed)), _vp(_ptr(scales)),
                                        _vp(_ptr(zeros)), _vp(_ptr(logits)), _vp(_ptr(history)), _vp(_ptr(token)),
                                        ctypes.byref(d), encoding, bits, ctypes.byref(sd)), device.ctx)


__all__ = [
    "ARGMAX", "ARGMAX_WORKGROUPS", "Binding", "Buffer", "ComputeKernel", "Device", "ENC_OFFSET_ZEROS",
    "ENC_SIGNED", "EgError", "EgRangeError", "GREEDY", "GemvPlan", "GemvSegment", "Graph", "KernelSpec", "MATMUL_Q4_DECODE",
    "MATMUL_Q4_PREFILL", "MAX_WORKGROUPS_PER_DIMENSION", "SAMPLE", "SAMPLE_WORKGROUPS", "SamplingParams",
    "argmax_dims", "coverage", "decode_grid_width", "embedding_dims", "embedding_head_spec",
    "embedding_gather_spec", "embedding_head_workgroups", "lm_head_argmax", "lm_head_sample", "matmul_q4_decode_workgroups", "matmul_q4_dims",
    "matmul_q4_prefill_workgroups", "sample_dims", "with_format",
]
