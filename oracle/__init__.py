"""ctypes view of the CPU oracle (oracle/libeg_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against. Only tests/,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this package; the
product (``enargeia_amd``) never does. Every function restates the reference file:line named in
``eg_oracle.c``; the numpy helpers below only allocate arrays and forward to the C code.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libeg_oracle.so")

ENC_OFFSET_ZEROS = 0
ENC_SIGNED = 1

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)


def build() -> None:
    """Compile the oracle with its Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE, "libeg_oracle.so"], check=True)


def _load() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    lib.eo_mulberry32_next.restype = ctypes.c_double
    lib.eo_dequant.restype = ctypes.c_double
    lib.eo_argmax.restype = ctypes.c_uint32
    lib.eo_argmax_wgsl.restype = ctypes.c_uint32
    lib.eo_sample.restype = ctypes.c_uint32
    lib.eo_bf16_round.restype = ctypes.c_float
    lib.eo_bf16_round.argtypes = [ctypes.c_float]
    lib.eo_f16_round.restype = ctypes.c_float
    lib.eo_f16_round.argtypes = [ctypes.c_float]
    lib.eo_silu.restype = ctypes.c_float
    lib.eo_silu.argtypes = [ctypes.c_float]
    return lib


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


class Mulberry32(ctypes.Structure):
    _fields_ = [("s", ctypes.c_uint32)]


def mulberry32_sequence(seed: int, count: int) -> np.ndarray:
    r = Mulberry32()
    lib().eo_mulberry32_init(ctypes.byref(r), ctypes.c_uint32(seed))
    return np.array([lib().eo_mulberry32_next(ctypes.byref(r)) for _ in range(count)])


class Mulberry32Stream:
    """The session's per-step draw source (session.ts:75-83, :125 default seed 0x5eed)."""

    def __init__(self, seed: int = 0x5EED):
        self._r = Mulberry32()
        lib().eo_mulberry32_init(ctypes.byref(self._r), ctypes.c_uint32(seed))

    def __call__(self) -> float:
        return lib().eo_mulberry32_next(ctypes.byref(self._r))


def random_floats(count: int, seed: int = 1) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    lib().eo_random_floats(_p(out), ctypes.c_size_t(count), ctypes.c_uint32(seed))
    return out


def normal_floats(count: int, seed: int, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    lib().eo_normal_floats(_p(out), ctypes.c_size_t(count), ctypes.c_uint32(seed),
                           ctypes.c_double(sigma))
    return out


def random_ids(count: int, seed: int, bound: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint32)
    lib().eo_random_ids(_p(out), ctypes.c_size_t(count), ctypes.c_uint32(seed),
                        ctypes.c_uint32(bound))
    return out


@dataclass
class QuantizedMatrix:
    """Three streams, exactly as the reference uploads them (weights.ts:56-67)."""

    rows: int
    cols: int
    block_size: int
    bits: int
    encoding: int
    packed: np.ndarray  # u32
    scales: np.ndarray  # f32
    zeros: np.ndarray | None  # u32, None for the signed encoding

    @property
    def blocks(self) -> int:
        return self.rows * self.cols // self.block_size

    def nbytes(self) -> int:
        z = 0 if self.zeros is None else self.zeros.nbytes
        return self.packed.nbytes + self.scales.nbytes + z


def _check(status: int, what: str) -> None:
    if status != 0:
        raise ValueError(f"{what}: oracle returned {status}")


def quantize_q4_ref(values: np.ndarray, rows: int, cols: int, block_size: int = 64) -> QuantizedMatrix:
    """test/reference/quant.ts:24-74"""
    v = np.ascontiguousarray(values, dtype=np.float32)
    blocks = rows * cols // block_size
    packed = np.zeros(rows * cols // 8, dtype=np.uint32)
    scales = np.zeros(blocks, dtype=np.float32)
    zeros = np.zeros((blocks + 7) // 8, dtype=np.uint32)
    _check(lib().eo_quantize_q4_ref(_p(v), rows, cols, block_size, _p(packed), _p(scales), _p(zeros)),
           "quantize_q4_ref")
    return QuantizedMatrix(rows, cols, block_size, 4, ENC_OFFSET_ZEROS, packed, scales, zeros)


def quantize_blocks_n(values: np.ndarray, rows: int, cols: int, bits: int, block_size: int = 64) -> QuantizedMatrix:
    """tools/quantize.py:74-103"""
    v = np.ascontiguousarray(values, dtype=np.float32)
    per_word = 32 // bits
    blocks = rows * cols // block_size
    packed = np.zeros(rows * cols // per_word, dtype=np.uint32)
    scales = np.zeros(blocks, dtype=np.float32)
    zeros = np.zeros((blocks + per_word - 1) // per_word, dtype=np.uint32)
    _check(lib().eo_quantize_blocks_n(_p(v), rows, cols, block_size, bits, _p(packed), _p(scales),
                                      _p(zeros)), "quantize_blocks_n")
    return QuantizedMatrix(rows, cols, block_size, bits, ENC_OFFSET_ZEROS, packed, scales, zeros)


def quantize_sym(values: np.ndarray, rows: int, cols: int, bits: int, block_size: int) -> QuantizedMatrix:
    """BASELINE symmetric int4 (group 32) / int8 (per row, block_size = cols)."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    per_word = 32 // bits
    packed = np.zeros(rows * cols // per_word, dtype=np.uint32)
    scales = np.zeros(rows * cols // block_size, dtype=np.float32)
    _check(lib().eo_quantize_sym(_p(v), rows, cols, block_size, bits, _p(packed), _p(scales)),
           "quantize_sym")
    return QuantizedMatrix(rows, cols, block_size, bits, ENC_SIGNED, packed, scales, None)


def dequant_element(q: QuantizedMatrix, row: int, col: int) -> float:
    return lib().eo_dequant(_p(q.packed), _p(q.scales), _p(q.zeros), q.bits, q.encoding, q.cols,
                            q.block_size, row, col)


def dequantize(q: QuantizedMatrix) -> np.ndarray:
    """Whole matrix in float64, vectorised restatement of eo_dequant (checked against it)."""
    per_word = 32 // q.bits
    mask = (1 << q.bits) - 1
    shifts = (np.arange(per_word, dtype=np.uint32) * q.bits)
    codes = ((q.packed[:, None] >> shifts[None, :]) & mask).reshape(-1).astype(np.int64)
    if q.encoding == ENC_SIGNED:
        codes = np.where(codes >= (1 << (q.bits - 1)), codes - (1 << q.bits), codes)
        zero = np.zeros(q.blocks, dtype=np.int64)
    else:
        zero = ((q.zeros[:, None] >> shifts[None, :]) & mask).reshape(-1)[: q.blocks].astype(np.int64)
    vals = (codes.reshape(q.blocks, q.block_size) - zero[:, None]).astype(np.float64)
    vals *= q.scales.astype(np.float64)[:, None]
    return vals.reshape(q.rows, q.cols)


def linear_q(x: np.ndarray, q: QuantizedMatrix, bias: np.ndarray | None, m: int,
             out: np.ndarray | None = None, out_stride: int | None = None, out_offset: int = 0) -> np.ndarray:
    """test/reference/quant.ts:95-111 (float64 accumulate, f32 store)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, k = q.rows, q.cols
    stride = n if out_stride is None else out_stride
    if out is None:
        out = np.zeros((m - 1) * stride + n + out_offset, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().eo_linear_q(_p(x), m, k, n, _p(q.packed), _p(q.scales), _p(q.zeros), q.block_size,
                      q.bits, q.encoding, _p(b), _p(out), stride, out_offset)
    return out


def linear_q_fast(x: np.ndarray, q: QuantizedMatrix, bias: np.ndarray | None, m: int) -> np.ndarray:
    """Same values as linear_q for large shapes: float64 matmul over the float64 dequantized
    matrix (each product and the f32 store identical; only float64 summation order differs)."""
    w = dequantize(q)
    y = np.asarray(x, dtype=np.float64).reshape(m, q.cols) @ w.T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)[None, :]
    return y.astype(np.float32).reshape(-1)


def linear_q_bf16(x: np.ndarray, q: QuantizedMatrix, bias: np.ndarray | None, m: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(m * q.rows, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().eo_linear_q_bf16(_p(x), m, q.cols, q.rows, _p(q.packed), _p(q.scales), _p(q.zeros),
                           q.block_size, q.bits, q.encoding, _p(b), _p(out), q.rows, 0)
    return out


def bf16_round_array(a: np.ndarray) -> np.ndarray:
    """Vectorised RNE to bf16 (checked against eo_bf16_round)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def linear_q_bf16_fast(x: np.ndarray, q: QuantizedMatrix, bias: np.ndarray | None, m: int) -> np.ndarray:
    """eo_linear_q_bf16 for large shapes: bf16(x) @ bf16(f32 dequant)^T in float64."""
    w32 = dequantize(q).astype(np.float32)  # the device's f32 (code - zero) * scale
    wb = bf16_round_array(w32).astype(np.float64)
    xb = bf16_round_array(np.asarray(x, dtype=np.float32)).astype(np.float64).reshape(m, q.cols)
    y = xb @ wb.T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)[None, :]
    return y.astype(np.float32).reshape(-1)


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().eo_argmax(_p(x), ctypes.c_size_t(x.size)))


def argmax_wgsl(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().eo_argmax_wgsl(_p(x), ctypes.c_size_t(x.size)))


class SampleInfo(ctypes.Structure):
    _fields_ = [
        ("token", ctypes.c_uint32),
        ("greedy", ctypes.c_int),
        ("max_scaled", ctypes.c_float),
        ("argmax", ctypes.c_uint32),
        ("total", ctypes.c_float),
        ("threshold", ctypes.c_float),
        ("kept", ctypes.c_float),
        ("target", ctypes.c_float),
        ("bisect_margin", ctypes.c_double),
        ("threshold_gap", ctypes.c_double),
        ("draw_margin", ctypes.c_double),
        ("kept_count", ctypes.c_uint32),
    ]


def sample(logits: np.ndarray, history: np.ndarray, temperature: float, top_p: float,
           penalty: float, random: float) -> tuple[int, SampleInfo, np.ndarray]:
    """sample.wgsl:143-332. Returns (token, diagnostics, the penalized logits)."""
    l = np.array(logits, dtype=np.float32, copy=True)
    h = np.ascontiguousarray(history, dtype=np.uint32)
    info = SampleInfo()
    tok = lib().eo_sample(_p(l), ctypes.c_uint32(l.size), _p(h) if h.size else None,
                          ctypes.c_uint32(h.size), ctypes.c_float(temperature), ctypes.c_float(top_p),
                          ctypes.c_float(penalty), ctypes.c_float(random), ctypes.byref(info))
    return int(tok), info, l


def rmsnorm(x: np.ndarray, w: np.ndarray, seq: int, features: int, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    lib().eo_rmsnorm(_p(x), _p(w), _p(out), seq, features, ctypes.c_double(eps))
    return out


def rope(x: np.ndarray, seq: int, heads: int, head_dim: int, theta: float, position_offset: int = 0) -> np.ndarray:
    out = np.array(x, dtype=np.float32, copy=True)
    lib().eo_rope(_p(out), seq, heads, head_dim, ctypes.c_double(theta), position_offset)
    return out


def gemv_threads(x: np.ndarray, q: QuantizedMatrix, bias: np.ndarray | None, threads: int) -> np.ndarray:
    """The CPU baseline loop (linearQ4 at m=1) over `threads` POSIX threads."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(q.rows, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().eo_gemv_threads(_p(x), q.cols, q.rows, _p(q.packed), _p(q.scales), _p(q.zeros),
                          q.block_size, q.bits, q.encoding, _p(b), _p(out), threads)
    return out


def f16_round(v: float) -> float:
    return float(lib().eo_f16_round(ctypes.c_float(v)))


def bf16_round(v: float) -> float:
    return float(lib().eo_bf16_round(ctypes.c_float(v)))


def silu(v: float) -> float:
    return float(lib().eo_silu(ctypes.c_float(v)))
