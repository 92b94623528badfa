"""Offline quantizers that write the three weight streams the kernels read.

The reference quantizes offline (tools/quantize.py:74-103 writes the shipped asymmetric format,
test/reference/quant.ts:24-74 is its float64 twin). This module writes:

* ``quantize_sym``: the BASELINE symmetric formats -- int4 with an f32 scale per group of 32
  along K (scale = absmax/7, codes -8..7 as two's-complement nibbles, element 2j in the low
  nibble of byte j) and int8 per row (scale = absmax/127, two's-complement bytes);
* ``quantize_asym``: the reference's asymmetric format with numpy's float32 rint, exactly as
  tools/quantize.py computes it (codes and zero-points at 4 or 8 bits, block size along K).

Vectorised numpy, used to build synthetic models for benchmarks and examples. tests/test_quant
checks every stream bit-for-bit against the CPU oracle.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

ENC_OFFSET_ZEROS = 0
ENC_SIGNED = 1


@dataclass
class QuantTensor:
    """One quantized matrix as three device-ready streams (weights.ts:56-67)."""

    rows: int
    cols: int
    block_size: int
    bits: int
    encoding: int
    packed: np.ndarray  # u32
    scales: np.ndarray  # f32
    zeros: np.ndarray | None  # u32 (offset encoding only)

    def nbytes(self) -> int:
        return self.packed.nbytes + self.scales.nbytes + (0 if self.zeros is None else self.zeros.nbytes)


def _pack(codes: np.ndarray, bits: int) -> np.ndarray:
    per = 32 // bits
    c = codes.reshape(-1, per).astype(np.uint32) & np.uint32((1 << bits) - 1)
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    return np.bitwise_or.reduce(c << shifts, axis=1).astype(np.uint32)


def dense_table(values: np.ndarray, rows: int, cols: int, bits: int = 16) -> QuantTensor:
    """A table stored as it is, the reference's 'f16' and 'f32' embedding dtypes
    (embedding_variants.ts:26-74): bits 16 packs two halves per u32 (element 2j in the low half,
    as unpack2x16float reads them), bits 32 plain floats. No scales or zero-points (an empty
    scale stream); block_size is the row."""
    if bits not in (16, 32):
        raise ValueError(f"a dense table is f16 (16) or f32 (32) bits, not {bits}")
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    if bits == 16 and v.size % 2:
        raise ValueError("an f16 table needs an even element count (two halves per word)")
    raw = v.astype(np.float16).view(np.uint16).astype(np.uint32) if bits == 16 else v.view(np.uint32)
    packed = (raw[0::2] | (raw[1::2] << np.uint32(16))).astype(np.uint32) if bits == 16 else raw.copy()
    return QuantTensor(rows, cols, cols, bits, ENC_SIGNED, packed, np.zeros(0, np.float32), None)


def quantize_sym(values: np.ndarray, rows: int, cols: int, bits: int = 4, block_size: int = 32) -> QuantTensor:
    if bits not in (4, 8) or cols % block_size:
        raise ValueError(f"reduction axis {cols} is not a multiple of {block_size}")
    qmax = 7 if bits == 4 else 127
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1, block_size)
    absmax = np.abs(v).max(axis=1)
    scale = np.where(absmax > 0, absmax / np.float32(qmax), np.float32(1.0)).astype(np.float32)
    codes = np.rint(v / scale[:, None]).astype(np.float32)
    codes = np.clip(codes, -qmax - 1, qmax).astype(np.int32)
    return QuantTensor(rows, cols, block_size, bits, ENC_SIGNED, _pack(codes.reshape(-1), bits), scale, None)


def quantize_asym(values: np.ndarray, rows: int, cols: int, bits: int = 4, block_size: int = 64) -> QuantTensor:
    if bits not in (4, 8) or cols % block_size:
        raise ValueError(f"reduction axis {cols} is not a multiple of {block_size}")
    levels = (1 << bits) - 1
    blocks = np.ascontiguousarray(values, dtype=np.float32).reshape(-1, block_size)
    lo = blocks.min(axis=1)
    hi = blocks.max(axis=1)
    scale = ((hi - lo) / np.float32(levels)).astype(np.float32)
    degenerate = scale <= 0
    scale = np.where(degenerate, np.where(hi != 0, np.abs(hi) / np.float32(levels), np.float32(1.0)),
                     scale).astype(np.float32)
    zero = np.clip(np.rint(-lo / scale), 0, levels).astype(np.int64)
    q = np.clip(np.rint((blocks / scale[:, None]).astype(np.float64) + zero[:, None]), 0, levels)
    per = 32 // bits
    nblk = zero.shape[0]
    padded = np.zeros(-(-nblk // per) * per, dtype=np.int64)
    padded[:nblk] = zero
    return QuantTensor(rows, cols, block_size, bits, ENC_OFFSET_ZEROS, _pack(q.reshape(-1), bits), scale,
                       _pack(padded, bits))


def normal(count: int, seed: int, sigma: float) -> np.ndarray:
    """N(0, sigma) float32 from numpy's PCG64 (synthetic weights for benchmarks)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(count, dtype=np.float32) * np.float32(sigma)).astype(np.float32)
