"""The package's offline quantizers write the same streams as the CPU oracle, bit for bit."""

import numpy as np
import pytest

import oracle
from enargeia_amd import quant


@pytest.mark.parametrize("bits,group,rows,cols", [(4, 32, 64, 896), (4, 32, 8, 4864), (8, 896, 32, 896),
                                                   (8, 64, 16, 128)])
def test_sym_matches_oracle(bits, group, rows, cols):
    v = oracle.normal_floats(rows * cols, bits * 1000 + cols, 0.02)
    v[5] = 0.0
    v[group:2 * group] = 0.0  # an all-zero group
    a = quant.quantize_sym(v, rows, cols, bits, group)
    b = oracle.quantize_sym(v, rows, cols, bits, group)
    assert np.array_equal(a.packed, b.packed)
    assert np.array_equal(a.scales.view(np.uint32), b.scales.view(np.uint32))
    assert a.encoding == b.encoding == oracle.ENC_SIGNED


@pytest.mark.parametrize("bits,bs", [(4, 64), (8, 64), (4, 32)])
def test_asym_matches_quantize_py_restatement(bits, bs):
    v = oracle.random_floats(48 * 256, 5 + bits)
    v[:bs] = 0.375           # constant block
    v[bs:2 * bs] = 0.0       # zero block
    v[2 * bs:3 * bs] = -2.0  # negative constant block
    a = quant.quantize_asym(v, 48, 256, bits, bs)
    b = oracle.quantize_blocks_n(v, 48, 256, bits, bs)
    assert np.array_equal(a.packed, b.packed)
    assert np.array_equal(a.scales.view(np.uint32), b.scales.view(np.uint32))
    assert np.array_equal(a.zeros, b.zeros)


def test_rejects_ragged_reduction_axis():
    with pytest.raises(ValueError, match="not a multiple of 32"):
        quant.quantize_sym(np.zeros(40, np.float32), 1, 40)
