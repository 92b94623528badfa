"""The C ABI library and the host mirror, without a GPU: the library loads, exports exactly the
symbols include/enargeia_hip.h declares, and the host-side interface keeps the reference's
uniform layouts and error behaviour (kernel.ts:70-111)."""

import ctypes
import os
import re
import struct
import subprocess

import numpy as np
import pytest

from enargeia_amd import _lib
from enargeia_amd import kernels as K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "enargeia_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^EG_API\s+[\w\s\*]+?\b(eg_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_ops():
    syms = declared_symbols()
    for name in ("eg_matmul_q4_decode", "eg_matmul_q4_prefill", "eg_lm_head", "eg_lm_head_argmax",
                 "eg_argmax", "eg_sample", "eg_create", "eg_graph_launch"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert set(declared_symbols()) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = sorted({ln.split()[-1] for ln in out.splitlines() if " T " in ln and ln.split()[-1].startswith("eg_")})
    assert exported == declared_symbols()
    assert lib.eg_abi_version() == 1


def test_profiling_build_exports_the_same_symbols():
    # libenargeia_hip_prof.so: the same sources with the launch stamps compiled in
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.PROF_LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = sorted({ln.split()[-1] for ln in out.splitlines() if " T " in ln and ln.split()[-1].startswith("eg_")})
    assert exported == declared_symbols()
    assert b"gfx950" in open(_lib.PROF_LIB_PATH, "rb").read()


def test_library_is_gfx950_code():
    # The device code object inside the library targets gfx950.
    data = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_null_context_errors_without_touching_a_device():
    lib = _lib.load()
    assert lib.eg_sync(None) == _lib.EG_ERR_INVALID
    assert b"ctx is NULL" in lib.eg_last_error(None)
    assert lib.eg_matmul_q4_decode(None, None, None, None, None, None, None, None, 0, 4) != 0


def test_dims_layouts_match_reference_builders():
    # matmulQ4Dims (matmul_q4.ts:50-64): 12 u32, gridWidth = min(n, 65535)
    d = struct.unpack("<12I", K.matmul_q4_dims(1, 151936, 896, True, 64, 151936, 7))
    assert d == (1, 151936, 896, 1, 64, 14, 151936, 7, 65535, 0, 0, 0)
    assert ctypes.sizeof(K.MatmulDims) == 48
    # embeddingDims (embedding_variants.ts:207-221)
    e = struct.unpack("<12I", K.embedding_dims(1, 896, 0, 151936, 896, 151936, 0))
    assert e == (1, 896, 0, 151936, 896, 1, 151936, 0, 65535, 0, 0, 0)
    assert struct.unpack("<4I", K.argmax_dims(151936, 0)) == (151936, 0, 0, 0)
    s = K.sample_dims(151936, 512, K.SamplingParams(0.7, 0.9, 1.1), 0.25)
    assert len(s) == 32 and ctypes.sizeof(K.SampleDims) == 32
    assert struct.unpack("<2I4f2I", s) == (151936, 512, np.float32(0.7), np.float32(0.9), np.float32(1.1), 0.25, 0, 0)


def test_workgroup_helpers_match_reference():
    assert K.matmul_q4_decode_workgroups(151936) == (65535, 3, 1)   # matmul_q4.ts:87-90
    assert K.matmul_q4_prefill_workgroups(256, 4864) == (152, 4, 1)  # matmul_q4.ts:72-78
    assert K.embedding_head_workgroups(151936) == (65535, 3, 1)
    assert K.coverage(K.MATMUL_Q4_DECODE, (0, 1, 1)) == (1, 1, 1)


class _NoDevice:
    ctx = None


def test_bind_group_counts_bindings():
    kern = K.ComputeKernel(_NoDevice(), K.MATMUL_Q4_DECODE)
    with pytest.raises(K.EgError, match="matmul_q4_decode: expected 7 bindings, got 6"):
        kern.bind_group([0] * 6)


def test_encode_rejects_grid_over_limit_as_range_error():
    kern = K.ComputeKernel(_NoDevice(), K.MATMUL_Q4_DECODE)
    bg = kern.bind_group([0] * 6 + [kern.uniform()])
    with pytest.raises(K.EgRangeError, match="70000 workgroups on axis 0 exceeds the device limit of 65535"):
        kern.encode(bg, (70000, 1, 1))


def test_unknown_op_is_refused():
    with pytest.raises(K.EgError, match="not an op of this library"):
        K.ComputeKernel(_NoDevice(), K.KernelSpec("rmsnorm", ("read", "read_write", "uniform"), (256, 1, 1), 16))
    with pytest.raises(K.EgError, match="the dtypes are q4, q8, f16 and f32"):
        K.embedding_head_spec("bf16")
    # the reference's four embedding dtypes (embedding_variants.ts:26): codes, or the table itself
    assert [K.embedding_head_spec(d).bits for d in ("q4", "q8", "f16", "f32")] == [4, 8, 16, 32]
    assert K.embedding_gather_spec("f32").name == "embed_gather_f32" and K.embedding_gather_spec("f32").bits == 32
