"""ctypes binding of libenargeia_hip.so (the C ABI declared in include/enargeia_hip.h).

The library must exist: nothing here falls back to a CPU or PyTorch implementation. A missing
or stale build raises ``NativeLibraryMissing`` naming the build command.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libenargeia_hip.so")
# the profiling build (per-wave launch stamps compiled in: eg_test_launch_stamps records)
PROF_LIB_PATH = os.path.join(HERE, "libenargeia_hip_prof.so")

EG_OK = 0
EG_ERR_INVALID = -1
EG_ERR_RANGE = -2
EG_ERR_DEVICE = -3
EG_ERR_NOMEM = -4
EG_ERR_STATE = -5
EG_ERR_FORMAT = -6
EG_ERR_IO = -7
EG_ERR_NOT_FOUND = -8

ENC_OFFSET_ZEROS = 0
ENC_SIGNED = 1

# Every symbol include/enargeia_hip.h declares, with (restype, argtypes).
_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
SIGNATURES: dict[str, tuple] = {
    "eg_abi_version": (_i, []),
    "eg_create": (_i, [_i, ctypes.POINTER(_vp)]),
    "eg_destroy": (_i, [_vp]),
    "eg_last_error": (ctypes.c_char_p, [_vp]),
    "eg_get_stream": (_i, [_vp, ctypes.POINTER(_vp)]),
    "eg_set_stream": (_i, [_vp, _vp]),
    "eg_sync": (_i, [_vp]),
    "eg_buf_alloc": (_i, [_vp, _sz, ctypes.POINTER(_vp)]),
    "eg_buf_free": (_i, [_vp, _vp]),
    "eg_buf_write": (_i, [_vp, _vp, _sz, _vp, _sz]),
    "eg_buf_read": (_i, [_vp, _vp, _sz, _vp, _sz]),
    "eg_buf_zero": (_i, [_vp, _vp, _sz, _sz]),
    "eg_matmul_q4_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eg_matmul_q4_prefill": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eg_matmul_q4_prefill_swiglu": (_i, [_vp] * 11 + [_i, _i]),
    "eg_lm_head": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eg_lm_head_argmax": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eg_lm_head_argmax_noalloc": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eg_gemv_plan_create": (_i, [_vp, ctypes.c_uint32, ctypes.c_uint32, _i, _i, _vp, ctypes.c_uint32,
                                 ctypes.POINTER(_vp)]),
    "eg_gemv_plan_launch": (_i, [_vp, _vp, _vp]),
    "eg_gemv_plan_destroy": (_i, [_vp, _vp]),
    "eg_argmax": (_i, [_vp, _vp, _vp, _vp]),
    "eg_sample": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "eg_lm_head_sample": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp]),
    "eg_test_sample_spin": (_i, [_vp, ctypes.c_int, ctypes.c_uint32]),
    "eg_test_launch_stamps": (_i, [_vp, _vp, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32)]),
    "eg_embed_gather": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eg_attention_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "eg_attention_decode_f32": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "eg_attention_combine": (_i, [_vp, _vp, _vp, _vp]),
    "eg_gemv_plan_launch_input": (_i, [_vp, _vp, _vp]),
    "eg_gemv_swiglu_plan_create": (_i, [_vp, ctypes.c_uint32, ctypes.c_uint32, _i, _i, _vp, ctypes.POINTER(_vp)]),
    "eg_lm_head_argmax_input": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eg_decode_advance": (_i, [_vp, _vp, _vp, _vp, _vp, ctypes.c_uint32]),
    "eg_decoder_create": (_i, [_vp, _vp, ctypes.POINTER(_vp)]),
    "eg_decoder_create_cache": (_i, [_vp, _vp, _i, ctypes.POINTER(_vp)]),
    "eg_attention_prefill": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "eg_attention_prefill_f32": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "eg_container_open": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "eg_container_close": (_i, [_vp]),
    "eg_container_header_get": (_i, [_vp, _vp]),
    "eg_container_tensor": (_i, [_vp, ctypes.c_uint32, _vp]),
    "eg_container_find": (_i, [_vp, ctypes.c_char_p, _vp]),
    "eg_container_upload": (_i, [_vp, _vp, ctypes.POINTER(_vp)]),
    "eg_container_model_desc": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_uint32]),
    "eg_decoder_destroy": (_i, [_vp]),
    "eg_decoder_buffers_get": (_i, [_vp, _vp]),
    "eg_decoder_reset": (_i, [_vp, ctypes.c_uint32, ctypes.c_uint32]),
    "eg_decoder_step": (_i, [_vp, _vp]),
    "eg_decoder_capture": (_i, [_vp]),
    "eg_decoder_set_sampling": (_i, [_vp, _vp]),
    "eg_decoder_seed": (_i, [_vp, ctypes.c_uint32]),
    "eg_decoder_launches": (_i, [_vp, ctypes.POINTER(ctypes.c_uint32)]),
    "eg_decoder_set_position": (_i, [_vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float]),
    "eg_decoder_set_history": (_i, [_vp, _vp, ctypes.c_uint32]),
    "eg_decoder_prefill": (_i, [_vp, ctypes.c_uint32, _vp, ctypes.c_uint32, _vp]),
    "eg_decoder_set_prefill_chunk": (_i, [_vp, ctypes.c_uint32]),
    "eg_graph_begin": (_i, [_vp]),
    "eg_graph_end": (_i, [_vp, ctypes.POINTER(_vp)]),
    "eg_graph_launch": (_i, [_vp, _vp]),
    "eg_graph_destroy": (_i, [_vp]),
}


class NativeLibraryMissing(RuntimeError):
    pass


class EgError(RuntimeError):
    """A failed entry point; ``status`` is the eg_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class EgRangeError(EgError, IndexError):
    """EG_ERR_RANGE, the reference's RangeError (kernel.ts:97-107, kvcache.ts:118-127)."""


_lib: ctypes.CDLL | None = None


def use_profiling_build() -> None:
    """Load the profiling build (launch stamps compiled in) instead of the product library; only
    before the library is first loaded in this process."""
    global LIB_PATH
    if _lib is not None and LIB_PATH != PROF_LIB_PATH:
        raise RuntimeError("use_profiling_build: the product library is already loaded in this process")
    LIB_PATH = PROF_LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryMissing(
            f"{LIB_PATH} is not built; run `python -m enargeia_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.eg_abi_version() != 1:
        raise NativeLibraryMissing(f"{LIB_PATH}: ABI version {lib.eg_abi_version()} != 1")
    _lib = lib
    return lib


def check(status: int, ctx) -> None:
    if status == EG_OK:
        return
    msg = load().eg_last_error(ctx)
    text = msg.decode() if msg else f"status {status}"
    if status == EG_ERR_RANGE:
        raise EgRangeError(status, text)
    raise EgError(status, text)
