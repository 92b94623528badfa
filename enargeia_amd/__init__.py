"""MI355X-native quantized projection path of Enargeia (int4 GEMV/GEMM, int8 tied LM head,
GPU argmax and sampling) behind the reference's kernel-op interface.

The compute lives in ``libenargeia_hip.so`` (HIP, gfx950), reached through the C ABI of
``include/enargeia_hip.h``; ``kernels`` mirrors the reference's ``KernelSpec`` /
``ComputeKernel`` for the ops on the path.
"""

from . import _lib  # noqa: F401
