"""The Node boundary: the N-API addon (enargeia_amd/js/eg_napi.node) and the JS facade that
mirrors the reference's gpu layer and ComputeKernel, run under the image's Node.

The CPU case checks the addon's exports, the uniform layouts and the synchronous errors
without a device; the GPU case drives the ops from Node the way test/kernels/matmul_q4.test.ts
drives them (reference shapes and seeds, the reference's FP32 tolerance), through the C ABI.
"""

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS_TESTS = os.path.join(ROOT, "tests", "js")
ADDON = os.path.join(ROOT, "enargeia_amd", "js", "eg_napi.node")
NODE = shutil.which("node")

needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")


def _run(script: str, timeout: int) -> None:
    assert os.path.exists(ADDON), f"{ADDON} is not built (python -m enargeia_amd.build)"
    print(f"node {script}", flush=True)
    res = subprocess.run([NODE, os.path.join(JS_TESTS, script)], cwd=ROOT, capture_output=True, text=True,
                         timeout=timeout)
    sys.stdout.write(res.stdout[-20000:])
    assert res.returncode == 0, f"{script} exited {res.returncode}:\n{res.stdout[-4000:]}\n{res.stderr[-4000:]}"


@needs_node
def test_node_facade_cpu():
    _run("facade_cpu.test.js", timeout=60)


@needs_node
@pytest.mark.gpu
def test_node_kernels_gpu():
    _run("kernels_gpu.test.js", timeout=110)
