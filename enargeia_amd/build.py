"""Builds the HIP library in-tree: enargeia_amd/libenargeia_hip.so (gfx950 only).

Every ``csrc/*.hip`` translation unit is compiled with hipcc for ``--offload-arch=gfx950``
(packed-FP32 instructions disabled) and linked into one shared library whose exported symbols
are exactly the ``extern "C"`` entry points of ``include/enargeia_hip.h``. The Node N-API addon
(``js/eg_napi.node``) is then compiled with g++ against the node headers and linked to that
library through an ``$ORIGIN`` rpath. Run directly (``python -m enargeia_amd.build``) or
through ``__graft_entry__.build()``.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(ROOT, "_build")
LIB_PATH = os.path.join(HERE, "libenargeia_hip.so")
# The profiling build: the same sources with EG_LAUNCH_STAMPS, whose kernels can record per-wave
# wall-clock stamps (eg_test_launch_stamps; bench.py --decode-timeline loads it). The product
# library carries no stamp code: compiled in, even unused, it slows every kernel.
PROF_LIB_PATH = os.path.join(HERE, "libenargeia_hip_prof.so")
NAPI_SRC = os.path.join(HERE, "js", "eg_napi.cc")
NAPI_PATH = os.path.join(HERE, "js", "eg_napi.node")
NODE_INCLUDE = os.environ.get("NODE_INCLUDE", "/usr/include/node")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    # No packed FP32 (v_pk_fma_f32 and friends) anywhere in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-file additions: the chunk attention keeps its MFMA results in ordinary VGPRs (its softmax
# reads and rescales them every key tile; held in AGPRs, each of those accesses is a copy).
FILE_FLAGS = {"eg_prefill_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(job: tuple[str, bool]) -> str:
    src, prof = job
    obj_dir = os.path.join(BUILD_DIR, "prof" if prof else "prod")
    os.makedirs(obj_dir, exist_ok=True)
    obj = os.path.join(obj_dir, os.path.basename(src)[:-4] + ".o")
    extra = FILE_FLAGS.get(os.path.basename(src), []) + (["-DEG_LAUNCH_STAMPS"] if prof else [])
    cmd = [HIPCC, *HIP_FLAGS, *extra, "-I", os.path.join(ROOT, "include"), "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> str:
    """Both libraries: the product (LIB_PATH) and the profiling build (PROF_LIB_PATH)."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    jobs = [(src, prof) for prof in (False, True) for src in srcs]
    workers = min(len(jobs), max(1, (os.cpu_count() or 4) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, jobs))
    for path, group in ((LIB_PATH, objs[:len(srcs)]), (PROF_LIB_PATH, objs[len(srcs):])):
        tmp = path + ".tmp"
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *group]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stderr}")
        os.replace(tmp, path)
        if verbose:
            print(f"built {path} from {len(srcs)} sources", file=sys.stderr)
    build_napi(verbose)
    return LIB_PATH


def build_napi(verbose: bool = True) -> str | None:
    """The N-API addon. Needs only node_api.h (Node 12 ships N-API 8); skipped with a notice
    where the node headers are absent, since the addon is a host binding, not compute."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        print(f"node headers not found under {NODE_INCLUDE}: N-API addon not built", file=sys.stderr)
        return None
    tmp = NAPI_PATH + ".tmp"
    cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-fvisibility=hidden",
           "-DNAPI_VERSION=8", "-DNODE_GYP_MODULE_NAME=eg_napi",
           "-I", NODE_INCLUDE, "-I", os.path.join(ROOT, "include"), NAPI_SRC,
           "-L", HERE, "-lenargeia_hip", "-Wl,-rpath,$ORIGIN/..", "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"N-API addon build failed:\n{res.stderr}")
    os.replace(tmp, NAPI_PATH)
    if verbose:
        print(f"built {NAPI_PATH}", file=sys.stderr)
    return NAPI_PATH


if __name__ == "__main__":
    build()
