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

import numpy as np
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


def _write_model(host, directory):
    """Raw tensor bytes + a JSON manifest (offsets 256-byte aligned, as the reference's container
    aligns its streams), for the Node decoder test to load."""
    import json
    import numpy as np

    tensors, chunks, offset = {}, [], 0

    def add(name, array):
        nonlocal offset
        raw = np.ascontiguousarray(array).tobytes()
        tensors[name] = {"offset": offset, "bytes": len(raw)}
        pad = (-len(raw)) % 256
        chunks.append(raw + b"\0" * pad)
        offset += len(raw) + pad

    for i, L in enumerate(host.layers):
        for name, q in L.mats.items():
            add(f"layers.{i}.{name}.packed", q.packed)
            add(f"layers.{i}.{name}.scales", q.scales)
        for name, b in L.biases.items():
            add(f"layers.{i}.{name}.bias", b)
        add(f"layers.{i}.input_norm", L.input_norm)
        add(f"layers.{i}.post_attention_norm", L.post_attention_norm)
    add("embedding.packed", host.embedding.packed)
    add("embedding.scales", host.embedding.scales)
    add("final_norm", host.final_norm)
    c = host.cfg
    manifest = {"config": {k: getattr(c, k) for k in ("layers", "hidden", "heads", "kv_heads", "head_dim",
                                                      "intermediate", "vocab", "max_context", "rms_eps",
                                                      "rope_theta", "group", "bits")},
                "first_token": 17, "tensors": tensors}
    with open(os.path.join(directory, "tensors.bin"), "wb") as f:
        for c_ in chunks:
            f.write(c_)
    with open(os.path.join(directory, "manifest.json"), "w") as f:
        json.dump(manifest, f)
    return manifest


@needs_node
@pytest.mark.gpu
def test_node_decoder_matches_python_decoder(tmp_path, device):
    """The same model driven from Node (N-API decoder binding) and from Python (ctypes) gives the
    same greedy tokens, eagerly and as a replayed graph, and over an f32 KV cache."""
    import json

    from enargeia_amd.model import Decoder, DeviceModel, ModelConfig, synthetic_model

    cfg = ModelConfig(layers=2, vocab=4096, max_context=256)
    host = synthetic_model(cfg)
    manifest = _write_model(host, str(tmp_path))
    steps = 12
    print(f"node tests/js/decoder_gpu.test.js {tmp_path} {steps}", flush=True)
    res = subprocess.run([NODE, os.path.join(JS_TESTS, "decoder_gpu.test.js"), str(tmp_path), str(steps)], cwd=ROOT,
                         capture_output=True, text=True, timeout=110)
    sys.stdout.write(res.stdout[-4000:])
    assert res.returncode == 0, f"node exited {res.returncode}:\n{res.stdout[-3000:]}\n{res.stderr[-3000:]}"
    node_tokens = json.loads(next(line for line in res.stdout.splitlines() if line.startswith('{"eager"')))
    dm = DeviceModel(device, host)
    dec = Decoder(dm)
    dec32 = Decoder(dm, cache="f32")
    try:
        dec.reset(0, manifest["first_token"])
        py_tokens = [dec.step() for _ in range(steps)]
        dec32.reset(0, manifest["first_token"])
        py_tokens32 = [dec32.step() for _ in range(steps)]
    finally:
        dec.close()
        dec32.close()
        dm.release()
    assert node_tokens["eager"] == py_tokens
    assert node_tokens["graph"] == py_tokens
    assert node_tokens["f32"] == py_tokens32


@needs_node
@pytest.mark.gpu
def test_node_session_over_decode_graph_matches_python(tmp_path, device):
    """The reference's Session.generate / decodeStep restated in JS over the DecodeGraph-shaped
    binding (host-driven steps: tokenId, history, setPosition with the host's mulberry32 draw,
    encode, submit, readBuffer) yields the same sampled tokens as the Python Session, whose
    decoder chains the steps and draws on the device; eager and as a replayed graph."""
    import json

    from enargeia_amd.kernels import SamplingParams
    from enargeia_amd.model import Decoder, DeviceModel, ModelConfig, synthetic_model
    from enargeia_amd.session import Session

    cfg = ModelConfig(layers=2, vocab=4096, max_context=256)
    host = synthetic_model(cfg)
    _write_model(host, str(tmp_path))
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, cfg.vocab, 12)]
    steps = 24
    arg = ",".join(map(str, prompt))
    print(f"node tests/js/decode_graph_gpu.test.js {tmp_path} {arg} {steps}", flush=True)
    res = subprocess.run([NODE, os.path.join(JS_TESTS, "decode_graph_gpu.test.js"), str(tmp_path), arg, str(steps)],
                         cwd=ROOT, capture_output=True, text=True, timeout=110)
    sys.stdout.write(res.stdout[-4000:])
    assert res.returncode == 0, f"node exited {res.returncode}:\n{res.stdout[-3000:]}\n{res.stderr[-3000:]}"
    node = json.loads(next(line for line in res.stdout.splitlines() if line.startswith('{"tokens"')))
    dm = DeviceModel(device, host)
    dec = Decoder(dm)
    try:
        py = Session(dec, SamplingParams(0.7, 0.9, 1.1), seed=0x5EED, capture=False).generate(prompt, steps).tokens
    finally:
        dec.close()
        dm.release()
    assert node["tokens"] == py
    assert node["graph"] == py


def _reference_checkpoint(directory, vocab=4096):
    from enargeia_amd.container import qwen2_tensors, write_enargeia
    from enargeia_amd.model import ModelConfig, synthetic_model

    cfg = ModelConfig(layers=2, vocab=vocab, max_context=256, group=64)
    host = synthetic_model(cfg, base=0xC0DE, fmt="reference")
    path = os.path.join(directory, "qwen2-tiny.enargeia")
    header = write_enargeia(path, qwen2_tensors(host))
    return cfg, path, header


@needs_node
def test_node_reads_container_headers(tmp_path):
    """readEnargeiaHeader from Node over the C++ parser: the same ranges the writer recorded, and
    EnargeiaError for a foreign file."""
    import json

    from enargeia_amd.container import write_raw

    _, path, header = _reference_checkpoint(str(tmp_path), vocab=512)
    bad = os.path.join(str(tmp_path), "bad.enargeia")
    write_raw(bad, b"{}", b"", magic=b"SAFETENS")
    assert os.path.exists(ADDON), f"{ADDON} is not built (python -m enargeia_amd.build)"
    res = subprocess.run([NODE, os.path.join(JS_TESTS, "container_cpu.test.js"), path, bad], cwd=ROOT,
                         capture_output=True, text=True, timeout=60)
    sys.stdout.write(res.stdout[-4000:])
    assert res.returncode == 0, f"node exited {res.returncode}:\n{res.stdout[-3000:]}\n{res.stderr[-3000:]}"
    got = json.loads(next(line[7:] for line in res.stdout.splitlines() if line.startswith("HEADER ")))
    assert got["blockSize"] == 64 and got["quantization"] == header["quantization"]
    assert set(got["tensors"]) == set(header["tensors"])
    for name, entry in header["tensors"].items():
        for field, rng in entry["offsets"].items():
            assert got["tensors"][name][field] == rng, (name, field)
        assert got["tensors"][name]["dtype"] == entry["dtype"]


@needs_node
@pytest.mark.gpu
def test_node_container_decoder_matches_python(tmp_path, device):
    """The same checkpoint loaded from Node (loadQuantized + Decoder) and from Python
    (Container.load + Decoder) gives the same greedy tokens."""
    import json

    from enargeia_amd.container import Container
    from enargeia_amd.model import Decoder

    cfg, path, _ = _reference_checkpoint(str(tmp_path))
    first, steps = 11, 10
    print(f"node tests/js/container_gpu.test.js {path} {first} {steps}", flush=True)
    res = subprocess.run([NODE, os.path.join(JS_TESTS, "container_gpu.test.js"), path, str(first), str(steps)],
                         cwd=ROOT, capture_output=True, text=True, timeout=110)
    sys.stdout.write(res.stdout[-4000:])
    assert res.returncode == 0, f"node exited {res.returncode}:\n{res.stdout[-3000:]}\n{res.stderr[-3000:]}"
    node_tokens = json.loads(next(line for line in res.stdout.splitlines() if line.startswith('{"tokens"')))
    with Container(path) as c:
        model = c.load(device, head_dim=64, max_context=256)
    dec = Decoder(model)
    try:
        dec.reset(0, first)
        py_tokens = [dec.step() for _ in range(steps)]
    finally:
        dec.close()
        model.release()
    assert node_tokens["tokens"] == py_tokens
