"""The .enargeia container through the C++ parser (eg_container_*), on the CPU.

The layout and every check follow the reference's reader (src/model/enargeia.ts:96-242) and
writer (tools/quantize.py:190-260): a round trip through enargeia_amd.container.write_enargeia,
then one malformed file per check the reference makes, each asserting the reference's message.
Parsing needs no device; the upload and the decoder run in tests/test_gpu_container.py.
"""

import json
import os
import struct

import numpy as np
import pytest

from enargeia_amd import _lib
from enargeia_amd.container import ALIGN, Container, write_enargeia, write_raw
from enargeia_amd.quant import normal, quantize_asym


def _open_error(path) -> str:
    with pytest.raises(_lib.EgError) as e:
        Container(str(path))
    return str(e.value)


def _header_file(tmp_path, header: dict, blob: bytes = b"\0" * 4096, name="h.enargeia"):
    path = tmp_path / name
    write_raw(str(path), json.dumps(header).encode(), blob)
    return path


def test_round_trip_ranges_and_header(tmp_path):
    w = normal(96 * 128, 3, 0.02)
    q4 = quantize_asym(w, 96, 128, 4, 64)
    q8 = quantize_asym(normal(40 * 64, 4, 0.02), 40, 64, 8, 64)
    norm = np.linspace(0.5, 1.5, 128, dtype=np.float32)
    half = np.arange(6, dtype=np.float16).reshape(2, 3)
    path = tmp_path / "m.enargeia"
    header = write_enargeia(str(path), {"w.q4": q4, "e.q8": q8, "n": norm, "h": half})
    with Container(str(path)) as c:
        h = c.header()
        raw_len = len(json.dumps(header, separators=(",", ":")).encode())
        assert h["version"] == 1 and h["blockSize"] == 64 and h["tensorCount"] == 4
        assert h["quantization"] == "asymmetric-int4-blockwise"
        assert h["headerLength"] == raw_len
        # the blob starts at the first 256-byte boundary after magic + version + length + header
        assert h["dataOffset"] == -(-(16 + raw_len) // ALIGN) * ALIGN
        assert h["fileSize"] == os.path.getsize(path)
        names = [t.name for t in c.tensors()]
        assert names == ["w.q4", "e.q8", "n", "h"]  # header order (Object.entries)
        t = c.find("w.q4")
        assert (t.dtype, t.bits, t.shape, t.block_size, t.blocks_per_row, t.total_blocks) == \
            ("Q4", 4, (96, 128), 64, 2, 192)
        off = header["tensors"]["w.q4"]["offsets"]
        assert t.packed == tuple(off["packed"]) and t.scales == tuple(off["scales"]) and t.zeros == tuple(off["zeros"])
        assert all(r[0] % ALIGN == 0 for r in (t.packed, t.scales, t.zeros))
        t8 = c.find("e.q8")
        assert (t8.dtype, t8.bits, t8.total_blocks) == ("Q8", 8, 40)
        assert t8.zeros[1] - t8.zeros[0] == 40  # ceil(40 / 4) words
        assert c.find("n").dtype == "F32" and c.find("n").shape == (128,)
        assert c.find("h").dtype == "F16" and c.find("h").data[1] - c.find("h").data[0] == 12
        # the bytes at those ranges are the streams, verbatim
        blob = path.read_bytes()[h["dataOffset"]:]
        assert blob[t.packed[0]:t.packed[1]] == q4.packed.tobytes()
        assert blob[t.scales[0]:t.scales[1]] == q4.scales.tobytes()
        assert blob[t.zeros[0]:t.zeros[1]] == q4.zeros.tobytes()
        with pytest.raises(_lib.EgError, match="^nope is missing$"):
            c.find("nope")


@pytest.mark.parametrize("header_len", [0, 1, 239, 240, 241, 495, 496])
def test_blob_offset_at_256_boundaries(tmp_path, header_len):
    # enargeia.ts:146: dataOffset = total + (-total mod 256), total = 16 + headerLength
    body = {"tensors": {}}
    raw = json.dumps(body).encode()
    raw = raw + b" " * max(0, header_len - len(raw))
    path = tmp_path / "b.enargeia"
    write_raw(str(path), raw, b"")
    with Container(str(path)) as c:
        total = 16 + len(raw)
        assert c.header()["dataOffset"] == total + (-total % 256)


def test_prefix_errors(tmp_path):
    short = tmp_path / "short"
    short.write_bytes(b"ENARG")
    assert _open_error(short) == "need at least 16 bytes to read the header length"
    bad = tmp_path / "bad"
    write_raw(str(bad), b"{}", b"", magic=b"SAFETENS")
    assert _open_error(bad) == 'not a .enargeia file: magic is "SAFETENS"'
    v2 = tmp_path / "v2"
    write_raw(str(v2), b"{}", b"", version=2)
    assert _open_error(v2) == "unsupported .enargeia version 2, expected 1"
    big = tmp_path / "big"
    big.write_bytes(b"ENARGEIA" + struct.pack("<II", 1, 64 * 1024 * 1024 + 1))
    assert _open_error(big) == "header length 67108865 exceeds the 67108864 byte limit"
    cut = tmp_path / "cut"
    cut.write_bytes(b"ENARGEIA" + struct.pack("<II", 1, 100) + b"{")
    assert _open_error(cut) == "header needs 116 bytes, got 17"
    missing = tmp_path / "missing"
    with pytest.raises(_lib.EgError, match="cannot open"):
        Container(str(missing))


def test_header_errors(tmp_path):
    p = tmp_path / "j"
    write_raw(str(p), b'{"tensors": {', b"")
    assert _open_error(p).startswith("header is not valid JSON: ")
    assert _open_error(_header_file(tmp_path, {"blockSize": 64})) == 'header has no "tensors" object'
    assert _open_error(_header_file(tmp_path, {"tensors": []})) == 'header has no "tensors" object'


def _tensor_error(tmp_path, entry, block=64) -> str:
    return _open_error(_header_file(tmp_path, {"blockSize": block, "tensors": {"a": entry}}))


def test_tensor_errors(tmp_path):
    q = {"dtype": "Q4", "shape": [2, 64], "offsets": {"packed": [0, 64], "scales": [256, 264], "zeros": [512, 516]}}
    assert _tensor_error(tmp_path, [1, 2]) == 'tensor "a" is not an object'
    assert _tensor_error(tmp_path, dict(q, shape=[2, 0])) == 'tensor "a" has a malformed shape'
    assert _tensor_error(tmp_path, dict(q, shape=[2, 1.5])) == 'tensor "a" has a malformed shape'
    assert _tensor_error(tmp_path, dict(q, shape="2x64")) == 'tensor "a" has a malformed shape'
    assert _tensor_error(tmp_path, {"dtype": "Q4", "shape": [2, 64]}) == 'tensor "a" has no offsets'
    f = {"dtype": "F32", "shape": [4], "offsets": {"data": [0, 12]}}
    assert _tensor_error(tmp_path, f) == "a: F32 range is 12 bytes, shape needs 16"
    assert _tensor_error(tmp_path, dict(f, dtype="F16", offsets={"data": [0, 4]})) == \
        "a: F16 range is 4 bytes, shape needs 8"
    assert _tensor_error(tmp_path, dict(q, dtype="BF16")) == 'tensor "a" has unsupported dtype "BF16"'
    assert _tensor_error(tmp_path, dict(q, shape=[2, 64, 1])) == "a: Q4 tensors must be 2-D, got [2, 64, 1]"
    assert _tensor_error(tmp_path, dict(q, shape=[2, 96])) == "a: reduction axis 96 is not a multiple of block size 64"
    # a tensor's own blockSize overrides the header's
    assert _tensor_error(tmp_path, dict(q, shape=[2, 96], blockSize=32)) == "a: packed is 64 bytes, expected 96"
    assert _tensor_error(tmp_path, dict(q, offsets={"scales": [0, 8], "zeros": [0, 4]})) == \
        "a: offsets.packed is malformed"
    assert _tensor_error(tmp_path, dict(q, offsets={**q["offsets"], "scales": [264, 256]})) == \
        "a: offsets.scales runs backwards"
    assert _tensor_error(tmp_path, dict(q, offsets={**q["offsets"], "packed": [0, -64]})) == \
        "a: offsets.packed is malformed"
    assert _tensor_error(tmp_path, dict(q, offsets={**q["offsets"], "packed": [0, 60]})) == \
        "a: packed is 60 bytes, expected 64"
    assert _tensor_error(tmp_path, dict(q, offsets={**q["offsets"], "scales": [256, 260]})) == \
        "a: scales is 4 bytes, expected 8"
    assert _tensor_error(tmp_path, dict(q, offsets={**q["offsets"], "zeros": [512, 520]})) == \
        "a: zeros is 8 bytes, expected 4"
    q8 = {"dtype": "Q8", "shape": [3, 64], "offsets": {"packed": [0, 192], "scales": [256, 268], "zeros": [512, 516]}}
    with Container(str(_header_file(tmp_path, {"tensors": {"a": q8}}))) as c:
        assert c.find("a").total_blocks == 3  # ceil(3 / 4) zero words = 4 bytes


def test_ranges_must_lie_in_the_file(tmp_path):
    f = {"dtype": "F32", "shape": [4], "offsets": {"data": [4096, 4112]}}
    msg = _open_error(_header_file(tmp_path, {"tensors": {"a": f}}, blob=b"\0" * 64))
    assert "past the end of the" in msg


def test_library_symbols_without_a_device():
    lib = _lib.load()
    for name in ("eg_container_open", "eg_container_upload", "eg_container_model_desc"):
        assert hasattr(lib, name)


# ---- the decoder description over Qwen2 checkpoint names ------------------------------------

FAKE_BLOB = 0x7F0000000000  # describe() only adds offsets to it


@pytest.fixture(scope="module")
def ref_checkpoint(tmp_path_factory):
    from enargeia_amd.container import qwen2_tensors
    from enargeia_amd.model import ModelConfig, synthetic_model
    cfg = ModelConfig(layers=3, hidden=128, heads=4, kv_heads=2, head_dim=32, intermediate=256, vocab=512,
                      max_context=256, group=64)
    host = synthetic_model(cfg, fmt="reference")
    tensors = qwen2_tensors(host)
    path = tmp_path_factory.mktemp("ckpt") / "tiny.enargeia"
    header = write_enargeia(str(path), tensors)
    return cfg, host, tensors, header, path


def test_model_desc_points_into_the_blob(ref_checkpoint):
    cfg, host, tensors, header, path = ref_checkpoint
    offs = {n: e["offsets"] for n, e in header["tensors"].items()}
    with Container(str(path)) as c:
        desc, layers, got = c.describe(FAKE_BLOB, head_dim=32, max_context=256, rms_eps=1e-5, rope_theta=1e4)
    assert (desc.layers, desc.hidden, desc.heads, desc.kv_heads, desc.head_dim, desc.intermediate, desc.vocab) == \
        (3, 128, 4, 2, 32, 256, 512)
    assert (desc.encoding, desc.bits, desc.block_size, desc.embed_encoding, desc.embed_bits, desc.embed_block_size) == \
        (_lib.ENC_OFFSET_ZEROS, 4, 64, _lib.ENC_OFFSET_ZEROS, 8, 64)
    assert desc.max_context == 256 and abs(desc.rms_eps - 1e-5) < 1e-12 and desc.rope_theta == 1e4
    e = offs["model.embed_tokens.weight"]
    assert (desc.embedding.packed, desc.embedding.scales, desc.embedding.zeros) == \
        (FAKE_BLOB + e["packed"][0], FAKE_BLOB + e["scales"][0], FAKE_BLOB + e["zeros"][0])
    assert desc.final_norm == FAKE_BLOB + offs["model.norm.weight"]["data"][0]
    for i in range(3):
        p = f"model.layers.{i}."
        L = layers[i]
        assert L.down.packed == FAKE_BLOB + offs[p + "mlp.down_proj.weight"]["packed"][0]
        assert L.k.zeros == FAKE_BLOB + offs[p + "self_attn.k_proj.weight"]["zeros"][0]
        assert L.v_bias == FAKE_BLOB + offs[p + "self_attn.v_proj.bias"]["data"][0]
        assert L.post_attention_norm == FAKE_BLOB + offs[p + "post_attention_layernorm.weight"]["data"][0]
    assert got.heads == 4 and got.group == 64


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_model_desc_takes_f16_and_f32_tables(tmp_path, ref_checkpoint, dtype):
    """An F16 / F32 tied table (--embed-dtype f16 / f32): the description points at its data
    range with 16 / 32 embedding bits and no scales or zero-points."""
    cfg, host, tensors, header, path = ref_checkpoint
    t = dict(tensors, **{"model.embed_tokens.weight": np.zeros((512, 128), dtype)})
    p = tmp_path / "dense.enargeia"
    h = write_enargeia(str(p), t)
    with Container(str(p)) as c:
        desc, layers, got = c.describe(FAKE_BLOB, head_dim=32, max_context=256, rms_eps=1e-5, rope_theta=1e4)
    assert (desc.vocab, desc.hidden, desc.embed_bits, desc.embed_block_size) == \
        (512, 128, 16 if dtype == np.float16 else 32, 128)
    assert desc.embedding.packed == FAKE_BLOB + h["tensors"]["model.embed_tokens.weight"]["offsets"]["data"][0]
    assert not desc.embedding.scales and not desc.embedding.zeros


def _describe_error(tmp_path, tensors, **kw) -> str:
    path = tmp_path / "bad.enargeia"
    write_enargeia(str(path), tensors)
    with Container(str(path)) as c:
        with pytest.raises(_lib.EgError) as e:
            c.describe(FAKE_BLOB, **{"head_dim": 32, **kw})
    return str(e.value)


def test_model_desc_errors(tmp_path, ref_checkpoint):
    cfg, host, tensors, header, path = ref_checkpoint
    t = dict(tensors)
    del t["model.norm.weight"]
    assert _describe_error(tmp_path, t) == "model.norm.weight is missing"
    t = dict(tensors)
    del t["model.layers.1.mlp.up_proj.weight"]
    assert _describe_error(tmp_path, t) == "model.layers.1.mlp.up_proj.weight is missing"
    t = dict(tensors, **{"lm_head.weight": tensors["model.embed_tokens.weight"]})
    assert "tied embeddings only" in _describe_error(tmp_path, t)
    t = dict(tensors, **{"model.embed_tokens.weight": np.zeros(512 * 128, np.float16)})
    assert _describe_error(tmp_path, t) == "model.embed_tokens.weight: an F16 table must be 2-D"
    from enargeia_amd.quant import normal, quantize_asym
    t = dict(tensors, **{"model.layers.2.mlp.gate_proj.weight": quantize_asym(normal(256 * 128, 5, 0.02), 256, 128, 4, 32)})
    assert "4-bit blocks of 32, the model's first projection has 4-bit blocks of 64" in _describe_error(tmp_path, t)
    assert "not multiples of head_dim 48" in _describe_error(tmp_path, tensors, head_dim=48)
    t = dict(tensors, **{"model.layers.0.input_layernorm.weight": np.ones(64, np.float32)})
    assert _describe_error(tmp_path, t) == "model.layers.0.input_layernorm.weight: expected an F32 vector of 128"
