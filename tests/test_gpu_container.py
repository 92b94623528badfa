"""A .enargeia checkpoint in the reference quantizer's formats (asymmetric int4 projections in
blocks of 64 with zero-points, a Q8 tied embedding, F32 norms and biases; tools/quantize.py
--embed-dtype q8) loaded through eg_container_upload / eg_container_model_desc and decoded on
the GPU, against the CPU oracle decoder over the same host tensors."""

import ctypes

import numpy as np
import pytest

from enargeia_amd import _lib
from enargeia_amd.container import Container, qwen2_tensors, write_enargeia
from enargeia_amd.model import Decoder, ModelConfig, synthetic_model
from oracle.decode import OracleDecoder
from test_gpu_decode import check_step, prompt_ids

pytestmark = pytest.mark.gpu

CFG = ModelConfig(layers=2, vocab=4096, max_context=256, group=64)


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    host = synthetic_model(CFG, base=0xE4A, fmt="reference")
    path = tmp_path_factory.mktemp("ckpt") / "qwen2-tiny.enargeia"
    write_enargeia(str(path), qwen2_tensors(host))
    return host, path


def test_upload_is_the_blob_verbatim(device, checkpoint):
    host, path = checkpoint
    with Container(str(path)) as c:
        h = c.header()
        blob = c.upload(device)
        try:
            want = np.frombuffer(path.read_bytes()[h["dataOffset"]:], np.uint8)
            got = device.read_array(blob, np.uint8, h["blobBytes"])
            np.testing.assert_array_equal(got, want[:h["blobBytes"]])
        finally:
            _lib.check(_lib.load().eg_buf_free(device.ctx, ctypes.c_void_p(blob)), device.ctx)


def test_loaded_checkpoint_decodes_like_the_oracle(device, checkpoint):
    host, path = checkpoint
    with Container(str(path)) as c:
        model = c.load(device, head_dim=CFG.head_dim, max_context=CFG.max_context, rms_eps=CFG.rms_eps,
                       rope_theta=CFG.rope_theta)
    assert (model.cfg.layers, model.cfg.heads, model.cfg.kv_heads, model.cfg.vocab) == (2, 14, 2, 4096)
    dec = Decoder(model)
    ora = OracleDecoder(host, max_context=CFG.max_context)
    prompt = prompt_ids(24, CFG.vocab, seed=0xE4A)
    checked = 0
    try:
        for pos, tok in enumerate(prompt):
            dec.reset(pos, tok)
            got = dec.step()
            check_step(dec.logits(), ora.step(tok, pos), got, f"prompt pos {pos}")
            checked += 1
        tok = got
        for pos in range(len(prompt), len(prompt) + 12):
            got = dec.step()
            check_step(dec.logits(), ora.step(tok, pos), got, f"greedy pos {pos}")
            tok = got
            checked += 1
    finally:
        dec.close()
        model.release()
    assert checked == 36


def test_f16_table_checkpoint_decodes_like_the_oracle(device, tmp_path):
    """The same checkpoint with its tied table written as F16 (--embed-dtype f16): loaded through
    eg_container_model_desc (16 embedding bits, the table's data range) and decoded against the
    oracle over the same halves, at the decoder bar."""
    host = synthetic_model(CFG, base=0xE4A, fmt="reference", embed_dtype="f16")
    path = tmp_path / "qwen2-tiny-f16.enargeia"
    write_enargeia(str(path), qwen2_tensors(host))
    with Container(str(path)) as c:
        model = c.load(device, head_dim=CFG.head_dim, max_context=CFG.max_context, rms_eps=CFG.rms_eps,
                       rope_theta=CFG.rope_theta)
    assert model.desc.embed_bits == 16
    dec = Decoder(model)
    ora = OracleDecoder(host, max_context=CFG.max_context)
    try:
        prompt = prompt_ids(12, CFG.vocab, seed=0xF16)
        for pos, tok in enumerate(prompt):
            dec.reset(pos, tok)
            got = dec.step()
            check_step(dec.logits(), ora.step(tok, pos), got, f"f16 table prompt pos {pos}")
        tok = got
        for pos in range(len(prompt), len(prompt) + 8):
            got = dec.step()
            check_step(dec.logits(), ora.step(tok, pos), got, f"f16 table greedy pos {pos}")
            tok = got
    finally:
        dec.close()
        model.release()
