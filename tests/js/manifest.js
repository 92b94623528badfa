// A model that tests/test_js_facade.py wrote (raw tensor bytes plus a JSON manifest, as a loader
// would read a checkpoint), uploaded through the facade and described as decoderCreate expects.
'use strict';

const fs = require('fs');
const path = require('path');

function loadModel(eg, dev, dir) {
  const manifest = JSON.parse(fs.readFileSync(path.join(dir, 'manifest.json'), 'utf8'));
  const blob = fs.readFileSync(path.join(dir, 'tensors.bin'));
  const uploads = [];
  const upload = (name) => {
    const t = manifest.tensors[name];
    if (!t) return null;
    const buf = dev.createBuffer({ size: t.bytes, usage: eg.BufferUsage.STORAGE | eg.BufferUsage.COPY_DST, label: name });
    dev.queue.writeBuffer(buf, 0, blob.subarray(t.offset, t.offset + t.bytes));
    uploads.push(buf);
    return buf.ptr;
  };
  const c = manifest.config;
  const mat = (prefix) => ({ packed: upload(`${prefix}.packed`), scales: upload(`${prefix}.scales`), zeros: null });
  const layer = [];
  for (let l = 0; l < c.layers; l++) {
    const p = `layers.${l}`;
    layer.push({
      q: mat(`${p}.q`), k: mat(`${p}.k`), v: mat(`${p}.v`), o: mat(`${p}.o`),
      gate: mat(`${p}.gate`), up: mat(`${p}.up`), down: mat(`${p}.down`),
      qBias: upload(`${p}.q.bias`), kBias: upload(`${p}.k.bias`), vBias: upload(`${p}.v.bias`),
      inputNorm: upload(`${p}.input_norm`), postAttentionNorm: upload(`${p}.post_attention_norm`),
    });
  }
  const desc = {
    layers: c.layers, hidden: c.hidden, heads: c.heads, kvHeads: c.kv_heads, headDim: c.head_dim,
    intermediate: c.intermediate, vocab: c.vocab, maxContext: c.max_context, rmsEps: c.rms_eps,
    ropeTheta: c.rope_theta, encoding: eg.ENCODING.SIGNED, bits: c.bits, blockSize: c.group,
    embedding: mat('embedding'), embedEncoding: eg.ENCODING.SIGNED, embedBits: 8, embedBlockSize: c.hidden,
    finalNorm: upload('final_norm'), layer,
  };
  return { manifest, desc, uploads };
}

module.exports = { loadModel };
