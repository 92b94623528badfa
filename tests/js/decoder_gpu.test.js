// The decoder from Node: loads a model that tests/test_js_facade.py wrote (raw tensor bytes plus
// a JSON manifest, as a loader would read a checkpoint), uploads it, and runs greedy steps
// eagerly and as a replayed hipGraph. Prints the tokens as one JSON line ({"eager": [...],
// "graph": [...]}) so the Python side can compare them with its own decoder over the same weights.
//
//   node tests/js/decoder_gpu.test.js <model directory> <steps>
'use strict';

const fs = require('fs');
const path = require('path');
const { describe, it, afterAll, expect, expectThrows, run } = require('./harness.js');
const eg = require(path.join(__dirname, '..', '..', 'enargeia_amd', 'js', 'index.js'));

const dir = process.argv[2];
const steps = Number(process.argv[3] || 8);
const manifest = JSON.parse(fs.readFileSync(path.join(dir, 'manifest.json'), 'utf8'));
const blob = fs.readFileSync(path.join(dir, 'tensors.bin'));

let ctx = null;
const uploads = [];
const results = {};

async function device() {
  if (!ctx) ctx = await eg.initGPU();
  return ctx;
}

afterAll(() => {
  for (const b of uploads) b.destroy();
  if (ctx) ctx.device.destroy();
  process.stdout.write(JSON.stringify(results) + '\n');
});

/** Uploads one tensor of the manifest; returns its device pointer (null for an absent one). */
function upload(dev, name) {
  const t = manifest.tensors[name];
  if (!t) return null;
  const buf = dev.createBuffer({ size: t.bytes, usage: eg.BufferUsage.STORAGE | eg.BufferUsage.COPY_DST, label: name });
  dev.queue.writeBuffer(buf, 0, blob.subarray(t.offset, t.offset + t.bytes));
  uploads.push(buf);
  return buf.ptr;
}

function describeModel(dev) {
  const c = manifest.config;
  const mat = (prefix) => ({ packed: upload(dev, `${prefix}.packed`), scales: upload(dev, `${prefix}.scales`), zeros: null });
  const layer = [];
  for (let l = 0; l < c.layers; l++) {
    const p = `layers.${l}`;
    layer.push({
      q: mat(`${p}.q`), k: mat(`${p}.k`), v: mat(`${p}.v`), o: mat(`${p}.o`),
      gate: mat(`${p}.gate`), up: mat(`${p}.up`), down: mat(`${p}.down`),
      qBias: upload(dev, `${p}.q.bias`), kBias: upload(dev, `${p}.k.bias`), vBias: upload(dev, `${p}.v.bias`),
      inputNorm: upload(dev, `${p}.input_norm`), postAttentionNorm: upload(dev, `${p}.post_attention_norm`),
    });
  }
  return {
    layers: c.layers, hidden: c.hidden, heads: c.heads, kvHeads: c.kv_heads, headDim: c.head_dim,
    intermediate: c.intermediate, vocab: c.vocab, maxContext: c.max_context, rmsEps: c.rms_eps,
    ropeTheta: c.rope_theta, encoding: eg.ENCODING.SIGNED, bits: c.bits, blockSize: c.group,
    embedding: mat('embedding'), embedEncoding: eg.ENCODING.SIGNED, embedBits: 8, embedBlockSize: c.hidden,
    finalNorm: upload(dev, 'final_norm'), layer,
  };
}

let desc = null;

describe('decoder', () => {
  it('runs greedy steps eagerly', async () => {
    const { device: dev } = await device();
    desc = describeModel(dev);
    const dec = new eg.Decoder(dev, desc);
    dec.reset(0, manifest.first_token);
    const tokens = [];
    for (let s = 0; s < steps; s++) tokens.push(dec.step());
    const logits = dec.logits();
    expect(logits.length === manifest.config.vocab && logits.every(Number.isFinite), 'finite logits');
    results.eager = tokens;
    dec.destroy();
  });

  it('replays a captured step to the same tokens', async () => {
    const { device: dev } = await device();
    const dec = new eg.Decoder(dev, desc);
    dec.reset(0, manifest.first_token);
    dec.capture();
    const tokens = [];
    for (let s = 0; s < steps; s++) tokens.push(dec.step());
    results.graph = tokens;
    expect(JSON.stringify(tokens) === JSON.stringify(results.eager), `graph ${tokens} vs eager ${results.eager}`);
    dec.destroy();
  });

  it('refuses a full context, a bad token and a foreign handle', async () => {
    const { device: dev } = await device();
    const dec = new eg.Decoder(dev, desc);
    expectThrows(() => dec.reset(manifest.config.max_context, 0), (e) => expect(e instanceof RangeError, e.name), 'reset');
    expectThrows(() => dec.reset(0, manifest.config.vocab), (e) => expect(e.code === 'EG_ERR_INVALID', e.code), 'token');
    expectThrows(() => eg.native.decoderStep(dev.ctx, true), (e) => expect(e instanceof TypeError, e.name), 'handle');
    dec.destroy();
  });
});

run();
