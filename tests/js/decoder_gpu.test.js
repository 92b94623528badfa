// The decoder from Node: loads a model that tests/test_js_facade.py wrote (raw tensor bytes plus
// a JSON manifest, as a loader would read a checkpoint), uploads it, and runs greedy steps
// eagerly and as a replayed hipGraph. Prints the tokens as one JSON line ({"eager": [...],
// "graph": [...]}) so the Python side can compare them with its own decoder over the same weights.
//
//   node tests/js/decoder_gpu.test.js <model directory> <steps>
'use strict';

const path = require('path');
const { describe, it, afterAll, expect, expectThrows, run } = require('./harness.js');
const eg = require(path.join(__dirname, '..', '..', 'enargeia_amd', 'js', 'index.js'));
const { loadModel } = require('./manifest.js');

const dir = process.argv[2];
const steps = Number(process.argv[3] || 8);

let ctx = null;
let model = null;
const results = {};

async function device() {
  if (!ctx) ctx = await eg.initGPU();
  return ctx;
}

afterAll(() => {
  if (model) for (const b of model.uploads) b.destroy();
  if (ctx) ctx.device.destroy();
  process.stdout.write(JSON.stringify(results) + '\n');
});

let desc = null;

describe('decoder', () => {
  it('runs greedy steps eagerly', async () => {
    const { device: dev } = await device();
    model = loadModel(eg, dev, dir);
    desc = model.desc;
    const dec = new eg.Decoder(dev, desc);
    dec.reset(0, model.manifest.first_token);
    const tokens = [];
    for (let s = 0; s < steps; s++) tokens.push(dec.step());
    const logits = dec.logits();
    expect(logits.length === model.manifest.config.vocab && logits.every(Number.isFinite), 'finite logits');
    results.eager = tokens;
    dec.destroy();
  });

  it('replays a captured step to the same tokens', async () => {
    const { device: dev } = await device();
    const dec = new eg.Decoder(dev, desc);
    dec.reset(0, model.manifest.first_token);
    dec.capture();
    const tokens = [];
    for (let s = 0; s < steps; s++) tokens.push(dec.step());
    results.graph = tokens;
    expect(JSON.stringify(tokens) === JSON.stringify(results.eager), `graph ${tokens} vs eager ${results.eager}`);
    dec.destroy();
  });

  it('runs greedy steps over an f32 KV cache', async () => {
    const { device: dev } = await device();
    const dec = new eg.Decoder(dev, Object.assign({}, desc, { cacheDType: 'f32' }));
    dec.reset(0, model.manifest.first_token);
    const tokens = [];
    for (let s = 0; s < steps; s++) tokens.push(dec.step());
    results.f32 = tokens;
    dec.destroy();
    expectThrows(() => new eg.Decoder(dev, Object.assign({}, desc, { cacheDType: 'bf16' })),
      (e) => expect(e.code === 'EG_ERR_INVALID', e.code), 'cacheDType');
  });

  it('refuses a full context, a bad token and a foreign handle', async () => {
    const { device: dev } = await device();
    const dec = new eg.Decoder(dev, desc);
    expectThrows(() => dec.reset(model.manifest.config.max_context, 0), (e) => expect(e instanceof RangeError, e.name), 'reset');
    expectThrows(() => dec.reset(0, model.manifest.config.vocab), (e) => expect(e.code === 'EG_ERR_INVALID', e.code), 'token');
    expectThrows(() => eg.native.decoderStep(dev.ctx, true), (e) => expect(e instanceof TypeError, e.name), 'handle');
    dec.destroy();
  });
});

run();
