// A .enargeia checkpoint decoded from Node: loadQuantized (one device allocation for the blob,
// the description from the checkpoint names) feeding the decoder binding. Prints the greedy
// tokens as one JSON line for tests/test_js_facade.py to compare with the Python decoder over
// the same file.
//
//   node tests/js/container_gpu.test.js <checkpoint.enargeia> <first token> <steps>
'use strict';

const path = require('path');
const { describe, it, afterAll, expect, run } = require('./harness.js');
const eg = require(path.join(__dirname, '..', '..', 'enargeia_amd', 'js', 'index.js'));

const [file, first, steps] = [process.argv[2], Number(process.argv[3]), Number(process.argv[4] || 8)];
let ctx = null;
let model = null;
const results = {};

afterAll(() => {
  if (model) model.release();
  if (ctx) ctx.device.destroy();
  process.stdout.write(JSON.stringify(results) + '\n');
});

describe('checkpoint', () => {
  it('loads and decodes greedily', async () => {
    ctx = await eg.initGPU();
    const dev = ctx.device;
    model = eg.loadQuantized(dev, file, { headDim: 64, maxContext: 256, rmsEps: 1e-6, ropeTheta: 1e6 });
    expect(model.desc.layers === 2 && model.desc.encoding === eg.ENCODING.OFFSET_ZEROS, 'reference format');
    const dec = new eg.Decoder(dev, model.desc);
    dec.reset(0, first);
    const tokens = [];
    for (let s = 0; s < steps; s++) tokens.push(dec.step());
    results.tokens = tokens;
    dec.destroy();
  });
});

run();
