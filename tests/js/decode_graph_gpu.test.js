// The reference's runtime loop, restated line for line over the DecodeGraph-shaped binding:
// Session.generate / decodeStep (src/runtime/session.ts:347-375, 416-469) with its mulberry32
// draw source (:75-83) drive `DecodeGraph` through tokenId / history / setPosition / encode /
// submit / readBuffer(result), as they drive the reference's WGSL DecodeGraph. The first token
// comes from the binding's prefill (runPrefill + sampleFromPrefill in one call, whose draw is the
// same mulberry32 stream taken on the device), after which the host draws. Prints one JSON line
// {"tokens": [...], "graph": [...]} for the Python side to compare with its own decoder.
//
//   node tests/js/decode_graph_gpu.test.js <model directory> <prompt ids, comma-separated> <maxTokens>
'use strict';

const path = require('path');
const { describe, it, afterAll, expect, run } = require('./harness.js');
const eg = require(path.join(__dirname, '..', '..', 'enargeia_amd', 'js', 'index.js'));
const { loadModel } = require('./manifest.js');

const dir = process.argv[2];
const prompt = process.argv[3].split(',').map(Number);
const maxTokens = Number(process.argv[4] || 16);
const SAMPLING = { temperature: 0.7, topP: 0.9, repetitionPenalty: 1.1 };  // ui/engine.ts:261
const results = {};
let gpu = null;
let model = null;

afterAll(() => {
  if (model) for (const b of model.uploads) b.destroy();
  if (gpu) gpu.device.destroy();
  process.stdout.write(JSON.stringify(results) + '\n');
});

/** session.ts:75-83 */
function mulberry32(seed) {
  let s = seed >>> 0;
  return () => {
    s = (s + 0x6d2b79f5) >>> 0;
    let t = Math.imul(s ^ (s >>> 15), 1 | s);
    t = (t + Math.imul(t ^ (t >>> 7), 61 | t)) ^ t;
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  };
}

/** The parts of Session (session.ts) that drive the decode graph. */
class Session {
  constructor(ctx, decode, sampling, seed) {
    this.device = ctx.device;
    this.queue = ctx.queue;
    this.pool = new eg.BufferPool(ctx.device);
    this.decode = decode;
    this.random = mulberry32(seed);
    this.tokens = [];
    this.filled = 0;
    decode.setSampling(sampling);
    decode.seed(seed);
  }

  /** runPrefill + sampleFromPrefill (session.ts:326-344, 472-495): one draw. */
  async prefillAndSample(promptIds) {
    const first = this.decode.prefill(this.filled, promptIds);
    this.random();  // the draw sampleFromPrefill takes; the decoder took the same value
    this.filled += promptIds.length;
    this.tokens = [...promptIds];
    return first;
  }

  /** session.ts:347-375 */
  async decodeStep(token) {
    const position = this.filled;
    this.queue.writeBuffer(this.decode.tokenId.buffer, 0, new Uint32Array([token]));
    this.queue.writeBuffer(this.decode.history.buffer, 0, new Uint32Array(this.tokens));
    this.decode.setPosition(position, this.tokens.length, this.random());

    const encoder = this.device.createCommandEncoder({ label: 'decode' });
    this.decode.encode(encoder, position);
    this.queue.submit([encoder.finish()]);

    const bytes = await eg.readBuffer({ device: this.device, queue: this.queue }, this.pool, this.decode.result);
    this.filled += 1;
    return new Uint32Array(bytes)[0];
  }

  /** session.ts:416-469, without timing and telemetry */
  async generate(promptIds, max) {
    const produced = [];
    let next = await this.prefillAndSample(promptIds);
    produced.push(next);
    this.tokens.push(next);
    for (let i = 1; i < max; i++) {
      if (this.filled >= this.decode.config.maxContext) break;
      next = await this.decodeStep(next);
      produced.push(next);
      this.tokens.push(next);
    }
    return produced;
  }
}

describe('DecodeGraph', () => {
  it('runs Session.generate step by step', async () => {
    gpu = await eg.initGPU();
    model = loadModel(eg, gpu.device, dir);
    const decode = new eg.DecodeGraph(gpu.device, model.desc);
    const session = new Session(gpu, decode, SAMPLING, 0x5eed);
    results.tokens = await session.generate(prompt, maxTokens);
    expect(results.tokens.length === maxTokens, `${results.tokens.length} tokens`);
    // host-driven sampled steps: the layers (one persistent launch, or 5 per layer), the LM head,
    // the sampler, the tail and the input preparation
    const sampled = decode.dispatchCount;
    expect(sampled === 5 || sampled === 5 * model.desc.layers + 4, `dispatchCount ${sampled}`);
    decode.seed(0x5eed);  // device-chained again
    decode.setSampling({ temperature: 0, topP: 1, repetitionPenalty: 1 });
    expect(decode.dispatchCount === sampled - 2, `greedy dispatchCount ${decode.dispatchCount}`);
    decode.destroy();
  });

  it('replays a captured step to the same tokens', async () => {
    const decode = new eg.DecodeGraph(gpu.device, model.desc);
    const session = new Session(gpu, decode, SAMPLING, 0x5eed);
    decode.capture();
    results.graph = await session.generate(prompt, maxTokens);
    expect(JSON.stringify(results.graph) === JSON.stringify(results.tokens), `graph ${results.graph} vs ${results.tokens}`);
    decode.destroy();
  });
});

run();
