// Node facade without a GPU: the addon loads and exports every entry point, the uniform
// builders write the reference's byte layouts, and ComputeKernel raises the reference's two
// synchronous errors (kernel.ts:70-81, 97-107) before anything reaches the device.
//
//   node tests/js/facade_cpu.test.js
'use strict';

const path = require('path');
const { describe, it, expect, expectThrows, run } = require('./harness.js');

const eg = require(path.join(__dirname, '..', '..', 'enargeia_amd', 'js', 'index.js'));

const EXPORTS = ['abiVersion', 'create', 'destroy', 'sync', 'getStream', 'bufAlloc', 'bufFree', 'bufWrite', 'bufRead',
  'bufZero', 'matmulQ4Decode', 'matmulQ4Prefill', 'lmHead', 'lmHeadArgmax', 'argmax', 'sample', 'graphBegin',
  'graphEnd', 'graphLaunch', 'graphDestroy', 'decoderCreate', 'decoderReset', 'decoderStep', 'decoderCapture',
  'decoderBuffers', 'decoderDestroy', 'containerOpen', 'containerClose', 'containerHeader', 'containerLoad'];

// A device stand-in: ComputeKernel needs only the limits before it records anything.
const FAKE_DEVICE = { limits: { maxComputeWorkgroupsPerDimension: 65535 }, ctx: null };
const FAKE_PASS = { encoder: { record() { throw new Error('nothing may be recorded'); } } };

describe('addon', () => {
  it('exports every entry point', () => {
    for (const name of EXPORTS) expect(typeof eg.native[name] === 'function', `missing ${name}`);
    expect(eg.native.abiVersion() === 1, 'ABI version 1');
  });

  it('rejects a handle that is not a context', () => {
    expectThrows(() => eg.native.sync({}), (e) => {
      expect(e instanceof TypeError && e.code === 'EG_ERR_INVALID', `${e.name} ${e.code}`);
      expect(/not a context/.test(e.message), e.message);
    }, 'sync({})');
  });

  it('rejects an argument that is not a device pointer', () => {
    expectThrows(() => eg.native.bufFree({}, -4), (e) => expect(e instanceof TypeError, e.message), 'bufFree');
  });

  it('initGPU resolves on a GPU and rejects with GPUUnavailableError without one', async () => {
    let ctx = null;
    try {
      ctx = await eg.initGPU();
    } catch (err) {
      expect(err.name === 'GPUUnavailableError', `${err.name}: ${err.message}`);
      return;
    }
    ctx.device.destroy();
  });
});

describe('uniform builders', () => {
  it('matmulQ4Dims writes the 48-byte Dims of matmul_q4.ts:50-64', () => {
    const u = new Uint32Array(eg.matmulQ4Dims(1, 151936, 896, false, 64));
    expect(u.length === 12, 'twelve u32');
    expect([1, 151936, 896, 0, 64, 14, 151936, 0, 65535, 0, 0, 0].every((v, i) => u[i] === v), Array.from(u).join());
    const w = new Uint32Array(eg.matmulQ4Dims(2, 5, 64, true, 32, 6, 4));
    expect([2, 5, 64, 1, 32, 2, 6, 4, 5, 0, 0, 0].every((v, i) => w[i] === v), Array.from(w).join());
  });

  it('embeddingDims writes the 48-byte Dims of embedding_variants.ts:207-221', () => {
    const u = new Uint32Array(eg.embeddingDims(1, 896, 0, 151936, 896, 0, 3));
    expect([1, 896, 0, 151936, 896, 1, 0, 3, 65535, 0, 0, 0].every((v, i) => u[i] === v), Array.from(u).join());
    const e = new Uint32Array(eg.embeddingDims(1, 896, 0, 0, 64));
    expect(e[8] === 1, 'grid width at least 1');
  });

  it('argmaxDims and sampleDims', () => {
    expect(Array.from(new Uint32Array(eg.argmaxDims(151936, 7))).join() === '151936,7,0,0', 'argmax dims');
    const s = eg.sampleDims(151936, 512, { temperature: 0.7, topP: 0.9, repetitionPenalty: 1.1 }, 0.25);
    expect(s.byteLength === 32, '32 bytes');
    const u = new Uint32Array(s), f = new Float32Array(s);
    expect(u[0] === 151936 && u[1] === 512, 'vocab, historyLength');
    expect(f[2] === Math.fround(0.7) && f[3] === Math.fround(0.9) && f[4] === Math.fround(1.1) && f[5] === 0.25,
      'temperature, topP, repetitionPenalty, random as f32');
    expect(u[6] === 0 && u[7] === 0, 'padding');
  });

  it('workgroup helpers fold past 65535 as the reference does', () => {
    expect(eg.matmulQ4DecodeWorkgroups(151936).join() === '65535,3,1', 'decode fold');
    expect(eg.embeddingHeadWorkgroups(151936).join() === '65535,3,1', 'head fold');
    expect(eg.matmulQ4PrefillWorkgroups(15, 896).join() === '28,1,1', 'prefill tiles');
    expect(eg.coverage(eg.ARGMAX, [1000, 1, 1]).join() === '4,1,1', 'coverage');
  });
});

describe('ComputeKernel', () => {
  it('names the op and the counts on a wrong binding count', () => {
    const k = new eg.ComputeKernel(FAKE_DEVICE, null, eg.MATMUL_Q4_DECODE);
    expectThrows(() => k.bindGroup([1, 2, 3]), (e) => {
      expect(!(e instanceof RangeError), 'a plain Error');
      expect(e.message === 'matmul_q4_decode: expected 7 bindings, got 3', e.message);
    }, 'bindGroup');
  });

  it('throws RangeError for a grid over the limit before recording', () => {
    const k = new eg.ComputeKernel(FAKE_DEVICE, null, eg.embeddingHeadSpec('q8'));
    const bg = k.bindGroup([null, null, null, null, null, null]);
    expectThrows(() => k.encode(FAKE_PASS, bg, [151936, 1, 1]), (e) => {
      expect(e instanceof RangeError, e.name);
      expect(e.message === 'lm_head_q8: 151936 workgroups on axis 0 exceeds the device limit of 65535', e.message);
    }, 'encode');
  });

  it('refuses ops that are not on this path', () => {
    expectThrows(() => new eg.ComputeKernel(FAKE_DEVICE, null, { name: 'rmsnorm', bindings: [] }),
      (e) => expect(/not an op of this library/.test(e.message), e.message), 'constructor');
    expectThrows(() => eg.embeddingHeadSpec('bf16'), (e) => expect(/the dtypes are q4, q8, f16 and f32/.test(e.message), e.message), 'bf16');
    expect(['q4', 'q8', 'f16', 'f32'].map((d) => eg.embeddingHeadSpec(d).bits).join() === '4,8,16,32', 'dtypes');
    expect(eg.embeddingGatherSpec('f16').name === 'embed_gather_f16' && eg.embeddingGatherSpec('f16').bits === 16,
      'gather spec');
  });

  it('carries the format on the spec', () => {
    const s = eg.withFormat(eg.MATMUL_Q4_DECODE, 4, eg.ENCODING.SIGNED);
    expect(s.name === 'matmul_q4_decode' && s.bits === 4 && s.encoding === 1, 'withFormat');
    expect(eg.MATMUL_Q4_DECODE.encoding === 0, 'the original spec is unchanged');
  });
});

run();
