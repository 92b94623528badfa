// The ops of this path driven from Node exactly as the reference's kernel tests drive them
// (test/kernels/matmul_q4.test.ts:33-67: pool.acquire, queue.writeBuffer, kernel.uniform,
// encoder + pass + encode, submit, readFloats), through the N-API addon and the C ABI on the
// GPU. Expected values come from the JS statement of the reference's CPU math in
// tests/golden/gen_js_vectors.js (mulberry32, the block-wise int4 quantizer, float64 linearQ4).
//
//   node tests/js/kernels_gpu.test.js          (needs an MI355X)
'use strict';

const path = require('path');
const { describe, it, afterAll, expect, expectThrows, expectMatches, run: runAll } = require('./harness.js');
const ref = require('../golden/gen_js_vectors.js');
const eg = require(path.join(__dirname, '..', '..', 'enargeia_amd', 'js', 'index.js'));

const FP32_TOLERANCE = { abs: 1e-4, rel: 1e-4 };  // test/reference/matmul.ts:88
const STORAGE = eg.BufferUsage.STORAGE | eg.BufferUsage.COPY_DST | eg.BufferUsage.COPY_SRC;

let shared = null;
async function gpu() {
  if (!shared) {
    const ctx = await eg.initGPU();
    shared = { ctx, pool: new eg.BufferPool(ctx.device, { label: 'test' }), cache: new eg.PipelineCache(ctx.device) };
  }
  return shared;
}

afterAll(() => {
  if (shared) {
    shared.pool.destroy();
    shared.ctx.device.destroy();
  }
});

/** The reference test's run() (matmul_q4.test.ts:33-67); a null input binds no buffer. */
async function run(spec, inputs, outputElements, uniform, workgroups, outType) {
  const { ctx, pool, cache } = await gpu();
  const kernel = new eg.ComputeKernel(ctx.device, cache, spec);
  const buffers = [];
  for (const input of inputs) {
    if (input === null) {
      buffers.push(null);
      continue;
    }
    const buffer = pool.acquire(Math.max(4, input.byteLength), STORAGE, 'in');
    ctx.queue.writeBuffer(buffer.buffer, 0, input);
    buffers.push(buffer);
  }
  const out = pool.acquire(Math.max(4, outputElements * 4), STORAGE, 'out');
  const dims = kernel.uniform(pool);
  ctx.queue.writeBuffer(dims.buffer, 0, uniform);

  const encoder = ctx.device.createCommandEncoder();
  pool.clear(encoder, out);
  const pass = encoder.beginComputePass();
  kernel.encode(pass, kernel.bindGroup([...buffers, out, dims]), workgroups);
  pass.end();
  ctx.queue.submit([encoder.finish()]);

  const bytes = await eg.readBuffer(ctx, pool, out);
  pool.release(dims);
  pool.release(out);
  for (const buffer of buffers.reverse()) if (buffer) pool.release(buffer);
  const values = outType === 'u32' ? new Uint32Array(bytes) : new Float32Array(bytes);
  return values.subarray(0, outputElements);
}

// ---- reference-side arithmetic ----------------------------------------------------------------

const f32 = new Float32Array(1);
const u32 = new Uint32Array(f32.buffer);

/** f32 -> bf16, round to nearest even (finite inputs). */
function bf16(v) {
  f32[0] = v;
  const u = u32[0];
  u32[0] = ((u + 0x7fff + ((u >>> 16) & 1)) >>> 0) & 0xffff0000;
  return f32[0];
}

/** The bf16 model of the prefill: bf16(x) . bf16(f32 dequantized weight), float64 sum. */
function linearBf16(x, q, bias, m) {
  const n = q.rows, k = q.cols;
  const w = new Float32Array(n * k);
  for (let r = 0; r < n; r++) for (let c = 0; c < k; c++) w[r * k + c] = bf16(Math.fround(ref.weightAt(q, r, c)));
  const xb = Float32Array.from(x, bf16);
  const y = new Float32Array(m * n);
  for (let i = 0; i < m; i++) {
    for (let r = 0; r < n; r++) {
      let s = bias ? bias[r] : 0;
      for (let c = 0; c < k; c++) s += xb[i * k + c] * w[r * k + c];
      y[i * n + r] = s;
    }
  }
  return y;
}

function rmsOf(a) {
  let s = 0;
  for (const v of a) s += v * v;
  return Math.sqrt(s / Math.max(1, a.length));
}

/** Symmetric int8 per row (absmax/127), two's-complement bytes, 4 per u32 little-endian. */
function quantizeSym8Rows(values, rows, cols) {
  const scales = new Float32Array(rows);
  const packed = new Uint32Array((rows * cols) / 4);
  const codes = new Int8Array(rows * cols);
  for (let r = 0; r < rows; r++) {
    let amax = 0;
    for (let c = 0; c < cols; c++) amax = Math.max(amax, Math.abs(values[r * cols + c]));
    const s = Math.fround(amax > 0 ? amax / 127 : 1);
    scales[r] = s;
    for (let c = 0; c < cols; c++) {
      const e = r * cols + c;
      const q = Math.max(-127, Math.min(127, Math.round(values[e] / s)));
      codes[e] = q;
      packed[e >>> 2] = (packed[e >>> 2] | ((q & 0xff) << ((e & 3) * 8))) >>> 0;
    }
  }
  return { rows, cols, scales, packed, codes };
}

// ---- matmul_q4_decode (matmul_q4.test.ts:198-231) -----------------------------------------------

describe('matmul_q4_decode', () => {
  for (const n of [896, 128, 4864]) {
    it(`matches the reference for a single row at n=${n}`, async () => {
      const k = 896;
      const x = ref.uniformMinusHalf(k, 41);
      const q = ref.quantizeAsym4(ref.uniformMinusHalf(n * k, 42), n, k, 64);
      const bias = ref.uniformMinusHalf(n, 43);
      const actual = await run(eg.MATMUL_Q4_DECODE, [x, q.packed, q.scales, q.zeros, bias], n,
        eg.matmulQ4Dims(1, n, k, true, q.blockSize), eg.matmulQ4DecodeWorkgroups(n));
      expectMatches(actual, ref.gemm(x, q, bias, 1), FP32_TOLERANCE, `q4 decode n=${n}`);
    });
  }

  it('agrees with the prefill kernel at m=1', async () => {
    const n = 256, k = 192;
    const x = ref.uniformMinusHalf(k, 51);
    const q = ref.quantizeAsym4(ref.uniformMinusHalf(n * k, 52), n, k, 64);
    const decode = await run(eg.MATMUL_Q4_DECODE, [x, q.packed, q.scales, q.zeros, new Float32Array(n)], n,
      eg.matmulQ4Dims(1, n, k, false, q.blockSize), eg.matmulQ4DecodeWorkgroups(n));
    const prefill = await run(eg.MATMUL_Q4_PREFILL, [x, q.packed, q.scales, q.zeros, new Float32Array(n)], n,
      eg.matmulQ4Dims(1, n, k, false, q.blockSize), eg.matmulQ4PrefillWorkgroups(1, n));
    // The prefill multiplies in bf16: 2e-2 of the output scale, the bf16 bar.
    const rms = rmsOf(decode);
    expectMatches(prefill, decode, { abs: 2e-2 * rms, rel: 2e-2 }, 'decode vs prefill');
  });

  it('writes only [outOffset, outOffset + n)', async () => {
    const k = 64;
    const x = new Float32Array(k).fill(1);
    const q = ref.quantizeAsym4(new Float32Array(2 * k).fill(0.5), 2, k, 64);
    const actual = await run(eg.MATMUL_Q4_DECODE, [x, q.packed, q.scales, q.zeros, new Float32Array(2)], 6,
      eg.matmulQ4Dims(1, 2, k, false, q.blockSize, 2, 4), eg.matmulQ4DecodeWorkgroups(2));
    expect(actual[0] === 0 && actual[3] === 0, 'untouched below outOffset');
    expect(Math.abs(actual[4] - 32) < 1e-3 && Math.abs(actual[5] - 32) < 1e-3, `${actual[4]} ${actual[5]}`);
  });

  it('runs the BASELINE symmetric int4 g32 format (zeros unbound) at 4864x896', async () => {
    const n = 4864, k = 896;
    const values = ref.uniformMinusHalf(n * k, 71);
    const q = { rows: n, cols: k, blockSize: 32, packed: new Uint32Array((n * k) / 8), scales: new Float32Array((n * k) / 32) };
    for (let g = 0; g < (n * k) / 32; g++) {
      let amax = 0;
      for (let j = 0; j < 32; j++) amax = Math.max(amax, Math.abs(values[g * 32 + j]));
      const s = Math.fround(amax / 7);
      q.scales[g] = s;
      for (let j = 0; j < 32; j++) {
        const e = g * 32 + j;
        const c = Math.max(-7, Math.min(7, Math.round(values[e] / s)));
        q.packed[e >>> 3] = (q.packed[e >>> 3] | ((c & 15) << ((e & 7) * 4))) >>> 0;
      }
    }
    const x = ref.uniformMinusHalf(k, 72);
    const expected = new Float32Array(n);
    for (let r = 0; r < n; r++) {
      let s = 0;
      for (let c = 0; c < k; c++) {
        const e = r * k + c;
        let code = (q.packed[e >>> 3] >>> ((e & 7) * 4)) & 15;
        if (code >= 8) code -= 16;
        s += x[c] * code * q.scales[r * (k / 32) + (c >> 5)];
      }
      expected[r] = s;
    }
    const spec = eg.withFormat(eg.MATMUL_Q4_DECODE, 4, eg.ENCODING.SIGNED);
    const actual = await run(spec, [x, q.packed, q.scales, null, null], n, eg.matmulQ4Dims(1, n, k, false, 32),
      eg.matmulQ4DecodeWorkgroups(n));
    expectMatches(actual, expected, { abs: 1e-5 * rmsOf(expected), rel: 1e-3 }, 'sym int4 decode');
  });
});

// ---- matmul_q4_prefill (matmul_q4.test.ts:149-196) ----------------------------------------------

describe('matmul_q4_prefill', () => {
  for (const [m, n, k] of [[15, 896, 896], [15, 128, 896], [4, 4864, 896], [64, 32, 64]]) {
    it(`matches the bf16 model and the fp32 reference at ${m}x${n}x${k}`, async () => {
      const x = ref.uniformMinusHalf(m * k, 11);
      const q = ref.quantizeAsym4(ref.uniformMinusHalf(n * k, 12), n, k, 64);
      const bias = ref.uniformMinusHalf(n, 13);
      const actual = await run(eg.MATMUL_Q4_PREFILL, [x, q.packed, q.scales, q.zeros, bias], m * n,
        eg.matmulQ4Dims(m, n, k, true, q.blockSize), eg.matmulQ4PrefillWorkgroups(m, n));
      const model = linearBf16(x, q, bias, m);
      expectMatches(actual, model, { abs: 1e-4 * rmsOf(model), rel: 1e-4 }, `bf16 model ${m}x${n}x${k}`);
      const fp32 = ref.gemm(x, q, bias, m);
      expectMatches(actual, fp32, { abs: 2e-2 * rmsOf(fp32), rel: 2e-2 }, `fp32 reference ${m}x${n}x${k}`);
    });
  }

  it('writes at outOffset with outStride, as the tied LM head needs', async () => {
    const k = 64;
    const x = new Float32Array(k).fill(1);
    const q = ref.quantizeAsym4(new Float32Array(2 * k).fill(0.5), 2, k, 64);
    const actual = await run(eg.MATMUL_Q4_PREFILL, [x, q.packed, q.scales, q.zeros, new Float32Array(2)], 6,
      eg.matmulQ4Dims(1, 2, k, false, q.blockSize, 6, 4), eg.matmulQ4PrefillWorkgroups(1, 2));
    expect(actual[0] === 0, 'index 0 untouched');
    expect(Math.abs(actual[4] - 32) < 1e-3 && Math.abs(actual[5] - 32) < 1e-3, `${actual[4]} ${actual[5]}`);
  });
});

// ---- LM head, argmax, sample -------------------------------------------------------------------

describe('lm head', () => {
  const V = 151936, H = 896;
  let head = null;
  function config2() {
    if (!head) {
      const table = ref.uniformMinusHalf(V * H, 2);
      const q = quantizeSym8Rows(table, V, H);
      const h = ref.uniformMinusHalf(H, 3);
      const logits = new Float32Array(V);
      for (let r = 0; r < V; r++) {
        let s = 0;
        for (let c = 0; c < H; c++) s += h[c] * q.codes[r * H + c];
        logits[r] = s * q.scales[r];
      }
      head = { q, h, logits };
    }
    return head;
  }

  it('lm_head_q8 (int8 per row) computes the 151936 logits of config 2', async () => {
    const { q, h, logits } = config2();
    const spec = eg.embeddingHeadSpec('q8', eg.ENCODING.SIGNED);
    const actual = await run(spec, [h, q.packed, q.scales, null], V, eg.embeddingDims(1, H, 0, V, H),
      [65535, 3, 1]);
    expectMatches(actual, logits, { abs: 1e-5 * rmsOf(logits), rel: 1e-3 }, 'lm_head_q8');
  });

  it('the fused head + argmax returns only the token id', async () => {
    const { q, h, logits } = config2();
    const { ctx, pool } = await gpu();
    const bufs = [h, q.packed, q.scales].map((a) => {
      const b = pool.acquire(a.byteLength, STORAGE, 'in');
      ctx.queue.writeBuffer(b.buffer, 0, a);
      return b;
    });
    const result = pool.acquire(8, STORAGE, 'result');
    eg.native.lmHeadArgmax(ctx.device.ctx, bufs[0].buffer.ptr, bufs[1].buffer.ptr, bufs[2].buffer.ptr, null, null,
      result.buffer.ptr, eg.embeddingDims(1, H, 0, V, H), eg.ENCODING.SIGNED, 8);
    const got = new Uint32Array(await eg.readBuffer(ctx, pool, result));
    let best = 0, second = -Infinity;
    for (let i = 1; i < V; i++) if (logits[i] > logits[best]) best = i;
    for (let i = 0; i < V; i++) if (i !== best) second = Math.max(second, logits[i]);
    expect(logits[best] - second > 1e-3 * Math.abs(logits[best]), 'top-2 gap clears the GEMV tolerance');
    expect(got[0] === best, `argmax ${got[0]} expected ${best}`);
    for (const b of bufs) pool.release(b);
    pool.release(result);
  });
});

describe('argmax (forward_ops.test.ts:397-446)', () => {
  it('finds the planted maximum of a vocabulary-sized row', async () => {
    const logits = ref.uniformMinusHalf(151936, 101);
    logits[123456] = 99;
    const out = await run(eg.ARGMAX, [logits], 2, eg.argmaxDims(151936, 0), eg.ARGMAX_WORKGROUPS, 'u32');
    expect(out[0] === 123456, `index ${out[0]}`);
    f32[0] = 99;
    expect(out[1] === u32[0], 'value bits');
  });

  it('breaks ties toward the lower index', async () => {
    const logits = new Float32Array(1000);
    logits[100] = 5;
    logits[900] = 5;
    const out = await run(eg.ARGMAX, [logits], 2, eg.argmaxDims(1000, 0), eg.ARGMAX_WORKGROUPS, 'u32');
    expect(out[0] === 100, `index ${out[0]}`);
  });
});

describe('sample', () => {
  async function sample(logits, history, params, random) {
    const { ctx, pool, cache } = await gpu();
    const kernel = new eg.ComputeKernel(ctx.device, cache, eg.SAMPLE);
    const lb = pool.acquire(logits.byteLength, STORAGE, 'logits');
    ctx.queue.writeBuffer(lb.buffer, 0, logits);
    const hb = pool.acquire(Math.max(4, history.byteLength), STORAGE, 'history');
    ctx.queue.writeBuffer(hb.buffer, 0, history.length ? history : new Uint32Array(1));
    const out = pool.acquire(4, STORAGE, 'token');
    const dims = kernel.uniform(pool);
    ctx.queue.writeBuffer(dims.buffer, 0, eg.sampleDims(logits.length, history.length, params, random));
    const encoder = ctx.device.createCommandEncoder();
    const pass = encoder.beginComputePass();
    kernel.encode(pass, kernel.bindGroup([lb, hb, out, dims]), eg.SAMPLE_WORKGROUPS);
    pass.end();
    ctx.queue.submit([encoder.finish()]);
    const token = new Uint32Array(await eg.readBuffer(ctx, pool, out))[0];
    const after = new Float32Array(await eg.readBuffer(ctx, pool, lb));
    for (const b of [lb, hb, out, dims]) pool.release(b);
    return { token, after };
  }

  it('greedy is the argmax', async () => {
    const logits = ref.uniformMinusHalf(151936, 7);
    logits[4242] = 3;
    const { token } = await sample(logits, new Uint32Array(0), eg.GREEDY, 0.5);
    expect(token === 4242, `token ${token}`);
  });

  it('penalises each history id once, in place, by the sign rule', async () => {
    const logits = new Float32Array(1000);
    logits[7] = 2.0;
    logits[9] = 1.9;
    logits[11] = -1.0;
    const { token, after } = await sample(logits, Uint32Array.from([7, 7, 11, 7]), { temperature: 0, topP: 1, repetitionPenalty: 1.1 }, 0.5);
    expect(token === 9, `token ${token}`);
    expect(after[7] === Math.fround(Math.fround(2.0) / Math.fround(1.1)), `logit 7 = ${after[7]}`);
    expect(after[11] === Math.fround(Math.fround(-1.0) * Math.fround(1.1)), `logit 11 = ${after[11]}`);
    expect(after[9] === Math.fround(1.9), 'ids outside the history are unchanged');
  });

  it('a near-zero temperature with topP 1 is greedy (session.test.ts:292-309)', async () => {
    const logits = ref.uniformMinusHalf(151936, 8);
    logits[777] = 1.5;
    const { token } = await sample(logits, new Uint32Array(0), { temperature: 0.01, topP: 1, repetitionPenalty: 1 }, 0.6);
    expect(token === 777, `token ${token}`);
  });

  it('the same draw gives the same token', async () => {
    const logits = ref.uniformMinusHalf(151936, 9);
    const params = { temperature: 0.7, topP: 0.9, repetitionPenalty: 1.1 };
    const history = Uint32Array.from({ length: 64 }, (_, i) => (i * 2371) % 151936);
    const a = await sample(logits, history, params, 0.3125);
    const b = await sample(logits, history, params, 0.3125);
    expect(a.token === b.token, `${a.token} vs ${b.token}`);
    expect(a.token < 151936, 'in range');
  });
});

describe('errors and capture', () => {
  it('a shape the kernel cannot run is an Error naming the op, at submit', async () => {
    const { ctx, pool, cache } = await gpu();
    const kernel = new eg.ComputeKernel(ctx.device, cache, eg.MATMUL_Q4_DECODE);
    const bufs = [0, 1, 2, 3, 4, 5].map(() => pool.acquire(256, STORAGE, 'b'));
    const dims = kernel.uniform(pool);
    ctx.queue.writeBuffer(dims.buffer, 0, eg.matmulQ4Dims(1, 4, 40, false, 64));  // k % blockSize != 0
    const encoder = ctx.device.createCommandEncoder();
    kernel.encode(encoder.beginComputePass(), kernel.bindGroup([...bufs, dims]), [4, 1, 1]);
    expectThrows(() => ctx.queue.submit([encoder.finish()]), (e) => {
      expect(e.code === 'EG_ERR_INVALID', `${e.code}: ${e.message}`);
      expect(/^matmul_q4_decode/.test(e.message), e.message);
    }, 'submit');
    for (const b of [...bufs, dims]) pool.release(b);
  });

  it('a captured submit replays to the same result', async () => {
    const { ctx, pool, cache } = await gpu();
    const n = 896, k = 896;
    const x = ref.uniformMinusHalf(k, 81);
    const q = ref.quantizeAsym4(ref.uniformMinusHalf(n * k, 82), n, k, 64);
    const kernel = new eg.ComputeKernel(ctx.device, cache, eg.MATMUL_Q4_DECODE);
    const ins = [x, q.packed, q.scales, q.zeros, new Float32Array(n)].map((a) => {
      const b = pool.acquire(a.byteLength, STORAGE, 'in');
      ctx.queue.writeBuffer(b.buffer, 0, a);
      return b;
    });
    const out = pool.acquire(n * 4, STORAGE, 'out');
    const dims = kernel.uniform(pool);
    ctx.queue.writeBuffer(dims.buffer, 0, eg.matmulQ4Dims(1, n, k, false, 64));
    const encoder = ctx.device.createCommandEncoder();
    pool.clear(encoder, out);
    kernel.encode(encoder.beginComputePass(), kernel.bindGroup([...ins, out, dims]), eg.matmulQ4DecodeWorkgroups(n));
    const commands = encoder.finish();
    ctx.device.beginCapture();
    ctx.queue.submit([commands]);
    const graph = ctx.device.endCapture();
    const expected = ref.gemm(x, q, null, 1);
    for (let replay = 0; replay < 3; replay++) {
      graph.launch();
      const got = new Float32Array(await eg.readBuffer(ctx, pool, out));
      expectMatches(got.subarray(0, n), expected, FP32_TOLERANCE, `replay ${replay}`);
    }
    graph.destroy();
    for (const b of [...ins, out, dims]) pool.release(b);
  });
});

runAll();
