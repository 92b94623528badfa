// CPU baseline in the reference's own language: the reference CPU path's GEMV loop
// (test/reference/quant.ts:95-111, linearQ4: every weight dequantized on the fly by
// dequantElement, quant.ts:77-84, and accumulated in a float64 `sum` started from the bias),
// restated in plain JavaScript (Node 12, no TypeScript), timed on one core over one layer of
// BASELINE config 1 (q, k, v, o, gate, up 896 -> ..., down 4864 -> 896) in BASELINE's format:
// symmetric int4, one f32 scale per 32 weights, two's-complement nibbles (element 2j in the low
// nibble of byte j), so the dequantized weight is (nibble ^ 8) - 8 times the block's scale.
// Test and measurement infrastructure: bench.py's cpu_baseline leg runs it as a child process.
//
//   node oracle/linear_q4_time.js [reps]   -> one JSON line {bytes, seconds, gbs, node}
'use strict';

// mulberry32 (the reference's rng.ts:2-10, a published generator) for the synthetic inputs.
function makeRng(seed) {
  let state = seed >>> 0;
  return function next() {
    state = (state + 0x6d2b79f5) >>> 0;
    let z = Math.imul(state ^ (state >>> 15), state | 1);
    z ^= z + Math.imul(z ^ (z >>> 7), z | 61);
    return ((z ^ (z >>> 14)) >>> 0) / 4294967296;
  };
}

// A random matrix already in the packed format (random codes and positive scales): the loop
// below reads it exactly as it reads a quantized checkpoint.
function randomMatrix(rows, cols, seed) {
  const next = makeRng(seed);
  const packed = new Uint32Array((rows * cols) / 8);
  for (let i = 0; i < packed.length; i++) packed[i] = (next() * 4294967296) >>> 0;
  const scales = new Float32Array((rows * cols) / 32);
  for (let i = 0; i < scales.length; i++) scales[i] = 0.002 + 0.001 * next();
  return { rows, cols, blockSize: 32, packed, scales };
}

// dequantElement (quant.ts:77-84) for the symmetric format.
function dequantElement(q, row, col) {
  const e = row * q.cols + col;
  const code = ((q.packed[e >>> 3] >>> ((e & 7) * 4)) & 15) ^ 8;
  const blk = row * (q.cols / q.blockSize) + Math.floor(col / q.blockSize);
  return (code - 8) * q.scales[blk];
}

// linearQ4 (quant.ts:95-111) at m = 1.
function linearQ4(x, q, bias) {
  const out = new Float32Array(q.rows);
  for (let c = 0; c < q.rows; c++) {
    let sum = bias ? bias[c] : 0;
    for (let i = 0; i < q.cols; i++) sum += x[i] * dequantElement(q, c, i);
    out[c] = sum;
  }
  return out;
}

function main() {
  const reps = Number(process.argv[2] || 2);
  const H = 896, I = 4864, KV = 128;
  const shapes = [[H, H], [KV, H], [KV, H], [H, H], [I, H], [I, H], [H, I]];
  const mats = shapes.map(([n, k], i) => randomMatrix(n, k, 0x5eed ^ i));
  const next = makeRng(3);
  const xh = new Float32Array(H).map(() => next() - 0.5);
  const xi = new Float32Array(I).map(() => next() - 0.5);
  // algorithmic bytes of the layer: codes + f32 scales + x read + y written (bench.py's gemv_bytes)
  let bytes = 0;
  for (const q of mats) bytes += (q.rows * q.cols) / 2 + (q.rows * q.cols / 32) * 4 + q.cols * 4 + q.rows * 4;
  let checksum = 0;
  linearQ4(xh, mats[1], null);  // warm the JIT
  const t0 = process.hrtime.bigint();
  for (let r = 0; r < reps; r++)
    for (const q of mats) checksum += linearQ4(q.cols === H ? xh : xi, q, null)[0];
  const seconds = Number(process.hrtime.bigint() - t0) / 1e9 / reps;
  process.stdout.write(JSON.stringify({ bytes, seconds, gbs: bytes / seconds / 1e9, node: process.version,
                                        checksum }) + '\n');
}

if (require.main === module) main();
module.exports = { linearQ4, dequantElement, randomMatrix };
