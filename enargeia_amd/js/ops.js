// Specs and uniform builders of the ops on this path, with the reference's names, binding
// orders and uniform byte layouts: matmul_q4.ts:17-90, embedding_variants.ts:182-236,
// argmax.ts:8-20, sample.ts:16-52. `bits` / `encoding` name the code width and the zero-point
// convention (the reference's formats are bits 4 / 8 with packed zero-points; the symmetric
// formats bind null for zeros).
'use strict';

const { ENCODING } = require('./kernel.js');

const MAX_WORKGROUPS_PER_DIMENSION = 65535;
const Q4_BINDINGS = Object.freeze(['read', 'read', 'read', 'read', 'read', 'read_write', 'uniform']);
const EMBED_BINDINGS = Object.freeze(['read', 'read', 'read', 'read', 'read_write', 'uniform']);

const MATMUL_Q4_PREFILL = Object.freeze({
  name: 'matmul_q4_prefill', bindings: Q4_BINDINGS, workgroupSize: [16, 16, 1], uniformBytes: 48,
  bits: 4, encoding: ENCODING.OFFSET_ZEROS,
});

const MATMUL_Q4_DECODE = Object.freeze({
  name: 'matmul_q4_decode', bindings: Q4_BINDINGS, workgroupSize: [64, 1, 1], uniformBytes: 48,
  bits: 4, encoding: ENCODING.OFFSET_ZEROS,
});

const ARGMAX = Object.freeze({
  name: 'argmax', bindings: Object.freeze(['read', 'read_write', 'uniform']), workgroupSize: [256, 1, 1], uniformBytes: 16,
});

const SAMPLE = Object.freeze({
  name: 'sample', bindings: Object.freeze(['read_write', 'read', 'read_write', 'uniform']), workgroupSize: [256, 1, 1],
  uniformBytes: 32,
});

const ARGMAX_WORKGROUPS = [1, 1, 1];
const SAMPLE_WORKGROUPS = [1, 1, 1];
const GREEDY = Object.freeze({ temperature: 0, topP: 1, repetitionPenalty: 1 });

/** The same op over another code width / zero-point convention. */
function withFormat(spec, bits, encoding) {
  return Object.freeze(Object.assign({}, spec, { bits, encoding }));
}

/** embeddingGatherSpec (embedding_variants.ts:186-193): the rows of `seq` ids (binding 0 holds them). */
function embeddingGatherSpec(dtype, encoding) {
  return Object.freeze(Object.assign({}, embeddingHeadSpec(dtype, encoding), { name: `embed_gather_${dtype}` }));
}

/** embeddingHeadSpec (embedding_variants.ts:195-203): q4 and q8 codes, or an f16 / f32 table. */
function embeddingHeadSpec(dtype, encoding) {
  const bits = { q4: 4, q8: 8, f16: 16, f32: 32 }[dtype];
  if (!bits) throw new Error(`lm_head_${dtype}: the dtypes are q4, q8, f16 and f32`);
  return Object.freeze({
    name: `lm_head_${dtype}`, bindings: EMBED_BINDINGS, workgroupSize: [64, 1, 1], uniformBytes: 48,
    bits, encoding: encoding === undefined ? ENCODING.OFFSET_ZEROS : encoding,
  });
}

function decodeGridWidth(n) {
  return Math.min(n, MAX_WORKGROUPS_PER_DIMENSION);
}

/** matmulQ4Dims (matmul_q4.ts:50-64) */
function matmulQ4Dims(m, n, k, useBias, blockSize, outStride, outOffset) {
  const stride = outStride === undefined ? n : outStride;
  return new Uint32Array([m, n, k, useBias ? 1 : 0, blockSize, k / blockSize, stride, outOffset || 0,
    decodeGridWidth(n), 0, 0, 0]).buffer;
}

function matmulQ4PrefillWorkgroups(m, n) {
  return [Math.max(1, Math.ceil(n / 32)), Math.max(1, Math.ceil(m / 64)), 1];
}

function matmulQ4DecodeWorkgroups(n) {
  const width = decodeGridWidth(n);
  return [width, Math.ceil(n / width), 1];
}

/** embeddingDims (embedding_variants.ts:207-221) */
function embeddingDims(seq, hidden, rowBegin, rowCount, blockSize, outStride, outOffset) {
  return new Uint32Array([seq, hidden, rowBegin, rowCount, blockSize, hidden / blockSize, outStride || 0,
    outOffset || 0, Math.min(Math.max(rowCount, 1), MAX_WORKGROUPS_PER_DIMENSION), 0, 0, 0]).buffer;
}

function embeddingHeadWorkgroups(rows) {
  const width = Math.min(rows, MAX_WORKGROUPS_PER_DIMENSION);
  return [width, Math.ceil(rows / width), 1];
}

/** argmaxDims (argmax.ts:16-18) */
function argmaxDims(count, offset) {
  return new Uint32Array([count, offset, 0, 0]).buffer;
}

/** sampleDims (sample.ts:35-50) */
function sampleDims(vocab, historyLength, params, random) {
  const buffer = new ArrayBuffer(32);
  new Uint32Array(buffer, 0, 2).set([vocab, historyLength]);
  new Float32Array(buffer, 8, 4).set([params.temperature, params.topP, params.repetitionPenalty, random]);
  return buffer;
}

module.exports = {
  MAX_WORKGROUPS_PER_DIMENSION,
  MATMUL_Q4_PREFILL,
  MATMUL_Q4_DECODE,
  ARGMAX,
  SAMPLE,
  ARGMAX_WORKGROUPS,
  SAMPLE_WORKGROUPS,
  GREEDY,
  withFormat,
  embeddingHeadSpec,
  embeddingGatherSpec,
  decodeGridWidth,
  matmulQ4Dims,
  matmulQ4PrefillWorkgroups,
  matmulQ4DecodeWorkgroups,
  embeddingDims,
  embeddingHeadWorkgroups,
  argmaxDims,
  sampleDims,
};
