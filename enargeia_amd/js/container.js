// The `.enargeia` container for Node (src/model/enargeia.ts, WeightStore.loadQuantized in
// src/model/weights.ts:299-471) over the addon's C++ parser and one-allocation upload.
'use strict';

const native = require('./native.js');

const ENARGEIA_MAGIC = 'ENARGEIA';
const ENARGEIA_VERSION = 1;
const ENARGEIA_BLOCK = 64;

class EnargeiaError extends Error {
  constructor(message) {
    super(message);
    this.name = 'EnargeiaError';
  }
}

/** Runs fn, turning the addon's format errors into EnargeiaError (enargeia.ts:84-89). */
function wrap(fn) {
  try {
    return fn();
  } catch (err) {
    if (err && err.code === 'EG_ERR_FORMAT') throw new EnargeiaError(err.message);
    throw err;
  }
}

/** EnargeiaHeader (enargeia.ts:73-82) of the file at `path`; `tensors` is a Map by name. */
function readEnargeiaHeader(path) {
  const handle = wrap(() => native.containerOpen(path));
  try {
    const h = native.containerHeader(handle);
    return {
      version: h.version,
      blockSize: h.blockSize,
      quantization: h.quantization,
      tensors: new Map(h.tensors.map((t) => [t.name, t])),
      dataOffset: h.dataOffset,
      headerLength: h.headerLength,
      fileSize: h.fileSize,
    };
  } finally {
    native.containerClose(handle);
  }
}

/**
 * Loads a Qwen2 checkpoint for the decoder: the blob goes to the device in one allocation and
 * `desc` points into it (pass it to `new Decoder(device, desc)`). `config` gives what the file
 * does not: {headDim, maxContext, rmsEps, ropeTheta}. Call release() when the decoders are gone.
 */
function loadQuantized(device, path, config) {
  const handle = wrap(() => native.containerOpen(path));
  try {
    const pick = (v, d) => (v === undefined || v === null ? d : v);
    const c = config || {};
    const { blob, desc } = native.containerLoad(device.ctx, handle, {
      headDim: pick(c.headDim, 64),
      maxContext: pick(c.maxContext, 2048),
      rmsEps: pick(c.rmsEps, 1e-6),
      ropeTheta: pick(c.ropeTheta, 1e6),
    });
    let live = true;
    return {
      desc,
      blob,
      release() {
        if (live) native.bufFree(device.ctx, blob);
        live = false;
      },
    };
  } finally {
    native.containerClose(handle);
  }
}

module.exports = { ENARGEIA_MAGIC, ENARGEIA_VERSION, ENARGEIA_BLOCK, EnargeiaError, readEnargeiaHeader, loadQuantized };
