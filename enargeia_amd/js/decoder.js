// The decode-step driver for Node: DecodeGraph + Session.decodeStep (graph_decode.ts:185-448,
// session.ts:347-375) over the addon's eg_decoder_* binding. The model description mirrors
// eg_model_desc with camelCase names; every tensor is a device pointer (a HipBuffer's `ptr`).
'use strict';

const native = require('./native.js');

class Decoder {
  /** device: a HipDevice; desc: {layers, hidden, heads, kvHeads, headDim, intermediate, vocab,
   * maxContext, rmsEps, ropeTheta, encoding, bits, blockSize, embedding: {packed, scales, zeros},
   * embedEncoding, embedBits, embedBlockSize, finalNorm, layer: [{q, k, v, o, gate, up, down,
   * qBias, kBias, vBias, inputNorm, postAttentionNorm}]} */
  constructor(device, desc) {
    this.device = device;
    this.vocab = desc.vocab;
    this.handle = native.decoderCreate(device.ctx, desc);
    this.buffers = native.decoderBuffers(this.handle);
  }

  /** The next step runs at `position` on `token` (cache rows [0, position) are the history). */
  reset(position, token) {
    native.decoderReset(this.handle, position, token);
  }

  /** One greedy step; returns the new token id (the one readback), or undefined if !readToken. */
  step(readToken = true) {
    return native.decoderStep(this.handle, readToken);
  }

  /** Captures one step as a hipGraph; later steps replay it. */
  capture() {
    native.decoderCapture(this.handle);
  }

  logits() {
    return new Float32Array(native.bufRead(this.device.ctx, this.buffers.logits, 0, this.vocab * 4));
  }

  destroy() {
    if (this.handle) native.decoderDestroy(this.handle);
    this.handle = null;
  }
}

module.exports = { Decoder };
