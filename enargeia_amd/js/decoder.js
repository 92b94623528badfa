// The decode-step driver for Node: DecodeGraph + Session.decodeStep (graph_decode.ts:185-448,
// session.ts:347-375) over the addon's eg_decoder_* binding. The model description mirrors
// eg_model_desc with camelCase names; every tensor is a device pointer (a HipBuffer's `ptr`).
'use strict';

const native = require('./native.js');
const { HipBuffer, BufferUsage } = require('./gpu.js');

class Decoder {
  /** device: a HipDevice; desc: {layers, hidden, heads, kvHeads, headDim, intermediate, vocab,
   * maxContext, rmsEps, ropeTheta, encoding, bits, blockSize, embedding: {packed, scales, zeros},
   * embedEncoding, embedBits, embedBlockSize, finalNorm, layer: [{q, k, v, o, gate, up, down,
   * qBias, kBias, vBias, inputNorm, postAttentionNorm}], cacheDType?: 'f16' | 'f32'} (the KV
   * cache's element type, SessionOptions.cacheDType; 'f16' when absent) */
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

/** A buffer the decoder owns, seen through the facade's buffer type so queue.writeBuffer,
 * readBuffer and bindings reach it; destroy() leaves it to the decoder. */
function borrowed(device, ptr, size, label) {
  const buffer = Object.create(HipBuffer.prototype);
  Object.assign(buffer, {
    device, size, usage: BufferUsage.STORAGE | BufferUsage.COPY_SRC | BufferUsage.COPY_DST, label, uniform: false,
    host: null, ptr,
  });
  buffer.destroy = () => {};
  // the shape of a BufferPool entry (pool.ts:83-120), which the reference's graph fields are
  return { buffer, size, capacity: size, binding: { buffer, offset: 0, size } };
}

/**
 * DecodeGraph (src/model/graph_decode.ts:85-460) over eg_decoder, for a host that drives it the
 * way the reference's Session.decodeStep does (session.ts:347-375): write the token into
 * `tokenId` and the history into `history`, `setPosition(position, historyLength, random)`,
 * `encode` into a command encoder, submit, read `result`. The buffers are the decoder's own
 * device buffers. encode records one whole decode step (every layer, the LM head and the sample
 * step: one launch sequence, or one graph replay after capture()).
 */
class DecodeGraph {
  constructor(device, desc) {
    this.device = device;
    this.config = { layers: desc.layers, vocab: desc.vocab, maxContext: desc.maxContext };
    this.handle = native.decoderCreate(device.ctx, desc);
    const b = native.decoderBuffers(this.handle);
    this.tokenId = borrowed(device, b.token, 4, 'decode/token_id');
    this.result = borrowed(device, b.token, 4, 'decode/result');
    // The result is read with the decoder's status word (token[2]: steps that gave up, which moved
    // nothing), in the same copy; a failure is an Error, as the reference's
    // kernel layer fails loudly (kernel.ts:97-107), and the word is cleared.
    this.result.buffer.read = (size) => {
      const bytes = native.bufRead(device.ctx, b.token, 0, 12);
      const words = new Uint32Array(bytes);
      if (words[2] !== 0) {
        native.bufWrite(device.ctx, b.token, 8, new Uint32Array([0]));
        throw new Error(`decode: ${words[2]} step(s) gave up: a bounded wait timed out (not every workgroup was ` +
                        'resident at once); the position, history and draw state are as before');
      }
      return bytes.slice(0, size);
    };
    this.history = borrowed(device, b.history, desc.maxContext * 4, 'decode/history');
    this.logits = borrowed(device, b.logits, desc.vocab * 4, 'decode/logits');
    this.params = { temperature: 0, topP: 1, repetitionPenalty: 1 };
  }

  /** graph_decode.ts:387 */
  setSampling(params) {
    native.decoderSetSampling(this.handle, params);
    this.params = params;
  }

  /** graph_decode.ts:398-406: the per-token values of the next step (the one host write). */
  setPosition(position, historyLength, random) {
    native.decoderSetPosition(this.handle, position, historyLength, random);
  }

  /** graph_decode.ts:442-448: one decode step, run at submit. */
  encode(encoder, position) {
    const handle = this.handle;
    encoder.record(() => native.decoderStep(handle, false));
  }

  /** Captures the step as a hipGraph; later encodes replay it. */
  capture() {
    native.decoderCapture(this.handle);
  }

  /** The prompt and its first token (ForwardGraph + sampleFromPrefill in one call); the draw is
   * the decoder's own mulberry32 stream, restarted by seed(). */
  prefill(position, prompt) {
    return native.decoderPrefill(this.handle, position, new Uint32Array(prompt));
  }

  seed(seed) {
    native.decoderSeed(this.handle, seed);
  }

  /** launches per step (eg_decoder_launches): the layers (one persistent launch, or 5 per layer),
   * the LM head and the tail, the sampler's one launch when the parameters are not GREEDY, and the
   * input preparation a host-driven step (setPosition) runs first */
  get dispatchCount() {
    return native.decoderLaunches(this.handle);
  }

  destroy() {
    if (this.handle) native.decoderDestroy(this.handle);
    this.handle = null;
  }
}

module.exports = { Decoder, DecodeGraph };
