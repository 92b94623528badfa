// KernelSpec / ComputeKernel (src/kernels/kernel.ts:20-124) for the ops of this path.
//
// Same constructor, bindGroup, uniform and encode as the reference, with its two synchronous
// errors: a wrong binding count is an Error "<name>: expected N bindings, got M"
// (kernel.ts:70-81) and a grid axis over the per-dimension limit is a RangeError
// (kernel.ts:97-107). encode does not hand a WGSL pipeline to a pass: it records a call of the
// C entry point named by spec.name into the pass's encoder, which runs at queue.submit. The
// launch geometry is the library's own; the grid passed to encode is only checked.
'use strict';

const native = require('./native.js');
const { toBinding } = require('./gpu.js');

const ENCODING = Object.freeze({ OFFSET_ZEROS: 0, SIGNED: 1 });

function pointerOf(ref) {
  const b = toBinding(ref);
  if (b === null) return 0;
  if (b.buffer.uniform) throw new TypeError(`${b.buffer.label}: a uniform buffer bound as storage`);
  return b.buffer.ptr + (b.offset || 0);
}

function uniformBytes(ref, spec) {
  const b = toBinding(ref);
  if (b === null || !b.buffer.uniform) throw new TypeError(`${spec.name}: the last binding must be a uniform buffer`);
  return b.buffer.host.subarray(b.offset || 0, (b.offset || 0) + spec.uniformBytes);
}

// spec.name -> (ctx, pointers, uniform, spec) => void, over the C entry points.
const DISPATCH = {
  matmul_q4_decode: (ctx, p, u, s) => native.matmulQ4Decode(ctx, p[0], p[1], p[2], p[3], p[4], p[5], u, s.encoding, s.bits),
  matmul_q4_prefill: (ctx, p, u, s) => native.matmulQ4Prefill(ctx, p[0], p[1], p[2], p[3], p[4], p[5], u, s.encoding, s.bits),
  lm_head_q4: (ctx, p, u, s) => native.lmHead(ctx, p[0], p[1], p[2], p[3], p[4], u, s.encoding, s.bits),
  lm_head_q8: (ctx, p, u, s) => native.lmHead(ctx, p[0], p[1], p[2], p[3], p[4], u, s.encoding, s.bits),
  lm_head_f16: (ctx, p, u, s) => native.lmHead(ctx, p[0], p[1], p[2], p[3], p[4], u, s.encoding, s.bits),
  lm_head_f32: (ctx, p, u, s) => native.lmHead(ctx, p[0], p[1], p[2], p[3], p[4], u, s.encoding, s.bits),
  embed_gather_q4: (ctx, p, u, s) => native.embedGather(ctx, p[0], p[1], p[2], p[3], p[4], u, s.encoding, s.bits),
  embed_gather_q8: (ctx, p, u, s) => native.embedGather(ctx, p[0], p[1], p[2], p[3], p[4], u, s.encoding, s.bits),
  embed_gather_f16: (ctx, p, u, s) => native.embedGather(ctx, p[0], p[1], p[2], p[3], p[4], u, s.encoding, s.bits),
  embed_gather_f32: (ctx, p, u, s) => native.embedGather(ctx, p[0], p[1], p[2], p[3], p[4], u, s.encoding, s.bits),
  argmax: (ctx, p, u) => native.argmax(ctx, p[0], p[1], u),
  sample: (ctx, p, u) => native.sample(ctx, p[0], p[1], p[2], u),
};

class ComputeKernel {
  /** kernel.ts:42. `cache` is accepted for the reference's signature; nothing is cached. */
  constructor(device, cache, spec) {
    if (!DISPATCH[spec.name]) throw new Error(`${spec.name}: not an op of this library`);
    this.device = device;
    this.spec = Object.assign({ bits: 4, encoding: ENCODING.OFFSET_ZEROS }, spec);
  }

  /** kernel.ts:70-81. A null resource binds no buffer (the zeros of a symmetric format). */
  bindGroup(resources) {
    if (resources.length !== this.spec.bindings.length) {
      throw new Error(`${this.spec.name}: expected ${this.spec.bindings.length} bindings, got ${resources.length}`);
    }
    return { kernel: this, resources: resources.slice() };
  }

  /** kernel.ts:84-90 */
  uniform(pool) {
    return pool.acquire(this.spec.uniformBytes, 0x0040 | 0x0008, `${this.spec.name}.dims`);
  }

  /** kernel.ts:92-111 */
  encode(pass, bindGroup, workgroups) {
    const limit = this.device.limits.maxComputeWorkgroupsPerDimension;
    workgroups.forEach((count, axis) => {
      if (count > limit) {
        throw new RangeError(`${this.spec.name}: ${count} workgroups on axis ${axis} exceeds the device limit of ${limit}`);
      }
    });
    const spec = this.spec;
    const res = bindGroup.resources;
    const pointers = res.slice(0, -1).map(pointerOf);
    const uniformRef = res[res.length - 1];
    uniformBytes(uniformRef, spec);  // checked now, read at submit
    const device = this.device;
    pass.encoder.record(() => DISPATCH[spec.name](device.ctx, pointers, uniformBytes(uniformRef, spec).slice(), spec));
  }
}

/** coverage (kernel.ts:115-124) */
function coverage(spec, counts) {
  return [0, 1, 2].map((i) => Math.max(1, Math.ceil(counts[i] / spec.workgroupSize[i])));
}

module.exports = { ComputeKernel, coverage, ENCODING };
