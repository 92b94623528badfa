// The gpu layer the reference's kernels are driven through (src/gpu/device.ts, pool.ts,
// readback.ts), over HIP through the N-API addon instead of WebGPU.
//
// What keeps the reference's semantics:
//   - queue.writeBuffer is ordered before every command buffer submitted after it and after
//     every one submitted before it (it runs on the context's stream at call time);
//   - command encoders record; nothing runs until queue.submit, which enqueues the recorded
//     dispatches in order. A uniform buffer's bytes are therefore read at submit, as WebGPU
//     reads them at execution;
//   - readBuffer resolves after all previously submitted work, with one synchronous copy.
// What differs: there is no WGSL and no pipeline object; buffers are HIP allocations whose
// device address is `buffer.ptr`. Uniform buffers are host images (their bytes become the
// kernel's by-value argument), so they never occupy device memory.
'use strict';

const native = require('./native.js');

const BufferUsage = Object.freeze({
  MAP_READ: 0x0001,
  MAP_WRITE: 0x0002,
  COPY_SRC: 0x0004,
  COPY_DST: 0x0008,
  INDEX: 0x0010,
  VERTEX: 0x0020,
  UNIFORM: 0x0040,
  STORAGE: 0x0080,
  INDIRECT: 0x0100,
  QUERY_RESOLVE: 0x0200,
});

const MAX_WORKGROUPS_PER_DIMENSION = 65535;

/** device.ts:88 */
class GPUUnavailableError extends Error {
  constructor(message, cause) {
    super(message);
    this.name = 'GPUUnavailableError';
    this.cause = cause;
  }
}

function viewBytes(data, dataOffset, size) {
  let bytes;
  if (data instanceof ArrayBuffer) bytes = new Uint8Array(data);
  else if (ArrayBuffer.isView(data)) bytes = new Uint8Array(data.buffer, data.byteOffset, data.byteLength);
  else throw new TypeError('writeBuffer: data must be an ArrayBuffer or a view of one');
  // GPUQueue.writeBuffer: dataOffset and size count elements for typed arrays, bytes otherwise.
  const elem = ArrayBuffer.isView(data) && data.BYTES_PER_ELEMENT ? data.BYTES_PER_ELEMENT : 1;
  const begin = (dataOffset || 0) * elem;
  const end = size === undefined ? bytes.byteLength : begin + size * elem;
  if (begin > bytes.byteLength || end > bytes.byteLength) throw new RangeError('writeBuffer: data range out of bounds');
  return bytes.subarray(begin, end);
}

class HipBuffer {
  constructor(device, size, usage, label) {
    this.device = device;
    this.size = size;
    this.usage = usage;
    this.label = label || '';
    this.uniform = (usage & BufferUsage.UNIFORM) !== 0;
    if (this.uniform) {
      this.host = new Uint8Array(size);
      this.ptr = 0;
    } else {
      this.host = null;
      this.ptr = native.bufAlloc(device.ctx, size);
    }
  }

  destroy() {
    if (this.ptr) {
      native.bufFree(this.device.ctx, this.ptr);
      this.ptr = 0;
    }
    this.host = null;
  }
}

class CommandBuffer {
  constructor(commands) {
    this.commands = commands;
  }
}

class ComputePass {
  constructor(encoder) {
    this.encoder = encoder;
  }

  end() {}
}

class CommandEncoder {
  constructor(device, label) {
    this.device = device;
    this.label = label || '';
    this.commands = [];
  }

  beginComputePass() {
    return new ComputePass(this);
  }

  record(command) {
    this.commands.push(command);
  }

  clearBuffer(buffer, offset, size) {
    const off = offset || 0;
    const bytes = size === undefined ? buffer.size - off : size;
    this.record(() => native.bufZero(this.device.ctx, buffer.ptr, off, bytes));
  }

  finish() {
    return new CommandBuffer(this.commands.slice());
  }
}

class Queue {
  constructor(device) {
    this.device = device;
  }

  writeBuffer(buffer, offset, data, dataOffset, size) {
    const bytes = viewBytes(data, dataOffset, size);
    if (offset + bytes.byteLength > buffer.size) throw new RangeError(`writeBuffer: ${buffer.label} overflows`);
    if (buffer.uniform) buffer.host.set(bytes, offset);
    else native.bufWrite(this.device.ctx, buffer.ptr, offset, bytes);
  }

  submit(commandBuffers) {
    for (const cb of commandBuffers) for (const command of cb.commands) command();
  }

  onSubmittedWorkDone() {
    native.sync(this.device.ctx);
    return Promise.resolve();
  }
}

/** A captured sequence of submits (one hipGraph), replayed with launch(). */
class HipGraph {
  constructor(device, handle) {
    this.device = device;
    this.handle = handle;
  }

  launch() {
    native.graphLaunch(this.device.ctx, this.handle);
  }

  destroy() {
    if (this.handle) native.graphDestroy(this.handle);
    this.handle = null;
  }
}

class HipDevice {
  constructor(index) {
    this.ctx = native.create(index);
    this.index = index;
    this.limits = Object.freeze({ maxComputeWorkgroupsPerDimension: MAX_WORKGROUPS_PER_DIMENSION });
    this.queue = new Queue(this);
    this.lost = new Promise(() => {});
  }

  createBuffer(descriptor) {
    return new HipBuffer(this, Math.max(4, descriptor.size), descriptor.usage, descriptor.label);
  }

  createCommandEncoder(descriptor) {
    return new CommandEncoder(this, descriptor && descriptor.label);
  }

  /** Submits between beginCapture and endCapture are recorded into one graph. */
  beginCapture() {
    native.graphBegin(this.ctx);
  }

  endCapture() {
    return new HipGraph(this, native.graphEnd(this.ctx));
  }

  destroy() {
    if (this.ctx) native.destroy(this.ctx);
    this.ctx = null;
  }
}

/** initGPU (device.ts:116): the context of HIP device `deviceIndex`. */
async function initGPU(options) {
  const index = (options && options.deviceIndex) || 0;
  let device;
  try {
    device = new HipDevice(index);
  } catch (err) {
    throw new GPUUnavailableError(`no HIP device ${index}: ${err.message}`, err);
  }
  return {
    adapter: null,
    device,
    queue: device.queue,
    profile: { tier: 'discrete', vendor: 'amd', architecture: 'gfx950' },
  };
}

/** The pipeline cache has nothing to cache here: there are no pipelines. */
class PipelineCache {
  constructor(device) {
    this.device = device;
  }
}

function align4(n) {
  return Math.ceil(n / 4) * 4;
}

function classOf(bytes) {
  return Math.max(2, Math.ceil(Math.log2(bytes)));
}

/** BufferPool (pool.ts:55): power-of-two size classes per usage, idle buffers reused. */
class BufferPool {
  constructor(device, options) {
    this.device = device;
    this.label = (options && options.label) || 'pool';
    this.idle = new Map();
    this.live = new Set();
  }

  acquire(size, usage, label) {
    if (!Number.isFinite(size) || size <= 0) throw new RangeError(`[${this.label}] acquire(${size}): size must be positive`);
    const bound = align4(size);
    const cls = classOf(bound);
    const capacity = 2 ** cls;
    const key = `${usage}:${cls}`;
    const free = this.idle.get(key);
    const buffer = (free && free.pop()) ||
      this.device.createBuffer({ size: capacity, usage, label: `${this.label}/${label || 'scratch'}:${capacity}` });
    const entry = { buffer, size: bound, capacity, usage, binding: { buffer, offset: 0, size: bound }, key };
    this.live.add(entry);
    return entry;
  }

  release(entry) {
    if (!this.live.delete(entry)) return;
    if (!this.idle.has(entry.key)) this.idle.set(entry.key, []);
    this.idle.get(entry.key).push(entry.buffer);
  }

  clear(encoder, entry) {
    encoder.clearBuffer(entry.buffer, 0, entry.size);
  }

  destroy() {
    for (const entry of this.live) entry.buffer.destroy();
    for (const list of this.idle.values()) for (const buffer of list) buffer.destroy();
    this.live.clear();
    this.idle.clear();
  }
}

/** readBuffer (readback.ts:18): all `source.size` bytes, after all submitted work. A buffer with
 * its own `read(size)` (a decoder's result word, read with its status) is read through it. */
async function readBuffer(ctx, pool, source) {
  const buffer = source.buffer || source;
  if (buffer.read) return buffer.read(source.size);
  return native.bufRead(ctx.device.ctx, buffer.ptr, 0, source.size);
}

/** readFloats (readback.ts:40) */
async function readFloats(ctx, pool, source) {
  return new Float32Array(await readBuffer(ctx, pool, source));
}

/** toBinding (pool.ts:236): {buffer, offset, size} of any buffer reference. */
function toBinding(ref) {
  if (ref === null || ref === undefined) return null;
  if (ref.binding) return ref.binding;
  if (ref.buffer && ref.buffer instanceof HipBuffer) return { buffer: ref.buffer, offset: ref.offset || 0, size: ref.size };
  if (ref instanceof HipBuffer) return { buffer: ref, offset: 0, size: ref.size };
  throw new TypeError('not a buffer binding');
}

module.exports = {
  BufferUsage,
  MAX_WORKGROUPS_PER_DIMENSION,
  GPUUnavailableError,
  HipBuffer,
  HipDevice,
  HipGraph,
  CommandEncoder,
  ComputePass,
  PipelineCache,
  BufferPool,
  initGPU,
  readBuffer,
  readFloats,
  toBinding,
};
