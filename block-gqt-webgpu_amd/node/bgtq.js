'use strict';
// The reference's TypeScript runtime classes over the N-API addon.
//
// Same names, constructor and method arguments, validation order and error
// messages as src/webgpu/layout.ts, src/runtime/*.ts and src/attention/*.ts;
// every computation runs in the HIP kernels of libbgtq.so. Plain CommonJS so
// that any Node with N-API 6 loads it. Where the reference hands back a
// GPUBuffer (attend(), inspect(), PackedKeys.packed/norms) this module hands
// back a DeviceView whose read() copies the device data to a typed array;
// readBuffer(device, view) is that read, as in src/webgpu/buffers.ts.
const path = require('path');
const native = require(path.join(__dirname, 'bgtq_napi.node'));

const DTYPE_F32 = 0;
const DTYPE_F16 = 1;

// ---- GPUDevice facade ----------------------------------------------------
// createCommandEncoder / queue.submit / queue.onSubmittedWorkDone /
// createQuerySet / createBuffer keep the shapes of the WebGPU objects the
// reference's runtime classes, tests and benchmarks use
// (src/attention/attention.ts:44-58, benchmarks/timing.ts:7-31). Work a class
// records into an encoder runs on the device when the command buffer is
// submitted, in recording order; onSubmittedWorkDone resolves off the JS
// thread once the device has finished it.
const GPUBufferUsage = Object.freeze({ MAP_READ: 0x1, MAP_WRITE: 0x2, COPY_SRC: 0x4, COPY_DST: 0x8, INDEX: 0x10,
  VERTEX: 0x20, UNIFORM: 0x40, STORAGE: 0x80, INDIRECT: 0x100, QUERY_RESOLVE: 0x200 });
const GPUMapMode = Object.freeze({ READ: 0x1, WRITE: 0x2 });

class Queue {
  constructor(device) { this.device = device; }
  submit(commandBuffers) {
    for (const b of commandBuffers) {
      if (!(b instanceof CommandBuffer) || !b._ops) throw new Error('Invalid or already submitted command buffer');
      const ops = b._ops;
      b._ops = null;
      for (const op of ops) op();
    }
  }
  onSubmittedWorkDone() { return native.contextSynchronizeAsync(this.device.handle); }
  writeBuffer(buffer, offset, data, dataOffset, size) {
    const bytes = new Uint8Array(data.buffer || data, (data.byteOffset || 0) + (dataOffset || 0),
      size === undefined ? (data.byteLength - (dataOffset || 0)) : size);
    if (buffer instanceof HostBuffer) { buffer._write(offset, bytes); return; }
    if (offset % 4 || bytes.byteLength % 4 || offset + bytes.byteLength > buffer.size) {
      throw new RangeError('Unaligned/out-of-range buffer upload');
    }
    native.bufferWrite(buffer.handle, offset, bytes);
  }
}

// GPUQuerySet of type "timestamp" (HIP events on the context's stream).
class QuerySet {
  constructor(device, descriptor) {
    if (!descriptor || descriptor.type !== 'timestamp') throw new TypeError('Only timestamp query sets are supported');
    if (!Number.isInteger(descriptor.count) || descriptor.count < 1 || descriptor.count > 4096) {
      throw new RangeError('Invalid query set count');
    }
    this.device = device; this.type = 'timestamp'; this.count = descriptor.count;
    this.handle = native.timestampsCreate(device.handle, this.count);
  }
  destroy() { if (this.handle) native.timestampsDestroy(this.handle); this.handle = null; }
}

class CommandBuffer { constructor(ops) { this._ops = ops; } }

// A compute pass: its timestampWrites and the library work queued in it
// (_enqueue). WGSL pipelines do not exist on this device, so the raw
// setPipeline / dispatchWorkgroups calls are refused.
class ComputePass {
  constructor(encoder, descriptor) {
    this._encoder = encoder; this._ended = false;
    const tw = descriptor.timestampWrites;
    this._endWrite = tw && tw.endOfPassWriteIndex !== undefined ? [tw.querySet, tw.endOfPassWriteIndex] : null;
    if (tw && tw.beginningOfPassWriteIndex !== undefined) encoder._timestamp(tw.querySet, tw.beginningOfPassWriteIndex);
  }
  _enqueue(fn) {
    if (this._ended) throw new Error('Compute pass already ended');
    this._encoder._ops.push(fn);
  }
  setPipeline() { throw new Error('WGSL pipelines do not run on this device; record through the library classes'); }
  setBindGroup() { throw new Error('WGSL pipelines do not run on this device; record through the library classes'); }
  dispatchWorkgroups() { throw new Error('WGSL pipelines do not run on this device; record through the library classes'); }
  end() {
    if (this._ended) throw new Error('Compute pass already ended');
    this._ended = true;
    if (this._endWrite) this._encoder._timestamp(this._endWrite[0], this._endWrite[1]);
  }
}

class CommandEncoder {
  constructor(device) { this.device = device; this._ops = []; }
  _live() { if (!this._ops) throw new Error('Command encoder already finished'); }
  _timestamp(querySet, index) {
    this._live();
    if (!(querySet instanceof QuerySet) || !Number.isInteger(index) || index < 0 || index >= querySet.count) {
      throw new RangeError('Invalid timestamp write');
    }
    this._ops.push(() => native.timestampsWrite(querySet.handle, index));
  }
  beginComputePass(descriptor) { this._live(); return new ComputePass(this, descriptor || {}); }
  resolveQuerySet(querySet, firstQuery, queryCount, destination, destinationOffset) {
    this._live();
    const off = destinationOffset || 0;
    if (!(querySet instanceof QuerySet) || firstQuery + queryCount > querySet.count || !(destination instanceof HostBuffer) ||
        off % 8 || off + 8 * queryCount > destination.size) {
      throw new RangeError('Invalid query set resolve');
    }
    this._ops.push(() => destination._defer(() => destination._write(off,
      native.timestampsResolve(querySet.handle, firstQuery, queryCount))));
  }
  copyBufferToBuffer(source, sourceOffset, destination, destinationOffset, size) {
    this._live();
    if (sourceOffset % 4 || destinationOffset % 4 || size % 4 || destinationOffset + size > destination.size ||
        (source.size !== undefined && sourceOffset + size > source.size)) {
      throw new RangeError('Invalid buffer copy');
    }
    const bytes = () => sourceBytes(source, sourceOffset, size);
    if (destination instanceof HostBuffer) {
      this._ops.push(() => destination._defer(() => destination._write(destinationOffset, bytes())));
    } else {
      this._ops.push(() => native.bufferWrite(destination.handle, destinationOffset, bytes()));
    }
  }
  finish() { this._live(); const b = new CommandBuffer(this._ops); this._ops = null; return b; }
}

// A buffer the host maps (MAP_READ / MAP_WRITE) or that receives resolved
// queries: host memory whose copies and resolves, recorded in order, are
// carried out once the device has finished the work queued before them.
class HostBuffer {
  constructor(device, size, usage) {
    this.device = device; this.size = size; this.usage = usage;
    this._data = new ArrayBuffer(size); this._pending = []; this._mapped = false;
  }
  _defer(fn) { this._pending.push(fn); }
  _flush() { const p = this._pending; this._pending = []; for (const fn of p) fn(); }
  _write(offset, view) {
    const src = new Uint8Array(view.buffer, view.byteOffset, view.byteLength);
    new Uint8Array(this._data, offset, src.byteLength).set(src);
  }
  _bytes(offset, size) { this._flush(); return new Uint8Array(this._data.slice(offset, offset + size)); }
  async mapAsync(mode) {
    if (!(mode & (GPUMapMode.READ | GPUMapMode.WRITE))) throw new RangeError('Invalid map mode');
    await this.device.queue.onSubmittedWorkDone();
    this._flush();
    this._mapped = true;
  }
  getMappedRange(offset, size) {
    if (!this._mapped) throw new Error('Buffer is not mapped');
    offset = offset || 0;
    return this._data.slice(offset, size === undefined ? this.size : offset + size);
  }
  unmap() { this._mapped = false; }
  destroy() { this._data = new ArrayBuffer(0); this._pending = []; }
}

function sourceBytes(source, offset, size) {
  if (source instanceof HostBuffer) return source._bytes(offset, size);
  if (source instanceof DeviceView) {
    const a = source.read();
    return new Uint8Array(a.buffer, a.byteOffset + offset, size).slice();
  }
  return native.bufferRead(source.handle, offset, size);
}

class Device {
  constructor(index) {
    this.index = index === undefined ? 0 : index;
    this.handle = native.contextCreate(this.index);
    // HBM bounds capacity here, not the WebGPU dispatch limit.
    this.limits = { maxComputeWorkgroupsPerDimension: 0x7fffffff, maxBufferSize: MAX_BUFFER_SIZE,
                    maxStorageBufferBindingSize: MAX_BUFFER_SIZE };
    this.queue = new Queue(this);
  }
  createCommandEncoder() { return new CommandEncoder(this); }
  createQuerySet(descriptor) { return new QuerySet(this, descriptor); }
  createBuffer(descriptor) {
    const usage = descriptor.usage || 0;
    if (usage & (GPUBufferUsage.MAP_READ | GPUBufferUsage.MAP_WRITE | GPUBufferUsage.QUERY_RESOLVE)) {
      return new HostBuffer(this, descriptor.size, usage);
    }
    return storage(this, descriptor.size, descriptor.label || 'buffer');
  }
  destroy() {
    if (this.handle) native.contextDestroy(this.handle);
    this.handle = null;
  }
}
async function requestDevice(index) { return new Device(index); }

class DeviceView {
  constructor(read) { this.read = read; }
}

// ---- device buffers (src/webgpu/buffers.ts:3-25) ---------------------------
// A StorageBuffer stands for the reference's GPUBuffer of STORAGE usage:
// zero-filled device memory of `size` bytes.
class StorageBuffer {
  constructor(device, size, label) {
    this.device = device; this.size = size; this.label = label;
    this.handle = native.bufferCreate(device.handle, size);
  }
  destroy() {
    if (this.handle) native.bufferDestroy(this.handle);
    this.handle = null;
  }
}
const MAX_BUFFER_SIZE = 2 ** 40;
function storage(device, bytes, label) {
  const size = Math.ceil(bytes / 4) * 4;
  if (!Number.isSafeInteger(size) || size < 4 || size > MAX_BUFFER_SIZE) {
    throw new RangeError(`${label}: unsupported buffer size ${size}`);
  }
  return new StorageBuffer(device, size, label);
}
function upload(device, buffer, values, offset) {
  offset = offset === undefined ? 0 : offset;
  const data = new Uint8Array(Math.ceil(values.byteLength / 4) * 4);
  data.set(new Uint8Array(values.buffer, values.byteOffset, values.byteLength));
  if (offset % 4 || offset + data.byteLength > buffer.size) throw new RangeError('Unaligned/out-of-range buffer upload');
  native.bufferWrite(buffer.handle, offset, data);
}
async function readBuffer(device, buffer, bytes) {
  if (buffer instanceof DeviceView) return buffer.read();
  if (buffer instanceof HostBuffer) {
    await device.queue.onSubmittedWorkDone();
    return buffer._bytes(0, bytes === undefined ? buffer.size : bytes).buffer;
  }
  bytes = bytes === undefined ? buffer.size : bytes;
  if (bytes % 4 || bytes > buffer.size) throw new RangeError('Invalid readback length');
  return native.bufferRead(buffer.handle, 0, bytes);
}

// ---- the model step's kernel protocol (src/model/ops.ts) -------------------
// ModelOps.create(device).commands(): dispatch(name, parameters, buffers, x, y)
// records, submit() queues every dispatch in order in libbgtq.so and waits.
// The attention-path names are served (append, encode_k, dot,
// compressed_dot, softmax, weighted); the model's other kernels are refused.
// A buffer is a StorageBuffer, or a calibration head's config/table (its
// device tables) or ranges (unused by the library's kernels).
class TablesBinding {
  constructor(tables, host) { this.tables = tables; this.host = host; this.size = host.byteLength; }
}
class ModelOps {
  constructor(device) { this.device = device; }
  static async create(device) { return new ModelOps(device); }
  commands() { return new Commands(this); }
}
class Commands {
  constructor(ops) { this.ops = ops; this.list = []; this.uniformBytes = 0; }
  dispatch(name, parameters, buffers, x, y) {
    y = y === undefined ? 1 : y;
    const limit = this.ops.device.limits.maxComputeWorkgroupsPerDimension;
    if (x > limit || y > limit) throw new RangeError('Model dispatch limit');
    const params = Array.from({ length: 8 }, (_, i) => (parameters[i] === undefined ? 0 : parameters[i]) >>> 0);
    const bindings = buffers.map((b) => {
      if (b instanceof StorageBuffer) return [b.handle, null];
      if (b instanceof TablesBinding) return [null, b.tables];
      return null;
    });
    this.uniformBytes += 32;
    this.list.push([name, params, bindings, x, y]);
  }
  async submit() {
    const list = this.list;
    this.list = [];
    native.modelSubmit(this.ops.device.handle, list);
    await this.ops.device.queue.onSubmittedWorkDone();
  }
}

// ---- calibration tables (src/webgpu/layout.ts:8-31) ------------------------
function isInt(x) { return Number.isInteger(x); }
function validateLayout(p) {
  const d = p.dim;
  if (![d, p.groups, p.rowBytes, p.normStride, p.nibbleDims, p.maxCentroids].every(isInt) ||
      d < 2 || d > 128 || d % 2 || p.groups < 1 || p.groups > 8 || p.normStride < p.groups || p.nibbleDims < 0 ||
      p.nibbleDims > d || p.nibbleDims % 2 || p.rowBytes < p.nibbleDims / 2 + d - p.nibbleDims ||
      p.maxCentroids < 2 || p.maxCentroids > 256) {
    throw new RangeError('Invalid Block-GTQ layout');
  }
  const some = (a, f) => Array.prototype.some.call(a, f);
  if (p.permutation.length !== d || new Set(p.permutation).size !== d || some(p.permutation, (i) => i >= d) ||
      p.groupOf.length !== d || some(p.groupOf, (g) => g >= p.groups) || p.positionToCodebook.length !== d ||
      p.rotation.length !== d * d || p.centroids.length !== d * p.maxCentroids || p.offsets.length !== d ||
      p.inverseScales.length !== d || p.codeLut.length % 256 ||
      some(p.positionToCodebook, (c) => c * 256 >= p.codeLut.length)) {
    throw new RangeError('Invalid calibration table shape');
  }
  for (const values of [p.rotation, p.centroids, p.offsets, p.inverseScales]) {
    if (some(values, (x) => !Number.isFinite(x))) throw new RangeError('Nonfinite calibration table');
  }
  for (let i = 0; i < d; i++) {
    for (let bin = 0; bin < 256; bin++) {
      const code = p.codeLut[p.positionToCodebook[i] * 256 + bin];
      if (code >= p.maxCentroids || (i < p.nibbleDims && code > 15)) {
        throw new RangeError('Code LUT incompatible with packing');
      }
    }
  }
}
function tables(p) {
  validateLayout(p);
  const head = [p.dim, p.groups, p.rowBytes, p.normStride, p.nibbleDims, p.maxCentroids];
  const sections = [p.permutation, p.groupOf, p.positionToCodebook, p.codeLut];
  const integer = new Uint32Array(10 + sections.reduce((n, s) => n + s.length, 0));
  integer.set(head, 0);
  let at = 10;
  sections.forEach((s, k) => { integer[6 + k] = at; integer.set(s, at); at += s.length; });
  const floating = new Float32Array(p.rotation.length + p.centroids.length + p.offsets.length + p.inverseScales.length);
  let f = 0;
  for (const s of [p.rotation, p.centroids, p.offsets, p.inverseScales]) { floating.set(s, f); f += s.length; }
  return { integer, floating };
}

// ---- key stores (src/runtime/keys.ts, packed-keys.ts, compressed-keys.ts) ---
function appendCount(values, dim, length, capacity) {
  if (!values.length || values.length % dim) throw new RangeError('K append must contain whole nonempty rows');
  if (values.some((x) => (x & 0x7c00) === 0x7c00)) throw new RangeError('Finite FP16 K required');
  const count = values.length / dim;
  if (length + count > capacity) throw new RangeError('K capacity exceeded');
  return count;
}

class FP16Keys {
  constructor(device, dim, capacity) {
    if (!isInt(dim) || dim < 2 || dim % 2 || !isInt(capacity) || capacity < 1) throw new RangeError('Invalid K dimensions');
    this.kind = 'fp16';
    this.device = device; this.dim = dim; this.capacity = capacity;
    this.handle = native.fp16KeysCreate(device.handle, dim, capacity);
    this.allocations = native.keysAllocations(this.handle);
    const self = this;
    this.buffer = new DeviceView(() => native.keysReadFp16(self.handle, self.capacity * self.dim));
  }
  get length() { return keysLength(this); }
  async append(values) {
    if (this._pending) throw new Error('Concurrent K appends unsupported');
    appendCount(values, this.dim, this.length, this.capacity);
    await runAppend(this, values);
  }
  prepare() { return { buffer: this.buffer, format: 'f16' }; }
  destroy() { destroyAfterAppend(this); }
}

// The append runs off the JS thread and its Promise resolves once the rows
// are on the device (src/runtime/packed-keys.ts:39-49); destroy() during an
// append waits for it. As in the reference, the store reports its earlier
// length and is not ready until that Promise settles, even when the device
// work finished before (src/runtime/packed-keys.ts:43,47,49).
function keysLength(keys) { return keys._pending ? keys._lengthBefore : native.keysLength(keys.handle); }
function keysReady(keys) {
  if (keys._pending) throw new Error('K storage not ready');
  native.keysReady(keys.handle);
}
async function runAppend(keys, values) {
  keys._lengthBefore = native.keysLength(keys.handle);
  keys._pending = true;
  try {
    await native.keysAppendAsync(keys.handle, values);
  } finally {
    keys._pending = false;
    if (keys._destroyRequested) keys.destroy();
  }
}
function destroyAfterAppend(keys) {
  if (keys._pending) { keys._destroyRequested = true; return; }
  if (keys.handle) native.keysDestroy(keys.handle);
  if (keys.tablesHandle) native.tablesDestroy(keys.tablesHandle);
  keys.handle = keys.tablesHandle = null;
}

class PackedKeys {
  constructor(device, parameters, capacity, compressed) {
    if (!isInt(capacity) || capacity < 1 || capacity > device.limits.maxComputeWorkgroupsPerDimension) {
      throw new RangeError('Invalid capacity');
    }
    const t = tables(parameters);
    this.kind = 'block-gtq';
    this.device = device; this.parameters = parameters; this.capacity = capacity; this.dim = parameters.dim;
    this.tablesHandle = native.tablesCreate(device.handle, t.integer, t.floating);
    try {
      this.handle = native.packedKeysCreate(this.tablesHandle, capacity, !!compressed);
    } catch (e) {
      native.tablesDestroy(this.tablesHandle);
      throw e;
    }
    this.allocations = native.keysAllocations(this.handle);
    const self = this;
    const both = () => native.keysRead(self.handle, self.capacity * parameters.rowBytes, self.capacity * parameters.normStride);
    this.packed = new DeviceView(() => both()[0]);
    this.norms = new DeviceView(() => both()[1]);
  }
  static async create(device, p, capacity) { return new PackedKeys(device, p, capacity, false); }
  get length() { return keysLength(this); }
  async append(values) {
    if (this._pending) throw new Error('Concurrent K appends unsupported');
    appendCount(values, this.dim, this.length, this.capacity);
    await runAppend(this, values);
  }
  ready() { keysReady(this); }
  destroy() { destroyAfterAppend(this); }
}

class CompressedKeys extends PackedKeys {
  static async create(device, p, capacity) { return new CompressedKeys(device, p, capacity, true); }
  // prepare(encoder, start?) (src/runtime/compressed-keys.ts:51-57): a pass
  // that materialises FP32 K, with the caller's start timestamp; the view
  // reads the materialised rows.
  prepare(encoder, start) {
    if (this._pending) throw new Error('K append is still pending');
    const self = this;
    if (encoder) {
      const pass = encoder.beginComputePass(start ? { timestampWrites: start } : {});
      pass._enqueue(() => native.keysPrepareDevice(self.handle));
      pass.end();
    }
    return { buffer: new DeviceView(() => native.keysPrepare(self.handle, self.length * self.dim)), format: 'f32' };
  }
}

// ---- values (src/runtime/values.ts; the model path's FP16 cache) -----------
class Values {
  constructor(device, dim, capacity, dtype) {
    if (!isInt(dim) || dim < 1 || !isInt(capacity) || capacity < 1) throw new RangeError('Invalid V dimensions');
    this.device = device; this.dim = dim; this.capacity = capacity;
    this.dtype = dtype === 'f16' ? 'f16' : 'f32';
    this.handle = native.valuesCreate(device.handle, dim, capacity, this.dtype === 'f16' ? DTYPE_F16 : DTYPE_F32);
    this.allocations = native.valuesAllocations(this.handle);
  }
  get length() { return native.valuesLength(this.handle); }
  append(values) { native.valuesAppend(this.handle, values); }
  destroy() { if (this.handle) native.valuesDestroy(this.handle); this.handle = null; }
}

// ---- attention (src/attention/attention.ts, optimized.ts) -----------------
class Session {
  constructor(device, keys, values, maxQueries, materialize) {
    if (keys.device !== device || values.device !== device || keys.dim !== values.dim ||
        keys.capacity !== values.capacity || !isInt(maxQueries) || maxQueries < 1) {
      throw new RangeError('Incompatible attention storage');
    }
    this.device = device; this.keys = keys; this.values = values; this.maxQueries = maxQueries;
    this.handle = native.attentionCreate(keys.handle, values.handle, maxQueries, materialize !== false);
    this.allocations = native.attentionAllocations(this.handle);
    const self = this;
    const q = () => native.attentionQueries(self.handle);
    this.output = new DeviceView(() => native.attentionRead(self.handle, 2, q() * self.keys.dim));
    this._logits = new DeviceView(() => native.attentionRead(self.handle, 0, q() * self.keys.length));
    this._probabilities = new DeviceView(() => native.attentionRead(self.handle, 1, q() * self.keys.length));
  }
  setQueries(q, positions, causal) { native.attentionSetQueries(this.handle, q, positions, !!causal); }
  // record(encoder, timestamps?) (src/attention/attention.ts:44-58): one
  // compute pass (the fused kernel), timestamps index 0 at its start and 1 at
  // its end. Readiness is checked now, as the reference's record does; the
  // launch happens when the command buffer is submitted. Without an encoder
  // the work is queued at once.
  record(encoder, timestamps) {
    if (encoder === undefined) { native.attentionRecord(this.handle); return; }
    if (this._optimized) this.keys.ready();
    if (!native.attentionQueries(this.handle) || this.keys.length !== this.values.length) {
      throw new Error(this._optimized ? 'Attention not ready' : 'Queries/storage not ready');
    }
    const pass = encoder.beginComputePass(timestamps
      ? { timestampWrites: { querySet: timestamps, beginningOfPassWriteIndex: 0, endOfPassWriteIndex: 1 } } : {});
    const h = this.handle;
    pass._enqueue(() => native.attentionRecord(h));
    pass.end();
  }
  async attend(q, positions, causal) {
    this.setQueries(q, positions, causal);
    const encoder = this.device.createCommandEncoder();
    this.record(encoder);
    this.device.queue.submit([encoder.finish()]);
    await this.device.queue.onSubmittedWorkDone();
    return this.output;
  }
  inspect() {
    return { logits: this._logits, probabilities: this._probabilities, output: this.output,
             queries: native.attentionQueries(this.handle), tokens: this.keys.length };
  }
  destroy() { if (this.handle) native.attentionDestroy(this.handle); this.handle = null; }
}

class OptimizedAttention extends Session {
  static async create(device, keys, values, maxQueries, tailMode) {
    const s = new OptimizedAttention(device, keys, values, maxQueries === undefined ? 3 : maxQueries, true);
    s.tailMode = tailMode === undefined ? 'parallel' : tailMode;
    s._optimized = true;
    return s;
  }
}
class AttentionSession extends Session {}
class AttentionEngine {
  constructor(device) { this.device = device; }
  static async create(device) { return new AttentionEngine(device); }
  session(keys, values, maxQueries) {
    return new AttentionSession(this.device, keys, values, maxQueries === undefined ? 3 : maxQueries, true);
  }
}

// ---- calibration-table pipeline (libbgtq, host only) -----------------------
// allocateBits: the greedy allocation of src/reference/allocator.py:4-17.
// layoutGroups: [bits, dims] of each group of a width allocation (ascending
// widths). buildTables: the tables(p) blobs of an allocation, given each
// group's ascending centroids and its rotation (null = identity).
function allocateBits(scores, budget, minBits, maxBits) {
  return native.allocateBits(Float32Array.from(scores), budget, minBits === undefined ? 1 : minBits,
    maxBits === undefined ? 8 : maxBits);
}
function layoutGroups(widths) { return native.layoutGroups(Array.from(widths)); }
function buildTables(widths, groups, rowBytes, normStride) {
  return native.layoutBuild(Array.from(widths), groups.map((g) => [Float32Array.from(g.centroids),
    g.rotation ? Float32Array.from(g.rotation) : null]), rowBytes || 0, normStride || 0);
}

// ---- model calibration (src/model/calibration.ts:4-24) ---------------------
// base is a directory holding calibration.json and its payload. Each head
// keeps its host arrays and a device table set (tables) for the batched entry
// points; the checks and messages are the reference's.
class Calibration {
  constructor(device, sha256) {
    this.device = device; this.sha256 = sha256; this.heads = []; this.allocations = [];
  }
  static async load(device, adapter, base, modelRevision) {
    const fs = require('fs');
    const crypto = require('crypto');
    base = base === undefined ? path.join(process.cwd(), 'fixtures', 'model') : base;
    const m = JSON.parse(fs.readFileSync(path.join(base, 'calibration.json'), 'utf8'));
    const file = fs.readFileSync(path.join(base, m.binary));
    const payload = file.buffer.slice(file.byteOffset, file.byteOffset + file.byteLength);
    const sha = crypto.createHash('sha256').update(file).digest('hex');
    const expected = adapter ? adapter.layers * adapter.kvHeads : 90;
    const expectedRevision = modelRevision !== undefined ? modelRevision
      : (adapter ? undefined : '12fd25f77366fa6b3b4b768ec3050bf629380bac');
    if (sha !== m.sha256 || m.heads.length !== expected || (expectedRevision && m.model_revision !== expectedRevision) ||
        m.upstream_commit !== '3fe14e7d4b8a6c85402818f7e22052527ed42e93') {
      throw new Error('Calibration mismatch');
    }
    const c = new Calibration(device, sha);
    try {
      for (let i = 0; i < expected; i++) {
        const read = (name) => {
          const a = m.arrays[`h${i}_${name}`];
          if (!a || a.offset % 4 || a.offset + a.nbytes > payload.byteLength) throw new Error('Bad calibration descriptor');
          return payload.slice(a.offset, a.offset + a.nbytes);
        };
        const config = new Uint32Array(read('config')), table = new Float32Array(read('table'));
        const ranges = new Uint32Array(read('ranges'));
        if (config[0] !== 64 || config[1] > 8 || ranges.length !== 128 || table.some((x) => !Number.isFinite(x))) {
          throw new Error('Unsupported calibration');
        }
        for (let j = 0; j < 64; j++) {
          for (let k = 0; k < 64; k++) {
            if ((k < ranges[j * 2] || k >= ranges[j * 2 + 1]) && table[k * 64 + j] !== 0) throw new Error('Off-group rotation');
          }
        }
        const handle = native.tablesCreate(device.handle, config, table);
        // config/table bind the head's device tables in the model dispatches
        // (src/model/decoder.ts:52, :55), as the reference's GPU buffers do.
        c.heads.push({
          tables: handle, config: new TablesBinding(handle, config), table: new TablesBinding(handle, table),
          ranges: new TablesBinding(null, ranges), rowBytes: config[2], normStride: config[3],
        });
        c.allocations.push({ name: `head ${i} tables`, role: 'tables', bytes: native.tablesDeviceBytes(handle) });
      }
    } catch (e) {
      c.destroy();
      throw e;
    }
    return c;
  }
  destroy() {
    for (const h of this.heads) if (h.tables) native.tablesDestroy(h.tables);
    this.heads.forEach((h) => { h.tables = null; });
  }
}

module.exports = {
  native, Device, requestDevice, DeviceView, readBuffer, storage, upload, StorageBuffer, ModelOps, Commands,
  GPUBufferUsage, GPUMapMode, CommandEncoder, ComputePass, CommandBuffer, Queue, QuerySet, HostBuffer,
  validateLayout, tables, appendCount, allocateBits, layoutGroups, buildTables,
  FP16Keys, PackedKeys, CompressedKeys, Values, OptimizedAttention, AttentionEngine, AttentionSession, Calibration,
};
