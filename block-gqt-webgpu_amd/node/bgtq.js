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
class Device {
  constructor(index) {
    this.index = index === undefined ? 0 : index;
    this.handle = native.contextCreate(this.index);
    // HBM bounds capacity here, not the WebGPU dispatch limit.
    this.limits = { maxComputeWorkgroupsPerDimension: 0x7fffffff };
    const self = this;
    this.queue = { onSubmittedWorkDone: async function () { native.contextSynchronize(self.handle); } };
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
  get length() { return native.keysLength(this.handle); }
  async append(values) {
    appendCount(values, this.dim, this.length, this.capacity);
    native.keysAppend(this.handle, values);
  }
  prepare() { return { buffer: this.buffer, format: 'f16' }; }
  destroy() { if (this.handle) native.keysDestroy(this.handle); this.handle = null; }
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
  get length() { return native.keysLength(this.handle); }
  async append(values) {
    appendCount(values, this.dim, this.length, this.capacity);
    native.keysAppend(this.handle, values);  // resolves after the encode has completed
  }
  ready() { native.keysReady(this.handle); }
  destroy() {
    if (this.handle) native.keysDestroy(this.handle);
    if (this.tablesHandle) native.tablesDestroy(this.tablesHandle);
    this.handle = this.tablesHandle = null;
  }
}

class CompressedKeys extends PackedKeys {
  static async create(device, p, capacity) { return new CompressedKeys(device, p, capacity, true); }
  prepare() {
    const self = this;
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
  record() { native.attentionRecord(this.handle); }
  async attend(q, positions, causal) {
    this.setQueries(q, positions, causal);
    this.record();
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
  validateLayout, tables, appendCount, allocateBits, layoutGroups, buildTables,
  FP16Keys, PackedKeys, CompressedKeys, Values, OptimizedAttention, AttentionEngine, AttentionSession, Calibration,
};
