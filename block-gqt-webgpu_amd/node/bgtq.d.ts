// Type declarations for bgtq.js: the reference's public runtime types
// (src/webgpu/layout.ts:2-5, src/webgpu/buffers.ts:1, src/runtime/keys.ts:3-10,
// src/attention/attention.ts, src/attention/optimized.ts) with GPUDevice and
// GPUBuffer replaced by the HIP-backed Device and DeviceView, and the WebGPU
// encoder / queue / timestamp objects those classes take.

export type BlockGTQParameters = {
  dim: number; groups: number; rowBytes: number; normStride: number; nibbleDims: number; maxCentroids: number;
  permutation: Uint32Array; groupOf: Uint32Array; positionToCodebook: Uint32Array; codeLut: Uint8Array;
  rotation: Float32Array; centroids: Float32Array; offsets: Float32Array; inverseScales: Float32Array;
};
export type Allocation = { name: string; role: "persistent-k" | "persistent-v" | "shared" | "scratch"; bytes: number };

export const GPUBufferUsage: {
  readonly MAP_READ: number; readonly MAP_WRITE: number; readonly COPY_SRC: number; readonly COPY_DST: number;
  readonly INDEX: number; readonly VERTEX: number; readonly UNIFORM: number; readonly STORAGE: number;
  readonly INDIRECT: number; readonly QUERY_RESOLVE: number;
};
export const GPUMapMode: { readonly READ: number; readonly WRITE: number };

/** GPUQuerySet of type "timestamp": HIP events on the context's stream. */
export class QuerySet { readonly device: Device; readonly type: "timestamp"; readonly count: number; destroy(): void; }
export type TimestampWrites = { querySet: QuerySet; beginningOfPassWriteIndex?: number; endOfPassWriteIndex?: number };
/** A compute pass holds the library's work; WGSL pipeline calls throw. */
export class ComputePass { end(): void; }
export class CommandBuffer {}
/** GPUCommandEncoder: recorded work runs on the device at queue.submit, in order. */
export class CommandEncoder {
  readonly device: Device;
  beginComputePass(descriptor?: { timestampWrites?: TimestampWrites }): ComputePass;
  resolveQuerySet(querySet: QuerySet, firstQuery: number, queryCount: number, destination: HostBuffer,
                  destinationOffset?: number): void;
  copyBufferToBuffer(source: StorageBuffer | HostBuffer | DeviceView, sourceOffset: number,
                     destination: StorageBuffer | HostBuffer, destinationOffset: number, size: number): void;
  finish(): CommandBuffer;
}
/** A mappable (MAP_READ / MAP_WRITE) or query-resolve buffer in host memory. */
export class HostBuffer {
  readonly device: Device; readonly size: number; readonly usage: number;
  mapAsync(mode: number): Promise<void>;
  getMappedRange(offset?: number, size?: number): ArrayBuffer;
  unmap(): void;
  destroy(): void;
}
export class Queue {
  submit(commandBuffers: CommandBuffer[]): void;
  /** Resolves off the JS thread once the device finished the submitted work. */
  onSubmittedWorkDone(): Promise<void>;
  writeBuffer(buffer: StorageBuffer | HostBuffer, offset: number, data: ArrayBufferView | ArrayBuffer,
              dataOffset?: number, size?: number): void;
}
export class Device {
  readonly index: number;
  readonly limits: { maxComputeWorkgroupsPerDimension: number; maxBufferSize: number; maxStorageBufferBindingSize: number };
  readonly queue: Queue;
  createCommandEncoder(): CommandEncoder;
  createQuerySet(descriptor: { type: "timestamp"; count: number }): QuerySet;
  createBuffer(descriptor: { size: number; usage: number; label?: string }): StorageBuffer | HostBuffer;
  destroy(): void;
}
export function requestDevice(index?: number): Promise<Device>;

/** Device-resident data; read() copies it to host memory. */
export class DeviceView<T extends ArrayBufferView = ArrayBufferView> {
  read(): T;
}
export function readBuffer<T extends ArrayBufferView>(device: Device, view: DeviceView<T>): Promise<T>;
/** src/webgpu/buffers.ts:3-25 over device memory of libbgtq (zero-filled, size rounded up to 4). */
export class StorageBuffer { readonly device: Device; readonly size: number; readonly label: string; destroy(): void; }
export function storage(device: Device, bytes: number, label: string): StorageBuffer;
export function upload(device: Device, buffer: StorageBuffer, values: ArrayBufferView, offset?: number): void;
export function readBuffer(device: Device, buffer: StorageBuffer | HostBuffer, bytes?: number): Promise<ArrayBuffer>;
/** src/model/ops.ts: the attention-path names append, encode_k, dot, compressed_dot, softmax, weighted. */
export class ModelOps {
  static create(device: Device): Promise<ModelOps>;
  readonly device: Device;
  commands(): Commands;
}
export class Commands {
  uniformBytes: number;
  dispatch(name: string, parameters: number[], buffers: (StorageBuffer | TablesBinding | null)[], x: number,
           y?: number): void;
  submit(): Promise<void>;
}

export function validateLayout(p: BlockGTQParameters): void;
export function tables(p: BlockGTQParameters): { integer: Uint32Array; floating: Float32Array };
export function appendCount(values: Uint16Array, dim: number, length: number, capacity: number): number;
/** The table pipeline of libbgtq (host only): allocator, grouping, code LUT. */
export function allocateBits(scores: ArrayLike<number>, budget: number, minBits?: number, maxBits?: number): number[];
export function layoutGroups(widths: ArrayLike<number>): [bits: number, dims: number][];
export function buildTables(widths: ArrayLike<number>, groups: { centroids: ArrayLike<number>; rotation?: ArrayLike<number> | null }[],
                            rowBytes?: number, normStride?: number): { integer: Uint32Array; floating: Float32Array };

export type KeyView = { buffer: DeviceView<Uint16Array | Float32Array>; format: "f16" | "f32" };
export interface KeyStore {
  readonly device: Device; readonly dim: number; readonly capacity: number; readonly length: number;
  readonly allocations: Allocation[]; readonly kind: "fp16" | "block-gtq";
  append(values: Uint16Array): Promise<void>;
  prepare(encoder?: CommandEncoder, start?: TimestampWrites): KeyView;
  destroy(): void;
}

export class FP16Keys implements KeyStore {
  constructor(device: Device, dim: number, capacity: number);
  readonly device: Device; readonly dim: number; readonly capacity: number; readonly length: number;
  readonly allocations: Allocation[]; readonly kind: "fp16";
  readonly buffer: DeviceView<Uint16Array>;
  append(values: Uint16Array): Promise<void>;
  prepare(encoder?: CommandEncoder, start?: TimestampWrites): KeyView;
  destroy(): void;
}

export class PackedKeys {
  static create(device: Device, p: BlockGTQParameters, capacity: number): Promise<PackedKeys>;
  readonly device: Device; readonly parameters: BlockGTQParameters; readonly dim: number;
  readonly capacity: number; readonly length: number; readonly allocations: Allocation[];
  readonly kind: "block-gtq";
  readonly packed: DeviceView<Uint8Array>;
  readonly norms: DeviceView<Uint16Array>;
  append(values: Uint16Array): Promise<void>;
  ready(): void;
  destroy(): void;
}
export class CompressedKeys extends PackedKeys implements KeyStore {
  static create(device: Device, p: BlockGTQParameters, capacity: number): Promise<CompressedKeys>;
  /** A pass materialising FP32 K (with the caller's start timestamp), recorded into encoder. */
  prepare(encoder?: CommandEncoder, start?: TimestampWrites): KeyView;
}

export class Values {
  constructor(device: Device, dim: number, capacity: number, dtype?: "f32" | "f16");
  readonly device: Device; readonly dim: number; readonly capacity: number; readonly length: number;
  readonly dtype: "f32" | "f16"; readonly allocations: Allocation[];
  append(values: Float32Array): void;
  destroy(): void;
}

export type Inspection = {
  logits: DeviceView<Float32Array>; probabilities: DeviceView<Float32Array>; output: DeviceView<Float32Array>;
  queries: number; tokens: number;
};
declare class Session {
  readonly device: Device; readonly maxQueries: number; readonly allocations: Allocation[];
  readonly output: DeviceView<Float32Array>;
  setQueries(q: Float32Array, positions: Uint32Array, causal?: boolean): void;
  /** One compute pass (timestamps index 0 at its start, 1 at its end); without an encoder, queued at once. */
  record(encoder?: CommandEncoder, timestamps?: QuerySet): void;
  attend(q: Float32Array, positions: Uint32Array, causal?: boolean): Promise<DeviceView<Float32Array>>;
  inspect(): Inspection;
  destroy(): void;
}
export class OptimizedAttention extends Session {
  static create(device: Device, keys: PackedKeys, values: Values, maxQueries?: number,
                tailMode?: "serial" | "parallel"): Promise<OptimizedAttention>;
  readonly keys: PackedKeys; readonly values: Values; tailMode: "serial" | "parallel";
}
export class AttentionSession extends Session {
  readonly keys: KeyStore; readonly values: Values;
}
export class AttentionEngine {
  static create(device: Device): Promise<AttentionEngine>;
  readonly device: Device;
  session(keys: KeyStore, values: Values, maxQueries?: number): AttentionSession;
}

/** src/model/calibration.ts: base is a directory with calibration.json and its payload. */
/** A head's config/table: its device tables as a model dispatch binding (host copy in `host`). */
export class TablesBinding<T extends ArrayBufferView = ArrayBufferView> {
  readonly tables: unknown; readonly host: T; readonly size: number;
}
export type CalibrationHead = {
  tables: unknown; config: TablesBinding<Uint32Array>; table: TablesBinding<Float32Array>;
  ranges: TablesBinding<Uint32Array>; rowBytes: number; normStride: number;
};
export class Calibration {
  static load(device: Device, adapter?: { layers: number; kvHeads: number }, base?: string,
              modelRevision?: string): Promise<Calibration>;
  readonly device: Device;
  readonly sha256: string;
  readonly heads: CalibrationHead[];
  readonly allocations: { name: string; role: "tables"; bytes: number }[];
  destroy(): void;
}
