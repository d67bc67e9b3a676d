'use strict';
// Drop-in check through the Node classes (needs a GPU): the reference's
// attention validation flow (tests/webgpu/attention-test.ts:21-60), its
// optimized-attention flow (tests/webgpu/optimized-test.ts:18-45) and the
// encoder timing proxy of benchmarks/timing.ts:7-31 on committed golden
// workloads. Packed K and FP16 scales must equal the
// reference encoder's bytes; outputs must match the golden within the
// fixture's baseline tolerance; rejections keep the reference's messages.
//     node block-gqt-webgpu_amd/node/test_napi.js [fixture dir]
const fs = require('fs');
const path = require('path');
const bgtq = require('./bgtq.js');

const FIXTURES = process.argv[2] || path.join(__dirname, '..', '..', 'tests', 'golden', 'reference');

function readFixture(file) {
  const meta = JSON.parse(fs.readFileSync(file, 'utf8'));
  const bin = fs.readFileSync(path.join(path.dirname(file), meta.binary));
  const types = { f32: Float32Array, u32: Uint32Array, u8: Uint8Array, f16: Uint16Array, u16: Uint16Array };
  const arrays = {};
  for (const name of Object.keys(meta.arrays)) {
    const d = meta.arrays[name];
    const T = types[d.dtype];
    const copy = new Uint8Array(d.nbytes);
    copy.set(bin.subarray(d.offset, d.offset + d.nbytes));
    arrays[name] = new T(copy.buffer);
  }
  return { meta, arrays };
}

function parametersFromMixed(meta, a) {
  return {
    dim: meta.dim, groups: meta.n_groups, rowBytes: meta.row_bytes, normStride: meta.norm_stride,
    nibbleDims: meta.nopack_start, maxCentroids: meta.max_centroids, permutation: a.head_perm, groupOf: a.group_of,
    positionToCodebook: a.pos_to_cb, codeLut: a.code_lut, rotation: a.rotation, centroids: a.centroids,
    offsets: a.lut_offsets, inverseScales: a.lut_inv_scales,
  };
}

let failures = 0;
function check(ok, what) {
  if (!ok) { failures += 1; console.log('FAIL', what); } else console.log('ok  ', what);
}
async function rejects(fn, type, message, what) {
  try { await fn(); check(false, what + ' (no error)'); } catch (e) {
    check(e instanceof type && e.message === message, `${what}: ${e.constructor.name} "${e.message}"`);
  }
}

// Element-wise |actual - expected| <= atol + rtol |expected| (both -Infinity counts as equal),
// the rule of the reference's tests/webgpu/compare.ts.
function within(actual, expected, tol) {
  if (actual.length !== expected.length) return false;
  for (let i = 0; i < actual.length; i++) {
    if (actual[i] === -Infinity && expected[i] === -Infinity) continue;
    if (!(Math.abs(actual[i] - expected[i]) <= tol[0] + tol[1] * Math.abs(expected[i]))) return false;
  }
  return true;
}

// The reference's attention validation flow (tests/webgpu/attention-test.ts:21-60) over this
// device: FP16 and compressed key stores appended in two calls (an odd row boundary), an
// incomplete session refused, the compressed store's prepare(encoder) recorded, submitted and read
// back, rejections, then causal and non-causal attend() with every stage within the fixture's
// tolerances, probabilities summing to one and the first causal query returning V0 exactly.
async function attentionTestFlow(device, name) {
  const { meta: m, arrays: f } = readFixture(path.join(FIXTURES, 'attention', name + '.json'));
  const lay = readFixture(path.join(FIXTURES, 'mixed', m.layout + '.json'));
  const parameters = parametersFromMixed(lay.meta, lay.arrays);
  const engine = await bgtq.AttentionEngine.create(device);
  const T = m.context_length, d = m.dim;
  const values = new bgtq.Values(device, d, T);
  const paths = [new bgtq.FP16Keys(device, d, T), await bgtq.CompressedKeys.create(device, parameters, T)];
  try {
    for (const keys of paths) {
      await keys.append(f.k.subarray(0, 3 * d));
      const incomplete = engine.session(keys, values, m.queries);
      try {
        await rejects(() => incomplete.setQueries(f.q, f.positions), RangeError, 'K/V lengths must match and be nonzero',
          `${name} ${keys.kind}: mismatched K/V lengths`);
      } finally { incomplete.destroy(); }
      await keys.append(f.k.subarray(3 * d));
    }
    values.append(f.v.subarray(0, 3 * d));
    values.append(f.v.subarray(3 * d));
    for (const keys of paths) {
      const label = keys.kind === 'fp16' ? 'baseline' : 'compressed';
      const session = engine.session(keys, values, m.queries);
      try {
        if (keys.kind === 'block-gtq') {
          const encoder = device.createCommandEncoder(), view = keys.prepare(encoder);
          device.queue.submit([encoder.finish()]);
          const decoded = new Float32Array((await bgtq.readBuffer(device, view.buffer, T * d * 4)).buffer);
          check(within(decoded, f.reconstructed_k, [1e-4, 0]), `${name}: prepare(encoder) materialises the reconstructed K`);
        }
        await rejects(() => keys.append(new Uint16Array(d)), RangeError, 'K capacity exceeded', `${name} ${label}: capacity`);
        await rejects(() => session.setQueries(new Float32Array(d - 1), new Uint32Array([0])), RangeError,
          'Invalid query shape or causal positions', `${name} ${label}: query shape`);
        await rejects(() => session.setQueries(f.q, new Uint32Array([0, 0, T])), RangeError,
          'Invalid query shape or causal positions', `${name} ${label}: query position`);
        for (const causal of [false, true]) {
          await session.attend(f.q, f.positions, causal);
          const ins = session.inspect(), prefix = causal ? 'causal_' : '';
          const got = {
            logits: await bgtq.readBuffer(device, ins.logits), probabilities: await bgtq.readBuffer(device, ins.probabilities),
            output: await bgtq.readBuffer(device, ins.output),
          };
          for (const stage of ['logits', 'probabilities', 'output']) {
            const tol = m.tolerances[label === 'baseline' ? 'baseline' : 'port'][stage];
            check(within(got[stage], f[`${prefix}${label}_${stage}`], tol), `${name} ${label} causal=${causal}: ${stage}`);
          }
          let sums = true, zeros = true;
          for (let r = 0; r < m.queries; r++) {
            let sum = 0;
            for (let t = 0; t < T; t++) {
              const pr = got.probabilities[r * T + t];
              sum += pr;
              if (pr < 0 || (causal && t > f.positions[r] && pr !== 0)) zeros = false;
            }
            if (Math.abs(sum - 1) > 1e-4) sums = false;
          }
          check(sums && zeros, `${name} ${label} causal=${causal}: probabilities sum to one, causal zeros`);
          if (causal) check(got.output.subarray(0, d).every((x, i) => x === f.v[i]), `${name} ${label}: first causal query = V0`);
        }
      } finally { session.destroy(); }
    }
  } finally { paths.forEach((k) => k.destroy()); values.destroy(); }
}

// The timing flow of benchmarks/timing.ts:7-31 as a caller writes it against WebGPU: a
// timestamp query set, a resolve buffer, a mappable readback buffer, and an encoder proxy that
// adds timestampWrites to every compute pass the recorded work begins; per-pass durations from
// the resolved timestamps.
async function timePasses(device, record, passes, warmups, repetitions) {
  const query = device.createQuerySet({ type: 'timestamp', count: passes * 2 });
  const resolved = device.createBuffer({ size: passes * 16, usage: bgtq.GPUBufferUsage.QUERY_RESOLVE | bgtq.GPUBufferUsage.COPY_SRC });
  const mapped = device.createBuffer({ size: passes * 16, usage: bgtq.GPUBufferUsage.COPY_DST | bgtq.GPUBufferUsage.MAP_READ });
  const samples = Array.from({ length: passes }, () => []);
  try {
    for (let r = -warmups; r < repetitions; r++) {
      const encoder = device.createCommandEncoder();
      let index = 0;
      const proxy = new Proxy(encoder, {
        get(target, key) {
          if (key === 'beginComputePass') {
            return (descriptor) => {
              const i = index++;
              return target.beginComputePass(Object.assign({}, descriptor || {}, {
                timestampWrites: { querySet: query, beginningOfPassWriteIndex: i * 2, endOfPassWriteIndex: i * 2 + 1 } }));
            };
          }
          const v = Reflect.get(target, key, target);
          return typeof v === 'function' ? v.bind(target) : v;
        },
      });
      record(proxy);
      if (index !== passes) throw new Error(`Expected ${passes} passes, got ${index}`);
      encoder.resolveQuerySet(query, 0, passes * 2, resolved, 0);
      encoder.copyBufferToBuffer(resolved, 0, mapped, 0, passes * 16);
      device.queue.submit([encoder.finish()]);
      await mapped.mapAsync(bgtq.GPUMapMode.READ);
      const t = new BigUint64Array(mapped.getMappedRange());
      if (r >= 0) for (let i = 0; i < passes; i++) samples[i].push(Number(t[i * 2 + 1] - t[i * 2]) / 1000);
      mapped.unmap();
    }
    return samples;
  } finally { query.destroy(); resolved.destroy(); mapped.destroy(); }
}

async function main() {
  const device = await bgtq.requestDevice(0);
  for (const name of ['t128_d64', 't512_d128']) await attentionTestFlow(device, name);
  for (const name of ['t128_d64', 't256_d128']) {
    const { meta, arrays: a } = readFixture(path.join(FIXTURES, 'attention', name + '.json'));
    const lay = readFixture(path.join(FIXTURES, 'mixed', meta.layout + '.json'));
    const p = parametersFromMixed(lay.meta, lay.arrays);
    const T = meta.context_length, d = meta.dim;
    const keys = await bgtq.PackedKeys.create(device, p, T);
    const values = new bgtq.Values(device, d, T);
    const att = await bgtq.OptimizedAttention.create(device, keys, values, meta.queries);
    await keys.append(a.k.subarray(0, 3 * d));  // odd first append: rows share packed words
    await keys.append(a.k.subarray(3 * d));
    values.append(a.v.subarray(0, 3 * d));
    values.append(a.v.subarray(3 * d));
    const packed = await bgtq.readBuffer(device, keys.packed);
    const norms = await bgtq.readBuffer(device, keys.norms);
    check(packed.length === a.packed_k.length && packed.every((x, i) => x === a.packed_k[i]), `${name}: packed K bytes`);
    check(norms.length === a.norms.length && norms.every((x, i) => x === a.norms[i]), `${name}: FP16 scale bits`);
    check(keys.allocations.every((x) => x.role !== 'scratch' || x.bytes <= 4), `${name}: no K scratch`);
    const [atol, rtol] = meta.tolerances.baseline.output;
    for (const causal of [false, true]) {
      const out = await bgtq.readBuffer(device, await att.attend(a.q, a.positions, causal));
      const ref = a[(causal ? 'causal_' : '') + 'compressed_output'];
      let worst = 0;
      out.forEach((x, i) => { worst = Math.max(worst, Math.abs(x - ref[i]) / (atol + rtol * Math.abs(ref[i]))); });
      check(worst <= 1, `${name}: output causal=${causal} within the baseline tolerance (worst ratio ${worst.toFixed(3)})`);
      if (causal) {
        const first = out.subarray(0, d);
        check(first.every((x, i) => x === a.v[i]), `${name}: causal query at position 0 returns V0 exactly`);
      }
    }
    await rejects(() => keys.append(new Uint16Array(d)), RangeError, 'K capacity exceeded', `${name}: capacity`);
    await rejects(() => att.attend(a.q, new Uint32Array([0, 1, T]), false), RangeError,
      'Invalid Q/K/V shape or positions', `${name}: position out of range`);
    att.destroy(); values.destroy(); keys.destroy();
  }
  {
    // Encoder timing proxy over OptimizedAttention.record (one fused pass) and
    // AttentionSession.record(encoder, timestamps) with its own query set.
    const { meta, arrays: a } = readFixture(path.join(FIXTURES, 'attention', 't512_d128.json'));
    const lay = readFixture(path.join(FIXTURES, 'mixed', meta.layout + '.json'));
    const p = parametersFromMixed(lay.meta, lay.arrays);
    const T = meta.context_length, d = meta.dim;
    const keys = await bgtq.PackedKeys.create(device, p, T);
    const values = new bgtq.Values(device, d, T);
    const att = await bgtq.OptimizedAttention.create(device, keys, values, meta.queries);
    // The append resolves off the JS thread: while it runs the store is pending.
    const first = keys.append(a.k.subarray(0, 100 * d));
    await rejects(() => keys.append(a.k.subarray(100 * d)), Error, 'Concurrent K appends unsupported',
      'append: a second append while one is pending');
    let pendingReady = false;
    try { keys.ready(); } catch (e) { pendingReady = e.message === 'K storage not ready'; }
    check(pendingReady, 'append: the store is not ready while its append runs');
    await first;
    await keys.append(a.k.subarray(100 * d));
    check(keys.length === T, 'append: both appends committed');
    values.append(a.v);
    att.setQueries(a.q, a.positions, false);
    const samples = await timePasses(device, (e) => att.record(e), 1, 2, 5);
    check(samples[0].length === 5 && samples[0].every((x) => x > 0 && x < 1e6),
      `timing proxy: 5 samples of the fused pass, median ${samples[0].slice().sort((x, y) => x - y)[2].toFixed(1)} us`);
    const engine = await bgtq.AttentionEngine.create(device);
    const fk = new bgtq.FP16Keys(device, d, T);
    await fk.append(a.k);
    const session = engine.session(fk, values, meta.queries);
    session.setQueries(a.q, a.positions, true);
    const qs = device.createQuerySet({ type: 'timestamp', count: 2 });
    const res = device.createBuffer({ size: 16, usage: bgtq.GPUBufferUsage.QUERY_RESOLVE | bgtq.GPUBufferUsage.COPY_SRC });
    const enc = device.createCommandEncoder();
    session.record(enc, qs);
    enc.resolveQuerySet(qs, 0, 2, res, 0);
    device.queue.submit([enc.finish()]);
    const stamps = new BigUint64Array(await bgtq.readBuffer(device, res));
    check(stamps[1] > stamps[0], `record(encoder, timestamps): ${(Number(stamps[1] - stamps[0]) / 1000).toFixed(1)} us`);
    const out = await bgtq.readBuffer(device, session.output);
    check(within(out, a.causal_baseline_output, meta.tolerances.baseline.output), 'record(encoder, timestamps): output');
    let refused = false;
    try { device.createCommandEncoder().beginComputePass().setPipeline(null); } catch (e) { refused = true; }
    check(refused, 'raw WGSL pipelines are refused');
    qs.destroy(); session.destroy(); fk.destroy(); att.destroy(); values.destroy(); keys.destroy();
  }
  const lay = readFixture(path.join(FIXTURES, 'mixed', 'mixed_d64.json'));
  const keys = await bgtq.PackedKeys.create(device, parametersFromMixed(lay.meta, lay.arrays), 4);
  const bad = new Uint16Array(64); bad[5] = 0x7c00;
  await rejects(() => keys.append(bad), RangeError, 'Finite FP16 K required', 'non-finite FP16 K');
  await rejects(() => keys.append(new Uint16Array(63)), RangeError, 'K append must contain whole nonempty rows',
    'partial row');
  check(keys.length === 0, 'failed appends leave the length unchanged');
  let threw = false;
  try { keys.ready(); } catch (e) { threw = e.message === 'K storage not ready'; }
  check(threw, 'empty store is not ready');
  keys.destroy();
  // Model calibration (src/model/calibration.ts:7-21): 90 SmolLM2 heads on the device.
  const cal = await bgtq.Calibration.load(device, undefined, path.join(FIXTURES, 'model'));
  check(cal.heads.length === 90 && cal.allocations.every((x) => x.bytes > 0), 'calibration: 90 heads on the device');
  check(cal.heads[1].rowBytes === 37 && cal.heads[1].normStride === 4, 'calibration: head 1 row geometry');
  // The model codec flow of tests/webgpu/model-codec-test.ts:9-27 through the
  // dispatch protocol: append rounds the post-RoPE rows to FP16, encode_k of
  // every head writes what PackedKeys.append writes for those FP16 rows.
  const ops = await bgtq.ModelOps.create(device);
  const rope = readFixture(path.join(FIXTURES, 'model', 'rope.json')).arrays;
  const data = rope.h3_p4095_y;
  const x = bgtq.storage(device, data.byteLength, 'post-RoPE input');
  const halves = bgtq.storage(device, 3 * 3 * 64 * 2, 'FP16 append reference');
  bgtq.upload(device, x, data);
  const cmd = ops.commands();
  cmd.dispatch('append', [3, 0, 3, 3], [x, halves], 3);
  await cmd.submit();
  const half = new Uint16Array(await bgtq.readBuffer(device, halves));
  let exactHeads = 0;
  for (let h = 0; h < 90; h++) {
    const c = cal.heads[h], cfg = c.config.host, t = c.table.host, maxc = cfg[5], off = 4096 + 64 * maxc, head = h % 3;
    const p = {
      dim: 64, groups: cfg[1], rowBytes: cfg[2], normStride: cfg[3], nibbleDims: cfg[4], maxCentroids: maxc,
      permutation: cfg.slice(cfg[6], cfg[6] + 64), groupOf: cfg.slice(cfg[7], cfg[7] + 64),
      positionToCodebook: cfg.slice(cfg[8], cfg[8] + 64), codeLut: Uint8Array.from(cfg.slice(cfg[9])),
      rotation: t.slice(0, 4096), centroids: t.slice(4096, off), offsets: t.slice(off, off + 64),
      inverseScales: t.slice(off + 64, off + 128),
    };
    const reference = await bgtq.PackedKeys.create(device, p, 3);
    const packed = bgtq.storage(device, 3 * cfg[2], 'model codes'), norms = bgtq.storage(device, 3 * cfg[3] * 2, 'model norms');
    await reference.append(half.subarray(head * 3 * 64, (head + 1) * 3 * 64));
    const e = ops.commands();
    e.dispatch('encode_k', [3, 0, head, 3], [c.config, c.table, x, packed, norms], 3);
    await e.submit();
    const got = new Uint8Array(await bgtq.readBuffer(device, packed));
    const gotN = new Uint16Array(await bgtq.readBuffer(device, norms));
    const ref = await bgtq.readBuffer(device, reference.packed), refN = await bgtq.readBuffer(device, reference.norms);
    // storage() rounds sizes up to 4 bytes: the padding stays zero
    const same = (a, b) => b.every((v, i) => v === a[i]) && a.every((v, i) => i < b.length || v === 0);
    if (same(got, ref) && same(gotN, refN)) exactHeads += 1;
    reference.destroy(); packed.destroy(); norms.destroy();
  }
  check(exactHeads === 90, `model codec: encode_k equals PackedKeys on ${exactHeads} of 90 heads`);
  let limited = false;
  try { cmd.dispatch('softmax', [], [], 2 ** 31); } catch (err) { limited = err instanceof RangeError && err.message === 'Model dispatch limit'; }
  check(limited, 'model dispatch limit');
  await rejects(() => { const r = ops.commands(); r.dispatch('rope', [3, 64, 0, 0, 0, 3, 100000], [x, x, x, x], 1); return r.submit(); },
    Error, 'model kernel rope is outside the attention path this library serves', 'model: non-attention kernels refused');
  x.destroy(); halves.destroy();
  cal.destroy();
  await rejects(() => bgtq.Calibration.load(device, { layers: 2, kvHeads: 3 }, path.join(FIXTURES, 'model')), Error,
    'Calibration mismatch', 'calibration: wrong model geometry');
  device.destroy();
  console.log(failures ? `${failures} check(s) failed` : 'all N-API checks passed');
  process.exit(failures ? 1 : 0);
}

main().catch((e) => { console.log('error', e && e.stack ? e.stack : e); process.exit(2); });
