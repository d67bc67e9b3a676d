'use strict';
// Drop-in check through the Node classes (needs a GPU): the reference's
// optimized-attention flow (tests/webgpu/optimized-test.ts:18-45) on a
// committed golden workload. Packed K and FP16 scales must equal the
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

async function main() {
  const device = await bgtq.requestDevice(0);
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
