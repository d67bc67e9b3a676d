"""Host-side checks that need no GPU: the C ABI library, the Python mirror of the
reference's table/validation logic, and the calibration-table generator."""
import ctypes
import re

import numpy as np
import pytest

from conftest import REF, ROOT


def test_library_exports_every_declared_symbol():
    import bgtq
    header = (ROOT / "include" / "bgtq.h").read_text()
    decl = r"^(?:const\s+)?(?:bgtq_status|void|char|int32_t|uint32_t)\s*\*?\s*(bgtq_[a-z0-9_]+)\s*\("
    declared = set(re.findall(decl, header, re.MULTILINE))
    assert len(declared) > 30
    lib = ctypes.CDLL(str(bgtq.LIB_PATH))
    missing = [name for name in sorted(declared) if not hasattr(lib, name)]
    assert not missing, missing
    assert lib.bgtq_abi_version() == 6
    lib.bgtq_model_submit.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    assert lib.bgtq_model_submit(None, None, 0) == 1  # BGTQ_ERR_RANGE: null context, nothing touched


def test_no_device_is_reported_cleanly():
    import bgtq
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(bgtq.DeviceError):
        bgtq.Device(0)


def _mixed(oracle, name):
    import bgtq
    m, a = oracle.read_fixture(REF / "mixed" / f"{name}.json")
    return m, a, bgtq.BlockGTQParameters.from_mixed_fixture(m, a)


def test_tables_serialization_matches_model_blob(oracle):
    """tables(p) (src/webgpu/layout.ts:24-31) reproduces the committed per-head model blobs."""
    import bgtq
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    for i in range(len(m["heads"])):
        p = bgtq.BlockGTQParameters.from_serialized(a[f"h{i}_config"], a[f"h{i}_table"])
        ints, fl = bgtq.tables(p)
        np.testing.assert_array_equal(ints, a[f"h{i}_config"])
        np.testing.assert_array_equal(fl.view(np.uint32), a[f"h{i}_table"].view(np.uint32))


def test_validate_layout_messages(oracle):
    import bgtq
    m, a, p = _mixed(oracle, "mixed_d64")
    bgtq.validate_layout(p)
    for field, value, msg in (("dim", 130, "Invalid Block-GTQ layout"), ("groups", 9, "Invalid Block-GTQ layout"),
                              ("normStride", 1, "Invalid Block-GTQ layout"), ("rowBytes", 10, "Invalid Block-GTQ layout"),
                              ("maxCentroids", 1, "Invalid Block-GTQ layout")):
        bad = bgtq.BlockGTQParameters(**{**p.__dict__, field: value})
        with pytest.raises(bgtq.RangeError, match=msg):
            bgtq.validate_layout(bad)
    perm = np.array(p.permutation).copy()
    perm[1] = perm[0]
    with pytest.raises(bgtq.RangeError, match="Invalid calibration table shape"):
        bgtq.validate_layout(bgtq.BlockGTQParameters(**{**p.__dict__, "permutation": perm}))
    rot = np.array(p.rotation, np.float32).copy()
    rot[5] = np.inf
    with pytest.raises(bgtq.RangeError, match="Nonfinite calibration table"):
        bgtq.validate_layout(bgtq.BlockGTQParameters(**{**p.__dict__, "rotation": rot}))
    lut = np.array(p.codeLut).copy()
    lut[0] = 200  # position 0 is a nibble position
    with pytest.raises(bgtq.RangeError, match="Code LUT incompatible with packing"):
        bgtq.validate_layout(bgtq.BlockGTQParameters(**{**p.__dict__, "codeLut": lut}))


def test_append_count_messages():
    import bgtq
    with pytest.raises(bgtq.RangeError, match="whole nonempty rows"):
        bgtq.append_count(np.zeros(0, np.uint16), 4, 0, 8)
    with pytest.raises(bgtq.RangeError, match="whole nonempty rows"):
        bgtq.append_count(np.zeros(6, np.uint16), 4, 0, 8)
    with pytest.raises(bgtq.RangeError, match="Finite FP16 K required"):
        bgtq.append_count(np.array([0, 0x7C00, 0, 0], np.uint16), 4, 0, 8)
    with pytest.raises(bgtq.RangeError, match="Finite FP16 K required"):
        bgtq.append_count(np.array([0, 0xFE00, 0, 0], np.uint16), 4, 0, 8)
    with pytest.raises(bgtq.RangeError, match="K capacity exceeded"):
        bgtq.append_count(np.zeros(8, np.uint16), 4, 7, 8)
    assert bgtq.append_count(np.zeros(8, np.uint16), 4, 6, 8) == 2


def test_calibration_tables_reproduce_reference(oracle):
    """The table generator rebuilds every committed reference table set bit for bit: the 90 real
    SmolLM2 heads and the 10 mixed layouts, the 64-pair layouts' head_perm included (the tie
    order of calibrate.tie_order)."""
    import json
    import bgtq
    from bgtq import calibrate
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    for i in range(len(m["heads"])):
        p = calibrate.make_parameters(a[f"h{i}_widths"].astype(np.int64))
        ints, fl = bgtq.tables(p)
        np.testing.assert_array_equal(ints, a[f"h{i}_config"], err_msg=f"head {i}")
        np.testing.assert_array_equal(fl.view(np.uint32), a[f"h{i}_table"].view(np.uint32), err_msg=f"head {i}")
    for c in json.loads((REF / "mixed" / "index.json").read_text())["cases"]:
        mm, aa = oracle.read_fixture(REF / "mixed" / f"{c['name']}.json")
        p = calibrate.make_parameters(aa["allocation"].astype(np.int64), row_bytes=mm["row_bytes"],
                                      norm_stride=mm["norm_stride"])
        for key, mine in (("group_of", p.groupOf), ("pos_to_cb", p.positionToCodebook), ("code_lut", p.codeLut),
                          ("rotation", p.rotation), ("centroids", p.centroids), ("lut_offsets", p.offsets),
                          ("lut_inv_scales", p.inverseScales)):
            np.testing.assert_array_equal(np.asarray(mine).reshape(-1), aa[key].reshape(-1), err_msg=f"{c['name']} {key}")
        np.testing.assert_array_equal(p.permutation, aa["head_perm"], err_msg=c["name"])
        g = calibrate.grouping(aa["allocation"].astype(np.int64))
        for key in ("pair_order", "head_perm", "group_bits", "group_offsets", "group_of"):
            np.testing.assert_array_equal(g[key], aa[key], err_msg=f"{c['name']} {key}")
        assert g["nopack_start"] == mm["nopack_start"]


def _fixture_groups(calibrate, widths, integer, floating):
    """Each group's (centroids, rotation block) as the committed table holds them."""
    d, maxc = int(integer[0]), int(integer[5])
    rot = np.asarray(floating[:d * d]).reshape(d, d)
    cents = np.asarray(floating[d * d:d * d + d * maxc]).reshape(d, maxc)
    groups, s = [], 0
    for bits, dims in calibrate.native_layout_groups(widths):
        groups.append((cents[s, :1 << bits], rot[s:s + dims, s:s + dims]))
        s += dims
    return groups


def test_native_table_pipeline_reproduces_reference(oracle):
    """libbgtq's allocator -> grouping -> code LUT pipeline (bgtq_layout_build), given each
    group's codebook and rotation from the committed tables, rebuilds the whole table set
    bit for bit: the 90 SmolLM2 heads and the 10 mixed layouts, head_perm included."""
    import json
    import bgtq
    from bgtq import calibrate
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    for i in range(len(m["heads"])):
        w = a[f"h{i}_widths"].astype(np.int64)
        ints, fl = calibrate.native_tables(w, _fixture_groups(calibrate, w, a[f"h{i}_config"], a[f"h{i}_table"]))
        np.testing.assert_array_equal(ints, a[f"h{i}_config"], err_msg=f"head {i}")
        np.testing.assert_array_equal(fl.view(np.uint32), a[f"h{i}_table"].view(np.uint32), err_msg=f"head {i}")
    for c in json.loads((REF / "mixed" / "index.json").read_text())["cases"]:
        mm, aa = oracle.read_fixture(REF / "mixed" / f"{c['name']}.json")
        w = aa["allocation"].astype(np.int64)
        p = bgtq.BlockGTQParameters.from_mixed_fixture(mm, aa)
        ints, fl = calibrate.native_tables(w, _fixture_groups(calibrate, w, *bgtq.tables(p)), mm["row_bytes"],
                                           mm["norm_stride"])
        q = bgtq.BlockGTQParameters.from_serialized(ints, fl)
        for key, mine, ref in (("group_of", q.groupOf, aa["group_of"]), ("pos_to_cb", q.positionToCodebook, aa["pos_to_cb"]),
                               ("code_lut", q.codeLut, aa["code_lut"]), ("rotation", q.rotation, aa["rotation"]),
                               ("centroids", q.centroids, aa["centroids"]), ("offsets", q.offsets, aa["lut_offsets"]),
                               ("inv", q.inverseScales, aa["lut_inv_scales"])):
            np.testing.assert_array_equal(np.asarray(mine).reshape(-1), np.asarray(ref).reshape(-1),
                                          err_msg=f"{c['name']} {key}")
        assert (q.rowBytes, q.normStride, q.nibbleDims) == (mm["row_bytes"], mm["norm_stride"], mm["nopack_start"])
        np.testing.assert_array_equal(q.permutation, aa["head_perm"], err_msg=c["name"])


def test_tie_order_of_equal_widths(oracle):
    """The pair order of the grouping (torch's non-stable argsort as the reference's goldens were
    written): the committed pair orders of all 10 mixed layouts, among them the two 64-pair
    layouts whose ties a stable sort does not reproduce; on random allocations a sort (widths
    ascending, a permutation), equal to a stable sort up to 32 pairs, and the same in libbgtq."""
    import json
    import bgtq
    from bgtq import calibrate
    unstable = 0
    for c in json.loads((REF / "mixed" / "index.json").read_text())["cases"]:
        mm, aa = oracle.read_fixture(REF / "mixed" / f"{c['name']}.json")
        w = aa["allocation"].astype(np.int64)
        np.testing.assert_array_equal(calibrate.tie_order(w), aa["pair_order"], err_msg=c["name"])
        unstable += not np.array_equal(np.argsort(w, kind="stable"), aa["pair_order"])
    assert unstable == 2  # mixed_d128 and low_d128: the fixtures pin the partition's swaps
    rng = np.random.default_rng(11)
    for _ in range(300):
        n = int(rng.integers(1, 65))
        w = rng.integers(1, int(rng.integers(2, 10)), n).astype(np.int64)
        o = calibrate.tie_order(w)
        assert sorted(o.tolist()) == list(range(n))
        assert np.all(np.diff(w[o]) >= 0)
        if n <= 32:
            np.testing.assert_array_equal(o, np.argsort(w, kind="stable"))
    for _ in range(20):  # libbgtq's grouping: the same head_perm through bgtq_layout_build
        w = rng.integers(1, 9, int(rng.choice([33, 48, 64]))).astype(np.int64)
        p = calibrate.make_parameters(w)
        ints, _ = calibrate.native_tables(w, _fixture_groups(calibrate, w, *bgtq.tables(p)))
        q = bgtq.BlockGTQParameters.from_serialized(ints, bgtq.tables(p)[1])
        o = calibrate.tie_order(w)
        np.testing.assert_array_equal(q.permutation, np.stack([o, o + len(w)], 1).reshape(-1))


def test_native_table_pipeline_matches_python_generator(oracle):
    """Same tables as calibrate.make_parameters for layouts A and B and random allocations,
    with the generator's own codebooks and rotations as the groups' inputs; the allocator
    equals the oracle's."""
    import bgtq
    from bgtq import calibrate
    rng = np.random.default_rng(5)
    cases = []
    for d in (64, 128):
        cases.append(4 * calibrate.allocate_bits(calibrate.geometric_scores(d // 2), (3 * d // 2) // 2, 1, 2))
    for _ in range(6):
        n = int(rng.choice([8, 16, 32, 64]))
        cases.append(rng.integers(1, 9, n).astype(np.int64))
    for w in cases:
        p = calibrate.make_parameters(w)
        ints, fl = calibrate.native_tables(w, _fixture_groups(calibrate, w, *bgtq.tables(p)))
        ri, rf = bgtq.tables(p)
        np.testing.assert_array_equal(ints, ri)
        np.testing.assert_array_equal(fl.view(np.uint32), rf.view(np.uint32))
    for _ in range(200):
        n = int(rng.integers(1, 40))
        s = rng.exponential(size=n).astype(np.float32) * (rng.random(n) > 0.2)
        budget, lo = int(rng.integers(0, 8 * n + 4)), int(rng.integers(0, 3))
        hi = int(rng.integers(lo, 9))
        np.testing.assert_array_equal(calibrate.native_allocate_bits(s, budget, lo, hi),
                                      oracle.allocate_bits(s, budget, lo, hi))
    with pytest.raises(bgtq.RangeError, match="groups in this allocation"):
        calibrate.native_tables(np.array([4, 8]), [(np.arange(16, dtype=np.float32), None)])
    with pytest.raises(bgtq.RangeError, match="ascend"):
        calibrate.native_tables(np.array([1, 1]), [(np.array([1.0, -1.0], np.float32), None)])
    with pytest.raises(bgtq.RangeError, match="outside 1..8"):
        calibrate.native_layout_groups(np.array([0, 3]))


def test_node_table_pipeline(oracle):
    """buildTables / layoutGroups / allocateBits of the Node module (no device needed) rebuild the
    committed calibration tables of every head from their widths and group tables."""
    import json
    import shutil
    import subprocess
    node = shutil.which("node")
    addon = ROOT / "block-gqt-webgpu_amd" / "node" / "bgtq_napi.node"
    if node is None or not addon.exists():
        pytest.skip("node or the built addon is absent")
    script = r"""
const b = require(process.argv[1]); const fs = require('fs'); const path = require('path');
const dir = process.argv[2]; const m = JSON.parse(fs.readFileSync(path.join(dir, 'calibration.json')));
const bin = fs.readFileSync(path.join(dir, m.binary));
const arr = (name, T) => { const d = m.arrays[name]; const c = new Uint8Array(d.nbytes);
  c.set(bin.subarray(d.offset, d.offset + d.nbytes)); return new T(c.buffer); };
let exact = 0;
for (let h = 0; h < m.heads.length; h++) {
  const cfg = arr(`h${h}_config`, Uint32Array), tab = arr(`h${h}_table`, Float32Array);
  const w = Array.from(arr(`h${h}_widths`, Uint32Array));
  const d = cfg[0], maxc = cfg[5];
  let s = 0; const groups = [];
  for (const [bits, dims] of b.layoutGroups(w)) {
    const rot = new Float32Array(dims * dims);
    for (let i = 0; i < dims; i++) for (let j = 0; j < dims; j++) rot[i * dims + j] = tab[(s + i) * d + s + j];
    groups.push({ centroids: tab.subarray(d * d + s * maxc, d * d + s * maxc + (1 << bits)), rotation: rot });
    s += dims;
  }
  const t = b.buildTables(w, groups);
  const same = (x, y) => x.length === y.length && x.every((v, i) => Object.is(v, y[i]) || v === y[i]);
  if (same(t.integer, cfg) && same(new Uint32Array(t.floating.buffer), new Uint32Array(tab.buffer))) exact++;
}
const w = b.allocateBits(Array.from({ length: 32 }, (_, i) => 0.9 ** i), 48, 1, 2);
let msg = ''; try { b.layoutGroups([0, 4]); } catch (e) { msg = e.constructor.name + ': ' + e.message; }
console.log(JSON.stringify({ exact, heads: m.heads.length, ones: w.filter((x) => x === 1).length, msg }));
"""
    r = subprocess.run([node, "-e", script, str(addon.parent / "bgtq.js"), str(REF / "model")], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["exact"] == out["heads"] == 90, out
    assert out["ones"] == 16, out  # layout B: half the pairs at one bit (x4 = 4 bits), half at two
    assert out["msg"] == "RangeError: pair 0: width 0 outside 1..8", out


def test_layout_b_and_a_shapes():
    from bgtq import calibrate
    for d, rb, groups in ((64, 48, 2), (128, 96, 2)):
        p = calibrate.layout_b(d)
        widths = np.asarray(p.permutation)  # grouping sorted: first half 4-bit, second half 8-bit
        assert p.rowBytes == rb and p.groups == groups and p.nibbleDims == d // 2 and p.normStride == 2
        assert np.array_equal(np.asarray(p.groupOf), np.repeat([0, 1], d // 2))
        assert sorted(widths.tolist()) == list(range(d))
    pa = calibrate.layout_a(64)
    assert pa.groups == 3 and pa.rowBytes == 64 and pa.nibbleDims == 0
    pa = calibrate.layout_a(128)
    assert pa.groups == 5 and pa.rowBytes == 116


def test_allocator_mirror_matches_oracle(oracle):
    from bgtq import calibrate
    rng = np.random.default_rng(1)
    for _ in range(200):
        n = int(rng.integers(1, 40))
        s = rng.exponential(size=n).astype(np.float32) * (rng.random(n) > 0.2)
        budget = int(rng.integers(0, 8 * n + 4))
        lo = int(rng.integers(0, 3))
        hi = int(rng.integers(lo, 9))
        np.testing.assert_array_equal(calibrate.allocate_bits(s, budget, lo, hi), oracle.allocate_bits(s, budget, lo, hi))


def test_node_addon_loads_without_a_device():
    """The N-API addon and the JS classes load (no device work) and export every entry point."""
    import shutil
    import subprocess
    node = shutil.which("node")
    addon = ROOT / "block-gqt-webgpu_amd" / "node" / "bgtq_napi.node"
    if node is None or not addon.exists():
        pytest.skip("node or the built addon is absent")
    script = ("const b=require(process.argv[1]);"
              "const want=['contextCreate','tablesCreate','packedKeysCreate','keysAppend','keysRead','valuesCreate',"
              "'valuesAppend','attentionCreate','attentionSetQueries','attentionRecord','attentionRead','tablesDeviceBytes',"
                  "'bufferCreate','bufferWrite','bufferRead','bufferDestroy','modelSubmit'];"
              "const miss=want.filter(k=>typeof b.native[k]!=='function');"
              "const cls=['PackedKeys','CompressedKeys','FP16Keys','Values','OptimizedAttention','AttentionEngine','tables','Calibration',"
                  "'ModelOps','Commands','storage','upload','readBuffer'];"
              "const missc=cls.filter(k=>!b[k]);"
              "console.log(JSON.stringify({abi:b.native.abiVersion,miss,missc}));")
    r = subprocess.run([node, "-e", script, str(addon.parent / "bgtq.js")], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    import json
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out == {"abi": 6, "miss": [], "missc": []}, out


def _tampered_calibration(tmp_path, edit_manifest=None, edit_payload=None):
    """A copy of the committed SmolLM2 calibration with the manifest and/or payload changed
    (the payload's sha256 is rewritten unless the manifest edit says otherwise)."""
    import hashlib
    import json
    m = json.loads((REF / "model" / "calibration.json").read_text())
    payload = bytearray((REF / "model" / m["binary"]).read_bytes())
    if edit_payload:
        edit_payload(m, payload)
        m["sha256"] = hashlib.sha256(payload).hexdigest()
    if edit_manifest:
        edit_manifest(m)
    (tmp_path / m["binary"]).write_bytes(bytes(payload))
    (tmp_path / "calibration.json").write_text(json.dumps(m))
    return tmp_path


def test_calibration_loader_checks(oracle, tmp_path):
    """Calibration.load's manifest and per-head checks (src/model/calibration.ts:8-18), with the
    reference's messages, on the committed SmolLM2 calibration and tampered copies of it."""
    import bgtq
    from bgtq import calibration
    m, sha, blobs = calibration.read(REF / "model")
    _, a = oracle.read_fixture(REF / "model" / "calibration.json")
    assert len(blobs) == 90 and sha == m["sha256"]
    for i, b in enumerate(blobs):
        np.testing.assert_array_equal(b.config, a[f"h{i}_config"])
        np.testing.assert_array_equal(b.table.view(np.uint32), a[f"h{i}_table"].view(np.uint32))
        assert (b.row_bytes, b.norm_stride) == (m["heads"][i]["row_bytes"], m["heads"][i]["norm_stride"])
    # The model geometry given explicitly (30 layers x 3 KV heads) needs no pinned revision.
    assert len(calibration.read(REF / "model", layers=30, kv_heads=3, model_revision=m["model_revision"])[2]) == 90

    def f32_offset(mm, head, index):
        return mm["arrays"][f"h{head}_table"]["offset"] + 4 * index

    def poke(head, index, value):
        def edit(mm, payload):
            payload[f32_offset(mm, head, index):f32_offset(mm, head, index) + 4] = np.float32(value).tobytes()
        return edit

    r0 = a["h5_ranges"].reshape(64, 2)
    j = 0
    k = int(r0[j, 1]) if r0[j, 1] < 64 else int(r0[j, 0]) - 1  # a row outside position j's group
    assert 0 <= k < 64 and not (r0[j, 0] <= k < r0[j, 1])
    cases = [
        (dict(edit_manifest=lambda mm: mm.update(sha256="0" * 64)), {}, "Calibration mismatch"),
        (dict(edit_manifest=lambda mm: mm.update(model_revision="other")), {}, "Calibration mismatch"),
        (dict(edit_manifest=lambda mm: mm.update(upstream_commit="other")), {}, "Calibration mismatch"),
        (dict(edit_manifest=lambda mm: mm["heads"].pop()), {}, "Calibration mismatch"),
        (dict(), dict(layers=2, kv_heads=3), "Calibration mismatch"),
        (dict(edit_manifest=lambda mm: mm["arrays"].pop("h7_ranges")), {}, "Bad calibration descriptor"),
        (dict(edit_manifest=lambda mm: mm["arrays"]["h3_table"].update(offset=mm["arrays"]["h3_table"]["offset"] + 2)),
         {}, "Bad calibration descriptor"),
        (dict(edit_manifest=lambda mm: mm["arrays"]["h89_table"].update(nbytes=1 << 30)), {}, "Bad calibration descriptor"),
        (dict(edit_payload=poke(4, 5000, np.inf)), {}, "Unsupported calibration"),
        (dict(edit_payload=poke(5, k * 64 + j, 0.25)), {}, "Off-group rotation"),
    ]
    for n, (edit, kw, msg) in enumerate(cases):
        d = tmp_path / f"c{n}"
        d.mkdir()
        with pytest.raises(bgtq.StateError, match=msg):
            calibration.read(_tampered_calibration(d, **edit), **kw)
    # An in-group entry may change freely.
    lo = int(r0[j, 0])
    d = tmp_path / "ingroup"
    d.mkdir()
    assert len(calibration.read(_tampered_calibration(d, edit_payload=poke(5, lo * 64 + j, 0.25)))[2]) == 90


def test_node_calibration_checks(oracle, tmp_path):
    """The Node Calibration.load runs the same checks with the same messages (on head 0, before any
    device work: later heads are checked after the earlier heads' tables are on the device)."""
    import json
    import shutil
    import subprocess
    node = shutil.which("node")
    addon = ROOT / "block-gqt-webgpu_amd" / "node" / "bgtq_napi.node"
    if node is None or not addon.exists():
        pytest.skip("node or the built addon is absent")
    _, a = oracle.read_fixture(REF / "model" / "calibration.json")
    r0 = a["h0_ranges"].reshape(64, 2)
    k = int(r0[0, 1]) if r0[0, 1] < 64 else int(r0[0, 0]) - 1

    def poke(head, index, value):
        def edit(mm, payload):
            off = mm["arrays"][f"h{head}_table"]["offset"] + 4 * index
            payload[off:off + 4] = np.float32(value).tobytes()
        return edit

    cases = {
        "Calibration mismatch": dict(edit_manifest=lambda mm: mm.update(model_revision="other")),
        "Bad calibration descriptor": dict(edit_manifest=lambda mm: mm["arrays"].pop("h0_ranges")),
        "Unsupported calibration": dict(edit_payload=poke(0, 5000, np.nan)),
        "Off-group rotation": dict(edit_payload=poke(0, k * 64, 0.25)),
    }
    dirs = {}
    for n, (msg, edit) in enumerate(cases.items()):
        d = tmp_path / f"c{n}"
        d.mkdir()
        dirs[msg] = str(_tampered_calibration(d, **edit))
    script = ("const b=require(process.argv[1]);const dirs=JSON.parse(process.argv[2]);const out={};"
              "(async()=>{for(const [want,dir] of Object.entries(dirs)){"
              "try{await b.Calibration.load({handle:null},undefined,dir);out[want]='no error';}"
              "catch(e){out[want]=e.message;}}console.log(JSON.stringify(out));})();")
    r = subprocess.run([node, "-e", script, str(addon.parent / "bgtq.js"), json.dumps(dirs)],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out == {m: m for m in cases}, out


def test_bake_qproj_puts_queries_in_the_code_domain(oracle):
    """bgtq_bake_qproj (vendor/blockgtq/quantizer.py:1190-1244): for any x, the baked projection's
    query q' = W'x + b' satisfies q'.(c s) = q.k for every K row, where q = Wx + b and k is the
    oracle's reconstruction of the row's codes c and scales s (src/reference/production_math.py:27-31).
    Checked on oracle-encoded rows for layout B (d=64), layout A (d=128) and a SmolLM2 calibration
    head; the transposed fold fails the same check; in-place baking equals out-of-place."""
    import ctypes
    import bgtq
    from bgtq import _lib, calibrate
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    heads = [calibrate.layout_b(64), calibrate.layout_a(128),
             bgtq.BlockGTQParameters.from_serialized(a["h5_config"], a["h5_table"])]
    rng = np.random.default_rng(3)
    for p in heads:
        d, G, F = p.dim, 3, 40
        L = oracle.Layout(dim=p.dim, groups=p.groups, row_bytes=p.rowBytes, norm_stride=p.normStride,
                          nibble_dims=p.nibbleDims, max_centroids=p.maxCentroids, perm=p.permutation,
                          group_of=p.groupOf, pos_to_cb=p.positionToCodebook, code_lut=p.codeLut,
                          rotation=p.rotation, centroids=p.centroids, offsets=p.offsets, inv_scales=p.inverseScales)
        k16 = (rng.standard_normal((50, d)) * 0.9).astype(np.float16)
        packed, norms = oracle.encode_pack(L, k16.view(np.uint16))
        codes = oracle.unpack(packed, d, p.nibbleDims)
        scales = norms.view(np.float16).astype(np.float32)
        keff = oracle.reconstruct(L, codes, scales).astype(np.float64)
        cent = np.asarray(p.centroids, np.float64).reshape(d, p.maxCentroids)
        grp = np.asarray(p.groupOf)
        y = cent[np.arange(d)[None, :], codes] * scales[:, grp]  # code-domain rows (c s), [rows, d]
        W = rng.standard_normal((G * d, F)).astype(np.float32)
        b = rng.standard_normal(G * d).astype(np.float32)
        Wb, bb = calibrate.bake_qproj(p, W, b)
        x = rng.standard_normal((F, 5))
        q = (W.astype(np.float64) @ x + b[:, None]).reshape(G, d, 5)
        qb = (Wb.astype(np.float64) @ x + bb[:, None]).reshape(G, d, 5)
        ref = np.einsum("gdn,td->gtn", q, keff)
        got = np.einsum("gdn,td->gtn", qb, y)
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
        # the fold with the rotation transposed (R^T W[perm]) is a different map unless R is symmetric
        R = np.asarray(p.rotation, np.float64).reshape(d, d)
        if not np.allclose(R, R.T):
            perm = np.asarray(p.permutation)
            qt = np.stack([R.T @ q[g][perm] for g in range(G)])
            assert not np.allclose(np.einsum("gdn,td->gtn", qt, y), ref, rtol=1e-3, atol=1e-3)
        # in place (weight_out = weight, bias_out = bias), as upstream bakes
        ints, fl = bgtq.tables(p)
        Wi, bi = W.copy(), b.copy()
        _lib.check(_lib.lib().bgtq_bake_qproj(_lib.ptr(ints), len(ints), _lib.ptr(fl), len(fl), G, F, _lib.ptr(Wi),
                                              _lib.ptr(bi), _lib.ptr(Wi), _lib.ptr(bi)))
        np.testing.assert_array_equal(Wi, Wb)
        np.testing.assert_array_equal(bi, bb)
    with pytest.raises(bgtq.RangeError, match="multiple of dim"):
        calibrate.bake_qproj(heads[0], np.zeros((65, 4), np.float32))
    ints, fl = bgtq.tables(heads[0])
    bad = ints.copy()
    bad[int(bad[6])] = bad[int(bad[6]) + 1]  # perm no longer a permutation
    z = np.zeros((64, 4), np.float32)
    assert _lib.lib().bgtq_bake_qproj(_lib.ptr(bad), len(bad), _lib.ptr(fl), len(fl), 1, 4, _lib.ptr(z), None,
                                      _lib.ptr(z), None) == _lib.ERR_RANGE


def test_encoder_division_by_reciprocal(tmp_path):
    """The bulk encoder divides a group's 32 inputs by the group norm as x * r with one FMA
    correction (r = 1/norm correctly rounded): equal to IEEE x / norm on every nonzero FP16
    numerator for sampled divisors and group norms (the division check is plain C, built here)."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc is not installed")
    exe = tmp_path / "host_division_check"
    subprocess.run([gcc, "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", str(exe),
                    str(ROOT / "tests" / "host_division_check.c"), "-lm"], check=True)
    r = subprocess.run([str(exe), "600"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout
    assert r.stdout.strip().endswith("mismatches 0"), r.stdout
