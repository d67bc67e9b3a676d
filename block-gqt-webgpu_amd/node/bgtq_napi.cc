// Node N-API addon over the C ABI of libbgtq.so (include/bgtq.h).
//
// This is the native half of the drop-in for the reference's WebGPU substrate
// (src/webgpu): flat functions over opaque handles, one per C entry point the
// TypeScript runtime classes need. bgtq.js (next to this file) rebuilds the
// reference's classes (src/runtime/*.ts, src/attention/*.ts) on top of it with
// the same names, arguments and error behaviour. A bgtq status becomes a JS
// RangeError (BGTQ_ERR_RANGE, the reference's RangeError) or Error (every other
// failure) carrying bgtq_last_error().
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "bgtq.h"

namespace {

#define NAPI_TRY(env, call)                                      \
  do {                                                           \
    if ((call) != napi_ok) {                                     \
      napi_throw_error((env), nullptr, "N-API call failed: " #call); \
      return nullptr;                                            \
    }                                                            \
  } while (0)

napi_value throw_status(napi_env env, bgtq_status s) {
  const char *msg = bgtq_last_error();
  if (s == BGTQ_ERR_RANGE) napi_throw_range_error(env, nullptr, msg);
  else napi_throw_error(env, nullptr, msg);
  return nullptr;
}

#define BGTQ_TRY(env, call)                  \
  do {                                       \
    bgtq_status s_ = (call);                 \
    if (s_ != BGTQ_OK) return throw_status((env), s_); \
  } while (0)

struct Args {
  napi_value v[8];
  size_t n = 8;
};

bool get_args(napi_env env, napi_callback_info info, Args &a, size_t need) {
  if (napi_get_cb_info(env, info, &a.n, a.v, nullptr, nullptr) != napi_ok) return false;
  if (a.n < need) {
    napi_throw_type_error(env, nullptr, "missing arguments");
    return false;
  }
  return true;
}

void *handle(napi_env env, napi_value v) {
  void *p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok) return nullptr;
  return p;
}

napi_value wrap(napi_env env, void *p) {
  napi_value out;
  if (napi_create_external(env, p, nullptr, nullptr, &out) != napi_ok) return nullptr;
  return out;
}

napi_value num(napi_env env, double x) {
  napi_value out;
  napi_create_double(env, x, &out);
  return out;
}

napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

int64_t to_i64(napi_env env, napi_value v) {
  int64_t x = 0;
  napi_get_value_int64(env, v, &x);
  return x;
}

// Typed array view: data pointer and element count.
template <typename T>
bool typed(napi_env env, napi_value v, napi_typedarray_type want, T **data, size_t *count) {
  napi_typedarray_type type;
  size_t length = 0, offset = 0;
  void *ptr = nullptr;
  napi_value buffer;
  if (napi_get_typedarray_info(env, v, &type, &length, &ptr, &buffer, &offset) != napi_ok || type != want) {
    napi_throw_type_error(env, nullptr, "unexpected typed array type");
    return false;
  }
  *data = static_cast<T *>(ptr);
  *count = length;
  return true;
}

template <typename T>
napi_value new_typed(napi_env env, napi_typedarray_type type, size_t count, T **data) {
  napi_value ab, out;
  void *raw = nullptr;
  if (napi_create_arraybuffer(env, count * sizeof(T), &raw, &ab) != napi_ok) return nullptr;
  if (napi_create_typedarray(env, type, count, ab, 0, &out) != napi_ok) return nullptr;
  *data = static_cast<T *>(raw);
  return out;
}

napi_value allocations(napi_env env, bgtq_status (*fn)(const void *, bgtq_allocation *, size_t, size_t *),
                       const void *obj) {
  size_t n = 0;
  BGTQ_TRY(env, fn(obj, nullptr, 0, &n));
  std::vector<bgtq_allocation> items(n);
  BGTQ_TRY(env, fn(obj, items.data(), n, &n));
  static const char *roles[] = {"persistent-k", "persistent-v", "shared", "scratch"};
  napi_value arr;
  NAPI_TRY(env, napi_create_array_with_length(env, n, &arr));
  for (size_t i = 0; i < n; ++i) {
    napi_value o, name, role;
    NAPI_TRY(env, napi_create_object(env, &o));
    NAPI_TRY(env, napi_create_string_utf8(env, items[i].name, NAPI_AUTO_LENGTH, &name));
    NAPI_TRY(env, napi_create_string_utf8(env, roles[items[i].role & 3], NAPI_AUTO_LENGTH, &role));
    NAPI_TRY(env, napi_set_named_property(env, o, "name", name));
    NAPI_TRY(env, napi_set_named_property(env, o, "role", role));
    NAPI_TRY(env, napi_set_named_property(env, o, "bytes", num(env, (double)items[i].bytes)));
    NAPI_TRY(env, napi_set_element(env, arr, (uint32_t)i, o));
  }
  return arr;
}

bgtq_status keys_ledger(const void *o, bgtq_allocation *a, size_t cap, size_t *n) {
  return bgtq_keys_allocations(static_cast<const bgtq_keys *>(o), a, cap, n);
}
bgtq_status values_ledger(const void *o, bgtq_allocation *a, size_t cap, size_t *n) {
  return bgtq_values_allocations(static_cast<const bgtq_values *>(o), a, cap, n);
}
bgtq_status attention_ledger(const void *o, bgtq_allocation *a, size_t cap, size_t *n) {
  return bgtq_attention_allocations(static_cast<const bgtq_attention *>(o), a, cap, n);
}

// ---- context -------------------------------------------------------------
napi_value ContextCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bgtq_context *ctx = nullptr;
  BGTQ_TRY(env, bgtq_context_create((int32_t)to_i64(env, a.v[0]), &ctx));
  return wrap(env, ctx);
}
napi_value ContextDestroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bgtq_context_destroy(static_cast<bgtq_context *>(handle(env, a.v[0])));
  return undefined(env);
}
napi_value ContextSynchronize(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  BGTQ_TRY(env, bgtq_context_synchronize(static_cast<bgtq_context *>(handle(env, a.v[0]))));
  return undefined(env);
}

// ---- tables --------------------------------------------------------------
napi_value TablesCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  uint32_t *ints;
  float *fl;
  size_t ni, nf;
  if (!typed(env, a.v[1], napi_uint32_array, &ints, &ni) || !typed(env, a.v[2], napi_float32_array, &fl, &nf))
    return nullptr;
  bgtq_tables *t = nullptr;
  BGTQ_TRY(env, bgtq_tables_create(static_cast<bgtq_context *>(handle(env, a.v[0])), ints, ni, fl, nf, &t));
  return wrap(env, t);
}
napi_value TablesDeviceBytes(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bgtq_tables_info ti{};
  BGTQ_TRY(env, bgtq_tables_info_get(static_cast<bgtq_tables *>(handle(env, a.v[0])), &ti));
  napi_value v;
  NAPI_TRY(env, napi_create_double(env, (double)ti.device_bytes, &v));
  return v;
}
napi_value TablesDestroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bgtq_tables_destroy(static_cast<bgtq_tables *>(handle(env, a.v[0])));
  return undefined(env);
}

// ---- keys ----------------------------------------------------------------
napi_value Fp16KeysCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  bgtq_keys *k = nullptr;
  BGTQ_TRY(env, bgtq_fp16_keys_create(static_cast<bgtq_context *>(handle(env, a.v[0])), (uint32_t)to_i64(env, a.v[1]),
                                      (uint32_t)to_i64(env, a.v[2]), &k));
  return wrap(env, k);
}
napi_value PackedKeysCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  bool compressed = false;
  napi_get_value_bool(env, a.v[2], &compressed);
  bgtq_keys *k = nullptr;
  bgtq_tables *t = static_cast<bgtq_tables *>(handle(env, a.v[0]));
  const uint32_t cap = (uint32_t)to_i64(env, a.v[1]);
  BGTQ_TRY(env, compressed ? bgtq_compressed_keys_create(t, cap, &k) : bgtq_packed_keys_create(t, cap, &k));
  return wrap(env, k);
}
napi_value KeysAppend(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  uint16_t *bits;
  size_t n;
  if (!typed(env, a.v[1], napi_uint16_array, &bits, &n)) return nullptr;
  BGTQ_TRY(env, bgtq_keys_append(static_cast<bgtq_keys *>(handle(env, a.v[0])), bits, n));
  return undefined(env);
}
napi_value KeysReady(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  BGTQ_TRY(env, bgtq_keys_ready(static_cast<bgtq_keys *>(handle(env, a.v[0]))));
  return undefined(env);
}
napi_value KeysLength(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  return num(env, bgtq_keys_length(static_cast<bgtq_keys *>(handle(env, a.v[0]))));
}
napi_value KeysRead(napi_env env, napi_callback_info info) {
  // -> [Uint8Array packed (capacity*rowBytes), Uint16Array norms (capacity*normStride)]
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  bgtq_keys *k = static_cast<bgtq_keys *>(handle(env, a.v[0]));
  const size_t pb = (size_t)to_i64(env, a.v[1]), nc = (size_t)to_i64(env, a.v[2]);
  uint8_t *p;
  uint16_t *q;
  napi_value packed = new_typed<uint8_t>(env, napi_uint8_array, pb, &p);
  napi_value norms = new_typed<uint16_t>(env, napi_uint16_array, nc, &q);
  if (!packed || !norms) return nullptr;
  BGTQ_TRY(env, bgtq_keys_read_packed(k, p, pb, q, nc));
  napi_value out;
  NAPI_TRY(env, napi_create_array_with_length(env, 2, &out));
  NAPI_TRY(env, napi_set_element(env, out, 0, packed));
  NAPI_TRY(env, napi_set_element(env, out, 1, norms));
  return out;
}
napi_value KeysReadFp16(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  uint16_t *p;
  const size_t n = (size_t)to_i64(env, a.v[1]);
  napi_value out = new_typed<uint16_t>(env, napi_uint16_array, n, &p);
  if (!out) return nullptr;
  BGTQ_TRY(env, bgtq_keys_read_fp16(static_cast<bgtq_keys *>(handle(env, a.v[0])), p, n));
  return out;
}
napi_value KeysPrepare(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  float *p;
  const size_t n = (size_t)to_i64(env, a.v[1]);
  napi_value out = new_typed<float>(env, napi_float32_array, n, &p);
  if (!out) return nullptr;
  BGTQ_TRY(env, bgtq_keys_prepare(static_cast<bgtq_keys *>(handle(env, a.v[0])), p, n));
  return out;
}
napi_value KeysAllocations(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  return allocations(env, &keys_ledger, handle(env, a.v[0]));
}
napi_value KeysDestroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bgtq_keys_destroy(static_cast<bgtq_keys *>(handle(env, a.v[0])));
  return undefined(env);
}

// ---- values --------------------------------------------------------------
napi_value ValuesCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  bgtq_values *v = nullptr;
  BGTQ_TRY(env, bgtq_values_create(static_cast<bgtq_context *>(handle(env, a.v[0])), (uint32_t)to_i64(env, a.v[1]),
                                   (uint32_t)to_i64(env, a.v[2]), (int32_t)to_i64(env, a.v[3]), &v));
  return wrap(env, v);
}
napi_value ValuesAppend(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  float *x;
  size_t n;
  if (!typed(env, a.v[1], napi_float32_array, &x, &n)) return nullptr;
  BGTQ_TRY(env, bgtq_values_append(static_cast<bgtq_values *>(handle(env, a.v[0])), x, n));
  return undefined(env);
}
napi_value ValuesLength(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  return num(env, bgtq_values_length(static_cast<bgtq_values *>(handle(env, a.v[0]))));
}
napi_value ValuesAllocations(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  return allocations(env, &values_ledger, handle(env, a.v[0]));
}
napi_value ValuesDestroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bgtq_values_destroy(static_cast<bgtq_values *>(handle(env, a.v[0])));
  return undefined(env);
}

// ---- attention sessions --------------------------------------------------
napi_value AttentionCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  bool mat = true;
  napi_get_value_bool(env, a.v[3], &mat);
  bgtq_attention *s = nullptr;
  BGTQ_TRY(env, bgtq_attention_create(static_cast<bgtq_keys *>(handle(env, a.v[0])),
                                      static_cast<bgtq_values *>(handle(env, a.v[1])), (uint32_t)to_i64(env, a.v[2]),
                                      mat ? 1 : 0, &s));
  return wrap(env, s);
}
napi_value AttentionSetQueries(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  float *q;
  uint32_t *pos;
  size_t nq, np;
  if (!typed(env, a.v[1], napi_float32_array, &q, &nq) || !typed(env, a.v[2], napi_uint32_array, &pos, &np))
    return nullptr;
  bool causal = false;
  napi_get_value_bool(env, a.v[3], &causal);
  BGTQ_TRY(env, bgtq_attention_set_queries(static_cast<bgtq_attention *>(handle(env, a.v[0])), q, nq, pos, np,
                                           causal ? 1 : 0));
  return undefined(env);
}
napi_value AttentionRecord(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  BGTQ_TRY(env, bgtq_attention_record(static_cast<bgtq_attention *>(handle(env, a.v[0]))));
  return undefined(env);
}
napi_value AttentionRead(napi_env env, napi_callback_info info) {
  // which: 0 logits, 1 probabilities, 2 output
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  float *p;
  const size_t n = (size_t)to_i64(env, a.v[2]);
  napi_value out = new_typed<float>(env, napi_float32_array, n, &p);
  if (!out) return nullptr;
  BGTQ_TRY(env, bgtq_attention_read(static_cast<bgtq_attention *>(handle(env, a.v[0])), (int32_t)to_i64(env, a.v[1]),
                                    p, n));
  return out;
}
napi_value AttentionQueries(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  return num(env, bgtq_attention_queries(static_cast<bgtq_attention *>(handle(env, a.v[0]))));
}
napi_value AttentionAllocations(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  return allocations(env, &attention_ledger, handle(env, a.v[0]));
}
napi_value AttentionDestroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bgtq_attention_destroy(static_cast<bgtq_attention *>(handle(env, a.v[0])));
  return undefined(env);
}

// ---- calibration-table pipeline (host only) --------------------------------
std::vector<int64_t> int_list(napi_env env, napi_value arr, bool *ok) {
  uint32_t n = 0;
  std::vector<int64_t> out;
  *ok = napi_get_array_length(env, arr, &n) == napi_ok;
  for (uint32_t i = 0; *ok && i < n; ++i) {
    napi_value e;
    *ok = napi_get_element(env, arr, i, &e) == napi_ok;
    if (*ok) out.push_back(to_i64(env, e));
  }
  if (!*ok) napi_throw_type_error(env, nullptr, "expected an array of integers");
  return out;
}
napi_value AllocateBits(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  float *s;
  size_t n;
  if (!typed(env, a.v[0], napi_float32_array, &s, &n)) return nullptr;
  std::vector<int64_t> w(n);
  BGTQ_TRY(env, bgtq_allocate_bits(s, n, to_i64(env, a.v[1]), (int32_t)to_i64(env, a.v[2]), (int32_t)to_i64(env, a.v[3]),
                                   w.data()));
  napi_value arr;
  NAPI_TRY(env, napi_create_array_with_length(env, n, &arr));
  for (size_t i = 0; i < n; ++i) NAPI_TRY(env, napi_set_element(env, arr, (uint32_t)i, num(env, (double)w[i])));
  return arr;
}
napi_value LayoutGroups(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bool ok;
  std::vector<int64_t> w = int_list(env, a.v[0], &ok);
  if (!ok) return nullptr;
  int32_t ng = 0, bits[8], dims[8];
  BGTQ_TRY(env, bgtq_layout_groups(w.data(), w.size(), &ng, bits, dims));
  napi_value arr;
  NAPI_TRY(env, napi_create_array_with_length(env, ng, &arr));
  for (int32_t k = 0; k < ng; ++k) {
    napi_value pair;
    NAPI_TRY(env, napi_create_array_with_length(env, 2, &pair));
    NAPI_TRY(env, napi_set_element(env, pair, 0, num(env, bits[k])));
    NAPI_TRY(env, napi_set_element(env, pair, 1, num(env, dims[k])));
    NAPI_TRY(env, napi_set_element(env, arr, (uint32_t)k, pair));
  }
  return arr;
}
// layoutBuild(widths, [[Float32Array centroids, Float32Array|null rotation], ...], rowBytes, normStride)
napi_value LayoutBuild(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  bool ok;
  std::vector<int64_t> w = int_list(env, a.v[0], &ok);
  if (!ok) return nullptr;
  uint32_t ng = 0;
  NAPI_TRY(env, napi_get_array_length(env, a.v[1], &ng));
  std::vector<bgtq_group_tables> groups(ng);
  for (uint32_t k = 0; k < ng; ++k) {
    napi_value g, c, r;
    napi_valuetype rt;
    NAPI_TRY(env, napi_get_element(env, a.v[1], k, &g));
    NAPI_TRY(env, napi_get_element(env, g, 0, &c));
    NAPI_TRY(env, napi_get_element(env, g, 1, &r));
    float *cd, *rd = nullptr;
    size_t cn, rn;
    if (!typed(env, c, napi_float32_array, &cd, &cn)) return nullptr;
    NAPI_TRY(env, napi_typeof(env, r, &rt));
    if (rt == napi_object && !typed(env, r, napi_float32_array, &rd, &rn)) return nullptr;
    groups[k] = bgtq_group_tables{cd, rd};
  }
  const int32_t rb = (int32_t)to_i64(env, a.v[2]), ns = (int32_t)to_i64(env, a.v[3]);
  size_t ni = 0, nf = 0;
  BGTQ_TRY(env, bgtq_layout_build(w.data(), w.size(), groups.data(), groups.size(), rb, ns, nullptr, &ni, nullptr, &nf));
  uint32_t *ints;
  float *fl;
  napi_value vi = new_typed(env, napi_uint32_array, ni, &ints), vf = new_typed(env, napi_float32_array, nf, &fl);
  if (!vi || !vf) return nullptr;
  BGTQ_TRY(env, bgtq_layout_build(w.data(), w.size(), groups.data(), groups.size(), rb, ns, ints, &ni, fl, &nf));
  napi_value out;
  NAPI_TRY(env, napi_create_object(env, &out));
  NAPI_TRY(env, napi_set_named_property(env, out, "integer", vi));
  NAPI_TRY(env, napi_set_named_property(env, out, "floating", vf));
  return out;
}

// ---- device buffers (src/webgpu/buffers.ts storage/upload/readBuffer) ----
napi_value BufferCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  bgtq_buffer *b = nullptr;
  BGTQ_TRY(env, bgtq_buffer_create(static_cast<bgtq_context *>(handle(env, a.v[0])), (size_t)to_i64(env, a.v[1]), &b));
  return wrap(env, b);
}
napi_value BufferWrite(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  uint8_t *data;
  size_t n;
  if (!typed(env, a.v[2], napi_uint8_array, &data, &n)) return nullptr;
  BGTQ_TRY(env, bgtq_buffer_write(static_cast<bgtq_buffer *>(handle(env, a.v[0])), (size_t)to_i64(env, a.v[1]), data, n));
  return undefined(env);
}
napi_value BufferRead(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  const size_t n = (size_t)to_i64(env, a.v[2]);
  napi_value ab;
  void *raw = nullptr;
  NAPI_TRY(env, napi_create_arraybuffer(env, n, &raw, &ab));
  BGTQ_TRY(env, bgtq_buffer_read(static_cast<bgtq_buffer *>(handle(env, a.v[0])), (size_t)to_i64(env, a.v[1]), raw, n));
  return ab;
}
napi_value BufferDestroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bgtq_buffer_destroy(static_cast<bgtq_buffer *>(handle(env, a.v[0])));
  return undefined(env);
}

// ---- the model step's kernel protocol (src/model/ops.ts:24-31) -------------
// modelSubmit(ctx, [[name, params(8), bindings, x, y], ...]); a binding is
// [buffer handle, null] (device memory), [null, tables handle] or null.
napi_value ModelSubmit(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  uint32_t n = 0;
  NAPI_TRY(env, napi_get_array_length(env, a.v[1], &n));
  std::vector<std::string> names(n);
  std::vector<std::vector<bgtq_binding>> binds(n);
  std::vector<bgtq_model_dispatch> ds(n);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value item, v;
    NAPI_TRY(env, napi_get_element(env, a.v[1], i, &item));
    NAPI_TRY(env, napi_get_element(env, item, 0, &v));
    size_t len = 0;
    NAPI_TRY(env, napi_get_value_string_utf8(env, v, nullptr, 0, &len));
    names[i].resize(len + 1);
    NAPI_TRY(env, napi_get_value_string_utf8(env, v, &names[i][0], len + 1, &len));
    names[i].resize(len);
    bgtq_model_dispatch &d = ds[i];
    d = bgtq_model_dispatch{};
    NAPI_TRY(env, napi_get_element(env, item, 1, &v));
    for (uint32_t k = 0; k < 8; ++k) {
      napi_value e;
      NAPI_TRY(env, napi_get_element(env, v, k, &e));
      d.params[k] = (uint32_t)to_i64(env, e);
    }
    NAPI_TRY(env, napi_get_element(env, item, 2, &v));
    uint32_t nb = 0;
    NAPI_TRY(env, napi_get_array_length(env, v, &nb));
    binds[i].resize(nb);
    for (uint32_t k = 0; k < nb; ++k) {
      napi_value e;
      napi_valuetype t;
      NAPI_TRY(env, napi_get_element(env, v, k, &e));
      NAPI_TRY(env, napi_typeof(env, e, &t));
      bgtq_binding b{};
      if (t == napi_object) {
        napi_value buf, tab;
        napi_valuetype bt, tt;
        NAPI_TRY(env, napi_get_element(env, e, 0, &buf));
        NAPI_TRY(env, napi_get_element(env, e, 1, &tab));
        NAPI_TRY(env, napi_typeof(env, buf, &bt));
        NAPI_TRY(env, napi_typeof(env, tab, &tt));
        if (bt == napi_external) {
          const bgtq_buffer *bb = static_cast<const bgtq_buffer *>(handle(env, buf));
          b.ptr = bgtq_buffer_device_ptr(bb);
          b.bytes = bgtq_buffer_size(bb);
        }
        if (tt == napi_external) b.tables = static_cast<const bgtq_tables *>(handle(env, tab));
      }
      binds[i][k] = b;
    }
    NAPI_TRY(env, napi_get_element(env, item, 3, &v));
    d.x = (uint32_t)to_i64(env, v);
    NAPI_TRY(env, napi_get_element(env, item, 4, &v));
    d.y = (uint32_t)to_i64(env, v);
  }
  for (uint32_t i = 0; i < n; ++i) {
    ds[i].name = names[i].c_str();
    ds[i].bindings = binds[i].data();
    ds[i].n_bindings = binds[i].size();
  }
  BGTQ_TRY(env, bgtq_model_submit(static_cast<bgtq_context *>(handle(env, a.v[0])), ds.data(), ds.size()));
  return undefined(env);
}

// ---- work off the JS thread -------------------------------------------------
// A library call run by napi_async_work on a worker thread: the returned
// Promise resolves once the call (and the device work it waits for) has
// completed, or rejects with the call's RangeError / Error. The thread-local
// error message is taken on the worker thread.
struct AsyncCall {
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  std::function<bgtq_status()> fn;
  std::vector<uint16_t> data;  // a copy of the caller's typed array, owned by the call
  bgtq_status status = BGTQ_OK;
  std::string message;
};

void async_execute(napi_env, void *p) {
  auto *c = static_cast<AsyncCall *>(p);
  c->status = c->fn();
  if (c->status != BGTQ_OK) c->message = bgtq_last_error();
}

void async_complete(napi_env env, napi_status, void *p) {
  auto *c = static_cast<AsyncCall *>(p);
  if (c->status == BGTQ_OK) {
    napi_resolve_deferred(env, c->deferred, undefined(env));
  } else {
    napi_value msg, err;
    napi_create_string_utf8(env, c->message.c_str(), NAPI_AUTO_LENGTH, &msg);
    if (c->status == BGTQ_ERR_RANGE) napi_create_range_error(env, nullptr, msg, &err);
    else napi_create_error(env, nullptr, msg, &err);
    napi_reject_deferred(env, c->deferred, err);
  }
  napi_delete_async_work(env, c->work);
  delete c;
}

napi_value start_async(napi_env env, AsyncCall *c, const char *name) {
  napi_value promise, res;
  if (napi_create_promise(env, &c->deferred, &promise) != napi_ok ||
      napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &res) != napi_ok ||
      napi_create_async_work(env, nullptr, res, async_execute, async_complete, c, &c->work) != napi_ok ||
      napi_queue_async_work(env, c->work) != napi_ok) {
    delete c;
    napi_throw_error(env, nullptr, "could not queue asynchronous work");
    return nullptr;
  }
  return promise;
}

// keysAppendAsync(keys, Uint16Array) -> Promise: PackedKeys/CompressedKeys/FP16Keys.append,
// resolved after the encode has completed (src/runtime/packed-keys.ts:39-49).
napi_value KeysAppendAsync(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  uint16_t *bits;
  size_t n;
  if (!typed(env, a.v[1], napi_uint16_array, &bits, &n)) return nullptr;
  auto *c = new AsyncCall();
  c->data.assign(bits, bits + n);
  bgtq_keys *k = static_cast<bgtq_keys *>(handle(env, a.v[0]));
  c->fn = [c, k]() { return bgtq_keys_append(k, c->data.data(), c->data.size()); };
  return start_async(env, c, "bgtq.keysAppend");
}

// contextSynchronizeAsync(ctx) -> Promise: device.queue.onSubmittedWorkDone().
napi_value ContextSynchronizeAsync(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  auto *c = new AsyncCall();
  bgtq_context *ctx = static_cast<bgtq_context *>(handle(env, a.v[0]));
  c->fn = [ctx]() { return bgtq_context_synchronize(ctx); };
  return start_async(env, c, "bgtq.onSubmittedWorkDone");
}

// keysPrepareDevice(keys): CompressedKeys.prepare's materialisation, queued on the stream.
napi_value KeysPrepareDevice(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  BGTQ_TRY(env, bgtq_keys_prepare(static_cast<bgtq_keys *>(handle(env, a.v[0])), nullptr, 0));
  return undefined(env);
}

// ---- timestamps (GPUQuerySet of type "timestamp") ---------------------------
napi_value TimestampsCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  bgtq_timestamps *t = nullptr;
  BGTQ_TRY(env, bgtq_timestamps_create(static_cast<bgtq_context *>(handle(env, a.v[0])),
                                       (uint32_t)to_i64(env, a.v[1]), &t));
  return wrap(env, t);
}
napi_value TimestampsWrite(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  BGTQ_TRY(env, bgtq_timestamps_write(static_cast<bgtq_timestamps *>(handle(env, a.v[0])),
                                      (uint32_t)to_i64(env, a.v[1])));
  return undefined(env);
}
napi_value TimestampsResolve(napi_env env, napi_callback_info info) {
  // -> BigUint64Array of `count` nanosecond timestamps
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  const uint32_t first = (uint32_t)to_i64(env, a.v[1]), count = (uint32_t)to_i64(env, a.v[2]);
  uint64_t *ns;
  napi_value out = new_typed<uint64_t>(env, napi_biguint64_array, count, &ns);
  if (!out) return nullptr;
  BGTQ_TRY(env, bgtq_timestamps_resolve(static_cast<bgtq_timestamps *>(handle(env, a.v[0])), first, count, ns));
  return out;
}
napi_value TimestampsDestroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bgtq_timestamps_destroy(static_cast<bgtq_timestamps *>(handle(env, a.v[0])));
  return undefined(env);
}

napi_value Init(napi_env env, napi_value exports) {
  struct Fn {
    const char *name;
    napi_callback cb;
  } fns[] = {
      {"contextCreate", ContextCreate},       {"contextDestroy", ContextDestroy},
      {"contextSynchronize", ContextSynchronize}, {"tablesCreate", TablesCreate},
      {"tablesDestroy", TablesDestroy},       {"tablesDeviceBytes", TablesDeviceBytes},
      {"fp16KeysCreate", Fp16KeysCreate},
      {"packedKeysCreate", PackedKeysCreate}, {"keysAppend", KeysAppend},
      {"keysReady", KeysReady},               {"keysLength", KeysLength},
      {"keysRead", KeysRead},                 {"keysReadFp16", KeysReadFp16},
      {"keysPrepare", KeysPrepare},           {"keysAllocations", KeysAllocations},
      {"keysDestroy", KeysDestroy},           {"valuesCreate", ValuesCreate},
      {"valuesAppend", ValuesAppend},         {"valuesLength", ValuesLength},
      {"valuesAllocations", ValuesAllocations}, {"valuesDestroy", ValuesDestroy},
      {"attentionCreate", AttentionCreate},   {"attentionSetQueries", AttentionSetQueries},
      {"attentionRecord", AttentionRecord},   {"attentionRead", AttentionRead},
      {"attentionQueries", AttentionQueries}, {"attentionAllocations", AttentionAllocations},
      {"attentionDestroy", AttentionDestroy}, {"bufferCreate", BufferCreate},
      {"bufferWrite", BufferWrite},           {"bufferRead", BufferRead},
      {"bufferDestroy", BufferDestroy},       {"modelSubmit", ModelSubmit},
      {"allocateBits", AllocateBits},         {"layoutGroups", LayoutGroups},
      {"layoutBuild", LayoutBuild},
      {"keysAppendAsync", KeysAppendAsync},   {"contextSynchronizeAsync", ContextSynchronizeAsync},
      {"keysPrepareDevice", KeysPrepareDevice}, {"timestampsCreate", TimestampsCreate},
      {"timestampsWrite", TimestampsWrite},   {"timestampsResolve", TimestampsResolve},
      {"timestampsDestroy", TimestampsDestroy},
  };
  for (const Fn &f : fns) {
    napi_value fn;
    NAPI_TRY(env, napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn));
    NAPI_TRY(env, napi_set_named_property(env, exports, f.name, fn));
  }
  napi_value version;
  NAPI_TRY(env, napi_create_int32(env, bgtq_abi_version(), &version));
  NAPI_TRY(env, napi_set_named_property(env, exports, "abiVersion", version));
  return exports;
}

}  // namespace

NAPI_MODULE(bgtq_napi, Init)
