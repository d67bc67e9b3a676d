// Host side of the C ABI declared in include/bgtq.h.
//
// Each object validates its inputs with the reference's checks and messages
// before any device work, and mutates its state only after the device work
// it depends on has completed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/bgtq.h"
#include "bgtq_internal.h"

using namespace bgtq;

namespace {

thread_local std::string g_error;

bgtq_status fail(bgtq_status code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

}  // namespace

// The thread's last error, for the library's other host sources.
bgtq_status bgtq::set_error(bgtq_status code, const char *msg) {
  g_error = msg;
  return code;
}

namespace {

bgtq_status hip_fail(hipError_t e, const char *what) {
  return fail(BGTQ_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                   \
  do {                                        \
    hipError_t e_ = (expr);                   \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

// RNE FP32 -> FP16 bits with subnormals and overflow to infinity
// (src/webgpu/half.wgsl:2-12 states the same rule).
uint16_t f32_to_f16(float x) {
  uint32_t b;
  std::memcpy(&b, &x, 4);
  const uint32_t sign = (b >> 16) & 0x8000u, e = (b >> 23) & 0xffu, m = b & 0x7fffffu;
  if (e == 0xffu) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0u));
  const int32_t he = (int32_t)e - 112;
  if (he >= 31) return (uint16_t)(sign | 0x7c00u);
  uint32_t mant = m, shift = 13;
  if (he <= 0) {
    if (he < -10) return (uint16_t)sign;
    mant = m | 0x800000u;
    shift = (uint32_t)(14 - he);
  }
  const uint32_t base = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
  const uint32_t inc = (rem > half || (rem == half && (base & 1u))) ? 1u : 0u;
  return (uint16_t)(sign | ((he > 0 ? (uint32_t)he << 10 : 0u) + base + inc));
}

// FP32 -> FP16 bits rounded toward zero (subnormals kept, overflow to the
// largest finite value), and FP16 bits -> FP32.
uint16_t f32_to_f16_rtz(float x) {
  uint32_t b;
  std::memcpy(&b, &x, 4);
  const uint32_t sign = (b >> 16) & 0x8000u, e = (b >> 23) & 0xffu, m = b & 0x7fffffu;
  const int32_t he = (int32_t)e - 112;
  if (e == 0xffu) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0u));
  if (he >= 31) return (uint16_t)(sign | 0x7bffu);
  if (he <= 0) {
    if (he < -10) return (uint16_t)sign;
    return (uint16_t)(sign | ((m | 0x800000u) >> (14 - he)));
  }
  return (uint16_t)(sign | ((uint32_t)he << 10) | (m >> 13));
}
float f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
  float v;
  if (e == 0) {
    v = std::ldexp((float)m, -24);
    return sign ? -v : v;
  }
  const uint32_t bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
  std::memcpy(&v, &bits, 4);
  return v;
}

struct DeviceBuffer {
  void *ptr = nullptr;
  size_t bytes = 0;
  ~DeviceBuffer() {
    if (ptr) (void)hipFree(ptr);
  }
  bgtq_status alloc(size_t n, const char *what) {
    // Round up to 256 bytes: kernels may read the dword holding a row's last byte.
    const size_t padded = ((n + 16 + 255) / 256) * 256;
    hipError_t e = hipMalloc(&ptr, padded);
    if (e != hipSuccess) {
      ptr = nullptr;
      return fail(BGTQ_ERR_NOMEM, "%s: hipMalloc(%zu) failed: %s", what, padded, hipGetErrorString(e));
    }
    bytes = n;
    e = hipMemset(ptr, 0, padded);  // new buffers start zeroed (src/runtime/compressed-keys.ts:25)
    if (e != hipSuccess) return hip_fail(e, what);
    return BGTQ_OK;
  }
};

struct Ledger {
  std::vector<bgtq_allocation> items;
  void add(const char *name, int32_t role, uint64_t bytes) {
    bgtq_allocation a{};
    std::snprintf(a.name, sizeof(a.name), "%s", name);
    a.role = role;
    a.bytes = bytes;
    items.push_back(a);
  }
  bgtq_status copy(bgtq_allocation *out, size_t cap, size_t *n) const {
    if (n) *n = items.size();
    if (out) std::memcpy(out, items.data(), sizeof(bgtq_allocation) * std::min(cap, items.size()));
    return BGTQ_OK;
  }
};

}  // namespace

struct bgtq_context {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  DeviceBuffer staging;      // per-call upload area, never part of an object's ledger
  std::mutex staging_mutex;  // appends on several threads share the staging area
  // Device job table of the thread-per-row encoders (kEncodeJobTable jobs),
  // written on the stream by launch_encode_upload right before each encode
  // launch; the mutex keeps another thread's upload from landing between the
  // two on the stream.
  DeviceBuffer encode_jobs;
  std::mutex encode_mutex;
  hipEvent_t switch_event = nullptr;  // orders a newly set stream after the previous one
  uint8_t *scratch = nullptr;  // this device's bgtq_decode_noalloc workspace (library-owned array)
  bgtq_status use() {
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    return BGTQ_OK;
  }
  bgtq_status ensure_staging(size_t bytes) {
    if (staging.ptr && staging.bytes >= bytes) return BGTQ_OK;
    HIP_TRY(hipStreamSynchronize(stream), "hipStreamSynchronize");
    if (staging.ptr) {
      (void)hipFree(staging.ptr);
      staging.ptr = nullptr;
      staging.bytes = 0;
    }
    return staging.alloc(std::max<size_t>(bytes, 1 << 20), "upload staging");
  }
};

struct bgtq_tables {
  bgtq_context *ctx = nullptr;
  bgtq_tables_info info{};
  DeviceBuffer blob;
  std::vector<uint8_t> host;  // the DevTables image uploaded to blob
  const DevTables *dev() const { return static_cast<const DevTables *>(blob.ptr); }
  const DevTables *h() const { return reinterpret_cast<const DevTables *>(host.data()); }
};

struct bgtq_keys {
  int32_t kind = 0;
  bgtq_context *ctx = nullptr;
  bgtq_tables *tables = nullptr;
  uint32_t dim = 0, capacity = 0;
  // An append may run on another thread (the Node addon's asynchronous
  // append) while this thread reads the length or checks readiness.
  std::atomic<uint32_t> length{0};
  std::atomic<bool> pending{false};
  DeviceBuffer packed, norms, fp16, decoded;
  Ledger ledger;
};

struct bgtq_values {
  bgtq_context *ctx = nullptr;
  uint32_t dim = 0, capacity = 0, length = 0;
  int32_t dtype = BGTQ_DTYPE_F32;
  DeviceBuffer buf;
  // FP32 V: every appended |v| < 65504, so the fused kernel can split each
  // value into FP16 parts; a larger value sends the store to the general
  // kernels.
  bool fp16_range = true;
  Ledger ledger;
};

struct bgtq_attention {
  bgtq_keys *keys = nullptr;
  bgtq_values *values = nullptr;
  uint32_t max_queries = 0, queries = 0, max_splits = 1;
  int32_t causal = 0, materialize = 0;
  std::vector<uint32_t> positions;
  DeviceBuffer q, qr, out, logits, probs, part, stats, small;  // small: lengths[1] + ends[maxQ]
  DeviceBuffer counters;                                       // split arrival counter (zero between launches)
  uint32_t *pinned = nullptr;                                  // host staging of small
  Ledger ledger;
  ~bgtq_attention() {
    if (pinned) (void)hipHostFree(pinned);
  }
};

extern "C" {

const char *bgtq_last_error(void) { return g_error.c_str(); }
int32_t bgtq_abi_version(void) { return 6; }

// ---------------------------------------------------------------- context
bgtq_status bgtq_context_create(int32_t device, bgtq_context **out) {
  if (!out) return fail(BGTQ_ERR_RANGE, "null output pointer");
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) return fail(BGTQ_ERR_DEVICE, "no HIP device available");
  if (device < 0 || device >= count) return fail(BGTQ_ERR_RANGE, "device %d out of range", device);
  auto *c = new bgtq_context();
  c->device = device;
  if ((e = hipSetDevice(device)) != hipSuccess || (e = hipStreamCreate(&c->own)) != hipSuccess) {
    delete c;
    return hip_fail(e, "context");
  }
  c->stream = c->own;
  if ((e = decode_scratch_setup(device, c->own, &c->scratch)) != hipSuccess) {
    (void)hipStreamDestroy(c->own);
    delete c;
    return hip_fail(e, "decode scratch");
  }
  if (bgtq_status s = c->encode_jobs.alloc(sizeof(EncodeJobDev) * kEncodeJobTable, "encode job table")) {
    (void)hipStreamDestroy(c->own);
    delete c;
    return s;
  }
  if ((e = hipEventCreateWithFlags(&c->switch_event, hipEventDisableTiming)) != hipSuccess) {
    (void)hipStreamDestroy(c->own);
    delete c;
    return hip_fail(e, "context event");
  }
  *out = c;
  return BGTQ_OK;
}

void bgtq_context_destroy(bgtq_context *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->staging.ptr) {
    (void)hipFree(ctx->staging.ptr);
    ctx->staging.ptr = nullptr;
  }
  (void)hipEventDestroy(ctx->switch_event);
  (void)hipStreamDestroy(ctx->own);
  delete ctx;
}

bgtq_status bgtq_context_synchronize(bgtq_context *ctx) {
  if (!ctx) return fail(BGTQ_ERR_RANGE, "null context");
  if (bgtq_status s = ctx->use()) return s;
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  return BGTQ_OK;
}

void *bgtq_context_stream(bgtq_context *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

bgtq_status bgtq_context_set_stream(bgtq_context *ctx, void *hip_stream) {
  if (!ctx) return fail(BGTQ_ERR_RANGE, "null context");
  hipStream_t next = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own;
  if (next == ctx->stream) return BGTQ_OK;
  if (bgtq_status s = ctx->use()) return s;
  // Every call reuses the context's device-side state (the encode job table,
  // the staging area), so work queued on the new stream must not overtake
  // work still queued on the previous one. Outside stream capture an event
  // carries that order; a caller switching streams during capture orders the
  // two captures itself.
  hipStreamCaptureStatus prev_capture = hipStreamCaptureStatusNone, next_capture = hipStreamCaptureStatusNone;
  HIP_TRY(hipStreamIsCapturing(ctx->stream, &prev_capture), "hipStreamIsCapturing");
  HIP_TRY(hipStreamIsCapturing(next, &next_capture), "hipStreamIsCapturing");
  if (prev_capture == hipStreamCaptureStatusNone && next_capture == hipStreamCaptureStatusNone) {
    HIP_TRY(hipEventRecord(ctx->switch_event, ctx->stream), "hipEventRecord");
    HIP_TRY(hipStreamWaitEvent(next, ctx->switch_event, 0), "hipStreamWaitEvent");
  }
  ctx->stream = next;
  return BGTQ_OK;
}

// ---------------------------------------------------------------- timestamps
struct bgtq_timestamps {
  bgtq_context *ctx = nullptr;
  std::vector<hipEvent_t> events;
  std::vector<uint8_t> written;
};

bgtq_status bgtq_timestamps_create(bgtq_context *ctx, uint32_t count, bgtq_timestamps **out) {
  if (!ctx || !out) return fail(BGTQ_ERR_RANGE, "null argument");
  if (count < 1 || count > 4096) return fail(BGTQ_ERR_RANGE, "timestamp count must be 1..4096");
  if (bgtq_status s = ctx->use()) return s;
  auto *t = new bgtq_timestamps();
  t->ctx = ctx;
  t->written.assign(count, 0);
  for (uint32_t i = 0; i < count; ++i) {
    hipEvent_t e = nullptr;
    hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) {
      bgtq_timestamps_destroy(t);
      return hip_fail(err, "timestamp event");
    }
    t->events.push_back(e);
  }
  *out = t;
  return BGTQ_OK;
}

bgtq_status bgtq_timestamps_write(bgtq_timestamps *t, uint32_t index) {
  if (!t) return fail(BGTQ_ERR_RANGE, "null timestamps");
  if (index >= t->events.size()) return fail(BGTQ_ERR_RANGE, "timestamp index %u out of range", index);
  if (bgtq_status s = t->ctx->use()) return s;
  HIP_TRY(hipEventRecord(t->events[index], t->ctx->stream), "timestamp write");
  t->written[index] = 1;
  return BGTQ_OK;
}

bgtq_status bgtq_timestamps_resolve(bgtq_timestamps *t, uint32_t first, uint32_t count, uint64_t *ns) {
  if (!t || (count && !ns)) return fail(BGTQ_ERR_RANGE, "null argument");
  if (first > t->events.size() || count > t->events.size() - first)
    return fail(BGTQ_ERR_RANGE, "timestamp range out of range");
  if (bgtq_status s = t->ctx->use()) return s;
  // Time base: the first written index of the range, placed at 2^40 ns so
  // writes before it stay positive.
  int64_t ref = -1;
  for (uint32_t i = first; i < first + count && ref < 0; ++i)
    if (t->written[i]) ref = i;
  for (uint32_t i = first; i < first + count; ++i) {
    ns[i - first] = 0;
    if (!t->written[i]) continue;
    HIP_TRY(hipEventSynchronize(t->events[i]), "timestamp wait");
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, t->events[ref], t->events[i]), "timestamp resolve");
    ns[i - first] = (uint64_t)((int64_t)1 << 40) + (uint64_t)std::llround((double)ms * 1e6);
  }
  return BGTQ_OK;
}

void bgtq_timestamps_destroy(bgtq_timestamps *t) {
  if (!t) return;
  (void)t->ctx->use();
  for (hipEvent_t e : t->events) (void)hipEventDestroy(e);
  delete t;
}

// ---------------------------------------------------------------- tables
bgtq_status bgtq_tables_create(bgtq_context *ctx, const uint32_t *integer, size_t n_integer,
                               const float *floating, size_t n_floating, bgtq_tables **out) {
  if (!ctx || !out) return fail(BGTQ_ERR_RANGE, "null argument");
  if (!integer || n_integer < 10) return fail(BGTQ_ERR_RANGE, "Invalid Block-GTQ layout");
  // validateLayout (src/webgpu/layout.ts:8-23)
  const int64_t d = integer[0], ng = integer[1], rb = integer[2], nstride = integer[3], nib = integer[4],
                mc = integer[5];
  if (d < 2 || d > 128 || d % 2 || ng < 1 || ng > 8 || nstride < ng || nib < 0 || nib > d || nib % 2 ||
      rb < nib / 2 + d - nib || mc < 2 || mc > 256)
    return fail(BGTQ_ERR_RANGE, "Invalid Block-GTQ layout");
  const uint64_t o_perm = integer[6], o_group = integer[7], o_cb = integer[8], o_lut = integer[9];
  const auto in_range = [&](uint64_t o, uint64_t n) { return o <= n_integer && n <= n_integer - o; };
  if (!in_range(o_perm, d) || !in_range(o_group, d) || !in_range(o_cb, d) || o_lut > n_integer)
    return fail(BGTQ_ERR_RANGE, "Invalid calibration table shape");
  const uint64_t lut_len = n_integer - o_lut;
  const uint32_t *perm = integer + o_perm, *group_of = integer + o_group, *pos_cb = integer + o_cb;
  const uint32_t *lut = integer + o_lut;
  std::vector<int> seen(d, 0);
  bool bad = lut_len % 256 != 0 || lut_len == 0;
  for (int64_t i = 0; i < d && !bad; ++i) {
    if (perm[i] >= d || seen[perm[i]]++) bad = true;
    if (group_of[i] >= ng) bad = true;
    if ((uint64_t)pos_cb[i] * 256 >= lut_len) bad = true;
  }
  if (!floating || n_floating != (size_t)(d * d + d * mc + 2 * d)) bad = true;
  if (bad) return fail(BGTQ_ERR_RANGE, "Invalid calibration table shape");
  for (size_t i = 0; i < n_floating; ++i)
    if (!std::isfinite(floating[i])) return fail(BGTQ_ERR_RANGE, "Nonfinite calibration table");
  for (int64_t i = 0; i < d; ++i)
    for (int bin = 0; bin < 256; ++bin) {
      const uint32_t code = lut[(uint64_t)pos_cb[i] * 256 + bin];
      if (code >= mc || (i < nib && code > 15)) return fail(BGTQ_ERR_RANGE, "Code LUT incompatible with packing");
    }
  const float *rot = floating, *cent = floating + d * d, *off = cent + d * mc, *inv = off + d;
  // PackedKeys constructor checks (src/runtime/packed-keys.ts:16-23).
  int32_t gstart[8], gend[8], gsize[8];
  for (int g = 0; g < 8; ++g) gstart[g] = gend[g] = gsize[g] = 0;
  for (int64_t j = 0; j < d; ++j) {
    int64_t first = -1, last = -1, members = 0;
    for (int64_t i = 0; i < d; ++i)
      if (group_of[i] == group_of[j]) {
        if (first < 0) first = i;
        last = i;
        ++members;
      }
    if (last + 1 - first != members) return fail(BGTQ_ERR_STATE, "Non-contiguous transform group");
    for (int64_t i = 0; i < d; ++i)
      if ((i < first || i > last) && rot[i * d + j] != 0.0f)
        return fail(BGTQ_ERR_STATE, "Off-group transform is nonzero");
    gstart[group_of[j]] = (int32_t)first;
    gend[group_of[j]] = (int32_t)(last + 1);
    gsize[group_of[j]] = (int32_t)members;
  }
  for (int g = 0; g < ng; ++g)
    if (gsize[g] == 0) return fail(BGTQ_ERR_UNSUPPORTED, "group %d has no positions", g);
  // Distinct centroid rows ("books"), as build_code_lut groups positions by signature.
  std::vector<int> pos_book(d);
  std::vector<int64_t> book_rows;
  for (int64_t j = 0; j < d; ++j) {
    int found = -1;
    for (size_t b = 0; b < book_rows.size() && found < 0; ++b)
      if (std::memcmp(cent + book_rows[b] * mc, cent + j * mc, sizeof(float) * mc) == 0) found = (int)b;
    if (found < 0) {
      found = (int)book_rows.size();
      book_rows.push_back(j);
    }
    pos_book[j] = found;
  }
  const int nb = (int)book_rows.size(), ncb = (int)(lut_len / 256);
  if (nb > 255 || ncb > 255) return fail(BGTQ_ERR_UNSUPPORTED, "more than 255 distinct codebooks");
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  const size_t off_lut = align(sizeof(DevTables));
  const size_t off_books = align(off_lut + lut_len);
  const size_t off_rot = align(off_books + sizeof(float) * nb * mc);
  const size_t off_rot_t = align(off_rot + sizeof(float) * d * d);
  const size_t off_mfma = align(off_rot_t + sizeof(float) * d * d);
  const size_t off_rot_q = align(off_mfma + (size_t)kMfmaTableBytes * nb);
  const size_t off_gdesc = align(off_rot_q + (d % 32 == 0 ? (size_t)rot_q_bytes((int)d) : 0));
  const size_t off_glane = align(off_gdesc + sizeof(uint32_t) * d);
  const size_t total = off_glane + (d % 32 == 0 ? sizeof(uint32_t) * kLaneRecordWords * 4 * (d / 32) : 0);
  auto *t = new bgtq_tables();
  t->ctx = ctx;
  t->host.assign(total, 0);
  auto *T = reinterpret_cast<DevTables *>(t->host.data());
  T->dim = (int32_t)d;
  T->groups = (int32_t)ng;
  T->row_bytes = (int32_t)rb;
  T->norm_stride = (int32_t)nstride;
  T->nibble_dims = (int32_t)nib;
  T->max_centroids = (int32_t)mc;
  T->n_books = nb;
  T->n_codebooks = ncb;
  for (int g = 0; g < 8; ++g) {
    T->gstart[g] = gstart[g];
    T->gend[g] = gend[g];
    T->gsize[g] = gsize[g];
  }
  T->off_lut = (uint32_t)off_lut;
  T->off_books = (uint32_t)off_books;
  T->off_rot = (uint32_t)off_rot;
  T->off_rot_t = (uint32_t)off_rot_t;
  T->off_mfma = (uint32_t)off_mfma;
  T->off_rot_q = (uint32_t)off_rot_q;
  T->off_gdesc = (uint32_t)off_gdesc;
  T->off_glane = (uint32_t)off_glane;
  T->total_bytes = (uint32_t)total;
  float cmax = 0.0f;
  for (int64_t i = 0; i < d * mc; ++i) cmax = std::max(cmax, std::fabs(cent[i]));
  T->cent_exp = cmax > 0.0f ? 14 - (int32_t)std::ceil(std::log2(cmax)) : 0;
  for (int64_t j = 0; j < d; ++j) {
    T->perm[j] = (uint8_t)perm[j];
    T->group_of[j] = (uint8_t)group_of[j];
    T->pos_cb[j] = (uint8_t)pos_cb[j];
    T->pos_book[j] = (uint8_t)pos_book[j];
    T->lut_off[j] = off[j];
    T->lut_inv[j] = inv[j];
  }
  uint8_t *h = t->host.data();
  {
    // Per-position rebuild descriptors (src/reference/mixed_layout.py:21-27 row format).
    uint32_t *gd = reinterpret_cast<uint32_t *>(h + off_gdesc);
    for (int64_t j = 0; j < d; ++j) {
      const bool nibble = j < nib;
      const uint32_t off = (uint32_t)(nibble ? j / 2 : nib / 2 + (j - nib));
      gd[j] = off | (uint32_t)(nibble ? 4 * (j & 1) : 0) << 8 | (uint32_t)nibble << 11 | (uint32_t)pos_book[j] << 12 |
              (uint32_t)group_of[j] << 16;
    }
  }
  T->pair_lead = 0;
  T->pair_books = 0xffffffffu;
  if (d % 32 == 0) {
    // The fused decode's per-lane code-lookup records (layout in DevTables).
    const int bspan = std::max(256, (int)(mc * 4 + 255) / 256 * 256) + 32;
    uint32_t *rec = reinterpret_cast<uint32_t *>(h + off_glane);
    auto off_of = [&](int64_t j) { return j < nib ? j / 2 : nib / 2 + (j - nib); };
    // Leading pair K-steps, while their books fit the pair slots.
    std::vector<int> pair_slot_of(nb, -1);
    int n_pair = 0;
    for (int64_t s = 0; s < d / 32; ++s) {
      bool ok = 32 * s + 32 <= nib;
      for (int64_t j = 32 * s; ok && j < 32 * s + 32; j += 2) ok = pos_book[j] == pos_book[j + 1];
      std::vector<int> fresh;
      for (int64_t j = 32 * s; ok && j < 32 * s + 32; j += 2)
        if (pair_slot_of[pos_book[j]] < 0 && std::find(fresh.begin(), fresh.end(), pos_book[j]) == fresh.end())
          fresh.push_back(pos_book[j]);
      if (!ok || n_pair + (int)fresh.size() > kPairSlots) break;
      for (int b : fresh) {
        pair_slot_of[b] = n_pair;
        T->pair_books = (T->pair_books & ~(0xffu << (8 * n_pair))) | (uint32_t)b << (8 * n_pair);
        ++n_pair;
      }
      T->pair_lead = (int32_t)(s + 1);
    }
    for (int64_t s = 0; s < d / 32; ++s)
      for (int gq = 0; gq < 4; ++gq, rec += kLaneRecordWords) {
        const int64_t j0 = 32 * s + 8 * gq;
        const int glo = (int)group_of[32 * s];
        int bo[8], grp[8];
        for (int k = 0; k < 8; ++k) {
          const int64_t j = j0 + k;
          bo[k] = (int)(8 * (off_of(j) - off_of(j0)) + (j < nib ? 4 * (j & 1) : 0));
          grp[k] = (int)group_of[j] - glo;
          rec[12 + k] = (uint32_t)(pos_book[j] * bspan + (j < nib ? 4 : 8));
        }
        const int hib = bo[4] >> 3;
        rec[0] = (uint32_t)off_of(j0);
        rec[1] = (uint32_t)hib;
        rec[2] = (uint32_t)glo;
        rec[3] = (uint32_t)((int)group_of[32 * s + 31] - glo + 1);
        for (int k = 0; k < 8; ++k) rec[4 + k] = (uint32_t)(k < 4 ? bo[k] : bo[k] - 8 * hib);
        for (int i = 0; i < 4; ++i)
          for (int k2 = 0; k2 < 4; ++k2)
            rec[20 + 4 * i + k2] = (grp[2 * k2] == i ? 0x0000ffffu : 0u) | (grp[2 * k2 + 1] == i ? 0xffff0000u : 0u);
        for (int k2 = 0; k2 < 4; ++k2) {
          const int slot = s < T->pair_lead ? pair_slot_of[pos_book[j0 + 2 * k2]] : 0;
          rec[36 + k2] = (uint32_t)(slot * 2048);
          rec[40 + k2] = (uint32_t)(slot * 2048 + 1024);
        }
      }
  }
  for (uint64_t i = 0; i < lut_len; ++i) h[off_lut + i] = (uint8_t)lut[i];
  for (int b = 0; b < nb; ++b)
    std::memcpy(h + off_books + sizeof(float) * b * mc, cent + book_rows[b] * mc, sizeof(float) * mc);
  std::memcpy(h + off_rot, rot, sizeof(float) * d * d);
  float *rot_t = reinterpret_cast<float *>(h + off_rot_t);
  for (int64_t j = 0; j < d; ++j)
    for (int64_t i = 0; i < d; ++i) rot_t[i * d + j] = rot[j * d + i];
  // MFMA lookup tables: c * 2^cent_exp = hi + lo, hi and lo fp16 rounded toward zero.
  const float csc = std::ldexp(1.0f, T->cent_exp);
  for (int b = 0; b < nb; ++b) {
    const float *c = cent + book_rows[b] * mc;
    uint8_t *tb = h + off_mfma + (size_t)kMfmaTableBytes * b;
    uint32_t *pair = reinterpret_cast<uint32_t *>(tb);         // [256][hi pair, lo pair]
    uint32_t *code = reinterpret_cast<uint32_t *>(tb + 2048);  // [256] hi | lo << 16
    auto split = [&](int e, uint16_t *hi, uint16_t *lo) {
      const float x = e < mc ? c[e] * csc : 0.0f;
      *hi = f32_to_f16_rtz(x);
      *lo = f32_to_f16_rtz(x - f16_to_f32(*hi));
    };
    for (int e = 0; e < 256; ++e) {
      uint16_t h0, l0, h1, l1;
      split(e & 15, &h0, &l0);
      split(e >> 4, &h1, &l1);
      pair[2 * e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
      pair[2 * e + 1] = (uint32_t)l0 | ((uint32_t)l1 << 16);
      uint16_t ch, cl;
      split(e, &ch, &cl);
      code[e] = (uint32_t)ch | ((uint32_t)cl << 16);
    }
  }
  // Query rotation operands (prefill): Rq[j][perm[i]] = R[j][i], split like
  // the centroids (entries of an orthogonal rotation lie in [-1, 1]).
  if (d % 32 == 0) {
    std::vector<float> rq((size_t)(d * d));
    for (int64_t j = 0; j < d; ++j)
      for (int64_t i = 0; i < d; ++i) rq[j * d + perm[i]] = rot[j * d + i];
    uint16_t *op = reinterpret_cast<uint16_t *>(h + off_rot_q);
    for (int64_t n = 0; n < d / 16; ++n)
      for (int64_t s = 0; s < d / 32; ++s)
        for (int l = 0; l < 64; ++l) {
          uint16_t *dst = op + ((n * (d / 32) + s) * 64 + l) * 16;
          for (int jv = 0; jv < 8; ++jv) {
            const float x = rq[(16 * n + l % 16) * d + 32 * s + 8 * (l / 16) + jv];
            dst[jv] = f32_to_f16_rtz(x);
            dst[8 + jv] = f32_to_f16_rtz(x - f16_to_f32(dst[jv]));
          }
        }
  }
  t->info = bgtq_tables_info{(int32_t)d, (int32_t)ng, (int32_t)rb, (int32_t)nstride, (int32_t)nib, (int32_t)mc, ncb, nb,
                             (uint64_t)total};
  bgtq_status s = ctx->use();
  if (!s) s = t->blob.alloc(total, "K tables");
  if (!s) {
    hipError_t e = hipMemcpy(t->blob.ptr, h, total, hipMemcpyHostToDevice);
    if (e != hipSuccess) s = hip_fail(e, "upload tables");
  }
  if (s) {
    delete t;
    return s;
  }
  *out = t;
  return BGTQ_OK;
}

bgtq_status bgtq_tables_info_get(const bgtq_tables *t, bgtq_tables_info *out) {
  if (!t || !out) return fail(BGTQ_ERR_RANGE, "null argument");
  *out = t->info;
  return BGTQ_OK;
}

void bgtq_tables_destroy(bgtq_tables *t) {
  if (!t) return;
  (void)t->ctx->use();
  (void)hipStreamSynchronize(t->ctx->stream);
  delete t;
}

// ---------------------------------------------------------------- keys
static bool encode_dim_supported(int d) { return d == 16 || d == 32 || d == 64 || d == 128; }

bgtq_status bgtq_fp16_keys_create(bgtq_context *ctx, uint32_t dim, uint32_t capacity, bgtq_keys **out) {
  if (!ctx || !out) return fail(BGTQ_ERR_RANGE, "null argument");
  if (dim < 2 || dim % 2 || dim > 128 || capacity < 1) return fail(BGTQ_ERR_RANGE, "Invalid K dimensions");
  auto *k = new bgtq_keys();
  k->kind = BGTQ_KEYS_FP16;
  k->ctx = ctx;
  k->dim = dim;
  k->capacity = capacity;
  bgtq_status s = ctx->use();
  if (!s) s = k->fp16.alloc((size_t)capacity * dim * 2, "FP16 K");
  if (s) {
    delete k;
    return s;
  }
  k->ledger.add("FP16 K", BGTQ_ROLE_PERSISTENT_K, (size_t)capacity * dim * 2);
  *out = k;
  return BGTQ_OK;
}

static bgtq_status make_packed(bgtq_tables *t, uint32_t capacity, int32_t kind, bgtq_keys **out) {
  if (!t || !out) return fail(BGTQ_ERR_RANGE, "null argument");
  // The reference bounds capacity by maxComputeWorkgroupsPerDimension (65535,
  // src/runtime/packed-keys.ts:13); HBM is the only bound here.
  if (capacity < 1 || capacity > 0x7fffffffu) return fail(BGTQ_ERR_RANGE, "Invalid capacity");
  if (!encode_dim_supported(t->info.dim))
    return fail(BGTQ_ERR_UNSUPPORTED, "K encode is built for dim 16, 32, 64 and 128 (got %d)", t->info.dim);
  auto *k = new bgtq_keys();
  k->kind = kind;
  k->ctx = t->ctx;
  k->tables = t;
  k->dim = (uint32_t)t->info.dim;
  k->capacity = capacity;
  const size_t pb = (size_t)capacity * t->info.row_bytes, nb = (size_t)capacity * t->info.norm_stride * 2;
  bgtq_status s = t->ctx->use();
  if (!s) s = k->packed.alloc(pb, "K nibble/byte capacity");
  if (!s) s = k->norms.alloc(nb, "K FP16 scale capacity");
  if (!s && kind == BGTQ_KEYS_COMPRESSED) s = k->decoded.alloc((size_t)capacity * k->dim * 4, "materialized FP32 K");
  if (s) {
    delete k;
    return s;
  }
  k->ledger.add("K tables", BGTQ_ROLE_SHARED, t->blob.bytes);
  k->ledger.add("K nibble/byte capacity", BGTQ_ROLE_PERSISTENT_K, pb);
  k->ledger.add("K FP16 scale capacity", BGTQ_ROLE_PERSISTENT_K, nb);
  if (kind == BGTQ_KEYS_COMPRESSED)
    k->ledger.add("materialized FP32 K", BGTQ_ROLE_SCRATCH, (size_t)capacity * k->dim * 4);
  *out = k;
  return BGTQ_OK;
}

bgtq_status bgtq_packed_keys_create(bgtq_tables *t, uint32_t capacity, bgtq_keys **out) {
  return make_packed(t, capacity, BGTQ_KEYS_PACKED, out);
}
bgtq_status bgtq_compressed_keys_create(bgtq_tables *t, uint32_t capacity, bgtq_keys **out) {
  return make_packed(t, capacity, BGTQ_KEYS_COMPRESSED, out);
}

// appendCount (src/runtime/keys.ts:11-15)
static bgtq_status append_count(const uint16_t *v, size_t n, uint32_t dim, uint32_t length, uint32_t capacity,
                                uint32_t *count) {
  if (!n || n % dim || !v) return fail(BGTQ_ERR_RANGE, "K append must contain whole nonempty rows");
  for (size_t i = 0; i < n; ++i)
    if ((v[i] & 0x7c00u) == 0x7c00u) return fail(BGTQ_ERR_RANGE, "Finite FP16 K required");
  const uint64_t c = n / dim;
  if ((uint64_t)length + c > capacity) return fail(BGTQ_ERR_RANGE, "K capacity exceeded");
  *count = (uint32_t)c;
  return BGTQ_OK;
}

// An append first claims the store (pending), so two threads appending at
// once cannot both pass the capacity check on the same length: the loser is
// refused as the reference refuses a second append while one is in flight.
// The length is read once, after the claim, and used for both the capacity
// check and the destination row; it grows before the claim is released.
bgtq_status bgtq_keys_append(bgtq_keys *k, const uint16_t *v, size_t n) {
  if (!k) return fail(BGTQ_ERR_RANGE, "null keys");
  bool idle = false;
  if (!k->pending.compare_exchange_strong(idle, true, std::memory_order_acq_rel))
    return fail(BGTQ_ERR_STATE, "Concurrent K appends unsupported");
  struct Release {
    std::atomic<bool> &flag;
    ~Release() { flag.store(false, std::memory_order_release); }
  } release{k->pending};
  const uint32_t length = k->length.load(std::memory_order_acquire);
  uint32_t count = 0;
  if (bgtq_status s = append_count(v, n, k->dim, length, k->capacity, &count)) return s;
  bgtq_context *ctx = k->ctx;
  if (bgtq_status s = ctx->use()) return s;
  if (k->kind == BGTQ_KEYS_FP16) {
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    HIP_TRY(hipMemcpy(static_cast<uint16_t *>(k->fp16.ptr) + (size_t)length * k->dim, v, n * 2,
                      hipMemcpyHostToDevice),
            "FP16 K upload");
    k->length.store(length + count, std::memory_order_release);
    return BGTQ_OK;
  }
  std::lock_guard<std::mutex> lock(ctx->staging_mutex);
  bgtq_status s = ctx->ensure_staging(n * 2);
  if (!s) {
    hipError_t e = hipMemcpy(ctx->staging.ptr, v, n * 2, hipMemcpyHostToDevice);
    if (e != hipSuccess) s = hip_fail(e, "K append upload");
  }
  if (!s) {
    bgtq_encode_job job{k->tables, ctx->staging.ptr, (int64_t)k->dim, (int64_t)count,
                        static_cast<uint8_t *>(k->packed.ptr), static_cast<uint16_t *>(k->norms.ptr),
                        (int64_t)length};
    s = bgtq_encode_batched(ctx, BGTQ_DTYPE_F16, &job, 1);
  }
  if (!s) {
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) s = hip_fail(e, "K encode");
  }
  if (!s) k->length.store(length + count, std::memory_order_release);  // only after the encode has completed
  return s;
}

bgtq_status bgtq_keys_ready(const bgtq_keys *k) {
  if (!k) return fail(BGTQ_ERR_RANGE, "null keys");
  if (k->pending || !k->length) return fail(BGTQ_ERR_STATE, "K storage not ready");
  return BGTQ_OK;
}
int32_t bgtq_keys_kind(const bgtq_keys *k) { return k ? k->kind : -1; }
uint32_t bgtq_keys_length(const bgtq_keys *k) { return k ? k->length.load() : 0u; }
uint32_t bgtq_keys_capacity(const bgtq_keys *k) { return k ? k->capacity : 0; }
uint32_t bgtq_keys_dim(const bgtq_keys *k) { return k ? k->dim : 0; }

bgtq_status bgtq_keys_read_packed(const bgtq_keys *k, uint8_t *packed, size_t packed_bytes, uint16_t *norms,
                                  size_t norm_count) {
  if (!k || k->kind == BGTQ_KEYS_FP16) return fail(BGTQ_ERR_RANGE, "packed read needs packed keys");
  if (packed_bytes > k->packed.bytes || norm_count * 2 > k->norms.bytes)
    return fail(BGTQ_ERR_RANGE, "Invalid readback length");
  if (bgtq_status s = k->ctx->use()) return s;
  HIP_TRY(hipStreamSynchronize(k->ctx->stream), "hipStreamSynchronize");
  if (packed && packed_bytes) HIP_TRY(hipMemcpy(packed, k->packed.ptr, packed_bytes, hipMemcpyDeviceToHost), "read packed");
  if (norms && norm_count) HIP_TRY(hipMemcpy(norms, k->norms.ptr, norm_count * 2, hipMemcpyDeviceToHost), "read norms");
  return BGTQ_OK;
}

bgtq_status bgtq_keys_read_fp16(const bgtq_keys *k, uint16_t *out, size_t count) {
  if (!k || k->kind != BGTQ_KEYS_FP16 || !out) return fail(BGTQ_ERR_RANGE, "FP16 read needs FP16 keys");
  if (count * 2 > k->fp16.bytes) return fail(BGTQ_ERR_RANGE, "Invalid readback length");
  if (bgtq_status s = k->ctx->use()) return s;
  HIP_TRY(hipStreamSynchronize(k->ctx->stream), "hipStreamSynchronize");
  HIP_TRY(hipMemcpy(out, k->fp16.ptr, count * 2, hipMemcpyDeviceToHost), "read FP16 K");
  return BGTQ_OK;
}

bgtq_status bgtq_keys_prepare(bgtq_keys *k, float *out, size_t count) {
  if (!k || k->kind != BGTQ_KEYS_COMPRESSED) return fail(BGTQ_ERR_RANGE, "prepare needs compressed keys");
  if (k->pending) return fail(BGTQ_ERR_STATE, "K append is still pending");
  if (count > (size_t)k->length * k->dim) return fail(BGTQ_ERR_RANGE, "Invalid readback length");
  if (bgtq_status s = k->ctx->use()) return s;
  if (k->length) {
    HIP_TRY(launch_reconstruct(k->tables->dev(), static_cast<const uint8_t *>(k->packed.ptr),
                               static_cast<const uint16_t *>(k->norms.ptr), k->length,
                               static_cast<float *>(k->decoded.ptr), k->ctx->stream),
            "reconstruct");
  }
  if (out && count) {
    HIP_TRY(hipStreamSynchronize(k->ctx->stream), "hipStreamSynchronize");
    HIP_TRY(hipMemcpy(out, k->decoded.ptr, count * 4, hipMemcpyDeviceToHost), "read decoded K");
  }
  return BGTQ_OK;
}

bgtq_status bgtq_keys_allocations(const bgtq_keys *k, bgtq_allocation *out, size_t cap, size_t *n) {
  if (!k) return fail(BGTQ_ERR_RANGE, "null keys");
  return k->ledger.copy(out, cap, n);
}

void bgtq_keys_destroy(bgtq_keys *k) {
  if (!k) return;
  (void)k->ctx->use();
  (void)hipStreamSynchronize(k->ctx->stream);
  delete k;
}

// ---------------------------------------------------------------- values
bgtq_status bgtq_values_create(bgtq_context *ctx, uint32_t dim, uint32_t capacity, int32_t dtype,
                               bgtq_values **out) {
  if (!ctx || !out) return fail(BGTQ_ERR_RANGE, "null argument");
  if (dim < 1 || dim > 128 || capacity < 1 || (dtype != BGTQ_DTYPE_F32 && dtype != BGTQ_DTYPE_F16))
    return fail(BGTQ_ERR_RANGE, "Invalid V dimensions");
  auto *v = new bgtq_values();
  v->ctx = ctx;
  v->dim = dim;
  v->capacity = capacity;
  v->dtype = dtype;
  const size_t bytes = (size_t)capacity * dim * (dtype == BGTQ_DTYPE_F32 ? 4 : 2);
  bgtq_status s = ctx->use();
  if (!s) s = v->buf.alloc(bytes, "V");
  if (s) {
    delete v;
    return s;
  }
  v->ledger.add(dtype == BGTQ_DTYPE_F32 ? "FP32 V" : "FP16 V", BGTQ_ROLE_PERSISTENT_V, bytes);
  *out = v;
  return BGTQ_OK;
}

bgtq_status bgtq_values_append(bgtq_values *v, const float *values, size_t n) {
  if (!v) return fail(BGTQ_ERR_RANGE, "null values");
  if (!n || n % v->dim || !values) return fail(BGTQ_ERR_RANGE, "V append must contain whole rows");
  for (size_t i = 0; i < n; ++i)
    if (!std::isfinite(values[i])) return fail(BGTQ_ERR_RANGE, "V: finite inputs required");
  const uint64_t count = n / v->dim;
  if (v->length + count > v->capacity) return fail(BGTQ_ERR_RANGE, "V capacity exceeded");
  if (bgtq_status s = v->ctx->use()) return s;
  HIP_TRY(hipStreamSynchronize(v->ctx->stream), "hipStreamSynchronize");
  if (v->dtype == BGTQ_DTYPE_F32) {
    HIP_TRY(hipMemcpy(static_cast<float *>(v->buf.ptr) + (size_t)v->length * v->dim, values, n * 4,
                      hipMemcpyHostToDevice),
            "V upload");
    for (size_t i = 0; i < n; ++i)
      if (std::fabs(values[i]) >= 65504.0f) v->fp16_range = false;
  } else {
    std::vector<uint16_t> h(n);
    for (size_t i = 0; i < n; ++i) h[i] = f32_to_f16(values[i]);
    HIP_TRY(hipMemcpy(static_cast<uint16_t *>(v->buf.ptr) + (size_t)v->length * v->dim, h.data(), n * 2,
                      hipMemcpyHostToDevice),
            "V upload");
  }
  v->length += (uint32_t)count;
  return BGTQ_OK;
}

uint32_t bgtq_values_length(const bgtq_values *v) { return v ? v->length : 0; }
bgtq_status bgtq_values_allocations(const bgtq_values *v, bgtq_allocation *out, size_t cap, size_t *n) {
  if (!v) return fail(BGTQ_ERR_RANGE, "null values");
  return v->ledger.copy(out, cap, n);
}
void bgtq_values_destroy(bgtq_values *v) {
  if (!v) return;
  (void)v->ctx->use();
  (void)hipStreamSynchronize(v->ctx->stream);
  delete v;
}

// Compute units of the current device (cached per device).
static int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Below this many rows per launch the wave-per-row encoder (short latency per
// row) runs; larger launches use a thread-per-row encoder (more rows per
// instruction): the bulk one where the layout qualifies, else the generic one.
constexpr int64_t kEncodeWaveMaxRows = 16384;

// ---------------------------------------------------------------- batched entry points
bgtq_status bgtq_encode_batched(bgtq_context *ctx, int32_t src_dtype, const bgtq_encode_job *jobs, size_t n_jobs) {
  if (!ctx) return fail(BGTQ_ERR_RANGE, "null context");
  if (src_dtype != BGTQ_DTYPE_F16 && src_dtype != BGTQ_DTYPE_F32) return fail(BGTQ_ERR_RANGE, "invalid source dtype");
  if (n_jobs && !jobs) return fail(BGTQ_ERR_RANGE, "null jobs");
  for (size_t i = 0; i < n_jobs; ++i) {
    const bgtq_encode_job &j = jobs[i];
    if (!j.tables) return fail(BGTQ_ERR_RANGE, "encode job %zu: null tables", i);
    if (!encode_dim_supported(j.tables->info.dim))
      return fail(BGTQ_ERR_UNSUPPORTED, "K encode is built for dim 16, 32, 64 and 128 (got %d)", j.tables->info.dim);
    if (j.rows < 0 || j.dst_row0 < 0) return fail(BGTQ_ERR_RANGE, "encode job %zu: negative rows", i);
    if (j.rows && (!j.src || !j.packed || !j.norms)) return fail(BGTQ_ERR_RANGE, "encode job %zu: null buffer", i);
    if (j.src_row_stride < j.tables->info.dim) return fail(BGTQ_ERR_RANGE, "encode job %zu: row stride below dim", i);
    if (j.src_row_stride > INT32_MAX) return fail(BGTQ_ERR_RANGE, "encode job %zu: row stride above 2^31 - 1", i);
  }
  if (bgtq_status s = ctx->use()) return s;
  // Group jobs by dimension and bulk-encoder kind. Few rows in all (a decode
  // step's appended tokens) go to the wave-per-row encoder, its jobs in kernel
  // arguments (kEncodeJobsPerLaunch per launch); otherwise one thread-per-row
  // launch covers up to kEncodeJobTable jobs through the context's job table,
  // so every job's rows share one grid and one round of workgroups.
  std::map<std::pair<int, int>, std::vector<size_t>> by_kind;
  for (size_t i = 0; i < n_jobs; ++i)
    if (jobs[i].rows > 0) {
      const bgtq_tables *t = jobs[i].tables;
      by_kind[{t->info.dim, encode_bulk_kind(t->h())}].push_back(i);
    }
  const bool src_f32 = src_dtype == BGTQ_DTYPE_F32;
  auto job_dev = [&](const bgtq_encode_job &j) {
    EncodeJobDev J{};
    J.t = j.tables->dev();
    J.src = j.src;
    J.src_stride = (int32_t)j.src_row_stride;
    J.rows = j.rows;
    J.packed = j.packed;
    J.norms = j.norms;
    J.dst_row0 = j.dst_row0;
    J.dst_step = 1;
    J.enc_bytes = (int32_t)j.tables->h()->off_rot;
    J.off_rot_t = (int32_t)j.tables->h()->off_rot_t;
    return J;
  };
  for (auto &kv : by_kind) {
    const int dim = kv.first.first, kind = kv.first.second;
    const std::vector<size_t> &idx = kv.second;
    int64_t total_rows = 0;
    int wave_lds = 0;
    for (size_t i : idx) {
      total_rows += jobs[i].rows;
      wave_lds = std::max(wave_lds, encode_wave_lds_bytes(dim, (int)jobs[i].tables->h()->off_rot));
    }
    if (wave_lds <= 160 * 1024 && total_rows < kEncodeWaveMaxRows) {
      for (size_t b = 0; b < idx.size(); b += kEncodeJobsPerLaunch) {
        EncodeLaunch L{};
        int64_t max_rows = 0, rows = 0;
        for (size_t k = b; k < std::min(idx.size(), b + kEncodeJobsPerLaunch); ++k) {
          L.jobs[L.n_jobs++] = job_dev(jobs[idx[k]]);
          max_rows = std::max(max_rows, jobs[idx[k]].rows);
          rows += jobs[idx[k]].rows;
        }
        // One wave per row, each wave striding over enough rows to keep about
        // sixteen waves per compute unit busy.
        const int64_t target_waves = 16 * (int64_t)device_cus();
        const int64_t rows_per_wave = std::max<int64_t>(1, (rows + target_waves - 1) / target_waves);
        const int64_t wgs = std::max<int64_t>(1, (max_rows + 4 * rows_per_wave - 1) / (4 * rows_per_wave));
        HIP_TRY(launch_encode_wave(L, dim, src_f32, (int)std::min<int64_t>(wgs, 65535), wave_lds, ctx->stream),
                "encode launch");
      }
      continue;
    }
    EncodeJobDev *table = static_cast<EncodeJobDev *>(ctx->encode_jobs.ptr);
    std::lock_guard<std::mutex> lock(ctx->encode_mutex);
    for (size_t b = 0; b < idx.size(); b += kEncodeJobTable) {
      const size_t e = std::min(idx.size(), b + kEncodeJobTable);
      int64_t max_rows = 0;
      int lut_max = 0, books_max = 0;
      for (size_t c = b; c < e; c += kEncodeJobsPerLaunch) {
        EncodeLaunch L{};
        for (size_t k = c; k < std::min(e, c + kEncodeJobsPerLaunch); ++k) {
          const bgtq_encode_job &j = jobs[idx[k]];
          L.jobs[L.n_jobs++] = job_dev(j);
          max_rows = std::max(max_rows, j.rows);
          lut_max = std::max(lut_max, j.tables->info.n_codebooks * 256);
          books_max = std::max(books_max, j.tables->info.n_books * j.tables->info.max_centroids);
        }
        HIP_TRY(launch_encode_upload(L, table, (int)(c - b), ctx->stream), "encode job upload");
      }
      const int n = (int)(e - b);
      const int wg = kind == 1 ? 256 : 128;
      if (kind && encode_bulk_lds_bytes(kind, wg, lut_max, books_max) <= 64 * 1024) {
        // Bulk encodes of layout-B-shaped tables: thread per row, structure at compile time.
        HIP_TRY(launch_encode_bulk(table, n, kind, wg, src_f32, max_rows, lut_max, books_max, ctx->stream),
                "encode launch");
      } else {
        HIP_TRY(launch_encode(table, n, dim, src_f32, max_rows, ctx->stream), "encode launch");
      }
    }
  }
  return BGTQ_OK;
}

// Token splits per (sequence, KV head): at least 128 tokens each (one 32-token
// chunk per wave of the fused kernel), at most 256 splits (the fused kernel
// merges them through LDS). By default enough splits for two resident
// workgroups per compute unit: more, shorter-lived workgroups only add
// per-workgroup set-up and merge round trips.
static int choose_splits(int64_t units, uint32_t max_length, int32_t requested) {
  const int64_t max_splits = std::min<int64_t>(256, std::max<int64_t>(1, (max_length + 127) / 128));
  if (requested > 0) return (int)std::min<int64_t>(requested, max_splits);
  const int64_t target = 2 * (int64_t)device_cus();
  const int64_t want = std::max<int64_t>(1, (target + units - 1) / units);
  return (int)std::min<int64_t>(want, max_splits);
}

// Decodes of few (sequence, KV head) units at d=64 on a structured layout or
// FP16 K (at most one four-wave workgroup per compute unit): eight-wave
// workgroups, each split covering twice the tokens (256), so the last
// workgroup of a unit merges half as many partials (C2 step 289 -> 276 us).
// The per-position path (nn < 0) measured slower that way (339 -> 372 us)
// and keeps four. The split count only shrinks, so the workspace sized for
// four waves still holds the partials. Forced split counts keep four waves.
static void choose_waves(DecodeParams &p, int nn) {
  p.waves = 4;
  if (p.dim != 64 || p.splits_forced || nn < 0 || p.v_dtype != BGTQ_DTYPE_F16) return;
  if ((int64_t)p.batch * p.kv_heads * p.splits > device_cus()) return;
  p.waves = 8;
  p.splits = (int)std::min<int64_t>(p.splits, std::max<int64_t>(1, ((int64_t)p.max_length + 255) / 256));
}

struct DecodeWorkspace {
  size_t counters, qr, part, stats, total;
};

// The split counters come first, in a prefix of at least
// BGTQ_DECODE_COUNTER_UNITS counters: every call with at most that many
// (sequence, KV head) units writes its rotated queries and partials past it,
// so calls of any such geometries can share a workspace in any order and its
// counters stay zero.
static DecodeWorkspace decode_ws(int64_t units, int64_t heads, int dim, int splits) {
  auto al = [](size_t x) { return (x + 255) & ~size_t(255); };
  DecodeWorkspace w;
  w.counters = 0;
  w.qr = al(sizeof(uint32_t) * kCounterStride * std::max<int64_t>(units, BGTQ_DECODE_COUNTER_UNITS));
  w.part = w.qr + al(sizeof(float) * heads * dim);
  // Partials of the splits and of a decode-step append's token (one more per head).
  w.stats = w.part + al(sizeof(float) * heads * (splits + 1) * (dim + 2));
  w.total = w.stats + al(sizeof(float) * heads * 2);
  return w;
}

static bgtq_status validate_decode(const bgtq_decode_desc *d, int *splits) {
  if (!d) return fail(BGTQ_ERR_RANGE, "null descriptor");
  if (d->batch < 1 || d->kv_heads < 1 || d->kv_heads > kMaxKvHeads || d->q_heads < d->kv_heads ||
      d->q_heads % d->kv_heads || d->q_heads / d->kv_heads > 16)
    return fail(BGTQ_ERR_RANGE, "invalid head geometry");
  if (d->batch > 65535) return fail(BGTQ_ERR_UNSUPPORTED, "decode handles up to 65535 sequences per call");
  if (d->dim < 2 || d->dim > 128 || d->dim % 2) return fail(BGTQ_ERR_RANGE, "invalid head dim");
  if (d->max_length < 1 || d->max_length > (1u << 24)) return fail(BGTQ_ERR_RANGE, "max_length must be in 1..2^24");
  if (d->key_format == BGTQ_KEYS_PACKED) {
    for (int h = 0; h < d->kv_heads; ++h) {
      if (!d->tables[h]) return fail(BGTQ_ERR_RANGE, "null tables for KV head %d", h);
      if (d->tables[h]->info.dim != d->dim) return fail(BGTQ_ERR_RANGE, "tables dim mismatch");
    }
    if (!d->packed || !d->norms) return fail(BGTQ_ERR_RANGE, "null packed K");
  } else if (d->key_format == BGTQ_KEYS_FP16) {
    if (!d->k_f16) return fail(BGTQ_ERR_RANGE, "null FP16 K");
  } else {
    return fail(BGTQ_ERR_RANGE, "invalid key format");
  }
  if (!d->v || (d->v_dtype != BGTQ_DTYPE_F16 && d->v_dtype != BGTQ_DTYPE_F32)) return fail(BGTQ_ERR_RANGE, "invalid V");
  if (!d->q || !d->out || !d->lengths) return fail(BGTQ_ERR_RANGE, "null q/out/lengths");
  if (d->q_rotated != 0 && d->q_rotated != 1) return fail(BGTQ_ERR_RANGE, "q_rotated must be 0 or 1");
  if (d->q_rotated && d->key_format != BGTQ_KEYS_PACKED) return fail(BGTQ_ERR_RANGE, "q_rotated needs packed K");
  *splits = choose_splits((int64_t)d->batch * d->kv_heads, d->max_length, d->splits);
  return BGTQ_OK;
}

bgtq_status bgtq_decode_workspace_size(const bgtq_decode_desc *d, size_t *bytes) {
  int splits = 1;
  if (bgtq_status s = validate_decode(d, &splits)) return s;
  if (!bytes) return fail(BGTQ_ERR_RANGE, "null output");
  *bytes = decode_ws((int64_t)d->batch * d->kv_heads, (int64_t)d->batch * d->q_heads, d->dim, splits).total;
  return BGTQ_OK;
}

// Whether the fused kernel reads p's V: FP16 rows, or FP32 rows known to
// lie within FP16's range in a decode without an appended token; 16-byte
// aligned base and strides.
static bool fused_v(const DecodeParams &p) {
  const bool f32 = p.v_dtype == BGTQ_DTYPE_F32;
  if (f32 ? !p.v_f32_split || p.k_new || p.starts : p.v_dtype != BGTQ_DTYPE_F16) return false;
  const int64_t vb = f32 ? 4 : 2;
  return (reinterpret_cast<uintptr_t>(p.v) & 15) == 0 && (p.v_seq_stride * vb) % 16 == 0 &&
         (p.v_head_stride * vb) % 16 == 0;
}

// Whether the fused matrix-core kernel handles this launch (FastLayout in
// bgtq_internal.h); on success fills the K-step books, nn and sg.
static bool fast_layout(const DecodeParams &p, const bgtq_tables *const *tables, FastLayout *fl, int *nn, int *sg) {
  auto a16 = [](const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  if (!fused_v(p) || (p.dim != 64 && p.dim != 128) || p.G > 16) return false;
  const int ks = p.dim / 32;
  if (p.key_format == 0) {
    *nn = 0;
    *sg = ks;
    return a16(p.k) && (p.k_seq_stride * 2) % 16 == 0 && (p.k_head_stride * 2) % 16 == 0;
  }
  if (p.key_format != 1) return false;
  if ((reinterpret_cast<uintptr_t>(p.packed) & 7) || p.packed_seq_stride % 8 || p.packed_head_stride % 8) return false;
  if (!a16(p.norms) || (p.norms_seq_stride * 2) % 16 || (p.norms_head_stride * 2) % 16) return false;
  for (int h = 0; h < p.kv_heads; ++h) {
    const DevTables *T = tables[h]->h();
    if (T->row_bytes % 8 || T->norm_stride != 2 || T->groups > 2 || T->nibble_dims % 32) return false;
    const int n = T->nibble_dims / 32;
    if (T->row_bytes != decode_fast_row_bytes(p.dim, n)) return false;
    if (p.k_new && (int64_t)T->off_rot > decode_fast_enc_capacity(p.dim, n)) return false;
    int g0 = 0;
    for (int s = 0; s < ks; ++s) {
      const int g = T->group_of[32 * s], bk = T->pos_book[32 * s];
      for (int j = 32 * s; j < 32 * s + 32; ++j)
        if (T->group_of[j] != g || T->pos_book[j] != bk) return false;
      if (g == 0) {
        if (g0 != s) return false;  // group 0 steps first
        ++g0;
      }
      if (h == 0) fl->book[s] = bk;
      else if (fl->book[s] != bk) return false;
    }
    const uint8_t *base = reinterpret_cast<const uint8_t *>(tables[h]->dev());
    fl->mfma[h] = base + T->off_mfma;
    fl->rot_q[h] = base + T->off_rot_q;
    fl->rot_t[h] = reinterpret_cast<const float *>(base + T->off_rot_t);
    fl->enc_bytes[h] = (int32_t)T->off_rot;  // header, LUT, books
    fl->cent_exp[h] = T->cent_exp;
    const int sgv = T->groups == 1 ? ks : g0;
    if (h == 0) {
      *nn = n;
      *sg = sgv;
    } else if (*nn != n || *sg != sgv) {
      return false;
    }
  }
  return decode_fast_supported(p.dim, 1, *nn, *sg);
}

// Whether the fused kernel's per-position code lookup serves a packed layout
// the structured check (fast_layout) refused: FP16 V; 16-byte aligned packed
// and scale bases and strides; per KV head up to 8 books of up to 256
// centroids whose code tables fit the kernel's LDS, each book's positions
// all nibble or all byte codes, norm stride up to 8, groups in ascending
// position order with at most four in any 32 positions. Fills the per-head
// fields of fl.
static bool general_layout(const DecodeParams &p, const bgtq_tables *const *tables, FastLayout *fl) {
  auto a16 = [](const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  if (p.key_format != 1 || !fused_v(p) || (p.dim != 64 && p.dim != 128) || p.G > 16) return false;
  if (!a16(p.packed) || p.packed_seq_stride % 16 || p.packed_head_stride % 16) return false;
  if (!a16(p.norms) || (p.norms_seq_stride * 2) % 16 || (p.norms_head_stride * 2) % 16) return false;
  for (int h = 0; h < p.kv_heads; ++h) {
    const DevTables *T = tables[h]->h();
    const int bstride = std::max(256, (T->max_centroids * 4 + 255) / 256 * 256);
    if (T->n_books > 8 || T->max_centroids > 256 || T->n_books * (bstride + 32) > decode_general_table_bytes(p.dim) ||
        T->norm_stride > decode_general_max_norm_stride(p.dim) || T->row_bytes > p.dim || T->groups > 8)
      return false;
    for (int j = 1; j < p.dim; ++j)
      if (T->group_of[j] < T->group_of[j - 1] || T->group_of[j] > T->group_of[j - 1] + 1) return false;
    for (int s = 0; s < p.dim / 32; ++s)
      if (T->group_of[32 * s + 31] >= T->group_of[32 * s] + kDecodeGeneralMaxGroupsPerStep) return false;
    uint32_t nib_books = 0, byte_books = 0;
    for (int j = 0; j < p.dim; ++j) (j < T->nibble_dims ? nib_books : byte_books) |= 1u << T->pos_book[j];
    if (nib_books & byte_books) return false;
    const uint8_t *base = reinterpret_cast<const uint8_t *>(tables[h]->dev());
    fl->rot_q[h] = base + T->off_rot_q;
    fl->rot_t[h] = reinterpret_cast<const float *>(base + T->off_rot_t);
    // The append's encoder reads an LDS copy of the header, LUT and books
    // when they fit a ring slot, else of the LUT and books (the header in
    // device memory), else (0) the tables in device memory.
    const int64_t cap = decode_fast_enc_capacity(p.dim, -1);
    fl->enc_from[h] = 0;
    fl->enc_bytes[h] = 0;
    if ((int64_t)T->off_rot <= cap) {
      fl->enc_bytes[h] = (int32_t)T->off_rot;
    } else if ((int64_t)(T->off_rot - T->off_lut) <= cap) {
      fl->enc_from[h] = (int32_t)T->off_lut;
      fl->enc_bytes[h] = (int32_t)(T->off_rot - T->off_lut);
    }
    fl->cent_exp[h] = T->cent_exp;
    fl->mfma[h] = base + T->off_mfma;
    fl->gdesc[h] = reinterpret_cast<const uint32_t *>(base + T->off_gdesc);
    fl->glane[h] = reinterpret_cast<const uint32_t *>(base + T->off_glane);
    fl->grb[h] = (int16_t)T->row_bytes;
    fl->gns[h] = (int16_t)T->norm_stride;
    fl->gnb[h] = (int16_t)T->n_books;
    fl->gbstride[h] = (int16_t)bstride;
    fl->gbnib[h] = (uint8_t)nib_books;
    fl->galign[h] = T->row_bytes % 4 == 0 && T->nibble_dims % 8 == 0;
    fl->gpair[h] = T->pair_books;
    fl->gpair_lead = h == 0 ? T->pair_lead : std::min(fl->gpair_lead, T->pair_lead);
  }
  return true;
}

static bgtq_status launch_decode_common(bgtq_context *ctx, DecodeParams &p, const float *q,
                                        const bgtq_tables *const *tables) {
  p.q = q;
  FastLayout fl{};
  int nn = 0, sg = 0;
  bool fused = p.counters && fast_layout(p, tables, &fl, &nn, &sg);
  if (p.counters && !fused && general_layout(p, tables, &fl)) {
    nn = -1;
    fused = true;
  }
  if (fused) {
    if (!p.starts) choose_waves(p, nn);
    HIP_TRY(launch_decode_fast(p, fl, nn, sg, ctx->stream), "decode launch");
    if (p.probs) HIP_TRY(launch_decode_probs(p, ctx->stream), "probabilities launch");
    return BGTQ_OK;
  }
  int lds = 0;
  for (int h = 0; h < (p.key_format == 1 ? p.kv_heads : 1); ++h) {
    const bgtq_tables_info *ti = p.key_format == 1 ? &tables[h]->info : nullptr;
    const int books = ti ? ti->n_books * ti->max_centroids * 4 : 0;
    lds = std::max(lds, decode_lds_bytes(p.G, p.dim, p.key_format, books, ti ? ti->row_bytes : 0,
                                         ti ? ti->norm_stride : 0));
  }
  if (lds > 65536) return fail(BGTQ_ERR_UNSUPPORTED, "decode needs %d bytes of LDS (limit 65536)", lds);
  HIP_TRY(launch_rotate_q(p, q, const_cast<float *>(p.qr), ctx->stream), "rotate_q launch");
  HIP_TRY(launch_decode(p, lds, ctx->stream), "decode launch");
  return BGTQ_OK;
}

static bgtq_status decode_impl(bgtq_context *ctx, const bgtq_decode_desc *d, const bgtq_append_desc *a);

bgtq_status bgtq_decode(bgtq_context *ctx, const bgtq_decode_desc *d) { return decode_impl(ctx, d, nullptr); }

bgtq_status bgtq_decode_append(bgtq_context *ctx, const bgtq_decode_desc *d, const bgtq_append_desc *a) {
  if (!a) return fail(BGTQ_ERR_RANGE, "null append descriptor");
  if (!a->k_new || !a->v_new) return fail(BGTQ_ERR_RANGE, "null new K or V");
  for (int32_t t : {a->k_new_dtype, a->v_new_dtype})
    if (t != BGTQ_DTYPE_F16 && t != BGTQ_DTYPE_F32) return fail(BGTQ_ERR_RANGE, "invalid new K/V dtype");
  if (d && (a->k_new_seq_stride < 0 || a->k_new_head_stride < 0 || a->v_new_seq_stride < 0 || a->v_new_head_stride < 0))
    return fail(BGTQ_ERR_RANGE, "negative new K/V stride");
  // The kernel reads the new rows as 4-byte words.
  if (reinterpret_cast<uintptr_t>(a->k_new) % 4 || reinterpret_cast<uintptr_t>(a->v_new) % 4)
    return fail(BGTQ_ERR_RANGE, "new K and V must be 4-byte aligned");
  if ((a->k_new_dtype == BGTQ_DTYPE_F16 && (a->k_new_seq_stride % 2 || a->k_new_head_stride % 2)) ||
      (a->v_new_dtype == BGTQ_DTYPE_F16 && (a->v_new_seq_stride % 2 || a->v_new_head_stride % 2)))
    return fail(BGTQ_ERR_RANGE, "FP16 new K/V strides must be even");
  return decode_impl(ctx, d, a);
}

bgtq_status bgtq_decode_noalloc(bgtq_context *ctx, const bgtq_decode_desc *d) {
  if (!ctx) return fail(BGTQ_ERR_RANGE, "null context");
  int splits = 1;
  if (bgtq_status s = validate_decode(d, &splits)) return s;
  if ((int64_t)d->batch * d->kv_heads > BGTQ_DECODE_COUNTER_UNITS)
    return fail(BGTQ_ERR_RANGE, "bgtq_decode_noalloc takes up to %d (sequence, KV head) pairs per call",
                BGTQ_DECODE_COUNTER_UNITS);
  const size_t need = decode_ws((int64_t)d->batch * d->kv_heads, (int64_t)d->batch * d->q_heads, d->dim, splits).total;
  if (need > BGTQ_DECODE_SCRATCH_BYTES)
    return fail(BGTQ_ERR_RANGE, "decode needs %zu bytes of workspace, above the %u-byte scratch of bgtq_decode_noalloc",
                need, (unsigned)BGTQ_DECODE_SCRATCH_BYTES);
  bgtq_decode_desc own = *d;
  own.workspace = ctx->scratch;
  own.workspace_bytes = BGTQ_DECODE_SCRATCH_BYTES;
  return decode_impl(ctx, &own, nullptr);
}

static bgtq_status decode_impl(bgtq_context *ctx, const bgtq_decode_desc *d, const bgtq_append_desc *a) {
  if (!ctx) return fail(BGTQ_ERR_RANGE, "null context");
  int splits = 1;
  if (bgtq_status s = validate_decode(d, &splits)) return s;
  const int64_t heads = (int64_t)d->batch * d->q_heads;
  const DecodeWorkspace w = decode_ws((int64_t)d->batch * d->kv_heads, heads, d->dim, splits);
  if (!d->workspace || d->workspace_bytes < w.total)
    return fail(BGTQ_ERR_RANGE, "workspace of %zu bytes required", w.total);
  if (bgtq_status s = ctx->use()) return s;
  DecodeParams p{};
  for (int h = 0; h < d->kv_heads; ++h) p.tables[h] = d->key_format == BGTQ_KEYS_PACKED ? d->tables[h]->dev() : nullptr;
  p.batch = d->batch;
  p.q_heads = d->q_heads;
  p.kv_heads = d->kv_heads;
  p.dim = d->dim;
  p.G = d->q_heads / d->kv_heads;
  p.key_format = d->key_format == BGTQ_KEYS_PACKED ? 1 : 0;
  p.packed = d->packed;
  p.packed_seq_stride = d->packed_seq_stride;
  p.packed_head_stride = d->packed_head_stride;
  p.norms = d->norms;
  p.norms_seq_stride = d->norms_seq_stride;
  p.norms_head_stride = d->norms_head_stride;
  p.k = d->k_f16;
  p.k_seq_stride = d->k_seq_stride;
  p.k_head_stride = d->k_head_stride;
  p.v = d->v;
  p.v_dtype = d->v_dtype;
  p.v_seq_stride = d->v_seq_stride;
  p.v_head_stride = d->v_head_stride;
  uint8_t *ws = static_cast<uint8_t *>(d->workspace);
  p.counters = reinterpret_cast<uint32_t *>(ws + w.counters);
  p.counter_stride = kCounterStride;
  p.qr = reinterpret_cast<float *>(ws + w.qr);
  p.part = reinterpret_cast<float *>(ws + w.part);
  p.stats = reinterpret_cast<float *>(ws + w.stats);
  p.lengths = d->lengths;
  p.q_rotated = d->q_rotated;
  p.max_length = (int32_t)d->max_length;
  p.ends = nullptr;
  p.splits = splits;
  p.splits_forced = d->splits > 0;
  p.split_tokens = (int)((d->max_length + p.splits - 1) / p.splits);
  p.split_tokens = ((p.split_tokens + 127) / 128) * 128;
  p.inv_sqrt_d = (float)(1.0 / std::sqrt((double)d->dim));
  p.out = d->out;
  p.logits = nullptr;
  p.probs = nullptr;
  p.logit_stride = 0;
  if (a) {
    p.k_new = a->k_new;
    p.k_new_f32 = a->k_new_dtype == BGTQ_DTYPE_F32;
    p.k_new_seq_stride = a->k_new_seq_stride;
    p.k_new_head_stride = a->k_new_head_stride;
    p.v_new = a->v_new;
    p.v_new_f32 = a->v_new_dtype == BGTQ_DTYPE_F32;
    p.v_new_seq_stride = a->v_new_seq_stride;
    p.v_new_head_stride = a->v_new_head_stride;
    p.app_parts = 1;  // packed K: one append workgroup per (sequence, KV head)
    FastLayout fl{};
    int nn = 0, sg = 0;
    p.q = d->q;
    bool fused = fast_layout(p, d->tables, &fl, &nn, &sg);
    if (!fused && general_layout(p, d->tables, &fl)) {
      nn = -1;
      fused = true;
    }
    if (!fused)
      return fail(BGTQ_ERR_UNSUPPORTED,
                  "decode_append needs the fused kernel's layouts; use bgtq_encode_batched and bgtq_decode");
    choose_waves(p, nn);
    HIP_TRY(launch_decode_fast(p, fl, nn, sg, ctx->stream), "decode append launch");
    return BGTQ_OK;
  }
  return launch_decode_common(ctx, p, d->q, d->tables);
}

// ---------------------------------------------------------------- chunked prefill
struct PrefillPlan {
  int tiles, tile_queries, ranges, range_blocks;
  size_t records;    // bytes of the workgroups' partial records
  size_t workspace;  // records, then the tile table (16 bytes per tile)
  bool rowwise;      // the fused decode kernel, units of 16 (row, head) query columns
  int qgroups;       // rowwise: units per (sequence, KV head)
  int unit_cols;     // rowwise: query columns per unit
  int splits;        // rowwise: token splits per unit (a unit uses those its history needs)
  int split_floor;   // rowwise: tokens per split at least
  int app_parts;     // rowwise with appended rows: their workgroups per unit (one row per wave)
  size_t counters, part;  // rowwise: workspace offsets (the split counters first)
};

// Query tiles: four waves of one 16-query block each for small chunks (more
// tiles to spread), of prefill_column_blocks(dim) blocks each for long ones
// (the K operand rebuilt once per block serves more queries). Workgroups:
// the flattened work (every KV head, sequence and tile's causal history in
// 32-token blocks) is cut into equal ranges, about two workgroups per
// compute unit, sized here for the most work (every chunk at the end of the
// cache: the starts are device values) and by the kernel for the actual one;
// split_tokens > 0 fixes the range length instead.
// append: the chunk's rows are appended in the same launch (bgtq_prefill_append).
static bgtq_status plan_prefill(const bgtq_prefill_desc *d, PrefillPlan *plan, bool append = false) {
  if (!d) return fail(BGTQ_ERR_RANGE, "null descriptor");
  if (d->batch < 1 || d->rows < 1 || d->kv_heads < 1 || d->kv_heads > kMaxKvHeads || d->q_heads < d->kv_heads ||
      d->q_heads % d->kv_heads || d->q_heads / d->kv_heads > 16)
    return fail(BGTQ_ERR_RANGE, "invalid head geometry");
  if (d->dim != 64 && d->dim != 128) return fail(BGTQ_ERR_UNSUPPORTED, "prefill handles head dim 64 or 128");
  if (d->max_length < 1 || d->max_length > (1u << 24)) return fail(BGTQ_ERR_RANGE, "max_length must be in 1..2^24");
  if ((uint32_t)d->rows > d->max_length) return fail(BGTQ_ERR_RANGE, "rows exceed max_length");
  if (d->key_format == BGTQ_KEYS_PACKED) {
    for (int h = 0; h < d->kv_heads; ++h) {
      if (!d->tables[h]) return fail(BGTQ_ERR_RANGE, "null tables for KV head %d", h);
      if (d->tables[h]->info.dim != d->dim) return fail(BGTQ_ERR_RANGE, "tables dim mismatch");
    }
    if (!d->packed || !d->norms) return fail(BGTQ_ERR_RANGE, "null packed K");
  } else if (d->key_format == BGTQ_KEYS_FP16) {
    if (!d->k_f16) return fail(BGTQ_ERR_RANGE, "null FP16 K");
  } else {
    return fail(BGTQ_ERR_RANGE, "invalid key format");
  }
  if (!d->v || !d->q || !d->out || !d->starts) return fail(BGTQ_ERR_RANGE, "null v/q/out/starts");
  if (d->q_rotated != 0 && d->q_rotated != 1) return fail(BGTQ_ERR_RANGE, "q_rotated must be 0 or 1");
  if (d->q_rotated && d->key_format != BGTQ_KEYS_PACKED) return fail(BGTQ_ERR_RANGE, "q_rotated needs packed K");
  if (d->split_tokens < 0) return fail(BGTQ_ERR_RANGE, "negative split_tokens");
  if ((int64_t)d->batch * d->kv_heads > 65535) return fail(BGTQ_ERR_UNSUPPORTED, "prefill handles up to 65535 sequence x KV head units");
  const int64_t G = d->q_heads / d->kv_heads, nq = (int64_t)d->rows * G;
  const int64_t uc = kPrefillUnitCols, qgroups = (nq + uc - 1) / uc;
  const int64_t row_units = (int64_t)d->batch * qgroups * d->kv_heads;
  plan->rowwise = d->rows <= kPrefillRowwiseRows && (int64_t)d->batch * qgroups <= 65535;
  if (plan->rowwise) {
    // Splits of at least split_floor tokens (two 32-token chunks per wave
    // by default: below that a split merge costs more than the chunks it
    // saves), as many as the longest history allowed needs, at most enough
    // for the workgroups a compute unit holds (two of four waves, one of
    // eight) and kPrefillMaxSplits.
    const int64_t floor_tok = d->split_tokens > 0 ? d->split_tokens : prefill_split_floor(d->dim);
    const int64_t per_cu = decode_fast_prefill_waves(d->dim) == 8 ? 1 : 2;
    int64_t splits = ((int64_t)d->max_length + floor_tok - 1) / floor_tok;
    if (d->split_tokens <= 0)
      splits = std::min<int64_t>(splits, std::max<int64_t>(1, per_cu * (int64_t)device_cus() / row_units));
    // Appended rows: one more workgroup per unit for every
    // kPrefillAppendRowsPerWave rows per wave, each leaving a partial; the
    // merge takes up to kPrefillMaxSplits.
    const int per_wg = decode_fast_prefill_waves(d->dim) * kPrefillAppendRowsPerWave;
    const int app_max = (d->rows + per_wg - 1) / per_wg;
    plan->app_parts = append ? app_max : 0;
    // With appended rows the history splits leave room for their workgroups
    // in the same round of compute units.
    if (append && d->split_tokens <= 0)
      splits = std::min<int64_t>(splits, std::max<int64_t>(1, per_cu * (int64_t)device_cus() / row_units - app_max));
    plan->qgroups = (int)qgroups;
    plan->unit_cols = (int)uc;
    plan->splits = (int)std::max<int64_t>(1, std::min<int64_t>(splits, kPrefillMaxSplits - plan->app_parts));
    plan->split_floor = (int)std::max<int64_t>(floor_tok, ((int64_t)d->max_length + plan->splits - 1) / plan->splits);
    plan->counters = 0;
    plan->part = kPrefillCounterBytes;
    // Partial rows o[dim], m, l, pad: the splits' and, whichever entry point
    // takes the workspace, the appended rows' workgroups'.
    const int64_t splits_plain = std::max<int64_t>(1, std::min<int64_t>(splits, kPrefillMaxSplits));
    plan->workspace =
        kPrefillCounterBytes + sizeof(float) * (size_t)row_units * uc * (splits_plain + app_max) * (d->dim + 4);
    return BGTQ_OK;
  }
  plan->tile_queries = nq >= 2048 ? 64 * prefill_column_blocks(d->dim) : 64;
  plan->tiles = (int)((nq + plan->tile_queries - 1) / plan->tile_queries);
  if ((int64_t)d->batch * plan->tiles > INT32_MAX / 2) return fail(BGTQ_ERR_UNSUPPORTED, "too many query tiles");
  // The most work (in the kernel's cost units: a segment's set-up plus 32-token blocks of every tile's
  // history) with each chunk at the end of the cache.
  const int64_t start = (int64_t)d->max_length - d->rows, tq = plan->tile_queries;
  int64_t w1 = 0;
  for (int64_t t = 0; t < plan->tiles; ++t)
    w1 += kPrefillSegmentCost + (start + (std::min(nq, (t + 1) * tq) - 1) / G + 1 + 31) / 32;
  const int64_t w_max = w1 * d->batch * d->kv_heads;
  if (w_max > INT32_MAX / 2) return fail(BGTQ_ERR_UNSUPPORTED, "prefill work above 2^30 blocks of 32 tokens");
  int64_t ranges, range_blocks = 0;
  if (d->split_tokens > 0) {
    range_blocks = (d->split_tokens + 31) / 32;
    ranges = (w_max + range_blocks - 1) / range_blocks;
    if (ranges > kPrefillMaxRanges) {
      ranges = kPrefillMaxRanges;
      range_blocks = (w_max + ranges - 1) / ranges;
    }
  } else {
    ranges = std::min<int64_t>(2 * (int64_t)device_cus(), (w_max + kPrefillMinRange - 1) / kPrefillMinRange);
  }
  plan->ranges = (int)std::max<int64_t>(1, ranges);
  plan->range_blocks = (int)range_blocks;
  plan->records = plan->ranges > 1 ? sizeof(float) * (size_t)plan->ranges * 2 * tq * (d->dim + 2) : 0;
  const size_t info = plan->ranges > 1 ? 16 * (size_t)d->batch * d->kv_heads * plan->tiles : 0;
  plan->workspace = kPrefillCounterBytes + plan->records + info;
  return BGTQ_OK;
}

bgtq_status bgtq_prefill_workspace_size(const bgtq_prefill_desc *d, size_t *bytes) {
  PrefillPlan plan{};
  if (bgtq_status s = plan_prefill(d, &plan)) return s;
  if (!bytes) return fail(BGTQ_ERR_RANGE, "null output");
  *bytes = std::max<size_t>(plan.workspace, 256);
  return BGTQ_OK;
}

static bgtq_status prefill_impl(bgtq_context *ctx, const bgtq_prefill_desc *d, const bgtq_prefill_append_desc *a);

bgtq_status bgtq_prefill(bgtq_context *ctx, const bgtq_prefill_desc *d) { return prefill_impl(ctx, d, nullptr); }

bgtq_status bgtq_prefill_append(bgtq_context *ctx, const bgtq_prefill_desc *d, const bgtq_prefill_append_desc *a) {
  if (!a) return fail(BGTQ_ERR_RANGE, "null append descriptor");
  if (!a->k_new || !a->v_new) return fail(BGTQ_ERR_RANGE, "null new K or V");
  for (int32_t t : {a->k_new_dtype, a->v_new_dtype})
    if (t != BGTQ_DTYPE_F16 && t != BGTQ_DTYPE_F32) return fail(BGTQ_ERR_RANGE, "invalid new K/V dtype");
  if (a->k_new_seq_stride < 0 || a->k_new_row_stride < 0 || a->k_new_head_stride < 0 || a->v_new_seq_stride < 0 ||
      a->v_new_row_stride < 0 || a->v_new_head_stride < 0)
    return fail(BGTQ_ERR_RANGE, "negative new K/V stride");
  // The kernel reads the new rows as 4-byte words.
  if (reinterpret_cast<uintptr_t>(a->k_new) % 4 || reinterpret_cast<uintptr_t>(a->v_new) % 4)
    return fail(BGTQ_ERR_RANGE, "new K and V must be 4-byte aligned");
  if ((a->k_new_dtype == BGTQ_DTYPE_F16 && (a->k_new_seq_stride % 2 || a->k_new_row_stride % 2 || a->k_new_head_stride % 2)) ||
      (a->v_new_dtype == BGTQ_DTYPE_F16 && (a->v_new_seq_stride % 2 || a->v_new_row_stride % 2 || a->v_new_head_stride % 2)))
    return fail(BGTQ_ERR_RANGE, "FP16 new K/V strides must be even");
  if (d && d->key_format != BGTQ_KEYS_PACKED) return fail(BGTQ_ERR_UNSUPPORTED, "prefill_append needs packed K");
  if (d && d->rows > kPrefillRowwiseRows)
    return fail(BGTQ_ERR_UNSUPPORTED, "prefill_append takes chunks of up to %d rows", kPrefillRowwiseRows);
  return prefill_impl(ctx, d, a);
}

static bgtq_status prefill_impl(bgtq_context *ctx, const bgtq_prefill_desc *d, const bgtq_prefill_append_desc *a) {
  if (!ctx) return fail(BGTQ_ERR_RANGE, "null context");
  PrefillPlan plan{};
  if (bgtq_status s = plan_prefill(d, &plan, a != nullptr)) return s;
  if (a && !plan.rowwise) return fail(BGTQ_ERR_UNSUPPORTED, "prefill_append needs the row-wise path (batch x query groups up to 65535)");
  if (plan.workspace && (!d->workspace || d->workspace_bytes < plan.workspace))
    return fail(BGTQ_ERR_RANGE, "workspace of %zu bytes required", plan.workspace);
  if (plan.workspace && (reinterpret_cast<uintptr_t>(d->workspace) & 15))
    return fail(BGTQ_ERR_RANGE, "workspace must be 16-byte aligned");
  // The layout check shares the fused decode's requirements.
  DecodeParams dp{};
  for (int h = 0; h < d->kv_heads; ++h) dp.tables[h] = d->key_format == BGTQ_KEYS_PACKED ? d->tables[h]->dev() : nullptr;
  dp.batch = d->batch;
  dp.q_heads = d->q_heads;
  dp.kv_heads = d->kv_heads;
  dp.dim = d->dim;
  dp.G = d->q_heads / d->kv_heads;
  dp.key_format = d->key_format == BGTQ_KEYS_PACKED ? 1 : 0;
  dp.packed = d->packed;
  dp.packed_seq_stride = d->packed_seq_stride;
  dp.packed_head_stride = d->packed_head_stride;
  dp.norms = d->norms;
  dp.norms_seq_stride = d->norms_seq_stride;
  dp.norms_head_stride = d->norms_head_stride;
  dp.k = d->k_f16;
  dp.k_seq_stride = d->k_seq_stride;
  dp.k_head_stride = d->k_head_stride;
  dp.v = d->v;
  dp.v_dtype = BGTQ_DTYPE_F16;
  dp.v_seq_stride = d->v_seq_stride;
  dp.v_head_stride = d->v_head_stride;
  dp.k_new = a ? a->k_new : nullptr;  // the layout checks include the encoders' table copies
  FastLayout fl{};
  int nn = 0, sg = 0;
  bool fused = fast_layout(dp, d->tables, &fl, &nn, &sg);
  if (!fused && general_layout(dp, d->tables, &fl)) {  // any packed layout: per-position K build
    fused = true;
    nn = -1;
    for (int h = 0; h < d->kv_heads; ++h) {
      const DevTables *T = d->tables[h]->h();
      if (T->n_books * T->max_centroids * 4 > prefill_general_book_bytes(d->dim)) fused = false;
    }
  }
  if (!fused)
    return fail(BGTQ_ERR_UNSUPPORTED, "prefill needs 16-byte aligned FP16 V/K/scales and a packed layout the "
                                      "fused kernels hold (books, groups per 32 dims and norm stride within their limits)");
  if (reinterpret_cast<uintptr_t>(d->q) & 15) return fail(BGTQ_ERR_RANGE, "q must be 16-byte aligned");
  if (bgtq_status s = ctx->use()) return s;
  if (plan.rowwise) {  // every query row as a decode step over its causal history
    uint8_t *ws = static_cast<uint8_t *>(d->workspace);
    dp.q = d->q;
    dp.q_rotated = d->q_rotated;
    dp.rows = d->rows;
    dp.starts = d->starts;
    dp.max_length = (int32_t)d->max_length;
    dp.qgroups = plan.qgroups;
    dp.unit_cols = plan.unit_cols;
    dp.splits = plan.splits;
    dp.split_floor = plan.split_floor;
    dp.split_tokens = 0;
    dp.inv_sqrt_d = (float)(1.0 / std::sqrt((double)d->dim));
    if (a) {
      dp.k_new = a->k_new;
      dp.k_new_f32 = a->k_new_dtype == BGTQ_DTYPE_F32;
      dp.k_new_seq_stride = a->k_new_seq_stride;
      dp.k_new_row_stride = a->k_new_row_stride;
      dp.k_new_head_stride = a->k_new_head_stride;
      dp.v_new = a->v_new;
      dp.v_new_f32 = a->v_new_dtype == BGTQ_DTYPE_F32;
      dp.v_new_seq_stride = a->v_new_seq_stride;
      dp.v_new_row_stride = a->v_new_row_stride;
      dp.v_new_head_stride = a->v_new_head_stride;
      dp.app_parts = plan.app_parts;
    }
    dp.counters = reinterpret_cast<uint32_t *>(ws + plan.counters);
    // The counter prefix holds 65536 words: units on lines of their own while they fit.
    dp.counter_stride = (int)std::max<int64_t>(
        1, std::min<int64_t>(kCounterStride, 65536 / ((int64_t)d->batch * plan.qgroups * d->kv_heads)));
    dp.part = reinterpret_cast<float *>(ws + plan.part);
    dp.out = d->out;
    HIP_TRY(launch_decode_fast(dp, fl, nn, sg, ctx->stream), "prefill launch");
    return BGTQ_OK;
  }
  PrefillParams p{};
  for (int h = 0; h < d->kv_heads; ++h) p.tables[h] = dp.tables[h];
  p.batch = d->batch;
  p.rows = d->rows;
  p.q_heads = d->q_heads;
  p.kv_heads = d->kv_heads;
  p.dim = d->dim;
  p.G = dp.G;
  p.key_format = dp.key_format;
  p.packed = d->packed;
  p.packed_seq_stride = d->packed_seq_stride;
  p.packed_head_stride = d->packed_head_stride;
  p.norms = d->norms;
  p.norms_seq_stride = d->norms_seq_stride;
  p.norms_head_stride = d->norms_head_stride;
  p.k = d->k_f16;
  p.k_seq_stride = d->k_seq_stride;
  p.k_head_stride = d->k_head_stride;
  p.v = d->v;
  p.v_seq_stride = d->v_seq_stride;
  p.v_head_stride = d->v_head_stride;
  p.q = d->q;
  p.q_rotated = d->q_rotated;
  p.inv_sqrt_d = (float)(1.0 / std::sqrt((double)d->dim));
  p.starts = d->starts;
  p.max_length = (int32_t)d->max_length;
  p.tiles = plan.tiles;
  p.tile_queries = plan.tile_queries;
  p.ranges = plan.ranges;
  p.range_blocks = plan.range_blocks;
  // Two workgroups per compute unit: the first one dispatched to each gets
  // most of its issue slots (measured: the second takes about 1.3 times as
  // long for the same work), so the first round gets the longer ranges.
  p.first_round = plan.range_blocks == 0 && plan.ranges == 2 * device_cus() ? device_cus() : 0;
  p.part = reinterpret_cast<float *>(static_cast<uint8_t *>(d->workspace) + kPrefillCounterBytes);
  p.tile_info = reinterpret_cast<int32_t *>(static_cast<uint8_t *>(d->workspace) + kPrefillCounterBytes + plan.records);
  p.out = d->out;
  HIP_TRY(launch_prefill(p, fl, nn, sg, ctx->stream), "prefill launch");
  return BGTQ_OK;
}

// ---------------------------------------------------------------- attention sessions
bgtq_status bgtq_attention_create(bgtq_keys *k, bgtq_values *v, uint32_t max_queries, int32_t materialize,
                                  bgtq_attention **out) {
  if (!k || !v || !out) return fail(BGTQ_ERR_RANGE, "null argument");
  if (k->ctx != v->ctx || k->dim != v->dim || k->capacity != v->capacity || max_queries < 1 || max_queries > 16)
    return fail(BGTQ_ERR_RANGE, "Incompatible attention storage");
  auto *a = new bgtq_attention();
  a->keys = k;
  a->values = v;
  a->max_queries = max_queries;
  a->materialize = materialize ? 1 : 0;
  a->max_splits = (uint32_t)std::min<int64_t>(256, std::max<int64_t>(1, ((int64_t)k->capacity + 255) / 256));
  const size_t d = k->dim, Q = max_queries;
  bgtq_status s = k->ctx->use();
  struct Item {
    DeviceBuffer *b;
    const char *name;
    size_t bytes;
  } items[] = {
      {&a->q, "Q", Q * d * 4},
      {&a->small, "query positions", (Q + 1) * 4},
      {&a->logits, "logits", a->materialize ? Q * k->capacity * 4 : 0},
      {&a->probs, "probabilities", a->materialize ? Q * k->capacity * 4 : 0},
      {&a->out, "output", Q * d * 4},
      {&a->qr, "rotated Q", Q * d * 4},
      {&a->part, "split partials", Q * a->max_splits * (d + 2) * 4},
      {&a->stats, "softmax statistics", Q * 2 * 4},
      {&a->counters, "split counter", 4},
  };
  for (auto &it : items) {
    if (s || !it.bytes) continue;
    s = it.b->alloc(it.bytes, it.name);
    if (!s) a->ledger.add(it.name, BGTQ_ROLE_SCRATCH, it.bytes);
  }
  if (!s) {
    hipError_t e = hipHostMalloc((void **)&a->pinned, (Q + 1) * 4, hipHostMallocDefault);
    if (e != hipSuccess) s = hip_fail(e, "pinned staging");
  }
  if (s) {
    delete a;
    return s;
  }
  *out = a;
  return BGTQ_OK;
}

static bool optimized(const bgtq_attention *a) { return a->keys->kind == BGTQ_KEYS_PACKED; }

bgtq_status bgtq_attention_set_queries(bgtq_attention *a, const float *q, size_t n_q, const uint32_t *positions,
                                       size_t n_pos, int32_t causal) {
  if (!a) return fail(BGTQ_ERR_RANGE, "null attention");
  bgtq_keys *k = a->keys;
  const size_t d = k->dim;
  if (optimized(a)) {
    // OptimizedAttention.setQueries (src/attention/optimized.ts:28-32)
    if (bgtq_status s = bgtq_keys_ready(k)) return s;
    const bool whole = n_q % d == 0;
    const size_t n = n_q / d;
    bool bad = k->length != a->values->length || !whole || n < 1 || n > a->max_queries || n_pos != n || !positions;
    for (size_t i = 0; !bad && i < n; ++i) bad = positions[i] >= k->length;
    if (bad) return fail(BGTQ_ERR_RANGE, "Invalid Q/K/V shape or positions");
  } else {
    // AttentionSession.setQueries (src/attention/attention.ts:35-41)
    if (k->length != a->values->length || !k->length) return fail(BGTQ_ERR_RANGE, "K/V lengths must match and be nonzero");
    const bool whole = n_q % d == 0;
    const size_t n = n_q / d;
    bool bad = !whole || n < 1 || n > a->max_queries || n_pos != n || !positions;
    for (size_t i = 0; !bad && i < n; ++i) bad = positions[i] >= k->length;
    if (bad) return fail(BGTQ_ERR_RANGE, "Invalid query shape or causal positions");
  }
  for (size_t i = 0; i < n_q; ++i)
    if (!std::isfinite(q[i])) return fail(BGTQ_ERR_RANGE, "Q: finite inputs required");
  if (bgtq_status s = k->ctx->use()) return s;
  HIP_TRY(hipStreamSynchronize(k->ctx->stream), "hipStreamSynchronize");
  HIP_TRY(hipMemcpy(a->q.ptr, q, n_q * 4, hipMemcpyHostToDevice), "Q upload");
  a->positions.assign(positions, positions + n_pos);
  a->queries = (uint32_t)(n_q / d);
  a->causal = causal ? 1 : 0;
  return BGTQ_OK;
}

// record(), with timestamps ts[i0] and ts[i1] (ts may be null) written on the
// stream right around the attention passes, after the queries' upload.
static bgtq_status attention_record(bgtq_attention *a, bgtq_timestamps *ts, uint32_t i0, uint32_t i1) {
  if (!a) return fail(BGTQ_ERR_RANGE, "null attention");
  bgtq_keys *k = a->keys;
  bgtq_values *v = a->values;
  if (optimized(a))
    if (bgtq_status s = bgtq_keys_ready(k)) return s;
  if (!a->queries || k->length != v->length) return fail(BGTQ_ERR_STATE, "Attention not ready");
  if (k->kind == BGTQ_KEYS_COMPRESSED)
    if (bgtq_status s = bgtq_keys_prepare(k, nullptr, 0)) return s;
  bgtq_context *ctx = k->ctx;
  if (bgtq_status s = ctx->use()) return s;
  const uint32_t T = k->length, nq = a->queries;
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  a->pinned[0] = T;
  for (uint32_t i = 0; i < nq; ++i) a->pinned[1 + i] = a->causal ? a->positions[i] + 1 : T;
  HIP_TRY(hipMemcpyAsync(a->small.ptr, a->pinned, (nq + 1) * 4, hipMemcpyHostToDevice, ctx->stream), "query upload");
  DecodeParams p{};
  p.batch = 1;
  p.q_heads = (int32_t)nq;
  p.kv_heads = 1;
  p.dim = (int32_t)k->dim;
  p.G = (int32_t)nq;
  if (k->kind == BGTQ_KEYS_PACKED) {
    p.key_format = 1;
    p.tables[0] = k->tables->dev();
    p.packed = static_cast<const uint8_t *>(k->packed.ptr);
    p.norms = static_cast<const uint16_t *>(k->norms.ptr);
  } else if (k->kind == BGTQ_KEYS_FP16) {
    p.key_format = 0;
    p.k = k->fp16.ptr;
  } else {
    p.key_format = 2;
    p.k = k->decoded.ptr;
  }
  p.v = v->buf.ptr;
  p.v_dtype = v->dtype;
  p.v_f32_split = v->dtype == BGTQ_DTYPE_F32 && v->fp16_range;
  p.qr = static_cast<float *>(a->qr.ptr);
  p.lengths = static_cast<const uint32_t *>(a->small.ptr);
  p.max_length = (int32_t)T;
  p.ends = reinterpret_cast<const int32_t *>(static_cast<const uint32_t *>(a->small.ptr) + 1);
  p.splits = choose_splits(1, T, 0);
  p.splits = (int)std::min<uint32_t>((uint32_t)p.splits, a->max_splits);
  p.split_tokens = (int)(((T + p.splits - 1) / p.splits + 127) / 128 * 128);
  p.part = static_cast<float *>(a->part.ptr);
  p.stats = static_cast<float *>(a->stats.ptr);
  p.counters = static_cast<uint32_t *>(a->counters.ptr);
  p.counter_stride = 1;
  p.inv_sqrt_d = (float)(1.0 / std::sqrt((double)k->dim));
  p.out = static_cast<float *>(a->out.ptr);
  if (a->materialize) {
    p.logits = static_cast<float *>(a->logits.ptr);
    p.probs = static_cast<float *>(a->probs.ptr);
    p.logit_stride = T;  // inspect() buffers are [queries x tokens]
  }
  const bgtq_tables *tabs[1] = {k->tables};
  const float *q = static_cast<const float *>(a->q.ptr);
  if (ts)
    if (bgtq_status s = bgtq_timestamps_write(ts, i0)) return s;
  bgtq_status st = launch_decode_common(ctx, p, q, tabs);
  if (!st && ts) st = bgtq_timestamps_write(ts, i1);
  return st;
}

bgtq_status bgtq_attention_record(bgtq_attention *a) { return attention_record(a, nullptr, 0, 0); }

bgtq_status bgtq_attention_record_timed(bgtq_attention *a, bgtq_timestamps *ts, uint32_t begin_index,
                                        uint32_t end_index) {
  if (!ts) return fail(BGTQ_ERR_RANGE, "null timestamps");
  if (begin_index >= ts->events.size() || end_index >= ts->events.size())
    return fail(BGTQ_ERR_RANGE, "Invalid timestamp write");
  return attention_record(a, ts, begin_index, end_index);
}

bgtq_status bgtq_attention_attend(bgtq_attention *a, const float *q, size_t n_q, const uint32_t *positions,
                                  size_t n_pos, int32_t causal) {
  if (bgtq_status s = bgtq_attention_set_queries(a, q, n_q, positions, n_pos, causal)) return s;
  if (bgtq_status s = bgtq_attention_record(a)) return s;
  HIP_TRY(hipStreamSynchronize(a->keys->ctx->stream), "attention");
  return BGTQ_OK;
}

bgtq_status bgtq_attention_read(const bgtq_attention *a, int32_t which, float *out, size_t count) {
  if (!a || !out) return fail(BGTQ_ERR_RANGE, "null argument");
  const DeviceBuffer *b = which == 0 ? &a->logits : which == 1 ? &a->probs : which == 2 ? &a->out : nullptr;
  if (!b) return fail(BGTQ_ERR_RANGE, "invalid buffer selector");
  if (!b->ptr) return fail(BGTQ_ERR_STATE, "intermediates are not materialised by this session");
  if (count * 4 > b->bytes) return fail(BGTQ_ERR_RANGE, "Invalid readback length");
  if (bgtq_status s = a->keys->ctx->use()) return s;
  HIP_TRY(hipStreamSynchronize(a->keys->ctx->stream), "hipStreamSynchronize");
  HIP_TRY(hipMemcpy(out, b->ptr, count * 4, hipMemcpyDeviceToHost), "readback");
  return BGTQ_OK;
}

uint32_t bgtq_attention_queries(const bgtq_attention *a) { return a ? a->queries : 0; }
bgtq_status bgtq_attention_allocations(const bgtq_attention *a, bgtq_allocation *out, size_t cap, size_t *n) {
  if (!a) return fail(BGTQ_ERR_RANGE, "null attention");
  return a->ledger.copy(out, cap, n);
}
void bgtq_attention_destroy(bgtq_attention *a) {
  if (!a) return;
  (void)a->keys->ctx->use();
  (void)hipStreamSynchronize(a->keys->ctx->stream);
  delete a;
}

/* ---- device buffers ------------------------------------------------------ */

struct bgtq_buffer {
  bgtq_context *ctx = nullptr;
  DeviceBuffer mem;
};

bgtq_status bgtq_buffer_create(bgtq_context *ctx, size_t bytes, bgtq_buffer **out) {
  if (!ctx || !out) return fail(BGTQ_ERR_RANGE, "null argument");
  const size_t size = (bytes + 3) / 4 * 4;
  if (size < 4) return fail(BGTQ_ERR_RANGE, "unsupported buffer size %zu", size);
  if (bgtq_status s = ctx->use()) return s;
  std::unique_ptr<bgtq_buffer> b(new bgtq_buffer());
  b->ctx = ctx;
  if (bgtq_status s = b->mem.alloc(size, "buffer")) return s;  // zero-filled
  *out = b.release();
  return BGTQ_OK;
}
void *bgtq_buffer_device_ptr(const bgtq_buffer *b) { return b ? b->mem.ptr : nullptr; }
size_t bgtq_buffer_size(const bgtq_buffer *b) { return b ? b->mem.bytes : 0; }
bgtq_status bgtq_buffer_write(bgtq_buffer *b, size_t offset, const void *src, size_t bytes) {
  if (!b || (bytes && !src)) return fail(BGTQ_ERR_RANGE, "null argument");
  if (offset > b->mem.bytes || bytes > b->mem.bytes - offset)
    return fail(BGTQ_ERR_RANGE, "Unaligned/out-of-range buffer upload");
  if (!bytes) return BGTQ_OK;
  if (bgtq_status s = b->ctx->use()) return s;
  HIP_TRY(hipMemcpyAsync(static_cast<uint8_t *>(b->mem.ptr) + offset, src, bytes, hipMemcpyHostToDevice,
                         b->ctx->stream), "buffer upload");
  HIP_TRY(hipStreamSynchronize(b->ctx->stream), "hipStreamSynchronize");
  return BGTQ_OK;
}
bgtq_status bgtq_buffer_read(const bgtq_buffer *b, size_t offset, void *dst, size_t bytes) {
  if (!b || (bytes && !dst)) return fail(BGTQ_ERR_RANGE, "null argument");
  if (offset > b->mem.bytes || bytes > b->mem.bytes - offset) return fail(BGTQ_ERR_RANGE, "Invalid readback length");
  if (!bytes) return BGTQ_OK;
  if (bgtq_status s = b->ctx->use()) return s;
  HIP_TRY(hipStreamSynchronize(b->ctx->stream), "hipStreamSynchronize");
  HIP_TRY(hipMemcpy(dst, static_cast<const uint8_t *>(b->mem.ptr) + offset, bytes, hipMemcpyDeviceToHost),
          "buffer readback");
  return BGTQ_OK;
}
void bgtq_buffer_destroy(bgtq_buffer *b) {
  if (!b) return;
  (void)b->ctx->use();
  (void)hipStreamSynchronize(b->ctx->stream);
  delete b;
}

/* ---- the model step's kernel protocol ----------------------------------- */

}  // extern "C"

namespace {

enum class ModelOp { Append, Encode, Scores, Softmax, Weighted };

struct ModelStep {
  ModelOp op;
  ModelAppendParams append{};
  bgtq_encode_job encode{};
  ModelScoresParams scores{};
  int kv_count = 0, lds = 0;
  ModelAttnParams attn{};
  int64_t score_rows = 0;
};

bool aligned(const void *p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

// Checks one dispatch and turns it into a queued step; nothing is queued here.
bgtq_status plan_model_dispatch(const bgtq_model_dispatch &D, size_t idx, ModelStep *st) {
  if (!D.name) return fail(BGTQ_ERR_RANGE, "dispatch %zu: null name", idx);
  const std::string name(D.name);
  const uint32_t *P = D.params;
  auto count = [&](size_t want) -> bgtq_status {
    if (D.n_bindings != want || (want && !D.bindings))
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (%s): %zu bindings, %zu expected", idx, D.name, D.n_bindings, want);
    return BGTQ_OK;
  };
  auto need = [&](int b, uint64_t bytes, size_t align) -> bgtq_status {
    const bgtq_binding &B = D.bindings[b];
    if (!bytes) return BGTQ_OK;
    if (!B.ptr) return fail(BGTQ_ERR_RANGE, "dispatch %zu (%s): binding %d is null", idx, D.name, b);
    if (B.bytes < bytes)
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (%s): binding %d holds %zu bytes, %llu needed", idx, D.name, b,
                  B.bytes, (unsigned long long)bytes);
    if (!aligned(B.ptr, align))
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (%s): binding %d is not %zu-byte aligned", idx, D.name, b, align);
    return BGTQ_OK;
  };
  auto tables_of = [&](const bgtq_tables **t) -> bgtq_status {
    *t = D.bindings[0].tables;
    if (!*t || (D.bindings[1].tables && D.bindings[1].tables != *t))
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (%s): config and table bindings must name one calibration table set",
                  idx, D.name);
    return BGTQ_OK;
  };
  const uint64_t x = D.x, y = D.y;
  if (name == "append") {
    if (bgtq_status s = count(2)) return s;
    const uint64_t rows = P[0], start = P[1], capacity = P[2], heads = P[3];
    if (rows && (!heads || start + rows > capacity))
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (append): rows %llu from %llu exceed capacity %llu", idx,
                  (unsigned long long)rows, (unsigned long long)start, (unsigned long long)capacity);
    const uint64_t pairs = std::min<uint64_t>(x * 128, rows * heads * 32);
    if (bgtq_status s = need(0, pairs * 8, 8)) return s;
    if (bgtq_status s = need(1, pairs ? heads * capacity * 64 * 2 : 0, 4)) return s;
    st->op = ModelOp::Append;
    st->append.input = static_cast<const float *>(D.bindings[0].ptr);
    st->append.cache = static_cast<uint32_t *>(D.bindings[1].ptr);
    st->append.pairs = (int64_t)pairs;
    st->append.start = (int32_t)start;
    st->append.capacity = (int32_t)capacity;
    st->append.heads = (int32_t)heads;
    return BGTQ_OK;
  }
  if (name == "encode_k") {
    if (bgtq_status s = count(5)) return s;
    const bgtq_tables *t = nullptr;
    if (bgtq_status s = tables_of(&t)) return s;
    const uint64_t rows = std::min<uint64_t>(P[0], x), start = P[1], head = P[2], kvh = P[3];
    const uint64_t d = (uint64_t)t->info.dim, rb = (uint64_t)t->info.row_bytes, ns = (uint64_t)t->info.norm_stride;
    if (rows && head >= kvh)
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (encode_k): head %llu of %llu", idx, (unsigned long long)head,
                  (unsigned long long)kvh);
    if (bgtq_status s = need(2, rows ? ((rows - 1) * kvh + head + 1) * d * 4 : 0, 4)) return s;
    if (bgtq_status s = need(3, rows ? (start + rows) * rb : 0, 4)) return s;
    if (bgtq_status s = need(4, rows ? (start + rows) * ns * 2 : 0, 2)) return s;
    if (kvh * d > INT32_MAX) return fail(BGTQ_ERR_RANGE, "dispatch %zu (encode_k): row stride above 2^31 - 1", idx);
    st->op = ModelOp::Encode;
    st->encode.tables = t;
    st->encode.src = static_cast<const float *>(D.bindings[2].ptr) + head * d;
    st->encode.src_row_stride = (int64_t)(kvh * d);
    st->encode.rows = (int64_t)rows;
    st->encode.packed = static_cast<uint8_t *>(D.bindings[3].ptr);
    st->encode.norms = static_cast<uint16_t *>(D.bindings[4].ptr);
    st->encode.dst_row0 = (int64_t)start;
    return BGTQ_OK;
  }
  const bool compressed = name == "compressed_dot";
  if (compressed || name == "dot" || name == "softmax" || name == "weighted") {
    if (bgtq_status s = count(compressed ? 7 : 6)) return s;
    // compressed_dot [rows,start,head,tokens,qHeads,gqa,headDim];
    // the others [rows,tokens,capacity,start,qHeads,kvHeads,gqa,headDim].
    const uint64_t rows = P[0];
    const uint64_t start = compressed ? P[1] : P[3], tokens = compressed ? P[3] : P[1];
    const uint64_t qh = P[4], gqa = compressed ? P[5] : P[6], d = compressed ? P[6] : P[7];
    const uint64_t capacity = compressed ? 0 : P[2], kvh = compressed ? 0 : P[5];
    if (d != 64 && d != 128)
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (%s): head_dim %llu (64 or 128)", idx, D.name, (unsigned long long)d);
    if (gqa < 1 || gqa > 16)
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (%s): gqa %llu (1 to 16)", idx, D.name, (unsigned long long)gqa);
    if (!compressed && qh != kvh * gqa)
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (%s): q_heads must be kv_heads * gqa", idx, D.name);
    if (rows > 65535 || kvh > 65535 || tokens > INT32_MAX || start + rows > INT32_MAX)
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (%s): sizes beyond the launch limits", idx, D.name);
    // Tokens a query row can read: up to its causal end start + row.
    const uint64_t span = std::min<uint64_t>(tokens, start + rows);
    if (name == "dot" || compressed) {
      const uint64_t n_tok = std::min<uint64_t>(tokens, x);
      const uint64_t read = std::min<uint64_t>(n_tok, start + rows);
      ModelScoresParams &sp = st->scores;
      st->op = ModelOp::Scores;
      sp.rows = (int32_t)rows;
      sp.start = (int32_t)start;
      sp.q_heads = (int32_t)qh;
      sp.gqa = (int32_t)gqa;
      sp.dim = (int32_t)d;
      sp.tokens = (int32_t)tokens;
      sp.n_tok = (int32_t)n_tok;
      sp.y_limit = (int32_t)std::min<uint64_t>(y, INT32_MAX);
      sp.scale = (float)(1.0 / std::sqrt((double)d));
      const int sb = compressed ? 6 : 3, qb = 2 - (compressed ? 0 : 2);
      uint64_t q_heads_used = qh;
      if (compressed) {
        const bgtq_tables *t = nullptr;
        if (bgtq_status s = tables_of(&t)) return s;
        const uint64_t head = P[2];
        if ((head + 1) * gqa > qh)
          return fail(BGTQ_ERR_RANGE, "dispatch %zu (compressed_dot): query heads beyond q_heads", idx);
        if ((uint64_t)t->info.dim != d)
          return fail(BGTQ_ERR_RANGE, "dispatch %zu (compressed_dot): tables of dim %d for head_dim %llu", idx,
                      t->info.dim, (unsigned long long)d);
        q_heads_used = (head + 1) * gqa;
        if (bgtq_status s = need(3, read * (uint64_t)t->info.row_bytes, 1)) return s;
        if (bgtq_status s = need(4, read * (uint64_t)t->info.norm_stride * 2, 2)) return s;
        sp.tables = t->dev();
        sp.packed = static_cast<const uint8_t *>(D.bindings[3].ptr);
        sp.norms = static_cast<const uint16_t *>(D.bindings[4].ptr);
        sp.head0 = (int32_t)head;
        st->kv_count = 1;
        st->lds = model_scores_lds_bytes((int)d, t->info.n_books * t->info.max_centroids);
        if (st->lds > 64 * 1024)
          return fail(BGTQ_ERR_UNSUPPORTED, "dispatch %zu (compressed_dot): centroid books too large", idx);
      } else {
        if (read > capacity)
          return fail(BGTQ_ERR_RANGE, "dispatch %zu (dot): tokens beyond capacity %llu", idx,
                      (unsigned long long)capacity);
        if (bgtq_status s = need(1, (n_tok && rows) ? kvh * capacity * d * 2 : 0, 2)) return s;
        sp.k = static_cast<const uint16_t *>(D.bindings[1].ptr);
        sp.capacity = (int32_t)capacity;
        sp.head0 = 0;
        st->kv_count = (int)kvh;
        st->lds = model_scores_lds_bytes((int)d, 0);
      }
      if (rows && n_tok) {
        if (bgtq_status s = need(qb, ((rows - 1) * qh + q_heads_used) * d * 4, 4)) return s;
        if (bgtq_status s = need(sb, (((rows - 1) * qh + q_heads_used - 1) * tokens + n_tok) * 4, 4)) return s;
      }
      sp.q = static_cast<const float *>(D.bindings[qb].ptr);
      sp.scores = static_cast<float *>(D.bindings[sb].ptr);
      return BGTQ_OK;
    }
    ModelAttnParams &ap = st->attn;
    ap.tokens = (int32_t)tokens;
    ap.start = (int32_t)start;
    ap.q_heads = (int32_t)qh;
    ap.gqa = (int32_t)gqa;
    ap.dim = (int32_t)d;
    ap.capacity = (int32_t)capacity;
    ap.scores = static_cast<const float *>(D.bindings[3].ptr);
    ap.probs = static_cast<float *>(D.bindings[4].ptr);
    ap.v = static_cast<const uint16_t *>(D.bindings[2].ptr);
    ap.out = static_cast<float *>(D.bindings[5].ptr);
    if (name == "softmax") {
      st->op = ModelOp::Softmax;
      st->score_rows = (int64_t)std::min<uint64_t>(x, rows * qh);
      if (bgtq_status s = need(3, (uint64_t)st->score_rows * tokens * 4, 4)) return s;
      if (bgtq_status s = need(4, (uint64_t)st->score_rows * tokens * 4, 4)) return s;
      return BGTQ_OK;
    }
    st->op = ModelOp::Weighted;
    const uint64_t outs = std::min<uint64_t>(x, rows * qh * d);
    ap.x_limit = (int64_t)outs;
    st->score_rows = (int64_t)((outs + d - 1) / d);
    if (outs && span > capacity)
      return fail(BGTQ_ERR_RANGE, "dispatch %zu (weighted): tokens beyond capacity %llu", idx,
                  (unsigned long long)capacity);
    if (bgtq_status s = need(4, (uint64_t)st->score_rows * tokens * 4, 4)) return s;
    if (bgtq_status s = need(2, outs ? kvh * capacity * d * 2 : 0, 2)) return s;
    if (bgtq_status s = need(5, outs * 4, 4)) return s;
    return BGTQ_OK;
  }
  static const char *const kOther[] = {"embedding", "matmul", "norm", "element", "rope"};
  for (const char *o : kOther)
    if (name == o)
      return fail(BGTQ_ERR_UNSUPPORTED, "model kernel %s is outside the attention path this library serves", D.name);
  return fail(BGTQ_ERR_RANGE, "dispatch %zu: unknown model kernel %s", idx, D.name);
}

}  // namespace

extern "C" {

bgtq_status bgtq_model_submit(bgtq_context *ctx, const bgtq_model_dispatch *dispatches, size_t n) {
  if (!ctx) return fail(BGTQ_ERR_RANGE, "null context");
  if (n && !dispatches) return fail(BGTQ_ERR_RANGE, "null dispatches");
  std::vector<ModelStep> steps(n);
  for (size_t i = 0; i < n; ++i)
    if (bgtq_status s = plan_model_dispatch(dispatches[i], i, &steps[i])) return s;
  if (bgtq_status s = ctx->use()) return s;
  std::vector<bgtq_encode_job> jobs;
  auto flush = [&]() -> bgtq_status {
    if (jobs.empty()) return BGTQ_OK;
    const bgtq_status s = bgtq_encode_batched(ctx, BGTQ_DTYPE_F32, jobs.data(), jobs.size());
    jobs.clear();
    return s;
  };
  for (const ModelStep &st : steps) {
    if (st.op == ModelOp::Encode) {
      jobs.push_back(st.encode);
      continue;
    }
    if (bgtq_status s = flush()) return s;
    switch (st.op) {
      case ModelOp::Append: HIP_TRY(launch_model_append(st.append, ctx->stream), "model append"); break;
      case ModelOp::Scores:
        HIP_TRY(launch_model_scores(st.scores, st.kv_count, st.lds, ctx->stream), "model scores");
        break;
      case ModelOp::Softmax: HIP_TRY(launch_model_softmax(st.attn, st.score_rows, ctx->stream), "model softmax"); break;
      case ModelOp::Weighted:
        HIP_TRY(launch_model_weighted(st.attn, st.score_rows, ctx->stream), "model weighted");
        break;
      default: break;
    }
  }
  return flush();
}

}  // extern "C"
