// XLA GPU custom-call handlers for the rxw8 ops.
//
// The reference appends backend custom calls to a lazy trace with
// CustomCall::{typed_ffi, backend_config, api_version}
// (crates/rxla-core/src/tensor_handle.rs:276-345) and registers their
// process-lifetime handlers with a PJRT plugin's GPU custom-call extension
// (crates/rxla-pjrt/src/runtime.rs:380-428, GpuCustomCallApi::{Legacy,
// TypedFfi}). These handlers use XLA's untyped ("legacy") GPU custom-call
// signature with a status argument (HLO api_version 2, status-returning):
//
//   void handler(stream, void **buffers, const char *opaque, size_t opaque_len,
//                XlaCustomCallStatus *status)
//
// buffers = the operands in order, then the result; opaque = the call's
// backend_config, "key=value;key=value" text carrying shapes and dtypes. Each
// handler wraps the device pointers as rxw8 buffers (no copy) and runs the
// same validated `_into` entry point as the C ABI on the stream XLA passes, so
// results are those of the direct calls bit for bit. A failure (bad opaque,
// shapes the entry point rejects) launches nothing; it is reported through
// XlaCustomCallStatusSetFailure when the hosting process exports it (every XLA
// runtime does), and always through rxw8_last_error().
//
// The typed-FFI handlers (rxw8_xla_ffi_*, HLO api_version 4, the reference's
// default for CustomCall::typed_ffi, registered as GpuCustomCallApi::TypedFfi)
// are XLA_FFI_Handler functions: they receive XLA's call frame -- operand and
// result buffers with their dtypes and dims, the backend_config dictionary as
// typed attributes, the execution context that yields the stream -- and return
// NULL or an error made by the frame's own API table. They run the same `_into`
// entry points as the untyped handlers.
#include <dlfcn.h>

#include <cmath>
#include <cstddef>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "internal.h"

using namespace rxw8;

namespace {

// One runtime per (device, stream), created on first use and kept for the
// process (XLA handlers are process-lifetime). Each runtime owns its
// workspaces (split-K partials, attention split partials and arrival
// counters), so handlers that XLA runs concurrently on different streams never
// share them; calls on one stream are ordered by that stream.
rxw8_runtime *stream_runtime(void *stream, int *rc) {
  static std::mutex mu;
  static std::map<std::pair<int, void *>, rxw8_runtime *> rts;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0) {
    *rc = hip_fail(e == hipSuccess ? hipErrorInvalidDevice : e, "hipGetDevice");
    return nullptr;
  }
  std::lock_guard<std::mutex> g(mu);
  rxw8_runtime *&rt = rts[{dev, stream}];
  if (!rt) {
    *rc = rxw8_runtime_create(dev, &rt);
    if (!*rc) *rc = rxw8_runtime_set_stream(rt, stream);  // for good: all its work runs there
    if (*rc) {
      if (rt) rxw8_runtime_destroy(rt);
      rts.erase({dev, stream});
      return nullptr;
    }
  }
  *rc = RXW8_OK;
  return rt;
}

struct Opaque {
  std::string text;
  bool has(const char *key) const { return find(key) != nullptr; }
  const char *find(const char *key) const {
    const size_t n = std::strlen(key);
    size_t pos = 0;
    while (pos < text.size()) {
      size_t end = text.find(';', pos);
      if (end == std::string::npos) end = text.size();
      if (end - pos > n && text.compare(pos, n, key) == 0 && text[pos + n] == '=')
        return text.c_str() + pos + n + 1;
      pos = end + 1;
    }
    return nullptr;
  }
  bool i64(const char *key, int64_t *out) const {
    const char *v = find(key);
    if (!v) return false;
    char *end = nullptr;
    const long long x = std::strtoll(v, &end, 10);
    if (end == v || (*end && *end != ';')) return false;
    *out = x;
    return true;
  }
  bool f32(const char *key, float *out) const {
    const char *v = find(key);
    if (!v) return false;
    char *end = nullptr;
    const float x = std::strtof(v, &end);
    if (end == v || (*end && *end != ';')) return false;
    *out = x;
    return true;
  }
  bool dtype(const char *key, int *out) const {
    const char *v = find(key);
    if (!v) return false;
    static const struct {
      const char *name;
      int dtype;
    } names[] = {{"f32", RXW8_F32}, {"bf16", RXW8_BF16}, {"f16", RXW8_F16}, {"u8", RXW8_U8},
                 {"i32", RXW8_I32}};
    for (const auto &n : names) {
      const size_t len = std::strlen(n.name);
      if (std::strncmp(v, n.name, len) == 0 && (v[len] == ';' || v[len] == 0)) {
        *out = n.dtype;
        return true;
      }
    }
    return false;
  }
};

// Device-pointer views (rxw8_buffer_wrap), released on scope exit.
struct Views {
  rxw8_buffer *b[8] = {nullptr};
  int n = 0;
  ~Views() {
    for (int i = 0; i < n; ++i)
      if (b[i]) rxw8_buffer_release(b[i]);
  }
  int wrap(rxw8_runtime *rt, int dtype, std::initializer_list<int64_t> dims, void *ptr,
           rxw8_buffer **out) {
    int64_t d[RXW8_MAX_RANK];
    int r = 0;
    for (int64_t x : dims) d[r++] = x;
    const int rc = rxw8_buffer_wrap(rt, dtype, d, r, ptr, &b[n]);
    if (rc) return rc;
    *out = b[n++];
    return RXW8_OK;
  }
};

// Run `body` on the runtime of (current device, XLA's stream).
template <typename F>
void run_on_stream(void *stream, const char *what, void *status, F body) {
  int rc = RXW8_OK;
  rxw8_runtime *rt = stream_runtime(stream, &rc);
  if (rt) {
    std::lock_guard<std::recursive_mutex> g(rt->mu);
    rc = body(rt);
  }
  if (rc && status) {
    using SetFailure = void (*)(void *, const char *, size_t);
    static SetFailure set_failure =
        reinterpret_cast<SetFailure>(dlsym(RTLD_DEFAULT, "XlaCustomCallStatusSetFailure"));
    if (set_failure) {
      std::string msg = std::string(what) + ": " + rxw8_last_error();
      set_failure(status, msg.c_str(), msg.size());
    }
  }
}

// ---- XLA FFI C ABI --------------------------------------------------------
// The subset of XLA's public FFI C API (xla/ffi/api/c_api.h, FFI API version
// 0.1, the API of XLA releases that ship PJRT C API 0.115, the version the
// reference vendors) that the handlers read: the layouts must match XLA's, so
// the structs and enum values follow that header; the names carry an Xf
// prefix here. Every struct starts with struct_size and an extension chain.
struct XfExtensionBase {
  size_t struct_size;
  int type;  // XLA_FFI_Extension_Type; 1 = XLA_FFI_Extension_Metadata
  XfExtensionBase *next;
};
struct XfApiVersion {
  size_t struct_size;
  XfExtensionBase *extension_start;
  int major_version, minor_version;
};
struct XfErrorCreateArgs {
  size_t struct_size;
  XfExtensionBase *extension_start;
  const char *message;
  int errc;  // XLA_FFI_Error_Code: the absl::StatusCode numbering (= rxw8_status)
};
struct XfStreamGetArgs {
  size_t struct_size;
  XfExtensionBase *extension_start;
  void *ctx;     // XLA_FFI_ExecutionContext*
  void *stream;  // out: the platform stream (hipStream_t)
};
typedef void *(*XfErrorCreate)(XfErrorCreateArgs *);
typedef void *(*XfStreamGet)(XfStreamGetArgs *);
struct XfApi {
  size_t struct_size;
  XfExtensionBase *extension_start;
  XfApiVersion api_version;
  void *internal_api;
  XfErrorCreate error_create;  // XLA_FFI_Error_Create
  void *error_get_message;     // XLA_FFI_Error_GetMessage
  void *error_destroy;         // XLA_FFI_Error_Destroy
  void *handler_register;      // XLA_FFI_Handler_Register
  XfStreamGet stream_get;      // XLA_FFI_Stream_Get
};
struct XfBuffer {
  size_t struct_size;
  XfExtensionBase *extension_start;
  int dtype;  // XLA_FFI_DataType
  void *data;
  int64_t rank;
  int64_t *dims;
};
struct XfArgs {  // XLA_FFI_Args and XLA_FFI_Rets share this layout
  size_t struct_size;
  XfExtensionBase *extension_start;
  int64_t size;
  int *types;  // XLA_FFI_ArgType / XLA_FFI_RetType: 1 = buffer
  void **args;
};
struct XfByteSpan {
  const char *ptr;
  size_t len;
};
struct XfScalar {
  int dtype;
  void *value;
};
struct XfAttrs {
  size_t struct_size;
  XfExtensionBase *extension_start;
  int64_t size;
  int *types;  // XLA_FFI_AttrType: 1 array, 2 dictionary, 3 scalar, 4 string
  XfByteSpan **names;
  void **attrs;
};
struct XfCallFrame {
  size_t struct_size;
  XfExtensionBase *extension_start;
  const XfApi *api;
  void *ctx;
  int stage;  // XLA_FFI_ExecutionStage: 3 = execute
  XfArgs args;
  XfArgs rets;
  XfAttrs attrs;
};
struct XfMetadata {
  size_t struct_size;
  XfApiVersion api_version;
  uint32_t traits;  // XLA_FFI_Handler_Traits (0: not command-buffer compatible)
};
struct XfMetadataExtension {
  XfExtensionBase extension_base;
  XfMetadata *metadata;
};
constexpr int kXfMetadataExtension = 1;
constexpr int kXfStageExecute = 3;
constexpr int kXfBuffer = 1;
constexpr int kXfAttrScalar = 3, kXfAttrString = 4;
constexpr int kXfApiMajor = 0, kXfApiMinor = 1;
// XLA_FFI_DataType (= xla::PrimitiveType, the reference's vendored
// xla_data.proto) -> rxw8 dtype; 0 for types no handler takes
int xf_dtype(int t) {
  switch (t) {
    case 4: return RXW8_I32;    // S32
    case 6: return RXW8_U8;     // U8
    case 10: return RXW8_F16;   // F16
    case 11: return RXW8_F32;   // F32
    case 16: return RXW8_BF16;  // BF16
    default: return 0;
  }
}

// A typed call's operands (n_args buffers then n_rets) as rxw8 views, and its
// attributes by name. check() validates the frame's structure before anything
// touches a device, so malformed frames fail without a GPU.
struct XfCall {
  const XfCallFrame *f;
  const char *what;
  const XfBuffer *buf[8] = {nullptr};
  int n = 0;

  int check(int n_args, int n_rets) {
    if (f->struct_size < offsetof(XfCallFrame, attrs) + sizeof(XfAttrs))
      return fail(RXW8_INVALID_ARGUMENT, "%s: XLA FFI call frame of %zu bytes is too small", what,
                  f->struct_size);
    if (f->args.size != n_args || f->rets.size != n_rets)
      return fail(RXW8_INVALID_ARGUMENT, "%s: expects %d operands and %d result, got %lld and %lld",
                  what, n_args, n_rets, (long long)f->args.size, (long long)f->rets.size);
    for (int i = 0; i < n_args + n_rets; ++i) {
      const XfArgs &a = i < n_args ? f->args : f->rets;
      const int j = i < n_args ? i : i - n_args;
      if (a.types[j] != kXfBuffer || !a.args[j])
        return fail(RXW8_INVALID_ARGUMENT, "%s: operand %d is not a buffer", what, i);
      buf[n] = static_cast<const XfBuffer *>(a.args[j]);
      if (xf_dtype(buf[n]->dtype) == 0 || buf[n]->rank < 0 || buf[n]->rank > RXW8_MAX_RANK)
        return fail(RXW8_INVALID_ARGUMENT, "%s: operand %d has XLA dtype %d and rank %lld", what, i,
                    buf[n]->dtype, (long long)buf[n]->rank);
      ++n;
    }
    return RXW8_OK;
  }
  // attribute `name` of the given kind, or null when absent
  const void *attr(const char *name, int kind) const {
    const size_t len = std::strlen(name);
    for (int64_t i = 0; i < f->attrs.size; ++i) {
      const XfByteSpan *nm = f->attrs.names[i];
      if (nm && nm->len == len && std::memcmp(nm->ptr, name, len) == 0)
        return f->attrs.types[i] == kind ? f->attrs.attrs[i] : nullptr;
    }
    return nullptr;
  }
  bool has(const char *name) const {
    const size_t len = std::strlen(name);
    for (int64_t i = 0; i < f->attrs.size; ++i)
      if (f->attrs.names[i] && f->attrs.names[i]->len == len &&
          std::memcmp(f->attrs.names[i]->ptr, name, len) == 0)
        return true;
    return false;
  }
  // f32 / f64 scalar attribute
  int scale(float *out) const {
    if (!has("scale")) return RXW8_OK;
    const XfScalar *sc = static_cast<const XfScalar *>(attr("scale", kXfAttrScalar));
    if (sc && sc->dtype == 11) *out = *static_cast<const float *>(sc->value);
    else if (sc && sc->dtype == 12) *out = (float)*static_cast<const double *>(sc->value);
    else return fail(RXW8_INVALID_ARGUMENT, "%s: attribute scale must be an f32 or f64 scalar", what);
    return RXW8_OK;
  }
  // string attribute naming a dtype (f32 / bf16)
  int dtype_attr(const char *name, int *out) const {
    if (!has(name)) return RXW8_OK;
    const XfByteSpan *sp = static_cast<const XfByteSpan *>(attr(name, kXfAttrString));
    const std::string v = sp ? std::string(sp->ptr, sp->len) : std::string();
    if (v == "bf16") *out = RXW8_BF16;
    else if (v == "f32") *out = RXW8_F32;
    else return fail(RXW8_INVALID_ARGUMENT, "%s: attribute %s must be the string bf16 or f32", what, name);
    return RXW8_OK;
  }
  int view(Views &v, rxw8_runtime *rt, int i, rxw8_buffer **out) const {
    const XfBuffer *b = buf[i];
    const int rc = rxw8_buffer_wrap(rt, xf_dtype(b->dtype), b->dims, (int)b->rank, b->data, &v.b[v.n]);
    if (rc) return rc;
    *out = v.b[v.n++];
    return RXW8_OK;
  }
};

// Options a typed call reads from its attributes.
struct XfOptions {
  int compute = RXW8_BF16;
  float scale = 0.f;
};

// Runs a typed call: the metadata query (the frame carries
// XLA_FFI_Metadata_Extension: report API 0.1, no traits), stages other than
// execute (nothing to do), then the frame's structure and attributes
// (`parse`, before any device work), and `body` on the runtime of the
// context's stream; a failure becomes the frame's XLA_FFI_Error.
template <typename P, typename F>
void *run_typed(void *frame, const char *what, int n_args, int n_rets, P parse, F body) {
  XfCallFrame *f = static_cast<XfCallFrame *>(frame);
  if (!f) {
    fail(RXW8_INVALID_ARGUMENT, "%s: call frame is NULL", what);
    return nullptr;  // no API table to report through
  }
  if (f->extension_start && f->extension_start->type == kXfMetadataExtension) {
    XfMetadata *m = reinterpret_cast<XfMetadataExtension *>(f->extension_start)->metadata;
    if (m) {
      m->api_version.major_version = kXfApiMajor;
      m->api_version.minor_version = kXfApiMinor;
      m->traits = 0;
    }
    return nullptr;
  }
  if (f->stage != kXfStageExecute) return nullptr;
  XfCall call{f, what};
  XfOptions opt;
  int rc = call.check(n_args, n_rets);
  if (!rc) rc = parse(call, opt);
  if (!rc) {
    XfStreamGetArgs sa{sizeof(XfStreamGetArgs), nullptr, f->ctx, nullptr};
    void *err = f->api && f->api->stream_get ? f->api->stream_get(&sa) : nullptr;
    if (err) return err;  // XLA's own error, passed through
    if (!f->api || !f->api->stream_get)
      rc = fail(RXW8_INVALID_ARGUMENT, "%s: XLA FFI API table has no stream getter", what);
    rxw8_runtime *rt = rc ? nullptr : stream_runtime(sa.stream, &rc);
    if (rt) {
      std::lock_guard<std::recursive_mutex> g(rt->mu);
      rc = body(rt, call, opt);
    }
  }
  if (!rc) return nullptr;
  if (!f->api || !f->api->error_create) return nullptr;
  std::string msg = std::string(what) + ": " + rxw8_last_error();
  XfErrorCreateArgs ea{sizeof(XfErrorCreateArgs), nullptr, msg.c_str(), rc};
  return f->api->error_create(&ea);
}

int bad_opaque(const char *what) {
  return fail(RXW8_INVALID_ARGUMENT, "%s: backend_config is missing a key or has a malformed value",
              what);
}

}  // namespace

extern "C" {

void rxw8_xla_quantized_linear(void *stream, void **buffers, const char *opaque,
                               size_t opaque_len, void *status) {
  const char *what = "rxw8_quantized_linear";
  run_on_stream(stream, what, status, [&](rxw8_runtime *rt) -> int {
    const Opaque o{std::string(opaque ? opaque : "", opaque ? opaque_len : 0)};
    int64_t m, n, k, g;
    int xd, yd, cd = RXW8_BF16;
    if (!buffers || !o.i64("m", &m) || !o.i64("n", &n) || !o.i64("k", &k) || !o.i64("g", &g) ||
        !o.dtype("x", &xd) || !o.dtype("y", &yd) || (o.has("compute") && !o.dtype("compute", &cd)) ||
        g <= 0 || k % g != 0)
      return bad_opaque(what);
    Views v;
    rxw8_buffer *x, *w, *s, *y;
    int rc;
    if ((rc = v.wrap(rt, xd, {m, k}, buffers[0], &x)) || (rc = v.wrap(rt, RXW8_U8, {n, k}, buffers[1], &w)) ||
        (rc = v.wrap(rt, RXW8_F32, {n, k / g}, buffers[2], &s)) ||
        (rc = v.wrap(rt, yd, {m, n}, buffers[3], &y)))
      return rc;
    return rxw8_quantized_linear_into(rt, x, w, s, cd, y);
  });
}

void rxw8_xla_gqa_decode(void *stream, void **buffers, const char *opaque, size_t opaque_len,
                         void *status) {
  const char *what = "rxw8_gqa_decode";
  run_on_stream(stream, what, status, [&](rxw8_runtime *rt) -> int {
    const Opaque o{std::string(opaque ? opaque : "", opaque ? opaque_len : 0)};
    int64_t b, hq, hkv, lmax, d;
    float scale = 0.f;
    int qd, cd, od;
    if (!buffers || !o.i64("b", &b) || !o.i64("hq", &hq) || !o.i64("hkv", &hkv) ||
        !o.i64("lmax", &lmax) || !o.i64("d", &d) || !o.dtype("q", &qd) || !o.dtype("cache", &cd) ||
        !o.dtype("out", &od) || (o.has("scale") && !o.f32("scale", &scale)))
      return bad_opaque(what);
    Views v;
    rxw8_buffer *q, *kc, *vc, *lens, *out;
    int rc;
    if ((rc = v.wrap(rt, qd, {b, hq, d}, buffers[0], &q)) ||
        (rc = v.wrap(rt, cd, {b, hkv, lmax, d}, buffers[1], &kc)) ||
        (rc = v.wrap(rt, cd, {b, hkv, lmax, d}, buffers[2], &vc)) ||
        (rc = v.wrap(rt, RXW8_I32, {b}, buffers[3], &lens)) ||
        (rc = v.wrap(rt, od, {b, hq, d}, buffers[4], &out)))
      return rc;
    return rxw8_gqa_decode_into(rt, q, kc, vc, lens, nullptr, scale, out);
  });
}

void rxw8_xla_gqa_prefill(void *stream, void **buffers, const char *opaque, size_t opaque_len,
                          void *status) {
  const char *what = "rxw8_gqa_prefill";
  run_on_stream(stream, what, status, [&](rxw8_runtime *rt) -> int {
    const Opaque o{std::string(opaque ? opaque : "", opaque ? opaque_len : 0)};
    int64_t b, s, hq, hkv, lmax, d = 128;
    float scale = 0.f;
    int qd, od;
    if (!buffers || !o.i64("b", &b) || !o.i64("s", &s) || !o.i64("hq", &hq) || !o.i64("hkv", &hkv) ||
        !o.i64("lmax", &lmax) || (o.has("d") && !o.i64("d", &d)) || !o.dtype("q", &qd) ||
        !o.dtype("out", &od) || (o.has("scale") && !o.f32("scale", &scale)))
      return bad_opaque(what);
    Views v;
    rxw8_buffer *q, *kc, *vc, *starts, *out;
    int rc;
    if ((rc = v.wrap(rt, qd, {b, s, hq, d}, buffers[0], &q)) ||
        (rc = v.wrap(rt, RXW8_BF16, {b, hkv, lmax, d}, buffers[1], &kc)) ||
        (rc = v.wrap(rt, RXW8_BF16, {b, hkv, lmax, d}, buffers[2], &vc)) ||
        (rc = v.wrap(rt, RXW8_I32, {b}, buffers[3], &starts)) ||
        (rc = v.wrap(rt, od, {b, s, hq, d}, buffers[4], &out)))
      return rc;
    return rxw8_gqa_prefill_into(rt, q, kc, vc, starts, scale, out);
  });
}

// ---- typed FFI (api_version 4) ---------------------------------------------

void *rxw8_xla_ffi_quantized_linear(void *call_frame) {
  // operands x [..., k], weight U8 [n, k] (or packed), scale F32 [n, k/g];
  // result y [..., n]; attribute compute = "bf16" (default) or "f32"
  return run_typed(
      call_frame, "rxw8_quantized_linear", 3, 1,
      [](const XfCall &c, XfOptions &o) { return c.dtype_attr("compute", &o.compute); },
      [](rxw8_runtime *rt, const XfCall &c, const XfOptions &o) {
        Views v;
        rxw8_buffer *x, *w, *s, *y;
        int rc;
        if ((rc = c.view(v, rt, 0, &x)) || (rc = c.view(v, rt, 1, &w)) || (rc = c.view(v, rt, 2, &s)) ||
            (rc = c.view(v, rt, 3, &y)))
          return rc;
        return rxw8_quantized_linear_into(rt, x, w, s, o.compute, y);
      });
}

void *rxw8_xla_ffi_gqa_decode(void *call_frame) {
  // operands q [b, hq, d], k_cache, v_cache [b, hkv, lmax, d], lens S32 [b];
  // result out [b, hq, d]; attribute scale (optional f32 / f64)
  return run_typed(
      call_frame, "rxw8_gqa_decode", 4, 1,
      [](const XfCall &c, XfOptions &o) { return c.scale(&o.scale); },
      [](rxw8_runtime *rt, const XfCall &c, const XfOptions &o) {
        Views v;
        rxw8_buffer *q, *kc, *vc, *lens, *out;
        int rc;
        if ((rc = c.view(v, rt, 0, &q)) || (rc = c.view(v, rt, 1, &kc)) || (rc = c.view(v, rt, 2, &vc)) ||
            (rc = c.view(v, rt, 3, &lens)) || (rc = c.view(v, rt, 4, &out)))
          return rc;
        return rxw8_gqa_decode_into(rt, q, kc, vc, lens, nullptr, o.scale, out);
      });
}

void *rxw8_xla_ffi_gqa_prefill(void *call_frame) {
  // operands q [b, s, hq, d], k_cache, v_cache BF16 [b, hkv, lmax, d], starts
  // S32 [b]; result out [b, s, hq, d]; attribute scale (optional)
  return run_typed(
      call_frame, "rxw8_gqa_prefill", 4, 1,
      [](const XfCall &c, XfOptions &o) { return c.scale(&o.scale); },
      [](rxw8_runtime *rt, const XfCall &c, const XfOptions &o) {
        Views v;
        rxw8_buffer *q, *kc, *vc, *starts, *out;
        int rc;
        if ((rc = c.view(v, rt, 0, &q)) || (rc = c.view(v, rt, 1, &kc)) || (rc = c.view(v, rt, 2, &vc)) ||
            (rc = c.view(v, rt, 3, &starts)) || (rc = c.view(v, rt, 4, &out)))
          return rc;
        return rxw8_gqa_prefill_into(rt, q, kc, vc, starts, o.scale, out);
      });
}

}  // extern "C"
