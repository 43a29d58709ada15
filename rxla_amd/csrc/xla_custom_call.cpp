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
#include <dlfcn.h>

#include <cmath>
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

}  // extern "C"
