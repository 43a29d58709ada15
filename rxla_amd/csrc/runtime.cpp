// rxw8 runtime: status/error model, device runtime + stream, refcounted device
// buffers with a stream-ordered caching allocator, and gfx950 code objects
// loaded with hipModuleLoadData (the kernels are embedded in this library).
//
// Mirrors the ownership rules of crates/rxla-pjrt/src/runtime.rs: buffers
// retain their runtime (Buffer/BufferInner :1446,:1523), status codes follow
// PJRT_Error_Code (vendor/xla/pjrt/c/pjrt_c_api.h:168-186) and
// PjrtErrorCode::is_retryable (:93-104).
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "internal.h"

// Code objects embedded by kernels_blob.S (.incbin of the gfx950 .hsaco files).
extern "C" {
extern const unsigned char rxw8_co_gemv[], rxw8_co_gemv_end[];
extern const unsigned char rxw8_co_gemv_rc[], rxw8_co_gemv_rc_end[];
extern const unsigned char rxw8_co_misc[], rxw8_co_misc_end[];
extern const unsigned char rxw8_co_attention[], rxw8_co_attention_end[];
extern const unsigned char rxw8_co_gemm[], rxw8_co_gemm_end[];
extern const unsigned char rxw8_co_decoder[], rxw8_co_decoder_end[];
extern const unsigned char rxw8_co_qwen35[], rxw8_co_qwen35_end[];
}

namespace rxw8 {

static thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t err, const char *what) {
  int code = RXW8_INTERNAL;
  if (err == hipErrorOutOfMemory || err == hipErrorMemoryAllocation)
    code = RXW8_RESOURCE_EXHAUSTED;
  else if (err == hipErrorNoDevice || err == hipErrorInvalidDevice)
    code = RXW8_FAILED_PRECONDITION;
  else if (err == hipErrorNotReady)
    code = RXW8_UNAVAILABLE;
  return fail(code, "HIP error %d (%s) in %s", (int)err, hipGetErrorString(err), what);
}

size_t dtype_size(int dtype) {
  switch (dtype) {
    case RXW8_U8: return 1;
    case RXW8_I32: return 4;
    case RXW8_F16: return 2;
    case RXW8_BF16: return 2;
    case RXW8_F32: return 4;
    default: return 0;
  }
}

const char *dtype_name(int dtype) {
  switch (dtype) {
    case RXW8_U8: return "U8";
    case RXW8_I32: return "I32";
    case RXW8_F16: return "F16";
    case RXW8_BF16: return "BF16";
    case RXW8_F32: return "F32";
    default: return "?";
  }
}

std::string dims_str(const Buffer *b) {
  std::string s = "[";
  for (int i = 0; i < b->rank; ++i) {
    if (i) s += ",";
    s += std::to_string(b->dims[i]);
  }
  return s + "]";
}

// Code object holding a kernel, by name prefix (index into `modules`, in the
// load order of runtime_create). Looking a kernel up only where it lives keeps
// hipModuleGetFunction from failing: a failed call would leave HIP's per-thread
// last error set, and the caller's next HIP API check (torch's included)
// would report it as its own.
static int module_of(const char *kname) {
  static const struct {
    const char *prefix;
    int module;
  } routes[] = {{"rxw8_gemv_rc_", 6}, {"rxw8_gemv_", 0},      {"rxw8_pack_tiles", 0},     {"rxw8_dequant", 1},
                {"rxw8_linear_generic", 1}, {"rxw8_linear_f32_", 1}, {"rxw8_kv_update", 1},
                {"rxw8_quantize_w8", 1},
                {"rxw8_gqa_", 2},
                {"rxw8_w8a16_gemm", 3}, {"rxw8_gemm_", 3},   {"rxw8_dec_", 4},
                {"rxw8_q35_", 5}};
  for (const auto &r : routes)
    if (std::strncmp(kname, r.prefix, std::strlen(r.prefix)) == 0) return r.module;
  return -1;
}

hipFunction_t Runtime::fn(const char *kname) {
  auto it = functions.find(kname);
  if (it != functions.end()) return it->second;
  const int mi = module_of(kname);
  if (mi < 0 || mi >= (int)modules.size()) return nullptr;
  hipFunction_t f = nullptr;
  if (hipModuleGetFunction(&f, modules[mi], kname) == hipSuccess && f) {
    functions.emplace(kname, f);
    return f;
  }
  (void)hipGetLastError();  // internal naming error; reported by the caller
  return nullptr;
}

static size_t round_size(size_t bytes) {
  const size_t align = 256;
  if (bytes == 0) bytes = align;
  return (bytes + align - 1) / align * align;
}

int rt_alloc(Runtime *rt, size_t bytes, void **out) {
  bytes = round_size(bytes);
  auto it = rt->free_blocks.find(bytes);
  if (it != rt->free_blocks.end()) {
    *out = it->second;
    rt->cached_bytes -= bytes;
    rt->free_blocks.erase(it);
    return RXW8_OK;
  }
  hipError_t e = hipMalloc(out, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    // release the cache and retry once
    RXW8_HIP(hipStreamSynchronize(rt->stream));
    for (auto &kv : rt->free_blocks) (void)hipFree(kv.second);
    rt->free_blocks.clear();
    rt->cached_bytes = 0;
    e = hipMalloc(out, bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  }
  return RXW8_OK;
}

void rt_free(Runtime *rt, void *ptr, size_t bytes) {
  if (!ptr) return;
  bytes = round_size(bytes);
  // Stream-ordered reuse: later work on the same stream runs after every
  // kernel that used this block.
  rt->free_blocks.emplace(bytes, ptr);
  rt->cached_bytes += bytes;
}

int ensure_workspace(Runtime *rt, Workspace &ws, size_t bytes, bool zero) {
  if (ws.bytes >= bytes) return RXW8_OK;
  // Growing synchronizes the stream and reallocates: not possible inside a
  // stream capture (an XLA command buffer, a caller's graph). Such callers
  // run the call once outside capture first, which sizes the workspace.
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(rt->stream, &cs) != hipSuccess) {
    (void)hipGetLastError();
    cs = hipStreamCaptureStatusNone;
  }
  if (cs != hipStreamCaptureStatusNone)
    return fail(RXW8_FAILED_PRECONDITION,
                "a workspace of %zu bytes (now %zu) must grow while the stream is being captured; "
                "run the call once outside the capture first",
                bytes, ws.bytes);
  if (ws.ptr) {
    RXW8_HIP(hipStreamSynchronize(rt->stream));
    RXW8_HIP(hipFree(ws.ptr));
    ws.ptr = nullptr;
    ws.bytes = 0;
  }
  size_t want = round_size(bytes < (1u << 20) ? (1u << 20) : bytes);
  RXW8_HIP(hipMalloc(&ws.ptr, want));
  if (zero) {
    RXW8_HIP(hipMemsetAsync(ws.ptr, 0, want, rt->stream));
    RXW8_HIP(hipStreamSynchronize(rt->stream));
  }
  ws.bytes = want;
  return RXW8_OK;
}

int buffer_extent(int dtype, const int64_t *dims, int rank, size_t *bytes) {
  const size_t esz = dtype_size(dtype);
  if (esz == 0) return fail(RXW8_INVALID_ARGUMENT, "unsupported dtype %d", dtype);
  if (rank < 0 || rank > RXW8_MAX_RANK)
    return fail(RXW8_INVALID_ARGUMENT, "rank %d outside [0, %d]", rank, RXW8_MAX_RANK);
  if (rank > 0 && !dims) return fail(RXW8_INVALID_ARGUMENT, "dims is NULL");
  bool empty = false;
  for (int i = 0; i < rank; ++i) {
    if (dims[i] < 0) return fail(RXW8_INVALID_ARGUMENT, "negative dimension %lld", (long long)dims[i]);
    empty = empty || dims[i] == 0;
  }
  // checked products: the element count and the byte size must fit int64
  int64_t n = 1;
  for (int i = 0; i < rank && !empty; ++i)
    if (__builtin_mul_overflow(n, dims[i], &n))
      return fail(RXW8_INVALID_ARGUMENT, "shape overflows a 64-bit element count");
  int64_t total = 0;
  if (!empty && __builtin_mul_overflow(n, (int64_t)esz, &total))
    return fail(RXW8_INVALID_ARGUMENT, "shape overflows a 64-bit byte size");
  *bytes = (size_t)total;
  return RXW8_OK;
}

int new_buffer(Runtime *rt, int dtype, const int64_t *dims, int rank, bool zero,
               Buffer **out) {
  size_t bytes = 0;
  if (int rc = buffer_extent(dtype, dims, rank, &bytes)) return rc;
  auto *b = new rxw8_buffer();
  b->rt = rt;
  b->dtype = dtype;
  b->rank = rank;
  for (int i = 0; i < rank; ++i) b->dims[i] = dims[i];
  b->bytes = bytes;
  int rc = rt_alloc(rt, b->bytes, &b->ptr);
  if (rc) {
    delete b;
    return rc;
  }
  if (zero && b->bytes) {
    hipError_t e = hipMemsetAsync(b->ptr, 0, b->bytes, rt->stream);
    if (e != hipSuccess) {
      rt_free(rt, b->ptr, b->bytes);
      delete b;
      return hip_fail(e, "hipMemsetAsync");
    }
  }
  rt->refs.fetch_add(1);
  *out = b;
  return RXW8_OK;
}

static void runtime_free(Runtime *rt) {
  if (rt->stream) (void)hipStreamSynchronize(rt->stream);
  for (auto &kv : rt->free_blocks) (void)hipFree(kv.second);
  for (Workspace *w : {&rt->partials, &rt->scratch, &rt->xcast, &rt->wdeq, &rt->attn_counters})
    if (w->ptr) (void)hipFree(w->ptr);
  for (hipModule_t m : rt->modules) (void)hipModuleUnload(m);
  if (rt->own_stream) (void)hipStreamDestroy(rt->own_stream);
  delete static_cast<rxw8_runtime *>(rt);
}

void runtime_release(Runtime *rt) {
  if (rt->refs.fetch_sub(1) == 1) runtime_free(rt);
}

}  // namespace rxw8

using namespace rxw8;

extern "C" {

const char *rxw8_last_error(void) { return g_last_error.c_str(); }

int rxw8_status_is_retryable(int status) {
  return status == RXW8_CANCELLED || status == RXW8_DEADLINE_EXCEEDED ||
         status == RXW8_RESOURCE_EXHAUSTED || status == RXW8_ABORTED ||
         status == RXW8_UNAVAILABLE;
}

int rxw8_abi_version(void) { return RXW8_ABI_VERSION; }

int rxw8_runtime_create(int device, rxw8_runtime **out) {
  if (!out) return fail(RXW8_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) {
    (void)hipGetLastError();
    return fail(RXW8_FAILED_PRECONDITION, "no HIP device available");
  }
  if (device < 0 || device >= count)
    return fail(RXW8_INVALID_ARGUMENT, "device %d outside [0, %d)", device, count);
  RXW8_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  RXW8_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(RXW8_FAILED_PRECONDITION, "device %d is %s; rxw8 kernels are built for gfx950",
                device, prop.gcnArchName);
  auto *rt = new rxw8_runtime();
  rt->device = device;
  rt->cus = prop.multiProcessorCount;
  rt->lds_max = prop.sharedMemPerBlock;
  rt->name = prop.name;
  const struct {
    const char *name;
    const unsigned char *begin, *end;
  } blobs[] = {{"gemv", rxw8_co_gemv, rxw8_co_gemv_end},
               {"misc", rxw8_co_misc, rxw8_co_misc_end},
               {"attention", rxw8_co_attention, rxw8_co_attention_end},
               {"gemm", rxw8_co_gemm, rxw8_co_gemm_end},
               {"decoder", rxw8_co_decoder, rxw8_co_decoder_end},
               {"qwen35", rxw8_co_qwen35, rxw8_co_qwen35_end},
               {"gemv_rc", rxw8_co_gemv_rc, rxw8_co_gemv_rc_end}};
  for (auto &blob : blobs) {  // order = module indices of module_of()
    if (blob.end - blob.begin <= 0) {
      for (hipModule_t mm : rt->modules) (void)hipModuleUnload(mm);
      delete rt;
      return fail(RXW8_INTERNAL, "embedded code object %s is empty", blob.name);
    }
    hipModule_t m = nullptr;
    e = hipModuleLoadData(&m, blob.begin);
    if (e != hipSuccess) {
      int rc = hip_fail(e, "hipModuleLoadData");
      for (hipModule_t mm : rt->modules) (void)hipModuleUnload(mm);
      delete rt;
      return rc;
    }
    rt->modules.push_back(m);
  }
  e = hipStreamCreateWithFlags(&rt->own_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    int rc = hip_fail(e, "hipStreamCreateWithFlags");
    for (hipModule_t mm : rt->modules) (void)hipModuleUnload(mm);
    delete rt;
    return rc;
  }
  rt->stream = rt->own_stream;
  if (int rc = noalloc_device_setup(device, rt->own_stream)) {
    (void)hipStreamDestroy(rt->own_stream);
    for (hipModule_t mm : rt->modules) (void)hipModuleUnload(mm);
    delete rt;
    return rc;
  }
  *out = rt;
  return RXW8_OK;
}

int rxw8_runtime_destroy(rxw8_runtime *rt) {
  if (!rt) return fail(RXW8_INVALID_ARGUMENT, "runtime is NULL");
  {
    std::lock_guard<std::recursive_mutex> g(rt->mu);
    if (rt->destroyed) return fail(RXW8_FAILED_PRECONDITION, "runtime already destroyed");
    rt->destroyed = true;
  }
  runtime_release(rt);
  return RXW8_OK;
}

int rxw8_runtime_set_stream(rxw8_runtime *rt, void *hip_stream) {
  if (!rt) return fail(RXW8_INVALID_ARGUMENT, "runtime is NULL");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  hipStream_t next = hip_stream ? (hipStream_t)hip_stream : rt->own_stream;
  if (next == rt->stream) return RXW8_OK;
  // Cached blocks were last used on the old stream: drain it before reuse.
  RXW8_HIP(hipStreamSynchronize(rt->stream));
  rt->stream = next;
  return RXW8_OK;
}

int rxw8_runtime_stream(rxw8_runtime *rt, void **hip_stream) {
  if (!rt || !hip_stream) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  *hip_stream = (void *)rt->stream;
  return RXW8_OK;
}

int rxw8_runtime_synchronize(rxw8_runtime *rt) {
  if (!rt) return fail(RXW8_INVALID_ARGUMENT, "runtime is NULL");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  RXW8_HIP(hipStreamSynchronize(rt->stream));
  return RXW8_OK;
}

int rxw8_runtime_device_info(rxw8_runtime *rt, int *compute_units, char *name,
                             size_t name_len) {
  if (!rt) return fail(RXW8_INVALID_ARGUMENT, "runtime is NULL");
  if (compute_units) *compute_units = rt->cus;
  if (name && name_len) {
    std::strncpy(name, rt->name.c_str(), name_len - 1);
    name[name_len - 1] = 0;
  }
  return RXW8_OK;
}

int rxw8_buffer_create(rxw8_runtime *rt, int dtype, const int64_t *dims, int rank,
                       rxw8_buffer **out) {
  size_t bytes = 0;  // the shape is validated before anything else
  if (int rc = buffer_extent(dtype, dims, rank, &bytes)) return rc;
  if (!rt || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  Buffer *b = nullptr;
  int rc = new_buffer(rt, dtype, dims, rank, true, &b);
  if (rc) return rc;
  *out = static_cast<rxw8_buffer *>(b);
  return RXW8_OK;
}

int rxw8_buffer_from_host(rxw8_runtime *rt, int dtype, const int64_t *dims, int rank,
                          const void *data, rxw8_buffer **out) {
  size_t bytes = 0;
  if (int rc = buffer_extent(dtype, dims, rank, &bytes)) return rc;
  if (!rt || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  Buffer *b = nullptr;
  int rc = new_buffer(rt, dtype, dims, rank, false, &b);
  if (rc) return rc;
  if (b->bytes) {
    if (!data) {
      rxw8_buffer_release(static_cast<rxw8_buffer *>(b));
      return fail(RXW8_INVALID_ARGUMENT, "data is NULL for a non-empty buffer");
    }
    hipError_t e = hipMemcpyAsync(b->ptr, data, b->bytes, hipMemcpyHostToDevice, rt->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
    if (e != hipSuccess) {
      rxw8_buffer_release(static_cast<rxw8_buffer *>(b));
      return hip_fail(e, "host to device copy");
    }
  }
  *out = static_cast<rxw8_buffer *>(b);
  return RXW8_OK;
}

int rxw8_buffer_wrap(rxw8_runtime *rt, int dtype, const int64_t *dims, int rank,
                     void *device_ptr, rxw8_buffer **out) {
  size_t bytes = 0;
  if (int rc = buffer_extent(dtype, dims, rank, &bytes)) return rc;
  if (!rt || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (bytes > 0 && !device_ptr) return fail(RXW8_INVALID_ARGUMENT, "device_ptr is NULL");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  auto *b = new rxw8_buffer();
  b->rt = rt;
  b->dtype = dtype;
  b->rank = rank;
  for (int i = 0; i < rank; ++i) b->dims[i] = dims[i];
  b->bytes = bytes;
  b->ptr = device_ptr;
  b->owned = false;
  rt->refs.fetch_add(1);
  *out = b;
  return RXW8_OK;
}

int rxw8_buffer_to_host(rxw8_buffer *buf, void *dst, size_t bytes) {
  if (!buf) return fail(RXW8_INVALID_ARGUMENT, "buffer is NULL");
  if (bytes != buf->bytes)
    return fail(RXW8_INVALID_ARGUMENT, "destination holds %zu bytes, buffer has %zu", bytes,
                buf->bytes);
  if (!bytes) return RXW8_OK;
  if (!dst) return fail(RXW8_INVALID_ARGUMENT, "dst is NULL");
  Runtime *rt = buf->rt;
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  RXW8_HIP(hipMemcpyAsync(dst, buf->ptr, bytes, hipMemcpyDeviceToHost, rt->stream));
  RXW8_HIP(hipStreamSynchronize(rt->stream));
  return RXW8_OK;
}

int rxw8_buffer_copy_from_host(rxw8_buffer *buf, const void *src, size_t bytes) {
  if (!buf) return fail(RXW8_INVALID_ARGUMENT, "buffer is NULL");
  if (bytes != buf->bytes)
    return fail(RXW8_INVALID_ARGUMENT, "source holds %zu bytes, buffer has %zu", bytes,
                buf->bytes);
  if (!bytes) return RXW8_OK;
  if (!src) return fail(RXW8_INVALID_ARGUMENT, "src is NULL");
  Runtime *rt = buf->rt;
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  RXW8_HIP(hipMemcpyAsync(buf->ptr, src, bytes, hipMemcpyHostToDevice, rt->stream));
  RXW8_HIP(hipStreamSynchronize(rt->stream));
  return RXW8_OK;
}

int rxw8_buffer_retain(rxw8_buffer *buf) {
  if (!buf) return fail(RXW8_INVALID_ARGUMENT, "buffer is NULL");
  buf->refs.fetch_add(1);
  return RXW8_OK;
}

int rxw8_buffer_release(rxw8_buffer *buf) {
  if (!buf) return fail(RXW8_INVALID_ARGUMENT, "buffer is NULL");
  if (buf->refs.fetch_sub(1) != 1) return RXW8_OK;
  Runtime *rt = buf->rt;
  {
    std::lock_guard<std::recursive_mutex> g(rt->mu);
    if (buf->owned) rt_free(rt, buf->ptr, buf->bytes);
  }
  delete buf;
  runtime_release(rt);
  return RXW8_OK;
}

int rxw8_buffer_dtype(const rxw8_buffer *buf, int *dtype) {
  if (!buf || !dtype) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  *dtype = buf->dtype;
  return RXW8_OK;
}

int rxw8_buffer_dims(const rxw8_buffer *buf, int64_t *dims, int *rank) {
  if (!buf || !rank) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  *rank = buf->rank;
  if (dims)
    for (int i = 0; i < buf->rank; ++i) dims[i] = buf->dims[i];
  return RXW8_OK;
}

int rxw8_buffer_device_ptr(const rxw8_buffer *buf, void **ptr) {
  if (!buf || !ptr) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  *ptr = buf->ptr;
  return RXW8_OK;
}

}  // extern "C"
