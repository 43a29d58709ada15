// Decode attention that allocates nothing: rxw8_gqa_decode_noalloc.
//
// The split-K decode attention keeps per-split (max, sum, acc) partials and
// per-(row, kv head) arrival counters in device memory beyond its inputs and
// outputs. rxw8_gqa_decode_into takes them from runtime workspaces that grow
// with hipMalloc on demand; callers that cannot allocate (code under HIP graph
// capture, serving loops that forbid allocation) use this entry point, whose
// workspace is the file-scope device array `scratch` below: each GPU holds its
// own copy for the life of the process.
//
// `scratch` is a host-side stand-in in host code, not a device address. Its
// address on a device is taken once, with that device current, by
// noalloc_device_setup (called from rxw8_runtime_create) through
// hipGetSymbolAddress, and only that address is used afterwards.
//
// Every call on one GPU shares that GPU's array: calls that overlap on one GPU
// (two streams, two runtimes, two host threads) race and must be serialised by
// the caller. The counter region starts zeroed (set-up clears it) and every
// launch re-arms each counter it uses to zero, so it is zero again whenever no
// call is in flight.
#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.h"

// Counters first (16384 (row, kv head) pairs), then the split partials.
static constexpr size_t kCounterBytes = RXW8_NOALLOC_COUNTER_BYTES;
static constexpr size_t kPartialBytes = RXW8_NOALLOC_PARTIAL_BYTES;
static constexpr size_t kScratchBytes = kCounterBytes + kPartialBytes;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices] = {nullptr};  // device address of `scratch`, per device

}  // namespace

namespace rxw8 {

// Once per device, with that device current: the device address of `scratch`
// and a cleared counter region (cleared on `stream`, the creating runtime's
// own new stream, and waited for there: no device-wide synchronisation, which
// would stall other streams and break a capture in progress elsewhere).
int noalloc_device_setup(int device, hipStream_t stream) {
  if (device < 0 || device >= kMaxDevices)
    return fail(RXW8_INVALID_ARGUMENT, "device %d outside [0, %d) for the no-allocation scratch",
                device, kMaxDevices);
  std::lock_guard<std::mutex> g(g_mu);
  if (g_ptr[device]) return RXW8_OK;
  void *ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr) return hip_fail(e, "hipGetSymbolAddress(scratch)");
  e = hipMemsetAsync(ptr, 0, kCounterBytes, stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemsetAsync(scratch counters)");
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  g_ptr[device] = ptr;
  return RXW8_OK;
}

}  // namespace rxw8

using namespace rxw8;

extern "C" {

int rxw8_gqa_decode_noalloc(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k_cache,
                            rxw8_buffer *v_cache, rxw8_buffer *lens, rxw8_buffer *mask,
                            float scale, rxw8_buffer *out) {
  if (!rt) return fail(RXW8_INVALID_ARGUMENT, "runtime is NULL");
  void *base = nullptr;
  {
    std::lock_guard<std::mutex> g(g_mu);
    if (rt->device >= 0 && rt->device < kMaxDevices) base = g_ptr[rt->device];
  }
  if (!base)
    return fail(RXW8_FAILED_PRECONDITION, "no-allocation scratch is not set up on device %d",
                rt->device);
  AttnWorkspace ws;
  ws.counters = (int *)base;
  ws.counter_bytes = kCounterBytes;
  ws.partials = (float *)((unsigned char *)base + kCounterBytes);
  ws.partial_bytes = kPartialBytes;
  return gqa_decode_into(rt, q, k_cache, v_cache, lens, mask, scale, out, &ws);
}

}  // extern "C"
