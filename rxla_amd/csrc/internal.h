// Internal runtime structures shared by runtime.cpp, ops.cpp and decoder.cpp.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "rxw8.h"

namespace rxw8 {

// GEMV options. Activation prologue (applied while the activations are
// staged): mode 0 plain rows; 1 RMSNorm of f32 rows (norm_w, eps); 2 SwiGLU of
// bf16 gate|up rows; 3 RMSNorm with the rows' sums of squares taken from
// ss_in (ss_parts producer partials). stride/off: source row stride and offset
// in elements (0 = dense rows). prefer_ks1: one launch without a split-K
// reduce kernel. Epilogue: swiglu (weights in 8 gate + 8 up row tiles, y bf16
// [M, N/2]) and ss_out (per-16-channel sums of squares of the updated
// residual, with y_mode 1); both need the single-launch plan.
struct GemvOptions {
  int mode = 0;
  int64_t stride = 0, off = 0;
  const float *norm_w = nullptr;
  float eps = 0.f;
  const float *ss_in = nullptr;
  int ss_parts = 0;
  bool prefer_ks1 = false;
  bool swiglu = false;
  float *ss_out = nullptr;
  // mode 0 with bf16 rows x = bf16(h * norm weight): multiply row b's result
  // by 1/sqrt(sum_p ss_in[p * M + b] / K + eps) (ss_in, ss_parts, eps above)
  bool row_norm = false;
  // y_mode 1 with ss_out: also write xw_out[b, n] = bf16(h_new[b, n] * xw_norm[n])
  const float *xw_norm = nullptr;
  uint16_t *xw_out = nullptr;
  // compute dtype F32 (packed weights): f32 x rows split into bf16 hi + lo
  // parts, exact codes u - 128, f32 results without bf16 rounding (modes 0,
  // 1, 3; y_mode 0 / 1 and swiglu; no row_norm / xw_out)
  bool f32c = false;
};

// Records the thread-local error message and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t err, const char *what);

#define RXW8_HIP(expr)                                        \
  do {                                                        \
    hipError_t e_ = (expr);                                   \
    if (e_ != hipSuccess) return ::rxw8::hip_fail(e_, #expr); \
  } while (0)

size_t dtype_size(int dtype);
const char *dtype_name(int dtype);

// Decode-step attention that also applies q/k RMSNorm + RoPE and appends the
// new k/v (one new token per row; see rxw8_gqa_decode_d128_g*).
struct AttnRope {
  const uint16_t *qkv;           // [R, Hq + 2 Hkv, D] bf16 projection rows
  const float *q_norm, *k_norm;  // [D] or null
  const float *table;            // [Lmax, D] RoPE table (cos then sin per position)
  float eps;                     // the new token of row r sits at lens[r] - 1
};

struct Runtime;

struct Buffer {
  Runtime *rt = nullptr;
  int dtype = 0;
  int rank = 0;
  int64_t dims[RXW8_MAX_RANK] = {0};
  size_t bytes = 0;
  void *ptr = nullptr;
  bool owned = true;
  std::atomic<int> refs{1};

  // (buffer_extent admitted the shape: the product fits int64)
  int64_t numel() const {
    int64_t n = 1;
    for (int i = 0; i < rank; ++i) n *= dims[i];
    return n;
  }
};

// A split-K / scratch workspace owned by the runtime; grown on demand.
struct Workspace {
  void *ptr = nullptr;
  size_t bytes = 0;
};

struct Runtime {
  int device = 0;
  int cus = 0;
  size_t lds_max = 65536;  // LDS bytes one workgroup may allocate (160 KiB on gfx950)
  std::string name;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  std::vector<hipModule_t> modules;
  std::unordered_map<std::string, hipFunction_t> functions;
  std::recursive_mutex mu;
  std::atomic<int> refs{1};
  bool destroyed = false;
  // caching allocator: size -> free blocks (stream-ordered reuse)
  std::multimap<size_t, void *> free_blocks;
  size_t cached_bytes = 0;
  // workspaces
  Workspace partials;  // f32 split-K partials
  Workspace scratch;   // general f32 scratch (attention split-K)
  Workspace xcast;     // bf16 copy of f32 activations ahead of the GEMM
  Workspace wdeq;      // bf16 dequantised weights ahead of the large-M GEMM
  Workspace attn_counters;  // i32 split arrival counters of decode attention (zeroed once)

  hipFunction_t fn(const char *name);
};

// y[M,N] = x . W^T on the GEMV kernels (u8 or bf16 weights, row-major or
// packed). RXW8_UNIMPLEMENTED (nothing launched) when no GEMV tiling fits.
// Whether gemv_launch can run [M,K] x [N,K]^T (u8 weights, group G) in one
// launch (no split-K reduce), as the fused epilogues require.
bool gemv_single_launch(const Runtime *rt, int64_t M, int64_t N, int64_t K, int64_t G);
int gemv_launch(Runtime *rt, const void *x, int x_f32, const void *w, bool w_bf16, bool packed,
                const float *scale, void *y, int y_f32, int64_t M, int64_t N, int64_t K, int64_t G,
                int y_mode, const GemvOptions &pro);


// Caller-provided attention workspace (split partials and arrival counters)
// used in place of the runtime's own, which would grow on demand. A launch
// whose plan needs more than either capacity fails with RESOURCE_EXHAUSTED
// and launches nothing. The counters must be zero before the first use; the
// kernel re-arms each one it uses to zero.
struct AttnWorkspace {
  float *partials = nullptr;
  size_t partial_bytes = 0;
  int *counters = nullptr;
  size_t counter_bytes = 0;
};

// Decode attention over a contiguous [R|B, Hkv, Lmax, D] cache (ops.cpp).
int attention_launch(Runtime *rt, const void *q, int q_f32, const void *kc, const void *vc,
                     int cache_f32, const int32_t *lens, const int32_t *row_seq,
                     const float *mask, int64_t mask_sb, int64_t mask_sh, void *out, int out_f32,
                     int64_t R, int64_t Hq, int64_t Hkv, int64_t Lmax, int64_t D, float scale,
                     const AttnRope *rope = nullptr, const AttnWorkspace *ws = nullptr);

// rxw8_gqa_decode_into with an optional caller workspace (ops.cpp).
int gqa_decode_into(Runtime *rt, Buffer *q, Buffer *k_cache, Buffer *v_cache, Buffer *lens,
                    Buffer *mask, float scale, Buffer *out, const AttnWorkspace *ws);

// Takes the device address of the no-allocation scratch array on `device`
// (current) and clears its counters on `stream`; once per device (noalloc.hip).
int noalloc_device_setup(int device, hipStream_t stream);

// Device-side allocation through the runtime's cache.
int rt_alloc(Runtime *rt, size_t bytes, void **out);
void rt_free(Runtime *rt, void *ptr, size_t bytes);
int ensure_workspace(Runtime *rt, Workspace &ws, size_t bytes, bool zero);
// Validates a buffer shape (known dtype, rank <= RXW8_MAX_RANK, dims >= 0,
// element count and byte size within int64 by checked products) and returns
// its byte size; INVALID_ARGUMENT otherwise. Every buffer is created through
// it, so Buffer::numel cannot overflow.
int buffer_extent(int dtype, const int64_t *dims, int rank, size_t *bytes);
// New owned buffer (uninitialised contents unless zero).
int new_buffer(Runtime *rt, int dtype, const int64_t *dims, int rank, bool zero,
               Buffer **out);
void runtime_release(Runtime *rt);

// Launch helper: kernel takes one by-value struct argument.
template <typename Args>
int launch(Runtime *rt, const char *kernel, dim3 grid, dim3 block, const Args &args,
           size_t shmem = 0) {
  hipFunction_t f = rt->fn(kernel);
  if (!f) return fail(RXW8_INTERNAL, "kernel %s not found in the loaded code objects", kernel);
  Args copy = args;
  void *params[] = {&copy};
  RXW8_HIP(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                 (unsigned)shmem, rt->stream, params, nullptr));
  return RXW8_OK;
}

std::string dims_str(const Buffer *b);

}  // namespace rxw8

struct rxw8_runtime : rxw8::Runtime {};
struct rxw8_buffer : rxw8::Buffer {};
