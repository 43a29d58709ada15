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

  hipFunction_t fn(const char *name);
};

// Device-side allocation through the runtime's cache.
int rt_alloc(Runtime *rt, size_t bytes, void **out);
void rt_free(Runtime *rt, void *ptr, size_t bytes);
int ensure_workspace(Runtime *rt, Workspace &ws, size_t bytes, bool zero);
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
