// K1: W8A16 decode GEMV / skinny GEMM on gfx950 MFMA.
//
//   y[m, n] = bf16( sum_g s[n, g] * sum_{k in g} bf16(x[m, k]) * (u8[n, k] - 128) )
//
// Layout: u8 weights [N, K] row-major (RXLA's U8 = int8 + 128 storage,
// crates/rxla-nn/src/layers.rs:277-287), f32 scales [N, K/G], activations
// [M, K] bf16 (or f32, rounded to bf16 on load), output [M, N] bf16 or f32.
//
// Mapping: one wave owns 16 output channels; a 256-thread workgroup owns 64
// channels and one K-split of length Kc = K / ksplit. Every lane streams
// 16-byte slices of one weight row (lane = row + 16 * slice), so a wave load
// covers 16 rows x 64 contiguous bytes. The 16 codes of a slice become two
// bf16x8 A-fragments of v_mfma_f32_16x16x32_bf16 (u8 -> f32 -> bf16 is exact
// for 0..255); the activations are the B operand (batch rows as columns).
// The -128 offset is folded exactly by a second MFMA with an all-ones A
// operand, which yields sum_k x[m, k] per column: acc - 128 * ones.
// Scales are applied per group (G a multiple of 64) or once per channel
// (G == K) after accumulation. Split-K partials are reduced deterministically
// by the last-arriving workgroup of each 64-channel tile.
#include <type_traits>
#include "common.h"

struct GemvArgs {
  const void *x;      // [M, K] bf16 or f32
  const void *w;      // [N, K] u8 (or bf16 for the dense variant)
  const float *scale; // [N, K / G] (unused for the dense variant)
  void *y;            // [M, N] bf16 or f32
  float *ws;          // [ksplit, M, N] split-K partials
  unsigned *counters; // [ceil(N / 64)] split-K arrival counters (zeroed once)
  int M, N, K, G;     // G == K for per-channel scales
  int ksplit;
  int x_f32, y_f32;
};

namespace {

constexpr int kRowsPerWave = 16;
constexpr int kWaves = 4;
constexpr int kRowsPerBlock = kRowsPerWave * kWaves;

template <int MB>
__device__ __forceinline__ void store_out(const GemvArgs &a, int b, int n, f32x4 v) {
  if (b >= a.M) return;
  if (a.y_f32) {
    float4 o = {round_bf16(v[0]), round_bf16(v[1]), round_bf16(v[2]), round_bf16(v[3])};
    *(float4 *)((float *)a.y + (int64_t)b * a.N + n) = o;
  } else {
    uint2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    *(uint2 *)((uint16_t *)a.y + (int64_t)b * a.N + n) = o;
  }
}

// Finish a 16-channel x (16*MB) batch tile: either write it out (ksplit == 1)
// or publish the partial and let the last workgroup reduce.
template <int MB>
__device__ __forceinline__ void finish_tile(const GemvArgs &a, bool active, int row0,
                                            int sp, f32x4 (&total)[MB], bool per_channel) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, col = lane & 15;
  const int n = row0 + 4 * j;
  f32x4 sc = {1.f, 1.f, 1.f, 1.f};
  if (active && per_channel) {
    const float4 s4 = *(const float4 *)(a.scale + n);
    sc[0] = s4.x; sc[1] = s4.y; sc[2] = s4.z; sc[3] = s4.w;
  }
  if (a.ksplit == 1) {
    if (active)
      for (int mb = 0; mb < MB; ++mb) store_out<MB>(a, col + 16 * mb, n, total[mb] * sc);
    return;
  }
  if (active)
    for (int mb = 0; mb < MB; ++mb) {
      const int b = col + 16 * mb;
      if (b < a.M) *(f32x4 *)(a.ws + ((int64_t)sp * a.M + b) * a.N + n) = total[mb];
    }
  const int tile = blockIdx.x / a.ksplit;
  if (!splitk_arrive(a.counters + tile, (unsigned)a.ksplit)) return;
  if (!active) return;
  for (int mb = 0; mb < MB; ++mb) {
    const int b = col + 16 * mb;
    if (b >= a.M) continue;
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < a.ksplit; ++s) {
      const float *p = a.ws + ((int64_t)s * a.M + b) * a.N + n;
      for (int i = 0; i < 4; ++i)
        sum[i] += __hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    store_out<MB>(a, b, n, sum * sc);
  }
}

// Process NU consecutive 64-k chunks starting at chunk c (relative to k0).
template <int MB, int NU>
__device__ __forceinline__ void w8_chunks(const GemvArgs &a, const uint8_t *wrow, int k0,
                                          int c, int row0, int chunks_per_group,
                                          bool per_channel, f32x4 (&acc)[MB],
                                          f32x4 (&ones)[MB], f32x4 (&total)[MB]) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, col = lane & 15;
  u32x4 wv[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u)
    wv[u] = __builtin_nontemporal_load((const u32x4 *)(wrow + (int64_t)(c + u) * 64));
  u32x4 xv[NU][MB][2];
#pragma unroll
  for (int u = 0; u < NU; ++u)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int b = col + 16 * mb;
      if (b < a.M) {
        const int64_t off = (int64_t)b * a.K + k0 + (int64_t)(c + u) * 64 + j * 16;
        xv[u][mb][0] = load_x8(a.x, off, a.x_f32);
        xv[u][mb][1] = load_x8(a.x, off + 8, a.x_f32);
      } else {
        xv[u][mb][0] = u32x4{0, 0, 0, 0};
        xv[u][mb][1] = u32x4{0, 0, 0, 0};
      }
    }
  const u32x4 ones_bits = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  const bf16x8 onesf = as_bf16x8(ones_bits);
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const uint2 p0 = u8x4_to_bf16x4(wv[u][0]), p1 = u8x4_to_bf16x4(wv[u][1]);
    const uint2 p2 = u8x4_to_bf16x4(wv[u][2]), p3 = u8x4_to_bf16x4(wv[u][3]);
    const u32x4 a0 = {p0.x, p0.y, p1.x, p1.y}, a1 = {p2.x, p2.y, p3.x, p3.y};
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const bf16x8 x0 = as_bf16x8(xv[u][mb][0]), x1 = as_bf16x8(xv[u][mb][1]);
      acc[mb] = mfma16x16x32(as_bf16x8(a0), x0, acc[mb]);
      acc[mb] = mfma16x16x32(as_bf16x8(a1), x1, acc[mb]);
      ones[mb] = mfma16x16x32(onesf, x0, ones[mb]);
      ones[mb] = mfma16x16x32(onesf, x1, ones[mb]);
    }
    if (!per_channel && ((c + u + 1) % chunks_per_group) == 0) {
      // fold one scale group: total += s[n, g] * (acc - 128 * ones)
      const int groups = a.K / a.G;
      const int g = (k0 + (c + u) * 64) / a.G;
      f32x4 sc;
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[i] = a.scale[(int64_t)(row0 + 4 * j + i) * groups + g];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        total[mb] += sc * (acc[mb] - 128.f * ones[mb]);
        acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
        ones[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  }
}

template <int MB, int U>
__device__ __forceinline__ void gemv_w8(const GemvArgs &a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tile = blockIdx.x / a.ksplit;
  const int sp = blockIdx.x - tile * a.ksplit;
  const int Kc = a.K / a.ksplit;
  const int k0 = sp * Kc;
  const int row0 = tile * kRowsPerBlock + wave * kRowsPerWave;
  const bool active = row0 < a.N;
  const bool per_channel = a.G == a.K;
  const int chunks = Kc / 64;
  const int chunks_per_group = per_channel ? chunks : a.G / 64;

  f32x4 acc[MB], ones[MB], total[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    ones[mb] = acc[mb];
    total[mb] = acc[mb];
  }
  if (active) {
    const int r = lane & 15, j = lane >> 4;
    const uint8_t *wrow = (const uint8_t *)a.w + (int64_t)(row0 + r) * a.K + k0 + j * 16;
    int c = 0;
    for (; c + U <= chunks; c += U)
      w8_chunks<MB, U>(a, wrow, k0, c, row0, chunks_per_group, per_channel, acc, ones, total);
    for (; c < chunks; ++c)
      w8_chunks<MB, 1>(a, wrow, k0, c, row0, chunks_per_group, per_channel, acc, ones, total);
    if (per_channel)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) total[mb] = acc[mb] - 128.f * ones[mb];
  }
  finish_tile<MB>(a, active, row0, sp, total, per_channel);
}

// Dense bf16 weights (lm_head): one 16-byte slice = one MFMA A-fragment.
template <int MB, int U>
__device__ __forceinline__ void gemv_bf16(const GemvArgs &a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tile = blockIdx.x / a.ksplit;
  const int sp = blockIdx.x - tile * a.ksplit;
  const int Kc = a.K / a.ksplit;
  const int k0 = sp * Kc;
  const int row0 = tile * kRowsPerBlock + wave * kRowsPerWave;
  const bool active = row0 < a.N;
  const int r = lane & 15, j = lane >> 4, col = lane & 15;
  f32x4 total[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) total[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (active) {
    const uint16_t *wrow = (const uint16_t *)a.w + (int64_t)(row0 + r) * a.K + k0 + j * 8;
    const int steps = Kc / 32;
    int c = 0;
    auto run = [&](auto nu_tag) {
      constexpr int NU = decltype(nu_tag)::value;
      u32x4 wv[NU];
#pragma unroll
      for (int u = 0; u < NU; ++u)
        wv[u] = __builtin_nontemporal_load((const u32x4 *)(wrow + (int64_t)(c + u) * 32));
      u32x4 xv[NU][MB];
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int b = col + 16 * mb;
          xv[u][mb] = b < a.M ? load_x8(a.x, (int64_t)b * a.K + k0 + (int64_t)(c + u) * 32 + j * 8,
                                        a.x_f32)
                              : u32x4{0, 0, 0, 0};
        }
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          total[mb] = mfma16x16x32(as_bf16x8(wv[u]), as_bf16x8(xv[u][mb]), total[mb]);
    };
    for (; c + U <= steps; c += U) run(std::integral_constant<int, U>{});
    for (; c < steps; ++c) run(std::integral_constant<int, 1>{});
  }
  // no scale for dense weights: finish with scale 1
  const int jj = lane >> 4;
  const int n = row0 + 4 * jj;
  if (a.ksplit == 1) {
    if (active)
      for (int mb = 0; mb < MB; ++mb) store_out<MB>(a, col + 16 * mb, n, total[mb]);
    return;
  }
  if (active)
    for (int mb = 0; mb < MB; ++mb) {
      const int b = col + 16 * mb;
      if (b < a.M) *(f32x4 *)(a.ws + ((int64_t)sp * a.M + b) * a.N + n) = total[mb];
    }
  if (!splitk_arrive(a.counters + tile, (unsigned)a.ksplit)) return;
  if (!active) return;
  for (int mb = 0; mb < MB; ++mb) {
    const int b = col + 16 * mb;
    if (b >= a.M) continue;
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < a.ksplit; ++s) {
      const float *p = a.ws + ((int64_t)s * a.M + b) * a.N + n;
      for (int i = 0; i < 4; ++i)
        sum[i] += __hip_atomic_load(p + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    store_out<MB>(a, b, n, sum);
  }
}

}  // namespace

#define RXW8_GEMV_W8(MB, U)                                                          \
  extern "C" __global__ void __launch_bounds__(256) rxw8_gemv_w8_mb##MB(GemvArgs a) { \
    gemv_w8<MB, U>(a);                                                               \
  }
RXW8_GEMV_W8(1, 8)
RXW8_GEMV_W8(2, 4)
RXW8_GEMV_W8(4, 2)

#define RXW8_GEMV_BF16(MB, U)                                                          \
  extern "C" __global__ void __launch_bounds__(256) rxw8_gemv_bf16_mb##MB(GemvArgs a) { \
    gemv_bf16<MB, U>(a);                                                               \
  }
RXW8_GEMV_BF16(1, 8)
RXW8_GEMV_BF16(2, 4)
RXW8_GEMV_BF16(4, 2)
