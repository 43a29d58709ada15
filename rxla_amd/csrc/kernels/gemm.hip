// K2: W8A16 prefill dequant-GEMM on gfx950 MFMA.
//
//   y[m, n] = bf16( sum_k x[m, k] * bf16((u8[n, k] - 128) * s[n, k / G]) )
//
// with x already bf16: exactly the reference's cast points (crates/rxla-nn/
// src/layers.rs:277-296): the weight is dequantised in f32 (one rounding),
// rounded to bf16, contracted against bf16 activations with f32
// accumulation, and the result rounded to bf16. (f32 activations are rounded
// to bf16 by rxw8_gemm_cast_x first, the x.cast(BF16) of the same layer.)
//
// Tiling. A 256-thread workgroup (4 waves) computes a 128 (weight rows n) x TM
// (activation rows m) output tile, TM = 256 or 128, over k tiles of BK = 64.
// Wave w owns all 128 n and the m rows [w*TM/4, (w+1)*TM/4): 8 x TM/64
// v_mfma_f32_16x16x32_bf16 accumulators with the weights as the A operand, so
// each weight fragment read from LDS feeds TM/64 MFMAs and each activation
// fragment feeds 8.
//
// Staging (double-buffered in LDS, both operands bf16, rows of 64 values =
// 128 B whose 16-byte chunks are XOR-swizzled by row & 7 so the fragment reads
// of 8 consecutive rows hit 8 different bank groups):
//   * activations go global -> LDS by global_load_lds_dwordx4 (LDS DMA: no
//     VGPRs, no VALU; see dma16); each lane picks the source chunk that lands
//     in the swizzled slot of its fixed LDS destination;
//   * int8 weights go through VGPRs and are dequantised once per workgroup:
//     fma(f32(u), s, -128 s) is the correctly rounded (u - 128) * s (the
//     exact product plus an exact addend, one rounding; -128 s is exact in f32
//     for every finite scale below 2^120), then rounded to bf16.
// The loads of k tile t+1 are issued before the MFMAs of tile t.
//
// Tile order is XCD-aware: workgroup b runs on XCD b % 8 and takes the tile
// b / 8 of that XCD's contiguous share; inside a share tiles go in groups of
// 8 n tiles with n fastest, so the workgroups an XCD runs at once cover about
// 8 n x 4 m tiles and reuse both operands from that XCD's L2.
#include "common.h"

#include <type_traits>


struct GemmArgs {
  const uint16_t *x;   // [M, K] bf16
  const uint8_t *w;    // [N, K] u8 or packed [N/16, K/64, 1024]
  const float *scale;  // [N, K / G]
  void *y;             // [M, N]
  int M, N, K, G;
  int y_f32, y_mode, w_packed;
  int group_n;         // n tiles per tile-order group of the 256 x 256 kernel (0: default)
  int ksplit;          // 256 x 256 u8 kernel: k splits (f32 partials to ws, reduced after)
  float *ws;           // [ksplit, M, N] f32 partials when ksplit > 1
};

struct CastArgs {
  const float *x;
  uint16_t *y;
  int64_t n;
};

namespace {

constexpr int TN = 128, BK = 64, GROUP_N = 8;
#ifndef RXW8_GEMM_PREFETCH
#define RXW8_GEMM_PREFETCH 2
#endif

// global -> LDS DMA of 16 bytes per lane (global_load_lds_dwordx4; lane l
// writes LDS bytes [lds + 16 l, +16)). Issued from inline asm on purpose: the
// compiler models the builtin as a flat access of both global memory and LDS
// and then answers every later LDS or VGPR-load dependency with lgkmcnt(0) /
// vmcnt(0), which serialises the fragment reads with the MFMAs. The kernels
// wait for the DMA'd data themselves (explicit vmcnt before each barrier); the
// compiler, not knowing these loads, can only over-wait for its own.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void *base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, %2"
               :: "v"(voff), "s"(lds), "s"(base) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const char *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}


// Byte offset of 16-byte chunk c (0..7) of row r in a swizzled 128-B-row tile.
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }

// Epilogue of one accumulator: lane holds y[m, n .. n+3]. Called by every
// lane of the wave (y_mode 2 exchanges values between lanes).
//   y_mode 0: bf16 or (bf16-rounded) f32 y;  1: f32 residual y += bf16(v);
//   2: SwiGLU over weight rows interleaved in 16-row tiles of 8 gate + 8 up
//      rows (16 t + j and 16 t + 8 + j are channel 8 t + j): y bf16 [M, N/2]
//      gets bf16(silu(bf16(g)) * bf16(u)) (ops.rs:331-342); the up partner of
//      a gate lane (n % 16 < 8) sits 32 lanes higher.
__device__ __forceinline__ void gemm_store(const GemmArgs &a, int m, int n, f32x4 v) {
  if (a.y_mode == 2) {
    f32x4 up;
#pragma unroll
    for (int i = 0; i < 4; ++i) up[i] = __shfl_xor(v[i], 32);
    if ((n & 15) < 8 && m < a.M) {
      const int c = (n >> 4) * 8 + (n & 7);
      *(uint2 *)((uint16_t *)a.y + (int64_t)m * (a.N / 2) + c) =
          uint2{pack_bf16x2(silu_mul_f32(round_bf16(v[0]), round_bf16(up[0])),
                            silu_mul_f32(round_bf16(v[1]), round_bf16(up[1]))),
                pack_bf16x2(silu_mul_f32(round_bf16(v[2]), round_bf16(up[2])),
                            silu_mul_f32(round_bf16(v[3]), round_bf16(up[3])))};
    }
    return;
  }
  if (m >= a.M) return;
  if (a.y_mode == 1) {
    float4 *h = (float4 *)((float *)a.y + (int64_t)m * a.N + n);
    float4 o = *h;
    o.x += round_bf16(v[0]);
    o.y += round_bf16(v[1]);
    o.z += round_bf16(v[2]);
    o.w += round_bf16(v[3]);
    *h = o;
  } else if (a.y_f32) {
    float4 o = {round_bf16(v[0]), round_bf16(v[1]), round_bf16(v[2]), round_bf16(v[3])};
    *(float4 *)((float *)a.y + (int64_t)m * a.N + n) = o;
  } else {
    uint2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    *(uint2 *)((uint16_t *)a.y + (int64_t)m * a.N + n) = o;
  }
}

template <int TM>
__device__ __forceinline__ void gemm_tile(const GemmArgs &a) {
  constexpr int WM = TM / 4;             // m rows per wave
  constexpr int FJ = WM / 16;            // m fragments per wave
  constexpr int W_BYTES = TN * BK * 2;   // bf16 weight tile
  constexpr int X_BYTES = TM * BK * 2;   // bf16 activation tile
  constexpr int STAGE = W_BYTES + X_BYTES;
  constexpr int X_DMA = TM / 32;         // LDS-DMA instructions per wave per k tile
  constexpr int LOADS = X_DMA + 4;       // vector-memory instructions per lane per k tile
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int tiles_m = (a.M + TM - 1) / TM, tiles_n = a.N / TN;
  const int ntiles = tiles_m * tiles_n;
  const int per_xcd = (ntiles + 7) / 8;
  const int t = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (t >= ntiles) return;
  const int group = t / (GROUP_N * tiles_m);
  const int first_n = group * GROUP_N;
  const int gw = min(GROUP_N, tiles_n - first_n);
  const int r = t - group * GROUP_N * tiles_m;
  const int n0 = (first_n + r % gw) * TN, m0 = (r / gw) * TM;
  const int KT = a.K / BK, groups = a.K / a.G, last = KT - 1;

  // Three LDS stages, stage s = [bf16 weight tile | bf16 activation tile];
  // k tile kt lives in stage kt % 3.
  __shared__ __attribute__((aligned(1024))) char smem[3 * STAGE];

  // activation DMA: instruction i of this wave fills LDS rows 8*(wave*X_DMA+i) ..+8;
  // lane -> row += lane / 8, physical chunk lane % 8 <- logical chunk (lane%8)^(row&7).
  // Byte offsets from x stay below 2^31 (checked by the host).
  uint32_t xoff[X_DMA];
#pragma unroll
  for (int i = 0; i < X_DMA; ++i) {
    const int row = (wave * X_DMA + i) * 8 + (lane >> 3);
    const int m = min(m0 + row, a.M - 1);  // rows past M repeat the last row (not stored)
    xoff[i] = (uint32_t)m * (uint32_t)a.K * 2u + ((uint32_t)((lane & 7) ^ (row & 7)) << 4);
  }
  const char *xbase = (const char *)a.x;
  auto issue_x = [&](int kt, int stage) {
#pragma unroll
    for (int i = 0; i < X_DMA; ++i)
      dma16(xbase, xoff[i] + (uint32_t)(kt * (BK * 2)),
            lds_addr(smem + stage * STAGE + W_BYTES + (wave * X_DMA + i) * 1024));
  };

  // weights: 512 slices of 16 codes per k tile, 2 per thread (row = id / 4,
  // kq = id % 4); G % 64 == 0, so one scale per row and k tile.
  const int kstride = a.w_packed ? 1024 : BK;  // bytes between k tiles of a slice
  uint32_t woff[2], soff[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int id = tid + 256 * p, row = id >> 2, kq = id & 3;
    const int n = n0 + row;
    woff[p] = a.w_packed
                  ? ((uint32_t)(n >> 4) * (uint32_t)KT * 1024u + (uint32_t)((row & 15) + 16 * kq) * 16u)
                  : (uint32_t)n * (uint32_t)a.K + (uint32_t)kq * 16u;
    soff[p] = (uint32_t)n * (uint32_t)groups;
  }
  struct WSet {
    u32x4 w[2];
    float s[2];
  };
  auto load_w = [&](int kt, WSet &ws) {
    const int gi = kt * BK / a.G;  // uniform
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      ws.w[p] = *(const u32x4 *)(a.w + woff[p] + (uint32_t)(kt * kstride));
      ws.s[p] = a.scale[soff[p] + gi];
    }
  };
  f32x4 acc[8][FJ];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Fragment addresses: rows 16 i + r16 share row & 7, so the swizzled chunk
  // of a fragment depends on (ks, kg, r16) only and i, j move by whole rows.
  const int r16 = lane & 15, kg = lane >> 4;
  auto frag_a = [&](int stage, int i, int ks) {
    return as_bf16x8(*(const u32x4 *)(smem + stage * STAGE + swz(16 * i + r16, ks * 4 + kg)));
  };
  auto frag_b = [&](int stage, int j, int ks) {
    return as_bf16x8(
        *(const u32x4 *)(smem + stage * STAGE + W_BYTES + swz(wave * WM + 16 * j + r16, ks * 4 + kg)));
  };

  // One piece of the dequantisation of a weight set: 4 codes of slice p,
  // dword e; after the last dword of a slice its two LDS chunks are stored.
  uint32_t hq[8];
  auto dequant_piece = [&](const WSet &ws, int piece, int stage) {
    const int p = piece >> 2, e = piece & 3;
    const float sc = ws.s[p], o = -128.0f * sc;
    const uint32_t w4 = ws.w[p][e];
    const float f0 = __builtin_fmaf((float)(w4 & 0xffu), sc, o);
    const float f1 = __builtin_fmaf((float)((w4 >> 8) & 0xffu), sc, o);
    const float f2 = __builtin_fmaf((float)((w4 >> 16) & 0xffu), sc, o);
    const float f3 = __builtin_fmaf((float)(w4 >> 24), sc, o);
    hq[2 * e] = pack_bf16x2(f0, f1);
    hq[2 * e + 1] = pack_bf16x2(f2, f3);
    if (e == 3) {
      const int id = tid + 256 * p, row = id >> 2, kq = id & 3;
      char *dst = smem + stage * STAGE;
      *(u32x4 *)(dst + swz(row, 2 * kq)) = u32x4{hq[0], hq[1], hq[2], hq[3]};
      *(u32x4 *)(dst + swz(row, 2 * kq + 1)) = u32x4{hq[4], hq[5], hq[6], hq[7]};
    }
  };

  // Pipeline: activations are DMA'd 2 k tiles ahead, weights loaded 3 ahead
  // into registers (three sets); tile kt+1's weights are dequantised into
  // LDS while tile kt is multiplied. Past the last tile the loads repeat tile
  // KT-1 into slots nobody reads again, so every k tile issues the same
  // LOADS vector-memory instructions and the wait counts below hold.
  // Barriers are plain s_barrier after explicit waits: __syncthreads()'s
  // workgroup fence would also wait for every load in flight (vmcnt(0)),
  // draining the prefetch each k tile. The "memory" clobbers keep the compiler
  // from moving LDS accesses across them.
  WSet w0, w1, w2;
  issue_x(0, 0);
  load_w(0, w0);
  issue_x(min(1, last), 1);
  load_w(min(1, last), w1);
  load_w(min(2, last), w2);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int piece = 0; piece < 8; ++piece) dequant_piece(w0, piece, 0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // One k tile in 16 groups (ks, i): the 4 (FJ) MFMAs of weight fragment i
  // run while the next fragment is read from LDS; during ks = 1 each group
  // also dequantises a piece of tile kt+1's weights. sched_barrier pins the
  // group order so register use stays at two weight fragments.
  auto step = [&](int kt, auto xs, WSet &load_set, const WSet &deq_set) {
    constexpr int cur = decltype(xs)::value, nxt = (cur + 1) % 3, fut = (cur + 2) % 3;
    issue_x(min(kt + 2, last), fut);
    load_w(min(kt + 3, last), load_set);
    bf16x8 af[2], bf[FJ], bn[FJ];
#pragma unroll
    for (int j = 0; j < FJ; ++j) bf[j] = frag_b(cur, j, 0);
    af[0] = frag_a(cur, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // ks = 0
      if (i < 7) {
        af[(i + 1) & 1] = frag_a(cur, i + 1, 0);
      } else {
        af[0] = frag_a(cur, 0, 1);
#pragma unroll
        for (int j = 0; j < FJ; ++j) bn[j] = frag_b(cur, j, 1);
      }
#pragma unroll
      for (int j = 0; j < FJ; ++j) acc[i][j] = mfma16x16x32(af[i & 1], bf[j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // weights of tile kt+1 were loaded two k tiles ago: at least the 2 * LOADS
    // instructions of the last two k tiles are younger
    if constexpr (LOADS == 12) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // ks = 1
      if (i < 7) af[(i + 1) & 1] = frag_a(cur, i + 1, 1);
#pragma unroll
      for (int j = 0; j < FJ; ++j) acc[i][j] = mfma16x16x32(af[i & 1], bn[j], acc[i][j]);
      dequant_piece(deq_set, i, nxt);
      __builtin_amdgcn_sched_barrier(0);
    }
    // activation tile kt+1 was DMA'd last k tile: this tile's LOADS are younger
    if constexpr (LOADS == 12) asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  int kt = 0;
  for (; kt + 3 <= KT; kt += 3) {
    step(kt, S0{}, w0, w1);
    step(kt + 1, S1{}, w1, w2);
    step(kt + 2, S2{}, w2, w0);
  }
  if (kt < KT) step(kt, S0{}, w0, w1);
  if (kt + 1 < KT) step(kt + 1, S1{}, w1, w2);

  // lane holds D[n = 16 i + 4 kg + r][m = 16 j + r16]
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
      gemm_store(a, m0 + wave * WM + 16 * j + r16, n0 + 16 * i + 4 * kg, acc[i][j]);
}


// 256 x 256 output tiles for long inputs: 512 threads (8 waves, two per SIMD,
// so one wave's LDS and memory waits are covered by the other's MFMAs). Wave w
// owns weight rows [128 (w & 1), +128) and activation rows [64 (w >> 1), +64):
// 8 x 4 accumulators, 12 fragment reads per 32 MFMAs. Two LDS stages of
// [bf16 weight tile 32 KB | bf16 activation tile 32 KB]; activations are DMA'd
// one k tile ahead, weights loaded two ahead into two register sets.
// TNB: weight rows per tile, 256 or 192 (wave w then owns weight rows
// [TNB/2 (w & 1), +TNB/2): FI = TNB / 32 weight fragments; at 192 the 768
// weight slices of a k tile leave threads 256-511 one slice each, their second
// load re-reading a valid row that is never stored, so every wave issues the
// same loads and the wait counts stay exact).
template <int TNB>
__device__ __forceinline__ void gemm_tile_big(const GemmArgs &a) {
  constexpr int TMB = 256;
  constexpr int FI = TNB / 32;        // weight fragments per wave
  constexpr int SLICES = TNB * 4;     // 16-code weight slices per k tile
  constexpr int W_BYTES = TNB * BK * 2, X_BYTES = TMB * BK * 2, STAGE = W_BYTES + X_BYTES;
  constexpr int X_DMA = TMB * BK * 2 / 1024 / 8;  // 4 LDS-DMA instructions per wave per k tile
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1, wm = wave >> 1;

  const int tiles_m = (a.M + TMB - 1) / TMB, tiles_n = a.N / TNB;
  const int ntiles = tiles_m * tiles_n;
  const int S = a.ksplit > 1 ? a.ksplit : 1;  // split = the slowest index of the work
  const int per_xcd = (ntiles * S + 7) / 8;
  const int t_all = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (t_all >= ntiles * S) return;
  const int split = t_all / ntiles, t = t_all - split * ntiles;
  // n tiles per group: the 32 workgroups of an XCD cover ~4 n x 8 m tiles
  const int GN = a.group_n > 0 ? a.group_n : 4;
  const int group = t / (GN * tiles_m);
  const int first_n = group * GN;
  const int gw = min(GN, tiles_n - first_n);
  const int r = t - group * GN * tiles_m;
  const int n0 = (first_n + r % gw) * TNB, m0 = (r / gw) * TMB;
  // k tiles [kb, ke) of this split
  const int KTall = a.K / BK, groups = a.K / a.G;
  const int kb = split * KTall / S, ke = (split + 1) * KTall / S, last = ke - 1;

  __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];

  uint32_t xoff[X_DMA];
#pragma unroll
  for (int i = 0; i < X_DMA; ++i) {
    const int row = (wave * X_DMA + i) * 8 + (lane >> 3);
    const int m = min(m0 + row, a.M - 1);  // rows past M repeat the last row (not stored)
    xoff[i] = (uint32_t)m * (uint32_t)a.K * 2u + ((uint32_t)((lane & 7) ^ (row & 7)) << 4);
  }
  const char *xbase = (const char *)a.x;
  auto issue_x = [&](int kt, int stage) {
#pragma unroll
    for (int i = 0; i < X_DMA; ++i)
      dma16(xbase, xoff[i] + (uint32_t)(kt * (BK * 2)),
            lds_addr(smem + stage * STAGE + W_BYTES + (wave * X_DMA + i) * 1024));
  };

  // weights: SLICES slices of 16 codes per k tile, 2 per thread (row = id / 4, kq = id % 4)
  const int kstride = a.w_packed ? 1024 : BK;
  uint32_t woff[2], soff[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int id = SLICES == 1024 ? tid + 512 * p : min(tid + 512 * p, SLICES - 1);
    const int row = id >> 2, kq = id & 3;
    const int n = n0 + row;
    woff[p] = a.w_packed
                  ? ((uint32_t)(n >> 4) * (uint32_t)KTall * 1024u + (uint32_t)((row & 15) + 16 * kq) * 16u)
                  : (uint32_t)n * (uint32_t)a.K + (uint32_t)kq * 16u;
    soff[p] = (uint32_t)n * (uint32_t)groups;
  }
  struct WSet {
    u32x4 w[2];
    float s[2];
  };
  auto load_w = [&](int kt, WSet &ws) {
    const int gi = kt * BK / a.G;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      ws.w[p] = *(const u32x4 *)(a.w + woff[p] + (uint32_t)(kt * kstride));
      ws.s[p] = a.scale[soff[p] + gi];
    }
  };
  uint32_t hq[8];
  auto dequant_piece = [&](const WSet &ws, int piece, int stage) {
    const int p = piece >> 2, e = piece & 3;
    if (SLICES < 1024 && tid + 512 * p >= SLICES) return;  // a re-read slice (uniform per wave)
    const float sc = ws.s[p], o = -128.0f * sc;
    const uint32_t w4 = ws.w[p][e];
    const float f0 = __builtin_fmaf((float)(w4 & 0xffu), sc, o);
    const float f1 = __builtin_fmaf((float)((w4 >> 8) & 0xffu), sc, o);
    const float f2 = __builtin_fmaf((float)((w4 >> 16) & 0xffu), sc, o);
    const float f3 = __builtin_fmaf((float)(w4 >> 24), sc, o);
    hq[2 * e] = pack_bf16x2(f0, f1);
    hq[2 * e + 1] = pack_bf16x2(f2, f3);
    if (e == 3) {
      const int id = tid + 512 * p, row = id >> 2, kq = id & 3;
      char *dst = smem + stage * STAGE;
      *(u32x4 *)(dst + swz(row, 2 * kq)) = u32x4{hq[0], hq[1], hq[2], hq[3]};
      *(u32x4 *)(dst + swz(row, 2 * kq + 1)) = u32x4{hq[4], hq[5], hq[6], hq[7]};
    }
  };

  f32x4 acc[FI][4];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15, kg = lane >> 4;
  auto frag_a = [&](int stage, int i, int ks) {
    return as_bf16x8(*(const u32x4 *)(smem + stage * STAGE + swz(wn * (TNB / 2) + 16 * i + r16, ks * 4 + kg)));
  };
  auto frag_b = [&](int stage, int j, int ks) {
    return as_bf16x8(
        *(const u32x4 *)(smem + stage * STAGE + W_BYTES + swz(wm * 64 + 16 * j + r16, ks * 4 + kg)));
  };

  // Every k tile issues X_DMA activation DMAs, then 4 weight/scale loads per
  // lane (past the split's last tile they repeat it into slots nobody reads),
  // so the wait counts are exact. Plain s_barrier after explicit waits, as
  // __syncthreads()'s fence would wait for all loads in flight.
  WSet w0, w1;
  issue_x(kb, 0);
  load_w(kb, w0);
  load_w(min(kb + 1, last), w1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int piece = 0; piece < 8; ++piece) dequant_piece(w0, piece, 0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // 2 FI groups per k tile, g = FI ks + i: the 4 MFMAs of weight fragment
  // (ks, i); fragment reads run PREFETCH groups ahead (a ring of PREFETCH + 1
  // weight fragments), the activation fragments of ks = 1 two groups before
  // use; the 8 dequantisation pieces of the next tile spread over the ks = 1
  // groups (at FI = 6 the last two groups take two each, a slice's e = 3
  // piece, which stores it, last).
  constexpr int PREFETCH = RXW8_GEMM_PREFETCH;
  auto step = [&](int kt, auto xs, WSet &load_set, const WSet &deq_set) {
    constexpr int cur = decltype(xs)::value, nxt = cur ^ 1;
    issue_x(min(kt + 1, last), nxt);
    __builtin_amdgcn_sched_barrier(0);
    load_w(min(kt + 2, last), load_set);
    bf16x8 af[PREFETCH + 1], bf[4], bn[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = frag_b(cur, j, 0);
#pragma unroll
    for (int g = 0; g < PREFETCH; ++g) af[g] = frag_a(cur, g % FI, g / FI);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < 2 * FI; ++g) {
      const int i = g % FI, ks = g / FI;
      if (g + PREFETCH < 2 * FI)
        af[(g + PREFETCH) % (PREFETCH + 1)] = frag_a(cur, (g + PREFETCH) % FI, (g + PREFETCH) / FI);
      if (g == FI - 2)
#pragma unroll
        for (int j = 0; j < 4; ++j) bn[j] = frag_b(cur, j, 1);
      // weights of tile kt+1 were loaded last k tile: this tile's 8 loads are younger
      if (g == FI) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = mfma16x16x32(af[g % (PREFETCH + 1)], ks ? bn[j] : bf[j], acc[i][j]);
      if (ks) {
        dequant_piece(deq_set, i, nxt);
        if (FI == 6 && i >= 4) dequant_piece(deq_set, i + 2, nxt);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // activation tile kt+1 (this tile's DMAs) is older than this tile's 4 weight loads
    asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  int kt = kb;
  for (; kt + 2 <= ke; kt += 2) {
    step(kt, S0{}, w0, w1);
    step(kt + 1, S1{}, w1, w0);
  }
  if (kt < ke) step(kt, S0{}, w0, w1);

  if (S > 1) {  // raw f32 partials; rxw8_gemv_splitk_reduce sums them in split order
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = m0 + wm * 64 + 16 * j + r16;
        if (m < a.M)
          *(f32x4 *)(a.ws + ((int64_t)split * a.M + m) * a.N + n0 + wn * (TNB / 2) + 16 * i + 4 * kg) =
              acc[i][j];
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      gemm_store(a, m0 + wm * 64 + 16 * j + r16, n0 + wn * (TNB / 2) + 16 * i + 4 * kg, acc[i][j]);
}

// 256 x 256 tiles over weights already dequantised to bf16 (row-major
// [N, K], written by rxw8_gemm_dequant_w): both operands go global -> LDS by
// LDS DMA, so the k loop issues only DMAs, fragment reads and MFMAs. Same
// waves, fragments and tile order as gemm_tile_big; two stages, the DMAs of
// tile kt+1 in flight while tile kt is multiplied.
__device__ __forceinline__ void gemm_tile_bf16w(const GemmArgs &a) {
  constexpr int TNB = 256, TMB = 256;
  constexpr int W_BYTES = TNB * BK * 2, X_BYTES = TMB * BK * 2, STAGE = W_BYTES + X_BYTES;
  constexpr int DMA = TMB * BK * 2 / 1024 / 8;  // 4 LDS-DMA instructions per wave per operand
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1, wm = wave >> 1;

  const int tiles_m = (a.M + TMB - 1) / TMB, tiles_n = a.N / TNB;
  const int ntiles = tiles_m * tiles_n;
  const int per_xcd = (ntiles + 7) / 8;
  const int t = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (t >= ntiles) return;
  const int GN = a.group_n > 0 ? a.group_n : 4;
  const int group = t / (GN * tiles_m);
  const int first_n = group * GN;
  const int gw = min(GN, tiles_n - first_n);
  const int r = t - group * GN * tiles_m;
  const int n0 = (first_n + r % gw) * TNB, m0 = (r / gw) * TMB;
  const int KT = a.K / BK, last = KT - 1;

  __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];

  // DMA instruction i of this wave fills tile rows 8 (wave DMA + i) .. + 8;
  // lane -> row += lane / 8, physical chunk lane % 8 <- logical chunk (lane % 8) ^ (row & 7)
  uint32_t xoff[DMA], woff[DMA];
#pragma unroll
  for (int i = 0; i < DMA; ++i) {
    const int row = (wave * DMA + i) * 8 + (lane >> 3);
    const uint32_t chunk = (uint32_t)((lane & 7) ^ (row & 7)) << 4;
    const int m = min(m0 + row, a.M - 1);  // rows past M repeat the last row (not stored)
    xoff[i] = (uint32_t)m * (uint32_t)a.K * 2u + chunk;
    woff[i] = (uint32_t)(n0 + row) * (uint32_t)a.K * 2u + chunk;
  }
  const char *xbase = (const char *)a.x, *wbase = (const char *)a.w;
  auto issue = [&](int kt, int stage) {
#pragma unroll
    for (int i = 0; i < DMA; ++i)
      dma16(wbase, woff[i] + (uint32_t)(kt * (BK * 2)),
            lds_addr(smem + stage * STAGE + (wave * DMA + i) * 1024));
#pragma unroll
    for (int i = 0; i < DMA; ++i)
      dma16(xbase, xoff[i] + (uint32_t)(kt * (BK * 2)),
            lds_addr(smem + stage * STAGE + W_BYTES + (wave * DMA + i) * 1024));
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15, kg = lane >> 4;
  auto frag_a = [&](int stage, int i, int ks) {
    return as_bf16x8(*(const u32x4 *)(smem + stage * STAGE + swz(wn * (TNB / 2) + 16 * i + r16, ks * 4 + kg)));
  };
  auto frag_b = [&](int stage, int j, int ks) {
    return as_bf16x8(
        *(const u32x4 *)(smem + stage * STAGE + W_BYTES + swz(wm * 64 + 16 * j + r16, ks * 4 + kg)));
  };

  issue(0, 0);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  constexpr int PREFETCH = RXW8_GEMM_PREFETCH;
  auto step = [&](int kt, auto xs) {
    constexpr int cur = decltype(xs)::value, nxt = cur ^ 1;
    issue(min(kt + 1, last), nxt);
    bf16x8 af[PREFETCH + 1], bf[4], bn[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = frag_b(cur, j, 0);
#pragma unroll
    for (int g = 0; g < PREFETCH; ++g) af[g] = frag_a(cur, g & 7, g >> 3);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      const int i = g & 7, ks = g >> 3;
      if (g + PREFETCH < 16) af[(g + PREFETCH) % (PREFETCH + 1)] = frag_a(cur, (g + PREFETCH) & 7, (g + PREFETCH) >> 3);
      if (g == 6)
#pragma unroll
        for (int j = 0; j < 4; ++j) bn[j] = frag_b(cur, j, 1);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = mfma16x16x32(af[g % (PREFETCH + 1)], ks ? bn[j] : bf[j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // tile kt+1 is in LDS once this wave's DMAs land; the barrier covers every wave's
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  int kt = 0;
  for (; kt + 2 <= KT; kt += 2) {
    step(kt, S0{});
    step(kt + 1, S1{});
  }
  if (kt < KT) step(kt, S0{});

#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      gemm_store(a, m0 + wm * 64 + 16 * j + r16, n0 + wn * 128 + 16 * i + 4 * kg, acc[i][j]);
}

// ---- W8 linear with compute dtype F32 for long inputs (Qwen3.5 prefill,
// the tied LM head; layers.rs:277-298 with an f32 compute dtype):
//   y[m, n] = sum_g s[n, g] * sum_{k in g} (xh[m, k] + xl[m, k]) * (u8[n, k] - 128)
// with x = xh + xl + r split into bf16 parts (rxw8_gemm_split_x; |r| <= 2^-17
// |x|) and the codes u - 128 exact in bf16, so every MFMA product is exact and
// accumulates in f32; each scale group's f32 sum is then scaled into the
// total, the arithmetic of rxw8_linear_f32_mfma (a reassociation of the
// reference's x . (q s): both are f32 sums of the same terms).
//
// 256 (weight rows n) x 128 (activation rows m) output tiles, 8 waves of 64 x
// 64 (4 along n, 2 along m), k tiles of 64 in two LDS stages of [bf16 codes
// 256 x 64 | xh 128 x 64 | xl 128 x 64]. The codes go global -> VGPRs ->
// (u - 128 as bf16) -> LDS once per workgroup, loaded a tile ahead; xh / xl
// go global -> LDS by LDS DMA, a tile ahead. The tile's scales sit in LDS as
// [group][256 rows] (K / G <= 32). Per k tile a wave issues 64 MFMAs (hi and
// lo for each of its 4 x 4 fragment pairs and both k halves), so the weights
// are read once per 128 rows of x instead of once per 32.
//
// Split K (ksplit > 1, for shapes with too few tiles to fill the CUs): work
// item (split, tile) covers split's share of the scale groups (of the k tiles
// when there is one group), scales its group sums into an f32 partial tile
// written to ws[split], and rxw8_gemm_f32c_reduce adds the partials in split
// order into y.
struct LinearF32GemmArgs {
  const uint16_t *xh, *xl;  // [M, K] bf16 hi / lo parts of x
  const uint8_t *w;         // [N, K] u8 codes, or packed [N/16, K/64, 1024]
  const float *scale;       // [N, K / G]
  float *y;                 // [M, N]
  int M, N, K, G;
  int y_mode;               // 0: y = result; 1: y += result
  int w_packed;
  int ksplit;               // 1, or the number of K splits
  float *ws;                // [ksplit, M, N] f32 partials when ksplit > 1
};

__device__ __forceinline__ void linear_f32_gemm_tile(const LinearF32GemmArgs &a) {
  constexpr int TNB = 256, TMB = 128;
  constexpr int W_BYTES = TNB * BK * 2, X_BYTES = TMB * BK * 2;
  constexpr int STAGE = W_BYTES + 2 * X_BYTES;  // 64 KiB
  constexpr int XDMA = X_BYTES / 1024 / 8;       // 2 LDS-DMA instructions per wave per part
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 3, wm = wave >> 2;

  const int tiles_m = (a.M + TMB - 1) / TMB, tiles_n = (a.N + TNB - 1) / TNB;
  const int ntiles = tiles_m * tiles_n;
  const int S = a.ksplit > 1 ? a.ksplit : 1;  // split = the slowest index of the work
  const int per_xcd = (ntiles * S + 7) / 8;
  const int t_all = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (t_all >= ntiles * S) return;
  const int split = t_all / ntiles, t = t_all - split * ntiles;
  constexpr int GN = 4;  // n tiles per tile-order group
  const int group = t / (GN * tiles_m);
  const int first_n = group * GN;
  const int gw = min(GN, tiles_n - first_n);
  const int r = t - group * GN * tiles_m;
  const int n0 = (first_n + r % gw) * TNB, m0 = (r / gw) * TMB;
  const int KT = a.K / BK, ng = a.K / a.G, tpg = a.G / BK;  // k tiles per scale group
  // k tiles [kb, ke) of this split: whole scale groups, or k tiles of the one group
  const int units = ng > 1 ? ng : KT, upt = ng > 1 ? tpg : 1;
  const int kb = split * units / S * upt, ke = (split + 1) * units / S * upt;

  __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];
  __shared__ float sc[32 * TNB];  // [group][row]

  // activation DMA: instruction i of this wave fills rows 8 (2 wave + i) .. + 8
  uint32_t xoff[XDMA];
#pragma unroll
  for (int i = 0; i < XDMA; ++i) {
    const int row = (wave * XDMA + i) * 8 + (lane >> 3);
    const int m = min(m0 + row, a.M - 1);  // rows past M repeat the last row (not stored)
    xoff[i] = (uint32_t)m * (uint32_t)a.K * 2u + ((uint32_t)((lane & 7) ^ (row & 7)) << 4);
  }
  auto issue_x = [&](int kt, int stage) {
#pragma unroll
    for (int i = 0; i < XDMA; ++i) {
      const uint32_t l = lds_addr(smem + stage * STAGE + W_BYTES + (wave * XDMA + i) * 1024);
      dma16(a.xh, xoff[i] + (uint32_t)(kt * (BK * 2)), l);
      dma16(a.xl, xoff[i] + (uint32_t)(kt * (BK * 2)), l + X_BYTES);
    }
  };
  // codes: 1024 slices of 16 per k tile, 2 per thread (row = id / 4, kq = id % 4)
  const int kstride = a.w_packed ? 1024 : BK;
  uint32_t woff[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int id = tid + 512 * p, row = id >> 2, kq = id & 3;
    const int n = min(n0 + row, a.N - 1);
    woff[p] = a.w_packed ? ((uint32_t)(n >> 4) * (uint32_t)KT * 1024u + (uint32_t)((n & 15) + 16 * kq) * 16u)
                         : (uint32_t)n * (uint32_t)a.K + (uint32_t)kq * 16u;
  }
  u32x4 wr[2];
  auto load_w = [&](int kt) {
#pragma unroll
    for (int p = 0; p < 2; ++p) wr[p] = *(const u32x4 *)(a.w + woff[p] + (uint32_t)(kt * kstride));
  };
  auto store_w = [&](int stage) {  // u - 128, exact in bf16
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int id = tid + 512 * p, row = id >> 2, kq = id & 3;
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t q = wr[p][e];
        h[2 * e] = pack_bf16x2((float)(q & 0xffu) - 128.f, (float)((q >> 8) & 0xffu) - 128.f);
        h[2 * e + 1] = pack_bf16x2((float)((q >> 16) & 0xffu) - 128.f, (float)(q >> 24) - 128.f);
      }
      char *dst = smem + stage * STAGE;
      *(u32x4 *)(dst + swz(row, 2 * kq)) = u32x4{h[0], h[1], h[2], h[3]};
      *(u32x4 *)(dst + swz(row, 2 * kq + 1)) = u32x4{h[4], h[5], h[6], h[7]};
    }
  };

  f32x4 acc[4][4], tot[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      tot[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  const int r16 = lane & 15, kg = lane >> 4;

  load_w(kb);
  issue_x(kb, 0);
  // this split's scale groups only (sc keeps the absolute group index), their
  // loads behind the first tile's: rows past N (the last n tile of N % 256 ==
  // 128) repeat row N - 1 and are not stored
  {
    const int g_lo = kb / tpg, g_hi = (ke - 1) / tpg + 1;
    for (int e = g_lo * TNB + tid; e < g_hi * TNB; e += 512) {
      const int g = e / TNB, row = e - g * TNB;
      sc[e] = a.scale[(int64_t)min(n0 + row, a.N - 1) * ng + g];
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  store_w(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  for (int kt = kb; kt < ke; ++kt) {
    const int cur = (kt - kb) & 1, nxt = cur ^ 1;
    const bool more = kt + 1 < ke;  // uniform
    if (more) {
      load_w(kt + 1);     // 2 loads, then 4 DMAs: vmcnt(4) waits for the loads alone
      issue_x(kt + 1, nxt);
    }
    const char *st = smem + cur * STAGE;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 fa[4], fh[4], fl[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        fa[i] = as_bf16x8(*(const u32x4 *)(st + swz(wn * 64 + 16 * i + r16, ks * 4 + kg)));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        fh[j] = as_bf16x8(*(const u32x4 *)(st + W_BYTES + swz(wm * 64 + 16 * j + r16, ks * 4 + kg)));
        fl[j] = as_bf16x8(*(const u32x4 *)(st + W_BYTES + X_BYTES + swz(wm * 64 + 16 * j + r16, ks * 4 + kg)));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[i][j] = mfma16x16x32(fa[i], fh[j], acc[i][j]);
          acc[i][j] = mfma16x16x32(fa[i], fl[j], acc[i][j]);
        }
    }
    if ((kt + 1) % tpg == 0 || kt + 1 == ke) {  // a scale group's end (or the split's): tot += s[n, g] * acc
      const int g = kt / tpg;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 sv = *(const f32x4 *)(sc + g * TNB + wn * 64 + 16 * i + 4 * kg);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          tot[i][j] += sv * acc[i][j];
          acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
    if (more) {
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
      store_w(nxt);  // stage nxt was last read in step kt - 1, before the barrier
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }

  // lane holds D[n = 16 i + 4 kg + e][m = 16 j + r16]
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + wm * 64 + 16 * j + r16;
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = n0 + wn * 64 + 16 * i + 4 * kg;
      if (n >= a.N) continue;  // (N % 16 == 0: a lane's 4 channels are all in or all out)
      if (S > 1) {
        *(f32x4 *)(a.ws + ((int64_t)split * a.M + m) * a.N + n) = tot[i][j];
      } else {
        f32x4 *yp = (f32x4 *)(a.y + (int64_t)m * a.N + n);
        *yp = a.y_mode == 1 ? *yp + tot[i][j] : tot[i][j];
      }
    }
  }
}

}  // namespace

// Exact dequantisation into a bf16 [N, K] row-major workspace, the input of
// rxw8_w8a16_gemm_bf16w_t256: w = bf16(fma(f32(u), s, -128 s)), the same
// arithmetic as the in-loop dequantisation (layers.rs:277-294). One thread per
// 16 codes (G % 16 == 0, so one scale); row-major or packed source.
struct DequantWArgs {
  const uint8_t *w;
  const float *scale;
  uint16_t *out;
  int N, K, G, packed;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_gemm_dequant_w(DequantWArgs a) {
  const int64_t slices = (int64_t)a.N * (a.K / 16);
  const int64_t sl = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (sl >= slices) return;
  int row, k0;
  if (a.packed) {  // [N/16][K/64][64 lanes][16 B]: lane l holds row 16 t + l % 16, k 64 c + 16 (l / 16)
    const int l = (int)(sl & 63);
    const int64_t tc = sl >> 6;
    const int kc = a.K / 64;
    const int tt = (int)(tc / kc), c = (int)(tc - (int64_t)tt * kc);
    row = 16 * tt + (l & 15);
    k0 = 64 * c + 16 * (l >> 4);
  } else {
    const int per_row = a.K / 16;
    row = (int)(sl / per_row);
    k0 = (int)(sl - (int64_t)row * per_row) * 16;
  }
  const u32x4 w = __builtin_nontemporal_load((const u32x4 *)(a.w + sl * 16));
  const float sc = a.scale[(int64_t)row * (a.K / a.G) + k0 / a.G], o = -128.0f * sc;
  uint32_t h[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t w4 = w[e];
    h[2 * e] = pack_bf16x2(__builtin_fmaf((float)(w4 & 0xffu), sc, o),
                           __builtin_fmaf((float)((w4 >> 8) & 0xffu), sc, o));
    h[2 * e + 1] = pack_bf16x2(__builtin_fmaf((float)((w4 >> 16) & 0xffu), sc, o),
                               __builtin_fmaf((float)(w4 >> 24), sc, o));
  }
  u32x4 *dst = (u32x4 *)(a.out + (int64_t)row * a.K + k0);
  dst[0] = u32x4{h[0], h[1], h[2], h[3]};
  dst[1] = u32x4{h[4], h[5], h[6], h[7]};
}

extern "C" __global__ void __launch_bounds__(512) rxw8_w8a16_gemm_bf16w_t256(GemmArgs a) {
  gemm_tile_bf16w(a);
}

// Launch contract (checked by the host): N % 128 == 0, K % 64 == 0,
// G % 64 == 0 and K % G == 0, M >= 1, M * K * 2 < 2^31 and the weight bytes
// < 2^32; grid = 8 * ceil(tiles / 8) workgroups.
extern "C" __global__ void __launch_bounds__(512) rxw8_w8a16_gemm_t256(GemmArgs a) {
  gemm_tile_big<256>(a);
}
extern "C" __global__ void __launch_bounds__(512) rxw8_w8a16_gemm_t192(GemmArgs a) {
  gemm_tile_big<192>(a);
}

extern "C" __global__ void __launch_bounds__(256) rxw8_w8a16_gemm_m256(GemmArgs a) {
  gemm_tile<256>(a);
}

extern "C" __global__ void __launch_bounds__(256) rxw8_w8a16_gemm_m128(GemmArgs a) {
  gemm_tile<128>(a);
}

// f32 activations -> bf16 (RNE), the x.cast(BF16) ahead of the GEMM.
extern "C" __global__ void __launch_bounds__(256) rxw8_gemm_cast_x(CastArgs a) {
  const int64_t n4 = a.n / 4;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float4 v = ((const float4 *)a.x)[i];
    ((uint2 *)a.y)[i] = uint2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
  }
  const int64_t tail = a.n - 4 * n4;
  if (blockIdx.x == 0 && (int64_t)threadIdx.x < tail)
    a.y[4 * n4 + threadIdx.x] = f32_to_bf16_bits(a.x[4 * n4 + threadIdx.x]);
}

// Launch contract (checked by the host): N % 16 == 0, K % 64 == 0, G % 64
// == 0, K % G == 0, K / G <= 32, M >= 1, M * K * 2 < 2^31, N * K < 2^32,
// ksplit <= the split units; grid = 8 * ceil(tiles * ksplit / 8) workgroups
// of 512 threads.
extern "C" __global__ void __launch_bounds__(512) rxw8_gemm_f32c(LinearF32GemmArgs a) {
  linear_f32_gemm_tile(a);
}

// y = (or +=) the sum of the split partials of rxw8_gemm_f32c in split order.
struct F32ReduceArgs {
  const float *ws;  // [ksplit, M * N]
  float *y;         // [M * N]
  int64_t mn;       // M * N (a multiple of 4)
  int ksplit, y_mode;
};
extern "C" __global__ void __launch_bounds__(256) rxw8_gemm_f32c_reduce(F32ReduceArgs a) {
  const int64_t q4 = a.mn / 4;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < q4;
       i += (int64_t)gridDim.x * blockDim.x) {
    const f32x4 h = a.y_mode == 1 ? ((const f32x4 *)a.y)[i] : f32x4{0.f, 0.f, 0.f, 0.f};
    // partials in batches of 8 loaded before they are added (a loop adding
    // each as it arrives waited one memory round trip per split); the sum
    // stays in split order (indices past the last split re-read it, unused)
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < a.ksplit; s0 += 8) {
      f32x4 p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        p[j] = ((const f32x4 *)(a.ws + (int64_t)min(s0 + j, a.ksplit - 1) * a.mn))[i];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < a.ksplit) sum = s0 + j == 0 ? p[j] : sum + p[j];
    }
    ((f32x4 *)a.y)[i] = a.y_mode == 1 ? h + sum : sum;
  }
}

// f32 rows -> their bf16 parts hi = bf16(x), lo = bf16(x - hi) (RNE both), the
// operand split of rxw8_gemm_f32c.
struct SplitXArgs {
  const float *x;
  uint16_t *hi, *lo;
  int64_t n;
};
// Four values per thread (a 16-byte load, two 8-byte stores) when x is
// 16-byte aligned (n is a multiple of 64: K % 64 == 0), else one.
extern "C" __global__ void __launch_bounds__(256) rxw8_gemm_split_x(SplitXArgs a) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if (((uintptr_t)a.x & 15) == 0) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n / 4; i += stride) {
      const float4 v = ((const float4 *)a.x)[i];
      const uint32_t h01 = pack_bf16x2(v.x, v.y), h23 = pack_bf16x2(v.z, v.w);
      ((uint2 *)a.hi)[i] = uint2{h01, h23};
      ((uint2 *)a.lo)[i] = uint2{pack_bf16x2(v.x - bf16_bits_to_f32((uint16_t)h01),
                                             v.y - bf16_bits_to_f32((uint16_t)(h01 >> 16))),
                                 pack_bf16x2(v.z - bf16_bits_to_f32((uint16_t)h23),
                                             v.w - bf16_bits_to_f32((uint16_t)(h23 >> 16)))};
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) {
    const float v = a.x[i];
    const uint16_t h = f32_to_bf16_bits(v);
    a.hi[i] = h;
    a.lo[i] = f32_to_bf16_bits(v - bf16_bits_to_f32(h));
  }
}
