// K1: W8A16 decode GEMV / skinny GEMM on gfx950 MFMA.
//
// The default (gemv_rc, RC) form is the reference's product
// (crates/rxla-nn/src/layers.rs:277-296):
//   y[m, n] = bf16( sum_k bf16(x[m, k]) * bf16((u8[n, k] - 128) * s[n, k / G]) )
// The exact-code form (gemv, RXW8_GEMV_REF_CAST=0) moves the scale after the sum:
//   y[m, n] = bf16( sum_g s[n, g] * sum_{k in g} bf16(x[m, k]) * (u8[n, k] - 128) )
//
// Layout: u8 weights [N, K] row-major (RXLA's U8 = int8 + 128 storage,
// crates/rxla-nn/src/layers.rs:277-287), f32 scales [N, K/G], activations
// [M, K] bf16 (or f32, rounded to bf16 when staged), output [M, N] bf16 or f32.
//
// Mapping: a 256-thread workgroup (4 waves) owns 16*RW output channels and
// one K-split [k0, k0 + Kc) (Kc = K / ksplit). Its waves form RW row groups
// of 16 channels x KW = 4 / RW slices of Kc; the KW slices of a row group are
// reduced through LDS in slice order at the end. The workgroup first stages
// its activation slice x[0:M, k0:k0+Kc] in LDS as bf16 (padded rows) and, for
// grouped scales, its scale tile, so the streaming loop issues nothing but
// weight loads to global memory. Every lane streams 16-byte slices of one
// weight row (lane = row + 16 * slice): a wave load covers 16 rows x 64
// contiguous bytes. Loads are double-buffered in two register sets of U slices
// (issue B, consume A, issue A', consume B): U to 2U loads per lane stay in
// flight, and the straight-line buffers keep the compiler's vmcnt waits exact.
// The 16 codes of a slice become two bf16x8 A-fragments of
// v_mfma_f32_16x16x32_bf16 (u8 -> f32 -> bf16 is exact for 0..255); the
// activations from LDS are the B operand (batch rows as columns; columns >= M
// read a valid row and are never stored). The -128 offset is folded exactly by
// a second MFMA with an all-ones A operand, which yields sum_k x[m, k] per
// column: acc - 128 * ones. Scales are applied per group (G a multiple of 64)
// or once per channel (G == K).
//
// With ksplit > 1 each workgroup writes its unscaled (per-channel) or scaled
// (grouped) f32 partial tile with plain stores and rxw8_gemv_splitk_reduce sums
// the partials in split order in a second launch: deterministic, and the
// kernel boundary makes the partials visible without device-scope fences.
#include <type_traits>

#include "common.h"

struct GemvArgs {
  const void *x;      // activations, see x_mode
  const void *w;      // [N, K] u8 (or bf16 for the dense variant)
  const float *scale; // [N, K / G] (unused for the dense variant)
  void *y;            // [M, N] bf16 or f32
  float *ws;          // [ksplit, M, N] split-K partials
  int M, N, K, G;     // G == K for per-channel scales
  int ksplit;
  int x_f32, y_f32;
  // 0: store y; 1: y is an f32 residual, y += bf16(result);
  // 2: SwiGLU pairs (ksplit 1): in every 16-row weight tile t, rows 0-7 are
  //    gate channels 8t..8t+7 and rows 8-15 the matching up channels; y is
  //    bf16 [M, N/2] and receives bf16(silu(bf16(gate)) * bf16(up))
  int y_mode;
  // with y_mode 1 and ksplit 1 (optional): per 16-channel group g, the
  // partial sum of squares of the updated residual row b, ss_out[g * M + b]
  float *ss_out;
  // Activation prologue, applied while x is staged:
  //   0: x row m at x + m * x_stride + x_off (bf16, or f32 when x_f32)
  //   1: RMSNorm of f32 rows: x = bf16((h * 1/sqrt(mean(h^2) + eps)) * norm_w)
  //      with h the full K-row at x + m * x_stride + x_off (x_f32 must be 1)
  //   2: SwiGLU: x = bf16(silu(g) * u) with g = row[k], u = row[K + k] of the
  //      bf16 gate|up rows at x + m * x_stride (x_stride = 2K)
  //   3: RMSNorm as mode 1 with the row's sum of squares taken from
  //      ss_in[p * M + b] summed over p < ss_parts (partials of the producer)
  int x_mode;
  int64_t x_stride, x_off;  // elements
  const float *norm_w;      // [K] (modes 1, 3)
  float eps;
  const float *ss_in;       // mode 3
  int ss_parts;
  // plain rows (x_mode 0) with per-channel scales: every wave stages only its
  // own K slice of the rows in an LDS region of its own and starts without a
  // workgroup barrier (host-chosen; the LDS holds NW regions of M rows)
  int wave_stage;
  // bf16 rows (x_mode 0, Kc % 512 == 0, 16-byte aligned; host-checked) are
  // staged by LDS DMA: global_load_lds_dwordx4 copies 16 bytes per lane
  // straight into LDS -- no registers, every copy of the workgroup in flight
  // at once
  int lds_dma;
  // RMSNorm applied after the product (x_mode 0, ksplit 1, ss_parts <= 256;
  // host-checked): the rows of x hold
  // bf16(h * norm_w) and row b's result is multiplied by
  // 1/sqrt(sum_p ss_in[p * M + b] / K + eps) before the scale and epilogue.
  // The factors live in LDS at byte offset rs_off.
  int row_norm;
  int rs_off;
  // y_mode 1 with ss_out (optional): also write xw_out[b * N + n] =
  // bf16(h_new * xw_norm[n]), the next RMSNorm's weighted rows
  const float *xw_norm;
  uint16_t *xw_out;
  // row stride of the sum-of-squares partials (ss_in[p * ss_ld + b],
  // ss_out[g * ss_ld + b]): the rows of the whole product when the host runs
  // it in chunks of rows (the pointers then start at the chunk)
  int ss_ld;
  // F32-compute kernels: grid row blockIdx.y takes rows [blockIdx.y *
  // chunk_rows, min(M, (blockIdx.y + 1) * chunk_rows)) (x, y and the
  // sum-of-squares pointers start at row 0 of the whole product)
  int chunk_rows;
  int fc_kmajor;  // F32 staging: column-major piece order where it fits (host switch)
};

// Grouped launch: several independent products, each with its own operands
// and shape, in one grid; problem p owns workgroups [tile_begin, next
// problem's tile_begin). Every problem runs the same tiling (the kernel's
// template) with its own staging flags.
struct GemvProblem {
  const void *x;
  const void *w;
  const float *scale;
  void *y;
  int M, N, K, G;
  int tile_begin;
  int x_f32, y_f32, lds_dma, wave_stage;
};
constexpr int kGemvGroupMax = 16;
struct GemvGroupArgs {
  GemvArgs base;  // settings shared by every problem (plain rows, plain stores, no split)
  int count;
  GemvProblem p[kGemvGroupMax];
};

struct SplitkReduceArgs {
  const float *ws;    // [ksplit, M, N]
  const float *scale; // [N] per-channel scale or null
  void *y;            // [M, N]
  int M, N, ksplit;
  int y_f32;
  int y_mode;
};

namespace {

constexpr int kXPad = 8;  // bf16 elements of padding per staged activation row

// Returns the squared norm of the updated residual values (y_mode 1, with h0
// the residual values loaded earlier), else 0. With xw_out (y_mode 1), also
// writes the updated values times the next RMSNorm's weights as bf16.
// (The caller loads h0 and w together: a load placed after the store of h
// could alias it and would wait for that store.)
__device__ __forceinline__ float store_out(void *y, int y_f32, int y_mode, int64_t N, int b, int n,
                                           f32x4 v, float4 h0, uint16_t *xw_out = nullptr,
                                           float4 w = float4{0.f, 0.f, 0.f, 0.f}) {
  if (y_mode == 1) {  // residual: h += f32(bf16(result)) (layers.rs:295-296 + add)
    float4 *h = (float4 *)((float *)y + (int64_t)b * N + n);
    float4 o = h0;
    o.x += round_bf16(v[0]);
    o.y += round_bf16(v[1]);
    o.z += round_bf16(v[2]);
    o.w += round_bf16(v[3]);
    *h = o;
    if (xw_out)
      *(uint2 *)(xw_out + (int64_t)b * N + n) =
          uint2{pack_bf16x2(o.x * w.x, o.y * w.y), pack_bf16x2(o.z * w.z, o.w * w.w)};
    return ((o.x * o.x + o.y * o.y) + o.z * o.z) + o.w * o.w;
  } else if (y_f32) {
    float4 o = {round_bf16(v[0]), round_bf16(v[1]), round_bf16(v[2]), round_bf16(v[3])};
    *(float4 *)((float *)y + (int64_t)b * N + n) = o;
  } else {
    uint2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    *(uint2 *)((uint16_t *)y + (int64_t)b * N + n) = o;
  }
  return 0.f;
}

// 16-byte bf16 pieces per thread whose global loads the staging loops issue
// before storing any of them: one round trip per batch (a load-then-store loop
// waits for every load in turn). Sized so staging needs no more registers than
// the streaming loop (every path's peak sets the kernel's occupancy).
constexpr int kStageBatch = 4;

// Copy rows [0, M) x pieces [0, per_row) of 8 activations (row m at x + m *
// stride + off; bf16, or f32 rounded to bf16) into LDS rows of stride ld.
// The caller's thread t0 of nt takes pieces t0, t0 + nt, ..., loading
// kStageBatch (f32: half as many) of them before storing any.
__device__ __forceinline__ void stage_rows(const void *x, bool x_f32, int64_t stride, int64_t off,
                                           int M, int per_row, uint16_t *dst, int ld, int t0, int nt) {
  const int total = M * per_row;
  if (x_f32) {
    constexpr int SB = kStageBatch / 2;
    for (int i0 = t0; i0 < total; i0 += SB * nt) {
      float4 v[SB][2];
#pragma unroll
      for (int s = 0; s < SB; ++s) {
        const int i = i0 + s * nt;
        if (i < total) {
          const int b = i / per_row, kk = (i - b * per_row) * 8;
          const float4 *p = (const float4 *)((const float *)x + b * stride + off + kk);
          v[s][0] = p[0];
          v[s][1] = p[1];
        }
      }
#pragma unroll
      for (int s = 0; s < SB; ++s) {
        const int i = i0 + s * nt;
        if (i < total) {
          const int b = i / per_row, kk = (i - b * per_row) * 8;
          u32x4 r;
          r[0] = pack_bf16x2(v[s][0].x, v[s][0].y);
          r[1] = pack_bf16x2(v[s][0].z, v[s][0].w);
          r[2] = pack_bf16x2(v[s][1].x, v[s][1].y);
          r[3] = pack_bf16x2(v[s][1].z, v[s][1].w);
          *(u32x4 *)(dst + b * ld + kk) = r;
        }
      }
    }
    return;
  }
  constexpr int SB = kStageBatch;
  for (int i0 = t0; i0 < total; i0 += SB * nt) {
    u32x4 v[SB];
#pragma unroll
    for (int s = 0; s < SB; ++s) {
      const int i = i0 + s * nt;
      if (i < total) {
        const int b = i / per_row, kk = (i - b * per_row) * 8;
        v[s] = *(const u32x4 *)((const uint16_t *)x + b * stride + off + kk);
      }
    }
#pragma unroll
    for (int s = 0; s < SB; ++s) {
      const int i = i0 + s * nt;
      if (i < total) {
        const int b = i / per_row, kk = (i - b * per_row) * 8;
        *(u32x4 *)(dst + b * ld + kk) = v[s];
      }
    }
  }
}

typedef __attribute__((address_space(3))) void lds_void;

// One LDS DMA instruction of the wave: lane l copies 16 bytes from g (its own
// address) to LDS at l_base + 16 l (l_base wave-uniform). Completion is
// counted by vmcnt.
__device__ __forceinline__ void lds_dma16(const void *g, void *l_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_void *)l_base, 16, 0, 0);
}

// FC (compute dtype F32): stage f32 rows x[0:M, k0:k0+Kc] as their bf16
// parts, hi = bf16(v) in LDS row b and lo = bf16(v - hi) in row LO + b
// (|v - hi - lo| <= 2^-17 |v|), with v the row value (x_mode 0) or its
// RMSNorm (h * factor) * w (modes 1, 3, the f32 value the reference's norm
// produces), and the workgroup's nsc grouped scales (ss[row_in_block * gps +
// g_local], see gemv_w8). Pieces of 8 values, SB per thread per round.
//
// stage_x_fc_impl (short inputs): the scales, the norm's sum-of-squares
// partials (mode 3) and the first round of pieces are requested before any
// of them is used, so they share one memory round trip with the first weight
// group. They are raw buffer loads: a lane past the end reads an offset
// beyond its buffer's size and gets zeros without touching memory, so no
// lane branches around them (a load under a branch made the compiler wait
// for it at once, to copy its register at the join). The mode is
// compile-time, so the idle lanes issue no loads their mode does not use
// (zero-filled returns still take the return path's cycles: with them,
// one-row launches ran 0.3-0.7 us slower).
__device__ __forceinline__ void norm_row_scales(const GemvArgs &a, float *row_scale, float *red);
template <int NT, int MODE, int SB>
__device__ __forceinline__ void stage_x_fc_impl(const GemvArgs &a, uint16_t *xs, float *ss, int k0,
                                                int Kc, int LO, int nsc, int rows0, int gps) {
  const int ldx = Kc + kXPad;
  const int per_row = Kc / 8;
  const int total = a.M * per_row;
  constexpr bool norm = MODE != 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int NWV = NT / 64;
  __shared__ float red[4];
  __shared__ float row_scale[16];
  constexpr uint32_t kOob = 0x80000000u;
  const int groups = a.K / a.G, g0 = k0 / a.G;
  const int gpsd = gps > 0 ? gps : 1;
  auto scale_off = [&](int i) {  // byte offset of staged scale i (kOob past nsc)
    const int rr = i / gpsd, gl = i - rr * gpsd;
    return i < nsc ? (uint32_t)(min(rows0 + rr, a.N - 1) * groups + g0 + gl) * 4u : kOob;
  };
  const auto srsrc = buf_rsrc(a.scale, (uint32_t)(a.N * groups) * 4u);
  float sv[SB];
#pragma unroll
  for (int q = 0; q < SB; ++q)
    sv[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srsrc, scale_off(threadIdx.x + q * NT), 0, 0));
  // mode 3: the first 4 partials (p = lane + 64 s) of this wave's first SB
  // rows (b = wave + r NWV)
  float t0[SB][4];
  if constexpr (MODE == 3) {
    const auto trsrc =
        buf_rsrc(a.ss_in, a.ss_parts > 0 ? (uint32_t)((a.ss_parts - 1) * a.ss_ld + a.M) * 4u : 0u);
#pragma unroll
    for (int r = 0; r < SB; ++r) {
      const int b = wave + r * NWV;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int pp = lane + 64 * q;
        const uint32_t off = b < a.M && pp < a.ss_parts ? (uint32_t)(pp * a.ss_ld + b) * 4u : kOob;
        t0[r][q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(trsrc, off, 0, 0));
      }
    }
  }
  u32x4 hv[SB][2], wv[SB][2];
  const auto xrsrc = buf_rsrc((const float *)a.x + a.x_off + k0, (uint32_t)((a.M - 1) * a.x_stride + Kc) * 4u);
  const auto wrsrc = buf_rsrc(norm ? a.norm_w + k0 : (const float *)a.x, norm ? (uint32_t)Kc * 4u : 0u);
  auto load_pieces = [&](int i0) {
#pragma unroll
    for (int q = 0; q < SB; ++q) {
      const int i = i0 + q * NT;
      const int b = i / per_row, kk = (i - b * per_row) * 8;
      const uint32_t xo = i < total ? (uint32_t)(b * a.x_stride + kk) * 4u : kOob;
      hv[q][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, xo, 0, 0));
      hv[q][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, xo + 16u, 0, 0));
      if constexpr (norm) {
        const uint32_t wo = i < total ? (uint32_t)kk * 4u : kOob;
        wv[q][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, wo, 0, 0));
        wv[q][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, wo + 16u, 0, 0));
      }
    }
  };
  auto store_pieces = [&](int i0) {
#pragma unroll
    for (int q = 0; q < SB; ++q) {
      const int i = i0 + q * NT;
      if (i < total) {
        const int b = i / per_row, kk = (i - b * per_row) * 8;
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = __uint_as_float(hv[q][0][e]);
          v[4 + e] = __uint_as_float(hv[q][1][e]);
        }
        if constexpr (norm) {
          const float sc = row_scale[b];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = (v[e] * sc) * __uint_as_float(wv[q][0][e]);
            v[4 + e] = (v[4 + e] * sc) * __uint_as_float(wv[q][1][e]);
          }
        }
        u32x4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float h0 = round_bf16(v[2 * e]), h1 = round_bf16(v[2 * e + 1]);
          hi[e] = pack_bf16x2(h0, h1);
          lo[e] = pack_bf16x2(v[2 * e] - h0, v[2 * e + 1] - h1);
        }
        *(u32x4 *)(xs + b * ldx + kk) = hi;
        *(u32x4 *)(xs + (LO + b) * ldx + kk) = lo;
      }
    }
  };
  load_pieces(threadIdx.x);
  // scales to LDS (rows past N weigh 0; any beyond SB per thread in a loop)
#pragma unroll
  for (int q = 0; q < SB; ++q) {
    const int i = threadIdx.x + q * NT;
    if (i < nsc) ss[i] = rows0 + i / gpsd < a.N ? sv[q] : 0.f;
  }
  for (int i = threadIdx.x + SB * NT; i < nsc; i += NT)
    ss[i] = rows0 + i / gpsd < a.N ? a.scale[scale_off(i) / 4u] : 0.f;
  if constexpr (MODE == 3) {
    // one wave per row, lane l adding partials l, l + 64, ... in that order,
    // then a fixed butterfly (deterministic)
    auto row_sum = [&](int b, const float(&tf)[4], bool pre) {
      float sum = 0.f;
      for (int p0 = lane; p0 < a.ss_parts; p0 += 256) {
        float t[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          t[q] = pre && p0 == lane ? tf[q] : a.ss_in[(int64_t)min(p0 + 64 * q, a.ss_parts - 1) * a.ss_ld + b];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (p0 + 64 * q < a.ss_parts) sum += t[q];
      }
      sum = wave_sum64(sum);
      if (lane == 0) row_scale[b] = 1.0f / sqrtf(sum / (float)a.K + a.eps);
    };
#pragma unroll
    for (int r = 0; r < SB; ++r)
      if (wave + r * NWV < a.M) row_sum(wave + r * NWV, t0[r], true);
    for (int b = wave + SB * NWV; b < a.M; b += NWV) row_sum(b, t0[0], false);
  } else if constexpr (MODE == 1) {
    norm_row_scales(a, row_scale, red);
  }
  if constexpr (norm) __syncthreads();
  store_pieces(threadIdx.x);
  for (int i0 = threadIdx.x + SB * NT; i0 < total; i0 += SB * NT) {
    load_pieces(i0);
    store_pieces(i0);
  }
}
// stage_x_fc_rounds (longer inputs): the scales, then the norm factors, then
// rounds of SB = 2 pieces per thread, each a memory round trip after the one
// before (measured faster there than two batches requested up front: the
// Qwen3.5-0.8B forward at 16 rows, 1.39 against 1.42 ms).
template <int NT>
__device__ __forceinline__ void stage_x_fc_rounds(const GemvArgs &a, uint16_t *xs, float *ss, int k0, int Kc,
                                                  int LO, int nsc, int rows0, int gps) {
  if (nsc > 0) {
    const int groups = a.K / a.G, g0 = k0 / a.G;
    for (int i = threadIdx.x; i < nsc; i += NT) {
      const int rr = i / gps, gl = i - rr * gps;
      const int n = rows0 + rr;
      ss[i] = n < a.N ? a.scale[(int64_t)n * groups + g0 + gl] : 0.f;
    }
  }
  const int ldx = Kc + kXPad;
  const int per_row = Kc / 8;
  const int total = a.M * per_row;
  const int nt = NT;
  const bool norm = a.x_mode == 1 || a.x_mode == 3;
  __shared__ float red[4];
  __shared__ float row_scale[16];
  if (norm) {
    norm_row_scales(a, row_scale, red);
    __syncthreads();
  }
  constexpr int SB = 2;
  for (int i0 = threadIdx.x; i0 < total; i0 += SB * nt) {
    float4 hv[SB][2], wv[SB][2];
#pragma unroll
    for (int s = 0; s < SB; ++s) {
      const int i = i0 + s * nt;
      if (i < total) {
        const int b = i / per_row, kk = (i - b * per_row) * 8;
        const float *h = (const float *)a.x + b * a.x_stride + a.x_off + k0 + kk;
        hv[s][0] = *(const float4 *)h;
        hv[s][1] = *(const float4 *)(h + 4);
        if (norm) {
          wv[s][0] = *(const float4 *)(a.norm_w + k0 + kk);
          wv[s][1] = *(const float4 *)(a.norm_w + k0 + kk + 4);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < SB; ++s) {
      const int i = i0 + s * nt;
      if (i < total) {
        const int b = i / per_row, kk = (i - b * per_row) * 8;
        float v[8] = {hv[s][0].x, hv[s][0].y, hv[s][0].z, hv[s][0].w,
                      hv[s][1].x, hv[s][1].y, hv[s][1].z, hv[s][1].w};
        if (norm) {
          const float sc = row_scale[b];
          const float w[8] = {wv[s][0].x, wv[s][0].y, wv[s][0].z, wv[s][0].w,
                              wv[s][1].x, wv[s][1].y, wv[s][1].z, wv[s][1].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = (v[e] * sc) * w[e];
        }
        u32x4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float h0 = round_bf16(v[2 * e]), h1 = round_bf16(v[2 * e + 1]);
          hi[e] = pack_bf16x2(h0, h1);
          lo[e] = pack_bf16x2(v[2 * e] - h0, v[2 * e + 1] - h1);
        }
        *(u32x4 *)(xs + b * ldx + kk) = hi;
        *(u32x4 *)(xs + (LO + b) * ldx + kk) = lo;
      }
    }
  }
}

// stage_x_fc_kmajor (up to 4 rows per thread): thread t takes the piece at
// k = 8 (t % (Kc / 8)) of rows t / (Kc / 8) + j NT / (Kc / 8), j < 4, so its
// norm weights load once for all of its rows, and every row piece, the
// scales and the norm partials are requested before any is used (one memory
// round trip instead of the rounds' three or four).
template <int NT>
__device__ __forceinline__ void stage_x_fc_kmajor(const GemvArgs &a, uint16_t *xs, float *ss, int k0, int Kc,
                                                  int LO, int nsc, int rows0, int gps) {
  const int ldx = Kc + kXPad;
  const int per_row = Kc / 8, rpb = NT / per_row;  // pieces per row, rows per batch
  const bool norm = a.x_mode == 3;
  const int kk = ((int)threadIdx.x % per_row) * 8, b0 = (int)threadIdx.x / per_row;
  __shared__ float red[4];
  __shared__ float row_scale[16];
  float4 xv[4][2], wv[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = b0 + j * rpb;
    if (b < a.M) {
      const float *h = (const float *)a.x + b * a.x_stride + a.x_off + k0 + kk;
      xv[j][0] = *(const float4 *)h;
      xv[j][1] = *(const float4 *)(h + 4);
    }
  }
  if (norm) {
    wv[0] = *(const float4 *)(a.norm_w + k0 + kk);
    wv[1] = *(const float4 *)(a.norm_w + k0 + kk + 4);
  }
  if (nsc > 0) {
    const int groups = a.K / a.G, g0 = k0 / a.G;
    for (int i = threadIdx.x; i < nsc; i += NT) {
      const int rr = i / gps, gl = i - rr * gps;
      const int n = rows0 + rr;
      ss[i] = n < a.N ? a.scale[(int64_t)n * groups + g0 + gl] : 0.f;
    }
  }
  if (norm) {
    norm_row_scales(a, row_scale, red);
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = b0 + j * rpb;
    if (b < a.M) {
      float v[8] = {xv[j][0].x, xv[j][0].y, xv[j][0].z, xv[j][0].w,
                    xv[j][1].x, xv[j][1].y, xv[j][1].z, xv[j][1].w};
      if (norm) {
        const float sc = row_scale[b];
        const float w[8] = {wv[0].x, wv[0].y, wv[0].z, wv[0].w, wv[1].x, wv[1].y, wv[1].z, wv[1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (v[e] * sc) * w[e];
      }
      u32x4 hi, lo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float h0 = round_bf16(v[2 * e]), h1 = round_bf16(v[2 * e + 1]);
        hi[e] = pack_bf16x2(h0, h1);
        lo[e] = pack_bf16x2(v[2 * e] - h0, v[2 * e + 1] - h1);
      }
      *(u32x4 *)(xs + b * ldx + kk) = hi;
      *(u32x4 *)(xs + (LO + b) * ldx + kk) = lo;
    }
  }
}
// One straight-line prologue per mode when one batch of pieces and scales
// per thread covers the rows (up to a few rows: the Qwen3.5-0.8B forward at
// one row 0.892 against 0.904 ms staged in rounds), else rounds, or (KM: the
// 16-row kernels) the column-major pieces where they fit.
template <int NT, bool KM>
__device__ __forceinline__ void stage_x_fc(const GemvArgs &a, uint16_t *xs, float *ss, int k0, int Kc,
                                           int LO, int nsc, int rows0, int gps) {
  const bool one = a.M * (Kc / 8) <= NT && nsc <= NT && a.M <= NT / 64;
  const int per_row = Kc / 8;
  const bool kmajor = KM && a.fc_kmajor && (a.x_mode == 0 || a.x_mode == 3) && per_row <= NT &&
                      NT % per_row == 0 && a.M <= 4 * (NT / per_row) && a.M <= 16;
  if (KM && !one && kmajor)
    stage_x_fc_kmajor<NT>(a, xs, ss, k0, Kc, LO, nsc, rows0, gps);
  else if (!one)
    stage_x_fc_rounds<NT>(a, xs, ss, k0, Kc, LO, nsc, rows0, gps);
  else if (a.x_mode == 3)
    stage_x_fc_impl<NT, 3, 1>(a, xs, ss, k0, Kc, LO, nsc, rows0, gps);
  else if (a.x_mode == 1)
    stage_x_fc_impl<NT, 1, 1>(a, xs, ss, k0, Kc, LO, nsc, rows0, gps);
  else
    stage_x_fc_impl<NT, 0, 1>(a, xs, ss, k0, Kc, LO, nsc, rows0, gps);
}

// RMSNorm factors 1/sqrt(mean(h^2) + eps) of rows [0, M) into row_scale
// (LDS; the caller's barrier publishes them). Mode 3: the sums of squares
// from the producer's partials, one wave per row, lane l adding partials l,
// l + 64, ... in that order (loads issued in batches of 4), then a fixed
// butterfly (deterministic). Mode 1: each row summed with the thread stride
// and block reduction of rxw8_dec_rmsnorm (256-thread workgroups only,
// host-checked).
__device__ __forceinline__ void norm_row_scales(const GemvArgs &a, float *row_scale, float *red) {
  const int nt = blockDim.x;
  if (a.x_mode == 3) {
    const int lane = threadIdx.x & 63, nwaves = nt >> 6;
    for (int b = threadIdx.x >> 6; b < a.M; b += nwaves) {
      float ss = 0.f;
      for (int p0 = lane; p0 < a.ss_parts; p0 += 256) {
        float t[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int p = p0 + 64 * s;
          t[s] = p < a.ss_parts ? a.ss_in[(int64_t)p * a.ss_ld + b] : 0.f;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
          if (p0 + 64 * s < a.ss_parts) ss += t[s];
      }
      ss = wave_sum64(ss);
      if (lane == 0) row_scale[b] = 1.0f / sqrtf(ss / (float)a.K + a.eps);
    }
  } else {
    for (int b = 0; b < a.M; ++b) {
      const float *h = (const float *)a.x + b * a.x_stride + a.x_off;
      float ss = 0.f;
      for (int i = threadIdx.x; i < a.K; i += nt) ss += h[i] * h[i];
      ss = block_sum_256(ss, red);
      if (threadIdx.x == 0) row_scale[b] = 1.0f / sqrtf(ss / (float)a.K + a.eps);
    }
  }
}

// Stage x[0:M, k0:k0+Kc] as bf16 into LDS rows of stride Kc + kXPad, applying
// the activation prologue (x_mode). Mode 1 sums each full row first with the
// same thread stride and block reduction as rxw8_dec_rmsnorm, so the staged
// bits equal that kernel's output. Row pieces of the norm modes are staged one
// per round trip (a piece pairs 8 row values with 8 norm weights; a batch of
// them would raise the kernel's register peak).
__device__ __forceinline__ void stage_x(const GemvArgs &a, uint16_t *xs, int k0, int Kc) {
  const int ldx = Kc + kXPad;
  const int per_row = Kc / 8;
  const int total = a.M * per_row;
  const int nt = blockDim.x;
  if (a.lds_dma) {  // x_mode 0 bf16 rows: one instruction = 64 pieces of one row
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = nt >> 6;
    for (int t = wave; t < total / 64; t += nwaves) {
      const int q0 = 64 * t, b = q0 / per_row, kk0 = (q0 - b * per_row) * 8;
      lds_dma16((const uint16_t *)a.x + b * a.x_stride + a.x_off + k0 + kk0 + 8 * lane,
                xs + b * ldx + kk0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the caller's barrier publishes the rows
    return;
  }
  if (a.x_mode == 1 || a.x_mode == 3) {
    __shared__ float red[4];
    __shared__ float row_scale[32];
    constexpr int SB = 1;
    float4 hv[SB][2], wv[SB][2];
    auto fetch = [&](int i0) {
#pragma unroll
      for (int s = 0; s < SB; ++s) {
        const int i = i0 + s * nt;
        if (i < total) {
          const int b = i / per_row, kk = (i - b * per_row) * 8;
          const float *h = (const float *)a.x + b * a.x_stride + a.x_off + k0 + kk;
          hv[s][0] = *(const float4 *)h;
          hv[s][1] = *(const float4 *)(h + 4);
          wv[s][0] = *(const float4 *)(a.norm_w + k0 + kk);
          wv[s][1] = *(const float4 *)(a.norm_w + k0 + kk + 4);
        }
      }
    };
    auto put = [&](int i0) {
#pragma unroll
      for (int s = 0; s < SB; ++s) {
        const int i = i0 + s * nt;
        if (i < total) {
          const int b = i / per_row, kk = (i - b * per_row) * 8;
          const float sc = row_scale[b];
          const float4 h0 = hv[s][0], h1 = hv[s][1], w0 = wv[s][0], w1 = wv[s][1];
          u32x4 v;
          v[0] = pack_bf16x2((h0.x * sc) * w0.x, (h0.y * sc) * w0.y);
          v[1] = pack_bf16x2((h0.z * sc) * w0.z, (h0.w * sc) * w0.w);
          v[2] = pack_bf16x2((h1.x * sc) * w1.x, (h1.y * sc) * w1.y);
          v[3] = pack_bf16x2((h1.z * sc) * w1.z, (h1.w * sc) * w1.w);
          *(u32x4 *)(xs + b * ldx + kk) = v;
        }
      }
    };
    norm_row_scales(a, row_scale, red);
    __syncthreads();
    for (int i0 = threadIdx.x; i0 < total; i0 += SB * nt) {
      fetch(i0);
      put(i0);
    }
    return;
  }
  if (a.x_mode == 2) {
    constexpr int SB = kStageBatch / 2;
    for (int i0 = threadIdx.x; i0 < total; i0 += SB * nt) {
      u32x4 gv[SB], uv[SB];
#pragma unroll
      for (int s = 0; s < SB; ++s) {
        const int i = i0 + s * nt;
        if (i < total) {
          const int b = i / per_row, kk = (i - b * per_row) * 8;
          const uint16_t *row = (const uint16_t *)a.x + b * a.x_stride;
          gv[s] = *(const u32x4 *)(row + k0 + kk);
          uv[s] = *(const u32x4 *)(row + a.K + k0 + kk);
        }
      }
#pragma unroll
      for (int s = 0; s < SB; ++s) {
        const int i = i0 + s * nt;
        if (i < total) {
          const int b = i / per_row, kk = (i - b * per_row) * 8;
          u32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float g0 = bf16_bits_to_f32(gv[s][e] & 0xffffu), g1 = bf16_bits_to_f32(gv[s][e] >> 16);
            const float u0 = bf16_bits_to_f32(uv[s][e] & 0xffffu), u1 = bf16_bits_to_f32(uv[s][e] >> 16);
            v[e] = pack_bf16x2(silu_mul_f32(g0, u0), silu_mul_f32(g1, u1));
          }
          *(u32x4 *)(xs + b * ldx + kk) = v;
        }
      }
    }
    return;
  }
  stage_rows(a.x, a.x_f32 != 0, a.x_stride, a.x_off + k0, a.M, per_row, xs, ldx, threadIdx.x, nt);
}

// row_norm: the wave loads row b's partial sums of squares, lane l taking
// partials l, l + 64, l + 128, l + 192 (ss_parts <= 256); rows b >= M load
// nothing.
__device__ __forceinline__ void row_norm_load(const GemvArgs &a, int b, float (&v)[4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int p = lane + 64 * s;
    v[s] = b < a.M && p < a.ss_parts ? a.ss_in[(int64_t)p * a.ss_ld + b] : 0.f;
  }
}

// Sums them (the order of the x_mode 3 prologue, so the factor has the same
// bits) and stores row b's factor 1/sqrt(mean + eps) in LDS at rs_off.
__device__ __forceinline__ void row_norm_store(const GemvArgs &a, int b, const float (&v)[4],
                                               void *lds) {
  const float ss = wave_sum64(((v[0] + v[1]) + v[2]) + v[3]);
  if ((threadIdx.x & 63) == 0 && b < a.M)
    ((float *)((char *)lds + a.rs_off))[b] = 1.0f / sqrtf(ss / (float)a.K + a.eps);
}

// FC epilogue (ksplit 1, N % 16 == 0): the hi and lo sums of row t (batch
// columns t and LO + t: the same lane for MB == 2, lanes col and col ^ 8 for
// MB == 1) are added, scaled (per-channel) and stored as f32 without bf16
// rounding: y_mode 0 y[t, n] = v; 1 h[t, n] += v (with ss_out); 2 (SwiGLU
// tiles) y[t, c] = silu(gate) * up.
template <int MB>
__device__ __forceinline__ void finish_fc(const GemvArgs &a, int rows0, int rg, f32x4 (&total)[MB],
                                          bool scale_here) {
  const int lane = threadIdx.x & 63, j = lane >> 4, col = lane & 15;
  f32x4 v;
  if (MB == 2) {
    v = total[0] + total[MB - 1];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = total[0][i] + __shfl_xor(total[0][i], 8);
  }
  const int t = col;
  const bool valid = (MB == 2 || col < 8) && t < a.M;
  const int n = rows0 + rg * 16 + 4 * j;
  if (n >= a.N) return;  // uniform per wave (N % 16 == 0)
  if (scale_here) {
    const float4 s4 = *(const float4 *)(a.scale + n);
    v *= f32x4{s4.x, s4.y, s4.z, s4.w};
  }
  if (a.y_mode == 2) {  // gate values in lanes j < 2, the matching up values 32 lanes higher
    f32x4 up;
#pragma unroll
    for (int i = 0; i < 4; ++i) up[i] = value_xor32(v[i]);
    if (j < 2 && valid) {
      const int c = (rows0 + rg * 16) / 2 + 4 * j;
      *(float4 *)((float *)a.y + (int64_t)t * (a.N / 2) + c) =
          float4{silu_mul_f32(v[0], up[0]), silu_mul_f32(v[1], up[1]), silu_mul_f32(v[2], up[2]),
                 silu_mul_f32(v[3], up[3])};
    }
    return;
  }
  float ss = 0.f;
  if (valid) {
    float4 *yp = (float4 *)((float *)a.y + (int64_t)t * a.N + n);
    if (a.y_mode == 1) {  // f32 residual: h += result
      float4 o = *yp;
      o.x += v[0], o.y += v[1], o.z += v[2], o.w += v[3];
      *yp = o;
      ss = ((o.x * o.x + o.y * o.y) + o.z * o.z) + o.w * o.w;
    } else {
      *yp = float4{v[0], v[1], v[2], v[3]};
    }
  }
  if (a.ss_out) {  // 4 lanes (j) hold the group's 16 channels of row t
    ss = sum_xor16(ss);
    ss = sum_xor32(ss);
    if (j == 0 && valid) a.ss_out[(int64_t)((rows0 + rg * 16) / 16) * a.ss_ld + t] = ss;
  }
}

// Reduce the KW k-slices of each row group through LDS (slice order), then
// write the tile (ksplit == 1, scaled here when per-channel) or its partial.
// With row_norm, every wave of the workgroup calls this after storing its
// rows' factors in LDS (at rs_off); the first barrier here publishes them.
// Residual operands of the epilogue (y_mode 1, one split) that the kernel
// loaded at its start, beside its first weight group: row b = col + 16 mb's
// values h[b, n .. n + 3] and the next norm's weights (with xw_out), so the
// epilogue waits on no memory round trip of its own.
template <int MB>
struct ResidualPrefetch {
  bool valid = false;
  float4 h[MB];
  float4 w;
};

template <int MB, int RW, int NW = 4, bool RN = false, bool FC = false>
__device__ __forceinline__ void finish_tile(const GemvArgs &a, float *red, int rows0, int sp,
                                            f32x4 (&total)[MB], bool scale_here,
                                            const ResidualPrefetch<MB> *pre = nullptr) {
  constexpr int KW = NW / RW;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rg = wave % RW, kq = wave / RW;
  if (KW == 1 && RN) __syncthreads();
  if (KW > 1) {
    __syncthreads();  // staged x/scales are no longer read; reuse LDS
    if (kq > 0)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        *(f32x4 *)(red + (((kq - 1) * RW + rg) * MB + mb) * 256 + lane * 4) = total[mb];
    __syncthreads();
    if (kq > 0) return;
#pragma unroll
    for (int q = 1; q < KW; ++q)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        total[mb] += *(const f32x4 *)(red + (((q - 1) * RW + rg) * MB + mb) * 256 + lane * 4);
  }
  if (FC) {
    finish_fc<MB>(a, rows0, rg, total, scale_here);
    return;
  }
  const int j = lane >> 4, col = lane & 15;
  if (RN) {
    const float *rs = (const float *)((const char *)red + a.rs_off);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) total[mb] *= rs[min(col + 16 * mb, a.M - 1)];
  }
  const int n = rows0 + rg * 16 + 4 * j;
  if (n >= a.N) return;  // uniform per wave when N % 16 == 0 (the only case modes 2 and ss use)
  if (a.ksplit > 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int b = col + 16 * mb;
      if (b < a.M) *(f32x4 *)(a.ws + ((int64_t)sp * a.M + b) * a.N + n) = total[mb];
    }
    return;
  }
  f32x4 sc = {1.f, 1.f, 1.f, 1.f};
  if (scale_here) {
    const float4 s4 = *(const float4 *)(a.scale + n);
    sc = f32x4{s4.x, s4.y, s4.z, s4.w};
  }
  if (a.y_mode == 2) {
    // gate values sit in lanes j < 2, the matching up values 32 lanes higher
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const f32x4 v = total[mb] * sc;
      f32x4 up;
#pragma unroll
      for (int i = 0; i < 4; ++i) up[i] = value_xor32(v[i]);
      const int b = col + 16 * mb;
      if (j < 2 && b < a.M) {
        const int c = (rows0 + rg * 16) / 2 + 4 * j;  // first of 4 output channels
        uint2 o = {pack_bf16x2(silu_mul_f32(round_bf16(v[0]), round_bf16(up[0])),
                               silu_mul_f32(round_bf16(v[1]), round_bf16(up[1]))),
                   pack_bf16x2(silu_mul_f32(round_bf16(v[2]), round_bf16(up[2])),
                               silu_mul_f32(round_bf16(v[3]), round_bf16(up[3])))};
        *(uint2 *)((uint16_t *)a.y + (int64_t)b * (a.N / 2) + c) = o;
      }
    }
    return;
  }
  const bool have_pre = pre && pre->valid;
  const float4 xw_w = have_pre ? pre->w
                      : a.xw_out ? *(const float4 *)(a.xw_norm + n) : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int b = col + 16 * mb;
    float ss = b < a.M ? store_out(a.y, a.y_f32, a.y_mode, a.N, b, n, total[mb] * sc,
                                   have_pre ? pre->h[mb]
                                   : a.y_mode == 1 ? *(const float4 *)((const float *)a.y + (int64_t)b * a.N + n)
                                                   : float4{0.f, 0.f, 0.f, 0.f},
                                   a.xw_out, xw_w)
                       : 0.f;
    if (a.ss_out) {  // 4 lanes (j) hold the group's 16 channels of row b
      ss = sum_xor16(ss);
      ss = sum_xor32(ss);
      if (j == 0 && b < a.M) a.ss_out[(int64_t)((rows0 + rg * 16) / 16) * a.ss_ld + b] = ss;
    }
  }
}

// PK (packed): weights in the tiled layout [N/16][K/64][64 lanes][16 B] where
// block (t, c) holds, for lane l, the 16 codes W[16t + l%16][64c + 16(l/16) ..]:
// every wave load is then one contiguous 1 KiB block (rxw8_pack_w8 builds it).
// Row-major weights ([N, K], the reference's U8 storage) use PK = false.
// NW: waves per workgroup (4, or 8 / 16 for the wide decode variants that
// give one workgroup more loads in flight instead of splitting K over
// workgroups).
// XG: bf16 activation rows (x_mode 0, per-channel scales) are read as MFMA B
// fragments straight from global memory -- the rows are tiny next to the
// weights and shared by every workgroup, so they stay in L2 -- and prefetched
// with the weights in the same double-buffered groups: no LDS staging, no
// barrier before the stream, and LDS only for the cross-wave reduction (so it
// does not limit how many workgroups a CU holds).
// RN: row_norm (the _rn kernels; the host sets a.row_norm for them only).
// FC: compute dtype F32 (the _fc kernels): f32 rows staged as bf16 hi / lo
// parts (stage_x_fc; rows b and LO + b, LO = 8 MB), the codes as the exact
// bf16 values u - 128 (no all-ones correction), f32 results (finish_fc).
// RC: the reference's cast point (the _rc kernels, layers.rs:277-296): each
// A-fragment element is the dequantised weight rounded to bf16,
// bf16((u - 128) * s[n, k / G]), so the product is
// sum_k bf16(x) * bf16(dequant(W)) in f32, with no all-ones correction and no
// scale after the sum. Lane l's row n takes its scale from global memory once
// (per-channel) or from the staged scale tile per 64-k chunk (grouped).
// blk: the workgroup's tile (x split) index, blockIdx.x except in grouped
// launches.
template <int MB, int RW, int U, bool PK, int NW = 4, bool XG = false, bool RN = false,
          bool FC = false, bool RC = false>
__device__ __forceinline__ void gemv_w8(const GemvArgs &a, const int blk) {
  constexpr int LO = 8 * MB;  // FC: staged row of the lo part of row 0
  constexpr int KW = NW / RW;
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rg = wave % RW, kq = wave / RW;
  const int tile = blk / a.ksplit;
  const int sp = blk - tile * a.ksplit;
  const int Kc = a.K / a.ksplit;
  const int k0 = sp * Kc;
  const int Kw = Kc / KW;                   // this wave's slice of the split
  const int rows0 = tile * 16 * RW;
  const int row0 = rows0 + rg * 16;
  const bool active = row0 < a.N;
  const bool per_channel = a.G == a.K;
  const int chunks = Kw / 64;
  const int chunks_per_group = per_channel ? chunks : a.G / 64;
  const int groups = a.K / a.G;
  const int ldx = Kc + kXPad;
  const int r = lane & 15, j = lane >> 4, col = lane & 15;
  const int kbase = kq * Kw;  // offset of this wave's slice within the split
  // Inactive row groups (past N) re-read the tile's first rows; nothing of
  // theirs is stored.
  const int wrow16 = (active ? row0 : rows0) / 16;
  const uint8_t *wp;
  int64_t wstep;
  if (PK) {
    wp = (const uint8_t *)a.w + ((int64_t)wrow16 * (a.K / 64) + (k0 + kbase) / 64) * 1024 + lane * 16;
    wstep = 1024;
  } else {
    wp = (const uint8_t *)a.w + (int64_t)(wrow16 * 16 + r) * a.K + k0 + kbase + j * 16;
    wstep = 64;
  }
  const int last = chunks - 1;
  // B-operand rows: batch column col + 16*mb, clamped to a valid row (LDS
  // rows are set after staging; XG reads the global rows)
  const uint16_t *xrow[MB];
  if (XG)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int b = col + 16 * mb;
      xrow[mb] = (const uint16_t *)a.x + (int64_t)(b < a.M ? b : a.M - 1) * a.x_stride + a.x_off +
                 k0 + kbase + j * 16;
    }
  u32x4 bufA[U], bufB[U];
  u32x4 xgA[XG ? U : 1][MB][2], xgB[XG ? U : 1][MB][2];
  auto load_group = [&](u32x4(&wb)[U], u32x4(&xg)[XG ? U : 1][MB][2], int c0) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      wb[u] = __builtin_nontemporal_load((const u32x4 *)(wp + (int64_t)min(c0 + u, last) * wstep));
    if (XG)
#pragma unroll
      for (int u = 0; u < (XG ? U : 1); ++u)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const u32x4 *xp = (const u32x4 *)(xrow[mb] + (int64_t)min(c0 + u, last) * 64);
          xg[u][mb][0] = xp[0];
          xg[u][mb][1] = xp[1];
        }
  };
  // The first weight group is in flight while x and the scales are staged.
  load_group(bufA, xgA, 0);
  // Residual epilogue in this launch (the waves that run it): its h values
  // and next-norm weights load now, with the first weights.
  ResidualPrefetch<MB> pre;
  if (!FC && a.y_mode == 1 && a.ksplit == 1 && kq == 0 && active) {
    const int n = row0 + 4 * j;
    pre.valid = true;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int b = col + 16 * mb;
      pre.h[mb] = b < a.M ? *(const float4 *)((const float *)a.y + (int64_t)b * a.N + n)
                          : float4{0.f, 0.f, 0.f, 0.f};
    }
    pre.w = a.xw_out ? *(const float4 *)(a.xw_norm + n) : float4{0.f, 0.f, 0.f, 0.f};
  }
  // row_norm: the partials arrive during the stream and are reduced after it
  // (KW > 1: finish_tile's first barrier publishes the factors)
  // (wave w: row w; rows past the wave count are loaded after the stream)
  float rnv[4];
  if (RN) row_norm_load(a, wave, rnv);

  // Plain activation rows with per-channel scales (when the host chose it):
  // every wave stages only its own K slice of the rows, in its own LDS region
  // (M rows of stride Kw + kXPad), and starts its loop as soon as that slice
  // is in -- no workgroup barrier before the weights stream. (Waves of
  // different row groups stage the same slice.)
  const bool wave_stage = a.wave_stage && a.x_mode == 0 && per_channel;
  const uint16_t *xbase = xs;
  int xld = ldx;
  const int gps = per_channel ? 0 : Kc / a.G;
  float *ss = (float *)(xs + (FC ? 2 * LO : a.M) * ldx);
  if (XG) {
    // nothing to stage: per-channel scales are read in the epilogue
  } else if (wave_stage) {
    uint16_t *xw = xs + wave * a.M * (Kw + kXPad);
    stage_rows(a.x, a.x_f32 != 0, a.x_stride, a.x_off + k0 + kbase, a.M, Kw / 8, xw, Kw + kXPad,
               lane, 64);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    xbase = xw - kbase;  // row b of the slice starts at xbase + b * xld + kbase
    xld = Kw + kXPad;
  } else {
    // Grouped scales of this workgroup's rows and K-split, staged after x:
    // ss[row_in_block * gps + g_local] (f32).
    if (FC) {
      stage_x_fc<NW * 64, MB == 2>(a, xs, ss, k0, Kc, LO, per_channel ? 0 : 16 * RW * gps, rows0, gps);
    } else {
      if (!per_channel) {
        const int g0 = k0 / a.G;
        for (int i = threadIdx.x; i < 16 * RW * gps; i += blockDim.x) {
          const int rr = i / gps, gl = i - rr * gps;
          const int n = rows0 + rr;
          ss[i] = n < a.N ? a.scale[(int64_t)n * groups + g0 + gl] : 0.f;
        }
      }
      stage_x(a, xs, k0, Kc);
    }
    __syncthreads();
  }

  f32x4 acc[MB], ones[MB], total[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    ones[mb] = acc[mb];
    total[mb] = acc[mb];
  }
  if (!XG)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int b = col + 16 * mb;
      // FC: column b < LO reads the hi part of row b, column LO + t the lo
      // part of row t (rows clamped to M - 1, never stored)
      const int row = FC ? (b >= LO ? LO : 0) + min(b >= LO ? b - LO : b, a.M - 1)
                         : (b < a.M ? b : a.M - 1);
      xrow[mb] = xbase + row * xld + kbase + j * 16;
    }
  const u32x4 ones_bits = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  const bf16x8 onesf = as_bf16x8(ones_bits);
  // RC with per-channel scales: lane l's row scale (rows of inactive groups
  // repeat the tile's first rows, as their weights do)
  float s_lane = 0.f;
  if (RC && per_channel) s_lane = a.scale[(int64_t)wrow16 * 16 + r];

  // Process one 64-k chunk c (of this wave's slice) held in register slice w
  // (XG: with its activation fragments xg).
  auto process = [&](const u32x4 w, const u32x4(&xg)[MB][2], const int c) {
    uint2 p0, p1, p2, p3;
    if (RC) {
      const float s = per_channel ? s_lane : ss[(rg * 16 + r) * gps + (kbase + c * 64) / a.G];
      const float ms = -128.f * s;
      p0 = u8x4_to_dq_bf16x4(w[0], s, ms), p1 = u8x4_to_dq_bf16x4(w[1], s, ms);
      p2 = u8x4_to_dq_bf16x4(w[2], s, ms), p3 = u8x4_to_dq_bf16x4(w[3], s, ms);
    } else if (FC) {
      p0 = u8x4_to_signed_bf16x4(w[0]), p1 = u8x4_to_signed_bf16x4(w[1]);
      p2 = u8x4_to_signed_bf16x4(w[2]), p3 = u8x4_to_signed_bf16x4(w[3]);
    } else {
      p0 = u8x4_to_bf16x4(w[0]), p1 = u8x4_to_bf16x4(w[1]);
      p2 = u8x4_to_bf16x4(w[2]), p3 = u8x4_to_bf16x4(w[3]);
    }
    const u32x4 a0 = {p0.x, p0.y, p1.x, p1.y}, a1 = {p2.x, p2.y, p3.x, p3.y};
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const u32x4 *xp = (const u32x4 *)(xrow[mb] + c * 64);
      const bf16x8 x0 = as_bf16x8(XG ? xg[mb][0] : xp[0]), x1 = as_bf16x8(XG ? xg[mb][1] : xp[1]);
      acc[mb] = mfma16x16x32(as_bf16x8(a0), x0, acc[mb]);
      acc[mb] = mfma16x16x32(as_bf16x8(a1), x1, acc[mb]);
      if (!FC && !RC) {
        ones[mb] = mfma16x16x32(onesf, x0, ones[mb]);
        ones[mb] = mfma16x16x32(onesf, x1, ones[mb]);
      }
    }
    if (!RC && !per_channel && ((c + 1) % chunks_per_group) == 0) {
      // fold one scale group: total += s[n, g] * (acc - 128 * ones) (FC: acc)
      const int gl = (kbase + c * 64) / a.G;
      const float *srow = ss + (rg * 16 + 4 * j) * gps + gl;
      const f32x4 sc = {srow[0], srow[gps], srow[2 * gps], srow[3 * gps]};
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        total[mb] += sc * (FC ? acc[mb] : acc[mb] - 128.f * ones[mb]);
        acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
        ones[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  // A/B double buffer: issue B, consume A, issue A', consume B.
  // chunks % (2U) == 0 (host); loads past the last chunk are clamped to it.
  for (int c0 = 0; c0 < chunks; c0 += 2 * U) {
    load_group(bufB, xgB, c0 + U);
#pragma unroll
    for (int u = 0; u < U; ++u) process(bufA[u], xgA[XG ? u : 0], c0 + u);
    load_group(bufA, xgA, c0 + 2 * U);
#pragma unroll
    for (int u = 0; u < U; ++u) process(bufB[u], xgB[XG ? u : 0], c0 + U + u);
  }
  if (per_channel || RC)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) total[mb] = (FC || RC) ? acc[mb] : acc[mb] - 128.f * ones[mb];
  if (RN) {
    row_norm_store(a, wave, rnv, xs);
    for (int b = wave + NW; b < a.M; b += NW) {  // rows beyond the wave count
      row_norm_load(a, b, rnv);
      row_norm_store(a, b, rnv, xs);
    }
  }
  finish_tile<MB, RW, NW, RN, FC>(a, (float *)xs, rows0, sp, total, per_channel && !RC, &pre);
}

// One workgroup of a grouped launch: find its problem (uniform scan of the
// problem table), then run that problem's tile with the problem's operands.
template <int RW, int U, bool PK, int NW, bool RC>
__device__ __forceinline__ void gemv_group(const GemvGroupArgs &g) {
  int p = 0;
  while (p + 1 < g.count && (int)blockIdx.x >= g.p[p + 1].tile_begin) ++p;
  const GemvProblem &q = g.p[p];
  GemvArgs a = g.base;
  a.x = q.x;
  a.w = q.w;
  a.scale = q.scale;
  a.y = q.y;
  a.M = q.M;
  a.N = q.N;
  a.K = q.K;
  a.G = q.G;
  a.x_f32 = q.x_f32;
  a.y_f32 = q.y_f32;
  a.lds_dma = q.lds_dma;
  a.wave_stage = q.wave_stage;
  a.x_stride = q.K;
  a.ss_ld = q.M;
  gemv_w8<1, RW, U, PK, NW, false, false, false, RC>(a, (int)blockIdx.x - q.tile_begin);
}

// Dense bf16 weights (lm_head): one 16-byte slice = one MFMA A-fragment.
// PK: tiled layout [N/16][K/32][64 lanes][16 B], lane l holding
// W[16t + l%16][32c + 8(l/16) .. +8] (rxw8_pack_bf16 builds it).
template <int MB, int RW, int U, bool PK, bool RN = false>
__device__ __forceinline__ void gemv_bf16(const GemvArgs &a) {
  constexpr int KW = 4 / RW;
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rg = wave % RW, kq = wave / RW;
  const int tile = blockIdx.x / a.ksplit;
  const int sp = blockIdx.x - tile * a.ksplit;
  const int Kc = a.K / a.ksplit;
  const int k0 = sp * Kc;
  const int Kw = Kc / KW;
  const int rows0 = tile * 16 * RW;
  const int row0 = rows0 + rg * 16;
  const bool active = row0 < a.N;
  const int ldx = Kc + kXPad;
  const int r = lane & 15, j = lane >> 4, col = lane & 15;

  const int wrow16 = (active ? row0 : rows0) / 16;
  const uint16_t *wrow;
  int64_t wstep;
  if (PK) {
    wrow = (const uint16_t *)a.w + ((int64_t)wrow16 * (a.K / 32) + (k0 + kq * Kw) / 32) * 512 +
           lane * 8;
    wstep = 512;
  } else {
    wrow = (const uint16_t *)a.w + (int64_t)(wrow16 * 16 + r) * a.K + k0 + kq * Kw + j * 8;
    wstep = 32;
  }
  const int steps = Kw / 32;
  const int last = steps - 1;
  u32x4 bufA[U], bufB[U];
  // The first weight group is in flight while x is staged.
#pragma unroll
  for (int u = 0; u < U; ++u)
    bufA[u] = __builtin_nontemporal_load((const u32x4 *)(wrow + (int64_t)min(u, last) * wstep));
  // row_norm: the factors are published by the staging barrier (KW may be
  // 1); wave w takes rows w, w + 4, ... (the first row's partials load
  // while x is staged)
  float rnv[4];
  if (RN) row_norm_load(a, wave, rnv);
  stage_x(a, xs, k0, Kc);
  if (RN) {
    row_norm_store(a, wave, rnv, xs);
    for (int b = wave + 4; b < a.M; b += 4) {
      row_norm_load(a, b, rnv);
      row_norm_store(a, b, rnv, xs);
    }
  }
  __syncthreads();

  f32x4 total[MB];
  const uint16_t *xrow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    total[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int b = col + 16 * mb;
    xrow[mb] = xs + (b < a.M ? b : a.M - 1) * ldx + kq * Kw + j * 8;
  }
  {
    auto process = [&](const u32x4 w, const int c) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        total[mb] = mfma16x16x32(as_bf16x8(w), as_bf16x8(*(const u32x4 *)(xrow[mb] + c * 32)),
                                 total[mb]);
    };
    for (int c0 = 0; c0 < steps; c0 += 2 * U) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        bufB[u] = __builtin_nontemporal_load(
            (const u32x4 *)(wrow + (int64_t)min(c0 + U + u, last) * wstep));
#pragma unroll
      for (int u = 0; u < U; ++u) process(bufA[u], c0 + u);
#pragma unroll
      for (int u = 0; u < U; ++u)
        bufA[u] = __builtin_nontemporal_load(
            (const u32x4 *)(wrow + (int64_t)min(c0 + 2 * U + u, last) * wstep));
#pragma unroll
      for (int u = 0; u < U; ++u) process(bufB[u], c0 + U + u);
    }
  }
  finish_tile<MB, RW, 4, RN>(a, (float *)xs, rows0, sp, total, false);
}

}  // namespace

// Kernel instances. The file is compiled twice: as the gemv code object
// (names rxw8_gemv_*, the exact-code products) and, with RXW8_GEMV_RC defined
// (kernels/w8a16_gemv_rc.hip), as the gemv_rc code object: the same u8 tilings
// with the reference's cast point (template flag RC, names rxw8_gemv_rc_*).
// Building them as two objects keeps each compile at the size of one.
#ifdef RXW8_GEMV_RC
#define RXW8_RC true
#define RXW8_KN(rest) rxw8_gemv_rc_##rest
#else
#define RXW8_RC false
#define RXW8_KN(rest) rxw8_gemv_##rest
#endif

#define RXW8_GEMV_W8(MB, RW, U)                                                 \
  extern "C" __global__ void __launch_bounds__(256)                             \
      RXW8_KN(w8_mb##MB##_rw##RW##_u##U)(GemvArgs a) {                          \
    gemv_w8<MB, RW, U, false, 4, false, false, false, RXW8_RC>(a, blockIdx.x);              \
  }                                                                             \
  extern "C" __global__ void __launch_bounds__(256)                             \
      RXW8_KN(w8_pk_mb##MB##_rw##RW##_u##U)(GemvArgs a) {                       \
    gemv_w8<MB, RW, U, true, 4, false, false, false, RXW8_RC>(a, blockIdx.x);               \
  }
#define RXW8_GEMV_W8_U(MB, RW) \
  RXW8_GEMV_W8(MB, RW, 8)      \
  RXW8_GEMV_W8(MB, RW, 4)      \
  RXW8_GEMV_W8(MB, RW, 2)      \
  RXW8_GEMV_W8(MB, RW, 1)
// Wide variants: 8, 12, 14 or 16 waves per workgroup = RW row groups x NW/RW k
// slices (12 waves: 3 row groups of 4, e.g. N = 12288 in 256 workgroups).
#define RXW8_GEMV_WIDE(MB, RW, U, NW)                                           \
  extern "C" __global__ void __launch_bounds__(NW * 64)                         \
      RXW8_KN(w8_mb##MB##_rw##RW##_u##U##_w##NW)(GemvArgs a) {                  \
    gemv_w8<MB, RW, U, false, NW, false, false, false, RXW8_RC>(a, blockIdx.x);             \
  }                                                                             \
  extern "C" __global__ void __launch_bounds__(NW * 64)                         \
      RXW8_KN(w8_pk_mb##MB##_rw##RW##_u##U##_w##NW)(GemvArgs a) {               \
    gemv_w8<MB, RW, U, true, NW, false, false, false, RXW8_RC>(a, blockIdx.x);              \
  }
#define RXW8_GEMV_WIDE_U(MB, RW, NW) \
  RXW8_GEMV_WIDE(MB, RW, 4, NW)      \
  RXW8_GEMV_WIDE(MB, RW, 3, NW)      \
  RXW8_GEMV_WIDE(MB, RW, 2, NW)      \
  RXW8_GEMV_WIDE(MB, RW, 1, NW)
#define RXW8_GEMV_WIDE_RW(MB, NW) \
  RXW8_GEMV_WIDE_U(MB, 1, NW)     \
  RXW8_GEMV_WIDE_U(MB, 2, NW)     \
  RXW8_GEMV_WIDE_U(MB, 4, NW)
// XG: activations from global memory (bf16 rows, per-channel scales, M <= 16)
#define RXW8_GEMV_XG(RW, U, NW)                                                 \
  extern "C" __global__ void __launch_bounds__(NW * 64)                         \
      RXW8_KN(w8_mb1_rw##RW##_u##U##_w##NW##_xg)(GemvArgs a) {                  \
    gemv_w8<1, RW, U, false, NW, true, false, false, RXW8_RC>(a, blockIdx.x);               \
  }                                                                             \
  extern "C" __global__ void __launch_bounds__(NW * 64)                         \
      RXW8_KN(w8_pk_mb1_rw##RW##_u##U##_w##NW##_xg)(GemvArgs a) {               \
    gemv_w8<1, RW, U, true, NW, true, false, false, RXW8_RC>(a, blockIdx.x);                \
  }
#define RXW8_GEMV_XG_U(RW, NW) \
  RXW8_GEMV_XG(RW, 4, NW)      \
  RXW8_GEMV_XG(RW, 3, NW)      \
  RXW8_GEMV_XG(RW, 2, NW)      \
  RXW8_GEMV_XG(RW, 1, NW)
RXW8_GEMV_XG_U(1, 4)
RXW8_GEMV_XG_U(4, 4)
RXW8_GEMV_XG_U(1, 8)
RXW8_GEMV_XG_U(2, 8)
RXW8_GEMV_XG_U(4, 8)
RXW8_GEMV_XG_U(3, 12)
RXW8_GEMV_XG_U(1, 16)
RXW8_GEMV_XG_U(2, 16)
RXW8_GEMV_XG_U(4, 16)
RXW8_GEMV_XG_U(1, 14)
RXW8_GEMV_WIDE_RW(1, 8)
RXW8_GEMV_WIDE_RW(1, 16)
RXW8_GEMV_WIDE_RW(2, 8)
RXW8_GEMV_WIDE_RW(2, 16)
RXW8_GEMV_WIDE_U(1, 3, 12)
RXW8_GEMV_WIDE_U(2, 3, 12)
// 12 waves as 6 row groups x 2 k slices: 96-row tiles stage x once per 96
// rows (many activation rows, e.g. N = 24576 in 256 workgroups)
RXW8_GEMV_WIDE_U(1, 6, 12)
// 14 waves over K (K = 14 x 256, e.g. 3584) for narrow N in one launch
RXW8_GEMV_WIDE_U(1, 1, 14)
RXW8_GEMV_WIDE_U(2, 1, 14)

// Row-norm variants (packed weights, up to 16 rows): the decoder's projections
// whose rows are bf16(h * norm weight), and its bf16 lm_head. Names: the
// plain kernel's name + "_rn".
#define RXW8_GEMV_XG_RN(RW, U, NW)                                              \
  extern "C" __global__ void __launch_bounds__(NW * 64)                         \
      RXW8_KN(w8_pk_mb1_rw##RW##_u##U##_w##NW##_xg_rn)(GemvArgs a) {            \
    gemv_w8<1, RW, U, true, NW, true, true, false, RXW8_RC>(a, blockIdx.x);                 \
  }
#define RXW8_GEMV_WIDE_RN(RW, U, NW)                                            \
  extern "C" __global__ void __launch_bounds__(NW * 64)                         \
      RXW8_KN(w8_pk_mb1_rw##RW##_u##U##_w##NW##_rn)(GemvArgs a) {               \
    gemv_w8<1, RW, U, true, NW, false, true, false, RXW8_RC>(a, blockIdx.x);                \
  }                                                                             \
  RXW8_GEMV_XG_RN(RW, U, NW)
#define RXW8_GEMV_WIDE_RN_U(RW, NW) \
  RXW8_GEMV_WIDE_RN(RW, 4, NW)      \
  RXW8_GEMV_WIDE_RN(RW, 3, NW)      \
  RXW8_GEMV_WIDE_RN(RW, 2, NW)      \
  RXW8_GEMV_WIDE_RN(RW, 1, NW)
RXW8_GEMV_WIDE_RN_U(1, 8)
RXW8_GEMV_WIDE_RN_U(2, 8)
RXW8_GEMV_WIDE_RN_U(4, 8)
RXW8_GEMV_WIDE_RN_U(3, 12)
RXW8_GEMV_WIDE_RN_U(6, 12)
RXW8_GEMV_WIDE_RN_U(1, 16)
RXW8_GEMV_WIDE_RN_U(2, 16)
RXW8_GEMV_WIDE_RN_U(4, 16)
RXW8_GEMV_WIDE_RN_U(1, 14)
// 4-wave plans: the staged kernels (U up to 8) and the XG ones (U up to 4)
#define RXW8_GEMV_RN4(RW, U)                                                    \
  extern "C" __global__ void __launch_bounds__(256)                             \
      RXW8_KN(w8_pk_mb1_rw##RW##_u##U##_rn)(GemvArgs a) {                       \
    gemv_w8<1, RW, U, true, 4, false, true, false, RXW8_RC>(a, blockIdx.x);                 \
  }
#define RXW8_GEMV_RN4_U(RW) \
  RXW8_GEMV_RN4(RW, 8)      \
  RXW8_GEMV_RN4(RW, 4)      \
  RXW8_GEMV_RN4(RW, 2)      \
  RXW8_GEMV_RN4(RW, 1)      \
  RXW8_GEMV_XG_RN(RW, 4, 4) \
  RXW8_GEMV_XG_RN(RW, 3, 4) \
  RXW8_GEMV_XG_RN(RW, 2, 4) \
  RXW8_GEMV_XG_RN(RW, 1, 4)
RXW8_GEMV_RN4_U(1)
RXW8_GEMV_RN4_U(4)

RXW8_GEMV_W8_U(1, 1)
RXW8_GEMV_W8_U(1, 4)
RXW8_GEMV_W8_U(2, 1)
RXW8_GEMV_W8_U(2, 4)

// Grouped launches (rxw8_quantized_linear_group): 12 waves, staged x, up to
// 16 activation rows, RW row groups of 16 rows x 12 / RW k slices (the host
// picks 6 up to 4 rows, 12 beyond: x staged once per 96 / 192 weight rows).
#define RXW8_GEMV_GRP(RW, U)                                                    \
  extern "C" __global__ void __launch_bounds__(768)                             \
      RXW8_KN(w8_mb1_rw##RW##_u##U##_w12_grp)(GemvGroupArgs g) {                \
    gemv_group<RW, U, false, 12, RXW8_RC>(g);                                   \
  }                                                                             \
  extern "C" __global__ void __launch_bounds__(768)                             \
      RXW8_KN(w8_pk_mb1_rw##RW##_u##U##_w12_grp)(GemvGroupArgs g) {             \
    gemv_group<RW, U, true, 12, RXW8_RC>(g);                                    \
  }
RXW8_GEMV_GRP(3, 4)
RXW8_GEMV_GRP(3, 2)
RXW8_GEMV_GRP(3, 1)
RXW8_GEMV_GRP(6, 4)
RXW8_GEMV_GRP(6, 2)
RXW8_GEMV_GRP(6, 1)
RXW8_GEMV_GRP(12, 4)
RXW8_GEMV_GRP(12, 2)
RXW8_GEMV_GRP(12, 1)

#ifndef RXW8_GEMV_RC
// Dense bf16 weights and the F32-compute kernels exist once (no RC form).
#define RXW8_GEMV_BF16(MB, RW, U)                                               \
  extern "C" __global__ void __launch_bounds__(256)                             \
      rxw8_gemv_bf16_mb##MB##_rw##RW##_u##U(GemvArgs a) {                       \
    gemv_bf16<MB, RW, U, false>(a);                                             \
  }                                                                             \
  extern "C" __global__ void __launch_bounds__(256)                             \
      rxw8_gemv_bf16_pk_mb##MB##_rw##RW##_u##U(GemvArgs a) {                    \
    gemv_bf16<MB, RW, U, true>(a);                                              \
  }
#define RXW8_GEMV_BF16_U(MB, RW) \
  RXW8_GEMV_BF16(MB, RW, 8)      \
  RXW8_GEMV_BF16(MB, RW, 4)      \
  RXW8_GEMV_BF16(MB, RW, 2)      \
  RXW8_GEMV_BF16(MB, RW, 1)
RXW8_GEMV_BF16_U(1, 1)
RXW8_GEMV_BF16_U(1, 4)
RXW8_GEMV_BF16_U(2, 1)
RXW8_GEMV_BF16_U(2, 4)
#define RXW8_GEMV_BF16_RN(RW, U)                                                \
  extern "C" __global__ void __launch_bounds__(256)                             \
      rxw8_gemv_bf16_pk_mb1_rw##RW##_u##U##_rn(GemvArgs a) {                    \
    gemv_bf16<1, RW, U, true, true>(a);                                         \
  }
RXW8_GEMV_BF16_RN(1, 8)
RXW8_GEMV_BF16_RN(1, 4)
RXW8_GEMV_BF16_RN(1, 2)
RXW8_GEMV_BF16_RN(1, 1)
RXW8_GEMV_BF16_RN(4, 8)
RXW8_GEMV_BF16_RN(4, 4)
RXW8_GEMV_BF16_RN(4, 2)
RXW8_GEMV_BF16_RN(4, 1)

// F32-compute variants (packed weights, up to 16 rows as 2 x 16 staged
// rows, MB = 2; up to 8 rows as 2 x 8, MB = 1). Names: plain name + "_fc".
// Workgroup (x, y) runs tile x over row chunk y, so the chunks of a longer
// input run side by side (they write disjoint rows). (No gridDim or division
// here: reading the grid size put a vector load and its wait in front of the
// first weight group's use.)
template <int MB, int RW, int U, int NW>
__device__ __forceinline__ void gemv_fc_rows(const GemvArgs &a) {
  const int m0 = (int)blockIdx.y * a.chunk_rows;
  GemvArgs c = a;
  c.x = (const float *)a.x + m0 * a.x_stride;
  c.y = (float *)a.y + (int64_t)m0 * (a.y_mode == 2 ? a.N / 2 : a.N);
  if (a.ss_out) c.ss_out = a.ss_out + m0;
  if (a.ss_in) c.ss_in = a.ss_in + m0;
  c.M = min(a.chunk_rows, a.M - m0);
  gemv_w8<MB, RW, U, true, NW, false, false, true>(c, blockIdx.x);
}
#define RXW8_GEMV_FC_WIDE(MB, RW, U, NW)                                        \
  extern "C" __global__ void __launch_bounds__(NW * 64)                         \
      rxw8_gemv_w8_pk_mb##MB##_rw##RW##_u##U##_w##NW##_fc(GemvArgs a) {         \
    gemv_fc_rows<MB, RW, U, NW>(a);                                             \
  }
#define RXW8_GEMV_FC_WIDE_U(MB, RW, NW) \
  RXW8_GEMV_FC_WIDE(MB, RW, 4, NW)      \
  RXW8_GEMV_FC_WIDE(MB, RW, 3, NW)      \
  RXW8_GEMV_FC_WIDE(MB, RW, 2, NW)      \
  RXW8_GEMV_FC_WIDE(MB, RW, 1, NW)
#define RXW8_GEMV_FC4(MB, RW, U)                                                \
  extern "C" __global__ void __launch_bounds__(256)                             \
      rxw8_gemv_w8_pk_mb##MB##_rw##RW##_u##U##_fc(GemvArgs a) {                 \
    gemv_fc_rows<MB, RW, U, 4>(a);                                              \
  }
#define RXW8_GEMV_FC_MB(MB)      \
  RXW8_GEMV_FC4(MB, 1, 8)        \
  RXW8_GEMV_FC4(MB, 1, 4)        \
  RXW8_GEMV_FC4(MB, 1, 2)        \
  RXW8_GEMV_FC4(MB, 1, 1)        \
  RXW8_GEMV_FC4(MB, 4, 8)        \
  RXW8_GEMV_FC4(MB, 4, 4)        \
  RXW8_GEMV_FC4(MB, 4, 2)        \
  RXW8_GEMV_FC4(MB, 4, 1)        \
  RXW8_GEMV_FC_WIDE_U(MB, 1, 8)  \
  RXW8_GEMV_FC_WIDE_U(MB, 2, 8)  \
  RXW8_GEMV_FC_WIDE_U(MB, 4, 8)  \
  RXW8_GEMV_FC_WIDE_U(MB, 1, 16) \
  RXW8_GEMV_FC_WIDE_U(MB, 2, 16) \
  RXW8_GEMV_FC_WIDE_U(MB, 4, 16) \
  RXW8_GEMV_FC_WIDE_U(MB, 3, 12) \
  RXW8_GEMV_FC_WIDE_U(MB, 1, 14)
RXW8_GEMV_FC_MB(1)
RXW8_GEMV_FC_MB(2)
RXW8_GEMV_FC_WIDE_U(1, 6, 12)

// Second launch of a split GEMV: y[b, n] = s[n] * sum_sp ws[sp, b, n] (split
// order), rounded to bf16. One thread per 4 consecutive outputs.
extern "C" __global__ void __launch_bounds__(256) rxw8_gemv_splitk_reduce(SplitkReduceArgs a) {
  const int64_t quads = (int64_t)a.M * a.N / 4;
  for (int64_t qd = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; qd < quads;
       qd += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = qd * 4;
    const int b = (int)(e / a.N), n = (int)(e - (int64_t)b * a.N);
    // residual and scale loads go out with the first batch of partials
    const float4 h0 = a.y_mode == 1 ? *(const float4 *)((const float *)a.y + (int64_t)b * a.N + n)
                                    : float4{0.f, 0.f, 0.f, 0.f};
    const float4 s4 = a.scale ? *(const float4 *)(a.scale + n) : float4{1.f, 1.f, 1.f, 1.f};
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < a.ksplit; s0 += 4) {  // 4 partial loads in flight, summed in split order
      float4 p[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (s0 + t < a.ksplit) p[t] = *(const float4 *)(a.ws + ((int64_t)(s0 + t) * a.M + b) * a.N + n);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (s0 + t < a.ksplit) sum += f32x4{p[t].x, p[t].y, p[t].z, p[t].w};
    }
    if (a.scale) sum *= f32x4{s4.x, s4.y, s4.z, s4.w};
    store_out(a.y, a.y_f32, a.y_mode, a.N, b, n, sum, h0);
  }
}


// Tiled weight layouts for the packed GEMV kernels. One thread moves one
// 16-byte lane slice: dst block (t, c), lane l <- src row 16t + l%16.
struct PackArgs {
  const void *src;   // [N, K] row-major
  void *dst;         // [N/16, K/kb, 1024 B]
  int64_t n, k;      // elements
  int kb;            // k per block: 64 (u8) or 32 (bf16)
  int esize;         // bytes per element: 1 or 2
  int64_t ilv_half;  // 0, or N / 2: interleave gate/up rows (SwiGLU epilogue order)
};

extern "C" __global__ void __launch_bounds__(256) rxw8_pack_tiles(PackArgs a) {
  const int64_t blocks_k = a.k / a.kb;
  const int64_t slices = a.n / 16 * blocks_k * 64;
  const int per_lane = 16 / a.esize;  // elements per 16-byte slice
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < slices;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t blk = i >> 6;
    const int lane = (int)(i & 63);
    const int64_t t = blk / blocks_k, c = blk - t * blocks_k;
    int64_t row = 16 * t + (lane & 15);
    if (a.ilv_half)  // SwiGLU row order: 8 gate rows then the 8 matching up rows
      row = (lane & 15) < 8 ? 8 * t + (lane & 15) : a.ilv_half + 8 * t + (lane & 15) - 8;
    const int64_t kk = c * a.kb + (int64_t)(lane >> 4) * per_lane;
    const u32x4 v = *(const u32x4 *)((const char *)a.src + (row * a.k + kk) * a.esize);
    *(u32x4 *)((char *)a.dst + i * 16) = v;
  }
}
#endif  // !RXW8_GEMV_RC
