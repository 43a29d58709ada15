// K2: W8A16 prefill dequant-GEMM on gfx950 MFMA.
//
//   y[m, n] = bf16( sum_k bf16(x[m, k]) * bf16((u8[n, k] - 128) * s[n, k / G]) )
//
// i.e. exactly the reference's cast points (crates/rxla-nn/src/layers.rs:
// 277-296): the weight is dequantised in f32, rounded to bf16, contracted
// against bf16 activations with f32 accumulation, and the result rounded to
// bf16. In a GEMM each weight element is reused by a whole tile of
// activation rows, so the dequantisation is done once per element while the
// tile is staged into LDS.
//
// Tiling: a 256-thread workgroup (4 waves) computes a 128 (weight rows n) x
// 128 (activation rows m) output tile; BK = 64. Both operands are staged as
// bf16 in LDS (double-buffered; the global loads of tile k+1 are in flight
// while tile k is multiplied). Each wave owns 64 n x 64 m = 4 x 4 tiles of
// v_mfma_f32_16x16x32_bf16 with the weights as the A operand, so each lane's
// accumulators hold 4 consecutive n of one m (8-byte bf16 stores).
// Workgroups are assigned XCD-major: the GPU dispatches workgroup b to XCD
// b % 8, and this kernel maps the workgroups of one XCD onto a contiguous
// range of tiles with m fastest, so a weight tile is reused from that XCD's L2.
// Weights may be row-major [N, K] or in the tiled layout of rxw8_pack_weight.
#include "common.h"

struct GemmArgs {
  const void *x;       // [M, K] bf16 or f32
  const uint8_t *w;    // [N, K] u8 or packed [N/16, K/64, 1024]
  const float *scale;  // [N, K / G]
  void *y;             // [M, N]
  int M, N, K, G;
  int x_f32, y_f32, y_mode, w_packed;
};

namespace {

constexpr int TN = 128, TM = 128, BK = 64, LDK = BK + 8;  // LDS row stride (bf16)

__device__ __forceinline__ void gemm_store(const GemmArgs &a, int m, int n, f32x4 v) {
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

}  // namespace

extern "C" __global__ void __launch_bounds__(256) rxw8_w8a16_gemm(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sw[2][TN * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sx[2][TM * LDK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tiles_m = (a.M + TM - 1) / TM, tiles_n = a.N / TN;
  const int ntiles = tiles_m * tiles_n;
  // XCD-major tile order: workgroup b runs on XCD b % 8.
  const int b = blockIdx.x;
  const int per_xcd = (ntiles + 7) / 8;
  const int tile = (b % 8) * per_xcd + b / 8;
  if (tile >= ntiles) return;
  const int tn = tile / tiles_m, tm = tile - tn * tiles_m;
  const int n0 = tn * TN, m0 = tm * TM;
  const int groups = a.K / a.G;
  const int KT = a.K / BK;

  // staging assignment: W: 512 slices of 16 codes (row = id / 4, kq = id % 4);
  // X: 1024 slices of 8 values (row = id / 8, kq = id % 8).
  u32x4 wreg[2], xreg[4];
  float wsc[2];
  auto load_tile = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int id = tid + 256 * p, row = id >> 2, kq = id & 3;
      const int n = n0 + row;
      const uint8_t *src;
      if (a.w_packed) {
        const int l = (row & 15) + 16 * kq;
        src = a.w + (((int64_t)(n >> 4) * (a.K / 64) + kt) * 1024 + l * 16);
      } else {
        src = a.w + (int64_t)n * a.K + k0 + kq * 16;
      }
      wreg[p] = *(const u32x4 *)src;
      wsc[p] = a.scale[(int64_t)n * groups + (k0 + kq * 16) / a.G];
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int id = tid + 256 * p, row = id >> 3, kq = id & 7;
      const int m = m0 + row;
      xreg[p] = m < a.M ? load_x8(a.x, (int64_t)m * a.K + k0 + kq * 8, a.x_f32 != 0)
                        : u32x4{0, 0, 0, 0};
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int id = tid + 256 * p, row = id >> 2, kq = id & 3;
      const float s = wsc[p];
      u32x4 lo, hi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w4 = wreg[p][e];
        const float f0 = ((float)(w4 & 0xffu) + -128.0f) * s;
        const float f1 = ((float)((w4 >> 8) & 0xffu) + -128.0f) * s;
        const float f2 = ((float)((w4 >> 16) & 0xffu) + -128.0f) * s;
        const float f3 = ((float)(w4 >> 24) + -128.0f) * s;
        const uint32_t p01 = pack_bf16x2(f0, f1), p23 = pack_bf16x2(f2, f3);
        if (e < 2) {
          lo[2 * e] = p01;
          lo[2 * e + 1] = p23;
        } else {
          hi[2 * (e - 2)] = p01;
          hi[2 * (e - 2) + 1] = p23;
        }
      }
      u32x4 *dst = (u32x4 *)(sw[buf] + row * LDK + kq * 16);
      dst[0] = lo;
      dst[1] = hi;
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int id = tid + 256 * p, row = id >> 3, kq = id & 7;
      *(u32x4 *)(sx[buf] + row * LDK + kq * 8) = xreg[p];
    }
  };

  const int wn = wave & 1, wm = wave >> 1;  // wave's 64 n x 64 m quadrant
  const int r16 = lane & 15, kg = lane >> 4;
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) load_tile(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = as_bf16x8(*(const u32x4 *)(sw[buf] + (wn * 64 + i * 16 + r16) * LDK + ks * 32 + kg * 8));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bfr[j] = as_bf16x8(*(const u32x4 *)(sx[buf] + (wm * 64 + j * 16 + r16) * LDK + ks * 32 + kg * 8));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < KT) store_tile(buf ^ 1);
    __syncthreads();
  }
  // epilogue: lane holds D[n = 16i + 4kg + r][m = 16j + r16]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      gemm_store(a, m0 + wm * 64 + j * 16 + r16, n0 + wn * 64 + i * 16 + 4 * kg, acc[i][j]);
}
