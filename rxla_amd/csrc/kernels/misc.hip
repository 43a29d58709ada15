// Small kernels: exact W8 dequantisation, a generic reference-order linear for
// shapes outside the MFMA tiling, and the paired KV dynamic_update_slice.
#include "common.h"

// ---- dequantisation: W = (f32(u8) + (-128)) * scale[n, k / G]
// (crates/rxla-nn/src/layers.rs:277-287). One correctly rounded f32 multiply,
// then optionally RNE to bf16 (weight.cast(BF16), layers.rs:294).
struct DequantArgs {
  const uint8_t *w;
  const float *scale;
  void *out;
  int64_t n, k, g;
  int out_bf16;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_dequant(DequantArgs a) {
  const int64_t total = a.n * a.k;
  const int64_t groups = a.k / a.g;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / a.k, c = e - r * a.k;
    const float v = ((float)a.w[e] + -128.0f) * a.scale[r * groups + c / a.g];
    if (a.out_bf16)
      ((uint16_t *)a.out)[e] = f32_to_bf16_bits(v);
    else
      ((float *)a.out)[e] = v;
  }
}

// ---- W8 encoder (benchmarks/quantize_qwen3_5_w8.py:27-44): per row and
// group of G columns, s = max(amax, 1e-12) / 127 and
// u8 = clamp(rne(w / s), -127, 127) + 128, all in f32 with a correctly rounded
// division (not a reciprocal multiply), as the encoder's torch ops compute.
// One wave per (row, group): lanes stride the group for the amax (a NaN makes
// the scale NaN, as torch's amax propagates it), a butterfly reduces it, and
// a second pass over the same (cache-resident) group writes the codes.
// A group containing NaN gets code 128 throughout: the reference's codes for
// it come from a NaN-to-uint8 cast, which torch leaves unspecified.
struct QuantizeArgs {
  const void *w;   // [n, k] f32 or bf16
  uint8_t *u8;     // [n, k]
  float *scale;    // [n, k / g]
  int64_t n, k, g;
  int w_bf16;
};

__device__ __forceinline__ float quant_load(const QuantizeArgs &a, int64_t i) {
  return a.w_bf16 ? bf16_bits_to_f32(((const uint16_t *)a.w)[i]) : ((const float *)a.w)[i];
}

extern "C" __global__ void __launch_bounds__(256) rxw8_quantize_w8(QuantizeArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t groups = a.k / a.g;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= a.n * groups) return;  // whole waves only; no barriers below
  const int64_t r = unit / groups, gi = unit - r * groups;
  const int64_t base = r * a.k + gi * a.g;
  float amax = 0.f;
  int nan = 0;
  for (int64_t i = lane; i < a.g; i += 64) {
    const float v = fabsf(quant_load(a, base + i));
    nan |= v != v;
    amax = fmaxf(amax, v);
  }
  for (int o = 32; o > 0; o >>= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, o));
    nan |= __shfl_xor(nan, o);
  }
  const float s = nan ? __builtin_nanf("") : (amax >= 1e-12f ? amax : 1e-12f) / 127.0f;
  if (lane == 0) a.scale[r * groups + gi] = s;
  for (int64_t i = lane; i < a.g; i += 64) {
    const float qf = rintf(quant_load(a, base + i) / s);
    const int code = nan ? 128 : (int)fminf(fmaxf(qf, -127.0f), 127.0f) + 128;
    a.u8[base + i] = (uint8_t)code;
  }
}

// ---- generic linear in reference order: one thread per output element.
//   compute BF16: y = bf16( sum_k bf16(x) * bf16((u8 - 128) * s) )
//   compute F32:  y = sum_k x * ((u8 - 128) * s)
// Weight kinds: 0 = u8 + scale, 1 = dense bf16.
struct GenericLinearArgs {
  const void *x;
  const void *w;
  const float *scale;
  void *y;
  int64_t m, n, k, g;
  int x_f32, y_f32, compute_bf16, w_kind;
  int y_mode;  // 1: y is an f32 residual, y += f32(bf16(result))
};

extern "C" __global__ void __launch_bounds__(256) rxw8_linear_generic(GenericLinearArgs a) {
  const int64_t total = a.m * a.n;
  const int64_t groups = a.w_kind == 0 ? a.k / a.g : 1;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = e / a.n, col = e - row * a.n;
    float acc = 0.f;
    for (int64_t i = 0; i < a.k; ++i) {
      float xv = a.x_f32 ? ((const float *)a.x)[row * a.k + i]
                         : bf16_bits_to_f32(((const uint16_t *)a.x)[row * a.k + i]);
      float wv;
      if (a.w_kind == 0)
        wv = ((float)((const uint8_t *)a.w)[col * a.k + i] + -128.0f) *
             a.scale[col * groups + i / a.g];
      else
        wv = bf16_bits_to_f32(((const uint16_t *)a.w)[col * a.k + i]);
      if (a.compute_bf16) {
        xv = round_bf16(xv);
        wv = round_bf16(wv);
      }
      acc = __fadd_rn(acc, __fmul_rn(xv, wv));
    }
    if (a.compute_bf16) acc = round_bf16(acc);
    if (a.y_mode == 1)
      ((float *)a.y)[e] += acc;
    else if (a.y_f32)
      ((float *)a.y)[e] = acc;
    else
      ((uint16_t *)a.y)[e] = f32_to_bf16_bits(acc);
  }
}

// ---- W8 linear with compute dtype F32 on the matrix cores:
//   y[t, n] = sum_k x[t, k] * ((u8[n, k] - 128) * s[n, k / G])
// (layers.rs:277-298 with an f32 compute dtype; also the tied LM head,
// qwen3_5/mod.rs:158-173). Each f32 activation is split into bf16 parts
// x = hi + lo + r, hi = bf16(x), lo = bf16(x - hi), |r| <= 2^-17 |x|; the codes
// u - 128 are exact in bf16, so v_mfma_f32_16x16x32_bf16 forms the products of
// both parts exactly and accumulates them in f32. The scale is applied per
// group to the f32 group sums (a reassociation of the reference's
// x . (q * s): both are f32 sums of the same terms up to f32 rounding).
//
// Workgroup: WV waves, 16 output channels per wave (16 WV per workgroup) and
// 16 R rows of x. The R row tiles of x (hi and lo, rows padded by 16 bytes so
// the 16 lanes reading one column group hit distinct banks) and the
// workgroup's scales are staged in LDS once; each lane then streams 16-byte
// slices of one weight row (lane = row + 16 * slice, 64 contiguous bytes per
// row per wave load) with PF loads in flight, all other reads being LDS. The
// 16 codes of a slice are the B operands of two MFMAs (k permuted identically
// in A and B). Rows of x >= T and channels >= N read clamped, valid addresses
// and are never stored. PK: the weights in the GEMV tile layout ([N / 16]
// [K / 64] tiles of 1 KiB, lane l's 16 bytes at l * 16: row l % 16, k 16 (l /
// 16) of the tile), so each wave load is one contiguous KiB (nontemporal)
// instead of 16 rows x 64 bytes.
struct LinearF32Args {
  const float *x;      // [T, K] rows of ldx elements
  const uint8_t *w;    // [N, K] rows of ldw bytes (PK: tile (0, k0 / 64) of the K range)
  const float *scale;  // [N, K / G] rows of ldsc elements
  float *y;            // [T, N]
  int T, N, K, G;
  int y_mode;          // 0: y = result; 1: y += result (f32 residual)
  int tiles;           // channel tiles (16 WV channels each) per workgroup
  int64_t ldx, ldw, ldsc;  // row strides: a K-range of a wider product (host K chunks);
                           // PK: ldw = 64-k tiles per 16-row group
};

template <int R, int WV, bool PK = false>
__device__ __forceinline__ void linear_f32_mfma(const LinearF32Args &a) {
  constexpr int PF = 8;
  extern __shared__ __attribute__((aligned(16))) uint16_t f32lin_lds[];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int K = a.K, ng = K / a.G, gs = a.G / 64, steps = K / 64;
  const int rowp = K + 8;  // bf16 elements per staged row (16-byte pad)
  uint16_t *ah = f32lin_lds;
  uint16_t *al = ah + 16 * R * rowp;
  float *sc = (float *)(al + 16 * R * rowp);
  const int m0 = blockIdx.y * 16 * R;
  // ---- stage x (split into hi / lo) once for all of this workgroup's channel tiles
  for (int e = threadIdx.x * 4; e < 16 * R * K; e += blockDim.x * 4) {
    const int m = e / K, c = e - m * K;
    const int t = min(m0 + m, a.T - 1);
    const float4 v = *(const float4 *)(a.x + (int64_t)t * a.ldx + c);
    const float xs[4] = {v.x, v.y, v.z, v.w};
    uint32_t hb[4], lb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      hb[i] = f32_to_bf16_bits(xs[i]);
      lb[i] = f32_to_bf16_bits(xs[i] - bf16_bits_to_f32(hb[i]));
    }
    *(uint2 *)(ah + m * rowp + c) = uint2{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16)};
    *(uint2 *)(al + m * rowp + c) = uint2{lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16)};
  }
  const int col = lane & 15, part = lane >> 4;
  for (int ct = 0; ct < a.tiles; ++ct) {
  const int n0 = (blockIdx.x * a.tiles + ct) * 16 * WV;
  if (n0 >= a.N) break;  // uniform
  if (ct > 0) __syncthreads();  // every wave is done with the previous tile's scales
  for (int e = threadIdx.x; e < 16 * WV * ng; e += blockDim.x) {
    const int r = e / ng, g = e - r * ng;
    const int n = min(n0 + r, a.N - 1);
    sc[e] = a.scale[(int64_t)n * a.ldsc + g];
  }
  __syncthreads();
  // ---- stream the weight rows
  const int nrow = min(n0 + 16 * wv + col, a.N - 1);
  // (PK: the wave's 16-row group, clamped like the rows; N % 16 == 0)
  const uint8_t *wp = PK ? a.w + (int64_t)min((n0 + 16 * wv) / 16, a.N / 16 - 1) * a.ldw * 1024 + lane * 16
                         : a.w + (int64_t)nrow * a.ldw + 16 * part;
  constexpr int wstep = PK ? 1024 : 64;  // bytes from one 64-k step to the next
  auto wload = [&](int st) {
    const u32x4 *p = (const u32x4 *)(wp + (int64_t)wstep * st);
    return PK ? __builtin_nontemporal_load(p) : *p;
  };
  const float *scl = sc + (16 * wv + col) * ng;
  f32x4 acc[R], accg[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    accg[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // one K step of 64: the lane's 16 codes as two bf16x8 B operands (u - 128,
  // exact), four MFMAs per row tile (hi, lo x two k halves); at the end of a
  // scale group the group sums are scaled into acc (branch-free selects keep
  // the loop body one basic block, so the load waits stay counted)
  auto step = [&](const u32x4 cur, int s) {
    u32x4 b[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const uint32_t q = cur[2 * h + d];
        b[h][2 * d] = pack_bf16x2((float)(q & 0xffu) - 128.f, (float)((q >> 8) & 0xffu) - 128.f);
        b[h][2 * d + 1] = pack_bf16x2((float)((q >> 16) & 0xffu) - 128.f, (float)(q >> 24) - 128.f);
      }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int off = (16 * r + col) * rowp + 64 * s + 16 * part;
      const u32x4 h0 = *(const u32x4 *)(ah + off), h1 = *(const u32x4 *)(ah + off + 8);
      const u32x4 l0 = *(const u32x4 *)(al + off), l1 = *(const u32x4 *)(al + off + 8);
      accg[r] = mfma16x16x32(as_bf16x8(h0), as_bf16x8(b[0]), accg[r]);
      accg[r] = mfma16x16x32(as_bf16x8(l0), as_bf16x8(b[0]), accg[r]);
      accg[r] = mfma16x16x32(as_bf16x8(h1), as_bf16x8(b[1]), accg[r]);
      accg[r] = mfma16x16x32(as_bf16x8(l1), as_bf16x8(b[1]), accg[r]);
    }
    const bool fold = (s + 1) % gs == 0;
    const float sg = fold ? scl[s / gs] : 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[r][i] += sg * accg[r][i];
        accg[r][i] = fold ? 0.f : accg[r][i];
      }
  };
  // PF slices in flight: the slice of step s + PF is requested as step s is
  // consumed (clamped to the last slice at the end: re-reads of cached bytes)
  u32x4 buf[PF];
#pragma unroll
  for (int j = 0; j < PF; ++j) buf[j] = wload(min(j, steps - 1));
  int s0 = 0;
  for (; s0 + PF <= steps; s0 += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const u32x4 cur = buf[j];
      buf[j] = wload(min(s0 + j + PF, steps - 1));
      step(cur, s0 + j);
    }
  }
#pragma unroll
  for (int j = 0; j < PF; ++j)
    if (s0 + j < steps) step(buf[j], s0 + j);
  // ---- store: lane holds rows 4 part + i of each row tile, channel n0 + 16 wv + col
  const int n = n0 + 16 * wv + col;
  if (n < a.N) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = m0 + 16 * r + 4 * part + i;
        if (t < a.T) {
          float *yp = a.y + (int64_t)t * a.N + n;
          *yp = a.y_mode == 1 ? *yp + acc[r][i] : acc[r][i];
        }
      }
  }
  }  // channel tiles
}

#define RXW8_LINEAR_F32(R, WV)                                                          \
  extern "C" __global__ void __launch_bounds__(64 * WV)                                 \
      rxw8_linear_f32_mfma_r##R##_w##WV(LinearF32Args a) {                              \
    linear_f32_mfma<R, WV>(a);                                                          \
  }                                                                                     \
  extern "C" __global__ void __launch_bounds__(64 * WV)                                 \
      rxw8_linear_f32_mfma_pk_r##R##_w##WV(LinearF32Args a) {                           \
    linear_f32_mfma<R, WV, true>(a);                                                    \
  }
RXW8_LINEAR_F32(1, 8)
RXW8_LINEAR_F32(2, 8)

// ---- paired dynamic_update_slice (KvCache::update_at[_checked],
// crates/rxla-core/src/kv_cache.rs:53-111, indexing.rs:663-678).
// starts: device I32 [rank]. Unchecked: start_i clamped to [0, dim_i - udim_i].
// Checked: no element is written unless every start is in range; accepted
// (optional) receives 1.0f or 0.0f.
struct KvUpdateArgs {
  void *kc;
  void *vc;
  const void *ku;
  const void *vu;
  const int32_t *starts;
  float *accepted;
  int64_t dims[8];
  int64_t udims[8];
  int64_t total;  // elements in the update
  int rank;
  int elem;       // bytes per element: 1, 2, 4
  int checked;
};

template <typename T>
__device__ __forceinline__ void kv_copy(const KvUpdateArgs &a, const int64_t *st) {
  int64_t ostride[8], ustride[8];
  ostride[a.rank - 1] = 1;
  ustride[a.rank - 1] = 1;
  for (int d = a.rank - 2; d >= 0; --d) {
    ostride[d] = ostride[d + 1] * a.dims[d + 1];
    ustride[d] = ustride[d + 1] * a.udims[d + 1];
  }
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < a.total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int64_t rem = e, off = 0;
    for (int d = 0; d < a.rank; ++d) {
      const int64_t idx = rem / ustride[d];
      rem -= idx * ustride[d];
      off += (st[d] + idx) * ostride[d];
    }
    ((T *)a.kc)[off] = ((const T *)a.ku)[e];
    ((T *)a.vc)[off] = ((const T *)a.vu)[e];
  }
}

extern "C" __global__ void __launch_bounds__(256) rxw8_kv_update(KvUpdateArgs a) {
  int64_t st[8];
  bool ok = true;
  for (int d = 0; d < a.rank; ++d) {
    const int64_t s = a.starts[d];
    const int64_t hi = a.dims[d] - a.udims[d];
    if (s < 0 || (hi < 2147483647LL && s > hi)) ok = false;
    st[d] = s < 0 ? 0 : (s > hi ? hi : s);
  }
  if (a.accepted && blockIdx.x == 0 && threadIdx.x == 0)
    *a.accepted = (a.checked && !ok) ? 0.0f : 1.0f;
  if (a.checked && !ok) return;
  if (a.elem == 4)
    kv_copy<uint32_t>(a, st);
  else if (a.elem == 2)
    kv_copy<uint16_t>(a, st);
  else
    kv_copy<uint8_t>(a, st);
}
