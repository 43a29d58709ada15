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
