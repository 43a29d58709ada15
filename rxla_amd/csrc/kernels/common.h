// Shared device helpers for the rxw8 gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned u32x4;

#define RXW8_WAVE 64

// bf16 bits -> f32 (exact).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

// f32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  bf16_t b = (bf16_t)f;
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two f32 -> packed bf16x2 (low half = a), round to nearest even: one
// v_cvt_pk_bf16_f32, the same conversion as f32_to_bf16_bits.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// Four u8 codes of one dword -> two dwords of bf16 pairs (exact: 0..255 fit
// bf16's 8 significant bits). v_cvt_f32_ubyte{0..3} + v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint2 u8x4_to_bf16x4(uint32_t w) {
  float f0 = (float)(w & 0xffu);
  float f1 = (float)((w >> 8) & 0xffu);
  float f2 = (float)((w >> 16) & 0xffu);
  float f3 = (float)(w >> 24);
  return uint2{pack_bf16x2(f0, f1), pack_bf16x2(f2, f3)};
}

// Four u8 codes of one dword -> two dwords of the bf16 pairs of u - 128
// (exact: -128..127 fit bf16's 8 significant bits).
__device__ __forceinline__ uint2 u8x4_to_signed_bf16x4(uint32_t w) {
  float f0 = (float)(w & 0xffu) - 128.f;
  float f1 = (float)((w >> 8) & 0xffu) - 128.f;
  float f2 = (float)((w >> 16) & 0xffu) - 128.f;
  float f3 = (float)(w >> 24) - 128.f;
  return uint2{pack_bf16x2(f0, f1), pack_bf16x2(f2, f3)};
}

// Four u8 codes of one dword -> two dwords of bf16 pairs of the dequantised
// weights bf16((u - 128) * s), round to nearest even: the reference's
// dequantise-then-cast order (crates/rxla-nn/src/layers.rs:277-296). The f32
// product (u - 128) * s is formed as fma(u, s, ms) with ms = -128 s: -128 s is
// exact (a power-of-two multiple), so the fma's single rounding of
// u s - 128 s gives the correctly rounded product.
__device__ __forceinline__ uint2 u8x4_to_dq_bf16x4(uint32_t w, float s, float ms) {
  const float f0 = fmaf((float)(w & 0xffu), s, ms);
  const float f1 = fmaf((float)((w >> 8) & 0xffu), s, ms);
  const float f2 = fmaf((float)((w >> 16) & 0xffu), s, ms);
  const float f3 = fmaf((float)(w >> 24), s, ms);
  return uint2{pack_bf16x2(f0, f1), pack_bf16x2(f2, f3)};
}

// The values of lanes l and l ^ 16 (resp. l ^ 32), in some order, through
// v_permlane16_swap / v_permlane32_swap with both operands v: a VALU exchange
// instead of an LDS round trip (ds_bpermute). Combined with a commutative
// operation the result equals v op v[l ^ 16] bit for bit.
__device__ __forceinline__ uint2 pair_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return uint2{r[0], r[1]};
}
__device__ __forceinline__ uint2 pair_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return uint2{r[0], r[1]};
}
__device__ __forceinline__ float sum_xor16(float v) {
  const uint2 p = pair_xor16(v);
  return __uint_as_float(p.x) + __uint_as_float(p.y);
}
__device__ __forceinline__ float sum_xor32(float v) {
  const uint2 p = pair_xor32(v);
  return __uint_as_float(p.x) + __uint_as_float(p.y);
}
// v of lane l ^ 32 (the member of the pair that is not this lane's bits; equal
// bits make either the answer)
__device__ __forceinline__ float value_xor32(float v) {
  const uint2 p = pair_xor32(v);
  return __uint_as_float(p.x == __float_as_uint(v) ? p.y : p.x);
}
// Sum over the 64 lanes, butterfly order 32, 16, 8, 4, 2, 1 (the first two
// steps on the VALU exchanges)
__device__ __forceinline__ float wave_sum64(float v) {
  v = sum_xor32(v);
  v = sum_xor16(v);
  for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Raw buffer resource over [base, base + bytes) (stride 0; the gfx9 word 3
// with a 32-bit data format): a raw buffer load at a byte offset whose
// access reaches past `bytes` returns zeros and reads no memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Load 8 consecutive activations as a bf16x8 fragment from bf16 or f32 storage
// (f32 rounded to bf16, RNE -- the x.cast(BF16) of the W8A16 layer).
__device__ __forceinline__ u32x4 load_x8(const void *x, int64_t off, bool x_f32) {
  if (x_f32) {
    const float4 *p = (const float4 *)((const float *)x + off);
    float4 a = p[0], b = p[1];
    u32x4 r;
    r[0] = pack_bf16x2(a.x, a.y);
    r[1] = pack_bf16x2(a.z, a.w);
    r[2] = pack_bf16x2(b.x, b.y);
    r[3] = pack_bf16x2(b.z, b.w);
    return r;
  }
  return *(const u32x4 *)((const uint16_t *)x + off);
}

// silu(g) * u in f32 (ops.rs:331-342): sigmoid with a nonpositive exponent
// argument, so exp never overflows. Shared by the SwiGLU kernel and the GEMV
// activation prologue so both produce identical bits.
__device__ __forceinline__ float silu_mul_f32(float g, float u) {
  const float e = __expf(-fabsf(g));
  const float sig = g >= 0.f ? 1.0f / (1.0f + e) : e / (1.0f + e);
  return (g * sig) * u;
}

// Deterministic sum over a 256-thread block: wave butterfly, then the four
// wave sums in a fixed order. `red` holds 4 floats of LDS.
__device__ __forceinline__ float block_sum_256(float v, float *red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

