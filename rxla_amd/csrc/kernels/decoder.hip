// Decoder-step kernels for the synthetic Qwen-style dense W8 decoder
// (composition of crates/rxla-models/src/qwen3_5/mod.rs:199-273 and
// layers.rs:28-101,270-293 with dense full-attention layers):
// token positions, embedding gather, RMSNorm to bf16, per-head q/k RMSNorm +
// RoPE + KV-cache append, SiLU(gate) * up, first-max argmax, length advance.
// Every kernel reads sequence lengths from device memory, so a decode step
// can be captured once in a HIP graph and replayed.
#include "common.h"

// ---- positions: token t = (b, i) sits at pos = lens[b] + i --------------------
struct DecPosArgs {
  const int32_t *lens;  // [B]
  int32_t *pos;         // [T]
  int32_t *row_seq;     // [T] cache slot of token t
  int32_t *row_len;     // [T] keys visible to token t (causal: pos + 1)
  int b, s;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_dec_positions(DecPosArgs a) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= a.b * a.s) return;
  const int bi = t / a.s;
  const int p = a.lens[bi] + (t - bi * a.s);
  a.pos[t] = p;
  a.row_seq[t] = bi;
  a.row_len[t] = p + 1;
}



// ---- embedding: h[t] = f32(E[clamp(ids[t], 0, V-1)]) (indexing.rs:637-656) ----
// Also the token positions (when lens is set): token t = (b, i) sits at
// pos = lens[b] + i, in cache slot b, and sees pos + 1 keys. With ss the
// row's sum of squares.
//
// One row by a 256-thread slice (thread t of it): with H % 8 == 0 (and
// 16-byte aligned rows), 16-byte
// pieces p = t, t + 256, ... of 8 values (loads issued 4 at a time), each
// thread summing its squares in element order; otherwise elements t, t + 256,
// .... Returns the thread's partial sum (the caller adds the slice's partials
// in block_sum_256 order). With xw, also writes xw[i] = bf16(dst[i] *
// xw_norm[i]) (the first layer's RMSNorm rows before the row factor).
__device__ __forceinline__ float embed_row(const uint16_t *src, float *dst, int64_t H, int t,
                                           const float *xw_norm = nullptr, uint16_t *xw = nullptr) {
  float ss = 0.f;
  if (H % 8 || ((uintptr_t)src | (uintptr_t)dst | (uintptr_t)xw | (uintptr_t)xw_norm) % 16) {
    for (int64_t i = t; i < H; i += 256) {
      const float v = bf16_bits_to_f32(src[i]);
      dst[i] = v;
      if (xw) xw[i] = f32_to_bf16_bits(v * xw_norm[i]);
      ss += v * v;
    }
    return ss;
  }
  const int64_t pieces = H / 8;
  for (int64_t p0 = t; p0 < pieces; p0 += 4 * 256) {
    u32x4 v[4];
    float4 wn[4][2];  // the norm weights load with the row (not after the stores)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (p0 + 256 * q < pieces) {
        v[q] = *(const u32x4 *)(src + 8 * (p0 + 256 * q));
        if (xw) {
          wn[q][0] = *(const float4 *)(xw_norm + 8 * (p0 + 256 * q));
          wn[q][1] = *(const float4 *)(xw_norm + 8 * (p0 + 256 * q) + 4);
        }
      }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (p0 + 256 * q >= pieces) break;
      float f[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[2 * e] = bf16_bits_to_f32(v[q][e] & 0xffffu);
        f[2 * e + 1] = bf16_bits_to_f32(v[q][e] >> 16);
      }
      float4 *d = (float4 *)(dst + 8 * (p0 + 256 * q));
      d[0] = float4{f[0], f[1], f[2], f[3]};
      d[1] = float4{f[4], f[5], f[6], f[7]};
      if (xw) {
        const float4 w0 = wn[q][0], w1 = wn[q][1];
        *(u32x4 *)(xw + 8 * (p0 + 256 * q)) =
            u32x4{pack_bf16x2(f[0] * w0.x, f[1] * w0.y), pack_bf16x2(f[2] * w0.z, f[3] * w0.w),
                  pack_bf16x2(f[4] * w1.x, f[5] * w1.y), pack_bf16x2(f[6] * w1.z, f[7] * w1.w)};
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
  }
  return ss;
}
struct EmbedArgs {
  const int32_t *ids;
  const uint16_t *table;  // [V, H] bf16
  float *h;               // [T, H]
  float *ss;              // optional [T]: sum of squares of each written row
  int64_t T, V, H;
  const int32_t *lens;    // optional [B]: write the positions below
  int32_t *pos, *row_seq, *row_len;  // [T]
  int s;                  // tokens per sequence
  const float *xw_norm;   // optional [H]: also write xw [T, H] = bf16(row * xw_norm)
  uint16_t *xw;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_dec_embed(EmbedArgs a) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  if (a.lens && threadIdx.x == 0) {
    const int bi = (int)(t / a.s);
    const int p = a.lens[bi] + (int)(t - (int64_t)bi * a.s);
    a.pos[t] = p;
    a.row_seq[t] = bi;
    a.row_len[t] = p + 1;
  }
  int64_t id = a.ids[t];
  id = id < 0 ? 0 : (id > a.V - 1 ? a.V - 1 : id);
  float ss = embed_row(a.table + id * a.H, a.h + t * a.H, a.H, threadIdx.x, a.xw_norm,
                       a.xw ? a.xw + t * a.H : nullptr);
  if (a.ss) {
    ss = block_sum_256(ss, red);
    if (threadIdx.x == 0) a.ss[t] = ss;
  }
}

// ---- residual rows from the caller: h[t] = h_in[t] -----------------------------
// The input of a layer run by the teacher-forcing entry point
// (rxw8_decoder_forward_layers): writes what rxw8_dec_embed writes for a row
// -- the positions, the f32 row, its sum of squares and the first layer's
// weighted bf16 row -- from an f32 row instead of an embedding row. One
// workgroup of 256 threads per row, thread t taking elements t, t + 256, ...
struct LoadRowsArgs {
  const float *h_in;      // [T, H]
  float *h;               // [T, H]
  float *ss;              // optional [T]
  int64_t H;
  const int32_t *lens;    // [B]
  int32_t *pos, *row_seq, *row_len;  // [T]
  int s;
  const float *xw_norm;   // optional [H]: also write xw [T, H] = bf16(row * xw_norm)
  uint16_t *xw;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_dec_load_rows(LoadRowsArgs a) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  if (threadIdx.x == 0) {
    const int bi = (int)(t / a.s);
    const int p = a.lens[bi] + (int)(t - (int64_t)bi * a.s);
    a.pos[t] = p;
    a.row_seq[t] = bi;
    a.row_len[t] = p + 1;
  }
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < a.H; i += 256) {
    const float v = a.h_in[t * a.H + i];
    a.h[t * a.H + i] = v;
    if (a.xw) a.xw[t * a.H + i] = f32_to_bf16_bits(v * a.xw_norm[i]);
    ss += v * v;
  }
  if (a.ss) {
    ss = block_sum_256(ss, red);
    if (threadIdx.x == 0) a.ss[t] = ss;
  }
}

// Row permutation of the fused gate|up projection used by the SwiGLU GEMV
// epilogue: output row R takes input row (R % 16 < 8 ? 8 (R / 16) + R % 16
// : half + 8 (R / 16) + R % 16 - 8), i.e. 16-row tiles of 8 gate rows then the
// 8 matching up rows. Applied to the f32 scales [2 half, cols] here; the
// weights get it inside rxw8_pack_tiles.
struct InterleaveArgs {
  const float *src;
  float *dst;
  int64_t half, cols;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_dec_interleave_rows(InterleaveArgs a) {
  const int64_t total = 2 * a.half * a.cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t R = e / a.cols, c = e - R * a.cols;
    const int64_t t = R / 16, r = R % 16;
    const int64_t src_row = r < 8 ? 8 * t + r : a.half + 8 * t + r - 8;
    a.dst[e] = a.src[src_row * a.cols + c];
  }
}

// ---- RMSNorm (ops.rs:929-944): y = bf16((x * rsqrt(mean(x^2) + eps)) * w) -------
// One workgroup per output row; src_rows (optional) picks the input row.
struct RmsNormArgs {
  const float *x;          // [rows_in, H]
  const float *w;          // [H]
  uint16_t *y;             // [rows, H] bf16
  const int32_t *src_row;  // optional: input row of output row r
  int64_t H;
  int rows;
  int src_stride, src_offset;  // without src_row: input row = r * stride + offset
  float eps;
};

// Thread t sums elements t, t + 256, ... in that order, then block_sum_256
// (the fused GEMV's x_mode 1 prologue repeats this order). Rows of up to
// 16 x 256 elements are read once: all of a thread's x and weight loads are
// issued before any is used, and the write reuses them.
extern "C" __global__ void __launch_bounds__(256) rxw8_dec_rmsnorm(RmsNormArgs a) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const int64_t src = a.src_row ? a.src_row[r] : (int64_t)r * a.src_stride + a.src_offset;
  const float *x = a.x + src * a.H;
  uint16_t *y = a.y + (int64_t)r * a.H;
  const int t = threadIdx.x;
  constexpr int R = 16;
  if (a.H <= 256 * R) {
    float v[R], w[R];
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const int64_t i = t + 256 * s;
      v[s] = i < a.H ? x[i] : 0.f;
      w[s] = i < a.H ? a.w[i] : 0.f;
    }
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < R; ++s) ss += v[s] * v[s];  // zeros past H add nothing
    ss = block_sum_256(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)a.H + a.eps);
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const int64_t i = t + 256 * s;
      if (i < a.H) y[i] = f32_to_bf16_bits((v[s] * scale) * w[s]);
    }
    return;
  }
  float ss = 0.f;
  for (int64_t i = t; i < a.H; i += blockDim.x) ss += x[i] * x[i];
  ss = block_sum_256(ss, red);
  const float scale = 1.0f / sqrtf(ss / (float)a.H + a.eps);
  for (int64_t i = t; i < a.H; i += blockDim.x)
    y[i] = f32_to_bf16_bits((x[i] * scale) * a.w[i]);
}

// ---- q/k RMSNorm + RoPE + KV append (qwen3_5/layers.rs:28-101; rotary.rs:17-74;
// kv_cache.rs:53-68 at start [seq, head, pos, 0]).
// qkv [T, (Hq + 2 Hkv) * D] bf16 (the bf16 result of the fused projection).
// One wave per head: lane l owns the SplitHalf pairs (i, i + D/2), i = l + 64 j.
// ---- RoPE table: row p = cos(p f_i) for i < D/2, then sin(p f_i), with
// f_i = theta^(-2i/D) in f32 and the angle p * f_i rounded to f32
// (rotary.rs:17-74 with qwen3_5/mod.rs:211-228). Built once per decoder; the
// RoPE kernels read it instead of evaluating sin/cos per token.
struct RopeTableArgs {
  const float *freqs;  // [D/2]
  float *tab;          // [Lmax, D]
  int half;
};

extern "C" __global__ void __launch_bounds__(64) rxw8_dec_rope_table(RopeTableArgs a) {
  const int p = blockIdx.x;
  float *row = a.tab + (int64_t)p * 2 * a.half;
  for (int i = threadIdx.x; i < a.half; i += blockDim.x) {
    float sn, cs;
    sincosf((float)p * a.freqs[i], &sn, &cs);
    row[i] = cs;
    row[a.half + i] = sn;
  }
}

struct QkRopeArgs {
  const uint16_t *qkv;
  const float *q_norm;  // [D] or null
  const float *k_norm;  // [D] or null
  const float *rope;    // [Lmax, D] RoPE table (rxw8_dec_rope_table)
  const int32_t *pos;   // [T]
  const int32_t *row_seq;
  float *q_out;         // [T, Hq, D] f32
  uint16_t *kc;         // [Bc, Hkv, Lmax, D] bf16 (this layer)
  uint16_t *vc;
  int T, Hq, Hkv, D, Lmax;
  float eps;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_dec_qk_rope_kv(QkRopeArgs a) {
  const int lane = threadIdx.x & 63;
  const int heads = a.Hq + 2 * a.Hkv;
  const int gw = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);  // global wave
  const int t = gw / heads, h = gw - t * heads;
  if (t >= a.T) return;
  const int D = a.D, half = D / 2;
  const uint16_t *src = a.qkv + ((int64_t)t * heads + h) * D;
  const int seq = a.row_seq[t];
  const int p = a.pos[t];
  if (h >= a.Hq + a.Hkv) {  // value head: copy the bf16 projection into the cache
    const int kvh = h - a.Hq - a.Hkv;
    uint16_t *dst = a.vc + (((int64_t)seq * a.Hkv + kvh) * a.Lmax + p) * D;
    for (int i = lane; i < D; i += 64) dst[i] = src[i];
    return;
  }
  const bool is_q = h < a.Hq;
  const float *nw = is_q ? a.q_norm : a.k_norm;
  float ss = 0.f;
  for (int i = lane; i < D; i += 64) {
    const float v = bf16_bits_to_f32(src[i]);
    ss += v * v;
  }
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float scale = nw ? 1.0f / sqrtf(ss / (float)D + a.eps) : 1.0f;
  const float *rope = a.rope + (int64_t)p * D;
  for (int i = lane; i < half; i += 64) {
    float x0 = bf16_bits_to_f32(src[i]), x1 = bf16_bits_to_f32(src[i + half]);
    if (nw) {
      x0 = (x0 * scale) * nw[i];
      x1 = (x1 * scale) * nw[i + half];
    }
    const float cs = rope[i], sn = rope[half + i];
    const float r0 = x0 * cs - x1 * sn;
    const float r1 = x1 * cs + x0 * sn;
    if (is_q) {
      float *dst = a.q_out + ((int64_t)t * a.Hq + h) * D;
      dst[i] = r0;
      dst[i + half] = r1;
    } else {
      const int kvh = h - a.Hq;
      uint16_t *dst = a.kc + (((int64_t)seq * a.Hkv + kvh) * a.Lmax + p) * D;
      dst[i] = f32_to_bf16_bits(r0);
      dst[i + half] = f32_to_bf16_bits(r1);
    }
  }
}

// The same for D = 128 with 8 lanes per (token, head) row: lane j handles
// dims 8j .. 8j+7 and their RoPE partners 64 + 8j .. (16-byte loads and
// stores); the row's sum of squares is reduced over its 8 lanes.
extern "C" __global__ void __launch_bounds__(256) rxw8_dec_qk_rope_kv_d128(QkRopeArgs a) {
  constexpr int D = 128, HALF = 64;
  const int heads = a.Hq + 2 * a.Hkv;
  const int64_t unit = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 3;
  const int j = threadIdx.x & 7;
  const bool live = unit < (int64_t)a.T * heads;  // lanes past the end still join the shuffles
  const int64_t u = live ? unit : 0;
  const int t = (int)(u / heads), h = (int)(u - (int64_t)t * heads);
  const uint16_t *src = a.qkv + ((int64_t)t * heads + h) * D;
  const int seq = a.row_seq[t];
  const int p = a.pos[t];
  const int i0 = 8 * j;
  const u32x4 lo = *(const u32x4 *)(src + i0), hi = *(const u32x4 *)(src + HALF + i0);
  if (h >= a.Hq + a.Hkv) {  // value head (uniform over the 8 lanes)
    if (live) {
      uint16_t *dst = a.vc + (((int64_t)seq * a.Hkv + (h - a.Hq - a.Hkv)) * a.Lmax + p) * D;
      *(u32x4 *)(dst + i0) = lo;
      *(u32x4 *)(dst + HALF + i0) = hi;
    }
    return;
  }
  float x0[8], x1[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x0[2 * e] = bf16_bits_to_f32(lo[e] & 0xffffu);
    x0[2 * e + 1] = bf16_bits_to_f32(lo[e] >> 16);
    x1[2 * e] = bf16_bits_to_f32(hi[e] & 0xffffu);
    x1[2 * e + 1] = bf16_bits_to_f32(hi[e] >> 16);
  }
  const bool is_q = h < a.Hq;
  const float *nw = is_q ? a.q_norm : a.k_norm;
  // norm weights and the position's RoPE row, 16-byte loads issued before
  // the reduction that precedes their use
  const float *rope = a.rope + (int64_t)p * D;
  float w0[8], w1[8], cs[8], sn[8];
#pragma unroll
  for (int c = 0; c < 8; c += 4) {
    const float4 a4 = *(const float4 *)(rope + i0 + c), b4 = *(const float4 *)(rope + HALF + i0 + c);
    cs[c] = a4.x, cs[c + 1] = a4.y, cs[c + 2] = a4.z, cs[c + 3] = a4.w;
    sn[c] = b4.x, sn[c + 1] = b4.y, sn[c + 2] = b4.z, sn[c + 3] = b4.w;
    if (nw) {
      const float4 c4 = *(const float4 *)(nw + i0 + c), d4 = *(const float4 *)(nw + HALF + i0 + c);
      w0[c] = c4.x, w0[c + 1] = c4.y, w0[c + 2] = c4.z, w0[c + 3] = c4.w;
      w1[c] = d4.x, w1[c + 1] = d4.y, w1[c + 2] = d4.z, w1[c + 3] = d4.w;
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x0[e] * x0[e] + x1[e] * x1[e];
  ss += __shfl_xor(ss, 1);
  ss += __shfl_xor(ss, 2);
  ss += __shfl_xor(ss, 4);
  if (nw) {
    const float sc = 1.0f / sqrtf(ss / (float)D + a.eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x0[e] = (x0[e] * sc) * w0[e];
      x1[e] = (x1[e] * sc) * w1[e];
    }
  }
  float r0[8], r1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    r0[e] = x0[e] * cs[e] - x1[e] * sn[e];
    r1[e] = x1[e] * cs[e] + x0[e] * sn[e];
  }
  if (!live) return;
  if (is_q) {
    float *dst = a.q_out + ((int64_t)t * a.Hq + h) * D;
    *(f32x4 *)(dst + i0) = f32x4{r0[0], r0[1], r0[2], r0[3]};
    *(f32x4 *)(dst + i0 + 4) = f32x4{r0[4], r0[5], r0[6], r0[7]};
    *(f32x4 *)(dst + HALF + i0) = f32x4{r1[0], r1[1], r1[2], r1[3]};
    *(f32x4 *)(dst + HALF + i0 + 4) = f32x4{r1[4], r1[5], r1[6], r1[7]};
  } else {
    uint16_t *dst = a.kc + (((int64_t)seq * a.Hkv + (h - a.Hq)) * a.Lmax + p) * D;
    *(u32x4 *)(dst + i0) = u32x4{pack_bf16x2(r0[0], r0[1]), pack_bf16x2(r0[2], r0[3]),
                                 pack_bf16x2(r0[4], r0[5]), pack_bf16x2(r0[6], r0[7])};
    *(u32x4 *)(dst + HALF + i0) = u32x4{pack_bf16x2(r1[0], r1[1]), pack_bf16x2(r1[2], r1[3]),
                                        pack_bf16x2(r1[4], r1[5]), pack_bf16x2(r1[6], r1[7])};
  }
}

// ---- SwiGLU middle (ops.rs:331-342): act = bf16(silu(g) * u), gu = [g | u] ----
struct SiluMulArgs {
  const uint16_t *gu;  // [T, 2I]: gate columns then up columns, or interleaved
  uint16_t *act;       // [T, I]
  int64_t T, I;
  int interleaved;     // 1: columns in blocks of 8 gate + 8 up (rxw8_dec_interleave_rows order)
};

extern "C" __global__ void __launch_bounds__(256) rxw8_dec_silu_mul(SiluMulArgs a) {
  const int64_t total = a.T * a.I;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = e / a.I, i = e - t * a.I;
    const int64_t gc = a.interleaved ? 16 * (i / 8) + i % 8 : i;
    const int64_t uc = a.interleaved ? gc + 8 : a.I + i;
    const float g = bf16_bits_to_f32(a.gu[t * 2 * a.I + gc]);
    const float u = bf16_bits_to_f32(a.gu[t * 2 * a.I + uc]);
    a.act[e] = f32_to_bf16_bits(silu_mul_f32(g, u));
  }
}

// ---- argmax (indexing.rs:350-374): lowest index of the maximum; a NaN beats
// every number and the first NaN wins. Pass 1: per-chunk partials; pass 2:
// chunks in order.
struct ArgmaxArgs {
  const float *x;   // [outer, cols, inner]; row r = (r / inner, :, r % inner)
  float *pval;      // [rows, chunks]
  int32_t *pidx;
  int32_t *out;     // [rows]
  int64_t cols;
  int rows, chunks;
  int64_t inner;    // stride of the reduced axis (1: rows are contiguous)
};

__device__ __forceinline__ bool am_better(float a, int ia, float b, int ib) {
  // is (a, ia) preferred over (b, ib)?
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}

// (value, index) pair of a wave with the lowest index on ties (am_better is a
// total order, so any reduction order returns the same winner); index
// 0x7fffffff marks "no element".
__device__ __forceinline__ void am_wave_reduce(float &bv, int &bi) {
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (oi != 0x7fffffff && (bi == 0x7fffffff || am_better(ov, oi, bv, bi))) {
      bv = ov;
      bi = oi;
    }
  }
}

extern "C" __global__ void __launch_bounds__(256) rxw8_dec_argmax_partial(ArgmaxArgs a) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int r = blockIdx.x / a.chunks, c = blockIdx.x - r * a.chunks;
  if (a.inner == 1 && (a.cols & 3) == 0 && ((uintptr_t)a.x & 15) == 0) {
    // contiguous rows of whole float4s: chunks of whole float4s, each
    // thread's loads issued together, wave butterflies, then the 4 waves
    const int64_t q4 = a.cols >> 2, per4 = (q4 + a.chunks - 1) / a.chunks;
    const int64_t lo4 = c * per4, hi4 = min(q4, lo4 + per4);
    const float4 *xr = (const float4 *)(a.x + (int64_t)r * a.cols);
    float bv = -__builtin_huge_valf();
    int bi = 0x7fffffff;
    for (int64_t q0 = lo4 + threadIdx.x; q0 < hi4; q0 += 4 * 256) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (q0 + 256 * u < hi4) v[u] = xr[q0 + 256 * u];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t q = q0 + 256 * u;
        if (q < hi4) {
          const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int i = (int)(4 * q + k);
            if (bi == 0x7fffffff || am_better(e[k], i, bv, bi)) {
              bv = e[k];
              bi = i;
            }
          }
        }
      }
    }
    am_wave_reduce(bv, bi);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
      sv[wave] = bv;
      si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < 4; ++w)
        if (si[w] != 0x7fffffff && (bi == 0x7fffffff || am_better(sv[w], si[w], bv, bi))) {
          bv = sv[w];
          bi = si[w];
        }
      a.pval[blockIdx.x] = bv;
      a.pidx[blockIdx.x] = bi;
    }
    return;
  }
  const int64_t per = (a.cols + a.chunks - 1) / a.chunks;
  const int64_t lo = c * per, hi = min(a.cols, lo + per);
  const int64_t o = r / a.inner, j = r - o * a.inner;
  const float *xr = a.x + o * a.cols * a.inner + j;
  float bv = -__builtin_huge_valf();
  int bi = (int)(lo < hi ? lo : 0);
  bool have = false;
  for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) {
    const float v = xr[i * a.inner];
    if (!have || am_better(v, (int)i, bv, bi)) {
      bv = v;
      bi = (int)i;
      have = true;
    }
  }
  sv[threadIdx.x] = have ? bv : -__builtin_huge_valf();
  si[threadIdx.x] = have ? bi : 0x7fffffff;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (threadIdx.x < st) {
      const float ov = sv[threadIdx.x + st];
      const int oi = si[threadIdx.x + st];
      if (oi != 0x7fffffff &&
          (si[threadIdx.x] == 0x7fffffff || am_better(ov, oi, sv[threadIdx.x], si[threadIdx.x]))) {
        sv[threadIdx.x] = ov;
        si[threadIdx.x] = oi;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    a.pval[blockIdx.x] = sv[0];
    a.pidx[blockIdx.x] = si[0];
  }
}

// Pass 2 plus the end of a forward step, in one launch: one wave per row
// reduces the row's chunk partials (lane c holds chunk c; (value, index) under
// am_better is a total order, so the butterfly returns the same winner as a
// sequential scan), writes next[r] and advances lens[r] by s; with `rec_out`
// (generate) it also stores next[r] in column *step of rec_out and then
// advances *step. With `table` (generate) it then does the work of the next
// single-token step's rxw8_dec_embed: row r of h = f32(E[next[r]]) with its
// sum of squares (each 256-thread slice of the workgroup takes one row through
// embed_row, as that kernel does, so the bits agree) and the positions
// pos[r] = lens[r], row_seq[r] = r, row_len[r] = lens[r] + 1. One workgroup
// of 64 * min(rows, 16) threads, or 1024 with `table`.
struct ArgmaxFinalArgs {
  const float *pval;  // [rows, chunks]
  const int32_t *pidx;
  int32_t *next;      // [rows]
  int32_t *lens;      // optional [rows] advanced by s
  int32_t *rec_out;   // optional [rows, ncols]
  int32_t *rec_step;  // device column counter (with rec_out)
  int rows, chunks, s, ncols;
  const uint16_t *table;  // optional [V, H] bf16 embedding (needs lens)
  float *h;               // [rows, H]
  float *ss;              // optional [rows]
  int32_t *pos, *row_seq, *row_len;  // [rows]
  int64_t V, H;
  const float *xw_norm;   // optional [H]: also write xw [rows, H] = bf16(row * xw_norm)
  uint16_t *xw;
};

extern "C" __global__ void __launch_bounds__(1024) rxw8_dec_argmax_final(ArgmaxFinalArgs a) {
  __shared__ int col;
  __shared__ int ids[256];  // the winners of rows < 256 for the embedding pass
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  if (threadIdx.x == 0) col = a.rec_out ? *a.rec_step : 0;
  __syncthreads();
  for (int r = wave; r < a.rows; r += nwaves) {
    float bv = -__builtin_huge_valf();
    int bi = 0x7fffffff;
    if (lane < a.chunks) {  // both loads in flight (the value is unused for an empty chunk)
      bi = a.pidx[r * a.chunks + lane];
      bv = a.pval[r * a.chunks + lane];
    }
    am_wave_reduce(bv, bi);
    if (lane == 0) {
      const int id = bi == 0x7fffffff ? 0 : bi;
      if (r < 256) ids[r] = id;
      a.next[r] = id;
      if (a.lens) a.lens[r] += a.s;
      if (a.rec_out && col < a.ncols) a.rec_out[r * a.ncols + col] = id;
    }
  }
  __syncthreads();
  if (a.rec_out && threadIdx.x == 0) *a.rec_step = col + 1;
  if (!a.table) return;
  __shared__ float red[16];
  const int groups = blockDim.x >> 8, g = threadIdx.x >> 8, t = threadIdx.x & 255;
  for (int r0 = 0; r0 < a.rows; r0 += groups) {  // uniform trip count (barriers inside)
    const int r = r0 + g;
    float ss = 0.f;
    if (r < a.rows) {
      int64_t id = r < 256 ? ids[r] : a.next[r];
      id = id < 0 ? 0 : (id > a.V - 1 ? a.V - 1 : id);
      ss = embed_row(a.table + id * a.H, a.h + (int64_t)r * a.H, a.H, t, a.xw_norm,
                     a.xw ? a.xw + (int64_t)r * a.H : nullptr);
      if (t == 0) {
        const int p = a.lens[r];
        a.pos[r] = p;
        a.row_seq[r] = r;
        a.row_len[r] = p + 1;
      }
    }
    // block_sum_256 of the slice: wave butterfly, then its 4 wave sums in order
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    __syncthreads();
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    if (a.ss && r < a.rows && t == 0)
      a.ss[r] = (red[4 * g] + red[4 * g + 1]) + (red[4 * g + 2] + red[4 * g + 3]);
  }
}

