// Kernels of the hybrid Qwen3.5 W8 text model
// (crates/rxla-models/src/qwen3_5/mod.rs:158-273, layers.rs:4-293): the W8
// embedding, zero-centred / gated RMSNorm, the full-attention prologue (gate,
// q/k norm, partial RoPE), the gated-delta pieces (causal depthwise conv +
// SiLU, L2 norms, beta / decay, the delta-rule recurrence) and SwiGLU. The
// projections run on the shared W8A16 GEMM/GEMV paths; the full-sequence
// attention on the shared GQA kernels. Token t = b * S + i sits at position i
// of sequence b (the reference runs whole sequences from position 0).
#include "common.h"

namespace {
__device__ __forceinline__ float sigmoid_f32(float x) {  // rxla-core ops.rs:330-338
  const float e = __expf(-fabsf(x));
  return x >= 0.f ? 1.0f / (1.0f + e) : e / (1.0f + e);
}
__device__ __forceinline__ float ld(const void *p, int64_t i, int f32) {
  return f32 ? ((const float *)p)[i] : bf16_bits_to_f32(((const uint16_t *)p)[i]);
}
}  // namespace

// One DPP move within a row of 16 lanes (CTRL: row_ror:n = 0x120 + n, or a
// quad_perm pattern).
template <int CTRL>
__device__ __forceinline__ float dpp_rot(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// ---- W8 embedding: h[t, c] = (f32(u8[id, c]) - 128) * scale[id, c / G], ids
// clamped to [0, V - 1] (mod.rs:134-157, indexing.rs:637-656); one workgroup
// per token, which also writes the row's sum of squares (ss, optional) for the
// RMSNorm prologue of the first projection.
struct Q35EmbedArgs {
  const int32_t *ids;
  const uint8_t *w;     // [V, H]
  const float *scale;   // [V, H / G]
  float *h;             // [T, H]
  float *ss;            // [T] or null
  int64_t T, V, H, G;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_q35_embed(Q35EmbedArgs a) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  int64_t id = a.ids[t];
  id = id < 0 ? 0 : (id > a.V - 1 ? a.V - 1 : id);
  float ss = 0.f;
  for (int64_t c = threadIdx.x; c < a.H; c += blockDim.x) {
    const float v = ((float)a.w[id * a.H + c] + -128.0f) * a.scale[id * (a.H / a.G) + c / a.G];
    a.h[t * a.H + c] = v;
    ss += v * v;
  }
  ss = block_sum_256(ss, red);
  if (a.ss && threadIdx.x == 0) a.ss[t] = ss;
}

// ---- RMSNorm over rows of L values (rxla-nn layers.rs:459-495):
//   y = x * rsqrt(mean(x^2) + eps) * (zero_centered ? 1 + w : w)
// optionally times silu(z) (the gated output norm, layers.rs:241-259).
// Row r reads x + r * x_stride, writes out + r * out_stride (bf16 or f32);
// its gate row is z + (r / z_group) * z_stride + (r % z_group) * L.
struct Q35NormArgs {
  const float *x;
  const float *w;        // [L]
  const void *z;         // gate rows (bf16 or f32) or null
  void *out;
  int64_t rows, L, x_stride, out_stride, z_stride, z_group;
  float eps;
  int zero_centered, out_f32, z_f32;
  // non-null: instead of out, the F32 GEMM's operand split of each result y,
  // hi = bf16(y) and lo = bf16(y - hi) at the same index (rxw8_gemm_split_x's
  // arithmetic, so the GEMM sees the bits the split launch would give it)
  uint16_t *hi, *lo;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_q35_rmsnorm(Q35NormArgs a) {
  __shared__ float red[8];
  const int64_t r = blockIdx.x;
  if (r >= a.rows) return;
  const float *x = a.x + r * a.x_stride;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < a.L; i += blockDim.x) ss += x[i] * x[i];
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) tot += red[i];
  const float sc = 1.0f / sqrtf(tot / (float)a.L + a.eps);
  // four elements' loads per thread go out before their stores (a load after
  // a store the compiler cannot tell apart from it would wait for it)
  const int64_t zrow = (r / a.z_group) * a.z_stride + (r % a.z_group) * a.L;
  for (int64_t i0 = threadIdx.x; i0 < a.L; i0 += 4 * (int64_t)blockDim.x) {
    float xv[4], wv[4], zv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t i = i0 + e * (int64_t)blockDim.x;
      const bool in = i < a.L;
      xv[e] = in ? x[i] : 0.f;
      wv[e] = in ? a.w[i] : 0.f;
      zv[e] = in && a.z ? ld(a.z, zrow + i, a.z_f32) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t i = i0 + e * (int64_t)blockDim.x;
      if (i >= a.L) continue;
      float y = (xv[e] * sc) * (a.zero_centered ? 1.0f + wv[e] : wv[e]);
      if (a.z) y *= zv[e] * sigmoid_f32(zv[e]);
      if (a.hi) {
        const uint16_t h = f32_to_bf16_bits(y);
        a.hi[r * a.out_stride + i] = h;
        a.lo[r * a.out_stride + i] = f32_to_bf16_bits(y - bf16_bits_to_f32(h));
      } else if (a.out_f32) {
        ((float *)a.out)[r * a.out_stride + i] = y;
      } else {
        ((uint16_t *)a.out)[r * a.out_stride + i] = f32_to_bf16_bits(y);
      }
    }
  }
}

// The same norm with one wave per row (rows of L <= 64 E values, 4 rows per
// workgroup): lane l holds elements l + 64 e. Every load of the row (x, the
// weight, the gate) is a raw buffer load issued before any arithmetic (lanes
// past L read zeros without touching memory), the sum of squares is a wave
// butterfly (no barrier), so a row costs one memory round trip; the
// 256-thread kernel above waits for x, a barrier, then w and z. (The sum is
// taken in another order than there: per lane, then across the wave.)
template <int E>
__device__ __forceinline__ void q35_rmsnorm_wave(const Q35NormArgs &a) {
  const int lane = threadIdx.x & 63;
  // (the row as a wave-uniform value, so the buffer descriptors sit in
  // scalar registers: from a plain thread index the compiler wraps each
  // buffer load in a loop over the lanes' descriptors)
  const int64_t r = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (r >= a.rows) return;  // uniform per wave
  const uint32_t L = (uint32_t)a.L;
  const auto xr = buf_rsrc(a.x + r * a.x_stride, L * 4u);
  const auto wr = buf_rsrc(a.w, L * 4u);
  const int64_t zrow = (r / a.z_group) * a.z_stride + (r % a.z_group) * a.L;
  const int zsz = a.z_f32 ? 4 : 2;
  const auto zr = buf_rsrc(a.z ? (const char *)a.z + zrow * zsz : (const char *)a.x, a.z ? L * zsz : 0u);
  float xv[E], wv[E], zv[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t i = lane + 64 * e;
    xv[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, i * 4u, 0, 0));
    wv[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(wr, i * 4u, 0, 0));
    zv[e] = a.z_f32 ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(zr, i * 4u, 0, 0))
                    : bf16_bits_to_f32(__builtin_amdgcn_raw_buffer_load_b16(zr, i * 2u, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);  // (all of them issued before the first use)
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss += xv[e] * xv[e];
  ss = wave_sum64(ss);
  const float sc = 1.0f / sqrtf(ss / (float)a.L + a.eps);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int64_t i = lane + 64 * e;
    if (i >= a.L) continue;
    float y = (xv[e] * sc) * (a.zero_centered ? 1.0f + wv[e] : wv[e]);
    if (a.z) y *= zv[e] * sigmoid_f32(zv[e]);
    if (a.hi) {
      const uint16_t h = f32_to_bf16_bits(y);
      a.hi[r * a.out_stride + i] = h;
      a.lo[r * a.out_stride + i] = f32_to_bf16_bits(y - bf16_bits_to_f32(h));
    } else if (a.out_f32) {
      ((float *)a.out)[r * a.out_stride + i] = y;
    } else {
      ((uint16_t *)a.out)[r * a.out_stride + i] = f32_to_bf16_bits(y);
    }
  }
}
#define RXW8_Q35_NORM_W(E)                                                      \
  extern "C" __global__ void __launch_bounds__(256) rxw8_q35_rmsnorm_w##E(Q35NormArgs a) { \
    q35_rmsnorm_wave<E>(a);                                                     \
  }
RXW8_Q35_NORM_W(1)
RXW8_Q35_NORM_W(2)
RXW8_Q35_NORM_W(4)
RXW8_Q35_NORM_W(8)
RXW8_Q35_NORM_W(16)

// ---- full attention prologue (layers.rs:28-99): one wave per (token, head).
// Query heads h < Hq: qg[t, h] = [query (D) | gate (D)] (bf16 projection);
// gate_out[t, h*D + d] = sigmoid(gate); q_out[t, h, :] = RoPE(norm(query)).
// KV heads: k = RoPE(norm(k)), v copied; both into f32 [B, Hkv, Lmax, D] at
// the token's position. norm: zero-centred RMSNorm over D; RoPE: split-half
// over the first rot channels with angle pos * freqs[i] (mod.rs:209-229).
struct Q35FaPrepArgs {
  const void *qg;        // [T, Hq * 2D] rows of `stride` elements
  const void *kp;        // [T, Hkv * D] rows of `stride` elements
  const void *vp;        // [T, Hkv * D] rows of `stride` elements
  const float *q_norm, *k_norm;  // [D]
  const float *freqs;    // [rot / 2]
  float *q_out;          // [T, Hq, D]
  float *gate_out;       // [T, Hq * D]
  float *kc, *vc;        // [B, Hkv, Lmax, D]
  int T, S, Hq, Hkv, D, rot, Lmax, stride;
  float eps;
  int src_f32;           // projection rows in f32 (F32 compute) or bf16
};

template <bool F32>
__device__ __forceinline__ void q35_fa_prep(const Q35FaPrepArgs &a) {
  __shared__ float rowbuf[4][256 + 8];
  // (wv wave-uniform: the buffer descriptors below then sit in scalar registers)
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int heads = a.Hq + a.Hkv;
  const int64_t unit = (int64_t)blockIdx.x * 4 + wv;
  if (unit >= (int64_t)a.T * heads) return;  // wave-uniform
  const int t = (int)(unit / heads), h = (int)(unit - (int64_t)t * heads);
  const int bseq = t / a.S, pos = t - bseq * a.S;
  const int D = a.D;
  const bool is_q = h < a.Hq;
  const int64_t src = is_q ? (int64_t)t * a.stride + (int64_t)h * 2 * D
                            : (int64_t)t * a.stride + (int64_t)(h - a.Hq) * D;
  const void *sbase = is_q ? a.qg : a.kp;
  float *row = rowbuf[wv];
  // Every load of the unit goes out at once, as raw buffer loads (lanes past
  // D or rot read zeros, no branch): the row, its norm weight, the RoPE
  // frequencies and the gate / v row. (Loaded in that order of need, they
  // cost three memory round trips.)
  constexpr int NE = 4;  // D <= 256
  const int half = a.rot / 2;
  constexpr int esz = F32 ? 4 : 2;
  const int64_t gsrc = is_q ? src + D : (int64_t)t * a.stride + (int64_t)(h - a.Hq) * D;
  const auto rr = buf_rsrc((const char *)sbase + src * esz, (uint32_t)(D * esz));
  const auto gr = buf_rsrc((const char *)(is_q ? a.qg : a.vp) + gsrc * esz, (uint32_t)(D * esz));
  const auto nr = buf_rsrc(is_q ? a.q_norm : a.k_norm, (uint32_t)D * 4u);
  const auto fq = buf_rsrc(a.freqs, (uint32_t)half * 4u);
  auto ldb = [&](const __amdgpu_buffer_rsrc_t &r, int i) {
    if constexpr (F32)
      return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (uint32_t)i * 4u, 0, 0));
    else
      return bf16_bits_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, (uint32_t)i * 2u, 0, 0));
  };
  float xv[NE], nv[NE], fr[NE], gq[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const int i = lane + 64 * e;
    xv[e] = ldb(rr, i);
    gq[e] = ldb(gr, i);
    nv[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(nr, (uint32_t)i * 4u, 0, 0));
    const uint32_t fo = i < a.rot ? (uint32_t)(i < half ? i : i - half) * 4u : 0x80000000u;
    fr[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(fq, fo, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);  // (all of them issued before the first use)
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < NE; ++e) ss += xv[e] * xv[e];
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float sc = 1.0f / sqrtf(ss / (float)D + a.eps);
#pragma unroll
  for (int e = 0; e < NE; ++e)
    if (lane + 64 * e < D) row[lane + 64 * e] = (xv[e] * sc) * (1.0f + nv[e]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float *dst = is_q ? a.q_out + ((int64_t)t * a.Hq + h) * D
                    : a.kc + (((int64_t)bseq * a.Hkv + (h - a.Hq)) * a.Lmax + pos) * D;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const int i = lane + 64 * e;
    if (i >= D) continue;
    float y = row[i];
    if (i < a.rot) {
      float sn, cs;
      sincosf((float)pos * fr[e], &sn, &cs);
      y = i < half ? row[i] * cs - row[i + half] * sn : row[i] * cs + row[i - half] * sn;
    }
    dst[i] = y;
  }
  if (is_q) {
    float *go = a.gate_out + (int64_t)t * a.Hq * D + (int64_t)h * D;
#pragma unroll
    for (int e = 0; e < NE; ++e)
      if (lane + 64 * e < D) go[lane + 64 * e] = sigmoid_f32(gq[e]);
  } else {
    float *vd = a.vc + (((int64_t)bseq * a.Hkv + (h - a.Hq)) * a.Lmax + pos) * D;
#pragma unroll
    for (int e = 0; e < NE; ++e)
      if (lane + 64 * e < D) vd[lane + 64 * e] = gq[e];
  }
}
// (one straight-line body per source dtype)
extern "C" __global__ void __launch_bounds__(256) rxw8_q35_fa_prep(Q35FaPrepArgs a) {
  if (a.src_f32)
    q35_fa_prep<true>(a);
  else
    q35_fa_prep<false>(a);
}

// ---- causal full-sequence attention in f32 on the matrix cores
// (layers.rs:78-92: softmax(q k^T * scale + causal mask) v over positions
// 0..S-1 of each sequence, GQA head h reading kv head h / G). q, k and v are
// f32 (v holds bf16 values); v_mfma_f32_16x16x4_f32 multiplies f32 operands
// and accumulates in f32, and the softmax is the online (flash) form in f32.
//
// Workgroup: 4 waves for one (sequence, kv head, query tile); wave w takes
// query head kv * G + w % G and the 16 queries of sub-tile w / G (4 / G
// sub-tiles, G in {1, 2, 4}), keeping its q rows (16 x D) and its output rows
// in registers. Keys go in tiles of 16 through LDS (K and V, f32, rows padded
// by 4 floats), double-buffered: the next tile's global loads are in flight
// while the current one is used. Per tile a wave forms S = q k^T (D / 4
// MFMAs; lane l holds q[l % 16][D/4 * (l / 16) + c] and k[l % 16][same]),
// masks and rescales with the row max / sum over the 16 lanes of a DPP row,
// stores P (16 x 16) to its own LDS slice and accumulates O += P V (4 MFMAs
// per 16 output columns; key 4 (l / 16) + c of the tile for lane l).
struct Q35AttnArgs {
  const float *q;        // [T, Hq, D], token t = b * S + i
  const float *kc, *vc;  // [B, Hkv, Lmax, D]
  const float *gate;     // [T, Hq * D] output gate (layers.rs:93-94), multiplied in at the store
  float *out;            // [T, Hq * D]
  // nsplit > 1: each (sequence, kv head, query tile) is split into nsplit
  // ranges of key tiles; every range writes its unnormalised rows
  // [m, l, o[D]] to part[((t * Hq + h) * nsplit + split)] and
  // rxw8_q35_attention_combine merges them (and applies the gate)
  float *part;
  int B, S, Hq, Hkv, Lmax, qtiles, nsplit;
  float scale;
};

__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_rot<0x128>(v));
  v = fmaxf(v, dpp_rot<0x124>(v));
  v = fmaxf(v, dpp_rot<0x4e>(v));
  return fmaxf(v, dpp_rot<0xb1>(v));
}
__device__ __forceinline__ float row_add16(float v) {
  v += dpp_rot<0x128>(v);
  v += dpp_rot<0x124>(v);
  v += dpp_rot<0x4e>(v);
  return v + dpp_rot<0xb1>(v);
}

// global -> LDS DMA of 16 bytes per active lane (global_load_lds_dwordx4:
// lane l writes LDS bytes [lds + 16 l, +16)), from inline asm so the compiler
// does not answer later LDS reads with waits on it (the caller waits).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void q35_dma16(const void *base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, %2"
               :: "v"(voff), "s"(lds), "s"(base) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t q35_lds_addr(const float *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float *)p;
}

template <int D>
__device__ void q35_attention(const Q35AttnArgs &a) {
  constexpr int DC = D / 4, DT = D / 16, KS = D + 4, PS = 20;
  constexpr int TILE = 16 * KS;                  // floats of one K (or V) tile
  extern __shared__ __attribute__((aligned(16))) float attn_lds[];
  float *plds = attn_lds + 4 * TILE;             // [4 waves][16 q][PS]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int j = lane >> 4, col = lane & 15;
  const int G = a.Hq / a.Hkv, sub = 4 / G;
  int blk = blockIdx.x;
  const int split = blk % a.nsplit;
  blk /= a.nsplit;
  const int qt = a.qtiles - 1 - blk % a.qtiles;  // longest tiles first
  blk /= a.qtiles;
  const int hk = blk % a.Hkv, b = blk / a.Hkv;
  const int h = hk * G + wv % G;
  const int q0 = (qt * sub + wv / G) * 16;
  const int last_q = min(a.S, (qt + 1) * sub * 16) - 1;
  const int all_tiles = last_q / 16 + 1;
  const int per = (all_tiles + a.nsplit - 1) / a.nsplit;
  const int t_begin = split * per;
  const int ntiles = min(all_tiles, t_begin + per);  // this split walks tiles [t_begin, ntiles)
  const float *kbase = a.kc + ((int64_t)b * a.Hkv + hk) * a.Lmax * D;
  const float *vbase = a.vc + ((int64_t)b * a.Hkv + hk) * a.Lmax * D;
  // q rows of this wave (clamped to S - 1 for loads; rows >= S are not stored)
  float qreg[DC];
  {
    const int qi = min(q0 + col, a.S - 1);
    const float *qp = a.q + (((int64_t)b * a.S + qi) * a.Hq + h) * D + DC * j;
#pragma unroll
    for (int c = 0; c < DC; c += 4) {
      const float4 v = *(const float4 *)(qp + c);
      qreg[c] = v.x, qreg[c + 1] = v.y, qreg[c + 2] = v.z, qreg[c + 3] = v.w;
    }
  }
  // K/V rows go global -> LDS by LDS DMA, 8 of a tile's 32 rows (16 K, 16
  // V) per wave, one instruction per row with lanes [0, D/4) active (lane l
  // copies d 4l..4l+3 into the padded row; masked lanes write nothing). No
  // registers hold a tile in flight, so tile t + 1 loads while tile t is
  // used; the loop waits for the DMAs itself before each barrier. Keys past
  // S repeat row S - 1 (never visible).
  const int wvu = __builtin_amdgcn_readfirstlane(wv);
  auto issue_tile = [&](int t, int buf) {
    if (lane < D / 4) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = wvu * 8 + i, kv = row >> 4, kr = row & 15;
        const int key = min(16 * t + kr, a.S - 1);
        q35_dma16(kv ? vbase : kbase, (uint32_t)(key * D + 4 * lane) * 4u,
                  q35_lds_addr(attn_lds + (2 * buf + kv) * TILE + kr * KS));
      }
    }
  };
  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) m[i] = -__builtin_huge_valf(), l[i] = 0.f;
  float *pw = plds + wv * 16 * PS;
  if (t_begin < ntiles) issue_tile(t_begin, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  for (int t = t_begin; t < ntiles; ++t) {
    const int buf = (t - t_begin) & 1;
    if (t + 1 < ntiles) issue_tile(t + 1, buf ^ 1);  // that buffer's tile was used before the last barrier
    if (16 * t <= q0 + 15) {  // some key of the tile is visible to this wave's queries
      const float *kt = attn_lds + (2 * buf) * TILE + col * KS + DC * j;
      // four independent accumulators keep the MFMA pipe busy (no chain of
      // D / 4 dependent MFMAs)
      f32x4 s4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) s4[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < DC; c += 4) {
        const float4 kk = *(const float4 *)(kt + c);
        s4[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(qreg[c], kk.x, s4[0], 0, 0, 0);
        s4[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(qreg[c + 1], kk.y, s4[1], 0, 0, 0);
        s4[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(qreg[c + 2], kk.z, s4[2], 0, 0, 0);
        s4[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(qreg[c + 3], kk.w, s4[3], 0, 0, 0);
      }
      const f32x4 sc = (s4[0] + s4[1]) + (s4[2] + s4[3]);
      const int key = 16 * t + col;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qpos = q0 + 4 * j + i;
        const float s_ = key <= qpos ? sc[i] * a.scale : -__builtin_huge_valf();
        const float mn = fmaxf(m[i], row_max16(s_));
        // a split may start at tiles where a row sees no key yet (m, mn = -inf)
        const float alpha = m[i] == -__builtin_huge_valf() ? 0.f : __expf(m[i] - mn);
        const float pv = mn == -__builtin_huge_valf() ? 0.f : __expf(s_ - mn);
        l[i] = l[i] * alpha + row_add16(pv);
        m[i] = mn;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt][i] *= alpha;
        pw[(4 * j + i) * PS + col] = pv;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const float4 pa = *(const float4 *)(pw + col * PS + 4 * j);
      const float *vt = attn_lds + (2 * buf + 1) * TILE + 4 * j * KS + col;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.x, vt[0 * KS + 16 * dt], o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.y, vt[1 * KS + 16 * dt], o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.z, vt[2 * KS + 16 * dt], o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa.w, vt[3 * KS + 16 * dt], o[dt], 0, 0, 0);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the next tile's DMAs
    __syncthreads();
  }
  if (a.nsplit > 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qpos = q0 + 4 * j + i;
      if (qpos < a.S) {
        float *pp = a.part + ((((int64_t)b * a.S + qpos) * a.Hq + h) * a.nsplit + split) * (2 + D);
        if (col == 0) pp[0] = m[i], pp[1] = l[i];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) pp[2 + 16 * dt + col] = o[dt][i];
      }
    }
    return;
  }
  // a row's gate values are all loaded before its stores (a load after a
  // store to possibly the same memory would wait for it: one round trip per
  // value)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int qpos = q0 + 4 * j + i;
    if (qpos < a.S) {
      const float inv = 1.0f / l[i];
      const int64_t off = ((int64_t)b * a.S + qpos) * a.Hq * D + (int64_t)h * D + col;
      float gv[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) gv[dt] = a.gate[off + 16 * dt];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) a.out[off + 16 * dt] = (o[dt][i] * inv) * gv[dt];
    }
  }
}

// Merge of the key-range splits of one (token, query head) row, split order:
// out = gate * sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s. One wave per row.
template <int D>
__device__ void q35_attention_combine(const Q35AttnArgs &a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // t * Hq + h
  if (row >= (int64_t)a.B * a.S * a.Hq) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const float *pp = a.part + row * a.nsplit * (2 + D);
  float M = -__builtin_huge_valf();
  for (int sp = 0; sp < a.nsplit; ++sp) M = fmaxf(M, pp[sp * (2 + D)]);
  float L = 0.f, o[D / 64];
#pragma unroll
  for (int e = 0; e < D / 64; ++e) o[e] = 0.f;
  for (int sp = 0; sp < a.nsplit; ++sp) {
    const float ms = pp[sp * (2 + D)];
    const float f = ms == -__builtin_huge_valf() ? 0.f : __expf(ms - M);
    L += f * pp[sp * (2 + D) + 1];
#pragma unroll
    for (int e = 0; e < D / 64; ++e) o[e] += f * pp[sp * (2 + D) + 2 + 64 * e + lane];
  }
  const float inv = 1.0f / L;
  const int64_t off = row * D;  // [T, Hq * D] = row-major (t * Hq + h) * D
  float gv[D / 64];  // loaded before the stores (see q35_attention)
#pragma unroll
  for (int e = 0; e < D / 64; ++e) gv[e] = a.gate[off + 64 * e + lane];
#pragma unroll
  for (int e = 0; e < D / 64; ++e) a.out[off + 64 * e + lane] = (o[e] * inv) * gv[e];
}

#define RXW8_Q35_ATTN(D)                                                                    \
  extern "C" __global__ void __launch_bounds__(256) rxw8_q35_attention_d##D(Q35AttnArgs a) { \
    q35_attention<D>(a);                                                                    \
  }                                                                                         \
  extern "C" __global__ void __launch_bounds__(256) rxw8_q35_attention_combine_d##D(Q35AttnArgs a) { \
    q35_attention_combine<D>(a);                                                            \
  }
RXW8_Q35_ATTN(64)
RXW8_Q35_ATTN(128)
RXW8_Q35_ATTN(256)

// ---- 1 + w of a zero-centred norm weight (layers.rs(nn):476-491), stored once
// for the GEMV's RMSNorm prologue (which multiplies by the weight as given)
struct Q35ShiftArgs {
  const float *w;
  float *out;
  int64_t n;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_q35_one_plus(Q35ShiftArgs a) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < a.n) a.out[e] = 1.0f + a.w[e];
}

// ---- elementwise product (attended * gate, layers.rs:93-94), in place ------
struct Q35MulArgs {
  float *x;
  const float *y;
  int64_t n;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_q35_mul(Q35MulArgs a) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < a.n;
       e += (int64_t)gridDim.x * blockDim.x)
    a.x[e] *= a.y[e];
}

// ---- gated-delta prologue for one (token, head) per workgroup
// (layers.rs:131-195): the causal depthwise conv + SiLU of the head's q, k and
// v channels, out[t, c] = silu(sum_j w[c, j] * x[t - (k-1) + j, c]) (zero
// before position 0 of the sequence; a correlation, conv2d_oihw with padding
// (k-1, 0)); q = l2norm(q) / sqrt(Dl), k = l2norm(k) with
// l2norm(x) = x * rsqrt(sum x^2 + 1e-6) (layers.rs:102-111); and the head's
// beta = sigmoid(b), g = exp(softplus(a + dt_bias) * -exp(A_log)) with
// softplus(x) = max(x, 0) + log1p(exp(-|x|)) (ops.rs:256-262).
// The projection row of token t (bf16, `stride` elements) holds the conv
// input channels [0, 3W), then z [3W, 4W), b [4W, 4W + Hl), a after b.
struct Q35MixPrepArgs {
  const void *raw;               // [T, stride], f32 (F32 compute) or bf16
  const float *conv_w;           // [3W, k]
  const float *a_log, *dt_bias;  // [Hl]
  float *mixed;                  // [T, 3W]: q (normed, scaled), k (normed), v
  float *beta, *g;               // [T, Hl]
  float *lg;                     // [T, Hl] log g (the chunked recurrence's decays), or null
  int64_t stride;
  int S, Hl, Dl, k;
  float q_scale;
  int raw_f32;
};

// Every load of the workgroup goes out before the first use (one memory
// round trip): the k taps of its channels at clamped rows (a tap before
// position 0 adds an exact 0 in its place, so each sum keeps the order and
// value of the skipped form), the conv weights, and the head's b, a, dt_bias
// and A_log (loaded by every thread, used by thread 0). One body per source
// dtype and for k = 4 (any other k takes the loop after the loads).
template <bool F32, int KT>
__device__ __forceinline__ void q35_mix_prep(const Q35MixPrepArgs &a) {
  __shared__ float red[2][2];
  const int64_t t = blockIdx.x / a.Hl;
  const int h = (int)(blockIdx.x - t * a.Hl);
  const int pos = (int)(t % a.S);
  const int64_t W = (int64_t)a.Hl * a.Dl;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int k = KT > 0 ? KT : a.k;
  auto ldr = [&](int64_t i) {
    if constexpr (F32)
      return ((const float *)a.raw)[i];
    else
      return bf16_bits_to_f32(((const uint16_t *)a.raw)[i]);
  };
  const int64_t hrow = t * a.stride + 4 * W;
  const float b_raw = ldr(hrow + h), a_raw = ldr(hrow + a.Hl + h);
  const float dtb = a.dt_bias[h], alog = a.a_log[h];
  constexpr int NK = KT > 0 ? KT : 1;
  float xv[2][3][NK], cw[2][3][NK];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int c = min((int)threadIdx.x + 128 * r, a.Dl - 1);  // (lanes past Dl: clamped, not stored)
#pragma unroll
    for (int part = 0; part < 3; ++part) {
      const int64_t ch = part * W + (int64_t)h * a.Dl + c;
#pragma unroll
      for (int j = 0; j < NK; ++j) {
        const int src = max(pos - (k - 1) + j, 0);
        xv[r][part][j] = ldr((t - pos + src) * a.stride + ch);
        cw[r][part][j] = a.conv_w[ch * k + j];
      }
    }
  }
  float qv[2], kv[2], vv[2];  // channels c = threadIdx.x and c + 128 (Dl <= 256)
  float sq = 0.f, sk = 0.f;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int c = threadIdx.x + 128 * r;
    qv[r] = kv[r] = vv[r] = 0.f;
    float acc[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int part = 0; part < 3; ++part) {
      if constexpr (KT > 0) {
#pragma unroll
        for (int j = 0; j < KT; ++j)
          acc[part] += pos - (KT - 1) + j >= 0 ? cw[r][part][j] * xv[r][part][j] : 0.f;
      } else {
        const int64_t ch = part * W + (int64_t)h * a.Dl + min(c, a.Dl - 1);
        for (int j = 0; j < k; ++j) {
          const int src = pos - (k - 1) + j;
          if (src < 0) continue;
          acc[part] += a.conv_w[ch * k + j] * ldr((t - pos + src) * a.stride + ch);
        }
      }
    }
    if (c < a.Dl) {
      qv[r] = acc[0] * sigmoid_f32(acc[0]);
      kv[r] = acc[1] * sigmoid_f32(acc[1]);
      vv[r] = acc[2] * sigmoid_f32(acc[2]);
      sq += qv[r] * qv[r];
      sk += kv[r] * kv[r];
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    sq += __shfl_xor(sq, o);
    sk += __shfl_xor(sk, o);
  }
  if (lane == 0) red[wv][0] = sq, red[wv][1] = sk;
  __syncthreads();
  const float qs = (1.0f / sqrtf(red[0][0] + red[1][0] + 1e-6f)) * a.q_scale;
  const float ks = 1.0f / sqrtf(red[0][1] + red[1][1] + 1e-6f);
  float *m = a.mixed + t * 3 * W + (int64_t)h * a.Dl;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int c = threadIdx.x + 128 * r;
    if (c < a.Dl) {
      m[c] = qv[r] * qs;
      m[W + c] = kv[r] * ks;
      m[2 * W + c] = vv[r];
    }
  }
  if (threadIdx.x == 0) {
    a.beta[t * a.Hl + h] = sigmoid_f32(b_raw);
    const float x = a_raw + dtb;
    const float sp = fmaxf(x, 0.f) + log1pf(expf(-fabsf(x)));
    const float lgv = sp * -expf(alog);
    a.g[t * a.Hl + h] = expf(lgv);
    if (a.lg) a.lg[t * a.Hl + h] = lgv;
  }
}
extern "C" __global__ void __launch_bounds__(128) rxw8_q35_mix_prep(Q35MixPrepArgs a) {
  if (a.k == 4) {
    if (a.raw_f32)
      q35_mix_prep<true, 4>(a);
    else
      q35_mix_prep<false, 4>(a);
  } else {
    if (a.raw_f32)
      q35_mix_prep<true, 0>(a);
    else
      q35_mix_prep<false, 0>(a);
  }
}

// ---- delta-rule recurrence (layers.rs:197-234): one workgroup of DL threads
// per (sequence, head); thread j keeps column j of the state S (DL x DL, f32)
// in registers and walks the positions in order:
//   S *= g_t;  pred_j = sum_i S_ij k_i;  delta_j = (v_j - pred_j) beta_t;
//   S_ij += k_i delta_j;  out_j = sum_i S_ij q_i.
// q_t and k_t go through LDS (double-buffered); the next step's values are
// loaded while the current one is computed.
struct Q35DeltaArgs {
  const float *mixed;  // [T, 3W]: q (scaled, normed), k (normed), v
  const float *beta, *g;  // [T, Hl]
  float *out;          // [T, Hl, Dl]
  int B, S, Hl;
};

template <int DL>
__device__ void delta_rule(const Q35DeltaArgs &a) {
  __shared__ float qk[2][2][DL];
  const int j = threadIdx.x;
  const int bh = blockIdx.x, b = bh / a.Hl, h = bh - b * a.Hl;
  const int64_t W = (int64_t)a.Hl * DL;
  float st[DL];
#pragma unroll
  for (int i = 0; i < DL; ++i) st[i] = 0.f;
  auto row = [&](int pos) { return (int64_t)b * a.S + pos; };
  float qn = 0.f, kn = 0.f, vn = 0.f, bn = 0.f, gn = 0.f;
  auto fetch = [&](int pos) {
    const float *m = a.mixed + row(pos) * 3 * W + (int64_t)h * DL + j;
    qn = m[0];
    kn = m[W];
    vn = m[2 * W];
    bn = a.beta[row(pos) * a.Hl + h];
    gn = a.g[row(pos) * a.Hl + h];
  };
  fetch(0);
  for (int pos = 0; pos < a.S; ++pos) {
    const int buf = pos & 1;
    qk[buf][0][j] = qn;
    qk[buf][1][j] = kn;
    const float v = vn, beta = bn, gt = gn;
    __syncthreads();  // q_t, k_t visible; the other buffer is free again
    if (pos + 1 < a.S) fetch(pos + 1);
    float pred = 0.f;
#pragma unroll
    for (int i = 0; i < DL; ++i) {
      st[i] *= gt;
      pred += st[i] * qk[buf][1][i];
    }
    const float delta = (v - pred) * beta;
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < DL; ++i) {
      st[i] += qk[buf][1][i] * delta;
      o += st[i] * qk[buf][0][i];
    }
    a.out[row(pos) * W + (int64_t)h * DL + j] = o;
  }
}

// Launched with exactly DL threads (every thread takes part in the barriers).
#define RXW8_Q35_DELTA(DL)                                                         \
  extern "C" __global__ void __launch_bounds__(DL) rxw8_q35_delta_rule_d##DL(Q35DeltaArgs a) { \
    delta_rule<DL>(a);                                                             \
  }
RXW8_Q35_DELTA(8)
RXW8_Q35_DELTA(16)
RXW8_Q35_DELTA(32)

// Sum over the 16 lanes of a DPP row, the same bits in every lane (each
// stage adds a lane's value to a rotation of the row: row_ror 8, row_ror 4,
// then the quad swaps 2 and 1; addition is commutative, so lanes agree).
__device__ __forceinline__ float row_sum16(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));
  return v;
}

// The same recurrence with each state column spread over LPC lanes (a DPP row
// of 16, or two rows joined by v_permlane16_swap): lane p of column j keeps
// S[i][j] for i = E p .. E p + E - 1 (E = DL / LPC), and a (sequence, head)
// runs on DL / (64 / LPC * NWV) workgroups (the columns of S evolve
// independently). With S' the state
// before position t, the step is evaluated as
//   a_k = S'^T k,  a_q = S'^T q,  kq = k . q      (three sums, one DPP pass)
//   pred = g a_k,  delta = (v - pred) beta,  o = g a_q + delta kq,
//   S = g S' + k delta^T,
// the same quantities as the reference's order (g S' first) with g factored
// out of the sums, so one reduction round (not two) sits on the serial chain.
// The inputs of the next NPF positions are in flight while one is computed;
// beta and g of NPF positions come as one lane-indexed vector load (lane i of
// the wave holds position t0 + i) and reach the step by v_readlane, so no
// scalar-cache load (whose waits cannot be counted per load) sits in the loop.
template <int DL, int LPC = 16, int NWV = 4, int NPF = 16>
__device__ void delta_rule_rows(const Q35DeltaArgs &a) {
  // LPC lanes per column (16 or 32), NWV waves per workgroup, NPF positions in flight
  constexpr int E = DL / LPC, CPG = 64 / LPC * NWV, GROUPS = DL / CPG;
  static_assert((LPC == 16 || LPC == 32) && E % 4 == 0 && DL % CPG == 0, "layout");
  const int lane = threadIdx.x & 63, p = lane & (LPC - 1);
  const int bh = blockIdx.x / GROUPS, grp = blockIdx.x - bh * GROUPS;
  const int b = bh / a.Hl, h = bh - b * a.Hl;
  const int j = grp * CPG + threadIdx.x / LPC;
  const int64_t W = (int64_t)a.Hl * DL;
  struct Vals {
    float q[E], k[E], v;
  };
  auto fetch = [&](int pos, Vals &o) {
    const int64_t row = (int64_t)b * a.S + pos;
    const float *m = a.mixed + row * 3 * W + (int64_t)h * DL;
#pragma unroll
    for (int e = 0; e < E; e += 4) {
      const float4 qq = *(const float4 *)(m + E * p + e);
      const float4 kk = *(const float4 *)(m + W + E * p + e);
      o.q[e] = qq.x, o.q[e + 1] = qq.y, o.q[e + 2] = qq.z, o.q[e + 3] = qq.w;
      o.k[e] = kk.x, o.k[e + 1] = kk.y, o.k[e + 2] = kk.z, o.k[e + 3] = kk.w;
    }
    o.v = m[2 * W + j];
  };
  // beta, g of positions t0 .. t0 + NPF - 1 in lanes 0 .. NPF - 1
  auto fetch_bg = [&](int t0, float &bb, float &gg) {
    const int64_t row = (int64_t)b * a.S + min(t0 + (lane & (NPF - 1)), a.S - 1);
    bb = a.beta[row * a.Hl + h];
    gg = a.g[row * a.Hl + h];
  };
  float st[E];
#pragma unroll
  for (int e = 0; e < E; ++e) st[e] = 0.f;
  auto step = [&](const Vals &c, float beta, float g, int pos) {
    float ak[2] = {0.f, 0.f}, aq[2] = {0.f, 0.f}, kq[2] = {0.f, 0.f};
#pragma unroll
    for (int e = 0; e < E; ++e) {
      ak[e & 1] += st[e] * c.k[e];
      aq[e & 1] += st[e] * c.q[e];
      kq[e & 1] += c.k[e] * c.q[e];
    }
    float sk = ak[0] + ak[1], sq = aq[0] + aq[1], skq = kq[0] + kq[1];
    if (LPC == 32) sk = sum_xor16(sk), sq = sum_xor16(sq), skq = sum_xor16(skq);
    sk += dpp_rot<0x128>(sk), sq += dpp_rot<0x128>(sq), skq += dpp_rot<0x128>(skq);
    sk += dpp_rot<0x124>(sk), sq += dpp_rot<0x124>(sq), skq += dpp_rot<0x124>(skq);
    sk += dpp_rot<0x4e>(sk), sq += dpp_rot<0x4e>(sq), skq += dpp_rot<0x4e>(skq);
    sk += dpp_rot<0xb1>(sk), sq += dpp_rot<0xb1>(sq), skq += dpp_rot<0xb1>(skq);
    const float delta = (c.v - g * sk) * beta;
#pragma unroll
    for (int e = 0; e < E; ++e) st[e] = g * st[e] + c.k[e] * delta;
    if (p == 0) a.out[((int64_t)b * a.S + pos) * W + (int64_t)h * DL + j] = g * sq + delta * skq;
  };
  auto lane_value = [](float v, int i) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), i));
  };
  Vals buf[NPF];
#pragma unroll
  for (int i = 0; i < NPF; ++i) fetch(min(i, a.S - 1), buf[i]);
  float bcur, gcur;
  fetch_bg(0, bcur, gcur);
  int t0 = 0;
  for (; t0 + NPF <= a.S; t0 += NPF) {
    float bnext, gnext;
    fetch_bg(t0 + NPF, bnext, gnext);
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      const Vals cur = buf[i];
      fetch(min(t0 + i + NPF, a.S - 1), buf[i]);
      step(cur, lane_value(bcur, i), lane_value(gcur, i), t0 + i);
    }
    bcur = bnext, gcur = gnext;
  }
#pragma unroll
  for (int i = 0; i < NPF; ++i)
    if (t0 + i < a.S) step(buf[i], lane_value(bcur, i), lane_value(gcur, i), t0 + i);
}

// ---- chunked delta rule (layers.rs:197-234, the same recurrence in chunks of
// C = 64 positions). With S0 the state before a chunk, Gamma_t = prod_{u<=t}
// g_u = exp(gam_t) (gam the inclusive cumulative log decay, so every ratio
// Gamma_t / Gamma_s with s <= t is exp(gam_t - gam_s) <= 1), unrolling
// S_t = g_t S_{t-1} + k_t delta_t^T gives
//   (I + A) Delta = diag(beta) (V - diag(Gamma) K S0),
//     A_ts = beta_t (Gamma_t / Gamma_s) k_t . k_s  (s < t),
//   O = diag(Gamma) Q S0 + P Delta,  P_ts = (Gamma_t / Gamma_s) q_t . k_s (s <= t),
//   S_end = Gamma_end S0 + sum_s (Gamma_end / Gamma_s) k_s Delta_s^T.
// With U = (I + A)^-1 diag(beta) V and W = (I + A)^-1 diag(beta Gamma) K,
// Delta = U - W S0. rxw8_q35_delta_chunk_d* forms, for every chunk in
// parallel, U, W, P, Qg = diag(Gamma) Q, KdT = (diag(Gamma_end / Gamma) K)^T
// (state rows major, so the walk reads it in 16-byte pieces) and gam;
// rxw8_q35_delta_scan_d* walks the chunks in order with the state on the
// matrix cores. Rows past the sequence are zero (beta = 0, k = q = v = 0,
// lg = 0), so every chunk is processed as 64 rows.
struct Q35ChunkArgs {
  const float *mixed;        // [T, 3W]: q, k, v
  const float *beta, *lg;    // [T, Hl]
  // per chunk of each (sequence, head): [64][DL], [64][DL], [64][64], [64],
  // [64][DL], [DL][64]
  float *u, *wm, *pm, *gam, *qg, *kdt;
  float *out;                // [T, W] (the scan)
  int S, Hl, NC;
};

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One chunk of one (sequence, head): 256 threads (4 waves).
template <int DL>
__device__ void delta_chunk(const Q35ChunkArgs &a) {
  constexpr int C = 64, KP = DL + 4, KQ = DL / 4;
  __shared__ __attribute__((aligned(16))) float ks[C][KP], qs[C][KP];
  __shared__ __attribute__((aligned(16))) float as[C][C + 4];
  __shared__ float bs[C], gs[C];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t ch = blockIdx.x;
  const int bh = (int)(ch / a.NC), c = (int)(ch - (int64_t)bh * a.NC);
  const int b = bh / a.Hl, h = bh - b * a.Hl;
  const int t0 = c * C, n = min(C, a.S - t0);
  const int64_t W = (int64_t)a.Hl * DL;
  const int64_t row0 = (int64_t)b * a.S + t0;
  // the v column of the U half of the solve, loaded first (thread = column)
  float x[C];
#pragma unroll
  for (int t = 0; t < C; ++t)
    x[t] = tid < DL && t < n ? a.mixed[(row0 + t) * 3 * W + 2 * W + (int64_t)h * DL + tid] : 0.f;
  // k and q rows of the chunk (rows past the sequence zero)
  for (int e = tid; e < C * KQ; e += 256) {
    const int t = e / KQ, d4 = e - t * KQ;
    float4 qv = {0.f, 0.f, 0.f, 0.f}, kv = qv;
    if (t < n) {
      const float *m = a.mixed + (row0 + t) * 3 * W + (int64_t)h * DL + 4 * d4;
      qv = *(const float4 *)m;
      kv = *(const float4 *)(m + W);
    }
    *(float4 *)&qs[t][4 * d4] = qv;
    *(float4 *)&ks[t][4 * d4] = kv;
  }
  if (wave == 0) {  // inclusive scan of the log decays; beta
    float x = lane < n ? a.lg[(row0 + lane) * a.Hl + h] : 0.f;
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    gs[lane] = x;
    bs[lane] = lane < n ? a.beta[(row0 + lane) * a.Hl + h] : 0.f;
  }
  __syncthreads();
  // Qg = diag(Gamma) Q; KdT[i][s] = (Gamma_end / Gamma_s) k_s[i]
  {
    float *qg = a.qg + ch * C * DL, *kdt = a.kdt + ch * C * DL;
    const float gend = gs[C - 1];
    for (int e = tid; e < C * KQ; e += 256) {
      const int t = e / KQ, d4 = e - t * KQ;
      const float f = expf(gs[t]);
      const float4 q4 = *(const float4 *)&qs[t][4 * d4];
      *(float4 *)(qg + t * DL + 4 * d4) = float4{f * q4.x, f * q4.y, f * q4.z, f * q4.w};
    }
    for (int e = tid; e < DL * (C / 4); e += 256) {
      const int i = e / (C / 4), s4 = 4 * (e - i * (C / 4));
      float4 o;
      o.x = expf(gend - gs[s4]) * ks[s4][i];
      o.y = expf(gend - gs[s4 + 1]) * ks[s4 + 1][i];
      o.z = expf(gend - gs[s4 + 2]) * ks[s4 + 2][i];
      o.w = expf(gend - gs[s4 + 3]) * ks[s4 + 3][i];
      *(float4 *)(kdt + i * C + s4) = o;
    }
  }
  // K K^T and Q K^T, row tile = wave, column tiles 0..3; the MFMA k index of
  // lane l at step kk is 4 kk + l / 16 (the same in both operands; rows 132
  // floats apart put a step's 64 reads on distinct banks two by two)
  f32x4 kk_acc[4], qk_acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) kk_acc[j] = qk_acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int kk = 0; kk < KQ; ++kk) {
    const int d = 4 * kk + g;
    const float ak = ks[16 * wave + r16][d], aq = qs[16 * wave + r16][d];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float bk = ks[16 * j + r16][d];
      kk_acc[j] = mfma4(ak, bk, kk_acc[j]);
      qk_acc[j] = mfma4(aq, bk, qk_acc[j]);
    }
  }
  // lane holds rows t = 16 wave + 4 g + r, columns s = 16 j + r16
  float *pm = a.pm + ch * C * C;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * wave + 4 * g + r, s2 = 16 * j + r16;
      // (gam is non-increasing, so the exponent is <= 0 wherever s <= t)
      const float e = expf(fminf(gs[t] - gs[s2], 0.f));
      as[t][s2] = s2 < t ? bs[t] * e * kk_acc[j][r] : 0.f;
      pm[t * C + s2] = s2 <= t ? e * qk_acc[j][r] : 0.f;
    }
  __syncthreads();
  // forward substitution, thread = one column of X = [U | W]:
  //   X_t = B_t - sum_{s<t} A_ts X_s,  B_t = beta_t v_t (U), beta_t Gamma_t k_t (W)
  if (tid < 2 * DL) {
    const bool is_w = tid >= DL;
    const int col = is_w ? tid - DL : tid;
#pragma unroll
    for (int t = 0; t < C; ++t) x[t] = (is_w ? bs[t] * expf(gs[t]) * ks[t][col] : bs[t] * x[t]);
    // row t's A values are read while row t - 1 is reduced (one LDS round
    // trip per row, not one per pair of reads)
    float4 arow[2][C / 4];
    arow[1][0] = *(const float4 *)&as[1][0];
#pragma unroll
    for (int t = 1; t < C; ++t) {
      const int cur = t & 1;
      if (t + 1 < C)
#pragma unroll
        for (int q = 0; q < (t + 4) / 4; ++q) arow[cur ^ 1][q] = *(const float4 *)&as[t + 1][4 * q];
      float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < t; s2 += 4) {  // A_ts = 0 for s >= t
        const float4 a4 = arow[cur][s2 / 4];
        p0 += a4.x * x[s2];
        if (s2 + 1 < t) p1 += a4.y * x[s2 + 1];
        if (s2 + 2 < t) p2 += a4.z * x[s2 + 2];
        if (s2 + 3 < t) p3 += a4.w * x[s2 + 3];
      }
      x[t] -= (p0 + p1) + (p2 + p3);
    }
    float *dst = (is_w ? a.wm : a.u) + ch * C * DL + col;
#pragma unroll
    for (int t = 0; t < C; ++t) dst[t * DL] = x[t];
  }
  if (tid < C) a.gam[ch * C + tid] = gs[tid];
}

// The chunks of one (sequence, head) in order for 16 columns of the state
// (grid B * Hl * DL / 16, 256 threads). Wave w owns rows 16 w .. 16 w + 15 of
// the chunk for Delta and O, and state rows 16 it .. + 15 for it = w,
// w + 4, .. (DL / 64 tiles per wave) for the update. The state and Delta pass
// between waves through LDS.
template <int DL>
__device__ void delta_scan(const Q35ChunkArgs &a) {
  constexpr int C = 64, KQ = DL / 4, GROUPS = DL / 16, IT = DL / 64;
  __shared__ float ss[DL][17], ds[C][17];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int bh = blockIdx.x / GROUPS, grp = blockIdx.x - bh * GROUPS;
  const int b = bh / a.Hl, h = bh - b * a.Hl;
  const int c0 = grp * 16;
  const int64_t W = (int64_t)a.Hl * DL;
  for (int e = tid; e < DL * 17; e += 256) (&ss[0][0])[e] = 0.f;
  // Operands of one chunk, each loaded a chunk ahead, right after the current
  // chunk has consumed the registers it goes to:
  //   wreg / qreg  W and Qg rows of this wave's tile (lane k index KQ (l / 16) + kk)
  //   preg         P row (lane k index 16 (l / 16) + kk), ureg  U in the output layout
  //   kreg         KdT rows 16 it + l % 16, columns s = 16 (l / 16) + kk
  float wreg[KQ], qreg[KQ], preg[16], ureg[4], kreg[IT][16], gend;
  auto load_wq = [&](int c) {
    const int64_t ch = (int64_t)bh * a.NC + c;
    const int t = 16 * wave + r16;
    const float *wr = a.wm + (ch * C + t) * DL + KQ * g;
    const float *qr = a.qg + (ch * C + t) * DL + KQ * g;
#pragma unroll
    for (int kk = 0; kk < KQ; kk += 4) {
      const float4 w4 = *(const float4 *)(wr + kk);
      const float4 q4 = *(const float4 *)(qr + kk);
      wreg[kk] = w4.x, wreg[kk + 1] = w4.y, wreg[kk + 2] = w4.z, wreg[kk + 3] = w4.w;
      qreg[kk] = q4.x, qreg[kk + 1] = q4.y, qreg[kk + 2] = q4.z, qreg[kk + 3] = q4.w;
    }
  };
  auto load_pu = [&](int c) {
    const int64_t ch = (int64_t)bh * a.NC + c;
    const float *pr = a.pm + (ch * C + 16 * wave + r16) * C + 16 * g;
#pragma unroll
    for (int kk = 0; kk < 16; kk += 4) {
      const float4 p4 = *(const float4 *)(pr + kk);
      preg[kk] = p4.x, preg[kk + 1] = p4.y, preg[kk + 2] = p4.z, preg[kk + 3] = p4.w;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) ureg[r] = a.u[(ch * C + 16 * wave + 4 * g + r) * DL + c0 + r16];
  };
  auto load_k = [&](int c) {
    const int64_t ch = (int64_t)bh * a.NC + c;
#pragma unroll
    for (int q2 = 0; q2 < IT; ++q2) {
      const float *kr = a.kdt + (ch * DL + 16 * (wave + 4 * q2) + r16) * C + 16 * g;
#pragma unroll
      for (int kk = 0; kk < 16; kk += 4) {
        const float4 k4 = *(const float4 *)(kr + kk);
        kreg[q2][kk] = k4.x, kreg[q2][kk + 1] = k4.y, kreg[q2][kk + 2] = k4.z, kreg[q2][kk + 3] = k4.w;
      }
    }
    gend = a.gam[ch * C + C - 1];
  };
  load_wq(0);
  load_pu(0);
  load_k(0);
  __syncthreads();
  for (int c = 0; c < a.NC; ++c) {
    const int n = min(C, a.S - c * C);
    const int64_t row0 = (int64_t)b * a.S + c * C;
    // the next chunk's operands (the last chunk re-reads its own: every
    // iteration issues the same loads, so the waits for them stay counted)
    const int cn = min(c + 1, a.NC - 1);
    // W S0 and Qg S0 (16 x 16 each); the state fragments read first
    f32x4 wsa, qsa;
    {
      float sv[KQ];
#pragma unroll
      for (int kk = 0; kk < KQ; ++kk) sv[kk] = ss[KQ * g + kk][r16];
      f32x4 w2[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}}, q2v[2] = {w2[0], w2[0]};
#pragma unroll
      for (int kk = 0; kk < KQ; ++kk) {
        w2[kk & 1] = mfma4(wreg[kk], sv[kk], w2[kk & 1]);
        q2v[kk & 1] = mfma4(qreg[kk], sv[kk], q2v[kk & 1]);
      }
      wsa = w2[0] + w2[1];
      qsa = q2v[0] + q2v[1];
    }
    load_wq(cn);
#pragma unroll
    for (int r = 0; r < 4; ++r) ds[16 * wave + 4 * g + r][r16] = ureg[r] - wsa[r];
    __syncthreads();  // Delta in LDS; every read of S0 for W S0 / Qg S0 done
    // O = Qg S0 + P Delta (the Delta fragments, read once, also feed the update)
    float dv[16];
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) dv[kk] = ds[16 * g + kk][r16];
    f32x4 o = qsa, o2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 16; kk += 2) {
      o = mfma4(preg[kk], dv[kk], o);
      o2 = mfma4(preg[kk + 1], dv[kk + 1], o2);
    }
    o += o2;
    load_pu(cn);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * wave + 4 * g + r;
      if (t < n) a.out[(row0 + t) * W + (int64_t)h * DL + c0 + r16] = o[r];
    }
    // S_end = Gamma_end S0 + KdT Delta
    f32x4 sn[IT];
    const float eg = expf(gend);
#pragma unroll
    for (int q2 = 0; q2 < IT; ++q2) {
      const int it = wave + 4 * q2;
#pragma unroll
      for (int r = 0; r < 4; ++r) sn[q2][r] = eg * ss[16 * it + 4 * g + r][r16];
      f32x4 s2v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 16; kk += 2) {
        sn[q2] = mfma4(kreg[q2][kk], dv[kk], sn[q2]);
        s2v = mfma4(kreg[q2][kk + 1], dv[kk + 1], s2v);
      }
      sn[q2] += s2v;
    }
    load_k(cn);
    __syncthreads();  // every read of S0 done
#pragma unroll
    for (int q2 = 0; q2 < IT; ++q2) {
      const int it = wave + 4 * q2;
#pragma unroll
      for (int r = 0; r < 4; ++r) ss[16 * it + 4 * g + r][r16] = sn[q2][r];
    }
    __syncthreads();  // the new state in LDS; Delta free
  }
}

#define RXW8_Q35_CHUNK(DL)                                                         \
  extern "C" __global__ void __launch_bounds__(256) rxw8_q35_delta_chunk_d##DL(Q35ChunkArgs a) { \
    delta_chunk<DL>(a);                                                            \
  }                                                                                \
  extern "C" __global__ void __launch_bounds__(256) rxw8_q35_delta_scan_d##DL(Q35ChunkArgs a) { \
    delta_scan<DL>(a);                                                             \
  }
RXW8_Q35_CHUNK(64)
RXW8_Q35_CHUNK(128)

// Dl 64: 256 threads = 16 columns x 16 lanes, grid B * Hl * 4; Dl 128: 256
// threads = 8 columns x 32 lanes (4 rows per lane), grid B * Hl * 16, which
// measured 3% faster per forward than 16 lanes (0.8B model, S = 1024:
// 11.85 against 12.15-12.29 ms); 8-wave workgroups (two waves per SIMD) were
// slower with either width. 16 positions in flight instead of 8: 11.38
// against 12.14 ms (the loads of position t + 8 had not landed by its turn).
// (Two positions per reduction round, with the second position's sums
// regrouped, measured no faster than this.)
extern "C" __global__ void __launch_bounds__(256) rxw8_q35_delta_rule_d64(Q35DeltaArgs a) {
  delta_rule_rows<64, 16, 4>(a);
}
extern "C" __global__ void __launch_bounds__(256) rxw8_q35_delta_rule_d128(Q35DeltaArgs a) {
  delta_rule_rows<128, 32, 4>(a);
}

// ---- the gated-delta mixer of a short sequence in one launch: one workgroup
// of 512 threads per (sequence, head) forms, for the token rows of the
// sequence in chunks of CH positions,
//   (A) the causal conv (kernel 4) + SiLU of the head's q, k and v channels,
//       the q / k L2 norms, beta and g (the arithmetic of rxw8_q35_mix_prep);
//       thread c < 3 DL owns channel c and all CH positions of the chunk, so
//       the chunk's inputs are one round of loads and the convolution needs
//       no neighbours;
//   (B) the delta-rule recurrence over the chunk's positions, as
//       rxw8_q35_delta_rule_d* evaluates it (S = g S' + k delta^T,
//       o = g S'^T q + delta (k . q), delta = (v - g S'^T k) beta), column j of
//       the state on the LPC = 512 / DL lanes LPC j.. (E = DL / LPC rows
//       each): the columns evolve independently, so this walk has no barrier;
//   (C) the gated RMSNorm o * rsqrt(mean(o^2) + eps) * w * silu(z) of
//       rxw8_q35_rmsnorm for every position of the chunk
// (layers.rs:131-259). Replaces three launches for short sequences; on long
// ones the token-parallel prologue and the 16-lane recurrence are faster
// (here each position's k and q reach all DL columns from one CU's LDS).
struct Q35ShortMixArgs {
  const void *raw;               // [T, stride]: conv channels [0, 3W), z [3W, 4W), b, a
  const float *conv_w;           // [3W, 4]
  const float *a_log, *dt_bias;  // [Hl]
  const float *norm_w;           // [DL] gated-norm weight (applied as given)
  void *out;                     // [T, Hl * DL] gated rows (f32 or bf16)
  int64_t stride;
  int S, Hl, k;                  // k = 4 (the host checks)
  float q_scale, eps;
  int raw_f32, out_f32;
};

template <int DL>
__device__ void linear_short(const Q35ShortMixArgs &a) {
  constexpr int NT = 512, LPC = NT / DL, E = DL / LPC, CH = 16, C3 = 3 * DL, WPP = DL / 64, K = 4;
  static_assert(E % 4 == 0 && C3 <= NT && DL % 64 == 0 && (LPC == 4 || LPC == 8), "layout");
  __shared__ __attribute__((aligned(16))) float qn[CH][DL], kn[CH][DL];
  __shared__ float vn[CH][DL], on[CH][DL], red[CH][8], bb[CH], gg[CH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bh = blockIdx.x, b = bh / a.Hl, h = bh - b * a.Hl;
  const int64_t W = (int64_t)a.Hl * DL;
  // (A) roles: channel threads (waves of one part each), then beta / g threads
  const bool chan = tid < C3;
  const int part = tid / DL, c = tid - part * DL;
  const int64_t col = (int64_t)part * W + (int64_t)h * DL + c;
  float cw[K] = {0.f, 0.f, 0.f, 0.f};
  if (chan)
#pragma unroll
    for (int jj = 0; jj < K; ++jj) cw[jj] = a.conv_w[col * K + jj];
  float hist[K - 1] = {0.f, 0.f, 0.f};  // x at the 3 positions before the chunk (0 before 0)
  const float nw = tid < DL ? a.norm_w[tid] : 0.f;
  // (B) roles
  const int j = tid / LPC, p = tid - j * LPC;
  float st[E];
#pragma unroll
  for (int e = 0; e < E; ++e) st[e] = 0.f;
  // sum over the wave (every lane gets the same bits): lanes l ^ 32, l ^ 16
  // by the VALU exchanges, then within each row of 16
  auto wave_sum = [](float v) {
    v = sum_xor32(v);
    v = sum_xor16(v);
    return row_sum16(v);
  };
  // sum over the LPC lanes of a column (quads, then the half-row mirror)
  auto col_sum = [](float v) {
    v += dpp_rot<0xb1>(v);
    v += dpp_rot<0x4e>(v);
    if (LPC == 8) v += dpp_rot<0x141>(v);
    return v;
  };
  for (int p0 = 0; p0 < a.S; p0 += CH) {
    const int n = min(CH, a.S - p0);
    const int64_t row0 = (int64_t)b * a.S + p0;
    float xv[CH], zv[CH];
#pragma unroll
    for (int r = 0; r < CH; ++r) {  // (the branches on r < n are uniform)
      const int64_t row = (row0 + r) * a.stride;
      xv[r] = chan && r < n ? ld(a.raw, row + col, a.raw_f32) : 0.f;
      zv[r] = tid < DL && r < n ? ld(a.raw, row + 3 * W + (int64_t)h * DL + tid, a.raw_f32) : 0.f;
    }
    if (tid >= C3 && tid - C3 < n) {
      const int r = tid - C3;
      const int64_t row = (row0 + r) * a.stride + 4 * W;
      bb[r] = sigmoid_f32(ld(a.raw, row + h, a.raw_f32));
      const float xg = ld(a.raw, row + a.Hl + h, a.raw_f32) + a.dt_bias[h];
      const float sp = fmaxf(xg, 0.f) + log1pf(expf(-fabsf(xg)));
      gg[r] = expf(sp * -expf(a.a_log[h]));
    }
    float y[CH];
#pragma unroll
    for (int r = 0; r < CH; ++r) {
      y[r] = 0.f;
      if (r >= n) continue;
      float acc = 0.f;
#pragma unroll
      for (int jj = 0; jj < K; ++jj) {
        const int src = r - (K - 1) + jj;
        acc += cw[jj] * (src >= 0 ? xv[src] : hist[K - 1 + src]);
      }
      y[r] = acc * sigmoid_f32(acc);
    }
    if (n == CH) hist[0] = xv[CH - 3], hist[1] = xv[CH - 2], hist[2] = xv[CH - 1];
    if (chan && part < 2)
#pragma unroll
      for (int r = 0; r < CH; ++r) {
        if (r >= n) continue;
        const float sq = wave_sum(y[r] * y[r]);
        if (lane == 0) red[r][wave] = sq;
      }
    __syncthreads();
    if (chan)
#pragma unroll
      for (int r = 0; r < CH; ++r) {
        if (r >= n) continue;
        if (part == 2) {
          vn[r][c] = y[r];
          continue;
        }
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < WPP; ++w) tot += red[r][part * WPP + w];
        if (part == 0)
          qn[r][c] = y[r] * ((1.0f / sqrtf(tot + 1e-6f)) * a.q_scale);
        else
          kn[r][c] = y[r] * (1.0f / sqrtf(tot + 1e-6f));
      }
    __syncthreads();
    // (B)
    for (int r = 0; r < n; ++r) {
      const float beta = bb[r], g = gg[r], v = vn[r][j];
      float ak[2] = {0.f, 0.f}, aq[2] = {0.f, 0.f}, kq[2] = {0.f, 0.f};
      float kk[E];
#pragma unroll
      for (int e = 0; e < E; e += 4) {
        const float4 k4 = *(const float4 *)(&kn[r][E * p + e]);
        const float4 q4 = *(const float4 *)(&qn[r][E * p + e]);
        kk[e] = k4.x, kk[e + 1] = k4.y, kk[e + 2] = k4.z, kk[e + 3] = k4.w;
        const float qq[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          ak[u & 1] += st[e + u] * kk[e + u];
          aq[u & 1] += st[e + u] * qq[u];
          kq[u & 1] += kk[e + u] * qq[u];
        }
      }
      const float sk = col_sum(ak[0] + ak[1]), sqq = col_sum(aq[0] + aq[1]), skq = col_sum(kq[0] + kq[1]);
      const float delta = (v - g * sk) * beta;
#pragma unroll
      for (int e = 0; e < E; ++e) st[e] = g * st[e] + kk[e] * delta;
      if (p == 0) on[r][j] = g * sqq + delta * skq;
    }
    __syncthreads();
    // (C)
    float o[CH];
    if (tid < DL)
#pragma unroll
      for (int r = 0; r < CH; ++r) {
        o[r] = 0.f;
        if (r >= n) continue;
        o[r] = on[r][tid];
        const float so = wave_sum(o[r] * o[r]);
        if (lane == 0) red[r][wave] = so;
      }
    __syncthreads();
    if (tid < DL)
#pragma unroll
      for (int r = 0; r < CH; ++r) {
        if (r >= n) continue;
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < WPP; ++w) tot += red[r][w];
        const float sc = 1.0f / sqrtf(tot / (float)DL + a.eps);
        float res = (o[r] * sc) * nw;
        res *= zv[r] * sigmoid_f32(zv[r]);
        const int64_t at = (row0 + r) * W + (int64_t)h * DL + tid;
        if (a.out_f32)
          ((float *)a.out)[at] = res;
        else
          ((uint16_t *)a.out)[at] = f32_to_bf16_bits(res);
      }
    __syncthreads();  // the next chunk reuses red, qn .. on
  }
}

// 512 threads; grid B * Hl.
#define RXW8_Q35_SHORT(DL)                                                         \
  extern "C" __global__ void __launch_bounds__(512) rxw8_q35_linear_short_d##DL(Q35ShortMixArgs a) { \
    linear_short<DL>(a);                                                           \
  }
RXW8_Q35_SHORT(64)
RXW8_Q35_SHORT(128)

// ---- F32 LoRA on the tied head (mod.rs:174-195): down = x A^T, then
// logits += (alpha / rank) * down B^T. One thread per output element.
struct Q35LoraArgs {
  const float *x;   // [T, K]
  const float *w;   // [N, K]
  float *y;         // [T, N]
  int64_t T, N, K;
  float alpha;
  int accumulate;   // 0: y = x w^T; 1: y += alpha * (x w^T)
};

extern "C" __global__ void __launch_bounds__(256) rxw8_q35_lora(Q35LoraArgs a) {
  const int64_t n = a.T * a.N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = e / a.N, c = e - t * a.N;
    float acc = 0.f;
    for (int64_t k = 0; k < a.K; ++k) acc += a.x[t * a.K + k] * a.w[c * a.K + k];
    if (a.accumulate)
      a.y[e] += acc * a.alpha;
    else
      a.y[e] = acc;
  }
}

// ---- SwiGLU of separate gate / up projections (layers.rs:270-293):
// act = silu(g) * u with g, u the projection outputs: f32 throughout under F32
// compute, else bf16 inputs and a bf16-rounded result.
struct Q35SiluArgs {
  const void *g, *u;  // [T, I] rows of `stride` elements
  void *act;          // [T, I]
  int64_t n, I, stride;
  int f32;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_q35_silu_mul(Q35SiluArgs a) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < a.n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = e / a.I, c = e - t * a.I;
    const float y = silu_mul_f32(ld(a.g, t * a.stride + c, a.f32), ld(a.u, t * a.stride + c, a.f32));
    if (a.f32)
      ((float *)a.act)[e] = y;
    else
      ((uint16_t *)a.act)[e] = f32_to_bf16_bits(y);
  }
}
