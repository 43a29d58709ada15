// K3: grouped-query decode attention over a contiguous bf16 KV cache.
//
// Semantics (crates/rxla-core/src/attention.rs:83-252, F32 throughout):
//   s_j = (q . k_j) * scale + mask_j,  p = softmax(s),  out = sum_j p_j v_j
// for the keys j < lens[b] of sequence b; query head h reads kv head
// h / (Hq / Hkv) (consecutive heads share a kv head, attention.rs:83-135).
//
// Layout: q [R, Hq, D] f32|bf16 (one query row per decoding sequence, or one
// per prompt token in prefill), caches [Bc, Hkv, Lmax, D] bf16, out
// [R, Hq, D] f32|bf16. Row r reads cache slot row_seq[r] (r when null) and
// sees its first lens[r] keys. One workgroup (8 waves) handles one (row, kv
// head, split); each wave walks tiles of 16 keys (double-buffered in
// registers) with its own online softmax. The G = Hq/Hkv query heads of the kv
// head share every K/V byte the workgroup loads. Splits are uniform per row,
// or, for few long ragged rows, apportioned by length on the device.
//
// QK^T runs on v_mfma_f32_16x16x32_bf16 with K as the A operand (16 keys x
// 32 dims per fragment, 16-byte loads of contiguous K rows) and q^T as the B
// operand. q is f32, so it is split into bf16 hi + lo parts and both are
// contracted (two MFMAs), which keeps the scores at f32 accuracy; K is exactly
// bf16. Softmax statistics are reduced per wave with cross-lane shuffles,
// probabilities go through LDS, and P.V runs on the VALU in f32 with each lane
// owning 8 dims of every fourth key (16-byte V loads, 1 KiB per wave load).
// Waves merge (max, sum, acc) in LDS. With one split the workgroup writes the
// output; otherwise every split writes (max, sum, acc) partials, which are
// merged in split order (deterministic) either by the last workgroup of the
// (row, kv head) to arrive -- device-coherent partial stores and loads around
// an arrival counter make the other splits' partials visible to it -- or,
// without counters, by
// rxw8_gqa_decode_combine in a second launch (the kernel boundary makes the
// partials visible). Both merges run the same code, so they agree bit for bit.
#include "common.h"

struct AttnArgs {
  const void *q;           // [R, Hq, D]
  const uint16_t *kc;      // [Bc, Hkv, Lmax, D] bf16
  const uint16_t *vc;      // [Bc, Hkv, Lmax, D] bf16
  const int32_t *lens;     // [R] visible keys of row r
  const int32_t *row_seq;  // [R] cache slot of row r, or null (slot r)
  const float *mask;       // additive, mask[r * mask_sb + h * mask_sh + j], or null
  void *out;               // [R, Hq, D]
  // split partials, (G, 2 + D) floats per slot: slot bh * max_chunks + split
  // for uniform splits; slot kvh * units + u (one per workgroup) for
  // length-proportional ones
  float *ws;
  int64_t mask_sb, mask_sh;
  int R, Hq, Hkv, Lmax, max_chunks;
  float scale;
  int q_f32, out_f32;
  // Decode steps (one new token per row, at position lens[r] - 1): when qkv
  // is set, q and the new k / v come from the bf16 projection row
  // qkv[r, Hq + 2 Hkv, D] (optional per-head RMSNorm with q_norm / k_norm,
  // then split-half RoPE), and the new k (rounded to bf16) and v are appended
  // to the caches here: the q/k RoPE + KV append kernel folded into this
  // launch.
  const uint16_t *qkv;
  const float *q_norm, *k_norm;  // [D] or null
  const float *rope;             // [Lmax, D] RoPE table: cos then sin per position
  float eps;
  // [R * Hkv] arrival counters (zero between launches), or null: with S > 1
  // splits the last workgroup of a (row, kv head) to finish merges the
  // partials itself; null leaves that to rxw8_gqa_decode_combine.
  int *counters;
  // > 0: length-proportional splits, `units` workgroups per kv head shared by
  // the R rows (row_units); 0: max_chunks splits for every row
  int units;
};

namespace {

constexpr int D = 128;
constexpr int KW = 64;            // split granularity (keys)
constexpr int KT = 16;            // keys per wave tile
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float wave_max4(float v) {
  uint2 p = pair_xor16(v);
  v = fmaxf(__uint_as_float(p.x), __uint_as_float(p.y));
  p = pair_xor32(v);
  return fmaxf(__uint_as_float(p.x), __uint_as_float(p.y));
}
__device__ __forceinline__ float wave_sum4(float v) {
  uint2 p = pair_xor16(v);
  v = __uint_as_float(p.x) + __uint_as_float(p.y);
  p = pair_xor32(v);
  return __uint_as_float(p.x) + __uint_as_float(p.y);
}

// Per-head RMSNorm (when nw is set) and split-half RoPE of one head held by
// the 4 lanes with the same lane & 15, with rope = the RoPE table row of the
// position (cos of the D/2 frequencies, then sin): the lane holds dims
// 32 t + 8 g4 + e (t < 4, e < 8); dims of t = 0, 1 pair with t + 2 (d + 64).
// Same arithmetic as rxw8_dec_qk_rope_kv (ops.rs:929-944, rotary.rs:17-74).
__device__ __forceinline__ void norm_rope_lane(float (&x)[4][8], const float *nw,
                                               const float *rope, float eps, int g4) {
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[t][e] * x[t][e];
  ss = wave_sum4(ss);
  const float sc = nw ? 1.0f / sqrtf(ss / (float)D + eps) : 1.0f;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int i0 = 32 * t + 8 * g4;
    f32x4 cs[2], sn[2], w0[2], w1[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      cs[j] = *(const f32x4 *)(rope + i0 + 4 * j);
      sn[j] = *(const f32x4 *)(rope + D / 2 + i0 + 4 * j);
      if (nw) {
        w0[j] = *(const f32x4 *)(nw + i0 + 4 * j);
        w1[j] = *(const f32x4 *)(nw + D / 2 + i0 + 4 * j);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x0 = x[t][e], x1 = x[t + 2][e];
      if (nw) {
        x0 = (x0 * sc) * w0[e >> 2][e & 3];
        x1 = (x1 * sc) * w1[e >> 2][e & 3];
      }
      const float c = cs[e >> 2][e & 3], s = sn[e >> 2][e & 3];
      x[t][e] = x0 * c - x1 * s;
      x[t + 2][e] = x1 * c + x0 * s;
    }
  }
}

// The rope row's and the norm weights' values norm_rope_lane reads, loaded
// ahead (issued before a K/V tile's loads, the q prologue then waits for
// these alone, not for the tile behind them: vector loads complete in order).
struct RopeRow {
  f32x4 cs[2][2], sn[2][2], w0[2][2], w1[2][2];
};
__device__ __forceinline__ void load_rope_row(RopeRow &r, const float *nw, const float *rope, int g4) {
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = 32 * t + 8 * g4 + 4 * j;
      r.cs[t][j] = *(const f32x4 *)(rope + i);
      r.sn[t][j] = *(const f32x4 *)(rope + D / 2 + i);
      r.w0[t][j] = *(const f32x4 *)(nw + i);
      r.w1[t][j] = *(const f32x4 *)(nw + D / 2 + i);
    }
}
// norm_rope_lane on preloaded values (nw non-null: the norm is applied)
__device__ __forceinline__ void norm_rope_lane(float (&x)[4][8], const RopeRow &r, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[t][e] * x[t][e];
  ss = wave_sum4(ss);
  const float sc = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x0 = (x[t][e] * sc) * r.w0[t][e >> 2][e & 3];
      const float x1 = (x[t + 2][e] * sc) * r.w1[t][e >> 2][e & 3];
      const float c = r.cs[t][e >> 2][e & 3], s = r.sn[t][e >> 2][e & 3];
      x[t][e] = x0 * c - x1 * s;
      x[t + 2][e] = x1 * c + x0 * s;
    }
}

__device__ __forceinline__ void unpack_bf16x8(const u32x4 &r, float *x) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[2 * e] = bf16_bits_to_f32(r[e] & 0xffffu);
    x[2 * e + 1] = bf16_bits_to_f32(r[e] >> 16);
  }
}

// Length-proportional splits: the `units` workgroups of a kv head go to the R
// rows in proportion to their clamped lengths, at least one each: row b owns
// units [u_b, u_{b+1}) with u_0 = 0 and u_{b+1} = clamp(round(C_{b+1} * units
// / T), u_b + 1, units - (R - 1 - b)) (f32), C_b the lengths of rows < b and T their
// total, so every workgroup walks about T / units keys. Returns row b's split
// count; for unit u (>= 0), also the row and the split within it, and the
// row's first unit u_r (unit0). Uniform per workgroup; R < units
// (host-checked).
__device__ __forceinline__ int row_units(const AttnArgs &a, int b, int u, int *row, int *split,
                                         int *row_len = nullptr, int *unit0 = nullptr) {
  int T = 0;  // R * Lmax < 2^31 (host-checked)
  for (int r = 0; r < a.R; ++r) T += min(max(a.lens[r], 1), a.Lmax);
  const float per_key = (float)a.units / (float)T;  // same value in every workgroup
  int C = 0;
  int ub = 0;  // u_r of the current row
  for (int r = 0; r < a.R; ++r) {
    const int len = min(max(a.lens[r], 1), a.Lmax);
    C += len;
    const int ideal = (int)((float)C * per_key + 0.5f);
    const int un = min(max(ub + 1, ideal), a.units - (a.R - 1 - r));  // u_{r+1}
    if ((u >= 0 && u < un) || (u < 0 && r == b)) {
      if (row) *row = r;
      if (split) *split = u - ub;
      if (row_len) *row_len = len;
      if (unit0) *unit0 = ub;
      return un - ub;
    }
    ub = un;
  }
  return 1;
}

// Split partials: device-coherent (write-through, sc1) stores and loads when
// the last-arriving workgroup merges them within the launch, plain ones when
// a second launch does (the kernel boundary then publishes them).
__device__ __forceinline__ void store_part(float *p, float v, bool coherent) {
  if (coherent)
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *p = v;
}
template <bool COH>
__device__ __forceinline__ float load_part(const float *p) {
  if constexpr (COH)
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    return *p;
}

// Merge the S split partials of (row, kv head) bh in split order and write
// the output rows of its G heads; any workgroup size. slot0: the partial slot
// of the row's split 0 (-1: found here). Thread (head, dim):
// M = max_c m_c, then L = sum_c f_c l_c and O = sum_c f_c o_c in split order
// with f_c = exp(m_c - M) (0 for empty splits). Up to 32 splits, all of an
// output's partials are loaded first (one round trip), with the same
// arithmetic order as the general loop (empty slots add exact zeros).
template <int G, bool COH>
__device__ void combine_pair(const AttnArgs &a, int bh, int nchunks = 0, int slot0 = -1) {
  const int b = bh / a.Hkv, kvh = bh - b * a.Hkv;
  // every split of the row wrote a partial (empty: max -inf)
  if (a.units > 0) {
    int u0 = 0;
    const int n = row_units(a, b, -1, nullptr, nullptr, nullptr, &u0);
    if (nchunks == 0) nchunks = n;
    if (slot0 < 0) slot0 = kvh * a.units + u0;
  } else {
    if (nchunks == 0) nchunks = a.max_chunks;
    if (slot0 < 0) slot0 = bh * a.max_chunks;
  }
  if (nchunks == 1) return;  // a single split wrote the output itself
  const float *base = a.ws + (int64_t)slot0 * G * (2 + D);
  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int h = idx / D, d = idx - h * D;
    float M = kNegInf, L = 0.f, O = 0.f;
    // up to NC splits: every partial of this output is loaded before any
    // arithmetic (one round trip); unused slots weigh 0
    auto merge_upto = [&](auto nc) {
      constexpr int NC = decltype(nc)::value;
      float mc[NC], lc[NC], oc[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        mc[c] = kNegInf;
        lc[c] = 0.f;
        oc[c] = 0.f;
        if (c < nchunks) {
          const float *ph = base + ((int64_t)c * G + h) * (2 + D);
          mc[c] = load_part<COH>(ph);
          lc[c] = load_part<COH>(ph + 1);
          oc[c] = load_part<COH>(ph + 2 + d);
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) M = fmaxf(M, mc[c]);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float f = mc[c] == kNegInf ? 0.f : __expf(mc[c] - M);
        L += f * lc[c];
        O += f * oc[c];
      }
    };
    if (nchunks <= 8) {
      merge_upto(std::integral_constant<int, 8>{});
    } else if (nchunks <= 32) {
      merge_upto(std::integral_constant<int, 32>{});
    } else {
      for (int c = 0; c < nchunks; ++c) M = fmaxf(M, load_part<COH>(base + ((int64_t)c * G + h) * (2 + D)));
      for (int c = 0; c < nchunks; ++c) {
        const float *ph = base + ((int64_t)c * G + h) * (2 + D);
        const float mc = load_part<COH>(ph);
        const float f = mc == kNegInf ? 0.f : __expf(mc - M);
        L += f * load_part<COH>(ph + 1);
        O += f * load_part<COH>(ph + 2 + d);
      }
    }
    const float r = O / L;
    const int64_t oi = ((int64_t)b * a.Hq + kvh * G + h) * D + d;
    if (a.out_f32)
      ((float *)a.out)[oi] = r;
    else
      ((uint16_t *)a.out)[oi] = f32_to_bf16_bits(r);
  }
}

// After this workgroup stored its partials (device-coherent stores): wait
// until every thread's stores completed, then count its arrival for (row, kv
// head) bh; the workgroup that brings the count to S merges all S partials
// with device-coherent loads (its increment follows every other split's
// completed stores) and re-arms the counter for the next launch. No
// device-scope fences: on this part a release fence writes back the whole L2
// and costs ~100 us per launch. Uniform per workgroup.
template <int G>
__device__ void arrive_and_merge(const AttnArgs &a, int bh, int nsplit, int slot0) {
  __shared__ int is_last;
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are done
  __syncthreads();
  if (threadIdx.x == 0)
    is_last = __hip_atomic_fetch_add(a.counters + bh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              nsplit - 1;
  __syncthreads();
  if (!is_last) return;
  combine_pair<G, true>(a, bh, nsplit, slot0);
  if (threadIdx.x == 0) __hip_atomic_store(a.counters + bh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Multi-pass variant: one workgroup of NP waves per (row, kv head, split).
// Split s of a row covers keys [s * per, min(len, (s + 1) * per)), per =
// ceil(len / S) rounded up to 64; the workgroup walks it in passes of NP * 64
// keys (wave w takes keys base + 64 w ..), keeping a per-wave online softmax
// (running max, sum and P.V accumulators rescaled by exp(m_old - m_new)) in
// registers across passes. S = 1 writes the output directly; otherwise every
// split writes (max, sum, acc) partials (empty splits: max -inf, sum 0) for
// rxw8_gqa_decode_combine. a.max_chunks carries S.
template <int G, int NP, bool FUSE>
__device__ void attn_pass(const AttnArgs &a) {
  constexpr int GP = (G + 3) / 4 * 4;
  __shared__ float p_lds[NP][KT][GP];
  __shared__ float m_lds[NP][G], l_lds[NP][G];
  __shared__ float o_lds[NP][G][D];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int S = a.max_chunks;  // partial slots per (row, kv head)
  int split, b, kvh, nsplit;
  int len;
  int slot0;  // partial slot of the row's split 0 (this workgroup's: slot0 + split)
  if (a.units > 0) {  // length-proportional splits
    kvh = blockIdx.x / a.units;
    const int u = blockIdx.x - kvh * a.units;
    nsplit = row_units(a, 0, u, &b, &split, &len);
    slot0 = kvh * a.units + u - split;
  } else {
    split = blockIdx.x % S;
    b = (blockIdx.x / S) / a.Hkv;
    kvh = (blockIdx.x / S) - b * a.Hkv;
    nsplit = S;
    len = a.lens[b];
    len = len < 1 ? 1 : (len > a.Lmax ? a.Lmax : len);
    slot0 = (b * a.Hkv + kvh) * S;
  }
  const int bh = b * a.Hkv + kvh;  // row * Hkv + kvh
  const int per = ((len + nsplit - 1) / nsplit + KW - 1) / KW * KW;
  const int start = split * per;
  int end = min(len, start + per);
  float *part = a.ws + ((int64_t)(slot0 + split) * G) * (2 + D);
  if (start >= end) {  // empty split (uniform per workgroup)
    for (int idx = threadIdx.x; idx < G * (2 + D); idx += blockDim.x)
      store_part(part + idx, (idx % (2 + D)) == 0 ? kNegInf : 0.f, a.counters != nullptr);
    if (a.counters) arrive_and_merge<G>(a, bh, nsplit, slot0);
    return;
  }
  const int seq = a.row_seq ? a.row_seq[b] : b;
  const int64_t row_base = ((int64_t)seq * a.Hkv + kvh) * a.Lmax;
  const int col = lane & 15, g4 = lane >> 4;

  // raw q (B operand source): lane (head = col, dgroup = g4), 8 dims per step
  u32x4 qraw[4][2];
  // Fused decode step: the row's new token sits at position pnew = len - 1.
  // q is its raw bf16 projection (norm + RoPE applied below, after the first
  // K/V loads are in flight). The split holding key pnew walks only keys
  // [start, pnew) and its wave 0 adds the new key (raw k / v staged in LDS)
  // as a last online-softmax step, then appends it to the caches.
  __shared__ u32x4 new_kv[32];  // raw bf16 k row (16 x 16 B), then v row
  const uint16_t *src = nullptr;
  const int pnew = len - 1;
  const bool own_new = FUSE && end == len;  // uniform
  if (own_new) end = pnew;
  if constexpr (FUSE) {
    src = a.qkv + (int64_t)b * (a.Hq + 2 * a.Hkv) * D;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      qraw[t][0] = *(const u32x4 *)(src + (kvh * G + (col < G ? col : 0)) * D + 32 * t + 8 * g4);
      qraw[t][1] = u32x4{0, 0, 0, 0};
    }
  } else {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t off = ((int64_t)b * a.Hq + kvh * G + (col < G ? col : 0)) * D + 32 * t + 8 * g4;
    if (a.q_f32) {
      const u32x4 *p = (const u32x4 *)((const float *)a.q + off);
      qraw[t][0] = p[0];
      qraw[t][1] = p[1];
    } else {
      qraw[t][0] = *(const u32x4 *)((const uint16_t *)a.q + off);
      qraw[t][1] = u32x4{0, 0, 0, 0};
    }
  }
  }
  // Tiles of KT = 16 keys per wave, double-buffered in registers: the loads of
  // tile n+1 are in flight while tile n is scored and accumulated, so every
  // wave keeps K and V streaming (a 64-key tile loaded and then consumed left
  // the memory idle during each pass's compute; a 32-key pair of tiles spills).
  // Wave w takes the tiles at first + 16 w + 128 n. K fragments (A operand):
  // lane (key = col, dgroup = g4); V rows: lane (kq = g4, dgroup = col) takes
  // keys 4 * it + kq, dims 8 col .. +7.
  struct Tile {
    u32x4 k[4], v[4];
  };
  auto load = [&](Tile &T, int j0) {
    {
      const int key = j0 + col;
      const bool valid = key < end;
      const uint16_t *krow = a.kc + (row_base + (valid ? key : 0)) * D + 8 * g4;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        T.k[t] = valid ? __builtin_nontemporal_load((const u32x4 *)(krow + 32 * t)) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int key = j0 + 4 * it + g4;
      T.v[it] = key < end ? __builtin_nontemporal_load(
                                (const u32x4 *)(a.vc + (row_base + key) * D + 8 * col))
                          : u32x4{0, 0, 0, 0};
    }
  };
  const int first = start + wave * KT;
  constexpr int kStep = NP * KT;
  Tile ta, tb;
  // The first tile is in flight during the q prologue; the q norm weights and
  // the RoPE row go out before it (with a q norm; without one the plain
  // form below reads them after the tile)
  RopeRow rrow;
  const bool pre_rope = FUSE && a.q_norm != nullptr;  // uniform
  if (pre_rope) load_rope_row(rrow, a.q_norm, a.rope + (int64_t)pnew * D, g4);
  load(ta, first);
  float m_run = kNegInf, l_run = 0.f;  // per lane: head col (all g4 lanes agree)
  float o[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.f;

  // fused: q norm + RoPE up front (q then holds f32 bits)
  if constexpr (FUSE) {
    float qv[4][8];
#pragma unroll
    for (int t = 0; t < 4; ++t) unpack_bf16x8(qraw[t][0], qv[t]);
    if (pre_rope)
      norm_rope_lane(qv, rrow, a.eps);
    else
      norm_rope_lane(qv, a.q_norm, a.rope + (int64_t)pnew * D, a.eps, g4);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qraw[t][0][e] = __float_as_uint(qv[t][e]);
        qraw[t][1][e] = __float_as_uint(qv[t][4 + e]);
      }
  }
  // raw new k (lanes 0-15) and v (lanes 16-31) rows, 16 B per lane; staged
  // in LDS after the blocks so the load never stalls them
  u32x4 stage = {0, 0, 0, 0};
  if (own_new && wave == 0 && lane < 32)
    stage = *(const u32x4 *)(src + (lane < 16 ? (a.Hq + kvh) * D + 8 * lane
                                              : (a.Hq + a.Hkv + kvh) * D + 8 * (lane - 16)));
  // q -> bf16 hi + lo (B operand), once
  u32x4 qhi[4], qlo[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
      float qv[8];
      if (col < G) {
        if (FUSE || a.q_f32) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            qv[e] = __uint_as_float(qraw[t][0][e]);
            qv[4 + e] = __uint_as_float(qraw[t][1][e]);
          }
        } else {
          unpack_bf16x8(qraw[t][0], qv);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float h0 = round_bf16(qv[2 * e]), h1 = round_bf16(qv[2 * e + 1]);
        qhi[t][e] = pack_bf16x2(h0, h1);
        qlo[t][e] = pack_bf16x2(qv[2 * e] - h0, qv[2 * e + 1] - h1);
      }
  }
  // One online-softmax step over the tile at j0 (keys >= end score -inf and
  // carry zero V rows).
  auto consume = [&](const Tile &T, int j0) {
    float s[4];
    {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc = mfma16x16x32(as_bf16x8(T.k[t]), as_bf16x8(qhi[t]), acc);
        acc = mfma16x16x32(as_bf16x8(T.k[t]), as_bf16x8(qlo[t]), acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = j0 + 4 * g4 + i;
        float v = kNegInf;
        if (key < end) {
          v = acc[i] * a.scale;
          if (a.mask && col < G)
            v += a.mask[(int64_t)b * a.mask_sb + (int64_t)(kvh * G + col) * a.mask_sh + key];
        }
        s[i] = v;
      }
    }
    float m_blk = kNegInf;
#pragma unroll
    for (int i = 0; i < 4; ++i) m_blk = fmaxf(m_blk, s[i]);
    m_blk = wave_max4(m_blk);
    const float m_new = fmaxf(m_run, m_blk);
    const bool any = m_new != kNegInf;
    const float f_old = (m_run == kNegInf) ? 0.f : __expf(m_run - m_new);
    float l_blk = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = any ? __expf(s[i] - m_new) : 0.f;
      s[i] = e;
      l_blk += e;
    }
    l_blk = wave_sum4(l_blk);
    l_run = l_run * f_old + l_blk;
    m_run = m_new;
    if (col < G)
#pragma unroll
      for (int i = 0; i < 4; ++i) p_lds[wave][4 * g4 + i][col] = s[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // rescale the running P.V of head h by head h's factor (held by lane h;
    // v_readlane, no LDS round trip)
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float fh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f_old), h));
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] *= fh;
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = bf16_bits_to_f32(T.v[it][e] & 0xffffu);
        v[2 * e + 1] = bf16_bits_to_f32(T.v[it][e] >> 16);
      }
      const float *prow = p_lds[wave][4 * it + g4];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float p = prow[h];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] += p * v[e];
      }
    }
    // p_lds[wave] is rewritten next tile only after every lane read it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // A/B register sets: issue B, consume A, issue A', consume B. Loads past
  // the split are masked per lane (no memory access); a B tile past the end
  // is not consumed (uniform per wave).
  for (int j0 = first; j0 < end; j0 += 2 * kStep) {
    load(tb, j0 + kStep);
    consume(ta, j0);
    load(ta, j0 + 2 * kStep);
    if (j0 + kStep < end) consume(tb, j0 + kStep);
  }
  if (own_new && wave == 0) {
    // the new key: k = bf16(RoPE(norm(raw k))), scored against q in f32, one
    // online-softmax step, then append k, v
    if (lane < 32) new_kv[lane] = stage;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float x[4][8];
#pragma unroll
    for (int t = 0; t < 4; ++t) unpack_bf16x8(new_kv[4 * t + g4], x[t]);
    norm_rope_lane(x, a.k_norm, a.rope + (int64_t)pnew * D, a.eps, g4);
    u32x4 kb[4];
    float dot = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kb[t][e] = pack_bf16x2(x[t][2 * e], x[t][2 * e + 1]);
        const float k0 = bf16_bits_to_f32(kb[t][e] & 0xffffu), k1 = bf16_bits_to_f32(kb[t][e] >> 16);
        const float q0 = __uint_as_float(qraw[t][e >> 1][2 * (e & 1)]);
        const float q1 = __uint_as_float(qraw[t][e >> 1][2 * (e & 1) + 1]);
        dot += q0 * k0 + q1 * k1;
      }
    dot = wave_sum4(dot);
    float sc = dot * a.scale;
    if (a.mask && col < G)
      sc += a.mask[(int64_t)b * a.mask_sb + (int64_t)(kvh * G + col) * a.mask_sh + pnew];
    const float m_new = fmaxf(m_run, sc);
    const float f_old = m_run == kNegInf ? 0.f : __expf(m_run - m_new);
    const float pe = m_new == kNegInf ? 0.f : __expf(sc - m_new);
    l_run = l_run * f_old + pe;
    m_run = m_new;
    float v[8];
    const u32x4 vraw = new_kv[16 + col];
    unpack_bf16x8(vraw, v);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float fh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f_old), h));
      const float ph = g4 == 0 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe), h)) : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = o[h][e] * fh + ph * v[e];
    }
    uint16_t *kd = (uint16_t *)a.kc + (row_base + pnew) * D;
    uint16_t *vd = (uint16_t *)a.vc + (row_base + pnew) * D;
    if (col == 0)
#pragma unroll
      for (int t = 0; t < 4; ++t) *(u32x4 *)(kd + 32 * t + 8 * g4) = kb[t];
    if (g4 == 0) *(u32x4 *)(vd + 8 * col) = vraw;
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = wave_sum4(o[h][e]);
  if (col < G && g4 == 0) {
    m_lds[wave][col] = m_run;
    l_lds[wave][col] = l_run;
  }
  if (g4 == 0)
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) o_lds[wave][h][8 * col + e] = o[h][e];
  __syncthreads();

  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int h = idx / D, d = idx - h * D;
    float M = kNegInf;
    for (int w = 0; w < NP; ++w) M = fmaxf(M, m_lds[w][h]);
    float L = 0.f, O = 0.f;
    for (int w = 0; w < NP; ++w) {
      const float mw = m_lds[w][h];
      const float f = mw == kNegInf ? 0.f : __expf(mw - M);
      L += f * l_lds[w][h];
      O += f * o_lds[w][h][d];
    }
    if (nsplit == 1) {
      const float r = O / L;
      const int64_t oi = ((int64_t)b * a.Hq + kvh * G + h) * D + d;
      if (a.out_f32)
        ((float *)a.out)[oi] = r;
      else
        ((uint16_t *)a.out)[oi] = f32_to_bf16_bits(r);
    } else {
      float *ph = part + h * (2 + D);
      const bool coh = a.counters != nullptr;
      if (d == 0) {
        store_part(ph, M, coh);
        store_part(ph + 1, L, coh);
      }
      store_part(ph + 2 + d, O, coh);
    }
  }
  if (nsplit > 1 && a.counters) arrive_and_merge<G>(a, bh, nsplit, slot0);
}

}  // namespace

// NP = 8 waves per workgroup (512 threads) for G <= 4. G = 8 holds 64 f32
// P.V accumulators per lane: at 8 waves (2 per SIMD, at most 256 registers)
// it spilled 116 / 276 bytes per lane to scratch, so it runs 4 waves (256
// threads, one per SIMD), which keeps the overflow in AGPRs: 78.0 -> 60.2 us
// for B 8, 64 / 8 heads, lengths 512-8192.
#define RXW8_ATTN_NP(G) ((G) == 8 ? 4 : 8)
#define RXW8_ATTN(G)                                                                 \
  extern "C" __global__ void __launch_bounds__(RXW8_ATTN_NP(G) * 64)                 \
      rxw8_gqa_decode_d128_g##G(AttnArgs a) {                                        \
    attn_pass<G, RXW8_ATTN_NP(G), false>(a);                                         \
  }                                                                                  \
  extern "C" __global__ void __launch_bounds__(RXW8_ATTN_NP(G) * 64)                 \
      rxw8_gqa_decode_rope_d128_g##G(AttnArgs a) {                                   \
    attn_pass<G, RXW8_ATTN_NP(G), true>(a);                                          \
  }                                                                                  \
  extern "C" __global__ void __launch_bounds__(256)                                  \
      rxw8_gqa_decode_combine_d128_g##G(AttnArgs a) {                                \
    combine_pair<G, false>(a, blockIdx.x);                                           \
  }
RXW8_ATTN(1)
RXW8_ATTN(2)
RXW8_ATTN(4)
RXW8_ATTN(8)

// ---- causal prefill attention (flash-style): S query rows per sequence ----
//
// Query row i of sequence b sits at position starts[b] + i and sees keys
// 0 .. starts[b] + i of its cache slot (the causal mask key_pos <= q_pos,
// attention.rs:14-32, over the grouped heads of attention.rs:83-135). One
// workgroup (4 waves) takes 64 consecutive query rows of one (sequence, kv
// head) and the G query heads sharing it; wave w owns rows 16 w .. 16 w + 15.
// Keys go by in blocks of 64, staged once per workgroup in LDS: K row-major
// with 16-byte chunks XOR-swizzled by row (conflict-free fragment reads), V
// transposed (V^T rows of 64 keys) so P.V can read its MFMA operand along
// keys. Per wave and head:
//   S^T = K Q^T   on v_mfma_f32_16x16x32_bf16 (A = K from LDS, B = q split
//                 into bf16 hi + lo parts, so the scores keep f32 accuracy),
//   online softmax per query row (lane & 15 = row; the 4 lanes of a row hold
//                 16 keys each and reduce with two shuffles),
//   O^T += V^T P^T  (A = V^T from LDS, B = P rounded to bf16 straight from
//                 the score registers: lane (row, g) holds keys 4g..4g+3 of two
//                 16-key tiles, and the V^T operand is read in that key order).
// Blocks past a wave's last visible key are skipped; the last row block of a
// ragged S computes clamped rows and stores only the valid ones. Workgroups
// are ordered longest-first (late row blocks see the most keys).
struct PrefillArgs {
  const void *q;            // element (b, i, h, d) at b*q_sb + i*q_ss + h*q_sh + d
  const uint16_t *kc, *vc;  // [Bc, Hkv, Lmax, D] bf16
  const int32_t *starts;    // [B] position of row 0 of sequence b
  const int32_t *slots;     // [B] cache slot of sequence b, or null (slot b)
  void *out;                // element (b, i, h, d) at b*o_sb + i*o_ss + h*o_sh + d
  int64_t q_sb, q_ss, q_sh, o_sb, o_ss, o_sh;
  int B, S, Hq, Hkv, Lmax, nqb;
  float scale;
  int q_f32, out_f32;
};

namespace {

constexpr int PKB = 64;        // keys per block
// V^T row pitch (elements): 144 B. A 4-key (8-byte) write per (d, key group)
// puts 16 key groups of one d row in 128 contiguous bytes and the next d row
// 32 banks further, so a half-wave of writes is conflict-free.
constexpr int VROW = PKB + 8;
// LDS bytes: K and V^T blocks, double-buffered
constexpr int PREFILL_LDS = 2 * (PKB * D + D * VROW) * 2;

template <int G>
__device__ void attn_prefill(const PrefillArgs &a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t pf_lds[];  // [2][K block | V^T block]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, g4 = lane >> 4;
  const int per_qb = a.B * a.Hkv;
  const int qb = a.nqb - 1 - (int)(blockIdx.x / per_qb);
  const int rem = blockIdx.x - (a.nqb - 1 - qb) * per_qb;
  const int b = rem / a.Hkv, kvh = rem - (rem / a.Hkv) * a.Hkv;
  int start = a.starts[b];  // clamped so rows sit in [0, Lmax) (host: S <= Lmax)
  start = start < 0 ? 0 : (start > a.Lmax - a.S ? a.Lmax - a.S : start);
  const int slot = a.slots ? a.slots[b] : b;
  const int64_t kv_base = ((int64_t)slot * a.Hkv + kvh) * a.Lmax * D;
  const int i0 = qb * 64 + wave * 16;
  const int kv_end = min(start + min(a.S, qb * 64 + 64), a.Lmax);  // keys the workgroup reads
  const int nblk = (kv_end + PKB - 1) / PKB;
  const int my_i = min(i0 + col, a.S - 1);
  const int my_pos = start + my_i;  // last visible key of this lane's row
  const int wave_last = start + min(i0 + 15, a.S - 1);

  // q^T fragments: lane (row col, dims 32 t + 8 g4 ..), bf16 hi + lo
  u32x4 qhi[G][4], qlo[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int64_t off = (int64_t)b * a.q_sb + (int64_t)my_i * a.q_ss +
                          (int64_t)(kvh * G + h) * a.q_sh + 32 * t + 8 * g4;
      float v[8];
      if (a.q_f32) {
        const f32x4 lo = *(const f32x4 *)((const float *)a.q + off);
        const f32x4 hi = *(const f32x4 *)((const float *)a.q + off + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = lo[e];
          v[4 + e] = hi[e];
        }
      } else {
        unpack_bf16x8(*(const u32x4 *)((const uint16_t *)a.q + off), v);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float h0 = round_bf16(v[2 * e]), h1 = round_bf16(v[2 * e + 1]);
        qhi[h][t][e] = pack_bf16x2(h0, h1);
        qlo[h][t][e] = pack_bf16x2(v[2 * e] - h0, v[2 * e + 1] - h1);
      }
    }

  f32x4 o[G][8];
  float m_run[G], l_run[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m_run[h] = kNegInf;
    l_run[h] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[h][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // block staging. K: thread chunk q = tid + 256 u is (key q / 16, 16-byte
  // chunk q % 16). V: thread t holds keys 4 (t % 16) .. + 3 of the 8 dims of
  // chunk t / 16, written as one 8-byte V^T entry (4 keys) per dim.
  u32x4 kreg[4], vreg[4];
  auto gload = [&](int blk) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int qc = threadIdx.x + 256 * u;
      const int key = blk * PKB + (qc >> 4);
      const bool ok = key < kv_end;
      kreg[u] = ok ? *(const u32x4 *)(a.kc + kv_base + (int64_t)key * D + (qc & 15) * 8)
                   : u32x4{0, 0, 0, 0};
      const int vkey = blk * PKB + 4 * (threadIdx.x & 15) + u;
      vreg[u] = vkey < kv_end
                    ? *(const u32x4 *)(a.vc + kv_base + (int64_t)vkey * D + (threadIdx.x >> 4) * 8)
                    : u32x4{0, 0, 0, 0};
    }
  };
  auto lds_store = [&](int buf) {
    uint16_t *ks_lds = pf_lds + buf * (PKB * D + D * VROW);
    uint16_t *vt_lds = ks_lds + PKB * D;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int qc = threadIdx.x + 256 * u;
      const int r = qc >> 4, c = qc & 15;
      *(u32x4 *)(ks_lds + r * D + ((c ^ (r & 15)) << 3)) = kreg[u];
    }
    const int c = threadIdx.x >> 4, k4 = 4 * (threadIdx.x & 15);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int sh = 16 * (e & 1);
      const uint32_t k0 = (vreg[0][e >> 1] >> sh) & 0xffffu, k1 = (vreg[1][e >> 1] >> sh) & 0xffffu;
      const uint32_t k2 = (vreg[2][e >> 1] >> sh) & 0xffffu, k3 = (vreg[3][e >> 1] >> sh) & 0xffffu;
      *(uint2 *)(vt_lds + (8 * c + e) * VROW + k4) = uint2{k0 | (k1 << 16), k2 | (k3 << 16)};
    }
  };

  gload(0);
  lds_store(0);
  __syncthreads();
  for (int blk = 0; blk < nblk; ++blk) {
    const int buf = blk & 1;
    const uint16_t *ks_lds = pf_lds + buf * (PKB * D + D * VROW);
    const uint16_t *vt_lds = ks_lds + PKB * D;
    if (blk + 1 < nblk) gload(blk + 1);  // in flight while this block is used
    const int j0 = blk * PKB;
    if (j0 <= wave_last) {  // wave-uniform: else every key of the block is in this wave's future
    // S^T tiles: s[h][kt] lane (key j0 + 16 kt + 4 g4 + i, row col)
    f32x4 s[G][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const int r = kt * 16 + col;
      u32x4 kf[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) kf[t] = *(const u32x4 *)(ks_lds + r * D + (((4 * t + g4) ^ col) << 3));
#pragma unroll
      for (int h = 0; h < G; ++h) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          acc = mfma16x16x32(as_bf16x8(kf[t]), as_bf16x8(qhi[h][t]), acc);
          acc = mfma16x16x32(as_bf16x8(kf[t]), as_bf16x8(qlo[h][t]), acc);
        }
        s[h][kt] = acc;
      }
    }
    u32x4 pb[G][2];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mb = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = j0 + 16 * kt + 4 * g4 + i;
          const float v = key <= my_pos ? s[h][kt][i] * a.scale : kNegInf;
          s[h][kt][i] = v;
          mb = fmaxf(mb, v);
        }
      mb = wave_max4(mb);
      // key 0 is visible to every row and block 0 is never skipped, so m_new
      // is finite from the first block on
      const float m_new = fmaxf(m_run[h], mb);
      const float f = m_run[h] == kNegInf ? 0.f : __expf(m_run[h] - m_new);
      float ls = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = __expf(s[h][kt][i] - m_new);
          s[h][kt][i] = e;
          ls += e;
        }
      l_run[h] = l_run[h] * f + wave_sum4(ls);
      m_run[h] = m_new;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[h][dt] *= f;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        pb[h][ks] = u32x4{pack_bf16x2(s[h][2 * ks][0], s[h][2 * ks][1]),
                          pack_bf16x2(s[h][2 * ks][2], s[h][2 * ks][3]),
                          pack_bf16x2(s[h][2 * ks + 1][0], s[h][2 * ks + 1][1]),
                          pack_bf16x2(s[h][2 * ks + 1][2], s[h][2 * ks + 1][3])};
    }
    // O^T += V^T P^T: the V^T operand in the key order of pb
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint16_t *vrow = vt_lds + (dt * 16 + col) * VROW + 32 * ks + 4 * g4;
        const uint2 lo = *(const uint2 *)vrow, hi = *(const uint2 *)(vrow + 16);
        const u32x4 va = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int h = 0; h < G; ++h) o[h][dt] = mfma16x16x32(as_bf16x8(va), as_bf16x8(pb[h][ks]), o[h][dt]);
      }
    }
    // the other buffer was last read in the previous block, before the barrier
    if (blk + 1 < nblk) lds_store(buf ^ 1);
    __syncthreads();
  }
  if (i0 + col >= a.S) return;
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float inv = 1.0f / l_run[h];
    const int64_t ob = (int64_t)b * a.o_sb + (int64_t)(i0 + col) * a.o_ss + (int64_t)(kvh * G + h) * a.o_sh;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f32x4 r = o[h][dt] * inv;
      const int64_t oi = ob + dt * 16 + 4 * g4;
      if (a.out_f32)
        *(f32x4 *)((float *)a.out + oi) = r;
      else
        *(uint2 *)((uint16_t *)a.out + oi) = uint2{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])};
    }
  }
}

}  // namespace

// One head per wave: a workgroup of 4 G waves takes 64 query rows of one
// (sequence, kv head); wave w computes query head kvh * G + w / 4 for rows
// 16 (w % 4) .. + 15. The K and V^T blocks staged in LDS serve the waves of
// all G heads, while a wave's registers hold one head (q hi + lo, O, softmax
// state): twice the waves of attn_prefill per CU hide the LDS, softmax and
// load latencies between MFMAs. Same arithmetic per (row, head) as
// attn_prefill, so the outputs agree bit for bit.
template <int G>
__device__ void attn_prefill_wh(const PrefillArgs &a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t pf_lds[];  // [2][K block | V^T block]
  constexpr int NT = 256 * G;
  constexpr int KU = 4 / G;  // 16-byte K chunks per thread per block
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, g4 = lane >> 4;
  const int head = wave >> 2, rg = wave & 3;
  const int per_qb = a.B * a.Hkv;
  const int qb = a.nqb - 1 - (int)(blockIdx.x / per_qb);
  const int rem = blockIdx.x - (a.nqb - 1 - qb) * per_qb;
  const int b = rem / a.Hkv, kvh = rem - (rem / a.Hkv) * a.Hkv;
  int start = a.starts[b];  // clamped so rows sit in [0, Lmax) (host: S <= Lmax)
  start = start < 0 ? 0 : (start > a.Lmax - a.S ? a.Lmax - a.S : start);
  const int slot = a.slots ? a.slots[b] : b;
  const int64_t kv_base = ((int64_t)slot * a.Hkv + kvh) * a.Lmax * D;
  const int i0 = qb * 64 + rg * 16;
  const int kv_end = min(start + min(a.S, qb * 64 + 64), a.Lmax);  // keys the workgroup reads
  const int nblk = (kv_end + PKB - 1) / PKB;
  const int my_i = min(i0 + col, a.S - 1);
  const int my_pos = start + my_i;  // last visible key of this lane's row
  const int wave_last = start + min(i0 + 15, a.S - 1);
  const int hq = kvh * G + head;

  // q^T fragments: lane (row col, dims 32 t + 8 g4 ..), bf16 hi + lo
  u32x4 qhi[4], qlo[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t off = (int64_t)b * a.q_sb + (int64_t)my_i * a.q_ss + (int64_t)hq * a.q_sh + 32 * t + 8 * g4;
    float v[8];
    if (a.q_f32) {
      const f32x4 lo = *(const f32x4 *)((const float *)a.q + off);
      const f32x4 hi = *(const f32x4 *)((const float *)a.q + off + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = lo[e];
        v[4 + e] = hi[e];
      }
    } else {
      unpack_bf16x8(*(const u32x4 *)((const uint16_t *)a.q + off), v);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float h0 = round_bf16(v[2 * e]), h1 = round_bf16(v[2 * e + 1]);
      qhi[t][e] = pack_bf16x2(h0, h1);
      qlo[t][e] = pack_bf16x2(v[2 * e] - h0, v[2 * e + 1] - h1);
    }
  }

  f32x4 o[8];
  float m_run = kNegInf, l_run = 0.f;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // block staging. K: thread chunk q = tid + NT u is (key q / 16, 16-byte
  // chunk q % 16). V (threads < 256): thread t holds keys 4 (t % 16) .. + 3 of
  // the 8 dims of chunk t / 16, written as one 8-byte V^T entry (4 keys) per dim.
  u32x4 kreg[KU], vreg[4];
  const bool vthread = threadIdx.x < 256;
  auto gload = [&](int blk) {
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int qc = threadIdx.x + NT * u;
      const int key = blk * PKB + (qc >> 4);
      kreg[u] = key < kv_end ? *(const u32x4 *)(a.kc + kv_base + (int64_t)key * D + (qc & 15) * 8)
                             : u32x4{0, 0, 0, 0};
    }
    if (vthread)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int vkey = blk * PKB + 4 * (threadIdx.x & 15) + u;
        vreg[u] = vkey < kv_end
                      ? *(const u32x4 *)(a.vc + kv_base + (int64_t)vkey * D + (threadIdx.x >> 4) * 8)
                      : u32x4{0, 0, 0, 0};
      }
  };
  auto lds_store = [&](int buf) {
    uint16_t *ks_lds = pf_lds + buf * (PKB * D + D * VROW);
    uint16_t *vt_lds = ks_lds + PKB * D;
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int qc = threadIdx.x + NT * u;
      const int r = qc >> 4, c = qc & 15;
      *(u32x4 *)(ks_lds + r * D + ((c ^ (r & 15)) << 3)) = kreg[u];
    }
    if (vthread) {
      const int c = threadIdx.x >> 4, k4 = 4 * (threadIdx.x & 15);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int sh = 16 * (e & 1);
        const uint32_t k0 = (vreg[0][e >> 1] >> sh) & 0xffffu, k1 = (vreg[1][e >> 1] >> sh) & 0xffffu;
        const uint32_t k2 = (vreg[2][e >> 1] >> sh) & 0xffffu, k3 = (vreg[3][e >> 1] >> sh) & 0xffffu;
        *(uint2 *)(vt_lds + (8 * c + e) * VROW + k4) = uint2{k0 | (k1 << 16), k2 | (k3 << 16)};
      }
    }
  };

  gload(0);
  lds_store(0);
  __syncthreads();
  for (int blk = 0; blk < nblk; ++blk) {
    const int buf = blk & 1;
    const uint16_t *ks_lds = pf_lds + buf * (PKB * D + D * VROW);
    const uint16_t *vt_lds = ks_lds + PKB * D;
    if (blk + 1 < nblk) gload(blk + 1);  // in flight while this block is used
    const int j0 = blk * PKB;
    if (j0 <= wave_last) {  // wave-uniform: else every key of the block is in this wave's future
      // S^T tiles: s[kt] lane (key j0 + 16 kt + 4 g4 + i, row col)
      f32x4 s[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const int r = kt * 16 + col;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4 kf = *(const u32x4 *)(ks_lds + r * D + (((4 * t + g4) ^ col) << 3));
          acc = mfma16x16x32(as_bf16x8(kf), as_bf16x8(qhi[t]), acc);
          acc = mfma16x16x32(as_bf16x8(kf), as_bf16x8(qlo[t]), acc);
        }
        s[kt] = acc;
      }
      float mb = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = j0 + 16 * kt + 4 * g4 + i;
          const float v = key <= my_pos ? s[kt][i] * a.scale : kNegInf;
          s[kt][i] = v;
          mb = fmaxf(mb, v);
        }
      mb = wave_max4(mb);
      // key 0 is visible to every row and block 0 is never skipped, so m_new
      // is finite from the first block on
      const float m_new = fmaxf(m_run, mb);
      const float f = m_run == kNegInf ? 0.f : __expf(m_run - m_new);
      float ls = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = __expf(s[kt][i] - m_new);
          s[kt][i] = e;
          ls += e;
        }
      l_run = l_run * f + wave_sum4(ls);
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt] *= f;
      u32x4 pb[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        pb[ks] = u32x4{pack_bf16x2(s[2 * ks][0], s[2 * ks][1]), pack_bf16x2(s[2 * ks][2], s[2 * ks][3]),
                       pack_bf16x2(s[2 * ks + 1][0], s[2 * ks + 1][1]),
                       pack_bf16x2(s[2 * ks + 1][2], s[2 * ks + 1][3])};
      // O^T += V^T P^T: the V^T operand in the key order of pb
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const uint16_t *vrow = vt_lds + (dt * 16 + col) * VROW + 32 * ks + 4 * g4;
          const uint2 lo = *(const uint2 *)vrow, hi = *(const uint2 *)(vrow + 16);
          const u32x4 va = {lo.x, lo.y, hi.x, hi.y};
          o[dt] = mfma16x16x32(as_bf16x8(va), as_bf16x8(pb[ks]), o[dt]);
        }
    }
    // the other buffer was last read in the previous block, before the barrier
    if (blk + 1 < nblk) lds_store(buf ^ 1);
    __syncthreads();
  }
  if (i0 + col >= a.S) return;
  const float inv = 1.0f / l_run;
  const int64_t ob = (int64_t)b * a.o_sb + (int64_t)(i0 + col) * a.o_ss + (int64_t)hq * a.o_sh;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    const f32x4 r = o[dt] * inv;
    const int64_t oi = ob + dt * 16 + 4 * g4;
    if (a.out_f32)
      *(f32x4 *)((float *)a.out + oi) = r;
    else
      *(uint2 *)((uint16_t *)a.out + oi) = uint2{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])};
  }
}

typedef __attribute__((address_space(3))) void lds_void;

// One LDS DMA instruction of the wave: lane l copies 16 bytes from g (its own
// address) to LDS at l_base + 16 l (l_base wave-uniform); completion is
// counted by vmcnt.
__device__ __forceinline__ void lds_dma16(const void *g, void *l_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_void *)l_base, 16, 0, 0);
}

// The same copy from inline asm, base + voff (base wave-uniform in SGPRs, byte
// offset per lane) into LDS at lds + 16 l: the compiler then does not answer
// LDS reads of the other buffer with waits on the copy (the caller waits
// before the barrier that publishes it).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16_asm(const void *base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, %2"
               :: "v"(voff), "s"(lds), "s"(base) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_u32(const uint16_t *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t *)p;
}

// R row tiles per wave: as attn_prefill_wh, but wave w owns rows
// 16 R (w % 4) .. + 16 R - 1 of a workgroup's 64 R query rows, as R 16-row
// tiles of one head. Every K and V^T fragment read from LDS then feeds R
// tiles' MFMAs (the LDS reads per block per wave stay 32 KiB, the matrix work
// grows R-fold), and each staged K/V block serves 64 R rows. Same arithmetic
// per (row, head) as attn_prefill.
template <int G, int R>
__device__ void attn_prefill_rt(const PrefillArgs &a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t pf_lds[];  // [2][K block] [2][V block]
  constexpr int QROWS = 64 * R;   // query rows per workgroup
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, g4 = lane >> 4;
  // HW = min(G, 2) query heads per workgroup (4 HW waves): G = 4 runs two
  // workgroups per (sequence, kv head, query block), heads 2 hp and 2 hp + 1
  constexpr int HW = G < 2 ? G : 2, HP = G / HW;
  const int head = wave >> 2, rg = wave & 3;
  const int per_qb = a.B * a.Hkv * HP;
  const int qb = a.nqb - 1 - (int)(blockIdx.x / per_qb);
  const int rem3 = blockIdx.x - (a.nqb - 1 - qb) * per_qb;
  const int hp = HP > 1 ? rem3 % HP : 0, rem = HP > 1 ? rem3 / HP : rem3;
  const int b = rem / a.Hkv, kvh = rem - (rem / a.Hkv) * a.Hkv;
  int start = a.starts[b];  // clamped so rows sit in [0, Lmax) (host: S <= Lmax)
  start = start < 0 ? 0 : (start > a.Lmax - a.S ? a.Lmax - a.S : start);
  const int slot = a.slots ? a.slots[b] : b;
  const int64_t kv_base = ((int64_t)slot * a.Hkv + kvh) * a.Lmax * D;
  const int i0 = qb * QROWS + rg * 16 * R;  // the wave's first row
  const int kv_end = min(start + min(a.S, qb * QROWS + QROWS), a.Lmax);  // keys the workgroup reads
  const int nblk = (kv_end + PKB - 1) / PKB;
  int my_pos[R];  // last visible key of this lane's row in tile r
#pragma unroll
  for (int r = 0; r < R; ++r) my_pos[r] = start + min(i0 + 16 * r + col, a.S - 1);
  const int wave_last = start + min(i0 + 16 * R - 1, a.S - 1);
  const int hq = kvh * G + hp * HW + head;
  const float c_exp = a.scale * 1.4426950408889634f;  // scale * log2(e)

  // q^T fragments: lane (row col of tile r, dims 32 t + 8 g4 ..), bf16 hi + lo
  // of c q in f32, so the scores come out as c s (c = scale * log2(e))
  u32x4 qhi[R][4], qlo[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int my_i = min(i0 + 16 * r + col, a.S - 1);
      const int64_t off = (int64_t)b * a.q_sb + (int64_t)my_i * a.q_ss + (int64_t)hq * a.q_sh + 32 * t + 8 * g4;
      float v[8];
      if (a.q_f32) {
        const f32x4 lo = *(const f32x4 *)((const float *)a.q + off);
        const f32x4 hi = *(const f32x4 *)((const float *)a.q + off + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = lo[e];
          v[4 + e] = hi[e];
        }
      } else {
        unpack_bf16x8(*(const u32x4 *)((const uint16_t *)a.q + off), v);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] *= c_exp;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float h0 = round_bf16(v[2 * e]), h1 = round_bf16(v[2 * e + 1]);
        qhi[r][t][e] = pack_bf16x2(h0, h1);
        qlo[r][t][e] = pack_bf16x2(v[2 * e] - h0, v[2 * e + 1] - h1);
      }
    }

  f32x4 o[R][8];
  float m_run[R], l_run[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m_run[r] = kNegInf;
    l_run[r] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[r][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Block staging by LDS DMA (no registers held across the block), both
  // operands double-buffered and row-major with 16-byte chunks XOR-swizzled
  // by row (the lane writing LDS chunk slot c' of row r fetches global chunk
  // c' ^ f(r)): K with f(r) = r & 15 (conflict-free fragment reads of 16 rows
  // of one chunk), V with f(r) = 2 (r & 7), whose transposing reads (below)
  // then hit 16 distinct slots per half wave. K rows past kv_end are not
  // copied (their scores are masked to -inf); V rows past kv_end repeat key
  // kv_end - 1, so whatever P multiplies there is finite (and P is 0).
  uint16_t *k_lds0 = pf_lds;                 // [2][64 keys][128] swizzled
  uint16_t *v_lds0 = pf_lds + 2 * PKB * D;   // [2][64 keys][128] swizzled
  auto dma_block = [&](int blk) {
    uint16_t *kb = k_lds0 + (blk & 1) * PKB * D;
    uint16_t *vb = v_lds0 + (blk & 1) * PKB * D;
    // 2 x 16 instructions of 64 lanes (K, then V), spread over the waves
    for (int ins = __builtin_amdgcn_readfirstlane(wave); ins < 32; ins += 4 * HW) {
      const int gidx = 64 * (ins & 15) + lane;  // 16-byte granule of the block
      const int r = gidx >> 4, c = gidx & 15;
      const int key = blk * PKB + r;
      if (ins < 16) {
        if (key < kv_end)
          lds_dma16_asm(a.kc + kv_base, (uint32_t)(key * D + ((c ^ (r & 15)) << 3)) * 2u,
                        lds_u32(kb + 64 * 8 * (ins & 15)));
      } else {
        lds_dma16_asm(a.vc + kv_base, (uint32_t)(min(key, kv_end - 1) * D + ((c ^ (2 * (r & 7))) << 3)) * 2u,
                      lds_u32(vb + 64 * 8 * (ins & 15)));
      }
    }
  };
  // The V^T operand of O^T += V^T P^T straight from row-major V by
  // ds_read_b64_tr_b16: in each 16-lane group, lane 4j + q reads the 4
  // values d0 + 4q .. + 3 of key row k_j, and lane i receives the values at
  // d = d0 + i of rows k_0 .. k_3. Lane (col, g4) needs, for step ks, keys
  // 32 ks + 4 g4 + 0..3 and 32 ks + 16 + 4 g4 + 0..3 (the key order of its P
  // operand) at d = 16 dt + col: two reads.
  const int tr_j = col >> 2, tr_q = col & 3;
  auto v_frag = [&](const uint16_t *vb, int ks, int dt) {
    u32x4 va;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = 32 * ks + 16 * h + 4 * g4 + tr_j;
      const int d0 = 16 * dt + 4 * tr_q;
      const int slot = (d0 >> 3) ^ (2 * (row & 7));
      const uint16_t *src = vb + row * D + slot * 8 + (d0 & 7);
      typedef short v4i16 __attribute__((ext_vector_type(4)));
      const v4i16 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4i16 *)(src));
      const uint2 u = __builtin_bit_cast(uint2, t);
      va[2 * h] = u.x;
      va[2 * h + 1] = u.y;
    }
    return va;
  };

  dma_block(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  for (int blk = 0; blk < nblk; ++blk) {
    const uint16_t *ks_lds = k_lds0 + (blk & 1) * PKB * D;
    const uint16_t *vs_lds = v_lds0 + (blk & 1) * PKB * D;
    if (blk + 1 < nblk) dma_block(blk + 1);  // in flight while this block is used
    const int j0 = blk * PKB;
    if (j0 <= wave_last) {  // wave-uniform: else every key of the block is in this wave's future
      // S^T tiles: s[r][kt] lane (key j0 + 16 kt + 4 g4 + i, row col of tile r)
      f32x4 s[R][4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const int kr = kt * 16 + col;
        f32x4 acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4 kf = *(const u32x4 *)(ks_lds + kr * D + (((4 * t + g4) ^ col) << 3));
#pragma unroll
          for (int r = 0; r < R; ++r) {
            acc[r] = mfma16x16x32(as_bf16x8(kf), as_bf16x8(qhi[r][t]), acc[r]);
            acc[r] = mfma16x16x32(as_bf16x8(kf), as_bf16x8(qlo[r][t]), acc[r]);
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) s[r][kt] = acc[r];
      }
      u32x4 pb[R][2];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        // Scores c s (the scale and log2(e) are folded into q); the causal
        // mask only where some key of the block lies past the tile's first
        // row (wave-uniform).
        if (j0 + PKB - 1 > start + i0 + 16 * r) {
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (j0 + 16 * kt + 4 * g4 + i > my_pos[r]) s[r][kt][i] = kNegInf;
        }
        float mb = kNegInf;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) mb = fmaxf(mb, s[r][kt][i]);
        mb = wave_max4(mb);
        // key 0 is visible to every row and block 0 is never skipped, so
        // m_new is finite from the first block on (f = exp2(-inf) = 0 there).
        // p = exp(scale (s - m)) = exp2(c s - c m) on v_exp_f32 (terms below
        // 2^-126 of the reference flush to zero). The reference m moves only
        // when a block's maximum exceeds it by more than 8 (log2 units), so
        // p <= 2^8 (exact in bf16's range; l and O carry the same factor and
        // O / l is unchanged) and most blocks rescale nothing
        const float m_new = mb > m_run[r] + 8.f ? mb : m_run[r];
        const float f = __builtin_amdgcn_exp2f(m_run[r] - m_new);
        float ls = 0.f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = __builtin_amdgcn_exp2f(s[r][kt][i] - m_new);
            s[r][kt][i] = e;
            ls += e;
          }
        l_run[r] = l_run[r] * f + wave_sum4(ls);
        m_run[r] = m_new;
        if (__ballot(f != 1.f))  // no row's maximum moved: nothing to rescale
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) o[r][dt] *= f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          pb[r][ks] = u32x4{pack_bf16x2(s[r][2 * ks][0], s[r][2 * ks][1]),
                            pack_bf16x2(s[r][2 * ks][2], s[r][2 * ks][3]),
                            pack_bf16x2(s[r][2 * ks + 1][0], s[r][2 * ks + 1][1]),
                            pack_bf16x2(s[r][2 * ks + 1][2], s[r][2 * ks + 1][3])};
      }
      // O^T += V^T P^T: the V^T operand in the key order of pb
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const u32x4 va = v_frag(vs_lds, ks, dt);
#pragma unroll
          for (int r = 0; r < R; ++r) o[r][dt] = mfma16x16x32(as_bf16x8(va), as_bf16x8(pb[r][ks]), o[r][dt]);
        }
    }
    // the next block's copies are in; every wave is done with this block
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (i0 + 16 * r + col >= a.S) continue;
    const float inv = 1.0f / l_run[r];
    const int64_t ob = (int64_t)b * a.o_sb + (int64_t)(i0 + 16 * r + col) * a.o_ss + (int64_t)hq * a.o_sh;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f32x4 v = o[r][dt] * inv;
      const int64_t oi = ob + dt * 16 + 4 * g4;
      if (a.out_f32)
        *(f32x4 *)((float *)a.out + oi) = v;
      else
        *(uint2 *)((uint16_t *)a.out + oi) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
  }
}

#define RXW8_PREFILL(G)                                                              \
  extern "C" __global__ void __launch_bounds__(256) rxw8_gqa_prefill_d128_g##G(PrefillArgs a) { \
    attn_prefill<G>(a);                                                              \
  }                                                                                  \
  extern "C" __global__ void __launch_bounds__(256 * G)                              \
      rxw8_gqa_prefill_wh_d128_g##G(PrefillArgs a) {                                 \
    attn_prefill_wh<G>(a);                                                           \
  }                                                                                  \
  extern "C" __global__ void __launch_bounds__(256 * (G < 2 ? G : 2))                \
      __attribute__((amdgpu_waves_per_eu(2))) rxw8_gqa_prefill_r2_d128_g##G(PrefillArgs a) { \
    attn_prefill_rt<G, 2>(a);                                                        \
  }
RXW8_PREFILL(1)
RXW8_PREFILL(2)
RXW8_PREFILL(4)
// 8 query heads per kv head: the two-tile kernel only (four workgroups of
// two heads per kv head)
extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
rxw8_gqa_prefill_r2_d128_g8(PrefillArgs a) {
  attn_prefill_rt<8, 2>(a);
}

// ---- generic decode attention (any D <= 256, any group, f32 or bf16 cache):
// one workgroup per (b, query head); scores staged in LDS (Lmax <= 8192).
struct AttnGenericArgs {
  const void *q;
  const void *kc;
  const void *vc;
  const int32_t *lens;     // [R]
  const int32_t *row_seq;  // [R] cache slot, or null
  const float *mask;
  void *out;
  int64_t mask_sb, mask_sh;
  int B, Hq, Hkv, Lmax, D;
  float scale;
  int q_f32, cache_f32, out_f32;
};

__device__ __forceinline__ float ld_elem(const void *p, int64_t i, int f32) {
  return f32 ? ((const float *)p)[i] : bf16_bits_to_f32(((const uint16_t *)p)[i]);
}

extern "C" __global__ void __launch_bounds__(256) rxw8_gqa_decode_generic(AttnGenericArgs a) {
  __shared__ float sc[8192];
  __shared__ float red[256];
  const int bh = blockIdx.x;
  const int b = bh / a.Hq, h = bh - b * a.Hq;  // b: query row
  const int kvh = h / (a.Hq / a.Hkv);
  int len = a.lens[b];
  len = len < 1 ? 1 : (len > a.Lmax ? a.Lmax : len);
  const int seq = a.row_seq ? a.row_seq[b] : b;
  const int64_t qoff = ((int64_t)b * a.Hq + h) * a.D;
  const int64_t kvoff = ((int64_t)seq * a.Hkv + kvh) * a.Lmax * a.D;
  float mx = -__builtin_huge_valf();
  for (int j = threadIdx.x; j < len; j += blockDim.x) {
    float acc = 0.f;
    for (int d = 0; d < a.D; ++d)
      acc += ld_elem(a.q, qoff + d, a.q_f32) * ld_elem(a.kc, kvoff + (int64_t)j * a.D + d, a.cache_f32);
    float s = acc * a.scale;
    if (a.mask) s += a.mask[(int64_t)b * a.mask_sb + (int64_t)h * a.mask_sh + j];
    sc[j] = s;
    mx = fmaxf(mx, s);
  }
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int st = blockDim.x / 2; st > 0; st >>= 1) {
    if (threadIdx.x < st) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + st]);
    __syncthreads();
  }
  mx = red[0];
  __syncthreads();
  float sum = 0.f;
  for (int j = threadIdx.x; j < len; j += blockDim.x) {
    const float e = __expf(sc[j] - mx);
    sc[j] = e;
    sum += e;
  }
  red[threadIdx.x] = sum;
  __syncthreads();
  for (int st = blockDim.x / 2; st > 0; st >>= 1) {
    if (threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
    __syncthreads();
  }
  sum = red[0];
  for (int d = threadIdx.x; d < a.D; d += blockDim.x) {
    float acc = 0.f;
    for (int j = 0; j < len; ++j)
      acc += (sc[j] / sum) * ld_elem(a.vc, kvoff + (int64_t)j * a.D + d, a.cache_f32);
    const int64_t oi = qoff + d;
    if (a.out_f32)
      ((float *)a.out)[oi] = acc;
    else
      ((uint16_t *)a.out)[oi] = f32_to_bf16_bits(acc);
  }
}

// ---- general grouped-query attention (attention.rs:83-135 with SDPA
// :150-252): query row (b, h, i) with i < Sq, keys j < Sk of kv head
// h / (Hq / Hkv); scores q.k * scale + mask, softmax over the keys in f32,
// out (b, h, i, :) = sum_j p_j v_j. Element strides (batch b, head, row) for
// q, out, k and v (rows of D, resp. Dv, contiguous), so one kernel serves
// head-major [..., H, S, D] tensors and the token-major [B, S, Hq, D] prefill
// queries over a [B, Hkv, Lmax, D] cache. q, k, v are f32 or bf16 (widened
// exactly), out f32 or bf16. The additive mask broadcasts to [..., Hq, Sq,
// Sk]: element (b, h, i, j) sits at moff(b) + h * msh + i * msi + j * msj,
// moff summing the batch index's digits (bdim) times their mask strides (0
// where the mask broadcasts). With starts (causal prefill), row i of batch b
// sees keys 0 .. st + i only, st = clamp(starts[b], 0, Sk - Sq) (the
// reference's causal mask key_pos <= q_pos for rows at positions st + i;
// the keys past it are skipped, which adds exactly nothing to the softmax).
//
// One wave per output row (b, h, i). The row's q sits in the wave's LDS
// slice; keys go in chunks of 64 (lane = key: a sequential f32 dot product
// over D), with an online softmax (running max m, sum l, accumulators rescaled
// by exp(m_old - m_new)); P.V accumulates with lanes over the Dv outputs and
// each chunk probability broadcast by a lane shuffle. A row whose keys are all
// masked (-inf) ends as 0 / 0 = NaN, the reference's max-subtract softmax of
// such a row. The reference orders the softmax as max, exp, sum, divide over
// the whole row; the online form reassociates those sums (f32 rounding
// differences only).
struct GqaGeneralArgs {
  const void *q, *k, *v;
  const float *mask;        // or null
  void *out;
  int64_t bdim[4];          // batch prefix dims (innermost last), 1 where absent
  int64_t mb[4];            // mask stride of each batch dim (0: broadcast)
  int64_t msh, msi, msj;    // mask strides of head, query, key (0: broadcast)
  int64_t rows;             // NB * Hq * Sq
  int Hq, Hkv, Sq, Sk, D, Dv;
  float scale;
  int64_t q_sb, q_sh, q_si;  // element strides of q (batch, head, row)
  int64_t o_sb, o_sh, o_si;  // of out
  int64_t k_sb, k_sh;        // of k (rows of D), v: v_sb, v_sh (rows of Dv)
  int64_t v_sb, v_sh;
  int q_bf16, kv_bf16, out_bf16;
  const int32_t *starts;     // [NB] causal prefill starts, or null
};

constexpr int kGqaMaxD = 1024;   // q row staged in LDS
constexpr int kGqaMaxDv = 512;   // 8 accumulators per lane

__device__ __forceinline__ float gqa_ld(const void *p, int64_t i, int bf16) {
  return bf16 ? bf16_bits_to_f32(((const uint16_t *)p)[i]) : ((const float *)p)[i];
}

extern "C" __global__ void __launch_bounds__(256) rxw8_gqa_general(GqaGeneralArgs a) {
  __shared__ float qrow[4][kGqaMaxD];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + wv;
  if (row >= a.rows) return;  // whole waves; no workgroup barrier below
  const int i = (int)(row % a.Sq);
  const int64_t bh = row / a.Sq;
  const int h = (int)(bh % a.Hq);
  const int64_t b = bh / a.Hq;
  const int kvh = h / (a.Hq / a.Hkv);
  const int64_t qo = b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)i * a.q_si;
  const int64_t ko = b * a.k_sb + (int64_t)kvh * a.k_sh;
  const int64_t vo = b * a.v_sb + (int64_t)kvh * a.v_sh;
  int nkeys = a.Sk;
  if (a.starts) {
    const int st = min(max(a.starts[b], 0), a.Sk - a.Sq);
    nkeys = st + i + 1;
  }
  const float *mp = nullptr;
  if (a.mask) {
    int64_t off = 0, rest = b;
    for (int t = 3; t >= 0; --t) {
      const int64_t digit = rest % a.bdim[t];
      rest /= a.bdim[t];
      off += digit * a.mb[t];
    }
    mp = a.mask + off + (int64_t)h * a.msh + (int64_t)i * a.msi;
  }
  float *ql = qrow[wv];
  for (int d = lane; d < a.D; d += 64) ql[d] = gqa_ld(a.q, qo + d, a.q_bf16);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float ninf = -__builtin_huge_valf();
  float m = ninf, l = 0.f;
  float acc[kGqaMaxDv / 64];
#pragma unroll
  for (int r = 0; r < kGqaMaxDv / 64; ++r) acc[r] = 0.f;
  for (int c0 = 0; c0 < nkeys; c0 += 64) {
    const int j = c0 + lane;
    const bool valid = j < nkeys;
    float s = ninf;
    if (valid) {
      const int64_t kr = ko + (int64_t)j * a.D;
      float dot = 0.f;
      for (int d = 0; d < a.D; ++d) dot += ql[d] * gqa_ld(a.k, kr + d, a.kv_bf16);
      s = dot * a.scale;
      if (mp) s += mp[(int64_t)j * a.msj];
    }
    float cmax = valid ? s : ninf;
    for (int o = 32; o > 0; o >>= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, o));
    const float m_new = fmaxf(m, cmax);
    if (m_new == ninf) continue;  // nothing visible yet: keep m = -inf, l = 0
    const float alpha = expf(m - m_new);
    const float p = valid ? expf(s - m_new) : 0.f;
    float ps = p;
    for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o);
    l = l * alpha + ps;
    const int nk = min(64, nkeys - c0);
#pragma unroll
    for (int r = 0; r < kGqaMaxDv / 64; ++r) acc[r] *= alpha;
    for (int jj = 0; jj < nk; ++jj) {
      const float pj = __shfl(p, jj);
      const int64_t vr = vo + (int64_t)(c0 + jj) * a.Dv;
#pragma unroll
      for (int r = 0; r < kGqaMaxDv / 64; ++r) {
        const int d = lane + 64 * r;
        if (d < a.Dv) acc[r] += pj * gqa_ld(a.v, vr + d, a.kv_bf16);
      }
    }
    m = m_new;
  }
  // all keys masked: the reference's softmax of an all -inf row is NaN
  const float inv = m == ninf ? __builtin_nanf("") : 1.0f / l;
  const int64_t oo = b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)i * a.o_si;
#pragma unroll
  for (int r = 0; r < kGqaMaxDv / 64; ++r) {
    const int d = lane + 64 * r;
    if (d < a.Dv) {
      const float y = m == ninf ? inv : acc[r] * inv;
      if (a.out_bf16)
        ((uint16_t *)a.out)[oo + d] = f32_to_bf16_bits(y);
      else
        ((float *)a.out)[oo + d] = y;
    }
  }
}

// Tensor::causal_attention_mask (attention.rs:14-32): out [Q, K] f32, entry
// (i, j) = 0 iff key_pos[j] <= query_pos[i] (signed I32 compare, no
// subtraction or float conversion), else -inf.
struct CausalMaskArgs {
  const int32_t *qpos, *kpos;
  float *out;
  int64_t Q, K;
};

extern "C" __global__ void __launch_bounds__(256) rxw8_gqa_causal_mask(CausalMaskArgs a) {
  const int64_t n = a.Q * a.K;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / a.K, j = e - i * a.K;
    a.out[e] = a.kpos[j] <= a.qpos[i] ? 0.0f : -__builtin_huge_valf();
  }
}
