/*
 * rxw8 CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference (SunDoge/rxla) semantics for the
 * W8A16 decode/prefill hot path. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library; the product path
 * (rxla_amd/, librxw8.so) never calls it.
 *
 * Every function names the reference file:line it restates. Each one is
 * pinned by the checks listed in its comment (reference golden vectors,
 * closed forms, brute force); see tests/test_oracle_*.py.
 */
#ifndef RXW8_ORACLE_H
#define RXW8_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions -------------------------------------------------- */

/* f32 -> bf16 bits, round-to-nearest-even, NaN kept quiet.
 * Restates stablehlo.convert f32->bf16 (crates/rxla-core/src/ops.rs:8 cast,
 * dtype_rules.rs:14-18). Pinned by tests/cast.rs:14-28 KATs and the
 * exhaustive 65,536-pattern round trip (rxla-pjrt/tests/bf16.rs:3-49). */
uint16_t rxo_bf16_from_f32(float x);
float rxo_f32_from_bf16(uint16_t b);
void rxo_f32_to_bf16(const float *x, uint16_t *out, int64_t n);
void rxo_bf16_to_f32(const uint16_t *x, float *out, int64_t n);

/* ---- a1: W8 encoder ------------------------------------------------------ */

/* benchmarks/quantize_qwen3_5_w8.py:27-44: per row, per group of G inputs,
 * s = max(amax, 1e-12) / 127 (f32); q = clamp(rne(w / s), -127, 127);
 * u8 = q + 128. Returns 0 or -1 for bad shapes (K % G != 0). */
int rxo_quantize_w8(const float *w, int64_t n, int64_t k, int64_t g,
                    uint8_t *u8_out, float *scale_out);

/* ---- a2: dequantisation -------------------------------------------------- */

/* crates/rxla-nn/src/layers.rs:277-287: W = (f32(u8) + (-128)) * scale[n, k/G].
 * One correctly rounded f32 multiply. */
int rxo_dequantize_w8(const uint8_t *u8, const float *scale, int64_t n,
                      int64_t k, int64_t g, float *w_out);

/* ---- a2/a3: W8A16 linear -------------------------------------------------- */

#define RXO_COMPUTE_F32 0
#define RXO_COMPUTE_BF16 1
#define RXO_ACCUM_F32 0 /* sequential f32 sum in k order */
#define RXO_ACCUM_F64 1 /* f64 sum ("ideal"), rounded once */

/* crates/rxla-nn/src/layers.rs:257-298 (+ nn.rs:286-309, lib.rs:795-926,
 * emitter.rs:45-58, dtype_rules.rs:35-47). y[M,N] (f32) from x[M,K] f32.
 * compute F32:  y = x . Wdq^T.
 * compute BF16: y = f32(bf16(bf16(x) . bf16(Wdq)^T)), the bf16 dot result
 *               rounded once (RNE) from the accumulator. */
int rxo_quantized_linear(const float *x, int64_t m, int64_t k, const uint8_t *u8,
                         const float *scale, int64_t n, int64_t g, int compute,
                         int accum, float *y, int threads);

/* Dense bf16 linear (bf16 embedding reused as lm_head):
 * y = f32(bf16(bf16(x) . W^T)), W bf16 [N,K]. */
int rxo_linear_bf16w(const float *x, int64_t m, int64_t k, const uint16_t *w,
                     int64_t n, int accum, float *y, int threads);

/* ---- a5-a7: attention ----------------------------------------------------- */

/* crates/rxla-core/src/attention.rs:83-252 with the portable lowering order
 * crates/rxla-ir/src/pliron/stablehlo/conversion.rs:363-499:
 *   s = (q . k) * scale + mask ; m = max s ; e = exp(s - m) ; p = e / sum e ;
 *   out = p . v
 * GQA: query head h uses kv head h / (Hq / Hkv) (attention.rs:83-135).
 * q [B,Hq,Sq,D], k [B,Hkv,Sk,D], v [B,Hkv,Sk,Dv], out [B,Hq,Sq,Dv].
 * mask: additive f32 addressed as mask[b*mask_sb + h*mask_sh + i*mask_si + j]
 * (stride 0 = broadcast), or NULL. precision: 0 = f32 in reference order,
 * 1 = f64 (pinned against tests/gqa.rs:32-102, tests/masked_decode.rs). */
int rxo_gqa_attention(const float *q, const float *k, const float *v,
                      int64_t b, int64_t hq, int64_t hkv, int64_t sq,
                      int64_t sk, int64_t d, int64_t dv, const float *mask,
                      int64_t mask_sb, int64_t mask_sh, int64_t mask_si,
                      float scale, int precision, float *out, int threads);

/* Decode form over a contiguous per-sequence cache. q [B,Hq,D] f32,
 * caches [B,Hkv,Lmax,D] stored as bf16 bits, lens[b] visible keys (the
 * mask key_pos <= q_pos of attention.rs:14-32 with q_pos = lens[b]-1).
 * Keys at positions >= lens[b] are not read. out [B,Hq,D] f32. */
int rxo_gqa_decode_bf16cache(const float *q, const uint16_t *kc,
                             const uint16_t *vc, const int32_t *lens,
                             int64_t b, int64_t hq, int64_t hkv, int64_t lmax,
                             int64_t d, float scale, int precision, float *out,
                             int threads);

/* ---- a8: KV cache ---------------------------------------------------------- */

/* crates/rxla-core/src/indexing.rs:663-678 (XLA dynamic_update_slice):
 * start_i is clamped to [0, dim_i - udim_i]. operand/update are row-major
 * with elem_size-byte elements; result written into `operand` in place. */
int rxo_dynamic_update_slice(void *operand, const int64_t *dims, int rank,
                             int64_t elem_size, const void *update,
                             const int64_t *udims, const int32_t *starts);

/* crates/rxla-core/src/kv_cache.rs:53-68 (update_at: paired DUS, clamped)
 * and :79-111 (update_at_checked: accepted iff every 0 <= start_i <=
 * dim_i - udim_i; otherwise both caches unchanged). accepted may be NULL. */
int rxo_kv_update_at(void *kc, void *vc, const int64_t *dims, int rank,
                     int64_t elem_size, const void *ku, const void *vu,
                     const int64_t *udims, const int32_t *starts, int checked,
                     float *accepted);

/* ---- a10-a14: elementwise / reductions ----------------------------------- */

/* crates/rxla-models/src/qwen3_5/mod.rs:211-228: freq_i = theta^(-2i/rot)
 * in f32 (powf); angle = f32(pos) * freq_i. */
void rxo_rope_freqs(float theta, int64_t rot_dim, float *freqs);

/* crates/rxla-core/src/rotary.rs:17-74 SplitHalf on the first rot_dim
 * channels of each [D] row (qwen3_5/layers.rs:11-26 partial rotary):
 * (a cos - b sin, b cos + a sin); channels >= rot_dim pass through.
 * x [rows, D] in place; pos[row / rows_per_pos]. */
void rxo_rope_split_half(float *x, int64_t rows, int64_t d, int64_t rot_dim,
                         const int32_t *pos, int64_t rows_per_pos,
                         float theta);

/* crates/rxla-core/src/ops.rs:929-944 (+ layers.rs:455-495 zero_centered):
 * y = (x * rsqrt(mean(x^2) + eps)) * (w or 1 + w). */
void rxo_rms_norm(const float *x, int64_t rows, int64_t h, const float *w,
                  float eps, int zero_centered, float *y);

/* ops.rs:331-342: silu(x) = x * sigmoid(x); out = silu(gate) * up. */
void rxo_silu_mul(const float *gate, const float *up, int64_t n, float *out);

/* crates/rxla-core/src/indexing.rs:637-656: rows of table gathered with
 * ids clamped to [0, V-1]. */
void rxo_take_rows(const void *table, int64_t v, int64_t row_bytes,
                   const int32_t *ids, int64_t n, void *out);

/* crates/rxla-core/src/indexing.rs:350-374: lowest index of the maximum;
 * a NaN wins over any number and the first NaN wins (tests/argmax.rs:30-40). */
void rxo_argmax_rows(const float *x, int64_t rows, int64_t cols, int32_t *out);

/* ---- a15: synthetic Qwen-style dense decoder ----------------------------- */

typedef struct rxo_decoder_config {
  int64_t layers, hidden, q_heads, kv_heads, head_dim, intermediate, vocab;
  int64_t max_seq; /* KV capacity per sequence */
  int64_t group;   /* W8 group size; 0 = per-output-channel (G = input width) */
  float eps, theta;
  int32_t qk_norm; /* per-head RMSNorm on q and k before RoPE */
  int32_t accum;   /* RXO_ACCUM_F32 (sequential f32, the default) or RXO_ACCUM_F64
                    * for every dot product: two summation orders of the same
                    * cast points, to measure how far the reference's semantics
                    * themselves move under a change of accumulation */
} rxo_decoder_config;

/* Parameters, per layer l (arrays of pointers, length `layers`):
 *   in_norm[l] f32[H], qkv_w[l] u8[(Hq+2Hkv)D, H], qkv_s[l] f32[(Hq+2Hkv)D, H/G]
 *   q_norm[l] f32[D], k_norm[l] f32[D] (when qk_norm),
 *   o_w[l] u8[H, HqD], o_s[l] f32[H, HqD/G], post_norm[l] f32[H],
 *   gu_w[l] u8[2I, H] (gate rows then up rows), gu_s[l] f32[2I, H/G],
 *   down_w[l] u8[H, I], down_s[l] f32[H, I/G]
 * Shared: embed bf16[V,H] (also the tied lm_head), final_norm f32[H]. */
typedef struct rxo_decoder_params {
  const float **in_norm, **q_norm, **k_norm, **post_norm;
  const uint8_t **qkv_w, **o_w, **gu_w, **down_w;
  const float **qkv_s, **o_s, **gu_s, **down_s;
  const uint16_t *embed;
  const float *final_norm;
} rxo_decoder_params;

/* Runs `s` new tokens per sequence (prefill when s > 1, decode when s == 1)
 * starting at position lens[b] for each of the `b` sequences: embeddings,
 * `layers` x (norm, fused QKV, q/k norm, RoPE, KV append into the bf16 caches
 * [L][B][Hkv][max_seq][D], causal GQA attention, o_proj, residual, norm,
 * fused gate/up, SiLU*up, down, residual), final norm, lm_head on the last
 * new position. logits [b, V] f32; next_ids [b] = argmax. lens[] advanced by s.
 * Composition follows crates/rxla-models/src/qwen3_5/mod.rs:199-273 and
 * layers.rs:28-101,270-293 (dense full-attention layers, no output gate). */
int rxo_decoder_forward(const rxo_decoder_config *cfg,
                        const rxo_decoder_params *p, uint16_t *k_cache,
                        uint16_t *v_cache, int32_t *lens, int64_t b, int64_t s,
                        const int32_t *ids, float *logits, int32_t *next_ids,
                        int threads);

/* rxo_decoder_forward that also records the residual stream: trace
 * [layers + 1, b * s, H] f32 receives the input of every layer (row bi * s + t)
 * and, last, the output of the final layer (before the final norm). */
int rxo_decoder_forward_trace(const rxo_decoder_config *cfg,
                              const rxo_decoder_params *p, uint16_t *k_cache,
                              uint16_t *v_cache, int32_t *lens, int64_t b,
                              int64_t s, const int32_t *ids, float *logits,
                              int32_t *next_ids, int threads, float *trace);

#ifdef __cplusplus
}
#endif

#endif
