/*
 * rxw8 -- MI355X-native (gfx950) W8A16 decode/prefill hot path of RXLA,
 * exposed as a plain C ABI.
 *
 * The reference (SunDoge/rxla) reaches this path through Rust:
 *   rxla_nn::QuantizedLinear::apply            crates/rxla-nn/src/layers.rs:251-298
 *   Tensor::grouped_query_attention            crates/rxla-core/src/attention.rs:83-135
 *   Tensor::scaled_dot_product_attention       crates/rxla-core/src/attention.rs:150-252
 *   KvCache::{update_at, update_at_checked}    crates/rxla-core/src/kv_cache.rs:53-111
 *   AppliedModel::compile / CompiledModel::{bind_parameters, run}
 *                                              crates/rxla-nn/src/applied.rs:135-239,808-815
 * and executes through a PJRT plugin (crates/rxla-pjrt/src/runtime.rs). This
 * header replaces that plugin boundary for the path: status codes use the
 * PJRT_Error_Code numbering (vendor/xla/pjrt/c/pjrt_c_api.h:168-186), buffers
 * are refcounted device allocations owned by a runtime (runtime.rs:1446,1523),
 * and every entry point validates shapes and dtypes before anything is
 * launched, leaving outputs and state untouched on error.
 *
 * Threading: a runtime owns one HIP stream; all work on it is stream-ordered.
 * Entry points are thread-safe (internal mutex). Entry points that return
 * new buffers enqueue work and return; rxw8_buffer_to_host and
 * rxw8_runtime_synchronize block until the stream has drained.
 */
#ifndef RXW8_H
#define RXW8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RXW8_ABI_VERSION 1

/* ---- status (PJRT_Error_Code numbering, pjrt_c_api.h:168-186) ------------ */
typedef enum rxw8_status {
  RXW8_OK = 0,
  RXW8_CANCELLED = 1,
  RXW8_UNKNOWN = 2,
  RXW8_INVALID_ARGUMENT = 3,
  RXW8_DEADLINE_EXCEEDED = 4,
  RXW8_NOT_FOUND = 5,
  RXW8_ALREADY_EXISTS = 6,
  RXW8_PERMISSION_DENIED = 7,
  RXW8_RESOURCE_EXHAUSTED = 8,
  RXW8_FAILED_PRECONDITION = 9,
  RXW8_ABORTED = 10,
  RXW8_OUT_OF_RANGE = 11,
  RXW8_UNIMPLEMENTED = 12,
  RXW8_INTERNAL = 13,
  RXW8_UNAVAILABLE = 14,
  RXW8_DATA_LOSS = 15,
  RXW8_UNAUTHENTICATED = 16
} rxw8_status;

/* Message of the last failing call on this thread (UTF-8, never NULL). */
const char *rxw8_last_error(void);
/* PjrtErrorCode::is_retryable (crates/rxla-pjrt/src/runtime.rs:93-104). */
int rxw8_status_is_retryable(int status);
int rxw8_abi_version(void);

/* ---- dtypes (the Element types of crates/rxla-pjrt/src/runtime.rs:1422-1440) */
typedef enum rxw8_dtype {
  RXW8_U8 = 1,
  RXW8_I32 = 2,
  RXW8_F16 = 3,
  RXW8_BF16 = 4,
  RXW8_F32 = 5
} rxw8_dtype;

#define RXW8_MAX_RANK 8

typedef struct rxw8_runtime rxw8_runtime;
typedef struct rxw8_buffer rxw8_buffer;

/* ---- runtime (replaces Client::load, runtime.rs:768) --------------------- */

/* Select HIP device `device`, create its stream, load the gfx950 kernels.
 * FAILED_PRECONDITION when the device is not gfx950 or no device exists. */
int rxw8_runtime_create(int device, rxw8_runtime **out);
/* Drops the caller's reference; the runtime lives until its last buffer is
 * released. */
int rxw8_runtime_destroy(rxw8_runtime *rt);
/* Enqueue subsequent work on an external hipStream_t (NULL: the runtime's
 * own stream). The caller keeps the stream alive while it is in use. */
int rxw8_runtime_set_stream(rxw8_runtime *rt, void *hip_stream);
int rxw8_runtime_stream(rxw8_runtime *rt, void **hip_stream);
int rxw8_runtime_synchronize(rxw8_runtime *rt);
/* Compute units and device name (for roofline bookkeeping). */
int rxw8_runtime_device_info(rxw8_runtime *rt, int *compute_units,
                             char *name, size_t name_len);

/* ---- buffers (Client::buffer runtime.rs:920, Buffer::to_vec :1885) -------- */

/* New device buffer of dtype/dims; contents zeroed. */
int rxw8_buffer_create(rxw8_runtime *rt, int dtype, const int64_t *dims,
                       int rank, rxw8_buffer **out);
/* New device buffer holding a copy of `data` (row-major, packed). */
int rxw8_buffer_from_host(rxw8_runtime *rt, int dtype, const int64_t *dims,
                          int rank, const void *data, rxw8_buffer **out);
/* Non-owning view of caller-owned device memory (e.g. a torch tensor). The
 * caller keeps the memory alive for the lifetime of the view. */
int rxw8_buffer_wrap(rxw8_runtime *rt, int dtype, const int64_t *dims,
                     int rank, void *device_ptr, rxw8_buffer **out);
/* Blocking copy of the whole buffer to host; `bytes` must equal its size. */
int rxw8_buffer_to_host(rxw8_buffer *buf, void *dst, size_t bytes);
/* Blocking copy from host into an existing buffer. */
int rxw8_buffer_copy_from_host(rxw8_buffer *buf, const void *src, size_t bytes);
int rxw8_buffer_retain(rxw8_buffer *buf);
int rxw8_buffer_release(rxw8_buffer *buf);
int rxw8_buffer_dtype(const rxw8_buffer *buf, int *dtype);
/* Writes up to RXW8_MAX_RANK dims; *rank receives the rank. */
int rxw8_buffer_dims(const rxw8_buffer *buf, int64_t *dims, int *rank);
int rxw8_buffer_device_ptr(const rxw8_buffer *buf, void **ptr);

/* ---- ops --------------------------------------------------------------------
 * Allocating forms return a new buffer in *out; `_into` forms write into a
 * caller buffer of the exact shape/dtype and allocate nothing per call
 * (split-K workspaces are runtime-owned, grown on first use). */

/* The W8 encoder (benchmarks/quantize_qwen3_5_w8.py:27-44): for each row and
 * group of group_size columns, s = max(amax, 1e-12) / 127 and
 * u8 = clamp(rne(w / s), -127, 127) + 128, in f32 with a correctly rounded
 * division, as the encoder's torch ops compute.
 *   w F32|BF16 [N,K] (BF16 widens exactly, the encoder's value.float());
 *   weight U8 [N,K] and scale F32 [N, K/group_size] are new buffers.
 * group_size = K gives per-output-channel scales. INVALID_ARGUMENT for a
 * non-positive group size or one that does not divide K (the encoder's
 * ValueErrors). A group holding a NaN gets a NaN scale and code 128 (the
 * encoder's codes there come from an unspecified NaN-to-uint8 cast). */
int rxw8_quantize_w8(rxw8_runtime *rt, rxw8_buffer *w, int64_t group_size,
                     rxw8_buffer **weight, rxw8_buffer **scale);

/* W8 dequantisation (layers.rs:277-287): W = (f32(u8) - 128) * scale[n, k/G]
 * -> F32 (bit-exact) or BF16 (RNE of the f32 value). weight U8 [N,K],
 * scale F32 [N,K/G]. */
int rxw8_dequantize(rxw8_runtime *rt, rxw8_buffer *weight, rxw8_buffer *scale,
                    int out_dtype, rxw8_buffer **out);

/* Tiled copy of a weight for the packed GEMV kernels (no counterpart in the
 * reference, which hands XLA row-major U8/BF16 parameters): U8 [N,K] ->
 * U8 [N/16, K/64, 1024] and BF16 [N,K] -> BF16 [N/16, K/32, 512]. Block (t, c)
 * holds, for lane l = 0..63, the 16 bytes of row 16t + l%16 starting at column
 * c*kb + (l/16)*(kb/4) (kb = 64 for U8, 32 for BF16), so one wavefront load is
 * one contiguous KiB. Requires N % 16 == 0 and K % kb == 0. The packed buffer
 * is accepted wherever the row-major weight is (quantized_linear, linear_bf16,
 * decoder parameters), holds the same bytes and gives the same results. */
int rxw8_pack_weight(rxw8_runtime *rt, rxw8_buffer *weight, rxw8_buffer **packed);

/* QuantizedLinear::apply (layers.rs:257-298) with the layer compute dtype:
 *   x [..., K] F32 or BF16; weight U8 [N,K] (int8 + 128), or its packed form
 *   U8 [N/16, K/64, 1024] (rxw8_pack_weight); scale F32 [N,K/G];
 *   compute_dtype BF16 (W8A16: bf16(x) . bf16 weights, f32 accumulation,
 *   bf16-rounded result) or F32 (f32 x, f32 dequantised weights; with the
 *   packed form, N % 16 == 0).
 *   y [..., N] of out_dtype F32 or BF16 (same values: the BF16 compute result
 *   is bf16-valued; F32 compute requires F32 out).
 * Errors (before launch): INVALID_ARGUMENT for rank 0, non-positive widths,
 * K % G != 0, weight/scale shape or dtype mismatch (the InvalidLayerInput
 * checks of layers.rs:258-274 and validate_buffer of applied.rs:1274). */
int rxw8_quantized_linear(rxw8_runtime *rt, rxw8_buffer *x, rxw8_buffer *weight,
                          rxw8_buffer *scale, int compute_dtype, int out_dtype,
                          rxw8_buffer **y);
int rxw8_quantized_linear_into(rxw8_runtime *rt, rxw8_buffer *x,
                               rxw8_buffer *weight, rxw8_buffer *scale,
                               int compute_dtype, rxw8_buffer *y);

/* Several independent QuantizedLinear::apply calls with BF16 compute in one
 * grouped launch (no counterpart in the reference, which compiles each linear
 * into its own XLA op): for i < count, y[i] = the product rxw8_quantized_linear_into
 * computes for (x[i], weight[i], scale[i]). One launch per class of rows
 * (<= 4: 96-row tiles; 5..16: 192-row tiles) runs every product of the class
 * on one tiling, so the per-launch cost is paid once per class instead of
 * once per product.
 * Requirements beyond rxw8_quantized_linear_into's: count in [1, 16];
 * 1..16 rows (the product of x's leading dims) per product; N % 16 == 0,
 * K % 512 == 0, per-channel scales or groups that divide K/4; all weights
 * row-major or all packed. Results agree with the single call within one
 * bf16 ulp (the tilings, and so the f32 summation order, may differ).
 * INVALID_ARGUMENT / UNIMPLEMENTED before any launch. */
int rxw8_quantized_linear_group(rxw8_runtime *rt, int count, rxw8_buffer *const *x,
                                rxw8_buffer *const *weight, rxw8_buffer *const *scale,
                                rxw8_buffer *const *y);

/* Dense linear with BF16 weights (bf16-stored embedding reused as lm_head,
 * layers.rs Linear with parameter storage BF16, lib.rs:478-487):
 * y = bf16(bf16(x) . W^T). x [..., K] F32|BF16, weight BF16 [N,K] or its
 * packed form BF16 [N/16, K/32, 512]. */
int rxw8_linear_bf16(rxw8_runtime *rt, rxw8_buffer *x, rxw8_buffer *weight,
                     int out_dtype, rxw8_buffer **y);
int rxw8_linear_bf16_into(rxw8_runtime *rt, rxw8_buffer *x, rxw8_buffer *weight,
                          rxw8_buffer *y);

/* Grouped-query decode attention (attention.rs:83-135 + SDPA :150-252, F32
 * semantics) over a contiguous per-sequence KV cache:
 *   q [B,Hq,D] F32|BF16; k_cache/v_cache [B,Hkv,Lmax,D] BF16|F32;
 *   lens I32 [B] (device): sequence b sees keys 0..lens[b]-1, which is the
 *   causal mask key_pos <= q_pos (attention.rs:14-32) for q_pos = lens[b]-1;
 *   mask: optional additive F32 [B|1, Hq|1, Lmax] (NULL = none);
 *   scale: <= 0 selects 1/sqrt(D).
 * Query head h reads kv head h / (Hq/Hkv). out [B,Hq,D] F32|BF16.
 * lens entries outside [1, Lmax] are clamped into it by the kernel. */
int rxw8_gqa_decode(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k_cache,
                    rxw8_buffer *v_cache, rxw8_buffer *lens, rxw8_buffer *mask,
                    float scale, int out_dtype, rxw8_buffer **out);
int rxw8_gqa_decode_into(rxw8_runtime *rt, rxw8_buffer *q,
                         rxw8_buffer *k_cache, rxw8_buffer *v_cache,
                         rxw8_buffer *lens, rxw8_buffer *mask, float scale,
                         rxw8_buffer *out);

/* Tensor::grouped_query_attention(k, v, mask, scale) (attention.rs:83-135)
 * with SDPA semantics (:150-252) for any query count:
 *   q [..., Hq, Sq, D], k [..., Hkv, Sk, D], v [..., Hkv, Sk, Dv], all F32,
 *   equal batch prefixes (up to 4 dims), Hq % Hkv == 0, Sk > 0;
 *   mask: optional additive F32, broadcastable (right-aligned, size-1 dims)
 *   to the scores [..., Hq, Sq, Sk] before grouping; NULL = none;
 *   scale: NULL selects 1/sqrt(D), else it must be finite.
 * Query head h reads kv head h / (Hq/Hkv); softmax over the keys in f32;
 * out F32 [..., Hq, Sq, Dv]. A row whose keys are all masked is NaN, as in
 * the reference. INVALID_ARGUMENT mirrors the reference's shape, dtype and
 * scale errors; UNIMPLEMENTED beyond D 1024 / Dv 512. */
int rxw8_gqa_attention(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k,
                       rxw8_buffer *v, rxw8_buffer *mask, const float *scale,
                       rxw8_buffer **out);
int rxw8_gqa_attention_into(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k,
                            rxw8_buffer *v, rxw8_buffer *mask,
                            const float *scale, rxw8_buffer *out);

/* Tensor::causal_attention_mask (attention.rs:14-32): from runtime query
 * positions I32 [Q] and key positions I32 [K], the additive F32 mask [Q, K]
 * whose (i, j) entry is 0 iff key_positions[j] <= query_positions[i] (signed
 * I32 compare, exact at any I32 value), else -inf. */
int rxw8_causal_attention_mask(rxw8_runtime *rt, rxw8_buffer *query_positions,
                               rxw8_buffer *key_positions, rxw8_buffer **out);

/* rxw8_gqa_decode_into that allocates nothing. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops and harnesses that forbid hipMalloc).
 * Same arguments, validation and results (bit for bit) as
 * rxw8_gqa_decode_into. The split partials and arrival counters live in a
 * fixed device array that each GPU holds for the life of the process
 * (RXW8_NOALLOC_PARTIAL_BYTES + RXW8_NOALLOC_COUNTER_BYTES); a call whose plan
 * needs more fails with RXW8_RESOURCE_EXHAUSTED before any launch. The split
 * plans of the D = 128 kernel (Hq/Hkv in {1, 2, 4, 8}) use at most 4 x CUs
 * partial slots of Hq/Hkv x 130 floats -- 4.1 MiB on 256 CUs -- and the
 * general kernel none, so on MI355X that happens only for a counter need
 * (rows x kv heads) above 16384.
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (other streams, runtimes or threads) race and must be serialised by the
 * caller. The device must have had a runtime created on it (set-up). */
#define RXW8_NOALLOC_PARTIAL_BYTES ((size_t)16 << 20)
#define RXW8_NOALLOC_COUNTER_BYTES ((size_t)64 << 10)
int rxw8_gqa_decode_noalloc(rxw8_runtime *rt, rxw8_buffer *q,
                            rxw8_buffer *k_cache, rxw8_buffer *v_cache,
                            rxw8_buffer *lens, rxw8_buffer *mask, float scale,
                            rxw8_buffer *out);

/* Causal grouped-query prefill attention (attention.rs:83-135 + SDPA
 * :150-252 with the causal mask key_pos <= q_pos of attention.rs:14-32;
 * F32 softmax) for S new query rows per sequence whose keys and values are
 * already in the cache:
 *   q [B,S,Hq,D] F32|BF16 (token-major, the layout of the projection output);
 *   k_cache/v_cache [B,Hkv,Lmax,D] BF16, Hq % Hkv == 0, D <= 512 (D = 128
 *   with Hq/Hkv in {1,2,4} runs on the matrix-core flash kernel, other
 *   shapes on the general GQA kernel with f32 probabilities);
 *   starts I32 [B] (device): row i of sequence b sits at position
 *   starts[b] + i and sees keys 0 .. starts[b] + i; entries are clamped by
 *   the kernel into [0, Lmax - S]; S <= Lmax;
 *   scale: <= 0 selects 1/sqrt(D).
 * out [B,S,Hq,D] F32|BF16. Scores use q in f32 accuracy (bf16 hi + lo
 * parts), probabilities enter P.V rounded to bf16, f32 accumulation. */
int rxw8_gqa_prefill(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k_cache,
                     rxw8_buffer *v_cache, rxw8_buffer *starts, float scale,
                     int out_dtype, rxw8_buffer **out);
int rxw8_gqa_prefill_into(rxw8_runtime *rt, rxw8_buffer *q,
                          rxw8_buffer *k_cache, rxw8_buffer *v_cache,
                          rxw8_buffer *starts, float scale, rxw8_buffer *out);

/* Tensor::argmax(axis, keep_dims) (crates/rxla-core/src/indexing.rs:350-374):
 * index of the first maximum along `axis` of an F32 tensor, as I32 with that
 * axis removed (keep_dims: kept with length 1). Ties choose the lowest index;
 * a NaN beats every number and the first NaN wins. INVALID_ARGUMENT unless
 * 0 <= axis < rank and 0 < dims[axis] <= INT32_MAX; other empty axes give an
 * empty result. The same two kernels end every decoder step (greedy ids). */
int rxw8_argmax(rxw8_runtime *rt, rxw8_buffer *x, int axis, int keep_dims,
                rxw8_buffer **out);

/* KvCache::update_at / update_at_checked (kv_cache.rs:53-111): paired
 * dynamic_update_slice of k_update/v_update (equal shapes, rank = cache rank,
 * same dtype) into k_cache/v_cache in place, at `starts` (device I32 [rank]).
 * Unchecked: each start is clamped to [0, dim - update_dim]
 * (indexing.rs:663-678). Checked: the update happens only when every start
 * lies in that range; otherwise both caches stay unchanged. accepted
 * (optional, device F32 scalar [] or [1]) receives 1 or 0. */
int rxw8_kv_update_at(rxw8_runtime *rt, rxw8_buffer *k_cache,
                      rxw8_buffer *v_cache, rxw8_buffer *k_update,
                      rxw8_buffer *v_update, rxw8_buffer *starts, int checked,
                      rxw8_buffer *accepted);

/* ---- safetensors checkpoints (crates/rxla-safetensors/src/model.rs:340-440;
 *      the W8 layout written by benchmarks/quantize_qwen3_5_w8.py:27-55) ----
 * The file is memory-mapped and every header entry is validated at open
 * (known dtype, offsets inside the data section matching numel, no overlap);
 * payloads are read only by rxw8_safetensors_upload. Tensors of dtypes with no
 * rxw8 counterpart (I64, F64, ...) are listed with dtype 0 and cannot be
 * uploaded. The handle is immutable after open; it must outlive no runtime. */
typedef struct rxw8_safetensors rxw8_safetensors;

int rxw8_safetensors_open(const char *path, rxw8_safetensors **out);
int rxw8_safetensors_close(rxw8_safetensors *st);
int rxw8_safetensors_num_tensors(rxw8_safetensors *st, int64_t *count);
/* name stays valid until close; dims receives up to RXW8_MAX_RANK values */
int rxw8_safetensors_tensor_info(rxw8_safetensors *st, int64_t index,
                                 const char **name, int *dtype, int64_t *dims,
                                 int *rank);
/* NOT_FOUND when absent */
int rxw8_safetensors_find(rxw8_safetensors *st, const char *name,
                          int64_t *index);
/* "__metadata__" string value (e.g. "format", "group_size"); NOT_FOUND when absent */
int rxw8_safetensors_metadata(rxw8_safetensors *st, const char *key,
                              const char **value);
/* Copy tensor `index` into dst at element offset `offset` (elements of dst's
 * dtype), converting as the reference loader does: U8 -> U8 and I32 -> I32
 * verbatim; F32 / F16 / BF16 -> F32 / F16 / BF16 exactly when widening or
 * equal, round-to-nearest-even when narrowing. Several tensors may fill one
 * buffer (fused projections: q, k, v rows one after another). */
int rxw8_safetensors_upload(rxw8_safetensors *st, int64_t index,
                            rxw8_buffer *dst, int64_t offset);

/* ---- decoder plan (AppliedModel::compile -> CompiledModel::bind_parameters
 *      -> run, applied.rs:135-239,808-815; model composition
 *      crates/rxla-models/src/qwen3_5/mod.rs:199-273) ------------------------ */

typedef struct rxw8_decoder_config {
  int64_t layers, hidden, q_heads, kv_heads, head_dim, intermediate, vocab;
  int64_t max_batch, max_seq; /* KV capacity */
  int64_t group;              /* W8 group size; 0 = per output channel (every projection) */
  float eps, theta;
  int32_t qk_norm; /* per-head q/k RMSNorm before RoPE */
} rxw8_decoder_config;

typedef struct rxw8_decoder rxw8_decoder;

/* Validate the config and allocate the KV cache and activations. */
int rxw8_decoder_create(rxw8_runtime *rt, const rxw8_decoder_config *cfg,
                        rxw8_decoder **out);
int rxw8_decoder_destroy(rxw8_decoder *dec);
/* Number of parameter paths and the i-th path / dtype / dims (schema). */
int rxw8_decoder_num_parameters(rxw8_decoder *dec, int *count);
int rxw8_decoder_parameter_info(rxw8_decoder *dec, int index, const char **path,
                                int *dtype, int64_t *dims, int *rank);
/* Bind one parameter by path (order_parameters / validate_buffer,
 * applied.rs:948-990,1274): NOT_FOUND for an unknown path, ALREADY_EXISTS
 * for a second binding, INVALID_ARGUMENT for a shape/dtype mismatch. The
 * decoder retains the buffer. */
int rxw8_decoder_bind_parameter(rxw8_decoder *dec, const char *path,
                                rxw8_buffer *buffer);
/* Reset every sequence length to 0 (cache contents become unreachable). */
int rxw8_decoder_reset(rxw8_decoder *dec);
/* Run `s` tokens per sequence for `b` sequences (ids device I32 [b, s]),
 * starting at each sequence's current length: prefill when s > 1, one decode
 * step when s == 1. FAILED_PRECONDITION when a parameter is unbound,
 * OUT_OF_RANGE when a sequence would exceed max_seq (nothing is mutated).
 * next_ids (device I32 [b]) receives the greedy argmax of the last position's
 * logits; logits (optional, device F32 [b, vocab]) receives those logits. */
int rxw8_decoder_forward(rxw8_decoder *dec, rxw8_buffer *ids, int64_t b,
                         int64_t s, rxw8_buffer *next_ids, rxw8_buffer *logits);
/* Teacher forcing, for parity tests that isolate each layer's own error (no
 * counterpart in the reference, whose compiled model runs whole): layers
 * [first, last) of one forward step of s tokens for b sequences, run as
 * rxw8_decoder_forward runs them, with the residual stream entering layer
 * `first` read from hidden_in (device F32 [b, s, hidden]) instead of the
 * embedding. The tokens sit at each sequence's current length; every layer
 * run appends its k/v there. hidden_out (device F32 [b, s, hidden]) receives
 * the residual stream leaving layer last - 1. With logits (device F32
 * [b, vocab]; needs last == layers) the step's tail runs too: final norm of
 * the last position and lm_head. commit != 0 advances every length by s (once
 * per step, with its last layer). INVALID_ARGUMENT unless 0 <= first < last
 * <= layers and the shapes match; otherwise as rxw8_decoder_forward. */
int rxw8_decoder_forward_layers(rxw8_decoder *dec, rxw8_buffer *hidden_in,
                                int64_t b, int64_t s, int64_t first,
                                int64_t last, rxw8_buffer *hidden_out,
                                rxw8_buffer *logits, int commit);
/* Prefill `prompt` (device I32 [b, s]) then `steps` greedy decode steps;
 * out_ids (device I32 [b, steps + 1]) receives the token chosen after the
 * prompt followed by one token per decode step. With use_graph != 0 the
 * decode step is captured once into a HIP graph and replayed. */
int rxw8_decoder_generate(rxw8_decoder *dec, rxw8_buffer *prompt, int64_t b,
                          int64_t s, int64_t steps, rxw8_buffer *out_ids,
                          int use_graph);
/* Copy of the current sequence lengths to host (int32 [max_batch]). */
int rxw8_decoder_lens(rxw8_decoder *dec, int32_t *lens, int64_t n);

/* ---- Qwen3.5 hybrid W8 text model ------------------------------------------
 * Replaces qwen3_5(cx, token_ids, config) (crates/rxla-models/src/qwen3_5/
 * mod.rs:197-273) compiled and bound through the applied-model flow
 * (crates/rxla-nn/src/applied.rs:156-239): full-sequence inference, token ids
 * [batch, sequence] -> logits [batch, sequence, vocabulary], every sequence
 * starting at position 0. Gated-delta linear-attention layers
 * (qwen3_5/layers.rs:113-268) and output-gated full-attention layers
 * (:28-100), the SwiGLU MLP (:270-293), the W8 embedding and tied W8 LM head
 * (mod.rs:134-195, optional F32 LoRA on the head). The fields follow
 * Qwen3_5Config (mod.rs:16-33); layer i is full attention iff
 * layer_kinds[i] != 0 (or, with layer_kinds NULL, iff (i + 1) %
 * full_attention_interval == 0, the 0.8B topology with interval 4). */
typedef struct rxw8_qwen35_config {
  int64_t vocab, hidden, intermediate, layers;
  int64_t heads, kv_heads, head_dim;      /* full attention */
  int64_t linear_heads, linear_head_dim;  /* gated delta */
  int64_t conv_kernel, max_positions, rotary_dim, group;
  int64_t full_attention_interval;
  const int32_t *layer_kinds; /* [layers] 0 = linear, 1 = full (copied at create), or NULL */
  float theta, eps;
  int64_t lora_rank; /* 0 = no LoRA on the tied head */
  float lora_alpha;
  int64_t max_batch, max_seq; /* activation capacity of one forward */
  /* Compute dtype of every projection: RXW8_F32 (also selected by 0), the
   * reference's: qwen3_5/layers.rs:4-9 takes cx.layer_compute_dtype(), which
   * qwen3_5() leaves at the Cx default F32 (rxla-nn lib.rs:432); activations
   * stay f32 throughout. RXW8_BF16 is an opt-in (with_layer_compute_dtype):
   * bf16(x) . bf16(W) rounded to bf16, on the packed W8A16 GEMV / GEMM. */
  int32_t compute_dtype;
} rxw8_qwen35_config;

typedef struct rxw8_qwen35 rxw8_qwen35;

/* Validate the config (Qwen3_5Config::validate, mod.rs:100-131, plus the
 * widths the kernels support) and allocate activations. */
int rxw8_qwen35_create(rxw8_runtime *rt, const rxw8_qwen35_config *cfg,
                       rxw8_qwen35 **out);
int rxw8_qwen35_destroy(rxw8_qwen35 *m);
/* Parameter schema under the reference's paths ("model.language_model.
 * layers.{i}.linear_attn.in_proj_qkv.weight", ...): U8 codes + F32 scales
 * for every projection, F32 norms / conv / A_log / dt_bias. */
int rxw8_qwen35_num_parameters(rxw8_qwen35 *m, int *count);
int rxw8_qwen35_parameter_info(rxw8_qwen35 *m, int index, const char **path,
                               int *dtype, int64_t *dims, int *rank);
/* Same contract as rxw8_decoder_bind_parameter (applied.rs:948-990,1274). */
int rxw8_qwen35_bind_parameter(rxw8_qwen35 *m, const char *path,
                               rxw8_buffer *buffer);
/* ids: device I32 [b, s]; logits: device F32 [b, s, vocab]. INVALID_ARGUMENT
 * for a sequence outside [1, max_positions] (InvalidQwenTokens, mod.rs:
 * 201-209) or a shape mismatch, OUT_OF_RANGE beyond the activation capacity,
 * FAILED_PRECONDITION while a parameter is unbound. */
int rxw8_qwen35_forward(rxw8_qwen35 *m, rxw8_buffer *ids, rxw8_buffer *logits);

/* ---- XLA GPU custom-call handlers ------------------------------------------
 * For a PJRT plugin's GPU custom-call registration
 * (crates/rxla-pjrt/src/runtime.rs:380-428, GpuCustomCallApi::Legacy) of the
 * calls the reference appends with CustomCall (crates/rxla-core/src/
 * tensor_handle.rs:276-345, api_version 2 = status-returning). XLA's untyped
 * GPU signature: `stream` is the hipStream_t of the call, `buffers` the
 * operand device pointers in order and then the result's, `opaque` the
 * backend_config text ("key=value;..."), `status` XLA's XlaCustomCallStatus*
 * (failures are reported through XlaCustomCallStatusSetFailure when the
 * process exports it, and always through rxw8_last_error; nothing launches).
 * Each runs the matching `_into` entry point on the current device.
 *   rxw8_quantized_linear: [x [m,k], weight U8 [n,k], scale F32 [n,k/g]] ->
 *     y [m,n]; keys m, n, k, g, x, y (dtype names f32 / bf16), compute
 *     (bf16 by default, or f32).
 *   rxw8_gqa_decode: [q [b,hq,d], k_cache, v_cache [b,hkv,lmax,d], lens I32
 *     [b]] -> out [b,hq,d]; keys b, hq, hkv, lmax, d, q, cache, out, scale
 *     (optional; 1/sqrt(d) when absent).
 *   rxw8_gqa_prefill: [q [b,s,hq,d], k_cache, v_cache BF16 [b,hkv,lmax,d],
 *     starts I32 [b]] -> out [b,s,hq,d]; keys b, s, hq, hkv, lmax, d (128),
 *     q, out, scale (optional). */
void rxw8_xla_quantized_linear(void *stream, void **buffers, const char *opaque,
                               size_t opaque_len, void *status);
void rxw8_xla_gqa_decode(void *stream, void **buffers, const char *opaque,
                         size_t opaque_len, void *status);
void rxw8_xla_gqa_prefill(void *stream, void **buffers, const char *opaque,
                          size_t opaque_len, void *status);

/* ---- XLA typed-FFI handlers (HLO api_version 4) ----------------------------
 * The same three calls for the reference's default custom-call form,
 * CustomCall::typed_ffi (crates/rxla-core/src/tensor_handle.rs:278-300,
 * api_version 4), registered as GpuCustomCallApi::TypedFfi with an execute
 * handler (crates/rxla-pjrt/src/runtime.rs:265-308,395-428). Each is an
 * XLA_FFI_Handler of XLA's FFI C API 0.1 (xla/ffi/api/c_api.h): call_frame is
 * an XLA_FFI_CallFrame*, and the return value NULL or an XLA_FFI_Error* made
 * with the frame's api->XLA_FFI_Error_Create (code = the rxw8_status, which is
 * XLA's numbering). A frame carrying the metadata extension is answered with
 * API version 0.1 and no traits; stages other than execute do nothing. Shapes
 * and dtypes come from the buffers (XLA_FFI_DataType S32, U8, F16, F32, BF16),
 * the stream from api->XLA_FFI_Stream_Get, options from the backend_config
 * dictionary's attributes. Malformed frames (operand count, non-buffer
 * operands, other dtypes, attribute kinds) fail before any device work.
 *   rxw8_xla_ffi_quantized_linear: x [..., k], weight U8 [n, k] or packed,
 *     scale F32 [n, k/g] -> y [..., n]; compute = "bf16" (default) | "f32".
 *   rxw8_xla_ffi_gqa_decode: q [b, hq, d], k_cache, v_cache [b, hkv, lmax, d],
 *     lens S32 [b] -> out [b, hq, d]; scale (optional f32 / f64 scalar).
 *   rxw8_xla_ffi_gqa_prefill: q [b, s, hq, d], k_cache, v_cache BF16, starts
 *     S32 [b] -> out [b, s, hq, d]; scale (optional). */
void *rxw8_xla_ffi_quantized_linear(void *call_frame);
void *rxw8_xla_ffi_gqa_decode(void *call_frame);
void *rxw8_xla_ffi_gqa_prefill(void *call_frame);

#ifdef __cplusplus
}
#endif

#endif /* RXW8_H */
