// Decoder plan: a compiled, fixed-schedule Qwen-style dense W8 decoder.
//
// Mirrors the reference's model ABI flow (crates/rxla-nn/src/applied.rs):
// AppliedModel::compile (:808-815) -> CompiledModel::bind_parameters
// (:156-172; path-addressed, validated by order_parameters :948-990 and
// validate_buffer :1274) -> run (:183-239). The layer composition follows
// crates/rxla-models/src/qwen3_5/mod.rs:199-273 (embed, per-layer pre-norm
// attention and SwiGLU blocks with residuals, final norm, tied lm_head) with
// dense full-attention layers (layers.rs:28-101, no output gate) and the fused
// projection groups of crates/rxla-models/src/qwen_image_2_1/projections.rs
// (qkv_proj = [q; k; v] rows, gate_up_proj = [gate; up] rows).
//
// Parameter schema (paths, dtype, shape):
//   embed_tokens.weight                      BF16 [V, H]   (also the lm_head)
//   layers.{l}.input_layernorm.weight        F32  [H]
//   layers.{l}.self_attn.qkv_proj.{weight,scale}  U8 [(Hq+2Hkv)D, H], F32 [.., H/G]
//   layers.{l}.self_attn.{q_norm,k_norm}.weight   F32 [D]    (qk_norm only)
//   layers.{l}.self_attn.o_proj.{weight,scale}    U8 [H, Hq D], F32 [H, Hq D/G]
//   layers.{l}.post_attention_layernorm.weight    F32 [H]
//   layers.{l}.mlp.gate_up_proj.{weight,scale}    U8 [2I, H], F32 [2I, H/G]
//   layers.{l}.mlp.down_proj.{weight,scale}       U8 [H, I], F32 [H, I/G]
//   norm.weight                                   F32 [H]
// G = config.group, or each linear's input width when group == 0
// (per-output-channel scales).
#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "internal.h"

namespace rxw8 {

int qlinear_launch(Runtime *rt, const void *x, int x_f32, const uint8_t *w, bool packed,
                   const float *s, void *y, int y_f32, int64_t M, int64_t N, int64_t K,
                   int64_t G, int compute_bf16, int y_mode);
int bf16_linear_launch(Runtime *rt, const void *x, int x_f32, const uint16_t *w, bool packed,
                       void *y, int y_f32, int64_t M, int64_t N, int64_t K);
bool prefill_supported(int64_t Hq, int64_t Hkv, int64_t D, int cache_f32);
bool gemm_eligible(int64_t M, int64_t N, int64_t K, int64_t G);
int prefill_launch(Runtime *rt, const void *q, int q_f32, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                   const uint16_t *kc, const uint16_t *vc, const int32_t *starts,
                   const int32_t *slots, void *out, int out_f32, int64_t o_sb, int64_t o_ss,
                   int64_t o_sh, int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t Lmax,
                   float scale);

// Kernel argument structs (match kernels/decoder.hip and w8a16_gemv.hip).
struct EmbedArgs {
  const int32_t *ids;
  const uint16_t *table;
  float *h;
  float *ss;
  int64_t T, V, H;
  const int32_t *lens;
  int32_t *pos, *row_seq, *row_len;
  int s;
  const float *xw_norm = nullptr;
  uint16_t *xw = nullptr;
};
struct LoadRowsArgs {
  const float *h_in;
  float *h;
  float *ss;
  int64_t H;
  const int32_t *lens;
  int32_t *pos, *row_seq, *row_len;
  int s;
  const float *xw_norm;
  uint16_t *xw;
};
struct InterleaveArgs {
  const float *src;
  float *dst;
  int64_t half, cols;
};
struct RmsNormArgs {
  const float *x;
  const float *w;
  uint16_t *y;
  const int32_t *src_row;
  int64_t H;
  int rows;
  int src_stride, src_offset;
  float eps;
};
struct RopeTableArgs {
  const float *freqs;
  float *tab;
  int half;
};
struct QkRopeArgs {
  const uint16_t *qkv;
  const float *q_norm, *k_norm, *rope;
  const int32_t *pos, *row_seq;
  float *q_out;
  uint16_t *kc, *vc;
  int T, Hq, Hkv, D, Lmax;
  float eps;
};
struct SiluMulArgs {
  const uint16_t *gu;
  uint16_t *act;
  int64_t T, I;
  int interleaved;
};
struct ArgmaxArgs {
  const float *x;
  float *pval;
  int32_t *pidx;
  int32_t *out;
  int64_t cols;
  int rows, chunks;
  int64_t inner;
};
struct PackArgs {
  const void *src;
  void *dst;
  int64_t n, k;
  int kb;
  int esize;
  int64_t ilv_half;
};
struct ArgmaxFinalArgs {
  const float *pval;
  const int32_t *pidx;
  int32_t *next;
  int32_t *lens;
  int32_t *rec_out;
  int32_t *rec_step;
  int rows, chunks, s, ncols;
  const uint16_t *table = nullptr;  // optional: embed the winners (generate)
  float *h = nullptr;
  float *ss = nullptr;
  int32_t *pos = nullptr, *row_seq = nullptr, *row_len = nullptr;
  int64_t V = 0, H = 0;
  const float *xw_norm = nullptr;
  uint16_t *xw = nullptr;
};
struct RecordArgs {
  const int32_t *next;
  int32_t *out;
  int32_t *step;
  int b, ncols;
};

enum ParamKind { P_EMBED, P_IN_NORM, P_QKV_W, P_QKV_S, P_QN, P_KN, P_O_W, P_O_S, P_POST_NORM,
                 P_GU_W, P_GU_S, P_DOWN_W, P_DOWN_S, P_FINAL_NORM };

struct ParamSpec {
  std::string path;
  int kind = 0, layer = -1;
  int dtype = 0, rank = 0;
  int64_t dims[2] = {0, 0};
  Buffer *bound = nullptr;   // retained caller buffer
  Buffer *packed = nullptr;  // tiled copy owned by the decoder (U8 weights, embedding)
  Buffer *perm = nullptr;    // gate|up scales in SwiGLU row order (owned by the decoder)
};

struct Decoder {
  Runtime *rt = nullptr;
  rxw8_decoder_config cfg{};
  int64_t H = 0, D = 0, Hq = 0, Hkv = 0, I = 0, V = 0, QKV = 0, L = 0, Bmax = 0, Lmax = 0;
  std::vector<ParamSpec> params;
  std::unordered_map<std::string, int> index;
  std::vector<int> by_layer_kind;  // [layer * 14 + kind] -> param index (or -1)
  // device state
  void *kc = nullptr, *vc = nullptr;
  size_t cache_bytes = 0;
  int32_t *d_lens = nullptr, *d_step = nullptr;
  std::vector<int32_t> h_lens;
  float *d_freqs = nullptr;
  float *d_rope = nullptr;  // [Lmax, D] cos / sin table
  // activations (capacity cap_T tokens)
  int64_t cap_T = 0;
  float *h = nullptr, *q = nullptr;
  uint16_t *xn = nullptr, *qkv = nullptr, *attn = nullptr, *gu = nullptr, *act = nullptr;
  int32_t *pos = nullptr, *row_seq = nullptr, *row_len = nullptr;
  size_t act_bytes = 0;
  void *act_block = nullptr;
  // tail (max_batch rows)
  uint16_t *xl = nullptr;
  float *logits = nullptr, *am_val = nullptr;
  int32_t *am_idx = nullptr, *next = nullptr, *ids1 = nullptr;
  // sums of squares of residual rows for the fused schedule (<= 32 tokens):
  // embedding rows [T]; o_proj and down partials [H/16][T]
  float *ss_embed = nullptr, *ss_o = nullptr, *ss_down = nullptr;
  bool gu_ilv = false;  // gate|up weights and scales stored in SwiGLU row order
  void *tail_block = nullptr;
  size_t tail_bytes = 0;
  int am_chunks = 64;  // argmax partials per row; <= 64 (one lane each in the final pass)
  // decode-step graph and the values it bakes in (see graph_key)
  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  int64_t g_key[10] = {-1};

  const ParamSpec &p(int layer, int kind) const {
    return params[by_layer_kind[(size_t)(layer < 0 ? 0 : layer) * 14 + kind]];
  }
  int64_t group_for(int64_t k) const { return cfg.group > 0 ? cfg.group : k; }
};

static void add_param(Decoder *d, const std::string &path, int kind, int layer, int dtype,
                      int64_t d0, int64_t d1) {
  ParamSpec s;
  s.path = path;
  s.kind = kind;
  s.layer = layer;
  s.dtype = dtype;
  s.rank = d1 > 0 ? 2 : 1;
  s.dims[0] = d0;
  s.dims[1] = d1;
  d->index[path] = (int)d->params.size();
  d->by_layer_kind[(size_t)(layer < 0 ? 0 : layer) * 14 + kind] = (int)d->params.size();
  d->params.push_back(s);
}

static void free_decoder_memory(Decoder *d) {
  Runtime *rt = d->rt;
  if (d->gexec) (void)hipGraphExecDestroy(d->gexec);
  if (d->graph) (void)hipGraphDestroy(d->graph);
  d->gexec = nullptr;
  d->graph = nullptr;
  (void)hipStreamSynchronize(rt->stream);
  for (void *p : {d->kc, d->vc, (void *)d->d_lens, (void *)d->d_freqs, (void *)d->d_rope,
                  d->act_block, d->tail_block})
    if (p) (void)hipFree(p);
  for (ParamSpec &s : d->params) {
    if (s.bound) rxw8_buffer_release(static_cast<rxw8_buffer *>(s.bound));
    if (s.packed) rxw8_buffer_release(static_cast<rxw8_buffer *>(s.packed));
    if (s.perm) rxw8_buffer_release(static_cast<rxw8_buffer *>(s.perm));
  }
}

static int ensure_activations(Decoder *d, int64_t T) {
  if (T <= d->cap_T) return RXW8_OK;
  Runtime *rt = d->rt;
  if (d->act_block) {
    RXW8_HIP(hipStreamSynchronize(rt->stream));
    RXW8_HIP(hipFree(d->act_block));
    d->act_block = nullptr;
  }
  auto al = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t sz_h = al(T * d->H * 4), sz_q = al(T * d->Hq * d->D * 4);
  const size_t sz_xn = al(T * std::max(d->H, d->I) * 2), sz_qkv = al(T * d->QKV * 2);
  const size_t sz_attn = al(T * d->Hq * d->D * 2), sz_gu = al(T * 2 * d->I * 2);
  const size_t sz_act = al(T * d->I * 2), sz_i = al(T * 4);
  const size_t total = sz_h + sz_q + sz_xn + sz_qkv + sz_attn + sz_gu + sz_act + 3 * sz_i;
  RXW8_HIP(hipMalloc(&d->act_block, total));
  char *p = (char *)d->act_block;
  d->h = (float *)p; p += sz_h;
  d->q = (float *)p; p += sz_q;
  d->xn = (uint16_t *)p; p += sz_xn;
  d->qkv = (uint16_t *)p; p += sz_qkv;
  d->attn = (uint16_t *)p; p += sz_attn;
  d->gu = (uint16_t *)p; p += sz_gu;
  d->act = (uint16_t *)p; p += sz_act;
  d->pos = (int32_t *)p; p += sz_i;
  d->row_seq = (int32_t *)p; p += sz_i;
  d->row_len = (int32_t *)p; p += sz_i;
  d->cap_T = T;
  d->act_bytes = total;
  return RXW8_OK;
}

// What a captured decode step depends on beyond the decoder's fixed state.
static void graph_key(const Decoder *d, int64_t b, int64_t ncols, const void *out, int64_t key[10]) {
  const Runtime *rt = d->rt;
  const void *ptrs[7] = {out, d->act_block, rt->partials.ptr, rt->scratch.ptr, rt->xcast.ptr,
                         rt->wdeq.ptr, rt->attn_counters.ptr};
  key[0] = b;
  key[1] = ncols;
  key[2] = d->cap_T;
  for (int i = 0; i < 7; ++i) key[3 + i] = (int64_t)(intptr_t)ptrs[i];
}

// Whether a fused step of T rows applies the RMSNorms after the projections:
// the row-norm GEMV kernels take packed weights, up to 16 rows and at most
// 256 sum-of-squares partials per row (H <= 4096).
static bool row_norm_enabled(const Decoder *d, int64_t T) {
  const char *env = std::getenv("RXW8_DEC_ROW_NORM");
  return !(env && *env == '0') && T <= 16 && d->H % 16 == 0 && d->H / 16 <= 256 &&
         d->p(0, P_QKV_W).packed && d->p(0, P_GU_W).packed;
}

static unsigned blocks(int64_t n, int per = 256) { return (unsigned)std::max<int64_t>(1, (n + per - 1) / per); }

// Part of a forward step run by the teacher-forcing entry point: the residual
// rows entering layer `first` come from h_in (instead of the embedding),
// layers [first, last) run, and the tail (final norm, lm_head, argmax) runs
// only with `tail` (last == layers), advancing the device lengths only with
// `advance`.
struct LayerRange {
  const float *h_in = nullptr;
  int first = 0, last = 0;
  bool tail = false, advance = false;
};

// Enqueue one forward pass over ids[b, s] (device) starting at the current
// lengths; writes next ids and logits of the last position; advances lengths.
// rec (generate): also store the chosen ids in column *rec->step of rec->out.
// embedded: h, the positions and (fused) ss_embed already hold this step's
// input rows -- written by the previous step's argmax launch, which embeds
// its winners when embed_next is set (generate's decode steps: ids == next,
// s == 1 for the following step).
static int enqueue_forward(Decoder *d, const int32_t *ids, int64_t b, int64_t s,
                           const RecordArgs *rec = nullptr, bool embedded = false,
                           bool embed_next = false, const LayerRange *range = nullptr) {
  Runtime *rt = d->rt;
  const int64_t T = b * s;
  const int l_first = range ? range->first : 0, l_end = range ? range->last : (int)d->L;
  int rc;
  // Decode-sized steps run the fused schedule, 7 launches per layer: the
  // residual-writing GEMVs (o_proj, down) also emit per-16-channel sums of
  // squares of the new residual rows, from which the next projection (QKV,
  // gate|up) forms the RMSNorm scale while it stages its activations; gate|up
  // applies SiLU*up in its epilogue (weights in 8 gate + 8 up row tiles); no
  // split-K reduce launches. It needs every projection in one GEMV launch.
  // Longer inputs (prefill) use the GEMM and separate norm/SwiGLU kernels.
  const char *unfused = std::getenv("RXW8_DEC_UNFUSED");
  const bool fused =
      T <= 32 && !(unfused && *unfused == '1') && d->gu_ilv && d->H % 16 == 0 &&
      gemv_single_launch(rt, T, d->QKV, d->H, d->group_for(d->H)) &&
      gemv_single_launch(rt, T, d->H, d->Hq * d->D, d->group_for(d->Hq * d->D)) &&
      gemv_single_launch(rt, T, 2 * d->I, d->H, d->group_for(d->H)) &&
      gemv_single_launch(rt, T, d->H, d->I, d->group_for(d->I));
  // Prompts of 16 or more rows per sequence take the causal prefill kernel
  // (K/V read once per 64 rows instead of once per row).
  const char *no_prefill = std::getenv("RXW8_DEC_ROWWISE_PREFILL");
  const bool use_prefill = s >= 16 && prefill_supported(d->Hq, d->Hkv, d->D, 0) &&
                           !(no_prefill && *no_prefill == '1');
  // RoPE and the KV append fold into the attention launch when every row is a
  // different sequence's single new token and the D = 128 kernel runs.
  const char *unfused_rope = std::getenv("RXW8_DEC_UNFUSED_ROPE");
  const bool fused_rope = fused && s == 1 && d->D == 128 && d->Hq % d->Hkv == 0 &&
                          (d->Hq / d->Hkv == 1 || d->Hq / d->Hkv == 2 || d->Hq / d->Hkv == 4 ||
                           d->Hq / d->Hkv == 8) &&
                          !(unfused_rope && *unfused_rope == '1');
  // Fused steps apply each RMSNorm after its projection: the producer of the
  // residual rows (embedding, o_proj, down) also writes bf16(h * norm weight)
  // into xn, and the next projection's GEMV reads those rows and multiplies
  // each row's result by 1/sqrt(mean(h^2) + eps), formed from the producer's
  // sum-of-squares partials. Off the critical path of the weight stream,
  // unlike normalising the rows while staging them (RXW8_DEC_ROW_NORM=0).
  const bool rn = fused && row_norm_enabled(d, T);
  const float *in_norm0 = (const float *)d->p(0, P_IN_NORM).bound->ptr;
  if (range) {
    // the caller's residual rows enter layer l_first (positions as embedded)
    LoadRowsArgs a{range->h_in, d->h, fused ? d->ss_embed : nullptr, d->H, d->d_lens, d->pos,
                   d->row_seq, d->row_len, (int)s, nullptr, nullptr};
    if (rn) a.xw_norm = (const float *)d->p(l_first, P_IN_NORM).bound->ptr, a.xw = d->xn;
    if ((rc = launch(rt, "rxw8_dec_load_rows", dim3((unsigned)T), dim3(256), a))) return rc;
  } else if (!embedded) {
    const ParamSpec &e = d->p(-1, P_EMBED);
    // the embedding launch also writes the token positions
    EmbedArgs a{ids, (const uint16_t *)e.bound->ptr, d->h, fused ? d->ss_embed : nullptr, T, d->V,
                d->H, d->d_lens, d->pos, d->row_seq, d->row_len, (int)s};
    if (rn) a.xw_norm = in_norm0, a.xw = d->xn;
    if ((rc = launch(rt, "rxw8_dec_embed", dim3((unsigned)T), dim3(256), a))) return rc;
  }
  const size_t layer_cache = (size_t)d->Bmax * d->Hkv * d->Lmax * d->D;
  const float scale = 1.0f / std::sqrt((float)d->D);
  for (int l = l_first; l < l_end; ++l) {
    auto wptr = [&](int kind) -> const uint8_t * {
      const ParamSpec &ps = d->p(l, kind);
      return (const uint8_t *)(ps.packed ? ps.packed->ptr : ps.bound->ptr);
    };
    auto packed = [&](int kind) { return d->p(l, kind).packed != nullptr; };
    auto fptr = [&](int kind) {
      const ParamSpec &ps = d->p(l, kind);
      return (const float *)(ps.perm ? ps.perm->ptr : ps.bound->ptr);
    };
    // input RMSNorm -> fused QKV projection. Decode-sized steps fold the norm
    // into the GEMV's activation staging (one launch instead of two).
    if (fused) {
      GemvOptions o;
      o.mode = rn ? 0 : 3, o.row_norm = rn, o.norm_w = fptr(P_IN_NORM), o.eps = d->cfg.eps;
      o.prefer_ks1 = true;
      o.ss_in = l == l_first ? d->ss_embed : d->ss_down;
      o.ss_parts = l == l_first ? 1 : (int)(d->H / 16);
      if ((rc = gemv_launch(rt, rn ? (const void *)d->xn : (const void *)d->h, rn ? 0 : 1,
                            wptr(P_QKV_W), false, packed(P_QKV_W), fptr(P_QKV_S), d->qkv, 0, T,
                            d->QKV, d->H, d->group_for(d->H), 0, o)))
        return rc;
    } else {
      RmsNormArgs a{d->h, fptr(P_IN_NORM), d->xn, nullptr, d->H, (int)T, 1, 0, d->cfg.eps};
      if ((rc = launch(rt, "rxw8_dec_rmsnorm", dim3((unsigned)T), dim3(256), a))) return rc;
      if ((rc = qlinear_launch(rt, d->xn, 0, wptr(P_QKV_W), packed(P_QKV_W), fptr(P_QKV_S),
                               d->qkv, 0, T, d->QKV, d->H, d->group_for(d->H), 1, 0)))
        return rc;
    }
    uint16_t *kcl = (uint16_t *)d->kc + (size_t)l * layer_cache;
    uint16_t *vcl = (uint16_t *)d->vc + (size_t)l * layer_cache;
    if (fused_rope) {
      // one new token per sequence: q/k norm + RoPE + KV append inside attention
      AttnRope rp{d->qkv,
                  d->cfg.qk_norm ? fptr(P_QN) : nullptr,
                  d->cfg.qk_norm ? fptr(P_KN) : nullptr,
                  d->d_rope, d->cfg.eps};
      if ((rc = attention_launch(rt, d->qkv, 0, kcl, vcl, 0, d->row_len, d->row_seq, nullptr, 0, 0,
                                 d->attn, 0, T, d->Hq, d->Hkv, d->Lmax, d->D, scale, &rp)))
        return rc;
    } else {
      QkRopeArgs a{d->qkv,
                   d->cfg.qk_norm ? fptr(P_QN) : nullptr,
                   d->cfg.qk_norm ? fptr(P_KN) : nullptr,
                   d->d_rope, d->pos, d->row_seq, d->q, kcl, vcl, (int)T, (int)d->Hq, (int)d->Hkv,
                   (int)d->D, (int)d->Lmax, d->cfg.eps};
      const int64_t rows = T * (d->Hq + 2 * d->Hkv);
      const char *generic_rope = std::getenv("RXW8_DEC_GENERIC_ROPE");
      if (d->D == 128 && !(generic_rope && *generic_rope == '1')) {  // 8 lanes per (token, head) row
        if ((rc = launch(rt, "rxw8_dec_qk_rope_kv_d128", dim3(blocks(rows, 32)), dim3(256), a)))
          return rc;
      } else if ((rc = launch(rt, "rxw8_dec_qk_rope_kv", dim3(blocks(rows, 4)), dim3(256), a))) {
        return rc;
      }
      if (use_prefill) {
        // causal blocks of 64 prompt rows per (sequence, kv head); lens still
        // holds each sequence's length before this forward = its first position
        const int64_t rs = d->Hq * d->D;
        if ((rc = prefill_launch(rt, d->q, 1, s * rs, rs, d->D, kcl, vcl, d->d_lens, nullptr,
                                 d->attn, 0, s * rs, rs, d->D, b, s, d->Hq, d->Hkv, d->Lmax,
                                 scale)))
          return rc;
      } else if ((rc = attention_launch(rt, d->q, 1, kcl, vcl, 0, d->row_len, d->row_seq, nullptr,
                                        0, 0, d->attn, 0, T, d->Hq, d->Hkv, d->Lmax, d->D, scale))) {
        return rc;
      }
    }
    if (fused) {
      GemvOptions o;
      o.prefer_ks1 = true, o.ss_out = d->ss_o;
      if (rn) o.xw_norm = fptr(P_POST_NORM), o.xw_out = d->xn;
      if ((rc = gemv_launch(rt, d->attn, 0, wptr(P_O_W), false, packed(P_O_W), fptr(P_O_S), d->h, 1,
                            T, d->H, d->Hq * d->D, d->group_for(d->Hq * d->D), 1, o)))
        return rc;
      GemvOptions g;
      g.mode = rn ? 0 : 3, g.row_norm = rn, g.norm_w = fptr(P_POST_NORM), g.eps = d->cfg.eps;
      g.ss_in = d->ss_o, g.ss_parts = (int)(d->H / 16), g.prefer_ks1 = true, g.swiglu = true;
      if ((rc = gemv_launch(rt, rn ? (const void *)d->xn : (const void *)d->h, rn ? 0 : 1,
                            wptr(P_GU_W), false, packed(P_GU_W), fptr(P_GU_S), d->act, 0, T,
                            2 * d->I, d->H, d->group_for(d->H), 0, g)))
        return rc;
      GemvOptions dn;
      dn.prefer_ks1 = true, dn.ss_out = d->ss_down;
      if (rn) {  // the next layer's input norm, or the final norm after the last layer
        dn.xw_norm = l + 1 < d->L ? (const float *)d->p(l + 1, P_IN_NORM).bound->ptr
                                  : (const float *)d->p(-1, P_FINAL_NORM).bound->ptr;
        dn.xw_out = d->xn;
      }
      if ((rc = gemv_launch(rt, d->act, 0, wptr(P_DOWN_W), false, packed(P_DOWN_W), fptr(P_DOWN_S),
                            d->h, 1, T, d->H, d->I, d->group_for(d->I), 1, dn)))
        return rc;
      continue;
    }
    if ((rc = qlinear_launch(rt, d->attn, 0, wptr(P_O_W), packed(P_O_W), fptr(P_O_S), d->h, 1, T,
                             d->H, d->Hq * d->D, d->group_for(d->Hq * d->D), 1, 1)))
      return rc;
    {
      RmsNormArgs a{d->h, fptr(P_POST_NORM), d->xn, nullptr, d->H, (int)T, 1, 0, d->cfg.eps};
      if ((rc = launch(rt, "rxw8_dec_rmsnorm", dim3((unsigned)T), dim3(256), a))) return rc;
    }
    if (d->gu_ilv && gemm_eligible(T, 2 * d->I, d->H, d->group_for(d->H))) {
      // the GEMM epilogue applies SiLU(gate) * up over the interleaved tiles
      if ((rc = qlinear_launch(rt, d->xn, 0, wptr(P_GU_W), packed(P_GU_W), fptr(P_GU_S), d->act, 0,
                               T, 2 * d->I, d->H, d->group_for(d->H), 1, 2)))
        return rc;
    } else {
      if ((rc = qlinear_launch(rt, d->xn, 0, wptr(P_GU_W), packed(P_GU_W), fptr(P_GU_S), d->gu, 0,
                               T, 2 * d->I, d->H, d->group_for(d->H), 1, 0)))
        return rc;
      SiluMulArgs a{d->gu, d->act, T, d->I, d->gu_ilv ? 1 : 0};
      if ((rc = launch(rt, "rxw8_dec_silu_mul", dim3(blocks(T * d->I, 256 * 4)), dim3(256), a)))
        return rc;
    }
    if ((rc = qlinear_launch(rt, d->act, 0, wptr(P_DOWN_W), packed(P_DOWN_W), fptr(P_DOWN_S), d->h,
                             1, T, d->H, d->I, d->group_for(d->I), 1, 1)))
      return rc;
  }
  if (range && !range->tail) return RXW8_OK;
  // final norm on the last position of each sequence, tied bf16 lm_head, argmax
  const ParamSpec &e = d->p(-1, P_EMBED);
  const bool pk = e.packed != nullptr;
  const uint16_t *ew = (const uint16_t *)(pk ? e.packed->ptr : e.bound->ptr);
  const float *final_norm = (const float *)d->p(-1, P_FINAL_NORM).bound->ptr;
  // single-token steps: every row is a last position, and the lm_head GEMV
  // applies the final norm to the rows the last down projection wrote
  rc = RXW8_UNIMPLEMENTED;
  if (rn && s == 1) {
    GemvOptions o;
    o.row_norm = true, o.ss_in = d->ss_down, o.ss_parts = (int)(d->H / 16), o.eps = d->cfg.eps;
    rc = gemv_launch(rt, d->xn, 0, ew, true, pk, nullptr, d->logits, 1, b, d->V, d->H, d->H, 0, o);
    if (rc && rc != RXW8_UNIMPLEMENTED) return rc;
  }
  if (rc == RXW8_UNIMPLEMENTED) {
    RmsNormArgs a{d->h, final_norm, d->xl, nullptr, d->H, (int)b, (int)s, (int)s - 1, d->cfg.eps};
    if ((rc = launch(rt, "rxw8_dec_rmsnorm", dim3((unsigned)b), dim3(256), a))) return rc;
    if ((rc = bf16_linear_launch(rt, d->xl, 0, ew, pk, d->logits, 1, b, d->V, d->H))) return rc;
  }
  {
    ArgmaxArgs a{d->logits, d->am_val, d->am_idx, d->next, d->V, (int)b, d->am_chunks, 1};
    if ((rc = launch(rt, "rxw8_dec_argmax_partial", dim3((unsigned)(b * d->am_chunks)), dim3(256), a)))
      return rc;
    ArgmaxFinalArgs f{d->am_val, d->am_idx, d->next, range && !range->advance ? nullptr : d->d_lens,
                      rec ? rec->out : nullptr,
                      rec ? rec->step : nullptr, (int)b, d->am_chunks, (int)s, rec ? rec->ncols : 0};
    unsigned threads = 64u * (unsigned)std::min<int64_t>(b, 16);
    if (embed_next) {
      // the next step's input rows (its fused QKV prologue reads ss_embed,
      // sized for the 32 rows a fused step takes)
      f.table = (const uint16_t *)e.bound->ptr, f.h = d->h, f.ss = b <= 32 ? d->ss_embed : nullptr;
      f.pos = d->pos, f.row_seq = d->row_seq, f.row_len = d->row_len, f.V = d->V, f.H = d->H;
      if (row_norm_enabled(d, b)) f.xw_norm = in_norm0, f.xw = d->xn;
      threads = 1024;
    }
    if ((rc = launch(rt, "rxw8_dec_argmax_final", dim3(1), dim3(threads), f))) return rc;
  }
  return RXW8_OK;
}

static int check_ready(Decoder *d, int64_t b, int64_t s) {
  for (const ParamSpec &ps : d->params)
    if (!ps.bound) return fail(RXW8_FAILED_PRECONDITION, "missing parameter binding \"%s\"", ps.path.c_str());
  if (b < 1 || b > d->Bmax)
    return fail(RXW8_INVALID_ARGUMENT, "batch %lld outside [1, %lld]", (long long)b, (long long)d->Bmax);
  if (s < 1) return fail(RXW8_INVALID_ARGUMENT, "sequence length must be positive");
  for (int64_t i = 0; i < b; ++i)
    if (d->h_lens[i] + s > d->Lmax)
      return fail(RXW8_OUT_OF_RANGE, "sequence %lld would reach %lld positions (capacity %lld)",
                  (long long)i, (long long)(d->h_lens[i] + s), (long long)d->Lmax);
  return RXW8_OK;
}

}  // namespace rxw8

using namespace rxw8;

struct rxw8_decoder : rxw8::Decoder {};

extern "C" {

int rxw8_decoder_create(rxw8_runtime *rt, const rxw8_decoder_config *cfg, rxw8_decoder **out) {
  if (!rt || !cfg || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  const rxw8_decoder_config &c = *cfg;
  const int64_t G = c.group;
  const bool ok = c.layers > 0 && c.hidden > 0 && c.q_heads > 0 && c.kv_heads > 0 &&
                  c.q_heads % c.kv_heads == 0 && c.head_dim > 0 && c.head_dim % 2 == 0 &&
                  c.intermediate > 0 && c.vocab > 0 && c.max_batch > 0 && c.max_seq > 0 &&
                  G >= 0 && (G == 0 || (c.hidden % G == 0 && c.intermediate % G == 0 &&
                                        (c.q_heads * c.head_dim) % G == 0)) &&
                  std::isfinite(c.eps) && c.eps > 0 && std::isfinite(c.theta) && c.theta > 0;
  if (!ok) return fail(RXW8_INVALID_ARGUMENT, "invalid decoder configuration");
  std::lock_guard<std::recursive_mutex> guard(rt->mu);
  auto *d = new rxw8_decoder();
  d->rt = rt;
  d->cfg = c;
  d->H = c.hidden;
  d->D = c.head_dim;
  d->Hq = c.q_heads;
  d->Hkv = c.kv_heads;
  d->I = c.intermediate;
  d->V = c.vocab;
  d->L = c.layers;
  d->Bmax = c.max_batch;
  d->Lmax = c.max_seq;
  d->QKV = (d->Hq + 2 * d->Hkv) * d->D;
  d->by_layer_kind.assign((size_t)d->L * 14, -1);
  auto gs = [&](int64_t k) { return k / (G > 0 ? G : k); };
  add_param(d, "embed_tokens.weight", P_EMBED, -1, RXW8_BF16, d->V, d->H);
  for (int l = 0; l < d->L; ++l) {
    const std::string pre = "layers." + std::to_string(l) + ".";
    add_param(d, pre + "input_layernorm.weight", P_IN_NORM, l, RXW8_F32, d->H, 0);
    add_param(d, pre + "self_attn.qkv_proj.weight", P_QKV_W, l, RXW8_U8, d->QKV, d->H);
    add_param(d, pre + "self_attn.qkv_proj.scale", P_QKV_S, l, RXW8_F32, d->QKV, gs(d->H));
    if (c.qk_norm) {
      add_param(d, pre + "self_attn.q_norm.weight", P_QN, l, RXW8_F32, d->D, 0);
      add_param(d, pre + "self_attn.k_norm.weight", P_KN, l, RXW8_F32, d->D, 0);
    }
    add_param(d, pre + "self_attn.o_proj.weight", P_O_W, l, RXW8_U8, d->H, d->Hq * d->D);
    add_param(d, pre + "self_attn.o_proj.scale", P_O_S, l, RXW8_F32, d->H, gs(d->Hq * d->D));
    add_param(d, pre + "post_attention_layernorm.weight", P_POST_NORM, l, RXW8_F32, d->H, 0);
    add_param(d, pre + "mlp.gate_up_proj.weight", P_GU_W, l, RXW8_U8, 2 * d->I, d->H);
    add_param(d, pre + "mlp.gate_up_proj.scale", P_GU_S, l, RXW8_F32, 2 * d->I, gs(d->H));
    add_param(d, pre + "mlp.down_proj.weight", P_DOWN_W, l, RXW8_U8, d->H, d->I);
    add_param(d, pre + "mlp.down_proj.scale", P_DOWN_S, l, RXW8_F32, d->H, gs(d->I));
  }
  add_param(d, "norm.weight", P_FINAL_NORM, -1, RXW8_F32, d->H, 0);

  // KV caches [L][Bmax][Hkv][Lmax][D] bf16, lengths, RoPE frequencies, tail.
  int rc = RXW8_OK;
  d->cache_bytes = (size_t)d->L * d->Bmax * d->Hkv * d->Lmax * d->D * 2;
  hipError_t e = hipMalloc(&d->kc, d->cache_bytes);
  if (e == hipSuccess) e = hipMalloc(&d->vc, d->cache_bytes);
  if (e == hipSuccess) e = hipMalloc((void **)&d->d_lens, 256 + (size_t)d->Bmax * 4);
  if (e == hipSuccess) e = hipMalloc((void **)&d->d_freqs, (size_t)d->D / 2 * 4);
  if (e == hipSuccess) e = hipMalloc((void **)&d->d_rope, (size_t)d->Lmax * d->D * 4);
  const size_t ss_floats = 32 + 2 * (size_t)(d->H / 16) * 32;
  const size_t tail = (size_t)d->Bmax * d->H * 2 + (size_t)d->Bmax * d->V * 4 +
                      (size_t)d->Bmax * d->am_chunks * 8 + (size_t)d->Bmax * 8 + ss_floats * 4 +
                      4096;
  if (e == hipSuccess) e = hipMalloc(&d->tail_block, tail);
  if (e != hipSuccess) {
    rc = hip_fail(e, "hipMalloc (decoder state)");
    free_decoder_memory(d);
    delete d;
    return rc;
  }
  d->tail_bytes = tail;
  char *p = (char *)d->tail_block;
  auto take = [&](size_t n) { char *r = p; p += (n + 255) / 256 * 256; return r; };
  d->xl = (uint16_t *)take((size_t)d->Bmax * d->H * 2);
  d->logits = (float *)take((size_t)d->Bmax * d->V * 4);
  d->am_val = (float *)take((size_t)d->Bmax * d->am_chunks * 4);
  d->am_idx = (int32_t *)take((size_t)d->Bmax * d->am_chunks * 4);
  d->next = (int32_t *)take((size_t)d->Bmax * 4);
  d->ss_embed = (float *)take(32 * 4);
  d->ss_o = (float *)take((size_t)(d->H / 16) * 32 * 4);
  d->ss_down = (float *)take((size_t)(d->H / 16) * 32 * 4);
  d->gu_ilv = d->I % 8 == 0 && (2 * d->I) % 16 == 0 && d->H % 64 == 0;
  d->d_step = d->d_lens + 64;  // device step counter for generate
  std::vector<float> freqs((size_t)d->D / 2);
  for (int64_t i = 0; i < d->D / 2; ++i)
    freqs[i] = std::pow(c.theta, -2.0f * (float)i / (float)d->D);  // qwen3_5/mod.rs:213-219
  d->h_lens.assign((size_t)d->Bmax, 0);
  e = hipMemsetAsync(d->kc, 0, d->cache_bytes, rt->stream);
  if (e == hipSuccess) e = hipMemsetAsync(d->vc, 0, d->cache_bytes, rt->stream);
  if (e == hipSuccess) e = hipMemsetAsync(d->d_lens, 0, 256 + (size_t)d->Bmax * 4, rt->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(d->d_freqs, freqs.data(), freqs.size() * 4, hipMemcpyHostToDevice, rt->stream);
  if (e == hipSuccess) {
    RopeTableArgs a{d->d_freqs, d->d_rope, (int)(d->D / 2)};
    rc = launch(rt, "rxw8_dec_rope_table", dim3((unsigned)d->Lmax), dim3(64), a);
  }
  if (e == hipSuccess && rc == RXW8_OK) e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess || rc != RXW8_OK) {
    if (rc == RXW8_OK) rc = hip_fail(e, "decoder state initialisation");
    free_decoder_memory(d);
    delete d;
    return rc;
  }
  rt->refs.fetch_add(1);
  *out = d;
  return RXW8_OK;
}

int rxw8_decoder_destroy(rxw8_decoder *d) {
  if (!d) return fail(RXW8_INVALID_ARGUMENT, "decoder is NULL");
  Runtime *rt = d->rt;
  {
    std::lock_guard<std::recursive_mutex> g(rt->mu);
    free_decoder_memory(d);
  }
  delete d;
  runtime_release(rt);
  return RXW8_OK;
}

int rxw8_decoder_num_parameters(rxw8_decoder *d, int *count) {
  if (!d || !count) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  *count = (int)d->params.size();
  return RXW8_OK;
}

int rxw8_decoder_parameter_info(rxw8_decoder *d, int index, const char **path, int *dtype,
                                int64_t *dims, int *rank) {
  if (!d) return fail(RXW8_INVALID_ARGUMENT, "decoder is NULL");
  if (index < 0 || index >= (int)d->params.size())
    return fail(RXW8_OUT_OF_RANGE, "parameter index %d outside [0, %zu)", index, d->params.size());
  const ParamSpec &s = d->params[(size_t)index];
  if (path) *path = s.path.c_str();
  if (dtype) *dtype = s.dtype;
  if (rank) *rank = s.rank;
  if (dims)
    for (int i = 0; i < s.rank; ++i) dims[i] = s.dims[i];
  return RXW8_OK;
}

int rxw8_decoder_bind_parameter(rxw8_decoder *d, const char *path, rxw8_buffer *buf) {
  if (!d || !path || !buf) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  auto it = d->index.find(path);
  if (it == d->index.end()) return fail(RXW8_NOT_FOUND, "parameter \"%s\" is absent from the schema", path);
  ParamSpec &s = d->params[(size_t)it->second];
  if (s.bound) return fail(RXW8_ALREADY_EXISTS, "duplicate parameter binding \"%s\"", path);
  if (buf->rt != d->rt)
    return fail(RXW8_INVALID_ARGUMENT, "parameter \"%s\": buffer belongs to another runtime", path);
  bool shape_ok = buf->rank == s.rank;
  for (int i = 0; shape_ok && i < s.rank; ++i) shape_ok = buf->dims[i] == s.dims[i];
  if (!shape_ok)
    return fail(RXW8_INVALID_ARGUMENT, "parameter \"%s\" %s: shape does not match the schema", path,
                dims_str(buf).c_str());
  if (buf->dtype != s.dtype)
    return fail(RXW8_INVALID_ARGUMENT, "parameter \"%s\": dtype %s does not match the schema (%s)",
                path, dtype_name(buf->dtype), dtype_name(s.dtype));
  std::lock_guard<std::recursive_mutex> g(d->rt->mu);
  // Weights the GEMV reads are repacked once into the tiled layout.
  const bool u8w = s.dtype == RXW8_U8;
  const bool emb = s.kind == P_EMBED;
  if ((u8w && s.dims[0] % 16 == 0 && s.dims[1] % 64 == 0) ||
      (emb && s.dims[0] % 16 == 0 && s.dims[1] % 32 == 0)) {
    const int kb = u8w ? 64 : 32;
    const int64_t pd[3] = {s.dims[0] / 16, s.dims[1] / kb, u8w ? 1024 : 512};
    Buffer *pk = nullptr;
    int rc = new_buffer(d->rt, s.dtype, pd, 3, false, &pk);
    if (rc) return rc;
    const int64_t ilv = (s.kind == P_GU_W && d->gu_ilv) ? s.dims[0] / 2 : 0;
    PackArgs a{buf->ptr, pk->ptr, s.dims[0], s.dims[1], kb, u8w ? 1 : 2, ilv};
    const int64_t slices = s.dims[0] / 16 * (s.dims[1] / kb) * 64;
    rc = launch(d->rt, "rxw8_pack_tiles", dim3((unsigned)std::min<int64_t>((slices + 255) / 256, 1 << 14)),
                dim3(256), a);
    if (rc) {
      rxw8_buffer_release(static_cast<rxw8_buffer *>(pk));
      return rc;
    }
    s.packed = pk;
  }
  if (s.kind == P_GU_S && d->gu_ilv) {  // scales follow the interleaved weight rows
    Buffer *pm = nullptr;
    int rc = new_buffer(d->rt, RXW8_F32, s.dims, s.rank, false, &pm);
    if (rc) return rc;
    InterleaveArgs a{(const float *)buf->ptr, (float *)pm->ptr, s.dims[0] / 2, s.dims[1]};
    rc = launch(d->rt, "rxw8_dec_interleave_rows", dim3(blocks(s.dims[0] * s.dims[1])), dim3(256), a);
    if (rc) {
      rxw8_buffer_release(static_cast<rxw8_buffer *>(pm));
      return rc;
    }
    s.perm = pm;
  }
  buf->refs.fetch_add(1);
  s.bound = buf;
  return RXW8_OK;
}

int rxw8_decoder_reset(rxw8_decoder *d) {
  if (!d) return fail(RXW8_INVALID_ARGUMENT, "decoder is NULL");
  std::lock_guard<std::recursive_mutex> g(d->rt->mu);
  RXW8_HIP(hipMemsetAsync(d->d_lens, 0, (size_t)d->Bmax * 4, d->rt->stream));
  RXW8_HIP(hipStreamSynchronize(d->rt->stream));
  std::fill(d->h_lens.begin(), d->h_lens.end(), 0);
  return RXW8_OK;
}

int rxw8_decoder_lens(rxw8_decoder *d, int32_t *lens, int64_t n) {
  if (!d || (!lens && n)) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  for (int64_t i = 0; i < n && i < d->Bmax; ++i) lens[i] = d->h_lens[(size_t)i];
  return RXW8_OK;
}

int rxw8_decoder_forward(rxw8_decoder *d, rxw8_buffer *ids, int64_t b, int64_t s,
                         rxw8_buffer *next_ids, rxw8_buffer *logits) {
  if (!d || !ids || !next_ids) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (ids->dtype != RXW8_I32 || ids->rank != 2 || ids->dims[0] != b || ids->dims[1] != s)
    return fail(RXW8_INVALID_ARGUMENT, "ids must be I32 [b, s]");
  if (next_ids->dtype != RXW8_I32 || next_ids->numel() != b)
    return fail(RXW8_INVALID_ARGUMENT, "next_ids must be I32 [b]");
  if (logits && (logits->dtype != RXW8_F32 || logits->numel() != b * d->V))
    return fail(RXW8_INVALID_ARGUMENT, "logits must be F32 [b, vocab]");
  std::lock_guard<std::recursive_mutex> g(d->rt->mu);
  int rc = check_ready(d, b, s);
  if (rc) return rc;
  if ((rc = ensure_activations(d, b * s))) return rc;
  if ((rc = enqueue_forward(d, (const int32_t *)ids->ptr, b, s))) return rc;
  RXW8_HIP(hipMemcpyAsync(next_ids->ptr, d->next, (size_t)b * 4, hipMemcpyDeviceToDevice, d->rt->stream));
  if (logits)
    RXW8_HIP(hipMemcpyAsync(logits->ptr, d->logits, (size_t)b * d->V * 4, hipMemcpyDeviceToDevice,
                            d->rt->stream));
  for (int64_t i = 0; i < b; ++i) d->h_lens[(size_t)i] += (int32_t)s;
  return RXW8_OK;
}

int rxw8_decoder_forward_layers(rxw8_decoder *d, rxw8_buffer *hidden_in, int64_t b, int64_t s,
                                int64_t first, int64_t last, rxw8_buffer *hidden_out,
                                rxw8_buffer *logits, int commit) {
  if (!d || !hidden_in || !hidden_out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (first < 0 || last <= first || last > d->L)
    return fail(RXW8_INVALID_ARGUMENT, "layer range [%lld, %lld) outside [0, %lld]", (long long)first,
                (long long)last, (long long)d->L);
  if (b < 1 || s < 1 || b > d->Bmax || s > d->Lmax)
    return fail(RXW8_INVALID_ARGUMENT, "b and s must lie in [1, max_batch] and [1, max_seq]");
  for (rxw8_buffer *hb : {hidden_in, hidden_out})
    if (hb->dtype != RXW8_F32 || hb->numel() != b * s * d->H || hb->rt != d->rt)
      return fail(RXW8_INVALID_ARGUMENT, "hidden_in / hidden_out must be F32 [b, s, hidden] of this runtime");
  if (logits && (last != d->L || logits->dtype != RXW8_F32 || logits->numel() != b * d->V))
    return fail(RXW8_INVALID_ARGUMENT, "logits need last == layers and F32 [b, vocab]");
  std::lock_guard<std::recursive_mutex> g(d->rt->mu);
  int rc = check_ready(d, b, s);
  if (rc) return rc;
  if ((rc = ensure_activations(d, b * s))) return rc;
  LayerRange range;
  range.h_in = (const float *)hidden_in->ptr;
  range.first = (int)first;
  range.last = (int)last;
  range.tail = logits != nullptr;
  range.advance = logits && commit;
  if ((rc = enqueue_forward(d, nullptr, b, s, nullptr, false, false, &range))) return rc;
  Runtime *rt = d->rt;
  RXW8_HIP(hipMemcpyAsync(hidden_out->ptr, d->h, (size_t)(b * s * d->H) * 4,
                          hipMemcpyDeviceToDevice, rt->stream));
  if (logits)
    RXW8_HIP(hipMemcpyAsync(logits->ptr, d->logits, (size_t)b * d->V * 4, hipMemcpyDeviceToDevice,
                            rt->stream));
  if (commit) {
    for (int64_t i = 0; i < b; ++i) d->h_lens[(size_t)i] += (int32_t)s;
    if (!logits) {  // no argmax pass to advance the device lengths
      RXW8_HIP(hipMemcpyAsync(d->d_lens, d->h_lens.data(), (size_t)b * 4, hipMemcpyHostToDevice,
                              rt->stream));
      RXW8_HIP(hipStreamSynchronize(rt->stream));
    }
  }
  return RXW8_OK;
}

int rxw8_argmax(rxw8_runtime *rt, rxw8_buffer *x, int axis, int keep_dims, rxw8_buffer **out) {
  if (!rt || !x || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (x->dtype != RXW8_F32) return fail(RXW8_INVALID_ARGUMENT, "argmax: x must be F32");
  if (axis < 0 || axis >= x->rank || x->dims[axis] <= 0 || x->dims[axis] > INT32_MAX)
    return fail(RXW8_INVALID_ARGUMENT, "argmax requires a nonempty axis with I32-sized length");
  int64_t outer = 1, inner = 1;
  for (int i = 0; i < axis; ++i) outer *= x->dims[i];
  for (int i = axis + 1; i < x->rank; ++i) inner *= x->dims[i];
  const int64_t cols = x->dims[axis], rows = outer * inner;
  // partials: up to 64 chunks of >= 2048 columns per row, one lane each in
  // the final pass; the grid is rows x chunks workgroups
  const int chunks = (int)std::min<int64_t>(64, std::max<int64_t>(1, cols / 2048));
  if (rows > (int64_t)INT32_MAX / 64)
    return fail(RXW8_UNIMPLEMENTED, "argmax: %lld rows exceed the kernel's grid", (long long)rows);
  int64_t od[RXW8_MAX_RANK];
  int orank = 0;
  for (int i = 0; i < x->rank; ++i) {
    if (i == axis && !keep_dims) continue;
    od[orank++] = i == axis ? 1 : x->dims[i];
  }
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  Buffer *o = nullptr;
  int rc = new_buffer(rt, RXW8_I32, od, orank, false, &o);
  if (rc) return rc;
  if (rows > 0) {
    void *part = nullptr;
    const size_t pbytes = (size_t)rows * chunks * 8;
    if ((rc = rt_alloc(rt, pbytes, &part))) {
      rxw8_buffer_release(static_cast<rxw8_buffer *>(o));
      return rc;
    }
    float *pval = (float *)part;
    int32_t *pidx = (int32_t *)((char *)part + (size_t)rows * chunks * 4);
    ArgmaxArgs a{(const float *)x->ptr, pval, pidx, nullptr, cols, (int)rows, chunks, inner};
    rc = launch(rt, "rxw8_dec_argmax_partial", dim3((unsigned)(rows * chunks)), dim3(256), a);
    ArgmaxFinalArgs f{pval, pidx, (int32_t *)o->ptr, nullptr, nullptr, nullptr, (int)rows, chunks, 0, 0};
    if (!rc) rc = launch(rt, "rxw8_dec_argmax_final", dim3(1), dim3((unsigned)(64 * std::min<int64_t>(rows, 16))), f);
    rt_free(rt, part, pbytes);
    if (rc) {
      rxw8_buffer_release(static_cast<rxw8_buffer *>(o));
      return rc;
    }
  }
  *out = static_cast<rxw8_buffer *>(o);
  return RXW8_OK;
}

int rxw8_decoder_generate(rxw8_decoder *d, rxw8_buffer *prompt, int64_t b, int64_t s,
                          int64_t steps, rxw8_buffer *out_ids, int use_graph) {
  if (!d || !prompt || !out_ids) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (prompt->dtype != RXW8_I32 || prompt->rank != 2 || prompt->dims[0] != b || prompt->dims[1] != s)
    return fail(RXW8_INVALID_ARGUMENT, "prompt must be I32 [b, s]");
  if (steps < 0) return fail(RXW8_INVALID_ARGUMENT, "steps must be >= 0");
  if (out_ids->dtype != RXW8_I32 || out_ids->rank != 2 || out_ids->dims[0] != b ||
      out_ids->dims[1] != steps + 1)
    return fail(RXW8_INVALID_ARGUMENT, "out_ids must be I32 [b, steps + 1]");
  std::lock_guard<std::recursive_mutex> g(d->rt->mu);
  Runtime *rt = d->rt;
  int rc = check_ready(d, b, s + steps);
  if (rc) return rc;
  if ((rc = ensure_activations(d, b * s))) return rc;
  RXW8_HIP(hipMemsetAsync(d->d_step, 0, 4, rt->stream));
  RecordArgs rec{d->next, (int32_t *)out_ids->ptr, d->d_step, (int)b, (int)(steps + 1)};
  // With decode steps to follow, every forward's argmax launch also embeds
  // its winners as the next step's input rows (one launch fewer per step).
  if ((rc = enqueue_forward(d, (const int32_t *)prompt->ptr, b, s, &rec, false, steps > 0)))
    return rc;
  for (int64_t i = 0; i < b; ++i) d->h_lens[(size_t)i] += (int32_t)s;
  if (steps == 0) return RXW8_OK;
  // One decode step: its input rows (the previous argmax, d->next) are embedded.
  auto step = [&]() -> int { return enqueue_forward(d, d->next, b, 1, &rec, true, true); };
  int64_t done = 0;
  if (use_graph) {
    // A captured step holds the batch, the out_ids row stride (steps + 1) and
    // address, the activation block and every runtime workspace it used. Any
    // of these can change between calls (a longer prompt regrows the
    // activations; another op regrows a workspace; a freed out_ids block of
    // the same rounded size is handed out again for another `steps`), so the
    // graph is kept only while all of them match.
    int64_t key[10];
    graph_key(d, b, steps + 1, out_ids->ptr, key);
    if (!d->gexec || !std::equal(key, key + 10, d->g_key)) {
      if ((rc = step())) return rc;  // eager step sizes every workspace first
      for (int64_t i = 0; i < b; ++i) d->h_lens[(size_t)i] += 1;
      done = 1;
      if (d->gexec) (void)hipGraphExecDestroy(d->gexec);
      if (d->graph) (void)hipGraphDestroy(d->graph);
      d->gexec = nullptr;
      d->graph = nullptr;
      d->g_key[0] = -1;
      RXW8_HIP(hipStreamBeginCapture(rt->stream, hipStreamCaptureModeThreadLocal));
      rc = step();
      hipGraph_t graph = nullptr;
      hipError_t e = hipStreamEndCapture(rt->stream, &graph);
      if (rc) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
      }
      if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
      e = hipGraphInstantiate(&d->gexec, graph, nullptr, nullptr, 0);
      if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(e, "hipGraphInstantiate");
      }
      d->graph = graph;
      // the eager step above sized every workspace, so the key taken now is
      // the one the capture used
      graph_key(d, b, steps + 1, out_ids->ptr, d->g_key);
    }
    for (; done < steps; ++done) {
      RXW8_HIP(hipGraphLaunch(d->gexec, rt->stream));
      for (int64_t i = 0; i < b; ++i) d->h_lens[(size_t)i] += 1;
    }
  } else {
    for (; done < steps; ++done) {
      if ((rc = step())) return rc;
      for (int64_t i = 0; i < b; ++i) d->h_lens[(size_t)i] += 1;
    }
  }
  return RXW8_OK;
}

}  // extern "C"
