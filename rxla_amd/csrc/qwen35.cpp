// Qwen3.5 hybrid W8 text model: full-sequence inference behind the C ABI.
//
// Follows qwen3_5(cx, token_ids, config) (crates/rxla-models/src/qwen3_5/
// mod.rs:197-273) through the applied-model flow (crates/rxla-nn/src/
// applied.rs:156-239): W8 embedding gather (mod.rs:134-157); per layer a
// zero-centred input RMSNorm, a gated-delta (layers.rs:113-268) or
// output-gated full-attention (layers.rs:28-100) mixer with residual, a
// zero-centred post-attention RMSNorm and the SwiGLU MLP (layers.rs:270-293)
// with residual; the final zero-centred norm and the tied W8 LM head with an
// optional F32 LoRA update (mod.rs:158-195). Every sequence of the batch runs
// from position 0 (mod.rs:211-229: positions iota, angles pos * theta^(-2i/r)).
//
// Projections are QuantizedLinear at the layer compute dtype
// (qwen3_5/layers.rs:4-9 takes cx.layer_compute_dtype()). The default is the
// reference's, F32 (rxla-nn lib.rs:432): f32 x against the f32 dequantised
// weights on the F32 matrix-core linear, with every activation between
// kernels in f32. The BF16 opt-in (bf16 x, bf16 dequantised weights, f32
// accumulation, bf16-rounded result) runs on the packed W8A16 GEMV / GEMM with
// bf16 activations. The LM head computes in F32 either way (a plain linear
// against the f32 dequantised table). Token t = b * S + i is position i of
// sequence b.
//
// Parameter schema (prefix P = "model.language_model."):
//   P embed_tokens.{weight U8 [V, H], scale F32 [V, H/G]}        (tied head)
//   P embed_tokens.lora_{A,B}.weight F32 [r, H], [V, r]          (lora_rank r > 0)
//   P layers.{i}.{input,post_attention}_layernorm.weight F32 [H]
//   linear layers, P layers.{i}.linear_attn.:
//     in_proj_qkv [3W, H], in_proj_z [W, H], in_proj_b [Hl, H], in_proj_a [Hl, H],
//     out_proj [H, W] (U8 weight + F32 scale [N, K/G] each); conv1d.weight
//     F32 [3W, 1, k]; A_log, dt_bias F32 [Hl]; norm.weight F32 [Dl]   (W = Hl Dl)
//   full layers, P layers.{i}.self_attn.:
//     q_proj [2 Hq D, H], k_proj / v_proj [Hkv D, H], o_proj [H, Hq D];
//     q_norm.weight / k_norm.weight F32 [D]
//   P layers.{i}.mlp.{gate_proj, up_proj} [I, H], down_proj [H, I]
//   P norm.weight F32 [H]
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "internal.h"

namespace rxw8 {

int qlinear_launch(Runtime *rt, const void *x, int x_f32, const uint8_t *w, bool packed,
                   const float *s, void *y, int y_f32, int64_t M, int64_t N, int64_t K,
                   int64_t G, int compute_bf16, int y_mode);
bool gemm_eligible(int64_t M, int64_t N, int64_t K, int64_t G);
bool f32_gemm_applies(const void *w, const float *y, int64_t M, int64_t N, int64_t K, int64_t G);
int f32_gemm_operands(Runtime *rt, int64_t M, int64_t K, uint16_t **hi, uint16_t **lo);
int f32_gemm_presplit(Runtime *rt, const uint8_t *w, bool packed, const float *scale, float *y,
                      int64_t M, int64_t N, int64_t K, int64_t G, int y_mode);

namespace {

// Kernel argument structs (match kernels/qwen35.hip and kernels/decoder.hip).
struct DecPosArgs {
  const int32_t *lens;
  int32_t *pos, *row_seq, *row_len;
  int b, s;
};
struct Q35EmbedArgs {
  const int32_t *ids;
  const uint8_t *w;
  const float *scale;
  float *h;
  float *ss;
  int64_t T, V, H, G;
};
struct Q35NormArgs {
  const float *x;
  const float *w;
  const void *z;
  void *out;
  int64_t rows, L, x_stride, out_stride, z_stride, z_group;
  float eps;
  int zero_centered, out_f32, z_f32;
  uint16_t *hi, *lo;  // the F32 GEMM's operand split instead of out
};
struct Q35FaPrepArgs {
  const void *qg, *kp, *vp;
  const float *q_norm, *k_norm, *freqs;
  float *q_out, *gate_out, *kc, *vc;
  int T, S, Hq, Hkv, D, rot, Lmax, stride;
  float eps;
  int src_f32;
};
struct Q35AttnArgs {
  const float *q, *kc, *vc, *gate;
  float *out;
  float *part;
  int B, S, Hq, Hkv, Lmax, qtiles, nsplit;
  float scale;
};
struct Q35MulArgs {
  float *x;
  const float *y;
  int64_t n;
};
struct Q35MixPrepArgs {
  const void *raw;
  const float *conv_w;
  const float *a_log, *dt_bias;
  float *mixed;
  float *beta, *g;
  float *lg;
  int64_t stride;
  int S, Hl, Dl, k;
  float q_scale;
  int raw_f32;
};
struct Q35DeltaArgs {
  const float *mixed, *beta, *g;
  float *out;
  int B, S, Hl;
};
struct Q35ChunkArgs {
  const float *mixed;
  const float *beta, *lg;
  float *u, *wm, *pm, *gam, *qg, *kdt;
  float *out;
  int S, Hl, NC;
};
struct Q35ShortMixArgs {
  const void *raw;
  const float *conv_w;
  const float *a_log, *dt_bias;
  const float *norm_w;
  void *out;
  int64_t stride;
  int S, Hl, k;
  float q_scale, eps;
  int raw_f32, out_f32;
};
struct Q35SiluArgs {
  const void *g, *u;
  void *act;
  int64_t n, I, stride;
  int f32;
};
struct PackArgs {
  const void *src;
  void *dst;
  int64_t n, k;
  int kb;
  int esize;
  int64_t ilv_half;
};
struct InterleaveArgs {
  const float *src;
  float *dst;
  int64_t half, cols;
};
struct SiluMulArgs {
  const uint16_t *gu;
  uint16_t *act;
  int64_t T, I;
  int interleaved;
};
struct Q35ShiftArgs {
  const float *w;
  float *out;
  int64_t n;
};
struct Q35LoraArgs {
  const float *x;   // [T, K]
  const float *w;   // [N, K]
  float *y;         // [T, N]
  int64_t T, N, K;
  float alpha;      // y = x w^T (accumulate == 0) or y += alpha * x w^T
  int accumulate;
};

constexpr int kAttnMaxSplit = 4;  // key-range splits of the full attention (at most)

unsigned grid_n(int64_t n, int64_t cap = 1 << 16) {
  int64_t g = (n + 255) / 256;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(g, cap));
}

const char *kRoot = "model.language_model.";

struct Param {
  std::string path;
  int dtype = 0, rank = 0;
  int64_t dims[3] = {0, 0, 0};
  Buffer *bound = nullptr;
};

// Parameter indices of one layer (-1 where the layer kind has none).
struct Layer {
  int full = 0;
  int in_norm = -1, post_norm = -1;
  int qkv = -1, conv = -1, z = -1, b = -1, a = -1, a_log = -1, dt_bias = -1, lnorm = -1, out = -1;
  int q = -1, k = -1, v = -1, qn = -1, kn = -1, o = -1;
  int gate = -1, up = -1, down = -1;  // a projection's index is its weight; scale = index + 1
  // fused input projections (copied at bind time): linear layers [qkv; z; b; a],
  // full layers [q; k; v], the MLP [gate; up]; rows padded to a multiple of 128
  uint8_t *in_w = nullptr, *gu_w = nullptr;
  float *in_s = nullptr, *gu_s = nullptr;
  int64_t n_in = 0, n_gu = 0;
  // packed mode: every projection weight in the GEMV tile layout (gate|up
  // rows in SwiGLU order, its scales likewise), the residual projections'
  // packed copies, and the zero-centred norm weights as 1 + w
  uint8_t *out_pk = nullptr, *down_pk = nullptr;
  float *in_nw = nullptr, *post_nw = nullptr;
  // the tile-layout copies the chained GEMVs read: in packed mode in_w / gu_w
  // / gu_s themselves; under F32 compute (fc) extra packed copies beside the
  // row-major ones
  uint8_t *in_pk = nullptr, *gu_pk = nullptr;
  float *gu_spk = nullptr;
};

}  // namespace

struct Qwen35 {
  Runtime *rt = nullptr;
  rxw8_qwen35_config cfg{};
  int64_t H = 0, I = 0, V = 0, Hq = 0, Hkv = 0, D = 0, Hl = 0, Dl = 0, W = 0, G = 0;
  int64_t Bmax = 0, Smax = 0;
  std::vector<Param> params;
  std::unordered_map<std::string, int> index;
  std::vector<Layer> layers;
  int embed = -1, final_norm = -1, lora_a = -1, lora_b = -1;
  bool any_full = false, any_linear = false;
  // device memory: one block for activations, caches and constants; one for
  // the fused projection weights (built when the last parameter is bound)
  void *block = nullptr;
  void *fused = nullptr;
  // the tied head's table in the GEMV tile layout (packed and F32-compute
  // models, V % 16 == 0), read by the head of inputs up to 16 rows
  uint8_t *head_pk = nullptr;
  int64_t n_in_max = 0;
  bool packed = false;  // BF16 compute and widths that allow the tile layout (decided at create)
  // F32 compute and widths that allow the tile layout: packed copies beside
  // the row-major weights, for the chained F32 GEMVs of short inputs
  bool fc = false;
  bool f32c = true;     // projection compute dtype F32 (activations f32), else BF16
  int64_t esz = 4;      // bytes per element of xn, raw, gated, gu, act (4: f32, 2: bf16)
  // row sums of squares of the residual h (<= 32 rows): embedding [T], residual
  // GEMV partials [H / 16][T]; ss_cur / ss_parts describe h's current state
  float *ss_embed = nullptr, *ss_o = nullptr, *ss_down = nullptr;
  const float *ss_cur = nullptr;
  int ss_parts = 0;
  bool chain = false;
  float *freqs = nullptr;
  int32_t *zero_lens = nullptr, *pos = nullptr, *row_seq = nullptr, *row_len = nullptr;
  float *h = nullptr, *fin = nullptr, *lora_mid = nullptr;
  void *xn = nullptr;  // normed activations (f32 or bf16, per esz)
  // fused input projection output [T, n_in] (either layer kind)
  void *raw = nullptr;
  // linear layers
  void *gated = nullptr;
  float *mixed = nullptr, *beta = nullptr, *g = nullptr, *dout = nullptr;
  // chunked delta rule: log decays [T, Hl]; per chunk of each (sequence,
  // head) U, W, Qg [64, Dl], KdT [Dl, 64], P [64, 64], cumulative log decays [64]
  float *lg = nullptr, *chunk_ws = nullptr;
  // full layers
  float *q = nullptr, *gate = nullptr, *att = nullptr, *kc = nullptr, *vc = nullptr;
  float *attn_part = nullptr;  // key-range split partials [T, Hq, splits, 2 + D]
  // MLP: [gate | up] projection [T, 2I], SwiGLU output [T, I]
  void *gu = nullptr, *act = nullptr;

  // forward graph: captured on the second consecutive call with the same
  // (batch, sequence, ids, logits), replayed while that key repeats
  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  int64_t g_key[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int g_calls = 0;

  void *ptr(int i) const { return params[(size_t)i].bound->ptr; }
  // element `e` of an activation buffer of element size esz
  void *at(void *p, int64_t e) const { return (char *)p + e * esz; }
  const float *f32(int i) const { return (const float *)ptr(i); }
};

namespace {

int add_param(Qwen35 *m, const std::string &path, int dtype, int64_t d0, int64_t d1 = 0,
              int64_t d2 = 0) {
  Param p;
  p.path = path;
  p.dtype = dtype;
  p.rank = d2 > 0 ? 3 : (d1 > 0 ? 2 : 1);
  p.dims[0] = d0;
  p.dims[1] = d1;
  p.dims[2] = d2;
  m->index[path] = (int)m->params.size();
  m->params.push_back(p);
  return (int)m->params.size() - 1;
}

// U8 weight [n, k] then F32 scale [n, k / G]; returns the weight's index.
int add_proj(Qwen35 *m, const std::string &base, int64_t n, int64_t k) {
  const int w = add_param(m, base + ".weight", RXW8_U8, n, k);
  add_param(m, base + ".scale", RXW8_F32, n, k / m->G);
  return w;
}

void build_schema(Qwen35 *m) {
  const std::string root = kRoot;
  m->embed = add_proj(m, root + "embed_tokens", m->V, m->H);
  if (m->cfg.lora_rank > 0) {
    m->lora_a = add_param(m, root + "embed_tokens.lora_A.weight", RXW8_F32, m->cfg.lora_rank, m->H);
    m->lora_b = add_param(m, root + "embed_tokens.lora_B.weight", RXW8_F32, m->V, m->cfg.lora_rank);
  }
  for (size_t i = 0; i < m->layers.size(); ++i) {
    Layer &L = m->layers[i];
    const std::string pre = root + "layers." + std::to_string(i) + ".";
    L.in_norm = add_param(m, pre + "input_layernorm.weight", RXW8_F32, m->H);
    if (L.full) {
      const std::string a = pre + "self_attn.";
      L.q = add_proj(m, a + "q_proj", 2 * m->Hq * m->D, m->H);
      L.qn = add_param(m, a + "q_norm.weight", RXW8_F32, m->D);
      L.k = add_proj(m, a + "k_proj", m->Hkv * m->D, m->H);
      L.kn = add_param(m, a + "k_norm.weight", RXW8_F32, m->D);
      L.v = add_proj(m, a + "v_proj", m->Hkv * m->D, m->H);
      L.o = add_proj(m, a + "o_proj", m->H, m->Hq * m->D);
    } else {
      const std::string a = pre + "linear_attn.";
      L.qkv = add_proj(m, a + "in_proj_qkv", 3 * m->W, m->H);
      L.conv = add_param(m, a + "conv1d.weight", RXW8_F32, 3 * m->W, 1, m->cfg.conv_kernel);
      L.z = add_proj(m, a + "in_proj_z", m->W, m->H);
      L.b = add_proj(m, a + "in_proj_b", m->Hl, m->H);
      L.a = add_proj(m, a + "in_proj_a", m->Hl, m->H);
      L.a_log = add_param(m, a + "A_log", RXW8_F32, m->Hl);
      L.dt_bias = add_param(m, a + "dt_bias", RXW8_F32, m->Hl);
      L.lnorm = add_param(m, a + "norm.weight", RXW8_F32, m->Dl);
      L.out = add_proj(m, a + "out_proj", m->H, m->W);
    }
    L.post_norm = add_param(m, pre + "post_attention_layernorm.weight", RXW8_F32, m->H);
    L.gate = add_proj(m, pre + "mlp.gate_proj", m->I, m->H);
    L.up = add_proj(m, pre + "mlp.up_proj", m->I, m->H);
    L.down = add_proj(m, pre + "mlp.down_proj", m->H, m->I);
  }
  m->final_norm = add_param(m, root + "norm.weight", RXW8_F32, m->H);
  auto pad128 = [](int64_t n) { return (n + 127) / 128 * 128; };
  for (Layer &L : m->layers) {
    L.n_in = pad128(L.full ? 2 * m->Hq * m->D + 2 * m->Hkv * m->D : 4 * m->W + 2 * m->Hl);
    L.n_gu = m->packed ? 2 * m->I : pad128(2 * m->I);
    m->n_in_max = std::max(m->n_in_max, L.n_in);
  }
}

// Carve the device block: [offset, bytes] pairs, 256-byte aligned.
struct Carver {
  size_t off = 0;
  std::vector<std::pair<void **, size_t>> items;
  template <typename T>
  void add(T **p, int64_t count) {
    items.push_back({(void **)p, (size_t)count * sizeof(T)});
  }
  void add_bytes(void **p, int64_t bytes) { items.push_back({p, (size_t)bytes}); }
  size_t total() const {
    size_t o = 0;
    for (auto &it : items) o += (it.second + 255) & ~(size_t)255;
    return o;
  }
  void assign(void *base) {
    size_t o = 0;
    for (auto &it : items) {
      *it.first = it.second ? (char *)base + o : nullptr;
      o += (it.second + 255) & ~(size_t)255;
    }
  }
};

int allocate(Qwen35 *m) {
  const int64_t T = m->Bmax * m->Smax;
  Carver c;
  c.add(&m->freqs, std::max<int64_t>(1, m->cfg.rotary_dim / 2));
  c.add(&m->zero_lens, m->Bmax);
  c.add(&m->pos, T);
  c.add(&m->row_seq, T);
  c.add(&m->row_len, T);
  c.add(&m->h, T * m->H);
  c.add(&m->fin, T * m->H);
  c.add_bytes(&m->xn, T * std::max(m->H, m->I) * m->esz);
  if (m->cfg.lora_rank > 0) c.add(&m->lora_mid, T * m->cfg.lora_rank);
  c.add_bytes(&m->raw, T * m->n_in_max * m->esz);
  if (m->any_linear) {
    c.add(&m->mixed, T * 3 * m->W);
    c.add(&m->beta, T * m->Hl);
    c.add(&m->g, T * m->Hl);
    c.add(&m->dout, T * m->W);
    c.add(&m->lg, T * m->Hl);
    if (m->Dl == 64 || m->Dl == 128)
      c.add(&m->chunk_ws, m->Bmax * m->Hl * ((m->Smax + 63) / 64) * (4 * 64 * m->Dl + 64 * 64 + 64));
    c.add_bytes(&m->gated, T * m->W * m->esz);
  }
  if (m->any_full) {
    c.add(&m->q, T * m->Hq * m->D);
    c.add(&m->gate, T * m->Hq * m->D);
    c.add(&m->att, T * m->Hq * m->D);
    c.add(&m->attn_part, T * m->Hq * kAttnMaxSplit * (2 + m->D));
    c.add(&m->kc, m->Bmax * m->Hkv * m->Smax * m->D);
    c.add(&m->vc, m->Bmax * m->Hkv * m->Smax * m->D);
  }
  c.add_bytes(&m->gu, T * 2 * m->I * m->esz);
  c.add(&m->ss_embed, 32);
  c.add(&m->ss_o, 32 * ((m->H + 15) / 16));
  c.add(&m->ss_down, 32 * ((m->H + 15) / 16));
  c.add_bytes(&m->act, T * m->I * m->esz);
  const size_t bytes = c.total();
  hipError_t e = hipMalloc(&m->block, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(RXW8_RESOURCE_EXHAUSTED, "qwen35: cannot allocate %zu bytes of activations", bytes);
  }
  c.assign(m->block);
  RXW8_HIP(hipMemsetAsync(m->block, 0, bytes, m->rt->stream));
  // RoPE frequencies theta^(-2i / rotary_dim) in f32 on the host (mod.rs:211-219).
  std::vector<float> f((size_t)std::max<int64_t>(1, m->cfg.rotary_dim / 2), 0.f);
  for (int64_t i = 0; i < m->cfg.rotary_dim / 2; ++i)
    f[(size_t)i] = powf(m->cfg.theta, -2.0f * (float)i / (float)m->cfg.rotary_dim);
  RXW8_HIP(hipMemcpyAsync(m->freqs, f.data(), f.size() * sizeof(float), hipMemcpyHostToDevice,
                          m->rt->stream));
  RXW8_HIP(hipStreamSynchronize(m->rt->stream));
  return RXW8_OK;
}

// Whether the environment switch `name` is set to 0.
bool env_off(const char *name) {
  const char *v = std::getenv(name);
  return v && v[0] == '0';
}

// QuantizedLinear at the model's compute dtype on projection `p` (weight p,
// scale p + 1): y [T, N] an activation (f32 under F32 compute, else bf16), or
// (y_mode 1) the f32 residual [T, N] that receives y += result.
int proj(Qwen35 *m, int p, const void *x, int x_f32, void *y, int y_mode, int64_t T) {
  const Param &w = m->params[(size_t)p];
  return qlinear_launch(m->rt, x, x_f32, (const uint8_t *)m->ptr(p), false, m->f32(p + 1), y,
                        y_mode == 1 || m->f32c ? 1 : 0, T, w.dims[0], w.dims[1], m->G,
                        m->f32c ? 0 : 1, y_mode);
}

// The same on a fused (row-major) weight of n rows; x and y are activations.
int proj_fused(Qwen35 *m, const uint8_t *w, const float *sc, int64_t n, const void *x, void *y,
               int64_t T) {
  return qlinear_launch(m->rt, x, m->f32c, w, false, sc, y, m->f32c, T, n, m->H, m->G,
                        m->f32c ? 0 : 1, 0);
}

// The RMSNorm launch: rows of up to 1024 values one wave each (the
// rxw8_q35_rmsnorm_w* kernels: one memory round trip per row,
// RXW8_Q35_NORM_WAVE=0 turns them off), longer ones a workgroup each.
int launch_norm(Qwen35 *m, const Q35NormArgs &a) {
  int e = 1;
  while (64 * e < a.L) e *= 2;
  if (e <= 16 && !env_off("RXW8_Q35_NORM_WAVE")) {
    char kname[32];
    std::snprintf(kname, sizeof kname, "rxw8_q35_rmsnorm_w%d", e);
    return launch(m->rt, kname, dim3((unsigned)((a.rows + 3) / 4)), dim3(256), a);
  }
  return launch(m->rt, "rxw8_q35_rmsnorm", dim3((unsigned)a.rows), dim3(256), a);
}

int norm(Qwen35 *m, const float *x, const float *w, void *out, int64_t rows, int64_t L,
         bool zero_centered, bool out_f32, const void *z = nullptr, int64_t z_stride = 0,
         int64_t z_group = 1) {
  // z (the output gate of the linear layers) is a projection output: f32
  // under F32 compute, else bf16
  Q35NormArgs a{x, w, z, out, rows, L, L, L, z_stride, z_group, m->cfg.eps, zero_centered ? 1 : 0,
                out_f32 ? 1 : 0, m->f32c ? 1 : 0, nullptr, nullptr};
  return launch_norm(m, a);
}

// y (+)= norm(x) w^T under F32 compute on the GEMM tiles (from 17 rows): the
// norm writes the GEMM's bf16 hi / lo operand parts itself, so neither the
// f32 normed rows nor the split launch exist. The norm's rows of L values
// tile the T x K operand row-major (K = rows * L / T). Returns UNIMPLEMENTED
// (nothing launched) where the GEMM does not apply; the caller then runs
// norm and projection apart.
int norm_linear(Qwen35 *m, const float *x, const float *nw, int64_t rows, int64_t L, bool zero_centered,
                const void *z, int64_t z_stride, int64_t z_group, const uint8_t *w, const float *sc,
                float *y, int64_t T, int64_t N, int y_mode) {
  const int64_t K = rows * L / T;
  if (!m->f32c || m->packed || !f32_gemm_applies(w, y, T, N, K, m->G) || env_off("RXW8_Q35_NORM_SPLIT"))
    return RXW8_UNIMPLEMENTED;
  uint16_t *hi, *lo;
  int rc = f32_gemm_operands(m->rt, T, K, &hi, &lo);
  if (rc) return rc;
  Q35NormArgs a{x, nw, z, nullptr, rows, L, L, L, z_stride, z_group, m->cfg.eps, zero_centered ? 1 : 0,
                1, 1, hi, lo};
  if ((rc = launch_norm(m, a))) return rc;
  return f32_gemm_presplit(m->rt, w, false, sc, y, T, N, K, m->G, y_mode);
}

// raw = norm_in(h) [parts]^T (linear layers [qkv; z; b; a], full layers [q; k; v]).
// Packed mode at up to 64 rows: one GEMV whose prologue applies the RMSNorm.
int in_proj(Qwen35 *m, const Layer &L, int64_t T) {
  int rc;
  if (m->chain && m->ss_cur) {
    GemvOptions o;
    o.mode = 3, o.norm_w = L.in_nw, o.eps = m->cfg.eps, o.ss_in = m->ss_cur, o.ss_parts = m->ss_parts;
    o.prefer_ks1 = true, o.f32c = m->f32c;
    rc = gemv_launch(m->rt, m->h, 1, L.in_pk, false, true, L.in_s, m->raw, m->f32c ? 1 : 0, T, L.n_in,
                     m->H, m->G, 0, o);
    if (rc != RXW8_UNIMPLEMENTED) return rc;
  }
  rc = norm_linear(m, m->h, m->f32(L.in_norm), T, m->H, true, nullptr, 0, 1, L.in_w, L.in_s,
                   (float *)m->raw, T, L.n_in, 0);
  if (rc != RXW8_UNIMPLEMENTED) return rc;
  if ((rc = norm(m, m->h, m->f32(L.in_norm), m->xn, T, m->H, true, m->f32c))) return rc;
  return qlinear_launch(m->rt, m->xn, m->f32c, L.in_w, m->packed, L.in_s, m->raw, m->f32c, T,
                        L.n_in, m->H, m->G, m->f32c ? 0 : 1, 0);
}

// h += x w^T for a residual projection (packed copy w_pk in packed mode). In
// the chained mode the GEMV also writes h's new row sums of squares to ss.
int residual(Qwen35 *m, const uint8_t *w_pk, int p, const void *x, int x_f32, int64_t T, float *ss) {
  const Param &w = m->params[(size_t)p];
  if (m->chain) {
    GemvOptions o;
    o.prefer_ks1 = true, o.ss_out = ss, o.f32c = m->f32c;
    const int rc = gemv_launch(m->rt, x, x_f32, w_pk, false, true, m->f32(p + 1), m->h, 1, T,
                               w.dims[0], w.dims[1], m->G, 1, o);
    if (rc != RXW8_UNIMPLEMENTED) {
      m->ss_cur = ss, m->ss_parts = (int)(m->H / 16);
      return rc;
    }
  }
  m->ss_cur = nullptr;
  if (!m->packed) return proj(m, p, x, x_f32, m->h, 1, T);
  return qlinear_launch(m->rt, x, x_f32, w_pk, true, m->f32(p + 1), m->h, 1, T, w.dims[0],
                        w.dims[1], m->G, 1, 1);
}

int out_proj(Qwen35 *m, const Layer &L, int p, const void *x, int x_f32, int64_t T) {
  return residual(m, L.out_pk, p, x, x_f32, T, m->ss_o);
}

// h += down(silu(gate(x)) * up(x)), x = norm_post(h).
int mlp(Qwen35 *m, const Layer &L, int64_t T) {
  Runtime *rt = m->rt;
  int rc = RXW8_UNIMPLEMENTED;
  // chained GEMV: gate|up rows in SwiGLU order, the norm in the prologue, act
  // = silu(gate) * up (bf16, or f32 under F32 compute) from the epilogue
  if (m->chain && m->ss_cur) {
    GemvOptions o;
    o.mode = 3, o.norm_w = L.post_nw, o.eps = m->cfg.eps, o.ss_in = m->ss_cur;
    o.ss_parts = m->ss_parts, o.swiglu = true, o.prefer_ks1 = true, o.f32c = m->f32c;
    rc = gemv_launch(rt, m->h, 1, L.gu_pk, false, true, L.gu_spk, m->act, m->f32c ? 1 : 0, T,
                     2 * m->I, m->H, m->G, 0, o);
    if (rc != RXW8_UNIMPLEMENTED && rc) return rc;
  }
  if (rc == RXW8_UNIMPLEMENTED && !m->packed) {
    rc = norm_linear(m, m->h, m->f32(L.post_norm), T, m->H, true, nullptr, 0, 1, L.gu_w, L.gu_s,
                     (float *)m->gu, T, L.n_gu, 0);
    if (rc == RXW8_UNIMPLEMENTED) {
      if ((rc = norm(m, m->h, m->f32(L.post_norm), m->xn, T, m->H, true, m->f32c))) return rc;
      rc = proj_fused(m, L.gu_w, L.gu_s, L.n_gu, m->xn, m->gu, T);
    }
    if (rc) return rc;
    Q35SiluArgs sa{m->gu, m->at(m->gu, m->I), m->act, T * m->I, m->I, L.n_gu, m->f32c ? 1 : 0};
    if ((rc = launch(rt, "rxw8_q35_silu_mul", dim3(grid_n(T * m->I)), dim3(256), sa))) return rc;
    m->ss_cur = nullptr;
    return proj(m, L.down, m->act, m->f32c, m->h, 1, T);
  }
  if (rc == RXW8_UNIMPLEMENTED) {
    if ((rc = norm(m, m->h, m->f32(L.post_norm), m->xn, T, m->H, true, false))) return rc;
    if (gemm_eligible(T, 2 * m->I, m->H, m->G)) {
      if ((rc = qlinear_launch(rt, m->xn, 0, L.gu_w, true, L.gu_s, m->act, 0, T, 2 * m->I, m->H,
                               m->G, 1, 2)))
        return rc;
    } else {
      if ((rc = qlinear_launch(rt, m->xn, 0, L.gu_w, true, L.gu_s, m->gu, 0, T, 2 * m->I, m->H,
                               m->G, 1, 0)))
        return rc;
      SiluMulArgs sa{(const uint16_t *)m->gu, (uint16_t *)m->act, T, m->I, 1};
      if ((rc = launch(rt, "rxw8_dec_silu_mul", dim3(grid_n(T * m->I)), dim3(256), sa))) return rc;
    }
  }
  return residual(m, L.down_pk, L.down, m->act, m->f32c ? 1 : 0, T, m->ss_down);
}

// gated RMSNorm over each (token, head) row of Dl (plain weight, times
// silu(z); row r = (t, head) takes z at raw + t * n_in + head * Dl), then out_proj.
int finish_linear(Qwen35 *m, const Layer &L, int64_t T, const void *zp) {
  int rc;
  if (!m->chain) {  // (chained short inputs: out_proj is a GEMV writing h's row sums)
    rc = norm_linear(m, m->dout, m->f32(L.lnorm), T * m->Hl, m->Dl, false, zp, L.n_in, m->Hl,
                     (const uint8_t *)m->ptr(L.out), m->f32(L.out + 1), m->h, T, m->H, 1);
    if (rc != RXW8_UNIMPLEMENTED) {
      m->ss_cur = nullptr;
      return rc;
    }
  }
  if ((rc = norm(m, m->dout, m->f32(L.lnorm), m->gated, T * m->Hl, m->Dl, false, m->f32c, zp,
                 L.n_in, m->Hl)))
    return rc;
  return out_proj(m, L, L.out, m->gated, m->f32c, T);
}

int linear_mixer(Qwen35 *m, const Layer &L, int64_t B, int64_t S) {
  Runtime *rt = m->rt;
  const int64_t T = B * S;
  int rc;
  // raw = xn [qkv; z; b; a]^T: columns [0, 3W) mixed, [3W, 4W) z, then b, a
  if ((rc = in_proj(m, L, T))) return rc;
  const void *zp = m->at(m->raw, 3 * m->W);
  char kname[40];
  // Short sequences (up to 4 positions; RXW8_Q35_SHORT=0 / 1 forces it off /
  // on at any length): the prologue, the recurrence and the gated norm in one
  // launch of a workgroup per (sequence, head). Its recurrence walks a
  // position in ~1 us (every state column reads all of k and q from one CU's
  // LDS), the 16-lane kernel spread over DL / 16 CUs per head in ~0.15 us, so
  // from ~8 positions on the three launches are faster.
  const char *short_env = std::getenv("RXW8_Q35_SHORT");
  const int short_mode = short_env && short_env[0] ? (short_env[0] == '1' ? 1 : 0) : -1;
  if ((m->Dl == 64 || m->Dl == 128) && m->cfg.conv_kernel == 4 &&
      (short_mode == 1 || (short_mode < 0 && S <= 4))) {
    Q35ShortMixArgs sa{m->raw, m->f32(L.conv), m->f32(L.a_log), m->f32(L.dt_bias), m->f32(L.lnorm),
                       m->gated, L.n_in, (int)S, (int)m->Hl, (int)m->cfg.conv_kernel,
                       1.0f / sqrtf((float)m->Dl), m->cfg.eps, m->f32c ? 1 : 0, m->f32c ? 1 : 0};
    std::snprintf(kname, sizeof kname, "rxw8_q35_linear_short_d%d", (int)m->Dl);
    if ((rc = launch(rt, kname, dim3((unsigned)(B * m->Hl)), dim3(512), sa))) return rc;
    return out_proj(m, L, L.out, m->gated, m->f32c, T);
  }
  // conv + SiLU, q / k L2 norms, beta and decay: one workgroup per (token, head)
  // Sequences of 256 positions or more (Dl 64 / 128) take the chunked delta
  // rule: the chunks' triangular solves in parallel, then one walk over the
  // chunks per 16 state columns on the matrix cores (RXW8_Q35_CHUNKED=0 / 1
  // forces it off / on). Its chunk pass costs ~33 us per layer whatever the
  // length, the walk ~4.5 us per 64 positions, the sequential kernel ~0.2 us
  // per position: the 0.8B forward measured even at 128-192 positions and
  // 5-15% faster from 256 (S = 1024: 9.50 against 11.75 ms).
  const char *ch_env = std::getenv("RXW8_Q35_CHUNKED");
  const int ch_mode = ch_env && ch_env[0] ? (ch_env[0] == '1' ? 1 : 0) : -1;
  const bool chunked = m->chunk_ws && (ch_mode == 1 || (ch_mode < 0 && S >= 256));
  Q35MixPrepArgs mp{m->raw, m->f32(L.conv), m->f32(L.a_log), m->f32(L.dt_bias), m->mixed, m->beta,
                    m->g, chunked ? m->lg : nullptr, L.n_in, (int)S, (int)m->Hl, (int)m->Dl,
                    (int)m->cfg.conv_kernel, 1.0f / sqrtf((float)m->Dl), m->f32c ? 1 : 0};
  if ((rc = launch(rt, "rxw8_q35_mix_prep", dim3((unsigned)(T * m->Hl)), dim3(128), mp))) return rc;
  if (chunked) {
    const int64_t NC = (S + 63) / 64, units = B * m->Hl * NC;
    float *u = m->chunk_ws, *wm = u + units * 64 * m->Dl, *qg = wm + units * 64 * m->Dl,
          *kdt = qg + units * 64 * m->Dl, *pm = kdt + units * 64 * m->Dl, *gam = pm + units * 64 * 64;
    Q35ChunkArgs ca{m->mixed, m->beta, m->lg, u, wm, pm, gam, qg, kdt, m->dout, (int)S, (int)m->Hl,
                    (int)NC};
    std::snprintf(kname, sizeof kname, "rxw8_q35_delta_chunk_d%d", (int)m->Dl);
    if ((rc = launch(rt, kname, dim3((unsigned)units), dim3(256), ca))) return rc;
    std::snprintf(kname, sizeof kname, "rxw8_q35_delta_scan_d%d", (int)m->Dl);
    if ((rc = launch(rt, kname, dim3((unsigned)(B * m->Hl * (m->Dl / 16))), dim3(256), ca))) return rc;
    return finish_linear(m, L, T, zp);
  }
  Q35DeltaArgs da{m->mixed, m->beta, m->g, m->dout, (int)B, (int)S, (int)m->Hl};
  std::snprintf(kname, sizeof kname, "rxw8_q35_delta_rule_d%d", (int)m->Dl);
  // Dl <= 32: one workgroup of Dl threads per (sequence, head), one column per
  // thread; Dl >= 64: lpc lanes per column (16 at Dl 64, 32 at Dl 128),
  // workgroups of 256 threads (256 / lpc columns each)
  const bool rows = m->Dl >= 64;
  const int lpc = m->Dl >= 128 ? 32 : 16;
  const dim3 grid((unsigned)(B * m->Hl * (rows ? m->Dl / (256 / lpc) : 1)));
  if ((rc = launch(rt, kname, grid, dim3(rows ? 256u : (unsigned)m->Dl), da))) return rc;
  return finish_linear(m, L, T, zp);
}

int full_mixer(Qwen35 *m, const Layer &L, int64_t B, int64_t S) {
  Runtime *rt = m->rt;
  const int64_t T = B * S;
  int rc;
  // raw = xn [q; k; v]^T
  if ((rc = in_proj(m, L, T))) return rc;
  const void *kp = m->at(m->raw, 2 * m->Hq * m->D), *vp = m->at(m->raw, (2 * m->Hq + m->Hkv) * m->D);
  Q35FaPrepArgs fa{m->raw, kp, vp, m->f32(L.qn), m->f32(L.kn), m->freqs, m->q, m->gate,
                   m->kc, m->vc, (int)T, (int)S, (int)m->Hq, (int)m->Hkv, (int)m->D,
                   (int)m->cfg.rotary_dim, (int)m->Smax, (int)L.n_in, m->cfg.eps, m->f32c ? 1 : 0};
  const int64_t units = T * (m->Hq + m->Hkv);
  if ((rc = launch(rt, "rxw8_q35_fa_prep", dim3((unsigned)((units + 3) / 4)), dim3(256), fa))) return rc;
  const float scale = 1.0f / sqrtf((float)m->D);
  const int64_t G = m->Hq / m->Hkv;
  if ((m->D == 64 || m->D == 128 || m->D == 256) && 4 % G == 0) {
    // f32 matrix-core flash attention: 4 waves per (sequence, kv head, query tile)
    const int64_t qtiles = (S + 16 * (4 / G) - 1) / (16 * (4 / G));
    // key-range splits when the (sequence, kv head, query tile) workgroups
    // alone leave CUs idle and the longest tile walks at least 8 key tiles
    const int64_t base = B * m->Hkv * qtiles, longest = (S + 15) / 16;
    int64_t nsplit = 1;
    while (nsplit < kAttnMaxSplit && base * nsplit < 2 * rt->cus && longest >= 8 * nsplit) nsplit *= 2;
    Q35AttnArgs at{m->q, m->kc, m->vc, m->gate, m->att, m->attn_part, (int)B, (int)S, (int)m->Hq,
                   (int)m->Hkv, (int)m->Smax, (int)qtiles, (int)nsplit, scale};
    const size_t lds = (size_t)4 * 16 * (m->D + 4) * 4 + 4 * 16 * 20 * 4;
    char an[48];
    std::snprintf(an, sizeof an, "rxw8_q35_attention_d%d", (int)m->D);
    // the kernel (or the combine) multiplies the output by the gate
    if ((rc = launch(rt, an, dim3((unsigned)(base * nsplit)), dim3(256), at, lds))) return rc;
    if (nsplit > 1) {
      std::snprintf(an, sizeof an, "rxw8_q35_attention_combine_d%d", (int)m->D);
      if ((rc = launch(rt, an, dim3((unsigned)((T * m->Hq + 3) / 4)), dim3(256), at))) return rc;
    }
  } else {
    if ((rc = attention_launch(rt, m->q, 1, m->kc, m->vc, 1, m->row_len, m->row_seq, nullptr, 0, 0,
                               m->att, 1, T, m->Hq, m->Hkv, m->Smax, m->D, scale, nullptr)))
      return rc;
    Q35MulArgs mu{m->att, m->gate, T * m->Hq * m->D};
    if ((rc = launch(rt, "rxw8_q35_mul", dim3(grid_n(T * m->Hq * m->D)), dim3(256), mu))) return rc;
  }
  return out_proj(m, L, L.o, m->att, 1, T);
}

int enqueue_forward(Qwen35 *m, const int32_t *ids, float *logits, int64_t B, int64_t S) {
  Runtime *rt = m->rt;
  const int64_t T = B * S;
  int rc;
  DecPosArgs pa{m->zero_lens, m->pos, m->row_seq, m->row_len, (int)B, (int)S};
  if ((rc = launch(rt, "rxw8_dec_positions", dim3(grid_n(T)), dim3(256), pa))) return rc;
  // packed mode up to 32 rows: the residual's row sums of squares travel with
  // it (embedding, then the residual GEMVs' per-16-channel partials), so the
  // projections after each RMSNorm take it in their prologue (GEMV mode 3)
  // (F32 compute: up to 16 rows, two bf16 parts each, on the packed copies)
  m->chain = ((m->packed && T <= 32) || (m->fc && T <= 16 && !env_off("RXW8_Q35_FC"))) &&
             m->H % 16 == 0;
  Q35EmbedArgs ea{ids, (const uint8_t *)m->ptr(m->embed), m->f32(m->embed + 1), m->h,
                  m->chain ? m->ss_embed : nullptr, T, m->V, m->H, m->G};
  if ((rc = launch(rt, "rxw8_q35_embed", dim3((unsigned)T), dim3(256), ea))) return rc;
  m->ss_cur = m->chain ? m->ss_embed : nullptr;
  m->ss_parts = 1;
  for (const Layer &L : m->layers) {
    if ((rc = L.full ? full_mixer(m, L, B, S) : linear_mixer(m, L, B, S))) return rc;
    if ((rc = mlp(m, L, T))) return rc;
  }
  if ((rc = norm(m, m->h, m->f32(m->final_norm), m->fin, T, m->H, true, true))) return rc;
  // tied head: f32 hidden . f32 dequantised table (compute F32); up to 16
  // rows from the tile-layout copy (one contiguous KiB per wave load)
  const bool hpk = m->head_pk && T <= 16;
  if ((rc = qlinear_launch(rt, m->fin, 1, hpk ? m->head_pk : (const uint8_t *)m->ptr(m->embed), hpk,
                           m->f32(m->embed + 1), logits, 1, T, m->V, m->H, m->G, 0, 0)))
    return rc;
  if (m->cfg.lora_rank > 0) {
    const int64_t r = m->cfg.lora_rank;
    Q35LoraArgs down{m->fin, m->f32(m->lora_a), m->lora_mid, T, r, m->H, 1.0f, 0};
    if ((rc = launch(rt, "rxw8_q35_lora", dim3(grid_n(T * r)), dim3(256), down))) return rc;
    Q35LoraArgs upd{m->lora_mid, m->f32(m->lora_b), logits, T, m->V, r,
                    m->cfg.lora_alpha / (float)r, 1};
    if ((rc = launch(rt, "rxw8_q35_lora", dim3(grid_n(T * m->V)), dim3(256), upd))) return rc;
  }
  return RXW8_OK;
}

// Fused input projections: the rows of each part copied one after another
// (row-major U8 [n, H] and F32 scales [n, H / G] stack along dim 0), padded
// with codes 128 and scales 0 (rows of zeros) to n_in / n_gu rows. In packed
// mode the stacked rows go through a staging buffer into the tile layout of
// the W8 GEMV / GEMM kernels (rxw8_pack_tiles; the [gate; up] rows in SwiGLU
// order with their scale rows interleaved to match), the residual projections
// are packed from the bound weights, and the zero-centred norm weights are
// stored as 1 + w for the GEMV's RMSNorm prologue.
int prepare(Qwen35 *m) {
  Runtime *rt = m->rt;
  const int64_t ng = m->H / m->G;
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  size_t total = 0, stage = 0;
  for (const Layer &L : m->layers) {
    total += al((size_t)L.n_in * m->H) + al((size_t)L.n_in * ng * 4) + al((size_t)L.n_gu * m->H) +
             al((size_t)L.n_gu * ng * 4);
    if (m->packed || m->fc) {
      const int64_t ko = L.full ? m->Hq * m->D : m->W;
      total += al((size_t)m->H * ko) + al((size_t)m->H * m->I) + 2 * al((size_t)m->H * 4);
      stage = std::max(stage, al((size_t)std::max(L.n_in, L.n_gu) * m->H) +
                                  al((size_t)L.n_gu * ng * 4));
    }
    if (m->fc)  // packed copies of the fused input projections and gate|up (+ scales)
      total += al((size_t)L.n_in * m->H) + al((size_t)2 * m->I * m->H) + al((size_t)2 * m->I * ng * 4);
  }
  const bool head_pk = (m->packed || m->fc) && m->V % 16 == 0 && m->H % 64 == 0;
  if (head_pk) total += al((size_t)m->V * m->H);
  hipError_t e = hipMalloc(&m->fused, total);
  void *tmp = nullptr;
  if (e == hipSuccess && stage) e = hipMalloc(&tmp, stage);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    if (m->fused) (void)hipFree(m->fused);
    m->fused = nullptr;
    return fail(RXW8_RESOURCE_EXHAUSTED, "qwen35: cannot allocate %zu bytes of fused weights",
                total + stage);
  }
  uint8_t *tmp_w = (uint8_t *)tmp;
  float *tmp_s = nullptr;
  char *p = (char *)m->fused;
  auto take = [&](size_t bytes) {
    char *r = p;
    p += al(bytes);
    return r;
  };
  auto stack = [&](const std::vector<int> &parts, int64_t n, uint8_t *w, float *sc) -> int {
    int64_t row = 0;
    for (int i : parts) {
      const int64_t rows = m->params[(size_t)i].dims[0];
      RXW8_HIP(hipMemcpyAsync(w + row * m->H, m->ptr(i), (size_t)rows * m->H,
                              hipMemcpyDeviceToDevice, rt->stream));
      RXW8_HIP(hipMemcpyAsync(sc + row * ng, m->ptr(i + 1), (size_t)rows * ng * 4,
                              hipMemcpyDeviceToDevice, rt->stream));
      row += rows;
    }
    if (row < n) {
      RXW8_HIP(hipMemsetAsync(w + row * m->H, 128, (size_t)(n - row) * m->H, rt->stream));
      RXW8_HIP(hipMemsetAsync(sc + row * ng, 0, (size_t)(n - row) * ng * 4, rt->stream));
    }
    return RXW8_OK;
  };
  auto pack = [&](const void *src, void *dst, int64_t n, int64_t k, int64_t ilv) -> int {
    PackArgs a{src, dst, n, k, 64, 1, ilv};
    const int64_t slices = n / 16 * (k / 64) * 64;
    return launch(rt, "rxw8_pack_tiles", dim3((unsigned)std::min<int64_t>((slices + 255) / 256, 1 << 14)),
                  dim3(256), a);
  };
  int rc = RXW8_OK;
  for (Layer &L : m->layers) {
    const std::vector<int> in = L.full ? std::vector<int>{L.q, L.k, L.v}
                                       : std::vector<int>{L.qkv, L.z, L.b, L.a};
    L.in_w = (uint8_t *)take((size_t)L.n_in * m->H);
    L.in_s = (float *)take((size_t)L.n_in * ng * 4);
    L.gu_w = (uint8_t *)take((size_t)L.n_gu * m->H);
    L.gu_s = (float *)take((size_t)L.n_gu * ng * 4);
    if (!m->packed) {
      if ((rc = stack(in, L.n_in, L.in_w, L.in_s))) break;
      if ((rc = stack({L.gate, L.up}, L.n_gu, L.gu_w, L.gu_s))) break;
      if (!m->fc) continue;
      // F32 compute: tile-layout copies of the stacked rows (gate|up: its
      // first 2 I rows in SwiGLU order, scale rows to match)
      L.in_pk = (uint8_t *)take((size_t)L.n_in * m->H);
      if ((rc = pack(L.in_w, L.in_pk, L.n_in, m->H, 0))) break;
      L.gu_pk = (uint8_t *)take((size_t)2 * m->I * m->H);
      if ((rc = pack(L.gu_w, L.gu_pk, 2 * m->I, m->H, m->I))) break;
      L.gu_spk = (float *)take((size_t)2 * m->I * ng * 4);
      InterleaveArgs il{L.gu_s, L.gu_spk, m->I, ng};
      if ((rc = launch(rt, "rxw8_dec_interleave_rows", dim3(grid_n(2 * m->I * ng)), dim3(256), il))) break;
    } else {
      tmp_s = (float *)((char *)tmp + al((size_t)std::max(L.n_in, L.n_gu) * m->H));
      if ((rc = stack(in, L.n_in, tmp_w, L.in_s))) break;
      if ((rc = pack(tmp_w, L.in_w, L.n_in, m->H, 0))) break;
      if ((rc = stack({L.gate, L.up}, L.n_gu, tmp_w, tmp_s))) break;
      if ((rc = pack(tmp_w, L.gu_w, L.n_gu, m->H, m->I))) break;
      InterleaveArgs il{tmp_s, L.gu_s, m->I, ng};
      if ((rc = launch(rt, "rxw8_dec_interleave_rows", dim3(grid_n(2 * m->I * ng)), dim3(256), il))) break;
      L.in_pk = L.in_w, L.gu_pk = L.gu_w, L.gu_spk = L.gu_s;
    }
    const int o = L.full ? L.o : L.out;
    const int64_t ko = m->params[(size_t)o].dims[1];
    L.out_pk = (uint8_t *)take((size_t)m->H * ko);
    if ((rc = pack(m->ptr(o), L.out_pk, m->H, ko, 0))) break;
    L.down_pk = (uint8_t *)take((size_t)m->H * m->I);
    if ((rc = pack(m->ptr(L.down), L.down_pk, m->H, m->I, 0))) break;
    L.in_nw = (float *)take((size_t)m->H * 4);
    L.post_nw = (float *)take((size_t)m->H * 4);
    Q35ShiftArgs s1{m->f32(L.in_norm), L.in_nw, m->H}, s2{m->f32(L.post_norm), L.post_nw, m->H};
    if ((rc = launch(rt, "rxw8_q35_one_plus", dim3(grid_n(m->H)), dim3(256), s1))) break;
    if ((rc = launch(rt, "rxw8_q35_one_plus", dim3(grid_n(m->H)), dim3(256), s2))) break;
  }
  if (!rc && head_pk) {
    m->head_pk = (uint8_t *)take((size_t)m->V * m->H);
    rc = pack(m->ptr(m->embed), m->head_pk, m->V, m->H, 0);
  }
  const hipError_t se = hipStreamSynchronize(rt->stream);  // the staging buffer is free after this
  if (tmp) (void)hipFree(tmp);
  if (!rc && se != hipSuccess) rc = hip_fail(se, "hipStreamSynchronize");
  if (rc) {
    (void)hipFree(m->fused);
    m->fused = nullptr;
    m->head_pk = nullptr;
  }
  return rc;
}

void drop_graph(Qwen35 *m) {
  if (m->gexec) (void)hipGraphExecDestroy(m->gexec);
  if (m->graph) (void)hipGraphDestroy(m->graph);
  m->gexec = nullptr;
  m->graph = nullptr;
}

// One forward: eager on a new key; the second consecutive call with the same
// key captures the launch sequence into a HIP graph (every workspace has been
// sized by the eager call, and the sequence holds kernel launches only); later
// calls with that key replay it.
int run_forward(Qwen35 *m, const int32_t *ids, float *logits, int64_t B, int64_t S) {
  static const bool no_graph = std::getenv("RXW8_Q35_NO_GRAPH") && std::getenv("RXW8_Q35_NO_GRAPH")[0] == '1';
  Runtime *rt = m->rt;
  // the runtime's workspaces are part of the key: another call that grows
  // (reallocates) one invalidates the addresses a captured graph holds
  const int64_t key[8] = {B, S, (int64_t)(intptr_t)ids, (int64_t)(intptr_t)logits,
                          (int64_t)(intptr_t)rt->partials.ptr, (int64_t)(intptr_t)rt->scratch.ptr,
                          (int64_t)(intptr_t)rt->xcast.ptr, (int64_t)(intptr_t)rt->wdeq.ptr};
  const bool same = std::equal(key, key + 8, m->g_key);
  if (!same) {
    drop_graph(m);
    std::copy(key, key + 8, m->g_key);
    m->g_calls = 0;
  }
  ++m->g_calls;
  if (no_graph || m->g_calls < 2) return enqueue_forward(m, ids, logits, B, S);
  if (!m->gexec) {
    RXW8_HIP(hipStreamBeginCapture(rt->stream, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue_forward(m, ids, logits, B, S);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(rt->stream, &graph);
    if (rc) {
      if (graph) (void)hipGraphDestroy(graph);
      return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    e = hipGraphInstantiate(&m->gexec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
      (void)hipGraphDestroy(graph);
      m->gexec = nullptr;
      return hip_fail(e, "hipGraphInstantiate");
    }
    m->graph = graph;
  }
  RXW8_HIP(hipGraphLaunch(m->gexec, rt->stream));
  return RXW8_OK;
}

void free_model(Qwen35 *m) {
  drop_graph(m);
  if (m->block || m->fused) (void)hipStreamSynchronize(m->rt->stream);
  if (m->block) (void)hipFree(m->block);
  if (m->fused) (void)hipFree(m->fused);
  m->block = m->fused = nullptr;
  m->head_pk = nullptr;
  for (Param &p : m->params)
    if (p.bound) rxw8_buffer_release(static_cast<rxw8_buffer *>(p.bound));
}

}  // namespace
}  // namespace rxw8

using namespace rxw8;

struct rxw8_qwen35 : rxw8::Qwen35 {};

extern "C" {

int rxw8_qwen35_create(rxw8_runtime *rt, const rxw8_qwen35_config *cfg, rxw8_qwen35 **out) {
  if (!rt || !cfg || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  const rxw8_qwen35_config &c = *cfg;
  // Qwen3_5Config::validate (mod.rs:100-131)
  const bool valid = c.vocab > 0 && c.hidden > 0 && c.intermediate > 0 && c.layers > 0 &&
                     c.heads > 0 && c.kv_heads > 0 && c.heads % c.kv_heads == 0 && c.head_dim > 0 &&
                     c.linear_heads > 0 && c.linear_head_dim > 0 && c.conv_kernel > 0 &&
                     c.max_positions > 0 && c.rotary_dim > 0 && c.rotary_dim <= c.head_dim &&
                     c.rotary_dim % 2 == 0 && c.group > 0 && c.hidden % c.group == 0 &&
                     std::isfinite(c.theta) && c.theta > 0 && std::isfinite(c.eps) && c.eps > 0 &&
                     c.lora_rank >= 0 && (c.lora_rank == 0 || std::isfinite(c.lora_alpha)) &&
                     (c.layer_kinds || c.full_attention_interval > 0);
  if (!valid)
    return fail(RXW8_INVALID_ARGUMENT, "invalid Qwen3.5 configuration (InvalidQwenConfiguration)");
  if (c.max_batch <= 0 || c.max_seq <= 0)
    return fail(RXW8_INVALID_ARGUMENT, "max_batch and max_seq must be positive");
  std::unique_ptr<rxw8_qwen35> m(new rxw8_qwen35());
  Qwen35 *q = m.get();
  q->cfg = c;
  q->cfg.layer_kinds = nullptr;
  q->H = c.hidden, q->I = c.intermediate, q->V = c.vocab, q->Hq = c.heads, q->Hkv = c.kv_heads;
  q->D = c.head_dim, q->Hl = c.linear_heads, q->Dl = c.linear_head_dim, q->W = c.linear_heads * c.linear_head_dim;
  q->G = c.group;
  q->Bmax = c.max_batch;
  q->Smax = std::min<int64_t>(c.max_seq, c.max_positions);
  q->layers.resize((size_t)c.layers);
  for (int64_t i = 0; i < c.layers; ++i) {
    const int full = c.layer_kinds ? (c.layer_kinds[i] != 0) : ((i + 1) % c.full_attention_interval == 0);
    q->layers[(size_t)i].full = full;
    (full ? q->any_full : q->any_linear) = true;
  }
  // every projection's input width must be a whole number of groups
  std::vector<int64_t> widths = {c.hidden, c.intermediate};
  if (q->any_full) widths.push_back(c.heads * c.head_dim);
  if (q->any_linear) widths.push_back(q->W);
  for (int64_t k : widths)
    if (k % c.group != 0)
      return fail(RXW8_INVALID_ARGUMENT, "qwen35: group %lld does not divide projection width %lld",
                  (long long)c.group, (long long)k);
  if (q->any_linear && !(q->Dl == 8 || q->Dl == 16 || q->Dl == 32 || q->Dl == 64 || q->Dl == 128))
    return fail(RXW8_UNIMPLEMENTED, "qwen35: linear_head_dim %lld (supported: 8, 16, 32, 64, 128)",
                (long long)q->Dl);
  if (q->any_full && (q->D > 256 || q->D % 2 != 0))
    return fail(RXW8_UNIMPLEMENTED, "qwen35: head_dim %lld (supported: even, <= 256)", (long long)q->D);
  if (q->any_full && q->Smax > 8192)
    return fail(RXW8_UNIMPLEMENTED, "qwen35: full-attention sequences of at most 8192 positions");
  if (c.compute_dtype != 0 && c.compute_dtype != RXW8_F32 && c.compute_dtype != RXW8_BF16)
    return fail(RXW8_INVALID_ARGUMENT, "qwen35: compute_dtype %d (F32 or BF16)", (int)c.compute_dtype);
  q->f32c = c.compute_dtype != RXW8_BF16;
  q->esz = q->f32c ? 4 : 2;
  // tile layout (BF16 compute): 16-row tiles, 64-byte k blocks, gate|up pairs of 8 rows
  const bool tiles = c.hidden % 64 == 0 && c.intermediate % 64 == 0 &&
                     (!q->any_linear || q->W % 64 == 0) && (!q->any_full || (c.heads * c.head_dim) % 64 == 0) &&
                     !(std::getenv("RXW8_Q35_UNPACKED") && std::getenv("RXW8_Q35_UNPACKED")[0] == '1');
  q->packed = !q->f32c && tiles;
  q->fc = q->f32c && tiles && c.hidden % 16 == 0;
  const int64_t T = q->Bmax * q->Smax;
  if (T > (1LL << 31) / std::max<int64_t>({q->H, 3 * q->W, q->I, 2 * q->Hq * q->D}))
    return fail(RXW8_INVALID_ARGUMENT, "qwen35: max_batch * max_seq too large");
  q->rt = rt;
  rt->refs.fetch_add(1);
  build_schema(q);
  int rc;
  {
    std::lock_guard<std::recursive_mutex> g(rt->mu);
    rc = allocate(q);
  }
  if (rc) {
    free_model(q);
    runtime_release(rt);
    return rc;
  }
  *out = m.release();
  return RXW8_OK;
}

int rxw8_qwen35_destroy(rxw8_qwen35 *m) {
  if (!m) return fail(RXW8_INVALID_ARGUMENT, "model is NULL");
  Runtime *rt = m->rt;
  {
    std::lock_guard<std::recursive_mutex> g(rt->mu);
    free_model(m);
  }
  delete m;
  runtime_release(rt);
  return RXW8_OK;
}

int rxw8_qwen35_num_parameters(rxw8_qwen35 *m, int *count) {
  if (!m || !count) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  *count = (int)m->params.size();
  return RXW8_OK;
}

int rxw8_qwen35_parameter_info(rxw8_qwen35 *m, int index, const char **path, int *dtype,
                               int64_t *dims, int *rank) {
  if (!m) return fail(RXW8_INVALID_ARGUMENT, "model is NULL");
  if (index < 0 || index >= (int)m->params.size())
    return fail(RXW8_OUT_OF_RANGE, "parameter index %d outside [0, %zu)", index, m->params.size());
  const Param &p = m->params[(size_t)index];
  if (path) *path = p.path.c_str();
  if (dtype) *dtype = p.dtype;
  if (rank) *rank = p.rank;
  if (dims)
    for (int i = 0; i < p.rank; ++i) dims[i] = p.dims[i];
  return RXW8_OK;
}

int rxw8_qwen35_bind_parameter(rxw8_qwen35 *m, const char *path, rxw8_buffer *buf) {
  if (!m || !path || !buf) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  auto it = m->index.find(path);
  if (it == m->index.end()) return fail(RXW8_NOT_FOUND, "parameter \"%s\" is absent from the schema", path);
  Param &p = m->params[(size_t)it->second];
  if (p.bound) return fail(RXW8_ALREADY_EXISTS, "duplicate parameter binding \"%s\"", path);
  if (buf->rt != m->rt)
    return fail(RXW8_INVALID_ARGUMENT, "parameter \"%s\": buffer belongs to another runtime", path);
  bool shape_ok = buf->rank == p.rank;
  for (int i = 0; shape_ok && i < p.rank; ++i) shape_ok = buf->dims[i] == p.dims[i];
  if (!shape_ok)
    return fail(RXW8_INVALID_ARGUMENT, "parameter \"%s\" %s: shape does not match the schema", path,
                dims_str(buf).c_str());
  if (buf->dtype != p.dtype)
    return fail(RXW8_INVALID_ARGUMENT, "parameter \"%s\": dtype %s does not match the schema (%s)",
                path, dtype_name(buf->dtype), dtype_name(p.dtype));
  rxw8_buffer_retain(buf);
  p.bound = buf;
  // once the last parameter is bound, copy the fused projection weights
  for (const Param &q : m->params)
    if (!q.bound) return RXW8_OK;
  std::lock_guard<std::recursive_mutex> g(m->rt->mu);
  return m->fused ? (int)RXW8_OK : prepare(m);
}

int rxw8_qwen35_forward(rxw8_qwen35 *m, rxw8_buffer *ids, rxw8_buffer *logits) {
  if (!m || !ids || !logits) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (ids->dtype != RXW8_I32 || ids->rank != 2)
    return fail(RXW8_INVALID_ARGUMENT, "token ids must be I32 [batch, sequence] (InvalidQwenTokenShape)");
  const int64_t B = ids->dims[0], S = ids->dims[1];
  if (S <= 0 || S > m->cfg.max_positions || B <= 0)
    return fail(RXW8_INVALID_ARGUMENT, "sequence %lld outside [1, %lld] (InvalidQwenTokens)",
                (long long)S, (long long)m->cfg.max_positions);
  if (B > m->Bmax || S > m->Smax)
    return fail(RXW8_OUT_OF_RANGE, "batch %lld x sequence %lld exceeds the capacity %lld x %lld",
                (long long)B, (long long)S, (long long)m->Bmax, (long long)m->Smax);
  if (logits->dtype != RXW8_F32 || logits->rank != 3 || logits->dims[0] != B ||
      logits->dims[1] != S || logits->dims[2] != m->V)
    return fail(RXW8_INVALID_ARGUMENT, "logits must be F32 [batch, sequence, vocab]");
  if (ids->rt != m->rt || logits->rt != m->rt)
    return fail(RXW8_INVALID_ARGUMENT, "buffers belong to another runtime");
  for (const Param &p : m->params)
    if (!p.bound) return fail(RXW8_FAILED_PRECONDITION, "missing parameter binding \"%s\"", p.path.c_str());
  std::lock_guard<std::recursive_mutex> g(m->rt->mu);
  if (!m->fused) {
    const int rc = prepare(m);
    if (rc) return rc;
  }
  return run_forward(m, (const int32_t *)ids->ptr, (float *)logits->ptr, B, S);
}

}  // extern "C"
