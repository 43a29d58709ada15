/*
 * rxw8 CPU oracle -- TEST INFRASTRUCTURE ONLY (see rxw8_oracle.h).
 *
 * Plain C restatement of the reference's PJRT-CPU ("Portable" lowering)
 * semantics for the W8A16 hot path. Loaded only by tests/, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg.
 *
 * Accumulation order: the reference leaves the order of its f32 sums to XLA
 * (Eigen on CPU), which is not observable from the reference sources. This
 * restatement fixes one: eight interleaved f32 partial sums (index mod 8)
 * combined pairwise at the end. Any order is a valid f32 restatement; the
 * f64 mode gives the order-free "ideal" result for tolerance checks.
 */
#include "rxw8_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define LANES 8

/* ---- scalar conversions -------------------------------------------------- */

static inline uint32_t f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

static inline float bits_f32(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

uint16_t rxo_bf16_from_f32(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) /* NaN: keep sign, force quiet */
    return (uint16_t)((u >> 16) | 0x0040u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

float rxo_f32_from_bf16(uint16_t b) { return bits_f32((uint32_t)b << 16); }

void rxo_f32_to_bf16(const float *x, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = rxo_bf16_from_f32(x[i]);
}

void rxo_bf16_to_f32(const uint16_t *x, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = rxo_f32_from_bf16(x[i]);
}

static inline float round_bf16(float x) {
  return rxo_f32_from_bf16(rxo_bf16_from_f32(x));
}

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
}

/* f32 dot in the fixed 8-lane order described at the top of the file. */
static float dot_f32(const float *a, const float *b, int64_t n) {
  float lane[LANES] = {0};
  int64_t i = 0;
  for (; i + LANES <= n; i += LANES)
    for (int l = 0; l < LANES; ++l) lane[l] += a[i + l] * b[i + l];
  for (int l = 0; i < n; ++i, ++l) lane[l] += a[i] * b[i];
  float s4[4], s2[2];
  for (int l = 0; l < 4; ++l) s4[l] = lane[l] + lane[l + 4];
  for (int l = 0; l < 2; ++l) s2[l] = s4[l] + s4[l + 2];
  return s2[0] + s2[1];
}

static double dot_f64(const float *a, const float *b, int64_t n) {
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) s += (double)a[i] * (double)b[i];
  return s;
}

static float sum_f32(const float *a, int64_t n) {
  float lane[LANES] = {0};
  int64_t i = 0;
  for (; i + LANES <= n; i += LANES)
    for (int l = 0; l < LANES; ++l) lane[l] += a[i + l];
  for (int l = 0; i < n; ++i, ++l) lane[l] += a[i];
  float s4[4], s2[2];
  for (int l = 0; l < 4; ++l) s4[l] = lane[l] + lane[l + 4];
  for (int l = 0; l < 2; ++l) s2[l] = s4[l] + s4[l + 2];
  return s2[0] + s2[1];
}

/* ---- a1: W8 encoder (benchmarks/quantize_qwen3_5_w8.py:27-44) ------------ */

int rxo_quantize_w8(const float *w, int64_t n, int64_t k, int64_t g,
                    uint8_t *u8_out, float *scale_out) {
  if (n <= 0 || k <= 0 || g <= 0 || k % g != 0) return -1;
  const int64_t groups = k / g;
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t gi = 0; gi < groups; ++gi) {
      const float *src = w + r * k + gi * g;
      float amax = 0.0f;
      for (int64_t i = 0; i < g; ++i) {
        float a = fabsf(src[i]);
        if (a > amax || isnan(a)) amax = a; /* torch amax propagates NaN */
      }
      /* clamp_min(1e-12) / 127.0, both in f32 */
      float lo = 1e-12f;
      float clamped = (isnan(amax) || amax >= lo) ? amax : lo;
      float s = clamped / 127.0f;
      scale_out[r * groups + gi] = s;
      for (int64_t i = 0; i < g; ++i) {
        float qf = nearbyintf(src[i] / s); /* f32 division, RNE */
        if (qf > 127.0f) qf = 127.0f;
        if (qf < -127.0f) qf = -127.0f;
        u8_out[r * k + gi * g + i] = (uint8_t)((int)qf + 128);
      }
    }
  }
  return 0;
}

/* ---- a2: dequantisation (crates/rxla-nn/src/layers.rs:277-287) ---------- */

int rxo_dequantize_w8(const uint8_t *u8, const float *scale, int64_t n,
                      int64_t k, int64_t g, float *w_out) {
  if (n <= 0 || k <= 0 || g <= 0 || k % g != 0) return -1;
  const int64_t groups = k / g;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t i = 0; i < k; ++i) {
      float c = (float)u8[r * k + i] + -128.0f;
      w_out[r * k + i] = c * scale[r * groups + i / g];
    }
  return 0;
}

/* ---- a2/a3: linear -------------------------------------------------------- */

int rxo_quantized_linear(const float *x, int64_t m, int64_t k, const uint8_t *u8,
                         const float *scale, int64_t n, int64_t g, int compute,
                         int accum, float *y, int threads) {
  if (m < 0 || n <= 0 || k <= 0 || g <= 0 || k % g != 0) return -1;
  if (compute != RXO_COMPUTE_F32 && compute != RXO_COMPUTE_BF16) return -1;
  const int64_t groups = k / g;
  /* bf16(x) (layers.rs:292-293 input.cast(compute_dtype)) */
  float *xc = (float *)malloc(sizeof(float) * (size_t)(m * k + 1));
  if (!xc) return -2;
  for (int64_t i = 0; i < m * k; ++i)
    xc[i] = compute == RXO_COMPUTE_BF16 ? round_bf16(x[i]) : x[i];
  set_threads(threads);
  int fail = 0;
#pragma omp parallel
  {
    float *wrow = (float *)malloc(sizeof(float) * (size_t)k);
    if (!wrow) {
#pragma omp atomic write
      fail = 1;
    } else {
#pragma omp for schedule(static)
      for (int64_t r = 0; r < n; ++r) {
        for (int64_t i = 0; i < k; ++i) {
          float wdq = ((float)u8[r * k + i] + -128.0f) * scale[r * groups + i / g];
          /* weight.cast(compute_dtype) (layers.rs:294) */
          wrow[i] = compute == RXO_COMPUTE_BF16 ? round_bf16(wdq) : wdq;
        }
        for (int64_t row = 0; row < m; ++row) {
          float acc = accum == RXO_ACCUM_F64 ? (float)dot_f64(xc + row * k, wrow, k)
                                             : dot_f32(xc + row * k, wrow, k);
          /* bf16 dot_general result type, then .cast(F32) (layers.rs:295-296) */
          y[row * n + r] = compute == RXO_COMPUTE_BF16 ? round_bf16(acc) : acc;
        }
      }
      free(wrow);
    }
  }
  free(xc);
  return fail ? -2 : 0;
}

int rxo_linear_bf16w(const float *x, int64_t m, int64_t k, const uint16_t *w,
                     int64_t n, int accum, float *y, int threads) {
  if (m < 0 || n <= 0 || k <= 0) return -1;
  float *xc = (float *)malloc(sizeof(float) * (size_t)(m * k + 1));
  if (!xc) return -2;
  for (int64_t i = 0; i < m * k; ++i) xc[i] = round_bf16(x[i]);
  set_threads(threads);
  int fail = 0;
#pragma omp parallel
  {
    float *wrow = (float *)malloc(sizeof(float) * (size_t)k);
    if (!wrow) {
#pragma omp atomic write
      fail = 1;
    } else {
#pragma omp for schedule(static)
      for (int64_t r = 0; r < n; ++r) {
        for (int64_t i = 0; i < k; ++i) wrow[i] = rxo_f32_from_bf16(w[r * k + i]);
        for (int64_t row = 0; row < m; ++row) {
          float acc = accum == RXO_ACCUM_F64 ? (float)dot_f64(xc + row * k, wrow, k)
                                             : dot_f32(xc + row * k, wrow, k);
          y[row * n + r] = round_bf16(acc);
        }
      }
      free(wrow);
    }
  }
  free(xc);
  return fail ? -2 : 0;
}

/* ---- a5-a7: attention ------------------------------------------------------ */

/* One query row against `sk` keys, reference lowering order
 * (conversion.rs:363-499): dot, *scale, +mask, max, sub, exp, sum, divide,
 * dot with V. k_at/v_at give row pointers (f32). */
static void attend_row_f32(const float *q, int64_t d, int64_t dv, int64_t sk,
                           const float *const *krows, const float *const *vrows,
                           const float *mask_row, float scale, float *scores,
                           float *out) {
  float mx = -INFINITY;
  for (int64_t j = 0; j < sk; ++j) {
    float s = dot_f32(q, krows[j], d) * scale;
    if (mask_row) s += mask_row[j];
    scores[j] = s;
    if (s > mx) mx = s;
  }
  for (int64_t j = 0; j < sk; ++j) scores[j] = expf(scores[j] - mx);
  float denom = sum_f32(scores, sk);
  for (int64_t j = 0; j < sk; ++j) scores[j] = scores[j] / denom;
  for (int64_t c = 0; c < dv; ++c) {
    float lane[LANES] = {0};
    int64_t j = 0;
    for (; j + LANES <= sk; j += LANES)
      for (int l = 0; l < LANES; ++l) lane[l] += scores[j + l] * vrows[j + l][c];
    for (int l = 0; j < sk; ++j, ++l) lane[l] += scores[j] * vrows[j][c];
    float s4[4], s2[2];
    for (int l = 0; l < 4; ++l) s4[l] = lane[l] + lane[l + 4];
    for (int l = 0; l < 2; ++l) s2[l] = s4[l] + s4[l + 2];
    out[c] = s2[0] + s2[1];
  }
}

static void attend_row_f64(const float *q, int64_t d, int64_t dv, int64_t sk,
                           const float *const *krows, const float *const *vrows,
                           const float *mask_row, float scale, double *scores,
                           float *out) {
  double mx = -INFINITY;
  for (int64_t j = 0; j < sk; ++j) {
    double s = dot_f64(q, krows[j], d) * (double)scale;
    if (mask_row) s += (double)mask_row[j];
    scores[j] = s;
    if (s > mx) mx = s;
  }
  double denom = 0.0;
  for (int64_t j = 0; j < sk; ++j) {
    scores[j] = exp(scores[j] - mx);
    denom += scores[j];
  }
  for (int64_t c = 0; c < dv; ++c) {
    double acc = 0.0;
    for (int64_t j = 0; j < sk; ++j) acc += scores[j] / denom * (double)vrows[j][c];
    out[c] = (float)acc;
  }
}

int rxo_gqa_attention(const float *q, const float *k, const float *v,
                      int64_t b, int64_t hq, int64_t hkv, int64_t sq,
                      int64_t sk, int64_t d, int64_t dv, const float *mask,
                      int64_t mask_sb, int64_t mask_sh, int64_t mask_si,
                      float scale, int precision, float *out, int threads) {
  if (b < 0 || hq <= 0 || hkv <= 0 || hq % hkv != 0 || sq < 0 || sk <= 0 ||
      d <= 0 || dv <= 0)
    return -1;
  const int64_t group = hq / hkv;
  set_threads(threads);
  int fail = 0;
#pragma omp parallel
  {
    const float **krows = (const float **)malloc(sizeof(float *) * (size_t)sk);
    const float **vrows = (const float **)malloc(sizeof(float *) * (size_t)sk);
    double *scores = (double *)malloc(sizeof(double) * (size_t)sk);
    if (!krows || !vrows || !scores) {
#pragma omp atomic write
      fail = 1;
    } else {
#pragma omp for collapse(2) schedule(static)
      for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t h = 0; h < hq; ++h) {
          const int64_t kv = h / group; /* consecutive heads share a kv head */
          for (int64_t j = 0; j < sk; ++j) {
            krows[j] = k + ((bi * hkv + kv) * sk + j) * d;
            vrows[j] = v + ((bi * hkv + kv) * sk + j) * dv;
          }
          for (int64_t i = 0; i < sq; ++i) {
            const float *qrow = q + ((bi * hq + h) * sq + i) * d;
            const float *mrow =
                mask ? mask + bi * mask_sb + h * mask_sh + i * mask_si : NULL;
            float *orow = out + ((bi * hq + h) * sq + i) * dv;
            if (precision == 1)
              attend_row_f64(qrow, d, dv, sk, krows, vrows, mrow, scale, scores, orow);
            else
              attend_row_f32(qrow, d, dv, sk, krows, vrows, mrow, scale,
                             (float *)scores, orow);
          }
        }
    }
    free(krows);
    free(vrows);
    free(scores);
  }
  return fail ? -2 : 0;
}

int rxo_gqa_decode_bf16cache(const float *q, const uint16_t *kc,
                             const uint16_t *vc, const int32_t *lens,
                             int64_t b, int64_t hq, int64_t hkv, int64_t lmax,
                             int64_t d, float scale, int precision, float *out,
                             int threads) {
  if (b < 0 || hq <= 0 || hkv <= 0 || hq % hkv != 0 || lmax <= 0 || d <= 0)
    return -1;
  for (int64_t bi = 0; bi < b; ++bi)
    if (lens[bi] < 1 || lens[bi] > lmax) return -1;
  const int64_t group = hq / hkv;
  set_threads(threads);
  int fail = 0;
#pragma omp parallel
  {
    float *kf = (float *)malloc(sizeof(float) * (size_t)(lmax * d));
    float *vf = (float *)malloc(sizeof(float) * (size_t)(lmax * d));
    const float **krows = (const float **)malloc(sizeof(float *) * (size_t)lmax);
    const float **vrows = (const float **)malloc(sizeof(float *) * (size_t)lmax);
    double *scores = (double *)malloc(sizeof(double) * (size_t)lmax);
    if (!kf || !vf || !krows || !vrows || !scores) {
#pragma omp atomic write
      fail = 1;
    } else {
#pragma omp for collapse(2) schedule(dynamic)
      for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t kv = 0; kv < hkv; ++kv) {
          const int64_t len = lens[bi];
          const uint16_t *ks = kc + (bi * hkv + kv) * lmax * d;
          const uint16_t *vs = vc + (bi * hkv + kv) * lmax * d;
          rxo_bf16_to_f32(ks, kf, len * d);
          rxo_bf16_to_f32(vs, vf, len * d);
          for (int64_t j = 0; j < len; ++j) {
            krows[j] = kf + j * d;
            vrows[j] = vf + j * d;
          }
          for (int64_t gi = 0; gi < group; ++gi) {
            const int64_t h = kv * group + gi;
            const float *qrow = q + (bi * hq + h) * d;
            float *orow = out + (bi * hq + h) * d;
            if (precision == 1)
              attend_row_f64(qrow, d, d, len, krows, vrows, NULL, scale, scores, orow);
            else
              attend_row_f32(qrow, d, d, len, krows, vrows, NULL, scale,
                             (float *)scores, orow);
          }
        }
    }
    free(kf);
    free(vf);
    free(krows);
    free(vrows);
    free(scores);
  }
  return fail ? -2 : 0;
}

/* ---- a8: KV cache ------------------------------------------------------------ */

int rxo_dynamic_update_slice(void *operand, const int64_t *dims, int rank,
                             int64_t elem_size, const void *update,
                             const int64_t *udims, const int32_t *starts) {
  if (rank <= 0 || rank > 8 || elem_size <= 0) return -1;
  int64_t st[8], ustride[8], ostride[8];
  int64_t total = 1;
  for (int a = 0; a < rank; ++a) {
    if (udims[a] < 0 || udims[a] > dims[a]) return -1;
    int64_t hi = dims[a] - udims[a];
    int64_t s = starts[a];
    st[a] = s < 0 ? 0 : (s > hi ? hi : s); /* XLA start clamping */
    total *= udims[a];
  }
  ustride[rank - 1] = 1;
  ostride[rank - 1] = 1;
  for (int a = rank - 2; a >= 0; --a) {
    ustride[a] = ustride[a + 1] * udims[a + 1];
    ostride[a] = ostride[a + 1] * dims[a + 1];
  }
  for (int64_t e = 0; e < total; ++e) {
    int64_t rem = e, off = 0;
    for (int a = 0; a < rank; ++a) {
      int64_t idx = rem / ustride[a];
      rem %= ustride[a];
      off += (st[a] + idx) * ostride[a];
    }
    memcpy((char *)operand + off * elem_size, (const char *)update + e * elem_size,
           (size_t)elem_size);
  }
  return 0;
}

int rxo_kv_update_at(void *kc, void *vc, const int64_t *dims, int rank,
                     int64_t elem_size, const void *ku, const void *vu,
                     const int64_t *udims, const int32_t *starts, int checked,
                     float *accepted) {
  if (rank <= 0 || rank > 8) return -1;
  for (int a = 0; a < rank; ++a)
    if (udims[a] < 0 || udims[a] > dims[a]) return -1;
  if (checked) {
    /* kv_cache.rs:96-103: 0 <= start, and start <= dim - udim when that
     * limit is below i32::MAX. */
    int ok = 1;
    for (int a = 0; a < rank; ++a) {
      int64_t limit = dims[a] - udims[a];
      if (starts[a] < 0) ok = 0;
      if (limit < 2147483647LL && (int64_t)starts[a] > limit) ok = 0;
    }
    if (accepted) *accepted = ok ? 1.0f : 0.0f;
    if (!ok) return 0;
  } else if (accepted) {
    *accepted = 1.0f;
  }
  int rc = rxo_dynamic_update_slice(kc, dims, rank, elem_size, ku, udims, starts);
  if (rc) return rc;
  return rxo_dynamic_update_slice(vc, dims, rank, elem_size, vu, udims, starts);
}

/* ---- a10-a14 ------------------------------------------------------------------ */

void rxo_rope_freqs(float theta, int64_t rot_dim, float *freqs) {
  for (int64_t i = 0; i < rot_dim / 2; ++i)
    freqs[i] = powf(theta, -2.0f * (float)i / (float)rot_dim);
}

void rxo_rope_split_half(float *x, int64_t rows, int64_t d, int64_t rot_dim,
                         const int32_t *pos, int64_t rows_per_pos,
                         float theta) {
  const int64_t half = rot_dim / 2;
  float *freqs = (float *)malloc(sizeof(float) * (size_t)(half + 1));
  if (!freqs) return;
  rxo_rope_freqs(theta, rot_dim, freqs);
  for (int64_t r = 0; r < rows; ++r) {
    float *row = x + r * d;
    const float p = (float)pos[r / rows_per_pos];
    for (int64_t i = 0; i < half; ++i) {
      const float ang = p * freqs[i];
      const float c = cosf(ang), s = sinf(ang);
      const float a = row[i], bb = row[i + half];
      row[i] = a * c - bb * s;
      row[i + half] = bb * c + a * s;
    }
  }
  free(freqs);
}

void rxo_rms_norm(const float *x, int64_t rows, int64_t h, const float *w,
                  float eps, int zero_centered, float *y) {
  float *sq = (float *)malloc(sizeof(float) * (size_t)h);
  if (!sq) return;
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * h;
    for (int64_t i = 0; i < h; ++i) sq[i] = xr[i] * xr[i];
    const float mean = sum_f32(sq, h) / (float)h;
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < h; ++i) {
      const float wi = zero_centered ? 1.0f + w[i] : w[i];
      y[r * h + i] = (xr[i] * scale) * wi;
    }
  }
  free(sq);
}

void rxo_silu_mul(const float *gate, const float *up, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) {
    const float g = gate[i];
    const float sig = 1.0f / (1.0f + expf(-g));
    out[i] = (g * sig) * up[i];
  }
}

void rxo_take_rows(const void *table, int64_t v, int64_t row_bytes,
                   const int32_t *ids, int64_t n, void *out) {
  for (int64_t i = 0; i < n; ++i) {
    int64_t id = ids[i];
    if (id < 0) id = 0;
    if (id > v - 1) id = v - 1;
    memcpy((char *)out + i * row_bytes, (const char *)table + id * row_bytes,
           (size_t)row_bytes);
  }
}

void rxo_argmax_rows(const float *x, int64_t rows, int64_t cols, int32_t *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * cols;
    int64_t best = 0;
    for (int64_t c = 1; c < cols; ++c) {
      const float a = xr[c], bcur = xr[best];
      if (!isnan(bcur) && (isnan(a) || a > bcur)) best = c;
    }
    out[r] = (int32_t)best;
  }
}

/* ---- a15: decoder ------------------------------------------------------------- */

int rxo_decoder_forward(const rxo_decoder_config *cfg,
                        const rxo_decoder_params *p, uint16_t *k_cache,
                        uint16_t *v_cache, int32_t *lens, int64_t b, int64_t s,
                        const int32_t *ids, float *logits, int32_t *next_ids,
                        int threads) {
  return rxo_decoder_forward_trace(cfg, p, k_cache, v_cache, lens, b, s, ids,
                                   logits, next_ids, threads, NULL);
}

int rxo_decoder_forward_trace(const rxo_decoder_config *cfg,
                              const rxo_decoder_params *p, uint16_t *k_cache,
                              uint16_t *v_cache, int32_t *lens, int64_t b,
                              int64_t s, const int32_t *ids, float *logits,
                              int32_t *next_ids, int threads, float *trace) {
  const int64_t H = cfg->hidden, HQ = cfg->q_heads, HKV = cfg->kv_heads;
  const int64_t D = cfg->head_dim, I = cfg->intermediate, V = cfg->vocab;
  const int64_t L = cfg->max_seq, G = cfg->group;
  const int64_t QKV = (HQ + 2 * HKV) * D;
  const int64_t T = b * s; /* token rows, row = bi * s + t */
  /* group 0: per-output-channel scales (each linear's G is its input width) */
  const int64_t G_H = G > 0 ? G : H, G_I = G > 0 ? G : I, G_O = G > 0 ? G : HQ * D;
  if (b <= 0 || s <= 0 || HQ % HKV || H % G_H || I % G_I || (HQ * D) % G_O) return -1;
  for (int64_t bi = 0; bi < b; ++bi)
    if (lens[bi] < 0 || lens[bi] + s > L) return -1;

  float *h = (float *)malloc(sizeof(float) * (size_t)(T * H));
  float *n = (float *)malloc(sizeof(float) * (size_t)(T * (H > I ? H : I)));
  float *qkv = (float *)malloc(sizeof(float) * (size_t)(T * QKV));
  float *q = (float *)malloc(sizeof(float) * (size_t)(T * HQ * D));
  float *kn = (float *)malloc(sizeof(float) * (size_t)(T * HKV * D));
  float *att = (float *)malloc(sizeof(float) * (size_t)(T * HQ * D));
  float *tmp = (float *)malloc(sizeof(float) * (size_t)(T * H));
  float *gu = (float *)malloc(sizeof(float) * (size_t)(T * 2 * I));
  float *act = (float *)malloc(sizeof(float) * (size_t)(T * I));
  int32_t *pos = (int32_t *)malloc(sizeof(int32_t) * (size_t)T);
  uint16_t *emb = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(T * H));
  int rc = 0;
  if (!h || !n || !qkv || !q || !kn || !att || !tmp || !gu || !act || !pos || !emb) {
    rc = -2;
    goto done;
  }
  for (int64_t bi = 0; bi < b; ++bi)
    for (int64_t t = 0; t < s; ++t) pos[bi * s + t] = lens[bi] + (int32_t)t;

  /* embedding: bf16 row gather with clamped ids, widened to f32 */
  rxo_take_rows(p->embed, V, H * 2, ids, T, emb);
  rxo_bf16_to_f32(emb, h, T * H);

  const float scale = 1.0f / sqrtf((float)D);
  for (int64_t l = 0; l < cfg->layers; ++l) {
    if (trace) memcpy(trace + l * T * H, h, sizeof(float) * (size_t)(T * H));
    uint16_t *kcl = k_cache + l * b * HKV * L * D;
    uint16_t *vcl = v_cache + l * b * HKV * L * D;
    rxo_rms_norm(h, T, H, p->in_norm[l], cfg->eps, 0, n);
    rc = rxo_quantized_linear(n, T, H, p->qkv_w[l], p->qkv_s[l], QKV, G_H,
                              RXO_COMPUTE_BF16, cfg->accum, qkv, threads);
    if (rc) goto done;
    for (int64_t r = 0; r < T; ++r) {
      memcpy(q + r * HQ * D, qkv + r * QKV, sizeof(float) * (size_t)(HQ * D));
      memcpy(kn + r * HKV * D, qkv + r * QKV + HQ * D, sizeof(float) * (size_t)(HKV * D));
    }
    if (cfg->qk_norm) {
      rxo_rms_norm(q, T * HQ, D, p->q_norm[l], cfg->eps, 0, q);
      rxo_rms_norm(kn, T * HKV, D, p->k_norm[l], cfg->eps, 0, kn);
    }
    rxo_rope_split_half(q, T * HQ, D, D, pos, HQ, cfg->theta);
    rxo_rope_split_half(kn, T * HKV, D, D, pos, HKV, cfg->theta);
    /* KV append (bf16 cache) at each token's position */
    for (int64_t r = 0; r < T; ++r) {
      const int64_t bi = r / s;
      for (int64_t kv = 0; kv < HKV; ++kv) {
        uint16_t *kd = kcl + ((bi * HKV + kv) * L + pos[r]) * D;
        uint16_t *vd = vcl + ((bi * HKV + kv) * L + pos[r]) * D;
        rxo_f32_to_bf16(kn + (r * HKV + kv) * D, kd, D);
        rxo_f32_to_bf16(qkv + r * QKV + (HQ + HKV + kv) * D, vd, D);
      }
    }
    /* causal GQA attention: token r sees keys 0..pos[r] */
    set_threads(threads);
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int64_t r = 0; r < T; ++r)
      for (int64_t hh = 0; hh < HQ; ++hh) {
        const int64_t bi = r / s;
        const int32_t len = pos[r] + 1;
        rxo_gqa_decode_bf16cache(q + (r * HQ + hh) * D,
                                 kcl + (bi * HKV + hh / (HQ / HKV)) * L * D,
                                 vcl + (bi * HKV + hh / (HQ / HKV)) * L * D, &len,
                                 1, 1, 1, L, D, scale, 0, att + (r * HQ + hh) * D, 1);
      }
    rc = rxo_quantized_linear(att, T, HQ * D, p->o_w[l], p->o_s[l], H, G_O,
                              RXO_COMPUTE_BF16, cfg->accum, tmp, threads);
    if (rc) goto done;
    for (int64_t i = 0; i < T * H; ++i) h[i] += tmp[i];
    rxo_rms_norm(h, T, H, p->post_norm[l], cfg->eps, 0, n);
    rc = rxo_quantized_linear(n, T, H, p->gu_w[l], p->gu_s[l], 2 * I, G_H,
                              RXO_COMPUTE_BF16, cfg->accum, gu, threads);
    if (rc) goto done;
    for (int64_t r = 0; r < T; ++r)
      rxo_silu_mul(gu + r * 2 * I, gu + r * 2 * I + I, I, act + r * I);
    rc = rxo_quantized_linear(act, T, I, p->down_w[l], p->down_s[l], H, G_I,
                              RXO_COMPUTE_BF16, cfg->accum, tmp, threads);
    if (rc) goto done;
    for (int64_t i = 0; i < T * H; ++i) h[i] += tmp[i];
  }
  if (trace) memcpy(trace + cfg->layers * T * H, h, sizeof(float) * (size_t)(T * H));
  /* final norm + tied bf16 lm_head on the last new position of each sequence */
  for (int64_t bi = 0; bi < b; ++bi)
    memcpy(tmp + bi * H, h + (bi * s + s - 1) * H, sizeof(float) * (size_t)H);
  rxo_rms_norm(tmp, b, H, p->final_norm, cfg->eps, 0, n);
  rc = rxo_linear_bf16w(n, b, H, p->embed, V, cfg->accum, logits, threads);
  if (rc) goto done;
  rxo_argmax_rows(logits, b, V, next_ids);
  for (int64_t bi = 0; bi < b; ++bi) lens[bi] += (int32_t)s;
done:
  free(h);
  free(n);
  free(qkv);
  free(q);
  free(kn);
  free(att);
  free(tmp);
  free(gu);
  free(act);
  free(pos);
  free(emb);
  return rc;
}
