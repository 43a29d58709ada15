// rxw8 op entry points: validation (before any launch) and kernel dispatch.
//
// Validation mirrors the reference's InvalidLayerInput / BufferShape /
// BufferDType checks (crates/rxla-nn/src/layers.rs:258-274,
// crates/rxla-nn/src/applied.rs:1274-1297, attention.rs:83-252,
// kv_cache.rs:53-111); a rejected call launches nothing and mutates nothing.
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "internal.h"

namespace rxw8 {

// Kernel argument structs (must match the .hip definitions byte for byte).
struct GemvArgs {
  const void *x;
  const void *w;
  const float *scale;
  void *y;
  float *ws;
  int M, N, K, G;
  int ksplit;
  int x_f32, y_f32;
  int y_mode;
  float *ss_out;
  int x_mode;
  int64_t x_stride, x_off;
  const float *norm_w;
  float eps;
  const float *ss_in;
  int ss_parts;
  int wave_stage;
  int lds_dma;  // bf16 rows staged by LDS DMA
  int row_norm;  // RMSNorm factor applied after the product (x = bf16(h * w))
  int rs_off;    // LDS byte offset of the row factors
  const float *xw_norm;
  uint16_t *xw_out;
  int ss_ld;  // row stride of the sum-of-squares partials
  int chunk_rows;  // F32-compute kernels: rows per grid row (blockIdx.y)
  int fc_kmajor;   // F32 staging in column-major piece order where it fits
};

struct PackArgs {
  const void *src;
  void *dst;
  int64_t n, k;
  int kb;
  int esize;
  int64_t ilv_half;
};

// Grouped GEMV launch (matches kernels/w8a16_gemv.hip).
struct GemvProblem {
  const void *x;
  const void *w;
  const float *scale;
  void *y;
  int M, N, K, G;
  int tile_begin;
  int x_f32, y_f32, lds_dma, wave_stage;
};
constexpr int kGemvGroupMax = 16;
struct GemvGroupArgs {
  GemvArgs base;
  int count;
  GemvProblem p[kGemvGroupMax];
};

struct SplitkReduceArgs {
  const float *ws;
  const float *scale;
  void *y;
  int M, N, ksplit;
  int y_f32;
  int y_mode;
};

struct GemmArgs {
  const uint16_t *x;
  const uint8_t *w;
  const float *scale;
  void *y;
  int M, N, K, G;
  int y_f32, y_mode, w_packed;
  int group_n;
  int ksplit;
  float *ws;
};

struct DequantWArgs {
  const uint8_t *w;
  const float *scale;
  uint16_t *out;
  int N, K, G, packed;
};

struct CastArgs {
  const float *x;
  uint16_t *y;
  int64_t n;
};

struct DequantArgs {
  const uint8_t *w;
  const float *scale;
  void *out;
  int64_t n, k, g;
  int out_bf16;
};

struct QuantizeArgs {
  const void *w;
  uint8_t *u8;
  float *scale;
  int64_t n, k, g;
  int w_bf16;
};

struct GqaGeneralArgs {
  const void *q, *k, *v;
  const float *mask;
  void *out;
  int64_t bdim[4];
  int64_t mb[4];
  int64_t msh, msi, msj;
  int64_t rows;
  int Hq, Hkv, Sq, Sk, D, Dv;
  float scale;
  int64_t q_sb, q_sh, q_si;
  int64_t o_sb, o_sh, o_si;
  int64_t k_sb, k_sh;
  int64_t v_sb, v_sh;
  int q_bf16, kv_bf16, out_bf16;
  const int32_t *starts;
};

struct CausalMaskArgs {
  const int32_t *qpos, *kpos;
  float *out;
  int64_t Q, K;
};

struct GenericLinearArgs {
  const void *x;
  const void *w;
  const float *scale;
  void *y;
  int64_t m, n, k, g;
  int x_f32, y_f32, compute_bf16, w_kind;
  int y_mode;
};

struct LinearF32Args {
  const float *x;
  const uint8_t *w;
  const float *scale;
  float *y;
  int T, N, K, G;
  int y_mode;
  int tiles;
  int64_t ldx, ldw, ldsc;
};

struct KvUpdateArgs {
  void *kc;
  void *vc;
  const void *ku;
  const void *vu;
  const int32_t *starts;
  float *accepted;
  int64_t dims[8];
  int64_t udims[8];
  int64_t total;
  int rank;
  int elem;
  int checked;
};

struct AttnArgs {
  const void *q;
  const uint16_t *kc;
  const uint16_t *vc;
  const int32_t *lens;
  const int32_t *row_seq;
  const float *mask;
  void *out;
  float *ws;
  int64_t mask_sb, mask_sh;
  int R, Hq, Hkv, Lmax, max_chunks;
  float scale;
  int q_f32, out_f32;
  const uint16_t *qkv;
  const float *q_norm, *k_norm;
  const float *rope;
  float eps;
  int *counters;
  int units;
};

struct PrefillArgs {
  const void *q;
  const uint16_t *kc, *vc;
  const int32_t *starts;
  const int32_t *slots;
  void *out;
  int64_t q_sb, q_ss, q_sh, o_sb, o_ss, o_sh;
  int B, S, Hq, Hkv, Lmax, nqb;
  float scale;
  int q_f32, out_f32;
};

struct AttnGenericArgs {
  const void *q;
  const void *kc;
  const void *vc;
  const int32_t *lens;
  const int32_t *row_seq;
  const float *mask;
  void *out;
  int64_t mask_sb, mask_sh;
  int B, Hq, Hkv, Lmax, D;
  float scale;
  int q_f32, cache_f32, out_f32;
};

static unsigned grid_for(int64_t n, int per_block = 256, int64_t cap = 1 << 16) {
  int64_t g = (n + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

static int env_int(const char *name, int dflt) {
  const char *v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

// GEMV launch plan: row groups per workgroup (RW), K-split, double-buffer depth.
struct GemvPlan {
  int rw = 0, ks = 0, u = 0, mb = 1, nw = 4;  // nw: waves per workgroup
  size_t lds = 0;
};

// Whether plain rows (x_mode 0) are staged per wave (each wave its own K
// slice, no workgroup barrier): per-channel u8 weights with one row, or up to
// RXW8_GEMV_WAVE_M rows (default 4) with one row group per workgroup.
static bool gemv_wave_stage(int64_t m, int64_t k, int64_t g, int rw, bool w_bf16) {
  static const int max_m = [] {
    const char *v = std::getenv("RXW8_GEMV_WAVE_M");
    return v && *v ? std::atoi(v) : 4;
  }();
  return g == k && !w_bf16 && (m == 1 || (rw == 1 && m <= max_m));
}

// LDS of one GEMV workgroup: the [m, kc] bf16 activation slice (rows padded by
// 8), the grouped-scale tile [16*rw, kc/g] f32, and the cross-wave reduction
// area (reused after the loop) of (4/rw - 1) * rw * mb f32 tiles of 16x16.
static size_t gemv_lds(int64_t m, int64_t kc, int64_t k, int64_t g, int rw, int mb,
                       bool w_bf16, int nw = 4) {
  size_t stage = (size_t)m * (kc + 8) * 2 + (g == k ? 0 : (size_t)16 * rw * (kc / g) * 4);
  // per-wave staging: each of the nw waves stages its own K slice
  // (kc / (nw / rw) values) of the m rows in a region of its own
  if (gemv_wave_stage(m, k, g, rw, w_bf16)) {
    const size_t per_wave = (size_t)nw * m * (kc / (nw / rw) + 8) * 2;
    if (per_wave > stage) stage = per_wave;
  }
  const size_t red = (size_t)(nw / rw - 1) * rw * mb * 256 * 4;
  return stage > red ? stage : red;
}

// Workgroups cover 16 channels (4 waves split K) for m <= 4, else 64 channels
// (x staged once for 4 row groups). The split is the smallest power of two
// that gives every CU a workgroup while the staged slice fits 64 KiB and each
// wave gets an even number of 16-byte slices. RXW8_GEMV_KSPLIT /
// RXW8_GEMV_RW override for tuning.
static GemvPlan plan_gemv(const Runtime *rt, int64_t m, int64_t n, int64_t k, int64_t g,
                          bool w_bf16, bool prefer_ks1 = false, bool allow_wide = true) {
  GemvPlan p;
  p.mb = m <= 16 ? 1 : 2;
  const int forced_rw = env_int("RXW8_GEMV_RW", 0);
  p.rw = forced_rw == 1 || forced_rw == 4 ? forced_rw : (m <= 4 || prefer_ks1 ? 1 : 4);
  const int64_t slice = w_bf16 ? 32 : 64;  // k per 16-byte lane load
  const bool per_channel = g == k;
  // A single launch without a split-K reduce: 16, 14, 12 or 8 waves per
  // workgroup split K inside the workgroup when each wave still gets an even
  // number of 64-k slices (u8 weights, rw groups of 16 rows per workgroup).
  // Wider row tiles cut the staging each workgroup does per weight byte. First
  // choice: the widest tiling whose workgroups fill the CUs in whole rounds
  // (no CU idles behind a partial last round); else the widest that still
  // gives every CU a workgroup. U: the deepest unroll (of 4, 3, 2, 1) that
  // divides the wave's slices into A/B groups.
  if (prefer_ks1 && allow_wide && !w_bf16 && forced_rw == 0) {
    const int forced_nw = env_int("RXW8_GEMV_NW", 0);
    // Many activation rows (m > 4) make staging the cost per weight byte:
    // 96-row tiles (12 waves as 6 row groups) come first there, and 8-wave
    // workgroups before 16-wave ones (half the cross-wave reduction per tile;
    // measured at 8 and 16 rows, e.g. 8 x 4096 x 2048: 4.8 vs 4.8 us, 16 x
    // 4096 x 4096: 9.2 vs 10.4 us).
    static const int shapes_few[][2] = {{16, 4}, {12, 3}, {16, 2}, {16, 1}, {14, 1},
                                        {8, 4}, {8, 2}, {8, 1}, {12, 6}};
    static const int shapes_many[][2] = {{12, 6}, {12, 3}, {8, 4}, {8, 2}, {8, 1},
                                         {16, 4}, {16, 2}, {16, 1}, {14, 1}};
    const auto &shapes = m > 4 ? shapes_many : shapes_few;
    const int forced_rw6 = env_int("RXW8_GEMV_RW6", -1);
    for (int pass = 0; pass < 2; ++pass) {
      for (const auto &sh : shapes) {
        const int nw = sh[0], rw = sh[1];
        if (rw == 6 && (p.mb != 1 || pass == 1 || !(forced_rw6 >= 0 ? forced_rw6 : m > 4))) continue;
        if (forced_nw && forced_nw != nw) continue;
        const int kw = nw / rw;
        const int64_t tiles = (n + 16 * rw - 1) / (16 * rw);
        if (pass == 0 && (n % (16 * rw) || tiles % rt->cus)) continue;
        if (pass == 1 && rw > 1 && tiles < rt->cus) continue;
        if (pass == 1 && rw == 3) continue;
        if (k % kw || (k / kw) % (2 * slice)) continue;
        // grouped scales: every wave's K slice holds whole groups (the kernel
        // folds a group's sum within one wave)
        if (!per_channel && (k / kw) % g) continue;
        const size_t lds = gemv_lds(m, k, k, g, rw, p.mb, w_bf16, nw);
        if (lds + 256 > rt->lds_max) continue;
        p.nw = nw;
        p.rw = rw;
        p.ks = 1;
        p.lds = lds;
        const int64_t chunks = k / kw / slice;
        p.u = 4;
        while (chunks % (2 * p.u)) --p.u;
        return p;
      }
    }
  }
  // 4-wave plans: rw = 1 splits K over the 4 waves, so K per split must hold
  // 4 waves x an even number of slices (and whole scale groups per wave);
  // otherwise (narrow K such as 256, wide groups) rw = 4 (one wave per
  // 16-row group, the whole split each)
  if (forced_rw == 0 && p.rw == 1) {
    bool any = false;
    for (int ks = 1; ks <= 64 && !any; ++ks)
      any = k % ks == 0 && (k / ks) % 4 == 0 && (k / ks / 4) % (2 * slice) == 0 &&
            (per_channel || (k / ks / 4) % g == 0);
    if (!any) p.rw = 4;
  }
  const int kw = 4 / p.rw;
  const int64_t tiles = (n + 16 * p.rw - 1) / (16 * p.rw);
  const int forced_ks = env_int("RXW8_GEMV_KSPLIT", 0);
  // k splits: powers of two, and multiples of 3 for widths like 6144 whose
  // scale groups (e.g. 2048) no power-of-two split keeps whole
  static const int splits[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64};
  // Staged slices up to 64 KiB keep two or more workgroups per CU; larger ones
  // (up to the 160 KiB a workgroup may hold) only when no split fits in 64 KiB.
  // 256 B stay free for the kernels' static LDS (prologue reductions).
  int valid[12], nvalid = 0;
  for (size_t cap : {(size_t)65536, rt->lds_max}) {
    for (int ks : splits) {
      if (k % ks) continue;
      const int64_t kc = k / ks;
      if (kc % kw || (kc / kw) % (2 * slice)) continue;  // even slices per wave
      if (!per_channel && (kc / kw) % g) continue;         // whole groups per wave
      if (gemv_lds(m, kc, k, g, p.rw, p.mb, w_bf16) + 256 > cap) continue;
      valid[nvalid++] = ks;
    }
    if (nvalid) break;
  }
  if (nvalid == 0) return p;
  int pick = valid[nvalid - 1];
  if (forced_ks) {
    pick = 0;
    for (int i = 0; i < nvalid; ++i)
      if (valid[i] == forced_ks) pick = forced_ks;
    if (!pick) return p;
  } else if (prefer_ks1 && valid[0] == 1) {
    pick = 1;  // one launch, no reduce kernel: cheaper when launches dominate
  } else {
    for (int i = 0; i < nvalid; ++i)
      if (tiles * valid[i] >= rt->cus) {
        pick = valid[i];
        break;
      }
  }
  p.ks = pick;
  p.lds = gemv_lds(m, k / pick, k, g, p.rw, p.mb, w_bf16);
  const int64_t chunks = k / pick / kw / slice;
  // bf16 weights: 2-deep groups (48-54 VGPRs, 8 waves per SIMD) stream
  // faster than 4-deep (74-76, 6 waves): the lm_head's 622 MB (8 rows x
  // 2048 x 151936) in 101.5 against 104.6-105.0 us
  const int forced_u = env_int("RXW8_GEMV_U", 0);
  p.u = forced_u == 8 || forced_u == 4 || forced_u == 2 || forced_u == 1 ? forced_u : (w_bf16 ? 2 : 4);
  while (chunks % (2 * p.u)) p.u /= 2;
  return p;
}

static bool is_f(int dt) { return dt == RXW8_F32 || dt == RXW8_BF16; }

// y[M, N] = linear(x[M, K]) on the GEMV kernel in chunks of <= 32 rows, with an
// optional activation prologue (RMSNorm / SwiGLU applied while x is staged).
// Returns UNIMPLEMENTED (nothing launched) when no plan fits.
static int run_gemv(Runtime *rt, const void *x, int x_f32, const void *w, bool w_bf16,
                    bool packed, const float *scale, void *y, int y_f32, int64_t M, int64_t N,
                    int64_t K, int64_t G, int y_mode = 0, const GemvOptions *pro = nullptr) {
  // Plain calls take the wide single-launch tilings when even 64-row tiles
  // give every CU a workgroup (e.g. N = 24576) and there are several rows: x
  // is then staged once per 64 rows and no split-K reduce runs; so do 8 or
  // more rows over at most 17 MB of weights (one launch beats a split plus
  // its reduce there). Other shapes keep the 4-wave plans, which fill the CUs
  // with more, narrower tiles.
  // u8 weights enter the product at the reference's cast point, each weight
  // bf16((u - 128) * s) (the gemv_rc kernels); RXW8_GEMV_REF_CAST=0 selects
  // the exact codes u - 128 with the scale applied after the f32 sum instead
  const char *rc_env = std::getenv("RXW8_GEMV_REF_CAST");
  const bool ref_cast = !w_bf16 && !(rc_env && *rc_env == '0');
  // (one row at the reference's cast point: the 4-wave plan, 1536 workgroups
  // of 16 rows for N = 24576, streams faster than the wide tiles, 18.4
  // against 18.8 us; from 4 rows on the wide tiles win)
  GemvOptions plain;
  const int wide_env = env_int("RXW8_GEMV_PREFER_WIDE", -1);
  plain.prefer_ks1 =
      wide_env >= 0 ? wide_env != 0
                    : (!w_bf16 && ((N / 64 >= rt->cus && !(ref_cast && M == 1)) ||
                                   (M >= 8 && N * K <= 17000000)));
  if (!pro) pro = &plain;
  // Activations as MFMA fragments from global memory (XG) paid off for the
  // exact-code kernels when the weights are small next to the staging each
  // workgroup would do: up to 8 rows and 17 MB of weights (8 x 4096 x 2048
  // 5.6 -> 4.8 us; 25 MB and more, or 16 rows, stream slower because the
  // fragment reads load L2). With the reference cast point (16 more VALU ops
  // per 16 bytes of weights) staged rows are faster from 8 rows on: the C5
  // decode step's o_proj 4.84 -> 4.48 us, down 8.12 -> 7.32, QKV 5.96 ->
  // 5.80; up to 4 rows XG still wins (4 x 4096 x 4096: 6.0 against 6.8 us).
  // RXW8_GEMV_XG=0 / 1 forces it off / on (where it applies).
  static const int xg_env = env_int("RXW8_GEMV_XG", -1);
  const int xg_mode = xg_env >= 0 ? xg_env : (M <= (ref_cast ? 4 : 8) && N * K <= 17000000);
  const int64_t mchunk = M <= 16 ? 16 : 32;
  GemvPlan p = plan_gemv(rt, M < mchunk ? M : mchunk, N, K, G, w_bf16, pro->prefer_ks1,
                         pro->mode != 1);
  if (p.ks == 0 || N % 4) return RXW8_UNIMPLEMENTED;
  // the fused epilogues need the whole reduction in one launch and whole
  // 16-channel groups; one chunk of rows keeps the partial layout [g][M]
  if ((pro->swiglu || pro->ss_out) && (p.ks != 1 || N % 16 || M > mchunk)) return RXW8_UNIMPLEMENTED;
  if (pro->mode == 3 && M > mchunk) return RXW8_UNIMPLEMENTED;
  // the post-product RMSNorm reads its rows' partials (one chunk of rows,
  // at most 256 partials per row) and needs the whole sum in one launch
  // (kernels for packed weights and up to 16 rows)
  if (pro->row_norm && (pro->mode != 0 || x_f32 || !pro->ss_in || pro->ss_parts < 1 ||
                        pro->ss_parts > 256 || M > 16 || p.ks != 1 || !packed))
    return RXW8_UNIMPLEMENTED;
  if (pro->xw_out && (y_mode != 1 || p.ks != 1 || M > mchunk || N % 4)) return RXW8_UNIMPLEMENTED;
  const int64_t tiles = (N + 16 * p.rw - 1) / (16 * p.rw);
  const size_t xe = x_f32 ? 4 : 2, ye = y_f32 ? 4 : 2;
  if (p.ks > 1) {
    int rc = ensure_workspace(rt, rt->partials, (size_t)p.ks * mchunk * N * sizeof(float), false);
    if (rc) return rc;
  }
  // row stride of the activation source, in elements
  const int64_t xstride = pro->stride > 0 ? pro->stride : (pro->mode == 2 ? 2 * K : K);
  const size_t xe_src = (pro->mode == 1 || pro->mode == 3) ? 4 : (pro->mode == 2 ? 2 : xe);
  for (int64_t m0 = 0; m0 < M; m0 += mchunk) {
    const int64_t mm = M - m0 < mchunk ? M - m0 : mchunk;
    GemvArgs a;
    a.x = (const char *)x + m0 * xstride * xe_src;
    a.x_mode = pro->mode;
    a.x_stride = xstride;
    a.x_off = pro->off;
    a.norm_w = pro->norm_w;
    a.eps = pro->eps;
    a.ss_in = pro->ss_in;
    a.ss_parts = pro->ss_parts;
    a.ss_out = pro->ss_out;
    a.w = w;
    a.scale = scale;
    a.y = (char *)y + m0 * N * ye;
    a.ws = (float *)rt->partials.ptr;
    a.M = (int)mm;
    a.N = (int)N;
    a.K = (int)K;
    a.G = (int)G;
    a.ksplit = p.ks;
    a.x_f32 = x_f32;
    a.y_f32 = y_f32;
    a.y_mode = pro->swiglu ? 2 : y_mode;
    a.wave_stage = pro->mode == 0 && gemv_wave_stage(mm, K, G, p.rw, w_bf16);
    const int mb = mm <= 16 ? 1 : 2;
    // bf16 activation rows with per-channel u8 weights: the variant that reads
    // them as MFMA fragments from global memory (no LDS staging)
    // (XG kernels exist for every wide tiling but the 96-row one)
    const bool xg = xg_mode != 0 && pro->mode == 0 && !x_f32 && !w_bf16 && G == K && mb == 1 &&
                    (p.nw != 4 || p.rw == 1 || p.rw == 4) && p.rw != 6;
    const int u = xg && p.u > 4 ? 4 : p.u;
    char kname[64];
    char wide[12] = "";
    if (xg)
      std::snprintf(wide, sizeof wide, "_w%d_xg", p.nw);
    else if (p.nw != 4)
      std::snprintf(wide, sizeof wide, "_w%d", p.nw);
    std::snprintf(kname, sizeof kname, "rxw8_gemv_%s%s%s_mb%d_rw%d_u%d%s%s", ref_cast ? "rc_" : "",
                  w_bf16 ? "bf16" : "w8", packed ? "_pk" : "", mb, p.rw, u, wide,
                  pro->row_norm ? "_rn" : "");
    size_t lds = xg ? (size_t)(p.nw / p.rw - 1) * p.rw * mb * 256 * 4 + 16
                    : gemv_lds(mm, K / p.ks, K, G, p.rw, mb, w_bf16, p.nw);
    a.row_norm = pro->row_norm ? 1 : 0;
    a.rs_off = 0;
    if (pro->row_norm) {  // the row factors follow everything else in LDS
      lds = (lds + 15) / 16 * 16;
      a.rs_off = (int)lds;
      lds += 32 * sizeof(float);
    }
    a.xw_norm = pro->xw_norm;
    a.xw_out = pro->xw_out;
    a.ss_ld = (int)M;  // (ss modes run as one chunk of rows)
    a.chunk_rows = (int)mm;
    // bf16 rows whose split is whole 512-element runs, 16-byte aligned, are
    // staged by LDS DMA (B = 16, K = 4096: 8.9 -> 7.4 us for N = 4096).
    // RXW8_GEMV_LDS_DMA=0 turns it off.
    static const int dma_env = env_int("RXW8_GEMV_LDS_DMA", 1);
    a.lds_dma = dma_env && !xg && pro->mode == 0 && !x_f32 && !a.wave_stage &&
                (K / p.ks) % 512 == 0 && xstride % 8 == 0 && pro->off % 8 == 0 &&
                (uintptr_t)a.x % 16 == 0;
    int rc = launch(rt, kname, dim3((unsigned)(tiles * p.ks)), dim3(64 * p.nw), a, lds);
    if (rc) return rc;
    if (p.ks > 1) {
      SplitkReduceArgs r;
      r.ws = (const float *)rt->partials.ptr;
      // (the reference-cast partials already hold the dequantised products)
      r.scale = (!w_bf16 && G == K && !ref_cast) ? scale : nullptr;
      r.y = a.y;
      r.M = (int)mm;
      r.N = (int)N;
      r.ksplit = p.ks;
      r.y_f32 = y_f32;
      r.y_mode = y_mode;
      rc = launch(rt, "rxw8_gemv_splitk_reduce", dim3(grid_for(mm * N / 4, 256, 4096)),
                  dim3(256), r);
      if (rc) return rc;
    }
  }
  return RXW8_OK;
}

// F32-compute GEMV (the _fc kernels): f32 rows x (x_mode 0, or the RMSNorm
// prologues 1 / 3), packed u8 weights, f32 y (y_mode 0), f32 residual
// (y_mode 1, optional ss_out) or f32 SwiGLU activation (y_mode 2, interleaved
// gate|up tiles). Each f32 row is staged as two bf16 rows (hi, lo), so a
// workgroup takes up to 16 rows (2 x 16 staged rows), or 8 when 32 staged
// rows of K do not fit in LDS; longer inputs run as chunks of rows side by
// side in the same launch (the ss partials carry the whole product's row
// stride). UNIMPLEMENTED (nothing launched) when no single-launch plan fits.
static int run_gemv_fc(Runtime *rt, const float *x, const uint8_t *w, const float *scale, float *y,
                       int64_t M, int64_t N, int64_t K, int64_t G, int y_mode, const GemvOptions *pro) {
  GemvOptions plain;
  if (!pro) pro = &plain;
  if (M < 1 || N % 16 || K % 64 || (G != K && G % 64) || M > (1 << 30) || N > (1 << 30) ||
      pro->mode == 2 || pro->row_norm || pro->xw_out || (pro->swiglu && y_mode != 0) ||
      (pro->mode == 3 && !pro->ss_in))
    return RXW8_UNIMPLEMENTED;
  const bool allow_wide = pro->mode != 1;  // mode 1 sums rows with 256-thread reductions
  GemvPlan p;
  int rows = 0;  // staged rows per workgroup: 2 x 16 or 2 x 8
  // RXW8_GEMV_FC_ROWS=8 takes chunks of 8 rows also where 16 would fit
  static const int rows_env = env_int("RXW8_GEMV_FC_ROWS", 0);
  for (int r : {M > 8 && rows_env != 8 ? 32 : 16, 16}) {
    GemvPlan q = plan_gemv(rt, r, N, K, G, false, true, allow_wide);
    if (q.ks == 1 && q.lds + 256 <= rt->lds_max) {
      p = q;
      rows = r;
      break;
    }
  }
  if (!rows) return RXW8_UNIMPLEMENTED;
  const int64_t mchunk = rows / 2, mb = rows / 16;
  char kname[64], wide[8] = "";
  if (p.nw != 4) std::snprintf(wide, sizeof wide, "_w%d", p.nw);
  std::snprintf(kname, sizeof kname, "rxw8_gemv_w8_pk_mb%d_rw%d_u%d%s_fc", (int)mb, p.rw, p.u, wide);
  const int64_t xstride = pro->stride > 0 ? pro->stride : K;
  // Longer inputs: one launch whose grid holds a row of tiles per chunk of
  // rows (blockIdx.y), so the chunks run side by side (each workgroup re-reads
  // its weight tile, mostly from the caches; 2 x 8 rows of the Qwen3.5-0.8B
  // down projection, K = 3584: one launch of 8.96 us instead of two of 7.96)
  const int64_t chunks = (M + mchunk - 1) / mchunk;
  const int64_t tiles = (N + 16 * p.rw - 1) / (16 * p.rw);
  if (tiles * chunks >= ((int64_t)1 << 31) || chunks > 65535) return RXW8_UNIMPLEMENTED;
  // the staging reads x, the scales and the sum-of-squares partials through
  // raw buffer loads (32-bit byte offsets)
  constexpr int64_t kBufMax = (int64_t)1 << 31;
  if (((M - 1) * xstride + pro->off + K) * 4 >= kBufMax || N * (K / G) * 4 >= kBufMax ||
      (pro->mode == 3 && ((int64_t)pro->ss_parts * M) * 4 >= kBufMax))
    return RXW8_UNIMPLEMENTED;
  GemvArgs a{};
  a.x = x;
  a.w = w;
  a.scale = scale;
  a.y = y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = (int)G;
  a.ksplit = 1;
  a.x_f32 = 1;
  a.y_f32 = 1;
  a.y_mode = pro->swiglu ? 2 : y_mode;
  a.ss_out = pro->ss_out;
  a.x_mode = pro->mode;
  a.x_stride = xstride;
  a.x_off = pro->off;
  a.norm_w = pro->norm_w;
  a.eps = pro->eps;
  a.ss_in = pro->ss_in;
  a.ss_parts = pro->ss_parts;
  a.ss_ld = (int)M;
  a.chunk_rows = (int)mchunk;
  a.fc_kmajor = env_int("RXW8_GEMV_FC_KMAJOR", 1) != 0;
  const size_t lds = gemv_lds(rows, K, K, G, p.rw, (int)mb, false, p.nw);
  return launch(rt, kname, dim3((unsigned)tiles, (unsigned)chunks), dim3(64 * p.nw), a, lds);
}

bool gemv_single_launch(const Runtime *rt, int64_t M, int64_t N, int64_t K, int64_t G) {
  return M <= 32 && N % 16 == 0 && plan_gemv(rt, M, N, K, G, false, true).ks == 1;
}

int gemv_launch(Runtime *rt, const void *x, int x_f32, const void *w, bool w_bf16, bool packed,
                const float *scale, void *y, int y_f32, int64_t M, int64_t N, int64_t K, int64_t G,
                int y_mode, const GemvOptions &pro) {
  if (M == 0) return RXW8_OK;
  if (pro.f32c) {
    if (!x_f32 || !(y_f32 || y_mode == 1) || w_bf16 || !packed) return RXW8_UNIMPLEMENTED;
    return run_gemv_fc(rt, (const float *)x, (const uint8_t *)w, scale, (float *)y, M, N, K, G,
                       y_mode, &pro);
  }
  return run_gemv(rt, x, x_f32, w, w_bf16, packed, scale, y, y_f32, M, N, K, G, y_mode, &pro);
}

static int run_generic_linear(Runtime *rt, const void *x, int x_f32, const void *w, int w_kind,
                              const float *scale, void *y, int y_f32, int64_t M, int64_t N,
                              int64_t K, int64_t G, int compute_bf16, int y_mode = 0) {
  GenericLinearArgs a;
  a.x = x;
  a.w = w;
  a.scale = scale;
  a.y = y;
  a.m = M;
  a.n = N;
  a.k = K;
  a.g = G;
  a.x_f32 = x_f32;
  a.y_f32 = y_f32;
  a.compute_bf16 = compute_bf16;
  a.w_kind = w_kind;
  a.y_mode = y_mode;
  return launch(rt, "rxw8_linear_generic", dim3(grid_for(M * N)), dim3(256), a);
}

struct LinearF32GemmArgs {
  const uint16_t *xh, *xl;
  const uint8_t *w;
  const float *scale;
  float *y;
  int M, N, K, G;
  int y_mode, w_packed;
  int ksplit;
  float *ws;
};
struct F32ReduceArgs {
  const float *ws;
  float *y;
  int64_t mn;
  int ksplit, y_mode;
};
struct SplitXArgs {
  const float *x;
  uint16_t *hi, *lo;
  int64_t n;
};

// F32-compute W8 linear for long inputs on the GEMM tiles
// (rxw8_gemm_f32c): x split into bf16 hi / lo parts in the runtime's
// staging buffer, then 256 x 128 output tiles that read each weight tile
// once per 128 rows of x. Shapes with fewer tiles than half a round of CUs
// split K (at scale-group boundaries, at least 4 k tiles per split, up to 8
// splits) toward a round of work items, and a reduce launch adds the
// partials in split order. Taken from 17 rows on (RXW8_F32_GEMM=0 / 1
// forces it off / on where it applies; RXW8_F32_GEMM_KSPLIT=n forces n
// splits): even with mostly empty 128-row tiles and 32-64 work items it
// beats the row kernels, which read the weights once per 32 rows and cut K
// into LDS-sized launches (Qwen3.5-0.8B forward at 17 / 64 positions: 2.80
// / 3.39 ms against 3.95 / 4.61); up to 16 rows the F32 GEMV stays.
// UNIMPLEMENTED (nothing launched) when the shape or the 16-byte alignment
// of the weights and y does not fit its contract.
bool f32_gemm_applies(const void *w, const float *y, int64_t M, int64_t N, int64_t K, int64_t G) {
  const int env = env_int("RXW8_F32_GEMM", -1);
  return !(env == 0 || N % 16 || K % 64 || G % 64 || K % G || K / G > 32 || M * K * 2 >= (1LL << 31) ||
           N * K >= (1LL << 32) || ((uintptr_t)w | (uintptr_t)y) % 16 != 0 || (env < 0 && M <= 16));
}

// The operand buffers of the F32 GEMM's x parts: hi and lo, [M, K] bf16 each.
int f32_gemm_operands(Runtime *rt, int64_t M, int64_t K, uint16_t **hi, uint16_t **lo) {
  const int rc = ensure_workspace(rt, rt->xcast, (size_t)(M * K) * 4, false);
  if (rc) return rc;
  *hi = (uint16_t *)rt->xcast.ptr;
  *lo = *hi + M * K;
  return RXW8_OK;
}

// (x == nullptr: the caller has written x's parts into f32_gemm_operands'
// buffers, e.g. the Qwen3.5 RMSNorm; no split launch)
static int run_linear_f32_gemm(Runtime *rt, const float *x, const uint8_t *w, bool packed,
                               const float *scale, float *y, int64_t M, int64_t N, int64_t K,
                               int64_t G, int y_mode) {
  if (!f32_gemm_applies(w, y, M, N, K, G)) return RXW8_UNIMPLEMENTED;
  const int64_t tiles = (M + 127) / 128 * ((N + 255) / 256);
  // split units: scale groups, or the k tiles of a single group
  const int64_t ng = K / G, units = ng > 1 ? ng : K / 64, upt = ng > 1 ? G / 64 : 1;
  const int ks_env = env_int("RXW8_F32_GEMM_KSPLIT", 0);
  int64_t ks = 1;
  if (ks_env > 0) {
    ks = std::min<int64_t>(ks_env, units);
  } else if (2 * tiles < rt->cus) {
    for (int c : {2, 3, 4, 6, 8}) {
      if (units / c * upt < 4) break;
      ks = c;
      if (tiles * c >= rt->cus) break;
    }
  }
  uint16_t *xh, *xl;
  int rc = f32_gemm_operands(rt, M, K, &xh, &xl);
  if (rc) return rc;
  if (ks > 1 && (rc = ensure_workspace(rt, rt->partials, (size_t)(ks * M * N) * 4, false))) return rc;
  SplitXArgs sx{x, xh, xl, M * K};
  if (x && (rc = launch(rt, "rxw8_gemm_split_x", dim3(grid_for(M * K / 4, 256, 4096)), dim3(256), sx)))
    return rc;
  LinearF32GemmArgs a{xh, xl, w, scale, y, (int)M, (int)N, (int)K, (int)G, y_mode, packed ? 1 : 0,
                      (int)ks, ks > 1 ? (float *)rt->partials.ptr : nullptr};
  if ((rc = launch(rt, "rxw8_gemm_f32c", dim3((unsigned)((tiles * ks + 7) / 8 * 8)), dim3(512), a)))
    return rc;
  if (ks == 1) return RXW8_OK;
  F32ReduceArgs r{(const float *)rt->partials.ptr, y, M * N, (int)ks, y_mode};
  return launch(rt, "rxw8_gemm_f32c_reduce", dim3(grid_for(M * N / 4, 256, 4096)), dim3(256), r);
}

// The F32 GEMM on operands already split into f32_gemm_operands' buffers
// (f32_gemm_applies must hold).
int f32_gemm_presplit(Runtime *rt, const uint8_t *w, bool packed, const float *scale, float *y,
                      int64_t M, int64_t N, int64_t K, int64_t G, int y_mode) {
  return run_linear_f32_gemm(rt, nullptr, w, packed, scale, y, M, N, K, G, y_mode);
}

// QuantizedLinear with compute dtype F32 on the matrix cores (x split into
// bf16 hi + lo parts, exact codes, f32 accumulation): f32 x, row-major or
// packed (N % 16 == 0) U8 weights, K and G multiples of 64, 16-byte aligned
// operands and the staged rows of x within the LDS limit. Returns
// UNIMPLEMENTED otherwise.
static int run_linear_f32(Runtime *rt, const float *x, const uint8_t *w, bool packed,
                          const float *scale, float *y, int64_t M, int64_t N, int64_t K, int64_t G,
                          int y_mode) {
  {
    const int rc = run_linear_f32_gemm(rt, x, w, packed, scale, y, M, N, K, G, y_mode);
    if (rc != RXW8_UNIMPLEMENTED) return rc;
  }
  if (K % 64 != 0 || G % 64 != 0 || K > (1 << 24) || N > (1LL << 30) || M > (1LL << 30) ||
      ((uintptr_t)x | (uintptr_t)w) % 16 != 0 || (packed && N % 16) || env_int("RXW8_FORCE_GENERIC", 0))
    return RXW8_UNIMPLEMENTED;
  constexpr int WV = 8;
  // x (hi and lo) of the workgroup's rows is staged in LDS for its K range:
  // a K too wide for LDS runs as several launches over K ranges, each
  // accumulating into y (the first one stores when y_mode is 0). Ranges hold
  // whole scale groups, or, when one group is too wide, equal parts of every
  // group (each part then scales its own partial sum). The group sums are
  // reassociated across ranges: f32 rounding only.
  auto lds_for = [&](int R, int64_t kc, int64_t g) {
    return (size_t)2 * 16 * R * (kc + 8) * 2 + (size_t)16 * WV * (kc / g) * 4;
  };
  for (int R : {M > 16 ? 2 : 1, 1}) {
    int64_t kc_max = 0, gk = G;
    if (lds_for(R, K, G) <= rt->lds_max) {
      kc_max = K;
    } else if (lds_for(R, G, G) <= rt->lds_max) {
      int64_t fit = G;
      while (fit + G <= K && lds_for(R, fit + G, G) <= rt->lds_max) fit += G;
      const int64_t chunks = (K + fit - 1) / fit;
      kc_max = (K / G + chunks - 1) / chunks * G;
    } else {
      for (int64_t d = G; d >= 64; d -= 64)
        if (G % d == 0 && lds_for(R, d, d) <= rt->lds_max) {
          kc_max = gk = d;
          break;
        }
    }
    if (kc_max == 0) continue;
    const int64_t gy = (M + 16 * R - 1) / (16 * R);
    if (gy > 65535) return RXW8_UNIMPLEMENTED;
    // several channel tiles per workgroup, so the staged rows of x are
    // reused: just enough that the workgroups fit one round at the LDS-bound
    // residency (the Qwen3.5 head at 16 rows: 4 tiles each, 485 workgroups,
    // 69.7 -> 64.2 us packed, 82.7 -> 71.1 us row-major; 3 tiles each spill
    // into a second round: 70.9 us)
    const int64_t ntiles = (N + 16 * WV - 1) / (16 * WV);
    const int64_t resident = std::max<int64_t>(1, (int64_t)rt->lds_max / (int64_t)lds_for(R, kc_max, gk)) * rt->cus;
    const int64_t per = std::max<int64_t>(1, std::min<int64_t>(16, (ntiles * gy + resident - 1) / resident));
    char kname[40];
    std::snprintf(kname, sizeof kname, "rxw8_linear_f32_mfma%s_r%d_w%d", packed ? "_pk" : "", R, WV);
    for (int64_t k0 = 0; k0 < K; k0 += kc_max) {
      const int64_t kc = std::min(kc_max, K - k0);
      // packed: the K range starts at tile column k0 / 64 of row group 0, and
      // a row group holds K / 64 tiles
      LinearF32Args a{x + k0, packed ? w + k0 / 64 * 1024 : w + k0, scale + k0 / G, y, (int)M, (int)N,
                      (int)kc, (int)gk, k0 == 0 ? y_mode : 1, (int)per, K, packed ? K / 64 : K, K / G};
      int rc = launch(rt, kname, dim3((unsigned)((ntiles + per - 1) / per), (unsigned)gy),
                      dim3(64 * WV), a, lds_for(R, kc, gk));
      if (rc) return rc;
    }
    return RXW8_OK;
  }
  return RXW8_UNIMPLEMENTED;
}

// Shared validation of QuantizedLinear operands; fills M, N, K, G.
static int check_qlinear(const Buffer *x, const Buffer *w, const Buffer *s, int compute,
                         int64_t *M, int64_t *N, int64_t *K, int64_t *G) {
  if (!x || !w || !s) return fail(RXW8_INVALID_ARGUMENT, "QuantizedLinear: NULL buffer");
  if (x->rt != w->rt || x->rt != s->rt)
    return fail(RXW8_INVALID_ARGUMENT, "QuantizedLinear: buffers belong to different runtimes");
  if (compute != RXW8_BF16 && compute != RXW8_F32)
    return fail(RXW8_INVALID_ARGUMENT, "QuantizedLinear: compute dtype must be BF16 or F32");
  if (x->rank < 1 || !is_f(x->dtype))
    return fail(RXW8_INVALID_ARGUMENT,
                "QuantizedLinear requires an F32 (or bf16-valued BF16) input with rank at least one");
  if (compute == RXW8_F32 && x->dtype != RXW8_F32)
    return fail(RXW8_INVALID_ARGUMENT, "QuantizedLinear: F32 compute requires an F32 input");
  const bool packed = w->rank == 3;
  if (w->dtype != RXW8_U8 || (w->rank != 2 && !(packed && w->dims[2] == 1024)))
    return fail(RXW8_INVALID_ARGUMENT,
                "QuantizedLinear weight: dtype does not match the schema (U8 [out, in], or packed "
                "U8 [out/16, in/64, 1024])");
  if (s->dtype != RXW8_F32 || s->rank != 2)
    return fail(RXW8_INVALID_ARGUMENT, "QuantizedLinear scale: dtype does not match the schema (F32 [out, groups])");
  *K = x->dims[x->rank - 1];
  *N = packed ? w->dims[0] * 16 : w->dims[0];
  const int64_t groups = s->dims[1];
  if (*N <= 0 || *K <= 0 || groups <= 0 || *K % groups != 0)
    return fail(RXW8_INVALID_ARGUMENT,
                "QuantizedLinear requires positive widths and a group size dividing the input width");
  if ((packed ? w->dims[1] * 64 : w->dims[1]) != *K)
    return fail(RXW8_INVALID_ARGUMENT, "QuantizedLinear weight %s: shape does not match input width %lld",
                dims_str(w).c_str(), (long long)*K);
  if (s->dims[0] != *N)
    return fail(RXW8_INVALID_ARGUMENT, "QuantizedLinear scale %s: shape does not match weight %s",
                dims_str(s).c_str(), dims_str(w).c_str());
  *G = *K / groups;
  *M = 1;
  for (int i = 0; i < x->rank - 1; ++i) *M *= x->dims[i];
  return RXW8_OK;
}

int qlinear_launch(Runtime *rt, const void *x, int x_f32, const uint8_t *w, bool packed,
                   const float *s, void *y, int y_f32, int64_t M, int64_t N, int64_t K,
                   int64_t G, int compute_bf16, int y_mode = 0);

}  // namespace rxw8

using namespace rxw8;

namespace rxw8 {

// Prefill-sized products go to the MFMA GEMM (128 x 128 output tiles; the
// weight tile is dequantised once per 128 activation rows); smaller M stays on
// the GEMV, which streams the weights once per 16/32-row chunk.
bool gemm_eligible(int64_t M, int64_t N, int64_t K, int64_t G) {
  static const int64_t min_m = env_int("RXW8_GEMM_MIN_M", 64);
  // 32-bit byte offsets inside the kernel: activations M*K*2, weights N*K
  return M > min_m && N % 128 == 0 && K % 64 == 0 && G % 64 == 0 && M * K * 2 < (1LL << 31) &&
         N * K < (1LL << 32) && !env_int("RXW8_NO_GEMM", 0);
}

// Requires gemm_eligible(): one scale per weight row and 64-deep k tile.
static int run_gemm(Runtime *rt, const void *x, int x_f32, const uint8_t *w, bool packed,
                    const float *s, void *y, int y_f32, int64_t M, int64_t N, int64_t K,
                    int64_t G, int y_mode) {
  int rc;
  if (x_f32) {  // x.cast(BF16) into the runtime's staging buffer, then the bf16 GEMM
    if ((rc = ensure_workspace(rt, rt->xcast, (size_t)(M * K) * 2, false))) return rc;
    CastArgs c{(const float *)x, (uint16_t *)rt->xcast.ptr, M * K};
    if ((rc = launch(rt, "rxw8_gemm_cast_x", dim3(grid_for(M * K / 4 + 1, 256, 4096)), dim3(256), c)))
      return rc;
    x = rt->xcast.ptr;
  }
  GemmArgs a;
  a.x = (const uint16_t *)x;
  a.w = w;
  a.scale = s;
  a.y = y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = (int)G;
  a.y_f32 = y_f32;
  a.y_mode = y_mode;
  a.w_packed = packed ? 1 : 0;
  a.group_n = env_int("RXW8_GEMM_GN", 0);
  a.ksplit = 1;
  a.ws = nullptr;
  // Three tilings (one workgroup per CU each): 256 x 256 (8 waves), 256 x 128
  // and 128 x 128 (4 waves); the 256 x 256 one may also split K (f32 partials
  // summed in split order by a second launch). Pick the least modelled time:
  // whole rounds of workgroups x one tile's MFMA time at the tiling's measured
  // efficiency, plus the partials' HBM round trip for splits.
  struct Tiling {
    const char *kernel;
    int tm, tn, threads;
    double eff;
  };
  // 256 x 192 (the 8-wave kernel with 6 weight fragments per wave) fills
  // whole rounds where 256-wide tiles leave half a round, e.g. M = 2048,
  // N = 12288: 512 tiles instead of 384.
  static const Tiling tilings[] = {{"rxw8_w8a16_gemm_t256", 256, 256, 512, 0.50},
                                   {"rxw8_w8a16_gemm_t192", 256, 192, 512, 0.44},
                                   {"rxw8_w8a16_gemm_m256", 256, 128, 256, 0.36},
                                   {"rxw8_w8a16_gemm_m128", 128, 128, 256, 0.30}};
  // RXW8_GEMM_TILE: 256x256 = 256, 256x192 = 192, 256x128 = 2, 128x128 = 128
  const int forced = env_int("RXW8_GEMM_TILE", 0);
  const int forced_ks = env_int("RXW8_GEMM_KSPLIT", 0);
  const double cu_flops = 2.5e15 / 256.0, hbm = 4.0e12;  // per-CU bf16 MFMA peak, B/s
  const Tiling *best = nullptr;
  int best_ks = 1;
  double best_t = 1e30;
  for (const Tiling &tl : tilings) {
    if (N % tl.tn) continue;
    const int code = tl.tn == 256 || tl.tn == 192 ? tl.tn : (tl.tm == 256 ? 2 : 128);
    if (forced && forced != code) continue;
    const int64_t tiles = (M + tl.tm - 1) / tl.tm * (N / tl.tn);
    for (int ks : {1, 2, 3, 4, 6, 8}) {
      if (ks > 1 && (tl.tn != 256 || ks > K / 64 || y_mode == 2)) continue;
      if (forced_ks && forced_ks != ks && (tl.tn != 256 || forced_ks <= K / 64 || ks > 1)) continue;
      const int64_t rounds = (tiles * ks + rt->cus - 1) / rt->cus;
      double t = (double)rounds * tl.tm * tl.tn * (double)K / ks * 2.0 / (cu_flops * tl.eff);
      if (ks > 1) t += (ks + 1.0) * (double)M * N * 4.0 / hbm + 3e-6;
      if (t < best_t) best_t = t, best = &tl, best_ks = ks;
    }
  }
  if (!best) return fail(RXW8_INVALID_ARGUMENT, "no GEMM tiling for N=%lld", (long long)N);
  const int64_t tiles = (M + best->tm - 1) / best->tm * (N / best->tn);
  const int64_t per_xcd = (tiles + 7) / 8;
  // Long inputs: dequantise the weights once into a bf16 workspace (a
  // bandwidth-bound pass of N K (1 + 2) bytes) and run the 256 x 256 tiles on
  // bf16 x bf16, both operands DMA'd into LDS: the k loop then carries no
  // dequantisation, which costs more than the pass once M reaches a few
  // thousand rows. Same weight values bit for bit.
  const int bf16w_env = env_int("RXW8_GEMM_BF16W", -1);
  const bool bf16w = best->tn == 256 && best_ks == 1 && N * K * 2 < (1LL << 31) &&
                     (bf16w_env == 1 || (bf16w_env < 0 && M >= 4096));
  if (bf16w) {
    if ((rc = ensure_workspace(rt, rt->wdeq, (size_t)(N * K) * 2, false))) return rc;
    DequantWArgs d{w, s, (uint16_t *)rt->wdeq.ptr, (int)N, (int)K, (int)G, packed ? 1 : 0};
    const int64_t slices = N * (K / 16);
    if ((rc = launch(rt, "rxw8_gemm_dequant_w", dim3((unsigned)((slices + 255) / 256)), dim3(256), d)))
      return rc;
    a.w = (const uint8_t *)rt->wdeq.ptr;
    a.w_packed = 0;
    return launch(rt, "rxw8_w8a16_gemm_bf16w_t256", dim3((unsigned)(per_xcd * 8)), dim3(512), a);
  }
  if (best_ks > 1) {
    if ((rc = ensure_workspace(rt, rt->partials, (size_t)best_ks * M * N * 4, false))) return rc;
    a.ksplit = best_ks;
    a.ws = (float *)rt->partials.ptr;
    const int64_t work = (tiles * best_ks + 7) / 8 * 8;
    if ((rc = launch(rt, best->kernel, dim3((unsigned)work), dim3(best->threads), a))) return rc;
    SplitkReduceArgs r;
    r.ws = (const float *)rt->partials.ptr;
    r.scale = nullptr;
    r.y = y;
    r.M = (int)M;
    r.N = (int)N;
    r.ksplit = best_ks;
    r.y_f32 = y_f32;
    r.y_mode = y_mode;
    return launch(rt, "rxw8_gemv_splitk_reduce", dim3(grid_for(M * N / 4, 256, 4096)), dim3(256), r);
  }
  return launch(rt, best->kernel, dim3((unsigned)(per_xcd * 8)), dim3(best->threads), a);
}

int qlinear_launch(Runtime *rt, const void *x, int x_f32, const uint8_t *w, bool packed,
                   const float *s, void *y, int y_f32, int64_t M, int64_t N, int64_t K,
                   int64_t G, int compute_bf16, int y_mode) {
  if (M == 0) return RXW8_OK;
  if (y_mode == 1) y_f32 = 1;  // the residual y is f32 (row offsets of M chunks use it)
  if (packed) {
    if (compute_bf16 && gemm_eligible(M, N, K, G))
      return run_gemm(rt, x, x_f32, w, true, s, y, y_f32, M, N, K, G, y_mode);
    // F32 compute on packed weights: the GEMM tiles for long inputs, else the
    // _fc GEMV in chunks of rows
    if (!compute_bf16 && x_f32 && y_f32) {
      const int rc = run_linear_f32_gemm(rt, (const float *)x, w, true, s, (float *)y, M, N, K, G, y_mode);
      if (rc != RXW8_UNIMPLEMENTED) return rc;
      // many channel tiles (an LM head): the row kernel that stages x once
      // per workgroup for several 128-channel tiles
      if (N / 128 >= 4 * (int64_t)rt->cus) {
        const int rl = run_linear_f32(rt, (const float *)x, w, true, s, (float *)y, M, N, K, G, y_mode);
        if (rl != RXW8_UNIMPLEMENTED) return rl;
      }
    }
    int rc = compute_bf16 ? run_gemv(rt, x, x_f32, w, false, true, s, y, y_f32, M, N, K, G, y_mode)
             : x_f32 && y_f32
                 ? run_gemv_fc(rt, (const float *)x, w, s, (float *)y, M, N, K, G, y_mode, nullptr)
                 : (int)RXW8_UNIMPLEMENTED;
    if (rc == RXW8_UNIMPLEMENTED)
      return fail(RXW8_UNIMPLEMENTED,
                  "packed W8 weights need a GEMV tiling for N=%lld K=%lld G=%lld (F32 compute: "
                  "N %% 16 == 0)",
                  (long long)N, (long long)K, (long long)G);
    return rc;
  }
  if (!compute_bf16 && x_f32 && y_f32) {
    int rc = run_linear_f32(rt, (const float *)x, w, false, s, (float *)y, M, N, K, G, y_mode);
    if (rc != RXW8_UNIMPLEMENTED) return rc;
  }
  const bool mfma_ok = compute_bf16 && K % 64 == 0 && N % 16 == 0 && (G == K || G % 64 == 0) &&
                       K <= (1LL << 30) && N <= (1LL << 30) && !env_int("RXW8_FORCE_GENERIC", 0);
  if (mfma_ok) {
    if (gemm_eligible(M, N, K, G)) return run_gemm(rt, x, x_f32, w, false, s, y, y_f32, M, N, K, G, y_mode);
    int rc = run_gemv(rt, x, x_f32, w, false, false, s, y, y_f32, M, N, K, G, y_mode);
    if (rc != RXW8_UNIMPLEMENTED) return rc;
  }
  return run_generic_linear(rt, x, x_f32, w, 0, s, y, y_f32, M, N, K, G, compute_bf16, y_mode);
}

int bf16_linear_launch(Runtime *rt, const void *x, int x_f32, const uint16_t *w, bool packed,
                       void *y, int y_f32, int64_t M, int64_t N, int64_t K) {
  if (M == 0) return RXW8_OK;
  if (packed) {
    int rc = run_gemv(rt, x, x_f32, w, true, true, nullptr, y, y_f32, M, N, K, K);
    if (rc == RXW8_UNIMPLEMENTED)
      return fail(RXW8_UNIMPLEMENTED, "packed BF16 weights need a GEMV tiling for N=%lld K=%lld",
                  (long long)N, (long long)K);
    return rc;
  }
  if (K % 32 == 0 && N % 16 == 0 && !env_int("RXW8_FORCE_GENERIC", 0)) {
    int rc = run_gemv(rt, x, x_f32, w, true, false, nullptr, y, y_f32, M, N, K, K);
    if (rc != RXW8_UNIMPLEMENTED) return rc;
  }
  return run_generic_linear(rt, x, x_f32, w, 1, nullptr, y, y_f32, M, N, K, K, 1);
}

int attention_launch(Runtime *rt, const void *q, int q_f32, const void *kc, const void *vc,
                     int cache_f32, const int32_t *lens, const int32_t *row_seq,
                     const float *mask, int64_t mask_sb, int64_t mask_sh, void *out, int out_f32,
                     int64_t R, int64_t Hq, int64_t Hkv, int64_t Lmax, int64_t D, float scale,
                     const AttnRope *rope, const AttnWorkspace *ext) {
  if (R == 0) return RXW8_OK;
  const int64_t G = Hq / Hkv;
  const bool fast = !cache_f32 && D == 128 && (G == 1 || G == 2 || G == 4 || G == 8) &&
                    !env_int("RXW8_FORCE_GENERIC", 0);
  if (rope && !fast) return fail(RXW8_INTERNAL, "fused RoPE attention needs the D = 128 kernel");
  if (fast) {
    // 8 waves walk a split of a row's keys in 16-key tiles with an online
    // softmax; one such workgroup fills a CU (VGPR-bound). S splits per (row,
    // kv head) minimise rounds x (fixed cost + keys per split), with the fixed
    // cost (launch, q set-up, wave merge, partial store) worth ~125 keys and
    // Lmax standing in for the row lengths: whole rounds of workgroups win
    // over a partial last round (64 pairs: S = 4 beats 6). S = 1 (no combine
    // launch) once the rows alone fill the GPU (prefill). The combine keeps at
    // most 64 partials, and every split holds at least 64 keys.
    const int forced = env_int("RXW8_ATTN_SPLITS", 0);
    const int64_t pairs = R * Hkv;
    const int64_t smax = std::max<int64_t>(1, std::min<int64_t>(64, (Lmax + 63) / 64));
    int64_t S = 1;
    double best = 0.0;
    // At most 4 x cus split workgroups (partial slots): beyond that the
    // estimate is flat (rounds x keys per split stays ~pairs x Lmax / cus),
    // and the bound keeps every plan's partials within cus x 4 x G (2 + D)
    // floats (4.1 MiB at G = 8 on 256 CUs).
    for (int64_t s = 1; s <= smax && (s == 1 || pairs * s <= 4 * (int64_t)rt->cus); ++s) {
      const double rounds = (double)((pairs * s + rt->cus - 1) / rt->cus);
      const double est = rounds * (125.0 + (double)Lmax / (double)s);
      if (s == 1 || est < best) {
        best = est;
        S = s;
      }
    }
    if (forced > 0) S = forced;
    if (S > 64) S = 64;
    if (pairs >= 2 * rt->cus && !forced) S = 1;
    // Ragged rows: when splitting pays (S > 1), the rows fit one round and the
    // cache is long (Lmax >= 2048: for short rows the apportioning pass costs
    // more than the imbalance it removes), the kernel gives each row a share
    // of cus / Hkv workgroups per kv head in proportion to its length
    // (device-side, from lens), so no workgroup walks far more keys than the
    // rest. RXW8_ATTN_SPLITS or RXW8_ATTN_UNIFORM=1 force uniform splits.
    int64_t units = 0;
    if (S > 1 && !forced && !env_int("RXW8_ATTN_UNIFORM", 0) && rt->cus / Hkv > R &&
        Lmax >= 2048 && R * Lmax < (int64_t)1 << 30)
      units = std::min<int64_t>(rt->cus / Hkv, R + 63);
    if (units > 0) S = units - R + 1;  // the most splits a row can get (> 1: a split plan)
    const int64_t max_chunks = S;
    // Splits are merged by the last workgroup of each (row, kv head) to finish
    // (arrival counters, zeroed once at allocation and re-armed by the kernel);
    // RXW8_ATTN_TWO_PASS=1 uses the separate combine launch instead.
    const bool two_pass = env_int("RXW8_ATTN_TWO_PASS", 0) != 0;
    float *ws_partials = nullptr;
    int *ws_counters = nullptr;
    if (max_chunks > 1) {
      // one partial slot per workgroup: Hkv x units (length-proportional) or
      // R x Hkv x S (uniform splits)
      const size_t slots = units > 0 ? (size_t)Hkv * units : (size_t)R * Hkv * max_chunks;
      const size_t need_p = slots * G * (2 + D) * sizeof(float);
      const size_t need_c = two_pass ? 0 : (size_t)R * Hkv * sizeof(int);
      if (ext) {
        if (need_p > ext->partial_bytes || need_c > ext->counter_bytes)
          return fail(RXW8_RESOURCE_EXHAUSTED,
                      "decode attention (B=%lld Hkv=%lld Lmax=%lld, %lld splits) needs %zu bytes of "
                      "split partials and %zu of counters; the caller's workspace holds %zu and %zu",
                      (long long)R, (long long)Hkv, (long long)Lmax, (long long)max_chunks, need_p,
                      need_c, ext->partial_bytes, ext->counter_bytes);
        ws_partials = ext->partials;
        ws_counters = ext->counters;
      } else {
        int rc = ensure_workspace(rt, rt->scratch, need_p, false);
        if (rc) return rc;
        if (need_c && (rc = ensure_workspace(rt, rt->attn_counters, need_c, true))) return rc;
        ws_partials = (float *)rt->scratch.ptr;
        ws_counters = (int *)rt->attn_counters.ptr;
      }
    }
    AttnArgs a;
    a.q = q;
    a.kc = (const uint16_t *)kc;
    a.vc = (const uint16_t *)vc;
    a.lens = lens;
    a.row_seq = row_seq;
    a.mask = mask;
    a.out = out;
    a.ws = ws_partials;
    a.mask_sb = mask_sb;
    a.mask_sh = mask_sh;
    a.R = (int)R;
    a.Hq = (int)Hq;
    a.Hkv = (int)Hkv;
    a.Lmax = (int)Lmax;
    a.max_chunks = (int)max_chunks;
    a.scale = scale;
    a.q_f32 = q_f32;
    a.out_f32 = out_f32;
    a.qkv = rope ? rope->qkv : nullptr;
    a.q_norm = rope ? rope->q_norm : nullptr;
    a.k_norm = rope ? rope->k_norm : nullptr;
    a.rope = rope ? rope->table : nullptr;
    a.eps = rope ? rope->eps : 0.f;
    a.counters = max_chunks > 1 && !two_pass ? ws_counters : nullptr;
    a.units = (int)units;
    char kname[64];
    // G = 8 runs 4-wave workgroups (no register spills); the others 8 waves
    const unsigned threads = G == 8 ? 256 : 512;
    std::snprintf(kname, sizeof kname, rope ? "rxw8_gqa_decode_rope_d128_g%d" : "rxw8_gqa_decode_d128_g%d",
                  (int)G);
    const int64_t grid = units > 0 ? Hkv * units : R * Hkv * max_chunks;
    int rc = launch(rt, kname, dim3((unsigned)grid), dim3(threads), a);
    if (rc || max_chunks == 1 || a.counters) return rc;
    std::snprintf(kname, sizeof kname, "rxw8_gqa_decode_combine_d128_g%d", (int)G);
    return launch(rt, kname, dim3((unsigned)(R * Hkv)), dim3(256), a);
  }
  if (Lmax > 8192)
    return fail(RXW8_UNIMPLEMENTED, "decode attention: the generic kernel supports Lmax <= 8192");
  AttnGenericArgs a;
  a.q = q;
  a.kc = kc;
  a.vc = vc;
  a.lens = lens;
  a.row_seq = row_seq;
  a.mask = mask;
  a.out = out;
  a.mask_sb = mask_sb;
  a.mask_sh = mask_sh;
  a.B = (int)R;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.Lmax = (int)Lmax;
  a.D = (int)D;
  a.scale = scale;
  a.q_f32 = q_f32;
  a.cache_f32 = cache_f32;
  a.out_f32 = out_f32;
  return launch(rt, "rxw8_gqa_decode_generic", dim3((unsigned)(R * Hq)), dim3(256), a);
}

// Causal prefill attention: q / out element (b, i, h, d) at b*sb + i*ss + h*sh
// + d; row i of sequence b at position starts[b] + i (clamped on the device
// into [0, Lmax - S]). D = 128, bf16 caches, Hq / Hkv in {1, 2, 4}.
bool prefill_supported(int64_t Hq, int64_t Hkv, int64_t D, int cache_f32) {
  const int64_t G = Hkv > 0 ? Hq / Hkv : 0;
  return !cache_f32 && D == 128 && Hkv > 0 && Hq % Hkv == 0 && (G == 1 || G == 2 || G == 4 || G == 8);
}

// Causal prefill on the general GQA kernel: q / out element (b, i, h, d) at
// b*sb + i*ss + h*sh + d, bf16 cache [B, Hkv, Lmax, D], row i of sequence b
// seeing keys 0 .. clamp(starts[b], 0, Lmax - S) + i. Any head dim up to 512
// and any group size.
static int prefill_general(Runtime *rt, const void *q, int q_bf16, int64_t q_sb, int64_t q_ss,
                           int64_t q_sh, const uint16_t *kc, const uint16_t *vc,
                           const int32_t *starts, void *out, int out_bf16, int64_t o_sb,
                           int64_t o_ss, int64_t o_sh, int64_t B, int64_t S, int64_t Hq,
                           int64_t Hkv, int64_t Lmax, int64_t D, float scale) {
  if (D > 512) return fail(RXW8_UNIMPLEMENTED, "prefill attention: head dim %lld > 512", (long long)D);
  GqaGeneralArgs a{};
  a.q = q, a.k = kc, a.v = vc, a.out = out;
  for (int t = 0; t < 4; ++t) a.bdim[t] = 1, a.mb[t] = 0;
  a.bdim[3] = B;
  a.rows = B * Hq * S;
  a.Hq = (int)Hq, a.Hkv = (int)Hkv, a.Sq = (int)S, a.Sk = (int)Lmax, a.D = (int)D, a.Dv = (int)D;
  a.scale = scale;
  a.q_sb = q_sb, a.q_sh = q_sh, a.q_si = q_ss;
  a.o_sb = o_sb, a.o_sh = o_sh, a.o_si = o_ss;
  a.k_sb = a.v_sb = Hkv * Lmax * D;
  a.k_sh = a.v_sh = Lmax * D;
  a.q_bf16 = q_bf16, a.kv_bf16 = 1, a.out_bf16 = out_bf16;
  a.starts = starts;
  if ((a.rows + 3) / 4 >= ((int64_t)1 << 31))
    return fail(RXW8_UNIMPLEMENTED, "prefill attention: %lld rows exceed the grid", (long long)a.rows);
  return launch(rt, "rxw8_gqa_general", dim3((unsigned)((a.rows + 3) / 4)), dim3(256), a);
}

int prefill_launch(Runtime *rt, const void *q, int q_f32, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                   const uint16_t *kc, const uint16_t *vc, const int32_t *starts,
                   const int32_t *slots, void *out, int out_f32, int64_t o_sb, int64_t o_ss,
                   int64_t o_sh, int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t Lmax,
                   float scale) {
  if (B == 0 || S == 0) return RXW8_OK;
  if (S > Lmax) return fail(RXW8_INVALID_ARGUMENT, "prefill attention: S %lld > Lmax %lld",
                            (long long)S, (long long)Lmax);
  if (!prefill_supported(Hq, Hkv, 128, 0)) {
    // other group sizes: the general GQA kernel with the same causal-from-
    // starts rule (one wave per query row; D = 128 here)
    if (slots || Hkv <= 0 || Hq % Hkv)
      return fail(RXW8_UNIMPLEMENTED, "prefill attention: no kernel for Hq=%lld Hkv=%lld",
                  (long long)Hq, (long long)Hkv);
    return prefill_general(rt, q, !q_f32, q_sb, q_ss, q_sh, kc, vc, starts, out, !out_f32, o_sb,
                           o_ss, o_sh, B, S, Hq, Hkv, Lmax, 128, scale);
  }
  PrefillArgs a;
  a.q = q;
  a.kc = kc;
  a.vc = vc;
  a.starts = starts;
  a.slots = slots;
  a.out = out;
  a.q_sb = q_sb, a.q_ss = q_ss, a.q_sh = q_sh;
  a.o_sb = o_sb, a.o_ss = o_ss, a.o_sh = o_sh;
  a.B = (int)B;
  a.S = (int)S;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.Lmax = (int)Lmax;
  a.nqb = (int)((S + 63) / 64);
  a.scale = scale;
  a.q_f32 = q_f32;
  a.out_f32 = out_f32;
  char kname[48];
  const int G = (int)(Hq / Hkv);
  // The two-tile kernel: one query head per wave, min(G, 2) heads per
  // workgroup (4 waves each; G = 4 takes two workgroups per kv head), two
  // 16-row tiles per wave (128 query rows per workgroup), K and V by LDS
  // DMA: at the C5 prompt shape 72.8 us against 94.3 (one tile) and 120.5
  // (all heads per wave, one wave per SIMD). RXW8_PREFILL_R2=0 selects the
  // one-tile kernel for G <= 2 and the all-heads one for G = 4;
  // RXW8_PREFILL_R2=0 RXW8_PREFILL_WH=0 the all-heads one for every G.
  static const int wh_env = env_int("RXW8_PREFILL_WH", 1);
  static const int r2_env = env_int("RXW8_PREFILL_R2", 1);
  // (the two-tile kernel addresses a cache plane with 32-bit byte offsets)
  const bool r2 = r2_env && (G <= 4 || G == 8) && Lmax <= ((int64_t)1 << 22);
  const bool wh = wh_env && G <= 2;
  if (G == 8 && !r2) {  // no all-heads kernel for 8 heads: the general GQA kernel
    if (slots)
      return fail(RXW8_UNIMPLEMENTED, "prefill attention: 8 heads per kv head with cache slots "
                                      "needs the two-tile kernel (Lmax <= 2^22)");
    return prefill_general(rt, q, !q_f32, q_sb, q_ss, q_sh, kc, vc, starts, out, !out_f32, o_sb,
                           o_ss, o_sh, B, S, Hq, Hkv, Lmax, 128, scale);
  }
  if (r2) a.nqb = (int)((S + 127) / 128);
  std::snprintf(kname, sizeof kname,
                r2 ? "rxw8_gqa_prefill_r2_d128_g%d"
                   : (wh ? "rxw8_gqa_prefill_wh_d128_g%d" : "rxw8_gqa_prefill_d128_g%d"),
                G);
  // K and V^T blocks of 64 keys, double-buffered (2 x (64*128 + 128*72) bf16)
  constexpr size_t lds = 2 * (64 * 128 + 128 * 72) * 2;
  // the two-tile kernel: min(G, 2) heads per workgroup, G / min(G, 2) workgroups per kv head
  const int hw = G < 2 ? G : 2;
  if (r2)
    return launch(rt, kname, dim3((unsigned)(a.nqb * B * Hkv * (G / hw))), dim3(256 * hw), a, lds);
  return launch(rt, kname, dim3((unsigned)(a.nqb * B * Hkv)), dim3(wh ? 256 * G : 256), a, lds);
}


}  // namespace rxw8

extern "C" {

int rxw8_dequantize(rxw8_runtime *rt, rxw8_buffer *weight, rxw8_buffer *scale, int out_dtype,
                    rxw8_buffer **out) {
  if (!rt || !weight || !scale || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (weight->dtype != RXW8_U8 || weight->rank != 2)
    return fail(RXW8_INVALID_ARGUMENT, "dequantize: weight must be U8 [out, in]");
  if (scale->dtype != RXW8_F32 || scale->rank != 2 || scale->dims[0] != weight->dims[0])
    return fail(RXW8_INVALID_ARGUMENT, "dequantize: scale must be F32 [out, groups]");
  if (out_dtype != RXW8_F32 && out_dtype != RXW8_BF16)
    return fail(RXW8_INVALID_ARGUMENT, "dequantize: out dtype must be F32 or BF16");
  const int64_t n = weight->dims[0], k = weight->dims[1], groups = scale->dims[1];
  if (n <= 0 || k <= 0 || groups <= 0 || k % groups)
    return fail(RXW8_INVALID_ARGUMENT, "dequantize: group count must divide the input width");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  Buffer *o = nullptr;
  int rc = new_buffer(rt, out_dtype, weight->dims, 2, false, &o);
  if (rc) return rc;
  DequantArgs a;
  a.w = (const uint8_t *)weight->ptr;
  a.scale = (const float *)scale->ptr;
  a.out = o->ptr;
  a.n = n;
  a.k = k;
  a.g = k / groups;
  a.out_bf16 = out_dtype == RXW8_BF16;
  rc = launch(rt, "rxw8_dequant", dim3(grid_for(n * k, 256, 1 << 14)), dim3(256), a);
  if (rc) {
    rxw8_buffer_release(static_cast<rxw8_buffer *>(o));
    return rc;
  }
  *out = static_cast<rxw8_buffer *>(o);
  return RXW8_OK;
}

int rxw8_quantize_w8(rxw8_runtime *rt, rxw8_buffer *w, int64_t group_size, rxw8_buffer **weight,
                     rxw8_buffer **scale) {
  if (!rt || !w || !weight || !scale) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if ((w->dtype != RXW8_F32 && w->dtype != RXW8_BF16) || w->rank != 2)
    return fail(RXW8_INVALID_ARGUMENT, "quantize_w8: weight must be F32 or BF16 [rows, columns]");
  if (group_size <= 0) return fail(RXW8_INVALID_ARGUMENT, "group size must be positive");
  const int64_t n = w->dims[0], k = w->dims[1];
  if (n <= 0 || k <= 0) return fail(RXW8_INVALID_ARGUMENT, "quantize_w8: empty weight %s", dims_str(w).c_str());
  if (k % group_size)
    return fail(RXW8_INVALID_ARGUMENT, "quantize_w8: width %lld is not divisible by %lld",
                (long long)k, (long long)group_size);
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  Buffer *u = nullptr, *sc = nullptr;
  const int64_t sd[2] = {n, k / group_size};
  int rc = new_buffer(rt, RXW8_U8, w->dims, 2, false, &u);
  if (!rc) rc = new_buffer(rt, RXW8_F32, sd, 2, false, &sc);
  if (!rc) {
    QuantizeArgs a{w->ptr, (uint8_t *)u->ptr, (float *)sc->ptr, n, k, group_size,
                   w->dtype == RXW8_BF16};
    const int64_t units = n * (k / group_size);  // one wave each, 4 per workgroup
    if (units / 4 >= (int64_t)1 << 31)
      rc = fail(RXW8_UNIMPLEMENTED, "quantize_w8: %lld groups exceed the grid", (long long)units);
    else
      rc = launch(rt, "rxw8_quantize_w8", dim3((unsigned)((units + 3) / 4)), dim3(256), a);
  }
  if (rc) {
    if (u) rxw8_buffer_release(static_cast<rxw8_buffer *>(u));
    if (sc) rxw8_buffer_release(static_cast<rxw8_buffer *>(sc));
    return rc;
  }
  *weight = static_cast<rxw8_buffer *>(u);
  *scale = static_cast<rxw8_buffer *>(sc);
  return RXW8_OK;
}

int rxw8_pack_weight(rxw8_runtime *rt, rxw8_buffer *weight, rxw8_buffer **packed) {
  if (!rt || !weight || !packed) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  const bool u8 = weight->dtype == RXW8_U8;
  if ((!u8 && weight->dtype != RXW8_BF16) || weight->rank != 2)
    return fail(RXW8_INVALID_ARGUMENT, "pack_weight: weight must be U8 or BF16 [out, in]");
  const int64_t n = weight->dims[0], k = weight->dims[1];
  const int kb = u8 ? 64 : 32;
  if (n <= 0 || k <= 0 || n % 16 || k % kb)
    return fail(RXW8_INVALID_ARGUMENT, "pack_weight: out %% 16 and in %% %d must be 0 (got [%lld, %lld])",
                kb, (long long)n, (long long)k);
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  const int64_t dims[3] = {n / 16, k / kb, u8 ? 1024 : 512};
  Buffer *o = nullptr;
  int rc = new_buffer(rt, weight->dtype, dims, 3, false, &o);
  if (rc) return rc;
  PackArgs a;
  a.src = weight->ptr;
  a.dst = o->ptr;
  a.n = n;
  a.k = k;
  a.kb = kb;
  a.esize = u8 ? 1 : 2;
  a.ilv_half = 0;
  rc = launch(rt, "rxw8_pack_tiles", dim3(grid_for(n / 16 * (k / kb) * 64, 256, 1 << 14)),
              dim3(256), a);
  if (rc) {
    rxw8_buffer_release(static_cast<rxw8_buffer *>(o));
    return rc;
  }
  *packed = static_cast<rxw8_buffer *>(o);
  return RXW8_OK;
}

int rxw8_quantized_linear_into(rxw8_runtime *rt, rxw8_buffer *x, rxw8_buffer *weight,
                               rxw8_buffer *scale, int compute_dtype, rxw8_buffer *y) {
  if (!rt || !y) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  int64_t M, N, K, G;
  int rc = check_qlinear(x, weight, scale, compute_dtype, &M, &N, &K, &G);
  if (rc) return rc;
  if (!is_f(y->dtype) || (compute_dtype == RXW8_F32 && y->dtype != RXW8_F32))
    return fail(RXW8_INVALID_ARGUMENT, "QuantizedLinear output: dtype does not match the schema");
  bool shape_ok = y->rank == x->rank && y->dims[y->rank - 1] == N;
  for (int i = 0; shape_ok && i < x->rank - 1; ++i) shape_ok = y->dims[i] == x->dims[i];
  if (!shape_ok)
    return fail(RXW8_INVALID_ARGUMENT, "QuantizedLinear output %s: shape does not match the schema",
                dims_str(y).c_str());
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  return qlinear_launch(rt, x->ptr, x->dtype == RXW8_F32, (const uint8_t *)weight->ptr,
                        weight->rank == 3, (const float *)scale->ptr, y->ptr,
                        y->dtype == RXW8_F32, M, N, K, G, compute_dtype == RXW8_BF16);
}

int rxw8_quantized_linear_group(rxw8_runtime *rt, int count, rxw8_buffer *const *x,
                                rxw8_buffer *const *weight, rxw8_buffer *const *scale,
                                rxw8_buffer *const *y) {
  if (!rt || !x || !weight || !scale || !y) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (count < 1 || count > kGemvGroupMax)
    return fail(RXW8_INVALID_ARGUMENT, "group of %d linears outside [1, %d]", count, kGemvGroupMax);
  // Every product runs a 12-wave tiling with the whole K in one workgroup and
  // staged activations: up to 4 rows, 6 row groups of 16 rows (96-row tiles)
  // x 2 k slices; beyond, 12 row groups (192-row tiles), each wave the whole
  // K of its 16 rows. The 5-16-row class holds one workgroup per CU (131 KB
  // of staged rows at K = 4096): 192-row tiles fit the sweep's B = 16 shapes
  // in one round (182 workgroups) where 96-row tiles take 1.4 (sweep 4.80 ->
  // 5.00 TB/s); up to 4 rows, 96-row tiles measured 2% above 48-row ones and
  // 4% above 192-row ones. RXW8_GEMV_GRP_RW_FEW / _RW override (3, 6 or 12).
  constexpr int kNw = 12;
  auto rw_env = [](const char *name, int dflt) {
    const int v = env_int(name, dflt);
    return v == 3 || v == 6 || v == 12 ? v : dflt;
  };
  static const int rw_many = rw_env("RXW8_GEMV_GRP_RW", 12);
  static const int rw_few = rw_env("RXW8_GEMV_GRP_RW_FEW", 6);
  auto rw_for = [](int64_t m) { return m > 4 ? rw_many : rw_few; };
  struct Item {
    int64_t M, N, K, G;
    size_t lds;
    bool wave_stage;
  } it[kGemvGroupMax];
  bool packed = false;
  for (int i = 0; i < count; ++i) {
    if (!y[i]) return fail(RXW8_INVALID_ARGUMENT, "group linear %d: NULL output", i);
    Item &t = it[i];
    int rc = check_qlinear(x[i], weight[i], scale[i], RXW8_BF16, &t.M, &t.N, &t.K, &t.G);
    if (rc) return fail(rc, "group linear %d: %s", i, std::string(rxw8_last_error()).c_str());
    if (x[i]->rt != rt) return fail(RXW8_INVALID_ARGUMENT, "group linear %d: buffers of another runtime", i);
    bool shape_ok = is_f(y[i]->dtype) && y[i]->rank == x[i]->rank && y[i]->dims[y[i]->rank - 1] == t.N;
    for (int d = 0; shape_ok && d < x[i]->rank - 1; ++d) shape_ok = y[i]->dims[d] == x[i]->dims[d];
    if (!shape_ok)
      return fail(RXW8_INVALID_ARGUMENT, "group linear %d: output %s does not match", i,
                  dims_str(y[i]).c_str());
    if (i == 0) packed = weight[0]->rank == 3;
    if ((weight[i]->rank == 3) != packed)
      return fail(RXW8_INVALID_ARGUMENT, "group linears must all take packed or all row-major weights");
    if (t.M < 1 || t.M > 16 || t.N % 16 || t.K % 512 || (t.G != t.K && (t.K / 4) % t.G))
      return fail(RXW8_UNIMPLEMENTED,
                  "group linear %d: needs 1..16 rows, N %% 16 == 0, K %% 512 == 0 and whole scale "
                  "groups per quarter of K (M=%lld N=%lld K=%lld G=%lld)",
                  i, (long long)t.M, (long long)t.N, (long long)t.K, (long long)t.G);
    const int rw = rw_for(t.M);
    t.wave_stage = gemv_wave_stage(t.M, t.K, t.G, rw, false);
    t.lds = gemv_lds(t.M, t.K, t.K, t.G, rw, 1, false, kNw);
    if (t.lds + 256 > rt->lds_max)
      return fail(RXW8_UNIMPLEMENTED, "group linear %d: staged rows need %zu bytes of LDS", i, t.lds);
  }
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  const char *rc_env = std::getenv("RXW8_GEMV_REF_CAST");
  const bool ref_cast = !(rc_env && *rc_env == '0');
  // One launch per class of staged rows: up to 4 rows need at most 33 KB of
  // LDS per workgroup (K = 4096), 16 rows 131 KB; a launch's LDS is its
  // largest problem's.
  for (int cls = 0; cls < 2; ++cls) {
    GemvGroupArgs a{};
    a.base.ksplit = 1;
    a.base.y_mode = 0;
    a.base.x_mode = 0;
    size_t lds = 0;
    int tiles = 0, u = 4;
    const int rw = cls == 1 ? rw_many : rw_few;
    for (int i = 0; i < count; ++i) {
      if ((it[i].M > 4) != (cls == 1)) continue;
      GemvProblem &q = a.p[a.count++];
      q.x = x[i]->ptr;
      q.w = weight[i]->ptr;
      q.scale = (const float *)scale[i]->ptr;
      q.y = y[i]->ptr;
      q.M = (int)it[i].M;
      q.N = (int)it[i].N;
      q.K = (int)it[i].K;
      q.G = (int)it[i].G;
      q.tile_begin = tiles;
      q.x_f32 = x[i]->dtype == RXW8_F32;
      q.y_f32 = y[i]->dtype == RXW8_F32;
      q.wave_stage = it[i].wave_stage;
      q.lds_dma = !q.x_f32 && !q.wave_stage && (uintptr_t)q.x % 16 == 0;
      tiles += (int)((it[i].N + 16 * rw - 1) / (16 * rw));
      lds = std::max(lds, it[i].lds);
      const int64_t chunks = it[i].K / (kNw / rw) / 64;
      while (chunks % (2 * u)) u /= 2;
    }
    if (a.count == 0) continue;
    char kname[64];
    std::snprintf(kname, sizeof kname, "rxw8_gemv_%sw8%s_mb1_rw%d_u%d_w12_grp", ref_cast ? "rc_" : "",
                  packed ? "_pk" : "", rw, u);
    if (int rc = launch(rt, kname, dim3((unsigned)tiles), dim3(64 * kNw), a, lds)) return rc;
  }
  return RXW8_OK;
}

int rxw8_quantized_linear(rxw8_runtime *rt, rxw8_buffer *x, rxw8_buffer *weight,
                          rxw8_buffer *scale, int compute_dtype, int out_dtype,
                          rxw8_buffer **y) {
  if (!rt || !y) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  int64_t M, N, K, G;
  int rc = check_qlinear(x, weight, scale, compute_dtype, &M, &N, &K, &G);
  if (rc) return rc;
  if (!is_f(out_dtype) || (compute_dtype == RXW8_F32 && out_dtype != RXW8_F32))
    return fail(RXW8_INVALID_ARGUMENT, "QuantizedLinear: out dtype must be F32 (or BF16 with BF16 compute)");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  int64_t dims[RXW8_MAX_RANK];
  for (int i = 0; i < x->rank; ++i) dims[i] = x->dims[i];
  dims[x->rank - 1] = N;
  Buffer *o = nullptr;
  rc = new_buffer(rt, out_dtype, dims, x->rank, false, &o);
  if (rc) return rc;
  rc = rxw8_quantized_linear_into(rt, x, weight, scale, compute_dtype, static_cast<rxw8_buffer *>(o));
  if (rc) {
    rxw8_buffer_release(static_cast<rxw8_buffer *>(o));
    return rc;
  }
  *y = static_cast<rxw8_buffer *>(o);
  return RXW8_OK;
}

static int check_bf16_linear(const Buffer *x, const Buffer *w, int64_t *M, int64_t *N, int64_t *K) {
  if (!x || !w) return fail(RXW8_INVALID_ARGUMENT, "Linear: NULL buffer");
  if (x->rt != w->rt) return fail(RXW8_INVALID_ARGUMENT, "Linear: buffers belong to different runtimes");
  if (x->rank < 1 || !is_f(x->dtype))
    return fail(RXW8_INVALID_ARGUMENT, "Linear requires an F32 or BF16 input with rank at least one");
  const bool packed = w->rank == 3;
  if (w->dtype != RXW8_BF16 || (w->rank != 2 && !(packed && w->dims[2] == 512)))
    return fail(RXW8_INVALID_ARGUMENT,
                "Linear weight: dtype does not match the schema (BF16 [out, in], or packed BF16 "
                "[out/16, in/32, 512])");
  *K = x->dims[x->rank - 1];
  *N = packed ? w->dims[0] * 16 : w->dims[0];
  if (*K <= 0 || *N <= 0 || (packed ? w->dims[1] * 32 : w->dims[1]) != *K)
    return fail(RXW8_INVALID_ARGUMENT, "Linear weight %s: shape does not match input width %lld",
                dims_str(w).c_str(), (long long)*K);
  *M = 1;
  for (int i = 0; i < x->rank - 1; ++i) *M *= x->dims[i];
  return RXW8_OK;
}

int rxw8_linear_bf16_into(rxw8_runtime *rt, rxw8_buffer *x, rxw8_buffer *weight, rxw8_buffer *y) {
  if (!rt || !y) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  int64_t M, N, K;
  int rc = check_bf16_linear(x, weight, &M, &N, &K);
  if (rc) return rc;
  bool shape_ok = is_f(y->dtype) && y->rank == x->rank && y->dims[y->rank - 1] == N;
  for (int i = 0; shape_ok && i < x->rank - 1; ++i) shape_ok = y->dims[i] == x->dims[i];
  if (!shape_ok) return fail(RXW8_INVALID_ARGUMENT, "Linear output: shape or dtype mismatch");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  return bf16_linear_launch(rt, x->ptr, x->dtype == RXW8_F32, (const uint16_t *)weight->ptr,
                            weight->rank == 3, y->ptr, y->dtype == RXW8_F32, M, N, K);
}

int rxw8_linear_bf16(rxw8_runtime *rt, rxw8_buffer *x, rxw8_buffer *weight, int out_dtype,
                     rxw8_buffer **y) {
  if (!rt || !y) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  int64_t M, N, K;
  int rc = check_bf16_linear(x, weight, &M, &N, &K);
  if (rc) return rc;
  if (!is_f(out_dtype)) return fail(RXW8_INVALID_ARGUMENT, "Linear: out dtype must be F32 or BF16");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  int64_t dims[RXW8_MAX_RANK];
  for (int i = 0; i < x->rank; ++i) dims[i] = x->dims[i];
  dims[x->rank - 1] = N;
  Buffer *o = nullptr;
  rc = new_buffer(rt, out_dtype, dims, x->rank, false, &o);
  if (rc) return rc;
  rc = rxw8_linear_bf16_into(rt, x, weight, static_cast<rxw8_buffer *>(o));
  if (rc) {
    rxw8_buffer_release(static_cast<rxw8_buffer *>(o));
    return rc;
  }
  *y = static_cast<rxw8_buffer *>(o);
  return RXW8_OK;
}


static int check_prefill(const Buffer *q, const Buffer *k, const Buffer *v, const Buffer *starts) {
  if (!q || !k || !v || !starts) return fail(RXW8_INVALID_ARGUMENT, "GQA prefill: NULL buffer");
  if (q->rank != 4 || k->rank != 4 || v->rank != 4)
    return fail(RXW8_INVALID_ARGUMENT, "GQA prefill requires q [B,S,Hq,D] and caches [B,Hkv,Lmax,D]");
  if (!is_f(q->dtype) || k->dtype != RXW8_BF16 || v->dtype != RXW8_BF16)
    return fail(RXW8_INVALID_ARGUMENT, "GQA prefill requires F32/BF16 q and BF16 caches");
  for (int i = 0; i < 4; ++i)
    if (k->dims[i] != v->dims[i])
      return fail(RXW8_INVALID_ARGUMENT, "GQA: K/V caches must have equal shapes");
  const int64_t B = q->dims[0], S = q->dims[1], Hq = q->dims[2], D = q->dims[3];
  if (k->dims[0] != B || k->dims[3] != D || S < 1 || S > k->dims[2])
    return fail(RXW8_INVALID_ARGUMENT, "GQA prefill: batch/dim mismatch or S outside [1, Lmax]");
  if (Hq <= 0 || k->dims[1] <= 0 || Hq % k->dims[1] != 0)
    return fail(RXW8_INVALID_ARGUMENT,
                "GQA requires equal batch prefixes and divisible positive head counts");
  if (D > 512) return fail(RXW8_UNIMPLEMENTED, "GQA prefill: head dim %lld > 512", (long long)D);
  if (starts->dtype != RXW8_I32 || starts->rank != 1 || starts->dims[0] != B)
    return fail(RXW8_INVALID_ARGUMENT, "GQA prefill: starts must be I32 [B]");
  return RXW8_OK;
}

static int check_gqa(const Buffer *q, const Buffer *k, const Buffer *v, const Buffer *lens,
                     const Buffer *mask, int64_t *mask_sb, int64_t *mask_sh) {
  if (!q || !k || !v || !lens) return fail(RXW8_INVALID_ARGUMENT, "GQA: NULL buffer");
  if (q->rank != 3 || k->rank != 4 || v->rank != 4)
    return fail(RXW8_INVALID_ARGUMENT, "GQA decode requires q [B,Hq,D] and caches [B,Hkv,Lmax,D]");
  if (!is_f(q->dtype) || !is_f(k->dtype) || k->dtype != v->dtype)
    return fail(RXW8_INVALID_ARGUMENT, "GQA decode requires F32/BF16 q and matching F32/BF16 caches");
  const int64_t B = q->dims[0], Hq = q->dims[1], D = q->dims[2];
  for (int i = 0; i < 4; ++i)
    if (k->dims[i] != v->dims[i])
      return fail(RXW8_INVALID_ARGUMENT, "GQA: K/V caches must have equal shapes");
  if (k->dims[0] != B || Hq <= 0 || k->dims[1] <= 0 || Hq % k->dims[1] != 0 || k->dims[3] != D ||
      D <= 0 || k->dims[2] <= 0)
    return fail(RXW8_INVALID_ARGUMENT,
                "GQA requires equal batch prefixes and divisible positive head counts");
  if (lens->dtype != RXW8_I32 || lens->rank != 1 || lens->dims[0] != B)
    return fail(RXW8_INVALID_ARGUMENT, "GQA: lens must be I32 [B]");
  *mask_sb = *mask_sh = 0;
  if (mask) {
    const int64_t L = k->dims[2];
    if (mask->dtype != RXW8_F32 || mask->rank != 3 || mask->dims[2] != L ||
        (mask->dims[0] != 1 && mask->dims[0] != B) || (mask->dims[1] != 1 && mask->dims[1] != Hq))
      return fail(RXW8_INVALID_ARGUMENT, "GQA: mask must be F32 [B|1, Hq|1, Lmax]");
    *mask_sh = mask->dims[1] == 1 ? 0 : L;
    *mask_sb = mask->dims[0] == 1 ? 0 : mask->dims[1] * L;
  }
  return RXW8_OK;
}

int rxw8_causal_attention_mask(rxw8_runtime *rt, rxw8_buffer *query_positions,
                               rxw8_buffer *key_positions, rxw8_buffer **out) {
  if (!rt || !query_positions || !key_positions || !out)
    return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (query_positions->dtype != RXW8_I32 || key_positions->dtype != RXW8_I32)
    return fail(RXW8_INVALID_ARGUMENT, "causal positions must be I32 tensors");
  if (query_positions->rank != 1 || key_positions->rank != 1)
    return fail(RXW8_INVALID_ARGUMENT, "causal positions must be rank-one I32 tensors");
  const int64_t Q = query_positions->dims[0], K = key_positions->dims[0];
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  const int64_t od[2] = {Q, K};
  Buffer *o = nullptr;
  int rc = new_buffer(rt, RXW8_F32, od, 2, false, &o);
  if (rc) return rc;
  if (Q * K > 0) {
    CausalMaskArgs a{(const int32_t *)query_positions->ptr, (const int32_t *)key_positions->ptr,
                     (float *)o->ptr, Q, K};
    rc = launch(rt, "rxw8_gqa_causal_mask", dim3(grid_for(Q * K, 256, 1 << 14)), dim3(256), a);
    if (rc) {
      rxw8_buffer_release(static_cast<rxw8_buffer *>(o));
      return rc;
    }
  }
  *out = static_cast<rxw8_buffer *>(o);
  return RXW8_OK;
}

int rxw8_gqa_attention_into(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k, rxw8_buffer *v,
                            rxw8_buffer *mask, const float *scale, rxw8_buffer *out) {
  if (!rt || !q || !k || !v || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  const int r = q->rank;
  if (r < 3 || k->rank != r || v->rank != r)
    return fail(RXW8_INVALID_ARGUMENT, "GQA requires matching ranks >= 3");
  if (q->dtype != RXW8_F32 || k->dtype != RXW8_F32 || v->dtype != RXW8_F32 ||
      (mask && mask->dtype != RXW8_F32))
    return fail(RXW8_INVALID_ARGUMENT, "attention requires F32 Q/K/V and mask tensors");
  const int hd = r - 3;
  bool ok = q->dims[hd] > 0 && k->dims[hd] > 0 && v->dims[hd] == k->dims[hd] &&
            q->dims[hd] % k->dims[hd] == 0;
  for (int i = 0; ok && i < hd; ++i) ok = q->dims[i] == k->dims[i] && q->dims[i] == v->dims[i];
  if (!ok)
    return fail(RXW8_INVALID_ARGUMENT, "GQA requires equal batch prefixes and divisible positive head counts");
  const int64_t Hq = q->dims[hd], Hkv = k->dims[hd], Sq = q->dims[hd + 1], D = q->dims[hd + 2];
  const int64_t Sk = k->dims[hd + 1], Dv = v->dims[hd + 2];
  if (D <= 0 || k->dims[hd + 2] != D || Sk == 0 || v->dims[hd + 1] != Sk)
    return fail(RXW8_INVALID_ARGUMENT, "attention requires matching positive Q/K depth and K/V length");
  const float sc = scale ? *scale : 1.0f / std::sqrt((float)D);
  if (!std::isfinite(sc)) return fail(RXW8_INVALID_ARGUMENT, "attention scale must be finite");
  bool out_ok = out->dtype == RXW8_F32 && out->rank == r && out->dims[hd + 2] == Dv;
  for (int i = 0; out_ok && i < hd + 2; ++i) out_ok = out->dims[i] == q->dims[i];
  if (!out_ok) return fail(RXW8_INVALID_ARGUMENT, "GQA output must be F32 [..., Hq, Sq, Dv]");
  if (hd > 4 || D > 1024 || Dv > 512)
    return fail(RXW8_UNIMPLEMENTED,
                "GQA: supported up to 4 batch dimensions, depth 1024 and value depth 512");
  GqaGeneralArgs a{};
  a.q = q->ptr;
  a.k = k->ptr;
  a.v = v->ptr;
  a.out = out->ptr;
  // contiguous [NB, H, S, D] operands
  a.q_si = D, a.q_sh = Sq * D, a.q_sb = Hq * Sq * D;
  a.o_si = Dv, a.o_sh = Sq * Dv, a.o_sb = Hq * Sq * Dv;
  a.k_sh = Sk * D, a.k_sb = Hkv * Sk * D;
  a.v_sh = Sk * Dv, a.v_sb = Hkv * Sk * Dv;
  for (int t = 0; t < 4; ++t) a.bdim[t] = 1, a.mb[t] = 0;
  int64_t NB = 1;
  for (int i = 0; i < hd; ++i) {
    a.bdim[4 - hd + i] = q->dims[i];
    NB *= q->dims[i];
  }
  if (mask) {
    // right-aligned broadcast against the scores [..., Hq, Sq, Sk]
    int64_t sd[RXW8_MAX_RANK];
    for (int i = 0; i < hd + 2; ++i) sd[i] = q->dims[i];
    sd[hd + 2] = Sk;
    if (mask->rank > r)
      return fail(RXW8_INVALID_ARGUMENT, "GQA mask %s cannot broadcast to the scores", dims_str(mask).c_str());
    int64_t stride[RXW8_MAX_RANK] = {0}, st = 1;
    for (int i = mask->rank - 1; i >= 0; --i) {
      stride[i] = mask->dims[i] == 1 ? 0 : st;
      st *= mask->dims[i];
    }
    int64_t ms[RXW8_MAX_RANK] = {0};
    for (int t = 0; t < r; ++t) {
      const int mt = t - (r - mask->rank);
      if (mt < 0) continue;
      if (mask->dims[mt] != 1 && mask->dims[mt] != sd[t])
        return fail(RXW8_INVALID_ARGUMENT, "GQA mask %s cannot broadcast to the scores", dims_str(mask).c_str());
      ms[t] = stride[mt];
    }
    for (int i = 0; i < hd; ++i) a.mb[4 - hd + i] = ms[i];
    a.mask = (const float *)mask->ptr;
    a.msh = ms[hd];
    a.msi = ms[hd + 1];
    a.msj = ms[hd + 2];
  }
  a.rows = NB * Hq * Sq;
  a.Hq = (int)Hq, a.Hkv = (int)Hkv, a.Sq = (int)Sq, a.Sk = (int)Sk, a.D = (int)D, a.Dv = (int)Dv;
  a.scale = sc;
  if (a.rows == 0) return RXW8_OK;
  if ((a.rows + 3) / 4 >= ((int64_t)1 << 31) || Sq > INT32_MAX || Sk > INT32_MAX)
    return fail(RXW8_UNIMPLEMENTED, "GQA: %lld rows exceed the kernel's grid", (long long)a.rows);
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  return launch(rt, "rxw8_gqa_general", dim3((unsigned)((a.rows + 3) / 4)), dim3(256), a);
}

int rxw8_gqa_attention(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k, rxw8_buffer *v,
                       rxw8_buffer *mask, const float *scale, rxw8_buffer **out) {
  if (!rt || !q || !k || !v || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (q->rank < 3 || v->rank != q->rank)
    return fail(RXW8_INVALID_ARGUMENT, "GQA requires matching ranks >= 3");
  int64_t od[RXW8_MAX_RANK];
  for (int i = 0; i < q->rank; ++i) od[i] = q->dims[i];
  od[q->rank - 1] = v->dims[v->rank - 1];
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  Buffer *o = nullptr;
  int rc = new_buffer(rt, RXW8_F32, od, q->rank, false, &o);
  if (rc) return rc;
  rc = rxw8_gqa_attention_into(rt, q, k, v, mask, scale, static_cast<rxw8_buffer *>(o));
  if (rc) {
    rxw8_buffer_release(static_cast<rxw8_buffer *>(o));
    return rc;
  }
  *out = static_cast<rxw8_buffer *>(o);
  return RXW8_OK;
}

}  // extern "C"

namespace rxw8 {
int gqa_decode_into(Runtime *rt, Buffer *q, Buffer *k_cache, Buffer *v_cache, Buffer *lens,
                    Buffer *mask, float scale, Buffer *out, const AttnWorkspace *ws) {
  if (!rt || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  int64_t sb, sh;
  int rc = check_gqa(q, k_cache, v_cache, lens, mask, &sb, &sh);
  if (rc) return rc;
  if (!is_f(out->dtype) || out->rank != 3 || out->dims[0] != q->dims[0] ||
      out->dims[1] != q->dims[1] || out->dims[2] != q->dims[2])
    return fail(RXW8_INVALID_ARGUMENT, "GQA output: shape or dtype mismatch");
  if (!std::isfinite(scale)) return fail(RXW8_INVALID_ARGUMENT, "attention scale must be finite");
  const int64_t D = q->dims[2];
  if (scale <= 0.f) scale = 1.0f / std::sqrt((float)D);
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  return attention_launch(rt, q->ptr, q->dtype == RXW8_F32, k_cache->ptr, v_cache->ptr,
                          k_cache->dtype == RXW8_F32, (const int32_t *)lens->ptr, nullptr,
                          mask ? (const float *)mask->ptr : nullptr, sb, sh, out->ptr,
                          out->dtype == RXW8_F32, q->dims[0], q->dims[1], k_cache->dims[1],
                          k_cache->dims[2], D, scale, nullptr, ws);
}
}  // namespace rxw8

extern "C" {

int rxw8_gqa_decode_into(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k_cache,
                         rxw8_buffer *v_cache, rxw8_buffer *lens, rxw8_buffer *mask, float scale,
                         rxw8_buffer *out) {
  return rxw8::gqa_decode_into(rt, q, k_cache, v_cache, lens, mask, scale, out, nullptr);
}

int rxw8_gqa_decode(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k_cache, rxw8_buffer *v_cache,
                    rxw8_buffer *lens, rxw8_buffer *mask, float scale, int out_dtype,
                    rxw8_buffer **out) {
  if (!rt || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  int64_t sb, sh;
  int rc = check_gqa(q, k_cache, v_cache, lens, mask, &sb, &sh);
  if (rc) return rc;
  if (!is_f(out_dtype)) return fail(RXW8_INVALID_ARGUMENT, "GQA: out dtype must be F32 or BF16");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  Buffer *o = nullptr;
  rc = new_buffer(rt, out_dtype, q->dims, 3, false, &o);
  if (rc) return rc;
  rc = rxw8_gqa_decode_into(rt, q, k_cache, v_cache, lens, mask, scale, static_cast<rxw8_buffer *>(o));
  if (rc) {
    rxw8_buffer_release(static_cast<rxw8_buffer *>(o));
    return rc;
  }
  *out = static_cast<rxw8_buffer *>(o);
  return RXW8_OK;
}

int rxw8_gqa_prefill_into(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k_cache,
                          rxw8_buffer *v_cache, rxw8_buffer *starts, float scale,
                          rxw8_buffer *out) {
  if (!rt || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  int rc = check_prefill(q, k_cache, v_cache, starts);
  if (rc) return rc;
  if (!is_f(out->dtype) || out->rank != 4)
    return fail(RXW8_INVALID_ARGUMENT, "GQA prefill output: shape or dtype mismatch");
  for (int i = 0; i < 4; ++i)
    if (out->dims[i] != q->dims[i])
      return fail(RXW8_INVALID_ARGUMENT, "GQA prefill output: shape or dtype mismatch");
  if (!std::isfinite(scale)) return fail(RXW8_INVALID_ARGUMENT, "attention scale must be finite");
  const int64_t B = q->dims[0], S = q->dims[1], Hq = q->dims[2], D = q->dims[3];
  if (scale <= 0.f) scale = 1.0f / std::sqrt((float)D);
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  if (!prefill_supported(Hq, k_cache->dims[1], D, 0))
    return prefill_general(rt, q->ptr, q->dtype != RXW8_F32, S * Hq * D, Hq * D, D,
                           (const uint16_t *)k_cache->ptr, (const uint16_t *)v_cache->ptr,
                           (const int32_t *)starts->ptr, out->ptr, out->dtype != RXW8_F32,
                           S * Hq * D, Hq * D, D, B, S, Hq, k_cache->dims[1], k_cache->dims[2], D,
                           scale);
  return prefill_launch(rt, q->ptr, q->dtype == RXW8_F32, S * Hq * D, Hq * D, D,
                        (const uint16_t *)k_cache->ptr, (const uint16_t *)v_cache->ptr,
                        (const int32_t *)starts->ptr, nullptr, out->ptr, out->dtype == RXW8_F32,
                        S * Hq * D, Hq * D, D, B, S, Hq, k_cache->dims[1], k_cache->dims[2], scale);
}

int rxw8_gqa_prefill(rxw8_runtime *rt, rxw8_buffer *q, rxw8_buffer *k_cache, rxw8_buffer *v_cache,
                     rxw8_buffer *starts, float scale, int out_dtype, rxw8_buffer **out) {
  if (!rt || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  int rc = check_prefill(q, k_cache, v_cache, starts);
  if (rc) return rc;
  if (!is_f(out_dtype)) return fail(RXW8_INVALID_ARGUMENT, "GQA prefill: out dtype must be F32 or BF16");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  Buffer *o = nullptr;
  rc = new_buffer(rt, out_dtype, q->dims, 4, false, &o);
  if (rc) return rc;
  rc = rxw8_gqa_prefill_into(rt, q, k_cache, v_cache, starts, scale, static_cast<rxw8_buffer *>(o));
  if (rc) {
    rxw8_buffer_release(static_cast<rxw8_buffer *>(o));
    return rc;
  }
  *out = static_cast<rxw8_buffer *>(o);
  return RXW8_OK;
}

int rxw8_kv_update_at(rxw8_runtime *rt, rxw8_buffer *k_cache, rxw8_buffer *v_cache,
                      rxw8_buffer *k_update, rxw8_buffer *v_update, rxw8_buffer *starts,
                      int checked, rxw8_buffer *accepted) {
  if (!rt || !k_cache || !v_cache || !k_update || !v_update || !starts)
    return fail(RXW8_INVALID_ARGUMENT, "KvCache::update_at: NULL argument");
  if (k_update->rank != v_update->rank || k_update->dtype != v_update->dtype)
    return fail(RXW8_INVALID_ARGUMENT, "K/V updates must have equal shapes");
  for (int i = 0; i < k_update->rank; ++i)
    if (k_update->dims[i] != v_update->dims[i])
      return fail(RXW8_INVALID_ARGUMENT, "K/V updates must have equal shapes");
  const int rank = k_cache->rank;
  if (rank < 1 || rank > 8 || v_cache->rank != rank || k_update->rank != rank)
    return fail(RXW8_INVALID_ARGUMENT, "KvCache::update_at: cache and update ranks must match (1..8)");
  if (k_cache->dtype != v_cache->dtype || k_update->dtype != k_cache->dtype)
    return fail(RXW8_INVALID_ARGUMENT, "KvCache::update_at: cache/update dtypes must match");
  for (int i = 0; i < rank; ++i) {
    if (k_cache->dims[i] != v_cache->dims[i])
      return fail(RXW8_INVALID_ARGUMENT, "KvCache::update_at: K/V caches must have equal shapes");
    if (k_update->dims[i] > k_cache->dims[i])
      return fail(RXW8_INVALID_ARGUMENT, "KvCache::update_at: update larger than the cache");
  }
  if (starts->dtype != RXW8_I32 || starts->rank != 1 || starts->dims[0] != rank)
    return fail(RXW8_INVALID_ARGUMENT, "KvCache::update_at: starts must be I32 [rank]");
  if (accepted && (accepted->dtype != RXW8_F32 || accepted->numel() != 1))
    return fail(RXW8_INVALID_ARGUMENT, "KvCache::update_at: accepted must be an F32 scalar");
  if (k_cache == v_cache) return fail(RXW8_INVALID_ARGUMENT, "K and V caches must be distinct buffers");
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  KvUpdateArgs a;
  std::memset(&a, 0, sizeof a);
  a.kc = k_cache->ptr;
  a.vc = v_cache->ptr;
  a.ku = k_update->ptr;
  a.vu = v_update->ptr;
  a.starts = (const int32_t *)starts->ptr;
  a.accepted = accepted ? (float *)accepted->ptr : nullptr;
  for (int i = 0; i < rank; ++i) {
    a.dims[i] = k_cache->dims[i];
    a.udims[i] = k_update->dims[i];
  }
  a.total = k_update->numel();
  a.rank = rank;
  a.elem = (int)dtype_size(k_cache->dtype);
  a.checked = checked ? 1 : 0;
  return launch(rt, "rxw8_kv_update", dim3(grid_for(a.total, 256, 4096)), dim3(256), a);
}

}  // extern "C"
