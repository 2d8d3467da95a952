/*
 * fmd_oracle.c -- CPU restatement of the batched Qwen3 decoder hot path of
 * cnmoro/fast-moss-diarization.  TEST INFRASTRUCTURE ONLY (the checker):
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it;
 * the product library never does.
 *
 * Each function names the reference file:line it restates.  Paths are
 * relative to crates/fmd-core/src/.
 *
 * Rounding model: the reference keeps every candle tensor in the activation
 * dtype (precision.rs:32-41), so each op's output is rounded to that dtype
 * here (or_round).  Inside one op the arithmetic is f32 (candle's fused
 * kernels accumulate in f32: linear.rs:294-296).  What candle does *inside*
 * an op (reduction order, whether rms_norm multiplies before or after the
 * weight, how QMatMul treats f16 inputs) is not visible from the reference
 * and is tolerance-governed.
 */
#include "fmd_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[512];
static void set_err(const char* msg) { snprintf(g_err, sizeof g_err, "%s", msg); }
const char* or_last_error(void) { return g_err; }

static inline uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

/* Approximately normal deviates for synthetic data: the sum of four 16-bit
 * uniforms from one SplitMix64 draw (Irwin-Hall, rescaled to unit variance). */
static inline float approx_normal(uint64_t key) {
  const uint64_t z = splitmix64(key);
  const float s = (float)(z & 0xffff) + (float)((z >> 16) & 0xffff) + (float)((z >> 32) & 0xffff) +
                  (float)(z >> 48);
  return (s * (1.0f / 65536.0f) - 2.0f) * 1.7320508f;
}

void or_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------------------ */
/* IEEE conversions, written from the binary16 / bfloat16 definitions.      */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t or_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) {                     /* inf / nan */
    if (man == 0) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | (man >> 13));
  }
  if (exp == 0) return (uint16_t)sign;    /* f32 zero/subnormal -> +-0 */
  int e = (int)exp - 127;                 /* unbiased */
  if (e >= -14) {                         /* f16 normal range (or overflow) */
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    uint32_t m10 = man >> 13, rem = man & 0x1fffu;
    uint32_t r = ((uint32_t)(e + 15) << 10) + m10;
    if (rem > 0x1000u || (rem == 0x1000u && (m10 & 1u))) r += 1; /* carries */
    if (r >= 0x7c00u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | r);
  }
  /* f16 subnormal: value = M * 2^(e-23), unit 2^-24 -> M >> s, s = -e-1 */
  uint32_t M = man | 0x800000u;
  int s = -e - 1;
  if (s >= 25) return (uint16_t)sign;
  uint32_t q = M >> s, rem = M & ((1u << s) - 1u), half = 1u << (s - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  return (uint16_t)(sign | q);
}

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0x1fu) return u2f(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    float v = (float)man * (1.0f / 16777216.0f);   /* man * 2^-24, exact */
    return sign ? -v : v;
  }
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t or_f32_to_bf16(float f) {
  uint32_t x = f2u(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

float or_round(float x, int prec) {
  switch (prec) {
    case OR_F16:
    case OR_INT8: return or_f16_to_f32(or_f32_to_f16(x));
    case OR_BF16: return or_bf16_to_f32(or_f32_to_bf16(x));
    default: return x;
  }
}

void or_round_array(float* x, int64_t n, int prec) {
  if (prec == OR_F32) return;
  for (int64_t i = 0; i < n; ++i) x[i] = or_round(x[i], prec);
}

/* ------------------------------------------------------------------------ */
/* Q8_0: candle QTensor::quantize(&w_f32, GgmlDType::Q8_0), reached from     */
/* linear.rs:194-201 (Loader::linear_with) and 239-251 (fused_linear).       */
/* Per 32-value block along the input axis: amax = max|x| (f32), d = amax/127*/
/* (f32), id = d != 0 ? 1/d : 0 (f32), q = (i8) round_half_away(x*id) with   */
/* Rust's saturating float->int cast (NaN -> 0); d stored as f16 (RNE).     */
/* Block bytes: f16 d little-endian, then 32 x int8 (GGML block_q8_0).      */
/* ------------------------------------------------------------------------ */

static inline int8_t rust_f32_to_i8(float v) {
  if (v != v) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int8_t)v;
}

void or_quantize_q8_0(const float* x, int64_t rows, int64_t cols, uint8_t* out) {
  const int64_t nb = cols / 32;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t b = 0; b < nb; ++b) {
      const float* xs = x + r * cols + b * 32;
      uint8_t* blk = out + (r * nb + b) * 34;
      float amax = 0.0f;
      for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(xs[j]));
      float d = amax / 127.0f;
      float id = (d != 0.0f) ? 1.0f / d : 0.0f;
      uint16_t dh = or_f32_to_f16(d);
      blk[0] = (uint8_t)(dh & 0xff);
      blk[1] = (uint8_t)(dh >> 8);
      for (int j = 0; j < 32; ++j) {
        float v = xs[j] * id;
        blk[2 + j] = (uint8_t)rust_f32_to_i8(roundf(v));
      }
    }
  }
}

void or_dequantize_q8_0(const uint8_t* blocks, int64_t rows, int64_t cols, float* out) {
  const int64_t nb = cols / 32;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + (r * nb + b) * 34;
      float d = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      for (int j = 0; j < 32; ++j) out[r * cols + b * 32 + j] = d * (float)(int8_t)blk[2 + j];
    }
}

/* ------------------------------------------------------------------------ */
/* Single ops                                                               */
/* ------------------------------------------------------------------------ */

/* Rope::new (qwen3.rs:117-136): inv_freq in f64 then f32; freqs = pos(f32)
 * x inv_freq (f32 product); cos/sin in f32 then cast to the dtype. */
void or_rope_tables(int head_dim, double theta, int max_len, int prec, float* cos_out,
                    float* sin_out) {
  const int half = head_dim / 2;
  float* inv = (float*)malloc(sizeof(float) * (size_t)half);
  for (int i = 0; i < half; ++i)
    inv[i] = (float)(1.0 / pow(theta, 2.0 * (double)i / (double)head_dim));
#pragma omp parallel for schedule(static)
  for (int p = 0; p < max_len; ++p)
    for (int i = 0; i < half; ++i) {
      float f = (float)p * inv[i];
      cos_out[(size_t)p * half + i] = or_round(cosf(f), prec);
      sin_out[(size_t)p * half + i] = or_round(sinf(f), prec);
    }
  free(inv);
}

/* Qwen3::build_mask (qwen3.rs:523-562): additive (B, 1, repeat*q_len, kv_len);
 * -inf where k > abs_q, or where abs_q >= pad && k < pad; rows tiled repeat
 * times (row r*q_len + qi carries query qi). */
void or_build_mask(int batch, int repeat, int q_offset, int q_len, int kv_len,
                   const int32_t* pad, float* out) {
  const int rows = repeat * q_len;
  const float neg = -INFINITY;
  for (int b = 0; b < batch; ++b)
    for (int qi = 0; qi < q_len; ++qi) {
      int abs_q = q_offset + qi;
      int padding_applies = abs_q >= pad[b];
      float* first = out + ((size_t)b * rows + qi) * kv_len;
      for (int k = 0; k < kv_len; ++k)
        first[k] = (k > abs_q || (padding_applies && k < pad[b])) ? neg : 0.0f;
      for (int r = 1; r < repeat; ++r)
        memcpy(out + ((size_t)b * rows + (size_t)r * q_len + qi) * kv_len, first,
               sizeof(float) * (size_t)kv_len);
    }
}

/* RmsNorm::forward (linear.rs:293-302) -> candle_nn::ops::rms_norm:
 * y = x * (1/sqrt(mean(x^2) + eps)) * w, sum of squares in f32. */
void or_rmsnorm(const float* x, const float* w, int64_t rows, int dim, float eps, int prec,
                float* y) {
#pragma omp parallel for schedule(static) if (rows > 16)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * dim;
    float ss = 0.0f;
#pragma omp simd reduction(+ : ss)
    for (int i = 0; i < dim; ++i) ss += xr[i] * xr[i];
    float scale = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = 0; i < dim; ++i) y[r * dim + i] = or_round(xr[i] * scale * w[i], prec);
  }
}

static inline float dotf(const float* a, const float* b, int n) {
  float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
  for (int i = 0; i < n; ++i) acc += a[i] * b[i];
  return acc;
}

/* Linear::forward Dense (linear.rs:39-46): y = x W^T, W (out, in).
 * Tiled 64 x 64 over (out, rows) so a tile's operands stay in cache. */
void or_linear_dense(const float* x, const float* w, int64_t rows, int in, int out, int prec,
                     float* y) {
  const int64_t nbn = (out + 63) / 64, nbm = (rows + 63) / 64;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t bn = 0; bn < nbn; ++bn)
    for (int64_t bm = 0; bm < nbm; ++bm) {
      const int64_t n1 = (bn + 1) * 64 < out ? (bn + 1) * 64 : out;
      const int64_t m1 = (bm + 1) * 64 < rows ? (bm + 1) * 64 : rows;
      for (int64_t n = bn * 64; n < n1; ++n)
        for (int64_t m = bm * 64; m < m1; ++m)
          y[m * out + n] = or_round(dotf(x + m * in, w + n * in, in), prec);
    }
}

/* Linear::forward Quantized (linear.rs:47-54): y = x deq(Wq)^T with exact
 * dequantisation f32(d) * q and f32 accumulation. */
void or_linear_q8_0(const float* x, const uint8_t* blocks, int64_t rows, int in, int out,
                    int prec, float* y) {
  const int nb = in / 32;
  const int64_t nbn = (out + 63) / 64;
#pragma omp parallel
  {
    float* wt = (float*)malloc(sizeof(float) * (size_t)in * 64);
#pragma omp for schedule(dynamic)
    for (int64_t bn = 0; bn < nbn; ++bn) {
      const int64_t n0 = bn * 64, n1 = (bn + 1) * 64 < out ? (bn + 1) * 64 : out;
      for (int64_t n = n0; n < n1; ++n)
        for (int b = 0; b < nb; ++b) {
          const uint8_t* blk = blocks + ((size_t)n * nb + b) * 34;
          float d = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
          for (int j = 0; j < 32; ++j)
            wt[(n - n0) * in + b * 32 + j] = d * (float)(int8_t)blk[2 + j];
        }
      for (int64_t bm = 0; bm < rows; bm += 64) {
        const int64_t m1 = bm + 64 < rows ? bm + 64 : rows;
        for (int64_t n = n0; n < n1; ++n)
          for (int64_t m = bm; m < m1; ++m)
            y[m * out + n] = or_round(dotf(x + m * in, wt + (n - n0) * in, in), prec);
      }
    }
    free(wt);
  }
}

/* Attention core of Attention::forward (qwen3.rs:237-257) on the regrouped
 * queries.  q: (b, heads, t, hd); k, v: (b, kv_heads, kv_stride, hd) of which
 * [0, kv_len) is read; mask: (b, 1, repeat*t, kv_len) additive or NULL.
 * scores = rd(rd(q.k) * rd(scale)) + mask; probs = rd(softmax); ctx =
 * rd(probs . v); out (b, t, heads*hd), head-major. */
void or_attention(const float* q, const float* k, const float* v, const float* mask, int b,
                  int heads, int kv_heads, int t, int kv_len, int kv_stride, int hd, int prec,
                  float* out) {
  const int repeat = heads / kv_heads;
  const int rows = repeat * t;
  const float scale = or_round((float)(1.0 / sqrt((double)hd)), prec);
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)(kv_len > 0 ? kv_len : 1));
    float* acc = (float*)malloc(sizeof(float) * (size_t)hd);
#pragma omp for collapse(3) schedule(dynamic, 4)
    for (int bi = 0; bi < b; ++bi)
      for (int g = 0; g < kv_heads; ++g)
        for (int row = 0; row < rows; ++row) {
          const int r = row / t, qi = row % t;
          const int h = g * repeat + r;
          const float* qv = q + (((size_t)bi * heads + h) * t + qi) * hd;
          const float* kb = k + ((size_t)bi * kv_heads + g) * (size_t)kv_stride * hd;
          const float* vb = v + ((size_t)bi * kv_heads + g) * (size_t)kv_stride * hd;
          const float* mrow = mask ? mask + ((size_t)bi * rows + row) * kv_len : NULL;
          float mx = -INFINITY;
          for (int j = 0; j < kv_len; ++j) {
            float s = or_round(or_round(dotf(qv, kb + (size_t)j * hd, hd), prec) * scale, prec);
            if (mrow) s = or_round(s + mrow[j], prec);
            sc[j] = s;
            if (s > mx) mx = s;
          }
          float sum = 0.0f;
          for (int j = 0; j < kv_len; ++j) {
            float e = (sc[j] == -INFINITY) ? 0.0f : expf(sc[j] - mx);
            sc[j] = e;
            sum += e;
          }
          for (int d = 0; d < hd; ++d) acc[d] = 0.0f;
          for (int j = 0; j < kv_len; ++j) {
            float p = or_round(sc[j] / sum, prec);
            if (p == 0.0f) continue;
            const float* vr = vb + (size_t)j * hd;
            for (int d = 0; d < hd; ++d) acc[d] += p * vr[d];
          }
          float* o = out + (((size_t)bi * t + qi) * heads + h) * hd;
          for (int d = 0; d < hd; ++d) o[d] = or_round(acc[d], prec);
        }
    free(sc);
    free(acc);
  }
}

/* ------------------------------------------------------------------------ */
/* Model                                                                    */
/* ------------------------------------------------------------------------ */

typedef struct or_linear {
  int out, in;
  float* w;      /* dense (out, in), dtype-rounded; NULL when quantised */
  uint8_t* q;    /* Q8_0 blocks; NULL when dense */
} or_linear;

typedef struct or_layer {
  or_linear qkv, o, gate_up, down;
  float *in_norm, *post_norm, *q_norm, *k_norm;
  uint32_t set_mask;
} or_layer;

struct or_model {
  or_cfg cfg;
  int prec, max_len;
  or_layer* layers;
  float* embed;
  float* norm;
  or_linear lm_head;
  int embed_set, norm_set, lm_head_set;
  float *cos, *sin;
  float* embed_f32_src; /* kept only for the int8 tied head */
};

struct or_kv {
  int batch, cap, len, layers, kvh, hd;
  float** k;
  float** v;
};

static int is_quant(const or_model* m) { return m->prec == OR_INT8; }

static void lin_alloc(const or_model* m, or_linear* l, int out, int in) {
  l->out = out;
  l->in = in;
  if (is_quant(m)) {
    l->q = (uint8_t*)calloc((size_t)out * (in / 32) * 34, 1);
    l->w = NULL;
  } else {
    l->w = (float*)calloc((size_t)out * in, sizeof(float));
    l->q = NULL;
  }
}

static void lin_free(or_linear* l) {
  free(l->w);
  free(l->q);
}

/* Store rows [row0, row0+rows) of a (possibly fused) linear from an f32
 * source.  Fused weights are cat'ed along the out axis before quantising
 * (linear.rs:239-251); Q8_0 blocks run along the input axis, so quantising
 * each part into its row range is the same operation. */
static void lin_set_rows(const or_model* m, or_linear* l, int row0, int rows, const float* src) {
  if (is_quant(m)) {
    or_quantize_q8_0(src, rows, l->in, l->q + (size_t)row0 * (l->in / 32) * 34);
  } else {
    float* dst = l->w + (size_t)row0 * l->in;
    for (int64_t i = 0; i < (int64_t)rows * l->in; ++i) dst[i] = or_round(src[i], m->prec);
  }
}

static void lin_forward(const or_model* m, const or_linear* l, const float* x, int64_t rows,
                        float* y) {
  if (l->q)
    or_linear_q8_0(x, l->q, rows, l->in, l->out, m->prec, y);
  else
    or_linear_dense(x, l->w, rows, l->in, l->out, m->prec, y);
}

or_model* or_model_new(const or_cfg* cfg, int prec, int max_len) {
  if (cfg->num_attention_heads % cfg->num_key_value_heads || cfg->head_dim % 2 ||
      (prec == OR_INT8 && (cfg->hidden_size % 32 || cfg->intermediate_size % 32 ||
                           (cfg->num_attention_heads * cfg->head_dim) % 32))) {
    set_err("invalid config");
    return NULL;
  }
  if (cfg->attention_bias) {
    set_err("attention_bias is not supported");
    return NULL;
  }
  or_model* m = (or_model*)calloc(1, sizeof(or_model));
  m->cfg = *cfg;
  m->prec = prec;
  m->max_len = max_len;
  const int H = cfg->hidden_size, I = cfg->intermediate_size, hd = cfg->head_dim;
  const int qd = cfg->num_attention_heads * hd, kd = cfg->num_key_value_heads * hd;
  m->layers = (or_layer*)calloc((size_t)cfg->num_hidden_layers, sizeof(or_layer));
  for (int i = 0; i < cfg->num_hidden_layers; ++i) {
    or_layer* L = &m->layers[i];
    lin_alloc(m, &L->qkv, qd + 2 * kd, H);
    lin_alloc(m, &L->o, H, qd);
    lin_alloc(m, &L->gate_up, 2 * I, H);
    lin_alloc(m, &L->down, H, I);
    L->in_norm = (float*)calloc((size_t)H, sizeof(float));
    L->post_norm = (float*)calloc((size_t)H, sizeof(float));
    L->q_norm = (float*)calloc((size_t)hd, sizeof(float));
    L->k_norm = (float*)calloc((size_t)hd, sizeof(float));
  }
  m->embed = (float*)calloc((size_t)cfg->vocab_size * H, sizeof(float));
  m->norm = (float*)calloc((size_t)H, sizeof(float));
  lin_alloc(m, &m->lm_head, cfg->vocab_size, H);
  m->cos = (float*)malloc(sizeof(float) * (size_t)max_len * (hd / 2));
  m->sin = (float*)malloc(sizeof(float) * (size_t)max_len * (hd / 2));
  or_rope_tables(hd, cfg->rope_theta, max_len, prec, m->cos, m->sin);
  return m;
}

void or_model_free(or_model* m) {
  if (!m) return;
  for (int i = 0; i < m->cfg.num_hidden_layers; ++i) {
    or_layer* L = &m->layers[i];
    lin_free(&L->qkv);
    lin_free(&L->o);
    lin_free(&L->gate_up);
    lin_free(&L->down);
    free(L->in_norm);
    free(L->post_norm);
    free(L->q_norm);
    free(L->k_norm);
  }
  free(m->layers);
  free(m->embed);
  free(m->norm);
  lin_free(&m->lm_head);
  free(m->cos);
  free(m->sin);
  free(m);
}

static void vec_set(const or_model* m, float* dst, const float* src, int n) {
  for (int i = 0; i < n; ++i) dst[i] = or_round(src[i], m->prec);
}

/* Name map of Qwen3::load / Attention::load / Mlp::load / Layer::load
 * (qwen3.rs:177-200, 268-286, 303-320, 354-390). */
int or_model_set(or_model* m, const char* name, const float* data) {
  const char* pfx = "model.language_model.";
  if (strncmp(name, pfx, strlen(pfx)) == 0) name += strlen(pfx);
  const or_cfg* c = &m->cfg;
  const int H = c->hidden_size, I = c->intermediate_size, hd = c->head_dim;
  const int qd = c->num_attention_heads * hd, kd = c->num_key_value_heads * hd;
  if (strcmp(name, "embed_tokens.weight") == 0) {
    vec_set(m, m->embed, data, c->vocab_size * H);
    m->embed_set = 1;
    if (!m->lm_head_set) lin_set_rows(m, &m->lm_head, 0, c->vocab_size, data); /* tied */
    return 0;
  }
  if (strcmp(name, "lm_head.weight") == 0) {
    lin_set_rows(m, &m->lm_head, 0, c->vocab_size, data);
    m->lm_head_set = 1;
    return 0;
  }
  if (strcmp(name, "norm.weight") == 0) {
    vec_set(m, m->norm, data, H);
    m->norm_set = 1;
    return 0;
  }
  int li = -1, used = 0;
  if (sscanf(name, "layers.%d.%n", &li, &used) == 1 && li >= 0 && li < c->num_hidden_layers) {
    or_layer* L = &m->layers[li];
    const char* rest = name + used;
    struct { const char* n; int bit; } tab[] = {
        {"self_attn.q_proj.weight", 0}, {"self_attn.k_proj.weight", 1},
        {"self_attn.v_proj.weight", 2}, {"self_attn.o_proj.weight", 3},
        {"mlp.gate_proj.weight", 4},    {"mlp.up_proj.weight", 5},
        {"mlp.down_proj.weight", 6},    {"input_layernorm.weight", 7},
        {"post_attention_layernorm.weight", 8}, {"self_attn.q_norm.weight", 9},
        {"self_attn.k_norm.weight", 10}};
    for (size_t t = 0; t < sizeof tab / sizeof tab[0]; ++t) {
      if (strcmp(rest, tab[t].n) != 0) continue;
      switch (tab[t].bit) {
        case 0: lin_set_rows(m, &L->qkv, 0, qd, data); break;
        case 1: lin_set_rows(m, &L->qkv, qd, kd, data); break;
        case 2: lin_set_rows(m, &L->qkv, qd + kd, kd, data); break;
        case 3: lin_set_rows(m, &L->o, 0, H, data); break;
        case 4: lin_set_rows(m, &L->gate_up, 0, I, data); break;
        case 5: lin_set_rows(m, &L->gate_up, I, I, data); break;
        case 6: lin_set_rows(m, &L->down, 0, H, data); break;
        case 7: vec_set(m, L->in_norm, data, H); break;
        case 8: vec_set(m, L->post_norm, data, H); break;
        case 9: vec_set(m, L->q_norm, data, hd); break;
        case 10: vec_set(m, L->k_norm, data, hd); break;
      }
      L->set_mask |= 1u << tab[t].bit;
      return 0;
    }
  }
  char buf[300];
  snprintf(buf, sizeof buf, "unknown tensor name %s", name);
  set_err(buf);
  return -1;
}

static void fill_normal(float* dst, int64_t n, uint64_t seed, float mean, float std) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i)
    dst[i] = mean + std * approx_normal(seed * 0x632be59bd9b4e019ull + (uint64_t)i);
}

/* Synthetic checkpoint generated in place (for the CPU baseline): linears
 * and embedding N(0, std^2), norm gains 1 + N(0, std^2), tied lm_head. */
int or_model_fill_random(or_model* m, uint64_t seed, float std) {
  const or_cfg* c = &m->cfg;
  const int H = c->hidden_size, I = c->intermediate_size, hd = c->head_dim;
  const int qd = c->num_attention_heads * hd, kd = c->num_key_value_heads * hd;
  size_t maxn = (size_t)c->vocab_size * H;
  if ((size_t)2 * I * H > maxn) maxn = (size_t)2 * I * H;
  if ((size_t)(qd + 2 * kd) * H > maxn) maxn = (size_t)(qd + 2 * kd) * H;
  float* buf = (float*)malloc(sizeof(float) * maxn);
  if (!buf) {
    set_err("allocation failed");
    return -1;
  }
  uint64_t k = seed * 1000003ull;
  for (int li = 0; li < c->num_hidden_layers; ++li) {
    or_layer* L = &m->layers[li];
    fill_normal(buf, (int64_t)(qd + 2 * kd) * H, ++k, 0.f, std);
    lin_set_rows(m, &L->qkv, 0, qd + 2 * kd, buf);
    fill_normal(buf, (int64_t)H * qd, ++k, 0.f, std);
    lin_set_rows(m, &L->o, 0, H, buf);
    fill_normal(buf, (int64_t)2 * I * H, ++k, 0.f, std);
    lin_set_rows(m, &L->gate_up, 0, 2 * I, buf);
    fill_normal(buf, (int64_t)H * I, ++k, 0.f, std);
    lin_set_rows(m, &L->down, 0, H, buf);
    fill_normal(buf, H, ++k, 1.f, std);
    vec_set(m, L->in_norm, buf, H);
    fill_normal(buf, H, ++k, 1.f, std);
    vec_set(m, L->post_norm, buf, H);
    fill_normal(buf, hd, ++k, 1.f, std);
    vec_set(m, L->q_norm, buf, hd);
    fill_normal(buf, hd, ++k, 1.f, std);
    vec_set(m, L->k_norm, buf, hd);
    L->set_mask = 0x7ffu;
  }
  fill_normal(buf, (int64_t)c->vocab_size * H, ++k, 0.f, std);
  vec_set(m, m->embed, buf, c->vocab_size * H);
  lin_set_rows(m, &m->lm_head, 0, c->vocab_size, buf);
  fill_normal(buf, H, ++k, 1.f, std);
  vec_set(m, m->norm, buf, H);
  m->embed_set = m->norm_set = 1;
  free(buf);
  return 0;
}

int or_model_ready(const or_model* m) {
  for (int i = 0; i < m->cfg.num_hidden_layers; ++i)
    if (m->layers[i].set_mask != 0x7ffu) return 0;
  return m->embed_set && m->norm_set;
}

or_kv* or_kv_new(const or_model* m, int batch, int capacity) {
  or_kv* kv = (or_kv*)calloc(1, sizeof(or_kv));
  kv->batch = batch;
  kv->cap = capacity;
  kv->layers = m->cfg.num_hidden_layers;
  kv->kvh = m->cfg.num_key_value_heads;
  kv->hd = m->cfg.head_dim;
  kv->k = (float**)calloc((size_t)kv->layers, sizeof(float*));
  kv->v = (float**)calloc((size_t)kv->layers, sizeof(float*));
  size_t n = (size_t)batch * kv->kvh * capacity * kv->hd;
  for (int l = 0; l < kv->layers; ++l) {
    kv->k[l] = (float*)calloc(n, sizeof(float));
    kv->v[l] = (float*)calloc(n, sizeof(float));
    if (!kv->k[l] || !kv->v[l]) {
      set_err("kv allocation failed");
      or_kv_free(kv);
      return NULL;
    }
  }
  return kv;
}

void or_kv_free(or_kv* kv) {
  if (!kv) return;
  for (int l = 0; l < kv->layers; ++l) {
    free(kv->k[l]);
    free(kv->v[l]);
  }
  free(kv->k);
  free(kv->v);
  free(kv);
}

int or_kv_len(const or_kv* kv) { return kv->len; }

int or_kv_read(const or_kv* kv, int layer, int which, float* out) {
  if (layer < 0 || layer >= kv->layers) return -1;
  size_t n = (size_t)kv->batch * kv->kvh * kv->cap * kv->hd;
  memcpy(out, which ? kv->v[layer] : kv->k[layer], n * sizeof(float));
  return 0;
}

int or_kv_write(or_kv* kv, int layer, int which, const float* src) {
  if (layer < 0 || layer >= kv->layers) return -1;
  size_t n = (size_t)kv->batch * kv->kvh * kv->cap * kv->hd;
  memcpy(which ? kv->v[layer] : kv->k[layer], src, n * sizeof(float));
  return 0;
}

/* Synthetic context for the CPU baseline: approximately N(0,1) K/V (rounded to
 * the dtype) at positions [0, len) of every row, zeros elsewhere. */
int or_kv_fill_random(or_kv* kv, uint64_t seed, int len, int prec) {
  if (len < 0 || len > kv->cap) return -1;
  const int64_t rows = (int64_t)kv->batch * kv->kvh;
  for (int l = 0; l < kv->layers; ++l)
    for (int which = 0; which < 2; ++which) {
      float* dst = which ? kv->v[l] : kv->k[l];
      const uint64_t base = seed * 0x632be59bd9b4e019ull + (uint64_t)(2 * l + which) * 0x9e3779b97f4a7c15ull;
#pragma omp parallel for schedule(static)
      for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = (int64_t)r * kv->cap * kv->hd; i < ((int64_t)r * kv->cap + len) * kv->hd; ++i)
          dst[i] = or_round(approx_normal(base + (uint64_t)i), prec);
    }
  kv->len = len;
  return 0;
}

int or_kv_set_len(or_kv* kv, int len) {
  if (len < 0 || len > kv->cap) return -1;
  kv->len = len;
  return 0;
}

/* Qwen3::embed (qwen3.rs:405-412). */
void or_embed(const or_model* m, const uint32_t* ids, int64_t n, float* out) {
  const int H = m->cfg.hidden_size;
  for (int64_t i = 0; i < n; ++i)
    memcpy(out + i * H, m->embed + (size_t)ids[i] * H, sizeof(float) * (size_t)H);
}

/* Rope::apply (qwen3.rs:139-144) -> candle rope (rotate-half): for the i-th
 * pair (x[i], x[i+hd/2]) at position p: (x1 c - x2 s, x2 c + x1 s).
 * x (b, heads, t, hd) in place; tables (max_len, hd/2). */
void or_rope_apply(float* x, int b, int heads, int t, int hd, int offset, const float* cos_t,
                   const float* sin_t, int prec) {
  const int half = hd / 2;
  for (int bi = 0; bi < b; ++bi)
    for (int h = 0; h < heads; ++h)
      for (int ti = 0; ti < t; ++ti) {
        float* v = x + (((size_t)bi * heads + h) * t + ti) * hd;
        const float* c = cos_t + (size_t)(offset + ti) * half;
        const float* s = sin_t + (size_t)(offset + ti) * half;
        for (int i = 0; i < half; ++i) {
          float x1 = v[i], x2 = v[i + half];
          v[i] = or_round(x1 * c[i] - x2 * s[i], prec);
          v[i + half] = or_round(x2 * c[i] + x1 * s[i], prec);
        }
      }
}

static void rope_rows(const or_model* m, float* x, int b, int heads, int t, int offset) {
  or_rope_apply(x, b, heads, t, m->cfg.head_dim, offset, m->cos, m->sin, m->prec);
}

/* Layer::forward (qwen3.rs:322-339) with Attention::forward (203-259) and
 * Mlp::forward (288-292).  xs: (b, t, H) in/out. */
static int layer_forward(or_model* m, int li, or_kv* kv, float* xs, int b, int t, int offset,
                         const float* mask) {
  const or_cfg* c = &m->cfg;
  const or_layer* L = &m->layers[li];
  const int H = c->hidden_size, I = c->intermediate_size, hd = c->head_dim;
  const int nh = c->num_attention_heads, nkv = c->num_key_value_heads;
  const int qd = nh * hd, kd = nkv * hd, qkvd = qd + 2 * kd;
  const int64_t rows = (int64_t)b * t;
  const float eps = (float)c->rms_norm_eps;

  if (kv->len + t > kv->cap) {
    char buf[200];
    snprintf(buf, sizeof buf, "kv cache overflow: %d + %d exceeds capacity %d", kv->len, t,
             kv->cap);
    set_err(buf);
    return -1;
  }

  float* xn = (float*)malloc(sizeof(float) * rows * (I > H ? 2 * I : H));
  float* qkv = (float*)malloc(sizeof(float) * rows * qkvd);
  float* q = (float*)malloc(sizeof(float) * rows * qd);
  float* ctx = (float*)malloc(sizeof(float) * rows * qd);
  float* h = (float*)malloc(sizeof(float) * rows * (2 * I > H ? 2 * I : H));

  or_rmsnorm(xs, L->in_norm, rows, H, eps, m->prec, xn);
  lin_forward(m, &L->qkv, xn, rows, qkv);

  /* split, per-head q/k norm on (b,t,heads,hd), transpose to (b,heads,t,hd) */
  float* kt = (float*)malloc(sizeof(float) * rows * kd);
  float* vt = (float*)malloc(sizeof(float) * rows * kd);
  for (int bi = 0; bi < b; ++bi)
    for (int ti = 0; ti < t; ++ti) {
      const float* row = qkv + ((size_t)bi * t + ti) * qkvd;
      for (int hh = 0; hh < nh; ++hh)
        or_rmsnorm(row + hh * hd, L->q_norm, 1, hd, eps, m->prec,
                   q + (((size_t)bi * nh + hh) * t + ti) * hd);
      for (int hh = 0; hh < nkv; ++hh) {
        or_rmsnorm(row + qd + hh * hd, L->k_norm, 1, hd, eps, m->prec,
                   kt + (((size_t)bi * nkv + hh) * t + ti) * hd);
        memcpy(vt + (((size_t)bi * nkv + hh) * t + ti) * hd, row + qd + kd + hh * hd,
               sizeof(float) * hd);
      }
    }
  rope_rows(m, q, b, nh, t, offset);
  rope_rows(m, kt, b, nkv, t, offset);

  /* KvCache::append (qwen3.rs:86-101): write t rows at [len, len+t). */
  float* K = kv->k[li];
  float* V = kv->v[li];
  for (int bi = 0; bi < b; ++bi)
    for (int hh = 0; hh < nkv; ++hh)
      for (int ti = 0; ti < t; ++ti) {
        size_t dst = (((size_t)bi * nkv + hh) * kv->cap + kv->len + ti) * hd;
        size_t src = (((size_t)bi * nkv + hh) * t + ti) * hd;
        memcpy(K + dst, kt + src, sizeof(float) * hd);
        memcpy(V + dst, vt + src, sizeof(float) * hd);
      }
  const int kv_len = kv->len + t;

  or_attention(q, K, V, mask, b, nh, nkv, t, kv_len, kv->cap, hd, m->prec, ctx);
  lin_forward(m, &L->o, ctx, rows, h);
  for (int64_t i = 0; i < rows * H; ++i) xs[i] = or_round(xs[i] + h[i], m->prec);

  or_rmsnorm(xs, L->post_norm, rows, H, eps, m->prec, xn);
  lin_forward(m, &L->gate_up, xn, rows, h);
  /* silu(gate) * up, each op's output in the dtype (qwen3.rs:289-291) */
  for (int64_t r = 0; r < rows; ++r)
    for (int i = 0; i < I; ++i) {
      float g = h[r * 2 * I + i], u = h[r * 2 * I + I + i];
      float s = or_round(g / (1.0f + expf(-g)), m->prec);
      xn[r * I + i] = or_round(s * u, m->prec);
    }
  lin_forward(m, &L->down, xn, rows, h);
  for (int64_t i = 0; i < rows * H; ++i) xs[i] = or_round(xs[i] + h[i], m->prec);

  free(xn);
  free(qkv);
  free(q);
  free(ctx);
  free(h);
  free(kt);
  free(vt);
  return 0;
}

/* forward_embeds (qwen3.rs:444-456): 28 layers then the final norm.  The
 * cache length advances once per pass (every layer's cache has the same
 * length; the single `len` here is the reference's caches[i].len()). */
static int forward_embeds(or_model* m, or_kv* kv, float* xs, int b, int t, int offset,
                          const float* mask, float* out_norm) {
  for (int li = 0; li < m->cfg.num_hidden_layers; ++li)
    if (layer_forward(m, li, kv, xs, b, t, offset, mask)) return -1;
  kv->len += t;
  or_rmsnorm(xs, m->norm, (int64_t)b * t, m->cfg.hidden_size, (float)m->cfg.rms_norm_eps,
             m->prec, out_norm);
  return 0;
}

/* Qwen3::logits (qwen3.rs:459-463): lm_head in the dtype, then widened to f32. */
static void logits_of(const or_model* m, const float* hidden, int b, float* logits) {
  lin_forward(m, &m->lm_head, hidden, b, logits);
}

int or_prefill(or_model* m, or_kv* kv, const float* embeds, const int32_t* pad, int batch,
               int total, int block, float* logits) {
  const int H = m->cfg.hidden_size;
  const int repeat = m->cfg.num_attention_heads / m->cfg.num_key_value_heads;
  if (total <= 0) {
    set_err("empty prompt");
    return -1;
  }
  if (block <= 0) block = 256;
  float* last = (float*)malloc(sizeof(float) * (size_t)batch * H);
  int start = 0;
  while (start < total) {
    int len = block < total - start ? block : total - start;
    float* blk = (float*)malloc(sizeof(float) * (size_t)batch * len * H);
    float* nrm = (float*)malloc(sizeof(float) * (size_t)batch * len * H);
    for (int bi = 0; bi < batch; ++bi)
      memcpy(blk + (size_t)bi * len * H, embeds + ((size_t)bi * total + start) * H,
             sizeof(float) * (size_t)len * H);
    float* mask = (float*)malloc(sizeof(float) * (size_t)batch * repeat * len * (start + len));
    or_build_mask(batch, repeat, start, len, start + len, pad, mask);
    /* the mask is materialised in the dtype (qwen3.rs:561): 0 and -inf exact */
    int rc = forward_embeds(m, kv, blk, batch, len, start, mask, nrm);
    if (rc == 0)
      for (int bi = 0; bi < batch; ++bi)
        memcpy(last + (size_t)bi * H, nrm + ((size_t)bi * len + len - 1) * H,
               sizeof(float) * H);
    free(mask);
    free(blk);
    free(nrm);
    if (rc) {
      free(last);
      return -1;
    }
    start += len;
  }
  if (logits) logits_of(m, last, batch, logits);
  free(last);
  return 0;
}

int or_decode_step(or_model* m, or_kv* kv, const uint32_t* ids, const int32_t* pad, int batch,
                   float* logits) {
  const int H = m->cfg.hidden_size;
  const int repeat = m->cfg.num_attention_heads / m->cfg.num_key_value_heads;
  const int offset = kv->len;
  float* xs = (float*)malloc(sizeof(float) * (size_t)batch * H);
  float* nrm = (float*)malloc(sizeof(float) * (size_t)batch * H);
  or_embed(m, ids, batch, xs);
  float* mask = (float*)malloc(sizeof(float) * (size_t)batch * repeat * (offset + 1));
  or_build_mask(batch, repeat, offset, 1, offset + 1, pad, mask);
  int rc = forward_embeds(m, kv, xs, batch, 1, offset, mask, nrm);
  if (rc == 0 && logits) logits_of(m, nrm, batch, logits);
  free(mask);
  free(xs);
  free(nrm);
  return rc;
}

int or_layer_decode(or_model* m, or_kv* kv, int layer, float* x, const int32_t* pad, int batch) {
  if (layer < 0 || layer >= m->cfg.num_hidden_layers) {
    set_err("layer out of range");
    return -1;
  }
  const int repeat = m->cfg.num_attention_heads / m->cfg.num_key_value_heads;
  const int offset = kv->len;
  float* mask = (float*)malloc(sizeof(float) * (size_t)batch * repeat * (offset + 1));
  or_build_mask(batch, repeat, offset, 1, offset + 1, pad, mask);
  const int rc = layer_forward(m, layer, kv, x, batch, 1, offset, mask);
  free(mask);
  return rc;
}

void or_final_logits(const or_model* m, const float* x, int rows, float* logits) {
  float* nrm = (float*)malloc(sizeof(float) * (size_t)rows * m->cfg.hidden_size);
  or_rmsnorm(x, m->norm, rows, m->cfg.hidden_size, (float)m->cfg.rms_norm_eps, m->prec, nrm);
  logits_of(m, nrm, rows, logits);
  free(nrm);
}

void or_argmax_rows(const float* logits, int rows, int vocab, uint32_t* out) {
  for (int r = 0; r < rows; ++r) {
    const float* l = logits + (size_t)r * vocab;
    int best = 0;
    for (int i = 1; i < vocab; ++i)
      if (l[i] > l[best]) best = i;
    out[r] = (uint32_t)best;
  }
}

int or_generate(or_model* m, const float* embeds, const int32_t* pad, int batch, int total,
                int block, int budget, uint32_t eos, const int32_t* force_eot_step,
                uint32_t* tokens, int32_t* ntok, int32_t* finish) {
  const int V = m->cfg.vocab_size;
  or_kv* kv = or_kv_new(m, batch, total + budget);
  if (!kv) return -1;
  float* logits = (float*)malloc(sizeof(float) * (size_t)batch * V);
  uint32_t* next = (uint32_t*)malloc(sizeof(uint32_t) * batch);
  int* done = (int*)calloc((size_t)batch, sizeof(int));
  int rc = or_prefill(m, kv, embeds, pad, batch, total, block, logits);
  for (int bi = 0; bi < batch; ++bi) {
    ntok[bi] = 0;
    finish[bi] = 0;
  }
  for (int step = 0; rc == 0 && step < budget; ++step) {
    or_argmax_rows(logits, batch, V, next);
    int all_done = 1;
    for (int bi = 0; bi < batch; ++bi) {
      if (done[bi]) continue;
      uint32_t tok = next[bi];
      if (force_eot_step && force_eot_step[bi] == step) tok = eos;
      if (tok == eos) {
        done[bi] = 1;
        finish[bi] = 1;
      } else {
        tokens[(size_t)bi * budget + ntok[bi]++] = tok;
        all_done = 0;
      }
    }
    if (all_done || step + 1 == budget) break;
    for (int bi = 0; bi < batch; ++bi)
      if (done[bi]) next[bi] = eos;
    rc = or_decode_step(m, kv, next, pad, batch, logits);
  }
  free(done);
  free(next);
  free(logits);
  or_kv_free(kv);
  return rc;
}
