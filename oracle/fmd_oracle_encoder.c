/*
 * fmd_oracle_encoder.c -- CPU restatement of the audio path of
 * cnmoro/fast-moss-diarization: the Whisper encoder
 * (crates/fmd-core/src/model/whisper_encoder.rs), the VqAdaptor
 * (model/adaptor.rs) and the chunk reassembly of MossModel::encode_audio
 * (model/mod.rs:82-126).  TEST INFRASTRUCTURE ONLY (the checker): tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; the
 * product library never does.
 *
 * Rounding model, as for the decoder: every tensor the reference keeps is in
 * the activation dtype (the dense VarBuilder view, linear.rs:119-141, and
 * the mel cast, engine.rs:334-339), so each op's output is rounded to that
 * dtype here; inside one op the arithmetic is f32.  Where candle's op order is
 * not visible from the reference (conv1d's summation order, layer_norm's
 * variance formula, gelu_erf's evaluation), the choice is stated at the
 * function and is tolerance-governed.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "fmd_oracle.h"

static __thread char g_enc_err[256];
static int enc_fail(const char* msg) {
  snprintf(g_enc_err, sizeof g_enc_err, "%s", msg);
  return -1;
}
const char* or_enc_last_error(void) { return g_enc_err; }

/* ------------------------------------------------------------------------ */
/* Single ops                                                               */
/* ------------------------------------------------------------------------ */

/* Tensor::conv1d(kernel, padding = 1, stride, dilation 1, groups 1)
 * (whisper_encoder.rs:142-152): x (b, cin, t), w (cout, cin, 3) ->
 * out (b, cout, tout), tout = (t + 2 - 3) / stride + 1, rounded to prec.
 * Each output sums w[o][c][k] * x[c][t*stride + k - 1] over (c, k) in f32,
 * channels outermost; taps outside [0, t) read zero. */
void or_conv1d(const float* x, const float* w, int b, int cin, int cout, int t, int stride,
               int prec, float* out) {
  const int tout = (t + 2 - 3) / stride + 1;
#pragma omp parallel for collapse(2) schedule(static)
  for (int bi = 0; bi < b; ++bi)
    for (int o = 0; o < cout; ++o) {
      float* orow = out + ((size_t)bi * cout + o) * tout;
      for (int j = 0; j < tout; ++j) orow[j] = 0.0f;
      for (int c = 0; c < cin; ++c) {
        const float* xr = x + ((size_t)bi * cin + c) * t;
        const float* wr = w + ((size_t)o * cin + c) * 3;
        for (int j = 0; j < tout; ++j) {
          float s = orow[j];
          for (int k = 0; k < 3; ++k) {
            const int src = j * stride + k - 1;
            if (src >= 0 && src < t) s += wr[k] * xr[src];
          }
          orow[j] = s;
        }
      }
      for (int j = 0; j < tout; ++j) orow[j] = or_round(orow[j], prec);
    }
}

/* Tensor::gelu_erf (whisper_encoder.rs:144, 149, 97): 0.5 x (1 + erf(x / sqrt 2))
 * evaluated in f32 (erff), rounded to prec. */
void or_gelu_erf(float* x, int64_t n, int prec) {
#pragma omp parallel for schedule(static) if (n > 65536)
  for (int64_t i = 0; i < n; ++i) {
    const float v = x[i];
    x[i] = or_round(0.5f * v * (1.0f + erff(v * 0.70710678118654752f)), prec);
  }
}

/* candle_nn::ops::silu (adaptor.rs:58): x / (1 + exp(-x)) in f32, rounded. */
void or_silu(float* x, int64_t n, int prec) {
  for (int64_t i = 0; i < n; ++i) x[i] = or_round(x[i] / (1.0f + expf(-x[i])), prec);
}

/* LayerNorm::forward (linear.rs:323-330) -> candle_nn::ops::layer_norm, f32
 * accumulation: mean = sum(x)/n, var = sum((x - mean)^2)/n (two passes),
 * y = (x - mean) * (1/sqrt(var + eps)) * w + b, rounded to prec. */
void or_layernorm(const float* x, const float* w, const float* bias, int64_t rows, int dim,
                  float eps, int prec, float* y) {
#pragma omp parallel for schedule(static) if (rows > 16)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * dim;
    float s = 0.0f;
    for (int i = 0; i < dim; ++i) s += xr[i];
    const float mean = s / (float)dim;
    float ss = 0.0f;
    for (int i = 0; i < dim; ++i) {
      const float dlt = xr[i] - mean;
      ss += dlt * dlt;
    }
    const float rinv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = 0; i < dim; ++i)
      y[r * dim + i] = or_round((xr[i] - mean) * rinv * w[i] + bias[i], prec);
  }
}

/* rd(y + b) per row: Tensor::broadcast_add of a bias in the dtype
 * (linear.rs:41-44). */
static void add_bias(float* y, const float* b, int64_t rows, int out, int prec) {
#pragma omp parallel for schedule(static) if (rows > 64)
  for (int64_t r = 0; r < rows; ++r)
    for (int i = 0; i < out; ++i) y[r * out + i] = or_round(y[r * out + i] + b[i], prec);
}

/* Dense attention without mask (whisper_encoder.rs:44-64) for one window:
 * q, k, v (t, heads*hd) row-major as projected (q and k already scaled);
 * scores = rd(q.k) (the matmul of two dtype tensors), probs = rd(softmax)
 * (softmax_last_dim: max-subtracted exp and sum in f32), ctx = rd(probs . v),
 * out (t, heads*hd). */
void or_attention_dense(const float* q, const float* k, const float* v, int t, int heads, int hd,
                        int prec, float* out) {
  const int d = heads * hd;
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)t);
    float* acc = (float*)malloc(sizeof(float) * (size_t)hd);
#pragma omp for collapse(2) schedule(dynamic, 8)
    for (int h = 0; h < heads; ++h)
      for (int i = 0; i < t; ++i) {
        const float* qv = q + (size_t)i * d + h * hd;
        float mx = -INFINITY;
        for (int j = 0; j < t; ++j) {
          const float* kv = k + (size_t)j * d + h * hd;
          float s = 0.0f;
          for (int e = 0; e < hd; ++e) s += qv[e] * kv[e];
          s = or_round(s, prec);
          sc[j] = s;
          if (s > mx) mx = s;
        }
        float sum = 0.0f;
        for (int j = 0; j < t; ++j) {
          sc[j] = expf(sc[j] - mx);
          sum += sc[j];
        }
        for (int e = 0; e < hd; ++e) acc[e] = 0.0f;
        for (int j = 0; j < t; ++j) {
          const float p = or_round(sc[j] / sum, prec);
          const float* vr = v + (size_t)j * d + h * hd;
          for (int e = 0; e < hd; ++e) acc[e] += p * vr[e];
        }
        float* o = out + (size_t)i * d + h * hd;
        for (int e = 0; e < hd; ++e) o[e] = or_round(acc[e], prec);
      }
    free(sc);
    free(acc);
  }
}

/* ------------------------------------------------------------------------ */
/* Encoder + adaptor model                                                  */
/* ------------------------------------------------------------------------ */

typedef struct or_enc_layer {
  float *q_w, *q_b, *k_w, *v_w, *v_b, *o_w, *o_b;
  float *ln1_w, *ln1_b, *fc1_w, *fc1_b, *fc2_w, *fc2_b, *ln2_w, *ln2_b;
  uint32_t set;
} or_enc_layer;

struct or_enc {
  or_audio_cfg cfg;
  int prec;
  float *conv1_w, *conv1_b, *conv2_w, *conv2_b, *pos, *ln_w, *ln_b;
  float *a_fc1_w, *a_fc1_b, *a_fc2_w, *a_fc2_b, *a_ln_w, *a_ln_b;
  uint32_t set;
  or_enc_layer* layers;
};

static float* zalloc(size_t n) { return (float*)calloc(n ? n : 1, sizeof(float)); }

or_enc* or_enc_new(const or_audio_cfg* cfg, int prec) {
  if (cfg->d_model <= 0 || cfg->encoder_attention_heads <= 0 ||
      cfg->d_model % cfg->encoder_attention_heads || cfg->audio_merge_size <= 0 ||
      cfg->adaptor_input_dim != cfg->d_model * cfg->audio_merge_size) {
    enc_fail("invalid audio config");
    return NULL;
  }
  or_enc* e = (or_enc*)calloc(1, sizeof(or_enc));
  e->cfg = *cfg;
  e->prec = prec;
  const size_t d = (size_t)cfg->d_model, f = (size_t)cfg->encoder_ffn_dim;
  const size_t m = (size_t)cfg->num_mel_bins, H = (size_t)cfg->hidden_size;
  e->conv1_w = zalloc(d * m * 3);
  e->conv1_b = zalloc(d);
  e->conv2_w = zalloc(d * d * 3);
  e->conv2_b = zalloc(d);
  e->pos = zalloc((size_t)cfg->max_source_positions * d);
  e->ln_w = zalloc(d);
  e->ln_b = zalloc(d);
  e->a_fc1_w = zalloc(H * (size_t)cfg->adaptor_input_dim);
  e->a_fc1_b = zalloc(H);
  e->a_fc2_w = zalloc(H * H);
  e->a_fc2_b = zalloc(H);
  e->a_ln_w = zalloc(H);
  e->a_ln_b = zalloc(H);
  e->layers = (or_enc_layer*)calloc((size_t)cfg->encoder_layers, sizeof(or_enc_layer));
  for (int i = 0; i < cfg->encoder_layers; ++i) {
    or_enc_layer* L = &e->layers[i];
    L->q_w = zalloc(d * d);
    L->q_b = zalloc(d);
    L->k_w = zalloc(d * d);
    L->v_w = zalloc(d * d);
    L->v_b = zalloc(d);
    L->o_w = zalloc(d * d);
    L->o_b = zalloc(d);
    L->ln1_w = zalloc(d);
    L->ln1_b = zalloc(d);
    L->fc1_w = zalloc(f * d);
    L->fc1_b = zalloc(f);
    L->fc2_w = zalloc(d * f);
    L->fc2_b = zalloc(d);
    L->ln2_w = zalloc(d);
    L->ln2_b = zalloc(d);
  }
  return e;
}

void or_enc_free(or_enc* e) {
  if (!e) return;
  for (int i = 0; i < e->cfg.encoder_layers; ++i) {
    or_enc_layer* L = &e->layers[i];
    float* ps[] = {L->q_w, L->q_b, L->k_w, L->v_w, L->v_b, L->o_w, L->o_b, L->ln1_w,
                   L->ln1_b, L->fc1_w, L->fc1_b, L->fc2_w, L->fc2_b, L->ln2_w, L->ln2_b};
    for (size_t j = 0; j < sizeof ps / sizeof ps[0]; ++j) free(ps[j]);
  }
  free(e->layers);
  float* ps[] = {e->conv1_w, e->conv1_b, e->conv2_w, e->conv2_b, e->pos, e->ln_w, e->ln_b,
                 e->a_fc1_w, e->a_fc1_b, e->a_fc2_w, e->a_fc2_b, e->a_ln_w, e->a_ln_b};
  for (size_t j = 0; j < sizeof ps / sizeof ps[0]; ++j) free(ps[j]);
  free(e);
}

static void put(const or_enc* e, float* dst, const float* src, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = or_round(src[i], e->prec);
}

/* Checkpoint names of WhisperEncoder::load (whisper_encoder.rs:118-138,
 * 27-42, 73-80) under "model.whisper_encoder." and VqAdaptor::load
 * (adaptor.rs:18-35) under "model.vq_adaptor.".  Everything is dense in the
 * activation dtype (linear_dense, also in int8). */
int or_enc_set(or_enc* e, const char* name, const float* data) {
  const or_audio_cfg* c = &e->cfg;
  const size_t d = (size_t)c->d_model, f = (size_t)c->encoder_ffn_dim;
  const size_t H = (size_t)c->hidden_size;
  const char* ep = "model.whisper_encoder.";
  const char* ap = "model.vq_adaptor.";
  if (strncmp(name, ap, strlen(ap)) == 0) {
    const char* n = name + strlen(ap);
    struct { const char* n; float* p; size_t len; int bit; } tab[] = {
        {"layers.0.weight", e->a_fc1_w, H * (size_t)c->adaptor_input_dim, 0},
        {"layers.0.bias", e->a_fc1_b, H, 1},
        {"layers.2.weight", e->a_fc2_w, H * H, 2},
        {"layers.2.bias", e->a_fc2_b, H, 3},
        {"layers.3.weight", e->a_ln_w, H, 4},
        {"layers.3.bias", e->a_ln_b, H, 5}};
    for (size_t i = 0; i < sizeof tab / sizeof tab[0]; ++i)
      if (strcmp(n, tab[i].n) == 0) {
        put(e, tab[i].p, data, tab[i].len);
        e->set |= 1u << (8 + tab[i].bit);
        return 0;
      }
    return enc_fail("unknown adaptor tensor");
  }
  if (strncmp(name, ep, strlen(ep)) != 0) return enc_fail("unknown tensor");
  const char* n = name + strlen(ep);
  struct { const char* n; float* p; size_t len; int bit; } top[] = {
      {"conv1.weight", e->conv1_w, d * (size_t)c->num_mel_bins * 3, 0},
      {"conv1.bias", e->conv1_b, d, 1},
      {"conv2.weight", e->conv2_w, d * d * 3, 2},
      {"conv2.bias", e->conv2_b, d, 3},
      {"embed_positions.weight", e->pos, (size_t)c->max_source_positions * d, 4},
      {"layer_norm.weight", e->ln_w, d, 5},
      {"layer_norm.bias", e->ln_b, d, 6}};
  for (size_t i = 0; i < sizeof top / sizeof top[0]; ++i)
    if (strcmp(n, top[i].n) == 0) {
      put(e, top[i].p, data, top[i].len);
      e->set |= 1u << top[i].bit;
      return 0;
    }
  int li = -1, used = 0;
  if (sscanf(n, "layers.%d.%n", &li, &used) != 1 || li < 0 || li >= c->encoder_layers || !used)
    return enc_fail("unknown encoder tensor");
  or_enc_layer* L = &e->layers[li];
  const char* rest = n + used;
  struct { const char* n; float* p; size_t len; } lt[] = {
      {"self_attn.q_proj.weight", L->q_w, d * d}, {"self_attn.q_proj.bias", L->q_b, d},
      {"self_attn.k_proj.weight", L->k_w, d * d}, {"self_attn.v_proj.weight", L->v_w, d * d},
      {"self_attn.v_proj.bias", L->v_b, d},       {"self_attn.out_proj.weight", L->o_w, d * d},
      {"self_attn.out_proj.bias", L->o_b, d},     {"self_attn_layer_norm.weight", L->ln1_w, d},
      {"self_attn_layer_norm.bias", L->ln1_b, d}, {"fc1.weight", L->fc1_w, f * d},
      {"fc1.bias", L->fc1_b, f},                  {"fc2.weight", L->fc2_w, d * f},
      {"fc2.bias", L->fc2_b, d},                  {"final_layer_norm.weight", L->ln2_w, d},
      {"final_layer_norm.bias", L->ln2_b, d}};
  for (size_t i = 0; i < sizeof lt / sizeof lt[0]; ++i)
    if (strcmp(rest, lt[i].n) == 0) {
      put(e, lt[i].p, data, lt[i].len);
      L->set |= 1u << i;
      return 0;
    }
  return enc_fail("unknown encoder layer tensor");
}

int or_enc_ready(const or_enc* e) {
  if ((e->set & 0x7fu) != 0x7fu || ((e->set >> 8) & 0x3fu) != 0x3fu) return 0;
  for (int i = 0; i < e->cfg.encoder_layers; ++i)
    if (e->layers[i].set != 0x7fffu) return 0;
  return 1;
}

/* EncoderLayer::forward (whisper_encoder.rs:82-97) on rows x (rows, d) in
 * place, `t` rows per window (attention never crosses windows).  Attention
 * (44-64): q = rd(rd(h Wq^T + bq) * rd(s)), k = rd(rd(h Wk^T) * rd(s)) with
 * s = head_dim^-1/4 (whisper_encoder.rs:41, 53-56; `Tensor * f64` scales in
 * the dtype, the multiplier rounded to it), v = rd(h Wv^T + bv). */
static void enc_layer(const or_enc* e, const or_enc_layer* L, float* x, int windows, int t) {
  const or_audio_cfg* c = &e->cfg;
  const int d = c->d_model, f = c->encoder_ffn_dim, heads = c->encoder_attention_heads;
  const int hd = d / heads, prec = e->prec;
  const int64_t rows = (int64_t)windows * t;
  const float s = or_round((float)pow((double)hd, -0.25), prec);
  float* h = zalloc((size_t)rows * d);
  float* q = zalloc((size_t)rows * d);
  float* k = zalloc((size_t)rows * d);
  float* v = zalloc((size_t)rows * d);
  float* ctx = zalloc((size_t)rows * d);
  float* y = zalloc((size_t)rows * d);
  float* ff = zalloc((size_t)rows * f);
  or_layernorm(x, L->ln1_w, L->ln1_b, rows, d, 1e-5f, prec, h);
  or_linear_dense(h, L->q_w, rows, d, d, prec, q);
  add_bias(q, L->q_b, rows, d, prec);
  or_linear_dense(h, L->k_w, rows, d, d, prec, k);
  or_linear_dense(h, L->v_w, rows, d, d, prec, v);
  add_bias(v, L->v_b, rows, d, prec);
  for (int64_t i = 0; i < rows * d; ++i) {
    q[i] = or_round(q[i] * s, prec);
    k[i] = or_round(k[i] * s, prec);
  }
  for (int w = 0; w < windows; ++w) {
    const size_t o = (size_t)w * t * d;
    or_attention_dense(q + o, k + o, v + o, t, heads, hd, prec, ctx + o);
  }
  or_linear_dense(ctx, L->o_w, rows, d, d, prec, y);
  add_bias(y, L->o_b, rows, d, prec);
  for (int64_t i = 0; i < rows * d; ++i) x[i] = or_round(x[i] + y[i], prec);
  or_layernorm(x, L->ln2_w, L->ln2_b, rows, d, 1e-5f, prec, h);
  or_linear_dense(h, L->fc1_w, rows, d, f, prec, ff);
  add_bias(ff, L->fc1_b, rows, f, prec);
  or_gelu_erf(ff, rows * f, prec);
  or_linear_dense(ff, L->fc2_w, rows, f, d, prec, y);
  add_bias(y, L->fc2_b, rows, d, prec);
  for (int64_t i = 0; i < rows * d; ++i) x[i] = or_round(x[i] + y[i], prec);
  free(h);
  free(q);
  free(k);
  free(v);
  free(ctx);
  free(y);
  free(ff);
}

int or_enc_layers(or_enc* e, float* x, int windows, int t, int first, int n, int final_norm) {
  if (first < 0 || n < 0 || first + n > e->cfg.encoder_layers) return enc_fail("bad layer range");
  for (int i = first; i < first + n; ++i) enc_layer(e, &e->layers[i], x, windows, t);
  if (final_norm) {
    const int64_t rows = (int64_t)windows * t;
    float* y = zalloc((size_t)rows * e->cfg.d_model);
    or_layernorm(x, e->ln_w, e->ln_b, rows, e->cfg.d_model, 1e-5f, e->prec, y);
    memcpy(x, y, sizeof(float) * (size_t)rows * e->cfg.d_model);
    free(y);
  }
  return 0;
}

/* The convolutional stem of WhisperEncoder::forward (whisper_encoder.rs:
 * 139-157): mel (b, n_mels, frames) -> x (b, frames/2, d): the mel rounded
 * to the dtype (engine.rs:339), conv1 (stride 1) + bias + gelu_erf, conv2
 * (stride 2) + bias + gelu_erf, transpose, + embed_positions[0, t). */
int or_enc_stem(or_enc* e, const float* mel, int b, int frames, float* x) {
  const or_audio_cfg* c = &e->cfg;
  const int d = c->d_model, m = c->num_mel_bins, prec = e->prec;
  const int t2 = (frames + 2 - 3) / 2 + 1;
  if (t2 > c->max_source_positions) return enc_fail("more frames than embed_positions rows");
  float* in = zalloc((size_t)b * m * frames);
  for (size_t i = 0; i < (size_t)b * m * frames; ++i) in[i] = or_round(mel[i], prec);
  float* h1 = zalloc((size_t)b * d * frames);
  or_conv1d(in, e->conv1_w, b, m, d, frames, 1, prec, h1);
  for (int bi = 0; bi < b; ++bi)
    for (int o = 0; o < d; ++o)
      for (int j = 0; j < frames; ++j) {
        float* p = h1 + ((size_t)bi * d + o) * frames + j;
        *p = or_round(*p + e->conv1_b[o], prec);
      }
  or_gelu_erf(h1, (int64_t)b * d * frames, prec);
  float* h2 = zalloc((size_t)b * d * t2);
  or_conv1d(h1, e->conv2_w, b, d, d, frames, 2, prec, h2);
  for (int bi = 0; bi < b; ++bi)
    for (int o = 0; o < d; ++o)
      for (int j = 0; j < t2; ++j) {
        float* p = h2 + ((size_t)bi * d + o) * t2 + j;
        *p = or_round(*p + e->conv2_b[o], prec);
      }
  or_gelu_erf(h2, (int64_t)b * d * t2, prec);
  for (int bi = 0; bi < b; ++bi)
    for (int j = 0; j < t2; ++j)
      for (int o = 0; o < d; ++o)
        x[((size_t)bi * t2 + j) * d + o] =
            or_round(h2[((size_t)bi * d + o) * t2 + j] + e->pos[(size_t)j * d + o], prec);
  free(in);
  free(h1);
  free(h2);
  return 0;
}

/* WhisperEncoder::forward (whisper_encoder.rs:139-163). */
int or_enc_forward(or_enc* e, const float* mel, int b, int frames, float* out) {
  const int t2 = (frames + 2 - 3) / 2 + 1;
  if (or_enc_stem(e, mel, b, frames, out)) return -1;
  return or_enc_layers(e, out, b, t2, 0, e->cfg.encoder_layers, 1);
}

/* VqAdaptor::merge_and_project (adaptor.rs:41-64) of one audio's frames
 * (rows, d): groups of merge_size consecutive frames concatenated (a trailing
 * partial group is dropped), then rd(fc1 + b) -> rd(silu) -> rd(fc2 + b) ->
 * LayerNorm (eps = text rms_norm_eps, mod.rs:47-53).  out (rows/merge, H). */
int or_enc_adaptor(or_enc* e, const float* frames, int rows, float* out) {
  const or_audio_cfg* c = &e->cfg;
  const int g = rows / c->audio_merge_size, in = c->adaptor_input_dim, H = c->hidden_size;
  const int prec = e->prec;
  if (g == 0) return 0;
  /* (rows, d) row-major: group i is rows [merge*i, merge*(i+1)) back to back */
  float* h = zalloc((size_t)g * H);
  float* h2 = zalloc((size_t)g * H);
  or_linear_dense(frames, e->a_fc1_w, g, in, H, prec, h);
  add_bias(h, e->a_fc1_b, g, H, prec);
  or_silu(h, (int64_t)g * H, prec);
  or_linear_dense(h, e->a_fc2_w, g, H, H, prec, h2);
  add_bias(h2, e->a_fc2_b, g, H, prec);
  or_layernorm(h2, e->a_ln_w, e->a_ln_b, g, H, (float)c->norm_eps, prec, out);
  free(h);
  free(h2);
  return 0;
}

/* MossModel::encode_audio (mod.rs:82-126): every chunk through the encoder
 * (in batches of encoder_batch, which does not change the result), chunk i
 * trimmed to chunk_token_lengths[i] * merge frames, the chunks of each audio
 * concatenated in order (chunk_mapping[i] = its audio), then merge and
 * project per audio.  out: the audios' rows back to back; offsets
 * (num_audios + 1) receive each audio's first row. */
int or_enc_encode_audio(or_enc* e, const float* mel, int n_chunks, int frames,
                        const int32_t* chunk_tokens, const int32_t* chunk_mapping, int num_audios,
                        float* out, int64_t* offsets) {
  const or_audio_cfg* c = &e->cfg;
  const int d = c->d_model, merge = c->audio_merge_size;
  const int t2 = (frames + 2 - 3) / 2 + 1;
  float* enc = zalloc((size_t)n_chunks * t2 * d);
  if (or_enc_forward(e, mel, n_chunks, frames, enc)) {
    free(enc);
    return -1;
  }
  int64_t row = 0;
  for (int a = 0; a < num_audios; ++a) {
    int64_t nfr = 0;
    for (int i = 0; i < n_chunks; ++i)
      if (chunk_mapping[i] == a) {
        int64_t keep = (int64_t)chunk_tokens[i] * merge;
        nfr += keep < t2 ? keep : t2;
      }
    float* joined = zalloc((size_t)nfr * d);
    int64_t at = 0;
    for (int i = 0; i < n_chunks; ++i)
      if (chunk_mapping[i] == a) {
        int64_t keep = (int64_t)chunk_tokens[i] * merge;
        if (keep > t2) keep = t2;
        memcpy(joined + at * d, enc + (size_t)i * t2 * d, sizeof(float) * (size_t)keep * d);
        at += keep;
      }
    offsets[a] = row;
    const int g = (int)(nfr / merge);
    if (g > 0) or_enc_adaptor(e, joined, (int)nfr, out + row * c->hidden_size);
    row += g;
    free(joined);
  }
  offsets[num_audios] = row;
  free(enc);
  return 0;
}
