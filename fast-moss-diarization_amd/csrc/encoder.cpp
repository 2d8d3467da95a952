// C ABI of the audio path: WhisperEncoder (whisper_encoder.rs), VqAdaptor
// (adaptor.rs) and MossModel::encode_audio (mod.rs:82-126) on gfx950.
//
// Every linear and both convolutions run on the MFMA GEMM with the
// EPI_AFFINE epilogue (bias, q/k scale, gelu_erf / silu, residual,
// positions); LayerNorm and the dense attention are the kernels of
// encoder_kernels.hip.  Row-wise buffers hold `windows` windows of t positions,
// (t + 1) rows apart (the layout encoder_kernels.hip describes).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "fmd_dec.h"
#include "fmd_internal.h"
#include "fmd_kernels.h"

#define HIPCHK(expr)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fmd_fail(FMD_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)
#define CHK(expr)        \
  do {                   \
    int rc_ = (expr);    \
    if (rc_) return rc_; \
  } while (0)
#define LAUNCH(expr)                                                                    \
  do {                                                                                  \
    hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess)                                                               \
      return fmd_fail(FMD_ERR_HIP, std::string("launch ") + #expr + ": " + hipGetErrorString(e_)); \
  } while (0)

namespace {

struct EncLayer {
  LinWeights qkv{}, o{}, fc1{}, fc2{};
  void *qkv_b = nullptr, *o_b = nullptr, *fc1_b = nullptr, *fc2_b = nullptr;
  void *ln1_w = nullptr, *ln1_b = nullptr, *ln2_w = nullptr, *ln2_b = nullptr;
  uint32_t set = 0;
};

constexpr uint32_t kLayerBits = 0x7fffu;  // the 15 tensors of an encoder layer

}  // namespace

struct fmd_enc {
  fmd_audio_config cfg{};
  int prec = 0, act = 0, device = 0;
  size_t esz = 2;
  int d = 0, f = 0, heads = 0, nm = 0, cp = 0, T = 0, H = 0, merge = 0, ain = 0;
  float scale = 0.f, eps_ada = 1e-6f;
  hipStream_t own_stream = nullptr, stream = nullptr;
  LinWeights conv1{}, conv2{}, a_fc1{}, a_fc2{};
  void *conv1_b = nullptr, *conv2_b = nullptr, *pos = nullptr, *ln_w = nullptr, *ln_b = nullptr;
  void *a_fc1_b = nullptr, *a_fc2_b = nullptr, *a_ln_w = nullptr, *a_ln_b = nullptr;
  std::vector<EncLayer> layers;
  uint32_t set = 0;  // top-level tensors: bits 0-6 encoder, 8-13 adaptor
  std::vector<void*> allocs;
  DevBuf staging, staging2;
  // workspace
  DevBuf mel, melp, h1, x, xn, qkv, ctx, ff, frames, idx, joined, a1, a2, aout, hin;
};

namespace {

constexpr float kLnEps = 1e-5f;  // whisper_encoder.rs:14-15

int act_of(int prec) {
  switch (prec) {
    case FMD_F32: return ACT_F32;
    case FMD_F16: return ACT_F16;
    case FMD_BF16: return ACT_BF16;
    case FMD_INT8: return ACT_F16;  // the audio path stays dense in f16 (whisper_encoder.rs:31-33)
  }
  return -1;
}

size_t dtype_size(int dt) { return dt == FMD_DT_F32 ? 4 : 2; }

int dev_alloc(fmd_enc* e, void** p, size_t bytes) {
  if (hipMalloc(p, bytes ? bytes : 256) != hipSuccess) {
    *p = nullptr;
    return fmd_fail(FMD_ERR_OOM, "device allocation of " + std::to_string(bytes) + " bytes failed");
  }
  e->allocs.push_back(*p);
  HIPCHK(hipMemset(*p, 0, bytes ? bytes : 256));
  return 0;
}

int alloc_lin(fmd_enc* e, LinWeights& w, int out, int in) {
  w.kind = WK_DENSE;
  w.out = out;
  w.in = in;
  w.sc = nullptr;
  return dev_alloc(e, (void**)&w.w, (size_t)out * in * e->esz);
}

int alloc_vec(fmd_enc* e, void** p, size_t n) { return dev_alloc(e, p, n * e->esz); }

// Rows [row0, row0 + rows) of a dense linear from a device source.
int set_lin(fmd_enc* e, LinWeights& w, int row0, int rows, const void* src, int dt) {
  LAUNCH(launch_pack_dense(e->act, src, dt, rows, w.in, row0, w, e->stream));
  return 0;
}

int set_vec(fmd_enc* e, void* dst, const void* src, int dt, size_t n) {
  LAUNCH(launch_convert(e->act, src, dt, (int64_t)n, dst, e->stream));
  return 0;
}

// A convolution weight (cout, cin, 3) into the GEMM's (cout, 3 cinp) rows.
int set_conv(fmd_enc* e, LinWeights& w, int cin, int cinp, const void* src, int dt) {
  CHK(e->staging2.ensure((size_t)w.out * 3 * cinp * 4));
  LAUNCH(launch_conv_weight(src, dt, w.out, cin, cinp, e->staging2.as<float>(), e->stream));
  LAUNCH(launch_pack_dense(e->act, e->staging2.p, FMD_DT_F32, w.out, 3 * cinp, 0, w, e->stream));
  return 0;
}

int stage(fmd_enc* e, DevBuf& buf, const void* data, size_t bytes, int on_dev, const void** dev) {
  if (on_dev) {
    *dev = data;
    return 0;
  }
  CHK(buf.ensure(bytes));
  HIPCHK(hipMemcpyAsync(buf.p, data, bytes, hipMemcpyHostToDevice, e->stream));
  *dev = buf.p;
  return 0;
}

GemmArgs gemm(const void* x, int ldx, const LinWeights& w, int M, void* y, int ldy) {
  GemmArgs g{};
  g.x = x;
  g.ldx = ldx;
  g.W = w;
  g.M = M;
  g.y = y;
  g.ldy = ldy;
  return g;
}

// Workspace for `windows` windows of t positions from `frames` mel frames
// (frames 0: the layers alone).
int ensure_ws(fmd_enc* e, int windows, int t, int frames) {
  const size_t P = (size_t)t + 1, rows = (size_t)windows * P, es = e->esz;
  CHK(e->x.ensure(rows * e->d * es));
  CHK(e->xn.ensure(rows * e->d * es));
  CHK(e->qkv.ensure(rows * 3 * e->d * es));
  CHK(e->ctx.ensure(rows * e->d * es));
  CHK(e->ff.ensure(rows * e->f * es));
  if (frames > 0) {
    CHK(e->melp.ensure(((size_t)windows * (frames + 2) + 1) * e->cp * es));
    CHK(e->h1.ensure(((size_t)windows * (frames + 2) + 1) * e->d * es));
  }
  return 0;
}

// The layers [first, first + n) and (final_norm) the final LayerNorm over the
// rows of e->x (windows of t positions, t + 1 rows apart); the normalised
// rows go to `out` (windows * t rows of d, contiguous, device).
int run_layers(fmd_enc* e, int windows, int t, int first, int n, bool final_norm, void* out) {
  hipStream_t s = e->stream;
  const int P = t + 1, rows = windows * P, d = e->d, act = e->act;
  for (int l = first; l < first + n; ++l) {
    const EncLayer& L = e->layers[l];
    LAUNCH(launch_layernorm(act, e->x.p, d, L.ln1_w, L.ln1_b, rows, d, kLnEps, e->xn.p, d, s));
    // q | k | v: rd(rd(h W^T) + b), q and k then rd(. * rd(head_dim^-1/4))
    GemmArgs g = gemm(e->xn.p, d, L.qkv, rows, e->qkv.p, 3 * d);
    g.aff.bias = L.qkv_b;
    g.aff.scale = e->scale;
    g.aff.scale_cols = 2 * d;
    LAUNCH(launch_gemm(act, EPI_AFFINE, g, s));
    EncAttnArgs a{};
    a.qkv = e->qkv.p;
    a.ld = 3 * d;
    a.d = d;
    a.t = t;
    a.period = P;
    a.out = e->ctx.p;
    a.ldo = d;
    LAUNCH(launch_enc_attn(act, a, e->heads, windows, s));
    // x = rd(x + rd(rd(ctx Wo^T) + bo))
    g = gemm(e->ctx.p, d, L.o, rows, e->x.p, d);
    g.aff.bias = L.o_b;
    g.resid = e->x.p;
    LAUNCH(launch_gemm(act, EPI_AFFINE, g, s));
    LAUNCH(launch_layernorm(act, e->x.p, d, L.ln2_w, L.ln2_b, rows, d, kLnEps, e->xn.p, d, s));
    g = gemm(e->xn.p, d, L.fc1, rows, e->ff.p, e->f);
    g.aff.bias = L.fc1_b;
    g.aff.act = 1;
    LAUNCH(launch_gemm(act, EPI_AFFINE, g, s));
    g = gemm(e->ff.p, e->f, L.fc2, rows, e->x.p, d);
    g.aff.bias = L.fc2_b;
    g.resid = e->x.p;
    LAUNCH(launch_gemm(act, EPI_AFFINE, g, s));
  }
  const size_t es = e->esz;
  if (final_norm) {
    LAUNCH(launch_layernorm(act, e->x.p, d, e->ln_w, e->ln_b, rows, d, kLnEps, e->xn.p, d, s));
    HIPCHK(hipMemcpy2DAsync(out, (size_t)t * d * es, e->xn.p, (size_t)P * d * es,
                            (size_t)t * d * es, windows, hipMemcpyDeviceToDevice, s));
  } else {
    HIPCHK(hipMemcpy2DAsync(out, (size_t)t * d * es, e->x.p, (size_t)P * d * es,
                            (size_t)t * d * es, windows, hipMemcpyDeviceToDevice, s));
  }
  return 0;
}

// WhisperEncoder::forward (whisper_encoder.rs:139-163) of `windows` mel
// chunks (device, src dtype) into `out` (windows * frames/2 rows of d).
int forward_windows(fmd_enc* e, const void* mel_dev, int mel_dtype, int windows, int frames,
                    void* out) {
  hipStream_t s = e->stream;
  const int t = frames / 2, P = t + 1, d = e->d, act = e->act;
  CHK(ensure_ws(e, windows, t, frames));
  const size_t es = e->esz;
  LAUNCH(launch_mel_pack(act, mel_dev, mel_dtype, windows, e->nm, frames, e->cp, e->melp.p, s));
  // conv1's pad rows (the zero row before and after each window) stay zero:
  // its epilogue stores only the frame rows
  HIPCHK(hipMemsetAsync(e->h1.p, 0, ((size_t)windows * (frames + 2) + 1) * d * es, s));
  // conv1 (stride 1) + bias + gelu_erf: GEMM row j reads rows j .. j + 2 of
  // the packed mel and is frame j % (frames + 2) of its window; it lands on
  // conv1's row j + 1
  GemmArgs g = gemm(e->melp.p, e->cp, e->conv1, windows * (frames + 2) - 2,
                    (char*)e->h1.p + (size_t)d * es, d);
  g.aff.bias = e->conv1_b;
  g.aff.act = 1;
  g.aff.period = frames + 2;
  g.aff.valid = frames;
  LAUNCH(launch_gemm(act, EPI_AFFINE, g, s));
  // conv2 (stride 2) + bias + gelu_erf + positions: GEMM row j = w P + t'
  // reads conv1 rows 2j .. 2j + 2 (stride 2 d elements), which are window w's
  // frames 2t' - 1 .. 2t' + 1
  g = gemm(e->h1.p, 2 * d, e->conv2, windows * P - 1, e->x.p, d);
  g.aff.bias = e->conv2_b;
  g.aff.act = 1;
  g.aff.table = e->pos;
  g.aff.period = P;
  g.aff.valid = t;
  LAUNCH(launch_gemm(act, EPI_AFFINE, g, s));
  return run_layers(e, windows, t, 0, (int)e->layers.size(), true, out);
}

int check_frames(const fmd_enc* e, int frames) {
  if (frames < 2 || frames % 2) return fmd_fail(FMD_ERR_ARG, "mel frames must be even and >= 2");
  if (frames / 2 > e->T)
    return fmd_fail(FMD_ERR_ARG, "mel chunk of " + std::to_string(frames) + " frames exceeds " +
                                     std::to_string(e->T) + " positions");
  return 0;
}

// VqAdaptor::forward (adaptor.rs:56-60) of `g` merged rows (device, g x
// merge*d) into `out` (device, g x H).
int adaptor_rows(fmd_enc* e, const void* merged, int g, void* out) {
  if (g <= 0) return 0;
  hipStream_t s = e->stream;
  const size_t es = e->esz;
  CHK(e->a1.ensure((size_t)g * e->H * es));
  CHK(e->a2.ensure((size_t)g * e->H * es));
  GemmArgs ga = gemm(merged, e->ain, e->a_fc1, g, e->a1.p, e->H);
  ga.aff.bias = e->a_fc1_b;
  ga.aff.act = 2;
  LAUNCH(launch_gemm(e->act, EPI_AFFINE, ga, s));
  ga = gemm(e->a1.p, e->H, e->a_fc2, g, e->a2.p, e->H);
  ga.aff.bias = e->a_fc2_b;
  LAUNCH(launch_gemm(e->act, EPI_AFFINE, ga, s));
  LAUNCH(launch_layernorm(e->act, e->a2.p, e->H, e->a_ln_w, e->a_ln_b, g, e->H, e->eps_ada, out,
                          e->H, s));
  return 0;
}

int ready_check(const fmd_enc* e) {
  if (!fmd_enc_ready(e)) return fmd_fail(FMD_ERR_STATE, "audio weights are incomplete");
  return 0;
}

}  // namespace

extern "C" int fmd_enc_create(const fmd_audio_config* cfg, fmd_precision precision, int device,
                              fmd_enc** out) {
  if (!cfg || !out) return fmd_fail(FMD_ERR_ARG, "null argument");
  *out = nullptr;
  const int act = act_of(precision);
  if (act < 0) return fmd_fail(FMD_ERR_ARG, "unknown precision");
  const int d = cfg->d_model, heads = cfg->encoder_attention_heads;
  if (d <= 0 || heads <= 0 || d % heads || d / heads != 64)
    return fmd_fail(FMD_ERR_ARG, "encoder head_dim (d_model / encoder_attention_heads) must be 64");
  if (cfg->encoder_ffn_dim <= 0 || cfg->encoder_ffn_dim % 64 || cfg->hidden_size <= 0 ||
      cfg->hidden_size % 64 || cfg->num_mel_bins <= 0 || cfg->encoder_layers < 0 ||
      cfg->max_source_positions <= 0)
    return fmd_fail(FMD_ERR_ARG, "encoder_ffn_dim and hidden_size must be multiples of 64");
  if (cfg->audio_merge_size <= 0 || cfg->adaptor_input_dim != d * cfg->audio_merge_size)
    return fmd_fail(FMD_ERR_ARG, "adaptor_input_dim must be d_model * audio_merge_size");
  fmd_enc* e = new fmd_enc();
  e->cfg = *cfg;
  e->prec = precision;
  e->act = act;
  e->device = device;
  e->esz = act == ACT_F32 ? 4 : 2;
  e->d = d;
  e->f = cfg->encoder_ffn_dim;
  e->heads = heads;
  e->nm = cfg->num_mel_bins;
  e->cp = (cfg->num_mel_bins + 63) / 64 * 64;
  e->T = cfg->max_source_positions;
  e->H = cfg->hidden_size;
  e->merge = cfg->audio_merge_size;
  e->ain = cfg->adaptor_input_dim;
  e->eps_ada = (float)cfg->norm_eps;
  // `Tensor * f64` scales in the dtype with the multiplier rounded to it
  e->scale = host_round_act((float)std::pow(64.0, -0.25), act);
  int rc = hipSetDevice(device) == hipSuccess ? 0 : fmd_fail(FMD_ERR_HIP, "hipSetDevice failed");
  if (!rc && hipStreamCreateWithFlags(&e->own_stream, hipStreamNonBlocking) != hipSuccess)
    rc = fmd_fail(FMD_ERR_HIP, "stream creation failed");
  e->stream = e->own_stream;
  if (!rc) rc = alloc_lin(e, e->conv1, d, 3 * e->cp);
  if (!rc) rc = alloc_lin(e, e->conv2, d, 3 * d);
  if (!rc) rc = alloc_lin(e, e->a_fc1, e->H, e->ain);
  if (!rc) rc = alloc_lin(e, e->a_fc2, e->H, e->H);
  for (void** v : {&e->conv1_b, &e->conv2_b, &e->ln_w, &e->ln_b})
    if (!rc) rc = alloc_vec(e, v, (size_t)d);
  if (!rc) rc = alloc_vec(e, &e->pos, (size_t)e->T * d);
  for (void** v : {&e->a_fc1_b, &e->a_fc2_b, &e->a_ln_w, &e->a_ln_b})
    if (!rc) rc = alloc_vec(e, v, (size_t)e->H);
  e->layers.resize(cfg->encoder_layers);
  for (EncLayer& L : e->layers) {
    if (!rc) rc = alloc_lin(e, L.qkv, 3 * d, d);
    if (!rc) rc = alloc_lin(e, L.o, d, d);
    if (!rc) rc = alloc_lin(e, L.fc1, e->f, d);
    if (!rc) rc = alloc_lin(e, L.fc2, d, e->f);
    if (!rc) rc = alloc_vec(e, &L.qkv_b, (size_t)3 * d);  // k_proj has no bias: stays zero
    if (!rc) rc = alloc_vec(e, &L.fc1_b, (size_t)e->f);
    for (void** v : {&L.o_b, &L.fc2_b, &L.ln1_w, &L.ln1_b, &L.ln2_w, &L.ln2_b})
      if (!rc) rc = alloc_vec(e, v, (size_t)d);
  }
  if (rc) {
    std::string keep = fmd_last_error();
    fmd_enc_destroy(e);
    fmd_fail(rc, keep);
    return rc;
  }
  *out = e;
  return 0;
}

extern "C" int fmd_enc_destroy(fmd_enc* e) {
  if (!e) return 0;
  hipSetDevice(e->device);
  if (e->stream) hipStreamSynchronize(e->stream);
  for (void* p : e->allocs) hipFree(p);
  for (DevBuf* b : {&e->staging, &e->staging2, &e->mel, &e->melp, &e->h1, &e->x, &e->xn, &e->qkv,
                    &e->ctx, &e->ff, &e->frames, &e->idx, &e->joined, &e->a1, &e->a2, &e->aout,
                    &e->hin})
    b->release();
  if (e->own_stream) hipStreamDestroy(e->own_stream);
  delete e;
  return 0;
}

extern "C" int fmd_enc_set_stream(fmd_enc* e, void* s) {
  if (!e) return fmd_fail(FMD_ERR_ARG, "null handle");
  HIPCHK(hipStreamSynchronize(e->stream));
  e->stream = s ? (hipStream_t)s : e->own_stream;
  return 0;
}

extern "C" int fmd_enc_set_weight(fmd_enc* e, const char* name, fmd_dtype dtype,
                                  const int64_t* shape, int ndim, const void* data,
                                  int data_on_device) {
  if (!e || !name || !data || !shape) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (dtype < FMD_DT_F32 || dtype > FMD_DT_BF16) return fmd_fail(FMD_ERR_ARG, "bad dtype");
  HIPCHK(hipSetDevice(e->device));
  const int d = e->d, f = e->f, H = e->H;
  const std::string n(name);
  const std::string ep = "model.whisper_encoder.", ap = "model.vq_adaptor.";
  // (kind, target): 0 linear rows, 1 vector, 2 conv
  struct T {
    int kind = -1;
    LinWeights* lin = nullptr;
    void* vec = nullptr;
    int row0 = 0;
    std::vector<int64_t> shape;
    uint32_t* bits = nullptr;
    uint32_t bit = 0;
    int cin = 0;
  } t;
  auto vec = [&](void* p, int64_t len, uint32_t* bits, int bit) {
    t.kind = 1;
    t.vec = p;
    t.shape = {len};
    t.bits = bits;
    t.bit = bit;
  };
  auto lin = [&](LinWeights* w, int row0, int64_t rows, int64_t cols, uint32_t* bits, int bit) {
    t.kind = 0;
    t.lin = w;
    t.row0 = row0;
    t.shape = {rows, cols};
    t.bits = bits;
    t.bit = bit;
  };
  if (n.compare(0, ap.size(), ap) == 0) {
    const std::string r = n.substr(ap.size());
    if (r == "layers.0.weight") lin(&e->a_fc1, 0, H, e->ain, &e->set, 8);
    else if (r == "layers.0.bias") vec(e->a_fc1_b, H, &e->set, 9);
    else if (r == "layers.2.weight") lin(&e->a_fc2, 0, H, H, &e->set, 10);
    else if (r == "layers.2.bias") vec(e->a_fc2_b, H, &e->set, 11);
    else if (r == "layers.3.weight") vec(e->a_ln_w, H, &e->set, 12);
    else if (r == "layers.3.bias") vec(e->a_ln_b, H, &e->set, 13);
  } else if (n.compare(0, ep.size(), ep) == 0) {
    const std::string r = n.substr(ep.size());
    if (r == "conv1.weight") {
      t.kind = 2;
      t.lin = &e->conv1;
      t.shape = {d, e->nm, 3};
      t.cin = e->nm;
      t.bits = &e->set;
      t.bit = 0;
    } else if (r == "conv2.weight") {
      t.kind = 2;
      t.lin = &e->conv2;
      t.shape = {d, d, 3};
      t.cin = d;
      t.bits = &e->set;
      t.bit = 2;
    } else if (r == "conv1.bias") vec(e->conv1_b, d, &e->set, 1);
    else if (r == "conv2.bias") vec(e->conv2_b, d, &e->set, 3);
    else if (r == "embed_positions.weight") {
      vec(e->pos, (int64_t)e->T * d, &e->set, 4);
      t.shape = {e->T, d};
    } else if (r == "layer_norm.weight") vec(e->ln_w, d, &e->set, 5);
    else if (r == "layer_norm.bias") vec(e->ln_b, d, &e->set, 6);
    else {
      int li = -1, used = 0;
      if (sscanf(r.c_str(), "layers.%d.%n", &li, &used) == 1 && used > 0 && li >= 0 &&
          li < (int)e->layers.size()) {
        EncLayer& L = e->layers[li];
        const std::string rest = r.substr(used);
        uint32_t* b = &L.set;
        if (rest == "self_attn.q_proj.weight") lin(&L.qkv, 0, d, d, b, 0);
        else if (rest == "self_attn.q_proj.bias") { vec(L.qkv_b, d, b, 1); }
        else if (rest == "self_attn.k_proj.weight") lin(&L.qkv, d, d, d, b, 2);
        else if (rest == "self_attn.v_proj.weight") lin(&L.qkv, 2 * d, d, d, b, 3);
        else if (rest == "self_attn.v_proj.bias") { vec((char*)L.qkv_b + (size_t)2 * d * e->esz, d, b, 4); }
        else if (rest == "self_attn.out_proj.weight") lin(&L.o, 0, d, d, b, 5);
        else if (rest == "self_attn.out_proj.bias") vec(L.o_b, d, b, 6);
        else if (rest == "self_attn_layer_norm.weight") vec(L.ln1_w, d, b, 7);
        else if (rest == "self_attn_layer_norm.bias") vec(L.ln1_b, d, b, 8);
        else if (rest == "fc1.weight") lin(&L.fc1, 0, f, d, b, 9);
        else if (rest == "fc1.bias") vec(L.fc1_b, f, b, 10);
        else if (rest == "fc2.weight") lin(&L.fc2, 0, d, f, b, 11);
        else if (rest == "fc2.bias") vec(L.fc2_b, d, b, 12);
        else if (rest == "final_layer_norm.weight") vec(L.ln2_w, d, b, 13);
        else if (rest == "final_layer_norm.bias") vec(L.ln2_b, d, b, 14);
      }
    }
  }
  if (t.kind < 0) return fmd_fail(FMD_ERR_ARG, std::string("unknown tensor ") + name);
  bool ok = ndim == (int)t.shape.size();
  int64_t numel = 1;
  for (int i = 0; ok && i < ndim; ++i) {
    ok = shape[i] == t.shape[i];
    numel *= shape[i];
  }
  if (!ok) return fmd_fail(FMD_ERR_ARG, std::string("shape mismatch for ") + name);
  const void* src = nullptr;
  CHK(stage(e, e->staging, data, (size_t)numel * dtype_size(dtype), data_on_device, &src));
  if (t.kind == 0) CHK(set_lin(e, *t.lin, t.row0, (int)t.shape[0], src, dtype));
  else if (t.kind == 1) CHK(set_vec(e, t.vec, src, dtype, (size_t)numel));
  else CHK(set_conv(e, *t.lin, t.cin, t.lin == &e->conv1 ? e->cp : d, src, dtype));
  *t.bits |= 1u << t.bit;
  HIPCHK(hipStreamSynchronize(e->stream));
  return 0;
}

extern "C" int fmd_enc_ready(const fmd_enc* e) {
  if (!e) return 0;
  if ((e->set & 0x7fu) != 0x7fu || ((e->set >> 8) & 0x3fu) != 0x3fu) return 0;
  for (const EncLayer& L : e->layers)
    if (L.set != kLayerBits) return 0;
  return 1;
}

extern "C" int fmd_enc_forward(fmd_enc* e, const void* mel, fmd_dtype mel_dtype, int mel_on_device,
                               int n, int frames, void* out, int out_on_device) {
  if (!e || !mel || !out) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (n < 0 || mel_dtype < FMD_DT_F32 || mel_dtype > FMD_DT_BF16)
    return fmd_fail(FMD_ERR_ARG, "bad argument");
  CHK(ready_check(e));
  CHK(check_frames(e, frames));
  if (n == 0) return 0;
  HIPCHK(hipSetDevice(e->device));
  const size_t mel_bytes = (size_t)n * e->nm * frames * dtype_size(mel_dtype);
  const void* src = nullptr;
  CHK(stage(e, e->mel, mel, mel_bytes, mel_on_device, &src));
  const int t = frames / 2;
  const size_t out_bytes = (size_t)n * t * e->d * e->esz;
  void* dst = out;
  if (!out_on_device) {
    CHK(e->frames.ensure(out_bytes));
    dst = e->frames.p;
  }
  CHK(forward_windows(e, src, mel_dtype, n, frames, dst));
  if (!out_on_device) HIPCHK(hipMemcpyAsync(out, dst, out_bytes, hipMemcpyDeviceToHost, e->stream));
  HIPCHK(hipStreamSynchronize(e->stream));
  return 0;
}

extern "C" int fmd_enc_layers(fmd_enc* e, const void* x, int x_on_device, int windows, int t,
                              int first, int n, int final_norm, void* out, int out_on_device) {
  if (!e || !x || !out) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (windows < 0 || t <= 0 || first < 0 || n < 0 || first + n > (int)e->layers.size())
    return fmd_fail(FMD_ERR_ARG, "bad layer range or shape");
  CHK(ready_check(e));
  if (windows == 0) return 0;
  HIPCHK(hipSetDevice(e->device));
  CHK(ensure_ws(e, windows, t, 0));
  const size_t es = e->esz, row = (size_t)e->d * es, bytes = (size_t)windows * t * row;
  const void* src = nullptr;
  CHK(stage(e, e->hin, x, bytes, x_on_device, &src));
  // into the (t + 1)-row window layout
  HIPCHK(hipMemcpy2DAsync(e->x.p, (size_t)(t + 1) * row, src, (size_t)t * row, (size_t)t * row,
                          windows, hipMemcpyDeviceToDevice, e->stream));
  void* dst = out;
  if (!out_on_device) {
    CHK(e->frames.ensure(bytes));
    dst = e->frames.p;
  }
  CHK(run_layers(e, windows, t, first, n, final_norm != 0, dst));
  if (!out_on_device) HIPCHK(hipMemcpyAsync(out, dst, bytes, hipMemcpyDeviceToHost, e->stream));
  HIPCHK(hipStreamSynchronize(e->stream));
  return 0;
}

extern "C" int fmd_enc_adaptor(fmd_enc* e, const void* frames, int frames_on_device, int rows,
                               void* out, int out_on_device) {
  if (!e || !frames || !out) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (rows < 0) return fmd_fail(FMD_ERR_ARG, "negative row count");
  CHK(ready_check(e));
  const int g = rows / e->merge;  // a trailing partial group is dropped (adaptor.rs:41-52)
  if (g == 0) return 0;
  HIPCHK(hipSetDevice(e->device));
  const size_t es = e->esz;
  const void* src = nullptr;
  CHK(stage(e, e->joined, frames, (size_t)g * e->ain * es, frames_on_device, &src));
  void* dst = out;
  if (!out_on_device) {
    CHK(e->aout.ensure((size_t)g * e->H * es));
    dst = e->aout.p;
  }
  CHK(adaptor_rows(e, src, g, dst));
  if (!out_on_device)
    HIPCHK(hipMemcpyAsync(out, dst, (size_t)g * e->H * es, hipMemcpyDeviceToHost, e->stream));
  HIPCHK(hipStreamSynchronize(e->stream));
  return 0;
}

extern "C" int fmd_enc_encode_audio(fmd_enc* e, const void* mel, fmd_dtype mel_dtype,
                                    int mel_on_device, int n_chunks, int frames,
                                    const int32_t* chunk_tokens, const int32_t* chunk_mapping,
                                    int num_audios, int encoder_batch, void* out,
                                    int out_on_device, int64_t* offsets) {
  if (!e || !offsets || (n_chunks > 0 && (!chunk_tokens || !chunk_mapping || (out && !mel))))
    return fmd_fail(FMD_ERR_ARG, "null argument");
  if (n_chunks < 0 || num_audios < 0 || mel_dtype < FMD_DT_F32 || mel_dtype > FMD_DT_BF16)
    return fmd_fail(FMD_ERR_ARG, "bad argument");
  CHK(check_frames(e, frames));
  const int t = frames / 2, merge = e->merge;
  // Per audio, the kept frames of its chunks in chunk order (mod.rs:108-125)
  // and the rows they merge into (adaptor.rs:41-52).
  std::vector<int64_t> nfr(num_audios, 0);
  for (int i = 0; i < n_chunks; ++i) {
    if (chunk_mapping[i] < 0 || chunk_mapping[i] >= num_audios)
      return fmd_fail(FMD_ERR_ARG, "chunk_mapping entry outside [0, num_audios)");
    if (chunk_tokens[i] < 0) return fmd_fail(FMD_ERR_ARG, "negative chunk token length");
    nfr[chunk_mapping[i]] += std::min<int64_t>((int64_t)chunk_tokens[i] * merge, t);
  }
  offsets[0] = 0;
  for (int a = 0; a < num_audios; ++a) offsets[a + 1] = offsets[a] + nfr[a] / merge;
  const int64_t G = offsets[num_audios];
  if (!out) return 0;  // size query
  CHK(ready_check(e));
  if (n_chunks == 0 || G == 0) return 0;
  if (G > (1 << 26)) return fmd_fail(FMD_ERR_ARG, "too many audio rows");
  HIPCHK(hipSetDevice(e->device));
  const size_t es = e->esz;
  // every chunk through the encoder, encoder_batch at a time (mod.rs:94-103)
  CHK(e->frames.ensure((size_t)n_chunks * t * e->d * es));
  const int eb = std::max(encoder_batch, 1);
  const size_t chunk_bytes = (size_t)e->nm * frames * dtype_size(mel_dtype);
  for (int c0 = 0; c0 < n_chunks; c0 += eb) {
    const int take = std::min(eb, n_chunks - c0);
    const void* src = nullptr;
    CHK(stage(e, e->mel, (const char*)mel + c0 * chunk_bytes, take * chunk_bytes, mel_on_device, &src));
    CHK(forward_windows(e, src, mel_dtype, take, frames,
                        (char*)e->frames.p + (size_t)c0 * t * e->d * es));
  }
  // frame gather: merged row g of audio a is frames merge*g .. merge*g + merge-1
  // of the audio's joined frames
  std::vector<int32_t> src_row((size_t)G * merge);
  for (int a = 0; a < num_audios; ++a) {
    int64_t k = 0;
    const int64_t want = (offsets[a + 1] - offsets[a]) * merge;
    int32_t* dst = src_row.data() + offsets[a] * merge;
    for (int i = 0; i < n_chunks && k < want; ++i) {
      if (chunk_mapping[i] != a) continue;
      const int64_t keep = std::min<int64_t>((int64_t)chunk_tokens[i] * merge, t);
      for (int64_t r = 0; r < keep && k < want; ++r) dst[k++] = (int32_t)((int64_t)i * t + r);
    }
  }
  CHK(e->idx.ensure(src_row.size() * 4));
  HIPCHK(hipMemcpyAsync(e->idx.p, src_row.data(), src_row.size() * 4, hipMemcpyHostToDevice, e->stream));
  CHK(e->joined.ensure((size_t)G * e->ain * es));
  LAUNCH(launch_gather_rows(e->act, e->frames.p, e->d, e->idx.as<int32_t>(), (int)(G * merge), e->d,
                            e->joined.p, e->d, e->stream));
  void* dst = out;
  if (!out_on_device) {
    CHK(e->aout.ensure((size_t)G * e->H * es));
    dst = e->aout.p;
  }
  CHK(adaptor_rows(e, e->joined.p, (int)G, dst));
  if (!out_on_device)
    HIPCHK(hipMemcpyAsync(out, dst, (size_t)G * e->H * es, hipMemcpyDeviceToHost, e->stream));
  HIPCHK(hipStreamSynchronize(e->stream));
  return 0;
}
