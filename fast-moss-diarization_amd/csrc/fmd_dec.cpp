// C ABI of the gfx950 decoder: model and KV-cache handles, weight loading,
// prefill / decode orchestration and the graph-launched greedy loop.
//
// Reference: crates/fmd-core/src/model/qwen3.rs (Qwen3, KvCache),
// model/linear.rs (Loader, Linear, FusedLinear, RmsNorm) and
// engine.rs::generate_batch (463-559).
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

int attn_prefill_tile_rows(int rep);

static thread_local std::string g_err;

int fmd_fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

extern "C" const char* fmd_last_error(void) { return g_err.c_str(); }

#define HIPCHK(expr)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fmd_fail(FMD_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

#define CHK(expr)           \
  do {                      \
    int rc_ = (expr);       \
    if (rc_) return rc_;    \
  } while (0)

int DevBuf::ensure(size_t bytes, bool* fresh) {
  if (fresh) *fresh = false;
  if (n >= bytes && p) return 0;
  if (fresh) *fresh = true;
  if (p) hipFree(p);
  p = nullptr;
  n = 0;
  if (bytes == 0) bytes = 256;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    p = nullptr;
    return fmd_fail(FMD_ERR_OOM, "device allocation of " + std::to_string(bytes) + " bytes failed");
  }
  n = bytes;
  return 0;
}

void DevBuf::release() {
  if (p) hipFree(p);
  p = nullptr;
  n = 0;
}

static int act_of(int prec) {
  switch (prec) {
    case FMD_F32: return ACT_F32;
    case FMD_F16: return ACT_F16;
    case FMD_BF16: return ACT_BF16;
    case FMD_INT8: return ACT_F16;
  }
  return -1;
}

// ---------------------------------------------------------------------------
// model handle
// ---------------------------------------------------------------------------

static int alloc_lin(fmd_dec* d, Lin& l, int out, int in) {
  l.w.kind = d->quant ? WK_Q8 : WK_DENSE;
  l.w.out = out;
  l.w.in = in;
  l.wbytes = (size_t)out * in * (d->quant ? 1 : d->esz);
  l.sbytes = d->quant ? (size_t)out * (in / 64) * 4 : 0;
  if (hipMalloc((void**)&l.w.w, l.wbytes) != hipSuccess)
    return fmd_fail(FMD_ERR_OOM, "weight allocation failed");
  HIPCHK(hipMemset(l.w.w, 0, l.wbytes));
  l.w.sc = nullptr;
  if (l.sbytes) {
    if (hipMalloc((void**)&l.w.sc, l.sbytes) != hipSuccess)
      return fmd_fail(FMD_ERR_OOM, "weight allocation failed");
    HIPCHK(hipMemset(l.w.sc, 0, l.sbytes));
  }
  return 0;
}

static void free_lin(Lin& l) {
  if (l.w.w) hipFree(l.w.w);
  if (l.w.sc) hipFree(l.w.sc);
  l.w.w = nullptr;
  l.w.sc = nullptr;
}

static int alloc_vec(fmd_dec* d, void** p, size_t n) {
  if (hipMalloc(p, n * d->esz) != hipSuccess) return fmd_fail(FMD_ERR_OOM, "allocation failed");
  HIPCHK(hipMemset(*p, 0, n * d->esz));
  return 0;
}

extern "C" int fmd_dec_create(const fmd_text_config* cfg, fmd_precision precision, int device,
                              int max_len, fmd_dec** out) {
  if (!cfg || !out) return fmd_fail(FMD_ERR_ARG, "null argument");
  *out = nullptr;
  const int act = act_of(precision);
  if (act < 0) return fmd_fail(FMD_ERR_ARG, "unknown precision");
  if (cfg->head_dim != 128) return fmd_fail(FMD_ERR_ARG, "head_dim must be 128");
  if (cfg->attention_bias) return fmd_fail(FMD_ERR_ARG, "attention_bias is not supported");
  if (cfg->num_key_value_heads <= 0 || cfg->num_attention_heads % cfg->num_key_value_heads)
    return fmd_fail(FMD_ERR_ARG, "num_attention_heads must be a multiple of num_key_value_heads");
  const int rep = cfg->num_attention_heads / cfg->num_key_value_heads;
  if (rep != 1 && rep != 2 && rep != 4)
    return fmd_fail(FMD_ERR_ARG, "heads per kv head must be 1, 2 or 4");
  const int qd = cfg->num_attention_heads * cfg->head_dim;
  if (cfg->hidden_size % 256 || cfg->intermediate_size % 256 || qd % 256 ||
      cfg->hidden_size > 4096 || cfg->intermediate_size > 4096 || qd > 4096)
    return fmd_fail(FMD_ERR_ARG,
                    "hidden_size, intermediate_size and q width must be multiples of 256, <= 4096");
  if (cfg->vocab_size <= 0 || cfg->vocab_size % 16)
    return fmd_fail(FMD_ERR_ARG, "vocab_size must be a positive multiple of 16");
  if (cfg->num_hidden_layers <= 0 || max_len <= 0) return fmd_fail(FMD_ERR_ARG, "bad sizes");
  HIPCHK(hipSetDevice(device));

  fmd_dec* d = new fmd_dec();
  d->cfg = *cfg;
  d->prec = precision;
  d->act = act;
  d->quant = precision == FMD_INT8;
  d->device = device;
  d->max_len = max_len;
  d->esz = act == ACT_F32 ? 4 : 2;
  d->H = cfg->hidden_size;
  d->I = cfg->intermediate_size;
  d->hd = cfg->head_dim;
  d->nh = cfg->num_attention_heads;
  d->nkv = cfg->num_key_value_heads;
  d->rep = rep;
  d->qd = qd;
  d->kd = d->nkv * d->hd;
  d->qkvd = d->qd + 2 * d->kd;
  d->V = cfg->vocab_size;
  d->L = cfg->num_hidden_layers;
  d->eps = (float)cfg->rms_norm_eps;
  d->scale = (float)(1.0 / std::sqrt((double)d->hd));
  if (hipStreamCreateWithFlags(&d->own_stream, hipStreamNonBlocking) != hipSuccess) {
    delete d;
    return fmd_fail(FMD_ERR_HIP, "stream creation failed");
  }
  d->stream = d->own_stream;

  int rc = noalloc_scratch_init(device, d->stream);
  d->layers.resize(d->L);
  for (auto& ly : d->layers) {
    if (rc) break;
    if ((rc = alloc_lin(d, ly.qkv, d->qkvd, d->H))) break;
    if ((rc = alloc_lin(d, ly.o, d->H, d->qd))) break;
    if ((rc = alloc_lin(d, ly.gate_up, 2 * d->I, d->H))) break;
    if ((rc = alloc_lin(d, ly.down, d->H, d->I))) break;
    if ((rc = alloc_vec(d, &ly.in_norm, d->H))) break;
    if ((rc = alloc_vec(d, &ly.post_norm, d->H))) break;
    if ((rc = alloc_vec(d, &ly.q_norm, d->hd))) break;
    if ((rc = alloc_vec(d, &ly.k_norm, d->hd))) break;
  }
  if (!rc) rc = alloc_lin(d, d->lm_head, d->V, d->H);
  if (!rc) rc = alloc_vec(d, &d->embed, (size_t)d->V * d->H);
  if (!rc) rc = alloc_vec(d, &d->norm, d->H);
  if (!rc) {
    // Rope::new (qwen3.rs:117-136): inv_freq in f64 then f32; freqs = pos(f32) *
    // inv_freq (f32); cos/sin in f32, then cast to the activation dtype.
    const int half = d->hd / 2;
    std::vector<float> inv(half), cs((size_t)max_len * half), sn((size_t)max_len * half);
    for (int i = 0; i < half; ++i)
      inv[i] = (float)(1.0 / std::pow(cfg->rope_theta, 2.0 * (double)i / (double)d->hd));
    for (int p = 0; p < max_len; ++p)
      for (int i = 0; i < half; ++i) {
        const float f = (float)p * inv[i];
        cs[(size_t)p * half + i] = cosf(f);
        sn[(size_t)p * half + i] = sinf(f);
      }
    rc = alloc_vec(d, &d->cos, cs.size());
    if (!rc) rc = alloc_vec(d, &d->sin, sn.size());
    if (!rc) rc = d->staging.ensure(cs.size() * 4);
    if (!rc && hipMemcpy(d->staging.p, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      rc = fmd_fail(FMD_ERR_HIP, "rope upload failed");
    if (!rc && launch_convert(d->act, d->staging.p, 0, (int64_t)cs.size(), d->cos, d->stream) != hipSuccess)
      rc = fmd_fail(FMD_ERR_HIP, "rope convert failed");
    if (!rc && hipStreamSynchronize(d->stream) != hipSuccess) rc = fmd_fail(FMD_ERR_HIP, "sync failed");
    if (!rc && hipMemcpy(d->staging.p, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      rc = fmd_fail(FMD_ERR_HIP, "rope upload failed");
    if (!rc && launch_convert(d->act, d->staging.p, 0, (int64_t)sn.size(), d->sin, d->stream) != hipSuccess)
      rc = fmd_fail(FMD_ERR_HIP, "rope convert failed");
    if (!rc && hipStreamSynchronize(d->stream) != hipSuccess) rc = fmd_fail(FMD_ERR_HIP, "sync failed");
  }
  if (rc) {
    std::string keep = g_err;
    fmd_dec_destroy(d);
    g_err = keep;
    return rc;
  }
  *out = d;
  return 0;
}

extern "C" int fmd_dec_destroy(fmd_dec* d) {
  if (!d) return 0;
  hipSetDevice(d->device);
  if (d->stream) hipStreamSynchronize(d->stream);
  for (auto& ly : d->layers) {
    free_lin(ly.qkv);
    free_lin(ly.o);
    free_lin(ly.gate_up);
    free_lin(ly.down);
    for (void* p : {ly.in_norm, ly.post_norm, ly.q_norm, ly.k_norm})
      if (p) hipFree(p);
  }
  free_lin(d->lm_head);
  for (void* p : {d->embed, d->norm, d->cos, d->sin})
    if (p) hipFree(p);
  d->staging.release();
  d->staging2.release();
  d->ws.release_all();
  if (d->host_mirror) hipHostFree(d->host_mirror);
  if (d->host_stage) hipHostFree(d->host_stage);
  if (d->own_stream) hipStreamDestroy(d->own_stream);
  delete d;
  return 0;
}

extern "C" int fmd_dec_set_stream(fmd_dec* d, void* s) {
  if (!d) return fmd_fail(FMD_ERR_ARG, "null handle");
  HIPCHK(hipStreamSynchronize(d->stream));
  d->stream = s ? (hipStream_t)s : d->own_stream;
  return 0;
}

extern "C" void* fmd_dec_stream(const fmd_dec* d) { return d ? (void*)d->stream : nullptr; }

// --- weights ---------------------------------------------------------------

static size_t dtype_size(int dt) { return dt == FMD_DT_F32 ? 4 : 2; }

// Bring a source tensor to the device (staging) and return its device pointer.
static int stage_source(fmd_dec* d, const void* data, int dt, size_t n, int on_dev,
                        const void** dev) {
  if (on_dev) {
    *dev = data;
    return 0;
  }
  CHK(d->staging.ensure(n * dtype_size(dt)));
  HIPCHK(hipMemcpyAsync(d->staging.p, data, n * dtype_size(dt), hipMemcpyHostToDevice, d->stream));
  *dev = d->staging.p;
  return 0;
}

// Write rows [row0, row0+rows) of a (possibly fused) linear.  Quantised linears
// read the f32 value of the source (the reference's f32 VarBuilder view,
// linear.rs:126-134); fused parts quantise into their own row range, which is
// identical to quantising the concatenation (blocks run along the input axis,
// linear.rs:217-219).
static int set_lin_rows(fmd_dec* d, Lin& l, int row0, int rows, const void* src_dev, int dt) {
  if (d->quant) {
    const float* f = (const float*)src_dev;
    if (dt != FMD_DT_F32) {
      CHK(d->staging2.ensure((size_t)rows * l.w.in * 4));
      if (launch_convert(ACT_F32, src_dev, dt, (int64_t)rows * l.w.in, d->staging2.p, d->stream) !=
          hipSuccess)
        return fmd_fail(FMD_ERR_HIP, "convert launch failed");
      f = (const float*)d->staging2.p;
    }
    if (launch_quantize_q8_0_tiles(f, rows, l.w.in, row0, l.w, d->stream) != hipSuccess)
      return fmd_fail(FMD_ERR_HIP, "quantize launch failed");
  } else {
    if (launch_pack_dense(d->act, src_dev, dt, rows, l.w.in, row0, l.w, d->stream) != hipSuccess)
      return fmd_fail(FMD_ERR_HIP, "pack launch failed");
  }
  return 0;
}

static int set_vec(fmd_dec* d, void* dst, const void* src_dev, int dt, size_t n) {
  if (launch_convert(d->act, src_dev, dt, (int64_t)n, dst, d->stream) != hipSuccess)
    return fmd_fail(FMD_ERR_HIP, "convert launch failed");
  return 0;
}

// Resolve a checkpoint name to (target, row range).  Names follow
// qwen3.rs:177-200, 268-286, 303-320, 354-376.
struct Target {
  enum Kind { NONE, LIN, VEC, EMBED, LMHEAD, NORM } kind = NONE;
  Lin* lin = nullptr;
  void** vec = nullptr;
  int row0 = 0, rows = 0, cols = 0, bit = 0, layer = -1;
};

static Target resolve(fmd_dec* d, const char* name) {
  Target t;
  std::string n(name);
  const std::string pfx = "model.language_model.";
  if (n.compare(0, pfx.size(), pfx) == 0) n = n.substr(pfx.size());
  if (n == "embed_tokens.weight") {
    t.kind = Target::EMBED;
    t.rows = d->V;
    t.cols = d->H;
    return t;
  }
  if (n == "lm_head.weight") {
    t.kind = Target::LMHEAD;
    t.lin = &d->lm_head;
    t.rows = d->V;
    t.cols = d->H;
    return t;
  }
  if (n == "norm.weight") {
    t.kind = Target::NORM;
    t.rows = 1;
    t.cols = d->H;
    return t;
  }
  int li = -1, used = 0;
  if (sscanf(n.c_str(), "layers.%d.%n", &li, &used) != 1 || li < 0 || li >= d->L || used == 0)
    return t;
  Layer& ly = d->layers[li];
  const std::string rest = n.substr(used);
  t.layer = li;
  struct Row { const char* nm; int bit; Lin* lin; void** vec; int row0, rows, cols; };
  const Row tab[] = {
      {"self_attn.q_proj.weight", 0, &ly.qkv, nullptr, 0, d->qd, d->H},
      {"self_attn.k_proj.weight", 1, &ly.qkv, nullptr, d->qd, d->kd, d->H},
      {"self_attn.v_proj.weight", 2, &ly.qkv, nullptr, d->qd + d->kd, d->kd, d->H},
      {"self_attn.o_proj.weight", 3, &ly.o, nullptr, 0, d->H, d->qd},
      {"mlp.gate_proj.weight", 4, &ly.gate_up, nullptr, 0, d->I, d->H},
      {"mlp.up_proj.weight", 5, &ly.gate_up, nullptr, d->I, d->I, d->H},
      {"mlp.down_proj.weight", 6, &ly.down, nullptr, 0, d->H, d->I},
      {"input_layernorm.weight", 7, nullptr, &ly.in_norm, 0, 1, d->H},
      {"post_attention_layernorm.weight", 8, nullptr, &ly.post_norm, 0, 1, d->H},
      {"self_attn.q_norm.weight", 9, nullptr, &ly.q_norm, 0, 1, d->hd},
      {"self_attn.k_norm.weight", 10, nullptr, &ly.k_norm, 0, 1, d->hd},
  };
  for (const Row& r : tab) {
    if (rest != r.nm) continue;
    t.kind = r.lin ? Target::LIN : Target::VEC;
    t.lin = r.lin;
    t.vec = r.vec;
    t.row0 = r.row0;
    t.rows = r.rows;
    t.cols = r.cols;
    t.bit = r.bit;
    return t;
  }
  return t;
}

extern "C" int fmd_dec_set_weight(fmd_dec* d, const char* name, fmd_dtype dtype,
                                  const int64_t* shape, int ndim, const void* data,
                                  int data_on_device) {
  if (!d || !name || !data || !shape) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (dtype < FMD_DT_F32 || dtype > FMD_DT_BF16) return fmd_fail(FMD_ERR_ARG, "bad dtype");
  HIPCHK(hipSetDevice(d->device));
  Target t = resolve(d, name);
  if (t.kind == Target::NONE) return fmd_fail(FMD_ERR_ARG, std::string("unknown tensor ") + name);
  int64_t numel = 1;
  for (int i = 0; i < ndim; ++i) numel *= shape[i];
  const bool vec_shape = ndim == 1 && shape[0] == t.cols;
  const bool mat_shape = ndim == 2 && shape[0] == t.rows && shape[1] == t.cols;
  if (!((t.rows == 1 && t.kind != Target::EMBED) ? vec_shape : mat_shape))
    return fmd_fail(FMD_ERR_ARG, std::string("shape mismatch for ") + name);
  const void* src = nullptr;
  CHK(stage_source(d, data, dtype, (size_t)numel, data_on_device, &src));
  switch (t.kind) {
    case Target::LIN:
      CHK(set_lin_rows(d, *t.lin, t.row0, t.rows, src, dtype));
      d->layers[t.layer].set |= 1u << t.bit;
      break;
    case Target::VEC:
      CHK(set_vec(d, *t.vec, src, dtype, (size_t)t.cols));
      d->layers[t.layer].set |= 1u << t.bit;
      break;
    case Target::NORM:
      CHK(set_vec(d, d->norm, src, dtype, (size_t)t.cols));
      d->norm_set = true;
      break;
    case Target::EMBED:
      CHK(set_vec(d, d->embed, src, dtype, (size_t)numel));
      d->embed_set = true;
      // build_tied_head (qwen3.rs:566-578): the output projection reuses the
      // embedding -- quantised from the f32 source in INT8, a dense copy otherwise.
      if (!d->lm_head_explicit) {
        CHK(set_lin_rows(d, d->lm_head, 0, d->V, src, dtype));
        d->lm_head_set = true;
      }
      break;
    case Target::LMHEAD:
      CHK(set_lin_rows(d, d->lm_head, 0, d->V, src, dtype));
      d->lm_head_explicit = true;
      d->lm_head_set = true;
      break;
    default: break;
  }
  HIPCHK(hipStreamSynchronize(d->stream));
  return 0;
}

extern "C" int fmd_dec_ready(const fmd_dec* d) {
  if (!d) return 0;
  for (const auto& ly : d->layers)
    if (ly.set != 0x7ffu) return 0;
  return d->embed_set && d->norm_set && d->lm_head_set ? 1 : 0;
}

extern "C" int fmd_dec_weight_bytes(const fmd_dec* d, size_t* out) {
  if (!d || !out) return fmd_fail(FMD_ERR_ARG, "null argument");
  size_t s = d->lm_head.wbytes + d->lm_head.sbytes;
  for (const auto& ly : d->layers)
    for (const Lin* l : {&ly.qkv, &ly.o, &ly.gate_up, &ly.down}) s += l->wbytes + l->sbytes;
  *out = s;
  return 0;
}

extern "C" int fmd_dec_get_q8_0(const fmd_dec* dc, const char* name, void* out_blocks) {
  fmd_dec* d = const_cast<fmd_dec*>(dc);
  if (!d || !name || !out_blocks) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (!d->quant) return fmd_fail(FMD_ERR_STATE, "model is not quantised");
  HIPCHK(hipSetDevice(d->device));
  Target t = resolve(d, name);
  Lin* l = t.lin;
  int row0 = t.row0, rows = t.rows;
  if (t.kind == Target::EMBED) {
    l = &d->lm_head;
    row0 = 0;
    rows = d->V;
  }
  if (!l) return fmd_fail(FMD_ERR_ARG, std::string("not a quantised projection: ") + name);
  const size_t bytes = (size_t)rows * (l->w.in / 32) * 34;
  CHK(d->staging.ensure(bytes));
  if (launch_unpack_q8_0(l->w, row0, rows, (uint8_t*)d->staging.p, d->stream) != hipSuccess)
    return fmd_fail(FMD_ERR_HIP, "unpack launch failed");
  HIPCHK(hipMemcpyAsync(out_blocks, d->staging.p, bytes, hipMemcpyDeviceToHost, d->stream));
  HIPCHK(hipStreamSynchronize(d->stream));
  return 0;
}

// --- KV cache ----------------------------------------------------------------

extern "C" size_t fmd_kv_bytes(const fmd_dec* d, int batch, int capacity) {
  if (!d) return 0;
  // KvCache::bytes_per_layer (qwen3.rs:70-78) x layers.
  return (size_t)d->L * 2 * batch * d->nkv * (size_t)capacity * d->hd * d->esz;
}

extern "C" int fmd_kv_create(fmd_dec* d, int batch, int capacity, fmd_kv** out) {
  if (!d || !out) return fmd_fail(FMD_ERR_ARG, "null argument");
  *out = nullptr;
  if (batch <= 0 || capacity <= 0) return fmd_fail(FMD_ERR_ARG, "batch and capacity must be > 0");
  if (capacity > kMaxCapacity)
    return fmd_fail(FMD_ERR_ARG, "capacity above 65536 positions is not supported");
  HIPCHK(hipSetDevice(d->device));
  fmd_kv* kv = new fmd_kv();
  kv->dec = d;
  kv->batch = batch;
  kv->cap = capacity;
  kv->layer_bytes = (size_t)batch * d->nkv * capacity * d->hd * d->esz;
  kv->k.assign(d->L, nullptr);
  kv->v.assign(d->L, nullptr);
  int rc = 0;
  for (int l = 0; l < d->L && !rc; ++l) {
    if (hipMalloc(&kv->k[l], kv->layer_bytes) != hipSuccess ||
        hipMalloc(&kv->v[l], kv->layer_bytes) != hipSuccess) {
      rc = fmd_fail(FMD_ERR_OOM, "kv cache allocation failed");
      break;
    }
    if (hipMemsetAsync(kv->k[l], 0, kv->layer_bytes, d->stream) != hipSuccess ||
        hipMemsetAsync(kv->v[l], 0, kv->layer_bytes, d->stream) != hipSuccess)
      rc = fmd_fail(FMD_ERR_HIP, "kv memset failed");
  }
  if (!rc && hipMalloc((void**)&kv->state, 16 * sizeof(int32_t)) != hipSuccess)
    rc = fmd_fail(FMD_ERR_OOM, "state allocation failed");
  if (!rc && hipMemsetAsync(kv->state, 0, 16 * sizeof(int32_t), d->stream) != hipSuccess)
    rc = fmd_fail(FMD_ERR_HIP, "memset failed");
  if (!rc && hipStreamSynchronize(d->stream) != hipSuccess) rc = fmd_fail(FMD_ERR_HIP, "sync failed");
  if (rc) {
    std::string keep = g_err;
    fmd_kv_destroy(kv);
    g_err = keep;
    return rc;
  }
  *out = kv;
  return 0;
}

extern "C" int fmd_kv_destroy(fmd_kv* kv) {
  if (!kv) return 0;
  hipSetDevice(kv->dec->device);
  hipStreamSynchronize(kv->dec->stream);
  // the decoder's whole-layer table points at this cache's buffers: drop it
  // (a later cache may be allocated at this handle's address)
  for (void* p : kv->k)
    if (p) hipFree(p);
  for (void* p : kv->v)
    if (p) hipFree(p);
  if (kv->state) hipFree(kv->state);
  delete kv;
  return 0;
}

int kv_sync_state(fmd_kv* kv) {
  // state[0] = length (write cursor), [1] = greedy step, [2] = rows done.
  int32_t st[4] = {kv->len, 0, 0, 0};
  HIPCHK(hipMemcpyAsync(kv->state, st, sizeof st, hipMemcpyHostToDevice, kv->dec->stream));
  return 0;
}

extern "C" int fmd_kv_len(const fmd_kv* kv) { return kv ? kv->len : -1; }

extern "C" int fmd_kv_truncate(fmd_kv* kv, int len) {
  if (!kv) return fmd_fail(FMD_ERR_ARG, "null handle");
  kv->len = std::min(kv->len, std::max(len, 0));
  CHK(kv_sync_state(kv));
  HIPCHK(hipStreamSynchronize(kv->dec->stream));
  return 0;
}

extern "C" int fmd_kv_set_len(fmd_kv* kv, int len) {
  if (!kv) return fmd_fail(FMD_ERR_ARG, "null handle");
  if (len < 0 || len > kv->cap) return fmd_fail(FMD_ERR_ARG, "length outside the capacity");
  kv->len = len;
  CHK(kv_sync_state(kv));
  HIPCHK(hipStreamSynchronize(kv->dec->stream));
  return 0;
}

extern "C" int fmd_kv_read(const fmd_kv* kv, int layer, int which, void* out) {
  if (!kv || !out || layer < 0 || layer >= kv->dec->L) return fmd_fail(FMD_ERR_ARG, "bad argument");
  HIPCHK(hipSetDevice(kv->dec->device));
  HIPCHK(hipMemcpyAsync(out, which ? kv->v[layer] : kv->k[layer], kv->layer_bytes,
                        hipMemcpyDeviceToHost, kv->dec->stream));
  HIPCHK(hipStreamSynchronize(kv->dec->stream));
  return 0;
}

extern "C" int fmd_kv_write(fmd_kv* kv, int layer, int which, const void* src) {
  if (!kv || !src || layer < 0 || layer >= kv->dec->L) return fmd_fail(FMD_ERR_ARG, "bad argument");
  HIPCHK(hipSetDevice(kv->dec->device));
  HIPCHK(hipMemcpyAsync(which ? kv->v[layer] : kv->k[layer], src, kv->layer_bytes,
                        hipMemcpyHostToDevice, kv->dec->stream));
  HIPCHK(hipStreamSynchronize(kv->dec->stream));
  return 0;
}

extern "C" int fmd_kv_fill_random(fmd_kv* kv, uint64_t seed, int len) {
  if (!kv) return fmd_fail(FMD_ERR_ARG, "null handle");
  if (len < 0 || len > kv->cap) return fmd_fail(FMD_ERR_ARG, "length outside the capacity");
  fmd_dec* d = kv->dec;
  HIPCHK(hipSetDevice(d->device));
  const int64_t n = (int64_t)(kv->layer_bytes / d->esz);
  for (int l = 0; l < d->L; ++l) {
    if (launch_fill_normal(d->act, kv->k[l], n, seed * 1000003ull + 2 * l, 1.0f, d->stream) != hipSuccess ||
        launch_fill_normal(d->act, kv->v[l], n, seed * 1000003ull + 2 * l + 1, 1.0f, d->stream) != hipSuccess)
      return fmd_fail(FMD_ERR_HIP, "fill launch failed");
  }
  kv->len = len;
  CHK(kv_sync_state(kv));
  HIPCHK(hipStreamSynchronize(d->stream));
  return 0;
}

extern "C" int fmd_quantize_q8_0(const float* src, int64_t rows, int64_t cols, void* out) {
  if (!src || !out || rows < 0 || cols % 32) return fmd_fail(FMD_ERR_ARG, "bad argument");
  host_quantize_q8_0(src, rows, cols, (uint8_t*)out);
  return 0;
}
