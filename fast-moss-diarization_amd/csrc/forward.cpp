// Forward passes: chunked prefill (qwen3.rs:475-496), decode step
// (qwen3.rs:499-511), and the device-resident greedy loop of
// Engine::generate_batch (engine.rs:463-541).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "fmd_dec.h"
#include "fmd_internal.h"
#include "fmd_kernels.h"

int attn_prefill_tile_rows(int rep);

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

constexpr int kMaxDecodeRows = 16;

float act_scale(const fmd_dec* d) {
  // scores * scale runs in the activation dtype (qwen3.rs:243).
  return host_round_act(d->scale, d->act);
}

// Split plan of decode attention for a cache of `cap` positions.
AttnDecodePlan split_geom(const fmd_dec* d, int B, int cap) {
  return attn_decode_plan(d->act, d->rep, cap, B * d->nkv);
}

// Score words per (unit, head) of the single-launch attention kernel.
int xsc_stride(const AttnDecodePlan& pl) { return pl.max_splits * pl.split / 2 + 1; }

// Error code left by a single-launch attention wait that gave up (the
// work-groups of a unit did not all run within the spin limit, e.g. while
// another kernel held the device); read after the streams are synchronised.
int check_attn_sync(fmd_dec* d) {
  DecodeLane& ln = d->ws.dec;
  if (!ln.xsync.p) return 0;
  uint32_t code = 0;
  HIPCHK(hipMemcpy(&code, ln.xsync.as<uint32_t>() + 2, 4, hipMemcpyDeviceToHost));
  if (!code) return 0;
  const uint32_t zero = 0;
  HIPCHK(hipMemcpy(ln.xsync.as<uint32_t>() + 2, &zero, 4, hipMemcpyHostToDevice));
  return fmd_fail(FMD_ERR_HIP, "decode attention: work-groups of one (row, KV head) did not meet "
                               "within the spin limit (code " + std::to_string(code) + ")");
}

// Attention of `layer` for the B rows of the cache on the decode buffers.
AttnDecodeArgs attn_args(fmd_dec* d, fmd_kv* kv, int layer, int B, const void* qkv,
                         const int32_t* pad_dev, const int32_t* state, const int32_t* done_dev,
                         void* out) {
  const AttnDecodePlan sg = split_geom(d, B, kv->cap);
  const Layer& ly = d->layers[layer];
  DecodeLane& ln = d->ws.dec;
  AttnDecodeArgs a{};
  a.qkv = qkv;
  a.ldqkv = d->qkvd;
  a.qn_w = ly.q_norm;
  a.kn_w = ly.k_norm;
  a.cos = d->cos;
  a.sin = d->sin;
  a.eps = d->eps;
  a.kc = kv->k[layer];
  a.vc = kv->v[layer];
  a.cap = kv->cap;
  a.nkv = d->nkv;
  a.rep = d->rep;
  a.batch = B;
  a.start = pad_dev;
  a.state = state;
  a.done = done_dev;
  a.scores = ln.scores.p;
  a.ml = ln.attn_ml.as<float>();
  a.part = ln.attn_part.as<float>();
  a.max_splits = sg.max_splits;
  a.split = sg.split;
  a.out = out;
  a.scale = host_round_act(d->scale, d->act);  // scores * scale in the dtype (qwen3.rs:243)
  a.fused = sg.fused;
  a.sync = ln.xsync.as<uint32_t>();
  a.xml = ln.xml.as<uint64_t>();
  a.xpart = ln.xpart.as<uint64_t>();
  a.xsc = ln.xsc.as<uint64_t>();
  a.xsc_stride = xsc_stride(sg);
  a.xnew = ln.xnew.as<uint64_t>();
  a.spin_limit = d->spin_limit;
  a.count_units = 1;
  return a;
}

// The decode buffers for up to B rows over a cache of capacity cap.
int ensure_lane(fmd_dec* d, DecodeLane& w, int B, int cap) {
  CHK(w.qkv.ensure((size_t)B * d->qkvd * d->esz));
  CHK(w.ctx.ensure((size_t)B * d->qd * d->esz));
  CHK(w.act.ensure((size_t)B * d->I * d->esz));
  const AttnDecodePlan plan = split_geom(d, B, cap);
  const size_t units = (size_t)B * d->nkv * plan.max_splits * d->rep;
  CHK(w.attn_part.ensure(units * d->hd * 4));
  CHK(w.attn_ml.ensure(units * 2 * 4));
  if (plan.fused) {
    // Exchange words start at epoch 0 and the launch epoch at 1, so no word
    // is valid before a launch writes it.  The state block is sized for the
    // largest batch once; every (re)allocated exchange buffer is cleared --
    // its memory may hold another handle's words, whose epochs count from 1
    // too.
    bool fresh_sync = false, f_ml = false, f_part = false, f_sc = false, f_new = false, f_qkv = false;
    CHK(w.xsync.ensure((size_t)(4 + kMaxDecodeRows * d->nkv) * 4, &fresh_sync));
    CHK(w.xml.ensure(units * 2 * 8, &f_ml));
    CHK(w.xpart.ensure(units * d->hd * 8, &f_part));
    CHK(w.xsc.ensure((size_t)B * d->nkv * d->rep * xsc_stride(plan) * 8, &f_sc));
    CHK(w.xnew.ensure((size_t)B * d->nkv * d->rep * 8, &f_new));
    CHK(w.xqkv.ensure((size_t)B * (d->qkvd / 2) * 8, &f_qkv));
    if (fresh_sync || f_qkv) HIPCHK(hipMemsetAsync(w.xqkv.p, 0, w.xqkv.n, d->stream));
    if (fresh_sync || f_ml) HIPCHK(hipMemsetAsync(w.xml.p, 0, w.xml.n, d->stream));
    if (fresh_sync || f_part) HIPCHK(hipMemsetAsync(w.xpart.p, 0, w.xpart.n, d->stream));
    if (fresh_sync || f_sc) HIPCHK(hipMemsetAsync(w.xsc.p, 0, w.xsc.n, d->stream));
    if (fresh_sync || f_new) HIPCHK(hipMemsetAsync(w.xnew.p, 0, w.xnew.n, d->stream));
    if (fresh_sync) {
      HIPCHK(hipMemsetAsync(w.xsync.p, 0, w.xsync.n, d->stream));
      const uint32_t one = 1;
      HIPCHK(hipMemcpyAsync(w.xsync.p, &one, 4, hipMemcpyHostToDevice, d->stream));
      HIPCHK(hipStreamSynchronize(d->stream));
    }
  }
  CHK(w.scores.ensure((size_t)B * d->nh * cap * d->esz));
  return 0;
}

// Decode workspaces for `B` rows over a cache of capacity `cap`: the
// residual stream, logits, argmax keys, ids, pads and the decode buffers.
int ensure_decode_ws(fmd_dec* d, int B, int cap) {
  Workspace& w = d->ws;
  CHK(w.x.ensure((size_t)B * d->H * d->esz));
  CHK(w.logits.ensure((size_t)B * d->V * 4));
  CHK(w.amax.ensure((size_t)gemv_logits_nparts(d->act, d->quant, true, d->H, d->V) * B * 8));
  CHK(ensure_lane(d, w.dec, B, cap));
  CHK(w.ids.ensure((size_t)B * 4));
  CHK(w.pad.ensure((size_t)B * 4));
  CHK(w.opstate.ensure(64));
  if (!d->host_mirror) {
    HIPCHK(hipHostMalloc((void**)&d->host_mirror, 64, hipHostMallocMapped | hipHostMallocCoherent));
    std::memset(d->host_mirror, 0, 64);
  }
  return 0;
}

// The single-launch attention also runs the qkv projection (16-bit
// activations, hidden a multiple of 256 up to 1024).
bool qkv_in_attention(const fmd_dec* d, const AttnDecodeArgs& a, const DecodeLane& ln) {
  return a.fused && d->act != ACT_F32 && d->H % 256 == 0 && d->H <= 1024 && d->qkvd % 16 == 0 &&
         ln.xqkv.p != nullptr;
}

GemvArgs gemv_args(const void* x, int ldx, const void* norm, float eps, const LinWeights& W,
                   int rows, void* y, int ldy, const void* resid, uint64_t* amax) {
  GemvArgs g{};
  g.x = x;
  g.ldx = ldx;
  g.norm_w = norm;
  g.eps = eps;
  g.W = W;
  g.rows = rows;
  g.y = y;
  g.ldy = ldy;
  g.resid = resid;
  g.amax_part = amax;
  return g;
}

// Decoder layer `l` of a decode step for B <= 16 rows (Layer::forward,
// qwen3.rs:322-339): the qkv projection (inside the attention launch for
// 16-bit activations), the attention with the q/k norm, RoPE and cache
// append, then O + residual, RMSNorm + gate|up + SwiGLU, down + residual.
// The residual stream is ws.x; the write position is kv->state[0].
int decode_layer(fmd_dec* d, fmd_kv* kv, int l, int B, const int32_t* pad_dev,
                 const int32_t* done_dev, hipStream_t s) {
  Workspace& w = d->ws;
  DecodeLane& ln = w.dec;
  const int act = d->act;
  Layer& ly = d->layers[l];
  void* x = w.x.p;
  AttnDecodeArgs a = attn_args(d, kv, l, B, ln.qkv.p, pad_dev, kv->state, done_dev, ln.ctx.p);
  if (qkv_in_attention(d, a, ln)) {
    a.nq = d->qkvd / 16;
    a.x = x;
    a.ldx = d->H;
    a.hidden = d->H;
    a.norm_w = ly.in_norm;
    a.Wqkv = ly.qkv.w;
    a.xqkv = ln.xqkv.as<uint64_t>();
  } else {
    LAUNCH(launch_gemv(act, EPI_STORE, true,
                       gemv_args(x, d->H, ly.in_norm, d->eps, ly.qkv.w, B, ln.qkv.p, d->qkvd,
                                 nullptr, nullptr),
                       s));
  }
  // The O projection right after the single-launch attention advances its
  // epoch (its first thread runs once every attention work-group has ended).
  GemvArgs go = gemv_args(ln.ctx.p, d->qd, nullptr, d->eps, ly.o.w, B, x, d->H, x, nullptr);
  if (a.fused && act != ACT_F32) {
    a.count_units = 0;
    go.epoch = a.sync;
  }
  LAUNCH(launch_attn_decode(act, a, s));
  LAUNCH(launch_gemv(act, EPI_RESID, false, go, s));
  LAUNCH(launch_gemv(act, EPI_SWIGLU, true,
                     gemv_args(x, d->H, ly.post_norm, d->eps, ly.gate_up.w, B, ln.act.p, d->I,
                               nullptr, nullptr),
                     s));
  LAUNCH(launch_gemv(act, EPI_RESID, false,
                     gemv_args(ln.act.p, d->I, nullptr, d->eps, ly.down.w, B, x, d->H, x, nullptr),
                     s));
  return 0;
}

// Final RMSNorm fused into the lm_head projection (qwen3.rs:455, 459-463):
// f32 logits of `rows` rows of x plus the per-work-group argmax keys.
int launch_logits(fmd_dec* d, const void* x, int rows, float* logits, hipStream_t s) {
  LAUNCH(launch_gemv(d->act, EPI_LOGITS, true,
                     gemv_args(x, d->H, d->norm, d->eps, d->lm_head.w, rows, logits, d->V, nullptr,
                               d->ws.amax.as<uint64_t>()),
                     s));
  return 0;
}

// One decode step for B <= 16 rows: every decoder layer, then the final norm
// fused into the lm_head projection (f32 logits + argmax keys).  Reads the
// write position from kv->state[0].
int decode_layers(fmd_dec* d, fmd_kv* kv, int B, const int32_t* pad_dev, const int32_t* done_dev,
                  hipStream_t s) {
  for (int l = 0; l < d->L; ++l) CHK(decode_layer(d, kv, l, B, pad_dev, done_dev, s));
  return launch_logits(d, d->ws.x.p, B, d->ws.logits.as<float>(), s);
}

int check_common(fmd_dec* d, fmd_kv* kv, int batch) {
  if (!d || !kv) return fmd_fail(FMD_ERR_ARG, "null handle");
  if (kv->dec != d) return fmd_fail(FMD_ERR_STATE, "cache belongs to another decoder");
  if (!fmd_dec_ready(d)) return fmd_fail(FMD_ERR_STATE, "decoder weights are incomplete");
  if (batch != kv->batch) return fmd_fail(FMD_ERR_ARG, "batch does not match the cache");
  return 0;
}

int overflow(const fmd_kv* kv, int t) {
  return fmd_fail(FMD_ERR_OVERFLOW, "kv cache overflow: " + std::to_string(kv->len) + " + " +
                                        std::to_string(t) + " exceeds capacity " +
                                        std::to_string(kv->cap));
}

// Device state for a greedy run: flags, counters, token buffer, forced steps.
int setup_greedy(fmd_dec* d, fmd_kv* kv, int B, int budget, const int32_t* force) {
  Workspace& w = d->ws;
  CHK(w.done.ensure((size_t)B * 4));
  CHK(w.ntok.ensure((size_t)B * 4));
  CHK(w.finish.ensure((size_t)B * 4));
  CHK(w.tokens.ensure((size_t)B * std::max(budget, 1) * 4));
  CHK(w.force.ensure((size_t)B * 4));
  HIPCHK(hipMemsetAsync(w.done.p, 0, (size_t)B * 4, d->stream));
  HIPCHK(hipMemsetAsync(w.ntok.p, 0, (size_t)B * 4, d->stream));
  HIPCHK(hipMemsetAsync(w.finish.p, 0, (size_t)B * 4, d->stream));
  if (force)
    HIPCHK(hipMemcpyAsync(w.force.p, force, (size_t)B * 4, hipMemcpyHostToDevice, d->stream));
  CHK(kv_sync_state(kv));
  std::memset(d->host_mirror, 0, 64);
  return 0;
}

GreedyArgs greedy_args(fmd_dec* d, fmd_kv* kv, int B, int budget, bool use_force, uint32_t eos,
                       int advance) {
  Workspace& w = d->ws;
  GreedyArgs g{};
  g.part = w.amax.as<uint64_t>();
  g.nparts = gemv_logits_nparts(d->act, d->quant, true, d->H, d->V);
  g.batch = B;
  g.state = kv->state;
  g.host_state = d->host_mirror;
  g.advance = advance;
  g.done = w.done.as<int32_t>();
  g.ntok = w.ntok.as<int32_t>();
  g.finish = w.finish.as<int32_t>();
  g.tokens = w.tokens.as<uint32_t>();
  g.budget = budget;
  g.force = use_force ? w.force.as<int32_t>() : nullptr;
  g.eos = eos;
  g.next_ids = w.ids.as<uint32_t>();
  g.embed = d->embed;
  g.x = w.x.p;
  g.hidden = d->H;
  g.vocab = d->V;
  return g;
}

template <class F>
int capture(hipStream_t s, hipGraphExec_t* out, F&& body) {
  hipGraph_t graph = nullptr;
  HIPCHK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  int rc = body();
  hipError_t e = hipStreamEndCapture(s, &graph);
  if (rc) {
    if (graph) hipGraphDestroy(graph);
    return rc;
  }
  if (e != hipSuccess) return fmd_fail(FMD_ERR_HIP, std::string("graph capture: ") + hipGetErrorString(e));
  e = hipGraphInstantiate(out, graph, nullptr, nullptr, 0);
  hipGraphDestroy(graph);
  if (e != hipSuccess) return fmd_fail(FMD_ERR_HIP, std::string("graph instantiate: ") + hipGetErrorString(e));
  return 0;
}

// Launch up to `max_steps` (decode step + greedy update) pairs, as one
// captured HIP graph replayed per step.  The host keeps at most two steps in
// flight and stops once every row is done.
int run_decode_steps(fmd_dec* d, fmd_kv* kv, int B, int max_steps, int budget, bool use_force,
                     uint32_t eos, int* steps_run) {
  hipStream_t s = d->stream;
  const int32_t* pad_dev = d->ws.pad.as<int32_t>();
  const int32_t* done_dev = d->ws.done.as<int32_t>();
  const GreedyArgs g = greedy_args(d, kv, B, budget, use_force, eos, 1);
  *steps_run = 0;
  HIPCHK(hipStreamSynchronize(s));
  volatile int32_t* mirror = d->host_mirror;
  if (mirror[2] >= B || max_steps <= 0) return 0;

  struct Exec {
    hipGraphExec_t e = nullptr;
    ~Exec() {
      if (e) hipGraphExecDestroy(e);
    }
  } graph;
  CHK(capture(s, &graph.e, [&]() {
    CHK(decode_layers(d, kv, B, pad_dev, done_dev, s));
    return launch_greedy(d->act, g, s) != hipSuccess ? fmd_fail(FMD_ERR_HIP, "greedy launch failed") : 0;
  }));
  hipEvent_t ev[2];
  HIPCHK(hipEventCreateWithFlags(&ev[0], hipEventDisableTiming));
  HIPCHK(hipEventCreateWithFlags(&ev[1], hipEventDisableTiming));
  int rc = 0;
  for (int step = 0; step < max_steps; ++step) {
    if (step >= 2) {
      if (hipEventSynchronize(ev[step & 1]) != hipSuccess) {
        rc = fmd_fail(FMD_ERR_HIP, "event sync failed");
        break;
      }
      if (mirror[2] >= B) break;
    }
    if (hipGraphLaunch(graph.e, s) != hipSuccess) {
      rc = fmd_fail(FMD_ERR_HIP, "graph launch failed");
      break;
    }
    if (hipEventRecord(ev[step & 1], s) != hipSuccess) {
      rc = fmd_fail(FMD_ERR_HIP, "event record failed");
      break;
    }
    *steps_run += 1;
  }
  hipError_t e = hipStreamSynchronize(s);
  hipEventDestroy(ev[0]);
  hipEventDestroy(ev[1]);
  if (!rc && e != hipSuccess) rc = fmd_fail(FMD_ERR_HIP, std::string("decode loop: ") + hipGetErrorString(e));
  if (!rc) rc = check_attn_sync(d);
  kv->len += *steps_run;
  return rc;
}

int copy_greedy_out(fmd_dec* d, int B, int budget, uint32_t* tokens, int32_t* ntok,
                    int32_t* finish) {
  Workspace& w = d->ws;
  if (tokens)
    HIPCHK(hipMemcpyAsync(tokens, w.tokens.p, (size_t)B * budget * 4, hipMemcpyDeviceToHost, d->stream));
  if (ntok) HIPCHK(hipMemcpyAsync(ntok, w.ntok.p, (size_t)B * 4, hipMemcpyDeviceToHost, d->stream));
  if (finish)
    HIPCHK(hipMemcpyAsync(finish, w.finish.p, (size_t)B * 4, hipMemcpyDeviceToHost, d->stream));
  HIPCHK(hipStreamSynchronize(d->stream));
  return 0;
}

}  // namespace

// ---------------------------------------------------------------------------

extern "C" int fmd_dec_embed(fmd_dec* d, const uint32_t* ids, int64_t n, void* out) {
  if (!d || (!ids && n) || (!out && n)) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (n <= 0) return 0;
  HIPCHK(hipSetDevice(d->device));
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] >= (uint32_t)d->V) return fmd_fail(FMD_ERR_ARG, "token id out of range");
  CHK(d->ws.ids.ensure((size_t)n * 4));
  CHK(d->ws.embeds.ensure((size_t)n * d->H * d->esz));
  HIPCHK(hipMemcpyAsync(d->ws.ids.p, ids, (size_t)n * 4, hipMemcpyHostToDevice, d->stream));
  LAUNCH(launch_embed(d->act, d->ws.ids.as<uint32_t>(), (int)n, d->embed, d->H, d->ws.embeds.p, d->stream));
  HIPCHK(hipMemcpyAsync(out, d->ws.embeds.p, (size_t)n * d->H * d->esz, hipMemcpyDeviceToHost, d->stream));
  HIPCHK(hipStreamSynchronize(d->stream));
  return 0;
}

extern "C" int fmd_dec_assemble(fmd_dec* d, const uint32_t* ids, const int64_t* offsets, int batch,
                                const void* audio, int audio_dtype, int audio_on_device,
                                int64_t n_audio, const int64_t* audio_first,
                                const int64_t* audio_count, uint32_t audio_token_id, int total,
                                void* out, int32_t* pad) {
  if (!d || !offsets || !out || batch <= 0 || total <= 0)
    return fmd_fail(FMD_ERR_ARG, "null argument or empty batch");
  if (audio_dtype < 0 || audio_dtype > 2) return fmd_fail(FMD_ERR_ARG, "unknown audio dtype");
  if (n_audio < 0 || (n_audio > 0 && !audio) || n_audio > (int64_t)INT32_MAX - 2)
    return fmd_fail(FMD_ERR_ARG, "bad audio rows");
  if ((int64_t)batch * total > (int64_t)INT32_MAX) return fmd_fail(FMD_ERR_ARG, "prompt block too large");
  HIPCHK(hipSetDevice(d->device));
  // src per output row: token id, -1 for the left pad, -2 - r for audio row r
  std::vector<int32_t> src((size_t)batch * total, -1);
  std::vector<int32_t> pads(batch);
  for (int b = 0; b < batch; ++b) {
    const int64_t s0 = offsets[b], s1 = offsets[b + 1], len = s1 - s0;
    if (s0 < 0 || len < 0) return fmd_fail(FMD_ERR_ARG, "offsets must be non-decreasing from 0");
    if (len > 0 && !ids) return fmd_fail(FMD_ERR_ARG, "null ids");
    if (len > total) return fmd_fail(FMD_ERR_ARG, "prompt longer than the assembled length");
    int64_t slots = 0;
    for (int64_t i = s0; i < s1; ++i) slots += ids[i] == audio_token_id;
    const int64_t first = audio_first ? audio_first[b] : 0;
    const int64_t count = audio_count ? audio_count[b] : 0;
    if (slots != count)   // mod.rs:145-150
      return fmd_fail(FMD_ERR_ARG, "prompt has " + std::to_string(slots) +
                                       " audio placeholders but the encoder produced " +
                                       std::to_string(count) + " embeddings");
    if (count > 0 && (first < 0 || first + count > n_audio))
      return fmd_fail(FMD_ERR_ARG, "audio rows out of range");
    pads[b] = (int32_t)(total - len);
    int64_t used = 0;
    for (int64_t i = 0; i < len; ++i) {
      const uint32_t id = ids[s0 + i];
      int32_t& v = src[(size_t)b * total + pads[b] + i];
      if (id == audio_token_id) {
        v = (int32_t)(-2 - (first + used++));
      } else {
        if (id >= (uint32_t)d->V) return fmd_fail(FMD_ERR_ARG, "token id out of range");
        v = (int32_t)id;
      }
    }
  }
  const size_t rows = (size_t)batch * total;
  CHK(d->ws.asrc.ensure(rows * 4));
  HIPCHK(hipMemcpyAsync(d->ws.asrc.p, src.data(), rows * 4, hipMemcpyHostToDevice, d->stream));
  const void* audio_dev = audio;
  if (n_audio > 0 && !audio_on_device) {
    const size_t bytes = (size_t)n_audio * d->H * (audio_dtype == 0 ? 4 : 2);
    CHK(d->ws.audio.ensure(bytes));
    HIPCHK(hipMemcpyAsync(d->ws.audio.p, audio, bytes, hipMemcpyHostToDevice, d->stream));
    audio_dev = d->ws.audio.p;
  }
  LAUNCH(launch_assemble(d->act, d->ws.asrc.as<int32_t>(), (int)rows, d->embed, audio_dev,
                         audio_dtype, d->H, out, d->stream));
  HIPCHK(hipStreamSynchronize(d->stream));
  if (pad) std::copy(pads.begin(), pads.end(), pad);
  return 0;
}

namespace {

// Chunked prefill over real (non-pad) rows; leaves the last rows' logits and
// argmax keys in the workspace.  `emb_dev` is (B, total, H) on the device.
int prefill_impl(fmd_dec* d, fmd_kv* kv, const void* emb_dev, const int32_t* pad, int B, int total,
                 int chunk) {
  Workspace& w = d->ws;
  hipStream_t s = d->stream;
  const int act = d->act;
  const int QT = attn_prefill_tile_rows(d->rep);
  const int maxM = B * std::min(chunk, total);
  CHK(ensure_decode_ws(d, std::min(B, kMaxDecodeRows), kv->cap));
  CHK(w.x.ensure((size_t)(maxM + 1) * d->H * d->esz));
  CHK(w.xn.ensure((size_t)maxM * std::max(d->H, d->I) * d->esz));
  CHK(w.qkv.ensure((size_t)maxM * d->qkvd * d->esz));
  CHK(w.q.ensure((size_t)maxM * d->qd * d->esz));
  CHK(w.ctx.ensure((size_t)maxM * d->qd * d->esz));
  CHK(w.act.ensure((size_t)maxM * d->I * d->esz));
  CHK(w.lastx.ensure((size_t)B * d->H * d->esz));
  const int maxTiles = B * ((std::min(chunk, total) + QT - 1) / QT + 1);
  // items: each tile's keys cut into pieces of `split` keys (a multiple of
  // 64), sized per chunk so that about kItemsPerHead pieces per KV head share
  // the chunk's attention work; at most maxTiles + kItemsPerHead of them.
  // Measured on a full chunk of the 8-prompt workload (4096 rows at
  // positions 7168-7679, 1500-8000-token prompts), passes + combine: 96
  // pieces per head 474.6 us, 128 460.2, 192 443.0, 256 457.7, 384 472.2
  // (fewer pieces leave the longest piece's work-group as the tail; more make
  // the combine grow).
  const int kItemsPerHead = 192 * 64 / QT;
  const int maxItems = maxTiles + kItemsPerHead + 1;
  CHK(w.rowmeta.ensure((size_t)maxM * 3 * 4 + (size_t)B * 4 + 64));
  CHK(w.tiles.ensure((size_t)(6 * maxTiles + 4 * maxItems) * 4 + 64));
  if (act != ACT_F32) {
    CHK(w.pml.ensure((size_t)maxItems * d->nkv * QT * d->rep * 2 * 4));
    CHK(w.po.ensure((size_t)maxItems * d->nkv * QT * d->rep * d->hd * 4));
  }
  CHK(w.pad.ensure((size_t)B * 4));
  HIPCHK(hipMemcpyAsync(w.pad.p, pad, (size_t)B * 4, hipMemcpyHostToDevice, s));

  // The chunk tables are built in two pinned host slots, used alternately,
  // so their uploads are asynchronous and the host prepares chunk c + 1
  // while the device runs chunk c.  A slot is rewritten only once the event
  // recorded behind its previous uploads has passed.
  const size_t meta_n = (size_t)maxM * 3 + B, tiles_n = (size_t)6 * maxTiles + 4 * maxItems;
  const size_t slot_bytes = (meta_n + tiles_n) * 4;
  if (d->host_stage_n < 2 * slot_bytes) {
    if (d->host_stage) {
      HIPCHK(hipStreamSynchronize(s));
      HIPCHK(hipHostFree(d->host_stage));
      d->host_stage = nullptr;
      d->host_stage_n = 0;
    }
    HIPCHK(hipHostMalloc(&d->host_stage, 2 * slot_bytes, hipHostMallocDefault));
    std::memset(d->host_stage, 0, 2 * slot_bytes);
    d->host_stage_n = 2 * slot_bytes;
  }
  struct StageEvents {
    hipEvent_t ev[2] = {nullptr, nullptr};
    ~StageEvents() {
      for (hipEvent_t e : ev)
        if (e) {
          hipEventSynchronize(e);  // the slots outlive this call
          hipEventDestroy(e);
        }
    }
  } stage;
  HIPCHK(hipEventCreateWithFlags(&stage.ev[0], hipEventDisableTiming));
  HIPCHK(hipEventCreateWithFlags(&stage.ev[1], hipEventDisableTiming));
  std::vector<int> last_row(B, -1);
  const int32_t* dmeta = w.rowmeta.as<int32_t>();
  const int32_t* dtiles = w.tiles.as<int32_t>();

  for (int start = 0, c = 0; start < total; start += chunk, ++c) {
    const int len = std::min(chunk, total - start);
    if (c >= 2) HIPCHK(hipEventSynchronize(stage.ev[c & 1]));
    int32_t* meta = (int32_t*)d->host_stage + (size_t)(c & 1) * (meta_n + tiles_n);
    int32_t* tiles = meta + meta_n;
    int32_t* row_b = meta;
    int32_t* row_pos = row_b + maxM;
    int32_t* row_src = row_pos + maxM;
    int32_t* lastsel = row_src + maxM;
    int M = 0, nt = 0;
    for (int b = 0; b < B; ++b) {
      const int lo = std::max(start, pad[b]), hi = start + len;
      for (int p0 = lo; p0 < hi; p0 += QT) {
        tiles[nt] = b;
        tiles[maxTiles + nt] = M + (p0 - lo);
        tiles[2 * maxTiles + nt] = p0;
        tiles[3 * maxTiles + nt] = std::min(QT, hi - p0);
        ++nt;
      }
      for (int p = lo; p < hi; ++p) {
        row_b[M] = b;
        row_pos[M] = p;
        row_src[M] = b * total + p;
        if (p == total - 1) last_row[b] = M;
        ++M;
      }
    }
    if (M == 0) continue;
    // Items: split every tile's keys [pad_b, pos0 + n) into pieces of
    // `split` keys, with `split` chosen so the chunk's key blocks spread over
    // about kItemsPerHead items per KV head.  When every tile fits in one
    // piece (short prompts), one launch runs both softmax passes.
    int nitems = 0;
    {
      long blocks = 0;
      for (int t = 0; t < nt; ++t)
        blocks += (tiles[2 * maxTiles + t] + tiles[3 * maxTiles + t] - pad[tiles[t]] + 63) / 64;
      // items per tile <= its blocks / split_blocks + 1, so nitems <= nt + kItemsPerHead
      const long split_blocks = std::max(4L, (blocks + kItemsPerHead - 1) / kItemsPerHead);
      const int split = (int)(64 * split_blocks);
      int32_t* t_first = tiles + 4 * maxTiles;
      int32_t* t_ns = tiles + 5 * maxTiles;
      int32_t* i_tile = tiles + 6 * maxTiles;
      int32_t* i_k0 = i_tile + maxItems;
      int32_t* i_k1 = i_k0 + maxItems;
      for (int t = 0; t < nt; ++t) {
        const int k_lo = pad[tiles[t]], k_hi = tiles[2 * maxTiles + t] + tiles[3 * maxTiles + t];
        t_first[t] = nitems;
        t_ns[t] = 0;
        for (int k0 = k_lo; k0 < k_hi && nitems < maxItems; k0 += split) {
          i_tile[nitems] = t;
          i_k0[nitems] = k0;
          i_k1[nitems] = std::min(k0 + split, k_hi);
          ++nitems;
          ++t_ns[t];
        }
      }
      if (act != ACT_F32 && nitems >= maxItems)
        return fmd_fail(FMD_ERR_STATE, "prefill attention item table overflow");
      // Work order of a split launch: per sequence (its tiles are adjacent),
      // key piece m of every tile, then piece m + 1: the pieces of one m start
      // at the same key (the sequence's pad) and so read the same K/V.
      int32_t* i_order = i_k1 + maxItems;
      int no = 0;
      for (int t0 = 0; t0 < nt;) {
        int t1 = t0, most = 0;
        while (t1 < nt && tiles[t1] == tiles[t0]) most = std::max(most, t_ns[t1++]);
        for (int m = 0; m < most; ++m)
          for (int t = t0; t < t1; ++t)
            if (m < t_ns[t]) i_order[no++] = t_first[t] + m;
        t0 = t1;
      }
      if (no != nitems) return fmd_fail(FMD_ERR_STATE, "prefill attention item order mismatch");
    }
    HIPCHK(hipMemcpyAsync(w.rowmeta.p, meta, (size_t)maxM * 3 * 4, hipMemcpyHostToDevice, s));
    HIPCHK(hipMemcpyAsync(w.tiles.p, tiles, tiles_n * 4, hipMemcpyHostToDevice, s));
    LAUNCH(launch_gather_rows(act, emb_dev, d->H, dmeta + 2 * maxM, M, d->H, w.x.p, d->H, s));
    for (int l = 0; l < d->L; ++l) {
      Layer& ly = d->layers[l];
      LAUNCH(launch_rmsnorm(act, w.x.p, d->H, ly.in_norm, M, d->H, d->eps, w.xn.p, d->H, s));
      GemmArgs g{};
      g.x = w.xn.p;
      g.ldx = d->H;
      g.W = ly.qkv.w;
      g.M = M;
      g.y = w.qkv.p;
      g.ldy = d->qkvd;
      RopeArgs r{};
      r.qkv = w.qkv.p;
      r.ldqkv = d->qkvd;
      r.rows = M;
      r.row_b = dmeta;
      r.batch = B;
      r.row_pos = dmeta + maxM;
      r.state = kv->state;
      r.nh = d->nh;
      r.nkv = d->nkv;
      r.qn_w = ly.q_norm;
      r.kn_w = ly.k_norm;
      r.cos = d->cos;
      r.sin = d->sin;
      r.q_out = w.q.p;
      r.kc = kv->k[l];
      r.vc = kv->v[l];
      r.cap = kv->cap;
      r.eps = d->eps;
      if (act == ACT_F32) {
        LAUNCH(launch_gemm(act, EPI_STORE, g, s));
        LAUNCH(launch_rope_store(act, r, s));
      } else {
        // 16-bit activations: the q/k norm, RoPE and cache stores run in the
        // projection's epilogue
        g.rope = r;
        LAUNCH(launch_gemm(act, EPI_ROPE, g, s));
      }
      AttnPrefillArgs a{};
      a.q = w.q.p;
      a.kc = kv->k[l];
      a.vc = kv->v[l];
      a.cap = kv->cap;
      a.nkv = d->nkv;
      a.tile_b = dtiles;
      a.tile_row0 = dtiles + maxTiles;
      a.tile_pos0 = dtiles + 2 * maxTiles;
      a.tile_n = dtiles + 3 * maxTiles;
      a.start = w.pad.as<int32_t>();
      a.ntiles = nt;
      a.tile_first = dtiles + 4 * maxTiles;
      a.tile_nsplit = dtiles + 5 * maxTiles;
      a.item_tile = dtiles + 6 * maxTiles;
      a.item_k0 = dtiles + 6 * maxTiles + maxItems;
      a.item_order = dtiles + 6 * maxTiles + 3 * maxItems;
      a.item_k1 = dtiles + 6 * maxTiles + 2 * maxItems;
      a.nitems = nitems;
      a.part_ml = w.pml.as<float>();
      a.part_o = w.po.as<float>();
      a.out = w.ctx.p;
      a.scale = act_scale(d);
      LAUNCH(launch_attn_prefill(act, d->rep, a, s));
      g = GemmArgs{};
      g.x = w.ctx.p;
      g.ldx = d->qd;
      g.W = ly.o.w;
      g.M = M;
      g.y = w.x.p;
      g.ldy = d->H;
      g.resid = w.x.p;
      LAUNCH(launch_gemm(act, EPI_RESID, g, s));
      LAUNCH(launch_rmsnorm(act, w.x.p, d->H, ly.post_norm, M, d->H, d->eps, w.xn.p, d->H, s));
      g = GemmArgs{};
      g.x = w.xn.p;
      g.ldx = d->H;
      g.W = ly.gate_up.w;
      g.M = M;
      g.y = w.act.p;
      g.ldy = d->I;
      LAUNCH(launch_gemm(act, EPI_SWIGLU, g, s));
      g = GemmArgs{};
      g.x = w.act.p;
      g.ldx = d->I;
      g.W = ly.down.w;
      g.M = M;
      g.y = w.x.p;
      g.ldy = d->H;
      g.resid = w.x.p;
      LAUNCH(launch_gemm(act, EPI_RESID, g, s));
    }
    if (start + len == total) {
      // last_hidden (qwen3.rs:466-469): each row's position total-1; a row whose
      // prompt is empty is all padding, whose hidden state is exactly zero.
      HIPCHK(hipMemsetAsync((char*)w.x.p + (size_t)M * d->H * d->esz, 0, d->H * d->esz, s));
      for (int b = 0; b < B; ++b) lastsel[b] = last_row[b] >= 0 ? last_row[b] : M;
      HIPCHK(hipMemcpyAsync((int32_t*)w.rowmeta.p + 3 * (size_t)maxM, lastsel, (size_t)B * 4,
                            hipMemcpyHostToDevice, s));
      LAUNCH(launch_gather_rows(act, w.x.p, d->H, dmeta + 3 * maxM, B, d->H, w.lastx.p, d->H, s));
    }
    HIPCHK(hipEventRecord(stage.ev[c & 1], s));
  }
  if (B > kMaxDecodeRows) return fmd_fail(FMD_ERR_ARG, "logits for more than 16 rows per call");
  // Qwen3::logits on the final-normed last rows (qwen3.rs:455, 459-463).
  CHK(launch_logits(d, w.lastx.p, B, w.logits.as<float>(), s));
  kv->len = total;
  d->logits_rows = B;
  CHK(kv_sync_state(kv));
  return 0;
}

int upload_embeds(fmd_dec* d, const void* embeds, int on_dev, int B, int total, const void** dev) {
  if (on_dev) {
    *dev = embeds;
    return 0;
  }
  const size_t bytes = (size_t)B * total * d->H * d->esz;
  CHK(d->ws.embeds.ensure(bytes));
  HIPCHK(hipMemcpyAsync(d->ws.embeds.p, embeds, bytes, hipMemcpyHostToDevice, d->stream));
  *dev = d->ws.embeds.p;
  return 0;
}

int prefill_checks(fmd_dec* d, fmd_kv* kv, const void* embeds, const int32_t* pad, int B,
                   int total) {
  CHK(check_common(d, kv, B));
  if (!embeds || !pad) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (B > kMaxDecodeRows) return fmd_fail(FMD_ERR_ARG, "batch above 16 rows");
  if (total <= 0) return fmd_fail(FMD_ERR_ARG, "empty prompt");
  if (kv->len != 0) return fmd_fail(FMD_ERR_STATE, "prefill needs an empty cache");
  if (total > kv->cap) return overflow(kv, total);
  if (total > d->max_len) return fmd_fail(FMD_ERR_ARG, "prompt longer than the RoPE table");
  bool any_real = false;
  for (int b = 0; b < B; ++b) {
    if (pad[b] < 0 || pad[b] > total) return fmd_fail(FMD_ERR_ARG, "pad outside [0, total]");
    any_real = any_real || pad[b] < total;
  }
  // Qwen3::prefill needs a prompt (qwen3.rs:494); a block that is padding in
  // every row has no last hidden state to take the logits of.
  if (!any_real) return fmd_fail(FMD_ERR_ARG, "empty prompt");
  return 0;
}

// Decode calls attend row b to [pad[b], kv_len]: the pad must lie in the cache.
int decode_pad_checks(const fmd_kv* kv, const int32_t* pad, int B) {
  for (int b = 0; b < B; ++b)
    if (pad[b] < 0 || pad[b] > kv->len) return fmd_fail(FMD_ERR_ARG, "pad outside the cache");
  return 0;
}

// generate_batch for at most kMaxDecodeRows rows (see fmd_dec_generate).
int generate_group(fmd_dec* d, const void* emb_src, int on_dev, const int32_t* pad, int B, int total,
                   int chunk, int budget, uint32_t eos, const int32_t* force, uint32_t* tokens,
                   int32_t* ntok, int32_t* finish) {
  // Decode step s (1 <= s < budget) writes position total + s - 1, whose RoPE
  // row must exist (Rope::apply narrows the table, qwen3.rs:139-144): at most
  // max_len - total steps can run.  The cache holds what can be written.
  const int steps_allowed = std::max(0, std::min(budget - 1, d->max_len - total));
  fmd_kv* kv = nullptr;
  CHK(fmd_kv_create(d, B, std::max(total, 1) + steps_allowed, &kv));
  // events around the prefill and the decode loop (device time of each part)
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  bool timed = true;
  for (hipEvent_t& e : ev) timed = timed && hipEventCreate(&e) == hipSuccess;
  int rc = prefill_checks(d, kv, emb_src, pad, B, total);
  const void* emb = nullptr;
  if (!rc) rc = upload_embeds(d, emb_src, on_dev, B, total, &emb);
  if (!rc && timed) timed = hipEventRecord(ev[0], d->stream) == hipSuccess;
  if (!rc) rc = prefill_impl(d, kv, emb, pad, B, total, chunk);
  if (!rc && timed) timed = hipEventRecord(ev[1], d->stream) == hipSuccess;
  if (!rc) rc = setup_greedy(d, kv, B, budget, force);
  if (!rc) {
    // greedy step 0 on the prefill logits
    if (launch_greedy(d->act, greedy_args(d, kv, B, budget, force != nullptr, eos, 0), d->stream) != hipSuccess)
      rc = fmd_fail(FMD_ERR_HIP, "greedy launch failed");
  }
  int steps = 0;
  if (!rc) rc = run_decode_steps(d, kv, B, steps_allowed, budget, force != nullptr, eos, &steps);
  if (!rc && timed) timed = hipEventRecord(ev[2], d->stream) == hipSuccess;
  if (!rc && steps_allowed < budget - 1 && d->host_mirror[2] < B)
    // rows still generating when the table runs out: the reference's next
    // decode_step fails, and with it the batch
    rc = fmd_fail(FMD_ERR_ARG, "rope position " + std::to_string(total + steps_allowed) +
                                   " beyond the table of " + std::to_string(d->max_len) +
                                   " positions");
  if (!rc) rc = copy_greedy_out(d, B, budget, tokens, ntok, finish);
  if (!rc && timed) {
    // copy_greedy_out has synchronised the stream
    float ms0 = 0.f, ms1 = 0.f;
    if (hipEventElapsedTime(&ms0, ev[0], ev[1]) == hipSuccess &&
        hipEventElapsedTime(&ms1, ev[1], ev[2]) == hipSuccess) {
      d->t_prefill += ms0 * 1e-3;
      d->t_decode += ms1 * 1e-3;
    }
  }
  for (hipEvent_t e : ev)
    if (e) (void)hipEventDestroy(e);
  std::string keep = fmd_last_error();
  fmd_kv_destroy(kv);
  if (rc) fmd_fail(rc, keep);
  return rc;
}

}  // namespace

extern "C" int fmd_dec_prefill(fmd_dec* d, fmd_kv* kv, const void* embeds, int on_dev,
                               const int32_t* pad, int B, int total, int chunk, float* logits) {
  CHK(prefill_checks(d, kv, embeds, pad, B, total));
  HIPCHK(hipSetDevice(d->device));
  if (chunk <= 0) chunk = 256;
  const void* emb = nullptr;
  CHK(upload_embeds(d, embeds, on_dev, B, total, &emb));
  CHK(prefill_impl(d, kv, emb, pad, B, total, chunk));
  if (logits)
    HIPCHK(hipMemcpyAsync(logits, d->ws.logits.p, (size_t)B * d->V * 4, hipMemcpyDeviceToHost, d->stream));
  HIPCHK(hipStreamSynchronize(d->stream));
  return 0;
}

extern "C" int fmd_dec_decode_step(fmd_dec* d, fmd_kv* kv, const uint32_t* ids, const int32_t* pad,
                                   int B, float* logits) {
  CHK(check_common(d, kv, B));
  if (!ids || !pad) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (B > kMaxDecodeRows) return fmd_fail(FMD_ERR_ARG, "batch above 16 rows");
  if (kv->len + 1 > kv->cap) return overflow(kv, 1);
  if (kv->len + 1 > d->max_len) return fmd_fail(FMD_ERR_ARG, "position beyond the RoPE table");
  for (int b = 0; b < B; ++b)
    if (ids[b] >= (uint32_t)d->V) return fmd_fail(FMD_ERR_ARG, "token id out of range");
  CHK(decode_pad_checks(kv, pad, B));
  HIPCHK(hipSetDevice(d->device));
  CHK(ensure_decode_ws(d, B, kv->cap));
  Workspace& w = d->ws;
  HIPCHK(hipMemcpyAsync(w.ids.p, ids, (size_t)B * 4, hipMemcpyHostToDevice, d->stream));
  HIPCHK(hipMemcpyAsync(w.pad.p, pad, (size_t)B * 4, hipMemcpyHostToDevice, d->stream));
  LAUNCH(launch_embed(d->act, w.ids.as<uint32_t>(), B, d->embed, d->H, w.x.p, d->stream));
  CHK(kv_sync_state(kv));
  CHK(decode_layers(d, kv, B, w.pad.as<int32_t>(), nullptr, d->stream));
  kv->len += 1;
  d->logits_rows = B;
  if (logits)
    HIPCHK(hipMemcpyAsync(logits, w.logits.p, (size_t)B * d->V * 4, hipMemcpyDeviceToHost, d->stream));
  HIPCHK(hipStreamSynchronize(d->stream));
  return check_attn_sync(d);
}

extern "C" int fmd_dec_generate(fmd_dec* d, const void* embeds, int on_dev, const int32_t* pad,
                                int B, int total, int chunk, int budget, uint32_t eos,
                                const int32_t* force, uint32_t* tokens, int32_t* ntok,
                                int32_t* finish) {
  if (!d) return fmd_fail(FMD_ERR_ARG, "null handle");
  if (budget < 1) return fmd_fail(FMD_ERR_ARG, "budget must be >= 1");
  if (B < 1) return fmd_fail(FMD_ERR_ARG, "batch must be >= 1");
  if (!embeds || !pad || !tokens || !ntok || !finish) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (eos >= (uint32_t)d->V) return fmd_fail(FMD_ERR_ARG, "eos id outside the vocabulary");
  if (total > d->max_len) return fmd_fail(FMD_ERR_ARG, "prompt longer than the RoPE table");
  HIPCHK(hipSetDevice(d->device));
  if (chunk <= 0) chunk = 256;
  // new_caches(batch, max_prompt + budget) (engine.rs:470, 493).  A batch of
  // more than kMaxDecodeRows rows runs as groups of at most that many rows
  // over the same padded length: each row's tokens depend only on its own
  // padded prompt (the kernels' per-row reductions do not depend on the
  // batch), so they are the tokens of the whole batch run at once.
  const size_t row_bytes = (size_t)total * d->H * d->esz;
  for (int g0 = 0; g0 < B; g0 += kMaxDecodeRows) {
    const int n = std::min(kMaxDecodeRows, B - g0);
    CHK(generate_group(d, (const char*)embeds + g0 * row_bytes, on_dev, pad + g0, n, total, chunk,
                       budget, eos, force ? force + g0 : nullptr, tokens + (size_t)g0 * budget,
                       ntok + g0, finish + g0));
  }
  return 0;
}

extern "C" int fmd_dec_decode_loop(fmd_dec* d, fmd_kv* kv, const uint32_t* first_ids,
                                   const int32_t* pad, int B, int max_steps, uint32_t eos,
                                   const int32_t* force, uint32_t* tokens, int32_t* ntok,
                                   int32_t* finish, int32_t* steps_run) {
  CHK(check_common(d, kv, B));
  if (!first_ids || !pad) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (B > kMaxDecodeRows) return fmd_fail(FMD_ERR_ARG, "batch above 16 rows");
  if (max_steps < 0) return fmd_fail(FMD_ERR_ARG, "negative step count");
  if (eos >= (uint32_t)d->V) return fmd_fail(FMD_ERR_ARG, "eos id outside the vocabulary");
  if (kv->len + max_steps > kv->cap) return overflow(kv, max_steps);
  if (kv->len + max_steps > d->max_len) return fmd_fail(FMD_ERR_ARG, "positions beyond the RoPE table");
  for (int b = 0; b < B; ++b)
    if (first_ids[b] >= (uint32_t)d->V) return fmd_fail(FMD_ERR_ARG, "token id out of range");
  CHK(decode_pad_checks(kv, pad, B));
  HIPCHK(hipSetDevice(d->device));
  CHK(ensure_decode_ws(d, B, kv->cap));
  Workspace& w = d->ws;
  const int budget = std::max(max_steps, 1);
  HIPCHK(hipMemcpyAsync(w.pad.p, pad, (size_t)B * 4, hipMemcpyHostToDevice, d->stream));
  HIPCHK(hipMemcpyAsync(w.ids.p, first_ids, (size_t)B * 4, hipMemcpyHostToDevice, d->stream));
  LAUNCH(launch_embed(d->act, w.ids.as<uint32_t>(), B, d->embed, d->H, w.x.p, d->stream));
  CHK(setup_greedy(d, kv, B, budget, force));
  int steps = 0;
  CHK(run_decode_steps(d, kv, B, max_steps, budget, force != nullptr, eos, &steps));
  if (steps_run) *steps_run = steps;
  return copy_greedy_out(d, B, budget, tokens, ntok, finish);
}

extern "C" int fmd_op_linear(fmd_dec* d, int layer, int proj, const void* x, int rows, void* y) {
  if (!d || !x || !y) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (proj < 0 || proj > 4 || (proj < 4 && (layer < 0 || layer >= d->L)))
    return fmd_fail(FMD_ERR_ARG, "bad layer or projection");
  if (rows <= 0) return 0;
  HIPCHK(hipSetDevice(d->device));
  const Lin* l = proj == 4 ? &d->lm_head
                           : (proj == 0 ? &d->layers[layer].qkv
                              : proj == 1 ? &d->layers[layer].o
                              : proj == 2 ? &d->layers[layer].gate_up
                                          : &d->layers[layer].down);
  const int in = l->w.in, out = l->w.out;
  CHK(d->ws.amax.ensure((size_t)gemv_logits_nparts(d->act, d->quant, false, in, out) * kMaxDecodeRows * 8));
  for (int r0 = 0; r0 < rows;) {
    const int n = (proj == 4 || rows - r0 <= kMaxDecodeRows) ? std::min(kMaxDecodeRows, rows - r0)
                                                             : rows - r0;
    const char* xs = (const char*)x + (size_t)r0 * in * d->esz;
    if (proj == 4) {
      float* ys = (float*)y + (size_t)r0 * out;
      LAUNCH(launch_gemv(d->act, EPI_LOGITS, false,
                         gemv_args(xs, in, nullptr, d->eps, l->w, n, ys, out, nullptr,
                                   d->ws.amax.as<uint64_t>()),
                         d->stream));
    } else if (n <= kMaxDecodeRows) {
      char* ys = (char*)y + (size_t)r0 * out * d->esz;
      LAUNCH(launch_gemv(d->act, EPI_STORE, false,
                         gemv_args(xs, in, nullptr, d->eps, l->w, n, ys, out, nullptr, nullptr),
                         d->stream));
    } else {
      GemmArgs g{};
      g.x = xs;
      g.ldx = in;
      g.W = l->w;
      g.M = n;
      g.y = (char*)y + (size_t)r0 * out * d->esz;
      g.ldy = out;
      LAUNCH(launch_gemm(d->act, EPI_STORE, g, d->stream));
    }
    r0 += n;
  }
  if (d->stream == d->own_stream) HIPCHK(hipStreamSynchronize(d->stream));
  return 0;
}

extern "C" int fmd_op_attention_decode(fmd_dec* d, fmd_kv* kv, int layer, const void* qkv,
                                       const int32_t* pad, int B, void* ctx) {
  CHK(check_common(d, kv, B));
  if (!qkv || !pad || !ctx || layer < 0 || layer >= d->L) return fmd_fail(FMD_ERR_ARG, "bad argument");
  if (kv->len + 1 > kv->cap) return overflow(kv, 1);
  if (kv->len + 1 > d->max_len) return fmd_fail(FMD_ERR_ARG, "position beyond the RoPE table");
  if (B > kMaxDecodeRows) return fmd_fail(FMD_ERR_ARG, "batch above 16 rows");
  CHK(decode_pad_checks(kv, pad, B));
  HIPCHK(hipSetDevice(d->device));
  CHK(ensure_decode_ws(d, B, kv->cap));
  Workspace& w = d->ws;
  // Upload the position and pads only when they changed since the last call,
  // so back-to-back calls time the attention kernels alone.
  CHK(w.oppad.ensure(64 * 4));
  const std::vector<int32_t> padv(pad, pad + B);
  if (d->op_len != kv->len || d->op_pad != padv || d->op_state_buf != w.opstate.p ||
      d->op_pad_buf != w.oppad.p) {
    int32_t st[4] = {kv->len, 0, 0, 0};
    HIPCHK(hipMemcpyAsync(w.opstate.p, st, sizeof st, hipMemcpyHostToDevice, d->stream));
    HIPCHK(hipMemcpyAsync(w.oppad.p, pad, (size_t)B * 4, hipMemcpyHostToDevice, d->stream));
    d->op_len = kv->len;
    d->op_pad = padv;
    d->op_state_buf = w.opstate.p;
    d->op_pad_buf = w.oppad.p;
  }
  const AttnDecodeArgs a = attn_args(d, kv, layer, B, qkv, w.oppad.as<int32_t>(),
                                     w.opstate.as<int32_t>(), nullptr, ctx);
  LAUNCH(launch_attn_decode(d->act, a, d->stream));
  // Synchronous on the handle's own stream; asynchronous on a caller's stream
  // (so the caller can time it with events on that stream; a wait that gave
  // up there is reported by the next synchronous call on this handle).
  if (d->stream == d->own_stream) {
    HIPCHK(hipStreamSynchronize(d->stream));
    return check_attn_sync(d);
  }
  return 0;
}

extern "C" int fmd_dec_greedy(fmd_dec* d, int B, uint32_t eos, const int32_t* force, int step,
                              int32_t* done, uint32_t* next_ids, uint32_t* emitted) {
  if (!d || !done || !next_ids) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (B < 1 || B > kMaxDecodeRows) return fmd_fail(FMD_ERR_ARG, "batch must be in [1, 16]");
  if (d->logits_rows != B)
    return fmd_fail(FMD_ERR_STATE, "no logits for this batch: call prefill or decode_step first");
  if (eos >= (uint32_t)d->V) return fmd_fail(FMD_ERR_ARG, "eos id outside the vocabulary");
  HIPCHK(hipSetDevice(d->device));
  Workspace& w = d->ws;
  CHK(w.done.ensure((size_t)B * 4));
  CHK(w.ntok.ensure((size_t)B * 4));
  CHK(w.finish.ensure((size_t)B * 4));
  CHK(w.tokens.ensure((size_t)B * 4));
  CHK(w.force.ensure((size_t)B * 4));
  CHK(w.opstate.ensure(64));
  CHK(w.ids.ensure((size_t)B * 4));
  CHK(w.x.ensure((size_t)B * d->H * d->esz));
  hipStream_t s = d->stream;
  // one greedy update with a token budget of 1: ntok[b] tells whether row b
  // emitted a token this step
  const int32_t st[4] = {0, step, 0, 0};
  HIPCHK(hipMemcpyAsync(w.opstate.p, st, sizeof st, hipMemcpyHostToDevice, s));
  HIPCHK(hipMemcpyAsync(w.done.p, done, (size_t)B * 4, hipMemcpyHostToDevice, s));
  HIPCHK(hipMemsetAsync(w.ntok.p, 0, (size_t)B * 4, s));
  HIPCHK(hipMemsetAsync(w.finish.p, 0, (size_t)B * 4, s));
  if (force) HIPCHK(hipMemcpyAsync(w.force.p, force, (size_t)B * 4, hipMemcpyHostToDevice, s));
  GreedyArgs g{};
  g.part = w.amax.as<uint64_t>();
  g.nparts = gemv_logits_nparts(d->act, d->quant, true, d->H, d->V);
  g.batch = B;
  g.state = w.opstate.as<int32_t>();
  g.host_state = nullptr;
  g.advance = 0;
  g.done = w.done.as<int32_t>();
  g.ntok = w.ntok.as<int32_t>();
  g.finish = w.finish.as<int32_t>();
  g.tokens = w.tokens.as<uint32_t>();
  g.budget = 1;
  g.force = force ? w.force.as<int32_t>() : nullptr;
  g.eos = eos;
  g.next_ids = w.ids.as<uint32_t>();
  g.embed = d->embed;
  g.x = w.x.p;
  g.hidden = d->H;
  g.vocab = d->V;
  LAUNCH(launch_greedy(d->act, g, s));
  std::vector<int32_t> ntok(B);
  std::vector<uint32_t> tok(B);
  HIPCHK(hipMemcpyAsync(done, w.done.p, (size_t)B * 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipMemcpyAsync(next_ids, w.ids.p, (size_t)B * 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipMemcpyAsync(ntok.data(), w.ntok.p, (size_t)B * 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipMemcpyAsync(tok.data(), w.tokens.p, (size_t)B * 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipStreamSynchronize(s));
  if (emitted)
    for (int b = 0; b < B; ++b) emitted[b] = ntok[b] ? tok[b] : 0xffffffffu;
  return 0;
}

extern "C" int fmd_dec_set_spin_limit(fmd_dec* d, int polls) {
  if (!d) return fmd_fail(FMD_ERR_ARG, "null handle");
  if (polls < 0) return fmd_fail(FMD_ERR_ARG, "negative poll count");
  d->spin_limit = polls;
  return 0;
}

extern "C" int fmd_op_layer_decode(fmd_dec* d, fmd_kv* kv, int layer, void* x, const int32_t* pad,
                                   int B) {
  CHK(check_common(d, kv, B));
  if (!x || !pad || layer < 0 || layer >= d->L) return fmd_fail(FMD_ERR_ARG, "bad argument");
  if (B > kMaxDecodeRows) return fmd_fail(FMD_ERR_ARG, "batch above 16 rows");
  if (kv->len + 1 > kv->cap) return overflow(kv, 1);
  if (kv->len + 1 > d->max_len) return fmd_fail(FMD_ERR_ARG, "position beyond the RoPE table");
  CHK(decode_pad_checks(kv, pad, B));
  HIPCHK(hipSetDevice(d->device));
  CHK(ensure_decode_ws(d, B, kv->cap));
  Workspace& w = d->ws;
  const size_t bytes = (size_t)B * d->H * d->esz;
  HIPCHK(hipMemcpyAsync(w.pad.p, pad, (size_t)B * 4, hipMemcpyHostToDevice, d->stream));
  HIPCHK(hipMemcpyAsync(w.x.p, x, bytes, hipMemcpyDeviceToDevice, d->stream));
  CHK(kv_sync_state(kv));
  CHK(decode_layer(d, kv, layer, B, w.pad.as<int32_t>(), nullptr, d->stream));
  HIPCHK(hipMemcpyAsync(x, w.x.p, bytes, hipMemcpyDeviceToDevice, d->stream));
  HIPCHK(hipStreamSynchronize(d->stream));
  return check_attn_sync(d);
}

extern "C" int fmd_op_logits(fmd_dec* d, const void* x, int rows, float* logits) {
  if (!d || !x || !logits) return fmd_fail(FMD_ERR_ARG, "null argument");
  if (rows < 1 || rows > kMaxDecodeRows) return fmd_fail(FMD_ERR_ARG, "rows must be in [1, 16]");
  if (!fmd_dec_ready(d)) return fmd_fail(FMD_ERR_STATE, "decoder weights are incomplete");
  HIPCHK(hipSetDevice(d->device));
  CHK(d->ws.amax.ensure((size_t)gemv_logits_nparts(d->act, d->quant, true, d->H, d->V) *
                        kMaxDecodeRows * 8));
  CHK(launch_logits(d, x, rows, logits, d->stream));
  HIPCHK(hipStreamSynchronize(d->stream));
  return 0;
}

// ---------------------------------------------------------------------------
// Decode attention without allocation.  Its scratch -- the launch state and
// exchange words, split partials and scores of the attention kernels, the
// write position and the pads -- lives in one file-scope device array per GPU
// for the life of the process.  On the host the array's name is only a
// stand-in, never a device address: each device's address comes from
// hipGetSymbolAddress, resolved once per device when the first decoder is
// created on it (fmd_dec_create), with that device current.

constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_scratch_mu;
std::vector<unsigned char*> g_scratch_ptr;  // per device index, nullptr until resolved

unsigned char* scratch_of(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return device >= 0 && device < (int)g_scratch_ptr.size() ? g_scratch_ptr[device] : nullptr;
}

// Byte offsets of the pieces the no-allocation attention uses, for B rows
// over a cache of capacity cap.  The launch state (epoch, finished units,
// error code, per-unit counters) comes first and keeps its offset, so its
// epoch carries over from call to call.
struct NoAllocLayout {
  size_t sync, state, pad, sticky, xml, xpart, xsc, xnew, scores, ml, part, total;
};
NoAllocLayout noalloc_layout(const fmd_dec* d, int B, int cap) {
  const AttnDecodePlan plan = split_geom(d, B, cap);
  const size_t units = (size_t)B * d->nkv * plan.max_splits * d->rep;
  NoAllocLayout L{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += (bytes + 255) / 256 * 256;
    return at;
  };
  L.sync = take((size_t)(4 + kMaxDecodeRows * d->nkv) * 4);
  L.state = take(16);
  L.sticky = take(4);
  L.pad = take((size_t)B * 4);
  if (plan.fused) {
    L.xml = take(units * 2 * 8);
    L.xpart = take(units * d->hd * 8);
    L.xsc = take((size_t)B * d->nkv * d->rep * xsc_stride(plan) * 8);
    L.xnew = take((size_t)B * d->nkv * d->rep * 8);
  } else {
    L.scores = take((size_t)B * d->nh * cap * d->esz);
    L.ml = take(units * 2 * 4);
    L.part = take(units * d->hd * 4);
  }
  L.total = o;
  return L;
}


// Stream-ordered set-up of one no-allocation launch, from by-value kernel
// arguments only (so a graph capture of the call records no host memory):
// the write position, the pads, and the launch's error word, whose previous
// value is first folded into the sticky word that the next synchronous call
// reports.
struct NoAllocSetup {
  int32_t pad[kMaxDecodeRows];
  int32_t len, batch;
};
__global__ void noalloc_setup_kernel(NoAllocSetup a, int32_t* state, int32_t* pad,
                                     uint32_t* sync, uint32_t* sticky) {
  const int t = threadIdx.x;
  if (t < a.batch) pad[t] = a.pad[t];
  if (t < 4) state[t] = t == 0 ? a.len : 0;
  if (t == 0) {
    const uint32_t prev = __hip_atomic_load(sync + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev) __hip_atomic_store(sticky, prev, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(sync + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

// Resolves (once per device) the scratch address of `device`, which must be
// current, and clears it: exchange words at epoch 0, the launch epoch at 1,
// so that no word is valid before a launch writes it.
int noalloc_scratch_init(int device, hipStream_t s) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (device < 0) return fmd_fail(FMD_ERR_ARG, "bad device");
  if ((int)g_scratch_ptr.size() <= device) g_scratch_ptr.resize(device + 1, nullptr);
  if (g_scratch_ptr[device]) return 0;
  unsigned char* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr)
    return fmd_fail(FMD_ERR_HIP, std::string("scratch symbol address: ") + hipGetErrorString(e));
  LAUNCH(launch_fill_i32((int32_t*)ptr, (int64_t)(kNoAllocScratchBytes / 4), 0, s));
  LAUNCH(launch_fill_i32((int32_t*)ptr, 1, 1, s));
  HIPCHK(hipStreamSynchronize(s));
  g_scratch_ptr[device] = ptr;
  return 0;
}

extern "C" int fmd_op_attention_decode_noalloc(fmd_dec* d, fmd_kv* kv, int layer, const void* qkv,
                                               const int32_t* pad, int B, void* ctx) {
  CHK(check_common(d, kv, B));
  if (!qkv || !pad || !ctx || layer < 0 || layer >= d->L) return fmd_fail(FMD_ERR_ARG, "bad argument");
  if (kv->len + 1 > kv->cap) return overflow(kv, 1);
  if (kv->len + 1 > d->max_len) return fmd_fail(FMD_ERR_ARG, "position beyond the RoPE table");
  if (B > kMaxDecodeRows) return fmd_fail(FMD_ERR_ARG, "batch above 16 rows");
  CHK(decode_pad_checks(kv, pad, B));
  unsigned char* base = scratch_of(d->device);
  if (!base) return fmd_fail(FMD_ERR_STATE, "no scratch for this device (create a decoder on it first)");
  const NoAllocLayout L = noalloc_layout(d, B, kv->cap);
  if (L.total > kNoAllocScratchBytes)
    return fmd_fail(FMD_ERR_ARG, "batch " + std::to_string(B) + " at capacity " +
                                     std::to_string(kv->cap) + " needs " + std::to_string(L.total) +
                                     " bytes of scratch; the static scratch holds " +
                                     std::to_string(kNoAllocScratchBytes));
  HIPCHK(hipSetDevice(d->device));
  NoAllocSetup su{};
  for (int b = 0; b < B; ++b) su.pad[b] = pad[b];
  su.len = kv->len;
  su.batch = B;
  uint32_t* const sync = (uint32_t*)(base + L.sync);
  uint32_t* const sticky = (uint32_t*)(base + L.sticky);
  hipLaunchKernelGGL(noalloc_setup_kernel, dim3(1), dim3(64), 0, d->stream, su,
                     (int32_t*)(base + L.state), (int32_t*)(base + L.pad), sync, sticky);
  LAUNCH(hipGetLastError());
  AttnDecodeArgs a = attn_args(d, kv, layer, B, qkv, (const int32_t*)(base + L.pad),
                               (const int32_t*)(base + L.state), nullptr, ctx);
  a.sync = sync;
  a.xml = a.fused ? (uint64_t*)(base + L.xml) : nullptr;
  a.xpart = a.fused ? (uint64_t*)(base + L.xpart) : nullptr;
  a.xsc = a.fused ? (uint64_t*)(base + L.xsc) : nullptr;
  a.xnew = a.fused ? (uint64_t*)(base + L.xnew) : nullptr;
  a.scores = a.fused ? nullptr : (void*)(base + L.scores);
  a.ml = a.fused ? nullptr : (float*)(base + L.ml);
  a.part = a.fused ? nullptr : (float*)(base + L.part);
  LAUNCH(launch_attn_decode(d->act, a, d->stream));
  // Under graph capture, or on a caller's stream, the call returns without
  // waiting: a wait that gave up in this launch is reported by the next
  // synchronous call on this device (any handle).
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIPCHK(hipStreamIsCapturing(d->stream, &cap));
  if (cap != hipStreamCaptureStatusNone || d->stream != d->own_stream) return 0;
  HIPCHK(hipStreamSynchronize(d->stream));
  uint32_t codes[2] = {0, 0};
  HIPCHK(hipMemcpy(&codes[0], sync + 2, 4, hipMemcpyDeviceToHost));
  HIPCHK(hipMemcpy(&codes[1], sticky, 4, hipMemcpyDeviceToHost));
  if (!codes[0] && !codes[1]) return 0;
  const uint32_t zero = 0;
  HIPCHK(hipMemcpy(sync + 2, &zero, 4, hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(sticky, &zero, 4, hipMemcpyHostToDevice));
  return fmd_fail(FMD_ERR_HIP, std::string("decode attention: work-groups of one (row, KV head) did "
                                           "not meet within the spin limit (code ") +
                                   std::to_string(codes[0] ? codes[0] : codes[1]) + ")" +
                                   (codes[0] ? "" : " in an earlier asynchronous call on this device"));
}
