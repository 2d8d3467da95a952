// Host-side structures shared by the C ABI implementation files.
#pragma once
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>
#include <vector>

#include "fmd_dec.h"
#include "fmd_kernels.h"

int fmd_fail(int code, const std::string& msg);

// Grow-only device buffer.  ensure() sets *fresh when it (re)allocated: a
// new allocation can land at the old address, so the address alone does not
// tell.
struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
  int ensure(size_t bytes, bool* fresh = nullptr);
  void release();
  template <class T> T* as() const { return (T*)p; }
};

struct Lin {
  LinWeights w{};
  size_t wbytes = 0, sbytes = 0;
};

struct Layer {
  Lin qkv, o, gate_up, down;
  void* in_norm = nullptr;
  void* post_norm = nullptr;
  void* q_norm = nullptr;
  void* k_norm = nullptr;
  uint32_t set = 0;
};

// Decode buffers of the projections and the attention (its split partials,
// scores, exchange words and launch state).
struct DecodeLane {
  DevBuf qkv, ctx, act, attn_part, attn_ml, scores, xsync, xml, xpart, xsc, xnew, xqkv;
  void release_all() {
    for (DevBuf* b : {&qkv, &ctx, &act, &attn_part, &attn_ml, &scores, &xsync, &xml, &xpart,
                      &xsc, &xnew, &xqkv})
      b->release();
  }
};

// Per-handle device scratch, sized on demand (never inside a graph capture).
struct Workspace {
  DevBuf x, xn, qkv, q, ctx, act, logits, amax, pml, po, ids, pad, rowmeta, tiles, lastx, embeds,
      done, ntok, finish, tokens, force, opstate, oppad, asrc, audio;
  DecodeLane dec;
  void release_all() {
    for (DevBuf* b : {&x, &xn, &qkv, &q, &ctx, &act, &logits, &amax, &pml, &po, &ids, &pad,
                      &rowmeta, &tiles, &lastx, &embeds, &done, &ntok, &finish, &tokens, &force,
                      &opstate, &oppad, &asrc, &audio})
      b->release();
    dec.release_all();
  }
};

struct fmd_dec {
  fmd_text_config cfg{};
  int prec = 0, act = 0, device = 0, max_len = 0;
  bool quant = false;
  size_t esz = 2;
  int H = 0, I = 0, hd = 0, nh = 0, nkv = 0, rep = 0, qd = 0, kd = 0, qkvd = 0, V = 0, L = 0;
  float eps = 1e-6f, scale = 0.f;
  hipStream_t own_stream = nullptr, stream = nullptr;
  std::vector<Layer> layers;
  Lin lm_head;
  void* embed = nullptr;
  void* norm = nullptr;
  void* cos = nullptr;
  void* sin = nullptr;
  bool embed_set = false, norm_set = false, lm_head_set = false, lm_head_explicit = false;
  DevBuf staging, staging2;
  Workspace ws;
  int32_t* host_mirror = nullptr;  // host-mapped copy of the greedy state
  void* host_stage = nullptr;      // pinned host staging of prefill chunk tables
  size_t host_stage_n = 0;
  // what fmd_op_attention_decode last uploaded (repeated calls skip the copies)
  std::vector<int32_t> op_pad;
  int op_len = -1;
  int logits_rows = 0;  // rows of the last logits launch (prefill / decode step), 0 = none
  const void* op_state_buf = nullptr;
  const void* op_pad_buf = nullptr;
  // Polls of one wait in the single-launch attention before it gives up and
  // the call fails (fmd_dec_set_spin_limit); each poll is a device-memory
  // round trip, about a microsecond.
  int spin_limit = 20000;
  // Device seconds of the prefills and the greedy decode loops run by
  // fmd_dec_generate since the last reset (HIP events around each part).
  double t_prefill = 0.0, t_decode = 0.0;
};

// Largest KV-cache capacity: decode attention runs at most 128 splits of 512 keys.
constexpr int kMaxCapacity = 65536;

struct fmd_kv {
  fmd_dec* dec = nullptr;
  int batch = 0, cap = 0, len = 0;
  size_t layer_bytes = 0;
  std::vector<void*> k, v;
  int32_t* state = nullptr;  // device: [0] length, [1] greedy step, [2] rows done
};

int kv_sync_state(fmd_kv* kv);
// Resolves and clears the no-allocation attention's static scratch of
// `device` (current) once per process.
int noalloc_scratch_init(int device, hipStream_t s);

// Host copies of the IEEE round-to-nearest-even conversions.
inline uint16_t host_f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xffu, man = x & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | (man ? 0x7e00u | (man >> 13) : 0x7c00u));
  if (exp == 0) return (uint16_t)sign;
  const int e = (int)exp - 127;
  if (e >= -14) {
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    const uint32_t m10 = man >> 13, rem = man & 0x1fffu;
    uint32_t r = ((uint32_t)(e + 15) << 10) + m10;
    if (rem > 0x1000u || (rem == 0x1000u && (m10 & 1u))) r += 1;
    if (r >= 0x7c00u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | r);
  }
  const uint32_t M = man | 0x800000u;
  const int s = -e - 1;
  if (s >= 25) return (uint16_t)sign;
  uint32_t q = M >> s;
  const uint32_t rem = M & ((1u << s) - 1u), half = 1u << (s - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  return (uint16_t)(sign | q);
}
inline float host_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0x1fu) u = sign | 0x7f800000u | (man << 13);
  else if (exp == 0) {
    float v = (float)man * (1.0f / 16777216.0f);
    return sign ? -v : v;
  } else u = sign | ((exp + 112u) << 23) | (man << 13);
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint16_t host_f32_to_bf16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}
inline float host_bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline float host_round_act(float v, int act) {
  if (act == ACT_F16) return host_f16_to_f32(host_f32_to_f16(v));
  if (act == ACT_BF16) return host_bf16_to_f32(host_f32_to_bf16(v));
  return v;
}

void host_quantize_q8_0(const float* src, int64_t rows, int64_t cols, uint8_t* out);
