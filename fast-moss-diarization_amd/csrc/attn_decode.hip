// GQA decode attention over the left-padded batched KV cache, with the
// per-head q/k RMSNorm, RoPE and the KV-cache append of the new token fused in.
//
// Reference: Attention::forward (qwen3.rs:213-257) with the decode mask of
// build_mask (qwen3.rs:523-562): the new query of row b at position `pos`
// attends to keys [pad_b, pos]; query head h reads KV head h / repeat
// (qwen3.rs:237-241).  q and k are RMS-normalised over head_dim before RoPE
// (qwen3.rs:218-225); the new K/V land at ((b*nkv + h)*cap + pos)*hd
// (KvCache::append, qwen3.rs:86-101).
//
// Rounding follows the reference's tensor dtypes: scores are
// rd(rd(q.k) * rd(1/sqrt(hd))) (qwen3.rs:243); softmax_last_dim returns the
// probabilities in the activation dtype, so each p_j = rd(exp(s_j - M) / S)
// is rounded with the GLOBAL max M and sum S of its row before the value
// product (qwen3.rs:248-249); the context is rd(sum_j p_j v_j).  Rounding p_j
// needs M and S first, so the keys are visited twice -- but each pass reads
// only one of K and V, so the cache is still read once in total:
//
//  attn_score_kernel: one work-group per (split of the cached keys
//    [pad_b, pos), KV head, row).  Each wave normalises and rotates its REP
//    query heads from the raw qkv projection, then streams K in chunks of 32
//    keys: a 16-lane row of the wave holds one key (8 dims per lane, one
//    16-byte load), so each wave load is 1 KiB contiguous, with two chunks in
//    flight.  Scores go to a (B, nh, cap) buffer in the activation dtype
//    (they are dtype values already); each split writes its (max, sum of exp)
//    per query head.  The first wave of split 0 also owns the new token: it
//    normalises and rotates its k, appends k and v at `pos` and scores it
//    from registers.  (Splitting the cached keys only keeps a 4096-key
//    context at 16 splits per row instead of 17 -- the 17th, one key long,
//    would start late and stretch the whole launch.)
//  attn_value_kernel: same grid.  Every work-group of a (row, KV head) derives
//    M and S from the split partials in the same order, so all of them round
//    p_j identically; it then streams V with the scores and writes its share
//    of sum_j p_j v_j (split 0's first wave adds the new token's).
//  attn_combine_kernel: one work-group per (KV head, row) adds the splits'
//    shares in split order and stores the context.
// These three kernels serve f32 activations.  16-bit activations run the
// same two passes and the combine in ONE launch (attn_fused_kernel below):
// the work-groups exchange their partials through epoch-tagged words written
// and read with device-scope atomics, so no agent-scope fence (an L2
// write-back plus invalidate on this multi-XCD part) is needed.
#include <stdlib.h>

#include <algorithm>

#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

constexpr int HD = 128;
// Work-groups per role the split aims for at full capacity (see
// attn_decode_split).  Measured, ms per decode step, target 1024 / 768 / 640:
// int8 batch 8 at 4096 keys 1.345 / 1.346 / 1.345; int8 batch 8 with rows of
// U[1024, 4096] keys 1.204 / 1.152 / 1.158 (a ragged batch fills far fewer
// work-groups than its capacity promises, and the 128-key split the larger
// target picked there halves every work-group's stream); bf16 batch 8
// U[2048, 6144] 1.413 / 1.415 / 1.429; int8 batch 16 unchanged.
#ifndef FMD_ATTN_TARGET_WGS
#define FMD_ATTN_TARGET_WGS 768
#endif
constexpr int CH = 32;  // keys per wave chunk
constexpr float kLog2e = 1.4426950408889634f;

// Raw 16-byte (or 32-byte for f32) piece of one key row: 8 dims.
template <int A> struct Chunk { u32x4 v; };
template <> struct Chunk<ACT_F32> { u32x4 v0, v1; };

template <int A>
__device__ __forceinline__ Chunk<A> load_chunk(const void* base, size_t elem) {
  Chunk<A> c;
  if constexpr (A == ACT_F32) {
    const u32x4* p = (const u32x4*)((const float*)base + elem);
    c.v0 = __builtin_nontemporal_load(p);
    c.v1 = __builtin_nontemporal_load(p + 1);
  } else {
    c.v = __builtin_nontemporal_load((const u32x4*)((const uint16_t*)base + elem));
  }
  return c;
}

// 16-byte piece at a byte offset (< 4 GiB) from a work-group-uniform base:
// one 32-bit offset register per load instead of a 64-bit address.
__device__ __forceinline__ u32x4 load16_at(const void* ubase, uint32_t byte_off) {
  return __builtin_nontemporal_load((const u32x4*)((const char*)ubase + byte_off));
}

template <int A>
__device__ __forceinline__ void chunk_f32(const Chunk<A>& c, float* o) {
  if constexpr (A == ACT_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // copy the element out first: bit-casting a vector-element expression
      // directly reads element 0
      const uint32_t a = c.v0[i], b = c.v1[i];
      o[i] = __builtin_bit_cast(float, a);
      o[4 + i] = __builtin_bit_cast(float, b);
    }
  } else {
    unpack8<A>(c.v, o);
  }
}

template <int A>
__device__ __forceinline__ void load8(const void* base, size_t elem, float* o) {
  chunk_f32<A>(load_chunk<A>(base, elem), o);
}


// Max / sum over the 8 lanes of a half-row (lanes dc and dc' with equal
// dc >> 3): quad xor 1, quad xor 2, then the half-row mirror.
__device__ __forceinline__ float half8_max(float v) {
  v = fmaxf(v, FMD_DPP(v, 0xB1));
  v = fmaxf(v, FMD_DPP(v, 0x4E));
  return fmaxf(v, FMD_DPP(v, 0x141));
}
__device__ __forceinline__ float half8_sum(float v) {
  v += FMD_DPP(v, 0xB1);
  v += FMD_DPP(v, 0x4E);
  return v + FMD_DPP(v, 0x141);
}

// Reduce-scatter of 16 per-lane partials over the 16 lanes of a row: lane dc
// returns the row sum of v[dc].  Each level keeps the half of the values
// whose index bit matches the lane's bit and adds the partner's copy of it
// (partners: row rotate by 8, half-row mirror, quad xor 2, quad xor 1 --
// each flips exactly the level's bit among the bits still in play).
__device__ __forceinline__ float rscatter16(const float* v, int dc) {
  const bool b3 = dc & 8, b2 = dc & 4, b1 = dc & 2, b0 = dc & 1;
  float w[8], x[4], y[2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float keep = b3 ? v[8 + j] : v[j], send = b3 ? v[j] : v[8 + j];
    w[j] = keep + FMD_DPP(send, 0x128);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float keep = b2 ? w[4 + j] : w[j], send = b2 ? w[j] : w[4 + j];
    x[j] = keep + FMD_DPP(send, 0x141);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float keep = b1 ? x[2 + j] : x[j], send = b1 ? x[j] : x[2 + j];
    y[j] = keep + FMD_DPP(send, 0x4E);
  }
  const float keep = b0 ? y[1] : y[0], send = b0 ? y[0] : y[1];
  return keep + FMD_DPP(send, 0xB1);
}

// q.k partial over this lane's 8 dims: packed dot products for 16-bit
// activations (exact products, f32 sums), FMAs for f32.
template <int A>
__device__ __forceinline__ float dot8(const uint32_t* q2, const float* qf, const Chunk<A>& k) {
  if constexpr (A == ACT_F32) {
    float kf[8];
    chunk_f32<A>(k, kf);
    float d = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) d += qf[t] * kf[t];
    return d;
  } else if constexpr (A == ACT_F16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    float d = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      d = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, q2[t]), __builtin_bit_cast(h2, (uint32_t)k.v[t]), d, false);
    return d;
  } else {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    float d = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, q2[t]), __builtin_bit_cast(b2, (uint32_t)k.v[t]), d, false);
    return d;
  }
}

// c + a.x * b.x + a.y * b.y for packed 16-bit pairs (exact products, f32 sum).
template <int A>
__device__ __forceinline__ float dot2acc(uint32_t a, uint32_t b, float c) {
  if constexpr (A == ACT_F16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
  } else {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, a), __builtin_bit_cast(b2, b), c, false);
  }
}

// Key range of one wave: split `split` of row b covers the cached keys
// [k0, k1) of [s0, pos); wave w takes [kw0, kw1) of it (possibly empty).
// A row with no cached key still has one split, for the new token.
struct WaveRange {
  int pos, nsplit, k0, k1, kw0, kw1;
  bool active, owner;  // owner: split 0, wave 0 -- the new token's wave
};
__device__ __forceinline__ int row_splits(int pos, int s0, int split) {
  return max(1, (pos - s0 + split - 1) / split);
}
template <int NCH>
__device__ __forceinline__ WaveRange wave_range(const AttnDecodeArgs& p, int split, int b, int w) {
  WaveRange r;
  r.pos = p.state[0];
  const int s0 = p.start[b];
  r.nsplit = row_splits(r.pos, s0, p.split);
  r.k0 = s0 + split * p.split;
  r.k1 = min(r.k0 + p.split, r.pos);
  r.kw0 = r.k0 + w * (NCH * CH);  // p.split == 4 * NCH * CH
  r.kw1 = max(min(r.kw0 + NCH * CH, r.k1), r.kw0);
  r.active = split < r.nsplit;
  r.owner = split == 0 && w == 0;
  return r;
}

// Score element of key j for query head h of row b.
__device__ __forceinline__ size_t score_index(const AttnDecodeArgs& p, int b, int h, int j) {
  return ((size_t)b * p.nkv * p.rep + h) * p.cap + j;
}

template <int A, int REP, int NCH>
__global__ void __launch_bounds__(256) attn_score_kernel(AttnDecodeArgs p) {
  typedef typename ActT<A>::T T;
  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  if (p.done && p.done[b]) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int grp = lane >> 4, dc = lane & 15;
  const WaveRange wr = wave_range<NCH>(p, split, b, w);
  if (!wr.active) return;
  const int pos = wr.pos, kw0 = wr.kw0, kw1 = wr.kw1;
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;
  T* sc_out = (T*)p.scores;

  // Loads in the order they are needed, all before any arithmetic (the
  // vector-memory counter retires in order): the REP query heads, the new
  // token's k and v, the norm gains and the RoPE row of `pos`; then the
  // first NB chunks of K.  Key indices are clamped to a cached key of this
  // split (or to `pos` itself when the row has none), so no load sits behind
  // a branch; keys outside [kw0, kw1) are masked.
  const int qd = p.nkv * REP * HD;
  const size_t qrow = (size_t)b * p.ldqkv;
  Chunk<A> qraw[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r)
    qraw[r] = load_chunk<A>(p.qkv, qrow + (g * REP + r) * HD + dc * 8);
  const Chunk<A> kraw = load_chunk<A>(p.qkv, qrow + qd + g * HD + dc * 8);
  const Chunk<A> vraw = load_chunk<A>(p.qkv, qrow + qd + p.nkv * HD + g * HD + dc * 8);
  const Chunk<A> gq = load_chunk<A>(p.qn_w, dc * 8);
  const Chunk<A> gk = load_chunk<A>(p.kn_w, dc * 8);
  const Chunk<A> cr = load_chunk<A>(p.cos, (size_t)pos * 64 + (dc & 7) * 8);
  const Chunk<A> sr = load_chunk<A>(p.sin, (size_t)pos * 64 + (dc & 7) * 8);

  constexpr int NB = NCH < 2 ? NCH : 2;  // chunks in flight
  const int kc = max(wr.k1 - 1, wr.k0);
  Chunk<A> kbuf[NB][CH / 4];
  auto load = [&](int c0, Chunk<A>* kk) {
#pragma unroll
    for (int i = 0; i < CH / 4; ++i)
      kk[i] = load_chunk<A>(p.kc, (kvbase + min(c0 + 4 * i + grp, kc)) * HD + dc * 8);
  };
#pragma unroll
  for (int c = 0; c < NB; ++c) load(kw0 + c * CH, kbuf[c]);
  __builtin_amdgcn_sched_barrier(0);

  float qf[REP][8], cf[8], sf[8], gf[8];
  chunk_f32<A>(cr, cf);
  chunk_f32<A>(sr, sf);
  chunk_f32<A>(gq, gf);
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    chunk_f32<A>(qraw[r], qf[r]);
    norm_rope8<A>(qf[r], gf, cf, sf, dc, p.eps);  // q_norm + RoPE (qwen3.rs:220, 224)
  }

  // Scores of a chunk: each lane forms the 16 partials (8 keys x 2 heads of
  // a head pair) over its 8 dims, and a reduce-scatter across the row leaves
  // lane (grp, dc) with the full q.k of key c0 + 4*(dc & 7) + grp and head
  // 2u + (dc >> 3).  The lane then rounds, stores and folds that one score
  // into the running (max, sum of exp) of its head, shared by the 8 lanes of
  // its half-row.
  constexpr int NP = (REP + 1) / 2;  // head pairs
  const int hsel = dc >> 3, isel = dc & 7;
  uint32_t q2[REP][4];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int t = 0; t < 4; ++t)
      q2[r][t] = (uint32_t)st_act<A>(qf[r][2 * t]) | ((uint32_t)st_act<A>(qf[r][2 * t + 1]) << 16);
  float m[NP], l[NP];
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    m[u] = -INFINITY;
    l[u] = 0.f;
  }
  auto fold = [&](int u, float sc) {
    const float cm = half8_max(sc);
    const float mn = fmaxf(m[u], cm);
    const float e = half8_sum((sc == -INFINITY) ? 0.f : __expf(sc - mn));
    if (mn != -INFINITY) {
      l[u] = ((m[u] == -INFINITY) ? 0.f : l[u] * __expf(m[u] - mn)) + e;
      m[u] = mn;
    }
  };
  auto score = [&](int c0, const Chunk<A>* kk) {
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      float v[16];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = 2 * u + hh;
          v[8 * hh + i] = r < REP ? dot8<A>(q2[r < REP ? r : 0], qf[r < REP ? r : 0], kk[i]) : 0.f;
        }
      const float d = rscatter16(v, dc);
      const int r = 2 * u + hsel, key = c0 + 4 * isel + grp;
      const bool ok = r < REP && key < kw1;
      const float sc = ok ? rd<A>(rd<A>(d) * p.scale) : -INFINITY;
      if (ok) sc_out[score_index(p, b, g * REP + r, key)] = st_act<A>(sc);
      fold(u, sc);
    }
  };
  // Fully unrolled over a compile-time number of chunks, so the compiler
  // waits for exactly the chunk being scored; the buffer just scored is
  // refilled with the chunk NB ahead.
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    score(kw0 + c * CH, kbuf[c % NB]);
    if (c + NB < NCH) {
      __builtin_amdgcn_sched_barrier(0);
      load(kw0 + (c + NB) * CH, kbuf[c % NB]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (wr.owner) {
    // The new token (qwen3.rs:221, 225-227): k_norm + RoPE, cache append at
    // `pos`, and its score, added by lane-row 0 of this wave.
    float kf[8], vf[8];
    chunk_f32<A>(kraw, kf);
    chunk_f32<A>(vraw, vf);
    chunk_f32<A>(gk, gf);
    norm_rope8<A>(kf, gf, cf, sf, dc, p.eps);
    if (grp == 0) {
      T* kd = (T*)p.kc + (kvbase + pos) * HD + dc * 8;
      T* vd = (T*)p.vc + (kvbase + pos) * HD + dc * 8;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        kd[t] = st_act<A>(kf[t]);
        vd[t] = st_act<A>(vf[t]);
      }
    }
    float sn[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      float d = 0.f;
#pragma unroll
      for (int t = 0; t < 8; ++t) d += qf[r][t] * kf[t];
      sn[r] = rd<A>(rd<A>(row16_sum(d)) * p.scale);
    }
    if (grp == 0) {
#pragma unroll
      for (int u = 0; u < NP; ++u) {
        const int r = 2 * u + hsel;
        if (r >= REP) continue;
        float snr = sn[0];
#pragma unroll
        for (int rr = 1; rr < REP; ++rr)
          if (rr == r) snr = sn[rr];
        if (isel == 0) sc_out[score_index(p, b, g * REP + r, pos)] = st_act<A>(snr);
        const float mn = fmaxf(m[u], snr);
        l[u] = ((m[u] == -INFINITY) ? 0.f : l[u] * __expf(m[u] - mn)) + __expf(snr - mn);
        m[u] = mn;
      }
    }
  }

  // Merge the 16 lane-rows (4 per wave x 4 waves) of this work-group; the
  // first lane of each half-row holds its head's state.
  __shared__ float s_ml[16][REP][2];
  const int gi = w * 4 + grp;
  if (isel == 0) {
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int r = 2 * u + hsel;
      if (r < REP) {
        s_ml[gi][r][0] = m[u];
        s_ml[gi][r][1] = l[u];
      }
    }
  }
  __syncthreads();
  if (threadIdx.x < REP) {
    const int r = threadIdx.x;
    float M = -INFINITY;
    for (int i = 0; i < 16; ++i) M = fmaxf(M, s_ml[i][r][0]);
    float L = 0.f;
    for (int i = 0; i < 16; ++i)
      if (s_ml[i][r][0] != -INFINITY) L += s_ml[i][r][1] * __expf(s_ml[i][r][0] - M);
    float* dst = p.ml + ((((size_t)b * p.nkv + g) * p.max_splits + split) * REP + r) * 2;
    dst[0] = M;
    dst[1] = L;
  }
}

template <int A, int REP, int NCH>
__global__ void __launch_bounds__(256) attn_value_kernel(AttnDecodeArgs p) {
  typedef typename ActT<A>::T T;
  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  if (p.done && p.done[b]) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int grp = lane >> 4, dc = lane & 15;
  const WaveRange wr = wave_range<NCH>(p, split, b, w);
  if (!wr.active) return;
  const int pos = wr.pos, kw0 = wr.kw0, kw1 = wr.kw1;
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;
  const size_t unit = (size_t)b * p.nkv + g;
  const T* scores = (const T*)p.scores;

  // Loads first, in the order they are needed: the split partials (max, sum
  // of exp) of this (row, KV head) -- at most 128 splits, two per lane --
  // the new token's V row and scores, then the first NB chunks of V with
  // their scores.  Key indices are clamped to a key this split may read, so
  // no load sits behind a branch.
  constexpr int NS = (REP + 1) / 2;
  constexpr int NB = NCH < 2 ? NCH : 2;
  float mlm[REP][2], mll[REP][2];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = min(lane + 64 * h, wr.nsplit - 1);
      const float* ml = p.ml + ((unit * p.max_splits + j) * REP + r) * 2;
      mlm[r][h] = ml[0];
      mll[r][h] = ml[1];
    }
  const Chunk<A> vnew = load_chunk<A>(p.vc, (kvbase + pos) * HD + dc * 8);
  T snew[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) snew[r] = scores[score_index(p, b, g * REP + r, pos)];
  const int kl = max(wr.k1 - 1, wr.k0);
  // The scores of a chunk: lane L holds key c0 + (L & 31) of heads
  // (L >> 5) + 2u (REP >= 2) or of head 0 (REP == 1).
  auto load = [&](int c0, Chunk<A>* vv, T* ss) {
#pragma unroll
    for (int i = 0; i < CH / 4; ++i)
      vv[i] = load_chunk<A>(p.vc, (kvbase + min(c0 + 4 * i + grp, kl)) * HD + dc * 8);
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int r = REP == 1 ? 0 : (lane >> 5) + 2 * u;
      ss[u] = scores[score_index(p, b, g * REP + r, min(c0 + (lane & 31), kl))];
    }
  };
  Chunk<A> vbuf[NB][CH / 4];
  T sbuf[NB][NS];
#pragma unroll
  for (int c = 0; c < NB; ++c) load(kw0 + c * CH, vbuf[c], sbuf[c]);
  __builtin_amdgcn_sched_barrier(0);

  // Global max and sum of exp of each query head, from the split partials in
  // a fixed order (identical in every work-group of this (row, KV head)).
  // Kept as (M log2 e, 1/S): p = rd(2^(s log2 e - M log2 e) * (1/S)).
  float M[REP], S[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    float mx = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (lane + 64 * h < wr.nsplit) mx = fmaxf(mx, mlm[r][h]);
    mx = wave_max(mx);
    float sm = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (lane + 64 * h < wr.nsplit && mlm[r][h] != -INFINITY)
        sm += mll[r][h] * __expf(mlm[r][h] - mx);
    sm = wave_sum(sm);
    M[r] = mx * kLog2e;
    S[r] = 1.f / sm;
  }

  float acc[REP][8];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[r][t] = 0.f;

  auto accumulate = [&](int c0, const Chunk<A>* vv, const T* ss) {
    // p_j = rd(exp(s_j - M) / S), one key and head per lane (qwen3.rs:248)
    float pr[NS];
    const bool ok = c0 + (lane & 31) < kw1;
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int r = REP == 1 ? 0 : (lane >> 5) + 2 * u;
      float Mr = M[0], Sr = S[0];
#pragma unroll
      for (int rr = 1; rr < REP; ++rr)
        if (rr == r) {
          Mr = M[rr];
          Sr = S[rr];
        }
      const float sv = ld_act<A>(ss[u]);
      const float pv = rd<A>(__builtin_amdgcn_exp2f(fmaf(sv, kLog2e, -Mr)) * Sr);   // masked below
      pr[u] = ok ? pv : 0.f;
    }
#pragma unroll
    for (int i = 0; i < CH / 4; ++i) {
      float vf[8];
      chunk_f32<A>(vv[i], vf);
#pragma unroll
      for (int r = 0; r < REP; ++r) {
        const int src = (REP == 1 ? 0 : (r & 1) * 32) + 4 * i + grp;
        const float pj = __shfl(pr[REP == 1 ? 0 : r >> 1], src);
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[r][t] += pj * vf[t];
      }
    }
  };
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    accumulate(kw0 + c * CH, vbuf[c % NB], sbuf[c % NB]);
    if (c + NB < NCH) {
      __builtin_amdgcn_sched_barrier(0);
      load(kw0 + (c + NB) * CH, vbuf[c % NB], sbuf[c % NB]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (wr.owner && grp == 0) {
    // the new token at `pos`, added by lane-row 0 of split 0's first wave
    float vf[8];
    chunk_f32<A>(vnew, vf);
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      const float pn = rd<A>(__builtin_amdgcn_exp2f(fmaf(ld_act<A>(snew[r]), kLog2e, -M[r])) * S[r]);
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[r][t] += pn * vf[t];
    }
  }

  // Add the 16 lane-rows of this work-group.
  __shared__ float s_acc[16][REP][HD];
  const int gi = w * 4 + grp;
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int t = 0; t < 8; ++t) s_acc[gi][r][dc * 8 + t] = acc[r][t];
  __syncthreads();
  for (int t = threadIdx.x; t < REP * HD; t += blockDim.x) {
    const int r = t / HD, d = t % HD;
    float O = 0.f;
    for (int i = 0; i < 16; ++i) O += s_acc[i][r][d];
    p.part[((unit * p.max_splits + split) * REP + r) * HD + d] = O;
  }
}

// Add the splits' shares of one (KV head g, row b) in split order and store
// the context in the activation dtype.
template <int A, int REP>
__global__ void __launch_bounds__(REP * HD) attn_combine_kernel(AttnDecodeArgs p) {
  typedef typename ActT<A>::T T;
  constexpr int MAXU = 16;  // split shares loaded per pass
  const int g = blockIdx.x, b = blockIdx.y;
  if (p.done && p.done[b]) return;
  const int nsplit = row_splits(p.state[0], p.start[b], p.split);
  const size_t unit = (size_t)b * p.nkv + g;
  const int r = threadIdx.x / HD, d = threadIdx.x % HD;
  float O = 0.f;
  for (int j0 = 0; j0 < nsplit; j0 += MAXU) {
    float oj[MAXU];
#pragma unroll
    for (int u = 0; u < MAXU; ++u) {
      const int j = min(j0 + u, nsplit - 1);
      oj[u] = p.part[((unit * p.max_splits + j) * REP + r) * HD + d];
    }
#pragma unroll
    for (int u = 0; u < MAXU; ++u)
      if (j0 + u < nsplit) O += oj[u];
  }
  ((T*)p.out)[(size_t)b * p.nkv * REP * HD + (g * REP + r) * HD + d] = st_act<A>(O);
}

// ---------------------------------------------------------------------------
// Single-launch path (16-bit activations).  The grid is (splits, KV heads,
// 2B): work-groups with z < B do the score pass of row z, work-groups with
// z >= B the value pass and the combine of row z - B.  Every score
// work-group precedes every value work-group in dispatch order and never
// waits, so a value work-group only waits for work that is already running
// or done -- the grid need not be resident at once.
//
//  score work-group: streams K and scores it as attn_score_kernel does;
//    publishes the scores (two keys per word), the new token's score and its
//    (max, sum of exp) per head, then exits.
//  value work-group: issues its V loads first, then reads every split's
//    (max, sum of exp) of its (row, KV head) -- the "unit" -- in split order
//    (so all of them derive the identical M and S), its scores, and forms
//    sum_j rd(exp(s_j - M) / S) v_j; publishes that share, and the last
//    value work-group of the unit to finish (a counter) adds the shares in
//    split order and stores the context.
//
// Exchange words are 64-bit: the launch's epoch in the high half, data in
// the low half, written and read with relaxed device-scope atomics (stores
// and loads that bypass the per-XCD caches, which are not coherent with each
// other).  A word is valid only when it carries the current epoch, so no
// ordering between words is needed and nothing is cleared between launches.
// The epoch advances once per launch: the last unit to finish increments
// it, after every work-group of the launch has read it.  Every wait is
// bounded: past `spin_limit` polls the work-group records an error code in
// sync[2] and goes on, so the launch always drains; the host checks the code.
__device__ __forceinline__ uint64_t tag_word(uint32_t epoch, uint32_t v) {
  return ((uint64_t)epoch << 32) | v;
}
__device__ __forceinline__ void put_word(uint64_t* p, uint64_t w) {
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_word(uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float word_f32(uint64_t w) {
  return __builtin_bit_cast(float, (uint32_t)(w & 0xffffffffu));
}
__device__ __forceinline__ bool word_ok(uint64_t w, uint32_t epoch) {
  return (uint32_t)(w >> 32) == epoch;
}
// The tag of a work-group's exchange words is the launch epoch.  A
// work-group reads the epoch only once the work-group's cache or
// weight loads are out, so that round trip overlaps them instead of
// delaying them.  Reading it late is safe: the epoch advances only when the
// last unit is done, which takes every work-group's published output, and
// each work-group reads the epoch before it publishes.
// (A select, not a branch: a branch around the load would make the compiler
// wait for every load in flight where the paths join.)
struct EpochTag {
  uint32_t* sync;
  __device__ __forceinline__ uint32_t load() const {
    return __hip_atomic_load(sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __device__ __forceinline__ uint32_t make(uint32_t e) const { return e; }
  __device__ __forceinline__ uint32_t get() const { return make(load()); }
};
__device__ __forceinline__ void fail_sync(uint32_t* sync, uint32_t code) {
  __hip_atomic_store(sync + 2, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A wait gives up past `limit` polls (recording `code`), or as soon as some
// other wait of the launch has given up (every 64 polls it checks), so a
// failing launch drains after about one limit's worth of polls.
__device__ __forceinline__ bool give_up(uint32_t* sync, int spins, int limit, uint32_t code) {
  if (spins >= limit) {
    fail_sync(sync, code);
    return true;
  }
  return (spins & 63) == 63 &&
         __hip_atomic_load(sync + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Score work-group of split `split`, KV head g, row b.
template <int A, int REP, int NCH, bool QP>
__device__ __forceinline__ void fused_score(const AttnDecodeArgs& p, int split, int g, int b,
                                            EpochTag tag) {
  typedef typename ActT<A>::T T;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int grp = lane >> 4, dc = lane & 15;
  const WaveRange wr = wave_range<NCH>(p, split, b, w);
  const int pos = wr.pos, kw0 = wr.kw0, kw1 = wr.kw1, s0 = p.start[b];
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;
  const size_t unit = (size_t)b * p.nkv + g;

  const int qd = p.nkv * REP * HD;
  const size_t qrow = (size_t)b * p.ldqkv;
  constexpr int NB = NCH < 2 ? NCH : 2;
  const int kc = max(wr.k1 - 1, wr.k0);
  const void* kb = (const uint16_t*)p.kc + kvbase * HD;  // this unit's keys
  Chunk<A> kbuf[NB][CH / 4];
  auto load = [&](int c0, Chunk<A>* kk) {
#pragma unroll
    for (int i = 0; i < CH / 4; ++i)
      kk[i].v = load16_at(kb, (uint32_t)(min(c0 + 4 * i + grp, kc) * HD + dc * 8) * 2u);
  };
  Chunk<A> qraw[REP], kraw, vraw;
  uint32_t E = 0;
  // q_norm and k_norm gains and RoPE at pos; the k_norm gain, which only
  // the new token's wave uses, is loaded later, which keeps the projected
  // launch within its register budget.
  Chunk<A> gq, gk, cr, sr;
  auto load_small = [&]() {
    gq = load_chunk<A>(p.qn_w, dc * 8);
    cr = load_chunk<A>(p.cos, (size_t)pos * 64 + (dc & 7) * 8);
    sr = load_chunk<A>(p.sin, (size_t)pos * 64 + (dc & 7) * 8);
  };
  if constexpr (QP) {
    // The cached keys do not depend on this launch: they stream in while the
    // projection work-groups produce q, k and v, which lanes 0-15 of wave 0
    // poll for (k and v only in split 0, whose first wave owns the new
    // token) and hand to the work-group through LDS.
#pragma unroll
    for (int c = 0; c < NB; ++c) load(kw0 + c * CH, kbuf[c]);
    load_small();
    __builtin_amdgcn_sched_barrier(0);
    __shared__ u32x4 s_q[REP][16];
    __shared__ uint32_t s_tag;
    if (w == 0 && lane < 16) {
      // The first poll and the epoch go out right behind the keys, so one
      // round trip brings all three when q is already there.  Every split
      // reads k and v (split 0 uses them) so the loads need no branch.
      const int nw = split == 0 ? REP + 2 : REP;
      uint64_t* src = p.xqkv + (size_t)b * (p.ldqkv / 2);
      uint64_t wv[REP + 2][4];
      auto fetch = [&]() {
#pragma unroll
        for (int r = 0; r < REP + 2; ++r) {
          const int col = (r < REP ? (g * REP + r) * HD : qd + (r - REP) * p.nkv * HD + g * HD) + dc * 8;
#pragma unroll
          for (int t = 0; t < 4; ++t) wv[r][t] = get_word(src + col / 2 + t);
        }
      };
      fetch();
      const uint32_t Ew = tag.get();
      for (int spins = 0;; ++spins) {
        bool ok = true;
#pragma unroll
        for (int r = 0; r < REP + 2; ++r)
#pragma unroll
          for (int t = 0; t < 4; ++t) ok = ok && (r >= nw || word_ok(wv[r][t], Ew));
        if (__all(ok)) break;
        if (give_up(p.sync, spins, p.spin_limit, 5)) break;
        __builtin_amdgcn_s_sleep(2);
        fetch();
      }
#pragma unroll
      for (int r = 0; r < REP + 2; ++r) {
        const u32x4 c = {(uint32_t)wv[r][0], (uint32_t)wv[r][1], (uint32_t)wv[r][2], (uint32_t)wv[r][3]};
        if (r < REP) qraw[r].v = c;
        else if (r == REP) kraw.v = c;
        else vraw.v = c;
      }
#pragma unroll
      for (int r = 0; r < REP; ++r) s_q[r][lane] = qraw[r].v;
      if (lane == 0) s_tag = Ew;
    }
    __syncthreads();
    E = s_tag;
#pragma unroll
    for (int r = 0; r < REP; ++r) qraw[r].v = s_q[r][dc];
    gk = load_chunk<A>(p.kn_w, dc * 8);
  } else {
    E = tag.get();  // first in issue order: using it waits for nothing else
#pragma unroll
    for (int r = 0; r < REP; ++r)
      qraw[r] = load_chunk<A>(p.qkv, qrow + (g * REP + r) * HD + dc * 8);
    kraw = load_chunk<A>(p.qkv, qrow + qd + g * HD + dc * 8);
    vraw = load_chunk<A>(p.qkv, qrow + qd + p.nkv * HD + g * HD + dc * 8);
  }
  if constexpr (!QP) {
    load_small();
    gk = load_chunk<A>(p.kn_w, dc * 8);
#pragma unroll
    for (int c = 0; c < NB; ++c) load(kw0 + c * CH, kbuf[c]);
  }
  __builtin_amdgcn_sched_barrier(0);

  float cf[8], sf[8];
  chunk_f32<A>(cr, cf);
  chunk_f32<A>(sr, sf);
  constexpr int NP = (REP + 1) / 2;
  const int hsel = dc >> 3, isel = dc & 7;
  uint32_t q2[REP][4];
  {
    float gf[8];
    chunk_f32<A>(gq, gf);
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      float qf[8];
      chunk_f32<A>(qraw[r], qf);
      norm_rope8<A>(qf, gf, cf, sf, dc, p.eps);  // q_norm + RoPE (qwen3.rs:220, 224)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        q2[r][t] = (uint32_t)st_act<A>(qf[2 * t]) | ((uint32_t)st_act<A>(qf[2 * t + 1]) << 16);
    }
  }
  float m[NP], l[NP];
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    m[u] = -INFINITY;
    l[u] = 0.f;
  }
  if (wr.owner) {
    // The new token (qwen3.rs:221, 225-227): k_norm + RoPE, cache append at
    // `pos`, its score published and counted by lane-row 0 (m = s, l = 1).
    float kf[8], gkf[8];
    chunk_f32<A>(kraw, kf);
    chunk_f32<A>(gk, gkf);
    norm_rope8<A>(kf, gkf, cf, sf, dc, p.eps);
    Chunk<A> kn;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      kn.v[t] = (uint32_t)st_act<A>(kf[2 * t]) | ((uint32_t)st_act<A>(kf[2 * t + 1]) << 16);
    if (grp == 0) {
      *(u32x4*)((T*)p.kc + (kvbase + pos) * HD + dc * 8) = kn.v;
      *(u32x4*)((T*)p.vc + (kvbase + pos) * HD + dc * 8) = vraw.v;
    }
    float sn[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) sn[r] = rd<A>(rd<A>(row16_sum(dot8<A>(q2[r], nullptr, kn))) * p.scale);
    float mine = sn[0];
#pragma unroll
    for (int r = 1; r < REP; ++r)
      if (lane == r) mine = sn[r];
    if (lane < REP) put_word(p.xnew + unit * REP + lane, tag_word(E, __builtin_bit_cast(uint32_t, mine)));
    if (grp == 0) {
#pragma unroll
      for (int u = 0; u < NP; ++u) {
        const int r = 2 * u + hsel;
        float snr = sn[0];
#pragma unroll
        for (int rr = 1; rr < REP; ++rr)
          if (rr == r) snr = sn[rr];
        if (r < REP) {
          m[u] = snr;
          l[u] = 1.f;
        }
      }
    }
  }
  auto fold = [&](int u, float sc) {
    const float cm = half8_max(sc);
    const float mn = fmaxf(m[u], cm);
    const float e = half8_sum((sc == -INFINITY) ? 0.f : __expf(sc - mn));
    if (mn != -INFINITY) {
      l[u] = ((m[u] == -INFINITY) ? 0.f : l[u] * __expf(m[u] - mn)) + e;
      m[u] = mn;
    }
  };
  // Scores of key pairs (key - s0 even, odd) share a word: the even key's
  // lane-row (grp even) packs its score with the partner row's.
  uint64_t* xsc = p.xsc + unit * REP * (size_t)p.xsc_stride;
  auto score = [&](int c0, const Chunk<A>* kk) {
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      float v[16];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = 2 * u + hh;
          v[8 * hh + i] = r < REP ? dot8<A>(q2[r < REP ? r : 0], nullptr, kk[i]) : 0.f;
        }
      const float d = rscatter16(v, dc);
      const int r = 2 * u + hsel, key = c0 + 4 * isel + grp;
      const bool ok = r < REP && key < kw1;
      const float sc = ok ? rd<A>(rd<A>(d) * p.scale) : -INFINITY;
      const float other = __shfl_xor(sc, 16);
      if (!(grp & 1) && r < REP && key < kw1)
        put_word(xsc + (size_t)r * p.xsc_stride + (key - s0) / 2,
                 tag_word(E, (uint32_t)st_act<A>(sc) | ((uint32_t)st_act<A>(other) << 16)));
      fold(u, sc);
    }
  };
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    score(kw0 + c * CH, kbuf[c % NB]);
    if (c + NB < NCH) {
      __builtin_amdgcn_sched_barrier(0);
      load(kw0 + (c + NB) * CH, kbuf[c % NB]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Merge the 16 lane-rows and publish (max, sum of exp) per head.
  __shared__ float s_ml[16][REP][2];
  const int gi = w * 4 + grp;
  if (isel == 0) {
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int r = 2 * u + hsel;
      if (r < REP) {
        s_ml[gi][r][0] = m[u];
        s_ml[gi][r][1] = l[u];
      }
    }
  }
  __syncthreads();
  if (threadIdx.x < REP) {
    const int r = threadIdx.x;
    float M = -INFINITY;
    for (int i = 0; i < 16; ++i) M = fmaxf(M, s_ml[i][r][0]);
    float L = 0.f;
    for (int i = 0; i < 16; ++i)
      if (s_ml[i][r][0] != -INFINITY) L += s_ml[i][r][1] * __expf(s_ml[i][r][0] - M);
    uint64_t* dst = p.xml + ((unit * p.max_splits + split) * REP + r) * 2;
    put_word(dst, tag_word(E, __builtin_bit_cast(uint32_t, M)));
    put_word(dst + 1, tag_word(E, __builtin_bit_cast(uint32_t, L)));
  }
}

// Value work-group of split `split`, KV head g, row b.
template <int A, int REP, int NCH, bool QP>
__device__ __forceinline__ void fused_value(const AttnDecodeArgs& p, int split, int g, int b,
                                            EpochTag tag) {
  typedef typename ActT<A>::T T;
  constexpr int NS = (REP + 1) / 2;
  constexpr int NB = NCH < 2 ? NCH : 2;
  constexpr int NOUT = REP * HD;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int grp = lane >> 4, dc = lane & 15;
  const WaveRange wr = wave_range<NCH>(p, split, b, w);
  const int kw0 = wr.kw0, kw1 = wr.kw1, nsplit = wr.nsplit, s0 = p.start[b];
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;
  const size_t unit = (size_t)b * p.nkv + g;

  // What this wave needs from the score work-groups: every split's (max,
  // sum of exp) of the unit (lane j holds split j; at most 64), the scores
  // of its keys (lane L holds key c0 + (L & 31) of head (L >> 5) + 2u, or of
  // head 0 when REP == 1, for every chunk) and, for split 0's first wave,
  // the new token's scores.  These loads go out before the V loads, so when
  // the score work-groups are done (the usual case) one round trip brings
  // both; otherwise the wave polls again.
  uint64_t* xml = p.xml + unit * p.max_splits * REP * 2;
  uint64_t* xsc = p.xsc + unit * REP * (size_t)p.xsc_stride;
  uint64_t wm[REP][2], ws[NCH][NS], wn[REP];
  auto poll = [&]() {
    const int j = min(lane, nsplit - 1);
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      wm[r][0] = get_word(xml + (j * REP + r) * 2);
      wm[r][1] = get_word(xml + (j * REP + r) * 2 + 1);
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int u = 0; u < NS; ++u) {
        const int r = REP == 1 ? 0 : (lane >> 5) + 2 * u;
        const int key = min(kw0 + c * CH + (lane & 31), max(kw1 - 1, kw0));
        ws[c][u] = get_word(xsc + (size_t)r * p.xsc_stride + max(key - s0, 0) / 2);
      }
    if (wr.owner) {
#pragma unroll
      for (int r = 0; r < REP; ++r) wn[r] = get_word(p.xnew + unit * REP + r);
    }
  };
  // The epoch goes out first, then the poll, then V: the first check waits
  // only for the first two.
  const uint32_t e0 = tag.load();
  uint32_t E = 0;
  auto polled = [&]() {
    bool ok = true;
#pragma unroll
    for (int r = 0; r < REP; ++r) ok = ok && word_ok(wm[r][0], E) && word_ok(wm[r][1], E);
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int u = 0; u < NS; ++u) ok = ok && (kw0 + c * CH >= kw1 || word_ok(ws[c][u], E));
    if (wr.owner) {
#pragma unroll
      for (int r = 0; r < REP; ++r) ok = ok && word_ok(wn[r], E);
    }
    return (bool)__all(ok);
  };
  poll();
  __builtin_amdgcn_sched_barrier(0);

  // V: it does not depend on anything this launch computes.  The new token's
  // v comes from the projection (split 0's first wave adds it).
  const int kl = max(wr.k1 - 1, wr.k0);
  const void* vb = (const uint16_t*)p.vc + kvbase * HD;  // this unit's values
  auto loadv = [&](int c0, Chunk<A>* vv) {
#pragma unroll
    for (int i = 0; i < CH / 4; ++i)
      vv[i].v = load16_at(vb, (uint32_t)(min(c0 + 4 * i + grp, kl) * HD + dc * 8) * 2u);
  };
  Chunk<A> vbuf[NB][CH / 4];
#pragma unroll
  for (int c = 0; c < NB; ++c) loadv(kw0 + c * CH, vbuf[c]);
  Chunk<A> vnew;
  const int vcol = p.nkv * REP * HD + p.nkv * HD + g * HD + dc * 8;  // the new token's v
  uint64_t vw[4];
  if constexpr (QP) {
    // From the projection work-groups; every wave reads it (no branch) and
    // lane-row 0 of split 0's first wave, the lanes that add the new token,
    // polls until it is there.
#pragma unroll
    for (int t = 0; t < 4; ++t) vw[t] = get_word(p.xqkv + (size_t)b * (p.ldqkv / 2) + vcol / 2 + t);
  } else {
    vnew = load_chunk<A>(p.qkv, (size_t)b * p.ldqkv + vcol);
  }
  __builtin_amdgcn_sched_barrier(0);
  E = tag.make(e0);
  if constexpr (QP) {
    if (wr.owner && grp == 0) {
      for (int spins = 0;; ++spins) {
        bool ok = true;
#pragma unroll
        for (int t = 0; t < 4; ++t) ok = ok && word_ok(vw[t], E);
        if (ok) break;
        if (give_up(p.sync, spins, p.spin_limit, 6)) break;
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
        for (int t = 0; t < 4; ++t) vw[t] = get_word(p.xqkv + (size_t)b * (p.ldqkv / 2) + vcol / 2 + t);
      }
    }
    vnew.v = u32x4{(uint32_t)vw[0], (uint32_t)vw[1], (uint32_t)vw[2], (uint32_t)vw[3]};
  }
  for (int spins = 0; !polled(); ++spins) {
    if (give_up(p.sync, spins, p.spin_limit, 1)) break;
    __builtin_amdgcn_s_sleep(2);
    poll();
  }

  // M and S of each head from the split pairs in a fixed order (identical in
  // every wave of the unit), kept as (M log2 e, 1/S):
  // p = rd(2^(s log2 e - M log2 e) * (1/S)).
  float M[REP], S[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    const float m = word_f32(wm[r][0]);
    const float mx = wave_max(lane < nsplit ? m : -INFINITY);
    const float sm =
        wave_sum((lane < nsplit && m != -INFINITY) ? word_f32(wm[r][1]) * __expf(m - mx) : 0.f);
    M[r] = mx * kLog2e;
    S[r] = 1.f / sm;
  }

  float acc[REP][8];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[r][t] = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    // p_j = rd(exp(s_j - M) / S), one key and head per lane (qwen3.rs:248);
    // keys outside [kw0, kw1) get p = 0.  Lane L then packs its p with the
    // p of key + 4 (lane L + 4), the key its lane-row holds in the next load.
    uint32_t pk[NS];
    const int key = kw0 + c * CH + (lane & 31);
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int r = REP == 1 ? 0 : (lane >> 5) + 2 * u;
      float Mr = M[0], Sr = S[0];
#pragma unroll
      for (int rr = 1; rr < REP; ++rr)
        if (rr == r) {
          Mr = M[rr];
          Sr = S[rr];
        }
      const uint32_t h16 = ((key - s0) & 1) ? (uint32_t)(ws[c][u] >> 16) & 0xffffu
                                             : (uint32_t)ws[c][u] & 0xffffu;
      const float sv = ld_act<A>((T)h16);
      const float pv = key < kw1 ? rd<A>(__builtin_amdgcn_exp2f(fmaf(sv, kLog2e, -Mr)) * Sr) : 0.f;
      const uint32_t mine = (uint32_t)st_act<A>(pv);
      const uint32_t next = (uint32_t)__shfl((int)mine, (lane & 32) | ((lane + 4) & 31));
      pk[u] = mine | (next << 16);
    }
    // sum_j p_j v_j two keys at a time: loads i and i + 1 of a lane hold keys
    // k and k + 4 with the same dims, so byte permutes give the (k, k + 4)
    // pair of each dim and one packed dot product adds both keys' terms
    // (exact 16-bit products, f32 sums).
    const Chunk<A>* vv = vbuf[c % NB];
#pragma unroll
    for (int i = 0; i < CH / 4; i += 2) {
      uint32_t x[4], y[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t a0 = vv[i].v[t], a1 = vv[i + 1].v[t];
        x[t] = __builtin_amdgcn_perm(a1, a0, 0x05040100u);  // (dim 2t of k, of k + 4)
        y[t] = __builtin_amdgcn_perm(a1, a0, 0x07060302u);  // (dim 2t + 1 of k, of k + 4)
      }
#pragma unroll
      for (int r = 0; r < REP; ++r) {
        const int src = (REP == 1 ? 0 : (r & 1) * 32) + 4 * i + grp;
        const uint32_t pp = (uint32_t)__shfl((int)pk[REP == 1 ? 0 : r >> 1], src);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          acc[r][2 * t] = dot2acc<A>(pp, x[t], acc[r][2 * t]);
          acc[r][2 * t + 1] = dot2acc<A>(pp, y[t], acc[r][2 * t + 1]);
        }
      }
    }
    if (c + NB < NCH) {
      __builtin_amdgcn_sched_barrier(0);
      loadv(kw0 + (c + NB) * CH, vbuf[c % NB]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (wr.owner && grp == 0) {
    float vf[8];
    chunk_f32<A>(vnew, vf);
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      const float pn = rd<A>(__builtin_amdgcn_exp2f(fmaf(word_f32(wn[r]), kLog2e, -M[r])) * S[r]);
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[r][t] += pn * vf[t];
    }
  }

  // This work-group's share: the 16 lane-rows added in LDS, then published.
  __shared__ float s_acc[16][REP][HD];
  const int gi = w * 4 + grp;
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int t = 0; t < 8; ++t) s_acc[gi][r][dc * 8 + t] = acc[r][t];
  __syncthreads();
  uint64_t* xpart = p.xpart + unit * p.max_splits * NOUT;
  float own[(NOUT + 255) / 256];
#pragma unroll
  for (int k = 0; k < (NOUT + 255) / 256; ++k) {
    const int t = threadIdx.x + 256 * k;
    own[k] = 0.f;
    if (t < NOUT) {
      const int r = t / HD, d = t % HD;
      float O = 0.f;
      for (int i = 0; i < 16; ++i) O += s_acc[i][r][d];
      own[k] = O;
      if (split != 0) put_word(xpart + (size_t)split * NOUT + t, tag_word(E, __builtin_bit_cast(uint32_t, O)));
    }
  }
  if (split != 0) return;

  // Split 0 adds the other splits' shares to its own in split order and
  // stores the context; the other value work-groups of the unit were
  // dispatched after it, so it waits only for running or queued work.
  constexpr int G = 16;
#pragma unroll
  for (int k = 0; k < (NOUT + 255) / 256; ++k) {
    const int t = threadIdx.x + 256 * k;
    if (t >= NOUT) continue;
    float O = own[k];
    for (int j0 = 1; j0 < nsplit; j0 += G) {
      float vj[G];
      for (int spins = 0;; ++spins) {
        bool ok = true;
#pragma unroll
        for (int u = 0; u < G; ++u) {
          const int j = min(j0 + u, nsplit - 1);
          const uint64_t x = get_word(xpart + (size_t)j * NOUT + t);
          ok = ok && word_ok(x, E);
          vj[u] = word_f32(x);
        }
        if (ok) break;
        if (give_up(p.sync, spins, p.spin_limit, 2)) break;
        __builtin_amdgcn_s_sleep(2);
      }
#pragma unroll
      for (int u = 0; u < G; ++u)
        if (j0 + u < nsplit) O += vj[u];
    }
    ((T*)p.out)[(size_t)b * p.nkv * NOUT + g * NOUT + t] = st_act<A>(O);
  }
  if (threadIdx.x == 0 && p.count_units) {
    // The last unit of the launch advances the epoch; by then every
    // work-group of the launch has read it.  (In a decode step the O
    // projection kernel that follows advances it instead, which keeps
    // these atomics' round trips off the end of the launch.)
    int live = 0;
    for (int bb = 0; bb < p.batch; ++bb) live += (p.done && p.done[bb]) ? 0 : 1;
    const uint32_t units = (uint32_t)(live * p.nkv);
    const uint32_t old = __hip_atomic_fetch_add(p.sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == units - 1) {
      __hip_atomic_fetch_sub(p.sync + 1, units, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(p.sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

__device__ __forceinline__ u32x4 q8_to_f16x8(uint32_t w0, uint32_t w1) {
  uint32_t a, b, c, d;
  i8x4_to_f16x4(w0, a, b);
  i8x4_to_f16x4(w1, c, d);
  return u32x4{a, b, c, d};
}

template <int A>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (A == ACT_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Dispatch order of the attention work-groups (U units of S splits each,
// unit u = KV head u % nkv of row u / nkv): every score work-group, then
// every value work-group, so a value work-group follows its unit's score
// work-groups.  (Interleaving value work-groups behind the score stream was
// measured slower: waiting value work-groups hold slots that score
// work-groups would stream with.  So was dispatching units in groups, each
// group's score then value work-groups: int8 batch 8 at 4096 keys, 1.74 /
// 1.71 / 1.62 ms per step for groups of 1 / 4 / 16 units against 1.34.)
__host__ __device__ inline void role_of(int i, int S, int U, bool* value, int* split, int* unit) {
  *value = i >= S * U;
  if (*value) i -= S * U;
  *unit = i / S;
  *split = i % S;
}

// --- projections inside a launch -----------------------------------------
// A projection work-group owns 16 output columns (one weight row-tile) for
// every row, as the decode projection kernel does: wave w multiplies inputs
// [k0 + 256w, k0 + 256w + 256) on the 16x16 MFMAs (rows = batch, zero-padded)
// and the partial tiles are added in wave order.  Its input comes either
// from plain memory written before the launch or from exchange words.

// Weights of row-tile `tile`, inputs [k0, k0 + 256): Q8_0 as 4 chunks of 64
// with their scales, dense 16-bit as 8 chunks of 32 (the B-operand tiling).
template <int WK>
__device__ __forceinline__ void load_wslice(const LinWeights& W, int tile, int k0, u32x4* wv,
                                            uint32_t* wsc) {
  const int lane = threadIdx.x & 63;
  if constexpr (WK == WK_Q8) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const size_t ch = (size_t)tile * (W.in / 64) + k0 / 64 + c;
      wv[c] = __builtin_nontemporal_load(((const u32x4*)W.w) + ch * 64 + lane);
      wsc[c] = __builtin_nontemporal_load(W.sc + ch * 16 + (lane & 15));
    }
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const size_t ch = (size_t)tile * (W.in / 32) + k0 / 32 + c;
      wv[c] = __builtin_nontemporal_load(((const u32x4*)W.w) + ch * 64 + lane);
    }
  }
}

template <int A, int WK>
__device__ __forceinline__ f32x4 slice_mfma(const u32x4* xa, const u32x4* wv, const uint32_t* wsc,
                                            f32x4 acc) {
  if constexpr (WK == WK_Q8) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      const f32x4 t0 = mfma16<ACT_F16>(xa[2 * c], q8_to_f16x8(wv[c][0], wv[c][1]), z);
      const f32x4 t1 = mfma16<ACT_F16>(xa[2 * c + 1], q8_to_f16x8(wv[c][2], wv[c][3]), z);
      acc += f16_to_f32((uint16_t)(wsc[c] & 0xffffu)) * t0;
      acc += f16_to_f32((uint16_t)(wsc[c] >> 16)) * t1;
    }
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) acc = mfma16<A>(xa[c], wv[c], acc);
  }
  return acc;
}

// Eight gain values per thread (threads past K / 8 repeat the last eight),
// loaded with x and staged through LDS by norm_slice, so that no load waits
// for the norm's barrier.  K is at most 2048.
__device__ __forceinline__ u32x4 load_gain(const void* gain, int K) {
  return *((const u32x4*)gain + min((int)threadIdx.x, K / 8 - 1));
}

// RMSNorm of the rows held in xa (this wave's slice at k0; waves < nw hold
// one), over `K` inputs, with the gain (g8 from load_gain) applied and the
// result rounded to the dtype (linear.rs:293-302) -- the same operations,
// in the same order, as the decode projection kernel.
template <int A>
__device__ __forceinline__ void norm_slice(u32x4* xa, u32x4 g8, int k0, int K, bool live, int nw,
                                           float eps, float (*s_ss)[16]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = lane & 15, kg = lane >> 4;
  __shared__ u32x4 s_g[256];
  s_g[min((int)threadIdx.x, K / 8 - 1)] = g8;
  float ss = 0.f;
  if (live) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v[8];
      unpack8<A>(xa[i], v);
#pragma unroll
      for (int t = 0; t < 8; ++t) ss += v[t] * v[t];
    }
  }
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  if (kg == 0) s_ss[w][row] = ss;
  __syncthreads();
  if (!live) return;
  float tot = 0.f;
  for (int i = 0; i < nw; ++i) tot += s_ss[i][row];
  const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(tot, (float)K), eps)));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float v[8], gg[8];
    unpack8<A>(xa[i], v);
    unpack8<A>(s_g[(k0 >> 3) + 4 * i + kg], gg);
    uint32_t o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      o[t] = (uint32_t)st_act<A>(__fmul_rn(__fmul_rn(v[2 * t], rinv), gg[2 * t])) |
             ((uint32_t)st_act<A>(__fmul_rn(__fmul_rn(v[2 * t + 1], rinv), gg[2 * t + 1])) << 16);
    xa[i] = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// Sum of the waves' partial tiles for output (b, n) = thread 16b + n: C[b][n]
// sits in lane 16(b/4) + n, element b%4.
__device__ __forceinline__ float reduce_tile(f32x4 acc, int nw, f32x4 (*s_red)[64]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  s_red[w][lane] = acc;
  __syncthreads();
  const int bb = threadIdx.x >> 4, n = threadIdx.x & 15;
  float v = 0.f;
  for (int ww = 0; ww < nw; ++ww) v += s_red[ww][16 * (bb >> 2) + n][bb & 3];
  return v;
}

// Publishes a 16-bit value per thread (b, n) two columns per word.
template <int A>
__device__ __forceinline__ void put_pair(uint64_t* xw, int ldw, int col0, int batch, float v,
                                         uint32_t tag) {
  const int lane = threadIdx.x & 63, bb = threadIdx.x >> 4, n = threadIdx.x & 15;
  const uint32_t h = (uint32_t)st_act<A>(v);
  const uint32_t hn = (uint32_t)__shfl((int)h, (lane + 1) & 63);
  if (!(n & 1) && bb < batch) put_word(xw + (size_t)bb * ldw + (col0 + n) / 2, tag_word(tag, h | (hn << 16)));
}

// q|k|v projection tile with the input RMSNorm (qwen3.rs:213) of the rows
// in plain memory, published two columns per exchange word.
template <int A, int WK>
__device__ __forceinline__ void fused_qkv(const AttnDecodeArgs& p, const void* xplain, int ldx,
                                          const void* gain, const LinWeights& W, int K, int tile,
                                          uint64_t* out, int ldo, EpochTag tag) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = lane & 15, kg = lane >> 4;
  const int NW = K / 256;
  const bool live = w < NW;
  __shared__ f32x4 s_red[4][64];
  __shared__ float s_ss[4][16];
  // Every load goes out before the first wait, without branches (which
  // would make the compiler wait at the join): waves past K (live false)
  // repeat the last slice and rows past the batch read the last row, and
  // neither is used.
  const int k0 = min(w, NW - 1) * 256;
  u32x4 xa[8];
  u32x4 wv[(WK == WK_Q8) ? 4 : 8];
  uint32_t wsc[4];
  load_wslice<WK>(W, tile, k0, wv, wsc);
  __builtin_amdgcn_sched_barrier(0);
  const u32x4 g8 = load_gain(gain, K);
  const uint16_t* x = (const uint16_t*)xplain + (size_t)min(row, p.batch - 1) * ldx + k0 + 8 * kg;
#pragma unroll
  for (int i = 0; i < 8; ++i) xa[i] = *(const u32x4*)(x + 32 * i);
  const uint32_t E = tag.get();
  // A launch whose rows are all done runs no score or value work, so no unit
  // finishes and its epoch does not advance: words published here would
  // carry the epoch the next launch uses and could be read by it in place of
  // that launch's own.  Such a launch publishes nothing.
  bool any_live = true;
  if (p.done) {
    any_live = false;
    for (int b = 0; b < p.batch; ++b) any_live = any_live || !p.done[b];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) xa[i] = (row < p.batch) ? xa[i] : u32x4{0, 0, 0, 0};
  norm_slice<A>(xa, g8, k0, K, live, NW, p.eps, s_ss);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (live) acc = slice_mfma<A, WK>(xa, wv, wsc, acc);
  const float v = reduce_tile(acc, NW, s_red);
  if (any_live) put_pair<A>(out, ldo, tile * 16, p.batch, v, E);
}

// Grid (1-D, in dispatch order): [nq projection tiles when QP] [score
// work-groups] [value work-groups]; work-group i of a role is split
// i % max_splits, KV head (i / max_splits) % nkv, row i / (max_splits nkv).
// Waves per SIMD the register budget is held to: 4 where the code fits in
// 128 registers without spilling (f16, up to 2 chunks per wave), else the
// compiler's choice.
template <int A, int NCH>
constexpr int fused_waves() {
  return (A == ACT_F16 && NCH <= 2) ? 4 : 1;
}

template <int A, int REP, int NCH, bool QP>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(fused_waves<A, NCH>())))
attn_fused_kernel(AttnDecodeArgs p) {
  static_assert(A != ACT_F32, "16-bit activations only");
  int i = blockIdx.x;
  const EpochTag T{p.sync};
  if constexpr (QP) {
    if (i < p.nq) {
      if (p.Wqkv.kind == WK_Q8) {
        if constexpr (A == ACT_F16)
          fused_qkv<A, WK_Q8>(p, p.x, p.ldx, p.norm_w, p.Wqkv, p.hidden, i, p.xqkv,
                              p.ldqkv / 2, T);
      } else {
        fused_qkv<A, WK_DENSE>(p, p.x, p.ldx, p.norm_w, p.Wqkv, p.hidden, i, p.xqkv,
                               p.ldqkv / 2, T);
      }
      return;
    }
    i -= p.nq;
  }
  bool value;
  int split, unit;
  role_of(i, p.max_splits, p.nkv * p.batch, &value, &split, &unit);
  const int g = unit % p.nkv, b = unit / p.nkv;
  if (p.done && p.done[b]) return;
  if (split >= row_splits(p.state[0], p.start[b], p.split)) return;  // uniform
  if (value)
    fused_value<A, REP, NCH, QP>(p, split, g, b, T);
  else
    fused_score<A, REP, NCH, QP>(p, split, g, b, T);
}

template <int A, int REP, int NCH>
hipError_t launch_fused(const AttnDecodeArgs& a, hipStream_t s) {
  const int roles = 2 * a.max_splits * a.nkv * a.batch;
  if (a.nq > 0) {
    if (!a.xqkv || a.hidden % 256 || a.hidden > 1024 || a.ldqkv % 2 || a.nq * 16 != a.ldqkv ||
        (a.Wqkv.kind == WK_Q8 && A != ACT_F16))
      return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_fused_kernel<A, REP, NCH, true>), dim3(a.nq + roles), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((attn_fused_kernel<A, REP, NCH, false>), dim3(roles), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

template <int A, int REP, int NCH>
hipError_t launch_nch(const AttnDecodeArgs& a, hipStream_t s) {
  const dim3 grid(a.max_splits, a.nkv, a.batch);
  hipLaunchKernelGGL((attn_score_kernel<A, REP, NCH>), grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_value_kernel<A, REP, NCH>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int A, int REP>
hipError_t launch_rep_split(const AttnDecodeArgs& a, hipStream_t s) {
  if (a.max_splits > 128 || a.rep != REP) return hipErrorInvalidValue;
  if (a.fused) {
    if constexpr (A != ACT_F32) {
      if (!a.sync || !a.xml || !a.xpart || !a.xsc || !a.xnew) return hipErrorInvalidValue;
      if constexpr (REP == 2) {
        if (a.max_splits > 64) return hipErrorInvalidValue;
        if (a.split == 4 * CH) return launch_fused<A, REP, 1>(a, s);
        if (a.split == 8 * CH) return launch_fused<A, REP, 2>(a, s);
        if (a.split == 16 * CH) return launch_fused<A, REP, 4>(a, s);
        if (a.split == 32 * CH) return launch_fused<A, REP, 8>(a, s);
      }
    }
    return hipErrorInvalidValue;
  }
  hipError_t e;
  if (a.split == 4 * CH)
    e = launch_nch<A, REP, 1>(a, s);
  else if (a.split == 8 * CH)
    e = launch_nch<A, REP, 2>(a, s);
  else if (a.split == 16 * CH)
    e = launch_nch<A, REP, 4>(a, s);
  else
    return hipErrorInvalidValue;
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_combine_kernel<A, REP>), dim3(a.nkv, a.batch), dim3(REP * HD), 0, s, a);
  return hipGetLastError();
}

template <int A>
hipError_t launch_rep(const AttnDecodeArgs& a, hipStream_t s) {
  switch (a.rep) {
    case 1: return launch_rep_split<A, 1>(a, s);
    case 2: return launch_rep_split<A, 2>(a, s);
    case 4: return launch_rep_split<A, 4>(a, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Keys per split (4 waves x 1, 2 or 4 chunks of CH keys) for a cache of
// `cap` positions and `units` (row, KV head) pairs: the longest split that
// still gives at least FMD_ATTN_TARGET_WGS work-groups at full capacity.
// Capacities needing more than 128 splits of 512 keys are rejected by the
// launcher.
int attn_decode_split(int cap, int units) {
  int split = 16 * CH;
  while (split > 4 * CH && (long)units * ((cap + split - 1) / split) < FMD_ATTN_TARGET_WGS)
    split /= 2;
  return split;
}

// The single-launch path runs for 16-bit activations and GQA repeat 2, with
// the three-kernel path's split (longer when that gives more than 64
// splits).  f32 activations and other repeats keep the three kernels.
AttnDecodePlan attn_decode_plan(int act, int rep, int cap, int units) {
  AttnDecodePlan pl{};
  pl.split = attn_decode_split(cap, units);
  pl.max_splits = (cap + pl.split - 1) / pl.split;
  if (act == ACT_F32 || rep != 2) return pl;
  // a value work-group reads every split's (max, sum of exp) with one lane
  // each: at most 64 splits, so long caches take longer splits
  while (pl.max_splits > 64 && pl.split < 32 * CH) {
    pl.split *= 2;
    pl.max_splits = (cap + pl.split - 1) / pl.split;
  }
  pl.fused = pl.max_splits <= 64;
  return pl;
}

hipError_t launch_attn_decode(int act, const AttnDecodeArgs& a, hipStream_t s) {
  if (a.batch <= 0) return hipSuccess;
  switch (act) {
    case ACT_F32: return launch_rep<ACT_F32>(a, s);
    case ACT_F16: return launch_rep<ACT_F16>(a, s);
    case ACT_BF16: return launch_rep<ACT_BF16>(a, s);
  }
  return hipErrorInvalidValue;
}
