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
//  attn_score_kernel: one work-group per (split of the keys [pad_b, pos],
//    KV head, row).  Each wave normalises and rotates its REP query heads from
//    the raw qkv projection, then streams K in chunks of 32 keys: a 16-lane row
//    of the wave holds one key (8 dims per lane, one 16-byte load), so each
//    wave load is 1 KiB contiguous, and chunk c+1's loads are in flight while
//    chunk c is scored.  Scores go to a (B, nh, cap) buffer in the activation
//    dtype (they are dtype values already); each split writes its (max, sum of
//    exp) per query head.  The wave whose range ends at the new token
//    normalises and rotates its k, appends k and v to the cache and scores it
//    from registers.
//  attn_value_kernel: same grid.  Every work-group of a (row, KV head) derives
//    M and S from the split partials in the same order, so all of them round
//    p_j identically; it then streams V with the scores and writes its share
//    of sum_j p_j v_j.
//  attn_combine_kernel: one work-group per (KV head, row) adds the splits'
//    shares in split order and stores the context.
// (A single kernel whose last work-group merges would need an agent-scope
// fence per work-group -- an L2 write-back plus invalidate on this multi-XCD
// part -- which costs far more than the extra launches.)
#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

constexpr int HD = 128;
#ifndef FMD_ATTN_TARGET_WGS
#define FMD_ATTN_TARGET_WGS 1024
#endif
constexpr int CH = 32;  // keys per wave chunk

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

// RMSNorm over head_dim then rotate-half RoPE, for the 8 dims dc*8..dc*8+7
// held by this lane of a 16-lane row (the row holds the whole head).  The
// rotation partner of dim i is i +- 64, held by lane dc ^ 8.  Explicitly
// rounded operations keep the stored bits equal to a plain IEEE evaluation.
template <int A>
__device__ __forceinline__ void norm_rope8(float* x, const void* gain, const void* cosb,
                                           const void* sinb, int pos, int dc, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) ss = __fadd_rn(ss, __fmul_rn(x[t], x[t]));
  ss = row16_sum(ss);
  const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(ss, 128.0f), eps)));
  float g[8], c[8], s[8];
  load8<A>(gain, dc * 8, g);
  load8<A>(cosb, (size_t)pos * 64 + (dc & 7) * 8, c);
  load8<A>(sinb, (size_t)pos * 64 + (dc & 7) * 8, s);
  float y[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) y[t] = rd<A>(__fmul_rn(__fmul_rn(x[t], rinv), g[t]));
  const bool lo = dc < 8;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float other = __shfl_xor(y[t], 8);  // partner dim (i +- 64)
    x[t] = lo ? rd<A>(__fsub_rn(__fmul_rn(y[t], c[t]), __fmul_rn(other, s[t])))
              : rd<A>(__fadd_rn(__fmul_rn(y[t], c[t]), __fmul_rn(other, s[t])));
  }
}

// Key range of one wave: split `split` of row b covers [k0, k1) of the row's
// keys [s0, pos]; wave w takes [kw0, kw1) of it.
struct WaveRange {
  int pos, nsplit, kw0, kw1;
  bool active;
};
template <int NCH>
__device__ __forceinline__ WaveRange wave_range(const AttnDecodeArgs& p, int split, int b, int w) {
  WaveRange r;
  r.pos = p.state[0];
  const int s0 = p.start[b];
  r.nsplit = (r.pos + 1 - s0 + p.split - 1) / p.split;
  const int k0 = s0 + split * p.split;
  const int k1 = min(k0 + p.split, r.pos + 1);
  r.kw0 = k0 + w * (NCH * CH);  // p.split == 4 * NCH * CH
  r.kw1 = min(r.kw0 + NCH * CH, k1);
  r.active = split < r.nsplit;
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
  const bool has_new = kw0 < kw1 && kw1 == pos + 1;
  const int kwc = has_new ? pos : kw1;  // keys read from the cache: [kw0, kwc)
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;
  T* sc_out = (T*)p.scores;

  float m[REP], l[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
  }

  if (kw0 < kw1) {
    const int kc = max(kwc - 1, kw0);  // clamp target inside the cached range
    auto load = [&](int c0, Chunk<A>* kk) {
#pragma unroll
      for (int i = 0; i < CH / 4; ++i)
        kk[i] = load_chunk<A>(p.kc, (kvbase + min(c0 + 4 * i + grp, kc)) * HD + dc * 8);
    };
    auto score = [&](int c0, const Chunk<A>* kk, const float (*qf)[8]) {
      float sc[REP][CH / 4];
#pragma unroll
      for (int i = 0; i < CH / 4; ++i) {
        float kf[8];
        chunk_f32<A>(kk[i], kf);
        const bool ok = c0 + 4 * i + grp < kwc;
#pragma unroll
        for (int r = 0; r < REP; ++r) {
          float d = 0.f;
#pragma unroll
          for (int t = 0; t < 8; ++t) d += qf[r][t] * kf[t];
          d = row16_sum(d);
          sc[r][i] = ok ? rd<A>(rd<A>(d) * p.scale) : -INFINITY;
        }
      }
      // Lane (grp, dc) of the row stores the score of key c0 + 4*(dc&7) + grp
      // for heads (dc>>3) + 2u: per head, the wave writes 32 consecutive keys.
      {
        const int i = dc & 7, key = c0 + 4 * i + grp;
#pragma unroll
        for (int u = 0; u < (REP + 1) / 2; ++u) {
          const int r = REP == 1 ? 0 : (dc >> 3) + 2 * u;
          float v = sc[0][0];
#pragma unroll
          for (int rr = 0; rr < REP; ++rr)
#pragma unroll
            for (int ii = 0; ii < CH / 4; ++ii)
              if (rr == r && ii == i) v = sc[rr][ii];
          if (key < kwc && (REP > 1 || dc < 8))
            sc_out[score_index(p, b, g * REP + r, key)] = st_act<A>(v);
        }
      }
#pragma unroll
      for (int r = 0; r < REP; ++r) {
        float cm = -INFINITY;
#pragma unroll
        for (int i = 0; i < CH / 4; ++i) cm = fmaxf(cm, sc[r][i]);
        const float mn = fmaxf(m[r], cm);
        if (mn == -INFINITY) continue;
        float e = (m[r] == -INFINITY) ? 0.f : l[r] * __expf(m[r] - mn);
#pragma unroll
        for (int i = 0; i < CH / 4; ++i)
          e += (sc[r][i] == -INFINITY) ? 0.f : __expf(sc[r][i] - mn);
        m[r] = mn;
        l[r] = e;
      }
    };
    // Two register buffers in ping-pong over a compile-time number of chunks,
    // fully unrolled: chunk c+1's loads are issued (back to back, pinned by
    // sched_barrier) before chunk c is scored, and the compiler waits for the
    // older chunk only.  Loads past the wave's last key clamp to it and hit
    // the cache.
    Chunk<A> kbuf[2][CH / 4];
    load(kw0, kbuf[0]);
    __builtin_amdgcn_sched_barrier(0);
    // the REP query heads: q_norm + RoPE of the raw projection (qwen3.rs:220, 224)
    float qf[REP][8];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      load8<A>(p.qkv, (size_t)b * p.ldqkv + (g * REP + r) * HD + dc * 8, qf[r]);
      norm_rope8<A>(qf[r], p.qn_w, p.cos, p.sin, pos, dc, p.eps);
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c + 1 < NCH) load(kw0 + (c + 1) * CH, kbuf[(c + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      score(kw0 + c * CH, kbuf[c & 1], qf);
    }
    if (has_new) {
      // The new token (qwen3.rs:221, 225-227): k_norm + RoPE, cache append,
      // and its score, added by lane-row 0 of this wave.
      const int qd = p.nkv * REP * HD;
      const size_t row = (size_t)b * p.ldqkv;
      float kf[8], vf[8];
      load8<A>(p.qkv, row + qd + g * HD + dc * 8, kf);
      load8<A>(p.qkv, row + qd + p.nkv * HD + g * HD + dc * 8, vf);
      norm_rope8<A>(kf, p.kn_w, p.cos, p.sin, pos, dc, p.eps);
      if (grp == 0) {
        T* kd = (T*)p.kc + (kvbase + pos) * HD + dc * 8;
        T* vd = (T*)p.vc + (kvbase + pos) * HD + dc * 8;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          kd[t] = st_act<A>(kf[t]);
          vd[t] = st_act<A>(vf[t]);
        }
      }
#pragma unroll
      for (int r = 0; r < REP; ++r) {
        float d = 0.f;
#pragma unroll
        for (int t = 0; t < 8; ++t) d += qf[r][t] * kf[t];
        d = row16_sum(d);
        if (grp == 0) {
          const float sn = rd<A>(rd<A>(d) * p.scale);
          if (dc == 0) sc_out[score_index(p, b, g * REP + r, pos)] = st_act<A>(sn);
          const float mn = fmaxf(m[r], sn);
          l[r] = ((m[r] == -INFINITY) ? 0.f : l[r] * __expf(m[r] - mn)) + __expf(sn - mn);
          m[r] = mn;
        }
      }
    }
  }

  // Merge the 16 lane-rows (4 per wave x 4 waves) of this work-group.
  __shared__ float s_ml[16][REP][2];
  const int gi = w * 4 + grp;
  if (dc == 0) {
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      s_ml[gi][r][0] = m[r];
      s_ml[gi][r][1] = l[r];
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
  const int kw0 = wr.kw0, kw1 = wr.kw1;
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;
  const size_t unit = (size_t)b * p.nkv + g;

  // Global max and sum of exp of each query head, from the split partials in
  // split order (identical in every work-group of this (row, KV head)).
  float M[REP], S[REP];
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    const float* ml = p.ml + (unit * p.max_splits) * REP * 2 + r * 2;
    float mx = -INFINITY;
    for (int j = lane; j < wr.nsplit; j += 64) mx = fmaxf(mx, ml[(size_t)j * REP * 2]);
    mx = wave_max(mx);
    float sm = 0.f;
    for (int j = lane; j < wr.nsplit; j += 64) {
      const float mj = ml[(size_t)j * REP * 2];
      if (mj != -INFINITY) sm += ml[(size_t)j * REP * 2 + 1] * __expf(mj - mx);
    }
    M[r] = mx;
    S[r] = wave_sum(sm);
  }

  float acc[REP][8];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[r][t] = 0.f;

  if (kw0 < kw1) {
    const T* scores = (const T*)p.scores;
    const int kl = kw1 - 1;
    // The scores of a chunk: lane L holds key c0 + (L & 31) of heads
    // (L >> 5) + 2u (REP >= 2) or of head 0 (REP == 1).
    constexpr int NS = (REP + 1) / 2;
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
        const float s = ld_act<A>(ss[u]);
        pr[u] = ok ? rd<A>(__fdiv_rn(expf(s - Mr), Sr)) : 0.f;
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
    Chunk<A> vbuf[2][CH / 4];
    T sbuf[2][NS];
    load(kw0, vbuf[0], sbuf[0]);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c + 1 < NCH) load(kw0 + (c + 1) * CH, vbuf[(c + 1) & 1], sbuf[(c + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      accumulate(kw0 + c * CH, vbuf[c & 1], sbuf[c & 1]);
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
  const int pos = p.state[0];
  const int nsplit = (pos + 1 - p.start[b] + p.split - 1) / p.split;
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

hipError_t launch_attn_decode(int act, const AttnDecodeArgs& a, hipStream_t s) {
  if (a.batch <= 0) return hipSuccess;
  switch (act) {
    case ACT_F32: return launch_rep<ACT_F32>(a, s);
    case ACT_F16: return launch_rep<ACT_F16>(a, s);
    case ACT_BF16: return launch_rep<ACT_BF16>(a, s);
  }
  return hipErrorInvalidValue;
}
