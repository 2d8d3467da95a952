// GQA decode attention over the left-padded batched KV cache, with the
// per-head q/k RMSNorm, RoPE and the KV-cache append of the new token fused in.
//
// Reference: Attention::forward (qwen3.rs:213-257) with the decode mask of
// build_mask (qwen3.rs:523-562): the new query of row b at position `pos`
// attends to keys [pad_b, pos]; query head h reads KV head h / repeat
// (qwen3.rs:237-241).  q and k are RMS-normalised over head_dim before RoPE
// (qwen3.rs:218-225); the new K/V land at ((b*nkv + h)*cap + pos)*hd
// (KvCache::append, qwen3.rs:86-101).  Scores are rd(rd(q.k) * rd(1/sqrt(hd)))
// as in qwen3.rs:243; softmax and the value sum run in f32 and the context is
// stored in the activation dtype.
//
// Two kernels per layer:
//  attn_decode_kernel: one work-group per (split of the keys [pad_b, pos],
//    KV head, row).  Each wave normalises and rotates its REP query heads
//    from the raw qkv projection, then streams its keys in chunks of 32: a
//    16-lane row of the wave holds one key (8 dims per lane, one 16-byte
//    load), so each wave load is 1 KiB contiguous, and chunk c+1's K/V loads
//    are in flight while chunk c is scored (online softmax per lane-row).
//    Key indices are clamped into range, so the loads carry no branches;
//    out-of-range keys are masked.  The wave whose range ends at the new
//    token normalises and rotates its k, appends k and v to the cache and
//    adds the new key from registers (no other work-group reads position
//    pos).  Each split writes (max, sum, acc) partials.
//  attn_combine_kernel: one work-group per (KV head, row) merges the
//    partials in split order.
// (A single kernel whose last work-group merges would need an agent-scope
// fence per work-group -- an L2 write-back plus invalidate on this multi-XCD
// part -- which costs far more than the extra launch.)
#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

constexpr int HD = 128;
#ifndef FMD_ATTN_CH
#define FMD_ATTN_CH 32
#endif
#ifndef FMD_ATTN_TARGET_WGS
#define FMD_ATTN_TARGET_WGS 1024
#endif
constexpr int CH = FMD_ATTN_CH;  // keys per wave chunk

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

template <int A, int REP, int NCH>
__global__ void __launch_bounds__(256) attn_decode_kernel(AttnDecodeArgs p) {
  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  if (p.done && p.done[b]) return;
  const int pos = p.state[0];
  const int s0 = p.start[b];
  const int nsplit = (pos + 1 - s0 + p.split - 1) / p.split;  // keys [s0, pos]
  if (split >= nsplit) return;
  const int k0 = s0 + split * p.split;
  const int k1 = min(k0 + p.split, pos + 1);

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int grp = lane >> 4, dc = lane & 15;
  constexpr int per_wave = NCH * CH;  // p.split == 4 * per_wave
  const int kw0 = k0 + w * per_wave;
  const int kw1 = min(kw0 + per_wave, k1);     // this wave's keys [kw0, kw1)
  const bool has_new = kw0 < kw1 && kw1 == pos + 1;
  const int kwc = has_new ? pos : kw1;         // keys read from the cache: [kw0, kwc)
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;

  float m[REP], l[REP], acc[REP][8];
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[r][t] = 0.f;
  }

  if (kw0 < kw1) {
    const int kc = max(kwc - 1, kw0);  // clamp target inside the cached range
    auto load = [&](int c0, Chunk<A>* kk, Chunk<A>* vv) {
#pragma unroll
      for (int i = 0; i < CH / 4; ++i) {
        const size_t e = (kvbase + min(c0 + 4 * i + grp, kc)) * HD + dc * 8;
        kk[i] = load_chunk<A>(p.kc, e);
        vv[i] = load_chunk<A>(p.vc, e);
      }
    };
    auto score = [&](int c0, const Chunk<A>* kk, const Chunk<A>* vv, const float (*qf)[8]) {
      float sc[REP][CH / 4];
      float cm[REP];
#pragma unroll
      for (int r = 0; r < REP; ++r) cm[r] = -INFINITY;
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
          cm[r] = fmaxf(cm[r], sc[r][i]);
        }
      }
#pragma unroll
      for (int r = 0; r < REP; ++r) {
        const float mn = fmaxf(m[r], cm[r]);
        const float corr = (m[r] == -INFINITY) ? 0.f : __expf(m[r] - mn);
        m[r] = mn;
        l[r] *= corr;
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[r][t] *= corr;
      }
#pragma unroll
      for (int i = 0; i < CH / 4; ++i) {
        float vf[8];
        chunk_f32<A>(vv[i], vf);
#pragma unroll
        for (int r = 0; r < REP; ++r) {
          const float e = (sc[r][i] == -INFINITY) ? 0.f : __expf(sc[r][i] - m[r]);
          l[r] += e;
#pragma unroll
          for (int t = 0; t < 8; ++t) acc[r][t] += e * vf[t];
        }
      }
    };
    // Two register buffers in ping-pong over a compile-time number of chunks,
    // fully unrolled: chunk c+1's 16 loads are issued (back to back, pinned by
    // sched_barrier) before chunk c is scored, and the compiler waits for the
    // older chunk only.  Loads past the wave's last key clamp to it and hit
    // the cache.
    Chunk<A> kbuf[2][CH / 4], vbuf[2][CH / 4];
    load(kw0, kbuf[0], vbuf[0]);
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
      if (c + 1 < NCH) load(kw0 + (c + 1) * CH, kbuf[(c + 1) & 1], vbuf[(c + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      score(kw0 + c * CH, kbuf[c & 1], vbuf[c & 1], qf);
    }
    if (has_new) {
      // The new token (qwen3.rs:221, 225-227): k_norm + RoPE, cache append,
      // and its contribution, added by lane-row 0 of this wave.
      typedef typename ActT<A>::T T;
      const int qd = p.nkv * REP * HD;
      const size_t row = (size_t)b * p.ldqkv;
      float kf[8], vf[8];
      load8<A>(p.qkv, row + qd + g * HD + dc * 8, kf);
      load8<A>(p.qkv, row + qd + p.nkv * HD + g * HD + dc * 8, vf);
      norm_rope8<A>(kf, p.kn_w, p.cos, p.sin, pos, dc, p.eps);
      if (grp == 0) {
        T* kd = (T*)p.kc + (((size_t)b * p.nkv + g) * p.cap + pos) * HD + dc * 8;
        T* vd = (T*)p.vc + (((size_t)b * p.nkv + g) * p.cap + pos) * HD + dc * 8;
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
          const float mn = fmaxf(m[r], sn);
          const float corr = (m[r] == -INFINITY) ? 0.f : __expf(m[r] - mn);
          const float en = __expf(sn - mn);
          m[r] = mn;
          l[r] = l[r] * corr + en;
#pragma unroll
          for (int t = 0; t < 8; ++t) acc[r][t] = acc[r][t] * corr + en * vf[t];
        }
      }
    }
  }

  // Merge the 16 lane-rows (4 per wave x 4 waves) of this work-group.
  __shared__ float s_acc[16][REP][HD];
  __shared__ float s_ml[16][REP][2];
  const int gi = w * 4 + grp;
#pragma unroll
  for (int r = 0; r < REP; ++r) {
#pragma unroll
    for (int t = 0; t < 8; ++t) s_acc[gi][r][dc * 8 + t] = acc[r][t];
    if (dc == 0) {
      s_ml[gi][r][0] = m[r];
      s_ml[gi][r][1] = l[r];
    }
  }
  __syncthreads();
  const size_t pidx = ((size_t)b * p.nkv + g) * p.max_splits;
  constexpr int PSTRIDE = HD + 2;
  for (int t = threadIdx.x; t < REP * HD; t += blockDim.x) {
    const int r = t / HD, d = t % HD;
    float M = -INFINITY;
    for (int i = 0; i < 16; ++i) M = fmaxf(M, s_ml[i][r][0]);
    float L = 0.f, O = 0.f;
    for (int i = 0; i < 16; ++i) {
      const float mi = s_ml[i][r][0];
      if (mi == -INFINITY) continue;
      const float f = __expf(mi - M);
      L += s_ml[i][r][1] * f;
      O += s_acc[i][r][d] * f;
    }
    float* dst = p.part + ((pidx + split) * REP + r) * PSTRIDE;
    dst[d] = O;
    if (d == 0) {
      dst[HD] = M;
      dst[HD + 1] = L;
    }
  }
}

// Merge the splits of one (KV head g, row b) in split order: global max,
// rescaled sums and context.  All partial loads are issued up front.
template <int A, int REP>
__global__ void __launch_bounds__(REP * HD) attn_combine_kernel(AttnDecodeArgs p) {
  typedef typename ActT<A>::T T;
  constexpr int PSTRIDE = HD + 2;
  constexpr int MAXU = 16;  // splits merged per pass
  const int g = blockIdx.x, b = blockIdx.y;
  if (p.done && p.done[b]) return;
  const int pos = p.state[0];
  const int nsplit = (pos + 1 - p.start[b] + p.split - 1) / p.split;
  const size_t pidx = ((size_t)b * p.nkv + g) * p.max_splits;
  const int r = threadIdx.x / HD, d = threadIdx.x % HD;
  float M = -INFINITY, L = 0.f, O = 0.f;
  for (int j0 = 0; j0 < nsplit; j0 += MAXU) {
    float mj[MAXU], lj[MAXU], oj[MAXU];
#pragma unroll
    for (int u = 0; u < MAXU; ++u) {
      const int j = min(j0 + u, nsplit - 1);
      const float* src = p.part + ((pidx + j) * REP + r) * PSTRIDE;
      mj[u] = src[HD];
      lj[u] = src[HD + 1];
      oj[u] = src[d];
    }
    float Mn = M;
#pragma unroll
    for (int u = 0; u < MAXU; ++u)
      if (j0 + u < nsplit) Mn = fmaxf(Mn, mj[u]);
    const float corr = (M == -INFINITY) ? 0.f : __expf(M - Mn);
    L *= corr;
    O *= corr;
#pragma unroll
    for (int u = 0; u < MAXU; ++u) {
      if (j0 + u >= nsplit || mj[u] == -INFINITY) continue;
      const float f = __expf(mj[u] - Mn);
      L += lj[u] * f;
      O += oj[u] * f;
    }
    M = Mn;
  }
  ((T*)p.out)[(size_t)b * p.nkv * REP * HD + (g * REP + r) * HD + d] = st_act<A>(O / L);
}

template <int A, int REP>
hipError_t launch_pair(const AttnDecodeArgs& a, hipStream_t s) {
  if (a.max_splits > 128 || (a.split != 4 * CH && a.split != 8 * CH && a.split != 16 * CH))
    return hipErrorInvalidValue;
  const dim3 grid(a.max_splits, a.nkv, a.batch);
  if (a.split == 4 * CH)
    hipLaunchKernelGGL((attn_decode_kernel<A, REP, 1>), grid, dim3(256), 0, s, a);
  else if (a.split == 8 * CH)
    hipLaunchKernelGGL((attn_decode_kernel<A, REP, 2>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((attn_decode_kernel<A, REP, 4>), grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_combine_kernel<A, REP>), dim3(a.nkv, a.batch), dim3(REP * HD), 0, s, a);
  return hipGetLastError();
}

template <int A>
hipError_t launch_rep(int rep, const AttnDecodeArgs& a, hipStream_t s) {
  switch (rep) {
    case 1: return launch_pair<A, 1>(a, s);
    case 2: return launch_pair<A, 2>(a, s);
    case 4: return launch_pair<A, 4>(a, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Keys per split (4 waves x 1, 2 or 4 chunks of CH keys) for a cache of
// `cap` positions and `units` (row, KV head) pairs: the longest split that
// still gives at least FMD_ATTN_TARGET_WGS work-groups at full capacity.
int attn_decode_split(int cap, int units) {
  int split = 16 * CH;
  while (split > 4 * CH && (long)units * ((cap + split - 1) / split) < FMD_ATTN_TARGET_WGS)
    split /= 2;
  while ((cap + split - 1) / split > 128) split *= 2;  // beyond 128 splits: unsupported
  return split;
}

hipError_t launch_attn_decode(int act, int rep, const AttnDecodeArgs& a, hipStream_t s) {
  if (a.batch <= 0) return hipSuccess;
  switch (act) {
    case ACT_F32: return launch_rep<ACT_F32>(rep, a, s);
    case ACT_F16: return launch_rep<ACT_F16>(rep, a, s);
    case ACT_BF16: return launch_rep<ACT_BF16>(rep, a, s);
  }
  return hipErrorInvalidValue;
}
