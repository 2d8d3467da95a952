// GQA decode attention over the left-padded batched KV cache.
//
// Reference: Attention::forward (qwen3.rs:227-257) with the decode mask of
// build_mask (qwen3.rs:523-562): the new query of row b at position `pos`
// attends to keys [pad_b, pos]; query head h reads KV head h / repeat
// (qwen3.rs:237-241).  Scores are rd(rd(q.k) * rd(1/sqrt(hd))) as in
// qwen3.rs:243; softmax and the value sum run in f32 and the context is
// stored in the activation dtype.
//
// Work decomposition: one work-group per (split of 256 keys, KV head, row).
// The REP query heads of a KV head share every K/V byte read.  Each wave owns
// 64 keys; a 16-lane row of the wave holds one key (8 dims per lane, one
// 16-byte load), so every wave load is 1 KiB contiguous.  All K and V loads
// of a wave are issued before any arithmetic.  The last work-group of a
// (row, KV head) to finish merges the splits' (max, sum, acc) partials in
// split order and writes the context; counters reset themselves.
#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

constexpr int SPLIT = 256;       // keys per work-group
constexpr int KPW = 64;          // keys per wave
constexpr int HD = 128;

template <int A>
__device__ __forceinline__ void load_row8(const void* base, size_t elem, bool ok, float* out) {
  if constexpr (A == ACT_F32) {
    const f32x4* p = (const f32x4*)((const float*)base + elem);
    f32x4 a = ok ? p[0] : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 b = ok ? p[1] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = a[i];
      out[4 + i] = b[i];
    }
  } else {
    const u32x4 v = ok ? *(const u32x4*)((const uint16_t*)base + elem) : u32x4{0, 0, 0, 0};
    unpack8<A>(v, out);
  }
}

// Raw 16-byte (or 32-byte for f32) chunk of one key row, kept packed until use.
template <int A> struct Chunk { u32x4 v; };
template <> struct Chunk<ACT_F32> { u32x4 v0, v1; };

template <int A>
__device__ __forceinline__ Chunk<A> load_chunk(const void* base, size_t elem, bool ok) {
  Chunk<A> c;
  if constexpr (A == ACT_F32) {
    const u32x4* p = (const u32x4*)((const float*)base + elem);
    c.v0 = ok ? __builtin_nontemporal_load(p) : u32x4{0, 0, 0, 0};
    c.v1 = ok ? __builtin_nontemporal_load(p + 1) : u32x4{0, 0, 0, 0};
  } else {
    c.v = ok ? __builtin_nontemporal_load((const u32x4*)((const uint16_t*)base + elem))
             : u32x4{0, 0, 0, 0};
  }
  return c;
}

template <int A>
__device__ __forceinline__ void chunk_f32(const Chunk<A>& c, float* o) {
  if constexpr (A == ACT_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[i] = __builtin_bit_cast(float, c.v0[i]);
      o[4 + i] = __builtin_bit_cast(float, c.v1[i]);
    }
  } else {
    unpack8<A>(c.v, o);
  }
}

template <int A, int REP>
__global__ void __launch_bounds__(256) attn_decode_kernel(AttnDecodeArgs p) {
  typedef typename ActT<A>::T T;
  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  if (p.done && p.done[b]) return;
  const int pos = p.state[0];
  const int s0 = p.start[b];
  const int end = pos + 1;
  const int nsplit = (end - s0 + SPLIT - 1) / SPLIT;
  if (split >= nsplit) return;
  const int k0 = s0 + split * SPLIT;
  const int k1 = min(k0 + SPLIT, end);

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int grp = lane >> 4, dc = lane & 15;
  const int kw0 = k0 + w * KPW;
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;

  // Issue all K and V loads of this wave.
  Chunk<A> kr[KPW / 4], vr[KPW / 4];
#pragma unroll
  for (int i = 0; i < KPW / 4; ++i) {
    const int key = kw0 + 4 * i + grp;
    const bool ok = key < k1;
    const size_t e = (kvbase + key) * HD + dc * 8;
    kr[i] = load_chunk<A>(p.kc, e, ok);
  }
#pragma unroll
  for (int i = 0; i < KPW / 4; ++i) {
    const int key = kw0 + 4 * i + grp;
    const bool ok = key < k1;
    const size_t e = (kvbase + key) * HD + dc * 8;
    vr[i] = load_chunk<A>(p.vc, e, ok);
  }

  float qf[REP][8];
#pragma unroll
  for (int r = 0; r < REP; ++r)
    load_row8<A>(p.q, ((size_t)b * p.nkv * REP + g * REP + r) * HD + dc * 8, true, qf[r]);

  // Scores for this lane-row's 16 keys.
  float sc[REP][KPW / 4];
#pragma unroll
  for (int i = 0; i < KPW / 4; ++i) {
    float kf[8];
    chunk_f32<A>(kr[i], kf);
    const bool ok = kw0 + 4 * i + grp < k1;
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      float d = 0.f;
#pragma unroll
      for (int t = 0; t < 8; ++t) d += qf[r][t] * kf[t];
      d = row16_sum(d);
      sc[r][i] = ok ? rd<A>(rd<A>(d) * p.scale) : -INFINITY;
    }
  }
  float m[REP], l[REP], acc[REP][8];
#pragma unroll
  for (int r = 0; r < REP; ++r) {
    m[r] = -INFINITY;
#pragma unroll
    for (int i = 0; i < KPW / 4; ++i) m[r] = fmaxf(m[r], sc[r][i]);
    l[r] = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[r][t] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < KPW / 4; ++i) {
    float vf[8];
    chunk_f32<A>(vr[i], vf);
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      const float e = (sc[r][i] == -INFINITY) ? 0.f : __expf(sc[r][i] - m[r]);
      l[r] += e;
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[r][t] += e * vf[t];
    }
  }

  // Merge the 16 lane-rows (4 per wave x 4 waves) of this work-group.
  __shared__ float s_acc[16][REP][HD];
  __shared__ float s_ml[16][REP][2];
  __shared__ int s_last;
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
    if (nsplit == 1) {
      ((T*)p.out)[(size_t)b * p.nkv * REP * HD + (g * REP + r) * HD + d] = st_act<A>(O / L);
    } else {
      float* dst = p.part + ((pidx + split) * REP + r) * PSTRIDE;
      dst[d] = O;
      if (d == 0) {
        dst[HD] = M;
        dst[HD + 1] = L;
      }
    }
  }
  if (nsplit == 1) return;

  // Last-arriving work-group of this (row, KV head) merges all splits.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = atomicAdd(&p.counters[(size_t)b * p.nkv + g], 1u);
    s_last = (prev == (uint32_t)(nsplit - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int t = threadIdx.x; t < REP * HD; t += blockDim.x) {
    const int r = t / HD, d = t % HD;
    float M = -INFINITY;
    for (int j = 0; j < nsplit; ++j)
      M = fmaxf(M, __builtin_nontemporal_load(p.part + ((pidx + j) * REP + r) * PSTRIDE + HD));
    float L = 0.f, O = 0.f;
    for (int j = 0; j < nsplit; ++j) {
      const float* src = p.part + ((pidx + j) * REP + r) * PSTRIDE;
      const float f = __expf(__builtin_nontemporal_load(src + HD) - M);
      L += __builtin_nontemporal_load(src + HD + 1) * f;
      O += __builtin_nontemporal_load(src + d) * f;
    }
    ((T*)p.out)[(size_t)b * p.nkv * REP * HD + (g * REP + r) * HD + d] = st_act<A>(O / L);
  }
  if (threadIdx.x == 0) p.counters[(size_t)b * p.nkv + g] = 0u;
}

template <int A>
hipError_t launch_rep(int rep, const AttnDecodeArgs& a, hipStream_t s) {
  const dim3 grid(a.max_splits, a.nkv, a.batch);
  switch (rep) {
    case 1: hipLaunchKernelGGL((attn_decode_kernel<A, 1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attn_decode_kernel<A, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((attn_decode_kernel<A, 4>), grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

int attn_decode_split() { return SPLIT; }

hipError_t launch_attn_decode(int act, int rep, const AttnDecodeArgs& a, hipStream_t s) {
  if (a.batch <= 0) return hipSuccess;
  switch (act) {
    case ACT_F32: return launch_rep<ACT_F32>(rep, a, s);
    case ACT_F16: return launch_rep<ACT_F16>(rep, a, s);
    case ACT_BF16: return launch_rep<ACT_BF16>(rep, a, s);
  }
  return hipErrorInvalidValue;
}
