// Causal GQA attention for chunked prefill.
//
// Reference: Attention::forward (qwen3.rs:227-257) for a block of query rows
// with the additive mask of build_mask (qwen3.rs:523-562): query row at
// absolute position q of sequence b sees keys [pad_b, q].  Left-pad rows are
// not computed at all: with zero embeddings and no biases every pad row, and
// its K/V, is exactly zero in the reference, and a zero-initialised cache
// already holds that.  Rows arrive packed (real tokens only) with explicit
// positions.
//
// The softmax probabilities are rounded to the activation dtype after
// normalisation, p = rd(exp(s - M) / S) with the row's global max M and sum S
// (softmax_last_dim returns a tensor of the activation dtype, qwen3.rs:248),
// so each query row is visited twice: pass 1 finds M and S, pass 2 recomputes
// the scores and accumulates p V.
//
// MFMA path (16-bit): one work-group per (tile of 64/REP query positions of one
// sequence, KV head); wave w owns query head g*REP + w%REP and 16 positions.
// Per 32-key block: S^T = K Q^T (keys are the MFMA's M side, so the f32 result
// already sits in the B-operand layout of P^T), then O^T += V^T P^T with V
// staged transposed in LDS.
#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

constexpr int HD = 128;
constexpr int KB = 32;          // keys per block
constexpr int LDK = HD + 8;     // padded K row pitch (elements)
constexpr int LDV = KB + 8;     // padded V^T row pitch (elements)

template <int A>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (A == ACT_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <int A, int REP>
__global__ void __launch_bounds__(256) attn_prefill_kernel(AttnPrefillArgs p) {
  typedef typename ActT<A>::T T;
  __shared__ uint16_t sK[KB * LDK];
  __shared__ uint16_t sVt[HD * LDV];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int t = blockIdx.x, g = blockIdx.y;
  const int b = p.tile_b[t], row0 = p.tile_row0[t], pos0 = p.tile_pos0[t], n = p.tile_n[t];
  const int nh = p.nkv * REP;
  const int r = w % REP, sub = w / REP;
  const int h = g * REP + r;
  const int qr = lane & 15, kg = lane >> 4;
  const int myrow = 16 * sub + qr;           // row within the tile
  const bool row_ok = myrow < n;
  const int qpos = pos0 + myrow;
  const int kstart = p.start[b];
  const int kend = pos0 + n;                 // exclusive: last query position + 1
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;

  // Q^T fragments (B operand): row qr, dims 32ks + 8kg + [0,8).
  u32x4 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qf[ks] = row_ok ? *(const u32x4*)((const uint16_t*)p.q +
                                      ((size_t)(row0 + myrow) * nh + h) * HD + ks * 32 + kg * 8)
                    : u32x4{0, 0, 0, 0};

  const int nblk = (kend - kstart + KB - 1) / KB;
  // K block -> sK[key][dim] (and, when `with_v`, V block -> sVt[dim][key]);
  // 512 16-byte pieces each.
  auto stage = [&](int k0, bool with_v) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + 256 * i;
      const int key = idx >> 4, c = idx & 15;
      const bool ok = k0 + key < kend;
      const size_t e = (kvbase + k0 + key) * HD + c * 8;
      const u32x4 kv = ok ? *(const u32x4*)((const uint16_t*)p.kc + e) : u32x4{0, 0, 0, 0};
      *(u32x4*)&sK[key * LDK + c * 8] = kv;
      if (with_v) {
        const u32x4 vv = ok ? *(const u32x4*)((const uint16_t*)p.vc + e) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sVt[(c * 8 + 2 * j) * LDV + key] = (uint16_t)(vv[j] & 0xffffu);
          sVt[(c * 8 + 2 * j + 1) * LDV + key] = (uint16_t)(vv[j] >> 16);
        }
      }
    }
  };
  // Scaled, masked scores S^T for keys k0 + 16mt + 4kg + i of query row qr:
  // rd(rd(q.k) * rd(scale)) as qwen3.rs:243, -inf outside [pad_b, qpos].
  auto scores = [&](int k0, f32x4* s) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      s[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4 ka = *(const u32x4*)&sK[(16 * mt + qr) * LDK + ks * 32 + kg * 8];
        s[mt] = mfma16<A>(ka, qf[ks], s[mt]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = k0 + 16 * mt + 4 * kg + i;
        const float v = rd<A>(rd<A>(s[mt][i]) * p.scale);
        s[mt][i] = (!row_ok || key > qpos || key >= kend) ? -INFINITY : v;
      }
    }
  };

  // Pass 1: max and sum of exp of each query row over all its keys (every
  // lane covers 8 keys per block; the four lanes of a row merge at the end).
  float m = -INFINITY, l = 0.f;
  for (int blk = 0; blk < nblk; ++blk) {
    const int k0 = kstart + blk * KB;
    __syncthreads();
    stage(k0, false);
    __syncthreads();
    f32x4 s[2];
    scores(k0, s);
    float bm = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) bm = fmaxf(bm, s[mt][i]);
    const float mn = fmaxf(m, bm);
    if (mn == -INFINITY) continue;
    float e = (m == -INFINITY) ? 0.f : l * __expf(m - mn);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) e += (s[mt][i] == -INFINITY) ? 0.f : __expf(s[mt][i] - mn);
    m = mn;
    l = e;
  }
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const float mo = __shfl_xor(m, off), lo = __shfl_xor(l, off);
    const float mn = fmaxf(m, mo);
    if (mn != -INFINITY)
      l = ((m == -INFINITY) ? 0.f : l * __expf(m - mn)) + ((mo == -INFINITY) ? 0.f : lo * __expf(mo - mn));
    m = mn;
  }

  // Pass 2: p = rd(exp(s - M) / S) in the activation dtype (softmax_last_dim,
  // qwen3.rs:248), then O^T += V^T P^T and the context rd(O) (qwen3.rs:252).
  f32x4 o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int blk = 0; blk < nblk; ++blk) {
    const int k0 = kstart + blk * KB;
    __syncthreads();
    stage(k0, true);
    __syncthreads();
    f32x4 s[2];
    scores(k0, s);
    uint32_t pk[4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const float p0 = (s[mt][i] == -INFINITY) ? 0.f : __fdiv_rn(expf(s[mt][i] - m), l);
        const float p1 = (s[mt][i + 1] == -INFINITY) ? 0.f : __fdiv_rn(expf(s[mt][i + 1] - m), l);
        pk[mt * 2 + i / 2] = (uint32_t)st_act<A>(p0) | ((uint32_t)st_act<A>(p1) << 16);
      }
    const u32x4 pb = {pk[0], pk[1], pk[2], pk[3]};
    // k-slot s of lane group kg holds key 4kg+s (s<4) or 16+4kg+(s-4),
    // matching where S^T put those keys.
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint16_t* vrow = &sVt[(16 * dt + qr) * LDV];
      const uint2 lo = *(const uint2*)(vrow + 4 * kg);
      const uint2 hi = *(const uint2*)(vrow + 16 + 4 * kg);
      const u32x4 va = {lo.x, lo.y, hi.x, hi.y};
      o[dt] = mfma16<A>(va, pb, o[dt]);
    }
  }
  if (!row_ok) return;
  T* out = (T*)p.out + ((size_t)(row0 + myrow) * nh + h) * HD;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) out[16 * dt + 4 * kg + i] = st_act<A>(o[dt][i]);
}

// f32 path: one wave per (packed row, query head), keys in lane-rows of 16.
__global__ void __launch_bounds__(64) attn_prefill_f32_kernel(AttnPrefillArgs p, int rep,
                                                              int rows_per_tile) {
  const int lane = threadIdx.x;
  const int t = blockIdx.x / rows_per_tile, rr = blockIdx.x % rows_per_tile;
  const int h = blockIdx.y;
  const int n = p.tile_n[t];
  if (rr >= n) return;
  const int b = p.tile_b[t], row = p.tile_row0[t] + rr, qpos = p.tile_pos0[t] + rr;
  const int nh = p.nkv * rep, g = h / rep;
  const int grp = lane >> 4, dc = lane & 15;
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;
  const float* q = (const float*)p.q + ((size_t)row * nh + h) * HD + dc * 8;
  float qf[8];
  for (int i = 0; i < 8; ++i) qf[i] = q[i];
  float m = -INFINITY, l = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int k0 = p.start[b]; k0 <= qpos; k0 += 4) {
    const int key = k0 + grp;
    const bool ok = key <= qpos;
    const float* kr = (const float*)p.kc + (kvbase + (ok ? key : k0)) * HD + dc * 8;
    const float* vr = (const float*)p.vc + (kvbase + (ok ? key : k0)) * HD + dc * 8;
    float d = 0.f;
    for (int i = 0; i < 8; ++i) d += qf[i] * kr[i];
    d = row16_sum(d) * p.scale;
    if (!ok) continue;
    const float mn = fmaxf(m, d);
    const float corr = (m == -INFINITY) ? 0.f : __expf(m - mn);
    const float e = __expf(d - mn);
    l = l * corr + e;
    for (int i = 0; i < 8; ++i) acc[i] = acc[i] * corr + e * vr[i];
    m = mn;
  }
  // merge the four lane-rows
  for (int off = 16; off <= 32; off <<= 1) {
    const float mo = __shfl_xor(m, off), lo = __shfl_xor(l, off);
    const float mn = fmaxf(m, mo);
    const float ca = (m == -INFINITY) ? 0.f : __expf(m - mn);
    const float cb = (mo == -INFINITY) ? 0.f : __expf(mo - mn);
    for (int i = 0; i < 8; ++i) {
      const float ao = __shfl_xor(acc[i], off);
      acc[i] = acc[i] * ca + ao * cb;
    }
    l = l * ca + lo * cb;
    m = mn;
  }
  if (grp == 0) {
    float* out = (float*)p.out + ((size_t)row * nh + h) * HD + dc * 8;
    for (int i = 0; i < 8; ++i) out[i] = acc[i] / l;
  }
}

template <int A>
hipError_t launch_rep(int rep, const AttnPrefillArgs& a, hipStream_t s) {
  const dim3 grid(a.ntiles, a.nkv);
  switch (rep) {
    case 1: hipLaunchKernelGGL((attn_prefill_kernel<A, 1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attn_prefill_kernel<A, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((attn_prefill_kernel<A, 4>), grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

// Query positions per prefill attention tile for a given GQA repeat.
int attn_prefill_tile_rows(int rep) { return 64 / rep; }

hipError_t launch_attn_prefill(int act, int rep, const AttnPrefillArgs& a, hipStream_t s) {
  if (a.ntiles <= 0) return hipSuccess;
  if (rep != 1 && rep != 2 && rep != 4) return hipErrorInvalidValue;
  switch (act) {
    case ACT_F32: {
      const int rpt = 64 / rep;
      hipLaunchKernelGGL(attn_prefill_f32_kernel, dim3(a.ntiles * rpt, a.nkv * rep), dim3(64), 0,
                         s, a, rep, rpt);
      return hipGetLastError();
    }
    case ACT_F16: return launch_rep<ACT_F16>(rep, a, s);
    case ACT_BF16: return launch_rep<ACT_BF16>(rep, a, s);
  }
  return hipErrorInvalidValue;
}
