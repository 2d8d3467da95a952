// Row-wise kernels of the decoder: RMSNorm, per-head q/k RMSNorm + RoPE with
// the fused KV-cache store, embedding gathers and the on-device greedy step.
#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

// RmsNorm::forward (linear.rs:293-302): y = rd(x * (1/sqrt(mean(x^2)+eps)) * w).
// One work-group (256 threads) per row.
template <int A>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const void* xv, int ldx, const void* wv,
                                                      int dim, float eps, void* yv, int ldy) {
  typedef typename ActT<A>::T T;
  const T* x = (const T*)xv + (size_t)blockIdx.x * ldx;
  const T* w = (const T*)wv;
  T* y = (T*)yv + (size_t)blockIdx.x * ldy;
  __shared__ float red[4];
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += 256) {
    const float v = ld_act<A>(x[i]);
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(tot, (float)dim), eps)));
  for (int i = threadIdx.x; i < dim; i += 256)
    y[i] = st_act<A>(__fmul_rn(__fmul_rn(ld_act<A>(x[i]), rinv), ld_act<A>(w[i])));
}

// The same for 16-bit activations and dim = 512 * NC: one wave per row, four
// rows per work-group; each lane loads its NC 8-element pieces of x and of
// the gain once (16-byte loads), sums its squares in order, then the wave.
template <int A, int NC>
__global__ void __launch_bounds__(256) rmsnorm16_kernel(const void* xv, int ldx, const void* wv,
                                                        int rows, float eps, void* yv, int ldy) {
  typedef typename ActT<A>::T T;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // whole waves leave together
  const T* x = (const T*)xv + (size_t)r * ldx;
  T* y = (T*)yv + (size_t)r * ldy;
  u32x4 xr[NC], wr[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    xr[i] = *(const u32x4*)(x + (i * 64 + lane) * 8);
    wr[i] = *(const u32x4*)((const T*)wv + (i * 64 + lane) * 8);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    float v[8];
    unpack8<A>(xr[i], v);
#pragma unroll
    for (int t = 0; t < 8; ++t) ss += v[t] * v[t];
  }
  ss = wave_sum(ss);
  const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(ss, (float)(NC * 512)), eps)));
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    float v[8], g[8];
    unpack8<A>(xr[i], v);
    unpack8<A>(wr[i], g);
    uint32_t o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      o[t] = (uint32_t)st_act<A>(__fmul_rn(__fmul_rn(v[2 * t], rinv), g[2 * t])) |
             ((uint32_t)st_act<A>(__fmul_rn(__fmul_rn(v[2 * t + 1], rinv), g[2 * t + 1])) << 16);
    *(u32x4*)(y + (i * 64 + lane) * 8) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// Attention::forward steps 3-5 (qwen3.rs:214-227): per-head RMSNorm of q and k
// over head_dim (before RoPE), rotate-half RoPE at the absolute position
// (qwen3.rs:139-144), then KvCache::append's in-place write (qwen3.rs:86-101)
// at element ((b*nkv + h)*cap + pos)*hd + d.  f32 activations: one wave per
// (row, head slot); head_dim is 128: lane l owns the rotation pair (l, l+64).
template <int A>
__global__ void __launch_bounds__(256) rope_store_kernel(RopeArgs p) {
  typedef typename ActT<A>::T T;
  const int lane = threadIdx.x & 63;
  const int slot = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int r = blockIdx.x;
  const int nslots = p.nh + 2 * p.nkv;
  if (slot >= nslots || r >= p.rows) return;
  const int b = p.row_b ? p.row_b[r] : r;
  const int pos = p.row_pos ? p.row_pos[r] : p.state[0];
  const T* src = (const T*)p.qkv + (size_t)r * p.ldqkv + slot * 128;
  float x0 = ld_act<A>(src[lane]), x1 = ld_act<A>(src[lane + 64]);
  if (slot >= p.nh + p.nkv) {  // value head: stored as projected
    T* dst = (T*)p.vc + (((size_t)b * p.nkv + (slot - p.nh - p.nkv)) * p.cap + pos) * 128;
    dst[lane] = src[lane];
    dst[lane + 64] = src[lane + 64];
    return;
  }
  const bool is_q = slot < p.nh;
  const T* g = (const T*)(is_q ? p.qn_w : p.kn_w);
  // Explicitly rounded operations (no FMA contraction) so the stored K is the
  // same bit pattern a plain IEEE evaluation of the formula gives.
  const float ss = wave_sum(__fmul_rn(x0, x0) + __fmul_rn(x1, x1));
  const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(ss, 128.0f), p.eps)));
  const float y0 = rd<A>(__fmul_rn(__fmul_rn(x0, rinv), ld_act<A>(g[lane])));
  const float y1 = rd<A>(__fmul_rn(__fmul_rn(x1, rinv), ld_act<A>(g[lane + 64])));
  const float c = ld_act<A>(((const T*)p.cos)[(size_t)pos * 64 + lane]);
  const float s = ld_act<A>(((const T*)p.sin)[(size_t)pos * 64 + lane]);
  const T o0 = st_act<A>(__fsub_rn(__fmul_rn(y0, c), __fmul_rn(y1, s)));
  const T o1 = st_act<A>(__fadd_rn(__fmul_rn(y1, c), __fmul_rn(y0, s)));
  T* dst;
  if (is_q)
    dst = (T*)p.q_out + ((size_t)r * p.nh + slot) * 128;
  else
    dst = (T*)p.kc + (((size_t)b * p.nkv + (slot - p.nh)) * p.cap + pos) * 128;
  dst[lane] = o0;
  dst[lane + 64] = o1;
}

// Qwen3::embed (qwen3.rs:405-412): row gather from the (V, H) table.
template <int A>
__global__ void embed_kernel(const uint32_t* ids, const void* table, int hidden, void* out) {
  typedef typename ActT<A>::T T;
  const T* src = (const T*)table + (size_t)ids[blockIdx.x] * hidden;
  T* dst = (T*)out + (size_t)blockIdx.x * hidden;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) dst[i] = src[i];
}

// Prompt assembly (MossTranscribeDiarize::splice_audio, mod.rs:128-180, then
// the left pad of engine.rs:476-491): output row r takes src[r] >= 0 -> that
// token's embedding, -1 -> zeros (left pad), <= -2 -> audio row -2 - src[r],
// converted from the audio dtype (0 f32, 1 f16, 2 bf16) to the activation
// dtype with round-to-nearest-even, as to_dtype does.
template <int A>
__global__ void assemble_kernel(const int32_t* src, const void* table, const void* audio,
                                int audio_dtype, int hidden, void* out) {
  typedef typename ActT<A>::T T;
  const int s = src[blockIdx.x];
  T* dst = (T*)out + (size_t)blockIdx.x * hidden;
  if (s >= 0) {
    const T* e = (const T*)table + (size_t)s * hidden;
    for (int i = threadIdx.x; i < hidden; i += blockDim.x) dst[i] = e[i];
  } else if (s == -1) {
    for (int i = threadIdx.x; i < hidden; i += blockDim.x) dst[i] = st_act<A>(0.f);
  } else {
    const size_t row = (size_t)(-2 - s) * hidden;
    for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
      float v;
      if (audio_dtype == 0) v = ((const float*)audio)[row + i];
      else if (audio_dtype == 1) v = f16_to_f32(((const uint16_t*)audio)[row + i]);
      else v = bf16_to_f32(((const uint16_t*)audio)[row + i]);
      dst[i] = st_act<A>(v);
    }
  }
}

template <int A>
__global__ void gather_rows_kernel(const void* src, int ld_src, const int32_t* rows, int dim,
                                   void* dst, int ld_dst) {
  typedef typename ActT<A>::T T;
  const T* s = (const T*)src + (size_t)rows[blockIdx.x] * ld_src;
  T* d = (T*)dst + (size_t)blockIdx.x * ld_dst;
  for (int i = threadIdx.x; i < dim; i += blockDim.x) d[i] = s[i];
}

// One greedy step of Engine::generate_batch (engine.rs:505-531) on the device:
// argmax_rows (550-559; ties go to the smallest index), end-of-turn
// bookkeeping (a row that emits eos is done with FinishReason::Stop and the
// token is not kept), feeding eos to finished rows, and the embedding of the
// next step's input.  A single work-group, so the shared state update is
// race-free.
template <int A>
__global__ void __launch_bounds__(1024) greedy_kernel(GreedyArgs p) {
  typedef typename ActT<A>::T T;
  __shared__ uint64_t wbest[16][16];
  __shared__ uint32_t nxt[16];
  __shared__ int ndone;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // The row state this kernel reads (nothing before it in the step changes
  // it) is loaded first, so its round trip overlaps the parts'.
  int done0 = 0, force0 = -1, ntok0 = 0, step0 = 0, len0 = 0, ndone0 = 0;
  if (threadIdx.x == 0) {
    len0 = p.state[0];
    ndone0 = p.state[2];
  }
  if ((int)threadIdx.x < p.batch) {
    const int b = threadIdx.x;
    done0 = p.done[b];
    ntok0 = p.ntok[b];
    if (p.force) force0 = p.force[b];
    step0 = p.state[1];
  }
  // Every row's keys of a part are contiguous: one pass over the parts reads
  // all rows (one memory round trip, not one per row), then each row is
  // reduced across the wave.
  uint64_t best[16];
#pragma unroll
  for (int b = 0; b < 16; ++b) best[b] = 0;
  for (int i = threadIdx.x; i < p.nparts; i += blockDim.x) {
    const uint64_t* k = p.part + (size_t)i * p.batch;
#pragma unroll
    for (int b = 0; b < 16; ++b)
      if (b < p.batch) best[b] = k[b] > best[b] ? k[b] : best[b];
  }
#pragma unroll
  for (int b = 0; b < 16; ++b) {
    if (b >= p.batch) break;
    for (int off = 32; off > 0; off >>= 1) {
      const uint64_t o = __shfl_xor(best[b], off);
      best[b] = o > best[b] ? o : best[b];
    }
    if (lane == 0) wbest[b][w] = best[b];
  }
  if (threadIdx.x == 0) ndone = 0;
  __syncthreads();
  const int step = step0;
  if ((int)threadIdx.x < p.batch) {
    const int b = threadIdx.x;
    uint64_t best = 0;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) best = wbest[b][i] > best ? wbest[b][i] : best;
    uint32_t tok = argmax_key_index(best);
    if (tok >= (uint32_t)p.vocab) tok = 0;  // unreachable for finite key sets; keeps the gather in bounds
    int done = done0;
    if (!done) {
      if (p.force && force0 == step) tok = p.eos;
      if (tok == p.eos) {
        done = 1;
        p.done[b] = 1;
        p.finish[b] = 1;
      } else if (ntok0 < p.budget) {
        p.tokens[(size_t)b * p.budget + ntok0] = tok;
        p.ntok[b] = ntok0 + 1;
      }
    }
    const uint32_t feed = done ? p.eos : tok;
    nxt[b] = feed;
    p.next_ids[b] = feed;
    if (done) atomicAdd(&ndone, 1);
  }
  __syncthreads();
  // next inputs: all rows' embedding loads are issued before any store (the
  // table and x could alias as far as the compiler knows, which would
  // otherwise order each row's loads after the previous row's stores)
  for (int i = threadIdx.x; i < p.hidden; i += blockDim.x) {
    T v[16];
#pragma unroll
    for (int b = 0; b < 16; ++b)
      if (b < p.batch) v[b] = ((const T*)p.embed)[(size_t)nxt[b] * p.hidden + i];
#pragma unroll
    for (int b = 0; b < 16; ++b)
      if (b < p.batch) ((T*)p.x)[(size_t)b * p.hidden + i] = v[b];
  }
  if (threadIdx.x == 0) {
    const int len = len0 + p.advance;
    const bool changed = ndone0 != ndone;
    p.state[0] = len;
    p.state[1] = step + 1;
    p.state[2] = ndone;
    // The host reads only the done count, through host-mapped memory: a store
    // there crosses the bus and the kernel's end waits for it, so it is made
    // only when the count changes (the host clears the mirror with the state).
    if (p.host_state && changed) p.host_state[2] = ndone;
  }
}

__global__ void fill_i32_kernel(int32_t* dst, int64_t n, int32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = v;
}

}  // namespace

template <int A>
hipError_t launch_rmsnorm16(const void* x, int ldx, const void* w, int rows, int dim, float eps,
                            void* y, int ldy, hipStream_t s) {
  const dim3 grid((rows + 3) / 4);
  switch (dim / 512) {
    case 1: hipLaunchKernelGGL((rmsnorm16_kernel<A, 1>), grid, dim3(256), 0, s, x, ldx, w, rows, eps, y, ldy); break;
    case 2: hipLaunchKernelGGL((rmsnorm16_kernel<A, 2>), grid, dim3(256), 0, s, x, ldx, w, rows, eps, y, ldy); break;
    case 4: hipLaunchKernelGGL((rmsnorm16_kernel<A, 4>), grid, dim3(256), 0, s, x, ldx, w, rows, eps, y, ldy); break;
    case 8: hipLaunchKernelGGL((rmsnorm16_kernel<A, 8>), grid, dim3(256), 0, s, x, ldx, w, rows, eps, y, ldy); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rmsnorm(int act, const void* x, int ldx, const void* w, int rows, int dim,
                          float eps, void* y, int ldy, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  // 16-bit rows of 512, 1024, 2048 or 4096 with 16-byte aligned rows: one wave per row
  const bool vec = dim % 512 == 0 && (dim / 512 == 1 || dim / 512 == 2 || dim / 512 == 4 ||
                                      dim / 512 == 8) &&
                   ldx % 8 == 0 && ldy % 8 == 0 && ((uintptr_t)x | (uintptr_t)y | (uintptr_t)w) % 16 == 0;
  if (vec && act == ACT_F16) return launch_rmsnorm16<ACT_F16>(x, ldx, w, rows, dim, eps, y, ldy, s);
  if (vec && act == ACT_BF16) return launch_rmsnorm16<ACT_BF16>(x, ldx, w, rows, dim, eps, y, ldy, s);
  switch (act) {
    case ACT_F32: hipLaunchKernelGGL(rmsnorm_kernel<ACT_F32>, dim3(rows), dim3(256), 0, s, x, ldx, w, dim, eps, y, ldy); break;
    case ACT_F16: hipLaunchKernelGGL(rmsnorm_kernel<ACT_F16>, dim3(rows), dim3(256), 0, s, x, ldx, w, dim, eps, y, ldy); break;
    case ACT_BF16: hipLaunchKernelGGL(rmsnorm_kernel<ACT_BF16>, dim3(rows), dim3(256), 0, s, x, ldx, w, dim, eps, y, ldy); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// f32 activations only: 16-bit prefill runs this step in the q|k|v GEMM's
// EPI_ROPE epilogue.
hipError_t launch_rope_store(int act, const RopeArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  if (act != ACT_F32) return hipErrorInvalidValue;
  const dim3 grid(a.rows, (a.nh + 2 * a.nkv + 3) / 4);
  hipLaunchKernelGGL(rope_store_kernel<ACT_F32>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_embed(int act, const uint32_t* ids, int n, const void* table, int hidden,
                        void* out, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  switch (act) {
    case ACT_F32: hipLaunchKernelGGL(embed_kernel<ACT_F32>, dim3(n), dim3(256), 0, s, ids, table, hidden, out); break;
    case ACT_F16: hipLaunchKernelGGL(embed_kernel<ACT_F16>, dim3(n), dim3(256), 0, s, ids, table, hidden, out); break;
    case ACT_BF16: hipLaunchKernelGGL(embed_kernel<ACT_BF16>, dim3(n), dim3(256), 0, s, ids, table, hidden, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_assemble(int act, const int32_t* src, int rows, const void* table,
                           const void* audio, int audio_dtype, int hidden, void* out, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (audio_dtype < 0 || audio_dtype > 2) return hipErrorInvalidValue;
  switch (act) {
    case ACT_F32: hipLaunchKernelGGL(assemble_kernel<ACT_F32>, dim3(rows), dim3(256), 0, s, src, table, audio, audio_dtype, hidden, out); break;
    case ACT_F16: hipLaunchKernelGGL(assemble_kernel<ACT_F16>, dim3(rows), dim3(256), 0, s, src, table, audio, audio_dtype, hidden, out); break;
    case ACT_BF16: hipLaunchKernelGGL(assemble_kernel<ACT_BF16>, dim3(rows), dim3(256), 0, s, src, table, audio, audio_dtype, hidden, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gather_rows(int act, const void* src, int ld_src, const int32_t* rows, int n,
                              int dim, void* dst, int ld_dst, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  switch (act) {
    case ACT_F32: hipLaunchKernelGGL(gather_rows_kernel<ACT_F32>, dim3(n), dim3(256), 0, s, src, ld_src, rows, dim, dst, ld_dst); break;
    case ACT_F16: hipLaunchKernelGGL(gather_rows_kernel<ACT_F16>, dim3(n), dim3(256), 0, s, src, ld_src, rows, dim, dst, ld_dst); break;
    case ACT_BF16: hipLaunchKernelGGL(gather_rows_kernel<ACT_BF16>, dim3(n), dim3(256), 0, s, src, ld_src, rows, dim, dst, ld_dst); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_greedy(int act, const GreedyArgs& a, hipStream_t s) {
  if (a.batch < 1 || a.batch > 16) return hipErrorInvalidValue;
  switch (act) {
    case ACT_F32: hipLaunchKernelGGL(greedy_kernel<ACT_F32>, dim3(1), dim3(1024), 0, s, a); break;
    case ACT_F16: hipLaunchKernelGGL(greedy_kernel<ACT_F16>, dim3(1), dim3(1024), 0, s, a); break;
    case ACT_BF16: hipLaunchKernelGGL(greedy_kernel<ACT_BF16>, dim3(1), dim3(1024), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_fill_i32(int32_t* dst, int64_t n, int32_t v, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  int grid = (int)((n + 255) / 256);
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(fill_i32_kernel, dim3(grid), dim3(256), 0, s, dst, n, v);
  return hipGetLastError();
}
