// Skinny projections for decode (rows <= 16): y = x W^T on the 16x16 MFMAs.
//
// The batch rows are the MFMA's M side (A operand, zero-padded to 16) and 16
// weight rows are its N side (B operand), so every output lane owns one weight
// row and one Q8_0 scale per 32-wide block.  Weights are pre-tiled in B-operand
// order (fmd_kernels.h), so each wave loads whole 1 KiB chunks with one 16-byte
// load per lane.  A work-group of K/256 waves splits K; each wave holds its
// 256-wide slice of x in registers (with the RMSNorm of the projection's input
// fused in), and the partial 16x16 tiles are reduced in LDS in a fixed order,
// so a row's result does not depend on how many rows the batch has.
//
// Reference: Linear::forward (linear.rs:29-65), FusedLinear (78-100),
// RmsNorm::forward (293-302); call sites qwen3.rs:213, 258, 288-291, 459-463.
#include <cstdlib>

#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

constexpr int KBW = 8;  // 32-wide k-blocks per wave: a wave covers 256 of K

template <int A>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (A == ACT_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ u32x4 q8_to_f16x8(uint32_t w0, uint32_t w1) {
  uint32_t a, b, c, d;
  i8x4_to_f16x4(w0, a, b);
  i8x4_to_f16x4(w1, c, d);
  return u32x4{a, b, c, d};
}

// Shared epilogue: reduce the per-wave partial tiles and write the outputs.
// red: [NW][TPW][64 lanes][4]; output element e = jj*256 + b*16 + n.
// Residuals of the EPI_RESID epilogue: TPW == 1, so the thread handles the
// output elements e = threadIdx.x + i * blockDim.x < 256 / RS, i < 4 (a
// work-group has at least one wave); resv[i] is element i's residual.  A
// launch bound above 256 threads means at least five waves, hence i == 0
// only.
struct Resid4 {
  float v[4];
};

// Output element e0 of a work-group that computes the columns
// [sub*16/RS, (sub+1)*16/RS) of its tiles (sub = blockIdx.x % RS): slot jj,
// batch row b, column n of the 16-column tile.
template <int RS>
__device__ __forceinline__ void out_elem(int e0, int& jj, int& b, int& n) {
  constexpr int C = 16 / RS;
  jj = e0 / (16 * C);
  const int r = e0 % (16 * C);
  b = r / C;
  n = (int)(blockIdx.x % RS) * C + r % C;
}

template <int A, int EPI, int TPW, int RS = 1>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs& p, float* red, uint64_t* keys,
                                              int NW, const Resid4& resv) {
  typedef typename ActT<A>::T T;
  const int ntiles = p.W.out / 16;
  const int blk = blockIdx.x / RS;
  constexpr int NSLOT_OUT = (EPI == EPI_SWIGLU) ? TPW / 2 : TPW;
  int it = 0;
  for (int e0 = threadIdx.x; e0 < NSLOT_OUT * 256 / RS; e0 += blockDim.x, ++it) {
    int jj, b, n;
    out_elem<RS>(e0, jj, b, n);
    const int e = jj * 256 + b * 16 + n;
    const int li = 16 * (b >> 2) + n, r = b & 3;
    auto slot_sum = [&](int j) {
      float s = 0.f;
      for (int ww = 0; ww < NW; ++ww) s += red[((ww * TPW + j) * 64 + li) * 4 + r];
      return s;
    };
    if constexpr (EPI == EPI_SWIGLU) {
      const int pair = blk * (TPW / 2) + jj;
      if (pair >= ntiles / 2 || b >= p.rows) continue;
      const float g = rd<A>(slot_sum(2 * jj)), u = rd<A>(slot_sum(2 * jj + 1));
      const float s = rd<A>(g / (1.0f + __expf(-g)));
      ((T*)p.y)[(size_t)b * p.ldy + pair * 16 + n] = st_act<A>(s * u);
    } else {
      const int tile = blk * TPW + jj;
      const bool ok = tile < ntiles && b < p.rows;
      const int col = tile * 16 + n;
      const float v = ok ? slot_sum(jj) : 0.f;
      if constexpr (EPI == EPI_STORE) {
        if (ok) ((T*)p.y)[(size_t)b * p.ldy + col] = st_act<A>(v);
      } else if constexpr (EPI == EPI_RESID) {
        // the residual of this element, loaded at kernel start (selected, not
        // indexed: a run-time index would put resv in scratch memory)
        const int sl = it & 3;
        const float rv = sl == 0 ? resv.v[0] : sl == 1 ? resv.v[1] : sl == 2 ? resv.v[2] : resv.v[3];
        if (ok) ((T*)p.y)[(size_t)b * p.ldy + col] = st_act<A>(rv + rd<A>(v));
      } else {  // EPI_LOGITS
        const float lv = rd<A>(v);
        if (ok) ((float*)p.y)[(size_t)b * p.ldy + col] = lv;
        keys[e] = ok ? argmax_key(lv, (uint32_t)col) : 0ull;
      }
    }
  }
  if constexpr (EPI == EPI_LOGITS) {
    __syncthreads();
    if ((int)threadIdx.x < p.rows) {
      const int b = threadIdx.x;
      uint64_t best = 0;
      for (int jj = 0; jj < TPW; ++jj)
        for (int n = 0; n < 16; ++n) {
          const uint64_t k = keys[jj * 256 + b * 16 + n];
          best = k > best ? k : best;
        }
      p.amax_part[(size_t)blockIdx.x * p.rows + b] = best;
    }
  }
}

// The residual elements the epilogue will add for this thread (EPI_RESID:
// TPW == 1; element e = threadIdx.x + i * blockDim.x < 256 / RS goes to slot i).
template <int A, int EPI, int MAXT, int RS = 1>
__device__ __forceinline__ Resid4 prefetch_resid(const GemvArgs& p) {
  Resid4 r{{0.f, 0.f, 0.f, 0.f}};
  if constexpr (EPI == EPI_RESID) {
    typedef typename ActT<A>::T T;
    const int tile = blockIdx.x / RS;
    constexpr int NSLOT = MAXT > 256 ? 1 : 4;
#pragma unroll
    for (int i = 0; i < NSLOT; ++i) {
      const int e = threadIdx.x + i * blockDim.x;
      int jj, b, n;
      out_elem<RS>(e, jj, b, n);
      if (e < 256 / RS && b < p.rows && tile < p.W.out / 16)
        r.v[i] = ld_act<A>(((const T*)p.resid)[(size_t)b * p.ldy + tile * 16 + n]);
    }
  }
  return r;
}

// 16-bit activations (f16 / bf16) with dense 16-bit or Q8_0 weights.
template <int A, int WK, int TPW, int EPI, bool NORM, int MAXT, int RS>
__global__ void __launch_bounds__(MAXT) gemv16_kernel(GemvArgs p) {
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int NW = blockDim.x >> 6;
  const int K = p.W.in;
  const int row = lane & 15, kg = lane >> 4;
  const int ntiles = p.W.out / 16;
  float* red = smem;                                   // NW*TPW*256 floats
  float* sred = smem + NW * TPW * 256;                 // 16*NW floats
  uint64_t* keys = (uint64_t*)(sred + 16 * NW + 16);   // TPW*256 keys (EPI_LOGITS)

  // Slot j -> weight row-tile.  SwiGLU pairs gate tile t with up tile t + ntiles/2.
  // RS work-groups share a tile, each loading the weight rows of its own
  // 16/RS output columns (the MFMA's other columns then hold zeros).
  const int blk = blockIdx.x / RS;
  const bool mine = RS == 1 || row / (16 / RS) == (int)(blockIdx.x % RS);
  int tile[TPW];
  bool valid[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    if constexpr (EPI == EPI_SWIGLU) {
      const int pair = blk * (TPW / 2) + j / 2;
      valid[j] = pair < ntiles / 2 && mine;
      tile[j] = pair + ((j & 1) ? ntiles / 2 : 0);
    } else {
      tile[j] = blk * TPW + j;
      valid[j] = tile[j] < ntiles && mine;
    }
  }

  // Loads, in the order they are needed: with a fused RMSNorm the input
  // slice comes first (the norm runs while the weights stream in; the
  // vector-memory counter retires in order), otherwise the weights lead;
  // the residual of the epilogue goes last.
  u32x4 xa[KBW];
  const uint16_t* x = (const uint16_t*)p.x;
  const int kbase = w * (KBW * 32);
  auto load_x = [&]() {
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
      const int k = kbase + 32 * i + 8 * kg;
      xa[i] = (row < p.rows) ? *(const u32x4*)(x + (size_t)row * p.ldx + k) : u32x4{0, 0, 0, 0};
    }
  };
  u32x4 gain[NORM ? KBW : 1];
  if constexpr (NORM) {
    load_x();
    const uint16_t* nw = (const uint16_t*)p.norm_w;
#pragma unroll
    for (int i = 0; i < KBW; ++i) gain[i] = *(const u32x4*)(nw + kbase + 32 * i + 8 * kg);
  }
  constexpr int NCH = (WK == WK_Q8) ? KBW / 2 : KBW;
  u32x4 wv[TPW][NCH];
  uint32_t ws[TPW][(WK == WK_Q8) ? KBW / 2 : 1];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if constexpr (WK == WK_Q8) {
        const size_t ch = (size_t)tile[j] * (K / 64) + w * (KBW / 2) + c;
        wv[j][c] = valid[j] ? __builtin_nontemporal_load(((const u32x4*)p.W.w) + ch * 64 + lane)
                            : u32x4{0, 0, 0, 0};
        ws[j][c] = valid[j] ? __builtin_nontemporal_load(p.W.sc + ch * 16 + row) : 0u;
      } else {
        const size_t ch = (size_t)tile[j] * (K / 32) + w * KBW + c;
        wv[j][c] = valid[j] ? __builtin_nontemporal_load(((const u32x4*)p.W.w) + ch * 64 + lane)
                            : u32x4{0, 0, 0, 0};
      }
    }
  }
  if constexpr (!NORM) load_x();
  const Resid4 resv = prefetch_resid<A, EPI, MAXT, RS>(p);
  // every work-group of the attention launch before this kernel has ended
  if (p.epoch && blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_fetch_add(p.epoch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
      float v[8];
      unpack8<A>(xa[i], v);
#pragma unroll
      for (int t = 0; t < 8; ++t) ss += v[t] * v[t];
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    if (kg == 0) sred[w * 16 + row] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < NW; ++i) tot += sred[i * 16 + row];
    const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(tot, (float)K), p.eps)));
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
      float v[8], g[8];
      unpack8<A>(xa[i], v);
      unpack8<A>(gain[i], g);
      uint32_t o[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        o[t] = (uint32_t)st_act<A>(__fmul_rn(__fmul_rn(v[2 * t], rinv), g[2 * t])) |
               ((uint32_t)st_act<A>(__fmul_rn(__fmul_rn(v[2 * t + 1], rinv), g[2 * t + 1])) << 16);
      xa[i] = u32x4{o[0], o[1], o[2], o[3]};
    }
  }

  f32x4 acc[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if constexpr (WK == WK_Q8) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        const f32x4 t0 = mfma16<ACT_F16>(xa[2 * c], q8_to_f16x8(wv[j][c][0], wv[j][c][1]), z);
        const f32x4 t1 = mfma16<ACT_F16>(xa[2 * c + 1], q8_to_f16x8(wv[j][c][2], wv[j][c][3]), z);
        const float d0 = f16_to_f32((uint16_t)(ws[j][c] & 0xffffu));
        const float d1 = f16_to_f32((uint16_t)(ws[j][c] >> 16));
        acc[j] += d0 * t0;
        acc[j] += d1 * t1;
      } else {
        acc[j] = mfma16<A>(xa[c], wv[j][c], acc[j]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < TPW; ++j) *(f32x4*)&red[((w * TPW + j) * 64 + lane) * 4] = acc[j];
  __syncthreads();
  gemv_epilogue<A, EPI, TPW, RS>(p, red, keys, NW, resv);
}

// The lm_head (EPI_LOGITS) for 16-bit activations, as a persistent stream:
// a grid of about two work-groups per CU, each normalising x once and then
// walking NG groups of TPW 16-row weight tiles (group blockIdx.x + i*gridDim.x)
// with the next group's loads in flight while the current one is reduced.
// Each thread keeps the running argmax keys of its output slots; the
// work-group writes one key per row at the end (argmax: ties -> first index,
// engine.rs:480-485).
template <int A, int WK, int TPW, int NG, int MAXT, bool PF>
__global__ void __launch_bounds__(MAXT) logits16_kernel(GemvArgs p) {
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int NW = blockDim.x >> 6;
  const int K = p.W.in;
  const int row = lane & 15, kg = lane >> 4;
  const int ntiles = p.W.out / 16;
  float* red = smem;                                     // [2][NW][TPW][64][4]
  float* sred = smem + 2 * NW * TPW * 256;               // [NW][16]
  float* stage = sred + 16 * NW;                         // [NG][TPW*256] logits

  constexpr int NCH = (WK == WK_Q8) ? KBW / 2 : KBW;
  constexpr int NSC = (WK == WK_Q8) ? KBW / 2 : 1;
  constexpr int NB = PF ? 2 : 1;
  u32x4 wv[NB][TPW][NCH];
  uint32_t ws[NB][TPW][NSC];
  auto load = [&](int i, int buf) {
    const int g = blockIdx.x + i * gridDim.x;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int tile = g * TPW + j;
      const bool ok = tile < ntiles;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if constexpr (WK == WK_Q8) {
          const size_t ch = (size_t)tile * (K / 64) + w * (KBW / 2) + c;
          wv[buf][j][c] = ok ? __builtin_nontemporal_load(((const u32x4*)p.W.w) + ch * 64 + lane)
                             : u32x4{0, 0, 0, 0};
          ws[buf][j][c] = ok ? __builtin_nontemporal_load(p.W.sc + ch * 16 + row) : 0u;
        } else {
          const size_t ch = (size_t)tile * (K / 32) + w * KBW + c;
          wv[buf][j][c] = ok ? __builtin_nontemporal_load(((const u32x4*)p.W.w) + ch * 64 + lane)
                             : u32x4{0, 0, 0, 0};
        }
      }
    }
  };
  load(0, 0);
  __builtin_amdgcn_sched_barrier(0);

  // A operand: this wave's 256-wide slice of the final-norm output.
  u32x4 xa[KBW];
  const uint16_t* x = (const uint16_t*)p.x;
  const int kbase = w * (KBW * 32);
#pragma unroll
  for (int i = 0; i < KBW; ++i) {
    const int k = kbase + 32 * i + 8 * kg;
    xa[i] = (row < p.rows) ? *(const u32x4*)(x + (size_t)row * p.ldx + k) : u32x4{0, 0, 0, 0};
  }
  {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
      float v[8];
      unpack8<A>(xa[i], v);
#pragma unroll
      for (int t = 0; t < 8; ++t) ss += v[t] * v[t];
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    if (kg == 0) sred[w * 16 + row] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < NW; ++i) tot += sred[i * 16 + row];
    const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(tot, (float)K), p.eps)));
    const uint16_t* nw = (const uint16_t*)p.norm_w;
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
      const int k = kbase + 32 * i + 8 * kg;
      float v[8], g[8];
      unpack8<A>(xa[i], v);
      unpack8<A>(*(const u32x4*)(nw + k), g);
      uint32_t o[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        o[t] = (uint32_t)st_act<A>(__fmul_rn(__fmul_rn(v[2 * t], rinv), g[2 * t])) |
               ((uint32_t)st_act<A>(__fmul_rn(__fmul_rn(v[2 * t + 1], rinv), g[2 * t + 1])) << 16);
      xa[i] = u32x4{o[0], o[1], o[2], o[3]};
    }
  }

  __shared__ unsigned long long s_best[16];  // running argmax key per row
  if (threadIdx.x < 16) s_best[threadIdx.x] = 0ull;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    if constexpr (PF) {
      if (i + 1 < NG) load(i + 1, (i + 1) & 1);
    } else if (i > 0) {
      load(i, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int buf = PF ? (i & 1) : 0;
    float* rb = red + (i & 1) * NW * TPW * 256;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if constexpr (WK == WK_Q8) {
          const f32x4 z = {0.f, 0.f, 0.f, 0.f};
          const f32x4 t0 =
              mfma16<ACT_F16>(xa[2 * c], q8_to_f16x8(wv[buf][j][c][0], wv[buf][j][c][1]), z);
          const f32x4 t1 =
              mfma16<ACT_F16>(xa[2 * c + 1], q8_to_f16x8(wv[buf][j][c][2], wv[buf][j][c][3]), z);
          const float d0 = f16_to_f32((uint16_t)(ws[buf][j][c] & 0xffffu));
          const float d1 = f16_to_f32((uint16_t)(ws[buf][j][c] >> 16));
          acc += d0 * t0;
          acc += d1 * t1;
        } else {
          acc = mfma16<A>(xa[c], wv[buf][j][c], acc);
        }
      }
      *(f32x4*)&rb[((w * TPW + j) * 64 + lane) * 4] = acc;
    }
    // One barrier per group: the two reduction buffers alternate, and every
    // read of a buffer precedes the barrier of the next group.
    __syncthreads();
    const int g = blockIdx.x + i * gridDim.x;
    // Output slot e = jj*256 + b*16 + n; the 16 lanes of a slot row share
    // (jj, b), so their keys are max-reduced before one LDS atomic.  Waves
    // are whole slot rows (blockDim and TPW*256 are multiples of 64).
    for (int e = threadIdx.x; e < TPW * 256; e += blockDim.x) {
      const int jj = e >> 8, b = (e >> 4) & 15, n = e & 15;
      const int li = 16 * (b >> 2) + n, r = b & 3;
      const int tile = g * TPW + jj;
      uint64_t key = 0;
      if (tile < ntiles && b < p.rows) {
        float v = 0.f;
        for (int ww = 0; ww < NW; ++ww) v += rb[((ww * TPW + jj) * 64 + li) * 4 + r];
        const float lv = rd<A>(v);
        stage[i * TPW * 256 + e] = lv;
        key = argmax_key(lv, (uint32_t)(tile * 16 + n));
      }
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) {
        const uint64_t o = __shfl_xor(key, off);
        key = o > key ? o : key;
      }
      if (n == 0 && key != 0) atomicMax(&s_best[b], (unsigned long long)key);
    }
  }
  __syncthreads();
  // The logits leave in one burst after the stream: global stores inside the
  // group loop would make the compiler drain every outstanding load with them.
  for (int f = threadIdx.x; f < NG * TPW * 256; f += blockDim.x) {
    const int i = f / (TPW * 256), e = f % (TPW * 256);
    const int jj = e >> 8, b = (e >> 4) & 15, n = e & 15;
    const int tile = (blockIdx.x + i * gridDim.x) * TPW + jj;
    if (tile < ntiles && b < p.rows) ((float*)p.y)[(size_t)b * p.ldy + tile * 16 + n] = stage[f];
  }
  if ((int)threadIdx.x < p.rows)
    p.amax_part[(size_t)blockIdx.x * p.rows + threadIdx.x] = s_best[threadIdx.x];
}

// lm_head variant with independent waves: each wave owns whole 16-row weight
// tiles over the full K (no cross-wave reduction, no barrier in the stream).
// The final-norm output sits in LDS, padded against bank conflicts, and feeds
// the MFMA A operand; the weights stream in stages of 256 K, PD stages ahead,
// over NT tiles per wave (tile = wave + t * total waves).  Logits are staged
// in LDS and leave in one burst; each work-group writes one argmax key per row.
template <int A, int WK, int NW, int NT, int PD>
__global__ void __launch_bounds__(256) logits_wave_kernel(GemvArgs p) {
  extern __shared__ float smem[];
  constexpr int K = NW * 256;
  constexpr int LDX = K + 8;                       // f16/bf16 elements per LDS row
  constexpr int SK = 256;                          // K per stage
  constexpr int NS = K / SK;                       // stages per tile
  constexpr int CPS = (WK == WK_Q8) ? SK / 64 : SK / 32;  // 16-byte chunks per stage
  uint16_t* xs = (uint16_t*)smem;                  // [16][LDX]
  float* stage_out = (float*)(xs + 16 * LDX);      // [4 waves][NT][256]
  __shared__ unsigned long long s_best[16];
  __shared__ float s_ss[16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = lane & 15, kg = lane >> 4;
  const int ntiles = p.W.out / 16;
  const int nwaves = gridDim.x * 4;
  const int wid = blockIdx.x * 4 + w;

  u32x4 wv[PD + 1][CPS];
  uint32_t ws[PD + 1][(WK == WK_Q8) ? CPS : 1];
  auto load = [&](int st, int buf) {               // flattened stage index st
    const int t = st / NS, sk = st % NS;
    const int tile = wid + t * nwaves;
    const bool ok = tile < ntiles;
#pragma unroll
    for (int c = 0; c < CPS; ++c) {
      if constexpr (WK == WK_Q8) {
        const size_t ch = (size_t)tile * (K / 64) + sk * CPS + c;
        wv[buf][c] = ok ? __builtin_nontemporal_load(((const u32x4*)p.W.w) + ch * 64 + lane)
                        : u32x4{0, 0, 0, 0};
        ws[buf][c] = ok ? __builtin_nontemporal_load(p.W.sc + ch * 16 + row) : 0u;
      } else {
        const size_t ch = (size_t)tile * (K / 32) + sk * CPS + c;
        wv[buf][c] = ok ? __builtin_nontemporal_load(((const u32x4*)p.W.w) + ch * 64 + lane)
                        : u32x4{0, 0, 0, 0};
      }
    }
  };
  constexpr int NST = NT * NS;
#pragma unroll
  for (int st = 0; st < PD && st < NST; ++st) load(st, st);
  __builtin_amdgcn_sched_barrier(0);

  // Final RMSNorm (qwen3.rs:455) of the rows into LDS; rows >= p.rows are 0.
  // A wave's 64 pieces of 8 elements lie in one row (K/8 >= 64), so each
  // piece's sum of squares is a wave sum.
  if (threadIdx.x < 16) {
    s_ss[threadIdx.x] = 0.f;
    s_best[threadIdx.x] = 0ull;
  }
  __syncthreads();
  {
    // All loads first (row index clamped into range), then the arithmetic.
    const uint16_t* x = (const uint16_t*)p.x;
    const uint16_t* nw = (const uint16_t*)p.norm_w;
    constexpr int PER = 16 * K / 8 / 256;          // 8-element pieces per thread
    u32x4 xv[PER], gv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int piece = threadIdx.x + i * 256, r = piece / (K / 8), k = (piece % (K / 8)) * 8;
      xv[i] = *(const u32x4*)(x + (size_t)min(r, p.rows - 1) * p.ldx + k);
      gv[i] = *(const u32x4*)(nw + k);
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int r = (threadIdx.x + i * 256) / (K / 8);
      float v[8];
      unpack8<A>(xv[i], v);
      float ss = 0.f;
#pragma unroll
      for (int t = 0; t < 8; ++t) ss += v[t] * v[t];
      ss = wave_sum(ss);
      if (lane == 0 && r < p.rows) atomicAdd(&s_ss[r], ss);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int piece = threadIdx.x + i * 256, r = piece / (K / 8), k = (piece % (K / 8)) * 8;
      const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(s_ss[r], (float)K), p.eps)));
      float v[8], g[8];
      unpack8<A>(xv[i], v);
      unpack8<A>(gv[i], g);
      uint32_t o[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        o[t] = (uint32_t)st_act<A>(__fmul_rn(__fmul_rn(v[2 * t], rinv), g[2 * t])) |
               ((uint32_t)st_act<A>(__fmul_rn(__fmul_rn(v[2 * t + 1], rinv), g[2 * t + 1])) << 16);
      *(u32x4*)&xs[r * LDX + k] = r < p.rows ? u32x4{o[0], o[1], o[2], o[3]} : u32x4{0, 0, 0, 0};
    }
  }
  __syncthreads();

  float* myout = stage_out + w * NT * 256;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < NST; ++st) {
    if (st + PD < NST) load(st + PD, (st + PD) % (PD + 1));
    __builtin_amdgcn_sched_barrier(0);
    const int buf = st % (PD + 1), sk = st % NS;
#pragma unroll
    for (int c = 0; c < CPS; ++c) {
      if constexpr (WK == WK_Q8) {
        const int k0 = sk * SK + c * 64;
        const u32x4 a0 = *(const u32x4*)&xs[row * LDX + k0 + 8 * kg];
        const u32x4 a1 = *(const u32x4*)&xs[row * LDX + k0 + 32 + 8 * kg];
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        u32x4 b0 = q8_to_f16x8(wv[buf][c][0], wv[buf][c][1]);
        u32x4 b1 = q8_to_f16x8(wv[buf][c][2], wv[buf][c][3]);
        // Tie this block's operands to the running sum (an empty asm), so the
        // compiler cannot hoist later blocks' MFMAs: their unscaled results
        // would pile up in registers and cut occupancy.
        asm volatile("" : "+v"(b0), "+v"(b1) : "v"(acc));
        const f32x4 t0 = mfma16<ACT_F16>(a0, b0, z);
        const f32x4 t1 = mfma16<ACT_F16>(a1, b1, z);
        acc += f16_to_f32((uint16_t)(ws[buf][c] & 0xffffu)) * t0;
        acc += f16_to_f32((uint16_t)(ws[buf][c] >> 16)) * t1;
      } else {
        const int k0 = sk * SK + c * 32;
        const u32x4 a0 = *(const u32x4*)&xs[row * LDX + k0 + 8 * kg];
        acc = mfma16<A>(a0, wv[buf][c], acc);
      }
    }
    if (sk == NS - 1) {
      // tile done: lane holds rows 4*kg + i of column `row`
      const int t = st / NS;
#pragma unroll
      for (int i = 0; i < 4; ++i) myout[t * 256 + (4 * kg + i) * 16 + row] = rd<A>(acc[i]);
      acc = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // Keys per row: reduce the staged logits of this wave's tiles.
  for (int t = 0; t < NT; ++t) {
    const int tile = wid + t * nwaves;
    if (tile >= ntiles) break;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = 4 * kg + i;
      const float lv = myout[t * 256 + b * 16 + row];
      uint64_t key = b < p.rows ? argmax_key(lv, (uint32_t)(tile * 16 + row)) : 0ull;
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) {
        const uint64_t o = __shfl_xor(key, off);
        key = o > key ? o : key;
      }
      if (row == 0 && key != 0) atomicMax(&s_best[b], (unsigned long long)key);
      if (b < p.rows) ((float*)p.y)[(size_t)b * p.ldy + tile * 16 + row] = lv;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < p.rows)
    p.amax_part[(size_t)blockIdx.x * p.rows + threadIdx.x] = s_best[threadIdx.x];
}

// f32 activations and weights on v_mfma_f32_16x16x4f32.
template <int TPW, int EPI, bool NORM, int MAXT>
__global__ void __launch_bounds__(MAXT) gemv32_kernel(GemvArgs p) {
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int NW = blockDim.x >> 6;
  const int K = p.W.in;
  const int row = lane & 15, kg = lane >> 4;
  const int ntiles = p.W.out / 16;
  float* red = smem;
  float* sred = smem + NW * TPW * 256;
  uint64_t* keys = (uint64_t*)(sred + 16 * NW + 16);
  constexpr int NCH = 2 * KBW;  // 16-wide chunks per wave slice

  int tile[TPW];
  bool valid[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    if constexpr (EPI == EPI_SWIGLU) {
      const int pair = blockIdx.x * (TPW / 2) + j / 2;
      valid[j] = pair < ntiles / 2;
      tile[j] = pair + ((j & 1) ? ntiles / 2 : 0);
    } else {
      tile[j] = blockIdx.x * TPW + j;
      valid[j] = tile[j] < ntiles;
    }
  }
  f32x4 xa[NCH];
  const float* x = (const float*)p.x;
  const int kbase = w * (KBW * 32);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int k = kbase + 16 * c + 4 * kg;
    xa[c] = (row < p.rows) ? *(const f32x4*)(x + (size_t)row * p.ldx + k)
                           : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) ss += xa[c][t] * xa[c][t];
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    if (kg == 0) sred[w * 16 + row] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < NW; ++i) tot += sred[i * 16 + row];
    const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(tot, (float)K), p.eps)));
    const float* nw = (const float*)p.norm_w;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const f32x4 g = *(const f32x4*)(nw + kbase + 16 * c + 4 * kg);
#pragma unroll
      for (int t = 0; t < 4; ++t) xa[c][t] = __fmul_rn(__fmul_rn(xa[c][t], rinv), g[t]);
    }
  }
  f32x4 acc[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 wv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const size_t ch = (size_t)tile[j] * (K / 16) + w * NCH + c;
      wv[c] = valid[j] ? __builtin_nontemporal_load(((const f32x4*)p.W.w) + ch * 64 + lane)
                       : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[c][t], wv[c][t], acc[j], 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < TPW; ++j) *(f32x4*)&red[((w * TPW + j) * 64 + lane) * 4] = acc[j];
  __syncthreads();
  gemv_epilogue<ACT_F32, EPI, TPW>(p, red, keys, NW, prefetch_resid<ACT_F32, EPI, MAXT>(p));
}

template <int EPI> constexpr int tpw_of() {
  return EPI == EPI_SWIGLU ? 2 : (EPI == EPI_LOGITS ? 4 : 1);
}

// Work-groups per 16-column tile (16-bit activations).  Measured, int8 batch
// 8 at 4096 keys, ms per decode step: O and down split 1 / 2 / 4 ways
// (64 / 128 / 256 work-groups) 1.351 / 1.344 / 1.377; gate|up split 2 ways
// (384 work-groups) 1.422.
template <int EPI> constexpr int rs_of() { return EPI == EPI_RESID ? 2 : 1; }

template <int A, int WK, int EPI, bool NORM>
hipError_t launch_one(const GemvArgs& a, hipStream_t s) {
  constexpr int TPW = tpw_of<EPI>();
  const int NW = a.W.in / 256;
  const int ntiles = a.W.out / 16;
  const int units = (EPI == EPI_SWIGLU) ? ntiles / 2 : ntiles;
  const int per = (EPI == EPI_SWIGLU) ? TPW / 2 : TPW;
  constexpr int RS = A == ACT_F32 ? 1 : rs_of<EPI>();
  const int grid = (units + per - 1) / per * RS;
  const size_t smem = sizeof(float) * (NW * TPW * 256 + 16 * NW + 16) +
                      (EPI == EPI_LOGITS ? sizeof(uint64_t) * TPW * 256 : 0);
  // The launch bound follows the work-group size (K/256 waves) so that small
  // work-groups keep a large register budget.
  if constexpr (A == ACT_F32) {
    if (NW <= 4)
      hipLaunchKernelGGL((gemv32_kernel<TPW, EPI, NORM, 256>), dim3(grid), dim3(NW * 64), smem, s, a);
    else if (NW <= 8)
      hipLaunchKernelGGL((gemv32_kernel<TPW, EPI, NORM, 512>), dim3(grid), dim3(NW * 64), smem, s, a);
    else
      hipLaunchKernelGGL((gemv32_kernel<TPW, EPI, NORM, 1024>), dim3(grid), dim3(NW * 64), smem, s, a);
  } else {
    if (NW <= 4)
      hipLaunchKernelGGL((gemv16_kernel<A, WK, TPW, EPI, NORM, 256, RS>), dim3(grid), dim3(NW * 64), smem, s, a);
    else if (NW <= 8)
      hipLaunchKernelGGL((gemv16_kernel<A, WK, TPW, EPI, NORM, 512, RS>), dim3(grid), dim3(NW * 64), smem, s, a);
    else
      hipLaunchKernelGGL((gemv16_kernel<A, WK, TPW, EPI, NORM, 1024, RS>), dim3(grid), dim3(NW * 64), smem, s, a);
  }
  return hipGetLastError();
}

template <int A, int WK>
hipError_t dispatch_epi(int epi, bool norm, const GemvArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE:
      return norm ? launch_one<A, WK, EPI_STORE, true>(a, s)
                  : launch_one<A, WK, EPI_STORE, false>(a, s);
    case EPI_RESID:
      return norm ? launch_one<A, WK, EPI_RESID, true>(a, s)
                  : launch_one<A, WK, EPI_RESID, false>(a, s);
    case EPI_SWIGLU:
      return norm ? launch_one<A, WK, EPI_SWIGLU, true>(a, s)
                  : launch_one<A, WK, EPI_SWIGLU, false>(a, s);
    case EPI_LOGITS:
      return norm ? launch_one<A, WK, EPI_LOGITS, true>(a, s)
                  : launch_one<A, WK, EPI_LOGITS, false>(a, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

#ifndef FMD_LOGITS_TPW
#define FMD_LOGITS_TPW 4
#endif
#ifndef FMD_LOGITS_PF
#define FMD_LOGITS_PF 0
#endif
constexpr int kLogitsTpw = FMD_LOGITS_TPW;
constexpr bool kLogitsPf = FMD_LOGITS_PF;

// Geometry of the 16-bit logits stream: one 16-row weight tile per group and
// the fewest groups per work-group (from a fixed menu) that keep the grid
// within two work-groups per CU, so every work-group is resident at once.
struct LogitsGeom {
  int ng, grid;
};
constexpr int kLogitsMaxGrid = 512;
LogitsGeom logits_geom(int out_rows) {
  const int ngroups = (out_rows / 16 + kLogitsTpw - 1) / kLogitsTpw;
  int ng = 1;
  for (int c : {1, 2, 4, 5, 8, 12, 16, 20, 24}) {
    ng = c;
    if ((ngroups + c - 1) / c <= kLogitsMaxGrid) break;
  }
  return {ng, (ngroups + ng - 1) / ng};
}

template <int A, int WK, int TPW, int NG>
hipError_t launch_logits_ng(const GemvArgs& a, int grid, hipStream_t s) {
  const int NW = a.W.in / 256;
  const size_t smem = sizeof(float) * (2 * NW * TPW * 256 + 16 * NW + NG * TPW * 256);
  if (NW <= 4)
    hipLaunchKernelGGL((logits16_kernel<A, WK, TPW, NG, 256, kLogitsPf>), dim3(grid), dim3(NW * 64), smem, s, a);
  else if (NW <= 8)
    hipLaunchKernelGGL((logits16_kernel<A, WK, TPW, NG, 512, kLogitsPf>), dim3(grid), dim3(NW * 64), smem, s, a);
  else
    hipLaunchKernelGGL((logits16_kernel<A, WK, TPW, NG, 1024, kLogitsPf>), dim3(grid), dim3(NW * 64), smem, s, a);
  return hipGetLastError();
}

// Tiles per wave of the lm_head stream: the fewest (from a fixed menu) that
// keep the grid within kLogitsMaxGrid work-groups of four waves (two per
// CU, all resident).  Measured at vocab 151936 (us per launch): at most 512
// work-groups with 2, 3 or 4 weight stages in flight per wave: 37.45, 36.88,
// 36.79; at most 768: 39.68 (2 stages), 45.21 (3); 1024: 40.28 (2), 42.84
// (3); 256: 48.11.  Deeper prefetch gains under 2%: two stages are kept.
constexpr int kLogitsStages = 2;
int logits_wave_nt(int out_rows) {
  const int ntiles = out_rows / 16;
  for (int c : {1, 2, 3, 4, 5, 6, 8, 10, 12}) {
    if ((ntiles + 4 * c - 1) / (4 * c) <= kLogitsMaxGrid) return c;
  }
  return 12;
}
int logits_wave_grid(int out_rows) {
  const int nt = logits_wave_nt(out_rows);
  return (out_rows / 16 + 4 * nt - 1) / (4 * nt);
}

template <int A, int WK, int NW, int NT>
hipError_t launch_logits_wave_nt(const GemvArgs& a, hipStream_t s) {
  constexpr int K = NW * 256;
  const size_t smem = sizeof(uint16_t) * 16 * (K + 8) + sizeof(float) * 4 * NT * 256;
  const dim3 grid(logits_wave_grid(a.W.out));
  hipLaunchKernelGGL((logits_wave_kernel<A, WK, NW, NT, kLogitsStages>), grid, dim3(256), smem, s, a);
  return hipGetLastError();
}

template <int A, int WK, int NW>
hipError_t launch_logits_wave(const GemvArgs& a, hipStream_t s) {
  switch (logits_wave_nt(a.W.out)) {
    case 1: return launch_logits_wave_nt<A, WK, NW, 1>(a, s);
    case 2: return launch_logits_wave_nt<A, WK, NW, 2>(a, s);
    case 3: return launch_logits_wave_nt<A, WK, NW, 3>(a, s);
    case 4: return launch_logits_wave_nt<A, WK, NW, 4>(a, s);
    case 5: return launch_logits_wave_nt<A, WK, NW, 5>(a, s);
    case 6: return launch_logits_wave_nt<A, WK, NW, 6>(a, s);
    case 8: return launch_logits_wave_nt<A, WK, NW, 8>(a, s);
    case 10: return launch_logits_wave_nt<A, WK, NW, 10>(a, s);
    case 12: return launch_logits_wave_nt<A, WK, NW, 12>(a, s);
  }
  return hipErrorInvalidValue;
}

template <int A, int WK>
hipError_t launch_logits16(const GemvArgs& a, hipStream_t s) {
  // hidden 512 and 1024 (K/8 >= 64 pieces per row for the norm's wave sums)
  if (a.W.in == 1024) return launch_logits_wave<A, WK, 4>(a, s);
  if (a.W.in == 512) return launch_logits_wave<A, WK, 2>(a, s);
  const LogitsGeom g = logits_geom(a.W.out);
  constexpr int T = kLogitsTpw;
  switch (g.ng) {
    case 1: return launch_logits_ng<A, WK, T, 1>(a, g.grid, s);
    case 2: return launch_logits_ng<A, WK, T, 2>(a, g.grid, s);
    case 4: return launch_logits_ng<A, WK, T, 4>(a, g.grid, s);
    case 5: return launch_logits_ng<A, WK, T, 5>(a, g.grid, s);
    case 8: return launch_logits_ng<A, WK, T, 8>(a, g.grid, s);
    case 12: return launch_logits_ng<A, WK, T, 12>(a, g.grid, s);
    case 16: return launch_logits_ng<A, WK, T, 16>(a, g.grid, s);
    case 20: return launch_logits_ng<A, WK, T, 20>(a, g.grid, s);
    case 24: return launch_logits_ng<A, WK, T, 24>(a, g.grid, s);
  }
  return hipErrorInvalidValue;
}

int gemv_logits_nparts(int act, bool q8, bool norm, int hidden, int out_rows) {
  if (act == ACT_F32 || !norm) {
    constexpr int TPW = tpw_of<EPI_LOGITS>();
    return (out_rows / 16 + TPW - 1) / TPW;
  }
  (void)q8;
  return hidden == 1024 || hidden == 512 ? logits_wave_grid(out_rows) : logits_geom(out_rows).grid;
}

hipError_t launch_gemv(int act, int epi, bool norm, const GemvArgs& a, hipStream_t s) {
  if (a.rows < 1 || a.rows > 16 || a.W.in % 256 || a.W.in > 4096 || a.W.out % 16 ||
      (epi == EPI_SWIGLU && a.W.out % 32))
    return hipErrorInvalidValue;
  if (epi == EPI_LOGITS && norm && act != ACT_F32) {
    if (a.W.kind == WK_Q8)
      return act == ACT_F16 ? launch_logits16<ACT_F16, WK_Q8>(a, s) : hipErrorInvalidValue;
    return act == ACT_F16 ? launch_logits16<ACT_F16, WK_DENSE>(a, s)
                          : launch_logits16<ACT_BF16, WK_DENSE>(a, s);
  }
  if (a.W.kind == WK_Q8) {
    if (act != ACT_F16) return hipErrorInvalidValue;
    return dispatch_epi<ACT_F16, WK_Q8>(epi, norm, a, s);
  }
  switch (act) {
    case ACT_F32: return dispatch_epi<ACT_F32, WK_DENSE>(epi, norm, a, s);
    case ACT_F16: return dispatch_epi<ACT_F16, WK_DENSE>(epi, norm, a, s);
    case ACT_BF16: return dispatch_epi<ACT_BF16, WK_DENSE>(epi, norm, a, s);
  }
  return hipErrorInvalidValue;
}
