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
template <int A, int EPI, int TPW>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs& p, float* red, uint64_t* keys,
                                              int NW) {
  typedef typename ActT<A>::T T;
  const int ntiles = p.W.out / 16;
  constexpr int NSLOT_OUT = (EPI == EPI_SWIGLU) ? TPW / 2 : TPW;
  for (int e = threadIdx.x; e < NSLOT_OUT * 256; e += blockDim.x) {
    const int jj = e >> 8, b = (e >> 4) & 15, n = e & 15;
    const int li = 16 * (b >> 2) + n, r = b & 3;
    auto slot_sum = [&](int j) {
      float s = 0.f;
      for (int ww = 0; ww < NW; ++ww) s += red[((ww * TPW + j) * 64 + li) * 4 + r];
      return s;
    };
    if constexpr (EPI == EPI_SWIGLU) {
      const int pair = blockIdx.x * (TPW / 2) + jj;
      if (pair >= ntiles / 2 || b >= p.rows) continue;
      const float g = rd<A>(slot_sum(2 * jj)), u = rd<A>(slot_sum(2 * jj + 1));
      const float s = rd<A>(g / (1.0f + __expf(-g)));
      ((T*)p.y)[(size_t)b * p.ldy + pair * 16 + n] = st_act<A>(s * u);
    } else {
      const int tile = blockIdx.x * TPW + jj;
      const bool ok = tile < ntiles && b < p.rows;
      const int col = tile * 16 + n;
      const float v = ok ? slot_sum(jj) : 0.f;
      if constexpr (EPI == EPI_STORE) {
        if (ok) ((T*)p.y)[(size_t)b * p.ldy + col] = st_act<A>(v);
      } else if constexpr (EPI == EPI_RESID) {
        if (ok) {
          const float res = ld_act<A>(((const T*)p.resid)[(size_t)b * p.ldy + col]);
          ((T*)p.y)[(size_t)b * p.ldy + col] = st_act<A>(res + rd<A>(v));
        }
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

// 16-bit activations (f16 / bf16) with dense 16-bit or Q8_0 weights.
template <int A, int WK, int TPW, int EPI, bool NORM, int MAXT>
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

  // Issue the weight loads first: they are the stream this kernel exists for.
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

  // A operand: this wave's 256-wide slice of the input rows.
  u32x4 xa[KBW];
  const uint16_t* x = (const uint16_t*)p.x;
  const int kbase = w * (KBW * 32);
#pragma unroll
  for (int i = 0; i < KBW; ++i) {
    const int k = kbase + 32 * i + 8 * kg;
    xa[i] = (row < p.rows) ? *(const u32x4*)(x + (size_t)row * p.ldx + k) : u32x4{0, 0, 0, 0};
  }
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
  gemv_epilogue<A, EPI, TPW>(p, red, keys, NW);
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
  gemv_epilogue<ACT_F32, EPI, TPW>(p, red, keys, NW);
}

template <int EPI> constexpr int tpw_of() {
  return EPI == EPI_SWIGLU ? 2 : (EPI == EPI_LOGITS ? 4 : 1);
}

template <int A, int WK, int EPI, bool NORM>
hipError_t launch_one(const GemvArgs& a, hipStream_t s) {
  constexpr int TPW = tpw_of<EPI>();
  const int NW = a.W.in / 256;
  const int ntiles = a.W.out / 16;
  const int units = (EPI == EPI_SWIGLU) ? ntiles / 2 : ntiles;
  const int per = (EPI == EPI_SWIGLU) ? TPW / 2 : TPW;
  const int grid = (units + per - 1) / per;
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
      hipLaunchKernelGGL((gemv16_kernel<A, WK, TPW, EPI, NORM, 256>), dim3(grid), dim3(NW * 64), smem, s, a);
    else if (NW <= 8)
      hipLaunchKernelGGL((gemv16_kernel<A, WK, TPW, EPI, NORM, 512>), dim3(grid), dim3(NW * 64), smem, s, a);
    else
      hipLaunchKernelGGL((gemv16_kernel<A, WK, TPW, EPI, NORM, 1024>), dim3(grid), dim3(NW * 64), smem, s, a);
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

int gemv_logits_nparts(int out_rows) {
  constexpr int TPW = tpw_of<EPI_LOGITS>();
  return (out_rows / 16 + TPW - 1) / TPW;
}

hipError_t launch_gemv(int act, int epi, bool norm, const GemvArgs& a, hipStream_t s) {
  if (a.rows < 1 || a.rows > 16 || a.W.in % 256 || a.W.in > 4096 || a.W.out % 16 ||
      (epi == EPI_SWIGLU && a.W.out % 32))
    return hipErrorInvalidValue;
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
