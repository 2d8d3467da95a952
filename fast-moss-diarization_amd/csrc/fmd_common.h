// Shared device helpers for the gfx950 decoder kernels: element types, exact
// conversions, MFMA operand vectors and wavefront reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef uint16_t bf16_t;  // bfloat16 kept as raw bits in memory

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#include "fmd_kernels.h"

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
// Round-to-nearest-even f32 -> bf16: gfx950's v_cvt_pk_bf16_f32 (a
// branch-free single instruction; NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(f16, h);
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (f16)f);
}

// Storage element type per activation dtype.
template <int A> struct ActT;
template <> struct ActT<ACT_F32> { typedef float T; };
template <> struct ActT<ACT_F16> { typedef uint16_t T; };
template <> struct ActT<ACT_BF16> { typedef uint16_t T; };

template <int A> __device__ __forceinline__ float ld_act(const typename ActT<A>::T v);
template <> __device__ __forceinline__ float ld_act<ACT_F32>(float v) { return v; }
template <> __device__ __forceinline__ float ld_act<ACT_F16>(uint16_t v) { return f16_to_f32(v); }
template <> __device__ __forceinline__ float ld_act<ACT_BF16>(uint16_t v) { return bf16_to_f32(v); }

template <int A> __device__ __forceinline__ typename ActT<A>::T st_act(float v);
template <> __device__ __forceinline__ float st_act<ACT_F32>(float v) { return v; }
template <> __device__ __forceinline__ uint16_t st_act<ACT_F16>(float v) { return f32_to_f16(v); }
template <> __device__ __forceinline__ uint16_t st_act<ACT_BF16>(float v) { return f32_to_bf16(v); }

// Round a value to the activation dtype and widen it back (the reference
// stores every op's output in that dtype).
template <int A> __device__ __forceinline__ float rd(float v) { return ld_act<A>(st_act<A>(v)); }
// bf16: v_cvt_pk_bf16_f32 of (0, v) leaves bf16(v) in the high half over a
// zero low half, which is that value as an f32 -- one instruction where the
// conversion and the widening took two.  Same bits (round to nearest even).
template <> __device__ __forceinline__ float rd<ACT_BF16>(float v) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(float, __builtin_convertvector((f32x2_t){0.f, v}, bf16x2_t));
}

// Unpack 8 16-bit values held in a u32x4 to floats.
template <int A> __device__ __forceinline__ void unpack8(u32x4 w, float* o) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = ld_act<A>((uint16_t)(w[i] & 0xffffu));
    o[2 * i + 1] = ld_act<A>((uint16_t)(w[i] >> 16));
  }
}

// Reductions within 16-lane rows using DPP (all lanes of the row receive the
// result).  quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, row_half_mirror =
// 0x141, row_mirror = 0x140.
__device__ __forceinline__ float dpp_f(float v, int ctrl_dummy);
#define FMD_DPP(v, ctrl)                                                               \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), \
                                                        (ctrl), 0xf, 0xf, false))
__device__ __forceinline__ float row16_sum(float v) {
  v += FMD_DPP(v, 0xB1);
  v += FMD_DPP(v, 0x4E);
  v += FMD_DPP(v, 0x141);
  v += FMD_DPP(v, 0x140);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, FMD_DPP(v, 0xB1));
  v = fmaxf(v, FMD_DPP(v, 0x4E));
  v = fmaxf(v, FMD_DPP(v, 0x141));
  v = fmaxf(v, FMD_DPP(v, 0x140));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// RMSNorm over head_dim then rotate-half RoPE, for the 8 dims dc*8..dc*8+7
// held by this lane of a 16-lane row (the row holds the whole head); gain,
// cos and sin arrive already loaded.  The rotation partner of dim i is
// i +- 64, held by lane dc ^ 8.  Explicitly rounded operations keep the
// stored bits equal to a plain IEEE evaluation.
__device__ __forceinline__ float nr_rinv(const float* x, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) ss = __fadd_rn(ss, __fmul_rn(x[t], x[t]));
  ss = row16_sum(ss);
  return __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(ss, 128.0f), eps)));
}
template <int A>
__device__ __forceinline__ void norm_rope8(float* x, const float* g, const float* c,
                                           const float* s, int dc, float eps) {
  const float rinv = nr_rinv(x, eps);
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

// Exact int8 -> f16 for 4 packed signed bytes: bias each byte by 128, splice it
// under the exponent of 1024 (f16 0x6400 | u == 1024 + u) and subtract 1152.
__device__ __forceinline__ void i8x4_to_f16x4(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  // v_perm_b32 selector bytes: 0-3 pick from src1, 4-7 from src0.
  lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // [0x64,b1,0x64,b0]
  hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // [0x64,b3,0x64,b2]
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 bias = {(f16)1152.0f, (f16)1152.0f};
  lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, lo) - bias);
  hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, hi) - bias);
}

// Orderable 64-bit argmax key: larger value first, then the smaller index.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)b << 32) | (uint64_t)(0xffffffffu - idx);
}
__device__ __forceinline__ uint32_t argmax_key_index(uint64_t k) {
  return 0xffffffffu - (uint32_t)(k & 0xffffffffu);
}

// ---- direct global -> LDS copies (global_load_lds_dwordx4) ----

// One wave instruction: lane l's 16 bytes at gbase + goff land at LDS byte
// lds + 16 l (lds uniform across the wave).  Issued from asm so that the
// compiler, which cannot tell the ring stages apart, does not wait for every
// copy in flight before each LDS read; the loop's own vmcnt waits order the
// copies before the reads of their stage.  The LDS-DMA load reads M0 one
// wait state after it is written (the s_nop).  M0 is clobbered: the kernels
// that use this hold no value of their own in M0 (their code writes M0 only
// here), which is what the compiler's reserved-register warning is about.
// lds, gbase: wave-uniform; goff: per lane, gbase + goff 16-byte aligned.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_copy16(const void* gbase, uint32_t goff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds), "v"(goff), "s"(gbase) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Barrier ordering LDS accesses only: outstanding global copies keep flowing.
__device__ __forceinline__ void barrier_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// s_waitcnt vmcnt(N) (N < 64: low four bits at [3:0], high two at [15:14]).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
