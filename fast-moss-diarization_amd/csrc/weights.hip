// Load-time weight preparation: Q8_0 quantisation straight into the tiled
// MFMA layout, dense casts/packing, the inverse unpack to GGML block_q8_0
// bytes (for bit-exact checks), and synthetic fills.
#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

// Source element loads by source dtype code (0 f32, 1 f16, 2 bf16).
__device__ __forceinline__ float ld_src(const void* p, int dt, size_t i) {
  if (dt == 0) return ((const float*)p)[i];
  if (dt == 1) return f16_to_f32(((const uint16_t*)p)[i]);
  return bf16_to_f32(((const uint16_t*)p)[i]);
}

// QTensor::quantize(&w_f32, Q8_0) as reached from linear.rs:194-201 and
// 239-251.  Per 32-value block: amax = max|x| (f32), d = amax / 127 (f32,
// correctly rounded), id = d != 0 ? 1/d : 0, q = (i8) round-half-away(x*id)
// with a saturating cast (NaN -> 0), d stored as f16 (round to nearest even).
// One thread per block; output goes to the tiled layout of fmd_kernels.h.
__global__ void quantize_q8_0_tiles_kernel(const float* src, int rows, int cols, int row0,
                                           uint8_t* qs, uint32_t* sc) {
  const int nb = cols / 32;
  const int64_t id = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (id >= (int64_t)rows * nb) return;
  const int r = (int)(id / nb), j = (int)(id % nb);
  const float* xs = src + (size_t)r * cols + (size_t)j * 32;
  float v[32];
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    v[e] = xs[e];
    amax = fmaxf(amax, fabsf(v[e]));
  }
  const float d = __fdiv_rn(amax, 127.0f);
  const float inv = (d != 0.f) ? __fdiv_rn(1.0f, d) : 0.f;
  const int n = row0 + r, t = n >> 4, rr = n & 15;
  const int KC = cols / 64, c = j >> 1, half = j & 1;
  uint8_t* chunk = qs + ((size_t)t * KC + c) * 1024;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const float qv = roundf(__fmul_rn(v[e], inv));
    int8_t q;
    if (qv != qv) q = 0;
    else if (qv >= 127.f) q = 127;
    else if (qv <= -128.f) q = -128;
    else q = (int8_t)qv;
    const int lane = rr + 16 * (e >> 3);
    chunk[lane * 16 + half * 8 + (e & 7)] = (uint8_t)q;
  }
  ((uint16_t*)sc)[(((size_t)t * KC + c) * 16 + rr) * 2 + half] = f32_to_f16(d);
}

// Inverse of the tiled Q8_0 layout: rows [row0, row0+rows) as 34-byte blocks.
__global__ void unpack_q8_0_kernel(const uint8_t* qs, const uint32_t* sc, int cols, int row0,
                                   int rows, uint8_t* out) {
  const int nb = cols / 32;
  const int64_t id = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (id >= (int64_t)rows * nb) return;
  const int r = (int)(id / nb), j = (int)(id % nb);
  const int n = row0 + r, t = n >> 4, rr = n & 15;
  const int KC = cols / 64, c = j >> 1, half = j & 1;
  const uint8_t* chunk = qs + ((size_t)t * KC + c) * 1024;
  uint8_t* blk = out + ((size_t)r * nb + j) * 34;
  const uint16_t d = ((const uint16_t*)sc)[(((size_t)t * KC + c) * 16 + rr) * 2 + half];
  blk[0] = (uint8_t)(d & 0xff);
  blk[1] = (uint8_t)(d >> 8);
  for (int e = 0; e < 32; ++e) blk[2 + e] = chunk[(rr + 16 * (e >> 3)) * 16 + half * 8 + (e & 7)];
}

// Dense weights: cast to the activation dtype (round to nearest even) and
// scatter into the tiled layout.
template <int A>
__global__ void pack_dense_kernel(const void* src, int sdt, int rows, int cols, int row0,
                                  uint8_t* wt) {
  const int64_t id = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (id >= (int64_t)rows * cols) return;
  const int r = (int)(id / cols), k = (int)(id % cols);
  const float v = ld_src(src, sdt, id);
  const int n = row0 + r, t = n >> 4, rr = n & 15;
  if constexpr (A == ACT_F32) {
    const int c = k >> 4, e = k & 15;
    const size_t o = (((size_t)t * (cols / 16) + c) * 64 + rr + 16 * (e >> 2)) * 4 + (e & 3);
    ((float*)wt)[o] = v;
  } else {
    const int kb = k >> 5, e = k & 31;
    const size_t o = (((size_t)t * (cols / 32) + kb) * 64 + rr + 16 * (e >> 3)) * 8 + (e & 7);
    ((uint16_t*)wt)[o] = st_act<A>(v);
  }
}

template <int A>
__global__ void convert_kernel(const void* src, int sdt, int64_t n, void* dst) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    ((typename ActT<A>::T*)dst)[i] = st_act<A>(ld_src(src, sdt, i));
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

// Synthetic N(0, std^2) fill (Box-Muller on a counter-based SplitMix64 stream).
template <int A>
__global__ void fill_normal_kernel(void* dst, int64_t n, uint64_t seed, float stdv) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t r = splitmix64(seed * 0x632be59bd9b4e019ull + (uint64_t)i);
    const float u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777217.0f);
    const float u2 = (float)((r >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
    const float z = sqrtf(-2.0f * __logf(u1)) * __cosf(6.28318530718f * u2);
    ((typename ActT<A>::T*)dst)[i] = st_act<A>(stdv * z);
  }
}

inline int grid_for(int64_t n, int block) {
  int64_t g = (n + block - 1) / block;
  return (int)(g > 65535 ? 65535 : (g < 1 ? 1 : g));
}

}  // namespace

hipError_t launch_quantize_q8_0_tiles(const float* src, int rows, int cols, int row0,
                                      LinWeights W, hipStream_t s) {
  if (cols % 64 || row0 % 16 || W.kind != WK_Q8) return hipErrorInvalidValue;
  const int64_t n = (int64_t)rows * (cols / 32);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(quantize_q8_0_tiles_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     s, src, rows, cols, row0, W.w, W.sc);
  return hipGetLastError();
}

hipError_t launch_unpack_q8_0(LinWeights W, int row0, int rows, uint8_t* out, hipStream_t s) {
  const int64_t n = (int64_t)rows * (W.in / 32);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(unpack_q8_0_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, W.w,
                     W.sc, W.in, row0, rows, out);
  return hipGetLastError();
}

hipError_t launch_pack_dense(int act, const void* src, int src_dtype, int rows, int cols,
                             int row0, LinWeights W, hipStream_t s) {
  if (row0 % 16 || W.kind != WK_DENSE) return hipErrorInvalidValue;
  const int64_t n = (int64_t)rows * cols;
  if (n == 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256));
  switch (act) {
    case ACT_F32: hipLaunchKernelGGL(pack_dense_kernel<ACT_F32>, grid, dim3(256), 0, s, src, src_dtype, rows, cols, row0, W.w); break;
    case ACT_F16: hipLaunchKernelGGL(pack_dense_kernel<ACT_F16>, grid, dim3(256), 0, s, src, src_dtype, rows, cols, row0, W.w); break;
    case ACT_BF16: hipLaunchKernelGGL(pack_dense_kernel<ACT_BF16>, grid, dim3(256), 0, s, src, src_dtype, rows, cols, row0, W.w); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_convert(int act, const void* src, int src_dtype, int64_t n, void* dst,
                          hipStream_t s) {
  if (n == 0) return hipSuccess;
  const dim3 grid(grid_for(n, 256));
  switch (act) {
    case ACT_F32: hipLaunchKernelGGL(convert_kernel<ACT_F32>, grid, dim3(256), 0, s, src, src_dtype, n, dst); break;
    case ACT_F16: hipLaunchKernelGGL(convert_kernel<ACT_F16>, grid, dim3(256), 0, s, src, src_dtype, n, dst); break;
    case ACT_BF16: hipLaunchKernelGGL(convert_kernel<ACT_BF16>, grid, dim3(256), 0, s, src, src_dtype, n, dst); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_fill_normal(int act, void* dst, int64_t n, uint64_t seed, float stdv,
                              hipStream_t s) {
  if (n == 0) return hipSuccess;
  const dim3 grid(grid_for(n, 256));
  switch (act) {
    case ACT_F32: hipLaunchKernelGGL(fill_normal_kernel<ACT_F32>, grid, dim3(256), 0, s, dst, n, seed, stdv); break;
    case ACT_F16: hipLaunchKernelGGL(fill_normal_kernel<ACT_F16>, grid, dim3(256), 0, s, dst, n, seed, stdv); break;
    case ACT_BF16: hipLaunchKernelGGL(fill_normal_kernel<ACT_BF16>, grid, dim3(256), 0, s, dst, n, seed, stdv); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
