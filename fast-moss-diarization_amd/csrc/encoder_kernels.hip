// Kernels of the audio path: the Whisper encoder's convolution inputs,
// LayerNorm and dense bidirectional attention (whisper_encoder.rs:44-163) and
// the adaptor's LayerNorm (adaptor.rs:56-60).  The projections and both
// convolutions run on the MFMA GEMM (gemm.hip, EPI_AFFINE).
//
// Layout of a batch of W windows (T = frames / 2 positions each, T = 1500
// for 30 s of audio): every row-wise buffer holds W * (T + 1) rows, window w
// at rows [w (T + 1), w (T + 1) + T) and one spare row after it.  conv2 reads
// three consecutive conv1 output rows per position at a stride of two rows,
// so with conv1's output laid out as W * (2T + 2) rows (a zero row before and
// after each window's 2T frames), conv2 is a GEMM over rows at stride 2 d
// whose windows are (T + 1) rows apart -- no im2col copy; the spare row is
// computed and never stored.
#include <algorithm>
#include <type_traits>

#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

// ---------------------------------------------------------------------------
// conv1's input: the mel chunks cast to the activation dtype (the reference's
// `.to_dtype`, engine.rs:334-339) and laid out time-major, cp channels per
// row (n_mels zero-padded to cp), with a zero row before and after each
// window: row w (frames + 2) + 1 + f holds frame f.
template <int A>
__global__ void __launch_bounds__(256) mel_pack_kernel(const void* mel, int src_dtype, int windows,
                                                       int n_mels, int frames, int cp, void* out) {
  typedef typename ActT<A>::T T;
  const int64_t n = (int64_t)windows * (frames + 2) * cp;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % cp);
    const int64_t r = i / cp;
    const int w = (int)(r / (frames + 2)), f = (int)(r % (frames + 2)) - 1;
    float v = 0.f;
    if (c < n_mels && f >= 0 && f < frames) {
      const int64_t s = ((int64_t)w * n_mels + c) * frames + f;
      v = src_dtype == 0 ? ((const float*)mel)[s]
          : src_dtype == 1 ? f16_to_f32(((const uint16_t*)mel)[s])
                           : bf16_to_f32(((const uint16_t*)mel)[s]);
    }
    ((T*)out)[i] = st_act<A>(v);
  }
}

// A conv1d weight (cout, cin, 3) as the GEMM's (cout, 3 cinp) f32 rows:
// element (o, k cinp + c) = w[o][c][k] (zero for c >= cin), so that GEMM row
// t (three consecutive input rows t-1, t, t+1 of cinp channels) is the
// convolution at t.
__global__ void __launch_bounds__(256) conv_weight_kernel(const void* src, int src_dtype, int cout,
                                                          int cin, int cinp, float* dst) {
  const int64_t n = (int64_t)cout * 3 * cinp;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int o = (int)(i / (3 * cinp));
    const int rem = (int)(i % (3 * cinp));
    const int k = rem / cinp, c = rem % cinp;
    float v = 0.f;
    if (c < cin) {
      const int64_t s = ((int64_t)o * cin + c) * 3 + k;
      v = src_dtype == 0 ? ((const float*)src)[s]
          : src_dtype == 1 ? f16_to_f32(((const uint16_t*)src)[s])
                           : bf16_to_f32(((const uint16_t*)src)[s]);
    }
    dst[i] = v;
  }
}

// ---------------------------------------------------------------------------
// LayerNorm::forward (linear.rs:323-330): mean = sum(x)/n, var = sum((x -
// mean)^2)/n, y = rd((x - mean) * (1/sqrt(var + eps)) * w + b), f32
// arithmetic with the output products and sums rounded as written.
// 16-bit rows of NC * 512: one wave per row, x held in registers.
template <int A, int NC>
__global__ void __launch_bounds__(256) layernorm16_kernel(const void* xv, int ldx, const void* wv,
                                                          const void* bv, int rows, float eps,
                                                          void* yv, int ldy) {
  typedef typename ActT<A>::T T;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // whole waves leave together
  const T* x = (const T*)xv + (size_t)r * ldx;
  float v[NC][8];
#pragma unroll
  for (int i = 0; i < NC; ++i) unpack8<A>(*(const u32x4*)(x + (i * 64 + lane) * 8), v[i]);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i)
#pragma unroll
    for (int t = 0; t < 8; ++t) s += v[i][t];
  const float mean = __fdiv_rn(wave_sum(s), (float)(NC * 512));
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float dl = __fsub_rn(v[i][t], mean);
      ss = __fmaf_rn(dl, dl, ss);
    }
  const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(wave_sum(ss), (float)(NC * 512)), eps)));
  T* y = (T*)yv + (size_t)r * ldy;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    float g[8], b[8];
    unpack8<A>(*(const u32x4*)((const T*)wv + (i * 64 + lane) * 8), g);
    unpack8<A>(*(const u32x4*)((const T*)bv + (i * 64 + lane) * 8), b);
    uint32_t o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float y0 = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[i][2 * t], mean), rinv), g[2 * t]), b[2 * t]);
      const float y1 = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[i][2 * t + 1], mean), rinv), g[2 * t + 1]),
                                 b[2 * t + 1]);
      o[t] = (uint32_t)st_act<A>(y0) | ((uint32_t)st_act<A>(y1) << 16);
    }
    *(u32x4*)(y + (i * 64 + lane) * 8) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// Any width and dtype: one work-group per row.
template <int A>
__global__ void __launch_bounds__(256) layernorm_kernel(const void* xv, int ldx, const void* wv,
                                                        const void* bv, int dim, float eps, void* yv,
                                                        int ldy) {
  typedef typename ActT<A>::T T;
  __shared__ float part[4];
  const int r = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const T* x = (const T*)xv + (size_t)r * ldx;
  auto block_sum = [&](float v) {
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) part[w] = v;
    __syncthreads();
    return (part[0] + part[1]) + (part[2] + part[3]);
  };
  float s = 0.f;
  for (int i = threadIdx.x; i < dim; i += 256) s += ld_act<A>(x[i]);
  const float mean = __fdiv_rn(block_sum(s), (float)dim);
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += 256) {
    const float dl = __fsub_rn(ld_act<A>(x[i]), mean);
    ss = __fmaf_rn(dl, dl, ss);
  }
  const float rinv = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(block_sum(ss), (float)dim), eps)));
  T* y = (T*)yv + (size_t)r * ldy;
  for (int i = threadIdx.x; i < dim; i += 256)
    y[i] = st_act<A>(__fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(ld_act<A>(x[i]), mean), rinv),
                                         ld_act<A>(((const T*)wv)[i])),
                               ld_act<A>(((const T*)bv)[i])));
}

// ---------------------------------------------------------------------------
// Dense bidirectional attention of the encoder (whisper_encoder.rs:44-64) for
// head_dim 64: q and k arrive already scaled by head_dim^-1/4, so the scores
// are rd(q . k) with no further scale, the probabilities rd(exp(s - M) / S)
// with each row's global max M and sum S (softmax_last_dim returns the
// dtype), and the context rd(P V).  Rounding after normalisation needs M and
// S first, so each work-group visits its keys twice: pass 1 finds (M, S),
// pass 2 recomputes the scores and accumulates P V.
//
// One work-group per (64-query tile, head, window), four waves of 16 queries.
// Keys come in blocks of 64 (K, and in pass 2 V: 8 KiB each), copied global
// -> LDS by direct-to-LDS loads, double-buffered, the next block in flight
// while the current one is computed.  S^T = K Q^T puts keys on the MFMA's M
// side, so the f32 result already sits in the B-operand layout of P^T, and
// O^T += V^T P^T reads V^T from the row-major V block by LDS transpose reads.
//
// LDS rows are 128 bytes (64 dims), unpadded; the 16-byte chunk c of key row
// r sits at chunk position c ^ swk(r) (K) or c ^ swv(r) (V): the K fragment
// reads (16 rows, one chunk) and the transposed V reads (4 rows x 32 bytes per
// 16 lanes) then fall in distinct banks.
constexpr int EHD = 64;   // head_dim
constexpr int EKB = 64;   // keys per block
__device__ __forceinline__ int swk(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int swv(int r) { return ((r >> 1) & 3) << 1; }

template <int A>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (A == ACT_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two values rounded to the activation dtype and packed low | high.
template <int A>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (A == ACT_BF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  } else {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  }
}
template <int A>
__device__ __forceinline__ f32x2 unpack2(uint32_t v) {
  if constexpr (A == ACT_BF16) {
    return f32x2{__builtin_bit_cast(float, v << 16), __builtin_bit_cast(float, v & 0xffff0000u)};
  } else {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_convertvector(__builtin_bit_cast(f16x2, v), f32x2);
  }
}

constexpr float kLog2e = 1.4426950408889634f;

template <int A>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
enc_attn_kernel(EncAttnArgs p) {
  typedef typename ActT<A>::T T;
  constexpr int BLK = EKB * EHD;   // elements of one K or V block
  __shared__ __attribute__((aligned(1024))) uint16_t sK[2 * BLK];
  __shared__ __attribute__((aligned(1024))) uint16_t sV[2 * BLK];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int qr = lane & 15, kg = lane >> 4;
  // Work-groups go to the 8 XCDs round-robin by linear index; the grid is
  // read so that each XCD takes a contiguous eighth of the (query tile,
  // head, window) order -- all query tiles of a (head, window) on one XCD,
  // whose L2 then holds that head's K and V once (instead of every XCD
  // fetching them): audio path +1.0-1.3% in alternating pairs.
  const int nx = gridDim.x, ny = gridDim.y, nb = nx * ny * gridDim.z;
  const int id = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
  const int lid = nb % 8 == 0 ? (id & 7) * (nb >> 3) + (id >> 3) : id;
  const int h = (lid / nx) % ny;
  const size_t row0 = (size_t)(lid / (nx * ny)) * p.period;
  const uint16_t* base = (const uint16_t*)p.qkv + row0 * p.ld;
  const int q0 = (lid % nx) * 64 + 16 * w;
  const int nblk = (p.t + EKB - 1) / EKB;

  // Q^T fragments (B operand): query q0 + qr (rows past t read row t - 1;
  // their outputs are not stored), dims 32 ks + 8 kg .. + 7.
  u32x4 qf[2];
  {
    const int qrow = min(q0 + qr, p.t - 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      qf[ks] = *(const u32x4*)(base + (size_t)qrow * p.ld + h * EHD + ks * 32 + kg * 8);
  }

  // Block copies: 8 wave instructions of 1 KiB (8 key rows) per operand;
  // wave w issues instructions j = 2 w, 2 w + 1.  Lane l of instruction j
  // fetches row 8 j + l / 8 at the logical chunk stored at position l % 8.
  // Keys past t read key t - 1 (their scores are masked, p = 0).
  const int wu = __builtin_amdgcn_readfirstlane(w);
  int crow[2];
  uint32_t kch[2], vch[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int j = 2 * wu + i, rr = 8 * j + (lane >> 3), pc = lane & 7;
    crow[i] = rr;
    kch[i] = (uint32_t)(p.d + h * EHD + ((pc ^ swk(rr)) << 3)) * 2u;
    vch[i] = (uint32_t)(2 * p.d + h * EHD + ((pc ^ swv(rr)) << 3)) * 2u;
  }
  const uint32_t lk = lds_addr(sK), lv = lds_addr(sV);
  auto issue = [&](int blk, auto with_v_tag) {
    constexpr bool WV = decltype(with_v_tag)::value;
    const int k0 = blk * EKB;
    const uint32_t boff = (uint32_t)(blk & 1) * (BLK * 2);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t j = (uint32_t)(2 * wu + i);
      const uint32_t roff = (uint32_t)min(k0 + crow[i], p.t - 1) * (uint32_t)p.ld * 2u;
      lds_copy16(base, roff + kch[i], lk + boff + j * 1024u);
      if constexpr (WV) lds_copy16(base, roff + vch[i], lv + boff + j * 1024u);
    }
  };

  // Raw S^T of sub-block mt (keys 16 mt .. 16 mt + 15 of the block).
  auto qk = [&](const uint16_t* kb, int mt) {
    f32x4 sv = {0.f, 0.f, 0.f, 0.f};
    const int r = 16 * mt + qr;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4 ka = *(const u32x4*)&kb[r * EHD + (((4 * ks + kg) ^ swk(r)) << 3)];
      sv = mfma16<A>(ka, qf[ks], sv);
    }
    return sv;
  };
  // rd(q . k) in place; with MASKED (the last block, when t is not a
  // multiple of the block), keys at or past t become -inf.  The flag is a
  // compile-time one so that full blocks run without branches and their
  // four sub-blocks' products and roundings can interleave.
  auto round_mask = [&](f32x4& sv, int kbase, auto masked_tag) {
    if constexpr (A == ACT_BF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = rd<A>(sv[i]);   // one conversion each
    } else {
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const f32x2 v = unpack2<A>(pack2<A>(sv[i], sv[i + 1]));
        sv[i] = v.x;
        sv[i + 1] = v.y;
      }
    }
    if constexpr (decltype(masked_tag)::value) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (kbase + 4 * kg + i >= p.t) sv[i] = -INFINITY;
    }
  };

  // Pass 1: max and sum of exp of each query row (each lane covers 16 keys
  // of a block; the four lanes of a row merge at the end).
  float m = -INFINITY, l = 0.f;
  auto pass1_block = [&](int blk, auto masked_tag) {
    const uint16_t* kb = sK + (blk & 1) * BLK;
    f32x4 sv[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) sv[mt] = qk(kb, mt);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) round_mask(sv[mt], blk * EKB + 16 * mt, masked_tag);
    float bm = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) bm = fmaxf(bm, sv[mt][i]);
    const float mn = fmaxf(m, bm);
    const float ml2 = (mn == -INFINITY ? 0.f : mn) * kLog2e;
    float e = l * __builtin_amdgcn_exp2f(fmaf(m, kLog2e, -ml2));
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) e += __builtin_amdgcn_exp2f(fmaf(sv[mt][i], kLog2e, -ml2));
    m = mn;
    l = e;
  };
  issue(0, std::false_type{});
  for (int blk = 0; blk < nblk; ++blk) {
    wait_vm<0>();      // this block's copies (the only ones in flight) have landed
    barrier_lds();     // for every wave; and block blk - 1's buffer is free
    if (blk + 1 < nblk) issue(blk + 1, std::false_type{});
    if ((blk + 1) * EKB > p.t) pass1_block(blk, std::true_type{});
    else pass1_block(blk, std::false_type{});
  }
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const float mo = __shfl_xor(m, off), lo = __shfl_xor(l, off);
    const float mn = fmaxf(m, mo);
    const float mref = mn == -INFINITY ? 0.f : mn;
    l = l * __expf(m - mref) + lo * __expf(mo - mref);
    m = mn;
  }
  // exp(s - M) / S as one power of two, exp2(s log2 e - (M log2 e + log2 S)):
  // the division folds into the exponent's offset (one multiply less per
  // score; a few f32 ulps before the probability's rounding)
  const float mlog = fmaf(m == -INFINITY ? 0.f : m, kLog2e, __log2f(l > 0.f ? l : 1.f));
  barrier_lds();   // pass 1's last reads of the K buffers precede pass 2's copies

  // Pass 2: p = rd(exp(s - M) / S), O^T += V^T P^T.
  f32x4 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const int ts = lane & 15;
  auto pass2_block = [&](int blk, auto masked_tag) {
    const uint16_t* kb = sK + (blk & 1) * BLK;
    const uint16_t* vb = sV + (blk & 1) * BLK;
    f32x4 sv[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) sv[mt] = qk(kb, mt);
    uint32_t pp[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      round_mask(sv[mt], blk * EKB + 16 * mt, masked_tag);
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const float e0 = __builtin_amdgcn_exp2f(fmaf(sv[mt][i], kLog2e, -mlog));
        const float e1 = __builtin_amdgcn_exp2f(fmaf(sv[mt][i + 1], kLog2e, -mlog));
        pp[mt][i / 2] = pack2<A>(e0, e1);
      }
    }
    // keys 32 hb .. 32 hb + 31: k-slot s of lane group kg holds key 32 hb +
    // 4 kg + s (s < 4) or 32 hb + 16 + 4 kg + (s - 4), where S^T put them.
    // For the V^T operand (row = dim 16 dt + ts), lane ts supplies the
    // 64-bit row piece of key 32 hb + 4 kg + ts / 4 (+16 for the second
    // read) at dims 16 dt + 4 (ts % 4) .. + 3.
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const u32x4 pb = u32x4{pp[2 * hb][0], pp[2 * hb][1], pp[2 * hb + 1][0], pp[2 * hb + 1][1]};
      const int key1 = 32 * hb + 4 * kg + (ts >> 2);
      const int sw = swv(key1);   // = swv(key1 + 16)
      s16x4 r1[4], r2[4];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int e = (((2 * dt + ((ts & 3) >> 1)) ^ sw) << 3) + 4 * (ts & 1);
        r1[dt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + key1 * EHD + e));
        r2[dt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + (key1 + 16) * EHD + e));
      }
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const u32x4 va =
            __builtin_bit_cast(u32x4, __builtin_shufflevector(r1[dt], r2[dt], 0, 1, 2, 3, 4, 5, 6, 7));
        o[dt] = mfma16<A>(va, pb, o[dt]);
      }
    }
  };
  issue(0, std::true_type{});
  for (int blk = 0; blk < nblk; ++blk) {
    wait_vm<0>();
    barrier_lds();
    if (blk + 1 < nblk) issue(blk + 1, std::true_type{});
    if ((blk + 1) * EKB > p.t) pass2_block(blk, std::true_type{});
    else pass2_block(blk, std::false_type{});
  }
  // Context rd(O): lane holds dims 16 dt + 4 kg .. + 3 of query q0 + qr.
  if (q0 + qr < p.t) {
    T* out = (T*)p.out + (row0 + q0 + qr) * p.ldo + h * EHD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      *(uint2*)&out[16 * dt + 4 * kg] =
          uint2{pack2<A>(o[dt][0], o[dt][1]), pack2<A>(o[dt][2], o[dt][3])};
  }
}

// f32 activations: one wave per (query, head, window), lanes over keys, the
// same two passes; the P V sums are reduced across lanes through LDS.
__global__ void __launch_bounds__(64) enc_attn_f32_kernel(EncAttnArgs p) {
  __shared__ float red[64][EHD + 1];
  const int lane = threadIdx.x;
  const int q = blockIdx.x, h = blockIdx.y;
  const size_t row0 = (size_t)blockIdx.z * p.period;
  const float* base = (const float*)p.qkv + row0 * p.ld;
  float qv[EHD];
#pragma unroll
  for (int e = 0; e < EHD; ++e) qv[e] = base[(size_t)q * p.ld + h * EHD + e];
  auto score = [&](int j) {
    const float* k = base + (size_t)j * p.ld + p.d + h * EHD;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < EHD; ++e) s += qv[e] * k[e];
    return s;
  };
  float m = -INFINITY;
  for (int j = lane; j < p.t; j += 64) m = fmaxf(m, score(j));
  m = wave_max(m);
  float l = 0.f;
  for (int j = lane; j < p.t; j += 64) l += __expf(score(j) - m);
  l = wave_sum(l);
  const float inv = 1.f / l;
  float acc[EHD];
#pragma unroll
  for (int e = 0; e < EHD; ++e) acc[e] = 0.f;
  for (int j = lane; j < p.t; j += 64) {
    const float pj = __expf(score(j) - m) * inv;
    const float* v = base + (size_t)j * p.ld + 2 * p.d + h * EHD;
#pragma unroll
    for (int e = 0; e < EHD; ++e) acc[e] += pj * v[e];
  }
#pragma unroll
  for (int e = 0; e < EHD; ++e) red[lane][e] = acc[e];
  __syncthreads();
  float s = 0.f;
  for (int j = 0; j < 64; ++j) s += red[j][lane];
  ((float*)p.out)[(row0 + q) * p.ldo + h * EHD + lane] = s;
}

}  // namespace

hipError_t launch_mel_pack(int act, const void* mel, int src_dtype, int windows, int n_mels,
                           int frames, int cp, void* out, hipStream_t s) {
  const int64_t n = (int64_t)windows * (frames + 2) * cp;
  if (n <= 0) return hipSuccess;
  const int grid = (int)std::min<int64_t>((n + 255) / 256, 8192);
  switch (act) {
    case ACT_F32: hipLaunchKernelGGL(mel_pack_kernel<ACT_F32>, dim3(grid), dim3(256), 0, s, mel, src_dtype, windows, n_mels, frames, cp, out); break;
    case ACT_F16: hipLaunchKernelGGL(mel_pack_kernel<ACT_F16>, dim3(grid), dim3(256), 0, s, mel, src_dtype, windows, n_mels, frames, cp, out); break;
    case ACT_BF16: hipLaunchKernelGGL(mel_pack_kernel<ACT_BF16>, dim3(grid), dim3(256), 0, s, mel, src_dtype, windows, n_mels, frames, cp, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_conv_weight(const void* src, int src_dtype, int cout, int cin, int cinp,
                              float* dst, hipStream_t s) {
  const int64_t n = (int64_t)cout * 3 * cinp;
  if (n <= 0) return hipSuccess;
  const int grid = (int)std::min<int64_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(conv_weight_kernel, dim3(grid), dim3(256), 0, s, src, src_dtype, cout, cin,
                     cinp, dst);
  return hipGetLastError();
}

template <int A>
static hipError_t launch_ln16(const void* x, int ldx, const void* w, const void* b, int rows,
                              int dim, float eps, void* y, int ldy, hipStream_t s) {
  const dim3 grid((rows + 3) / 4);
  switch (dim / 512) {
    case 1: hipLaunchKernelGGL((layernorm16_kernel<A, 1>), grid, dim3(256), 0, s, x, ldx, w, b, rows, eps, y, ldy); break;
    case 2: hipLaunchKernelGGL((layernorm16_kernel<A, 2>), grid, dim3(256), 0, s, x, ldx, w, b, rows, eps, y, ldy); break;
    case 4: hipLaunchKernelGGL((layernorm16_kernel<A, 4>), grid, dim3(256), 0, s, x, ldx, w, b, rows, eps, y, ldy); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_layernorm(int act, const void* x, int ldx, const void* w, const void* b,
                            int rows, int dim, float eps, void* y, int ldy, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  const bool vec = dim % 512 == 0 && (dim == 512 || dim == 1024 || dim == 2048) && ldx % 8 == 0 &&
                   ldy % 8 == 0 &&
                   ((uintptr_t)x | (uintptr_t)y | (uintptr_t)w | (uintptr_t)b) % 16 == 0;
  if (vec && act == ACT_F16) return launch_ln16<ACT_F16>(x, ldx, w, b, rows, dim, eps, y, ldy, s);
  if (vec && act == ACT_BF16) return launch_ln16<ACT_BF16>(x, ldx, w, b, rows, dim, eps, y, ldy, s);
  switch (act) {
    case ACT_F32: hipLaunchKernelGGL(layernorm_kernel<ACT_F32>, dim3(rows), dim3(256), 0, s, x, ldx, w, b, dim, eps, y, ldy); break;
    case ACT_F16: hipLaunchKernelGGL(layernorm_kernel<ACT_F16>, dim3(rows), dim3(256), 0, s, x, ldx, w, b, dim, eps, y, ldy); break;
    case ACT_BF16: hipLaunchKernelGGL(layernorm_kernel<ACT_BF16>, dim3(rows), dim3(256), 0, s, x, ldx, w, b, dim, eps, y, ldy); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_enc_attn(int act, const EncAttnArgs& a, int heads, int windows, hipStream_t s) {
  if (windows <= 0 || a.t <= 0) return hipSuccess;
  if (heads <= 0 || a.d != heads * EHD || a.period < a.t || a.ld % 8 || a.ldo % 4)
    return hipErrorInvalidValue;
  switch (act) {
    case ACT_F32:
      hipLaunchKernelGGL(enc_attn_f32_kernel, dim3(a.t, heads, windows), dim3(64), 0, s, a);
      break;
    case ACT_F16:
      hipLaunchKernelGGL(enc_attn_kernel<ACT_F16>, dim3((a.t + 63) / 64, heads, windows), dim3(256), 0, s, a);
      break;
    case ACT_BF16:
      hipLaunchKernelGGL(enc_attn_kernel<ACT_BF16>, dim3((a.t + 63) / 64, heads, windows), dim3(256), 0, s, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
