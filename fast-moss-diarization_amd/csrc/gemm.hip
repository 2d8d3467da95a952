// Prefill projections: Y = X W^T for many rows on the MFMA units.
//
// Block tiles of 64, 128 or 256 rows x 128 weight rows, four waves in a 2x2
// arrangement, MFMA 16x16x32, B fragments from the tiled weight layout
// shared with the decode GEMV (one 16-byte piece per lane per 16x32
// fragment):
// - dense 16-bit weights (gemm_dma_kernel, 64, 128 or 256 rows): both
//   operands go global -> LDS by direct-to-LDS loads through a ring of 32-k
//   stages; waves hold 32 x 64, 64 x 64 or 128 x 64.
// - 64 rows (gemm16_kernel), for the smallest grids and for Q8_0: K step 64,
//   X staged global -> registers -> LDS, double-buffered
//   with one barrier per K step (row pitch padded to 72 elements so the
//   MFMA-order 16-byte reads are bank-conflict free); dense weights take the
//   same route, Q8_0 fragments are read straight from global memory one K
//   step ahead; waves hold 32 x 64.
// Every global load is unconditional (out-of-range rows and tiles read
// clamped addresses), so no wait depends on a branch.  Work-groups are
// mapped to tiles over an XCD grid chosen per shape (see tile_of).  Q8_0
// weights are converted to f16 exactly and each 32-wide block's partial
// product is scaled by its f16 scale in f32.
//
// Reference: Linear::forward / FusedLinear::forward (linear.rs:29-100) over
// (b*t, in) rows; call sites qwen3.rs:213, 258, 288-291.
#include <cstdlib>
#include <type_traits>

#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

constexpr int BM = 128, BK = 64, LDA = BK + 8;

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

// 16-byte load at a byte offset (< 4 GiB) from a work-group-uniform base: one
// 32-bit offset register per load instead of 64-bit address arithmetic.
__device__ __forceinline__ u32x4 ld16(const void* ubase, uint32_t byte_off) {
  return *(const u32x4*)((const char*)ubase + byte_off);
}
__device__ __forceinline__ uint32_t ld4(const void* ubase, uint32_t byte_off) {
  return *(const uint32_t*)((const char*)ubase + byte_off);
}

// Weight n-tile handled by a wave's ni-th fragment column in column group cg.
template <int EPI>
__device__ __forceinline__ int wave_tile(int cg, int ntiles, int wn, int ni) {
  if constexpr (EPI == EPI_SWIGLU) {
    const int base = cg * 4 + wn * 2 + (ni & 1);
    return ni < 2 ? base : base + ntiles / 2;
  } else {
    return cg * 8 + wn * 4 + ni;
  }
}

// Row tile mt and column group cg of work-group id.  Work-groups are dealt
// to the 8 XCDs round-robin (id % 8), each XCD with its own L2.  The XCDs
// form an a x (8/a) grid over (row tiles x column groups): XCD x takes the
// row-tile block x / (8/a) and the column-group block x % (8/a), so the X
// rows are fetched by 8/a XCDs and each weight tile by a of them (a is
// chosen per shape by the host to minimise that traffic).  The grid holds
// 8 * Ma * Cb work-groups (Ma = ceil(mtiles / a), Cb = cols / (8/a));
// those past the last row tile return at once (mt >= mtiles).
__device__ __forceinline__ void tile_of(int id, int mtiles, int cols, int a, int& mt, int& cg) {
  const int b = 8 / a, x = id & 7, j = id >> 3;
  const int Ma = (mtiles + a - 1) / a, Cb = cols / b;
  if (Cb < 16) {
    mt = (x / b) * Ma + j / Cb;
    cg = (x % b) * Cb + j % Cb;
    return;
  }
  // A wide block (16 or more column groups): groups of GM row tiles with the
  // row tile fastest, so that an XCD's concurrent work-groups (about 64)
  // span GM row tiles x 64/GM column groups, whose X and weight tiles fit
  // its L2 better than 64/Cb row tiles x all Cb column groups (audio path
  // q|k|v and fc1 at 24,016 rows: 439.5 -> 449.8 windows/s with GM = 8;
  // GM = 16 another +0.6-0.8%, q|k|v 178 -> 171 us; 4 and 32 no better,
  // grouping blocks of 8 column groups too slower; prefill unchanged).
  constexpr int GM = 16;
  const int g = j / (GM * Cb), r = j - g * (GM * Cb);
  const int gm = min(GM, Ma - g * GM);
  mt = (x / b) * Ma + g * GM + r % gm;
  cg = (x % b) * Cb + r / gm;
}

// EPI_ROPE: the work-group's 128 columns are head slot cg of q|k|v, and the
// tile (64 or 128 rows) goes on through Attention::forward's q/k RMSNorm,
// RoPE and KvCache::append (qwen3.rs:214-227, 139-144, 86-101) instead of
// being stored.  Its rounded products (rd(x W^T), qwen3.rs:213) are staged
// in LDS, chunk c of row r at chunk position c ^ rope_sw(r), so that the
// 2-byte stores of a wave's four 16-lane groups (rows 4 apart) fall in
// distinct banks; then each 16-lane group finishes
// rows gi, gi + 16, ... (8 dims per lane): q and k heads through norm_rope8,
// the decode attention's routine for the new token (so prefill and decode
// store the same bits for a token), into q_out or the K cache, v heads as
// projected into the V cache.
__device__ __forceinline__ int rope_sw(int r) { return ((r >> 2) & 3) << 1; }

// Position and batch index (pos * 16 + b: b < 16, the prefill batch bound)
// of the rows gi + 16 j (j < BMT / 16) of the tile that this thread's 16-lane
// group finishes, loaded before the K loop; rows past M read row M - 1's
// (they are not stored).
template <int BMT>
struct RopeRows {
  int pb[BMT / 16];
};

template <int BMT>
__device__ __forceinline__ RopeRows<BMT> rope_rows(const GemmArgs& p, int m0) {
  RopeRows<BMT> rr;
  const int gi = threadIdx.x >> 4;
#pragma unroll
  for (int j = 0; j < BMT / 16; ++j) {
    const int gr = min(m0 + gi + 16 * j, p.M - 1);
    rr.pb[j] = p.rope.row_pos[gr] * 16 + p.rope.row_b[gr];
  }
  return rr;
}

// acc: the wave's BMT/2 x 64 accumulators (2 x 2 waves, as the epilogues
// below); stg: BMT x 128 activations of LDS, free once the caller's K loop
// has ended.
template <int A, int BMT, int MI>
__device__ __forceinline__ void rope_epilogue(const GemmArgs& p, const f32x4 (&acc)[MI][4],
                                              typename ActT<A>::T* stg, int m0, int cg,
                                              const RopeRows<BMT>& rr) {
  static_assert(BMT == 64 || BMT == 128, "rope tiles");
  typedef typename ActT<A>::T T;
  constexpr int NJ = BMT / 16;   // rows per 16-lane group
  const RopeArgs& q = p.rope;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1;
  const int row = lane & 15, kg = lane >> 4;
  const int dc = threadIdx.x & 15, gi = threadIdx.x >> 4;
  const int slot = cg;
  const bool is_q = slot < q.nh, is_v = slot >= q.nh + q.nkv;
  float g[8];
  u32x4 cr[NJ], sr[NJ];
  if (!is_v) {
    // gain and cos / sin rows, in flight while the tile is staged
    unpack8<A>(*(const u32x4*)((const T*)(is_q ? q.qn_w : q.kn_w) + dc * 8), g);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const size_t o = (size_t)(rr.pb[j] >> 4) * 64 + (dc & 7) * 8;
      cr[j] = *(const u32x4*)((const T*)q.cos + o);
      sr[j] = *(const u32x4*)((const T*)q.sin + o);
    }
  }
  barrier_lds();   // every wave is done with the K loop's LDS
  // The rows this lane writes are 4 kg + (a multiple of 4) + r, r < 4, so
  // their rope_sw is 2 kg and column wn*64 + ni*16 + row lands at wn*64 +
  // (ni ^ kg)*16 + row.
  T* const wb = stg + (wm * (BMT / 2) + 4 * kg) * 128 + wn * 64 + row;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) wb[(mi * 16 + r) * 128 + (ni ^ kg) * 16] = st_act<A>(acc[mi][ni][r]);
  barrier_lds();
  // rows gi + 16 j: rope_sw(gi + 16 j) = rope_sw(gi)
  const T* const rb = stg + gi * 128 + ((dc ^ rope_sw(gi)) << 3);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int gr = m0 + gi + 16 * j;
    // a whole 16-lane group leaves together (norm_rope8 reads its lanes)
    if (gr >= p.M) break;
    const u32x4 raw = *(const u32x4*)(rb + j * 16 * 128);
    const int b = rr.pb[j] & 15, pos = rr.pb[j] >> 4;
    if (is_v) {
      T* dst = (T*)q.vc + (((size_t)b * q.nkv + (slot - q.nh - q.nkv)) * q.cap + pos) * 128;
      *(u32x4*)(dst + dc * 8) = raw;
      continue;
    }
    float x[8], c[8], sn[8];
    unpack8<A>(raw, x);
    unpack8<A>(cr[j], c);
    unpack8<A>(sr[j], sn);
    norm_rope8<A>(x, g, c, sn, dc, q.eps);
    uint32_t o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      o[t] = (uint32_t)st_act<A>(x[2 * t]) | ((uint32_t)st_act<A>(x[2 * t + 1]) << 16);
    T* dst = is_q ? (T*)q.q_out + ((size_t)gr * q.nh + slot) * 128
                  : (T*)q.kc + (((size_t)b * q.nkv + (slot - q.nh)) * q.cap + pos) * 128;
    *(u32x4*)(dst + dc * 8) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// GELU-erf, 0.5 v (1 + erf(v / sqrt 2)), branch-free, from Abramowitz &
// Stegun 7.1.26: erfc(x) ~ t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-x^2)
// with t = 1 / (1 + p x), |error| <= 1.5e-7 for x >= 0.  With
// h = erfc(|v| / sqrt 2) / 2, the GELU is max(v, 0) - |v| h for either sign
// of v (v - v h for v > 0, v h for v < 0: no cancellation for negative v),
// one fma.  1/sqrt 2 is folded into p, 1/2 into the a_k (exact), and
// exp(-v^2 / 2) is exp2(v (v (-log2(e) / 2))).  The device erff branches on
// the size of its argument, which diverges within a wave.
__device__ __forceinline__ float gelu_erf(float v) {
  constexpr float kP = 0.3275911f;
  constexpr float kA1 = 0.254829592f, kA2 = -0.284496736f, kA3 = 1.421413741f,
                  kA4 = -1.453152027f, kA5 = 1.061405429f;
  constexpr float kRsqrt2 = 0.70710678118654752f, kE = -0.72134752044448170f;
  const float av = fabsf(v);
  const float t = __builtin_amdgcn_rcpf(fmaf(kP * kRsqrt2, av, 1.0f));
  const float poly =
      t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, 0.5f * kA5, 0.5f * kA4), 0.5f * kA3), 0.5f * kA2), 0.5f * kA1);
  const float h = poly * __builtin_amdgcn_exp2f(v * (v * kE));
  // max(v, 0) as one v_max_f32 (fmaxf adds a canonicalising max(v, v) per
  // element; a NaN v makes h NaN, so the result is NaN either way)
  float pos;
  asm("v_max_f32 %0, 0, %1" : "=v"(pos) : "v"(v));
  return fmaf(-av, h, pos);
}

// EPI_AFFINE for an output element from its f32 accumulator (the steps and
// their rounding as AffineArgs states), given the element's bias, residual
// and table values (each used only when its pointer is set).
template <int A>
__device__ __forceinline__ float affine_steps(const GemmArgs& p, float acc, int col, float bias,
                                              float resid, float table) {
  const AffineArgs& f = p.aff;
  float v = rd<A>(acc);
  if (f.bias) v = rd<A>(v + bias);
  if (col < f.scale_cols) v = rd<A>(v * f.scale);
  if (f.act == 1) v = rd<A>(gelu_erf(v));
  else if (f.act == 2) v = rd<A>(v / (1.0f + __expf(-v)));
  if (p.resid) v = rd<A>(resid + v);
  if (f.table) v = rd<A>(v + table);
  return v;
}
// affine_steps over N elements at once, step by step: the same operations
// in the same order for each element, but every step's uniform branch is
// taken once for the block, so the elements' chains are independent
// instructions the compiler can interleave (element by element, each step
// sat in its own basic block and only one chain was in flight).
// Inputs already rounded to the dtype (ROUNDED) skip the first rounding.
// The scale step multiplies each element by its scl (f.scale for the
// scaled columns, 1 for the others: rd(v * 1) = v for a rounded v), so it
// needs no per-element select.  The residual and table values arrive as
// stored (rv, tv) and are widened inside their steps, so the wait for their
// loads falls after the steps that do not need them.
template <int A, int N, bool ROUNDED>
__device__ __forceinline__ void affine_block(const GemmArgs& p, float (&v)[N], const float (&scl)[N],
                                             const float (&bias)[N],
                                             const typename ActT<A>::T (&rv)[N],
                                             const typename ActT<A>::T (&tv)[N]) {
  const AffineArgs& f = p.aff;
  if constexpr (!ROUNDED) {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = rd<A>(v[e]);
  }
  if (f.bias) {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = rd<A>(v[e] + bias[e]);
  }
  if (f.scale_cols > 0) {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = rd<A>(v[e] * scl[e]);
  }
  if (f.act == 1) {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = rd<A>(gelu_erf(v[e]));
  } else if (f.act == 2) {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = rd<A>(v[e] / (1.0f + __expf(-v[e])));
  }
  if (p.resid) {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = rd<A>(ld_act<A>(rv[e]) + v[e]);
  }
  if (f.table) {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = rd<A>(v[e] + ld_act<A>(tv[e]));
  }
}

// The same for output element (gr, col), loading its values.
template <int A>
__device__ __forceinline__ float affine_value(const GemmArgs& p, float acc, int gr, int col) {
  typedef typename ActT<A>::T T;
  const AffineArgs& f = p.aff;
  const float bias = f.bias ? ld_act<A>(((const T*)f.bias)[col]) : 0.f;
  const float resid = p.resid ? ld_act<A>(((const T*)p.resid)[(size_t)gr * p.ldy + col]) : 0.f;
  const float table = f.table ? ld_act<A>(((const T*)f.table)[(size_t)(gr % f.period) * p.W.out + col]) : 0.f;
  return affine_steps<A>(p, acc, col, bias, resid, table);
}
// Whether output row gr is stored (EPI_AFFINE skips the rows between windows).
__device__ __forceinline__ bool affine_row(const GemmArgs& p, int gr) {
  return p.aff.period <= 0 || gr % p.aff.period < p.aff.valid;
}

// EPI_RESID: the residual of every output element a lane stores (rows
// 4 kg + r of each 16-row fragment, column `row` of tile[ni]), loaded before
// the K loop so that these scattered 2-byte loads are in flight behind it
// instead of exposed in the epilogue.  Rows past M and tiles past the end
// read clamped addresses (they are not stored).  MI is 2 or 4: the 64- and
// 128-row tiles.
template <int A, int MI>
struct ResidRows {
  typename ActT<A>::T v[MI][4][4];
};

template <int A, int BMT, int MI>
__device__ __forceinline__ ResidRows<A, MI> load_resid(const GemmArgs& p, int m0, const int (&tile)[4],
                                                       const bool (&tv)[4]) {
  typedef typename ActT<A>::T T;
  ResidRows<A, MI> rr;
  const int lane = threadIdx.x & 63, wm = (threadIdx.x >> 6) >> 1;
  const int row = lane & 15, kg = lane >> 4;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int gr = min(m0 + wm * (BMT / 2) + mi * 16 + 4 * kg + r, p.M - 1);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        rr.v[mi][r][ni] = ((const T*)p.resid)[(size_t)gr * p.ldy + (tv[ni] ? tile[ni] : 0) * 16 + row];
    }
  return rr;
}

// EPI_SWIGLU epilogue (Mlp::forward's silu(gate) * up, qwen3.rs:288-291):
// tiles 0, 1 of the wave hold gate columns, tiles 2, 3 the matching up
// columns.  Each 16-row fragment's eight products are computed before any
// of them is stored -- rd(gate), rd(up), rd(silu(gate)), rd(s * u) in that
// order per element -- with no branch between them, so their chains (an
// exponential and a division each) interleave; the row and tile checks
// only guard the stores.
template <int A, int BMT, int MI>
__device__ __forceinline__ void swiglu_epilogue(const GemmArgs& p, const f32x4 (&acc)[MI][4], int m0,
                                                const int (&tile)[4], const bool (&tv)[4]) {
  typedef typename ActT<A>::T T;
  const int lane = threadIdx.x & 63, wm = (threadIdx.x >> 6) >> 1;
  const int row = lane & 15, kg = lane >> 4;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    float o[4][2];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const float gg = rd<A>(acc[mi][ni][r]), u = rd<A>(acc[mi][ni + 2][r]);
        o[r][ni] = rd<A>(gg / (1.0f + __expf(-gg))) * u;
      }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int gr = m0 + wm * (BMT / 2) + mi * 16 + 4 * kg + r;
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
        if (gr < p.M && tv[ni]) ((T*)p.y)[(size_t)gr * p.ldy + tile[ni] * 16 + row] = st_act<A>(o[r][ni]);
    }
  }
}

// EPI_SWIGLU on the direct-to-LDS tiles with 16-byte stores: the same
// products as swiglu_epilogue, staged row-major in the freed ring (BMT rows
// x the work-group's 64 output columns; 16-byte chunk c of row R at position
// c ^ rope_sw(R), so the four 16-lane groups' writes and the row reads are
// bank-conflict-free), then 8 lanes per row store 8 columns each.
template <int A, int BMT, int MI>
__device__ __forceinline__ void swiglu_staged_epilogue(const GemmArgs& p, const f32x4 (&acc)[MI][4], int m0,
                                                       int cg, uint16_t* stg) {
  typedef typename ActT<A>::T T;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1, row = lane & 15, kg = lane >> 4;
  barrier_lds();   // every wave's last fragment reads are done
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    float o[4][2];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const float gg = rd<A>(acc[mi][ni][r]), u = rd<A>(acc[mi][ni + 2][r]);
        o[r][ni] = rd<A>(gg / (1.0f + __expf(-gg))) * u;
      }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int R = wm * (BMT / 2) + mi * 16 + 4 * kg + r;
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const int C = (wn * 2 + ni) * 16 + row;
        stg[R * 64 + ((((C >> 3) ^ rope_sw(R)) << 3) | (C & 7))] = st_act<A>(o[r][ni]);
      }
    }
  }
  barrier_lds();
  const int ch = threadIdx.x & 7, r0 = threadIdx.x >> 3;    // chunk, first row
  const int gc = cg * 64 + ch * 8;                           // its first output column
  if (gc >= p.W.out / 2) return;                             // (no barrier follows)
  const int rows = min(BMT, p.M - m0);
  T* const y = (T*)p.y + (size_t)m0 * p.ldy + gc;
  for (int R = r0; R < rows; R += 32)
    *(u32x4*)(y + (size_t)R * p.ldy) = *(const u32x4*)&stg[R * 64 + ((ch ^ rope_sw(R)) << 3)];
}

// LB: the work-group's weight block (8 tiles x 64 k) is staged through LDS
// like X, so each weight byte is fetched once per work-group instead of once
// per wave column (dense weights only).
template <int A, int WK, int EPI, int BMT, bool LB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
gemm16_kernel(GemmArgs p) {
  typedef typename ActT<A>::T T;
  static_assert(!LB || WK == WK_DENSE, "LDS-staged weights are dense only");
  constexpr int MI = BMT / 32;   // 16-row fragments per wave (waves are 2 x 2)
  constexpr int NA = BMT / 32;   // 16-byte pieces of the X tile per thread
  __shared__ uint16_t sA[2 * BMT * LDA];
  // [buffer][local tile 0..7][chunk 0..1][64 lanes][8], B-operand lane order
  __shared__ uint16_t sB[LB ? 2 * 8 * 2 * 512 : 1];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int K = p.W.in, ntiles = p.W.out / 16;
  const int cols = EPI == EPI_SWIGLU ? (ntiles / 2 + 3) / 4 : (ntiles + 7) / 8;
  int mt, cg;
  tile_of(blockIdx.x, (p.M + BMT - 1) / BMT, cols, p.map, mt, cg);
  if (mt * BMT >= p.M) return;   // padding of the last row-tile block
  const int m0 = mt * BMT;
  const int row = lane & 15, kg = lane >> 4;
  [[maybe_unused]] RopeRows<EPI == EPI_ROPE ? BMT : 16> rrows;
  if constexpr (EPI == EPI_ROPE) rrows = rope_rows<BMT>(p, m0);

  // Every global load below is unconditional (a branch around a load makes
  // the compiler wait for all outstanding loads at the next join, which
  // serialises the prefetch): rows past M read row M - 1 and weight tiles
  // past the end read the last tile.  Each output depends only on its own X
  // row and weight tile, and those outputs are never stored.
  int tile[4], ltile[4];
  bool tv[4];
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    tile[ni] = wave_tile<EPI>(cg, ntiles, wn, ni);
    tv[ni] = (EPI == EPI_SWIGLU) ? (cg * 4 + wn * 2 + (ni & 1)) < ntiles / 2
                                 : tile[ni] < ntiles;
    ltile[ni] = tv[ni] ? tile[ni] : ntiles - 1;
  }
  [[maybe_unused]] ResidRows<A, EPI == EPI_RESID ? MI : 1> rres;
  if constexpr (EPI == EPI_RESID) rres = load_resid<A, BMT, MI>(p, m0, tile, tv);

  // Global -> register staging of the X tile (BMT rows x 64 k), two register
  // sets: X of step j lives in set j & 1 from its load, two steps ahead,
  // until it is written to LDS.
  // byte offsets of this thread's X pieces from the work-group's first row
  const uint16_t* xbase = (const uint16_t*)p.x + (size_t)m0 * p.ldx;
  uint32_t xoff[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int idx = threadIdx.x + 256 * i;
    const int r = idx >> 3, c = idx & 7;
    xoff[i] = (uint32_t)((min(m0 + r, p.M - 1) - m0) * p.ldx + c * 8) * 2u;
  }
  u32x4 ra[2][NA];
  auto load_a = [&](int kt, int set) {
#pragma unroll
    for (int i = 0; i < NA; ++i) ra[set][i] = ld16(xbase, xoff[i] + (uint32_t)(kt * BK * 2));
  };
  auto store_a = [&](int buf, int set) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int r = idx >> 3, c = idx & 7;
      *(u32x4*)&sA[buf * BMT * LDA + r * LDA + c * 8] = ra[set][i];
    }
  };
  // LB staging: thread piece i is local tile lt = 2 i + threadIdx.x / 128
  // (wave column lt / 4, fragment lt % 4), chunk (threadIdx.x / 64) & 1 and
  // lane threadIdx.x & 63 of that 1 KiB fragment.
  int gtile[LB ? 4 : 1];
  if constexpr (LB) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int lt = 2 * i + (threadIdx.x >> 7);
      const int tl = wave_tile<EPI>(cg, ntiles, lt >> 2, lt & 3);
      const bool ok = (EPI == EPI_SWIGLU) ? (cg * 4 + (lt >> 2) * 2 + (lt & 1)) < ntiles / 2
                                          : tl < ntiles;
      gtile[i] = ok ? tl : ntiles - 1;
    }
  }
  u32x4 rg[LB ? 2 : 1][LB ? 4 : 1];
  auto load_bg = [&](int kt, int set) {
    if constexpr (LB) {
      const int c = (threadIdx.x >> 6) & 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t ch = (uint32_t)gtile[i] * (K / 32) + 2 * kt + c;
        rg[set][i] = ld16(p.W.w, (ch * 64 + lane) * 16u);
      }
    }
  };
  auto store_bg = [&](int buf, int set) {
    if constexpr (LB) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int piece = threadIdx.x + 256 * i;  // (lt, c, lane) in LDS order
        *(u32x4*)&sB[buf * 8192 + piece * 8] = rg[set][i];
      }
    }
  };
  constexpr int NCH = (WK == WK_Q8) ? 1 : 2;  // weight chunks per tile per K step
  // B fragments, double-buffered by step parity: step kt reads set kt & 1,
  // which was loaded during step kt - 1, and loads set (kt + 1) & 1.
  u32x4 rb[2][4][NCH];
  uint32_t rs[2][4];
  auto load_b = [&](int kt, int set) {
    if constexpr (LB) return;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      if constexpr (WK == WK_Q8) {
        const uint32_t ch = (uint32_t)ltile[ni] * (K / 64) + kt;
        rb[set][ni][0] = ld16(p.W.w, (ch * 64 + lane) * 16u);
        rs[set][ni] = ld4(p.W.sc, (ch * 16 + row) * 4u);
      } else {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const uint32_t ch = (uint32_t)ltile[ni] * (K / 32) + 2 * kt + c;
          rb[set][ni][c] = ld16(p.W.w, (ch * 64 + lane) * 16u);
        }
      }
    }
  };

  f32x4 acc[MI][4];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Pipeline: step kt computes from LDS buffer kt & 1 and the B fragments
  // loaded during the previous step; at its end X of step kt + 1 goes from
  // registers into the other buffer and X of step kt + 3 is loaded.  One
  // barrier per step: it orders this step's writes of buffer (kt+1) & 1
  // before the next step's reads, and this step's reads of buffer kt & 1
  // before the next step's writes to it.  The loop is unrolled by two so that
  // every register set index is a compile-time constant.  Loads past the last
  // step re-read it; their data is never used.
  const int KT = K / BK;
  load_a(0, 0);
  load_b(0, 0);
  load_bg(0, 0);
  load_a(min(1, KT - 1), 1);
  load_bg(min(1, KT - 1), 1);
  store_a(0, 0);
  store_bg(0, 0);
  load_a(min(2, KT - 1), 0);
  load_bg(min(2, KT - 1), 0);
  __syncthreads();
  auto step = [&](auto par, int kt) {
    constexpr int P = decltype(par)::value;
    u32x4 cb[4][NCH];
    uint32_t cs[4];
    if constexpr (LB) {
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          cb[ni][c] = *(const u32x4*)&sB[P * 8192 + ((wn * 4 + ni) * 2 + c) * 512 + lane * 8];
    } else {
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) cb[ni][c] = rb[P][ni][c];
        cs[ni] = rs[P][ni];
      }
    }
    load_b(min(kt + 1, KT - 1), P ^ 1);
    const uint16_t* a = sA + P * BMT * LDA;
    u32x4 fa[MI][2];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        fa[mi][ks] = *(const u32x4*)&a[(wm * (BMT / 2) + mi * 16 + row) * LDA + ks * 32 + kg * 8];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      if constexpr (WK == WK_Q8) {
        const u32x4 b0 = q8_to_f16x8(cb[ni][0][0], cb[ni][0][1]);
        const u32x4 b1 = q8_to_f16x8(cb[ni][0][2], cb[ni][0][3]);
        const float d0 = f16_to_f32((uint16_t)(cs[ni] & 0xffffu));
        const float d1 = f16_to_f32((uint16_t)(cs[ni] >> 16));
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
          const f32x4 t0 = mfma16<ACT_F16>(fa[mi][0], b0, z);
          const f32x4 t1 = mfma16<ACT_F16>(fa[mi][1], b1, z);
          acc[mi][ni] += d0 * t0;
          acc[mi][ni] += d1 * t1;
        }
      } else {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
          acc[mi][ni] = mfma16<A>(fa[mi][0], cb[ni][0], acc[mi][ni]);
          acc[mi][ni] = mfma16<A>(fa[mi][1], cb[ni][1], acc[mi][ni]);
        }
      }
    }
    store_a(P ^ 1, P ^ 1);
    store_bg(P ^ 1, P ^ 1);
    load_a(min(kt + 3, KT - 1), P ^ 1);
    load_bg(min(kt + 3, KT - 1), P ^ 1);
    __syncthreads();
  };
  for (int kt = 0; kt < KT; kt += 2) {
    step(std::integral_constant<int, 0>{}, kt);
    if (kt + 1 < KT) step(std::integral_constant<int, 1>{}, kt + 1);
  }

  if constexpr (EPI == EPI_ROPE) {
    rope_epilogue<A, BMT, MI>(p, acc, sA, m0, cg, rrows);
    return;
  }
  if constexpr (EPI == EPI_SWIGLU) {
    swiglu_epilogue<A, BMT, MI>(p, acc, m0, tile, tv);
    return;
  }
  // Epilogue.  Lane holds rows 4*kg + r of each 16-row fragment, column `row`.
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int gr = m0 + wm * (BMT / 2) + mi * 16 + 4 * kg + r;
      if (gr >= p.M) continue;
      {
        if constexpr (EPI == EPI_AFFINE)
          if (!affine_row(p, gr)) continue;
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
          if (!tv[ni]) continue;
          const size_t o = (size_t)gr * p.ldy + tile[ni] * 16 + row;
          if constexpr (EPI == EPI_RESID)
            ((T*)p.y)[o] = st_act<A>(ld_act<A>(rres.v[mi][r][ni]) + rd<A>(acc[mi][ni][r]));
          else if constexpr (EPI == EPI_AFFINE)
            ((T*)p.y)[o] = st_act<A>(affine_value<A>(p, acc[mi][ni][r], gr, tile[ni] * 16 + row));
          else
            ((T*)p.y)[o] = st_act<A>(acc[mi][ni][r]);
        }
      }
    }
  }
}

// 16-bit activations with dense 16-bit weights, both operands copied global
// -> LDS by the direct-to-LDS loads (no register staging): a ring of NS
// stages of BK2 = 32 k, NS - 1 steps in flight, one barrier per step.  Tile
// BMT x 128 (BMT 64, 128 or 256), four waves of BMT/2 x 64 (same fragments, same
// epilogue, same XCD work order as gemm16_kernel).  X stage: BMT rows x 4
// chunks of 8 elements, chunk c of row r at slot r * 4 + (c ^ swz(r)), so
// that the fragment reads of any 8 consecutive lanes fall in distinct
// 16-byte bank groups of 128 bytes and those of any 16 in distinct groups of
// 256 bytes; W stage: the work-group's 8 weight tiles, each one 1 KiB
// fragment of the tiled layout.  LDS: NS * (BMT * 64 + 8192) bytes, so two
// work-groups per CU at (128, 4) and (256, 3), three at (64, 4).
constexpr int BK2 = 32;

// EPI_SWIGLU with 16-byte stores on the direct-to-LDS tiles (the host picks
// it when the output allows them).
constexpr int EPI_SWIGLU_STAGED = 102;



__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

// Two values already rounded to the 16-bit activation dtype, packed (lo in
// the low half).  bf16: the high halves of the two f32 (their low halves are
// zero), one v_perm_b32.
template <int A>
__device__ __forceinline__ uint32_t pack2_rounded(float lo, float hi) {
  if constexpr (A == ACT_BF16)
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, lo), 0x07060302u);
  else
    return (uint32_t)st_act<A>(lo) | ((uint32_t)st_act<A>(hi) << 16);
}

// EPI_AFFINE on the direct-to-LDS BMT x 128 tiles, through LDS: the
// accumulators, rounded to the activation dtype (the first affine step), are
// staged row-major in the freed ring -- the 16-byte chunk c of tile row R at
// chunk position c ^ rope_sw(R), so the 2-byte writes of a wave's four
// 16-lane groups (rows 4 apart) fall in distinct banks and a row's 16 chunk
// reads cover all of them -- then 16 lanes per row finish 8 columns each,
// two rows per pass (16 independent chains through affine_block), with
// 16-byte residual and table loads and 16-byte stores instead of 2-byte
// accesses in the accumulators' layout.
template <int A, int BMT, int MI>
__device__ __forceinline__ void staged_affine_epilogue(const GemmArgs& p, const f32x4 (&acc)[MI][4], int m0,
                                                       int cg, uint16_t* stg) {
  typedef typename ActT<A>::T T;
  const AffineArgs& f = p.aff;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1, row = lane & 15, kg = lane >> 4;
  const int ch = threadIdx.x & 15, r0 = threadIdx.x >> 4;   // chunk, first row
  const int gc = cg * 128 + ch * 8;                          // its first output column
  const bool col_ok = gc < p.W.out;
  const int rows = min(BMT, p.M - m0);
  // The bias and the residual or table values (a product has at most one
  // of the two: staged_ok) of the lane's rows r0, r0 + 16, ... are loaded
  // first, so the loads run under the staging below and none follows a
  // store: a vector-memory wait also counts the stores issued before it, so
  // a load placed after a store would hold the lane until that store
  // completed.  A lane loads the residual of exactly the outputs it stores
  // (the output may be the residual itself).  The loads are unconditional
  // (a load inside a branch is waited for where the branches join): without
  // a residual or table every row reads the tile's first output row, and
  // without a bias the bias load reads that row too (values affine_block
  // does not use); rows past the tile read its last row and lanes past the
  // last column read column 0 (neither is stored).
  constexpr int NR = BMT / 16;
  const int gl = col_ok ? gc : 0;
  const T* xb = (const T*)p.y + (size_t)m0 * p.ldy + gl;
  int xs = 0;
  if (p.resid) {
    xb = (const T*)p.resid + (size_t)m0 * p.ldy + gl;
    xs = p.ldy;
  } else if (f.table) {
    xb = (const T*)f.table + gl;
    xs = p.W.out;
  }
  const bool by_period = f.table && !p.resid;
  const u32x4 bias4 = *(const u32x4*)(f.bias ? (const T*)f.bias + gl : xb);
  u32x4 xv4[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int R = min(r0 + 16 * i, rows - 1);
    const int xr = by_period ? max(min((m0 + R) % f.period, f.valid - 1), 0) : R;
    xv4[i] = *(const u32x4*)(xb + (size_t)xr * xs);
  }
  barrier_lds();   // every wave's last fragment reads are done
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int R = wm * (BMT / 2) + mi * 16 + 4 * kg + r;
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        const int C = wn * 64 + ni * 16 + row;
        stg[R * 128 + ((((C >> 3) ^ rope_sw(R)) << 3) | (C & 7))] = st_act<A>(acc[mi][ni][r]);
      }
    }
  barrier_lds();
  if (!col_ok) return;                                       // (no barrier follows)
  T* const y = (T*)p.y + (size_t)m0 * p.ldy + gc;
  float bias[8], scl[8];
  unpack8<A>(bias4, bias);
#pragma unroll
  for (int e = 0; e < 8; ++e) scl[e] = gc + e < f.scale_cols ? f.scale : 1.0f;
  // two rows (16 independent chains) per pass
#pragma unroll
  for (int i = 0; i < NR; i += 2) {
    if (r0 + 16 * i >= rows) break;
    float v[16], bs[16], sc[16];
    T xv[16];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int R = min(r0 + 16 * (i + q), rows - 1);
      unpack8<A>(*(const u32x4*)&stg[R * 128 + ((ch ^ rope_sw(R)) << 3)], &v[8 * q]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xv[8 * q + e] = (T)(xv4[i + q][e / 2] >> (16 * (e & 1)));
        bs[8 * q + e] = bias[e];
        sc[8 * q + e] = scl[e];
      }
    }
    affine_block<A, 16, true>(p, v, sc, bs, xv, xv);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int R = r0 + 16 * (i + q);
      if (R >= rows || !affine_row(p, m0 + R)) continue;
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) o[e / 2] = pack2_rounded<A>(v[8 * q + e], v[8 * q + e + 1]);
      *(u32x4*)(y + (size_t)R * p.ldy) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

template <int A, int EPI, int BMT, int NS>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
gemm_dma_kernel(GemmArgs p) {
  typedef typename ActT<A>::T T;
  static_assert(((BMT == 64 || BMT == 128) && NS == 4) || (BMT == 256 && NS == 3), "tile / ring");
  constexpr int MI = BMT / 32;           // 16-row fragments per wave
  constexpr int NX = BMT / 64;           // X copies per thread per stage
  constexpr int PER = NX + 2;            // copies per thread per stage
  constexpr int SA = BMT * BK2;          // X elements per stage
  constexpr int SB = 8 * 512;            // weight elements per stage (8 KB)
  static_assert(NS * (SA + SB) >= BMT * 128, "the staged epilogue reuses the ring");
  __shared__ __attribute__((aligned(1024))) uint16_t smem[NS * (SA + SB)];
  uint16_t* const sA = smem;
  uint16_t* const sB = smem + NS * SA;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int K = p.W.in, ntiles = p.W.out / 16;
  constexpr int WEPI = EPI == EPI_SWIGLU_STAGED ? EPI_SWIGLU : EPI;   // the tiles' layout
  const int cols = WEPI == EPI_SWIGLU ? (ntiles / 2 + 3) / 4 : (ntiles + 7) / 8;
  int mt, cg;
  tile_of(blockIdx.x, (p.M + BMT - 1) / BMT, cols, p.map, mt, cg);
  if (mt * BMT >= p.M) return;
  const int m0 = mt * BMT;
  const int row = lane & 15, kg = lane >> 4;
  [[maybe_unused]] RopeRows<EPI == EPI_ROPE ? BMT : 16> rrows;
  if constexpr (EPI == EPI_ROPE) rrows = rope_rows<BMT>(p, m0);
  int tile[4];
  bool tv[4];
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    tile[ni] = wave_tile<WEPI>(cg, ntiles, wn, ni);
    tv[ni] = (WEPI == EPI_SWIGLU) ? (cg * 4 + wn * 2 + (ni & 1)) < ntiles / 2 : tile[ni] < ntiles;
  }
  static_assert(EPI != EPI_RESID || BMT <= 128, "residual prefetch: 64- and 128-row tiles");
  [[maybe_unused]] ResidRows<A, EPI == EPI_RESID ? MI : 1> rres;
  if constexpr (EPI == EPI_RESID) rres = load_resid<A, BMT, MI>(p, m0, tile, tv);
  // This thread's copies per stage: X slots j * 64 + lane of instructions
  // j = NX w .. NX w + NX - 1 (rows 16 j + lane / 4; rows past M read row
  // M - 1), weight tiles t = 2w, 2w + 1 (past the end: the last tile).
  const uint16_t* xbase = (const uint16_t*)p.x + (size_t)m0 * p.ldx;
  uint32_t xoff[NX], woff[2];
#pragma unroll
  for (int i = 0; i < NX; ++i) {
    const int j = NX * w + i;
    const int slot = j * 64 + lane, r = slot >> 2, cs = slot & 3;
    const int c = cs ^ swz(r);
    xoff[i] = (uint32_t)((min(m0 + r, p.M - 1) - m0) * p.ldx + c * 8) * 2u;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int t = 2 * w + i;
    int tl = wave_tile<WEPI>(cg, ntiles, t >> 2, t & 3);
    const bool ok = (WEPI == EPI_SWIGLU) ? (cg * 4 + (t >> 2) * 2 + (t & 1)) < ntiles / 2 : tl < ntiles;
    tl = ok ? tl : ntiles - 1;
    woff[i] = ((uint32_t)tl * (K / 32) * 64 + lane) * 16u;
  }
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const uint32_t la = lds_addr(sA) + (uint32_t)wu * (NX * 1024u);
  const uint32_t lb = lds_addr(sB) + (uint32_t)wu * 2048u;
  auto issue = [&](int kt, int buf) {
#pragma unroll
    for (int i = 0; i < NX; ++i)
      lds_copy16(xbase, xoff[i] + (uint32_t)(kt * BK2 * 2), la + (uint32_t)(buf * SA * 2 + i * 1024));
#pragma unroll
    for (int i = 0; i < 2; ++i)
      lds_copy16(p.W.w, woff[i] + (uint32_t)(kt * 1024), lb + (uint32_t)(buf * SB * 2 + i * 1024));
  };

  f32x4 acc[MI][4];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Stages past the last step re-read it (their copies only make the waits
  // below conservative).
  const int KT = K / BK2;
#pragma unroll
  for (int s0 = 0; s0 < NS - 1; ++s0) issue(min(s0, KT - 1), s0);
  for (int kt = 0; kt < KT; ++kt) {
    // this step's copies have landed (those of the `after` later stages may
    // still be in flight, PER copies each), then every thread's are visible
    const int after = min(NS - 2, KT - 1 - kt);
    if (after == 2) wait_vm<2 * PER>();
    else if (after == 1) wait_vm<PER>();
    else wait_vm<0>();
    barrier_lds();
    // refill the stage computed in the previous step
    if (kt + NS - 1 < KT) issue(kt + NS - 1, (kt + NS - 1) % NS);
    const uint16_t* a = sA + (kt % NS) * SA;
    const uint16_t* bb = sB + (kt % NS) * SB;
    u32x4 fb[4];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) fb[ni] = *(const u32x4*)&bb[(wn * 4 + ni) * 512 + lane * 8];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const int r = wm * (BMT / 2) + mi * 16 + row;
      const u32x4 fa = *(const u32x4*)&a[(r * 4 + (kg ^ swz(r))) * 8];
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma16<A>(fa, fb[ni], acc[mi][ni]);
    }
  }

  if constexpr (EPI == EPI_ROPE) {
    rope_epilogue<A, BMT, MI>(p, acc, sA, m0, cg, rrows);
    return;
  }
  if constexpr (EPI == EPI_AFFINE) {
    staged_affine_epilogue<A, BMT, MI>(p, acc, m0, cg, smem);
    return;
  }
  if constexpr (EPI == EPI_SWIGLU_STAGED) {
    swiglu_staged_epilogue<A, BMT, MI>(p, acc, m0, cg, smem);
    return;
  }
  if constexpr (EPI == EPI_SWIGLU) {
    swiglu_epilogue<A, BMT, MI>(p, acc, m0, tile, tv);
    return;
  }
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int gr = m0 + wm * (BMT / 2) + mi * 16 + 4 * kg + r;
      if (gr >= p.M) continue;
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        if (!tv[ni]) continue;
        const size_t o = (size_t)gr * p.ldy + tile[ni] * 16 + row;
        if constexpr (EPI == EPI_RESID)
          ((T*)p.y)[o] = st_act<A>(ld_act<A>(rres.v[mi][r][ni]) + rd<A>(acc[mi][ni][r]));
        else
          ((T*)p.y)[o] = st_act<A>(acc[mi][ni][r]);
      }
    }
  }
}

// f32 activations / weights on v_mfma_f32_16x16x4f32; same tiling, K chunks of 16.
template <int EPI>
__global__ void __launch_bounds__(256) gemm32_kernel(GemmArgs p) {
  constexpr int LDF = BK + 4;
  __shared__ float sA[BM * LDF];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int K = p.W.in, ntiles = p.W.out / 16;
  const int m0 = blockIdx.x * BM;
  const int row = lane & 15, kg = lane >> 4;
  int tile[4];
  bool tv[4];
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    tile[ni] = wave_tile<EPI>(blockIdx.y, ntiles, wn, ni);
    tv[ni] = (EPI == EPI_SWIGLU) ? (blockIdx.y * 4 + wn * 2 + (ni & 1)) < ntiles / 2
                                 : tile[ni] < ntiles;
  }
  f32x4 acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int KT = K / BK;
  for (int kt = 0; kt < KT; ++kt) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int idx = threadIdx.x + 256 * i;  // 2048 float4 pieces
      const int r = idx >> 4, c = idx & 15;
      const int gr = m0 + r;
      *(f32x4*)&sA[r * LDF + c * 4] =
          gr < p.M ? *(const f32x4*)((const float*)p.x + (size_t)gr * p.ldx + kt * BK + c * 4)
                   : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      f32x4 fb[4];
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        const size_t ch = (size_t)tile[ni] * (K / 16) + kt * 4 + c;
        fb[ni] = tv[ni] ? ((const f32x4*)p.W.w)[ch * 64 + lane] : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        const f32x4 fa = *(const f32x4*)&sA[(wm * 64 + mi * 16 + row) * LDF + c * 16 + kg * 4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[j], fb[ni][j], acc[mi][ni], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int gr = m0 + wm * 64 + mi * 16 + 4 * kg + r;
      if (gr >= p.M) continue;
      if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          if (!tv[ni]) continue;
          const float gg = acc[mi][ni][r], u = acc[mi][ni + 2][r];
          ((float*)p.y)[(size_t)gr * p.ldy + tile[ni] * 16 + row] = (gg / (1.0f + __expf(-gg))) * u;
        }
      } else {
        if constexpr (EPI == EPI_AFFINE)
          if (!affine_row(p, gr)) continue;
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
          if (!tv[ni]) continue;
          const size_t o = (size_t)gr * p.ldy + tile[ni] * 16 + row;
          if constexpr (EPI == EPI_RESID)
            ((float*)p.y)[o] = ((const float*)p.resid)[o] + acc[mi][ni][r];
          else if constexpr (EPI == EPI_AFFINE)
            ((float*)p.y)[o] = affine_value<ACT_F32>(p, acc[mi][ni][r], gr, tile[ni] * 16 + row);
          else
            ((float*)p.y)[o] = acc[mi][ni][r];
        }
      }
    }
  }
}

// Tile of the 16-bit dense kernels (512 work-groups = two per CU), chosen
// from bf16 sweeps over the prefill shapes and row counts:
// - 256 rows (DMA) where 256-row tiles fill at least 7/8 of the slots and do
//   not end in a last round of fewer than 128 work-groups (qkv M = 3584 36.5
//   against 38.9 us, M = 4096 39.2 against 42.4; gate|up M = 2560 38.0
//   against 41.4, M = 4096 59.8 against 62.9, but M = 3072, 576 tiles, 56.2
//   against 51.9);
// - 128 rows (DMA) where their grid fills the slots, and for wide outputs
//   (16 or more column groups) also below that (qkv M = 1328 19.5 against
//   22.3 us for 64-row tiles, M = 1560 20.9 against 27.6);
// - narrow outputs (O and down, N = 1024) otherwise take 64-row tiles: the
//   register-staged kernel up to one tile per CU, the DMA kernel above
//   (O M = 2048 23.3 against 25.3 us; M = 2455 28.4 against 32.3, M = 4096
//   31.7 against 34.7; down M = 2455 37.5 against 43.0, M = 4096 42.0
//   against 46.0).
enum GemmTile { TILE64 = 0, TILE64_DMA = 1, TILE128 = 2, TILE256 = 3 };
GemmTile gemm_tile(int M, int col_groups) {
  const int tiles64 = (M + 63) / 64 * col_groups;
  const int tiles128 = (M + 127) / 128 * col_groups;
  const int tiles256 = (M + 255) / 256 * col_groups;
  if (tiles256 >= 448 && (tiles256 % 512 == 0 || tiles256 % 512 >= 128)) return TILE256;
  if (tiles128 >= 512 || col_groups >= 16) return TILE128;
  return tiles64 > 256 ? TILE64_DMA : TILE64;
}

// 16-byte output, bias, residual and table accesses for the staged
// epilogues, which also hold a residual or a table, not both.
bool staged_ok(const GemmArgs& a) {
  auto al = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  return !(a.resid && a.aff.table) && a.ldy % 8 == 0 && al(a.y) && (!a.aff.bias || al(a.aff.bias)) &&
         (!a.aff.table || al(a.aff.table)) && (!a.resid || al(a.resid)) && a.W.out % 8 == 0;
}

template <int A, int BMT, int NS>
hipError_t launch_dma(int epi, dim3 grid, const GemmArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL((gemm_dma_kernel<A, EPI_STORE, BMT, NS>), grid, dim3(256), 0, s, a); break;
    case EPI_RESID:
      if constexpr (BMT > 128) return hipErrorInvalidValue;
      else hipLaunchKernelGGL((gemm_dma_kernel<A, EPI_RESID, BMT, NS>), grid, dim3(256), 0, s, a);
      break;
    case EPI_SWIGLU:
      if (staged_ok(a)) hipLaunchKernelGGL((gemm_dma_kernel<A, EPI_SWIGLU_STAGED, BMT, NS>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((gemm_dma_kernel<A, EPI_SWIGLU, BMT, NS>), grid, dim3(256), 0, s, a);
      break;
    case EPI_ROPE:
      if constexpr (BMT > 128) return hipErrorInvalidValue;
      else hipLaunchKernelGGL((gemm_dma_kernel<A, EPI_ROPE, BMT, NS>), grid, dim3(256), 0, s, a);
      break;
    case EPI_AFFINE:
      if (!staged_ok(a)) return hipErrorInvalidValue;  // dispatch routes these to the 64-row tiles
      hipLaunchKernelGGL((gemm_dma_kernel<A, EPI_AFFINE, BMT, NS>), grid, dim3(256), 0, s, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int A, int WK, int BMT, bool LB>
hipError_t launch16_lb(int epi, dim3 grid, const GemmArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL((gemm16_kernel<A, WK, EPI_STORE, BMT, LB>), grid, dim3(256), 0, s, a); break;
    case EPI_RESID: hipLaunchKernelGGL((gemm16_kernel<A, WK, EPI_RESID, BMT, LB>), grid, dim3(256), 0, s, a); break;
    case EPI_SWIGLU: hipLaunchKernelGGL((gemm16_kernel<A, WK, EPI_SWIGLU, BMT, LB>), grid, dim3(256), 0, s, a); break;
    case EPI_ROPE: hipLaunchKernelGGL((gemm16_kernel<A, WK, EPI_ROPE, BMT, LB>), grid, dim3(256), 0, s, a); break;
    case EPI_AFFINE:
      if constexpr (WK == WK_Q8) return hipErrorInvalidValue;  // the audio path is dense
      else hipLaunchKernelGGL((gemm16_kernel<A, WK, EPI_AFFINE, BMT, LB>), grid, dim3(256), 0, s, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Dense weights of 64-row tiles go through LDS; 128-row tiles read them from
// global memory (measured: staging made the 64-row tiles ~4% faster and the
// 128-row tiles ~8% slower, whose LDS reads then outlast the MFMAs).
template <int A, int WK, int BMT>
hipError_t launch16(int epi, dim3 grid, const GemmArgs& a, hipStream_t s) {
  if constexpr (WK == WK_DENSE && BMT == 64) return launch16_lb<A, WK, BMT, true>(epi, grid, a, s);
  return launch16_lb<A, WK, BMT, false>(epi, grid, a, s);
}

// XCD rows a (1, 2, 4 or 8; the XCD grid is a x 8/a) for an M x N x K
// product: the X bytes are fetched 8/a times and the weight bytes a times;
// the column groups must split evenly over 8/a.
int xcd_rows(const GemmArgs& p, int cols, int bm) {
  const double xb = (double)p.M * p.W.in * 2;
  const double wb = (double)p.W.out * p.W.in * (p.W.kind == WK_Q8 ? 34.0 / 32 : 2.0);
  int best = 1;
  double cost = 1e300;
  for (int a = 1; a <= 8; a *= 2) {
    if (cols % (8 / a)) continue;
    const double c = (8 / a) * xb + a * wb;
    if (c < cost) cost = c, best = a;
  }
  (void)bm;
  return best;
}

template <int A, int WK>
hipError_t dispatch(int epi, const GemmArgs& a, hipStream_t s) {
  const int ntiles = a.W.out / 16;
  const int cols = epi == EPI_SWIGLU ? (ntiles / 2 + 3) / 4 : (ntiles + 7) / 8;
  if constexpr (A == ACT_F32) {
    const dim3 grid((a.M + BM - 1) / BM, cols);
    switch (epi) {
      case EPI_STORE: hipLaunchKernelGGL(gemm32_kernel<EPI_STORE>, grid, dim3(256), 0, s, a); break;
      case EPI_RESID: hipLaunchKernelGGL(gemm32_kernel<EPI_RESID>, grid, dim3(256), 0, s, a); break;
      case EPI_SWIGLU: hipLaunchKernelGGL(gemm32_kernel<EPI_SWIGLU>, grid, dim3(256), 0, s, a); break;
      case EPI_AFFINE: hipLaunchKernelGGL(gemm32_kernel<EPI_AFFINE>, grid, dim3(256), 0, s, a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  } else {
    GemmTile tt = WK == WK_Q8 ? TILE64 : gemm_tile(a.M, cols);
    // the direct-to-LDS tiles' affine epilogue moves 16 bytes at a time; an
    // output, residual, bias or table that does not allow it takes the
    // register-staged tiles (element by element)
    if (epi == EPI_AFFINE && tt != TILE64 && !staged_ok(a)) tt = TILE64;
    // the fused q/k norm + RoPE epilogue stages at most 128 rows (a 256-row
    // tile would spill), and the residuals a 256-row tile would prefetch do
    // not fit its registers: 128-row tiles instead
    if ((epi == EPI_ROPE || epi == EPI_RESID) && tt == TILE256) tt = TILE128;
    const int bm = tt == TILE256 ? 256 : tt == TILE128 ? 128 : 64;
    GemmArgs g = a;
    g.map = xcd_rows(a, cols, bm);
    const int mtiles = (a.M + bm - 1) / bm, Ma = (mtiles + g.map - 1) / g.map;
    const dim3 grid(8 * Ma * (cols / (8 / g.map)));
    // Q8_0 tiles scale each block's product in f32 on the VALU, so their
    // accumulators live in VGPRs: only the 64-row tile fits without spills.
    if (tt == TILE64) return launch16<A, WK, 64>(epi, grid, g, s);
    if constexpr (WK != WK_Q8) {
      if (tt == TILE256) return launch_dma<A, 256, 3>(epi, grid, g, s);
      if (tt == TILE128) return launch_dma<A, 128, 4>(epi, grid, g, s);
      return launch_dma<A, 64, 4>(epi, grid, g, s);
    }
    return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_gemm(int act, int epi, const GemmArgs& a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.W.in % BK || a.W.out % 16 || (epi == EPI_SWIGLU && a.W.out % 32))
    return hipErrorInvalidValue;
  // EPI_ROPE: 16-bit activations, one 128-wide head slot per column group,
  // at most 16 sequences (a row's position and sequence travel as pos * 16 + b)
  if (epi == EPI_ROPE && (act == ACT_F32 || a.W.out != (a.rope.nh + 2 * a.rope.nkv) * 128 ||
                          !a.rope.row_b || !a.rope.row_pos || a.rope.batch < 1 ||
                          a.rope.batch > 16))
    return hipErrorInvalidValue;
  if (epi == EPI_AFFINE && ((a.aff.table && (a.aff.period <= 0 || a.aff.valid < 1)) ||
                            (a.aff.period > 0 && (a.aff.valid < 0 || a.aff.valid > a.aff.period)) ||
                            a.aff.act < 0 || a.aff.act > 2 || a.aff.scale_cols < 0))
    return hipErrorInvalidValue;
  if (a.W.kind == WK_Q8) {
    if (act != ACT_F16) return hipErrorInvalidValue;
    return dispatch<ACT_F16, WK_Q8>(epi, a, s);
  }
  switch (act) {
    case ACT_F32: return dispatch<ACT_F32, WK_DENSE>(epi, a, s);
    case ACT_F16: return dispatch<ACT_F16, WK_DENSE>(epi, a, s);
    case ACT_BF16: return dispatch<ACT_BF16, WK_DENSE>(epi, a, s);
  }
  return hipErrorInvalidValue;
}
