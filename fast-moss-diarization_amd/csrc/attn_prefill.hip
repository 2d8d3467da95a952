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
// MFMA path (16-bit): each tile's keys are cut into items (pieces of a
// multiple of 64 keys, so long contexts spread over more work-groups); pass 1
// writes each item's per-row (max, sum of exp), pass 2 merges a tile's items
// in order and writes its share of P V (or, for a one-item tile, the context
// itself), and a combine kernel adds the shares of split tiles.  One
// work-group per (item, KV head), 4*REP/QS waves; wave w owns query head g*REP + w%REP and
// 16*QS positions (with QS sets, each K or V^T fragment read from LDS feeds
// QS MFMAs; a tile covers 64 * QS positions).  Keys come in blocks of 64, staged global -> registers -> LDS
// with the next block's loads in flight while the current one is computed
// (double-buffered LDS, one barrier per block).  Per block: S^T = K Q^T (keys
// are the MFMA's M side, so the f32 result already sits in the B-operand
// layout of P^T), then O^T += V^T P^T with the V^T operand read from the
// row-major V block by LDS transpose reads.
#include <type_traits>

#include "fmd_common.h"
#include "fmd_kernels.h"

namespace {

constexpr int HD = 128;

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

// Two f32 values rounded to the activation dtype (round to nearest even) and
// packed low | high; one conversion instruction for bf16.
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

// a.lo * b.lo + a.hi * b.hi in f32 (v_dot2_f32_f16 / v_dot2_f32_bf16)
template <int A>
__device__ __forceinline__ float dot2f(uint32_t a, uint32_t b) {
  if constexpr (A == ACT_BF16) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, a), __builtin_bit_cast(b2, b), 0.f, false);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), 0.f, false);
  }
}

// PASS 0: one work-group does pass 1 and pass 2 of a one-item tile.
// PASS 1 / PASS 2: the two passes of a split tile as separate launches.
template <int A, int REP, int QS, int PASS>
__global__ void __launch_bounds__(256 * REP / QS)
__attribute__((amdgpu_waves_per_eu(REP == 4 ? 4 : 2 * REP / QS))) attn_prefill_kernel(AttnPrefillArgs p) {
  typedef typename ActT<A>::T T;
  constexpr int NTH = 256 * REP / QS;     // waves: (query head, 16*QS positions)
  constexpr int TR = 64;                  // query positions per tile
  constexpr int KB = 64;                  // keys per block
  constexpr int LDK = HD + 8;             // padded K row pitch (elements)
  constexpr int LDV = HD + 16;            // padded V row pitch (elements)
  constexpr int PIECES = KB * HD / 8;     // 16-byte pieces of a K (or V) block
  constexpr int PPT = PIECES / NTH;       // pieces per thread
  // 70 KiB: gfx950 gives a work-group up to 160 KiB of LDS
  __shared__ __attribute__((aligned(16))) uint16_t sK[2 * KB * LDK];    // [2][KB][LDK]
  __shared__ __attribute__((aligned(16))) uint16_t sV[(PASS == 1 ? 0 : 2) * KB * LDV + 8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // Work-group -> (item, KV head): work-groups are dealt to the 8 XCDs
  // round-robin (linear id % 8), and each XCD has its own L2.  Adjacent
  // entries of the work list of one KV head (the tiles of one prompt, or in a
  // split launch the items of one prompt that cover the same key range, in
  // item_order) read the same K/V blocks, so each XCD takes a contiguous run
  // of the (head-major) work list, and the run's concurrent work-groups share
  // those blocks in its L2.
  int item, g;
  {
    const int n = gridDim.x * gridDim.y, L = blockIdx.y * gridDim.x + blockIdx.x;
    const int per = n >> 3;
    const int w = (L < 8 * per) ? (L & 7) * per + (L >> 3) : L;
    item = w % gridDim.x;
    g = w / gridDim.x;
    if (PASS != 0 && p.item_order) item = p.item_order[item];
  }
  const int t = PASS == 0 ? item : p.item_tile[item];
  const int b = p.tile_b[t], row0 = p.tile_row0[t], pos0 = p.tile_pos0[t], n = p.tile_n[t];
  const int nh = p.nkv * REP;
  const int r = w % REP, half = w / REP;  // head g*REP + r, positions 16*QS*half ..
  const int h = g * REP + r;
  const int qr = lane & 15, kg = lane >> 4;
  // this work-group's keys [kstart, kend): all of [pad_b, pos0 + n) for a
  // one-item tile, else a piece of it whose length is a multiple of 64
  const int kstart = PASS == 0 ? p.start[b] : p.item_k0[item];
  const int kend = PASS == 0 ? pos0 + n : p.item_k1[item];
  const size_t kvbase = ((size_t)b * p.nkv + g) * p.cap;
  const int nblk = (kend - kstart + KB - 1) / KB;
  int myrow[QS], qpos[QS];
  bool row_ok[QS];
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) {
    myrow[qs] = 16 * QS * half + 16 * qs + qr;
    row_ok[qs] = myrow[qs] < n;
    qpos[qs] = pos0 + myrow[qs];
  }

  // Q^T fragments (B operand), per query set: row qr, dims 32ks + 8kg + [0,8).
  u32x4 qf[QS][4];
#pragma unroll
  for (int qs = 0; qs < QS; ++qs)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[qs][ks] = row_ok[qs] ? *(const u32x4*)((const uint16_t*)p.q +
                                                ((size_t)(row0 + myrow[qs]) * nh + h) * HD +
                                                ks * 32 + kg * 8)
                              : u32x4{0, 0, 0, 0};

  // Block staging: global -> registers (one block ahead) -> LDS (double
  // buffered), K and V row-major.  The V^T operand of O^T = V^T P^T is read
  // with ds_read_b64_tr_b16, which transposes 16-bit data across each group
  // of 16 lanes: lane l of a group receives element l%4 of the 64-bit rows
  // addressed by lanes l/4, l/4 + 4, l/4 + 8 and l/4 + 12.
  u32x4 pk[PPT], pv[PPT];
  auto fetch = [&](int blk, bool with_v) {
    const int k0 = kstart + blk * KB;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int idx = tid + NTH * i, key = idx >> 4, c = idx & 15;
      const bool ok = k0 + key < kend;
      const size_t e = (kvbase + (ok ? k0 + key : kstart)) * HD + c * 8;
      pk[i] = ok ? *(const u32x4*)((const uint16_t*)p.kc + e) : u32x4{0, 0, 0, 0};
      if (with_v) pv[i] = ok ? *(const u32x4*)((const uint16_t*)p.vc + e) : u32x4{0, 0, 0, 0};
    }
  };
  auto stage = [&](int buf, bool with_v) {
    uint16_t* k = sK + buf * KB * LDK;
    uint16_t* v = sV + buf * KB * LDV;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int idx = tid + NTH * i, key = idx >> 4, c = idx & 15;
      *(u32x4*)&k[key * LDK + c * 8] = pk[i];
      if (PASS != 1 && with_v) *(u32x4*)&v[key * LDV + c * 8] = pv[i];
    }
  };
  // Scaled scores S^T for keys k0 + 16mt + 4kg + i of query row qr of each
  // set: rd(rd(q.k) * rd(scale)) as qwen3.rs:243, rounded two at a time.  A
  // block past the tile's first position is masked: -inf past the row's last
  // visible key (its position, or -1 for rows past the tile's end).  Blocks
  // wholly at or below the first position need no mask (rows past the tile's
  // end are then left unmasked: their output is never stored).  The two
  // variants are separate instantiations so no per-element branch remains.
  // Each K fragment read from LDS feeds all query sets.
  int lim[QS];
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) lim[qs] = row_ok[qs] ? qpos[qs] : -1;
  const uint32_t sc_lo = pack2<A>(p.scale, 0.f), sc_hi = pack2<A>(0.f, p.scale);
  auto scores_t = [&](auto full_tag, int buf, int k0, f32x4 (*s4)[KB / 16]) {
    constexpr bool FULL = decltype(full_tag)::value;
    const uint16_t* k = sK + buf * KB * LDK;
#pragma unroll
    for (int mt = 0; mt < KB / 16; ++mt) {
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) s4[qs][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4 ka = *(const u32x4*)&k[(16 * mt + qr) * LDK + ks * 32 + kg * 8];
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) s4[qs][mt] = mfma16<A>(ka, qf[qs][ks], s4[qs][mt]);
      }
#pragma unroll
      for (int qs = 0; qs < QS; ++qs)
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          // rd(q.k) of two keys packed; each times rd(scale) by a packed dot
          // product against (scale, 0) or (0, scale): the product of two
          // dtype values is exact in f32, so this is rd(q.k) * rd(scale)
          // without unpacking
          const uint32_t r = pack2<A>(s4[qs][mt][i], s4[qs][mt][i + 1]);
          const f32x2 v = unpack2<A>(pack2<A>(dot2f<A>(r, sc_lo), dot2f<A>(r, sc_hi)));
          if constexpr (FULL) {
            s4[qs][mt][i] = v.x;
            s4[qs][mt][i + 1] = v.y;
          } else {
            const int key = k0 + 16 * mt + 4 * kg + i;
            s4[qs][mt][i] = key <= lim[qs] ? v.x : -INFINITY;
            s4[qs][mt][i + 1] = key + 1 <= lim[qs] ? v.y : -INFINITY;
          }
        }
    }
  };
  auto scores = [&](int buf, int k0, f32x4 (*s4)[KB / 16]) {
    if (k0 + KB - 1 <= pos0)
      scores_t(std::true_type{}, buf, k0, s4);
    else
      scores_t(std::false_type{}, buf, k0, s4);
  };

  // Per-item (max, sum of exp) of row myrow, head h: part_ml slot.
  auto ml_index = [&](int it, int qs) {
    return (((size_t)it * p.nkv + g) * TR + myrow[qs]) * REP + r;
  };

  // The row's max M (as M log2 e) and 1 / S; stand-ins (0, 1) for rows with
  // no valid key, whose output is never stored.
  float mlog[QS], inv[QS];
  if constexpr (PASS != 2) {
    // Pass 1: max and sum of exp of each query row over the keys (each lane
    // covers 16 keys per block; the four lanes of a row merge at the end).
    // Branch-free: exp(-inf) is 0, and a row with no valid key keeps
    // (max, sum) = (-inf, 0) through a finite stand-in for its max.
    float m[QS], l[QS];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      m[qs] = -INFINITY;
      l[qs] = 0.f;
    }
    if (nblk > 0) fetch(0, false);
    for (int blk = 0; blk < nblk; ++blk) {
      const int k0 = kstart + blk * KB;
      stage(blk & 1, false);
      if (blk + 1 < nblk) fetch(blk + 1, false);
      __syncthreads();
      f32x4 s4[QS][KB / 16];
      scores(blk & 1, k0, s4);
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) {
        float bm = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < KB / 16; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) bm = fmaxf(bm, s4[qs][mt][i]);
        const float mn = fmaxf(m[qs], bm);
        const float ml2 = (mn == -INFINITY ? 0.f : mn) * kLog2e;
        float e = l[qs] * __builtin_amdgcn_exp2f(fmaf(m[qs], kLog2e, -ml2));
#pragma unroll
        for (int mt = 0; mt < KB / 16; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) e += __builtin_amdgcn_exp2f(fmaf(s4[qs][mt][i], kLog2e, -ml2));
        m[qs] = mn;
        l[qs] = e;
      }
    }
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
#pragma unroll
      for (int off = 16; off <= 32; off <<= 1) {
        const float mo = __shfl_xor(m[qs], off), lo = __shfl_xor(l[qs], off);
        const float mn = fmaxf(m[qs], mo);
        const float mref = mn == -INFINITY ? 0.f : mn;
        l[qs] = l[qs] * __expf(m[qs] - mref) + lo * __expf(mo - mref);
        m[qs] = mn;
      }
      if constexpr (PASS == 1) {
        if (kg == 0) {
          float* dst = p.part_ml + ml_index(item, qs) * 2;
          dst[0] = m[qs];
          dst[1] = l[qs];
        }
      } else {
        mlog[qs] = (m[qs] == -INFINITY ? 0.f : m[qs]) * kLog2e;
        inv[qs] = 1.f / (l[qs] > 0.f ? l[qs] : 1.f);
      }
    }
    if constexpr (PASS == 1) return;
    __syncthreads();   // pass 1's last reads of the LDS buffers precede pass 2's writes
  } else {
    // The row's global max M and sum S from its tile's items, in item order.
    const int first = p.tile_first[t], ns = p.tile_nsplit[t];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      float pm[8], pl[8];
      float M = -INFINITY, S = 0.f;
      for (int j0 = 0; j0 < ns; j0 += 8) {
        const int nj = ns - j0 < 8 ? ns - j0 : 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const f32x2 v = j < nj ? *(const f32x2*)(p.part_ml + ml_index(first + j0 + j, qs) * 2)
                                 : f32x2{-INFINITY, 0.f};
          pm[j] = v.x;
          pl[j] = v.y;
        }
        float mn = M;
#pragma unroll
        for (int j = 0; j < 8; ++j) mn = fmaxf(mn, pm[j]);
        const float mr = mn == -INFINITY ? 0.f : mn;
        S *= __expf(M - mr);
#pragma unroll
        for (int j = 0; j < 8; ++j) S += pl[j] * __expf(pm[j] - mr);
        M = mn;
      }
      mlog[qs] = (M == -INFINITY ? 0.f : M) * kLog2e;
      inv[qs] = 1.f / (S > 0.f ? S : 1.f);
    }
  }

  if constexpr (PASS != 1) {
    // Pass 2: p = rd(exp(s - M) / S) in the activation dtype (softmax_last_dim,
    // qwen3.rs:248), then O^T += V^T P^T over the keys.
    f32x4 o[QS][8];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs)
#pragma unroll
      for (int i = 0; i < 8; ++i) o[qs][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nblk > 0) fetch(0, true);
    for (int blk = 0; blk < nblk; ++blk) {
      const int k0 = kstart + blk * KB;
      stage(blk & 1, true);
      if (blk + 1 < nblk) fetch(blk + 1, true);
      __syncthreads();
      f32x4 s4[QS][KB / 16];
      scores(blk & 1, k0, s4);
      typedef short s16x4 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
      const uint16_t* vb = sV + (blk & 1) * KB * LDV;
      const int ts = lane & 15;   // this lane's row-supplier role in the transposed read
#pragma unroll
      for (int hb = 0; hb < KB / 32; ++hb) {
        u32x4 pb[QS];
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) {
          uint32_t pp[4];
#pragma unroll
          for (int mm = 0; mm < 2; ++mm)
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
              const f32x4& sv = s4[qs][2 * hb + mm];
              // exp(s - M) as 2^(s log2 e - M log2 e); -inf -> 0
              const float e0 = __builtin_amdgcn_exp2f(fmaf(sv[i], kLog2e, -mlog[qs]));
              const float e1 = __builtin_amdgcn_exp2f(fmaf(sv[i + 1], kLog2e, -mlog[qs]));
              pp[mm * 2 + i / 2] = pack2<A>(e0 * inv[qs], e1 * inv[qs]);
            }
          pb[qs] = u32x4{pp[0], pp[1], pp[2], pp[3]};
        }
        // k-slot s of lane group kg holds key 32hb + 4kg + s (s < 4) or
        // 32hb + 16 + 4kg + (s - 4), matching where S^T put those keys.  For
        // the A operand (row = dim 16dt + l%16), lane ts of group kg supplies
        // the 64-bit row of key 32hb + 4kg + ts/4 (+16 for the second read)
        // at dims 16dt + 4(ts%4) .. +3.
        s16x4 r1[8], r2[8];
        const int key1 = 32 * hb + 4 * kg + (ts >> 2);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const int dim = 16 * dt + 4 * (ts & 3);
          r1[dt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + key1 * LDV + dim));
          r2[dt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + (key1 + 16) * LDV + dim));
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const u32x4 va = __builtin_bit_cast(u32x4, __builtin_shufflevector(r1[dt], r2[dt], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
          for (int qs = 0; qs < QS; ++qs) o[qs][dt] = mfma16<A>(va, pb[qs], o[qs][dt]);
        }
      }
    }
    // A one-item tile stores its context rd(O) (qwen3.rs:252); a split tile
    // stores this item's share of sum_j p_j v_j for the combine.
    const bool single = PASS == 0 || p.tile_nsplit[t] == 1;
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      if (!row_ok[qs]) continue;
      if (single) {
        T* out = (T*)p.out + ((size_t)(row0 + myrow[qs]) * nh + h) * HD;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          *(uint32_t*)&out[16 * dt + 4 * kg] = pack2<A>(o[qs][dt][0], o[qs][dt][1]);
          *(uint32_t*)&out[16 * dt + 4 * kg + 2] = pack2<A>(o[qs][dt][2], o[qs][dt][3]);
        }
      } else {
        float* po = p.part_o + ml_index(item, qs) * HD;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) *(f32x4*)&po[16 * dt + 4 * kg] = o[qs][dt];
      }
    }
  }
}

// Context of split tiles: the items' shares added in item order, stored in
// the activation dtype.  One work-group per (tile, KV head, 16 query rows);
// each thread adds 2*REP four-float pieces of those rows.  TR: tile rows.
template <int A, int REP, int TR>
__global__ void __launch_bounds__(256) attn_prefill_combine_kernel(AttnPrefillArgs p) {
  typedef typename ActT<A>::T T;
  constexpr int ROWF4 = REP * HD / 4;          // four-float pieces per row (all REP heads)
  constexpr int V = 16 * ROWF4 / 256;          // pieces per thread
  const int t = blockIdx.x, g = blockIdx.y, rbase = 16 * blockIdx.z;
  const int ns = p.tile_nsplit[t], n = p.tile_n[t];
  if (ns == 1 || rbase >= n) return;
  const int first = p.tile_first[t], row0 = p.tile_row0[t];
  const int nh = p.nkv * REP;
  f32x4 acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = f32x4{0.f, 0.f, 0.f, 0.f};
  // rows past the tile's end read (unused) slots of the TR-row item block
  for (int j = 0; j < ns; ++j) {
    const float* src = p.part_o + (((size_t)(first + j) * p.nkv + g) * TR + rbase) * REP * HD;
    f32x4 x[V];
#pragma unroll
    for (int v = 0; v < V; ++v) x[v] = *(const f32x4*)(src + 4 * (threadIdx.x + 256 * v));
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] += x[v];
  }
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int idx = threadIdx.x + 256 * v, row = rbase + idx / ROWF4, c = idx % ROWF4;
    if (row < n) {
      T* out = (T*)p.out + ((size_t)(row0 + row) * nh + g * REP) * HD + 4 * c;
      *(uint32_t*)&out[0] = pack2<A>(acc[v][0], acc[v][1]);
      *(uint32_t*)&out[2] = pack2<A>(acc[v][2], acc[v][3]);
    }
  }
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

// Query sets per wave: with two (GQA repeat 2), a 64-position tile takes 2 REP
// waves of 32 positions, and each K or V^T fragment read from LDS feeds two
// MFMAs; other repeats keep one set (4 REP waves of 16 positions).
constexpr int qs_of(int rep) { return rep == 2 ? 2 : 1; }

template <int A, int REP>
hipError_t launch_three(const AttnPrefillArgs& a, hipStream_t s) {
  constexpr int QS = qs_of(REP);
  constexpr int NT = 256 * REP / QS;
  if (a.nitems == a.ntiles) {   // no tile split: both passes in one launch
    hipLaunchKernelGGL((attn_prefill_kernel<A, REP, QS, 0>), dim3(a.ntiles, a.nkv), dim3(NT), 0, s, a);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((attn_prefill_kernel<A, REP, QS, 1>), dim3(a.nitems, a.nkv), dim3(NT), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_prefill_kernel<A, REP, QS, 2>), dim3(a.nitems, a.nkv), dim3(NT), 0, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.nitems > a.ntiles)
    hipLaunchKernelGGL((attn_prefill_combine_kernel<A, REP, 64>), dim3(a.ntiles, a.nkv, 4),
                       dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int A>
hipError_t launch_rep(int rep, const AttnPrefillArgs& a, hipStream_t s) {
  switch (rep) {
    case 1: return launch_three<A, 1>(a, s);
    case 2: return launch_three<A, 2>(a, s);
    case 4: return launch_three<A, 4>(a, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Query positions per prefill attention tile (16-bit path: 16 * QS positions
// per wave, 4 waves per query head; the f32 path takes any tile size).
int attn_prefill_tile_rows(int rep) {
  (void)rep;
  return 64;
}

hipError_t launch_attn_prefill(int act, int rep, const AttnPrefillArgs& a, hipStream_t s) {
  if (a.ntiles <= 0) return hipSuccess;
  if (rep != 1 && rep != 2 && rep != 4) return hipErrorInvalidValue;
  switch (act) {
    case ACT_F32: {
      const int rpt = attn_prefill_tile_rows(rep);
      hipLaunchKernelGGL(attn_prefill_f32_kernel, dim3(a.ntiles * rpt, a.nkv * rep), dim3(64), 0,
                         s, a, rep, rpt);
      return hipGetLastError();
    }
    case ACT_F16: return launch_rep<ACT_F16>(rep, a, s);
    case ACT_BF16: return launch_rep<ACT_BF16>(rep, a, s);
  }
  return hipErrorInvalidValue;
}
