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

// rd(x) to bf16 (round to nearest even), as an f32: v_cvt_pk_bf16_f32 with a
// zero low half.
__device__ __forceinline__ float rd_hi(float x) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(float, __builtin_convertvector((f32x2){0.f, x}, bf16x2));
}

// a.lo * b.lo + a.hi * b.hi in f32 (v_dot2c_f32_f16 / v_dot2c_f32_bf16 on a
// zeroed destination).
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

// K / V block layout in LDS (64 keys x 128 dims, 16 KiB, unpadded): row r
// (key k0 + r) at byte 256 r, its 16-byte chunk c (dims 8c .. 8c + 7) at
// chunk position c ^ swk(r) for K and c ^ swv(r) for V.  The K fragment reads
// (16 rows, one chunk) and the transposed V reads (per 16 lanes: 4 rows x 32
// bytes) then fall in distinct banks, for 8- and 16-lane bank groups alike.
// A block is copied global -> LDS by 16 wave instructions of 1 KiB (4 rows
// each) whose lanes fetch the chunks in swizzled order.
__device__ __forceinline__ int swk(int r) { return r & 15; }
__device__ __forceinline__ int swv(int r) { return (r & 7) << 1; }

// PASS 0: one work-group does pass 1 and pass 2 of a one-item tile.
// PASS 1 / PASS 2: the two passes of a split tile as separate launches.
template <int A, int REP, int QS, int PASS>
__global__ void __launch_bounds__(256 * REP / QS)
__attribute__((amdgpu_waves_per_eu(REP == 4 ? 4 : 2 * REP / QS))) attn_prefill_kernel(AttnPrefillArgs p) {
  typedef typename ActT<A>::T T;
  constexpr int NTH = 256 * REP / QS;     // waves: (query head, 16*QS positions)
  constexpr int NW = NTH / 64;
  constexpr int TR = 64;                  // query positions per tile
  constexpr int KB = 64;                  // keys per block
  constexpr int BLK = KB * HD;            // elements of a K (or V) block
  constexpr int CPW = 16 / NW;            // 1 KiB copies per wave per block and operand
  // 64 KiB (two K and two V blocks); pass 1 stages K only
  __shared__ __attribute__((aligned(1024))) uint16_t sK[2 * BLK];
  __shared__ __attribute__((aligned(1024))) uint16_t sV[PASS == 1 ? 8 : 2 * BLK];
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

  // Block copies: wave w issues instructions j = i NW + w (i < CPW) of each
  // operand; lane l of instruction j fetches row 4j + l/16 at the logical
  // chunk stored at position l % 16.  A block wholly inside the item reads
  // from the block's first row (a wave-uniform base) at per-lane offsets
  // fixed for the whole loop; in the item's last block, keys past its end
  // read its last key: they lie past every row's last visible key, so their
  // scores are masked and their probabilities are 0.
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const uint16_t* kbase = (const uint16_t*)p.kc + kvbase * HD;
  const uint16_t* vbase = (const uint16_t*)p.vc + kvbase * HD;
  int crow[CPW];
  uint32_t kch[CPW], vch[CPW];
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const int j = i * NW + wu, rr = 4 * j + (lane >> 4), pc = lane & 15;
    crow[i] = rr;
    kch[i] = (uint32_t)rr * (HD * 2) + (uint32_t)(pc ^ swk(rr)) * 16u;
    vch[i] = (uint32_t)rr * (HD * 2) + (uint32_t)(pc ^ swv(rr)) * 16u;
  }
  const uint32_t lk = lds_addr(sK), lv = lds_addr(sV);
  auto issue = [&](int blk, auto with_v_tag) {
    constexpr bool WV = decltype(with_v_tag)::value;
    const int k0 = kstart + blk * KB;
    const uint32_t boff = (uint32_t)(blk & 1) * (BLK * 2);
    if (k0 + KB <= kend) {
      const uint16_t* kb = kbase + (size_t)k0 * HD;
      const uint16_t* vb = vbase + (size_t)k0 * HD;
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const uint32_t j = (uint32_t)(i * NW + wu);
        lds_copy16(kb, kch[i], lk + boff + j * 1024u);
        if constexpr (WV) lds_copy16(vb, vch[i], lv + boff + j * 1024u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const uint32_t j = (uint32_t)(i * NW + wu);
        const uint32_t off = (uint32_t)(min(k0 + crow[i], kend - 1) - crow[i]) * (HD * 2);
        lds_copy16(kbase, off + kch[i], lk + boff + j * 1024u);
        if constexpr (WV) lds_copy16(vbase, off + vch[i], lv + boff + j * 1024u);
      }
    }
  };
  // Blocks wholly at or below the tile's first position (no mask) come
  // first: blocks [0, nfull).  Each loop runs one variant, so its
  // accumulators stay in place across iterations.
  const int nfull = max(0, min(nblk, (pos0 - kstart + 1) / KB));

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
  const float scale_f = __builtin_bit_cast(float, sc_hi);   // rd(scale) (bf16)
  // raw S^T of sub-block mt (keys 16mt .. 16mt + 15 of the block)
  auto qk = [&](const uint16_t* kb, int mt, f32x4* sv) {
    u32x4 ka[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      ka[ks] = *(const u32x4*)&kb[(16 * mt + qr) * HD + (((4 * ks + kg) ^ qr) << 3)];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) sv[qs] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) sv[qs] = mfma16<A>(ka[ks], qf[qs][ks], sv[qs]);
  };
  // sv <- scaled, rounded (and for a masked block, masked) scores
  auto scale_mask = [&](auto full_tag, int kmt, f32x4* sv) {
    constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
    for (int qs = 0; qs < QS; ++qs)
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        // rd(rd(q.k) * rd(scale)); the product of two dtype values is exact
        // in f32
        f32x2 v;
        if constexpr (A == ACT_BF16) {
          // one conversion per rounding: bf16 in the high half over a zero
          // low half is that value as an f32
          v.x = rd_hi(rd_hi(sv[qs][i]) * scale_f);
          v.y = rd_hi(rd_hi(sv[qs][i + 1]) * scale_f);
        } else {
          // f16: rd(q.k) of two keys packed, each times rd(scale) by a packed
          // dot product against (scale, 0) or (0, scale)
          const uint32_t rr = pack2<A>(sv[qs][i], sv[qs][i + 1]);
          v = unpack2<A>(pack2<A>(dot2f<A>(rr, sc_lo), dot2f<A>(rr, sc_hi)));
        }
        if constexpr (FULL) {
          sv[qs][i] = v.x;
          sv[qs][i + 1] = v.y;
        } else {
          const int key = kmt + 4 * kg + i;
          sv[qs][i] = key <= lim[qs] ? v.x : -INFINITY;
          sv[qs][i + 1] = key + 1 <= lim[qs] ? v.y : -INFINITY;
        }
      }
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
    auto stats = [&](auto full_tag, const uint16_t* kb, int k0) {
      f32x4 sv[4][QS];
      qk(kb, 0, sv[0]);
      qk(kb, 1, sv[1]);
      scale_mask(full_tag, k0, sv[0]);
      qk(kb, 2, sv[2]);
      scale_mask(full_tag, k0 + 16, sv[1]);
      qk(kb, 3, sv[3]);
      scale_mask(full_tag, k0 + 32, sv[2]);
      scale_mask(full_tag, k0 + 48, sv[3]);
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) {
        float bm = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < KB / 16; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) bm = fmaxf(bm, sv[mt][qs][i]);
        const float mn = fmaxf(m[qs], bm);
        const float ml2 = (mn == -INFINITY ? 0.f : mn) * kLog2e;
        float e = l[qs] * __builtin_amdgcn_exp2f(fmaf(m[qs], kLog2e, -ml2));
#pragma unroll
        for (int mt = 0; mt < KB / 16; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) e += __builtin_amdgcn_exp2f(fmaf(sv[mt][qs][i], kLog2e, -ml2));
        m[qs] = mn;
        l[qs] = e;
      }
    };
    auto run = [&](auto full_tag, int b0, int b1) {
      for (int blk = b0; blk < b1; ++blk) {
        wait_vm<0>();      // this block's copies (the only ones in flight) have landed
        barrier_lds();     // for every wave; and block blk - 1's buffer is free
        if (blk + 1 < nblk) issue(blk + 1, std::false_type{});
        stats(full_tag, sK + (blk & 1) * BLK, kstart + blk * KB);
      }
    };
    if (nblk > 0) issue(0, std::false_type{});
    run(std::true_type{}, 0, nfull);
    run(std::false_type{}, nfull, nblk);
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
    barrier_lds();   // pass 1's last reads of the K buffers precede pass 2's copies
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
    // probabilities of one sub-block, packed two keys per word: pp[2 qs + i/2]
    // holds keys 4kg + i, 4kg + i + 1
    auto probs = [&](const f32x4* sv, uint32_t* pp) {
#pragma unroll
      for (int qs = 0; qs < QS; ++qs)
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          // exp(s - M) as 2^(s log2 e - M log2 e); -inf -> 0
          const float e0 = __builtin_amdgcn_exp2f(fmaf(sv[qs][i], kLog2e, -mlog[qs]));
          const float e1 = __builtin_amdgcn_exp2f(fmaf(sv[qs][i + 1], kLog2e, -mlog[qs]));
          pp[2 * qs + i / 2] = pack2<A>(e0 * inv[qs], e1 * inv[qs]);
        }
    };
    // O^T += V^T P^T over keys 32hb .. 32hb + 31 of the block.  k-slot s of
    // lane group kg holds key 32hb + 4kg + s (s < 4) or 32hb + 16 + 4kg +
    // (s - 4), matching where S^T put those keys.  For the A operand (row =
    // dim 16dt + l%16), lane ts of group kg supplies the 64-bit row of key
    // 32hb + 4kg + ts/4 (+16 for the second read) at dims 16dt + 4(ts%4) ..
    // +3, i.e. bytes 8 (ts % 4) of logical chunk 2dt + (ts % 4) / 2.
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const int ts = lane & 15;
    auto pv = [&](const uint16_t* vb, int hb, const uint32_t* pa, const uint32_t* pc) {
      u32x4 pb[QS];
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) pb[qs] = u32x4{pa[2 * qs], pa[2 * qs + 1], pc[2 * qs], pc[2 * qs + 1]};
      const int key1 = 32 * hb + 4 * kg + (ts >> 2);
      const int sw = swv(key1);   // = swv(key1 + 16)
#pragma unroll
      for (int dh = 0; dh < 2; ++dh) {
        s16x4 r1[4], r2[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const int dt = 4 * dh + d;
          const int e = (((2 * dt + ((ts & 3) >> 1)) ^ sw) << 3) + 4 * (ts & 1);
          r1[d] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + key1 * HD + e));
          r2[d] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + (key1 + 16) * HD + e));
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const u32x4 va = __builtin_bit_cast(u32x4, __builtin_shufflevector(r1[d], r2[d], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
          for (int qs = 0; qs < QS; ++qs) o[qs][4 * dh + d] = mfma16<A>(va, pb[qs], o[qs][4 * dh + d]);
        }
      }
    };
    // One block, software-pipelined by 16-key sub-blocks: each sub-block's
    // probabilities are computed beside the next sub-block's Q.K^T MFMAs or
    // the previous pair's P.V MFMAs.
    auto block = [&](auto full_tag, const uint16_t* kb, const uint16_t* vb, int k0) {
      f32x4 sv[4][QS];
      uint32_t pp[4][2 * QS];
      qk(kb, 0, sv[0]);
      qk(kb, 1, sv[1]);
      scale_mask(full_tag, k0, sv[0]);
      probs(sv[0], pp[0]);
      qk(kb, 2, sv[2]);
      scale_mask(full_tag, k0 + 16, sv[1]);
      probs(sv[1], pp[1]);
      qk(kb, 3, sv[3]);
      scale_mask(full_tag, k0 + 32, sv[2]);
      probs(sv[2], pp[2]);
      pv(vb, 0, pp[0], pp[1]);
      scale_mask(full_tag, k0 + 48, sv[3]);
      probs(sv[3], pp[3]);
      pv(vb, 1, pp[2], pp[3]);
    };
    auto run = [&](auto full_tag, int b0, int b1) {
      for (int blk = b0; blk < b1; ++blk) {
        wait_vm<0>();      // this block's copies (the only ones in flight) have landed
        barrier_lds();     // for every wave; and block blk - 1's buffers are free
        if (blk + 1 < nblk) issue(blk + 1, std::true_type{});
        block(full_tag, sK + (blk & 1) * BLK, sV + (blk & 1) * BLK, kstart + blk * KB);
      }
    };
    if (nblk > 0) issue(0, std::true_type{});
    run(std::true_type{}, 0, nfull);
    run(std::false_type{}, nfull, nblk);
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
