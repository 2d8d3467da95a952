// Launch interfaces of the gfx950 decoder kernels (host side).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Activation dtype codes (the activation dtype of each precision, precision.rs:32-41).
enum ActDtype { ACT_F32 = 0, ACT_F16 = 1, ACT_BF16 = 2 };
// Weight storage kinds.
enum WeightKind { WK_DENSE = 0, WK_Q8 = 1 };

// Epilogues of the projection kernels.
enum LinEpilogue {
  EPI_STORE = 0,   // y = rd(x W^T)
  EPI_RESID = 1,   // y = rd(resid + rd(x W^T))            (qwen3.rs:334, 338)
  EPI_SWIGLU = 2,  // y = rd(rd(silu(rd(g))) * rd(u))       (qwen3.rs:289-291)
  EPI_LOGITS = 3,  // f32 y = rd(x W^T), plus per-block argmax keys (qwen3.rs:459-463)
  EPI_ROPE = 4,    // prefill q|k|v: rd(x W^T), then per head the q/k RMSNorm, RoPE and
                   // the store of q and the K/V cache rows (qwen3.rs:213-241)
  EPI_AFFINE = 5,  // the audio path's linears and convolutions: see AffineArgs
};

// EPI_AFFINE, in this order, each step rounded to the activation dtype:
// v = rd(x W^T); + bias[col] (a Linear's bias, linear.rs:41-44); * scale for
// col < scale_cols (the encoder's q/k scaling, whisper_encoder.rs:53-56);
// gelu_erf / silu; + resid[row, col] (GemmArgs::resid, row stride ldy, may
// alias y); + table[row % period, col] (the encoder's positions,
// whisper_encoder.rs:155-157).  With period > 0 a row is stored only when
// row % period < valid (the padding rows between windows are skipped).
struct AffineArgs {
  const void* bias;   // (N) in the activation dtype, or NULL
  float scale;        // already rounded to the activation dtype
  int scale_cols;     // 0: no scaling
  int act;            // 0 none, 1 gelu_erf, 2 silu
  const void* table;  // (period, N) in the activation dtype, or NULL
  int period, valid;
};

// Weight tiles (B operand order of the 16x16 MFMAs):
//  16-bit dense: [N/16][K/32][64 lanes][8]: lane l -> row 16t + l%16,
//                k = 32kb + 8(l/16) + [0,8)
//  Q8_0:  qs [N/16][K/64][64 lanes][16 B]: lane l -> row 16t + l%16,
//                bytes 0-7: k = 64c + 8(l/16) + [0,8), bytes 8-15: the same +32
//         sc [N/16][K/64][16 rows] u32: f16 d of block 2c | d of block 2c+1 << 16
//  f32 dense:    [N/16][K/16][64 lanes][4]: lane l -> row 16t + l%16,
//                k = 16c + 4(l/16) + [0,4)  (element j feeds the j-th 16x16x4 MFMA)
struct LinWeights {
  int kind;  // 0 dense, 1 q8_0
  int out, in;
  uint8_t* w;
  uint32_t* sc;
};

struct GemvArgs {
  const void* x;       // (rows, K) activations, row stride ldx
  int ldx;
  const void* norm_w;  // RMSNorm gain (K) when the prologue normalises x
  float eps;
  LinWeights W;
  int rows;            // <= 16
  void* y;             // output, row stride ldy
  int ldy;
  const void* resid;   // EPI_RESID input, row stride ldy (may alias y)
  uint64_t* amax_part; // EPI_LOGITS: (gridDim.x, rows) argmax keys
  uint32_t* epoch;     // when set, the kernel advances this single-launch attention
                       // epoch: the attention launch before it left that to it
};

struct RopeArgs {
  const void* qkv;        // (rows, nh*hd + 2*nkv*hd)
  int ldqkv;
  int rows;
  const int32_t* row_b;   // batch index of each row (NULL: row r is sequence r)
  int batch;              // sequences in the cache (the EPI_ROPE epilogue packs a row's
                          // sequence in 4 bits: at most 16)
  const int32_t* row_pos; // absolute position of each row (NULL: state[0])
  const int32_t* state;
  int nh, nkv;
  const void* qn_w;
  const void* kn_w;
  const void* cos;        // (max_len, hd/2) in the activation dtype
  const void* sin;
  void* q_out;            // (rows, nh, hd)
  void* kc;               // (B, nkv, cap, hd)
  void* vc;
  int cap;
  float eps;
};

struct GemmArgs {
  const void* x;  // (M, K) activations, row stride ldx
  int ldx;
  LinWeights W;
  int M;
  void* y;
  int ldy;
  const void* resid;
  int map;        // work-group -> tile order (set by launch_gemm)
  RopeArgs rope;  // EPI_ROPE: everything but qkv / ldqkv (the product is not stored)
  AffineArgs aff; // EPI_AFFINE
};

struct AttnDecodeArgs {
  const void* qkv;        // (B, ldqkv) raw projection of the new token: q | k | v
  int ldqkv;
  const void* qn_w;       // q_norm / k_norm gains (hd)
  const void* kn_w;
  const void* cos;        // (max_len, hd/2) RoPE tables in the activation dtype
  const void* sin;
  float eps;
  void* kc;               // (B, nkv, cap, hd); the new K/V are appended at state[0]
  void* vc;
  int cap, nkv, rep, batch;
  const int32_t* start;   // first valid key per row (= left pad)
  const int32_t* state;   // state[0] = position of the new token
  const int32_t* done;    // rows with done[b] != 0 are skipped (NULL: none)
  void* scores;           // (B, nh, cap) scores in the activation dtype
  float* ml;              // (B, nkv, max_splits, REP, 2) per-split (max, sum of exp)
  float* part;            // (B, nkv, max_splits, REP, hd) per-split sum of p * v
  int max_splits;
  int split;              // existing keys per work-group (multiple of 128)
  void* out;              // (B, nh*hd)
  float scale;
  // Single-launch path (fused != 0): exchange words of the work-groups of
  // one (row, KV head) -- epoch << 32 | data -- and the launch state
  // sync = [epoch, units finished, error code, 0, per-unit counters...].
  int fused;
  uint32_t* sync;
  uint64_t* xml;          // (B*nkv, max_splits, REP, 2) per-split (max, sum of exp), f32
  uint64_t* xpart;        // (B*nkv, max_splits, REP*hd) per-split sum of p * v, f32
  uint64_t* xsc;          // (B*nkv, REP, xsc_stride) scores of keys pad+2i, pad+2i+1 (dtype bits)
  int xsc_stride;         // >= max_splits * split / 2
  uint64_t* xnew;         // (B*nkv, REP) the new token's score, f32
  int spin_limit;         // polls before a wait gives up and records an error
  int count_units;        // the launch advances its own epoch once its last unit is
                          // combined (0: the kernel after it advances the epoch)
  // With nq > 0 the launch also computes qkv itself (ldqkv = nq * 16 columns):
  // rd(RMSNorm(x) W^T) published two columns per word in xqkv (B, ldqkv/2),
  // instead of reading `qkv`.
  int nq;
  const void* x;          // (B, hidden) layer input, row stride ldx
  int ldx, hidden;
  const void* norm_w;     // input_layernorm gain (hidden)
  LinWeights Wqkv;
  uint64_t* xqkv;
};

// Split plan of decode attention for `units` (row, KV head) pairs over a
// cache of `cap` positions: keys per work-group, work-groups per unit, and
// whether the single-launch path applies.
struct AttnDecodePlan {
  int split, max_splits, fused;
};
AttnDecodePlan attn_decode_plan(int act, int rep, int cap, int units);

struct AttnPrefillArgs {
  const void* q;          // (rows, nh, hd), rows packed per sequence
  const void* kc;
  const void* vc;
  int cap, nkv;
  const int32_t* tile_b;     // per 64-query tile: sequence
  const int32_t* tile_row0;  // first packed row of the tile
  const int32_t* tile_pos0;  // absolute position of that row
  const int32_t* tile_n;     // rows in the tile (<= 64)
  const int32_t* start;      // per sequence: first valid key (= pad)
  int ntiles;
  // Split of each tile's keys into items [k0, k1) (16-bit path): item i of
  // tile t is tile_first[t] + j, j < tile_nsplit[t].
  const int32_t* item_tile;
  const int32_t* item_k0;
  const int32_t* item_k1;
  const int32_t* tile_first;
  const int32_t* tile_nsplit;
  // Order in which work-groups take the items of a split launch (NULL: item
  // order): items that read the same key range of the same sequence adjacent.
  const int32_t* item_order;
  int nitems;
  float* part_ml;         // (nitems, nkv, 64, REP, 2): per-item (max, sum of exp) per row
  float* part_o;          // (nitems, nkv, 64, REP, hd): per-item sum of p v (split tiles)
  void* out;              // (rows, nh*hd)
  float scale;
};

// Dense attention of the Whisper encoder (head_dim 64) over windows of t
// positions stored `period` rows apart: q | k | v of a row are the column
// blocks [0, d), [d, 2d), [2d, 3d) of `qkv` (q and k already scaled).
struct EncAttnArgs {
  const void* qkv;
  int ld;         // row stride of qkv (elements)
  int d;          // heads * 64
  int t;          // positions per window
  int period;     // rows per window in qkv and out (>= t)
  void* out;      // (rows, ldo) context, head h at columns [64 h, 64 h + 64)
  int ldo;
};

struct GreedyArgs {
  const uint64_t* part;   // (nparts, B) argmax keys
  int nparts, batch;
  int32_t* state;         // [0] kv length, [1] greedy step, [2] rows done
  int32_t* host_state;    // host-mapped mirror of state[2], written when it changes (may be NULL)
  int advance;            // 1 when a decode step appended a key since the last call
  int32_t* done;
  int32_t* ntok;
  int32_t* finish;
  uint32_t* tokens;       // (B, budget)
  int budget;
  const int32_t* force;   // (B) forced end-of-turn step, or NULL
  uint32_t eos;
  uint32_t* next_ids;
  const void* embed;      // (V, H) table, activation dtype
  void* x;                // (B, H) next step's input
  int hidden;
  int vocab;
};

// All launchers return hipError_t of the launch.
hipError_t launch_gemv(int act, int epi, bool norm, const GemvArgs& a, hipStream_t s);
hipError_t launch_gemm(int act, int epi, const GemmArgs& a, hipStream_t s);
// Prompt assembly: row r of `out` is the embedding of token src[r] (>= 0),
// zeros (-1) or audio row -2 - src[r] (audio dtype 0 f32, 1 f16, 2 bf16).
hipError_t launch_assemble(int act, const int32_t* src, int rows, const void* table,
                           const void* audio, int audio_dtype, int hidden, void* out, hipStream_t s);
hipError_t launch_rmsnorm(int act, const void* x, int ldx, const void* w, int rows, int dim,
                          float eps, void* y, int ldy, hipStream_t s);
hipError_t launch_rope_store(int act, const RopeArgs& a, hipStream_t s);
hipError_t launch_attn_decode(int act, const AttnDecodeArgs& a, hipStream_t s);
hipError_t launch_attn_prefill(int act, int rep, const AttnPrefillArgs& a, hipStream_t s);
hipError_t launch_greedy(int act, const GreedyArgs& a, hipStream_t s);
hipError_t launch_embed(int act, const uint32_t* ids, int n, const void* table, int hidden,
                        void* out, hipStream_t s);
hipError_t launch_gather_rows(int act, const void* src, int ld_src, const int32_t* rows, int n,
                              int dim, void* dst, int ld_dst, hipStream_t s);
hipError_t launch_quantize_q8_0_tiles(const float* src, int rows, int cols, int row0,
                                      LinWeights W, hipStream_t s);
hipError_t launch_pack_dense(int act, const void* src, int src_dtype, int rows, int cols,
                             int row0, LinWeights W, hipStream_t s);
hipError_t launch_convert(int act, const void* src, int src_dtype, int64_t n, void* dst,
                          hipStream_t s);
hipError_t launch_unpack_q8_0(LinWeights W, int row0, int rows, uint8_t* out, hipStream_t s);
hipError_t launch_fill_normal(int act, void* dst, int64_t n, uint64_t seed, float std,
                              hipStream_t s);
hipError_t launch_fill_i32(int32_t* dst, int64_t n, int32_t v, hipStream_t s);

// Audio path (encoder_kernels.hip).  mel (windows, n_mels, frames) in src_dtype (0
// f32, 1 f16, 2 bf16) -> (windows * (frames + 2), cp) time-major rows in the
// activation dtype, one zero row before and after each window's frames and
// channels past n_mels zero.
hipError_t launch_mel_pack(int act, const void* mel, int src_dtype, int windows, int n_mels,
                           int frames, int cp, void* out, hipStream_t s);
// conv1d weight (cout, cin, 3) in src_dtype -> f32 (cout, 3 cinp): element
// (o, k cinp + c) = w[o][c][k], zero for c >= cin.
hipError_t launch_conv_weight(const void* src, int src_dtype, int cout, int cin, int cinp,
                              float* dst, hipStream_t s);
// LayerNorm with gain w and bias b (activation dtype) over rows of dim.
hipError_t launch_layernorm(int act, const void* x, int ldx, const void* w, const void* b,
                            int rows, int dim, float eps, void* y, int ldy, hipStream_t s);
hipError_t launch_enc_attn(int act, const EncAttnArgs& a, int heads, int windows, hipStream_t s);

// Number of argmax partial keys the EPI_LOGITS projection writes per row.
// Work-groups (= argmax partials per row) of the EPI_LOGITS projection.
int gemv_logits_nparts(int act, bool q8, bool norm, int hidden, int out_rows);
