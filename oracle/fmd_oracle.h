/*
 * fmd_oracle.h -- CPU restatement of the batched Qwen3 decoder hot path of
 * cnmoro/fast-moss-diarization (crates/fmd-core/src/model/qwen3.rs,
 * model/linear.rs, precision.rs, engine.rs::generate_batch).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  The
 * product library (libfmd_dec.so) never links, loads or calls it.
 *
 * Numerics follow the reference's storage points: every tensor the reference
 * materialises in the activation dtype (f32, f16 or bf16) is rounded to that
 * dtype here at the same point; arithmetic inside one op runs in f32.
 *
 * How each part is pinned (tests/test_oracle.py, tests/golden/):
 *  - conversions: against numpy (f16) and torch (bf16) on special values;
 *  - or_quantize_q8_0: GGML block_q8_0 known answers (ramps, ties, zero
 *    blocks, f16-subnormal and overflowing scales) and an independent numpy
 *    restatement; dequantisation exactness;
 *  - or_build_mask: the reference's own mask tests (qwen3.rs:722-820);
 *  - or_rope_tables / or_rope_apply: closed form and shift invariance;
 *  - or_rmsnorm, or_linear_dense (known answer [3,7]), or_attention
 *    (grouped == expanded heads, repeat_kv order), or_argmax_rows;
 *  - the model (prefill, decode, generate): a second restatement in torch
 *    (tests/torch_ref.py) to 1e-4 in f32, and with the same rounding model
 *    in bf16/f16 to the fp32 summation-order floor.
 * Parity unpinned: how candle 0.11.0 (absent here) rounds INSIDE its bf16/f16
 * kernels (rms_norm, rope, silu, softmax_last_dim, QMatMul's activation
 * handling) and its argmax tie-break; the oracle rounds each op's output once
 * and breaks ties to the first index.
 */
#ifndef FMD_ORACLE_H
#define FMD_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Precision (precision.rs:10-17).  INT8 = Q8_0 weights + f16 activations. */
enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2, OR_INT8 = 3 };

/* TextConfig (config.rs:8-28). */
typedef struct or_cfg {
  int32_t vocab_size, hidden_size, intermediate_size, num_hidden_layers;
  int32_t num_attention_heads, num_key_value_heads, head_dim;
  int32_t max_position_embeddings;
  double rms_norm_eps, rope_theta;
  int32_t tie_word_embeddings, attention_bias;
} or_cfg;

typedef struct or_model or_model;
typedef struct or_kv or_kv;

/* --- scalar conversions (IEEE round-to-nearest-even) --------------------- */
uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);
float or_bf16_to_f32(uint16_t h);
float or_round(float x, int prec);             /* storage rounding for prec */
void or_round_array(float* x, int64_t n, int prec);

/* --- Q8_0 (linear.rs:194-201, 239-251 -> QTensor::quantize Q8_0) -------- */
void or_quantize_q8_0(const float* x, int64_t rows, int64_t cols, uint8_t* blocks);
void or_dequantize_q8_0(const uint8_t* blocks, int64_t rows, int64_t cols, float* out);

/* --- single ops, for unit tests ----------------------------------------- */
void or_rope_tables(int head_dim, double theta, int max_len, int prec,
                    float* cos_out, float* sin_out);
void or_rope_apply(float* x, int b, int heads, int t, int hd, int offset, const float* cos_t,
                   const float* sin_t, int prec);
void or_build_mask(int batch, int repeat, int q_offset, int q_len, int kv_len,
                   const int32_t* pad, float* out);
void or_rmsnorm(const float* x, const float* w, int64_t rows, int dim, float eps,
                int prec, float* y);
void or_linear_dense(const float* x, const float* w, int64_t rows, int in, int out,
                     int prec, float* y);
void or_linear_q8_0(const float* x, const uint8_t* blocks, int64_t rows, int in,
                    int out, int prec, float* y);
void or_attention(const float* q, const float* k, const float* v, const float* mask,
                  int b, int heads, int kv_heads, int t, int kv_len, int kv_stride,
                  int hd, int prec, float* out);

/* --- model (qwen3.rs:342-511) ------------------------------------------- */
or_model* or_model_new(const or_cfg* cfg, int prec, int max_len);
void or_model_free(or_model* m);
/* Names as in the checkpoint (qwen3.rs:355-372), with or without the
 * "model.language_model." prefix.  `data` is the f32 source tensor. */
int or_model_set(or_model* m, const char* name, const float* data);
int or_model_ready(const or_model* m);
/* Synthetic weights generated in place (CPU baseline only). */
int or_model_fill_random(or_model* m, uint64_t seed, float std);
const char* or_last_error(void);

or_kv* or_kv_new(const or_model* m, int batch, int capacity);
void or_kv_free(or_kv* kv);
int or_kv_len(const or_kv* kv);
/* Copy layer `layer`'s K (which=0) or V (which=1) cache, (B, kvh, cap, hd). */
int or_kv_read(const or_kv* kv, int layer, int which, float* out);
/* Overwrite a layer's K/V (used to synthesise a long context) and set len. */
int or_kv_write(or_kv* kv, int layer, int which, const float* src);
int or_kv_set_len(or_kv* kv, int len);
/* Synthetic N(0,1) context at [0, len) of every row (for the CPU baseline). */
int or_kv_fill_random(or_kv* kv, uint64_t seed, int len, int prec);

void or_embed(const or_model* m, const uint32_t* ids, int64_t n, float* out);
/* prefill (qwen3.rs:475-496) + logits (459-463): embeds (B,P,H) left-padded;
 * `block` query rows per pass (PREFILL_BLOCK = 256 in the reference). */
int or_prefill(or_model* m, or_kv* kv, const float* embeds, const int32_t* pad,
               int batch, int total, int block, float* logits);
/* decode_step (qwen3.rs:499-511) at offset kv->len. */
int or_decode_step(or_model* m, or_kv* kv, const uint32_t* ids, const int32_t* pad,
                   int batch, float* logits);
/* One decoder layer (Layer::forward, qwen3.rs:322-339) for one new token per
 * row at offset kv->len, as decode_step runs layer `layer`
 * (qwen3.rs:499-511, decode mask of build_mask, qwen3.rs:523-562): x (B, H)
 * is the layer input in the activation dtype's values and receives the
 * output; the new K/V land at kv->len, which is not advanced. */
int or_layer_decode(or_model* m, or_kv* kv, int layer, float* x, const int32_t* pad, int batch);
/* The final RMSNorm (qwen3.rs:455) and logits (459-463) of `rows` rows x. */
void or_final_logits(const or_model* m, const float* x, int rows, float* logits);
/* argmax_rows (engine.rs:550-559): first index of the maximum. */
void or_argmax_rows(const float* logits, int rows, int vocab, uint32_t* out);
/* generate_batch (engine.rs:463-541).  embeds (B,P,H) already left-padded by
 * `pad`; tokens (B, budget); finish: 0 = Length, 1 = Stop.  force_eot_step
 * (may be NULL): at greedy step s == force_eot_step[b] row b's argmax is
 * replaced by eos (synthetic end-of-turn for benchmarks). */
int or_generate(or_model* m, const float* embeds, const int32_t* pad, int batch,
                int total, int block, int budget, uint32_t eos,
                const int32_t* force_eot_step, uint32_t* tokens, int32_t* ntok,
                int32_t* finish);

void or_set_threads(int n);

/* --- audio path (fmd_oracle_encoder.c): Whisper encoder, VqAdaptor and the
 * chunk reassembly of MossModel::encode_audio ----------------------------- */

/* AudioConfig (config.rs:60-75) and the adaptor widths MossModel::load passes
 * (mod.rs:47-53): adaptor_input_dim = d_model * audio_merge_size, the text
 * hidden size, and the text rms_norm_eps as the adaptor's LayerNorm eps. */
typedef struct or_audio_cfg {
  int32_t num_mel_bins, d_model, encoder_layers, encoder_attention_heads, encoder_ffn_dim;
  int32_t max_source_positions, adaptor_input_dim, hidden_size, audio_merge_size;
  double norm_eps;
} or_audio_cfg;
typedef struct or_enc or_enc;

void or_conv1d(const float* x, const float* w, int b, int cin, int cout, int t, int stride,
               int prec, float* out);
void or_gelu_erf(float* x, int64_t n, int prec);
void or_silu(float* x, int64_t n, int prec);
void or_layernorm(const float* x, const float* w, const float* bias, int64_t rows, int dim,
                  float eps, int prec, float* y);
void or_attention_dense(const float* q, const float* k, const float* v, int t, int heads, int hd,
                        int prec, float* out);

or_enc* or_enc_new(const or_audio_cfg* cfg, int prec);
void or_enc_free(or_enc* e);
/* Full checkpoint names: model.whisper_encoder.* and model.vq_adaptor.*. */
int or_enc_set(or_enc* e, const char* name, const float* data);
int or_enc_ready(const or_enc* e);
const char* or_enc_last_error(void);
/* Stem: mel (b, n_mels, frames) -> x (b, frames/2, d). */
int or_enc_stem(or_enc* e, const float* mel, int b, int frames, float* x);
/* Layers [first, first + n) in place on x (windows, t, d), then the final
 * LayerNorm when final_norm. */
int or_enc_layers(or_enc* e, float* x, int windows, int t, int first, int n, int final_norm);
/* WhisperEncoder::forward: mel (b, n_mels, frames) -> out (b, frames/2, d). */
int or_enc_forward(or_enc* e, const float* mel, int b, int frames, float* out);
/* VqAdaptor::merge_and_project of one audio's frames (rows, d). */
int or_enc_adaptor(or_enc* e, const float* frames, int rows, float* out);
/* MossModel::encode_audio: out rows of all audios back to back, offsets
 * (num_audios + 1). */
int or_enc_encode_audio(or_enc* e, const float* mel, int n_chunks, int frames,
                        const int32_t* chunk_tokens, const int32_t* chunk_mapping, int num_audios,
                        float* out, int64_t* offsets);

#ifdef __cplusplus
}
#endif
#endif
