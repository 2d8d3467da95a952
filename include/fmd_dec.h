/*
 * fmd_dec.h -- C ABI of the MI355X (gfx950) batched Qwen3 decoder.
 *
 * Drop-in for the decoder path of cnmoro/fast-moss-diarization: the Rust type
 * `Qwen3` + `KvCache` (crates/fmd-core/src/model/qwen3.rs), the dense/Q8_0
 * linears it uses (model/linear.rs) and the greedy loop of
 * `Engine::generate_batch` (engine.rs:463-559).  Each entry point below names
 * the reference item it replaces.
 *
 * Conventions
 *  - Every call returns 0 on success and a negative status on failure; the
 *    message is available from fmd_last_error() (thread-local).
 *  - Host pointers unless a parameter says "device".  Calls that return host
 *    data are synchronous.  One HIP stream per decoder handle; a handle is not
 *    re-entrant (callers serialise, as the reference's Mutex<Engine> does,
 *    fmd-py/src/lib.rs:178-183).
 *  - Activation dtype per precision (precision.rs:32-41): F32 -> f32,
 *    F16 -> f16, BF16 -> bf16, INT8 -> f16 activations, KV and embedding with
 *    Q8_0 weights for every decoder linear and the lm_head.
 */
#ifndef FMD_DEC_H
#define FMD_DEC_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define FMD_OK 0
#define FMD_ERR_ARG -1      /* bad argument / shape            */
#define FMD_ERR_STATE -2    /* missing weights, wrong handle   */
#define FMD_ERR_HIP -3      /* HIP runtime failure             */
#define FMD_ERR_OOM -4      /* device allocation failed        */
#define FMD_ERR_OVERFLOW -5 /* KV cache overflow (qwen3.rs:88-94) */

/* Precision (precision.rs:10-17). */
typedef enum { FMD_F32 = 0, FMD_F16 = 1, FMD_BF16 = 2, FMD_INT8 = 3 } fmd_precision;
/* Element type of a host/device buffer handed to the library. */
typedef enum { FMD_DT_F32 = 0, FMD_DT_F16 = 1, FMD_DT_BF16 = 2 } fmd_dtype;

/* TextConfig (config.rs:8-28).  head_dim must be 128; hidden_size,
 * intermediate_size and num_attention_heads*head_dim must be multiples of
 * 256; vocab_size a multiple of 16; heads/kv_heads in {1, 2, 4}. */
typedef struct fmd_text_config {
  int32_t vocab_size;
  int32_t hidden_size;
  int32_t intermediate_size;
  int32_t num_hidden_layers;
  int32_t num_attention_heads;
  int32_t num_key_value_heads;
  int32_t head_dim;
  int32_t max_position_embeddings;
  double rms_norm_eps;
  double rope_theta;
  int32_t tie_word_embeddings;
  int32_t attention_bias; /* must be 0 (Qwen3) */
} fmd_text_config;

typedef struct fmd_dec fmd_dec;
typedef struct fmd_kv fmd_kv;

const char* fmd_last_error(void);

/* --- model ------------------------------------------------------------- */

/* Qwen3::load (qwen3.rs:354-390) without the file I/O: allocates the model on
 * HIP device `device` with RoPE tables for `max_len` positions (Rope::new,
 * qwen3.rs:117-136; the engine passes min(max_position_embeddings, 65536),
 * engine.rs:239-243).  Weights arrive through fmd_dec_set_weight. */
int fmd_dec_create(const fmd_text_config* cfg, fmd_precision precision, int device, int max_len,
                   fmd_dec** out);
int fmd_dec_destroy(fmd_dec* dec);

/* Route all work of this handle to an existing HIP stream (hipStream_t);
 * NULL restores the handle's own stream. */
int fmd_dec_set_stream(fmd_dec* dec, void* hip_stream);
void* fmd_dec_stream(const fmd_dec* dec);

/* Watchdog of the decode attention (no counterpart in the reference, whose
 * kernels do not wait on each other): the work-groups of one (row, KV head)
 * exchange partial results inside one launch, and a wait that is not met
 * within `polls` polls (about a microsecond each; default 20000) gives up,
 * so the launch drains and the call fails with an error instead of hanging.
 * 0 gives up at the first unmet poll (used by the tests of that path). */
int fmd_dec_set_spin_limit(fmd_dec* dec, int polls);

/* Loader::linear_with / fused_linear / get / build_tied_head
 * (linear.rs:166-265, qwen3.rs:355-372, 566-578).  `name` is the checkpoint
 * name (with or without "model.language_model."), e.g.
 * "layers.3.self_attn.q_proj.weight", "norm.weight", "embed_tokens.weight",
 * "lm_head.weight".  `data` is host memory, or device memory when
 * `data_on_device` != 0, in `dtype`.  Linears are stored fused (q|k|v and
 * gate|up, as FusedLinear); in INT8 they are quantised to Q8_0 from the f32
 * value of the source, bit-exactly as QTensor::quantize.  Without an explicit
 * lm_head the output projection is tied to embed_tokens (a Q8_0 copy in INT8,
 * a dense copy otherwise). */
int fmd_dec_set_weight(fmd_dec* dec, const char* name, fmd_dtype dtype, const int64_t* shape,
                       int ndim, const void* data, int data_on_device);
/* 1 when every tensor the decoder needs has been set. */
int fmd_dec_ready(const fmd_dec* dec);
/* Device bytes of the decoder linears + lm_head as stored (Q8_0 blocks count
 * 34 bytes per 32 weights). */
int fmd_dec_weight_bytes(const fmd_dec* dec, size_t* out);
/* A quantised projection's rows as GGML block_q8_0 bytes (34 B per 32
 * weights), for bit-exact checks.  `name` as for set_weight; fused parts
 * return their own rows. */
int fmd_dec_get_q8_0(const fmd_dec* dec, const char* name, void* out_blocks);

/* Q8_0 quantisation on the host (QTensor::quantize, linear.rs:197, 246):
 * rows x cols f32 (cols % 32 == 0) -> rows*cols/32 blocks of 34 bytes. */
int fmd_quantize_q8_0(const float* src, int64_t rows, int64_t cols, void* out_blocks);

/* --- KV cache (qwen3.rs:33-108, 415-440) -------------------------------- */

/* new_caches: all layers' K and V, (batch, kv_heads, capacity, head_dim) in
 * the activation dtype, zero-initialised.  capacity <= 65536 (the engine's
 * RoPE table bound, engine.rs:239-243). */
int fmd_kv_create(fmd_dec* dec, int batch, int capacity, fmd_kv** out);
int fmd_kv_destroy(fmd_kv* kv);
/* cache_bytes (qwen3.rs:431-440). */
size_t fmd_kv_bytes(const fmd_dec* dec, int batch, int capacity);
/* KvCache::len / truncate (qwen3.rs:57, 105-107). */
int fmd_kv_len(const fmd_kv* kv);
int fmd_kv_truncate(fmd_kv* kv, int len);
/* Raw copies of one layer's K (which = 0) or V (which = 1) cache in the
 * activation dtype, (batch, kv_heads, capacity, head_dim). */
int fmd_kv_read(const fmd_kv* kv, int layer, int which, void* host_out);
int fmd_kv_write(fmd_kv* kv, int layer, int which, const void* host_src);
/* Synthetic context for benchmarks: fill every layer's K and V with
 * N(0, 1) values (seeded, on the device) and set the length. */
int fmd_kv_fill_random(fmd_kv* kv, uint64_t seed, int len);
/* Set the length (write cursor) without touching the contents. */
int fmd_kv_set_len(fmd_kv* kv, int len);

/* --- forward ------------------------------------------------------------ */

/* Qwen3::embed (qwen3.rs:405-412): ids -> (n, hidden) activation-dtype rows. */
int fmd_dec_embed(fmd_dec* dec, const uint32_t* ids, int64_t n, void* host_out);

/* Prompt assembly on the device for one micro-batch:
 * MossTranscribeDiarize::splice_audio (mod.rs:128-180) per row, then the
 * engine's left pad to a common length (engine.rs:476-491).  Row b's prompt
 * is ids[offsets[b] .. offsets[b+1]) (offsets has batch+1 entries).  Its
 * positions holding audio_token_id take, in order, rows audio_first[b] ..
 * audio_first[b] + audio_count[b] - 1 of `audio` (n_audio rows of hidden
 * values, audio_dtype 0 f32 / 1 f16 / 2 bf16, host memory or device memory
 * when audio_on_device), rounded to the activation dtype; its other positions
 * take their token embedding.  Writes (batch, total, hidden) activation-dtype
 * rows to the device buffer `out` (row b left-padded with zeros) and
 * pad[b] = total - length of prompt b to `pad` (host, may be NULL): the
 * inputs of fmd_dec_prefill / fmd_dec_generate with embeds_on_device.  A row
 * whose placeholder count differs from audio_count[b] fails with the
 * reference's message.  audio_first / audio_count may be NULL when no prompt
 * has placeholders. */
int fmd_dec_assemble(fmd_dec* dec, const uint32_t* ids, const int64_t* offsets, int batch,
                     const void* audio, int audio_dtype, int audio_on_device, int64_t n_audio,
                     const int64_t* audio_first, const int64_t* audio_count,
                     uint32_t audio_token_id, int total, void* out_device, int32_t* pad);

/* Qwen3::prefill + Qwen3::logits (qwen3.rs:475-496, 459-463).  `embeds` is
 * (batch, total, hidden) left-padded in the activation dtype (host, or device
 * when embeds_on_device); pad[b] = left padding of row b.  Queries are taken
 * `chunk` positions at a time (the reference uses 256; pad rows are exactly
 * zero in the reference and are skipped).  Writes f32 logits (batch, vocab)
 * of each row's last position to `logits` (host) when non-NULL.  The cache
 * must be empty; its length becomes `total`. */
int fmd_dec_prefill(fmd_dec* dec, fmd_kv* kv, const void* embeds, int embeds_on_device,
                    const int32_t* pad, int batch, int total, int chunk, float* logits);

/* Qwen3::decode_step (qwen3.rs:499-511): one token per row at offset
 * kv_len; f32 logits (batch, vocab) to `logits` (host) when non-NULL. */
int fmd_dec_decode_step(fmd_dec* dec, fmd_kv* kv, const uint32_t* ids, const int32_t* pad,
                        int batch, float* logits);

/* Greedy generation over a left-padded batch: Engine::generate_batch
 * (engine.rs:463-541) from the prefill on.  argmax (ties -> smallest index),
 * end-of-turn tracking and feeding eos to finished rows run on the device;
 * finished rows are retired from attention.  tokens: (batch, budget);
 * ntok[b] tokens kept per row; finish[b]: 0 = Length, 1 = Stop.
 * force_eot_step (may be NULL): row b's argmax is replaced by eos at greedy
 * step force_eot_step[b] (synthetic end-of-turn).  Any batch size: above 16
 * rows, groups of 16 rows run one after another over the same padded length,
 * which gives each row the tokens of one batched run.  Decode positions come
 * from the RoPE table (max_len of fmd_dec_create): if rows are still
 * generating when position max_len would be written, the call fails, as the
 * reference's decode_step does at Rope::apply (qwen3.rs:139-144). */
int fmd_dec_generate(fmd_dec* dec, const void* embeds, int embeds_on_device, const int32_t* pad,
                     int batch, int total, int chunk, int budget, uint32_t eos,
                     const int32_t* force_eot_step, uint32_t* tokens, int32_t* ntok,
                     int32_t* finish);

/* The greedy loop alone, from an existing cache (a prefilled or synthetic
 * context): `first_ids` are fed at the first decode step, which writes
 * position kv_len.  Runs at most `max_steps` decode steps; each step is one
 * graph launch (decode step + greedy update), and the host looks at the
 * done-count every step without blocking the stream.  steps_run receives the
 * number of decode steps executed. */
int fmd_dec_decode_loop(fmd_dec* dec, fmd_kv* kv, const uint32_t* first_ids, const int32_t* pad,
                        int batch, int max_steps, uint32_t eos, const int32_t* force_eot_step,
                        uint32_t* tokens, int32_t* ntok, int32_t* finish, int32_t* steps_run);

/* One iteration of the reference's greedy bookkeeping for a host-side loop:
 * argmax_rows + engine.rs:505-531 on the device, over the logits of the last
 * fmd_dec_prefill / fmd_dec_decode_step on this handle (same batch).  For a
 * row not yet done, its token is the argmax (ties -> first index), or eos
 * when force_eot_step[b] == step (force_eot_step may be NULL); eos marks the
 * row done (FinishReason::Stop) and is not emitted.  done[b] (0/1) is read
 * and updated; next_ids[b] receives the id to feed at the next decode step
 * (eos for done rows); emitted[b] (may be NULL) the token emitted this step,
 * or 0xFFFFFFFF. */
int fmd_dec_greedy(fmd_dec* dec, int batch, uint32_t eos, const int32_t* force_eot_step, int step,
                   int32_t* done, uint32_t* next_ids, uint32_t* emitted);

/* --- request scheduling (engine.rs:382-392) ------------------------------ */

/* Generate for `n` token-id prompts (concatenated in `ids`, lengths in
 * `lens`): sort by prompt length (stable), cut into micro-batches of
 * max(max_batch_size, 1) -- with no upper bound, as pending.chunks does
 * (engine.rs:385-387) -- and run generate per micro-batch (prompts embedded
 * on the device, left-padded).  Outputs are indexed by request: tokens (n,
 * budget), ntok, finish; status[i] is 0 or the error of request i's
 * micro-batch (a batch failure is reported against every member,
 * engine.rs:414-421).  error_text (may be NULL) holds n strings of
 * error_stride bytes: request i's is empty or "batch generation failed: {e}"
 * (engine.rs:419), truncated to error_stride - 1 bytes.  force_eot_step is
 * per request (may be NULL). */
typedef struct fmd_batch_stats {
  double generate_seconds;   /* wall time of the call (engine.rs:384, 424) */
  int64_t generated_tokens;
  int32_t micro_batches;
  /* Device time inside generate_seconds (HIP events, summed over the
   * micro-batches; no counterpart in the reference's BatchStats): the
   * prefills up to the first logits, and the greedy decode loops after. */
  double prefill_seconds;
  double decode_seconds;
} fmd_batch_stats;
int fmd_engine_generate(fmd_dec* dec, const uint32_t* ids, const int64_t* lens, int n,
                        int max_batch_size, int budget, uint32_t eos,
                        const int32_t* force_eot_step, int chunk, uint32_t* tokens,
                        int32_t* ntok, int32_t* finish, int32_t* status, char* error_text,
                        int error_stride, fmd_batch_stats* stats);

/* --- single operations on device buffers (used by tests and benchmarks) --- */

/* One decoder linear of layer `layer` on device rows (Linear::forward,
 * linear.rs:29-65): proj 0 = qkv, 1 = o, 2 = gate_up, 3 = down,
 * 4 = lm_head (layer ignored; f32 output).  x (rows, in) and y (rows, out)
 * are device buffers in the activation dtype. */
int fmd_op_linear(fmd_dec* dec, int layer, int proj, const void* x_dev, int rows, void* y_dev);
/* Decode attention of layer `layer` (Attention::forward's q/k norm, RoPE,
 * cache append and attention, qwen3.rs:213-257) for one new token per row:
 * qkv_dev (batch, q_dim + 2*kv_dim) is the raw fused projection on the
 * device; the new K/V are written at position kv_len and the token attends to
 * [pad_b, kv_len]; ctx (batch, heads*head_dim) on the device.  The cache
 * length is not advanced.  Only the attention kernels are launched. */
int fmd_op_attention_decode(fmd_dec* dec, fmd_kv* kv, int layer, const void* qkv_dev,
                            const int32_t* pad, int batch, void* ctx_dev);
/* Decoder layer `layer` for one new token per row, as decode_step runs it
 * (Layer::forward, qwen3.rs:322-339, with the decode mask of build_mask,
 * qwen3.rs:523-562): x_dev (batch, hidden) on the device in the activation
 * dtype is the layer input and receives the layer output; the new K/V are
 * written at position kv_len, which is not advanced, and row b attends to
 * [pad[b], kv_len].  batch <= 16. */
int fmd_op_layer_decode(fmd_dec* dec, fmd_kv* kv, int layer, void* x_dev, const int32_t* pad,
                        int batch);
/* fmd_op_attention_decode without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory -- code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Same arguments, kernels and results as
 * fmd_op_attention_decode; its scratch (launch state, exchange words, split
 * partials, scores, write position, pads) is a static 16 MiB device array per
 * GPU, held until the process ends, and calls fail with FMD_ERR_ARG when the
 * batch and capacity need more (the 0.6B shape fits batch 16 at capacity
 * 8192).  The write position and the pads reach the device as kernel
 * arguments of a set-up kernel, so a graph capture of the call records no
 * host memory (a replay uses the values of the captured call).  On the
 * handle's own stream outside capture the call waits and reports a wait that
 * gave up; under capture or on a caller's stream it returns at once, and such
 * an error is reported by the next synchronous call on that GPU (errors are
 * per device, not per handle).  The array keeps the last call's contents;
 * concurrent calls on one GPU (from any handle or stream) race. */
int fmd_op_attention_decode_noalloc(fmd_dec* dec, fmd_kv* kv, int layer, const void* qkv_dev,
                                    const int32_t* pad, int batch, void* ctx_dev);
/* Final RMSNorm + lm_head (qwen3.rs:455, 459-463) of `rows` (<= 16) device
 * rows x_dev (rows, hidden) in the activation dtype: f32 logits (rows, vocab)
 * to the device buffer logits_dev, rounded to the activation dtype first as
 * Qwen3::logits does. */
int fmd_op_logits(fmd_dec* dec, const void* x_dev, int rows, float* logits_dev);

/* --- audio path: Whisper encoder + VqAdaptor ------------------------------
 *
 * WhisperEncoder (model/whisper_encoder.rs), VqAdaptor (model/adaptor.rs) and
 * MossModel::encode_audio (model/mod.rs:82-126) on the same device.  Every
 * tensor is dense in the activation dtype of the precision (INT8 runs the
 * audio path in f16, whisper_encoder.rs:31-33, adaptor.rs:27-29).  The
 * encoder's head_dim (d_model / encoder_attention_heads) must be 64;
 * encoder_ffn_dim and hidden_size multiples of 64. */

/* AudioConfig (config.rs:60-75) plus the adaptor widths MossModel::load
 * passes (mod.rs:47-53): adaptor_input_dim = d_model * audio_merge_size, the
 * decoder's hidden_size, and the decoder's rms_norm_eps as the adaptor
 * LayerNorm's eps. */
typedef struct fmd_audio_config {
  int32_t num_mel_bins;
  int32_t d_model;
  int32_t encoder_layers;
  int32_t encoder_attention_heads;
  int32_t encoder_ffn_dim;
  int32_t max_source_positions;
  int32_t adaptor_input_dim;
  int32_t hidden_size;
  int32_t audio_merge_size;
  double norm_eps;
} fmd_audio_config;

typedef struct fmd_enc fmd_enc;

/* WhisperEncoder::load + VqAdaptor::load (whisper_encoder.rs:118-138,
 * adaptor.rs:18-35) without the file I/O; weights arrive through
 * fmd_enc_set_weight. */
int fmd_enc_create(const fmd_audio_config* cfg, fmd_precision precision, int device,
                   fmd_enc** out);
int fmd_enc_destroy(fmd_enc* enc);
int fmd_enc_set_stream(fmd_enc* enc, void* hip_stream);
/* Checkpoint names with their prefix: "model.whisper_encoder.conv1.weight"
 * (d_model, num_mel_bins, 3), ..., "model.whisper_encoder.layers.{i}.fc1.bias",
 * "model.vq_adaptor.layers.{0,2,3}.{weight,bias}" (whisper_encoder.rs:27-42,
 * 73-80, 118-138; adaptor.rs:18-35).  k_proj has no bias. */
int fmd_enc_set_weight(fmd_enc* enc, const char* name, fmd_dtype dtype, const int64_t* shape,
                       int ndim, const void* data, int data_on_device);
int fmd_enc_ready(const fmd_enc* enc);
/* WhisperEncoder::forward (whisper_encoder.rs:139-163): n log-mel chunks
 * (n, num_mel_bins, frames) in mel_dtype (host, or device when mel_on_device;
 * cast to the activation dtype first, engine.rs:334-339) -> (n, frames/2,
 * d_model) activation-dtype frames to `out` (host, or device when
 * out_on_device).  frames must be even with frames/2 <= max_source_positions. */
int fmd_enc_forward(fmd_enc* enc, const void* mel, fmd_dtype mel_dtype, int mel_on_device, int n,
                    int frames, void* out, int out_on_device);
/* EncoderLayer::forward (whisper_encoder.rs:82-97) for layers [first,
 * first + n), then the final LayerNorm (whisper_encoder.rs:162) when
 * final_norm: x (windows, t, d_model) activation-dtype hidden states -> out
 * (same shape).  For tests of single layers. */
int fmd_enc_layers(fmd_enc* enc, const void* x, int x_on_device, int windows, int t, int first,
                   int n, int final_norm, void* out, int out_on_device);
/* VqAdaptor::merge_and_project (adaptor.rs:41-64) of one audio's frames
 * (rows, d_model): rows / audio_merge_size merged rows (a trailing partial
 * group dropped) -> (rows / audio_merge_size, hidden_size). */
int fmd_enc_adaptor(fmd_enc* enc, const void* frames, int frames_on_device, int rows, void* out,
                    int out_on_device);
/* MossModel::encode_audio (mod.rs:82-126): every chunk through the encoder,
 * encoder_batch chunks per pass; chunk i keeps min(chunk_tokens[i] *
 * audio_merge_size, frames/2) frames and belongs to audio chunk_mapping[i];
 * each audio's kept frames, joined in chunk order, are merged and projected.
 * Audio a's embeddings are rows offsets[a] .. offsets[a+1] of `out` (host or
 * device, activation dtype, hidden_size wide); offsets has num_audios + 1
 * entries.  With out == NULL only offsets are written (the size query). */
int fmd_enc_encode_audio(fmd_enc* enc, const void* mel, fmd_dtype mel_dtype, int mel_on_device,
                         int n_chunks, int frames, const int32_t* chunk_tokens,
                         const int32_t* chunk_mapping, int num_audios, int encoder_batch,
                         void* out, int out_on_device, int64_t* offsets);

#ifdef __cplusplus
}
#endif
#endif
