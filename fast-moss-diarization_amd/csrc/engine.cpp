// Request scheduling of Engine::transcribe (engine.rs:382-424): sort the
// prompts by length, cut them into micro-batches and run generate_batch on
// each, plus the host Q8_0 quantiser.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <numeric>
#include <string>
#include <vector>

#include "fmd_dec.h"
#include "fmd_internal.h"
#include "fmd_kernels.h"

// QTensor::quantize(Q8_0) on the host (linear.rs:197, 246): per 32-value
// block, d = max|x| / 127, id = d != 0 ? 1/d : 0, q = round-half-away(x * id)
// with a saturating cast (NaN -> 0), d stored as f16.
void host_quantize_q8_0(const float* src, int64_t rows, int64_t cols, uint8_t* out) {
  const int64_t nb = cols / 32;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const float* xs = src + r * cols + b * 32;
      uint8_t* blk = out + (r * nb + b) * 34;
      float amax = 0.f;
      for (int j = 0; j < 32; ++j) amax = std::fmax(amax, std::fabs(xs[j]));
      const float d = amax / 127.0f;
      const float id = d != 0.f ? 1.0f / d : 0.f;
      const uint16_t dh = host_f32_to_f16(d);
      blk[0] = (uint8_t)(dh & 0xff);
      blk[1] = (uint8_t)(dh >> 8);
      for (int j = 0; j < 32; ++j) {
        const float v = std::round(xs[j] * id);
        int8_t q;
        if (v != v) q = 0;
        else if (v >= 127.f) q = 127;
        else if (v <= -128.f) q = -128;
        else q = (int8_t)v;
        blk[2 + j] = (uint8_t)q;
      }
    }
}

extern "C" int fmd_engine_generate(fmd_dec* d, const uint32_t* ids, const int64_t* lens, int n,
                                   int max_batch_size, int budget, uint32_t eos,
                                   const int32_t* force, int chunk, uint32_t* tokens,
                                   int32_t* ntok, int32_t* finish, int32_t* status,
                                   char* error_text, int error_stride, fmd_batch_stats* stats) {
  if (!d || (n > 0 && (!ids || !lens || !tokens || !ntok || !finish || !status)))
    return fmd_fail(FMD_ERR_ARG, "null argument");
  if (budget < 1) return fmd_fail(FMD_ERR_ARG, "budget must be >= 1");
  if (eos >= (uint32_t)d->V) return fmd_fail(FMD_ERR_ARG, "eos id outside the vocabulary");
  if (error_text && error_stride < 1) return fmd_fail(FMD_ERR_ARG, "error_stride must be >= 1");
  // pending.chunks(max_batch_size.max(1)) (engine.rs:387): no upper bound;
  // fmd_dec_generate runs a micro-batch above 16 rows as 16-row groups.
  const int mbs = std::max(max_batch_size, 1);
  const auto t0 = std::chrono::steady_clock::now();
  std::vector<int64_t> off(n + 1, 0);
  for (int i = 0; i < n; ++i) {
    if (lens[i] < 0) return fmd_fail(FMD_ERR_ARG, "negative prompt length");
    off[i + 1] = off[i] + lens[i];
  }
  for (int64_t i = 0; i < off[n]; ++i)
    if (ids[i] >= (uint32_t)d->V) return fmd_fail(FMD_ERR_ARG, "token id out of range");
  // pending.sort_by_key(|p| p.tokens.len()) is a stable sort (engine.rs:385).
  std::vector<int> order(n);
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return lens[a] < lens[b]; });
  if (stats) *stats = fmd_batch_stats{};
  d->t_prefill = d->t_decode = 0.0;
  for (int i = 0; i < n; ++i) {
    ntok[i] = 0;
    finish[i] = 0;
    status[i] = 0;
    if (error_text) error_text[(size_t)i * error_stride] = 0;
  }
  std::vector<uint32_t> gtok;
  std::vector<int32_t> gnt, gfin, gforce, pad;
  for (int g0 = 0; g0 < n; g0 += mbs) {
    const int B = std::min(mbs, n - g0);
    if (stats) stats->micro_batches += 1;
    int P = 0;
    for (int j = 0; j < B; ++j) P = std::max<int>(P, (int)lens[order[g0 + j]]);
    pad.assign(B, 0);
    gforce.assign(B, -1);
    for (int j = 0; j < B; ++j) {
      pad[j] = P - (int)lens[order[g0 + j]];
      if (force) gforce[j] = force[order[g0 + j]];
    }
    int rc = 0;
    if (P == 0) rc = fmd_fail(FMD_ERR_ARG, "empty prompt");
    // Left-pad the prompt embeddings into one (B, P, H) device buffer (engine.rs:476-491).
    if (!rc) rc = d->ws.embeds.ensure((size_t)B * P * d->H * d->esz);
    if (!rc) rc = d->ws.ids.ensure((size_t)std::max<int64_t>(off[n], 1) * 4);
    if (!rc && hipMemsetAsync(d->ws.embeds.p, 0, (size_t)B * P * d->H * d->esz, d->stream) != hipSuccess)
      rc = fmd_fail(FMD_ERR_HIP, "memset failed");
    if (!rc && off[n] > 0 &&
        hipMemcpyAsync(d->ws.ids.p, ids, (size_t)off[n] * 4, hipMemcpyHostToDevice, d->stream) != hipSuccess)
      rc = fmd_fail(FMD_ERR_HIP, "id upload failed");
    for (int j = 0; j < B && !rc; ++j) {
      const int r = order[g0 + j];
      if (lens[r] == 0) continue;
      char* dst = (char*)d->ws.embeds.p + ((size_t)j * P + pad[j]) * d->H * d->esz;
      if (launch_embed(d->act, d->ws.ids.as<uint32_t>() + off[r], (int)lens[r], d->embed, d->H, dst,
                       d->stream) != hipSuccess)
        rc = fmd_fail(FMD_ERR_HIP, "embed launch failed");
    }
    gtok.assign((size_t)B * budget, 0);
    gnt.assign(B, 0);
    gfin.assign(B, 0);
    if (!rc)
      rc = fmd_dec_generate(d, d->ws.embeds.p, 1, pad.data(), B, P, chunk, budget, eos,
                            force ? gforce.data() : nullptr, gtok.data(), gnt.data(), gfin.data());
    // A batch failure is reported against every member, as
    // "batch generation failed: {e}" (engine.rs:414-421).
    const std::string msg = rc ? "batch generation failed: " + std::string(fmd_last_error()) : "";
    for (int j = 0; j < B; ++j) {
      const int r = order[g0 + j];
      if (rc) {
        status[r] = rc;
        if (error_text) {
          char* dst = error_text + (size_t)r * error_stride;
          const size_t k = std::min(msg.size(), (size_t)error_stride - 1);
          std::memcpy(dst, msg.data(), k);
          dst[k] = 0;
        }
        continue;
      }
      ntok[r] = gnt[j];
      finish[r] = gfin[j];
      std::copy(gtok.begin() + (size_t)j * budget, gtok.begin() + (size_t)(j + 1) * budget,
                tokens + (size_t)r * budget);
      if (stats) stats->generated_tokens += gnt[j];
    }
  }
  if (stats) {
    stats->generate_seconds =
        std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    stats->prefill_seconds = d->t_prefill;
    stats->decode_seconds = d->t_decode;
  }
  return 0;
}
