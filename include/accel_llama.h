/*
 * The Llama decode loop on one MI355X: weights, activations, the KV cache, the sampler's
 * state and the chosen ids stay in HBM; the host sends prompt ids and receives the chosen
 * ids. Replaces AccelEP's accel_llama_* (include/accel/sim_api.h:38-115, src/llama_model.cc)
 * with the same names, argument meaning and return convention (0 on success, 1 on failure
 * with the message in accel_llama_last_error(); create returns NULL on failure).
 *
 * Every step runs as HIP kernels of libaccel_hip (the same kernels as the accel_hip_* entry
 * points): int8 or fp32 linear layers, RMSNorm, RoPE, KV append, attention, SiLU and the
 * residual adds (fused into the o and down projections' stores), and the sampler. The
 * tokenizer calls encode and decode on the host (a byte-level BPE of a Hugging Face
 * tokenizer.json in the SmolLM2 form, src/bpe.cc) around the same generate loop.
 */
#ifndef ACCEL_LLAMA_H_
#define ACCEL_LLAMA_H_

#include <stdint.h>

#define ACCEL_LLAMA_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

typedef struct AccelLlama AccelLlama;

/* AccelLlamaConfig (include/accel/sim_api.h:42-52). */
typedef struct AccelLlamaConfig {
  int32_t vocab;
  int32_t hidden;
  int32_t layers;
  int32_t heads;
  int32_t kv_heads;
  int32_t intermediate;
  int32_t context;
  float eps;
  float rope_theta;
} AccelLlamaConfig;

/* Weight kinds (include/accel/sim_api.h:54-67). */
enum {
  ACCEL_W_EMBED = 1,
  ACCEL_W_FINAL_NORM = 2,
  ACCEL_W_LM_HEAD = 3,
  ACCEL_W_ATTN_NORM = 4,
  ACCEL_W_POST_NORM = 5,
  ACCEL_W_Q = 6,
  ACCEL_W_K = 7,
  ACCEL_W_V = 8,
  ACCEL_W_O = 9,
  ACCEL_W_GATE = 10,
  ACCEL_W_UP = 11,
  ACCEL_W_DOWN = 12
};

ACCEL_LLAMA_API AccelLlama* accel_llama_create(const AccelLlamaConfig* config);
ACCEL_LLAMA_API void accel_llama_destroy(AccelLlama* model);
/* Hugging Face layout: matrices [out, in], norms [dim] with cols == 1 (sim_api.h:72-73).
 * Matrices are held transposed, [in, out], in fp32. */
ACCEL_LLAMA_API int accel_llama_weight(AccelLlama* model, int32_t kind, int32_t layer, const float* data, int64_t rows,
                                       int64_t cols);
/* An int8 matrix with one fp32 scale per output row: w[o, i] = q[o, i] * row_scale[o]
 * (no reference counterpart as a call; the reference receives these same values as the
 * floats fl(q * s)). Held as int8 [in, out] with a per-column scale; the embedding keeps
 * [vocab, hidden] with a per-row scale. Not for norms. */
ACCEL_LLAMA_API int accel_llama_weight_q8(AccelLlama* model, int32_t kind, int32_t layer, const int8_t* q,
                                          const float* row_scale, int64_t rows, int64_t cols);
/* accel_llama_generate (sim_api.h:79-84): prefill the prompt, then sample up to max_new ids
 * (stopping at eos_id or a full context); the ids are copied back once at the end. */
ACCEL_LLAMA_API int accel_llama_generate(AccelLlama* model, const int32_t* prompt, int32_t prompt_count,
                                         int32_t max_new, int32_t eos_id, float temperature, uint32_t seed,
                                         int32_t top_k, int32_t* out_ids, int32_t* out_count);
/* accel_llama_tokenizer (sim_api.h:76-77, src/llama_model.cc:449-464): load a Hugging Face
 * tokenizer.json (model BPE; no normalizer or post-processor; pre-tokenizer Digits with
 * individual digits then ByteLevel without prefix space; ByteLevel decoder). */
ACCEL_LLAMA_API int accel_llama_tokenizer(AccelLlama* model, const char* path);
/* accel_llama_encode (sim_api.h:84-88, src/llama_model.cc:466-492): ids of text_len bytes
 * (NUL allowed; not valid UTF-8 is an error); fails with "encode buffer is too small" when
 * out_cap is below the count. */
ACCEL_LLAMA_API int accel_llama_encode(AccelLlama* model, const char* text, int32_t text_len, int32_t* out_ids,
                                       int32_t out_cap, int32_t* out_count);
/* accel_llama_decode (sim_api.h:89-91, src/llama_model.cc:494-519): UTF-8 text of the ids
 * (skip_special nonzero leaves out special tokens; invalid UTF-8 comes out as U+FFFD per
 * byte), *out_len bytes with no trailing NUL; "decode buffer is too small" past out_cap. */
ACCEL_LLAMA_API int accel_llama_decode(AccelLlama* model, const int32_t* ids, int32_t count, int32_t skip_special,
                                       char* out_text, int32_t out_cap, int32_t* out_len);
/* accel_llama_complete (sim_api.h:92-98, src/llama_model.cc:521-527, :183-206): encode the
 * prompt (prompt_len bytes, NUL allowed), generate as accel_llama_generate does, and decode
 * the chosen ids without special tokens. out_ids_cap must be at least max_new; the prompt
 * must encode to 1 .. context ids. Counted copies: the prompt ids in, the ids and the text
 * back. */
ACCEL_LLAMA_API int accel_llama_complete(AccelLlama* model, const char* prompt, int32_t prompt_len, int32_t max_new,
                                         int32_t eos_id, float temperature, uint32_t seed, int32_t top_k,
                                         char* out_text, int32_t out_text_cap, int32_t* out_text_len, int32_t* out_ids,
                                         int32_t out_ids_cap, int32_t* out_count, int32_t* prompt_tokens);
/* AccelLlamaTokenFn (sim_api.h:99-101): called with each chosen id once it has been read
 * back (an uncounted read), before the eos check; it must not call back into the model. */
typedef void (*AccelLlamaTokenFn)(int32_t token_id, void* user);
/* accel_llama_complete_stream (sim_api.h:102-108, src/llama_model.cc:530-551): the same result
 * as accel_llama_complete, with on_token (may be NULL) called per id. */
ACCEL_LLAMA_API int accel_llama_complete_stream(AccelLlama* model, const char* prompt, int32_t prompt_len,
                                                int32_t max_new, int32_t eos_id, float temperature, uint32_t seed,
                                                int32_t top_k, char* out_text, int32_t out_text_cap,
                                                int32_t* out_text_len, int32_t* out_ids, int32_t out_ids_cap,
                                                int32_t* out_count, int32_t* prompt_tokens, AccelLlamaTokenFn on_token,
                                                void* user);
/* Test seams (sim_api.h:106-112): a forward over ids (reset nonzero clears the cache) that
 * leaves the last row's logits on the device, and max |logits - reference|. */
ACCEL_LLAMA_API int accel_llama_forward_ids(AccelLlama* model, const int32_t* ids, int32_t count, int32_t reset);
ACCEL_LLAMA_API int accel_llama_logit_max_abs(AccelLlama* model, const float* reference, int32_t count,
                                             float* out_max_abs);
/* Uncounted read of the logit row (no reference counterpart; for tests). */
ACCEL_LLAMA_API int accel_llama_logits(AccelLlama* model, float* out, int32_t count);
/* No reference counterpart (a test seam) for a one-row (decode) forward. enable is a bit
 * mask, default 7. Bit 0: the RMSNorms and SiLU*up run inside the next int8 GEMV (the norm is
 * applied to the product's sums, which rounds differently from normalizing first) instead of
 * as separate kernels. Bit 1: RoPE + KV append, attention and chunk combine run as one kernel
 * instead of three (same bits). Bit 2 (not in exact-products mode; over bit 1): the attention
 * runs in a fixed number of position splits and the o-projection GEMV combines their partials
 * in its input prologue (softmax sums in another order: rounding only). Values outside
 * 0 .. 7 are an invalid argument. */
ACCEL_LLAMA_API int accel_llama_set_fused_inputs(AccelLlama* model, int32_t enable);
ACCEL_LLAMA_API void accel_llama_reset(AccelLlama* model);
ACCEL_LLAMA_API const char* accel_llama_last_error(void);
/* The stats serve/llama.py reads beside these calls (accel_sim_reset_stats, accel_sim_matmuls,
 * accel_sim_bytes_to_device / _to_host) are declared in accel_sim.h. */

#ifdef __cplusplus
}
#endif

#endif /* ACCEL_LLAMA_H_ */
