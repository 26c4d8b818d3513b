/*
 * CPU oracle for the AccelEP SimDevice hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and there only to check results. The product path (accelep_amd/)
 * never links or calls it.
 *
 * Each function restates the reference algorithm in plain C, compiled with
 * -ffp-contract=off so every float product is rounded before its add, as the
 * reference's split multiply-then-add order requires. References are
 * path:line in the AccelEP tree.
 *
 * Pinning (how each function is checked, so a plausible mistake fails a test):
 *   orc_reference_matmul   KATs {19,22,43,50} and 0xB5200000 (tests/test_runtime.cc:39-46,413-425),
 *                          bit-exact vs the compiled reference (oracle/_ref) on the LCG fixtures.
 *   orc_dequant_at /
 *   orc_matmul_quantized   DQ KAT -48.5 (tests/test_ep.py:336-343), bit-exact vs oracle/_ref
 *                          MatMulQuantized on 8x160x300 per-row scale+zero and scalar scale,
 *                          per-column scale, batch-axis planes.
 *   orc_gemm_epilogue      nonfinite bit KATs (tests/test_runtime.cc:427-459), Gemm KAT
 *                          {9,13,21,25}, bit-exact vs oracle/_ref GemmEpilogue incl. erf Gelu.
 *   orc_rmsnorm            double closed form within 1e-6 (tests/test_sim_kernels.cc:26-41),
 *                          bit-exact vs oracle/_ref.
 *   orc_embed/rope/append/attention/silu_mul/add
 *                          hand values (tests/test_sim_kernels.cc:47-185), bit-exact vs oracle/_ref.
 *   orc_sample_token       integer KATs (tests/test_sim_kernels.cc:187-231), vs oracle/_ref.
 *   orc_rope_tables        bit-exact vs the reference tables (through oracle/_ref llama).
 *   orc_llama_*            greedy ids and logits bit-exact vs oracle/_ref accel_llama_* on
 *                          reduced configs.
 */
#ifndef ACCEL_ORACLE_H_
#define ACCEL_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes shared with the device layer: 0 ok, 1 invalid argument. */
#define ORC_OK 0
#define ORC_INVALID 1

/* accel::QuantPlane (include/accel/runtime.h:71-78) flattened to plain C. */
typedef struct OrcQuantPlane {
  const int8_t* q;
  const float* scale;
  const int8_t* zero; /* NULL when the op has no zero point */
  int32_t rank;
  int64_t shape[8];
  int64_t axis; /* < 0: one scale for the whole tensor */
  int64_t offset;
} OrcQuantPlane;

enum { ORC_ACT_NONE = 0, ORC_ACT_RELU = 1, ORC_ACT_GELU = 2 };

void orc_reference_matmul(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n);
float orc_dequant_at(const OrcQuantPlane* plane, int64_t index);
int orc_matmul_quantized(const float* a, const OrcQuantPlane* a_quant, const float* b, const OrcQuantPlane* b_quant,
                         float* c, int64_t m, int64_t k, int64_t n);
int64_t orc_bias_offset(int32_t rank, const int64_t* shape, int64_t i, int64_t j);
void orc_gemm_epilogue(float* c, int64_t m, int64_t n, float alpha, const float* bias, int32_t bias_rank,
                       const int64_t* bias_shape, float beta, int32_t activation);
void orc_transpose(const float* src, float* dst, int64_t rows, int64_t cols);
void orc_rmsnorm(const float* x, const float* weight, float* y, int64_t rows, int64_t dim, float eps,
                 int64_t row_offset);
int orc_embed(const int32_t* ids, int64_t id_offset, const float* table, float* out, int64_t seq, int64_t hidden,
              int64_t vocab);
void orc_rope(float* states, const float* cos_table, const float* sin_table, int64_t seq, int64_t n_heads,
              int64_t head_dim, int64_t position);
void orc_append_cache(const float* src, float* cache, int64_t seq, int64_t position, int64_t n_heads,
                      int64_t head_dim);
void orc_attention(const float* q, const float* k, const float* v, float* scores, float* out, int64_t seq,
                   int64_t position, int64_t heads, int64_t kv_heads, int64_t head_dim);
void orc_silu_mul(float* gate, const float* up, int64_t count);
void orc_add(float* dest, const float* extra, int64_t count);
void orc_sample_token(const float* logits, int32_t* chosen_ids, int64_t chosen_index, int64_t vocab,
                      float temperature, uint32_t* rng_state, int32_t top_k);
void orc_rope_tables(int32_t context, int32_t head_dim, float theta, float* cos_out, float* sin_out);

/* Llama forward/generate over float weights (src/llama_model.cc:101-131,209-247). */
typedef struct OrcLlama OrcLlama;
typedef struct OrcLlamaConfig {
  int32_t vocab, hidden, layers, heads, kv_heads, intermediate, context;
  float eps, rope_theta;
} OrcLlamaConfig;
enum {
  ORC_W_EMBED = 1, ORC_W_FINAL_NORM = 2, ORC_W_LM_HEAD = 3, ORC_W_ATTN_NORM = 4, ORC_W_POST_NORM = 5,
  ORC_W_Q = 6, ORC_W_K = 7, ORC_W_V = 8, ORC_W_O = 9, ORC_W_GATE = 10, ORC_W_UP = 11, ORC_W_DOWN = 12
};
OrcLlama* orc_llama_create(const OrcLlamaConfig* config);
void orc_llama_destroy(OrcLlama* model);
/* Hugging Face layout: matrices [out, in], norms [dim] with cols == 1. */
int orc_llama_weight(OrcLlama* model, int32_t kind, int32_t layer, const float* data, int64_t rows, int64_t cols);
int orc_llama_generate(OrcLlama* model, const int32_t* prompt, int32_t prompt_count, int32_t max_new, int32_t eos_id,
                       float temperature, uint32_t seed, int32_t top_k, int32_t* out_ids, int32_t* out_count);
int orc_llama_forward_ids(OrcLlama* model, const int32_t* ids, int32_t count, int32_t reset);
/* Copies the current logit row (vocab floats). */
int orc_llama_logits(OrcLlama* model, float* out, int32_t count);

#ifdef __cplusplus
}
#endif

#endif /* ACCEL_ORACLE_H_ */
