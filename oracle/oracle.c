/*
 * CPU oracle for the AccelEP SimDevice hot path. TEST INFRASTRUCTURE ONLY:
 * loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg to
 * check results, never by the product. Build: oracle/Makefile (gcc -O2
 * -ffp-contract=off, so no product is ever fused into its add).
 *
 * Every function states the reference behaviour it follows (path:line in the
 * AccelEP tree). How each one is pinned is listed in oracle.h.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ReferenceMatMul, src/sim_device.cc:387-402. For every (i, j) the sum runs
 * over k in ascending order; each product is rounded to float before it is
 * added. SimDevice::MatMul's 64/256/64 blocking keeps that order, so its
 * output is bit-identical (tests/test_runtime.cc:234-271). */
void orc_reference_matmul(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n) {
  for (int64_t i = 0; i < m; ++i) {
    float* row = c + i * n;
    for (int64_t j = 0; j < n; ++j) row[j] = 0.f;
    for (int64_t p = 0; p < k; ++p) {
      const float lhs = a[i * k + p];
      const float* rhs = b + p * n;
      for (int64_t j = 0; j < n; ++j) {
        const float product = lhs * rhs[j];
        row[j] = row[j] + product;
      }
    }
  }
}

/* DequantAt, src/sim_device.cc:406-424: w = (float(q) - float(zero)) * scale,
 * rounded after the subtraction and again after the multiply. The coordinate
 * along `axis` is (index / stride) % shape[axis], stride being the product of
 * the dimensions after `axis`. axis < 0 uses scale[0] and zero[0]. */
float orc_dequant_at(const OrcQuantPlane* plane, int64_t index) {
  float scale = plane->scale[0];
  float zero = 0.f;
  if (plane->axis >= 0) {
    int64_t stride = 1;
    for (int32_t d = plane->rank - 1; d > plane->axis; --d) stride *= plane->shape[d];
    const int64_t coord = (index / stride) % plane->shape[plane->axis];
    scale = plane->scale[coord];
    if (plane->zero != NULL) zero = (float)plane->zero[coord];
  } else if (plane->zero != NULL) {
    zero = (float)plane->zero[0];
  }
  const float centered = (float)plane->q[index] - zero;
  return centered * scale;
}

/* accel::MatMulQuantized, src/sim_device.cc:541-602. The reference fills a
 * 64x256 float panel with DequantAt values and accumulates each output in k
 * order with a rounded product, so its result equals ReferenceMatMul on the
 * dequantized operands (tests/test_runtime.cc:325-392 checks this with memcmp).
 * Here the right operand is dequantized one k-row at a time and every output
 * row is advanced by that k: the per-element order (k ascending, product
 * rounded before the add) is unchanged. */
int orc_matmul_quantized(const float* a, const OrcQuantPlane* a_quant, const float* b, const OrcQuantPlane* b_quant,
                         float* c, int64_t m, int64_t k, int64_t n) {
  if (m < 0 || k < 0 || n < 0 || (m > 0 && n > 0 && c == NULL)) return ORC_INVALID;
  if ((a == NULL && a_quant == NULL && m * k != 0) || (b == NULL && b_quant == NULL && k * n != 0)) return ORC_INVALID;
  for (int64_t i = 0; i < m * n; ++i) c[i] = 0.f;
  float* brow = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  if (brow == NULL) return ORC_INVALID;
  for (int64_t p = 0; p < k; ++p) {
    const float* rhs = NULL;
    if (b_quant != NULL) {
      for (int64_t j = 0; j < n; ++j) brow[j] = orc_dequant_at(b_quant, b_quant->offset + p * n + j);
      rhs = brow;
    } else {
      rhs = b + p * n;
    }
    for (int64_t i = 0; i < m; ++i) {
      const float lhs = a_quant != NULL ? orc_dequant_at(a_quant, a_quant->offset + i * k + p) : a[i * k + p];
      float* row = c + i * n;
      for (int64_t j = 0; j < n; ++j) {
        const float product = lhs * rhs[j];
        row[j] = row[j] + product;
      }
    }
  }
  free(brow);
  return ORC_OK;
}

/* BiasOffset, src/sim_device.cc:104-124: a bias of rank <= 2 is right-aligned
 * against [m, n]; a dimension of size 1 broadcasts. */
int64_t orc_bias_offset(int32_t rank, const int64_t* shape, int64_t i, int64_t j) {
  if (rank <= 0) return 0;
  int64_t strides[2] = {1, 1};
  for (int32_t d = rank - 2; d >= 0; --d) strides[d] = strides[d + 1] * shape[d + 1];
  const int64_t coords[2] = {i, j};
  int64_t offset = 0;
  for (int32_t d = 0; d < rank; ++d) {
    const int64_t coord = shape[d] == 1 ? 0 : coords[2 - rank + d];
    offset += coord * strides[d];
  }
  return offset;
}

/* SimDevice::GemmEpilogue, src/sim_device.cc:211-245. v = alpha*c (rounded);
 * with a bias v = v + (beta*bias) (each rounded). Relu replaces v only when
 * v < 0, so NaN and -0 pass through. Gelu is the exact erf form with the
 * multiplications in source order: (0.5*v) * (1 + erf(v*0.70710678)). */
void orc_gemm_epilogue(float* c, int64_t m, int64_t n, float alpha, const float* bias, int32_t bias_rank,
                       const int64_t* bias_shape, float beta, int32_t activation) {
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t j = 0; j < n; ++j) {
      float value = alpha * c[i * n + j];
      if (bias != NULL) {
        const float scaled = beta * bias[orc_bias_offset(bias_rank, bias_shape, i, j)];
        value = value + scaled;
      }
      if (activation == ORC_ACT_RELU) {
        if (value < 0.f) value = 0.f;
      } else if (activation == ORC_ACT_GELU) {
        const float half = 0.5f * value;
        const float arg = value * 0.7071067811865476f;
        value = half * (1.f + erff(arg));
      }
      c[i * n + j] = value;
    }
  }
}

/* SimDevice::Transpose, src/sim_device.cc:198-209: dst[j, i] = src[i, j]. */
void orc_transpose(const float* src, float* dst, int64_t rows, int64_t cols) {
  for (int64_t i = 0; i < rows; ++i)
    for (int64_t j = 0; j < cols; ++j) dst[j * rows + i] = src[i * cols + j];
}

/* SimRmsNorm, src/sim_rmsnorm.cc:7-20: sum of squares in double (ascending
 * index), inv = 1/sqrt(ss/dim + eps) in double, y = float(x*inv) * w in float. */
void orc_rmsnorm(const float* x, const float* weight, float* y, int64_t rows, int64_t dim, float eps,
                 int64_t row_offset) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* in = x + (row_offset + r) * dim;
    float* out = y + r * dim;
    double ss = 0.0;
    for (int64_t i = 0; i < dim; ++i) ss += (double)in[i] * (double)in[i];
    const double inv = 1.0 / sqrt(ss / (double)dim + (double)eps);
    for (int64_t i = 0; i < dim; ++i) {
      const float normed = (float)((double)in[i] * inv);
      out[i] = normed * weight[i];
    }
  }
}

/* SimEmbed, src/sim_embed.cc:9-20: row copy; an id outside [0, vocab) is an
 * error (the reference throws std::invalid_argument). Rows before the bad id
 * have already been written, as in the reference. */
int orc_embed(const int32_t* ids, int64_t id_offset, const float* table, float* out, int64_t seq, int64_t hidden,
              int64_t vocab) {
  for (int64_t s = 0; s < seq; ++s) {
    const int32_t id = ids[id_offset + s];
    if (id < 0 || id >= vocab) return ORC_INVALID;
    memcpy(out + s * hidden, table + (int64_t)id * hidden, sizeof(float) * (size_t)hidden);
  }
  return ORC_OK;
}

/* SimRope, src/sim_rope.cc:5-21: rotate-half with cos/sin rows at absolute
 * position (position + s). Both products are rounded before the add/sub. */
void orc_rope(float* states, const float* cos_table, const float* sin_table, int64_t seq, int64_t n_heads,
              int64_t head_dim, int64_t position) {
  const int64_t half = head_dim / 2;
  for (int64_t s = 0; s < seq; ++s) {
    const float* cs = cos_table + (position + s) * head_dim;
    const float* sn = sin_table + (position + s) * head_dim;
    for (int64_t h = 0; h < n_heads; ++h) {
      float* row = states + (s * n_heads + h) * head_dim;
      for (int64_t i = 0; i < half; ++i) {
        const float x0 = row[i];
        const float x1 = row[half + i];
        const float a0 = x0 * cs[i];
        const float b0 = x1 * sn[i];
        const float a1 = x1 * cs[half + i];
        const float b1 = x0 * sn[half + i];
        row[i] = a0 - b0;
        row[half + i] = a1 + b1;
      }
    }
  }
}

/* SimAppendCache, src/sim_cache.cc:8-13: copy seq rows of n_heads*head_dim
 * floats to row `position` of the cache. */
void orc_append_cache(const float* src, float* cache, int64_t seq, int64_t position, int64_t n_heads,
                      int64_t head_dim) {
  const int64_t row = n_heads * head_dim;
  memcpy(cache + position * row, src, sizeof(float) * (size_t)(seq * row));
}

/* SimAttend, src/sim_attend.cc:9-46: causal GQA. Query row s sees keys
 * 0..position+s; head h reads kv head h / (heads/kv_heads). Score = dot*scale
 * with scale = 1/sqrtf(head_dim); softmax subtracts the running max, exps in
 * float, sums in t order; out[d] = sum_t (score_t/sum) * v[t][d] in t order. */
void orc_attention(const float* q, const float* k, const float* v, float* scores, float* out, int64_t seq,
                   int64_t position, int64_t heads, int64_t kv_heads, int64_t head_dim) {
  const float scale = 1.f / sqrtf((float)head_dim);
  const int64_t group = heads / kv_heads;
  for (int64_t s = 0; s < seq; ++s) {
    const int64_t last = position + s;
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t kv = h / group;
      const float* qrow = q + (s * heads + h) * head_dim;
      float top = -INFINITY;
      for (int64_t t = 0; t <= last; ++t) {
        const float* krow = k + (t * kv_heads + kv) * head_dim;
        float dot = 0.f;
        for (int64_t d = 0; d < head_dim; ++d) {
          const float product = qrow[d] * krow[d];
          dot = dot + product;
        }
        scores[t] = dot * scale;
        if (scores[t] > top) top = scores[t];
      }
      float total = 0.f;
      for (int64_t t = 0; t <= last; ++t) {
        scores[t] = expf(scores[t] - top);
        total = total + scores[t];
      }
      float* dest = out + (s * heads + h) * head_dim;
      for (int64_t d = 0; d < head_dim; ++d) {
        float acc = 0.f;
        for (int64_t t = 0; t <= last; ++t) {
          const float weight = scores[t] / total;
          const float product = weight * v[(t * kv_heads + kv) * head_dim + d];
          acc = acc + product;
        }
        dest[d] = acc;
      }
    }
  }
}

/* SimSiluMul, src/sim_silu.cc:8-13: gate = (x / (1 + expf(-x))) * up. */
void orc_silu_mul(float* gate, const float* up, int64_t count) {
  for (int64_t i = 0; i < count; ++i) {
    const float x = gate[i];
    const float denom = 1.f + expf(-x);
    const float silu = x / denom;
    gate[i] = silu * up[i];
  }
}

/* SimAdd, src/sim_add.cc:5-9. */
void orc_add(float* dest, const float* extra, int64_t count) {
  for (int64_t i = 0; i < count; ++i) dest[i] = dest[i] + extra[i];
}

/* xorshift32 step, src/sim_sample.cc:9-16. */
static uint32_t orc_xorshift32(uint32_t* state) {
  uint32_t x = *state;
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  *state = x;
  return x;
}

typedef struct {
  int64_t id;
  float logit;
} OrcSlot;

/* SimSampleToken, src/sim_sample.cc:25-115.
 *  - !(T > 0): argmax, the earliest id wins a tie (strict >).
 *  - full draw when top_k <= 0 or top_k >= vocab (compared before the 64 cap).
 *  - otherwise a table of at most min(top_k, 64) slots: the first entries fill
 *    it, later logits replace the worst slot (lowest logit, later id on a tie)
 *    when strictly larger, or equal with a smaller id; the table is then
 *    sorted by id (insertion sort).
 *  - weights exp((l - max) / T) in double, drawn with (xorshift + 0.5)/2^32 *
 *    sum; the first cumulative weight >= draw wins; a non-positive sum picks 0;
 *    falling off the end picks the last candidate. */
void orc_sample_token(const float* logits, int32_t* chosen_ids, int64_t chosen_index, int64_t vocab,
                      float temperature, uint32_t* rng_state, int32_t top_k) {
  if (!(temperature > 0.f)) {
    int64_t best = 0;
    float best_value = logits[0];
    for (int64_t i = 1; i < vocab; ++i) {
      if (logits[i] > best_value) {
        best_value = logits[i];
        best = i;
      }
    }
    chosen_ids[chosen_index] = (int32_t)best;
    return;
  }
  const int full = top_k <= 0 || (int64_t)top_k >= vocab;
  const int cap = top_k > 64 ? 64 : top_k;
  OrcSlot table[64];
  int filled = 0;
  if (!full) {
    for (int64_t i = 0; i < vocab; ++i) {
      const float value = logits[i];
      if (filled < cap) {
        table[filled].id = i;
        table[filled].logit = value;
        ++filled;
        continue;
      }
      int worst = 0;
      for (int s = 1; s < filled; ++s) {
        const int lower = table[s].logit < table[worst].logit;
        const int later_tie = table[s].logit == table[worst].logit && table[s].id > table[worst].id;
        if (lower || later_tie) worst = s;
      }
      if (value > table[worst].logit || (value == table[worst].logit && i < table[worst].id)) {
        table[worst].id = i;
        table[worst].logit = value;
      }
    }
    for (int i = 1; i < filled; ++i) {
      const OrcSlot key = table[i];
      int j = i;
      while (j > 0 && table[j - 1].id > key.id) {
        table[j] = table[j - 1];
        --j;
      }
      table[j] = key;
    }
  }
  float top = full ? logits[0] : table[0].logit;
  if (full) {
    for (int64_t i = 1; i < vocab; ++i)
      if (logits[i] > top) top = logits[i];
  } else {
    for (int s = 1; s < filled; ++s)
      if (table[s].logit > top) top = table[s].logit;
  }
  const double inv_t = 1.0 / (double)temperature;
  const int64_t span = full ? vocab : filled;
  double sum = 0.0;
  for (int64_t s = 0; s < span; ++s) {
    const int64_t id = full ? s : table[s].id;
    sum += exp(((double)logits[id] - (double)top) * inv_t);
  }
  if (!(sum > 0.0)) {
    chosen_ids[chosen_index] = 0;
    return;
  }
  const double draw = ((double)orc_xorshift32(rng_state) + 0.5) / 4294967296.0 * sum;
  double acc = 0.0;
  for (int64_t s = 0; s < span; ++s) {
    const int64_t id = full ? s : table[s].id;
    acc += exp(((double)logits[id] - (double)top) * inv_t);
    if (acc >= draw) {
      chosen_ids[chosen_index] = (int32_t)id;
      return;
    }
  }
  chosen_ids[chosen_index] = (int32_t)(full ? vocab - 1 : table[filled - 1].id);
}

/* Rope tables, src/llama_model.cc:333-349: for pair i < dim/2 the angle is
 * pos / theta^(2i/dim) in double; cos/sin are rounded to float and written to
 * both halves of the row. */
void orc_rope_tables(int32_t context, int32_t head_dim, float theta, float* cos_out, float* sin_out) {
  const int32_t half = head_dim / 2;
  for (int32_t pos = 0; pos < context; ++pos) {
    for (int32_t i = 0; i < half; ++i) {
      const double inv = 1.0 / pow((double)theta, (2.0 * i) / (double)head_dim);
      const double angle = (double)pos * inv;
      const float cv = (float)cos(angle);
      const float sv = (float)sin(angle);
      cos_out[(int64_t)pos * head_dim + i] = cv;
      cos_out[(int64_t)pos * head_dim + half + i] = cv;
      sin_out[(int64_t)pos * head_dim + i] = sv;
      sin_out[(int64_t)pos * head_dim + half + i] = sv;
    }
  }
}

/* ---- Llama (src/llama_model.cc) over float weights ----------------------- */

typedef struct {
  float *attn_norm, *post_norm, *q, *k, *v, *o, *gate, *up, *down; /* matrices stored [in, out] */
} OrcLayer;

struct OrcLlama {
  OrcLlamaConfig cfg;
  int32_t head_dim;
  int32_t filled;
  float *embed, *final_norm, *lm_head; /* lm_head stored [hidden, vocab] */
  float *rope_cos, *rope_sin;
  float *hidden, *normed, *query, *key, *value, *mixed, *delta, *gate, *up, *logits, *scores;
  int32_t *chosen, *prompt_ids;
  OrcLayer* layers;
  float** k_cache;
  float** v_cache;
};

static float* orc_zeros(size_t count) { return (float*)calloc(count > 0 ? count : 1, sizeof(float)); }

/* accel_llama_create, src/llama_model.cc:318-395. */
OrcLlama* orc_llama_create(const OrcLlamaConfig* c) {
  if (c == NULL || c->vocab <= 0 || c->hidden <= 0 || c->layers <= 0 || c->heads <= 0 || c->kv_heads <= 0 ||
      c->intermediate <= 0 || c->context <= 0 || c->hidden % c->heads != 0 || c->heads % c->kv_heads != 0)
    return NULL;
  OrcLlama* m = (OrcLlama*)calloc(1, sizeof(OrcLlama));
  m->cfg = *c;
  m->head_dim = c->hidden / c->heads;
  const size_t ctx = (size_t)c->context;
  const size_t dim = (size_t)m->head_dim;
  m->rope_cos = orc_zeros(ctx * dim);
  m->rope_sin = orc_zeros(ctx * dim);
  orc_rope_tables(c->context, m->head_dim, c->rope_theta, m->rope_cos, m->rope_sin);
  m->hidden = orc_zeros(ctx * (size_t)c->hidden);
  m->normed = orc_zeros(ctx * (size_t)c->hidden);
  m->query = orc_zeros(ctx * (size_t)c->heads * dim);
  m->key = orc_zeros(ctx * (size_t)c->kv_heads * dim);
  m->value = orc_zeros(ctx * (size_t)c->kv_heads * dim);
  m->mixed = orc_zeros(ctx * (size_t)c->heads * dim);
  m->delta = orc_zeros(ctx * (size_t)c->hidden);
  m->gate = orc_zeros(ctx * (size_t)c->intermediate);
  m->up = orc_zeros(ctx * (size_t)c->intermediate);
  m->logits = orc_zeros((size_t)c->vocab);
  m->scores = orc_zeros(ctx);
  m->chosen = (int32_t*)calloc(ctx, sizeof(int32_t));
  m->prompt_ids = (int32_t*)calloc(ctx, sizeof(int32_t));
  m->layers = (OrcLayer*)calloc((size_t)c->layers, sizeof(OrcLayer));
  m->k_cache = (float**)calloc((size_t)c->layers, sizeof(float*));
  m->v_cache = (float**)calloc((size_t)c->layers, sizeof(float*));
  for (int32_t l = 0; l < c->layers; ++l) {
    m->k_cache[l] = orc_zeros(ctx * (size_t)c->kv_heads * dim);
    m->v_cache[l] = orc_zeros(ctx * (size_t)c->kv_heads * dim);
  }
  return m;
}

void orc_llama_destroy(OrcLlama* m) {
  if (m == NULL) return;
  for (int32_t l = 0; l < m->cfg.layers; ++l) {
    OrcLayer* L = &m->layers[l];
    free(L->attn_norm); free(L->post_norm); free(L->q); free(L->k); free(L->v); free(L->o);
    free(L->gate); free(L->up); free(L->down);
    free(m->k_cache[l]); free(m->v_cache[l]);
  }
  free(m->layers); free(m->k_cache); free(m->v_cache);
  free(m->embed); free(m->final_norm); free(m->lm_head); free(m->rope_cos); free(m->rope_sin);
  free(m->hidden); free(m->normed); free(m->query); free(m->key); free(m->value); free(m->mixed);
  free(m->delta); free(m->gate); free(m->up); free(m->logits); free(m->scores); free(m->chosen);
  free(m->prompt_ids);
  free(m);
}

/* ShapeOk, src/llama_model.cc:288-314. */
static int orc_shape_ok(const OrcLlama* m, int32_t kind, int64_t rows, int64_t cols) {
  const int32_t hidden = m->cfg.hidden;
  const int32_t q_out = m->cfg.heads * m->head_dim;
  const int32_t k_out = m->cfg.kv_heads * m->head_dim;
  switch (kind) {
    case ORC_W_EMBED:
    case ORC_W_LM_HEAD: return rows == m->cfg.vocab && cols == hidden;
    case ORC_W_FINAL_NORM:
    case ORC_W_ATTN_NORM:
    case ORC_W_POST_NORM: return rows == hidden && cols == 1;
    case ORC_W_Q: return rows == q_out && cols == hidden;
    case ORC_W_K:
    case ORC_W_V: return rows == k_out && cols == hidden;
    case ORC_W_O: return rows == hidden && cols == q_out;
    case ORC_W_DOWN: return rows == hidden && cols == m->cfg.intermediate;
    case ORC_W_GATE:
    case ORC_W_UP: return rows == m->cfg.intermediate && cols == hidden;
    default: return 0;
  }
}

/* accel_llama_weight, src/llama_model.cc:399-422: norms and the embedding keep
 * the file layout; every other matrix is stored transposed to [in, out]. */
int orc_llama_weight(OrcLlama* m, int32_t kind, int32_t layer, const float* data, int64_t rows, int64_t cols) {
  if (m == NULL || data == NULL || rows <= 0 || cols <= 0 || !orc_shape_ok(m, kind, rows, cols)) return ORC_INVALID;
  float** slot = NULL;
  if (kind == ORC_W_EMBED) slot = &m->embed;
  else if (kind == ORC_W_FINAL_NORM) slot = &m->final_norm;
  else if (kind == ORC_W_LM_HEAD) slot = &m->lm_head;
  else {
    if (layer < 0 || layer >= m->cfg.layers) return ORC_INVALID;
    OrcLayer* L = &m->layers[layer];
    switch (kind) {
      case ORC_W_ATTN_NORM: slot = &L->attn_norm; break;
      case ORC_W_POST_NORM: slot = &L->post_norm; break;
      case ORC_W_Q: slot = &L->q; break;
      case ORC_W_K: slot = &L->k; break;
      case ORC_W_V: slot = &L->v; break;
      case ORC_W_O: slot = &L->o; break;
      case ORC_W_GATE: slot = &L->gate; break;
      case ORC_W_UP: slot = &L->up; break;
      case ORC_W_DOWN: slot = &L->down; break;
      default: return ORC_INVALID;
    }
  }
  const size_t count = (size_t)rows * (size_t)cols;
  float* store = (float*)malloc(sizeof(float) * count);
  const int keep = kind == ORC_W_EMBED || kind == ORC_W_FINAL_NORM || kind == ORC_W_ATTN_NORM || kind == ORC_W_POST_NORM;
  if (keep) {
    memcpy(store, data, sizeof(float) * count);
  } else {
    for (int64_t o = 0; o < rows; ++o)
      for (int64_t i = 0; i < cols; ++i) store[i * rows + o] = data[o * cols + i];
  }
  free(*slot);
  *slot = store;
  return ORC_OK;
}

static int orc_ready(const OrcLlama* m) {
  if (m->embed == NULL || m->final_norm == NULL || m->lm_head == NULL) return 0;
  for (int32_t l = 0; l < m->cfg.layers; ++l) {
    const OrcLayer* L = &m->layers[l];
    if (!L->attn_norm || !L->post_norm || !L->q || !L->k || !L->v || !L->o || !L->gate || !L->up || !L->down) return 0;
  }
  return 1;
}

/* LlamaModel::Forward, src/llama_model.cc:209-247: the device call order of
 * one forward, ending with the final norm of the last row and one logit row. */
static int orc_forward(OrcLlama* m, const int32_t* ids, int32_t seq, int64_t id_offset) {
  const OrcLlamaConfig* c = &m->cfg;
  if (seq <= 0 || m->filled < 0 || seq > c->context || m->filled > c->context - seq) return ORC_INVALID;
  const int64_t hid = c->hidden;
  const int64_t pos = m->filled;
  const int64_t hd = m->head_dim;
  if (orc_embed(ids, id_offset, m->embed, m->hidden, seq, hid, c->vocab) != ORC_OK) return ORC_INVALID;
  for (int32_t l = 0; l < c->layers; ++l) {
    OrcLayer* L = &m->layers[l];
    orc_rmsnorm(m->hidden, L->attn_norm, m->normed, seq, hid, c->eps, 0);
    orc_reference_matmul(m->normed, L->q, m->query, seq, hid, (int64_t)c->heads * hd);
    orc_reference_matmul(m->normed, L->k, m->key, seq, hid, (int64_t)c->kv_heads * hd);
    orc_reference_matmul(m->normed, L->v, m->value, seq, hid, (int64_t)c->kv_heads * hd);
    orc_rope(m->query, m->rope_cos, m->rope_sin, seq, c->heads, hd, pos);
    orc_rope(m->key, m->rope_cos, m->rope_sin, seq, c->kv_heads, hd, pos);
    orc_append_cache(m->key, m->k_cache[l], seq, pos, c->kv_heads, hd);
    orc_append_cache(m->value, m->v_cache[l], seq, pos, c->kv_heads, hd);
    orc_attention(m->query, m->k_cache[l], m->v_cache[l], m->scores, m->mixed, seq, pos, c->heads, c->kv_heads, hd);
    orc_reference_matmul(m->mixed, L->o, m->delta, seq, hid, hid);
    orc_add(m->hidden, m->delta, seq * hid);
    orc_rmsnorm(m->hidden, L->post_norm, m->normed, seq, hid, c->eps, 0);
    orc_reference_matmul(m->normed, L->gate, m->gate, seq, hid, c->intermediate);
    orc_reference_matmul(m->normed, L->up, m->up, seq, hid, c->intermediate);
    orc_silu_mul(m->gate, m->up, seq * (int64_t)c->intermediate);
    orc_reference_matmul(m->gate, L->down, m->delta, seq, c->intermediate, hid);
    orc_add(m->hidden, m->delta, seq * hid);
  }
  orc_rmsnorm(m->hidden, m->final_norm, m->normed, 1, hid, c->eps, (int64_t)seq - 1);
  orc_reference_matmul(m->normed, m->lm_head, m->logits, 1, hid, c->vocab);
  return ORC_OK;
}

/* LlamaModel::Generate, src/llama_model.cc:101-131 (seed 0 becomes 0x6d2b79f5;
 * stop on eos or a full context; each decode forward reads id `produced-1`). */
int orc_llama_generate(OrcLlama* m, const int32_t* prompt, int32_t prompt_count, int32_t max_new, int32_t eos_id,
                       float temperature, uint32_t seed, int32_t top_k, int32_t* out_ids, int32_t* out_count) {
  if (m == NULL || prompt == NULL || out_ids == NULL || out_count == NULL || prompt_count <= 0 || max_new < 0)
    return ORC_INVALID;
  if (!orc_ready(m)) return ORC_INVALID;
  m->filled = 0;
  if (prompt_count > m->cfg.context) return ORC_INVALID;
  memcpy(m->prompt_ids, prompt, sizeof(int32_t) * (size_t)prompt_count);
  if (orc_forward(m, m->prompt_ids, prompt_count, 0) != ORC_OK) return ORC_INVALID;
  m->filled = prompt_count;
  uint32_t rng = seed == 0 ? 0x6d2b79f5u : seed;
  int32_t produced = 0;
  for (int32_t step = 0; step < max_new; ++step) {
    if (produced >= m->cfg.context) return ORC_INVALID;
    orc_sample_token(m->logits, m->chosen, produced, m->cfg.vocab, temperature, &rng, top_k);
    const int32_t id = m->chosen[produced];
    produced += 1;
    if (id == eos_id || m->filled >= m->cfg.context) break;
    if (orc_forward(m, m->chosen, 1, (int64_t)produced - 1) != ORC_OK) return ORC_INVALID;
    m->filled += 1;
  }
  memcpy(out_ids, m->chosen, sizeof(int32_t) * (size_t)produced);
  *out_count = produced;
  return ORC_OK;
}

/* LlamaModel::ForwardIds, src/llama_model.cc:150-166. */
int orc_llama_forward_ids(OrcLlama* m, const int32_t* ids, int32_t count, int32_t reset) {
  if (m == NULL || !orc_ready(m) || ids == NULL || count <= 0) return ORC_INVALID;
  if (reset) m->filled = 0;
  if (m->filled < 0 || count > m->cfg.context - m->filled) return ORC_INVALID;
  memcpy(m->prompt_ids, ids, sizeof(int32_t) * (size_t)count);
  if (orc_forward(m, m->prompt_ids, count, 0) != ORC_OK) return ORC_INVALID;
  m->filled += count;
  return ORC_OK;
}

int orc_llama_logits(OrcLlama* m, float* out, int32_t count) {
  if (m == NULL || out == NULL || count != m->cfg.vocab) return ORC_INVALID;
  memcpy(out, m->logits, sizeof(float) * (size_t)count);
  return ORC_OK;
}
