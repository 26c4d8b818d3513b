// C entry points over the compiled reference (AccelEP's own src/*.cc), so the
// tests can load it with ctypes. TEST INFRASTRUCTURE ONLY: it exists to pin the
// oracle restatement and, in bench.py's cpu_baseline leg, to time the reference
// CPU path. Built by oracle/Makefile into oracle/_ref/ from the sources where they
// lie; none of the reference's sources are copied into this repository.
//
// Every function returns 0 on success and 1 when the reference threw.
#include "accel/device.h"
#include "accel/runtime.h"
#include "accel/sim_add.h"
#include "accel/sim_attend.h"
#include "accel/sim_cache.h"
#include "accel/sim_embed.h"
#include "accel/sim_rmsnorm.h"
#include "accel/sim_rope.h"
#include "accel/sim_sample.h"
#include "accel/sim_silu.h"

#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <vector>

#define REF_API extern "C" __attribute__((visibility("default")))

namespace {

// Same field order as OrcQuantPlane in oracle/oracle.h.
struct RefPlane {
  const int8_t* q;
  const float* scale;
  const int8_t* zero;
  int32_t rank;
  int64_t shape[8];
  int64_t axis;
  int64_t offset;
};

accel::QuantPlane ToPlane(const RefPlane* p) {
  accel::QuantPlane out;
  out.q = p->q;
  out.scale = p->scale;
  out.zero = p->zero;
  out.shape.assign(p->shape, p->shape + p->rank);
  out.axis = p->axis;
  out.offset = p->offset;
  return out;
}

accel::OwnedBuffer Put(accel::Device& dev, const void* data, size_t bytes) {
  accel::OwnedBuffer owned;
  owned.device = &dev;
  owned.buffer = dev.Allocate(bytes);
  if (bytes > 0 && data != nullptr) dev.CopyHostToDevice(owned.buffer, data, bytes);
  return owned;
}

}  // namespace

// accel::ReferenceMatMul (src/sim_device.cc:387-402).
REF_API void ref_reference_matmul(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n) {
  accel::ReferenceMatMul(a, b, c, m, k, n);
}

// SimDevice::MatMul (src/sim_device.cc:185-196) through a fresh SimDevice.
REF_API int ref_device_matmul(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n) {
  try {
    auto dev = accel::CreateSimDevice();
    auto A = Put(*dev, a, sizeof(float) * static_cast<size_t>(m * k));
    auto B = Put(*dev, b, sizeof(float) * static_cast<size_t>(k * n));
    auto C = Put(*dev, nullptr, sizeof(float) * static_cast<size_t>(m * n));
    dev->MatMul(A.buffer, B.buffer, C.buffer, m, k, n);
    if (m * n > 0) dev->CopyDeviceToHost(c, C.buffer, sizeof(float) * static_cast<size_t>(m * n));
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

// accel::MatMulQuantized (src/sim_device.cc:541-602) on host pointers.
REF_API int ref_matmul_quantized(const float* a, const RefPlane* aq, const float* b, const RefPlane* bq, float* c,
                                 int64_t m, int64_t k, int64_t n) {
  try {
    accel::QuantPlane ap;
    accel::QuantPlane bp;
    if (aq != nullptr) ap = ToPlane(aq);
    if (bq != nullptr) bp = ToPlane(bq);
    accel::MatMulQuantized(a, aq ? &ap : nullptr, b, bq ? &bp : nullptr, c, m, k, n);
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

// SimDevice::GemmEpilogue (src/sim_device.cc:211-245), in place on host memory.
REF_API int ref_gemm_epilogue(float* c, int64_t m, int64_t n, float alpha, const float* bias, int32_t bias_rank,
                              const int64_t* bias_shape, float beta, int32_t activation) {
  try {
    auto dev = accel::CreateSimDevice();
    auto C = Put(*dev, c, sizeof(float) * static_cast<size_t>(m * n));
    std::vector<int64_t> shape;
    size_t bias_count = 1;
    for (int32_t d = 0; d < bias_rank; ++d) {
      shape.push_back(bias_shape[d]);
      bias_count *= static_cast<size_t>(bias_shape[d]);
    }
    accel::OwnedBuffer B;
    if (bias != nullptr) B = Put(*dev, bias, sizeof(float) * bias_count);
    dev->GemmEpilogue(C.buffer, m, n, alpha, bias ? &B.buffer : nullptr, shape, beta,
                      static_cast<accel::Activation>(activation));
    if (m * n > 0) dev->CopyDeviceToHost(c, C.buffer, sizeof(float) * static_cast<size_t>(m * n));
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

REF_API void ref_rmsnorm(const float* x, const float* w, float* y, int64_t rows, int64_t dim, float eps,
                         int64_t row_offset) {
  accel::SimRmsNorm(x, w, y, rows, dim, eps, row_offset);
}

REF_API int ref_embed(const int32_t* ids, int64_t id_offset, const float* table, float* out, int64_t seq,
                      int64_t hidden, int64_t vocab) {
  try {
    accel::SimEmbed(ids, id_offset, table, out, seq, hidden, vocab);
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}

REF_API void ref_rope(float* states, const float* cos_table, const float* sin_table, int64_t seq, int64_t n_heads,
                      int64_t head_dim, int64_t position) {
  accel::SimRope(states, cos_table, sin_table, seq, n_heads, head_dim, position);
}

REF_API void ref_append_cache(const float* src, float* cache, int64_t seq, int64_t position, int64_t n_heads,
                              int64_t head_dim) {
  accel::SimAppendCache(src, cache, seq, position, n_heads, head_dim);
}

REF_API void ref_attention(const float* q, const float* k, const float* v, float* scores, float* out, int64_t seq,
                           int64_t position, int64_t heads, int64_t kv_heads, int64_t head_dim) {
  accel::SimAttend(q, k, v, scores, out, seq, position, heads, kv_heads, head_dim);
}

REF_API void ref_silu_mul(float* gate, const float* up, int64_t count) { accel::SimSiluMul(gate, up, count); }

REF_API void ref_add(float* dest, const float* extra, int64_t count) { accel::SimAdd(dest, extra, count); }

REF_API void ref_sample_token(const float* logits, int32_t* chosen, int64_t index, int64_t vocab, float temperature,
                              uint32_t* rng, int32_t top_k) {
  accel::SimSampleToken(logits, chosen, index, vocab, temperature, rng, top_k);
}

// The reference's \p{L} and \p{N} tables (src/unicode_cats.inc, compiled where it lies), as
// flat [first, last] pairs; which 0 = letters, 1 = numbers.
namespace ref_unicode {
#include "unicode_cats.inc"
}  // namespace ref_unicode

REF_API int ref_unicode_ranges(int32_t which, const uint32_t** pairs, int32_t* count) {
  if (which == 0) {
    *pairs = ref_unicode::k_letter_ranges;
    *count = ref_unicode::k_letter_ranges_count;
    return 0;
  }
  if (which == 1) {
    *pairs = ref_unicode::k_number_ranges;
    *count = ref_unicode::k_number_ranges_count;
    return 0;
  }
  return 1;
}
