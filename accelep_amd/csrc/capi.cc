// C-ABI compute entry points of libaccel_hip: the reference's argument checks and error
// behaviour (src/sim_device.cc:185-328,541-548), the choice of kernel, and the counters
// each call notes. Every kernel runs on the library's stream.
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.h"
#include "host_util.h"

namespace accel_hip {

void NoteStat(int which, int64_t amount);  // context.cc
constexpr int kStatDeviceTransposes = 6;

namespace {

void CheckPlane(const AccelHipQuantPlane* p, const char* side) {
  if (p->rank < 1 || p->rank > 8) Fail(ACCEL_HIP_INVALID_ARGUMENT, std::string(side) + " quant plane rank out of range");
  if (p->q == nullptr || p->scale == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, std::string(side) + " quant plane is missing data");
  if (p->axis >= p->rank) Fail(ACCEL_HIP_INVALID_ARGUMENT, std::string(side) + " quant plane axis out of range");
  for (int32_t d = 0; d < p->rank; ++d)
    if (p->shape[d] < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, std::string(side) + " quant plane shape is negative");
  if (p->offset < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, std::string(side) + " quant plane offset is negative");
}

// Maps DequantAt's coordinate rule (src/sim_device.cc:406-424) for the [rows, cols] matrix
// starting at plane.offset onto one of the kernel modes. False: needs the generic path.
bool PlaneView(const AccelHipQuantPlane& p, int64_t rows, int64_t cols, Q8View* out) {
  out->q = p.q + p.offset;
  out->scale = p.scale;
  out->zero = p.zero;
  out->mode = kScaleConst;
  out->const_index = 0;
  if (p.axis < 0) return true;
  int64_t stride = 1;
  for (int32_t d = p.rank - 1; d > p.axis; --d) stride *= p.shape[d];
  const int64_t dim = p.shape[p.axis];
  const int64_t elems = rows * cols;
  if (elems == 0) return true;
  if (stride == 1 && dim == cols && p.offset % cols == 0) {
    out->mode = kScalePerCol;
    return true;
  }
  if (stride == cols && dim == rows && p.offset % elems == 0) {
    out->mode = kScalePerRow;
    return true;
  }
  if (stride % elems == 0 && p.offset % elems == 0) {
    out->mode = kScaleConst;
    out->const_index = (p.offset / stride) % dim;
    return true;
  }
  return false;
}

}  // namespace

Epilogue ToEpilogue(const AccelHipEpilogue* e) {
  Epilogue out;
  if (e == nullptr) return out;
  out.alpha = e->alpha;
  out.beta = e->beta;
  out.bias = e->bias;
  out.bias_rank = e->bias_rank;
  if (e->bias != nullptr) {
    if (e->bias_rank < 0 || e->bias_rank > 2) Fail(ACCEL_HIP_INVALID_ARGUMENT, "bias rank must be 0..2");
    for (int d = 0; d < e->bias_rank; ++d) {
      if (e->bias_shape[d] < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "negative bias shape");
      out.bias_shape[d] = e->bias_shape[d];
    }
  }
  if (e->activation < ACCEL_HIP_ACT_NONE || e->activation > ACCEL_HIP_ACT_GELU)
    Fail(ACCEL_HIP_INVALID_ARGUMENT, "unknown activation");
  out.activation = e->activation;
  out.residual = e->residual;
  out.rms_weight = e->rms_weight;
  out.rms_eps = e->rms_eps;
  out.rms_out = e->rms_out;
  if (out.rms_weight != nullptr && out.rms_out == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "rms epilogue needs an output");
  return out;
}

namespace {

// The bias of a fused epilogue must fit [m, n] by right-aligned broadcast.
void CheckBias(const Epilogue& e, int64_t m, int64_t n) {
  if (e.bias == nullptr) return;
  const int64_t target[2] = {m, n};
  for (int d = 0; d < e.bias_rank; ++d) {
    const int64_t dim = e.bias_shape[d];
    const int64_t want = target[2 - e.bias_rank + d];
    if (dim != 1 && dim != want) Fail(ACCEL_HIP_INVALID_ARGUMENT, "bias does not broadcast to the output");
  }
}

}  // namespace

// Runs the matmul with the fused epilogue; the trailing RmsNorm (if any) reads C.
void RunMatmul(const float* a, const AccelHipQuantPlane* aq, const float* b, const AccelHipQuantPlane* bq, float* c,
               int64_t m, int64_t k, int64_t n, const Epilogue& epi, bool stage_weights) {
  Context& ctx = Ctx();
  if (m * n == 0) return;
  CheckBias(epi, m, n);
  bool rms_done = false;
  NoteDeviceWrite(c, static_cast<size_t>(m * n) * sizeof(float));
  if (epi.rms_out != nullptr) NoteDeviceWrite(epi.rms_out, static_cast<size_t>(m * n) * sizeof(float));
  if (k == 0) {
    LaunchFill(c, 0.f, m * n, ctx.stream);
    if (!epi.Identity()) LaunchEpilogueInPlace(c, m, n, epi, ctx.stream);
  } else {
    const float* a_f = a;
    if (aq != nullptr) {
      float* tmp = static_cast<float*>(Temp(kTempDequantA, static_cast<size_t>(m * k) * sizeof(float)));
      LaunchDequantize(*aq, m * k, tmp, ctx.stream);
      a_f = tmp;
    }
    Q8View view;
    bool q8 = false;
    const float* b_f = b;
    if (bq != nullptr) {
      if (PlaneView(*bq, k, n, &view)) {
        q8 = true;
      } else {
        float* tmp = static_cast<float*>(Temp(kTempDequantB, static_cast<size_t>(k * n) * sizeof(float)));
        LaunchDequantize(*bq, k * n, tmp, ctx.stream);
        b_f = tmp;
      }
    }
    Epilogue main = epi;
    main.rms_weight = nullptr;
    main.rms_out = nullptr;
    if (ctx.exact_products) {
      LaunchExactMatmul(a_f, q8 ? nullptr : b_f, q8 ? view : Q8View{}, c, m, k, n, main, ctx.stream);
    } else if (q8 && m <= 16) {
      if (GemvWantsGroups(m, k, n, view)) view.grouped = StagedGroupTiles(view.q, k, n, ctx.stream, stage_weights);
      else if (m <= 4) view.tiled = StagedColumnTiles(view.q, k, n, ctx.stream, stage_weights);
      LaunchGemvQ8(a_f, view, c, m, k, n, main, ctx.stream);
    } else {
      if (q8 && GemmWantsBf16Image(m, k, n, view)) view.bf16 = StagedBf16Image(view.q, k, n, ctx.stream, stage_weights);
      else if (q8 && GemmWantsSmall(m, k, n, view)) view.bf16x16 = StagedBf16x16(view.q, k, n, ctx.stream, stage_weights);
      RmsRequest rms;
      rms.weight = epi.rms_weight;
      rms.eps = epi.rms_eps;
      rms.out = epi.rms_out;
      rms_done = LaunchGemmF32(a_f, q8 ? nullptr : b_f, q8 ? view : Q8View{}, c, m, k, n, main, ctx.stream,
                               epi.rms_weight != nullptr ? &rms : nullptr, stage_weights && b_f == b);
    }
  }
  if (epi.rms_weight != nullptr && !rms_done)
    LaunchRmsNormRows(c, epi.rms_weight, epi.rms_out, m, n, epi.rms_eps, ctx.stream);
}

void QuantizedChecks(const float* a, const AccelHipQuantPlane* aq, const float* b, const AccelHipQuantPlane* bq,
                     float* c, int64_t m, int64_t k, int64_t n) {
  if (m < 0 || k < 0 || n < 0 || (m > 0 && n > 0 && c == nullptr))
    Fail(ACCEL_HIP_INVALID_ARGUMENT, "quantized MatMul is out of range");
  if ((a == nullptr && aq == nullptr && m * k != 0) || (b == nullptr && bq == nullptr && k * n != 0))
    Fail(ACCEL_HIP_INVALID_ARGUMENT, "quantized MatMul is missing an operand");
  if (aq != nullptr) CheckPlane(aq, "A");
  if (bq != nullptr) CheckPlane(bq, "B");
}

}  // namespace accel_hip

using namespace accel_hip;

extern "C" {

ACCEL_HIP_API int accel_hip_set_exact_products(int32_t on) {
  return Guard([&] { Ctx().exact_products = on != 0; });
}

ACCEL_HIP_API int32_t accel_hip_exact_products(void) {
  int32_t on = 0;
  Guard([&] { on = Ctx().exact_products ? 1 : 0; });
  return on;
}

// Device::MatMul (src/sim_device.cc:185-196).
ACCEL_HIP_API int accel_hip_matmul(AccelHipBuffer a, AccelHipBuffer b, AccelHipBuffer c, int64_t m, int64_t k,
                                   int64_t n) {
  return Guard([&] {
    RequireBytes(a, CheckedBytes(m, k), "MatMul A is out of range");
    RequireBytes(b, CheckedBytes(k, n), "MatMul B is out of range");
    RequireBytes(c, CheckedBytes(m, n), "MatMul C is out of range");
    RunMatmul(static_cast<const float*>(a.data), nullptr, static_cast<const float*>(b.data), nullptr,
              static_cast<float*>(c.data), m, k, n, Epilogue{}, true);
    NotePackedCall(k);
    NoteKernelMatmul();
  });
}

ACCEL_HIP_API int accel_hip_matmul_fused(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n,
                                         const AccelHipEpilogue* epilogue) {
  return Guard([&] {
    if (m < 0 || k < 0 || n < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "negative matrix dimension");
    if ((m * n > 0 && c == nullptr) || (m * k > 0 && a == nullptr) || (k * n > 0 && b == nullptr))
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "MatMul operand is missing");
    RunMatmul(a, nullptr, b, nullptr, c, m, k, n, ToEpilogue(epilogue), true);
    NotePackedCall(k);
    NoteKernelMatmul();
  });
}

// accel::MatMulQuantized (src/sim_device.cc:541-602).
ACCEL_HIP_API int accel_hip_matmul_quantized(const float* a, const AccelHipQuantPlane* a_quant, const float* b,
                                             const AccelHipQuantPlane* b_quant, float* c, int64_t m, int64_t k,
                                             int64_t n) {
  return Guard([&] {
    QuantizedChecks(a, a_quant, b, b_quant, c, m, k, n);
    RunMatmul(a, a_quant, b, b_quant, c, m, k, n, Epilogue{}, true);
    NotePackedCall(k);
    NoteKernelMatmul();
  });
}

ACCEL_HIP_API int accel_hip_matmul_quantized_fused(const float* a, const AccelHipQuantPlane* a_quant, const float* b,
                                                   const AccelHipQuantPlane* b_quant, float* c, int64_t m, int64_t k,
                                                   int64_t n, const AccelHipEpilogue* epilogue) {
  return Guard([&] {
    QuantizedChecks(a, a_quant, b, b_quant, c, m, k, n);
    RunMatmul(a, a_quant, b, b_quant, c, m, k, n, ToEpilogue(epilogue), true);
    NotePackedCall(k);
    NoteKernelMatmul();
  });
}

// Weight preparation: the staged copies of an int8 weight built now instead of at first use.
ACCEL_HIP_API int accel_hip_prepare_quantized(const AccelHipQuantPlane* b_quant, int64_t k, int64_t n,
                                              uint32_t layouts, uint32_t* staged) {
  return Guard([&] {
    if (staged != nullptr) *staged = 0;
    if (b_quant == nullptr || k < 0 || n < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "prepare needs a quant plane and k, n >= 0");
    if ((layouts & ~static_cast<uint32_t>(ACCEL_HIP_STAGE_ALL)) != 0)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "prepare: unknown layout bits");
    CheckPlane(b_quant, "B");
    RefuseInCapture("preparing staged weight copies");
    if (k * n == 0) return;
    Q8View view;
    if (!PlaneView(*b_quant, k, n, &view)) {
      if (layouts != 0)
        Fail(ACCEL_HIP_INVALID_ARGUMENT, "prepare: this plane's scale coordinates fit no staged form (it is dequantized per call)");
      return;
    }
    const bool groups_ok = k % kGemvGroupRows == 0 && view.zero == nullptr &&
                           (view.mode == kScalePerCol || view.mode == kScaleConst);
    const bool bf16_ok = GemmBf16Stageable(k, n, view);
    const bool small_ok = GemmSmallStageable(k, n, view);
    const uint32_t want = layouts != 0 ? layouts
                                       : ACCEL_HIP_STAGE_GEMV_TILES | (groups_ok ? ACCEL_HIP_STAGE_GEMV_GROUPS : 0u) |
                                             (bf16_ok ? ACCEL_HIP_STAGE_GEMM_BF16 : 0u) |
                                             (small_ok ? ACCEL_HIP_STAGE_GEMM_SMALL : 0u);
    if ((want & ACCEL_HIP_STAGE_GEMV_GROUPS) != 0 && !groups_ok)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "prepare: the group-interleaved copy needs k % 32 == 0, no zero points and a "
                                       "per-column or whole-tensor scale");
    if ((want & ACCEL_HIP_STAGE_GEMM_BF16) != 0 && !bf16_ok)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "prepare: the bf16 copy needs k % 32 == 0, k >= 64, n % 8 == 0, no zero points "
                                       "and a per-column or whole-tensor scale");
    if ((want & ACCEL_HIP_STAGE_GEMM_SMALL) != 0 && !small_ok)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "prepare: the small GEMM's bf16 copy needs k % 32 == 0, k <= 768, n % 8 == 0, "
                                       "no zero points and a per-column or whole-tensor scale");
    const hipStream_t s = Ctx().stream;
    const auto built = [](const void* p) {
      if (p == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "prepare: the weight is not inside a live allocation of this library");
    };
    uint32_t done = 0;
    if ((want & ACCEL_HIP_STAGE_GEMV_TILES) != 0) {
      built(StagedColumnTiles(view.q, k, n, s));
      done |= ACCEL_HIP_STAGE_GEMV_TILES;
    }
    if ((want & ACCEL_HIP_STAGE_GEMV_GROUPS) != 0) {
      built(StagedGroupTiles(view.q, k, n, s));
      done |= ACCEL_HIP_STAGE_GEMV_GROUPS;
    }
    if ((want & ACCEL_HIP_STAGE_GEMM_BF16) != 0) {
      built(StagedBf16Image(view.q, k, n, s));
      done |= ACCEL_HIP_STAGE_GEMM_BF16;
    }
    if ((want & ACCEL_HIP_STAGE_GEMM_SMALL) != 0) {
      built(StagedBf16x16(view.q, k, n, s));
      done |= ACCEL_HIP_STAGE_GEMM_SMALL;
    }
    if (staged != nullptr) *staged = done;
  });
}

// Device::Transpose (src/sim_device.cc:198-209).
ACCEL_HIP_API int accel_hip_transpose(AccelHipBuffer src, AccelHipBuffer dst, int64_t rows, int64_t cols) {
  return Guard([&] {
    RequireBytes(src, CheckedBytes(rows, cols), "Transpose source is out of range");
    RequireBytes(dst, CheckedBytes(cols, rows), "Transpose destination is out of range");
    NoteDeviceWrite(dst.data, CheckedBytes(cols, rows));
    LaunchTranspose(static_cast<const float*>(src.data), static_cast<float*>(dst.data), rows, cols, Ctx().stream);
    NoteStat(kStatDeviceTransposes, 1);
  });
}

// Device::GemmEpilogue (src/sim_device.cc:211-245).
ACCEL_HIP_API int accel_hip_gemm_epilogue(AccelHipBuffer c, int64_t m, int64_t n, float alpha,
                                          const AccelHipBuffer* bias, int32_t bias_rank, const int64_t* bias_shape,
                                          float beta, int32_t activation) {
  return Guard([&] {
    RequireBytes(c, CheckedBytes(m, n), "Gemm epilogue destination is out of range");
    Epilogue e;
    e.alpha = alpha;
    e.beta = beta;
    if (activation < ACCEL_HIP_ACT_NONE || activation > ACCEL_HIP_ACT_GELU)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "unknown activation");
    e.activation = activation;
    if (bias != nullptr) {
      if (bias_rank < 0 || (bias_rank > 0 && bias_shape == nullptr)) Fail(ACCEL_HIP_INVALID_ARGUMENT, "bad bias shape");
      int64_t elems = 1;
      for (int32_t d = 0; d < bias_rank; ++d) {
        if (bias_shape[d] < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "negative bias shape");
        elems *= bias_shape[d];
      }
      RequireBytes(*bias, static_cast<size_t>(elems) * sizeof(float), "Gemm bias is out of range");
      if (bias_rank > 2) Fail(ACCEL_HIP_INVALID_ARGUMENT, "bias rank must be 0..2");
      e.bias = static_cast<const float*>(bias->data);
      e.bias_rank = bias_rank;
      for (int32_t d = 0; d < bias_rank; ++d) e.bias_shape[d] = bias_shape[d];
    }
    NoteDeviceWrite(c.data, CheckedBytes(m, n));
    LaunchEpilogueInPlace(static_cast<float*>(c.data), m, n, e, Ctx().stream);
  });
}

// Device::Embedding (src/sim_device.cc:247-255, src/sim_embed.cc:9-20).
ACCEL_HIP_API int accel_hip_embedding(AccelHipBuffer ids, int64_t id_offset, AccelHipBuffer table, AccelHipBuffer out,
                                      int64_t seq, int64_t hidden, int64_t vocab) {
  return Guard([&] {
    const int64_t id_count = CheckedSpan(id_offset, seq);
    RequireBytes(ids, CheckedIntBytes(id_count), "Embedding ids are out of range");
    RequireBytes(table, CheckedBytes(vocab, hidden), "Embedding table is out of range");
    RequireBytes(out, CheckedBytes(seq, hidden), "Embedding output is out of range");
    if (seq == 0 || hidden == 0) return;
    Context& ctx = Ctx();
    RefuseInCapture("Embedding (it reads its range flag back)");
    int32_t* bad = static_cast<int32_t*>(Temp(kTempFlags, 64));
    Check(hipMemsetAsync(bad, 0, sizeof(int32_t), ctx.stream), "hipMemsetAsync");
    NoteDeviceWrite(out.data, CheckedBytes(seq, hidden));
    LaunchEmbedding(static_cast<const int32_t*>(ids.data) + id_offset, static_cast<const float*>(table.data), nullptr,
                    nullptr, static_cast<float*>(out.data), seq, hidden, vocab, bad, ctx.stream);
    int32_t flag = 0;
    Check(hipMemcpyAsync(&flag, bad, sizeof(flag), hipMemcpyDeviceToHost, ctx.stream), "hipMemcpyAsync");
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    if (flag != 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "token id is outside the vocabulary");
  });
}

ACCEL_HIP_API int accel_hip_embedding_q8(AccelHipBuffer ids, int64_t id_offset, const int8_t* table,
                                         const float* row_scale, AccelHipBuffer out, int64_t seq, int64_t hidden,
                                         int64_t vocab) {
  return Guard([&] {
    const int64_t id_count = CheckedSpan(id_offset, seq);
    RequireBytes(ids, CheckedIntBytes(id_count), "Embedding ids are out of range");
    RequireBytes(out, CheckedBytes(seq, hidden), "Embedding output is out of range");
    if (table == nullptr || row_scale == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Embedding table is out of range");
    if (seq == 0 || hidden == 0) return;
    Context& ctx = Ctx();
    RefuseInCapture("Embedding (it reads its range flag back)");
    int32_t* bad = static_cast<int32_t*>(Temp(kTempFlags, 64));
    Check(hipMemsetAsync(bad, 0, sizeof(int32_t), ctx.stream), "hipMemsetAsync");
    NoteDeviceWrite(out.data, CheckedBytes(seq, hidden));
    LaunchEmbedding(static_cast<const int32_t*>(ids.data) + id_offset, nullptr, table, row_scale,
                    static_cast<float*>(out.data), seq, hidden, vocab, bad, ctx.stream);
    int32_t flag = 0;
    Check(hipMemcpyAsync(&flag, bad, sizeof(flag), hipMemcpyDeviceToHost, ctx.stream), "hipMemcpyAsync");
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    if (flag != 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "token id is outside the vocabulary");
  });
}

// Device::RmsNorm (src/sim_device.cc:257-265).
ACCEL_HIP_API int accel_hip_rms_norm(AccelHipBuffer x, AccelHipBuffer weight, AccelHipBuffer y, int64_t rows,
                                     int64_t dim, float eps, int64_t row_offset) {
  return Guard([&] {
    const int64_t x_rows = CheckedSpan(row_offset, rows);
    RequireBytes(x, CheckedBytes(x_rows, dim), "RmsNorm input is out of range");
    RequireBytes(weight, CheckedBytes(dim, 1), "RmsNorm weight is out of range");
    RequireBytes(y, CheckedBytes(rows, dim), "RmsNorm output is out of range");
    NoteDeviceWrite(y.data, CheckedBytes(rows, dim));
    LaunchRmsNormRows(static_cast<const float*>(x.data) + row_offset * dim, static_cast<const float*>(weight.data),
                      static_cast<float*>(y.data), rows, dim, eps, Ctx().stream);
  });
}

// Device::Rope (src/sim_device.cc:267-275).
ACCEL_HIP_API int accel_hip_rope(AccelHipBuffer states, AccelHipBuffer cos_table, AccelHipBuffer sin_table,
                                 int64_t seq, int64_t n_heads, int64_t head_dim, int64_t position) {
  return Guard([&] {
    const int64_t positions = CheckedSpan(position, seq);
    RequireBytes(states, CheckedFloats(seq, n_heads, head_dim), "Rope states are out of range");
    RequireBytes(cos_table, CheckedBytes(positions, head_dim), "Rope cos table is out of range");
    RequireBytes(sin_table, CheckedBytes(positions, head_dim), "Rope sin table is out of range");
    NoteDeviceWrite(states.data, CheckedFloats(seq, n_heads, head_dim));
    LaunchRope(static_cast<float*>(states.data), static_cast<const float*>(cos_table.data),
               static_cast<const float*>(sin_table.data), seq, n_heads, head_dim, position, Ctx().stream);
  });
}

// Device::AppendCache (src/sim_device.cc:277-284).
ACCEL_HIP_API int accel_hip_append_cache(AccelHipBuffer src, AccelHipBuffer cache, int64_t seq, int64_t position,
                                         int64_t n_heads, int64_t head_dim) {
  return Guard([&] {
    const int64_t rows = CheckedSpan(position, seq);
    RequireBytes(src, CheckedFloats(seq, n_heads, head_dim), "AppendCache source is out of range");
    RequireBytes(cache, CheckedFloats(rows, n_heads, head_dim), "AppendCache cache is out of range");
    const int64_t row = n_heads * head_dim;
    NoteDeviceWrite(static_cast<float*>(cache.data) + position * row, static_cast<size_t>(seq * row) * sizeof(float));
    LaunchCopy(static_cast<float*>(cache.data) + position * row, src.data,
               static_cast<size_t>(seq * row) * sizeof(float), Ctx().stream);
  });
}

// Device::Attention (src/sim_device.cc:286-300).
ACCEL_HIP_API int accel_hip_attention(AccelHipBuffer q, AccelHipBuffer k, AccelHipBuffer v, AccelHipBuffer scores,
                                      AccelHipBuffer out, int64_t seq, int64_t position, int64_t heads,
                                      int64_t kv_heads, int64_t head_dim) {
  return Guard([&] {
    if (kv_heads <= 0 || (heads > 0 && heads % kv_heads != 0))
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention kv heads are out of range");
    const int64_t seen = CheckedSpan(position, seq);
    RequireBytes(q, CheckedFloats(seq, heads, head_dim), "Attention query is out of range");
    RequireBytes(k, CheckedFloats(seen, kv_heads, head_dim), "Attention key is out of range");
    RequireBytes(v, CheckedFloats(seen, kv_heads, head_dim), "Attention value is out of range");
    RequireBytes(scores, CheckedBytes(seen, 1), "Attention scores are out of range");
    RequireBytes(out, CheckedFloats(seq, heads, head_dim), "Attention output is out of range");
    if (seq == 0 || heads == 0 || head_dim == 0) return;
    NoteDeviceWrite(out.data, CheckedFloats(seq, heads, head_dim));
    LaunchAttention(static_cast<const float*>(q.data), static_cast<const float*>(k.data),
                    static_cast<const float*>(v.data), static_cast<float*>(out.data), seq, position, heads, kv_heads,
                    head_dim, Ctx().stream);
  });
}

// Device::SiluMul (src/sim_device.cc:302-307).
ACCEL_HIP_API int accel_hip_silu_mul(AccelHipBuffer gate, AccelHipBuffer up, int64_t count) {
  return Guard([&] {
    const size_t bytes = CheckedBytes(count, 1);
    RequireBytes(gate, bytes, "SiluMul gate is out of range");
    RequireBytes(up, bytes, "SiluMul up is out of range");
    NoteDeviceWrite(gate.data, bytes);
    LaunchSiluMul(static_cast<float*>(gate.data), static_cast<const float*>(up.data), count, Ctx().stream);
  });
}

// Device::ResidualAdd (src/sim_device.cc:309-314).
ACCEL_HIP_API int accel_hip_residual_add(AccelHipBuffer dest, AccelHipBuffer extra, int64_t count) {
  return Guard([&] {
    const size_t bytes = CheckedBytes(count, 1);
    RequireBytes(dest, bytes, "ResidualAdd destination is out of range");
    RequireBytes(extra, bytes, "ResidualAdd extra is out of range");
    NoteDeviceWrite(dest.data, bytes);
    LaunchResidualAdd(static_cast<float*>(dest.data), static_cast<const float*>(extra.data), count, Ctx().stream);
  });
}

// Device::SampleToken (src/sim_device.cc:316-328). The state word makes a round trip only
// when a draw can happen (temperature > 0).
ACCEL_HIP_API int accel_hip_sample_token(AccelHipBuffer logits, AccelHipBuffer chosen_ids, int64_t chosen_index,
                                         int64_t vocab, float temperature, uint32_t* rng_state, int32_t top_k) {
  return Guard([&] {
    if (vocab <= 0 || chosen_index < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "SampleToken is out of range");
    if (rng_state == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "SampleToken rng is out of range");
    RequireBytes(logits, CheckedBytes(vocab, 1), "SampleToken logits are out of range");
    RequireBytes(chosen_ids, CheckedIntBytes(CheckedSpan(chosen_index, 1)), "SampleToken ids are out of range");
    Context& ctx = Ctx();
    const bool draw = temperature > 0.f;
    if (draw) RefuseInCapture("SampleToken with temperature > 0 (its rng state makes a host round trip)");
    uint32_t* word = static_cast<uint32_t*>(Temp(kTempFlags, 64)) + 4;
    if (draw) Check(hipMemcpyAsync(word, rng_state, sizeof(uint32_t), hipMemcpyHostToDevice, ctx.stream), "hipMemcpyAsync");
    if (draw) Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    NoteDeviceWrite(static_cast<int32_t*>(chosen_ids.data) + chosen_index, sizeof(int32_t));
    void* greedy = draw ? nullptr : Temp(kTempGreedy, GreedyWorkBytes(vocab));
    LaunchSampleToken(static_cast<const float*>(logits.data), static_cast<int32_t*>(chosen_ids.data) + chosen_index,
                      vocab, temperature, word, top_k, ctx.stream, nullptr, greedy, draw ? 0 : GreedyWorkBytes(vocab));
    if (draw) {
      Check(hipMemcpyAsync(rng_state, word, sizeof(uint32_t), hipMemcpyDeviceToHost, ctx.stream), "hipMemcpyAsync");
      Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    }
  });
}

}  // extern "C"
