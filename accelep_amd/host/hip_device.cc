// accel::Device on one MI355X, over the accel_hip C-ABI (include/accel_hip.h).
//
// Takes the place of AccelEP's SimDevice (src/sim_device.cc:127-377) and of the free
// functions that file defines (MatMulQuantized, LiveDeviceAllocs, the packed-GEMM probes):
// every call is forwarded to the library, whose status codes are rethrown as the exception
// types SimDevice throws for the same condition. The runtime counters are noted here as
// SimDevice notes them (src/sim_device.cc:171,182,193-195,208,599-601), so code that reads
// GetAcceleratorStats() sees the same values.
//
// It needs only include/accel/device.h and runtime.h (source-compatible with the reference's),
// include/accel/hip_device.h and include/accel_hip.h, so it also builds inside the reference
// tree in place of src/sim_device.cc.
#include <new>
#include <stdexcept>
#include <string>

#include "accel/device.h"
#include "accel/hip_device.h"
#include "accel/runtime.h"
#include "accel_hip.h"

namespace accel {
namespace {

[[noreturn]] void ThrowStatus(int rc) {
  const std::string message = accel_hip_last_error();
  switch (rc) {
    case ACCEL_HIP_INVALID_ARGUMENT:
      throw std::invalid_argument(message);
    case ACCEL_HIP_OVERFLOW:
      throw std::overflow_error(message);
    case ACCEL_HIP_LOGIC_ERROR:
      throw std::logic_error(message);
    case ACCEL_HIP_BAD_ALLOC:
      throw std::bad_alloc();
    default:
      throw std::runtime_error(message.empty() ? std::string("HIP device call failed") : message);
  }
}

void Check(int rc) {
  if (rc != ACCEL_HIP_OK) ThrowStatus(rc);
}

AccelHipBuffer ToHip(DeviceBuffer b) { return AccelHipBuffer{b.data, b.bytes, b.id}; }

int32_t ToHip(Activation activation) {
  switch (activation) {
    case Activation::Relu:
      return ACCEL_HIP_ACT_RELU;
    case Activation::Gelu:
      return ACCEL_HIP_ACT_GELU;
    case Activation::None:
      break;
  }
  return ACCEL_HIP_ACT_NONE;
}

// QuantPlane (shape as a vector) -> the C-ABI plane (shape inline, rank <= 8).
AccelHipQuantPlane ToHip(const QuantPlane& plane) {
  if (plane.shape.size() > 8) throw std::invalid_argument("quantized plane rank is out of range");
  AccelHipQuantPlane out{};
  out.q = plane.q;
  out.scale = plane.scale;
  out.zero = plane.zero;
  out.rank = static_cast<int32_t>(plane.shape.size());
  for (size_t d = 0; d < plane.shape.size(); ++d) out.shape[d] = plane.shape[d];
  out.axis = plane.axis;
  out.offset = plane.offset;
  return out;
}

AccelHipEpilogue ToHip(const FusedEpilogue& e) {
  if (e.bias != nullptr && e.bias_shape.size() > 2) throw std::invalid_argument("Gemm bias rank is out of range");
  AccelHipEpilogue out{};
  out.alpha = e.alpha;
  out.beta = e.beta;
  out.bias = e.bias;
  out.bias_rank = e.bias == nullptr ? 0 : static_cast<int32_t>(e.bias_shape.size());
  for (size_t d = 0; e.bias != nullptr && d < e.bias_shape.size(); ++d) out.bias_shape[d] = e.bias_shape[d];
  out.activation = ToHip(e.activation);
  out.residual = e.residual;
  out.rms_weight = nullptr;
  out.rms_eps = 0.f;
  out.rms_out = nullptr;
  return out;
}

class HipDevice final : public Device {
 public:
  HipDevice() { Check(accel_hip_init()); }
  // Frees nothing: an allocation never freed stays in LiveDeviceAllocs(), as with SimDevice.
  ~HipDevice() override = default;

  const char* Name() const override { return "hip"; }

  DeviceBuffer Allocate(size_t bytes) override {
    AccelHipBuffer b{};
    Check(accel_hip_allocate(bytes, &b));
    return DeviceBuffer{b.data, b.bytes, b.id};
  }

  void Free(DeviceBuffer buffer) override { Check(accel_hip_free(ToHip(buffer))); }

  void CopyHostToDevice(DeviceBuffer dst, const void* src, size_t bytes) override {
    Check(accel_hip_copy_h2d(ToHip(dst), src, bytes));
    if (bytes != 0) NoteBytesToDevice(bytes);
  }

  void CopyDeviceToHost(void* dst, DeviceBuffer src, size_t bytes) override {
    Check(accel_hip_copy_d2h(dst, ToHip(src), bytes));
    if (bytes != 0) NoteBytesToHost(bytes);
  }

  void MatMul(DeviceBuffer a, DeviceBuffer b, DeviceBuffer c, int64_t m, int64_t k, int64_t n) override {
    Check(accel_hip_matmul(ToHip(a), ToHip(b), ToHip(c), m, k, n));
    NoteKernelMatmul();
  }

  void Transpose(DeviceBuffer src, DeviceBuffer dst, int64_t rows, int64_t cols) override {
    Check(accel_hip_transpose(ToHip(src), ToHip(dst), rows, cols));
    NoteDeviceTranspose();
  }

  void GemmEpilogue(DeviceBuffer c, int64_t m, int64_t n, float alpha, const DeviceBuffer* bias,
                    const std::vector<int64_t>& bias_shape, float beta, Activation activation) override {
    AccelHipBuffer hb{};
    if (bias != nullptr) hb = ToHip(*bias);
    Check(accel_hip_gemm_epilogue(ToHip(c), m, n, alpha, bias != nullptr ? &hb : nullptr,
                                  static_cast<int32_t>(bias_shape.size()), bias_shape.data(), beta, ToHip(activation)));
  }

  void Embedding(DeviceBuffer ids, int64_t id_offset, DeviceBuffer table, DeviceBuffer out, int64_t seq,
                 int64_t hidden, int64_t vocab) override {
    Check(accel_hip_embedding(ToHip(ids), id_offset, ToHip(table), ToHip(out), seq, hidden, vocab));
  }

  void RmsNorm(DeviceBuffer x, DeviceBuffer weight, DeviceBuffer y, int64_t rows, int64_t dim, float eps,
               int64_t row_offset) override {
    Check(accel_hip_rms_norm(ToHip(x), ToHip(weight), ToHip(y), rows, dim, eps, row_offset));
  }

  void Rope(DeviceBuffer states, DeviceBuffer cos_table, DeviceBuffer sin_table, int64_t seq, int64_t n_heads,
            int64_t head_dim, int64_t position) override {
    Check(accel_hip_rope(ToHip(states), ToHip(cos_table), ToHip(sin_table), seq, n_heads, head_dim, position));
  }

  void AppendCache(DeviceBuffer src, DeviceBuffer cache, int64_t seq, int64_t position, int64_t n_heads,
                   int64_t head_dim) override {
    Check(accel_hip_append_cache(ToHip(src), ToHip(cache), seq, position, n_heads, head_dim));
  }

  void Attention(DeviceBuffer q, DeviceBuffer k, DeviceBuffer v, DeviceBuffer scores, DeviceBuffer out, int64_t seq,
                 int64_t position, int64_t heads, int64_t kv_heads, int64_t head_dim) override {
    Check(accel_hip_attention(ToHip(q), ToHip(k), ToHip(v), ToHip(scores), ToHip(out), seq, position, heads,
                              kv_heads, head_dim));
  }

  void SiluMul(DeviceBuffer gate, DeviceBuffer up, int64_t count) override {
    Check(accel_hip_silu_mul(ToHip(gate), ToHip(up), count));
  }

  void ResidualAdd(DeviceBuffer dest, DeviceBuffer extra, int64_t count) override {
    Check(accel_hip_residual_add(ToHip(dest), ToHip(extra), count));
  }

  void SampleToken(DeviceBuffer logits, DeviceBuffer chosen_ids, int64_t chosen_index, int64_t vocab,
                   float temperature, uint32_t* rng_state, int top_k) override {
    Check(accel_hip_sample_token(ToHip(logits), ToHip(chosen_ids), chosen_index, vocab, temperature, rng_state,
                                 top_k));
  }
};

}  // namespace

std::unique_ptr<Device> CreateHipDevice() { return std::make_unique<HipDevice>(); }

int64_t LiveDeviceAllocs() { return accel_hip_live_allocs(); }

int64_t PackedMatMulCalls() { return accel_hip_packed_matmul_calls(); }
int64_t PackedKTrips() { return accel_hip_packed_k_trips(); }
void ResetPackedGemmProbes() { accel_hip_reset_packed_probes(); }

void MatMulQuantized(const float* a, const QuantPlane* a_quant, const float* b, const QuantPlane* b_quant, float* c,
                     int64_t m, int64_t k, int64_t n) {
  AccelHipQuantPlane aq{}, bq{};
  if (a_quant != nullptr) aq = ToHip(*a_quant);
  if (b_quant != nullptr) bq = ToHip(*b_quant);
  Check(accel_hip_matmul_quantized(a, a_quant != nullptr ? &aq : nullptr, b, b_quant != nullptr ? &bq : nullptr, c, m,
                                   k, n));
  NoteKernelMatmul();
}

bool IsHipDevice(const Device& device) { return dynamic_cast<const HipDevice*>(&device) != nullptr; }

void HipMatMulFused(Device& device, DeviceBuffer a, DeviceBuffer b, DeviceBuffer c, int64_t m, int64_t k, int64_t n,
                    const FusedEpilogue& epilogue) {
  if (!IsHipDevice(device)) throw std::invalid_argument("fused matmul needs the HIP device");
  // The fused entry takes raw pointers: check the buffers as MatMul does.
  auto need = [](int64_t rows, int64_t cols) -> size_t {
    if (rows < 0 || cols < 0) throw std::invalid_argument("negative matrix dimension");
    if (cols != 0 && rows > static_cast<int64_t>(SIZE_MAX / sizeof(float)) / cols)
      throw std::overflow_error("matrix is too large");
    return static_cast<size_t>(rows * cols) * sizeof(float);
  };
  auto require = [](DeviceBuffer buf, size_t bytes, const char* what) {
    if (bytes != 0 && (buf.data == nullptr || buf.bytes < bytes)) throw std::invalid_argument(what);
  };
  require(a, need(m, k), "MatMul A is out of range");
  require(b, need(k, n), "MatMul B is out of range");
  require(c, need(m, n), "MatMul C is out of range");
  const AccelHipEpilogue e = ToHip(epilogue);
  Check(accel_hip_matmul_fused(static_cast<const float*>(a.data), static_cast<const float*>(b.data),
                               static_cast<float*>(c.data), m, k, n, &e));
  NoteKernelMatmul();
}

void HipMatMulQuantizedFused(const float* a, const QuantPlane* a_quant, const float* b, const QuantPlane* b_quant,
                             float* c, int64_t m, int64_t k, int64_t n, const FusedEpilogue& epilogue) {
  AccelHipQuantPlane aq{}, bq{};
  if (a_quant != nullptr) aq = ToHip(*a_quant);
  if (b_quant != nullptr) bq = ToHip(*b_quant);
  const AccelHipEpilogue e = ToHip(epilogue);
  Check(accel_hip_matmul_quantized_fused(a, a_quant != nullptr ? &aq : nullptr, b, b_quant != nullptr ? &bq : nullptr,
                                         c, m, k, n, &e));
  NoteKernelMatmul();
}

void HipPrepareQuantized(const QuantPlane& weight) {
  if (weight.shape.size() < 2) throw std::invalid_argument("prepare needs a matrix weight");
  const int64_t k = weight.shape[weight.shape.size() - 2];
  const int64_t n = weight.shape.back();
  int64_t batches = 1;
  for (size_t d = 0; d + 2 < weight.shape.size(); ++d) batches *= weight.shape[d];
  AccelHipQuantPlane plane = ToHip(weight);
  for (int64_t b = 0; b < batches; ++b) {
    plane.offset = weight.offset + b * k * n;
    Check(accel_hip_prepare_quantized(&plane, k, n, 0, nullptr));
  }
}

void HipSynchronize() { Check(accel_hip_synchronize()); }

void HipSetExactProducts(bool on) { Check(accel_hip_set_exact_products(on ? 1 : 0)); }
bool HipExactProducts() { return accel_hip_exact_products() != 0; }

}  // namespace accel
