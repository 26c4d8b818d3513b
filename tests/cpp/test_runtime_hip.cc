// The runtime's tests on the MI355X device: the checks of AccelEP tests/test_runtime.cc
// (same inputs, hand values, bit patterns and counter values; file:line cited per test),
// run through accel::CreateHipDevice(). Products the reference compares bit for bit with
// its sequential k-order loop are checked here against Higham's inner-product bound
// |got - A@B| <= 2*gamma_K*(|A|@|B|), gamma_K = K*2^-24/(1 - K*2^-24), because the matrix
// cores add in another order. Every other value is compared exactly.
//
// A pass-through device (Recorder) sends the runtime down its generic path (MatMul, then
// GemmEpilogue passes); the HIP device takes the fused path. Both must store identical bits.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "accel/device.h"
#include "accel/hip_device.h"
#include "accel/runtime.h"

namespace {

int g_failures = 0;
int g_checks = 0;

void Expect(bool ok, const char* what, int line) {
  ++g_checks;
  if (!ok) {
    std::fprintf(stderr, "FAIL line %d: %s\n", line, what);
    ++g_failures;
  }
}
#define EXPECT(cond) Expect(static_cast<bool>(cond), #cond, __LINE__)

uint32_t Bits(float v) {
  uint32_t b;
  std::memcpy(&b, &v, 4);
  return b;
}
float FromBits(uint32_t b) {
  float v;
  std::memcpy(&v, &b, 4);
  return v;
}

void ExpectValues(const std::vector<float>& got, const std::vector<float>& want, int line) {
  bool ok = got.size() == want.size();
  for (size_t i = 0; ok && i < got.size(); ++i) {
    const float tol = 1e-5f * std::max(1.f, std::fabs(want[i]));
    if (!(std::fabs(got[i] - want[i]) <= tol)) {
      std::fprintf(stderr, "  index %zu: got %.9g want %.9g\n", i, got[i], want[i]);
      ok = false;
    }
  }
  Expect(ok, "values match", line);
}
#define EXPECT_VALUES(got, ...) ExpectValues(got, std::vector<float> __VA_ARGS__, __LINE__)

void ExpectSameBits(const std::vector<float>& got, const std::vector<float>& want, int line) {
  bool ok = got.size() == want.size() && std::memcmp(got.data(), want.data(), got.size() * 4) == 0;
  if (!ok && got.size() == want.size()) {
    for (size_t i = 0; i < got.size(); ++i)
      if (Bits(got[i]) != Bits(want[i])) {
        std::fprintf(stderr, "  index %zu: %08x vs %08x\n", i, Bits(got[i]), Bits(want[i]));
        break;
      }
  }
  Expect(ok, "identical bits", line);
}

// C = A @ B against the gamma_K bound, from a double-precision host product.
void ExpectProductBound(const std::vector<float>& got, const std::vector<float>& a, const std::vector<float>& b,
                        int64_t m, int64_t k, int64_t n, int line) {
  const double u = std::ldexp(1.0, -24);
  const double gamma = k * u / (1.0 - k * u);
  bool ok = got.size() == static_cast<size_t>(m * n);
  for (int64_t i = 0; ok && i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double exact = 0, mag = 0;
      for (int64_t p = 0; p < k; ++p) {
        exact += static_cast<double>(a[i * k + p]) * b[p * n + j];
        mag += std::fabs(static_cast<double>(a[i * k + p]) * b[p * n + j]);
      }
      const double err = std::fabs(got[i * n + j] - exact);
      if (!(err <= 2 * gamma * mag + 1e-30)) {
        std::fprintf(stderr, "  (%lld, %lld): got %.9g exact %.9g bound %.3g\n", static_cast<long long>(i),
                     static_cast<long long>(j), got[i * n + j], exact, 2 * gamma * mag);
        ok = false;
        break;
      }
    }
  Expect(ok, "product within 2*gamma_K*(|A|@|B|)", line);
}

// The LCG of tests/test_runtime.cc:225-232.
void FillLcg(std::vector<float>* out, int64_t count, uint32_t* seed) {
  out->resize(static_cast<size_t>(count));
  for (int64_t i = 0; i < count; ++i) {
    *seed = *seed * 1664525u + 1013904223u;
    (*out)[static_cast<size_t>(i)] =
        static_cast<float>(static_cast<double>(static_cast<int>(*seed % 10007u) - 5003) * 0.1);
  }
}

template <typename F>
bool Throws(F f, const char* substring = nullptr) {
  try {
    f();
  } catch (const std::invalid_argument& e) {
    return substring == nullptr || std::strstr(e.what(), substring) != nullptr;
  }
  return false;
}

accel::Operand Host(const std::vector<float>& v, std::vector<int64_t> shape) {
  accel::Operand op;
  op.host = v.data();
  op.shape = std::move(shape);
  return op;
}

accel::OwnedBuffer UploadBytes(accel::Device& device, const void* data, size_t bytes) {
  accel::OwnedBuffer owned;
  owned.device = &device;
  owned.buffer = device.Allocate(bytes);
  if (bytes > 0) device.CopyHostToDevice(owned.buffer, data, bytes);
  return owned;
}

// Forwards every call to an inner device and records what was called.
struct Op {
  std::string name;
  uint64_t id = 0;
  size_t bytes = 0;
  int64_t m = 0, k = 0, n = 0;
  float alpha = 0, beta = 0;
  bool has_bias = false;
  void* dst = nullptr;
};

class Recorder final : public accel::Device {
 public:
  explicit Recorder(accel::Device& inner) : inner_(inner) {}
  std::vector<Op> ops;

  const char* Name() const override { return "recorder"; }
  accel::DeviceBuffer Allocate(size_t bytes) override {
    const accel::DeviceBuffer b = inner_.Allocate(bytes);
    ops.push_back(Op{"Allocate", b.id, bytes});
    return b;
  }
  void Free(accel::DeviceBuffer b) override {
    ops.push_back(Op{"Free", b.id, b.bytes});
    inner_.Free(b);
  }
  void CopyHostToDevice(accel::DeviceBuffer d, const void* s, size_t n) override {
    ops.push_back(Op{"CopyHostToDevice", d.id, n});
    inner_.CopyHostToDevice(d, s, n);
  }
  void CopyDeviceToHost(void* d, accel::DeviceBuffer s, size_t n) override {
    ops.push_back(Op{"CopyDeviceToHost", s.id, n});
    inner_.CopyDeviceToHost(d, s, n);
  }
  void MatMul(accel::DeviceBuffer a, accel::DeviceBuffer b, accel::DeviceBuffer c, int64_t m, int64_t k,
              int64_t n) override {
    Op op{"MatMul", c.id, c.bytes};
    op.m = m, op.k = k, op.n = n, op.dst = c.data;
    ops.push_back(op);
    inner_.MatMul(a, b, c, m, k, n);
  }
  void Transpose(accel::DeviceBuffer s, accel::DeviceBuffer d, int64_t rows, int64_t cols) override {
    Op op{"Transpose", d.id, d.bytes};
    op.m = rows, op.n = cols, op.dst = d.data;
    ops.push_back(op);
    inner_.Transpose(s, d, rows, cols);
  }
  void GemmEpilogue(accel::DeviceBuffer c, int64_t m, int64_t n, float alpha, const accel::DeviceBuffer* bias,
                    const std::vector<int64_t>& shape, float beta, accel::Activation act) override {
    Op op{"GemmEpilogue", c.id, c.bytes};
    op.m = m, op.n = n, op.alpha = alpha, op.beta = beta, op.has_bias = bias != nullptr;
    ops.push_back(op);
    inner_.GemmEpilogue(c, m, n, alpha, bias, shape, beta, act);
  }
  void Embedding(accel::DeviceBuffer i, int64_t o, accel::DeviceBuffer t, accel::DeviceBuffer out, int64_t s,
                 int64_t h, int64_t v) override {
    inner_.Embedding(i, o, t, out, s, h, v);
  }
  void RmsNorm(accel::DeviceBuffer x, accel::DeviceBuffer w, accel::DeviceBuffer y, int64_t r, int64_t d, float e,
               int64_t o) override {
    inner_.RmsNorm(x, w, y, r, d, e, o);
  }
  void Rope(accel::DeviceBuffer s, accel::DeviceBuffer c, accel::DeviceBuffer sn, int64_t q, int64_t h, int64_t d,
            int64_t p) override {
    inner_.Rope(s, c, sn, q, h, d, p);
  }
  void AppendCache(accel::DeviceBuffer s, accel::DeviceBuffer c, int64_t q, int64_t p, int64_t h, int64_t d) override {
    inner_.AppendCache(s, c, q, p, h, d);
  }
  void Attention(accel::DeviceBuffer q, accel::DeviceBuffer k, accel::DeviceBuffer v, accel::DeviceBuffer s,
                 accel::DeviceBuffer o, int64_t sq, int64_t p, int64_t h, int64_t kh, int64_t d) override {
    inner_.Attention(q, k, v, s, o, sq, p, h, kh, d);
  }
  void SiluMul(accel::DeviceBuffer g, accel::DeviceBuffer u, int64_t c) override { inner_.SiluMul(g, u, c); }
  void ResidualAdd(accel::DeviceBuffer d, accel::DeviceBuffer e, int64_t c) override { inner_.ResidualAdd(d, e, c); }
  void SampleToken(accel::DeviceBuffer l, accel::DeviceBuffer c, int64_t i, int64_t v, float t, uint32_t* r,
                   int k) override {
    inner_.SampleToken(l, c, i, v, t, r, k);
  }

  std::vector<Op> Named(const char* name) const {
    std::vector<Op> out;
    for (const Op& op : ops)
      if (op.name == name) out.push_back(op);
    return out;
  }
  std::vector<Op> Compute() const {
    std::vector<Op> out;
    for (const Op& op : ops)
      if (op.name == "Transpose" || op.name == "MatMul" || op.name == "GemmEpilogue") out.push_back(op);
    return out;
  }

 private:
  accel::Device& inner_;
};

// ---- tests/test_runtime.cc:39-201 -------------------------------------------------------

void TestHandValues(accel::Device& dev) {
  std::vector<float> out(4);
  accel::ExecuteMatMul(dev, Host({1, 2, 3, 4}, {2, 2}), Host({5, 6, 7, 8}, {2, 2}), out.data());
  EXPECT_VALUES(out, {19, 22, 43, 50});

  const std::vector<float> a8 = {1, 2, 3, 4, 5, 6, 7, 8};
  std::vector<float> out8(8);
  accel::ExecuteMatMul(dev, Host(a8, {2, 2, 2}), Host({1, 0, 0, 1}, {2, 2}), out8.data());
  EXPECT_VALUES(out8, {1, 2, 3, 4, 5, 6, 7, 8});

  // (2,1,2,2) @ (1,2,2,2): broadcast both ways (tests/test_runtime.cc:57-69).
  std::vector<float> out16(16);
  accel::ExecuteMatMul(dev, Host({1, 2, 3, 4, 1, 2, 3, 4}, {2, 1, 2, 2}), Host({1, 0, 0, 1, 0, 1, 1, 0}, {1, 2, 2, 2}),
                       out16.data());
  EXPECT_VALUES(out16, {1, 2, 3, 4, 2, 1, 4, 3, 1, 2, 3, 4, 2, 1, 4, 3});

  // Gemm transB, alpha 2, bias [2] (:71-84).
  accel::GemmConfig cfg;
  cfg.trans_b = true;
  cfg.alpha = 2.f;
  const std::vector<float> bias = {1, 3};
  const accel::Operand bias_op = Host(bias, {2});
  accel::ExecuteGemm(dev, Host({1, 2, 3, 4, 5, 6}, {2, 3}), Host({1, 0, 1, 0, 1, 1}, {2, 3}), &bias_op, cfg,
                     out.data());
  EXPECT_VALUES(out, {9, 13, 21, 25});

  // FusedMatMul transA, alpha 1.5 (:144-156); batched transB (:158-169).
  accel::FusedMatMulConfig fcfg;
  fcfg.trans_a = true;
  fcfg.alpha = 1.5f;
  accel::ExecuteFusedMatMul(dev, Host({1, 2, 3, 4, 5, 6}, {3, 2}), Host({1, 0, 0, 1, 1, 1}, {3, 2}), fcfg,
                            accel::Activation::None, out.data());
  EXPECT_VALUES(out, {9, 12, 12, 15});
  accel::FusedMatMulConfig tb;
  tb.trans_b = true;
  accel::ExecuteFusedMatMul(dev, Host({1, 2, 3, 4, 5, 6, 1, 0, 1, 0, 1, 1}, {2, 2, 3}),
                            Host({1, 0, 1, 0, 1, 1}, {2, 3}), tb, accel::Activation::None, out8.data());
  EXPECT_VALUES(out8, {4, 5, 10, 11, 2, 1, 1, 2});

  // k = 0 writes zeros (:106-113).
  std::vector<float> out6(6, 7.f);
  const std::vector<float> empty;
  accel::ExecuteMatMul(dev, Host(empty, {2, 0}), Host(empty, {0, 3}), out6.data());
  EXPECT_VALUES(out6, {0, 0, 0, 0, 0, 0});
}

void TestCountersAndResidency(accel::Device& dev) {
  // tests/test_runtime.cc:86-104: a device weight is not uploaded again.
  std::vector<float> b = {5, 6, 7, 8};
  accel::OwnedBuffer weight = accel::Upload(dev, b.data(), {2, 2});
  b[0] = 0;
  accel::ResetAcceleratorStats();
  std::vector<float> out(4);
  accel::Operand b_op;
  b_op.on_device = &weight;
  b_op.shape = weight.shape;
  accel::ExecuteMatMul(dev, Host({1, 2, 3, 4}, {2, 2}), b_op, out.data());
  EXPECT_VALUES(out, {19, 22, 43, 50});
  accel::AcceleratorStats s = accel::GetAcceleratorStats();
  EXPECT(s.bytes_to_device == 16 && s.matmul_ops == 1 && s.kernel_matmuls == 1 && s.bytes_to_host == 16);

  // Relu stays on the device (:171-185).
  accel::ResetAcceleratorStats();
  std::vector<float> relu(4, 9.f);
  accel::ExecuteMatMul(dev, Host({1, -2, -3, 4}, {2, 2}), Host({1, 0, 0, 1}, {2, 2}), relu.data(),
                       accel::Activation::Relu);
  EXPECT_VALUES(relu, {1, 0, 0, 4});
  s = accel::GetAcceleratorStats();
  EXPECT(s.relu_epilogues == 1 && s.matmul_ops == 1 && s.bytes_to_host == 16 && s.bytes_to_device == 32);

  // Gemm bias + Relu (:187-201).
  accel::ResetAcceleratorStats();
  const std::vector<float> bias = {-2, 3};
  const accel::Operand bias_op = Host(bias, {2});
  accel::ExecuteGemm(dev, Host({1, 0, 0, 1}, {2, 2}), Host({1, 0, 0, 1}, {2, 2}), &bias_op, accel::GemmConfig{},
                     out.data(), accel::Activation::Relu);
  EXPECT_VALUES(out, {0, 3, 0, 4});
  EXPECT(accel::GetAcceleratorStats().relu_epilogues == 1 && accel::GetAcceleratorStats().gemm_ops == 1);

  // Residual orientation (:461-484).
  accel::ResetAcceleratorStats();
  const std::vector<float> residual = {-1, 5, 0, -4};
  const accel::Operand res_op = Host(residual, {2, 2});
  std::vector<float> out9(4, 9.f);
  accel::ExecuteMatMul(dev, Host({1, 2, 3, 4}, {2, 2}), Host({1, 0, 0, 1}, {2, 2}), out9.data(),
                       accel::Activation::None, &res_op);
  EXPECT_VALUES(out9, {0, 7, 3, 0});
  s = accel::GetAcceleratorStats();
  EXPECT(s.add_epilogues == 1 && s.relu_epilogues == 0 && s.kernel_matmuls == 1);
  accel::ResetAcceleratorStats();
  const float dummy = 0.f;
  accel::Operand empty_res;
  empty_res.host = &dummy;
  empty_res.shape = {0};
  accel::Operand a0;
  a0.host = &dummy;
  a0.shape = {0, 1};
  accel::Operand b0;
  b0.host = &dummy;
  b0.shape = {1, 1};
  accel::ExecuteMatMul(dev, a0, b0, nullptr, accel::Activation::None, &empty_res);
  EXPECT(accel::GetAcceleratorStats().add_epilogues == 1 && accel::GetAcceleratorStats().kernel_matmuls == 1);

  // Stats survive a scope and count from the last reset (:547-563).
  accel::ResetAcceleratorStats();
  accel::ExecuteMatMul(dev, Host({1, 0, 0, 1}, {2, 2}), Host({1, 0, 0, 1}, {2, 2}), out.data());
  accel::ExecuteMatMul(dev, Host({1, 0, 0, 1}, {2, 2}), Host({1, 0, 0, 1}, {2, 2}), out.data());
  EXPECT(accel::GetAcceleratorStats().matmul_ops == 2);
}

void TestRejections(accel::Device& dev) {
  std::vector<int64_t> shape;
  EXPECT(!accel::InferMatMulShape({2, 3}, {4, 5}, &shape));
  EXPECT(!accel::InferGemmShape({2, 3}, false, {2, 3}, false, nullptr, &shape));
  EXPECT(!accel::InferFusedMatMulShape({2, 3}, true, {3, 4}, false, &shape));
  EXPECT(!accel::InferMatMulShape({-1, 8}, {8, 4}, &shape));
  EXPECT(!accel::InferMatMulShape({2, -1}, {-1, 4}, &shape));
  std::vector<float> six(6, 1.f), c(4);
  EXPECT(Throws([&] { accel::ExecuteMatMul(dev, Host(six, {2, 3}), Host(six, {2, 3}), c.data()); }));
  // Freeing memory the device never gave out is a logic_error (:132-142).
  float local = 1.f;
  bool logic = false;
  try {
    dev.Free(accel::DeviceBuffer{&local, sizeof(local), 0});
  } catch (const std::logic_error&) {
    logic = true;
  }
  EXPECT(logic);
}

// ---- packed-GEMM probes and product accuracy (:234-271) ----------------------------------

void TestProbesAndProducts(accel::Device& dev) {
  for (const auto& [m, k, n, seed0] : std::vector<std::tuple<int64_t, int64_t, int64_t, uint32_t>>{
           {128, 160, 96, 1}, {13, 19, 17, 2}}) {
    uint32_t seed = seed0;
    std::vector<float> a, b;
    FillLcg(&a, m * k, &seed);
    FillLcg(&b, k * n, &seed);
    accel::ResetPackedGemmProbes();
    std::vector<float> out(static_cast<size_t>(m * n), 1.f);
    accel::ExecuteMatMul(dev, Host(a, {m, k}), Host(b, {k, n}), out.data());
    ExpectProductBound(out, a, b, m, k, n, __LINE__);
    EXPECT(accel::PackedMatMulCalls() == 1 && accel::PackedKTrips() == k);
    accel::ResetAcceleratorStats();  // does not touch the probes
    EXPECT(accel::PackedMatMulCalls() == 1 && accel::PackedKTrips() == k);
  }
  accel::ResetPackedGemmProbes();
  accel::ResetAcceleratorStats();
  std::vector<float> one(1, 3.f);
  const float dummy = 0.f;
  accel::Operand a0, b0;
  a0.host = &dummy;
  a0.shape = {1, 0};
  b0.host = &dummy;
  b0.shape = {0, 1};
  accel::ExecuteMatMul(dev, a0, b0, one.data());
  EXPECT(one[0] == 0.f && accel::PackedMatMulCalls() == 1 && accel::PackedKTrips() == 0);
  EXPECT(accel::GetAcceleratorStats().kernel_matmuls == 1);

  // The split-product KAT (:413-425): 0xBE2694CD*1 + 0x3E41AF7D*0x3F5C2CB8 = 0xB5200000 with
  // each product rounded. The matrix cores do not round the products of one instruction
  // before adding them, so by default the value is checked against the fp32 tolerance;
  // TestExactProducts checks the bits.
  const float ah[2] = {FromBits(0xBE2694CDu), FromBits(0x3E41AF7Du)};
  const float bh[2] = {FromBits(0x3F800000u), FromBits(0x3F5C2CB8u)};
  accel::OwnedBuffer a = accel::Upload(dev, ah, {1, 2});
  accel::OwnedBuffer b = accel::Upload(dev, bh, {2, 1});
  accel::DeviceBuffer cbuf = dev.Allocate(sizeof(float));
  dev.MatMul(a.buffer, b.buffer, cbuf, 1, 2, 1);
  float got = 0.f;
  dev.CopyDeviceToHost(&got, cbuf, sizeof(got));
  dev.Free(cbuf);
  std::printf("  split-product KAT by default: %08x (the reference's bits: b5200000)\n", Bits(got));
  EXPECT(std::fabs(got - FromBits(0xB5200000u)) <= 1e-5f);
}

// ---- quantized operand (:325-405) ------------------------------------------------------

void TestQuantized(accel::Device& dev) {
  constexpr int64_t m = 8, k = 160, n = 300;
  uint32_t seed = 3;
  std::vector<float> a;
  FillLcg(&a, m * k, &seed);
  std::vector<int8_t> q(static_cast<size_t>(k * n));
  std::vector<float> scale(k);
  std::vector<int8_t> zero(k);
  for (auto& v : q) {
    seed = seed * 1664525u + 1013904223u;
    v = static_cast<int8_t>(static_cast<int>(seed % 251u) - 125);
  }
  for (int64_t r = 0; r < k; ++r) {
    scale[r] = static_cast<float>(r % 5) * 0.25f + 0.5f;
    zero[r] = static_cast<int8_t>(r % 7 - 3);
  }
  std::vector<float> w(static_cast<size_t>(k * n)), w_scalar(static_cast<size_t>(k * n));
  for (int64_t i = 0; i < k * n; ++i) {
    w[i] = (static_cast<float>(q[i]) - static_cast<float>(zero[i / n])) * scale[i / n];
    w_scalar[i] = static_cast<float>(q[i]) * 0.5f;
  }
  accel::OwnedBuffer qb = UploadBytes(dev, q.data(), q.size());
  accel::OwnedBuffer sb = UploadBytes(dev, scale.data(), scale.size() * 4);
  accel::OwnedBuffer zb = UploadBytes(dev, zero.data(), zero.size());
  accel::Operand bq;
  bq.quant = true;
  bq.shape = {k, n};
  bq.quant_plane.q = static_cast<const int8_t*>(qb.buffer.data);
  bq.quant_plane.scale = static_cast<const float*>(sb.buffer.data);
  bq.quant_plane.zero = static_cast<const int8_t*>(zb.buffer.data);
  bq.quant_plane.shape = {k, n};
  bq.quant_plane.axis = 0;
  accel::ResetPackedGemmProbes();
  accel::ResetAcceleratorStats();
  std::vector<float> out(static_cast<size_t>(m * n), 1.f);
  accel::ExecuteMatMul(dev, Host(a, {m, k}), bq, out.data());
  ExpectProductBound(out, a, w, m, k, n, __LINE__);
  EXPECT(accel::PackedMatMulCalls() == 1 && accel::PackedKTrips() == k);
  const accel::AcceleratorStats s = accel::GetAcceleratorStats();
  EXPECT(s.kernel_matmuls == 1 && s.matmul_ops == 1);
  EXPECT(s.bytes_to_device == m * k * 4 && s.bytes_to_host == m * n * 4);

  const float half = 0.5f;
  accel::OwnedBuffer hb = UploadBytes(dev, &half, sizeof(half));
  bq.quant_plane.scale = static_cast<const float*>(hb.buffer.data);
  bq.quant_plane.zero = nullptr;
  bq.quant_plane.axis = -1;
  accel::ExecuteMatMul(dev, Host(a, {m, k}), bq, out.data());
  ExpectProductBound(out, a, w_scalar, m, k, n, __LINE__);

  accel::FusedMatMulConfig cfg;
  cfg.trans_b = true;
  accel::Operand flipped = bq;
  flipped.shape = {n, k};
  EXPECT(Throws(
      [&] { accel::ExecuteFusedMatMul(dev, Host(a, {m, k}), flipped, cfg, accel::Activation::None, out.data()); },
      "transpose"));
}

// ---- non-finite epilogue bits (:427-459) -------------------------------------------------

void TestNonFiniteBits(accel::Device& dev) {
  const std::vector<float> pinf = {FromBits(0x7F800000u)}, ninf = {FromBits(0xFF800000u)}, zero = {0.f},
                           one = {1.f};
  std::vector<float> out(1);
  accel::ResetAcceleratorStats();
  accel::ExecuteMatMul(dev, Host(pinf, {1, 1}), Host(zero, {1, 1}), out.data(), accel::Activation::Relu);
  EXPECT(((Bits(out[0]) >> 23) & 0xffu) == 0xffu && (Bits(out[0]) & 0x7fffffu) != 0u);  // NaN survives Relu
  EXPECT(accel::GetAcceleratorStats().relu_epilogues == 1);
  accel::ExecuteMatMul(dev, Host(pinf, {1, 1}), Host(one, {1, 1}), out.data());
  EXPECT(Bits(out[0]) == 0x7F800000u);
  accel::ExecuteMatMul(dev, Host(ninf, {1, 1}), Host(one, {1, 1}), out.data(), accel::Activation::Relu);
  EXPECT(Bits(out[0]) == 0x00000000u);
  accel::GemmConfig cfg;
  cfg.alpha = -1.f;
  accel::ExecuteGemm(dev, Host(zero, {1, 1}), Host(one, {1, 1}), nullptr, cfg, out.data(), accel::Activation::Relu);
  EXPECT(Bits(out[0]) == 0x80000000u);  // -0 is not < 0: Relu keeps it
}

// ---- PretransposeLastTwo, KvTableStore, ids, private copies (:486-545,565-606,696-706) ----

void TestBuffersAndTables(accel::Device& dev) {
  const std::vector<float> v = {1, 2, 3, 4, 5, 6};
  accel::OwnedBuffer src = accel::Upload(dev, v.data(), {3, 2});
  accel::ResetAcceleratorStats();
  accel::OwnedBuffer dst;
  accel::PretransposeLastTwo(dev, src, &dst);
  EXPECT(dst.shape == std::vector<int64_t>({2, 3}));
  std::vector<float> back(6);
  dev.CopyDeviceToHost(back.data(), dst.buffer, 24);
  EXPECT_VALUES(back, {1, 3, 5, 2, 4, 6});
  EXPECT(accel::GetAcceleratorStats().device_transposes == 1);

  accel::KvTableStore store(dev);
  store.Create("k", 4, 2);
  float host[4] = {1, 2, 3, 4};
  store.Append("k", host, 2);
  host[0] = 0;
  const void* storage = store.Storage("k");
  accel::ResetAcceleratorStats();
  const float extra[2] = {5, 6};
  store.Append("k", extra, 1);
  EXPECT(accel::GetAcceleratorStats().bytes_to_device == 8);
  EXPECT(store.Storage("k") == storage && store.Filled("k") == 3);
  float rows[6] = {};
  store.Read("k", rows, 3);
  EXPECT_VALUES(std::vector<float>(rows, rows + 6), {1, 2, 3, 4, 5, 6});
  accel::KvTableStore other(dev);
  EXPECT(!other.Contains("k") && store.Contains("k"));
  EXPECT(Throws([&] { store.Update("k", 10, extra, 1); }));
  EXPECT(Throws([&] { store.Append("k", extra, 5); }));

  const int64_t before = accel::LiveDeviceAllocs();
  accel::DeviceBuffer first = dev.Allocate(128);
  const uint64_t first_id = first.id;
  dev.Free(first);
  accel::DeviceBuffer second = dev.Allocate(128);
  EXPECT(second.id > first_id);
  dev.Free(second);
  EXPECT(accel::LiveDeviceAllocs() == before);
  {
    auto leaking = accel::CreateHipDevice();
    accel::DeviceBuffer leaked = leaking->Allocate(64);
    const int64_t live = accel::LiveDeviceAllocs();
    leaking.reset();
    EXPECT(accel::LiveDeviceAllocs() == live);
    auto later = accel::CreateHipDevice();
    accel::DeviceBuffer after = later->Allocate(64);
    EXPECT(after.id > leaked.id);
    later->Free(after);
    later->Free(leaked);
  }

  float h[4] = {1, 2, 3, 4};
  accel::OwnedBuffer up = accel::Upload(dev, h, {2, 2});
  h[0] = 0;
  float b2[4] = {};
  dev.CopyDeviceToHost(b2, up.buffer, sizeof(b2));
  EXPECT(b2[0] == 1 && b2[1] == 2 && b2[2] == 3 && b2[3] == 4 && up.buffer.data != h);
}

// ---- call sequence of the generic path (:608-694) -----------------------------------------

void TestRecordedSequence(accel::Device& hip) {
  Recorder rec(hip);
  accel::ResetAcceleratorStats();
  std::vector<float> out(4);
  accel::FusedMatMulConfig cfg;
  cfg.trans_a = true;
  cfg.alpha = 1.5f;
  accel::ExecuteFusedMatMul(rec, Host({1, 2, 3, 4, 5, 6}, {3, 2}), Host({1, 0, 0, 1, 1, 1}, {3, 2}), cfg,
                            accel::Activation::None, out.data());
  EXPECT_VALUES(out, {9, 12, 12, 15});
  const std::vector<Op> allocs = rec.Named("Allocate"), frees = rec.Named("Free");
  EXPECT(allocs.size() == 4 && frees.size() == 4);
  EXPECT(rec.Named("CopyHostToDevice").size() == 2 && rec.Named("CopyDeviceToHost").size() == 1);
  if (allocs.size() == 4 && frees.size() == 4) {
    // A, B, C, then A transposed; ids rise in that order and are freed in reverse.
    EXPECT(allocs[0].bytes == 24 && allocs[1].bytes == 24 && allocs[2].bytes == 16 && allocs[3].bytes == 24);
    EXPECT(allocs[0].id < allocs[1].id && allocs[1].id < allocs[2].id && allocs[2].id < allocs[3].id);
    EXPECT(frees[0].id == allocs[3].id && frees[1].id == allocs[2].id && frees[2].id == allocs[1].id &&
           frees[3].id == allocs[0].id);
  }
  const std::vector<Op> compute = rec.Compute();
  EXPECT(compute.size() == 3);
  if (compute.size() == 3) {
    EXPECT(compute[0].name == "Transpose" && compute[0].m == 3 && compute[0].n == 2);
    EXPECT(compute[1].name == "MatMul" && compute[1].m == 2 && compute[1].k == 3 && compute[1].n == 2);
    EXPECT(compute[2].name == "GemmEpilogue" && compute[2].m == 4 && compute[2].n == 1 && compute[2].alpha == 1.5f &&
           compute[2].beta == 0.f && !compute[2].has_bias);
  }
  const accel::AcceleratorStats s = accel::GetAcceleratorStats();
  EXPECT(s.bytes_to_device == 48 && s.bytes_to_host == 16 && s.matmul_ops == 1 && s.gemm_ops == 0 &&
         s.kernel_matmuls == 1 && s.relu_epilogues == 0);

  // Batched transB: one transposed buffer reused per batch.
  Recorder rb(hip);
  std::vector<float> bo(8);
  accel::FusedMatMulConfig tb;
  tb.trans_b = true;
  accel::ExecuteFusedMatMul(rb, Host({1, 2, 3, 4, 5, 6, 1, 0, 1, 0, 1, 1}, {2, 2, 3}), Host({1, 0, 1, 0, 1, 1}, {2, 3}),
                            tb, accel::Activation::None, bo.data());
  EXPECT_VALUES(bo, {4, 5, 10, 11, 2, 1, 1, 2});
  const std::vector<Op> bc = rb.Compute();
  EXPECT(bc.size() == 4);
  if (bc.size() == 4) {
    EXPECT(bc[0].name == "Transpose" && bc[1].name == "MatMul" && bc[2].name == "Transpose" && bc[3].name == "MatMul");
    EXPECT(bc[0].dst == bc[2].dst);
  }
}

// ---- fused store == the reference's pass sequence, bit for bit ------------------------------

void TestFusedEqualsPasses(accel::Device& hip) {
  uint32_t seed = 11;
  const int64_t m = 37, k = 96, n = 70;
  std::vector<float> a, b, res, bias_row, bias_col;
  FillLcg(&a, m * k, &seed);
  FillLcg(&b, k * n, &seed);
  FillLcg(&res, m * n, &seed);
  FillLcg(&bias_row, n, &seed);
  FillLcg(&bias_col, m, &seed);
  for (auto* v : {&a, &b}) for (float& x : *v) x *= 0.01f;
  Recorder generic(hip);
  const accel::Operand res_op = Host(res, {m, n});
  for (const accel::Activation act : {accel::Activation::None, accel::Activation::Relu, accel::Activation::Gelu}) {
    // MatMul + activation + residual.
    std::vector<float> fused(m * n), passes(m * n);
    accel::ExecuteMatMul(hip, Host(a, {m, k}), Host(b, {k, n}), fused.data(), act, &res_op);
    accel::ExecuteMatMul(generic, Host(a, {m, k}), Host(b, {k, n}), passes.data(), act, &res_op);
    ExpectSameBits(fused, passes, __LINE__);
    // FusedMatMul alpha.
    accel::FusedMatMulConfig fc;
    fc.alpha = 0.3f;
    accel::ExecuteFusedMatMul(hip, Host(a, {m, k}), Host(b, {k, n}), fc, act, fused.data());
    accel::ExecuteFusedMatMul(generic, Host(a, {m, k}), Host(b, {k, n}), fc, act, passes.data());
    ExpectSameBits(fused, passes, __LINE__);
    // Gemm alpha/beta with row, column and scalar biases.
    for (int shape = 0; shape < 3; ++shape) {
      accel::GemmConfig gc;
      gc.alpha = 0.7f;
      gc.beta = -1.25f;
      const std::vector<float>& bv = shape == 1 ? bias_col : bias_row;
      const accel::Operand bias_op =
          Host(bv, shape == 0 ? std::vector<int64_t>{n} : shape == 1 ? std::vector<int64_t>{m, 1} : std::vector<int64_t>{1});
      accel::ExecuteGemm(hip, Host(a, {m, k}), Host(b, {k, n}), &bias_op, gc, fused.data(), act);
      accel::ExecuteGemm(generic, Host(a, {m, k}), Host(b, {k, n}), &bias_op, gc, passes.data(), act);
      ExpectSameBits(fused, passes, __LINE__);
    }
  }
  // Quantized B with Relu and a residual.
  std::vector<int8_t> q(static_cast<size_t>(k * n));
  for (auto& v : q) {
    seed = seed * 1664525u + 1013904223u;
    v = static_cast<int8_t>(static_cast<int>(seed % 255u) - 127);
  }
  std::vector<float> scale(n);
  for (int64_t j = 0; j < n; ++j) scale[j] = 0.001f * static_cast<float>(1 + j % 9);
  accel::OwnedBuffer qb = UploadBytes(hip, q.data(), q.size());
  accel::OwnedBuffer sb = UploadBytes(hip, scale.data(), scale.size() * 4);
  accel::Operand bq;
  bq.quant = true;
  bq.shape = {k, n};
  bq.quant_plane.q = static_cast<const int8_t*>(qb.buffer.data);
  bq.quant_plane.scale = static_cast<const float*>(sb.buffer.data);
  bq.quant_plane.shape = {k, n};
  bq.quant_plane.axis = 1;
  for (const int64_t rows : {int64_t{1}, int64_t{4}, m}) {
    std::vector<float> fused(rows * n), passes(rows * n);
    const accel::Operand r = Host(res, {rows, n});
    accel::ExecuteMatMul(hip, Host(a, {rows, k}), bq, fused.data(), accel::Activation::Relu, &r);
    accel::ExecuteMatMul(generic, Host(a, {rows, k}), bq, passes.data(), accel::Activation::Relu, &r);
    ExpectSameBits(fused, passes, __LINE__);
  }
}

// ---- exact products: the reference's bits (:234-271, 325-405, 413-425) ---------------------

// ReferenceMatMul (src/sim_device.cc:387-402) restated: C from zero, k order, rounded products.
std::vector<float> HostReference(const std::vector<float>& a, const std::vector<float>& b, int64_t m, int64_t k,
                                 int64_t n) {
  std::vector<float> c(static_cast<size_t>(m * n), 0.f);
  for (int64_t i = 0; i < m; ++i)
    for (int64_t p = 0; p < k; ++p) {
      const float x = a[i * k + p];
      for (int64_t j = 0; j < n; ++j) {
        const float prod = x * b[p * n + j];
        c[i * n + j] = c[i * n + j] + prod;
      }
    }
  return c;
}

void TestExactProducts(accel::Device& dev) {
  accel::HipSetExactProducts(true);
  EXPECT(accel::HipExactProducts());
  // The split-product KAT.
  const float ah[2] = {FromBits(0xBE2694CDu), FromBits(0x3E41AF7Du)};
  const float bh[2] = {FromBits(0x3F800000u), FromBits(0x3F5C2CB8u)};
  accel::OwnedBuffer ka = accel::Upload(dev, ah, {1, 2});
  accel::OwnedBuffer kb = accel::Upload(dev, bh, {2, 1});
  accel::DeviceBuffer kc = dev.Allocate(sizeof(float));
  dev.MatMul(ka.buffer, kb.buffer, kc, 1, 2, 1);
  float got = 0.f;
  dev.CopyDeviceToHost(&got, kc, sizeof(got));
  dev.Free(kc);
  EXPECT(Bits(got) == 0xB5200000u);

  // The LCG products, memcmp against the reference loop (GEMV and GEMM shapes).
  for (const auto& [m, k, n, seed0] : std::vector<std::tuple<int64_t, int64_t, int64_t, uint32_t>>{
           {128, 160, 96, 1}, {13, 19, 17, 2}, {1, 576, 1536, 5}, {4, 1536, 576, 6}, {70, 333, 129, 7}}) {
    uint32_t seed = seed0;
    std::vector<float> a, b;
    FillLcg(&a, m * k, &seed);
    FillLcg(&b, k * n, &seed);
    std::vector<float> out(static_cast<size_t>(m * n), 1.f);
    accel::ExecuteMatMul(dev, Host(a, {m, k}), Host(b, {k, n}), out.data());
    ExpectSameBits(out, HostReference(a, b, m, k, n), __LINE__);
  }

  // The quantized panel: per-row scale and zero, then a whole-tensor scale (:325-405), and
  // per-column scales at decode shapes with Relu and a residual.
  constexpr int64_t m = 8, k = 160, n = 300;
  uint32_t seed = 3;
  std::vector<float> a;
  FillLcg(&a, m * k, &seed);
  std::vector<int8_t> q(static_cast<size_t>(k * n));
  std::vector<float> scale(k);
  std::vector<int8_t> zero(k);
  for (auto& v : q) {
    seed = seed * 1664525u + 1013904223u;
    v = static_cast<int8_t>(static_cast<int>(seed % 251u) - 125);
  }
  for (int64_t r = 0; r < k; ++r) {
    scale[r] = static_cast<float>(r % 5) * 0.25f + 0.5f;
    zero[r] = static_cast<int8_t>(r % 7 - 3);
  }
  std::vector<float> w(static_cast<size_t>(k * n)), w_half(static_cast<size_t>(k * n));
  for (int64_t i = 0; i < k * n; ++i) {
    w[i] = (static_cast<float>(q[i]) - static_cast<float>(zero[i / n])) * scale[i / n];
    w_half[i] = static_cast<float>(q[i]) * 0.5f;
  }
  accel::OwnedBuffer qb = UploadBytes(dev, q.data(), q.size());
  accel::OwnedBuffer sb = UploadBytes(dev, scale.data(), scale.size() * 4);
  accel::OwnedBuffer zb = UploadBytes(dev, zero.data(), zero.size());
  accel::Operand bq;
  bq.quant = true;
  bq.shape = {k, n};
  bq.quant_plane.q = static_cast<const int8_t*>(qb.buffer.data);
  bq.quant_plane.scale = static_cast<const float*>(sb.buffer.data);
  bq.quant_plane.zero = static_cast<const int8_t*>(zb.buffer.data);
  bq.quant_plane.shape = {k, n};
  bq.quant_plane.axis = 0;
  std::vector<float> out(static_cast<size_t>(m * n), 1.f);
  accel::ExecuteMatMul(dev, Host(a, {m, k}), bq, out.data());
  ExpectSameBits(out, HostReference(a, w, m, k, n), __LINE__);
  const float half = 0.5f;
  accel::OwnedBuffer hb = UploadBytes(dev, &half, sizeof(half));
  bq.quant_plane.scale = static_cast<const float*>(hb.buffer.data);
  bq.quant_plane.zero = nullptr;
  bq.quant_plane.axis = -1;
  accel::ExecuteMatMul(dev, Host(a, {m, k}), bq, out.data());
  ExpectSameBits(out, HostReference(a, w_half, m, k, n), __LINE__);

  std::vector<float> col_scale(n);
  for (int64_t j = 0; j < n; ++j) col_scale[j] = 0.001f * static_cast<float>(1 + j % 13);
  accel::OwnedBuffer cb = UploadBytes(dev, col_scale.data(), col_scale.size() * 4);
  bq.quant_plane.scale = static_cast<const float*>(cb.buffer.data);
  bq.quant_plane.axis = 1;
  std::vector<float> w_col(static_cast<size_t>(k * n));
  for (int64_t i = 0; i < k * n; ++i) w_col[i] = static_cast<float>(q[i]) * col_scale[i % n];
  std::vector<float> res;
  FillLcg(&res, m * n, &seed);
  for (const int64_t rows : {int64_t{1}, int64_t{4}, m}) {
    const accel::Operand r = Host(res, {rows, n});
    std::vector<float> got_rows(static_cast<size_t>(rows * n));
    accel::ExecuteMatMul(dev, Host(a, {rows, k}), bq, got_rows.data(), accel::Activation::Relu, &r);
    std::vector<float> want = HostReference(a, w_col, rows, k, n);
    for (size_t i = 0; i < want.size(); ++i) {
      float v = want[i];
      if (v < 0.f) v = 0.f;
      want[i] = v + res[i];
    }
    ExpectSameBits(got_rows, want, __LINE__);
  }
  accel::HipSetExactProducts(false);
  EXPECT(!accel::HipExactProducts());
}

}  // namespace

int main() {
  auto device = accel::CreateHipDevice();
  accel::Device& dev = *device;
  std::printf("device %s\n", dev.Name());
  const struct {
    const char* name;
    void (*fn)(accel::Device&);
  } tests[] = {
      {"hand values", TestHandValues},
      {"counters and residency", TestCountersAndResidency},
      {"rejections", TestRejections},
      {"probes and products", TestProbesAndProducts},
      {"quantized operand", TestQuantized},
      {"non-finite bits", TestNonFiniteBits},
      {"buffers and tables", TestBuffersAndTables},
      {"recorded sequence", TestRecordedSequence},
      {"fused equals passes", TestFusedEqualsPasses},
      {"exact products", TestExactProducts},
  };
  for (const auto& t : tests) {
    const int before = g_failures;
    try {
      t.fn(dev);
    } catch (const std::exception& e) {
      std::fprintf(stderr, "FAIL %s: threw %s\n", t.name, e.what());
      ++g_failures;
    }
    std::printf("%-24s %s\n", t.name, g_failures == before ? "ok" : "FAILED");
    std::fflush(stdout);
  }
  const int64_t live = accel::LiveDeviceAllocs();
  std::printf("%d checks, %d failed, %lld live allocations at exit\n", g_checks, g_failures,
              static_cast<long long>(live));
  return g_failures == 0 ? 0 : 1;
}
