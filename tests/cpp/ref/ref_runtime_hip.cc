// AccelEP's own runtime (src/runtime.cc, src/device_buffer.cc, compiled from the reference
// tree against its own include/) driving the MI355X device (accelep_amd/host/hip_device.cc over
// libaccel_hip.so): the drop-in the plugin makes when its constructor calls CreateHipDevice().
// Built by oracle/Makefile (`make -C oracle dropin`) into oracle/_ref/ref_runtime_hip; run by
// tests/test_gpu_dropin.py. TEST INFRASTRUCTURE ONLY: no product code links the reference.
//
// The operands are built the way the plugin builds them: a constant int8 weight uploaded as-is
// and handed over as a QuantPlane of device pointers (BindConstant, src/ep.cc:1430-1463), a
// constant float weight as an on-device OwnedBuffer, runtime inputs as host pointers. The step
// sequences are RunKernel's (src/ep.cc:1602-1650): plain, has_rms (ExecuteMatMul retaining the
// pre-norm sum, RmsNorm into the next input) and has_skip (ExecuteMatMul, then ResidualAdd of
// the held sum and NoteAddEpilogue), and a leading-dynamic MatMul's runtime batch (src/ep.cc:
// 418-486,1546-1593) with float and int8 weights, batched B and FusedMatMul's transposes. Every
// input is small integers or halves, so every product and sum is exact in fp32 and the expected
// values are exact; the one full-size product (the decode GEMV shape) is checked against
// Higham's gamma_K bound.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
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

void ExpectExact(const std::vector<float>& got, const std::vector<float>& want, int line) {
  bool ok = got.size() == want.size();
  for (size_t i = 0; ok && i < got.size(); ++i) {
    if (std::memcmp(&got[i], &want[i], sizeof(float)) != 0) {
      std::fprintf(stderr, "  index %zu: got %.9g want %.9g\n", i, got[i], want[i]);
      ok = false;
    }
  }
  Expect(ok, "values are exact", line);
}
#define EXPECT_EXACT(got, want) ExpectExact(got, want, __LINE__)

// Uploads host data into a new device buffer (counted, like the plugin's Compile upload).
accel::OwnedBuffer Upload(accel::Device& device, const void* data, size_t bytes, std::vector<int64_t> shape) {
  accel::OwnedBuffer out;
  out.device = &device;
  out.shape = std::move(shape);
  out.buffer = device.Allocate(bytes);
  device.CopyHostToDevice(out.buffer, data, bytes);
  return out;
}

std::vector<float> Download(accel::Device& device, const accel::OwnedBuffer& b) {
  std::vector<float> out(static_cast<size_t>(accel::ElementCount(b.shape)));
  if (!out.empty()) device.CopyDeviceToHost(out.data(), b.buffer, out.size() * sizeof(float));
  return out;
}

// Row-major [m, n] = [m, k] @ [k, n] in double (exact for the small-integer inputs used here).
std::vector<float> HostMatMul(const std::vector<float>& a, const std::vector<float>& b, int64_t m, int64_t k, int64_t n) {
  std::vector<float> c(static_cast<size_t>(m * n));
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double s = 0;
      for (int64_t p = 0; p < k; ++p) s += double(a[i * k + p]) * double(b[p * n + j]);
      c[i * n + j] = static_cast<float>(s);
    }
  return c;
}

accel::Operand Host(const std::vector<float>& v, std::vector<int64_t> shape) {
  accel::Operand op;
  op.host = v.data();
  op.shape = std::move(shape);
  return op;
}

accel::Operand OnDevice(const accel::OwnedBuffer& b) {
  accel::Operand op;
  op.on_device = &b;
  op.shape = b.shape;
  return op;
}

// tests/test_ep.py:336-370: DequantizeLinear(W8 [[-128,127],[1,-2]], S [0.5,2], Z [1,-3],
// axis 0) -> MatMul(X [[1,2],[0,-1]]): Y[0,0] = -48.5 exactly; one matmul op, one kernel
// matmul, 16 bytes in and 16 bytes out per run; the constant touch names the int8 buffer.
void TestDequantizeKat(accel::Device& device) {
  const int8_t w8[4] = {-128, 127, 1, -2};
  const float scale[2] = {0.5f, 2.0f};
  const int8_t zero[2] = {1, -3};
  accel::OwnedBuffer q = Upload(device, w8, sizeof(w8), {2, 2});
  accel::OwnedBuffer s = Upload(device, scale, sizeof(scale), {2});
  accel::OwnedBuffer z = Upload(device, zero, sizeof(zero), {2});
  accel::ResetAcceleratorStats();
  accel::ClearConstantTouches();
  // BindConstant's operand for the packed weight.
  accel::NoteConstantTouch(q.buffer.id, q.buffer.data, q.buffer.bytes);
  accel::Operand b;
  b.quant = true;
  b.shape = {2, 2};
  b.quant_plane.q = static_cast<const int8_t*>(q.buffer.data);
  b.quant_plane.scale = static_cast<const float*>(s.buffer.data);
  b.quant_plane.zero = static_cast<const int8_t*>(z.buffer.data);
  b.quant_plane.shape = {2, 2};
  b.quant_plane.axis = 0;
  b.quant_plane.offset = 0;
  const std::vector<float> x = {1, 2, 0, -1};
  std::vector<float> y(4, 7.f);
  accel::ExecuteMatMul(device, Host(x, {2, 2}), b, y.data());
  EXPECT_EXACT(y, (std::vector<float>{-48.5f, 67.f, -8.f, -2.f}));
  const accel::AcceleratorStats st = accel::GetAcceleratorStats();
  EXPECT(st.matmul_ops == 1);
  EXPECT(st.kernel_matmuls == 1);
  EXPECT(st.gemm_ops == 0);
  EXPECT(st.bytes_to_device == 16);
  EXPECT(st.bytes_to_host == 16);
  EXPECT(st.relu_epilogues == 0 && st.gelu_epilogues == 0 && st.add_epilogues == 0);
  EXPECT(accel::ConstantTouchCount() == 1);
  EXPECT(accel::ConstantTouchId(0) == q.buffer.id);
  EXPECT(accel::ConstantTouchBytes(0) == 4);
  // The packed weight cannot be transposed (src/runtime.cc:273-275).
  accel::FusedMatMulConfig trans;
  trans.trans_b = true;
  bool threw = false;
  try {
    accel::ExecuteFusedMatMul(device, Host(x, {2, 2}), b, trans, accel::Activation::None, y.data());
  } catch (const std::invalid_argument& e) {
    threw = std::string(e.what()).find("transpose") != std::string::npos;
  }
  EXPECT(threw);
}

// RunKernel's three step kinds over one chain: X[3,4] @ W1[4,5] + R (residual epilogue,
// retained as the pre-norm sum) -> RmsNorm -> @ W2[5,5] (retained) -> + held sum
// (ResidualAdd) -> host. A non-symmetric residual pins its orientation.
void TestStepSequences(accel::Device& device) {
  const int64_t rows = 3, k = 4, n = 5;
  std::vector<float> x(rows * k), w1(k * n), w2(n * n), r(rows * n), gamma(n);
  for (int64_t i = 0; i < rows * k; ++i) x[i] = static_cast<float>((i * 7) % 5 - 2);
  for (int64_t i = 0; i < k * n; ++i) w1[i] = static_cast<float>((i * 3) % 7 - 3) * 0.5f;
  for (int64_t i = 0; i < n * n; ++i) w2[i] = static_cast<float>((i * 5) % 9 - 4);
  for (int64_t i = 0; i < rows * n; ++i) r[i] = static_cast<float>(i * 10 + (i % n));
  for (int64_t i = 0; i < n; ++i) gamma[i] = 1.0f + 0.25f * static_cast<float>(i);
  accel::OwnedBuffer w1d = Upload(device, w1.data(), w1.size() * 4, {k, n});
  accel::OwnedBuffer w2d = Upload(device, w2.data(), w2.size() * 4, {n, n});
  accel::OwnedBuffer gd = Upload(device, gamma.data(), gamma.size() * 4, {n});
  const int64_t live = accel::LiveDeviceAllocs();
  accel::ResetAcceleratorStats();

  // has_rms step: keep the pre-norm sum on the device, the normed rows become the next input.
  accel::OwnedBuffer skip_hold;
  const accel::Operand residual = Host(r, {rows, n});
  accel::ExecuteMatMul(device, Host(x, {rows, k}), OnDevice(w1d), nullptr, accel::Activation::None, &residual,
                       &skip_hold);
  EXPECT(skip_hold.shape == (std::vector<int64_t>{rows, n}));
  std::vector<float> sum = HostMatMul(x, w1, rows, k, n);
  for (int64_t i = 0; i < rows * n; ++i) sum[i] += r[i];
  EXPECT_EXACT(Download(device, skip_hold), sum);
  accel::OwnedBuffer normed;
  normed.device = &device;
  normed.shape = skip_hold.shape;
  normed.buffer = device.Allocate(static_cast<size_t>(rows * n) * sizeof(float));
  device.RmsNorm(skip_hold.buffer, gd.buffer, normed.buffer, rows, n, 1e-5f, 0);
  // SimRmsNorm (src/sim_rmsnorm.cc:7-20): exact double sums for these integers.
  std::vector<float> want_norm(rows * n);
  for (int64_t i = 0; i < rows; ++i) {
    double ss = 0;
    for (int64_t j = 0; j < n; ++j) ss += double(sum[i * n + j]) * double(sum[i * n + j]);
    const double inv = 1.0 / std::sqrt(ss / double(n) + double(1e-5f));
    for (int64_t j = 0; j < n; ++j)
      want_norm[i * n + j] = static_cast<float>(double(sum[i * n + j]) * inv) * gamma[j];
  }
  EXPECT_EXACT(Download(device, normed), want_norm);

  // has_skip step: the chain tail, then the closing residual of the held sum.
  accel::OwnedBuffer produced;
  accel::ExecuteMatMul(device, OnDevice(normed), OnDevice(w2d), nullptr, accel::Activation::None, nullptr, &produced);
  device.ResidualAdd(produced.buffer, skip_hold.buffer, rows * n);
  accel::NoteAddEpilogue();
  std::vector<float> out(rows * n);
  device.CopyDeviceToHost(out.data(), produced.buffer, out.size() * sizeof(float));
  // The tail product of the normed rows is not exact in fp32: out = fl(fl(sum_p normed*w2) +
  // held sum) lies within gamma_n (|normed| @ |w2|) + one rounding of |out| of the exact value.
  const double u = std::ldexp(1.0, -24), gn = n * u / (1 - n * u);
  bool close = true;
  for (int64_t i = 0; i < rows; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double exact = double(sum[i * n + j]), mag = 0;
      for (int64_t p = 0; p < n; ++p) {
        exact += double(want_norm[i * n + p]) * double(w2[p * n + j]);
        mag += std::fabs(double(want_norm[i * n + p]) * double(w2[p * n + j]));
      }
      const double got = double(out[i * n + j]);
      if (!(std::fabs(got - exact) <= 2 * gn * mag + 2 * u * std::fabs(got) + 1e-30)) close = false;
    }
  EXPECT(close);
  const accel::AcceleratorStats st = accel::GetAcceleratorStats();
  EXPECT(st.matmul_ops == 2);
  EXPECT(st.kernel_matmuls == 2);
  EXPECT(st.add_epilogues == 2);  // the residual epilogue and the closing add
  EXPECT(st.bytes_to_device == static_cast<int64_t>((x.size() + r.size()) * 4));
  // Counted copies back: the two checks of the held sum and the normed rows, and the result.
  EXPECT(st.bytes_to_host == static_cast<int64_t>(3 * out.size() * 4));
  skip_hold = accel::OwnedBuffer();
  normed = accel::OwnedBuffer();
  produced = accel::OwnedBuffer();
  EXPECT(accel::LiveDeviceAllocs() == live);
}

// ExecuteGemm (src/runtime.cc:653-723) with runtime operands, both transposed (two device
// transposes per run), alpha, beta, a row bias and Relu; ExecuteFusedMatMul with trans_b.
void TestGemmAndFused(accel::Device& device) {
  const int64_t m = 3, k = 4, n = 2;
  std::vector<float> at(k * m), bt(n * k), bias = {1.5f, -40.f};
  for (int64_t i = 0; i < k * m; ++i) at[i] = static_cast<float>(i % 5 - 1);
  for (int64_t i = 0; i < n * k; ++i) bt[i] = static_cast<float>((i * 3) % 4 - 1);
  accel::ResetAcceleratorStats();
  accel::GemmConfig cfg;
  cfg.trans_a = true;
  cfg.trans_b = true;
  cfg.alpha = 2.f;
  cfg.beta = 0.5f;
  const accel::Operand bias_op = Host(bias, {n});
  std::vector<float> y(m * n, 9.f);
  accel::ExecuteGemm(device, Host(at, {k, m}), Host(bt, {n, k}), &bias_op, cfg, y.data(), accel::Activation::Relu);
  std::vector<float> want(m * n);
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float acc = 0;
      for (int64_t p = 0; p < k; ++p) acc += at[p * m + i] * bt[j * k + p];
      float v = 2.f * acc + 0.5f * bias[j];
      want[i * n + j] = v < 0 ? 0.f : v;
    }
  EXPECT_EXACT(y, want);
  accel::AcceleratorStats st = accel::GetAcceleratorStats();
  EXPECT(st.gemm_ops == 1 && st.relu_epilogues == 1 && st.device_transposes == 2 && st.kernel_matmuls == 1);

  accel::FusedMatMulConfig fcfg;
  fcfg.trans_b = true;
  fcfg.alpha = -0.5f;
  std::vector<float> a(m * k);
  for (int64_t i = 0; i < m * k; ++i) a[i] = static_cast<float>(i % 3);
  std::vector<float> yf(m * n);
  accel::ExecuteFusedMatMul(device, Host(a, {m, k}), Host(bt, {n, k}), fcfg, accel::Activation::None, yf.data());
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float acc = 0;
      for (int64_t p = 0; p < k; ++p) acc += a[i * k + p] * bt[j * k + p];
      want[i * n + j] = -0.5f * acc;
    }
  EXPECT_EXACT(yf, want);
}

// The decode GEMV shape through the reference runtime: X[1,4096] @ int8 W[4096,14336] with a
// per-column scale (a constant QuantPlane), within 2 gamma_K (|X| @ |W|) of the exact product.
void TestDecodeGemvShape(accel::Device& device) {
  const int64_t k = 4096, n = 14336;
  std::vector<int8_t> q(static_cast<size_t>(k * n));
  std::vector<float> scale(n), x(k);
  uint32_t s = 12345;
  auto next = [&s] {
    s = s * 1664525u + 1013904223u;
    return s;
  };
  for (auto& v : q) v = static_cast<int8_t>(static_cast<int>(next() % 255) - 127);
  for (auto& v : scale) v = 1e-3f + 9e-3f * static_cast<float>(next() % 1000) / 1000.f;
  for (auto& v : x) v = static_cast<float>(static_cast<int>(next() % 2001) - 1000) / 500.f;
  accel::OwnedBuffer qd = Upload(device, q.data(), q.size(), {k, n});
  accel::OwnedBuffer sd = Upload(device, scale.data(), scale.size() * 4, {n});
  accel::Operand b;
  b.quant = true;
  b.shape = {k, n};
  b.quant_plane.q = static_cast<const int8_t*>(qd.buffer.data);
  b.quant_plane.scale = static_cast<const float*>(sd.buffer.data);
  b.quant_plane.shape = {k, n};
  b.quant_plane.axis = 1;
  std::vector<float> y(n);
  for (int rep = 0; rep < 2; ++rep) {  // the second call reads the staged copy
    accel::ExecuteMatMul(device, Host(x, {1, k}), b, y.data());
    const double gk = k * std::ldexp(1.0, -24) / (1 - k * std::ldexp(1.0, -24));
    bool ok = true;
    for (int64_t j = 0; j < n && ok; ++j) {
      double exact = 0, mag = 0;
      for (int64_t p = 0; p < k; ++p) {
        const double w = double(static_cast<float>(q[p * n + j]) * scale[j]);
        exact += double(x[p]) * w;
        mag += std::fabs(double(x[p]) * w);
      }
      if (!(std::fabs(double(y[j]) - exact) <= 2 * gk * mag + 1e-30)) {
        std::fprintf(stderr, "  column %lld: got %.9g exact %.9g\n", static_cast<long long>(j), y[j], exact);
        ok = false;
      }
    }
    EXPECT(ok);
  }
}

// A leading-dynamic MatMul (src/ep.cc:418-486): RunKernel checks the runtime shapes against the
// compiled contract (:1546-1593) and hands the runtime batch to ExecuteMatMul as the leading
// dimension of A. The same constant weight serves three batch sizes, as an on-device float
// weight and as an int8 plane with power-of-two column scales; then a batched B (one matrix per
// batch) and FusedMatMul's trans_a / trans_b / alpha on batched operands. Small integers and
// halves keep every product and sum exact.
void TestLeadingBatchAndTrans(accel::Device& device) {
  const int64_t k = 48, n = 20, rows = 5;
  std::vector<float> wf(static_cast<size_t>(k * n));
  std::vector<int8_t> w8(static_cast<size_t>(k * n));
  std::vector<float> scale(static_cast<size_t>(n));
  for (int64_t i = 0; i < k * n; ++i) {
    wf[i] = static_cast<float>((i * 7 + 3) % 7 - 3);
    w8[i] = static_cast<int8_t>((i * 5 + 1) % 17 - 8);
  }
  for (int64_t j = 0; j < n; ++j) scale[j] = (j % 2 == 0) ? 0.5f : 0.25f;
  std::vector<float> wq(static_cast<size_t>(k * n));
  for (int64_t i = 0; i < k * n; ++i) wq[i] = static_cast<float>(w8[i]) * scale[i % n];
  accel::OwnedBuffer wd = Upload(device, wf.data(), wf.size() * sizeof(float), {k, n});
  accel::OwnedBuffer q = Upload(device, w8.data(), w8.size(), {k, n});
  accel::OwnedBuffer s = Upload(device, scale.data(), scale.size() * sizeof(float), {n});
  accel::Operand bq;
  bq.quant = true;
  bq.shape = {k, n};
  bq.quant_plane.q = static_cast<const int8_t*>(q.buffer.data);
  bq.quant_plane.scale = static_cast<const float*>(s.buffer.data);
  bq.quant_plane.shape = {k, n};
  bq.quant_plane.axis = 1;
  for (const int64_t batch : {3, 1, 2}) {
    std::vector<float> a(static_cast<size_t>(batch * rows * k));
    for (size_t i = 0; i < a.size(); ++i) a[i] = 0.5f * static_cast<float>(static_cast<int64_t>(i * 11 + batch) % 9 - 4);
    std::vector<float> y(static_cast<size_t>(batch * rows * n), 7.f);
    accel::ExecuteMatMul(device, Host(a, {batch, rows, k}), OnDevice(wd), y.data());
    EXPECT_EXACT(y, HostMatMul(a, wf, batch * rows, k, n));
    std::fill(y.begin(), y.end(), 7.f);
    accel::ExecuteMatMul(device, Host(a, {batch, rows, k}), bq, y.data());
    EXPECT_EXACT(y, HostMatMul(a, wq, batch * rows, k, n));
  }
  // Batched B: [2, 4, 16] @ [2, 16, 8], one matrix per batch.
  {
    const int64_t bb = 2, m = 4, kk = 16, nn = 8;
    std::vector<float> a(static_cast<size_t>(bb * m * kk)), b(static_cast<size_t>(bb * kk * nn));
    for (size_t i = 0; i < a.size(); ++i) a[i] = static_cast<float>(static_cast<int64_t>(i * 3) % 7 - 3);
    for (size_t i = 0; i < b.size(); ++i) b[i] = static_cast<float>(static_cast<int64_t>(i * 5) % 9 - 4);
    std::vector<float> y(static_cast<size_t>(bb * m * nn), 7.f), want;
    accel::ExecuteMatMul(device, Host(a, {bb, m, kk}), Host(b, {bb, kk, nn}), y.data());
    for (int64_t t = 0; t < bb; ++t) {
      const std::vector<float> at(a.begin() + t * m * kk, a.begin() + (t + 1) * m * kk);
      const std::vector<float> bt(b.begin() + t * kk * nn, b.begin() + (t + 1) * kk * nn);
      const std::vector<float> c = HostMatMul(at, bt, m, kk, nn);
      want.insert(want.end(), c.begin(), c.end());
    }
    EXPECT_EXACT(y, want);
  }
  // FusedMatMul, batched A stored [2, k, m] with trans_a, B stored [n, k] with trans_b,
  // alpha 0.5: Y[t] = 0.5 * A[t]^T @ B^T.
  {
    const int64_t bb = 2, m = 6, kk = 12, nn = 10;
    std::vector<float> a(static_cast<size_t>(bb * kk * m)), b(static_cast<size_t>(nn * kk));
    for (size_t i = 0; i < a.size(); ++i) a[i] = static_cast<float>(static_cast<int64_t>(i * 7) % 11 - 5);
    for (size_t i = 0; i < b.size(); ++i) b[i] = static_cast<float>(static_cast<int64_t>(i * 3) % 5 - 2);
    accel::FusedMatMulConfig cfg;
    cfg.trans_a = true;
    cfg.trans_b = true;
    cfg.alpha = 0.5f;
    std::vector<float> y(static_cast<size_t>(bb * m * nn), 7.f), want;
    accel::ExecuteFusedMatMul(device, Host(a, {bb, kk, m}), Host(b, {nn, kk}), cfg, accel::Activation::None, y.data());
    std::vector<float> bt(static_cast<size_t>(kk * nn));
    for (int64_t r = 0; r < nn; ++r)
      for (int64_t c = 0; c < kk; ++c) bt[c * nn + r] = b[r * kk + c];
    for (int64_t t = 0; t < bb; ++t) {
      std::vector<float> at(static_cast<size_t>(m * kk));
      for (int64_t r = 0; r < kk; ++r)
        for (int64_t c = 0; c < m; ++c) at[c * kk + r] = a[t * kk * m + r * m + c];
      std::vector<float> c = HostMatMul(at, bt, m, kk, nn);
      for (float& v : c) v *= 0.5f;
      want.insert(want.end(), c.begin(), c.end());
    }
    EXPECT_EXACT(y, want);
  }
}

}  // namespace

int main() {
  try {
    std::unique_ptr<accel::Device> device = accel::CreateHipDevice();
    const int64_t live = accel::LiveDeviceAllocs();
    TestDequantizeKat(*device);
    TestStepSequences(*device);
    TestGemmAndFused(*device);
    TestDecodeGemvShape(*device);
    TestLeadingBatchAndTrans(*device);
    EXPECT(accel::LiveDeviceAllocs() == live);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "FAIL: exception %s\n", e.what());
    return 2;
  }
  std::printf("%d checks, %d failures (reference runtime.cc over the HIP device)\n", g_checks, g_failures);
  return g_failures == 0 ? 0 : 1;
}
