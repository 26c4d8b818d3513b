// AccelEP's own device-call recorder (tests/recording_device.cc, compiled from the reference
// tree) wrapped around the reference's SimDevice records whole call sequences: the runtime's
// Execute* steps (src/runtime.cc) and a small Llama generation through the reference's own
// llama_model.cc (compiled with its CreateSimDevice() call pointed at the recorder). Every
// recorded call is then replayed, one by one, on the MI355X device (CreateHipDevice(), exact
// products on), and each call's output is compared with the FNV-1a hash the recorder took on
// SimDevice. Built by oracle/Makefile (`make -C oracle dropin`) into
// oracle/_ref/ref_trace_replay_hip; run by tests/test_gpu_trace_replay.py. TEST INFRASTRUCTURE
// ONLY: no product code links the reference.
//
// Bit for bit: MatMul (exact-products mode), Transpose, GemmEpilogue without Gelu, Embedding,
// Rope, AppendCache, ResidualAdd and SampleToken. Within a stated tolerance, for the calls whose
// arithmetic goes through erf, exp or a double sum in another order (the device's erff / expf
// against glibc's, a fixed tree of double adds against a sequential one): GemmEpilogue with Gelu
// (rtol 1e-6, atol 2e-7), SiluMul (rtol 1e-6), Attention (rtol 1e-5, atol 2e-6) and RmsNorm
// (rtol 2e-7, atol 1e-7). After such a call the replay writes the recorded output into the
// device buffer, so every later call starts from the recorded inputs and is checked alone.
//
// The recorder keeps its host-to-device payloads private; a tape device between the recorder
// and SimDevice keeps them (and each call's output bytes) for the replay.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "accel/device.h"
#include "accel/hip_device.h"
#include "accel/runtime.h"
#include "accel/sim_api.h"
#include "recording_device.h"

namespace accel {
std::unique_ptr<Device> CreateTracedDevice();
}

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

using Bytes = std::vector<unsigned char>;

Bytes Read(accel::Device& device, accel::DeviceBuffer buffer) {
  Bytes out(buffer.bytes);
  if (!out.empty()) device.CopyDeviceToHost(out.data(), buffer, out.size());
  return out;
}

// Forwards every call to `inner` and keeps the payload of every host-to-device copy and the
// output of every compute call, in call order.
class TapeDevice final : public accel::Device {
 public:
  explicit TapeDevice(accel::Device& inner) : inner_(inner) {}
  std::vector<Bytes> uploads;
  std::vector<Bytes> outputs;

  const char* Name() const override { return inner_.Name(); }
  accel::DeviceBuffer Allocate(size_t bytes) override { return inner_.Allocate(bytes); }
  void Free(accel::DeviceBuffer buffer) override { inner_.Free(buffer); }
  void CopyHostToDevice(accel::DeviceBuffer dst, const void* src, size_t bytes) override {
    const auto* p = static_cast<const unsigned char*>(src);
    uploads.emplace_back(p, p + (src == nullptr ? 0 : bytes));
    inner_.CopyHostToDevice(dst, src, bytes);
  }
  void CopyDeviceToHost(void* dst, accel::DeviceBuffer src, size_t bytes) override {
    inner_.CopyDeviceToHost(dst, src, bytes);
  }
  void MatMul(accel::DeviceBuffer a, accel::DeviceBuffer b, accel::DeviceBuffer c, int64_t m, int64_t k,
              int64_t n) override {
    inner_.MatMul(a, b, c, m, k, n);
    Keep(c);
  }
  void Transpose(accel::DeviceBuffer src, accel::DeviceBuffer dst, int64_t rows, int64_t cols) override {
    inner_.Transpose(src, dst, rows, cols);
    Keep(dst);
  }
  void GemmEpilogue(accel::DeviceBuffer c, int64_t m, int64_t n, float alpha, const accel::DeviceBuffer* bias,
                    const std::vector<int64_t>& bias_shape, float beta, accel::Activation activation) override {
    inner_.GemmEpilogue(c, m, n, alpha, bias, bias_shape, beta, activation);
    Keep(c);
  }
  void Embedding(accel::DeviceBuffer ids, int64_t id_offset, accel::DeviceBuffer table, accel::DeviceBuffer out,
                 int64_t seq, int64_t hidden, int64_t vocab) override {
    inner_.Embedding(ids, id_offset, table, out, seq, hidden, vocab);
    Keep(out);
  }
  void RmsNorm(accel::DeviceBuffer x, accel::DeviceBuffer weight, accel::DeviceBuffer y, int64_t rows, int64_t dim,
               float eps, int64_t row_offset) override {
    inner_.RmsNorm(x, weight, y, rows, dim, eps, row_offset);
    Keep(y);
  }
  void Rope(accel::DeviceBuffer states, accel::DeviceBuffer cos_table, accel::DeviceBuffer sin_table, int64_t seq,
            int64_t n_heads, int64_t head_dim, int64_t position) override {
    inner_.Rope(states, cos_table, sin_table, seq, n_heads, head_dim, position);
    Keep(states);
  }
  void AppendCache(accel::DeviceBuffer src, accel::DeviceBuffer cache, int64_t seq, int64_t position, int64_t n_heads,
                   int64_t head_dim) override {
    inner_.AppendCache(src, cache, seq, position, n_heads, head_dim);
    Keep(cache);
  }
  void Attention(accel::DeviceBuffer q, accel::DeviceBuffer k, accel::DeviceBuffer v, accel::DeviceBuffer scores,
                 accel::DeviceBuffer out, int64_t seq, int64_t position, int64_t heads, int64_t kv_heads,
                 int64_t head_dim) override {
    inner_.Attention(q, k, v, scores, out, seq, position, heads, kv_heads, head_dim);
    Keep(out);
  }
  void SiluMul(accel::DeviceBuffer gate, accel::DeviceBuffer up, int64_t count) override {
    inner_.SiluMul(gate, up, count);
    Keep(gate);
  }
  void ResidualAdd(accel::DeviceBuffer dest, accel::DeviceBuffer extra, int64_t count) override {
    inner_.ResidualAdd(dest, extra, count);
    Keep(dest);
  }
  void SampleToken(accel::DeviceBuffer logits, accel::DeviceBuffer chosen_ids, int64_t chosen_index, int64_t vocab,
                   float temperature, uint32_t* rng_state, int top_k) override {
    inner_.SampleToken(logits, chosen_ids, chosen_index, vocab, temperature, rng_state, top_k);
    Keep(chosen_ids);
  }

 private:
  void Keep(accel::DeviceBuffer buffer) { outputs.push_back(Read(inner_, buffer)); }
  accel::Device& inner_;
};

// SimDevice <- tape <- the reference's recorder, owned together and used as one device.
class TracedDevice final : public accel::Device {
 public:
  TracedDevice() : sim_(accel::CreateSimDevice()), tape_(*sim_), rec_(tape_) {}
  const accel::RecordingDevice& Recorder() const { return rec_; }
  const TapeDevice& Tape() const { return tape_; }

  const char* Name() const override { return rec_.Name(); }
  accel::DeviceBuffer Allocate(size_t bytes) override { return rec_.Allocate(bytes); }
  void Free(accel::DeviceBuffer buffer) override { rec_.Free(buffer); }
  void CopyHostToDevice(accel::DeviceBuffer dst, const void* src, size_t bytes) override {
    rec_.CopyHostToDevice(dst, src, bytes);
  }
  void CopyDeviceToHost(void* dst, accel::DeviceBuffer src, size_t bytes) override {
    rec_.CopyDeviceToHost(dst, src, bytes);
  }
  void MatMul(accel::DeviceBuffer a, accel::DeviceBuffer b, accel::DeviceBuffer c, int64_t m, int64_t k,
              int64_t n) override {
    rec_.MatMul(a, b, c, m, k, n);
  }
  void Transpose(accel::DeviceBuffer src, accel::DeviceBuffer dst, int64_t rows, int64_t cols) override {
    rec_.Transpose(src, dst, rows, cols);
  }
  void GemmEpilogue(accel::DeviceBuffer c, int64_t m, int64_t n, float alpha, const accel::DeviceBuffer* bias,
                    const std::vector<int64_t>& bias_shape, float beta, accel::Activation activation) override {
    rec_.GemmEpilogue(c, m, n, alpha, bias, bias_shape, beta, activation);
  }
  void Embedding(accel::DeviceBuffer ids, int64_t id_offset, accel::DeviceBuffer table, accel::DeviceBuffer out,
                 int64_t seq, int64_t hidden, int64_t vocab) override {
    rec_.Embedding(ids, id_offset, table, out, seq, hidden, vocab);
  }
  void RmsNorm(accel::DeviceBuffer x, accel::DeviceBuffer weight, accel::DeviceBuffer y, int64_t rows, int64_t dim,
               float eps, int64_t row_offset) override {
    rec_.RmsNorm(x, weight, y, rows, dim, eps, row_offset);
  }
  void Rope(accel::DeviceBuffer states, accel::DeviceBuffer cos_table, accel::DeviceBuffer sin_table, int64_t seq,
            int64_t n_heads, int64_t head_dim, int64_t position) override {
    rec_.Rope(states, cos_table, sin_table, seq, n_heads, head_dim, position);
  }
  void AppendCache(accel::DeviceBuffer src, accel::DeviceBuffer cache, int64_t seq, int64_t position, int64_t n_heads,
                   int64_t head_dim) override {
    rec_.AppendCache(src, cache, seq, position, n_heads, head_dim);
  }
  void Attention(accel::DeviceBuffer q, accel::DeviceBuffer k, accel::DeviceBuffer v, accel::DeviceBuffer scores,
                 accel::DeviceBuffer out, int64_t seq, int64_t position, int64_t heads, int64_t kv_heads,
                 int64_t head_dim) override {
    rec_.Attention(q, k, v, scores, out, seq, position, heads, kv_heads, head_dim);
  }
  void SiluMul(accel::DeviceBuffer gate, accel::DeviceBuffer up, int64_t count) override {
    rec_.SiluMul(gate, up, count);
  }
  void ResidualAdd(accel::DeviceBuffer dest, accel::DeviceBuffer extra, int64_t count) override {
    rec_.ResidualAdd(dest, extra, count);
  }
  void SampleToken(accel::DeviceBuffer logits, accel::DeviceBuffer chosen_ids, int64_t chosen_index, int64_t vocab,
                   float temperature, uint32_t* rng_state, int top_k) override {
    rec_.SampleToken(logits, chosen_ids, chosen_index, vocab, temperature, rng_state, top_k);
  }

 private:
  std::unique_ptr<accel::Device> sim_;
  TapeDevice tape_;
  accel::RecordingDevice rec_;
};

TracedDevice* g_traced = nullptr;  // the device the last CreateTracedDevice() made

// Replay tally per call name.
struct Tally {
  int calls = 0, exact = 0, within = 0, failed = 0;
  double worst = 0.0;  // largest |got - want| / (atol + rtol |want|) of the tolerance calls
};

struct Tolerance {
  double rtol, atol;
};

// The calls checked within a tolerance, and how (null: bit for bit).
const Tolerance* ToleranceFor(const accel::TraceOp& op) {
  static const Tolerance gelu{1e-6, 2e-7}, silu{1e-6, 1e-30}, attention{1e-5, 2e-6}, rms{2e-7, 1e-7};
  if (op.op == "GemmEpilogue" && op.activation == "gelu") return &gelu;
  if (op.op == "SiluMul") return &silu;
  if (op.op == "Attention") return &attention;
  if (op.op == "RmsNorm") return &rms;
  return nullptr;
}

// Worst |got - want| / (atol + rtol |want|) over the floats of two outputs; NaNs must agree as
// NaNs and infinities exactly. Returns +inf on a mismatch of that kind or of size.
double Ratio(const Bytes& got, const Bytes& want, const Tolerance& t) {
  if (got.size() != want.size() || got.size() % 4 != 0) return INFINITY;
  double worst = 0.0;
  for (size_t i = 0; i < got.size(); i += 4) {
    float g = 0.f, w = 0.f;
    std::memcpy(&g, &got[i], 4);
    std::memcpy(&w, &want[i], 4);
    if (std::isnan(g) || std::isnan(w)) {
      if (!(std::isnan(g) && std::isnan(w))) return INFINITY;
      continue;
    }
    if (std::isinf(g) || std::isinf(w)) {
      if (g != w) return INFINITY;
      continue;
    }
    const double r = std::fabs(double(g) - double(w)) / (t.atol + t.rtol * std::fabs(double(w)));
    if (r > worst) worst = r;
  }
  return worst;
}

accel::DeviceBuffer Place(const std::unordered_map<uint64_t, accel::DeviceBuffer>& allocs, const accel::SliceRef& ref) {
  auto it = allocs.find(ref.id);
  if (it == allocs.end()) throw std::runtime_error("trace names an allocation that is not live");
  auto* base = static_cast<unsigned char*>(it->second.data);
  return accel::DeviceBuffer{base + ref.byte_offset, static_cast<size_t>(ref.length), 0};
}

accel::Activation ActivationFrom(const std::string& name) {
  if (name == "relu") return accel::Activation::Relu;
  if (name == "gelu") return accel::Activation::Gelu;
  if (name == "none") return accel::Activation::None;
  throw std::runtime_error("unknown activation in trace: " + name);
}

// Replays the traced calls on `target`, checking every call's output against the recorder's
// hash (or, for the tolerance calls, against the recorded output bytes). Returns the tally.
std::map<std::string, Tally> Replay(const TracedDevice& traced, accel::Device& target, const char* label) {
  const std::vector<accel::TraceOp>& trace = traced.Recorder().Trace();
  const TapeDevice& tape = traced.Tape();
  std::map<std::string, Tally> tally;
  std::unordered_map<uint64_t, accel::DeviceBuffer> allocs;
  size_t upload = 0, output = 0;
  for (size_t index = 0; index < trace.size(); ++index) {
    const accel::TraceOp& op = trace[index];
    accel::DeviceBuffer out{};  // the call's output on the target
    uint64_t want = 0;          // its hash on SimDevice
    if (op.op == "Allocate") {
      allocs.emplace(op.id, target.Allocate(static_cast<size_t>(op.bytes)));
      continue;
    }
    if (op.op == "Free") {
      auto it = allocs.find(op.id);
      if (it == allocs.end()) throw std::runtime_error("trace frees an allocation that is not live");
      target.Free(it->second);
      allocs.erase(it);
      continue;
    }
    if (op.op == "CopyHostToDevice") {
      const Bytes& payload = tape.uploads.at(upload++);
      if (payload.size() != op.bytes) throw std::runtime_error("upload size differs from the trace");
      target.CopyHostToDevice(Place(allocs, op.dst), payload.empty() ? nullptr : payload.data(), payload.size());
      continue;
    }
    if (op.op == "CopyDeviceToHost") {
      Bytes tmp(static_cast<size_t>(op.bytes));
      target.CopyDeviceToHost(tmp.empty() ? nullptr : tmp.data(), Place(allocs, op.src), tmp.size());
      continue;
    }
    if (op.op == "MatMul") {
      out = Place(allocs, op.c);
      target.MatMul(Place(allocs, op.a), Place(allocs, op.b), out, op.m, op.k, op.n);
      want = op.c_hash;
    } else if (op.op == "Transpose") {
      out = Place(allocs, op.dst);
      target.Transpose(Place(allocs, op.src), out, op.rows, op.cols);
      want = op.dst_hash;
    } else if (op.op == "GemmEpilogue") {
      out = Place(allocs, op.c);
      accel::DeviceBuffer bias{};
      std::vector<int64_t> bias_shape;
      if (op.has_bias) {
        bias = Place(allocs, op.bias);
        bias_shape.push_back(static_cast<int64_t>(op.bias.length / sizeof(float)));  // 1-D, as recorded
      }
      target.GemmEpilogue(out, op.m, op.n, op.alpha, op.has_bias ? &bias : nullptr, bias_shape, op.beta,
                          ActivationFrom(op.activation));
      want = op.hash_after;
    } else if (op.op == "Embedding") {
      out = Place(allocs, op.c);
      target.Embedding(Place(allocs, op.a), op.rows, Place(allocs, op.b), out, op.m, op.k, op.n);
      want = op.c_hash;
    } else if (op.op == "RmsNorm") {
      out = Place(allocs, op.c);
      target.RmsNorm(Place(allocs, op.a), Place(allocs, op.b), out, op.rows, op.cols, op.alpha, op.m);
      want = op.c_hash;
    } else if (op.op == "Rope") {
      out = Place(allocs, op.a);
      target.Rope(out, Place(allocs, op.b), Place(allocs, op.c), op.m, op.k, op.n, op.rows);
      want = op.a_hash;
    } else if (op.op == "AppendCache") {
      out = Place(allocs, op.dst);
      target.AppendCache(Place(allocs, op.src), out, op.m, op.k, op.n, op.rows);
      want = op.dst_hash;
    } else if (op.op == "Attention") {
      out = Place(allocs, op.dst);
      target.Attention(Place(allocs, op.a), Place(allocs, op.b), Place(allocs, op.c), Place(allocs, op.src), out, op.m,
                       op.k, op.n, op.rows, op.cols);
      want = op.dst_hash;
    } else if (op.op == "SiluMul") {
      out = Place(allocs, op.a);
      target.SiluMul(out, Place(allocs, op.b), op.m);
      want = op.a_hash;
    } else if (op.op == "ResidualAdd") {
      out = Place(allocs, op.a);
      target.ResidualAdd(out, Place(allocs, op.b), op.m);
      want = op.a_hash;
    } else if (op.op == "SampleToken") {
      out = Place(allocs, op.dst);
      uint32_t rng = static_cast<uint32_t>(op.hash);
      target.SampleToken(Place(allocs, op.a), out, op.m, op.n, op.alpha, &rng, static_cast<int>(op.k));
      want = op.dst_hash;
    } else {
      throw std::runtime_error("unknown call in trace: " + op.op);
    }
    const Bytes& recorded = tape.outputs.at(output++);
    const Bytes got = Read(target, out);
    std::string name = op.op;
    if (op.op == "GemmEpilogue") name += "(" + op.activation + ")";
    Tally& t = tally[name];
    ++t.calls;
    if (accel::Fnv1a64(got.empty() ? nullptr : got.data(), got.size()) == want) {
      ++t.exact;
      continue;
    }
    const Tolerance* tol = ToleranceFor(op);
    const double r = tol == nullptr ? INFINITY : Ratio(got, recorded, *tol);
    if (r <= 1.0) {
      ++t.within;
      if (r > t.worst) t.worst = r;
      // Later calls start from the recorded values.
      target.CopyHostToDevice(out, recorded.data(), recorded.size());
    } else {
      ++t.failed;
      std::fprintf(stderr, "%s: call %zu (%s) differs on the HIP device (tolerance ratio %g)\n", label, index,
                   name.c_str(), r);
      target.CopyHostToDevice(out, recorded.data(), recorded.size());
    }
  }
  for (auto& [id, buffer] : allocs) target.Free(buffer);
  return tally;
}

void Report(const char* label, const std::map<std::string, Tally>& tally) {
  std::printf("%s\n", label);
  for (const auto& [name, t] : tally)
    std::printf("  %-22s calls %4d  bit-exact %4d  within tolerance %4d (worst %.3g)  failed %d\n", name.c_str(),
                t.calls, t.exact, t.within, t.worst, t.failed);
  for (const auto& [name, t] : tally) {
    EXPECT(t.failed == 0);
    // The calls without erf, exp or a reordered double sum must be bit for bit.
    const bool exact_only = name != "GemmEpilogue(gelu)" && name != "SiluMul" && name != "Attention" &&
                            name != "RmsNorm";
    if (exact_only) EXPECT(t.exact == t.calls);
  }
}

// Deterministic values: small integers times a power of two, or a N(0, s)-like spread from an LCG.
uint32_t g_lcg = 12345u;
float NextUnit() {
  g_lcg = g_lcg * 1664525u + 1013904223u;
  return static_cast<float>((g_lcg >> 8) & 0xffffff) / 16777216.0f;  // [0, 1)
}
std::vector<float> Spread(size_t count, float scale) {
  std::vector<float> v(count);
  for (float& x : v) x = (NextUnit() + NextUnit() + NextUnit() - 1.5f) * scale;
  return v;
}

// The runtime's steps on float operands (src/runtime.cc:254-416,653-723): MatMul with alpha and
// activations, Gemm with a bias and Gelu, FusedMatMul with both transposes and alpha, a leading
// batch, the residual epilogue, and RmsNorm / ResidualAdd as RunKernel issues them.
void TraceRuntimeSteps() {
  auto device = accel::CreateTracedDevice();
  TracedDevice* traced = g_traced;
  const int64_t m = 48, k = 96, n = 80;
  const std::vector<float> a = Spread(m * k, 1.f), b = Spread(k * n, 0.05f), bias = Spread(n, 0.1f);
  const std::vector<float> res = Spread(m * n, 1.f), gamma = Spread(n, 0.2f);
  std::vector<float> out(m * n), out2(m * n);
  // Gemm + bias + Gelu (a C2-shaped step, small)
  accel::GemmConfig gc;
  gc.alpha = 1.f;
  gc.beta = 1.f;
  const accel::Operand bias_op{bias.data(), nullptr, {n}};
  accel::ExecuteGemm(*device, {a.data(), nullptr, {m, k}}, {b.data(), nullptr, {k, n}}, &bias_op, gc, out.data(),
                     accel::Activation::Gelu);
  // MatMul + Relu, and MatMul + residual (the single-MatMul group the plugin fuses an Add into)
  accel::ExecuteMatMul(*device, {a.data(), nullptr, {m, k}}, {b.data(), nullptr, {k, n}}, out.data(),
                       accel::Activation::Relu);
  const accel::Operand res_op{res.data(), nullptr, {m, n}};
  accel::ExecuteMatMul(*device, {a.data(), nullptr, {m, k}}, {b.data(), nullptr, {k, n}}, out2.data(),
                       accel::Activation::None, &res_op);
  // FusedMatMul: transA, transB, alpha
  const std::vector<float> at = Spread(k * m, 1.f), bt = Spread(n * k, 0.05f);
  accel::FusedMatMulConfig fc;
  fc.trans_a = true;
  fc.trans_b = true;
  fc.alpha = 0.75f;
  accel::ExecuteFusedMatMul(*device, {at.data(), nullptr, {k, m}}, {bt.data(), nullptr, {n, k}}, fc,
                            accel::Activation::None, out.data());
  // A leading batch of 3 over one B
  const std::vector<float> ab = Spread(3 * 16 * k, 1.f);
  std::vector<float> outb(3 * 16 * n);
  accel::ExecuteMatMul(*device, {ab.data(), nullptr, {3, 16, k}}, {b.data(), nullptr, {k, n}}, outb.data(),
                       accel::Activation::None);
  // RunKernel's prenorm and skip steps on device buffers (src/ep.cc:1602-1650)
  accel::OwnedBuffer x = accel::Upload(*device, res.data(), {m, n});
  accel::OwnedBuffer extra = accel::Upload(*device, out2.data(), {m, n});
  accel::OwnedBuffer g = accel::Upload(*device, gamma.data(), {n});
  accel::OwnedBuffer y;
  y.device = device.get();
  y.shape = {m, n};
  y.buffer = device->Allocate(static_cast<size_t>(m * n) * sizeof(float));
  device->RmsNorm(x.buffer, g.buffer, y.buffer, m, n, 1e-5f, 0);
  device->ResidualAdd(x.buffer, extra.buffer, m * n);
  device->CopyDeviceToHost(out.data(), x.buffer, out.size() * sizeof(float));
  x.Reset();
  extra.Reset();
  g.Reset();
  y.Reset();

  auto hip = accel::CreateHipDevice();
  Report("runtime steps (ExecuteGemm/MatMul/FusedMatMul, batch, RmsNorm, ResidualAdd)",
         Replay(*traced, *hip, "runtime steps"));
}

// A small Llama through the reference's own llama_model.cc on the recorder: a 12-id prompt and
// 6 greedy tokens, then a 5-id prompt and 5 top-k sampled tokens (src/llama_model.cc:101-131,
// 209-247): Embedding, RmsNorm, MatMul, Rope, AppendCache, Attention, ResidualAdd, SiluMul and
// SampleToken at prompt and decode positions.
void TraceLlama() {
  AccelLlamaConfig cfg{};
  cfg.vocab = 320;
  cfg.hidden = 128;
  cfg.layers = 2;
  cfg.heads = 4;
  cfg.kv_heads = 2;
  cfg.intermediate = 256;
  cfg.context = 32;
  cfg.eps = 1e-5f;
  cfg.rope_theta = 10000.f;
  AccelLlama* model = accel_llama_create(&cfg);
  EXPECT(model != nullptr);
  if (model == nullptr) return;
  TracedDevice* traced = g_traced;
  const int64_t h = cfg.hidden, hd = h / cfg.heads, q = cfg.heads * hd, kv = cfg.kv_heads * hd, inter = cfg.intermediate;
  auto weight = [&](int32_t kind, int32_t layer, int64_t rows, int64_t cols, float scale, float shift) {
    std::vector<float> w = Spread(static_cast<size_t>(rows * cols), scale);
    for (float& x : w) x += shift;
    EXPECT(accel_llama_weight(model, kind, layer, w.data(), rows, cols) == 0);
  };
  weight(ACCEL_W_EMBED, -1, cfg.vocab, h, 0.5f, 0.f);
  weight(ACCEL_W_LM_HEAD, -1, cfg.vocab, h, 0.1f, 0.f);
  weight(ACCEL_W_FINAL_NORM, -1, h, 1, 0.1f, 1.f);
  for (int32_t l = 0; l < cfg.layers; ++l) {
    weight(ACCEL_W_ATTN_NORM, l, h, 1, 0.1f, 1.f);
    weight(ACCEL_W_POST_NORM, l, h, 1, 0.1f, 1.f);
    weight(ACCEL_W_Q, l, q, h, 0.1f, 0.f);
    weight(ACCEL_W_K, l, kv, h, 0.1f, 0.f);
    weight(ACCEL_W_V, l, kv, h, 0.1f, 0.f);
    weight(ACCEL_W_O, l, h, q, 0.1f, 0.f);
    weight(ACCEL_W_GATE, l, inter, h, 0.1f, 0.f);
    weight(ACCEL_W_UP, l, inter, h, 0.1f, 0.f);
    weight(ACCEL_W_DOWN, l, h, inter, 0.1f, 0.f);
  }
  std::vector<int32_t> prompt(12);
  for (size_t i = 0; i < prompt.size(); ++i) prompt[i] = static_cast<int32_t>((i * 37 + 11) % cfg.vocab);
  int32_t ids[16] = {};
  int32_t count = 0;
  EXPECT(accel_llama_generate(model, prompt.data(), 12, 6, -1, 0.f, 0, 0, ids, &count) == 0);
  EXPECT(count == 6);
  EXPECT(accel_llama_generate(model, prompt.data(), 5, 5, -1, 0.8f, 7, 8, ids, &count) == 0);
  EXPECT(count == 5);

  auto hip = accel::CreateHipDevice();
  Report("Llama generate (2 layers, hidden 128, 4/2 heads): prompt 12 + 6 greedy, prompt 5 + 5 top-k",
         Replay(*traced, *hip, "llama"));
  accel_llama_destroy(model);
}

}  // namespace

namespace accel {
// llama_model.cc is compiled with its CreateSimDevice() call renamed to this one.
std::unique_ptr<Device> CreateTracedDevice() {
  auto device = std::make_unique<TracedDevice>();
  g_traced = device.get();
  return device;
}
}  // namespace accel

int main() {
  try {
    accel::HipSetExactProducts(true);  // MatMul stores the reference's k-ordered bits
    TraceRuntimeSteps();
    TraceLlama();
    accel::HipSetExactProducts(false);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "FAIL: exception %s\n", e.what());
    ++g_failures;
  }
  std::printf("%d checks, %d failures\n", g_checks, g_failures);
  return g_failures == 0 ? 0 : 1;
}
