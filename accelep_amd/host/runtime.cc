// AccelEP's host runtime over the MI355X device: what src/runtime.cc does for the plugin
// (operand binding, numpy-broadcast batch loops, transposes, epilogues, counters, profile
// and touch logs, KvTableStore), written for this device.
//
// Semantics follow src/runtime.cc:51-823: the same shape rules, exception types, counter
// values, allocation order and delivery. One thing differs in how the work is done: on the
// HIP device the epilogue passes the reference runs after each product (alpha and
// activation over C, then the residual add, src/runtime.cc:332-344,709-719; the Gemm bias
// epilogue, :785-795) are applied in the matmul kernel's store instead. Each stored value
// goes through the same rounded steps in the same order, so the result is the same, and C
// is written once instead of three times.
#include <algorithm>
#include <atomic>
#include <fstream>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <utility>

#include "accel/hip_device.h"
#include "accel/runtime.h"

namespace accel {
namespace {

// ---- counters and logs -----------------------------------------------------------------

enum Counter : int {
  kMatmulOps,
  kGemmOps,
  kKernelMatmuls,
  kReluEpilogues,
  kGeluEpilogues,
  kAddEpilogues,
  kDeviceTransposes,
  kBytesToDevice,
  kBytesToHost,
  kCounterCount
};

std::atomic<int64_t>* Counters() {
  static std::atomic<int64_t> counters[kCounterCount];
  return counters;
}

void Bump(Counter which, int64_t amount) { Counters()[which].fetch_add(amount, std::memory_order_relaxed); }

struct Logs {
  std::mutex profile_mu;
  std::vector<ProfileRecord> profile;
  std::mutex touch_mu;
  std::vector<ConstantTouch> touches;
};

Logs& TheLogs() {
  static Logs logs;
  return logs;
}

// ---- shapes ----------------------------------------------------------------------------

// Right-aligned numpy broadcast of two batch shapes. A zero-length dim is allowed, a
// negative one is not (src/runtime.cc:51-72).
bool BroadcastBatch(const std::vector<int64_t>& a, const std::vector<int64_t>& b, std::vector<int64_t>* out) {
  const size_t rank = std::max(a.size(), b.size());
  out->assign(rank, 1);
  for (size_t i = 0; i < rank; ++i) {
    const int64_t da = i + a.size() >= rank ? a[i + a.size() - rank] : 1;
    const int64_t db = i + b.size() >= rank ? b[i + b.size() - rank] : 1;
    if (da < 0 || db < 0) return false;
    if (da != db && da != 1 && db != 1) return false;
    (*out)[i] = da == 1 ? db : da;
  }
  return true;
}

// A Gemm bias of rank <= 2 whose dims are 1 or the matching dim of [m, n] (src/runtime.cc:74-89).
bool BiasFits(const std::vector<int64_t>& shape, int64_t m, int64_t n) {
  if (shape.size() > 2) return false;
  const int64_t target[2] = {m, n};
  for (size_t d = 0; d < shape.size(); ++d) {
    const int64_t want = target[2 - shape.size() + d];
    if (shape[d] < 0 || (shape[d] != 1 && shape[d] != want)) return false;
  }
  return true;
}

bool NoNegative(const std::vector<int64_t>& shape) {
  return std::all_of(shape.begin(), shape.end(), [](int64_t d) { return d >= 0; });
}

// Row-major index of the batch matrix an operand with batch dims `dims` contributes to the
// output batch `out_index` (dims right-aligned; a dim of 1 is broadcast) (src/runtime.cc:91-111).
int64_t BatchMatrix(const std::vector<int64_t>& dims, const std::vector<int64_t>& out_index) {
  int64_t linear = 0;
  const size_t skip = out_index.size() - dims.size();
  for (size_t i = 0; i < dims.size(); ++i) {
    const int64_t coord = dims[i] == 1 ? 0 : out_index[skip + i];
    linear = linear * dims[i] + coord;
  }
  return linear;
}

// Odometer step over `shape`.
void Advance(std::vector<int64_t>* index, const std::vector<int64_t>& shape) {
  for (size_t axis = index->size(); axis-- > 0;) {
    if (++(*index)[axis] < shape[axis]) return;
    (*index)[axis] = 0;
  }
}

// ---- operands and buffers --------------------------------------------------------------

// The device buffer of a float operand, uploading host data into *upload (src/runtime.cc:122-139).
DeviceBuffer BindFloat(Device& device, const Operand& op, OwnedBuffer* upload) {
  if (op.quant) throw std::invalid_argument("quantized operand has no float buffer");
  if (op.on_device != nullptr) {
    if (op.host != nullptr) throw std::invalid_argument("an operand needs exactly one of host or device memory");
    if (op.on_device->shape != op.shape) throw std::invalid_argument("device operand shape does not match");
    return op.on_device->buffer;
  }
  if (op.host == nullptr && ElementCount(op.shape) != 0) throw std::invalid_argument("missing host data");
  *upload = Upload(device, op.host, op.shape);
  return upload->buffer;
}

// A float operand of a quantized product: its base pointer (src/runtime.cc:285-306).
const float* BindFloatPointer(Device& device, const Operand& op, OwnedBuffer* upload) {
  if (op.on_device != nullptr) {
    if (op.host != nullptr || op.on_device->shape != op.shape)
      throw std::invalid_argument("device operand shape does not match");
    return static_cast<const float*>(op.on_device->buffer.data);
  }
  *upload = Upload(device, op.host, op.shape);
  return static_cast<const float*>(upload->buffer.data);
}

// Elements [offset, offset + count) of a float buffer, as a slice (id 0).
DeviceBuffer Slice(DeviceBuffer base, int64_t offset, int64_t count) {
  return DeviceBuffer{static_cast<float*>(base.data) + offset, static_cast<size_t>(count) * sizeof(float), 0};
}

OwnedBuffer NewBuffer(Device& device, std::vector<int64_t> shape) {
  OwnedBuffer out;
  out.device = &device;
  out.buffer = device.Allocate(static_cast<size_t>(ElementCount(shape)) * sizeof(float));
  out.shape = std::move(shape);
  return out;
}

void NoteActivation(Activation activation) {
  if (activation == Activation::Relu) NoteReluEpilogue();
  if (activation == Activation::Gelu) NoteGeluEpilogue();
}

// Hands the result over: into *retain, or one counted copy to the host (src/runtime.cc:171-180).
void Deliver(Device& device, OwnedBuffer* out, int64_t count, float* out_host, OwnedBuffer* retain) {
  if (retain != nullptr) {
    retain->Reset();
    *retain = std::move(*out);
  } else if (count > 0) {
    device.CopyDeviceToHost(out_host, out->buffer, static_cast<size_t>(count) * sizeof(float));
  }
}

// The residual of a fused store, bound and range-checked as the reference's residual
// epilogue checks its bias operand (src/sim_device.cc:214-223).
const float* BindResidual(Device& device, const Operand& residual, int64_t count, OwnedBuffer* upload) {
  const DeviceBuffer buf = BindFloat(device, residual, upload);
  const size_t need = static_cast<size_t>(count) * sizeof(float);
  if (need != 0 && (buf.data == nullptr || buf.bytes < need)) throw std::invalid_argument("Gemm bias is out of range");
  return static_cast<const float*>(buf.data);
}

// ---- MatMul / FusedMatMul (src/runtime.cc:254-416) --------------------------------------

void RunMatMul(Device& device, const Operand& a, const Operand& b, const FusedMatMulConfig& config,
               Activation activation, const Operand* residual, float* out_host, OwnedBuffer* retain) {
  std::vector<int64_t> out_shape;
  if (!InferFusedMatMulShape(a.shape, config.trans_a, b.shape, config.trans_b, &out_shape))
    throw std::invalid_argument("FusedMatMul shapes are not supported");
  const int64_t a_rows = a.shape[a.shape.size() - 2], a_cols = a.shape.back();
  const int64_t b_rows = b.shape[b.shape.size() - 2], b_cols = b.shape.back();
  const int64_t m = config.trans_a ? a_cols : a_rows;
  const int64_t k = config.trans_a ? a_rows : a_cols;
  const int64_t n = config.trans_b ? b_rows : b_cols;
  const std::vector<int64_t> a_batch(a.shape.begin(), a.shape.end() - 2);
  const std::vector<int64_t> b_batch(b.shape.begin(), b.shape.end() - 2);
  const std::vector<int64_t> out_batch(out_shape.begin(), out_shape.end() - 2);
  const bool quant = a.quant || b.quant;
  if (quant && (config.trans_a || config.trans_b))
    throw std::invalid_argument("quantized MatMul does not transpose its operands");

  const int64_t out_count = ElementCount(out_shape);
  OwnedBuffer a_upload, b_upload;
  DeviceBuffer a_buf{}, b_buf{};
  const float* a_base = nullptr;
  const float* b_base = nullptr;
  if (quant) {
    // The quantized path checks the output before binding its operands.
    if (retain == nullptr && out_count > 0 && out_host == nullptr)
      throw std::invalid_argument("missing FusedMatMul output");
    if (!a.quant) a_base = BindFloatPointer(device, a, &a_upload);
    if (!b.quant) b_base = BindFloatPointer(device, b, &b_upload);
  } else {
    a_buf = BindFloat(device, a, &a_upload);
    b_buf = BindFloat(device, b, &b_upload);
    if (retain == nullptr && out_count > 0 && out_host == nullptr)
      throw std::invalid_argument("missing FusedMatMul output");
  }
  OwnedBuffer out = NewBuffer(device, out_shape);
  OwnedBuffer a_t, b_t;
  if (!quant && config.trans_a) a_t = NewBuffer(device, {m, k});
  if (!quant && config.trans_b) b_t = NewBuffer(device, {k, n});

  const bool scale_or_act = out_count > 0 && (config.alpha != 1.f || activation != Activation::None);
  const bool fuse = IsHipDevice(device);
  FusedEpilogue epilogue;
  epilogue.alpha = config.alpha;
  epilogue.activation = activation;
  OwnedBuffer residual_upload;
  const float* residual_base = nullptr;
  if (fuse && residual != nullptr && out_count > 0)
    residual_base = BindResidual(device, *residual, out_count, &residual_upload);
  const bool fused_store = fuse && (scale_or_act || residual_base != nullptr);

  const int64_t batches = out_batch.empty() ? 1 : ElementCount(out_batch);
  std::vector<int64_t> index(out_batch.size(), 0);
  for (int64_t batch = 0; batch < batches; ++batch) {
    const int64_t a_off = BatchMatrix(a_batch, index) * a_rows * a_cols;
    const int64_t b_off = BatchMatrix(b_batch, index) * b_rows * b_cols;
    const int64_t c_off = batch * m * n;
    epilogue.residual = residual_base == nullptr ? nullptr : residual_base + c_off;
    if (quant) {
      QuantPlane a_plane = a.quant_plane, b_plane = b.quant_plane;
      if (a.quant) a_plane.offset += a_off;
      if (b.quant) b_plane.offset += b_off;
      const float* ap = a.quant ? nullptr : a_base + a_off;
      const float* bp = b.quant ? nullptr : b_base + b_off;
      float* cp = out_count == 0 ? nullptr : static_cast<float*>(out.buffer.data) + c_off;
      if (fused_store) {
        HipMatMulQuantizedFused(ap, a.quant ? &a_plane : nullptr, bp, b.quant ? &b_plane : nullptr, cp, m, k, n,
                                epilogue);
      } else {
        MatMulQuantized(ap, a.quant ? &a_plane : nullptr, bp, b.quant ? &b_plane : nullptr, cp, m, k, n);
      }
    } else {
      DeviceBuffer a_mat = Slice(a_buf, a_off, a_rows * a_cols);
      DeviceBuffer b_mat = Slice(b_buf, b_off, b_rows * b_cols);
      if (config.trans_a) {
        device.Transpose(a_mat, a_t.buffer, a_rows, a_cols);
        a_mat = a_t.buffer;
      }
      if (config.trans_b) {
        device.Transpose(b_mat, b_t.buffer, b_rows, b_cols);
        b_mat = b_t.buffer;
      }
      const DeviceBuffer c_mat = Slice(out.buffer, c_off, m * n);
      if (fused_store) {
        HipMatMulFused(device, a_mat, b_mat, c_mat, m, k, n, epilogue);
      } else {
        device.MatMul(a_mat, b_mat, c_mat, m, k, n);
      }
    }
    if (batch + 1 < batches) Advance(&index, out_batch);
  }
  if (!fuse && scale_or_act) device.GemmEpilogue(out.buffer, out_count, 1, config.alpha, nullptr, {}, 0.f, activation);
  NoteActivation(activation);
  if (residual != nullptr) {
    if (!fuse && out_count > 0) {
      const DeviceBuffer r = BindFloat(device, *residual, &residual_upload);
      device.GemmEpilogue(out.buffer, 1, out_count, 1.f, &r, std::vector<int64_t>{out_count}, 1.f, Activation::None);
    }
    NoteAddEpilogue();
  }
  Deliver(device, &out, out_count, out_host, retain);
  NoteMatmulOp();
}

// ---- profile JSON (the byte format of src/runtime.cc:182-252) ------------------------------

void AppendEscaped(std::string* out, const std::string& text) {
  for (const char ch : text) {
    if (ch == '"' || ch == '\\') out->push_back('\\');
    out->push_back(ch);
  }
}

void AppendShape(std::string* out, const std::vector<int64_t>& shape) {
  out->push_back('[');
  for (size_t i = 0; i < shape.size(); ++i) {
    if (i != 0) out->push_back(',');
    *out += std::to_string(shape[i]);
  }
  out->push_back(']');
}

void AppendTensor(std::string* out, const ProfileTensor& t) {
  *out += "{\"name\":\"";
  AppendEscaped(out, t.name);
  *out += "\",\"shape\":";
  AppendShape(out, t.shape);
  out->push_back('}');
}

std::string ProfileJson() {
  Logs& logs = TheLogs();
  std::lock_guard<std::mutex> lock(logs.profile_mu);
  std::string out = "{\"records\":[";
  for (size_t r = 0; r < logs.profile.size(); ++r) {
    const ProfileRecord& rec = logs.profile[r];
    if (r != 0) out.push_back(',');
    out += "{\"op\":\"";
    AppendEscaped(&out, rec.op);
    out += "\",\"activation\":\"";
    AppendEscaped(&out, rec.activation);
    out += "\",\"inputs\":[";
    for (size_t i = 0; i < rec.inputs.size(); ++i) {
      if (i != 0) out.push_back(',');
      AppendTensor(&out, rec.inputs[i]);
    }
    out += "],\"output\":";
    AppendTensor(&out, rec.output);
    out += ",\"bytes_to_device\":" + std::to_string(rec.bytes_to_device);
    out += ",\"bytes_to_host\":" + std::to_string(rec.bytes_to_host);
    out.push_back('}');
  }
  out += "]}";
  return out;
}

template <typename Field>
uint64_t TouchField(int64_t index, Field field) {
  Logs& logs = TheLogs();
  std::lock_guard<std::mutex> lock(logs.touch_mu);
  if (index < 0 || static_cast<size_t>(index) >= logs.touches.size()) return 0;
  return field(logs.touches[static_cast<size_t>(index)]);
}

}  // namespace

// ---- counters --------------------------------------------------------------------------

void ResetAcceleratorStats() {
  for (int i = 0; i < kCounterCount; ++i) Counters()[i].store(0, std::memory_order_relaxed);
  Logs& logs = TheLogs();
  std::lock_guard<std::mutex> lock(logs.profile_mu);
  logs.profile.clear();
}

AcceleratorStats GetAcceleratorStats() {
  const std::atomic<int64_t>* c = Counters();
  AcceleratorStats s;
  s.matmul_ops = c[kMatmulOps].load();
  s.gemm_ops = c[kGemmOps].load();
  s.kernel_matmuls = c[kKernelMatmuls].load();
  s.relu_epilogues = c[kReluEpilogues].load();
  s.gelu_epilogues = c[kGeluEpilogues].load();
  s.add_epilogues = c[kAddEpilogues].load();
  s.device_transposes = c[kDeviceTransposes].load();
  s.bytes_to_device = c[kBytesToDevice].load();
  s.bytes_to_host = c[kBytesToHost].load();
  return s;
}

void NoteMatmulOp() { Bump(kMatmulOps, 1); }
void NoteGemmOp() { Bump(kGemmOps, 1); }
void NoteKernelMatmul() { Bump(kKernelMatmuls, 1); }
void NoteReluEpilogue() { Bump(kReluEpilogues, 1); }
void NoteGeluEpilogue() { Bump(kGeluEpilogues, 1); }
void NoteAddEpilogue() { Bump(kAddEpilogues, 1); }
void NoteDeviceTranspose() { Bump(kDeviceTransposes, 1); }
void NoteBytesToDevice(size_t bytes) { Bump(kBytesToDevice, static_cast<int64_t>(bytes)); }
void NoteBytesToHost(size_t bytes) { Bump(kBytesToHost, static_cast<int64_t>(bytes)); }

// ---- profile and constant touches --------------------------------------------------------

void AppendProfileRecord(ProfileRecord record) {
  Logs& logs = TheLogs();
  std::lock_guard<std::mutex> lock(logs.profile_mu);
  logs.profile.push_back(std::move(record));
}

int WriteProfile(const char* path) {
  if (path == nullptr) return 1;
  const std::string json = ProfileJson();
  std::ofstream file(path, std::ios::binary | std::ios::trunc);
  if (!file) return 1;
  file << json;
  return file ? 0 : 1;
}

void ClearProfileForTest() {
  Logs& logs = TheLogs();
  std::lock_guard<std::mutex> lock(logs.profile_mu);
  logs.profile.clear();
}

void NoteConstantTouch(uint64_t id, const void* address, uint64_t bytes) {
  Logs& logs = TheLogs();
  std::lock_guard<std::mutex> lock(logs.touch_mu);
  logs.touches.push_back(ConstantTouch{id, reinterpret_cast<uint64_t>(address), bytes});
}

void ClearConstantTouches() {
  Logs& logs = TheLogs();
  std::lock_guard<std::mutex> lock(logs.touch_mu);
  logs.touches.clear();
}

int64_t ConstantTouchCount() {
  Logs& logs = TheLogs();
  std::lock_guard<std::mutex> lock(logs.touch_mu);
  return static_cast<int64_t>(logs.touches.size());
}

uint64_t ConstantTouchId(int64_t index) {
  return TouchField(index, [](const ConstantTouch& t) { return t.id; });
}
uint64_t ConstantTouchAddress(int64_t index) {
  return TouchField(index, [](const ConstantTouch& t) { return t.address; });
}
uint64_t ConstantTouchBytes(int64_t index) {
  return TouchField(index, [](const ConstantTouch& t) { return t.bytes; });
}

// ---- shapes ----------------------------------------------------------------------------

int64_t ElementCount(const std::vector<int64_t>& shape) {
  int64_t count = 1;
  for (const int64_t dim : shape) {
    if (dim < 0) throw std::invalid_argument("dynamic dimension");
    if (dim != 0 && count > std::numeric_limits<int64_t>::max() / dim) throw std::overflow_error("tensor is too large");
    count *= dim;
  }
  return count;
}

bool InferMatMulShape(const std::vector<int64_t>& a, const std::vector<int64_t>& b, std::vector<int64_t>* out) {
  if (out == nullptr || a.size() < 2 || b.size() < 2 || !NoNegative(a) || !NoNegative(b)) return false;
  if (a.back() != b[b.size() - 2]) return false;
  std::vector<int64_t> shape;
  if (!BroadcastBatch(std::vector<int64_t>(a.begin(), a.end() - 2), std::vector<int64_t>(b.begin(), b.end() - 2),
                      &shape))
    return false;
  shape.push_back(a[a.size() - 2]);
  shape.push_back(b.back());
  *out = std::move(shape);
  return true;
}

bool InferFusedMatMulShape(const std::vector<int64_t>& a, bool trans_a, const std::vector<int64_t>& b, bool trans_b,
                           std::vector<int64_t>* out) {
  std::vector<int64_t> la = a, lb = b;
  if (trans_a) {
    if (la.size() < 2) return false;
    std::swap(la[la.size() - 2], la.back());
  }
  if (trans_b) {
    if (lb.size() < 2) return false;
    std::swap(lb[lb.size() - 2], lb.back());
  }
  return InferMatMulShape(la, lb, out);
}

bool InferGemmShape(const std::vector<int64_t>& a, bool trans_a, const std::vector<int64_t>& b, bool trans_b,
                    const std::vector<int64_t>* bias, std::vector<int64_t>* out) {
  if (out == nullptr || a.size() != 2 || b.size() != 2 || !NoNegative(a) || !NoNegative(b)) return false;
  if ((trans_a ? a[0] : a[1]) != (trans_b ? b[1] : b[0])) return false;
  const int64_t m = trans_a ? a[1] : a[0];
  const int64_t n = trans_b ? b[0] : b[1];
  if (bias != nullptr && !BiasFits(*bias, m, n)) return false;
  *out = {m, n};
  return true;
}

// ---- uploads and transposes ------------------------------------------------------------

OwnedBuffer Upload(Device& device, const float* data, const std::vector<int64_t>& shape) {
  const int64_t count = ElementCount(shape);
  if (count > 0 && data == nullptr) throw std::invalid_argument("missing host data");
  OwnedBuffer owned = NewBuffer(device, shape);
  if (count > 0) device.CopyHostToDevice(owned.buffer, data, static_cast<size_t>(count) * sizeof(float));
  return owned;
}

void PretransposeLastTwo(Device& device, const OwnedBuffer& src, OwnedBuffer* dst) {
  if (dst == nullptr || src.shape.size() < 2 || src.buffer.data == nullptr)
    throw std::invalid_argument("pretranspose needs a matrix");
  const int64_t rows = src.shape[src.shape.size() - 2];
  const int64_t cols = src.shape.back();
  std::vector<int64_t> shape = src.shape;
  std::swap(shape[shape.size() - 2], shape.back());
  const int64_t batches = ElementCount(std::vector<int64_t>(src.shape.begin(), src.shape.end() - 2));
  dst->Reset();
  *dst = NewBuffer(device, std::move(shape));
  const int64_t tile = rows * cols;
  for (int64_t b = 0; b < batches; ++b)
    device.Transpose(Slice(src.buffer, b * tile, tile), Slice(dst->buffer, b * tile, tile), rows, cols);
}

// ---- Execute* ----------------------------------------------------------------------------

void ExecuteFusedMatMul(Device& device, const Operand& a, const Operand& b, const FusedMatMulConfig& config,
                        Activation activation, float* out_host, OwnedBuffer* retain) {
  RunMatMul(device, a, b, config, activation, nullptr, out_host, retain);
}

void ExecuteMatMul(Device& device, const Operand& a, const Operand& b, float* out_host, Activation activation,
                   const Operand* residual, OwnedBuffer* retain) {
  RunMatMul(device, a, b, FusedMatMulConfig{}, activation, residual, out_host, retain);
}

void ExecuteGemm(Device& device, const Operand& a, const Operand& b, const Operand* bias, const GemmConfig& config,
                 float* out_host, Activation activation, OwnedBuffer* retain) {
  std::vector<int64_t> out_shape;
  if (!InferGemmShape(a.shape, config.trans_a, b.shape, config.trans_b, bias == nullptr ? nullptr : &bias->shape,
                      &out_shape))
    throw std::invalid_argument("Gemm shapes are not supported");
  const int64_t m = config.trans_a ? a.shape[1] : a.shape[0];
  const int64_t k = config.trans_a ? a.shape[0] : a.shape[1];
  const int64_t n = config.trans_b ? b.shape[0] : b.shape[1];

  OwnedBuffer a_upload, b_upload, bias_upload, a_t, b_t;
  DeviceBuffer a_mat = BindFloat(device, a, &a_upload);
  DeviceBuffer b_mat = BindFloat(device, b, &b_upload);
  if (config.trans_a) {
    a_t = NewBuffer(device, {m, k});
    device.Transpose(a_mat, a_t.buffer, k, m);
    a_mat = a_t.buffer;
  }
  if (config.trans_b) {
    b_t = NewBuffer(device, {k, n});
    device.Transpose(b_mat, b_t.buffer, n, k);
    b_mat = b_t.buffer;
  }
  const int64_t out_count = m * n;
  if (retain == nullptr && out_count > 0 && out_host == nullptr) throw std::invalid_argument("missing Gemm output");
  OwnedBuffer out = NewBuffer(device, out_shape);

  const bool epilogue_pass = bias != nullptr || config.alpha != 1.f || activation != Activation::None;
  DeviceBuffer bias_buf{};
  if (IsHipDevice(device)) {
    FusedEpilogue e;
    e.alpha = config.alpha;
    e.beta = config.beta;
    e.activation = activation;
    if (bias != nullptr) {
      bias_buf = BindFloat(device, *bias, &bias_upload);
      const size_t need = static_cast<size_t>(ElementCount(bias->shape)) * sizeof(float);
      if (need != 0 && (bias_buf.data == nullptr || bias_buf.bytes < need))
        throw std::invalid_argument("Gemm bias is out of range");
      e.bias = static_cast<const float*>(bias_buf.data);
      e.bias_shape = bias->shape;
    }
    if (epilogue_pass) {
      HipMatMulFused(device, a_mat, b_mat, out.buffer, m, k, n, e);
    } else {
      device.MatMul(a_mat, b_mat, out.buffer, m, k, n);
    }
  } else {
    device.MatMul(a_mat, b_mat, out.buffer, m, k, n);
    if (epilogue_pass) {
      const DeviceBuffer* bias_ptr = nullptr;
      if (bias != nullptr) {
        bias_buf = BindFloat(device, *bias, &bias_upload);
        bias_ptr = &bias_buf;
      }
      device.GemmEpilogue(out.buffer, m, n, config.alpha, bias_ptr,
                          bias == nullptr ? std::vector<int64_t>{} : bias->shape, config.beta, activation);
    }
  }
  NoteActivation(activation);
  Deliver(device, &out, out_count, out_host, retain);
  NoteGemmOp();
}

// ---- KvTableStore (src/runtime.cc:725-821) -------------------------------------------------

KvTableStore::KvTableStore(Device& device) : device_(&device) {}

KvTableStore::Table* KvTableStore::Find(const std::string& name) {
  for (Table& t : tables_)
    if (t.name == name) return &t;
  return nullptr;
}

const KvTableStore::Table* KvTableStore::Find(const std::string& name) const {
  for (const Table& t : tables_)
    if (t.name == name) return &t;
  return nullptr;
}

void KvTableStore::Create(const std::string& name, int64_t rows, int64_t cols) {
  if (name.empty() || rows < 0 || cols < 0 || Find(name) != nullptr)
    throw std::invalid_argument("KvTable Create rejected");
  Table t;
  t.name = name;
  t.rows = rows;
  t.cols = cols;
  t.buffer = NewBuffer(*device_, {rows, cols});
  tables_.push_back(std::move(t));
}

void KvTableStore::Append(const std::string& name, const float* data, int64_t n_rows) {
  Table* t = Find(name);
  if (t == nullptr || n_rows < 0 || t->filled > t->rows - n_rows || (n_rows > 0 && data == nullptr))
    throw std::invalid_argument("KvTable Append rejected");
  if (n_rows > 0) {
    const DeviceBuffer rows = Slice(t->buffer.buffer, t->filled * t->cols, n_rows * t->cols);
    device_->CopyHostToDevice(rows, data, rows.bytes);
  }
  t->filled += n_rows;
}

void KvTableStore::Update(const std::string& name, int64_t row, const float* data, int64_t n_rows) {
  Table* t = Find(name);
  if (t == nullptr || row < 0 || n_rows < 0 || row > t->filled || n_rows > t->filled - row ||
      (n_rows > 0 && data == nullptr))
    throw std::invalid_argument("KvTable Update rejected");
  if (n_rows > 0) {
    const DeviceBuffer rows = Slice(t->buffer.buffer, row * t->cols, n_rows * t->cols);
    device_->CopyHostToDevice(rows, data, rows.bytes);
  }
}

bool KvTableStore::Contains(const std::string& name) const { return Find(name) != nullptr; }

void KvTableStore::Read(const std::string& name, float* dst, int64_t n_rows) const {
  const Table* t = Find(name);
  if (t == nullptr || dst == nullptr || n_rows < 0 || n_rows > t->filled)
    throw std::invalid_argument("KvTable Read rejected");
  if (n_rows == 0) return;
  // The table's own id, so the copy is checked against the whole allocation.
  const DeviceBuffer src{t->buffer.buffer.data, static_cast<size_t>(n_rows * t->cols) * sizeof(float),
                         t->buffer.buffer.id};
  device_->CopyDeviceToHost(dst, src, src.bytes);
}

const void* KvTableStore::Storage(const std::string& name) const {
  const Table* t = Find(name);
  if (t == nullptr) throw std::invalid_argument("KvTable Storage rejected");
  return t->buffer.buffer.data;
}

int64_t KvTableStore::Filled(const std::string& name) const {
  const Table* t = Find(name);
  if (t == nullptr) throw std::invalid_argument("KvTable Filled rejected");
  return t->filled;
}

}  // namespace accel
