// AccelEP's host runtime over the MI355X device: operand binding, numpy-broadcast batching,
// transposes, epilogues, counters, profile records, constant touches and the KV table store.
//
// Declarations are source-compatible with AccelEP include/accel/runtime.h:9-205 (same
// names, parameter order and meaning), so the plugin's calls (src/ep.cc) bind to these.
// The implementation (accelep_amd/host/runtime.cc) is this library's own: it keeps the
// reference's semantics and counter values and fuses the epilogue passes into the matmul
// kernel's store when the device is the HIP device.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "accel/device.h"

namespace accel {

// Process-wide counters, read and reset as one snapshot (not atomic as a group).
struct AcceleratorStats {
  int64_t matmul_ops = 0;
  int64_t gemm_ops = 0;
  int64_t kernel_matmuls = 0;
  int64_t relu_epilogues = 0;
  int64_t gelu_epilogues = 0;
  int64_t add_epilogues = 0;
  int64_t device_transposes = 0;
  int64_t bytes_to_device = 0;
  int64_t bytes_to_host = 0;
};

// Also clears the profile log.
void ResetAcceleratorStats();
AcceleratorStats GetAcceleratorStats();
void NoteMatmulOp();
void NoteGemmOp();
void NoteKernelMatmul();
void NoteReluEpilogue();
void NoteGeluEpilogue();
void NoteAddEpilogue();
void NoteDeviceTranspose();
void NoteBytesToDevice(size_t bytes);
void NoteBytesToHost(size_t bytes);

struct ProfileTensor {
  std::string name;
  std::vector<int64_t> shape;
};

struct ProfileRecord {
  std::string op;
  std::string activation;
  std::vector<ProfileTensor> inputs;
  ProfileTensor output;
  int64_t bytes_to_device = 0;
  int64_t bytes_to_host = 0;
};

void AppendProfileRecord(ProfileRecord record);
// Writes {"records":[...]} to path; 0 on success, 1 on failure.
int WriteProfile(const char* path);
void ClearProfileForTest();

struct ConstantTouch {
  uint64_t id = 0;
  uint64_t address = 0;
  uint64_t bytes = 0;
};

void NoteConstantTouch(uint64_t id, const void* address, uint64_t bytes);
void ClearConstantTouches();
int64_t ConstantTouchCount();
// Out-of-range indexes read 0.
uint64_t ConstantTouchId(int64_t index);
uint64_t ConstantTouchAddress(int64_t index);
uint64_t ConstantTouchBytes(int64_t index);

// A constant int8 weight kept packed on the device: w = (q - zero) * scale at the
// coordinate ((offset + index) / stride(axis)) % shape[axis]; axis < 0 is one scale for
// the tensor. zero is null when the op has none. q, scale and zero are device pointers.
struct QuantPlane {
  const int8_t* q = nullptr;
  const float* scale = nullptr;
  const int8_t* zero = nullptr;
  std::vector<int64_t> shape;
  int64_t axis = -1;
  int64_t offset = 0;
};

// One input: host floats, a device buffer, or (quant) a packed plane.
struct Operand {
  const float* host = nullptr;
  const OwnedBuffer* on_device = nullptr;
  std::vector<int64_t> shape;
  bool quant = false;
  QuantPlane quant_plane{};
};

struct GemmConfig {
  bool trans_a = false;
  bool trans_b = false;
  float alpha = 1.f;
  float beta = 1.f;
};

// com.microsoft.FusedMatMul: transposes of the last two dims and a scale.
struct FusedMatMulConfig {
  bool trans_a = false;
  bool trans_b = false;
  float alpha = 1.f;
};

// Product of the dims; a negative dim throws invalid_argument, overflow throws overflow_error.
int64_t ElementCount(const std::vector<int64_t>& shape);

bool InferMatMulShape(const std::vector<int64_t>& a, const std::vector<int64_t>& b, std::vector<int64_t>* out);
bool InferFusedMatMulShape(const std::vector<int64_t>& a, bool trans_a, const std::vector<int64_t>& b, bool trans_b,
                           std::vector<int64_t>* out);
bool InferGemmShape(const std::vector<int64_t>& a, bool trans_a, const std::vector<int64_t>& b, bool trans_b,
                    const std::vector<int64_t>* bias, std::vector<int64_t>* out);

// Allocates and fills a device copy of host floats (one counted copy).
OwnedBuffer Upload(Device& device, const float* data, const std::vector<int64_t>& shape);

// dst = src with its last two dims swapped (one Device::Transpose per leading batch).
void PretransposeLastTwo(Device& device, const OwnedBuffer& src, OwnedBuffer* dst);

// C = A @ B where either side may be a packed plane (a null plane reads the float pointer).
// All pointers are device pointers. Notes one kernel matmul and one packed-GEMM probe.
void MatMulQuantized(const float* a, const QuantPlane* a_quant, const float* b, const QuantPlane* b_quant, float* c,
                     int64_t m, int64_t k, int64_t n);

// MatMul with an optional activation and then an optional elementwise residual; the result
// goes to out_host (a counted copy) or, when retain is set, stays on the device in *retain.
void ExecuteMatMul(Device& device, const Operand& a, const Operand& b, float* out_host,
                   Activation activation = Activation::None, const Operand* residual = nullptr,
                   OwnedBuffer* retain = nullptr);

void ExecuteFusedMatMul(Device& device, const Operand& a, const Operand& b, const FusedMatMulConfig& config,
                        Activation activation, float* out_host, OwnedBuffer* retain = nullptr);

// Gemm: alpha * op(A) @ op(B) + beta * bias, then the activation.
void ExecuteGemm(Device& device, const Operand& a, const Operand& b, const Operand* bias, const GemmConfig& config,
                 float* out_host, Activation activation = Activation::None, OwnedBuffer* retain = nullptr);

// Named device tables of fixed row capacity (one map per instance).
class KvTableStore {
 public:
  explicit KvTableStore(Device& device);

  void Create(const std::string& name, int64_t rows, int64_t cols);
  void Append(const std::string& name, const float* data, int64_t n_rows);
  void Update(const std::string& name, int64_t row, const float* data, int64_t n_rows);
  bool Contains(const std::string& name) const;
  void Read(const std::string& name, float* dst, int64_t n_rows) const;
  const void* Storage(const std::string& name) const;
  int64_t Filled(const std::string& name) const;

 private:
  struct Table {
    std::string name;
    OwnedBuffer buffer;
    int64_t rows = 0;
    int64_t cols = 0;
    int64_t filled = 0;
  };

  Device* device_ = nullptr;
  std::vector<Table> tables_;

  Table* Find(const std::string& name);
  const Table* Find(const std::string& name) const;
};

}  // namespace accel
