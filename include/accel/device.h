// The accelerator contract AccelEP's runtime and plugin call, as a C++ interface over the
// accel_hip C-ABI (include/accel_hip.h) on one MI355X.
//
// Declarations are source-compatible with AccelEP include/accel/device.h:10-145: the same
// names, parameter order and meaning, so code written against the reference's Device
// (src/runtime.cc, src/ep.cc, src/llama_model.cc) compiles against this header and runs on
// the GPU through CreateHipDevice(). Exceptions are the reference's: invalid_argument for
// shapes and ranges, overflow_error, logic_error for a free of an unknown buffer, bad_alloc;
// a HIP runtime failure is runtime_error.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <utility>
#include <vector>

namespace accel {

enum class Activation { None, Relu, Gelu };

// "none", "relu" or "gelu" (the profile JSON spelling).
const char* ActivationName(Activation activation);

// Device memory. Host code passes `data` back to the Device that allocated it and never
// dereferences it. Allocations carry a process-wide id from 1; a slice has id 0.
struct DeviceBuffer {
  void* data = nullptr;
  size_t bytes = 0;
  uint64_t id = 0;
};

class Device;

// Move-only owner of one allocation; frees it on `device` when reset or destroyed.
struct OwnedBuffer {
  Device* device = nullptr;
  DeviceBuffer buffer{};
  std::vector<int64_t> shape;

  OwnedBuffer() = default;
  OwnedBuffer(const OwnedBuffer&) = delete;
  OwnedBuffer& operator=(const OwnedBuffer&) = delete;
  OwnedBuffer(OwnedBuffer&& other) noexcept { TakeFrom(other); }
  OwnedBuffer& operator=(OwnedBuffer&& other) noexcept {
    if (this != &other) {
      Reset();
      TakeFrom(other);
    }
    return *this;
  }
  ~OwnedBuffer() { Reset(); }

  // Frees the allocation (if any) and clears the handle. Never throws.
  void Reset() noexcept;

 private:
  void TakeFrom(OwnedBuffer& other) noexcept {
    device = other.device;
    buffer = other.buffer;
    shape = std::move(other.shape);
    other.device = nullptr;
    other.buffer = DeviceBuffer{};
  }
};

class Device {
 public:
  virtual ~Device() = default;

  virtual const char* Name() const = 0;

  // Zero-filled; a 0-byte request still returns a non-null pointer.
  virtual DeviceBuffer Allocate(size_t bytes) = 0;
  // A null `data` is a no-op; an unknown (data, bytes, id) throws logic_error.
  virtual void Free(DeviceBuffer buffer) = 0;

  // Counted copies (bytes_to_device / bytes_to_host).
  virtual void CopyHostToDevice(DeviceBuffer dst, const void* src, size_t bytes) = 0;
  virtual void CopyDeviceToHost(void* dst, DeviceBuffer src, size_t bytes) = 0;

  // C[m, n] = A[m, k] @ B[k, n], row-major fp32; C is overwritten.
  virtual void MatMul(DeviceBuffer a, DeviceBuffer b, DeviceBuffer c, int64_t m, int64_t k, int64_t n) = 0;

  // dst[cols, rows] = transpose of src[rows, cols].
  virtual void Transpose(DeviceBuffer src, DeviceBuffer dst, int64_t rows, int64_t cols) = 0;

  // In place: c = alpha*c (+ beta*bias broadcast, bias_shape right-aligned to [m, n]),
  // then the activation. bias == nullptr: no bias.
  virtual void GemmEpilogue(DeviceBuffer c, int64_t m, int64_t n, float alpha, const DeviceBuffer* bias,
                            const std::vector<int64_t>& bias_shape, float beta,
                            Activation activation = Activation::None) = 0;

  // out[s, :] = table[ids[id_offset + s], :]; ids are int32; an id outside [0, vocab) throws.
  virtual void Embedding(DeviceBuffer ids, int64_t id_offset, DeviceBuffer table, DeviceBuffer out, int64_t seq,
                         int64_t hidden, int64_t vocab) = 0;

  // y[row, :] = RMSNorm(x[row_offset + row, :]) * weight.
  virtual void RmsNorm(DeviceBuffer x, DeviceBuffer weight, DeviceBuffer y, int64_t rows, int64_t dim, float eps,
                       int64_t row_offset) = 0;

  // Rotate-half RoPE in place; table rows are head_dim wide, indexed by absolute position.
  virtual void Rope(DeviceBuffer states, DeviceBuffer cos_table, DeviceBuffer sin_table, int64_t seq, int64_t n_heads,
                    int64_t head_dim, int64_t position) = 0;

  // cache[position + s, :] = src[s, :] for s < seq (rows of n_heads * head_dim floats).
  virtual void AppendCache(DeviceBuffer src, DeviceBuffer cache, int64_t seq, int64_t position, int64_t n_heads,
                           int64_t head_dim) = 0;

  // Causal grouped-query attention over cache rows [0, position + seq).
  virtual void Attention(DeviceBuffer q, DeviceBuffer k, DeviceBuffer v, DeviceBuffer scores, DeviceBuffer out,
                         int64_t seq, int64_t position, int64_t heads, int64_t kv_heads, int64_t head_dim) = 0;

  // gate = silu(gate) * up.
  virtual void SiluMul(DeviceBuffer gate, DeviceBuffer up, int64_t count) = 0;

  // dest += extra.
  virtual void ResidualAdd(DeviceBuffer dest, DeviceBuffer extra, int64_t count) = 0;

  // chosen_ids[chosen_index] = the sampled id (int32): argmax (earlier id on a tie) when
  // !(temperature > 0), else a draw over all logits or the top_k (at most 64) of them.
  virtual void SampleToken(DeviceBuffer logits, DeviceBuffer chosen_ids, int64_t chosen_index, int64_t vocab,
                           float temperature, uint32_t* rng_state, int top_k) = 0;
};

// The MI355X device (one process-wide GPU context shared by every instance). Destroying
// an instance frees nothing: allocations that are never freed stay in LiveDeviceAllocs().
std::unique_ptr<Device> CreateHipDevice();

// Device allocations not yet freed, process-wide.
int64_t LiveDeviceAllocs();

// Packed-GEMM probes: calls of MatMul / MatMulQuantized, and the sum of their k.
int64_t PackedMatMulCalls();
int64_t PackedKTrips();
void ResetPackedGemmProbes();

}  // namespace accel
