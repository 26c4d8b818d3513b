// Calls of the MI355X device beyond the accel::Device contract (no reference counterpart):
// a matmul with its epilogue fused into the kernel's store. The runtime uses them when the
// device is the HIP device, in place of the reference's MatMul -> GemmEpilogue ->
// GemmEpilogue(residual) sequence (src/runtime.cc:332-344); the stored values are the
// same, element for element, as that sequence's.
#pragma once

#include <cstdint>
#include <memory>
#include <vector>

#include "accel/runtime.h"

namespace accel {

// What the fused store applies, in order: v = alpha*acc; if bias: v = v + beta*bias
// (bias_shape right-aligned to [m, n]); activation; if residual: v = v + residual[i*n + j].
// Pointers are device pointers; bias and residual may be null.
struct FusedEpilogue {
  float alpha = 1.f;
  float beta = 1.f;
  const float* bias = nullptr;
  std::vector<int64_t> bias_shape;
  Activation activation = Activation::None;
  const float* residual = nullptr;
};

// The MI355X device (also declared in accel/device.h; repeated here so that a source built
// against another copy of accel/device.h, such as AccelEP's own, needs only this header).
std::unique_ptr<Device> CreateHipDevice();

// True for devices made by CreateHipDevice().
bool IsHipDevice(const Device& device);

// C = epilogue(A @ B), fp32; one kernel matmul. The buffers are bounds-checked like MatMul.
void HipMatMulFused(Device& device, DeviceBuffer a, DeviceBuffer b, DeviceBuffer c, int64_t m, int64_t k, int64_t n,
                    const FusedEpilogue& epilogue);

// MatMulQuantized with the epilogue fused into the store; one kernel matmul.
void HipMatMulQuantizedFused(const float* a, const QuantPlane* a_quant, const float* b, const QuantPlane* b_quant,
                             float* c, int64_t m, int64_t k, int64_t n, const FusedEpilogue& epilogue);

// Builds the staged copies MatMulQuantized reads for this int8 weight now (every layout its
// form allows; each batch matrix of a plane of rank > 2), instead of at the weight's first
// use: for BindConstant (src/ep.cc:1430-1463), outside any graph capture.
void HipPrepareQuantized(const QuantPlane& weight);

// Waits until every kernel the library has launched has finished.
void HipSynchronize();

// Exact products on or off, process-wide: on, every matmul stores the bits of the
// reference's k-ordered split-product loop (accel_hip_set_exact_products).
void HipSetExactProducts(bool on);
bool HipExactProducts();

}  // namespace accel
