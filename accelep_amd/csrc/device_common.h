// Device-side helpers shared by the kernel files (HIP only).
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace accel_hip {

// Bias index of element (i, j) for a bias of rank 0..2 right-aligned against [m, n];
// a dimension of size 1 broadcasts (BiasOffset, src/sim_device.cc:104-124).
__device__ __forceinline__ int64_t BiasIndex(const Epilogue& e, int64_t i, int64_t j) {
  if (e.bias_rank == 0) return 0;
  if (e.bias_rank == 1) return e.bias_shape[0] == 1 ? 0 : j;
  const int64_t r = e.bias_shape[0] == 1 ? 0 : i;
  const int64_t c = e.bias_shape[1] == 1 ? 0 : j;
  return r * e.bias_shape[1] + c;
}

// The reference's epilogue steps with their roundings (src/sim_device.cc:229-241,
// src/runtime.cc:332-344): v = alpha*acc; v = v + beta*bias; relu keeps NaN and -0
// (replaces only v < 0); gelu = (0.5*v) * (1 + erf(v*0.70710678)); then the residual.
__device__ __forceinline__ float ApplyEpilogue(float acc, int64_t i, int64_t j, int64_t n, const Epilogue& e) {
  float v = __fmul_rn(e.alpha, acc);
  if (e.bias != nullptr) v = __fadd_rn(v, __fmul_rn(e.beta, e.bias[BiasIndex(e, i, j)]));
  if (e.activation == ACCEL_HIP_ACT_RELU) {
    if (v < 0.f) v = 0.f;
  } else if (e.activation == ACCEL_HIP_ACT_GELU) {
    const float half = __fmul_rn(0.5f, v);
    const float arg = __fmul_rn(v, 0.7071067811865476f);
    v = __fmul_rn(half, __fadd_rn(1.f, erff(arg)));
  }
  if (e.residual != nullptr) v = __fadd_rn(v, e.residual[i * n + j]);
  return v;
}

// Stores output element (i, j) of an [m, n] product, following the epilogue's column split.
__device__ __forceinline__ void StoreC(float* c, int64_t i, int64_t j, int64_t n, const Epilogue& e, float v) {
  if (e.split[0] == 0) {
    c[i * n + j] = v;
  } else if (j < e.split[0]) {
    c[i * e.split[0] + j] = v;
  } else if (j < e.split[1]) {
    e.c2[i * (e.split[1] - e.split[0]) + (j - e.split[0])] = v;
  } else {
    e.c3[i * (n - e.split[1]) + (j - e.split[1])] = v;
  }
}

// Signed byte b of a dword to float, exact.
__device__ __forceinline__ float ByteToFloat(uint32_t word, int b) {
  return static_cast<float>(static_cast<int32_t>(word << (24 - 8 * b)) >> 24);
}

}  // namespace accel_hip
