// Device-side helpers shared by the kernel files (HIP only).
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace accel_hip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats to one word of two bf16 (round to nearest even), x in the low half.
__device__ __forceinline__ uint32_t PackBf16(float x, float y) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x, y}, bf16x2));
}
// The low / high bf16 of a word as the fp32 value it holds exactly.
__device__ __forceinline__ float Bf16Low(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float Bf16High(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// x = hi + mid + lo for two floats at once, each part a bf16 (round to nearest even):
// hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid). Both differences are exact in fp32,
// and after two roundings to 8 significant bits at most 8 bits of x remain, so lo holds them
// exactly and the three parts carry all 24 significand bits (for finite |x| >= 2^-110 and below
// the bf16 overflow threshold 0x1.fep127), with |mid| about 2^-8 |x| at most and |lo| about
// 2^-16 |x| at most.
__device__ __forceinline__ void SplitBf16Pair(float x0, float x1, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  hi = PackBf16(x0, x1);
  const float r0 = x0 - Bf16Low(hi);
  const float r1 = x1 - Bf16High(hi);
  mid = PackBf16(r0, r1);
  lo = PackBf16(r0 - Bf16Low(mid), r1 - Bf16High(mid));
}

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
// bias_v and res_v are the element's bias and residual values, already loaded (read only
// when the epilogue has a bias or residual).
__device__ __forceinline__ float ApplyEpilogueLoaded(float acc, const Epilogue& e, float bias_v, float res_v) {
  float v = __fmul_rn(e.alpha, acc);
  if (e.bias != nullptr) v = __fadd_rn(v, __fmul_rn(e.beta, bias_v));
  if (e.activation == ACCEL_HIP_ACT_RELU) {
    if (v < 0.f) v = 0.f;
  } else if (e.activation == ACCEL_HIP_ACT_GELU) {
    const float half = __fmul_rn(0.5f, v);
    const float arg = __fmul_rn(v, 0.7071067811865476f);
    v = __fmul_rn(half, __fadd_rn(1.f, erff(arg)));
  }
  if (e.residual != nullptr) v = __fadd_rn(v, res_v);
  return v;
}

__device__ __forceinline__ float ApplyEpilogue(float acc, int64_t i, int64_t j, int64_t n, const Epilogue& e) {
  const float bias_v = e.bias != nullptr ? e.bias[BiasIndex(e, i, j)] : 0.f;
  const float res_v = e.residual != nullptr ? e.residual[i * n + j] : 0.f;
  return ApplyEpilogueLoaded(acc, e, bias_v, res_v);
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

// Lane exchange without LDS: the value of lane l ^ kOff (kOff in 1, 2, 4, 8, 16, 32), as
// __shfl_xor returns it, from VALU lane moves instead of an LDS permute round trip. Across
// wave halves and 16-lane rows, v_permlane32_swap / v_permlane16_swap of x with itself leaves
// the partner half (row) in one of its two results; inside a row, DPP: row_ror:8 is xor 8,
// row_shr:4 into banks 1 and 3 plus row_shl:4 into banks 0 and 2 is xor 4, and quad_perm
// gives xor 2 and xor 1.
template <int kOff>
__device__ __forceinline__ unsigned XorLaneBits(unsigned x) {
  static_assert(kOff == 1 || kOff == 2 || kOff == 4 || kOff == 8 || kOff == 16 || kOff == 32, "lane xor offset");
  if constexpr (kOff == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (__lane_id() & 32) ? r[0] : r[1];
  } else if constexpr (kOff == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (__lane_id() & 16) ? r[0] : r[1];
  } else if constexpr (kOff == 8) {
    return static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x128, 0xf, 0xf, false));
  } else if constexpr (kOff == 4) {
    const int up = __builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x114, 0xf, 0xa, false);
    return static_cast<unsigned>(__builtin_amdgcn_update_dpp(up, static_cast<int>(x), 0x104, 0xf, 0x5, false));
  } else if constexpr (kOff == 2) {
    return static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x4e, 0xf, 0xf, false));
  } else {
    return static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0xb1, 0xf, 0xf, false));
  }
}
template <int kOff, typename T>
__device__ __forceinline__ T XorLane(T x) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "4- or 8-byte lane values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, XorLaneBits<kOff>(__builtin_bit_cast(unsigned, x)));
  } else {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, x);
    const unsigned lo = XorLaneBits<kOff>(static_cast<unsigned>(b));
    const unsigned hi = XorLaneBits<kOff>(static_cast<unsigned>(b >> 32));
    return __builtin_bit_cast(T, (static_cast<unsigned long long>(hi) << 32) | lo);
  }
}
// x = op(x, x of lane l ^ off) for off = 32, 16, 8, 4, 2, 1: the butterfly of a
// `for (off = 32; off > 0; off >>= 1)` loop over __shfl_xor, with the same operands.
template <typename T, typename Op>
__device__ __forceinline__ T WaveButterfly(T x, Op op) {
  x = op(x, XorLane<32>(x));
  x = op(x, XorLane<16>(x));
  x = op(x, XorLane<8>(x));
  x = op(x, XorLane<4>(x));
  x = op(x, XorLane<2>(x));
  return op(x, XorLane<1>(x));
}

// Signed byte b of a dword to float, exact.
// Workgroup barrier that orders LDS only: each wave's LDS reads and writes before it are
// complete and visible to the workgroup after it. Unlike __syncthreads (whose workgroup
// release also waits for the wave's global loads), loads issued for later iterations stay in
// flight across it. For loops whose waves exchange data through LDS alone.
__device__ __forceinline__ void LdsBarrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float ByteToFloat(uint32_t word, int b) {
  return static_cast<float>(static_cast<int32_t>(word << (24 - 8 * b)) >> 24);
}

// An unsigned key whose order is the float order (-0 below +0, NaNs by their bits).
__device__ __forceinline__ uint32_t OrderKey(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// Greedy pick key of value v at id i: OrderKey(v == 0 ? +0 : v) << 32 | (2^32 - 1 - i), and 0
// for a NaN. The largest key is the largest value and, among equal values (-0 equals +0), the
// earliest id; a NaN never wins.
__device__ __forceinline__ uint64_t GreedyKey(float v, uint32_t i) {
  if (isnan(v)) return 0;
  const float c = v == 0.f ? 0.f : v;
  return (static_cast<uint64_t>(OrderKey(c)) << 32) | static_cast<uint64_t>(0xffffffffu - i);
}

__device__ __forceinline__ unsigned FloatBits(float x) { return __builtin_bit_cast(unsigned, x); }
__device__ __forceinline__ float BitsFloat(unsigned x) { return __builtin_bit_cast(float, x); }
// x from lane l ^ 8 (row_ror:8 inside each 16-lane row), l + 7 - 2 (l % 8) (row_half_mirror),
// l ^ 2 and l ^ 1 (quad_perm).
template <int kCtrl>
__device__ __forceinline__ float Dpp(float x) {
  return BitsFloat(static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(FloatBits(x)), kCtrl, 0xf, 0xf,
                                                                     false)));
}
constexpr int kDppRowRor8 = 0x128;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppQuadXor2 = 0x4e;  // quad_perm [2, 3, 0, 1]
constexpr int kDppQuadXor1 = 0xb1;  // quad_perm [1, 0, 3, 2]

// Sums one value per column over the 64 lanes of a wave: three halving exchanges leave lane l
// with column (l >> 3) & 7 summed over its 8-lane group, three more finish the sum. The
// exchanges are VALU lane moves (v_permlane32_swap between wave halves, v_permlane16_swap
// between 16-lane rows, DPP inside a row), not LDS round trips. With A = column i and
// B = column i + 4, the 32-lane swap leaves [A.lo, B.lo] and [A.hi, B.hi], whose sum holds
// column i in the low half and column i + 4 in the high half; the 16-lane swap does the same
// between rows 0/1 and 2/3.
__device__ __forceinline__ float WaveColumnSum8(const float (&v8)[8], int lane) {
  float v4[4], v2[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(FloatBits(v8[i]), FloatBits(v8[i + 4]), false, false);
    v4[i] = BitsFloat(r[0]) + BitsFloat(r[1]);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(FloatBits(v4[i]), FloatBits(v4[i + 2]), false, false);
    v2[i] = BitsFloat(r[0]) + BitsFloat(r[1]);
  }
  const bool h3 = lane & 8;
  float v = (h3 ? v2[1] : v2[0]) + Dpp<kDppRowRor8>(h3 ? v2[0] : v2[1]);
  v = v + Dpp<kDppRowHalfMirror>(v);
  v = v + Dpp<kDppQuadXor2>(v);
  v = v + Dpp<kDppQuadXor1>(v);
  return v;
}

}  // namespace accel_hip
