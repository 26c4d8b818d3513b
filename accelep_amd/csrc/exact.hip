// Exact-order products: C = A @ B with every output summed in k order from zero, each
// product rounded before its add, and an int8 weight dequantized per element as
// w = fl((float(q) - float(z)) * scale). That is the arithmetic of the reference's MatMul
// and MatMulQuantized (src/sim_device.cc:331-369,387-402,541-602: one accumulator per
// output, split multiply-then-add), so the stored bits equal the reference's.
//
// Used when exact products are switched on (accel_hip_set_exact_products): the default
// kernels (MFMA GEMM, VALU GEMV) add in another order and meet the fp32 tolerance, not the
// bits. The parallelism here is across outputs only, since one output's sum is a single
// dependent chain.
//
//  * ExactGemvKernel (m <= 16): one thread per output column holding its m accumulators;
//    W is read row by row (consecutive threads, consecutive columns) and A comes through
//    the scalar path (uniform across the wave).
//  * ExactGemmKernel (m > 16): 64 x 64 output tiles, 256 threads with 4 x 4 accumulators
//    each; A and B (dequantized) are staged in LDS 32 rows of k at a time.
#include "device_common.h"

namespace accel_hip {
namespace {

// Weight element (p, j): fp32 B, or the int8 view dequantized as the reference does.
template <bool kQ8>
__device__ __forceinline__ float WeightAt(const float* b, const Q8View& v, int64_t p, int64_t j, int64_t n) {
  if (!kQ8) return b[p * n + j];
  const float q = static_cast<float>(v.q[p * n + j]);
  int64_t idx = v.const_index;
  if (v.mode == kScalePerCol) idx = j;
  if (v.mode == kScalePerRow) idx = p;
  const float z = v.zero != nullptr ? static_cast<float>(v.zero[idx]) : 0.f;
  return __fmul_rn(__fsub_rn(q, z), v.scale[idx]);
}

constexpr int kGemvThreads = 256;
constexpr int kGemvMaxRows = 16;

template <bool kQ8>
__global__ __launch_bounds__(kGemvThreads) void ExactGemvKernel(const float* a, const float* b, Q8View v, float* c,
                                                                int64_t m, int64_t k, int64_t n, Epilogue epi) {
  const int64_t j = blockIdx.x * static_cast<int64_t>(kGemvThreads) + threadIdx.x;
  if (j >= n) return;
  float acc[kGemvMaxRows];
#pragma unroll
  for (int r = 0; r < kGemvMaxRows; ++r) acc[r] = 0.f;
  for (int64_t p = 0; p < k; ++p) {
    const float w = WeightAt<kQ8>(b, v, p, j, n);
#pragma unroll
    for (int r = 0; r < kGemvMaxRows; ++r)
      if (r < m) acc[r] = __fadd_rn(acc[r], __fmul_rn(a[r * k + p], w));
  }
#pragma unroll
  for (int r = 0; r < kGemvMaxRows; ++r)
    if (r < m) StoreC(c, r, j, n, epi, ApplyEpilogue(acc[r], r, j, n, epi));
}

constexpr int kTile = 64;
constexpr int kSlab = 32;  // rows of k staged per step
constexpr int kGemmThreads = 256;

template <bool kQ8>
__global__ __launch_bounds__(kGemmThreads) void ExactGemmKernel(const float* a, const float* b, Q8View v, float* c,
                                                                int64_t m, int64_t k, int64_t n, Epilogue epi) {
  __shared__ float as[kSlab][kTile + 1];  // as[p][row]
  __shared__ float bs[kSlab][kTile + 1];  // bs[p][col]
  const int tid = threadIdx.x;
  const int tx = tid % 16;  // column group: columns tx + 16*c
  const int ty = tid / 16;  // row group: rows ty + 16*r
  const int64_t row0 = blockIdx.y * static_cast<int64_t>(kTile);
  const int64_t col0 = blockIdx.x * static_cast<int64_t>(kTile);
  float acc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) acc[r][cc] = 0.f;

  for (int64_t k0 = 0; k0 < k; k0 += kSlab) {
    const int depth = static_cast<int>(min<int64_t>(kSlab, k - k0));
    // Stage A[row0 .. +64, k0 .. +depth] and B[k0 .. +depth, col0 .. +64]; cells past the
    // matrix edge are never read below, so they are left as they are.
    for (int idx = tid; idx < kSlab * kTile; idx += kGemmThreads) {
      const int p = idx / kTile;
      const int e = idx % kTile;
      if (p < depth) {
        const int64_t ar = row0 + e;
        if (ar < m) as[p][e] = a[ar * k + k0 + p];
        const int64_t bc = col0 + e;
        if (bc < n) bs[p][e] = WeightAt<kQ8>(b, v, k0 + p, bc, n);
      }
    }
    __syncthreads();
    for (int p = 0; p < depth; ++p) {
      float av[4], bv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) av[r] = as[p][ty + 16 * r];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) bv[cc] = bs[p][tx + 16 * cc];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) acc[r][cc] = __fadd_rn(acc[r][cc], __fmul_rn(av[r], bv[cc]));
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t i = row0 + ty + 16 * r;
    if (i >= m) continue;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int64_t j = col0 + tx + 16 * cc;
      if (j < n) StoreC(c, i, j, n, epi, ApplyEpilogue(acc[r][cc], i, j, n, epi));
    }
  }
}

}  // namespace

void LaunchExactMatmul(const float* a, const float* b, const Q8View& bq, float* c, int64_t m, int64_t k, int64_t n,
                       const Epilogue& epi, hipStream_t stream) {
  const bool q8 = bq.q != nullptr;
  if (m <= kGemvMaxRows) {
    const int64_t blocks = (n + kGemvThreads - 1) / kGemvThreads;
    if (blocks > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "exact GEMV grid too large");
    if (q8) {
      hipLaunchKernelGGL(ExactGemvKernel<true>, dim3(static_cast<uint32_t>(blocks)), dim3(kGemvThreads), 0, stream, a,
                         nullptr, bq, c, m, k, n, epi);
    } else {
      hipLaunchKernelGGL(ExactGemvKernel<false>, dim3(static_cast<uint32_t>(blocks)), dim3(kGemvThreads), 0, stream, a,
                         b, bq, c, m, k, n, epi);
    }
  } else {
    const int64_t gx = (n + kTile - 1) / kTile;
    const int64_t gy = (m + kTile - 1) / kTile;
    if (gx > 0x7fffffff || gy > 65535) Fail(ACCEL_HIP_INVALID_ARGUMENT, "exact GEMM grid too large");
    const dim3 grid(static_cast<uint32_t>(gx), static_cast<uint32_t>(gy));
    if (q8) {
      hipLaunchKernelGGL(ExactGemmKernel<true>, grid, dim3(kGemmThreads), 0, stream, a, nullptr, bq, c, m, k, n, epi);
    } else {
      hipLaunchKernelGGL(ExactGemmKernel<false>, grid, dim3(kGemmThreads), 0, stream, a, b, bq, c, m, k, n, epi);
    }
  }
  Check(hipGetLastError(), "exact matmul launch");
}

}  // namespace accel_hip
