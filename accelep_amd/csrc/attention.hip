// Causal grouped-query attention (SimAttend, src/sim_attend.cc:9-46). One workgroup per
// (query row, head): query s sees keys 0..position+s, head h reads kv head
// h / (heads / kv_heads), scores = (q . k) * (1 / sqrt(head_dim)), softmax with the max
// subtracted, out[d] = sum_t (p_t / sum) * v[t][d].
//
// Each dot product runs over d in order with separately rounded products, as the
// reference does, so scores match it bit for bit; exp, the softmax sum (a fixed tree) and
// the weighted sum (8 interleaved partial sums per d at head_dim 64, combined in order)
// differ from the reference's sequential loops only by rounding. 512 threads per (query
// row, head): a decode step has few such rows, so each spreads over a whole CU.
#include "device_common.h"

namespace accel_hip {
namespace {

constexpr int kThreads = 512;
constexpr int kLdsScores = 16384;

// q . k for one key row in the reference's order (d ascending, each product rounded before
// its add). kVec > 0: the row is 16-byte aligned and head_dim == 4 * kVec, so it is loaded as
// kVec 16-byte pieces before the sum starts (one memory round trip per row, not head_dim).
template <int kVec>
__device__ __forceinline__ float Dot(const float* qs, const float* krow, int64_t head_dim) {
  float dot = 0.f;
  if (kVec > 0) {
    float4 x[kVec > 0 ? kVec : 1];
#pragma unroll
    for (int j = 0; j < kVec; ++j) x[j] = reinterpret_cast<const float4*>(krow)[j];
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 0], x[j].x));
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 1], x[j].y));
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 2], x[j].z));
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 3], x[j].w));
    }
  } else {
    for (int64_t d = 0; d < head_dim; ++d) dot = __fadd_rn(dot, __fmul_rn(qs[d], krow[d]));
  }
  return dot;
}

template <int kVec>
__global__ __launch_bounds__(kThreads) void AttentionKernel(const float* q, const float* k, const float* v, float* out,
                                                            int64_t seq, int64_t position_arg, int64_t heads,
                                                            int64_t kv_heads, int64_t head_dim, float* spill,
                                                            int64_t spill_rows, const int32_t* position_dev) {
  const int64_t position = position_dev != nullptr ? *position_dev : position_arg;
  __shared__ float lds_scores[kLdsScores];
  __shared__ float qs[256];
  __shared__ float red[kThreads / 64];
  __shared__ float acc_part[kThreads];

  const int64_t s = blockIdx.x / heads;
  const int64_t h = blockIdx.x % heads;
  const int64_t kv = h / (heads / kv_heads);
  const int64_t total = position + s + 1;
  float* scores = spill == nullptr ? lds_scores : spill + static_cast<int64_t>(blockIdx.x) * spill_rows;
  const int tid = threadIdx.x;
  const float* qrow = q + (s * heads + h) * head_dim;
  for (int64_t d = tid; d < head_dim; d += kThreads) qs[d] = qrow[d];
  __syncthreads();
  const float scale = __fdiv_rn(1.f, __fsqrt_rn(static_cast<float>(head_dim)));

  // Scores (bit for bit the reference's), then the max.
  float local_max = -INFINITY;
  for (int64_t t = tid; t < total; t += kThreads) {
    const float sc = __fmul_rn(Dot<kVec>(qs, k + (t * kv_heads + kv) * head_dim, head_dim), scale);
    scores[t] = sc;
    local_max = fmaxf(local_max, sc);
  }
  for (int off = 32; off > 0; off >>= 1) local_max = fmaxf(local_max, __shfl_xor(local_max, off));
  if ((tid & 63) == 0) red[tid >> 6] = local_max;
  __syncthreads();
  float top = red[0];
  for (int w = 1; w < kThreads / 64; ++w) top = fmaxf(top, red[w]);
  __syncthreads();

  // exp(score - max) and their sum (each thread's terms in order, then a fixed tree).
  float local_sum = 0.f;
  for (int64_t t = tid; t < total; t += kThreads) {
    const float e = expf(__fsub_rn(scores[t], top));
    scores[t] = e;
    local_sum = __fadd_rn(local_sum, e);
  }
  for (int off = 32; off > 0; off >>= 1) local_sum = __fadd_rn(local_sum, __shfl_xor(local_sum, off));
  if ((tid & 63) == 0) red[tid >> 6] = local_sum;
  __syncthreads();
  float sum = red[0];
  for (int w = 1; w < kThreads / 64; ++w) sum = __fadd_rn(sum, red[w]);
  // p_t = e_t / sum once per position (the reference forms the same quotient for every d).
  for (int64_t t = tid; t < total; t += kThreads) scores[t] = __fdiv_rn(scores[t], sum);
  __syncthreads();

  // out[d] = sum_t p_t * v[t][d]: thread (g, d) adds t = g, g + G, ... (G groups), then
  // the G partial sums are added in group order.
  const int64_t groups = kThreads / head_dim;
  const int64_t d = tid % head_dim;
  const int64_t g = tid / head_dim;
  float acc = 0.f;
  if (g < groups) {
    const float* vcol = v + kv * head_dim + d;
    const int64_t vstride = kv_heads * head_dim;
    int64_t t = g;
    for (; t + 3 * groups < total; t += 4 * groups) {
      const float v0 = vcol[t * vstride];
      const float v1 = vcol[(t + groups) * vstride];
      const float v2 = vcol[(t + 2 * groups) * vstride];
      const float v3 = vcol[(t + 3 * groups) * vstride];
      acc = __fadd_rn(acc, __fmul_rn(scores[t], v0));
      acc = __fadd_rn(acc, __fmul_rn(scores[t + groups], v1));
      acc = __fadd_rn(acc, __fmul_rn(scores[t + 2 * groups], v2));
      acc = __fadd_rn(acc, __fmul_rn(scores[t + 3 * groups], v3));
    }
    for (; t < total; t += groups) acc = __fadd_rn(acc, __fmul_rn(scores[t], vcol[t * vstride]));
  }
  acc_part[tid] = acc;
  __syncthreads();
  if (tid < head_dim) {
    float o = acc_part[tid];
    for (int64_t gg = 1; gg < groups; ++gg) o = __fadd_rn(o, acc_part[gg * head_dim + tid]);
    out[(s * heads + h) * head_dim + tid] = o;
  }
}

}  // namespace

void LaunchAttention(const float* q, const float* k, const float* v, float* out, int64_t seq, int64_t position,
                     int64_t heads, int64_t kv_heads, int64_t head_dim, hipStream_t stream, const int32_t* position_dev,
                     int64_t max_position) {
  if (seq <= 0 || heads <= 0) return;
  if (head_dim <= 0 || head_dim > 256) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention head_dim must be in 1..256");
  const int64_t blocks = seq * heads;
  if (blocks > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention is too large");
  // With a device position the scores must fit the largest position it can hold.
  const int64_t rows = (position_dev != nullptr ? max_position : position) + seq;
  float* spill = nullptr;
  if (rows > kLdsScores) {
    Context& ctx = Scratch(static_cast<size_t>(blocks * rows) * sizeof(float));
    spill = static_cast<float*>(ctx.workspace);
  }
  const bool aligned = (reinterpret_cast<uintptr_t>(k) % 16 == 0) && head_dim % 4 == 0;
  const dim3 grid(static_cast<uint32_t>(blocks)), block(kThreads);
  switch (aligned ? head_dim : 0) {
    case 16:
      hipLaunchKernelGGL(AttentionKernel<4>, grid, block, 0, stream, q, k, v, out, seq, position, heads, kv_heads,
                         head_dim, spill, rows, position_dev);
      break;
    case 32:
      hipLaunchKernelGGL(AttentionKernel<8>, grid, block, 0, stream, q, k, v, out, seq, position, heads, kv_heads,
                         head_dim, spill, rows, position_dev);
      break;
    case 64:
      hipLaunchKernelGGL(AttentionKernel<16>, grid, block, 0, stream, q, k, v, out, seq, position, heads, kv_heads,
                         head_dim, spill, rows, position_dev);
      break;
    case 128:
      hipLaunchKernelGGL(AttentionKernel<32>, grid, block, 0, stream, q, k, v, out, seq, position, heads, kv_heads,
                         head_dim, spill, rows, position_dev);
      break;
    default:
      hipLaunchKernelGGL(AttentionKernel<0>, grid, block, 0, stream, q, k, v, out, seq, position, heads, kv_heads,
                         head_dim, spill, rows, position_dev);
      break;
  }
  Check(hipGetLastError(), "AttentionKernel launch");
}

}  // namespace accel_hip
