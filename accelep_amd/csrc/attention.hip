// Causal grouped-query attention (SimAttend, src/sim_attend.cc:9-46). One workgroup per
// (query row, head): query s sees keys 0..position+s, head h reads kv head
// h / (heads / kv_heads), scores = (q . k) * (1 / sqrt(head_dim)), softmax with the max
// subtracted, out[d] = sum_t (p_t / sum) * v[t][d].
//
// Each dot product runs over d in order with separately rounded products, as the
// reference does, so scores match it bit for bit; exp, the softmax sum (a fixed tree) and
// the weighted sum (4 interleaved partial sums per d, combined in order) differ from the
// reference's sequential loops only by rounding.
#include "device_common.h"

namespace accel_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kLdsScores = 16384;

__global__ __launch_bounds__(kThreads) void AttentionKernel(const float* q, const float* k, const float* v, float* out,
                                                            int64_t seq, int64_t position, int64_t heads,
                                                            int64_t kv_heads, int64_t head_dim, float* spill) {
  __shared__ float lds_scores[kLdsScores];
  __shared__ float qs[256];
  __shared__ float red[kThreads / 64];
  __shared__ float acc_part[kThreads];

  const int64_t s = blockIdx.x / heads;
  const int64_t h = blockIdx.x % heads;
  const int64_t kv = h / (heads / kv_heads);
  const int64_t total = position + s + 1;
  float* scores = total <= kLdsScores ? lds_scores : spill + static_cast<int64_t>(blockIdx.x) * (position + seq);
  const int tid = threadIdx.x;
  const float* qrow = q + (s * heads + h) * head_dim;
  for (int64_t d = tid; d < head_dim; d += kThreads) qs[d] = qrow[d];
  __syncthreads();
  const float scale = __fdiv_rn(1.f, __fsqrt_rn(static_cast<float>(head_dim)));

  float local_max = -INFINITY;
  for (int64_t t = tid; t < total; t += kThreads) {
    const float* krow = k + (t * kv_heads + kv) * head_dim;
    float dot = 0.f;
    for (int64_t d = 0; d < head_dim; ++d) dot = __fadd_rn(dot, __fmul_rn(qs[d], krow[d]));
    const float sc = __fmul_rn(dot, scale);
    scores[t] = sc;
    local_max = fmaxf(local_max, sc);
  }
  for (int off = 32; off > 0; off >>= 1) local_max = fmaxf(local_max, __shfl_xor(local_max, off));
  if ((tid & 63) == 0) red[tid >> 6] = local_max;
  __syncthreads();
  float top = red[0];
  for (int w = 1; w < kThreads / 64; ++w) top = fmaxf(top, red[w]);
  __syncthreads();

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

  // Thread (g, d): d = tid % head_dim, g = tid / head_dim handles t = g, g + G, ...
  const int64_t groups = kThreads / head_dim;
  const int64_t d = tid % head_dim;
  const int64_t g = tid / head_dim;
  float acc = 0.f;
  if (g < groups) {
    for (int64_t t = g; t < total; t += groups) {
      const float p = __fdiv_rn(scores[t], sum);
      acc = __fadd_rn(acc, __fmul_rn(p, v[(t * kv_heads + kv) * head_dim + d]));
    }
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
                     int64_t heads, int64_t kv_heads, int64_t head_dim, hipStream_t stream) {
  if (seq <= 0 || heads <= 0) return;
  if (head_dim <= 0 || head_dim > 256) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention head_dim must be in 1..256");
  const int64_t blocks = seq * heads;
  if (blocks > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention is too large");
  float* spill = nullptr;
  if (position + seq > kLdsScores) {
    Context& ctx = Scratch(static_cast<size_t>(blocks * (position + seq)) * sizeof(float));
    spill = static_cast<float*>(ctx.workspace);
  }
  hipLaunchKernelGGL(AttentionKernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream, q, k, v, out,
                     seq, position, heads, kv_heads, head_dim, spill);
  Check(hipGetLastError(), "AttentionKernel launch");
}

}  // namespace accel_hip
