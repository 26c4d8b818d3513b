// Streaming kernels of the device contract: the standalone epilogue, transpose, RMSNorm,
// residual add, SiLU*up, embedding gather, RoPE, fill and the generic int8 dequantizer.
// All HBM-bound; each keeps the reference's per-element rounding steps.
#include "device_common.h"

namespace accel_hip {
namespace {

constexpr int kBlock = 256;

int64_t GridFor(int64_t count, int64_t per_block = kBlock) {
  int64_t g = (count + per_block - 1) / per_block;
  return g < 1 ? 1 : (g > (1ll << 30) ? (1ll << 30) : g);
}

__global__ void FillKernel(float* dst, float value, int64_t count) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    dst[i] = value;
}

// GemmEpilogue in place (src/sim_device.cc:211-245).
__global__ void EpilogueKernel(float* c, int64_t m, int64_t n, Epilogue e) {
  const int64_t total = m * n;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = idx / n;
    const int64_t j = idx - i * n;
    c[idx] = ApplyEpilogue(c[idx], i, j, n, e);
  }
}

// dst[j, i] = src[i, j] through a 32x33 LDS tile.
__global__ void TransposeKernel(const float* src, float* dst, int64_t rows, int64_t cols) {
  __shared__ float tile[32][33];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int tx = threadIdx.x & 31;
  const int ty = threadIdx.x >> 5;  // 0..7
  for (int y = ty; y < 32; y += 8) {
    const int64_t r = r0 + y;
    const int64_t c = c0 + tx;
    if (r < rows && c < cols) tile[y][tx] = src[r * cols + c];
  }
  __syncthreads();
  for (int y = ty; y < 32; y += 8) {
    const int64_t c = c0 + y;   // output row
    const int64_t r = r0 + tx;  // output column
    if (c < cols && r < rows) dst[c * rows + r] = tile[tx][y];
  }
}

// RmsNorm (src/sim_rmsnorm.cc:7-20): sum of squares in double, inv in double,
// y = float(double(x) * inv) * w. One workgroup per row; the double sum is a fixed tree.
__global__ void RmsNormKernel(const float* x, const float* w, float* y, int64_t dim, float eps) {
  __shared__ double partial[kBlock / 64];
  const int64_t row = blockIdx.x;
  const float* in = x + row * dim;
  float* out = y + row * dim;
  double ss = 0.0;
  for (int64_t i = threadIdx.x; i < dim; i += kBlock) {
    const double v = static_cast<double>(in[i]);
    ss += v * v;
  }
  ss = WaveButterfly(ss, [](double a, double b) { return a + b; });
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
  __syncthreads();
  double total = 0.0;
  for (int wv = 0; wv < kBlock / 64; ++wv) total += partial[wv];
  const double inv = 1.0 / sqrt(total / static_cast<double>(dim) + static_cast<double>(eps));
  for (int64_t i = threadIdx.x; i < dim; i += kBlock) {
    const float normed = static_cast<float>(static_cast<double>(in[i]) * inv);
    out[i] = __fmul_rn(normed, w[i]);
  }
}

__global__ void AddKernel(float* dest, const float* extra, int64_t count) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    dest[i] = __fadd_rn(dest[i], extra[i]);
}

// SimSiluMul (src/sim_silu.cc:8-13): (x / (1 + exp(-x))) * up.
__global__ void SiluMulKernel(float* gate, const float* up, int64_t count) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float x = gate[i];
    const float denom = __fadd_rn(1.f, expf(-x));
    gate[i] = __fmul_rn(__fdiv_rn(x, denom), up[i]);
  }
}

// SimEmbed (src/sim_embed.cc:9-20). Float table, or int8 table with a per-row scale
// (value = float(q) * scale[id], the fl(q*s) a float table quantized per row holds).
// The arguments a row's loads depend on come first: the leading 14 dwords are preloaded into
// SGPRs at wave launch, so the id chain (index, id, row) starts without a kernarg round trip.
__global__ void EmbeddingKernel(const int32_t* index_dev, const int32_t* ids, const int8_t* qtable,
                                const float* row_scale, int64_t hidden, int64_t vocab, const float* table, float* out,
                                int32_t* bad) {
  const int64_t s = blockIdx.x;
  const int32_t id = ids[(index_dev != nullptr ? *index_dev : 0) + s];
  if (id < 0 || id >= vocab) {
    if (threadIdx.x == 0) *bad = 1;
    return;
  }
  float* dst = out + s * hidden;
  if (table != nullptr) {
    const float* src = table + static_cast<int64_t>(id) * hidden;
    for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x) dst[i] = src[i];
  } else {
    const int8_t* src = qtable + static_cast<int64_t>(id) * hidden;
    const float sc = row_scale[id];
    for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x) dst[i] = __fmul_rn(static_cast<float>(src[i]), sc);
  }
}

// SimRope (src/sim_rope.cc:5-21): rotate-half at absolute position (position + s).
__global__ void RopeKernel(float* states, const float* cos_t, const float* sin_t, int64_t seq, int64_t heads,
                           int64_t head_dim, int64_t position_arg, const int32_t* position_dev) {
  const int64_t position = position_dev != nullptr ? *position_dev : position_arg;
  const int64_t half = head_dim / 2;
  const int64_t total = seq * heads * half;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = idx % half;
    const int64_t sh = idx / half;  // s * heads + h
    const int64_t s = sh / heads;
    float* row = states + sh * head_dim;
    const float* cs = cos_t + (position + s) * head_dim;
    const float* sn = sin_t + (position + s) * head_dim;
    const float x0 = row[i];
    const float x1 = row[half + i];
    row[i] = __fsub_rn(__fmul_rn(x0, cs[i]), __fmul_rn(x1, sn[i]));
    row[half + i] = __fadd_rn(__fmul_rn(x1, cs[half + i]), __fmul_rn(x0, sn[half + i]));
  }
}

// The reference's Rope(q), Rope(k), AppendCache(k), AppendCache(v) (src/llama_model.cc:222-225)
// as one pass: q and k rotated (rotate-half, same roundings as RopeKernel), the rotated k and
// v written into cache rows [position, position + seq). q is rotated in place; k and v are
// only read.
__global__ void RopeAppendKernel(float* q, const float* k, const float* v, float* k_cache, float* v_cache,
                                 const float* cos_t, const float* sin_t, int64_t seq, int64_t heads,
                                 int64_t kv_heads, int64_t head_dim, int64_t position_arg,
                                 const int32_t* position_dev) {
  const int64_t position = position_dev != nullptr ? *position_dev : position_arg;
  const int64_t half = head_dim / 2;
  const int64_t q_pairs = seq * heads * half;
  const int64_t k_pairs = seq * kv_heads * half;
  const int64_t v_elems = seq * kv_heads * head_dim;
  const int64_t total = q_pairs + k_pairs + v_elems;
  const int64_t kv_row = kv_heads * head_dim;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (idx < q_pairs + k_pairs) {
      const bool is_q = idx < q_pairs;
      const int64_t e = is_q ? idx : idx - q_pairs;
      const int64_t nh = is_q ? heads : kv_heads;
      const int64_t i = e % half;
      const int64_t sh = e / half;  // s * nh + h
      const int64_t s = sh / nh;
      const float* cs = cos_t + (position + s) * head_dim;
      const float* sn = sin_t + (position + s) * head_dim;
      const float* src = (is_q ? q : k) + sh * head_dim;
      const float x0 = src[i];
      const float x1 = src[half + i];
      const float y0 = __fsub_rn(__fmul_rn(x0, cs[i]), __fmul_rn(x1, sn[i]));
      const float y1 = __fadd_rn(__fmul_rn(x1, cs[half + i]), __fmul_rn(x0, sn[half + i]));
      if (is_q) {
        q[sh * head_dim + i] = y0;
        q[sh * head_dim + half + i] = y1;
      } else {
        float* dst = k_cache + position * kv_row + sh * head_dim;
        dst[i] = y0;
        dst[half + i] = y1;
      }
    } else {
      const int64_t e = idx - q_pairs - k_pairs;
      v_cache[position * kv_row + e] = v[e];
    }
  }
}

// One decode step done: position and produced count both move on by one.
__global__ void AdvanceKernel(int32_t* state) {
  if (threadIdx.x == 0) {
    state[0] = state[0] + 1;
    state[1] = state[1] + 1;
  }
}

// DequantAt (src/sim_device.cc:406-424) for any plane: coordinate (index / stride) % dim.
__global__ void DequantizeKernel(AccelHipQuantPlane plane, int64_t stride, int64_t count, float* out) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t index = plane.offset + i;
    float scale = plane.scale[0];
    float zero = 0.f;
    if (plane.axis >= 0) {
      const int64_t coord = (index / stride) % plane.shape[plane.axis];
      scale = plane.scale[coord];
      if (plane.zero != nullptr) zero = static_cast<float>(plane.zero[coord]);
    } else if (plane.zero != nullptr) {
      zero = static_cast<float>(plane.zero[0]);
    }
    out[i] = __fmul_rn(static_cast<float>(plane.q[index]) - zero, scale);
  }
}

}  // namespace

void LaunchFill(float* dst, float value, int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  hipLaunchKernelGGL(FillKernel, dim3(static_cast<uint32_t>(GridFor(count, kBlock * 4))), dim3(kBlock), 0, stream, dst,
                     value, count);
  Check(hipGetLastError(), "FillKernel launch");
}

void LaunchEpilogueInPlace(float* c, int64_t m, int64_t n, const Epilogue& epi, hipStream_t stream) {
  if (m * n <= 0) return;
  hipLaunchKernelGGL(EpilogueKernel, dim3(static_cast<uint32_t>(GridFor(m * n, kBlock * 4))), dim3(kBlock), 0, stream,
                     c, m, n, epi);
  Check(hipGetLastError(), "EpilogueKernel launch");
}

void LaunchTranspose(const float* src, float* dst, int64_t rows, int64_t cols, hipStream_t stream) {
  if (rows <= 0 || cols <= 0) return;
  const int64_t gx = (cols + 31) / 32;
  const int64_t gy = (rows + 31) / 32;
  if (gx > 0x7fffffff || gy > 65535) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Transpose is too large");
  hipLaunchKernelGGL(TransposeKernel, dim3(static_cast<uint32_t>(gx), static_cast<uint32_t>(gy)), dim3(256), 0, stream,
                     src, dst, rows, cols);
  Check(hipGetLastError(), "TransposeKernel launch");
}

void LaunchRmsNormRows(const float* x, const float* weight, float* y, int64_t rows, int64_t dim, float eps,
                       hipStream_t stream) {
  if (rows <= 0 || dim <= 0) return;
  if (rows > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "RmsNorm has too many rows");
  hipLaunchKernelGGL(RmsNormKernel, dim3(static_cast<uint32_t>(rows)), dim3(kBlock), 0, stream, x, weight, y, dim, eps);
  Check(hipGetLastError(), "RmsNormKernel launch");
}

void LaunchResidualAdd(float* dest, const float* extra, int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  hipLaunchKernelGGL(AddKernel, dim3(static_cast<uint32_t>(GridFor(count, kBlock * 4))), dim3(kBlock), 0, stream, dest,
                     extra, count);
  Check(hipGetLastError(), "AddKernel launch");
}

void LaunchSiluMul(float* gate, const float* up, int64_t count, hipStream_t stream) {
  if (count <= 0) return;
  hipLaunchKernelGGL(SiluMulKernel, dim3(static_cast<uint32_t>(GridFor(count, kBlock * 4))), dim3(kBlock), 0, stream,
                     gate, up, count);
  Check(hipGetLastError(), "SiluMulKernel launch");
}

void LaunchEmbedding(const int32_t* ids, const float* table, const int8_t* qtable, const float* row_scale, float* out,
                     int64_t seq, int64_t hidden, int64_t vocab, int32_t* bad, hipStream_t stream,
                     const int32_t* index_dev) {
  if (seq <= 0 || hidden <= 0) return;
  if (seq > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Embedding is too large");
  hipLaunchKernelGGL(EmbeddingKernel, dim3(static_cast<uint32_t>(seq)), dim3(kBlock), 0, stream, index_dev, ids, qtable,
                     row_scale, hidden, vocab, table, out, bad);
  Check(hipGetLastError(), "EmbeddingKernel launch");
}

void LaunchRope(float* states, const float* cos_table, const float* sin_table, int64_t seq, int64_t heads,
                int64_t head_dim, int64_t position, hipStream_t stream, const int32_t* position_dev) {
  const int64_t total = seq * heads * (head_dim / 2);
  if (total <= 0) return;
  hipLaunchKernelGGL(RopeKernel, dim3(static_cast<uint32_t>(GridFor(total))), dim3(kBlock), 0, stream, states,
                     cos_table, sin_table, seq, heads, head_dim, position, position_dev);
  Check(hipGetLastError(), "RopeKernel launch");
}

void LaunchRopeAppend(float* q, const float* k, const float* v, float* k_cache, float* v_cache, const float* cos_table,
                      const float* sin_table, int64_t seq, int64_t heads, int64_t kv_heads, int64_t head_dim,
                      int64_t position, hipStream_t stream, const int32_t* position_dev) {
  const int64_t total = seq * (heads + kv_heads) * (head_dim / 2) + seq * kv_heads * head_dim;
  if (total <= 0) return;
  hipLaunchKernelGGL(RopeAppendKernel, dim3(static_cast<uint32_t>(GridFor(total))), dim3(kBlock), 0, stream, q, k, v,
                     k_cache, v_cache, cos_table, sin_table, seq, heads, kv_heads, head_dim, position, position_dev);
  Check(hipGetLastError(), "RopeAppendKernel launch");
}

void LaunchAdvance(int32_t* state, hipStream_t stream) {
  hipLaunchKernelGGL(AdvanceKernel, dim3(1), dim3(64), 0, stream, state);
  Check(hipGetLastError(), "AdvanceKernel launch");
}

void LaunchCopy(void* dst, const void* src, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return;
  Check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream), "hipMemcpyAsync(D2D)");
}

void LaunchDequantize(const AccelHipQuantPlane& plane, int64_t count, float* out, hipStream_t stream) {
  if (count <= 0) return;
  int64_t stride = 1;
  if (plane.axis >= 0)
    for (int32_t d = plane.rank - 1; d > plane.axis; --d) stride *= plane.shape[d];
  hipLaunchKernelGGL(DequantizeKernel, dim3(static_cast<uint32_t>(GridFor(count, kBlock * 4))), dim3(kBlock), 0,
                     stream, plane, stride, count, out);
  Check(hipGetLastError(), "DequantizeKernel launch");
}

}  // namespace accel_hip
