// Causal grouped-query attention (SimAttend, src/sim_attend.cc:9-46): query s sees keys
// 0..position+s, head h reads kv head h / (heads / kv_heads), scores = (q . k) / sqrt(head_dim),
// softmax with the max subtracted, out[d] = sum_t (p_t / sum) * v[t][d].
//
// For a prompt (seq > 4), one 512-thread workgroup per (query row, head) holds all of that
// row's scores in LDS. For a decode step the positions are split over workgroups
// (AttentionChunkKernel + AttentionCombineKernel below).
//
// Each dot product runs over d in order with separately rounded products, as the
// reference does, so scores match it bit for bit; exp, the softmax sums and the weighted
// sums (interleaved partial sums combined in a fixed order) differ from the reference's
// sequential loops only by rounding.
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
  __shared__ float acc_part[kThreads * 4];  // [group][column]: groups * head_dim <= 4 * kThreads

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
  local_max = WaveButterfly(local_max, [](float a, float b) { return fmaxf(a, b); });
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
  local_sum = WaveButterfly(local_sum, [](float a, float b) { return __fadd_rn(a, b); });
  if ((tid & 63) == 0) red[tid >> 6] = local_sum;
  __syncthreads();
  float sum = red[0];
  for (int w = 1; w < kThreads / 64; ++w) sum = __fadd_rn(sum, red[w]);
  // p_t = e_t / sum once per position (the reference forms the same quotient for every d).
  for (int64_t t = tid; t < total; t += kThreads) scores[t] = __fdiv_rn(scores[t], sum);
  __syncthreads();

  // out[d] = sum_t p_t * v[t][d]. Thread (g, c) adds t = g, g + G, ... (G groups) for the
  // columns of chunk c (4 columns, one 16-byte load, when kVec > 0; else 1 column); then the G
  // partial sums of each column are added in group order.
  constexpr int kCols = kVec > 0 ? 4 : 1;
  const int64_t chunks = head_dim / kCols;
  const int64_t groups = kThreads / chunks;
  const int64_t c = tid % chunks;
  const int64_t g = tid / chunks;
  float acc[kCols];
#pragma unroll
  for (int j = 0; j < kCols; ++j) acc[j] = 0.f;
  if (g < groups) {
    const float* vcol = v + kv * head_dim + c * kCols;
    const int64_t vstride = kv_heads * head_dim;
    auto load = [&](int64_t t, float (&x)[kCols]) {
      if (kVec > 0) {
        const float4 q4 = *reinterpret_cast<const float4*>(vcol + t * vstride);
        x[0] = q4.x;
        x[1 % kCols] = q4.y;
        x[2 % kCols] = q4.z;
        x[3 % kCols] = q4.w;
      } else {
        x[0] = vcol[t * vstride];
      }
    };
    int64_t t = g;
    for (; t + 3 * groups < total; t += 4 * groups) {
      float x0[kCols], x1[kCols], x2[kCols], x3[kCols];
      load(t, x0);
      load(t + groups, x1);
      load(t + 2 * groups, x2);
      load(t + 3 * groups, x3);
#pragma unroll
      for (int j = 0; j < kCols; ++j) {
        acc[j] = __fadd_rn(acc[j], __fmul_rn(scores[t], x0[j]));
        acc[j] = __fadd_rn(acc[j], __fmul_rn(scores[t + groups], x1[j]));
        acc[j] = __fadd_rn(acc[j], __fmul_rn(scores[t + 2 * groups], x2[j]));
        acc[j] = __fadd_rn(acc[j], __fmul_rn(scores[t + 3 * groups], x3[j]));
      }
    }
    for (; t < total; t += groups) {
      float x0[kCols];
      load(t, x0);
#pragma unroll
      for (int j = 0; j < kCols; ++j) acc[j] = __fadd_rn(acc[j], __fmul_rn(scores[t], x0[j]));
    }
  }
  // acc_part[g][column]
#pragma unroll
  for (int j = 0; j < kCols; ++j)
    if (g < groups) acc_part[g * head_dim + c * kCols + j] = acc[j];
  __syncthreads();
  if (tid < head_dim) {
    float o = acc_part[tid];
    for (int64_t gg = 1; gg < groups; ++gg) o = __fadd_rn(o, acc_part[gg * head_dim + tid]);
    out[(s * heads + h) * head_dim + tid] = o;
  }
}

// ---- decode: positions split over workgroups --------------------------------------------
// A decode step has seq * heads = 9 (query row, head) pairs: one workgroup each would leave
// the GPU idle. Here each pair's positions are cut into 64-position chunks, one workgroup per
// (pair, chunk): it writes the chunk's max score m, l = sum exp(score - m) and the unscaled
// sum acc[d] = sum exp(score - m) * v[t][d]; a second kernel combines the chunks with the
// usual rescaling, out[d] = sum_c e^(m_c - M) acc_c[d] / sum_c e^(m_c - M) l_c. Scores are
// the reference's bits; the softmax differs from its global-max form only by rounding.
constexpr int kChunk = 64;
constexpr int kSplitThreads = 256;

template <int kVec>
__global__ __launch_bounds__(kSplitThreads) void AttentionChunkKernel(const float* q, const float* k, const float* v,
                                                                      int64_t seq, int64_t position_arg,
                                                                      int64_t heads, int64_t kv_heads,
                                                                      int64_t head_dim, int64_t chunks,
                                                                      float* partial, const int32_t* position_dev) {
  __shared__ float qs[256];
  __shared__ float es[kChunk];
  __shared__ float acc_part[kSplitThreads * 4];
  __shared__ float red[2];
  const int64_t position = position_dev != nullptr ? *position_dev : position_arg;
  const int64_t row = blockIdx.x;  // s * heads + h
  const int64_t c = blockIdx.y;
  const int64_t s = row / heads;
  const int64_t h = row % heads;
  const int64_t kv = h / (heads / kv_heads);
  const int64_t total = position + s + 1;
  const int64_t t0 = c * kChunk;
  const int tid = threadIdx.x;
  float* out = partial + (row * chunks + c) * (2 + head_dim);
  if (t0 >= total) {  // nothing in this chunk (the position is read on the device)
    if (tid == 0) {
      out[0] = -INFINITY;
      out[1] = 0.f;
    }
    for (int64_t d = tid; d < head_dim; d += kSplitThreads) out[2 + d] = 0.f;
    return;
  }
  const int64_t n = min<int64_t>(kChunk, total - t0);
  for (int64_t d = tid; d < head_dim; d += kSplitThreads) qs[d] = q[row * head_dim + d];
  __syncthreads();
  const float scale = __fdiv_rn(1.f, __fsqrt_rn(static_cast<float>(head_dim)));
  if (tid < n) es[tid] = __fmul_rn(Dot<kVec>(qs, k + ((t0 + tid) * kv_heads + kv) * head_dim, head_dim), scale);
  __syncthreads();
  if (tid < 64) {  // wave 0: chunk max, exps, their sum
    const float x = tid < n ? es[tid] : -INFINITY;
    float m = x;
    m = WaveButterfly(m, [](float a, float b) { return fmaxf(a, b); });
    const float e = tid < n ? expf(__fsub_rn(x, m)) : 0.f;
    if (tid < n) es[tid] = e;
    float l = e;
    l = WaveButterfly(l, [](float a, float b) { return __fadd_rn(a, b); });
    if (tid == 0) {
      red[0] = m;
      red[1] = l;
    }
  }
  __syncthreads();
  // acc[d] over the chunk: thread (g, col chunk) adds positions g, g + G, ...
  constexpr int kCols = kVec > 0 ? 4 : 1;
  const int64_t col_chunks = head_dim / kCols;
  const int64_t groups = kSplitThreads / col_chunks;
  const int64_t cc = tid % col_chunks;
  const int64_t g = tid / col_chunks;
  float acc[kCols];
#pragma unroll
  for (int j = 0; j < kCols; ++j) acc[j] = 0.f;
  if (g < groups) {
    const float* vcol = v + kv * head_dim + cc * kCols;
    const int64_t vstride = kv_heads * head_dim;
    for (int64_t t = g; t < n; t += groups) {
      const float e = es[t];
      if (kVec > 0) {
        const float4 x4 = *reinterpret_cast<const float4*>(vcol + (t0 + t) * vstride);
        const float xs[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
        for (int j = 0; j < kCols; ++j) acc[j] = __fadd_rn(acc[j], __fmul_rn(e, xs[j]));
      } else {
        acc[0] = __fadd_rn(acc[0], __fmul_rn(e, vcol[(t0 + t) * vstride]));
      }
    }
#pragma unroll
    for (int j = 0; j < kCols; ++j) acc_part[g * head_dim + cc * kCols + j] = acc[j];
  }
  __syncthreads();
  for (int64_t d = tid; d < head_dim; d += kSplitThreads) {
    float o = acc_part[d];
    for (int64_t gg = 1; gg < groups; ++gg) o = __fadd_rn(o, acc_part[gg * head_dim + d]);
    out[2 + d] = o;
  }
  if (tid == 0) {
    out[0] = red[0];
    out[1] = red[1];
  }
}

constexpr int kMaxChunks = 1024;  // kMaxChunks * kChunk positions: 65536

// One workgroup of 64 threads per (query row, head). The chunks' (m, l) pairs are loaded in
// parallel into LDS and turned into weights w_c = e^(m_c - M) (0 for an empty chunk), then
// each thread adds w_c * acc_c[d] over the chunks with its loads issued 8 at a time.
__global__ __launch_bounds__(64) void AttentionCombineKernel(const float* partial, float* out, int64_t chunks,
                                                             int64_t head_dim) {
  __shared__ float wts[kMaxChunks];
  __shared__ float lsum[kMaxChunks];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t stride = 2 + head_dim;
  const float* p = partial + row * chunks * stride;
  float big = -INFINITY;
  for (int64_t c = tid; c < chunks; c += 64) {
    wts[c] = p[c * stride];
    lsum[c] = p[c * stride + 1];
    big = fmaxf(big, wts[c]);
  }
  big = WaveButterfly(big, [](float a, float b) { return fmaxf(a, b); });
  __syncthreads();
  for (int64_t c = tid; c < chunks; c += 64) wts[c] = wts[c] == -INFINITY ? 0.f : expf(__fsub_rn(wts[c], big));
  __syncthreads();
  float l = 0.f;
  for (int64_t c = 0; c < chunks; ++c) l = __fadd_rn(l, __fmul_rn(wts[c], lsum[c]));
  for (int64_t d = tid; d < head_dim; d += 64) {
    float o = 0.f;
    int64_t c = 0;
    for (; c + 8 <= chunks; c += 8) {
      float x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = p[(c + u) * stride + 2 + d];
#pragma unroll
      for (int u = 0; u < 8; ++u) o = __fadd_rn(o, __fmul_rn(wts[c + u], x[u]));
    }
    for (; c < chunks; ++c) o = __fadd_rn(o, __fmul_rn(wts[c], p[c * stride + 2 + d]));
    out[row * head_dim + d] = __fdiv_rn(o, l);
  }
}


// ---- prompt rows, head_dim 64, fast mode: online softmax over key stages ------------------
// One workgroup per (16 query rows, head), in a 1D grid; its eight waves take an eighth of
// the keys each and the eighths are combined at the end. Each wave stages 16 keys of K and V
// in its own LDS slice (coalesced loads; the next stage's loads are issued while the current
// one is multiplied), so K and V are read once per 16 query rows instead of once per row. The
// summation order differs from the reference's sequential loops (rounding only), so this
// path serves the fast mode; the per-row kernel above keeps the reference's score bits.
constexpr int kFlashRows = 16;
constexpr int kFlashWaves = 8;
constexpr int kFlashStage = 16;  // keys per LDS stage
constexpr int kFlashDim = 64;

constexpr int kFlashStageLoads = kFlashStage * kFlashDim / 4 / 64;  // 16-byte pieces of K (and of V) per lane
typedef float f4 __attribute__((ext_vector_type(4)));

// Lane l brings float4 (f & 15) of key t0 + (f >> 4), f = i * 64 + l, of K and V; keys past
// the range read key kend - 1 (masked at use).
__device__ __forceinline__ void FlashLoadStage(const float* k, const float* v, int64_t t0, int64_t kend,
                                               int64_t kv_stride, int64_t kv, int lane,
                                               f4 (&kx)[kFlashStageLoads], f4 (&vx)[kFlashStageLoads]) {
#pragma unroll
  for (int i = 0; i < kFlashStageLoads; ++i) {
    const int f = i * 64 + lane;
    const int64_t t = min<int64_t>(t0 + (f >> 4), kend - 1);
    kx[i] = *reinterpret_cast<const f4*>(k + t * kv_stride + kv * kFlashDim + (f & 15) * 4);
    vx[i] = *reinterpret_cast<const f4*>(v + t * kv_stride + kv * kFlashDim + (f & 15) * 4);
  }
}

// Both products run on v_mfma_f32_16x16x4f32. Per stage a wave forms S^T = K Q^T (16 keys x 16
// rows, 16 MFMAs over the 64 dims) and O^T += V^T P^T (64 dims x 16 rows, 16 MFMAs). Lane l
// serves row j = l % 16 and key group g = l / 16: the S^T tile leaves it the scores of keys
// 4g .. 4g + 3 for row j, which is exactly its operand of P^T when the k slot g of step s is
// key 4g + s, and the O^T tiles hold row j too, so the softmax rescale needs no lane exchange.
// A row's max and sum meet over the four key groups through two lane swaps.
constexpr int kMfmaPad = kFlashDim + 4;  // LDS row stride: the 16 key rows fall on distinct banks

typedef float mv4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kFlashWaves * 64) void AttentionFlashMfmaKernel(
    const float* q, const float* k, const float* v, float* out, const int32_t* position_dev, int32_t seq,
    int32_t position_arg, int32_t heads, int32_t kv_heads) {
  __shared__ __align__(16) float ks[kFlashWaves][kFlashStage][kMfmaPad];
  __shared__ __align__(16) float vs[kFlashWaves][kFlashStage][kMfmaPad];
  __shared__ float part_m[kFlashWaves][kFlashRows];
  __shared__ float part_l[kFlashWaves][kFlashRows];
  const int64_t position = position_dev != nullptr ? *position_dev : position_arg;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int j = lane & 15;  // query row of the block
  const int g = lane >> 4;  // key group / dim group
  // Heaviest row blocks first, over all heads: the workgroups beyond one per CU are then the
  // blocks with the fewest keys, and no two long blocks share a CU.
  const int32_t unit = static_cast<int32_t>(blockIdx.x);
  const int32_t qblocks = static_cast<int32_t>(gridDim.x) / heads;
  const int32_t rank = unit / heads;
  const int64_t s0 = static_cast<int64_t>(qblocks - 1 - rank) * kFlashRows;
  const int64_t h = unit - rank * heads;
  const int64_t kv = h / (heads / kv_heads);
  const int64_t row = s0 + j;
  const bool live = row < seq;
  const int64_t last_key = position + (live ? row : -1);  // keys 0 .. last_key (causal)
  const float scale = __fdiv_rn(1.f, __fsqrt_rn(static_cast<float>(kFlashDim)));

  // B operand of S^T: q[row j][16 g + s], s = 0 .. 15.
  float qb[16];
  {
    const float* qrow = q + ((live ? row : 0) * heads + h) * kFlashDim + 16 * g;
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const float4 x = *reinterpret_cast<const float4*>(qrow + i);
      qb[i] = x.x;
      qb[i + 1] = x.y;
      qb[i + 2] = x.z;
      qb[i + 3] = x.w;
    }
  }
  const int64_t nkeys = position + min<int64_t>(s0 + kFlashRows, seq);
  const int64_t per = ((nkeys + kFlashWaves - 1) / kFlashWaves + kFlashStage - 1) / kFlashStage * kFlashStage;
  const int64_t kbeg = min<int64_t>(wave * per, nkeys);
  const int64_t kend = min<int64_t>(kbeg + per, nkeys);
  const int64_t kv_stride = kv_heads * kFlashDim;

  float m = -INFINITY;
  float l = 0.f;  // this lane's share (its key groups) of row j's sum
  mv4 acc_o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc_o[t] = mv4{0.f, 0.f, 0.f, 0.f};

  f4 kx[kFlashStageLoads], vx[kFlashStageLoads];
  if (kbeg < kend) FlashLoadStage(k, v, kbeg, kend, kv_stride, kv, lane, kx, vx);
  for (int64_t t0 = kbeg; t0 < kend; t0 += kFlashStage) {  // uniform across the wave
#pragma unroll
    for (int i = 0; i < kFlashStageLoads; ++i) {
      const int f = i * 64 + lane;
      *reinterpret_cast<f4*>(&ks[wave][f >> 4][(f & 15) * 4]) = kx[i];
      *reinterpret_cast<f4*>(&vs[wave][f >> 4][(f & 15) * 4]) = vx[i];
    }
    if (t0 + kFlashStage < kend) FlashLoadStage(k, v, t0 + kFlashStage, kend, kv_stride, kv, lane, kx, vx);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // S^T[key i][row j]: A = K[key l % 16][16 g + s], B = q[row][16 g + s].
    float kr[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const float4 x = *reinterpret_cast<const float4*>(&ks[wave][j][16 * g + i]);
      kr[i] = x.x;
      kr[i + 1] = x.y;
      kr[i + 2] = x.z;
      kr[i + 3] = x.w;
    }
    mv4 st = mv4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 16; ++s) st = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[s], qb[s], st, 0, 0, 0);
    // Lane (j, g) holds the scores of keys t0 + 4 g + r, r = 0 .. 3, for row j.
    float sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t t = t0 + 4 * g + r;
      sc[r] = (t < kend && t <= last_key) ? __fmul_rn(st[r], scale) : -INFINITY;
      mx = fmaxf(mx, sc[r]);
    }
    mx = fmaxf(mx, XorLane<16>(mx));
    mx = fmaxf(mx, XorLane<32>(mx));
    const float m_new = fmaxf(m, mx);
    const bool none = m_new == -INFINITY;  // nothing of this row so far
    const float corr = (m == -INFINITY || none) ? (none ? 1.f : 0.f) : expf(m - m_new);
    float pr[4];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pr[r] = sc[r] == -INFINITY ? 0.f : expf(sc[r] - m_new);
      psum = psum + pr[r];
    }
    l = l * corr + psum;
    m = none ? m : m_new;
#pragma unroll
    for (int t = 0; t < 4; ++t) acc_o[t] = acc_o[t] * corr;
    // O^T[dim 16 t + i][row j] += V^T[dim][key 4 g + s] P^T[key 4 g + s][row j].
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        acc_o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vs[wave][4 * g + s][16 * t + j], pr[s], acc_o[t], 0, 0, 0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // the stage is read before the next one overwrites it
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // Row j's sum over the four key groups; then the waves' eighths meet in LDS. acc_o[t][r] is
  // O^T[dim 16 t + 4 g + r][row j]; the wave's stage rows hold its 16 x 64 block.
  l = l + XorLane<16>(l);
  l = l + XorLane<32>(l);
  float* part_acc = &ks[wave][0][0];  // [16 rows][kMfmaPad]: this wave's stage, no longer read
  if (g == 0) {
    part_m[wave][j] = m;
    part_l[wave][j] = l;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
    *reinterpret_cast<float4*>(&part_acc[j * kMfmaPad + 16 * t + 4 * g]) =
        make_float4(acc_o[t][0], acc_o[t][1], acc_o[t][2], acc_o[t][3]);
  __syncthreads();
  if (wave == 0 && live) {
    float big = part_m[0][j];
#pragma unroll
    for (int w = 1; w < kFlashWaves; ++w) big = fmaxf(big, part_m[w][j]);
    float wts[kFlashWaves];
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kFlashWaves; ++w) {
      wts[w] = part_m[w][j] == -INFINITY ? 0.f : expf(part_m[w][j] - big);
      total = total + wts[w] * part_l[w][j];
    }
    float* orow = out + (row * heads + h) * kFlashDim;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < kFlashWaves; ++w) {
        const float4 x = *reinterpret_cast<const float4*>(&ks[w][0][0] + j * kMfmaPad + 16 * t + 4 * g);
        o[0] = o[0] + wts[w] * x.x;
        o[1] = o[1] + wts[w] * x.y;
        o[2] = o[2] + wts[w] * x.z;
        o[3] = o[3] + wts[w] * x.w;
      }
      *reinterpret_cast<float4*>(orow + 16 * t + 4 * g) =
          make_float4(o[0] / total, o[1] / total, o[2] / total, o[3] / total);
    }
  }
}

// ---- decode row, head_dim 64: RoPE, KV append, chunked attention and combine in one kernel --
// One workgroup per (head, 64-position chunk), as AttentionChunkKernel, for the single query
// row of a decode step. Each workgroup rotates its head's q itself (RopeAppendKernel's
// arithmetic); the workgroup of the chunk holding the new position rotates the new k, uses
// the new k and v from LDS for that position, and, for the first query head of the kv
// group, stores them into the cache rows. No workgroup reads the cache row being written.
// The chunk's (m, l, acc) go to `partial`; the last workgroup of a head to finish (counted in
// `arrivals[h]`) adds the chunks in chunk order as AttentionCombineKernel does, writes the
// output row and sets the count back to zero for the next launch. Chunks past the position
// exit at once. The scores, the chunk sums and the combine are those of the three-kernel
// path, bit for bit.
constexpr int kStepDim = 64;
constexpr int kStepFastChunks = 16;

__global__ __launch_bounds__(kSplitThreads) void DecodeAttentionKernel(
    const float* q_raw, const float* k_raw, const float* v_raw, float* k_cache, float* v_cache, const float* cos_t,
    const float* sin_t, float* out, int32_t position_arg, const int32_t* position_dev, int32_t group,
    int32_t kv_heads, int32_t chunks_max, float* partial, uint32_t* arrivals) {
  __shared__ __align__(16) float qs[kStepDim];
  __shared__ __align__(16) float knew[kStepDim];
  __shared__ __align__(16) float vnew[kStepDim];
  __shared__ float es[kChunk];
  __shared__ float acc_part[kSplitThreads / (kStepDim / 4) * kStepDim];
  __shared__ float red[2];
  __shared__ float wts[kMaxChunks];
  __shared__ float lsum[kMaxChunks];
  __shared__ int is_last;
  // 32-bit indexes (the launcher checks that the caches and partials fit them): no 64-bit
  // division or multiply stands between the position read and the first loads. The pointer
  // arguments are read in the same round as the position's address (the compiler would read
  // them after the position and the live-chunk test).
  asm volatile("" ::"s"(k_cache), "s"(v_cache), "s"(q_raw), "s"(k_raw), "s"(v_raw), "s"(cos_t), "s"(sin_t),
               "s"(position_arg), "s"(group), "s"(kv_heads), "s"(chunks_max));
  const int position = position_dev != nullptr ? *position_dev : position_arg;
  const int h = blockIdx.x;
  const int c = blockIdx.y;
  const int kv = h / group;  // group = heads / kv_heads
  const int total = position + 1;
  const int live = (total + kChunk - 1) / kChunk;
  if (c >= live) return;  // uniform over the workgroup
  const int t0 = c * kChunk;
  const int n = min(kChunk, total - t0);
  const bool tail = t0 + n == total;  // this chunk holds the new position
  const int tid = threadIdx.x;
  const int kv_row = kv_heads * kStepDim;

  // The rotation's inputs are loaded first (every thread, from valid addresses), then the key
  // row of this lane (wave 0) and the value rows of this thread's (position group, column
  // quad). Loads complete in issue order; the rotation runs in waves 1 and 2, which load no
  // key rows, so it waits only for its own values and the four value rows, not for the keys.
  constexpr int kHalf = kStepDim / 2;
  const int ri = tid % kHalf;
  const bool rot_q = (tid >> 5) == 2;  // tid 64 .. 95: q; 96 .. 127: the new k
  const float* rsrc = rot_q ? q_raw + h * kStepDim : k_raw + kv * kStepDim;
  const float rx0 = rsrc[ri];
  const float rx1 = rsrc[kHalf + ri];
  const float rc0 = cos_t[position * kStepDim + ri];
  const float rc1 = cos_t[position * kStepDim + kHalf + ri];
  const float rs0 = sin_t[position * kStepDim + ri];
  const float rs1 = sin_t[position * kStepDim + kHalf + ri];
  const float rv = v_raw[kv * kStepDim + (tid & (kStepDim - 1))];
  constexpr int kCols = 4;
  constexpr int kGroups = kSplitThreads / (kStepDim / kCols);  // 16
  const int cc = tid % (kStepDim / kCols);
  const int g = tid / (kStepDim / kCols);
  float4 kx[kStepDim / 4];
  const bool score_lane = tid < n && t0 + tid != position;
  if (score_lane) {
    const float4* kr = reinterpret_cast<const float4*>(k_cache + (t0 + tid) * kv_row + kv * kStepDim);
#pragma unroll
    for (int j = 0; j < kStepDim / 4; ++j) kx[j] = kr[j];
  }
  // Value rows past the chunk's end read its last row and the new position reads the stale
  // cache row: both are replaced at use, so the loads need no branches.
  float4 vx[kChunk / kGroups];
#pragma unroll
  for (int i = 0; i < kChunk / kGroups; ++i) {
    const int t = min(g + i * kGroups, n - 1);
    vx[i] = *reinterpret_cast<const float4*>(v_cache + (t0 + t) * kv_row + kv * kStepDim + cc * kCols);
  }

  // RoPE (RopeAppendKernel's arithmetic) of q, and in the tail chunk of the new k; new v.
  if (rot_q || (tail && (tid >> 5) == 3)) {
    float* dst = rot_q ? qs : knew;
    dst[ri] = __fsub_rn(__fmul_rn(rx0, rc0), __fmul_rn(rx1, rs0));
    dst[kHalf + ri] = __fadd_rn(__fmul_rn(rx1, rc1), __fmul_rn(rx0, rs1));
  } else if (tail && (tid >> 6) == 2) {
    vnew[tid - 128] = rv;
  }
  __syncthreads();
  if (tail && h == kv * group && tid < kStepDim) {
    k_cache[position * kv_row + kv * kStepDim + tid] = knew[tid];
    v_cache[position * kv_row + kv * kStepDim + tid] = vnew[tid];
  }

  // Scores: d ascending, each product rounded before its add (Dot<16>).
  const float scale = __fdiv_rn(1.f, __fsqrt_rn(static_cast<float>(kStepDim)));
  if (tid < n) {
    if (!score_lane) {
#pragma unroll
      for (int j = 0; j < kStepDim / 4; ++j) kx[j] = reinterpret_cast<const float4*>(knew)[j];
    }
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < kStepDim / 4; ++j) {
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 0], kx[j].x));
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 1], kx[j].y));
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 2], kx[j].z));
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 3], kx[j].w));
    }
    es[tid] = __fmul_rn(dot, scale);
  }
  __syncthreads();
  if (tid < 64) {  // wave 0: chunk max, exps, their sum
    const float x = tid < n ? es[tid] : -INFINITY;
    float m = x;
    m = WaveButterfly(m, [](float a, float b) { return fmaxf(a, b); });
    const float e = tid < n ? expf(__fsub_rn(x, m)) : 0.f;
    if (tid < n) es[tid] = e;
    float l = e;
    l = WaveButterfly(l, [](float a, float b) { return __fadd_rn(a, b); });
    if (tid == 0) {
      red[0] = m;
      red[1] = l;
    }
  }
  __syncthreads();
  // acc[d] over the chunk: thread (g, cc) adds positions g, g + 16, ... in order.
  // Branch-free: a position past n adds e * x = 0 * 0, which leaves the sum's bits unchanged
  // (the sum starts at +0 and never becomes -0).
  float acc[kCols] = {0.f, 0.f, 0.f, 0.f};
  const float4 vn4 = reinterpret_cast<const float4*>(vnew)[cc];
  float ev[kChunk / kGroups];
#pragma unroll
  for (int i = 0; i < kChunk / kGroups; ++i) ev[i] = es[min(g + i * kGroups, kChunk - 1)];
#pragma unroll
  for (int i = 0; i < kChunk / kGroups; ++i) {
    const int t = g + i * kGroups;
    const bool in = t < n;
    const bool fresh = t0 + t == position;
    const float e = in ? ev[i] : 0.f;
    const float x0 = in ? (fresh ? vn4.x : vx[i].x) : 0.f;
    const float x1 = in ? (fresh ? vn4.y : vx[i].y) : 0.f;
    const float x2 = in ? (fresh ? vn4.z : vx[i].z) : 0.f;
    const float x3 = in ? (fresh ? vn4.w : vx[i].w) : 0.f;
    acc[0] = __fadd_rn(acc[0], __fmul_rn(e, x0));
    acc[1] = __fadd_rn(acc[1], __fmul_rn(e, x1));
    acc[2] = __fadd_rn(acc[2], __fmul_rn(e, x2));
    acc[3] = __fadd_rn(acc[3], __fmul_rn(e, x3));
  }
#pragma unroll
  for (int j = 0; j < kCols; ++j) acc_part[g * kStepDim + cc * kCols + j] = acc[j];
  __syncthreads();
  // The chunk's partial goes out with device-scope (agent) stores, which are written through
  // to the level every XCD reads; each thread waits until its stores are done before the
  // barrier, and only then is the chunk counted. The workgroup that brings the count to
  // `live` reads the partials with device-scope loads. No cache-wide writeback or
  // invalidate is needed for these few hundred bytes.
  float* mine = partial + (h * chunks_max + c) * (2 + kStepDim);
  if (tid < kStepDim) {
    float o = acc_part[tid];
    for (int gg = 1; gg < kGroups; ++gg) o = __fadd_rn(o, acc_part[gg * kStepDim + tid]);
    __hip_atomic_store(&mine[2 + tid], o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (tid == 0) {
    __hip_atomic_store(&mine[0], red[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&mine[1], red[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) is_last = atomicAdd(&arrivals[h], 1u) == static_cast<uint32_t>(live - 1);
  __syncthreads();
  if (!is_last) return;
  const float* p = partial + h * chunks_max * (2 + kStepDim);
  const auto load = [](const float* x) { return __hip_atomic_load(x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
  if (live <= kStepFastChunks) {
    // Up to 16 chunks (1024 positions): wave 0 issues every load of the combine at once (lane
    // c: chunk c's m and l; lane d: column d of each chunk), then combines: one memory round
    // trip instead of one for (m, l) and more for the columns. Same arithmetic and order.
    if (tid < 64) {
      const int chl = min(tid, live - 1);
      float mc = load(&p[chl * (2 + kStepDim)]);
      const float lc = load(&p[chl * (2 + kStepDim) + 1]);
      float xs[kStepFastChunks];
#pragma unroll
      for (int ch = 0; ch < kStepFastChunks; ++ch) xs[ch] = load(&p[min(ch, live - 1) * (2 + kStepDim) + 2 + tid]);
      if (tid >= live) mc = -INFINITY;
      const float big = WaveButterfly(mc, [](float a, float b) { return fmaxf(a, b); });
      wts[tid] = mc == -INFINITY ? 0.f : expf(__fsub_rn(mc, big));
      lsum[tid] = lc;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float l = 0.f;
      float o = 0.f;
#pragma unroll
      for (int ch = 0; ch < kStepFastChunks; ++ch) {
        if (ch < live) {
          l = __fadd_rn(l, __fmul_rn(wts[ch], lsum[ch]));
          o = __fadd_rn(o, __fmul_rn(wts[ch], xs[ch]));
        }
      }
      out[h * kStepDim + tid] = __fdiv_rn(o, l);
      if (tid == 0) atomicExch(&arrivals[h], 0u);
    }
    return;
  }
  if (tid < 64) {
    float big = -INFINITY;
    for (int ch = tid; ch < live; ch += 64) {
      wts[ch] = load(&p[ch * (2 + kStepDim)]);
      lsum[ch] = load(&p[ch * (2 + kStepDim) + 1]);
      big = fmaxf(big, wts[ch]);
    }
    big = WaveButterfly(big, [](float a, float b) { return fmaxf(a, b); });
    for (int ch = tid; ch < live; ch += 64) wts[ch] = wts[ch] == -INFINITY ? 0.f : expf(__fsub_rn(wts[ch], big));
  }
  __syncthreads();
  if (tid < kStepDim) {
    float l = 0.f;
    for (int ch = 0; ch < live; ++ch) l = __fadd_rn(l, __fmul_rn(wts[ch], lsum[ch]));
    float o = 0.f;
    int ch = 0;
    for (; ch + 8 <= live; ch += 8) {
      float x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = load(&p[(ch + u) * (2 + kStepDim) + 2 + tid]);
#pragma unroll
      for (int u = 0; u < 8; ++u) o = __fadd_rn(o, __fmul_rn(wts[ch + u], x[u]));
    }
    for (; ch < live; ++ch) o = __fadd_rn(o, __fmul_rn(wts[ch], load(&p[ch * (2 + kStepDim) + 2 + tid])));
    out[h * kStepDim + tid] = __fdiv_rn(o, l);
  }
  if (tid == 0) atomicExch(&arrivals[h], 0u);
}

// ---- decode row, head_dim 64, fast mode: a fixed number of splits, combined by the consumer --
// One workgroup per (head, split). The position range [0, position] is cut into `splits`
// contiguous ranges of ceil((position + 1) / splits) positions (at most 256: one key row per
// thread, one memory round after the position arrives). Each workgroup rotates its head's q,
// and the one holding the new position rotates the new k, uses the new k and v from LDS for
// it and, for the first query head of the kv group, stores them into the cache rows, as
// DecodeAttentionKernel does. It writes its split's (max m, sum l, acc[64]) to `partial`
// [heads][splits][2 + 64] and stops there: no arrival count, no combine. A split with no
// positions writes m = -inf, l = 0, acc = 0. The reader combines the splits in split order:
// w_s = e^(m_s - max m) (0 for m_s = -inf), out = sum_s w_s acc_s / sum_s w_s l_s
// (StageInputRow's attention prologue of the int8 GEMV). The scores keep the reference's dot
// order; the softmax sums run in another order (rounding only), so this is a fast-mode path.
constexpr int kDecodeSplitThreads = 256;
constexpr int kDecodeSplitRows = kDecodeSplitThreads;  // positions per split at most
constexpr int kDecodeSplitMin = 8;  // the GEMV prologue reads the first 8 splits unconditionally
constexpr int kDecodeSplitMax = 64;
static_assert(kDecodeSplitMaxBytesPerHead == kDecodeSplitMax * (2 + kStepDim) * sizeof(float), "partial room");

// The position's pointer, the sizes and the key/value cache and q/k pointers lead the arguments:
// the first 14 dwords are preloaded into SGPRs at wave launch, so the position load issues at
// once and every load that depends on it right after; the others are read in its shadow.
__global__ __launch_bounds__(kDecodeSplitThreads) void DecodeSplitAttentionKernel(
    const int32_t* position_dev, int32_t position_arg, int32_t group, int32_t kv_heads, int32_t splits,
    float* k_cache, float* v_cache, const float* q_raw, const float* k_raw, const float* v_raw, const float* cos_t,
    const float* sin_t, float* partial) {
  constexpr int kWaves = kDecodeSplitThreads / 64;
  constexpr int kCols = 4;
  constexpr int kQuads = kStepDim / kCols;                 // 16 column quads
  constexpr int kGroups = kDecodeSplitThreads / kQuads;    // 16 position groups
  constexpr int kPerGroup = kDecodeSplitRows / kGroups;    // 16 positions per group at most
  __shared__ __align__(16) float qs[kStepDim];
  __shared__ __align__(16) float knew[kStepDim];
  __shared__ __align__(16) float vnew[kStepDim];
  __shared__ float es[kDecodeSplitRows];
  __shared__ float acc_part[kGroups * kStepDim];
  __shared__ float wred[2][kWaves];
  const int position = position_dev != nullptr ? *position_dev : position_arg;
  const int h = blockIdx.x;
  const int sp = blockIdx.y;
  const int kv = h / group;
  const int total = position + 1;
  const int len = (total + splits - 1) / splits;  // <= kDecodeSplitRows (launcher)
  const int t0 = sp * len;
  const int n = min(len, total - t0);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  float* mine = partial + (h * splits + sp) * (2 + kStepDim);
  if (n <= 0) {  // uniform over the workgroup
    if (tid < kStepDim) mine[2 + tid] = 0.f;
    if (tid == 0) {
      mine[0] = -INFINITY;
      mine[1] = 0.f;
    }
    return;
  }
  const bool tail = t0 + n == total;  // this split holds the new position
  const int kv_row = kv_heads * kStepDim;

  // Every load of the workgroup is issued here, in one round: the rotation's inputs, this
  // thread's key row, and the value rows of its (position group, column quad).
  constexpr int kHalf = kStepDim / 2;
  const int ri = tid % kHalf;
  const bool rot_q = (tid >> 5) == 2;  // tid 64 .. 95: q; 96 .. 127: the new k
  const float* rsrc = rot_q ? q_raw + h * kStepDim : k_raw + kv * kStepDim;
  const float rx0 = rsrc[ri];
  const float rx1 = rsrc[kHalf + ri];
  const float rc0 = cos_t[position * kStepDim + ri];
  const float rc1 = cos_t[position * kStepDim + kHalf + ri];
  const float rs0 = sin_t[position * kStepDim + ri];
  const float rs1 = sin_t[position * kStepDim + kHalf + ri];
  const float rv = v_raw[kv * kStepDim + (tid & (kStepDim - 1))];
  const int cq = tid % kQuads;
  const int g = tid / kQuads;
  float4 kx[kStepDim / 4];
  const bool score_lane = tid < n && t0 + tid != position;
  if (score_lane) {
    const float4* kr = reinterpret_cast<const float4*>(k_cache + (t0 + tid) * kv_row + kv * kStepDim);
#pragma unroll
    for (int j = 0; j < kStepDim / 4; ++j) kx[j] = kr[j];
  }
  float4 vx[kPerGroup];
#pragma unroll
  for (int i = 0; i < kPerGroup; ++i) {
    const int t = g + i * kGroups;
    if (t < n) vx[i] = *reinterpret_cast<const float4*>(v_cache + (t0 + t) * kv_row + kv * kStepDim + cq * kCols);
  }

  if (rot_q || (tail && (tid >> 5) == 3)) {
    float* dst = rot_q ? qs : knew;
    dst[ri] = __fsub_rn(__fmul_rn(rx0, rc0), __fmul_rn(rx1, rs0));
    dst[kHalf + ri] = __fadd_rn(__fmul_rn(rx1, rc1), __fmul_rn(rx0, rs1));
  } else if (tail && (tid >> 6) == 2) {
    vnew[tid - 128] = rv;
  }
  __syncthreads();
  if (tail && h == kv * group && tid < kStepDim) {
    k_cache[position * kv_row + kv * kStepDim + tid] = knew[tid];
    v_cache[position * kv_row + kv * kStepDim + tid] = vnew[tid];
  }

  // Scores: d ascending, each product rounded before its add.
  const float scale = __fdiv_rn(1.f, __fsqrt_rn(static_cast<float>(kStepDim)));
  float x = -INFINITY;
  if (tid < n) {
    if (!score_lane) {
#pragma unroll
      for (int j = 0; j < kStepDim / 4; ++j) kx[j] = reinterpret_cast<const float4*>(knew)[j];
    }
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < kStepDim / 4; ++j) {
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 0], kx[j].x));
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 1], kx[j].y));
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 2], kx[j].z));
      dot = __fadd_rn(dot, __fmul_rn(qs[4 * j + 3], kx[j].w));
    }
    x = __fmul_rn(dot, scale);
  }
  // The split's max, then e = exp(x - max) and its sum: waves, then the wave values in order.
  const float wmax = WaveButterfly(x, [](float a, float b) { return fmaxf(a, b); });
  if (lane == 0) wred[0][wave] = wmax;
  __syncthreads();
  float m = wred[0][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) m = fmaxf(m, wred[0][w]);
  const float e = tid < n ? expf(__fsub_rn(x, m)) : 0.f;
  es[tid] = e;
  const float wsum = WaveButterfly(e, [](float a, float b) { return __fadd_rn(a, b); });
  if (lane == 0) wred[1][wave] = wsum;
  __syncthreads();
  // acc[d] over the split: thread (g, cq) adds positions g, g + 16, ... in order.
  float acc[kCols] = {0.f, 0.f, 0.f, 0.f};
  const float4 vn4 = reinterpret_cast<const float4*>(vnew)[cq];
#pragma unroll
  for (int i = 0; i < kPerGroup; ++i) {
    const int t = g + i * kGroups;
    if (t < n) {
      const float ev = es[t];
      const float4 v4 = t0 + t == position ? vn4 : vx[i];
      acc[0] = __fadd_rn(acc[0], __fmul_rn(ev, v4.x));
      acc[1] = __fadd_rn(acc[1], __fmul_rn(ev, v4.y));
      acc[2] = __fadd_rn(acc[2], __fmul_rn(ev, v4.z));
      acc[3] = __fadd_rn(acc[3], __fmul_rn(ev, v4.w));
    }
  }
#pragma unroll
  for (int j = 0; j < kCols; ++j) acc_part[g * kStepDim + cq * kCols + j] = acc[j];
  __syncthreads();
  if (tid < kStepDim) {
    float o = acc_part[tid];
    for (int gg = 1; gg < kGroups; ++gg) o = __fadd_rn(o, acc_part[gg * kStepDim + tid]);
    mine[2 + tid] = o;
  }
  if (tid == 0) {
    float l = wred[1][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) l = __fadd_rn(l, wred[1][w]);
    mine[0] = m;
    mine[1] = l;
  }
}

constexpr int64_t kSplitMaxSeq = 4;

}  // namespace

size_t AttentionWorkBytes(int64_t seq, int64_t heads, int64_t max_position, int64_t head_dim) {
  const int64_t rows = max_position + seq;
  if (seq <= kSplitMaxSeq) {
    const int64_t chunks = (rows + kChunk - 1) / kChunk;
    return static_cast<size_t>(seq * heads * chunks * (2 + head_dim)) * sizeof(float);
  }
  if (rows > kLdsScores) return static_cast<size_t>(seq * heads * rows) * sizeof(float);
  return 0;
}

void LaunchAttention(const float* q, const float* k, const float* v, float* out, int64_t seq, int64_t position,
                     int64_t heads, int64_t kv_heads, int64_t head_dim, hipStream_t stream, const int32_t* position_dev,
                     int64_t max_position, float* work, size_t work_bytes, bool fast) {
  if (seq <= 0 || heads <= 0) return;
  if (head_dim <= 0 || head_dim > 256) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention head_dim must be in 1..256");
  const int64_t blocks = seq * heads;
  if (blocks > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention is too large");
  // With a device position the scratch must fit the largest position it can hold.
  const int64_t top = position_dev != nullptr ? max_position : position;
  const int64_t rows = top + seq;
  const size_t need = AttentionWorkBytes(seq, heads, top, head_dim);
  float* scratch = nullptr;
  if (need > 0) {
    if (work != nullptr) {
      if (work_bytes < need) Fail(ACCEL_HIP_INVALID_ARGUMENT, "attention scratch is too small");
      scratch = work;
    } else {
      scratch = static_cast<float*>(Workspace(need));
    }
  }
  const bool aligned = (reinterpret_cast<uintptr_t>(k) % 16 == 0) && (reinterpret_cast<uintptr_t>(v) % 16 == 0) &&
                       head_dim % 4 == 0;
  const int vec = aligned ? static_cast<int>(head_dim) : 0;
  if (seq <= kSplitMaxSeq) {
    const int64_t chunks = (rows + kChunk - 1) / kChunk;
    if (chunks > kMaxChunks) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention context is too long for a decode step");
    const dim3 grid(static_cast<uint32_t>(blocks), static_cast<uint32_t>(chunks)), block(kSplitThreads);
#define ACCEL_ATTN_CHUNK(V)                                                                                        \
  hipLaunchKernelGGL(AttentionChunkKernel<V>, grid, block, 0, stream, q, k, v, seq, position, heads, kv_heads, \
                     head_dim, chunks, scratch, position_dev)
    switch (vec) {
      case 16: ACCEL_ATTN_CHUNK(4); break;
      case 32: ACCEL_ATTN_CHUNK(8); break;
      case 64: ACCEL_ATTN_CHUNK(16); break;
      case 128: ACCEL_ATTN_CHUNK(32); break;
      default: ACCEL_ATTN_CHUNK(0); break;
    }
#undef ACCEL_ATTN_CHUNK
    Check(hipGetLastError(), "AttentionChunkKernel launch");
    hipLaunchKernelGGL(AttentionCombineKernel, dim3(static_cast<uint32_t>(blocks)), dim3(64), 0, stream, scratch, out,
                       chunks, head_dim);
    Check(hipGetLastError(), "AttentionCombineKernel launch");
    return;
  }
  if (fast && head_dim == kFlashDim && aligned && (reinterpret_cast<uintptr_t>(q) % 16 == 0) &&
      (reinterpret_cast<uintptr_t>(out) % 16 == 0)) {
    const int64_t qblocks = (seq + kFlashRows - 1) / kFlashRows;
    if (qblocks > 0x7fffffff || heads > 65535 || seq > 0x7fffffff || position > 0x7fffffff || kv_heads > 65535)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention is too large");
    if (qblocks * heads > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention is too large");
    hipLaunchKernelGGL(AttentionFlashMfmaKernel, dim3(static_cast<uint32_t>(qblocks * heads)),
                       dim3(kFlashWaves * 64), 0, stream, q, k, v, out, position_dev, static_cast<int32_t>(seq),
                       static_cast<int32_t>(position), static_cast<int32_t>(heads), static_cast<int32_t>(kv_heads));
    Check(hipGetLastError(), "AttentionFlashMfmaKernel launch");
    return;
  }
  float* spill = rows > kLdsScores ? scratch : nullptr;
  const dim3 grid(static_cast<uint32_t>(blocks)), block(kThreads);
#define ACCEL_ATTN(V)                                                                                          \
  hipLaunchKernelGGL(AttentionKernel<V>, grid, block, 0, stream, q, k, v, out, seq, position, heads, kv_heads, \
                     head_dim, spill, rows, position_dev)
  switch (vec) {
    case 16: ACCEL_ATTN(4); break;
    case 32: ACCEL_ATTN(8); break;
    case 64: ACCEL_ATTN(16); break;
    case 128: ACCEL_ATTN(32); break;
    default: ACCEL_ATTN(0); break;
  }
#undef ACCEL_ATTN
  Check(hipGetLastError(), "AttentionKernel launch");
}


bool LaunchDecodeAttention(const float* q, const float* k, const float* v, float* k_cache, float* v_cache,
                           const float* cos_table, const float* sin_table, float* out, int64_t position,
                           int64_t heads, int64_t kv_heads, int64_t head_dim, hipStream_t stream,
                           const int32_t* position_dev, int64_t max_position, float* work, size_t work_bytes,
                           uint32_t* arrivals) {
  if (head_dim != kStepDim || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || arrivals == nullptr ||
      work == nullptr)
    return false;
  const auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!aligned(k_cache) || !aligned(v_cache)) return false;
  const int64_t top = position_dev != nullptr ? max_position : position;
  const int64_t chunks = (top + 1 + kChunk - 1) / kChunk;
  if (chunks > kMaxChunks || heads > 65535 || chunks * kChunk * kv_heads * kStepDim > 0x7fffffff ||
      heads * chunks * (2 + kStepDim) > 0x7fffffff)
    Fail(ACCEL_HIP_INVALID_ARGUMENT, "Attention context is too long for a decode step");
  if (work_bytes < AttentionWorkBytes(1, heads, top, head_dim)) Fail(ACCEL_HIP_INVALID_ARGUMENT, "attention scratch is too small");
  hipLaunchKernelGGL(DecodeAttentionKernel, dim3(static_cast<uint32_t>(heads), static_cast<uint32_t>(chunks)),
                     dim3(kSplitThreads), 0, stream, q, k, v, k_cache, v_cache, cos_table, sin_table, out,
                     static_cast<int32_t>(position), position_dev, static_cast<int32_t>(heads / kv_heads),
                     static_cast<int32_t>(kv_heads), static_cast<int32_t>(chunks), work, arrivals);
  Check(hipGetLastError(), "DecodeAttentionKernel launch");
  return true;
}


int DecodeAttentionSplits(int64_t max_position) {
  // A power of two (the combine's butterflies), at least 8, each split at most 256 positions.
  const int64_t need = (max_position + 1 + kDecodeSplitRows - 1) / kDecodeSplitRows;
  int64_t splits = kDecodeSplitMin;
  while (splits < need) splits *= 2;
  return splits > kDecodeSplitMax ? 0 : static_cast<int>(splits);
}

int LaunchDecodeSplitAttention(const float* q, const float* k, const float* v, float* k_cache, float* v_cache,
                               const float* cos_table, const float* sin_table, int64_t position, int64_t heads,
                               int64_t kv_heads, int64_t head_dim, hipStream_t stream, const int32_t* position_dev,
                               int64_t max_position, float* partial, size_t partial_bytes) {
  if (head_dim != kStepDim || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || partial == nullptr) return 0;
  const auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!aligned(k_cache) || !aligned(v_cache)) return 0;
  const int64_t top = position_dev != nullptr ? max_position : position;
  const int splits = DecodeAttentionSplits(top);
  if (splits == 0 || heads > 65535 || (top + 1) * kv_heads * kStepDim > 0x7fffffff ||
      heads * splits * (2 + kStepDim) > 0x7fffffff)
    return 0;
  if (partial_bytes < static_cast<size_t>(heads * splits * (2 + kStepDim)) * sizeof(float))
    Fail(ACCEL_HIP_INVALID_ARGUMENT, "attention scratch is too small");
  hipLaunchKernelGGL(DecodeSplitAttentionKernel, dim3(static_cast<uint32_t>(heads), static_cast<uint32_t>(splits)),
                     dim3(kDecodeSplitThreads), 0, stream, position_dev, static_cast<int32_t>(position),
                     static_cast<int32_t>(heads / kv_heads), static_cast<int32_t>(kv_heads),
                     static_cast<int32_t>(splits), k_cache, v_cache, q, k, v, cos_table, sin_table, partial);
  Check(hipGetLastError(), "DecodeSplitAttentionKernel launch");
  return splits;
}


}  // namespace accel_hip
