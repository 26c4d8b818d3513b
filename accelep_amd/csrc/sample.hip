// SampleToken (SimSampleToken, src/sim_sample.cc:25-115) on one workgroup, logits in HBM.
//
//  * temperature <= 0 (or NaN): argmax, the earliest id wins a tie; a NaN at id 0 gives 0,
//    later NaNs never win (the reference's strict > scan).
//  * top_k in (0, vocab): the table holds the min(top_k, 64) largest logits, equal logits
//    resolved toward smaller ids (what the reference's replace-the-worst scan keeps), in
//    id order. The table is found by a radix select on an order-preserving key and an
//    id-ordered compaction; the draw over it then runs on one lane in the reference's
//    order (double exp, cumulative sum, first sum >= draw).
//  * otherwise the whole vocabulary: max, double sum and the cumulative search are block
//    reductions/scans over contiguous id ranges (same result up to double rounding).
// The xorshift32 state is read from and written back to a device word; it advances only
// when a draw happens (sum > 0), as in the reference.
#include "device_common.h"

namespace accel_hip {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ uint32_t XorShift32(uint32_t x) {
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  return x;
}

template <class T>
__device__ T BlockSum(T v, T* scratch) {
  v = WaveButterfly(v, [](T a, T b) { return a + b; });
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  T total = scratch[0];
  for (int w = 1; w < kWaves; ++w) total += scratch[w];
  return total;
}

// Exclusive prefix over threads of a per-thread value (thread order == id order).
template <class T>
__device__ T BlockExclusiveScan(T v, T* scratch, T* total_out) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  T inc = v;
  for (int off = 1; off < 64; off <<= 1) {
    const T other = __shfl_up(inc, off);
    if (lane >= off) inc += other;
  }
  __syncthreads();
  if (lane == 63) scratch[wave] = inc;
  __syncthreads();
  T base = 0;
  for (int w = 0; w < wave; ++w) base += scratch[w];
  T total = 0;
  for (int w = 0; w < kWaves; ++w) total += scratch[w];
  *total_out = total;
  return base + inc - v;
}

struct Best {
  float v;
  int64_t i;  // -1: no candidate
};

__device__ __forceinline__ Best Better(Best a, Best b) {
  if (a.i < 0) return b;
  if (b.i < 0) return a;
  if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
  return a;
}

__device__ Best BlockArgmax(Best b, float* sv, int64_t* si) {
  b = Better(b, Best{XorLane<32>(b.v), XorLane<32>(b.i)});
  b = Better(b, Best{XorLane<16>(b.v), XorLane<16>(b.i)});
  b = Better(b, Best{XorLane<8>(b.v), XorLane<8>(b.i)});
  b = Better(b, Best{XorLane<4>(b.v), XorLane<4>(b.i)});
  b = Better(b, Best{XorLane<2>(b.v), XorLane<2>(b.i)});
  b = Better(b, Best{XorLane<1>(b.v), XorLane<1>(b.i)});
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = b.v;
    si[threadIdx.x >> 6] = b.i;
  }
  __syncthreads();
  Best r{sv[0], si[0]};
  for (int w = 1; w < kWaves; ++w) r = Better(r, Best{sv[w], si[w]});
  return r;
}

__global__ __launch_bounds__(kThreads) void SampleKernel(const float* logits, int32_t* chosen, int64_t vocab,
                                                         float temperature, uint32_t* rng, int32_t top_k,
                                                         const int32_t* index_dev) {
  if (index_dev != nullptr) chosen += *index_dev;  // the slot is read from device memory
  __shared__ float sv[kWaves];
  __shared__ int64_t si[kWaves];
  __shared__ double sd[kWaves];
  __shared__ uint32_t su[kWaves];
  __shared__ int64_t table_id[64];
  __shared__ float table_logit[64];
  const int tid = threadIdx.x;

  if (!(temperature > 0.f)) {
    // Better is a total order (larger value, then smaller id), so the order in which
    // candidates meet does not change the winner. The row is read as 16-byte pieces, twelve
    // in flight per thread: a 49152-id row is one round of loads.
    constexpr int kVec = 12;
    Best b{0.f, -1};
    const int64_t nvec = reinterpret_cast<uintptr_t>(logits) % 16 == 0 ? vocab / 4 : 0;
    const float4* l4 = reinterpret_cast<const float4*>(logits);
    int64_t j = tid;
    for (; j + (kVec - 1) * kThreads < nvec; j += kVec * kThreads) {
      float4 v[kVec];
#pragma unroll
      for (int u = 0; u < kVec; ++u) v[u] = l4[j + u * kThreads];
#pragma unroll
      for (int u = 0; u < kVec; ++u) {
        const int64_t i0 = 4 * (j + u * kThreads);
        if (!isnan(v[u].x)) b = Better(b, Best{v[u].x, i0});
        if (!isnan(v[u].y)) b = Better(b, Best{v[u].y, i0 + 1});
        if (!isnan(v[u].z)) b = Better(b, Best{v[u].z, i0 + 2});
        if (!isnan(v[u].w)) b = Better(b, Best{v[u].w, i0 + 3});
      }
    }
    for (; j < nvec; j += kThreads) {
      const float4 v = l4[j];
      if (!isnan(v.x)) b = Better(b, Best{v.x, 4 * j});
      if (!isnan(v.y)) b = Better(b, Best{v.y, 4 * j + 1});
      if (!isnan(v.z)) b = Better(b, Best{v.z, 4 * j + 2});
      if (!isnan(v.w)) b = Better(b, Best{v.w, 4 * j + 3});
    }
    for (int64_t i = 4 * nvec + tid; i < vocab; i += kThreads) {
      const float v = logits[i];
      if (!isnan(v)) b = Better(b, Best{v, i});
    }
    const Best r = BlockArgmax(b, sv, si);
    if (tid == 0) *chosen = (isnan(logits[0]) || r.i < 0) ? 0 : static_cast<int32_t>(r.i);
    return;
  }

  const bool full = top_k <= 0 || static_cast<int64_t>(top_k) >= vocab;
  const double inv_t = 1.0 / static_cast<double>(temperature);
  // Contiguous id range of this thread.
  const int64_t per = (vocab + kThreads - 1) / kThreads;
  const int64_t lo = min(vocab, static_cast<int64_t>(tid) * per);
  const int64_t hi = min(vocab, lo + per);

  if (!full) {
    const int cap = top_k > 64 ? 64 : top_k;
    // Radix select: the largest key K with count(key >= K) >= cap.
    uint32_t prefix = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = prefix | (1u << bit);
      uint32_t cnt = 0;
      for (int64_t i = lo; i < hi; ++i) {
        const float v = logits[i];
        if (!isnan(v) && OrderKey(v) >= cand) ++cnt;
      }
      if (BlockSum<uint32_t>(cnt, su) >= static_cast<uint32_t>(cap)) prefix = cand;
    }
    uint32_t gt = 0, eq = 0;
    for (int64_t i = lo; i < hi; ++i) {
      const float v = logits[i];
      if (isnan(v)) continue;
      const uint32_t key = OrderKey(v);
      gt += key > prefix;
      eq += key == prefix;
    }
    uint32_t gt_total = 0, eq_total = 0;
    const uint32_t eq_before = BlockExclusiveScan<uint32_t>(eq, su, &eq_total);
    uint32_t dummy = 0;
    const uint32_t gt_all = BlockSum<uint32_t>(gt, su);
    const uint32_t need = static_cast<uint32_t>(cap) - gt_all;
    // Selected in this range: all keys > K, and keys == K whose rank among equals < need.
    uint32_t sel = 0;
    {
      uint32_t rank = eq_before;
      for (int64_t i = lo; i < hi; ++i) {
        const float v = logits[i];
        if (isnan(v)) continue;
        const uint32_t key = OrderKey(v);
        if (key > prefix) ++sel;
        else if (key == prefix) {
          if (rank < need) ++sel;
          ++rank;
        }
      }
    }
    (void)gt_total;
    (void)dummy;
    uint32_t sel_total = 0;
    uint32_t pos = BlockExclusiveScan<uint32_t>(sel, su, &sel_total);
    {
      uint32_t rank = eq_before;
      for (int64_t i = lo; i < hi; ++i) {
        const float v = logits[i];
        if (isnan(v)) continue;
        const uint32_t key = OrderKey(v);
        bool take = key > prefix;
        if (key == prefix) {
          take = rank < need;
          ++rank;
        }
        if (take && pos < 64) {
          table_id[pos] = i;
          table_logit[pos] = v;
          ++pos;
        }
      }
    }
    __syncthreads();
    if (tid == 0) {
      const int filled = static_cast<int>(sel_total < 64 ? sel_total : 64);
      float top = table_logit[0];
      for (int s = 1; s < filled; ++s)
        if (table_logit[s] > top) top = table_logit[s];
      double sum = 0.0;
      for (int s = 0; s < filled; ++s)
        sum += exp((static_cast<double>(table_logit[s]) - static_cast<double>(top)) * inv_t);
      if (!(sum > 0.0)) {
        *chosen = 0;
        return;
      }
      const uint32_t state = XorShift32(*rng);
      *rng = state;
      const double draw = (static_cast<double>(state) + 0.5) / 4294967296.0 * sum;
      double acc = 0.0;
      for (int s = 0; s < filled; ++s) {
        acc += exp((static_cast<double>(table_logit[s]) - static_cast<double>(top)) * inv_t);
        if (acc >= draw) {
          *chosen = static_cast<int32_t>(table_id[s]);
          return;
        }
      }
      *chosen = static_cast<int32_t>(table_id[filled - 1]);
    }
    return;
  }

  // Full vocabulary. Max as the reference's scan: start at logits[0], strict >.
  float local = -INFINITY;
  bool any = false;
  for (int64_t i = lo; i < hi; ++i) {
    const float v = logits[i];
    if (!isnan(v) && (!any || v > local)) {
      local = v;
      any = true;
    }
  }
  Best b{local, any ? 0 : -1};
  const Best mx = BlockArgmax(b, sv, si);
  const float top = isnan(logits[0]) ? logits[0] : mx.v;
  double part = 0.0;
  for (int64_t i = lo; i < hi; ++i) part += exp((static_cast<double>(logits[i]) - static_cast<double>(top)) * inv_t);
  double sum = 0.0;
  const double before = BlockExclusiveScan<double>(part, sd, &sum);
  __shared__ int64_t pick;
  __shared__ uint32_t draw_state;
  __shared__ int drew;
  if (tid == 0) {
    pick = vocab - 1;
    drew = sum > 0.0;
    if (drew) {
      draw_state = XorShift32(*rng);
      *rng = draw_state;
    }
  }
  __syncthreads();
  if (!drew) {
    if (tid == 0) *chosen = 0;
    return;
  }
  const double draw = (static_cast<double>(draw_state) + 0.5) / 4294967296.0 * sum;
  // The first id whose cumulative weight reaches the draw lies in the first range whose
  // end does.
  if (before + part >= draw && before < draw + 0.0) {
    double acc = before;
    for (int64_t i = lo; i < hi; ++i) {
      acc += exp((static_cast<double>(logits[i]) - static_cast<double>(top)) * inv_t);
      if (acc >= draw) {
        atomicMin(reinterpret_cast<unsigned long long*>(&pick), static_cast<unsigned long long>(i));
        break;
      }
    }
  }
  __syncthreads();
  if (tid == 0) *chosen = static_cast<int32_t>(pick);
}

// ---- greedy over many workgroups ----------------------------------------------------------
// Each workgroup takes 2048 ids (two 16-byte pieces per thread) and keeps the largest key
//   key(v, i) = OrderKey(v == 0 ? +0 : v) << 32 | (2^32 - 1 - i),   0 for a NaN,
// so the largest key is the largest value, the earliest id among equal values (-0 equals +0),
// and NaNs never win: the reference's strict > scan, whose answer is 0 when id 0 holds a NaN
// (checked by the last workgroup). Thread 0 of each workgroup stores its key to part[b]
// (device scope), then counts its arrival with a device-scope acquire-release add: the
// release orders the key before the count, and in the workgroup whose add completes the
// grid the acquire, followed by the workgroup barrier, orders every thread's device-scope
// reads of part[] after all the keys. That workgroup picks the largest key, writes the id and
// sets the count back to zero for the next launch (launches on one stream are ordered).
constexpr int kGreedyThreads = 256;
constexpr int kGreedyIds = 2048;  // ids per workgroup
constexpr int kGreedyMaxBlocks = 1024;

__device__ uint64_t BlockMaxKey(uint64_t k, uint64_t* sk) {
  k = max(k, XorLane<32>(k));
  k = max(k, XorLane<16>(k));
  k = max(k, XorLane<8>(k));
  k = max(k, XorLane<4>(k));
  k = max(k, XorLane<2>(k));
  k = max(k, XorLane<1>(k));
  if ((threadIdx.x & 63) == 0) sk[threadIdx.x >> 6] = k;
  __syncthreads();
  uint64_t r = sk[0];
  for (int w = 1; w < kGreedyThreads / 64; ++w) r = max(r, sk[w]);
  return r;
}

__global__ __launch_bounds__(kGreedyThreads) void GreedyKernel(const float* logits, int32_t* chosen, int32_t vocab,
                                                               const int32_t* index_dev, uint64_t* part,
                                                               uint32_t* count) {
  __shared__ uint64_t sk[kGreedyThreads / 64];
  __shared__ int is_last;
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const float4* l4 = reinterpret_cast<const float4*>(logits);
  const int n4 = vocab / 4;  // vocab % 4 == 0 (launcher)
  uint64_t best = 0;
#pragma unroll
  for (int j = 0; j < kGreedyIds / 4 / kGreedyThreads; ++j) {
    const int i4 = b * (kGreedyIds / 4) + j * kGreedyThreads + tid;
    if (i4 < n4) {
      const float4 v = l4[i4];
      const uint32_t i0 = 4u * static_cast<uint32_t>(i4);
      best = max(best, GreedyKey(v.x, i0));
      best = max(best, GreedyKey(v.y, i0 + 1));
      best = max(best, GreedyKey(v.z, i0 + 2));
      best = max(best, GreedyKey(v.w, i0 + 3));
    }
  }
  best = BlockMaxKey(best, sk);
  if (tid == 0) {
    __hip_atomic_store(&part[b], best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = __hip_atomic_fetch_add(count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  }
  __syncthreads();
  if (!is_last) return;
  uint64_t k = 0;
  for (int i = tid; i < static_cast<int>(gridDim.x); i += kGreedyThreads)
    k = max(k, __hip_atomic_load(&part[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  __syncthreads();  // sk is reused
  k = BlockMaxKey(k, sk);
  if (tid == 0) {
    const int32_t id = (k == 0 || isnan(logits[0])) ? 0 : static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(k));
    chosen[index_dev != nullptr ? *index_dev : 0] = id;
    __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---- greedy from per-tile keys ----------------------------------------------------------------
// The keys a GEMV stored per 8-column tile (GemvPrologue::greedy_keys) hold the same maximum as
// GreedyKernel's per-workgroup keys, so one workgroup reduces them (8 loads a thread in flight
// at once) and answers as GreedyKernel's last workgroup does. No other workgroup is involved.
constexpr int kKeysThreads = 1024;
constexpr int kKeysBatch = 8;

__global__ __launch_bounds__(kKeysThreads) void GreedyKeysKernel(const uint64_t* keys, int32_t count,
                                                                 const float* logits, int32_t* chosen,
                                                                 const int32_t* index_dev) {
  __shared__ uint64_t sk[kKeysThreads / 64];
  const int tid = threadIdx.x;
  int32_t index = 0;
  float first = 0.f;
  if (tid == 0) {
    index = index_dev != nullptr ? *index_dev : 0;
    first = logits[0];
  }
  uint64_t best = 0;
  for (int i0 = 0; i0 < count; i0 += kKeysBatch * kKeysThreads) {
    uint64_t v[kKeysBatch];
#pragma unroll
    for (int u = 0; u < kKeysBatch; ++u) {
      const int i = i0 + u * kKeysThreads + tid;
      v[u] = i < count ? keys[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kKeysBatch; ++u) best = max(best, v[u]);
  }
  best = max(best, XorLane<32>(best));
  best = max(best, XorLane<16>(best));
  best = max(best, XorLane<8>(best));
  best = max(best, XorLane<4>(best));
  best = max(best, XorLane<2>(best));
  best = max(best, XorLane<1>(best));
  if ((tid & 63) == 0) sk[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    uint64_t k = sk[0];
    for (int w = 1; w < kKeysThreads / 64; ++w) k = max(k, sk[w]);
    chosen[index] = (k == 0 || isnan(first)) ? 0 : static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(k));
  }
}

// GreedyKeysKernel's pick followed by the embedding of the picked id (EmbeddingKernel's row:
// the fp32 table row, or fl(float(q) * row_scale[id]) of the int8 table), in one workgroup:
// the first kernel of a decode step whose previous step left its greedy keys. The id goes to
// chosen[*index_dev] as the sampler would write it, and the row to `out`.
__global__ __launch_bounds__(kKeysThreads) void GreedyEmbedKernel(const uint64_t* keys, int32_t count,
                                                                  const int32_t* index_dev, const int8_t* qtable,
                                                                  const float* row_scale, const float* table,
                                                                  const float* logits, int32_t* chosen, float* out,
                                                                  int32_t hidden) {
  __shared__ uint64_t sk[kKeysThreads / 64];
  __shared__ int32_t picked;
  const int tid = threadIdx.x;
  int32_t index = 0;
  float first = 0.f;
  if (tid == 0) {
    index = *index_dev;
    first = logits[0];
  }
  uint64_t best = 0;
  for (int i0 = 0; i0 < count; i0 += kKeysBatch * kKeysThreads) {
    uint64_t v[kKeysBatch];
#pragma unroll
    for (int u = 0; u < kKeysBatch; ++u) {
      const int i = i0 + u * kKeysThreads + tid;
      v[u] = i < count ? keys[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kKeysBatch; ++u) best = max(best, v[u]);
  }
  best = max(best, XorLane<32>(best));
  best = max(best, XorLane<16>(best));
  best = max(best, XorLane<8>(best));
  best = max(best, XorLane<4>(best));
  best = max(best, XorLane<2>(best));
  best = max(best, XorLane<1>(best));
  if ((tid & 63) == 0) sk[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    uint64_t k = sk[0];
    for (int w = 1; w < kKeysThreads / 64; ++w) k = max(k, sk[w]);
    const int32_t id = (k == 0 || isnan(first)) ? 0 : static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(k));
    chosen[index] = id;
    picked = id;
  }
  __syncthreads();
  const int64_t id = picked;
  if (table != nullptr) {
    const float* src = table + id * hidden;
    for (int i = tid; i < hidden; i += kKeysThreads) out[i] = src[i];
  } else {
    const int8_t* src = qtable + id * hidden;
    const float sc = row_scale[id];
    for (int i = tid; i < hidden; i += kKeysThreads) out[i] = __fmul_rn(static_cast<float>(src[i]), sc);
  }
}

}  // namespace

void LaunchGreedyEmbed(const uint64_t* keys, int64_t count, const int32_t* index_dev, const int8_t* qtable,
                       const float* row_scale, const float* table, const float* logits, int32_t* chosen, float* out,
                       int64_t hidden, hipStream_t stream) {
  if (keys == nullptr || logits == nullptr || chosen == nullptr || index_dev == nullptr || out == nullptr ||
      count < 1 || count > kGreedyKeysMax || hidden < 1 || hidden > 0x7fffffff ||
      (table == nullptr && (qtable == nullptr || row_scale == nullptr)))
    Fail(ACCEL_HIP_INVALID_ARGUMENT, "greedy embed: need 1 .. 65536 keys, the index, a table and the output row");
  hipLaunchKernelGGL(GreedyEmbedKernel, dim3(1), dim3(kKeysThreads), 0, stream, keys, static_cast<int32_t>(count),
                     index_dev, qtable, row_scale, table, logits, chosen, out, static_cast<int32_t>(hidden));
  Check(hipGetLastError(), "GreedyEmbedKernel launch");
}

void LaunchGreedyKeys(const uint64_t* keys, int64_t count, const float* logits, int32_t* chosen,
                      const int32_t* index_dev, hipStream_t stream) {
  if (keys == nullptr || logits == nullptr || chosen == nullptr || count < 1 || count > kGreedyKeysMax)
    Fail(ACCEL_HIP_INVALID_ARGUMENT, "greedy keys: need 1 .. 65536 keys, the logits and the chosen ids");
  hipLaunchKernelGGL(GreedyKeysKernel, dim3(1), dim3(kKeysThreads), 0, stream, keys, static_cast<int32_t>(count),
                     logits, chosen, index_dev);
  Check(hipGetLastError(), "GreedyKeysKernel launch");
}

size_t GreedyWorkBytes(int64_t vocab) {
  return 64 + static_cast<size_t>((vocab + kGreedyIds - 1) / kGreedyIds) * sizeof(uint64_t);
}

void LaunchSampleToken(const float* logits, int32_t* chosen, int64_t vocab, float temperature, uint32_t* rng_inout,
                       int32_t top_k, hipStream_t stream, const int32_t* index_dev, void* greedy_work,
                       size_t greedy_bytes) {
  const int64_t blocks = (vocab + kGreedyIds - 1) / kGreedyIds;
  if (!(temperature > 0.f) && greedy_work != nullptr && greedy_bytes >= GreedyWorkBytes(vocab) && blocks > 1 &&
      blocks <= kGreedyMaxBlocks && vocab % 4 == 0 && reinterpret_cast<uintptr_t>(logits) % 16 == 0) {
    uint32_t* count = static_cast<uint32_t*>(greedy_work);
    uint64_t* part = reinterpret_cast<uint64_t*>(static_cast<char*>(greedy_work) + 64);
    hipLaunchKernelGGL(GreedyKernel, dim3(static_cast<uint32_t>(blocks)), dim3(kGreedyThreads), 0, stream, logits,
                       chosen, static_cast<int32_t>(vocab), index_dev, part, count);
    Check(hipGetLastError(), "GreedyKernel launch");
    return;
  }
  hipLaunchKernelGGL(SampleKernel, dim3(1), dim3(kThreads), 0, stream, logits, chosen, vocab, temperature, rng_inout,
                     top_k, index_dev);
  Check(hipGetLastError(), "SampleKernel launch");
}

}  // namespace accel_hip
