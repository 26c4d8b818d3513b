// int8-weight GEMV: C[m, n] = A[m, k] @ dequant(W)[k, n] for m <= 16, W int8 row-major
// [k, n] exactly as accel::MatMulQuantized receives it (src/sim_device.cc:541-602).
//
// Bound: HBM. Algorithmic bytes per call = k*n (int8 W) + 4*n (scale) + 4*m*k (A) + 4*m*n (C).
//
// Both kernels stream W with 16-byte loads (16 int8 columns of one row per lane), convert
// the bytes to fp32 exactly and let the matrix cores do the multiply-adds. Per-column (or
// whole-tensor) scale multiplies each finished sum once; a per-row scale is folded into A;
// zero points are subtracted from the exact integer before the product. Every sum runs in a
// fixed order, so results are deterministic.
//
// Narrow kernel (m <= 4), the decode path:
//  * a workgroup (8 waves) owns a 64-column tile over its whole K range, so no workgroup
//    waits for another; 4 lanes cover one 64-byte row segment and a wave loads 16 rows
//    (1 KB) per instruction, 8 loads in flight per wave;
//  * v_mfma_f32_4x4x1_16b_f32: block b of lane l = 4b+j holds row slot b and columns
//    16j+t (t = byte of the load), A rows 0..3; the 16 row slots are summed with lane
//    shuffles, the 8 waves through LDS;
//  * tiles go to XCDs in contiguous runs (workgroup i runs on XCD i % 8), so the two tiles
//    that share each 128-byte line of W are read through the same L2.
// Wide kernel (4 < m <= 16): 256-column tiles, 16 lanes per 256-byte row segment, 4 rows per
// wave load feed v_mfma_f32_16x16x4_f32 as its K = 4; A staged in LDS.
// Split-K (only where the tile count cannot fill the GPU): each split writes its partial
// sums to the workspace and a second kernel adds them in split order (no inter-workgroup
// synchronization inside a kernel).
#include "device_common.h"

namespace accel_hip {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kXcds = 8;

struct GemvArgs {
  const float* a;
  const int8_t* q;
  const float* scale;
  const int8_t* zero;
  int32_t mode;
  int64_t const_index;
  float* c;
  int64_t m, k, n;
  int32_t tiles;
  int32_t tiles_per_xcd;
  int32_t splits;
  int64_t rows_per_split;
  float* partials;  // [splits][m][n] when splits > 1
  // Column-tiled copy of W (narrow kernel): 64-column tile t, row r at tiled + (t*k + r)*64,
  // columns past n zero. nullptr: read W in its [k, n] layout.
  const int8_t* tiled;
  Epilogue epi;
};

// The 16 bytes at columns [col, col + 16) of one row (`row` must point inside W); zero past
// n or when !valid. The 16-byte form loads unconditionally from a clamped column (n >= 16
// there) and selects, so no branch forces an early wait on the load.
template <bool kVec>
__device__ __forceinline__ uint4 LoadRow16(const int8_t* row, int64_t col, int64_t n, bool valid) {
  if (kVec) {
    // Columns past n read a clamped in-range chunk: their sums land in columns >= n, which
    // are never stored. Invalid rows are neutralized by a zero A operand at use.
    const int64_t cc = col < n ? col : n - 16;
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + cc));
    return make_uint4(v[0], v[1], v[2], v[3]);
  }
  uint32_t w[4] = {0, 0, 0, 0};
  if (valid) {
    for (int b = 0; b < 16; ++b) {
      if (col + b < n) w[b >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(row[col + b])) << (8 * (b & 3));
    }
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ uint32_t Word(const uint4& v, int d) {
  return d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w;
}

__device__ __forceinline__ float ColScale(const GemvArgs& p, int64_t col) {
  if (p.mode == kScalePerCol) return p.scale[col];
  if (p.mode == kScaleConst) return p.scale[p.const_index];
  return 1.f;  // per-row scale was folded into A
}

// Zero points of the 16 columns [col, col + 16) (per-column or whole-tensor), as floats.
template <bool kZero>
__device__ __forceinline__ void ColumnZeros(const GemvArgs& p, int64_t col, float (&zc)[16]) {
  for (int j = 0; j < 16; ++j) zc[j] = 0.f;
  if (!kZero) return;
  if (p.mode == kScalePerCol) {
    for (int j = 0; j < 16; ++j) zc[j] = (col + j < p.n) ? static_cast<float>(p.zero[col + j]) : 0.f;
  } else if (p.mode == kScaleConst) {
    const float z = static_cast<float>(p.zero[p.const_index]);
    for (int j = 0; j < 16; ++j) zc[j] = z;
  }
}

// Stores one finished sum: to the split's partials, or scaled + epilogue into C.
__device__ __forceinline__ void Emit(const GemvArgs& p, int split, int64_t mm, int64_t col, float s) {
  if (p.splits > 1) {
    p.partials[(static_cast<int64_t>(split) * p.m + mm) * p.n + col] = s;
  } else {
    p.c[mm * p.n + col] = ApplyEpilogue(__fmul_rn(s, ColScale(p, col)), mm, col, p.n, p.epi);
  }
}

// ---- narrow kernel: m <= 4, staged column tiles -----------------------------------------------
constexpr int kNarrowWaves = 8;
constexpr int kNarrowThreads = kNarrowWaves * 64;
constexpr int kNarrowTile = 64;
constexpr int kNarrowUnroll = 4;

// One batch of kNarrowUnroll 16-row loads of one wave, as loaded: no value is inspected
// until ComputeNarrowBatch, so issuing a batch never waits for memory.
struct NarrowBatch {
  uint4 w[kNarrowUnroll];
  float a[kNarrowUnroll];
  float s[kNarrowUnroll];   // per-row scale (kRowScale)
  int8_t z[kNarrowUnroll];  // per-row zero (kZero && kRowScale)
};

// kRowScale: the plane's scale (and zero) runs along k; the scale is folded into A.
// `tbase` is this lane's 16 bytes of row 0 in its tile of the staged copy.
template <bool kZero, bool kRowScale>
__device__ __forceinline__ void LoadNarrowBatch(const GemvArgs& p, int64_t r0, int slot, int64_t ke,
                                                const int8_t* tbase, int64_t a_row, NarrowBatch& b) {
  constexpr int64_t kStep = kNarrowWaves * 16;
#pragma unroll
  for (int u = 0; u < kNarrowUnroll; ++u) {
    const int64_t row = r0 + u * kStep + slot;
    const int64_t rc = row < ke ? row : ke - 1;  // rows past ke re-read a valid row
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tbase + rc * kNarrowTile));
    b.w[u] = make_uint4(v[0], v[1], v[2], v[3]);
    b.a[u] = p.a[a_row * p.k + rc];
    if (kRowScale) b.s[u] = p.scale[rc];
    if (kZero && kRowScale) b.z[u] = p.zero[rc];
  }
}

// kValu (m == 1): the product runs on the VALU (one fma per byte); otherwise
// v_mfma_f32_4x4x1_16b_f32 multiplies A rows 0..3 at once.
template <bool kZero, bool kRowScale, bool kValu>
__device__ __forceinline__ void ComputeNarrowBatch(const NarrowBatch& b, int64_t r0, int slot, int64_t ke,
                                                   bool a_live, const float (&zc)[16], v4f (&acc)[16],
                                                   float (&accv)[16]) {
  constexpr int64_t kStep = kNarrowWaves * 16;
#pragma unroll
  for (int u = 0; u < kNarrowUnroll; ++u) {
    const bool valid = r0 + u * kStep + slot < ke;
    float a = kRowScale ? __fmul_rn(b.a[u], b.s[u]) : b.a[u];
    a = (valid && a_live) ? a : 0.f;
    const float zr = (kZero && kRowScale) ? static_cast<float>(b.z[u]) : 0.f;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float x = ByteToFloat(Word(b.w[u], t >> 2), t & 3);
      if (kZero) x = x - (zc[t] + zr);
      if (kValu) {
        accv[t] = __builtin_fmaf(a, x, accv[t]);
      } else {
        acc[t] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, x, acc[t], 0, 0, 0);
      }
    }
  }
}

template <bool kZero, bool kRowScale, bool kValu>
__global__ __launch_bounds__(kNarrowThreads) void GemvNarrowKernel(GemvArgs p) {
  __shared__ float red[kNarrowWaves][4][kNarrowTile];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tile = (blockIdx.x % kXcds) * p.tiles_per_xcd + blockIdx.x / kXcds;
  if (tile >= p.tiles) return;
  const int split = blockIdx.y;
  const int64_t kb = static_cast<int64_t>(split) * p.rows_per_split;
  const int64_t ke = min(p.k, kb + p.rows_per_split);

  const int slot = lane >> 2;  // row of a 16-row load (MFMA: the block index)
  const int nj = lane & 3;     // 16-column chunk (MFMA: the block column)
  const int64_t col = static_cast<int64_t>(tile) * kNarrowTile + nj * 16;
  // A operand: the VALU form uses row 0 everywhere; the MFMA form feeds row l % 4 from lane l.
  const bool a_live = kValu || nj < p.m;
  const int64_t a_row = (kValu || !a_live) ? 0 : nj;
  float zc[16];
  ColumnZeros<kZero>(p, col, zc);

  v4f acc[16];
  float accv[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
    accv[t] = 0.f;
  }

  // Batches of kNarrowUnroll 16-row loads, double buffered: the next batch is in flight
  // while the current one is multiplied. Rows past ke are clamped to a valid address and
  // contribute through a zero A operand, so the loads need no branches. The steady-state
  // loop issues its loads unconditionally (a load inside a branch makes the compiler wait
  // for every outstanding load where the paths merge); the last batches are peeled, and
  // sched_barrier keeps the scheduler from sinking the next batch's loads into the current
  // batch's arithmetic.
  constexpr int64_t kStep = kNarrowWaves * 16;
  constexpr int64_t kBatchRows = kStep * kNarrowUnroll;
  const int8_t* tbase = p.tiled + static_cast<int64_t>(tile) * p.k * kNarrowTile + nj * 16;
  NarrowBatch bx, by;
  const int64_t first = kb + wave * 16;
  const int64_t batches = first < ke ? (ke - first + kBatchRows - 1) / kBatchRows : 0;
  int64_t r0 = first;
  if (batches > 0) LoadNarrowBatch<kZero, kRowScale>(p, r0, slot, ke, tbase, a_row, bx);
  int64_t i = 0;
  for (; i + 2 < batches; i += 2) {
    LoadNarrowBatch<kZero, kRowScale>(p, r0 + kBatchRows, slot, ke, tbase, a_row, by);
    __builtin_amdgcn_sched_barrier(0);
    ComputeNarrowBatch<kZero, kRowScale, kValu>(bx, r0, slot, ke, a_live, zc, acc, accv);
    __builtin_amdgcn_sched_barrier(0);
    LoadNarrowBatch<kZero, kRowScale>(p, r0 + 2 * kBatchRows, slot, ke, tbase, a_row, bx);
    __builtin_amdgcn_sched_barrier(0);
    ComputeNarrowBatch<kZero, kRowScale, kValu>(by, r0 + kBatchRows, slot, ke, a_live, zc, acc, accv);
    __builtin_amdgcn_sched_barrier(0);
    r0 += 2 * kBatchRows;
  }
  if (i + 2 == batches) {
    LoadNarrowBatch<kZero, kRowScale>(p, r0 + kBatchRows, slot, ke, tbase, a_row, by);
    ComputeNarrowBatch<kZero, kRowScale, kValu>(bx, r0, slot, ke, a_live, zc, acc, accv);
    ComputeNarrowBatch<kZero, kRowScale, kValu>(by, r0 + kBatchRows, slot, ke, a_live, zc, acc, accv);
  } else if (i + 1 == batches) {
    ComputeNarrowBatch<kZero, kRowScale, kValu>(bx, r0, slot, ke, a_live, zc, acc, accv);
  }

  // Sum the 16 row slots (lanes 4b + j, b = 0..15) of each live A row; lanes 0..3 then hold
  // columns 16*lane + t. MFMA block b's VGPR r is A row r.
  if (kValu) {
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float v = accv[t];
      v = v + __shfl_xor(v, 4);
      v = v + __shfl_xor(v, 8);
      v = v + __shfl_xor(v, 16);
      v = v + __shfl_xor(v, 32);
      acc[t][0] = v;
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (r < p.m) {
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          float v = acc[t][r];
          v = v + __shfl_xor(v, 4);
          v = v + __shfl_xor(v, 8);
          v = v + __shfl_xor(v, 16);
          v = v + __shfl_xor(v, 32);
          acc[t][r] = v;
        }
      }
    }
  }
  if (lane < 4) {
    for (int r = 0; r < 4; ++r)
      for (int t = 0; t < 16; ++t) red[wave][r][lane * 16 + t] = acc[t][r];
  }
  __syncthreads();
  if (tid < 4 * kNarrowTile) {
    const int mm = tid / kNarrowTile;
    const int c = tid % kNarrowTile;
    const int64_t out_col = static_cast<int64_t>(tile) * kNarrowTile + c;
    if (mm < p.m && out_col < p.n) {
      float s = red[0][mm][c];
      for (int wv = 1; wv < kNarrowWaves; ++wv) s = s + red[wv][mm][c];
      Emit(p, split, mm, out_col, s);
    }
  }
}

// ---- wide kernel: 4 < m <= 16 ----------------------------------------------------------------
constexpr int kWideThreads = 256;
constexpr int kWideWaves = kWideThreads / 64;
constexpr int kWideTile = 256;
constexpr int kWideMaxRows = 1024;
constexpr int kWideUnroll = 4;

template <bool kVec, bool kZero, bool kRowScale>
__global__ __launch_bounds__(kWideThreads) void GemvWideKernel(GemvArgs p) {
  __shared__ float smem[16 * kWideMaxRows];  // A stage [row][16]; reused for the wave sums
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tile = (blockIdx.x % kXcds) * p.tiles_per_xcd + blockIdx.x / kXcds;
  if (tile >= p.tiles) return;
  const int split = blockIdx.y;
  const int64_t k0 = static_cast<int64_t>(split) * p.rows_per_split;
  const int rows = static_cast<int>(min(p.rows_per_split, p.k - k0));

  for (int idx = tid; idx < rows * 16; idx += kWideThreads) {
    const int r = idx >> 4;
    const int mm = idx & 15;
    float v = 0.f;
    if (mm < p.m) {
      v = p.a[mm * p.k + k0 + r];
      if (kRowScale) v = __fmul_rn(v, p.scale[k0 + r]);
    }
    smem[idx] = v;
  }
  __syncthreads();

  const int lane_row = lane >> 4;  // MFMA k of this lane
  const int lane_col = lane & 15;  // MFMA column of this lane
  const int64_t col = static_cast<int64_t>(tile) * kWideTile + lane_col * 16;
  float zc[16];
  ColumnZeros<kZero>(p, col, zc);
  v4f acc[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

  const int groups = (rows + 3) >> 2;
  const int8_t* wbase = p.q + k0 * p.n;
  for (int g0 = wave; g0 < groups; g0 += kWideWaves * kWideUnroll) {
    uint4 w[kWideUnroll];
    float av[kWideUnroll];
    float zr[kWideUnroll];
#pragma unroll
    for (int u = 0; u < kWideUnroll; ++u) {
      const int g = g0 + u * kWideWaves;
      const int r = g * 4 + lane_row;
      const bool valid = g < groups && r < rows;
      const int rc = valid ? r : rows - 1;
      w[u] = LoadRow16<kVec>(wbase + static_cast<int64_t>(rc) * p.n, col, p.n, valid);
      const float a = smem[rc * 16 + lane_col];  // A[l % 16][row of l]
      av[u] = valid ? a : 0.f;
      zr[u] = (kZero && kRowScale) ? static_cast<float>(p.zero[k0 + rc]) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kWideUnroll; ++u) {
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        float b = ByteToFloat(Word(w[u], t >> 2), t & 3);
        if (kZero) b = b - (zc[t] + zr[u]);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], b, acc[t], 0, 0, 0);
      }
    }
  }
  __syncthreads();  // A stage done; smem becomes [wave][16][kWideTile]
  // Lane l holds m = 4*(l/16) + r, column 16*(l%16) + t.
  for (int r = 0; r < 4; ++r)
    for (int t = 0; t < 16; ++t) smem[(wave * 16 + 4 * lane_row + r) * kWideTile + lane_col * 16 + t] = acc[t][r];
  __syncthreads();
  const int64_t out_col = static_cast<int64_t>(tile) * kWideTile + tid;
  if (out_col >= p.n) return;
  for (int mm = 0; mm < p.m; ++mm) {
    float s = smem[mm * kWideTile + tid];
    for (int wv = 1; wv < kWideWaves; ++wv) s = s + smem[(wv * 16 + mm) * kWideTile + tid];
    Emit(p, split, mm, out_col, s);
  }
}

// ---- split-K reduction ----------------------------------------------------------------------
__global__ void SplitReduceKernel(const float* partials, int32_t splits, int64_t m, int64_t n, float* c,
                                  int32_t mode, const float* scale, int64_t const_index, Epilogue epi) {
  const int64_t total = m * n;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = idx / n;
    const int64_t j = idx - i * n;
    float s = partials[idx];
    for (int sp = 1; sp < splits; ++sp) s = s + partials[static_cast<int64_t>(sp) * total + idx];
    float cs = 1.f;
    if (scale != nullptr && mode == kScalePerCol) cs = scale[j];
    if (scale != nullptr && mode == kScaleConst) cs = scale[const_index];
    c[idx] = ApplyEpilogue(__fmul_rn(s, cs), i, j, n, epi);
  }
}

// dst[(t*k + r)*64 + c] = q[r*n + 64t + c] (0 past n): 64-column tiles, each contiguous.
// One thread moves 16 bytes: a 16-byte-aligned chunk when n allows it, bytes otherwise.
__global__ void TileColumnsKernel(const int8_t* q, int64_t k, int64_t n, int8_t* dst, int64_t tiles) {
  const int64_t chunks = tiles * k * (kGemvTileCols / 16);
  const bool vec = (n % 16 == 0) && (reinterpret_cast<uintptr_t>(q) % 16 == 0);
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < chunks;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t j = idx % (kGemvTileCols / 16);  // 16-byte chunk within the tile row
    const int64_t tr = idx / (kGemvTileCols / 16);
    const int64_t r = tr % k;
    const int64_t t = tr / k;
    const int64_t col = t * kGemvTileCols + j * 16;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (vec && col + 15 < n) {
      v = *reinterpret_cast<const uint4*>(q + r * n + col);
    } else {
      uint32_t w[4] = {0, 0, 0, 0};
      for (int b = 0; b < 16; ++b)
        if (col + b < n) w[b >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(q[r * n + col + b])) << (8 * (b & 3));
      v = make_uint4(w[0], w[1], w[2], w[3]);
    }
    *reinterpret_cast<uint4*>(dst + idx * 16) = v;
  }
}

}  // namespace

void LaunchTileColumns(const int8_t* q, int64_t k, int64_t n, int8_t* dst, hipStream_t stream) {
  const int64_t tiles = (n + kGemvTileCols - 1) / kGemvTileCols;
  const int64_t chunks = tiles * k * (kGemvTileCols / 16);
  int64_t grid = (chunks + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(TileColumnsKernel, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream, q, k, n, dst, tiles);
  Check(hipGetLastError(), "TileColumnsKernel launch");
}

void LaunchSplitReduce(const float* partials, int32_t splits, int64_t m, int64_t n, float* c, int32_t mode,
                       const float* scale, int64_t const_index, const Epilogue& epi, hipStream_t stream) {
  const int64_t total = m * n;
  int64_t grid = (total + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(SplitReduceKernel, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream, partials, splits, m, n,
                     c, mode, scale, const_index, epi);
  Check(hipGetLastError(), "SplitReduceKernel launch");
}

void LaunchGemvQ8(const float* a, const Q8View& b, float* c, int64_t m, int64_t k, int64_t n, const Epilogue& epi,
                  hipStream_t stream) {
  if (m < 1 || m > 16 || k < 1 || n < 1) Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMV shape out of range");
  Context& ctx0 = Ctx();
  const int64_t cus = ctx0.cu_count > 0 ? ctx0.cu_count : 256;
  // The narrow kernel reads the staged column tiles; without them the wide kernel, which
  // reads W in place, takes any m <= 16.
  const bool narrow = m <= 4 && b.tiled != nullptr;
  const int64_t tile_cols = narrow ? kNarrowTile : kWideTile;
  const int64_t tiles = (n + tile_cols - 1) / tile_cols;
  int64_t splits = 1;
  if (narrow) {
    // One workgroup per tile over all of K unless the tiles leave most CUs idle on a long K.
    if (tiles < cus / 2 && k >= 4096) splits = std::min<int64_t>((cus + tiles - 1) / tiles, k / 1024);
  } else {
    splits = std::max<int64_t>((cus + tiles - 1) / tiles, (k + kWideMaxRows - 1) / kWideMaxRows);
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, (k + 255) / 256));
  }
  int64_t rows = (k + splits - 1) / splits;
  rows = (rows + 15) / 16 * 16;
  if (!narrow) rows = std::min<int64_t>(rows, kWideMaxRows);
  splits = (k + rows - 1) / rows;
  const int64_t tiles_per_xcd = (tiles + kXcds - 1) / kXcds;
  if (tiles_per_xcd * kXcds > 0x7fffffff || splits > 65535) Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMV grid too large");

  GemvArgs args;
  args.a = a;
  args.q = b.q;
  args.scale = b.scale;
  args.zero = b.zero;
  args.mode = b.mode;
  args.const_index = b.const_index;
  args.c = c;
  args.m = m;
  args.k = k;
  args.n = n;
  args.tiles = static_cast<int32_t>(tiles);
  args.tiles_per_xcd = static_cast<int32_t>(tiles_per_xcd);
  args.splits = static_cast<int32_t>(splits);
  args.rows_per_split = rows;
  args.partials = nullptr;
  args.epi = epi;
  if (splits > 1) {
    Context& ctx = Scratch(static_cast<size_t>(splits * m * n) * sizeof(float));
    args.partials = static_cast<float*>(ctx.workspace);
  }
  static_assert(kNarrowTile == kGemvTileCols, "staged tiles must match the narrow kernel tile");
  args.tiled = narrow ? b.tiled : nullptr;
  const bool vec = (n % 16 == 0) && (reinterpret_cast<uintptr_t>(b.q) % 16 == 0);
  const bool zero = b.zero != nullptr;
  const bool row_scale = b.mode == kScalePerRow;
  const dim3 grid(static_cast<uint32_t>(tiles_per_xcd * kXcds), static_cast<uint32_t>(splits));
  const int variant = (vec ? 4 : 0) | (zero ? 2 : 0) | (row_scale ? 1 : 0);
  if (narrow) {
    const dim3 block(kNarrowThreads);
    switch ((m == 1 ? 4 : 0) + (zero ? 2 : 0) + (row_scale ? 1 : 0)) {
#define ACCEL_GEMV_CASE(V, Z, R) \
  case (V ? 4 : 0) + (Z ? 2 : 0) + (R ? 1 : 0): \
    hipLaunchKernelGGL((GemvNarrowKernel<Z, R, V>), grid, block, 0, stream, args); \
    break;
      ACCEL_GEMV_CASE(true, true, true) ACCEL_GEMV_CASE(true, true, false) ACCEL_GEMV_CASE(true, false, true)
      ACCEL_GEMV_CASE(true, false, false) ACCEL_GEMV_CASE(false, true, true) ACCEL_GEMV_CASE(false, true, false)
      ACCEL_GEMV_CASE(false, false, true) ACCEL_GEMV_CASE(false, false, false)
#undef ACCEL_GEMV_CASE
    }
  } else {
    const dim3 block(kWideThreads);
    switch (variant) {
#define ACCEL_GEMV_CASE(V, Z, R) \
  case (V ? 4 : 0) | (Z ? 2 : 0) | (R ? 1 : 0): \
    hipLaunchKernelGGL((GemvWideKernel<V, Z, R>), grid, block, 0, stream, args); \
    break;
      ACCEL_GEMV_CASE(true, true, true) ACCEL_GEMV_CASE(true, true, false) ACCEL_GEMV_CASE(true, false, true)
      ACCEL_GEMV_CASE(true, false, false) ACCEL_GEMV_CASE(false, true, true) ACCEL_GEMV_CASE(false, true, false)
      ACCEL_GEMV_CASE(false, false, true) ACCEL_GEMV_CASE(false, false, false)
#undef ACCEL_GEMV_CASE
    }
  }
  Check(hipGetLastError(), "GEMV launch");
  if (splits > 1) LaunchSplitReduce(args.partials, args.splits, m, n, c, b.mode, b.scale, b.const_index, epi, stream);
}

}  // namespace accel_hip
