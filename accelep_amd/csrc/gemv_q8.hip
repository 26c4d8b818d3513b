// int8-weight GEMV: C[m, n] = A[m, k] @ dequant(W)[k, n] for m <= 16, W int8 row-major
// [k, n] exactly as accel::MatMulQuantized receives it (src/sim_device.cc:541-602).
//
// Bound: HBM. Algorithmic bytes per call = k*n (int8 W) + 4*n (scale) + 4*m*k (A) + 4*m*n (C).
//
// Every kernel streams W with 16-byte loads and converts the bytes exactly. Per-column
// (or whole-tensor) scale multiplies each finished sum once; a per-row scale is folded into
// A; zero points are subtracted from the exact integer before the product. Every sum runs
// in a fixed order, so results are deterministic.
//
// Narrow kernel (m <= 4), the decode path, reads a staged copy of W in 8-column tiles (each
// tile k x 8 bytes, contiguous):
//  * a workgroup owns one tile over its K range, so no workgroup waits for another; a
//    4096 x 14336 matrix gives 1792 workgroups of 32 KB each, 7 per CU on 256 CUs;
//  * lane l loads rows (2l, 2l + 1) of the tile as one 16-byte load, a wave 128 rows (1 KB)
//    per instruction, and multiplies on the VALU (the product per byte is one conversion and
//    m fused multiply-adds, below the HBM time for m <= 4);
//  * the 8 column sums of the 64 lanes are reduce-scattered with lane shuffles, the waves'
//    sums added through LDS;
//  * tiles go to XCDs in contiguous runs (workgroup i runs on XCD i % 8).
// Split-bf16 kernel (2 < m <= 16, k a multiple of 32, no zero points or per-row scale): a
// group-interleaved staged copy of the tiles, exact products on v_mfma_f32_16x16x32_bf16
// with each activation split into three bf16 parts, split-K summed in split order by the
// last workgroup of each column group to arrive (no second kernel).
// Wide kernel (the other 4 < m <= 16 cases): W in place, 256-column tiles, 16 lanes per
// 256-byte row segment, 4 rows per wave load feed v_mfma_f32_16x16x4_f32 as its K = 4; A
// staged in LDS.
// Split-K of the narrow and wide kernels (only where the tile count cannot fill the GPU):
// each split writes its partial sums to the workspace and a second kernel adds them in
// split order.
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
  int32_t group_pairs;  // split-bf16 kernel: column groups x splits
  int64_t rows_per_split;
  float* partials;  // [splits][m][n] when splits > 1
  // Column-tiled copy of W (narrow kernel): 8-column tile t, row r at tiled + (t*kp + r)*8
  // (kp = k rounded up to even), columns past n and the pad row zero. nullptr: read W in
  // its [k, n] layout.
  const int8_t* tiled;
  // Group-interleaved copy of W (split-bf16 kernel; StagedGroupBytes' layout), and its
  // per-group arrival counters (zero between launches).
  const int8_t* grouped;
  uint32_t* arrivals;
  Epilogue epi;
  GemvPrologue pro;  // narrow m = 1 kernel with kAOp != 0
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
    StoreC(p.c, mm, col, p.n, p.epi, ApplyEpilogue(__fmul_rn(s, ColScale(p, col)), mm, col, p.n, p.epi));
  }
}

// ---- narrow kernel: m <= 4, staged 8-column tiles --------------------------------------------
// Staged tile t holds columns [8t, 8t + 8) for rows 0..kp-1 (kp = k rounded up to even), byte
// (r, c) at tiled[(t * kp + r) * 8 + c], zero past n and in the pad row. One workgroup owns
// one tile (over its split's rows): its bytes are one contiguous run, so the tiles of all
// workgroups stream W in order. Lane l of the workgroup loads rows (r, r + 1), r = 2l + step,
// as one 16-byte load (row r in bytes 0..7, row r + 1 in bytes 8..15); A rows are multiplied
// on the VALU (one conversion and m fused multiply-adds per byte).
constexpr int kNarrowTile = 8;

template <int M>
struct NarrowShape {
  static constexpr int kWaves = M == 1 ? 4 : 8;  // waves per workgroup
  static constexpr int kUnroll = M == 1 ? 8 : 4;  // 16-byte loads per lane per batch
  static constexpr int kThreads = kWaves * 64;
  static constexpr int64_t kStepRows = kThreads * 2;           // rows one load of the workgroup covers
  static constexpr int64_t kBatchRows = kStepRows * kUnroll;   // rows of one batch
};

// One batch of loads, as loaded: nothing is inspected until ComputeNarrowBatch, so issuing
// a batch never waits for memory.
template <int M, int U>
struct NarrowBatch {
  u32x4 w[U];
  float a[U][M][2];
  float s[U][2];   // per-row scale (kRowScale)
  int8_t z[U][2];  // per-row zero (kZero && kRowScale)
};

// Rows past ke are clamped to valid addresses (the W pair to kw - 2, kw = ke rounded up to
// even, which never passes the staged pad row; A, scale and zero to ke - 1) and are zeroed
// through A at use, so the loads need no branches. Row indexes are 32-bit: the launcher
// sends only k < 2^28 here.
// kPairA: k even and A 8-byte aligned, so (a[r], a[r + 1]) is one aligned 8-byte load.
// kClamp false: the caller has checked that every row of the batch lies below ke.
// kCached: a plain load instead of a streaming (nontemporal) one, for a weight that later
// calls read again while it can still sit in the last-level cache (Q8View::cached).
// Load u of a batch: the W pair.
template <int M, int U, bool kClamp, bool kCached = false>
__device__ __forceinline__ void LoadNarrowWAt(int u, int r0, int kw, const int8_t* tbase, NarrowBatch<M, U>& b) {
  using S = NarrowShape<M>;
  const int r = r0 + u * static_cast<int>(S::kStepRows);
  const int rw = !kClamp || r < kw - 2 ? r : kw - 2;
  const u32x4* at = reinterpret_cast<const u32x4*>(tbase + static_cast<uint32_t>(rw) * 8u);
  if constexpr (kCached)
    b.w[u] = *at;
  else
    b.w[u] = __builtin_nontemporal_load(at);
}

// Load u of a batch: the A rows (and per-row scale and zero).
template <int M, int U, bool kZero, bool kRowScale, bool kPairA, bool kClamp>
__device__ __forceinline__ void LoadNarrowAAt(int u, const GemvArgs& p, const float* const (&arow)[M], int r0, int ke,
                                              NarrowBatch<M, U>& b) {
  using S = NarrowShape<M>;
  const int r = r0 + u * static_cast<int>(S::kStepRows);
  const int r1 = !kClamp || r < ke - 1 ? r : ke - 1;
  const int r2 = !kClamp || r + 1 < ke - 1 ? r + 1 : ke - 1;
#pragma unroll
  for (int mm = 0; mm < M; ++mm) {
    // Offsets as 32-bit values from the uniform row base: one VGPR per address.
    const char* abase = reinterpret_cast<const char*>(arow[mm]);
    if (kPairA) {
      // k is even here, so ke is even and the pair (rp, rp + 1) is whole.
      const int rp = !kClamp || r < ke - 2 ? r : ke - 2;
      const float2 v = *reinterpret_cast<const float2*>(abase + static_cast<uint32_t>(rp) * 4u);
      b.a[u][mm][0] = v.x;
      b.a[u][mm][1] = v.y;
    } else {
      b.a[u][mm][0] = *reinterpret_cast<const float*>(abase + static_cast<uint32_t>(r1) * 4u);
      b.a[u][mm][1] = *reinterpret_cast<const float*>(abase + static_cast<uint32_t>(r2) * 4u);
    }
  }
  if (kRowScale) {
    b.s[u][0] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(p.scale) + static_cast<uint32_t>(r1) * 4u);
    b.s[u][1] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(p.scale) + static_cast<uint32_t>(r2) * 4u);
  }
  if (kZero && kRowScale) {
    b.z[u][0] = p.zero[static_cast<uint32_t>(r1)];
    b.z[u][1] = p.zero[static_cast<uint32_t>(r2)];
  }
}

// The whole batch, each W load followed by its A loads: loads complete in issue order, so
// load u's data is ready as soon as the first u loads are, and the products of u start while
// the later loads are still in flight. The scheduling barrier after each step keeps that
// order: left free, the compiler issued later steps' A loads behind most weight loads, and
// the products of steps 3..6 then waited for 14 of the 16 loads (m = 1, 4096 x 14336:
// 10.29 us against 10.06 us in this order).
template <int M, int U, bool kZero, bool kRowScale, bool kPairA, bool kClamp, bool kCached = false>
__device__ __forceinline__ void LoadNarrowBatch(const GemvArgs& p, const float* const (&arow)[M], int r0, int ke,
                                                int kw, const int8_t* tbase, NarrowBatch<M, U>& b) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    LoadNarrowWAt<M, U, kClamp, kCached>(u, r0, kw, tbase, b);
    LoadNarrowAAt<M, U, kZero, kRowScale, kPairA, kClamp>(u, p, arow, r0, ke, b);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int M, int U, bool kZero, bool kRowScale, bool kClamp>
__device__ __forceinline__ void ComputeNarrowBatch(const NarrowBatch<M, U>& b, int r0, int ke,
                                                   const float (&zc)[kNarrowTile], float (&acc)[M][kNarrowTile]) {
  using S = NarrowShape<M>;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int r = r0 + u * static_cast<int>(S::kStepRows);
    const bool v0 = !kClamp || r < ke;
    const bool v1 = !kClamp || r + 1 < ke;
    float a0[M], a1[M];
#pragma unroll
    for (int mm = 0; mm < M; ++mm) {
      const float x0 = kRowScale ? __fmul_rn(b.a[u][mm][0], b.s[u][0]) : b.a[u][mm][0];
      const float x1 = kRowScale ? __fmul_rn(b.a[u][mm][1], b.s[u][1]) : b.a[u][mm][1];
      a0[mm] = v0 ? x0 : 0.f;
      a1[mm] = v1 ? x1 : 0.f;
    }
    const float z0 = (kZero && kRowScale) ? static_cast<float>(b.z[u][0]) : 0.f;
    const float z1 = (kZero && kRowScale) ? static_cast<float>(b.z[u][1]) : 0.f;
#pragma unroll
    for (int c = 0; c < kNarrowTile; ++c) {
      float w0 = ByteToFloat(b.w[u][c >> 2], c & 3);
      float w1 = ByteToFloat(b.w[u][2 + (c >> 2)], c & 3);
      if (kZero) {
        w0 = w0 - (zc[c] + z0);
        w1 = w1 - (zc[c] + z1);
      }
#pragma unroll
      for (int mm = 0; mm < M; ++mm) {
        acc[mm][c] = __builtin_fmaf(a0[mm], w0, acc[mm][c]);
        acc[mm][c] = __builtin_fmaf(a1[mm], w1, acc[mm][c]);
      }
    }
  }
}


// Waves per SIMD the register budget must allow. For m = 1 with a per-column or whole-tensor
// scale, no zero points and no input prologue, 7 (<= 72 VGPRs): the 1792 tiles of a 4096 x
// 14336 matrix put 7 workgroups of 4 waves on each of 256 CUs, all resident at once. Other
// forms need more registers and take what the compiler gives them (1: no bound).
template <int M, bool kZero, bool kRowScale, int kAOp>
constexpr int NarrowMinWaves() {
  return (M == 1 && !kZero && !kRowScale && kAOp == 0) ? 7 : 1;
}

// Input transforms of the m = 1 kernel (GemvPrologue).
constexpr int kAOpNone = 0;
constexpr int kAOpRms = 1;
constexpr int kAOpSiluUp = 2;
// RMSNorm applied after the product (GemvPrologue::rms_after): A = fl(x * w) feeds the FMAs
// at once and the row's sum of squares is reduced beside them; each output is scaled by
// 1/rms at the store. Rounding differs from the normalize-first order (fast mode only).
constexpr int kAOpRmsAfter = 3;
// The decode attention's split partials combined into the row (GemvPrologue::attn_partial).
constexpr int kAOpAttn = 4;
// A = fl(x * second) (GemvPrologue::mul_up).
constexpr int kAOpMul = 5;
constexpr int kAttnDim = 64;
constexpr int kAttnMaxPairs = static_cast<int>(kGemvAttnMaxPairs);
constexpr int kAttnRegSplits = 8;  // splits loaded with the weights; more are read after them

// Rows (d, d + 1) of head hh from the split partials [heads][splits][2 + 64]: with ml[s] =
// (m_s, l_s) and ac[s] = (acc_s[d], acc_s[d + 1]) of the first kAttnRegSplits splits already
// loaded, w_s = e^(m_s - max m) (0 for an empty split, m_s = -inf), and the pair is
// (sum_s w_s acc_s) / (sum_s w_s l_s), every sum in split order. Each lane forms the weights
// of its own head; all lanes of all workgroups form them alike, so they agree bit for bit.
__device__ __forceinline__ void AttnCombinePair(const float* part, int splits, int hh, int d,
                                                const float2 (&ml)[kAttnRegSplits],
                                                const float2 (&ac)[kAttnRegSplits], float& a0, float& a1) {
  constexpr int kStride = 2 + kAttnDim;
  const float* head = part + hh * splits * kStride;
  float big = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < kAttnRegSplits; ++sp) big = fmaxf(big, ml[sp].x);
  for (int sp = kAttnRegSplits; sp < splits; ++sp) big = fmaxf(big, head[sp * kStride]);
  float l = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int sp = 0; sp < kAttnRegSplits; ++sp) {
    const float w = ml[sp].x == -INFINITY ? 0.f : expf(__fsub_rn(ml[sp].x, big));
    l = __fadd_rn(l, __fmul_rn(w, ml[sp].y));
    o0 = __fadd_rn(o0, __fmul_rn(w, ac[sp].x));
    o1 = __fadd_rn(o1, __fmul_rn(w, ac[sp].y));
  }
  for (int sp = kAttnRegSplits; sp < splits; ++sp) {
    const float2 m2 = *reinterpret_cast<const float2*>(head + sp * kStride);
    const float2 x2 = *reinterpret_cast<const float2*>(head + sp * kStride + 2 + d);
    const float w = m2.x == -INFINITY ? 0.f : expf(__fsub_rn(m2.x, big));
    l = __fadd_rn(l, __fmul_rn(w, m2.y));
    o0 = __fadd_rn(o0, __fmul_rn(w, x2.x));
    o1 = __fadd_rn(o1, __fmul_rn(w, x2.y));
  }
  a0 = __fdiv_rn(o0, l);
  a1 = __fdiv_rn(o1, l);
}

// Lane l's value x of lane (l & ~7) | j: a broadcast inside each group of 8 lanes (ds_swizzle in
// bit mode, and-mask 0x18 and or-mask j over the 32-lane halves; no LDS memory is touched).
template <int J>
__device__ __forceinline__ float Bcast8(float x) {
  static_assert(J >= 0 && J < 8, "lane of an 8-lane group");
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x18 | (J << 5)));
}

// AttnCombinePair for exactly 8 splits with the work spread over an 8-lane group: the 8 lanes
// of a group hold row pairs of one head (pairs 32h .. 32h + 31 form head h), so lane l loads
// only split l % 8's (m, l) beside its own 8 acc pairs, forms that split's weight (one expf),
// and the group exchanges the weights and the weighted l values. The max, every weight and
// both sums in split order are AttnCombinePair's, so the pair carries the same bits.
__device__ __forceinline__ void AttnCombinePairLanes(float2 mls, const float2 (&ac)[kAttnRegSplits], float& a0,
                                                     float& a1) {
  float big = mls.x;
  big = fmaxf(big, XorLane<1>(big));
  big = fmaxf(big, XorLane<2>(big));
  big = fmaxf(big, XorLane<4>(big));
  const float w = mls.x == -INFINITY ? 0.f : expf(__fsub_rn(mls.x, big));
  const float wl = __fmul_rn(w, mls.y);
  const float ws[kAttnRegSplits] = {Bcast8<0>(w), Bcast8<1>(w), Bcast8<2>(w), Bcast8<3>(w),
                                    Bcast8<4>(w), Bcast8<5>(w), Bcast8<6>(w), Bcast8<7>(w)};
  const float wls[kAttnRegSplits] = {Bcast8<0>(wl), Bcast8<1>(wl), Bcast8<2>(wl), Bcast8<3>(wl),
                                     Bcast8<4>(wl), Bcast8<5>(wl), Bcast8<6>(wl), Bcast8<7>(wl)};
  float l = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int sp = 0; sp < kAttnRegSplits; ++sp) {
    l = __fadd_rn(l, wls[sp]);
    o0 = __fadd_rn(o0, __fmul_rn(ws[sp], ac[sp].x));
    o1 = __fadd_rn(o1, __fmul_rn(ws[sp], ac[sp].y));
  }
  a0 = __fdiv_rn(o0, l);
  a1 = __fdiv_rn(o1, l);
}

// Writes the transformed input row (kAOp) into a_stage; every thread of the workgroup takes
// part and the row is complete when this returns.
template <int kAOp, int kThreads>
__device__ __forceinline__ void StageInputRow(const GemvArgs& p, float* a_stage, double* part) {
  const int tid = threadIdx.x;
  const int k32 = static_cast<int>(p.k);
  if (kAOp == kAOpRms) {
    double ss = 0.0;
    for (int i = tid; i < k32; i += kThreads) {
      const double v = static_cast<double>(p.a[i]);
      ss += v * v;
    }
    ss = WaveButterfly(ss, [](double a, double b) { return a + b; });
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    double total = 0.0;
    for (int wv = 0; wv < kThreads / 64; ++wv) total += part[wv];
    const double inv = 1.0 / sqrt(total / static_cast<double>(p.k) + static_cast<double>(p.pro.rms_eps));
    for (int i = tid; i < k32; i += kThreads)
      a_stage[i] = __fmul_rn(static_cast<float>(static_cast<double>(p.a[i]) * inv), p.pro.rms_weight[i]);
  } else {
    for (int i = tid; i < k32; i += kThreads) {
      const float x = p.a[i];
      a_stage[i] = __fmul_rn(__fdiv_rn(x, __fadd_rn(1.f, expf(-x))), p.pro.silu_up[i]);
    }
  }
  __syncthreads();
}

// kAOp != kAOpNone (m = 1, k <= one batch, no split): the workgroup issues its whole tile's
// loads, then writes the transformed input row into LDS while they are in flight, and the
// product reads the row from there. The RMS sum runs in RmsNormKernel's order (256 threads,
// stride 256, wave then fixed-order LDS sums), so the row equals that pass's output.
template <int M, bool kZero, bool kRowScale, bool kPairA, int kAOp = kAOpNone>
__global__ __launch_bounds__(NarrowShape<M>::kThreads)
__attribute__((amdgpu_waves_per_eu(NarrowMinWaves<M, kZero, kRowScale, kAOp>()))) void GemvNarrowKernel(
    const int8_t* tiled, const float* a, const float* scale, int32_t m, int32_t k, int32_t n, int32_t tiles,
    int32_t tiles_per_xcd, int32_t rows_per_split, GemvArgs p) {
  using S = NarrowShape<M>;
  static_assert(kAOp == kAOpNone || (M == 1 && S::kThreads == 256), "prologue: m = 1, RmsNormKernel's block");
  __shared__ float red[S::kWaves][M][kNarrowTile];
  __shared__ __align__(16) float a_stage[kAOp != kAOpNone ? kGemvPrologueMaxK : 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // A workgroup past the last tile (the grid is a multiple of the XCD count) recomputes the
  // last tile and stores nothing: no branch on the arguments before the loads are issued.
  const int tile_raw = (blockIdx.x % kXcds) * tiles_per_xcd + blockIdx.x / kXcds;
  const bool tile_live = tile_raw < tiles;
  const int tile = tile_live ? tile_raw : tiles - 1;
  const int split = blockIdx.y;
  const int64_t kb = static_cast<int64_t>(split) * rows_per_split;
  const int64_t ke = min(static_cast<int64_t>(k), kb + rows_per_split);
  const int64_t kw = ke + (ke & 1);
  const int64_t kp = k + (k & 1);
  const int64_t col0 = static_cast<int64_t>(tile) * kNarrowTile;

  float zc[kNarrowTile];
#pragma unroll
  for (int c = 0; c < kNarrowTile; ++c) zc[c] = 0.f;
  if (kZero && !kRowScale) {
#pragma unroll
    for (int c = 0; c < kNarrowTile; ++c) {
      const int64_t col = col0 + c < n ? col0 + c : n - 1;
      zc[c] = static_cast<float>(p.mode == kScalePerCol ? p.zero[col] : p.zero[p.const_index]);
    }
  }
  // The scale of the column this thread may store (c = tid % 8), loaded now so that storing
  // the sums waits for no memory. Every thread loads (from a clamped, valid index); a per-row
  // scale was folded into A and is not used here.
  const int64_t scol = col0 + (tid & 7) < n ? col0 + (tid & 7) : n - 1;
  const float col_scale = scale[p.mode == kScalePerCol ? scol : (p.mode == kScaleConst ? p.const_index : 0)];
  float acc[M][kNarrowTile];
#pragma unroll
  for (int mm = 0; mm < M; ++mm)
#pragma unroll
    for (int c = 0; c < kNarrowTile; ++c) acc[mm][c] = 0.f;

  // One batch in flight per wave: its loads are all issued before any of them is used. A
  // workgroup holds few registers, so several run per CU and cover each other's waits (a
  // second buffer would double the registers and halve the workgroups per CU).
  const int8_t* tbase = tiled + static_cast<int64_t>(tile) * kp * kNarrowTile;
  const float* arow[M];
#pragma unroll
  for (int mm = 0; mm < M; ++mm) arow[mm] = a + static_cast<int64_t>(mm < m ? mm : m - 1) * k;
  if (kAOp != kAOpNone) {
    // One clamped batch covers k (the launcher checks k <= kBatchRows and sends no split).
    __shared__ double part[S::kWaves];
    arow[0] = a_stage;
    const int r0 = 2 * tid;
    NarrowBatch<M, S::kUnroll> bx;
#pragma unroll
    for (int u = 0; u < S::kUnroll; ++u) LoadNarrowWAt<M, S::kUnroll, true>(u, r0, static_cast<int>(kw), tbase, bx);
    StageInputRow<kAOp, S::kThreads>(p, a_stage, part);
#pragma unroll
    for (int u = 0; u < S::kUnroll; ++u)
      LoadNarrowAAt<M, S::kUnroll, false, false, kPairA, true>(u, p, arow, r0, static_cast<int>(ke), bx);
    ComputeNarrowBatch<M, S::kUnroll, false, false, true>(bx, r0, static_cast<int>(ke), zc, acc);
  }
  const int ke32 = static_cast<int>(ke);
  const int kw32 = static_cast<int>(kw);
  // Whole batches (every row below ke, a workgroup-uniform test) issue all their loads at
  // once and skip the clamps and selects. The last, partial batch goes half a batch at a
  // time and stops where the rows end, so its clamped form does not raise the register count
  // of the kernel (which sets how many workgroups share a CU) and a short K waits on memory
  // once or twice. sched_barrier keeps the scheduler from moving conversions between
  // the loads, which would make each load wait for the one before it.
  constexpr int kTailUnroll = S::kUnroll / 2;
  static_assert(S::kUnroll % kTailUnroll == 0, "tail steps");
  for (int r0 = static_cast<int>(kb) + 2 * tid; kAOp == kAOpNone && r0 - 2 * tid < ke32;
       r0 += static_cast<int>(S::kBatchRows)) {
    if (r0 - 2 * tid + static_cast<int>(S::kBatchRows) <= ke32) {
      NarrowBatch<M, S::kUnroll> bx;
      LoadNarrowBatch<M, S::kUnroll, kZero, kRowScale, kPairA, false>(p, arow, r0, ke32, kw32, tbase, bx);
      __builtin_amdgcn_sched_barrier(0);
      ComputeNarrowBatch<M, S::kUnroll, kZero, kRowScale, false>(bx, r0, ke32, zc, acc);
    } else {
#pragma unroll 1
      for (int u = 0; u < S::kUnroll; u += kTailUnroll) {
        const int rt = r0 + u * static_cast<int>(S::kStepRows);
        if (rt - 2 * tid >= ke32) break;  // the rest of the batch lies past ke (workgroup-uniform)
        NarrowBatch<M, kTailUnroll> bt;
        LoadNarrowBatch<M, kTailUnroll, kZero, kRowScale, kPairA, true>(p, arow, rt, ke32, kw32, tbase, bt);
        __builtin_amdgcn_sched_barrier(0);
        ComputeNarrowBatch<M, kTailUnroll, kZero, kRowScale, true>(bt, rt, ke32, zc, acc);
      }
    }
  }

#pragma unroll
  for (int mm = 0; mm < M; ++mm) {
    const float v = WaveColumnSum8(acc[mm], lane);
    if ((lane & 7) == 0) red[wave][mm][lane >> 3] = v;
  }
  __syncthreads();
  if (tile_live && tid < M * kNarrowTile) {
    const int mm = tid / kNarrowTile;
    const int c = tid % kNarrowTile;
    const int64_t col = col0 + c;
    if (mm < m && col < n) {
      float s = red[0][mm][c];
      for (int wv = 1; wv < S::kWaves; ++wv) s = s + red[wv][mm][c];
      if (p.splits > 1) {
        p.partials[(static_cast<int64_t>(split) * m + mm) * n + col] = s;
      } else {
        const float cs = p.mode == kScalePerRow ? 1.f : col_scale;
        StoreC(p.c, mm, col, n, p.epi, ApplyEpilogue(__fmul_rn(s, cs), mm, col, n, p.epi));
      }
    }
  }
}

// The m = 1 product on staged tiles with k <= 4096 (one batch), no zero points and no per-row
// scale: the headline shape and the decode GEMVs without an input prologue. The arithmetic is
// GemvNarrowKernel<1>'s (the same load, compute and reduction helpers), so both kernels store
// the same bits. What differs is the entry and the exit. The pointers and sizes come first
// among the arguments and nothing branches on an argument before the weight loads are
// issued (the general kernel reads its fields from one argument struct, and the compiler
// spreads those reads over three or four dependent rounds ahead of the first weight load).
// The epilogue's arguments, bias and residual values are read while the weight loads are in
// flight instead of after the sums, so the last workgroup's store waits for no memory. The
// leading 14 argument dwords (the pointers, c among them, the sizes, `second` the input
// transform's second operand) are preloaded into SGPRs at wave launch, so every load a step
// needs and the store issue without waiting for the kernarg segment (a late scalar load of c
// cost about 1 % of the 4096 x 14336 product); the epilogue and the prologue are read behind
// them. With
// an input prologue (kAOp) the weight loads are issued first, the transformed row is staged
// in LDS (StageInputRow) while they are in flight, and A is read from there.
// kWaves: 4, or 8 for a single step (k <= 1024): every lane then forms at most one row pair
// of the input transform, where 4 waves would form a second, mostly clamped, one.
template <int kSteps, bool kClamp, bool kPlain, int kAOp, bool kCached, int kWaves = NarrowShape<1>::kWaves>
__global__ __launch_bounds__(64 * kWaves)
__attribute__((amdgpu_waves_per_eu(NarrowMinWaves<1, false, false, kAOp>()))) void GemvM1Kernel(
    const int8_t* tiled, const float* a, const float* scale, float* c, int32_t k, int32_t n, const float* second,
    int32_t scale_index_mul, int32_t attn_splits, Epilogue epi, GemvPrologue pro) {
  using S = NarrowShape<1>;
  static_assert(kSteps >= 1 && kSteps <= S::kUnroll, "one batch");
  // The load helpers step by S::kStepRows (4 waves); a wider workgroup takes one step only.
  static_assert(kWaves == S::kWaves || (kSteps == 1 && kWaves == 8 && kAOp != kAOpRms), "8 waves: one step");
  __shared__ float red[kWaves][kNarrowTile];
  __shared__ __align__(16) float a_stage[kAOp == kAOpRms ? kGemvPrologueMaxK : 1];  // the staged row
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tiles = (n + kNarrowTile - 1) / kNarrowTile;  // the launcher's tile count and grid
  const int tiles_per_xcd = (tiles + kXcds - 1) / kXcds;
  const int tile_raw = (blockIdx.x % kXcds) * tiles_per_xcd + blockIdx.x / kXcds;
  const bool tile_live = tile_raw < tiles;
  const int tile = tile_live ? tile_raw : tiles - 1;
  const int8_t* tbase = tiled + static_cast<int64_t>(tile) * k * kNarrowTile;  // k is even
  const int col = tile * kNarrowTile + (tid & 7);
  const int colc = col < n ? col : n - 1;
  // Per-column scale: index col (scale_index_mul 1); whole tensor: the launcher points scale at
  // the tensor's one value (mul 0).
  const float col_scale = scale[scale_index_mul * colc];
  const GemvArgs unused{};
  NarrowBatch<1, kSteps> b;
  double ss = 0.0;  // kAOpRmsAfter: this lane's share of sum(double(x)^2)
  if (kAOp == kAOpNone) {
    const float* const arow[1] = {a};
    LoadNarrowBatch<1, kSteps, false, false, true, kClamp, kCached>(unused, arow, 2 * tid, k, k, tbase, b);
  } else if (kAOp == kAOpRmsAfter || kAOp == kAOpSiluUp || kAOp == kAOpMul) {
    // Elementwise inputs: each lane forms its own A pairs from x and the second operand (the
    // norm weight, or up for SiLU*up), with no LDS stage and no barrier.
#pragma unroll
    for (int u = 0; u < kSteps; ++u) LoadNarrowWAt<1, kSteps, kClamp, kCached>(u, 2 * tid, k, tbase, b);
    float2 xv[kSteps], wv[kSteps];
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const int r = 2 * tid + u * static_cast<int>(S::kStepRows);
      const int rp = !kClamp || r < k - 2 ? r : k - 2;  // k is even: the pair is whole
      xv[u] = *reinterpret_cast<const float2*>(a + rp);
      wv[u] = *reinterpret_cast<const float2*>(second + rp);
    }
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const int r = 2 * tid + u * static_cast<int>(S::kStepRows);
      if (kAOp == kAOpRmsAfter) {
        b.a[u][0][0] = __fmul_rn(xv[u].x, wv[u].x);
        b.a[u][0][1] = __fmul_rn(xv[u].y, wv[u].y);
        if (!kClamp || r < k) {
          ss += static_cast<double>(xv[u].x) * static_cast<double>(xv[u].x);
          ss += static_cast<double>(xv[u].y) * static_cast<double>(xv[u].y);
        }
      } else if (kAOp == kAOpMul) {
        b.a[u][0][0] = __fmul_rn(xv[u].x, wv[u].x);
        b.a[u][0][1] = __fmul_rn(xv[u].y, wv[u].y);
      } else {  // SiluMulKernel's formula
        b.a[u][0][0] = __fmul_rn(__fdiv_rn(xv[u].x, __fadd_rn(1.f, expf(-xv[u].x))), wv[u].x);
        b.a[u][0][1] = __fmul_rn(__fdiv_rn(xv[u].y, __fadd_rn(1.f, expf(-xv[u].y))), wv[u].y);
      }
    }
  } else if (kAOp == kAOpAttn) {
    // The attention combine per lane (AttnCombinePair): its pairs' partials are loaded with
    // the weights, so the row costs no extra memory round and no barrier.
#pragma unroll
    for (int u = 0; u < kSteps; ++u) LoadNarrowWAt<1, kSteps, kClamp, kCached>(u, 2 * tid, k, tbase, b);
    constexpr int kStride = 2 + kAttnDim;
    const int splits = attn_splits;
    if (splits == kAttnRegSplits) {
      // Eight splits: the weights are formed once per 8-lane group (AttnCombinePairLanes). The
      // groups never mix heads or live and clamped rows: k is 64 x heads, so a head's 32 pairs
      // and the live pairs both end on a multiple of 8 lanes.
      float2 mls[kSteps], ac[kSteps][kAttnRegSplits];
#pragma unroll
      for (int u = 0; u < kSteps; ++u) {
        const int r = 2 * tid + u * static_cast<int>(S::kStepRows);
        const int rp = !kClamp || r < k - 2 ? r : k - 2;  // k is even: the pair is whole, in one head
        const float* head = second + (rp / kAttnDim) * kAttnRegSplits * kStride;
        mls[u] = *reinterpret_cast<const float2*>(head + (lane & 7) * kStride);
#pragma unroll
        for (int sp = 0; sp < kAttnRegSplits; ++sp)
          ac[u][sp] = *reinterpret_cast<const float2*>(head + sp * kStride + 2 + rp % kAttnDim);
      }
#pragma unroll
      for (int u = 0; u < kSteps; ++u) AttnCombinePairLanes(mls[u], ac[u], b.a[u][0][0], b.a[u][0][1]);
    } else {
      float2 ml[kSteps][kAttnRegSplits], ac[kSteps][kAttnRegSplits];
#pragma unroll
      for (int u = 0; u < kSteps; ++u) {
        const int r = 2 * tid + u * static_cast<int>(S::kStepRows);
        const int rp = !kClamp || r < k - 2 ? r : k - 2;  // k is even: the pair is whole, in one head
        const float* head = second + (rp / kAttnDim) * splits * kStride;
#pragma unroll
        for (int sp = 0; sp < kAttnRegSplits; ++sp) {
          ml[u][sp] = *reinterpret_cast<const float2*>(head + sp * kStride);
          ac[u][sp] = *reinterpret_cast<const float2*>(head + sp * kStride + 2 + rp % kAttnDim);
        }
      }
#pragma unroll
      for (int u = 0; u < kSteps; ++u) {
        const int r = 2 * tid + u * static_cast<int>(S::kStepRows);
        const int rp = !kClamp || r < k - 2 ? r : k - 2;
        AttnCombinePair(second, splits, rp / kAttnDim, rp % kAttnDim, ml[u], ac[u], b.a[u][0][0],
                        b.a[u][0][1]);
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < kSteps; ++u) LoadNarrowWAt<1, kSteps, kClamp, kCached>(u, 2 * tid, k, tbase, b);
    __shared__ double part[S::kWaves];
    GemvArgs staged{};
    staged.a = a;
    staged.k = k;
    staged.pro = pro;
    StageInputRow<kAOp, S::kThreads>(staged, a_stage, part);
    const float* const srow[1] = {a_stage};
#pragma unroll
    for (int u = 0; u < kSteps; ++u) LoadNarrowAAt<1, kSteps, false, false, true, kClamp>(u, unused, srow, 2 * tid, k, b);
  }
  __builtin_amdgcn_sched_barrier(0);
  // The norm's eps (not among the preloaded arguments) is read now, behind the loads, not
  // where the norm factor needs it.
  if constexpr (kAOp == kAOpRmsAfter) asm volatile("" ::"s"(pro.rms_eps));
  float bias_v = 0.f;
  float res_v = 0.f;
  if (!kPlain) {
    if (epi.bias != nullptr) bias_v = epi.bias[BiasIndex(epi, 0, colc)];
    if (epi.residual != nullptr) res_v = epi.residual[colc];
    asm volatile("" ::"s"(epi.alpha), "s"(epi.beta), "s"(epi.activation), "s"(epi.split[0]), "s"(epi.split[1]),
                 "s"(epi.c2), "s"(epi.c3));
  }
  float acc[1][kNarrowTile];
  float zc[kNarrowTile];
#pragma unroll
  for (int cc = 0; cc < kNarrowTile; ++cc) {
    acc[0][cc] = 0.f;
    zc[cc] = 0.f;
  }
  ComputeNarrowBatch<1, kSteps, false, false, kClamp>(b, 2 * tid, k, zc, acc);
  const float v = WaveColumnSum8(acc[0], lane);
  if ((lane & 7) == 0) red[wave][lane >> 3] = v;
  __shared__ double ss_part[kWaves];
  if (kAOp == kAOpRmsAfter) {
    const double w_ss = WaveButterfly(ss, [](double x, double y) { return x + y; });
    if (lane == 0) ss_part[wave] = w_ss;
  }
  __syncthreads();
  [[maybe_unused]] float out = 0.f;
  [[maybe_unused]] uint64_t key = 0;
  if (tile_live && tid < kNarrowTile && col < n) {
    float sum = red[0][tid];
#pragma unroll
    for (int wv = 1; wv < kWaves; ++wv) sum = sum + red[wv][tid];
    if (kAOp == kAOpRmsAfter) {
      double total = ss_part[0];
#pragma unroll
      for (int wv = 1; wv < kWaves; ++wv) total += ss_part[wv];
      const double inv = 1.0 / sqrt(total / static_cast<double>(k) + static_cast<double>(pro.rms_eps));
      sum = __fmul_rn(sum, static_cast<float>(inv));
    }
    const float x = __fmul_rn(sum, col_scale);
    if (kPlain) {
      c[col] = x;
    } else {
      out = ApplyEpilogueLoaded(x, epi, bias_v, res_v);
      if constexpr (kAOp == kAOpRmsAfter) {
        if (pro.silu_split0 && col < epi.split[0]) out = __fdiv_rn(out, __fadd_rn(1.f, expf(-out)));
      }
      StoreC(c, 0, col, n, epi, out);
      if constexpr (kAOp == kAOpNone) key = GreedyKey(out, static_cast<uint32_t>(col));
    }
  }
  if constexpr (!kPlain && kAOp == kAOpNone) {
    // Side outputs (GemvPrologue): the tile's largest greedy key, from lanes 0..7 of wave 0
    // (the other lanes hold key 0 and only lanes 0..7 meet in the xor 4, 2, 1 exchanges), and
    // the decode loop's advance.
    if (pro.greedy_keys != nullptr && wave == 0) {
      key = max(key, XorLane<4>(key));
      key = max(key, XorLane<2>(key));
      key = max(key, XorLane<1>(key));
      if (lane == 0 && tile_live) pro.greedy_keys[tile] = key;
    }
    if (pro.advance != nullptr && blockIdx.x == 0 && tid == 0) {
      pro.advance[0] = pro.advance[0] + 1;
      pro.advance[1] = pro.advance[1] + 1;
    }
  }
}

// ---- one wave per tile: m = 1, a wide product with a short k (the LM head) -------------------
// Each wave owns one staged 8-column tile over all of k (k <= 1024: at most 8 row pairs a
// lane, all loads issued first), four tiles a workgroup, and its 8 column sums meet inside the
// wave (WaveColumnSum8): no LDS stage and no barrier. For 576 x 49152 the 6144 tiles take
// 1536 workgroups, all resident at once, where one workgroup per tile took three rounds of
// resident workgroups of 4.6 KB each. Identity epilogue; with kSide the side outputs of
// GemvPrologue (the tile's greedy key from lanes 0, 8, .., 56, which hold its 8 stored
// values, and workgroup 0's advance). A lane adds its row pairs in order, then the wave sums:
// another association than GemvM1Kernel's (rounding only). kRms: the RMSNorm after the
// product (GemvPrologue::rms_after, weight `second`): every wave holds the whole row, so it
// reduces the double sum of squares itself (no barrier) and scales its sums by float(1/rms).
constexpr int kWaveTileWaves = 4;

template <int kLoads, bool kCached, bool kSide, bool kRms>
__global__ __launch_bounds__(64 * kWaveTileWaves) void GemvWaveTileKernel(const int8_t* tiled, const float* a,
                                                                          const float* second, const float* scale,
                                                                          int32_t k, int32_t n,
                                                                          int32_t scale_index_mul, int32_t const_index,
                                                                          float* c, GemvPrologue pro) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tiles = (n + kNarrowTile - 1) / kNarrowTile;
  const int groups = (tiles + kWaveTileWaves - 1) / kWaveTileWaves;
  const int groups_per_xcd = (groups + kXcds - 1) / kXcds;
  const int group = (blockIdx.x % kXcds) * groups_per_xcd + blockIdx.x / kXcds;
  const int tile_raw = group * kWaveTileWaves + wave;
  const bool tile_live = tile_raw < tiles;
  const int tile = tile_live ? tile_raw : tiles - 1;
  const int8_t* tbase = tiled + static_cast<int64_t>(tile) * k * kNarrowTile;  // k is even
  u32x4 w[kLoads];
  float2 x[kLoads];
  [[maybe_unused]] float2 g[kLoads];
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const int r = 2 * (lane + 64 * j);
    const int rw = r < k - 2 ? r : k - 2;
    const u32x4* at = reinterpret_cast<const u32x4*>(tbase + static_cast<uint32_t>(rw) * 8u);
    if constexpr (kCached)
      w[j] = *at;
    else
      w[j] = __builtin_nontemporal_load(at);
    x[j] = *reinterpret_cast<const float2*>(a + rw);
    if constexpr (kRms) g[j] = *reinterpret_cast<const float2*>(second + rw);
  }
  const int col = tile * kNarrowTile + (lane >> 3);
  const int colc = col < n ? col : n - 1;
  const float col_scale = scale[scale_index_mul * colc + const_index];
  asm volatile("" ::"s"(c));
  if constexpr (kRms) asm volatile("" ::"s"(pro.rms_eps));
  __builtin_amdgcn_sched_barrier(0);
  float acc[kNarrowTile];
#pragma unroll
  for (int cc = 0; cc < kNarrowTile; ++cc) acc[cc] = 0.f;
  [[maybe_unused]] double ss = 0.0;  // kRms: this lane's share of sum(double(x)^2)
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const bool live = 2 * (lane + 64 * j) < k;
    float x0 = live ? x[j].x : 0.f;
    float x1 = live ? x[j].y : 0.f;
    if constexpr (kRms) {
      ss += static_cast<double>(x0) * static_cast<double>(x0);
      ss += static_cast<double>(x1) * static_cast<double>(x1);
      x0 = __fmul_rn(x0, g[j].x);
      x1 = __fmul_rn(x1, g[j].y);
    }
#pragma unroll
    for (int cc = 0; cc < kNarrowTile; ++cc) {
      acc[cc] = __builtin_fmaf(x0, ByteToFloat(w[j][cc >> 2], cc & 3), acc[cc]);
      acc[cc] = __builtin_fmaf(x1, ByteToFloat(w[j][2 + (cc >> 2)], cc & 3), acc[cc]);
    }
  }
  float v = WaveColumnSum8(acc, lane);
  if constexpr (kRms) {
    const double total = WaveButterfly(ss, [](double p, double q) { return p + q; });
    const double inv = 1.0 / sqrt(total / static_cast<double>(k) + static_cast<double>(pro.rms_eps));
    v = __fmul_rn(v, static_cast<float>(inv));
  }
  const bool store = tile_live && (lane & 7) == 0 && col < n;
  const float out = __fmul_rn(v, col_scale);
  if (store) c[col] = out;
  if constexpr (kSide) {
    if (pro.greedy_keys != nullptr) {
      uint64_t key = store ? GreedyKey(out, static_cast<uint32_t>(col)) : 0;
      key = max(key, XorLane<8>(key));
      key = max(key, XorLane<16>(key));
      key = max(key, XorLane<32>(key));
      if (lane == 0 && tile_live) pro.greedy_keys[tile] = key;
    }
    if (pro.advance != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
      pro.advance[0] = pro.advance[0] + 1;
      pro.advance[1] = pro.advance[1] + 1;
    }
  }
}

// ---- wide kernel: 4 < m <= 16 ----------------------------------------------------------------
constexpr int kWideThreads = 256;
constexpr int kWideWaves = kWideThreads / 64;
constexpr int kWideTile = 256;
constexpr int kWideMaxRows = 1024;
constexpr int kWideUnroll = 4;

// One step of the wide kernel: row group g = g0 + u * waves holds rows 4g .. 4g + 3, lane row
// l / 16 of it; rows past `rows` read a clamped row and are zeroed through A.
template <bool kVec>
__device__ __forceinline__ void WideLoad(const GemvArgs& p, const int8_t* wbase, int64_t col, int rows, int groups,
                                         int g0, int lane_row, uint4 (&w)[kWideUnroll]) {
#pragma unroll
  for (int u = 0; u < kWideUnroll; ++u) {
    const int g = g0 + u * kWideWaves;
    const int r = g * 4 + lane_row;
    const bool valid = g < groups && r < rows;
    const int rc = valid ? r : rows - 1;
    w[u] = LoadRow16<kVec>(wbase + static_cast<int64_t>(rc) * p.n, col, p.n, valid);
  }
}

template <bool kZero, bool kRowScale>
__device__ __forceinline__ void WideStep(const GemvArgs& p, const float* smem, int64_t k0, int rows, int groups, int g0,
                                         int lane_row, int lane_col, const float (&zc)[16],
                                         const uint4 (&w)[kWideUnroll], v4f (&acc)[16]) {
#pragma unroll
  for (int u = 0; u < kWideUnroll; ++u) {
    const int g = g0 + u * kWideWaves;
    const int r = g * 4 + lane_row;
    const bool valid = g < groups && r < rows;
    const int rc = valid ? r : rows - 1;
    const float a = smem[rc * 16 + lane_col];  // A[l % 16][row of l]
    const float av = valid ? a : 0.f;
    const float zr = (kZero && kRowScale) ? static_cast<float>(p.zero[k0 + rc]) : 0.f;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float b = ByteToFloat(Word(w[u], t >> 2), t & 3);
      if (kZero) b = b - (zc[t] + zr);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b, acc[t], 0, 0, 0);
    }
  }
}

template <bool kVec, bool kZero, bool kRowScale>
__global__ __launch_bounds__(kWideThreads) void GemvWideKernel(GemvArgs p) {
  __shared__ __align__(16) float smem[16 * kWideMaxRows];  // A stage [row][16]; reused for the wave sums
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tile = blockIdx.x;
  if (tile >= p.tiles) return;
  const int split = blockIdx.y;
  const int64_t k0 = static_cast<int64_t>(split) * p.rows_per_split;
  const int rows = static_cast<int>(min(p.rows_per_split, p.k - k0));

  // A stage: smem[r * 16 + mm] = A[mm][k0 + r] (times the row's scale when per-row), 0 for
  // mm >= m. Thread r reads its row's 16 values down A's columns (consecutive threads,
  // consecutive addresses) and issues all of them before storing any, so the stage costs one
  // memory round trip per 256 rows instead of one per element.
  for (int r0 = 0; r0 < rows; r0 += kWideThreads) {
    const int r = r0 + tid;
    const int rc = r < rows ? r : rows - 1;
    float v[16];
#pragma unroll
    for (int mm = 0; mm < 16; ++mm) {
      const int64_t mc = mm < p.m ? mm : p.m - 1;  // a valid row; zeroed below
      v[mm] = p.a[mc * p.k + k0 + rc];
    }
    const float rs = kRowScale ? p.scale[k0 + rc] : 1.f;
    if (r < rows) {
#pragma unroll
      for (int mm = 0; mm < 16; mm += 4) {
        float4 q;
        q.x = mm + 0 < p.m ? (kRowScale ? __fmul_rn(v[mm + 0], rs) : v[mm + 0]) : 0.f;
        q.y = mm + 1 < p.m ? (kRowScale ? __fmul_rn(v[mm + 1], rs) : v[mm + 1]) : 0.f;
        q.z = mm + 2 < p.m ? (kRowScale ? __fmul_rn(v[mm + 2], rs) : v[mm + 2]) : 0.f;
        q.w = mm + 3 < p.m ? (kRowScale ? __fmul_rn(v[mm + 3], rs) : v[mm + 3]) : 0.f;
        *reinterpret_cast<float4*>(&smem[r * 16 + mm]) = q;
      }
    }
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
  // The next step's rows are requested before this step's MFMAs (one set in flight while
  // one is multiplied).
  constexpr int kStride = kWideWaves * kWideUnroll;
  uint4 wn[kWideUnroll];
  WideLoad<kVec>(p, wbase, col, rows, groups, wave, lane_row, wn);
  for (int g0 = wave; g0 < groups; g0 += kStride) {
    uint4 w[kWideUnroll];
#pragma unroll
    for (int u = 0; u < kWideUnroll; ++u) w[u] = wn[u];
    if (g0 + kStride < groups) WideLoad<kVec>(p, wbase, col, rows, groups, g0 + kStride, lane_row, wn);
    WideStep<kZero, kRowScale>(p, smem, k0, rows, groups, g0, lane_row, lane_col, zc, w, acc);
  }
  __syncthreads();  // A stage done; smem becomes [wave][16][kWideTile]
  // Lane l holds m = 4*(l/16) + r, column 16*(l%16) + t.
  for (int r = 0; r < 4; ++r)
    for (int t = 0; t < 16; ++t) smem[(wave * 16 + 4 * lane_row + r) * kWideTile + lane_col * 16 + t] = acc[t][r];
  __syncthreads();
  const int64_t out_col = static_cast<int64_t>(tile) * kWideTile + tid;
  if (out_col >= p.n) return;
  // All 16 rows' wave sums are read at once (one LDS round trip), then stored.
  float sums[16];
#pragma unroll
  for (int mm = 0; mm < 16; ++mm) {
    float s = smem[mm * kWideTile + tid];
#pragma unroll
    for (int wv = 1; wv < kWideWaves; ++wv) s = s + smem[(wv * 16 + mm) * kWideTile + tid];
    sums[mm] = s;
  }
  if (p.splits > 1) {
    float* dst = p.partials + static_cast<int64_t>(split) * p.m * p.n + out_col;
#pragma unroll
    for (int mm = 0; mm < 16; ++mm)
      if (mm < p.m) dst[mm * p.n] = sums[mm];
    return;  // SplitReduceKernel applies the scale and the epilogue
  }
#pragma unroll
  for (int mm = 0; mm < 16; ++mm)
    if (mm < p.m) Emit(p, split, mm, out_col, sums[mm]);
}

// ---- split-bf16 MFMA kernel: 1 < m <= 16, group-interleaved tiles, k a multiple of 32 ---------
// The products run on v_mfma_f32_16x16x32_bf16 (A: 16 rows x 32 k, B: 32 k x 16 columns)
// without rounding either operand:
//  * every weight byte is an integer in [-128, 127], which bf16 holds exactly;
//  * every activation x is split as x = hi + mid + lo with hi = bf16(x), mid = bf16(x - hi),
//    lo = bf16(x - hi - mid); both differences are exact in fp32 and the three parts carry all
//    24 significand bits of x (for |x| >= 2^-110; below that the last part may lose bits), so
//    three MFMAs multiply by x exactly and only the fp32 accumulation rounds.
// A workgroup (4 waves) owns one group of 16 staged tiles (128 columns) over one split of K.
// Lane l takes tile slot l % 16 as the B column of its MFMAs and, for the 8 columns c of that
// tile, the operand of the c-th MFMA. A 32-row block is read as 4 loads of 16 bytes per lane:
// load h of lane group g = l / 16 holds rows 8g + 2h and 8g + 2h + 1 of the tile (one load of
// the wave is 1 KB of the staged copy), so lane group g's four loads are rows 8g .. 8g + 7
// and A lane (row l % 16, group g) reads those 8 activations as two 16-byte loads; the k
// slots agree. The waves take interleaved blocks, and their sums are added
// through LDS in wave order. With splits, each workgroup stores its partial sums and the last
// one of a group to arrive adds them in split order and applies the scale and the epilogue.
constexpr int kSplitWaves = 4;
constexpr int kSplitThreads = kSplitWaves * 64;
constexpr int kSplitTiles = static_cast<int>(kGemvGroupTiles);      // tiles of a group (128 columns)
constexpr int kSplitBlockRows = static_cast<int>(kGemvGroupRows);  // K of one MFMA
constexpr int kSplitBatch = 2;  // blocks a wave loads before using any
constexpr int kSplitGroupBytes = kSplitTiles * kNarrowTile;  // bytes of one row of a group

// One 32-row block of a lane: its four weight loads w (rows 8g + 2h, 8g + 2h + 1 of its tile
// in load h) and its 8 activations x (rows 8g .. 8g + 7) into the 8 accumulators, hi, then
// mid, then lo parts.
__device__ __forceinline__ void SplitBf16Block(const u32x4 (&w)[4], const f32x2 (&x)[4], v4f (&acc)[kNarrowTile]) {
  u32x4 ah, am, al;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const float x0 = x[h][0];
    const float x1 = x[h][1];
    ah[h] = PackBf16(x0, x1);
    const float r0 = x0 - Bf16Low(ah[h]);
    const float r1 = x1 - Bf16High(ah[h]);
    am[h] = PackBf16(r0, r1);
    al[h] = PackBf16(r0 - Bf16Low(am[h]), r1 - Bf16High(am[h]));
  }
  // Column c of the tile: row 8g + 2h in byte c of words 0..1 of load h, row 8g + 2h + 1 in
  // words 2..3.
  u32x4 bw[kNarrowTile];
#pragma unroll
  for (int c = 0; c < kNarrowTile; ++c)
#pragma unroll
    for (int h = 0; h < 4; ++h)
      bw[c][h] = PackBf16(ByteToFloat(w[h][c >> 2], c & 3), ByteToFloat(w[h][2 + (c >> 2)], c & 3));
#pragma unroll
  for (int c = 0; c < kNarrowTile; ++c)
    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah), __builtin_bit_cast(bf16x8, bw[c]),
                                                     acc[c], 0, 0, 0);
#pragma unroll
  for (int c = 0; c < kNarrowTile; ++c)
    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, am), __builtin_bit_cast(bf16x8, bw[c]),
                                                     acc[c], 0, 0, 0);
#pragma unroll
  for (int c = 0; c < kNarrowTile; ++c)
    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al), __builtin_bit_cast(bf16x8, bw[c]),
                                                     acc[c], 0, 0, 0);
}

// The end of a split-bf16 workgroup: the waves' accumulators meet in LDS (`red`, wave order),
// then either the group's sums are scaled and stored, or, with K splits, this split's partial
// sums are stored and the last workgroup of the group to arrive adds the splits in split order.
template <bool kPlain>
__device__ __forceinline__ void SplitBf16Finish(const GemvArgs& p, int32_t m, int32_t splits, float* partials,
                                                uint32_t* arrivals, const v4f (&acc)[kNarrowTile],
                                                float (*red)[32][65], bool* is_last_flag, int group, int split) {
  bool& is_last = *is_last_flag;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Element r of MFMA c in lane l: row 4 * (l / 16) + r, column 8 * (16 * group + l % 16) + c.
#pragma unroll
  for (int c = 0; c < kNarrowTile; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * c + r][lane] = acc[c][r];
  __syncthreads();
  // Thread: one column of the group, rows 8 * (tid / 128) .. + 7.
  const int cc = tid & (kSplitGroupBytes - 1);
  const int jt = cc >> 3;
  const int c = cc & 7;
  const int64_t col = static_cast<int64_t>(group * kSplitTiles + jt) * kNarrowTile + c;
  const int m0 = (tid >> 7) * 8;
  const int mend = min(m, m0 + 8);
  float sum[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int mm = m0 + i;
    const int ln = 16 * (mm >> 2) + jt;
    const int ri = 4 * c + (mm & 3);
    float s = red[0][ri][ln];
#pragma unroll
    for (int wv = 1; wv < kSplitWaves; ++wv) s = s + red[wv][ri][ln];
    sum[i] = s;
  }
  const bool live_col = col < p.n;
  if (splits > 1) {
    // Partial sums out (agent scope: the last workgroup, on any XCD, reads them), then the
    // arrival count of the group. Split sp's [m, n] block starts at the uniform (scalar)
    // offset sp * m * n; rows within it are 32-bit offsets (the launcher checks m * n < 2^31).
    const int n32 = static_cast<int>(p.n);
    const int64_t split_stride = static_cast<int64_t>(m) * p.n;
    float* part = partials + col;
    float* mine = part + split * split_stride;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (live_col && m0 + i < mend)
        __hip_atomic_store(&mine[(m0 + i) * n32], sum[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) is_last = atomicAdd(&arrivals[group], 1u) == static_cast<uint32_t>(splits - 1);
    __syncthreads();
    if (!is_last) return;
    if (tid == 0) atomicExch(&arrivals[group], 0u);  // ready for the next launch
    if (!live_col || m0 >= mend) return;
    // The splits' sums in split order; kChunk splits of all 8 rows are requested at once
    // (clamped to valid rows and splits; the extra values are not used).
    constexpr int kChunk = 4;
    for (int sp0 = 0; sp0 < splits; sp0 += kChunk) {
      float v[kChunk][8];
#pragma unroll
      for (int t = 0; t < kChunk; ++t)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int sp = min(sp0 + t, splits - 1);
          const int mm = min(m0 + i, mend - 1);
          v[t][i] = __hip_atomic_load(&part[sp * split_stride + mm * n32], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
      for (int t = 0; t < kChunk; ++t)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (sp0 + t < splits) sum[i] = sp0 + t == 0 ? v[t][i] : sum[i] + v[t][i];
    }
  }
  if (!live_col) return;
  const float cs = ColScale(p, col);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int mm = m0 + i;
    if (mm >= mend) break;
    if (kPlain) p.c[mm * static_cast<int>(p.n) + col] = __fmul_rn(sum[i], cs);
    else StoreC(p.c, mm, col, p.n, p.epi, ApplyEpilogue(__fmul_rn(sum[i], cs), mm, col, p.n, p.epi));
  }
}

// kPlain: the epilogue is the identity and C one [m, n] matrix, so each sum is stored as
// sum * scale with no epilogue code (which costs about 1 us of the m = 16 kernel's tail).
// What the loads and the arrival need leads the arguments (13 dwords, preloaded into SGPRs
// at wave launch, so the first weight loads issue without a kernarg round trip); the
// epilogue's fields are read from `p` behind the loads.
// Grid: one dimension, `slots` workgroups (a multiple of 8); the workgroups of one XCD
// (blockIdx.x % 8) take consecutive (group, split) pairs, so the splits of a group and
// neighbouring groups run on one XCD; slots past groups x splits exit at once.
// Rows m .. 15 of the MFMA tile are lanes that read row m - 1's activations; their sums are
// never stored, so they need no zeroing.
template <bool kPlain>
__global__ __launch_bounds__(kSplitThreads) void GemvSplitBf16Kernel(const int8_t* grouped, const float* a,
                                                                     float* partials, uint32_t* arrivals, int32_t m,
                                                                     int32_t k, int32_t rows_per_split, int32_t splits,
                                                                     int32_t group_pairs, GemvArgs p) {
  __shared__ float red[kSplitWaves][32][65];  // [wave][4 * column + row of the MFMA tile][lane]
  __shared__ bool is_last;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slot = lane & 15;  // B column slot (tile) and A row
  const int g = lane >> 4;     // k group
  const int per_xcd = static_cast<int>(gridDim.x / kXcds);
  const int pair = static_cast<int>(blockIdx.x % kXcds) * per_xcd + static_cast<int>(blockIdx.x / kXcds);
  if (pair >= group_pairs) return;
  const int group = pair / splits;
  const int split = pair - group * splits;
  const int64_t kb = static_cast<int64_t>(split) * rows_per_split;
  const int64_t ke = min(static_cast<int64_t>(k), kb + rows_per_split);
  const int blocks = static_cast<int>((ke - kb) / kSplitBlockRows);
  const int8_t* tb = grouped + (static_cast<int64_t>(group) * k + kb) * kSplitGroupBytes + 64 * slot + 16 * g;
  const float* ab = a + static_cast<int64_t>(slot < m ? slot : m - 1) * k + kb + 8 * g;

  v4f acc[kNarrowTile];
#pragma unroll
  for (int c = 0; c < kNarrowTile; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};

  // The wave's blocks wave, wave + 4, ...: whole batches, then the rest one at a time.
  const int nb = blocks > wave ? (blocks - wave + kSplitWaves - 1) / kSplitWaves : 0;
  auto load_block = [&](int j, u32x4 (&w)[4], f32x2 (&x)[4]) {
    const int blk = wave + kSplitWaves * j;
    const u32x4* wb = reinterpret_cast<const u32x4*>(tb + static_cast<int64_t>(blk) * (kSplitBlockRows * kSplitGroupBytes));
    const v4f* xb = reinterpret_cast<const v4f*>(ab + static_cast<int64_t>(blk) * kSplitBlockRows);
#pragma unroll
    for (int h = 0; h < 4; ++h) w[h] = __builtin_nontemporal_load(wb + 64 * h);  // rows 8g + 2h, 8g + 2h + 1
    // This lane's 8 activations of the block, rows 8g .. 8g + 7: two 16-byte loads.
    const v4f x0 = xb[0], x1 = xb[1];
    x[0] = f32x2{x0[0], x0[1]};
    x[1] = f32x2{x0[2], x0[3]};
    x[2] = f32x2{x1[0], x1[1]};
    x[3] = f32x2{x1[2], x1[3]};
  };
  int j = 0;
  for (; j + kSplitBatch <= nb; j += kSplitBatch) {
    u32x4 w[kSplitBatch][4];
    f32x2 x[kSplitBatch][4];
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u) load_block(j + u, w[u], x[u]);
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before any is used
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u) SplitBf16Block(w[u], x[u], acc);
  }
  for (; j < nb; ++j) {
    u32x4 w[4];
    f32x2 x[4];
    load_block(j, w, x);
    SplitBf16Block(w, x, acc);
  }

  SplitBf16Finish<kPlain>(p, m, splits, partials, arrivals, acc, red, &is_last, group, split);
}

// dst (group-interleaved, see StagedGroupBytes) from q [k, n]: one thread writes the 16 bytes
// of one row pair of one tile; consecutive threads write consecutive 16-byte pieces.
__global__ void TileGroupsKernel(const int8_t* q, int64_t k, int64_t n, int8_t* dst, int64_t groups) {
  const int64_t pieces = groups * k * kSplitTiles / 2;
  const bool vec = (n % 8 == 0) && (reinterpret_cast<uintptr_t>(q) % 8 == 0);
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < pieces;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t pair = idx & 3;
    const int64_t j = (idx >> 2) % kSplitTiles;
    const int64_t go = (idx >> 2) / kSplitTiles;  // G * k/8 + o
    const int64_t o = go % (k / 8);
    const int64_t grp = go / (k / 8);
    const int64_t col = (grp * kSplitTiles + j) * kNarrowTile;
    uint32_t w[4] = {0, 0, 0, 0};
    for (int h = 0; h < 2; ++h) {
      // Piece (octet o, pair) of a 32-row block holds rows 8 * pair + 2 * (o % 4) + h of it.
      const int64_t r = 32 * (o >> 2) + 8 * pair + 2 * (o & 3) + h;
      if (vec && col + 7 < n) {
        const uint2 v = *reinterpret_cast<const uint2*>(q + r * n + col);
        w[2 * h] = v.x;
        w[2 * h + 1] = v.y;
      } else {
        for (int b = 0; b < 8; ++b)
          if (col + b < n)
            w[2 * h + (b >> 2)] |= static_cast<uint32_t>(static_cast<uint8_t>(q[r * n + col + b])) << (8 * (b & 3));
      }
    }
    *reinterpret_cast<uint4*>(dst + idx * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ---- split-K reduction ----------------------------------------------------------------------
// One thread per output column of a row (blockIdx.y strides over rows): no index division.
// Every load of an element (the first kReduceRegSplits partial sums, the column scale, the bias
// and the residual) is issued before the first add, so an element costs one memory round trip
// instead of one per split pair and one more for the epilogue; the sums are still added in
// split order, so the bits are unchanged.
constexpr int kReduceRegSplits = 8;

__global__ void SplitReduceKernel(const float* partials, int32_t splits, int64_t m, int64_t n, float* c,
                                  int32_t mode, const float* scale, int64_t const_index, Epilogue epi) {
  const int64_t j = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (j >= n) return;
  const int64_t total = m * n;
  const float* sc = nullptr;
  if (scale != nullptr && mode == kScalePerCol) sc = scale + j;
  if (scale != nullptr && mode == kScaleConst) sc = scale + const_index;
  for (int64_t i = blockIdx.y; i < m; i += gridDim.y) {
    const int64_t idx = i * n + j;
    float v[kReduceRegSplits];
#pragma unroll
    for (int sp = 0; sp < kReduceRegSplits; ++sp) v[sp] = sp < splits ? partials[sp * total + idx] : 0.f;
    const float cs = sc != nullptr ? *sc : 1.f;
    const float bias_v = epi.bias != nullptr ? epi.bias[BiasIndex(epi, i, j)] : 0.f;
    const float res_v = epi.residual != nullptr ? epi.residual[idx] : 0.f;
    float s = v[0];
#pragma unroll
    for (int sp = 1; sp < kReduceRegSplits; ++sp)
      if (sp < splits) s = s + v[sp];
    for (int sp = kReduceRegSplits; sp < splits; ++sp) s = s + partials[static_cast<int64_t>(sp) * total + idx];
    StoreC(c, i, j, n, epi, ApplyEpilogueLoaded(__fmul_rn(s, cs), epi, bias_v, res_v));
  }
}

// dst[(t*kp + r)*8 + c] = q[r*n + 8t + c] (0 past n and in the pad row r = k when k is odd):
// 8-column tiles, each contiguous. One thread writes the 16 bytes of one row pair of one tile;
// consecutive threads take consecutive tiles of the same rows, so the reads of a wave are
// contiguous runs of each row.
__global__ void TileColumnsKernel(const int8_t* q, int64_t k, int64_t n, int8_t* dst, int64_t tiles) {
  const int64_t kp = k + (k & 1);
  const int64_t chunks = tiles * (kp / 2);
  const bool vec = (n % 8 == 0) && (reinterpret_cast<uintptr_t>(q) % 8 == 0);
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < chunks;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = idx % tiles;
    const int64_t rp = idx / tiles;
    const int64_t col = t * kGemvTileCols;
    uint32_t w[4] = {0, 0, 0, 0};
    for (int h = 0; h < 2; ++h) {
      const int64_t r = 2 * rp + h;
      if (r >= k) continue;
      if (vec && col + 7 < n) {
        const uint2 v = *reinterpret_cast<const uint2*>(q + r * n + col);
        w[2 * h] = v.x;
        w[2 * h + 1] = v.y;
      } else {
        for (int b = 0; b < 8; ++b)
          if (col + b < n)
            w[2 * h + (b >> 2)] |= static_cast<uint32_t>(static_cast<uint8_t>(q[r * n + col + b])) << (8 * (b & 3));
      }
    }
    *reinterpret_cast<uint4*>(dst + (t * kp + 2 * rp) * kGemvTileCols) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

}  // namespace

void LaunchTileColumns(const int8_t* q, int64_t k, int64_t n, int8_t* dst, hipStream_t stream) {
  const int64_t tiles = (n + kGemvTileCols - 1) / kGemvTileCols;
  const int64_t chunks = tiles * ((k + 1) / 2);
  int64_t grid = (chunks + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(TileColumnsKernel, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream, q, k, n, dst, tiles);
  Check(hipGetLastError(), "TileColumnsKernel launch");
}

void LaunchTileGroups(const int8_t* q, int64_t k, int64_t n, int8_t* dst, hipStream_t stream) {
  if (k % kGemvGroupRows != 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "group tiles need k % 32 == 0");
  const int64_t groups = (n + kSplitGroupBytes - 1) / kSplitGroupBytes;
  const int64_t pieces = groups * k * kSplitTiles / 2;
  int64_t grid = (pieces + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(TileGroupsKernel, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream, q, k, n, dst, groups);
  Check(hipGetLastError(), "TileGroupsKernel launch");
}

void LaunchSplitReduce(const float* partials, int32_t splits, int64_t m, int64_t n, float* c, int32_t mode,
                       const float* scale, int64_t const_index, const Epilogue& epi, hipStream_t stream) {
  const int64_t gx = (n + 255) / 256;
  const int64_t gy = std::min<int64_t>(m, 65535);
  if (gx > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "split reduction grid too large");
  hipLaunchKernelGGL(SplitReduceKernel, dim3(static_cast<uint32_t>(gx), static_cast<uint32_t>(gy)), dim3(256), 0, stream,
                     partials, splits, m, n, c, mode, scale, const_index, epi);
  Check(hipGetLastError(), "SplitReduceKernel launch");
}

namespace {

template <int M>
// The leading arguments of GemvNarrowKernel (preloaded into SGPRs at wave launch), from `g`.
#define ACCEL_NARROW_LEAD(g)                                                                                   \
  (g).tiled, (g).a, (g).scale, static_cast<int32_t>((g).m), static_cast<int32_t>((g).k),                        \
      static_cast<int32_t>((g).n), (g).tiles, (g).tiles_per_xcd, static_cast<int32_t>((g).rows_per_split)

void LaunchNarrow(const GemvArgs& args, dim3 grid, bool zero, bool row_scale, bool pair_a, hipStream_t stream) {
  const dim3 block(NarrowShape<M>::kThreads);
  switch ((zero ? 4 : 0) | (row_scale ? 2 : 0) | (pair_a ? 1 : 0)) {
#define ACCEL_GEMV_CASE(Z, R, P) \
  case (Z ? 4 : 0) | (R ? 2 : 0) | (P ? 1 : 0): \
    hipLaunchKernelGGL((GemvNarrowKernel<M, Z, R, P>), grid, block, 0, stream, ACCEL_NARROW_LEAD(args), args); \
    break;
    ACCEL_GEMV_CASE(true, true, true) ACCEL_GEMV_CASE(true, true, false) ACCEL_GEMV_CASE(true, false, true)
    ACCEL_GEMV_CASE(true, false, false) ACCEL_GEMV_CASE(false, true, true) ACCEL_GEMV_CASE(false, true, false)
    ACCEL_GEMV_CASE(false, false, true) ACCEL_GEMV_CASE(false, false, false)
#undef ACCEL_GEMV_CASE
  }
}

// The split-bf16 kernel's grid for a k x n product (k a multiple of the 32-row block): column
// groups of 128 and K splits, about 1.75 workgroups per CU (4 splits for 4096 x 14336, measured
// best there; twice the splits costs more in partial sums and arrivals than it gains in
// parallelism), each split at least one batch of every wave.
void SplitBf16Grid(int64_t k, int64_t n, int64_t cus, int64_t* groups, int64_t* splits) {
  const int64_t target = 7 * cus / 4;
  const int64_t tiles = (n + kNarrowTile - 1) / kNarrowTile;
  *groups = (tiles + kSplitTiles - 1) / kSplitTiles;
  const int64_t blocks = k / kSplitBlockRows;
  *splits = std::max<int64_t>(1, std::min<int64_t>((target + *groups - 1) / *groups, blocks / (kSplitWaves * kSplitBatch)));
}

int64_t CuCount() {
  const Context& ctx = Ctx();
  return ctx.cu_count > 0 ? ctx.cu_count : 256;
}

}  // namespace

bool GemvWantsGroups(int64_t m, int64_t k, int64_t n, const Q8View& v) {
  if (m < kGemvGroupMinM || m > 16 || k % kGemvGroupRows != 0 || v.zero != nullptr ||
      (v.mode != kScalePerCol && v.mode != kScaleConst))
    return false;
  if (m > 4) return true;  // the narrow kernel takes m <= 4 only
  int64_t groups = 0, splits = 0;
  SplitBf16Grid(k, n, CuCount(), &groups, &splits);
  return groups * splits >= CuCount();
}

bool GemvWaveTileApplies(int64_t m, int64_t k, int64_t n) {
  const Context& ctx = Ctx();
  const int64_t cus = ctx.cu_count > 0 ? ctx.cu_count : 256;
  return m == 1 && k >= 2 && k <= 1024 && k % 2 == 0 && n < (int64_t(1) << 30) && (n + kNarrowTile - 1) / kNarrowTile >= 8 * cus;
}

void LaunchGemvQ8(const float* a, const Q8View& b, float* c, int64_t m, int64_t k, int64_t n, const Epilogue& epi,
                  hipStream_t stream, const GemvPrologue* prologue) {
  if (m < 1 || m > 16 || k < 1 || n < 1) Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMV shape out of range");
  int a_op = prologue == nullptr                                        ? kAOpNone
                   : prologue->attn_partial != nullptr                     ? kAOpAttn
                   : prologue->rms_weight != nullptr && prologue->rms_after ? kAOpRmsAfter
                   : prologue->rms_weight != nullptr                       ? kAOpRms
                   : prologue->silu_up != nullptr                          ? kAOpSiluUp
                   : prologue->mul_up != nullptr                           ? kAOpMul
                                                                           : kAOpNone;
  static_assert(kGemvPrologueMaxK <= NarrowShape<1>::kBatchRows, "prologue rows fit one batch");
  const bool side = prologue != nullptr && (prologue->greedy_keys != nullptr || prologue->advance != nullptr);
  if (a_op != kAOpNone && (m != 1 || b.tiled == nullptr || b.zero != nullptr || b.mode == kScalePerRow ||
                           k > kGemvPrologueMaxK))
    Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMV input prologue needs m = 1, staged tiles, no zero points, k <= 4096");
  if (a_op == kAOpAttn && (k % kAttnDim != 0 || prologue->attn_splits < kAttnRegSplits ||
                           (k / kAttnDim) * prologue->attn_splits > kAttnMaxPairs))
    Fail(ACCEL_HIP_INVALID_ARGUMENT,
         "GEMV attention prologue needs k = 64 x heads, at least 8 splits and heads x splits <= 2048");
  Context& ctx0 = Ctx();
  const int64_t cus = ctx0.cu_count > 0 ? ctx0.cu_count : 256;
  // The narrow kernel reads the staged column tiles (and indexes rows in 32 bits); without
  // them the wide kernel, which reads W in place, takes any m <= 16.
  const bool zero = b.zero != nullptr;
  const bool row_scale = b.mode == kScalePerRow;
  // The split-bf16 MFMA kernel: group-interleaved copy, whole 32-row blocks, A 16-byte aligned.
  const bool split_bf16 = m > 1 && b.grouped != nullptr && !zero && !row_scale && a_op == kAOpNone &&
                          k % kSplitBlockRows == 0 && k < (int64_t(1) << 28) && m * n <= 0x7fffffff &&
                          reinterpret_cast<uintptr_t>(a) % 16 == 0 && (b.mode == kScalePerCol || b.mode == kScaleConst);
  const bool narrow = !split_bf16 && m <= 4 && b.tiled != nullptr && k < (int64_t(1) << 28);
  if (side && !narrow)
    Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMV greedy keys and advance need the m = 1 kernel (m = 1, staged tiles)");
  const int64_t tile_cols = narrow || split_bf16 ? kNarrowTile : kWideTile;
  const int64_t tiles = (n + tile_cols - 1) / tile_cols;
  int64_t splits = 1;
  int64_t rows = k;
  if (split_bf16) {
    int64_t groups = 0;
    SplitBf16Grid(k, n, cus, &groups, &splits);
    const int64_t blocks = k / kSplitBlockRows;
    rows = (blocks + splits - 1) / splits * kSplitBlockRows;
  } else if (narrow) {
    // One workgroup per tile over all of K, unless the tiles leave the CUs short of work on a
    // K of several batches: then K is split so that about four workgroups run per CU.
    const int64_t step_rows = m == 1 ? NarrowShape<1>::kStepRows : NarrowShape<2>::kStepRows;
    const int64_t batch_rows = m == 1 ? NarrowShape<1>::kBatchRows : NarrowShape<2>::kBatchRows;
    if (tiles < 4 * cus && k >= 2 * batch_rows)
      splits = std::min<int64_t>((4 * cus + tiles - 1) / tiles, k / batch_rows);
    rows = (k + splits - 1) / splits;
    rows = (rows + step_rows - 1) / step_rows * step_rows;
  } else {
    // About 1.75 workgroups per CU (measured best for 4096 x 14336 at m = 16), and no split
    // longer than the A stage.
    splits = std::max<int64_t>((7 * cus / 4 + tiles - 1) / tiles, (k + kWideMaxRows - 1) / kWideMaxRows);
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, (k + 255) / 256));
    rows = (k + splits - 1) / splits;
    rows = std::min<int64_t>((rows + 15) / 16 * 16, kWideMaxRows);
  }
  splits = (k + rows - 1) / rows;
  if (a_op != kAOpNone && splits != 1) Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMV input prologue needs one split");
  const int64_t tiles_per_xcd = (tiles + kXcds - 1) / kXcds;
  if (split_bf16 && (tiles + kSplitTiles - 1) / kSplitTiles > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMV too large");
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
    args.partials = static_cast<float*>(Workspace(static_cast<size_t>(splits * m * n) * sizeof(float)));
  }
  static_assert(kNarrowTile == kGemvTileCols, "staged tiles must match the narrow kernel tile");
  args.tiled = narrow ? b.tiled : nullptr;
  args.grouped = split_bf16 ? b.grouped : nullptr;
  args.arrivals = nullptr;
  if (prologue != nullptr) args.pro = *prologue;
  const dim3 grid(static_cast<uint32_t>(tiles_per_xcd * kXcds), static_cast<uint32_t>(splits));
  if (split_bf16) {
    const int64_t groups = (tiles + kSplitTiles - 1) / kSplitTiles;
    if (splits > 1) args.arrivals = static_cast<uint32_t*>(Temp(kTempArrivals, static_cast<size_t>(groups) * 4));
    const int64_t pairs = groups * splits;
    if (pairs > 0x7ffffff0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMV too large");
    args.group_pairs = static_cast<int32_t>(pairs);
    const dim3 sgrid(static_cast<uint32_t>((pairs + kXcds - 1) / kXcds * kXcds));
    const int32_t m32 = static_cast<int32_t>(m), k32 = static_cast<int32_t>(k), rows32 = static_cast<int32_t>(rows);
    const int32_t splits32 = static_cast<int32_t>(splits), pairs32 = static_cast<int32_t>(pairs);
    if (epi.Identity() && epi.split[0] == 0)
      hipLaunchKernelGGL(GemvSplitBf16Kernel<true>, sgrid, dim3(kSplitThreads), 0, stream, b.grouped, a, args.partials,
                         args.arrivals, m32, k32, rows32, splits32, pairs32, args);
    else
      hipLaunchKernelGGL(GemvSplitBf16Kernel<false>, sgrid, dim3(kSplitThreads), 0, stream, b.grouped, a, args.partials,
                         args.arrivals, m32, k32, rows32, splits32, pairs32, args);
  } else if (narrow) {
    const bool pair_a = (k % 2 == 0) && (reinterpret_cast<uintptr_t>(a) % 8 == 0);
    // The staged prologue row lives in LDS (16-byte aligned), so only an even k is needed
    // there; the norm-after form reads x and the norm weight in pairs from memory.
    const bool m1_pairs = a_op == kAOpNone ? pair_a
                          : a_op == kAOpRmsAfter
                              ? pair_a && reinterpret_cast<uintptr_t>(prologue->rms_weight) % 8 == 0
                          : a_op == kAOpSiluUp ? pair_a && reinterpret_cast<uintptr_t>(prologue->silu_up) % 8 == 0
                          : a_op == kAOpMul    ? pair_a && reinterpret_cast<uintptr_t>(prologue->mul_up) % 8 == 0
                          : a_op == kAOpAttn
                              ? k % 2 == 0 && reinterpret_cast<uintptr_t>(prologue->attn_partial) % 8 == 0
                              : k % 2 == 0;  // kAOpRms: the row is staged in LDS
    const bool m1 = m == 1 && !zero && !row_scale && splits == 1 && m1_pairs && k <= NarrowShape<1>::kBatchRows &&
                    n < (int64_t(1) << 30) && (b.mode == kScalePerCol || b.mode == kScaleConst) &&
                    epi.rms_weight == nullptr;
    // The side outputs: the m = 1 kernel without an input transform, or the one-wave-per-tile
    // kernel (k <= 1024 over at least 8 x CUs tiles) with the norm after the product.
    const bool wave_tile_rms = a_op == kAOpRmsAfter && GemvWaveTileApplies(m, k, n) && epi.Identity() &&
                               epi.split[0] == 0;
    if (side && (!m1 || (a_op != kAOpNone && !wave_tile_rms)))
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMV greedy keys and advance need the m = 1 kernel (m = 1, k <= 4096, "
                                       "staged tiles, per-column or tensor scale, aligned pairs) and no input "
                                       "prologue but the norm over a wide product");
    if (prologue != nullptr && prologue->silu_split0 && (!m1 || a_op != kAOpRmsAfter || epi.split[0] <= 0))
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMV SiLU store needs the m = 1 kernel with the norm after the product "
                                       "and a column split");
    if (!m1 && a_op == kAOpRmsAfter) a_op = kAOpRms;  // the general kernel normalizes first
    if (!m1 && (a_op == kAOpAttn || a_op == kAOpMul))
      Fail(ACCEL_HIP_INVALID_ARGUMENT,
           "GEMV attention and mul prologues need the m = 1 kernel (per-column or tensor scale, aligned pairs)");
    if (m1) {
      const int steps = static_cast<int>((k + NarrowShape<1>::kStepRows - 1) / NarrowShape<1>::kStepRows);
      const bool clamp = k != steps * NarrowShape<1>::kStepRows;
      const bool plain = epi.Identity() && epi.split[0] == 0 && a_op == kAOpNone && !side;
      const GemvPrologue pro = prologue != nullptr ? *prologue : GemvPrologue{};
      // The input transform's second operand (its pointer is among the preloaded arguments).
      const float* second = a_op == kAOpRmsAfter ? pro.rms_weight
                            : a_op == kAOpSiluUp ? pro.silu_up
                            : a_op == kAOpMul    ? pro.mul_up
                            : a_op == kAOpAttn   ? pro.attn_partial
                                                 : nullptr;
      const int32_t attn_splits = a_op == kAOpAttn ? pro.attn_splits : 0;
      const int32_t mul = b.mode == kScalePerCol ? 1 : 0;
      const int32_t cidx = b.mode == kScalePerCol ? 0 : static_cast<int32_t>(b.const_index);
      const dim3 block(NarrowShape<1>::kThreads);
#define ACCEL_GEMV_M1_KC(ST, CL, PL, OP, CA)                                                                   \
  hipLaunchKernelGGL((GemvM1Kernel<ST, CL, PL, OP, CA>), grid, block, 0, stream, b.tiled, a, b.scale + cidx, c, \
                     static_cast<int32_t>(k), static_cast<int32_t>(n), second, mul, attn_splits, epi, pro)
#define ACCEL_GEMV_M1_K(ST, CL, PL, OP)          \
  do {                                           \
    if (b.cached)                                \
      ACCEL_GEMV_M1_KC(ST, CL, PL, OP, true);    \
    else                                         \
      ACCEL_GEMV_M1_KC(ST, CL, PL, OP, false);   \
  } while (0)
#define ACCEL_GEMV_M1(ST, CL)                                                               \
  do {                                                                                      \
    if (a_op == kAOpRms) ACCEL_GEMV_M1_K(ST, CL, false, kAOpRms);                           \
    else if (a_op == kAOpAttn) ACCEL_GEMV_M1_K(ST, CL, false, kAOpAttn);                    \
    else if (a_op == kAOpRmsAfter) ACCEL_GEMV_M1_K(ST, CL, false, kAOpRmsAfter);            \
    else if (a_op == kAOpSiluUp) ACCEL_GEMV_M1_K(ST, CL, false, kAOpSiluUp);                \
    else if (a_op == kAOpMul) ACCEL_GEMV_M1_K(ST, CL, false, kAOpMul);                      \
    else if (plain) ACCEL_GEMV_M1_K(ST, CL, true, kAOpNone);                                \
    else ACCEL_GEMV_M1_K(ST, CL, false, kAOpNone);                                          \
  } while (0)
      const int64_t wave_tile_loads = (k / 2 + 63) / 64;  // row pairs a lane covers (k is even here)
      if ((a_op == kAOpNone || a_op == kAOpRmsAfter) && epi.Identity() && epi.split[0] == 0 &&
          !pro.silu_split0 && GemvWaveTileApplies(m, k, n)) {
        const bool rms = a_op == kAOpRmsAfter;
        const int64_t groups = (tiles + kWaveTileWaves - 1) / kWaveTileWaves;
        const dim3 wgrid(static_cast<uint32_t>((groups + kXcds - 1) / kXcds * kXcds));
        const dim3 wblock(64 * kWaveTileWaves);
#define ACCEL_GEMV_WT(L, CA, SD, RM)                                                                         \
  hipLaunchKernelGGL((GemvWaveTileKernel<L, CA, SD, RM>), wgrid, wblock, 0, stream, b.tiled, a, second, b.scale, \
                     static_cast<int32_t>(k), static_cast<int32_t>(n), mul, cidx, c, pro)
#define ACCEL_GEMV_WT_R(L, RM)                             \
  do {                                                     \
    if (b.cached && side) ACCEL_GEMV_WT(L, true, true, RM);    \
    else if (b.cached) ACCEL_GEMV_WT(L, true, false, RM);      \
    else if (side) ACCEL_GEMV_WT(L, false, true, RM);          \
    else ACCEL_GEMV_WT(L, false, false, RM);                   \
  } while (0)
#define ACCEL_GEMV_WT_L(L)              \
  do {                                  \
    if (rms) ACCEL_GEMV_WT_R(L, true);  \
    else ACCEL_GEMV_WT_R(L, false);     \
  } while (0)
        switch (wave_tile_loads) {
          case 1: ACCEL_GEMV_WT_L(1); break;
          case 2: ACCEL_GEMV_WT_L(2); break;
          case 3: ACCEL_GEMV_WT_L(3); break;
          case 4: ACCEL_GEMV_WT_L(4); break;
          case 5: ACCEL_GEMV_WT_L(5); break;
          case 6: ACCEL_GEMV_WT_L(6); break;
          case 7: ACCEL_GEMV_WT_L(7); break;
          default: ACCEL_GEMV_WT_L(8); break;
        }
#undef ACCEL_GEMV_WT_L
#undef ACCEL_GEMV_WT_R
#undef ACCEL_GEMV_WT
      } else if (a_op == kAOpAttn && k <= 2 * 512) {
        // One step of 512 lanes: each lane combines at most one row pair of the attention.
        const dim3 block8(512);
        const bool clamp8 = k != 1024;
#define ACCEL_GEMV_M1_ATTN8(CL, CA)                                                                          \
  hipLaunchKernelGGL((GemvM1Kernel<1, CL, false, kAOpAttn, CA, 8>), grid, block8, 0, stream, b.tiled, a,     \
                     b.scale + cidx, c, static_cast<int32_t>(k), static_cast<int32_t>(n), second, mul, attn_splits, \
                     epi, pro)
        if (clamp8 && b.cached) ACCEL_GEMV_M1_ATTN8(true, true);
        else if (clamp8) ACCEL_GEMV_M1_ATTN8(true, false);
        else if (b.cached) ACCEL_GEMV_M1_ATTN8(false, true);
        else ACCEL_GEMV_M1_ATTN8(false, false);
#undef ACCEL_GEMV_M1_ATTN8
      } else {
      switch (steps * 2 + (clamp ? 1 : 0)) {
        case 2: ACCEL_GEMV_M1(1, false); break;
        case 3: ACCEL_GEMV_M1(1, true); break;
        case 4: ACCEL_GEMV_M1(2, false); break;
        case 5: ACCEL_GEMV_M1(2, true); break;
        case 6: ACCEL_GEMV_M1(3, false); break;
        case 7: ACCEL_GEMV_M1(3, true); break;
        case 8: ACCEL_GEMV_M1(4, false); break;
        case 9: ACCEL_GEMV_M1(4, true); break;
        case 10: ACCEL_GEMV_M1(5, false); break;
        case 11: ACCEL_GEMV_M1(5, true); break;
        case 12: ACCEL_GEMV_M1(6, false); break;
        case 13: ACCEL_GEMV_M1(6, true); break;
        case 14: ACCEL_GEMV_M1(7, false); break;
        case 15: ACCEL_GEMV_M1(7, true); break;
        case 16: ACCEL_GEMV_M1(8, false); break;
        default: ACCEL_GEMV_M1(8, true); break;
      }
      }
#undef ACCEL_GEMV_M1
#undef ACCEL_GEMV_M1_K
#undef ACCEL_GEMV_M1_KC
    } else if (a_op == kAOpRms) {
      // The staged row in LDS is 16-byte aligned and k is whole, so pairs load as one.
      if (k % 2 == 0) hipLaunchKernelGGL((GemvNarrowKernel<1, false, false, true, kAOpRms>), grid,
                                         dim3(NarrowShape<1>::kThreads), 0, stream, ACCEL_NARROW_LEAD(args), args);
      else hipLaunchKernelGGL((GemvNarrowKernel<1, false, false, false, kAOpRms>), grid,
                              dim3(NarrowShape<1>::kThreads), 0, stream, ACCEL_NARROW_LEAD(args), args);
    } else if (a_op == kAOpSiluUp) {
      if (k % 2 == 0) hipLaunchKernelGGL((GemvNarrowKernel<1, false, false, true, kAOpSiluUp>), grid,
                                         dim3(NarrowShape<1>::kThreads), 0, stream, ACCEL_NARROW_LEAD(args), args);
      else hipLaunchKernelGGL((GemvNarrowKernel<1, false, false, false, kAOpSiluUp>), grid,
                              dim3(NarrowShape<1>::kThreads), 0, stream, ACCEL_NARROW_LEAD(args), args);
    } else if (m == 1) {
      LaunchNarrow<1>(args, grid, zero, row_scale, pair_a, stream);
    } else if (m == 2) {
      LaunchNarrow<2>(args, grid, zero, row_scale, pair_a, stream);
    } else {
      LaunchNarrow<4>(args, grid, zero, row_scale, pair_a, stream);
    }
  } else {
    const bool vec = (n % 16 == 0) && (reinterpret_cast<uintptr_t>(b.q) % 16 == 0);
    const dim3 block(kWideThreads);
    switch ((vec ? 4 : 0) | (zero ? 2 : 0) | (row_scale ? 1 : 0)) {
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
  if (splits > 1 && !split_bf16)
    LaunchSplitReduce(args.partials, args.splits, m, n, c, b.mode, b.scale, b.const_index, epi, stream);
}

}  // namespace accel_hip
