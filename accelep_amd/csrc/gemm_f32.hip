// fp32 GEMM on the matrix cores: C[m, n] = A[m, k] @ B[k, n] (+ fused epilogue), B either
// fp32 (Device::MatMul, src/sim_device.cc:185-196) or an int8 plane dequantized panel by
// panel into LDS (accel::MatMulQuantized for m > 16, src/sim_device.cc:541-602).
//
// Bound: MFMA (fp32, v_mfma_f32_32x32x2_f32). 2*m*n*k flops per call.
//
//  * Workgroup tile BM x BN (64 or 128 each), K step 16, 256 threads = 2x2 waves; each
//    wave owns a (BM/2) x (BN/2) block made of 32x32 MFMA tiles.
//  * A is staged k-major in LDS ([k][m]) so the A operand of a 32x32x2 step is 32
//    consecutive floats; B is staged row-major ([k][n]). Both are double buffered: the
//    next panel is fetched into registers while the current one feeds the MFMAs.
//  * The int8 panel is dequantized on its way into LDS with the reference's rounding,
//    w = (float(q) - float(zero)) * scale, so only the summation order differs from the
//    reference's k-ascending loop. Its bytes stay raw in registers while the current panel
//    is multiplied, and the column scales are loaded once per workgroup.
//  * Split-K over workgroups when the tile count cannot fill the GPU: partial tiles go to
//    the workspace and a second kernel sums them in split order and applies the epilogue
//    (deterministic, no synchronization between workgroups).
#include "device_common.h"

namespace accel_hip {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBK = 16;

struct GemmArgs {
  const float* a;
  const float* b;
  const int8_t* q;
  const float* scale;
  const int8_t* zero;
  int32_t mode;
  int64_t const_index;
  float* c;
  int64_t m, k, n;
  int32_t splits;
  int64_t k_per_split;  // multiple of kBK
  int32_t vec_a;        // A rows 16-byte aligned (k % 4 == 0)
  int32_t vec_b;        // B rows aligned for the panel loads
  float* partials;      // [splits][m][n]
  Epilogue epi;
};

template <int BM, int BN, bool kQ8>
struct Panels {
  // A: BM rows x 16 k, loaded as float4 along k. B fp32: 16 x BN as float4 along n.
  // B int8: 16 x BN bytes, kBBytes consecutive columns of one row per thread, kept as loaded
  // (dequantized only when stored to LDS, so the load is not waited for early).
  static constexpr int kAVec = BM * kBK / 4 / kThreads;  // float4 per thread
  static constexpr int kBVec = kQ8 ? 1 : BN * kBK / 4 / kThreads;
  static constexpr int kBBytes = BN * kBK / kThreads;  // int8 bytes per thread (4 or 8)
  float4 a[kAVec];
  float4 b[kBVec];
  uint32_t bq[kQ8 ? kBBytes / 4 : 1];
  float row_scale;  // per-row mode: scale and zero of this thread's row
  float row_zero;
};

// Where thread `tid` puts its int8 bytes: row of the 16-row panel and first column.
template <int BN>
__device__ __forceinline__ void Q8Slot(int tid, int* row, int* c0) {
  constexpr int kPerThread = BN * kBK / kThreads;
  constexpr int kThreadsPerRow = BN / kPerThread;
  *row = tid / kThreadsPerRow;
  *c0 = (tid % kThreadsPerRow) * kPerThread;
}

// kFull: the tile lies inside [m, n], the chunk inside k and the rows are aligned, so the
// loads need no checks.
template <int BM, int BN, bool kQ8, bool kFull>
__device__ __forceinline__ void LoadPanels(const GemmArgs& p, int64_t m0, int64_t n0, int64_t kc, int tid,
                                           Panels<BM, BN, kQ8>& r) {
  using P = Panels<BM, BN, kQ8>;
  // A: thread -> (row = idx / 4, k quad = idx % 4): four lanes read one 64-byte row segment.
#pragma unroll
  for (int v = 0; v < P::kAVec; ++v) {
    const int idx = tid + v * kThreads;
    const int row = idx >> 2;
    const int kq = idx & 3;
    const int64_t gr = m0 + row;
    const int64_t gk = kc + kq * 4;
    if (kFull) {
      r.a[v] = *reinterpret_cast<const float4*>(p.a + gr * p.k + gk);
      continue;
    }
    float4 val = make_float4(0.f, 0.f, 0.f, 0.f);
    if (gr < p.m) {
      const float* src = p.a + gr * p.k + gk;
      if (p.vec_a && gk + 3 < p.k) {
        val = *reinterpret_cast<const float4*>(src);
      } else {
        if (gk + 0 < p.k) val.x = src[0];
        if (gk + 1 < p.k) val.y = src[1];
        if (gk + 2 < p.k) val.z = src[2];
        if (gk + 3 < p.k) val.w = src[3];
      }
    }
    r.a[v] = val;
  }
  if (!kQ8) {
    constexpr int kQuadsPerRow = BN / 4;
#pragma unroll
    for (int v = 0; v < P::kBVec; ++v) {
      const int idx = tid + v * kThreads;
      const int row = idx / kQuadsPerRow;
      const int c4 = idx % kQuadsPerRow;
      const int64_t gk = kc + row;
      const int64_t gc = n0 + c4 * 4;
      if (kFull) {
        r.b[v] = *reinterpret_cast<const float4*>(p.b + gk * p.n + gc);
        continue;
      }
      float4 val = make_float4(0.f, 0.f, 0.f, 0.f);
      if (gk < p.k) {
        const float* src = p.b + gk * p.n + gc;
        if (p.vec_b && gc + 3 < p.n) {
          val = *reinterpret_cast<const float4*>(src);
        } else {
          if (gc + 0 < p.n) val.x = src[0];
          if (gc + 1 < p.n) val.y = src[1];
          if (gc + 2 < p.n) val.z = src[2];
          if (gc + 3 < p.n) val.w = src[3];
        }
      }
      r.b[v] = val;
    }
  } else {
    constexpr int kPerThread = P::kBBytes;
    int row, c0;
    Q8Slot<BN>(tid, &row, &c0);
    const int64_t gk = kc + row;
    const int64_t gc = n0 + c0;
    for (int w = 0; w < kPerThread / 4; ++w) r.bq[w] = 0;
    if (kFull || gk < p.k) {
      const int8_t* src = p.q + gk * p.n + gc;
      if (kFull || (p.vec_b && gc + kPerThread - 1 < p.n)) {
        if (kPerThread == 8) {
          const uint2 w = *reinterpret_cast<const uint2*>(src);
          r.bq[0] = w.x;
          r.bq[kPerThread / 4 - 1] = w.y;
        } else {
          r.bq[0] = *reinterpret_cast<const uint32_t*>(src);
        }
      } else {
        for (int e = 0; e < kPerThread; ++e)
          if (gc + e < p.n) r.bq[e >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(src[e])) << (8 * (e & 3));
      }
      if (p.mode == kScalePerRow) {
        r.row_scale = p.scale[gk];
        r.row_zero = p.zero != nullptr ? static_cast<float>(p.zero[gk]) : 0.f;
      }
    }
  }
}

// Per-thread constants of the int8 panel: the scale and zero of the thread's columns (per-
// column or whole-tensor modes), loaded once per workgroup.
template <int BN>
struct ColumnQuant {
  float scale[BN * kBK / kThreads];
  float zero[BN * kBK / kThreads];
};

template <int BN>
__device__ __forceinline__ void LoadColumnQuant(const GemmArgs& p, int64_t n0, int tid, ColumnQuant<BN>& cq) {
  constexpr int kPerThread = BN * kBK / kThreads;
  int row, c0;
  Q8Slot<BN>(tid, &row, &c0);
  for (int e = 0; e < kPerThread; ++e) {
    const int64_t gc = min(n0 + c0 + e, p.n - 1);
    const int64_t idx = p.mode == kScalePerCol ? gc : p.const_index;
    cq.scale[e] = p.mode == kScalePerRow ? 1.f : p.scale[idx];
    cq.zero[e] = (p.mode == kScalePerRow || p.zero == nullptr) ? 0.f : static_cast<float>(p.zero[idx]);
  }
}

template <int BM, int BN, bool kQ8, bool kFull>
__device__ __forceinline__ void StorePanels(const GemmArgs& p, float (*As)[BM + 4], float (*Bs)[BN + 4], int64_t n0,
                                            int64_t kc, int tid, const Panels<BM, BN, kQ8>& r,
                                            const ColumnQuant<BN>& cq) {
  using P = Panels<BM, BN, kQ8>;
#pragma unroll
  for (int v = 0; v < P::kAVec; ++v) {
    const int idx = tid + v * kThreads;
    const int row = idx >> 2;
    const int kq = idx & 3;
    As[kq * 4 + 0][row] = r.a[v].x;
    As[kq * 4 + 1][row] = r.a[v].y;
    As[kq * 4 + 2][row] = r.a[v].z;
    As[kq * 4 + 3][row] = r.a[v].w;
  }
  if (!kQ8) {
    constexpr int kQuadsPerRow = BN / 4;
#pragma unroll
    for (int v = 0; v < P::kBVec; ++v) {
      const int idx = tid + v * kThreads;
      const int row = idx / kQuadsPerRow;
      const int c4 = idx % kQuadsPerRow;
      *reinterpret_cast<float4*>(&Bs[row][c4 * 4]) = r.b[v];
    }
  } else {
    // w = (float(q) - float(zero)) * scale, the reference's rounding; 0 past k or n.
    constexpr int kPerThread = P::kBBytes;
    int row, c0;
    Q8Slot<BN>(tid, &row, &c0);
    const bool row_ok = kc + row < p.k;
    float w[kPerThread];
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
      const float q = ByteToFloat(r.bq[e >> 2], e & 3);
      const float s = p.mode == kScalePerRow ? r.row_scale : cq.scale[e];
      const float z = p.mode == kScalePerRow ? r.row_zero : cq.zero[e];
      const bool ok = kFull || (row_ok && n0 + c0 + e < p.n);
      w[e] = ok ? __fmul_rn(__fsub_rn(q, z), s) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < kPerThread; e += 4)
      *reinterpret_cast<float4*>(&Bs[row][c0 + e]) = make_float4(w[e], w[e + 1], w[e + 2], w[e + 3]);
  }
}

template <int BM, int BN, bool kQ8, bool kFull, int kPF>
__device__ __forceinline__ void GemmTile(const GemmArgs& p, float (*As)[kBK][BM + 4], float (*Bs)[kBK][BN + 4]) {
  constexpr int WM = BM / 2;
  constexpr int WN = BN / 2;
  constexpr int SM = WM / 32;
  constexpr int SN = WN / 32;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN;
  const int split = blockIdx.z;
  const int64_t kb = static_cast<int64_t>(split) * p.k_per_split;
  const int64_t ke = min(p.k, kb + p.k_per_split);
  const int chunks = static_cast<int>((ke - kb + kBK - 1) / kBK);

  v16f acc[SM][SN];
#pragma unroll
  for (int i = 0; i < SM; ++i)
#pragma unroll
    for (int j = 0; j < SN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  ColumnQuant<BN> cq;
  if (kQ8) LoadColumnQuant<BN>(p, n0, tid, cq);
  // kStages register sets: chunk ch + kStages is requested while chunk ch is multiplied, so a
  // panel's global latency is covered by kStages chunks of MFMA work (the LDS stays double
  // buffered). Edge tiles keep one set.
  constexpr int kStages = kFull ? kPF : 1;
  Panels<BM, BN, kQ8> regs[kStages];
#pragma unroll
  for (int st = 0; st < kStages; ++st)
    if (st < chunks) LoadPanels<BM, BN, kQ8, kFull>(p, m0, n0, kb + st * kBK, tid, regs[st]);
  if (chunks > 0) StorePanels<BM, BN, kQ8, kFull>(p, As[0], Bs[0], n0, kb, tid, regs[0], cq);
  __syncthreads();
  // Panels past ke read zeros only when ke == k; a split boundary inside k is a multiple
  // of kBK, so every chunk of a split lies inside [kb, ke). The chunk loop is unrolled by
  // kStages so that every register set is named at compile time.
  for (int base = 0; base < chunks; base += kStages) {
#pragma unroll
  for (int st = 0; st < kStages; ++st) {
    const int ch = base + st;
    if (ch >= chunks) break;  // workgroup-uniform
    const int cur = ch & 1;
    if (ch + kStages < chunks) LoadPanels<BM, BN, kQ8, kFull>(p, m0, n0, kb + (ch + kStages) * kBK, tid, regs[st]);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 2) {
      float av[SM];
      float bv[SN];
#pragma unroll
      for (int i = 0; i < SM; ++i) av[i] = As[cur][kk + (lane >> 5)][wm * WM + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < SN; ++j) bv[j] = Bs[cur][kk + (lane >> 5)][wn * WN + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < SM; ++i)
#pragma unroll
        for (int j = 0; j < SN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (ch + 1 < chunks)
      StorePanels<BM, BN, kQ8, kFull>(p, As[cur ^ 1], Bs[cur ^ 1], n0, kb + (ch + 1) * kBK, tid,
                                      regs[(st + 1) % kStages], cq);
    __syncthreads();
  }
  }

  // Epilogue through LDS: for each i, every wave parks its 32-row band acc[i][*] in the
  // stage ([64 rows][BN + 4], reusing the panel buffers), then the workgroup walks the 64 x BN
  // band in float4 steps along rows. Keeps the per-element epilogue out of the unrolled
  // accumulator code (register use) and makes the stores row-contiguous.
  float* stage = &As[0][0][0];
  constexpr int kStride = BN + 4;
  constexpr int kQuads = 64 * BN / 4;
  const bool vec_c = (p.n & 3) == 0 &&
                     (p.splits > 1 ? (reinterpret_cast<uintptr_t>(p.partials) & 15) == 0
                                   : p.epi.split[0] == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15) == 0);
  float* part = p.splits > 1 ? p.partials + static_cast<int64_t>(split) * p.m * p.n : nullptr;
#pragma unroll
  for (int i = 0; i < SM; ++i) {
    __syncthreads();  // the last panel reads, or the previous band's, are done
    // Element r of a 32x32 tile sits at row 8*(r/4) + 4*(lane/32) + r%4, column lane%32.
#pragma unroll
    for (int j = 0; j < SN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int sr = wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        stage[sr * kStride + wn * WN + j * 32 + (lane & 31)] = acc[i][j][r];
      }
    __syncthreads();
    for (int e = tid; e < kQuads; e += kThreads) {
      const int sr = e / (BN / 4);
      const int c4 = e % (BN / 4);
      const float4 v = *reinterpret_cast<const float4*>(&stage[sr * kStride + c4 * 4]);
      const int64_t gr = m0 + (sr >> 5) * WM + i * 32 + (sr & 31);
      const int64_t gc = n0 + c4 * 4;
      if (!kFull && gr >= p.m) continue;
      const float vals[4] = {v.x, v.y, v.z, v.w};
      if (part != nullptr) {  // SplitReduceKernel adds the splits in order and applies the epilogue
        if (vec_c && (kFull || gc + 3 < p.n)) {
          *reinterpret_cast<float4*>(part + gr * p.n + gc) = v;
        } else {
          for (int t = 0; t < 4; ++t)
            if (gc + t < p.n) part[gr * p.n + gc + t] = vals[t];
        }
        continue;
      }
      if (vec_c && (kFull || gc + 3 < p.n)) {
        float4 o;
        o.x = ApplyEpilogue(v.x, gr, gc + 0, p.n, p.epi);
        o.y = ApplyEpilogue(v.y, gr, gc + 1, p.n, p.epi);
        o.z = ApplyEpilogue(v.z, gr, gc + 2, p.n, p.epi);
        o.w = ApplyEpilogue(v.w, gr, gc + 3, p.n, p.epi);
        *reinterpret_cast<float4*>(p.c + gr * p.n + gc) = o;
      } else {
        for (int t = 0; t < 4; ++t)
          if (gc + t < p.n) StoreC(p.c, gr, gc + t, p.n, p.epi, ApplyEpilogue(vals[t], gr, gc + t, p.n, p.epi));
      }
    }
  }
}

// Waves per SIMD the register budget must allow. 128x128: 3 (at most 168 registers a lane),
// which holds the 64 accumulators and three panel sets without spilling; 64x64: 4.
template <int BM>
constexpr int GemmMinWaves() {
  return BM == 128 ? 3 : 4;
}

template <int BM, int BN, bool kQ8>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(GemmMinWaves<BM>()))) void GemmKernel(
    GemmArgs p) {
  // Panels (double buffered A and B) and, after the main loop, the epilogue stage.
  static_assert(BM == BN, "the epilogue stage [64][BN + 4] must fit the panel buffers");
  constexpr int kPanelFloats = 2 * kBK * (BM + 4) + 2 * kBK * (BN + 4);
  static_assert(64 * (BN + 4) <= kPanelFloats, "epilogue stage larger than the panels");
  __shared__ __align__(16) float lds[kPanelFloats];
  auto* As = reinterpret_cast<float(*)[kBK][BM + 4]>(lds);
  auto* Bs = reinterpret_cast<float(*)[kBK][BN + 4]>(lds + 2 * kBK * (BM + 4));
  // Interior tiles (most of a large product) take the unchecked loads; edge tiles and
  // unaligned operands the checked ones. The choice is uniform across the workgroup.
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN;
  const int64_t kb = static_cast<int64_t>(blockIdx.z) * p.k_per_split;
  const int64_t ke = min(p.k, kb + p.k_per_split);
  const bool full = p.vec_a && p.vec_b && m0 + BM <= p.m && n0 + BN <= p.n && (ke - kb) % kBK == 0;
  constexpr int kPF = BM == 128 ? 3 : 4;  // register sets of the interior path
  if (full) GemmTile<BM, BN, kQ8, true, kPF>(p, As, Bs);
  else GemmTile<BM, BN, kQ8, false, kPF>(p, As, Bs);
}

template <int BM, int BN>
void Launch(const GemmArgs& args, bool q8, dim3 grid, hipStream_t stream) {
  if (q8) hipLaunchKernelGGL((GemmKernel<BM, BN, true>), grid, dim3(kThreads), 0, stream, args);
  else hipLaunchKernelGGL((GemmKernel<BM, BN, false>), grid, dim3(kThreads), 0, stream, args);
}

// ---- small grids: the waves of a workgroup split K, operands straight from memory ------
//
// A product whose 64 x 64 tiles barely cover the CUs (the MLP's 256 x 1024 x 4096 and
// 256 x 4096 x 1024) gives each SIMD one wave. In the LDS kernel above that wave runs one or
// two dependent MFMA chains and meets a barrier every 16 k. Here each of the 4 waves takes the
// whole 64 x 64 tile over a quarter of the workgroup's K range, as 4 x 4 independent
// v_mfma_f32_16x16x4f32 chains, with no LDS and no barrier until the end:
//  * the 16 k of one group are assigned to MFMA steps so that every load is a float4: lane
//    group q = lane / 16 of row tile i loads A[16i + lane % 16][kb + 4q .. 4q + 3], whose
//    element s is its A operand in step s (k = kb + 4q + s); in step s the lane loads
//    B[kb + 4q + s][4(lane % 16) .. + 3], whose element j is its B operand for column tile j,
//    so MFMA column c of tile j is the tile's column 4c + j. The product sums every k of the
//    group once, in another order; 8 loads feed 64 MFMAs;
//  * operands of the next three groups are in flight while one group's 64 MFMAs run;
//  * the four wave partials meet in LDS and are added in wave order; a K split across
//    workgroups (for grids with fewer tiles than CUs) goes through the workspace and
//    SplitReduceKernel, as above. (Combining the splits in the last workgroup to arrive, with
//    agent-scope stores and loads of the partial tiles, measured slower on the MLP's
//    256 x 4096 x 1024: 73 against 55 us per MLP step; 60.6 against 55.3 with every partial
//    load of a chunk of four splits requested at once.)
// Full tiles only: m and n multiples of 64, K per wave a multiple of 4 groups of 16, A and B
// 16-byte aligned.

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWsTile = 64;
constexpr int kWsGroupK = 16;
constexpr int kWsStages = 4;  // groups in flight (32 loads, below the 63 the load counter tracks)
constexpr int kWsPad = kWsTile + 1;  // LDS row stride of the partial tiles (no bank conflicts)
constexpr int kWsRowsPerThread = kWsTile * kWsTile / kThreads;  // output elements each thread stores
static_assert(kThreads % kWsTile == 0 && kThreads / kWsTile == 4, "store loop: 4 tile rows per pass");

struct WsArgs {
  const float* a;
  const float* b;
  float* c;
  int64_t m, k, n;
  int64_t k_per_wg;    // K range of one workgroup (a multiple of 4 * kWsGroupK)
  float* partials;     // [splits][m][n] when K is split across workgroups, else nullptr
  Epilogue epi;
};

struct WsOperands {
  float4 a[4];  // row tiles 0..3: 4 consecutive k of this lane's row
  float4 b[4];  // steps 0..3: 4 consecutive columns (one per column tile) of this lane's k row
};

__device__ __forceinline__ void LoadWsGroup(const WsArgs& p, int64_t m0, int64_t n0, int64_t kb, int lane,
                                            WsOperands& r) {
  const int q = lane >> 4, l16 = lane & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r.a[i] = *reinterpret_cast<const float4*>(p.a + (m0 + 16 * i + l16) * p.k + kb + 4 * q);
#pragma unroll
  for (int s = 0; s < 4; ++s) r.b[s] = *reinterpret_cast<const float4*>(p.b + (kb + 4 * q + s) * p.n + n0 + 4 * l16);
}

__device__ __forceinline__ float Lane4(const float4& v, int s) {
  return s == 0 ? v.x : s == 1 ? v.y : s == 2 ? v.z : v.w;
}

// kGroups > 0: the K range of a wave is exactly kGroups groups (a trip count the compiler
// knows). kGroups == 0: any multiple of kWsStages groups.
template <int kGroups>
__global__ __launch_bounds__(kThreads) void GemmF32WaveSplitKernel(WsArgs p) {
  __shared__ float red[4][kWsTile][kWsPad];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t tiles_n = p.n / kWsTile;
  const int64_t tile = blockIdx.x;
  const int64_t m0 = (tile / tiles_n) * kWsTile;
  const int64_t n0 = (tile % tiles_n) * kWsTile;
  const int64_t k_wave = p.k_per_wg / 4;
  const int64_t kbeg = static_cast<int64_t>(blockIdx.y) * p.k_per_wg + wave * k_wave;
  const int groups = kGroups > 0 ? kGroups : static_cast<int>(k_wave / kWsGroupK);

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // The store loop at the end gives thread tid column tid % 64 of tile rows 4u + tid / 64
  // (u < kWsRowsPerThread). Their bias and residual values are loaded here, so the loads
  // complete under the main loop instead of costing a memory round trip per stored batch.
  const bool final_out = p.partials == nullptr;
  const int ecol = tid % kWsTile;
  const int erow = tid / kWsTile;
  const bool bias_by_row = p.epi.bias_rank == 2 && p.epi.bias_shape[0] != 1;
  float bias_v = 0.f;
  if (final_out && p.epi.bias != nullptr && !bias_by_row) bias_v = p.epi.bias[BiasIndex(p.epi, 0, n0 + ecol)];
  float res_v[kWsRowsPerThread];
#pragma unroll
  for (int u = 0; u < kWsRowsPerThread; ++u)
    res_v[u] = final_out && p.epi.residual != nullptr ? p.epi.residual[(m0 + 4 * u + erow) * p.n + n0 + ecol] : 0.f;

  WsOperands ops[kWsStages];
#pragma unroll
  for (int st = 0; st < kWsStages; ++st)
    LoadWsGroup(p, m0, n0, kbeg + static_cast<int64_t>(min(st, groups - 1)) * kWsGroupK, lane, ops[st]);
  // groups is a multiple of kWsStages: the loop body is whole stage rings, so the loop head
  // sees one pattern of loads in flight and waits only for the group it needs. With kGroups
  // known the body is two rings (8 groups, 512 MFMAs): measured slightly faster than the
  // whole range unrolled straight (Gemm1 of the MLP, 21.4 against 22.1 us per launch).
#pragma unroll (kGroups > 0 ? 2 : 1)
  for (int base = 0; base < groups; base += kWsStages) {
#pragma unroll
    for (int st = 0; st < kWsStages; ++st) {
      const int g = base + st;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(Lane4(ops[st].a[i], s), Lane4(ops[st].b[s], j), acc[i][j], 0,
                                                             0, 0);
      // The group kWsStages ahead (repeating the last one past the end; never used), issued here:
      // the barrier keeps the scheduler from sinking the loads to their use.
      LoadWsGroup(p, m0, n0, kbeg + static_cast<int64_t>(min(g + kWsStages, groups - 1)) * kWsGroupK, lane, ops[st]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Element r of tile (i, j): row 16i + 4 * (lane / 16) + r, column 4 * (lane % 16) + j.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][16 * i + 4 * (lane >> 4) + r][4 * (lane & 15) + j] = acc[i][j][r];
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kWsRowsPerThread; ++u) {
    const int row = 4 * u + erow, col = ecol;
    const float v = red[0][row][col] + red[1][row][col] + red[2][row][col] + red[3][row][col];
    const int64_t gr = m0 + row, gc = n0 + col;
    if (!final_out) {
      p.partials[(static_cast<int64_t>(blockIdx.y) * p.m + gr) * p.n + gc] = v;
    } else {
      const float b = bias_by_row && p.epi.bias != nullptr ? p.epi.bias[BiasIndex(p.epi, gr, gc)] : bias_v;
      StoreC(p.c, gr, gc, p.n, p.epi, ApplyEpilogueLoaded(v, p.epi, b, res_v[u]));
    }
  }
}

}  // namespace

bool LaunchGemmF32(const float* a, const float* b, const Q8View& bq, float* c, int64_t m, int64_t k, int64_t n,
                   const Epilogue& epi, hipStream_t stream, const RmsRequest* rms) {
  if (m < 1 || n < 1 || k < 1) Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMM shape out of range");
  Context& ctx0 = Ctx();
  const bool q8 = bq.q != nullptr;
  bool rms_done = false;
  if (q8 && LaunchGemmQ8Bf16(a, bq, c, m, k, n, epi, stream, rms, &rms_done)) return rms_done;
  const int64_t cus = ctx0.cu_count > 0 ? ctx0.cu_count : 256;
  // Large tiles when they alone give about two workgroups per CU; 64x64 otherwise.
  int bm = 128, bn = 128;
  auto tiles_for = [&](int tm, int tn) { return ((m + tm - 1) / tm) * ((n + tn - 1) / tn); };
  if (!q8 && tiles_for(128, 128) < 2 * cus && m % kWsTile == 0 && n % kWsTile == 0 &&
      reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0 && m / kWsTile <= 65535) {
    // Small fp32 grid: waves split K (GemmF32WaveSplitKernel); K split across workgroups too
    // when the tiles leave CUs idle, into ranges of whole 4-wave groups.
    const int64_t wtiles = (m / kWsTile) * (n / kWsTile);
    const int64_t unit = 4 * kWsGroupK * kWsStages;  // per workgroup: 4 waves x whole stage rings
    int64_t wsplits = wtiles < cus ? std::max<int64_t>(1, std::min<int64_t>((cus + wtiles - 1) / wtiles, k / (4 * unit)))
                                   : 1;
    while (wsplits > 1 && k % (wsplits * unit) != 0) --wsplits;
    if (k % (wsplits * unit) == 0 && wtiles <= 0x7fffffff) {
      WsArgs ws;
      ws.a = a;
      ws.b = b;
      ws.c = c;
      ws.m = m;
      ws.k = k;
      ws.n = n;
      ws.k_per_wg = k / wsplits;
      ws.partials = wsplits > 1 ? static_cast<float*>(Workspace(static_cast<size_t>(wsplits * m * n) * sizeof(float)))
                                : nullptr;
      ws.epi = epi;
      const dim3 grid(static_cast<uint32_t>(wtiles), static_cast<uint32_t>(wsplits));
      if (ws.k_per_wg / 4 == 16 * kWsGroupK) hipLaunchKernelGGL(GemmF32WaveSplitKernel<16>, grid, dim3(kThreads), 0, stream, ws);
      else hipLaunchKernelGGL(GemmF32WaveSplitKernel<0>, grid, dim3(kThreads), 0, stream, ws);
      Check(hipGetLastError(), "GemmF32WaveSplitKernel launch");
      if (wsplits > 1)
        LaunchSplitReduce(ws.partials, static_cast<int32_t>(wsplits), m, n, c, kScalePerRow, nullptr, 0, epi, stream);
      return false;
    }
  }
  if (tiles_for(128, 128) < 2 * cus) {
    bm = 64;
    bn = 64;
  }
  const int64_t tiles_m = (m + bm - 1) / bm;
  const int64_t tiles_n = (n + bn - 1) / bn;
  const int64_t tiles = tiles_m * tiles_n;
  // Split K only when the tiles leave CUs idle: with a tile per CU the partial-sum traffic and
  // the extra pass cost more than the second wave per SIMD gains.
  int64_t splits = 1;
  if (tiles < cus) splits = std::min<int64_t>((2 * cus + tiles - 1) / tiles, std::max<int64_t>(1, k / 256));
  int64_t kper = (k + splits - 1) / splits;
  kper = (kper + kBK - 1) / kBK * kBK;
  splits = (k + kper - 1) / kper;
  if (tiles_n > 0x7fffffff || tiles_m > 65535 || splits > 65535) Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMM grid too large");

  GemmArgs args;
  args.a = a;
  args.b = b;
  args.q = bq.q;
  args.scale = bq.scale;
  args.zero = bq.zero;
  args.mode = bq.mode;
  args.const_index = bq.const_index;
  args.c = c;
  args.m = m;
  args.k = k;
  args.n = n;
  args.splits = static_cast<int32_t>(splits);
  args.k_per_split = kper;
  args.vec_a = (k % 4 == 0) && (reinterpret_cast<uintptr_t>(a) % 16 == 0);
  if (q8) {
    const int per = bn * kBK / kThreads;  // bytes per thread of the int8 panel
    args.vec_b = (n % per == 0) && (reinterpret_cast<uintptr_t>(bq.q) % per == 0);
  } else {
    args.vec_b = (n % 4 == 0) && (reinterpret_cast<uintptr_t>(b) % 16 == 0);
  }
  args.partials = nullptr;
  args.epi = epi;
  if (splits > 1) {
    args.partials = static_cast<float*>(Workspace(static_cast<size_t>(splits * m * n) * sizeof(float)));
  }
  const dim3 grid(static_cast<uint32_t>(tiles_n), static_cast<uint32_t>(tiles_m), static_cast<uint32_t>(splits));
  if (bm == 128) Launch<128, 128>(args, q8, grid, stream);
  else Launch<64, 64>(args, q8, grid, stream);
  Check(hipGetLastError(), "GemmKernel launch");
  if (splits > 1) LaunchSplitReduce(args.partials, args.splits, m, n, c, kScalePerRow, nullptr, 0, epi, stream);
  return false;
}

}  // namespace accel_hip
