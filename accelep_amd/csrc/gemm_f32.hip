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
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

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
// two dependent MFMA chains and meets a barrier every 16 k. Here each of the 4 waves of a
// workgroup takes the whole 64 x 64 tile over a quarter of the workgroup's K range, with no LDS
// and no barrier until the end; the four wave partials meet in LDS and are added in wave order,
// and a K split across workgroups (for grids with fewer tiles than CUs) goes through the
// workspace and SplitReduceKernel, as above. Full tiles only: m and n multiples of 64, K per
// wave a multiple of 64, A and B 16-byte aligned.
//
// Measured history on the MLP (X[256,1024] -> 4096 -> 1024, per step): the LDS kernel 64-66 us;
// the same split of K on v_mfma_f32_16x16x4f32 (4 x 4 fp32 MFMA chains per wave, a pure MFMA
// stream of 2 x 16.6 us) 54-56 us; the bf16 part products below 45.7-47 us. Summing the K splits
// in the last workgroup of a tile to arrive (agent-scope stores, an arrival count, agent-scope
// loads of the other partials) measured slower than SplitReduceKernel in both forms: on the
// fp32 form 60.6 against 55.3 us per MLP step, on the bf16 form 48-49.6 against 46.5-47.1 us
// (A/B/A/B on one box, graph replay). The same sum behind an acquire-release count (plain stores
// and loads) is slower still (lab: 29.7 against 21.8 us per launch): the acquire invalidates the
// XCD's L2 under the workgroups still streaming their operands.

constexpr int kWsTile = 64;
constexpr int kWsPad = kWsTile + 1;  // LDS row stride of the partial tiles (no bank conflicts)
constexpr int kWsRowsPerThread = kWsTile * kWsTile / kThreads;  // output elements each thread stores
constexpr int kWsUnitK = 256;  // K of a workgroup: whole multiples of 4 waves x 64
static_assert(kThreads % kWsTile == 0 && kThreads / kWsTile == 4, "store loop: 4 tile rows per pass");

struct WsArgs {
  const float* a;
  const float* b;
  float* c;
  int64_t m, k, n;
  int64_t k_per_wg;    // K range of one workgroup (a multiple of kWsUnitK)
  float* partials;     // [splits][m][n] when K is split across workgroups, else nullptr
  const u32x4* bparts;  // B as staged bf16 parts (the StagedF32Parts layout), or nullptr
  Epilogue epi;
};

// ---- the same small grids on the bf16 matrix cores: six exact part products per product ----
//
// Each fp32 operand x is split as hi + mid + lo (SplitBf16Pair: exact, |mid| about 2^-8 |x| at
// most, |lo| about 2^-16 |x| at most), and a product a*b is formed from six part products,
// hi*hi', hi*mid', mid*hi', mid*mid', hi*lo' and lo*hi', on v_mfma_f32_32x32x16_bf16. Each part
// product is exact in fp32 (8 x 8 significand bits), so only the accumulation rounds. The three
// left out, mid*lo' + lo*mid' + lo*lo', are below about 2^-23 |a b| together: less than two fp32
// roundings of the product, which the reference's k-ordered loop rounds once. The hi*hi'
// products accumulate apart from the five cross terms (together below about 2^-7 |a b|): the
// large sum takes one rounding per MFMA step, as one fp32 accumulation would, and the cross
// sum's roundings are 2^-7 as large; the two are added once at the end. Every output therefore
// stays within Higham's 2 gamma_K bound of the exact product even if an MFMA added its products
// one by one in fp32, for finite operands whose parts stay normal (|x| >= 2^-110) and below the
// bf16 overflow threshold. (Measured on single MFMAs, one adds its 16 products and the
// accumulator with about one fp32 rounding at the magnitude of the largest of them: 2^24 +
// fourteen 1s - 2^24 gives 15, not the 0 of a sequential fp32 sum. One accumulator for all six
// measured 0.3 us faster per MLP step, A/B on one box; not taken.)
//
// The bf16 matrix cores run 16 times the fp32 MFMA rate, so six passes are 2.7 times the
// throughput of one fp32 pass. The grid: a 64 x 64 tile per workgroup, each of its 4 waves
// over a quarter of the workgroup's K, 2 x 2 MFMA tiles of 32 x 32 per wave, K split across workgroups through SplitReduceKernel when the tiles leave CUs
// idle. Operands load in groups of 32 k, two groups in flight; lane l (r = l % 32, h = l / 32)
// loads per group:
//  * A: row 32i + r of row tile i, k 16h .. 16h + 15, four float4 loads, so the two lanes of a
//    row read its whole 128-byte line within one group (reading 16 k per group, half a line,
//    measured about 1.5 us slower per launch on the MLP's products);
//  * B: k rows 16h + 8s + t (MFMA step s < 2, t < 8), columns 2r and 2r + 1, one float2 load each:
//    element j is the lane's B operand of column tile j, whose MFMA column c is the tile's
//    column 2c + j.
// MFMA step s of a group covers k 16h + 8s .. + 7 of lane (r, h), for A and B alike. The split of
// the next step (VALU) is interleaved with the MFMAs of the current one.

struct SbOperands {
  float4 a[2][4];      // row tile i: k 16h .. 16h + 15 of the lane's row
  float2 b[2][8];      // step s, row 16h + 8s + t: the lane's columns of column tiles 0 and 1
  u32x4 bp[2][2][3];   // staged B: step s, column tile j, part hi / mid / lo
};

struct SbParts {
  u32x4 a[2][3];  // row tile i, part hi / mid / lo: 8 bf16, k ascending
  u32x4 b[2][3];  // column tile j, part hi / mid / lo
};

// kStaged: B's parts come from the staged copy, twelve 1 KB wave loads per group (one 16-byte
// load per lane each) in place of the sixteen float2 loads and the split.
template <bool kStaged>
__device__ __forceinline__ void LoadSbGroup(const WsArgs& p, int64_t m0, int64_t n0, int64_t kb, int lane,
                                            SbOperands& r) {
  const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float* src = p.a + (m0 + 32 * i + l32) * p.k + kb + 16 * h;
#pragma unroll
    for (int q = 0; q < 4; ++q) r.a[i][q] = *reinterpret_cast<const float4*>(src + 4 * q);
  }
  if (kStaged) {
    const u32x4* src = p.bparts + ((n0 / kWsTile) * (p.k / 32) + kb / 32) * (12 * 64) + lane;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 3; ++q) r.bp[s][j][q] = src[((2 * s + j) * 3 + q) * 64];
    return;
  }
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int t = 0; t < 8; ++t)
      r.b[s][t] = *reinterpret_cast<const float2*>(p.b + (kb + 16 * h + 8 * s + t) * p.n + n0 + 2 * l32);
}

// Eight floats (k ascending) to the three part operands of one MFMA tile.
__device__ __forceinline__ void SplitOperand(const float (&x)[8], u32x4 (&part)[3]) {
  uint32_t w[3][4];
#pragma unroll
  for (int v = 0; v < 4; ++v) SplitBf16Pair(x[2 * v], x[2 * v + 1], w[0][v], w[1][v], w[2][v]);
#pragma unroll
  for (int q = 0; q < 3; ++q) part[q] = u32x4{w[q][0], w[q][1], w[q][2], w[q][3]};
}

// The part operands of MFMA step s of a loaded group.
template <bool kStaged>
__device__ __forceinline__ void SplitSbStep(const SbOperands& r, int s, SbParts& q) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 u = r.a[i][2 * s], v = r.a[i][2 * s + 1];
    const float x[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
    SplitOperand(x, q.a[i]);
  }
  if (kStaged) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int c = 0; c < 3; ++c) q.b[j][c] = r.bp[s][j][c];
    return;
  }
  const float b0[8] = {r.b[s][0].x, r.b[s][1].x, r.b[s][2].x, r.b[s][3].x,
                       r.b[s][4].x, r.b[s][5].x, r.b[s][6].x, r.b[s][7].x};
  const float b1[8] = {r.b[s][0].y, r.b[s][1].y, r.b[s][2].y, r.b[s][3].y,
                       r.b[s][4].y, r.b[s][5].y, r.b[s][6].y, r.b[s][7].y};
  SplitOperand(b0, q.b[0]);
  SplitOperand(b1, q.b[1]);
}

__device__ __forceinline__ v16f Mfma16(const u32x4& a, const u32x4& b, const v16f& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

// The 24 MFMAs of one step, pass-major so that consecutive MFMAs feed different accumulators;
// one MFMA, seven VALU instructions of the next step's split and one load of a group alternate
// (pairs of MFMAs with 14 VALU measured 0.8 us slower per MLP step, quadruples 1.3 us).
__device__ __forceinline__ void SbStepMfmas(const SbParts& cur, v16f (&hh)[2][2], v16f (&cross)[2][2]) {
  // cross terms: lo*hi', hi*lo', mid*mid', mid*hi', hi*mid' (part 0 hi, 1 mid, 2 lo)
  constexpr int kPa[5] = {2, 0, 1, 1, 0};
  constexpr int kPb[5] = {0, 2, 1, 0, 1};
#pragma unroll
  for (int q = 0; q < 5; ++q)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) cross[i][j] = Mfma16(cur.a[i][kPa[q]], cur.b[j][kPb[q]], cross[i][j]);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) hh[i][j] = Mfma16(cur.a[i][0], cur.b[j][0], hh[i][j]);
#pragma unroll
  for (int u = 0; u < 24; ++u) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);  // VALU
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
  }
  __builtin_amdgcn_sched_barrier(0);
}

// The epilogue steps of ApplyEpilogueLoaded for one known form, over a thread's 16 outputs
// (rows 4u apart): the same operations in the same order, so the same bits.
template <int kAct, bool kBias, bool kRes>
__device__ __forceinline__ void StoreRows(const float (&v)[kWsRowsPerThread], const Epilogue& e, float bias_v,
                                          const float (&res_v)[kWsRowsPerThread], float* out, int64_t n) {
  Epilogue f = e;
  f.activation = kAct;
  f.bias = kBias ? e.bias : nullptr;
  f.residual = kRes ? e.residual : nullptr;
#pragma unroll
  for (int u = 0; u < kWsRowsPerThread; ++u) out[4 * u * n] = ApplyEpilogueLoaded(v[u], f, bias_v, res_v[u]);
}

// kGroups > 0: the K range of a wave is exactly kGroups groups of 32. kGroups == 0: any even
// number of groups. kStaged: B's parts are read from p.bparts (the same bits the split gives).
template <int kGroups, bool kStaged>
// The pointers and sizes the operand loads need lead the arguments (10 dwords, preloaded into
// SGPRs at wave launch, so the first loads issue without a kernarg round trip); the output
// pointers and the epilogue come from `args`, read behind the loads.
__global__ __launch_bounds__(kThreads) void GemmF32SplitBf16Kernel(const float* a, const float* b,
                                                                   const u32x4* bparts, int32_t m, int32_t k,
                                                                   int32_t n, int32_t k_per_wg, WsArgs args) {
  WsArgs p = args;
  p.a = a;
  p.b = b;
  p.bparts = bparts;
  p.m = m;
  p.k = k;
  p.n = n;
  p.k_per_wg = k_per_wg;
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
  const int groups = kGroups > 0 ? kGroups : static_cast<int>(k_wave / 32);

  v16f hh[2][2], cross[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        hh[i][j][r] = 0.f;
        cross[i][j][r] = 0.f;
      }

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

  // Group g sits in ops[g % 2]. Per group: split step 1 while step 0 multiplies, then split the
  // next group's step 0 and request group g + 2 into the freed set while step 1 multiplies
  // (requests past the end repeat the last group; never used).
  SbOperands ops[2];
  SbParts parts[2];
  LoadSbGroup<kStaged>(p, m0, n0, kbeg, lane, ops[0]);
  LoadSbGroup<kStaged>(p, m0, n0, kbeg + static_cast<int64_t>(min(1, groups - 1)) * 32, lane, ops[1]);
  SplitSbStep<kStaged>(ops[0], 0, parts[0]);
#pragma unroll (kGroups > 0 ? kGroups / 2 : 1)
  for (int g = 0; g < groups; g += 2) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      SplitSbStep<kStaged>(ops[st], 1, parts[1]);
      SbStepMfmas(parts[0], hh, cross);
      SplitSbStep<kStaged>(ops[st ^ 1], 0, parts[0]);
      LoadSbGroup<kStaged>(p, m0, n0, kbeg + static_cast<int64_t>(min(g + st + 2, groups - 1)) * 32, lane, ops[st]);
      SbStepMfmas(parts[1], hh, cross);
    }
  }
  // Element r of MFMA tile (i, j): row 32i + 8(r / 4) + 4(lane / 32) + r % 4, column
  // 2(lane % 32) + j.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        red[wave][32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)][2 * (lane & 31) + j] = hh[i][j][r] + cross[i][j][r];
  __syncthreads();
  float v[kWsRowsPerThread];
#pragma unroll
  for (int u = 0; u < kWsRowsPerThread; ++u) {
    const int row = 4 * u + erow;
    v[u] = red[0][row][ecol] + red[1][row][ecol] + red[2][row][ecol] + red[3][row][ecol];
  }
  if (p.partials != nullptr) {  // SplitReduceKernel adds the splits in order and applies the epilogue
#pragma unroll
    for (int u = 0; u < kWsRowsPerThread; ++u)
      p.partials[(static_cast<int64_t>(blockIdx.y) * p.m + m0 + 4 * u + erow) * p.n + n0 + ecol] = v[u];
    return;
  }
  if (p.epi.split[0] == 0 && !bias_by_row) {
    // One [m, n] output and a bias per column (or none): one straight run per form of the
    // epilogue over the thread's 16 values, so their erf and stores overlap instead of
    // following the epilogue's branches one value at a time.
    float* out = p.c + (m0 + erow) * p.n + n0 + ecol;
    const int form = (p.epi.activation == ACCEL_HIP_ACT_GELU ? 8 : p.epi.activation == ACCEL_HIP_ACT_RELU ? 4 : 0) |
                     (p.epi.bias != nullptr ? 2 : 0) | (p.epi.residual != nullptr ? 1 : 0);
    switch (form) {
#define ACCEL_WS_FORM(F)                                                                             \
  case F:                                                                                            \
    StoreRows<(F & 12) == 8 ? ACCEL_HIP_ACT_GELU : (F & 12) == 4 ? ACCEL_HIP_ACT_RELU : ACCEL_HIP_ACT_NONE, \
              (F & 2) != 0, (F & 1) != 0>(v, p.epi, bias_v, res_v, out, p.n);                           \
    break;
      ACCEL_WS_FORM(0) ACCEL_WS_FORM(1) ACCEL_WS_FORM(2) ACCEL_WS_FORM(3) ACCEL_WS_FORM(4) ACCEL_WS_FORM(5)
      ACCEL_WS_FORM(6) ACCEL_WS_FORM(7) ACCEL_WS_FORM(8) ACCEL_WS_FORM(9) ACCEL_WS_FORM(10) ACCEL_WS_FORM(11)
#undef ACCEL_WS_FORM
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < kWsRowsPerThread; ++u) {
    const int64_t gr = m0 + 4 * u + erow, gc = n0 + ecol;
    const float b = bias_by_row && p.epi.bias != nullptr ? p.epi.bias[BiasIndex(p.epi, gr, gc)] : bias_v;
    StoreC(p.c, gr, gc, p.n, p.epi, ApplyEpilogueLoaded(v[u], p.epi, b, res_v[u]));
  }
}

// dst in the StagedF32Parts layout from B [k, n] (n % 64 == 0, k % 32 == 0): one thread per
// 16-byte lane slot, split by the kernel's own SplitOperand, so the staged parts are the bits
// the split on the fly gives.
__global__ void StageF32PartsKernel(const float* b, int64_t k, int64_t n, u32x4* dst, int64_t slots) {
  const int64_t groups = k / 32;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < slots;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int lane = static_cast<int>(idx & 63);
    const int blk = static_cast<int>((idx >> 6) % 12);  // (2s + j) * 3 + part
    const int64_t tg = (idx >> 6) / 12;                 // column tile * groups + group
    const int part = blk % 3, s = blk / 6, j = (blk / 3) & 1;
    const int64_t col = (tg / groups) * kWsTile + 2 * (lane & 31) + j;
    const int64_t k0 = (tg % groups) * 32 + 16 * (lane >> 5) + 8 * s;
    float x[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) x[t] = b[(k0 + t) * n + col];
    u32x4 parts[3];
    SplitOperand(x, parts);
    dst[idx] = parts[part];
  }
}

}  // namespace

void LaunchStageF32Parts(const float* b, int64_t k, int64_t n, void* dst, hipStream_t stream) {
  if (n % kWsTile != 0 || k % 32 != 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "staged fp32 parts need n % 64 == 0, k % 32 == 0");
  const int64_t slots = static_cast<int64_t>(StagedF32PartsBytes(k, n) / 16);
  int64_t grid = (slots + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(StageF32PartsKernel, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream, b, k, n,
                     static_cast<u32x4*>(dst), slots);
  Check(hipGetLastError(), "StageF32PartsKernel launch");
}

bool LaunchGemmF32(const float* a, const float* b, const Q8View& bq, float* c, int64_t m, int64_t k, int64_t n,
                   const Epilogue& epi, hipStream_t stream, const RmsRequest* rms, bool stage_b) {
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
    // Small fp32 grid: waves split K (GemmF32SplitBf16Kernel); K split across workgroups too
    // when the tiles leave CUs idle, into ranges of whole 4-wave groups.
    const int64_t wtiles = (m / kWsTile) * (n / kWsTile);
    const int64_t unit = kWsUnitK;  // per workgroup: 4 waves x whole pairs of 32-k groups
    int64_t wsplits = wtiles < cus ? std::max<int64_t>(1, std::min<int64_t>((cus + wtiles - 1) / wtiles, k / (4 * unit)))
                                   : 1;
    while (wsplits > 1 && k % (wsplits * unit) != 0) --wsplits;
    if (k % (wsplits * unit) == 0 && wtiles <= 0x7fffffff && m <= 0x7fffffff && n <= 0x7fffffff && k <= 0x7fffffff) {
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
      // B's staged parts when it has them (a weight: built on its second use, StagedF32Parts).
      ws.bparts = static_cast<const u32x4*>(StagedF32Parts(b, k, n, stream, stage_b));
      const dim3 grid(static_cast<uint32_t>(wtiles), static_cast<uint32_t>(wsplits));
      const bool full = ws.k_per_wg / 4 == 256;
      const int32_t m32 = static_cast<int32_t>(m), k32 = static_cast<int32_t>(k), n32 = static_cast<int32_t>(n);
      const int32_t kpw32 = static_cast<int32_t>(ws.k_per_wg);
      if (ws.bparts != nullptr) {
        if (full) hipLaunchKernelGGL((GemmF32SplitBf16Kernel<8, true>), grid, dim3(kThreads), 0, stream, ws.a, ws.b,
                                     ws.bparts, m32, k32, n32, kpw32, ws);
        else hipLaunchKernelGGL((GemmF32SplitBf16Kernel<0, true>), grid, dim3(kThreads), 0, stream, ws.a, ws.b,
                                     ws.bparts, m32, k32, n32, kpw32, ws);
      } else {
        if (full) hipLaunchKernelGGL((GemmF32SplitBf16Kernel<8, false>), grid, dim3(kThreads), 0, stream, ws.a, ws.b,
                                     ws.bparts, m32, k32, n32, kpw32, ws);
        else hipLaunchKernelGGL((GemmF32SplitBf16Kernel<0, false>), grid, dim3(kThreads), 0, stream, ws.a, ws.b,
                                     ws.bparts, m32, k32, n32, kpw32, ws);
      }
      Check(hipGetLastError(), "GemmF32SplitBf16Kernel launch");
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
