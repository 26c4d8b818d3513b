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
//    reference's k-ascending loop.
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

__device__ __forceinline__ float Dequant(const GemmArgs& p, int8_t qv, int64_t row, int64_t col) {
  int64_t idx = p.const_index;
  if (p.mode == kScalePerCol) idx = col;
  if (p.mode == kScalePerRow) idx = row;
  const float z = p.zero != nullptr ? static_cast<float>(p.zero[idx]) : 0.f;
  return __fmul_rn(static_cast<float>(qv) - z, p.scale[idx]);
}

template <int BM, int BN, bool kQ8>
struct Panels {
  // A: BM rows x 16 k, loaded as float4 along k. B fp32: 16 x BN as float4 along n.
  // B int8: 16 x BN bytes.
  static constexpr int kAVec = BM * kBK / 4 / kThreads;  // float4 per thread
  static constexpr int kBVec = kQ8 ? 1 : BN * kBK / 4 / kThreads;
  static constexpr int kBBytes = BN * kBK / kThreads;  // int8 bytes per thread (4 or 8)
  float4 a[kAVec];
  float4 b[kBVec];
  float bq[kQ8 ? kBBytes : 1];
};

template <int BM, int BN, bool kQ8>
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
    constexpr int kPerThread = P::kBBytes;  // 4 or 8 consecutive columns of one row
    constexpr int kThreadsPerRow = BN / kPerThread;
    const int row = tid / kThreadsPerRow;
    const int c0 = (tid % kThreadsPerRow) * kPerThread;
    const int64_t gk = kc + row;
    const int64_t gc = n0 + c0;
    if (gk < p.k) {
      const int8_t* src = p.q + gk * p.n + gc;
      int8_t bytes[kPerThread];
      if (p.vec_b && gc + kPerThread - 1 < p.n) {
        if (kPerThread == 8) {
          const uint2 w = *reinterpret_cast<const uint2*>(src);
          for (int e = 0; e < 4; ++e) bytes[e] = static_cast<int8_t>(w.x >> (8 * e));
          for (int e = 0; e < 4; ++e) bytes[4 + e] = static_cast<int8_t>(w.y >> (8 * e));
        } else {
          const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
          for (int e = 0; e < 4; ++e) bytes[e] = static_cast<int8_t>(w >> (8 * e));
        }
      } else {
        for (int e = 0; e < kPerThread; ++e) bytes[e] = gc + e < p.n ? src[e] : 0;
      }
      for (int e = 0; e < kPerThread; ++e) r.bq[e] = gc + e < p.n ? Dequant(p, bytes[e], gk, gc + e) : 0.f;
    } else {
      for (int e = 0; e < kPerThread; ++e) r.bq[e] = 0.f;
    }
  }
}

template <int BM, int BN, bool kQ8>
__device__ __forceinline__ void StorePanels(float (*As)[BM + 4], float (*Bs)[BN + 4], int tid,
                                            const Panels<BM, BN, kQ8>& r) {
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
    constexpr int kPerThread = P::kBBytes;
    constexpr int kThreadsPerRow = BN / kPerThread;
    const int row = tid / kThreadsPerRow;
    const int c0 = (tid % kThreadsPerRow) * kPerThread;
    for (int e = 0; e < kPerThread; e += 4)
      *reinterpret_cast<float4*>(&Bs[row][c0 + e]) = make_float4(r.bq[e], r.bq[e + 1], r.bq[e + 2], r.bq[e + 3]);
  }
}

template <int BM, int BN, bool kQ8>
__global__ __launch_bounds__(kThreads) void GemmKernel(GemmArgs p) {
  constexpr int WM = BM / 2;
  constexpr int WN = BN / 2;
  constexpr int SM = WM / 32;
  constexpr int SN = WN / 32;
  __shared__ float As[2][kBK][BM + 4];
  __shared__ float Bs[2][kBK][BN + 4];

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

  Panels<BM, BN, kQ8> regs;
  if (chunks > 0) {
    LoadPanels<BM, BN, kQ8>(p, m0, n0, kb, tid, regs);
    StorePanels<BM, BN, kQ8>(As[0], Bs[0], tid, regs);
  }
  __syncthreads();
  // Panels past ke read zeros only when ke == k; a split boundary inside k is a multiple
  // of kBK, so every chunk of a split lies inside [kb, ke).
  for (int ch = 0; ch < chunks; ++ch) {
    const int cur = ch & 1;
    if (ch + 1 < chunks) LoadPanels<BM, BN, kQ8>(p, m0, n0, kb + (ch + 1) * kBK, tid, regs);
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
    if (ch + 1 < chunks) StorePanels<BM, BN, kQ8>(As[cur ^ 1], Bs[cur ^ 1], tid, regs);
    __syncthreads();
  }

  // Element r of a 32x32 tile sits at row 8*(r/4) + 4*(lane/32) + r%4, column lane%32.
  auto row_of = [&](int i, int r) -> int64_t {
    return m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
  };
  auto col_of = [&](int j) -> int64_t { return n0 + wn * WN + j * 32 + (lane & 31); };

  if (p.splits > 1) {
    float* part = p.partials + static_cast<int64_t>(split) * p.m * p.n;
#pragma unroll
    for (int i = 0; i < SM; ++i)
#pragma unroll
      for (int j = 0; j < SN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t gr = row_of(i, r);
          const int64_t gc = col_of(j);
          if (gr < p.m && gc < p.n) part[gr * p.n + gc] = acc[i][j][r];
        }
    return;  // SplitReduceKernel adds the splits in order and applies the epilogue
  }
#pragma unroll
  for (int i = 0; i < SM; ++i)
#pragma unroll
    for (int j = 0; j < SN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t gr = row_of(i, r);
        const int64_t gc = col_of(j);
        if (gr < p.m && gc < p.n) StoreC(p.c, gr, gc, p.n, p.epi, ApplyEpilogue(acc[i][j][r], gr, gc, p.n, p.epi));
      }
}

template <int BM, int BN>
void Launch(const GemmArgs& args, bool q8, dim3 grid, hipStream_t stream) {
  if (q8) hipLaunchKernelGGL((GemmKernel<BM, BN, true>), grid, dim3(kThreads), 0, stream, args);
  else hipLaunchKernelGGL((GemmKernel<BM, BN, false>), grid, dim3(kThreads), 0, stream, args);
}

}  // namespace

void LaunchGemmF32(const float* a, const float* b, const Q8View& bq, float* c, int64_t m, int64_t k, int64_t n,
                   const Epilogue& epi, hipStream_t stream) {
  if (m < 1 || n < 1 || k < 1) Fail(ACCEL_HIP_INVALID_ARGUMENT, "GEMM shape out of range");
  Context& ctx0 = Ctx();
  const bool q8 = bq.q != nullptr;
  const int64_t cus = ctx0.cu_count > 0 ? ctx0.cu_count : 256;
  // Large tiles when they alone give about two workgroups per CU; 64x64 otherwise.
  int bm = 128, bn = 128;
  auto tiles_for = [&](int tm, int tn) { return ((m + tm - 1) / tm) * ((n + tn - 1) / tn); };
  if (tiles_for(128, 128) < 2 * cus) {
    bm = 64;
    bn = 64;
  }
  const int64_t tiles_m = (m + bm - 1) / bm;
  const int64_t tiles_n = (n + bn - 1) / bn;
  const int64_t tiles = tiles_m * tiles_n;
  int64_t splits = 1;
  if (tiles < 2 * cus) splits = std::min<int64_t>((2 * cus + tiles - 1) / tiles, std::max<int64_t>(1, k / 256));
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
    Context& ctx = Scratch(static_cast<size_t>(splits * m * n) * sizeof(float));
    args.partials = static_cast<float*>(ctx.workspace);
  }
  const dim3 grid(static_cast<uint32_t>(tiles_n), static_cast<uint32_t>(tiles_m), static_cast<uint32_t>(splits));
  if (bm == 128) Launch<128, 128>(args, q8, grid, stream);
  else Launch<64, 64>(args, q8, grid, stream);
  Check(hipGetLastError(), "GemmKernel launch");
  if (splits > 1) LaunchSplitReduce(args.partials, args.splits, m, n, c, kScalePerRow, nullptr, 0, epi, stream);
}

}  // namespace accel_hip
