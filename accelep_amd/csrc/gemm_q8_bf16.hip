// int8-weight GEMM on the bf16 matrix cores: C[m, n] = A[m, k] @ (q[k, n] * scale) for
// accel::MatMulQuantized with m > 16 (src/sim_device.cc:541-602), per-column or whole-tensor
// scale, no zero points.
//
// Exact products on v_mfma_f32_32x32x16_bf16:
//  * every weight byte is an integer in [-128, 127], which bf16 holds exactly;
//  * every activation x is split as x = hi + mid + lo with hi = bf16(x), mid = bf16(x - hi),
//    lo = bf16(x - hi - mid); both differences are exact in fp32 and the parts carry all 24
//    significand bits (for |x| >= 2^-110), so three MFMAs per k step multiply by x exactly
//    and only the fp32 accumulation rounds, as in the fp32-MFMA GEMM. The hi products and
//    the mid + lo products go to separate accumulators, added at the end, so the large sum
//    takes one rounding per MFMA step. The column scale multiplies each finished sum once.
// Bound: MFMA. 2*m*n*k algorithmic flops per call run as 3 bf16 MFMA passes, so the
// roofline is a third of the dense bf16 peak (2.5 PFLOP/s / 3 = 833 TFLOP/s), 5.3 times the
// fp32-MFMA peak.
//
//  * Workgroup tile 128 x 128, K step 32, 256 threads = 2 x 2 waves of 64 x 64 (2 x 2 MFMA
//    tiles of 32 x 32).
//  * A is loaded as fp32 (float4 along k), split on its way into LDS into three bf16 planes
//    [part][row][k]; the int8 panel is converted to bf16 and stored transposed, [column][k],
//    so every MFMA operand (8 consecutive k of one row or column) is one 16-byte LDS read.
//    Each 64-byte row holds four 16-byte k groups, group g of row R at slot g ^ ((R/2) % 4):
//    the eight rows of one read phase then cover all 32 banks, and so do the two rows of one
//    write phase of A. Each thread writes its W columns in a rotated order (column
//    (c + oct) % 8 at step c), so that the lanes of one write hit different banks.
//  * kStages register sets (2 for the 128 tile, 3 for the 64 tile): chunk ch + kStages is
//    requested while chunk ch is multiplied; the LDS planes are double buffered, one barrier
//    per chunk.
//  * Tiles are dealt to the 8 XCDs in contiguous runs, ordered in bands of 4 row tiles, so
//    the workgroups resident on one XCD share A rows and W columns in its L2.
//  * A grid of fewer tiles than CUs splits K (whole chunks); the partial sums go to the
//    workspace and SplitReduceKernel adds them in split order, scales and applies the epilogue.
#include "device_common.h"

#include <algorithm>

namespace accel_hip {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBK = 32;
constexpr int kThreads = 256;
constexpr int kRowWords = kBK / 2;  // one LDS row: 32 bf16 (16 words), k groups swizzled

// Square workgroup tiles of BM = 128 (waves of 64 x 64, 2 x 2 MFMA tiles) or 64 (waves of
// 32 x 32, one MFMA tile).
template <int BM>
struct Tile {
  static constexpr int kAPlaneWords = BM * kRowWords;
  static constexpr int kBufWords = 4 * kAPlaneWords;  // three A planes + the W plane (BN = BM)
  static constexpr int kS = BM / 64;                  // MFMA tiles per wave along each side
  static constexpr int kARows = BM / 32;              // float4 loads of A per thread
  static constexpr int kOcts = BM / 8;                // 8-column octets of a W row
  // Register sets of panels in flight (the 128 tile's two accumulator sets leave room for 2).
  static constexpr int kStages = BM == 128 ? 2 : 3;
};
constexpr int kXcds = 8;
constexpr int kBand = 4;  // row tiles per band of the tile order

struct Q8GemmArgs {
  const float* a;
  const int8_t* q;
  const float* scale;
  int32_t mode;
  int64_t const_index;
  float* c;
  int64_t m, k, n;
  int32_t tiles_m, tiles_n, tiles, tiles_per_xcd;
  int64_t k_per_split;  // a multiple of kBK
  float* partials;      // [splits][m][n] raw sums when the K range is split, else nullptr
  Epilogue epi;
};

// The global part of one chunk, as loaded: A rows (tid / 8) + 32i, k quad tid % 8; W rows
// 2 * kp and 2 * kp + 1 of column octet oct, kp = tid / octets < 16 (for BM = 64 the upper
// half of the threads load no W).
template <int BM>
struct Panels {
  float4 a[Tile<BM>::kARows];
  u32x2 b[2];
};

// Rows and columns past the matrix read a clamped, valid element; their results are never
// stored (every chunk lies inside k, which is a multiple of kBK).
template <int BM>
__device__ __forceinline__ void LoadPanels(const Q8GemmArgs& p, int64_t m0, int64_t n0, int64_t k0, int tid,
                                           Panels<BM>& r) {
  const int kq = tid & 7;
#pragma unroll
  for (int i = 0; i < Tile<BM>::kARows; ++i) {
    const int64_t row = m0 + (tid >> 3) + 32 * i;
    const int64_t rc = row < p.m ? row : p.m - 1;
    r.a[i] = *reinterpret_cast<const float4*>(p.a + rc * p.k + k0 + 4 * kq);
  }
  constexpr int kOcts = Tile<BM>::kOcts;
  const int kp = tid / kOcts;
  if (kp >= kBK / 2) return;
  const int64_t col = n0 + 8 * (tid % kOcts);
  const int64_t cc = col < p.n ? col : p.n - 8;
  const int64_t kr = k0 + 2 * kp;
#pragma unroll
  for (int h = 0; h < 2; ++h) r.b[h] = *reinterpret_cast<const u32x2*>(p.q + (kr + h) * p.n + cc);
}

// Word offset of 16-byte k group g (0..3) of LDS row `row`.
__device__ __forceinline__ int GroupWord(int row, int g) { return row * kRowWords + 4 * (g ^ ((row >> 1) & 3)); }

template <int BM>
__device__ __forceinline__ void StorePanels(uint32_t* buf, int tid, const Panels<BM>& r) {
  constexpr int kAPlaneWords = Tile<BM>::kAPlaneWords;
  const int kq = tid & 7;
#pragma unroll
  for (int i = 0; i < Tile<BM>::kARows; ++i) {
    const int row = (tid >> 3) + 32 * i;
    const float x[4] = {r.a[i].x, r.a[i].y, r.a[i].z, r.a[i].w};
    uint32_t part[3][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float x0 = x[2 * h];
      const float x1 = x[2 * h + 1];
      part[0][h] = PackBf16(x0, x1);
      const float r0 = x0 - Bf16Low(part[0][h]);
      const float r1 = x1 - Bf16High(part[0][h]);
      part[1][h] = PackBf16(r0, r1);
      part[2][h] = PackBf16(r0 - Bf16Low(part[1][h]), r1 - Bf16High(part[1][h]));
    }
    const int wo = GroupWord(row, kq >> 1) + 2 * (kq & 1);
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) *reinterpret_cast<u32x2*>(&buf[pl * kAPlaneWords + wo]) = u32x2{part[pl][0], part[pl][1]};
  }
  // W transposed: word kp of column row nl holds rows (2kp, 2kp + 1). The 8 bytes of each W
  // row are rotated by s = oct % 8 first (byte c of the result is column (c + s) % 8).
  uint32_t* wplane = buf + 3 * kAPlaneWords;
  constexpr int kOcts = Tile<BM>::kOcts;
  const int kp = tid / kOcts;
  if (kp >= kBK / 2) return;
  const int oct = tid % kOcts;
  const int s = oct & 7;
  uint32_t rot[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t lo = (s & 4) ? r.b[h][1] : r.b[h][0];
    const uint32_t hi = (s & 4) ? r.b[h][0] : r.b[h][1];
    rot[h][0] = __builtin_amdgcn_alignbyte(hi, lo, s & 3);
    rot[h][1] = __builtin_amdgcn_alignbyte(lo, hi, s & 3);
  }
  const int wsub = kp & 3;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int nl = 8 * oct + ((c + s) & 7);
    wplane[GroupWord(nl, kp >> 2) + wsub] =
        PackBf16(ByteToFloat(rot[0][c >> 2], c & 3), ByteToFloat(rot[1][c >> 2], c & 3));
  }
}

// The hi parts accumulate into acc_hi, the mid and lo parts into acc_ml: the sum that carries
// the rounding of most consequence then takes one MFMA add per k step instead of three.
template <int BM>
__device__ __forceinline__ void ComputeChunk(const uint32_t* buf, int lane, int wm, int wn,
                                             v16f (&acc_hi)[Tile<BM>::kS][Tile<BM>::kS],
                                             v16f (&acc_ml)[Tile<BM>::kS][Tile<BM>::kS]) {
  constexpr int kAPlaneWords = Tile<BM>::kAPlaneWords;
  constexpr int S = Tile<BM>::kS;
  const uint32_t* wplane = buf + 3 * kAPlaneWords;
#pragma unroll
  for (int ks = 0; ks < kBK; ks += 16) {
    const int g = ks / 8 + (lane >> 5);  // k group: 8 consecutive k of this lane's row / column
    u32x4 bv[S];
#pragma unroll
    for (int j = 0; j < S; ++j)
      bv[j] = *reinterpret_cast<const u32x4*>(&wplane[GroupWord(wn * (BM / 2) + j * 32 + (lane & 31), g)]);
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) {
      u32x4 av[S];
#pragma unroll
      for (int i = 0; i < S; ++i)
        av[i] = *reinterpret_cast<const u32x4*>(
            &buf[pl * kAPlaneWords + GroupWord(wm * (BM / 2) + i * 32 + (lane & 31), g)]);
#pragma unroll
      for (int i = 0; i < S; ++i)
#pragma unroll
        for (int j = 0; j < S; ++j) {
          v16f& acc = pl == 0 ? acc_hi[i][j] : acc_ml[i][j];
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av[i]),
                                                        __builtin_bit_cast(bf16x8, bv[j]), acc, 0, 0, 0);
        }
    }
  }
}

template <int BM>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(BM == 128 ? 2 : 3))) void GemmQ8Bf16Kernel(
    Q8GemmArgs p) {
  constexpr int kBufWords = Tile<BM>::kBufWords;
  constexpr int S = Tile<BM>::kS;
  constexpr int kStages = Tile<BM>::kStages;
  __shared__ __align__(16) uint32_t lds[2 * kBufWords];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  // Contiguous runs of tiles per XCD (workgroup b runs on XCD b % 8), in bands of kBand row
  // tiles walked column by column.
  const int t = (blockIdx.x % kXcds) * p.tiles_per_xcd + blockIdx.x / kXcds;
  if (t >= p.tiles) return;
  const int band_tiles = kBand * p.tiles_n;
  const int band = t / band_tiles;
  const int in_band = t % band_tiles;
  const int rows_in_band = min(kBand, p.tiles_m - band * kBand);
  const int tm = band * kBand + in_band % rows_in_band;
  const int tn = in_band / rows_in_band;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  const int64_t n0 = static_cast<int64_t>(tn) * BM;
  const int64_t kb = static_cast<int64_t>(blockIdx.y) * p.k_per_split;
  const int chunks = static_cast<int>((min(p.k, kb + p.k_per_split) - kb) / kBK);

  v16f acc[S][S], acc_ml[S][S];
#pragma unroll
  for (int i = 0; i < S; ++i)
#pragma unroll
    for (int j = 0; j < S; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.f;
        acc_ml[i][j][r] = 0.f;
      }

  Panels<BM> regs[kStages];
#pragma unroll
  for (int st = 0; st < kStages; ++st)
    if (st < chunks) LoadPanels(p, m0, n0, kb + static_cast<int64_t>(st) * kBK, tid, regs[st]);
  StorePanels(lds, tid, regs[0]);
  __syncthreads();
  for (int base = 0; base < chunks; base += kStages) {
#pragma unroll
    for (int st = 0; st < kStages; ++st) {
      const int ch = base + st;
      if (ch >= chunks) break;  // workgroup-uniform
      // No branch inside a step, so the scheduler can interleave the next panel's conversion
      // and LDS stores with this chunk's MFMAs. Past the end, the loads repeat the last chunk
      // and the store goes to the idle buffer; neither is used.
      const int nxt = min(ch + kStages, chunks - 1);
      LoadPanels(p, m0, n0, kb + static_cast<int64_t>(nxt) * kBK, tid, regs[st]);
      ComputeChunk<BM>(lds + (ch & 1) * kBufWords, lane, wm, wn, acc, acc_ml);
      StorePanels(lds + ((ch + 1) & 1) * kBufWords, tid, regs[(st + 1) % kStages]);
      if (BM == 128) {
        // Interleave: one MFMA, then a share of the conversion work and of the LDS stores.
#pragma unroll
        for (int q = 0; q < 24; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // VALU
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
        }
      }
      LdsBarrier();  // the panels in flight for later chunks stay in flight
    }
  }

#pragma unroll
  for (int i = 0; i < S; ++i)
#pragma unroll
    for (int j = 0; j < S; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = acc[i][j][r] + acc_ml[i][j][r];

  // Element r of a 32 x 32 tile sits at row 8*(r/4) + 4*(lane/32) + r%4, column lane%32.
  if (p.partials != nullptr) {  // SplitReduceKernel adds the splits in order, scales, applies the epilogue
    float* part = p.partials + static_cast<int64_t>(blockIdx.y) * p.m * p.n;
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int64_t col = n0 + wn * (BM / 2) + j * 32 + (lane & 31);
      if (col >= p.n) continue;
#pragma unroll
      for (int i = 0; i < S; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (row < p.m) part[row * p.n + col] = acc[i][j][r];
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const int64_t col = n0 + wn * (BM / 2) + j * 32 + (lane & 31);
    if (col >= p.n) continue;
    const float cs = p.scale[p.mode == kScalePerCol ? col : p.const_index];
#pragma unroll
    for (int i = 0; i < S; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < p.m) StoreC(p.c, row, col, p.n, p.epi, ApplyEpilogue(__fmul_rn(acc[i][j][r], cs), row, col, p.n, p.epi));
      }
  }
}

// ---- the 128-tile GEMM from an activation image and a staged bf16 weight ---------------
//
// The kernel above spends most of its VALU issue splitting A (in each of the column tiles
// that read it) and converting W (in each of the row tiles). Here both happen once:
//  * SplitAImageKernel splits A once per call into the hi/mid/lo image: for row tile tm and
//    chunk c, 24 KB holding exactly what one chunk's three LDS planes hold (same swizzle), so
//    a tile copies it into LDS with 16-byte loads and stores and no arithmetic;
//  * the weight is staged once as bf16 in the B-operand order of v_mfma_f32_32x32x16_bf16
//    (StagedBf16Image), so each wave loads its B operands straight from memory, one 16-byte
//    load per lane and 32 x 16 block, with no LDS round trip and no conversion.
// Products stay exact (the same three parts and the same accumulators as above).
// With a fused RMSNorm each tile also leaves the double sum of squares of its stored values
// per row ([tiles_n][m]); RmsScaleKernel adds a row's tile sums in tile order and scales it.

constexpr int kImgRows = 128;
constexpr int kImgPlaneWords = kImgRows * kRowWords;  // 2048 words
constexpr int kImgBlockWords = 3 * kImgPlaneWords;    // 24 KB per (row tile, chunk)
constexpr int kImgBlockVecs = kImgBlockWords / 4;     // 1536 16-byte pieces, 6 per thread
constexpr int kImgBStages = 3;                         // weight-operand register sets in flight

// Word offset of 16-byte k group g of image row `row`: g ^ f(row) with f(row) = ((row >> 1) ^
// (row >> 2)) & 3. A 16-byte LDS read by 8 (32 banks) or 16 (64 banks) lanes of consecutive
// rows then covers every bank once: those rows' bases take 2 (or 4) bank quarters, and f sends
// the rows sharing a base to distinct groups.
template <int kSwz>
__device__ __forceinline__ int ImageWord(int row, int g) {
  if constexpr (kSwz == 0) return GroupWord(row, g);
  return row * kRowWords + 4 * (g ^ (((row >> 1) ^ (row >> 2)) & 3));
}

// One thread per (row tile, chunk, row, k group): the three parts of 8 activations.
template <int kSwz>
__global__ void SplitAImageKernel(const float* __restrict__ a, uint32_t* __restrict__ img, int64_t m, int64_t k,
                                  int32_t chunks, int64_t items) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= items) return;
  const int64_t blk = t >> 9;  // tm * chunks + c
  const int rem = static_cast<int>(t & 511);
  const int r = rem >> 2;
  const int g = rem & 3;
  const int64_t tm = blk / chunks;
  const int c = static_cast<int>(blk - tm * chunks);
  const int64_t row = tm * kImgRows + r;
  float x[8];
  if (row < m) {
    const float4* src = reinterpret_cast<const float4*>(a + row * k + static_cast<int64_t>(c) * kBK + 8 * g);
    const float4 v0 = src[0], v1 = src[1];
    x[0] = v0.x; x[1] = v0.y; x[2] = v0.z; x[3] = v0.w;
    x[4] = v1.x; x[5] = v1.y; x[6] = v1.z; x[7] = v1.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = 0.f;
  }
  uint32_t part[3][4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const float x0 = x[2 * h];
    const float x1 = x[2 * h + 1];
    part[0][h] = PackBf16(x0, x1);
    const float r0 = x0 - Bf16Low(part[0][h]);
    const float r1 = x1 - Bf16High(part[0][h]);
    part[1][h] = PackBf16(r0, r1);
    part[2][h] = PackBf16(r0 - Bf16Low(part[1][h]), r1 - Bf16High(part[1][h]));
  }
  uint32_t* dst = img + blk * kImgBlockWords + ImageWord<kSwz>(r, g);
#pragma unroll
  for (int pl = 0; pl < 3; ++pl)
    *reinterpret_cast<u32x4*>(dst + pl * kImgPlaneWords) = u32x4{part[pl][0], part[pl][1], part[pl][2], part[pl][3]};
}

// One thread per 16-byte lane piece of the staged bf16 weight (layout: StagedBf16Bytes).
__global__ void TileBf16Kernel(const int8_t* __restrict__ q, int64_t k, int64_t n, u32x4* __restrict__ out,
                               int64_t k_steps, int64_t items) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= items) return;
  const int lane = static_cast<int>(t & 63);
  const int64_t blk = t >> 6;
  const int64_t cb = blk / k_steps;
  const int64_t st = blk - cb * k_steps;
  const int64_t col = cb * 32 + (lane & 31);
  const int64_t k0 = st * 16 + 8 * (lane >> 5);
  uint32_t w[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const float q0 = col < n ? static_cast<float>(q[(k0 + 2 * h) * n + col]) : 0.f;
    const float q1 = col < n ? static_cast<float>(q[(k0 + 2 * h + 1) * n + col]) : 0.f;
    w[h] = PackBf16(q0, q1);
  }
  out[t] = u32x4{w[0], w[1], w[2], w[3]};
}

struct ImageArgs {
  const u32x4* a_img;  // [tiles_m][chunks] blocks of kImgBlockVecs
  const u32x4* w_img;  // staged bf16 weight, [col_blocks][k_steps][64]
  const float* scale;
  int32_t mode;
  int64_t const_index;
  float* c;
  int64_t m, k, n;
  int32_t tiles_m, tiles_n, tiles, tiles_per_xcd, chunks, col_blocks;
  int64_t k_steps;  // k / 16
  double* row_ss;   // [tiles_n][m] row sums of squares of the stored values, or nullptr
  Epilogue epi;
};

// One chunk's image block, copied by kNT threads (kImgBlockVecs / kNT 16-byte pieces each).
template <int kNT>
__device__ __forceinline__ void LoadImageA(const ImageArgs& p, int64_t a_block, int ch, int tid,
                                           u32x4 (&r)[kImgBlockVecs / kNT]) {
  const u32x4* src = p.a_img + (a_block + ch) * kImgBlockVecs;
#pragma unroll
  for (int i = 0; i < kImgBlockVecs / kNT; ++i) r[i] = src[i * kNT + tid];
}

// B operands of one chunk for this wave: k steps 2ch, 2ch + 1 of its kCB 32-column blocks
// (blocks past the weight repeat the last one; their columns are never stored).
template <int kCB>
__device__ __forceinline__ void LoadImageB(const ImageArgs& p, int cb0, int ch, int lane, u32x4 (&r)[2][kCB]) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int j = 0; j < kCB; ++j) {
      const int64_t cb = min(cb0 + j, p.col_blocks - 1);
      r[ks][j] = p.w_img[(cb * p.k_steps + 2 * ch + ks) * 64 + lane];
    }
}

template <int kNT>
__device__ __forceinline__ void StoreImageA(uint32_t* buf, int tid, const u32x4 (&r)[kImgBlockVecs / kNT]) {
#pragma unroll
  for (int i = 0; i < kImgBlockVecs / kNT; ++i) reinterpret_cast<u32x4*>(buf)[i * kNT + tid] = r[i];
}

// The chunk's six operand groups (2 k steps x 3 planes), each two 16-byte LDS reads of A and
// four MFMAs. The reads of group g + 1 are issued before the MFMAs of group g, so each LDS
// round trip runs under the previous group's matrix work instead of ahead of its own.
template <int kSwz>
__device__ __forceinline__ void ReadImageGroup(const uint32_t* buf, int lane, int wm, int grp, u32x4 (&av)[2]) {
  const int ks = grp / 3, pl = grp % 3;
  const int g = 2 * ks + (lane >> 5);
#pragma unroll
  for (int i = 0; i < 2; ++i)
    av[i] = *reinterpret_cast<const u32x4*>(&buf[pl * kImgPlaneWords + ImageWord<kSwz>(wm * 64 + i * 32 + (lane & 31), g)]);
}

template <int kSwz, int kCB>
__device__ __forceinline__ void ComputeImageChunk(const uint32_t* buf, const u32x4 (&bv)[2][kCB], int lane, int wm,
                                                  v16f (&acc_hi)[2][kCB], v16f (&acc_ml)[2][kCB]) {
  u32x4 av[2][2];
  ReadImageGroup<kSwz>(buf, lane, wm, 0, av[0]);
#pragma unroll
  for (int grp = 0; grp < 6; ++grp) {
    if (grp + 1 < 6) ReadImageGroup<kSwz>(buf, lane, wm, grp + 1, av[(grp + 1) & 1]);
    const int ks = grp / 3, pl = grp % 3;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < kCB; ++j) {
        v16f& acc = pl == 0 ? acc_hi[i][j] : acc_ml[i][j];
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av[grp & 1][i]),
                                                      __builtin_bit_cast(bf16x8, bv[ks][j]), acc, 0, 0, 0);
      }
  }
  // Keep that order: group g + 1's two LDS reads, then group g's 2 * kCB MFMAs.
#pragma unroll
  for (int grp = 0; grp < 6; ++grp) {
    if (grp + 1 < 6) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * kCB, 0);            // MFMA
  }
}

template <int kSwz, int kNB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void GemmQ8Bf16ImageKernel(ImageArgs p) {
  __shared__ __align__(16) uint32_t lds[2 * kImgBlockWords];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int t = (blockIdx.x % kXcds) * p.tiles_per_xcd + blockIdx.x / kXcds;
  if (t >= p.tiles) return;
  const int band_tiles = kBand * p.tiles_n;
  const int band = t / band_tiles;
  const int in_band = t % band_tiles;
  const int rows_in_band = min(kBand, p.tiles_m - band * kBand);
  const int tm = band * kBand + in_band % rows_in_band;
  const int tn = in_band / rows_in_band;
  const int64_t m0 = static_cast<int64_t>(tm) * kImgRows;
  const int64_t n0 = static_cast<int64_t>(tn) * kImgRows;
  const int64_t a_block = static_cast<int64_t>(tm) * p.chunks;
  const int cb0 = tn * 4 + wn * 2;
  const int chunks = p.chunks;

  v16f acc[2][2], acc_ml[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.f;
        acc_ml[i][j][r] = 0.f;
      }

  // A: chunk ch sits in LDS buffer ch % 2 while chunk ch + 1 waits in areg[(ch + 1) % 2] and
  // chunk ch + 2 is loading into areg[ch % 2]. B: chunk ch's operands in breg[ch % 3], the
  // next two chunks' loading. Loads past the last chunk repeat it (never used).
  u32x4 breg[kNB][2][2];
#pragma unroll
  for (int s = 0; s < kNB; ++s) LoadImageB<2>(p, cb0, min(s, chunks - 1), lane, breg[s]);
  u32x4 areg[2][kImgBlockVecs / kThreads];
  LoadImageA<kThreads>(p, a_block, 0, tid, areg[0]);
  LoadImageA<kThreads>(p, a_block, min(1, chunks - 1), tid, areg[1]);
  StoreImageA<kThreads>(lds, tid, areg[0]);
  __syncthreads();
  constexpr int kUnroll = kNB == 3 ? 6 : 2 * kNB;  // a multiple of both rings, so every ring index is static
  for (int base = 0; base < chunks; base += kUnroll) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int ch = base + u;
      if (ch >= chunks) break;  // workgroup-uniform
      LoadImageA<kThreads>(p, a_block, min(ch + 2, chunks - 1), tid, areg[u % 2]);
      ComputeImageChunk<kSwz, 2>(lds + (u % 2) * kImgBlockWords, breg[u % kNB], lane, wm, acc, acc_ml);
      StoreImageA<kThreads>(lds + ((u + 1) % 2) * kImgBlockWords, tid, areg[(u + 1) % 2]);
      LoadImageB<2>(p, cb0, min(ch + kNB, chunks - 1), lane, breg[u % kNB]);
      LdsBarrier();  // the A blocks and B operands in flight for later chunks stay in flight
    }
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = acc[i][j][r] + acc_ml[i][j][r];

  // Element r of a 32 x 32 tile sits at row 8*(r/4) + 4*(lane/32) + r%4, column lane%32.
  float cs[2];
  bool col_ok[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = n0 + wn * 64 + j * 32 + (lane & 31);
    col_ok[j] = col < p.n;
    cs[j] = col_ok[j] ? p.scale[p.mode == kScalePerCol ? col : p.const_index] : 0.f;
  }
  double* row_part = reinterpret_cast<double*>(lds);  // [2 wn][128 rows], after the last barrier
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int rl = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      const int64_t row = m0 + rl;
      double ss = 0.0;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t col = n0 + wn * 64 + j * 32 + (lane & 31);
        if (row < p.m && col_ok[j]) {  // the epilogue reads bias and residual only inside [m, n]
          const float v = ApplyEpilogue(__fmul_rn(acc[i][j][r], cs[j]), row, col, p.n, p.epi);
          StoreC(p.c, row, col, p.n, p.epi, v);
          ss += static_cast<double>(v) * static_cast<double>(v);
        }
      }
      if (p.row_ss != nullptr) {
        // Sum over the wave's 64 columns: the 32 lanes holding this row, then LDS per wave column.
        ss += XorLane<1>(ss);
        ss += XorLane<2>(ss);
        ss += XorLane<4>(ss);
        ss += XorLane<8>(ss);
        ss += XorLane<16>(ss);
        if ((lane & 31) == 0) row_part[wn * kImgRows + rl] = ss;
      }
    }
  if (p.row_ss != nullptr) {
    __syncthreads();
    if (tid < kImgRows && m0 + tid < p.m)
      p.row_ss[static_cast<int64_t>(tn) * p.m + m0 + tid] = row_part[tid] + row_part[kImgRows + tid];
  }
}

// ---- the wide grid: 8 waves per workgroup, tiles of 128 x 256 and 128 x 128 --------------
//
// The image kernel's 128 x 128 tiles read 40 KB of operands per 32-k chunk from L2 (the
// 24 KB A block, and 8 KB of B for each of the two wave rows) for 3.1 Mflop of MFMA work.
// With realistic operands the chip holds the kernel at its power limit (about 1.75 GHz against
// 2.37 with the matrix cores idle), so operand traffic costs clock as well as time. A
// workgroup of 8 waves (2 rows x 4 columns of 64 x 64) over a 128 x 256 tile shares each A
// block among four waves instead of two: 56 KB per chunk for 6.3 Mflop, 30 % less L2 traffic
// per flop and 17 % less LDS traffic. Such a workgroup holds a CU alone (2 waves per SIMD),
// so the tile count must divide evenly over the CUs: the grid mixes 128 x 256 tiles over
// the first columns (a whole number of rounds) with one round of 128 x 128 tiles (each wave
// 64 x 32) over the rest, which end together. WideGridFor picks the split.
constexpr int kWideThreads = 512;

struct WideGrid {
  int32_t big;        // 128 x 256 tiles (workgroups [0, big))
  int32_t big_tn;     // their column tiles per row tile
  int32_t small_tn;   // 128 x 128 column tiles per row tile, over columns [big_cols, n)
  int32_t big_cols;
};

// One tile of the wide grid: kCB 32-column blocks per wave (2: 128 x 256; 1: 128 x 128).
// slot is the 128-column index of the tile's first column in row_ss.
template <int kCB, int kNB>
__device__ __forceinline__ void WideTile(const ImageArgs& p, uint32_t* lds, int tm, int64_t n0, int cb0, int slot) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2;
  const int wn = wave & 3;
  const int64_t m0 = static_cast<int64_t>(tm) * kImgRows;
  const int64_t a_block = static_cast<int64_t>(tm) * p.chunks;
  const int chunks = p.chunks;
  v16f acc[2][kCB], acc_ml[2][kCB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < kCB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc[i][j][r] = 0.f;
        acc_ml[i][j][r] = 0.f;
      }
  // The image kernel's pipeline: A chunk ch in LDS buffer ch % 2, ch + 1 in registers, ch + 2
  // loading; B operands of chunks ch .. ch + kNB - 1 in the register ring.
  u32x4 breg[kNB][2][kCB];
#pragma unroll
  for (int s = 0; s < kNB; ++s) LoadImageB<kCB>(p, cb0, min(s, chunks - 1), lane, breg[s]);
  u32x4 areg[2][kImgBlockVecs / kWideThreads];
  LoadImageA<kWideThreads>(p, a_block, 0, tid, areg[0]);
  LoadImageA<kWideThreads>(p, a_block, min(1, chunks - 1), tid, areg[1]);
  StoreImageA<kWideThreads>(lds, tid, areg[0]);
  __syncthreads();
  constexpr int kUnroll = kNB == 3 ? 6 : 2 * kNB;
  for (int base = 0; base < chunks; base += kUnroll) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int ch = base + u;
      if (ch >= chunks) break;  // workgroup-uniform
      LoadImageA<kWideThreads>(p, a_block, min(ch + 2, chunks - 1), tid, areg[u % 2]);
      ComputeImageChunk<1, kCB>(lds + (u % 2) * kImgBlockWords, breg[u % kNB], lane, wm, acc, acc_ml);
      StoreImageA<kWideThreads>(lds + ((u + 1) % 2) * kImgBlockWords, tid, areg[(u + 1) % 2]);
      LoadImageB<kCB>(p, cb0, min(ch + kNB, chunks - 1), lane, breg[u % kNB]);
      LdsBarrier();
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < kCB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = acc[i][j][r] + acc_ml[i][j][r];

  // Element r of a 32 x 32 tile sits at row 8*(r/4) + 4*(lane/32) + r%4, column lane%32.
  float cs[kCB];
#pragma unroll
  for (int j = 0; j < kCB; ++j) {
    const int64_t col = n0 + wn * 32 * kCB + j * 32 + (lane & 31);  // < n: the grid covers whole tiles
    cs[j] = p.scale[p.mode == kScalePerCol ? col : p.const_index];
  }
  double* row_part = reinterpret_cast<double*>(lds);  // [4 wn][128 rows], after the last barrier
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int rl = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      const int64_t row = m0 + rl;
      double ss = 0.0;
#pragma unroll
      for (int j = 0; j < kCB; ++j) {
        const int64_t col = n0 + wn * 32 * kCB + j * 32 + (lane & 31);
        if (row < p.m) {  // the epilogue reads bias and residual only inside [m, n]
          const float v = ApplyEpilogue(__fmul_rn(acc[i][j][r], cs[j]), row, col, p.n, p.epi);
          StoreC(p.c, row, col, p.n, p.epi, v);
          ss += static_cast<double>(v) * static_cast<double>(v);
        }
      }
      if (p.row_ss != nullptr) {
        ss += XorLane<1>(ss);
        ss += XorLane<2>(ss);
        ss += XorLane<4>(ss);
        ss += XorLane<8>(ss);
        ss += XorLane<16>(ss);
        if ((lane & 31) == 0) row_part[wn * kImgRows + rl] = ss;
      }
    }
  if (p.row_ss != nullptr) {
    __syncthreads();
    if (tid < kImgRows && m0 + tid < p.m) {
      const double t = row_part[tid] + row_part[kImgRows + tid] + row_part[2 * kImgRows + tid] +
                       row_part[3 * kImgRows + tid];
      p.row_ss[static_cast<int64_t>(slot) * p.m + m0 + tid] = t;
      // A 256-column tile fills its second slot with zero: RmsScaleKernel adds every slot.
      if (kCB == 2) p.row_ss[static_cast<int64_t>(slot + 1) * p.m + m0 + tid] = 0.0;
    }
  }
}

// Tile index t of a run dealt to XCDs in contiguous runs and ordered in bands of kBand row
// tiles (as in the image kernel), for a grid of `count` tiles with tn_count column tiles.
__device__ __forceinline__ void WideTileIndex(int b, int count, int tiles_m, int tn_count, int& tm, int& tn) {
  const int t = (b % kXcds) * (count / kXcds) + b / kXcds;
  const int band_tiles = kBand * tn_count;
  const int band = t / band_tiles;
  const int in_band = t % band_tiles;
  const int rows_in_band = min(kBand, tiles_m - band * kBand);
  tm = band * kBand + in_band % rows_in_band;
  tn = in_band / rows_in_band;
}

template <int kNB>
__global__ __launch_bounds__(kWideThreads) __attribute__((amdgpu_waves_per_eu(2))) void GemmQ8Bf16WideKernel(
    ImageArgs p, WideGrid g) {
  __shared__ __align__(16) uint32_t lds[2 * kImgBlockWords];
  const int wn = (threadIdx.x >> 6) & 3;
  const int b = blockIdx.x;
  int tm, tn;
  if (b < g.big) {
    WideTileIndex(b, g.big, p.tiles_m, g.big_tn, tm, tn);
    WideTile<2, kNB>(p, lds, tm, static_cast<int64_t>(tn) * 256, tn * 8 + wn * 2, 2 * tn);
  } else {
    WideTileIndex(b - g.big, p.tiles_m * g.small_tn, p.tiles_m, g.small_tn, tm, tn);
    WideTile<1, kNB>(p, lds, tm, g.big_cols + static_cast<int64_t>(tn) * 128, g.big_cols / 32 + tn * 4 + wn,
                     g.big_cols / 128 + tn);
  }
}

// The wide grid's split for an m x n product on `cus` CUs, or false: n a multiple of 128,
// exactly one round of 128 x 128 tiles (one per CU) over the last columns and a whole number
// (at least 2) of rounds of 128 x 256 tiles over the others.
bool WideGridFor(int64_t m, int64_t n, int64_t cus, WideGrid* g) {
  const int64_t tiles_m = (m + kImgRows - 1) / kImgRows;
  if (n % 128 != 0 || cus <= 0 || cus % kXcds != 0 || cus % tiles_m != 0) return false;
  const int64_t nb = n / 128;
  const int64_t small_tn = cus / tiles_m;
  if (small_tn > nb || (nb - small_tn) % 2 != 0) return false;
  const int64_t big_tn = (nb - small_tn) / 2;
  if (big_tn < 1 || (tiles_m * big_tn) % cus != 0 || tiles_m * big_tn / cus < 2) return false;
  if (tiles_m * big_tn > 0x7fffffff / kBand) return false;
  g->big = static_cast<int32_t>(tiles_m * big_tn);
  g->big_tn = static_cast<int32_t>(big_tn);
  g->small_tn = static_cast<int32_t>(small_tn);
  g->big_cols = static_cast<int32_t>(big_tn * 256);
  return true;
}

// out[row, :] = float(double(c[row, :]) * inv) * w with inv = 1/sqrt(ss/n + eps) and ss the
// row's tile sums added in tile order (SimRmsNorm's arithmetic, src/sim_rmsnorm.cc:7-20).
// One workgroup per row; c and out may be the same buffer.
__global__ void RmsScaleKernel(const float* c, const double* __restrict__ row_ss, int32_t tiles_n,
                               const float* __restrict__ w, float* out, int64_t m, int64_t n, float eps, bool vec) {
  __shared__ double part[256];
  __shared__ double inv_s;
  const int64_t row = blockIdx.x;
  for (int t = threadIdx.x; t < tiles_n; t += blockDim.x) {
    if (t < 256) part[t] = row_ss[static_cast<int64_t>(t) * m + row];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double total = 0.0;
    for (int t = 0; t < tiles_n && t < 256; ++t) total += part[t];
    for (int t = 256; t < tiles_n; ++t) total += row_ss[static_cast<int64_t>(t) * m + row];
    inv_s = 1.0 / sqrt(total / static_cast<double>(n) + static_cast<double>(eps));
  }
  __syncthreads();
  const double inv = inv_s;
  const float* in = c + row * n;
  float* o = out + row * n;
  if (vec) {  // n % 4 == 0 and c, w, out 16-byte aligned
    for (int64_t i = 4 * threadIdx.x; i < n; i += 4 * blockDim.x) {
      const float4 x = *reinterpret_cast<const float4*>(in + i);
      const float4 g = *reinterpret_cast<const float4*>(w + i);
      float4 y;
      y.x = __fmul_rn(static_cast<float>(static_cast<double>(x.x) * inv), g.x);
      y.y = __fmul_rn(static_cast<float>(static_cast<double>(x.y) * inv), g.y);
      y.z = __fmul_rn(static_cast<float>(static_cast<double>(x.z) * inv), g.z);
      y.w = __fmul_rn(static_cast<float>(static_cast<double>(x.w) * inv), g.w);
      *reinterpret_cast<float4*>(o + i) = y;
    }
  } else {
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x)
      o[i] = __fmul_rn(static_cast<float>(static_cast<double>(in[i]) * inv), w[i]);
  }
}

// ---- small products: 16-row blocks over all of a short k, no LDS round trip per chunk ------
// An m > 16 product whose 128-tile grid leaves CUs idle and whose k is short (k <= 768: the
// Llama prompt's q/k/v, o and gate/up at 512 rows; k = 1536, its down projection, when the grid
// fits the CUs in one round) spends its time in GemmQ8Bf16Kernel's
// per-chunk chain of LDS stores, barrier and LDS reads, and in a split-K reduce launch. Here a
// workgroup of kSmallWaves waves owns one 16-row block and kSmallWaves 16-column blocks over
// all of k (no K split):
//  * the block's 16 activation rows are split once into hi/mid/lo bf16 planes in LDS, in the
//    A-operand order of v_mfma_f32_16x16x32_bf16 (piece (kb, part, lane) at (kb * 3 + part) *
//    64 + lane: row 16 rb + lane % 16, k = 32 kb + 8 (lane / 16) .. + 7), one barrier;
//  * each wave reads its column block's B operands straight from the staged copy
//    (StagedBf16x16), one 16-byte load per lane and 32 x 16 block, kSmallStages blocks in flight;
//  * three MFMAs per block, hi into one accumulator and mid + lo into another, added at the end,
//    as in the kernels above: exact products, only the fp32 accumulation rounds. The column
//    scale and the epilogue apply at the store.
constexpr int kSmallWaves = 8;
constexpr int kSmallThreads = kSmallWaves * 64;
constexpr int kSmallStages = 6;
constexpr int64_t kSmallMaxK = 768;
constexpr int kSmallMaxBlocks = static_cast<int>(kSmallMaxK / kBK);
// One longer k with an instance of its own (the Llama prompt's down projection): its activation
// parts take 144 KB of LDS, so one workgroup fills a CU; it is taken only where the grid fits
// the CUs in one round.
constexpr int64_t kSmallWideK = 1536;
constexpr int kSmallWideBlocks = static_cast<int>(kSmallWideK / kBK);

struct SmallArgs {
  const float* a;
  const u32x4* w16;  // StagedBf16x16 layout
  const float* scale;
  int32_t mode;
  int64_t const_index;
  float* c;
  int32_t m, k, n;     // k % 32 == 0, 32 <= k <= kSmallMaxK, or k == kSmallWideK
  int32_t col_groups;  // workgroups along n: ceil(ceil(n / 16) / kSmallWaves)
  Epilogue epi;
  SmallPrologue pro;   // the input transform (the kernel's kIn) and the SiLU store
};

// One thread per 16-byte lane piece of the staged copy (layout: StagedBf16x16Bytes).
__global__ void TileBf16x16Kernel(const int8_t* __restrict__ q, int64_t k, int64_t n, u32x4* __restrict__ out,
                                  int64_t kbs, int64_t items) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= items) return;
  const int lane = static_cast<int>(t & 63);
  const int64_t blk = t >> 6;
  const int64_t cb = blk / kbs;
  const int64_t kb = blk - cb * kbs;
  const int64_t col = cb * 16 + (lane & 15);
  const int64_t k0 = kb * 32 + 8 * (lane >> 4);
  uint32_t w[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const float q0 = col < n ? static_cast<float>(q[(k0 + 2 * h) * n + col]) : 0.f;
    const float q1 = col < n ? static_cast<float>(q[(k0 + 2 * h + 1) * n + col]) : 0.f;
    w[h] = PackBf16(q0, q1);
  }
  out[t] = u32x4{w[0], w[1], w[2], w[3]};
}

// kKbs: k / 32 fixed at compile time (every loop unrolled, constant LDS offsets), or 0 for any k.
// kIn: the input transform applied to A as it is split (SmallPrologue): kSmallInNone; kSmallInRms,
// the RMSNorm of each row applied after the product, as the decode GEMV's rms_after does: A =
// fl(x * w) enters the product and each stored sum is multiplied by float(1 / rms), with rms from
// the row's double sum of squares formed from the same loads (RmsNormKernel normalizes first and
// sums in another order, so the fast mode only); kSmallInMul, a = fl(x * mul) elementwise.
// The pointers and sizes the first loads need lead the arguments (preloaded into SGPRs at wave
// launch, so the weight and activation loads issue without a kernarg round trip); the output
// and the epilogue come from `args`, read behind the loads.
template <int kKbs, int kIn>
__global__ __launch_bounds__(kSmallThreads) void GemmQ8SmallKernel(const float* a, const u32x4* w16, const float* scale,
                                                                   int32_t m, int32_t k, int32_t n, int32_t col_groups,
                                                                   SmallArgs args) {
  SmallArgs p = args;
  p.a = a;
  p.w16 = w16;
  p.scale = scale;
  p.m = m;
  p.k = k;
  p.n = n;
  p.col_groups = col_groups;
  static_assert(kKbs >= 0 && (kKbs <= kSmallMaxBlocks || kKbs == kSmallWideBlocks), "k blocks");
  __shared__ u32x4 parts[(kKbs > 0 ? kKbs : kSmallMaxBlocks) * 3 * 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kbs = kKbs > 0 ? kKbs : p.k / kBK;
  const int cbs = (p.n + 15) / 16;
  const int rb = static_cast<int>(blockIdx.x) / p.col_groups;
  const int cb = (static_cast<int>(blockIdx.x) % p.col_groups) * kSmallWaves + wave;
  const int cbc = cb < cbs ? cb : cbs - 1;  // a wave past the last block loads a valid one, stores nothing
  const u32x4* wp = p.w16 + static_cast<int64_t>(cbc) * kbs * 64 + lane;
  // The first kSmallStages blocks of W are requested before the split, which they do not need.
  u32x4 rw[kSmallStages];
#pragma unroll
  for (int i = 0; i < kSmallStages; ++i) {
    rw[i] = wp[static_cast<int64_t>(i < kbs ? i : kbs - 1) * 64];
    __builtin_amdgcn_sched_barrier(0);
  }
  // kSmallInRms: each thread's pieces are all of one row (l % 16 = tid % 16); its share of the
  // row's double sum of squares, summed over the wave's four lanes of the row, then over the
  // waves through LDS after the split's barrier.
  __shared__ double row_ss[kIn == kSmallInRms ? kSmallWaves : 1][16];
  __shared__ float row_inv[kIn == kSmallInRms ? 16 : 1];
  double ss = 0.0;
  for (int pc = tid; pc < kbs * 64; pc += kSmallThreads) {
    const int kb = pc >> 6;
    const int l = pc & 63;
    const int row = rb * 16 + (l & 15);
    float x[8];
    if (row < p.m) {
      const int64_t at = static_cast<int64_t>(row) * p.k + kb * kBK + 8 * (l >> 4);
      const float4* src = reinterpret_cast<const float4*>(p.a + at);
      const float4 x0 = src[0], x1 = src[1];
      x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
      x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
      if constexpr (kIn == kSmallInRms) {
        const float4* wsrc = reinterpret_cast<const float4*>(p.pro.rms_weight + kb * kBK + 8 * (l >> 4));
        const float4 w0 = wsrc[0], w1 = wsrc[1];
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          ss += static_cast<double>(x[i]) * static_cast<double>(x[i]);
          x[i] = __fmul_rn(x[i], wv[i]);
        }
      } else if constexpr (kIn == kSmallInMul) {
        const float4* usrc = reinterpret_cast<const float4*>(p.pro.mul + at);
        const float4 u0 = usrc[0], u1 = usrc[1];
        const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = __fmul_rn(x[i], uv[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = 0.f;
    }
    u32x4 hi, mid, lo;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      uint32_t ph, pm, pl;
      SplitBf16Pair(x[2 * h], x[2 * h + 1], ph, pm, pl);
      hi[h] = ph;
      mid[h] = pm;
      lo[h] = pl;
    }
    parts[(kb * 3 + 0) * 64 + l] = hi;
    parts[(kb * 3 + 1) * 64 + l] = mid;
    parts[(kb * 3 + 2) * 64 + l] = lo;
  }
  if constexpr (kIn == kSmallInRms) {
    ss += XorLane<16>(ss);
    ss += XorLane<32>(ss);
    if (lane < 16) row_ss[wave][lane] = ss;
  }
  // An LDS-only barrier: the W blocks in flight stay in flight.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if constexpr (kIn == kSmallInRms) {
    // float(1 / rms) of each row, once: the 16 lanes of the last wave, before its products.
    if (wave == kSmallWaves - 1 && lane < 16) {
      double total = row_ss[0][lane];
#pragma unroll
      for (int wv = 1; wv < kSmallWaves; ++wv) total += row_ss[wv][lane];
      row_inv[lane] = static_cast<float>(1.0 / sqrt(total / static_cast<double>(p.k) + static_cast<double>(p.pro.rms_eps)));
    }
  }
  v4f acc_hi = v4f{0.f, 0.f, 0.f, 0.f};
  v4f acc_ml = v4f{0.f, 0.f, 0.f, 0.f};
  for (int kb0 = 0; kb0 < kbs; kb0 += kSmallStages) {
#pragma unroll
    for (int st = 0; st < kSmallStages; ++st) {
      const int kb = kb0 + st;
      if (kb >= kbs) break;  // uniform
      const u32x4 a0 = parts[(kb * 3 + 0) * 64 + lane];
      const u32x4 a1 = parts[(kb * 3 + 1) * 64 + lane];
      const u32x4 a2 = parts[(kb * 3 + 2) * 64 + lane];
      acc_hi = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a0), __builtin_bit_cast(bf16x8, rw[st]),
                                                       acc_hi, 0, 0, 0);
      acc_ml = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1), __builtin_bit_cast(bf16x8, rw[st]),
                                                       acc_ml, 0, 0, 0);
      acc_ml = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a2), __builtin_bit_cast(bf16x8, rw[st]),
                                                       acc_ml, 0, 0, 0);
      if (kb + kSmallStages < kbs) rw[st] = wp[static_cast<int64_t>(kb + kSmallStages) * 64];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if constexpr (kIn == kSmallInRms) LdsBarrier();  // row_inv is written
  if (cb >= cbs) return;
  // Element r of the 16 x 16 tile: row 16 rb + 4 (lane / 16) + r, column 16 cb + lane % 16.
  const int col = cb * 16 + (lane & 15);
  if (col >= p.n) return;
  const float cs = p.scale[p.mode == kScalePerCol ? col : p.const_index];
  // SmallPrologue::silu_split0: the stored values of columns [0, epi.split[0]) are SiLU(v),
  // SiluMulKernel's first half.
  const bool silu = p.pro.silu_split0 && col < p.epi.split[0];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = rb * 16 + 4 * (lane >> 4) + r;
    if (row < p.m) {
      float sum = acc_hi[r] + acc_ml[r];
      // The norm after the product: the sum of fl(x * w) * q times float(1 / rms) of the row.
      if constexpr (kIn == kSmallInRms) sum = __fmul_rn(sum, row_inv[4 * (lane >> 4) + r]);
      float v = ApplyEpilogue(__fmul_rn(sum, cs), row, col, p.n, p.epi);
      if (silu) v = __fdiv_rn(v, __fadd_rn(1.f, expf(-v)));
      StoreC(p.c, row, col, p.n, p.epi, v);
    }
  }
}

}  // namespace

void LaunchTileBf16(const int8_t* q, int64_t k, int64_t n, void* dst, hipStream_t stream) {
  const int64_t k_steps = k / 16;
  const int64_t items = (n + 31) / 32 * k_steps * 64;
  if (items <= 0) return;
  const int64_t grid = (items + kThreads - 1) / kThreads;
  if (grid > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "weight too large to stage");
  hipLaunchKernelGGL(TileBf16Kernel, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, stream, q, k, n,
                     static_cast<u32x4*>(dst), k_steps, items);
  Check(hipGetLastError(), "TileBf16Kernel launch");
}

void LaunchTileBf16x16(const int8_t* q, int64_t k, int64_t n, void* dst, hipStream_t stream) {
  const int64_t kbs = k / 32;
  const int64_t items = (n + 15) / 16 * kbs * 64;
  if (items <= 0) return;
  const int64_t grid = (items + kThreads - 1) / kThreads;
  if (grid > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "weight too large to stage");
  hipLaunchKernelGGL(TileBf16x16Kernel, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, stream, q, k, n,
                     static_cast<u32x4*>(dst), kbs, items);
  Check(hipGetLastError(), "TileBf16x16Kernel launch");
}

bool GemmSmallStageable(int64_t k, int64_t n, const Q8View& v) {
  if (v.q == nullptr || v.zero != nullptr || (v.mode != kScalePerCol && v.mode != kScaleConst)) return false;
  return k >= kBK && (k <= kSmallMaxK || k == kSmallWideK) && k % kBK == 0 && n >= 8 && n % 8 == 0 &&
         n < (int64_t(1) << 30);
}

bool GemmWantsSmall(int64_t m, int64_t k, int64_t n, const Q8View& v) {
  if (m <= 16 || m >= (int64_t(1) << 30) || !GemmSmallStageable(k, n, v) || GemmWantsBf16Image(m, k, n, v)) return false;
  const int64_t groups = ((n + 15) / 16 + kSmallWaves - 1) / kSmallWaves;
  const int64_t blocks = (m + 15) / 16 * groups;
  if (k == kSmallWideK) {
    Context& ctx = Ctx();
    return blocks <= (ctx.cu_count > 0 ? ctx.cu_count : 256);
  }
  return blocks <= 0x7fffffff;
}

bool GemmBf16Stageable(int64_t k, int64_t n, const Q8View& v) {
  if (v.q == nullptr || v.zero != nullptr || (v.mode != kScalePerCol && v.mode != kScaleConst)) return false;
  return k >= 2 * kBK && n >= 8 && k % kBK == 0 && n % 8 == 0 && k / kBK <= 0x7fffffff;
}

bool GemmWantsBf16Image(int64_t m, int64_t k, int64_t n, const Q8View& v) {
  if (m < 1 || !GemmBf16Stageable(k, n, v)) return false;
  Context& ctx = Ctx();
  const int64_t cus = ctx.cu_count > 0 ? ctx.cu_count : 256;
  return ((m + 127) / 128) * ((n + 127) / 128) >= cus;  // the 128-tile grid, no K split
}

bool LaunchGemmQ8Small(const float* a, const Q8View& b, float* c, int64_t m, int64_t k, int64_t n, const Epilogue& epi,
                       hipStream_t stream, const SmallPrologue* pro) {
  if (b.bf16x16 == nullptr || !GemmWantsSmall(m, k, n, b) || reinterpret_cast<uintptr_t>(a) % 16 != 0) return false;
  const SmallPrologue none{};
  const SmallPrologue& pr = pro != nullptr ? *pro : none;
  const int in = pr.rms_weight != nullptr ? kSmallInRms : pr.mul != nullptr ? kSmallInMul : kSmallInNone;
  const auto aligned = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  if ((in == kSmallInRms && !aligned(pr.rms_weight)) || (in == kSmallInMul && !aligned(pr.mul)) ||
      (pr.silu_split0 && epi.split[0] <= 0))
    return false;
  SmallArgs sa;
  sa.a = a;
  sa.w16 = static_cast<const u32x4*>(b.bf16x16);
  sa.scale = b.scale;
  sa.mode = b.mode;
  sa.const_index = b.const_index;
  sa.c = c;
  sa.m = static_cast<int32_t>(m);
  sa.k = static_cast<int32_t>(k);
  sa.n = static_cast<int32_t>(n);
  sa.col_groups = static_cast<int32_t>(((n + 15) / 16 + kSmallWaves - 1) / kSmallWaves);
  sa.epi = epi;
  sa.pro = pr;
  const int64_t blocks = (m + 15) / 16 * sa.col_groups;
  const dim3 grid(static_cast<uint32_t>(blocks));
#define ACCEL_SMALL_LAUNCH(KB, IN)                                                                              \
  hipLaunchKernelGGL((GemmQ8SmallKernel<KB, IN>), grid, dim3(kSmallThreads), 0, stream, sa.a, sa.w16, sa.scale, \
                     sa.m, sa.k, sa.n, sa.col_groups, sa)
#define ACCEL_SMALL_K(IN)                                          \
  do {                                                             \
    if (k == 576) ACCEL_SMALL_LAUNCH(18, IN);                      \
    else if (k == 768) ACCEL_SMALL_LAUNCH(24, IN);                 \
    else if (k == kSmallWideK) ACCEL_SMALL_LAUNCH(kSmallWideBlocks, IN); \
    else ACCEL_SMALL_LAUNCH(0, IN);                                \
  } while (0)
  if (in == kSmallInRms) ACCEL_SMALL_K(kSmallInRms);
  else if (in == kSmallInMul) ACCEL_SMALL_K(kSmallInMul);
  else ACCEL_SMALL_K(kSmallInNone);
#undef ACCEL_SMALL_K
#undef ACCEL_SMALL_LAUNCH
  Check(hipGetLastError(), "GemmQ8SmallKernel launch");
  return true;
}

bool LaunchGemmQ8Bf16(const float* a, const Q8View& b, float* c, int64_t m, int64_t k, int64_t n, const Epilogue& epi,
                      hipStream_t stream, const RmsRequest* rms, bool* rms_done) {
  if (rms_done != nullptr) *rms_done = false;
  if (b.q == nullptr || b.zero != nullptr || (b.mode != kScalePerCol && b.mode != kScaleConst)) return false;
  if (m < 1 || k < kBK || n < 8 || k % kBK != 0 || n % 8 != 0) return false;
  if (reinterpret_cast<uintptr_t>(a) % 16 != 0 || reinterpret_cast<uintptr_t>(b.q) % 8 != 0) return false;
  if (b.bf16 != nullptr && GemmWantsBf16Image(m, k, n, b)) {
    const int64_t tiles_m = (m + kImgRows - 1) / kImgRows;
    const int64_t tiles_n = (n + kImgRows - 1) / kImgRows;
    const int64_t chunks = k / kBK;
    const size_t img_bytes = static_cast<size_t>(tiles_m * chunks) * kImgBlockWords * sizeof(uint32_t);
    const size_t ss_bytes = rms != nullptr ? static_cast<size_t>(tiles_n * m) * sizeof(double) : 0;
    if (tiles_m * tiles_n * kBand <= 0x7fffffff && WorkspaceFits(img_bytes + ss_bytes + 512)) {
      ImageArgs ia;
      ia.a_img = static_cast<const u32x4*>(Temp(kTempSplitA, img_bytes));
      ia.w_img = static_cast<const u32x4*>(b.bf16);
      ia.scale = b.scale;
      ia.mode = b.mode;
      ia.const_index = b.const_index;
      ia.c = c;
      ia.m = m;
      ia.k = k;
      ia.n = n;
      ia.tiles_m = static_cast<int32_t>(tiles_m);
      ia.tiles_n = static_cast<int32_t>(tiles_n);
      ia.tiles = static_cast<int32_t>(tiles_m * tiles_n);
      ia.tiles_per_xcd = static_cast<int32_t>((ia.tiles + kXcds - 1) / kXcds);
      ia.chunks = static_cast<int32_t>(chunks);
      ia.col_blocks = static_cast<int32_t>((n + 31) / 32);
      ia.k_steps = k / 16;
      ia.row_ss = rms != nullptr ? static_cast<double*>(Temp(kTempRowSums, ss_bytes)) : nullptr;
      ia.epi = epi;
      const int64_t items = tiles_m * chunks * 512;
      const dim3 sgrid(static_cast<uint32_t>((items + kThreads - 1) / kThreads));
      uint32_t* img = const_cast<uint32_t*>(reinterpret_cast<const uint32_t*>(ia.a_img));
      hipLaunchKernelGGL(SplitAImageKernel<1>, sgrid, dim3(kThreads), 0, stream, a, img, m, k, ia.chunks, items);
      Check(hipGetLastError(), "SplitAImageKernel launch");
      const int64_t cus = Ctx().cu_count > 0 ? Ctx().cu_count : 256;
      WideGrid wg;
      if (WideGridFor(m, n, cus, &wg)) {
        const uint32_t blocks = static_cast<uint32_t>(wg.big + ia.tiles_m * wg.small_tn);
        hipLaunchKernelGGL((GemmQ8Bf16WideKernel<kImgBStages>), dim3(blocks), dim3(kWideThreads), 0, stream, ia, wg);
        Check(hipGetLastError(), "GemmQ8Bf16WideKernel launch");
      } else {
        hipLaunchKernelGGL((GemmQ8Bf16ImageKernel<1, kImgBStages>),
                           dim3(static_cast<uint32_t>(ia.tiles_per_xcd * kXcds)), dim3(kThreads), 0, stream, ia);
        Check(hipGetLastError(), "GemmQ8Bf16ImageKernel launch");
      }
      if (rms != nullptr) {
        if (m > 0x7fffffff) Fail(ACCEL_HIP_INVALID_ARGUMENT, "RmsNorm has too many rows");
        const bool vec = n % 4 == 0 && reinterpret_cast<uintptr_t>(c) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(rms->weight) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(rms->out) % 16 == 0;
        hipLaunchKernelGGL(RmsScaleKernel, dim3(static_cast<uint32_t>(m)), dim3(kThreads), 0, stream, c, ia.row_ss,
                           ia.tiles_n, rms->weight, rms->out, m, n, rms->eps, vec);
        Check(hipGetLastError(), "RmsScaleKernel launch");
        if (rms_done != nullptr) *rms_done = true;
      }
      return true;
    }
  }
  if (LaunchGemmQ8Small(a, b, c, m, k, n, epi, stream, nullptr)) return true;
  Context& ctx0 = Ctx();
  const int64_t cus = ctx0.cu_count > 0 ? ctx0.cu_count : 256;
  // 128 x 128 tiles when they give one per CU, else 64 x 64.
  const int bm = ((m + 127) / 128) * ((n + 127) / 128) >= cus ? 128 : 64;
  const int64_t tiles_m = (m + bm - 1) / bm;
  const int64_t tiles_n = (n + bm - 1) / bm;
  const int64_t tiles = tiles_m * tiles_n;
  if (tiles * kBand > 0x7fffffff) return false;
  // A grid short of one tile per CU splits K into ranges of whole chunks (at least 3 each),
  // to about two workgroups per CU; a second kernel adds the partial sums in split order.
  const int64_t chunks = k / kBK;
  int64_t splits = 1;
  if (tiles < cus) splits = std::max<int64_t>(1, std::min<int64_t>((2 * cus + tiles - 1) / tiles, chunks / 3));
  const int64_t kper = (chunks + splits - 1) / splits * kBK;
  splits = (k + kper - 1) / kper;
  if (splits > 65535) return false;
  Q8GemmArgs args;
  args.a = a;
  args.q = b.q;
  args.scale = b.scale;
  args.mode = b.mode;
  args.const_index = b.const_index;
  args.c = c;
  args.m = m;
  args.k = k;
  args.n = n;
  args.tiles_m = static_cast<int32_t>(tiles_m);
  args.tiles_n = static_cast<int32_t>(tiles_n);
  args.tiles = static_cast<int32_t>(tiles);
  args.tiles_per_xcd = static_cast<int32_t>((tiles + kXcds - 1) / kXcds);
  args.k_per_split = kper;
  args.partials = nullptr;
  args.epi = epi;
  if (splits > 1) args.partials = static_cast<float*>(Workspace(static_cast<size_t>(splits * m * n) * sizeof(float)));
  const dim3 grid(static_cast<uint32_t>(args.tiles_per_xcd * kXcds), static_cast<uint32_t>(splits));
  if (bm == 128) hipLaunchKernelGGL(GemmQ8Bf16Kernel<128>, grid, dim3(kThreads), 0, stream, args);
  else hipLaunchKernelGGL(GemmQ8Bf16Kernel<64>, grid, dim3(kThreads), 0, stream, args);
  Check(hipGetLastError(), "GemmQ8Bf16Kernel launch");
  if (splits > 1) LaunchSplitReduce(args.partials, static_cast<int32_t>(splits), m, n, c, b.mode, b.scale, b.const_index,
                                    epi, stream);
  return true;
}

}  // namespace accel_hip
