// Internal declarations shared by the host files (compiled with g++) and the kernel
// files (compiled with hipcc) of libaccel_hip.so. Not installed.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "accel_hip.h"

namespace accel_hip {

// Thrown inside the library, turned into a status code at the C-ABI edge.
struct Error {
  int code;
  std::string message;
};

[[noreturn]] void Fail(int code, const std::string& message);
void Check(hipError_t status, const char* what);

struct Context {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string arch;
  int cu_count = 0;
  // Scratch for split-K partial sums. Grown on demand (the stream is drained first).
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  // Matmuls use the exact-order kernels (exact.hip) instead of the MFMA GEMM / VALU GEMV.
  bool exact_products = false;
};

// Initialises GPU 0 and the stream on first use.
Context& Ctx();
// Takes the device address of the no-allocation entry point's fixed scratch array on
// ctx.device (which must be current); called once per device by the library's init.
void InitNoAllocScratch(const Context& ctx);
// True while the library stream is capturing a HIP graph.
bool Capturing();
// Fails with ACCEL_HIP_RUNTIME_ERROR while the library stream is capturing: `what` allocates,
// frees, synchronizes or writes with a memset, none of which a captured graph may hold.
void RefuseInCapture(const char* what);
// Split-K workspace of at least `bytes` (one per call: a later request may return the same
// memory). Grown on demand outside a capture; inside one it must already be large enough.
void* Workspace(size_t bytes);
// Library-owned device temporaries, one per purpose, grown on demand (the stream is
// drained before a buffer is replaced; a new buffer starts zeroed). Distinct from the
// split-K workspace. kTempArrivals holds counters that every kernel using them leaves zero.
enum TempSlot {
  kTempDequantA = 0,
  kTempDequantB = 1,
  kTempFlags = 2,
  kTempArrivals = 3,
  kTempSplitA = 4,   // the bf16 GEMM's hi/mid/lo activation image
  kTempRowSums = 5,  // per-tile row sums of squares of a GEMM with a fused RMSNorm
  kTempGreedy = 6,   // the many-workgroup greedy pick's count and keys
  kTempCount = 7
};
void* Temp(TempSlot slot, size_t bytes);
// Bumped whenever the split-K workspace or a temporary buffer is replaced. A graph captured
// under an older value may point into a replaced block: accel_hip_graph_launch refuses it.
uint64_t Generation();
void BumpGeneration();
// Whether a handle from accel_hip_capture_end may still be launched: no workspace or temporary
// replaced and no staged weight copy its capture read dropped since then.
bool GraphIsCurrent(const void* graph_exec);
// Device memory that kernels already queued (or a captured graph) may still read: freed at
// the next point where the stream can be drained (ReleasePending), never inside a capture or
// a no-allocation call.
void DeferFree(void* ptr);
void ReleasePending();

// A fixed block of device memory that serves Workspace() and Temp() requests for the calls
// made while it is installed on this thread (a bump allocator, reset per install), instead of
// the library's growable buffers: used by the entry point that must not allocate. A request
// that does not fit fails with ACCEL_HIP_INVALID_ARGUMENT; an arrival-counter request is
// zeroed with a fill kernel on the library stream.
struct Arena {
  char* base = nullptr;
  size_t bytes = 0;
  size_t used = 0;
};
class ScopedArena {
 public:
  explicit ScopedArena(Arena* arena);
  ~ScopedArena();
  ScopedArena(const ScopedArena&) = delete;
  ScopedArena& operator=(const ScopedArena&) = delete;

 private:
  Arena* previous_;
};
// The arena installed on this thread, or nullptr.
Arena* CurrentArena();
// Whether `bytes` more of scratch can be served: always without an arena, else if they fit
// in what the arena has left.
bool WorkspaceFits(size_t bytes);

// Stats of include/accel/runtime.h (AcceleratorStats) and the packed-GEMM probes.
void NoteKernelMatmul();
// count kernel matmuls at once (a fused caller noting the reference's logical calls).
void NoteKernelMatmuls(int64_t count);
void NotePackedCall(int64_t k);
void NoteBytesToDevice(size_t bytes);
void NoteBytesToHost(size_t bytes);

// ---- operand descriptions handed to the kernel launchers ------------------------------

// How the scale (and zero) index of element (row r, col c) of an int8 matrix view is found.
enum ScaleMode : int32_t { kScaleConst = 0, kScalePerCol = 1, kScalePerRow = 2 };

struct Q8View {
  const int8_t* q = nullptr;  // element (0, 0) of this matrix (plane.q + plane.offset)
  const float* scale = nullptr;
  const int8_t* zero = nullptr;  // nullptr: zero point 0
  int32_t mode = kScaleConst;
  int64_t const_index = 0;        // scale/zero index in kScaleConst mode
  const int8_t* tiled = nullptr;  // staged column-tiled copy of q (kGemvTileCols wide), or nullptr
  const int8_t* grouped = nullptr;  // staged group-interleaved copy of q, or nullptr
  const void* bf16 = nullptr;       // staged bf16 copy in the GEMM's MFMA operand order, or nullptr
  const void* bf16x16 = nullptr;    // staged bf16 copy in the small GEMM's operand order, or nullptr
  // Load policy of the one-row GEMV: false streams the weight (nontemporal loads, the right
  // choice for weights read once per pass over more than the 256 MB last-level cache); true
  // uses plain loads, for a caller whose whole working set stays cached between passes.
  bool cached = false;
};

// ---- weight staging (staging.cc) --------------------------------------------------------
// Width of the column tiles of a staged int8 matrix: tile t holds columns [8t, 8t + 8) of
// rows 0..kp-1 (kp = k rounded up to even), kp x 8 bytes contiguous; columns past n and the
// pad row are zero.
constexpr int64_t kGemvTileCols = 8;
inline size_t StagedTileBytes(int64_t k, int64_t n) {
  return static_cast<size_t>((n + kGemvTileCols - 1) / kGemvTileCols) * static_cast<size_t>(k + (k & 1)) *
         static_cast<size_t>(kGemvTileCols);
}
// The staged copy of the [k, n] int8 matrix at q, built on first use; nullptr when q is not
// inside a live allocation of this library (then the raw layout is read). With `create`
// false an existing copy is returned and none is built (no allocation). Building one inside
// a graph capture fails with ACCEL_HIP_RUNTIME_ERROR.
const int8_t* StagedColumnTiles(const int8_t* q, int64_t k, int64_t n, hipStream_t stream, bool create = true);
// The staged copies read by the calls recorded into a HIP graph: BeginStagedUses at the start
// of a capture, EndStagedUses at its end. StagedUsesLive is false once one of them has been
// dropped (the graph would read freed memory).
struct StagedUses {
  uint64_t drops = 0;  // copies dropped before the capture ended
  std::vector<uint64_t> serials;
};
void BeginStagedUses();
StagedUses EndStagedUses();
bool StagedUsesLive(const StagedUses& uses);
// Every write into device memory through this library calls this for the written range;
// staged copies of that allocation are dropped (their memory is freed later, DeferFree).
void NoteDeviceWrite(const void* ptr, size_t bytes);
// Heap hooks (context.cc): the allocation containing ptr; false if none.
bool FindAllocation(const void* ptr, uint64_t* id, const char** base, size_t* bytes);
void DropStagedForAllocation(uint64_t id);
void LaunchTileColumns(const int8_t* q, int64_t k, int64_t n, int8_t* dst, hipStream_t stream);
// Group-interleaved copy for the m > 1 GEMV (k a multiple of kGemvGroupRows): the 8-column
// tiles in groups of kGemvGroupTiles. For group G, slot o of the 32-row blocks (block
// b = o / 4, h = o % 4) and tile slot j, the 64 bytes at ((G * k/8 + o) * 16 + j) * 64 are
// four 16-byte pieces p = 0..3, each rows 32b + 8p + 2h and 32b + 8p + 2h + 1 of tile 16G + j
// (row-major, 8 bytes a row); 1 KB contiguous per slot o. Tiles past the last column are zero.
constexpr int64_t kGemvGroupTiles = 16;
constexpr int64_t kGemvGroupRows = 32;
inline size_t StagedGroupBytes(int64_t k, int64_t n) {
  const int64_t groups = (n + kGemvTileCols * kGemvGroupTiles - 1) / (kGemvTileCols * kGemvGroupTiles);
  return static_cast<size_t>(groups) * static_cast<size_t>(k) * static_cast<size_t>(kGemvTileCols * kGemvGroupTiles);
}
// The staged group-interleaved copy of the [k, n] int8 matrix at q (k % kGemvGroupRows == 0),
// built on first use; nullptr when q is not inside a live allocation of this library.
const int8_t* StagedGroupTiles(const int8_t* q, int64_t k, int64_t n, hipStream_t stream, bool create = true);
void LaunchTileGroups(const int8_t* q, int64_t k, int64_t n, int8_t* dst, hipStream_t stream);
// bf16 copy of a [k, n] int8 matrix (k % 32 == 0) in the operand order of
// v_mfma_f32_32x32x16_bf16's B operand, for the int8-weight GEMM: 32-column block cb (columns
// past n zero) and 16-row step s form 1 KB at (cb * k/16 + s) * 1024 bytes, 16 bytes per lane
// l = the 8 values W[16s + 8(l / 32) + j][32cb + l % 32], j = 0..7, each float(q) exactly.
inline size_t StagedBf16Bytes(int64_t k, int64_t n) {
  return static_cast<size_t>((n + 31) / 32) * static_cast<size_t>(k / 16) * 1024;
}
const void* StagedBf16Image(const int8_t* q, int64_t k, int64_t n, hipStream_t stream, bool create = true);
// fp32 B [k, n] (n % 64 == 0, k % 32 == 0) as bf16 parts in the B-operand order of the
// small-grid fp32 GEMM (GemmF32SplitBf16Kernel), each value split as hi + mid + lo: for 64-column
// tile T and 32-row group G, twelve 1 KB blocks at ((T * k/32 + G) * 12 + (2s + j) * 3 + p) * 1024
// bytes, 16 bytes per lane l = part p (0 hi, 1 mid, 2 lo) of B[32G + 16(l / 32) + 8s + t]
// [64T + 2(l % 32) + j], t = 0..7 (two values a word, the even t low).
inline size_t StagedF32PartsBytes(int64_t k, int64_t n) {
  return static_cast<size_t>(n / 64) * static_cast<size_t>(k / 32) * 12 * 1024;
}
// The staged parts of the fp32 matrix at b, or nullptr. With `create`, a copy is built on the
// second use of the same [k, n] range of an allocation of this library with no write to that
// allocation in between (a matrix that stays put across calls, i.e. a weight), never during a
// graph capture (the product then splits B on the fly).
const void* StagedF32Parts(const float* b, int64_t k, int64_t n, hipStream_t stream, bool create);
void LaunchStageF32Parts(const float* b, int64_t k, int64_t n, void* dst, hipStream_t stream);
void LaunchTileBf16(const int8_t* q, int64_t k, int64_t n, void* dst, hipStream_t stream);
// bf16 copy of a [k, n] int8 matrix (k % 32 == 0) in the operand order of
// v_mfma_f32_16x16x32_bf16's B operand, for the small int8-weight GEMM: 16-column block cb
// (columns past n zero) and 32-row block kb form 1 KB at (cb * k/32 + kb) * 1024 bytes, 16 bytes
// per lane l = the 8 values W[32kb + 8(l / 16) + j][16cb + l % 16], j = 0..7, each float(q)
// exactly (j even in the low half of a word).
inline size_t StagedBf16x16Bytes(int64_t k, int64_t n) {
  return static_cast<size_t>((n + 15) / 16) * static_cast<size_t>(k / 32) * 1024;
}
const void* StagedBf16x16(const int8_t* q, int64_t k, int64_t n, hipStream_t stream, bool create = true);
void LaunchTileBf16x16(const int8_t* q, int64_t k, int64_t n, void* dst, hipStream_t stream);
// Whether the int8-weight GEMM runs this product from a staged bf16 copy (the caller stages it).
bool GemmWantsBf16Image(int64_t m, int64_t k, int64_t n, const Q8View& v);
// Whether a weight of this form can have the small GEMM's bf16 copy at all (k <= 768).
bool GemmSmallStageable(int64_t k, int64_t n, const Q8View& v);
// Whether the int8-weight GEMM runs this m-row product (m > 16) on the small kernel from its
// bf16 copy (the caller stages it): a short k and a grid too small for the 128-tile image path.
bool GemmWantsSmall(int64_t m, int64_t k, int64_t n, const Q8View& v);
// Whether a weight of this form can have the staged bf16 copy at all (GemmWantsBf16Image
// without the grid condition on m).
bool GemmBf16Stageable(int64_t k, int64_t n, const Q8View& v);
// Whether LaunchGemvQ8 takes an m-row product with this k, n and weight view from the
// group-interleaved copy (the caller stages that copy instead of the 8-column tiles): 3 <= m
// <= 16, whole 32-row blocks, no zero points or per-row scale, and for m <= 4 a product large
// enough to give every CU a workgroup of the split-bf16 kernel (a smaller one runs on the
// narrow kernel's tiles, one workgroup per tile and no K-split exchange).
constexpr int64_t kGemvGroupMinM = 3;
bool GemvWantsGroups(int64_t m, int64_t k, int64_t n, const Q8View& v);

struct Epilogue {
  float alpha = 1.f;
  float beta = 1.f;
  const float* bias = nullptr;
  int32_t bias_rank = 0;
  int64_t bias_shape[2] = {1, 1};
  int32_t activation = ACCEL_HIP_ACT_NONE;
  const float* residual = nullptr;
  const float* rms_weight = nullptr;
  float rms_eps = 0.f;
  float* rms_out = nullptr;
  // Column split of the output (split[0] == 0: none, C is one [m, n] matrix). Otherwise
  // columns [0, split[0]) go to c as an [m, split[0]] matrix, [split[0], split[1]) to c2 and
  // [split[1], n) to c3, each row-major with its own width: one matmul over concatenated
  // weights fills several outputs (q/k/v, gate/up). Not combined with residual or rms.
  int64_t split[2] = {0, 0};
  float* c2 = nullptr;
  float* c3 = nullptr;
  // True when only alpha*acc with alpha == 1 and nothing else applies.
  bool Identity() const {
    return alpha == 1.f && bias == nullptr && activation == ACCEL_HIP_ACT_NONE && residual == nullptr &&
           rms_weight == nullptr;
  }
};

// ---- matmul dispatch shared by the C-ABI entry points (capi.cc) ------------------------
Epilogue ToEpilogue(const AccelHipEpilogue* e);
// The argument checks of accel::MatMulQuantized (src/sim_device.cc:541-548).
void QuantizedChecks(const float* a, const AccelHipQuantPlane* aq, const float* b, const AccelHipQuantPlane* bq,
                     float* c, int64_t m, int64_t k, int64_t n);
// C = A @ B with the fused epilogue, then the epilogue's RmsNorm pass (if any). With
// stage_weights false a GEMV only reads a staged weight copy that already exists and builds
// none (it reads W in place instead): no device memory is allocated.
void RunMatmul(const float* a, const AccelHipQuantPlane* aq, const float* b, const AccelHipQuantPlane* bq, float* c,
               int64_t m, int64_t k, int64_t n, const Epilogue& epi, bool stage_weights);

// ---- kernel launchers (defined in *.hip) ----------------------------------------------

// A transform the m = 1 GEMV applies to its input row before the product, inside each
// workgroup (the row is at most kGemvPrologueMaxK long):
//  * rms_weight: a = fl(float(double(x) * inv) * w), inv = 1/sqrt(sum(double(x)^2)/k + eps),
//    the sum taken exactly as RmsNormKernel takes it (same bits as the separate pass); or,
//    with rms_after, a = fl(x * w) and the sums times float(inv) at the store;
//  * silu_up: a = fl(fl(x / fl(1 + expf(-x))) * up), SiluMulKernel's formula;
//  * mul_up: a = fl(x * up), for an x that already holds fl(g / fl(1 + expf(-g))) (a GEMV that
//    stored it with silu_split0): the two kernels together form SiluMulKernel's bits.
struct GemvPrologue {
  const float* rms_weight = nullptr;
  float rms_eps = 0.f;
  // With rms_weight: multiply the sums by 1/rms at the store instead of normalizing the row
  // first (a = fl(x * w) enters the product at once; rounding differs, so fast mode only).
  // Used where the m = 1 entry kernel runs (even k <= 4096, x and w 8-byte aligned).
  bool rms_after = false;
  const float* silu_up = nullptr;
  const float* mul_up = nullptr;
  // m = 1 kernel with rms_after only: the stored values of columns [0, epi.split[0]) become
  // fl(v / fl(1 + expf(-v))), SiluMulKernel's first half (the gate of a gate/up product whose
  // down projection then takes mul_up).
  bool silu_split0 = false;
  // Decode attention partials [k / 64 heads][attn_splits][2 + 64] (m, l, acc[64]) of
  // LaunchDecodeSplitAttention: the input row is their combine, head h at rows 64h .. 64h + 63
  // (the GEMV's `a` is not read).
  const float* attn_partial = nullptr;
  int32_t attn_splits = 0;
  // Side outputs of the m = 1 entry kernel without an input transform (the launcher refuses
  // them elsewhere), for a decode step's LM head. greedy_keys [tiles of 8 columns]: each
  // tile's largest greedy key (GreedyKey of the stored value and its column), reduced by
  // LaunchGreedyKeys. advance: workgroup 0 adds 1 to advance[0] and advance[1]
  // (LaunchAdvance's step), which the product does not read.
  uint64_t* greedy_keys = nullptr;
  int32_t* advance = nullptr;
};
constexpr int64_t kGemvPrologueMaxK = 4096;
constexpr int64_t kGemvAttnMaxPairs = 2048;  // heads x splits of GemvPrologue::attn_partial

// C[m, n] = A[m, k] @ dequant(Bq)[k, n] for m <= 16 (int8 GEMV). With b.grouped (and no zero
// points or per-row scale, k % 32 == 0, A 16-byte aligned) the split-bf16 MFMA kernel runs;
// with b.tiled the 8-column tile kernels; otherwise W is read in place. A prologue needs m == 1,
// staged tiles, a per-column or whole-tensor scale without zero points and k <=
// kGemvPrologueMaxK.
void LaunchGemvQ8(const float* a, const Q8View& b, float* c, int64_t m, int64_t k, int64_t n, const Epilogue& epi,
                  hipStream_t stream, const GemvPrologue* prologue = nullptr);
// Whether an m = 1 GEMV of this shape (on staged tiles, aligned pairs, per-column or tensor scale,
// identity epilogue) runs one wave per tile: an even k <= 1024 over at least 8 tiles per CU. There
// the norm-after prologue may come with the greedy keys and the advance.
bool GemvWaveTileApplies(int64_t m, int64_t k, int64_t n);
// Input transforms of the small int8 GEMM (m > 16, GemmWantsSmall), applied to A as it is split
// into bf16 parts: the RMSNorm of each row (rms_weight, rms_eps: A = fl(x * w) and each sum times
// float(1 / rms) at the store, as GemvPrologue::rms_after; fast mode only) or a = fl(x * mul)
// elementwise (mul: [m, k] like A); and the SiLU of the stored values of columns
// [0, epi.split[0]) (silu_split0: SiluMulKernel's first half, for a gate/up product whose down
// projection takes mul = up).
constexpr int kSmallInNone = 0;
constexpr int kSmallInRms = 1;
constexpr int kSmallInMul = 2;
struct SmallPrologue {
  const float* rms_weight = nullptr;
  float rms_eps = 0.f;
  const float* mul = nullptr;
  bool silu_split0 = false;
};
// The int8-weight GEMM on the small kernel with an input transform (pro may be null): false,
// with nothing launched, where that kernel does not take the product (b.bf16x16 staged,
// GemmWantsSmall, A and the transform's operand 16-byte aligned, a column split for the SiLU).
bool LaunchGemmQ8Small(const float* a, const Q8View& b, float* c, int64_t m, int64_t k, int64_t n, const Epilogue& epi,
                       hipStream_t stream, const SmallPrologue* pro);
// An RMSNormalization of the product's rows (after the epilogue) that a GEMM may take over:
// out[i, :] = RmsNorm(C[i, :]) with the weight and eps given (SimRmsNorm's arithmetic).
struct RmsRequest {
  const float* weight = nullptr;
  float eps = 0.f;
  float* out = nullptr;
};
// C[m, n] = A[m, k] @ B[k, n]; B is fp32 (b) or int8 (bq.q != nullptr). fp32 MFMA. With rms,
// returns true when the kernel also produced the normalized rows (the caller runs the pass
// otherwise).
// stage_b: B may be staged as bf16 parts for the small-grid kernel (StagedF32Parts).
bool LaunchGemmF32(const float* a, const float* b, const Q8View& bq, float* c, int64_t m, int64_t k, int64_t n,
                   const Epilogue& epi, hipStream_t stream, const RmsRequest* rms = nullptr, bool stage_b = false);
// The int8-weight GEMM on the bf16 matrix cores (exact products, activations split into
// three bf16 parts): k % 32 == 0, n % 8 == 0, A 16-byte and q 8-byte aligned, per-column or
// whole-tensor scale, no zero points (a grid of fewer 128 x 128 tiles than CUs splits K).
// With b.bf16 (GemmWantsBf16Image) the activations are split once per call into an image
// the tiles copy as-is, the weight operands come from the staged bf16 copy, and an rms
// request is served inside (per-tile row sums of squares, then one scaling pass); *rms_done
// tells whether it was. Returns false, launching nothing, when the conditions do not hold.
bool LaunchGemmQ8Bf16(const float* a, const Q8View& b, float* c, int64_t m, int64_t k, int64_t n, const Epilogue& epi,
                      hipStream_t stream, const RmsRequest* rms = nullptr, bool* rms_done = nullptr);
// C = A @ B in the reference's order and rounding (one k-ordered chain per output, split
// products, per-element dequantization); B is fp32 (b) or int8 (bq.q != nullptr).
void LaunchExactMatmul(const float* a, const float* b, const Q8View& bq, float* c, int64_t m, int64_t k, int64_t n,
                       const Epilogue& epi, hipStream_t stream);
// partials [splits][m][n] -> C: sum in split order, times the column scale of `mode`
// (none when scale is null or mode is per-row), then the epilogue.
void LaunchSplitReduce(const float* partials, int32_t splits, int64_t m, int64_t n, float* c, int32_t mode,
                       const float* scale, int64_t const_index, const Epilogue& epi, hipStream_t stream);
// Generic dequantization of `count` elements starting at plane.offset into out (fp32).
void LaunchDequantize(const AccelHipQuantPlane& plane, int64_t count, float* out, hipStream_t stream);
void LaunchFill(float* dst, float value, int64_t count, hipStream_t stream);
void LaunchEpilogueInPlace(float* c, int64_t m, int64_t n, const Epilogue& epi, hipStream_t stream);
void LaunchRmsNormRows(const float* x, const float* weight, float* y, int64_t rows, int64_t dim, float eps,
                       hipStream_t stream);
void LaunchTranspose(const float* src, float* dst, int64_t rows, int64_t cols, hipStream_t stream);
void LaunchResidualAdd(float* dest, const float* extra, int64_t count, hipStream_t stream);
void LaunchSiluMul(float* gate, const float* up, int64_t count, hipStream_t stream);
// Writes 1 into *bad if any id is out of range (the output rows of good ids are written).
// The launchers below that take a `*_dev` pointer read that value (an id index or a
// position) from device memory when it is non-null, so a decode step can be replayed from
// a HIP graph; the scalar argument is used otherwise.
void LaunchEmbedding(const int32_t* ids, const float* table, const int8_t* qtable, const float* row_scale, float* out,
                     int64_t seq, int64_t hidden, int64_t vocab, int32_t* bad, hipStream_t stream,
                     const int32_t* index_dev = nullptr);
void LaunchRope(float* states, const float* cos_table, const float* sin_table, int64_t seq, int64_t heads,
                int64_t head_dim, int64_t position, hipStream_t stream, const int32_t* position_dev = nullptr);
void LaunchCopy(void* dst, const void* src, size_t bytes, hipStream_t stream);
// Rope on q [seq, heads, dim] in place and on k [seq, kv_heads, dim], with the rotated k and
// v [seq, kv_heads, dim] stored into cache rows [position, position + seq).
void LaunchRopeAppend(float* q, const float* k, const float* v, float* k_cache, float* v_cache, const float* cos_table,
                      const float* sin_table, int64_t seq, int64_t heads, int64_t kv_heads, int64_t head_dim,
                      int64_t position, hipStream_t stream, const int32_t* position_dev = nullptr);
// state[0] += 1, state[1] += 1 (position and produced count of a decode loop).
void LaunchAdvance(int32_t* state, hipStream_t stream);
// max_position: with position_dev, the largest position the device word may hold. work /
// work_bytes: caller-owned scratch (at least AttentionWorkBytes); null uses the library
// workspace.
// fast: prompt rows (seq > 4) with head_dim 64 may use the online-softmax kernel, whose sums
// run in another order than the reference's (rounding only); otherwise the scores keep the
// reference's bits.
void LaunchAttention(const float* q, const float* k, const float* v, float* out, int64_t seq, int64_t position,
                     int64_t heads, int64_t kv_heads, int64_t head_dim, hipStream_t stream,
                     const int32_t* position_dev = nullptr, int64_t max_position = 0, float* work = nullptr,
                     size_t work_bytes = 0, bool fast = false);
// A decode row (seq 1) with head_dim 64: RoPE of q and k, the KV append and the attention
// (LaunchRopeAppend + LaunchAttention) in one kernel, with the same output bits and the same
// cache rows. `work` holds at least AttentionWorkBytes(1, heads, max position, 64) bytes;
// `arrivals` is heads zeroed uint32 words, left zero again by each launch (launches that
// share it must not overlap). Returns false, launching nothing, when the sizes or the
// alignment do not fit (head_dim != 64, caches not 16-byte aligned).
bool LaunchDecodeAttention(const float* q, const float* k, const float* v, float* k_cache, float* v_cache,
                           const float* cos_table, const float* sin_table, float* out, int64_t position,
                           int64_t heads, int64_t kv_heads, int64_t head_dim, hipStream_t stream,
                           const int32_t* position_dev, int64_t max_position, float* work, size_t work_bytes,
                           uint32_t* arrivals);
// Fast mode, a decode row (seq 1) with head_dim 64: RoPE of q and k and the KV append as
// LaunchDecodeAttention does, then per-split softmax partials into `partial`
// [heads][splits][2 + 64] (m, l, acc) with no combine: the input prologue of the o-projection
// GEMV (GemvPrologue::attn_partial) combines them. Returns the split count (a power of two
// from 8 to 64, each split at most 256 positions; DecodeAttentionSplits(max position)), or 0,
// launching nothing, when the sizes or the alignment do not fit.
int LaunchDecodeSplitAttention(const float* q, const float* k, const float* v, float* k_cache, float* v_cache,
                               const float* cos_table, const float* sin_table, int64_t position, int64_t heads,
                               int64_t kv_heads, int64_t head_dim, hipStream_t stream, const int32_t* position_dev,
                               int64_t max_position, float* partial, size_t partial_bytes);
int DecodeAttentionSplits(int64_t max_position);
// Partial bytes per head of the largest split count (64 splits of 2 + 64 floats).
constexpr size_t kDecodeSplitMaxBytesPerHead = 64 * (2 + 64) * sizeof(float);
// Scratch bytes LaunchAttention needs for these sizes (0 when none).
size_t AttentionWorkBytes(int64_t seq, int64_t heads, int64_t max_position, int64_t head_dim);
// rng_inout is a device word holding the xorshift32 state; index_dev offsets `chosen`.
// greedy_work (at least GreedyWorkBytes(vocab) bytes, its first word zero and left zero by
// each launch; launches sharing it must not overlap) lets a greedy pick run over many
// workgroups; without it one workgroup scans the row.
void LaunchSampleToken(const float* logits, int32_t* chosen, int64_t vocab, float temperature, uint32_t* rng_inout,
                       int32_t top_k, hipStream_t stream, const int32_t* index_dev = nullptr,
                       void* greedy_work = nullptr, size_t greedy_bytes = 0);
size_t GreedyWorkBytes(int64_t vocab);
// The greedy pick from the per-tile keys a GEMV stored (GemvPrologue::greedy_keys, `count`
// keys over the logits row `logits`): chosen[*index_dev] = the id of the largest key, 0 when
// every value is a NaN or logits[0] is a NaN (the same id as LaunchSampleToken's greedy pick).
// One workgroup; count <= kGreedyKeysMax.
constexpr int64_t kGreedyKeysMax = 65536;
void LaunchGreedyKeys(const uint64_t* keys, int64_t count, const float* logits, int32_t* chosen,
                      const int32_t* index_dev, hipStream_t stream);
// LaunchGreedyKeys' pick, then the picked id's embedding row into `out` (hidden floats): the fp32
// `table` [vocab, hidden], or with table null the int8 `qtable` times row_scale[id]
// (LaunchEmbedding's row). One workgroup.
void LaunchGreedyEmbed(const uint64_t* keys, int64_t count, const int32_t* index_dev, const int8_t* qtable,
                       const float* row_scale, const float* table, const float* logits, int32_t* chosen, float* out,
                       int64_t hidden, hipStream_t stream);

}  // namespace accel_hip
