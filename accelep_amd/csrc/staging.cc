// Staged copies of constant weights in the layouts the GEMV and GEMM kernels stream best.
//
// accel::MatMulQuantized receives W as the row-major [k, n] int8 bytes the EP uploaded
// (src/ep.cc:843-900, src/runtime.cc:326-327). Read in that layout, a workgroup that owns a
// few columns walks k rows 14 KB apart, which HBM serves at well under half its streaming
// rate. On its first use by the GEMV, the matrix is copied once into 8-column tiles, each
// tile's k x 8 bytes contiguous (the m > 1 MFMA GEMV takes a group-interleaved form of the
// same tiles instead, and the int8-weight GEMM a bf16 copy in its MFMA operand order, or in the
// small GEMM's for a short k); later
// calls read the copy. The original bytes stay as
// they are, so every counted copy and every other kernel still sees the EP's layout.
//
// The small-grid fp32 GEMM reads an fp32 weight as bf16 parts (hi + mid + lo, its operand split)
// staged the same way, but only on the matrix's second use with no write to its allocation in
// between: a product whose B is rewritten before every call (an activation) never pays for a
// copy it could not reuse.
//
// A copy is keyed by (allocation id, byte offset, k, n) and dropped when its allocation is
// freed or written through this library (host-to-device copies, pokes, kernel outputs).
// Device memory is only writable through this library, so a copy can never go stale. A
// dropped copy's memory is freed later (DeferFree) and the generation moves, so a HIP graph
// that captured kernels reading it is refused instead of replayed. A copy is never built
// inside a graph capture: the build allocates and would only be recorded, not run.
#include <atomic>
#include <cstring>
#include <list>
#include <map>
#include <mutex>
#include <set>
#include <tuple>
#include <unordered_set>
#include <vector>

#include "common.h"
#include "host_util.h"

namespace accel_hip {
namespace {

enum Layout : int { kLayoutTiles = 0, kLayoutGroups = 1, kLayoutBf16 = 2, kLayoutF32Parts = 3, kLayoutBf16x16 = 4 };

struct Key {
  uint64_t id;
  size_t offset;
  int64_t k, n;
  int layout;
  bool operator<(const Key& o) const {
    return std::tie(id, offset, k, n, layout) < std::tie(o.id, o.offset, o.k, o.n, o.layout);
  }
};

struct Entry {
  int8_t* data;
  size_t bytes;
  uint64_t last_use;
  uint64_t serial;  // unique per built copy
};

std::mutex g_mu;
std::map<Key, Entry> g_staged;
size_t g_staged_bytes = 0;
uint64_t g_tick = 0;
std::atomic<bool> g_any{false};  // fast path for writes when nothing is staged or seen
// fp32 matrices used once since their allocation was last written (staged on the next use).
std::set<Key> g_seen;
constexpr size_t kStagedLimit = size_t(64) << 30;
uint64_t g_next_serial = 1;
std::unordered_set<uint64_t> g_live_serials;
std::atomic<uint64_t> g_drops{0};
// Serials of the copies that kernels recorded during the current graph capture read.
std::atomic<bool> g_recording{false};
std::vector<uint64_t> g_recorded;

void FreeEntry(Entry& e) {
  // Kernels already queued (or a captured graph) may still read the copy: it is freed once
  // the stream has been drained, and graphs whose capture read it are refused at launch.
  DeferFree(e.data);
  g_staged_bytes -= e.bytes;
  g_live_serials.erase(e.serial);
  g_drops.fetch_add(1);
}

void EvictFor(size_t bytes) {
  while (!g_staged.empty() && g_staged_bytes + bytes > kStagedLimit) {
    auto victim = g_staged.begin();
    for (auto it = g_staged.begin(); it != g_staged.end(); ++it)
      if (it->second.last_use < victim->second.last_use) victim = it;
    FreeEntry(victim->second);
    g_staged.erase(victim);
  }
}

const int8_t* Staged(const void* src, int64_t k, int64_t n, int layout, hipStream_t stream, bool create) {
  if (k <= 0 || n <= 0) return nullptr;
  uint64_t id = 0;
  const char* base = nullptr;
  size_t alloc_bytes = 0;
  if (!FindAllocation(src, &id, &base, &alloc_bytes)) return nullptr;
  const size_t offset = static_cast<size_t>(static_cast<const char*>(src) - base);
  const size_t elem = layout == kLayoutF32Parts ? sizeof(float) : 1;
  const size_t need = static_cast<size_t>(k) * static_cast<size_t>(n) * elem;
  if (offset + need > alloc_bytes) return nullptr;  // the matrix must lie inside one allocation
  std::lock_guard<std::mutex> lock(g_mu);
  const Key key{id, offset, k, n, layout};
  auto it = g_staged.find(key);
  if (it != g_staged.end()) {
    it->second.last_use = ++g_tick;
    if (g_recording.load(std::memory_order_relaxed)) g_recorded.push_back(it->second.serial);
    return it->second.data;
  }
  if (!create) return nullptr;
  if (layout == kLayoutF32Parts) {
    // Optional: B is split on the fly without it. Never built in a capture; built on the
    // second use since the allocation was last written.
    if (Capturing()) return nullptr;
    if (g_seen.insert(key).second) {
      g_any.store(true);
      return nullptr;
    }
    g_seen.erase(key);
  } else {
    RefuseInCapture("staging an int8 weight copy for the GEMV (its first use)");
  }
  ReleasePending();
  const size_t bytes = layout == kLayoutGroups     ? StagedGroupBytes(k, n)
                       : layout == kLayoutBf16     ? StagedBf16Bytes(k, n)
                       : layout == kLayoutBf16x16  ? StagedBf16x16Bytes(k, n)
                       : layout == kLayoutF32Parts ? StagedF32PartsBytes(k, n)
                                                   : StagedTileBytes(k, n);
  EvictFor(bytes);
  int8_t* dst = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&dst), bytes) != hipSuccess) return nullptr;  // fall back to raw
  const int8_t* q = static_cast<const int8_t*>(src);
  if (layout == kLayoutGroups) LaunchTileGroups(q, k, n, dst, stream);
  else if (layout == kLayoutBf16) LaunchTileBf16(q, k, n, dst, stream);
  else if (layout == kLayoutBf16x16) LaunchTileBf16x16(q, k, n, dst, stream);
  else if (layout == kLayoutF32Parts) LaunchStageF32Parts(static_cast<const float*>(src), k, n, dst, stream);
  else LaunchTileColumns(q, k, n, dst, stream);
  const uint64_t serial = g_next_serial++;
  g_staged.emplace(key, Entry{dst, bytes, ++g_tick, serial});
  g_live_serials.insert(serial);
  g_staged_bytes += bytes;
  g_any.store(true);
  return dst;
}

}  // namespace

const int8_t* StagedColumnTiles(const int8_t* q, int64_t k, int64_t n, hipStream_t stream, bool create) {
  return Staged(q, k, n, kLayoutTiles, stream, create);
}

const int8_t* StagedGroupTiles(const int8_t* q, int64_t k, int64_t n, hipStream_t stream, bool create) {
  if (k % kGemvGroupRows != 0) return nullptr;
  return Staged(q, k, n, kLayoutGroups, stream, create);
}

const void* StagedBf16Image(const int8_t* q, int64_t k, int64_t n, hipStream_t stream, bool create) {
  if (k % 32 != 0) return nullptr;
  return Staged(q, k, n, kLayoutBf16, stream, create);
}

const void* StagedBf16x16(const int8_t* q, int64_t k, int64_t n, hipStream_t stream, bool create) {
  if (k % 32 != 0) return nullptr;
  return Staged(q, k, n, kLayoutBf16x16, stream, create);
}

const void* StagedF32Parts(const float* b, int64_t k, int64_t n, hipStream_t stream, bool create) {
  if (b == nullptr || k % 32 != 0 || n % 64 != 0) return nullptr;
  return Staged(b, k, n, kLayoutF32Parts, stream, create);
}

void BeginStagedUses() {
  std::lock_guard<std::mutex> lock(g_mu);
  g_recorded.clear();
  g_recording.store(true);
}

StagedUses EndStagedUses() {
  std::lock_guard<std::mutex> lock(g_mu);
  g_recording.store(false);
  StagedUses uses;
  uses.drops = g_drops.load();
  uses.serials.swap(g_recorded);
  return uses;
}

bool StagedUsesLive(const StagedUses& uses) {
  if (uses.drops == g_drops.load()) return true;  // nothing dropped since the capture ended
  std::lock_guard<std::mutex> lock(g_mu);
  for (uint64_t serial : uses.serials)
    if (g_live_serials.count(serial) == 0) return false;
  return true;
}

void NoteDeviceWrite(const void* ptr, size_t bytes) {
  if (!g_any.load() || ptr == nullptr) return;
  uint64_t id = 0;
  const char* base = nullptr;
  size_t alloc_bytes = 0;
  (void)bytes;
  if (!FindAllocation(ptr, &id, &base, &alloc_bytes)) return;
  DropStagedForAllocation(id);
}

void DropStagedForAllocation(uint64_t id) {
  if (!g_any.load()) return;
  std::lock_guard<std::mutex> lock(g_mu);
  for (auto it = g_staged.lower_bound(Key{id, 0, INT64_MIN, INT64_MIN, 0}); it != g_staged.end() && it->first.id == id;) {
    FreeEntry(it->second);
    it = g_staged.erase(it);
  }
  for (auto it = g_seen.lower_bound(Key{id, 0, INT64_MIN, INT64_MIN, 0}); it != g_seen.end() && it->id == id;)
    it = g_seen.erase(it);
  g_any.store(!g_staged.empty() || !g_seen.empty());
}

}  // namespace accel_hip
