// Staged copies of constant int8 weights in the layout the GEMV streams best.
//
// accel::MatMulQuantized receives W as the row-major [k, n] int8 bytes the EP uploaded
// (src/ep.cc:843-900, src/runtime.cc:326-327). Read in that layout, a workgroup that owns a
// few columns walks k rows 14 KB apart, which HBM serves at well under half its streaming
// rate. On its first use by the GEMV, the matrix is copied once into 8-column tiles, each
// tile's k x 8 bytes contiguous (the m > 1 MFMA GEMV takes a group-interleaved form of the
// same tiles instead); later calls read the copy. The original bytes stay as
// they are, so every counted copy and every other kernel still sees the EP's layout.
//
// A copy is keyed by (allocation id, byte offset, k, n) and dropped when its allocation is
// freed or written through this library (host-to-device copies, pokes, kernel outputs).
// Device memory is only writable through this library, so a copy can never go stale.
#include <atomic>
#include <cstring>
#include <list>
#include <map>
#include <mutex>
#include <tuple>

#include "common.h"
#include "host_util.h"

namespace accel_hip {
namespace {

enum Layout : int { kLayoutTiles = 0, kLayoutGroups = 1 };

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
};

std::mutex g_mu;
std::map<Key, Entry> g_staged;
size_t g_staged_bytes = 0;
uint64_t g_tick = 0;
std::atomic<bool> g_any{false};  // fast path for writes when nothing is staged
std::atomic<uint64_t> g_epoch{0};  // counts dropped copies (a captured graph may hold one)
constexpr size_t kStagedLimit = size_t(64) << 30;

void FreeEntry(Entry& e) {
  // A kernel may still be reading the copy: drain the stream first.
  Check(hipStreamSynchronize(Ctx().stream), "hipStreamSynchronize");
  Check(hipFree(e.data), "hipFree(staged)");
  g_staged_bytes -= e.bytes;
  g_epoch.fetch_add(1);
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

const int8_t* Staged(const int8_t* q, int64_t k, int64_t n, int layout, hipStream_t stream) {
  if (k <= 0 || n <= 0) return nullptr;
  uint64_t id = 0;
  const char* base = nullptr;
  size_t alloc_bytes = 0;
  if (!FindAllocation(q, &id, &base, &alloc_bytes)) return nullptr;
  const size_t offset = static_cast<size_t>(reinterpret_cast<const char*>(q) - base);
  const size_t need = static_cast<size_t>(k) * static_cast<size_t>(n);
  if (offset + need > alloc_bytes) return nullptr;  // the matrix must lie inside one allocation
  std::lock_guard<std::mutex> lock(g_mu);
  const Key key{id, offset, k, n, layout};
  auto it = g_staged.find(key);
  if (it != g_staged.end()) {
    it->second.last_use = ++g_tick;
    return it->second.data;
  }
  const size_t bytes = layout == kLayoutGroups ? StagedGroupBytes(k, n) : StagedTileBytes(k, n);
  EvictFor(bytes);
  int8_t* dst = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&dst), bytes) != hipSuccess) return nullptr;  // fall back to raw
  if (layout == kLayoutGroups) LaunchTileGroups(q, k, n, dst, stream);
  else LaunchTileColumns(q, k, n, dst, stream);
  g_staged.emplace(key, Entry{dst, bytes, ++g_tick});
  g_staged_bytes += bytes;
  g_any.store(true);
  return dst;
}

}  // namespace

const int8_t* StagedColumnTiles(const int8_t* q, int64_t k, int64_t n, hipStream_t stream) {
  return Staged(q, k, n, kLayoutTiles, stream);
}

const int8_t* StagedGroupTiles(const int8_t* q, int64_t k, int64_t n, hipStream_t stream) {
  if (k % kGemvGroupRows != 0) return nullptr;
  return Staged(q, k, n, kLayoutGroups, stream);
}

uint64_t StagingEpoch() { return g_epoch.load(); }

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
  g_any.store(!g_staged.empty());
}

}  // namespace accel_hip
