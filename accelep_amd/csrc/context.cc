// Process-wide state of libaccel_hip: the bound GPU and its stream, the hipMalloc-backed
// device heap with the reference's Allocate/Free/copy semantics, the stats counters, the
// scratch workspace, timing events and graph capture.
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "host_util.h"

namespace accel_hip {
namespace {

thread_local std::string g_error;

struct Stats {
  std::atomic<int64_t> matmul_ops{0}, gemm_ops{0}, kernel_matmuls{0}, relu_epilogues{0}, gelu_epilogues{0},
      add_epilogues{0}, device_transposes{0}, bytes_to_device{0}, bytes_to_host{0};
};
Stats g_stats;
std::atomic<int64_t> g_packed_calls{0};
std::atomic<int64_t> g_packed_trips{0};

// Heap state. Ids and the live count are process-wide (src/sim_device.cc:39-40,133-161).
std::atomic<uint64_t> g_next_id{1};
std::atomic<int64_t> g_live{0};
struct LiveInfo {
  size_t bytes;
  uint64_t id;
  size_t block;  // bytes actually reserved
};
std::mutex g_heap_mu;
std::map<const char*, LiveInfo> g_live_map;  // ordered by address for range lookups
// Freed blocks by reserved size. Reuse is stream-ordered: every user of a block runs on
// the single library stream, so work queued after the Free cannot overtake earlier users.
std::multimap<size_t, void*> g_cache;
size_t g_cached_bytes = 0;
constexpr size_t kCacheLimit = size_t(8) << 30;

std::once_flag g_init_once;
Context g_ctx;
Error g_init_error{0, ""};
std::mutex g_scratch_mu;

constexpr int kEventSlots = 16;
hipEvent_t g_events[kEventSlots];

// What accel_hip_capture_end hands out: the executable graph, the Generation() at the start
// of its capture and the staged weight copies its kernels read.
struct GraphHandle {
  hipGraphExec_t exec;
  uint64_t generation;
  StagedUses staged;
};
uint64_t g_capture_generation = 0;

size_t BlockSize(size_t bytes) {
  const size_t store = bytes == 0 ? 1 : bytes;
  return (store + 255) & ~size_t(255);
}

void InitOnce() {
  int count = 0;
  hipError_t st = hipGetDeviceCount(&count);
  if (st != hipSuccess || count <= 0) {
    g_init_error = Error{ACCEL_HIP_RUNTIME_ERROR, "no HIP device is visible"};
    return;
  }
  hipDeviceProp_t prop;
  if (hipSetDevice(0) != hipSuccess || hipGetDeviceProperties(&prop, 0) != hipSuccess) {
    g_init_error = Error{ACCEL_HIP_RUNTIME_ERROR, "cannot bind HIP device 0"};
    return;
  }
  g_ctx.device = 0;
  g_ctx.arch = prop.gcnArchName;
  g_ctx.cu_count = prop.multiProcessorCount;
  if (g_ctx.arch.rfind("gfx950", 0) != 0) {
    g_init_error = Error{ACCEL_HIP_RUNTIME_ERROR, "libaccel_hip is built for gfx950 only; device is " + g_ctx.arch};
    return;
  }
  if (hipStreamCreateWithFlags(&g_ctx.stream, hipStreamNonBlocking) != hipSuccess) {
    g_init_error = Error{ACCEL_HIP_RUNTIME_ERROR, "cannot create the HIP stream"};
    return;
  }
  for (auto& ev : g_events) {
    if (hipEventCreate(&ev) != hipSuccess) {
      g_init_error = Error{ACCEL_HIP_RUNTIME_ERROR, "cannot create HIP events"};
      return;
    }
  }
  try {
    InitNoAllocScratch(g_ctx);  // with device 0 current
  } catch (const Error& e) {
    g_init_error = e;
  }
}

}  // namespace

void SetLastError(const std::string& message) { g_error = message; }
void ClearLastError() { g_error.clear(); }

[[noreturn]] void Fail(int code, const std::string& message) { throw Error{code, message}; }

void Check(hipError_t status, const char* what) {
  if (status != hipSuccess) {
    Fail(status == hipErrorOutOfMemory ? ACCEL_HIP_BAD_ALLOC : ACCEL_HIP_RUNTIME_ERROR,
         std::string(what) + ": " + hipGetErrorString(status));
  }
}

Context& Ctx() {
  std::call_once(g_init_once, InitOnce);
  if (g_init_error.code != 0) throw g_init_error;
  return g_ctx;
}

bool Capturing() {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  Check(hipStreamIsCapturing(Ctx().stream, &status), "hipStreamIsCapturing");
  return status != hipStreamCaptureStatusNone;
}

void RefuseInCapture(const char* what) {
  if (Capturing())
    Fail(ACCEL_HIP_RUNTIME_ERROR, std::string(what) +
                                      " cannot run while a HIP graph is being captured: it allocates, frees, "
                                      "synchronizes or writes with a memset; run it once before capturing");
}

namespace {
std::atomic<uint64_t> g_generation{1};
std::mutex g_pending_mu;
// Reserved up front so that DeferFree does not allocate host memory in the usual case.
std::vector<void*> g_pending = [] {
  std::vector<void*> v;
  v.reserve(256);
  return v;
}();
thread_local Arena* g_arena = nullptr;

// Serves a request from the installed arena (256-byte aligned), or returns nullptr when none.
void* FromArena(size_t bytes, const char* what) {
  Arena* arena = g_arena;
  if (arena == nullptr) return nullptr;
  const size_t start = (arena->used + 255) & ~size_t(255);
  if (start > arena->bytes || bytes > arena->bytes - start)
    Fail(ACCEL_HIP_INVALID_ARGUMENT, std::string(what) + " needs " + std::to_string(bytes) +
                                         " bytes, more than the no-allocation scratch has left (" +
                                         std::to_string(arena->bytes - std::min(start, arena->bytes)) + " of " +
                                         std::to_string(arena->bytes) + " bytes)");
  arena->used = start + bytes;
  return arena->base + start;
}
}  // namespace

uint64_t Generation() { return g_generation.load(); }
void BumpGeneration() { g_generation.fetch_add(1); }

bool GraphIsCurrent(const void* graph_exec) {
  const GraphHandle* g = static_cast<const GraphHandle*>(graph_exec);
  return g != nullptr && g->generation == Generation() && StagedUsesLive(g->staged);
}

void DeferFree(void* ptr) {
  if (ptr == nullptr) return;
  std::lock_guard<std::mutex> lock(g_pending_mu);
  g_pending.push_back(ptr);
}

void ReleasePending() {
  if (g_arena != nullptr) return;
  std::vector<void*> drop;
  {
    std::lock_guard<std::mutex> lock(g_pending_mu);
    if (g_pending.empty()) return;
    if (Capturing()) return;
    drop.swap(g_pending);
    g_pending.reserve(256);
  }
  // Kernels queued before the drop may still read these blocks; captured graphs that point
  // into them are stale (Generation moved) and are refused at launch.
  Check(hipStreamSynchronize(Ctx().stream), "hipStreamSynchronize");
  for (void* p : drop) Check(hipFree(p), "hipFree(deferred)");
}

ScopedArena::ScopedArena(Arena* arena) : previous_(g_arena) {
  arena->used = 0;
  g_arena = arena;
}
ScopedArena::~ScopedArena() { g_arena = previous_; }
Arena* CurrentArena() { return g_arena; }
bool WorkspaceFits(size_t bytes) {
  const Arena* arena = g_arena;
  if (arena == nullptr) return true;
  const size_t start = (arena->used + 255) & ~size_t(255);
  return start <= arena->bytes && bytes <= arena->bytes - start;
}

// Workspaces only grow. A replaced block goes to the deferred frees and the generation moves,
// so a graph captured before the growth is refused rather than replayed into freed memory.
void* Workspace(size_t bytes) {
  if (void* p = FromArena(bytes, "split-K workspace")) return p;
  Context& ctx = Ctx();
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (bytes > ctx.workspace_bytes) {
    RefuseInCapture("growing the split-K workspace");
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    if (ctx.workspace != nullptr) DeferFree(ctx.workspace);
    ctx.workspace = nullptr;
    BumpGeneration();
    const size_t grown = std::max(bytes, ctx.workspace_bytes * 2);
    Check(hipMalloc(&ctx.workspace, grown), "hipMalloc(workspace)");
    ctx.workspace_bytes = grown;
  }
  return ctx.workspace;
}

void* Temp(TempSlot slot, size_t bytes) {
  static void* buffers[kTempCount] = {};
  static size_t sizes[kTempCount] = {};
  if (void* p = FromArena(bytes, "temporary buffer")) {
    if (slot == kTempArrivals)  // counters must start at zero: cleared by a kernel, not a memset
      LaunchFill(static_cast<float*>(p), 0.f, static_cast<int64_t>((bytes + 3) / 4), Ctx().stream);
    return p;
  }
  Context& ctx = Ctx();
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (bytes > sizes[slot]) {
    RefuseInCapture("growing a temporary buffer");
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    if (buffers[slot] != nullptr) DeferFree(buffers[slot]);
    buffers[slot] = nullptr;
    BumpGeneration();
    const size_t grown = std::max<size_t>(bytes, std::max<size_t>(sizes[slot] * 2, 256));
    Check(hipMalloc(&buffers[slot], grown), "hipMalloc(temp)");
    // On the library stream: a null-stream memset is not ordered against it (the stream is
    // non-blocking) and could land after a kernel that already wrote the new buffer.
    Check(hipMemsetAsync(buffers[slot], 0, grown, ctx.stream), "hipMemsetAsync(temp)");
    sizes[slot] = grown;
  }
  return buffers[slot];
}

bool FindAllocation(const void* ptr, uint64_t* id, const char** base, size_t* bytes) {
  const char* p = static_cast<const char*>(ptr);
  std::lock_guard<std::mutex> lock(g_heap_mu);
  auto it = g_live_map.upper_bound(p);
  if (it == g_live_map.begin()) return false;
  --it;
  const size_t span = it->second.bytes == 0 ? 1 : it->second.bytes;
  if (p >= it->first + span) return false;
  *id = it->second.id;
  *base = it->first;
  *bytes = it->second.bytes;
  return true;
}

void NoteKernelMatmul() { g_stats.kernel_matmuls.fetch_add(1); }
void NoteKernelMatmuls(int64_t count) { g_stats.kernel_matmuls.fetch_add(count); }
void NotePackedCall(int64_t k) {
  g_packed_calls.fetch_add(1, std::memory_order_relaxed);
  g_packed_trips.fetch_add(k, std::memory_order_relaxed);
}
void NoteBytesToDevice(size_t bytes) { g_stats.bytes_to_device.fetch_add(static_cast<int64_t>(bytes)); }
void NoteBytesToHost(size_t bytes) { g_stats.bytes_to_host.fetch_add(static_cast<int64_t>(bytes)); }

// Used by the C++ runtime (accelep_amd/csrc/runtime.cc) for the counters it owns.
void NoteStat(int which, int64_t amount) {
  std::atomic<int64_t>* slots[] = {&g_stats.matmul_ops,        &g_stats.gemm_ops,       &g_stats.kernel_matmuls,
                                   &g_stats.relu_epilogues,    &g_stats.gelu_epilogues, &g_stats.add_epilogues,
                                   &g_stats.device_transposes, &g_stats.bytes_to_device, &g_stats.bytes_to_host};
  slots[which]->fetch_add(amount);
}

}  // namespace accel_hip

using namespace accel_hip;

extern "C" {

ACCEL_HIP_API const char* accel_hip_last_error(void) { return g_error.c_str(); }

ACCEL_HIP_API int accel_hip_init(void) {
  return Guard([] { Ctx(); });
}

ACCEL_HIP_API int accel_hip_synchronize(void) {
  return Guard([] { Check(hipStreamSynchronize(Ctx().stream), "hipStreamSynchronize"); });
}

ACCEL_HIP_API const char* accel_hip_device_arch(void) {
  try {
    return Ctx().arch.c_str();
  } catch (const Error& e) {
    SetLastError(e.message);
    return "";
  }
}

// Device::Allocate (src/sim_device.cc:133-147): zero-filled, non-null for 0 bytes, fresh id.
ACCEL_HIP_API int accel_hip_allocate(size_t bytes, AccelHipBuffer* out) {
  return Guard([&] {
    if (out == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "allocate needs an output buffer");
    Context& ctx = Ctx();
    RefuseInCapture("Allocate");
    ReleasePending();
    const size_t block = BlockSize(bytes);
    void* ptr = nullptr;
    {
      std::lock_guard<std::mutex> lock(g_heap_mu);
      auto it = g_cache.find(block);
      if (it != g_cache.end()) {
        ptr = it->second;
        g_cache.erase(it);
        g_cached_bytes -= block;
      }
    }
    if (ptr == nullptr) {
      hipError_t st = hipMalloc(&ptr, block);
      if (st == hipErrorOutOfMemory) {
        accel_hip_trim();
        st = hipMalloc(&ptr, block);
      }
      if (st != hipSuccess || ptr == nullptr) throw std::bad_alloc();
    }
    Check(hipMemsetAsync(ptr, 0, block, ctx.stream), "hipMemsetAsync");
    const uint64_t id = g_next_id.fetch_add(1, std::memory_order_relaxed);
    {
      std::lock_guard<std::mutex> lock(g_heap_mu);
      g_live_map.emplace(static_cast<const char*>(ptr), LiveInfo{bytes, id, block});
    }
    g_live.fetch_add(1, std::memory_order_relaxed);
    *out = AccelHipBuffer{ptr, bytes, id};
  });
}

// Device::Free (src/sim_device.cc:149-161).
ACCEL_HIP_API int accel_hip_free(AccelHipBuffer buffer) {
  return Guard([&] {
    if (buffer.data == nullptr) return;
    Context& ctx = Ctx();
    RefuseInCapture("Free");
    size_t block = 0;
    {
      std::lock_guard<std::mutex> lock(g_heap_mu);
      auto it = g_live_map.find(static_cast<const char*>(buffer.data));
      if (it == g_live_map.end() || it->second.bytes != buffer.bytes || it->second.id != buffer.id)
        Fail(ACCEL_HIP_LOGIC_ERROR, "free of unknown device buffer");
      block = it->second.block;
      g_live_map.erase(it);
      g_live.fetch_sub(1, std::memory_order_relaxed);
    }
    DropStagedForAllocation(buffer.id);
    ReleasePending();
    {
      std::lock_guard<std::mutex> lock(g_heap_mu);
      if (g_cached_bytes + block <= kCacheLimit) {
        g_cache.emplace(block, buffer.data);
        g_cached_bytes += block;
        return;
      }
    }
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    Check(hipFree(buffer.data), "hipFree");
  });
}

ACCEL_HIP_API int accel_hip_trim(void) {
  return Guard([] {
    Context& ctx = Ctx();
    RefuseInCapture("Trim");
    ReleasePending();
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    std::lock_guard<std::mutex> lock(g_heap_mu);
    for (auto& kv : g_cache) Check(hipFree(kv.second), "hipFree");
    g_cache.clear();
    g_cached_bytes = 0;
  });
}

// Device::CopyHostToDevice (src/sim_device.cc:163-172). Returns after the host bytes were
// consumed, so the caller may overwrite `src` (tests/test_runtime.cc:696-705).
ACCEL_HIP_API int accel_hip_copy_h2d(AccelHipBuffer dst, const void* src, size_t bytes) {
  return Guard([&] {
    if (bytes == 0) return;
    if (src == nullptr || dst.data == nullptr || bytes > dst.bytes)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "invalid host-to-device copy");
    Context& ctx = Ctx();
    RefuseInCapture("CopyHostToDevice");
    NoteDeviceWrite(dst.data, bytes);
    Check(hipMemcpyAsync(dst.data, src, bytes, hipMemcpyHostToDevice, ctx.stream), "hipMemcpyAsync(H2D)");
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    NoteBytesToDevice(bytes);
  });
}

// Device::CopyDeviceToHost (src/sim_device.cc:174-183).
ACCEL_HIP_API int accel_hip_copy_d2h(void* dst, AccelHipBuffer src, size_t bytes) {
  return Guard([&] {
    if (bytes == 0) return;
    if (dst == nullptr || src.data == nullptr || bytes > src.bytes)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "invalid device-to-host copy");
    Context& ctx = Ctx();
    RefuseInCapture("CopyDeviceToHost");
    Check(hipMemcpyAsync(dst, src.data, bytes, hipMemcpyDeviceToHost, ctx.stream), "hipMemcpyAsync(D2H)");
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    NoteBytesToHost(bytes);
  });
}

ACCEL_HIP_API int accel_hip_peek(void* dst, const void* device_src, size_t bytes) {
  return Guard([&] {
    if (bytes == 0) return;
    if (dst == nullptr || device_src == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "invalid peek");
    Context& ctx = Ctx();
    RefuseInCapture("peek");
    Check(hipMemcpyAsync(dst, device_src, bytes, hipMemcpyDeviceToHost, ctx.stream), "hipMemcpyAsync(peek)");
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
  });
}

ACCEL_HIP_API int accel_hip_poke(void* device_dst, const void* src, size_t bytes) {
  return Guard([&] {
    if (bytes == 0) return;
    if (src == nullptr || device_dst == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "invalid poke");
    Context& ctx = Ctx();
    RefuseInCapture("poke");
    NoteDeviceWrite(device_dst, bytes);
    Check(hipMemcpyAsync(device_dst, src, bytes, hipMemcpyHostToDevice, ctx.stream), "hipMemcpyAsync(poke)");
    Check(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
  });
}

ACCEL_HIP_API int64_t accel_hip_live_allocs(void) { return g_live.load(std::memory_order_relaxed); }

ACCEL_HIP_API void accel_hip_get_stats(AccelHipStats* out) {
  if (out == nullptr) return;
  out->matmul_ops = g_stats.matmul_ops.load();
  out->gemm_ops = g_stats.gemm_ops.load();
  out->kernel_matmuls = g_stats.kernel_matmuls.load();
  out->relu_epilogues = g_stats.relu_epilogues.load();
  out->gelu_epilogues = g_stats.gelu_epilogues.load();
  out->add_epilogues = g_stats.add_epilogues.load();
  out->device_transposes = g_stats.device_transposes.load();
  out->bytes_to_device = g_stats.bytes_to_device.load();
  out->bytes_to_host = g_stats.bytes_to_host.load();
}

// ResetAcceleratorStats (src/runtime.cc:420-433) for the counters; the profile log is the
// runtime's and is cleared there.
ACCEL_HIP_API void accel_hip_reset_stats(void) {
  g_stats.matmul_ops.store(0);
  g_stats.gemm_ops.store(0);
  g_stats.kernel_matmuls.store(0);
  g_stats.relu_epilogues.store(0);
  g_stats.gelu_epilogues.store(0);
  g_stats.add_epilogues.store(0);
  g_stats.device_transposes.store(0);
  g_stats.bytes_to_device.store(0);
  g_stats.bytes_to_host.store(0);
}

ACCEL_HIP_API int64_t accel_hip_packed_matmul_calls(void) { return g_packed_calls.load(); }
ACCEL_HIP_API int64_t accel_hip_packed_k_trips(void) { return g_packed_trips.load(); }
ACCEL_HIP_API void accel_hip_reset_packed_probes(void) {
  g_packed_calls.store(0);
  g_packed_trips.store(0);
}

ACCEL_HIP_API double accel_hip_time_ms(AccelHipWorkFn fn, void* user, int32_t iters) {
  double result = -1.0;
  const int rc = Guard([&] {
    Context& ctx = Ctx();
    Check(hipEventRecord(g_events[0], ctx.stream), "hipEventRecord");
    for (int32_t i = 0; i < iters; ++i) {
      if (fn(user) != 0) Fail(ACCEL_HIP_RUNTIME_ERROR, "timed work failed");
    }
    Check(hipEventRecord(g_events[1], ctx.stream), "hipEventRecord");
    Check(hipEventSynchronize(g_events[1]), "hipEventSynchronize");
    float ms = 0.f;
    Check(hipEventElapsedTime(&ms, g_events[0], g_events[1]), "hipEventElapsedTime");
    result = ms;
  });
  return rc == 0 ? result : -1.0;
}

ACCEL_HIP_API int accel_hip_event_record(int32_t slot) {
  return Guard([&] {
    if (slot < 0 || slot >= kEventSlots) Fail(ACCEL_HIP_INVALID_ARGUMENT, "event slot out of range");
    // Inside a capture only an external record node can be timed afterwards: a plain record
    // there leaves an event that hipEventElapsedTime refuses (invalid resource handle).
    if (Capturing())
      Check(hipEventRecordWithFlags(g_events[slot], Ctx().stream, hipEventRecordExternal), "hipEventRecordWithFlags");
    else
      Check(hipEventRecord(g_events[slot], Ctx().stream), "hipEventRecord");
  });
}

ACCEL_HIP_API int accel_hip_capture_begin(void) {
  return Guard([] {
    Context& ctx = Ctx();
    if (Capturing()) Fail(ACCEL_HIP_RUNTIME_ERROR, "a HIP graph capture is already in progress");
    ReleasePending();
    g_capture_generation = Generation();
    Check(hipStreamBeginCapture(ctx.stream, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
    BeginStagedUses();
  });
}

ACCEL_HIP_API int accel_hip_capture_end(void** graph_exec) {
  return Guard([&] {
    if (graph_exec == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "capture_end needs an output");
    *graph_exec = nullptr;
    StagedUses staged = EndStagedUses();
    hipGraph_t graph = nullptr;
    Check(hipStreamEndCapture(Ctx().stream, &graph), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    Check(st, "hipGraphInstantiate");
    // A workspace replaced or a read copy dropped since the capture began (during it too)
    // makes the graph stale.
    *graph_exec = new GraphHandle{exec, g_capture_generation, std::move(staged)};
  });
}

ACCEL_HIP_API int accel_hip_graph_launch(void* graph_exec, int32_t times) {
  return Guard([&] {
    if (graph_exec == nullptr) Fail(ACCEL_HIP_INVALID_ARGUMENT, "null graph");
    Context& ctx = Ctx();
    const GraphHandle* g = static_cast<const GraphHandle*>(graph_exec);
    if (!GraphIsCurrent(g))
      Fail(ACCEL_HIP_RUNTIME_ERROR,
           "stale HIP graph: device memory it points into (a staged weight copy, the split-K workspace or a "
           "temporary) was replaced or dropped after it was captured; capture it again");
    for (int32_t i = 0; i < times; ++i) Check(hipGraphLaunch(g->exec, ctx.stream), "hipGraphLaunch");
  });
}

ACCEL_HIP_API int accel_hip_graph_destroy(void* graph_exec) {
  return Guard([&] {
    if (graph_exec == nullptr) return;
    GraphHandle* g = static_cast<GraphHandle*>(graph_exec);
    const hipError_t st = hipGraphExecDestroy(g->exec);
    delete g;
    Check(st, "hipGraphExecDestroy");
  });
}

ACCEL_HIP_API double accel_hip_event_elapsed_ms(int32_t start_slot, int32_t end_slot) {
  double result = -1.0;
  const int rc = Guard([&] {
    if (start_slot < 0 || start_slot >= kEventSlots || end_slot < 0 || end_slot >= kEventSlots)
      Fail(ACCEL_HIP_INVALID_ARGUMENT, "event slot out of range");
    Ctx();
    Check(hipEventSynchronize(g_events[end_slot]), "hipEventSynchronize");
    float ms = 0.f;
    Check(hipEventElapsedTime(&ms, g_events[start_slot], g_events[end_slot]), "hipEventElapsedTime");
    result = ms;
  });
  return rc == 0 ? result : -1.0;
}

}  // extern "C"
