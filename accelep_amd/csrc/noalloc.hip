// accel_hip_matmul_quantized_fused_noalloc: accel_hip_matmul_quantized_fused for callers
// that must not allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// The scratch the matmul kernels need beyond the caller's inputs and outputs (split-K partial
// sums, the split-bf16 GEMV's arrival counters, a dequantized operand for plane layouts the
// kernels do not index directly) comes from one fixed device array, `scratch`, instead of the
// library's growable workspace. Each GPU holds its own copy of the array for the life of the
// process. In host code `scratch` names a host-side stand-in, not device memory: its device
// address is taken once per device with hipGetSymbolAddress (InitNoAllocScratch, called from
// the library's init with that device current) and only that address is ever handed to a
// kernel.
//
// Every call on a GPU shares that GPU's array and leaves its contents behind: calls that
// overlap on one GPU (two threads, or two captured graphs replayed concurrently) race. What
// must start at zero (the arrival counters) is cleared by a fill kernel in each call. A
// staged weight copy is read only if an earlier call built it; otherwise the GEMV reads W in
// place.
#include <hip/hip_runtime.h>

#include "common.h"
#include "host_util.h"

namespace accel_hip {
namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) char scratch[kScratchBytes];

char* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

void InitNoAllocScratch(const Context& ctx) {
  if (ctx.device < 0 || ctx.device >= kMaxDevices)
    Fail(ACCEL_HIP_RUNTIME_ERROR, "device ordinal out of range for the no-allocation scratch");
  void* ptr = nullptr;
  Check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  if (ptr == nullptr) Fail(ACCEL_HIP_RUNTIME_ERROR, "hipGetSymbolAddress(scratch) returned null");
  g_scratch_ptr[ctx.device] = static_cast<char*>(ptr);
}

}  // namespace accel_hip

using namespace accel_hip;

extern "C" {

ACCEL_HIP_API int accel_hip_matmul_quantized_fused_noalloc(const float* a, const AccelHipQuantPlane* a_quant,
                                                           const float* b, const AccelHipQuantPlane* b_quant, float* c,
                                                           int64_t m, int64_t k, int64_t n,
                                                           const AccelHipEpilogue* epilogue) {
  return Guard([&] {
    QuantizedChecks(a, a_quant, b, b_quant, c, m, k, n);
    Context& ctx = Ctx();
    char* base = g_scratch_ptr[ctx.device];
    if (base == nullptr) Fail(ACCEL_HIP_RUNTIME_ERROR, "the no-allocation scratch was not set up for this device");
    Arena arena;
    arena.base = base;
    arena.bytes = kScratchBytes;
    ScopedArena scope(&arena);
    RunMatmul(a, a_quant, b, b_quant, c, m, k, n, ToEpilogue(epilogue), /*stage_weights=*/false);
    NotePackedCall(k);
    NoteKernelMatmul();
  });
}

}  // extern "C"
