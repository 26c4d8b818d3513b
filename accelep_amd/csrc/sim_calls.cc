// The standalone device calls of AccelEP's C API (include/accel_sim.h) over this library's
// C-ABI: uploads are accel_hip_allocate + a counted copy, and accel_sim_matmul is the
// reference's sequence (src/sim_api.cc:77-107) on the GPU: allocate A and C, copy A in
// (counted), accel_hip_matmul (Device::MatMul), copy C back (counted), free.
#include <cstring>
#include <exception>
#include <mutex>
#include <new>
#include <string>

#include "accel_hip.h"
#include "accel_sim.h"

struct AccelSim {
  std::mutex mu;
};

struct AccelBuf {
  AccelHipBuffer buffer{};
};

namespace {

thread_local std::string g_sim_error;

// A device allocation freed on scope exit.
struct Scratch {
  AccelHipBuffer b{};
  ~Scratch() {
    if (b.data != nullptr) accel_hip_free(b);
  }
};

// The message of the accel_hip_* call that just failed, kept before anything else (a free in
// a destructor, say) replaces the library's last error. Returns false for `return Failed();`.
bool Failed() {
  g_sim_error = accel_hip_last_error();
  return false;
}

// Runs f; f returns Failed() after a failed accel_hip_* call, or throws.
template <typename F>
bool Run(F f) {
  try {
    if (f()) {
      g_sim_error.clear();
      return true;
    }
  } catch (const std::bad_alloc&) {
    g_sim_error = "out of memory";
  } catch (const std::exception& e) {
    g_sim_error = e.what();
  }
  return false;
}

}  // namespace

extern "C" {

ACCEL_SIM_API AccelSim* accel_sim_create(void) {
  AccelSim* sim = nullptr;
  Run([&] {
    if (accel_hip_init() != ACCEL_HIP_OK) return Failed();
    sim = new AccelSim();
    return true;
  });
  return sim;
}

ACCEL_SIM_API void accel_sim_destroy(AccelSim* sim) { delete sim; }

ACCEL_SIM_API AccelBuf* accel_sim_upload(AccelSim* sim, const float* data, int64_t count) {
  if (sim == nullptr || count < 0 || (count > 0 && data == nullptr)) {
    g_sim_error = "invalid upload";
    return nullptr;
  }
  AccelBuf* out = nullptr;
  Run([&] {
    std::lock_guard<std::mutex> lock(sim->mu);
    const size_t bytes = static_cast<size_t>(count) * sizeof(float);
    Scratch s;
    if (accel_hip_allocate(bytes, &s.b) != ACCEL_HIP_OK) return Failed();
    if (bytes > 0 && accel_hip_copy_h2d(s.b, data, bytes) != ACCEL_HIP_OK) return Failed();
    out = new AccelBuf();
    out->buffer = s.b;
    s.b = AccelHipBuffer{};  // owned by the handle now
    return true;
  });
  return out;
}

ACCEL_SIM_API void accel_sim_release(AccelSim* sim, AccelBuf* buf) {
  if (sim == nullptr || buf == nullptr) return;
  std::lock_guard<std::mutex> lock(sim->mu);
  if (buf->buffer.data != nullptr) accel_hip_free(buf->buffer);
  delete buf;
}

ACCEL_SIM_API int accel_sim_matmul(AccelSim* sim, const float* a, int64_t m, int64_t k, AccelBuf* b, int64_t n,
                                   float* c) {
  if (sim == nullptr || b == nullptr || m < 0 || k < 0 || n < 0 || (m > 0 && k > 0 && a == nullptr) ||
      (m > 0 && n > 0 && c == nullptr)) {
    g_sim_error = "invalid matmul";
    return 1;
  }
  const bool ok = Run([&] {
    std::lock_guard<std::mutex> lock(sim->mu);
    const size_t a_bytes = static_cast<size_t>(m) * static_cast<size_t>(k) * sizeof(float);
    const size_t c_bytes = static_cast<size_t>(m) * static_cast<size_t>(n) * sizeof(float);
    Scratch left, out;
    if (accel_hip_allocate(a_bytes, &left.b) != ACCEL_HIP_OK) return Failed();
    if (accel_hip_allocate(c_bytes, &out.b) != ACCEL_HIP_OK) return Failed();
    if (a_bytes > 0 && accel_hip_copy_h2d(left.b, a, a_bytes) != ACCEL_HIP_OK) return Failed();
    if (accel_hip_matmul(left.b, b->buffer, out.b, m, k, n) != ACCEL_HIP_OK) return Failed();
    if (c_bytes > 0 && accel_hip_copy_d2h(c, out.b, c_bytes) != ACCEL_HIP_OK) return Failed();
    return true;
  });
  return ok ? 0 : 1;
}

ACCEL_SIM_API void accel_sim_reset_stats(void) { accel_hip_reset_stats(); }

ACCEL_SIM_API int64_t accel_sim_matmuls(void) {
  AccelHipStats s{};
  accel_hip_get_stats(&s);
  return s.kernel_matmuls;
}

ACCEL_SIM_API int64_t accel_sim_bytes_to_device(void) {
  AccelHipStats s{};
  accel_hip_get_stats(&s);
  return s.bytes_to_device;
}

ACCEL_SIM_API int64_t accel_sim_bytes_to_host(void) {
  AccelHipStats s{};
  accel_hip_get_stats(&s);
  return s.bytes_to_host;
}

ACCEL_SIM_API const char* accel_sim_last_error(void) { return g_sim_error.c_str(); }

}  // extern "C"
