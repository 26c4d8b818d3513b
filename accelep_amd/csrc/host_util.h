// Host-side helpers for the C-ABI edge: status-code translation and argument checks
// with the reference's error behaviour (src/sim_device.cc:44-102).
#pragma once

#include <cstdint>
#include <exception>
#include <new>
#include <string>

#include "common.h"

namespace accel_hip {

void SetLastError(const std::string& message);
void ClearLastError();

// Runs f; maps library errors and exceptions to status codes and the thread's message.
template <class F>
int Guard(F&& f) {
  try {
    f();
    ClearLastError();
    return ACCEL_HIP_OK;
  } catch (const Error& e) {
    SetLastError(e.message);
    return e.code;
  } catch (const std::bad_alloc&) {
    SetLastError("std::bad_alloc");
    return ACCEL_HIP_BAD_ALLOC;
  } catch (const std::exception& e) {
    SetLastError(e.what());
    return ACCEL_HIP_RUNTIME_ERROR;
  }
}

// CheckedBytes (src/sim_device.cc:44-52): rows*cols*4 with negative -> invalid, overflow -> overflow.
inline size_t CheckedBytes(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "negative matrix dimension");
  if (rows != 0 && static_cast<uint64_t>(cols) > (UINT64_MAX / sizeof(float)) / static_cast<uint64_t>(rows))
    Fail(ACCEL_HIP_OVERFLOW, "matrix is too large");
  return static_cast<size_t>(rows) * static_cast<size_t>(cols) * sizeof(float);
}

// CheckedSpan (src/sim_device.cc:54-62).
inline int64_t CheckedSpan(int64_t offset, int64_t count) {
  if (offset < 0 || count < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "negative matrix dimension");
  if (offset > INT64_MAX - count) Fail(ACCEL_HIP_OVERFLOW, "matrix is too large");
  return offset + count;
}

// CheckedFloats (src/sim_device.cc:64-83): depth*rows*cols*4.
inline size_t CheckedFloats(int64_t depth, int64_t rows, int64_t cols) {
  if (depth < 0 || rows < 0 || cols < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "negative matrix dimension");
  if (depth == 0 || rows == 0 || cols == 0) return 0;
  if (static_cast<uint64_t>(rows) > UINT64_MAX / static_cast<uint64_t>(depth))
    Fail(ACCEL_HIP_OVERFLOW, "matrix is too large");
  const uint64_t plane = static_cast<uint64_t>(depth) * static_cast<uint64_t>(rows);
  if (static_cast<uint64_t>(cols) > UINT64_MAX / plane) Fail(ACCEL_HIP_OVERFLOW, "matrix is too large");
  const uint64_t count = plane * static_cast<uint64_t>(cols);
  if (count > UINT64_MAX / sizeof(float)) Fail(ACCEL_HIP_OVERFLOW, "matrix is too large");
  return static_cast<size_t>(count * sizeof(float));
}

// CheckedIntBytes (src/sim_device.cc:85-93).
inline size_t CheckedIntBytes(int64_t count) {
  if (count < 0) Fail(ACCEL_HIP_INVALID_ARGUMENT, "negative matrix dimension");
  if (count != 0 && static_cast<uint64_t>(count) > UINT64_MAX / sizeof(int32_t))
    Fail(ACCEL_HIP_OVERFLOW, "matrix is too large");
  return static_cast<size_t>(count) * sizeof(int32_t);
}

// RequireBytes (src/sim_device.cc:95-102).
inline void RequireBytes(const AccelHipBuffer& buffer, size_t need, const char* what) {
  if (need == 0) return;
  if (buffer.data == nullptr || buffer.bytes < need) Fail(ACCEL_HIP_INVALID_ARGUMENT, what);
}

}  // namespace accel_hip
