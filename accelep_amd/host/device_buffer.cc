// OwnedBuffer and ActivationName (AccelEP src/device_buffer.cc:5-12, include/accel/device.h:12-24).
#include "accel/device.h"

namespace accel {

const char* ActivationName(Activation activation) {
  switch (activation) {
    case Activation::Relu:
      return "relu";
    case Activation::Gelu:
      return "gelu";
    case Activation::None:
      break;
  }
  return "none";
}

void OwnedBuffer::Reset() noexcept {
  if (device != nullptr && buffer.data != nullptr) {
    try {
      device->Free(buffer);
    } catch (...) {
      // A destructor must not throw; the allocation then stays counted as live.
    }
  }
  device = nullptr;
  buffer = DeviceBuffer{};
  shape.clear();
}

}  // namespace accel
