// C entry points over accel_hip::ByteBpe (accelep_amd/csrc/tokenizer.cc) for the CPU tests:
// the same tokenizer accel_llama_tokenizer / encode / decode run, without a model or a GPU.
// TEST INFRASTRUCTURE ONLY. Each call returns 0, or 1 with the message in bpe_host_error().
#include <cstdint>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>
#include <vector>

#include "tokenizer.h"

#define BPE_HOST_API extern "C" __attribute__((visibility("default")))

namespace {
thread_local std::string g_error;

template <typename F>
int Guard(F f) {
  try {
    f();
    g_error.clear();
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return 1;
  }
}
}  // namespace

BPE_HOST_API void* bpe_host_create() { return new accel_hip::ByteBpe(); }
BPE_HOST_API void bpe_host_destroy(void* h) { delete static_cast<accel_hip::ByteBpe*>(h); }
BPE_HOST_API const char* bpe_host_error() { return g_error.c_str(); }
BPE_HOST_API int32_t bpe_host_vocab_size(void* h) { return static_cast<accel_hip::ByteBpe*>(h)->vocab_size(); }

BPE_HOST_API int bpe_host_load(void* h, const char* path) {
  return Guard([&] { static_cast<accel_hip::ByteBpe*>(h)->Load(path); });
}

BPE_HOST_API int bpe_host_encode(void* h, const char* text, int32_t len, int32_t* out, int32_t cap, int32_t* count) {
  return Guard([&] {
    const std::vector<int32_t> ids = static_cast<accel_hip::ByteBpe*>(h)->Encode(std::string_view(text, len));
    if (static_cast<int64_t>(ids.size()) > cap) throw std::invalid_argument("encode buffer is too small");
    if (!ids.empty()) std::memcpy(out, ids.data(), ids.size() * sizeof(int32_t));
    *count = static_cast<int32_t>(ids.size());
  });
}

BPE_HOST_API int bpe_host_decode(void* h, const int32_t* ids, int32_t count, int32_t skip_special, char* out,
                                 int32_t cap, int32_t* len) {
  return Guard([&] {
    const std::string text = static_cast<accel_hip::ByteBpe*>(h)->Decode(ids, count, skip_special != 0);
    if (static_cast<int64_t>(text.size()) > cap) throw std::invalid_argument("decode buffer is too small");
    if (!text.empty()) std::memcpy(out, text.data(), text.size());
    *len = static_cast<int32_t>(text.size());
  });
}
