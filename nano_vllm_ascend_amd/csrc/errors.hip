// The per-device index-error word: where the reference's indexing would raise, the kernels
// clamp or skip the access and OR a bit into this word (see nvamd.h, "Index errors").
//
// The word is a file-scope device variable, zero when the code object is loaded.  Every GPU the
// library runs on holds its own copy; host code never uses the variable's name as an address:
// index_error_word() looks the current device's copy up once (hipGetSymbolAddress) and keeps it
// per device, and the entry points pass that address to their kernels as an argument (the
// kernels live in other translation units, which cannot name this one's variables).
#include <atomic>
#include <mutex>

#include "common.h"

__device__ __align__(64) unsigned int nvamd_index_errors;

namespace nvamd {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_lock;
std::atomic<u32 *> g_word[kMaxDevices];

__global__ void clear_word_kernel(u32 *w) { *w = 0u; }

}  // namespace

u32 *index_error_word() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  u32 *w = g_word[dev].load(std::memory_order_acquire);
  if (w != nullptr) return w;
  std::lock_guard<std::mutex> guard(g_lock);
  w = g_word[dev].load(std::memory_order_relaxed);
  if (w == nullptr) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(nvamd_index_errors)) != hipSuccess) return nullptr;
    w = static_cast<u32 *>(p);
    g_word[dev].store(w, std::memory_order_release);
  }
  return w;
}

}  // namespace nvamd

using namespace nvamd;

extern "C" int nvamd_errors_fetch(unsigned *host, hipStream_t stream) {
  if (!host) return NVAMD_EINVAL;
  u32 *w = index_error_word();
  if (!w) return (int)hipErrorInvalidSymbol;
  return (int)hipMemcpyAsync(host, w, sizeof(u32), hipMemcpyDeviceToHost, stream);
}

extern "C" int nvamd_errors_clear(hipStream_t stream) {
  u32 *w = index_error_word();
  if (!w) return (int)hipErrorInvalidSymbol;
  hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(1), 0, stream, w);
  return launch_status();
}
