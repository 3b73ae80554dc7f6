// Library-level entry points: version, error strings, and the status of the
// bounded in-kernel waits.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "grid_sync.hpp"
#include "ppo_amd.h"

namespace ppo {

// Wait-status words, one copy per device: [0] is raised (atomic OR) by any
// workgroup whose bounded wait gave up; [1] receives [0]'s value when
// ppo_wait_status takes it.  Zero at load, held until the process ends.
__device__ __align__(256) unsigned wait_words[2];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
unsigned* g_words[kMaxDevices];     // device address of wait_words, per device
std::atomic<long> g_spin{kSlotSpin};  // poll limit of every bounded wait

// Device address of wait_words on the current device, looked up once per
// device with that device current (in host code the name is only a handle).
int words_address(unsigned** out) {
  int dev = 0;
  int st = hip_status(hipGetDevice(&dev));
  if (st) return st;
  if (dev < 0 || dev >= kMaxDevices) return PPO_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_words[dev]) {
    void* p = nullptr;
    if ((st = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(wait_words))))) return st;
    if (!p) return PPO_ERR_HIP_BASE + (int)hipErrorInvalidSymbol;
    g_words[dev] = static_cast<unsigned*>(p);
  }
  *out = g_words[dev];
  return PPO_OK;
}

// Moves the status word into its read-back word and clears it, atomically,
// so that a give-up raised concurrently is reported by this take or the next.
__global__ void wait_take_kernel(unsigned* words) {
  words[1] = __hip_atomic_exchange(words, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

int wait_ctl(WaitCtl& w) {
  w.spin = g_spin.load(std::memory_order_relaxed);
  return words_address(&w.status);
}

}  // namespace ppo

extern "C" int ppo_amd_version(void) { return 200; }  // 0.2.0

extern "C" const char* ppo_amd_strerror(int code) {
  switch (code) {
    case PPO_OK:
      return "ok";
    case PPO_ERR_INVALID_ARG:
      return "invalid argument (null pointer, negative size or bad parameter)";
    case PPO_ERR_WORKSPACE:
      return "workspace missing or smaller than the *_workspace_bytes() query";
    case PPO_ERR_TOO_LARGE:
      return "problem size beyond what the kernels index";
    case PPO_ERR_UNSUPPORTED:
      return "shape or option outside what the kernels implement";
    case PPO_ERR_WAIT_TIMEOUT:
      return "a workgroup's bounded wait for another workgroup gave up (grid not co-resident?); "
             "the outputs of the calls since the last status check are not valid";
    default:
      break;
  }
  if (code >= PPO_ERR_HIP_BASE) return hipGetErrorString((hipError_t)(code - PPO_ERR_HIP_BASE));
  return "unknown error";
}

extern "C" int ppo_wait_status(void* stream_ptr) {
  using namespace ppo;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  unsigned* words = nullptr;
  int st = words_address(&words);
  if (st) return st;
  hipLaunchKernelGGL(wait_take_kernel, dim3(1), dim3(1), 0, stream, words);
  if ((st = last_launch_status())) return st;
  unsigned host = 0;
  if ((st = hip_status(hipMemcpyAsync(&host, words + 1, sizeof(host), hipMemcpyDeviceToHost,
                                      stream))))
    return st;
  if ((st = hip_status(hipStreamSynchronize(stream)))) return st;
  if (!host) return PPO_OK;
  if ((st = scratch_clear(stream))) return st;
  if ((st = hip_status(hipStreamSynchronize(stream)))) return st;
  return PPO_ERR_WAIT_TIMEOUT;
}

extern "C" int ppo_wait_status_async(uint32_t* host_word, void* stream_ptr) {
  using namespace ppo;
  if (!host_word) return PPO_ERR_INVALID_ARG;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  unsigned* words = nullptr;
  int st = words_address(&words);
  if (st) return st;
  hipLaunchKernelGGL(wait_take_kernel, dim3(1), dim3(1), 0, stream, words);
  if ((st = last_launch_status())) return st;
  return hip_status(hipMemcpyAsync(host_word, words + 1, sizeof(unsigned), hipMemcpyDeviceToHost,
                                   stream));
}

extern "C" int ppo_wait_reset(void* stream_ptr) {
  using namespace ppo;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  int st = scratch_clear(stream);
  if (st) return st;
  return hip_status(hipStreamSynchronize(stream));
}

extern "C" int ppo_set_wait_limit(int64_t polls) {
  ppo::g_spin.store(polls < 0 ? ppo::kSlotSpin : (long)polls, std::memory_order_relaxed);
  return PPO_OK;
}
