// Library-level entry points: version and error strings.
#include <hip/hip_runtime.h>

#include "ppo_amd.h"

extern "C" int ppo_amd_version(void) { return 100; }  // 0.1.0

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
    default:
      break;
  }
  if (code >= PPO_ERR_HIP_BASE) return hipGetErrorString((hipError_t)(code - PPO_ERR_HIP_BASE));
  return "unknown error";
}
