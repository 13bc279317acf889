// ABI version, status strings and the per-thread record of the last HIP error.
#include "common.hpp"

namespace {
thread_local char g_last_hip_error[256] = "no HIP error recorded";
}

namespace tks {
void set_hip_error(hipError_t err) {
  const char *name = hipGetErrorName(err);
  const char *text = hipGetErrorString(err);
  __builtin_snprintf(g_last_hip_error, sizeof(g_last_hip_error), "%s: %s", name ? name : "?",
                     text ? text : "?");
}
}  // namespace tks

extern "C" int32_t tks_abi_version(void) { return 12; }

extern "C" const char *tks_status_string(int32_t status) {
  switch (status) {
    case TKS_OK:
      return "ok";
    case TKS_ERR_VALUE:
      return "invalid shape, size or range";
    case TKS_ERR_TYPE:
      return "unsupported dtype";
    case TKS_ERR_INDEX:
      return "layer_index is out of range";
    case TKS_ERR_WORKSPACE:
      return "workspace is missing or too small";
    case TKS_ERR_LAUNCH:
      return "HIP kernel launch failed";
    default:
      return "unknown status";
  }
}

extern "C" const char *tks_last_hip_error(void) { return g_last_hip_error; }
