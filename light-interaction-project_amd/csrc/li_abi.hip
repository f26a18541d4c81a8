// Version, status strings and the last launch error of the sparse-attention C ABI.
#include <stdio.h>

#include "li_common.hpp"

namespace {
thread_local char g_last_error[256] = "no launch error";
}

void li::record_launch_error(hipError_t e) {
  snprintf(g_last_error, sizeof(g_last_error), "%s: %s", hipGetErrorName(e), hipGetErrorString(e));
}

extern "C" const char* li_last_error(void) { return g_last_error; }

extern "C" int li_abi_version(void) { return 11; }

extern "C" const char* li_status_string(int status) {
  switch (status) {
    case LI_OK: return "ok";
    case LI_ERR_INVALID_ARG: return "invalid argument";
    case LI_ERR_SHAPE: return "inconsistent shape or geometry";
    case LI_ERR_K_LEN: return "K length not divisible by the logical block size";
    case LI_ERR_INDEX_RANGE: return "Sparse indices out of bounds.";
    case LI_ERR_UNSUPPORTED: return "unsupported head_dim, block size or dtype";
    case LI_ERR_LAUNCH: return "HIP kernel launch failed";
    case LI_ERR_TOO_LARGE: return "size above a built-in limit (mask builder key blocks, or the allocation-free entry point's scratch)";
    default: return "unknown status";
  }
}
