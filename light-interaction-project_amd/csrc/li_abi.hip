// Version and status strings of the sparse-attention C ABI.
#include "li_common.hpp"

extern "C" int li_abi_version(void) { return 1; }

extern "C" const char* li_status_string(int status) {
  switch (status) {
    case LI_OK: return "ok";
    case LI_ERR_INVALID_ARG: return "invalid argument";
    case LI_ERR_SHAPE: return "inconsistent shape or geometry";
    case LI_ERR_K_LEN: return "K length not divisible by the logical block size";
    case LI_ERR_INDEX_RANGE: return "Sparse indices out of bounds.";
    case LI_ERR_UNSUPPORTED: return "unsupported head_dim, block size or dtype";
    case LI_ERR_LAUNCH: return "HIP kernel launch failed";
    case LI_ERR_TOO_LARGE: return "too many key blocks for the mask builder";
    default: return "unknown status";
  }
}
