// Version and error-string entry points of libi4moe.
#include "i4moe.h"

extern "C" {

int i4_abi_version(void) { return I4_ABI_VERSION; }

const char* i4_strerror(int code) {
  switch (code) {
    case I4_OK: return "ok";
    case I4_ERR_NULL: return "i4: a required pointer is NULL";
    case I4_ERR_SHAPE: return "i4: dimension out of range or inconsistent";
    case I4_ERR_DTYPE: return "i4: unsupported element type";
    case I4_ERR_ALIGN: return "i4: pointer not 16-byte aligned";
    case I4_ERR_LAYOUT: return "i4: unsupported packed layout for this entry point";
    case I4_ERR_GROUP: return "i4: group size must be a positive multiple of 32";
    case I4_ERR_WORKSPACE: return "i4: workspace missing or too small";
    case I4_ERR_LAUNCH: return "i4: the HIP runtime rejected a kernel launch";
    case I4_ERR_STRIDE: return "i4: expert or row stride smaller than the data it spans";
    case I4_ERR_HANDOFF:
      return "i4: a decode workgroup gave up waiting for its launch's activations (NaN rows)";
    case I4_ERR_SCRATCH:
      return "i4: the call needs more scratch than the library's static buffer holds";
    default: return "i4: unknown error code";
  }
}

}  // extern "C"
