// Library-wide entry points: status messages and version.
#include "common.hpp"

extern "C" {

const char* nt_strerror(int code) {
  switch (code) {
    case NT_OK: return "success";
    case NT_ERR_INVALID_ARG: return "invalid argument (null pointer or negative size)";
    case NT_ERR_DTYPE: return "unsupported dtype code";
    case NT_ERR_TOO_MANY_EXPERTS: return "number of experts exceeds NT_MAX_EXPERTS (1024)";
    case NT_ERR_WORKSPACE: return "workspace missing or too small";
    case NT_ERR_LAUNCH: return "HIP kernel launch failed";
    case NT_ERR_TOO_LARGE: return "size exceeds the 32-bit row/index range of the kernels";
    case NT_ERR_SCRATCH:
      return "sizes need more workspace than the no-allocation scratch (NT_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown status code";
  }
}

int nt_version(void) { return 100; }  // 0.1.0

}  // extern "C"
