// Status strings and version of the C-ABI (the compute entry points live
// beside their kernels).  Host-only translation unit.
#include "mx_kernels.h"

extern "C" const char* mx_strerror(int code) {
  switch (code) {
    case MX_OK: return "ok";
    case MX_ERR_NULL: return "null pointer argument";
    case MX_ERR_SHAPE: return "invalid or unsupported shape";
    case MX_ERR_ALIGN: return "pointer or leading dimension not 16-byte aligned";
    case MX_ERR_DTYPE: return "unsupported dtype code";
    case MX_ERR_WORKSPACE: return "workspace missing or too small";
    case MX_ERR_ALIAS: return "output overlaps an input";
    case MX_ERR_LAUNCH: return "HIP kernel launch failed";
    case MX_ERR_UNSUPPORTED: return "no kernel for this configuration";
    default: return "unknown status code";
  }
}

extern "C" const char* mx_version(void) { return "mxkernels 0.1.0 gfx950"; }
