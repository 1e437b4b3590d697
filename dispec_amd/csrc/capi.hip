// Status strings and version of the C ABI declared in include/dispec_hip.h.
#include "dsp_common.h"

extern "C" const char* dsp_error_string(int status) {
  switch (status) {
    case DSP_OK: return "ok";
    case DSP_EINVAL: return "invalid argument (null pointer, negative size or inconsistent shape)";
    case DSP_EALIGN: return "misaligned pointer or stride for the vectorised kernel";
    case DSP_EUNSUPPORTED: return "dtype, head_dim or query-group size has no compiled kernel";
    case DSP_EWORKSPACE: return "workspace smaller than the size the launch needs";
    case DSP_ESCRATCH:
      return "the launch needs more split-K workspace than the no-allocation entry point's "
             "fixed scratch (DSP_NOALLOC_SCRATCH_BYTES)";
    default:
      if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
      return "unknown dispec_hip status";
  }
}

extern "C" int dsp_version(void) { return 1; }
