// Library-level C-ABI entry points: version and error text.
#include <hip/hip_runtime.h>

#include "../../include/qwen3mi.h"

extern "C" int qmi_version(void) { return 100; }  // 0.1.0

extern "C" const char* qmi_error_string(int code) {
  switch (code) {
    case QMI_OK:
      return "success";
    case QMI_E_NULL_POINTER:
      return "qwen3mi: a required pointer argument is NULL";
    case QMI_E_BAD_SHAPE:
      return "qwen3mi: invalid size argument";
    case QMI_E_BAD_STRIDE:
      return "qwen3mi: unsupported stride or misaligned pointer";
    case QMI_E_UNSUPPORTED:
      return "qwen3mi: unsupported configuration (head_dim, block size, GQA ratio or size limit)";
    case QMI_E_WORKSPACE_TOO_SMALL:
      return "qwen3mi: workspace missing or smaller than required";
    case QMI_E_SCRATCH_LIMIT:
      return "qwen3mi: problem needs more workspace than the library's static device scratch "
             "holds (use the entry point that takes a workspace)";
    default:
      break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "qwen3mi: unknown error code";
}
