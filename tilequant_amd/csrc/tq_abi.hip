// tq_abi.hip -- ABI version and error strings of libtilequant_hip.so.
#include "tq_common.h"

extern "C" int tq_abi_version(void) { return 3; }

extern "C" const char* tq_error_string(int code) {
  switch (code) {
    case TQ_OK: return "ok";
    case TQ_ERR_ARG: return "invalid argument (size, stride, null pointer or inconsistent shape)";
    case TQ_ERR_DTYPE: return "unsupported dtype or tile layout code";
    case TQ_ERR_ALIGN: return "tile pointer is not 16-byte aligned";
    case TQ_ERR_WORKSPACE: return "workspace missing or too small";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown tilequant error";
}
