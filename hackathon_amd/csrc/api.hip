// Library identification and status text for the C-ABI.
#include "ql_common.h"

extern "C" int qlora_abi_version(void) { return 3; }

extern "C" const char* qlora_strerror(int status) {
  switch (status) {
    case QL_OK: return "ok";
    case QL_EINVAL: return "invalid argument (null pointer, size or flag)";
    case QL_EDTYPE: return "unsupported dtype or dtype combination";
    case QL_EALIGN: return "pointer or stride alignment not met";
    case QL_ESHAPE: return "inconsistent sizes";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}
