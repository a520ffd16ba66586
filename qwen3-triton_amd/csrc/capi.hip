// Library-wide C ABI helpers: error strings and ABI version.
#include "common.h"

extern "C" {

const char* q3_error_string(int code) {
  if (code == Q3_OK) return "success";
  if (code == Q3_ERR_SCRATCH)
    return "q3hip: the request needs more scratch than the no-allocation entry point's fixed array holds";
  if (code == Q3_ERR_INVALID) return "q3hip: invalid argument (shape, dtype, pointer or size not supported)";
  return hipGetErrorString((hipError_t)code);
}

int q3_abi_version(void) { return 5; }

}  // extern "C"
