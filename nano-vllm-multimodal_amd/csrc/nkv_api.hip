// Error state and version of the nanokv C ABI.
#include <cstdarg>
#include <cstdio>
#include <string>

#include "nkv_common.h"

namespace {
thread_local std::string g_last_error;
}

int nkv_fail(int code, const char* fmt, ...) {
  char buffer[512];
  va_list args;
  va_start(args, fmt);
  std::vsnprintf(buffer, sizeof(buffer), fmt, args);
  va_end(args);
  g_last_error = buffer;
  return code;
}

// Reports a launch failure of the kernel just enqueued (invalid
// configuration, missing code object for this GPU, ...).
int nkv_check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return nkv_fail(NKV_E_HIP, "%s: kernel launch failed: %s (%d)", what,
                    hipGetErrorString(err), static_cast<int>(err));
  }
  return NKV_OK;
}

extern "C" int nkv_version(void) { return 100; }

// Fingerprint of the sources, headers, compiler flags and target this
// library was compiled from, passed in by the build recipe
// (nanokv/build.py); the loader recomputes it from the sources on disk and
// refuses a library built from other ones.
#ifndef NKV_BUILD_ID
#define NKV_BUILD_ID "unfingerprinted"
#endif
extern "C" const char* nkv_build_id(void) { return NKV_BUILD_ID; }

extern "C" const char* nkv_last_error(void) { return g_last_error.c_str(); }

namespace nkv {

int element_bytes(int32_t dtype) {
  switch (dtype) {
    case NKV_DTYPE_FLOAT16:
    case NKV_DTYPE_BFLOAT16:
      return 2;
    case NKV_DTYPE_FLOAT32:
      return 4;
    default:
      return 0;
  }
}

}  // namespace nkv
