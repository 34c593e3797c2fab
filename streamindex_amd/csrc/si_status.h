// Status codes and the thread-local error text shared by every C-ABI entry.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "streamindex.h"  // public C ABI: status codes and entry points

namespace si {

// Records `msg` as this thread's last error and returns `code`.
int set_error(int code, const std::string& msg);

// Converts a pending HIP launch error into SI_ERR_LAUNCH.
inline int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SI_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return SI_OK;
}

}  // namespace si
