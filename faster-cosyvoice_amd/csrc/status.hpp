// Error reporting shared by the C ABI translation units: a failed call stores its message in a
// thread-local string (read back by fcv_last_error) and returns its status code.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace fcv {

int fail(int code, const std::string& msg);

}  // namespace fcv

#define FCV_HIP(expr)                                                                        \
  do {                                                                                       \
    hipError_t e_ = (expr);                                                                  \
    if (e_ != hipSuccess)                                                                    \
      return ::fcv::fail(FCV_ERR_RUNTIME, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

#define FCV_CHECK(cond, code, msg)                \
  do {                                            \
    if (!(cond)) return ::fcv::fail(code, msg);   \
  } while (0)
