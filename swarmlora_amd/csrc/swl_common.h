// Internal helpers shared by the libswl translation units: error state, HIP
// checks, bf16 vector types for gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

namespace swl {

// Thread-local error text behind swl_last_error().
void set_error(const std::string& msg);
const std::string& last_error();

// Returns SWL_ERR_* after recording `msg`.
int fail(int code, const std::string& msg);

// A HIP failure is reported with the reference's prefix ("CUDA error: <text>",
// src/cpp_extensions/common/ipc_types.h:223-229) so callers that match on it
// keep working.
int hip_fail(hipError_t e, const char* where);

}  // namespace swl

#define SWL_HIP(call)                                   \
  do {                                                  \
    hipError_t _e = (call);                             \
    if (_e != hipSuccess) return swl::hip_fail(_e, #call); \
  } while (0)

#define SWL_CHECK(cond, code, msg)                      \
  do {                                                  \
    if (!(cond)) return swl::fail((code), (msg));       \
  } while (0)

#define SWL_LAUNCH_CHECK(what)                          \
  do {                                                  \
    hipError_t _e = hipGetLastError();                  \
    if (_e != hipSuccess) return swl::hip_fail(_e, what); \
  } while (0)
