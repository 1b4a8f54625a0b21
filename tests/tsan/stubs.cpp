// Stand-ins for the libswl symbols that the host protocol code references
// but the ThreadSanitizer harness never reaches: the error-state helpers
// (same behaviour as the library's) and the GPU launchers (abort if called).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>

#include "swl.h"

namespace swl {
thread_local std::string t_err;
void set_error(const std::string& msg) { t_err = msg; }
const std::string& last_error() { return t_err; }
int fail(int code, const std::string& msg) {
  t_err = msg;
  return code;
}
int hip_fail(hipError_t e, const char* where) {
  t_err = std::string("CUDA error ") + std::to_string((int)e) + " (" + where + ")";
  return SWL_ERR_HIP;
}

[[noreturn]] static void no_gpu(const char* what) {
  std::fprintf(stderr, "protocol_tsan: %s reached (no GPU work in this harness)\n", what);
  std::abort();
}
int embed_launch(int, const int64_t*, const void* const*, void* const*, const void*, int64_t, int64_t, hipStream_t) {
  no_gpu("embed_launch");
}
int lm_head_launch(int, const void* const*, const void*, int64_t, int64_t, void*, void*, int64_t*, void* const*,
                   const int32_t*, const float*, const int32_t*, const float*, uint64_t, hipStream_t) {
  no_gpu("lm_head_launch");
}
int round_launch(int, const int64_t*, const void* const*, void* const*, const void*, const void*, int64_t, int64_t,
                 const int32_t*, const swl_lora_entry*, const swl_lora_entry*, int, const int64_t*, hipStream_t,
                 const swl_round_fusion*) {
  no_gpu("round_launch");
}
int seq_wait_launch(int, const uint64_t* const*, const uint64_t*, const int32_t*, uint32_t*, uint32_t, hipStream_t) {
  no_gpu("seq_wait_launch");
}
int seq_write_launch(int, uint64_t* const*, const uint64_t*, hipStream_t) { no_gpu("seq_write_launch"); }
}  // namespace swl

extern "C" const char* swl_last_error(void) { return swl::last_error().c_str(); }
