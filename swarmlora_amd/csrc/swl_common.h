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

// GPU-ordered rounds: per slot two 64-bit sequence words live in a tail
// past the slot's output buffer (both processes map that buffer).  The
// worker's stream writes in_seq after its input copy; the aggregator's stream
// waits for it, runs the round and writes out_seq; the worker's stream waits
// for out_seq before reading the outputs.
constexpr size_t kSeqTailBytes = 256;
constexpr size_t kInSeqOffset = 0, kOutSeqOffset = 128;

// Waits on `stream` until *flag[i] >= want[i] for every i < n (one lane per
// flag, polled with system-scope loads and a sleep).  A flag still short after
// limit_us microseconds stops the wait for that flag and stores 1 into
// timed_out[tag[i]] (host-visible, one word per tag); the stream continues.
int seq_wait_launch(int n, const uint64_t* const* flag, const uint64_t* want, const int32_t* tag, uint32_t* timed_out,
                    uint32_t limit_us, hipStream_t stream);

// Writes *flag[i] = value[i] for every i < n on `stream`, in one kernel
// launch, after the stream's earlier work (system-scope release stores, one
// lane per flag).  Stands in for n hipStreamWriteValue64 calls, each of which
// is a kernel launch of its own that costs the host ~10-30 us.
int seq_write_launch(int n, uint64_t* const* flag, const uint64_t* value, hipStream_t stream);

// Copies `bytes` from src to dst on `stream` and then writes *flag = value
// (system-scope release after every thread's stores are written back), in
// one kernel launch of one workgroup: the GPU-ordered input copy of a worker
// without a second dependent launch.  For copies up to kCopySignalMax bytes
// with 16-byte aligned pointers; otherwise hipMemcpyAsync + seq_write_launch.
constexpr size_t kCopySignalMax = 256 * 1024;
int copy_signal_launch(void* dst, const void* src, size_t bytes, uint64_t* flag, uint64_t value, hipStream_t stream);

// GPU-ordered slot words handled inside a worker read's own launch (null
// flags: none): before reading, every workgroup waits until *wait_flag >=
// want (as seq_wait_launch, with its time-out report into timed_out[tag]);
// after its stores, the launch writes *signal_flag = value (system-scope
// release after the stores are written back), which needs the launch to be
// one workgroup: reads of at most kFusedSignalRows rows.
struct SeqSync {
  const uint64_t* wait_flag = nullptr;
  uint64_t want = 0;
  uint32_t* timed_out = nullptr;
  int32_t tag = 0;
  uint32_t limit_us = 0;
  uint64_t* signal_flag = nullptr;
  uint64_t value = 0;
};
constexpr int64_t kFusedSignalRows = 8;

// dst[i] = bf16(res[i] + bf16(src[i] + delta[i])) for i < n bf16 elements
// (delta and res optional: the same bf16 roundings as the two separate adds
// out + delta and residual + that), one launch; sync: a wait only.
int combine_rows_launch(void* dst, const void* src, int64_t n, const void* delta, const void* res,
                        hipStream_t stream, const SeqSync* sync = nullptr);

// The same read followed by LlamaRMSNorm of every row (rows x d): dst_h =
// h, dst_n (and dst_n2 when not null) = bf16(bf16(h * rsqrt(mean(h^2) +
// eps)) * w), bit for bit the separate read and rmsnorm_rows_kernel.
// d % 8 == 0, 16-byte aligned.
int combine_norm_rows_launch(void* dst_h, void* dst_n, void* dst_n2, const void* src, int64_t rows, int64_t d,
                             const void* delta, const void* res, const void* w, float eps, hipStream_t stream,
                             const SeqSync* sync = nullptr);
// A Gate+Up read (rows of 2 inter, optional delta) followed by SiLU*up into
// rows of inter (dst, and dst2 when not null), bit for bit the separate read
// and silu_mul_rows_kernel.
int combine_silu_rows_launch(void* dst, void* dst2, const void* src, int64_t rows, int64_t inter, const void* delta,
                             hipStream_t stream, const SeqSync* sync = nullptr);

// The converse of copy_signal_launch: waits on `stream` until *flag >= want
// (as seq_wait_launch, with its time-out report into timed_out[tag]), then
// copies `bytes` from src to dst, in one launch of one workgroup for copies
// up to kCopySignalMax bytes with 16-byte aligned pointers; otherwise
// seq_wait_launch + hipMemcpyAsync.
int wait_copy_launch(const uint64_t* flag, uint64_t want, int32_t tag, uint32_t* timed_out, uint32_t limit_us,
                     void* dst, const void* src, size_t bytes, hipStream_t stream);

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
