// Worker-side slot manager: maps the aggregator's slot buffers through HIP IPC
// handles and moves activations in and results out.  Semantics follow
// src/cpp_extensions/ext_unified_barrier.cpp.

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "swl_common.h"
#include "swl_runtime.h"

namespace {

constexpr int kMaxSlotsPerWorker = 8;

struct SlotCtx {
  int slot_id = -1;
  bool open = false;
  void* in = nullptr;
  void* out = nullptr;
  size_t in_size = 0, out_size = 0;
  int64_t bx = 0, tx = 0, dx = 0;
  uint64_t seq = 0;  // GPU-ordered mode: input sequence value of the last prepare_*
  // the next round's input already written into the input buffer by a fused
  // output read (swl_w_read_output_norm / _silu with stage_input), shape
  // [sbx, stx, sdx], waiting for swl_w_submit_staged_input
  bool staged = false;
  int64_t sbx = 0, stx = 0, sdx = 0;
  // GPU-ordered mode: the staging read also wrote the input sequence word
  // (value seq), so the staged submit launches nothing
  bool signaled = false;
};

// Limit of this worker's stream wait for a round's outputs (the aggregator's
// own input wait is 2 s; a round that long has already been evicted).
// SWL_OUT_WAIT_US overrides it (tests of the time-out path).
constexpr uint32_t kOutWaitLimitUs = 4000000;

uint32_t out_wait_limit_us() {
  static const uint32_t v = [] {
    const char* e = std::getenv("SWL_OUT_WAIT_US");
    const long long x = e ? std::atoll(e) : 0;
    return x > 0 && x < 0xFFFFFFFFll ? (uint32_t)x : kOutWaitLimitUs;
  }();
  return v;
}

struct Manager {
  int worker_id = -1;
  int worker_device = 0;
  int aggregator_device = 0;
  int hidden = 0, inter = 0, qkv = 0;
  SlotCtx slots[kMaxSlotsPerWorker];
  int nopen = 0;
  bool initialized = false;
  // GPU ordering: 0 none (host waits), 1 inputs and outputs, 2 inputs only
  // (outputs are read once the aggregator has signalled done, which it does
  // after its stream has finished the round)
  int gpu_ordered = 0;
  uint32_t* out_timeout = nullptr;  // host-visible words, one per slot id
} g_w;

uint64_t* seq_word(SlotCtx* c, size_t off) {
  return reinterpret_cast<uint64_t*>(static_cast<char*>(c->out) + c->out_size + off);
}

// GPU-ordered mode: the stream waits until the aggregator has written this
// slot's output sequence word for the last submitted input.
int wait_outputs(const char* fn, SlotCtx* c, hipStream_t st) {
  if (g_w.gpu_ordered != 1 || c->seq == 0) return SWL_OK;
  const uint64_t* flag = seq_word(c, swl::kOutSeqOffset);
  const int32_t tag = c->slot_id;
  int rc = swl::seq_wait_launch(1, &flag, &c->seq, &tag, g_w.out_timeout, out_wait_limit_us(), st);
  if (rc) return swl::fail(rc, std::string(fn) + ": " + swl::last_error());
  return SWL_OK;
}

// A GPU-ordered output wait that ran out of time sets the slot's word in
// out_timeout (the copy behind it then read a stale buffer).  The word is
// checked, and cleared, by every later call on the slot and right after the
// host synchronises in get_next_token_slot, so the worker learns of it before
// its next submit and treats the slot as evicted.
int check_out_timeout(const char* fn, const SlotCtx* c) {
  if (!g_w.out_timeout || c->slot_id < 0 || c->slot_id >= SWL_MAX_SLOTS) return SWL_OK;
  volatile uint32_t* word = g_w.out_timeout + c->slot_id;
  if (*word == 0) return SWL_OK;
  *word = 0;
  return swl::fail(SWL_ERR_TIMEOUT, std::string(fn) + ": slot " + std::to_string(c->slot_id) +
                                        " timed out waiting for the aggregator's output (slot evicted?)");
}

SlotCtx* find_slot(int slot_id) {
  for (auto& s : g_w.slots)
    if (s.open && s.slot_id == slot_id) return &s;
  return nullptr;
}

int need_slot(const char* fn, int slot_id, SlotCtx** out) {
  if (!g_w.initialized) return swl::fail(SWL_ERR_STATE, std::string(fn) + ": worker slot manager not initialized");
  *out = find_slot(slot_id);
  if (!*out) return swl::fail(SWL_ERR_NOT_FOUND, std::string(fn) + ": slot " + std::to_string(slot_id) + " not found");
  return SWL_OK;
}

// need_slot plus the time-out report, for the calls that move data (queries
// and close_slot do not fail on a pending time-out)
int need_data_slot(const char* fn, int slot_id, SlotCtx** out) {
  int rc = need_slot(fn, slot_id, out);
  return rc ? rc : check_out_timeout(fn, *out);
}

int copy_in(const char* fn, SlotCtx* c, const void* src, size_t bytes, hipStream_t st) {
  if (bytes > c->in_size)
    return swl::fail(SWL_ERR_INVALID, std::string(fn) + ": input tensor (" + std::to_string(bytes) +
                                          " bytes) exceeds slot buffer size (" + std::to_string(c->in_size) +
                                          " bytes)");
  if (g_w.gpu_ordered) {
    // the copy, then the value the aggregator's stream waits for before it
    // reads the buffer (one launch for small copies)
    ++c->seq;
    return swl::copy_signal_launch(c->in, src, bytes, seq_word(c, swl::kInSeqOffset), c->seq, st);
  }
  SWL_HIP(hipMemcpyAsync(c->in, src, bytes, hipMemcpyDeviceToDevice, st));
  // the aggregator reads the buffer from another process once this worker
  // signals ready: the copy must be complete, not just ordered
  SWL_HIP(hipStreamSynchronize(st));
  return SWL_OK;
}

// The GPU-ordered words a fused read handles in its own launch: the wait
// for the last round's output word (wait_outputs' condition), and, when it
// stages the next input of at most kFusedSignalRows rows, the signal of that
// input's word (value seq + 1, taken by commit_read_sync once the launch is
// queued).
swl::SeqSync read_sync(SlotCtx* c, bool staging, int64_t rows) {
  swl::SeqSync s;
  if (g_w.gpu_ordered == 1 && c->seq != 0) {
    s.wait_flag = seq_word(c, swl::kOutSeqOffset);
    s.want = c->seq;
    s.timed_out = g_w.out_timeout;
    s.tag = c->slot_id;
    s.limit_us = out_wait_limit_us();
  }
  if (staging && g_w.gpu_ordered && rows <= swl::kFusedSignalRows) {
    s.signal_flag = seq_word(c, swl::kInSeqOffset);
    s.value = c->seq + 1;
  }
  return s;
}

void commit_read_sync(SlotCtx* c, const swl::SeqSync& s) {
  if (!s.signal_flag) return;
  c->seq = s.value;
  c->signaled = true;
}

// Checks and records a fused read's staging of the next round's input
// ([bx, tx, d] bf16 rows into the slot's input buffer); null when not asked.
int stage_target(const char* fn, SlotCtx* c, int stage_input, int64_t bx, int64_t tx, int64_t d, void** dst) {
  *dst = nullptr;
  if (!stage_input) return SWL_OK;
  SWL_CHECK((size_t)(bx * tx * d) * sizeof(uint16_t) <= c->in_size, SWL_ERR_INVALID,
            std::string(fn) + ": staged input exceeds the slot input buffer");
  *dst = c->in;
  c->staged = true;
  c->signaled = false;
  c->sbx = bx;
  c->stx = tx;
  c->sdx = d;
  return SWL_OK;
}

}  // namespace

extern "C" {

int swl_w_init(int worker_id, int worker_device, int aggregator_device, int hidden_dim, int intermediate_dim,
               int qkv_dim) {
  SWL_HIP(hipSetDevice(worker_device));
  g_w.worker_id = worker_id;
  g_w.worker_device = worker_device;
  g_w.aggregator_device = aggregator_device;
  g_w.hidden = hidden_dim;
  g_w.inter = intermediate_dim;
  g_w.qkv = qkv_dim;
  for (auto& s : g_w.slots) s = SlotCtx();
  g_w.nopen = 0;
  g_w.gpu_ordered = 0;
  g_w.initialized = true;
  std::printf("[Worker-%d] Slot manager initialized (worker_device=%d, aggregator_device=%d)\n", worker_id,
              worker_device, aggregator_device);
  std::fflush(stdout);
  return SWL_OK;
}

int swl_w_open_slot(int slot_id, const uint8_t* input_handle, size_t input_handle_len, const uint8_t* output_handle,
                    size_t output_handle_len, size_t input_buffer_size, size_t output_buffer_size) {
  SWL_CHECK(g_w.initialized, SWL_ERR_STATE, "open_slot: worker slot manager not initialized");
  SWL_CHECK(g_w.nopen < kMaxSlotsPerWorker, SWL_ERR_FULL, "open_slot: max slots per worker exceeded");
  SWL_CHECK(input_handle_len == sizeof(hipIpcMemHandle_t) && output_handle_len == sizeof(hipIpcMemHandle_t),
            SWL_ERR_INVALID,
            "open_slot: invalid IPC handle size (got " + std::to_string(input_handle_len) + "/" +
                std::to_string(output_handle_len) + ", expected " + std::to_string(sizeof(hipIpcMemHandle_t)) + ")");
  SWL_CHECK(find_slot(slot_id) == nullptr, SWL_ERR_INVALID,
            "open_slot: slot " + std::to_string(slot_id) + " is already open");
  SWL_HIP(hipSetDevice(g_w.worker_device));
  SlotCtx* c = nullptr;
  for (auto& s : g_w.slots)
    if (!s.open) {
      c = &s;
      break;
    }
  SWL_CHECK(c != nullptr, SWL_ERR_FULL, "open_slot: no free slot context");
  hipIpcMemHandle_t hin, hout;
  std::memcpy(&hin, input_handle, sizeof(hin));
  std::memcpy(&hout, output_handle, sizeof(hout));
  void* pin = nullptr;
  void* pout = nullptr;
  hipError_t e = hipIpcOpenMemHandle(&pin, hin, hipIpcMemLazyEnablePeerAccess);
  if (e != hipSuccess)
    return swl::fail(SWL_ERR_HIP, std::string("open_slot: input IPC open failed: ") + hipGetErrorString(e));
  e = hipIpcOpenMemHandle(&pout, hout, hipIpcMemLazyEnablePeerAccess);
  if (e != hipSuccess) {
    (void)hipIpcCloseMemHandle(pin);
    return swl::fail(SWL_ERR_HIP, std::string("open_slot: output IPC open failed: ") + hipGetErrorString(e));
  }
  *c = SlotCtx();
  c->slot_id = slot_id;
  c->open = true;
  c->in = pin;
  c->out = pout;
  c->in_size = input_buffer_size;
  c->out_size = output_buffer_size;
  ++g_w.nopen;
  std::printf("[Worker-%d] Opened slot %d (input=%zu bytes, output=%zu bytes)\n", g_w.worker_id, slot_id,
              input_buffer_size, output_buffer_size);
  std::fflush(stdout);
  return SWL_OK;
}

int swl_w_close_slot(int slot_id) {
  SlotCtx* c;
  int rc = need_slot("close_slot", slot_id, &c);
  if (rc) return rc;
  // every stream of this process may still touch the mapping (a pending
  // GPU-ordered output wait ends by its own limit); a time-out not yet
  // reported is dropped with the slot
  SWL_HIP(hipDeviceSynchronize());
  if (g_w.out_timeout && slot_id >= 0 && slot_id < SWL_MAX_SLOTS)
    reinterpret_cast<volatile uint32_t*>(g_w.out_timeout)[slot_id] = 0;
  if (c->in) {
    const hipError_t e = hipIpcCloseMemHandle(c->in);
    if (e != hipSuccess)
      std::fprintf(stderr, "[Worker-%d] Warning: hipIpcCloseMemHandle(input) for slot %d: %s\n", g_w.worker_id,
                   slot_id, hipGetErrorString(e));
  }
  if (c->out) {
    const hipError_t e = hipIpcCloseMemHandle(c->out);
    if (e != hipSuccess)
      std::fprintf(stderr, "[Worker-%d] Warning: hipIpcCloseMemHandle(output) for slot %d: %s\n", g_w.worker_id,
                   slot_id, hipGetErrorString(e));
  }
  *c = SlotCtx();
  --g_w.nopen;
  std::printf("[Worker-%d] Closed slot %d\n", g_w.worker_id, slot_id);
  std::fflush(stdout);
  return SWL_OK;
}

int swl_w_prepare_input(int slot_id, const void* src, int64_t bx, int64_t tx, int64_t dx, size_t elem_size,
                        void* stream) {
  SlotCtx* c;
  int rc = need_data_slot("prepare_input_slot", slot_id, &c);
  if (rc) return rc;
  SWL_CHECK(src && bx > 0 && tx > 0 && dx > 0 && elem_size > 0, SWL_ERR_INVALID, "Input must be 3D [B, T, D]");
  c->staged = false;
  c->signaled = false;
  rc = copy_in("prepare_input_slot", c, src, (size_t)bx * tx * dx * elem_size, (hipStream_t)stream);
  if (rc) return rc;
  c->bx = bx;
  c->tx = tx;
  c->dx = dx;
  return SWL_OK;
}

int swl_w_slot_shape(int slot_id, int64_t* bx, int64_t* tx, int64_t* dx) {
  SlotCtx* c;
  int rc = need_slot("slot_shape", slot_id, &c);
  if (rc) return rc;
  *bx = c->bx;
  *tx = c->tx;
  *dx = c->dx;
  return SWL_OK;
}

int swl_w_slot_sizes(int slot_id, size_t* input_buffer_size, size_t* output_buffer_size) {
  SlotCtx* c;
  int rc = need_slot("slot_sizes", slot_id, &c);
  if (rc) return rc;
  *input_buffer_size = c->in_size;
  *output_buffer_size = c->out_size;
  return SWL_OK;
}

int swl_w_stage_input(int slot_id, int64_t bx, int64_t tx, int64_t dx, void** input_buffer) {
  SlotCtx* c;
  int rc = need_data_slot("prepare_input_slot", slot_id, &c);
  if (rc) return rc;
  SWL_CHECK(input_buffer != nullptr && bx > 0 && tx > 0 && dx > 0, SWL_ERR_INVALID, "stage_input: bad arguments");
  void* dst = nullptr;
  rc = stage_target("prepare_input_slot", c, 1, bx, tx, dx, &dst);
  if (rc) return rc;
  *input_buffer = dst;
  return SWL_OK;
}

int swl_w_copy_output(int slot_id, void* dst, size_t bytes, void* stream) {
  SlotCtx* c;
  int rc = need_data_slot("get_outputs_slot", slot_id, &c);
  if (rc) return rc;
  SWL_CHECK(dst != nullptr, SWL_ERR_INVALID, "get_outputs_slot: null destination");
  SWL_CHECK(bytes <= c->out_size, SWL_ERR_INVALID,
            "get_outputs_slot: output (" + std::to_string(bytes) + " bytes) exceeds slot output buffer (" +
                std::to_string(c->out_size) + " bytes)");
  if (g_w.gpu_ordered == 1 && c->seq > 0) {
    // the wait for the aggregator's output word and the copy, in one launch
    // for small outputs
    rc = swl::wait_copy_launch(seq_word(c, swl::kOutSeqOffset), c->seq, c->slot_id, g_w.out_timeout,
                               out_wait_limit_us(), dst, c->out, bytes, (hipStream_t)stream);
    if (rc) return swl::fail(rc, std::string("get_outputs_slot: ") + swl::last_error());
    return SWL_OK;
  }
  // stream-ordered; consumers of dst on the same stream see the copy
  SWL_HIP(hipMemcpyAsync(dst, c->out, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
  return SWL_OK;
}

int swl_w_read_output(int slot_id, void* dst, int64_t n, const void* delta, const void* residual, void* stream) {
  SlotCtx* c;
  int rc = need_data_slot("get_outputs_slot", slot_id, &c);
  if (rc) return rc;
  SWL_CHECK(dst != nullptr && n >= 0, SWL_ERR_INVALID, "get_outputs_slot: bad destination");
  SWL_CHECK((size_t)n * sizeof(uint16_t) <= c->out_size, SWL_ERR_INVALID,
            "get_outputs_slot: output (" + std::to_string(n * 2) + " bytes) exceeds slot output buffer (" +
                std::to_string(c->out_size) + " bytes)");
  const swl::SeqSync sync = read_sync(c, false, 0);  // the output wait inside the read's launch
  rc = swl::combine_rows_launch(dst, c->out, n, delta, residual, (hipStream_t)stream, &sync);
  if (rc) return swl::fail(rc, std::string("get_outputs_slot: ") + swl::last_error());
  return SWL_OK;
}

int swl_w_read_output_norm(int slot_id, void* dst_h, void* dst_norm, int64_t bx, int64_t tx, int64_t d,
                           const void* delta, const void* residual, const void* weight, float eps, int stage_input,
                           void* stream) {
  SlotCtx* c;
  int rc = need_data_slot("get_outputs_slot", slot_id, &c);
  if (rc) return rc;
  SWL_CHECK(bx > 0 && tx > 0 && d > 0 && (size_t)(bx * tx * d) * sizeof(uint16_t) <= c->out_size, SWL_ERR_INVALID,
            "get_outputs_slot: output rows exceed the slot output buffer");
  void* staged = nullptr;
  rc = stage_target("get_outputs_slot", c, stage_input, bx, tx, d, &staged);
  if (rc) return rc;
  const swl::SeqSync sync = read_sync(c, staged != nullptr, bx * tx);
  rc = swl::combine_norm_rows_launch(dst_h, dst_norm, staged, c->out, bx * tx, d, delta, residual, weight, eps,
                                     (hipStream_t)stream, &sync);
  if (rc) {
    c->staged = false;
    return swl::fail(rc, std::string("get_outputs_slot: ") + swl::last_error());
  }
  commit_read_sync(c, sync);
  return SWL_OK;
}

int swl_w_read_output_silu(int slot_id, void* dst, int64_t bx, int64_t tx, int64_t inter, const void* delta,
                           int stage_input, void* stream) {
  SlotCtx* c;
  int rc = need_data_slot("get_outputs_slot", slot_id, &c);
  if (rc) return rc;
  SWL_CHECK(bx > 0 && tx > 0 && inter > 0 && (size_t)(bx * tx * 2 * inter) * sizeof(uint16_t) <= c->out_size,
            SWL_ERR_INVALID, "get_outputs_slot: output rows exceed the slot output buffer");
  void* staged = nullptr;
  rc = stage_target("get_outputs_slot", c, stage_input, bx, tx, inter, &staged);
  if (rc) return rc;
  const swl::SeqSync sync = read_sync(c, staged != nullptr, bx * tx);
  rc = swl::combine_silu_rows_launch(dst, staged, c->out, bx * tx, inter, delta, (hipStream_t)stream, &sync);
  if (rc) {
    c->staged = false;
    return swl::fail(rc, std::string("get_outputs_slot: ") + swl::last_error());
  }
  commit_read_sync(c, sync);
  return SWL_OK;
}

int swl_w_submit_staged_input(int slot_id, int64_t bx, int64_t tx, int64_t dx, void* stream) {
  SlotCtx* c;
  int rc = need_data_slot("prepare_input_slot", slot_id, &c);
  if (rc) return rc;
  SWL_CHECK(c->staged, SWL_ERR_STATE, "prepare_input_slot: no staged input on slot " + std::to_string(slot_id));
  SWL_CHECK(bx == c->sbx && tx == c->stx && dx == c->sdx, SWL_ERR_INVALID,
            "prepare_input_slot: input shape differs from the staged rows");
  c->staged = false;
  c->bx = bx;
  c->tx = tx;
  c->dx = dx;
  hipStream_t st = (hipStream_t)stream;
  if (g_w.gpu_ordered && c->signaled) {
    c->signaled = false;  // the staging read wrote the word (value seq)
    return SWL_OK;
  }
  if (g_w.gpu_ordered) {
    // the value the aggregator's stream waits for, after the staging read
    ++c->seq;
    uint64_t* flag = seq_word(c, swl::kInSeqOffset);
    return swl::seq_write_launch(1, &flag, &c->seq, st);
  }
  // as copy_in: the rows must be complete before this worker signals ready
  SWL_HIP(hipStreamSynchronize(st));
  return SWL_OK;
}

int swl_w_prepare_token_ids(int slot_id, const void* src, int64_t bx, int64_t tx, void* stream) {
  SlotCtx* c;
  int rc = need_data_slot("prepare_token_ids_slot", slot_id, &c);
  if (rc) return rc;
  SWL_CHECK(src && bx > 0 && tx > 0, SWL_ERR_INVALID, "token_ids must be 2D [B, T]");
  rc = copy_in("prepare_token_ids_slot", c, src, (size_t)bx * tx * sizeof(int64_t), (hipStream_t)stream);
  if (rc) return rc;
  c->bx = bx;
  c->tx = tx;
  c->dx = g_w.hidden;
  return SWL_OK;
}

int swl_w_prepare_hidden_lm(int slot_id, const void* src, int64_t bx, int64_t tx, int64_t dx, size_t elem_size,
                            void* stream) {
  SlotCtx* c;
  int rc = need_data_slot("prepare_hidden_for_lm_head_slot", slot_id, &c);
  if (rc) return rc;
  SWL_CHECK(src && bx > 0 && tx > 0 && dx > 0, SWL_ERR_INVALID, "hidden_states must be 3D [B, T, D]");
  rc = copy_in("prepare_hidden_for_lm_head_slot", c, src, (size_t)bx * tx * dx * elem_size, (hipStream_t)stream);
  if (rc) return rc;
  c->bx = bx;
  c->tx = tx;
  c->dx = dx;
  return SWL_OK;
}

int swl_w_get_next_token(int slot_id, int64_t* token, void* stream) {
  SlotCtx* c;
  int rc = need_data_slot("get_next_token_slot", slot_id, &c);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  rc = wait_outputs("get_next_token_slot", c, st);
  if (rc) return rc;
  SWL_HIP(hipStreamSynchronize(st));
  rc = check_out_timeout("get_next_token_slot", c);
  if (rc) return rc;
  SWL_HIP(hipMemcpyAsync(token, c->out, sizeof(int64_t), hipMemcpyDeviceToHost, st));
  SWL_HIP(hipStreamSynchronize(st));
  return SWL_OK;
}

int swl_w_set_gpu_ordered(int enable) {
  SWL_CHECK(g_w.initialized, SWL_ERR_STATE, "set_gpu_ordered: worker slot manager not initialized");
  SWL_CHECK(enable >= 0 && enable <= 2, SWL_ERR_INVALID, "set_gpu_ordered: mode must be 0, 1 or 2");
  if (enable && !g_w.out_timeout) {
    SWL_HIP(hipHostMalloc((void**)&g_w.out_timeout, SWL_MAX_SLOTS * sizeof(uint32_t), hipHostMallocDefault));
    std::memset(g_w.out_timeout, 0, SWL_MAX_SLOTS * sizeof(uint32_t));
  }
  g_w.gpu_ordered = enable;
  return SWL_OK;
}

int swl_w_input_seq(int slot_id, uint64_t* seq) {
  SlotCtx* c;
  int rc = need_slot("input_seq", slot_id, &c);
  if (rc) return rc;
  *seq = c->seq;
  return SWL_OK;
}

int swl_w_cleanup(void) {
  if (!g_w.initialized) return SWL_OK;
  (void)hipSetDevice(g_w.worker_device);
  (void)hipDeviceSynchronize();
  for (auto& s : g_w.slots) {
    if (!s.open) continue;
    if (s.in) (void)hipIpcCloseMemHandle(s.in);
    if (s.out) (void)hipIpcCloseMemHandle(s.out);
    s = SlotCtx();
  }
  g_w.nopen = 0;
  g_w.initialized = false;
  g_w.gpu_ordered = 0;
  if (g_w.out_timeout) (void)hipHostFree(g_w.out_timeout);
  g_w.out_timeout = nullptr;
  return SWL_OK;
}

}  // extern "C"
