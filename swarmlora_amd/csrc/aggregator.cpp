// Aggregator runtime: slot pool, fused weights, adapter pool, batched rounds
// and the barrier-driven main loop.
//
// Behaviour follows src/cpp_extensions/ext_aggregator.cpp (slot pool :138-328,
// weight init :338-459, rounds :470-875, barrier :879-987, main loop
// :1024-1210); the compute of every round is libswl's own kernels (no torch).
// Deliberate differences, all documented in the repository's design notes:
//   * a command failing validation (slot range, ownership, size) evicts that
//     slot and the round proceeds for the others instead of ending the loop;
//   * slot buffer capacity is checked against every round's shape;
//   * LoRA deltas of pooled adapters are added in the round's epilogue.

#include <hip/hip_runtime.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "ipc_layout.h"
#include "queue_map.h"
#include "swl_common.h"
#include "swl_runtime.h"

namespace swl {
int round_launch(int n_seg, const int64_t* rows, const void* const* seg_in, void* const* seg_out, const void* w,
                 const void* bias, int64_t N, int64_t K, const int32_t* seg_lora, const swl_lora_entry* lora_table,
                 const swl_lora_entry* host_entries, int nblk, const int64_t* blk_cols, hipStream_t st,
                 const swl_round_fusion* fz = nullptr);
}  // namespace swl

using swl::AtomicMask;
using swl::Mask;

namespace {

struct alignas(64) SlotInfo {
  std::atomic<int> owner{-1};
  void* in = nullptr;
  void* out = nullptr;
  hipIpcMemHandle_t in_handle;
  hipIpcMemHandle_t out_handle;
};

struct Pool {
  SlotInfo slots[SWL_MAX_SLOTS];
  AtomicMask free_mask;
  AtomicMask active_mask;
  std::atomic<int> active_slot_count{0};
  int num_slots = 0;
  int device = 0;
  int hidden = 0, inter = 0, qkv = 0;
  int max_seq_per_step = 0;
  size_t in_size = 0, out_size = 0;
  bool initialized = false;
  uint32_t* seq_timeout = nullptr;  // host-visible, one word per slot (GPU-ordered input waits that timed out)
};
Pool g_pool;

// Limit of the aggregator stream's wait for a GPU-ordered worker's input.
constexpr uint32_t kSeqWaitLimitUs = 2000000;
// Largest buffer a hipIpc mapping can take here (2 GiB).
constexpr size_t kMaxIpcBytes = (size_t)1 << 31;

struct LayerW {
  void* qkv = nullptr;      // owned: [q+k+v, hidden]
  void* gate_up = nullptr;  // owned: [gate+up, hidden]
  const void* o = nullptr;
  const void* o_bias = nullptr;
  const void* down = nullptr;
  const void* down_bias = nullptr;
  int64_t q = 0, k = 0, v = 0, gate = 0, up = 0;
};
std::vector<LayerW> g_layers;
int g_num_layers = 0;
int g_device = 0;
bool g_weights_ready = false;
int64_t g_hidden = 0, g_inter = 0;

const void* g_embed = nullptr;
const void* g_lm_head = nullptr;
int64_t g_vocab = 0;
void* g_logits = nullptr;      // [MAX_SLOTS, vocab] bf16
void* g_last_hidden = nullptr; // [MAX_SLOTS, hidden] bf16
int64_t* g_next_tok = nullptr; // [MAX_SLOTS] int64

swl::QueueMap g_agg_q;
hipStream_t g_stream = nullptr;

// adapter pool: (adapter, layer, op) -> entry
std::mutex g_adapter_mu;
std::map<std::tuple<int, int, int>, int> g_adapter_index;
std::vector<swl_lora_entry> g_adapter_entries;
swl_lora_entry* g_adapter_dev = nullptr;
size_t g_adapter_dev_cap = 0;
bool g_adapter_dirty = false;

std::map<int, swl::SamplingParams> g_sampling;  // per worker (OP_SET_SAMPLING / join)

int g_evict_ms = 500;
int g_leave_check_ms = 10;

int stream_get(hipStream_t* out) {
  if (!g_stream) {
    SWL_HIP(hipSetDevice(g_device));
    SWL_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  }
  *out = g_stream;
  return SWL_OK;
}

int op_dims(int op, int64_t* K, int64_t* N, int* nblk, int64_t* blk) {
  const LayerW& l = g_layers[0];
  switch (op) {
    case SWL_OP_QKV_FUSED:
      *K = g_hidden; *N = l.q + l.k + l.v; *nblk = 3; blk[0] = l.q; blk[1] = l.k; blk[2] = l.v; return SWL_OK;
    case SWL_OP_O_PROJ:
      *K = g_hidden; *N = g_hidden; *nblk = 1; blk[0] = g_hidden; return SWL_OK;
    case SWL_OP_GATE_UP_FUSED:
      *K = g_hidden; *N = l.gate + l.up; *nblk = 2; blk[0] = l.gate; blk[1] = l.up; return SWL_OK;
    case SWL_OP_DOWN_PROJ:
      *K = g_inter; *N = g_hidden; *nblk = 1; blk[0] = g_hidden; return SWL_OK;
    default:
      return swl::fail(SWL_ERR_INVALID, "execute_batched_gemm: unknown op_type " + std::to_string(op));
  }
}

// Device copy of the adapter table.  Rounds already queued on the
// aggregator stream (GPU-ordered rounds are not host-synchronised) may still
// read the current table, so the stream is drained before the table is
// rewritten, and a table that has to grow is replaced by a new allocation
// while the old one stays allocated until the process ends.
std::vector<void*> g_adapter_dev_kept;

int upload_adapters() {
  std::lock_guard<std::mutex> lk(g_adapter_mu);
  if (!g_adapter_dirty) return SWL_OK;
  if (g_stream) SWL_HIP(hipStreamSynchronize(g_stream));
  const size_t need = std::max<size_t>(g_adapter_entries.size(), 1);
  if (g_adapter_dev_cap < need) {
    if (g_adapter_dev) g_adapter_dev_kept.push_back(g_adapter_dev);
    g_adapter_dev = nullptr;
    size_t cap = 64;
    while (cap < need) cap *= 2;
    SWL_HIP(hipMalloc(&g_adapter_dev, cap * sizeof(swl_lora_entry)));
    g_adapter_dev_cap = cap;
  }
  if (!g_adapter_entries.empty())
    SWL_HIP(hipMemcpy(g_adapter_dev, g_adapter_entries.data(), g_adapter_entries.size() * sizeof(swl_lora_entry),
                      hipMemcpyHostToDevice));
  g_adapter_dirty = false;
  return SWL_OK;
}

}  // namespace

namespace {
int drain_impl(uint64_t active_lo, uint64_t active_hi, int want, int32_t* slot_ids, int32_t* worker_ids, int32_t* ops,
               int32_t* layers, int64_t* tokens, uint64_t* x_keys, uint64_t* in_seqs, int32_t* out_host, int* got);
}  // namespace

extern "C" {

// ------------------------------------------------------------- slot pool
int swl_agg_init_slot_pool(int num_slots, int device_index, int hidden_dim, int intermediate_dim, int num_kv_heads,
                           int head_dim, int max_seq_per_step, int dtype_size, size_t* input_buffer_size,
                           size_t* output_buffer_size) {
  SWL_CHECK(num_slots > 0 && num_slots <= SWL_MAX_SLOTS, SWL_ERR_INVALID,
            "num_slots must be between 1 and " + std::to_string(SWL_MAX_SLOTS));
  SWL_CHECK(hidden_dim > 0 && intermediate_dim > 0 && max_seq_per_step > 0 && dtype_size > 0, SWL_ERR_INVALID,
            "init_slot_pool: dimensions must be positive");
  SWL_CHECK(!g_pool.initialized, SWL_ERR_STATE, "init_slot_pool: slot pool already initialized");
  const int qkv = hidden_dim + num_kv_heads * head_dim * 2;
  const size_t in_size = (size_t)max_seq_per_step * std::max(intermediate_dim, hidden_dim) * dtype_size;
  const size_t out_size = (size_t)max_seq_per_step * std::max(intermediate_dim * 2, qkv) * dtype_size;
  // IPC mappings of 2 GiB or more do not open on these devices: refuse such
  // buffers here rather than in every worker's open_slot
  SWL_CHECK(in_size < kMaxIpcBytes && out_size + swl::kSeqTailBytes < kMaxIpcBytes, SWL_ERR_INVALID,
            "init_slot_pool: slot buffers of " + std::to_string(in_size) + " / " +
                std::to_string(out_size + swl::kSeqTailBytes) +
                " bytes reach the 2 GiB limit of an IPC mapping (lower max_seq_per_step)");
  SWL_HIP(hipSetDevice(device_index));
  Pool& p = g_pool;
  p.num_slots = num_slots;
  p.device = device_index;
  p.hidden = hidden_dim;
  p.inter = intermediate_dim;
  p.qkv = qkv;
  p.max_seq_per_step = max_seq_per_step;
  p.in_size = in_size;
  p.out_size = out_size;
  p.free_mask.store(Mask::below(num_slots), std::memory_order_relaxed);
  p.active_mask.store(Mask(), std::memory_order_relaxed);
  p.active_slot_count.store(0, std::memory_order_relaxed);
  for (int i = 0; i < num_slots; ++i) {
    SlotInfo& s = p.slots[i];
    s.owner.store(-1, std::memory_order_relaxed);
    SWL_HIP(hipMalloc(&s.in, p.in_size));
    SWL_HIP(hipMemset(s.in, 0, p.in_size));
    SWL_HIP(hipIpcGetMemHandle(&s.in_handle, s.in));
    // the output buffer carries the slot's two sequence words in a tail past
    // out_size (GPU-ordered rounds)
    SWL_HIP(hipMalloc(&s.out, p.out_size + swl::kSeqTailBytes));
    SWL_HIP(hipMemset(s.out, 0, p.out_size + swl::kSeqTailBytes));
    SWL_HIP(hipIpcGetMemHandle(&s.out_handle, s.out));
  }
  SWL_HIP(hipHostMalloc((void**)&p.seq_timeout, SWL_MAX_SLOTS * sizeof(uint32_t), hipHostMallocDefault));
  std::memset(p.seq_timeout, 0, SWL_MAX_SLOTS * sizeof(uint32_t));
  p.initialized = true;
  if (input_buffer_size) *input_buffer_size = p.in_size;
  if (output_buffer_size) *output_buffer_size = p.out_size;
  std::printf("[Aggregator] Slot pool: %d slots, %zu KB input + %zu KB output per slot\n", num_slots,
              p.in_size / 1024, p.out_size / 1024);
  std::fflush(stdout);
  return SWL_OK;
}

int swl_agg_scrub_slot(int slot_id) {
  SWL_CHECK(slot_id >= 0 && slot_id < SWL_MAX_SLOTS, SWL_ERR_INVALID, "scrub_slot: invalid slot_id");
  // A previous tenant may have left a ready bit (signalled, then killed or
  // evicted) or an evicted bit (went silent): the new owner starts clean.
  if (g_agg_q.ctrl) {
    g_agg_q.ctrl->ready.clear_bits(Mask::bit(slot_id));
    g_agg_q.ctrl->evicted.clear_bits(Mask::bit(slot_id));
  }
  return SWL_OK;
}

int swl_agg_claim_slot(int worker_id, int* slot_id, uint8_t* input_handle, uint8_t* output_handle,
                       size_t* input_buffer_size, size_t* output_buffer_size) {
  SWL_CHECK(g_pool.initialized, SWL_ERR_STATE, "claim_slot: slot pool not initialized");
  static_assert(sizeof(hipIpcMemHandle_t) == SWL_IPC_HANDLE_BYTES, "IPC handle size");
  Pool& p = g_pool;
  while (true) {
    Mask fm = p.free_mask.load(std::memory_order_acquire);
    if (fm.empty()) return swl::fail(SWL_ERR_NOT_FOUND, "No free slots available");
    const int sid = fm.first();
    const int wi = sid >> 6;
    const uint64_t bit = 1ull << (sid & 63);
    uint64_t expected = fm.w[wi];
    if (!p.free_mask.w[wi].compare_exchange_weak(expected, expected & ~bit, std::memory_order_acq_rel,
                                                 std::memory_order_acquire))
      continue;
    SlotInfo& s = p.slots[sid];
    s.owner.store(worker_id, std::memory_order_release);
    (void)swl_agg_scrub_slot(sid);
    *slot_id = sid;
    if (input_handle) std::memcpy(input_handle, &s.in_handle, sizeof(hipIpcMemHandle_t));
    if (output_handle) std::memcpy(output_handle, &s.out_handle, sizeof(hipIpcMemHandle_t));
    if (input_buffer_size) *input_buffer_size = p.in_size;
    if (output_buffer_size) *output_buffer_size = p.out_size;
    std::printf("[Aggregator] Slot %d claimed by worker %d\n", sid, worker_id);
    std::fflush(stdout);
    return SWL_OK;
  }
}

int swl_agg_release_slot(int slot_id, int worker_id) {
  SWL_CHECK(g_pool.initialized, SWL_ERR_STATE, "release_slot: slot pool not initialized");
  SWL_CHECK(slot_id >= 0 && slot_id < g_pool.num_slots, SWL_ERR_INVALID, "release_slot: invalid slot_id");
  SlotInfo& s = g_pool.slots[slot_id];
  int expected = worker_id;
  if (!s.owner.compare_exchange_strong(expected, -1, std::memory_order_acq_rel, std::memory_order_acquire))
    return swl::fail(SWL_ERR_INVALID, "release_slot: worker does not own slot " + std::to_string(slot_id));
  // Zero both buffers and wait before the slot becomes claimable again: the
  // next tenant writes from another process with no ordering against this.
  SWL_HIP(hipSetDevice(g_pool.device));
  hipStream_t st;
  int rc = stream_get(&st);
  if (rc) return rc;
  SWL_HIP(hipMemsetAsync(s.in, 0, g_pool.in_size, st));
  SWL_HIP(hipMemsetAsync(s.out, 0, g_pool.out_size + swl::kSeqTailBytes, st));  // sequence words restart at 0
  SWL_HIP(hipStreamSynchronize(st));
  g_pool.free_mask.set_bit(slot_id);
  g_pool.active_mask.clear_bits(Mask::bit(slot_id));
  std::printf("[Aggregator] Slot %d released by worker %d\n", slot_id, worker_id);
  std::fflush(stdout);
  return SWL_OK;
}

int swl_agg_get_slot_owner(int slot_id) {
  if (!g_pool.initialized || slot_id < 0 || slot_id >= g_pool.num_slots) return -1;
  return g_pool.slots[slot_id].owner.load(std::memory_order_acquire);
}

int swl_agg_pool_status(swl_pool_status* out) {
  SWL_CHECK(out, SWL_ERR_INVALID, "get_slot_pool_status: null output");
  std::memset(out, 0, sizeof(*out));
  out->initialized = g_pool.initialized ? 1 : 0;
  out->num_slots = g_pool.num_slots;
  const Mask fm = g_pool.free_mask.load(), am = g_pool.active_mask.load();
  out->free_lo = fm.w[0];
  out->free_hi = fm.w[1];
  out->active_lo = am.w[0];
  out->active_hi = am.w[1];
  out->active_slot_count = g_pool.active_slot_count.load(std::memory_order_acquire);
  for (int i = 0; i < g_pool.num_slots; ++i) out->owners[i] = g_pool.slots[i].owner.load(std::memory_order_acquire);
  return SWL_OK;
}

int swl_agg_cleanup_slot_pool(void) {
  if (!g_pool.initialized) return SWL_OK;
  SWL_HIP(hipSetDevice(g_pool.device));
  SWL_HIP(hipDeviceSynchronize());
  for (int i = 0; i < g_pool.num_slots; ++i) {
    SlotInfo& s = g_pool.slots[i];
    if (s.in) SWL_HIP(hipFree(s.in));
    if (s.out) SWL_HIP(hipFree(s.out));
    s.in = s.out = nullptr;
    s.owner.store(-1);
  }
  if (g_pool.seq_timeout) SWL_HIP(hipHostFree(g_pool.seq_timeout));
  g_pool.seq_timeout = nullptr;
  g_pool.initialized = false;
  g_pool.num_slots = 0;
  std::printf("[Aggregator] Slot pool cleaned up\n");
  std::fflush(stdout);
  return SWL_OK;
}

int swl_agg_slot_buffers(int slot_id, void** input_buffer, void** output_buffer) {
  SWL_CHECK(g_pool.initialized, SWL_ERR_STATE, "slot pool not initialized");
  SWL_CHECK(slot_id >= 0 && slot_id < g_pool.num_slots, SWL_ERR_INVALID, "invalid slot_id");
  if (input_buffer) *input_buffer = g_pool.slots[slot_id].in;
  if (output_buffer) *output_buffer = g_pool.slots[slot_id].out;
  return SWL_OK;
}

// ---------------------------------------------------------------- weights
int swl_agg_begin(int num_layers, int device_index) {
  SWL_CHECK(num_layers > 0, SWL_ERR_INVALID, "init_aggregator_begin: num_layers must be positive");
  SWL_HIP(hipSetDevice(device_index));
  for (LayerW& l : g_layers) {
    if (l.qkv) SWL_HIP(hipFree(l.qkv));
    if (l.gate_up) SWL_HIP(hipFree(l.gate_up));
  }
  g_layers.assign(num_layers, LayerW());
  g_num_layers = num_layers;
  g_device = device_index;
  g_weights_ready = false;
  g_hidden = 0;
  g_inter = 0;
  std::printf("[Aggregator] Begin weight init: %d layers on device %d\n", num_layers, device_index);
  std::fflush(stdout);
  return SWL_OK;
}

int swl_agg_set_layer(int layer_idx, const void* q, int64_t q_rows, const void* k, int64_t k_rows, const void* v,
                      int64_t v_rows, const void* o, const void* o_bias, const void* gate, int64_t gate_rows,
                      const void* up, int64_t up_rows, const void* down, const void* down_bias, int64_t hidden_dim,
                      int64_t intermediate_dim) {
  SWL_CHECK(layer_idx >= 0 && layer_idx < g_num_layers, SWL_ERR_INVALID,
            "init_aggregator_layer: layer_idx " + std::to_string(layer_idx) + " out of range [0, " +
                std::to_string(g_num_layers) + ")");
  SWL_CHECK(q && k && v && o && gate && up && down, SWL_ERR_INVALID, "init_aggregator_layer: null weight");
  SWL_CHECK(hidden_dim > 0 && intermediate_dim > 0, SWL_ERR_INVALID, "init_aggregator_layer: bad dims");
  SWL_CHECK(hidden_dim % 64 == 0 && intermediate_dim % 64 == 0, SWL_ERR_INVALID,
            "init_aggregator_layer: hidden and intermediate sizes must be multiples of 64");
  if (g_hidden == 0) {
    g_hidden = hidden_dim;
    g_inter = intermediate_dim;
  }
  SWL_CHECK(g_hidden == hidden_dim && g_inter == intermediate_dim, SWL_ERR_INVALID,
            "init_aggregator_layer: all layers must share hidden/intermediate sizes");
  LayerW& l = g_layers[layer_idx];
  SWL_HIP(hipSetDevice(g_device));
  const size_t row = (size_t)hidden_dim * 2;
  if (l.qkv) SWL_HIP(hipFree(l.qkv));
  if (l.gate_up) SWL_HIP(hipFree(l.gate_up));
  SWL_HIP(hipMalloc(&l.qkv, (q_rows + k_rows + v_rows) * row));
  SWL_HIP(hipMemcpy(l.qkv, q, q_rows * row, hipMemcpyDeviceToDevice));
  SWL_HIP(hipMemcpy((char*)l.qkv + q_rows * row, k, k_rows * row, hipMemcpyDeviceToDevice));
  SWL_HIP(hipMemcpy((char*)l.qkv + (q_rows + k_rows) * row, v, v_rows * row, hipMemcpyDeviceToDevice));
  SWL_HIP(hipMalloc(&l.gate_up, (gate_rows + up_rows) * row));
  SWL_HIP(hipMemcpy(l.gate_up, gate, gate_rows * row, hipMemcpyDeviceToDevice));
  SWL_HIP(hipMemcpy((char*)l.gate_up + gate_rows * row, up, up_rows * row, hipMemcpyDeviceToDevice));
  l.o = o;
  l.o_bias = o_bias;
  l.down = down;
  l.down_bias = down_bias;
  l.q = q_rows;
  l.k = k_rows;
  l.v = v_rows;
  l.gate = gate_rows;
  l.up = up_rows;
  return SWL_OK;
}

int swl_agg_finalize(void) {
  SWL_CHECK(g_num_layers > 0, SWL_ERR_STATE, "init_aggregator_finalize: no layers");
  for (int i = 0; i < g_num_layers; ++i)
    SWL_CHECK(g_layers[i].qkv != nullptr, SWL_ERR_STATE,
              "init_aggregator_finalize: layer " + std::to_string(i) + " not initialized");
  SWL_HIP(hipSetDevice(g_device));
  SWL_HIP(hipDeviceSynchronize());
  g_weights_ready = true;
  const LayerW& l = g_layers[0];
  std::printf("[Aggregator] Weights initialized with fused QKV (%lld) and gate/up (%lld) per layer\n",
              (long long)(l.q + l.k + l.v), (long long)(l.gate + l.up));
  std::fflush(stdout);
  return SWL_OK;
}

int swl_agg_set_embed_lm_head(const void* embed, const void* lm_head, int64_t vocab_size, int64_t hidden_dim) {
  SWL_CHECK(embed && lm_head && vocab_size > 0 && hidden_dim > 0, SWL_ERR_INVALID,
            "init_embed_lm_head_weights: bad arguments");
  SWL_HIP(hipSetDevice(g_device));
  if (g_logits) SWL_HIP(hipFree(g_logits));
  if (g_last_hidden) SWL_HIP(hipFree(g_last_hidden));
  if (g_next_tok) SWL_HIP(hipFree(g_next_tok));
  SWL_HIP(hipMalloc(&g_logits, (size_t)SWL_MAX_SLOTS * vocab_size * 2));
  SWL_HIP(hipMalloc(&g_last_hidden, (size_t)SWL_MAX_SLOTS * hidden_dim * 2));
  SWL_HIP(hipMalloc(&g_next_tok, (size_t)SWL_MAX_SLOTS * sizeof(int64_t)));
  g_embed = embed;
  g_lm_head = lm_head;
  g_vocab = vocab_size;
  if (g_hidden == 0) g_hidden = hidden_dim;
  std::printf("[Aggregator] Embed/LM-head weights initialized: vocab=%lld, hidden=%lld\n", (long long)vocab_size,
              (long long)hidden_dim);
  std::fflush(stdout);
  return SWL_OK;
}

int swl_agg_attach_queue(const char* shm_name, int capacity) {
  SWL_CHECK(capacity > 0, SWL_ERR_INVALID, "init_aggregator_queue: capacity must be positive");
  SWL_CHECK(shm_name && shm_name[0], SWL_ERR_INVALID, "init_aggregator_queue: shm_name cannot be empty");
  return g_agg_q.open(shm_name, capacity);
}

// ---------------------------------------------------------- adapter pool
int swl_agg_register_adapter(int adapter_id, int layer_idx, int op_type, const void* a, const void* const* b,
                             int nblk, int rank, float scale) {
  SWL_CHECK(adapter_id >= 0, SWL_ERR_INVALID, "register_adapter: adapter_id must be >= 0");
  SWL_CHECK(a && b && nblk >= 1 && nblk <= SWL_MAX_LORA_BLOCKS && rank > 0 && rank <= 256, SWL_ERR_INVALID,
            "register_adapter: bad adapter description");
  SWL_CHECK(op_type == SWL_OP_QKV_FUSED || op_type == SWL_OP_O_PROJ || op_type == SWL_OP_GATE_UP_FUSED ||
                op_type == SWL_OP_DOWN_PROJ,
            SWL_ERR_INVALID, "register_adapter: op_type must be a projection op");
  swl_lora_entry e{};
  e.a = a;
  for (int j = 0; j < nblk; ++j) {
    SWL_CHECK(b[j] != nullptr, SWL_ERR_INVALID, "register_adapter: null lora_B");
    e.b[j] = b[j];
  }
  e.rank = rank;
  e.scale = scale;
  std::lock_guard<std::mutex> lk(g_adapter_mu);
  const auto key = std::make_tuple(adapter_id, layer_idx, op_type);
  auto it = g_adapter_index.find(key);
  if (it != g_adapter_index.end()) {
    g_adapter_entries[it->second] = e;
  } else {
    g_adapter_index[key] = (int)g_adapter_entries.size();
    g_adapter_entries.push_back(e);
  }
  g_adapter_dirty = true;
  return SWL_OK;
}

int swl_agg_clear_adapters(void) {
  std::lock_guard<std::mutex> lk(g_adapter_mu);
  g_adapter_index.clear();
  g_adapter_entries.clear();
  g_adapter_dirty = true;
  return SWL_OK;
}

// ------------------------------------------------------------------ rounds
int swl_agg_execute_round(int op_type, int layer_idx, int n, const int32_t* slot_ids, const int32_t* worker_ids,
                          const int64_t* tokens, const int32_t* adapter_ids, void* stream) {
  SWL_CHECK(g_pool.initialized, SWL_ERR_STATE, "execute_batched_gemm: slot pool not initialized");
  SWL_CHECK(g_weights_ready, SWL_ERR_STATE, "execute_batched_gemm: weights not initialized");
  SWL_CHECK(n >= 1 && n <= SWL_MAX_SLOTS && slot_ids && tokens, SWL_ERR_INVALID,
            "execute_batched_gemm: bad command list");
  SWL_CHECK(layer_idx >= 0 && layer_idx < g_num_layers, SWL_ERR_INVALID,
            "execute_batched_gemm_slots: layer_idx " + std::to_string(layer_idx) + " out of range [0, " +
                std::to_string(g_num_layers) + ")");
  int64_t K = 0, N = 0, blk[SWL_MAX_LORA_BLOCKS] = {0, 0, 0, 0};
  int nblk = 1;
  int rc = op_dims(op_type, &K, &N, &nblk, blk);
  if (rc) return rc;
  const LayerW& l = g_layers[layer_idx];
  const void* w = nullptr;
  const void* bias = nullptr;
  switch (op_type) {
    case SWL_OP_QKV_FUSED: w = l.qkv; break;
    case SWL_OP_O_PROJ: w = l.o; bias = l.o_bias; break;
    case SWL_OP_GATE_UP_FUSED: w = l.gate_up; break;
    default: w = l.down; bias = l.down_bias; break;
  }
  const void* seg_in[SWL_MAX_SLOTS];
  void* seg_out[SWL_MAX_SLOTS];
  int64_t rows[SWL_MAX_SLOTS];
  int32_t seg_lora[SWL_MAX_SLOTS];
  bool any_lora = false;
  for (int i = 0; i < n; ++i) {
    const int sid = slot_ids[i];
    SWL_CHECK(sid >= 0 && sid < g_pool.num_slots, SWL_ERR_INVALID,
              "execute_batched_gemm: invalid slot_id: " + std::to_string(sid));
    if (worker_ids) {
      const int owner = g_pool.slots[sid].owner.load(std::memory_order_acquire);
      SWL_CHECK(owner == worker_ids[i], SWL_ERR_INVALID,
                "execute_batched_gemm: worker " + std::to_string(worker_ids[i]) + " does not own slot " +
                    std::to_string(sid) + " (owner=" + std::to_string(owner) + ")");
    }
    SWL_CHECK(tokens[i] > 0 && tokens[i] <= (int64_t)65536 * 65536, SWL_ERR_INVALID,
              "execute_batched_gemm: invalid bx/tx dimensions");
    SWL_CHECK((size_t)tokens[i] * K * 2 <= g_pool.in_size && (size_t)tokens[i] * N * 2 <= g_pool.out_size,
              SWL_ERR_INVALID,
              "execute_batched_gemm: slot " + std::to_string(sid) + " round of " + std::to_string(tokens[i]) +
                  " tokens exceeds the slot buffers");
    seg_in[i] = g_pool.slots[sid].in;
    seg_out[i] = g_pool.slots[sid].out;
    rows[i] = tokens[i];
    seg_lora[i] = -1;
    if (adapter_ids && adapter_ids[i] >= 0) {
      std::lock_guard<std::mutex> lk(g_adapter_mu);
      auto it = g_adapter_index.find(std::make_tuple((int)adapter_ids[i], layer_idx, op_type));
      if (it != g_adapter_index.end()) {
        seg_lora[i] = it->second;
        any_lora = true;
      }
    }
  }
  hipStream_t st = (hipStream_t)stream;
  if (any_lora) {
    rc = upload_adapters();
    if (rc) return rc;
  }
  return swl::round_launch(n, rows, seg_in, seg_out, w, bias, N, K, any_lora ? seg_lora : nullptr,
                           any_lora ? g_adapter_dev : nullptr, any_lora ? g_adapter_entries.data() : nullptr, nblk,
                           blk, st);
}

// ----------------------------------------------------------------- barrier
int swl_agg_set_barrier_timeouts(int evict_ms, int leave_check_ms) {
  SWL_CHECK(evict_ms > 0 && leave_check_ms > 0, SWL_ERR_INVALID, "timeouts must be positive");
  g_evict_ms = evict_ms;
  g_leave_check_ms = leave_check_ms;
  return SWL_OK;
}

// Spin until every active slot has signalled ready.  Slots that ask to leave
// mid-op are dropped (checked every leave-check period); slots silent for the
// eviction period are evicted (their evicted bit tells the worker to abort).
int swl_agg_wait_for_slots(uint64_t* active_lo, uint64_t* active_hi, int* count_out) {
  SWL_CHECK(g_agg_q.ctrl, SWL_ERR_STATE, "Aggregator queue not initialized");
  swl::Control* c = g_agg_q.ctrl;
  Mask active{{*active_lo, *active_hi}};
  *count_out = active.count();
  if (active.empty()) return SWL_OK;
  using clk = std::chrono::steady_clock;
  auto start = clk::now();
  auto last_leave_check = start;
  int spins = 0;
  while (true) {
    const Mask missing = active & ~c->ready.load();
    if (missing.empty()) break;
    if (c->quit.load(std::memory_order_acquire) != 0) {
      *count_out = -1;
      return SWL_OK;
    }
    ++spins;
    if (spins < swl::kSpinTight) continue;
    if (spins < swl::kSpinYield) {
      swl::cpu_relax();
      continue;
    }
    const auto now = clk::now();
    if (now - last_leave_check > std::chrono::milliseconds(g_leave_check_ms)) {
      last_leave_check = now;
      const Mask leaving = c->leaves.load() & active;
      if (!leaving.empty()) {
        active = active & ~leaving;
        c->leaves.clear_bits(leaving, std::memory_order_acq_rel);
        c->active.store(active);
        c->active_count.store(active.count(), std::memory_order_release);
        std::printf("[Aggregator] Mid-op slot leave: mask=0x%llx:%llx, now waiting for %d slots\n",
                    (unsigned long long)leaving.w[1], (unsigned long long)leaving.w[0], active.count());
        std::fflush(stdout);
        if (active.empty()) break;
      }
    }
    if (now - start > std::chrono::milliseconds(g_evict_ms)) {
      const Mask stuck = active & ~c->ready.load();
      if (!stuck.empty()) {
        active = active & ~stuck;
        c->active.store(active);
        c->active_count.store(active.count(), std::memory_order_release);
        Mask rem = stuck;
        while (!rem.empty()) {
          const int sid = rem.first();
          rem.clear(sid);
          c->evicted.set_bit(sid);
        }
        std::fprintf(stderr, "[Aggregator] EVICTING stuck slot(s) after %d ms (mask=0x%llx:%llx). %d continue.\n",
                     g_evict_ms, (unsigned long long)stuck.w[1], (unsigned long long)stuck.w[0], active.count());
        std::fflush(stderr);
        if (active.empty()) break;
        start = clk::now();
        spins = 0;
      }
    }
    swl::cpu_relax();
    swl::cpu_relax();
  }
  *active_lo = active.w[0];
  *active_hi = active.w[1];
  *count_out = active.count();
  return SWL_OK;
}

int swl_agg_signal_done(void) {
  SWL_CHECK(g_agg_q.ctrl, SWL_ERR_STATE, "Aggregator queue not initialized");
  swl::Control* c = g_agg_q.ctrl;
  c->ready_count.store(0, std::memory_order_release);
  c->ready.clear_bits(c->active.load());
  c->epoch.fetch_add(1, std::memory_order_acq_rel);
  return SWL_OK;
}

int swl_agg_drain_commands(uint64_t active_lo, uint64_t active_hi, int want, int32_t* slot_ids, int32_t* worker_ids,
                           int32_t* ops, int32_t* layers, int64_t* tokens, uint64_t* x_keys, int* got) {
  return drain_impl(active_lo, active_hi, want, slot_ids, worker_ids, ops, layers, tokens, x_keys, nullptr, nullptr,
                    got);
}

int swl_agg_take_seq_timeouts(int32_t* slot_ids, int max_ids) {
  if (!g_pool.initialized || !g_pool.seq_timeout) return 0;
  int n = 0;
  for (int i = 0; i < SWL_MAX_SLOTS; ++i) {
    if (__atomic_exchange_n(&g_pool.seq_timeout[i], 0u, __ATOMIC_ACQ_REL) == 0) continue;
    if (slot_ids && n < max_ids) slot_ids[n] = i;
    ++n;
  }
  return n;
}

}  // extern "C"

namespace {
int drain_impl(uint64_t active_lo, uint64_t active_hi, int want, int32_t* slot_ids, int32_t* worker_ids, int32_t* ops,
               int32_t* layers, int64_t* tokens, uint64_t* x_keys, uint64_t* in_seqs, int32_t* out_host, int* got) {
  SWL_CHECK(g_agg_q.ctrl && g_agg_q.ring, SWL_ERR_STATE, "Aggregator queue not initialized");
  swl::Control* c = g_agg_q.ctrl;
  const Mask active{{active_lo, active_hi}};
  int tail = c->tail.load(std::memory_order_acquire);
  int n = 0, drained = 0;
  const int max_drain = SWL_MAX_SLOTS + 8;
  while (n < want && drained < max_drain) {
    swl::Command& cmd = g_agg_q.ring[tail];
    long spins = 0;
    bool quit = false;
    while (cmd.ready.load(std::memory_order_acquire) != 1) {
      if (c->quit.load(std::memory_order_acquire) != 0) {
        quit = true;
        break;
      }
      if (++spins > 10000000) {
        std::fprintf(stderr, "[Aggregator] ERROR: command not ready after eviction drain\n");
        c->quit.store(1, std::memory_order_release);
        quit = true;
        break;
      }
      if (spins > swl::kSpinTight) swl::cpu_relax();
    }
    if (quit) break;
    const int sid = cmd.slot_id;
    const bool keep = sid >= 0 && sid < SWL_MAX_SLOTS && active.test(sid);
    if (keep) {
      slot_ids[n] = sid;
      worker_ids[n] = cmd.worker_id;
      ops[n] = cmd.op_type;
      layers[n] = cmd.layer_idx;
      tokens[n] = cmd.bx * cmd.tx;
      x_keys[n] = cmd.x_key;
      if (in_seqs) in_seqs[n] = cmd.in_seq;
      if (out_host) out_host[n] = cmd.out_host;
      if (cmd.op_type == SWL_OP_SET_SAMPLING) {
        swl::SamplingParams p;
        p.do_sample = (cmd.x_key & 1) ? 1 : 0;
        p.temperature = (float)(cmd.x_key >> 1) / 10000.0f;
        p.top_k = (int32_t)cmd.y0_key;
        p.top_p = (float)cmd.y1_key / 10000.0f;
        g_sampling[cmd.worker_id] = p;
      }
      ++n;
    }
    cmd.ready.store(0, std::memory_order_release);
    tail = (tail + 1) % g_agg_q.capacity;
    ++drained;
  }
  c->tail.store(tail, std::memory_order_release);
  *got = n;
  return SWL_OK;
}
}  // namespace

// ----------------------------------------------------------- main loop ops
namespace swl {
int embed_launch(int n, const int64_t* rows, const void* const* ids, void* const* out, const void* table,
                 int64_t vocab, int64_t hidden, hipStream_t st);
int lm_head_launch(int n, const void* const* last_rows, const void* lm_head, int64_t vocab, int64_t hidden,
                   void* packed, void* logits, int64_t* next_tok, void* const* out_tok, const int32_t* do_sample,
                   const float* temperature, const int32_t* top_k, const float* top_p, uint64_t seed, hipStream_t st);
}  // namespace swl

namespace {

void apply_join_sampling(const Mask& joins) {
  swl::Control* c = g_agg_q.ctrl;
  const Mask todo = c->sampling_pending.load() & joins;
  Mask rem = todo;
  while (!rem.empty()) {
    const int sid = rem.first();
    rem.clear(sid);
    const int wid = g_pool.slots[sid].owner.load(std::memory_order_acquire);
    if (wid >= 0) g_sampling[wid] = c->sampling[sid];
  }
  c->sampling_pending.clear_bits(todo);
}

int run_op(int op, int layer, int n, const int32_t* sids, const int32_t* wids, const int64_t* toks,
           const uint64_t* keys, hipStream_t st, uint64_t step) {
  if (op == SWL_OP_EMBED || op == SWL_OP_LM_HEAD) {
    SWL_CHECK(g_embed && g_lm_head, SWL_ERR_STATE, "embed/LM-head weights not initialized");
    const void* src[SWL_MAX_SLOTS];
    void* dst[SWL_MAX_SLOTS];
    int64_t rows[SWL_MAX_SLOTS];
    for (int i = 0; i < n; ++i) {
      const int sid = sids[i];
      SWL_CHECK(sid >= 0 && sid < g_pool.num_slots, SWL_ERR_INVALID,
                "execute_batched_embed: invalid slot_id: " + std::to_string(sid));
      const int owner = g_pool.slots[sid].owner.load(std::memory_order_acquire);
      SWL_CHECK(owner == wids[i], SWL_ERR_INVALID,
                "worker " + std::to_string(wids[i]) + " does not own slot " + std::to_string(sid));
      SWL_CHECK(toks[i] > 0 && (size_t)toks[i] * g_hidden * 2 <= g_pool.out_size &&
                    (size_t)toks[i] * 8 <= g_pool.in_size && (size_t)toks[i] * g_hidden * 2 <= g_pool.in_size,
                SWL_ERR_INVALID, "execute_batched_embed: invalid bx/tx dimensions");
      rows[i] = toks[i];
      dst[i] = g_pool.slots[sid].out;
      src[i] = g_pool.slots[sid].in;
    }
    if (op == SWL_OP_EMBED) return swl::embed_launch(n, rows, src, dst, g_embed, g_vocab, g_hidden, st);
    const void* last[SWL_MAX_SLOTS];
    int32_t ds[SWL_MAX_SLOTS], tk[SWL_MAX_SLOTS];
    float te[SWL_MAX_SLOTS], tp[SWL_MAX_SLOTS];
    for (int i = 0; i < n; ++i) {
      last[i] = (const char*)src[i] + (size_t)(rows[i] - 1) * g_hidden * 2;
      auto it = g_sampling.find(wids[i]);
      const swl::SamplingParams p = (it != g_sampling.end()) ? it->second : swl::SamplingParams{0, 1.f, 0, 1.f};
      ds[i] = p.do_sample;
      te[i] = p.temperature < 0.01f ? 0.01f : p.temperature;
      tk[i] = p.top_k;
      tp[i] = p.top_p;
    }
    return swl::lm_head_launch(n, last, g_lm_head, g_vocab, g_hidden, g_last_hidden, g_logits, g_next_tok, dst, ds,
                               te, tk, tp, step, st);
  }
  int32_t adapters[SWL_MAX_SLOTS];
  for (int i = 0; i < n; ++i) adapters[i] = keys[i] ? (int32_t)(keys[i] - 1) : -1;
  return swl_agg_execute_round(op, layer, n, sids, wids, toks, adapters, st);
}

}  // namespace

extern "C" int swl_agg_token_boundary(uint64_t* active_lo, uint64_t* active_hi, int* count) {
  SWL_CHECK(g_agg_q.ctrl, SWL_ERR_STATE, "Aggregator queue not initialized");
  SWL_CHECK(active_lo && active_hi && count, SWL_ERR_INVALID, "token_boundary: null argument");
  swl::Control* c = g_agg_q.ctrl;
  Mask active;
  active.w[0] = *active_lo;
  active.w[1] = *active_hi;
  // leaves first, then joins (ext_aggregator.cpp:1053-1084)
  if (!c->leaves.load().empty()) {
    const Mask lv = c->leaves.take();
    active = active & ~lv;
    std::printf("[Aggregator] Slots LEFT: mask=0x%llx:%llx, active: %d slots\n", (unsigned long long)lv.w[1],
                (unsigned long long)lv.w[0], active.count());
    std::fflush(stdout);
  }
  if (!c->joins.load().empty()) {
    const Mask jn = c->joins.take();
    apply_join_sampling(jn);
    active = active | jn;
    std::printf("[Aggregator] Slots JOINED: mask=0x%llx:%llx, active: %d slots\n", (unsigned long long)jn.w[1],
                (unsigned long long)jn.w[0], active.count());
    std::fflush(stdout);
  }
  const int N = active.count();
  c->active.store(active);
  c->active_count.store(N, std::memory_order_release);
  g_pool.active_mask.store(active);
  g_pool.active_slot_count.store(N, std::memory_order_release);
  *active_lo = active.w[0];
  *active_hi = active.w[1];
  *count = N;
  return SWL_OK;
}

extern "C" int swl_agg_main_loop(int num_slots, int dtype_code) {
  SWL_CHECK(g_agg_q.ctrl && g_agg_q.ring, SWL_ERR_STATE, "Aggregator queue not initialized");
  SWL_CHECK(g_weights_ready, SWL_ERR_STATE, "Aggregator weights not initialized");
  SWL_CHECK(g_pool.initialized, SWL_ERR_STATE, "Slot pool not initialized");
  SWL_CHECK(dtype_code == 15, SWL_ERR_UNSUPPORTED, "aggregator_main_loop_slots: only bfloat16 (dtype_code 15)");
  (void)num_slots;
  SWL_HIP(hipSetDevice(g_device));
  hipStream_t st = nullptr;
  int rc = stream_get(&st);
  if (rc) return rc;
  swl::Control* c = g_agg_q.ctrl;
  Mask active;
  long tokens_done = 0, ops_done = 0;
  uint64_t step = 0;
  std::printf("[Aggregator] Starting slot-based main loop on device %d (%d slots)\n", g_device, g_pool.num_slots);
  std::fflush(stdout);
  int32_t sids[SWL_MAX_SLOTS], wids[SWL_MAX_SLOTS], ops[SWL_MAX_SLOTS], layers[SWL_MAX_SLOTS];
  int64_t toks[SWL_MAX_SLOTS];
  uint64_t keys[SWL_MAX_SLOTS], seqs[SWL_MAX_SLOTS];
  int32_t outh[SWL_MAX_SLOTS];
  auto seq_word = [](int sid, size_t off) {
    return reinterpret_cast<uint64_t*>(static_cast<char*>(g_pool.slots[sid].out) + g_pool.out_size + off);
  };
  // SWL_AGG_TIMING=1: per-round host phases (wait for every slot's ready,
  // drain, launch, stream sync) summed and printed when the loop exits
  const bool timing = std::getenv("SWL_AGG_TIMING") && std::atoi(std::getenv("SWL_AGG_TIMING")) != 0;
  using tclk = std::chrono::steady_clock;
  double t_ready = 0, t_drain = 0, t_launch = 0, t_sync = 0;
  long t_rounds = 0;
  auto us_since = [](tclk::time_point a) { return std::chrono::duration<double, std::micro>(tclk::now() - a).count(); };
  while (c->quit.load(std::memory_order_acquire) == 0) {
    int N = 0;
    rc = swl_agg_token_boundary(&active.w[0], &active.w[1], &N);
    if (rc) return rc;
    if (N == 0) {
      std::this_thread::sleep_for(std::chrono::milliseconds(1));
      continue;
    }
    const int ops_per_token = 1 + 4 * g_num_layers + 1;
    for (int op_idx = 0; op_idx < ops_per_token; ++op_idx) {
      int cnt = 0;
      auto tp = tclk::now();
      rc = swl_agg_wait_for_slots(&active.w[0], &active.w[1], &cnt);
      if (rc) return rc;
      if (timing) {
        t_ready += us_since(tp);
        tp = tclk::now();
      }
      if (cnt < 0) {
        swl_agg_signal_done();
        break;
      }
      if (cnt == 0) {
        N = 0;
        break;
      }
      N = cnt;
      if (c->quit.load(std::memory_order_acquire) != 0) break;
      int got = 0;
      rc = drain_impl(active.w[0], active.w[1], N, sids, wids, ops, layers, toks, keys, seqs, outh, &got);
      if (rc) return rc;
      if (timing) {
        t_drain += us_since(tp);
        tp = tclk::now();
      }
      if (got == 0 || c->quit.load(std::memory_order_acquire) != 0) {
        if (c->quit.load(std::memory_order_acquire) != 0) swl_agg_signal_done();
        continue;
      }
      const int op = ops[0];
      if (op != SWL_OP_SET_SAMPLING) {
        // the op of a round is the first command's (every worker runs the same
        // op sequence); commands that disagree are evicted rather than run
        int m = 0;
        for (int i = 0; i < got; ++i) {
          if (ops[i] == op && layers[i] == layers[0]) {
            sids[m] = sids[i]; wids[m] = wids[i]; toks[m] = toks[i]; keys[m] = keys[i]; seqs[m] = seqs[i];
            outh[m] = outh[i];
            ++m;
          } else {
            c->evicted.set_bit(sids[i]);
            active.clear(sids[i]);
          }
        }
        // GPU-ordered commands: the stream waits for each such slot's input
        // sequence word instead of the worker having waited on its host
        const uint64_t* wflag[SWL_MAX_SLOTS];
        uint64_t want[SWL_MAX_SLOTS];
        int32_t wtag[SWL_MAX_SLOTS];
        int nord = 0;
        for (int i = 0; i < m; ++i)
          if (seqs[i] > 0) {
            wflag[nord] = seq_word(sids[i], swl::kInSeqOffset);
            want[nord] = seqs[i];
            wtag[nord] = sids[i];
            ++nord;
          }
        if (nord > 0) {
          rc = swl::seq_wait_launch(nord, wflag, want, wtag, g_pool.seq_timeout, kSeqWaitLimitUs, st);
          if (rc) return rc;
        }
        rc = run_op(op, layers[0], m, sids, wids, toks, keys, st, step++);
        // ... and each ordered slot's output sequence word follows the round
        // on the stream (written even if the round failed, so no worker waits
        // out its limit on an evicted slot)
        {
          uint64_t* oflag[SWL_MAX_SLOTS];
          uint64_t oval[SWL_MAX_SLOTS];
          int nw = 0;
          for (int i = 0; i < m; ++i)
            if (seqs[i] > 0 && !outh[i]) {  // out_host workers read after done: no word to wait on
              oflag[nw] = seq_word(sids[i], swl::kOutSeqOffset);
              oval[nw] = seqs[i];
              ++nw;
            }
          const int wrc = swl::seq_write_launch(nw, oflag, oval, st);
          if (wrc && !rc) rc = wrc;
        }
        if (rc) {
          // a malformed command must not take every co-tenant down: evict the
          // slots of this round and keep serving the others
          std::fprintf(stderr, "[Aggregator] round failed (%s); evicting its %d slot(s)\n",
                       swl::last_error().c_str(), m);
          std::fflush(stderr);
          for (int i = 0; i < m; ++i) {
            c->evicted.set_bit(sids[i]);
            active.clear(sids[i]);
          }
          c->active.store(active);
        }
        // the host waits for the round unless every command is GPU-ordered
        // on both sides (its worker waits for the outputs on its stream)
        bool sync = nord < m;
        for (int i = 0; i < m; ++i) sync = sync || outh[i] != 0;
        if (timing) {
          t_launch += us_since(tp);
          tp = tclk::now();
        }
        if (sync) SWL_HIP(hipStreamSynchronize(st));
        if (timing) {
          t_sync += us_since(tp);
          ++t_rounds;
        }
        int32_t late[SWL_MAX_SLOTS];
        const int nlate = swl_agg_take_seq_timeouts(late, SWL_MAX_SLOTS);
        for (int i = 0; i < nlate && i < SWL_MAX_SLOTS; ++i) {
          std::fprintf(stderr, "[Aggregator] slot %d: GPU-ordered input not written within %u ms; evicting\n",
                       late[i], kSeqWaitLimitUs / 1000);
          c->evicted.set_bit(late[i]);
          active.clear(late[i]);
        }
        if (nlate) {
          std::fflush(stderr);
          c->active.store(active);
        }
      }
      swl_agg_signal_done();
      ++ops_done;
    }
    ++tokens_done;
  }
  if (timing && t_rounds)
    std::printf("[Aggregator] host phases per round (us, %ld rounds): ready wait %.1f, drain %.1f, launch %.1f, "
                "stream sync %.1f\n", t_rounds, t_ready / t_rounds, t_drain / t_rounds, t_launch / t_rounds,
                t_sync / t_rounds);
  std::printf("[Aggregator] Slot-based loop exited after %ld tokens (%ld ops)\n", tokens_done, ops_done);
  std::fflush(stdout);
  return SWL_OK;
}
