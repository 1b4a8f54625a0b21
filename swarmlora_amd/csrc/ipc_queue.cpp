// Command ring + slot barrier in POSIX shared memory (CPU only).
//
// The worker-facing half of the protocol: create/open the segment, slot
// join/leave/ready signalling, epoch waits, eviction flags, sampling state and
// command submission.  Semantics follow src/cpp_extensions/ext_ipc_queue.cpp;
// the segment layout is ipc_layout.h.

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cstring>
#include <string>
#include <thread>

#include "ipc_layout.h"
#include "queue_map.h"
#include "swl_common.h"
#include "swl_runtime.h"

namespace swl {

int QueueMap::create(int capacity, int max_tickets) {
  SWL_CHECK(capacity > 0, SWL_ERR_INVALID, "capacity must be > 0");
  SWL_CHECK(max_tickets > 0, SWL_ERR_INVALID, "max_tickets must be > 0");
  close_map();
  const auto ns = std::chrono::duration_cast<std::chrono::nanoseconds>(
                      std::chrono::steady_clock::now().time_since_epoch())
                      .count();
  std::string nm = "/swlq_" + std::to_string(getpid()) + "_" + std::to_string(ns);
  const size_t sz = segment_bytes(capacity);
  const int fd = shm_open(nm.c_str(), O_CREAT | O_EXCL | O_RDWR, 0600);
  SWL_CHECK(fd >= 0, SWL_ERR_STATE, "shm_open (create) failed");
  if (ftruncate(fd, (off_t)sz) != 0) {
    ::close(fd);
    shm_unlink(nm.c_str());
    return fail(SWL_ERR_STATE, "ftruncate failed for shm");
  }
  void* p = mmap(nullptr, sz, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  ::close(fd);
  if (p == MAP_FAILED) {
    shm_unlink(nm.c_str());
    return fail(SWL_ERR_STATE, "mmap failed for shm");
  }
  std::memset(p, 0, sz);  // fresh segment: all masks empty, ring entries not ready
  base = p;
  bytes = sz;
  name = nm;
  owner = true;
  ctrl = reinterpret_cast<Control*>(p);
  ring = reinterpret_cast<Command*>(reinterpret_cast<char*>(p) + sizeof(Control));
  this->capacity = capacity;
  ctrl->capacity = capacity;
  ctrl->max_tickets = max_tickets;
  ctrl->version = kQueueLayoutVersion;
  std::atomic_thread_fence(std::memory_order_release);
  ctrl->magic = kQueueMagic;
  return SWL_OK;
}

int QueueMap::open(const char* shm_name, int capacity) {
  SWL_CHECK(capacity > 0, SWL_ERR_INVALID, "capacity must be > 0");
  SWL_CHECK(shm_name && shm_name[0], SWL_ERR_INVALID, "shm_name cannot be empty");
  close_map();
  const size_t sz = segment_bytes(capacity);
  const int fd = shm_open(shm_name, O_RDWR, 0600);
  SWL_CHECK(fd >= 0, SWL_ERR_STATE, std::string("Failed to open shared memory: ") + shm_name);
  struct stat st;
  if (fstat(fd, &st) != 0 || (size_t)st.st_size < sz) {
    ::close(fd);
    return fail(SWL_ERR_INVALID, "shared memory segment is smaller than the requested capacity");
  }
  void* p = mmap(nullptr, sz, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  ::close(fd);
  SWL_CHECK(p != MAP_FAILED, SWL_ERR_STATE, "mmap failed for shm (open)");
  Control* c = reinterpret_cast<Control*>(p);
  if (c->magic != kQueueMagic || c->version != kQueueLayoutVersion || c->capacity != capacity) {
    munmap(p, sz);
    return fail(SWL_ERR_INVALID, "shared memory segment has a different layout or capacity");
  }
  base = p;
  bytes = sz;
  name = shm_name;
  owner = false;
  ctrl = c;
  ring = reinterpret_cast<Command*>(reinterpret_cast<char*>(p) + sizeof(Control));
  this->capacity = capacity;
  return SWL_OK;
}

void QueueMap::close_map() {
  if (base) {
    munmap(base, bytes);
    if (owner) shm_unlink(name.c_str());
  }
  base = nullptr;
  ctrl = nullptr;
  ring = nullptr;
  bytes = 0;
  capacity = 0;
  owner = false;
  name.clear();
}

QueueMap g_queue;  // this process's ext_ipc_queue mapping

}  // namespace swl

using swl::g_queue;
using swl::Mask;

namespace {

int check_slot(const char* fn, int slot_id) {
  if (!g_queue.ctrl) return swl::fail(SWL_ERR_STATE, std::string(fn) + ": queue not initialized");
  if (slot_id < 0 || slot_id >= SWL_MAX_SLOTS)
    return swl::fail(SWL_ERR_INVALID, std::string(fn) + ": slot_id out of range (0-" +
                                          std::to_string(SWL_MAX_SLOTS - 1) + ")");
  return SWL_OK;
}

}  // namespace

extern "C" {

int swl_q_create(int capacity, int max_tickets, char* name_out, int name_cap) {
  int rc = g_queue.create(capacity, max_tickets);
  if (rc) return rc;
  SWL_CHECK(name_out && name_cap > (int)g_queue.name.size(), SWL_ERR_INVALID, "name buffer too small");
  std::memcpy(name_out, g_queue.name.c_str(), g_queue.name.size() + 1);
  return SWL_OK;
}

int swl_q_open(const char* shm_name, int capacity, int max_tickets) {
  SWL_CHECK(max_tickets > 0, SWL_ERR_INVALID, "max_tickets must be > 0");
  return g_queue.open(shm_name, capacity);
}

int swl_q_close(void) {
  g_queue.close_map();
  return SWL_OK;
}

int swl_q_init_batch_control(int num_slots) {
  SWL_CHECK(g_queue.ctrl, SWL_ERR_STATE, "init_batch_control: queue not initialized");
  SWL_CHECK(num_slots > 0 && num_slots <= SWL_MAX_SLOTS, SWL_ERR_INVALID,
            "init_batch_control: num_slots must be between 1 and " + std::to_string(SWL_MAX_SLOTS));
  swl::Control* c = g_queue.ctrl;
  c->num_workers = num_slots;
  c->num_slots = num_slots;
  const Mask zero;
  c->active.store(zero, std::memory_order_relaxed);
  c->joins.store(zero, std::memory_order_relaxed);
  c->leaves.store(zero, std::memory_order_relaxed);
  c->ready.store(zero, std::memory_order_relaxed);
  c->evicted.store(zero, std::memory_order_relaxed);
  c->sampling_pending.store(zero, std::memory_order_relaxed);
  c->active_count.store(0, std::memory_order_relaxed);
  c->ready_count.store(0, std::memory_order_relaxed);
  c->epoch.store(0, std::memory_order_release);
  return SWL_OK;
}

int swl_q_set_quit(int value) {
  SWL_CHECK(g_queue.ctrl, SWL_ERR_STATE, "set_quit: queue not initialized");
  g_queue.ctrl->quit.store(value, std::memory_order_release);
  return SWL_OK;
}

int swl_q_set_pending_sampling(int slot_id, int do_sample, float temperature, int top_k, float top_p) {
  int rc = check_slot("slot_set_pending_sampling", slot_id);
  if (rc) return rc;
  swl::SamplingParams& p = g_queue.ctrl->sampling[slot_id];
  p.do_sample = do_sample ? 1 : 0;
  p.temperature = temperature;
  p.top_k = top_k;
  p.top_p = top_p;
  g_queue.ctrl->sampling_pending.set_bit(slot_id, std::memory_order_release);
  return SWL_OK;
}

int swl_q_signal_join(int slot_id) {
  int rc = check_slot("slot_signal_join", slot_id);
  if (rc) return rc;
  g_queue.ctrl->joins.set_bit(slot_id);
  return SWL_OK;
}

int swl_q_signal_leave(int slot_id) {
  int rc = check_slot("slot_signal_leave", slot_id);
  if (rc) return rc;
  g_queue.ctrl->leaves.set_bit(slot_id);
  return SWL_OK;
}

int swl_q_signal_ready(int slot_id) {
  int rc = check_slot("slot_signal_ready", slot_id);
  if (rc) return rc;
  g_queue.ctrl->ready.set_bit(slot_id);
  g_queue.ctrl->ready_count.fetch_add(1, std::memory_order_release);
  return SWL_OK;
}

int swl_q_wait_for_epoch(int64_t expected, int64_t* epoch_out) {
  SWL_CHECK(g_queue.ctrl, SWL_ERR_STATE, "wait_for_epoch: queue not initialized");
  swl::Control* c = g_queue.ctrl;
  int spins = 0;
  while (c->epoch.load(std::memory_order_acquire) <= expected) {
    if (c->quit.load(std::memory_order_acquire) != 0)
      return swl::fail(SWL_ERR_QUIT, "wait_for_epoch: quit flag set");
    ++spins;
    if (spins < swl::kSpinTight) {
    } else if (spins < swl::kSpinPause) {
      swl::cpu_relax();
    } else if (spins < swl::kSpinYield) {
      std::this_thread::yield();
    } else {
      std::this_thread::sleep_for(std::chrono::microseconds(10));
    }
  }
  if (epoch_out) *epoch_out = c->epoch.load(std::memory_order_acquire);
  return SWL_OK;
}

int swl_q_slot_is_active(int slot_id) {
  if (!g_queue.ctrl || slot_id < 0 || slot_id >= SWL_MAX_SLOTS) return 0;
  return g_queue.ctrl->active.test(slot_id) ? 1 : 0;
}

int swl_q_is_slot_evicted(int slot_id) {
  if (!g_queue.ctrl || slot_id < 0 || slot_id >= SWL_MAX_SLOTS) return 0;
  return g_queue.ctrl->evicted.test(slot_id) ? 1 : 0;
}

int swl_q_clear_evicted_slot(int slot_id) {
  if (!g_queue.ctrl || slot_id < 0 || slot_id >= SWL_MAX_SLOTS) return SWL_OK;
  g_queue.ctrl->evicted.clear_bits(Mask::bit(slot_id));
  return SWL_OK;
}

int64_t swl_q_get_epoch(void) {
  if (!g_queue.ctrl) return 0;
  return g_queue.ctrl->epoch.load(std::memory_order_acquire);
}

int swl_q_submit_seq_ex(int op_type, int layer_idx, int slot_id, int worker_id, int64_t bx, int64_t tx, int64_t dx,
                        uint64_t x_key, uint64_t y0_key, uint64_t y1_key, uint64_t y2_key, int ticket_id,
                        uint64_t in_seq, int out_host) {
  SWL_CHECK(g_queue.ctrl && g_queue.ring, SWL_ERR_STATE, "submit_slot_command: queue not initialized");
  // Validate everything before reserving an entry: a reserved entry whose
  // ready flag is never set would stall the aggregator's drain.
  SWL_CHECK(slot_id >= 0 && slot_id < SWL_MAX_SLOTS, SWL_ERR_INVALID,
            "submit_slot_command: slot_id out of range: " + std::to_string(slot_id));
  SWL_CHECK(worker_id >= 0 && worker_id <= 100000, SWL_ERR_INVALID,
            "submit_slot_command: invalid worker_id: " + std::to_string(worker_id));
  SWL_CHECK(bx > 0 && tx > 0 && bx <= 65536 && tx <= 65536, SWL_ERR_INVALID,
            "submit_slot_command: invalid bx/tx: bx=" + std::to_string(bx) + " tx=" + std::to_string(tx));
  swl::Control* c = g_queue.ctrl;
  const int cap = g_queue.capacity;
  int head, next;
  do {
    head = c->head.load(std::memory_order_acquire);
    next = (head + 1) % cap;
    if (next == c->tail.load(std::memory_order_acquire))
      return swl::fail(SWL_ERR_FULL, "command ring buffer FULL");
  } while (!c->head.compare_exchange_weak(head, next, std::memory_order_acq_rel, std::memory_order_acquire));
  swl::Command& cmd = g_queue.ring[head];
  cmd.op_type = op_type;
  cmd.layer_idx = layer_idx;
  cmd.slot_id = slot_id;
  cmd.worker_id = worker_id;
  cmd.ticket_id = ticket_id;
  cmd.bx = bx;
  cmd.tx = tx;
  cmd.dx = dx;
  cmd.x_key = x_key;
  cmd.y0_key = y0_key;
  cmd.y1_key = y1_key;
  cmd.y2_key = y2_key;
  cmd.in_seq = in_seq;
  cmd.out_host = (in_seq > 0 && out_host) ? 1 : 0;
  cmd.ready.store(1, std::memory_order_release);
  return SWL_OK;
}

int swl_q_submit_seq(int op_type, int layer_idx, int slot_id, int worker_id, int64_t bx, int64_t tx, int64_t dx,
                     uint64_t x_key, uint64_t y0_key, uint64_t y1_key, uint64_t y2_key, int ticket_id,
                     uint64_t in_seq) {
  return swl_q_submit_seq_ex(op_type, layer_idx, slot_id, worker_id, bx, tx, dx, x_key, y0_key, y1_key, y2_key,
                             ticket_id, in_seq, 0);
}

int swl_q_submit(int op_type, int layer_idx, int slot_id, int worker_id, int64_t bx, int64_t tx, int64_t dx,
                 uint64_t x_key, uint64_t y0_key, uint64_t y1_key, uint64_t y2_key, int ticket_id) {
  return swl_q_submit_seq_ex(op_type, layer_idx, slot_id, worker_id, bx, tx, dx, x_key, y0_key, y1_key, y2_key,
                             ticket_id, 0, 0);
}

size_t swl_q_control_bytes(void) { return sizeof(swl::Control); }
size_t swl_q_command_bytes(void) { return sizeof(swl::Command); }

}  // extern "C"
