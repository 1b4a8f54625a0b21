// Shared-memory layout of the command queue and slot barrier.  Every process
// that maps the segment (aggregator, workers) must be built from this header.
#pragma once

#include <atomic>
#include <cstddef>
#include <cstdint>

#include "swl.h"

namespace swl {

constexpr uint32_t kQueueMagic = 0x53574C51u;  // "SWLQ"
// 3: commands carry out_host (a process of an earlier layout would ignore
// it, so a worker reading its outputs without a GPU wait could meet an
// aggregator that does not finish the round first); attaching checks it
constexpr uint32_t kQueueLayoutVersion = 3;
constexpr int kSlotWords = SWL_MAX_SLOTS / 64;

// 128-bit slot set held in registers.
struct Mask {
  uint64_t w[kSlotWords] = {0, 0};
  bool test(int i) const { return (w[i >> 6] >> (i & 63)) & 1u; }
  void set(int i) { w[i >> 6] |= 1ull << (i & 63); }
  void clear(int i) { w[i >> 6] &= ~(1ull << (i & 63)); }
  bool empty() const { return (w[0] | w[1]) == 0; }
  int count() const { return __builtin_popcountll(w[0]) + __builtin_popcountll(w[1]); }
  int first() const {
    if (w[0]) return __builtin_ctzll(w[0]);
    if (w[1]) return 64 + __builtin_ctzll(w[1]);
    return -1;
  }
  Mask operator&(const Mask& o) const { return Mask{{w[0] & o.w[0], w[1] & o.w[1]}}; }
  Mask operator|(const Mask& o) const { return Mask{{w[0] | o.w[0], w[1] | o.w[1]}}; }
  Mask operator~() const { return Mask{{~w[0], ~w[1]}}; }
  static Mask below(int n) {
    Mask m;
    for (int i = 0; i < n && i < SWL_MAX_SLOTS; ++i) m.set(i);
    return m;
  }
  static Mask bit(int i) {
    Mask m;
    m.set(i);
    return m;
  }
};

// 128-bit slot set in shared memory.  Every update touches one bit or is a
// whole-set exchange, so per-word atomics suffice.
struct AtomicMask {
  std::atomic<uint64_t> w[kSlotWords];
  Mask load(std::memory_order o = std::memory_order_acquire) const {
    return Mask{{w[0].load(o), w[1].load(o)}};
  }
  void store(const Mask& m, std::memory_order o = std::memory_order_release) {
    w[0].store(m.w[0], o);
    w[1].store(m.w[1], o);
  }
  Mask take(std::memory_order o = std::memory_order_acq_rel) {
    return Mask{{w[0].exchange(0, o), w[1].exchange(0, o)}};
  }
  void set_bit(int i, std::memory_order o = std::memory_order_release) {
    w[i >> 6].fetch_or(1ull << (i & 63), o);
  }
  void clear_bits(const Mask& m, std::memory_order o = std::memory_order_release) {
    w[0].fetch_and(~m.w[0], o);
    w[1].fetch_and(~m.w[1], o);
  }
  bool test(int i, std::memory_order o = std::memory_order_acquire) const {
    return (w[i >> 6].load(o) >> (i & 63)) & 1u;
  }
};

struct SamplingParams {
  int32_t do_sample;
  float temperature;
  int32_t top_k;
  float top_p;
};

// One ring entry.  `ready` is written last with release ordering.
struct alignas(64) Command {
  std::atomic<int32_t> ready;
  int32_t op_type;
  int32_t layer_idx;
  int32_t slot_id;
  int32_t worker_id;
  int32_t ticket_id;
  int64_t bx, tx, dx;
  uint64_t x_key, y0_key, y1_key, y2_key;
  uint64_t in_seq;  // > 0: GPU-ordered command (the slot's input sequence word reaches this value)
  // 1 (GPU-ordered command only): the worker reads the round's outputs once
  // done is signalled, without a GPU wait, so the aggregator synchronises its
  // stream before signalling
  int32_t out_host;
};

// Control block at offset 0 of the segment; the ring follows it.  Producer
// and consumer cursors and the epoch sit on their own cache lines.
struct alignas(64) Control {
  uint32_t magic;
  uint32_t version;
  int32_t capacity;
  int32_t max_tickets;
  int32_t num_slots;
  int32_t num_workers;
  alignas(64) std::atomic<int32_t> head;
  alignas(64) std::atomic<int32_t> tail;
  alignas(64) std::atomic<int32_t> quit;
  alignas(64) AtomicMask active;           // slots in the current token's barrier
  AtomicMask joins;                        // slots asking to join at the next token
  AtomicMask leaves;                       // slots asking to leave
  AtomicMask ready;                        // slot i signalled ready for this op
  AtomicMask evicted;                      // slot i evicted by the barrier timeout
  AtomicMask sampling_pending;             // slot i has new sampling parameters
  std::atomic<int32_t> active_count;
  std::atomic<int32_t> ready_count;
  alignas(64) std::atomic<int64_t> epoch;  // ops completed
  alignas(64) SamplingParams sampling[SWL_MAX_SLOTS];
};

static_assert(sizeof(Command) == 128, "command layout");
static_assert(sizeof(Control) % 64 == 0, "control block keeps the ring 64-byte aligned");

inline size_t segment_bytes(int capacity) { return sizeof(Control) + (size_t)capacity * sizeof(Command); }

// Spin schedule shared by all waits: tight spins, then pause, then yield.
constexpr int kSpinTight = 64;
constexpr int kSpinPause = 1024;
constexpr int kSpinYield = 10000;

inline void cpu_relax() {
#if defined(__x86_64__)
  __builtin_ia32_pause();
#endif
}

}  // namespace swl
