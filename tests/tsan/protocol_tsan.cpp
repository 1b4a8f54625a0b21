// ThreadSanitizer harness of the shared-memory round protocol (no GPU).
//
// Worker threads drive the worker half (swl_q_*: join, submit, ready, epoch
// wait, leave, eviction check, pending sampling parameters) and one thread
// drives the aggregator half the way swl_agg_main_loop does (token boundary:
// leaves, then joins and their sampling parameters, then the active set is
// published; per op: swl_agg_wait_for_slots, swl_agg_drain_commands,
// swl_agg_signal_done).  The build maps the segment once for both halves
// (the aggregator's mapping is bound to this process's worker-side mapping),
// so every shared word is seen at one address and TSan checks each
// cross-role access.  Scenarios: lock-step ops over several tokens, a late
// join, a leave at a token boundary, a slot that goes silent and is evicted,
// a leave in the middle of an op, and ring wrap-around with a 16-entry ring.
//
// Exit status 0 when every protocol invariant held (TSan itself reports
// races on stderr and sets its own exit code).

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "ipc_layout.h"
#include "queue_map.h"
#include "swl.h"
#include "swl_runtime.h"

using swl::Mask;

namespace {

constexpr int kOp = 9;  // any round op code; the harness never launches it
constexpr int kOpsPerToken = 6;
constexpr int kTokens = 12;

std::atomic<int> g_failures{0};

#define EXPECT(cond, ...)                                  \
  do {                                                     \
    if (!(cond)) {                                         \
      std::fprintf(stderr, "protocol_tsan: FAILED %s: ", #cond); \
      std::fprintf(stderr, __VA_ARGS__);                   \
      std::fprintf(stderr, "\n");                          \
      g_failures.fetch_add(1);                             \
    }                                                      \
  } while (0)

struct WorkerPlan {
  int slot;
  int worker_id;
  int join_delay_tokens;  // wait for this many tokens of others before joining
  int leave_after;        // leave at the token boundary after this many tokens (-1: run all)
  int silent_after;       // stop signalling after this many tokens (-1: never)
  int leave_mid_op;       // in its last token, leave instead of signalling op 2
  bool sampling;          // set pending sampling parameters before joining
};

std::atomic<int> g_tokens_started{0};

void worker(const WorkerPlan p, std::atomic<int>* done_tokens) {
  if (p.sampling) swl_q_set_pending_sampling(p.slot, 1, 0.7f, 40, 0.9f);
  while (g_tokens_started.load() < p.join_delay_tokens) std::this_thread::sleep_for(std::chrono::microseconds(200));
  swl_q_signal_join(p.slot);
  const auto t0 = std::chrono::steady_clock::now();
  while (!swl_q_slot_is_active(p.slot)) {
    if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(30)) {
      EXPECT(false, "slot %d never became active", p.slot);
      return;
    }
    std::this_thread::yield();
  }
  const int n_tok = p.leave_after >= 0 ? p.leave_after : kTokens;
  for (int tok = 0; tok < n_tok; ++tok) {
    if (p.silent_after >= 0 && tok == p.silent_after) {
      // stop signalling: the barrier must evict this slot and tell it so
      const auto ts = std::chrono::steady_clock::now();
      while (!swl_q_is_slot_evicted(p.slot)) {
        if (std::chrono::steady_clock::now() - ts > std::chrono::seconds(30)) {
          EXPECT(false, "slot %d was never evicted", p.slot);
          return;
        }
        std::this_thread::sleep_for(std::chrono::milliseconds(1));
      }
      swl_q_clear_evicted_slot(p.slot);
      EXPECT(!swl_q_is_slot_evicted(p.slot), "evicted bit of slot %d not cleared", p.slot);
      return;
    }
    for (int op = 0; op < kOpsPerToken; ++op) {
      if (p.leave_mid_op && tok == n_tok - 1 && op == 2) {
        swl_q_signal_leave(p.slot);
        return;
      }
      const int64_t epoch = swl_q_get_epoch();
      // layer_idx carries (token, op) so the aggregator can check lock-step
      int rc;
      while ((rc = swl_q_submit(kOp, tok * 100 + op, p.slot, p.worker_id, 1, 1, 4096, 0, 0, 0, 0, 0)) ==
             SWL_ERR_FULL)
        std::this_thread::yield();
      EXPECT(rc == SWL_OK, "submit failed on slot %d: %d", p.slot, rc);
      swl_q_signal_ready(p.slot);
      int64_t now = 0;
      rc = swl_q_wait_for_epoch(epoch, &now);
      if (rc == SWL_ERR_QUIT) return;
      EXPECT(rc == SWL_OK && now > epoch, "epoch wait on slot %d", p.slot);
    }
    done_tokens->fetch_add(1);
  }
  swl_q_signal_leave(p.slot);
}

// The aggregator half: what swl_agg_main_loop does around the barrier calls.
void aggregator(swl::Control* c, std::atomic<bool>* stop, int* tokens_run, int* ops_run) {
  Mask active;
  int32_t sids[SWL_MAX_SLOTS], wids[SWL_MAX_SLOTS], ops[SWL_MAX_SLOTS], layers[SWL_MAX_SLOTS];
  int64_t toks[SWL_MAX_SLOTS];
  uint64_t keys[SWL_MAX_SLOTS];
  while (!stop->load()) {
    if (!c->leaves.load().empty()) active = active & ~c->leaves.take();
    if (!c->joins.load().empty()) {
      const Mask jn = c->joins.take();
      const Mask todo = c->sampling_pending.load() & jn;
      Mask rem = todo;
      while (!rem.empty()) {
        const int sid = rem.first();
        rem.clear(sid);
        const swl::SamplingParams sp = c->sampling[sid];
        EXPECT(sp.do_sample == 1 && sp.top_k == 40, "sampling parameters of slot %d", sid);
      }
      c->sampling_pending.clear_bits(todo);
      active = active | jn;
    }
    const int N = active.count();
    c->active.store(active);
    c->active_count.store(N, std::memory_order_release);
    if (N == 0) {
      std::this_thread::sleep_for(std::chrono::microseconds(200));
      continue;
    }
    g_tokens_started.fetch_add(1);
    ++*tokens_run;
    for (int op = 0; op < kOpsPerToken; ++op) {
      int cnt = 0;
      EXPECT(swl_agg_wait_for_slots(&active.w[0], &active.w[1], &cnt) == SWL_OK, "wait_for_slots");
      if (cnt < 0) {
        swl_agg_signal_done();
        return;
      }
      if (cnt == 0) break;
      int got = 0;
      EXPECT(swl_agg_drain_commands(active.w[0], active.w[1], cnt, sids, wids, ops, layers, toks, keys, &got) ==
                 SWL_OK,
             "drain");
      EXPECT(got == cnt, "op drained %d commands for %d ready slots", got, cnt);
      for (int i = 0; i < got; ++i) {
        EXPECT(active.test(sids[i]), "command of inactive slot %d", sids[i]);
        EXPECT(ops[i] == kOp && toks[i] == 1, "command fields of slot %d", sids[i]);
        // every slot is at the same op of its own token (late joiners count
        // their tokens from their join)
        EXPECT(layers[i] % 100 == op, "slot %d sent op %d during op %d", sids[i], layers[i] % 100, op);
      }
      swl_agg_signal_done();
      ++*ops_run;
    }
  }
}

int run_scenario(const char* name, int ring_capacity, const std::vector<WorkerPlan>& plans) {
  g_tokens_started.store(0);
  char shm[256];
  if (swl_q_create(ring_capacity, ring_capacity, shm, sizeof shm) != SWL_OK) {
    std::fprintf(stderr, "protocol_tsan: swl_q_create failed: %s\n", swl_last_error());
    return 1;
  }
  swl_q_init_batch_control(SWL_MAX_SLOTS);
  // no swl_agg_attach_queue: this build binds the aggregator's mapping to
  // the one swl_q_create just made
  swl_agg_set_barrier_timeouts(400, 2);
  swl::Control* c = swl::g_queue.ctrl;
  std::atomic<bool> stop{false};
  int tokens_run = 0, ops_run = 0;
  std::thread agg(aggregator, c, &stop, &tokens_run, &ops_run);
  std::vector<std::atomic<int>> done(plans.size());
  std::vector<std::thread> ws;
  for (size_t i = 0; i < plans.size(); ++i) ws.emplace_back(worker, plans[i], &done[i]);
  for (auto& t : ws) t.join();
  // every worker has left or been evicted: let the aggregator see it, then stop
  const auto t0 = std::chrono::steady_clock::now();
  while (c->active_count.load() != 0 && std::chrono::steady_clock::now() - t0 < std::chrono::seconds(10))
    std::this_thread::sleep_for(std::chrono::milliseconds(1));
  EXPECT(c->active_count.load() == 0, "%s: slots still active at the end", name);
  stop.store(true);
  swl_q_set_quit(1);
  agg.join();
  for (size_t i = 0; i < plans.size(); ++i) {
    const WorkerPlan& p = plans[i];
    const int want = p.silent_after >= 0 ? p.silent_after
                     : p.leave_mid_op    ? p.leave_after - 1
                     : p.leave_after >= 0 ? p.leave_after
                                          : kTokens;
    EXPECT(done[i].load() == want, "%s: slot %d finished %d tokens, expected %d", name, p.slot, done[i].load(),
           want);
  }
  std::printf("protocol_tsan: %s: %d tokens, %d ops through the barrier\n", name, tokens_run, ops_run);
  swl_q_close();
  return 0;
}

}  // namespace

int main() {
  // lock-step with a late join, a leave at a token boundary, a silent slot
  // that is evicted and a leave in the middle of an op
  std::vector<WorkerPlan> churn = {
      {0, 10, 0, -1, -1, 0, true},  {1, 11, 0, -1, -1, 0, false}, {2, 12, 0, 4, -1, 0, false},
      {3, 13, 0, -1, 3, 0, false},  {5, 15, 2, -1, -1, 0, true},  {7, 17, 0, 6, -1, 1, false},
      {9, 19, 0, -1, -1, 0, false}, {64, 20, 1, -1, -1, 0, false}};
  if (run_scenario("churn", 64, churn)) return 1;
  // twelve commands per op through a 16-entry ring: it wraps nearly every op
  std::vector<WorkerPlan> wrap;
  for (int s = 0; s < 12; ++s) wrap.push_back({s * 9 % 128, 30 + s, 0, -1, -1, 0, false});
  if (run_scenario("ring-wrap", 16, wrap)) return 1;
  const int f = g_failures.load();
  if (f) {
    std::fprintf(stderr, "protocol_tsan: %d invariant failures\n", f);
    return 2;
  }
  std::printf("protocol_tsan: all invariants held\n");
  return 0;
}
