/*
 * swl_runtime.h — C ABI of the slot-pool / command-ring / barrier runtime in
 * libswl.so.  These entry points are what the Python modules
 * swarmlora_amd.ext_ipc_queue, .ext_aggregator and .ext_unified_barrier bind
 * (same names, arguments and error texts as the reference's pybind modules
 * src/cpp_extensions/ext_ipc_queue.cpp:413-483, ext_aggregator.cpp:1436-1517
 * and ext_unified_barrier.cpp:562-630).
 *
 * Three independent pieces of process state live behind them, as in the
 * reference's three extension modules:
 *   swl_q_*    the command queue mapping of this process (ext_ipc_queue)
 *   swl_agg_*  the aggregator: slot pool, weights, adapter pool, its own queue
 *              mapping and the main loop (ext_aggregator)
 *   swl_w_*    the worker's slot manager (ext_unified_barrier)
 * All return SWL_OK (0) or an SWL_ERR_* code with swl_last_error() set,
 * unless documented otherwise.
 */
#ifndef SWL_RUNTIME_H
#define SWL_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#include "swl.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ======================================================= command queue ===
 * POSIX shared memory: one control block (slot masks, epoch, ring cursors,
 * per-slot sampling state) followed by `capacity` 128-byte commands.        */

/* create_queue (ext_ipc_queue.cpp:111-145): creates and maps a new segment;
 * its name ("/swlq_<pid>_<ns>") is written to name_out. */
int swl_q_create(int capacity, int max_tickets, char* name_out, int name_cap);
/* open_queue (ext_ipc_queue.cpp:147-176): maps an existing segment. */
int swl_q_open(const char* shm_name, int capacity, int max_tickets);
/* Unmaps this process's queue mapping (and unlinks it if it created it). */
int swl_q_close(void);
/* init_batch_control (ext_ipc_queue.cpp:180-209). */
int swl_q_init_batch_control(int num_slots);
/* set_quit (ext_ipc_queue.cpp:404-410). */
int swl_q_set_quit(int value);
/* slot_set_pending_sampling (ext_ipc_queue.cpp:216-232). */
int swl_q_set_pending_sampling(int slot_id, int do_sample, float temperature, int top_k, float top_p);
/* slot_signal_join / _leave / _ready (ext_ipc_queue.cpp:235-268). */
int swl_q_signal_join(int slot_id);
int swl_q_signal_leave(int slot_id);
int swl_q_signal_ready(int slot_id);
/* wait_for_epoch (ext_ipc_queue.cpp:272-300): spins until the barrier epoch
 * exceeds `expected`; writes the epoch seen.  SWL_ERR_QUIT if the quit flag
 * is raised while waiting. */
int swl_q_wait_for_epoch(int64_t expected, int64_t* epoch_out);
/* slot_is_active / is_slot_evicted return 1 or 0 (never an error). */
int swl_q_slot_is_active(int slot_id);
int swl_q_is_slot_evicted(int slot_id);
/* clear_evicted_slot (ext_ipc_queue.cpp:330-336). */
int swl_q_clear_evicted_slot(int slot_id);
/* get_barrier_done_epoch (ext_ipc_queue.cpp:314-319); 0 if not mapped. */
int64_t swl_q_get_epoch(void);
/* submit_slot_command (ext_ipc_queue.cpp:339-402): validates every field
 * before reserving a ring entry; "command ring buffer FULL" when full. */
int swl_q_submit(int op_type, int layer_idx, int slot_id, int worker_id, int64_t bx, int64_t tx, int64_t dx,
                 uint64_t x_key, uint64_t y0_key, uint64_t y1_key, uint64_t y2_key, int ticket_id);
/* submit_slot_command of a GPU-ordered worker (no counterpart in the
 * reference, whose worker waits for its input copy on the host before
 * submitting, ext_unified_barrier.cpp:262-266): in_seq is the slot's input
 * sequence value the worker's stream writes after the copy
 * (swl_w_input_seq); the aggregator's stream waits for it before the round
 * and writes it to the slot's output sequence word after the round, instead
 * of synchronising its stream before signalling done. */
int swl_q_submit_seq(int op_type, int layer_idx, int slot_id, int worker_id, int64_t bx, int64_t tx, int64_t dx,
                     uint64_t x_key, uint64_t y0_key, uint64_t y1_key, uint64_t y2_key, int ticket_id,
                     uint64_t in_seq);
/* swl_q_submit_seq with out_host (no counterpart in the reference): 1 when
 * the worker reads this round's outputs as soon as done is signalled, with
 * no wait on its stream (swl_w_set_gpu_ordered mode 2); the aggregator then
 * synchronises its stream before signalling done, as for a host-ordered
 * command.  Ignored when in_seq is 0. */
int swl_q_submit_seq_ex(int op_type, int layer_idx, int slot_id, int worker_id, int64_t bx, int64_t tx, int64_t dx,
                        uint64_t x_key, uint64_t y0_key, uint64_t y1_key, uint64_t y2_key, int ticket_id,
                        uint64_t in_seq, int out_host);
/* Layout sizes of the shared segment (for tests). */
size_t swl_q_control_bytes(void);
size_t swl_q_command_bytes(void);

/* =========================================================== aggregator === */

typedef struct swl_pool_status {
  int32_t initialized;
  int32_t num_slots;
  uint64_t free_lo, free_hi;
  uint64_t active_lo, active_hi;
  int32_t active_slot_count;
  int32_t owners[SWL_MAX_SLOTS];
} swl_pool_status;

/* init_slot_pool (ext_aggregator.cpp:138-187): one hipMalloc'd input and output
 * buffer per slot with a hipIpcGetMemHandle each. */
int swl_agg_init_slot_pool(int num_slots, int device_index, int hidden_dim, int intermediate_dim, int num_kv_heads,
                           int head_dim, int max_seq_per_step, int dtype_size, size_t* input_buffer_size,
                           size_t* output_buffer_size);
/* claim_slot (ext_aggregator.cpp:190-245): lock-free claim; writes the slot
 * id, the two 64-byte IPC handles and the buffer sizes.
 * "No free slots available" when the pool is exhausted. */
int swl_agg_claim_slot(int worker_id, int* slot_id, uint8_t* input_handle, uint8_t* output_handle,
                       size_t* input_buffer_size, size_t* output_buffer_size);
/* release_slot (ext_aggregator.cpp:248-292): owner check, synchronous zeroing
 * of both buffers, then back to the free mask. */
int swl_agg_release_slot(int slot_id, int worker_id);
/* get_slot_owner (ext_aggregator.cpp:295-300): owner id or -1. */
int swl_agg_get_slot_owner(int slot_id);
/* get_slot_pool_status (ext_aggregator.cpp:303-328). */
int swl_agg_pool_status(swl_pool_status* out);
/* cleanup_slot_pool (ext_aggregator.cpp:1410-1433). */
int swl_agg_cleanup_slot_pool(void);
/* Device pointers of slot i's buffers (this process; for local execution). */
int swl_agg_slot_buffers(int slot_id, void** input_buffer, void** output_buffer);

/* init_aggregator_begin / _layer / _finalize (ext_aggregator.cpp:338-410):
 * q/k/v and gate/up are copied into fused buffers the library owns; o and
 * down stay the caller's (kept alive by the caller, as the reference shares
 * them by detach()).  Biases may be NULL.  All weights bf16 row-major
 * [out, in]. */
int swl_agg_begin(int num_layers, int device_index);
int swl_agg_set_layer(int layer_idx, const void* q, int64_t q_rows, const void* k, int64_t k_rows, const void* v,
                      int64_t v_rows, const void* o, const void* o_bias, const void* gate, int64_t gate_rows,
                      const void* up, int64_t up_rows, const void* down, const void* down_bias, int64_t hidden_dim,
                      int64_t intermediate_dim);
int swl_agg_finalize(void);
/* init_embed_lm_head_weights (ext_aggregator.cpp:413-424): caller-owned bf16
 * [vocab, hidden] tables. */
int swl_agg_set_embed_lm_head(const void* embed, const void* lm_head, int64_t vocab_size, int64_t hidden_dim);
/* init_aggregator_queue (ext_aggregator.cpp:427-459). */
int swl_agg_attach_queue(const char* shm_name, int capacity);

/* Adapter pool (no counterpart in the reference, whose workers add their own
 * delta): registers adapter `adapter_id`'s weights for one (layer, op) so the
 * round adds its LoRA delta during the scatter.  a: bf16 [nblk*rank, in]
 * (stacked lora_A); b[j]: bf16 [cols_j, rank] (lora_B).  Caller-owned.  A
 * command whose x_key is adapter_id + 1 uses it; x_key == 0 means none. */
int swl_agg_register_adapter(int adapter_id, int layer_idx, int op_type, const void* a, const void* const* b,
                             int nblk, int rank, float scale);
int swl_agg_clear_adapters(void);

/* One batched round over the slot pool: execute_batched_gemm_slots
 * (ext_aggregator.cpp:470-626) for n slots in arrival order, plus the pooled
 * adapters' LoRA delta.  tokens[i] = bx*tx of slot i's command; adapter_ids
 * may be NULL (or hold -1) for no adapter.  Kernels go to `stream` as given
 * (NULL is the device's null stream, ordered with other null-stream work). */
int swl_agg_execute_round(int op_type, int layer_idx, int n, const int32_t* slot_ids, const int32_t* worker_ids,
                          const int64_t* tokens, const int32_t* adapter_ids, void* stream);

/* Barrier primitives of the main loop, exported for host-side tests:
 * aggregator_wait_for_slots (ext_aggregator.cpp:879-978) with the active mask
 * in/out; returns the remaining active count through *count_out (-1 = quit). */
int swl_agg_wait_for_slots(uint64_t* active_lo, uint64_t* active_hi, int* count_out);
/* aggregator_signal_done_slots (ext_aggregator.cpp:981-987). */
int swl_agg_signal_done(void);
/* Ring drain of the main loop (ext_aggregator.cpp:1129-1160): consumes
 * commands until `want` from active slots were read; writes their slot ids,
 * op, layer.  Commands of inactive slots are consumed and dropped. */
int swl_agg_drain_commands(uint64_t active_lo, uint64_t active_hi, int want, int32_t* slot_ids, int32_t* worker_ids,
                           int32_t* ops, int32_t* layers, int64_t* tokens, uint64_t* x_keys, int* got);
/* Eviction and leave-check periods of the barrier (defaults 500 ms, 10 ms). */
int swl_agg_set_barrier_timeouts(int evict_ms, int leave_check_ms);
/* The part of claim_slot that resets a slot's barrier bits for its next
 * owner (ext_aggregator.cpp:223-227): clears the slot's ready and evicted
 * bits in the attached queue, which a killed or evicted previous tenant may
 * have left set.  claim_slot calls it after winning the slot. */
int swl_agg_scrub_slot(int slot_id);
/* Slots whose GPU-ordered input did not arrive within the stream wait's
 * limit (2 s) since the last call: writes up to 128 slot ids, returns the
 * count and clears them (such slots are also evicted by the main loop). */
int swl_agg_take_seq_timeouts(int32_t* slot_ids, int max_ids);
/* The main loop's token boundary (ext_aggregator.cpp:1053-1084): removes the
 * slots that signalled leave from the active set *active_lo/_hi, adds the
 * slots that signalled join (with their pending sampling parameters),
 * publishes the result as the queue's active set and writes it back with its
 * size.  The main loop calls it once per token. */
int swl_agg_token_boundary(uint64_t* active_lo, uint64_t* active_hi, int* count);
/* aggregator_main_loop_slots (ext_aggregator.cpp:1024-1210): blocks until the
 * quit flag is set.  dtype_code 15 (bfloat16) only. */
int swl_agg_main_loop(int num_slots, int dtype_code);

/* ============================================================== worker === */

/* init_worker_slot_manager (ext_unified_barrier.cpp:60-92). */
int swl_w_init(int worker_id, int worker_device, int aggregator_device, int hidden_dim, int intermediate_dim,
               int qkv_dim);
/* open_slot (ext_unified_barrier.cpp:97-160): hipIpcOpenMemHandle of both
 * 64-byte handles. */
int swl_w_open_slot(int slot_id, const uint8_t* input_handle, size_t input_handle_len, const uint8_t* output_handle,
                    size_t output_handle_len, size_t input_buffer_size, size_t output_buffer_size);
/* close_slot (ext_unified_barrier.cpp:163-211): device sync, then close. */
int swl_w_close_slot(int slot_id);
/* prepare_input_slot (ext_unified_barrier.cpp:225-273): copies `bytes` from
 * src (device) into the slot input buffer on `stream` and waits for it;
 * records the [bx, tx, dx] shape. */
int swl_w_prepare_input(int slot_id, const void* src, int64_t bx, int64_t tx, int64_t dx, size_t elem_size,
                        void* stream);
/* Shape recorded by the last prepare_* call on the slot. */
int swl_w_slot_shape(int slot_id, int64_t* bx, int64_t* tx, int64_t* dx);
/* get_outputs_slot / get_embeddings_slot copy (ext_unified_barrier.cpp:
 * 276-347, 396-440): `bytes` from the slot output buffer into dst (device),
 * stream-ordered, no host sync. */
int swl_w_copy_output(int slot_id, void* dst, size_t bytes, void* stream);
/* get_outputs_slot followed by the worker's adds of its *_get_all methods
 * (worker_sync.py:314-319, :383-389: out + lora delta, then residual + that,
 * each rounded to bf16) in one launch: dst = residual + (out + delta) over
 * the first n bf16 elements of the slot output; delta and residual may be
 * null.  Stream-ordered; in GPU-ordered mode 1 it first waits for the
 * output word as swl_w_copy_output does. */
int swl_w_read_output(int slot_id, void* dst, int64_t n, const void* delta, const void* residual, void* stream);
/* swl_w_read_output of [bx, tx, d] followed by the worker's next
 * LlamaRMSNorm (worker_sync.py:1344-1350: the post-attention norm after the
 * O round, the next layer's input norm or the final norm after Down):
 * dst_h = residual + (out + delta), dst_norm = RMSNorm(dst_h) * weight, bit
 * for bit the separate read and norm.  d % 8 == 0, 16-byte aligned.
 * stage_input: the normalised rows are also written into the slot's input
 * buffer as the next round's input (swl_w_submit_staged_input then stands
 * in for that round's prepare_input_slot copy). */
int swl_w_read_output_norm(int slot_id, void* dst_h, void* dst_norm, int64_t bx, int64_t tx, int64_t d,
                           const void* delta, const void* residual, const void* weight, float eps, int stage_input,
                           void* stream);
/* The Gate+Up read (rows of gate | up, 2 inter wide, plus the fused delta)
 * followed by F.silu(gate) * up (worker_sync.py:158, :1397) into rows of
 * inter, bit for bit the separate read and SiLU*up; stage_input as above
 * (the Down round's input). */
int swl_w_read_output_silu(int slot_id, void* dst, int64_t bx, int64_t tx, int64_t inter, const void* delta,
                           int stage_input, void* stream);
/* prepare_input_slot (ext_unified_barrier.cpp:225-273) for rows a fused read
 * already staged in the input buffer: checks the shape against the staged
 * one, records it, and completes as prepare_input_slot does (host sync, or
 * the input sequence word in GPU-ordered mode). */
int swl_w_submit_staged_input(int slot_id, int64_t bx, int64_t tx, int64_t dx, void* stream);
/* The slot's input buffer for the caller to write the next round's
 * [bx, tx, dx] bf16 rows into directly (the worker's attention output, the
 * O round's input), recorded as staged: swl_w_submit_staged_input then
 * completes that round's prepare_input_slot without a copy.  The caller's
 * writes must be on the stream it later passes to the submit. */
int swl_w_stage_input(int slot_id, int64_t bx, int64_t tx, int64_t dx, void** input_buffer);
/* prepare_token_ids_slot (ext_unified_barrier.cpp:350-393): int64 ids. */
int swl_w_prepare_token_ids(int slot_id, const void* src, int64_t bx, int64_t tx, void* stream);
/* prepare_hidden_for_lm_head_slot (ext_unified_barrier.cpp:443-486). */
int swl_w_prepare_hidden_lm(int slot_id, const void* src, int64_t bx, int64_t tx, int64_t dx, size_t elem_size,
                            void* stream);
/* get_next_token_slot (ext_unified_barrier.cpp:489-520): host-synchronous. */
int swl_w_get_next_token(int slot_id, int64_t* token, void* stream);
/* cleanup_worker_slots (ext_unified_barrier.cpp:523-558). */
int swl_w_cleanup(void);
/* Buffer sizes of an open slot (for shape checks in the Python shim). */
int swl_w_slot_sizes(int slot_id, size_t* input_buffer_size, size_t* output_buffer_size);
/* GPU-ordered mode for every slot of this worker (no counterpart in the
 * reference).  enable 1 or 2: prepare_* no longer wait on the host; they
 * write the slot's next input sequence value on the stream after the copy.
 * 1: output reads (copy_output, get_next_token) first wait on the stream for
 * the aggregator's output sequence word to reach the last input value.
 * 2: output reads do not wait (the commands carry out_host, so the
 * aggregator signals done only after its stream has finished the round).
 * 0: the reference's host waits. */
int swl_w_set_gpu_ordered(int enable);
/* The input sequence value of the slot's last prepare_* (0 before any). */
int swl_w_input_seq(int slot_id, uint64_t* seq);

#ifdef __cplusplus
}
#endif

#endif /* SWL_RUNTIME_H */
