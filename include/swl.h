/*
 * swl.h — C ABI of libswl.so, the MI355X (gfx950) implementation of SwarmLoRA's
 * per-layer gather -> base-GEMM -> scatter rounds, the LoRA delta, the paged-KV
 * decode attention, and the slot-pool / command-ring runtime around them.
 *
 * Conventions
 *   - Every entry point returns an int status (SWL_OK == 0).  On failure the
 *     thread-local message behind swl_last_error() holds the text; the Python
 *     shims raise RuntimeError(text), which is what the reference's pybind
 *     modules do with the std::runtime_error they throw.
 *   - Tensors are plain device pointers to row-major bf16 (or int32/int64)
 *     arrays; sizes are int64 element counts.  `stream` is a hipStream_t passed
 *     as void* (NULL = the null stream).  No torch types cross this boundary.
 *   - Kernels are stream-ordered and never synchronise the host unless the
 *     comment says so.
 *   - Rounds, GEMMs, the segmented LoRA delta and paged attention use one
 *     library-owned scratch area per device (K-slice partials, shrink rows,
 *     attention part records, packed prefill rows): calls that use it must
 *     not overlap on one device, so callers on several streams of a device
 *     order them.  The area grows (hipMalloc) outside graph capture only;
 *     run a call once before capturing it.  Outgrown areas stay allocated
 *     until the process ends, so earlier captured graphs stay valid.
 *
 * Reference citations are relative to SHUs-Lab/SwarmLoRA's tree.
 */
#ifndef SWL_H
#define SWL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status */
enum {
  SWL_OK = 0,
  SWL_ERR_INVALID = 1,   /* bad argument / shape / range                      */
  SWL_ERR_HIP = 2,       /* a HIP runtime call failed ("CUDA error: ..." text)  */
  SWL_ERR_STATE = 3,     /* not initialised / wrong order of calls             */
  SWL_ERR_FULL = 4,      /* ring buffer full                                   */
  SWL_ERR_QUIT = 5,      /* quit flag observed                                 */
  SWL_ERR_NOT_FOUND = 6, /* slot not open / no free slot                       */
  SWL_ERR_UNSUPPORTED = 7,
  SWL_ERR_TIMEOUT = 8    /* a bounded device-side wait gave up                 */
};

/* Constants shared with the reference's ABI (src/cpp_extensions/common/ipc_types.h:16-25). */
#define SWL_MAX_SLOTS 128
#define SWL_OP_O_PROJ 3
#define SWL_OP_DOWN_PROJ 6
#define SWL_OP_QKV_FUSED 9
#define SWL_OP_GATE_UP_FUSED 10
#define SWL_OP_EMBED 11
#define SWL_OP_LM_HEAD 12
#define SWL_OP_SET_SAMPLING 13
#define SWL_IPC_HANDLE_BYTES 64
#define SWL_MAX_LORA_BLOCKS 4

/* Thread-local text of the last failure on the calling thread. */
const char* swl_last_error(void);
/* ABI version of this library (bumped on any signature/layout change;
 * 2: swl_round_fusion ends with a_layout, the chain and deferred-QKV entry
 * points are gone, swl_lora_rows_bf16 added).  A binding checks it against
 * SWL_ABI_VERSION of the header it was written from. */
#define SWL_ABI_VERSION 2
int swl_abi_version(void);
/* Number of HIP devices visible (0 on a host without a GPU); never faults. */
int swl_device_count(void);

/* ============================================================ kernels ====
 * Stateless, stream-ordered device entry points.  These are the compute path
 * the runtime entry points below and the Python worker classes call.
 */

/* Slot gather: packed[off_i + j, :] = slot_in[i][j, :] for j < rows[i], where
 * off = exclusive prefix sum of rows in the given (ring-arrival) order.
 * Replaces torch::cat of from_blob slot views, ext_aggregator.cpp:545-551.
 * slot_in / rows are HOST arrays of n (<= 128) entries; d in elements. */
int swl_gather_bf16(const void* const* slot_in, const int64_t* rows, int n,
                    int64_t d, void* packed, void* stream);

/* Slot scatter (+ optional delta add): slot_out[i][j, :] = y[off_i + j, :]
 * (+ delta[off_i + j, :], added in fp32 and rounded once to bf16).
 * Replaces the per-slot narrow().copy_() of ext_aggregator.cpp:564-570 and the
 * worker's `q + q_delta` adds of src/worker/worker_sync.py:276-284.
 * delta may be NULL.  Host arrays as for swl_gather_bf16. */
int swl_scatter_add_bf16(const void* y, const void* delta, void* const* slot_out,
                         const int64_t* rows, int n, int64_t d_out, void* stream);

/* Base projection y[m, n] = x[m, k] . w[n, k]^T (+ bias[n]); bf16 in/out,
 * fp32 accumulation, one rounding.  m <= 64 runs the skinny MFMA streaming
 * kernel, larger m the LDS-tiled MFMA kernel.  Replaces
 * torch::matmul_out(out, x, W.t()) (+ out.add_(bias)), ext_aggregator.cpp:562,
 * :576-580, :598, :612-616 and the N==1 fast path :506-522.  bias may be NULL.
 * Requires k % 32 == 0. */
int swl_gemm_bf16(const void* x, const void* w, const void* bias, void* y,
                  int64_t m, int64_t n, int64_t k, void* stream);

/* One adapter's weights for one (fused) projection, as the segmented LoRA
 * kernels read them.  `a` stacks the lora_A matrices of the column blocks:
 * bf16 [nblk * rank, k] (PEFT lora_A.weight layout [r, in] per block, block j
 * at rows j*rank..).  b[j] is block j's lora_B.weight, bf16 [blk_cols[j], rank].
 * delta = scale * (x . a_j^T) . b_j^T, i.e. PEFT's lora_B(lora_A(x)) * scaling
 * (src/worker/worker_sync.py:305, :375) and FusedLoRA's
 * (x @ cat(A_i^T * s)) @ blockdiag(B_i^T) (src/worker/model_builder.py:232-262). */
typedef struct swl_lora_entry {
  const void* a;
  const void* b[SWL_MAX_LORA_BLOCKS];
  int32_t rank;
  float scale;
} swl_lora_entry;

/* The fused round: gather -> base GEMM -> (+ per-segment LoRA delta) ->
 * (+ bias) -> scatter, for n_seg (<= 128) slots in arrival order.
 *   seg_in[i]  : device [rows[i], k] bf16 (slot input buffer)
 *   seg_out[i] : device [rows[i], n] bf16 (slot output buffer)
 *   seg_lora   : HOST [n_seg] index into lora_table (-1 = no adapter); NULL =
 *                no LoRA at all (the reference's aggregator-only behaviour)
 *   lora_table : DEVICE array of swl_lora_entry (read by the kernels)
 *   lora_table_host : the same records in HOST memory (read by the launcher to
 *                plan the shrink; no device-to-host copy, so the call can be
 *                captured into a HIP graph)
 *   nblk / blk_cols : column blocks of the fused output (QKV: 3 blocks
 *                {q, k, v}; Gate+Up: 2; O / Down: 1); sum(blk_cols) == n.
 * Equivalent to execute_batched_gemm_slots (ext_aggregator.cpp:470-626)
 * followed by the worker-side delta add (worker_sync.py:270-389) without the
 * bf16 rounding of the delta.  Scratch memory is owned by the library. */
int swl_round_bf16(int n_seg, const int64_t* rows, const void* const* seg_in,
                   void* const* seg_out, const void* w, const void* bias,
                   int64_t n, int64_t k, const int32_t* seg_lora,
                   const swl_lora_entry* lora_table,
                   const swl_lora_entry* lora_table_host, int nblk,
                   const int64_t* blk_cols, void* stream);

/* Optional fusions of a decode-shaped round (<= 64 token rows) with the
 * worker-side elementwise work on either side of it, for the in-process
 * batched decode step.  No counterpart in the reference: its worker runs this
 * work between rounds (worker_sync.py:158, :169-205, :314-319, :383-389,
 * :1344-1350, :1397); the results are the same up to fp32 summation order.
 *
 * Input side (norm_weight != NULL): the rows given as seg_in hold the residual
 * stream h [k]; the round multiplies LlamaRMSNorm(h) = bf16(bf16(h * r) * w),
 * r = rsqrt(sum(ss_in[t][0 .. ss_in_n)) / k + eps), instead of h.  ss_in
 * [ntok][ss_in_stride] fp32 holds partial sums of squares of each row, as an
 * out_mode 1 round writes them.
 *
 * Output side (out_mode):
 *   0  plain: seg_out rows get the round output.
 *   1  residual: seg_out rows hold h [n]; h = bf16(h + out), and the partial
 *      sums of squares of the new row go to ss_out [ntok][ss_out_stride]
 *      (ceil(n / 256) of them: ss_out_stride must be at least that).
 *   2  SiLU-mul: n = 2 * inter (gate | up); seg_out rows [inter] get
 *      bf16(bf16(silu(gate)) * up).
 *   3  RoPE + KV append (decode, one token per sequence; token t is sequence
 *      t): n = (hq + 2 * hkv) * 128; q columns of seg_out rows get the rotated
 *      q, the rotated k and the v of token t are written to its page slot
 *      (position cache_seqlens[t]) in k_cache / v_cache [num_blocks,
 *      block_size, hkv, 128] through block_table [ntok, max_blocks]; RoPE
 *      (NeoX halves) at positions[t] from cos_sin [max_pos, 128]. */
typedef struct swl_round_fusion {
  const void* norm_weight;
  float eps;
  const float* ss_in;
  int32_t ss_in_n, ss_in_stride;
  int32_t out_mode;
  float* ss_out;
  int32_t ss_out_stride;
  void* k_cache;
  void* v_cache;
  int32_t hq, hkv, block_size;
  const int32_t* block_table;
  int64_t max_blocks, num_blocks;
  const int32_t* cache_seqlens;
  const int64_t* positions;
  const void* cos_sin;
  int64_t max_pos;
  /* w_layout 1: w is in the fragment-tile layout of swl_pack_weight_bf16
   * (decode-shaped rounds only); 0: row-major [n, k].  2: the whole-K round
   * over the same fragment tiles (one launch, no partial sums; out_mode 0
   * with or without norm_weight, at most 32 token rows, k a multiple of 256
   * up to 4096, n a multiple of 16): the decode step's LM head, where it
   * beats the K-sliced round (one 1 GB weight); on the projection rounds it
   * is slower.  The round's LoRA shrink runs as a small kernel just before
   * it; neither uses cross-workgroup counters. */
  int32_t w_layout;
  /* a_layout 1: the stacked lora_A of every adapter entry the round uses is
   * in the fragment-tile layout of swl_pack_weight_bf16 (its nblk * rank rows
   * padded to 16 with zeros), streamed like the weight tiles; 0: row-major
   * [nblk * rank, k].  Decode-shaped rounds with w_layout 0 or 1 only. */
  int32_t a_layout;
} swl_round_fusion;

/* Segmented LoRA delta of a packed batch x [T, k] (segment i = rows
 * sum(seg_rows[0..i)) .. + seg_rows[i]), replacing the worker-side delta
 * products of FusedLoRA / SyncRemoteLoRALinear (model_builder.py:193-201,
 * :217-262; worker_sync.py:305, :375) for callers that keep the base GEMM
 * and the delta apart.  For a segment with seg_lora[i] >= 0 (an entry of
 * lora_table), delta = scale * (x . A^T) . B^T over the entry's nblk column
 * blocks (blk_cols, summing to n); fp32 throughout, one bf16 rounding.
 * mode 0: y [T, n] = delta (0 for segments without an adapter); mode 1:
 * y = y + delta in place (segments without an adapter untouched).  k a
 * multiple of 32, x 16-byte aligned, T <= 65535. */
int swl_lora_segmented_bf16(const void* x, int64_t k, int n_seg,
                            const int64_t* seg_rows, const int32_t* seg_lora,
                            const swl_lora_entry* lora_table,
                            const swl_lora_entry* lora_table_host, int nblk,
                            const int64_t* blk_cols, void* y, int64_t n,
                            int mode, void* stream);

/* Fragment-tile layout of a row-major weight w [n, k] (k a multiple of 32)
 * for decode-shaped rounds: 16-row tiles, each tile stored whole (16 x k),
 * k-step by k-step (32 columns); one k-step block is the 1 KiB A operand of a
 * 16x16x32 bf16 MFMA for those rows (lane l: row l % 16, columns
 * 8 (l / 16) .. + 7), so a wave streams each block with one fully coalesced
 * 16-byte load per lane.  Rows past n are zero.  out holds
 * ceil(n / 16) * 16 * k elements (16-byte aligned).  No counterpart in the
 * reference (its weights stay row-major torch tensors, ext_aggregator.cpp:
 * 347-376); the round results are bit-identical to the row-major ones. */
int swl_pack_weight_bf16(const void* w, int64_t n, int64_t k, void* out,
                         void* stream);

/* swl_round_bf16 with fusions (fusion may be NULL; a non-NULL fusion needs
 * at most 64 token rows). */
int swl_round_ex_bf16(int n_seg, const int64_t* rows, const void* const* seg_in,
                      void* const* seg_out, const void* w, const void* bias,
                      int64_t n, int64_t k, const int32_t* seg_lora,
                      const swl_lora_entry* lora_table,
                      const swl_lora_entry* lora_table_host, int nblk,
                      const int64_t* blk_cols, const swl_round_fusion* fusion,
                      void* stream);

/* Allocation-free variant of swl_round_ex_bf16.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops and harnesses that forbid hipMalloc).
 * Same arguments and results as swl_round_ex_bf16 (the same kernels run), for
 * rounds of at most 64 token rows; the K-slice partials live in a 64 MiB
 * device array of the library (one copy per GPU, held until the process
 * ends) instead of the growable library scratch, and the call allocates and
 * frees nothing.  A round whose partials need more than 64 MiB is refused
 * with an error (every 8B-shaped projection round fits at 64 token rows,
 * the 128256-wide LM head up to 32).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other streams, other threads) race and must be ordered by the
 * caller. */
int swl_round_ex_noalloc_bf16(int n_seg, const int64_t* rows, const void* const* seg_in,
                              void* const* seg_out, const void* w, const void* bias,
                              int64_t n, int64_t k, const int32_t* seg_lora,
                              const swl_lora_entry* lora_table,
                              const swl_lora_entry* lora_table_host, int nblk,
                              const int64_t* blk_cols, const swl_round_fusion* fusion,
                              void* stream);

/* Row-major matrix product with an explicit layout, used by the worker-side
 * LoRA modules: y[m, n] = alpha * x[m, k] . B where B is b[k, n] (trans_b = 0,
 * ldb = row stride of b) or b[n, k]^T (trans_b = 1).  fp32 accumulation,
 * bf16 output rounded once (the rounding torch's bf16 matmul performs).
 * Replaces the bf16 nn.Linear / `@` products of model_builder.py:261 and
 * worker_sync.py:305, :375. */
int swl_matmul_bf16(const void* x, int64_t ldx, const void* b, int64_t ldb,
                    int trans_b, void* y, int64_t ldy, int64_t m, int64_t n,
                    int64_t k, float alpha, void* stream);

/* A worker's LoRA delta of up to 4 token rows in one launch: the two bf16
 * products of FusedLoRA.forward (u = x . fused_A, then u . fused_B over its
 * diagonal blocks, model_builder.py:259-262) or of SyncRemoteLoRALinear
 * (lora_B(lora_A(x)) * scaling, worker_sync.py:305, :375).
 *   u[m, j] = bf16(sum_k x[m, k] * a[k*a_sk + j*a_sj]),  j < nr (<= 64)
 *   y[m, c] = bf16(alpha * sum_{rr < rank} u[m, blk*rank + rr] *
 *                  b[blk][rr*b_srr[blk] + (c - off_blk)*b_sc[blk]])
 * for the nblk (<= 4) column blocks of blk_cols[blk] columns each, laid out
 * one after another in y's rows (off_blk = sum of the earlier blocks).
 * x rows 16-byte aligned, k a multiple of 8.  fused_A [k, n*r] is a_sk = n*r,
 * a_sj = 1; lora_A [r, k] is a_sk = 1, a_sj = k; a diagonal block of fused_B
 * [n*r, sum(out)] is b = &fused_B[blk*r, off_blk], b_srr = sum(out), b_sc =
 * 1; lora_B [out, r] is b_srr = 1, b_sc = r. */
int swl_lora_rows_bf16(const void* x, int64_t ldx, int64_t m, int64_t k,
                       const void* a, int64_t a_sk, int64_t a_sj, int64_t nr,
                       int nblk, int64_t rank, const void* const* b,
                       const int64_t* b_srr, const int64_t* b_sc,
                       const int64_t* blk_cols, float alpha, void* y,
                       int64_t ldy, void* stream);

/* Paged-KV attention for one q_len group, replacing
 * WorkerBatchedOps.batch_flash_attention (worker_sync.py:169-205).  Token t
 * (t = seq * q_len + i) has its query heads at q + t*q_stride ([hq, d]), its
 * new key heads at k + t*k_stride and value heads at v + t*v_stride ([hkv, d]);
 * strides are in elements, so q/k/v can be read in place from the fused QKV
 * output rows ([q | k | v], stride hq*d + 2*hkv*d).
 *   1. NeoX RoPE in place on the q and k heads at positions[nseq * q_len]
 *      using cos_sin [max_pos, d] (cos | sin halves, the cache of
 *      paged_attention.py:131-142), when rope != 0;
 *   2. append k and v into the pages k_cache / v_cache
 *      [num_blocks, block_size, hkv, d] at cache_seqlens[s] + i through
 *      block_table [nseq, max_blocks] (int32);
 *   3. causal GQA attention of each query over cache_seqlens[s] + i + 1 keys,
 *      scale softmax_scale, written to out [nseq, q_len, hq * d].
 * d must be 128; hq % hkv == 0; q_len <= 1024. */
int swl_paged_attention_bf16(void* q, void* k, const void* v, int64_t q_stride,
                             int64_t k_stride, int64_t v_stride, int nseq, int q_len,
                             int hq, int hkv, int d, void* k_cache, void* v_cache,
                             int64_t num_blocks, int block_size,
                             const int32_t* block_table, int64_t max_blocks,
                             const int32_t* cache_seqlens, const int64_t* positions,
                             const void* cos_sin, int64_t max_pos, int rope,
                             float softmax_scale, void* out, void* stream);

/* Zero whole KV pages: cache[block_ids[i], ...] = 0 for i < nblocks, for each
 * of the ncache caches in `caches` (HOST array of device pointers; block_ids
 * is a device int64 array, each id < the cache's block count).
 * Replaces index_fill_(0, blocks, 0) per layer, paged_attention.py:77-89. */
int swl_zero_blocks_bf16(void* const* caches, int ncache, const int64_t* block_ids,
                         int64_t nblocks, int64_t block_elems, void* stream);

/* Embedding lookup for n segments of int64 token ids: out[i][j, :] =
 * table[clamp(ids[i][j], 0, vocab - 1), :].  ids / rows / out are HOST arrays
 * of device pointers / counts.  Replaces torch::embedding of clamped ids,
 * ext_aggregator.cpp:660-705. */
int swl_embed_bf16(const void* const* ids, const int64_t* rows, int n, const void* table, int64_t vocab,
                   int64_t hidden, void* const* out, void* stream);

/* Next token per logits row (logits bf16 [n, vocab], n <= 128): argmax (first
 * index of the maximum) when do_sample[i] == 0, otherwise temperature, top-k,
 * top-p and a multinomial draw from a counter-based generator seeded by
 * (seed, row).  out_tok[i] is a device int64 (the slot output buffer).
 * Replaces the sampling block of ext_aggregator.cpp:756-795 / :818-874.
 * Sampled tokens follow the same distribution as the reference, not its
 * random stream. */
int swl_sample_bf16(const void* logits, int64_t n, int64_t vocab, void* const* out_tok, const int32_t* do_sample,
                    const float* temperature, const int32_t* top_k, const float* top_p, uint64_t seed,
                    void* stream);

/* ------------------------------------------------------ launch timer ----
 * Benchmark instrumentation (no counterpart in the reference).  After
 * swl_timer_arm(capacity), each decode-shaped projection (a round or gemm of
 * at most 64 token rows) launched outside graph capture launches its base
 * kernel and its epilogue kernel with start/stop HIP events that take the
 * dispatches' own begin/end timestamps (hipExtLaunchKernelGGL), for up to
 * `capacity` launches.  swl_timer_collect waits for them, disarms, and returns per
 * launch: base/epilogue milliseconds, N, K, token rows and the base kernel's
 * algorithmic bytes (W + token rows + distinct stacked LoRA A).
 * Single-threaded use only. */
int swl_timer_arm(int capacity);
int swl_timer_collect(int max_records, float* base_ms, float* epilogue_ms, int64_t* n, int64_t* k, int32_t* ntok,
                      int64_t* bytes, int* count);

/* ----------------------------------------------- worker-side row ops ----
 * Token-row variants of the worker's per-layer elementwise work, so the
 * batched decode step reads and writes slot buffers directly (at most 64
 * rows; row arrays are HOST arrays of device pointers). */

/* Residual stream h [ntok, d] (contiguous): when add_rows is given,
 * h[t] = bf16(h[t] + add_rows[t]) (the worker's `residual + result`,
 * worker_sync.py:314-319, :383-389); then out_rows[t] = LlamaRMSNorm(h[t]) with
 * fp32 statistics, the normalised row rounded to bf16 and multiplied by the
 * bf16 weight (worker_sync.py:1344-1350). */
int swl_rmsnorm_rows_bf16(void* h, int64_t ntok, int64_t d, const void* const* add_rows, const void* weight,
                          float eps, void* const* out_rows, void* stream);

/* out_rows[t][j] = bf16(bf16(silu(g)) * u) with g = in_rows[t][j] and
 * u = in_rows[t][inter + j] (the fused Gate+Up output row): F.silu(gate) * up,
 * worker_sync.py:158, :1397. */
int swl_silu_mul_rows_bf16(const void* const* in_rows, void* const* out_rows, int64_t ntok, int64_t inter,
                           void* stream);

/* swl_paged_attention_bf16 with per-token rows: token t = seq * q_len + i
 * reads its fused [q | k | v] row at qkv_rows[t] (RoPE applied in place) and
 * writes its [hq * d] output row at out_rows[t].  rope = 2: q in the rows is
 * already rotated and k / v already appended to the pages (an out_mode 3
 * round), so only the attention itself runs. */
int swl_paged_attention_rows_bf16(void* const* qkv_rows, void* const* out_rows, int nseq, int q_len, int hq,
                                  int hkv, int d, void* k_cache, void* v_cache, int64_t num_blocks,
                                  int block_size, const int32_t* block_table, int64_t max_blocks,
                                  const int32_t* cache_seqlens, const int64_t* positions, const void* cos_sin,
                                  int64_t max_pos, int rope, float softmax_scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SWL_H */
