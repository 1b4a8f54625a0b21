// Persistent decode-layer chain for gfx950 (MI355X): one launch runs a
// sequence of dependent decode-shaped rounds (the O, Gate+Up and Down rounds
// of a layer and the next layer's fused QKV round) without kernel
// boundaries between them.
//
// Why: at 28 token rows a decode round is a stream of its weights (33-235 MB)
// through the MFMA units, and the per-kernel costs (launch, ramp-up of the
// first loads, the tail of the last workgroups, a second launch to reduce
// K-slices and finish the epilogue) are a large share of a 5-40 us round.
// Here every round is a phase of one persistent grid (one workgroup of 8
// waves per CU).  A workgroup requests the weights of its first tile of the
// next phase as soon as its own part of the current phase is stored, and only
// then waits for the other workgroups (a device-wide arrival counter per
// phase, bounded wait); its HBM requests are in flight while the phase
// boundary resolves.
//
// Each phase is a whole-K round: wave w holds k-steps w*S .. (w+1)*S - 1 of
// every token row as MFMA B fragments (registers; RMS-normalised on the way
// in when the phase reads the residual stream), multiplies them with its
// k-steps of a 16-row weight tile (fragment-tile layout, rows paired by the
// phase's pair offset), the 8 wave partials are summed in LDS and the
// workgroup finishes the tile: LoRA expand (lora_B rows moved into LDS by
// LDS-DMA with the tile's weights), then the out_mode fusion (residual add
// with per-tile sums of squares, SiLU(gate)*up, or RoPE with the KV-page
// append).  Rounds with K above 4096 (Down, K = 14336) stream the token rows
// with the weights, pass by pass, instead of holding them in registers.
//
// The LoRA shrink u = x . A^T of a phase is part of the same phase: the
// stacked lora_A rows of each adapter group are 16-row tiles processed like
// weight tiles by the workgroups with the fewest weight tiles, before their
// weight tiles; they store u (write-through) and count it on the phase's
// shrink counter, and every workgroup waits for that counter before its
// first expand.
//
// Memory ordering across XCDs (each has its own L2): everything a later
// phase of the same launch reads (outputs of modes 1 and 2, sums of squares,
// u) is stored written through to memory (system-scope buffer stores) and
// the store acknowledgements are awaited before the arrival is counted.  A
// later phase reads it with ordinary loads: every buffer a phase writes is
// read in this launch only after that phase (the caller passes distinct
// residual buffers for the O and Down outputs), so no XCD holds an older
// copy of those lines in its L2 (the caches are invalidated at kernel start).
//
// Counters: per phase an arrival and a shrink counter, and an exit counter;
// the last workgroup to exit resets them all to zero for the next launch.
// Every wait is bounded (spin_limit ticks of the 100 MHz real-time clock);
// a wait that runs out sets bit p of the status word and the grid carries
// on, so the launch always completes.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstring>
#include <new>

#include "dev_util.h"
#include "swl.h"
#include "swl_common.h"

namespace {

constexpr int kChWaves = 4;    // one wave per SIMD: 512 registers each (token rows 256, weights in flight 128)
constexpr int kChSteps = 32;   // k-steps per wave per pass
constexpr int kChPhases = SWL_CHAIN_MAX_ROUNDS;
constexpr int kChTok = 32;
constexpr int kChGroups = 32;
constexpr int kChBlk = 3;      // column blocks (q | k | v)
constexpr int kChURow = kChBlk * 16;
constexpr int kChUs = kChURow + 4;  // LDS row of u (padded)
constexpr int kChChunkSlots = 2;    // shrink chunks per workgroup (32 KiB of LDS each)

struct ChainPhase {
  const bf16* w;                // fragment tiles, rows paired by `off`
  int64_t N;
  int32_t K, steps;             // steps = K / 32
  int32_t n_wtiles, off, mode;
  int32_t nsw, npass;           // k-steps per wave per pass, passes per tile
  const bf16* x;                // input rows [ntok][ldx]
  int64_t ldx;
  const bf16* gamma;            // RMSNorm of x (null: none)
  const float* ss_in;           // [ntok][ld_ss_in] partial sums of squares
  int32_t ss_n, ld_ss_in;
  float eps;
  bf16* y;                      // output rows [ntok][ldy]
  int64_t ldy;
  const bf16* res;              // mode 1: y = res + out
  int64_t ldres;
  float* ss_out;                // mode 1: one sum of squares per 16-column tile
  int32_t ld_ss_out;
  int32_t inkernel;             // outputs read by a later phase: stored written through
  // LoRA (rank 16)
  int32_t n_atiles, ngroups, nblk, u_ld;
  int64_t blk_start[kChBlk + 1];
  const bf16* g_a[kChGroups];   // stacked lora_A rows [g_arows][K] of group g
  int32_t g_arows[kChGroups];
  int32_t g_tile0[kChGroups + 1];
  int32_t tok_grp[kChTok];      // adapter group of the token (-1: none)
  float tok_scale[kChTok];
  const bf16* tok_b[kChTok][kChBlk];  // lora_B [cols, 16] of the token's adapter, per block
  float* u;                     // [kChTok][u_ld]
};

struct ChainArgs {
  int32_t ntok, nphases;
  ChainPhase ph[kChPhases];
  // out_mode 3
  bf16* kc;
  bf16* vc;
  const int32_t* bt;
  const int32_t* seqlens;
  const int64_t* pos;
  const bf16* cs;
  int64_t max_blocks, num_blocks, max_pos;
  int32_t hq, hkv, bs;
  uint32_t* cnt;                // counter lines (kChLines each, kChLineWords apart): see cnt_arr / cnt_shr / cnt_exit
  uint32_t* status;             // bit p: a wait of phase p ran out
  uint64_t spin_limit;
  // optional timeline (null: off): per workgroup 2 + 3 * nphases stamps of
  // the 100 MHz clock: start, then per phase: barrier passed, first expand
  // ready (u in LDS), phase stored; exit
  uint64_t* trace;
};


typedef const __attribute__((address_space(4))) ChainArgs* chain_args_ptr;
typedef const __attribute__((address_space(4))) ChainPhase* chain_phase_ptr;

__device__ __forceinline__ void stamp(chain_args_ptr a, int slot) {
  if (a->trace && threadIdx.x == 0) {
    constexpr int kPer = 2 + 3 * kChPhases;
    *(__attribute__((address_space(1))) uint64_t*)(a->trace + (int64_t)blockIdx.x * kPer + slot) =
        __builtin_amdgcn_s_memrealtime();
  }
}


__device__ __forceinline__ uint32_t ld_counter(uint32_t* c) {
  return __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Device-wide counters.  Each counter is kChLines words, each on its own
// 128-byte line, that the workgroups (or waves) spread their increments
// over: increments of one address are serialised where the atomics execute,
// so 256 arrivals at one word take microseconds; a reader sums the lines.
constexpr int kChLines = 16;
constexpr int kChLineWords = 32;
constexpr int kChCounterWords = kChLines * kChLineWords;
__device__ __forceinline__ uint32_t* cnt_arr(uint32_t* cnt, int p) { return cnt + p * kChCounterWords; }
__device__ __forceinline__ uint32_t* cnt_shr(uint32_t* cnt, int p) {
  return cnt + (kChPhases + p) * kChCounterWords;
}
__device__ __forceinline__ uint32_t* cnt_exit(uint32_t* cnt) { return cnt + 2 * kChPhases * kChCounterWords; }
constexpr int kChCounterTotal = (2 * kChPhases + 2) * kChCounterWords;  // + the exit lines and the top exit word

__device__ __forceinline__ void line_add(uint32_t* c, int who) {
  __hip_atomic_fetch_add(c + (who % kChLines) * kChLineWords, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave 0 sums the counter's lines until the sum reaches `want` (bounded),
// then the workgroup continues.
__device__ __forceinline__ void wg_wait(chain_args_ptr a, uint32_t* c, uint32_t want, int p) {
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (true) {
      uint32_t v = l < kChLines ? __hip_atomic_load(c + l * kChLineWords, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                : 0u;
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
      if (__builtin_amdgcn_readfirstlane(v) >= want) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > a->spin_limit) {
        if (l == 0) __hip_atomic_fetch_or(a->status, 1u << p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
}

// This workgroup's stores are acknowledged, then the counter counts it.
__device__ __forceinline__ void wg_arrive(uint32_t* c) {
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __syncthreads();
  if (threadIdx.x == 0) line_add(c, blockIdx.x);
}

template <typename T>
__device__ __forceinline__ T ldgv(const T* p) { return *(const __attribute__((address_space(1))) T*)(p); }

__device__ __forceinline__ void st_wt16(__amdgpu_buffer_rsrc_t r, int64_t off_elems, bf16 v) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), r, (int)(off_elems * 2), 0, kStoreSys);
}
__device__ __forceinline__ void st_wt32(__amdgpu_buffer_rsrc_t r, int64_t off_elems, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, (int)(off_elems * 4), 0, kStoreSys);
}

// LDS of the chain kernel
template <int TT>
struct ChainLds {
  f32x4 red[kChWaves][TT][64];
  __attribute__((aligned(16))) bf16 bsm[2][kChTok][16][16];
  float us[kChTok][kChUs];
  float rsq[kChTok];
  const bf16* btab[kChPhases][kChTok][kChBlk];
  int32_t lgrp[kChPhases][kChTok];
  float lscale[kChPhases][kChTok];
  // shrink chunks of this workgroup's waves (at most 4): k-step s at [s][0..511]
  __attribute__((aligned(16))) bf16 achunk[kChChunkSlots][kChSteps][512];
};

// Weight tiles of workgroup j in a phase: j, j + G, ...
__device__ __forceinline__ int n_wtiles_of(chain_phase_ptr P, int j, int G) {
  return P->n_wtiles > j ? (P->n_wtiles - 1 - j) / G + 1 : 0;
}

// LoRA shrink chunks.  Chunk (A tile a, pass ps) of wave w is the 16 rows of
// lora_A tile a over wave w's k-steps of pass ps, i.e. the same k-steps the
// wave multiplies for every weight tile.  With G' = min(G, weight tiles) and
// c = a * npass + ps (c < n_chunks = n_atiles * npass <= G'), wave w of
// workgroup j = (c + stride * w) mod G' takes it (stride = G' / 8), so every
// chunk has one owner and a wave owns at most one.
struct ChainChunk {
  int has, a, ps, slot;
};
__device__ __forceinline__ ChainChunk chain_chunk_of(chain_phase_ptr P, int j, int G, int w) {
  ChainChunk c{0, 0, 0, 0};
  const int n_c = P->n_atiles * P->npass;
  const int Gp = min(G, P->n_wtiles);
  if (n_c == 0 || j >= Gp) return c;
  const int stride = max(1, Gp / kChWaves);
  int slot = 0;
  for (int v = 0; v < kChWaves; ++v) {
    const int cc = ((j - stride * v) % Gp + Gp) % Gp;
    if (cc >= n_c) continue;
    if (v == w) {
      c.has = 1;
      c.a = cc / P->npass;
      c.ps = cc % P->npass;
      c.slot = slot;
    }
    ++slot;
  }
  return c;
}

// lora_B rows of weight tile t into bsm[buf] by LDS-DMA: instruction i (two
// per wave, the last one repeated where there are fewer) moves tokens 2i and
// 2i + 1, each its adapter's 8 B rows under tile rows 0..7 and the 8 under
// rows 8..15, 256 bytes a piece (tokens without an adapter read harmless
// bytes of the weights)
template <int TT>
__device__ __forceinline__ void chain_issue_b(chain_phase_ptr P, ChainLds<TT>& sm, int p, int t, int buf, int ntok,
                                              int wv, int lane) {
  const int n_bins = (ntok + 1) >> 1;
  const int64_t c0 = paired_row(t, 0, P->off), c1 = c0 + P->off;
  const int b0 = (c0 >= P->blk_start[1]) + (c0 >= P->blk_start[2]);
  const int b1 = (c1 >= P->blk_start[1]) + (c1 >= P->blk_start[2]);
  const int64_t r0 = (c0 - P->blk_start[b0]) * 16, r1 = (c1 - P->blk_start[b1]) * 16;
  const int h = (lane >> 4) & 1;
#pragma unroll
  for (int jj = 0; jj < kChTok / 2 / kChWaves; ++jj) {
    const int ins = min(wv + kChWaves * jj, n_bins - 1);
    const int tk = 2 * ins + (lane >> 5);
    const bf16* src = sm.btab[p][tk < ntok ? tk : 0][h ? b1 : b0] + (h ? r1 : r0) + (lane & 15) * 8;
    __builtin_amdgcn_global_load_lds((gbl_ptr)src, (lds_ptr)(reinterpret_cast<char*>(&sm.bsm[buf][0][0][0]) + ins * 1024),
                                     16, 0, 0);
  }
}

// the loads of pass `pass` of weight tile `idx`: this wave's k-steps of the
// tile (and the tile's lora_B rows on its first pass)
template <int TT>
__device__ __forceinline__ void chain_issue(chain_phase_ptr P, ChainLds<TT>& sm, int p, int idx, int pass, int buf,
                                            int ntok, int wv, int lane, u32x4 (&wf)[kChSteps]) {
  const int nsw = P->nsw;
  const int s0 = wv * nsw * P->npass + pass * nsw;
  if (pass == 0 && P->n_atiles > 0) chain_issue_b<TT>(P, sm, p, idx, buf, ntok, wv, lane);
  const bf16* src = P->w + ((int64_t)idx * P->steps + s0) * 512 + 8 * lane;
  // steps past nsw re-read the last one (in bounds); their token fragments
  // are zero
#pragma unroll
  for (int s = 0; s < kChSteps; ++s) wf[s] = ldg16(src + (s < nsw ? s : nsw - 1) * 512);
}

// this wave's shrink chunk into LDS slot c.slot by LDS-DMA (lane l's 16 bytes
// of k-step s land at s * 1 KiB + 16 l: the MFMA A fragment it would load)
template <int TT>
__device__ __forceinline__ void chain_issue_chunk(chain_phase_ptr P, ChainLds<TT>& sm, const ChainChunk& c, int wv,
                                                  int lane) {
  if (!c.has) return;
  const int nsw = P->nsw;
  const int s0 = wv * nsw * P->npass + c.ps * nsw;
  // every adapter has rank 16: group g owns A tiles g * nblk .. + nblk - 1
  const int g = c.a / P->nblk;
  const int q = (c.a - g * P->nblk) * 16 + (lane & 15);
  const bf16* src = P->g_a[g] + (int64_t)min(q, P->g_arows[g] - 1) * P->K + 32 * s0 + 8 * (lane >> 4);
  char* dst = reinterpret_cast<char*>(&sm.achunk[c.slot][0][0]);
#pragma unroll
  for (int s = 0; s < kChSteps; ++s)
    if (s < nsw) __builtin_amdgcn_global_load_lds((gbl_ptr)(src + 32 * s), (lds_ptr)(dst + s * 1024), 16, 0, 0);
}

// the first loads of phase P for this workgroup (its first weight tile and
// its waves' shrink chunks)
template <int TT>
__device__ __forceinline__ void chain_prefetch(chain_phase_ptr P, ChainLds<TT>& sm, int p, int buf, int ntok, int wv,
                                               int lane, u32x4 (&wf)[kChSteps]) {
  const int G = gridDim.x, j = blockIdx.x;
  if (n_wtiles_of(P, j, G) == 0) return;
  chain_issue_chunk<TT>(P, sm, chain_chunk_of(P, j, G, wv), wv, lane);
  chain_issue<TT>(P, sm, p, j, 0, buf, ntok, wv, lane, wf);
}

// this wave's token-row fragments of pass `pass` (rows past ntok are zero)
template <int TT>
__device__ __forceinline__ void chain_load_x(chain_phase_ptr P, int pass, int ntok, int wv, int lane,
                                             u32x4 (&xf)[kChSteps][TT]) {
  const int nsw = P->nsw;
  const int s0 = wv * nsw * P->npass + pass * nsw;
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int tk = 16 * t + (lane & 15);
    const bf16* xr = P->x + (int64_t)(tk < ntok ? tk : 0) * P->ldx + 32 * s0 + 8 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < kChSteps; ++s)
      xf[s][t] = (tk < ntok && s < nsw) ? ldg16(xr + 32 * s) : u32x4{0u, 0u, 0u, 0u};
  }
}

// One phase of the chain for this workgroup: its weight tiles with the
// expand and the MODE fusion; its waves' shrink chunks ride along the first
// tile.  STREAM: token rows are loaded pass by pass with the weights
// (k > 4096) instead of held.
template <int TT, int MODE, bool STREAM>
__device__ __forceinline__ void chain_phase(chain_args_ptr a, int p, ChainLds<TT>& sm, u32x4 (&wf)[kChSteps],
                                            int& buf) {
  chain_phase_ptr P = &a->ph[p];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = gridDim.x, j = blockIdx.x;
  const int ntok = a->ntok;
  const int np = a->nphases;
  uint32_t* const cnt = a->cnt;
  const int nitems = n_wtiles_of(P, j, G);
  const int nsw = P->nsw, npass = STREAM ? P->npass : 1;
  const __amdgpu_buffer_rsrc_t rsrc_y =
      __builtin_amdgcn_make_buffer_rsrc(P->y, 0, (int)(ntok * P->ldy * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsrc_ss =
      __builtin_amdgcn_make_buffer_rsrc(P->ss_out, 0, P->ss_out ? (int)(ntok * P->ld_ss_out * 4) : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsrc_u =
      __builtin_amdgcn_make_buffer_rsrc(P->u, 0, P->u ? (int)(kChWaves * P->npass * kChTok * P->u_ld * 4) : 0,
                                        0x00020000);
  const ChainChunk ch = chain_chunk_of(P, j, G, wv);

  u32x4 xf[kChSteps][TT];
  if (!STREAM && nitems > 0) {
    chain_load_x<TT>(P, 0, ntok, wv, lane, xf);
    if (P->gamma) {
      // row factors r = rsqrt(sum of the row's partial sums of squares / K +
      // eps): 16 threads per token, every load in flight at once
      // (16 threads per token, the two halves of the tokens one after the
      // other)
#pragma unroll
      for (int half = 0; half < kChTok / (kChWaves * 4); ++half) {
        const int tk = threadIdx.x / 16 + half * (kChWaves * 4), l16 = threadIdx.x & 15;
        float part[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int i = l16 + 16 * q;
          part[q] = (tk < ntok && i < P->ss_n) ? ldgv(P->ss_in + (int64_t)tk * P->ld_ss_in + i) : 0.f;
        }
        float sq = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q) sq += part[q];
        sq += __shfl_xor(sq, 1, 64);
        sq += __shfl_xor(sq, 2, 64);
        sq += __shfl_xor(sq, 4, 64);
        sq += __shfl_xor(sq, 8, 64);
        if (l16 == 0) sm.rsq[tk] = rsqrtf(sq / (float)P->K + P->eps);
      }
      lds_barrier();
      const bf16* gp = P->gamma + 32 * wv * nsw + 8 * (lane >> 4);
#pragma unroll
      for (int s = 0; s < kChSteps; ++s) {
        if (s >= nsw) continue;
        const u32x4 gv = ldg16(gp + 32 * s);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          const int tk2 = 16 * t + (lane & 15);
          xf[s][t] = norm8(xf[s][t], sm.rsq[tk2 < ntok ? tk2 : 0], gv);
        }
      }
    }
  }

  bool u_ready = P->n_atiles == 0;
  for (int k = 0; k < nitems; ++k) {
    const int idx = j + k * G;
    const int cur_buf = buf;
    f32x4 acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int pass = 0; pass < npass; ++pass) {
      if (pass > 0) chain_issue<TT>(P, sm, p, idx, pass, cur_buf, ntok, wv, lane, wf);
      if (STREAM) chain_load_x<TT>(P, pass, ntok, wv, lane, xf);
      __builtin_amdgcn_s_waitcnt(kWaitVm0);  // the tile's loads, its lora_B rows and the chunk have landed
#pragma unroll
      for (int s = 0; s < kChSteps; ++s)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[t] = mfma16(wf[s], xf[s][t], acc[t]);
      if (k == 0 && ch.has && ch.ps == pass) {
        // the shrink chunk, with the token fragments this pass holds; its
        // group's tokens store their u partial (write-through) and the
        // wave counts it
        // the tile's partial sums wait in this wave's own LDS reduction slot
        // (no other wave reads it before the next barrier), the chunk's A
        // fragments are read from LDS eight k-steps at a time
#pragma unroll
        for (int t = 0; t < TT; ++t) sm.red[wv][t][lane] = acc[t];
        f32x4 au[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) au[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        const bf16* cs = &sm.achunk[ch.slot][0][0] + 8 * lane;
#pragma unroll
        for (int h = 0; h < kChSteps; h += 8) {
          u32x4 af[8];
#pragma unroll
          for (int s = 0; s < 8; ++s) af[s] = *reinterpret_cast<const u32x4*>(cs + 512 * (h + s < nsw ? h + s : nsw - 1));
#pragma unroll
          for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int t = 0; t < TT; ++t) au[t] = mfma16(af[s], xf[h + s][t], au[t]);
          __builtin_amdgcn_sched_barrier(0);
        }
        const int g = ch.a / P->nblk;
        const int q = (ch.a - g * P->nblk) * 16 + 4 * (lane >> 4);
        const int slot = wv * npass + ch.ps;
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          const int tk = 16 * t + (lane & 15);
          if (tk < ntok && sm.lgrp[p][tk] == g)
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4, au[t]), rsrc_u,
                (int)((((int64_t)slot * kChTok + tk) * P->u_ld + q) * 4), 0, kStoreSys);
        }
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        if (lane == 0) line_add(cnt_shr(cnt, p), blockIdx.x * kChWaves + wv);
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[t] = sm.red[wv][t][lane];
      }
    }
    const bool last = k + 1 == nitems;
    buf ^= 1;
    if (!last) chain_issue<TT>(P, sm, p, idx + G, 0, buf, ntok, wv, lane, wf);  // in flight during the epilogue
#pragma unroll
    for (int t = 0; t < TT; ++t) sm.red[wv][t][lane] = acc[t];
    lds_barrier();
    auto total = [&](int r, int tk) {
      const int l = (r >> 2) * 16 + (tk & 15), t = tk >> 4, e = r & 3;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kChWaves; ++w) v += sm.red[w][t][l][e];
      return v;
    };

    if (!u_ready) {
      // every shrink chunk of the phase is stored: u = the sum of the chunk
      // partials (waves x passes), summed in a fixed order
      wg_wait(a, cnt_shr(cnt, p), (uint32_t)(P->n_atiles * P->npass * kChWaves), p);
      const int nslot = kChWaves * npass;
      constexpr int kUPer = (kChTok * kChURow + kChWaves * 64 - 1) / (kChWaves * 64);
#pragma unroll
      for (int qq = 0; qq < kUPer; ++qq) {
        const int i = threadIdx.x + qq * kChWaves * 64;
        if (i >= ntok * P->u_ld) break;
        const int tk = i / P->u_ld, q = i - tk * P->u_ld;
        float v = 0.f;
        if (sm.lgrp[p][tk] >= 0) {
          for (int b0 = 0; b0 < nslot; b0 += kChWaves) {  // nslot = kChWaves * npass
            float part[kChWaves];
#pragma unroll
            for (int sl = 0; sl < kChWaves; ++sl) part[sl] = ldgv(P->u + ((int64_t)(b0 + sl) * kChTok + tk) * P->u_ld + q);
#pragma unroll
            for (int sl = 0; sl < kChWaves; ++sl) v += part[sl];
          }
        }
        sm.us[tk][q] = v;
      }
      lds_barrier();
      u_ready = true;
      stamp(a, 2 + 3 * p);
    }

    // thread (token tk, pair pp) finishes tile rows pp and pp + 8: output
    // columns c0 and c0 + off
    const int e = threadIdx.x;
    const int tk = e >> 3, pp = e & 7;
    const int64_t c0 = paired_row(idx, pp, P->off), c1 = c0 + P->off;
    const bool live = tk < ntok && c0 < P->N;
    float v0 = 0.f, v1 = 0.f;
    if (live) {
      v0 = total(pp, tk);
      v1 = total(pp + 8, tk);
      if (sm.lgrp[p][tk] >= 0) {
        const float sc = sm.lscale[p][tk];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int64_t c = h ? c1 : c0;
          const int b = (c >= P->blk_start[1]) + (c >= P->blk_start[2]);
          const float* ub = &sm.us[tk][b * 16];
          const bf16* bl = &sm.bsm[cur_buf][tk][8 * h + pp][0];
          float d = 0.f;
#pragma unroll
          for (int q = 0; q < 16; q += 8) {
            float bv[8];
            unpack8(*reinterpret_cast<const u32x4*>(bl + q), bv);
#pragma unroll
            for (int i = 0; i < 8; ++i) d += ub[q + i] * bv[i];
          }
          (h ? v1 : v0) += d * sc;
        }
      }
    }
    if constexpr (MODE == 1) {
      // y = bf16(res + bf16(out)); the tile's sum of squares of y per token
      float sq = 0.f;
      if (live) {
        const bf16* rr = P->res + (int64_t)tk * P->ldres;
        const bf16 h0 = f2bf(bf2f(ldg(rr + c0)) + bf2f(f2bf(v0)));
        const bf16 h1 = f2bf(bf2f(ldg(rr + c1)) + bf2f(f2bf(v1)));
        const int64_t o = (int64_t)tk * P->ldy;
        st_wt16(rsrc_y, o + c0, h0);
        st_wt16(rsrc_y, o + c1, h1);
        sq = bf2f(h0) * bf2f(h0) + bf2f(h1) * bf2f(h1);
      }
      sq += __shfl_xor(sq, 1, 64);
      sq += __shfl_xor(sq, 2, 64);
      sq += __shfl_xor(sq, 4, 64);
      if (live && pp == 0 && P->ss_out) st_wt32(rsrc_ss, (int64_t)tk * P->ld_ss_out + idx, sq);
    } else if constexpr (MODE == 2) {
      // c0 a gate column, c1 = c0 + inter its up column
      if (live) {
        const float g = bf2f(f2bf(v0)), uu = bf2f(f2bf(v1));
        st_wt16(rsrc_y, (int64_t)tk * P->ldy + c0, f2bf(bf2f(f2bf(g / (1.0f + __expf(-g)))) * uu));
      }
    } else {
      // c0 = head * 128 + d (d < 64), c1 = c0 + 64: NeoX RoPE pair of q / k
      // heads; k and v also appended to their KV pages (read by the next
      // launch: ordinary stores)
      if (live) {
        const int hh = (int)(c0 >> 7), d = (int)(c0 & 63);
        const bool is_q = hh < a->hq, is_k = !is_q && hh < a->hq + a->hkv;
        float x0 = bf2f(f2bf(v0)), x1 = bf2f(f2bf(v1));
        const int64_t ps = ldgv(a->pos + tk);
        if ((is_q || is_k) && ps >= 0 && ps < a->max_pos) {
          const float rc = bf2f(ldg(a->cs + ps * 128 + d)), rs = bf2f(ldg(a->cs + ps * 128 + 64 + d));
          const float n0 = bf2f(f2bf(x0 * rc - x1 * rs));
          const float n1 = bf2f(f2bf(x1 * rc + x0 * rs));
          x0 = n0;
          x1 = n1;
        }
        bf16* yr = P->y + (int64_t)tk * P->ldy;
        stg(yr + c0, f2bf(x0));
        stg(yr + c1, f2bf(x1));
        const int64_t slen = ldgv(a->seqlens + tk);
        if (!is_q && slen >= 0 && slen / a->bs < a->max_blocks) {
          const int32_t pb = ldgv(a->bt + (int64_t)tk * a->max_blocks + slen / a->bs);
          if (pb >= 0 && pb < a->num_blocks) {
            const int kvh = is_k ? hh - a->hq : hh - a->hq - a->hkv;
            const int64_t dst = ((int64_t)pb * a->bs + slen % a->bs) * a->hkv * 128 + kvh * 128 + d;
            bf16* cache = is_k ? a->kc : a->vc;
            stg(cache + dst, f2bf(x0));
            stg(cache + dst + 64, f2bf(x1));
          }
        }
      }
    }
    lds_barrier();  // red and bsm[cur_buf] are rewritten after this
  }
}

// Phase kinds (compile-time, so that each phase's registers are allocated
// on their own): 1 residual (token rows held), 2 SiLU * up, 3 RoPE + KV
// append, 4 residual with the token rows streamed (k > 4096).
template <int TT, int KIND>
__device__ __forceinline__ void chain_step(chain_args_ptr a, int p, ChainLds<TT>& sm, u32x4 (&wf)[kChSteps],
                                           int& buf) {
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = gridDim.x;
  uint32_t* const cnt = a->cnt;
  if (p > 0) wg_wait(a, cnt_arr(cnt, p - 1), (uint32_t)G, p);
  stamp(a, 1 + 3 * p);
  chain_phase<TT, KIND == 4 ? 1 : KIND, KIND == 4>(a, p, sm, wf, buf);
  stamp(a, 3 + 3 * p);
  // this workgroup's part of the phase is stored: count it, then request
  // the first loads of the next phase before waiting for the others
  wg_arrive(cnt_arr(cnt, p));
  if (p + 1 < a->nphases) chain_prefetch<TT>(&a->ph[p + 1], sm, p + 1, buf, a->ntok, wv, lane, wf);
}

template <int TT, int... KINDS>
__global__ __launch_bounds__(kChWaves * 64, 1) void chain_kernel(const ChainArgs* args) {
  chain_args_ptr a = (chain_args_ptr)args;
  __shared__ ChainLds<TT> sm;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = gridDim.x;
  const int ntok = a->ntok;
  constexpr int np = sizeof...(KINDS);
  uint32_t* const cnt = a->cnt;

  // per-phase token tables: adapter group, scale and lora_B bases
  for (int i = threadIdx.x; i < kChPhases * kChTok * kChBlk; i += kChWaves * 64) {
    const int p = i / (kChTok * kChBlk), r = i % (kChTok * kChBlk), tk = r / kChBlk, b = r % kChBlk;
    const bool on = p < np && tk < ntok && a->ph[p].tok_grp[tk] >= 0 && b < a->ph[p].nblk;
    sm.btab[p][tk][b] = on ? a->ph[p].tok_b[tk][b] : (p < np ? a->ph[p].w : nullptr);
    if (b == 0) {
      sm.lgrp[p][tk] = (p < np && tk < ntok) ? a->ph[p].tok_grp[tk] : -1;
      sm.lscale[p][tk] = (p < np && tk < ntok) ? a->ph[p].tok_scale[tk] : 0.f;
    }
  }
  __syncthreads();

  u32x4 wf[kChSteps];
  int buf = 0;  // bsm buffer the next weight tile's lora_B rows go to
  stamp(a, 0);
  chain_prefetch<TT>(&a->ph[0], sm, 0, buf, ntok, wv, lane, wf);
  int p = 0;
  (chain_step<TT, KINDS>(a, p++, sm, wf, buf), ...);

  // the last workgroup out resets the counters for the next launch
  __syncthreads();
  stamp(a, 1 + 3 * kChPhases);
  if (threadIdx.x == 0) {
    // two levels: the last workgroup of each exit line counts on the top
    // word, the last of those resets every counter
    uint32_t* ex = cnt_exit(cnt);
    const int line = blockIdx.x % kChLines;
    const uint32_t in_line = (uint32_t)((G - 1 - line) / kChLines + 1);
    const uint32_t prev = __hip_atomic_fetch_add(ex + line * kChLineWords, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    if (prev == in_line - 1) {
      uint32_t* top = ex + kChCounterWords;
      const uint32_t lines = (uint32_t)min(G, kChLines);
      const uint32_t done = __hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (done == lines - 1) {
        for (int p2 = 0; p2 < np; ++p2)
          for (int l = 0; l < kChLines; ++l) {
            __hip_atomic_store(cnt_arr(cnt, p2) + l * kChLineWords, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(cnt_shr(cnt, p2) + l * kChLineWords, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        for (int l = 0; l < kChLines; ++l)
          __hip_atomic_store(ex + l * kChLineWords, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(top, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// ------------------------------------------------------------------- host
int cu_count_here() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  return n;
}

struct PlanImpl {
  ChainArgs host;
  ChainArgs* dev = nullptr;
  float* u = nullptr;
  uint32_t* cnt = nullptr;
  uint32_t* status = nullptr;
  int grid = 0, tt = 1;
  int seq = -1;  // compiled phase sequence (chain_kernel instantiation)
  int device = 0;
  int64_t bytes = 0;  // algorithmic bytes of one launch
};

int plan_phase(ChainPhase& P, const swl_chain_round& r, int ntok, const swl_lora_entry* table_host, int n_entries,
               float* u, int64_t* bytes) {
  SWL_CHECK(r.w && r.x && r.y, SWL_ERR_INVALID, "chain round: w, x and y are required");
  SWL_CHECK(r.k >= 256 && r.k % 256 == 0, SWL_ERR_INVALID, "chain round: k must be a positive multiple of 256");
  SWL_CHECK(r.out_mode >= 1 && r.out_mode <= 3, SWL_ERR_INVALID, "chain round: out_mode must be 1, 2 or 3");
  const int64_t off = r.out_mode == 2 ? r.n / 2 : r.out_mode == 3 ? 64 : 8;
  SWL_CHECK(r.n >= 16 && off % 8 == 0 && r.n % (2 * off) == 0, SWL_ERR_INVALID,
            "chain round: n must be a multiple of 16 (of 2 * inter for out_mode 2, of 128 for out_mode 3)");
  SWL_CHECK(r.ldx >= r.k && r.ldy >= (r.out_mode == 2 ? r.n / 2 : r.n), SWL_ERR_INVALID,
            "chain round: row strides shorter than the rows");
  P.w = reinterpret_cast<const bf16*>(r.w);
  P.N = r.n;
  P.K = (int32_t)r.k;
  P.steps = (int32_t)(r.k / 32);
  P.n_wtiles = (int32_t)(r.n / 16);
  P.off = (int32_t)off;
  P.mode = r.out_mode;
  const int spw = P.steps / kChWaves;  // k-steps per wave
  int npass = (spw + kChSteps - 1) / kChSteps;
  while (spw % npass) ++npass;
  P.npass = npass;
  P.nsw = spw / npass;
  SWL_CHECK(P.nsw >= 1 && P.nsw <= kChSteps, SWL_ERR_INVALID, "chain round: k has no pass split of <= 32 k-steps");
  P.x = reinterpret_cast<const bf16*>(r.x);
  P.ldx = r.ldx;
  if (r.norm_weight) {
    SWL_CHECK(npass == 1, SWL_ERR_INVALID, "chain round: RMSNorm on the way in needs k <= 4096");
    SWL_CHECK(r.ss_in && r.ss_in_n >= 1 && r.ss_in_n <= 256 && r.ss_in_stride >= r.ss_in_n, SWL_ERR_INVALID,
              "chain round: RMSNorm needs ss_in [ntok, ss_in_n] with ss_in_n <= 256");
    P.gamma = reinterpret_cast<const bf16*>(r.norm_weight);
    P.ss_in = r.ss_in;
    P.ss_n = r.ss_in_n;
    P.ld_ss_in = r.ss_in_stride;
    P.eps = r.eps;
  }
  P.y = reinterpret_cast<bf16*>(r.y);
  P.ldy = r.ldy;
  if (r.out_mode == 1) {
    SWL_CHECK(r.res != nullptr && r.ldres >= r.n, SWL_ERR_INVALID, "chain round: out_mode 1 needs res rows");
    P.res = reinterpret_cast<const bf16*>(r.res);
    P.ldres = r.ldres;
    if (r.ss_out) {
      SWL_CHECK(r.ss_out_stride >= r.n / 16, SWL_ERR_INVALID, "chain round: ss_out_stride must be >= n / 16");
      P.ss_out = r.ss_out;
      P.ld_ss_out = r.ss_out_stride;
    }
  }
  P.inkernel = r.out_mode != 3;
  int64_t b = 2 * (r.n * r.k + (int64_t)ntok * r.k + (int64_t)ntok * (r.out_mode == 2 ? r.n / 2 : r.n));
  // LoRA: groups of tokens sharing an entry (every entry rank 16)
  bool any = false;
  if (r.lora)
    for (int i = 0; i < ntok; ++i) any |= r.lora[i] >= 0;
  for (int i = 0; i < ntok; ++i) P.tok_grp[i] = -1;
  if (any) {
    SWL_CHECK(table_host != nullptr, SWL_ERR_INVALID, "chain round: LoRA needs the host table");
    SWL_CHECK(r.nblk >= 1 && r.nblk <= kChBlk, SWL_ERR_INVALID, "chain round: 1..3 LoRA column blocks");
    int64_t s = 0;
    P.blk_start[0] = 0;
    for (int bb = 0; bb < r.nblk; ++bb) {
      SWL_CHECK(r.blk_cols[bb] > 0, SWL_ERR_INVALID, "chain round: LoRA block widths must be positive");
      s += r.blk_cols[bb];
      P.blk_start[bb + 1] = s;
    }
    SWL_CHECK(s == r.n, SWL_ERR_INVALID, "chain round: LoRA block widths must sum to n");
    for (int bb = r.nblk + 1; bb <= kChBlk; ++bb) P.blk_start[bb] = INT64_MAX / 4;
    P.nblk = r.nblk;
    P.u_ld = 16 * r.nblk;
    int entry_of[kChGroups];
    int ng = 0, tiles = 0;
    for (int i = 0; i < ntok; ++i) {
      const int e = r.lora[i];
      if (e < 0) continue;
      SWL_CHECK(e < n_entries, SWL_ERR_INVALID, "chain round: LoRA entry index out of range");
      const swl_lora_entry& E = table_host[e];
      SWL_CHECK(E.rank == 16, SWL_ERR_INVALID, "chain round: adapters must have rank 16");
      int g = 0;
      while (g < ng && entry_of[g] != e) ++g;
      if (g == ng) {
        entry_of[ng] = e;
        P.g_a[ng] = reinterpret_cast<const bf16*>(E.a);
        P.g_arows[ng] = 16 * r.nblk;
        P.g_tile0[ng] = tiles;
        tiles += r.nblk;
        b += 2 * (int64_t)(16 * r.nblk) * (r.k + r.n);
        ++ng;
      }
      P.tok_grp[i] = g;
      P.tok_scale[i] = E.scale;
      for (int bb = 0; bb < r.nblk; ++bb) {
        SWL_CHECK(E.b[bb] != nullptr, SWL_ERR_INVALID, "chain round: LoRA entry without a B block");
        P.tok_b[i][bb] = reinterpret_cast<const bf16*>(E.b[bb]);
      }
    }
    P.ngroups = ng;
    P.g_tile0[ng] = tiles;
    P.n_atiles = tiles;
    P.u = u;
  }
  *bytes += b;
  return SWL_OK;
}

}  // namespace

extern "C" {

int swl_chain_create(int ntok, int n_rounds, const swl_chain_round* rounds, const swl_lora_entry* lora_table_host,
                     int n_entries, const swl_round_fusion* kv, swl_chain_plan** out) {
  SWL_CHECK(out != nullptr, SWL_ERR_INVALID, "chain: null plan pointer");
  *out = nullptr;
  SWL_CHECK(ntok >= 1 && ntok <= kChTok, SWL_ERR_INVALID, "chain: 1..32 token rows");
  SWL_CHECK(n_rounds >= 1 && n_rounds <= kChPhases, SWL_ERR_INVALID, "chain: 1..4 rounds");
  SWL_CHECK(rounds != nullptr, SWL_ERR_INVALID, "chain: null rounds");
  PlanImpl* pl = new (std::nothrow) PlanImpl();
  SWL_CHECK(pl != nullptr, SWL_ERR_INVALID, "chain: out of host memory");
  std::memset(&pl->host, 0, sizeof(pl->host));
  ChainArgs& A = pl->host;
  A.ntok = ntok;
  A.nphases = n_rounds;
  auto fail_free = [&](int rc) {
    if (pl->dev) (void)hipFree(pl->dev);
    if (pl->u) (void)hipFree(pl->u);
    if (pl->cnt) (void)hipFree(pl->cnt);
    delete pl;
    return rc;
  };
  if (hipGetDevice(&pl->device) != hipSuccess) return fail_free(swl::fail(SWL_ERR_HIP, "chain: hipGetDevice failed"));
  const size_t u_floats = (size_t)kChPhases * kChWaves * 4 * kChTok * kChURow;
  if (hipMalloc(&pl->u, u_floats * sizeof(float)) != hipSuccess)
    return fail_free(swl::fail(SWL_ERR_HIP, "chain: hipMalloc failed"));
  int mode3 = 0;
  for (int p = 0; p < n_rounds; ++p) {
    int rc = plan_phase(A.ph[p], rounds[p], ntok, lora_table_host, n_entries,
                        pl->u + (size_t)p * kChWaves * 4 * kChTok * kChURow,
                        &pl->bytes);
    if (rc) return fail_free(rc);
    mode3 += rounds[p].out_mode == 3;
  }
  pl->grid = cu_count_here();
  // shrink chunks: every chunk has one owner wave, a workgroup's owners fit
  // its LDS slots
  for (int p = 0; p < n_rounds; ++p) {
    const ChainPhase& P = A.ph[p];
    if (P.n_atiles == 0) continue;
    if (P.npass > 4)
      return fail_free(swl::fail(SWL_ERR_UNSUPPORTED, "chain: LoRA rounds take at most 4 passes (k <= 16384)"));
    const int n_c = P.n_atiles * P.npass, Gp = std::min(pl->grid, P.n_wtiles);
    if (n_c > Gp)
      return fail_free(swl::fail(SWL_ERR_UNSUPPORTED, "chain: more LoRA rows than the round's weight tiles can carry"));
    const int stride = std::max(1, Gp / kChWaves);
    for (int j = 0; j < Gp; ++j) {
      int owners = 0;
      for (int v = 0; v < kChWaves; ++v) owners += (((j - stride * v) % Gp + Gp) % Gp) < n_c;
      if (owners > kChChunkSlots)
        return fail_free(swl::fail(SWL_ERR_UNSUPPORTED, "chain: too many LoRA rows per workgroup"));
    }
  }
  if (mode3) {
    if (!kv || !kv->k_cache || !kv->v_cache || !kv->block_table || !kv->cache_seqlens || !kv->positions ||
        !kv->cos_sin || kv->hq <= 0 || kv->hkv <= 0 || kv->block_size <= 0)
      return fail_free(swl::fail(SWL_ERR_INVALID, "chain: out_mode 3 needs the KV pages, block table, sequence "
                                                  "lengths, positions and cos/sin cache"));
    A.kc = reinterpret_cast<bf16*>(kv->k_cache);
    A.vc = reinterpret_cast<bf16*>(kv->v_cache);
    A.bt = kv->block_table;
    A.seqlens = kv->cache_seqlens;
    A.pos = kv->positions;
    A.cs = reinterpret_cast<const bf16*>(kv->cos_sin);
    A.max_blocks = kv->max_blocks;
    A.num_blocks = kv->num_blocks;
    A.max_pos = kv->max_pos;
    A.hq = kv->hq;
    A.hkv = kv->hkv;
    A.bs = kv->block_size;
  }
  const size_t cnt_words = kChCounterTotal + kChLineWords;  // + the status word
  if (hipMalloc(&pl->cnt, cnt_words * sizeof(uint32_t)) != hipSuccess ||
      hipMemset(pl->cnt, 0, cnt_words * sizeof(uint32_t)) != hipSuccess)
    return fail_free(swl::fail(SWL_ERR_HIP, "chain: counter allocation failed"));
  pl->status = pl->cnt + kChCounterTotal;
  A.cnt = pl->cnt;
  A.status = pl->status;
  A.spin_limit = 100ull * 1000 * 200;  // 200 ms of the 100 MHz clock
  if (hipMalloc(&pl->dev, sizeof(ChainArgs)) != hipSuccess ||
      hipMemcpy(pl->dev, &A, sizeof(ChainArgs), hipMemcpyHostToDevice) != hipSuccess)
    return fail_free(swl::fail(SWL_ERR_HIP, "chain: argument upload failed"));
  pl->tt = ntok > 16 ? 2 : 1;
  // the compiled phase sequences: kind 1 residual, 2 SiLU * up, 3 RoPE + KV
  // append, 4 residual with streamed token rows
  {
    int kinds[kChPhases] = {0, 0, 0, 0};
    for (int p = 0; p < n_rounds; ++p) kinds[p] = A.ph[p].mode == 1 && A.ph[p].npass > 1 ? 4 : A.ph[p].mode;
    static const int seqs[6][kChPhases + 1] = {{4, 1, 2, 4, 3}, {3, 1, 2, 4, 0}, {1, 1, 0, 0, 0},
                                               {1, 2, 0, 0, 0}, {1, 3, 0, 0, 0}, {1, 4, 0, 0, 0}};
    for (int q = 0; q < 6 && pl->seq < 0; ++q) {
      bool same = seqs[q][0] == n_rounds;
      for (int p = 0; p < n_rounds && same; ++p) same = seqs[q][p + 1] == kinds[p];
      if (same) pl->seq = q;
    }
    if (pl->seq < 0)
      return fail_free(swl::fail(SWL_ERR_UNSUPPORTED, "chain: supported round sequences are (residual, SiLU*up, "
                                                      "residual with k > 4096[, RoPE]) and single rounds"));
  }
  *out = reinterpret_cast<swl_chain_plan*>(pl);
  return SWL_OK;
}

int swl_chain_launch(swl_chain_plan* h, void* stream) {
  PlanImpl* pl = reinterpret_cast<PlanImpl*>(h);
  SWL_CHECK(pl != nullptr, SWL_ERR_INVALID, "chain: null plan");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(pl->grid), block(kChWaves * 64);
  switch (pl->seq * 2 + (pl->tt - 1)) {
#define SWL_CHAIN_CASE(id, ...)                                                                       \
  case 2 * (id): hipLaunchKernelGGL((chain_kernel<1, __VA_ARGS__>), grid, block, 0, st, pl->dev); break; \
  case 2 * (id) + 1: hipLaunchKernelGGL((chain_kernel<2, __VA_ARGS__>), grid, block, 0, st, pl->dev); break;
    SWL_CHAIN_CASE(0, 1, 2, 4, 3)
    SWL_CHAIN_CASE(1, 1, 2, 4)
    SWL_CHAIN_CASE(2, 1)
    SWL_CHAIN_CASE(3, 2)
    SWL_CHAIN_CASE(4, 3)
    SWL_CHAIN_CASE(5, 4)
#undef SWL_CHAIN_CASE
    default: return swl::fail(SWL_ERR_INVALID, "chain: no kernel for this sequence of rounds");
  }
  SWL_LAUNCH_CHECK("chain_kernel launch");
  return SWL_OK;
}

int swl_chain_status(swl_chain_plan* h, uint32_t* timed_out) {
  PlanImpl* pl = reinterpret_cast<PlanImpl*>(h);
  SWL_CHECK(pl != nullptr && timed_out != nullptr, SWL_ERR_INVALID, "chain: null argument");
  SWL_HIP(hipDeviceSynchronize());
  SWL_HIP(hipMemcpy(timed_out, pl->status, sizeof(uint32_t), hipMemcpyDeviceToHost));
  SWL_HIP(hipMemset(pl->status, 0, sizeof(uint32_t)));
  return SWL_OK;
}

int swl_chain_trace(swl_chain_plan* h, uint64_t* trace) {
  PlanImpl* pl = reinterpret_cast<PlanImpl*>(h);
  SWL_CHECK(pl != nullptr, SWL_ERR_INVALID, "chain: null plan");
  pl->host.trace = trace;
  SWL_HIP(hipMemcpy(pl->dev, &pl->host, sizeof(ChainArgs), hipMemcpyHostToDevice));
  return SWL_OK;
}

int swl_chain_grid(const swl_chain_plan* h) {
  const PlanImpl* pl = reinterpret_cast<const PlanImpl*>(h);
  return pl ? pl->grid : 0;
}

int64_t swl_chain_bytes(const swl_chain_plan* h) {
  const PlanImpl* pl = reinterpret_cast<const PlanImpl*>(h);
  return pl ? pl->bytes : 0;
}

int swl_chain_destroy(swl_chain_plan* h) {
  PlanImpl* pl = reinterpret_cast<PlanImpl*>(h);
  if (!pl) return SWL_OK;
  (void)hipFree(pl->dev);
  (void)hipFree(pl->u);
  (void)hipFree(pl->cnt);
  delete pl;
  return SWL_OK;
}

}  // extern "C"
