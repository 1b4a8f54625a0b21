// HIP kernels for gfx950 (MI355X) and their stream-ordered C-ABI launchers.
//
// Kernels
//   gather_rows_kernel      slot rows -> packed batch (128-bit copies)
//   scatter_rows_kernel     packed rows (+ delta) -> slot rows
//   split_kernel<TT,WAVES>  M <= 64 "decode" projection, part 1: one K-slice
//                           per workgroup (16 waves, one workgroup per CU, up
//                           to 64 token rows); the K-slice of every token's
//                           activation (read through per-token row pointers:
//                           the gather is fused) is staged once in LDS and
//                           shared by the waves, 16-row W tiles dealt over the
//                           slice's workgroups are streamed from HBM straight
//                           into MFMA A-fragments, fp32 partials go to
//                           scratch.  The stacked lora_A of each adapter of
//                           the round are extra row tiles: the LoRA shrink
//                           u = x . A^T rides the same stream.
//   epilogue_kernel         part 2: sums the K-slice partials, adds bias and
//                           the LoRA expand u . B^T * scale, rounds once and
//                           stores each token's row into its slot buffer (the
//                           scatter is fused).
//   gemm256_kernel          M > 64 "prefill" projection: 256x256 (or 256x192)
//                           MFMA tiles fed by LDS-DMA, rows read in place from
//                           the slot buffers, the LoRA delta as extra k-steps.
//   tiled_kernel            the prefill projection for K not a multiple of 64:
//                           128x128x64 LDS-staged MFMA tiles over a gathered
//                           copy, fp32 accumulation, same epilogue.
//   fullk_kernel            the whole-K decode round (the decode step's LM
//                           head): no K-slice partials, no epilogue launch.
//   lora_rows_kernel        a worker's LoRA delta of a few token rows.
//   matmul_generic_kernel   small row-major products with arbitrary strides
//                           (worker-side LoRA modules).
//   rope_append_kernel, attn_tile_kernel + attn_combine_kernel (decode),
//   attn_chunk_kernel, attention_kernel     paged-KV attention.
//
// MFMA used: v_mfma_f32_16x16x32_bf16 (decode rounds, attention, shrink) and
// v_mfma_f32_32x32x16_bf16 (gemm256_kernel).  16x16x32 operand layout
// (wave64): lane l feeds
// row (l % 16) of A and column (l % 16) of B with the 8 consecutive k values of
// k-group (l / 16); the 16x16 fp32 result lands in lane l as rows
// 4*(l/16)+j, j=0..3, of column (l % 16).  The k-group -> k assignment is the
// same for A and B, so any consistent assignment of memory k to (group, j)
// computes the same dot products.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "swl_common.h"
#include "swl.h"
#include "dev_util.h"

namespace {


constexpr int kMaxSeg = SWL_MAX_SLOTS;
constexpr int kSkinnyMaxTok = 64;


// ---------------------------------------------------------------- gather ---
struct SegPtrs {
  int32_t n;
  int32_t vec;                  // 1 = 16-byte path usable
  int64_t off[kMaxSeg + 1];     // exclusive prefix sum of rows
  const void* ptr[kMaxSeg];     // per-segment base pointer
};

__device__ __forceinline__ int find_seg(const int64_t* off, int n, int64_t row) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (off[mid] <= row) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// One workgroup per packed row; segment lookup is uniform per workgroup.
__global__ __launch_bounds__(256) void gather_rows_kernel(SegPtrs sp, int64_t d, bf16* __restrict__ packed) {
  const int64_t row = blockIdx.x;
  const int s = find_seg(sp.off, sp.n, row);
  const bf16* src = reinterpret_cast<const bf16*>(sp.ptr[s]) + (row - sp.off[s]) * d;
  bf16* dst = packed + row * d;
  if (sp.vec) {
    const int64_t nv = d >> 3;
    for (int64_t i = threadIdx.x; i < nv; i += blockDim.x)
      reinterpret_cast<u32x4*>(dst)[i] = reinterpret_cast<const u32x4*>(src)[i];
  } else {
    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src);
    uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
    for (int64_t i = threadIdx.x; i < d; i += blockDim.x) d16[i] = s16[i];
  }
}

__global__ __launch_bounds__(256) void scatter_rows_kernel(SegPtrs sp, int64_t d, const bf16* __restrict__ y,
                                                           const bf16* __restrict__ delta) {
  const int64_t row = blockIdx.x;
  const int s = find_seg(sp.off, sp.n, row);
  bf16* dst = reinterpret_cast<bf16*>(const_cast<void*>(sp.ptr[s])) + (row - sp.off[s]) * d;
  const bf16* src = y + row * d;
  const bf16* dl = delta ? delta + row * d : nullptr;
  if (sp.vec) {
    const int64_t nv = d >> 3;
    for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) {
      u32x4 v = reinterpret_cast<const u32x4*>(src)[i];
      if (dl) {
        float a[8], b[8];
        unpack8(v, a);
        unpack8(reinterpret_cast<const u32x4*>(dl)[i], b);
        bf16x8 o;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = f2bf(a[j] + b[j]);
        v = __builtin_bit_cast(u32x4, o);
      }
      reinterpret_cast<u32x4*>(dst)[i] = v;
    }
  } else {
    for (int64_t i = threadIdx.x; i < d; i += blockDim.x) {
      float v = bf2f(src[i]);
      if (dl) v += bf2f(dl[i]);
      dst[i] = dl ? f2bf(v) : src[i];
    }
  }
}

// ------------------------------------------------------- LoRA epilogue ----
// Column blocks of a fused projection output and the LoRA state a round
// carries into the base kernel's epilogue.
constexpr int kMaxURow = SWL_MAX_LORA_BLOCKS * 64;  // shrink row: blocks x rank (<= 64)

struct LoraEpi {
  const swl_lora_entry* table;  // device
  const float* u;               // [usplit][u_rows][u_ld] fp32 shrink partials
  int32_t usplit, u_ld;
  int64_t u_split_stride;       // u_rows * u_ld
  int32_t nblk;
  int64_t blk_start[SWL_MAX_LORA_BLOCKS + 1];
};

__device__ __forceinline__ int find_blk(const LoraEpi L, int64_t n) {
  int b = 0;
#pragma unroll
  for (int i = 1; i < SWL_MAX_LORA_BLOCKS; ++i)
    if (i < L.nblk && n >= L.blk_start[i]) b = i;
  return b;
}

__device__ __forceinline__ int64_t blk_start_of(const LoraEpi L, int b) {
  int64_t v = 0;
#pragma unroll
  for (int i = 0; i <= SWL_MAX_LORA_BLOCKS; ++i)
    if (i == b) v = L.blk_start[i];
  return v;
}

// delta for 4 consecutive output columns (all inside block `blk`, first one at
// in-block row `nin`) of the token whose shrink row is `urow`:
// scale * sum_q u[q] * B[nin + j][q].
__device__ __forceinline__ void lora_delta4(const LoraEpi L, const swl_lora_entry* ep, int urow, int blk,
                                            int64_t nin, float (&d)[4]) {
  const int r = ep->rank;
  const float scale = ep->scale;
  const bf16* b0 = reinterpret_cast<const bf16*>(ep->b[blk]) + nin * r;
  const float* up = L.u + (int64_t)urow * L.u_ld + blk * r;
  d[0] = d[1] = d[2] = d[3] = 0.f;
  if ((r & 7) == 0) {
    for (int q = 0; q < r; q += 8) {
      float uq[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) uq[i] = 0.f;
      for (int s = 0; s < L.usplit; ++s) {
        const f32x4* p = reinterpret_cast<const f32x4*>(up + s * L.u_split_stride + q);
        f32x4 a = p[0], c = p[1];
        uq[0] += a[0]; uq[1] += a[1]; uq[2] += a[2]; uq[3] += a[3];
        uq[4] += c[0]; uq[5] += c[1]; uq[6] += c[2]; uq[7] += c[3];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float bv[8];
        unpack8(ld16(b0 + (int64_t)j * r + q), bv);
#pragma unroll
        for (int i = 0; i < 8; ++i) d[j] += uq[i] * bv[i];
      }
    }
  } else {
    for (int q = 0; q < r; ++q) {
      float uq = 0.f;
      for (int s = 0; s < L.usplit; ++s) uq += up[s * L.u_split_stride + q];
#pragma unroll
      for (int j = 0; j < 4; ++j) d[j] += uq * bf2f(ldg(b0 + (int64_t)j * r + q));
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) d[j] *= scale;
}

__device__ __forceinline__ float lora_delta1(const LoraEpi L, const swl_lora_entry* ep, int urow, int64_t n) {
  const int blk = find_blk(L, n);
  const int r = ep->rank;
  const bf16* b0 = reinterpret_cast<const bf16*>(ep->b[blk]) + (n - blk_start_of(L, blk)) * r;
  const float* up = L.u + (int64_t)urow * L.u_ld + blk * r;
  float d = 0.f;
  for (int q = 0; q < r; ++q) {
    float uq = 0.f;
    for (int s = 0; s < L.usplit; ++s) uq += up[s * L.u_split_stride + q];
    d += uq * bf2f(ldg(b0 + q));
  }
  return d * ep->scale;
}

// Store 4 consecutive columns n..n+3 of one row (bf16, one rounding).
__device__ __forceinline__ void store4_bf16(const float (&v)[4], int64_t n, int64_t N, bf16* yrow) {
  if (n + 3 < N && ((reinterpret_cast<uintptr_t>(yrow + n) & 7) == 0)) {
    bf16 o0 = f2bf(v[0]), o1 = f2bf(v[1]), o2 = f2bf(v[2]), o3 = f2bf(v[3]);
    u32x2 pk;
    pk[0] = (uint32_t)__builtin_bit_cast(uint16_t, o0) | ((uint32_t)__builtin_bit_cast(uint16_t, o1) << 16);
    pk[1] = (uint32_t)__builtin_bit_cast(uint16_t, o2) | ((uint32_t)__builtin_bit_cast(uint16_t, o3) << 16);
    stg(yrow + n, pk);
  } else {
    for (int j = 0; j < 4; ++j)
      if (n + j < N) stg(yrow + n + j, f2bf(v[j]));
  }
}

// Finalise 4 consecutive columns n..n+3 of one token and store them (bf16).
// lora_idx < 0: no adapter for this token.
__device__ __forceinline__ void epilogue_store4(float (&v)[4], int64_t n, int64_t N, const bf16* bias,
                                                const LoraEpi L, int lora_idx, int urow, bf16* yrow) {
  if (bias) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (n + j < N) v[j] += bf2f(bias[n + j]);
  }
  if (lora_idx >= 0) {
    const swl_lora_entry* ep = L.table + lora_idx;
    const int blk = find_blk(L, n);
    const int64_t bs = blk_start_of(L, blk), be = blk_start_of(L, blk + 1);
    if (n + 3 < N && n + 3 < be) {
      float d[4];
      lora_delta4(L, ep, urow, blk, n - bs, d);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] += d[j];
    } else {
      for (int j = 0; j < 4; ++j)
        if (n + j < N) v[j] += lora_delta1(L, ep, urow, n + j);
    }
  }
  store4_bf16(v, n, N, yrow);
}

// ------------------------------------------------------ skinny (M<=64) ----
// Decode-shaped projections (<= 64 tokens) run as two kernels:
//   split_kernel     workgroup = 8 waves over 8 row tiles (16 rows each) and
//                    one K-slice.  The K-slice of every token's activation row
//                    is staged once in LDS and shared by the 8 waves
//                    (activation fetch is tokens/128 of the weight bytes);
//                    each wave streams its 16 rows from HBM into MFMA
//                    A-fragments and writes fp32 partial sums for its K-slice.
//                    The LoRA shrink rides along: the stacked A of each
//                    distinct adapter of the round forms extra row tiles after
//                    W's, streamed and multiplied the same way, and each token
//                    keeps only the columns of its own adapter's rows.
//   epilogue_kernel  sums the K-slice partials, adds bias and the LoRA expand,
//                    rounds once to bf16 and stores each token's row into its
//                    slot buffer (the scatter).
constexpr int kKDepth = 8;            // k-steps of W in flight per wave

struct SplitArgs {
  // base projection -> part[ks][tok][N]; LoRA shrink -> u[ks][tok][u_ld]
  const bf16* w;                      // row-major [N][K], or fragment tiles (w_packed)
  int64_t N, K;
  int32_t ntok;
  int32_t w_packed;
  int32_t a_packed;                   // the adapter groups' stacked A are fragment tiles too
  int32_t n_ks, n_workers;            // grid = n_ks x n_workers workgroups
  int32_t total_steps, ks_steps;      // k-steps of 32 in K; max per K-slice
  int32_t n_wtiles, n_tiles;          // W row tiles (ceil(N / 16)); all tiles incl. adapter rows
  int32_t ngroups, u_ld;
  float* part;
  float* u;
  int64_t u_split_stride;             // ntok * u_ld
  const bf16* x[kSkinnyMaxTok];
  // RMSNorm on staging (gamma != null): x = bf16(bf16(h * r) * gamma),
  // r = rsqrt(sum(ss[tok][0 .. ss_n)) / K + eps)
  const bf16* gamma;
  const float* ss;
  int32_t ss_n, ss_stride;
  float eps;
  const bf16* g_a[kSkinnyMaxTok];     // stacked lora_A [g_arows][K] of adapter group g
  int32_t g_arows[kSkinnyMaxTok];
  int32_t g_tile0[kSkinnyMaxTok + 1]; // first row tile of group g past W's; [ngroups] = total
  int8_t tok_grp[kSkinnyMaxTok];      // adapter group of each token, -1 for none
};

// LoRA shrink of the packed prefill batch: u[ks][row][q] = x[row] . A[q]
// over K-slice ks, for every segment with an adapter.  Work items are
// (64-row tile of the segment, 64-row block of its stacked A) pairs, item0 is
// their prefix over the segments.
struct ShrinkGemmArgs {
  const bf16* xs[kMaxSeg];  // rows of segment j (row stride K), in place or in the packed batch
  float* u;               // [n_ks][T][u_ld]
  int64_t K, u_split_stride;
  int32_t n_seg, n_ks, u_ld, total_steps;
  int32_t item0[kMaxSeg + 1];
  int32_t row0[kMaxSeg], rows[kMaxSeg], arows[kMaxSeg];
  const bf16* a[kMaxSeg];
};

struct EpiArgs {
  const float* part;
  int32_t n_ks, ntok;
  int64_t N;
  const bf16* bias;
  int32_t has_lora;
  // output fusions (swl_round_fusion.out_mode): 1 residual + sums of squares,
  // 2 SiLU-mul of the gate | up halves, 3 RoPE + KV-page append
  float* ss_out;
  int32_t ss_stride;
  int64_t inter;
  bf16* kc;
  bf16* vc;
  const int32_t* bt;
  const int32_t* seqlens;
  const int64_t* pos;
  const bf16* cs;
  int64_t max_blocks, num_blocks, max_pos;
  int32_t hq, hkv, bs;
  bf16* y[kSkinnyMaxTok];
  int32_t lora[kSkinnyMaxTok];
  int32_t urow[kSkinnyMaxTok];
  LoraEpi L;
};


// W fragment of k-step s of a K-slice with `n` steps; steps past the end read
// the slice's last step again (in bounds).  The caller zeroes them.
// SS: elements between consecutive k-steps (32 for a row-major row, 512 for
// fragment tiles).
template <int SS>
__device__ __forceinline__ u32x4 ld_w_step(const bf16* wp, int s, int n) {
  return ldg16_nt(wp + SS * (s < n ? s : n - 1));
}

template <int SS, int D>
__device__ __forceinline__ void issue_w(u32x4 (&w)[D], const bf16* wp, int n) {
#pragma unroll
  for (int d = 0; d < D; ++d) w[d] = ld_w_step<SS>(wp, d, n);
}

// W (one row per lane, k-group per lane quarter) streamed D steps at a time,
// the D loads of a group issued back to back (consecutive 64-byte pieces of
// each row reach the memory controller together, which streams faster from
// HBM than a rolling one-step-ahead prefetch); B-fragments of TT token tiles
// read from LDS (fragment order: step s, tile t at xl + (s * TT + t) *
// tstride).  The caller has already issued the first group into w[].  nsteps
// (a multiple of D) are run; W steps from nw on contribute zero.
template <int TT, int D, int SS>
__device__ __forceinline__ void kloop_lds(f32x4 (&acc)[TT], u32x4 (&w)[D], const bf16* wp, const bf16* xl,
                                          int tstride, int nsteps, int nw) {
  const int niter = (nsteps + D - 1) / D;
  for (int it = 0; it < niter; ++it) {
    const int base = it * D;
    if (it > 0) {
#pragma unroll
      for (int d = 0; d < D; ++d) w[d] = ld_w_step<SS>(wp, base + d, nw);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const u32x4 wd = (base + d < nw) ? w[d] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int t = 0; t < TT; ++t) acc[t] = mfma16(wd, lds16(xl + ((base + d) * TT + t) * tstride), acc[t]);
    }
  }
}

// One workgroup per (item, K-slice): 4 waves, each 16 token rows x the 64
// A rows of the item's block (4 MFMA tiles, A rows as the A-operand so the
// fp32 results land as 4 consecutive q per lane).  The K-slice runs in
// groups of 8 k-steps: every thread issues its 8 loads of the group at once
// (one 16-byte piece of the A block, one of its wave's token rows), the A
// block is shared through LDS in fragment order (a wave's fragment read is
// one contiguous 1 KiB), then the 32 MFMAs of the group.
__global__ __launch_bounds__(256) void shrink_gemm_kernel(ShrinkGemmArgs a) {
  constexpr int D = 8;
  // [k-step][A tile j][lane] fragments of the group's A block
  __shared__ __attribute__((aligned(16))) u32x4 als[D][4][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int ks = blockIdx.x % a.n_ks, item = blockIdx.x / a.n_ks;
  int lo = 0, hi = a.n_seg - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.item0[mid] <= item) lo = mid; else hi = mid - 1;
  }
  const int s = lo;
  const int nab = (a.arows[s] + 63) / 64;
  const int li = item - a.item0[s];
  const int rt = li / nab, ab = li - rt * nab;
  const int st0 = (int)((int64_t)a.total_steps * ks / a.n_ks);
  const int st1 = (int)((int64_t)a.total_steps * (ks + 1) / a.n_ks);
  const int nst = st1 - st0;
  const int tr = rt * 64 + wv * 16 + (lane & 15);  // token row of this lane within the segment
  const bf16* xp = a.xs[s] + (int64_t)min(tr, a.rows[s] - 1) * a.K + (int64_t)st0 * 32 + 8 * (lane >> 4);
  // A loader: thread t takes A row t / 4 of the block, 16-byte chunk t % 4
  // of each k-step, stored as lane (row % 16) + 16 chunk of tile row / 16
  const int ar = threadIdx.x >> 2, ac = threadIdx.x & 3;
  const bf16* ag = a.a[s] + (int64_t)min(ab * 64 + ar, a.arows[s] - 1) * a.K + (int64_t)st0 * 32 + 8 * ac;
  const int aj = ar >> 4, al = (ar & 15) + 16 * ac;
  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < nst; g += D) {
    u32x4 av[D], xv[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int st = 32 * (g + d < nst ? g + d : nst - 1);
      av[d] = ldg16(ag + st);
      xv[d] = ldg16(xp + st);
    }
    if (g > 0) __syncthreads();  // every wave is past its reads of the previous group
#pragma unroll
    for (int d = 0; d < D; ++d) als[d][aj][al] = av[d];
    __syncthreads();
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (g + d >= nst) break;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = mfma16(als[d][j][lane], xv[d], acc[j]);
    }
  }
  if (tr >= a.rows[s]) return;
  float* urow = a.u + ks * a.u_split_stride + (int64_t)(a.row0[s] + tr) * a.u_ld;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int q0 = ab * 64 + 16 * j + 4 * (lane >> 4);
    if (q0 < a.u_ld) *reinterpret_cast<f32x4*>(urow + q0) = acc[j];
  }
}

// u[0] += u[1] + ... + u[n_ks - 1] over [nvec] float4 (the shrink partials
// folded once, so the tiled epilogue's expand reads a single split).
// Every split's load is issued before the first add (n_ks <= kFoldMax),
// then the sum runs in split order.
constexpr int kFoldMax = 16;
__global__ __launch_bounds__(256) void u_fold_kernel(float* u, int64_t split_stride, int n_ks, int64_t nvec) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nvec) return;
  f32x4 v[kFoldMax];
#pragma unroll
  for (int k = 0; k < kFoldMax; ++k)
    if (k < n_ks) v[k] = reinterpret_cast<const f32x4*>(u + k * split_stride)[i];
  f32x4 s = v[0];
#pragma unroll
  for (int k = 1; k < kFoldMax; ++k)
    if (k < n_ks) s += v[k];
  reinterpret_cast<f32x4*>(u)[i] = s;
}

// LoRA expand of a packed batch (swl_lora_segmented_bf16): one thread per
// (row, 4 consecutive columns); y = delta (mode 0) or y + delta rounded
// once (mode 1), delta from the row's folded shrink row and its adapter's
// lora_B block; rows of segments without an adapter get 0 (mode 0) or are
// left as they are (mode 1).
struct ExpandArgs {
  bf16* y;
  int64_t N;
  int32_t mode, n_seg;
  int64_t off[kMaxSeg + 1];
  int32_t seg_lora[kMaxSeg];
  LoraEpi L;
};

__global__ __launch_bounds__(256) void lora_expand_kernel(ExpandArgs a) {
  const int64_t t = blockIdx.y;
  const int64_t n = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= a.N) return;
  const int s = find_seg(a.off, a.n_seg, t);
  const int lidx = a.seg_lora[s];
  if (a.mode == 1 && lidx < 0) return;
  bf16* yrow = a.y + t * a.N;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (a.mode == 1)
    for (int j = 0; j < 4; ++j)
      if (n + j < a.N) v[j] = bf2f(yrow[n + j]);
  epilogue_store4(v, n, a.N, nullptr, a.L, lidx, (int)t, yrow);
}

// Row pointer (this lane's row, at the K-slice start) of row tile `tile`: a
// tile of W, or a tile of one adapter group's stacked A (rows past the end of
// either re-read its last row; their results are never stored).  grp: -1 for
// W, the group for adapter rows.  Fragment tiles (W with w_packed, A with
// a_packed): this lane's 16 bytes of the slice's first k-step block; rows
// past the end are zero rows of the tile.
__device__ __forceinline__ const bf16* tile_rows(const SplitArgs& a, int tile, int lane, int64_t kbeg, int& grp,
                                                 int& qrow0) {
  const bf16* row;
  grp = -1;
  qrow0 = 0;
  if (tile < a.n_wtiles && a.w_packed) {
    // fragment tiles: this lane's 16 bytes of the slice's first k-step block
    return a.w + ((int64_t)tile * a.total_steps + (kbeg >> 5)) * 512 + 8 * lane;
  }
  if (tile < a.n_wtiles) {
    const int64_t r = (int64_t)tile * 16 + (lane & 15);
    row = a.w + (r < a.N ? r : a.N - 1) * a.K;
  } else {
    const int lt = tile - a.n_wtiles;
    int g = 0;
    while (g + 1 < a.ngroups && a.g_tile0[g + 1] <= lt) ++g;
    qrow0 = (lt - a.g_tile0[g]) * 16;
    grp = g;
    if (a.a_packed) return a.g_a[g] + ((int64_t)(lt - a.g_tile0[g]) * a.total_steps + (kbeg >> 5)) * 512 + 8 * lane;
    row = a.g_a[g] + (int64_t)min(qrow0 + (lane & 15), a.g_arows[g] - 1) * a.K;
  }
  return row + kbeg + 8 * (lane >> 4);
}

// Workgroup (K-slice ks, worker j): stages the K-slice of every token row in
// LDS once, then each wave walks row tiles j*WAVES + wv, + n_workers*WAVES,
// ... (W's tiles, then the adapter tiles), issuing the next tile's first W
// group before storing the current tile's partials so the stores and the
// loads overlap.  No workgroup waits on another.
// Resident waves per SIMD the registers are sized for: 6 for three 8-wave
// workgroups per CU up to 32 token rows (80 VGPRs), 4 for one 16-wave
// workgroup per CU or wider accumulators (128 VGPRs).
template <int TT, int WAVES, int KD = kKDepth>
__global__ __launch_bounds__(WAVES * 64, (TT <= 2 && WAVES < 16) ? 6 : 4) void split_kernel(SplitArgs a) {
  extern __shared__ __attribute__((aligned(16))) bf16 xs[];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int ks = blockIdx.x % a.n_ks, wk = blockIdx.x / a.n_ks;
  const int st0 = (int)((int64_t)a.total_steps * ks / a.n_ks);
  const int st1 = (int)((int64_t)a.total_steps * (ks + 1) / a.n_ks);
  const int nst = st1 - st0;
  const int npad = (nst + KD - 1) / KD * KD;
  const int64_t kbeg = (int64_t)st0 * 32;
  const int tstride = a.n_workers * WAVES;

  // tiles wk + n_workers * (wv + WAVES * m): the slice's tiles dealt over
  // its workers first, then over each worker's waves
  int tile = wk + a.n_workers * wv;
  int grp = -1, qrow0 = 0;
  const bf16* wp = nullptr;
  u32x4 w[KD];
  // fragment-tile W: k-steps 512 elements apart (uniform per tile)
  auto packed = [&](int t) { return t < a.n_wtiles ? a.w_packed != 0 : a.a_packed != 0; };

  // RMSNorm inputs first, so they return ahead of the weight stream: the
  // slice of gamma (512 elements per DMA block, clamped to the slice) into
  // LDS past the activation blocks, and each token row's partial sums of
  // squares, thread (token t / 16, partial t % 16 + 16 i) one load each for
  // up to 16 partials per row
  char* gs = reinterpret_cast<char*>(xs) + a.ks_steps * TT * 1024;
  float* rs = reinterpret_cast<float*>(gs + (a.ks_steps * 32 + 511) / 512 * 1024);
  constexpr int kTokPass = WAVES * 4;                          // tokens per pass (16 threads each)
  constexpr int kPass = (TT * 16 + kTokPass - 1) / kTokPass;   // passes over the token rows
  const int tk16 = threadIdx.x >> 4, j16 = threadIdx.x & 15;
  float ssp[kPass];
  if (a.gamma) {
    for (int i = wv; i < (npad * 32 + 511) / 512; i += WAVES) {
      const int64_t k = min(kbeg + (int64_t)i * 512 + 8 * lane, kbeg + (int64_t)nst * 32 - 8);
      __builtin_amdgcn_global_load_lds((gbl_ptr)(a.gamma + k), (lds_ptr)(gs + i * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int p = 0; p < kPass; ++p) {
      const int tk = tk16 + p * kTokPass;
      ssp[p] = (tk < a.ntok && j16 < a.ss_n) ? ldg_f32(a.ss + (int64_t)tk * a.ss_stride + j16) : 0.f;
    }
  }
  if (tile < a.n_tiles) {
    wp = tile_rows(a, tile, lane, kbeg, grp, qrow0);
    if (packed(tile))
      issue_w<512>(w, wp, nst);
    else
      issue_w<32>(w, wp, nst);
  }

  // Stage the activation K-slice in LDS in MFMA B-fragment order: block
  // (step s, token tile t) holds 64 lanes x 16 B, lane l = token 16t + l%16,
  // k-group l/16, so the k-loop's ds_read_b128 is conflict-free.  Token rows
  // past ntok load row 0 (their results are never stored); steps past the
  // slice reload its last step (the matching W fragments are zero).
  const int nblk = npad * TT;
  auto xsrc = [&](int i) {
    const int st = i / TT, t = i - st * TT;
    const int tk = 16 * t + (lane & 15);
    return a.x[tk < a.ntok ? tk : 0] + kbeg + 32 * (st < nst ? st : nst - 1) + 8 * (lane >> 4);
  };
  // LDS-DMA loads (global_load_lds_dwordx4), no VGPR round trip
  for (int i = wv; i < nblk; i += WAVES)
    __builtin_amdgcn_global_load_lds((gbl_ptr)xsrc(i), (lds_ptr)(reinterpret_cast<char*>(xs) + i * 1024), 16, 0, 0);
  // Residual-stream rows are RMS-normalised in place after staging: each
  // token row's r = rsqrt(sum of its partial sums of squares / K + eps) goes
  // to LDS next to gamma; after the barrier every wave rescales the blocks it
  // staged: h * r rounded to bf16, times gamma, rounded again, as
  // LlamaRMSNorm does.  Rows with more than 16 partials add the rest here.
  if (a.gamma) {
#pragma unroll
    for (int p = 0; p < kPass; ++p) {
      const int tk = tk16 + p * kTokPass;
      float v = ssp[p];
      if (tk < a.ntok)
        for (int j = j16 + 16; j < a.ss_n; j += 16) v += ldg_f32(a.ss + (int64_t)tk * a.ss_stride + j);
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      v += __shfl_xor(v, 8, 64);
      if (j16 == 0 && tk < TT * 16) rs[tk] = tk < a.ntok ? rsqrtf(v / (float)a.K + a.eps) : 0.f;
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this wave's LDS-DMA (and W) loads have landed
  __syncthreads();
  if (a.gamma) {
    for (int i = wv; i < nblk; i += WAVES) {
      const int st = i / TT, t = i - st * TT;
      const float r = rs[16 * t + (lane & 15)];
      u32x4* px = reinterpret_cast<u32x4*>(reinterpret_cast<char*>(xs) + i * 1024 + 16 * lane);
      float hv[8], gv[8];
      unpack8(*px, hv);
      unpack8(*reinterpret_cast<const u32x4*>(gs + (32 * st + 8 * (lane >> 4)) * 2), gv);
      bf16x8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = f2bf(bf2f(f2bf(hv[j] * r)) * gv[j]);
      *px = __builtin_bit_cast(u32x4, o);
    }
    __syncthreads();
  }

  const bf16* xl = xs + 8 * lane;  // block (s, t) at xs + (s * TT + t) * 512 elements
  // The fp32 partials are stored written through to memory (buffer stores
  // at system scope, sc0 sc1) instead of as dirty L2 lines: the epilogue
  // reads them from every XCD anyway, and the QKV and Down rounds measure
  // about 1 us faster this way.  The buffer's range covers the whole
  // partial array (the hardware drops stores past it).
  const __amdgpu_buffer_rsrc_t prsrc =
      __builtin_amdgcn_make_buffer_rsrc(a.part, 0, (int)((int64_t)a.n_ks * a.ntok * a.N * 4), 0x00020000);
  while (tile < a.n_tiles) {
    f32x4 acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (packed(tile))
      kloop_lds<TT, KD, 512>(acc, w, wp, xl, 512, npad, nst);
    else
      kloop_lds<TT, KD, 32>(acc, w, wp, xl, 512, npad, nst);

    const int cur = tile, cgrp = grp, cq = qrow0;
    tile += tstride;
    if (tile < a.n_tiles) {
      wp = tile_rows(a, tile, lane, kbeg, grp, qrow0);
      if (packed(tile))
        issue_w<512>(w, wp, nst);
      else
        issue_w<32>(w, wp, nst);
    }

    if (cgrp < 0) {
      const int64_t n0 = (int64_t)cur * 16 + 4 * (lane >> 4);
      if (n0 < a.N) {
        const bool vec = (n0 + 3 < a.N) && ((a.N & 3) == 0);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          const int tok = 16 * t + (lane & 15);
          if (tok >= a.ntok) continue;
          float* dst = a.part + ((int64_t)ks * a.ntok + tok) * a.N + n0;
          if (vec) {
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[t]), prsrc,
                                                   (int)((((int64_t)ks * a.ntok + tok) * a.N + n0) * 4), 0,
                                                   kStoreSys);
          } else {
            for (int j = 0; j < 4; ++j)
              if (n0 + j < a.N) dst[j] = acc[t][j];
          }
        }
      }
    } else {
      // shrink rows cq.. of adapter group cgrp: only that group's tokens keep
      // them (u_ld covers every padded tile, so the f32x4 store stays in the row)
      const int q = cq + 4 * (lane >> 4);
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const int tok = 16 * t + (lane & 15);
        if (tok < a.ntok && a.tok_grp[tok] == cgrp)
          *reinterpret_cast<f32x4*>(a.u + ks * a.u_split_stride + (int64_t)tok * a.u_ld + q) = acc[t];
      }
    }
  }
}

// One workgroup per (64 Q column quads, token); the four lane groups of a
// wave (lanes l, l^16, l^32, l^48) share 16 quads, Q times over (quad slot q
// of the lane at column offset q x 256 gridDim.x, so each slot of the grid
// is one contiguous run of columns).  Each lane group sums every fourth
// K-slice partial of the quads (all its loads issued at once), the groups
// fold with shuffles and lane group g keeps column g of each quad.  The
// token's LoRA shrink row is reduced over the K-slices by the whole
// workgroup into LDS, the lane's rows of lora_B having been requested
// before the reductions; bias and the expand are added and the result is
// rounded once to bf16.  MODE (swl_round_fusion.out_mode) then decides what
// is stored: 0 the row (the scatter), 1 the residual update and its sum of
// squares, 2 SiLU(gate) * up (each lane owns a gate and an up column of
// each quad slot), 3 the row with RoPE on q and k, k and v also appended to
// their KV pages.  Q > 1 (modes 0 and 2) takes the same columns in fewer
// workgroups, for rounds whose grid would not be resident at once.
template <int MODE, int Q = 1>
__global__ __launch_bounds__(256, (MODE == 2 ? 2 : 1) * Q >= 4 ? 4 : 1) void epilogue_kernel(EpiArgs a) {
  static_assert(Q == 1 || MODE == 0 || MODE == 2, "modes 1 and 3 reduce or exchange over one quad slot");
  constexpr int C = MODE == 2 ? 2 : 1;  // column sets per quad slot (gate, up)
  constexpr int CQ = C * Q;             // column sets per lane: set c = slot c / C, gate/up c % C
  __shared__ float us[kMaxURow];
  __shared__ float ured[256];
  __shared__ float xch[256];
  const int tok = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int kg = lane >> 4;
  const int64_t ncols = MODE == 2 ? a.inter : a.N;  // output columns
  const int64_t qoff = (int64_t)gridDim.x * 256;    // columns between quad slots
  const int64_t nq = (((int64_t)blockIdx.x * 4 + wv) * 16 + (lane & 15)) * 4;  // first column of the quad
  const int64_t n = nq + kg;                                                   // this lane's column
  const bool live = n < ncols;
  const int lora = a.has_lora ? a.lora[tok] : -1;
  const bool vec = (a.N & 3) == 0 && (MODE != 2 || (a.inter & 3) == 0);
  // output column of set c (within the ncols) and whether it exists
  auto col_of = [&](int c) { return n + (c / C) * qoff; };
  auto live_of = [&](int c) { return col_of(c) < ncols; };

  // values the output fusions need after the reduction, requested first:
  // the residual element (1); the position and the cache length (3)
  bf16* yrow = a.y[tok];
  float hres = 0.f;
  if constexpr (MODE == 1) {
    if (live) hres = bf2f(yrow[n]);
  }
  int64_t pos = -1, slen = -1;
  if constexpr (MODE == 3) {
    pos = a.pos[tok];
    slen = a.seqlens[tok];
  }

  // lora_B rows of this lane's column(s) (rank <= 16, multiple of 8: registers)
  const swl_lora_entry* ep = lora >= 0 ? a.L.table + lora : nullptr;
  int r = 0, blk[CQ];
  const bf16* brow[CQ];
  u32x4 bq[CQ][2];
#pragma unroll
  for (int c = 0; c < CQ; ++c) {
    blk[c] = 0;
    brow[c] = nullptr;
    bq[c][0] = bq[c][1] = u32x4{0u, 0u, 0u, 0u};
  }
  if (ep) {
    r = ep->rank;
#pragma unroll
    for (int c = 0; c < CQ; ++c) {
      const bool lc = live_of(c);
      const int64_t nc = (lc ? col_of(c) : 0) + (c % C) * a.inter;
      blk[c] = find_blk(a.L, nc);
      brow[c] = reinterpret_cast<const bf16*>(ep->b[blk[c]]) + (nc - blk_start_of(a.L, blk[c])) * r;
      if (lc && r <= 16 && (r & 7) == 0) {
        bq[c][0] = ldg16_nt(brow[c]);
        if (r == 16) bq[c][1] = ldg16_nt(brow[c] + 8);
      }
    }
  }

  // partial sums of the quad(s) over K-slices kg, kg + 4, ...: the first
  // batch of each lane group requested together (all of them up to 32
  // K-slices, 8 with two column sets)
  const int64_t kstride = (int64_t)a.ntok * a.N;
  auto ld_part = [&](int c, int ks) {
    f32x4 q = f32x4{0.f, 0.f, 0.f, 0.f};
    const int64_t nqc = nq + (c / C) * qoff;  // first column of the set's quad
    const int64_t qc = nqc + (c % C) * a.inter;
    if (nqc < ncols && ks < a.n_ks) {
      const float* pk = a.part + (int64_t)tok * a.N + qc + ks * kstride;
      if (vec) {  // read once: non-temporal
        q = __builtin_nontemporal_load((const __attribute__((address_space(1))) f32x4*)(const void*)pk);
      } else {
        for (int e = 0; e < 4; ++e)
          if (nqc + e < ncols) q[e] = pk[e];
      }
    }
    return q;
  };
  // first batch per lane group and set: 8 K-slices with one set, 2 with
  // two, 1 with four (registers for four waves per SIMD)
  constexpr int B0 = CQ >= 4 ? 1 : CQ >= 2 ? 2 : 8;
  f32x4 q0[CQ][B0];
#pragma unroll
  for (int c = 0; c < CQ; ++c)
#pragma unroll
    for (int j = 0; j < B0; ++j) q0[c][j] = ld_part(c, kg + 4 * j);

  // the token's shrink row over the K-slices: thread (split sp, row q) sums
  // splits sp, sp + nsp, ... (the first four requested here, with the
  // partials)
  const int ur = ep ? a.L.u_ld : 1, nsp = 256 / ur;
  const int uq = threadIdx.x % ur, usp = threadIdx.x / ur;
  const float* up = ep ? a.L.u + (int64_t)a.urow[tok] * a.L.u_ld + uq : nullptr;
  float u4[4] = {0.f, 0.f, 0.f, 0.f};
  if (ep && usp < nsp) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = usp + i * nsp;
      if (k < a.L.usplit) u4[i] = up[k * a.L.u_split_stride];
    }
  }

  // RoPE factors and the KV page slot (3), requested while the partials are
  // in flight
  const int d = (int)(n & 127), hh = (int)(n >> 7);
  const bool is_q = MODE == 3 && hh < a.hq, is_k = MODE == 3 && !is_q && hh < a.hq + a.hkv;
  float rc = 1.f, rsn = 0.f;
  bool rot = false;
  int64_t kv_dst = -1;
  if constexpr (MODE == 3) {
    if (live && (is_q || is_k) && pos >= 0 && pos < a.max_pos) {
      rot = true;
      rc = bf2f(a.cs[pos * 128 + (d & 63)]);
      rsn = bf2f(a.cs[pos * 128 + 64 + (d & 63)]);
    }
    if (live && !is_q && slen >= 0 && slen / a.bs < a.max_blocks) {
      const int32_t pb = a.bt[(int64_t)tok * a.max_blocks + slen / a.bs];
      if (pb >= 0 && pb < a.num_blocks) {
        const int kvh = is_k ? hh - a.hq : hh - a.hq - a.hkv;
        kv_dst = ((int64_t)pb * a.bs + slen % a.bs) * a.hkv * 128 + kvh * 128 + d;
      }
    }
  }

  f32x4 s[CQ];
#pragma unroll
  for (int c = 0; c < CQ; ++c) {
    s[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < B0; ++j) s[c] += q0[c][j];
    constexpr int NB = CQ >= 4 ? 4 : 8;  // later batches
    for (int ks0 = kg + 4 * B0; ks0 < a.n_ks; ks0 += 4 * NB) {
      f32x4 q[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j) q[j] = ld_part(c, ks0 + 4 * j);
#pragma unroll
      for (int j = 0; j < NB; ++j) s[c] += q[j];
    }
  }

  if (ep) {  // uniform over the workgroup
    if (usp < nsp) {
      float acc = (u4[0] + u4[1]) + (u4[2] + u4[3]);
      for (int k = usp + 4 * nsp; k < a.L.usplit; k += nsp) acc += up[k * a.L.u_split_stride];
      ured[threadIdx.x] = acc;
    }
    __syncthreads();
    if ((int)threadIdx.x < ur) {
      float acc = 0.f;
      for (int i = 0; i < nsp; ++i) acc += ured[i * ur + threadIdx.x];
      us[threadIdx.x] = acc;
    }
    __syncthreads();
  }

  // fold the four lane groups; lane group kg keeps component kg; then bias
  // and the LoRA expand
  float v[CQ];
#pragma unroll
  for (int c = 0; c < CQ; ++c) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[c][e] += __shfl_xor(s[c][e], 16, 64);
      s[c][e] += __shfl_xor(s[c][e], 32, 64);
    }
    v[c] = kg == 0 ? s[c][0] : kg == 1 ? s[c][1] : kg == 2 ? s[c][2] : s[c][3];
    if (!live_of(c)) continue;
    const int64_t nc = col_of(c) + (c % C) * a.inter;
    if (a.bias) v[c] += bf2f(a.bias[nc]);
    if (ep) {
      const float* ub = us + blk[c] * r;
      float d = 0.f;
      if (r <= 16 && (r & 7) == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (8 * h >= r) break;
          float bv[8];
          unpack8(bq[c][h], bv);
#pragma unroll
          for (int i = 0; i < 8; ++i) d += ub[8 * h + i] * bv[i];
        }
      } else if ((r & 7) == 0) {
        for (int q = 0; q < r; q += 8) {
          float bv[8];
          unpack8(ld16(brow[c] + q), bv);
#pragma unroll
          for (int i = 0; i < 8; ++i) d += ub[q + i] * bv[i];
        }
      } else {
        for (int q = 0; q < r; ++q) d += ub[q] * bf2f(brow[c][q]);
      }
      v[c] += d * ep->scale;
    }
  }

  if constexpr (MODE == 0) {
#pragma unroll
    for (int c = 0; c < CQ; ++c)
      if (live_of(c)) yrow[col_of(c)] = f2bf(v[c]);
  } else if constexpr (MODE == 1) {
    // h = bf16(h + out); the workgroup's sum of squares of the new h
    float sq = 0.f;
    if (live) {
      const bf16 hn = f2bf(hres + bf2f(f2bf(v[0])));
      yrow[n] = hn;
      sq = bf2f(hn) * bf2f(hn);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sq += __shfl_xor(sq, o, 64);
    if (lane == 0) ured[wv] = sq;
    __syncthreads();
    if (threadIdx.x == 0)
      a.ss_out[(int64_t)tok * a.ss_stride + blockIdx.x] = (ured[0] + ured[1]) + (ured[2] + ured[3]);
  } else if constexpr (MODE == 2) {
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      if (!live_of(2 * q)) continue;
      const float g = bf2f(f2bf(v[2 * q])), u = bf2f(f2bf(v[2 * q + 1]));
      yrow[col_of(2 * q)] = f2bf(bf2f(f2bf(g / (1.0f + __expf(-g)))) * u);
    }
  } else {
    // columns of this workgroup: 2 heads of 128; RoPE pairs (d, d + 64)
    const int cl = (wv * 16 + (lane & 15)) * 4 + kg;
    float x = bf2f(f2bf(v[0]));
    xch[cl] = x;
    __syncthreads();
    if (!live) return;
    if (rot) {
      const float other = xch[d < 64 ? cl + 64 : cl - 64];
      x = bf2f(f2bf(d < 64 ? x * rc - other * rsn : x * rc + other * rsn));
    }
    yrow[n] = f2bf(x);
    if (kv_dst >= 0) (is_k ? a.kc : a.vc)[kv_dst] = f2bf(x);
  }
}


// ------------------------------------------- decode: whole-K rounds -------
// Decode-shaped rounds with K <= 4096 (QKV, O, Gate+Up, LM head) without
// K-slice partials: a persistent workgroup of 8 waves per CU (two per SIMD,
// 256 registers each) keeps the K range of every token row in registers
// (wave w holds k-steps w * nsw .. + nsw of both 16-token tiles as MFMA B
// fragments, 128 registers at K = 4096, RMS-normalised on the way in when
// the round takes the residual stream), then walks its 16-row weight tiles
// (blockIdx.x, + gridDim.x, ...).  Each wave multiplies its k-steps of the
// tile, the next tile's 16 fragments are requested right after (128 KiB in
// flight per CU), the 8 wave partials are summed in LDS and the workgroup
// finishes the tile itself: bias and the LoRA expand, then the stores.  The LoRA shrink rows u = x . A^T of the round's adapters
// come from fullk_shrink_kernel, launched just before (K-slice partials,
// summed into LDS once per workgroup); with every adapter at rank 16 the
// lora_B rows a tile needs are moved into LDS by LDS-DMA together with the
// tile's weights.  The weights are in the fragment-tile layout of
// swl_pack_weight_bf16; thread (token, p) finishes tile rows p and p + 8.
constexpr int kFkWaves = 8;
constexpr int kFkMaxSteps = 16;  // k-steps per wave: K <= 8 * 16 * 32
constexpr int kFkShrinkKs = 4;   // K-slices of the shrink kernel

struct FullKArgs {
  const bf16* w;                // fragment tiles (swl_pack_weight_bf16)
  int64_t N, K;
  int32_t ntok, nsw, total_steps;
  int32_t n_tiles;              // ceil(N / 16)
  const bf16* x[32];
  bf16* y[32];
  // RMSNorm on the way in (gamma != null): x = bf16(bf16(h * r) * gamma)
  const bf16* gamma;
  const float* ss;
  int32_t ss_n, ss_stride;
  float eps;
  // LoRA
  int32_t has_lora, ngroups, u_ld, nblk;
  const swl_lora_entry* table;
  int64_t blk_start[SWL_MAX_LORA_BLOCKS + 1];
  const bf16* g_a[32];          // stacked lora_A [g_arows][K] of adapter group g
  int32_t g_arows[32];
  int32_t g_tile0[33];
  int8_t tok_grp[32];
  int32_t lora[32];             // table entry per token (-1: none)
  int32_t bdma;                 // every adapter of the round has rank 16: lora_B rows staged in LDS
  float* u;                     // [kFkShrinkKs][ntok][u_ld] shrink partials
  const bf16* bias;
};
typedef const __attribute__((address_space(4))) FullKArgs* fullk_args_ptr;

__device__ __forceinline__ int fk_blk(fullk_args_ptr a, int64_t n) {
  int b = 0;
#pragma unroll
  for (int i = 1; i < SWL_MAX_LORA_BLOCKS; ++i)
    if (i < a->nblk && n >= a->blk_start[i]) b = i;
  return b;
}


// RMSNorm row factors r = rsqrt(sum of the row's partial sums of squares / K
// + eps) into rsq[tk], one wave per token.
__device__ __forceinline__ void fk_row_factors(fullk_args_ptr a, float* rsq, int waves, int wv, int lane) {
  for (int tk = wv; tk < a->ntok; tk += waves) {
    float sq = 0.f;
    for (int j = lane; j < a->ss_n; j += 64) sq += a->ss[(int64_t)tk * a->ss_stride + j];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sq += __shfl_xor(sq, o, 64);
    if (lane == 0) rsq[tk] = rsqrtf(sq / (float)a->K + a->eps);
  }
}


// LoRA shrink of a whole-K round: workgroup (shrink tile t, K-slice ks),
// 4 waves over the slice's k-steps; tile t is 16 rows of adapter group g's
// stacked A, multiplied with every token row (its tokens keep the result).
// u[ks][tk][q0 + r] = partial sum over the slice.
__global__ __launch_bounds__(256) void fullk_shrink_kernel(FullKArgs args) {
  fullk_args_ptr a = (fullk_args_ptr)__builtin_amdgcn_kernarg_segment_ptr();
  __shared__ f32x4 red[4][2][64];
  __shared__ float rsq[32];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = blockIdx.x, ks = blockIdx.y;
  const int ntok = a->ntok;
  int g = 0;
  while (g + 1 < a->ngroups && a->g_tile0[g + 1] <= t) ++g;
  const int q0 = (t - a->g_tile0[g]) * 16;
  const int steps = a->total_steps / kFkShrinkKs;  // k-steps of the slice
  const int st0 = ks * steps;
  if (a->gamma) {
    fk_row_factors(a, rsq, 4, wv, lane);
    __syncthreads();
  }
  // wave wv takes the slice's k-steps wv * spw .. + spw (at most 8), every
  // load requested before the first product
  const int spw = (steps + 3) / 4;
  const int sw0 = st0 + wv * spw;
  const int nj = max(0, min(spw, st0 + steps - sw0));  // this wave's steps
  const bf16* ap = a->g_a[g] + (int64_t)min(q0 + (lane & 15), a->g_arows[g] - 1) * a->K + 8 * (lane >> 4);
  u32x4 wa[8], xv[8][2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int s = min(sw0 + j, st0 + steps - 1);
    wa[j] = ldg16(ap + 32 * s);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tk = 16 * tt + (lane & 15);
      const bool mine = j < nj && tk < ntok && a->tok_grp[tk] == g;
      xv[j][tt] = mine ? ldg16(a->x[tk] + 32 * s + 8 * (lane >> 4)) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (a->gamma && j < nj) {
      const u32x4 gv = ldg16(a->gamma + 32 * (sw0 + j) + 8 * (lane >> 4));
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int tk = 16 * tt + (lane & 15);
        xv[j][tt] = norm8(xv[j][tt], rsq[tk < ntok ? tk : 0], gv);
      }
    }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) acc[tt] = mfma16(wa[j], xv[j][tt], acc[tt]);
  }
  red[wv][0][lane] = acc[0];
  red[wv][1][lane] = acc[1];
  __syncthreads();
  const int e = threadIdx.x;  // (token, row): 32 x 16 = 512 > 256 threads: two passes
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int tk = (e >> 4) + 16 * pass, r = e & 15;
    if (tk < ntok && a->tok_grp[tk] == g && q0 + r < a->g_arows[g]) {
      const int l = (r >> 2) * 16 + (tk & 15);
      const float v = (red[0][tk >> 4][l][r & 3] + red[1][tk >> 4][l][r & 3]) +
                      (red[2][tk >> 4][l][r & 3] + red[3][tk >> 4][l][r & 3]);
      a->u[((int64_t)ks * ntok + tk) * a->u_ld + q0 + r] = v;
    }
  }
}

template <int TT>
__global__ __launch_bounds__(kFkWaves * 64, 1) void fullk_kernel(FullKArgs args) {
  fullk_args_ptr a = (fullk_args_ptr)__builtin_amdgcn_kernarg_segment_ptr();
  __shared__ f32x4 red[kFkWaves][TT][64];
  __shared__ float rsq[32];
  // lora_B rows of a weight tile (rank-16 rounds): [token][tile row][16],
  // two buffers (the next tile's rows land while this tile finishes)
  __shared__ __attribute__((aligned(16))) bf16 bsm[2][32][16][16];
  __shared__ const bf16* btab[32][SWL_MAX_LORA_BLOCKS];  // lora_B base of each token and column block
  // per-token values the epilogue needs, read once here so that no load of
  // the epilogue waits behind the next tile's weight loads: output row,
  // adapter entry (-1: none), its rank and scale
  __shared__ bf16* ytab[32];
  __shared__ int32_t ltab[32], rtab[32];
  __shared__ float stab[32];
  extern __shared__ float us[];  // [ntok][u_ld + 4] shrink rows (padded: tokens fall in different banks)
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nsw = a->nsw, ntok = a->ntok;
  const int s0 = wv * nsw;
  const int u_ld = a->u_ld, us_ld = a->u_ld + 4;

  // this wave's k-steps of weight tile `tile` (packed, k-steps 512 elements
  // apart); steps past nsw reload the last one (in bounds), their products
  // masked to zero by the zeroed token fragments
  u32x4 wf[kFkMaxSteps];
  auto issue = [&](int tile) {
    if (tile >= a->n_tiles) return;
    const bf16* p = a->w + ((int64_t)tile * a->total_steps + s0) * 512 + 8 * lane;
#pragma unroll
    for (int s = 0; s < kFkMaxSteps; ++s) {
      wf[s] = ldg16_nt(p);
      if (s + 1 < nsw) p += 512;
    }
  };
  // lora_B rows of weight tile `tile` into bsm[buf] with LDS-DMA:
  // instruction i (2 per wave, the last one repeated where there are fewer)
  // moves tokens 2 i and 2 i + 1, each the 8 rows of its adapter's B under
  // tile rows 0..7 (columns c0 ..) and under rows 8..15 (columns c0 + off
  // ..), 256 bytes a piece.  Tokens without an adapter read harmless bytes
  // of w.
  const int n_bins = (ntok + 1) >> 1;
  auto issue_b = [&](int tile, int buf) {
    const int64_t c0 = (int64_t)tile * 16, c1 = c0 + 8;
    const int b0 = fk_blk(a, c0), b1 = fk_blk(a, c1);
    const int64_t r0 = (c0 - a->blk_start[b0]) * 16, r1 = (c1 - a->blk_start[b1]) * 16;
    const int h = (lane >> 4) & 1;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ins = min(wv + kFkWaves * j, n_bins - 1);
      const int tk = 2 * ins + (lane >> 5);
      const bf16* src = btab[tk < ntok ? tk : 0][h ? b1 : b0] + (h ? r1 : r0) + (lane & 15) * 8;
      __builtin_amdgcn_global_load_lds((gbl_ptr)src, (lds_ptr)(reinterpret_cast<char*>(&bsm[buf][0][0][0]) + ins * 1024),
                                       16, 0, 0);
    }
  };

  // token rows: B fragments of this wave's k-steps (token 16 t + lane % 16,
  // k-group lane / 16), requested first; rows past ntok are zero
  u32x4 xf[kFkMaxSteps][TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int tk = 16 * t + (lane & 15);
    const bf16* xr = a->x[tk < ntok ? tk : 0] + 32 * s0 + 8 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < kFkMaxSteps; ++s)
      xf[s][t] = (tk < ntok && s < nsw) ? ldg16(xr + 32 * s) : u32x4{0u, 0u, 0u, 0u};
  }
  int tile = blockIdx.x;
  issue(tile);
  if (threadIdx.x < 32) {
    const int tk = threadIdx.x;
    const int li = (tk < ntok && a->has_lora) ? a->lora[tk] : -1;
    ytab[tk] = tk < ntok ? a->y[tk] : nullptr;
    ltab[tk] = li;
    rtab[tk] = li >= 0 ? a->table[li].rank : 0;
    stab[tk] = li >= 0 ? a->table[li].scale : 0.f;
  }
  if (a->has_lora) {
    // shrink rows: the sum of the shrink kernel's K-slice partials
    for (int i = threadIdx.x; i < ntok * u_ld; i += kFkWaves * 64) {
      const int tk = i / u_ld, q = i - tk * u_ld;
      float v = 0.f;
#pragma unroll
      for (int ks = 0; ks < kFkShrinkKs; ++ks) v += a->u[((int64_t)ks * ntok + tk) * u_ld + q];
      us[tk * us_ld + q] = v;
    }
  }
  if (a->bdma) {
    for (int i = threadIdx.x; i < 32 * SWL_MAX_LORA_BLOCKS; i += kFkWaves * 64) {
      const int tk = i / SWL_MAX_LORA_BLOCKS, b = i % SWL_MAX_LORA_BLOCKS;
      const int li = tk < ntok ? a->lora[tk] : -1;
      btab[tk][b] = (li >= 0 && b < a->nblk) ? reinterpret_cast<const bf16*>(a->table[li].b[b]) : a->w;
    }
  }
  if (a->gamma) fk_row_factors(a, rsq, kFkWaves, wv, lane);
  lds_barrier();
  int nb = 0;  // tiles whose lora_B rows were requested (buffer nb % 2 next)
  if (a->bdma && tile < a->n_tiles) issue_b(tile, nb++ & 1);
  if (a->gamma) {
    const bf16* gp = a->gamma + 32 * s0 + 8 * (lane >> 4);
#pragma unroll
    for (int s = 0; s < kFkMaxSteps; ++s) {
      if (s >= nsw) continue;
      const u32x4 gv = ldg16(gp + 32 * s);
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const int tk = 16 * t + (lane & 15);
        xf[s][t] = norm8(xf[s][t], rsq[tk < ntok ? tk : 0], gv);
      }
    }
  }

  while (tile < a->n_tiles) {
    f32x4 acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kFkMaxSteps; ++s)
#pragma unroll
      for (int t = 0; t < TT; ++t) acc[t] = mfma16(wf[s], xf[s][t], acc[t]);
    const int cur = tile;
    const int cur_buf = (nb + 1) & 1;  // the buffer cur's lora_B rows went to
    tile += gridDim.x;
    issue(tile);  // in flight during this tile's reduction and epilogue
    const bool next_b = a->bdma && tile < a->n_tiles;
    if (next_b) issue_b(tile, nb++ & 1);
#pragma unroll
    for (int t = 0; t < TT; ++t) red[wv][t][lane] = acc[t];
    lds_barrier();
    if (a->bdma) {
      // this tile's lora_B rows have landed: at most the next tile's 16
      // weight loads and 2 DMA are younger
      if (next_b)
        __builtin_amdgcn_s_waitcnt(wait_vm_imm(kFkMaxSteps + 2));
      else
        __builtin_amdgcn_s_waitcnt(wait_vm_imm(0));
      lds_barrier();
    }
    // sum of the wave partials of tile row r, token tk
    auto total = [&](int r, int tk) {
      const int l = (r >> 2) * 16 + (tk & 15), t = tk >> 4, e = r & 3;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kFkWaves; ++w) v += red[w][t][l][e];
      return v;
    };

    // thread (token tk, p) finishes tile rows p and p + 8, output columns c0
    // and c0 + 8
    const int e = threadIdx.x;
    const int tk = e >> 3, p = e & 7;
    const int64_t c0 = (int64_t)cur * 16 + p, c1 = c0 + 8;
    const bool live = tk < ntok && c0 < a->N;
    float v0 = 0.f, v1 = 0.f;
    if (live) {
      v0 = total(p, tk);
      v1 = total(p + 8, tk);
      if (a->bias) {
        v0 += bf2f(a->bias[c0]);
        v1 += bf2f(a->bias[c1]);
      }
      const int li = ltab[tk];
      if (li >= 0) {
        const int r = rtab[tk];
        const float scale = stab[tk];
        const float* ut = us + tk * us_ld;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int64_t c = h ? c1 : c0;
          const int b = fk_blk(a, c);
          const float* ub = ut + b * r;
          float d = 0.f;
          if (a->bdma) {
            const bf16* bl = &bsm[cur_buf][tk][8 * h + p][0];
#pragma unroll
            for (int q = 0; q < 16; q += 8) {
              float bv[8];
              unpack8(*reinterpret_cast<const u32x4*>(bl + q), bv);
#pragma unroll
              for (int i = 0; i < 8; ++i) d += ub[q + i] * bv[i];
            }
          } else {
            const bf16* brow =
                reinterpret_cast<const bf16*>(a->table[li].b[b]) + (c - a->blk_start[b]) * r;
            if ((r & 7) == 0) {
              for (int q = 0; q < r; q += 8) {
                float bv[8];
                unpack8(ld16(brow + q), bv);
#pragma unroll
                for (int i = 0; i < 8; ++i) d += ub[q + i] * bv[i];
              }
            } else {
              for (int q = 0; q < r; ++q) d += ub[q] * bf2f(ldg(brow + q));
            }
          }
          (h ? v1 : v0) += d * scale;
        }
      }
    }

    if (live) {
      stg(ytab[tk] + c0, f2bf(v0));
      stg(ytab[tk] + c1, f2bf(v1));
    }
    lds_barrier();  // red and bsm[cur_buf] are rewritten after this
  }
}

// ------------------------------------------------------- tiled (M>64) -----
// y[m, n] = sum_k x[m, k] w[n, k] for a packed x [M, K]; rows of y go to the
// segment (slot) the packed row belongs to.  128x128 output tile per
// workgroup (4 waves in 2x2, 64x64 each = 4x4 MFMA tiles), BK = 64 staged in
// LDS with a register prefetch of the next stage.
constexpr int TM = 128, TN = 128, TK = 64;
// LDS stages of the tiled kernel: one 32 KiB stage (two barriers per k-tile)
// leaves three workgroups resident per CU instead of two.
constexpr int kTiledBufs = 1;

struct TiledArgs {
  const bf16* x;          // packed [M, K], or null: row m of segment g read in place at xin[g] + (m - out.off[g]) * K
  const bf16* xin[kMaxSeg];
  const bf16* w;          // [N, K]
  const bf16* bias;
  int64_t M, N, K;
  int32_t has_lora;
  // output: either dense y (ldy) or per-segment rows
  bf16* y;                // dense output if non-null
  int64_t ldy;
  SegPtrs out;            // per-segment output base pointers (row stride N)
  int32_t seg_lora[kMaxSeg];
  LoraEpi L;              // u rows are packed rows
  // gemm256_kernel: LoRA delta as MFMA k-steps (every tile inside one column
  // block, ranks multiples of 8 up to 64) instead of in the epilogue
  int32_t lora_mfma;
};

// LDS rows of 64 bf16 (eight 16-byte chunks) with the chunks of row r
// XOR-permuted by (r / 2) % 8: a 16-lane fragment read (16 rows, one chunk)
// and a 16-lane staging write (2 rows, 8 chunks) each touch 16 distinct
// 16-byte bank groups (bank conflicts measured 70x lower than with padded
// rows).
__device__ __forceinline__ int swz(int row, int chunk) { return (chunk ^ ((row >> 1) & 7)) * 8; }

__global__ __launch_bounds__(256) void tiled_kernel(TiledArgs a) {
  // one LDS block: the A and B stages, reused by the epilogue (17 KiB)
  __shared__ __attribute__((aligned(16))) bf16 smem[kTiledBufs * (TM + TN) * TK];
  static_assert(kTiledBufs * (TM + TN) * TK * 2 >= 4 * 16 * (64 + 4) * 4, "epilogue staging must fit");
  bf16(*As)[TM][TK] = reinterpret_cast<bf16(*)[TM][TK]>(smem);
  bf16(*Bs)[TN][TK] = reinterpret_cast<bf16(*)[TN][TK]>(smem + kTiledBufs * TM * TK);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int64_t m0 = (int64_t)blockIdx.y * TM;
  const int64_t n0 = (int64_t)blockIdx.x * TN;

  // global -> LDS mapping: 8 threads per row (8 x 16 B = 128 B = TK bf16),
  // 32 rows per pass, 4 passes per 128-row tile.
  const int lr = tid >> 3, lc = (tid & 7) * 8;
  const bf16* xg[4];
  const bf16* wg[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int64_t mr = (m0 + lr + 32 * p < a.M) ? m0 + lr + 32 * p : a.M - 1;
    const int64_t nr = (n0 + lr + 32 * p < a.N) ? n0 + lr + 32 * p : a.N - 1;
    xg[p] = a.x + mr * a.K + lc;
    wg[p] = a.w + nr * a.K + lc;
  }
  u32x4 ra[4], rb[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) { ra[p] = ld16(xg[p]); rb[p] = ld16(wg[p]); }

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)(a.K / TK);
  int buf = 0;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    *reinterpret_cast<u32x4*>(&As[0][lr + 32 * p][swz(lr + 32 * p, lc >> 3)]) = ra[p];
    *reinterpret_cast<u32x4*>(&Bs[0][lr + 32 * p][swz(lr + 32 * p, lc >> 3)]) = rb[p];
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        ra[p] = ld16(xg[p] + (int64_t)(kt + 1) * TK);
        rb[p] = ld16(wg[p] + (int64_t)(kt + 1) * TK);
      }
    }
#pragma unroll
    for (int ks = 0; ks < TK / 32; ++ks) {
      u32x4 fa[4], fb[4];
      const int kch = ks * 4 + (lane >> 4);  // this lane's 16-byte k chunk
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ra_ = wm * 64 + i * 16 + (lane & 15), rb_ = wn * 64 + i * 16 + (lane & 15);
        fa[i] = *reinterpret_cast<const u32x4*>(&As[buf][ra_][swz(ra_, kch)]);
        fb[i] = *reinterpret_cast<const u32x4*>(&Bs[buf][rb_][swz(rb_, kch)]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(fa[i], fb[j], acc[i][j]);
    }
    if (kt + 1 < nk) {
      const int nb = kTiledBufs == 2 ? buf ^ 1 : 0;
      if (kTiledBufs == 1) __syncthreads();  // every wave is done reading the stage
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        *reinterpret_cast<u32x4*>(&As[nb][lr + 32 * p][swz(lr + 32 * p, lc >> 3)]) = ra[p];
        *reinterpret_cast<u32x4*>(&Bs[nb][lr + 32 * p][swz(lr + 32 * p, lc >> 3)]) = rb[p];
      }
      __syncthreads();
      buf = nb;
    }
  }

  // Epilogue.  acc[i][j] lane l holds rows (tokens) m0+wm*64+i*16+4*(l/16)+r,
  // column n0+wn*64+j*16+(l%16).  Transpose through LDS so each lane owns 4
  // consecutive columns of one token (8-byte stores, shared epilogue).
  __syncthreads();
  float* ct = reinterpret_cast<float*>(smem);  // reuse: 16 x (64 + 4) floats per wave pass
  // Each wave handles its own 64x64 sub-tile in 4 passes of 16 tokens.
  constexpr int CLD = 64 + 4;
  float* cw = ct + wv * 16 * CLD;  // 16 tokens x 64 columns per wave per pass
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) cw[(4 * (lane >> 4) + r) * CLD + j * 16 + (lane & 15)] = acc[i][j][r];
    __syncthreads();
    // lane -> (token = lane / 4 ... ) 16 tokens x 16 column-quads = 256 items, 4 per lane
    for (int it = 0; it < 4; ++it) {
      const int item = lane + 64 * it;
      const int tk = item >> 4;          // 0..15
      const int cq = (item & 15) * 4;    // 0..60
      const int64_t m = m0 + wm * 64 + i * 16 + tk;
      const int64_t n = n0 + wn * 64 + cq;
      if (m >= a.M || n >= a.N) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = cw[tk * CLD + cq + r];
      bf16* yrow;
      int lidx = -1;
      if (a.y) {
        yrow = a.y + m * a.ldy;
      } else {
        const int s = find_seg(a.out.off, a.out.n, m);
        yrow = reinterpret_cast<bf16*>(const_cast<void*>(a.out.ptr[s])) + (m - a.out.off[s]) * a.N;
        lidx = a.has_lora ? a.seg_lora[s] : -1;
      }
      epilogue_store4(v, n, a.N, a.bias, a.L, lidx, (int)m, yrow);
    }
    __syncthreads();
  }
}

// ------------------------------------------ prefill: 256 x 256 tiles ------
// y[m, n] = sum_k x[m, k] w[n, k] for the packed prefill batch, one
// 256 (columns) x 256 (tokens) output tile per workgroup of 4 waves, each
// wave 128 x 128 as 4 x 4 tiles of v_mfma_f32_32x32x16_bf16 (W rows as the A
// operand, token rows as B: a lane ends up with 4 consecutive columns of one
// token, the layout the epilogue stores; 256 fp32 accumulators a lane).  K
// advances 64 at a time through 2 LDS slots of 64 KiB (W 256 x 64 and x 256
// x 64), filled by LDS-DMA (global_load_lds, 16 bytes a lane, no register
// round trip) one stage ahead; every row a DMA instruction reads is one
// whole 128-byte line.  One barrier per stage separates the refill of a
// slot from the last reads of it.  LDS rows are 128 bytes (eight 16-byte
// chunks); chunk c of row r sits at c ^ (r % 8) ^ ((r / 8) % 2), so a
// fragment read (32 consecutive rows, one chunk) meets distinct banks in
// every 8 and every 16 of its lanes.  Workgroups are numbered so that each
// XCD (workgroup i runs on XCD i % 8) walks a contiguous run of tiles,
// tokens fastest: the W rows of a tile column are read by the XCD's
// workgroups together, from its L2.
constexpr int PG_M = 256, PG_N = 256, PG_K = 64, PG_SLOTS = 2;
constexpr int PG_ROW = PG_K * 2;                           // bytes of an LDS row
constexpr int PG_ELD = 64 + 4;                            // epilogue staging row (fp32)
// Waves 2 WM: two along the columns (128 each), WM along the token rows; NJ:
// 32-row MFMA tiles of tokens per wave, so 32 WM NJ token rows a tile (256
// or 192; W always 256 columns).  Stage: W 256 rows, then x MT rows.
template <int NJ, int WM>
struct PgGeom {
  static constexpr int MT = 32 * WM * NJ;                   // token rows of a tile
  static constexpr int STAGE = (PG_N + MT) * PG_ROW;        // 64 or 56 KiB
  static constexpr int EPI = 2 * WM * 32 * NJ * PG_ELD * 4; // epilogue staging, one region a wave
  static constexpr int AREA = PG_SLOTS * STAGE > EPI ? PG_SLOTS * STAGE : EPI;
  // then the tile's row table: output row pointer (8 bytes) and epilogue
  // adapter (4 bytes) of each of its token rows; then the LoRA entries
  // (lora_B block pointer, rank, scale) of the segments the tile overlaps
  static constexpr int LDS = AREA + PG_M * 12 + kMaxSeg * 16;
};

// LoRA entry of one segment of a prefill tile, as the k-step loop reads it
struct PgSegLora {
  const bf16* b;  // the adapter's lora_B rows of the tile's column block
  int32_t rank;   // 0: no adapter
  float scale;
};

__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

template <int NJ, int WM>
__global__ __launch_bounds__(128 * WM, 1) void gemm256_kernel(TiledArgs a, int tiles_m, int tiles, int per_xcd,
                                                               int gm) {
  // PG_SLOTS x [W 256 x 64 | x MT x 64]; then the epilogue's WAVES x [TPW][PG_ELD] fp32
  using Geo = PgGeom<NJ, WM>;
  constexpr int WAVES = 2 * WM;
  constexpr int MT = Geo::MT, TPW = 32 * NJ, XR = MT / WAVES;  // token rows: tile, wave, DMA rows a wave
  constexpr int WR = PG_N / WAVES;                              // W rows a wave moves per stage
  constexpr int MF = 4 * NJ, NR = 4 + NJ;                       // MFMAs and fragment reads per k-step
  constexpr int NREQ = WR / 8 + XR / 8;                         // DMA instructions a wave per stage
  static_assert(PG_N % (8 * WAVES) == 0 && MT % (8 * WAVES) == 0, "the waves' DMA rows must cover the stage");
  extern __shared__ __attribute__((aligned(16))) char pg_lds[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wv >> 1, wn = wv & 1;  // wave: tokens wm * TPW.., columns wn * 128..
  const int lin = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (lin >= tiles) return;  // uniform over the workgroup
  // linear tile lin: groups of gm row tiles, each group walking its column
  // tiles with the rows fastest (gm = tiles_m: one group)
  const int gsz = gm * (tiles / tiles_m);
  const int grp = lin / gsz, gl = lin - grp * gsz;
  const int gr = min(gm, tiles_m - grp * gm);  // row tiles in this group
  const int64_t m0 = (int64_t)(grp * gm + gl % gr) * MT;
  const int64_t n0 = (int64_t)(gl / gr) * PG_N;
  const int nk = (int)(a.K / PG_K);

  f32x16 acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  const int fr = lane & 31, fh = lane >> 5;
  auto mma = [&](const u32x4 (&fa)[4], const u32x4 (&fb)[NJ]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma32(fa[i], fb[j], acc[i][j]);
  };
  // One instruction group of the main loop: MFMA t of the 2 MF of half a
  // stage (k-step t / MF of the pair, tile ((t % MF) / NJ, t % NJ)), then at
  // most one fragment read and one DMA request, then a scheduling fence, so
  // the order written here is the order issued.  Spreading the requests
  // keeps the CU's address queue from blocking the wave (a 1 KiB LDS-DMA
  // request takes the queue about 16 cycles).
  auto mfma_at = [&](u32x4 (&a0)[4], u32x4 (&b0)[NJ], u32x4 (&a1)[4], u32x4 (&b1)[NJ], int t) {
    const int i = (t % MF) / NJ, j = t % NJ;
    if (t < MF)
      acc[i][j] = mfma32(a0[i], b0[j], acc[i][j]);
    else
      acc[i][j] = mfma32(a1[i], b1[j], acc[i][j]);
  };

  // the tile's row table in LDS, built while the first stages' DMA is in
  // flight
  bf16** rowtab = reinterpret_cast<bf16**>(pg_lds + Geo::AREA);
  int* lidxtab = reinterpret_cast<int*>(pg_lds + Geo::AREA + PG_M * 8);
  auto build_rowtab = [&]() {
    if (threadIdx.x < PG_M) {
      const int64_t m = m0 + threadIdx.x;
      bf16* yrow = nullptr;
      int lidx = -1;
      if (m < a.M) {
        if (a.y) {
          yrow = a.y + m * a.ldy;
        } else {
          const int sg = find_seg(a.out.off, a.out.n, m);
          yrow = reinterpret_cast<bf16*>(const_cast<void*>(a.out.ptr[sg])) + (m - a.out.off[sg]) * a.N;
          lidx = (a.has_lora && !a.lora_mfma) ? a.seg_lora[sg] : -1;
        }
      }
      rowtab[threadIdx.x] = yrow;
      lidxtab[threadIdx.x] = lidx;
    }
  };

  // LDS-DMA of stage kt into slot s: wave w moves W rows WR w .. + WR (WR /
  // 8 instructions) and x rows XR w .. + XR (XR / 8), 8 rows of 128 bytes an
  // instruction; lane l of instruction i -> row 8 i + l / 8 of the wave's,
  // stored chunk l % 8, read from global chunk (l % 8) ^ (l / 8) ^ (i % 2)
  // (the wave's first row is a multiple of 16)
  const int dr = lane >> 3;
  const bf16* wsrc[WR / 8];
  const bf16* xsrc[XR / 8];
#pragma unroll
  for (int i = 0; i < WR / 8; ++i) {
    const int64_t r = WR * wv + 8 * i + dr;
    const int dc = (lane & 7) ^ dr ^ (i & 1);
    wsrc[i] = a.w + min(n0 + r, a.N - 1) * a.K + 8 * dc;
  }
#pragma unroll
  for (int i = 0; i < XR / 8; ++i) {
    const int64_t r = XR * wv + 8 * i + dr;
    const int dc = (lane & 7) ^ dr ^ (i & 1);
    const int64_t mr = min(m0 + r, a.M - 1);
    if (a.x) {
      xsrc[i] = a.x + mr * a.K + 8 * dc;
    } else {  // the token row in its slot buffer (no packed copy)
      const int sg = find_seg(a.out.off, a.out.n, mr);
      xsrc[i] = a.xin[sg] + (mr - a.out.off[sg]) * a.K + 8 * dc;
    }
  }
  // DMA instruction q of a stage (W 0 .. WR / 8 - 1, then x): into slot s
  auto request_at = [&](int kt, int s, int q) {
    char* st = pg_lds + s * Geo::STAGE;
    constexpr int QW = WR / 8;
    if (q < QW)
      __builtin_amdgcn_global_load_lds((gbl_ptr)(wsrc[q] + (int64_t)kt * PG_K),
                                       (lds_ptr)(st + (WR * wv + 8 * q) * PG_ROW), 16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds((gbl_ptr)(xsrc[q - QW] + (int64_t)kt * PG_K),
                                       (lds_ptr)(st + PG_N * PG_ROW + (XR * wv + 8 * (q - QW)) * PG_ROW), 16, 0, 0);
  };
  auto issue = [&](int kt, int s) {
#pragma unroll
    for (int q = 0; q < NREQ; ++q) request_at(kt, s, q);
  };


  // fragment rows of this lane: W row wn * 128 + 32 i + l % 32, x row
  // wm * TPW + 32 j + l % 32 (both = l % 32 modulo 32, so one swizzle);
  // k chunk 2 kk + l / 32 of the stage
  const int sw = (fr & 7) ^ ((fr >> 3) & 1);
  auto read_at = [&](int s, int kk, u32x4 (&fa_)[4], u32x4 (&fb_)[NJ], int idx) {
    const char* st = pg_lds + s * Geo::STAGE + fr * PG_ROW + (((2 * kk + fh) ^ sw) << 4);
    if (idx < 4)
      fa_[idx] = *reinterpret_cast<const u32x4*>(st + (wn * 128 + 32 * idx) * PG_ROW);
    else
      fb_[idx - 4] = *reinterpret_cast<const u32x4*>(st + PG_N * PG_ROW + (wm * TPW + 32 * (idx - 4)) * PG_ROW);
  };

  // Fragments of the four k-steps of a stage sit in four register sets,
  // read two k-steps ahead of their MFMAs.  Stage kt + 2 is requested into
  // slot kt % 2 after the barrier at mid-stage kt that ends every wave's
  // reads of it (the fragments of k-steps 2 and 3 were read during k-steps
  // 0 and 1); the same barrier publishes stage kt + 1, whose first two
  // k-steps are read during the last two of stage kt.  The loop has no
  // branches: past the last stage the requests re-read stage nk - 1 into
  // the free slot, which only the discarded reads at the very end look at.
  u32x4 fa[4][4], fb[4][NJ];
  // LoRA entries of the segments the tile overlaps, requested ahead of the
  // DMA (so that waiting for them does not wait for it) and put in LDS
  // after it: thread t takes segment sg0 + t
  PgSegLora* segl = reinterpret_cast<PgSegLora*>(pg_lds + Geo::AREA + PG_M * 12);
  const bool lora_k = a.has_lora && a.lora_mfma;
  int lb = 0, sg0 = 0, nseg = 0;
  PgSegLora my{nullptr, 0, 0.f};
  if (lora_k) {
#pragma unroll
    for (int i = 1; i < SWL_MAX_LORA_BLOCKS; ++i)
      if (i < a.L.nblk && n0 >= a.L.blk_start[i]) lb = i;
    sg0 = find_seg(a.out.off, a.out.n, m0);
    nseg = find_seg(a.out.off, a.out.n, min<int64_t>(m0 + MT, a.M) - 1) - sg0 + 1;
    const int e = (int)threadIdx.x < nseg ? a.seg_lora[sg0 + threadIdx.x] : -1;
    if (e >= 0) {
      const char* ep = reinterpret_cast<const char*>(a.L.table + e);
      using bptr = const bf16*;
      my.b = *(const __attribute__((address_space(1))) bptr*)(ep + offsetof(swl_lora_entry, b) + lb * sizeof(void*));
      my.rank = *(const __attribute__((address_space(1))) int32_t*)(ep + offsetof(swl_lora_entry, rank));
      my.scale = *(const __attribute__((address_space(1))) float*)(ep + offsetof(swl_lora_entry, scale));
    }
  }
  issue(0, 0);
  issue(min(1, nk - 1), 1);
  build_rowtab();
  if ((int)threadIdx.x < nseg) segl[threadIdx.x] = my;
  __builtin_amdgcn_s_waitcnt(wait_vm_imm(NREQ));
  lds_barrier();
  // The main loop over a predicate live(j): whether the wave's 32-row block
  // j of token rows holds a row of the batch.  Every block does, except in
  // the batch's last row tile: there the MFMAs and fragment reads of the
  // empty blocks are skipped (a wave with none reads nothing), so that tile
  // costs a fraction of a full one; the DMA requests and barriers stay the
  // same in every wave.
  auto main_loop = [&](auto live) {
    auto read_live = [&](int idx) { return idx < 4 ? live(0) : live(idx - 4); };
#pragma unroll
    for (int idx = 0; idx < NR; ++idx)
      if (read_live(idx)) read_at(0, 0, fa[0], fb[0], idx);
#pragma unroll
    for (int idx = 0; idx < NR; ++idx)
      if (read_live(idx)) read_at(0, 1, fa[1], fb[1], idx);
    for (int kt = 0; kt < nk; ++kt) {
      const int s = kt & 1;
      // k-steps 0, 1 of stage kt; reads of its k-steps 2, 3 during the first
      // 2 NR
#pragma unroll
      for (int t = 0; t < 2 * MF; ++t) {
        if (live(t % NJ)) mfma_at(fa[0], fb[0], fa[1], fb[1], t);
        if (t < NR) {
          if (read_live(t)) read_at(s, 2, fa[2], fb[2], t);
        } else if (t < 2 * NR) {
          if (read_live(t - NR)) read_at(s, 3, fa[3], fb[3], t - NR);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // this wave's DMA of stage kt + 1 has landed (it is all that is
      // outstanding), then every wave's; every wave is past its reads of slot s
      __builtin_amdgcn_s_waitcnt(wait_vm_imm(0));
      lds_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // k-steps 2, 3; reads of stage kt + 1's k-steps 0, 1 during the first
      // 2 NR, the NREQ DMA requests of stage kt + 2 spread over the 2 MF MFMAs
      const int nx = min(kt + 2, nk - 1);
#pragma unroll
      for (int t = 0; t < 2 * MF; ++t) {
        if (live(t % NJ)) mfma_at(fa[2], fb[2], fa[3], fb[3], t);
        if (t < NR) {
          if (read_live(t)) read_at(s ^ 1, 0, fa[0], fb[0], t);
        } else if (t < 2 * NR) {
          if (read_live(t - NR)) read_at(s ^ 1, 1, fa[1], fb[1], t - NR);
        }
        if (t == 0 || (t * NREQ) / (2 * MF) != ((t - 1) * NREQ) / (2 * MF)) request_at(nx, s, (t * NREQ) / (2 * MF));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  const int jl = (int)min<int64_t>(NJ, max<int64_t>(0, (a.M - m0 - wm * TPW + 31) / 32));
  if (jl == NJ)
    main_loop([](int) { return true; });
  else
    main_loop([jl](int j) { return j < jl; });
  // the requests past the last stage land before the LDS is reused
  __builtin_amdgcn_s_waitcnt(wait_vm_imm(0));



  // LoRA delta as extra k-steps: for every segment of the tile's token rows
  // that has an adapter, A = the adapter's lora_B rows of the tile's
  // columns (k = rank), B = the segment's shrink rows u * scale rounded to
  // bf16 (zero for the other segments' rows), 16 ranks a step.  The steps
  // run as one loop over (segment, rank step) with the next step's loads in
  // flight while the current one's MFMAs issue (two register sets taking
  // turns), the entries read from the tile's LDS table.
  if (lora_k) {
    const int64_t bstart = blk_start_of(a.L, lb);
    auto first = [&](int i) {  // first segment from i with an adapter
      while (i < nseg && segl[i].rank <= 0) ++i;
      return i;
    };
    auto advance = [&](int& i, int& q0) {
      q0 += 16;
      if (q0 >= segl[i].rank) {
        q0 = 0;
        i = first(i + 1);
      }
    };
    auto load = [&](int i, int q0, u32x4 (&fa_)[4], u32x4 (&u_)[NJ][2]) {
      const PgSegLora e = segl[i];
      const int r = e.rank, q = q0 + 8 * fh;
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int64_t n = n0 + wn * 128 + 32 * i4 + fr;
        fa_[i4] = (n < a.N && q < r) ? ld16(e.b + (n - bstart) * r + q) : u32x4{0u, 0u, 0u, 0u};
      }
      const int64_t lo = a.out.off[sg0 + i], hi = a.out.off[sg0 + i + 1];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int64_t m = m0 + wm * TPW + 32 * j + fr;
        if (m >= lo && m < hi && q < r) {
          const float* up = a.L.u + m * a.L.u_ld + lb * r + q;
          u_[j][0] = ld16(up);
          u_[j][1] = ld16(up + 4);
        } else {
          u_[j][0] = u_[j][1] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    };
    auto use = [&](int i, const u32x4 (&fa_)[4], const u32x4 (&u_)[NJ][2]) {
      const float scale = segl[i].scale;
      u32x4 fb_[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const f32x4 u0 = __builtin_bit_cast(f32x4, u_[j][0]), u1 = __builtin_bit_cast(f32x4, u_[j][1]);
        bf16x8 o;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          o[t] = f2bf(u0[t] * scale);
          o[4 + t] = f2bf(u1[t] * scale);
        }
        fb_[j] = __builtin_bit_cast(u32x4, o);
      }
      mma(fa_, fb_);
    };
    // PD register sets taken in turn: while a step's MFMAs issue, the loads
    // of the next PD - 1 steps are in flight (a tile over many small
    // segments runs ~20 latency-bound steps)
    constexpr int PD = 3;
    u32x4 ra[PD][4], ru[PD][NJ][2];
    int di[PD];
    int li = first(0), lq = 0;  // the next step to load
#pragma unroll
    for (int p = 0; p < PD; ++p) {
      di[p] = li;
      if (li < nseg) {
        load(li, lq, ra[p], ru[p]);
        advance(li, lq);
      }
    }
    while (di[0] < nseg) {
#pragma unroll
      for (int p = 0; p < PD; ++p) {
        if (di[p] >= nseg) break;  // uniform: steps fill the sets in order
        use(di[p], ra[p], ru[p]);
        di[p] = li;
        if (li < nseg) {
          load(li, lq, ra[p], ru[p]);
          advance(li, lq);
        }
      }
    }
  }

  // Epilogue through LDS (the stages are free once every wave is past its
  // last reads), in two halves of the columns so each wave's share fits:
  // acc[i][j] element e of lane l is column 32 i + 8 (e / 4) + 4 (l / 32) +
  // e % 4 of the wave's 128, token 32 j + l % 32.  Wave w's half h lands in
  // region w as [TPW tokens][64 columns (+4 pad)] fp32; then thread t takes
  // quads of four columns, 16 threads a token row, and finishes them
  // (bias, LoRA expand, one bf16 rounding, the segment's row).
  constexpr int ELD = PG_ELD;
  float* reg = reinterpret_cast<float*>(pg_lds) + wv * TPW * ELD;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    lds_barrier();  // the previous half's (or the k-loop's) reads are done
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int tok = 32 * j + fr, col = 32 * ii + 8 * q + 4 * fh;
          const f32x16& c = acc[2 * h + ii][j];
          *reinterpret_cast<f32x4*>(reg + tok * ELD + col) = f32x4{c[4 * q], c[4 * q + 1], c[4 * q + 2], c[4 * q + 3]};
        }
    lds_barrier();
    // items: wave region w2 (tokens wm2 * TPW, columns wn2 * 128 + 64 h),
    // token row tr, quad cq; WAVES x TPW x 16 items, 8 NJ a thread (row
    // group t / 16 of RG, rows rg + RG kk of each region), all of one
    // thread's in the two column quads cq = t % 16 of the two wn2, whose
    // bias it loads once
    const int cq = threadIdx.x & 15;
    constexpr int RG = 4 * WAVES, KK = TPW / RG;  // row groups; rows of a region a thread takes
    float bq[2][4];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int64_t n = n0 + c * 128 + 64 * h + 4 * cq;
#pragma unroll
      for (int e = 0; e < 4; ++e) bq[c][e] = (a.bias && n + e < a.N) ? bf2f(a.bias[n + e]) : 0.f;
    }
    auto item = [&](int k, bool lora) {
      const int w2 = k / KK, tr = (threadIdx.x >> 4) + RG * (k % KK);
      const int row = (w2 >> 1) * TPW + tr;
      const int64_t m = m0 + row;
      const int64_t n = n0 + (w2 & 1) * 128 + 64 * h + 4 * cq;
      if (m >= a.M || n >= a.N) return;
      const f32x4 q4 = *reinterpret_cast<const f32x4*>(reinterpret_cast<float*>(pg_lds) + (w2 * TPW + tr) * ELD + 4 * cq);
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = q4[e] + bq[w2 & 1][e];
      epilogue_store4(v, n, a.N, nullptr, a.L, lora ? lidxtab[row] : -1, (int)m, rowtab[row]);
    };
    if (a.has_lora && !a.lora_mfma) {
      // the LoRA delta in the epilogue (per-quad loads of u and lora_B)
      for (int k = 0; k < 8 * NJ; ++k) item(k, true);
    } else {
      // k = KK w2 + kk: the KK staged quads and row pointers of a region
      // are read together, then stored
#pragma unroll
      for (int w2 = 0; w2 < WAVES; ++w2) {
        f32x4 q[KK];
        bf16* rp[KK];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          const int tr = (threadIdx.x >> 4) + RG * kk;
          q[kk] = *reinterpret_cast<const f32x4*>(reinterpret_cast<float*>(pg_lds) + (w2 * TPW + tr) * ELD + 4 * cq);
          rp[kk] = rowtab[(w2 >> 1) * TPW + tr];
        }
        const int64_t n = n0 + (w2 & 1) * 128 + 64 * h + 4 * cq;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          const int64_t m = m0 + (w2 >> 1) * TPW + (threadIdx.x >> 4) + RG * kk;
          if (m < a.M && n < a.N) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = q[kk][e] + bq[w2 & 1][e];
            store4_bf16(v, n, a.N, rp[kk]);
          }
        }
      }
    }
  }
}

// ----------------------------------------------- generic small matmul -----
// y[m, n] = alpha * sum_k x[m, k] * B(k, n), B(k, n) = b[k*ldb + n] (nn) or
// b[n*ldb + k] (nt).  Workgroup: 64 columns x 4 k-partitions, LDS reduce.
__global__ __launch_bounds__(256) void matmul_generic_kernel(const bf16* __restrict__ x, int64_t ldx,
                                                             const bf16* __restrict__ b, int64_t ldb, int trans_b,
                                                             bf16* __restrict__ y, int64_t ldy, int64_t N, int64_t K,
                                                             float alpha) {
  __shared__ float part[4][64];
  const int c = threadIdx.x & 63, p = threadIdx.x >> 6;
  const int64_t m = blockIdx.y;
  const int64_t n = (int64_t)blockIdx.x * 64 + c;
  float s = 0.f;
  if (n < N) {
    const bf16* xr = x + m * ldx;
    if (!trans_b) {
      for (int64_t k = p; k < K; k += 4) s += bf2f(xr[k]) * bf2f(b[k * ldb + n]);
    } else {
      const bf16* br = b + n * ldb;
      for (int64_t k = p; k < K; k += 4) s += bf2f(xr[k]) * bf2f(br[k]);
    }
  }
  part[p][c] = s;
  __syncthreads();
  if (p == 0 && n < N) {
    float t = part[0][c] + part[1][c] + part[2][c] + part[3][c];
    y[m * ldy + n] = f2bf(alpha * t);
  }
}

// Few output columns over long rows (the LoRA shrink x . A of a worker's
// few tokens: N = rank or a fused n * rank, K = hidden or intermediate).
// One 1024-thread workgroup per row m streams B once with 16-byte loads;
// x[m, :] is staged in LDS.  NT (B(k, n) = b[n*ldb + k]): wave w owns the
// columns n = w, w + 16, ..., its lanes stride k in 8-element vectors and a
// wave reduction finishes each column.  NN (B(k, n) = b[k*ldb + n]): thread
// t owns 8 adjacent columns (cv = t % N8) over the k-rows p, p + P, ... with
// P a power of two, and the P partial sums of each column are reduced as a
// tree in LDS.  fp32 accumulation, alpha applied before the one bf16
// rounding.  Host-checked: N <= 256, K % 8 == 0, 16-byte aligned rows,
// N % 8 == 0 (NN), K <= kShrinkMaxK.
constexpr int64_t kShrinkMaxK = 16384;

template <bool NT>
__global__ __launch_bounds__(1024) void matmul_shrink_kernel(const bf16* __restrict__ x, int64_t ldx,
                                                             const bf16* __restrict__ b, int64_t ldb,
                                                             bf16* __restrict__ y, int64_t ldy, int N, int64_t K,
                                                             float alpha, int P) {
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* xs = reinterpret_cast<bf16*>(smem);                      // [K]
  float* red = reinterpret_cast<float*>(smem + K * sizeof(bf16));  // NN: [P][N]
  const int64_t m = blockIdx.x;
  const bf16* xr = x + m * ldx;
  const int tid = threadIdx.x;
  const int64_t K8 = K >> 3;
  for (int64_t i = tid; i < K8; i += 1024)
    *reinterpret_cast<u32x4*>(xs + 8 * i) = ld16(xr + 8 * i);
  __syncthreads();
  if constexpr (NT) {
    const int w = tid >> 6, lane = tid & 63;
    for (int n = w; n < N; n += 16) {
      const bf16* br = b + (int64_t)n * ldb;
      float acc = 0.f;
#pragma unroll 4
      for (int64_t i = lane; i < K8; i += 64) {
        float xv[8], bv[8];
        unpack8(*reinterpret_cast<const u32x4*>(xs + 8 * i), xv);
        unpack8(ld16(br + 8 * i), bv);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc += xv[j] * bv[j];
      }
      for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
      if (lane == 0) y[m * ldy + n] = f2bf(alpha * acc);
    }
  } else {
    const int N8 = N >> 3;
    const int cv = tid % N8, p = tid / N8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (p < P) {
#pragma unroll 4
      for (int64_t k = p; k < K; k += P) {
        float bv[8];
        unpack8(ld16(b + k * ldb + 8 * cv), bv);
        const float xv = bf2f(xs[k]);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += xv * bv[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) red[(int64_t)p * N + 8 * cv + j] = acc[j];
    }
    __syncthreads();
    for (int s = P >> 1; s >= 1; s >>= 1) {
      for (int e = tid; e < s * N; e += 1024) red[e] += red[e + s * N];
      __syncthreads();
    }
    if (tid < N) y[m * ldy + tid] = f2bf(alpha * red[tid]);
  }
}

// ---------------------------------------------- worker-side LoRA delta ----
// One launch per adapter delta of a worker's few token rows: the reference's
// FusedLoRA.forward ((x . fused_A) . fused_B over the diagonal blocks,
// model_builder.py:217-262) and SyncRemoteLoRALinear's lora_B(lora_A(x)) *
// scaling (worker_sync.py:305, :375).  Every workgroup computes the whole
// shrink u[m, j] = bf16(sum_k x[m, k] A(k, j)), j < nr (A comes from L2 after
// the first workgroup's misses; K is split over the 256 threads in 8-element
// chunks, one wave reduction per column); workgroup g then writes its share
// of the columns c of y[m, c] = bf16(alpha * sum_rr u[m, b*rank + rr] *
// B_b(rr, c - off_b)), b the block holding c.  A(k, j) = a[k*a_sk + j*a_sj],
// B_b(rr, c) = b_b[rr*srr_b + c*sc_b].  Two bf16 roundings, as the two bf16
// matmuls of the reference.
constexpr int kLoraRowsMaxRows = 4, kLoraRowsMaxNr = 64, kLoraRowsMaxBlk = 4;

struct LoraRowsArgs {
  const bf16* x;
  int64_t ldx, K;
  int m, nr, nblk, rank;
  const bf16* a;
  int64_t a_sk, a_sj;
  int a_mode;  // 0: k-contiguous rows (16-byte loads over k), 1: j-contiguous rows (16-byte loads over j), 2: scalar
  const bf16* b[kLoraRowsMaxBlk];
  int64_t srr[kLoraRowsMaxBlk], sc[kLoraRowsMaxBlk], off[kLoraRowsMaxBlk + 1];
  float alpha;
  bf16* y;
  int64_t ldy;
};

template <int NRMAX>
__global__ __launch_bounds__(256) void lora_rows_kernel(LoraRowsArgs a) {
  __shared__ float red[4][NRMAX];
  __shared__ float us[kLoraRowsMaxRows][NRMAX];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t K8 = a.K >> 3;
  for (int m = 0; m < a.m; ++m) {
    const bf16* xr = a.x + m * a.ldx;
    float acc[NRMAX];
#pragma unroll
    for (int j = 0; j < NRMAX; ++j) acc[j] = 0.f;
    for (int64_t c = tid; c < K8; c += 256) {
      float xv[8];
      unpack8(ld16(xr + 8 * c), xv);
      if (a.a_mode == 0) {
#pragma unroll
        for (int j = 0; j < NRMAX; ++j)
          if (j < a.nr) {
            float av[8];
            unpack8(ld16(a.a + j * a.a_sj + 8 * c), av);
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) acc[j] += xv[kk] * av[kk];
          }
      } else if (a.a_mode == 1) {
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const bf16* ar = a.a + (8 * c + kk) * a.a_sk;
#pragma unroll
          for (int jg = 0; jg < NRMAX / 8; ++jg)
            if (8 * jg < a.nr) {
              float av[8];
              unpack8(ld16(ar + 8 * jg), av);
#pragma unroll
              for (int i = 0; i < 8; ++i) acc[8 * jg + i] += xv[kk] * av[i];
            }
        }
      } else {
        // scalar reads of A (any strides), one k of the chunk at a time: with
        // the 8 k unrolled, the 8 NRMAX reads and their 64-bit addresses
        // were all live at once and spilled
#pragma unroll 1
        for (int kk = 0; kk < 8; ++kk) {
          float xk = xv[0];
#pragma unroll
          for (int i = 1; i < 8; ++i) xk = kk == i ? xv[i] : xk;
          const bf16* ar = a.a + (8 * c + kk) * a.a_sk;
#pragma unroll
          for (int j = 0; j < NRMAX; ++j)
            if (j < a.nr) acc[j] += xk * bf2f(ar[j * a.a_sj]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NRMAX; ++j)
      if (j < a.nr) {
        float v = acc[j];
        for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
        if (lane == 0) red[w][j] = v;
      }
    __syncthreads();
    if (tid < a.nr) us[m][tid] = bf2f(f2bf(red[0][tid] + red[1][tid] + red[2][tid] + red[3][tid]));
    __syncthreads();
  }
  const int64_t N = a.off[a.nblk];
  for (int64_t c = (int64_t)blockIdx.x * 256 + tid; c < N; c += (int64_t)gridDim.x * 256) {
    int b = 0;
    while (b + 1 < a.nblk && c >= a.off[b + 1]) ++b;
    const bf16* bb = a.b[b] + (c - a.off[b]) * a.sc[b];
    const int64_t srr = a.srr[b];
    const int u0 = b * a.rank;
    for (int m = 0; m < a.m; ++m) {
      float s = 0.f;
      for (int rr = 0; rr < a.rank; ++rr) s += us[m][u0 + rr] * bf2f(bb[rr * srr]);
      a.y[m * a.ldy + c] = f2bf(a.alpha * s);
    }
  }
}

// ------------------------------------------------------ paged attention ---
struct AttnArgs {
  bf16* q;               // token t at q + t*qs: [hq, 128]
  bf16* k;               // token t at k + t*ks: [hkv, 128]
  const bf16* v;         // token t at v + t*vs: [hkv, 128]
  int64_t qs, ks, vs;    // token row strides (elements)
  bf16* kc;              // [num_blocks, bs, hkv, 128]
  bf16* vc;
  const int32_t* bt;     // [nseq, max_blocks]
  const int32_t* seqlens;
  const int64_t* pos;    // [nseq * L]
  const bf16* cs;        // [max_pos, 128]
  bf16* out;             // [nseq, L, hq*128]
  int64_t num_blocks, max_blocks, max_pos;
  int32_t nseq, L, hq, hkv, bs, rope;
  int32_t bs_shift;      // log2(bs) when bs is a power of two, else -1
  float scale;
  // row mode (rowmode != 0): token t reads its fused [q | k | v] row at
  // qkv_row[t] and writes its output row at out_row[t]
  int32_t rowmode;
  bf16* qkv_row[kSkinnyMaxTok];
  bf16* out_row[kSkinnyMaxTok];
};

__device__ __forceinline__ bf16* tok_q(const AttnArgs& a, int64_t t) {
  return a.rowmode ? a.qkv_row[t] : a.q + t * a.qs;
}
__device__ __forceinline__ bf16* tok_k(const AttnArgs& a, int64_t t) {
  return a.rowmode ? a.qkv_row[t] + a.hq * 128 : a.k + t * a.ks;
}
__device__ __forceinline__ const bf16* tok_v(const AttnArgs& a, int64_t t) {
  return a.rowmode ? a.qkv_row[t] + (a.hq + a.hkv) * 128 : a.v + t * a.vs;
}
__device__ __forceinline__ bf16* tok_out(const AttnArgs& a, int64_t t) {
  return a.rowmode ? a.out_row[t] : a.out + t * (int64_t)a.hq * 128;
}

// NeoX rotation of q and k at their positions, k/v appended to the pages.
// One 64-thread workgroup per (token, head) of the fused row: q heads are
// rotated in place, k heads rotated in place and copied to the K page, v
// heads copied to the V page (lane d handles dims d and d + 64).
__global__ __launch_bounds__(64) void rope_append_kernel(AttnArgs a) {
  const int tokid = blockIdx.x;  // s * L + i
  const int h = blockIdx.y;      // [0, hq): q, [hq, hq + hkv): k, then v
  const int d = threadIdx.x;
  const int s = tokid / a.L, i = tokid % a.L;
  const bool is_q = h < a.hq, is_k = !is_q && h < a.hq + a.hkv;
  bf16* row = is_q ? tok_q(a, tokid) + h * 128
                   : (is_k ? tok_k(a, tokid) + (h - a.hq) * 128
                           : const_cast<bf16*>(tok_v(a, tokid)) + (h - a.hq - a.hkv) * 128);
  float x1 = bf2f(row[d]), x2 = bf2f(row[d + 64]);
  if (!is_q && !is_k) {
    // v: copy only
  } else if (a.rope) {
    const int64_t pos = a.pos[tokid];
    if (pos >= 0 && pos < a.max_pos) {
      const bf16* cs = a.cs + pos * 128;
      const float c = bf2f(cs[d]), sn = bf2f(cs[64 + d]);
      const float y1 = x1 * c - x2 * sn, y2 = x2 * c + x1 * sn;
      const bf16 o1 = f2bf(y1), o2 = f2bf(y2);
      row[d] = o1;
      row[d + 64] = o2;
      x1 = bf2f(o1);
      x2 = bf2f(o2);
    }
  }
  if (is_q) return;
  const int64_t p = (int64_t)a.seqlens[s] + i;
  const int64_t blk_i = p / a.bs;
  if (p < 0 || blk_i >= a.max_blocks) return;
  const int32_t blk = a.bt[(int64_t)s * a.max_blocks + blk_i];
  if (blk < 0 || blk >= a.num_blocks) return;
  const int kvh = is_k ? h - a.hq : h - a.hq - a.hkv;
  bf16* dst = (is_k ? a.kc : a.vc) + ((int64_t)blk * a.bs + p % a.bs) * a.hkv * 128 + kvh * 128;
  dst[d] = f2bf(x1);
  dst[d + 64] = f2bf(x2);
}

// Attention of one query token over its causal context for one kv head and
// its G = hq / hkv query heads.  Workgroup = 4 waves; each 16-lane quarter of
// a wave owns one key at a time (lane holds 8 of the 128 dims), so a wave
// consumes 4 keys per step and the workgroup 16 keys (one page) per step.
// Online softmax per quarter; quarters are merged through LDS at the end.
template <int G>
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
  const int h = blockIdx.x;       // kv head
  const int i = blockIdx.y;       // query index within the group
  const int s = blockIdx.z;       // sequence
  const int tid = threadIdx.x, lane = tid & 63;
  const int quarter = tid >> 4;   // 0..15 across the workgroup
  const int dl = (lane & 15) * 8; // this lane's 8 dims
  const int64_t ctx = (int64_t)a.seqlens[s] + i + 1;

  float qv[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const bf16* qp = tok_q(a, (int64_t)s * a.L + i) + (h * G + g) * 128 + dl;
    unpack8(ld16(qp), qv[g]);
#pragma unroll
    for (int d = 0; d < 8; ++d) qv[g][d] *= a.scale;
  }
  float mx[G], sm[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mx[g] = -INFINITY;
    sm[g] = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[g][d] = 0.f;
  }
  const int32_t* bt = a.bt + (int64_t)s * a.max_blocks;
  const int64_t rowstride = (int64_t)a.hkv * 128;
  for (int64_t key = quarter; key < ctx; key += 16) {
    const int64_t bi = key / a.bs;
    int32_t blk = (bi < a.max_blocks) ? bt[bi] : -1;
    if (blk < 0 || blk >= a.num_blocks) continue;
    const int64_t off = ((int64_t)blk * a.bs + key % a.bs) * rowstride + h * 128 + dl;
    float kv[8], vv[8];
    unpack8(ld16(a.kc + off), kv);
    unpack8(ld16(a.vc + off), vv);
    float sc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float t = 0.f;
#pragma unroll
      for (int d = 0; d < 8; ++d) t += qv[g][d] * kv[d];
      sc[g] = t;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) sc[g] += __shfl_xor(sc[g], o, 16);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float nm = fmaxf(mx[g], sc[g]);
      const float corr = __expf(mx[g] - nm);
      const float p = __expf(sc[g] - nm);
      sm[g] = sm[g] * corr + p;
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[g][d] = acc[g][d] * corr + p * vv[d];
      mx[g] = nm;
    }
  }
  // merge the 16 quarters
  __shared__ float smx[16][G], ssm[16][G];
  __shared__ float sacc[16][G][128];
  if ((lane & 15) == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) { smx[quarter][g] = mx[g]; ssm[quarter][g] = sm[g]; }
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int d = 0; d < 8; ++d) sacc[quarter][g][dl + d] = acc[g][d];
  __syncthreads();
  for (int it = tid; it < G * 128; it += 256) {
    const int g = it >> 7, d = it & 127;
    float m = -INFINITY;
    for (int qq = 0; qq < 16; ++qq) m = fmaxf(m, smx[qq][g]);
    float l = 0.f, o = 0.f;
    if (m != -INFINITY) {
      for (int qq = 0; qq < 16; ++qq) {
        const float c = (smx[qq][g] == -INFINITY) ? 0.f : __expf(smx[qq][g] - m);
        l += ssm[qq][g] * c;
        o += sacc[qq][g][d] * c;
      }
    }
    const float r = (l > 0.f) ? o / l : 0.f;
    tok_out(a, (int64_t)s * a.L + i)[(h * G + g) * 128 + d] = f2bf(r);
  }
}

// ---- decode attention, split over the context (flash-decoding) ----------
// One workgroup (WAVES waves) per (kv head, chunk of C keys, sequence) of a
// one-token query: 16 lanes per key (8 dims each), every lane issues all of
// its U K-loads and U V-loads for the chunk at once (page offsets computed
// first), scores for the G query heads sharing the kv head, softmax within
// the chunk, then P.V.  Writes the chunk's max, sum and unnormalised output;
// attn_combine_kernel merges the chunks.  Keys past the context are masked.
constexpr int kAttnRec = 130;  // floats per (chunk, head): max, sum, 128 dims

__device__ __forceinline__ int64_t key_offset(const AttnArgs& a, const int32_t* bt, int64_t key, int h) {
  int64_t bi, in;
  if (a.bs_shift >= 0) {
    bi = key >> a.bs_shift;
    in = key & (a.bs - 1);
  } else {
    bi = key / a.bs;
    in = key - bi * a.bs;
  }
  int32_t blk = (bi < a.max_blocks) ? bt[bi] : 0;
  blk = (blk >= 0 && blk < a.num_blocks) ? blk : 0;
  return ((int64_t)blk * a.bs + in) * a.hkv * 128 + h * 128;
}

template <int G, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void attn_chunk_kernel(AttnArgs a, float* part, int maxch) {
  constexpr int NQ = 4 * WAVES, C = NQ * U, KPL = (C + 63) / 64;
  const int h = blockIdx.x, c = blockIdx.y, s = blockIdx.z;
  const int64_t ctx = (int64_t)a.seqlens[s] + 1;
  const int64_t k0 = (int64_t)c * C;
  if (k0 >= ctx) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int quarter = tid >> 4;  // keys k0 + quarter + NQ * j
  const int dl = (lane & 15) * 8;
  const int32_t* bt = a.bt + (int64_t)s * a.max_blocks;

  int64_t off[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const int64_t key = k0 + quarter + NQ * j;
    off[j] = key_offset(a, bt, key < ctx ? key : k0, h) + dl;
  }
  u32x4 kr[U], vr[U];
#pragma unroll
  for (int j = 0; j < U; ++j) kr[j] = ldg16(a.kc + off[j]);
#pragma unroll
  for (int j = 0; j < U; ++j) vr[j] = ldg16(a.vc + off[j]);
  float qv[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    unpack8(ld16(tok_q(a, s) + (h * G + g) * 128 + dl), qv[g]);
#pragma unroll
    for (int d = 0; d < 8; ++d) qv[g][d] *= a.scale;
  }

  __shared__ float sp[G][C];             // scores, then probabilities
  __shared__ float sred[WAVES][G][128];  // per-wave P.V partials
#pragma unroll
  for (int j = 0; j < U; ++j) {
    float kf[8];
    unpack8(kr[j], kf);
    const int64_t key = k0 + quarter + NQ * j;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float t = 0.f;
#pragma unroll
      for (int d = 0; d < 8; ++d) t += qv[g][d] * kf[d];
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) t += __shfl_xor(t, o, 16);
      if ((lane & 15) == 0) sp[g][quarter + NQ * j] = (key < ctx) ? t : -INFINITY;
    }
  }
  __syncthreads();
  // softmax within the chunk: one wave per head, ceil(C / 64) keys per lane
  float* rec = part + (((int64_t)s * a.hkv + h) * maxch + c) * G * kAttnRec;
  for (int g = wv; g < G; g += WAVES) {
    float sv[KPL];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      sv[i] = (lane + 64 * i < C) ? sp[g][lane + 64 * i] : -INFINITY;
      m = fmaxf(m, sv[i]);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float l = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      if (lane + 64 * i >= C) break;
      const float pi = __expf(sv[i] - m);
      sp[g][lane + 64 * i] = pi;
      l += pi;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o, 64);
    if (lane == 0) {
      rec[g * kAttnRec] = m;
      rec[g * kAttnRec + 1] = l;
    }
  }
  __syncthreads();
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[g][d] = 0.f;
#pragma unroll
  for (int j = 0; j < U; ++j) {
    float vf[8];
    unpack8(vr[j], vf);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float pj = sp[g][quarter + NQ * j];
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[g][d] += pj * vf[d];
    }
  }
  // the 4 quarters of a wave hold the same dims: fold them with shuffles
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      float v = acc[g][d];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      acc[g][d] = v;
    }
  if (lane < 16) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int d = 0; d < 8; ++d) sred[wv][g][dl + d] = acc[g][d];
  }
  __syncthreads();
  for (int it = tid; it < G * 128; it += WAVES * 64) {
    const int g = it >> 7, d = it & 127;
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) o += sred[w][g][d];
    rec[g * kAttnRec + 2 + d] = o;
  }
}

// Merges the chunk records of one (sequence, query head): out = sum_c o_c
// e^(m_c - M) / sum_c l_c e^(m_c - M).  Records are read 16 chunks at a
// time with every load of a batch in flight together (one batch covers
// 16 chunks of the context).
__global__ __launch_bounds__(128) void attn_combine_kernel(AttnArgs a, const float* part, int maxch, int G, int C) {
  constexpr int B = 16;
  const int s = blockIdx.y, hqi = blockIdx.x;
  const int h = hqi / G, g = hqi - h * G;
  const int d = threadIdx.x;
  const int64_t ctx = (int64_t)a.seqlens[s] + 1;
  const int nch = (int)min<int64_t>((ctx + C - 1) / C, maxch);  // contexts past the block table: records end there
  const float* rec = part + ((int64_t)s * a.hkv + h) * maxch * G * kAttnRec + g * kAttnRec;
  const int64_t cstride = (int64_t)G * kAttnRec;
  float M = -INFINITY, L = 0.f, O = 0.f;
  for (int c0 = 0; c0 < nch; c0 += B) {
    float m[B], l[B], o[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int c = c0 + j < nch ? c0 + j : nch - 1;
      m[j] = rec[c * cstride];
      l[j] = rec[c * cstride + 1];
      o[j] = rec[c * cstride + 2 + d];
    }
    float mn = M;
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (c0 + j < nch) mn = fmaxf(mn, m[j]);
    const float corr = (M == -INFINITY) ? 0.f : __expf(M - mn);
    L *= corr;
    O *= corr;
#pragma unroll
    for (int j = 0; j < B; ++j) {
      if (c0 + j >= nch) break;
      const float e = __expf(m[j] - mn);
      L += l[j] * e;
      O += o[j] * e;
    }
    M = mn;
  }
  tok_out(a, s)[hqi * 128 + d] = f2bf(L > 0.f ? O / L : 0.f);
}

// ---- decode attention over whole pages (flash-decoding by parts) --------
// One workgroup of W waves per (kv head, part of a sequence); wave w takes
// the part's tiles of 16 keys (a page, or a 16-key slice of one) w, w + W,
// ... and streams them into its own LDS ring with LDS-DMA, S tiles deep, so
// waves never wait on each other inside the loop.  K is stored in blocks of
// 8 keys x 8 16-byte dim groups (the 16 keys of an MFMA operand read sit in
// distinct banks), V key-major ([key][dims]).  Scores of the G query heads
// on MFMA (the 16 K rows as the A operand, q as the B operand, 16x16x32
// over 4 steps of 32 dims), then online softmax and P.V in-lane (lane group
// = query head, 8 dims a lane).  The W waves' partial results are merged in
// LDS into one record (max, sum, unnormalised output) per (part, query
// head); attn_combine_kernel merges the parts.  Keys past the context are
// masked and their V rows never read.
constexpr int kTileKeys = 16;
// K of a tile: four 1 KiB blocks (dim octet o, key half h at (2 o + h) *
// 1152): 8 keys x 128 bytes each, so every DMA instruction reads whole
// 128-byte lines; the 128-byte skew of the odd blocks puts a dim group's
// two key halves in different banks.  V follows as 16 key rows of 256 bytes.
constexpr int kTileKBlk = 1152;
constexpr int kTileKBytes = 4 * kTileKBlk;
constexpr int kTileBytes = kTileKBytes + kTileKeys * 256;  // one head's K and V rows of a tile

// Max / sum over the 16 lanes of a DPP row, every lane receiving the
// result: xor 1 and xor 2 by quad permutes, then the half-row and row
// mirrors join the quads and the halves.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
  return fmaxf(v, dpp_f<0x140>(v));  // row_mirror
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  return v + dpp_f<0x140>(v);
}

// Size-ordered part numbering for up to 64 sequences: workgroup b (linear
// over the grid) takes kv head b % hkv of part unit b / hkv, where units are
// every sequence's full parts (tpp tiles) in sequence order, then the partial
// last parts from the most tiles to the fewest (ties in sequence order).
// Workgroups past the last unit find none.  Consecutive workgroups land on
// different CUs, so each CU gets about the same number of full parts and at
// most one short one, and no workgroup slot goes to a part past a sequence's
// end.  Every wave computes it on its own (no LDS, no barrier).
__device__ __forceinline__ bool attn_unit_of(const AttnArgs& a, int maxparts, int tpp, int lane, int& h, int& p,
                                             int& s) {
  const int64_t b = blockIdx.x + (int64_t)gridDim.x * (blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
  h = (int)(b % a.hkv);
  const int64_t unit = b / a.hkv;
  // tiles ceil((len + 1) / 16), as the parts see them, capped at the grid's
  // maxparts parts (the parts the sequence-major numbering covers)
  const int64_t len1 = lane < a.nseq ? (int64_t)a.seqlens[lane] + 1 : 0;
  const int nt = (int)min<int64_t>(max<int64_t>(0, (len1 + kTileKeys - 1) / kTileKeys), (int64_t)maxparts * tpp);
  const int F = nt / tpp, R = nt - F * tpp;
  int pf = F;  // inclusive prefix of the full parts
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(pf, off);
    if (lane >= off) pf += y;
  }
  const int total_full = __shfl(pf, 63);
  if (unit < total_full) {
    const uint64_t m = __ballot(pf > unit);
    s = __builtin_ctzll(m);
    p = (int)(unit - (__shfl(pf, s) - __shfl(F, s)));
    return true;
  }
  const int64_t r = unit - total_full;
  int rank = 0;  // among the partial parts, by tiles descending
  for (int j = 0; j < a.nseq; ++j) {
    const int rj = __builtin_amdgcn_readlane(R, j);
    rank += (rj > R || (rj == R && j < lane)) ? 1 : 0;
  }
  const uint64_t m = __ballot(R > 0 && rank == r);
  if (m == 0) return false;
  s = __builtin_ctzll(m);
  p = __shfl(F, s);
  return true;
}

template <int G, int S, int W>
__global__ __launch_bounds__(64 * W) void attn_tile_kernel(AttnArgs a, float* part, int maxparts, int tpp, int order) {
  constexpr int GL = G < 4 ? G : 4;  // lane groups with a query head
  constexpr int HPG = G / GL;        // query heads per lane group
  constexpr int WAVE_LDS = S * kTileBytes + G * kTileKeys * 4 + G * kTileKeys * 2;
  static_assert(W * S * kTileBytes >= W * G * kAttnRec * 4, "merge area must fit in the rings");
  __shared__ __attribute__((aligned(16))) char lds[W * WAVE_LDS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int h = blockIdx.x, p = blockIdx.y, s = blockIdx.z;
  if (order && !attn_unit_of(a, maxparts, tpp, lane, h, p, s)) return;  // uniform over the workgroup
  const int64_t ctx = (int64_t)a.seqlens[s] + 1;
  const int64_t ntiles = (ctx + kTileKeys - 1) / kTileKeys;
  const int64_t tb = (int64_t)p * tpp;  // first tile of the part
  if (tb >= ntiles) return;             // uniform over the workgroup
  const int nt = (int)max<int64_t>(0, min<int64_t>(tpp, (ctx + kTileKeys - 1) / kTileKeys - tb));
  const int ntw = nt > w ? (nt - w + W - 1) / W : 0;  // this wave's tiles: w + j W
  char* ring = lds + w * WAVE_LDS;
  float* sc = reinterpret_cast<float*>(ring + S * kTileBytes);   // [G][16] scores
  bf16* pb = reinterpret_cast<bf16*>(sc + G * kTileKeys);        // [G][16] probabilities

  // key row 0 of each tile of the part (lane t holds tile t's), head h
  const int32_t* bt = a.bt + (int64_t)s * a.max_blocks;
  const int64_t krow = (int64_t)a.hkv * 128;
  int64_t tile_base = 0;
  if (lane < nt) {
    const int64_t key0 = (tb + lane) * kTileKeys;
    int64_t bi, ip;
    if (a.bs_shift >= 0) {
      bi = key0 >> a.bs_shift;
      ip = key0 & (a.bs - 1);
    } else {
      bi = key0 / a.bs;
      ip = key0 - bi * a.bs;
    }
    int32_t blk = bi < a.max_blocks ? bt[bi] : 0;
    blk = (blk >= 0 && blk < a.num_blocks) ? blk : 0;
    tile_base = ((int64_t)blk * a.bs + ip) * krow + (int64_t)h * 128;
  }
  // K: instruction i, lane c -> key 8 (i % 2) + c % 8, dim group
  // 8 (i / 2) + c / 8 (LDS block i, offset ((group % 8) * 8 + key % 8) * 16);
  // V: key 4 i + c / 16, group c % 16 (LDS offset key * 256 + group * 16)
  const int64_t koff = (int64_t)(lane & 7) * krow + 8 * (lane >> 3);
  const int64_t voff = (int64_t)(lane >> 4) * krow + 8 * (lane & 15);
  auto issue = [&](int j) {  // this wave's j-th tile into ring slot j % S
    const int t = w + j * W;
    const int64_t base = (int64_t)(uint32_t)__builtin_amdgcn_readlane((int)(tile_base & 0xffffffff), t) |
                         ((int64_t)__builtin_amdgcn_readlane((int)(tile_base >> 32), t) << 32);
    char* dst = ring + (j % S) * kTileBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds((gbl_ptr)(a.kc + base + koff + (i & 1) * 8 * krow + (i >> 1) * 64),
                                       (lds_ptr)(dst + i * kTileKBlk), 16, 0, kLoadNT);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds((gbl_ptr)(a.vc + base + voff + 4 * i * krow),
                                       (lds_ptr)(dst + kTileKBytes + i * 1024), 16, 0, kLoadNT);
  };

  // q of the G query heads as the MFMA B operand: lane l holds column l % 16
  // (query head, zero past G), dims 32 * step + 8 (l / 16) .. + 7
  u32x4 qf[4];
  {
    const int col = lane & 15;
    const bf16* qp = tok_q(a, s) + (int64_t)(h * G + (col < G ? col : 0)) * 128 + 8 * (lane >> 4);
#pragma unroll
    for (int st = 0; st < 4; ++st) qf[st] = col < G ? ldg16(qp + 32 * st) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < S; ++j)
    if (j < ntw) issue(j);

  const int gg = lane >> 4;  // lane group: query heads gg * HPG ..
  float m[HPG], l[HPG], acc[HPG][8];
#pragma unroll
  for (int j = 0; j < HPG; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[j][d] = 0.f;
  }

  for (int j = 0; j < ntw; ++j) {
    switch (min(S - 1, ntw - 1 - j)) {  // tiles issued after j: 8 DMA each
      case 3: __builtin_amdgcn_s_waitcnt(wait_vm_imm(24)); break;
      case 2: __builtin_amdgcn_s_waitcnt(wait_vm_imm(16)); break;
      case 1: __builtin_amdgcn_s_waitcnt(wait_vm_imm(8)); break;
      default: __builtin_amdgcn_s_waitcnt(wait_vm_imm(0)); break;
    }
    const char* kb = ring + (j % S) * kTileBytes;
    const char* vb = kb + kTileKBytes;
    const int64_t k0 = (tb + w + (int64_t)j * W) * kTileKeys;
    const int nk = (int)min<int64_t>(kTileKeys, ctx - k0);  // valid keys of the tile

    // scores: S[key 4 (l / 16) + i][query head l % 16]
    f32x4 sv = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      // dim group 4 st + gg: octet st / 2, index 4 (st % 2) + gg in it
      const u32x4 kf = *reinterpret_cast<const u32x4*>(kb + (2 * (st >> 1) + ((lane >> 3) & 1)) * kTileKBlk +
                                                       ((4 * (st & 1) + gg) * 8 + (lane & 7)) * 16);
      sv = mfma16(kf, qf[st], sv);
    }
    if ((lane & 15) < G) {
      f32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = (4 * gg + i < nk) ? sv[i] * a.scale : -INFINITY;
      *reinterpret_cast<f32x4*>(sc + (lane & 15) * kTileKeys + 4 * gg) = o;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // online softmax: lane l takes key l % 16 of its lane group's query
    // head; max and sum over the 16 lanes of the group, the probabilities
    // rounded to bf16 into LDS for the P.V pairs
#pragma unroll
    for (int e = 0; e < HPG; ++e) {
      const int g = gg < GL ? gg * HPG + e : 0;
      const float x = sc[g * kTileKeys + (lane & 15)];
      const float mn = fmaxf(m[e], row16_max(x));
      const float corr = __expf(m[e] - mn);
      const float pe = __expf(x - mn);
      l[e] = l[e] * corr + row16_sum(pe);
      m[e] = mn;
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[e][d] *= corr;
      if (gg < GL) pb[g * kTileKeys + (lane & 15)] = f2bf(pe);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the lane group's probabilities as bf16 pairs (keys 2i, 2i + 1)
    uint32_t pp[HPG][kTileKeys / 2];
#pragma unroll
    for (int e = 0; e < HPG; ++e) {
      const int g = gg < GL ? gg * HPG + e : 0;
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(pb + g * kTileKeys);
      const u32x4 a1 = *reinterpret_cast<const u32x4*>(pb + g * kTileKeys + 8);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pp[e][i] = a0[i];
        pp[e][4 + i] = a1[i];
      }
    }
    // P.V over key pairs (k, k + 1): bf16 dot2 of each dim's two V values
    // with the pair's probabilities (bf16, as flash attention's second
    // product takes P), fp32 accumulation.  A full tile unrolled (all V
    // reads in flight together); the context's last tile pair by pair, the
    // V row past its end zeroed (its probability is 0).
    auto pv2 = [&](int k, bool second) {
      const u32x4 w0 = *reinterpret_cast<const u32x4*>(vb + k * 256 + (lane & 15) * 16);
      u32x4 w1 = *reinterpret_cast<const u32x4*>(vb + (k + 1) * 256 + (lane & 15) * 16);
      if (!second) w1 = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < HPG; ++e) {
        const bf16x2 p2 = __builtin_bit_cast(bf16x2, pp[e][k >> 1]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = __builtin_amdgcn_perm(w1[q], w0[q], 0x05040100u);  // dim 2q of keys k, k + 1
          const uint32_t hi = __builtin_amdgcn_perm(w1[q], w0[q], 0x07060302u);  // dim 2q + 1
          acc[e][2 * q] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, lo), p2, acc[e][2 * q], false);
          acc[e][2 * q + 1] =
              __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, hi), p2, acc[e][2 * q + 1], false);
        }
      }
    };
    if (nk == kTileKeys) {
#pragma unroll
      for (int k = 0; k < kTileKeys; k += 2) pv2(k, true);
    } else {
#pragma unroll
      for (int k = 0; k < kTileKeys; k += 2) {
        if (k >= nk) break;
        pv2(k, k + 1 < nk);
      }
    }
    // every lane's LDS reads of this slot are done before it is refilled
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    if (j + S < ntw) issue(j + S);
  }

  // merge the W waves (all their DMA has landed) in LDS over the rings
  float* mg = reinterpret_cast<float*>(lds);  // [W][G][kAttnRec]
  if (W > 1) __syncthreads();
  if (gg < GL) {
#pragma unroll
    for (int e = 0; e < HPG; ++e) {
      float* r = mg + (w * G + gg * HPG + e) * kAttnRec;
      if ((lane & 15) == 0) {
        r[0] = m[e];
        r[1] = l[e];
      }
#pragma unroll
      for (int d = 0; d < 8; ++d) r[2 + (lane & 15) * 8 + d] = acc[e][d];
    }
  }
  __syncthreads();
  for (int it = threadIdx.x; it < G * 128; it += 64 * W) {
    const int g = it >> 7, d = it & 127;
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < W; ++v) M = fmaxf(M, mg[(v * G + g) * kAttnRec]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int v = 0; v < W; ++v) {
      const float* r = mg + (v * G + g) * kAttnRec;
      const float c = r[0] == -INFINITY ? 0.f : __expf(r[0] - M);
      L += r[1] * c;
      O += r[2 + d] * c;
    }
    float* rec = part + ((((int64_t)s * a.hkv + h) * maxparts + p) * G + g) * kAttnRec;
    if (d == 0) {
      rec[0] = M;
      rec[1] = L;
    }
    rec[2 + d] = O;
  }
}

// Fragment-tile packing of a row-major W [N][K]: output 16-byte chunk c =
// ((tile * steps + step) * 64 + lane) holds row 16 tile + lane % 16,
// columns step * 32 + 8 (lane / 16) .. + 7 (zero past row N).
__global__ __launch_bounds__(256) void pack_weight_kernel(const bf16* w, int64_t N, int64_t K, u32x4* out,
                                                         int64_t nchunks) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= nchunks) return;
  const int64_t steps = K >> 5;
  const int lane = (int)(c & 63);
  const int64_t ts = c >> 6;
  const int64_t tile = ts / steps, step = ts - tile * steps;
  const int64_t r = tile * 16 + (lane & 15);
  u32x4 v = u32x4{0u, 0u, 0u, 0u};
  if (r < N) v = ldg16(w + r * K + step * 32 + 8 * (lane >> 4));
  out[c] = v;
}

__global__ void zero_blocks_kernel(bf16* cache, const int64_t* ids, int64_t nblocks, int64_t block_elems) {
  const int64_t b = blockIdx.x;
  if (b >= nblocks) return;
  u32x4* p = reinterpret_cast<u32x4*>(cache + ids[b] * block_elems);
  const int64_t nv = block_elems >> 3;
  for (int64_t e = threadIdx.x; e < nv; e += blockDim.x) p[e] = u32x4{0u, 0u, 0u, 0u};
}

// ------------------------------------------------- worker elementwise ---
template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, Op op, T* sh) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if (lane == 0) sh[wv] = v;
  __syncthreads();
  T r = sh[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = op(r, sh[i]);
  return r;
}

struct RowPtrs {
  int32_t ntok;
  const bf16* in[kSkinnyMaxTok];
  bf16* out[kSkinnyMaxTok];
};

// h[t] = bf16(h[t] + in[t]) when has_add; out[t] = bf16(bf16(h * rsqrt(mean(h^2)
// + eps)) * w): LlamaRMSNorm on the residual stream (worker_sync.py:1344-1350,
// :314-319, :383-389).  One workgroup per token.
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(bf16* __restrict__ h, int64_t d, RowPtrs r,
                                                           const bf16* __restrict__ w, float eps, int has_add) {
  __shared__ float sh[4];
  const int t = blockIdx.x;
  bf16* hr = h + (int64_t)t * d;
  const int64_t nv = d >> 3;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) {
    float x[8];
    unpack8(ld16(hr + 8 * i), x);
    if (has_add) {
      float y[8];
      unpack8(ld16(r.in[t] + 8 * i), y);
      bf16x8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        o[j] = f2bf(x[j] + y[j]);
        x[j] = bf2f(o[j]);
      }
      *reinterpret_cast<u32x4*>(hr + 8 * i) = __builtin_bit_cast(u32x4, o);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
  }
  ss = block_reduce<float>(ss, [](float x, float y) { return x + y; }, sh);
  const float rs = rsqrtf(ss / (float)d + eps);
  for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) {
    float x[8], g[8];
    unpack8(ld16(hr + 8 * i), x);
    unpack8(ld16(w + 8 * i), g);
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = f2bf(bf2f(f2bf(x[j] * rs)) * g[j]);
    *reinterpret_cast<u32x4*>(r.out[t] + 8 * i) = __builtin_bit_cast(u32x4, o);
  }
}

// out[t][j] = bf16(bf16(silu(g)) * u), g = in[t][j], u = in[t][inter + j]
// (F.silu(gate) * up in bf16, worker_sync.py:158, :1397).
__global__ __launch_bounds__(256) void silu_mul_rows_kernel(RowPtrs r, int64_t inter) {
  const int t = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (inter >> 3)) return;
  float g[8], u[8];
  unpack8(ld16(r.in[t] + 8 * i), g);
  unpack8(ld16(r.in[t] + inter + 8 * i), u);
  bf16x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float sg = bf2f(f2bf(g[j] / (1.0f + __expf(-g[j]))));
    o[j] = f2bf(sg * u[j]);
  }
  *reinterpret_cast<u32x4*>(r.out[t] + 8 * i) = __builtin_bit_cast(u32x4, o);
}

// ------------------------------------------------------ embed / LM head ---
struct EmbedArgs {
  int32_t n;
  int64_t off[kMaxSeg + 1];
  const int64_t* ids[kMaxSeg];
  bf16* out[kMaxSeg];
  const bf16* table;
  int64_t vocab, hidden;
};

// One workgroup per token: out row = table[clamp(id, 0, vocab - 1)]
// (torch::embedding of clamped ids, ext_aggregator.cpp:660-705).
__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
  const int64_t row = blockIdx.x;
  const int s = find_seg(a.off, a.n, row);
  const int64_t j = row - a.off[s];
  int64_t id = a.ids[s][j];
  id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);
  const u32x4* src = reinterpret_cast<const u32x4*>(a.table + id * a.hidden);
  u32x4* dst = reinterpret_cast<u32x4*>(a.out[s] + j * a.hidden);
  for (int64_t i = threadIdx.x; i < (a.hidden >> 3); i += blockDim.x) dst[i] = src[i];
}

struct SampleArgs {
  const bf16* logits;       // [n, vocab]
  int64_t vocab;
  int64_t* out_tok[kMaxSeg];
  int32_t do_sample[kMaxSeg];
  float temperature[kMaxSeg];
  int32_t top_k[kMaxSeg];
  float top_p[kMaxSeg];
  uint64_t seed;
};

// order-preserving map of a float to uint32 (larger float -> larger key)
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdull;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ull;
  x ^= x >> 33;
  return x;
}

// One workgroup (1024 threads) per row.  Greedy: first index of the largest
// logit (argmax).  Sampling (ext_aggregator.cpp:756-795): logits/temperature,
// keep the top-k values (ties at the k-th value kept), keep the sorted
// prefix whose cumulative probability does not exceed top_p (the most likely
// token always kept), softmax over the kept set and draw one token with a
// counter-based generator seeded per (call, row).
__global__ __launch_bounds__(1024) void sample_kernel(SampleArgs a) {
  __shared__ float shf[16];
  __shared__ uint32_t shu[16];
  __shared__ unsigned long long shl[16];
  const int row = blockIdx.x;
  const bf16* lg = a.logits + (int64_t)row * a.vocab;
  const int64_t V = a.vocab;
  // argmax with first-index tie break: key = (fkey(v) << 32) | ~index.
  // 16-byte loads (8 logits), four per thread in flight, when the row is
  // 16-byte aligned; scalar loads for the rest.
  unsigned long long best = 0;
  auto take = [&](float v, int64_t i) {
    const unsigned long long k = ((unsigned long long)fkey(v) << 32) | (uint32_t)(~(uint32_t)i);
    best = k > best ? k : best;
  };
  const int64_t nv = (reinterpret_cast<uintptr_t>(lg) & 15) == 0 ? V / 8 : 0;
  for (int64_t j0 = threadIdx.x; j0 < nv; j0 += 4 * (int64_t)blockDim.x) {
    u32x4 q[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t j = j0 + u * (int64_t)blockDim.x;
      q[u] = j < nv ? ldg16(lg + 8 * j) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t j = j0 + u * (int64_t)blockDim.x;
      if (j >= nv) break;
      float f[8];
      unpack8(q[u], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) take(f[e], 8 * j + e);
    }
  }
  for (int64_t i = 8 * nv + threadIdx.x; i < V; i += blockDim.x) take(bf2f(lg[i]), i);
  best = block_reduce<unsigned long long>(best, [](unsigned long long x, unsigned long long y) { return x > y ? x : y; }, shl);
  const int64_t amax = (int64_t)(~(uint32_t)(best & 0xffffffffull));
  if (!a.do_sample[row]) {
    if (threadIdx.x == 0) a.out_tok[row][0] = amax;
    return;
  }
  const float invt = 1.0f / a.temperature[row];
  const float vmax = bf2f(lg[amax]) * invt;
  // top-k threshold key: largest key t with count(key >= t) >= k
  uint32_t tk = 0;
  const int K = a.top_k[row];
  if (K > 0 && K < V) {
    uint32_t lo = 0, hi = 0xffffffffu;
    while (lo < hi) {
      const uint32_t mid = lo + (uint32_t)(((uint64_t)hi - lo + 1) >> 1);
      uint32_t c = 0;
      for (int64_t i = threadIdx.x; i < V; i += blockDim.x) c += fkey(bf2f(lg[i]) * invt) >= mid;
      c = block_reduce<uint32_t>(c, [](uint32_t x, uint32_t y) { return x + y; }, shu);
      if (c >= (uint32_t)K) lo = mid; else hi = mid - 1;
    }
    tk = lo;
  }
  // softmax mass over the top-k set
  float z = 0.f;
  for (int64_t i = threadIdx.x; i < V; i += blockDim.x) {
    const float v = bf2f(lg[i]) * invt;
    if (fkey(v) >= tk) z += __expf(v - vmax);
  }
  z = block_reduce<float>(z, [](float x, float y) { return x + y; }, shf);
  // top-p threshold: smallest key t with mass(key >= t) <= top_p * z
  uint32_t tp = tk;
  const float P = a.top_p[row];
  if (P < 1.0f) {
    uint32_t lo = tk, hi = 0xffffffffu;
    while (lo < hi) {
      const uint32_t mid = lo + (uint32_t)(((uint64_t)hi - lo) >> 1);
      float m = 0.f;
      for (int64_t i = threadIdx.x; i < V; i += blockDim.x) {
        const float v = bf2f(lg[i]) * invt;
        if (fkey(v) >= mid) m += __expf(v - vmax);
      }
      m = block_reduce<float>(m, [](float x, float y) { return x + y; }, shf);
      if (m <= P * z) hi = mid; else lo = mid + 1;
    }
    tp = lo;
  }
  const uint32_t thr = tp > tk ? tp : tk;
  float zk = 0.f;
  for (int64_t i = threadIdx.x; i < V; i += blockDim.x) {
    const float v = bf2f(lg[i]) * invt;
    if (fkey(v) >= thr || i == amax) zk += __expf(v - vmax);
  }
  zk = block_reduce<float>(zk, [](float x, float y) { return x + y; }, shf);
  const uint64_t r = mix64(a.seed * 0x9e3779b97f4a7c15ull + (uint64_t)row + 1);
  const float target = (float)((r >> 40) * (1.0 / 16777216.0)) * zk;
  // inverse CDF in index order: chunk of blockDim elements at a time
  __shared__ float run;
  __shared__ int64_t pick;
  if (threadIdx.x == 0) { run = 0.f; pick = amax; }
  __syncthreads();
  for (int64_t base = 0; base < V; base += blockDim.x) {
    const int64_t i = base + threadIdx.x;
    float p = 0.f;
    if (i < V) {
      const float v = bf2f(lg[i]) * invt;
      if (fkey(v) >= thr || i == amax) p = __expf(v - vmax);
    }
    // inclusive scan of p across the workgroup
    float incl = p;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float t = __shfl_up(incl, o, 64);
      if ((threadIdx.x & 63) >= o) incl += t;
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 63) shf[threadIdx.x >> 6] = incl;
    __syncthreads();
    float wpre = 0.f;
    for (int w = 0; w < (int)(threadIdx.x >> 6); ++w) wpre += shf[w];
    const float before = run + wpre + incl - p;
    const float after = before + p;
    const bool hit = p > 0.f && before <= target && target < after;
    __syncthreads();
    if (hit) pick = i;
    float tot = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) tot += shf[w];
    __syncthreads();
    if (threadIdx.x == 0) run += tot;
    __syncthreads();
    if (run > target) break;
  }
  if (threadIdx.x == 0) a.out_tok[row][0] = pick;
}

// --------------------------------------------------- library scratch ------
// One growable device scratch area per device, used for the decode
// projection's fp32 K-slice partials, the LoRA shrink partials, the
// attention part records and the packed activations of the prefill path.
// Launches that use it must not overlap on one device (calls from several
// streams of one device are to be ordered by the caller; a graph captured
// on one stream is sized by an eager call on another).  Growth calls
// hipMalloc and is refused while the stream is being captured; an outgrown
// area is kept (not freed) until the process ends, because a graph captured
// earlier still references it.  Sizes grow by at least half, so the areas
// kept stay within twice the largest.
struct Scratch {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_scratch_mu;
std::vector<Scratch> g_scratch;
std::vector<void*> g_scratch_kept;

int scratch_get(size_t need, hipStream_t stream, void** out) {
  int dev = 0;
  SWL_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if ((int)g_scratch.size() <= dev) g_scratch.resize(dev + 1);
  Scratch& s = g_scratch[dev];
  if (s.bytes < need) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (stream) SWL_HIP(hipStreamIsCapturing(stream, &cs));
    SWL_CHECK(cs == hipStreamCaptureStatusNone, SWL_ERR_STATE,
              "scratch must grow outside graph capture (run the call once before capturing)");
    size_t nb = std::max({need, s.bytes + s.bytes / 2, (size_t)1 << 20});
    nb = (nb + 4095) & ~(size_t)4095;
    void* p = nullptr;
    SWL_HIP(hipMalloc(&p, nb));
    if (s.ptr) g_scratch_kept.push_back(s.ptr);
    s.ptr = p;
    s.bytes = nb;
  }
  *out = s.ptr;
  return SWL_OK;
}

// ---------------------------------------------------------- launch timer
// Optional HIP-event timing of the decode projection: when armed, every
// launch_skinny call (outside graph capture) launches its base kernel and
// its epilogue kernel with start/stop events that take the dispatches' own
// timestamps, and keeps the launch's algorithmic byte count.  Used by
// benchmarks; single-threaded use only.
struct LaunchTimer {
  bool armed = false;
  int cap = 0;
  int n = 0;
  std::vector<hipEvent_t> ev;  // 4 per record: base start/stop, epilogue start/stop
  std::vector<int64_t> N, K, bytes;
  std::vector<int32_t> ntok;
};
LaunchTimer g_timer;

// Returns the record slot to use for this launch, or -1.
int timer_slot(hipStream_t st) {
  if (!g_timer.armed || g_timer.n >= g_timer.cap) return -1;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return -1;
  return g_timer.n++;
}

hipEvent_t timer_event(int slot, int which) { return slot >= 0 ? g_timer.ev[4 * slot + which] : nullptr; }

// hipLaunchKernelGGL; when timing, hipExtLaunchKernelGGL with the events
// taking the dispatch's own start and end timestamps (no marker packets
// around the kernel)
template <typename K, typename... Args>
void launch_maybe_timed(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, hipEvent_t e0, hipEvent_t e1,
                        Args... args) {
  if (e0 || e1)
    hipExtLaunchKernelGGL(kernel, grid, block, lds, st, e0, e1, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
}

// -------------------------------------------------------------- launchers
int fill_segptrs(SegPtrs& sp, const void* const* ptrs, const int64_t* rows, int n, int64_t d, int64_t* total) {
  SWL_CHECK(n >= 1 && n <= kMaxSeg, SWL_ERR_INVALID, "segment count must be in [1, 128]");
  SWL_CHECK(d > 0, SWL_ERR_INVALID, "row length must be positive");
  sp.n = n;
  sp.off[0] = 0;
  bool vec = (d % 8) == 0;
  for (int i = 0; i < n; ++i) {
    SWL_CHECK(rows[i] >= 0, SWL_ERR_INVALID, "segment rows must be >= 0");
    SWL_CHECK(rows[i] == 0 || ptrs[i] != nullptr, SWL_ERR_INVALID, "null segment pointer");
    sp.off[i + 1] = sp.off[i] + rows[i];
    sp.ptr[i] = ptrs[i];
    if ((reinterpret_cast<uintptr_t>(ptrs[i]) & 15) != 0) vec = false;
  }
  sp.vec = vec ? 1 : 0;
  *total = sp.off[n];
  return SWL_OK;
}

// Launch-shape tuning of the decode path.  Defaults are the measured best on
// MI355X; SWL_SKINNY_WAVES (4, 8 or 16), SWL_SKINNY_WGCU (resident workgroups per
// CU the grid is sized for), SWL_SKINNY_LDS_KB and SWL_SKINNY_NKS override
// them for sweeps.
struct Tuning {
  int waves = 8;
  int wg_per_cu = 3;
  bool shape_forced = false;  // SWL_SKINNY_WAVES / SWL_SKINNY_WGCU given: no per-shape choice
  int lds_kb = 96;      // activation-slice LDS per workgroup (16..160 KiB)
  int slice_steps = 16; // K-slices hold at most this many 32-wide k-steps
  int kd = 8;           // k-steps of W in flight per wave (16: only with 16-wave workgroups)
  int nks = 0;          // forced K-slice count (0: chosen per shape)
  int long_slice = 1 << 20;  // slice cap when the row tiles alone overfill the slots (0: off; default:
                             // the longest slice the LDS holds)
};
const Tuning& tuning() {
  static Tuning t = [] {
    Tuning v;
    if (const char* e = getenv("SWL_SKINNY_WAVES")) {
      v.waves = (atoi(e) == 4 || atoi(e) == 16) ? atoi(e) : 8;
      v.shape_forced = true;
    }
    if (const char* e = getenv("SWL_SKINNY_WGCU")) {
      v.wg_per_cu = std::min(8, std::max(1, atoi(e)));
      v.shape_forced = true;
    }
    if (const char* e = getenv("SWL_SKINNY_LDS_KB")) v.lds_kb = std::min(160, std::max(16, atoi(e)));
    if (const char* e = getenv("SWL_SKINNY_NKS")) v.nks = std::max(0, atoi(e));
    if (const char* e = getenv("SWL_SKINNY_KD")) v.kd = atoi(e) == 16 ? 16 : 8;
    if (const char* e = getenv("SWL_SKINNY_SLICE")) v.slice_steps = std::max(1, atoi(e));
    if (const char* e = getenv("SWL_SKINNY_LONG_SLICE")) v.long_slice = std::max(0, atoi(e));
    return v;
  }();
  return t;
}

// Compute units of the current device (cached per device).
int cu_count() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Dynamic LDS above the default 64 KiB must be allowed per kernel.
template <typename K>
int allow_lds(K kernel, size_t bytes, size_t* allowed) {
  if (bytes <= 64 * 1024 || bytes <= *allowed) return SWL_OK;
  SWL_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)bytes));
  *allowed = bytes;
  return SWL_OK;
}

// Adapter groups for the LoRA shrink: tokens that share a lora table entry.
struct ShrinkPlan {
  int ngroups = 0, tiles = 0;
  int32_t g_entry[kSkinnyMaxTok];
  int32_t g_arows[kSkinnyMaxTok];
  int32_t g_tile0[kSkinnyMaxTok + 1];
  int8_t tok_grp[kSkinnyMaxTok];      // group of each token, -1 for none
};

// tok_lora[i] >= 0: token i uses entry tok_lora[i].  Tokens are grouped per
// entry so each adapter's A is read once per K-slice.
void plan_shrink(ShrinkPlan& p, int ntok, const int32_t* tok_lora, const swl_lora_entry* host_entries, int nblk) {
  p.ngroups = 0;
  p.tiles = 0;
  for (int i = 0; i < ntok; ++i) p.tok_grp[i] = -1;
  for (int i = 0; i < ntok; ++i) {
    const int e = tok_lora[i];
    if (e < 0 || p.tok_grp[i] >= 0) continue;
    const int g = p.ngroups++;
    p.g_entry[g] = e;
    p.g_arows[g] = host_entries[e].rank * nblk;
    p.g_tile0[g] = p.tiles;
    p.tiles += (p.g_arows[g] + 15) / 16;
    for (int j = i; j < ntok; ++j)
      if (tok_lora[j] == e) p.tok_grp[j] = (int8_t)g;
  }
  p.g_tile0[p.ngroups] = p.tiles;
}

template <int TT>
int launch_fullk_t(const FullKArgs& a, dim3 grid, size_t lds, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  static size_t allowed = 0;
  // static LDS: partial sums (16 KiB per token tile), lora_B buffers (16 KiB), tables
  int rc = allow_lds(fullk_kernel<TT>, lds + 16 * 1024 * TT + 16 * 1024 + 2048, &allowed);
  if (rc) return rc;
  launch_maybe_timed(fullk_kernel<TT>, grid, dim3(kFkWaves * 64), lds, st, e0, e1, a);
  return SWL_OK;
}

template <int TT, int W, int KD>
int launch_split_tw(const SplitArgs& a, dim3 grid, size_t lds, hipStream_t st, hipEvent_t tb0, hipEvent_t tb1) {
  static size_t allowed = 0;
  int rc = allow_lds(split_kernel<TT, W, KD>, lds, &allowed);
  if (rc) return rc;
  launch_maybe_timed(split_kernel<TT, W, KD>, grid, dim3(W * 64), lds, st, tb0, tb1, a);
  return SWL_OK;
}

template <int W>
int launch_split_w(int TT, int kd, const SplitArgs& a, dim3 grid, size_t lds, hipStream_t st, hipEvent_t tb0,
                   hipEvent_t tb1) {
  if (W == 16 && kd == 16 && TT <= 2)  // 16 k-steps in flight per wave (one 16-wave workgroup per CU)
    return TT == 1 ? launch_split_tw<1, 16, 16>(a, grid, lds, st, tb0, tb1)
                   : launch_split_tw<2, 16, 16>(a, grid, lds, st, tb0, tb1);
  switch (TT) {
    case 1: return launch_split_tw<1, W, kKDepth>(a, grid, lds, st, tb0, tb1);
    case 2: return launch_split_tw<2, W, kKDepth>(a, grid, lds, st, tb0, tb1);
    case 3: return launch_split_tw<3, W, kKDepth>(a, grid, lds, st, tb0, tb1);
    default: return launch_split_tw<4, W, kKDepth>(a, grid, lds, st, tb0, tb1);
  }
}

// Whole-K decode round (fullk_shrink_kernel when the round has adapters,
// then fullk_kernel): fragment-tile weights (w_layout 2), out_mode 0 (with
// RMSNorm on the way in allowed), at most 32 token rows, K a multiple of 256
// up to 4096.  The decode step's LM head.
int launch_fullk(const bf16* w, const bf16* bias, int64_t N, int64_t K, int ntok, const bf16* const* xrows,
                 bf16* const* yrows, const int32_t* tok_lora, const swl_lora_entry* table,
                 const swl_lora_entry* host_entries, const LoraEpi* Lblk, int nblk, const swl_round_fusion* fz,
                 hipStream_t st, void* ws, size_t ws_bytes) {
  SWL_CHECK(fz->out_mode == 0, SWL_ERR_INVALID, "whole-K round (w_layout 2): out_mode 0 only");
  SWL_CHECK(ntok >= 1 && ntok <= 32, SWL_ERR_INVALID, "whole-K round (w_layout 2): at most 32 token rows");
  SWL_CHECK(K % (32 * kFkWaves) == 0 && K / (32 * kFkWaves) <= kFkMaxSteps, SWL_ERR_INVALID,
            "whole-K round (w_layout 2): K must be a multiple of 256, at most 4096");
  SWL_CHECK(N % 16 == 0, SWL_ERR_INVALID, "whole-K round (w_layout 2): n must be a multiple of 16");
  const int TT = (ntok + 15) / 16;
  FullKArgs a{};
  a.w = w;
  a.N = N;
  a.K = K;
  a.ntok = ntok;
  a.nsw = (int)(K / (32 * kFkWaves));
  a.total_steps = (int)(K / 32);
  a.n_tiles = (int)(N / 16);
  for (int i = 0; i < ntok; ++i) {
    a.x[i] = xrows[i];
    a.y[i] = yrows[i];
  }
  if (fz->norm_weight) {
    a.gamma = reinterpret_cast<const bf16*>(fz->norm_weight);
    a.ss = fz->ss_in;
    a.ss_n = fz->ss_in_n;
    a.ss_stride = fz->ss_in_stride;
    a.eps = fz->eps;
  }
  a.bias = bias;
  bool has_lora = false;
  if (tok_lora)
    for (int i = 0; i < ntok; ++i) has_lora |= tok_lora[i] >= 0;
  ShrinkPlan sp;
  if (has_lora) {
    plan_shrink(sp, ntok, tok_lora, host_entries, nblk);
    int max_r = 0;
    a.ngroups = sp.ngroups;
    for (int g = 0; g < sp.ngroups; ++g) {
      a.g_a[g] = reinterpret_cast<const bf16*>(host_entries[sp.g_entry[g]].a);
      a.g_arows[g] = sp.g_arows[g];
      a.g_tile0[g] = sp.g_tile0[g];
      max_r = std::max(max_r, host_entries[sp.g_entry[g]].rank);
    }
    a.g_tile0[sp.ngroups] = sp.g_tile0[sp.ngroups];
    for (int i = 0; i < ntok; ++i) {
      a.tok_grp[i] = sp.tok_grp[i];
      a.lora[i] = tok_lora[i];
    }
    a.u_ld = max_r * nblk;
    SWL_CHECK(a.u_ld <= kMaxURow, SWL_ERR_INVALID, "round: LoRA rank x blocks exceeds 256");
    a.has_lora = 1;
    a.bdma = 1;
    for (int g = 0; g < sp.ngroups; ++g) a.bdma &= host_entries[sp.g_entry[g]].rank == 16 ? 1 : 0;
    a.nblk = nblk;
    a.table = table;
    for (int b = 0; b <= SWL_MAX_LORA_BLOCKS; ++b) a.blk_start[b] = Lblk->blk_start[b];
  } else {
    for (int i = 0; i < ntok; ++i) a.lora[i] = -1;
  }
  // LDS of the shrink rows: [ntok][u_ld + 4] floats
  const size_t us_bytes = has_lora ? sizeof(float) * (size_t)ntok * (a.u_ld + 4) : 0;
  if (has_lora) {
    const size_t u_bytes = sizeof(float) * (size_t)kFkShrinkKs * ntok * a.u_ld;
    void* scr = ws;
    if (ws) {
      SWL_CHECK(u_bytes <= ws_bytes, SWL_ERR_INVALID, "whole-K round: shrink rows exceed the allocation-free scratch");
    } else {
      int rc = scratch_get(u_bytes, st, &scr);
      if (rc) return rc;
    }
    a.u = reinterpret_cast<float*>(scr);
  }
  const dim3 grid((unsigned)std::min<int64_t>(a.n_tiles, cu_count()));
  const int tslot = timer_slot(st);
  if (has_lora) {
    // timed in the record's second slot (the K-sliced round's epilogue slot)
    launch_maybe_timed(fullk_shrink_kernel, dim3((unsigned)sp.tiles, (unsigned)kFkShrinkKs), dim3(256), 0, st,
                       timer_event(tslot, 2), timer_event(tslot, 3), a);
    SWL_LAUNCH_CHECK("fullk_shrink_kernel launch");
  }
  if (tslot >= 0) {
    int64_t bytes = 2 * (N * K + (int64_t)ntok * K);
    for (int g = 0; g < sp.ngroups && has_lora; ++g) bytes += 2 * (int64_t)sp.g_arows[g] * K;
    g_timer.N[tslot] = N;
    g_timer.K[tslot] = K;
    g_timer.ntok[tslot] = ntok;
    g_timer.bytes[tslot] = bytes;
  }
  hipEvent_t e0 = timer_event(tslot, 0), e1 = timer_event(tslot, 1);
  int rc = TT == 1 ? launch_fullk_t<1>(a, grid, us_bytes, st, e0, e1) : launch_fullk_t<2>(a, grid, us_bytes, st, e0, e1);
  if (rc) return rc;
  SWL_LAUNCH_CHECK("fullk_kernel launch");
  if (tslot >= 0 && !has_lora) {
    // no shrink kernel: its events mark an empty interval after the round
    SWL_HIP(hipEventRecord(timer_event(tslot, 2), st));
    SWL_HIP(hipEventRecord(timer_event(tslot, 3), st));
  }
  return SWL_OK;
}

// Epilogue workgroups resident per CU (registers bound it; cached)
template <int MODE, int Q>
int epi_occupancy() {
  static const int occ = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, epilogue_kernel<MODE, Q>, 256, 0) != hipSuccess || n <= 0)
      n = 1;
    return n;
  }();
  return occ;
}

// Decode-shaped projection of ntok (<= 64) token rows: y[i] = x[i] . W^T
// (+ bias) (+ LoRA delta of entry tok_lora[i]).  xrows[i] / yrows[i] are the
// token's input / output rows (slot buffers).
// ws / ws_bytes: a fixed workspace to use instead of the library scratch
// (the allocation-free entry point); the launch is refused if it does not fit.
int launch_skinny(const bf16* w, const bf16* bias, int64_t N, int64_t K, int ntok, const bf16* const* xrows,
                  bf16* const* yrows, const int32_t* tok_lora, const swl_lora_entry* table,
                  const swl_lora_entry* host_entries, const LoraEpi* Lblk, int nblk, const swl_round_fusion* fz,
                  hipStream_t st, void* ws = nullptr, size_t ws_bytes = 0) {
  const int TT = (ntok + 15) / 16;
  const int mode = fz ? fz->out_mode : 0;
  const int64_t epi_cols = mode == 2 ? N / 2 : N;
  if (fz) {
    SWL_CHECK(mode >= 0 && mode <= 3, SWL_ERR_INVALID, "round fusion: out_mode must be 0..3");
    SWL_CHECK(fz->w_layout >= 0 && fz->w_layout <= 2, SWL_ERR_INVALID, "round fusion: w_layout must be 0, 1 or 2");
    SWL_CHECK(fz->a_layout == 0 || (fz->a_layout == 1 && fz->w_layout != 2), SWL_ERR_INVALID,
              "round fusion: a_layout must be 0, or 1 (fragment-tile lora_A) with w_layout 0 or 1");
    if (fz->norm_weight)
      SWL_CHECK(fz->ss_in && fz->ss_in_n >= 1 && fz->ss_in_stride >= fz->ss_in_n, SWL_ERR_INVALID,
                "round fusion: norm_weight needs ss_in with ss_in_n >= 1 partial sums per row");
    if (mode == 1)
      SWL_CHECK(fz->ss_out && fz->ss_out_stride >= (N + 255) / 256, SWL_ERR_INVALID,
                "round fusion: out_mode 1 needs ss_out with ss_out_stride >= ceil(n / 256)");
    if (mode == 2) SWL_CHECK(N % 2 == 0, SWL_ERR_INVALID, "round fusion: out_mode 2 needs n = 2 * inter");
    if (mode == 3)
      SWL_CHECK(fz->hq > 0 && fz->hkv > 0 && N == (int64_t)(fz->hq + 2 * fz->hkv) * 128 && fz->k_cache &&
                    fz->v_cache && fz->block_table && fz->cache_seqlens && fz->positions && fz->cos_sin &&
                    fz->block_size > 0 && fz->max_blocks > 0 && fz->max_pos > 0,
                SWL_ERR_INVALID, "round fusion: out_mode 3 needs n = (hq + 2 hkv) * 128 and the KV / RoPE arguments");
  }
  if (fz && fz->w_layout == 2)
    return launch_fullk(w, bias, N, K, ntok, xrows, yrows, tok_lora, table, host_entries, Lblk, nblk, fz, st, ws,
                        ws_bytes);
  const int64_t total_steps = K / 32;
  SplitArgs a{};
  a.w = w;
  a.w_packed = (fz && fz->w_layout == 1) ? 1 : 0;
  a.a_packed = (fz && fz->a_layout == 1) ? 1 : 0;
  a.N = N;
  a.K = K;
  a.ntok = ntok;
  a.total_steps = (int)total_steps;
  a.n_wtiles = (int)((N + 15) / 16);
  for (int i = 0; i < ntok; ++i) a.x[i] = xrows[i];
  if (fz && fz->norm_weight) {
    a.gamma = reinterpret_cast<const bf16*>(fz->norm_weight);
    a.ss = fz->ss_in;
    a.ss_n = fz->ss_in_n;
    a.ss_stride = fz->ss_in_stride;
    a.eps = fz->eps;
  }

  bool has_lora = false;
  if (tok_lora)
    for (int i = 0; i < ntok; ++i) has_lora |= tok_lora[i] >= 0;
  ShrinkPlan sp;
  int max_r = 0;
  if (has_lora) {
    plan_shrink(sp, ntok, tok_lora, host_entries, nblk);
    a.ngroups = sp.ngroups;
    for (int g = 0; g < sp.ngroups; ++g) {
      a.g_a[g] = reinterpret_cast<const bf16*>(host_entries[sp.g_entry[g]].a);
      a.g_arows[g] = sp.g_arows[g];
      a.g_tile0[g] = sp.g_tile0[g];
      max_r = std::max(max_r, host_entries[sp.g_entry[g]].rank);
    }
    a.g_tile0[sp.ngroups] = sp.g_tile0[sp.ngroups];
    for (int i = 0; i < ntok; ++i) a.tok_grp[i] = sp.tok_grp[i];
    a.u_ld = ((max_r * nblk + 15) / 16) * 16;
    SWL_CHECK(a.u_ld <= kMaxURow, SWL_ERR_INVALID, "round: LoRA rank x blocks exceeds 256");
    a.u_split_stride = (int64_t)ntok * a.u_ld;
  }

  const Tuning& tu = tuning();
  int waves = tu.waves;
  a.n_tiles = a.n_wtiles + sp.tiles;
  const int64_t tile_groups = (a.n_tiles + waves - 1) / waves;
  // resident workgroups: the kernel keeps 6 waves per SIMD up to 32 token
  // rows (80 VGPRs), 4 beyond (wider accumulators)
  int64_t slots = (int64_t)cu_count() * (TT <= 2 ? tu.wg_per_cu : std::min(tu.wg_per_cu, 16 / waves));
  // K-slices: a power of two (slice starts on aligned byte offsets stream
  // best from HBM), the smallest whose slices hold at most slice_steps
  // k-steps (longer slices write fewer fp32 partials but stage more
  // activation rows per workgroup and leave fewer workgroups per CU; 16
  // steps measured best at 28 rows: O round 8 slices 19.9 us with its
  // epilogue, 16 slices 21.5, 4 slices 21.9), then as many more as the LDS
  // cap on the staged activation slice (padded steps x TT x 1 KiB) requires.
  // Every slice gets all the workers the resident slots allow.
  // When the row tiles alone outnumber the slots (the LM head), slices of up
  // to long_slice steps, by default the longest the 160 KiB of LDS holds:
  // fewer fp32 partials, and the one workgroup per CU the staged slice
  // leaves resident still has many tiles (LM head at 28 rows: 2 slices of
  // 64 steps 220 us, 4 of 32 steps 246 us).
  int kd = (tu.kd == 16 && waves == 16 && TT <= 2) ? 16 : kKDepth;
  auto padded = [&](int64_t nk) { return ((total_steps + nk - 1) / nk + kd - 1) / kd * kd; };
  const bool long_rows = tu.long_slice > 0 && tile_groups > slots;
  const int slice_cap = long_rows ? tu.long_slice : tu.slice_steps;
  auto lds_of = [&](int64_t nk) {  // staged slice (+ RMSNorm gamma and row factors)
    int64_t l = padded(nk) * TT * 1024;
    if (a.gamma) l += (padded(nk) * 32 + 511) / 512 * 1024 + 64 * (int64_t)sizeof(float);
    return l;
  };
  const int64_t lds_cap = long_rows ? 160 * 1024 : (int64_t)tu.lds_kb * 1024;
  int64_t n_ks = 1;
  if (tu.nks > 0) {
    n_ks = tu.nks;
  } else {
    while (n_ks < total_steps && (total_steps + n_ks - 1) / n_ks > slice_cap) n_ks *= 2;
  }
  while (n_ks < total_steps && lds_of(n_ks) > lds_cap) n_ks *= 2;
  n_ks = std::min<int64_t>(n_ks, total_steps);
  // One 16-wave workgroup per CU rather than several 8-wave ones (when the
  // row tiles do not overfill the slots): the workgroups of a CU would stage
  // the same K-slice of the token rows several times.  Waves with three
  // tiles or more (Gate+Up at 28 rows: 3.6) keep 16 k-steps of W in flight
  // instead of 8 (up to 32 token rows; the 16-deep variant is not built for
  // wider token tiles).  Measured per round (28 rows, us, three 8-wave
  // workgroups -> one 16-wave, depth 8 -> depth 16): QKV 18.6 -> 16.8, O 14.3
  // -> 13.0, Down 30.4 -> 29.2, Gate+Up 57.1 -> 57.6 -> 56.7; at 64 rows (two
  // 8-wave workgroups -> one 16-wave, round with its epilogue): QKV 26.7 ->
  // 25.1, O 20.4 -> 18.6, Gate+Up 97.1 -> 89.7, Down 49.5 -> 42.0.
  if (!tu.shape_forced && !long_rows && TT <= 4 && waves == 8) {
    waves = 16;
    slots = cu_count();
    if ((double)a.n_tiles * n_ks >= 3.0 * (double)slots * waves && (total_steps + n_ks - 1) / n_ks > 8) {
      if (TT <= 2) kd = 16;
      // and twice as long K-slices where the CU's one workgroup can stage
      // them (half the fp32 partials; Gate+Up 71.7 -> 70.5 us with its
      // epilogue at 4 slices of 32 steps)
      if (tu.nks == 0 && n_ks >= 2 && lds_of(n_ks / 2) <= 160 * 1024) n_ks /= 2;
    } else if (tu.nks == 0 && n_ks >= 32 && lds_of(n_ks / 2) <= 160 * 1024) {
      // long-K rounds (Down at 28 rows: 32 slices of 14 steps) take half as
      // many slices of twice the steps, 16 k-steps in flight: half the fp32
      // partials (Down 29.2 + 7.3 -> 28.9 + 6.3 us with its epilogue, 6.11 ->
      // 6.04 ms per config-4 step)
      if (TT <= 2) kd = 16;
      n_ks /= 2;
    }
  }
  a.n_ks = (int)n_ks;
  a.ks_steps = (int)padded(n_ks);  // the widest slice, padded to whole pipeline iterations
  // workgroups resident per CU given the staged slice's LDS (160 KiB per CU)
  size_t lds = (size_t)a.ks_steps * TT * 1024;
  if (a.gamma) lds += (size_t)(a.ks_steps * 32 + 511) / 512 * 1024 + 64 * sizeof(float);
  SWL_CHECK(lds <= 160 * 1024, SWL_ERR_INVALID, "round: staged activation slice exceeds LDS");
  const int64_t res_slots = std::min<int64_t>(slots, (int64_t)cu_count() * std::max<int64_t>(1, (160 * 1024) / lds));
  // workers per K-slice: every resident slot (grid = slots per CU x CUs,
  // the same number of workgroups on every CU), at most one per row tile.
  // The kernel deals a slice's tiles round-robin over its workers first, so
  // workgroups differ by at most one tile and every CU streams the same
  // bytes: a CU's share of HBM bandwidth is what sets how long its
  // workgroups run (measured per CU: end times follow the CU's bytes)
  a.n_workers = (int)std::max<int64_t>(1, std::min<int64_t>(a.n_tiles, res_slots / n_ks));

  const size_t part_bytes = sizeof(float) * (size_t)a.n_ks * ntok * N;
  SWL_CHECK(part_bytes < ((size_t)1 << 31), SWL_ERR_INVALID, "round: K-slice partials exceed 2 GiB");
  const size_t part_al = (part_bytes + 255) & ~(size_t)255;
  const size_t u_bytes = has_lora ? sizeof(float) * (size_t)a.n_ks * a.u_split_stride : 0;
  void* scr = ws;
  if (ws) {
    SWL_CHECK(part_al + u_bytes <= ws_bytes, SWL_ERR_INVALID,
              "round: needs " + std::to_string(part_al + u_bytes) + " bytes of K-slice partials, more than the " +
                  std::to_string(ws_bytes) + " bytes of the allocation-free scratch");
  } else {
    int rc = scratch_get(part_al + u_bytes, st, &scr);
    if (rc) return rc;
  }
  a.part = reinterpret_cast<float*>(scr);
  a.u = has_lora ? reinterpret_cast<float*>(reinterpret_cast<char*>(scr) + part_al) : nullptr;

  const dim3 grid((unsigned)(a.n_ks * a.n_workers));
  const int tslot = timer_slot(st);
  if (tslot >= 0) {
    // algorithmic bytes of the base kernel: W and the token rows once, each
    // distinct adapter's stacked A once
    int64_t bytes = 2 * (N * K + (int64_t)ntok * K);
    for (int g = 0; g < sp.ngroups && has_lora; ++g) bytes += 2 * (int64_t)sp.g_arows[g] * K;
    g_timer.N[tslot] = N;
    g_timer.K[tslot] = K;
    g_timer.ntok[tslot] = ntok;
    g_timer.bytes[tslot] = bytes;
  }
  hipEvent_t tb0 = timer_event(tslot, 0), tb1 = timer_event(tslot, 1);
  {
    int rc2 = SWL_OK;
    switch (waves) {
      case 4: rc2 = launch_split_w<4>(TT, kd, a, grid, lds, st, tb0, tb1); break;
      case 16: rc2 = launch_split_w<16>(TT, kd, a, grid, lds, st, tb0, tb1); break;
      default: rc2 = launch_split_w<8>(TT, kd, a, grid, lds, st, tb0, tb1); break;
    }
    if (rc2) return rc2;
  }
  SWL_LAUNCH_CHECK("split_kernel launch");


  EpiArgs e{};
  e.part = a.part;
  e.n_ks = a.n_ks;
  e.ntok = ntok;
  e.N = N;
  e.bias = bias;
  e.has_lora = has_lora ? 1 : 0;
  for (int i = 0; i < ntok; ++i) {
    e.y[i] = yrows[i];
    e.lora[i] = (has_lora && tok_lora[i] >= 0) ? tok_lora[i] : -1;
    e.urow[i] = i;
  }
  if (has_lora) {
    e.L = *Lblk;
    e.L.table = table;
    e.L.u = a.u;
    e.L.usplit = a.n_ks;
    e.L.u_ld = a.u_ld;
    e.L.u_split_stride = a.u_split_stride;
  }
  if (fz) {
    e.ss_out = fz->ss_out;
    e.ss_stride = fz->ss_out_stride;
    e.inter = N / 2;
    e.kc = reinterpret_cast<bf16*>(fz->k_cache);
    e.vc = reinterpret_cast<bf16*>(fz->v_cache);
    e.bt = fz->block_table;
    e.seqlens = fz->cache_seqlens;
    e.pos = fz->positions;
    e.cs = reinterpret_cast<const bf16*>(fz->cos_sin);
    e.max_blocks = fz->max_blocks;
    e.num_blocks = fz->num_blocks;
    e.max_pos = fz->max_pos;
    e.hq = fz->hq;
    e.hkv = fz->hkv;
    e.bs = fz->block_size;
  }
  // quad slots per lane (modes 0 and 2): the fewest with which the grid
  // runs in the fewest waves of resident workgroups (Gate+Up's SiLU
  // epilogue at 28 rows: 1568 workgroups of one slot, 784 of two)
  const int64_t quads = (epi_cols + 3) / 4;
  int q = 1;
  if (mode == 0 || mode == 2) {
    const int64_t cus = cu_count();
    auto waves_of = [&](int qq, int occ) {
      const int64_t wgs = (quads + 64 * qq - 1) / (64 * qq) * ntok;
      return (wgs + occ * cus - 1) / (occ * cus);
    };
    const int occ1 = mode == 2 ? epi_occupancy<2, 1>() : epi_occupancy<0, 1>();
    const int occ2 = mode == 2 ? epi_occupancy<2, 2>() : epi_occupancy<0, 2>();
    int64_t best = waves_of(1, occ1);
    if (waves_of(2, occ2) < best) {
      best = waves_of(2, occ2);
      q = 2;
    }
    if (mode == 0 && waves_of(4, epi_occupancy<0, 4>()) < best) q = 4;
  }
  const dim3 egrid((unsigned)((quads + 64 * q - 1) / (64 * q)), (unsigned)ntok);
  hipEvent_t te0 = timer_event(tslot, 2), te1 = timer_event(tslot, 3);
  switch (mode * 8 + q) {
    case 8 + 1: launch_maybe_timed(epilogue_kernel<1>, egrid, dim3(256), 0, st, te0, te1, e); break;
    case 16 + 1: launch_maybe_timed(epilogue_kernel<2>, egrid, dim3(256), 0, st, te0, te1, e); break;
    case 16 + 2: launch_maybe_timed(epilogue_kernel<2, 2>, egrid, dim3(256), 0, st, te0, te1, e); break;
    case 24 + 1: launch_maybe_timed(epilogue_kernel<3>, egrid, dim3(256), 0, st, te0, te1, e); break;
    case 2: launch_maybe_timed(epilogue_kernel<0, 2>, egrid, dim3(256), 0, st, te0, te1, e); break;
    case 4: launch_maybe_timed(epilogue_kernel<0, 4>, egrid, dim3(256), 0, st, te0, te1, e); break;
    default: launch_maybe_timed(epilogue_kernel<0>, egrid, dim3(256), 0, st, te0, te1, e); break;
  }
  SWL_LAUNCH_CHECK("epilogue_kernel launch");
  return SWL_OK;
}

// Prefill GEMM: gemm256_kernel (256 x 256 or 256 x 192 tiles); the 128 x
// 128 tiled_kernel over a gathered copy takes the rounds whose K is not a
// multiple of the 256 x 256 kernel's 64-wide stages.
bool prefill_uses_tiled(int64_t K) { return K % PG_K != 0 || K < PG_K; }

template <int NJ, int WM>
int launch_gemm256(const TiledArgs& a, int tiles_m, int tiles, int per_xcd, int gm, hipStream_t st) {
  constexpr size_t lds = PgGeom<NJ, WM>::LDS;
  static size_t allowed = 0;
  int rc = allow_lds(gemm256_kernel<NJ, WM>, lds, &allowed);
  if (rc) return rc;
  hipLaunchKernelGGL((gemm256_kernel<NJ, WM>), dim3((unsigned)(8 * per_xcd)), dim3(128 * WM), lds, st, a, tiles_m,
                     tiles, per_xcd, gm);
  return SWL_OK;
}

int launch_prefill_gemm(const TiledArgs& a, hipStream_t st) {
  if (prefill_uses_tiled(a.K)) {
    const dim3 grid((unsigned)((a.N + TN - 1) / TN), (unsigned)((a.M + TM - 1) / TM));
    hipLaunchKernelGGL(tiled_kernel, grid, dim3(256), 0, st, a);
    SWL_LAUNCH_CHECK("tiled_kernel launch");
    return SWL_OK;
  }
  // token rows a tile: 256, or 192 where the grid then covers the CUs in
  // fewer tile times (a 192-row tile measured at ~0.9 of a 256-row one: the
  // W side streams the same bytes): the O and Down rounds at 2325 rows have
  // 160 tiles of 256 for 256 CUs, 208 of 192 (146 -> 133 us, 370 -> 335).
  // A tile of the last row tile costs the share of its first row wave's
  // 32-row blocks that hold rows, at least 0.4 of a full tile (its stages
  // still wait for their DMA); such tiles first fill the CUs the last wave
  // of full tiles leaves idle.
  const int tiles_n = (int)((a.N + PG_N - 1) / PG_N);
  const int64_t cus = cu_count();
  auto cost = [&](int nj) {
    const int64_t mt = 64 * nj, full = (a.M / mt) * tiles_n, rem = a.M % mt;
    const double pc = rem ? std::max(0.4, (double)std::min<int64_t>(nj, (rem + 31) / 32) / nj) : 0.0;
    const int64_t waves = (full + cus - 1) / cus;
    const double spill = (rem ? pc * tiles_n : 0.0) - (double)(waves * cus - full);
    const double t = (double)waves + (spill > 0 ? std::ceil(spill / ((double)cus * pc)) * pc : 0.0);
    return t * (nj == 3 ? 0.9 : 1.0);
  };
  static const int forced = [] {
    const char* e = getenv("SWL_PREFILL_NJ");
    return e ? atoi(e) : 0;
  }();
  const int nj = (forced == 3 || forced == 4) ? forced : (cost(3) < cost(4) ? 3 : 4);
  const int tiles_m = (int)((a.M + 64 * nj - 1) / (64 * nj));
  const int tiles = tiles_m * tiles_n;
  const int per_xcd = (tiles + 7) / 8;
  // Tile order.  Every XCD (workgroup i on XCD i % 8) walks a contiguous run
  // of per_xcd linear tiles.  When all tiles run at once (no more tiles than
  // CUs), the run covers a near-square block of row x column tiles (groups
  // of gm ~ sqrt(per_xcd) row tiles): at each k-stage the XCD then reads
  // fewer distinct W and row slices than with all row tiles of a column
  // fastest.  Rounds of several waves keep the rows fastest (one group).
  int gm = tiles_m;
  if (tiles <= cus) gm = std::max(1, std::min(tiles_m, (int)std::lround(std::sqrt((double)per_xcd))));
  const int rc = nj == 3 ? launch_gemm256<3, 2>(a, tiles_m, tiles, per_xcd, gm, st)
                          : launch_gemm256<4, 2>(a, tiles_m, tiles, per_xcd, gm, st);
  if (rc) return rc;
  SWL_LAUNCH_CHECK("gemm256_kernel launch");
  return SWL_OK;
}

// LoRA shrink of the packed prefill batch (one launch for all segments with
// an adapter): seg_off / seg_rows are packed row offsets and counts; the u
// rows are packed rows; n_ks K-slices of partials, folded into the first.
int launch_shrink_gemm(const bf16* const* seg_x, int64_t K, int n_seg, const int64_t* seg_off,
                       const int64_t* seg_rows, const int32_t* seg_lora, const swl_lora_entry* host_entries, int nblk,
                       float* u, int u_ld, int64_t u_split_stride, int n_ks, hipStream_t st) {
  ShrinkGemmArgs a{};
  a.u = u;
  a.K = K;
  a.u_split_stride = u_split_stride;
  a.n_ks = n_ks;
  a.u_ld = u_ld;
  a.total_steps = (int)(K / 32);
  int items = 0;
  for (int i = 0; i < n_seg; ++i) {
    if (seg_lora[i] < 0 || seg_rows[i] == 0) continue;
    const int j = a.n_seg++;
    a.xs[j] = seg_x[i];
    a.item0[j] = items;
    a.row0[j] = (int32_t)seg_off[i];
    a.rows[j] = (int32_t)seg_rows[i];
    a.arows[j] = host_entries[seg_lora[i]].rank * nblk;
    a.a[j] = reinterpret_cast<const bf16*>(host_entries[seg_lora[i]].a);
    items += (int)((seg_rows[i] + 63) / 64) * ((a.arows[j] + 63) / 64);
  }
  if (a.n_seg == 0) return SWL_OK;
  a.item0[a.n_seg] = items;
  hipLaunchKernelGGL(shrink_gemm_kernel, dim3((unsigned)(items * n_ks)), dim3(256), 0, st, a);
  SWL_LAUNCH_CHECK("shrink_gemm_kernel launch");
  if (n_ks > 1) {
    SWL_CHECK(n_ks <= kFoldMax, SWL_ERR_INVALID, "shrink: at most 16 K-slices");
    const int64_t nvec = u_split_stride / 4;  // u_ld is a multiple of 16
    hipLaunchKernelGGL(u_fold_kernel, dim3((unsigned)((nvec + 255) / 256)), dim3(256), 0, st, u, u_split_stride,
                       n_ks, nvec);
    SWL_LAUNCH_CHECK("u_fold_kernel launch");
  }
  return SWL_OK;
}

template <int G, int WAVES, int U>
int launch_attn_decode(const AttnArgs& a, hipStream_t st) {
  // chunk count from the longest context the block table can hold (host
  // side geometry, never device memory)
  constexpr int C = 4 * WAVES * U;
  const int maxch = (int)((a.max_blocks * a.bs + C - 1) / C);
  void* scr = nullptr;
  const size_t need = sizeof(float) * (size_t)a.nseq * a.hkv * maxch * G * kAttnRec;
  int rc = scratch_get(need, st, &scr);
  if (rc) return rc;
  float* part = reinterpret_cast<float*>(scr);
  hipLaunchKernelGGL((attn_chunk_kernel<G, WAVES, U>), dim3((unsigned)a.hkv, (unsigned)maxch, (unsigned)a.nseq),
                     dim3(WAVES * 64), 0, st, a, part, maxch);
  SWL_LAUNCH_CHECK("attn_chunk_kernel launch");
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)a.hq, (unsigned)a.nseq), dim3(128), 0, st, a,
                     (const float*)part, maxch, G, C);
  SWL_LAUNCH_CHECK("attn_combine_kernel launch");
  return SWL_OK;
}

// keys per lane of the decode attention chunk (SWL_ATTN_U: 4, 8 or 16;
// G = 8 uses at most 8)
int attn_u() {
  static int u = [] {
    const char* e = getenv("SWL_ATTN_U");
    const int v = e ? atoi(e) : 8;
    return (v == 4 || v == 16) ? v : 8;
  }();
  return u;
}

template <int G>
int launch_attn_decode_u(const AttnArgs& a, hipStream_t st) {
  const int u = (G == 8 && attn_u() > 8) ? 8 : attn_u();
  switch (u) {
    case 4: return launch_attn_decode<G, 4, 4>(a, st);
    case 16: return launch_attn_decode<G, 4, (G == 8 ? 8 : 16)>(a, st);
    default: return launch_attn_decode<G, 4, 8>(a, st);
  }
}

// Page-streaming decode attention geometry: waves per workgroup (W, 1 2 4
// or 8), tiles of 16 keys per part (SWL_ATTN_TPP), LDS ring depth per wave
// (SWL_ATTN_STAGES, 2..4); SWL_ATTN_TILE=0 selects the per-chunk kernel.
struct AttnTileTuning {
  bool on = true;
  int waves = 2, tpp = 16, stages = 2, order = 1;
};
const AttnTileTuning& attn_tile_tuning() {
  static AttnTileTuning t = [] {
    AttnTileTuning v;
    if (const char* e = getenv("SWL_ATTN_TILE")) v.on = atoi(e) != 0;
    if (const char* e = getenv("SWL_ATTN_WAVES")) {
      const int x = atoi(e);
      v.waves = (x == 2 || x == 4 || x == 8) ? x : 1;
    }
    if (const char* e = getenv("SWL_ATTN_TPP")) v.tpp = std::max(1, std::min(64, atoi(e)));
    if (const char* e = getenv("SWL_ATTN_STAGES")) v.stages = std::max(2, std::min(4, atoi(e)));
    if (const char* e = getenv("SWL_ATTN_ORDER")) v.order = atoi(e) != 0;
    v.tpp = std::max(v.tpp, v.waves);
    return v;
  }();
  return t;
}

template <int G, int S, int W>
int launch_attn_tile_sw(const AttnArgs& a, hipStream_t st, int tpp, int order) {
  const int64_t max_tiles = (a.max_blocks * a.bs + kTileKeys - 1) / kTileKeys;
  const int maxparts = (int)((max_tiles + tpp - 1) / tpp);
  void* scr = nullptr;
  const size_t need = sizeof(float) * (size_t)a.nseq * a.hkv * maxparts * G * kAttnRec;
  int rc = scratch_get(need, st, &scr);
  if (rc) return rc;
  float* part = reinterpret_cast<float*>(scr);
  hipLaunchKernelGGL((attn_tile_kernel<G, S, W>), dim3((unsigned)a.hkv, (unsigned)maxparts, (unsigned)a.nseq),
                     dim3(64 * W), 0, st, a, part, maxparts, tpp, order && a.nseq <= 64 ? 1 : 0);
  SWL_LAUNCH_CHECK("attn_tile_kernel launch");
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)a.hq, (unsigned)a.nseq), dim3(128), 0, st, a,
                     (const float*)part, maxparts, G, kTileKeys * tpp);
  SWL_LAUNCH_CHECK("attn_combine_kernel launch");
  return SWL_OK;
}

template <int G, int S>
int launch_attn_tile_s(const AttnArgs& a, hipStream_t st, const AttnTileTuning& t) {
  switch (t.waves) {  // 8 waves only with 2 stages (LDS: 160 KiB per CU)
    case 2: return launch_attn_tile_sw<G, S, 2>(a, st, t.tpp, t.order);
    case 4: return launch_attn_tile_sw<G, S, 4>(a, st, t.tpp, t.order);
    case 8: return launch_attn_tile_sw<G, S, (S == 2 ? 8 : 4)>(a, st, t.tpp, t.order);
    default: return launch_attn_tile_sw<G, S, 1>(a, st, t.tpp, t.order);
  }
}

template <int G>
int launch_attn_tile(const AttnArgs& a, hipStream_t st) {
  const AttnTileTuning& t = attn_tile_tuning();
  switch (t.stages) {
    case 3: return launch_attn_tile_s<G, 3>(a, st, t);
    case 4: return launch_attn_tile_s<G, 4>(a, st, t);
    default: return launch_attn_tile_s<G, 2>(a, st, t);
  }
}

// The page-streaming kernel needs whole 16-key tiles inside a page.
bool attn_tile_fits(const AttnArgs& a) {
  return attn_tile_tuning().on && a.L == 1 && a.bs % kTileKeys == 0;
}

int launch_attention(const AttnArgs& a, int G, hipStream_t st) {
  if (a.rope <= 1) {  // 2: q rotated and k / v appended by the QKV round's epilogue
    hipLaunchKernelGGL(rope_append_kernel, dim3((unsigned)(a.nseq * a.L), (unsigned)(a.hq + 2 * a.hkv)), dim3(64),
                       0, st, a);
    SWL_LAUNCH_CHECK("rope_append_kernel launch");
  }
  if (a.L == 1 && attn_tile_fits(a)) {
    switch (G) {
      case 1: return launch_attn_tile<1>(a, st);
      case 2: return launch_attn_tile<2>(a, st);
      case 4: return launch_attn_tile<4>(a, st);
      default: return launch_attn_tile<8>(a, st);
    }
  }
  if (a.L == 1) {
    switch (G) {
      case 1: return launch_attn_decode_u<1>(a, st);
      case 2: return launch_attn_decode_u<2>(a, st);
      case 4: return launch_attn_decode_u<4>(a, st);
      default: return launch_attn_decode_u<8>(a, st);
    }
  }
  const dim3 grid((unsigned)a.hkv, (unsigned)a.L, (unsigned)a.nseq);
  switch (G) {
    case 1: hipLaunchKernelGGL(attention_kernel<1>, grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL(attention_kernel<2>, grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL(attention_kernel<4>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(attention_kernel<8>, grid, dim3(256), 0, st, a); break;
  }
  SWL_LAUNCH_CHECK("attention_kernel launch");
  return SWL_OK;
}

}  // namespace

// ================================================ allocation-free scratch ===
// Device memory of swl_round_ex_noalloc_bf16: the decode projection's K-slice
// partials of one round (64 MiB holds them for every 8B-shaped projection
// round at 64 token rows and for the 128256-wide LM head up to 32 rows).
// Every GPU the library runs on holds its own copy, at its own address, from
// module load until the process ends.  Host
// code never passes the array's name to a kernel (on the host it is only a
// stand-in for the symbol): the device address is looked up once per device
// with hipGetSymbolAddress and used instead.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace swl {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices] = {};
}  // namespace

// Device address of the current device's copy of `scratch` (looked up on the
// first call on that device, with the device current).
int noalloc_scratch(void** out, size_t* bytes) {
  int dev = 0;
  SWL_HIP(hipGetDevice(&dev));
  SWL_CHECK(dev >= 0 && dev < kMaxDevices, SWL_ERR_INVALID, "allocation-free scratch: device index out of range");
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    SWL_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    SWL_CHECK(p != nullptr, SWL_ERR_HIP, "allocation-free scratch: hipGetSymbolAddress returned null");
    g_noalloc_ptr[dev] = p;
  }
  *out = g_noalloc_ptr[dev];
  *bytes = kNoAllocScratchBytes;
  return SWL_OK;
}
}  // namespace swl

// ================================================================ C ABI ===
namespace swl {
thread_local std::string t_err;
void set_error(const std::string& msg) { t_err = msg; }
const std::string& last_error() { return t_err; }
int fail(int code, const std::string& msg) {
  t_err = msg;
  return code;
}
int hip_fail(hipError_t e, const char* where) {
  t_err = std::string("CUDA error: ") + hipGetErrorString(e) + " (" + where + ")";
  return SWL_ERR_HIP;
}

// Round planning shared with the aggregator runtime: builds and launches the
// shrink + base kernels for n_seg segments given host-side lora metadata.
int round_launch(int n_seg, const int64_t* rows, const void* const* seg_in, void* const* seg_out, const void* w,
                 const void* bias, int64_t N, int64_t K, const int32_t* seg_lora, const swl_lora_entry* lora_table,
                 const swl_lora_entry* host_entries, int nblk, const int64_t* blk_cols, hipStream_t st,
                 const swl_round_fusion* fz = nullptr);
int round_launch_ws(int n_seg, const int64_t* rows, const void* const* seg_in, void* const* seg_out, const void* w,
                    const void* bias, int64_t N, int64_t K, const int32_t* seg_lora, const swl_lora_entry* lora_table,
                    const swl_lora_entry* host_entries, int nblk, const int64_t* blk_cols, hipStream_t st,
                    const swl_round_fusion* fz, void* ws, size_t ws_bytes);
int noalloc_scratch(void** out, size_t* bytes);
int plan_lora(int n_seg, const int64_t* rows, int64_t N, const int32_t* seg_lora, const swl_lora_entry* lora_table,
              const swl_lora_entry* host_entries, int nblk, const int64_t* blk_cols, LoraEpi* L, bool* has_lora,
              int* max_r);
}  // namespace swl

extern "C" {

const char* swl_last_error(void) { return swl::last_error().c_str(); }
int swl_abi_version(void) { return SWL_ABI_VERSION; }
int swl_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int swl_gather_bf16(const void* const* slot_in, const int64_t* rows, int n, int64_t d, void* packed, void* stream) {
  SWL_CHECK(slot_in && rows && packed, SWL_ERR_INVALID, "swl_gather_bf16: null argument");
  SegPtrs sp;
  int64_t total = 0;
  int rc = fill_segptrs(sp, slot_in, rows, n, d, &total);
  if (rc) return rc;
  if ((reinterpret_cast<uintptr_t>(packed) & 15) != 0) sp.vec = 0;
  if (total == 0) return SWL_OK;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)total), dim3(256), 0, (hipStream_t)stream, sp, d,
                     reinterpret_cast<bf16*>(packed));
  SWL_LAUNCH_CHECK("gather_rows_kernel launch");
  return SWL_OK;
}

int swl_scatter_add_bf16(const void* y, const void* delta, void* const* slot_out, const int64_t* rows, int n,
                         int64_t d_out, void* stream) {
  SWL_CHECK(y && slot_out && rows, SWL_ERR_INVALID, "swl_scatter_add_bf16: null argument");
  SegPtrs sp;
  int64_t total = 0;
  int rc = fill_segptrs(sp, reinterpret_cast<const void* const*>(slot_out), rows, n, d_out, &total);
  if (rc) return rc;
  if ((reinterpret_cast<uintptr_t>(y) & 15) != 0) sp.vec = 0;
  if (delta && (reinterpret_cast<uintptr_t>(delta) & 15) != 0) sp.vec = 0;
  if (total == 0) return SWL_OK;
  hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)total), dim3(256), 0, (hipStream_t)stream, sp, d_out,
                     reinterpret_cast<const bf16*>(y), reinterpret_cast<const bf16*>(delta));
  SWL_LAUNCH_CHECK("scatter_rows_kernel launch");
  return SWL_OK;
}

int swl_gemm_bf16(const void* x, const void* w, const void* bias, void* y, int64_t m, int64_t n, int64_t k,
                  void* stream) {
  SWL_CHECK(x && w && y, SWL_ERR_INVALID, "swl_gemm_bf16: null argument");
  SWL_CHECK(m >= 0 && n > 0 && k > 0, SWL_ERR_INVALID, "swl_gemm_bf16: bad shape");
  SWL_CHECK(k % 32 == 0, SWL_ERR_INVALID, "swl_gemm_bf16: k must be a multiple of 32");
  SWL_CHECK((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0,
            SWL_ERR_INVALID, "swl_gemm_bf16: x and w must be 16-byte aligned");
  if (m == 0) return SWL_OK;
  hipStream_t st = (hipStream_t)stream;
  if (m <= kSkinnyMaxTok) {
    const bf16* xr[kSkinnyMaxTok];
    bf16* yr[kSkinnyMaxTok];
    for (int i = 0; i < m; ++i) {
      xr[i] = reinterpret_cast<const bf16*>(x) + (int64_t)i * k;
      yr[i] = reinterpret_cast<bf16*>(y) + (int64_t)i * n;
    }
    return launch_skinny(reinterpret_cast<const bf16*>(w), reinterpret_cast<const bf16*>(bias), n, k, (int)m, xr, yr,
                         nullptr, nullptr, nullptr, nullptr, 1, nullptr, st);
  }
  SWL_CHECK(k % TK == 0, SWL_ERR_INVALID, "swl_gemm_bf16: k must be a multiple of 64 for m > 64");
  TiledArgs a{};
  a.x = reinterpret_cast<const bf16*>(x);
  a.w = reinterpret_cast<const bf16*>(w);
  a.bias = reinterpret_cast<const bf16*>(bias);
  a.M = m;
  a.N = n;
  a.K = k;
  a.y = reinterpret_cast<bf16*>(y);
  a.ldy = n;
  a.has_lora = 0;
  return launch_prefill_gemm(a, st);
}

int swl_round_bf16(int n_seg, const int64_t* rows, const void* const* seg_in, void* const* seg_out, const void* w,
                   const void* bias, int64_t n, int64_t k, const int32_t* seg_lora, const swl_lora_entry* lora_table,
                   const swl_lora_entry* lora_table_host, int nblk, const int64_t* blk_cols, void* stream) {
  if (seg_lora) {
    SWL_CHECK(lora_table != nullptr && lora_table_host != nullptr, SWL_ERR_INVALID,
              "swl_round_bf16: seg_lora needs lora_table and lora_table_host");
  }
  return swl::round_launch(n_seg, rows, seg_in, seg_out, w, bias, n, k, seg_lora, lora_table, lora_table_host, nblk,
                           blk_cols, (hipStream_t)stream);
}

int swl_round_ex_bf16(int n_seg, const int64_t* rows, const void* const* seg_in, void* const* seg_out, const void* w,
                      const void* bias, int64_t n, int64_t k, const int32_t* seg_lora,
                      const swl_lora_entry* lora_table, const swl_lora_entry* lora_table_host, int nblk,
                      const int64_t* blk_cols, const swl_round_fusion* fusion, void* stream) {
  if (seg_lora) {
    SWL_CHECK(lora_table != nullptr && lora_table_host != nullptr, SWL_ERR_INVALID,
              "swl_round_ex_bf16: seg_lora needs lora_table and lora_table_host");
  }
  return swl::round_launch(n_seg, rows, seg_in, seg_out, w, bias, n, k, seg_lora, lora_table, lora_table_host, nblk,
                           blk_cols, (hipStream_t)stream, fusion);
}

int swl_round_ex_noalloc_bf16(int n_seg, const int64_t* rows, const void* const* seg_in, void* const* seg_out,
                              const void* w, const void* bias, int64_t n, int64_t k, const int32_t* seg_lora,
                              const swl_lora_entry* lora_table, const swl_lora_entry* lora_table_host, int nblk,
                              const int64_t* blk_cols, const swl_round_fusion* fusion, void* stream) {
  if (seg_lora) {
    SWL_CHECK(lora_table != nullptr && lora_table_host != nullptr, SWL_ERR_INVALID,
              "swl_round_ex_noalloc_bf16: seg_lora needs lora_table and lora_table_host");
  }
  void* ws = nullptr;
  size_t ws_bytes = 0;
  int rc = swl::noalloc_scratch(&ws, &ws_bytes);
  if (rc) return rc;
  return swl::round_launch_ws(n_seg, rows, seg_in, seg_out, w, bias, n, k, seg_lora, lora_table, lora_table_host,
                              nblk, blk_cols, (hipStream_t)stream, fusion, ws, ws_bytes);
}

int swl_lora_segmented_bf16(const void* x, int64_t k, int n_seg, const int64_t* seg_rows, const int32_t* seg_lora,
                            const swl_lora_entry* lora_table, const swl_lora_entry* lora_table_host, int nblk,
                            const int64_t* blk_cols, void* y, int64_t n, int mode, void* stream) {
  SWL_CHECK(x && seg_rows && seg_lora && lora_table && lora_table_host && y, SWL_ERR_INVALID,
            "swl_lora_segmented_bf16: null argument");
  SWL_CHECK(n_seg >= 1 && n_seg <= kMaxSeg, SWL_ERR_INVALID, "swl_lora_segmented_bf16: segment count must be in [1, 128]");
  SWL_CHECK(k > 0 && k % 32 == 0 && n > 0, SWL_ERR_INVALID, "swl_lora_segmented_bf16: k must be a positive multiple of 32");
  SWL_CHECK(mode == 0 || mode == 1, SWL_ERR_INVALID, "swl_lora_segmented_bf16: mode must be 0 or 1");
  SWL_CHECK((reinterpret_cast<uintptr_t>(x) & 15) == 0, SWL_ERR_INVALID, "swl_lora_segmented_bf16: x must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  ExpandArgs e{};
  e.y = reinterpret_cast<bf16*>(y);
  e.N = n;
  e.mode = mode;
  e.n_seg = n_seg;
  e.off[0] = 0;
  for (int i = 0; i < n_seg; ++i) {
    SWL_CHECK(seg_rows[i] >= 0, SWL_ERR_INVALID, "swl_lora_segmented_bf16: negative row count");
    e.off[i + 1] = e.off[i] + seg_rows[i];
    e.seg_lora[i] = (seg_lora[i] >= 0 && seg_rows[i] > 0) ? seg_lora[i] : -1;
  }
  const int64_t T = e.off[n_seg];
  if (T == 0) return SWL_OK;
  SWL_CHECK(T <= 65535, SWL_ERR_INVALID, "swl_lora_segmented_bf16: at most 65535 rows");
  bool has_lora = false;
  int max_r = 0;
  int rc = swl::plan_lora(n_seg, seg_rows, n, seg_lora, lora_table, lora_table_host, nblk, blk_cols, &e.L, &has_lora,
                          &max_r);
  if (rc) return rc;
  if (has_lora) {
    const int u_ld = ((max_r * nblk + 15) / 16) * 16;
    SWL_CHECK(u_ld <= kMaxURow, SWL_ERR_INVALID, "swl_lora_segmented_bf16: LoRA rank x blocks exceeds 256");
    int64_t items = 0;
    for (int i = 0; i < n_seg; ++i)
      if (e.seg_lora[i] >= 0) items += (seg_rows[i] + 63) / 64 * ((lora_table_host[e.seg_lora[i]].rank * nblk + 63) / 64);
    int u_ks = 1;
    while (u_ks < 16 && items * u_ks < 1024 && (k / 32) / (2 * u_ks) >= 8) u_ks *= 2;
    void* scr = nullptr;
    rc = scratch_get(sizeof(float) * (size_t)u_ks * (size_t)T * (size_t)u_ld, st, &scr);
    if (rc) return rc;
    float* u = reinterpret_cast<float*>(scr);
    const bf16* seg_x[kMaxSeg];
    for (int i = 0; i < n_seg; ++i) seg_x[i] = reinterpret_cast<const bf16*>(x) + e.off[i] * k;
    rc = launch_shrink_gemm(seg_x, k, n_seg, e.off, seg_rows, e.seg_lora, lora_table_host, nblk, u, u_ld, T * u_ld,
                            u_ks, st);
    if (rc) return rc;
    e.L.u = u;
    e.L.usplit = 1;  // folded into split 0
    e.L.u_ld = u_ld;
    e.L.u_split_stride = T * u_ld;
  } else if (mode == 1) {
    return SWL_OK;  // nothing to add
  }
  const dim3 grid((unsigned)((n + 1023) / 1024), (unsigned)T);
  hipLaunchKernelGGL(lora_expand_kernel, grid, dim3(256), 0, st, e);
  SWL_LAUNCH_CHECK("lora_expand_kernel launch");
  return SWL_OK;
}

int swl_pack_weight_bf16(const void* w, int64_t n, int64_t k, void* out, void* stream) {
  SWL_CHECK(w && out, SWL_ERR_INVALID, "swl_pack_weight_bf16: null argument");
  SWL_CHECK(n > 0 && k > 0 && k % 32 == 0, SWL_ERR_INVALID, "swl_pack_weight_bf16: k must be a positive multiple of 32");
  SWL_CHECK((reinterpret_cast<uintptr_t>(w) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0,
            SWL_ERR_INVALID, "swl_pack_weight_bf16: w and out must be 16-byte aligned");
  const int64_t nchunks = (n + 15) / 16 * 16 * k / 8;
  SWL_CHECK((nchunks + 255) / 256 < ((int64_t)1 << 31), SWL_ERR_INVALID, "swl_pack_weight_bf16: weight too large");
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)((nchunks + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const bf16*>(w), n, k, reinterpret_cast<u32x4*>(out), nchunks);
  SWL_LAUNCH_CHECK("pack_weight_kernel launch");
  return SWL_OK;
}

int swl_matmul_bf16(const void* x, int64_t ldx, const void* b, int64_t ldb, int trans_b, void* y, int64_t ldy,
                    int64_t m, int64_t n, int64_t k, float alpha, void* stream) {
  SWL_CHECK(x && b && y, SWL_ERR_INVALID, "swl_matmul_bf16: null argument");
  SWL_CHECK(m >= 0 && n > 0 && k > 0, SWL_ERR_INVALID, "swl_matmul_bf16: bad shape");
  SWL_CHECK(m <= 65535, SWL_ERR_INVALID, "swl_matmul_bf16: m too large");
  if (m == 0) return SWL_OK;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(b)) & 15) == 0 &&
                      ldx % 8 == 0 && ldb % 8 == 0 && k % 8 == 0;
  if (vec_ok && m <= kSkinnyMaxTok && n <= 256 && k >= 512 && k <= kShrinkMaxK && (trans_b || n % 8 == 0)) {
    int P = 0;
    size_t lds = (size_t)k * sizeof(bf16);
    if (!trans_b) {
      P = 1;
      while (P * 2 * (n / 8) <= 1024) P *= 2;
      lds += (size_t)P * n * sizeof(float);
    }
    if (trans_b)
      hipLaunchKernelGGL(matmul_shrink_kernel<true>, dim3((unsigned)m), dim3(1024), lds, (hipStream_t)stream,
                         reinterpret_cast<const bf16*>(x), ldx, reinterpret_cast<const bf16*>(b), ldb,
                         reinterpret_cast<bf16*>(y), ldy, (int)n, k, alpha, P);
    else
      hipLaunchKernelGGL(matmul_shrink_kernel<false>, dim3((unsigned)m), dim3(1024), lds, (hipStream_t)stream,
                         reinterpret_cast<const bf16*>(x), ldx, reinterpret_cast<const bf16*>(b), ldb,
                         reinterpret_cast<bf16*>(y), ldy, (int)n, k, alpha, P);
    SWL_LAUNCH_CHECK("matmul_shrink_kernel launch");
    return SWL_OK;
  }
  hipLaunchKernelGGL(matmul_generic_kernel, dim3((unsigned)((n + 63) / 64), (unsigned)m), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const bf16*>(x), ldx, reinterpret_cast<const bf16*>(b),
                     ldb, trans_b, reinterpret_cast<bf16*>(y), ldy, n, k, alpha);
  SWL_LAUNCH_CHECK("matmul_generic_kernel launch");
  return SWL_OK;
}

int swl_lora_rows_bf16(const void* x, int64_t ldx, int64_t m, int64_t k, const void* a, int64_t a_sk, int64_t a_sj,
                       int64_t nr, int nblk, int64_t rank, const void* const* b, const int64_t* b_srr,
                       const int64_t* b_sc, const int64_t* blk_cols, float alpha, void* y, int64_t ldy, void* stream) {
  SWL_CHECK(x && a && b && b_srr && b_sc && blk_cols && y, SWL_ERR_INVALID, "swl_lora_rows_bf16: null argument");
  SWL_CHECK(m >= 0 && m <= kLoraRowsMaxRows, SWL_ERR_INVALID, "swl_lora_rows_bf16: at most 4 rows");
  SWL_CHECK(k > 0 && k % 8 == 0 && ldx % 8 == 0 && ldx >= k, SWL_ERR_INVALID,
            "swl_lora_rows_bf16: k must be a positive multiple of 8 (rows of 16-byte multiples)");
  SWL_CHECK((reinterpret_cast<uintptr_t>(x) & 15) == 0, SWL_ERR_INVALID, "swl_lora_rows_bf16: x must be 16-byte aligned");
  SWL_CHECK(nr >= 1 && nr <= kLoraRowsMaxNr, SWL_ERR_INVALID, "swl_lora_rows_bf16: 1..64 shrink columns");
  SWL_CHECK(nblk >= 1 && nblk <= kLoraRowsMaxBlk && rank >= 1 && nblk * rank <= nr, SWL_ERR_INVALID,
            "swl_lora_rows_bf16: 1..4 blocks of rank columns within the shrink columns");
  SWL_CHECK(a_sk > 0 && a_sj > 0, SWL_ERR_INVALID, "swl_lora_rows_bf16: A strides must be positive");
  if (m == 0) return SWL_OK;
  LoraRowsArgs r{};
  r.x = reinterpret_cast<const bf16*>(x);
  r.ldx = ldx;
  r.K = k;
  r.m = (int)m;
  r.nr = (int)nr;
  r.nblk = nblk;
  r.rank = (int)rank;
  r.a = reinterpret_cast<const bf16*>(a);
  r.a_sk = a_sk;
  r.a_sj = a_sj;
  const bool a_al = (reinterpret_cast<uintptr_t>(a) & 15) == 0;
  if (a_sk == 1 && a_al && a_sj % 8 == 0)
    r.a_mode = 0;
  else if (a_sj == 1 && a_al && a_sk % 8 == 0 && nr % 8 == 0)
    r.a_mode = 1;
  else
    r.a_mode = 2;
  r.off[0] = 0;
  for (int i = 0; i < nblk; ++i) {
    SWL_CHECK(b[i] && blk_cols[i] > 0, SWL_ERR_INVALID, "swl_lora_rows_bf16: empty block");
    r.b[i] = reinterpret_cast<const bf16*>(b[i]);
    r.srr[i] = b_srr[i];
    r.sc[i] = b_sc[i];
    r.off[i + 1] = r.off[i] + blk_cols[i];
  }
  SWL_CHECK(ldy >= r.off[nblk], SWL_ERR_INVALID, "swl_lora_rows_bf16: ldy below the output columns");
  r.alpha = alpha;
  r.y = reinterpret_cast<bf16*>(y);
  r.ldy = ldy;
  const unsigned grid = (unsigned)std::min<int64_t>(32, std::max<int64_t>(1, (r.off[nblk] + 1023) / 1024));
  hipStream_t st = (hipStream_t)stream;
  if (nr <= 16)
    hipLaunchKernelGGL(lora_rows_kernel<16>, dim3(grid), dim3(256), 0, st, r);
  else if (nr <= 32)
    hipLaunchKernelGGL(lora_rows_kernel<32>, dim3(grid), dim3(256), 0, st, r);
  else
    hipLaunchKernelGGL(lora_rows_kernel<64>, dim3(grid), dim3(256), 0, st, r);
  SWL_LAUNCH_CHECK("lora_rows_kernel launch");
  return SWL_OK;
}

int swl_paged_attention_bf16(void* q, void* k, const void* v, int64_t q_stride, int64_t k_stride, int64_t v_stride,
                             int nseq, int q_len, int hq, int hkv, int d, void* k_cache, void* v_cache,
                             int64_t num_blocks, int block_size,
                             const int32_t* block_table, int64_t max_blocks, const int32_t* cache_seqlens,
                             const int64_t* positions, const void* cos_sin, int64_t max_pos, int rope,
                             float softmax_scale, void* out, void* stream) {
  SWL_CHECK(q && k && v && k_cache && v_cache && block_table && cache_seqlens && out, SWL_ERR_INVALID,
            "swl_paged_attention_bf16: null argument");
  SWL_CHECK(d == 128, SWL_ERR_INVALID, "swl_paged_attention_bf16: head_dim must be 128");
  SWL_CHECK(hq > 0 && hkv > 0 && hq % hkv == 0, SWL_ERR_INVALID, "swl_paged_attention_bf16: bad head counts");
  const int G = hq / hkv;
  SWL_CHECK(G == 1 || G == 2 || G == 4 || G == 8, SWL_ERR_INVALID,
            "swl_paged_attention_bf16: hq / hkv must be 1, 2, 4 or 8");
  SWL_CHECK(nseq >= 0 && q_len >= 1 && q_len <= 1024, SWL_ERR_INVALID, "swl_paged_attention_bf16: bad q_len");
  SWL_CHECK(block_size > 0 && num_blocks > 0 && max_blocks > 0, SWL_ERR_INVALID,
            "swl_paged_attention_bf16: bad page geometry");
  SWL_CHECK(rope == 0 || rope == 1, SWL_ERR_INVALID, "swl_paged_attention_bf16: rope must be 0 or 1");
  SWL_CHECK(!rope || (cos_sin && positions && max_pos > 0), SWL_ERR_INVALID,
            "swl_paged_attention_bf16: rope needs positions and cos_sin");
  SWL_CHECK(q_stride >= hq * d && k_stride >= hkv * d && v_stride >= hkv * d, SWL_ERR_INVALID,
            "swl_paged_attention_bf16: token strides smaller than a token row");
  SWL_CHECK(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15) ==
                    0 &&
                ((q_stride | k_stride | v_stride) & 7) == 0,
            SWL_ERR_INVALID, "swl_paged_attention_bf16: q/k/v rows must be 16-byte aligned");
  if (nseq == 0) return SWL_OK;
  AttnArgs a{};
  a.qs = q_stride;
  a.ks = k_stride;
  a.vs = v_stride;
  a.q = reinterpret_cast<bf16*>(q);
  a.k = reinterpret_cast<bf16*>(k);
  a.v = reinterpret_cast<const bf16*>(v);
  a.kc = reinterpret_cast<bf16*>(k_cache);
  a.vc = reinterpret_cast<bf16*>(v_cache);
  a.bt = block_table;
  a.seqlens = cache_seqlens;
  a.pos = positions;
  a.cs = reinterpret_cast<const bf16*>(cos_sin);
  a.out = reinterpret_cast<bf16*>(out);
  a.num_blocks = num_blocks;
  a.max_blocks = max_blocks;
  a.max_pos = max_pos;
  a.nseq = nseq;
  a.L = q_len;
  a.hq = hq;
  a.hkv = hkv;
  a.bs = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.rope = rope;
  a.scale = softmax_scale;
  return launch_attention(a, G, (hipStream_t)stream);
}

int swl_timer_arm(int capacity) {
  SWL_CHECK(capacity >= 0 && capacity <= (1 << 20), SWL_ERR_INVALID, "swl_timer_arm: bad capacity");
  if ((int)g_timer.ev.size() < 4 * capacity) {
    const size_t have = g_timer.ev.size();
    g_timer.ev.resize(4 * (size_t)capacity, nullptr);
    // timestamp-only markers: no system-scope cache writeback / invalidate
    // around the timed kernels
    for (size_t i = have; i < g_timer.ev.size(); ++i)
      SWL_HIP(hipEventCreateWithFlags(&g_timer.ev[i], hipEventReleaseToDevice));
    g_timer.N.resize(capacity);
    g_timer.K.resize(capacity);
    g_timer.bytes.resize(capacity);
    g_timer.ntok.resize(capacity);
  }
  g_timer.cap = capacity;
  g_timer.n = 0;
  g_timer.armed = capacity > 0;
  return SWL_OK;
}

int swl_timer_collect(int max_records, float* base_ms, float* epilogue_ms, int64_t* n, int64_t* k, int32_t* ntok,
                      int64_t* bytes, int* count) {
  SWL_CHECK(count && max_records >= 0, SWL_ERR_INVALID, "swl_timer_collect: null argument");
  g_timer.armed = false;
  const int m = std::min(g_timer.n, max_records);
  for (int i = 0; i < m; ++i) {
    SWL_HIP(hipEventSynchronize(g_timer.ev[4 * i + 1]));
    SWL_HIP(hipEventSynchronize(g_timer.ev[4 * i + 3]));
    float a = 0.f, b = 0.f;
    SWL_HIP(hipEventElapsedTime(&a, g_timer.ev[4 * i], g_timer.ev[4 * i + 1]));
    SWL_HIP(hipEventElapsedTime(&b, g_timer.ev[4 * i + 2], g_timer.ev[4 * i + 3]));
    if (base_ms) base_ms[i] = a;
    if (epilogue_ms) epilogue_ms[i] = b;
    if (n) n[i] = g_timer.N[i];
    if (k) k[i] = g_timer.K[i];
    if (ntok) ntok[i] = g_timer.ntok[i];
    if (bytes) bytes[i] = g_timer.bytes[i];
  }
  *count = m;
  g_timer.n = 0;
  return SWL_OK;
}

int swl_zero_blocks_bf16(void* const* caches, int ncache, const int64_t* block_ids, int64_t nblocks,
                         int64_t block_elems, void* stream) {
  SWL_CHECK(caches && block_ids, SWL_ERR_INVALID, "swl_zero_blocks_bf16: null argument");
  SWL_CHECK(block_elems % 8 == 0, SWL_ERR_INVALID, "swl_zero_blocks_bf16: block size must be a multiple of 8");
  if (nblocks == 0) return SWL_OK;
  for (int c = 0; c < ncache; ++c) {
    hipLaunchKernelGGL(zero_blocks_kernel, dim3((unsigned)nblocks), dim3(256), 0, (hipStream_t)stream,
                       reinterpret_cast<bf16*>(caches[c]), block_ids, nblocks, block_elems);
    SWL_LAUNCH_CHECK("zero_blocks_kernel launch");
  }
  return SWL_OK;
}

}  // extern "C"

// ============================================== GPU-ordered round flags ===
namespace {
struct SeqWaitArgs {
  int32_t n;
  uint32_t limit_ticks;  // s_memrealtime runs at 100 MHz
  uint32_t* timed_out;
  const uint64_t* flag[SWL_MAX_SLOTS];
  uint64_t want[SWL_MAX_SLOTS];
  int32_t tag[SWL_MAX_SLOTS];
};

// One lane per flag; every lane exits: when its flag reaches the wanted value
// or when the time limit has passed (then it reports its tag).
__global__ __launch_bounds__(SWL_MAX_SLOTS) void seq_wait_kernel(SeqWaitArgs a) {
  const int i = threadIdx.x;
  if (i >= a.n) return;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  while (__hip_atomic_load(a.flag[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) < a.want[i]) {
    if (__builtin_amdgcn_s_memrealtime() - t0 > a.limit_ticks) {
      __hip_atomic_store(a.timed_out + a.tag[i], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      break;
    }
    __builtin_amdgcn_s_sleep(32);
  }
}

struct SeqWriteArgs {
  int32_t n;
  uint64_t* flag[SWL_MAX_SLOTS];
  uint64_t value[SWL_MAX_SLOTS];
};

// One lane per flag: the value is stored with system-scope release order
// (vector stores; the kernel starts after the stream's earlier kernels have
// completed and released their writes).
__global__ __launch_bounds__(SWL_MAX_SLOTS) void seq_write_kernel(SeqWriteArgs a) {
  const int i = threadIdx.x;
  if (i < a.n) __hip_atomic_store(a.flag[i], a.value[i], __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// One workgroup copies n16 16-byte pieces and `tail` more bytes, then every
// thread releases its stores at agent scope (written back from the XCD's L2),
// and after the barrier one lane stores the flag with system-scope release.
__global__ __launch_bounds__(1024) void copy_signal_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                           int64_t n16, int tail, uint64_t* flag, uint64_t value) {
  for (int64_t i = threadIdx.x; i < n16; i += 1024) dst[i] = src[i];
  if ((int)threadIdx.x < tail)
    reinterpret_cast<unsigned char*>(dst + n16)[threadIdx.x] = reinterpret_cast<const unsigned char*>(src + n16)[threadIdx.x];
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(flag, value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A worker read's GPU-ordered slot words, handled inside its own launch.
struct SeqSyncDev {
  const uint64_t* wait_flag;  // or null: no wait
  uint64_t want;
  uint32_t* timed_out;
  int32_t tag;
  uint32_t limit_ticks;       // s_memrealtime runs at 100 MHz
  uint64_t* signal_flag;      // or null: no signal (single-workgroup launches only)
  uint64_t value;
};

// Every workgroup: lane 0 polls the flag (system-scope loads and a sleep,
// bounded like seq_wait_kernel; a wait that runs out reports its tag and the
// read still runs), then after the barrier every thread takes an agent-scope
// fence (the XCD's caches drop lines older than the producer's writes).
__device__ __forceinline__ void seq_sync_wait(const SeqSyncDev& s) {
  if (!s.wait_flag) return;
  if (threadIdx.x == 0) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(s.wait_flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) < s.want) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > s.limit_ticks) {
        __hip_atomic_store(s.timed_out + s.tag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        break;
      }
      __builtin_amdgcn_s_sleep(32);
    }
  }
  __syncthreads();
  __threadfence();
}

// The launch's only workgroup, after all of its stores: every thread
// releases its stores at agent scope (written back from the XCD's L2), and
// after the barrier one lane stores the flag with system-scope release.
__device__ __forceinline__ void seq_sync_signal(const SeqSyncDev& s) {
  if (!s.signal_flag) return;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(s.signal_flag, s.value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

struct CombineArgs {
  bf16* dst;
  const bf16* src;
  const bf16* delta;  // or null
  const bf16* res;    // or null
  int64_t n;
  int32_t vec;        // every pointer 16-byte aligned
  SeqSyncDev sync;    // wait only
};

// A worker's read of its round output: out (+ its LoRA delta) (+ the
// residual), each add rounded to bf16 as torch's bf16 adds are; 8 elements
// a thread.
__global__ __launch_bounds__(256) void combine_rows_kernel(CombineArgs a) {
  seq_sync_wait(a.sync);
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i0 >= a.n) return;
  auto one = [&](float s, float d, float r) {
    float v = s;
    if (a.delta) v = bf2f(f2bf(v + d));
    if (a.res) v = r + v;
    return f2bf(v);
  };
  if (a.vec && i0 + 8 <= a.n) {
    float s[8], d[8], r[8];
    unpack8(ld16(a.src + i0), s);
    if (a.delta) unpack8(ld16(a.delta + i0), d);
    if (a.res) unpack8(ld16(a.res + i0), r);
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = one(s[e], a.delta ? d[e] : 0.f, a.res ? r[e] : 0.f);
    *reinterpret_cast<u32x4*>(a.dst + i0) = __builtin_bit_cast(u32x4, o);
    return;
  }
  for (int64_t i = i0; i < a.n && i < i0 + 8; ++i)
    a.dst[i] = one(bf2f(a.src[i]), a.delta ? bf2f(a.delta[i]) : 0.f, a.res ? bf2f(a.res[i]) : 0.f);
}

// The read of an O or Down round's output followed by the next norm, a
// workgroup of 256 threads per token row (rows blockIdx.x, + gridDim.x, ...):
// h = bf16(res + bf16(out + delta))
// is written to dst_h, then LlamaRMSNorm of h to dst_n with the same
// per-thread sums and reduction as rmsnorm_rows_kernel, so both match the
// separate read and norm bit for bit.  d a multiple of 8, every pointer
// 16-byte aligned (the caller checks).
struct CombineNormArgs {
  bf16* dst_h;
  bf16* dst_n;
  bf16* dst_n2;       // a second copy of the normalised rows, or null
  const bf16* src;
  const bf16* delta;  // or null
  const bf16* res;    // or null
  const bf16* w;
  int64_t d;
  int64_t rows;
  float eps;
  SeqSyncDev sync;
};

__global__ __launch_bounds__(256) void combine_norm_rows_kernel(CombineNormArgs a) {
  __shared__ float sh[4];
  seq_sync_wait(a.sync);
  const int64_t nv = a.d >> 3;
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
  const int64_t off = row * a.d;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) {
    float s[8], dl[8], r[8];
    unpack8(ld16(a.src + off + 8 * i), s);
    if (a.delta) unpack8(ld16(a.delta + off + 8 * i), dl);
    if (a.res) unpack8(ld16(a.res + off + 8 * i), r);
    bf16x8 o;
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = s[j];
      if (a.delta) v = bf2f(f2bf(v + dl[j]));
      if (a.res) v = r[j] + v;
      o[j] = f2bf(v);
      x[j] = bf2f(o[j]);
    }
    *reinterpret_cast<u32x4*>(a.dst_h + off + 8 * i) = __builtin_bit_cast(u32x4, o);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
  }
  ss = block_reduce<float>(ss, [](float x, float y) { return x + y; }, sh);
  const float rs = rsqrtf(ss / (float)a.d + a.eps);
  for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) {
    float x[8], g[8];
    unpack8(ld16(a.dst_h + off + 8 * i), x);
    unpack8(ld16(a.w + 8 * i), g);
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = f2bf(bf2f(f2bf(x[j] * rs)) * g[j]);
    *reinterpret_cast<u32x4*>(a.dst_n + off + 8 * i) = __builtin_bit_cast(u32x4, o);
    if (a.dst_n2) *reinterpret_cast<u32x4*>(a.dst_n2 + off + 8 * i) = __builtin_bit_cast(u32x4, o);
  }
  }
  seq_sync_signal(a.sync);
}

// The read of a Gate+Up round's output followed by SiLU*up: g = bf16(gate +
// dgate), u = bf16(up + dup), act = bf16(bf16(silu(g)) * u) as
// silu_mul_rows_kernel computes it; rows of 2 inter (gate | up) in, inter
// out.  inter a multiple of 8, pointers 16-byte aligned.  Rows blockIdx.y,
// + gridDim.y, ...; 8-element groups of a row by a grid stride over x.
struct CombineSiluArgs {
  bf16* dst;
  bf16* dst2;         // a second copy, or null
  const bf16* src;
  const bf16* delta;  // [rows][2 inter] or null
  int64_t inter;
  int64_t rows;
  SeqSyncDev sync;
};

__global__ __launch_bounds__(1024) void combine_silu_rows_kernel(CombineSiluArgs a) {
  seq_sync_wait(a.sync);
  const int64_t nv = a.inter >> 3;
  for (int64_t t = blockIdx.y; t < a.rows; t += gridDim.y)
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += (int64_t)gridDim.x * blockDim.x) {
  const int64_t ri = t * 2 * a.inter + 8 * i;
  float g[8], u[8];
  unpack8(ld16(a.src + ri), g);
  unpack8(ld16(a.src + ri + a.inter), u);
  if (a.delta) {
    float dg[8], du[8];
    unpack8(ld16(a.delta + ri), dg);
    unpack8(ld16(a.delta + ri + a.inter), du);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      g[j] = bf2f(f2bf(g[j] + dg[j]));
      u[j] = bf2f(f2bf(u[j] + du[j]));
    }
  }
  bf16x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float sg = bf2f(f2bf(g[j] / (1.0f + __expf(-g[j]))));
    o[j] = f2bf(sg * u[j]);
  }
  *reinterpret_cast<u32x4*>(a.dst + t * a.inter + 8 * i) = __builtin_bit_cast(u32x4, o);
  if (a.dst2) *reinterpret_cast<u32x4*>(a.dst2 + t * a.inter + 8 * i) = __builtin_bit_cast(u32x4, o);
  }
  seq_sync_signal(a.sync);
}

struct WaitCopyArgs {
  const uint64_t* flag;
  uint64_t want;
  uint32_t* timed_out;
  int32_t tag;
  uint32_t limit_ticks;  // s_memrealtime runs at 100 MHz
  u32x4* dst;
  const u32x4* src;
  int64_t n16;
  int32_t tail;
};

// Lane 0 polls the flag (system-scope loads and a sleep, bounded like
// seq_wait_kernel); after the barrier every thread takes an agent-scope
// fence (the XCD's caches drop lines older than the producer's writes), then
// the workgroup copies.  A wait that ran out of time reports its tag and the
// copy still runs (the caller learns of it from timed_out).
__global__ __launch_bounds__(1024) void wait_copy_kernel(WaitCopyArgs a) {
  if (threadIdx.x == 0) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(a.flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) < a.want) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > a.limit_ticks) {
        __hip_atomic_store(a.timed_out + a.tag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        break;
      }
      __builtin_amdgcn_s_sleep(32);
    }
  }
  __syncthreads();
  __threadfence();
  for (int64_t i = threadIdx.x; i < a.n16; i += 1024) a.dst[i] = a.src[i];
  if ((int)threadIdx.x < a.tail)
    reinterpret_cast<unsigned char*>(a.dst + a.n16)[threadIdx.x] =
        reinterpret_cast<const unsigned char*>(a.src + a.n16)[threadIdx.x];
}
}  // namespace

namespace swl {
int seq_write_launch(int n, uint64_t* const* flag, const uint64_t* value, hipStream_t stream) {
  SWL_CHECK(n >= 0 && n <= SWL_MAX_SLOTS, SWL_ERR_INVALID, "seq_write: at most 128 flags");
  if (n == 0) return SWL_OK;
  SeqWriteArgs a{};
  a.n = n;
  for (int i = 0; i < n; ++i) {
    SWL_CHECK(flag[i] != nullptr, SWL_ERR_INVALID, "seq_write: null flag");
    a.flag[i] = flag[i];
    a.value[i] = value[i];
  }
  hipLaunchKernelGGL(seq_write_kernel, dim3(1), dim3(SWL_MAX_SLOTS), 0, stream, a);
  SWL_LAUNCH_CHECK("seq_write_kernel launch");
  return SWL_OK;
}

int copy_signal_launch(void* dst, const void* src, size_t bytes, uint64_t* flag, uint64_t value, hipStream_t stream) {
  SWL_CHECK(flag != nullptr, SWL_ERR_INVALID, "copy_signal: null flag");
  const bool fused = bytes <= kCopySignalMax && ((uintptr_t)dst % 16) == 0 && ((uintptr_t)src % 16) == 0;
  if (!fused) {
    if (bytes) SWL_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream));
    return seq_write_launch(1, &flag, &value, stream);
  }
  hipLaunchKernelGGL(copy_signal_kernel, dim3(1), dim3(1024), 0, stream, reinterpret_cast<u32x4*>(dst),
                     reinterpret_cast<const u32x4*>(src), (int64_t)(bytes / 16), (int)(bytes % 16), flag, value);
  SWL_LAUNCH_CHECK("copy_signal_kernel launch");
  return SWL_OK;
}

namespace {
// Host SeqSync -> kernel form; a signal only where the launch has one
// workgroup (single_wg).
int seq_sync_dev(const SeqSync* s, bool single_wg, const char* fn, SeqSyncDev* d) {
  *d = SeqSyncDev{};
  if (!s) return SWL_OK;
  if (s->wait_flag) {
    SWL_CHECK(s->timed_out != nullptr && s->tag >= 0 && s->tag < SWL_MAX_SLOTS, SWL_ERR_INVALID,
              std::string(fn) + ": bad wait time-out word");
    d->wait_flag = s->wait_flag;
    d->want = s->want;
    d->timed_out = s->timed_out;
    d->tag = s->tag;
    d->limit_ticks = (uint32_t)std::min<uint64_t>((uint64_t)s->limit_us * 100, 0xFFFFFFFFull);
  }
  if (s->signal_flag) {
    SWL_CHECK(single_wg, SWL_ERR_INVALID, std::string(fn) + ": a fused signal needs at most " +
                                              std::to_string(kFusedSignalRows) + " rows");
    d->signal_flag = s->signal_flag;
    d->value = s->value;
  }
  return SWL_OK;
}
}  // namespace

int combine_rows_launch(void* dst, const void* src, int64_t n, const void* delta, const void* res,
                        hipStream_t stream, const SeqSync* sync) {
  SWL_CHECK(dst && src && n >= 0, SWL_ERR_INVALID, "combine_rows: bad arguments");
  SWL_CHECK(!sync || !sync->signal_flag, SWL_ERR_INVALID, "combine_rows: no fused signal");
  if (n == 0) {  // nothing to read: the wait alone
    if (!sync || !sync->wait_flag) return SWL_OK;
    const uint64_t* f = sync->wait_flag;
    return seq_wait_launch(1, &f, &sync->want, &sync->tag, sync->timed_out, sync->limit_us, stream);
  }
  CombineArgs a{};
  a.dst = reinterpret_cast<bf16*>(dst);
  a.src = reinterpret_cast<const bf16*>(src);
  a.delta = reinterpret_cast<const bf16*>(delta);
  a.res = reinterpret_cast<const bf16*>(res);
  a.n = n;
  auto al = [](const void* p) { return p == nullptr || ((uintptr_t)p % 16) == 0; };
  a.vec = (al(dst) && al(src) && al(delta) && al(res)) ? 1 : 0;
  int rc = seq_sync_dev(sync, false, "combine_rows", &a.sync);
  if (rc) return rc;
  const int64_t threads = (n + 7) / 8;
  hipLaunchKernelGGL(combine_rows_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, a);
  SWL_LAUNCH_CHECK("combine_rows_kernel launch");
  return SWL_OK;
}

int combine_norm_rows_launch(void* dst_h, void* dst_n, void* dst_n2, const void* src, int64_t rows, int64_t d,
                             const void* delta, const void* res, const void* w, float eps, hipStream_t stream,
                             const SeqSync* sync) {
  auto al = [](const void* p) { return p == nullptr || ((uintptr_t)p % 16) == 0; };
  SWL_CHECK(dst_h && dst_n && src && w && rows >= 0 && d > 0 && d % 8 == 0, SWL_ERR_INVALID,
            "combine_norm_rows: bad arguments (d must be a multiple of 8)");
  SWL_CHECK(al(dst_h) && al(dst_n) && al(dst_n2) && al(src) && al(delta) && al(res) && al(w), SWL_ERR_INVALID,
            "combine_norm_rows: pointers must be 16-byte aligned");
  if (rows == 0 && !sync) return SWL_OK;
  SWL_CHECK(rows > 0, SWL_ERR_INVALID, "combine_norm_rows: no rows to wait or signal for");
  const bool one = sync && sync->signal_flag;  // the signal's one workgroup loops over the rows
  SWL_CHECK(!one || rows <= kFusedSignalRows, SWL_ERR_INVALID, "combine_norm_rows: too many rows for a fused signal");
  CombineNormArgs a{};
  a.dst_h = reinterpret_cast<bf16*>(dst_h);
  a.dst_n = reinterpret_cast<bf16*>(dst_n);
  a.dst_n2 = reinterpret_cast<bf16*>(dst_n2);
  a.src = reinterpret_cast<const bf16*>(src);
  a.delta = reinterpret_cast<const bf16*>(delta);
  a.res = reinterpret_cast<const bf16*>(res);
  a.w = reinterpret_cast<const bf16*>(w);
  a.d = d;
  a.rows = rows;
  a.eps = eps;
  int rc = seq_sync_dev(sync, one, "combine_norm_rows", &a.sync);
  if (rc) return rc;
  hipLaunchKernelGGL(combine_norm_rows_kernel, dim3(one ? 1u : (unsigned)rows), dim3(256), 0, stream, a);
  SWL_LAUNCH_CHECK("combine_norm_rows_kernel launch");
  return SWL_OK;
}

int combine_silu_rows_launch(void* dst, void* dst2, const void* src, int64_t rows, int64_t inter, const void* delta,
                             hipStream_t stream, const SeqSync* sync) {
  auto al = [](const void* p) { return p == nullptr || ((uintptr_t)p % 16) == 0; };
  SWL_CHECK(dst && src && rows >= 0 && inter > 0 && inter % 8 == 0, SWL_ERR_INVALID,
            "combine_silu_rows: bad arguments (inter must be a multiple of 8)");
  SWL_CHECK(rows <= 65535, SWL_ERR_INVALID, "combine_silu_rows: at most 65535 rows");
  SWL_CHECK(al(dst) && al(dst2) && al(src) && al(delta), SWL_ERR_INVALID,
            "combine_silu_rows: pointers must be 16-byte aligned");
  if (rows == 0 && !sync) return SWL_OK;
  SWL_CHECK(rows > 0, SWL_ERR_INVALID, "combine_silu_rows: no rows to wait or signal for");
  const bool one = sync && sync->signal_flag;  // one 1024-thread workgroup loops over everything
  SWL_CHECK(!one || rows <= kFusedSignalRows, SWL_ERR_INVALID, "combine_silu_rows: too many rows for a fused signal");
  CombineSiluArgs a{};
  a.dst = reinterpret_cast<bf16*>(dst);
  a.dst2 = reinterpret_cast<bf16*>(dst2);
  a.src = reinterpret_cast<const bf16*>(src);
  a.delta = reinterpret_cast<const bf16*>(delta);
  a.inter = inter;
  a.rows = rows;
  int rc = seq_sync_dev(sync, one, "combine_silu_rows", &a.sync);
  if (rc) return rc;
  const dim3 grid(one ? 1u : (unsigned)(((inter >> 3) + 255) / 256), one ? 1u : (unsigned)rows);
  hipLaunchKernelGGL(combine_silu_rows_kernel, grid, dim3(one ? 1024 : 256), 0, stream, a);
  SWL_LAUNCH_CHECK("combine_silu_rows_kernel launch");
  return SWL_OK;
}

int wait_copy_launch(const uint64_t* flag, uint64_t want, int32_t tag, uint32_t* timed_out, uint32_t limit_us,
                     void* dst, const void* src, size_t bytes, hipStream_t stream) {
  SWL_CHECK(flag != nullptr && timed_out != nullptr && tag >= 0 && tag < SWL_MAX_SLOTS, SWL_ERR_INVALID,
            "wait_copy: bad flag");
  const bool fused = bytes <= kCopySignalMax && ((uintptr_t)dst % 16) == 0 && ((uintptr_t)src % 16) == 0;
  if (!fused) {
    int rc = seq_wait_launch(1, &flag, &want, &tag, timed_out, limit_us, stream);
    if (rc) return rc;
    if (bytes) SWL_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream));
    return SWL_OK;
  }
  WaitCopyArgs a{};
  a.flag = flag;
  a.want = want;
  a.timed_out = timed_out;
  a.tag = tag;
  a.limit_ticks = (uint32_t)std::min<uint64_t>((uint64_t)limit_us * 100, 0xFFFFFFFFull);
  a.dst = reinterpret_cast<u32x4*>(dst);
  a.src = reinterpret_cast<const u32x4*>(src);
  a.n16 = (int64_t)(bytes / 16);
  a.tail = (int)(bytes % 16);
  hipLaunchKernelGGL(wait_copy_kernel, dim3(1), dim3(1024), 0, stream, a);
  SWL_LAUNCH_CHECK("wait_copy_kernel launch");
  return SWL_OK;
}

int seq_wait_launch(int n, const uint64_t* const* flag, const uint64_t* want, const int32_t* tag, uint32_t* timed_out,
                    uint32_t limit_us, hipStream_t stream) {
  SWL_CHECK(n >= 0 && n <= SWL_MAX_SLOTS, SWL_ERR_INVALID, "seq_wait: at most 128 flags");
  if (n == 0) return SWL_OK;
  SeqWaitArgs a{};
  a.n = n;
  a.limit_ticks = (uint32_t)std::min<uint64_t>((uint64_t)limit_us * 100, 0xFFFFFFFFull);
  a.timed_out = timed_out;
  for (int i = 0; i < n; ++i) {
    SWL_CHECK(flag[i] != nullptr && tag[i] >= 0 && tag[i] < SWL_MAX_SLOTS, SWL_ERR_INVALID, "seq_wait: bad flag");
    a.flag[i] = flag[i];
    a.want[i] = want[i];
    a.tag[i] = tag[i];
  }
  hipLaunchKernelGGL(seq_wait_kernel, dim3(1), dim3(SWL_MAX_SLOTS), 0, stream, a);
  SWL_LAUNCH_CHECK("seq_wait_kernel launch");
  return SWL_OK;
}
}  // namespace swl

// ======================================================== round planner ===
namespace swl {
// LoRA metadata of a round: column blocks (blk_cols, nblk of them, summing
// to N) into L, whether any non-empty segment has an adapter, and the largest
// rank among those (adapter entries checked).
int plan_lora(int n_seg, const int64_t* rows, int64_t N, const int32_t* seg_lora, const swl_lora_entry* lora_table,
              const swl_lora_entry* host_entries, int nblk, const int64_t* blk_cols, LoraEpi* L, bool* has_lora,
              int* max_r) {
  *has_lora = false;
  *max_r = 0;
  if (!seg_lora) return SWL_OK;
  SWL_CHECK(nblk >= 1 && nblk <= SWL_MAX_LORA_BLOCKS, SWL_ERR_INVALID, "round: nblk must be in [1, 4]");
  SWL_CHECK(blk_cols != nullptr, SWL_ERR_INVALID, "round: blk_cols required with LoRA");
  L->nblk = nblk;
  L->blk_start[0] = 0;
  for (int b = 0; b < nblk; ++b) {
    SWL_CHECK(blk_cols[b] > 0, SWL_ERR_INVALID, "round: column blocks must be positive");
    L->blk_start[b + 1] = L->blk_start[b] + blk_cols[b];
  }
  for (int b = nblk + 1; b <= SWL_MAX_LORA_BLOCKS; ++b) L->blk_start[b] = L->blk_start[nblk];
  SWL_CHECK(L->blk_start[nblk] == N, SWL_ERR_INVALID, "round: column blocks must sum to N");
  for (int i = 0; i < n_seg; ++i)
    if (seg_lora[i] >= 0 && rows[i] > 0) *has_lora = true;
  L->table = lora_table;
  if (!*has_lora) return SWL_OK;
  SWL_CHECK(host_entries != nullptr, SWL_ERR_INVALID, "round: missing adapter metadata");
  for (int i = 0; i < n_seg; ++i) {
    if (seg_lora[i] < 0 || rows[i] == 0) continue;
    const swl_lora_entry& e = host_entries[seg_lora[i]];
    SWL_CHECK(e.a != nullptr && e.rank > 0 && e.rank <= 256, SWL_ERR_INVALID, "round: bad adapter entry");
    for (int b = 0; b < nblk; ++b) SWL_CHECK(e.b[b] != nullptr, SWL_ERR_INVALID, "round: adapter missing lora_B");
    *max_r = std::max(*max_r, (int)e.rank);
  }
  return SWL_OK;
}


int round_launch(int n_seg, const int64_t* rows, const void* const* seg_in, void* const* seg_out, const void* w,
                 const void* bias, int64_t N, int64_t K, const int32_t* seg_lora, const swl_lora_entry* lora_table,
                 const swl_lora_entry* host_entries, int nblk, const int64_t* blk_cols, hipStream_t st,
                 const swl_round_fusion* fz) {
  return round_launch_ws(n_seg, rows, seg_in, seg_out, w, bias, N, K, seg_lora, lora_table, host_entries, nblk,
                         blk_cols, st, fz, nullptr, 0);
}

// ws != null: the decode regime only, its partials in [ws, ws + ws_bytes).
int round_launch_ws(int n_seg, const int64_t* rows, const void* const* seg_in, void* const* seg_out, const void* w,
                    const void* bias, int64_t N, int64_t K, const int32_t* seg_lora, const swl_lora_entry* lora_table,
                    const swl_lora_entry* host_entries, int nblk, const int64_t* blk_cols, hipStream_t st,
                    const swl_round_fusion* fz, void* ws, size_t ws_bytes) {
  SWL_CHECK(rows && seg_in && seg_out && w, SWL_ERR_INVALID, "round: null argument");
  SWL_CHECK(n_seg >= 1 && n_seg <= kMaxSeg, SWL_ERR_INVALID, "round: segment count must be in [1, 128]");
  SWL_CHECK(N > 0 && K > 0 && K % 32 == 0, SWL_ERR_INVALID, "round: K must be a positive multiple of 32");
  SWL_CHECK((reinterpret_cast<uintptr_t>(w) & 15) == 0, SWL_ERR_INVALID, "round: weight must be 16-byte aligned");
  int64_t T = 0;
  for (int i = 0; i < n_seg; ++i) {
    SWL_CHECK(rows[i] >= 0, SWL_ERR_INVALID, "round: negative row count");
    SWL_CHECK(rows[i] == 0 || (seg_in[i] && seg_out[i]), SWL_ERR_INVALID, "round: null slot buffer");
    SWL_CHECK((reinterpret_cast<uintptr_t>(seg_in[i]) & 15) == 0, SWL_ERR_INVALID,
              "round: slot input must be 16-byte aligned");
    T += rows[i];
  }
  if (T == 0) return SWL_OK;

  // LoRA planning.
  bool has_lora = false;
  LoraEpi L{};
  int max_r = 0;
  int rc0 = plan_lora(n_seg, rows, N, seg_lora, lora_table, host_entries, nblk, blk_cols, &L, &has_lora, &max_r);
  if (rc0) return rc0;

  const int u_ld = ((max_r * std::max(nblk, 1) + 15) / 16) * 16;  // A rows padded to 16-row tiles
  const bool fused = fz && (fz->norm_weight || fz->out_mode != 0 || fz->w_layout != 0 || fz->a_layout != 0);
  const int64_t out_cols = (fz && fz->out_mode == 2) ? N / 2 : N;
  if (fz && fz->out_mode == 3)
    for (int i = 0; i < n_seg; ++i)
      SWL_CHECK(rows[i] == 1, SWL_ERR_INVALID, "round fusion: out_modes 3 and 4 take one token row per sequence");

  if (T <= kSkinnyMaxTok) {
    // ---------------------------------------------------- decode regime
    const bf16* xr[kSkinnyMaxTok];
    bf16* yr[kSkinnyMaxTok];
    int32_t tl[kSkinnyMaxTok];
    int t = 0;
    for (int i = 0; i < n_seg; ++i) {
      for (int64_t j = 0; j < rows[i]; ++j, ++t) {
        xr[t] = reinterpret_cast<const bf16*>(seg_in[i]) + j * K;
        yr[t] = reinterpret_cast<bf16*>(seg_out[i]) + j * out_cols;
        tl[t] = (has_lora && seg_lora[i] >= 0) ? seg_lora[i] : -1;
      }
    }
    return launch_skinny(reinterpret_cast<const bf16*>(w), reinterpret_cast<const bf16*>(bias), N, K, (int)T, xr, yr,
                         has_lora ? tl : nullptr, lora_table, host_entries, &L, nblk, fz, st, ws, ws_bytes);
  }
  SWL_CHECK(!fused, SWL_ERR_INVALID, "round fusion / fragment-tile weights: at most 64 token rows");
  SWL_CHECK(!ws, SWL_ERR_INVALID, "allocation-free round: at most 64 token rows");

  // ------------------------------------------------------ prefill regime
  SWL_CHECK(K % TK == 0, SWL_ERR_INVALID, "round: K must be a multiple of 64 for > 64 tokens");
  // Segments by rows, most first (stable): the small ones (one-row slots)
  // share the last, partly empty row tile, whose skipped MFMA blocks leave
  // time for their LoRA k-steps, instead of adding a step run per segment
  // to a full tile (the slowest tile ends the launch).  A row's result does
  // not depend on its position in the batch.
  int ord[kMaxSeg];
  for (int i = 0; i < n_seg; ++i) ord[i] = i;
  std::stable_sort(ord, ord + n_seg, [&](int x, int y) { return rows[x] > rows[y]; });
  int64_t rows_by[kMaxSeg];
  const void* in_by[kMaxSeg];
  void* out_by[kMaxSeg];
  int32_t lora_by[kMaxSeg];
  for (int i = 0; i < n_seg; ++i) {
    rows_by[i] = rows[ord[i]];
    in_by[i] = seg_in[ord[i]];
    out_by[i] = seg_out[ord[i]];
    lora_by[i] = seg_lora ? seg_lora[ord[i]] : -1;
  }
  rows = rows_by;
  seg_in = in_by;
  seg_out = out_by;
  if (seg_lora) seg_lora = lora_by;
  // the 256 x 256 GEMM and the shrink read the token rows in place from the
  // slot buffers (16-byte aligned: checked above); only the 128 x 128
  // kernel takes a packed copy
  const bool packed_x = prefill_uses_tiled(K);
  const size_t xbytes = packed_x ? sizeof(bf16) * (size_t)T * (size_t)K : 0;
  const size_t xbytes_al = (xbytes + 255) & ~(size_t)255;
  // LoRA shrink K-slices: enough (item, slice) workgroups to fill the chip
  int u_ks = 1;
  if (has_lora) {
    int64_t items = 0;
    for (int i = 0; i < n_seg; ++i)
      if (seg_lora[i] >= 0 && rows[i] > 0)
        items += (rows[i] + 63) / 64 * ((host_entries[seg_lora[i]].rank * nblk + 63) / 64);
    while (u_ks < 16 && items * u_ks < 1024 && (K / 32) / (2 * u_ks) >= 8) u_ks *= 2;
  }
  size_t ubytes = 0;
  if (has_lora) ubytes = sizeof(float) * (size_t)u_ks * (size_t)T * (size_t)u_ld;
  void* scr = nullptr;
  int rc = scratch_get(xbytes_al + ubytes, st, &scr);
  if (rc) return rc;
  bf16* packed = reinterpret_cast<bf16*>(scr);
  if (packed_x) {
    rc = swl_gather_bf16(seg_in, rows, n_seg, K, packed, st);
    if (rc) return rc;
  }

  TiledArgs a{};
  a.x = packed_x ? packed : nullptr;
  for (int i = 0; i < n_seg; ++i) a.xin[i] = reinterpret_cast<const bf16*>(seg_in[i]);
  a.w = reinterpret_cast<const bf16*>(w);
  a.bias = reinterpret_cast<const bf16*>(bias);
  a.M = T;
  a.N = N;
  a.K = K;
  a.y = nullptr;
  int64_t dummy = 0;
  rc = fill_segptrs(a.out, reinterpret_cast<const void* const*>(seg_out), rows, n_seg, N, &dummy);
  if (rc) return rc;
  if (has_lora) {
    float* u = reinterpret_cast<float*>(reinterpret_cast<char*>(scr) + xbytes_al);
    int64_t rws[kMaxSeg];
    for (int i = 0; i < n_seg; ++i) {
      rws[i] = rows[i];
      a.seg_lora[i] = (seg_lora[i] >= 0 && rows[i] > 0) ? seg_lora[i] : -1;
    }
    const bf16* seg_x[kMaxSeg];
    for (int i = 0; i < n_seg; ++i) seg_x[i] = packed_x ? packed + a.out.off[i] * K : a.xin[i];
    rc = launch_shrink_gemm(seg_x, K, n_seg, a.out.off, rws, a.seg_lora, host_entries, nblk, u, u_ld,
                            (int64_t)T * u_ld, u_ks, st);
    if (rc) return rc;
    a.has_lora = 1;
    a.L = L;
    a.L.u = u;
    a.L.usplit = 1;  // folded into split 0
    a.L.u_ld = u_ld;
    a.L.u_split_stride = (int64_t)T * u_ld;
    // the 256 x 256 kernel adds the LoRA delta as MFMA k-steps when every
    // tile lies inside one column block and the ranks are multiples of 8
    a.lora_mfma = 1;
    for (int b = 1; b < nblk; ++b) a.lora_mfma &= (L.blk_start[b] % PG_N == 0) ? 1 : 0;
    for (int i = 0; i < n_seg; ++i)
      if (a.seg_lora[i] >= 0) {
        const int r = host_entries[a.seg_lora[i]].rank;
        a.lora_mfma &= (r % 8 == 0 && r <= 64) ? 1 : 0;
      }
  }
  return launch_prefill_gemm(a, st);
}

}  // namespace swl

namespace swl {

int embed_launch(int n, const int64_t* rows, const void* const* ids, void* const* out, const void* table,
                 int64_t vocab, int64_t hidden, hipStream_t st) {
  SWL_CHECK(n >= 1 && n <= kMaxSeg, SWL_ERR_INVALID, "embed: segment count must be in [1, 128]");
  SWL_CHECK(hidden % 8 == 0, SWL_ERR_INVALID, "embed: hidden size must be a multiple of 8");
  EmbedArgs a{};
  a.n = n;
  a.off[0] = 0;
  for (int i = 0; i < n; ++i) {
    a.off[i + 1] = a.off[i] + rows[i];
    a.ids[i] = reinterpret_cast<const int64_t*>(ids[i]);
    a.out[i] = reinterpret_cast<bf16*>(out[i]);
  }
  a.table = reinterpret_cast<const bf16*>(table);
  a.vocab = vocab;
  a.hidden = hidden;
  if (a.off[n] == 0) return SWL_OK;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)a.off[n]), dim3(256), 0, st, a);
  SWL_LAUNCH_CHECK("embed_kernel launch");
  return SWL_OK;
}

int lm_head_launch(int n, const void* const* last_rows, const void* lm_head, int64_t vocab, int64_t hidden,
                   void* packed, void* logits, int64_t* next_tok, void* const* out_tok, const int32_t* do_sample,
                   const float* temperature, const int32_t* top_k, const float* top_p, uint64_t seed,
                   hipStream_t st) {
  SWL_CHECK(n >= 1 && n <= kMaxSeg, SWL_ERR_INVALID, "lm_head: slot count must be in [1, 128]");
  (void)next_tok;
  int64_t ones[kMaxSeg];
  for (int i = 0; i < n; ++i) ones[i] = 1;
  int rc = swl_gather_bf16(last_rows, ones, n, hidden, packed, st);
  if (rc) return rc;
  rc = swl_gemm_bf16(packed, lm_head, nullptr, logits, n, vocab, hidden, st);
  if (rc) return rc;
  SampleArgs a{};
  a.logits = reinterpret_cast<const bf16*>(logits);
  a.vocab = vocab;
  a.seed = seed;
  for (int i = 0; i < n; ++i) {
    a.out_tok[i] = reinterpret_cast<int64_t*>(out_tok[i]);
    a.do_sample[i] = do_sample[i];
    a.temperature[i] = temperature[i];
    a.top_k[i] = top_k[i];
    a.top_p[i] = top_p[i];
  }
  hipLaunchKernelGGL(sample_kernel, dim3((unsigned)n), dim3(1024), 0, st, a);
  SWL_LAUNCH_CHECK("sample_kernel launch");
  return SWL_OK;
}

}  // namespace swl

extern "C" int swl_sample_bf16(const void* logits, int64_t n, int64_t vocab, void* const* out_tok,
                               const int32_t* do_sample, const float* temperature, const int32_t* top_k,
                               const float* top_p, uint64_t seed, void* stream) {
  SWL_CHECK(logits && out_tok && do_sample && temperature && top_k && top_p, SWL_ERR_INVALID,
            "swl_sample_bf16: null argument");
  SWL_CHECK(n >= 1 && n <= kMaxSeg && vocab > 0 && vocab < ((int64_t)1 << 31), SWL_ERR_INVALID,
            "swl_sample_bf16: bad shape");
  SampleArgs a{};
  a.logits = reinterpret_cast<const bf16*>(logits);
  a.vocab = vocab;
  a.seed = seed;
  for (int i = 0; i < n; ++i) {
    SWL_CHECK(out_tok[i] != nullptr, SWL_ERR_INVALID, "swl_sample_bf16: null output");
    SWL_CHECK(temperature[i] > 0.f, SWL_ERR_INVALID, "swl_sample_bf16: temperature must be > 0");
    a.out_tok[i] = reinterpret_cast<int64_t*>(out_tok[i]);
    a.do_sample[i] = do_sample[i];
    a.temperature[i] = temperature[i];
    a.top_k[i] = top_k[i];
    a.top_p[i] = top_p[i];
  }
  hipLaunchKernelGGL(sample_kernel, dim3((unsigned)n), dim3(1024), 0, (hipStream_t)stream, a);
  SWL_LAUNCH_CHECK("sample_kernel launch");
  return SWL_OK;
}

extern "C" int swl_embed_bf16(const void* const* ids, const int64_t* rows, int n, const void* table, int64_t vocab,
                              int64_t hidden, void* const* out, void* stream) {
  SWL_CHECK(ids && rows && table && out, SWL_ERR_INVALID, "swl_embed_bf16: null argument");
  return swl::embed_launch(n, rows, ids, out, table, vocab, hidden, (hipStream_t)stream);
}

// ============================================= worker-side row entry points
extern "C" int swl_rmsnorm_rows_bf16(void* h, int64_t ntok, int64_t d, const void* const* add_rows,
                                     const void* weight, float eps, void* const* out_rows, void* stream) {
  SWL_CHECK(h && weight && out_rows, SWL_ERR_INVALID, "swl_rmsnorm_rows_bf16: null argument");
  SWL_CHECK(ntok >= 0 && ntok <= kSkinnyMaxTok, SWL_ERR_INVALID, "swl_rmsnorm_rows_bf16: at most 64 rows");
  SWL_CHECK(d > 0 && d % 8 == 0, SWL_ERR_INVALID, "swl_rmsnorm_rows_bf16: d must be a multiple of 8");
  if (ntok == 0) return SWL_OK;
  RowPtrs r{};
  r.ntok = (int)ntok;
  for (int i = 0; i < ntok; ++i) {
    SWL_CHECK(out_rows[i] && (!add_rows || add_rows[i]), SWL_ERR_INVALID, "swl_rmsnorm_rows_bf16: null row");
    r.out[i] = reinterpret_cast<bf16*>(out_rows[i]);
    r.in[i] = add_rows ? reinterpret_cast<const bf16*>(add_rows[i]) : nullptr;
  }
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((unsigned)ntok), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<bf16*>(h), d, r, reinterpret_cast<const bf16*>(weight), eps, add_rows ? 1 : 0);
  SWL_LAUNCH_CHECK("rmsnorm_rows_kernel launch");
  return SWL_OK;
}

extern "C" int swl_silu_mul_rows_bf16(const void* const* in_rows, void* const* out_rows, int64_t ntok,
                                      int64_t inter, void* stream) {
  SWL_CHECK(in_rows && out_rows, SWL_ERR_INVALID, "swl_silu_mul_rows_bf16: null argument");
  SWL_CHECK(ntok >= 0 && ntok <= kSkinnyMaxTok, SWL_ERR_INVALID, "swl_silu_mul_rows_bf16: at most 64 rows");
  SWL_CHECK(inter > 0 && inter % 8 == 0, SWL_ERR_INVALID, "swl_silu_mul_rows_bf16: inter must be a multiple of 8");
  if (ntok == 0) return SWL_OK;
  RowPtrs r{};
  r.ntok = (int)ntok;
  for (int i = 0; i < ntok; ++i) {
    SWL_CHECK(in_rows[i] && out_rows[i], SWL_ERR_INVALID, "swl_silu_mul_rows_bf16: null row");
    r.in[i] = reinterpret_cast<const bf16*>(in_rows[i]);
    r.out[i] = reinterpret_cast<bf16*>(out_rows[i]);
  }
  const dim3 grid((unsigned)(((inter >> 3) + 255) / 256), (unsigned)ntok);
  hipLaunchKernelGGL(silu_mul_rows_kernel, grid, dim3(256), 0, (hipStream_t)stream, r, inter);
  SWL_LAUNCH_CHECK("silu_mul_rows_kernel launch");
  return SWL_OK;
}

extern "C" int swl_paged_attention_rows_bf16(void* const* qkv_rows, void* const* out_rows, int nseq, int q_len,
                                             int hq, int hkv, int d, void* k_cache, void* v_cache,
                                             int64_t num_blocks, int block_size, const int32_t* block_table,
                                             int64_t max_blocks, const int32_t* cache_seqlens,
                                             const int64_t* positions, const void* cos_sin, int64_t max_pos,
                                             int rope, float softmax_scale, void* stream) {
  SWL_CHECK(qkv_rows && out_rows && k_cache && v_cache && block_table && cache_seqlens, SWL_ERR_INVALID,
            "swl_paged_attention_rows_bf16: null argument");
  SWL_CHECK(d == 128 && hq > 0 && hkv > 0 && hq % hkv == 0, SWL_ERR_INVALID,
            "swl_paged_attention_rows_bf16: head_dim must be 128 and hq a multiple of hkv");
  const int G = hq / hkv;
  SWL_CHECK(G == 1 || G == 2 || G == 4 || G == 8, SWL_ERR_INVALID,
            "swl_paged_attention_rows_bf16: hq / hkv must be 1, 2, 4 or 8");
  SWL_CHECK(nseq >= 0 && q_len >= 1 && (int64_t)nseq * q_len <= kSkinnyMaxTok, SWL_ERR_INVALID,
            "swl_paged_attention_rows_bf16: at most 64 token rows");
  SWL_CHECK(block_size > 0 && num_blocks > 0 && max_blocks > 0, SWL_ERR_INVALID,
            "swl_paged_attention_rows_bf16: bad page geometry");
  SWL_CHECK(rope >= 0 && rope <= 2 && (rope < 2 || q_len == 1), SWL_ERR_INVALID,
            "swl_paged_attention_rows_bf16: rope must be 0, 1 or 2 (2: decode rows only)");
  SWL_CHECK(rope == 1 ? (cos_sin && positions && max_pos > 0) : true, SWL_ERR_INVALID,
            "swl_paged_attention_rows_bf16: rope needs positions and cos_sin");
  if (nseq == 0) return SWL_OK;
  AttnArgs a{};
  a.rowmode = 1;
  for (int t = 0; t < nseq * q_len; ++t) {
    SWL_CHECK(qkv_rows[t] && out_rows[t] && (reinterpret_cast<uintptr_t>(qkv_rows[t]) & 15) == 0, SWL_ERR_INVALID,
              "swl_paged_attention_rows_bf16: rows must be non-null and 16-byte aligned");
    a.qkv_row[t] = reinterpret_cast<bf16*>(qkv_rows[t]);
    a.out_row[t] = reinterpret_cast<bf16*>(out_rows[t]);
  }
  a.kc = reinterpret_cast<bf16*>(k_cache);
  a.vc = reinterpret_cast<bf16*>(v_cache);
  a.bt = block_table;
  a.seqlens = cache_seqlens;
  a.pos = positions;
  a.cs = reinterpret_cast<const bf16*>(cos_sin);
  a.num_blocks = num_blocks;
  a.max_blocks = max_blocks;
  a.max_pos = max_pos;
  a.nseq = nseq;
  a.L = q_len;
  a.hq = hq;
  a.hkv = hkv;
  a.bs = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.rope = rope;
  a.scale = softmax_scale;
  return launch_attention(a, G, (hipStream_t)stream);
}

