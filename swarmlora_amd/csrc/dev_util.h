// Device helpers shared by the HIP translation units of libswl (gfx950):
// bf16 vector types, loads and stores through global-address-space
// pointers, the 16x16x32 bf16 MFMA, s_waitcnt immediates and the LDS-only
// workgroup barrier.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// 16-byte load of device memory through a global-address-space pointer
// (global_load, not flat: a flat load also counts against lgkmcnt)
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const __attribute__((address_space(1))) u32x4*)(p); }

// Stores through global-address-space pointers (global_store, not flat): a
// flat store also counts against lgkmcnt, so every later wait for an LDS
// read would wait for the store too.  Every output row is device memory.
__device__ __forceinline__ void stg(bf16* p, u32x2 v) { *(__attribute__((address_space(1))) u32x2*)(p) = v; }
__device__ __forceinline__ void stg(bf16* p, bf16 v) { *(__attribute__((address_space(1))) bf16*)(p) = v; }
__device__ __forceinline__ bf16 ldg(const bf16* p) { return *(const __attribute__((address_space(1))) bf16*)(p); }

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ float bf2f(bf16 v) { return (float)v; }
__device__ __forceinline__ bf16 f2bf(float v) { return (bf16)v; }  // v_cvt_pk_bf16_f32, RNE

__device__ __forceinline__ void unpack8(u32x4 v, float (&f)[8]) {
  bf16x8 b = __builtin_bit_cast(bf16x8, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (float)b[i];
}

__device__ __forceinline__ u32x4 lds16(const bf16* p) { return *reinterpret_cast<const u32x4*>(p); }

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(1))) void* gbl_ptr;
// s_waitcnt immediate for vmcnt(0) alone (gfx9 encoding: expcnt and lgkmcnt
// at their maxima, i.e. not waited on)
constexpr unsigned kWaitVm0 = 0x0F70;
// Cache-policy operand of the buffer-store builtin: sc0 | sc1 (system scope).
constexpr int kStoreSys = 1 | 16;

// 16-byte load through a global-address-space pointer (global_load, not flat)
__device__ __forceinline__ u32x4 ldg16(const void* p) {
  return *(const __attribute__((address_space(1))) u32x4*)(p);
}
// The same load marked non-temporal, for bytes read once per pass (the
// projection weights and adapter rows of a decode step, the KV pages): a
// streaming read that does not displace reused lines (and reaches HBM's
// read rate more closely: 5.7-6.2 against 5.3-5.6 TB/s for a plain 16-byte
// grid-stride read of 1 GiB on MI355X).
__device__ __forceinline__ u32x4 ldg16_nt(const void* p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4*)(p));
}
// Cache-policy operand of global_load_lds for such streaming reads: nt.
constexpr int kLoadNT = 2;
__device__ __forceinline__ float ldg_f32(const float* p) {
  return *(const __attribute__((address_space(1))) float*)(p);
}

// s_waitcnt immediate for vmcnt(n) alone (gfx9 encoding: vmcnt in bits 3:0
// and 15:14, expcnt and lgkmcnt at their maxima)
__host__ __device__ constexpr unsigned wait_vm_imm(int n) {
  return 0x0F70u | (unsigned)(n & 15) | ((unsigned)(n >> 4) << 14);
}

// Workgroup barrier for LDS hand-offs only: this wave's LDS accesses are
// complete, then s_barrier.  Unlike __syncthreads it does not wait for the
// wave's outstanding global loads (the next tile's weights stay in flight);
// the signal fences keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// x = bf16(bf16(h * r) * gamma) of one B fragment (token row factor r,
// gamma of the fragment's 8 dims)
__device__ __forceinline__ u32x4 norm8(u32x4 h, float r, u32x4 g) {
  float hv[8], gv[8];
  unpack8(h, hv);
  unpack8(g, gv);
  bf16x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = f2bf(bf2f(f2bf(hv[j] * r)) * gv[j]);
  return __builtin_bit_cast(u32x4, o);
}

}  // namespace
