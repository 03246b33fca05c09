// Shared device/host helpers for the gfx950 kernels: bf16 conversion, wave64
// reductions, error plumbing for the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#define BLT_WAVE 64

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace blt {

// ---- error plumbing (host) -------------------------------------------------
void set_error(const std::string& msg);
int fail(int status, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

#define BLT_HIP_CHECK(expr)                                   \
  do {                                                        \
    hipError_t _e = (expr);                                   \
    if (_e != hipSuccess) return ::blt::hip_fail(_e, #expr);  \
  } while (0)

// Check the launch that was just queued.
#define BLT_LAUNCH_CHECK(what)                                \
  do {                                                        \
    hipError_t _e = hipGetLastError();                        \
    if (_e != hipSuccess) return ::blt::hip_fail(_e, what);   \
  } while (0)

// ---- bf16 <-> f32 ------------------------------------------------------------
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// Round to nearest even; NaN stays NaN.  On the device this is the gfx950
// v_cvt_pk_bf16_f32 instruction; the host path is the same rounding in integers.
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
#endif
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// two floats -> packed bf16 pair (lo in bits 0..15), one v_cvt_pk_bf16_f32
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// ---- wave64 reductions -----------------------------------------------------
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, BLT_WAVE));
  return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, BLT_WAVE);
  return v;
}

inline unsigned ceil_div(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

// Wait until at most N of this wave's vector-memory loads are outstanding and
// its LDS operations are done, then barrier; the memory clobber keeps the
// compiler from moving LDS accesses across it.
template <int N>
__device__ inline void dma_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// 16 bytes per lane from global memory straight into LDS (gfx950
// global_load_lds_dwordx4) with a wave-uniform 64-bit base (SGPRs) and a
// per-lane 32-bit byte offset: lane i's 16 bytes at base + off land at LDS
// byte lds_addr + 16 * i (lds_addr wave-uniform).  Issued from inline asm so
// the compiler does not serialise it against later LDS reads; callers order
// it with dma_wait_barrier.  M0 is restored.
__device__ inline void dma16_so(const void* base_in, unsigned off, unsigned lds_addr) {
  // the base is wave-uniform by construction; make that explicit so it is
  // held in SGPRs (readfirstlane returns int: each half goes through
  // uint32_t so the low word is not sign-extended into the high one)
  const uint64_t b = (uint64_t)(uintptr_t)base_in;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint64_t base = (uint64_t)lo | ((uint64_t)hi << 32);
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_addr), "v"(off), "s"(base)
      : "memory");
}

}  // namespace blt
