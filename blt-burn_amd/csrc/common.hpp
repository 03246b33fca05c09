// Shared device/host helpers for the gfx950 kernels: bf16 conversion, wave64
// reductions, error plumbing for the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
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
// All on the VALU (no LDS permutes): DPP quad permutes pair lanes xor 1 and
// xor 2, the row half-mirror pairs the two quads of each 8 lanes and the row
// mirror the two halves of each 16 lanes; v_permlane16_swap / v_permlane32_swap
// then hand each lane its partner in the neighbouring 16- and 32-lane group.
// Each step combines a lane's value with exactly one partner and both
// partners compute the same (commutative) result, so every lane of the group
// ends with the identical value.
template <int CTRL>
__device__ inline float dpp_f32(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// {own, partner} of lane ^ 16 (X = 16) or lane ^ 32 (X = 32), in some order
template <int X>
__device__ inline void swap_pair(float v, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  if constexpr (X == 16) {
    const auto s = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    a = __builtin_bit_cast(float, (unsigned)s[0]);
    b = __builtin_bit_cast(float, (unsigned)s[1]);
  } else {
    const auto s = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    a = __builtin_bit_cast(float, (unsigned)s[0]);
    b = __builtin_bit_cast(float, (unsigned)s[1]);
  }
}
// sum over each aligned group of 16 lanes, in every lane of the group
__device__ inline float sum16(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  return v;
}
__device__ inline float wave_sum(float v) {
  v = sum16(v);
  float a, b;
  swap_pair<16>(v, a, b);
  v = a + b;
  swap_pair<32>(v, a, b);
  return a + b;
}
// Inclusive prefix sums on the VALU (GFX9 DPP; lanes with no source add 0):
// row_shr 1, 2, 4, 8 within each 16-lane row, then row_bcast:15 (last lane of
// rows 0 / 2 into rows 1 / 3) and row_bcast:31 (lane 31 into rows 2 and 3).
template <int CTRL, int ROWS>
__device__ inline int dpp_i32(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, ROWS, 0xF, false);
}
__device__ inline int row16_incl_scan(int v) {
  v += dpp_i32<0x111, 0xF>(v);
  v += dpp_i32<0x112, 0xF>(v);
  v += dpp_i32<0x114, 0xF>(v);
  v += dpp_i32<0x118, 0xF>(v);
  return v;
}
__device__ inline int wave_incl_scan(int v) {
  v = row16_incl_scan(v);
  v += dpp_i32<0x142, 0xA>(v);
  v += dpp_i32<0x143, 0xC>(v);
  return v;
}
// max / sum over each 32-lane half of the wave, in every lane of the half
__device__ inline float half_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  float a, b;
  swap_pair<16>(v, a, b);
  return fmaxf(a, b);
}
__device__ inline float half_sum(float v) {
  v = sum16(v);
  float a, b;
  swap_pair<16>(v, a, b);
  return a + b;
}

// Softmax entropy (natural log) of one row held by the 32 lanes of a half
// wave: lane l has elements c * 128 + 4 l .. + 3 in v[c] (c < NH) and
// NH * 128 + 32 q + l in t[q] (-inf past the row's end).  With d = x - max
// and p = e^d, H = log sum p - sum(p d) / sum p, the same quantity as
// -sum exp(lsm) lsm; padding (-inf) contributes 0.  Shared by every kernel
// that computes entropies of rows below 512 elements, so their values agree
// bit for bit.
template <int NH, int VT>
__device__ inline float entropy_half_row(const float (&v)[NH > 0 ? NH : 1][4],
                                         const float (&t)[VT > 0 ? VT : 1]) {
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < NH; ++c)
    m = fmaxf(m, fmaxf(fmaxf(v[c][0], v[c][1]), fmaxf(v[c][2], v[c][3])));
#pragma unroll
  for (int q = 0; q < VT; ++q) m = fmaxf(m, t[q]);
  m = half_max(m);
  float sp = 0.f, sd = 0.f;
  auto acc = [&](float xv) {
    const float d = fmaxf(xv - m, -1e30f);
    const float pe = __expf(d);
    sp += pe;
    sd = fmaf(pe, d, sd);
  };
#pragma unroll
  for (int c = 0; c < NH; ++c)
#pragma unroll
    for (int k = 0; k < 4; ++k) acc(v[c][k]);
#pragma unroll
  for (int q = 0; q < VT; ++q) acc(t[q]);
  sp = half_sum(sp);
  sd = half_sum(sd);
  // hardware reciprocal (1 ulp) for the one quotient per row
  return __logf(sp) - sd * __builtin_amdgcn_rcpf(sp);
}

__device__ inline float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  float a, b;
  swap_pair<16>(v, a, b);
  v = fmaxf(a, b);
  swap_pair<32>(v, a, b);
  return fmaxf(a, b);
}

// the same reduction over 32-bit integers (max)
__device__ inline int wave_max_i32(int v) {
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));
  const auto s16 = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
  v = max((int)s16[0], (int)s16[1]);
  const auto s32 = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  return max((int)s32[0], (int)s32[1]);
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
