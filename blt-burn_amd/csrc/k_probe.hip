// Measurement helpers: the MFMA rate and the HBM copy bandwidth this GPU
// actually sustains, against which the kernels' roofline fractions can be
// read beside the published peaks (the clock under a full MFMA load sits
// below the one the 2.5 PFLOP/s figure assumes).
#include "blt_hip.h"
#include "rowops.hpp"

namespace blt {

namespace {

// Each wave keeps 4 independent accumulator chains of
// v_mfma_f32_32x32x16_bf16 busy for `iters` rounds.  The operands are
// lane-dependent constants; the results only reach memory if their sum hits
// an impossible value, so nothing is stored in practice.
__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, float* sink) {
  const int lane = threadIdx.x & 63;
  const bf16x8_t a = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3F803F80u + lane, 0x3F803F80u,
                                                          0x3F803F80u, 0x3F803F80u});
  const bf16x8_t b = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3C003C00u, 0x3C003C00u + lane,
                                                          0x3C003C00u, 0x3C003C00u});
  f32x16_t acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[u], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[u][r];
  if (s == -1.2345e-30f) sink[blockIdx.x * 256 + threadIdx.x] = s;
}

// One 16-byte piece per thread (the fastest copy shape measured here: grid-
// stride loops over fewer blocks reach 75-90% of its rate).
__global__ __launch_bounds__(256) void copy16_kernel(const u32x4_t* __restrict__ src,
                                                     u32x4_t* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

}  // namespace

}  // namespace blt

using namespace blt;

extern "C" {

int64_t blt_probe_mfma_flops(int32_t blocks, int32_t iters) {
  if (blocks <= 0 || iters <= 0) return -1;
  return (int64_t)blocks * 4 * iters * 4 * (32LL * 32 * 16 * 2);
}

int blt_probe_mfma_bf16(int32_t blocks, int32_t iters, float* sink, blt_stream_t stream) {
  if (blocks <= 0 || iters <= 0) return fail(BLT_ERR_SHAPE, "probe_mfma: blocks, iters > 0");
  if (!sink) return fail(BLT_ERR_INVALID, "probe_mfma: null sink");
  hipLaunchKernelGGL(mfma_peak_kernel, dim3(blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), iters, sink);
  BLT_LAUNCH_CHECK("mfma_peak_kernel");
  return BLT_OK;
}

int blt_probe_copy(const void* src, void* dst, int64_t bytes, blt_stream_t stream) {
  if (bytes < 0 || bytes % 16 != 0) return fail(BLT_ERR_SHAPE, "probe_copy: bytes % 16 == 0");
  if (bytes == 0) return BLT_OK;
  if (!src || !dst || (uintptr_t)src % 16 || (uintptr_t)dst % 16)
    return fail(BLT_ERR_INVALID, "probe_copy: 16-byte aligned buffers");
  const int64_t n = bytes / 16;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return fail(BLT_ERR_SHAPE, "probe_copy: too large");
  hipLaunchKernelGGL(copy16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const u32x4_t*>(src),
                     reinterpret_cast<u32x4_t*>(dst), n);
  BLT_LAUNCH_CHECK("copy16_kernel");
  return BLT_OK;
}

}  // extern "C"
