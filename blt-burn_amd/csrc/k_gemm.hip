// Launch selection for the bf16 MFMA GEMM (kernel in gemm_kernel.hpp).
#include "gemm_kernel.hpp"

namespace blt {

namespace {
template <int BM, int BN, int BK, int WM, int WN, int PF, int OCC>
int run_gemm(const GemmArgs& a, hipStream_t s) {
  const int64_t nb = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm::gemm_bf16_kernel<BM, BN, BK, WM, WN, PF, OCC>), dim3((unsigned)nb),
                     dim3(64 * WM * WN), 0, s, a);
  BLT_LAUNCH_CHECK("gemm_bf16_kernel");
  return 0;
}

}  // namespace

int launch_gemm(const GemmArgs& a_in, hipStream_t s) {
  GemmArgs a = a_in;
  if (a.M == 0 || a.N == 0) return 0;
  a.vec_ok = ((uintptr_t)a.C % 16 == 0) && (a.ldc % 4 == 0);
  if ((a.epi == EPI_BF16 || a.epi == EPI_RESID_F32 || a.epi == EPI_QKV_ROPE ||
       a.epi == EPI_SILU_GATE) && (a.N % 64 != 0 || a.ldc % 4 != 0 || (uintptr_t)a.C % 16 != 0))
    return fail(-2, "gemm: vector epilogues need N % 64 == 0, ldc % 4 == 0, 16-byte aligned C");
  if (a.K % 64 != 0) return fail(-2, "gemm: K must be a multiple of 64");
  // N % 256 == 0: 128x256 tiles over 8 waves (wave tile 64x64, BK 32, two
  // tiles in flight, 2 blocks per CU).  Otherwise 128x128 tiles over 4 waves.
  if (a.N % 256 == 0) return run_gemm<128, 256, 32, 2, 4, 2, 2>(a, s);
  return run_gemm<128, 128, 32, 2, 2, 2, 3>(a, s);
}

}  // namespace blt
