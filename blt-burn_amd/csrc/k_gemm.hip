// Launch selection for the bf16 MFMA GEMM (kernel in gemm_kernel.hpp).
#include "gemm_kernel.hpp"

namespace blt {

namespace {
template <int BM, int BN, int BK, int WM, int WN, int S, int OCC, int EPI>
int run_gemm_dma(const GemmArgs& a, hipStream_t s) {
  const int64_t nb = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm::gemm_bf16_dma_kernel<BM, BN, BK, WM, WN, S, OCC, EPI>),
                     dim3((unsigned)nb), dim3(64 * WM * WN), 0, s, a);
  BLT_LAUNCH_CHECK("gemm_bf16_dma_kernel");
  return 0;
}

// one kernel per epilogue, so each carries only its own registers and code
template <int BM, int BN, int BK, int WM, int WN, int S, int OCC>
int run_gemm_dma_epi(const GemmArgs& a, hipStream_t s) {
  switch (a.epi) {
    case EPI_BF16: return run_gemm_dma<BM, BN, BK, WM, WN, S, OCC, EPI_BF16>(a, s);
    case EPI_F32: return run_gemm_dma<BM, BN, BK, WM, WN, S, OCC, EPI_F32>(a, s);
    case EPI_RESID_F32: return run_gemm_dma<BM, BN, BK, WM, WN, S, OCC, EPI_RESID_F32>(a, s);
    case EPI_QKV_ROPE: return run_gemm_dma<BM, BN, BK, WM, WN, S, OCC, EPI_QKV_ROPE>(a, s);
    case EPI_SILU_GATE: return run_gemm_dma<BM, BN, BK, WM, WN, S, OCC, EPI_SILU_GATE>(a, s);
  }
  return fail(-2, "gemm: unknown epilogue");
}

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
  if ((a.xb_out != nullptr) != (a.ss_out != nullptr) ||
      (a.xb_out && (a.epi != EPI_RESID_F32 || a.ss_np * 64 != a.N || (uintptr_t)a.xb_out % 8)))
    return fail(-2, "gemm: norm partials need EPI_RESID_F32, xb_out and ss_out, ss_np = N / 64");

  if ((uintptr_t)a.A % 16 != 0 || (uintptr_t)a.Bt % 16 != 0 || a.lda % 8 != 0 || a.ldb % 8 != 0)
    return fail(-2, "gemm: A and Bt rows must be 16-byte aligned (lda, ldb % 8 == 0)");
  // Wide N (QKV, W1|W3): walk groups of 8 M-tiles so the blocks resident on
  // an XCD share A and Bt tiles in its L2; narrow N (O, W2: 3 tiles): N fastest.
  a.group_m = (a.N + 255) / 256 >= 8 ? 8 : 0;
  // N % 256 == 0: 256x256 tiles over 8 waves (wave tile 128x64), K tiles of
  // 64 moved by LDS DMA through 2 stages, LDS-staged epilogue.  Otherwise (the
  // 260-wide head) 128x128 register-staged tiles over 4 waves.
  if (a.N % 256 == 0) return run_gemm_dma_epi<256, 256, 64, 2, 4, 2, 2>(a, s);
  return run_gemm<128, 128, 32, 2, 2, 2, 3>(a, s);
}

}  // namespace blt
