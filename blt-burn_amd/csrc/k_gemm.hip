// Launch selection for the bf16 MFMA GEMM (kernel in gemm_kernel.hpp).
#include "gemm_kernel.hpp"

namespace blt {

namespace {
// Compute units of the current device (cached per device).
int device_cus() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

template <int BM, int BN, int BK, int WM, int WN, int EPI>
int run_gemm_persistent(const GemmArgs& a, hipStream_t s) {
  const int64_t nb = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  // as many blocks as fit on the CUs at once (256x256: one per CU, its LDS
  // holds 160 KB; 128x128: two, 80 KB each), a multiple of 8 blocks so each
  // keeps its XCD residue
  int64_t grid = (int64_t)device_cus() * (BM * BN <= 128 * 128 ? 2 : 1);
  grid = grid >= 8 ? grid & ~7 : grid;
  if (grid <= 0 || grid > nb) grid = nb;
  hipLaunchKernelGGL((gemm::gemm_bf16_dma_persistent_kernel<BM, BN, BK, WM, WN, EPI>),
                     dim3((unsigned)grid), dim3(64 * WM * WN), 0, s, a);
  BLT_LAUNCH_CHECK("gemm_bf16_dma_persistent_kernel");
  return 0;
}

// one kernel per epilogue, so each carries only its own registers and code
template <int BM, int BN, int BK, int WM, int WN>
int run_gemm_dma_epi(const GemmArgs& a, hipStream_t s) {
  switch (a.epi) {
    case EPI_BF16: return run_gemm_persistent<BM, BN, BK, WM, WN, EPI_BF16>(a, s);
    case EPI_F32: return run_gemm_persistent<BM, BN, BK, WM, WN, EPI_F32>(a, s);
    case EPI_RESID_F32: return run_gemm_persistent<BM, BN, BK, WM, WN, EPI_RESID_F32>(a, s);
    case EPI_QKV_ROPE: return run_gemm_persistent<BM, BN, BK, WM, WN, EPI_QKV_ROPE>(a, s);
    case EPI_SILU_GATE: return run_gemm_persistent<BM, BN, BK, WM, WN, EPI_SILU_GATE>(a, s);
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
  if (a.M >= (int64_t(1) << 31) - 256) return fail(-2, "gemm: M must be below 2^31 - 256");
  if (a.epi == EPI_QKV_ROPE && a.rope_cols > 0 &&
      (a.seq_len <= 0 || a.seq_len >= (int64_t(1) << 31)))
    return fail(-2, "gemm: the RoPE epilogue needs 0 < seq_len < 2^31");
  if ((a.xb_out != nullptr) != (a.ss_out != nullptr) ||
      (a.xb_out && (a.epi != EPI_RESID_F32 || a.ss_np * 64 != a.N || (uintptr_t)a.xb_out % 8)))
    return fail(-2, "gemm: norm partials need EPI_RESID_F32, xb_out and ss_out, ss_np = N / 64");
  if (a.col_scale && (!a.xb_out || (uintptr_t)a.col_scale % 16))
    return fail(-2, "gemm: col_scale scales the bf16 copy (xb_out) and must be 16-byte aligned");

  if ((uintptr_t)a.A % 16 != 0 || (uintptr_t)a.Bt % 16 != 0 || a.lda % 8 != 0 || a.ldb % 8 != 0)
    return fail(-2, "gemm: A and Bt rows must be 16-byte aligned (lda, ldb % 8 == 0)");
  // Wide N (QKV, W1|W3): walk groups of 8 M-tiles so the blocks resident on
  // an XCD share A and Bt tiles in its L2; narrow N (O, W2: 3 tiles): N fastest.
  a.group_m = (a.N + 255) / 256 >= 8 ? 8 : 0;
  // N % 256 == 0: persistent 256x256 tiles over 8 waves (wave tile 128x64),
  // K tiles of 64 moved by LDS DMA through 2 stages, LDS-staged epilogue; it
  // addresses a tile's operand and output rows with 32-bit byte offsets, so
  // their reach must fit.  Otherwise (the 260-wide head, huge strides)
  // 128x128 register-staged tiles over 4 waves.
  const int64_t two31 = int64_t(1) << 31;
  const bool fits = 256 * (a.lda > a.ldb ? a.lda : a.ldb) * 2 + a.K * 2 < two31 &&
                    256 * a.ldc * 4 < two31;
  if (a.N % 256 == 0 && fits) {
    // Fewer 256x256 tiles than CUs (a single document's forward, e.g. the
    // 768-wide projections at a few thousand rows): the same kernel on 128x128
    // tiles over 2x2 waves.  The wave tile keeps its 64 columns, the K order
    // per output and the per-64-column norm partials, so every output is
    // bit-identical to the 256x256 launch's.
    const int64_t nb256 = ((a.M + 255) / 256) * (a.N / 256);
    if (nb256 < device_cus()) return run_gemm_dma_epi<128, 128, 64, 2, 2>(a, s);
    return run_gemm_dma_epi<256, 256, 64, 2, 4>(a, s);
  }
  return run_gemm<128, 128, 32, 2, 2, 2, 3>(a, s);
}

}  // namespace blt
