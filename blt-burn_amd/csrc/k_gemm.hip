// bf16 MFMA GEMM for gfx950: C = A . Bt^T with f32 accumulation and fused
// epilogues (bf16 store, f32 store, in-place f32 residual add, RoPE on the
// q/k columns of the fused QKV projection, SiLU*gate of the fused W1|W3 FFN).
//
// Tiling: a BM x BN block tile is split over WM x WN wave64s; each wave owns a
// (BM/WM) x (BN/WN) tile made of 32x32 v_mfma_f32_32x32x16_bf16 sub-tiles.
// K advances 64 at a time through two LDS stages: the next stage's global
// loads are in flight while the current stage feeds the MFMAs, one barrier
// per K step.  LDS rows are 128 B (64 bf16); the 16-byte chunk c of row r is
// stored at chunk c ^ (r & 7) so that the 32 rows read by one MFMA operand
// load spread over all banks.  Blocks are renumbered so that consecutive
// tiles (same A rows, all N tiles) land on the same XCD and share its L2.
#include "rowops.hpp"

namespace blt {

namespace {

constexpr int BK = 64;  // bf16 per LDS row (128 bytes)

__device__ inline int swz(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 3); }

template <int BM, int BN, int WM, int WN>
struct GemmCfg {
  static constexpr int NT = 64 * WM * WN;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int A_LD = BM * 8 / NT;  // 16-byte chunks per thread per stage
  static constexpr int B_LD = BN * 8 / NT;
  static constexpr int STAGE = (BM + BN) * BK;  // bf16 elements per LDS stage
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert((BM * 8) % NT == 0 && (BN * 8) % NT == 0, "loads must divide evenly");
};

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_bf16_kernel(GemmArgs p) {
  using C = GemmCfg<BM, BN, WM, WN>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * C::STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / WN, wn = wid % WN;

  // XCD-aware tile order: dispatch round-robins blocks over 8 XCDs; give each
  // XCD a contiguous run of tiles (N fastest) so A rows are reused from its L2.
  const int ntm = (int)((p.M + BM - 1) / BM), ntn = (int)((p.N + BN - 1) / BN);
  const int nb = ntm * ntn;
  const int bid = blockIdx.x;
  const int nb8 = nb & ~7;
  const int id = bid < nb8 ? (bid & 7) * (nb8 >> 3) + (bid >> 3) : bid;
  const int64_t m0 = (int64_t)(id / ntn) * BM;
  const int64_t n0 = (int64_t)(id % ntn) * BN;

  // global -> register staging
  uint4 ra[C::A_LD], rb[C::B_LD];
  auto gload = [&](int kt) {
    const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) {
      const int id2 = tid + C::NT * i, r = id2 >> 3, c = id2 & 7;
      const int64_t gr = m0 + r;
      ra[i] = gr < p.M ? *reinterpret_cast<const uint4*>(p.A + gr * p.lda + k0 + c * 8)
                       : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i) {
      const int id2 = tid + C::NT * i, r = id2 >> 3, c = id2 & 7;
      const int64_t gr = n0 + r;
      rb[i] = gr < p.N ? *reinterpret_cast<const uint4*>(p.Bt + gr * p.ldb + k0 + c * 8)
                       : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int stage) {
    uint16_t* sa = lds + stage * C::STAGE;
    uint16_t* sb = sa + BM * BK;
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) {
      const int id2 = tid + C::NT * i, r = id2 >> 3, c = id2 & 7;
      *reinterpret_cast<uint4*>(sa + swz(r, c)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i) {
      const int id2 = tid + C::NT * i, r = id2 >> 3, c = id2 & 7;
      *reinterpret_cast<uint4*>(sb + swz(r, c)) = rb[i];
    }
  };

  f32x16_t acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int KT = (int)(p.K / BK);
  gload(0);
  sstore(0);
  __syncthreads();

  const int lrow = lane & 31, lhalf = lane >> 5;
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) gload(kt + 1);
    const uint16_t* sa = lds + (kt & 1) * C::STAGE;
    const uint16_t* sb = sa + BM * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int chunk = ks * 2 + lhalf;
      bf16x8_t af[C::TM], bfr[C::TN];
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8_t*>(sa + swz(wm * C::WTM + i * 32 + lrow, chunk));
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8_t*>(sb + swz(wn * C::WTN + j * 32 + lrow, chunk));
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) sstore((kt + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue.  acc[i][j][r]: row = 8*(r/4) + 4*lhalf + r%4, col = lane%32 ----
  const int64_t row_base = m0 + wm * C::WTM;
  const int64_t col_base = n0 + wn * C::WTN;
  if (p.epi == EPI_QKV_ROPE || p.epi == EPI_SILU_GATE) {
    // pairs: sub-tile 2j holds columns c, sub-tile 2j+1 holds c + 32 of the same 64-group
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; j += 2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = row_base + i * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
          if (row >= p.M) continue;
          const int64_t col = col_base + j * 32 + lrow;  // first half of a 64-group
          const float x1 = acc[i][j][r], x2 = acc[i][j + 1][r];
          uint16_t* out = reinterpret_cast<uint16_t*>(p.C);
          if (p.epi == EPI_SILU_GATE) {
            const int64_t h = (col >> 6) * 32 + (col & 31);
            out[row * p.ldc + h] = f32_to_bf16((x1 / (1.f + __expf(-x1))) * x2);
          } else if (col < p.rope_cols) {
            const int64_t pos = row % p.seq_len;
            const float2 cs = *reinterpret_cast<const float2*>(p.rope_cs + (pos * 32 + lrow) * 2);
            out[row * p.ldc + col] = f32_to_bf16(x1 * cs.x - x2 * cs.y);
            out[row * p.ldc + col + 32] = f32_to_bf16(x1 * cs.y + x2 * cs.x);
          } else {
            out[row * p.ldc + col] = f32_to_bf16(x1);
            out[row * p.ldc + col + 32] = f32_to_bf16(x2);
          }
        }
    return;
  }
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row_base + i * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
        const int64_t col = col_base + j * 32 + lrow;
        if (row >= p.M || col >= p.N) continue;
        const float v = acc[i][j][r];
        if (p.epi == EPI_BF16) {
          reinterpret_cast<uint16_t*>(p.C)[row * p.ldc + col] = f32_to_bf16(v);
        } else if (p.epi == EPI_F32) {
          if (col < p.n_valid) reinterpret_cast<float*>(p.C)[row * p.ldc + col] = v;
        } else {  // EPI_RESID_F32
          reinterpret_cast<float*>(p.C)[row * p.ldc + col] += v;
        }
      }
}

template <int BM, int BN, int WM, int WN>
int run_gemm(const GemmArgs& a, hipStream_t s) {
  const int64_t nb = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN>), dim3((unsigned)nb), dim3(64 * WM * WN),
                     0, s, a);
  BLT_LAUNCH_CHECK("gemm_bf16_kernel");
  return 0;
}

}  // namespace

int launch_gemm(const GemmArgs& a, hipStream_t s) {
  if (a.M == 0 || a.N == 0) return 0;
  if (a.K % BK != 0) return fail(-2, "gemm: K must be a multiple of 64");
  if ((a.epi == EPI_QKV_ROPE || a.epi == EPI_SILU_GATE) && a.N % 64 != 0)
    return fail(-2, "gemm: paired epilogues need N % 64 == 0");
  // Large problems: 256x256 tiles over 8 waves (wave tile 128x64).  Narrow or
  // short problems: 128x128 tiles over 4 waves (wave tile 64x64).
  const int64_t big_tiles = ((a.M + 255) / 256) * ((a.N + 255) / 256);
  if (a.N % 256 == 0 && big_tiles >= 512) return run_gemm<256, 256, 2, 4>(a, s);
  return run_gemm<128, 128, 2, 2>(a, s);
}

}  // namespace blt
