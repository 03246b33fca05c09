// bf16 MFMA GEMM kernel template for gfx950 (included by k_gemm.hip).
//
// C = A . Bt^T with f32 accumulation and fused epilogues (bf16 store, f32
// store, in-place f32 residual add, RoPE on the q/k columns of the fused QKV
// projection, SiLU*gate of the fused W1|W3 FFN).
//
// Tiling: a BM x BN block tile is split over WM x WN wave64s; each wave owns a
// (BM/WM) x (BN/WN) tile made of 32x32 v_mfma_f32_32x32x16_bf16 sub-tiles,
// issued with the Bt fragment as the MFMA A operand so the accumulator holds
// C^T: a lane owns one output row and 4 consecutive columns per register
// group (vector stores in the epilogue).  K advances BK (32 or 64) at a time
// through two LDS stages; PF register sets keep the global loads of the next
// PF K tiles in flight (tile t staged in set t % PF), one barrier per K tile.
// LDS rows are BK bf16 wide and swizzled per 16-byte chunk (see swz) so that
// operand loads and stores are bank-conflict free.  Blocks are renumbered so
// that consecutive tiles (same A rows, all N tiles) land on the same XCD and
// share its L2.
#pragma once
#include <type_traits>

#include "rowops.hpp"

namespace blt {

namespace gemm {

// Compile-time loop: f(std::integral_constant<int, U>) for U = I .. N-1.
template <int I, int N, class F>
__device__ inline void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// 16-byte chunk c of LDS row r lives at chunk c ^ ((r / RPB) & (CH - 1)),
// where CH = BK / 8 chunks per row and RPB = 128 / BK rows per 256 bytes:
// the 16 rows read by one LDS cycle of an operand load then hit 16
// distinct 16-byte bank groups.
template <int BK>
__device__ inline int swz(int row, int chunk) {
  constexpr int CH = BK / 8, RPB = 128 / BK;
  return row * BK + ((chunk ^ ((row / RPB) & (CH - 1))) << 3);
}

template <int BM, int BN, int BK, int WM, int WN>
struct GemmCfg {
  static constexpr int NT = 64 * WM * WN;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int CH = BK / 8;                // 16-byte chunks per LDS row
  static constexpr int A_LD = BM * CH / NT;        // chunks per thread per stage
  static constexpr int B_LD = BN * CH / NT;
  static constexpr int STAGE = (BM + BN) * BK;     // bf16 elements per LDS stage
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert((BM * CH) % NT == 0 && (BN * CH) % NT == 0, "loads must divide evenly");
  static_assert(BK == 32 || BK == 64, "BK is 32 or 64");
};

template <int BM, int BN, int BK, int WM, int WN, int PF, int OCC>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(OCC)))
void gemm_bf16_kernel(GemmArgs p) {
  using C = GemmCfg<BM, BN, BK, WM, WN>;
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

  // Global source rows are clamped into range: rows past M (or N) load a
  // valid row whose results land in rows/columns that are never stored.
  const int64_t am = p.M - 1 - m0, bn = p.N - 1 - n0;

  // PF register sets: K tile t is staged in set t % PF, so the loads of
  // tiles kt+1 .. kt+PF are in flight while tile kt feeds the MFMAs.
  u32x4_t ra[PF][C::A_LD], rb[PF][C::B_LD];
  auto gload = [&](u32x4_t (&xa)[C::A_LD], u32x4_t (&xb)[C::B_LD], int kt) {
    const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) {
      const int id2 = tid + C::NT * i, r = id2 / C::CH, c = id2 % C::CH;
      const int64_t gr = m0 + (r < am ? r : am);
      xa[i] = *reinterpret_cast<const u32x4_t*>(p.A + gr * p.lda + k0 + c * 8);
    }
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i) {
      const int id2 = tid + C::NT * i, r = id2 / C::CH, c = id2 % C::CH;
      const int64_t gr = n0 + (r < bn ? r : bn);
      xb[i] = *reinterpret_cast<const u32x4_t*>(p.Bt + gr * p.ldb + k0 + c * 8);
    }
  };
  auto sstore = [&](const u32x4_t (&xa)[C::A_LD], const u32x4_t (&xb)[C::B_LD], int stage) {
    uint16_t* sa = lds + stage * C::STAGE;
    uint16_t* sb = sa + BM * BK;
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) {
      const int id2 = tid + C::NT * i, r = id2 / C::CH, c = id2 % C::CH;
      *reinterpret_cast<u32x4_t*>(sa + swz<BK>(r, c)) = xa[i];
    }
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i) {
      const int id2 = tid + C::NT * i, r = id2 / C::CH, c = id2 % C::CH;
      *reinterpret_cast<u32x4_t*>(sb + swz<BK>(r, c)) = xb[i];
    }
  };

  f32x16_t acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int lrow = lane & 31, lhalf = lane >> 5;
  auto compute = [&](int stage) {
    const uint16_t* sa = lds + stage * C::STAGE;
    const uint16_t* sb = sa + BM * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int chunk = ks * 2 + lhalf;
      bf16x8_t af[C::TM], bfr[C::TN];
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8_t*>(sa + swz<BK>(wm * C::WTM + i * 32 + lrow, chunk));
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8_t*>(sb + swz<BK>(wn * C::WTN + j * 32 + lrow, chunk));
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
  };

  const int KT = (int)(p.K / BK);
  // prologue: tile 0 -> LDS stage 0, tiles 1 .. PF in flight in their sets
  gload(ra[0], rb[0], 0);
  sstore(ra[0], rb[0], 0);
#pragma unroll
  for (int t = 1; t <= PF; ++t)
    if (t < KT) gload(ra[t % PF], rb[t % PF], t);
  __syncthreads();

  for (int kt0 = 0; kt0 < KT; kt0 += PF) {
    static_for<0, PF>([&](auto uc) {
      constexpr int nx = (decltype(uc)::value + 1) % PF;  // set holding tile kt + 1
      const int kt = kt0 + decltype(uc)::value;
      if (kt < KT) {
        compute(kt & 1);
        if (kt + 1 < KT) sstore(ra[nx], rb[nx], (kt + 1) & 1);
        if (kt + 1 + PF < KT) gload(ra[nx], rb[nx], kt + 1 + PF);
        __syncthreads();
      }
    });
  }

  // ---- epilogue.  The MFMAs computed the transposed tile (B operand = A rows),
  // so acc[i][j][r] is C[row][col] with row = m-tile i + lane % 32 and
  // col = n-tile j + 8 * (r / 4) + 4 * (lane / 32) + r % 4: each lane owns one
  // output row and 4 consecutive columns per register group, which the
  // epilogues store as one 8-byte (bf16) or 16-byte (f32) vector.
  const int64_t row_base = m0 + wm * C::WTM + lrow;
  const int64_t col_base = n0 + wn * C::WTN + 4 * lhalf;
  if (p.epi == EPI_QKV_ROPE || p.epi == EPI_SILU_GATE) {
    // pairs: sub-tile 2j holds columns c, sub-tile 2j+1 holds c + 32 of the same 64-group
    uint16_t* out = reinterpret_cast<uint16_t*>(p.C);
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      const int64_t row = row_base + i * 32;
      if (row >= p.M) continue;
      const int64_t pos = p.epi == EPI_QKV_ROPE ? row % p.seq_len : 0;
#pragma unroll
      for (int j = 0; j < C::TN; j += 2)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t col = col_base + j * 32 + 8 * g;  // first of 4 columns, first half
          float x1[4], x2[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x1[e] = acc[i][j][4 * g + e];
            x2[e] = acc[i][j + 1][4 * g + e];
          }
          if (p.epi == EPI_SILU_GATE) {
            const int64_t h = (col >> 6) * 32 + (col & 31);
            u32x2_t w;
            w.x = pack_bf16x2((x1[0] / (1.f + __expf(-x1[0]))) * x2[0],
                              (x1[1] / (1.f + __expf(-x1[1]))) * x2[1]);
            w.y = pack_bf16x2((x1[2] / (1.f + __expf(-x1[2]))) * x2[2],
                              (x1[3] / (1.f + __expf(-x1[3]))) * x2[3]);
            *reinterpret_cast<u32x2_t*>(out + row * p.ldc + h) = w;
          } else {
            float o1[4], o2[4];
            if (col < p.rope_cols) {
              const float* cs = p.rope_cs + (pos * 32 + (col & 31)) * 2;
              const f32x4_t c01 = *reinterpret_cast<const f32x4_t*>(cs);
              const f32x4_t c23 = *reinterpret_cast<const f32x4_t*>(cs + 4);
              const float cv[4] = {c01.x, c01.z, c23.x, c23.z};
              const float sv[4] = {c01.y, c01.w, c23.y, c23.w};
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                o1[e] = x1[e] * cv[e] - x2[e] * sv[e];
                o2[e] = x1[e] * sv[e] + x2[e] * cv[e];
              }
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                o1[e] = x1[e];
                o2[e] = x2[e];
              }
            }
            u32x2_t w1, w2;
            w1.x = pack_bf16x2(o1[0], o1[1]);
            w1.y = pack_bf16x2(o1[2], o1[3]);
            w2.x = pack_bf16x2(o2[0], o2[1]);
            w2.y = pack_bf16x2(o2[2], o2[3]);
            *reinterpret_cast<u32x2_t*>(out + row * p.ldc + col) = w1;
            *reinterpret_cast<u32x2_t*>(out + row * p.ldc + col + 32) = w2;
          }
        }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < C::TM; ++i) {
    const int64_t row = row_base + i * 32;
    if (row >= p.M) continue;
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t col = col_base + j * 32 + 8 * g;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e];
        if (p.epi == EPI_BF16) {
          if (col >= p.N) continue;  // N % 64 == 0 for this epilogue: 4 columns in range
          u32x2_t w;
          w.x = pack_bf16x2(v[0], v[1]);
          w.y = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<u32x2_t*>(reinterpret_cast<uint16_t*>(p.C) + row * p.ldc + col) = w;
        } else if (p.epi == EPI_F32) {
          float* o = reinterpret_cast<float*>(p.C) + row * p.ldc + col;
          if (col + 3 < p.n_valid && p.vec_ok) {
            *reinterpret_cast<f32x4_t*>(o) = f32x4_t{v[0], v[1], v[2], v[3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (col + e < p.n_valid) o[e] = v[e];
          }
        } else {  // EPI_RESID_F32: N % 64 == 0, ldc % 4 == 0
          if (col >= p.N) continue;
          f32x4_t* o = reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(p.C) + row * p.ldc + col);
          f32x4_t x = *o;
          x.x += v[0];
          x.y += v[1];
          x.z += v[2];
          x.w += v[3];
          *o = x;
        }
      }
  }
}

}  // namespace gemm
}  // namespace blt
