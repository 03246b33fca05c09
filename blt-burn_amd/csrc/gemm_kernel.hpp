// bf16 MFMA GEMM kernel template for gfx950 (included by k_gemm.hip).
//
// C = A . Bt^T with f32 accumulation and fused epilogues (bf16 store, f32
// store, in-place f32 residual add, RoPE on the q/k columns of the fused QKV
// projection, SiLU*gate of the fused W1|W3 FFN).
//
// Two kernels share the tiling and the epilogue layout:
// gemm_bf16_dma_persistent_kernel (global -> LDS by DMA, 256 x 256 x 64 tiles
// with one persistent block per CU, or 128 x 128 x 64 tiles with two for
// launches that have fewer 256 x 256 tiles than CUs; LDS-staged epilogue; every
// projection of the model, N % 256 == 0) and gemm_bf16_kernel (register-staged
// loads; any N, e.g. the 260-wide head).
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

// ---- epilogue, shared by the kernels below.  The MFMAs computed the
// transposed tile (B operand = A rows), so acc[i][j][r] is C[row][col] with
// row = m-tile i + lane % 32 and col = n-tile j + 8 * (r / 4) + 4 * (lane / 32)
// + r % 4: each lane owns one output row and 4 consecutive columns per
// register group, which the epilogues store as one 8-byte (bf16) or 16-byte
// (f32) vector.
// RoPE position of output row `row` (a token of a [B, seq_len] batch): its
// index in the row, minus its segment's start when rows are packed.
__device__ inline int64_t rope_pos(const GemmArgs& p, int64_t row) {
  // 32-bit: the launcher keeps rows (incl. a last tile's overhang) and
  // seq_len below 2^31
  const int64_t t = (int64_t)((uint32_t)row % (uint32_t)p.seq_len);
  if (!p.seg_start) return t;
  int64_t s = p.seg_start[row < p.M ? row : p.M - 1];
  s = s < 0 ? 0 : (s > t ? t : s);
  return t - s;
}

// The factor of each of this lane's accumulator rows (row0 + 32 i); 1 when
// the GEMM does not carry a norm.
template <class C>
__device__ inline void load_row_scales(const GemmArgs& p, int64_t row0, float (&rs)[C::TM]) {
#pragma unroll
  for (int i = 0; i < C::TM; ++i) {
    const int64_t r = row0 + i * 32;
    rs[i] = p.row_scale ? p.row_scale[r < p.M ? r : p.M - 1] : 1.f;
  }
}

template <class C>
__device__ inline void scale_rows(f32x16_t (&acc)[C::TM][C::TN], const float (&rs)[C::TM]) {
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] *= rs[i];
}

template <class C>
__device__ inline void epilogue(const GemmArgs& p, f32x16_t (&acc)[C::TM][C::TN], int64_t m0,
                                int64_t n0, int wm, int wn, int lrow, int lhalf,
                                const float (&rs)[C::TM]) {
  const int64_t row_base = m0 + wm * C::WTM + lrow;
  const int64_t col_base = n0 + wn * C::WTN + 4 * lhalf;
  if (p.row_scale) scale_rows<C>(acc, rs);
  if (p.epi == EPI_RESID_F32) {
    // N % 64 == 0, ldc % 4 == 0.  Lanes l and l + 32 share a row and hold its
    // 64 columns of this wave tile between them.
    static_assert(C::WTN == 64, "norm partial sums are per 64 columns");
    const int64_t wcol = n0 + wn * C::WTN;
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      const int64_t row = row_base + i * 32;
      const bool rok = row < p.M;
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t col = col_base + j * 32 + 8 * g;
          if (!rok || col >= p.N) continue;
          f32x4_t* o =
              reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(p.C) + row * p.ldc + col);
          f32x4_t x = *o;
          x.x += acc[i][j][4 * g];
          x.y += acc[i][j][4 * g + 1];
          x.z += acc[i][j][4 * g + 2];
          x.w += acc[i][j][4 * g + 3];
          *o = x;
          if (p.xb_out) {
            f32x4_t y = x;
            if (p.col_scale) y *= *reinterpret_cast<const f32x4_t*>(p.col_scale + col);
            *reinterpret_cast<u32x2_t*>(p.xb_out + row * p.ldc + col) =
                u32x2_t{pack_bf16x2(y.x, y.y), pack_bf16x2(y.z, y.w)};
            ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
          }
        }
      if (p.ss_out) {
        ss += __shfl_xor(ss, 32, 64);
        if (lhalf == 0 && rok && wcol < p.N) p.ss_out[row * p.ss_np + wcol / 64] = ss;
      }
    }
    return;
  }
  if (p.epi == EPI_QKV_ROPE || p.epi == EPI_SILU_GATE) {
    // pairs: sub-tile 2j holds columns c, sub-tile 2j+1 holds c + 32 of the same 64-group
    uint16_t* out = reinterpret_cast<uint16_t*>(p.C);
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      const int64_t row = row_base + i * 32;
      if (row >= p.M) continue;
      const int64_t pos = p.epi != EPI_QKV_ROPE ? 0 : rope_pos(p, row);
#pragma unroll
      for (int j = 0; j < C::TN; j += 2)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t col = col_base + j * 32 + 8 * g;  // first of 4 columns, first half
          // N % 64 == 0: a 64-column pair group lies wholly inside or wholly
          // past N (the last N tile of a 128-wide block can overhang by 64)
          if (col >= p.N) continue;
          float x1[4], x2[4];
          // q heads of a QKV tile: the attention scale folded in before rounding
          const float qs = col < p.q_cols ? p.q_scale : 1.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x1[e] = acc[i][j][4 * g + e] * qs;
            x2[e] = acc[i][j + 1][4 * g + e] * qs;
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
        } else {  // EPI_F32
          float* o = reinterpret_cast<float*>(p.C) + row * p.ldc + col;
          if (col + 3 < p.n_valid && p.vec_ok) {
            *reinterpret_cast<f32x4_t*>(o) = f32x4_t{v[0], v[1], v[2], v[3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (col + e < p.n_valid) o[e] = v[e];
          }
        }
      }
  }
}

// Tile order.  Dispatch round-robins blocks over the 8 XCDs; each XCD gets a
// contiguous run of tile ids, and ids walk groups of group_m M-tiles with M
// fastest inside a group, so the blocks resident on one XCD share group_m A
// row-tiles and a few Bt column-tiles in that XCD's L2 (group_m = 0: N fastest).
// Odd groups walk the column tiles from the last one down, so a group starts
// on the Bt tiles the previous group ended on.
template <int BM, int BN>
__device__ inline void tile_origin(const GemmArgs& p, int bid, int64_t& m0, int64_t& n0) {
  const int ntm = (int)((p.M + BM - 1) / BM), ntn = (int)((p.N + BN - 1) / BN);
  const int nb = ntm * ntn;
  const int nb8 = nb & ~7;
  const int id = bid < nb8 ? (bid & 7) * (nb8 >> 3) + (bid >> 3) : bid;
  int tm, tn;
  if (p.group_m > 0) {
    const int gsz = p.group_m * ntn;
    const int g = id / gsz, first = g * p.group_m;
    const int gm = ntm - first < p.group_m ? ntm - first : p.group_m;
    const int local = id - g * gsz;
    tm = first + local % gm;
    tn = local / gm;
    if (g & 1) tn = ntn - 1 - tn;
  } else {
    tm = id / ntn;
    tn = id % ntn;
  }
  m0 = (int64_t)tm * BM;
  n0 = (int64_t)tn * BN;
}

template <int BM, int BN, int BK, int WM, int WN, int PF, int OCC>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(OCC)))
void gemm_bf16_kernel(GemmArgs p) {
  using C = GemmCfg<BM, BN, BK, WM, WN>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * C::STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / WN, wn = wid % WN;

  int64_t m0, n0;
  tile_origin<BM, BN>(p, blockIdx.x, m0, n0);

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
  // prologue: tile 0 -> LDS stage 0, tiles 1 .. PF in flight in their sets;
  // the row factors are fetched under tile 0's load latency
  gload(ra[0], rb[0], 0);
  float rs[C::TM];
  load_row_scales<C>(p, m0 + wm * C::WTM + lrow, rs);
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

  epilogue<C>(p, acc, m0, n0, wm, wn, lrow, lhalf, rs);
}

// ---- LDS-staged epilogue for the DMA kernel.  After the main loop each wave
// owns its (WTM x WTN) accumulator tile; it writes the finished values of 32
// (f32 outputs) or 64 (bf16 outputs) rows at a time into a private LDS region
// in row-major order, then streams them out as whole 16-byte pieces of rows,
// so a store instruction covers a few full cache lines instead of 32 rows.
// `smem` is the block's LDS (free after the main loop); each wave uses
// its own slice of `region` bytes.
// Lanes of one wave exchange data through LDS below.  A wave's LDS operations
// execute in order, but the compiler only sees per-lane addresses: this
// fence stops it from moving LDS accesses across the phase boundary and
// waits for the wave's outstanding LDS operations.
__device__ inline void wave_lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// RoPE (cos, sin) pairs of this lane's 16 frequencies (8 g + 4 (lane / 32) + e)
// for output row `row` of the QKV projection.
__device__ inline void load_rope_cs(const GemmArgs& p, int64_t row, int lane, f32x4_t (&cs)[8]) {
  const int64_t pos = rope_pos(p, row);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float* t = p.rope_cs + (pos * 32 + 8 * g + 4 * (lane >> 5)) * 2;
    cs[2 * g] = *reinterpret_cast<const f32x4_t*>(t);
    cs[2 * g + 1] = *reinterpret_cast<const f32x4_t*>(t + 4);
  }
}

// cs0: the table pairs of the lane's first row block, loaded by the caller
// ahead of time (QKV only).
template <class C, int EPI>
__device__ inline void epilogue_lds(const GemmArgs& p, f32x16_t (&acc)[C::TM][C::TN], int64_t m0,
                                    int64_t n0, int wid, int wm, int wn, int lane,
                                    unsigned char* smem, const float (&rs)[C::TM],
                                    const f32x4_t (&cs0)[8]) {
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int64_t row0 = m0 + wm * C::WTM;  // first row of this wave's tile
  const int64_t col0 = n0 + wn * C::WTN;  // first column (pre-epilogue index)
  // the row factor (1 without a carried norm) is applied as each value is
  // staged, so the accumulators leave their registers one slab at a time
  if constexpr (EPI == EPI_RESID_F32 || EPI == EPI_F32) {
    constexpr int LD = C::WTN + 2;  // f32 row pitch (8-byte pad)
    float* buf = reinterpret_cast<float*>(smem) + wid * 32 * LD;
    constexpr int CPR = C::WTN / 4;       // 16-byte pieces per row
    constexpr int NP = 32 * CPR / 64;     // pieces per lane per 32-row slab
    constexpr bool resid = EPI == EPI_RESID_F32;
    // Rows row0 + r and columns col0 + c exist for r < mrem, c < nrem; a
    // wave tile with none stores nothing.  Addresses are uniform bases plus
    // 32-bit element offsets (the launcher bounds the tile's reach).
    if (p.M <= row0 || p.N <= col0) return;
    const int mrem = (int)(p.M - row0 < C::WTM ? p.M - row0 : C::WTM);
    const int nrem = (int)(p.N - col0 < C::WTN ? p.N - col0 : C::WTN);
    const int ldc = (int)p.ldc;
    // byte addressing (uniform base + unsigned 32-bit offset) lets the
    // loads and stores use the scalar-base addressing form
    char* cb = reinterpret_cast<char*>(reinterpret_cast<float*>(p.C) + row0 * p.ldc + col0);
    char* xbb = p.xb_out ? reinterpret_cast<char*>(p.xb_out + row0 * p.ldc + col0) : nullptr;
    // Residual pieces: slab i + 1's are loaded as soon as slab i's have been
    // added, so their latency overlaps slab i's stores and slab i + 1's
    // staging (one buffer: the 8-wave kernels have no registers for two).
    f32x4_t res[NP];
    auto load_resid = [&](int i) {
#pragma unroll
      for (int t = 0; t < NP; ++t) {
        const int q = lane + 64 * t, r = i * 32 + q / CPR, c = (q % CPR) * 4;
        const int rr = r < mrem ? r : mrem - 1;  // out-of-range pieces are not stored
        const int cc = c < nrem ? c : nrem - 4;
        res[t] = *reinterpret_cast<const f32x4_t*>(cb + (unsigned)((rr * ldc + cc) * 4));
      }
    };
    if (resid) load_resid(0);
    // the consumer's norm weight for this lane's 4 columns (the same columns
    // in every slab: 64 | 64 * t), applied to the bf16 copy only
    f32x4_t csc = f32x4_t{1.f, 1.f, 1.f, 1.f};
    if (resid && p.col_scale) {
      const int c = (lane % CPR) * 4;
      csc = *reinterpret_cast<const f32x4_t*>(p.col_scale + col0 + (c < nrem ? c : nrem - 4));
    }
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float* d = buf + lrow * LD + j * 32 + 8 * g + 4 * lhalf;
#pragma unroll
          for (int e = 0; e < 4; ++e) d[e] = acc[i][j][4 * g + e] * rs[i];
        }
      wave_lds_fence();
      f32x4_t v[NP];
#pragma unroll
      for (int t = 0; t < NP; ++t) {
        const int q = lane + 64 * t, r = q / CPR, c = q % CPR;
        const float* sp = buf + r * LD + c * 4;
        v[t] = f32x4_t{sp[0], sp[1], sp[2], sp[3]};
        if (resid) v[t] += res[t];
      }
      if (resid && i + 1 < C::TM) load_resid(i + 1);
#pragma unroll
      for (int t = 0; t < NP; ++t) {
        const int q = lane + 64 * t, r = i * 32 + q / CPR, c = (q % CPR) * 4;
        const bool ok = r < mrem && c < nrem;
        const unsigned off = (unsigned)(r * ldc + c);
        float ss = 0.f;
        if (ok) {
          float* o = reinterpret_cast<float*>(cb + off * 4u);
          if (resid) {
            *reinterpret_cast<f32x4_t*>(o) = v[t];
            if (xbb) {
              const f32x4_t y = v[t] * csc;
              *reinterpret_cast<u32x2_t*>(xbb + off * 2u) =
                  u32x2_t{pack_bf16x2(y.x, y.y), pack_bf16x2(y.z, y.w)};
              ss = v[t].x * v[t].x + v[t].y * v[t].y + v[t].z * v[t].z + v[t].w * v[t].w;
            }
          } else if (col0 + c + 3 < p.n_valid && p.vec_ok) {
            *reinterpret_cast<f32x4_t*>(o) = v[t];
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (col0 + c + e < p.n_valid) o[e] = v[t][e];
          }
        }
        if (p.ss_out) {
          // CPR is a multiple of 16: lanes 16k .. 16k + 15 hold one aligned
          // 64-column group of one row
          static_assert(C::WTN % 64 == 0, "norm partial sums are per 64 columns");
          ss = sum16(ss);
          if ((q & 15) == 0 && ok) p.ss_out[(row0 + r) * p.ss_np + (col0 + c) / 64] = ss;
        }
      }
      wave_lds_fence();
    }
  } else {
  // bf16 outputs: BF16 (WTN columns), QKV_ROPE (WTN), SILU_GATE (WTN / 2)
  constexpr bool silu = EPI == EPI_SILU_GATE;
  // rope_cols % 64 == 0: each 64-column head is rotated or not as a whole
  const bool rope = EPI == EPI_QKV_ROPE && col0 < p.rope_cols;
  constexpr int LD = C::WTN + 4;  // bf16 row pitch (8-byte pad)
  uint16_t* buf = reinterpret_cast<uint16_t*>(smem) + wid * 64 * LD;
  // RoPE (cos, sin) pairs of this lane's 16 frequencies (8 g + 4 lhalf + e)
  // for its row of tile row i, loaded one row ahead
  f32x4_t cscur[8], csnext[8];
  auto load_cs = [&](int i) { load_rope_cs(p, row0 + i * 32 + lrow, lane, csnext); };
  if (rope) {
#pragma unroll
    for (int t = 0; t < 8; ++t) csnext[t] = cs0[t];
  }
#pragma unroll
  for (int i0 = 0; i0 < C::TM; i0 += 2) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = i0 + ii;
      const int rl = ii * 32 + lrow;  // row within this 64-row slab
      if constexpr (EPI == EPI_BF16) {
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *reinterpret_cast<u32x2_t*>(buf + rl * LD + j * 32 + 8 * g + 4 * lhalf) =
                u32x2_t{pack_bf16x2(acc[i][j][4 * g] * rs[i], acc[i][j][4 * g + 1] * rs[i]),
                        pack_bf16x2(acc[i][j][4 * g + 2] * rs[i], acc[i][j][4 * g + 3] * rs[i])};
        continue;
      }
      if (rope) {
#pragma unroll
        for (int t = 0; t < 8; ++t) cscur[t] = csnext[t];
        if (i + 1 < C::TM) load_cs(i + 1);
      }
#pragma unroll
      for (int j = 0; j < C::TN; j += 2)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int cl = j * 32 + 8 * g + 4 * lhalf;  // column within the wave tile
          // q heads of a QKV tile: the attention scale rides on the row factor
          const float rq = EPI == EPI_QKV_ROPE && col0 + j * 32 < p.q_cols ? rs[i] * p.q_scale
                                                                           : rs[i];
          float x1[4], x2[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x1[e] = acc[i][j][4 * g + e] * rq;
            x2[e] = acc[i][j + 1][4 * g + e] * rq;
          }
          if (silu) {
            // silu(g) * u with g = rs a1, u = rs a2 (rs > 0, the row factor):
            //   g / (1 + e^-g) * u = (a1 a2) / ((1 + e^-g) / rs^2),
            // four VALU ops per output beside the hardware exp2 and
            // reciprocal (about 1 ulp each)
            const float k1 = rs[i] * -1.44269504f;
            const float irs2 = __builtin_amdgcn_rcpf(rs[i] * rs[i]);
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float a1 = acc[i][j][4 * g + e], a2 = acc[i][j + 1][4 * g + e];
              const float ex = __builtin_amdgcn_exp2f(a1 * k1);
              o[e] = (a1 * a2) * __builtin_amdgcn_rcpf(fmaf(ex, irs2, irs2));
            }
            *reinterpret_cast<u32x2_t*>(buf + rl * LD + (j / 2) * 32 + 8 * g + 4 * lhalf) =
                u32x2_t{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
          } else {
            float o1[4], o2[4];
            if (rope && col0 + j * 32 < p.rope_cols) {
              const f32x4_t c01 = cscur[2 * g], c23 = cscur[2 * g + 1];
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
            *reinterpret_cast<u32x2_t*>(buf + rl * LD + cl) =
                u32x2_t{pack_bf16x2(o1[0], o1[1]), pack_bf16x2(o1[2], o1[3])};
            *reinterpret_cast<u32x2_t*>(buf + rl * LD + cl + 32) =
                u32x2_t{pack_bf16x2(o2[0], o2[1]), pack_bf16x2(o2[2], o2[3])};
          }
        }
    }
    wave_lds_fence();
    // stream the 64-row slab out: OW columns per row in 16-byte pieces
    const int OW = silu ? C::WTN / 2 : C::WTN;
    const int CPR = OW / 8;
    const int64_t ocol0 = silu ? col0 / 2 : col0;
    for (int q = lane; q < 64 * CPR; q += 64) {
      const int r = q / CPR, c = q % CPR;
      const int64_t row = row0 + i0 * 32 + r;
      const uint16_t* sp = buf + r * LD + c * 8;
      const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(sp);
      const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(sp + 4);
      // non-temporal: the tile's output is not read again by this launch, and
      // the next kernel's reads of it (the whole output exceeds the MALL) come
      // from HBM either way; every CU stores its slab at the same time here
      if (row < p.M)
        __builtin_nontemporal_store(u32x4_t{lo.x, lo.y, hi.x, hi.y},
                                    reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(p.C) +
                                                               row * p.ldc + ocol0 + c * 8));
    }
    wave_lds_fence();
  }
  }
}

// Same tiling and epilogues as gemm_bf16_kernel, but K tiles move global ->
// LDS by the LDS-DMA path (no VGPR staging, no ds_write) through two LDS
// stages, and the kernel is persistent: each resident block (one per CU on
// 256 x 256 tiles, two on 128 x 128) walks the tiles v = blockIdx.x,
// blockIdx.x + gridDim.x, ...  With gridDim.x a multiple of 8
// every tile of a block has the block's XCD residue, so the tile order of
// tile_origin holds.  The K-tile stream runs on across tiles: the next tile's
// first K tile is issued together with the current tile's last one, so its
// latency hides under the last MFMAs and the epilogue, and no block launch
// sits between tiles.  Each wave issues NI 1-KB DMA chunks per K tile; a
// chunk is RPC LDS rows of BK bf16, and lane i fetches the global 16-byte
// piece that the swizzle places at row i / CH, slot i % CH.  LDS holds stage
// 0 at byte 0, a gap of half a stage, then stage 1; the epilogue stages
// through the stage that held the last K tile plus the gap, while the other
// stage receives the next tile.  Operand rows are addressed as a per-tile
// uniform base plus a per-lane 32-bit byte offset (the launcher checks that
// a tile's reach fits).  Tiles whose first column has bit 10 set take their K
// tiles from the last down (k_rev): an XCD's consecutive rounds of 4 column
// tiles then alternate direction, and a round starts on the A and Bt K tiles
// the previous round left in L2 last.  The direction depends on the column
// only, so an output's K order is the same in every launch shape.
template <int BM, int BN, int BK, int WM, int WN, int EPI>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_bf16_dma_persistent_kernel(GemmArgs p) {
  using C = GemmCfg<BM, BN, BK, WM, WN>;
  constexpr int NW = WM * WN;
  constexpr int RPC = 64 / C::CH;        // LDS rows per 1-KB chunk
  constexpr int RPB = 128 / BK;          // rows per 256 bytes (swizzle period)
  constexpr int NCH = (BM + BN) / RPC;   // 1-KB chunks per stage
  constexpr int NI = NCH / NW;           // chunks per wave per stage
  constexpr int SB = C::STAGE * 2;       // bytes per stage
  constexpr int GAP = SB / 2;
  constexpr int SOFF = SB + GAP;         // byte offset of stage 1
  static_assert(NCH % NW == 0, "DMA chunks must divide over the waves");
  static_assert((BM / RPC) % NI == 0, "a wave's chunks are all A or all Bt rows");
  static_assert(NW * 64 * (C::WTN + 4) * 2 <= SB + GAP && NW * 32 * (C::WTN + 2) * 4 <= SB + GAP,
                "staged epilogue must fit in a stage plus the gap");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * SB + GAP];

  const int ntiles = (int)(((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN));
  int v = blockIdx.x;
  if (v >= ntiles) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int wm = wid / WN, wn = wid % WN;
  const int lrow = lane & 31, lhalf = lane >> 5;
  const unsigned lds_base = (unsigned)(uintptr_t)lds;

  // This wave's NI chunks are all A rows or all Bt rows; chunk q covers LDS
  // rows rb0 + q * RPC .. + RPC - 1 of that operand.
  const bool isA = wid * NI < BM / RPC;  // uniform
  const int rb0 = (isA ? wid * NI : wid * NI - BM / RPC) * RPC;
  const unsigned lofs0 = (isA ? 0u : (unsigned)(BM * BK * 2)) + (unsigned)(rb0 * BK * 2);
  const int64_t ld = isA ? p.lda : p.ldb;
  const int64_t lim = isA ? p.M : p.N;
  const uint16_t* opnd = isA ? p.A : p.Bt;
  const uint16_t* gbase;  // operand row of this tile's first row (uniform)
  unsigned goff[NI];      // byte offset of each lane's piece from gbase
  // ln is the lane index; the tile loop passes an opaque copy after the
  // epilogue so the offsets are recomputed there rather than held in
  // registers across it
  auto set_tile = [&](int64_t m0, int64_t n0, int ln) {
    const int64_t r0 = isA ? m0 : n0;
    const int64_t last = lim - 1 - r0;  // rows past the operand read its last row
    gbase = opnd + r0 * ld;
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int r = rb0 + q * RPC + ln / C::CH;
      const int c = (ln % C::CH) ^ ((r / RPB) & (C::CH - 1));
      goff[q] = (unsigned)(((r < last ? r : last) * ld + c * 8) * 2);
    }
  };
  auto dma_tile = [&](int kt, int stage) {
    const uint16_t* kb = gbase + (int64_t)kt * BK;
    const unsigned sbase = lds_base + (unsigned)(stage * SOFF) + lofs0;
#pragma unroll
    for (int q = 0; q < NI; ++q) dma16_so(kb, goff[q], sbase + (unsigned)(q * RPC * BK * 2));
  };
  auto load_frags = [&](int stage, int ks, bf16x8_t (&af)[C::TM], bf16x8_t (&bfr)[C::TN]) {
    const uint16_t* sa = reinterpret_cast<const uint16_t*>(lds + stage * SOFF);
    const uint16_t* sb = sa + BM * BK;
    const int chunk = ks * 2 + lhalf;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
      af[i] = *reinterpret_cast<const bf16x8_t*>(sa + swz<BK>(wm * C::WTM + i * 32 + lrow, chunk));
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
      bfr[j] = *reinterpret_cast<const bf16x8_t*>(sb + swz<BK>(wn * C::WTN + j * 32 + lrow, chunk));
  };
  f32x16_t acc[C::TM][C::TN];
  f32x4_t cs0[8];  // QKV: the RoPE pairs of the epilogue's first row block
  // Fragments are double-buffered: the LDS reads of K step ks + 1 are issued
  // before the MFMAs of step ks, and scheduling barriers keep the compiler
  // from sinking them back next to their uses, so each wave has LDS reads in
  // flight while its MFMAs run.
  auto compute = [&](int stage) {
    bf16x8_t af[2][C::TM], bfr[2][C::TN];
    load_frags(stage, 0, af[0], bfr[0]);
    static_for<0, BK / 16>([&](auto kc) {
      constexpr int ks = decltype(kc)::value;
      if constexpr (ks + 1 < BK / 16) load_frags(stage, ks + 1, af[(ks + 1) & 1], bfr[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[ks & 1][j], af[ks & 1][i],
                                                              acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  const int KT = (int)(p.K / BK);
  auto k_rev = [](int64_t n) { return (int)((n >> 10) & 1); };
  int64_t m0, n0;
  tile_origin<BM, BN>(p, v, m0, n0);
  set_tile(m0, n0, lane);
  int st = 0;  // stage of the current K tile
  int rev = k_rev(n0);
  dma_tile(rev ? KT - 1 : 0, 0);
  float rs[C::TM];
  load_row_scales<C>(p, m0 + wm * C::WTM + lrow, rs);
  dma_wait_barrier<0>();
  for (;;) {
    const int vn = v + (int)gridDim.x;
    const bool more = vn < ntiles;
    int64_t m0n = 0, n0n = 0;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    for (int kt = 0; kt < KT; ++kt) {
      // stage st ^ 1 was freed by the barrier that ended K tile kt - 1: it takes
      // K tile kt + 1, or after the last one the next tile's first (one DMA
      // issue site for both keeps the loop body to one block)
      bool dma_next = true;
      int kt_next = rev ? KT - 2 - kt : kt + 1;
      if (kt + 1 == KT) {
        kt_next = 0;
        dma_next = more;
        if (more) {
          tile_origin<BM, BN>(p, vn, m0n, n0n);
          int ln = lane;
          asm volatile("" : "+v"(ln));
          set_tile(m0n, n0n, ln);
          kt_next = k_rev(n0n) ? KT - 1 : 0;
        }
      }
      if (EPI == EPI_QKV_ROPE && kt + 1 == KT && n0 + wn * C::WTN < p.rope_cols)
        load_rope_cs(p, m0 + wm * C::WTM + lrow, lane, cs0);
      if (dma_next) dma_tile(kt_next, st ^ 1);
      compute(st);
      if (kt + 1 < KT) dma_wait_barrier<0>();
      st ^= 1;
    }
    // every wave is past its last LDS read of this tile (the next tile's
    // first K tile may still be in flight)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // an opaque lane index keeps the epilogue's per-lane addressing inside
    // the loop (hoisted out, it would occupy registers through the K loop)
    int le = lane;
    asm volatile("" : "+v"(le));
    epilogue_lds<C, EPI>(p, acc, m0, n0, wid, wm, wn, le, lds + (st == 0 ? SB : 0), rs, cs0);
    if (!more) break;
    v = vn;
    m0 = m0n;
    n0 = n0n;
    rev = k_rev(n0);
    int ln = lane;
    asm volatile("" : "+v"(ln));
    set_tile(m0, n0, ln);
    // consumed by the next tile's epilogue: the latency hides under its K loop
    load_row_scales<C>(p, m0 + wm * C::WTM + lrow, rs);
    // the next tile's first K tile has landed and every wave is done with
    // the epilogue's LDS
    dma_wait_barrier<0>();
  }
}

}  // namespace gemm
}  // namespace blt
