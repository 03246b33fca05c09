// The entropy model's last step in one pass over the residual (model.rs:
// 291-313): pre-norm L2 norms, the final RMSNorm (eps after the root,
// model.rs:758-770), the output head x W_out and the softmax entropy of each
// row's logits (patcher.rs:38-63), plus the coherence n^2 / (H + 1e-6).
//
// The head's input is carried at about 16 bits of precision: each element
// a = x * w_norm (f32) is split into a_hi = bf16(a) and a_lo = bf16(a - a_hi),
// and both go through the bf16 matrix cores against the exact bf16 weights,
// so the head adds no bf16 rounding of its input (a_hi + a_lo is within
// 2^-17 of a).  The row factor 1 / (rms + eps) is applied to the f32
// accumulators, so RMSNorm(x) W = (x * w) W / (rms + eps).
//
// Tiling: 4 waves x 32 rows per block; a wave computes its 32 rows times all
// V <= 288 columns (nine 32 x 32 blocks of v_mfma_f32_32x32x16_bf16 with the
// weight fragment as the A operand, so the accumulator is the transpose: lane
// l owns row l % 32 and, in block j, columns 32 j + 8 (r / 4) + 4 (l / 32) +
// r % 4).  K advances 64 at a time.  Lane l reads the 32 f32 of its row at k
// = 64 kt + 32 (l / 32) .. + 31 (one 128-byte line), and MFMA step ks takes
// its elements 8 ks .. 8 ks + 7 as k-slots 8 (l / 32) .. + 7, so the weight
// fragment of lane l for step ks is row n, k = 64 kt + 32 (l / 32) + 8 ks ..
// + 7: chunk 4 (l / 32) + ks of the tile's 64-wide row.  The weights are packed
// once (Model::create) as [K / 64][288][64] bf16 tiles in the LDS order (16-byte
// chunks XOR-swizzled by row pair, zero rows past V), and each K tile moves
// global -> LDS by LDS DMA through two stages.  The RMSNorm weight sits in LDS.
#include <type_traits>

#include "rowops.hpp"

namespace blt {

namespace {

constexpr int HD_BK = 64;                    // K per tile
constexpr int HD_NB = 9;                     // 32-column blocks (V <= 288)
constexpr int HD_NPAD = HD_NB * 32;          // 288 packed weight rows per tile
constexpr int HD_WAVES = 4;
constexpr int HD_ROWS = 32 * HD_WAVES;       // rows per block
constexpr int HD_TILE = HD_NPAD * HD_BK * 2; // bytes per weight tile (36 KB)
constexpr int HD_CHUNKS = HD_TILE / 1024;    // 1-KB DMA chunks per tile (36)
constexpr int HD_DMAX = 1024;                // largest dim (norm weight in LDS)
static_assert(HD_CHUNKS % HD_WAVES == 0, "DMA chunks divide over the waves");

// Compile-time loop: f(std::integral_constant<int, U>) for U = I .. N-1.
template <int I, int N, class F>
__device__ inline void gemm_static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    gemm_static_for<I + 1, N>(f);
  }
}

// A wave's LDS accesses before this point complete before any after it (the
// compiler sees only per-lane addresses when lanes exchange data through LDS).
__device__ inline void wave_lds_fence_head() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// element offset of 16-byte chunk c of packed row n within a tile
__host__ __device__ inline int head_swz(int n, int c) {
  return n * HD_BK + ((c ^ ((n >> 1) & 7)) << 3);
}

// a = x * w_norm for 32 elements (8 f32x4) split into bf16 hi + lo in the
// k-slot order of the four MFMA steps; ss += x^2
// (elements 16 I0 .. 16 I0 + 15 only: steps 2 I0 and 2 I0 + 1)
template <int I0 = 0, int I1 = 8>
__device__ inline void head_split(const f32x4_t (&xv)[8], const float* wrow, float& ss,
                                  bf16x8_t (&ahi)[4], bf16x8_t (&alo)[4]) {
#pragma unroll
  for (int i = I0; i < I1; ++i) {
    const f32x4_t w4 = *reinterpret_cast<const f32x4_t*>(wrow + 4 * i);
    const f32x4_t x4 = xv[i];
    ss = fmaf(x4.x, x4.x, ss);
    ss = fmaf(x4.y, x4.y, ss);
    ss = fmaf(x4.z, x4.z, ss);
    ss = fmaf(x4.w, x4.w, ss);
    const f32x4_t a = x4 * w4;
    const uint32_t h01 = pack_bf16x2(a.x, a.y), h23 = pack_bf16x2(a.z, a.w);
    const uint32_t l01 = pack_bf16x2(a.x - __builtin_bit_cast(float, h01 << 16),
                                     a.y - __builtin_bit_cast(float, h01 & 0xffff0000u));
    const uint32_t l23 = pack_bf16x2(a.z - __builtin_bit_cast(float, h23 << 16),
                                     a.w - __builtin_bit_cast(float, h23 & 0xffff0000u));
    // elements 4 i .. 4 i + 3 of the lane's 32 = step i / 2, slots 4 (i % 2) ..
    u32x4_t* ph = reinterpret_cast<u32x4_t*>(&ahi[i >> 1]);
    u32x4_t* pl = reinterpret_cast<u32x4_t*>(&alo[i >> 1]);
    (*ph)[2 * (i & 1)] = h01;
    (*ph)[2 * (i & 1) + 1] = h23;
    (*pl)[2 * (i & 1)] = l01;
    (*pl)[2 * (i & 1) + 1] = l23;
  }
}

// One wave per SIMD (up to 512 registers): the residual streams in three K
// tiles ahead of use (x loads of tile kt + 3 go out during tile kt), and tile
// kt + 1 is converted while tile kt's MFMAs run.
constexpr int HD_XBUF = 3;

template <bool LOGITS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void head_entropy_kernel(const float* __restrict__ x, const float* __restrict__ wn,
                         const uint16_t* __restrict__ wt, int64_t M, int D, int V, float eps,
                         float* __restrict__ logits, float* __restrict__ ent,
                         float* __restrict__ norms, float* __restrict__ coh) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * HD_TILE];
  __shared__ __attribute__((aligned(16))) float wn_s[HD_DMAX];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lrow = lane & 31, h = lane >> 5;
  const int64_t row0 = (int64_t)blockIdx.x * HD_ROWS + wid * 32;  // the wave's first row
  const int64_t row = row0 + lrow;
  const int64_t rr = row < M ? row : M - 1;  // rows past M read the last row, store nothing
  const int KT = D / HD_BK;
  const unsigned lds_base = (unsigned)(uintptr_t)lds;

  // chunk c of a tile: 1 KB at byte 1024 c of the packed tile and of the LDS
  // stage (uniform base per chunk, one per-lane offset for all of them)
  const unsigned loff = (unsigned)lane * 16u;
  auto dma_tile = [&](int kt, int stage) {
    const unsigned char* src =
        reinterpret_cast<const unsigned char*>(wt) + (int64_t)kt * HD_TILE;
#pragma unroll
    for (int q = 0; q < HD_CHUNKS / HD_WAVES; ++q) {
      const unsigned c = (unsigned)(q * HD_WAVES + wid);
      dma16_so(src + c * 1024u, loff, lds_base + (unsigned)(stage * HD_TILE) + c * 1024u);
    }
  };
  // this lane's 32 elements of row rr at k = 64 kt + 32 h .. (one 128-byte line)
  const float* xrow = x + rr * D + 32 * h;
  f32x4_t xb[HD_XBUF][8];
  auto load_x = [&](int kt, f32x4_t (&dst)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dst[i] = *(reinterpret_cast<const f32x4_t*>(xrow + kt * HD_BK) + i);
  };

  for (int i = tid * 4; i < D; i += 256 * 4)
    *reinterpret_cast<f32x4_t*>(wn_s + i) = *reinterpret_cast<const f32x4_t*>(wn + i);
  // issue order (the vmcnt wait below relies on it): W tile 0, x tiles 0, 1, 2
  dma_tile(0, 0);
#pragma unroll
  for (int t = 0; t < HD_XBUF; ++t)
    if (t < KT) load_x(t, xb[t]);
  dma_wait_barrier<0>();

  f32x16_t acc[HD_NB];
#pragma unroll
  for (int j = 0; j < HD_NB; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  float ss = 0.f;
  bf16x8_t ahi[4], alo[4];
  head_split<0, 8>(xb[0], wn_s + 32 * h, ss, ahi, alo);

  // K loop, unrolled by the register-buffer period so buffer indices are static
  for (int kt0 = 0; kt0 < KT; kt0 += HD_XBUF) {
    gemm_static_for<0, HD_XBUF>([&](auto u) {
      constexpr int U = decltype(u)::value;
      const int kt = kt0 + U;
      if (kt < KT) {
        const int st = kt & 1;
        // W tile kt + 1 into the stage tile kt - 1 used, then x tile kt + 3
        // into the buffer tile kt's x has just left
        if (kt + 1 < KT) dma_tile(kt + 1, st ^ 1);
        if (kt + HD_XBUF < KT) load_x(kt + HD_XBUF, xb[U]);
        bf16x8_t nhi[4], nlo[4];
        float ss_n = 0.f;
        const bool more = kt + 1 < KT;
        const uint16_t* tile = reinterpret_cast<const uint16_t*>(lds + st * HD_TILE);
        // weight fragments double-buffered across the four steps: step ks + 1's
        // LDS reads are in flight while step ks's MFMAs run
        bf16x8_t wf[2][HD_NB];
        auto load_wf = [&](int ks, bf16x8_t (&dst)[HD_NB]) {
#pragma unroll
          for (int j = 0; j < HD_NB; ++j)
            dst[j] = *reinterpret_cast<const bf16x8_t*>(tile + head_swz(32 * j + lrow, 4 * h + ks));
        };
        load_wf(0, wf[0]);
        gemm_static_for<0, 4>([&](auto kc) {
          constexpr int ks = decltype(kc)::value;
          if constexpr (ks + 1 < 4) load_wf(ks + 1, wf[(ks + 1) & 1]);
#pragma unroll
          for (int j = 0; j < HD_NB; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks & 1][j], ahi[ks], acc[j], 0, 0, 0);
#pragma unroll
          for (int j = 0; j < HD_NB; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks & 1][j], alo[ks], acc[j], 0, 0, 0);
          // the next tile's conversion rides under the MFMAs of steps 1 and 2
          // (its x was waited for at the end of the previous tile): one MFMA,
          // then six VALU instructions, in turn
          // (unconditional, so it shares the MFMAs' scheduling region: after
          // the last tile it converts a stale buffer, and the result, whose
          // sum of squares goes to ss_n, is dropped)
          if constexpr (ks == 1 || ks == 2) {
            head_split<4 * (ks - 1), 4 * ks>(xb[(U + 1) % HD_XBUF],
                                             wn_s + (more ? kt + 1 : 0) * HD_BK + 32 * h, ss_n,
                                             nhi, nlo);
            __builtin_amdgcn_sched_group_barrier(0x100, HD_NB, 0);  // fragment reads first
            gemm_static_for<0, 2 * HD_NB>([&](auto) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
            });
          }
        });
        if (more) {
          ss += ss_n;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            ahi[q] = nhi[q];
            alo[q] = nlo[q];
          }
        }
        // W tile kt + 1 and every x load issued before it have landed (the x
        // loads of tile kt + 3, issued after it, stay in flight), and every
        // wave is done reading stage st
        if (kt + HD_XBUF < KT) dma_wait_barrier<8>();
        else dma_wait_barrier<0>();
      }
    });
  }

  // the row's sum of squares: lanes l and l ^ 32 hold its two halves
  {
    float a, b;
    swap_pair<32>(ss, a, b);
    ss = a + b;
  }
  const float nrm = sqrtf(ss);
  const float rs = 1.f / (sqrtf(ss / (float)D) + eps);
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < HD_NB; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int col = 32 * j + 8 * (r >> 2) + 4 * h + (r & 3);
      const float v = col < V ? acc[j][r] * rs : -INFINITY;
      acc[j][r] = v;
      mx = fmaxf(mx, v);
    }
  if (LOGITS) {
    // The wave's 32 rows are one contiguous run of 32 V floats: staged
    // through the (now free) weight stages 16 rows at a time, then written
    // as whole 16-byte pieces of that run.
    float* buf = reinterpret_cast<float*>(lds) + wid * 16 * HD_NPAD;
    const int64_t nrows = M - row0 < 32 ? M - row0 : 32;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if ((lrow >> 4) == half) {
        float* brow = buf + (lrow & 15) * V;
#pragma unroll
        for (int j = 0; j < HD_NB; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col = 32 * j + 8 * g + 4 * h;  // V % 4 == 0: all four or none exist
            if (col < V)
              *reinterpret_cast<f32x4_t*>(brow + col) = f32x4_t{
                  acc[j][4 * g], acc[j][4 * g + 1], acc[j][4 * g + 2], acc[j][4 * g + 3]};
          }
      }
      wave_lds_fence_head();
      const int64_t r0 = 16 * half;
      const int64_t rows = nrows - r0 < 16 ? (nrows - r0 > 0 ? nrows - r0 : 0) : 16;
      const int n4 = (int)(rows * V / 4);
      float* dst = logits + (row0 + r0) * V;
      for (int q = lane; q < n4; q += 64)
        __builtin_nontemporal_store(*reinterpret_cast<const f32x4_t*>(buf + 4 * q),
                                    reinterpret_cast<f32x4_t*>(dst) + q);
      wave_lds_fence_head();
    }
  }
  {
    float a, b;
    swap_pair<32>(mx, a, b);
    mx = fmaxf(a, b);
  }
  // H = log sum p - sum(p d) / sum p with d = x - max, p = e^d: the same
  // quantity as -sum exp(lsm) lsm (patcher.rs:38-63)
  float sp = 0.f, sd = 0.f;
#pragma unroll
  for (int j = 0; j < HD_NB; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float d = fmaxf(acc[j][r] - mx, -1e30f);
      const float pe = __expf(d);
      sp += pe;
      sd = fmaf(pe, d, sd);
    }
  {
    float a, b;
    swap_pair<32>(sp, a, b);
    sp = a + b;
    swap_pair<32>(sd, a, b);
    sd = a + b;
  }
  if (h == 0 && row < M) {
    const float H = __logf(sp) - sd * __builtin_amdgcn_rcpf(sp);
    if (ent) ent[row] = H;
    if (norms) norms[row] = nrm;
    if (coh) coh[row] = nrm * nrm / (H + 1e-6f);
  }
}

}  // namespace

int64_t head_packed_elems(int dim) { return (int64_t)(dim / HD_BK) * HD_NPAD * HD_BK; }

void pack_head_weights(const uint16_t* bt, int V, int D, uint16_t* out) {
  for (int kt = 0; kt < D / HD_BK; ++kt)
    for (int n = 0; n < HD_NPAD; ++n)
      for (int c = 0; c < HD_BK / 8; ++c)
        for (int e = 0; e < 8; ++e)
          out[(int64_t)kt * HD_NPAD * HD_BK + head_swz(n, c) + e] =
              n < V ? bt[(int64_t)n * D + kt * HD_BK + c * 8 + e] : (uint16_t)0;
}

bool head_fused_ok(int dim, int vocab) {
  return vocab > 0 && vocab <= HD_NPAD && vocab % 4 == 0 && dim > 0 && dim % HD_BK == 0 &&
         dim <= HD_DMAX;
}

int launch_head_entropy(const float* x, const float* w_norm, const uint16_t* wpacked, int64_t M,
                        int D, int V, float eps, float* logits, float* ent, float* norms,
                        float* coh, hipStream_t s) {
  if (M == 0) return 0;
  if (!head_fused_ok(D, V)) return fail(BLT_ERR_SHAPE, "head: needs V % 4 == 0, V <= 288, "
                                                       "D % 64 == 0, D <= 1024");
  if (((uintptr_t)x | (uintptr_t)w_norm | (uintptr_t)logits) % 16)
    return fail(BLT_ERR_SHAPE, "head: 16-byte aligned residual, norm weight and logits");
  const unsigned grid = ceil_div(M, HD_ROWS);
  if (logits)
    hipLaunchKernelGGL(head_entropy_kernel<true>, dim3(grid), dim3(256), 0, s, x, w_norm, wpacked,
                       M, D, V, eps, logits, ent, norms, coh);
  else
    hipLaunchKernelGGL(head_entropy_kernel<false>, dim3(grid), dim3(256), 0, s, x, w_norm,
                       wpacked, M, D, V, eps, logits, ent, norms, coh);
  BLT_LAUNCH_CHECK("head_entropy_kernel");
  return 0;
}

}  // namespace blt
