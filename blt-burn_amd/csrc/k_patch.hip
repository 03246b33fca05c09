// Patch boundaries with many blocks per row, one or two boundary rules per
// read of the entropies, optionally fused with the softmax entropy that
// produces them.
//
//   flag[t] = 1 for t < 2; else monotonic: f32(H[t] - H[t-1]) > thr,
//   global: H[t] > thr                                     (patcher.rs:80-118)
//   starts = positions of the flags in order               (patcher.rs:124-142)
//   lengths[i] = starts[i + 1] (or T) - starts[i]          (patcher.rs:144-164)
//
// A row of T positions is cut into tiles (64 positions when the pass also
// computes the entropies, 1024 when it reads them) and no block ever waits
// on another:
//   flags kernel    one block per tile: the tile's entropies (or its H
//                   values) and, per rule, its flags (the mask), one 64-bit
//                   ballot per 64 positions and the tile's (count, last start)
//                   into the workspace;
//   scan kernel     only for rows of more than kDirectTiles tiles: one wave
//                   per (row, rule) turns the tile counts into exclusive
//                   prefixes;
//   compact kernel  one wave per (tile, rule): the tile's exclusive prefix
//                   (the sum over the row's earlier tiles, read directly from
//                   the workspace, or the scan's result), then its start
//                   indices, the length of every start whose successor it
//                   holds (the last start of the tiles before it included),
//                   and on the row's last tile the count and the final length
//                   (T - last start).
// The flags kernel writes every workspace word the later kernels read, so the
// workspace needs no initialisation and keeps no state between calls; calls
// that share one must be stream-ordered.
#include "../../include/blt_hip.h"
#include "rowops.hpp"

#include <math.h>

#include <algorithm>
#include <mutex>

namespace blt {

namespace {

constexpr int kTileL = 64;              // positions per tile with the entropies
constexpr int kTileH = 1024;            // positions per tile reading entropies
constexpr int64_t kDirectTiles = 4096;  // longer rows get the scan kernel

struct RuleDev {
  int mode;
  float thr;
  int32_t* mask;
  int32_t* starts;
  int32_t* lengths;
  int32_t* count;
};

// Workspace (u64 words), per rule r and tile t of S 64-position words:
//   agg[r * ntiles + t]              (count << 32) | last start (0: none)
//   bits[(r * ntiles + t) * S + k]   flag ballot of positions 64 k .. 64 k + 63
//   pre[r * ntiles + t]              exclusive (count << 32) | last start (scan)
struct PatchKArgs {
  const float* H;       // entropies [B, T] (flags kernel reading them)
  const float* logits;  // [B * T, vocab] (fused flags kernel)
  float* H_out;         // entropies out [B, T] (fused; may be null)
  int vocab;
  int64_t B, T;
  int tile;             // positions per tile
  int S;                // tile / 64
  int tpr;              // tiles per row
  uint32_t ntiles;      // B * tpr
  int n_rules;
  RuleDev rule[2];
  uint64_t* agg;
  uint64_t* bits;
  uint64_t* pre;        // null: prefixes are summed directly
};

// (a select, not a.rule[r]: a runtime index into the argument struct would
// copy it to private memory)
__device__ inline RuleDev rule_of(const PatchKArgs& a, int r) {
  return r == 0 ? a.rule[0] : a.rule[1];
}

__device__ inline uint64_t pack_cl(uint32_t cnt, uint32_t last) {
  return ((uint64_t)cnt << 32) | last;
}

// Flags of rule r over S * 64 positions from LDS (hs[0] = H[t0 - 1],
// hs[1 + i] = H[t0 + i]), run by one wave: the mask, and the ballots and the
// (count, last start) into the workspace.
template <int S>
__device__ inline void tile_flags(const PatchKArgs& a, int r, int64_t b, int64_t t0, uint32_t tile,
                                  const float* hs, int lane) {
  const RuleDev R = rule_of(a, r);
  const int64_t T = a.T, rowoff = b * T;
  uint32_t cnt = 0, last = 0;
  uint64_t mine = 0;  // lane k keeps ballot k
#pragma unroll
  for (int k = 0; k < S; ++k) {
    const int64_t p = t0 + k * 64 + lane;
    bool f = false;
    if (p < T) {
      const float h = hs[1 + k * 64 + lane];
      if (p < 2) f = true;
      else if (R.mode == BLT_PATCH_MONOTONIC) f = (h - hs[k * 64 + lane]) > R.thr;
      else f = h > R.thr;
      if (R.mask) R.mask[rowoff + p] = f ? 1 : 0;
    }
    const uint64_t bal = __ballot(f);
    if (lane == k) mine = bal;
    if (bal) {
      cnt += (uint32_t)__popcll(bal);
      last = (uint32_t)(t0 + k * 64 + 63 - __clzll(bal));
    }
  }
  const uint64_t w = (uint64_t)r * a.ntiles + tile;
  if (lane < S) a.bits[w * S + lane] = mine;
  if (lane == 0) a.agg[w] = pack_cl(cnt, last);
}

// ---- flags from entropies: tiles of 1024 positions, 4 per thread ------------
__global__ __launch_bounds__(256) void patch_flags_kernel(PatchKArgs a) {
  __shared__ float hs[kTileH + 4];
  const uint32_t tile = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t b = tile / (uint32_t)a.tpr;
  const int64_t t0 = (int64_t)(tile % (uint32_t)a.tpr) * kTileH;
  const float* h = a.H + b * a.T;
  const int64_t p0 = t0 + 4 * tid;
  float v[4];
  if (p0 + 4 <= a.T && ((uintptr_t)(h + p0) & 15) == 0) {
    const float4 q = *reinterpret_cast<const float4*>(h + p0);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = p0 + k < a.T ? h[p0 + k] : 0.f;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) hs[1 + 4 * tid + k] = v[k];
  if (tid == 0) hs[0] = t0 > 0 ? h[t0 - 1] : 0.f;
  __syncthreads();
  if (wid < a.n_rules) tile_flags<kTileH / 64>(a, wid, b, t0, tile, hs, lane);
}

// ---- entropies and flags in one pass: tiles of 64 positions ------------------
// W waves of R = 64 / W rows: wave w computes the softmax entropies of
// positions t0 + R w .. t0 + R w + R - 1, wave 0 also t0 - 1 (the monotonic
// rule's left neighbour of the tile), with the per-row arithmetic of
// entropy_tail_kernel, so the values equal fused_entropy's.  All of a wave's
// rows are loaded before any is reduced (rows of up to 511 elements; wider
// rows go in two halves).
template <int NF, int VT>
__device__ inline float entropy_row_regs(const float (&v)[NF > 0 ? NF : 1][4],
                                         const float (&t)[VT > 0 ? VT : 1]) {
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < NF; ++c)
    m = fmaxf(m, fmaxf(fmaxf(v[c][0], v[c][1]), fmaxf(v[c][2], v[c][3])));
#pragma unroll
  for (int q = 0; q < VT; ++q) m = fmaxf(m, t[q]);
  m = wave_max(m);
  float sp = 0.f, sd = 0.f;
  auto acc = [&](float xv) {
    const float d = fmaxf(xv - m, -1e30f);
    const float pe = __expf(d);
    sp += pe;
    sd = fmaf(pe, d, sd);
  };
#pragma unroll
  for (int c = 0; c < NF; ++c)
#pragma unroll
    for (int k = 0; k < 4; ++k) acc(v[c][k]);
#pragma unroll
  for (int q = 0; q < VT; ++q) acc(t[q]);
  sp = wave_sum(sp);
  sd = wave_sum(sd);
  return __logf(sp) - sd * __builtin_amdgcn_rcpf(sp);
}

template <int NF, int VT, int G>
struct RowGroup {
  float v[G][NF > 0 ? NF : 1][4];
  float t[G][VT > 0 ? VT : 1];
  // rows rowbase + p, p = p0 .. p0 + G - 1 clamped into [0, T) (T > 0)
  __device__ inline void load(const float* __restrict__ x, int64_t rowbase, int64_t p0, int64_t T,
                              int n, int lane) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      int64_t p = p0 + g;
      p = p < 0 ? 0 : (p >= T ? T - 1 : p);
      const float* xr = x + (rowbase + p) * (int64_t)n;
#pragma unroll
      for (int c = 0; c < NF; ++c) {
        const float4 q = *reinterpret_cast<const float4*>(xr + c * 256 + lane * 4);
        v[g][c][0] = q.x; v[g][c][1] = q.y; v[g][c][2] = q.z; v[g][c][3] = q.w;
      }
#pragma unroll
      for (int q = 0; q < VT; ++q) {
        const int e = NF * 256 + q * 64 + lane;
        t[g][q] = e < n ? xr[e] : -INFINITY;
      }
    }
  }
  // out[g] = H of position p0 + g for the positions inside [0, T)
  __device__ inline void compute(int64_t p0, int64_t T, int lane, float* out) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float H = entropy_row_regs<NF, VT>(v[g], t[g]);
      const int64_t p = p0 + g;
      if (lane == 0 && p >= 0 && p < T) out[g] = H;
    }
  }
};

template <int NF, int VT, int W>
__global__ __launch_bounds__(W * 64) void entropy_flags_kernel(PatchKArgs a) {
  constexpr int R = kTileL / W;  // rows per wave
  constexpr int G = NF <= 1 ? R : (R >= 4 ? R / 2 : R);
  __shared__ float hs[kTileL + 4];
  const uint32_t tile = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t T = a.T;
  const int64_t b = tile / (uint32_t)a.tpr;
  const int64_t t0 = (int64_t)(tile % (uint32_t)a.tpr) * kTileL;
  const int64_t rowoff = b * T, p0 = t0 + wid * R;
  if (T > 0) {
    RowGroup<NF, VT, G> rg;
    RowGroup<NF, VT, 1> left;
    rg.load(a.logits, rowoff, p0, T, a.vocab, lane);
    if (wid == 0 && t0 > 0) left.load(a.logits, rowoff, t0 - 1, T, a.vocab, lane);
    rg.compute(p0, T, lane, hs + 1 + wid * R);
#pragma unroll
    for (int k = G; k < R; k += G) {
      rg.load(a.logits, rowoff, p0 + k, T, a.vocab, lane);
      rg.compute(p0 + k, T, lane, hs + 1 + wid * R + k);
    }
    if (wid == 0 && t0 > 0) left.compute(t0 - 1, T, lane, hs);
  }
  __syncthreads();
  if (wid == W - 1 && a.H_out && t0 + lane < T) a.H_out[rowoff + t0 + lane] = hs[1 + lane];
  if (wid < a.n_rules) tile_flags<1>(a, wid, b, t0, tile, hs, lane);
}

// The same pass for rows below 512 elements: 32 lanes per row
// (entropy_half_row, the arithmetic of the entropy kernel for such rows), so
// wave w takes positions t0 + 4 w .. + 3 as two pairs, and wave 0 also t0 - 1
// (its upper half computes a copy).  All of a wave's rows are loaded first.
template <int NH, int VT, int W>
__global__ __launch_bounds__(W * 64) void entropy_flags_half_kernel(PatchKArgs a) {
  constexpr int R = kTileL / W;  // rows per wave
  static_assert(R % 2 == 0, "rows go in pairs");
  constexpr int P = R / 2;
  __shared__ float hs[kTileL + 4];
  const uint32_t tile = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, l32 = lane & 31, hf = lane >> 5;
  const int64_t T = a.T;
  const int64_t b = tile / (uint32_t)a.tpr;
  const int64_t t0 = (int64_t)(tile % (uint32_t)a.tpr) * kTileL;
  const int64_t rowoff = b * T, p0 = t0 + wid * R;
  const int n = a.vocab;
  auto load = [&](int64_t p, float (&v)[NH > 0 ? NH : 1][4], float (&t)[VT > 0 ? VT : 1]) {
    p = p < 0 ? 0 : (p >= T ? T - 1 : p);
    const float* xr = a.logits + (rowoff + p) * (int64_t)n;
#pragma unroll
    for (int c = 0; c < NH; ++c) {
      const float4 q = *reinterpret_cast<const float4*>(xr + c * 128 + l32 * 4);
      v[c][0] = q.x; v[c][1] = q.y; v[c][2] = q.z; v[c][3] = q.w;
    }
#pragma unroll
    for (int q = 0; q < VT; ++q) {
      const int e = NH * 128 + q * 32 + l32;
      t[q] = e < n ? xr[e] : -INFINITY;
    }
  };
  if (T > 0) {
    float v[P][NH > 0 ? NH : 1][4], t[P][VT > 0 ? VT : 1];
    float vl[NH > 0 ? NH : 1][4], tl[VT > 0 ? VT : 1];
#pragma unroll
    for (int j = 0; j < P; ++j) load(p0 + 2 * j + hf, v[j], t[j]);
    const bool left = wid == 0 && t0 > 0;  // uniform
    if (left) load(t0 - 1, vl, tl);
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const float H = entropy_half_row<NH, VT>(v[j], t[j]);
      const int64_t p = p0 + 2 * j + hf;
      if (l32 == 0 && p < T) hs[1 + wid * R + 2 * j + hf] = H;
    }
    if (left) {
      const float H = entropy_half_row<NH, VT>(vl, tl);
      if (lane == 0) hs[0] = H;
    }
  }
  __syncthreads();
  if (wid == W - 1 && a.H_out && t0 + lane < T) a.H_out[rowoff + t0 + lane] = hs[1 + lane];
  if (wid < a.n_rules) tile_flags<1>(a, wid, b, t0, tile, hs, lane);
}

// ---- exclusive prefixes of long rows: one wave per (row, rule) ---------------
__global__ __launch_bounds__(64) void patch_scan_kernel(PatchKArgs a) {
  const int64_t b = blockIdx.x / a.n_rules;
  const int r = (int)(blockIdx.x % a.n_rules);
  const int lane = threadIdx.x;
  const uint64_t w0 = (uint64_t)r * a.ntiles + (uint64_t)b * a.tpr;
  uint32_t carry = 0, carry_last = 0;
  for (int j0 = 0; j0 < a.tpr; j0 += 64) {
    const int j = j0 + lane;
    const uint64_t g = j < a.tpr ? a.agg[w0 + j] : 0;
    const uint32_t c = (uint32_t)(g >> 32), l = (uint32_t)g;
    const int incl = wave_incl_scan((int)c);
    // the last start before tile j: the largest last start of the lower
    // lanes (they grow along the row), or the carry
    const uint64_t has = __ballot(c > 0);
    const uint64_t lower = has & ((1ull << lane) - 1ull);
    const int src = lower ? 63 - __clzll(lower) : lane;
    const uint32_t l_lo = (uint32_t)__shfl((int)l, src);
    const uint32_t before = lower ? l_lo : carry_last;
    if (j < a.tpr) a.pre[w0 + j] = pack_cl(carry + (uint32_t)incl - c, before);
    carry += (uint32_t)__builtin_amdgcn_readlane(incl, 63);
    if (has) carry_last = (uint32_t)__builtin_amdgcn_readlane((int)l, 63 - __clzll(has));
  }
}

// ---- starts and lengths: one wave per (tile, rule) ---------------------------
template <int S>
__global__ __launch_bounds__(256) void patch_compact_kernel(PatchKArgs a) {
  const uint64_t q = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= (uint64_t)a.ntiles * a.n_rules) return;
  const uint32_t tile = (uint32_t)(q / a.n_rules);
  const int r = (int)(q % a.n_rules);
  const int lane = threadIdx.x & 63;
  const RuleDev R = rule_of(a, r);
  const int64_t T = a.T;
  const int64_t b = tile / (uint32_t)a.tpr;
  const int j = (int)(tile % (uint32_t)a.tpr);
  const int64_t t0 = (int64_t)j * a.tile, rowoff = b * T;
  const uint64_t w = (uint64_t)r * a.ntiles + tile;
  const uint64_t mine = lane < S ? a.bits[w * S + lane] : 0;
  // exclusive prefix: (count, last start) of the row's tiles before this one
  uint32_t ex_cnt = 0, ex_last = 0;
  if (a.pre) {
    const uint64_t p = a.pre[w];
    ex_cnt = (uint32_t)(p >> 32);
    ex_last = (uint32_t)p;
  } else if (j > 0) {
    // counts summed; the last start before the tile is the largest of the
    // earlier tiles' last starts (they grow along the row; 0 when none)
    uint32_t c = 0, l = 0;
    for (int i = lane; i < j; i += 64) {
      const uint64_t g = a.agg[w - (uint64_t)(j - i)];
      c += (uint32_t)(g >> 32);
      l = max(l, (uint32_t)g);
    }
    ex_cnt = (uint32_t)__builtin_amdgcn_readlane(wave_incl_scan((int)c), 63);
    ex_last = (uint32_t)wave_max_i32((int)l);
  }
  uint32_t idx = ex_cnt;
  int64_t prev = ex_last;  // the last start before this point (valid when idx > 0)
  const uint64_t below_me = (1ull << lane) - 1ull;
#pragma unroll
  for (int k = 0; k < S; ++k) {
    const uint64_t m =
        (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)mine, k) |
        ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(mine >> 32), k) << 32);
    if (!m) continue;
    const int64_t base = t0 + k * 64;
    if ((m >> lane) & 1ull) {
      const uint64_t below = m & below_me;
      const uint32_t g = idx + (uint32_t)__popcll(below);
      const int64_t pos = base + lane;
      if (R.starts) R.starts[rowoff + g] = (int32_t)pos;
      if (R.lengths && g > 0) {
        const int64_t pp = below ? base + 63 - __clzll(below) : prev;
        R.lengths[rowoff + g - 1] = (int32_t)(pos - pp);
      }
    }
    idx += (uint32_t)__popcll(m);
    prev = base + 63 - __clzll(m);
  }
  if (j == a.tpr - 1 && lane == 0) {
    if (R.count) R.count[b] = (int32_t)idx;
    if (R.lengths && idx > 0) R.lengths[rowoff + idx - 1] = (int32_t)(T - prev);
  }
}

int64_t tiles_per_row(int64_t T, int tile) { return T <= 0 ? 1 : (T + tile - 1) / tile; }

int64_t ws_words(int64_t B, int64_t T, int n_rules, int tile) {
  const int64_t nt = B * tiles_per_row(T, tile);
  return (int64_t)n_rules * nt * (2 + tile / 64);
}

int fill_rules(PatchKArgs& k, int n_rules, const blt_patch_rule* rules) {
  if (n_rules < 1 || n_rules > 2)
    return fail(BLT_ERR_INVALID, "patch rules: n_rules must be 1 or 2");
  if (!rules) return fail(BLT_ERR_INVALID, "patch rules: null rules");
  k.n_rules = n_rules;
  for (int r = 0; r < n_rules; ++r) {
    const blt_patch_rule& R = rules[r];
    if (R.mode != BLT_PATCH_MONOTONIC && R.mode != BLT_PATCH_GLOBAL)
      return fail(BLT_ERR_INVALID, "patch rules: bad mode");
    if (R.lengths && !R.starts)
      return fail(BLT_ERR_INVALID, "patch rules: lengths needs the starts buffer");
    k.rule[r] = RuleDev{R.mode, R.threshold, R.mask, R.starts, R.lengths, R.count};
  }
  return 0;
}

// Shared argument checks and the workspace carve-up of both flag passes.
int prepare(const float* H, const float* logits, float* H_out, int vocab, int64_t B, int64_t T,
            int n_rules, const blt_patch_rule* rules, void* ws, int64_t ws_bytes, int tile,
            PatchKArgs& k) {
  if (B < 0 || T < 0) return fail(BLT_ERR_SHAPE, "patch rules: negative shape");
  if (T > 0x7fffffff) return fail(BLT_ERR_SHAPE, "patch rules: T must fit int32");
  int rc;
  if ((rc = fill_rules(k, n_rules, rules))) return rc;
  const int64_t tpr = tiles_per_row(T, tile);
  if (B * tpr > 0x7fffffff / 4) return fail(BLT_ERR_SHAPE, "patch rules: too many tiles");
  if (B > 0 && !ws) return fail(BLT_ERR_INVALID, "patch rules: null workspace");
  if (ws_bytes < 8 * ws_words(B, T, n_rules, tile))
    return fail(BLT_ERR_SHAPE, "patch rules: workspace smaller than blt_patch_workspace_bytes");
  if ((uintptr_t)ws % 16)
    return fail(BLT_ERR_INVALID, "patch rules: workspace not 16-byte aligned");
  k.H = H;
  k.logits = logits;
  k.H_out = H_out;
  k.vocab = vocab;
  k.B = B;
  k.T = T;
  k.tile = tile;
  k.S = tile / 64;
  k.tpr = (int)tpr;
  k.ntiles = (uint32_t)(B * tpr);
  uint64_t* w = reinterpret_cast<uint64_t*>(ws);
  const uint64_t nw = (uint64_t)n_rules * k.ntiles;
  k.agg = w;
  k.bits = w + nw;
  k.pre = tpr > kDirectTiles ? w + nw + nw * k.S : nullptr;
  return 0;
}

// scan (long rows) and compaction after a flags kernel
int launch_tail(const PatchKArgs& k, hipStream_t s) {
  if (k.pre) {
    hipLaunchKernelGGL(patch_scan_kernel, dim3((unsigned)(k.B * k.n_rules)), dim3(64), 0, s, k);
    BLT_LAUNCH_CHECK("patch_scan_kernel");
  }
  const unsigned grid = ceil_div((int64_t)k.ntiles * k.n_rules, 4);
  if (k.S == 1)
    hipLaunchKernelGGL(patch_compact_kernel<1>, dim3(grid), dim3(256), 0, s, k);
  else
    hipLaunchKernelGGL(patch_compact_kernel<kTileH / 64>, dim3(grid), dim3(256), 0, s, k);
  BLT_LAUNCH_CHECK("patch_compact_kernel");
  return 0;
}

// waves per block of the fused flags kernel, kTileL / kFusedWaves rows each
// (config 1's [4, 8192, 260]: 16 waves of 4 rows 10.0 us, 8 of 8 rows 11.0 us)
constexpr int kFusedWaves = 16;

template <int NF, int VT>
int launch_fused(const PatchKArgs& k, hipStream_t s) {
  hipLaunchKernelGGL((entropy_flags_kernel<NF, VT, kFusedWaves>), dim3(k.ntiles),
                     dim3(kFusedWaves * 64), 0, s, k);
  BLT_LAUNCH_CHECK("entropy_flags_kernel");
  return launch_tail(k, s);
}

template <int NH, int VT>
int launch_fused_half(const PatchKArgs& k, hipStream_t s) {
  hipLaunchKernelGGL((entropy_flags_half_kernel<NH, VT, kFusedWaves>), dim3(k.ntiles),
                     dim3(kFusedWaves * 64), 0, s, k);
  BLT_LAUNCH_CHECK("entropy_flags_half_kernel");
  return launch_tail(k, s);
}

// The register layout of the entropy kernel for this row width: below 512
// elements the half-wave rows (NH, VT) of entropy_half_kernel (variants
// 100 + NH * 8 + VT), else (NF, VT) of entropy_tail_kernel; -1 when the width
// has none (the caller then runs entropy and the H pass apart)
int fused_variant(int n) {
  if (n <= 0 || n % 4 || n >= 1280) return -1;
  if (n < 512) return 100 + (n / 128) * 8 + (n % 128 + 31) / 32;
  return (n / 256) * 8 + (n % 256 + 63) / 64;
}
int launch_fused_variant(int v, const PatchKArgs& k, hipStream_t s) {
  switch (v) {
#define BLT_FH(NH, VT) case 100 + NH * 8 + VT: return launch_fused_half<NH, VT>(k, s);
    BLT_FH(0, 1) BLT_FH(0, 2) BLT_FH(0, 3) BLT_FH(0, 4)
    BLT_FH(1, 0) BLT_FH(1, 1) BLT_FH(1, 2) BLT_FH(1, 3) BLT_FH(1, 4)
    BLT_FH(2, 0) BLT_FH(2, 1) BLT_FH(2, 2) BLT_FH(2, 3) BLT_FH(2, 4)
    BLT_FH(3, 0) BLT_FH(3, 1) BLT_FH(3, 2) BLT_FH(3, 3) BLT_FH(3, 4)
#undef BLT_FH
#define BLT_FV(NF, VT) case NF * 8 + VT: return launch_fused<NF, VT>(k, s);
    BLT_FV(0, 1) BLT_FV(0, 2) BLT_FV(0, 3) BLT_FV(0, 4)
    BLT_FV(1, 0) BLT_FV(1, 1) BLT_FV(1, 2) BLT_FV(1, 3) BLT_FV(1, 4)
    BLT_FV(2, 0) BLT_FV(2, 1) BLT_FV(2, 2) BLT_FV(2, 3) BLT_FV(2, 4)
    BLT_FV(3, 0) BLT_FV(3, 1) BLT_FV(3, 2) BLT_FV(3, 3) BLT_FV(3, 4)
    BLT_FV(4, 0) BLT_FV(4, 1) BLT_FV(4, 2) BLT_FV(4, 3) BLT_FV(4, 4)
#undef BLT_FV
  }
  return fail(BLT_ERR_SHAPE, "entropy_patch: no fused variant for this vocab");
}

}  // namespace

int64_t patch_workspace_bytes(int64_t B, int64_t T, int n_rules) {
  if (B < 0 || T < 0 || n_rules < 1 || n_rules > 2) return 0;
  return 8 * std::max(ws_words(B, T, n_rules, kTileL), ws_words(B, T, n_rules, kTileH));
}

int launch_patch_rules(const float* H, int64_t B, int64_t T, int n_rules,
                       const blt_patch_rule* rules, void* ws, int64_t ws_bytes, hipStream_t s) {
  PatchKArgs k{};
  int rc;
  if ((rc = prepare(H, nullptr, nullptr, 0, B, T, n_rules, rules, ws, ws_bytes, kTileH, k)))
    return rc;
  if (B == 0) return 0;
  if (T > 0 && !H) return fail(BLT_ERR_INVALID, "patch rules: null entropies");
  hipLaunchKernelGGL(patch_flags_kernel, dim3(k.ntiles), dim3(256), 0, s, k);
  BLT_LAUNCH_CHECK("patch_flags_kernel");
  return launch_tail(k, s);
}

int launch_entropy_patch(const float* logits, int64_t B, int64_t T, int vocab, float* H_out,
                         int n_rules, const blt_patch_rule* rules, void* ws, int64_t ws_bytes,
                         hipStream_t s) {
  if (vocab <= 0) return fail(BLT_ERR_SHAPE, "entropy_patch: vocab must be > 0");
  const int v = fused_variant(vocab);
  if (v < 0 || (B * T > 0 && (uintptr_t)logits % 16)) {
    // no register layout for this row width (or unaligned rows): the entropy
    // kernel writes H_out, then the H pass reads it
    if (!H_out && B * T > 0)
      return fail(BLT_ERR_INVALID, "entropy_patch: this vocab needs the entropies out");
    PatchKArgs chk{};
    int rc;
    if ((rc = prepare(H_out, logits, H_out, vocab, B, T, n_rules, rules, ws, ws_bytes, kTileH,
                      chk)))
      return rc;
    if (B * T > 0 && (rc = launch_entropy_f32(logits, H_out, B * T, vocab, s))) return rc;
    return launch_patch_rules(H_out, B, T, n_rules, rules, ws, ws_bytes, s);
  }
  PatchKArgs k{};
  int rc;
  if ((rc = prepare(nullptr, logits, H_out, vocab, B, T, n_rules, rules, ws, ws_bytes, kTileL,
                    k)))
    return rc;
  if (B == 0) return 0;
  if (T > 0 && !logits) return fail(BLT_ERR_INVALID, "entropy_patch: null logits");
  return launch_fused_variant(v, k, s);
}

// ---- the H pass with its workspace in a static device array ----------------
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops): the per-tile counts and flag words live in
// `scratch`, kScratchBytes on each device, instead of a caller workspace.
// Nothing in it needs clearing (each call's flags kernel writes every word
// the later kernels read), but every call on a device shares that device's
// copy, so calls that overlap on one device race.
constexpr int64_t kScratchBytes = 1 << 20;
static __device__ __align__(256) uint64_t scratch[kScratchBytes / 8];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // scratch's device address, per device
}  // namespace

// The current device's copy of `scratch`, looked up with hipGetSymbolAddress
// on the first call on that device (the array's host-side name is not a
// device address).
static int scratch_address(void** out) {
  int dev = 0;
  BLT_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(BLT_ERR_NODEV, "patch scratch: device index");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    BLT_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(BLT_ERR_HIP, "patch scratch: no device address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

int launch_patch_rules_noalloc(const float* H, int64_t B, int64_t T, int n_rules,
                               const blt_patch_rule* rules, hipStream_t s) {
  if (B < 0 || T < 0) return fail(BLT_ERR_SHAPE, "patch rules (no-alloc): negative shape");
  if (n_rules < 1 || n_rules > 2)
    return fail(BLT_ERR_INVALID, "patch rules (no-alloc): n_rules must be 1 or 2");
  if (T > 0x7fffffff) return fail(BLT_ERR_SHAPE, "patch rules (no-alloc): T must fit int32");
  if (8 * ws_words(B, T, n_rules, kTileH) > kScratchBytes)
    return fail(BLT_ERR_SHAPE, "patch rules (no-alloc): n_rules * B * ceil(T / 1024) must be at "
                               "most 7281 (1 MiB of static scratch)");
  if (B == 0) {
    PatchKArgs k{};
    return fill_rules(k, n_rules, rules);
  }
  void* ws = nullptr;
  int rc;
  if ((rc = scratch_address(&ws))) return rc;
  return launch_patch_rules(H, B, T, n_rules, rules, ws, kScratchBytes, s);
}

}  // namespace blt
