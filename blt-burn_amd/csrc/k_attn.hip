// Causal (optionally sliding-window) attention for gfx950, head_dim 64, bf16
// operands on MFMA, f32 online softmax.
//
// One block = 4 wave64s = 128 or 256 queries of one (batch, head); K/V
// advance in 64-key tiles through three LDS stages shared by the four waves
// (moved by LDS DMA, two tiles in flight while one is consumed).
//
// Each wave computes S^T = K . Q^T (v_mfma_f32_32x32x16_bf16, keys as rows,
// its 32 queries as columns), so a lane owns one query column and 32 of the
// 64 scores of that query: the running max and sum need one cross-lane step
// (lane ^ 32) instead of a 32-lane reduction.  The output is accumulated
// transposed, O^T = V^T . P^T, which keeps the per-query rescale factor in
// the lane that owns the query.  The P^T registers feed the MFMA B operand
// directly (no LDS round trip).  The softmax is VALU-bound, so the rest of
// the per-score work is kept off the VALU: q arrives scaled by log2(e) /
// sqrt(64), and the first MFMA of each S^T chain starts from -m (the running
// max) instead of zero, so S^T comes out of the matrix core ready for exp2;
// the row sums of P are v_dot2_f32_bf16 over the same packed bf16 P the
// numerator uses (16 per tile, a lane's half of the keys; the two halves
// meet at the end).  V stays row-major in LDS; the V^T operand is read with
// ds_read_b64_tr_b16, whose 16-lane transpose hands each lane 4 consecutive
// keys of one head-dim column.
//
// Masking follows the reference's additive causal mask (model.rs:153-165:
// key j visible to query i iff j <= i), extended with a window W > 0
// (also j > i - W).  Tiles entirely outside a wave's visible band are
// skipped; fully visible tiles skip the per-element mask.
#include "rowops.hpp"

namespace blt {

namespace {

constexpr int BKV = 64;     // keys per tile
constexpr int D = 64;       // head dim
constexpr int V_LD = 72;    // V row pitch in bf16 (144 B): conflict-free transposing reads
constexpr int K_TILE = BKV * D;
constexpr int V_TILE = BKV * V_LD;
constexpr int STAGE = K_TILE + V_TILE;
constexpr int NSTAGE = 3;   // LDS stages: one tile consumed, two in flight

typedef short s16x4_t __attribute__((ext_vector_type(4)));
#define LDS_PTR(p) ((__attribute__((address_space(3))) s16x4_t*)(p))

// K rows are 128 B: chunk c of key row k is stored at c ^ ((k >> 1) & 7), so the
// 16 rows one LDS cycle serves for an operand load fall in 16 distinct banks.
__device__ inline int kswz(int key, int chunk) { return key * D + ((chunk ^ ((key >> 1) & 7)) << 3); }

// NQ 32-query column blocks per wave (QPW = 32 * NQ queries); each K and V^T
// fragment read from LDS feeds NQ MFMAs.  Block = 4 waves = 4 * QPW queries.
template <int NQ>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs p) {
  constexpr int QPW = 32 * NQ;
  constexpr int BQ = 4 * QPW;
  __shared__ __attribute__((aligned(1024))) uint16_t lds[NSTAGE * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int lrow = lane & 31, lhalf = lane >> 5;

  // XCD-aware order: consecutive query blocks of one (b, h) share K/V, so
  // keep them on one XCD (dispatch places block i on XCD i % 8).
  const int T = (int)p.T;
  const int nqb = (T + BQ - 1) / BQ;
  // 32-bit block decode: the launcher keeps the grid below 2^31 blocks
  const uint32_t nb = (uint32_t)nqb * (uint32_t)p.H * (uint32_t)p.B;
  const uint32_t bid = blockIdx.x;
  const uint32_t nb8 = nb & ~7u;
  const uint32_t id = bid < nb8 ? (bid & 7) * (nb8 >> 3) + (bid >> 3) : bid;
  const int qb = nqb - 1 - (int)(id % (uint32_t)nqb);  // longest causal rows first
  const uint32_t bh = id / (uint32_t)nqb;
  const int64_t h = bh % (uint32_t)p.H, b = bh / (uint32_t)p.H;

  const int q0 = qb * BQ;
  const int qw = q0 + wid * QPW;  // this wave's first query
  const int window = p.causal ? p.window : 0;

  // segment starts (packed rows): clamped to [0, t] so any input stays in range
  const int32_t* seg = p.seg_start ? p.seg_start + b * T : nullptr;
  auto seg_at = [&](int t) -> int {
    if (!seg) return 0;
    const int tc = t < T - 1 ? t : T - 1;
    const int v = seg[tc];
    return v < 0 ? 0 : (v > tc ? tc : v);
  };

  // block key range
  int lo = 0, hi = T - 1;
  if (p.causal) {
    hi = q0 + BQ - 1 < T - 1 ? q0 + BQ - 1 : T - 1;
    if (window > 0) lo = q0 - window + 1 > 0 ? q0 - window + 1 : 0;
    const int sl = seg_at(q0);  // smallest segment start of the block's queries
    lo = lo > sl ? lo : sl;
  }
  const int t_begin = lo / BKV, t_end = hi / BKV;
  // wave key range
  int wlo = 0, whi = T - 1, wseg_hi = 0;
  if (p.causal) {
    whi = qw + QPW - 1 < T - 1 ? qw + QPW - 1 : T - 1;
    if (window > 0) wlo = qw - window + 1 > 0 ? qw - window + 1 : 0;
    const int sl = seg_at(qw);
    wlo = wlo > sl ? wlo : sl;
    wseg_hi = seg_at(qw + QPW - 1);  // largest segment start of the wave's queries
  }
  const bool wave_active = qw < T;
  const int wt_begin = wlo / BKV, wt_end = whi / BKV;

  const uint16_t* kbase = p.k + b * p.sb_k + h * p.sh_k;
  const uint16_t* vbase = p.v + b * p.sb_v + h * p.sh_v;

  // Q fragments (B operand of S^T = K . Q^T): query qw + 32*qq + lrow,
  // d = 16*ks + 8*lhalf .. +8
  bf16x8_t qf[NQ][4];
#pragma unroll
  for (int qq = 0; qq < NQ; ++qq) {
    const int qi = qw + 32 * qq + lrow;
    const int qc = qi < T ? qi : T - 1;  // rows past T load a valid row, never stored
    const uint16_t* qrow = p.q + b * p.sb_q + h * p.sh_q + (int64_t)qc * p.st_q;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[qq][ks] = __builtin_bit_cast(
          bf16x8_t, *reinterpret_cast<const u32x4_t*>(qrow + ks * 16 + lhalf * 8));
    // q' = q log2(e) / sqrt(64) (unless the producer scaled it), rotated first
    // when a RoPE table is given, rounded to bf16 once
    const float qs = p.q_prescaled ? 1.f : kAttnQScale;
    if (p.q_rope_cs) {
      // fragments ks and ks + 2 hold the pair halves m and m + 32 of the same
      // 8 frequencies m = 16 ks + 8 lhalf + e: rotate them in registers
      const float* cs = p.q_rope_cs + (int64_t)qc * 64;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const f32x4_t* t = reinterpret_cast<const f32x4_t*>(cs + (16 * ks + 8 * lhalf) * 2);
        const u32x4_t lo = __builtin_bit_cast(u32x4_t, qf[qq][ks]);
        const u32x4_t hi = __builtin_bit_cast(u32x4_t, qf[qq][ks + 2]);
        u32x4_t o1, o2;
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {  // pairs 2 q2, 2 q2 + 1
          const f32x4_t c = t[q2] * qs;   // (cos, sin) of pair 2 q2, then of pair 2 q2 + 1
          const float a0 = bf16_to_f32((uint16_t)(lo[q2] & 0xffff));
          const float a1 = bf16_to_f32((uint16_t)(lo[q2] >> 16));
          const float b0 = bf16_to_f32((uint16_t)(hi[q2] & 0xffff));
          const float b1 = bf16_to_f32((uint16_t)(hi[q2] >> 16));
          o1[q2] = pack_bf16x2(a0 * c.x - b0 * c.y, a1 * c.z - b1 * c.w);
          o2[q2] = pack_bf16x2(a0 * c.y + b0 * c.x, a1 * c.w + b1 * c.z);
        }
        qf[qq][ks] = __builtin_bit_cast(bf16x8_t, o1);
        qf[qq][ks + 2] = __builtin_bit_cast(bf16x8_t, o2);
      }
    } else if (!p.q_prescaled) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        u32x4_t w = __builtin_bit_cast(u32x4_t, qf[qq][ks]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = pack_bf16x2(bf16_to_f32((uint16_t)(w[e] & 0xffff)) * qs,
                             bf16_to_f32((uint16_t)(w[e] >> 16)) * qs);
        qf[qq][ks] = __builtin_bit_cast(bf16x8_t, w);
      }
    }
  }
  // each query's segment start (lower key bound of packed rows)
  int qseg[NQ];
#pragma unroll
  for (int qq = 0; qq < NQ; ++qq) qseg[qq] = p.causal ? seg_at(qw + 32 * qq + lrow) : 0;
  // Consume the Q and segment loads here, before the K/V DMA is issued: the
  // compiler counts only its own loads, so a first use inside the tile loop
  // would wait for every DMA in flight as well.
#pragma unroll
  for (int qq = 0; qq < NQ; ++qq) {
    asm volatile("" ::"v"(qseg[qq]));
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) asm volatile("" ::"v"(qf[qq][ks]));
  }

  // K/V tiles move global -> LDS by DMA (global_load_lds_dwordx4: 1 KB per
  // instruction, lane i's 16 bytes land at slot i) through NSTAGE LDS stages,
  // two tiles in flight while one is consumed.  A tile is NKOP K ops (8 keys
  // x 8 chunks each, chunks in the kswz order) and NVOP V ops (64 rows of 9
  // slots: 8 chunks and a pad slot that fetches chunk 0 again, for the
  // 144-byte pitch); op o is issued by wave o % 4, so a wave issues ops
  // q = 0, 1 (K) and 2, 3 (and wave 0 also 4) (V).  Each lane keeps the byte
  // offset of its piece from the tile's first row; in the last, partial tile
  // keys past T load key T-1 (masked: a key >= T is never visible).
  constexpr int NKOP = K_TILE * 2 / 1024, NVOP = V_TILE * 2 / 1024, NOP = NKOP + NVOP;
  constexpr int QMAX = (NOP + 3) / 4;
  static_assert(NKOP == 8 && NVOP == 9 && QMAX == 5, "op split assumed below");
  const int wid_u = __builtin_amdgcn_readfirstlane(wid);
  const int nops = (NOP - wid_u + 3) / 4;  // 5 for wave 0, 4 for the others
  const unsigned lds_base = (unsigned)(uintptr_t)lds;
  uint32_t goff[QMAX];
  int gkey[QMAX];
#pragma unroll
  for (int q = 0; q < QMAX; ++q) {
    const int o = wid_u + 4 * q;
    if (q < 2) {
      const int slot = o * 64 + lane, key = slot >> 3;
      const int c = (slot & 7) ^ ((key >> 1) & 7);
      gkey[q] = key;
      goff[q] = ((uint32_t)key * (uint32_t)p.st_k + c * 8) * 2;  // < 2^32 (launcher)
    } else {
      const int slot = (o - NKOP) * 64 + lane, key = slot / 9, c9 = slot % 9;
      const int c = c9 < 8 ? c9 : 0;
      gkey[q] = key < BKV ? key : BKV - 1;
      goff[q] = ((uint32_t)gkey[q] * (uint32_t)p.st_v + c * 8) * 2;
    }
  }
  auto issue = [&](int t, int stage) {
    const int64_t k0 = (int64_t)t * BKV;
    const char* kb0 = reinterpret_cast<const char*>(kbase + k0 * p.st_k);
    const char* vb0 = reinterpret_cast<const char*>(vbase + k0 * p.st_v);
    const unsigned sb = lds_base + (unsigned)(stage * STAGE * 2);
    auto op = [&](int q, uint32_t off) {
      const int o = wid_u + 4 * q;
      const unsigned la = q < 2 ? sb + (unsigned)(o * 1024)
                                : sb + (unsigned)(K_TILE * 2 + (o - NKOP) * 1024);
      dma16_so(q < 2 ? kb0 : vb0, off, la);
    };
    // a whole tile (uniform, 32-bit: T < 2^30) takes the precomputed offsets
    // as they are; only the row's last, partial tile steps rows back
    if (t * BKV + BKV <= T) {
#pragma unroll
      for (int q = 0; q < QMAX; ++q) {
        if (q == QMAX - 1 && nops < QMAX) break;
        op(q, goff[q]);
      }
    } else {
#pragma unroll
      for (int q = 0; q < QMAX; ++q) {
        if (q == QMAX - 1 && nops < QMAX) break;
        const int64_t back = k0 + gkey[q] < T ? 0 : k0 + gkey[q] - (T - 1);  // rows to step back
        op(q, goff[q] - (uint32_t)(back * (q < 2 ? p.st_k : p.st_v) * 2));
      }
    }
  };

  // Transposing V reads: in each 16-lane group, source lane s points at
  // V[k0 + 4*lhalf + s/4][dcol + 4*(s%4)], so lane t of the group receives
  // V[k0 + 4*lhalf + e][dcol + t], e = 0..3 (t = lane % 16, dcol covers 16
  // columns per group: 16 * ((lane >> 4) & 1) within the 32-column half).
  const int s16 = lane & 15;
  const int vt_lane = (4 * lhalf + (s16 >> 2)) * V_LD + 16 * ((lane >> 4) & 1) + 4 * (s16 & 3);

  f32x16_t o[NQ][2];
  // m: the running max (log2 domain) of this lane's query, -inf until its
  // first visible key; mu: the offset the scores are taken relative to (m, or
  // 0 while m is -inf), held as -mu in every element of negm, the C operand
  // of each S^T chain's first MFMA; l: this lane's half of the row sum of P
  float m[NQ], mu[NQ], l[NQ];
  f32x16_t negm[NQ];
#pragma unroll
  for (int qq = 0; qq < NQ; ++qq) {
    m[qq] = -INFINITY;
    mu[qq] = 0.f;
    l[qq] = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) negm[qq][r] = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[qq][j][r] = 0.f;
  }
  const bf16x2_t ones2 = {(__bf16)1.0f, (__bf16)1.0f};

  issue(t_begin, 0);
  if (t_begin + 1 <= t_end) issue(t_begin + 1, 1);
  int stage = 0;  // stage of tile t
  for (int t = t_begin; t <= t_end; ++t) {
    // tile t has landed (only tile t + 1's ops may still be in flight) and
    // every wave is past tile t - 1, whose stage now takes tile t + 2
    if (t + 1 <= t_end) {
      if (nops == 5) dma_wait_barrier<5>(); else dma_wait_barrier<4>();
    } else {
      dma_wait_barrier<0>();
    }
    if (t + 2 <= t_end) issue(t + 2, stage == 0 ? NSTAGE - 1 : stage - 1);
    if (wave_active && t >= wt_begin && t <= wt_end) {
      const uint16_t* sk = lds + stage * STAGE;
      const uint16_t* sv = sk + K_TILE;
      const int kb = t * BKV;
      // ---- S^T = K . Q^T (two 32-key sub-tiles x NQ query blocks) ----
      // S^T - mu = K . Q'^T + negm: scores relative to the running max
      f32x16_t s[NQ][2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8_t a =
              *reinterpret_cast<const bf16x8_t*>(sk + kswz(sub * 32 + lrow, ks * 2 + lhalf));
#pragma unroll
          for (int qq = 0; qq < NQ; ++qq)
            s[qq][sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                a, qf[qq][ks], ks == 0 ? negm[qq] : s[qq][sub], 0, 0, 0);
        }
      // ---- mask, online softmax (log2 domain) ----
      // The offset mu only moves when a row's max grows by more than 2^8 over
      // it (checked wave-wide), so P <= 256 and the O / l rescale is skipped
      // for most tiles; O / l is unchanged by it.
      // upper bound (causal diagonal, keys past T) and lower bound (window
      // edge, segment start) are applied only in the tiles that cross them
      const bool mask_hi = (p.causal && kb + BKV - 1 > qw) || (kb + BKV > T);
      const bool mask_lo = (window > 0 && kb <= qw + QPW - 1 - window) || kb < wseg_hi;
      bf16x8_t pb[NQ][2][2];
#pragma unroll
      for (int qq = 0; qq < NQ; ++qq) {
        const int qi = qw + 32 * qq + lrow;
        // element (sub, r) holds key kb + 4 * lhalf + (a compile-time offset)
        if (mask_hi) {
          const int lim_hi = p.causal ? (qi < T - 1 ? qi : T - 1) : T - 1;  // key <= lim_hi
          const int hi_rel = lim_hi - kb - 4 * lhalf;
#pragma unroll
          for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int ko = sub * 32 + 8 * (r >> 2) + (r & 3);
              s[qq][sub][r] = ko <= hi_rel ? s[qq][sub][r] : -INFINITY;
            }
        }
        if (mask_lo) {
          int lim_lo = window > 0 ? qi - window : -1;  // key > lim_lo
          if (p.causal) {
            const int sg = qseg[qq] - 1;
            lim_lo = lim_lo > sg ? lim_lo : sg;
          }
          const int lo_rel = lim_lo - kb - 4 * lhalf;
#pragma unroll
          for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int ko = sub * 32 + 8 * (r >> 2) + (r & 3);
              s[qq][sub][r] = ko > lo_rel ? s[qq][sub][r] : -INFINITY;
            }
        }
        float mt = -INFINITY;  // this tile's max, relative to mu
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
          for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[qq][sub][r]);
        {
          // the partner lane (lane ^ 32) holds the other 32 keys of this
          // query: one VALU lane swap instead of an LDS permute round trip
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt),
                                                           __float_as_uint(mt), false, false);
          mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        const bool grow = mt > 8.f || (m[qq] == -INFINITY && mt > -INFINITY);
        if (__any(grow)) {
          const float m_new = fmaxf(m[qq], mt + mu[qq]);  // m <= m_new
          const float alpha = m[qq] == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m[qq] - m_new);
          m[qq] = m_new;
          const float mu_new = m_new == -INFINITY ? 0.f : m_new;
          const float shift = mu_new - mu[qq];
          mu[qq] = mu_new;
          l[qq] *= alpha;
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[qq][j][r] *= alpha;
#pragma unroll
          for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[qq][sub][r] -= shift;
#pragma unroll
          for (int r = 0; r < 16; ++r) negm[qq][r] = -mu_new;
        }
        float ls = l[qq];
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
              const float p0 = __builtin_amdgcn_exp2f(s[qq][sub][8 * u + e]);
              const float p1 = __builtin_amdgcn_exp2f(s[qq][sub][8 * u + e + 1]);
              w[e >> 1] = pack_bf16x2(p0, p1);
              ls = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[e >> 1]), ones2,
                                                    ls, false);
            }
            pb[qq][sub][u] = __builtin_bit_cast(bf16x8_t, u32x4_t{w[0], w[1], w[2], w[3]});
          }
        l[qq] = ls;
      }
      // ---- O^T += V^T . P^T ----
#pragma unroll
      for (int dsub = 0; dsub < 2; ++dsub)
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const uint16_t* vp = sv + (sub * 32 + u * 16) * V_LD + dsub * 32 + vt_lane;
            const s16x4_t t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(vp));
            const s16x4_t t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(vp + 8 * V_LD));
            const u32x2_t w0 = __builtin_bit_cast(u32x2_t, t0);
            const u32x2_t w1 = __builtin_bit_cast(u32x2_t, t1);
            const bf16x8_t a = __builtin_bit_cast(bf16x8_t, u32x4_t{w0.x, w0.y, w1.x, w1.y});
#pragma unroll
            for (int qq = 0; qq < NQ; ++qq)
              o[qq][dsub] =
                  __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[qq][sub][u], o[qq][dsub], 0, 0, 0);
          }
    }
    stage = stage + 1 < NSTAGE ? stage + 1 : 0;
  }

  if (!wave_active) return;
#pragma unroll
  for (int qq = 0; qq < NQ; ++qq) {
    const int qi = qw + 32 * qq + lrow;
    // the query's row sum: this lane's keys plus its partner's (lane ^ 32)
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l[qq]),
                                                     __float_as_uint(l[qq]), false, false);
    const float lt = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    if (qi >= T) continue;
    // hardware reciprocal (1 ulp): the output is rounded to bf16
    const float inv = lt > 0.f ? __builtin_amdgcn_rcpf(lt) : 0.f;
    uint16_t* orow = p.o + b * p.sb_o + h * p.sh_o + (int64_t)qi * p.st_o;
#pragma unroll
    for (int dsub = 0; dsub < 2; ++dsub)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = dsub * 32 + 8 * j + 4 * lhalf;
        u32x2_t w;
        w.x = pack_bf16x2(o[qq][dsub][4 * j] * inv, o[qq][dsub][4 * j + 1] * inv);
        w.y = pack_bf16x2(o[qq][dsub][4 * j + 2] * inv, o[qq][dsub][4 * j + 3] * inv);
        *reinterpret_cast<u32x2_t*>(orow + d0) = w;
      }
  }
}

template <int NQ>
int run_attention(const AttnArgs& a, hipStream_t s) {
  constexpr int BQ = 4 * 32 * NQ;
  const int64_t nb = ((a.T + BQ - 1) / BQ) * a.H * a.B;
  if (nb > 0x7fffffff) return fail(-2, "attention: grid too large");
  hipLaunchKernelGGL((attn_fwd_kernel<NQ>), dim3((unsigned)nb), dim3(256), 0, s, a);
  BLT_LAUNCH_CHECK("attn_fwd_kernel");
  return 0;
}

// ---- exact f32 attention: the reference kernel's semantics -----------------
// fused_attention_kernel (attention_kernel.rs:20-125): any head_dim up to 256,
// Tq and Tkv independent, causal means key j visible to query i iff j <= i,
// scores (q . k) * (1 / sqrt(d)) and the softmax in f32 throughout.  One
// block per (batch, head, 32 queries): the query tile, and 32-key tiles of K
// and V, in LDS; thread t owns query t / 8 and, in the score step, keys
// t % 8 + 8 m (m < 4), in the output step, head-dim columns t % 8 + 8 c; an
// online softmax carries the running max and sum across key tiles.
constexpr int FQ = 32, FK = 32, F_MAXD = 256;

__global__ __launch_bounds__(256) void attn_f32_kernel(const float* __restrict__ q,
                                                       const float* __restrict__ k,
                                                       const float* __restrict__ v,
                                                       float* __restrict__ o, int64_t H,
                                                       int64_t Tq, int64_t Tkv, int d,
                                                       int causal, float scale) {
  extern __shared__ float smem[];
  const int dp = d + 1;  // K row pitch: the 8 key rows a score step reads fall in distinct banks
  float* Qs = smem;                // [FQ][d]
  float* Ks = Qs + FQ * d;         // [FK][dp]
  float* Vs = Ks + FK * dp;        // [FK][d]
  float* Ps = Vs + FK * d;         // [FQ][FK + 1]
  const int tid = threadIdx.x, qi = tid >> 3, g = tid & 7;
  const int64_t q0 = (int64_t)blockIdx.x * FQ;
  const int64_t bh = (int64_t)blockIdx.z * H + blockIdx.y;
  const float* qb = q + bh * Tq * d;
  const float* kb = k + bh * Tkv * d;
  const float* vb = v + bh * Tkv * d;
  for (int i = tid; i < FQ * d; i += 256) {
    const int r = i / d;
    Qs[i] = q0 + r < Tq ? qb[(q0 + r) * d + (i % d)] : 0.f;
  }
  const int nd = (d + 7) / 8;  // output columns per thread
  float acc[F_MAXD / 8];
#pragma unroll
  for (int c = 0; c < F_MAXD / 8; ++c) acc[c] = 0.f;
  float m = -INFINITY, l = 0.f;
  const int64_t qabs = q0 + qi;
  const int64_t kend = causal ? (q0 + FQ < Tkv ? q0 + FQ : Tkv) : Tkv;
  for (int64_t k0 = 0; k0 < kend; k0 += FK) {
    __syncthreads();  // the previous tile's K, V and P are no longer read
    for (int i = tid; i < FK * d; i += 256) {
      const int r = i / d, e = i % d;
      const bool in = k0 + r < Tkv;
      Ks[r * dp + e] = in ? kb[(k0 + r) * d + e] : 0.f;
      Vs[i] = in ? vb[(k0 + r) * d + e] : 0.f;
    }
    __syncthreads();
    float sc[4];
    float mt = -INFINITY;
#pragma unroll
    for (int m2 = 0; m2 < 4; ++m2) {
      const int kj = g + 8 * m2;
      float dot = 0.f;
      for (int e = 0; e < d; ++e) dot += Qs[qi * d + e] * Ks[kj * dp + e];
      const int64_t kabs = k0 + kj;
      const bool vis = kabs < Tkv && (!causal || kabs <= qabs);
      sc[m2] = vis ? dot * scale : -INFINITY;
      mt = fmaxf(mt, sc[m2]);
    }
    // the query's 32 scores of this tile sit in 8 consecutive lanes
#pragma unroll
    for (int x = 1; x < 8; x <<= 1) mt = fmaxf(mt, __shfl_xor(mt, x, 8));
    const float m_new = fmaxf(m, mt);
    const float alpha = m == -INFINITY ? (m_new == -INFINITY ? 1.f : 0.f) : expf(m - m_new);
    float ls = 0.f;
#pragma unroll
    for (int m2 = 0; m2 < 4; ++m2) {
      const float pv = m_new == -INFINITY ? 0.f : expf(sc[m2] - m_new);
      Ps[qi * (FK + 1) + g + 8 * m2] = pv;
      ls += pv;
    }
#pragma unroll
    for (int x = 1; x < 8; x <<= 1) ls += __shfl_xor(ls, x, 8);
    l = l * alpha + ls;
    m = m_new;
#pragma unroll
    for (int c = 0; c < F_MAXD / 8; ++c) acc[c] *= alpha;
    __syncthreads();  // P of the tile complete
    for (int kj = 0; kj < FK; ++kj) {
      const float pk = Ps[qi * (FK + 1) + kj];
#pragma unroll
      for (int c = 0; c < F_MAXD / 8; ++c) {
        const int e = g + 8 * c;
        if (c < nd && e < d) acc[c] += pk * Vs[kj * d + e];
      }
    }
  }
  if (qabs >= Tq) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float* orow = o + (bh * Tq + qabs) * d;
#pragma unroll
  for (int c = 0; c < F_MAXD / 8; ++c) {
    const int e = g + 8 * c;
    if (c < nd && e < d) orow[e] = acc[c] * inv;
  }
}

}  // namespace

int launch_attention_f32(const float* q, const float* k, const float* v, float* o, int64_t B,
                         int64_t H, int64_t Tq, int64_t Tkv, int d, int causal, hipStream_t s) {
  if (B == 0 || H == 0 || Tq == 0) return 0;
  if (d < 1 || d > F_MAXD) return fail(-2, "attention_f32: head_dim must be 1 .. 256");
  if (H > 65535 || B > 65535 || (Tq + FQ - 1) / FQ > 0x7fffffff)
    return fail(-2, "attention_f32: grid too large");
  const size_t lds = (size_t)(FQ * d + FK * (d + 1) + FK * d + FQ * (FK + 1)) * sizeof(float);
  // beyond the default 64 KB of dynamic LDS the kernel's limit is raised (a
  // host-side setting of the current device, set on every such launch)
  if (lds > 64 * 1024)
    BLT_HIP_CHECK(hipFuncSetAttribute((const void*)attn_f32_kernel,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  const dim3 grid((unsigned)((Tq + FQ - 1) / FQ), (unsigned)H, (unsigned)B);
  hipLaunchKernelGGL(attn_f32_kernel, grid, dim3(256), lds, s, q, k, v, o, H, Tq, Tkv, d,
                     causal ? 1 : 0, 1.0f / sqrtf((float)d));
  BLT_LAUNCH_CHECK("attn_f32_kernel");
  return 0;
}

int launch_attention(const AttnArgs& a, hipStream_t s) {
  if (a.B == 0 || a.H == 0 || a.T == 0) return 0;
  if (a.T > 0x3fffffff) return fail(-2, "attention: T too large");
  // Q/K/V rows move as 16-byte pieces (K/V by LDS DMA)
  const bool al16 = (uintptr_t)a.q % 16 == 0 && (uintptr_t)a.k % 16 == 0 &&
                    (uintptr_t)a.v % 16 == 0 && (uintptr_t)a.o % 8 == 0;
  const bool st8 = a.sb_q % 8 == 0 && a.sh_q % 8 == 0 && a.st_q % 8 == 0 && a.sb_k % 8 == 0 &&
                   a.sh_k % 8 == 0 && a.st_k % 8 == 0 && a.sb_v % 8 == 0 && a.sh_v % 8 == 0 &&
                   a.st_v % 8 == 0 && a.sb_o % 4 == 0 && a.sh_o % 4 == 0 && a.st_o % 4 == 0;
  if (!al16 || !st8)
    return fail(-2, "attention: q/k/v need 16-byte aligned rows (pointers 16-byte aligned, "
                    "strides multiples of 8 elements)");
  // K/V rows of a tile are addressed by 32-bit byte offsets from the tile base
  const int64_t st = a.st_k > a.st_v ? a.st_k : a.st_v;
  if ((st * (BKV - 1) + D) * 2 >= ((int64_t)1 << 32))
    return fail(-2, "attention: K/V row stride too large");
  // 64 queries per wave (1 wave per SIMD) pays off for long full-causal rows;
  // with a window, 32 queries per wave (2 waves per SIMD) wastes less of
  // each masked band tile and hides latency better.
  const bool full_causal = a.causal && (a.window == 0 || a.window >= a.T);
  if (full_causal && a.T >= 2048 && a.T * a.H * a.B >= 256 * 256 * 4)
    return run_attention<2>(a, s);
  return run_attention<1>(a, s);
}

}  // namespace blt
