// Memory-bound row kernels for gfx950: softmax-entropy, RMSNorm(+L2), L2 norm,
// softmax, SiLU*gate, coherence, embedding gather, RoPE, patch boundaries.
//
// Layout rule for every row kernel: one wave64 owns one row; lane j holds the
// 4-element chunks j, j+64, j+128, ... of the row in registers (16-byte f32 /
// 8-byte bf16 vector loads, fully coalesced), so each row is read from HBM
// exactly once and all reductions are wave shuffles.  Rows wider than the
// register budget fall back to a streaming variant that re-reads the row.
#include "../../include/blt_hip.h"
#include <type_traits>

#include "rowops.hpp"

#include <math.h>

namespace blt {

// ---------------------------------------------------------------------------
// element access
// ---------------------------------------------------------------------------
__device__ inline float ld1(const float* p, int64_t i) { return p[i]; }
__device__ inline float ld1(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }

__device__ inline void ld4(const float* p, int64_t i, float v[4]) {
  float4 t = *reinterpret_cast<const float4*>(p + i);
  v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
}
__device__ inline void ld4(const uint16_t* p, int64_t i, float v[4]) {
  uint2 t = *reinterpret_cast<const uint2*>(p + i);
  v[0] = bf16_to_f32((uint16_t)(t.x & 0xffff));
  v[1] = bf16_to_f32((uint16_t)(t.x >> 16));
  v[2] = bf16_to_f32((uint16_t)(t.y & 0xffff));
  v[3] = bf16_to_f32((uint16_t)(t.y >> 16));
}
__device__ inline void st1(float* p, int64_t i, float v) { p[i] = v; }
__device__ inline void st1(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
__device__ inline void st4(float* p, int64_t i, const float v[4]) {
  *reinterpret_cast<float4*>(p + i) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ inline void st4(uint16_t* p, int64_t i, const float v[4]) {
  uint2 t;
  t.x = pack_bf16x2(v[0], v[1]);
  t.y = pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<uint2*>(p + i) = t;
}

// Row held in registers: VEC-element chunks, chunk c of lane l is row[(l + 64c)*VEC ..].
template <typename T, int VEC, int NC>
struct RowRegs {
  float v[NC][VEC];
  __device__ inline void load(const T* row, int n, int lane, float pad) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int e = (lane + BLT_WAVE * c) * VEC;
      if (e < n) {
        if constexpr (VEC == 4) ld4(row, e, v[c]);
        else v[c][0] = ld1(row, e);
      } else {
#pragma unroll
        for (int q = 0; q < VEC; ++q) v[c][q] = pad;
      }
    }
  }
};

// ---------------------------------------------------------------------------
// softmax entropy: H = -sum exp(lsm) * lsm, lsm = x - max - log(sum exp(x - max))
// (the NdArray form of patcher::entropy, patcher.rs:38-63)
// ---------------------------------------------------------------------------
template <typename T, int VEC, int NC>
__global__ __launch_bounds__(256) void entropy_kernel(const T* __restrict__ logits,
                                                      float* __restrict__ out, int64_t rows,
                                                      int n) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  RowRegs<T, VEC, NC> r;
  r.load(logits + row * n, n, lane, -INFINITY);
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int q = 0; q < VEC; ++q) m = fmaxf(m, r.v[c][q]);
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int q = 0; q < VEC; ++q) s += __expf(r.v[c][q] - m);  // padding: exp(-inf) = 0
  s = wave_sum(s);
  const float lse = __logf(s);
  float h = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int q = 0; q < VEC; ++q) {
      const int e = (lane + BLT_WAVE * c) * VEC + q;
      if (e < n) {
        const float lsm = (r.v[c][q] - m) - lse;
        h += __expf(lsm) * lsm;
      }
    }
  h = wave_sum(h);
  if (lane == 0) out[row] = -h;
}

// Rows below 512 elements (n % 4 == 0, aligned): 32 lanes per row, two rows
// per wave, eight per block.  A row of 260 f32 logits is two 16-byte loads
// and one element per lane instead of one load and a 4-element tail over 64
// lanes, so a wave's reductions and exponentials serve two rows at once
// (config 1: 5.5 us for 32,768 rows against 7.6 us one row per wave).  The
// upper half of a wave past the last row computes a valid row and stores
// nothing (both halves run the cross-lane steps).
template <typename T, int NH, int VT>
__global__ __launch_bounds__(256) void entropy_half_kernel(const T* __restrict__ logits,
                                                           float* __restrict__ out,
                                                           int64_t rows, int n) {
  const int l32 = threadIdx.x & 31;
  const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  const T* x = logits + (row < rows ? row : rows - 1) * n;
  float v[NH > 0 ? NH : 1][4], t[VT > 0 ? VT : 1];
#pragma unroll
  for (int c = 0; c < NH; ++c) ld4(x, c * 128 + l32 * 4, v[c]);
#pragma unroll
  for (int q = 0; q < VT; ++q) {
    const int e = NH * 128 + q * 32 + l32;
    t[q] = e < n ? ld1(x, e) : -INFINITY;
  }
  const float H = entropy_half_row<NH, VT>(v, t);
  if (l32 == 0 && row < rows) out[row] = H;
}

// Rows of n = 256 NF + 64 (VT - 1) + r elements (n % 4 == 0, NF <= 4, VT <= 4):
// NF full chunks of 256 (16-byte loads, 4 per lane) and a tail of VT
// elements per lane (e = 256 NF + 64 q + lane), so no lane computes an
// exponential for a chunk that is mostly padding.  One exponential per
// element: with d = x - max, p = exp(d), s = sum p, lse = log s,
//   H = -sum (p / s)(d - lse) = lse - (sum p d) / s,
// the same quantity as -sum exp(lsm) lsm (padding: p = 0, d clamped finite).
template <typename T, int NF, int VT>
__global__ __launch_bounds__(256) void entropy_tail_kernel(const T* __restrict__ logits,
                                                           float* __restrict__ out,
                                                           int64_t rows, int n) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* x = logits + row * n;
  float v[NF > 0 ? NF : 1][4], t[VT > 0 ? VT : 1];
#pragma unroll
  for (int c = 0; c < NF; ++c) ld4(x, c * 256 + lane * 4, v[c]);
#pragma unroll
  for (int q = 0; q < VT; ++q) {
    const int e = NF * 256 + q * 64 + lane;
    t[q] = e < n ? ld1(x, e) : -INFINITY;
  }
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < NF; ++c)
    m = fmaxf(m, fmaxf(fmaxf(v[c][0], v[c][1]), fmaxf(v[c][2], v[c][3])));
#pragma unroll
  for (int q = 0; q < VT; ++q) m = fmaxf(m, t[q]);
  m = wave_max(m);
  float sp = 0.f, sd = 0.f;
  auto acc = [&](float xv) {
    const float d = fmaxf(xv - m, -1e30f);  // padding (-inf) contributes 0
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
  // hardware reciprocal (1 ulp) for the one quotient per row
  if (lane == 0) out[row] = __logf(sp) - sd * __builtin_amdgcn_rcpf(sp);
}

// Any width: three streaming passes over the row.
template <typename T>
__global__ __launch_bounds__(256) void entropy_stream_kernel(const T* __restrict__ logits,
                                                             float* __restrict__ out,
                                                             int64_t rows, int n) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* x = logits + row * n;
  float m = -INFINITY;
  for (int e = lane; e < n; e += BLT_WAVE) m = fmaxf(m, ld1(x, e));
  m = wave_max(m);
  float s = 0.f;
  for (int e = lane; e < n; e += BLT_WAVE) s += __expf(ld1(x, e) - m);
  s = wave_sum(s);
  const float lse = __logf(s);
  float h = 0.f;
  for (int e = lane; e < n; e += BLT_WAVE) {
    const float lsm = (ld1(x, e) - m) - lse;
    h += __expf(lsm) * lsm;
  }
  h = wave_sum(h);
  if (lane == 0) out[row] = -h;
}

// ---------------------------------------------------------------------------
// RMSNorm with optional L2 norm of the input row.
//   after_sqrt:  y = x / (sqrt(mean x^2) + eps) * w     (model.rs:758-770)
//   inside_sqrt: y = x / sqrt(mean x^2 + eps) * w       (rms_norm_kernel.rs:40-43)
// ---------------------------------------------------------------------------
__device__ inline float rms_denominator(float ss, int n, float eps, int mode) {
  const float ms = ss / (float)n;
  return mode == 0 ? (sqrtf(ms) + eps) : sqrtf(ms + eps);
}

template <typename TX, typename TW, typename TY, int VEC, int NC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const TX* __restrict__ x,
                                                      const TW* __restrict__ w,
                                                      TY* __restrict__ y,
                                                      float* __restrict__ l2, int64_t rows,
                                                      int n, float eps, int mode) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  RowRegs<TX, VEC, NC> r;
  r.load(x + row * n, n, lane, 0.f);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int q = 0; q < VEC; ++q) ss += r.v[c][q] * r.v[c][q];
  ss = wave_sum(ss);
  // x / den as x * (1 / den): one correctly rounded reciprocal per row
  // instead of an IEEE division per element (within 1.5 ulp of the quotient)
  const float inv = 1.f / rms_denominator(ss, n, eps, mode);
  if (l2 != nullptr && lane == 0) l2[row] = sqrtf(ss);
  if (y == nullptr) return;
  TY* yr = y + row * n;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int e = (lane + BLT_WAVE * c) * VEC;
    if (e < n) {
      float wv[VEC], o[VEC];
      if constexpr (VEC == 4) ld4(w, e, wv);
      else wv[0] = ld1(w, e);
#pragma unroll
      for (int q = 0; q < VEC; ++q) o[q] = (r.v[c][q] * inv) * wv[q];
      if constexpr (VEC == 4) st4(yr, e, o);
      else st1(yr, e, o[0]);
    }
  }
}

// bf16 rows of n <= 1024 (n % 8 == 0), two rows per wave in 16-byte pieces:
// piece p = lane + 64 k covers row p / (n / 8), elements 8 (p % (n / 8)) ..
// + 8, so the wave's loads and stores are whole 16-byte pieces (the generic
// kernel moves 8 bytes per lane for bf16) and both rows' reads are in flight
// together.
template <int NP>
__global__ __launch_bounds__(256) void rmsnorm_bf16_pair_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
    float* __restrict__ l2, int64_t rows, int n, float eps, int mode) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 2;
  if (row0 >= rows) return;
  const int pr = n / 8;                       // pieces per row
  const int np = row0 + 1 < rows ? 2 * pr : pr;  // pieces of this wave's rows
  u32x4_t xv[NP], wv[NP];
  float ss0 = 0.f, ss1 = 0.f;
  // the weight pieces are loaded with the row pieces, so the stores after the
  // reductions wait on nothing further
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int p = lane + 64 * k;
    if (p < np) {
      const int r = p >= pr, c = (p - r * pr) * 8;
      xv[k] = *reinterpret_cast<const u32x4_t*>(x + (row0 + r) * n + c);
      if (y != nullptr) wv[k] = *reinterpret_cast<const u32x4_t*>(w + c);
    }
  }
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int p = lane + 64 * k;
    if (p < np) {
      float q = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = bf16_to_f32((uint16_t)(xv[k][e] & 0xffff));
        const float hi = bf16_to_f32((uint16_t)(xv[k][e] >> 16));
        q += lo * lo + hi * hi;
      }
      if (p >= pr) ss1 += q; else ss0 += q;
    }
  }
  ss0 = wave_sum(ss0);
  ss1 = wave_sum(ss1);
  // x / den as x * (1 / den), as the generic kernel
  const float inv0 = 1.f / rms_denominator(ss0, n, eps, mode);
  const float inv1 = 1.f / rms_denominator(ss1, n, eps, mode);
  if (l2 != nullptr && lane == 0) {
    l2[row0] = sqrtf(ss0);
    if (row0 + 1 < rows) l2[row0 + 1] = sqrtf(ss1);
  }
  if (y == nullptr) return;
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int p = lane + 64 * k;
    if (p < np) {
      const int r = p >= pr, c = (p - r * pr) * 8;
      const float inv = r ? inv1 : inv0;
      u32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = bf16_to_f32((uint16_t)(xv[k][e] & 0xffff));
        const float x1 = bf16_to_f32((uint16_t)(xv[k][e] >> 16));
        const float w0 = bf16_to_f32((uint16_t)(wv[k][e] & 0xffff));
        const float w1 = bf16_to_f32((uint16_t)(wv[k][e] >> 16));
        o[e] = pack_bf16x2((x0 * inv) * w0, (x1 * inv) * w1);
      }
      *reinterpret_cast<u32x4_t*>(y + (row0 + r) * n + c) = o;
    }
  }
}

template <typename TX, typename TW, typename TY>
__global__ __launch_bounds__(256) void rmsnorm_stream_kernel(const TX* __restrict__ x,
                                                             const TW* __restrict__ w,
                                                             TY* __restrict__ y,
                                                             float* __restrict__ l2,
                                                             int64_t rows, int n, float eps,
                                                             int mode) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const TX* xr = x + row * n;
  float ss = 0.f;
  for (int e = lane; e < n; e += BLT_WAVE) {
    const float v = ld1(xr, e);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float inv = 1.f / rms_denominator(ss, n, eps, mode);
  if (l2 != nullptr && lane == 0) l2[row] = sqrtf(ss);
  if (y == nullptr) return;
  for (int e = lane; e < n; e += BLT_WAVE) st1(y + row * n, e, (ld1(xr, e) * inv) * ld1(w, e));
}

// ---------------------------------------------------------------------------
// softmax over the last dim: exp(x - max) / sum (Burn activation::softmax)
// ---------------------------------------------------------------------------
template <int VEC, int NC>
__global__ __launch_bounds__(256) void softmax_kernel(const float* __restrict__ x,
                                                      float* __restrict__ y, int64_t rows,
                                                      int n) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  RowRegs<float, VEC, NC> r;
  r.load(x + row * n, n, lane, -INFINITY);
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int q = 0; q < VEC; ++q) m = fmaxf(m, r.v[c][q]);
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int q = 0; q < VEC; ++q) {
      r.v[c][q] = __expf(r.v[c][q] - m);
      s += r.v[c][q];
    }
  s = wave_sum(s);
  float* yr = y + row * n;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int e = (lane + BLT_WAVE * c) * VEC;
    if (e < n) {
      float o[VEC];
#pragma unroll
      for (int q = 0; q < VEC; ++q) o[q] = r.v[c][q] / s;
      if constexpr (VEC == 4) st4(yr, e, o);
      else st1(yr, e, o[0]);
    }
  }
}

__global__ __launch_bounds__(256) void softmax_stream_kernel(const float* __restrict__ x,
                                                             float* __restrict__ y,
                                                             int64_t rows, int n) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + row * n;
  float m = -INFINITY;
  for (int e = lane; e < n; e += BLT_WAVE) m = fmaxf(m, xr[e]);
  m = wave_max(m);
  float s = 0.f;
  for (int e = lane; e < n; e += BLT_WAVE) s += __expf(xr[e] - m);
  s = wave_sum(s);
  for (int e = lane; e < n; e += BLT_WAVE) y[row * n + e] = __expf(xr[e] - m) / s;
}

// ---------------------------------------------------------------------------
// elementwise: SiLU * gate, coherence
// ---------------------------------------------------------------------------
__device__ inline float silu_gate1(float g, float u) { return (g / (1.f + __expf(-g))) * u; }

__global__ __launch_bounds__(256) void silu_gate_f32_kernel(const float* __restrict__ g,
                                                            const float* __restrict__ u,
                                                            float* __restrict__ out,
                                                            int64_t n, int vec) {
  const int64_t n4 = vec ? n / 4 : 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    float4 a = reinterpret_cast<const float4*>(g)[i];
    float4 b = reinterpret_cast<const float4*>(u)[i];
    reinterpret_cast<float4*>(out)[i] = make_float4(silu_gate1(a.x, b.x), silu_gate1(a.y, b.y),
                                                    silu_gate1(a.z, b.z), silu_gate1(a.w, b.w));
  }
  for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = silu_gate1(g[i], u[i]);
}

// 8 bf16 per thread per step (16-byte loads and stores).
__global__ __launch_bounds__(256) void silu_gate_bf16_kernel(const uint16_t* __restrict__ g,
                                                             const uint16_t* __restrict__ u,
                                                             uint16_t* __restrict__ out,
                                                             int64_t n, int vec) {
  const int64_t n8 = vec ? n / 8 : 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
    uint4 a = reinterpret_cast<const uint4*>(g)[i];
    uint4 b = reinterpret_cast<const uint4*>(u)[i];
    const uint32_t* pa = reinterpret_cast<const uint32_t*>(&a);
    const uint32_t* pb = reinterpret_cast<const uint32_t*>(&b);
    uint4 o;
    uint32_t* po = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float g0 = bf16_to_f32((uint16_t)(pa[k] & 0xffff)), g1 = bf16_to_f32((uint16_t)(pa[k] >> 16));
      const float u0 = bf16_to_f32((uint16_t)(pb[k] & 0xffff)), u1 = bf16_to_f32((uint16_t)(pb[k] >> 16));
      po[k] = pack_bf16x2(silu_gate1(g0, u0), silu_gate1(g1, u1));
    }
    reinterpret_cast<uint4*>(out)[i] = o;
  }
  for (int64_t i = n8 * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = f32_to_bf16(silu_gate1(bf16_to_f32(g[i]), bf16_to_f32(u[i])));
}

__global__ __launch_bounds__(256) void coherence_kernel(const float* __restrict__ nrm,
                                                        const float* __restrict__ ent,
                                                        float* __restrict__ out, int64_t n,
                                                        float eps) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = (nrm[i] * nrm[i]) / (ent[i] + eps);
}

// ---------------------------------------------------------------------------
// token embedding gather: x[r, :] = f32(W[clamp(tok[r]), :])   (nn::Embedding)
// one wave per token row, 8-byte bf16 loads, 16-byte f32 stores.
// ---------------------------------------------------------------------------
// With xb / ss (dim % 64 == 0) the row, times the first layer's RMSNorm
// weight ws (one bf16 rounding of the f32 product; ws NULL = 1), goes to xb
// and the row's per-64-column sums of squares go to ss [rows, dim / 64]: the
// inputs of the first layer's QKV GEMM, which applies the row factor itself.
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ tok,
                                                    const uint16_t* __restrict__ table,
                                                    float* __restrict__ x, int64_t rows,
                                                    int dim, int vocab,
                                                    uint16_t* __restrict__ xb,
                                                    float* __restrict__ ss,
                                                    const float* __restrict__ ws) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  int t = tok[row];
  t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
  const uint16_t* src = table + (int64_t)t * dim;
  float* dst = x + row * dim;
  for (int e = lane * 4; e < dim; e += BLT_WAVE * 4) {
    float v[4];
    ld4(src, e, v);
    st4(dst, e, v);
    if (xb) {
      // the 16 lanes of each 16-lane group hold one 64-column group
      if (ws) {
        const f32x4_t w = *reinterpret_cast<const f32x4_t*>(ws + e);
        *reinterpret_cast<u32x2_t*>(xb + row * dim + e) =
            u32x2_t{pack_bf16x2(v[0] * w.x, v[1] * w.y), pack_bf16x2(v[2] * w.z, v[3] * w.w)};
      } else {
        *reinterpret_cast<u32x2_t*>(xb + row * dim + e) =
            *reinterpret_cast<const u32x2_t*>(src + e);
      }
      float q = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
      q = sum16(q);
      if ((lane & 15) == 0) ss[row * (dim / 64) + e / 64] = q;
    }
  }
}

// ---------------------------------------------------------------------------
// RoPE (half-split pairs (m, m + d/2), model.rs:107-147) from a strided bf16
// tensor into a dense [B, H, T, d] bf16 tensor.  One thread per (row, m).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* __restrict__ src,
                                                   uint16_t* __restrict__ dst,
                                                   const float* __restrict__ cs, int64_t B,
                                                   int64_t H, int64_t T, int d, int64_t sb,
                                                   int64_t sh, int64_t st) {
  const int half = d / 2;
  const int64_t total = B * H * T * half;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int m = (int)(i % half);
    const int64_t r = i / half;  // (b*H + h)*T + t
    const int64_t t = r % T;
    const int64_t bh = r / T;
    const int64_t h = bh % H, b = bh / H;
    const uint16_t* s = src + b * sb + h * sh + t * st;
    const float x1 = bf16_to_f32(s[m]), x2 = bf16_to_f32(s[m + half]);
    const float c = cs[(t * half + m) * 2], sn = cs[(t * half + m) * 2 + 1];
    uint16_t* o = dst + r * d;
    o[m] = f32_to_bf16(x1 * c - x2 * sn);
    o[m + half] = f32_to_bf16(x1 * sn + x2 * c);
  }
}

// The same for head_dim 64 with 16-byte rows: one thread per 8 pairs, 16-byte
// loads and stores of both halves and of the (cos, sin) table.
__global__ __launch_bounds__(256) void rope64_kernel(const uint16_t* __restrict__ src,
                                                     uint16_t* __restrict__ dst,
                                                     const float* __restrict__ cs, int64_t B,
                                                     int64_t H, int64_t T, int64_t sb,
                                                     int64_t sh, int64_t st) {
  constexpr int D = 64, HALF = 32, G = HALF / 8;
  const int64_t total = B * H * T * G;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int g = (int)(i % G);
    const int64_t r = i / G;  // (b*H + h)*T + t
    const int64_t t = r % T;
    const int64_t bh = r / T;
    const int64_t h = bh % H, b = bh / H;
    const uint16_t* s = src + b * sb + h * sh + t * st + 8 * g;
    const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(s);
    const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(s + HALF);
    const f32x4_t* c4 = reinterpret_cast<const f32x4_t*>(cs + (t * HALF + 8 * g) * 2);
    uint32_t o1[4], o2[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {  // pairs 2q, 2q + 1 of this group
      const f32x4_t c = c4[q];      // (cos, sin) of pair 2q, then of pair 2q + 1
      const float a0 = bf16_to_f32((uint16_t)(lo[q] & 0xffff)), a1 = bf16_to_f32((uint16_t)(lo[q] >> 16));
      const float b0 = bf16_to_f32((uint16_t)(hi[q] & 0xffff)), b1 = bf16_to_f32((uint16_t)(hi[q] >> 16));
      o1[q] = pack_bf16x2(a0 * c.x - b0 * c.y, a1 * c.z - b1 * c.w);
      o2[q] = pack_bf16x2(a0 * c.y + b0 * c.x, a1 * c.w + b1 * c.z);
    }
    uint16_t* o = dst + r * D + 8 * g;
    *reinterpret_cast<u32x4_t*>(o) = u32x4_t{o1[0], o1[1], o1[2], o1[3]};
    *reinterpret_cast<u32x4_t*>(o + HALF) = u32x4_t{o2[0], o2[1], o2[2], o2[3]};
  }
}

// ---------------------------------------------------------------------------
// Patch boundaries: one 1024-thread block per batch row.
//   flag[t] = 1 for t < 2; else monotonic: (H[t] - H[t-1]) > thr, global: H[t] > thr
//   (patcher.rs:80-118; T = 1 -> [1], T = 2 -> [1, 1] fall out of the t < 2 rule).
// Block-wide exclusive scan over the flags compacts the start indices
// (patch_start_indices_cpu, patcher.rs:124-142); a second sweep turns the
// starts into lengths (patch_lengths_from_start_indices, patcher.rs:144-164).
// ---------------------------------------------------------------------------
#define PB_THREADS 1024
#define PB_ITEMS 8  // the vector path below loads and stores them as two 16-byte pieces
// mode of patch_boundary_kernel whose input is a start mask (int32 bits read
// through the f32 pointer): flag[t] = (mask[t] == 1) at every t, the test of
// patch_start_indices_cpu (patcher.rs:131-136)
#define PB_MODE_MASK 2

// Row b covers H[off_b, off_b + T_b): off_b = b * T and T_b = T for a dense
// [B, T] input, or row_off[b] / row_len[b] for variable-length rows (the
// per-document pass of the ingest driver).  mask / starts / lengths use the
// same offsets as H.
__global__ __launch_bounds__(PB_THREADS) void patch_boundary_kernel(
    const float* __restrict__ H, int64_t T_dense, float thr, int mode,
    int32_t* __restrict__ mask, int32_t* __restrict__ starts, int32_t* __restrict__ lengths,
    int32_t* __restrict__ count, const int64_t* __restrict__ row_off,
    const int32_t* __restrict__ row_len) {
  __shared__ int wave_tot[PB_THREADS / BLT_WAVE];
  // this chunk's starts (chunk-local order), so lengths need no global
  // write-then-read round trip; the last start of a chunk waits for the
  // first start of a later chunk (or the row end)
  __shared__ int32_t chunk_starts[PB_THREADS * PB_ITEMS];
  __shared__ int carry_s, chunk_tot_s, pend_idx_s, pend_start_s;
  const int64_t b = blockIdx.x;
  const int64_t roff = row_off ? row_off[b] : b * T_dense;
  const int64_t T = row_len ? (int64_t)row_len[b] : T_dense;
  const float* h = H + roff;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const bool want_len = lengths && starts;
  if (tid == 0) {
    carry_s = 0;
    pend_idx_s = -1;
    pend_start_s = 0;
  }
  __syncthreads();
  for (int64_t t0 = 0; t0 < T; t0 += (int64_t)PB_THREADS * PB_ITEMS) {
    const int64_t p0 = t0 + (int64_t)tid * PB_ITEMS;
    int flags[PB_ITEMS];
    int local = 0;
    float prev = (p0 >= 1 && p0 - 1 < T) ? h[p0 - 1] : 0.f;
    // whole 16-byte pieces when the row is aligned and this thread's items
    // all exist (PB_ITEMS == 8: two float4 loads, two int4 mask stores)
    const bool full = p0 + PB_ITEMS <= T;
    const bool vec = full && ((uintptr_t)h & 15) == 0;
    const bool vec_st = full && ((uintptr_t)(mask + roff) & 15) == 0;
    float cur[PB_ITEMS];
    if (vec) {
      const float4 a = *reinterpret_cast<const float4*>(h + p0);
      const float4 c = *reinterpret_cast<const float4*>(h + p0 + 4);
      cur[0] = a.x; cur[1] = a.y; cur[2] = a.z; cur[3] = a.w;
      cur[4] = c.x; cur[5] = c.y; cur[6] = c.z; cur[7] = c.w;
    } else {
#pragma unroll
      for (int k = 0; k < PB_ITEMS; ++k) cur[k] = p0 + k < T ? h[p0 + k] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < PB_ITEMS; ++k) {
      const int64_t t = p0 + k;
      int f = 0;
      if (t < T) {
        if (mode == PB_MODE_MASK) f = __builtin_bit_cast(int32_t, cur[k]) == 1;
        else if (t < 2) f = 1;
        else if (mode == 0) f = (cur[k] - prev) > thr;
        else f = cur[k] > thr;
        prev = cur[k];
      }
      flags[k] = f;
      local += f;
    }
    if (mask) {
      if (vec_st) {
        *reinterpret_cast<int4*>(mask + roff + p0) = int4{flags[0], flags[1], flags[2], flags[3]};
        *reinterpret_cast<int4*>(mask + roff + p0 + 4) =
            int4{flags[4], flags[5], flags[6], flags[7]};
      } else {
#pragma unroll
        for (int k = 0; k < PB_ITEMS; ++k)
          if (p0 + k < T) mask[roff + p0 + k] = flags[k];
      }
    }
    // inclusive wave scan of per-thread counts
    const int incl = wave_incl_scan(local);
    if (lane == BLT_WAVE - 1) wave_tot[wid] = incl;
    __syncthreads();
    if (wid == 0) {
      static_assert(PB_THREADS / BLT_WAVE == 16, "wave totals scanned within one 16-lane row");
      const int wt = lane < PB_THREADS / BLT_WAVE ? wave_tot[lane] : 0;
      const int wincl = row16_incl_scan(wt);
      if (lane < PB_THREADS / BLT_WAVE) wave_tot[lane] = wincl - wt;  // exclusive
      if (lane == PB_THREADS / BLT_WAVE - 1) chunk_tot_s = wincl;
    }
    __syncthreads();
    const int carry = carry_s, n_chunk = chunk_tot_s;
    int loc = wave_tot[wid] + (incl - local);  // chunk-local index of this thread's first start
    if (starts) {
#pragma unroll
      for (int k = 0; k < PB_ITEMS; ++k)
        if (flags[k]) {
          starts[roff + carry + loc] = (int32_t)(p0 + k);
          chunk_starts[loc] = (int32_t)(p0 + k);
          ++loc;
        }
    }
    __syncthreads();  // chunk_starts complete; every thread has read carry_s
    if (want_len && n_chunk > 0) {
      for (int i = tid; i + 1 < n_chunk; i += PB_THREADS)
        lengths[roff + carry + i] = chunk_starts[i + 1] - chunk_starts[i];
      if (tid == 0) {
        if (pend_idx_s >= 0) lengths[roff + pend_idx_s] = chunk_starts[0] - pend_start_s;
        pend_idx_s = carry + n_chunk - 1;
        pend_start_s = chunk_starts[n_chunk - 1];
      }
    }
    if (tid == 0) carry_s = carry + n_chunk;
    __syncthreads();  // chunk_starts, carry_s and the pending start are reused next chunk
  }
  const int n = carry_s;
  if (tid == 0) {
    if (count) count[b] = n;
    if (want_len && pend_idx_s >= 0) lengths[roff + pend_idx_s] = (int32_t)T - pend_start_s;
  }
}

// ---------------------------------------------------------------------------
// Per-patch means: the mean entropy, mean prominence (pre-norm L2 norm) and
// mean coherence of every patch (compute_mean_entropy / compute_mean_prominence,
// pipeline.rs:240-258; the per-segment coherence of huggingface_loader.rs:
// 265-295).  Patch p of a row covers [starts[p], starts[p + 1]), the last one
// running to the row end; each sum runs left to right in f32 and is divided
// by the patch length, as the reference's iter().sum::<f32>() / n does, so the
// results are bit-identical to it.  Row layout as in patch_boundary_kernel;
// starts (ascending, as the boundary pass writes them) and the outputs share
// the row offsets.
//
// One block per row walks it in tiles of PM_TILE positions staged in LDS with
// coalesced loads.  Each patch that starts in a tile is one thread's serial
// chain over the tile's LDS copy; the one patch that runs past the tile end
// hands its partial sums (two LDS slots, alternating by tile) to thread 0 of
// the next tile, which continues the same chain, so a patch of any length
// costs LDS reads, not one dependent global load per element.
// ---------------------------------------------------------------------------
constexpr int PM_THREADS = 256;
constexpr int PM_TILE = 2048;

// One chain's sums over LDS positions [a, z), left to right: the reads go 16
// bytes at a time and run ahead of the dependent adds (unrolled body), the
// order of the adds is the element order.
template <bool HAS_C>
__device__ inline void pm_chain(const float* sH, const float* sN, const float* sC, int a, int z,
                                float& sh, float& sn, float& sc) {
  int t = a;
  for (; t < z && (t & 3); ++t) {
    sh += sH[t];
    sn += sN[t];
    if (HAS_C) sc += sC[t];
  }
#pragma unroll 4
  for (; t + 4 <= z; t += 4) {
    const float4 h = *reinterpret_cast<const float4*>(sH + t);
    const float4 q = *reinterpret_cast<const float4*>(sN + t);
    sh += h.x; sh += h.y; sh += h.z; sh += h.w;
    sn += q.x; sn += q.y; sn += q.z; sn += q.w;
    if (HAS_C) {
      const float4 c = *reinterpret_cast<const float4*>(sC + t);
      sc += c.x; sc += c.y; sc += c.z; sc += c.w;
    }
  }
  for (; t < z; ++t) {
    sh += sH[t];
    sn += sN[t];
    if (HAS_C) sc += sC[t];
  }
}

template <bool HAS_C>
__global__ __launch_bounds__(PM_THREADS) void patch_means_kernel(
    const float* __restrict__ H, const float* __restrict__ N, const float* __restrict__ C,
    const int32_t* __restrict__ starts, const int32_t* __restrict__ count, int64_t T_dense,
    const int64_t* __restrict__ row_off, const int32_t* __restrict__ row_len,
    float* __restrict__ mH, float* __restrict__ mN, float* __restrict__ mC,
    const int64_t* __restrict__ out_off) {
  __shared__ __attribute__((aligned(16))) float sH[PM_TILE];
  __shared__ __attribute__((aligned(16))) float sN[PM_TILE];
  __shared__ __attribute__((aligned(16))) float sC[HAS_C ? PM_TILE : 4];
  __shared__ float carry[2][3];  // partial sums handed to the next tile
  __shared__ int32_t last[2];    // last patch started in the tile (atomicMax)
  const int64_t b = blockIdx.x;
  const int64_t roff = row_off ? row_off[b] : b * T_dense;
  const int64_t T = row_len ? (int64_t)row_len[b] : T_dense;
  const int64_t ooff = out_off ? out_off[b] : roff;
  // without starts every row is one patch [0, T)
  int64_t n = starts ? (int64_t)count[b] : 1;
  n = n < 0 ? 0 : (n > T ? T : n);
  const int tid = threadIdx.x;
  // patch p's span, clamped to 0 <= st <= e <= T
  auto span = [&](int64_t p, int64_t& st, int64_t& e) {
    e = p + 1 < n ? (int64_t)starts[roff + p + 1] : T;
    e = e < 0 ? 0 : (e > T ? T : e);
    st = starts ? (int64_t)starts[roff + p] : 0;
    st = st < 0 ? 0 : (st > e ? e : st);
  };
  auto put = [&](int64_t p, float sh, float sn, float sc, int64_t len) {
    const bool any = len > 0;
    const float fl = (float)len;
    if (mH) mH[ooff + p] = any ? sh / fl : 0.f;
    if (mN) mN[ooff + p] = any ? sn / fl : 0.f;
    if (mC) mC[ooff + p] = any ? sc / fl : 0.f;
  };
  if (tid == 0) last[0] = -1;
  int64_t p0 = 0;   // first patch that has not started in an earlier tile
  int64_t cp = -1;  // patch continuing from the previous tile (-1: none)
  int k = 0;
  for (int64_t t0 = 0; t0 < T && (p0 < n || cp >= 0); t0 += PM_TILE, ++k) {
    const int64_t t1 = t0 + PM_TILE < T ? t0 + PM_TILE : T;
    const int w = (int)(t1 - t0);
    for (int i = tid; i < w; i += PM_THREADS) {
      sH[i] = H[roff + t0 + i];
      sN[i] = N[roff + t0 + i];
      if (HAS_C) sC[i] = C[roff + t0 + i];
    }
    __syncthreads();
    // the next tile's counter, free since that tile's last read two syncs ago
    if (tid == 0) last[(k + 1) & 1] = -1;
    const int nc0 = cp >= 0 ? 1 : 0;  // chain 0 continues patch cp
    for (int64_t j = tid;; j += PM_THREADS) {
      int64_t p, st, e;
      float sh = 0.f, sn = 0.f, sc = 0.f;
      if (j < nc0) {
        p = cp;
        span(p, st, e);
        sh = carry[k & 1][0];
        sn = carry[k & 1][1];
        sc = carry[k & 1][2];
      } else {
        p = p0 + (j - nc0);
        if (p >= n) break;
        span(p, st, e);
        if (st >= t1) break;  // starts ascend: this and later patches start further on
        atomicMax(&last[k & 1], (int32_t)p);
      }
      const int a = (int)((st > t0 ? st : t0) - t0);
      const int z = (int)((e < t1 ? e : t1) - t0);
      pm_chain<HAS_C>(sH, sN, sC, a, z, sh, sn, sc);
      if (e <= t1) {
        put(p, sh, sn, sc, e - st);
      } else {  // only the tile's last chain runs on
        carry[(k + 1) & 1][0] = sh;
        carry[(k + 1) & 1][1] = sn;
        carry[(k + 1) & 1][2] = sc;
      }
    }
    __syncthreads();
    // block-uniform: the patches that started here and the chain that runs on
    const int64_t lp = last[k & 1];
    const int64_t lastchain = lp >= p0 ? lp : cp;
    if (lp >= p0) p0 = lp + 1;
    cp = -1;
    if (lastchain >= 0) {
      int64_t st, e;
      span(lastchain, st, e);
      if (e > t1) cp = lastchain;
    }
  }
  // patches that start at or past the row end (only for malformed starts)
  for (int64_t p = p0 + tid; p < n; p += PM_THREADS) put(p, 0.f, 0.f, 0.f, 0);
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
namespace {
// Register-resident variants cover rows up to 64 * 4 * 8 = 2048 elements
// (vector path, n % 4 == 0) or 64 * 16 = 1024 (scalar path); wider rows stream.
template <class L>
int dispatch_row(int n, bool vec_ok, const typename L::Args& a) {
  if (n % 4 == 0 && vec_ok) {
    switch ((n / 4 + 63) / 64) {
      case 1: return L::template run<4, 1>(a);
      case 2: return L::template run<4, 2>(a);
      case 3: return L::template run<4, 3>(a);
      case 4: return L::template run<4, 4>(a);
      case 5: case 6: return L::template run<4, 6>(a);
      case 7: case 8: return L::template run<4, 8>(a);
      default: break;
    }
  } else if (n % 4 != 0 || !vec_ok) {
    switch ((n + 63) / 64) {
      case 1: return L::template run<1, 1>(a);
      case 2: return L::template run<1, 2>(a);
      case 3: case 4: return L::template run<1, 4>(a);
      case 5: case 6: case 7: case 8: return L::template run<1, 8>(a);
      case 9: case 10: case 11: case 12: case 13: case 14: case 15: case 16:
        return L::template run<1, 16>(a);
      default: break;
    }
  }
  return L::stream(a);
}

template <typename T>
struct EntropyL {
  struct Args { const T* x; float* out; int64_t rows; int n; hipStream_t s; };
  template <int VEC, int NC>
  static int run(const Args& a) {
    hipLaunchKernelGGL((entropy_kernel<T, VEC, NC>), dim3(ceil_div(a.rows, 4)), dim3(256), 0,
                       a.s, a.x, a.out, a.rows, a.n);
    BLT_LAUNCH_CHECK("entropy_kernel");
    return 0;
  }
  static int stream(const Args& a) {
    hipLaunchKernelGGL((entropy_stream_kernel<T>), dim3(ceil_div(a.rows, 4)), dim3(256), 0, a.s,
                       a.x, a.out, a.rows, a.n);
    BLT_LAUNCH_CHECK("entropy_stream_kernel");
    return 0;
  }
  template <int NF, int VT>
  static int tail(const Args& a) {
    hipLaunchKernelGGL((entropy_tail_kernel<T, NF, VT>), dim3(ceil_div(a.rows, 4)), dim3(256), 0,
                       a.s, a.x, a.out, a.rows, a.n);
    BLT_LAUNCH_CHECK("entropy_tail_kernel");
    return 0;
  }
  template <int NF>
  static int tail_vt(const Args& a, int vt) {
    switch (vt) {
      case 0: return NF > 0 ? tail<NF, 0>(a) : -1;
      case 1: return tail<NF, 1>(a);
      case 2: return tail<NF, 2>(a);
      case 3: return tail<NF, 3>(a);
      case 4: return tail<NF, 4>(a);
    }
    return -1;
  }
  template <int NH, int VT>
  static int half(const Args& a) {
    hipLaunchKernelGGL((entropy_half_kernel<T, NH, VT>), dim3(ceil_div(a.rows, 8)), dim3(256), 0,
                       a.s, a.x, a.out, a.rows, a.n);
    BLT_LAUNCH_CHECK("entropy_half_kernel");
    return 0;
  }
  template <int NH>
  static int half_vt(const Args& a, int vt) {
    switch (vt) {
      case 0: return NH > 0 ? half<NH, 0>(a) : -1;
      case 1: return half<NH, 1>(a);
      case 2: return half<NH, 2>(a);
      case 3: return half<NH, 3>(a);
      case 4: return half<NH, 4>(a);
    }
    return -1;
  }
  // n % 4 == 0 with 16-byte (f32) / 8-byte (bf16) aligned rows, n < 1280
  static int fast(const Args& a) {
    if (a.n < 512) {
      const int vt = (a.n % 128 + 31) / 32;
      switch (a.n / 128) {
        case 0: return half_vt<0>(a, vt);
        case 1: return half_vt<1>(a, vt);
        case 2: return half_vt<2>(a, vt);
        case 3: return half_vt<3>(a, vt);
      }
    }
    const int nf = a.n / 256, vt = (a.n % 256 + 63) / 64;
    switch (nf) {
      case 0: return tail_vt<0>(a, vt);
      case 1: return tail_vt<1>(a, vt);
      case 2: return tail_vt<2>(a, vt);
      case 3: return tail_vt<3>(a, vt);
      case 4: return tail_vt<4>(a, vt);
    }
    return -1;
  }
};

template <typename TX, typename TW, typename TY>
struct RmsL {
  struct Args {
    const TX* x; const TW* w; TY* y; float* l2; int64_t rows; int n; float eps; int mode;
    hipStream_t s;
  };
  template <int VEC, int NC>
  static int run(const Args& a) {
    hipLaunchKernelGGL((rmsnorm_kernel<TX, TW, TY, VEC, NC>), dim3(ceil_div(a.rows, 4)),
                       dim3(256), 0, a.s, a.x, a.w, a.y, a.l2, a.rows, a.n, a.eps, a.mode);
    BLT_LAUNCH_CHECK("rmsnorm_kernel");
    return 0;
  }
  static int stream(const Args& a) {
    hipLaunchKernelGGL((rmsnorm_stream_kernel<TX, TW, TY>), dim3(ceil_div(a.rows, 4)), dim3(256),
                       0, a.s, a.x, a.w, a.y, a.l2, a.rows, a.n, a.eps, a.mode);
    BLT_LAUNCH_CHECK("rmsnorm_stream_kernel");
    return 0;
  }
};

struct SoftmaxL {
  struct Args { const float* x; float* y; int64_t rows; int n; hipStream_t s; };
  template <int VEC, int NC>
  static int run(const Args& a) {
    hipLaunchKernelGGL((softmax_kernel<VEC, NC>), dim3(ceil_div(a.rows, 4)), dim3(256), 0, a.s,
                       a.x, a.y, a.rows, a.n);
    BLT_LAUNCH_CHECK("softmax_kernel");
    return 0;
  }
  static int stream(const Args& a) {
    hipLaunchKernelGGL(softmax_stream_kernel, dim3(ceil_div(a.rows, 4)), dim3(256), 0, a.s, a.x,
                       a.y, a.rows, a.n);
    BLT_LAUNCH_CHECK("softmax_stream_kernel");
    return 0;
  }
};

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// One work item per thread: blocks dispatched in order sweep memory linearly,
// which measured faster on HBM than grid-stride loops over a capped grid
// (the kernels still loop, so any grid size is correct).
unsigned elementwise_grid(int64_t work) {
  int64_t g = (work + 255) / 256;
  if (g > 0x7fffffff) g = 0x7fffffff;
  return (unsigned)(g < 1 ? 1 : g);
}
}  // namespace

int launch_entropy_f32(const float* x, float* out, int64_t rows, int n, hipStream_t s) {
  if (rows == 0) return 0;
  if (n > 0 && n % 4 == 0 && n < 1280 && aligned(x, 16))
    return EntropyL<float>::fast({x, out, rows, n, s});
  return dispatch_row<EntropyL<float>>(n, aligned(x, 16), {x, out, rows, n, s});
}
int launch_entropy_bf16(const uint16_t* x, float* out, int64_t rows, int n, hipStream_t s) {
  if (rows == 0) return 0;
  if (n > 0 && n % 4 == 0 && n < 1280 && aligned(x, 8))
    return EntropyL<uint16_t>::fast({x, out, rows, n, s});
  return dispatch_row<EntropyL<uint16_t>>(n, aligned(x, 8), {x, out, rows, n, s});
}

template <typename TX, typename TW, typename TY>
int launch_rmsnorm(const TX* x, const TW* w, TY* y, float* l2, int64_t rows, int n, float eps,
                   int mode, hipStream_t s) {
  if (rows == 0) return 0;
  if constexpr (std::is_same<TX, uint16_t>::value && std::is_same<TW, uint16_t>::value &&
                std::is_same<TY, uint16_t>::value) {
    if (n % 8 == 0 && n > 0 && n <= 1024 && aligned(x, 16) && aligned(w, 16) &&
        (y == nullptr || aligned(y, 16))) {
      const unsigned grid = ceil_div(rows, 8);
      const int np = (2 * (n / 8) + 63) / 64;
#define BLT_RMS_PAIR(NP)                                                                 \
  hipLaunchKernelGGL(rmsnorm_bf16_pair_kernel<NP>, dim3(grid), dim3(256), 0, s, x, w, y, l2, \
                     rows, n, eps, mode);                                                \
  BLT_LAUNCH_CHECK("rmsnorm_bf16_pair_kernel");                                          \
  return 0;
      switch (np) {
        case 1: BLT_RMS_PAIR(1)
        case 2: BLT_RMS_PAIR(2)
        case 3: BLT_RMS_PAIR(3)
        default: BLT_RMS_PAIR(4)
      }
#undef BLT_RMS_PAIR
    }
  }
  const bool vec = aligned(x, 4 * sizeof(TX)) && aligned(w, 4 * sizeof(TW)) &&
                   aligned(y, 4 * sizeof(TY));
  return dispatch_row<RmsL<TX, TW, TY>>(n, vec, {x, w, y, l2, rows, n, eps, mode, s});
}
template int launch_rmsnorm<float, float, float>(const float*, const float*, float*, float*,
                                                 int64_t, int, float, int, hipStream_t);
template int launch_rmsnorm<uint16_t, uint16_t, uint16_t>(const uint16_t*, const uint16_t*,
                                                          uint16_t*, float*, int64_t, int, float,
                                                          int, hipStream_t);
template int launch_rmsnorm<float, float, uint16_t>(const float*, const float*, uint16_t*,
                                                    float*, int64_t, int, float, int,
                                                    hipStream_t);

int launch_softmax_f32(const float* x, float* y, int64_t rows, int n, hipStream_t s) {
  if (rows == 0) return 0;
  return dispatch_row<SoftmaxL>(n, aligned(x, 16) && aligned(y, 16), {x, y, rows, n, s});
}

int launch_silu_gate_f32(const float* g, const float* u, float* o, int64_t n, hipStream_t s) {
  if (n == 0) return 0;
  const int vec = aligned(g, 16) && aligned(u, 16) && aligned(o, 16);
  hipLaunchKernelGGL(silu_gate_f32_kernel, dim3(elementwise_grid(n / 4 + 1)), dim3(256), 0, s, g,
                     u, o, n, vec);
  BLT_LAUNCH_CHECK("silu_gate_f32_kernel");
  return 0;
}
int launch_silu_gate_bf16(const uint16_t* g, const uint16_t* u, uint16_t* o, int64_t n,
                          hipStream_t s) {
  if (n == 0) return 0;
  const int vec = aligned(g, 16) && aligned(u, 16) && aligned(o, 16);
  hipLaunchKernelGGL(silu_gate_bf16_kernel, dim3(elementwise_grid(n / 8 + 1)), dim3(256), 0, s,
                     g, u, o, n, vec);
  BLT_LAUNCH_CHECK("silu_gate_bf16_kernel");
  return 0;
}
int launch_coherence(const float* nrm, const float* ent, float* out, int64_t n, float eps,
                     hipStream_t s) {
  if (n == 0) return 0;
  hipLaunchKernelGGL(coherence_kernel, dim3(elementwise_grid(n)), dim3(256), 0, s, nrm, ent, out,
                     n, eps);
  BLT_LAUNCH_CHECK("coherence_kernel");
  return 0;
}
__global__ __launch_bounds__(256) void row_rstd_kernel(const float* __restrict__ ss,
                                                       float* __restrict__ rstd, int64_t rows,
                                                       int np, int dim, float eps) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float* s = ss + r * np;
  float t = 0.f;
  for (int q = 0; q < np; ++q) t += s[q];
  rstd[r] = 1.f / (sqrtf(t / (float)dim) + eps);
}

int launch_row_rstd(const float* ss, float* rstd, int64_t rows, int np, int dim, float eps,
                    hipStream_t s) {
  if (rows == 0) return 0;
  hipLaunchKernelGGL(row_rstd_kernel, dim3(ceil_div(rows, 256)), dim3(256), 0, s, ss, rstd, rows,
                     np, dim, eps);
  BLT_LAUNCH_CHECK("row_rstd_kernel");
  return 0;
}

int launch_embed(const int32_t* tok, const uint16_t* table, float* x, int64_t rows, int dim,
                 int vocab, hipStream_t s, uint16_t* xb, float* ss, const float* col_scale) {
  if (rows == 0) return 0;
  if ((xb != nullptr) != (ss != nullptr) || (xb && dim % 64) || (col_scale && !xb) ||
      (uintptr_t)col_scale % 16)
    return fail(BLT_ERR_SHAPE, "embed: xb and ss together, dim % 64 == 0, 16-byte col_scale");
  hipLaunchKernelGGL(embed_kernel, dim3(ceil_div(rows, 4)), dim3(256), 0, s, tok, table, x, rows,
                     dim, vocab, xb, ss, col_scale);
  BLT_LAUNCH_CHECK("embed_kernel");
  return 0;
}
int launch_rope(const uint16_t* src, uint16_t* dst, const float* cs, int64_t B, int64_t H,
                int64_t T, int d, int64_t sb, int64_t sh, int64_t st, hipStream_t s) {
  const int64_t total = B * H * T * (d / 2);
  if (total == 0) return 0;
  if (d == 64 && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0 && sb % 8 == 0 &&
      sh % 8 == 0 && st % 8 == 0) {
    hipLaunchKernelGGL(rope64_kernel, dim3(elementwise_grid(total / 8)), dim3(256), 0, s, src,
                       dst, cs, B, H, T, sb, sh, st);
    BLT_LAUNCH_CHECK("rope64_kernel");
    return 0;
  }
  hipLaunchKernelGGL(rope_kernel, dim3(elementwise_grid(total)), dim3(256), 0, s, src, dst, cs, B,
                     H, T, d, sb, sh, st);
  BLT_LAUNCH_CHECK("rope_kernel");
  return 0;
}
int launch_patch_boundaries(const float* H, int64_t B, int64_t T, float thr, int mode,
                            int32_t* mask, int32_t* starts, int32_t* lengths, int32_t* count,
                            hipStream_t s) {
  if (B == 0) return 0;
  hipLaunchKernelGGL(patch_boundary_kernel, dim3((unsigned)B), dim3(PB_THREADS), 0, s, H, T, thr,
                     mode, mask, starts, lengths, count, nullptr, nullptr);
  BLT_LAUNCH_CHECK("patch_boundary_kernel");
  return 0;
}

int launch_patch_mask_starts(const int32_t* mask, int64_t B, int64_t T, int32_t* starts,
                             int32_t* lengths, int32_t* count, hipStream_t s) {
  if (B == 0) return 0;
  hipLaunchKernelGGL(patch_boundary_kernel, dim3((unsigned)B), dim3(PB_THREADS), 0, s,
                     reinterpret_cast<const float*>(mask), T, 0.f, PB_MODE_MASK, nullptr, starts,
                     lengths, count, nullptr, nullptr);
  BLT_LAUNCH_CHECK("patch_boundary_kernel");
  return 0;
}

// ---------------------------------------------------------------------------
// ingest helpers
// ---------------------------------------------------------------------------
// Stitch packed-row outputs into per-document order: dest[i] >= 0 sends token
// i's entropy / norm / coherence there; -1 drops it (overlap context or
// padding).  C / Co may be null.
__global__ __launch_bounds__(256) void scatter_tokens_kernel(
    const int32_t* __restrict__ dest, const float* __restrict__ H, const float* __restrict__ N,
    const float* __restrict__ C, float* __restrict__ Ho, float* __restrict__ No,
    float* __restrict__ Co, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int32_t d = dest[i];
    if (d >= 0) {
      Ho[d] = H[i];
      No[d] = N[i];
      if (C) Co[d] = C[i];
    }
  }
}

// The same stitch for [n, dim] f32 rows (pre-norm embeddings): one wave per
// row, 16-byte loads and stores (dim % 4 == 0, rows 16-byte aligned).
__global__ __launch_bounds__(256) void scatter_rows_kernel(const int32_t* __restrict__ dest,
                                                           const float* __restrict__ X,
                                                           float* __restrict__ Xo, int64_t n,
                                                           int dim) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const int32_t d = dest[row];
  if (d < 0) return;
  const f32x4_t* src = reinterpret_cast<const f32x4_t*>(X + row * dim);
  f32x4_t* dst = reinterpret_cast<f32x4_t*>(Xo + (int64_t)d * dim);
  for (int c = threadIdx.x & 63; c < dim / 4; c += 64) dst[c] = src[c];
}

int launch_scatter_tokens(const int32_t* dest, const float* H, const float* N, const float* C,
                          float* Ho, float* No, float* Co, int64_t n, hipStream_t s) {
  if (n == 0) return 0;
  if ((C == nullptr) != (Co == nullptr)) return fail(BLT_ERR_INVALID, "scatter: C and Co pair");
  hipLaunchKernelGGL(scatter_tokens_kernel, dim3(elementwise_grid(n)), dim3(256), 0, s, dest, H,
                     N, C, Ho, No, Co, n);
  BLT_LAUNCH_CHECK("scatter_tokens_kernel");
  return 0;
}
int launch_scatter_rows(const int32_t* dest, const float* X, float* Xo, int64_t n, int dim,
                        hipStream_t s) {
  if (n == 0) return 0;
  if (dim % 4 || ((uintptr_t)X | (uintptr_t)Xo) % 16)
    return fail(BLT_ERR_SHAPE, "scatter_rows: dim % 4 == 0 and 16-byte aligned rows");
  hipLaunchKernelGGL(scatter_rows_kernel, dim3(ceil_div(n, 4)), dim3(256), 0, s, dest, X, Xo, n,
                     dim);
  BLT_LAUNCH_CHECK("scatter_rows_kernel");
  return 0;
}
int launch_patch_boundaries_varlen(const float* H, const int64_t* row_off, const int32_t* row_len,
                                   int64_t rows, float thr, int mode, int32_t* mask,
                                   int32_t* starts, int32_t* lengths, int32_t* count,
                                   hipStream_t s) {
  if (rows == 0) return 0;
  hipLaunchKernelGGL(patch_boundary_kernel, dim3((unsigned)rows), dim3(PB_THREADS), 0, s, H,
                     (int64_t)0, thr, mode, mask, starts, lengths, count, row_off, row_len);
  BLT_LAUNCH_CHECK("patch_boundary_kernel");
  return 0;
}

int launch_patch_means(const float* H, const float* N, const float* C, const int32_t* starts,
                       const int32_t* count, int64_t B, int64_t T, const int64_t* row_off,
                       const int32_t* row_len, float* mH, float* mN, float* mC, hipStream_t s,
                       const int64_t* out_off) {
  if (B == 0) return 0;
  if (C)
    hipLaunchKernelGGL(patch_means_kernel<true>, dim3((unsigned)B), dim3(PM_THREADS), 0, s, H, N,
                       C, starts, count, T, row_off, row_len, mH, mN, mC, out_off);
  else
    hipLaunchKernelGGL(patch_means_kernel<false>, dim3((unsigned)B), dim3(PM_THREADS), 0, s, H, N,
                       C, starts, count, T, row_off, row_len, mH, mN, mC, out_off);
  BLT_LAUNCH_CHECK("patch_means_kernel");
  return 0;
}

}  // namespace blt
