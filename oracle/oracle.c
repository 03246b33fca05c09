/*
 * oracle.c — CPU restatement of blt-burn's entropy-patching path, as the
 * reference computes it with `--no-default-features` on Burn's NdArray
 * backend (f32 tensors throughout).  TEST INFRASTRUCTURE ONLY: it is the
 * checker for the gfx950 library (tests/, __graft_entry__.smoke(), and the
 * cpu_baseline leg of bench.py) and is never linked into or called by the
 * product path.
 *
 * Each function cites the reference lines it restates (paths relative to
 * SashimiSaketoro/blt-burn).  The reference itself (Rust, Burn 0.19.1) cannot
 * be built in this image: no rustc/cargo and no vendored crates.
 *
 * Pinning (what checks each function independently of this file; the tests
 * name them):
 *   oracle_entropy        closed forms (zeros -> ln V, one-hot -> 0, bounds
 *                         0 <= H <= ln V), reference KATs, fp64 numpy
 *   oracle_rms_norm       fp64 numpy of model.rs:758-770 / rms_norm_kernel.rs
 *   oracle_l2_norm, oracle_softmax, oracle_silu_gate, oracle_coherence
 *                         fp64 numpy + invariants (rows sum to 1, [0,1])
 *   oracle_patch_*        hand-built vectors + brute force (bit-exact);
 *                         patch_means also: sum(mean * length) = row sum,
 *                         constant rows -> the constant, numpy fsum / length
 *   oracle_rope_table     fp64 closed form, identity at pos 0
 *   oracle_attention      fp64 numpy with a materialised mask; row 0 = v[0];
 *                         window >= T equals full causal
 *   oracle_attention_kernel  fp64 numpy (any Tq, Tkv, d); one key -> v[0];
 *                         equals oracle_attention when Tq = Tkv
 *   oracle_model_forward  fp64 numpy forward on tiny configs
 * The matmul/softmax summation order of burn-ndarray (matrixmultiply sgemm
 * blocking) is not reproduced; it moves results at the 1e-6 level only.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ---- patcher.rs:38-63 — entropy = -sum(exp(lsm) * lsm), lsm = log_softmax(x) --- */
EXPORT void oracle_entropy(const float* logits, float* out, int64_t rows, int32_t V) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = logits + r * V;
    float m = -INFINITY;
    for (int v = 0; v < V; ++v) m = x[v] > m ? x[v] : m;
    float s = 0.f;
    for (int v = 0; v < V; ++v) s += expf(x[v] - m);
    const float lse = logf(s);
    float h = 0.f;
    for (int v = 0; v < V; ++v) {
      const float lsm = (x[v] - m) - lse;
      h += expf(lsm) * lsm;
    }
    out[r] = -h;
  }
}

/* ---- model.rs:758-770 (mode 0: eps after sqrt); rms_norm_kernel.rs:40-43 (mode 1) ---- */
EXPORT void oracle_rms_norm(const float* x, const float* w, float* y, int64_t rows, int32_t D,
                            float eps, int32_t mode) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * D;
    float ss = 0.f;
    for (int d = 0; d < D; ++d) ss += xr[d] * xr[d];
    const float ms = ss / (float)D;
    const float norm = mode == 0 ? sqrtf(ms) + eps : sqrtf(ms + eps);
    for (int d = 0; d < D; ++d) y[r * D + d] = (xr[d] / norm) * w[d];
  }
}

/* ---- model.rs:291-300, backend.rs:572-580 — sqrt(sum x^2) ---- */
EXPORT void oracle_l2_norm(const float* x, float* out, int64_t rows, int32_t D) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float ss = 0.f;
    for (int d = 0; d < D; ++d) ss += x[r * D + d] * x[r * D + d];
    out[r] = sqrtf(ss);
  }
}

/* ---- burn activation::softmax over the last dim (backend.rs:508-540) ---- */
EXPORT void oracle_softmax(const float* x, float* y, int64_t rows, int32_t N) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * N;
    float m = -INFINITY;
    for (int j = 0; j < N; ++j) m = xr[j] > m ? xr[j] : m;
    float s = 0.f;
    for (int j = 0; j < N; ++j) {
      y[r * N + j] = expf(xr[j] - m);
      s += y[r * N + j];
    }
    for (int j = 0; j < N; ++j) y[r * N + j] /= s;
  }
}

/* ---- model.rs:727-731 / backend.rs:583-593 — silu(g) * u, silu = x * sigmoid(x) ---- */
EXPORT void oracle_silu_gate(const float* g, const float* u, float* out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = (g[i] * (1.f / (1.f + expf(-g[i])))) * u[i];
}

/* ---- model.rs:311-313 / backend.rs:596-608 — n^2 / (H + eps) ---- */
EXPORT void oracle_coherence(const float* n, const float* H, float* out, int64_t count,
                             float eps) {
  for (int64_t i = 0; i < count; ++i) out[i] = (n[i] * n[i]) / (H[i] + eps);
}

/* ---- patcher.rs:80-118 — monotonic mask (mode 0); mode 1: same layout with H[t] > thr ---- */
EXPORT void oracle_patch_mask(const float* H, int64_t B, int64_t T, float thr, int32_t mode,
                              int32_t* mask) {
  for (int64_t b = 0; b < B; ++b) {
    const float* h = H + b * T;
    int32_t* m = mask + b * T;
    if (T == 0) continue;
    if (T <= 2) { /* T == 1 -> [1]; T == 2 -> [1, 1]  (patcher.rs:90-98) */
      for (int64_t t = 0; t < T; ++t) m[t] = 1;
      continue;
    }
    m[0] = 1;
    m[1] = 1;
    for (int64_t t = 2; t < T; ++t) {
      if (mode == 0) {
        const float diff = h[t] - h[t - 1]; /* entropies[:, 2:] - entropies[:, 1:-1] */
        m[t] = diff > thr ? 1 : 0;
      } else {
        m[t] = h[t] > thr ? 1 : 0;
      }
    }
  }
}

/* ---- patcher.rs:124-142 — indices of mask == 1 per row ---- */
EXPORT void oracle_patch_indices(const int32_t* mask, int64_t B, int64_t T, int32_t* starts,
                                 int32_t* counts) {
  for (int64_t b = 0; b < B; ++b) {
    int32_t c = 0;
    for (int64_t t = 0; t < T; ++t)
      if (mask[b * T + t] == 1) starts[b * T + c++] = (int32_t)t;
    counts[b] = c;
  }
}

/* ---- patcher.rs:144-164 — lengths: next start (or seq_len) minus start ---- */
EXPORT void oracle_patch_lengths(const int32_t* starts, const int32_t* counts, int64_t B,
                                 int64_t T, int32_t* lengths) {
  for (int64_t b = 0; b < B; ++b)
    for (int32_t i = 0; i < counts[b]; ++i) {
      const int32_t s = starts[b * T + i];
      const int32_t e = i + 1 < counts[b] ? starts[b * T + i + 1] : (int32_t)T;
      lengths[b * T + i] = e - s;
    }
}

/* ---- pipeline.rs:240-258 — compute_mean_entropy / compute_mean_prominence:
 * sum of the patch's values, left to right in f32, over its length (0 for an
 * empty range); huggingface_loader.rs:265-295 averages coherence the same way.
 * Patch i of row b covers [starts[b*T + i], next start or T).  C / mC may be NULL. */
EXPORT void oracle_patch_means(const float* H, const float* N, const float* C,
                               const int32_t* starts, const int32_t* counts, int64_t B,
                               int64_t T, float* mH, float* mN, float* mC) {
  for (int64_t b = 0; b < B; ++b)
    for (int32_t i = 0; i < counts[b]; ++i) {
      int64_t e = i + 1 < counts[b] ? starts[b * T + i + 1] : T;
      if (e > T) e = T;
      int64_t s = starts[b * T + i];
      if (s > e) s = e;
      float sh = 0.0f, sn = 0.0f, sc = 0.0f;
      for (int64_t t = s; t < e; ++t) {
        sh += H[b * T + t];
        sn += N[b * T + t];
        if (C) sc += C[b * T + t];
      }
      const float len = (float)(e - s);
      mH[b * T + i] = e > s ? sh / len : 0.0f;
      mN[b * T + i] = e > s ? sn / len : 0.0f;
      if (mC) mC[b * T + i] = e > s ? sc / len : 0.0f;
    }
}

/* ---- model.rs:24-52 — inv_freq = 1f32 / (f32)theta^(2i/d); angle = (f32)pos * inv_freq ---- */
EXPORT void oracle_rope_table(float* out, int32_t head_dim, int32_t max_seqlen, double theta) {
  const int half = head_dim / 2;
  float* inv = (float*)malloc(sizeof(float) * (size_t)half);
  for (int i = 0; i < half; ++i) {
    const float p = (float)pow(theta, (double)(2 * i) / (double)head_dim);
    inv[i] = 1.0f / p;
  }
  for (int pos = 0; pos < max_seqlen; ++pos) {
    const float fp = (float)pos;
    for (int i = 0; i < half; ++i) {
      const float ang = fp * inv[i];
      out[((int64_t)pos * half + i) * 2] = cosf(ang);
      out[((int64_t)pos * half + i) * 2 + 1] = sinf(ang);
    }
  }
  free(inv);
}

/* ---- model.rs:107-147 — half-split rotation of one [d] row at position pos ---- */
static void rope_row(float* x, const float* cs, int64_t pos, int d) {
  const int half = d / 2;
  for (int m = 0; m < half; ++m) {
    const float c = cs[(pos * half + m) * 2], s = cs[(pos * half + m) * 2 + 1];
    const float x1 = x[m], x2 = x[m + half];
    x[m] = x1 * c - x2 * s;
    x[m + half] = x1 * s + x2 * c;
  }
}

/* visibility of key j for query i (model.rs:153-165 plus the optional window) */
static int visible(int64_t i, int64_t j, int causal, int window) {
  if (!causal) return 1;
  if (j > i) return 0;
  if (window > 0 && j <= i - window) return 0;
  return 1;
}

/* One (b, h) head: q, k, v [T, d] with row stride `st`; o [T, d] row stride `so`.
 * scores = (q . k) / sqrt(d) + mask; softmax; o = p . v   (model.rs:653-667) */
static void attend_head(const float* q, const float* k, const float* v, float* o, int64_t T,
                        int d, int64_t st, int64_t so, int causal, int window, float* sc) {
  const float scale = sqrtf((float)d);
  for (int64_t i = 0; i < T; ++i) {
    float m = -INFINITY;
    for (int64_t j = 0; j < T; ++j) {
      if (!visible(i, j, causal, window)) {
        sc[j] = -INFINITY;
        continue;
      }
      float dot = 0.f;
      for (int e = 0; e < d; ++e) dot += q[i * st + e] * k[j * st + e];
      sc[j] = dot / scale;
      m = sc[j] > m ? sc[j] : m;
    }
    float s = 0.f;
    for (int64_t j = 0; j < T; ++j) {
      sc[j] = expf(sc[j] - m);
      s += sc[j];
    }
    for (int e = 0; e < d; ++e) o[i * so + e] = 0.f;
    for (int64_t j = 0; j < T; ++j) {
      const float p = sc[j] / s;
      if (p == 0.f) continue;
      for (int e = 0; e < d; ++e) o[i * so + e] += p * v[j * st + e];
    }
  }
}

/* ---- fused_attention semantics (backend.rs:611-651) + RoPE and window:
 * q, k, v, o f32 [B, H, T, d] head-major; rope_theta > 0 rotates q and k first. ---- */
EXPORT void oracle_attention(const float* q, const float* k, const float* v, float* o, int64_t B,
                             int64_t H, int64_t T, int32_t d, int32_t causal, int32_t window,
                             double rope_theta) {
  float* cs = NULL;
  if (rope_theta > 0) {
    cs = (float*)malloc(sizeof(float) * (size_t)(T * d));
    oracle_rope_table(cs, d, (int32_t)T, rope_theta);
  }
#pragma omp parallel for schedule(dynamic)
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const int64_t off = bh * T * d;
    float* qr = (float*)malloc(sizeof(float) * (size_t)(T * d));
    float* kr = (float*)malloc(sizeof(float) * (size_t)(T * d));
    float* sc = (float*)malloc(sizeof(float) * (size_t)T);
    memcpy(qr, q + off, sizeof(float) * (size_t)(T * d));
    memcpy(kr, k + off, sizeof(float) * (size_t)(T * d));
    if (cs)
      for (int64_t t = 0; t < T; ++t) {
        rope_row(qr + t * d, cs, t, d);
        rope_row(kr + t * d, cs, t, d);
      }
    attend_head(qr, kr, v + off, o + off, T, d, d, d, causal, window, sc);
    free(qr);
    free(kr);
    free(sc);
  }
  free(cs);
}

/* ---- fused_attention_kernel (attention_kernel.rs:20-125, launched by
 * backend.rs:334-383): q [B, H, Tq, d], k / v [B, H, Tkv, d], one query at a
 * time in three passes exactly as the kernel does them: the max of the visible
 * scores, the sum of exp(score - max), then for each d the sum of
 * exp(score - max) / sum * v.  score = (q . k) * (1 / sqrt(d)) in f32; with
 * causal, key j is visible to query i iff j <= i (the same indices for any Tq
 * and Tkv).  A query that sees no key gets 0. ---- */
EXPORT void oracle_attention_kernel(const float* q, const float* k, const float* v, float* o,
                                    int64_t B, int64_t H, int64_t Tq, int64_t Tkv, int32_t d,
                                    int32_t causal) {
  const float scale = 1.0f / sqrtf((float)d);
#pragma omp parallel for schedule(dynamic)
  for (int64_t bhq = 0; bhq < B * H * Tq; ++bhq) {
    const int64_t bh = bhq / Tq, i = bhq % Tq;
    const float* qr = q + (bh * Tq + i) * d;
    const float* kb = k + bh * Tkv * d;
    const float* vb = v + bh * Tkv * d;
    float* orow = o + (bh * Tq + i) * d;
    float mx = -INFINITY;
    for (int64_t j = 0; j < Tkv; ++j) {
      if (causal && j > i) continue;
      float dot = 0.f;
      for (int e = 0; e < d; ++e) dot += qr[e] * kb[j * d + e];
      const float sc = dot * scale;
      mx = sc > mx ? sc : mx;
    }
    float sum = 0.f;
    for (int64_t j = 0; j < Tkv; ++j) {
      if (causal && j > i) continue;
      float dot = 0.f;
      for (int e = 0; e < d; ++e) dot += qr[e] * kb[j * d + e];
      sum += expf(dot * scale - mx);
    }
    for (int e = 0; e < d; ++e) {
      float acc = 0.f;
      for (int64_t j = 0; j < Tkv; ++j) {
        if (causal && j > i) continue;
        float dot = 0.f;
        for (int e2 = 0; e2 < d; ++e2) dot += qr[e2] * kb[j * d + e2];
        acc += expf(dot * scale - mx) / sum * vb[j * d + e];
      }
      orow[e] = acc;
    }
  }
}

/* ---- the entropy model ------------------------------------------------------ */

typedef struct oracle_cfg {
  int32_t dim, n_layers, n_heads, hidden, vocab, max_seqlen;
  float norm_eps, rope_theta;
  int32_t window;
} oracle_cfg;

/* f32 weights in the reference layouts (Burn Linear weight [in, out]), per layer
 * concatenated: emb [V,D]; attn_norm, ffn_norm [L,D]; wq,wk,wv,wo [L,D,D];
 * w1,w3 [L,D,F]; w2 [L,F,D]; norm [D]; out [D,V]. */
typedef struct oracle_weights {
  const float *emb, *attn_norm, *ffn_norm, *wq, *wk, *wv, *wo, *w1, *w2, *w3, *norm, *out;
} oracle_weights;

/* y[M, N] = x[M, K] . W[K, N]  (nn::Linear without bias) */
static void linear(const float* x, const float* W, float* y, int64_t M, int64_t K, int64_t N) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i) {
    float* yr = y + i * N;
    for (int64_t n = 0; n < N; ++n) yr[n] = 0.f;
    for (int64_t kk = 0; kk < K; ++kk) {
      const float a = x[i * K + kk];
      const float* wr = W + kk * N;
      for (int64_t n = 0; n < N; ++n) yr[n] += a * wr[n];
    }
  }
}

/* ---- model.rs:269-322 forward_with_embeddings; tokens [B, T] int32.
 * outputs (any may be NULL): logits [B,T,V], pre [B,T,D], norms [B,T], H [B,T], coh [B,T] ---- */
EXPORT void oracle_model_forward(const oracle_cfg* c, const oracle_weights* w,
                                 const int32_t* tokens, int64_t B, int64_t T, float* logits,
                                 float* pre, float* norms, float* ent, float* coh) {
  const int64_t D = c->dim, F = c->hidden, V = c->vocab, L = c->n_layers, Hn = c->n_heads;
  const int64_t hd = D / Hn, M = B * T;
  float* x = (float*)malloc(sizeof(float) * (size_t)(M * D));
  float* a = (float*)malloc(sizeof(float) * (size_t)(M * D));
  float* q = (float*)malloc(sizeof(float) * (size_t)(M * D));
  float* k = (float*)malloc(sizeof(float) * (size_t)(M * D));
  float* v = (float*)malloc(sizeof(float) * (size_t)(M * D));
  float* att = (float*)malloc(sizeof(float) * (size_t)(M * D));
  float* h1 = (float*)malloc(sizeof(float) * (size_t)(M * F));
  float* h3 = (float*)malloc(sizeof(float) * (size_t)(M * F));
  float* lg = (float*)malloc(sizeof(float) * (size_t)(M * V));
  float* nr = (float*)malloc(sizeof(float) * (size_t)M);
  float* en = (float*)malloc(sizeof(float) * (size_t)M);
  float* cs = (float*)malloc(sizeof(float) * (size_t)(c->max_seqlen * hd));
  oracle_rope_table(cs, (int32_t)hd, c->max_seqlen, c->rope_theta); /* model.rs:278-279 */

  /* tok_embeddings.forward (model.rs:275) */
  for (int64_t r = 0; r < M; ++r) memcpy(x + r * D, w->emb + (int64_t)tokens[r] * D, sizeof(float) * D);

  for (int64_t l = 0; l < L; ++l) {
    /* h = x + attention(attention_norm(x))  (model.rs:515-520) */
    oracle_rms_norm(x, w->attn_norm + l * D, a, M, (int32_t)D, c->norm_eps, 0);
    linear(a, w->wq + l * D * D, q, M, D, D);
    linear(a, w->wk + l * D * D, k, M, D, D);
    linear(a, w->wv + l * D * D, v, M, D, D);
#pragma omp parallel for schedule(dynamic)
    for (int64_t bh = 0; bh < B * Hn; ++bh) {
      const int64_t b = bh / Hn, h = bh % Hn;
      float* sc = (float*)malloc(sizeof(float) * (size_t)T);
      float* qb = q + b * T * D + h * hd; /* [T, hd] rows of stride D */
      float* kb = k + b * T * D + h * hd;
      for (int64_t t = 0; t < T; ++t) { /* apply_rotary_emb (model.rs:641) */
        rope_row(qb + t * D, cs, t, (int)hd);
        rope_row(kb + t * D, cs, t, (int)hd);
      }
      attend_head(qb, kb, v + b * T * D + h * hd, att + b * T * D + h * hd, T, (int)hd, D, D, 1,
                  c->window, sc);
      free(sc);
    }
    linear(att, w->wo + l * D * D, a, M, D, D);
    for (int64_t i = 0; i < M * D; ++i) x[i] += a[i];
    /* x = h + feed_forward(ffn_norm(h))  (model.rs:521, 727-731) */
    oracle_rms_norm(x, w->ffn_norm + l * D, a, M, (int32_t)D, c->norm_eps, 0);
    linear(a, w->w1 + l * D * F, h1, M, D, F);
    linear(a, w->w3 + l * D * F, h3, M, D, F);
    oracle_silu_gate(h1, h3, h1, M * F);
    linear(h1, w->w2 + l * F * D, a, M, F, D);
    for (int64_t i = 0; i < M * D; ++i) x[i] += a[i];
  }
  if (pre) memcpy(pre, x, sizeof(float) * (size_t)(M * D)); /* model.rs:291 */
  oracle_l2_norm(x, nr, M, (int32_t)D);                      /* model.rs:296-300 */
  oracle_rms_norm(x, w->norm, a, M, (int32_t)D, c->norm_eps, 0); /* model.rs:303 */
  linear(a, w->out, lg, M, D, V);                            /* model.rs:304 */
  oracle_entropy(lg, en, M, (int32_t)V);                     /* model.rs:307 */
  if (logits) memcpy(logits, lg, sizeof(float) * (size_t)(M * V));
  if (norms) memcpy(norms, nr, sizeof(float) * (size_t)M);
  if (ent) memcpy(ent, en, sizeof(float) * (size_t)M);
  if (coh) oracle_coherence(nr, en, coh, M, 1e-6f);          /* model.rs:311-313 */
  free(x); free(a); free(q); free(k); free(v); free(att); free(h1); free(h3);
  free(lg); free(nr); free(en); free(cs);
}
