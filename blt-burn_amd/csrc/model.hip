// LMTransformer::forward_with_embeddings (model.rs:269-322) on gfx950.
//
// Device layout (one model handle per GPU):
//   packed weights, bf16, "Bt" = [out, in] so both MFMA operands read K-contiguous:
//     wqkv [L, 3D, D]   rows 0..D-1 = wq^T, D..2D-1 = wk^T, 2D..3D-1 = wv^T
//     wo   [L, D, D]    wo^T
//     w13  [L, 2F, D]   64-row groups: rows 64g..64g+31 = w1^T rows 32g..32g+31,
//                       rows 64g+32..64g+63 = w3^T rows 32g..32g+31 (gate/up pairs
//                       land in one lane of the GEMM epilogue)
//     w2   [L, D, F]    w2^T
//     wout [V, D]       output^T
//   norm weights f32: attn_nw [L, D], ffn_nw [L, D], final_norm [D]; the RoPE
//   cos/sin table [max_seqlen, 32, 2] f32.
//   workspace for max_tokens rows: residual x f32 [M, D], bf16 copy of the
//   residual times the next projection's norm weight (or of the final normed
//   rows) [M, D], per-64-column sums of
//   squares of the residual f32 [M, D / 64] and the row factors 1 / (rms +
//   eps) f32 [M] made from them, qkv bf16 [M, 3D] (q, k already
//   rotated), attention out bf16 [M, D], FFN hidden bf16 [M, F], logits f32
//   [M, V], entropies/norms f32 [M].
//
// Per layer: QKV GEMM (RMSNorm scale + RoPE) -> attention -> O GEMM (+=
// residual, bf16 copy + sums of squares) -> W1|W3 GEMM (RMSNorm scale +
// SiLU*gate) -> W2 GEMM (+= residual, bf16 copy + sums of squares).  The
// RMSNorm before each projection (model.rs:508-522, 758-770) is thereby split
// between the GEMM that produces the residual and the GEMM that consumes it:
// RMSNorm(x) W = (x * w) W / (rms(x) + eps).  The producer's epilogue writes
// A = bf16(x * w) (one rounding of the f32 product, as bf16(RMSNorm(x))
// would have) and the consumer applies the per-row factor to its
// accumulators; the projection weights stay exactly the bf16 values given.
#include "model.hpp"

#include <math.h>
#include <string.h>

#include <vector>

namespace blt {

void rope_table_host(float* out, int head_dim, int max_seqlen, double theta) {
  // precompute_freqs_cis (model.rs:24-52): inv_freq = 1f32 / (f32)theta^(2i/d),
  // angle = (f32)pos * inv_freq, in f32, stored (cos, sin) per (pos, i).
  const int half = head_dim / 2;
  std::vector<float> inv(half);
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
}

namespace {
template <typename T>
int dalloc(T** p, int64_t n, int64_t* total) {
  if (n <= 0) {
    *p = nullptr;
    return 0;
  }
  hipError_t e = hipMalloc((void**)p, (size_t)n * sizeof(T));
  if (e != hipSuccess) return fail(-4, std::string("hipMalloc failed: ") + hipGetErrorString(e));
  *total += n * (int64_t)sizeof(T);
  return 0;
}
}  // namespace

int Model::mark(int stage, hipStream_t s) {
  if (!profiling) return 0;
  if (ev_used == ev_pool.size()) {
    hipEvent_t e;
    BLT_HIP_CHECK(hipEventCreate(&e));
    ev_pool.push_back(e);
  }
  BLT_HIP_CHECK(hipEventRecord(ev_pool[ev_used], s));
  ev_marks.emplace_back(stage, ev_used);
  ev_stream = s;
  ++ev_used;
  return 0;
}

// Add the time between consecutive marks to the per-stage totals (stage -1 =
// the start mark of a forward), then recycle the events.
int Model::fold_profile() {
  if (ev_marks.empty()) return 0;
  BLT_HIP_CHECK(hipEventSynchronize(ev_pool[ev_marks.back().second]));
  for (size_t i = 1; i < ev_marks.size(); ++i) {
    const int st = ev_marks[i].first;
    if (st < 0 || st >= BLT_NUM_STAGES) continue;
    float t = 0.f;
    BLT_HIP_CHECK(hipEventElapsedTime(&t, ev_pool[ev_marks[i - 1].second],
                                      ev_pool[ev_marks[i].second]));
    acc_ms[st] += t;
    acc_n[st] += 1;
  }
  ev_marks.clear();
  ev_used = 0;
  return 0;
}

int Model::read_profile(double* ms, int64_t* launches, int n) {
  const int rc = fold_profile();
  for (int i = 0; i < n; ++i) {
    ms[i] = i < BLT_NUM_STAGES ? acc_ms[i] : 0.0;
    launches[i] = i < BLT_NUM_STAGES ? acc_n[i] : 0;
  }
  for (int i = 0; i < BLT_NUM_STAGES; ++i) {
    acc_ms[i] = 0.0;
    acc_n[i] = 0;
  }
  return rc;
}

Model::~Model() {
  for (hipEvent_t e : ev_pool) (void)hipEventDestroy(e);
  void* ptrs[] = {emb, final_norm, attn_nw, ffn_nw, wqkv, wo,   w13,  w2,     wout, wout_head,
                  rope_cs, x,     a,       ss,     rstd, qkv,  attn, hbuf, logits, ent, norms};
  int prev = -1;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(device);
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  if (prev >= 0) (void)hipSetDevice(prev);
}

int Model::create(int dev, const blt_model_config& c, const blt_model_weights& w,
                  int64_t max_tok, Model** out) {
  if (c.dim <= 0 || c.n_heads <= 0 || c.dim % c.n_heads != 0 || c.dim / c.n_heads != 64)
    return fail(-2, "model: head_dim = dim / n_heads must be 64");
  if (c.dim % 64 != 0) return fail(-2, "model: dim must be a multiple of 64");
  if (c.ffn_hidden <= 0 || c.ffn_hidden % 64 != 0)
    return fail(-2, "model: ffn_hidden must be a positive multiple of 64");
  if (c.vocab <= 0 || c.n_layers < 0 || c.max_seqlen <= 0 || max_tok <= 0)
    return fail(-2, "model: bad vocab / n_layers / max_seqlen / max_tokens");
  if (c.window < 0) return fail(-2, "model: window must be >= 0");
  if (!w.tok_embeddings || !w.norm || !w.output)
    return fail(-1, "model: null embedding / norm / output weight");
  if (c.n_layers > 0) {
    const void* per_layer[] = {w.attention_norm, w.ffn_norm, w.wq, w.wk, w.wv,
                               w.wo,             w.w1,       w.w2, w.w3};
    for (const void* q : per_layer)
      if (q == nullptr) return fail(-1, "model: null per-layer weight pointer");
  }
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || dev < 0 || dev >= ndev)
    return fail(-5, "model: no such HIP device");
  BLT_HIP_CHECK(hipSetDevice(dev));

  Model* m = new Model();
  m->device = dev;
  m->cfg = c;
  m->max_tokens = max_tok;
  const int64_t D = c.dim, F = c.ffn_hidden, V = c.vocab, L = c.n_layers;
  int64_t& tb = m->bytes;
  int rc = 0;
  rc |= dalloc(&m->emb, V * D, &tb);
  rc |= dalloc(&m->final_norm, D, &tb);
  rc |= dalloc(&m->attn_nw, L * D, &tb);
  rc |= dalloc(&m->ffn_nw, L * D, &tb);
  rc |= dalloc(&m->wqkv, L * 3 * D * D, &tb);
  rc |= dalloc(&m->wo, L * D * D, &tb);
  rc |= dalloc(&m->w13, L * 2 * F * D, &tb);
  rc |= dalloc(&m->w2, L * D * F, &tb);
  rc |= dalloc(&m->wout, V * D, &tb);
  if (head_fused_ok((int)D, (int)V)) rc |= dalloc(&m->wout_head, head_packed_elems((int)D), &tb);
  rc |= dalloc(&m->rope_cs, (int64_t)c.max_seqlen * 64, &tb);
  rc |= dalloc(&m->x, max_tok * D, &tb);
  rc |= dalloc(&m->a, max_tok * D, &tb);
  rc |= dalloc(&m->ss, max_tok * (D / 64), &tb);
  rc |= dalloc(&m->rstd, max_tok, &tb);
  rc |= dalloc(&m->qkv, max_tok * 3 * D, &tb);
  rc |= dalloc(&m->attn, max_tok * D, &tb);
  rc |= dalloc(&m->hbuf, max_tok * F, &tb);
  rc |= dalloc(&m->logits, max_tok * V, &tb);
  rc |= dalloc(&m->ent, max_tok, &tb);
  rc |= dalloc(&m->norms, max_tok, &tb);
  if (rc) {
    delete m;
    return -4;
  }

  // ---- pack on the host, copy once ----
  auto up = [&](void* dst, const void* src, int64_t bytes) -> int {
    BLT_HIP_CHECK(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyHostToDevice));
    return 0;
  };
  auto to_f32 = [](const uint16_t* s, int64_t n) {
    std::vector<float> v(n);
    for (int64_t i = 0; i < n; ++i) v[i] = bf16_to_f32(s[i]);
    return v;
  };
  // Bt[n][k] = W[k][n] for a [K, N] Burn Linear weight
  auto transpose_into = [](uint16_t* dst, const uint16_t* W, int64_t K, int64_t N) {
    for (int64_t k = 0; k < K; ++k)
      for (int64_t n = 0; n < N; ++n) dst[n * K + k] = W[k * N + n];
  };
  if ((rc = up(m->emb, w.tok_embeddings, V * D * 2))) { delete m; return rc; }
  {
    std::vector<float> f = to_f32(w.norm, D);
    if ((rc = up(m->final_norm, f.data(), D * 4))) { delete m; return rc; }
    std::vector<uint16_t> t(V * D);
    transpose_into(t.data(), w.output, D, V);
    if ((rc = up(m->wout, t.data(), V * D * 2))) { delete m; return rc; }
    if (m->wout_head) {
      std::vector<uint16_t> hp(head_packed_elems((int)D));
      pack_head_weights(t.data(), (int)V, (int)D, hp.data());
      if ((rc = up(m->wout_head, hp.data(), (int64_t)hp.size() * 2))) { delete m; return rc; }
    }
  }
  if (L > 0) {
    std::vector<float> f = to_f32(w.attention_norm, L * D);
    if ((rc = up(m->attn_nw, f.data(), L * D * 4))) { delete m; return rc; }
    f = to_f32(w.ffn_norm, L * D);
    if ((rc = up(m->ffn_nw, f.data(), L * D * 4))) { delete m; return rc; }
  }
  std::vector<uint16_t> tmp;
  for (int64_t l = 0; l < L; ++l) {
    tmp.assign(3 * D * D, 0);
    transpose_into(tmp.data(), w.wq + l * D * D, D, D);
    transpose_into(tmp.data() + D * D, w.wk + l * D * D, D, D);
    transpose_into(tmp.data() + 2 * D * D, w.wv + l * D * D, D, D);
    if ((rc = up(m->wqkv + l * 3 * D * D, tmp.data(), 3 * D * D * 2))) { delete m; return rc; }
    tmp.assign(D * D, 0);
    transpose_into(tmp.data(), w.wo + l * D * D, D, D);
    if ((rc = up(m->wo + l * D * D, tmp.data(), D * D * 2))) { delete m; return rc; }
    // w13 interleave in 32-row groups
    tmp.assign(2 * F * D, 0);
    const uint16_t* w1 = w.w1 + l * D * F;
    const uint16_t* w3 = w.w3 + l * D * F;
    for (int64_t n = 0; n < 2 * F; ++n) {
      const int64_t g = n / 64, cc = n % 64;
      const uint16_t* src = cc < 32 ? w1 : w3;
      const int64_t col = 32 * g + (cc & 31);
      for (int64_t k = 0; k < D; ++k) tmp[n * D + k] = src[k * F + col];
    }
    if ((rc = up(m->w13 + l * 2 * F * D, tmp.data(), 2 * F * D * 2))) { delete m; return rc; }
    tmp.assign(D * F, 0);
    transpose_into(tmp.data(), w.w2 + l * F * D, F, D);
    if ((rc = up(m->w2 + l * D * F, tmp.data(), D * F * 2))) { delete m; return rc; }
  }
  {
    std::vector<float> cs((size_t)c.max_seqlen * 64);
    rope_table_host(cs.data(), 64, c.max_seqlen, c.rope_theta);
    if ((rc = up(m->rope_cs, cs.data(), (int64_t)cs.size() * 4))) { delete m; return rc; }
  }
  *out = m;
  return 0;
}

int Model::forward(const int32_t* tokens, int64_t B, int64_t T, const blt_model_outputs& o,
                   hipStream_t s, const int32_t* seg_start) {
  if (tokens == nullptr) return fail(-1, "forward: tokens is null");
  if (B < 0 || T < 0) return fail(-2, "forward: negative shape");
  if (T > cfg.max_seqlen) return fail(-2, "forward: seq_len exceeds max_seqlen");
  const int64_t M = B * T;
  if (M > max_tokens) return fail(-2, "forward: B*T exceeds the model's max_tokens");
  if (M == 0) return 0;
  BLT_HIP_CHECK(hipSetDevice(device));
  const int64_t D = cfg.dim, F = cfg.ffn_hidden, V = cfg.vocab, H = cfg.n_heads;
  // The residual stream lives in the caller's pre_norm_embeddings buffer when
  // one is given (it is exactly the value to return), else in the workspace.
  float* xr = o.pre_norm_embeddings ? o.pre_norm_embeddings : x;
  int rc;
  if (profiling && ev_used + 16 * (cfg.n_layers + 1) > 4096) {
    // keep the event pool bounded: wait for the marks so far and sum them
    if ((rc = fold_profile())) return rc;
  }
  if ((rc = mark(-1, s))) return rc;
  // layer 0 reads the embedding rows as bf16 plus their sums of squares
  const bool carry = cfg.n_layers > 0;
  if ((rc = launch_embed(tokens, emb, xr, M, (int)D, (int)V, s, carry ? a : nullptr,
                         carry ? ss : nullptr, carry ? attn_nw : nullptr)))
    return rc;
  const int np = (int)(D / 64);
  if (carry && (rc = launch_row_rstd(ss, rstd, M, np, (int)D, cfg.norm_eps, s))) return rc;
  if ((rc = mark(BLT_STAGE_EMBED, s))) return rc;
  for (int64_t l = 0; l < cfg.n_layers; ++l) {
    GemmArgs g{};
    g.A = a; g.Bt = wqkv + l * 3 * D * D; g.C = qkv;
    g.M = M; g.N = 3 * D; g.K = D; g.lda = D; g.ldb = D; g.ldc = 3 * D;
    g.epi = EPI_QKV_ROPE; g.rope_cols = (int)(2 * D); g.seq_len = T; g.rope_cs = rope_cs;
    // q leaves the GEMM scaled by log2(e) / sqrt(head_dim) (one bf16 rounding):
    // the attention kernel's scores then come out of the MFMA in the log2 domain
    g.q_cols = (int)D; g.q_scale = kAttnQScale;
    g.seg_start = seg_start;
    g.row_scale = rstd;
    if ((rc = launch_gemm(g, s))) return rc;
    if ((rc = mark(BLT_STAGE_QKV_GEMM, s))) return rc;
    AttnArgs at{};
    at.q = qkv; at.k = qkv + D; at.v = qkv + 2 * D; at.o = attn;
    at.B = B; at.H = H; at.T = T;
    at.sb_q = T * 3 * D; at.sh_q = 64; at.st_q = 3 * D;
    at.sb_k = T * 3 * D; at.sh_k = 64; at.st_k = 3 * D;
    at.sb_v = T * 3 * D; at.sh_v = 64; at.st_v = 3 * D;
    at.sb_o = T * D; at.sh_o = 64; at.st_o = D;
    at.causal = 1; at.window = cfg.window; at.seg_start = seg_start; at.q_prescaled = 1;
    if ((rc = launch_attention(at, s))) return rc;
    if ((rc = mark(BLT_STAGE_ATTENTION, s))) return rc;
    g = GemmArgs{};
    g.A = attn; g.Bt = wo + l * D * D; g.C = xr;
    g.M = M; g.N = D; g.K = D; g.lda = D; g.ldb = D; g.ldc = D; g.epi = EPI_RESID_F32;
    g.xb_out = a; g.ss_out = ss; g.ss_np = np; g.col_scale = ffn_nw + l * D;
    if ((rc = launch_gemm(g, s))) return rc;
    if ((rc = launch_row_rstd(ss, rstd, M, np, (int)D, cfg.norm_eps, s))) return rc;
    if ((rc = mark(BLT_STAGE_O_GEMM, s))) return rc;
    g = GemmArgs{};
    g.A = a; g.Bt = w13 + l * 2 * F * D; g.C = hbuf;
    g.M = M; g.N = 2 * F; g.K = D; g.lda = D; g.ldb = D; g.ldc = F; g.epi = EPI_SILU_GATE;
    g.row_scale = rstd;
    if ((rc = launch_gemm(g, s))) return rc;
    if ((rc = mark(BLT_STAGE_W13_GEMM, s))) return rc;
    g = GemmArgs{};
    g.A = hbuf; g.Bt = w2 + l * D * F; g.C = xr;
    g.M = M; g.N = D; g.K = F; g.lda = F; g.ldb = F; g.ldc = D; g.epi = EPI_RESID_F32;
    const bool next = l + 1 < cfg.n_layers;  // the next layer's QKV GEMM input
    if (next) {
      g.xb_out = a; g.ss_out = ss; g.ss_np = np; g.col_scale = attn_nw + (l + 1) * D;
    }
    if ((rc = launch_gemm(g, s))) return rc;
    if (next && (rc = launch_row_rstd(ss, rstd, M, np, (int)D, cfg.norm_eps, s))) return rc;
    if ((rc = mark(BLT_STAGE_W2_GEMM, s))) return rc;
  }
  // Only what the caller asked for: the head (final norm, logits, entropy)
  // runs when logits, entropies or coherence are wanted; the norms alone are
  // one read of the residual; the residual alone (extract_embeddings,
  // model.rs:325-345) stops here.
  const bool need_head = o.logits || o.entropies || o.coherence_scores;
  const bool need_norms = o.embedding_norms || o.coherence_scores;
  float* nr = o.embedding_norms ? o.embedding_norms : norms;
  if (!need_head) {
    if (need_norms) {
      if ((rc = launch_rmsnorm<float, float, float>(xr, nullptr, nullptr, nr, M, (int)D, 0.f, 0,
                                                    s)))
        return rc;
      if ((rc = mark(BLT_STAGE_FINAL_NORM, s))) return rc;
    }
    return 0;
  }
  float* en = o.entropies ? o.entropies : ent;
  if (wout_head) {
    // final RMSNorm, pre-norm L2, head (split-bf16 input), entropy and
    // coherence in one pass over the residual; logits only when asked for
    if ((rc = launch_head_entropy(xr, final_norm, wout_head, M, (int)D, (int)V, cfg.norm_eps,
                                  o.logits, en, nr, o.coherence_scores, s)))
      return rc;
    return mark(BLT_STAGE_HEAD_GEMM, s);
  }
  // pre-norm L2 norms fused with the final RMSNorm (one read of the residual)
  if ((rc = launch_rmsnorm<float, float, uint16_t>(xr, final_norm, a, nr, M, (int)D, cfg.norm_eps,
                                                   0, s)))
    return rc;
  if ((rc = mark(BLT_STAGE_FINAL_NORM, s))) return rc;
  float* lg = o.logits ? o.logits : logits;
  GemmArgs g{};
  g.A = a; g.Bt = wout; g.C = lg;
  g.M = M; g.N = V; g.K = D; g.lda = D; g.ldb = D; g.ldc = V; g.epi = EPI_F32; g.n_valid = (int)V;
  if ((rc = launch_gemm(g, s))) return rc;
  if ((rc = mark(BLT_STAGE_HEAD_GEMM, s))) return rc;
  if ((rc = launch_entropy_f32(lg, en, M, (int)V, s))) return rc;
  if ((rc = mark(BLT_STAGE_ENTROPY, s))) return rc;
  if (o.coherence_scores) {
    if ((rc = launch_coherence(nr, en, o.coherence_scores, M, 1e-6f, s))) return rc;
    if ((rc = mark(BLT_STAGE_COHERENCE, s))) return rc;
  }
  return 0;
}

}  // namespace blt
