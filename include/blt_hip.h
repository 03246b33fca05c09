/*
 * blt_hip.h — C ABI of the MI355X (gfx950) entropy-patching library.
 *
 * Drop-in boundary for blt-burn's entropy-patching hot path.  Every entry
 * point below names the reference interface it replaces (file:line in
 * SashimiSaketoro/blt-burn).  Conventions:
 *
 *   - All tensors are caller-owned, dense, row-major device buffers.  The
 *     library never frees caller memory; a model handle owns only its packed
 *     weights and its workspace.
 *   - bf16 tensors are passed as uint16_t* holding IEEE bfloat16 bits.
 *   - Every call is stream-ordered: `stream` is a hipStream_t (NULL = the
 *     device's null stream).  Nothing synchronises unless the entry point
 *     says so.
 *   - Every call returns BLT_OK (0) or a negative blt_status.  The message of
 *     the last failure on the calling thread is returned by blt_last_error().
 *     No exception or abort crosses the ABI (the reference panics on bad
 *     shapes; the Rust binding maps a non-zero status to panic!).
 */
#ifndef BLT_HIP_H
#define BLT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* blt_stream_t; /* hipStream_t */

typedef enum blt_status {
  BLT_OK = 0,
  BLT_ERR_INVALID = -1,  /* null pointer / bad enum value */
  BLT_ERR_SHAPE = -2,    /* shape or size outside what the op accepts */
  BLT_ERR_HIP = -3,      /* HIP runtime error (launch, copy, device) */
  BLT_ERR_OOM = -4,      /* device allocation failed */
  BLT_ERR_NODEV = -5     /* no usable gfx950 device */
} blt_status;

/* RMSNorm epsilon placement (the reference has both, see fused_rms_norm). */
typedef enum blt_eps_mode {
  BLT_EPS_AFTER_SQRT = 0,  /* x / (sqrt(mean x^2) + eps) * w   model.rs:758-770, backend.rs:502-506 */
  BLT_EPS_INSIDE_SQRT = 1  /* x / sqrt(mean x^2 + eps) * w     rms_norm_kernel.rs:40-43 */
} blt_eps_mode;

/* Boundary rule for blt_patch_boundaries. */
typedef enum blt_patch_mode {
  BLT_PATCH_MONOTONIC = 0, /* m[0]=m[1]=1, m[t] = (H[t]-H[t-1]) > thr   patcher.rs:80-118 */
  BLT_PATCH_GLOBAL = 1     /* m[0]=m[1]=1, m[t] = H[t] > thr (build-defined layout, same specials) */
} blt_patch_mode;

/* Library-level --------------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). */
const char* blt_last_error(void);
/* Library version string. */
const char* blt_version(void);
/* Number of visible gfx950 devices (0 when there is no GPU); never fails. */
int blt_device_count(void);
/* Wait for all work queued on `stream`. */
int blt_stream_sync(blt_stream_t stream);

/* Fused ops: trait FusedOpsBackend (src/fused_ops/mod.rs:58-145) -------- */

/* fused_entropy (mod.rs:62, wrapper mod.rs:155-159; NdArray form patcher.rs:38-63).
 * logits [rows, vocab] f32 -> out [rows] f32, H = -sum softmax*log_softmax, natural log. */
int blt_fused_entropy_f32(const float* logits, float* out, int64_t rows, int32_t vocab,
                          blt_stream_t stream);
/* Same over bf16 logits (entropy accumulated in f32). */
int blt_fused_entropy_bf16(const uint16_t* logits, float* out, int64_t rows, int32_t vocab,
                           blt_stream_t stream);

/* fused_rms_norm (mod.rs:67-73, wrapper mod.rs:162-176).
 * x [rows, dim] -> y [rows, dim]; w [dim].  l2_out (may be NULL) receives
 * sqrt(sum x^2) of each input row (the pre-norm embedding norm, model.rs:291-300). */
int blt_fused_rms_norm_f32(const float* x, const float* w, float* y, float* l2_out,
                           int64_t rows, int32_t dim, float eps, int32_t eps_mode,
                           blt_stream_t stream);
int blt_fused_rms_norm_bf16(const uint16_t* x, const uint16_t* w, uint16_t* y, float* l2_out,
                            int64_t rows, int32_t dim, float eps, int32_t eps_mode,
                            blt_stream_t stream);

/* fused_softmax over the last dim (mod.rs:78, wrapper mod.rs:179-185). x,y [rows, n] f32. */
int blt_fused_softmax_f32(const float* x, float* y, int64_t rows, int32_t n,
                          blt_stream_t stream);

/* fused_l2_norm (mod.rs:83, wrapper mod.rs:188-192). x [rows, dim] -> out [rows]. */
int blt_fused_l2_norm_f32(const float* x, float* out, int64_t rows, int32_t dim,
                          blt_stream_t stream);
int blt_fused_l2_norm_bf16(const uint16_t* x, float* out, int64_t rows, int32_t dim,
                           blt_stream_t stream);

/* fused_silu_gate (mod.rs:89-92, wrapper mod.rs:195-205). out = silu(g) * u, n elements. */
int blt_fused_silu_gate_f32(const float* g, const float* u, float* out, int64_t n,
                            blt_stream_t stream);
int blt_fused_silu_gate_bf16(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t n,
                             blt_stream_t stream);

/* fused_coherence (mod.rs:97-101, wrapper mod.rs:208-220). out = n^2 / (H + eps). */
int blt_fused_coherence_f32(const float* norms, const float* entropies, float* out,
                            int64_t n, float eps, blt_stream_t stream);

/* fused_attention (mod.rs:104-114, wrapper mod.rs:225-236) extended with RoPE and
 * a sliding window.  q,k,v,o are bf16 [B, H, T, d] (head-major, as mod.rs:104-107)
 * when the strides below say so; any (b,h,t) strides with unit d-stride are
 * accepted, in elements.  Only d = 64 is supported.
 *   causal: 1 = key j visible to query i iff j <= i (model.rs:153-165)
 *   window: 0 = unlimited; W > 0 additionally requires j > i - W
 *   rope_theta: 0 = no rotation; > 0 rotates q and k (half-split pairs,
 *               model.rs:24-52,107-147) at positions t = 0..T-1 before QK^T.
 * Softmax in f32 with scale 1/sqrt(d); QK^T and PV on bf16 MFMA, f32 accumulate.
 * workspace: when rope_theta > 0, a device buffer of at least
 *            blt_attention_workspace_bytes(B,H,T,d) bytes (else may be NULL). */
int64_t blt_attention_workspace_bytes(int64_t B, int64_t H, int64_t T, int32_t d);
int blt_fused_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             uint16_t* o, int64_t B, int64_t H, int64_t T, int32_t d,
                             int64_t sb_q, int64_t sh_q, int64_t st_q,
                             int64_t sb_kv, int64_t sh_kv, int64_t st_kv,
                             int64_t sb_o, int64_t sh_o, int64_t st_o,
                             int32_t causal, int32_t window, float rope_theta,
                             void* workspace, blt_stream_t stream);

/* fused_attention on f32 tensors as the CubeCL kernel computes it
 * (attention_kernel.rs:20-125, launched by backend.rs:334-383): q [B, H, Tq, d],
 * k and v [B, H, Tkv, d], o [B, H, Tq, d], all f32, dense head-major; any
 * head_dim d <= 256; causal: key j visible to query i iff j <= i.  Scores
 * (q . k) / sqrt(d) and the softmax in f32 on the VALU (no bf16 rounding); a
 * query that sees no key gets 0.  blt_fused_attention_bf16 is the MFMA path
 * (d = 64, RoPE and windows) the model uses. */
int blt_fused_attention_f32(const float* q, const float* k, const float* v, float* o, int64_t B,
                            int64_t H, int64_t Tq, int64_t Tkv, int32_t d, int32_t causal,
                            blt_stream_t stream);

/* RoPE table, precompute_freqs_cis (model.rs:24-52): out [max_seqlen, head_dim/2, 2]
 * f32 (cos, sin), computed on the host in the reference's f32 order, copied to device. */
int blt_rope_table_f32(float* out_device, int32_t head_dim, int32_t max_seqlen, double theta,
                       blt_stream_t stream);

/* Patcher (src/patcher.rs) --------------------------------------------- */

/* patch_start_mask_from_entropy_with_monotonicity (patcher.rs:80-118) fused with
 * patch_start_indices_cpu (patcher.rs:124-142) and patch_lengths_from_start_indices
 * (patcher.rs:144-164), done on the device.
 *   H [B, T] f32.  Outputs (each may be NULL):
 *   mask    [B, T] int32: 1 = patch start, else 0
 *   starts  [B, T] int32: row b holds its count[b] start indices, ascending
 *   lengths [B, T] int32: row b holds count[b] patch lengths (sum = T)
 *   count   [B]    int32
 *   mode: blt_patch_mode; thr: delta (monotonic) or theta (global), compared in f32. */
int blt_patch_boundaries(const float* H, int64_t B, int64_t T, float thr, int32_t mode,
                         int32_t* mask, int32_t* starts, int32_t* lengths, int32_t* count,
                         blt_stream_t stream);

/* patch_start_indices_cpu (patcher.rs:124-142) and patch_lengths_from_start_indices
 * (patcher.rs:144-164) on the device, from a start mask such as
 * patch_start_mask_from_entropy_with_monotonicity returns: the starts of row b
 * are the positions t with mask[b*T + t] == 1 (exactly 1, as the reference
 * tests), ascending; lengths are next start (or T) minus start.
 *   mask [B, T] int32.  Outputs as blt_patch_boundaries writes them: starts /
 *   lengths [B, T] int32 with count[b] valid entries per row, count [B] int32
 *   (each may be NULL; lengths needs starts). */
int blt_patch_mask_starts(const int32_t* mask, int64_t B, int64_t T, int32_t* starts,
                          int32_t* lengths, int32_t* count, blt_stream_t stream);

/* One boundary rule and its outputs, laid out as blt_patch_boundaries writes
 * them (each output may be NULL; lengths needs starts). */
typedef struct blt_patch_rule {
  int32_t mode;      /* blt_patch_mode */
  float threshold;   /* delta (monotonic) or theta (global), compared in f32 */
  int32_t* mask;     /* [B, T] */
  int32_t* starts;   /* [B, T], count[b] valid entries in row b */
  int32_t* lengths;  /* [B, T], count[b] valid entries in row b */
  int32_t* count;    /* [B] */
} blt_patch_rule;

/* Device bytes of the workspace of blt_patch_boundaries_rules and
 * blt_entropy_patch_boundaries for [B, T] and n_rules (1 or 2) rules. */
int64_t blt_patch_workspace_bytes(int64_t B, int64_t T, int32_t n_rules);

/* The same outputs as blt_patch_boundaries (patcher.rs:80-164), for one or two
 * rules from one read of H (the reference calls the mask function once per
 * rule), with many blocks per row (per-tile flags, then per-tile compaction).
 * workspace: device memory of at least blt_patch_workspace_bytes(B, T, n_rules)
 * bytes, 16-byte aligned, holding per-tile counts and flag words between the
 * call's kernels; it needs no initialisation and keeps nothing between calls,
 * but calls that share one must be stream-ordered. */
int blt_patch_boundaries_rules(const float* H, int64_t B, int64_t T, int32_t n_rules,
                               const blt_patch_rule* rules, void* workspace,
                               int64_t workspace_bytes, blt_stream_t stream);

/* blt_patch_boundaries_rules without the workspace argument: no counterpart in
 * the reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops): the per-tile counts and flag words
 * live in a static device array of 1 MiB per device, so it needs
 * n_rules * B * ceil(T / 1024) <= 7281 (BLT_ERR_SHAPE otherwise) and calls no
 * allocator.  Every call on one device shares that array: calls that overlap
 * on one device race. */
int blt_patch_boundaries_rules_noalloc(const float* H, int64_t B, int64_t T, int32_t n_rules,
                                       const blt_patch_rule* rules, blt_stream_t stream);

/* patcher::entropy (patcher.rs:15-22; NdArray form 38-63) followed by the
 * rules of blt_patch_boundaries_rules, in one pass over the logits when
 * vocab % 4 == 0, vocab < 1280 and the rows are 16-byte aligned (otherwise
 * the entropy kernel and the rule pass run one after the other).
 * logits [B, T, vocab] f32; entropies [B, T] f32 out (may be NULL on the
 * one-pass path).  Workspace as for blt_patch_boundaries_rules. */
int blt_entropy_patch_boundaries(const float* logits, int64_t B, int64_t T, int32_t vocab,
                                 float* entropies, int32_t n_rules, const blt_patch_rule* rules,
                                 void* workspace, int64_t workspace_bytes, blt_stream_t stream);

/* Per-patch means over the patches blt_patch_boundaries found: for row b and
 * patch p < count[b], the patch covers [starts[b*T + p], starts[b*T + p + 1]) (the
 * last to T) and
 *   mean_entropy[b*T + p]    = sum(entropies) / length   (compute_mean_entropy)
 *   mean_prominence[b*T + p] = sum(norms) / length       (compute_mean_prominence)
 *   mean_coherence[b*T + p]  = sum(coherence) / length   (segment coherence)
 * with left-to-right f32 sums, as pipeline.rs:240-258 and huggingface_loader.rs:
 * 265-295 compute them; an empty patch gives 0.  entropies / norms / coherence
 * [B, T] f32; starts [B, T], count [B] int32 as blt_patch_boundaries writes them.
 * coherence and mean_coherence may both be NULL; any output may be NULL. */
int blt_patch_means(const float* entropies, const float* norms, const float* coherence,
                    const int32_t* starts, const int32_t* count, int64_t B, int64_t T,
                    float* mean_entropy, float* mean_prominence, float* mean_coherence,
                    blt_stream_t stream);

/* Entropy model: LMTransformer (src/model.rs) ------------------------- */

/* LMTransformerConfig (model.rs:167-180) with the derived sizes resolved. */
typedef struct blt_model_config {
  int32_t dim;        /* 768 */
  int32_t n_layers;   /* 14 */
  int32_t n_heads;    /* 12 (n_kv_heads == n_heads; head_dim = dim / n_heads = 64) */
  int32_t ffn_hidden; /* resolved FFN width: 768 as configured (model.rs:468-473), 2048 in real weights */
  int32_t vocab;      /* 260 */
  int32_t max_seqlen; /* 8192: bound of the RoPE table */
  float norm_eps;     /* 1e-5, eps after sqrt */
  float rope_theta;   /* 10000 */
  int32_t window;     /* 0 = full causal (reference semantics); W > 0 = sliding window */
} blt_model_config;

/* Host-side weights in the reference's layouts (Burn Linear weight is [in, out]):
 * every pointer is host memory holding bf16 bits; the library packs them into
 * its own device layout.  Per layer l, arrays are concatenated over layers:
 *   tok_embeddings [vocab, dim]                                model.rs:190
 *   attention_norm [L, dim], ffn_norm [L, dim]                 model.rs:481-498
 *   wq, wk, wv, wo [L, dim, dim]                               model.rs:536-550
 *   w1, w3 [L, dim, hidden], w2 [L, hidden, dim]               model.rs:704-714
 *   norm [dim], output [dim, vocab]                            model.rs:205-212 */
typedef struct blt_model_weights {
  const uint16_t* tok_embeddings;
  const uint16_t* attention_norm;
  const uint16_t* ffn_norm;
  const uint16_t* wq;
  const uint16_t* wk;
  const uint16_t* wv;
  const uint16_t* wo;
  const uint16_t* w1;
  const uint16_t* w2;
  const uint16_t* w3;
  const uint16_t* norm;
  const uint16_t* output;
} blt_model_weights;

/* ModelOutput (model.rs:229-245).  Device buffers owned by the caller; any may be NULL. */
typedef struct blt_model_outputs {
  float* logits;              /* [B, T, vocab] f32 */
  float* pre_norm_embeddings; /* [B, T, dim] f32 */
  float* embedding_norms;     /* [B, T] f32 */
  float* entropies;           /* [B, T] f32 */
  float* coherence_scores;    /* [B, T] f32, n^2 / (H + 1e-6) */
} blt_model_outputs;

typedef struct blt_model blt_model;

/* LMTransformerConfig::init + load_record (model.rs:182-226, model_loader.rs:103-145).
 * Packs the weights onto `device`.  max_tokens bounds B*T of later forwards (it
 * sizes the workspace). */
int blt_model_create(int32_t device, const blt_model_config* cfg, const blt_model_weights* w,
                     int64_t max_tokens, blt_model** out);
int blt_model_destroy(blt_model* m);
/* Device bytes held by the model (weights + workspace). */
int64_t blt_model_device_bytes(const blt_model* m);

/* LMTransformer::forward_with_embeddings (model.rs:269-322).
 * tokens [B, T] int32 device buffer; 1 <= T <= max_seqlen, B*T <= max_tokens. */
int blt_model_forward(blt_model* m, const int32_t* tokens, int64_t B, int64_t T,
                      const blt_model_outputs* out, blt_stream_t stream);

/* LMTransformer::extract_embeddings (model.rs:325-345, 413-431): the
 * pre-normalisation residual after the last layer, out [B, T, dim] f32 (device,
 * caller-owned).  It stops there: no final RMSNorm, head GEMM, entropy or
 * coherence runs.  (blt_model_forward likewise skips the head when its
 * logits, entropies and coherence_scores outputs are all NULL.) */
int blt_model_extract_embeddings(blt_model* m, const int32_t* tokens, int64_t B, int64_t T,
                                 float* out, blt_stream_t stream);

/* Packed rows: several independent sequences (segments) per row, as the
 * reference would run them one by one (model.rs:269-322 per sequence; the
 * document loop of batching.rs:5-15 / blt_core.rs:300-356).  seg_start [B, T]
 * int32 device buffer: for token t of row b, the index within the row of the
 * first token of t's segment (non-decreasing along the row).  Attention of a
 * token sees only keys of its own segment, and its RoPE position is
 * t - seg_start[b, t]; every other op is per token. */
int blt_model_forward_segments(blt_model* m, const int32_t* tokens, const int32_t* seg_start,
                               int64_t B, int64_t T, const blt_model_outputs* out,
                               blt_stream_t stream);

/* Per-stage timing of blt_model_forward with HIP events recorded on the
 * forward's stream between its kernels (for roofline reporting). */
typedef enum blt_stage {
  BLT_STAGE_EMBED = 0,
  BLT_STAGE_RMSNORM = 1,
  BLT_STAGE_QKV_GEMM = 2,
  BLT_STAGE_ATTENTION = 3,
  BLT_STAGE_O_GEMM = 4,
  BLT_STAGE_W13_GEMM = 5,
  BLT_STAGE_W2_GEMM = 6,
  BLT_STAGE_FINAL_NORM = 7,
  BLT_STAGE_HEAD_GEMM = 8,
  BLT_STAGE_ENTROPY = 9,
  BLT_STAGE_COHERENCE = 10,
  BLT_NUM_STAGES = 11
} blt_stage;
/* on != 0: record events in later forwards. */
int blt_model_set_profiling(blt_model* m, int32_t on);
/* Waits for the last recorded event; writes per-stage total milliseconds and
 * launch counts for the forwards since the previous read (n >= BLT_NUM_STAGES). */
int blt_model_read_profile(blt_model* m, double* ms, int64_t* launches, int32_t n);
const char* blt_stage_name(int32_t stage);

/* Byte tokenizer (host) ---------------------------------------------------- */

/* BltTokenizer::encode(String::from_utf8_lossy(bytes)) without BPE
 * (tokenizer.rs:76-103 on the text built at blt_core.rs:152-154): every
 * maximal ill-formed UTF-8 subsequence becomes U+FFFD (EF BF BD), each byte b
 * becomes b + 4, BOS (1) first and EOS (2) last when asked.  tokens may be
 * null to only count; otherwise at most cap tokens are written and a larger
 * result is BLT_ERR_SHAPE.  *n_tokens receives the count. */
int blt_tokenize_bytes(const uint8_t* bytes, int64_t n, int32_t add_bos, int32_t add_eos,
                       int32_t* tokens, int64_t cap, int64_t* n_tokens);

/* The same over n_docs documents bytes[byte_offsets[d], byte_offsets[d + 1])
 * (byte_offsets[0] = 0): document d's tokens go to tokens[token_offsets[d],
 * token_offsets[d + 1]) (token_offsets has n_docs + 1 entries, [0] = 0).
 * 3 * bytes + 2 * n_docs tokens always suffice; tokens may be null to only
 * count. */
int blt_tokenize_documents(const uint8_t* bytes, const int64_t* byte_offsets, int64_t n_docs,
                           int32_t add_bos, int32_t add_eos, int32_t* tokens, int64_t cap,
                           int64_t* token_offsets);

/* Streaming ingest --------------------------------------------------------- */

/* Replaces the per-document loop of blt_core.rs:145-228 after tokenization
 * (compute_all_signals_chunked at blt_core.rs:286-370, the monotonic or
 * global boundary pass, patch indices / lengths, coherence) for many
 * documents at once.  Chunks of at most chunk_len tokens (the first covers
 * [0, chunk_len - overlap); later ones start overlap tokens early and drop
 * their first overlap outputs) are packed into batches of `rows` rows of
 * `row_len` tokens, each chunk its own attention / RoPE segment.  A document
 * whose chunks fit one batch lies in one batch; a longer one (any length) is
 * cut into groups of consecutive chunks that each fit a batch, and its boundary
 * pass runs once its last group has landed.  Host packing of batch i + 1
 * overlaps the device work of batch i. */
typedef struct blt_ingest_config {
  int32_t rows;            /* packed rows per batch */
  int32_t row_len;         /* tokens per packed row (<= model max_seqlen) */
  int32_t chunk_len;       /* BltConfig::max_seq_len; 0 means row_len */
  int32_t overlap;         /* BltConfig::chunk_overlap; 2 * overlap <= chunk_len */
  float threshold;         /* BltConfig::threshold */
  int32_t mode;            /* blt_patch_mode (BltConfig::monotonicity) */
  int32_t with_embeddings; /* != 0: return pre-norm embeddings as well */
  /* device room, in tokens, for documents longer than one batch: their pieces
   * are stitched and their boundary pass runs on the device.  0 means 2^22; a
   * negative value means none.  A document the room cannot hold at the time
   * is gathered on the host and takes a synchronous pass of its own. */
  int32_t long_arena_tokens;
} blt_ingest_config;
typedef struct blt_ingest blt_ingest;

/* Host-only: the chunk plan of one document of doc_len tokens (blt_core.rs:
 * 300-356).  Writes up to cap entries; returns the number of chunks (>= 0)
 * or a negative blt_status. */
int blt_ingest_plan_chunks(int64_t doc_len, int32_t chunk_len, int32_t overlap, int64_t* starts,
                           int32_t* lens, int32_t* skips, int64_t cap);
/* Allocates two pinned host + device buffer sets, an upload and a download
 * stream.  The model must have max_tokens >= rows * row_len. */
int blt_ingest_create(blt_model* m, const blt_ingest_config* cfg, blt_ingest** out);
int blt_ingest_destroy(blt_ingest* g);
/* Document d is tokens[doc_offsets[d], doc_offsets[d + 1]) (doc_offsets[0] =
 * 0, n_docs + 1 entries).  Outputs are host memory indexed like the tokens:
 * entropies / norms / coherence [total], embeddings [total, dim] (only with
 * with_embeddings), starts / lengths [total] with document d's patches at
 * doc_offsets[d] .. + counts[d], counts [n_docs].  Any output may be null.
 * Starts are positions inside the document (patch_start_indices_cpu).
 * Returns when every output is written. */
int blt_ingest_run(blt_ingest* g, const int32_t* tokens, const int64_t* doc_offsets,
                   int64_t n_docs, float* entropies, float* norms, float* coherence,
                   float* embeddings, int32_t* starts, int32_t* lengths, int32_t* counts);
/* blt_ingest_run that also writes the per-patch means of every document
 * (PatchData.entropy / .prominence, pipeline.rs:47-60 and 240-258; segment
 * coherence, huggingface_loader.rs:265-295): patch_entropy / patch_prominence /
 * patch_coherence [total] host f32, document d's patches at doc_offsets[d] ..
 * + counts[d] like starts.  Any of them may be null. */
int blt_ingest_run_patch_means(blt_ingest* g, const int32_t* tokens, const int64_t* doc_offsets,
                               int64_t n_docs, float* entropies, float* norms, float* coherence,
                               float* embeddings, int32_t* starts, int32_t* lengths,
                               int32_t* counts, float* patch_entropy, float* patch_prominence,
                               float* patch_coherence);
/* Counts of the last blt_ingest_run: non-empty documents and their tokens,
 * tokens run through the model (chunks, overlap context included) and
 * packed-row slots launched (batches * rows * row_len, padding included). */
typedef struct blt_ingest_stats {
  int64_t batches;
  int64_t documents;
  int64_t tokens;
  int64_t tokens_computed;
  int64_t row_tokens;
  int64_t long_documents;       /* documents longer than one batch */
  int64_t long_documents_host;  /* of those, the ones gathered on the host */
} blt_ingest_stats;
int blt_ingest_last_stats(blt_ingest* g, blt_ingest_stats* out);

/* Streaming pipeline (pipeline.rs) ------------------------------------------ */

/* pipeline.rs:37-43: chunks of BLT_PIPELINE_CHUNK_SIZE raw bytes, every later
 * chunk starting BLT_PIPELINE_STRIDE bytes early; patches that start before
 * chunk start + BLT_PIPELINE_SAFE_ZONE_END are confirmed. */
#define BLT_PIPELINE_CHUNK_SIZE 4096
#define BLT_PIPELINE_STRIDE 2048
#define BLT_PIPELINE_SAFE_ZONE_END 2048

/* PipelineBuffer (pipeline.rs:74-104) bound to one model: the accumulated
 * entropies and norms stay in device memory, the raw bytes in host memory.
 * threshold is the monotonic rule's delta (patcher.rs:80-118, compared in
 * f32 as the reference's greater_elem does). */
typedef struct blt_pipeline blt_pipeline;
int blt_pipeline_create(blt_model* m, double threshold, blt_pipeline** out);
int blt_pipeline_destroy(blt_pipeline* p);

/* PipelineBuffer::process_chunk (pipeline.rs:111-238): one forward of the raw
 * bytes (tokens = byte values, no +4 offset, pipeline.rs:123) as a [1, n]
 * batch, the new outputs appended (all of the first chunk, the part after
 * BLT_PIPELINE_STRIDE of later ones), the monotonic boundary pass over what
 * has accumulated, and the patches it confirms: patch i starts at start[i],
 * spans length[i] bytes (to the next start, or to the end of what has
 * accumulated) and has the left-to-right f32 means of the norms (prominence)
 * and entropies over that span (pipeline.rs:240-258).  *n_patches receives
 * the count; at most min(cutoff, accumulated) - lower are written, where
 * lower / cutoff are the reference's confirmation window, so cap >= the
 * accumulated length after the call always suffices (BLT_ERR_SHAPE before
 * any work otherwise).  The work runs on `stream` (ordered after the caller's
 * earlier work there); returns when every output is written.  A call that
 * fails after its forward (a HIP error) may leave the handle part-way through
 * the chunk: blt_pipeline_reset it before the next document. */
int blt_pipeline_process_chunk(blt_pipeline* p, const uint8_t* chunk, int64_t n, int32_t is_last,
                               int64_t cap, int64_t* start, int64_t* length, float* prominence,
                               float* entropy, int64_t* n_patches, blt_stream_t stream);
/* Back to the state of PipelineBuffer::new (nothing accumulated, chunk 0
 * next), keeping the handle's buffers for the next document. */
int blt_pipeline_reset(blt_pipeline* p);
/* Number of accumulated positions (PipelineBuffer::entropies().len()). */
int blt_pipeline_accumulated(blt_pipeline* p, int64_t* len);
/* PipelineBuffer::entropies / norms / raw_bytes (pipeline.rs:260-273): copies
 * positions [offset, offset + n) of each non-null output. */
int blt_pipeline_read(blt_pipeline* p, int64_t offset, int64_t n, float* entropies, float* norms,
                      uint8_t* raw_bytes, blt_stream_t stream);

/* process_document (pipeline.rs:279-324) for n_docs documents at once:
 * document d is bytes[doc_offsets[d], doc_offsets[d + 1]).  The chunks of
 * every document run as independent segments of packed [rows, row_len]
 * forwards (row_len >= CHUNK_SIZE + STRIDE, rows * row_len <= the model's
 * max_tokens), then each document's patches are emitted exactly as the chunk
 * loop of process_document emits them (those starting before STRIDE twice
 * when a document has more than one chunk).  Outputs are host memory:
 * entropies / norms [total] indexed like the bytes; document d's patches are
 * [patch_offsets[d], patch_offsets[d + 1]) of start / length / prominence /
 * entropy, with starts inside the document.  total + STRIDE * n_docs entries
 * always suffice; a smaller cap that is too small is BLT_ERR_SHAPE.  The
 * handle's process_chunk state is untouched.  Waits for `stream`, then runs on
 * the ingest driver's streams; returns when every output is written. */
int blt_pipeline_process_documents(blt_pipeline* p, const uint8_t* bytes,
                                   const int64_t* doc_offsets, int64_t n_docs, int32_t rows,
                                   int32_t row_len, float* entropies, float* norms, int64_t cap,
                                   int64_t* start, int64_t* length, float* prominence,
                                   float* entropy, int64_t* patch_offsets, blt_stream_t stream);

/* Synthetic inputs (host memory, deterministic across C and Python) ----- */

/* splitmix64-seeded N(mean, std) samples (Box-Muller in double), as f32. */
int blt_synth_normal_f32(uint64_t seed, float* out, int64_t n, double mean, double std);
/* Same, rounded to bf16 (round to nearest even). */
int blt_synth_normal_bf16(uint64_t seed, uint16_t* out, int64_t n, double mean, double std);
/* Byte tokens: Zipf(s) over the 95 printable ASCII bytes (a seeded rank
 * permutation), a fraction `p_uniform` replaced by uniform bytes 0..255, plus
 * `offset` (4 = tokenizer.rs OFFSET). */
int blt_synth_tokens(uint64_t seed, int32_t* out, int64_t n, double zipf_s, double p_uniform,
                     int32_t offset);

/* Low-level: the GEMM used by the model, exposed for testing and benchmarking.
 * C[M,N] = A[M,K] * Bt[N,K]^T, bf16 in, f32 accumulate, bf16 out.
 * Requires K % 64 == 0, N % 64 == 0. */
int blt_gemm_bf16(const uint16_t* A, const uint16_t* Bt, uint16_t* C, int64_t M, int64_t N,
                  int64_t K, blt_stream_t stream);

/* The same GEMM with each fused epilogue the model uses (for testing and
 * benchmarking the kernels in isolation).  C = A[M,K] . Bt[N,K]^T, then:
 *   BLT_EPI_BF16:      C bf16 [M, ldc]
 *   BLT_EPI_F32:       C f32  [M, ldc], columns >= n_valid not written
 *   BLT_EPI_RESID_F32: C f32  [M, ldc] += result
 *   BLT_EPI_SILU_GATE: Bt rows in 64-row groups (32 gate rows, then the 32
 *                      matching up rows); C bf16 [M, ldc] gets silu(gate) * up,
 *                      N / 2 columns
 *   BLT_EPI_QKV_ROPE:  C bf16 [M, ldc]; columns < rope_cols are rotated in
 *                      64-wide heads (pairs (c, c + 32)) with the table rope_cs
 *                      [>= seq_len, 32, 2] at position row % seq_len
 * K % 64 == 0; N % 64 == 0 except for BLT_EPI_F32; rows 16-byte aligned. */
typedef enum blt_epilogue {
  BLT_EPI_BF16 = 0,
  BLT_EPI_F32 = 1,
  BLT_EPI_RESID_F32 = 2,
  BLT_EPI_QKV_ROPE = 3,
  BLT_EPI_SILU_GATE = 4
} blt_epilogue;
int blt_gemm_bf16_epilogue(const uint16_t* A, const uint16_t* Bt, void* C, int64_t M, int64_t N,
                           int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int32_t epilogue,
                           int32_t n_valid, int32_t rope_cols, int64_t seq_len,
                           const float* rope_cs, blt_stream_t stream);

/* Measurement helpers (no counterpart in the reference; bench.py reads the
 * rates this GPU sustains beside the published peaks) --------------------- */

/* FLOPs of one blt_probe_mfma_bf16 launch (-1 on bad arguments). */
int64_t blt_probe_mfma_flops(int32_t blocks, int32_t iters);
/* `blocks` blocks of 4 wave64s, each wave running iters x 4 independent
 * v_mfma_f32_32x32x16_bf16; sink (>= blocks * 256 floats) is never written in
 * practice. */
int blt_probe_mfma_bf16(int32_t blocks, int32_t iters, float* sink, blt_stream_t stream);
/* dst = src, `bytes` (a multiple of 16) with 16-byte loads and stores. */
int blt_probe_copy(const void* src, void* dst, int64_t bytes, blt_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BLT_HIP_H */
