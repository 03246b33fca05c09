// Host launchers of the kernels (each returns 0 or a negative blt_status).
#pragma once
#include "../../include/blt_hip.h"
#include "common.hpp"

namespace blt {

// k_rowops.hip
int launch_entropy_f32(const float* x, float* out, int64_t rows, int n, hipStream_t s);
int launch_entropy_bf16(const uint16_t* x, float* out, int64_t rows, int n, hipStream_t s);
template <typename TX, typename TW, typename TY>
int launch_rmsnorm(const TX* x, const TW* w, TY* y, float* l2, int64_t rows, int n, float eps,
                   int mode, hipStream_t s);
int launch_softmax_f32(const float* x, float* y, int64_t rows, int n, hipStream_t s);
int launch_silu_gate_f32(const float* g, const float* u, float* o, int64_t n, hipStream_t s);
int launch_silu_gate_bf16(const uint16_t* g, const uint16_t* u, uint16_t* o, int64_t n,
                          hipStream_t s);
int launch_coherence(const float* nrm, const float* ent, float* out, int64_t n, float eps,
                     hipStream_t s);
// x = f32 rows of the table; xb (optional) = the same rows in bf16 and ss
// (optional) = their per-64-column sums of squares [rows, dim / 64]
// rstd[r] = 1 / (sqrt(sum(ss[r, 0 .. np)) / dim) + eps): the model's RMSNorm
// factor (eps after the root) from per-64-column sums of squares
int launch_row_rstd(const float* ss, float* rstd, int64_t rows, int np, int dim, float eps,
                    hipStream_t s);
// (xb = bf16(row * col_scale) when col_scale is given: the first layer's norm weight)
int launch_embed(const int32_t* tok, const uint16_t* table, float* x, int64_t rows, int dim,
                 int vocab, hipStream_t s, uint16_t* xb = nullptr, float* ss = nullptr,
                 const float* col_scale = nullptr);
int launch_rope(const uint16_t* src, uint16_t* dst, const float* cs, int64_t B, int64_t H,
                int64_t T, int d, int64_t sb, int64_t sh, int64_t st, hipStream_t s);
int launch_patch_boundaries(const float* H, int64_t B, int64_t T, float thr, int mode,
                            int32_t* mask, int32_t* starts, int32_t* lengths, int32_t* count,
                            hipStream_t s);
// the same compaction from a start mask: starts = {t : mask[b, t] == 1}
int launch_patch_mask_starts(const int32_t* mask, int64_t B, int64_t T, int32_t* starts,
                             int32_t* lengths, int32_t* count, hipStream_t s);

// per-patch means of H / N / C over the patches starts[0 .. count) of each row
// (row_off / row_len NULL: dense rows of T); C, mH, mN, mC may be NULL.
// starts NULL: each row is one patch over the whole row (count unused).
// out_off (optional): row b's means go to m*[out_off[b] + p] instead of the
// row's own offset.
int launch_patch_means(const float* H, const float* N, const float* C, const int32_t* starts,
                       const int32_t* count, int64_t B, int64_t T, const int64_t* row_off,
                       const int32_t* row_len, float* mH, float* mN, float* mC, hipStream_t s,
                       const int64_t* out_off = nullptr);

int launch_scatter_tokens(const int32_t* dest, const float* H, const float* N, const float* C,
                          float* Ho, float* No, float* Co, int64_t n, hipStream_t s);
int launch_scatter_rows(const int32_t* dest, const float* X, float* Xo, int64_t n, int dim,
                        hipStream_t s);
int launch_patch_boundaries_varlen(const float* H, const int64_t* row_off, const int32_t* row_len,
                                   int64_t rows, float thr, int mode, int32_t* mask,
                                   int32_t* starts, int32_t* lengths, int32_t* count,
                                   hipStream_t s);

// k_patch.hip: boundary rules over many blocks per row; ws = a workspace of
// patch_workspace_bytes (no initialisation needed)
int64_t patch_workspace_bytes(int64_t B, int64_t T, int n_rules);
int launch_patch_rules(const float* H, int64_t B, int64_t T, int n_rules,
                       const blt_patch_rule* rules, void* ws, int64_t ws_bytes, hipStream_t s);
// launch_patch_rules with the workspace in a static device array (1 MiB per
// device; n_rules * B * ceil(T / 1024) <= 7281)
int launch_patch_rules_noalloc(const float* H, int64_t B, int64_t T, int n_rules,
                               const blt_patch_rule* rules, hipStream_t s);
// softmax entropy of logits [B * T, vocab] (into H_out, may be NULL when the
// vocab has a fused variant) and the rules in one pass
int launch_entropy_patch(const float* logits, int64_t B, int64_t T, int vocab, float* H_out,
                         int n_rules, const blt_patch_rule* rules, void* ws, int64_t ws_bytes,
                         hipStream_t s);

// k_head.hip: final RMSNorm + pre-norm L2 + head (input split into bf16 hi +
// lo) + entropy + coherence in one pass over the f32 residual x [M, D].
// wpacked = pack_head_weights of the transposed head weight Bt [V, D];
// logits, ent, norms, coh may each be NULL.
bool head_fused_ok(int dim, int vocab);
int64_t head_packed_elems(int dim);
void pack_head_weights(const uint16_t* bt, int V, int D, uint16_t* out);
int launch_head_entropy(const float* x, const float* w_norm, const uint16_t* wpacked, int64_t M,
                        int D, int V, float eps, float* logits, float* ent, float* norms,
                        float* coh, hipStream_t s);

// k_gemm.hip -----------------------------------------------------------------
// C[M, N] = A[M, K] . Bt[N, K]^T with bf16 operands and f32 accumulation; the
// epilogue decides what is written.  K % 64 == 0, N % 64 == 0 (Bt padded with
// zero rows by the caller where the logical N is smaller).
enum GemmEpi {
  EPI_BF16 = 0,      // C bf16 [M, ldc]
  EPI_F32 = 1,       // C f32 [M, ldc], columns >= n_valid dropped
  EPI_RESID_F32 = 2, // R f32 [M, ldc] += acc (in place)
  EPI_QKV_ROPE = 3,  // bf16 out; columns < rope_cols rotated (half-split pairs within 64-wide heads)
  EPI_SILU_GATE = 4  // Bt interleaved in 32-column (gate, up) groups; out bf16 [M, N/2]
};
struct GemmArgs {
  const uint16_t* A;
  const uint16_t* Bt;
  void* C;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int epi;
  int n_valid;      // EPI_F32
  int rope_cols;    // EPI_QKV_ROPE
  int q_cols;       // EPI_QKV_ROPE: columns < q_cols (whole 64-column heads) are
  float q_scale;    //   multiplied by q_scale before the bf16 rounding (0 = none)
  int64_t seq_len;  // EPI_QKV_ROPE: position = row % seq_len - seg_start[row]
  const int32_t* seg_start;  // segment starts within each row (NULL = 0)
  const float* rope_cs;  // [max_seqlen, 32, 2]
  int vec_ok;            // EPI_F32: C and ldc allow 16-byte row stores
  int group_m;           // tile order: M-tiles per group (0 = N fastest)
  // RMSNorm carried across GEMMs (model layers).  Producer: an EPI_RESID_F32
  // GEMM with xb_out set also writes bf16(new residual) to xb_out [M, ldc]
  // and, per row and 64-column group, the sum of squares of the new residual
  // to ss_out [M, ss_np] (launch_row_rstd turns those into row factors).
  // col_scale (optional, [N] f32) multiplies column c of that bf16 copy only
  // (the consumer's RMSNorm weight): xb_out = bf16(residual * col_scale).
  // Consumer: a GEMM with row_scale set (its A is such a scaled bf16 residual)
  // multiplies output row r by row_scale[r] before its epilogue.
  uint16_t* xb_out;
  float* ss_out;
  int ss_np;
  const float* row_scale;
  const float* col_scale;
};
int launch_gemm(const GemmArgs& a, hipStream_t s);

// k_attn.hip -----------------------------------------------------------------
// log2(e) / sqrt(64): the scores' scale in the log2 domain (q is multiplied by
// it before its bf16 rounding, so S = q' k comes out of the MFMA ready for exp2)
constexpr float kAttnQScale = 0.125f * 1.44269504088896340736f;
struct AttnArgs {
  const uint16_t* q; const uint16_t* k; const uint16_t* v; uint16_t* o;
  int64_t B, H, T;
  int64_t sb_q, sh_q, st_q, sb_k, sh_k, st_k, sb_v, sh_v, st_v, sb_o, sh_o, st_o;
  int causal, window;
  // Optional packed segments: seg_start[b * T + t] = index (within the row) of
  // the first token of t's segment, non-decreasing along a row.  Key j is
  // visible to query i only if j >= seg_start[i].  NULL = one segment per row.
  const int32_t* seg_start;
  // Optional: q is rotated (half-split RoPE pairs (m, m + 32)) as it is loaded,
  // with the (cos, sin) table [T, 32, 2] f32 at the query's row index.
  const float* q_rope_cs;
  // q already multiplied by log2(e) / sqrt(64) (the QKV epilogue of the
  // model); otherwise the kernel scales it as it is loaded
  int q_prescaled;
};
int launch_attention(const AttnArgs& a, hipStream_t s);
// f32 [B, H, Tq, d] x [B, H, Tkv, d] dense head-major, any d <= 256, f32 math
int launch_attention_f32(const float* q, const float* k, const float* v, float* o, int64_t B,
                         int64_t H, int64_t Tq, int64_t Tkv, int d, int causal, hipStream_t s);

}  // namespace blt
