// Model handle behind blt_model_* (see model.hip for the device layout).
#pragma once
#include <utility>
#include <vector>

#include "../../include/blt_hip.h"
#include "rowops.hpp"

namespace blt {

void rope_table_host(float* out, int head_dim, int max_seqlen, double theta);

struct Model {
  int device = 0;
  blt_model_config cfg{};
  int64_t max_tokens = 0;
  int64_t bytes = 0;
  // packed weights
  uint16_t* emb = nullptr;
  float* final_norm = nullptr;
  float* attn_nw = nullptr;  // RMSNorm weights before attention / FFN, [L, dim]
  float* ffn_nw = nullptr;
  uint16_t* wqkv = nullptr;
  uint16_t* wo = nullptr;
  uint16_t* w13 = nullptr;
  uint16_t* w2 = nullptr;
  uint16_t* wout = nullptr;
  uint16_t* wout_head = nullptr;  // the head's K tiles for the fused head kernel (k_head.hip)
  float* rope_cs = nullptr;
  // workspace
  float* x = nullptr;
  uint16_t* a = nullptr;
  float* ss = nullptr;
  float* rstd = nullptr;
  uint16_t* qkv = nullptr;
  uint16_t* attn = nullptr;
  uint16_t* hbuf = nullptr;
  float* logits = nullptr;
  float* ent = nullptr;
  float* norms = nullptr;

  // per-stage HIP-event timing (blt_model_set_profiling)
  bool profiling = false;
  std::vector<hipEvent_t> ev_pool;
  size_t ev_used = 0;
  std::vector<std::pair<int, size_t>> ev_marks;  // (stage, index of the event ending it)
  hipStream_t ev_stream = nullptr;
  int mark(int stage, hipStream_t s);  // records the event that ends `stage`
  double acc_ms[BLT_NUM_STAGES] = {};  // totals of folded marks
  int64_t acc_n[BLT_NUM_STAGES] = {};
  int fold_profile();
  int read_profile(double* ms, int64_t* launches, int n);

  ~Model();
  static int create(int dev, const blt_model_config& c, const blt_model_weights& w,
                    int64_t max_tok, Model** out);
  int forward(const int32_t* tokens, int64_t B, int64_t T, const blt_model_outputs& o,
              hipStream_t s, const int32_t* seg_start = nullptr);
};

}  // namespace blt
