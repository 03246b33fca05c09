// Streaming ingest: token documents -> per-document entropies, pre-norm
// embedding norms, coherence, (optionally) pre-norm embeddings and patch
// boundaries, through the packed-row entropy-model forward.  Also the host
// byte tokenizer that produces those token documents.
//
// Reference semantics (blt_core.rs:286-370, compute_all_signals_chunked): a
// document longer than one model sequence is cut into chunks of at most
// `chunk_len` tokens; the first chunk is [0, stride), every later chunk
// starts `overlap` tokens before the current position and its first
// `overlap` outputs are dropped (stride = chunk_len - overlap).  Each chunk is
// an independent forward; the document's stitched entropies then go through
// the boundary pass (blt_core.rs:182-199, patcher.rs:80-164) and coherence
// n^2 / (H + 1e-6) (blt_core.rs:202-207).
//
// Here the chunks of many documents are packed into [rows, row_len] batches
// (per-segment attention and RoPE positions keep every chunk independent, as
// the reference's one-chunk-per-forward loop does).  A document whose chunks
// fit one batch lands in one batch, so its boundary pass runs on the device
// right after the forward.  A longer one is cut into groups of consecutive
// chunks that each fit a batch; the groups run in any batches, their stitched
// outputs are gathered on the host, and the document's boundary pass runs on
// the device once its last group has landed.  Host packing of batch i+1
// overlaps the GPU work of batch i: two slots of pinned host + device
// buffers, uploads on one stream, the model on a compute stream, downloads on
// a third, events between them.
#include <string.h>

#include <algorithm>
#include <map>
#include <vector>

#include "model.hpp"

namespace blt {

struct ChunkPlan {
  int64_t start;  // first token of the chunk in the document
  int32_t len;    // tokens in the chunk
  int32_t skip;   // leading outputs that are overlap context (dropped)
};

// blt_core.rs:300-356.  With 2 * overlap <= chunk_len (checked by callers)
// every later chunk starts exactly `overlap` tokens before the current
// position, so kept output j of a chunk is document token start + j.
static void plan_chunks(int64_t L, int64_t chunk, int64_t overlap, std::vector<ChunkPlan>& out) {
  out.clear();
  const int64_t stride = chunk - overlap;
  int64_t pos = 0;
  while (pos < L) {
    const int64_t start = pos == 0 ? 0 : pos - overlap;
    const int64_t end = std::min(pos + stride, L);
    out.push_back({start, (int32_t)(end - start), (int32_t)(pos - start)});
    pos = end;
  }
}

// First-fit, longest chunk first, into rows of capacity T with current fill.
// On success fill is updated and row/col give each chunk's place.
static bool pack_chunks(const std::vector<ChunkPlan>& c, std::vector<int64_t>& fill, int64_t T,
                        std::vector<int>& order, std::vector<int64_t>& row,
                        std::vector<int64_t>& col) {
  const int64_t B = (int64_t)fill.size();
  order.resize(c.size());
  for (size_t i = 0; i < c.size(); ++i) order[i] = (int)i;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return c[a].len > c[b].len; });
  row.assign(c.size(), -1);
  col.assign(c.size(), 0);
  std::vector<int64_t> trial = fill;
  for (int ci : order) {
    int64_t r = 0;
    while (r < B && trial[r] + c[ci].len > T) ++r;
    if (r == B) return false;
    row[ci] = r;
    col[ci] = trial[r];
    trial[r] += c[ci].len;
  }
  fill.swap(trial);
  return true;
}

// Documents examined per batch after the oldest pending one; later ones that
// fit the space left are packed too (outputs go to each document's own
// offsets, so the order of batches does not matter).
static constexpr size_t kLookahead = 1024;

// A packing unit: chunks [c0, c1) of document `doc`'s plan, whose kept outputs
// are the document positions [out_lo, out_lo + out_len).  `whole` units hold
// every chunk of their document.
struct Unit {
  int64_t doc;
  int32_t c0, c1;
  int64_t out_lo, out_len;
  int64_t computed;  // tokens run through the model
  bool whole;
};

// A document that spans batches.  Its pieces are stitched into a range of the
// device arena (slot >= 0): each batch copies its pieces there on the compute
// stream, and the batch holding the last one also runs the document's boundary
// pass and per-patch means there and downloads them with its own outputs.  A
// document the arena cannot hold (slot < 0) is gathered on the host until its
// last unit lands, then takes a synchronous pass of its own.
struct LongDoc {
  int64_t remaining = 0;  // units not yet stitched (arena) / finished (host)
  int64_t L = 0;
  int32_t slot = -1;      // arena document slot, -1: host gather, -2: not placed yet
  int64_t base = 0;       // the document's first token in the arena
  std::vector<float> H, N, C;
};

struct Ingest {
  Model* m = nullptr;
  blt_ingest_config cfg{};
  int64_t BT = 0, dim = 0;
  hipStream_t up = nullptr, ks = nullptr, down = nullptr;
  blt_ingest_stats stats{};

  struct Slot {
    // pinned host
    int32_t* h_tok = nullptr;
    int32_t* h_seg = nullptr;
    int32_t* h_dest = nullptr;
    int64_t* h_doff = nullptr;
    int32_t* h_dlen = nullptr;
    float* h_H = nullptr;
    float* h_N = nullptr;
    float* h_C = nullptr;
    float* h_E = nullptr;
    int32_t* h_starts = nullptr;
    int32_t* h_lens = nullptr;
    int32_t* h_counts = nullptr;
    float* h_pH = nullptr;  // per-patch means, document order
    float* h_pN = nullptr;
    float* h_pC = nullptr;
    // device
    int32_t* d_tok = nullptr;
    int32_t* d_seg = nullptr;
    int32_t* d_dest = nullptr;
    int64_t* d_doff = nullptr;
    int32_t* d_dlen = nullptr;
    float* d_Hp = nullptr;  // packed-row outputs
    float* d_Np = nullptr;
    float* d_Cp = nullptr;
    float* d_Ep = nullptr;
    float* d_H = nullptr;   // document order
    float* d_N = nullptr;
    float* d_C = nullptr;
    float* d_E = nullptr;
    int32_t* d_starts = nullptr;
    int32_t* d_lens = nullptr;
    int32_t* d_counts = nullptr;
    float* d_pH = nullptr;
    float* d_pN = nullptr;
    float* d_pC = nullptr;
    hipEvent_t uploaded = nullptr, computed = nullptr, done = nullptr;
    bool busy = false;
    std::vector<int64_t> units;  // ids of the units in this batch
    int64_t out_tokens = 0;      // outputs of those units
    std::vector<int64_t> long_done;  // arena documents completed by this batch
  } slot[2];

  // Device arena of the documents that span batches (allocated at first use,
  // la_cap tokens and kArenaDocs document slots), its pinned result copies, and
  // a first-fit list of the token ranges in use (base -> length).
  static constexpr int32_t kArenaDocs = 64;
  int64_t la_cap = 0;
  float* la_H = nullptr;
  float* la_N = nullptr;
  float* la_C = nullptr;
  float* la_pH = nullptr;
  float* la_pN = nullptr;
  float* la_pC = nullptr;
  int32_t* la_starts = nullptr;
  int32_t* la_lens = nullptr;
  int64_t* la_off = nullptr;  // [kArenaDocs]
  int32_t* la_len = nullptr;
  int32_t* la_count = nullptr;
  int32_t* lh_starts = nullptr;
  int32_t* lh_lens = nullptr;
  float* lh_pH = nullptr;
  float* lh_pN = nullptr;
  float* lh_pC = nullptr;
  int64_t* lh_off = nullptr;  // [kArenaDocs]
  int32_t* lh_len = nullptr;
  int32_t* lh_count = nullptr;
  std::map<int64_t, int64_t> la_used;
  std::vector<char> la_slot_used;
  int64_t arena_tokens() const;
  int ensure_arena();
  // places a document in the arena (slot >= 0) or leaves it to the host pass
  int place_long(LongDoc& ld);
  void release_long(LongDoc& ld);

  // this run's packing units and the documents that span batches
  std::vector<Unit> units;
  std::map<int64_t, LongDoc> longs;
  // device buffers of the boundary pass of a document that spans batches
  // (grown to the longest such document)
  int64_t long_cap = 0;
  float* l_H = nullptr;
  float* l_N = nullptr;
  float* l_C = nullptr;
  int32_t* l_starts = nullptr;
  int32_t* l_lens = nullptr;
  float* l_pH = nullptr;
  float* l_pN = nullptr;
  float* l_pC = nullptr;
  int64_t* l_off = nullptr;  // [1] = 0
  int32_t* l_len = nullptr;  // [1]
  int32_t* l_count = nullptr;

  ~Ingest();
  int init(Model* model, const blt_ingest_config& c);
  void drain();  // waits for both slots and drops what they hold
  // per-patch outputs of a run (document d's patches at doc_off[d] .. + counts[d])
  struct PatchOut {
    float* ent = nullptr;
    float* prom = nullptr;
    float* coh = nullptr;
    bool any() const { return ent || prom || coh; }
  };
  int run(const int32_t* tokens, const int64_t* doc_off, int64_t n_docs, float* ent, float* nrm,
          float* coh, float* emb, int32_t* starts, int32_t* lens, int32_t* counts,
          const PatchOut& pm);
  int finish(Slot& s, const int64_t* doc_off, float* ent, float* nrm, float* coh, float* emb,
             int32_t* starts, int32_t* lens, int32_t* counts, const PatchOut& pm);
  // boundary pass (and per-patch means) of a document gathered on the host
  int long_pass(int64_t d, LongDoc& ld, const int64_t* doc_off, int32_t* starts, int32_t* lens,
                int32_t* counts, const PatchOut& pm);
  int ensure_long(int64_t L);
};

Ingest::~Ingest() {
  for (Slot& s : slot) {
    if (s.busy && s.done) (void)hipEventSynchronize(s.done);
    void* hp[] = {s.h_tok, s.h_seg, s.h_dest, s.h_doff,   s.h_dlen, s.h_H,    s.h_N,
                  s.h_C,   s.h_E,   s.h_starts, s.h_lens, s.h_counts, s.h_pH, s.h_pN, s.h_pC};
    for (void* p : hp)
      if (p) (void)hipHostFree(p);
    void* dp[] = {s.d_tok, s.d_seg, s.d_dest, s.d_doff, s.d_dlen,   s.d_Hp,   s.d_Np,
                  s.d_Cp,  s.d_Ep,  s.d_H,    s.d_N,    s.d_C,      s.d_E,    s.d_starts,
                  s.d_lens, s.d_counts, s.d_pH, s.d_pN, s.d_pC};
    for (void* p : dp)
      if (p) (void)hipFree(p);
    for (hipEvent_t e : {s.uploaded, s.computed, s.done})
      if (e) (void)hipEventDestroy(e);
  }
  void* lp[] = {l_H, l_N, l_C, l_starts, l_lens, l_pH, l_pN, l_pC, l_off, l_len, l_count,
                la_H, la_N, la_C, la_pH, la_pN, la_pC, la_starts, la_lens, la_off, la_len,
                la_count};
  for (void* p : lp)
    if (p) (void)hipFree(p);
  void* hp[] = {lh_starts, lh_lens, lh_pH, lh_pN, lh_pC, lh_off, lh_len, lh_count};
  for (void* p : hp)
    if (p) (void)hipHostFree(p);
  for (hipStream_t st : {up, ks, down})
    if (st) (void)hipStreamDestroy(st);
}

void Ingest::drain() {
  for (Slot& s : slot) {
    if (s.busy && s.done) (void)hipEventSynchronize(s.done);
    s.busy = false;
    s.units.clear();
    s.out_tokens = 0;
    s.long_done.clear();
  }
  la_used.clear();
  std::fill(la_slot_used.begin(), la_slot_used.end(), 0);
}

// Arena capacity in tokens: long_arena_tokens, 2^22 when 0, none when negative.
int64_t Ingest::arena_tokens() const {
  if (cfg.long_arena_tokens < 0) return 0;
  return cfg.long_arena_tokens > 0 ? (int64_t)cfg.long_arena_tokens : ((int64_t)1 << 22);
}

int Ingest::ensure_arena() {
  if (la_cap > 0) return 0;
  const int64_t n = arena_tokens();
  const size_t b = (size_t)n * 4;
  BLT_HIP_CHECK(hipMalloc((void**)&la_H, b));
  BLT_HIP_CHECK(hipMalloc((void**)&la_N, b));
  BLT_HIP_CHECK(hipMalloc((void**)&la_C, b));
  BLT_HIP_CHECK(hipMalloc((void**)&la_pH, b));
  BLT_HIP_CHECK(hipMalloc((void**)&la_pN, b));
  BLT_HIP_CHECK(hipMalloc((void**)&la_pC, b));
  BLT_HIP_CHECK(hipMalloc((void**)&la_starts, b));
  BLT_HIP_CHECK(hipMalloc((void**)&la_lens, b));
  BLT_HIP_CHECK(hipMalloc((void**)&la_off, kArenaDocs * 8));
  BLT_HIP_CHECK(hipMalloc((void**)&la_len, kArenaDocs * 4));
  BLT_HIP_CHECK(hipMalloc((void**)&la_count, kArenaDocs * 4));
  BLT_HIP_CHECK(hipHostMalloc((void**)&lh_starts, b, 0));
  BLT_HIP_CHECK(hipHostMalloc((void**)&lh_lens, b, 0));
  BLT_HIP_CHECK(hipHostMalloc((void**)&lh_pH, b, 0));
  BLT_HIP_CHECK(hipHostMalloc((void**)&lh_pN, b, 0));
  BLT_HIP_CHECK(hipHostMalloc((void**)&lh_pC, b, 0));
  BLT_HIP_CHECK(hipHostMalloc((void**)&lh_off, kArenaDocs * 8, 0));
  BLT_HIP_CHECK(hipHostMalloc((void**)&lh_len, kArenaDocs * 4, 0));
  BLT_HIP_CHECK(hipHostMalloc((void**)&lh_count, kArenaDocs * 4, 0));
  la_slot_used.assign(kArenaDocs, 0);
  la_cap = n;
  return 0;
}

// First fit over the arena's free token ranges.  The offset / length words of
// the document's slot go up on the compute stream, ahead of its pieces.  A
// slot's words and range are only rewritten after finish() has waited for the
// batch that completed its previous document.
int Ingest::place_long(LongDoc& ld) {
  ld.slot = -1;
  const int64_t cap = arena_tokens();
  if (ld.L <= 0 || ld.L > cap) return 0;
  int rc;
  if ((rc = ensure_arena())) return rc;
  int32_t sl = -1;
  for (int32_t i = 0; i < kArenaDocs; ++i)
    if (!la_slot_used[(size_t)i]) {
      sl = i;
      break;
    }
  if (sl < 0) return 0;
  int64_t at = 0;
  bool found = false;
  for (const auto& r : la_used) {
    if (r.first - at >= ld.L) {
      found = true;
      break;
    }
    at = r.first + r.second;
  }
  if (!found && la_cap - at < ld.L) return 0;
  la_used[at] = ld.L;
  la_slot_used[(size_t)sl] = 1;
  ld.slot = sl;
  ld.base = at;
  lh_off[sl] = at;
  lh_len[sl] = (int32_t)ld.L;
  BLT_HIP_CHECK(hipMemcpyAsync(la_off + sl, lh_off + sl, 8, hipMemcpyHostToDevice, ks));
  BLT_HIP_CHECK(hipMemcpyAsync(la_len + sl, lh_len + sl, 4, hipMemcpyHostToDevice, ks));
  return 0;
}

void Ingest::release_long(LongDoc& ld) {
  if (ld.slot >= 0) {
    la_used.erase(ld.base);
    la_slot_used[(size_t)ld.slot] = 0;
  }
  ld = LongDoc{};
}

int Ingest::ensure_long(int64_t L) {
  if (L <= long_cap) return 0;
  // buffers in use by an earlier long pass were synchronised at its end
  void* lp[] = {l_H, l_N, l_C, l_starts, l_lens, l_pH, l_pN, l_pC};
  for (void* p : lp)
    if (p) BLT_HIP_CHECK(hipFree(p));
  l_H = l_N = l_C = l_pH = l_pN = l_pC = nullptr;
  l_starts = l_lens = nullptr;
  long_cap = 0;
  BLT_HIP_CHECK(hipMalloc((void**)&l_H, (size_t)L * 4));
  BLT_HIP_CHECK(hipMalloc((void**)&l_N, (size_t)L * 4));
  BLT_HIP_CHECK(hipMalloc((void**)&l_C, (size_t)L * 4));
  BLT_HIP_CHECK(hipMalloc((void**)&l_starts, (size_t)L * 4));
  BLT_HIP_CHECK(hipMalloc((void**)&l_lens, (size_t)L * 4));
  BLT_HIP_CHECK(hipMalloc((void**)&l_pH, (size_t)L * 4));
  BLT_HIP_CHECK(hipMalloc((void**)&l_pN, (size_t)L * 4));
  BLT_HIP_CHECK(hipMalloc((void**)&l_pC, (size_t)L * 4));
  if (!l_off) {
    BLT_HIP_CHECK(hipMalloc((void**)&l_off, 8));
    BLT_HIP_CHECK(hipMalloc((void**)&l_len, 4));
    BLT_HIP_CHECK(hipMalloc((void**)&l_count, 4));
  }
  long_cap = L;
  return 0;
}

// The document's stitched signals are complete on the host: upload them and
// run the same boundary / per-patch-means kernels as a one-batch document,
// on the upload stream (which never waits on the model), then copy the
// patches out.
int Ingest::long_pass(int64_t d, LongDoc& ld, const int64_t* doc_off, int32_t* starts,
                      int32_t* lens, int32_t* counts, const PatchOut& pm) {
  const int64_t L = (int64_t)ld.H.size();
  if (L > 0x7fffffff) return fail(BLT_ERR_SHAPE, "ingest_run: a document of 2^31 tokens or more");
  int rc;
  if ((rc = ensure_long(L))) return rc;
  const int64_t zero = 0;
  const int32_t len32 = (int32_t)L;
  BLT_HIP_CHECK(hipMemcpyAsync(l_off, &zero, 8, hipMemcpyHostToDevice, up));
  BLT_HIP_CHECK(hipMemcpyAsync(l_len, &len32, 4, hipMemcpyHostToDevice, up));
  BLT_HIP_CHECK(hipMemcpyAsync(l_H, ld.H.data(), (size_t)L * 4, hipMemcpyHostToDevice, up));
  if ((rc = launch_patch_boundaries_varlen(l_H, l_off, l_len, 1, cfg.threshold, cfg.mode, nullptr,
                                           l_starts, l_lens, l_count, up)))
    return rc;
  if (pm.any()) {
    BLT_HIP_CHECK(hipMemcpyAsync(l_N, ld.N.data(), (size_t)L * 4, hipMemcpyHostToDevice, up));
    BLT_HIP_CHECK(hipMemcpyAsync(l_C, ld.C.data(), (size_t)L * 4, hipMemcpyHostToDevice, up));
    if ((rc = launch_patch_means(l_H, l_N, l_C, l_starts, l_count, 1, 0, l_off, l_len, l_pH, l_pN,
                                 l_pC, up)))
      return rc;
  }
  int32_t n = 0;
  BLT_HIP_CHECK(hipMemcpyAsync(&n, l_count, 4, hipMemcpyDeviceToHost, up));
  BLT_HIP_CHECK(hipStreamSynchronize(up));
  if (n < 0 || n > L) return fail(BLT_ERR_HIP, "ingest_run: bad patch count");
  const int64_t dst = doc_off[d];
  auto down_n = [&](void* host, const void* dev) -> int {
    if (host && n > 0)
      BLT_HIP_CHECK(hipMemcpyAsync(host, dev, (size_t)n * 4, hipMemcpyDeviceToHost, up));
    return 0;
  };
  if ((rc = down_n(starts ? starts + dst : nullptr, l_starts))) return rc;
  if ((rc = down_n(lens ? lens + dst : nullptr, l_lens))) return rc;
  if ((rc = down_n(pm.ent ? pm.ent + dst : nullptr, l_pH))) return rc;
  if ((rc = down_n(pm.prom ? pm.prom + dst : nullptr, l_pN))) return rc;
  if ((rc = down_n(pm.coh ? pm.coh + dst : nullptr, l_pC))) return rc;
  BLT_HIP_CHECK(hipStreamSynchronize(up));
  if (counts) counts[d] = n;
  ld = LongDoc{};  // release the gathered signals
  return 0;
}

int Ingest::init(Model* model, const blt_ingest_config& c) {
  m = model;
  cfg = c;
  if (cfg.chunk_len == 0) cfg.chunk_len = cfg.row_len;
  if (cfg.rows <= 0 || cfg.row_len <= 0 || cfg.chunk_len <= 0 || cfg.chunk_len > cfg.row_len)
    return fail(BLT_ERR_SHAPE, "ingest: rows > 0, 0 < chunk_len <= row_len");
  if (cfg.overlap < 0 || 2 * (int64_t)cfg.overlap > cfg.chunk_len)
    return fail(BLT_ERR_SHAPE,
                "ingest: 0 <= overlap and 2 * overlap <= chunk_len (with a larger overlap the "
                "reference chunk loop misplaces outputs)");
  if (cfg.row_len > m->cfg.max_seqlen) return fail(BLT_ERR_SHAPE, "ingest: row_len > max_seqlen");
  if (cfg.mode != BLT_PATCH_MONOTONIC && cfg.mode != BLT_PATCH_GLOBAL)
    return fail(BLT_ERR_INVALID, "ingest: bad patch mode");
  BT = (int64_t)cfg.rows * cfg.row_len;
  dim = m->cfg.dim;
  if (BT > m->max_tokens) return fail(BLT_ERR_SHAPE, "ingest: rows * row_len > model max_tokens");
  if (BT > 0x7fffffff) return fail(BLT_ERR_SHAPE, "ingest: rows * row_len >= 2^31");
  BLT_HIP_CHECK(hipSetDevice(m->device));
  BLT_HIP_CHECK(hipStreamCreateWithFlags(&up, hipStreamNonBlocking));
  BLT_HIP_CHECK(hipStreamCreateWithFlags(&ks, hipStreamNonBlocking));
  BLT_HIP_CHECK(hipStreamCreateWithFlags(&down, hipStreamNonBlocking));
  const int64_t ne = cfg.with_embeddings ? BT * dim : 0;
  for (Slot& s : slot) {
#define HALLOC(p, n) \
  if (n) BLT_HIP_CHECK(hipHostMalloc((void**)&(p), (size_t)(n) * sizeof(*(p)), 0))
#define DALLOC(p, n) \
  if (n) BLT_HIP_CHECK(hipMalloc((void**)&(p), (size_t)(n) * sizeof(*(p))))
    HALLOC(s.h_tok, BT); HALLOC(s.h_seg, BT); HALLOC(s.h_dest, BT);
    HALLOC(s.h_doff, BT); HALLOC(s.h_dlen, BT);
    HALLOC(s.h_H, BT); HALLOC(s.h_N, BT); HALLOC(s.h_C, BT); HALLOC(s.h_E, ne);
    HALLOC(s.h_starts, BT); HALLOC(s.h_lens, BT); HALLOC(s.h_counts, BT);
    HALLOC(s.h_pH, BT); HALLOC(s.h_pN, BT); HALLOC(s.h_pC, BT);
    DALLOC(s.d_tok, BT); DALLOC(s.d_seg, BT); DALLOC(s.d_dest, BT);
    DALLOC(s.d_doff, BT); DALLOC(s.d_dlen, BT);
    DALLOC(s.d_Hp, BT); DALLOC(s.d_Np, BT); DALLOC(s.d_Cp, BT); DALLOC(s.d_Ep, ne);
    DALLOC(s.d_H, BT); DALLOC(s.d_N, BT); DALLOC(s.d_C, BT); DALLOC(s.d_E, ne);
    DALLOC(s.d_starts, BT); DALLOC(s.d_lens, BT); DALLOC(s.d_counts, BT);
    DALLOC(s.d_pH, BT); DALLOC(s.d_pN, BT); DALLOC(s.d_pC, BT);
#undef HALLOC
#undef DALLOC
    BLT_HIP_CHECK(hipEventCreateWithFlags(&s.uploaded, hipEventDisableTiming));
    BLT_HIP_CHECK(hipEventCreateWithFlags(&s.computed, hipEventDisableTiming));
    BLT_HIP_CHECK(hipEventCreateWithFlags(&s.done, hipEventDisableTiming));
  }
  return 0;
}

// Wait for a slot's batch and copy its per-document results to the caller.
int Ingest::finish(Slot& s, const int64_t* doc_off, float* ent, float* nrm, float* coh,
                   float* emb, int32_t* starts, int32_t* lens, int32_t* counts,
                   const PatchOut& pm) {
  if (!s.busy) return 0;
  s.busy = false;
  BLT_HIP_CHECK(hipEventSynchronize(s.done));
  for (size_t j = 0; j < s.units.size(); ++j) {
    const Unit& u = units[(size_t)s.units[j]];
    const int64_t d = u.doc;
    const int64_t L = u.out_len;
    const int64_t src = s.h_doff[j], dst = doc_off[d] + u.out_lo;
    if (ent) memcpy(ent + dst, s.h_H + src, (size_t)L * 4);
    if (nrm) memcpy(nrm + dst, s.h_N + src, (size_t)L * 4);
    if (coh) memcpy(coh + dst, s.h_C + src, (size_t)L * 4);
    if (emb && s.h_E) memcpy(emb + dst * dim, s.h_E + src * dim, (size_t)(L * dim) * 4);
    if (!u.whole) {
      LongDoc& ld = longs[d];
      if (ld.slot >= 0) continue;  // stitched on the device
      if (ld.slot != -1 || (int64_t)ld.H.size() < u.out_lo + L ||
          (pm.any() && ((int64_t)ld.N.size() < u.out_lo + L || (int64_t)ld.C.size() < u.out_lo + L)))
        return fail(BLT_ERR_HIP, "ingest_run: a long document's piece has no host buffer");
      memcpy(ld.H.data() + u.out_lo, s.h_H + src, (size_t)L * 4);
      if (pm.any()) {
        memcpy(ld.N.data() + u.out_lo, s.h_N + src, (size_t)L * 4);
        memcpy(ld.C.data() + u.out_lo, s.h_C + src, (size_t)L * 4);
      }
      if (--ld.remaining == 0) {
        const int rc = long_pass(d, ld, doc_off, starts, lens, counts, pm);
        if (rc) return rc;
      }
      continue;
    }
    const int32_t n = s.h_counts[j];
    if (starts) memcpy(starts + dst, s.h_starts + src, (size_t)n * 4);
    if (lens) memcpy(lens + dst, s.h_lens + src, (size_t)n * 4);
    if (pm.ent) memcpy(pm.ent + dst, s.h_pH + src, (size_t)n * 4);
    if (pm.prom) memcpy(pm.prom + dst, s.h_pN + src, (size_t)n * 4);
    if (pm.coh) memcpy(pm.coh + dst, s.h_pC + src, (size_t)n * 4);
    if (counts) counts[d] = n;
  }
  for (int64_t d : s.long_done) {
    LongDoc& ld = longs[d];
    const int32_t n = lh_count[ld.slot];
    if (n < 0 || n > ld.L) return fail(BLT_ERR_HIP, "ingest_run: bad patch count");
    const int64_t dst = doc_off[d], b0 = ld.base;
    if (starts) memcpy(starts + dst, lh_starts + b0, (size_t)n * 4);
    if (lens) memcpy(lens + dst, lh_lens + b0, (size_t)n * 4);
    if (pm.ent) memcpy(pm.ent + dst, lh_pH + b0, (size_t)n * 4);
    if (pm.prom) memcpy(pm.prom + dst, lh_pN + b0, (size_t)n * 4);
    if (pm.coh) memcpy(pm.coh + dst, lh_pC + b0, (size_t)n * 4);
    if (counts) counts[d] = n;
    release_long(ld);
  }
  s.long_done.clear();
  return 0;
}

int Ingest::run(const int32_t* tokens, const int64_t* doc_off, int64_t n_docs, float* ent,
                float* nrm, float* coh, float* emb, int32_t* starts, int32_t* lens,
                int32_t* counts, const PatchOut& pm) {
  if (emb && !cfg.with_embeddings)
    return fail(BLT_ERR_INVALID, "ingest_run: embeddings asked of an ingest made without them");
  const int64_t T = cfg.row_len, B = cfg.rows;
  // a slot still holding a batch of an earlier run that ended in an error:
  // wait for it and drop its results (they belong to that run's arrays)
  drain();
  units.clear();
  longs.clear();
  stats = blt_ingest_stats{};
  std::vector<ChunkPlan> chunks, sub;
  std::vector<int> order;
  std::vector<int64_t> row, col, fill(B);
  auto fits_empty = [&](const std::vector<ChunkPlan>& c) {
    std::fill(fill.begin(), fill.end(), 0);
    return pack_chunks(c, fill, T, order, row, col);
  };
  // ---- plan: empty documents have no outputs (blt_core.rs:160-176) and
  // never enter a batch; a document whose chunks fit an empty batch is one
  // unit; a longer one is cut into runs of consecutive chunks that each fit
  // (every chunk alone fits: chunk_len <= row_len) ----
  for (int64_t d = 0; d < n_docs; ++d) {
    const int64_t L = doc_off[d + 1] - doc_off[d];
    if (L < 0) return fail(BLT_ERR_SHAPE, "ingest_run: doc_offsets must be non-decreasing");
    if (L == 0) continue;
    plan_chunks(L, cfg.chunk_len, cfg.overlap, chunks);
    stats.documents += 1;
    stats.tokens += L;
    auto add_unit = [&](int32_t c0, int32_t c1, bool whole) {
      Unit u{d, c0, c1, 0, 0, 0, whole};
      u.out_lo = chunks[c0].start + chunks[c0].skip;
      u.out_len = chunks[c1 - 1].start + chunks[c1 - 1].len - u.out_lo;
      for (int32_t c = c0; c < c1; ++c) u.computed += chunks[c].len;
      units.push_back(u);
    };
    if (fits_empty(chunks)) {
      add_unit(0, (int32_t)chunks.size(), true);
      continue;
    }
    const int32_t nc = (int32_t)chunks.size();
    int64_t nu = 0;
    for (int32_t c0 = 0; c0 < nc;) {
      int32_t c1 = c0 + 1;
      sub.assign(chunks.begin() + c0, chunks.begin() + c1);
      while (c1 < nc) {
        sub.push_back(chunks[c1]);
        if (!fits_empty(sub)) break;
        ++c1;
      }
      add_unit(c0, c1, false);
      ++nu;
      c0 = c1;
    }
    LongDoc& ld = longs[d];
    ld.remaining = nu;
    ld.L = L;
    ld.slot = -2;  // placed when its first unit is packed
    stats.long_documents += 1;
  }
  BLT_HIP_CHECK(hipSetDevice(m->device));
  std::vector<char> taken(units.size(), 0);
  size_t head = 0;
  int k = 0, rc;
  while (head < units.size()) {
    Slot& s = slot[k];
    if ((rc = finish(s, doc_off, ent, nrm, coh, emb, starts, lens, counts, pm))) return rc;
    std::fill(fill.begin(), fill.end(), 0);
    s.units.clear();
    s.out_tokens = 0;
    s.long_done.clear();
    // ---- pack units: the oldest pending one first (it always fits an empty
    // batch), then any of the next kLookahead that still fit ----
    int64_t free_tokens = BT;
    size_t scanned = 0;
    for (size_t i = head; i < units.size() && scanned < kLookahead && free_tokens > 0; ++i) {
      if (taken[i]) continue;
      ++scanned;
      const Unit& u = units[i];
      if (u.computed > free_tokens) continue;
      plan_chunks(doc_off[u.doc + 1] - doc_off[u.doc], cfg.chunk_len, cfg.overlap, chunks);
      sub.assign(chunks.begin() + u.c0, chunks.begin() + u.c1);
      if (!pack_chunks(sub, fill, T, order, row, col)) continue;
      taken[i] = 1;
      if (!u.whole) {
        LongDoc& ld = longs[u.doc];
        if (ld.slot == -2) {
          if ((rc = place_long(ld))) return rc;
          if (ld.slot < 0) {  // the host gathers it
            stats.long_documents_host += 1;
            ld.H.assign((size_t)ld.L, 0.f);
            if (pm.any()) {
              ld.N.assign((size_t)ld.L, 0.f);
              ld.C.assign((size_t)ld.L, 0.f);
            }
          }
        }
      }
      const int64_t jd = (int64_t)s.units.size();
      s.h_doff[jd] = s.out_tokens;
      s.h_dlen[jd] = (int32_t)u.out_len;
      const int32_t* src = tokens + doc_off[u.doc];
      for (size_t ci = 0; ci < sub.size(); ++ci) {
        const ChunkPlan& c = sub[ci];
        const int64_t base = row[ci] * T + col[ci];
        memcpy(s.h_tok + base, src + c.start, (size_t)c.len * 4);
        // kept output j of the chunk is document position c.start + j
        const int32_t out0 = (int32_t)(s.out_tokens + c.start - u.out_lo);
        for (int32_t j = 0; j < c.len; ++j) {
          s.h_seg[base + j] = (int32_t)col[ci];
          s.h_dest[base + j] = j < c.skip ? -1 : out0 + j;
        }
      }
      free_tokens -= u.computed;
      s.out_tokens += u.out_len;
      s.units.push_back((int64_t)i);
      stats.tokens_computed += u.computed;
    }
    while (head < units.size() && taken[head]) ++head;
    // padding: every free position is its own one-token segment, output dropped
    for (int64_t r = 0; r < B; ++r)
      for (int64_t c = fill[r]; c < T; ++c) {
        s.h_tok[r * T + c] = 0;
        s.h_seg[r * T + c] = (int32_t)c;
        s.h_dest[r * T + c] = -1;
      }
    const int64_t nd = (int64_t)s.units.size();
    stats.batches += 1;
    stats.row_tokens += BT;
    // ---- upload ----
    BLT_HIP_CHECK(hipMemcpyAsync(s.d_tok, s.h_tok, (size_t)BT * 4, hipMemcpyHostToDevice, up));
    BLT_HIP_CHECK(hipMemcpyAsync(s.d_seg, s.h_seg, (size_t)BT * 4, hipMemcpyHostToDevice, up));
    BLT_HIP_CHECK(hipMemcpyAsync(s.d_dest, s.h_dest, (size_t)BT * 4, hipMemcpyHostToDevice, up));
    BLT_HIP_CHECK(hipMemcpyAsync(s.d_doff, s.h_doff, (size_t)nd * 8, hipMemcpyHostToDevice, up));
    BLT_HIP_CHECK(hipMemcpyAsync(s.d_dlen, s.h_dlen, (size_t)nd * 4, hipMemcpyHostToDevice, up));
    BLT_HIP_CHECK(hipEventRecord(s.uploaded, up));
    // ---- compute: packed forward, stitch, boundary pass (its results are
    // used for whole-document units only) ----
    BLT_HIP_CHECK(hipStreamWaitEvent(ks, s.uploaded, 0));
    blt_model_outputs o{};
    o.entropies = s.d_Hp;
    o.embedding_norms = s.d_Np;
    o.coherence_scores = s.d_Cp;
    o.pre_norm_embeddings = s.d_Ep;  // null unless with_embeddings
    if ((rc = m->forward(s.d_tok, B, T, o, ks, s.d_seg))) return rc;
    if ((rc = launch_scatter_tokens(s.d_dest, s.d_Hp, s.d_Np, s.d_Cp, s.d_H, s.d_N, s.d_C, BT,
                                    ks)))
      return rc;
    if (s.d_E && (rc = launch_scatter_rows(s.d_dest, s.d_Ep, s.d_E, BT, (int)dim, ks))) return rc;
    if ((rc = launch_patch_boundaries_varlen(s.d_H, s.d_doff, s.d_dlen, nd, cfg.threshold,
                                             cfg.mode, nullptr, s.d_starts, s.d_lens,
                                             s.d_counts, ks)))
      return rc;
    // per-patch means (pipeline.rs:240-258) over the same per-document rows
    if (pm.any() && (rc = launch_patch_means(s.d_H, s.d_N, s.d_C, s.d_starts, s.d_counts, nd, 0,
                                             s.d_doff, s.d_dlen, s.d_pH, s.d_pN, s.d_pC, ks)))
      return rc;
    // pieces of arena documents: stitched on the device; the batch holding a
    // document's last piece runs its boundary pass and per-patch means
    for (size_t j = 0; j < s.units.size(); ++j) {
      const Unit& u = units[(size_t)s.units[j]];
      if (u.whole) continue;
      LongDoc& ld = longs[u.doc];
      if (ld.slot < 0) continue;
      const int64_t src = s.h_doff[j];
      if (u.out_lo < 0 || u.out_len < 0 || u.out_lo + u.out_len > ld.L || src < 0 ||
          src + u.out_len > s.out_tokens || ld.base + ld.L > la_cap)
        return fail(BLT_ERR_HIP, "ingest_run: a long document's piece is out of range");
      const size_t nbytes = (size_t)u.out_len * 4;
      const int64_t at = ld.base + u.out_lo;
      BLT_HIP_CHECK(hipMemcpyAsync(la_H + at, s.d_H + src, nbytes, hipMemcpyDeviceToDevice, ks));
      if (pm.any()) {
        BLT_HIP_CHECK(hipMemcpyAsync(la_N + at, s.d_N + src, nbytes, hipMemcpyDeviceToDevice, ks));
        BLT_HIP_CHECK(hipMemcpyAsync(la_C + at, s.d_C + src, nbytes, hipMemcpyDeviceToDevice, ks));
      }
      if (--ld.remaining > 0) continue;
      if ((rc = launch_patch_boundaries_varlen(la_H, la_off + ld.slot, la_len + ld.slot, 1,
                                               cfg.threshold, cfg.mode, nullptr, la_starts,
                                               la_lens, la_count + ld.slot, ks)))
        return rc;
      if (pm.any() &&
          (rc = launch_patch_means(la_H, la_N, la_C, la_starts, la_count + ld.slot, 1, 0,
                                   la_off + ld.slot, la_len + ld.slot, la_pH, la_pN, la_pC, ks)))
        return rc;
      s.long_done.push_back(u.doc);
    }
    BLT_HIP_CHECK(hipEventRecord(s.computed, ks));
    // ---- download ----
    BLT_HIP_CHECK(hipStreamWaitEvent(down, s.computed, 0));
    const size_t ob = (size_t)s.out_tokens * 4;
    BLT_HIP_CHECK(hipMemcpyAsync(s.h_H, s.d_H, ob, hipMemcpyDeviceToHost, down));
    BLT_HIP_CHECK(hipMemcpyAsync(s.h_N, s.d_N, ob, hipMemcpyDeviceToHost, down));
    BLT_HIP_CHECK(hipMemcpyAsync(s.h_C, s.d_C, ob, hipMemcpyDeviceToHost, down));
    if (s.d_E)
      BLT_HIP_CHECK(hipMemcpyAsync(s.h_E, s.d_E, ob * dim, hipMemcpyDeviceToHost, down));
    BLT_HIP_CHECK(hipMemcpyAsync(s.h_starts, s.d_starts, ob, hipMemcpyDeviceToHost, down));
    BLT_HIP_CHECK(hipMemcpyAsync(s.h_lens, s.d_lens, ob, hipMemcpyDeviceToHost, down));
    BLT_HIP_CHECK(hipMemcpyAsync(s.h_counts, s.d_counts, (size_t)nd * 4, hipMemcpyDeviceToHost,
                                 down));
    if (pm.ent) BLT_HIP_CHECK(hipMemcpyAsync(s.h_pH, s.d_pH, ob, hipMemcpyDeviceToHost, down));
    if (pm.prom) BLT_HIP_CHECK(hipMemcpyAsync(s.h_pN, s.d_pN, ob, hipMemcpyDeviceToHost, down));
    if (pm.coh) BLT_HIP_CHECK(hipMemcpyAsync(s.h_pC, s.d_pC, ob, hipMemcpyDeviceToHost, down));
    for (int64_t d : s.long_done) {
      const LongDoc& ld = longs[d];
      const size_t lb = (size_t)ld.L * 4;
      const int64_t b0 = ld.base;
      BLT_HIP_CHECK(hipMemcpyAsync(lh_count + ld.slot, la_count + ld.slot, 4,
                                   hipMemcpyDeviceToHost, down));
      if (starts)
        BLT_HIP_CHECK(hipMemcpyAsync(lh_starts + b0, la_starts + b0, lb, hipMemcpyDeviceToHost, down));
      if (lens)
        BLT_HIP_CHECK(hipMemcpyAsync(lh_lens + b0, la_lens + b0, lb, hipMemcpyDeviceToHost, down));
      if (pm.ent) BLT_HIP_CHECK(hipMemcpyAsync(lh_pH + b0, la_pH + b0, lb, hipMemcpyDeviceToHost, down));
      if (pm.prom) BLT_HIP_CHECK(hipMemcpyAsync(lh_pN + b0, la_pN + b0, lb, hipMemcpyDeviceToHost, down));
      if (pm.coh) BLT_HIP_CHECK(hipMemcpyAsync(lh_pC + b0, la_pC + b0, lb, hipMemcpyDeviceToHost, down));
    }
    BLT_HIP_CHECK(hipEventRecord(s.done, down));
    s.busy = true;
    k ^= 1;
  }
  // the older batch first (slot k would take the next one): a document is
  // released by the batch that holds its last piece, after its earlier pieces
  for (Slot* s : {&slot[k], &slot[k ^ 1]})
    if ((rc = finish(*s, doc_off, ent, nrm, coh, emb, starts, lens, counts, pm))) return rc;
  if (counts)
    for (int64_t dd = 0; dd < n_docs; ++dd)
      if (doc_off[dd + 1] == doc_off[dd]) counts[dd] = 0;
  return 0;
}

// ---- byte tokenizer ---------------------------------------------------------
// Length of the well-formed UTF-8 sequence starting at p[0] (1..4), or 0 when
// p[0] starts an ill-formed one; then *bad is the length of its maximal
// subpart (the prefix of a well-formed sequence, at least 1), which
// from_utf8_lossy replaces by one U+FFFD.  Well-formed sequences are those of
// the Unicode Standard, Table 3-7.
static int utf8_seq(const uint8_t* p, int64_t left, int* bad) {
  const uint8_t b0 = p[0];
  if (b0 < 0x80) return 1;
  int need;
  uint8_t lo = 0x80, hi = 0xBF;  // range of the second byte
  if (b0 >= 0xC2 && b0 <= 0xDF) {
    need = 2;
  } else if (b0 >= 0xE0 && b0 <= 0xEF) {
    need = 3;
    if (b0 == 0xE0) lo = 0xA0;
    if (b0 == 0xED) hi = 0x9F;
  } else if (b0 >= 0xF0 && b0 <= 0xF4) {
    need = 4;
    if (b0 == 0xF0) lo = 0x90;
    if (b0 == 0xF4) hi = 0x8F;
  } else {
    *bad = 1;
    return 0;
  }
  int i = 1;
  for (; i < need && i < left; ++i) {
    const uint8_t b = p[i];
    const uint8_t l = i == 1 ? lo : 0x80, h = i == 1 ? hi : 0xBF;
    if (b < l || b > h) break;
  }
  if (i == need) return need;
  *bad = i;
  return 0;
}

}  // namespace blt

using namespace blt;

extern "C" {

int blt_tokenize_bytes(const uint8_t* bytes, int64_t n, int32_t add_bos, int32_t add_eos,
                       int32_t* tokens, int64_t cap, int64_t* n_tokens) {
  if (n < 0 || (n > 0 && !bytes) || !n_tokens)
    return fail(BLT_ERR_INVALID, "tokenize_bytes: bad argument");
  const int32_t kOffset = 4, kBos = 1, kEos = 2;  // tokenizer.rs:4-8
  int64_t w = 0;
  auto put = [&](int32_t t) {
    if (tokens && w < cap) tokens[w] = t;
    ++w;
  };
  if (add_bos) put(kBos);
  int64_t i = 0;
  while (i < n) {
    int bad = 0;
    const int len = utf8_seq(bytes + i, n - i, &bad);
    if (len) {
      for (int j = 0; j < len; ++j) put((int32_t)bytes[i + j] + kOffset);
      i += len;
    } else {
      put(0xEF + kOffset);
      put(0xBF + kOffset);
      put(0xBD + kOffset);
      i += bad;
    }
  }
  if (add_eos) put(kEos);
  *n_tokens = w;
  if (tokens && w > cap) return fail(BLT_ERR_SHAPE, "tokenize_bytes: capacity too small");
  return BLT_OK;
}

int blt_tokenize_documents(const uint8_t* bytes, const int64_t* byte_offsets, int64_t n_docs,
                           int32_t add_bos, int32_t add_eos, int32_t* tokens, int64_t cap,
                           int64_t* token_offsets) {
  if (n_docs < 0 || !byte_offsets || !token_offsets)
    return fail(BLT_ERR_INVALID, "tokenize_documents: bad argument");
  if (byte_offsets[0] != 0) return fail(BLT_ERR_SHAPE, "tokenize_documents: offsets[0] != 0");
  token_offsets[0] = 0;
  for (int64_t d = 0; d < n_docs; ++d) {
    const int64_t n = byte_offsets[d + 1] - byte_offsets[d];
    if (n < 0) return fail(BLT_ERR_SHAPE, "tokenize_documents: offsets must be non-decreasing");
    const int64_t w = token_offsets[d];
    int64_t got = 0;
    const int rc = blt_tokenize_bytes(bytes + byte_offsets[d], n, add_bos, add_eos,
                                      tokens ? tokens + w : nullptr, tokens ? cap - w : 0, &got);
    if (rc) return rc;
    token_offsets[d + 1] = w + got;
  }
  return BLT_OK;
}

int blt_ingest_plan_chunks(int64_t doc_len, int32_t chunk_len, int32_t overlap,
                           int64_t* starts, int32_t* lens, int32_t* skips, int64_t cap) {
  if (doc_len < 0 || chunk_len <= 0 || overlap < 0 || 2 * (int64_t)overlap > chunk_len)
    return fail(BLT_ERR_SHAPE, "plan_chunks: doc_len >= 0, 0 <= 2 * overlap <= chunk_len");
  std::vector<ChunkPlan> c;
  plan_chunks(doc_len, chunk_len, overlap, c);
  if ((int64_t)c.size() > cap) return fail(BLT_ERR_SHAPE, "plan_chunks: capacity too small");
  if ((int64_t)c.size() > 0x7fffffff) return fail(BLT_ERR_SHAPE, "plan_chunks: too many chunks");
  for (size_t i = 0; i < c.size(); ++i) {
    if (starts) starts[i] = c[i].start;
    if (lens) lens[i] = c[i].len;
    if (skips) skips[i] = c[i].skip;
  }
  return (int)c.size();
}

int blt_ingest_create(blt_model* m, const blt_ingest_config* cfg, blt_ingest** out) {
  if (!m || !cfg || !out) return fail(BLT_ERR_INVALID, "ingest_create: null argument");
  Ingest* g = new Ingest();
  const int rc = g->init(reinterpret_cast<Model*>(m), *cfg);
  if (rc) {
    delete g;
    return rc;
  }
  *out = reinterpret_cast<blt_ingest*>(g);
  return BLT_OK;
}

int blt_ingest_last_stats(blt_ingest* g, blt_ingest_stats* out) {
  if (!g || !out) return fail(BLT_ERR_INVALID, "ingest_last_stats: null argument");
  *out = reinterpret_cast<Ingest*>(g)->stats;
  return BLT_OK;
}

int blt_ingest_destroy(blt_ingest* g) {
  delete reinterpret_cast<Ingest*>(g);
  return BLT_OK;
}

int blt_ingest_run(blt_ingest* g, const int32_t* tokens, const int64_t* doc_offsets,
                   int64_t n_docs, float* entropies, float* norms, float* coherence,
                   float* embeddings, int32_t* starts, int32_t* lengths, int32_t* counts) {
  return blt_ingest_run_patch_means(g, tokens, doc_offsets, n_docs, entropies, norms, coherence,
                                    embeddings, starts, lengths, counts, nullptr, nullptr,
                                    nullptr);
}

int blt_ingest_run_patch_means(blt_ingest* g, const int32_t* tokens, const int64_t* doc_offsets,
                               int64_t n_docs, float* entropies, float* norms, float* coherence,
                               float* embeddings, int32_t* starts, int32_t* lengths,
                               int32_t* counts, float* patch_entropy, float* patch_prominence,
                               float* patch_coherence) {
  if (!g) return fail(BLT_ERR_INVALID, "ingest_run: null handle");
  if (n_docs < 0) return fail(BLT_ERR_SHAPE, "ingest_run: n_docs >= 0");
  if (n_docs == 0) return BLT_OK;
  if (!doc_offsets || (!tokens && doc_offsets[n_docs] > 0))
    return fail(BLT_ERR_INVALID, "ingest_run: null argument");
  if (doc_offsets[0] != 0) return fail(BLT_ERR_SHAPE, "ingest_run: doc_offsets[0] must be 0");
  Ingest::PatchOut pm;
  pm.ent = patch_entropy;
  pm.prom = patch_prominence;
  pm.coh = patch_coherence;
  return reinterpret_cast<Ingest*>(g)->run(tokens, doc_offsets, n_docs, entropies, norms,
                                           coherence, embeddings, starts, lengths, counts, pm);
}

}  // extern "C"
