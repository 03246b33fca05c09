// Streaming pipeline: raw-byte documents -> accumulated entropies / norms and
// the confirmed patches of each chunk, through the entropy-model forward.
//
// Reference semantics (pipeline.rs:111-238, 279-324): a document is read in
// chunks of CHUNK_SIZE bytes; every later chunk also carries the STRIDE bytes
// before it as context, and only its outputs after those are appended to the
// accumulated entropies / norms.  After each chunk the monotonic boundary pass
// runs over everything accumulated, and the patches that start inside the
// chunk's confirmation window are emitted: those at or after (bytes processed
// - STRIDE) and before (chunk start + SAFE_ZONE_END), or all from that lower
// end on for the last chunk (the first chunk's lower end is 0).  A patch ends
// at the next start or at the accumulated end, and carries the left-to-right
// f32 means of the norms and entropies over its span.
//
// Here the accumulated signals stay in device memory.  A start at t >= 2
// depends only on H[t - 1] and H[t], so a chunk's boundary pass runs over the
// accumulated suffix that begins two positions before the window's lower end
// (the suffix's own first two positions are always starts and are dropped):
// the starts of a pass over everything, at a cost bounded by the chunk.  The
// per-patch means of that suffix pass end at the accumulated end, as the
// reference's do.
//
// The batched form (process_documents) runs the chunks of many documents as
// packed segments through the ingest driver: its chunk plan with chunk_len =
// CHUNK_SIZE + STRIDE and overlap = STRIDE is exactly this chunk loop (first
// chunk [0, CHUNK_SIZE), then [p - STRIDE, p + CHUNK_SIZE) keeping [p, ...)).
// The emitted patches of chunk k are then the final starts s inside its
// window, ending at min(next start, accumulated end after chunk k): starts
// below the accumulated end never change once accumulated.  Where that end
// clips a patch, its means are taken on the device over the clipped span.
#include <string.h>

#include <algorithm>
#include <vector>

#include "model.hpp"

namespace blt {
namespace {

constexpr int64_t kChunk = BLT_PIPELINE_CHUNK_SIZE;
constexpr int64_t kStride = BLT_PIPELINE_STRIDE;
constexpr int64_t kSafe = BLT_PIPELINE_SAFE_ZONE_END;
constexpr int64_t kNoCutoff = INT64_MAX;  // the last chunk confirms everything
// clipped spans gathered per device pass of the batched form
constexpr int64_t kSpanBatch = int64_t(1) << 24;

inline int64_t sat_sub(int64_t a, int64_t b) { return a > b ? a - b : 0; }

// Device buffer that only grows; keep = leading bytes carried over (stream-
// ordered copy on s, then the old block is released).
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  int reserve(size_t n, hipStream_t s, size_t keep = 0) {
    if (n <= bytes) return 0;
    const size_t c = std::max(n, 2 * bytes);
    void* q = nullptr;
    BLT_HIP_CHECK(hipMalloc(&q, c));
    if (p) {
      if (keep) BLT_HIP_CHECK(hipMemcpyAsync(q, p, keep, hipMemcpyDeviceToDevice, s));
      BLT_HIP_CHECK(hipStreamSynchronize(s));
      BLT_HIP_CHECK(hipFree(p));
    }
    p = q;
    bytes = c;
    return 0;
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// Pinned host buffer that only grows (contents not kept).
struct HostBuf {
  void* p = nullptr;
  size_t bytes = 0;
  ~HostBuf() {
    if (p) (void)hipHostFree(p);
  }
  int reserve(size_t n) {
    if (n <= bytes) return 0;
    const size_t c = std::max(n, 2 * bytes);
    if (p) BLT_HIP_CHECK(hipHostFree(p));
    p = nullptr;
    bytes = 0;
    BLT_HIP_CHECK(hipHostMalloc(&p, c, 0));
    bytes = c;
    return 0;
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

}  // namespace

struct Pipeline {
  Model* m = nullptr;
  float thr = 0.f;
  hipStream_t s = nullptr;  // the stream of the current call
  // PipelineBuffer state (pipeline.rs:74-89)
  DevBuf acc_H, acc_N;  // accumulated entropies / norms [acc_len]
  int64_t acc_len = 0;
  std::vector<uint8_t> raw;
  int64_t total_processed = 0, chunk_idx = 0, next_patch_idx = 0;
  // one chunk's forward
  HostBuf h_tok;
  DevBuf d_tok, c_H, c_N;
  // boundary pass and means of an accumulated suffix (or of clipped spans)
  DevBuf v_H, v_N, v_starts, v_lens, v_count, v_mH, v_mN, v_off;
  HostBuf hv_starts, hv_count, hv_mH, hv_mN, hv_H, hv_N, hv_off;
  // the batched form's ingest driver
  blt_ingest* ing = nullptr;
  int32_t ing_rows = 0, ing_row_len = 0;

  // every call returns after its stream has drained, so nothing is in flight
  ~Pipeline() {
    if (ing) blt_ingest_destroy(ing);
  }
  int init(Model* model, double threshold) {
    m = model;
    thr = (float)threshold;
    return 0;
  }
  // starts / means of the monotonic pass over H[0, n), N[0, n) (device);
  // leaves count, starts and means in the pinned hv_* buffers
  int suffix_pass(const float* H, const float* N, int64_t n);
  int process_chunk(const uint8_t* chunk, int64_t n, bool is_last, int64_t cap, int64_t* o_start,
                    int64_t* o_len, float* o_prom, float* o_ent, int64_t* n_out);
  int process_documents(const uint8_t* bytes, const int64_t* doc_off, int64_t n_docs,
                        int32_t rows, int32_t row_len, float* ent, float* nrm, int64_t cap,
                        int64_t* o_start, int64_t* o_len, float* o_prom, float* o_ent,
                        int64_t* patch_off);
};

int Pipeline::suffix_pass(const float* H, const float* N, int64_t n) {
  const size_t b = (size_t)n * 4;
  int rc;
  if ((rc = v_starts.reserve(b, s)) || (rc = v_lens.reserve(b, s)) ||
      (rc = v_count.reserve(4, s)) || (rc = v_mH.reserve(b, s)) || (rc = v_mN.reserve(b, s)) ||
      (rc = hv_starts.reserve(b)) || (rc = hv_count.reserve(4)) || (rc = hv_mH.reserve(b)) ||
      (rc = hv_mN.reserve(b)))
    return rc;
  if ((rc = launch_patch_boundaries(H, 1, n, thr, BLT_PATCH_MONOTONIC, nullptr,
                                    v_starts.as<int32_t>(), v_lens.as<int32_t>(),
                                    v_count.as<int32_t>(), s)))
    return rc;
  if ((rc = launch_patch_means(H, N, nullptr, v_starts.as<int32_t>(), v_count.as<int32_t>(), 1, n,
                               nullptr, nullptr, v_mH.as<float>(), v_mN.as<float>(), nullptr, s)))
    return rc;
  BLT_HIP_CHECK(hipMemcpyAsync(hv_count.p, v_count.p, 4, hipMemcpyDeviceToHost, s));
  BLT_HIP_CHECK(hipMemcpyAsync(hv_starts.p, v_starts.p, b, hipMemcpyDeviceToHost, s));
  BLT_HIP_CHECK(hipMemcpyAsync(hv_mH.p, v_mH.p, b, hipMemcpyDeviceToHost, s));
  BLT_HIP_CHECK(hipMemcpyAsync(hv_mN.p, v_mN.p, b, hipMemcpyDeviceToHost, s));
  BLT_HIP_CHECK(hipStreamSynchronize(s));
  const int32_t c = hv_count.as<int32_t>()[0];
  if (c < 0 || c > n) return fail(BLT_ERR_HIP, "pipeline: bad patch count from the device");
  return 0;
}

int Pipeline::process_chunk(const uint8_t* chunk, int64_t n, bool is_last, int64_t cap,
                            int64_t* o_start, int64_t* o_len, float* o_prom, float* o_ent,
                            int64_t* n_out) {
  if (!n_out) return fail(BLT_ERR_INVALID, "pipeline_process_chunk: null n_patches");
  if (n < 0) return fail(BLT_ERR_SHAPE, "pipeline_process_chunk: negative length");
  if (n > 0 && !chunk) return fail(BLT_ERR_INVALID, "pipeline_process_chunk: null chunk");
  if (n > m->cfg.max_seqlen)
    return fail(BLT_ERR_SHAPE, "pipeline_process_chunk: chunk longer than the model's max_seqlen");
  if (n > m->max_tokens)
    return fail(BLT_ERR_SHAPE, "pipeline_process_chunk: chunk longer than the model's max_tokens");
  *n_out = 0;
  const int64_t chunk_start = total_processed;
  const int64_t new_start = chunk_idx == 0 ? 0 : kStride;
  const int64_t added = chunk_idx == 0 ? n : (new_start < n ? n - new_start : 0);
  const int64_t acc_new = acc_len + added;
  const int64_t cutoff = is_last ? kNoCutoff : chunk_start + kSafe;
  const int64_t lower = chunk_idx == 0 ? 0 : sat_sub(total_processed, kStride);
  const int64_t bound = std::max<int64_t>(0, std::min(cutoff, acc_new) - lower);
  if (cap < bound)
    return fail(BLT_ERR_SHAPE, "pipeline_process_chunk: cap below the patches this chunk can "
                               "confirm (the accumulated length after the call suffices)");
  BLT_HIP_CHECK(hipSetDevice(m->device));
  int rc;
  // 1. the forward of this chunk's raw bytes (pipeline.rs:122-127)
  if (n > 0) {
    const size_t b = (size_t)n * 4;
    if ((rc = h_tok.reserve(b)) || (rc = d_tok.reserve(b, s)) || (rc = c_H.reserve(b, s)) ||
        (rc = c_N.reserve(b, s)))
      return rc;
    int32_t* t = h_tok.as<int32_t>();
    for (int64_t i = 0; i < n; ++i) t[i] = chunk[i];
    BLT_HIP_CHECK(hipMemcpyAsync(d_tok.p, h_tok.p, b, hipMemcpyHostToDevice, s));
    blt_model_outputs o{};
    o.entropies = c_H.as<float>();
    o.embedding_norms = c_N.as<float>();
    if ((rc = m->forward(d_tok.as<int32_t>(), 1, n, o, s))) return rc;
  }
  // 2. append the new outputs (pipeline.rs:140-160)
  if (added > 0) {
    const size_t keep = (size_t)acc_len * 4;
    if ((rc = acc_H.reserve((size_t)acc_new * 4, s, keep)) ||
        (rc = acc_N.reserve((size_t)acc_new * 4, s, keep)))
      return rc;
    BLT_HIP_CHECK(hipMemcpyAsync(acc_H.as<float>() + acc_len, c_H.as<float>() + new_start,
                                 (size_t)added * 4, hipMemcpyDeviceToDevice, s));
    BLT_HIP_CHECK(hipMemcpyAsync(acc_N.as<float>() + acc_len, c_N.as<float>() + new_start,
                                 (size_t)added * 4, hipMemcpyDeviceToDevice, s));
    raw.insert(raw.end(), chunk + new_start, chunk + n);
  }
  acc_len = acc_new;
  // 3-5. boundary pass over the accumulated suffix, confirmed patches
  // (pipeline.rs:162-226)
  int64_t w = 0;
  if (bound > 0) {
    const int64_t v0 = lower >= 2 ? lower - 2 : 0;
    const int64_t nv = acc_len - v0;
    if ((rc = suffix_pass(acc_H.as<float>() + v0, acc_N.as<float>() + v0, nv))) return rc;
    const int32_t c = hv_count.as<int32_t>()[0];
    const int32_t* st = hv_starts.as<int32_t>();
    const float* mH = hv_mH.as<float>();
    const float* mN = hv_mN.as<float>();
    for (int32_t j = 0; j < c; ++j) {
      if (v0 > 0 && st[j] < 2) continue;  // the suffix's own forced starts
      const int64_t a = v0 + st[j];
      if (a < lower || a >= cutoff) continue;
      const int64_t e = j + 1 < c ? v0 + st[j + 1] : acc_len;
      if (o_start) o_start[w] = a;
      if (o_len) o_len[w] = e - a;
      if (o_prom) o_prom[w] = mN[j];
      if (o_ent) o_ent[w] = mH[j];
      ++w;
    }
  } else {
    BLT_HIP_CHECK(hipStreamSynchronize(s));
  }
  // state update (pipeline.rs:228-235)
  next_patch_idx += w;
  total_processed = is_last ? chunk_start + n : chunk_start + sat_sub(n, kStride);
  chunk_idx += 1;
  *n_out = w;
  return 0;
}

int Pipeline::process_documents(const uint8_t* bytes, const int64_t* doc_off, int64_t n_docs,
                                int32_t rows, int32_t row_len, float* ent, float* nrm,
                                int64_t cap, int64_t* o_start, int64_t* o_len, float* o_prom,
                                float* o_ent, int64_t* patch_off) {
  if (n_docs < 0) return fail(BLT_ERR_SHAPE, "pipeline_process_documents: n_docs >= 0");
  if (!doc_off || !patch_off) return fail(BLT_ERR_INVALID, "pipeline_process_documents: null "
                                                           "doc_offsets or patch_offsets");
  if (doc_off[0] != 0) return fail(BLT_ERR_SHAPE, "pipeline_process_documents: doc_offsets[0] "
                                                  "must be 0");
  for (int64_t d = 0; d < n_docs; ++d)
    if (doc_off[d + 1] < doc_off[d])
      return fail(BLT_ERR_SHAPE, "pipeline_process_documents: doc_offsets must not decrease");
  const int64_t total = doc_off[n_docs];
  if (total > 0 && !bytes) return fail(BLT_ERR_INVALID, "pipeline_process_documents: null bytes");
  if (row_len < kChunk + kStride)
    return fail(BLT_ERR_SHAPE, "pipeline_process_documents: row_len below CHUNK_SIZE + STRIDE");
  patch_off[0] = 0;
  if (n_docs == 0) return 0;
  int rc;
  if (!ing || ing_rows != rows || ing_row_len != row_len) {
    if (ing) blt_ingest_destroy(ing);
    ing = nullptr;
    blt_ingest_config c{};
    c.rows = rows;
    c.row_len = row_len;
    c.chunk_len = (int32_t)(kChunk + kStride);
    c.overlap = (int32_t)kStride;
    c.threshold = thr;
    c.mode = BLT_PATCH_MONOTONIC;
    c.with_embeddings = 0;
    if ((rc = blt_ingest_create(reinterpret_cast<blt_model*>(m), &c, &ing))) return rc;
    ing_rows = rows;
    ing_row_len = row_len;
  }
  // raw bytes as tokens, no offset (pipeline.rs:123)
  std::vector<int32_t> tok((size_t)total);
  for (int64_t i = 0; i < total; ++i) tok[(size_t)i] = bytes[i];
  std::vector<float> own_H, own_N;
  if (!ent) own_H.resize((size_t)total), ent = own_H.data();
  if (!nrm) own_N.resize((size_t)total), nrm = own_N.data();
  std::vector<int32_t> S((size_t)total), counts((size_t)n_docs);
  std::vector<float> pH((size_t)total), pN((size_t)total);
  if ((rc = blt_ingest_run_patch_means(ing, tok.data(), doc_off, n_docs, ent, nrm, nullptr,
                                       nullptr, S.data(), nullptr, counts.data(), pH.data(),
                                       pN.data(), nullptr)))
    return rc;
  tok = std::vector<int32_t>();
  // The chunk loop of process_document (pipeline.rs:292-317) with the window
  // of process_chunk (pipeline.rs:176-202) over document d's final starts;
  // emit(i, end, clipped) per confirmed patch, in the reference's order.
  auto walk = [&](int64_t d, auto&& emit) {
    const int64_t L = doc_off[d + 1] - doc_off[d];
    const int32_t* st = S.data() + doc_off[d];
    const int64_t ns = counts[(size_t)d];
    int64_t tbp = 0, ci = 0, acc = 0, pos = 0;
    while (pos < L) {
      const int64_t chunk_end = std::min(pos + kChunk, L);
      const bool last = chunk_end >= L;
      const int64_t a = pos > 0 ? sat_sub(pos, kStride) : 0;
      const int64_t clen = chunk_end - a;
      const int64_t cstart = tbp;
      acc += ci == 0 ? clen : (kStride < clen ? clen - kStride : 0);
      const int64_t cutoff = last ? kNoCutoff : cstart + kSafe;
      const int64_t lower = ci == 0 ? 0 : sat_sub(tbp, kStride);
      int64_t i = std::lower_bound(st, st + ns, (int32_t)std::min<int64_t>(lower, INT32_MAX)) - st;
      for (; i < ns && st[i] < cutoff && st[i] < acc; ++i) {
        const int64_t fin = i + 1 < ns ? st[i + 1] : L;
        const int64_t e = std::min(fin, acc);
        emit(i, e, e != fin);
      }
      tbp = last ? cstart + clen : cstart + sat_sub(clen, kStride);
      ci += 1;
      if (last) break;
      pos = chunk_end;
    }
  };
  for (int64_t d = 0; d < n_docs; ++d) {
    int64_t k = 0;
    walk(d, [&](int64_t, int64_t, bool) { ++k; });
    patch_off[d + 1] = patch_off[d] + k;
  }
  if (patch_off[n_docs] > cap)
    return fail(BLT_ERR_SHAPE, "pipeline_process_documents: cap below the patches emitted "
                               "(total + STRIDE * n_docs suffices)");
  // clipped patches: spans gathered on the host, means on the device
  struct Clip {
    int64_t slot, off;
  };
  std::vector<Clip> clips;
  std::vector<float> span_H, span_N;
  int64_t span_n = 0;
  auto flush = [&]() -> int {
    if (clips.empty()) return 0;
    // one row (one block) per clipped span, its mean written to slot j
    const size_t nc = clips.size();
    const size_t b = (size_t)span_n * 4;
    int r;
    if ((r = v_H.reserve(b, s)) || (r = v_N.reserve(b, s)) || (r = v_mH.reserve(nc * 4, s)) ||
        (r = v_mN.reserve(nc * 4, s)) || (r = v_off.reserve(nc * 16, s)) ||
        (r = v_lens.reserve(nc * 4, s)) || (r = hv_H.reserve(b)) || (r = hv_N.reserve(b)) ||
        (r = hv_off.reserve(nc * 16)) || (r = hv_starts.reserve(nc * 4)) ||
        (r = hv_mH.reserve(nc * 4)) || (r = hv_mN.reserve(nc * 4)))
      return r;
    memcpy(hv_H.p, span_H.data(), b);
    memcpy(hv_N.p, span_N.data(), b);
    int64_t* ho = hv_off.as<int64_t>();  // [nc] span offsets, then [nc] output slots
    int32_t* hl = hv_starts.as<int32_t>();
    for (size_t j = 0; j < nc; ++j) {
      const int64_t end = j + 1 < nc ? clips[j + 1].off : span_n;
      ho[j] = clips[j].off;
      ho[nc + j] = (int64_t)j;
      hl[j] = (int32_t)(end - clips[j].off);
    }
    BLT_HIP_CHECK(hipSetDevice(m->device));
    BLT_HIP_CHECK(hipMemcpyAsync(v_H.p, hv_H.p, b, hipMemcpyHostToDevice, s));
    BLT_HIP_CHECK(hipMemcpyAsync(v_N.p, hv_N.p, b, hipMemcpyHostToDevice, s));
    BLT_HIP_CHECK(hipMemcpyAsync(v_off.p, hv_off.p, nc * 16, hipMemcpyHostToDevice, s));
    BLT_HIP_CHECK(hipMemcpyAsync(v_lens.p, hv_starts.p, nc * 4, hipMemcpyHostToDevice, s));
    const int64_t* d_off = v_off.as<int64_t>();
    if ((r = launch_patch_means(v_H.as<float>(), v_N.as<float>(), nullptr, nullptr, nullptr,
                                (int64_t)nc, 0, d_off, v_lens.as<int32_t>(), v_mH.as<float>(),
                                v_mN.as<float>(), nullptr, s, d_off + nc)))
      return r;
    BLT_HIP_CHECK(hipMemcpyAsync(hv_mH.p, v_mH.p, nc * 4, hipMemcpyDeviceToHost, s));
    BLT_HIP_CHECK(hipMemcpyAsync(hv_mN.p, v_mN.p, nc * 4, hipMemcpyDeviceToHost, s));
    BLT_HIP_CHECK(hipStreamSynchronize(s));
    for (size_t j = 0; j < nc; ++j) {
      if (o_prom) o_prom[clips[j].slot] = hv_mN.as<float>()[j];
      if (o_ent) o_ent[clips[j].slot] = hv_mH.as<float>()[j];
    }
    clips.clear();
    span_H.clear();
    span_N.clear();
    span_n = 0;
    return 0;
  };
  for (int64_t d = 0; d < n_docs; ++d) {
    const int64_t base = doc_off[d];
    const int32_t* st = S.data() + base;
    int64_t w = patch_off[d];
    int err = 0;
    walk(d, [&](int64_t i, int64_t e, bool clipped) {
      if (err) return;
      const int64_t a = st[i];
      if (o_start) o_start[w] = a;
      if (o_len) o_len[w] = e - a;
      if (!clipped) {
        if (o_prom) o_prom[w] = pN[(size_t)(base + i)];
        if (o_ent) o_ent[w] = pH[(size_t)(base + i)];
      } else if (o_prom || o_ent) {
        const int64_t len = e - a;
        if (span_n + len > kSpanBatch && (err = flush())) return;
        span_H.insert(span_H.end(), ent + base + a, ent + base + e);
        span_N.insert(span_N.end(), nrm + base + a, nrm + base + e);
        clips.push_back({w, span_n});
        span_n += len;
      }
      ++w;
    });
    if (err) return err;
  }
  return flush();
}

}  // namespace blt

using blt::fail;
using blt::Pipeline;

extern "C" {

int blt_pipeline_create(blt_model* m, double threshold, blt_pipeline** out) {
  if (!m || !out) return fail(BLT_ERR_INVALID, "pipeline_create: null argument");
  Pipeline* p = new Pipeline();
  const int rc = p->init(reinterpret_cast<blt::Model*>(m), threshold);
  if (rc) {
    delete p;
    return rc;
  }
  *out = reinterpret_cast<blt_pipeline*>(p);
  return BLT_OK;
}

int blt_pipeline_destroy(blt_pipeline* p) {
  delete reinterpret_cast<Pipeline*>(p);
  return BLT_OK;
}

int blt_pipeline_process_chunk(blt_pipeline* p, const uint8_t* chunk, int64_t n, int32_t is_last,
                               int64_t cap, int64_t* start, int64_t* length, float* prominence,
                               float* entropy, int64_t* n_patches, blt_stream_t stream) {
  if (!p) return fail(BLT_ERR_INVALID, "pipeline_process_chunk: null handle");
  reinterpret_cast<Pipeline*>(p)->s = reinterpret_cast<hipStream_t>(stream);
  return reinterpret_cast<Pipeline*>(p)->process_chunk(chunk, n, is_last != 0, cap, start, length,
                                                       prominence, entropy, n_patches);
}

int blt_pipeline_reset(blt_pipeline* p) {
  if (!p) return fail(BLT_ERR_INVALID, "pipeline_reset: null handle");
  Pipeline* q = reinterpret_cast<Pipeline*>(p);
  q->acc_len = 0;
  q->raw.clear();
  q->total_processed = q->chunk_idx = q->next_patch_idx = 0;
  return BLT_OK;
}

int blt_pipeline_accumulated(blt_pipeline* p, int64_t* len) {
  if (!p || !len) return fail(BLT_ERR_INVALID, "pipeline_accumulated: null argument");
  *len = reinterpret_cast<Pipeline*>(p)->acc_len;
  return BLT_OK;
}

int blt_pipeline_read(blt_pipeline* p, int64_t offset, int64_t n, float* entropies, float* norms,
                      uint8_t* raw_bytes, blt_stream_t stream) {
  if (!p) return fail(BLT_ERR_INVALID, "pipeline_read: null handle");
  Pipeline* q = reinterpret_cast<Pipeline*>(p);
  q->s = reinterpret_cast<hipStream_t>(stream);
  if (offset < 0 || n < 0 || offset + n > q->acc_len)
    return fail(BLT_ERR_SHAPE, "pipeline_read: range outside the accumulated positions");
  if (n == 0) return BLT_OK;
  BLT_HIP_CHECK(hipSetDevice(q->m->device));
  if (entropies)
    BLT_HIP_CHECK(hipMemcpyAsync(entropies, q->acc_H.as<float>() + offset, (size_t)n * 4,
                                 hipMemcpyDeviceToHost, q->s));
  if (norms)
    BLT_HIP_CHECK(hipMemcpyAsync(norms, q->acc_N.as<float>() + offset, (size_t)n * 4,
                                 hipMemcpyDeviceToHost, q->s));
  BLT_HIP_CHECK(hipStreamSynchronize(q->s));
  if (raw_bytes) memcpy(raw_bytes, q->raw.data() + offset, (size_t)n);
  return BLT_OK;
}

int blt_pipeline_process_documents(blt_pipeline* p, const uint8_t* bytes,
                                   const int64_t* doc_offsets, int64_t n_docs, int32_t rows,
                                   int32_t row_len, float* entropies, float* norms, int64_t cap,
                                   int64_t* start, int64_t* length, float* prominence,
                                   float* entropy, int64_t* patch_offsets,
                                   blt_stream_t stream) {
  if (!p) return fail(BLT_ERR_INVALID, "pipeline_process_documents: null handle");
  Pipeline* q = reinterpret_cast<Pipeline*>(p);
  q->s = reinterpret_cast<hipStream_t>(stream);
  // the ingest driver runs on streams of its own: let the caller's earlier
  // work on this model finish first
  if (q->m) {
    BLT_HIP_CHECK(hipSetDevice(q->m->device));
    BLT_HIP_CHECK(hipStreamSynchronize(q->s));
  }
  return reinterpret_cast<Pipeline*>(p)->process_documents(bytes, doc_offsets, n_docs, rows,
                                                           row_len, entropies, norms, cap, start,
                                                           length, prominence, entropy,
                                                           patch_offsets);
}

}  // extern "C"
