// extern "C" entry points (include/blt_hip.h): argument checks, error
// reporting, the synthetic-input generators and the model handle.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "model.hpp"

namespace blt {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
int fail(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}
int hip_fail(hipError_t e, const char* what) {
  g_last_error = std::string(what) + ": " + hipGetErrorString(e);
  return BLT_ERR_HIP;
}

namespace {

// splitmix64 evaluated at an arbitrary counter: the i-th output of a
// generator seeded with `seed` is mix(seed + (i + 1) * golden).
inline uint64_t sm64_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
// uniform in (0, 1)
inline double u01_at(uint64_t seed, uint64_t i) {
  return ((double)(sm64_at(seed, i) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}
// standard normal i: Box-Muller over the uniform pair (2*(i/2), 2*(i/2)+1),
// cos branch for even i, sin branch for odd i.
inline double normal_at(uint64_t seed, uint64_t i) {
  const uint64_t pr = i >> 1;
  const double u1 = u01_at(seed, 2 * pr), u2 = u01_at(seed, 2 * pr + 1);
  const double r = sqrt(-2.0 * log(u1));
  const double th = 6.283185307179586476925286766559 * u2;
  return (i & 1) ? r * sin(th) : r * cos(th);
}

// Split [0, n) over up to 16 host threads (the generators are counter based,
// so the output does not depend on the split).
template <typename F>
void parallel_for(int64_t n, F f) {
  int nt = (int)std::min<unsigned>(16u, std::max(1u, std::thread::hardware_concurrency()));
  if (n < (int64_t)1 << 16) nt = 1;
  if (nt == 1) {
    for (int64_t i = 0; i < n; ++i) f(i);
    return;
  }
  std::vector<std::thread> th;
  const int64_t chunk = (n + nt - 1) / nt;
  for (int t = 0; t < nt; ++t) {
    const int64_t lo = t * chunk, hi = std::min(n, lo + chunk);
    if (lo >= hi) break;
    th.emplace_back([=]() {
      for (int64_t i = lo; i < hi; ++i) f(i);
    });
  }
  for (auto& x : th) x.join();
}

int check_stream_ptrs(const void* a, const void* b) {
  if (a == nullptr || b == nullptr) return fail(BLT_ERR_INVALID, "null tensor pointer");
  return 0;
}

}  // namespace
}  // namespace blt

using namespace blt;

#define STREAM(s) reinterpret_cast<hipStream_t>(s)

extern "C" {

const char* blt_last_error(void) { return g_last_error.c_str(); }
const char* blt_version(void) { return "blt_hip 0.1.0 (gfx950)"; }

int blt_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

int blt_stream_sync(blt_stream_t stream) {
  BLT_HIP_CHECK(hipStreamSynchronize(STREAM(stream)));
  return BLT_OK;
}

// ---- fused ops -------------------------------------------------------------
int blt_fused_entropy_f32(const float* logits, float* out, int64_t rows, int32_t vocab,
                          blt_stream_t stream) {
  if (rows < 0 || vocab <= 0) return fail(BLT_ERR_SHAPE, "fused_entropy: rows >= 0, vocab > 0");
  if (rows == 0) return BLT_OK;
  if (int rc = check_stream_ptrs(logits, out)) return rc;
  return launch_entropy_f32(logits, out, rows, vocab, STREAM(stream));
}
int blt_fused_entropy_bf16(const uint16_t* logits, float* out, int64_t rows, int32_t vocab,
                           blt_stream_t stream) {
  if (rows < 0 || vocab <= 0) return fail(BLT_ERR_SHAPE, "fused_entropy: rows >= 0, vocab > 0");
  if (rows == 0) return BLT_OK;
  if (int rc = check_stream_ptrs(logits, out)) return rc;
  return launch_entropy_bf16(logits, out, rows, vocab, STREAM(stream));
}

static int rms_checks(const void* x, const void* w, const void* y, const void* l2, int64_t rows,
                      int32_t dim, int32_t eps_mode) {
  if (rows < 0 || dim <= 0) return fail(BLT_ERR_SHAPE, "fused_rms_norm: rows >= 0, dim > 0");
  if (eps_mode != BLT_EPS_AFTER_SQRT && eps_mode != BLT_EPS_INSIDE_SQRT)
    return fail(BLT_ERR_INVALID, "fused_rms_norm: bad eps_mode");
  if (rows == 0) return 1;
  if (x == nullptr || (y == nullptr && l2 == nullptr) || (y != nullptr && w == nullptr))
    return fail(BLT_ERR_INVALID, "fused_rms_norm: null pointer");
  return 0;
}
int blt_fused_rms_norm_f32(const float* x, const float* w, float* y, float* l2_out,
                           int64_t rows, int32_t dim, float eps, int32_t eps_mode,
                           blt_stream_t stream) {
  int rc = rms_checks(x, w, y, l2_out, rows, dim, eps_mode);
  if (rc) return rc > 0 ? BLT_OK : rc;
  return launch_rmsnorm<float, float, float>(x, w, y, l2_out, rows, dim, eps, eps_mode,
                                             STREAM(stream));
}
int blt_fused_rms_norm_bf16(const uint16_t* x, const uint16_t* w, uint16_t* y, float* l2_out,
                            int64_t rows, int32_t dim, float eps, int32_t eps_mode,
                            blt_stream_t stream) {
  int rc = rms_checks(x, w, y, l2_out, rows, dim, eps_mode);
  if (rc) return rc > 0 ? BLT_OK : rc;
  return launch_rmsnorm<uint16_t, uint16_t, uint16_t>(x, w, y, l2_out, rows, dim, eps, eps_mode,
                                                      STREAM(stream));
}

int blt_fused_softmax_f32(const float* x, float* y, int64_t rows, int32_t n,
                          blt_stream_t stream) {
  if (rows < 0 || n <= 0) return fail(BLT_ERR_SHAPE, "fused_softmax: rows >= 0, n > 0");
  if (rows == 0) return BLT_OK;
  if (int rc = check_stream_ptrs(x, y)) return rc;
  return launch_softmax_f32(x, y, rows, n, STREAM(stream));
}

int blt_fused_l2_norm_f32(const float* x, float* out, int64_t rows, int32_t dim,
                          blt_stream_t stream) {
  if (rows < 0 || dim <= 0) return fail(BLT_ERR_SHAPE, "fused_l2_norm: rows >= 0, dim > 0");
  if (rows == 0) return BLT_OK;
  if (int rc = check_stream_ptrs(x, out)) return rc;
  return launch_rmsnorm<float, float, float>(x, nullptr, nullptr, out, rows, dim, 0.f, 0,
                                             STREAM(stream));
}
int blt_fused_l2_norm_bf16(const uint16_t* x, float* out, int64_t rows, int32_t dim,
                           blt_stream_t stream) {
  if (rows < 0 || dim <= 0) return fail(BLT_ERR_SHAPE, "fused_l2_norm: rows >= 0, dim > 0");
  if (rows == 0) return BLT_OK;
  if (int rc = check_stream_ptrs(x, out)) return rc;
  return launch_rmsnorm<uint16_t, uint16_t, uint16_t>(x, nullptr, nullptr, out, rows, dim, 0.f,
                                                      0, STREAM(stream));
}

int blt_fused_silu_gate_f32(const float* g, const float* u, float* out, int64_t n,
                            blt_stream_t stream) {
  if (n < 0) return fail(BLT_ERR_SHAPE, "fused_silu_gate: n >= 0");
  if (n == 0) return BLT_OK;
  if (!g || !u || !out) return fail(BLT_ERR_INVALID, "fused_silu_gate: null pointer");
  return launch_silu_gate_f32(g, u, out, n, STREAM(stream));
}
int blt_fused_silu_gate_bf16(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t n,
                             blt_stream_t stream) {
  if (n < 0) return fail(BLT_ERR_SHAPE, "fused_silu_gate: n >= 0");
  if (n == 0) return BLT_OK;
  if (!g || !u || !out) return fail(BLT_ERR_INVALID, "fused_silu_gate: null pointer");
  return launch_silu_gate_bf16(g, u, out, n, STREAM(stream));
}

int blt_fused_coherence_f32(const float* norms, const float* entropies, float* out,
                            int64_t n, float eps, blt_stream_t stream) {
  if (n < 0) return fail(BLT_ERR_SHAPE, "fused_coherence: n >= 0");
  if (n == 0) return BLT_OK;
  if (!norms || !entropies || !out) return fail(BLT_ERR_INVALID, "fused_coherence: null pointer");
  return launch_coherence(norms, entropies, out, n, eps, STREAM(stream));
}

// ---- attention ---------------------------------------------------------------
int64_t blt_attention_workspace_bytes(int64_t B, int64_t H, int64_t T, int32_t d) {
  if (B < 0 || H < 0 || T < 0 || d <= 0) return 0;
  return B * H * T * d * 2 + T * d * 4 + 256;  // the rotated k copy (q is rotated in the kernel)
}

// RoPE tables of the fused attention entry, one per (device, head_dim, theta):
// built on the host in the reference's f32 order (so every value equals the
// reference table) and uploaded once; a longer sequence rebuilds it at the
// new length.  Tables live until the process ends.
namespace {
struct RopeCache {
  std::mutex mu;
  struct Entry {
    float* ptr = nullptr;
    int64_t len = 0;
  };
  std::map<std::tuple<int, int, uint32_t>, Entry> tables;
} g_rope;
}  // namespace

static int rope_table_device(int d, int64_t T, float theta, const float** out) {
  int dev = 0;
  BLT_HIP_CHECK(hipGetDevice(&dev));
  uint32_t tbits;
  memcpy(&tbits, &theta, 4);
  std::lock_guard<std::mutex> lock(g_rope.mu);
  RopeCache::Entry& e = g_rope.tables[std::make_tuple(dev, d, tbits)];
  if (e.len < T) {
    std::vector<float> host((size_t)T * d);
    rope_table_host(host.data(), d, (int)T, theta);
    float* p = nullptr;
    BLT_HIP_CHECK(hipMalloc((void**)&p, host.size() * 4));
    // synchronous: the table is complete before any launch can read it
    BLT_HIP_CHECK(hipMemcpy(p, host.data(), host.size() * 4, hipMemcpyHostToDevice));
    // kernels queued earlier may still read the old table; hipFree waits for them
    if (e.ptr) BLT_HIP_CHECK(hipFree(e.ptr));
    e.ptr = p;
    e.len = T;
  }
  *out = e.ptr;
  return 0;
}

int blt_fused_attention_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             uint16_t* o, int64_t B, int64_t H, int64_t T, int32_t d,
                             int64_t sb_q, int64_t sh_q, int64_t st_q, int64_t sb_kv,
                             int64_t sh_kv, int64_t st_kv, int64_t sb_o, int64_t sh_o,
                             int64_t st_o, int32_t causal, int32_t window, float rope_theta,
                             void* workspace, blt_stream_t stream) {
  if (d != 64) return fail(BLT_ERR_SHAPE, "fused_attention: only head_dim 64 is supported");
  if (B < 0 || H < 0 || T < 0) return fail(BLT_ERR_SHAPE, "fused_attention: negative shape");
  if (window < 0) return fail(BLT_ERR_SHAPE, "fused_attention: window must be >= 0");
  if (B == 0 || H == 0 || T == 0) return BLT_OK;
  if (!q || !k || !v || !o) return fail(BLT_ERR_INVALID, "fused_attention: null pointer");
  const int64_t strides[] = {sb_q, sh_q, st_q, sb_kv, sh_kv, st_kv, sb_o, sh_o, st_o};
  for (int64_t s : strides)
    if (s < 0 || s % 8 != 0)
      return fail(BLT_ERR_SHAPE, "fused_attention: strides must be >= 0 and multiples of 8");
  hipStream_t s = STREAM(stream);
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o;
  a.B = B; a.H = H; a.T = T;
  a.sb_q = sb_q; a.sh_q = sh_q; a.st_q = st_q;
  a.sb_k = sb_kv; a.sh_k = sh_kv; a.st_k = st_kv;
  a.sb_v = sb_kv; a.sh_v = sh_kv; a.st_v = st_kv;
  a.sb_o = sb_o; a.sh_o = sh_o; a.st_o = st_o;
  a.causal = causal ? 1 : 0; a.window = window;
  if (rope_theta > 0.f) {
    // k is rotated into a dense head-major copy in the workspace (each K row
    // is read by many query blocks); q is rotated inside the attention kernel
    // as it is loaded (once per query)
    if (workspace == nullptr)
      return fail(BLT_ERR_INVALID, "fused_attention: rope needs a workspace");
    uint16_t* kr = reinterpret_cast<uint16_t*>(workspace);
    const float* cs = nullptr;
    int rc;
    if ((rc = rope_table_device(d, T, rope_theta, &cs))) return rc;
    if ((rc = launch_rope(k, kr, cs, B, H, T, d, sb_kv, sh_kv, st_kv, s))) return rc;
    a.k = kr; a.sb_k = H * T * d; a.sh_k = T * d; a.st_k = d;
    a.q_rope_cs = cs;
  }
  return launch_attention(a, s);
}

int blt_fused_attention_f32(const float* q, const float* k, const float* v, float* o, int64_t B,
                            int64_t H, int64_t Tq, int64_t Tkv, int32_t d, int32_t causal,
                            blt_stream_t stream) {
  if (B < 0 || H < 0 || Tq < 0 || Tkv < 0) return fail(BLT_ERR_SHAPE, "attention_f32: negative shape");
  if (d < 1 || d > 256) return fail(BLT_ERR_SHAPE, "attention_f32: head_dim must be 1 .. 256");
  if (B == 0 || H == 0 || Tq == 0) return BLT_OK;
  if (!q || !o || (Tkv > 0 && (!k || !v)))
    return fail(BLT_ERR_INVALID, "attention_f32: null pointer");
  return launch_attention_f32(q, k, v, o, B, H, Tq, Tkv, d, causal, STREAM(stream));
}

int blt_rope_table_f32(float* out_device, int32_t head_dim, int32_t max_seqlen, double theta,
                       blt_stream_t stream) {
  if (head_dim <= 0 || head_dim % 2 || max_seqlen < 0)
    return fail(BLT_ERR_SHAPE, "rope_table: head_dim even > 0, max_seqlen >= 0");
  if (max_seqlen == 0) return BLT_OK;
  if (!out_device) return fail(BLT_ERR_INVALID, "rope_table: null pointer");
  std::vector<float> host((size_t)max_seqlen * head_dim);
  rope_table_host(host.data(), head_dim, max_seqlen, theta);
  BLT_HIP_CHECK(hipMemcpyAsync(out_device, host.data(), host.size() * 4, hipMemcpyHostToDevice,
                               STREAM(stream)));
  BLT_HIP_CHECK(hipStreamSynchronize(STREAM(stream)));
  return BLT_OK;
}

// ---- patcher -----------------------------------------------------------------
int blt_patch_boundaries(const float* H, int64_t B, int64_t T, float thr, int32_t mode,
                         int32_t* mask, int32_t* starts, int32_t* lengths, int32_t* count,
                         blt_stream_t stream) {
  if (B < 0 || T < 0) return fail(BLT_ERR_SHAPE, "patch_boundaries: negative shape");
  if (T > 0x7fffffff) return fail(BLT_ERR_SHAPE, "patch_boundaries: T must fit int32");
  if (mode != BLT_PATCH_MONOTONIC && mode != BLT_PATCH_GLOBAL)
    return fail(BLT_ERR_INVALID, "patch_boundaries: bad mode");
  if (lengths && !starts)
    return fail(BLT_ERR_INVALID, "patch_boundaries: lengths needs the starts buffer");
  if (B == 0) return BLT_OK;
  if (T > 0 && !H) return fail(BLT_ERR_INVALID, "patch_boundaries: null entropies");
  return launch_patch_boundaries(H, B, T, thr, mode, mask, starts, lengths, count,
                                 STREAM(stream));
}

int blt_patch_mask_starts(const int32_t* mask, int64_t B, int64_t T, int32_t* starts,
                          int32_t* lengths, int32_t* count, blt_stream_t stream) {
  if (B < 0 || T < 0) return fail(BLT_ERR_SHAPE, "patch_mask_starts: negative shape");
  if (T > 0x7fffffff) return fail(BLT_ERR_SHAPE, "patch_mask_starts: T must fit int32");
  if (lengths && !starts)
    return fail(BLT_ERR_INVALID, "patch_mask_starts: lengths needs the starts buffer");
  if (B == 0) return BLT_OK;
  if (T > 0 && !mask) return fail(BLT_ERR_INVALID, "patch_mask_starts: null mask");
  return launch_patch_mask_starts(mask, B, T, starts, lengths, count, STREAM(stream));
}

int blt_patch_means(const float* entropies, const float* norms, const float* coherence,
                    const int32_t* starts, const int32_t* count, int64_t B, int64_t T,
                    float* mean_entropy, float* mean_prominence, float* mean_coherence,
                    blt_stream_t stream) {
  if (B < 0 || T < 0) return fail(BLT_ERR_SHAPE, "patch_means: negative shape");
  if (T > 0x7fffffff) return fail(BLT_ERR_SHAPE, "patch_means: T must fit int32");
  if ((coherence == nullptr) != (mean_coherence == nullptr))
    return fail(BLT_ERR_INVALID, "patch_means: coherence and mean_coherence come as a pair");
  if (B == 0) return BLT_OK;
  if (!entropies || !norms || !starts || !count)
    return fail(BLT_ERR_INVALID, "patch_means: null entropies, norms, starts or count");
  return launch_patch_means(entropies, norms, coherence, starts, count, B, T, nullptr, nullptr,
                            mean_entropy, mean_prominence, mean_coherence, STREAM(stream));
}

int64_t blt_patch_workspace_bytes(int64_t B, int64_t T, int32_t n_rules) {
  return patch_workspace_bytes(B, T, n_rules);
}

int blt_patch_boundaries_rules(const float* H, int64_t B, int64_t T, int32_t n_rules,
                               const blt_patch_rule* rules, void* workspace,
                               int64_t workspace_bytes, blt_stream_t stream) {
  return launch_patch_rules(H, B, T, n_rules, rules, workspace, workspace_bytes, STREAM(stream));
}

int blt_patch_boundaries_rules_noalloc(const float* H, int64_t B, int64_t T, int32_t n_rules,
                                       const blt_patch_rule* rules, blt_stream_t stream) {
  return launch_patch_rules_noalloc(H, B, T, n_rules, rules, STREAM(stream));
}

int blt_entropy_patch_boundaries(const float* logits, int64_t B, int64_t T, int32_t vocab,
                                 float* entropies, int32_t n_rules, const blt_patch_rule* rules,
                                 void* workspace, int64_t workspace_bytes, blt_stream_t stream) {
  return launch_entropy_patch(logits, B, T, vocab, entropies, n_rules, rules, workspace,
                              workspace_bytes, STREAM(stream));
}

// ---- model -------------------------------------------------------------------
int blt_model_create(int32_t device, const blt_model_config* cfg, const blt_model_weights* w,
                     int64_t max_tokens, blt_model** out) {
  if (!cfg || !w || !out) return fail(BLT_ERR_INVALID, "model_create: null argument");
  Model* m = nullptr;
  int rc = Model::create(device, *cfg, *w, max_tokens, &m);
  if (rc) return rc;
  *out = reinterpret_cast<blt_model*>(m);
  return BLT_OK;
}
int blt_model_destroy(blt_model* m) {
  delete reinterpret_cast<Model*>(m);
  return BLT_OK;
}
int64_t blt_model_device_bytes(const blt_model* m) {
  return m ? reinterpret_cast<const Model*>(m)->bytes : 0;
}
int blt_model_forward(blt_model* m, const int32_t* tokens, int64_t B, int64_t T,
                      const blt_model_outputs* out, blt_stream_t stream) {
  if (!m || !out) return fail(BLT_ERR_INVALID, "model_forward: null argument");
  return reinterpret_cast<Model*>(m)->forward(tokens, B, T, *out, STREAM(stream));
}

int blt_model_extract_embeddings(blt_model* m, const int32_t* tokens, int64_t B, int64_t T,
                                 float* out, blt_stream_t stream) {
  if (!m) return fail(BLT_ERR_INVALID, "model_extract_embeddings: null model");
  if (!out && B * T > 0) return fail(BLT_ERR_INVALID, "model_extract_embeddings: null output");
  blt_model_outputs o{};
  o.pre_norm_embeddings = out;
  return reinterpret_cast<Model*>(m)->forward(tokens, B, T, o, STREAM(stream));
}

int blt_model_forward_segments(blt_model* m, const int32_t* tokens, const int32_t* seg_start,
                               int64_t B, int64_t T, const blt_model_outputs* out,
                               blt_stream_t stream) {
  if (!m || !out) return fail(BLT_ERR_INVALID, "model_forward_segments: null argument");
  if (!seg_start && B * T > 0)
    return fail(BLT_ERR_INVALID, "model_forward_segments: null seg_start");
  return reinterpret_cast<Model*>(m)->forward(tokens, B, T, *out, STREAM(stream), seg_start);
}

int blt_model_set_profiling(blt_model* m, int32_t on) {
  if (!m) return fail(BLT_ERR_INVALID, "model_set_profiling: null model");
  reinterpret_cast<Model*>(m)->profiling = on != 0;
  return BLT_OK;
}
int blt_model_read_profile(blt_model* m, double* ms, int64_t* launches, int32_t n) {
  if (!m || !ms || !launches) return fail(BLT_ERR_INVALID, "model_read_profile: null argument");
  if (n < BLT_NUM_STAGES) return fail(BLT_ERR_SHAPE, "model_read_profile: n < BLT_NUM_STAGES");
  return reinterpret_cast<Model*>(m)->read_profile(ms, launches, n);
}
const char* blt_stage_name(int32_t stage) {
  static const char* names[BLT_NUM_STAGES] = {
      "embed", "rmsnorm", "qkv_gemm_rope", "attention", "o_gemm_residual", "w13_gemm_silu",
      "w2_gemm_residual", "final_norm_l2", "head_gemm", "entropy", "coherence"};
  return (stage >= 0 && stage < BLT_NUM_STAGES) ? names[stage] : "";
}

// ---- synthetic inputs ------------------------------------------------------------
int blt_synth_normal_f32(uint64_t seed, float* out, int64_t n, double mean, double std) {
  if (n < 0) return fail(BLT_ERR_SHAPE, "synth: n >= 0");
  if (n > 0 && !out) return fail(BLT_ERR_INVALID, "synth: null output");
  parallel_for(n, [=](int64_t i) { out[i] = (float)(mean + std * normal_at(seed, (uint64_t)i)); });
  return BLT_OK;
}
int blt_synth_normal_bf16(uint64_t seed, uint16_t* out, int64_t n, double mean, double std) {
  if (n < 0) return fail(BLT_ERR_SHAPE, "synth: n >= 0");
  if (n > 0 && !out) return fail(BLT_ERR_INVALID, "synth: null output");
  parallel_for(n, [=](int64_t i) {
    out[i] = f32_to_bf16((float)(mean + std * normal_at(seed, (uint64_t)i)));
  });
  return BLT_OK;
}
int blt_synth_tokens(uint64_t seed, int32_t* out, int64_t n, double zipf_s, double p_uniform,
                     int32_t offset) {
  if (n < 0) return fail(BLT_ERR_SHAPE, "synth: n >= 0");
  if (n > 0 && !out) return fail(BLT_ERR_INVALID, "synth: null output");
  // rank -> byte: a seeded Fisher-Yates permutation of the printable bytes 0x20..0x7E
  int perm[95];
  for (int i = 0; i < 95; ++i) perm[i] = 0x20 + i;
  const uint64_t pseed = seed ^ 0x5EED5EED5EED5EEDull;
  for (int i = 94; i > 0; --i) {
    const int j = (int)(sm64_at(pseed, (uint64_t)i) % (uint64_t)(i + 1));
    const int t = perm[i]; perm[i] = perm[j]; perm[j] = t;
  }
  double cdf[95], acc = 0.0;
  for (int k = 0; k < 95; ++k) {
    acc += 1.0 / pow((double)(k + 1), zipf_s);
    cdf[k] = acc;
  }
  for (int k = 0; k < 95; ++k) cdf[k] /= acc;
  const int* pm = perm;
  const double* cd = cdf;
  parallel_for(n, [=](int64_t i) {
    const double ua = u01_at(seed, 2 * (uint64_t)i), ub = u01_at(seed, 2 * (uint64_t)i + 1);
    int byte;
    if (ua < p_uniform) {
      byte = (int)(ub * 256.0);
      if (byte > 255) byte = 255;
    } else {
      int lo = 0, hi = 94;  // first k with cdf[k] >= ub
      while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (cd[mid] >= ub) hi = mid; else lo = mid + 1;
      }
      byte = pm[lo];
    }
    out[i] = byte + offset;
  });
  return BLT_OK;
}

// ---- low-level GEMM -----------------------------------------------------------------
int blt_gemm_bf16(const uint16_t* A, const uint16_t* Bt, uint16_t* C, int64_t M, int64_t N,
                  int64_t K, blt_stream_t stream) {
  if (M < 0 || N < 0 || K <= 0 || K % 64 != 0 || N % 64 != 0)
    return fail(BLT_ERR_SHAPE, "gemm: need M >= 0, N % 64 == 0, K % 64 == 0, K > 0");
  if (M == 0 || N == 0) return BLT_OK;
  if (!A || !Bt || !C) return fail(BLT_ERR_INVALID, "gemm: null pointer");
  GemmArgs g{};
  g.A = A; g.Bt = Bt; g.C = C; g.M = M; g.N = N; g.K = K;
  g.lda = K; g.ldb = K; g.ldc = N; g.epi = EPI_BF16;
  return launch_gemm(g, STREAM(stream));
}

int blt_gemm_bf16_epilogue(const uint16_t* A, const uint16_t* Bt, void* C, int64_t M, int64_t N,
                           int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int32_t epilogue,
                           int32_t n_valid, int32_t rope_cols, int64_t seq_len,
                           const float* rope_cs, blt_stream_t stream) {
  if (epilogue < BLT_EPI_BF16 || epilogue > BLT_EPI_SILU_GATE)
    return fail(BLT_ERR_INVALID, "gemm_epilogue: bad epilogue");
  if (M < 0 || N <= 0 || K <= 0 || K % 64 != 0 || lda < K || ldb < K)
    return fail(BLT_ERR_SHAPE, "gemm_epilogue: need K % 64 == 0, lda, ldb >= K");
  if (epilogue != BLT_EPI_F32 && N % 64 != 0)
    return fail(BLT_ERR_SHAPE, "gemm_epilogue: N % 64 == 0 for this epilogue");
  const int64_t out_cols = epilogue == BLT_EPI_SILU_GATE ? N / 2
                           : epilogue == BLT_EPI_F32    ? n_valid
                                                        : N;
  if (epilogue == BLT_EPI_F32 && (n_valid <= 0 || n_valid > N))
    return fail(BLT_ERR_SHAPE, "gemm_epilogue: 0 < n_valid <= N");
  if (ldc < out_cols) return fail(BLT_ERR_SHAPE, "gemm_epilogue: ldc too small");
  if (epilogue == BLT_EPI_QKV_ROPE &&
      (rope_cols < 0 || rope_cols % 64 != 0 || rope_cols > N || seq_len <= 0 ||
       (rope_cols > 0 && rope_cs == nullptr)))
    return fail(BLT_ERR_SHAPE, "gemm_epilogue: rope needs rope_cols % 64 == 0, seq_len > 0, table");
  if (M == 0) return BLT_OK;
  if (!A || !Bt || !C) return fail(BLT_ERR_INVALID, "gemm_epilogue: null pointer");
  GemmArgs g{};
  g.A = A; g.Bt = Bt; g.C = C; g.M = M; g.N = N; g.K = K;
  g.lda = lda; g.ldb = ldb; g.ldc = ldc; g.epi = epilogue; g.n_valid = n_valid;
  g.rope_cols = rope_cols; g.seq_len = seq_len; g.rope_cs = rope_cs;
  return launch_gemm(g, STREAM(stream));
}

}  // extern "C"
