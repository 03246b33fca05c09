"""CPU oracle for the entropy-patching path (TEST INFRASTRUCTURE ONLY).

ctypes bindings to liboracle.so (oracle.c, a C restatement of blt-burn's
NdArray path).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this package, always as the checker.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


def build():
    """Compile liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboracle.so"], check=True)
    return LIB_PATH


class Cfg(ctypes.Structure):
    _fields_ = [("dim", _i32), ("n_layers", _i32), ("n_heads", _i32), ("hidden", _i32),
                ("vocab", _i32), ("max_seqlen", _i32), ("norm_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("window", _i32)]


class Weights(ctypes.Structure):
    _fields_ = [(n, _f32p) for n in
                ("emb", "attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "w1", "w2", "w3",
                 "norm", "out")]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_entropy.argtypes = [_f32p, _f32p, _i64, _i32]
        L.oracle_rms_norm.argtypes = [_f32p, _f32p, _f32p, _i64, _i32, ctypes.c_float, _i32]
        L.oracle_l2_norm.argtypes = [_f32p, _f32p, _i64, _i32]
        L.oracle_softmax.argtypes = [_f32p, _f32p, _i64, _i32]
        L.oracle_silu_gate.argtypes = [_f32p, _f32p, _f32p, _i64]
        L.oracle_coherence.argtypes = [_f32p, _f32p, _f32p, _i64, ctypes.c_float]
        L.oracle_patch_mask.argtypes = [_f32p, _i64, _i64, ctypes.c_float, _i32, _i32p]
        L.oracle_patch_indices.argtypes = [_i32p, _i64, _i64, _i32p, _i32p]
        L.oracle_patch_lengths.argtypes = [_i32p, _i32p, _i64, _i64, _i32p]
        L.oracle_rope_table.argtypes = [_f32p, _i32, _i32, ctypes.c_double]
        L.oracle_patch_means.argtypes = [_f32p, _f32p, _f32p, _i32p, _i32p, _i64, _i64, _f32p,
                                         _f32p, _f32p]
        L.oracle_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i32, _i32,
                                       _i32, ctypes.c_double]
        L.oracle_attention_kernel.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64,
                                              _i32, _i32]
        L.oracle_model_forward.argtypes = [ctypes.POINTER(Cfg), ctypes.POINTER(Weights), _i32p,
                                           _i64, _i64, _f32p, _f32p, _f32p, _f32p, _f32p]
        for f in ("oracle_entropy", "oracle_rms_norm", "oracle_l2_norm", "oracle_softmax",
                  "oracle_silu_gate", "oracle_coherence", "oracle_patch_mask",
                  "oracle_patch_indices", "oracle_patch_lengths", "oracle_patch_means",
                  "oracle_rope_table",
                  "oracle_attention", "oracle_attention_kernel", "oracle_model_forward"):
            getattr(L, f).restype = None
        _lib = L
    return _lib


def _f(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_f32p)


def _i(a):
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data_as(_i32p)


def entropy(logits):
    """[..., V] f32 -> [...] (patcher.rs:38-63)."""
    x, px = _f(logits)
    V = x.shape[-1]
    out = np.empty(x.shape[:-1], np.float32)
    lib().oracle_entropy(px, out.ctypes.data_as(_f32p), x.size // V if V else 0, V)
    return out


def rms_norm(x, w, eps, mode=0):
    x, px = _f(x)
    w, pw = _f(w)
    D = x.shape[-1]
    y = np.empty_like(x)
    lib().oracle_rms_norm(px, pw, y.ctypes.data_as(_f32p), x.size // D, D, eps, mode)
    return y


def l2_norm(x):
    x, px = _f(x)
    D = x.shape[-1]
    out = np.empty(x.shape[:-1], np.float32)
    lib().oracle_l2_norm(px, out.ctypes.data_as(_f32p), x.size // D, D)
    return out


def softmax(x):
    x, px = _f(x)
    N = x.shape[-1]
    y = np.empty_like(x)
    lib().oracle_softmax(px, y.ctypes.data_as(_f32p), x.size // N, N)
    return y


def silu_gate(g, u):
    g, pg = _f(g)
    u, pu = _f(u)
    out = np.empty_like(g)
    lib().oracle_silu_gate(pg, pu, out.ctypes.data_as(_f32p), g.size)
    return out


def coherence(n, H, eps):
    n, pn = _f(n)
    H, pH = _f(H)
    out = np.empty_like(n)
    lib().oracle_coherence(pn, pH, out.ctypes.data_as(_f32p), n.size, eps)
    return out


def patch_mask(H, thr, mode=0):
    """[B, T] f32 -> [B, T] int32 (patcher.rs:80-118; mode 1 = global H > thr)."""
    H, pH = _f(H)
    B, T = H.shape
    m = np.zeros((B, T), np.int32)
    lib().oracle_patch_mask(pH, B, T, thr, mode, m.ctypes.data_as(_i32p))
    return m


def patch_indices(mask):
    """[B, T] int32 -> list of per-row start lists (patcher.rs:124-142)."""
    mask, pm = _i(mask)
    B, T = mask.shape
    starts = np.zeros((B, T), np.int32)
    counts = np.zeros(B, np.int32)
    lib().oracle_patch_indices(pm, B, T, starts.ctypes.data_as(_i32p), counts.ctypes.data_as(_i32p))
    return [starts[b, :counts[b]].tolist() for b in range(B)]


def patch_lengths(starts, seq_len):
    """per-row start lists -> per-row length lists (patcher.rs:144-164)."""
    B = len(starts)
    T = max(seq_len, 1)
    st = np.zeros((B, T), np.int32)
    counts = np.array([len(s) for s in starts], np.int32)
    for b, s in enumerate(starts):
        st[b, :len(s)] = s
    ln = np.zeros((B, T), np.int32)
    lib().oracle_patch_lengths(st.ctypes.data_as(_i32p), counts.ctypes.data_as(_i32p), B, seq_len,
                               ln.ctypes.data_as(_i32p))
    return [ln[b, :counts[b]].tolist() for b in range(B)]


def patch_means(H, norms, starts, counts, coherence=None):
    """Per-patch means (pipeline.rs:240-258): H / norms / coherence [B, T] f32,
    starts [B, T] int32 (count[b] valid per row) -> (mean_H, mean_norm,
    mean_coherence or None), each [B, T] with count[b] valid entries per row."""
    H, pH = _f(H)
    N, pN = _f(norms)
    B, T = H.shape
    st, ps = _i(starts)
    ct, pc = _i(counts)
    mH = np.zeros((B, T), np.float32)
    mN = np.zeros((B, T), np.float32)
    if coherence is not None:
        C, pC = _f(coherence)
        mC = np.zeros((B, T), np.float32)
        pmC = mC.ctypes.data_as(_f32p)
    else:
        C, pC, mC, pmC = None, None, None, None
    lib().oracle_patch_means(pH, pN, pC, ps, pc, B, T, mH.ctypes.data_as(_f32p),
                             mN.ctypes.data_as(_f32p), pmC)
    return mH, mN, mC


def rope_table(head_dim, max_seqlen, theta):
    out = np.empty((max_seqlen, head_dim // 2, 2), np.float32)
    lib().oracle_rope_table(out.ctypes.data_as(_f32p), head_dim, max_seqlen, theta)
    return out


def attention(q, k, v, causal=True, window=0, rope_theta=0.0):
    """q, k, v f32 [B, H, T, d] -> o [B, H, T, d]."""
    q, pq = _f(q)
    k, pk = _f(k)
    v, pv = _f(v)
    B, H, T, d = q.shape
    o = np.empty_like(q)
    lib().oracle_attention(pq, pk, pv, o.ctypes.data_as(_f32p), B, H, T, d, int(causal),
                           window, rope_theta)
    return o


def attention_kernel(q, k, v, causal=True):
    """The reference's fused_attention_kernel: q f32 [B, H, Tq, d], k / v f32
    [B, H, Tkv, d] -> o [B, H, Tq, d] (causal: key j visible to query i iff j <= i)."""
    q, pq = _f(q)
    k, pk = _f(k)
    v, pv = _f(v)
    B, H, Tq, d = q.shape
    Tkv = k.shape[2]
    o = np.empty_like(q)
    lib().oracle_attention_kernel(pq, pk, pv, o.ctypes.data_as(_f32p), B, H, Tq, Tkv, d,
                                  int(causal))
    return o


WEIGHT_NAMES = ("emb", "attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "w1", "w2", "w3", "norm",
                "out")


def model_forward(cfg, weights, tokens):
    """cfg: dict(dim, n_layers, n_heads, hidden, vocab, max_seqlen, norm_eps, rope_theta, window);
    weights: dict of f32 arrays in the reference layouts (see oracle.c); tokens [B, T] int.
    Returns dict(logits, pre_norm_embeddings, embedding_norms, entropies, coherence_scores)."""
    tokens, pt = _i(tokens)
    B, T = tokens.shape
    c = Cfg(cfg["dim"], cfg["n_layers"], cfg["n_heads"], cfg["hidden"], cfg["vocab"],
            cfg["max_seqlen"], cfg["norm_eps"], cfg["rope_theta"], cfg.get("window", 0))
    keep = []
    ptrs = []
    for n in WEIGHT_NAMES:
        a, p = _f(weights[n])
        keep.append(a)
        ptrs.append(p)
    w = Weights(*ptrs)
    D, V = cfg["dim"], cfg["vocab"]
    out = {
        "logits": np.empty((B, T, V), np.float32),
        "pre_norm_embeddings": np.empty((B, T, D), np.float32),
        "embedding_norms": np.empty((B, T), np.float32),
        "entropies": np.empty((B, T), np.float32),
        "coherence_scores": np.empty((B, T), np.float32),
    }
    lib().oracle_model_forward(ctypes.byref(c), ctypes.byref(w), pt, B, T,
                               *[out[k].ctypes.data_as(_f32p) for k in
                                 ("logits", "pre_norm_embeddings", "embedding_norms",
                                  "entropies", "coherence_scores")])
    return out


def chunk_plan(total, chunk, overlap):
    """compute_all_signals_chunked's loop (blt_core.rs:286-356) as (start, end, skip)
    triples, stated exactly as the reference states it (saturating subtraction,
    skip = overlap for every later chunk)."""
    stride = chunk - overlap
    out = []
    pos = 0
    while pos < total:
        start = 0 if pos == 0 else max(pos - overlap, 0)
        end = min(pos + stride, total)
        skip = 0 if pos == 0 else overlap
        out.append((start, end, skip))
        pos = end
    return out


def signals_chunked(cfg, weights, tokens, chunk, overlap):
    """blt_core.rs:286-370 over one document: one B=1 forward per chunk, the
    kept outputs appended in order, then truncated / zero-padded to the
    document length.  Returns (entropies [n], embeddings [n, D], norms [n])."""
    tokens = np.asarray(tokens, dtype=np.int32)
    n = tokens.size
    D = cfg["dim"]
    H, E, N = [], [], []
    for start, end, skip in chunk_plan(n, chunk, overlap):
        o = model_forward(cfg, weights, tokens[None, start:end])
        for i in range(skip, end - start):
            if len(H) < n:
                H.append(o["entropies"][0, i])
                N.append(o["embedding_norms"][0, i])
                E.append(o["pre_norm_embeddings"][0, i])
    while len(H) < n:
        H.append(np.float32(0))
        N.append(np.float32(0))
        E.append(np.zeros(D, np.float32))
    return (np.array(H, np.float32), np.array(E, np.float32).reshape(n, D),
            np.array(N, np.float32))


def process_document(cfg, weights, tokens, chunk, overlap, threshold, mode=0):
    """process_bytes_with_embeddings after tokenization (blt_core.rs:178-207):
    dict(entropies, norms, embeddings, coherence, starts, lengths)."""
    H, E, N = signals_chunked(cfg, weights, tokens, chunk, overlap)
    if H.size == 0:
        z = np.zeros(0, np.int32)
        return dict(entropies=H, norms=N, embeddings=E, coherence=H.copy(), starts=z, lengths=z)
    m = patch_mask(H[None, :], threshold, mode)
    s = patch_indices(m)
    ln = patch_lengths(s, H.size)
    coh = (N * N) / (H + np.float32(1e-6))
    return dict(entropies=H, norms=N, embeddings=E, coherence=coh.astype(np.float32),
                starts=np.array(s[0], np.int32), lengths=np.array(ln[0], np.int32))


def mean_f32(x, start, end):
    """PipelineBuffer::compute_mean_prominence / compute_mean_entropy
    (pipeline.rs:241-258): end clamped to len(x), start to end, 0 for an empty
    span, else the left-to-right f32 sum over [start, end) divided by the
    length as f32."""
    end = min(end, len(x))
    start = min(start, end)
    if start >= end:
        return np.float32(0)
    s = np.add.accumulate(np.asarray(x[start:end], np.float32), dtype=np.float32)[-1]
    return np.float32(s / np.float32(end - start))


class PipelineBuffer:
    """PipelineBuffer (pipeline.rs:74-274) stated step by step; chunk_size /
    stride as in pipeline_process_document."""

    def __init__(self, threshold, chunk_size=4096, stride=2048):
        self.threshold = threshold
        self.stride = stride
        self.safe_zone_end = chunk_size - stride
        self.entropies = np.zeros(0, np.float32)
        self.norms = np.zeros(0, np.float32)
        self.raw = b""
        self.total_processed = 0
        self.chunk_idx = 0

    def process_chunk(self, chunk, forward, is_last):
        """pipeline.rs:111-238.  forward(tokens, start) -> (entropies, norms) of the
        model on this chunk, where start is the accumulated position of the
        chunk's first byte (its kept outputs land from position start +
        new_data_start on).  Returns [(start, length, prominence, entropy, bytes)]."""
        chunk = bytes(chunk)
        n = len(chunk)
        chunk_start_absolute = self.total_processed
        new_data_start = 0 if self.chunk_idx == 0 else self.stride
        h, nn = forward(np.frombuffer(chunk, np.uint8).astype(np.int32),
                        self.entropies.size - new_data_start)
        h = np.asarray(h, np.float32)
        nn = np.asarray(nn, np.float32)
        if self.chunk_idx == 0:
            self.entropies = np.concatenate([self.entropies, h])
            self.norms = np.concatenate([self.norms, nn])
            self.raw = self.raw + chunk
        elif new_data_start < n:
            self.entropies = np.concatenate([self.entropies, h[new_data_start:]])
            self.norms = np.concatenate([self.norms, nn[new_data_start:]])
            self.raw = self.raw + chunk[new_data_start:]
        acc = self.entropies.size
        starts = patch_indices(patch_mask(self.entropies[None, :], self.threshold, 0))[0] \
            if acc else []
        cutoff = None if is_last else chunk_start_absolute + self.safe_zone_end
        emit = []
        for i, s in enumerate(starts):
            if cutoff is None or s < cutoff:
                end = starts[i + 1] if i + 1 < len(starts) else acc
                if s >= max(self.total_processed - self.stride, 0) or self.chunk_idx == 0:
                    emit.append((s, end))
        out = []
        for s, end in emit:
            actual_end = min(end, len(self.raw))
            out.append((s, actual_end - s, mean_f32(self.norms, s, actual_end),
                        mean_f32(self.entropies, s, actual_end), self.raw[s:actual_end]))
        if not is_last:
            self.total_processed = chunk_start_absolute + max(n - self.stride, 0)
        else:
            self.total_processed = chunk_start_absolute + n
        self.chunk_idx += 1
        return out


def pipeline_process_document(data, forward, threshold, chunk_size=4096, stride=2048):
    """process_document (pipeline.rs:279-324) over PipelineBuffer.process_chunk.

    forward(tokens, start) -> (entropies, norms), f32 [n] each: the model on one
    chunk, whose tokens are the raw byte values (no +4 offset, pipeline.rs:123)
    and whose first byte is document position `start`.  chunk_size / stride are
    the reference's CHUNK_SIZE / STRIDE (4096 / 2048; SAFE_ZONE_END = chunk_size
    - stride); smaller values serve hand-worked cases.  Returns dict(patches=
    [(start, length, prominence, entropy, bytes)], entropies, norms)."""
    buf = PipelineBuffer(threshold, chunk_size, stride)
    data = bytes(data)
    patches = []
    total = len(data)
    position = 0
    while position < total:
        chunk_end = min(position + chunk_size, total)
        is_last = chunk_end >= total
        actual_start = max(position - stride, 0) if position > 0 else 0
        patches += buf.process_chunk(data[actual_start:chunk_end], forward, is_last)
        if is_last:
            break
        position = chunk_end
    return dict(patches=patches, entropies=buf.entropies, norms=buf.norms)
