"""The streaming pipeline on the GPU (blt_pipeline_*, pipeline.rs:74-324).

Three checks per document:
  - against the oracle's restatement of process_document with the oracle's
    model on every chunk: entropies 2e-2 abs, norms 1e-2 rel (the stated
    bound for the bf16 forward);
  - the emitted patches exactly (starts, lengths, bytes, and the f32 means
    bit for bit) against the oracle's chunk loop replayed on the GPU's own
    accumulated entropies / norms: the boundary pass, the confirmation
    windows, the clipped ends and the left-to-right means are the
    reference's;
  - the many-document form (packed segments) against the one-chunk-per-forward
    form: entropies and norms 5e-3 (the forward's online-softmax order differs
    between packed and separate runs), patches exactly on its own entropies.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from blt_burn_amd import BltError
from blt_burn_amd import model as M
from blt_burn_amd import pipeline as P
from blt_burn_amd import synth
from blt_burn_amd._lib import lib

pytestmark = pytest.mark.gpu

TINY = dict(dim=128, n_layers=2, n_heads=2, ffn_dim_multiplier=2.0, multiple_of=64,
            max_seqlen=8192, vocab_size=260)
THR = 1.335


def _oracle_model(cfg, w, hidden, window):
    f = {k: synth.bf16_to_f32(v) for k, v in w.items()}
    ow = {"emb": f["tok_embeddings"], "attn_norm": f["attention_norm"],
          "ffn_norm": f["ffn_norm"], "wq": f["wq"], "wk": f["wk"], "wv": f["wv"],
          "wo": f["wo"], "w1": f["w1"], "w2": f["w2"], "w3": f["w3"], "norm": f["norm"],
          "out": f["output"]}
    oc = dict(dim=cfg.dim, n_layers=cfg.n_layers, n_heads=cfg.resolved_n_heads(), hidden=hidden,
              vocab=cfg.vocab_size, max_seqlen=cfg.max_seqlen, norm_eps=cfg.norm_eps,
              rope_theta=cfg.rope_theta, window=window)

    def fwd(tokens, start):
        o = oracle.model_forward(oc, ow, tokens[None, :])
        return o["entropies"][0], o["embedding_norms"][0]
    return fwd


def _replay(H, N):
    """The model's outputs for a chunk, taken from accumulated signals: the
    chunk loop keeps exactly the positions it appends, so positions it drops
    (the overlap context) may come from anywhere."""
    def fwd(tokens, start):
        return H[start:start + tokens.size], N[start:start + tokens.size]
    return fwd


def _docs(seed):
    lens = [1, 2, 3, 100, 2048, 4096, 4097, 8193, 12289]
    docs = [synth.documents(seed + i, n)[0].tobytes() for i, n in enumerate(lens)]
    # long runs of one byte: few patch starts, patches longer than a chunk
    docs.append(b"a" * 9000 + bytes(range(256)) + b"b" * 3000)
    return docs


def _assert_patches_exact(got, want, data):
    assert len(got) == len(want), (len(got), len(want))
    for g, (s, n, p, h, b) in zip(got, want):
        assert (g.start_offset, g.length) == (s, n)
        assert g.bytes == b == data[s:s + n]
        assert np.float32(g.prominence) == p and np.float32(g.entropy) == h, (g, p, h)
        assert g.embedding.shape == (768,) and not g.embedding.any()


def _check_doc(res, data, ref_fwd=None, tolH=2e-2, tolN=1e-2):
    H, N = res.entropies, res.norms
    assert H.size == N.size == len(data)
    worst = (0.0, 0.0)
    if ref_fwd is not None and len(data):
        ref = oracle.pipeline_process_document(data, ref_fwd, THR)
        dH = float(np.abs(H - ref["entropies"]).max())
        dN = float((np.abs(N - ref["norms"]) / ref["norms"]).max())
        assert dH < tolH and dN < tolN, (len(data), dH, dN)
        worst = (dH, dN)
    rep = oracle.pipeline_process_document(data, _replay(H, N), THR)
    _assert_patches_exact(res.patches, rep["patches"], data)
    np.testing.assert_array_equal(rep["entropies"], H)
    return worst


@pytest.mark.parametrize("window", [0, 512])
def test_pipeline_vs_oracle_tiny(window):
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 41, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=2 * 8192, window=window)
    fwd = _oracle_model(cfg, w, 256, window)
    docs = _docs(900 + window)
    if window == 0:
        docs = docs[:7] + docs[-1:]  # the oracle's unwindowed attention is slow
    worst = [0.0, 0.0]
    for data in docs:
        res = P.process_document(data, m, threshold=THR)
        dH, dN = _check_doc(res, data, fwd)
        worst = [max(worst[0], dH), max(worst[1], dN)]
    print("pipeline vs oracle (window %d): entropy max|d|=%.2e norms max rel=%.2e"
          % (window, *worst))
    batched = P.process_documents(docs, m, threshold=THR, rows=2, row_len=8192)
    for data, res, b in zip(docs, [P.process_document(d, m, threshold=THR) for d in docs],
                            batched):
        _check_doc(b, data)
        if len(data):
            assert np.abs(b.entropies - res.entropies).max() < 5e-3
            assert (np.abs(b.norms - res.norms) / res.norms).max() < 5e-3


def test_pipeline_buffer_api_tiny():
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 42, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=8192, window=0)
    data = synth.documents(977, 9000)[0].tobytes()
    buf = P.PipelineBuffer(THR)
    p0 = buf.process_chunk(data[0:4096], m, None, None, False)
    assert buf.accumulated() == 4096 and buf.raw_bytes() == data[:4096]
    assert all(p.start_offset < P.SAFE_ZONE_END for p in p0)
    p1 = buf.process_chunk(data[2048:8192], m, None, None, False)
    assert buf.accumulated() == 8192 and buf.raw_bytes() == data[:8192]
    # chunk 1 confirms again what chunk 0 did (its window starts at 0)
    assert [p.start_offset for p in p1][:len(p0)] == [p.start_offset for p in p0]
    p2 = buf.process_chunk(data[6144:9000], m, None, None, True)
    assert buf.accumulated() == 9000 and buf.raw_bytes() == data
    res = P.process_document(data, m, threshold=THR)
    np.testing.assert_array_equal(buf.entropies(), res.entropies)
    np.testing.assert_array_equal(buf.norms(), res.norms)
    got = [(p.start_offset, p.length, p.prominence, p.entropy) for p in p0 + p1 + p2]
    assert got == [(p.start_offset, p.length, p.prominence, p.entropy) for p in res.patches]
    # another model on the same buffer is refused
    m2 = M.LMTransformer(cfg, w, device=0, max_tokens=8192, window=0)
    with pytest.raises(BltError):
        buf.process_chunk(b"xyz", m2)


def test_pipeline_errors_leave_state():
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 43, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=8192, window=0)
    buf = P.PipelineBuffer(THR)
    buf.process_chunk(bytes(range(200)), m, is_last_chunk=False)
    n0 = buf.accumulated()
    h = buf._h
    start = np.zeros(8, np.int64)
    cnt = ctypes.c_int64()
    chunk = np.frombuffer(bytes(300), np.uint8)
    # cap below what the chunk can confirm: refused before any work
    rc = lib().blt_pipeline_process_chunk(h, chunk.ctypes.data, chunk.size, 1, 1,
                                          start.ctypes.data, None, None, None,
                                          ctypes.byref(cnt), None)
    assert rc != 0 and buf.accumulated() == n0
    # a chunk longer than the model's max_seqlen / max_tokens
    with pytest.raises(BltError):
        buf.process_chunk(bytes(8193), m)
    assert buf.accumulated() == n0
    with pytest.raises(BltError):  # outside the accumulated range
        buf._read(0, n0 + 1)
    with pytest.raises(BltError):  # row_len below CHUNK_SIZE + STRIDE
        P.process_documents([b"abc"], m, rows=1, row_len=4096)
    empty = P.process_document(b"", m)
    assert empty.patches == [] and empty.entropies.size == 0
    assert [r.patches for r in P.process_documents([b"", b""], m, rows=1, row_len=8192)] \
        == [[], []]


def test_pipeline_entropy_model():
    """Real dims (14 x 768, FFN 2048, window 512): one-chunk-per-forward and
    packed forms against each other and, exactly, against the chunk loop on
    their own entropies; a short document also against the oracle."""
    cfg = M.entropy_model_config()
    w = M.random_weights(cfg, 44, hidden=2048)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=2 * 8192, window=512)
    data, off = synth.documents(synth.config_seed(5) + 11, 96 * 1024, max_len=24000)
    docs = [data[off[d]:off[d + 1]].tobytes() for d in range(off.size - 1)]
    docs.append(b"z" * 10000)
    batched = P.process_documents(docs, m, threshold=THR, rows=2, row_len=8192)
    worst = 0.0
    for data_d, b in zip(docs, batched):
        res = P.process_document(data_d, m, threshold=THR)
        _check_doc(res, data_d)
        _check_doc(b, data_d)
        if len(data_d):
            worst = max(worst, float(np.abs(b.entropies - res.entropies).max()))
            assert (np.abs(b.norms - res.norms) / res.norms).max() < 5e-3
    assert worst < 5e-3, worst
    fwd = _oracle_model(cfg, w, 2048, 512)
    short = [d for d in docs if 0 < len(d) <= 1500][:1]
    for data_d in short:
        _check_doc(P.process_document(data_d, m, threshold=THR), data_d, fwd)
    print("pipeline at real dims: %d documents (%d bytes), packed vs separate entropy "
          "max|d|=%.2e" % (len(docs), sum(map(len, docs)), worst))
    torch.cuda.synchronize()


def _replay_at(H, N):
    """Model outputs for a chunk whose first byte sits at accumulated position
    `start` (negative for the dropped context of an odd call sequence): the
    accumulated values where they exist, zeros elsewhere (never kept)."""
    def fwd(tokens, start):
        n = tokens.size
        h = np.zeros(n, np.float32)
        m = np.zeros(n, np.float32)
        lo, hi = max(start, 0), min(start + n, H.size)
        if hi > lo:
            h[lo - start:hi - start] = H[lo:hi]
            m[lo - start:hi - start] = N[lo:hi]
        return h, m
    return fwd


@pytest.mark.parametrize("calls", [
    [(3000, False), (100, False), (5000, False), (0, False), (2049, False), (700, True)],
    [(0, False), (10, False), (4096, True)],
    [(4000, True), (3000, False), (2500, True)],
    [(1, False), (2, False), (2048, False), (2050, False), (6144, False), (9, True)],
])
def test_pipeline_direct_chunk_calls_tiny(calls):
    """process_chunk called directly with chunks of any size (shorter than the
    context, empty, calls after a last chunk): every call's patches equal the
    oracle's PipelineBuffer on the same accumulated signals, bit for bit."""
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 45, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=8192, window=0)
    rng = np.random.default_rng(len(calls))
    chunks = [synth.documents(int(rng.integers(1 << 30)), n)[0].tobytes() if n else b""
              for n, _ in calls]
    buf = P.PipelineBuffer(THR)
    got = [buf.process_chunk(c, m, None, None, last) for c, (_, last) in zip(chunks, calls)]
    H, N = buf.entropies(), buf.norms()
    ref = oracle.PipelineBuffer(THR)
    fwd = _replay_at(H, N)
    raw = buf.raw_bytes()
    for c, (_, last), g in zip(chunks, calls, got):
        want = ref.process_chunk(c, fwd, last)
        _assert_patches_exact(g, want, raw)
    np.testing.assert_array_equal(ref.entropies, H)
    assert ref.raw == raw
