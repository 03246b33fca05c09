"""Streaming ingest on the GPU: packed-segment forwards and the native ingest
driver (blt_ingest_run) against the CPU oracle's restatement of
compute_all_signals_chunked + the boundary pass (blt_core.rs:178-207,
286-370), and against separate GPU forwards of each chunk.

Tolerances: entropies 2e-2 abs and norms 1e-2 rel against the oracle (the
stated bound); against separate GPU forwards of the same chunks the only
difference is the attention kernel's key-tile alignment (online-softmax
order), so 5e-3 abs / rel there.  Boundaries, patch lengths and coherence are
bit-exact given the same entropies / norms."""
import numpy as np
import pytest
import torch

import oracle
from blt_burn_amd import BltError
from blt_burn_amd import ingest as I
from blt_burn_amd import model as M
from blt_burn_amd import synth

pytestmark = pytest.mark.gpu

TINY = dict(dim=128, n_layers=2, n_heads=2, ffn_dim_multiplier=2.0, multiple_of=64,
            max_seqlen=512, vocab_size=260)


def _oracle_cfg(cfg, hidden, window):
    return dict(dim=cfg.dim, n_layers=cfg.n_layers, n_heads=cfg.resolved_n_heads(),
                hidden=hidden, vocab=cfg.vocab_size, max_seqlen=cfg.max_seqlen,
                norm_eps=cfg.norm_eps, rope_theta=cfg.rope_theta, window=window)


def _oracle_weights(w):
    f = {k: synth.bf16_to_f32(v) for k, v in w.items()}
    return {"emb": f["tok_embeddings"], "attn_norm": f["attention_norm"],
            "ffn_norm": f["ffn_norm"], "wq": f["wq"], "wk": f["wk"], "wv": f["wv"],
            "wo": f["wo"], "w1": f["w1"], "w2": f["w2"], "w3": f["w3"], "norm": f["norm"],
            "out": f["output"]}


def _seg_start(rows_lens, T):
    seg = np.zeros((len(rows_lens), T), np.int32)
    for b, lens in enumerate(rows_lens):
        assert sum(lens) == T
        p = 0
        for n in lens:
            seg[b, p:p + n] = p
            p += n
    return seg


def _check_segments(m, tok, rows_lens, tol):
    B, T = tok.shape
    seg = _seg_start(rows_lens, T)
    packed = m.forward_with_embeddings(torch.from_numpy(tok).cuda(),
                                       seg_start=torch.from_numpy(seg).cuda())
    H = packed.entropies.cpu().numpy()
    N = packed.embedding_norms.cpu().numpy()
    worst = [0.0, 0.0]
    for b, lens in enumerate(rows_lens):
        p = 0
        for n in lens:
            one = m.forward_with_embeddings(torch.from_numpy(tok[b:b + 1, p:p + n].copy()).cuda())
            h1 = one.entropies.cpu().numpy()[0]
            n1 = one.embedding_norms.cpu().numpy()[0]
            worst[0] = max(worst[0], np.abs(H[b, p:p + n] - h1).max())
            worst[1] = max(worst[1], (np.abs(N[b, p:p + n] - n1) / n1).max())
            p += n
    print("segments vs separate: entropy max|d|=%.2e norms max rel=%.2e" % tuple(worst))
    assert worst[0] < tol and worst[1] < tol, worst


@pytest.mark.parametrize("window", [0, 24])
def test_segments_match_separate_forwards_tiny(window):
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 21, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=2 * 256, window=window)
    tok = synth.tokens(synth.config_seed(5) + 1, (2, 256))
    _check_segments(m, tok, [[40, 100, 1, 115], [256]], 5e-3)


@pytest.mark.parametrize("window,B", [(512, 1), (0, 3)])
def test_segments_match_separate_forwards_entropy_model(window, B):
    # real dims and T = 8192; window 0 with B = 3 takes the 64-query-wave
    # attention path, window 512 the 32-query one
    cfg = M.entropy_model_config()
    cfg.n_layers = 2
    w = M.random_weights(cfg, 22, hidden=2048)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=B * 8192, window=window)
    tok = synth.tokens(synth.config_seed(5) + 2, (B, 8192))
    rows = [[3000, 64, 63, 5065], [8192], [1, 4095, 4096]][:B]
    _check_segments(m, tok, rows, 5e-3)


def _docs(seed, lens):
    toks = synth.tokens(seed, (max(1, sum(lens)),))[: sum(lens)]
    off = np.zeros(len(lens) + 1, np.int64)
    off[1:] = np.cumsum(lens)
    return toks.astype(np.int32), off


def _check_doc_outputs(res, d, ref_H, ref_N, tolH, tolN, thr, mode):
    H, N, C, S, Ln = res.doc(d)[:5]
    assert H.size == ref_H.size
    if H.size == 0:
        assert res.counts[d] == 0
        return 0.0, 0.0
    dH = np.abs(H - ref_H).max()
    dN = (np.abs(N - ref_N) / np.maximum(ref_N, 1e-30)).max()
    assert dH < tolH and dN < tolN, (d, dH, dN)
    # coherence exactly as blt_core.rs:202-207 on these norms / entropies
    np.testing.assert_array_equal(C, (N * N) / (H + np.float32(1e-6)))
    # boundaries bit-exact on the same entropies (patcher.rs:80-164)
    m = oracle.patch_mask(H[None, :], thr, mode)
    s = oracle.patch_indices(m)
    np.testing.assert_array_equal(S, np.array(s[0], np.int32))
    np.testing.assert_array_equal(Ln, np.array(oracle.patch_lengths(s, H.size)[0], np.int32))
    assert int(Ln.sum()) == H.size
    return dH, dN


@pytest.mark.parametrize("window", [0, 24])
def test_ingest_vs_oracle_tiny(window):
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 23, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=4 * 128, window=window)
    conf = I.BltConfig(threshold=0.35, max_seq_len=64, chunk_overlap=16)
    ing = I.StreamingIngest(m, conf, rows=4, row_len=128, with_embeddings=True)
    lens = [0, 1, 2, 37, 64, 65, 150, 300, 5, 0, 128, 49]
    toks, off = _docs(synth.config_seed(5) + 3, lens)
    res = ing.run(toks, off)
    oc, ow = _oracle_cfg(cfg, 256, window), _oracle_weights(w)
    worst = [0.0, 0.0]
    for d in range(len(lens)):
        ref = oracle.process_document(oc, ow, toks[off[d]:off[d + 1]], 64, 16, 0.35)
        dH, dN = _check_doc_outputs(res, d, ref["entropies"], ref["norms"], 2e-2, 1e-2, 0.35, 0)
        worst = [max(worst[0], dH), max(worst[1], dN)]
        if lens[d]:
            E = res.embeddings[off[d]:off[d + 1]]
            rel = np.abs(E - ref["embeddings"]).max() / np.abs(ref["embeddings"]).max()
            assert rel < 1e-2, (d, rel)
    print("ingest vs oracle: entropy max|d|=%.2e norms max rel=%.2e" % tuple(worst))
    assert res.counts[0] == 0 and res.counts[9] == 0


def _direct_chunks(m, toks, chunk, overlap):
    """The reference loop with the GPU model: one forward per chunk."""
    H = np.zeros(toks.size, np.float32)
    N = np.zeros(toks.size, np.float32)
    for s, n, k in I.plan_chunks(toks.size, chunk, overlap):
        o = m.forward_with_embeddings(torch.from_numpy(toks[None, s:s + n].copy()).cuda())
        H[s + k:s + n] = o.entropies.cpu().numpy()[0, k:]
        N[s + k:s + n] = o.embedding_norms.cpu().numpy()[0, k:]
    return H, N


def test_ingest_config5_sample_entropy_model():
    # config-5 shape at real dims: 8192-token rows, 512 overlap, log-normal
    # documents (a 160 KiB sample of the 1 GiB stream), full 14 layers
    cfg = M.entropy_model_config()
    w = M.random_weights(cfg, 24, hidden=2048)
    # a 16384-token document is chunks of 7680, 8192 and 1536 tokens: 3 rows
    m = M.LMTransformer(cfg, w, device=0, max_tokens=3 * 8192, window=512)
    conf = I.BltConfig(threshold=1.335, max_seq_len=8192, chunk_overlap=512)
    ing = I.StreamingIngest(m, conf, rows=3, row_len=8192)
    data, off = synth.documents(synth.config_seed(5), 160 * 1024, max_len=16384)
    toks = data.astype(np.int32) + 4
    res = ing.run(toks, off)
    st = ing.last_stats()
    lens = np.diff(off)
    assert st["documents"] == int((lens > 0).sum()) and st["tokens"] == int(lens.sum())
    assert st["tokens_computed"] == sum(n for L in lens for _, n, _ in I.plan_chunks(int(L), 8192,
                                                                                       512))
    assert st["row_tokens"] == st["batches"] * 3 * 8192 >= st["tokens_computed"]
    worst = [0.0, 0.0]
    for d in range(off.size - 1):
        H, N = _direct_chunks(m, toks[off[d]:off[d + 1]], 8192, 512)
        dH, dN = _check_doc_outputs(res, d, H, N, 5e-3, 5e-3, 1.335, 0)
        worst = [max(worst[0], dH), max(worst[1], dN)]
    print("ingest vs per-chunk forwards (%d docs): entropy max|d|=%.2e norms max rel=%.2e"
          % (off.size - 1, worst[0], worst[1]))


def test_ingest_config5_vs_oracle_entropy_model():
    """Config 5 at real dims (14 x 768, FFN 2048, window 512, chunks of 8192
    with 512 overlap) against the oracle's restatement of
    compute_all_signals_chunked + the boundary pass (blt_core.rs:178-207,
    286-370): a document of 8704 tokens (chunks of 7680 and 1536 tokens, the
    second starting 512 early) and the first documents of the seeded config-5
    stream, packed together into 8192-token rows."""
    cfg = M.entropy_model_config()
    w = M.random_weights(cfg, 27, hidden=2048)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=2 * 8192, window=512)
    conf = I.BltConfig(threshold=1.335, max_seq_len=8192, chunk_overlap=512)
    ing = I.StreamingIngest(m, conf, rows=2, row_len=8192, with_embeddings=True)
    data, off = synth.documents(synth.config_seed(5), 24 * 1024)
    stream_lens = [int(x) for x in np.diff(off)[:4]]
    long_doc = synth.tokens(synth.config_seed(5) + 7, (8704,))
    toks = np.concatenate([long_doc, data[:sum(stream_lens)].astype(np.int32) + 4])
    lens = [8704] + stream_lens
    offs = np.zeros(len(lens) + 1, np.int64)
    offs[1:] = np.cumsum(lens)
    assert [c[1] for c in I.plan_chunks(8704, 8192, 512)] == [7680, 1536]
    res = ing.run(toks.astype(np.int32), offs)
    oc, ow = _oracle_cfg(cfg, 2048, 512), _oracle_weights(w)
    worst = [0.0, 0.0, 0.0]
    for d in range(len(lens)):
        ref = oracle.process_document(oc, ow, toks[offs[d]:offs[d + 1]], 8192, 512, 1.335)
        dH, dN = _check_doc_outputs(res, d, ref["entropies"], ref["norms"], 2e-2, 1e-2, 1.335, 0)
        E = res.embeddings[offs[d]:offs[d + 1]]
        rel = np.abs(E - ref["embeddings"]).max() / np.abs(ref["embeddings"]).max()
        assert rel < 1e-2, (d, rel)
        worst = [max(worst[0], dH), max(worst[1], dN), max(worst[2], rel)]
    print("config-5 ingest vs oracle (%s): entropy max|d|=%.2e norms max rel=%.2e "
          "embeddings max rel=%.2e" % (lens, *worst))


def test_process_bytes_mirror():
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 25, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=512, window=0)
    conf = I.BltConfig(max_seq_len=64, chunk_overlap=16, add_bos=True, add_eos=True)
    data = "héllo, wörld \xff".encode("latin-1", errors="replace") + b"\xf0\x90 tail" * 9
    ex = I.process_bytes_with_embeddings(data, "doc-1", m, conf)
    toks = ex.core.tokens
    assert toks[0] == 1 and toks[-1] == 2
    assert ex.core.sample_id == "doc-1" and ex.core.mask.all() and ex.core.mask.size == toks.size
    assert ex.pre_norm_embeddings.size == toks.size * cfg.dim and ex.embedding_dim == cfg.dim
    assert int(ex.core.patch_lengths.sum()) == toks.size
    ref = oracle.process_document(_oracle_cfg(cfg, 256, 0), _oracle_weights(w), toks, 64, 16,
                                  1.335)
    assert np.abs(ex.core.entropies - ref["entropies"]).max() < 2e-2
    core = I.process_bytes(data, "doc-1", m, conf)
    np.testing.assert_array_equal(core.tokens, toks)
    assert np.abs(core.entropies - ex.core.entropies).max() < 1e-6
    empty = I.process_bytes(b"", "e", m, I.BltConfig(max_seq_len=64, chunk_overlap=16))
    assert empty.tokens.size == 0 and empty.patch_lengths.size == 0


def test_ingest_rejects_bad_shapes():
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 26, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=256, window=0)
    with pytest.raises(BltError):
        I.StreamingIngest(m, I.BltConfig(max_seq_len=64, chunk_overlap=40), rows=2, row_len=128)
    with pytest.raises(BltError):  # rows * row_len above the model's max_tokens
        I.StreamingIngest(m, I.BltConfig(max_seq_len=64, chunk_overlap=16), rows=4, row_len=128)
    ing = I.StreamingIngest(m, I.BltConfig(max_seq_len=64, chunk_overlap=16), rows=2, row_len=64)
    with pytest.raises(BltError):  # offsets that do not end at len(tokens)
        ing.run(np.zeros(10, np.int32) + 70, np.array([0, 5, 9], np.int64))
    res = ing.run(*_docs(8, [10, 20]))  # the handle still works after the error
    assert res.counts.size == 2 and int(res.lengths[:res.counts[0]].sum()) == 10


_LONG_RUNS = {}


@pytest.mark.parametrize("arena", [0, -1, 1100])
def test_ingest_long_documents_vs_oracle_tiny(arena):
    """Documents whose chunks need more rows than one batch has (the reference
    loops over any number of chunks, blt_core.rs:300-356): they span several
    batches and get their boundary pass and patch means once complete; short
    documents share the batches with them.  arena 0: every such document is
    stitched on the device; -1: none is (host gather); 1100 tokens: the
    1000-token document is, the 2049-token one cannot be.  All three give the
    same outputs bit for bit."""
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 31, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=2 * 128, window=0)
    conf = I.BltConfig(threshold=0.3, max_seq_len=64, chunk_overlap=16)
    ing = I.StreamingIngest(m, conf, rows=2, row_len=128, with_embeddings=True,
                            long_arena_tokens=arena)
    lens = [1000, 5, 0, 257, 400, 64, 2049, 3]
    toks, off = _docs(synth.config_seed(5) + 12, lens)
    res = ing.run(toks, off, patch_means=True)
    st = ing.last_stats()
    assert st["batches"] > 1 and st["tokens"] == sum(lens)
    assert st["long_documents"] == 4  # 1000, 257, 400 and 2049 tokens
    host = st["long_documents_host"]
    if arena == 0:
        assert host == 0
    elif arena < 0:
        assert host == 4
    else:
        assert 1 <= host <= 3
    _LONG_RUNS[arena] = res
    if len(_LONG_RUNS) > 1:
        first = next(iter(_LONG_RUNS.values()))
        for n in ("entropies", "norms", "coherence", "starts", "lengths", "counts",
                  "patch_entropy", "patch_prominence", "patch_coherence"):
            a, b = getattr(first, n), getattr(res, n)
            if n in ("starts", "lengths", "patch_entropy", "patch_prominence",
                     "patch_coherence"):  # only the written entries are outputs
                for d in range(len(lens)):
                    o, c = int(res.offsets[d]), int(res.counts[d])
                    assert np.array_equal(a[o:o + c], b[o:o + c]), (n, d)
            else:
                assert np.array_equal(a, b), n
    oc, ow = _oracle_cfg(cfg, 256, 0), _oracle_weights(w)
    for d, L in enumerate(lens):
        ref = oracle.process_document(oc, ow, toks[off[d]:off[d + 1]], 64, 16, 0.3)
        _check_doc_outputs(res, d, ref["entropies"], ref["norms"], 2e-2, 1e-2, 0.3, 0)
        if L == 0:
            continue
        E = res.embeddings[off[d]:off[d + 1]]
        assert np.abs(E - ref["embeddings"]).max() < 1e-2 * np.abs(ref["embeddings"]).max()
        H, N, C, S, Lp = res.doc(d)[:5]
        n = S.size
        st0 = np.zeros((1, L), np.int32)
        st0[0, :n] = S
        rH, rN, rC = oracle.patch_means(H[None], N[None], st0, np.array([n], np.int32), C[None])
        starts, lengths, pH, pN, pC = res.patches(d)
        assert np.array_equal(pH, rH[0, :n]) and np.array_equal(pN, rN[0, :n])
        assert np.array_equal(pC, rC[0, :n])
    # the same documents one by one give the same results
    for d in (0, 6):
        one = ing.run(toks[off[d]:off[d + 1]], np.array([0, lens[d]], np.int64))
        assert np.array_equal(one.entropies, res.doc(d)[0])
        assert np.array_equal(one.starts[:one.counts[0]], res.doc(d)[3])


def test_ingest_long_document_entropy_model():
    # real dims, one 8192-token row per batch: a 20000-token document is
    # chunks of 7680, 8192 and 5152 tokens in three batches
    cfg = M.entropy_model_config()
    cfg.n_layers = 2
    w = M.random_weights(cfg, 32, hidden=2048)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=8192, window=512)
    conf = I.BltConfig(threshold=1.335, max_seq_len=8192, chunk_overlap=512)
    ing = I.StreamingIngest(m, conf, rows=1, row_len=8192)
    toks, off = _docs(synth.config_seed(5) + 13, [20000, 300])
    assert [c[1] for c in I.plan_chunks(20000, 8192, 512)] == [7680, 8192, 5152]
    res = ing.run(toks, off)
    assert ing.last_stats()["batches"] == 3
    for d in range(2):
        H, N = _direct_chunks(m, toks[off[d]:off[d + 1]], 8192, 512)
        _check_doc_outputs(res, d, H, N, 5e-3, 5e-3, 1.335, 0)


def test_process_bytes_long_document_reuses_ingest():
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 33, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=256, window=0)
    conf = I.BltConfig(max_seq_len=64, chunk_overlap=16)
    data = (synth.tokens(synth.config_seed(5) + 14, (3000,)) - 4).astype(np.uint8).tobytes()
    ex = I.process_bytes_with_embeddings(data, "long", m, conf)
    toks = ex.core.tokens
    assert toks.size > 256 and int(ex.core.patch_lengths.sum()) == toks.size
    ref = oracle.process_document(_oracle_cfg(cfg, 256, 0), _oracle_weights(w), toks, 64, 16,
                                  conf.threshold)
    assert np.abs(ex.core.entropies - ref["entropies"]).max() < 2e-2
    np.testing.assert_array_equal(ex.patch_indices, oracle.patch_indices(
        oracle.patch_mask(ex.core.entropies[None], conf.threshold, 0))[0])
    ing = I.ingest_for(m, conf, with_embeddings=True)
    assert I.ingest_for(m, conf, with_embeddings=True) is ing
    ex2 = I.process_bytes_with_embeddings(data, "long", m, conf)
    assert np.array_equal(ex2.core.entropies, ex.core.entropies)


def test_ingest_patch_means_bit_exact():
    """Per-patch means of every document (PatchData.entropy / .prominence,
    pipeline.rs:240-258) from the ingest driver equal the oracle's restatement
    applied to that document's own stitched entropies, norms and starts."""
    cfg = M.LMTransformerConfig(**TINY)
    w = M.random_weights(cfg, 29, hidden=256)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=4 * 128, window=0)
    conf = I.BltConfig(threshold=0.3, max_seq_len=64, chunk_overlap=16)
    ing = I.StreamingIngest(m, conf, rows=4, row_len=128)
    lens = [0, 1, 3, 40, 64, 65, 200, 7, 0, 128]
    toks, off = _docs(synth.config_seed(5) + 11, lens)
    res = ing.run(toks, off, patch_means=True)
    plain = ing.run(toks, off)
    assert np.array_equal(plain.starts, res.starts) and np.array_equal(plain.entropies,
                                                                        res.entropies)
    for d, L in enumerate(lens):
        H, N, C, S, Lp = res.doc(d)
        starts, lengths, pH, pN, pC = res.patches(d)
        assert np.array_equal(starts, S) and int(Lp.sum()) == L
        if L == 0:
            assert pH.size == 0
            continue
        n = S.size
        st = np.zeros((1, L), np.int32)
        st[0, :n] = S
        rH, rN, rC = oracle.patch_means(H[None], N[None], st, np.array([n], np.int32), C[None])
        assert np.array_equal(pH, rH[0, :n]) and np.array_equal(pN, rN[0, :n])
        assert np.array_equal(pC, rC[0, :n])
    with pytest.raises(BltError):
        plain.patches(3)
