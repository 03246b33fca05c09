"""Drop-in pieces of the reference API beyond forward_with_embeddings:
LMTransformer::extract_embeddings (model.rs:325-345, 413-431),
patch_start_indices_cpu / patch_lengths_from_start_indices from a device mask
(patcher.rs:124-164), boundary passes on concurrent streams, and the lifetime
of the pipeline buffers cached on a model.  All through the C ABI."""
import gc
import weakref

import numpy as np
import pytest
import torch

import oracle
from blt_burn_amd import model as M
from blt_burn_amd import patcher, pipeline, synth

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _oracle_weights(w):
    f = {k: synth.bf16_to_f32(v) for k, v in w.items()}
    return {"emb": f["tok_embeddings"], "attn_norm": f["attention_norm"],
            "ffn_norm": f["ffn_norm"], "wq": f["wq"], "wk": f["wk"], "wv": f["wv"],
            "wo": f["wo"], "w1": f["w1"], "w2": f["w2"], "w3": f["w3"], "norm": f["norm"],
            "out": f["output"]}


def test_extract_embeddings_matches_oracle_and_skips_head():
    # real dimensions, window 512: the residual after the last layer equals the
    # oracle's pre_norm_embeddings (1e-2 of max, as forward_with_embeddings),
    # is bit-identical to the full forward's field, and no final norm, head,
    # entropy or coherence kernel is launched for it
    cfg = M.entropy_model_config()
    w = M.random_weights(cfg, 21, hidden=2048)
    B, T = 2, 600
    tok = synth.tokens(synth.config_seed(4) + 21, (B, T))
    m = M.LMTransformer(cfg, w, device=0, max_tokens=B * T, window=512)
    tk = torch.from_numpy(tok).to(DEV)
    full = m.forward_with_embeddings(tk)
    m.set_profiling(True)
    m.read_profile()  # start from zero
    emb = m.extract_embeddings(tk)
    prof = m.read_profile()
    m.set_profiling(False)
    assert tuple(emb.shape) == (B, T, 768) and emb.dtype == torch.float32
    assert torch.equal(emb, full.pre_norm_embeddings)
    for stage in ("final_norm_l2", "head_gemm", "entropy", "coherence"):
        assert prof[stage][1] == 0, (stage, prof[stage])
    for stage in ("embed", "qkv_gemm_rope", "attention", "o_gemm_residual", "w13_gemm_silu",
                  "w2_gemm_residual"):
        assert prof[stage][1] > 0, (stage, prof[stage])
    ref = oracle.model_forward(dict(dim=768, n_layers=14, n_heads=12, hidden=2048, vocab=260,
                                    max_seqlen=cfg.max_seqlen, norm_eps=cfg.norm_eps,
                                    rope_theta=cfg.rope_theta, window=512),
                               _oracle_weights(w), tok)
    pre = ref["pre_norm_embeddings"]
    d = np.abs(emb.cpu().numpy() - pre).max() / np.abs(pre).max()
    print("extract_embeddings vs oracle: max rel %.2e" % d)
    assert d < 1e-2, d
    # a preallocated output is filled in place
    out = torch.full((B, T, 768), 7.0, device=DEV)
    assert m.extract_embeddings(tk, out=out) is out and torch.equal(out, emb)
    with pytest.raises(M.BltError):
        m.extract_embeddings(tk, out=torch.empty((B, T, 767), device=DEV))


def test_forward_only_norms_skips_head():
    # ModelOutput fields left NULL are not computed: norms alone take one read
    # of the residual and no head
    cfg = M.LMTransformerConfig(dim=128, n_layers=2, n_heads=2, ffn_dim_multiplier=2.0,
                                multiple_of=64, max_seqlen=512, vocab_size=260)
    w = M.random_weights(cfg, 5, hidden=256)
    tok = torch.from_numpy(synth.tokens(synth.config_seed(4) + 5, (2, 300))).to(DEV)
    m = M.LMTransformer(cfg, w, device=0, max_tokens=600)
    full = m.forward_with_embeddings(tok)
    from blt_burn_amd import _lib
    from blt_burn_amd._torch import stream_ptr
    import ctypes
    norms = torch.zeros((2, 300), device=DEV)
    o = _lib.ModelOutputs(None, None, norms.data_ptr(), None, None)
    m.set_profiling(True)
    m.read_profile()
    _lib.check(_lib.lib().blt_model_forward(m._h, tok.to(torch.int32).data_ptr(), 2, 300,
                                            ctypes.byref(o), stream_ptr(DEV)), "forward")
    prof = m.read_profile()
    m.set_profiling(False)
    assert prof["head_gemm"][1] == 0 and prof["entropy"][1] == 0
    assert prof["final_norm_l2"][1] == 1
    torch.testing.assert_close(norms, full.embedding_norms, rtol=1e-6, atol=0)


@pytest.mark.parametrize("B,T", [(3, 0), (2, 1), (4, 5), (3, 8192), (2, 20000), (16, 8192)])
def test_patch_mask_starts_vs_host_scan(B, T):
    # starts are the positions whose mask is exactly 1 (other values such as 2
    # or -1 do not count, patcher.rs:133), ascending; lengths = next start (or
    # T) minus start; Sum(lengths) = T whenever position 0 starts a patch
    rng = np.random.default_rng(B * 100003 + T)
    mask = rng.choice(np.array([0, 0, 0, 1, 1, 2, -1], np.int32), size=(B, T))
    if T > 0:
        mask[0, 0] = 1
    md = torch.from_numpy(mask).to(DEV)
    starts, lengths, counts = patcher.patch_mask_starts(md)
    want = oracle.patch_indices(mask) if T > 0 else [[] for _ in range(B)]
    c = counts.cpu().numpy()
    st, ln = starts.cpu().numpy(), lengths.cpu().numpy()
    for b in range(B):
        assert c[b] == len(want[b])
        np.testing.assert_array_equal(st[b, :c[b]], want[b])
        if T > 0:
            np.testing.assert_array_equal(ln[b, :c[b]], oracle.patch_lengths([want[b]], T)[0])
    assert patcher.patch_start_indices_cpu(md) == want
    assert patcher.patch_start_indices_cpu(md) == patcher.patch_start_indices_cpu(md.cpu())
    if T > 0:
        assert int(ln[0, :c[0]].sum()) == T


def test_patch_mask_starts_of_boundary_mask():
    # the mask the monotonic pass writes compacts to the starts that pass wrote
    H = np.abs(synth.normal_f32(77, (4, 9000), 1.4, 0.6))
    mask, starts, lengths, counts = patcher.patch_boundaries(torch.from_numpy(H).to(DEV), 0.2)
    s2, l2, c2 = patcher.patch_mask_starts(mask)
    assert torch.equal(counts, c2)
    for b in range(4):
        n = int(counts[b])
        assert torch.equal(starts[b, :n], s2[b, :n]) and torch.equal(lengths[b, :n], l2[b, :n])


def test_patch_boundaries_on_two_streams():
    # two passes in flight at once on two streams (each call takes its own
    # workspace from the allocator on its stream): both match the oracle
    Ha = np.abs(synth.normal_f32(501, (16, 8192), 1.4, 0.6))
    Hb = np.abs(synth.normal_f32(502, (8, 20000), 1.1, 0.9))
    da, db = torch.from_numpy(Ha).to(DEV), torch.from_numpy(Hb).to(DEV)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    res = {}
    for it in range(3):
        with torch.cuda.stream(s1):
            res["a"] = patcher.patch_boundaries_rules(
                da, [(patcher.PATCH_MONOTONIC, 0.2), (patcher.PATCH_GLOBAL, 1.33)])
        with torch.cuda.stream(s2):
            res["b"] = patcher.patch_boundaries_rules(db, [(patcher.PATCH_MONOTONIC, 0.35)])
        torch.cuda.synchronize()
        for key, H, rules in (("a", Ha, [(0, 0.2), (1, 1.33)]), ("b", Hb, [(0, 0.35)])):
            for (mode, thr), (mask, starts, lengths, counts) in zip(rules, res[key]):
                np.testing.assert_array_equal(mask.cpu().numpy(), oracle.patch_mask(H, thr, mode))
                st, ln, ct = starts.cpu().numpy(), lengths.cpu().numpy(), counts.cpu().numpy()
                ws = oracle.patch_indices(oracle.patch_mask(H, thr, mode))
                wl = oracle.patch_lengths(ws, H.shape[1])
                for b in range(H.shape[0]):
                    np.testing.assert_array_equal(st[b, :ct[b]], ws[b])
                    np.testing.assert_array_equal(ln[b, :ct[b]], wl[b])


def test_pipeline_cache_does_not_keep_model_alive():
    # process_document caches its PipelineBuffer on the model; dropping the
    # model frees it at once (no reference cycle waiting for the collector)
    cfg = M.LMTransformerConfig(dim=128, n_layers=1, n_heads=2, ffn_dim_multiplier=2.0,
                                multiple_of=64, max_seqlen=8192, vocab_size=260)
    m = M.LMTransformer(cfg, M.random_weights(cfg, 3, hidden=256), device=0, max_tokens=8192)
    data = (synth.tokens(9, (1, 5000))[0] % 256).astype(np.uint8).tobytes()
    r1 = pipeline.process_document(data, m)
    r2 = pipeline.process_document(data, m)
    assert [(p.start_offset, p.length) for p in r1.patches] == \
        [(p.start_offset, p.length) for p in r2.patches]
    ref = weakref.ref(m)
    was = gc.isenabled()
    gc.disable()
    try:
        del m
        assert ref() is None, "the model outlived its last reference"
    finally:
        if was:
            gc.enable()
    # a buffer the caller holds keeps its model alive
    m2 = M.LMTransformer(cfg, M.random_weights(cfg, 3, hidden=256), device=0, max_tokens=8192)
    buf = pipeline.PipelineBuffer(1.335)
    buf.process_chunk(data[:4096], m2, is_last_chunk=True)
    ref2 = weakref.ref(m2)
    del m2
    assert ref2() is not None
    buf.close()
