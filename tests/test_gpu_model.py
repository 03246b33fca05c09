"""Parity of the whole entropy-model forward (blt_model_forward) with the CPU
oracle on identical seeded bf16 weights and tokens.  Tolerances (BASELINE):
entropies 2e-2 abs, pre-norm embedding norms 1e-2 rel, boundaries bit-exact
on the same entropies.  Logits and pre-norm embeddings (ModelOutput fields,
model.rs:229-245, 291-304) within 1e-2 of max |reference| each: the GEMM
operands are bf16 (relative rounding up to 2^-8 per element), so the expected
deviation is a few 1e-3 of the output scale; a permuted vocab column or a
dropped term moves them by O(1) of that scale.  At the full B=16 x 8192
size, size-independent properties instead: per-row independence and causal
prefix consistency."""
import numpy as np
import pytest
import torch

import np_ref
import oracle
from blt_burn_amd import model as M
from blt_burn_amd import patcher, synth

pytestmark = pytest.mark.gpu


def _oracle_weights(w):
    f = {k: synth.bf16_to_f32(v) for k, v in w.items()}
    return {"emb": f["tok_embeddings"], "attn_norm": f["attention_norm"],
            "ffn_norm": f["ffn_norm"], "wq": f["wq"], "wk": f["wk"], "wv": f["wv"],
            "wo": f["wo"], "w1": f["w1"], "w2": f["w2"], "w3": f["w3"], "norm": f["norm"],
            "out": f["output"]}


def _run(cfg, hidden, B, T, window, seed, w=None):
    w = M.random_weights(cfg, seed, hidden=hidden) if w is None else w
    tok = synth.tokens(synth.config_seed(4) + seed, (B, T))
    m = M.LMTransformer(cfg, w, device=0, max_tokens=B * T, window=window)
    out = m.forward_with_embeddings(torch.from_numpy(tok).cuda())
    torch.cuda.synchronize()
    ref = oracle.model_forward(dict(dim=cfg.dim, n_layers=cfg.n_layers,
                                    n_heads=cfg.resolved_n_heads(), hidden=hidden,
                                    vocab=cfg.vocab_size, max_seqlen=cfg.max_seqlen,
                                    norm_eps=cfg.norm_eps, rope_theta=cfg.rope_theta,
                                    window=window), _oracle_weights(w), tok)
    return out, ref


def _compare(out, ref, label):
    H = out.entropies.cpu().numpy()
    n = out.embedding_norms.cpu().numpy()
    pre = out.pre_norm_embeddings.cpu().numpy()
    dH = np.abs(H - ref["entropies"]).max()
    dn = (np.abs(n - ref["embedding_norms"]) / ref["embedding_norms"]).max()
    dpre = np.abs(pre - ref["pre_norm_embeddings"]).max() / np.abs(ref["pre_norm_embeddings"]).max()
    dl = np.abs(out.logits.cpu().numpy() - ref["logits"]).max()
    dl_rel = dl / np.abs(ref["logits"]).max()
    print("%s: entropy max|d|=%.2e norms max rel=%.2e pre max rel=%.2e logits max|d|=%.2e "
          "(rel %.2e)" % (label, dH, dn, dpre, dl, dl_rel))
    assert dH < 2e-2 and dn < 1e-2, (dH, dn)
    assert dpre < 1e-2, dpre
    assert dl_rel < 1e-2, (dl, dl_rel)
    np.testing.assert_allclose(out.coherence_scores.cpu().numpy(), ref["coherence_scores"],
                               rtol=3e-2)
    # boundaries: bit-exact given the same entropy array
    for mode, thr in ((patcher.PATCH_MONOTONIC, 0.2), (patcher.PATCH_GLOBAL, 1.33)):
        mask = patcher.patch_boundaries(out.entropies, thr, mode)[0].cpu().numpy()
        np.testing.assert_array_equal(mask, oracle.patch_mask(H, thr, mode))


@pytest.mark.parametrize("window", [0, 32, 100])
def test_tiny_model(window):
    cfg = M.LMTransformerConfig(dim=128, n_layers=2, n_heads=2, ffn_dim_multiplier=2.0,
                                multiple_of=64, max_seqlen=512, vocab_size=260)
    out, ref = _run(cfg, 256, 2, 200, window, seed=3)
    _compare(out, ref, "tiny w=%d" % window)


@pytest.mark.parametrize("window,T", [(0, 256), (512, 700), (300, 700)])
def test_entropy_model_dims(window, T):
    # the BLT entropy model at real size (14 x 768, 12 heads, FFN 2048, V 260), short T
    cfg = M.entropy_model_config()
    out, ref = _run(cfg, 2048, 1, T, window, seed=4)
    _compare(out, ref, "entropy-model T=%d w=%d" % (T, window))


def test_dim_192_model():
    # 3 heads: the QKV projection is 576 wide (576 % 128 == 64), which takes the
    # register-staged GEMM whose last N tile overhangs the output
    cfg = M.LMTransformerConfig(dim=192, n_layers=2, n_heads=3, ffn_dim_multiplier=2.0,
                                multiple_of=64, max_seqlen=512, vocab_size=260)
    out, ref = _run(cfg, 384, 2, 150, 0, seed=6)
    _compare(out, ref, "dim192")


def _far_norm_weights(cfg, seed, hidden):
    """Random weights whose RMSNorm weights are far from 1: 1 + N(0, 0.3), with
    one in ten of them 0.1 and one in twenty -0.5."""
    w = M.random_weights(cfg, seed, hidden=hidden)
    rng = np.random.default_rng(seed)
    for name in ("attention_norm", "ffn_norm", "norm"):
        shp = w[name].shape
        v = 1.0 + 0.3 * rng.standard_normal(shp)
        u = rng.random(shp)
        v[u < 0.1] = 0.1
        v[u > 0.95] = -0.5
        w[name] = synth.f32_to_bf16(v.astype(np.float32))
    return w


@pytest.mark.parametrize("B,T", [(1, 1), (1, 2), (3, 3), (2, 33)])
def test_entropy_model_few_tokens(B, T):
    # a handful of tokens at real size: every projection runs on 128 x 128
    # tiles that are almost all padding rows, attention on one partial key
    # tile, the boundary pass on its T <= 2 special cases
    cfg = M.entropy_model_config()
    out, ref = _run(cfg, 2048, B, T, 512, seed=6)
    _compare(out, ref, "entropy-model B=%d T=%d" % (B, T))


@pytest.mark.parametrize("window,T", [(0, 256), (512, 700)])
def test_entropy_model_far_norm_weights(window, T):
    # The RMSNorm weight scales the bf16 GEMM operand (bf16(x * w)); with
    # weights far from 1 any extra rounding or misplaced scale shows up here.
    cfg = M.entropy_model_config()
    out, ref = _run(cfg, 2048, 1, T, window, seed=8, w=_far_norm_weights(cfg, 8, 2048))
    _compare(out, ref, "far-norm T=%d w=%d" % (T, window))


def test_tiny_model_far_norm_weights():
    cfg = M.LMTransformerConfig(dim=128, n_layers=2, n_heads=2, ffn_dim_multiplier=2.0,
                                multiple_of=64, max_seqlen=512, vocab_size=260)
    out, ref = _run(cfg, 256, 2, 200, 0, seed=9, w=_far_norm_weights(cfg, 9, 256))
    _compare(out, ref, "tiny far-norm")


# Absolute ceilings on the entropy deviation from the fp32 oracle with spread
# entropies, just above what this build measures, so a precision regression
# fails even where the emulation bar below would still pass.  They exceed the
# 2e-2 bar of the N(0, 0.02) configurations: a known parity gap of bf16
# matrix-core operands on trained-like weights.
SPREAD_CEILING = {(0.1, 0.03): 5.5e-2, (0.12, 0.05): 0.24}


@pytest.mark.parametrize("out_std,std", [(0.1, 0.03), (0.12, 0.05)])
def test_entropy_model_spread_entropies(out_std, std):
    # With N(0, 0.02) weights every entropy sits near ln 260.  A larger output
    # head (and layer) scale spreads them over about 0.4 .. 3.4 nats, as a
    # trained model's are; there the bf16 operands the matrix cores take
    # (normalised activations, q/k/v, P, attention and SiLU-gate outputs, the
    # head's input) move the entropies by 0.05 .. 0.2 from the fp32 oracle.
    # The bar: within 1.5x of what a float32 forward with bf16 rounding at
    # exactly those operands deviates (np_ref, itself pinned to the oracle with
    # rounding off).  The two share most rounding decisions (0.1 / 0.03: 4.95e-2
    # against 4.92e-2), but the GPU rounds P against a running offset and sums
    # in another order, so single maxima over 1400 positions differ by up to
    # about 1.3x where the deep residual grows (0.12 / 0.05: 0.216 vs 0.169).
    cfg = M.entropy_model_config()
    w = M.random_weights(cfg, 11, hidden=2048, std=std)
    w["output"] = synth.normal_bf16(11 * 64 + 99, w["output"].shape, 0.0, out_std)
    out, ref = _run(cfg, 2048, 2, 700, 512, seed=11, w=w)
    ecfg = dict(dim=768, n_layers=14, n_heads=12, norm_eps=cfg.norm_eps,
                rope_theta=cfg.rope_theta, window=512)
    tok = synth.tokens(synth.config_seed(4) + 11, (2, 700))
    ow = _oracle_weights(w)
    exact = np_ref.model_forward_bf16_operands(ecfg, ow, tok, rounding=False)
    assert np.abs(exact["entropies"] - ref["entropies"]).max() < 1e-3
    # the GPU rounds every operand the emulation rounds except the head's
    # input, which the fused head carries as a bf16 hi + lo pair
    emu = np_ref.model_forward_bf16_operands(
        ecfg, ow, tok, points=[p for p in np_ref.ROUNDING_POINTS if p != "head_in"])

    def dev(r):
        return (np.abs(r["entropies"] - ref["entropies"]).max(),
                np.abs(r["logits"] - ref["logits"]).max(),
                np.abs(r["pre_norm_embeddings"] - ref["pre_norm_embeddings"]).max())

    got = {"entropies": out.entropies.cpu().numpy(), "logits": out.logits.cpu().numpy(),
           "pre_norm_embeddings": out.pre_norm_embeddings.cpu().numpy()}
    dg, de = dev(got), dev(emu)
    print("spread out_std=%g std=%g: GPU vs oracle entropy %.2e logits %.2e pre %.2e; "
          "bf16-operand emulation %.2e %.2e %.2e" % ((out_std, std) + dg + de))
    Hr = ref["entropies"]
    assert Hr.min() < 2.0 and Hr.max() - Hr.min() > 1.5, (Hr.min(), Hr.max())
    for g, e in zip(dg, de):
        assert g <= 1.5 * e + 1e-3, (dg, de)
    assert dg[0] < SPREAD_CEILING[(out_std, std)], dg
    n = out.embedding_norms.cpu().numpy()
    assert (np.abs(n - ref["embedding_norms"]) / ref["embedding_norms"]).max() < 1e-2
    # Boundaries from the GPU's entropies: bit-exact against the oracle's rule
    # on the same array, and equal to the oracle's own boundaries wherever its
    # entropy is clear of the threshold by more than the deviation allowed
    # above (twice that for the difference of two entropies).
    H = got["entropies"]
    tol = 1.5 * de[0] + 1e-3
    for mode, thr in ((patcher.PATCH_MONOTONIC, 0.2), (patcher.PATCH_GLOBAL, 1.33)):
        mask = patcher.patch_boundaries(out.entropies, thr, mode)[0].cpu().numpy()
        np.testing.assert_array_equal(mask, oracle.patch_mask(H, thr, mode))
        want = oracle.patch_mask(Hr, thr, mode)
        if mode == patcher.PATCH_GLOBAL:
            clear = np.abs(Hr - thr) > tol
        else:
            d = np.zeros_like(Hr)
            d[:, 1:] = Hr[:, 1:] - Hr[:, :-1]
            clear = np.abs(d - thr) > 2 * tol
        clear[:, :2] = True  # positions 0 and 1 start patches under either rule
        assert 0 < want.sum() < want.size, (mode, want.sum())
        np.testing.assert_array_equal(mask[clear], want[clear])
    # Starts the GPU moves against the oracle's own under the monotonic rule at
    # the reference default delta 1.335 (blt_core.rs:73) and at 0.2, beside the
    # emulation's: positions near the threshold flip, no more than the bf16
    # operands account for.
    for thr in (1.335, 0.2):
        want = oracle.patch_mask(Hr, thr, patcher.PATCH_MONOTONIC)
        g_d = int((oracle.patch_mask(H, thr, patcher.PATCH_MONOTONIC) != want).sum())
        e_d = int((oracle.patch_mask(emu["entropies"], thr, patcher.PATCH_MONOTONIC)
                   != want).sum())
        print("spread out_std=%g std=%g: delta %g starts differing from the oracle's: "
              "GPU %d, emulation %d, of %d starts over %d positions"
              % (out_std, std, thr, g_d, e_d, int(want.sum()), want.size))
        assert g_d <= 2 * e_d + 2, (thr, g_d, e_d)


@pytest.mark.parametrize("vocab", [100, 258])
def test_tiny_model_other_vocab(vocab):
    # V = 100 takes the fused head with most of its 288 packed columns zero;
    # V = 258 (not a multiple of 4) the separate final norm, head GEMM and
    # entropy kernels
    cfg = M.LMTransformerConfig(dim=128, n_layers=2, n_heads=2, ffn_dim_multiplier=2.0,
                                multiple_of=64, max_seqlen=512, vocab_size=vocab)
    w = M.random_weights(cfg, 13, hidden=256)
    B, T = 2, 150
    tok = synth.tokens(synth.config_seed(4) + 13, (B, T)) % vocab
    m = M.LMTransformer(cfg, w, device=0, max_tokens=B * T)
    out = m.forward_with_embeddings(torch.from_numpy(tok).cuda())
    torch.cuda.synchronize()
    ref = oracle.model_forward(dict(dim=128, n_layers=2, n_heads=2, hidden=256, vocab=vocab,
                                    max_seqlen=512, norm_eps=cfg.norm_eps,
                                    rope_theta=cfg.rope_theta, window=0),
                               _oracle_weights(w), tok)
    _compare(out, ref, "tiny vocab=%d" % vocab)


def test_reference_configured_ffn_768():
    # LMTransformerConfig::init as configured gives FFN 768 (model.rs:468-473)
    cfg = M.entropy_model_config()
    cfg.n_layers = 2
    out, ref = _run(cfg, cfg.ffn_hidden(), 2, 128, 0, seed=5)
    _compare(out, ref, "ffn768")


def test_full_size_properties():
    # config 4 size: B=16, T=8192, window 512.  Rows are independent and the
    # forward is causal: row b of the batch equals that sequence run alone, and
    # a prefix run gives the prefix of the outputs (bit-exact).
    cfg = M.entropy_model_config()
    w = M.random_weights(cfg, 11, hidden=2048)
    B, T = 16, 8192
    tok = torch.from_numpy(synth.tokens(synth.config_seed(4), (B, T))).cuda()
    m = M.LMTransformer(cfg, w, device=0, max_tokens=B * T, window=512)
    out = m.forward_with_embeddings(tok)
    H = out.entropies
    assert torch.isfinite(H).all() and (H >= 0).all() and (H <= np.log(260) + 1e-4).all()
    assert torch.isfinite(out.pre_norm_embeddings).all()
    one = m.forward_with_embeddings(tok[5:6].contiguous())
    assert torch.equal(one.entropies[0], H[5])
    assert torch.equal(one.embedding_norms[0], out.embedding_norms[5])
    pre = m.forward_with_embeddings(tok[2:3, :3000].contiguous())
    assert torch.equal(pre.entropies[0], H[2, :3000])
    _, starts, lengths, counts = patcher.patch_boundaries(H, 0.2, patcher.PATCH_MONOTONIC)
    c = counts.cpu()
    ln = lengths.cpu()
    for b in range(B):
        assert int(ln[b, :c[b]].sum()) == T


def test_from_safetensors_matches_in_memory_weights(tmp_path):
    """A facebook/blt-entropy style checkpoint (PyTorch [out, in] layout) loads
    to the same model: outputs are bit-identical to the in-memory weights, and
    the FFN width comes from the file (model_loader.rs:103-145)."""
    from blt_burn_amd import safetensors_io as st
    cfg = M.LMTransformerConfig(dim=128, n_layers=2, n_heads=2, ffn_dim_multiplier=1.0,
                                multiple_of=64, max_seqlen=256, vocab_size=260)
    w = M.random_weights(cfg, 11, hidden=384)  # the config rule alone would give 128
    path = str(tmp_path / "model.safetensors")
    st.save_entropy_weights(path, w)
    tok = torch.from_numpy(synth.tokens(synth.config_seed(4), (2, 100))).cuda()
    a = M.LMTransformer(cfg, w, device=0, max_tokens=200).forward_with_embeddings(tok)
    mb = M.LMTransformer.from_safetensors(path, cfg, device=0, max_tokens=200)
    assert mb.hidden == 384
    b = mb.forward_with_embeddings(tok)
    torch.cuda.synchronize()
    for n in ("logits", "pre_norm_embeddings", "embedding_norms", "entropies"):
        assert torch.equal(getattr(a, n), getattr(b, n)), n
    bad = M.LMTransformerConfig(dim=128, n_layers=3, n_heads=2, max_seqlen=256)
    with pytest.raises(M.BltError):
        M.LMTransformer.from_safetensors(path, bad, device=0, max_tokens=200)


def test_from_mpk_matches_in_memory_weights(tmp_path):
    """A Burn NamedMpkFileRecorder record (model_loader.rs:119-125: the `.mpk`
    branch, Linear weights in Burn's [d_input, d_output] layout) loads to the
    same model as the in-memory weights, through from_mpk and through
    from_checkpoint's file-name dispatch; outputs are bit-identical."""
    pytest.importorskip("msgpack")
    from blt_burn_amd import mpk_io
    cfg = M.LMTransformerConfig(dim=128, n_layers=2, n_heads=2, ffn_dim_multiplier=1.0,
                                multiple_of=64, max_seqlen=256, vocab_size=260)
    w = M.random_weights(cfg, 12, hidden=384)
    path = str(tmp_path / "blt_entropy_model.mpk")
    mpk_io.save_entropy_weights_mpk(path, w)
    tok = torch.from_numpy(synth.tokens(synth.config_seed(4), (2, 100))).cuda()
    a = M.LMTransformer(cfg, w, device=0, max_tokens=200).forward_with_embeddings(tok)
    for load in (M.LMTransformer.from_mpk, M.LMTransformer.from_checkpoint):
        mb = load(path, cfg, device=0, max_tokens=200)
        assert mb.hidden == 384
        b = mb.forward_with_embeddings(tok)
        torch.cuda.synchronize()
        for n in ("logits", "pre_norm_embeddings", "embedding_norms", "entropies"):
            assert torch.equal(getattr(a, n), getattr(b, n)), n
