"""Pins the CPU oracle (oracle/oracle.c) against the reference's known answers,
hand-worked patch vectors, closed forms and an independent float64 NumPy
statement (np_ref.py).  CPU only."""
import json
import math
import os

import numpy as np
import pytest

import np_ref
import oracle

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))
rng = np.random.default_rng(1234)


def _ent_input(case):
    x = np.full(case["shape"], case["fill"], np.float32)
    if "hot" in case:
        x[..., 0] = case["hot"]
    return x


@pytest.mark.parametrize("case", KAT["entropy"], ids=lambda c: c["name"])
def test_entropy_kat(case):
    H = oracle.entropy(_ent_input(case))
    assert H.shape == tuple(case["shape"][:-1])
    assert np.all(np.abs(H - case["expected"]) < case["tol"])


def test_entropy_vs_float64():
    x = rng.normal(0, 2.0, (4, 64, 260)).astype(np.float32)
    np.testing.assert_allclose(oracle.entropy(x), np_ref.entropy(x), atol=2e-5)
    x = rng.normal(0, 1.0, (2, 4, 10)).astype(np.float32)  # test_fused_entropy.rs:25-56 shape
    np.testing.assert_allclose(oracle.entropy(x), np_ref.entropy(x), atol=1e-5)


def test_entropy_extreme_bounds():
    x = rng.normal(50, 20, (1, 64, 260)).astype(np.float32)  # test_fused_entropy.rs:89-113
    H = oracle.entropy(x)
    assert np.all(np.isfinite(H)) and np.all(H >= 0) and np.all(H <= math.log(260) + 1e-5)


@pytest.mark.parametrize("mode", [0, 1])
def test_rms_norm_vs_float64(mode):
    x = rng.normal(0, 1, (2, 8, 64)).astype(np.float32)  # test_fused_ops.rs:19-57 shape
    w = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    np.testing.assert_allclose(oracle.rms_norm(x, w, 1e-6, mode), np_ref.rms_norm(x, w, 1e-6, mode),
                               rtol=2e-6, atol=2e-6)
    x = rng.normal(0, 1, (16, 768)).astype(np.float32)
    w = (1 + rng.normal(0, 0.02, 768)).astype(np.float32)
    np.testing.assert_allclose(oracle.rms_norm(x, w, 1e-5, mode), np_ref.rms_norm(x, w, 1e-5, mode),
                               rtol=2e-6, atol=2e-6)


def test_rms_norm_eps_placement_closed_form():
    # constant row c: after-sqrt gives c / (|c| + eps), inside-sqrt gives c / sqrt(c^2 + eps)
    c, eps = 0.01, 1e-3
    x = np.full((1, 32), c, np.float32)
    w = np.ones(32, np.float32)
    assert np.allclose(oracle.rms_norm(x, w, eps, 0), c / (c + eps), rtol=1e-6)
    assert np.allclose(oracle.rms_norm(x, w, eps, 1), c / math.sqrt(c * c + eps), rtol=1e-6)


def test_l2_softmax_silu_coherence_vs_float64():
    x = rng.normal(0, 1, (2, 16, 128)).astype(np.float32)
    np.testing.assert_allclose(oracle.l2_norm(x), np_ref.l2_norm(x), rtol=2e-6)
    s = rng.normal(0, 1, (2, 8, 32, 32)).astype(np.float32)
    p = oracle.softmax(s)
    np.testing.assert_allclose(p, np_ref.softmax(s), atol=1e-6)
    np.testing.assert_allclose(p.sum(-1), 1.0, atol=1e-5)
    big = rng.normal(50, 20, (2, 8, 64)).astype(np.float32)  # test_fused_ops.rs:269-287
    pb = oracle.softmax(big)
    assert np.all((pb >= 0) & (pb <= 1))
    g, u = (rng.normal(0, 1, (2, 8, 256)).astype(np.float32) for _ in range(2))
    np.testing.assert_allclose(oracle.silu_gate(g, u), np_ref.silu_gate(g, u), atol=1e-6)
    n = rng.uniform(0.1, 10, (4, 32)).astype(np.float32)
    H = rng.uniform(0.1, 5, (4, 32)).astype(np.float32)
    np.testing.assert_allclose(oracle.coherence(n, H, 1e-6),
                               n.astype(np.float64) ** 2 / (H + 1e-6), rtol=1e-6)


@pytest.mark.parametrize("case", KAT["patch"], ids=lambda c: c["name"])
def test_patch_kat(case):
    H = np.array(case["H"], np.float32)
    mode = 0 if case["mode"] == "monotonic" else 1
    mask = oracle.patch_mask(H, case["thr"], mode)
    assert mask.tolist() == case["mask"]
    starts = oracle.patch_indices(mask)
    assert starts == case["starts"]
    lengths = oracle.patch_lengths(starts, H.shape[1])
    assert lengths == case["lengths"]
    assert all(sum(l) == H.shape[1] for l in lengths)


def test_patch_empty_rows():
    H = np.zeros((3, 0), np.float32)
    assert oracle.patch_mask(H, 0.2, 0).shape == (3, 0)


def test_patch_properties_random():
    H = rng.normal(3.0, 0.5, (5, 1000)).astype(np.float32)
    for mode, thr in ((0, 0.2), (1, 3.1)):
        m = oracle.patch_mask(H, thr, mode)
        assert np.all(m[:, :2] == 1)
        starts = oracle.patch_indices(m)
        lengths = oracle.patch_lengths(starts, 1000)
        for s, l in zip(starts, lengths):
            assert sum(l) == 1000 and all(x > 0 for x in l)
            assert np.all(np.diff(s) == np.array(l[:-1]))


def test_rope_table():
    d, T, theta = 64, 8192, 10000.0
    cs = oracle.rope_table(d, T, theta)
    assert np.all(cs[0, :, 0] == 1.0) and np.all(cs[0, :, 1] == 0.0)  # position 0 = identity
    # closed form inv_freq = theta^(-2i/d); angles rounded to f32 as model.rs:24-52
    i = np.arange(d // 2)
    inv32 = (np.float32(1.0) / (theta ** (2.0 * i / d)).astype(np.float32)).astype(np.float32)
    ang32 = (np.arange(T, dtype=np.float32)[:, None] * inv32[None, :]).astype(np.float32)
    np.testing.assert_allclose(cs[..., 0], np.cos(ang32.astype(np.float64)), atol=2e-7)
    np.testing.assert_allclose(cs[..., 1], np.sin(ang32.astype(np.float64)), atol=2e-7)
    # and close to the exact-angle table (the f32 angle rounding is the only gap)
    a64 = np_ref.rope_angles(d, T, theta)
    assert np.abs(cs[..., 0] - np.cos(a64)).max() < 2e-3
    np.testing.assert_allclose(cs[..., 0] ** 2 + cs[..., 1] ** 2, 1.0, atol=1e-6)


@pytest.mark.parametrize("causal,window,theta", [(True, 0, 0.0), (True, 16, 0.0), (False, 0, 0.0),
                                                 (True, 0, 10000.0), (True, 24, 10000.0)])
def test_attention_vs_float64(causal, window, theta):
    q, k, v = (rng.normal(0, 1, (2, 3, 70, 64)).astype(np.float32) for _ in range(3))
    o = oracle.attention(q, k, v, causal, window, theta)
    np.testing.assert_allclose(o, np_ref.attention(q, k, v, causal, window, theta), atol=2e-5)


def test_attention_closed_forms():
    q, k, v = (rng.normal(0, 1, (1, 2, 40, 64)).astype(np.float32) for _ in range(3))
    o = oracle.attention(q, k, v, True, 0, 10000.0)
    np.testing.assert_allclose(o[:, :, 0], v[:, :, 0], atol=1e-6)  # causal row 0 sees only key 0
    ow = oracle.attention(q, k, v, True, 40, 10000.0)  # window >= T equals full causal
    np.testing.assert_array_equal(o, ow)
    o1 = oracle.attention(q, k, v, True, 1, 0.0)  # window 1: each query sees only itself
    np.testing.assert_allclose(o1, v, atol=1e-6)


@pytest.mark.parametrize("Tq,Tkv,d,causal", [(33, 33, 64, True), (20, 50, 16, True),
                                              (50, 20, 100, True), (17, 40, 256, False),
                                              (1, 7, 8, True)])
def test_attention_kernel_vs_float64(Tq, Tkv, d, causal):
    # the reference kernel's semantics: any head_dim, Tq != Tkv, causal j <= i
    q = rng.normal(0, 1, (2, 3, Tq, d)).astype(np.float32)
    k, v = (rng.normal(0, 1, (2, 3, Tkv, d)).astype(np.float32) for _ in range(2))
    o = oracle.attention_kernel(q, k, v, causal)
    np.testing.assert_allclose(o, np_ref.attention_qkv(q, k, v, causal), atol=2e-5)


def test_attention_kernel_closed_forms():
    q = rng.normal(0, 1, (1, 2, 30, 64)).astype(np.float32)
    k, v = (rng.normal(0, 1, (1, 2, 30, 64)).astype(np.float32) for _ in range(2))
    # the same semantics as the model's attention when Tq = Tkv
    np.testing.assert_allclose(oracle.attention_kernel(q, k, v, True),
                               oracle.attention(q, k, v, True, 0, 0.0), atol=1e-5)
    # one key: every query returns it
    o1 = oracle.attention_kernel(q, k[:, :, :1], v[:, :, :1], False)
    np.testing.assert_allclose(o1, np.broadcast_to(v[:, :, :1], o1.shape), atol=1e-6)
    # causal row 0 sees only key 0
    np.testing.assert_allclose(oracle.attention_kernel(q, k, v, True)[:, :, 0], v[:, :, 0],
                               atol=1e-6)


def _tiny_model(hidden=128, L=2, D=128, H=2, V=260, seed=5):
    r = np.random.default_rng(seed)
    g = lambda *s: r.normal(0, 0.05, s).astype(np.float32)  # noqa: E731
    w = {"emb": g(V, D), "attn_norm": 1 + g(L, D), "ffn_norm": 1 + g(L, D), "wq": g(L, D, D),
         "wk": g(L, D, D), "wv": g(L, D, D), "wo": g(L, D, D), "w1": g(L, D, hidden),
         "w2": g(L, hidden, D), "w3": g(L, D, hidden), "norm": 1 + g(D), "out": g(D, V)}
    cfg = dict(dim=D, n_layers=L, n_heads=H, hidden=hidden, vocab=V, max_seqlen=64,
               norm_eps=1e-5, rope_theta=10000.0)
    return cfg, w


@pytest.mark.parametrize("window", [0, 8])
def test_model_forward_vs_float64(window):
    cfg, w = _tiny_model()
    cfg["window"] = window
    tok = np.random.default_rng(9).integers(0, 260, (2, 33)).astype(np.int32)
    got = oracle.model_forward(cfg, w, tok)
    ref = np_ref.model_forward(cfg, w, tok)
    for k in ("logits", "pre_norm_embeddings", "embedding_norms", "entropies", "coherence_scores"):
        np.testing.assert_allclose(got[k], ref[k], rtol=1e-4, atol=1e-4, err_msg=k)


def test_bf16_round_and_operand_emulation():
    # bf16 rounding: nearest, ties to even, low 16 bits cleared
    x = np.array([1.0, 1.00390625, 1.005859375, 1.01171875, -3.14159, 65504.0], np.float32)
    np.testing.assert_array_equal(np_ref.bf16_round(x),
                                  np.array([1.0, 1.0, 1.0078125, 1.015625, -3.140625, 65536.0],
                                           np.float32))
    y = np.random.default_rng(3).normal(0, 10, 4096).astype(np.float32)
    r = np_ref.bf16_round(y)
    assert not (r.view(np.uint32) & 0xFFFF).any()
    assert (np.abs(r - y) <= np.abs(y) * 2.0 ** -8).all()  # half of an 8-bit significand step
    # the float32 forward with rounding off is the reference's math (the C oracle)
    cfg, w = _tiny_model()
    cfg["window"] = 8
    tok = np.random.default_rng(9).integers(0, 260, (2, 33)).astype(np.int32)
    ref = oracle.model_forward(cfg, w, tok)
    ex = np_ref.model_forward_bf16_operands(cfg, w, tok, rounding=False)
    for k in ("logits", "pre_norm_embeddings", "entropies"):
        np.testing.assert_allclose(ex[k], ref[k], rtol=1e-4, atol=1e-4, err_msg=k)
    # with rounding on it moves, by about the bf16 step and not more
    em = np_ref.model_forward_bf16_operands(cfg, w, tok)
    d = np.abs(em["logits"] - ref["logits"]).max() / np.abs(ref["logits"]).max()
    assert 1e-4 < d < 2e-2, d
