"""safetensors weight ingest and per-document export (CPU): the reader and
writer against the `safetensors` package, the PyTorch-layout weight mapping,
and the save_blt_safetensors schema (huggingface_loader.rs:144-247)."""
import os

import numpy as np
import pytest

from blt_burn_amd import safetensors_io as st, synth
from blt_burn_amd.tokenizer import tokenize_bytes


def _tiny_weights(seed=3, L=2, D=64, F=128, V=260):
    rng = np.random.default_rng(seed)
    bf = lambda *s: synth.f32_to_bf16(rng.normal(0, 0.02, s).astype(np.float32))
    return {"tok_embeddings": bf(V, D), "attention_norm": bf(L, D), "ffn_norm": bf(L, D),
            "wq": bf(L, D, D), "wk": bf(L, D, D), "wv": bf(L, D, D), "wo": bf(L, D, D),
            "w1": bf(L, D, F), "w2": bf(L, F, D), "w3": bf(L, D, F), "norm": bf(D),
            "output": bf(D, V)}


def test_roundtrip_and_package_agree(tmp_path):
    safetensors_numpy = pytest.importorskip("safetensors.numpy")
    a = np.arange(12, dtype=np.float32).reshape(3, 4) / 7
    b = np.array([[1, -2, 3]], np.int32)
    p = str(tmp_path / "x.safetensors")
    st.write_safetensors(p, {"a": a, "b": b}, {"k": "v"})
    got, meta = st.read_safetensors(p)
    assert meta == {"k": "v"}
    assert got["a"][0] == "F32" and np.array_equal(got["a"][1], a)
    assert got["b"][0] == "I32" and np.array_equal(got["b"][1], b)
    # the reference format as the safetensors package reads and writes it
    ref = safetensors_numpy.load_file(p)
    assert np.array_equal(ref["a"], a) and np.array_equal(ref["b"], b)
    q = str(tmp_path / "y.safetensors")
    safetensors_numpy.save_file({"a": a, "b": b}, q)
    got2, _ = st.read_safetensors(q)
    assert np.array_equal(got2["a"][1], a) and np.array_equal(got2["b"][1], b)


def test_bf16_bits_match_torch(tmp_path):
    torch = pytest.importorskip("torch")
    safetensors_torch = pytest.importorskip("safetensors.torch")
    x = torch.randn(5, 7).to(torch.bfloat16)
    p = str(tmp_path / "t.safetensors")
    safetensors_torch.save_file({"x": x}, p)
    got, _ = st.read_safetensors(p)
    assert got["x"][0] == "BF16"
    assert np.array_equal(got["x"][1], x.view(torch.int16).numpy().view(np.uint16))
    # and the other way round
    q = str(tmp_path / "u.safetensors")
    st.write_safetensors(q, {"x": ("BF16", got["x"][1])})
    back = safetensors_torch.load_file(q)["x"]
    assert back.dtype == torch.bfloat16 and torch.equal(back, x)


def test_entropy_weights_pytorch_layout(tmp_path):
    """A checkpoint in PyTorch nn.Linear layout ([out, in]) with the
    facebook/blt-entropy names loads into the Burn [in, out] layout
    (SafetensorsFileRecorder's PyTorch adapter); f32 files round to bf16."""
    w = _tiny_weights()
    p = str(tmp_path / "m.safetensors")
    st.save_entropy_weights(p, w)
    t, _ = st.read_safetensors(p)
    # the file holds the PyTorch orientation
    assert t["layers.1.attention.wq.weight"][1].shape == (64, 64)
    assert np.array_equal(t["layers.1.feed_forward.w1.weight"][1], w["w1"][1].T)
    assert np.array_equal(t["output.weight"][1], w["output"].T)
    got, shp = st.load_entropy_weights(p)
    assert shp == {"dim": 64, "n_layers": 2, "hidden": 128, "vocab": 260}
    for k in w:
        assert got[k].dtype == np.uint16 and np.array_equal(got[k], w[k]), k
    # f32 checkpoint under a "model." prefix: values round to nearest-even bf16
    f32 = {("model." + n): v[1].view(np.uint16).astype(np.uint32) << 16 for n, v in t.items()}
    f32 = {n: (v.view(np.float32) * np.float32(1.0009765625)).astype(np.float32)
           for n, v in f32.items()}
    q = str(tmp_path / "m32.safetensors")
    st.write_safetensors(q, f32)
    got32, shp32 = st.load_entropy_weights(q)
    assert shp32 == shp
    want = synth.f32_to_bf16(f32["model.layers.0.attention.wk.weight"]).T
    assert np.array_equal(got32["wk"][0], want)


def test_entropy_weights_errors(tmp_path):
    w = _tiny_weights()
    p = str(tmp_path / "bad.safetensors")
    t = {"tok_embeddings.weight": ("BF16", w["tok_embeddings"])}
    st.write_safetensors(p, t)
    with pytest.raises(st.SafetensorsError):
        st.load_entropy_weights(p)
    q = str(tmp_path / "short.safetensors")
    with open(q, "wb") as f:
        f.write(b"\x10\x00")
    with pytest.raises(st.SafetensorsError):
        st.read_safetensors(q)


def test_save_blt_example_schema(tmp_path):
    from blt_burn_amd.ingest import BltExample, BltExampleWithEmbeddings
    toks = tokenize_bytes(b"hello world")
    n, dim = toks.size, 8
    rng = np.random.default_rng(0)
    H = rng.random(n).astype(np.float32) * 5
    norms = rng.random(n).astype(np.float32) * 3
    ex = BltExampleWithEmbeddings(
        core=BltExample("doc-1", "hello world", toks, H, np.array([2, 4, 5], np.int32),
                        np.ones(n, bool)),
        pre_norm_embeddings=rng.random(n * dim).astype(np.float32), embedding_dim=dim,
        prominence=norms, coherence_scores=norms * norms / (H + 1e-6),
        patch_indices=np.array([0, 2, 6], np.int32))
    p = str(tmp_path / "doc-1.safetensors")
    assert st.save_blt_example(p, ex, "doc-1")
    t, meta = st.read_safetensors(p)
    assert meta == {"sample_id": "doc-1", "embedding_dim": "8",
                    "metadata_file": "doc-1.hypergraph.db"}
    expect = {"tokens": ("I32", (1, n)), "embeddings": ("F32", (1, n, dim)),
              "prominence": ("F32", (1, n)), "entropies": ("F32", (1, n)),
              "coherence_scores": ("F32", (1, n)), "patch_indices": ("I32", (3,)),
              "patch_lengths": ("I32", (3,)), "mask": ("I32", (1, n))}
    assert {k: (v[0], v[1].shape) for k, v in t.items()} == expect
    assert np.array_equal(t["tokens"][1][0], toks) and t["mask"][1].sum() == n
    # an empty document writes nothing (huggingface_loader.rs:152-154)
    empty = BltExampleWithEmbeddings(
        core=BltExample("e", "", np.zeros(0, np.int32), np.zeros(0, np.float32),
                        np.zeros(0, np.int32), np.zeros(0, bool)),
        pre_norm_embeddings=np.zeros(0, np.float32), embedding_dim=dim,
        prominence=np.zeros(0, np.float32), coherence_scores=np.zeros(0, np.float32),
        patch_indices=np.zeros(0, np.int32))
    q = str(tmp_path / "e.safetensors")
    assert not st.save_blt_example(q, empty, "e") and not os.path.exists(q)
