"""Burn `.mpk` weight records (CPU): the NamedMpkFileRecorder layout of the
entropy model (model_loader.rs:119-125) that mpk_io reads and writes.

No file written by burn itself exists here, so these pin the reader against
records built by hand, field by field, in each layout it accepts (current
ParamSerde/TensorData, a bare TensorData, the older DataSerialize list form,
dtype as name, index or one-key map) and against the writer."""
import numpy as np
import pytest

msgpack = pytest.importorskip("msgpack")

from blt_burn_amd import mpk_io, synth


def _tiny_weights(seed=5, L=2, D=64, F=128, V=260):
    rng = np.random.default_rng(seed)
    bf = lambda *s: synth.f32_to_bf16(rng.normal(0, 0.02, s).astype(np.float32))
    return {"tok_embeddings": bf(V, D), "attention_norm": bf(L, D), "ffn_norm": bf(L, D),
            "wq": bf(L, D, D), "wk": bf(L, D, D), "wv": bf(L, D, D), "wo": bf(L, D, D),
            "w1": bf(L, D, F), "w2": bf(L, F, D), "w3": bf(L, D, F), "norm": bf(D),
            "output": bf(D, V)}


def _f32(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def _hand_record(w, tensor):
    """A record in burn's module-tree layout, every tensor through `tensor`
    (f32 array -> its serialized form)."""
    L = w["wq"].shape[0]
    lin = lambda a: {"weight": tensor(_f32(a)), "bias": None}
    nrm = lambda a: {"weight": tensor(_f32(a)), "epsilon": None}
    layers = [{"attention_norm": nrm(w["attention_norm"][i]),
               "attention": {n: lin(w[n][i]) for n in ("wq", "wk", "wv", "wo")},
               "ffn_norm": nrm(w["ffn_norm"][i]),
               "feed_forward": {n: lin(w[n][i]) for n in ("w1", "w2", "w3")}}
              for i in range(L)]
    return {"metadata": {"float": "f32", "int": "i32", "format": "x", "version": "0.19.1",
                         "settings": "FullPrecisionSettings"},
            "item": {"tok_embeddings": {"weight": tensor(_f32(w["tok_embeddings"]))},
                     "layers": layers, "norm": nrm(w["norm"]), "output": lin(w["output"]),
                     "max_seqlen": None, "head_dim": None, "rope_theta": None}}


def _write(path, rec):
    with open(path, "wb") as f:
        f.write(msgpack.packb(rec, use_bin_type=True))


def _same(a, b):
    assert set(a) == set(b)
    for k in a:
        assert a[k].dtype == np.uint16 and a[k].shape == b[k].shape, k
        assert np.array_equal(a[k], b[k]), k


def test_writer_reader_roundtrip(tmp_path):
    w = _tiny_weights()
    p = str(tmp_path / "model.mpk")
    mpk_io.save_entropy_weights_mpk(p, w)
    got, shp = mpk_io.load_entropy_weights_mpk(p)
    _same(got, w)
    assert shp == {"dim": 64, "n_layers": 2, "hidden": 128, "vocab": 260}


def test_writer_layout(tmp_path):
    """The written record, decoded as plain MessagePack: BurnRecord metadata,
    the module tree by field name, ParamSerde { id, param: TensorData }, Burn's
    [d_input, d_output] linear layout and f32 little-endian element bytes."""
    w = _tiny_weights(L=3)
    p = str(tmp_path / "model.mpk")
    mpk_io.save_entropy_weights_mpk(p, w)
    with open(p, "rb") as f:
        rec = msgpack.unpackb(f.read(), raw=False)
    assert set(rec) == {"metadata", "item"}
    assert set(rec["metadata"]) == {"float", "int", "format", "version", "settings"}
    assert rec["metadata"]["float"] == "f32" and rec["metadata"]["version"] == "0.19.1"
    item = rec["item"]
    assert {"tok_embeddings", "layers", "norm", "output"} <= set(item)
    assert len(item["layers"]) == 3
    blk = item["layers"][1]
    assert set(blk) == {"attention_norm", "attention", "ffn_norm", "feed_forward"}
    wq = blk["attention"]["wq"]["weight"]
    assert set(wq) == {"id", "param"} and isinstance(wq["id"], str)
    td = wq["param"]
    assert td["dtype"] == "F32" and td["shape"] == [64, 64] and isinstance(td["bytes"], bytes)
    vals = np.frombuffer(td["bytes"], "<f4").reshape(64, 64)
    assert np.array_equal(vals, _f32(w["wq"][1]))
    w2 = blk["feed_forward"]["w2"]["weight"]["param"]
    assert w2["shape"] == [128, 64]  # [d_input = F, d_output = D]
    assert item["output"]["weight"]["param"]["shape"] == [64, 260]
    assert item["output"]["bias"] is None


@pytest.mark.parametrize("form", ["paramserde", "bare", "index_dtype", "map_dtype",
                                  "list_bytes", "dataserialize", "bf16", "f64"])
def test_reader_accepts_record_layouts(tmp_path, form):
    w = _tiny_weights(seed=9)

    def tensor(a):
        a = np.ascontiguousarray(a, "<f4")
        td = {"bytes": a.tobytes(), "shape": list(a.shape), "dtype": "F32"}
        if form == "bare":
            return td
        if form == "index_dtype":
            td["dtype"] = 1  # F32's variant index
        if form == "map_dtype":
            td["dtype"] = {"F32": None}
        if form == "list_bytes":
            td["bytes"] = list(a.tobytes())
        if form == "dataserialize":
            return {"id": "1", "param": {"value": a.reshape(-1).tolist(), "shape": list(a.shape)}}
        if form == "bf16":
            bits = synth.f32_to_bf16(a)
            td = {"bytes": bits.astype("<u2").tobytes(), "shape": list(a.shape), "dtype": "BF16"}
        if form == "f64":
            td = {"bytes": a.astype("<f8").tobytes(), "shape": list(a.shape), "dtype": "F64"}
        return {"id": "abc", "param": td}

    p = str(tmp_path / "m.mpk")
    _write(p, _hand_record(w, tensor))
    got, shp = mpk_io.load_entropy_weights_mpk(p)
    _same(got, w)
    assert shp["n_layers"] == 2 and shp["hidden"] == 128


def test_f32_values_round_to_nearest_even(tmp_path):
    """Full-precision weights that are not bf16 values load rounded to nearest
    even, as the safetensors path rounds F32 checkpoints."""
    w = _tiny_weights(seed=2)
    rng = np.random.default_rng(4)
    noise = rng.normal(0, 1e-4, w["wq"].shape).astype(np.float32)
    full = _f32(w["wq"]) + noise
    rec = _hand_record(w, lambda a: {"id": "i", "param": {
        "bytes": np.ascontiguousarray(a, "<f4").tobytes(), "shape": list(a.shape),
        "dtype": "F32"}})
    for i in range(2):
        a = np.ascontiguousarray(full[i], "<f4")
        rec["item"]["layers"][i]["attention"]["wq"]["weight"]["param"]["bytes"] = a.tobytes()
    p = str(tmp_path / "m.mpk")
    _write(p, rec)
    got, _ = mpk_io.load_entropy_weights_mpk(p)
    assert np.array_equal(got["wq"], synth.f32_to_bf16(full))
    # ties go to even: 1 + 2^-8 sits halfway between two bf16 values
    assert synth.f32_to_bf16(np.float32(1 + 2 ** -8)) == 0x3F80


def test_reader_rejects_bad_records(tmp_path):
    w = _tiny_weights()
    p = str(tmp_path / "m.mpk")
    mpk_io.save_entropy_weights_mpk(p, w)
    with open(p, "rb") as f:
        good = msgpack.unpackb(f.read(), raw=False)

    def bad(mut, match):
        rec = msgpack.unpackb(msgpack.packb(good, use_bin_type=True), raw=False)
        mut(rec)
        _write(p, rec)
        with pytest.raises(mpk_io.MpkError, match=match):
            mpk_io.load_entropy_weights_mpk(p)

    def transposed(r):  # PyTorch [out, in] orientation of a non-square linear
        td = r["item"]["layers"][0]["feed_forward"]["w2"]["weight"]["param"]
        td["shape"] = td["shape"][::-1]
    bad(transposed, "expected")
    bad(lambda r: r["item"]["layers"].clear(), "no transformer layers")
    bad(lambda r: r["item"]["layers"][1]["attention"].pop("wv"), "missing field wv")

    def short(r):
        td = r["item"]["norm"]["weight"]["param"]
        td["bytes"] = td["bytes"][:-4]
    bad(short, "bytes for shape")

    def biased(r):
        r["item"]["output"]["bias"] = {"id": "b", "param": {
            "bytes": np.ones(260, "<f4").tobytes(), "shape": [260], "dtype": "F32"}}
    bad(biased, "bias")

    def int_dtype(r):
        r["item"]["norm"]["weight"]["param"]["dtype"] = "I32"
    bad(int_dtype, "non-float")

    def str_bytes(r):
        r["item"]["norm"]["weight"]["param"]["bytes"] = "not bytes"
    bad(str_bytes, "tensor bytes of type")
    with open(p, "wb") as f:
        f.write(b"\xc1not msgpack")
    with pytest.raises(mpk_io.MpkError):
        mpk_io.load_entropy_weights_mpk(p)


def test_zero_bias_is_accepted(tmp_path):
    """A linear saved with an all-zero bias (with_bias(true) and never trained)
    computes the same function, so it loads."""
    w = _tiny_weights()
    p = str(tmp_path / "m.mpk")
    mpk_io.save_entropy_weights_mpk(p, w)
    with open(p, "rb") as f:
        rec = msgpack.unpackb(f.read(), raw=False)
    rec["item"]["output"]["bias"] = {"id": "b", "param": {
        "bytes": np.zeros(260, "<f4").tobytes(), "shape": [260], "dtype": "F32"}}
    _write(p, rec)
    got, _ = mpk_io.load_entropy_weights_mpk(p)
    _same(got, w)
