"""Burn `.mpk` weight files for the entropy model (host side, no GPU).

load_entropy_model (model_loader.rs:119-125) reads a checkpoint whose name
ends in `.mpk` with burn 0.19.1's NamedMpkFileRecorder<FullPrecisionSettings>
(Cargo.toml:23; burn is a crates.io dependency of the reference, not vendored
under it).  That recorder writes the module record with rmp_serde's named
MessagePack encoding, uncompressed:

    BurnRecord { metadata: BurnMetadata { float, int, format, version, settings },
                 item: <the LMTransformer record> }

The item mirrors the module tree.  Each #[derive(Module)] struct is a map keyed
by its field names:
- LMTransformer: tok_embeddings, layers, norm, output (model.rs:247-256);
- TransformerBlock: attention_norm, attention, ffn_norm, feed_forward
  (model.rs:491-497);
- Attention: wq, wk, wv, wo (model.rs:564-573);
- FeedForward: w1, w2, w3 (model.rs:720-725);
- RmsNorm: weight (model.rs:752-756);
- burn's Linear: weight, bias.  Its weight is [d_input, d_output], Burn's own
  layout, so it loads without the transpose a PyTorch checkpoint needs.
- burn's Embedding: weight [n_embedding, d_model].

A Vec<TransformerBlock> is an array.  A Param<Tensor> is ParamSerde { id, param },
with param = TensorData { bytes, shape, dtype }: the little-endian element bytes
as a MessagePack bin, the shape, and the element type as a DType variant name.
Plain usize / f64 fields (max_seqlen, head_dim, rope_theta, epsilon, n_heads,
...) are constants whose record is a unit value.

The reader also takes the layouts a hand-edited or older file may use.  The
param may come without its ParamSerde wrapper.  Burn before TensorData wrote
DataSerialize { value: [...], shape: [...] }.  The dtype may be a variant index
or a one-key map.

Parity with a file that burn itself wrote is unpinned: neither the reference
nor this image holds an .mpk checkpoint or burn's source.  The tests pin the
writer against the reader, and the reader against records built by hand in
each accepted layout.
"""
import numpy as np

from .synth import f32_to_bf16

try:
    import msgpack
except ImportError:  # pragma: no cover - msgpack ships with the image
    msgpack = None


class MpkError(ValueError):
    pass


# burn-tensor's DType variants in declaration order (a variant index maps here)
_DTYPE_ORDER = ("F64", "F32", "Flex32", "F16", "BF16", "I64", "I32", "I16", "I8",
                "U64", "U32", "U16", "U8", "Bool")
_FLOAT_NP = {"F64": "<f8", "F32": "<f4", "Flex32": "<f4", "F16": "<f2", "BF16": "<u2"}

BURN_VERSION = "0.19.1"
RECORDER = "burn::record::file::NamedMpkFileRecorder<burn::record::settings::FullPrecisionSettings>"


def _need_msgpack():
    if msgpack is None:
        raise MpkError("the msgpack package is needed to read .mpk weight files")


def _dtype_name(d):
    if isinstance(d, str):
        return d
    if isinstance(d, int) and 0 <= d < len(_DTYPE_ORDER):
        return _DTYPE_ORDER[d]
    if isinstance(d, dict) and len(d) == 1:
        return _dtype_name(next(iter(d)))
    raise MpkError("unrecognised tensor dtype %r" % (d,))


def _tensor(rec, what):
    """(dtype name, numpy array) of a Param / TensorData / DataSerialize record."""
    if isinstance(rec, dict) and "param" in rec:
        rec = rec["param"]
    if not isinstance(rec, dict) or "shape" not in rec:
        raise MpkError("%s: not a tensor record" % what)
    shape = tuple(int(s) for s in rec["shape"])
    n = int(np.prod(shape)) if shape else 1
    if "bytes" in rec:
        dt = _dtype_name(rec.get("dtype", "F32"))
        if dt not in _FLOAT_NP:
            raise MpkError("%s: non-float tensor dtype %s" % (what, dt))
        raw = rec["bytes"]
        if isinstance(raw, (list, tuple)):
            raw = bytes(raw)
        if not isinstance(raw, (bytes, bytearray)):
            raise MpkError("%s: tensor bytes of type %s" % (what, type(raw).__name__))
        npdt = np.dtype(_FLOAT_NP[dt])
        if len(raw) != n * npdt.itemsize:
            raise MpkError("%s: %d bytes for shape %s of %s" % (what, len(raw), shape, dt))
        return dt, np.frombuffer(raw, npdt).reshape(shape)
    if "value" in rec:
        v = np.asarray(rec["value"], np.float64)
        if v.size != n:
            raise MpkError("%s: %d values for shape %s" % (what, v.size, shape))
        return "F64", v.reshape(shape)
    raise MpkError("%s: tensor record without bytes or value" % what)


def _to_bf16(dt, arr):
    if dt == "BF16":
        return np.ascontiguousarray(arr, np.uint16)
    return f32_to_bf16(np.asarray(arr, np.float32))


def _field(rec, name, what):
    if not isinstance(rec, dict) or name not in rec:
        raise MpkError("%s: missing field %s" % (what, name))
    return rec[name]


def read_mpk(path):
    """The decoded BurnRecord map (metadata and item) of an .mpk file."""
    _need_msgpack()
    with open(path, "rb") as f:
        data = f.read()
    try:
        rec = msgpack.unpackb(data, raw=False, strict_map_key=False)
    except (ValueError, msgpack.exceptions.ExtraData) as e:
        raise MpkError("%s: not a MessagePack record (%s)" % (path, e)) from None
    if not isinstance(rec, dict) or "item" not in rec:
        raise MpkError("%s: no BurnRecord item" % path)
    return rec


def load_entropy_weights_mpk(path):
    """The weights of an .mpk entropy-model record in the model handle's layout,
    as load_entropy_weights returns them for safetensors: {tok_embeddings [V, D],
    attention_norm / ffn_norm [L, D], wq/wk/wv/wo [L, D, D], w1/w3 [L, D, F],
    w2 [L, F, D], norm [D], output [D, V]} as bf16 bits (f32 values rounded to
    nearest even), plus {"dim", "n_layers", "hidden", "vocab"}."""
    item = read_mpk(path)["item"]
    emb_dt, emb = _tensor(_field(_field(item, "tok_embeddings", path), "weight", path),
                          "tok_embeddings.weight")
    if emb.ndim != 2:
        raise MpkError("%s: tok_embeddings.weight has shape %s" % (path, emb.shape))
    V, D = emb.shape
    layers = _field(item, "layers", path)
    if not isinstance(layers, (list, tuple)) or not layers:
        raise MpkError("%s: no transformer layers" % path)

    def linear(rec, name, d_in, d_out):
        w = _field(rec, name, path)
        b = w.get("bias") if isinstance(w, dict) else None
        if b is not None:
            _, bv = _tensor(b, name + ".bias")
            if np.any(np.asarray(bv, np.float64) != 0):
                raise MpkError("%s: %s has a bias; the entropy model's linears have none"
                               % (path, name))
        dt, a = _tensor(_field(w, "weight", path), name + ".weight")
        if a.shape != (d_in, d_out):
            raise MpkError("%s: %s.weight has shape %s, expected %s"
                           % (path, name, a.shape, (d_in, d_out)))
        return _to_bf16(dt, a)

    def norm(rec, name):
        dt, a = _tensor(_field(_field(rec, name, path), "weight", path), name + ".weight")
        if a.shape != (D,):
            raise MpkError("%s: %s.weight has shape %s, expected %s" % (path, name, a.shape, (D,)))
        return _to_bf16(dt, a)

    ff0 = _field(_field(layers[0], "feed_forward", path), "w1", path)
    _, w1_0 = _tensor(_field(ff0, "weight", path), "layers.0.feed_forward.w1.weight")
    if w1_0.ndim != 2:
        raise MpkError("%s: layers.0.feed_forward.w1.weight has shape %s" % (path, w1_0.shape))
    F = w1_0.shape[1]
    per = {k: [] for k in ("attention_norm", "ffn_norm", "wq", "wk", "wv", "wo", "w1", "w2", "w3")}
    for blk in layers:
        per["attention_norm"].append(norm(blk, "attention_norm"))
        per["ffn_norm"].append(norm(blk, "ffn_norm"))
        att = _field(blk, "attention", path)
        for n in ("wq", "wk", "wv", "wo"):
            per[n].append(linear(att, n, D, D))
        ff = _field(blk, "feed_forward", path)
        per["w1"].append(linear(ff, "w1", D, F))
        per["w3"].append(linear(ff, "w3", D, F))
        per["w2"].append(linear(ff, "w2", F, D))
    w = {"tok_embeddings": _to_bf16(emb_dt, emb)}
    for k, v in per.items():
        w[k] = np.ascontiguousarray(np.stack(v))
    w["norm"] = norm(item, "norm")
    w["output"] = np.ascontiguousarray(linear(item, "output", D, V))
    return w, {"dim": D, "n_layers": len(layers), "hidden": F, "vocab": V}


def _param(arr_f32, pid):
    a = np.ascontiguousarray(arr_f32, "<f4")
    return {"id": "%016x" % pid, "param": {"bytes": a.tobytes(), "shape": list(a.shape),
                                            "dtype": "F32"}}


def save_entropy_weights_mpk(path, weights):
    """Inverse of load_entropy_weights_mpk: the record NamedMpkFileRecorder<
    FullPrecisionSettings> writes for an LMTransformer (f32 tensors, Burn's
    [d_input, d_output] linear layout, constants as unit records)."""
    _need_msgpack()
    f32 = lambda bits: (np.asarray(bits, np.uint32) << 16).view(np.float32)
    pid = iter(range(1, 1 << 30))
    lin = lambda a: {"weight": _param(f32(a), next(pid)), "bias": None}
    nrm = lambda a: {"weight": _param(f32(a), next(pid)), "epsilon": None}
    L = weights["wq"].shape[0]
    layers = []
    for i in range(L):
        layers.append({
            "attention_norm": nrm(weights["attention_norm"][i]),
            "attention": {"wq": lin(weights["wq"][i]), "wk": lin(weights["wk"][i]),
                          "wv": lin(weights["wv"][i]), "wo": lin(weights["wo"][i]),
                          "n_heads": None, "n_kv_heads": None, "head_dim": None},
            "ffn_norm": nrm(weights["ffn_norm"][i]),
            "feed_forward": {"w1": lin(weights["w1"][i]), "w2": lin(weights["w2"][i]),
                             "w3": lin(weights["w3"][i])},
        })
    item = {"tok_embeddings": {"weight": _param(f32(weights["tok_embeddings"]), next(pid))},
            "layers": layers, "norm": nrm(weights["norm"]), "output": lin(weights["output"]),
            "max_seqlen": None, "head_dim": None, "rope_theta": None}
    rec = {"metadata": {"float": "f32", "int": "i32", "format": RECORDER,
                        "version": BURN_VERSION, "settings": "FullPrecisionSettings"},
           "item": item}
    with open(path, "wb") as f:
        f.write(msgpack.packb(rec, use_bin_type=True))
