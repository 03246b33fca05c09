"""safetensors files of the entropy-patching path: model weights in, per-document
results out.

* load_entropy_weights / LMTransformer.from_safetensors: a local
  facebook/blt-entropy checkpoint (model_loader.rs:103-145, main.rs:141-155,
  bin/peek_weights.rs).  The checkpoint holds PyTorch nn.Linear weights
  [out, in]; Burn's SafetensorsFileRecorder (PyTorch adapter) stores Linear
  weights as [in, out], which is the layout the model handle takes.  The FFN
  width comes from the file (2048 for the real weights, whatever the config
  rule gives, model.rs:468-473).
* save_blt_example: the per-document file of save_blt_safetensors
  (huggingface_loader.rs:144-247): tokens, embeddings, prominence, entropies,
  coherence_scores, patch_indices, patch_lengths, mask, with the sample_id /
  embedding_dim / metadata_file metadata.

The container format (8-byte little-endian header length, JSON header with
dtype / shape / data_offsets per tensor, then the raw little-endian data) is
read and written here directly, so bf16 tensors stay as their 16-bit patterns
and nothing in a file is ever executed.
"""
import json
import struct

import numpy as np

from .synth import f32_to_bf16

_NP = {"F32": np.float32, "F16": np.float16, "F64": np.float64, "I32": np.int32,
       "I64": np.int64, "I16": np.int16, "I8": np.int8, "U8": np.uint8, "U16": np.uint16,
       "BOOL": np.bool_, "BF16": np.uint16}  # BF16: raw bit patterns
_DT = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.float64): "F64",
       np.dtype(np.int32): "I32", np.dtype(np.int64): "I64", np.dtype(np.int16): "I16",
       np.dtype(np.int8): "I8", np.dtype(np.uint8): "U8", np.dtype(np.bool_): "BOOL"}


class SafetensorsError(ValueError):
    pass


def read_safetensors(path):
    """{name: (dtype string, numpy array)} and the metadata dict.  BF16 arrays
    come back as uint16 bit patterns."""
    with open(path, "rb") as f:
        raw = f.read()
    if len(raw) < 8:
        raise SafetensorsError("%s: not a safetensors file" % path)
    (n,) = struct.unpack("<Q", raw[:8])
    if n > len(raw) - 8:
        raise SafetensorsError("%s: header length %d exceeds the file" % (path, n))
    header = json.loads(raw[8:8 + n].decode("utf-8"))
    data = memoryview(raw)[8 + n:]
    meta = header.pop("__metadata__", None) or {}
    out = {}
    for name, d in header.items():
        dt = d["dtype"]
        if dt not in _NP:
            raise SafetensorsError("%s: tensor %s has unsupported dtype %s" % (path, name, dt))
        a, b = d["data_offsets"]
        shape = tuple(int(s) for s in d["shape"])
        arr = np.frombuffer(data[a:b], dtype=_NP[dt])
        if arr.size != int(np.prod(shape, dtype=np.int64)):
            raise SafetensorsError("%s: tensor %s size does not match its shape" % (path, name))
        out[name] = (dt, arr.reshape(shape).copy())
    return out, meta


def write_safetensors(path, tensors, metadata=None):
    """tensors: {name: numpy array} or {name: (dtype string, array)} (use
    ("BF16", uint16 bits) for bf16).  Tensors are laid out in name order."""
    items = []
    for name in sorted(tensors):
        v = tensors[name]
        if isinstance(v, tuple):
            dt, arr = v
        else:
            arr = np.asarray(v)
            dt = _DT.get(arr.dtype)
            if dt is None:
                raise SafetensorsError("tensor %s: unsupported dtype %s" % (name, arr.dtype))
        arr = np.ascontiguousarray(arr, dtype=_NP[dt])
        items.append((name, dt, arr))
    header, off = {}, 0
    for name, dt, arr in items:
        header[name] = {"dtype": dt, "shape": list(arr.shape),
                        "data_offsets": [off, off + arr.nbytes]}
        off += arr.nbytes
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    h = json.dumps(header, separators=(",", ":")).encode("utf-8")
    h += b" " * (-len(h) % 8)  # data section starts 8-byte aligned
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for _, _, arr in items:
            f.write(arr.tobytes())


def _to_bf16(dt, arr):
    if dt == "BF16":
        return arr.astype(np.uint16)
    if dt in ("F32", "F16", "F64"):
        return f32_to_bf16(arr.astype(np.float32))
    raise SafetensorsError("weight tensor has non-float dtype %s" % dt)


def load_entropy_weights(path, n_layers=None):
    """Weights of a facebook/blt-entropy style checkpoint in the model handle's
    layout: {tok_embeddings [V, D], attention_norm [L, D], ffn_norm [L, D],
    wq/wk/wv/wo [L, D, D], w1/w3 [L, D, F], w2 [L, F, D], norm [D],
    output [D, V]} as bf16 bits, plus {"dim", "n_layers", "hidden", "vocab"}.
    A common name prefix (e.g. "model.") is tolerated."""
    t, _ = read_safetensors(path)
    key = "tok_embeddings.weight"
    prefix = ""
    if key not in t:
        cands = [n[:-len(key)] for n in t if n.endswith("." + key)]
        if len(cands) != 1:
            raise SafetensorsError("%s: no tok_embeddings.weight tensor" % path)
        prefix = cands[0]

    def get(name):
        n = prefix + name
        if n not in t:
            raise SafetensorsError("%s: missing tensor %s" % (path, n))
        return t[n]

    dt, emb = get("tok_embeddings.weight")
    V, D = emb.shape
    L = n_layers
    if L is None:
        L = 0
        while (prefix + "layers.%d.attention.wq.weight" % L) in t:
            L += 1
    if L == 0:
        raise SafetensorsError("%s: no transformer layers" % path)
    F = get("layers.0.feed_forward.w1.weight")[1].shape[0]

    def linear(name, out_dim, in_dim):
        d, a = get(name)
        if a.shape != (out_dim, in_dim):
            raise SafetensorsError("%s: %s has shape %s, expected %s"
                                   % (path, name, a.shape, (out_dim, in_dim)))
        return _to_bf16(d, a).T  # PyTorch [out, in] -> Burn [in, out]

    def vec(name, n):
        d, a = get(name)
        if a.shape != (n,):
            raise SafetensorsError("%s: %s has shape %s, expected %s" % (path, name, a.shape, (n,)))
        return _to_bf16(d, a)

    w = {"tok_embeddings": _to_bf16(dt, emb)}
    per = {k: [] for k in ("attention_norm", "ffn_norm", "wq", "wk", "wv", "wo", "w1", "w2", "w3")}
    for i in range(L):
        p = "layers.%d." % i
        per["attention_norm"].append(vec(p + "attention_norm.weight", D))
        per["ffn_norm"].append(vec(p + "ffn_norm.weight", D))
        for n in ("wq", "wk", "wv", "wo"):
            per[n].append(linear(p + "attention.%s.weight" % n, D, D))
        per["w1"].append(linear(p + "feed_forward.w1.weight", F, D))
        per["w3"].append(linear(p + "feed_forward.w3.weight", F, D))
        per["w2"].append(linear(p + "feed_forward.w2.weight", D, F))
    for k, v in per.items():
        w[k] = np.ascontiguousarray(np.stack(v))
    w["norm"] = vec("norm.weight", D)
    w["output"] = np.ascontiguousarray(linear("output.weight", V, D))
    return w, {"dim": D, "n_layers": L, "hidden": F, "vocab": V}


def save_entropy_weights(path, weights, metadata=None):
    """Inverse of load_entropy_weights: a PyTorch-layout bf16 checkpoint with
    facebook/blt-entropy tensor names."""
    L = weights["wq"].shape[0]
    out = {"tok_embeddings.weight": ("BF16", weights["tok_embeddings"]),
           "norm.weight": ("BF16", weights["norm"]),
           "output.weight": ("BF16", np.ascontiguousarray(weights["output"].T))}
    for i in range(L):
        p = "layers.%d." % i
        out[p + "attention_norm.weight"] = ("BF16", weights["attention_norm"][i])
        out[p + "ffn_norm.weight"] = ("BF16", weights["ffn_norm"][i])
        for n in ("wq", "wk", "wv", "wo"):
            out[p + "attention.%s.weight" % n] = ("BF16", np.ascontiguousarray(weights[n][i].T))
        for n in ("w1", "w2", "w3"):
            out[p + "feed_forward.%s.weight" % n] = ("BF16",
                                                     np.ascontiguousarray(weights[n][i].T))
    write_safetensors(path, out, metadata)


def save_blt_example(path, example, task_id):
    """save_blt_safetensors (huggingface_loader.rs:144-247) for one
    BltExampleWithEmbeddings: nothing is written for an empty document."""
    core = example.core
    n = int(len(core.tokens))
    if n == 0:
        return False
    dim = int(example.embedding_dim)
    tensors = {
        "tokens": np.asarray(core.tokens, np.int32).reshape(1, n),
        "embeddings": np.asarray(example.pre_norm_embeddings, np.float32).reshape(1, n, dim),
        "prominence": np.asarray(example.prominence, np.float32).reshape(1, n),
        "entropies": np.asarray(core.entropies, np.float32).reshape(1, n),
        "coherence_scores": np.asarray(example.coherence_scores, np.float32).reshape(1, n),
        "patch_indices": np.asarray(example.patch_indices, np.int32).reshape(-1),
        "patch_lengths": np.asarray(core.patch_lengths, np.int32).reshape(-1),
        "mask": np.asarray(core.mask, np.int32).reshape(1, n),
    }
    write_safetensors(path, tensors, {"sample_id": task_id, "embedding_dim": dim,
                                      "metadata_file": "%s.hypergraph.db" % task_id})
    return True

