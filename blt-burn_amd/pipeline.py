"""Streaming entropy pipeline (pipeline.rs) on one GPU.

Mirrors the reference's CHUNK_SIZE / STRIDE / SAFE_ZONE_END, PatchData,
ProcessingResult, PipelineBuffer and process_document (pipeline.rs:37-324)
over the blt_pipeline_* entry points of libblt_hip.so: every chunk's forward,
the boundary pass over the accumulated entropies and the per-patch means run
on the device, the accumulated entropies / norms stay in device memory.
process_documents is the many-document form: the chunks of all documents run
as packed segments of large forwards and each document's patches come out
exactly as process_document's chunk loop emits them.
"""
import ctypes
import weakref
from dataclasses import dataclass
from typing import List

import numpy as np

from . import _lib
from ._lib import BltError, check
from ._torch import stream_ptr

# pipeline.rs:37-43
CHUNK_SIZE = 4096
STRIDE = 2048
SAFE_ZONE_END = CHUNK_SIZE - STRIDE

# PatchData.embedding is a zero vector of this width (pipeline.rs:213-214)
EMBEDDING_DIM = 768


class PatchData:
    """pipeline.rs:46-60.  embedding is an f32 [768] zero vector of its own, as
    the reference emits it; it is allocated on first access (most callers read
    only the offsets, means and bytes, and a document yields hundreds of patches)."""
    __slots__ = ("start_offset", "length", "_embedding", "prominence", "entropy", "bytes")

    def __init__(self, start_offset, length, embedding=None, prominence=0.0, entropy=0.0,
                 bytes=b""):
        self.start_offset = start_offset
        self.length = length
        self._embedding = embedding
        self.prominence = prominence
        self.entropy = entropy
        self.bytes = bytes

    @property
    def embedding(self) -> np.ndarray:
        if self._embedding is None:
            self._embedding = np.zeros(EMBEDDING_DIM, np.float32)
        return self._embedding

    @embedding.setter
    def embedding(self, value):
        self._embedding = value

    def __eq__(self, other):
        if not isinstance(other, PatchData):
            return NotImplemented
        return (self.start_offset == other.start_offset and self.length == other.length and
                self.prominence == other.prominence and self.entropy == other.entropy and
                self.bytes == other.bytes and
                np.array_equal(self.embedding, other.embedding))

    def __repr__(self):
        return ("PatchData(start_offset=%d, length=%d, prominence=%r, entropy=%r, bytes=%r)"
                % (self.start_offset, self.length, self.prominence, self.entropy, self.bytes))


@dataclass
class ProcessingResult:
    """pipeline.rs:62-71."""
    patches: List[PatchData]
    entropies: np.ndarray  # f32 [n]
    norms: np.ndarray      # f32 [n]


def _ptr(a):
    return a.ctypes.data if a is not None and a.size else None


def _patches(starts, lengths, prom, ent, raw, base=0):
    # raw is one document or chunk window (small): one bytes copy, then slices
    if not isinstance(raw, bytes):
        raw = bytes(raw)
    return [PatchData(a, n, None, p, h, raw[base + a:base + a + n])
            for a, n, p, h in zip(starts.tolist(), lengths.tolist(), prom.tolist(), ent.tolist())]


class PipelineBuffer:
    """pipeline.rs:74-274.  PipelineBuffer(threshold) as PipelineBuffer::new;
    the model is bound on the first process_chunk (the reference passes it
    with every chunk; one buffer always runs one model)."""

    def __init__(self, threshold):
        self.threshold = float(threshold)
        self._h = None
        self._strong = None  # the bound model (None when bound weakly)
        self._wref = None

    @property
    def _model(self):
        return self._wref() if self._wref is not None else None

    def _bind(self, model, weak=False):
        """Bind the model on first use.  A buffer the caller holds keeps its
        model alive; the per-model buffers of process_document /
        process_documents bind weakly (they live on the model, which closes
        them before it frees itself), so no reference cycle holds the model's
        device memory after the caller drops it."""
        if self._h is None:
            if model is None or not hasattr(model, "_h"):
                raise BltError("PipelineBuffer.process_chunk needs the entropy model (an "
                               "LMTransformer) on its first call")
            h = ctypes.c_void_p()
            check(_lib.lib().blt_pipeline_create(model._h, self.threshold, ctypes.byref(h)),
                  "blt_pipeline_create")
            self._h = h
            self._strong = None if weak else model
            self._wref = weakref.ref(model)
        elif model is not None and model is not self._model:
            raise BltError("a PipelineBuffer runs one model; this one is bound to another")

    def close(self):
        """Free the device state (the accumulated signals and staging buffers)."""
        h = getattr(self, "_h", None)
        if h is not None and h.value and _lib is not None and _lib._lib is not None:
            _lib.lib().blt_pipeline_destroy(h)
        self._h = None

    def __del__(self):
        self.close()

    def _stream(self):
        return stream_ptr(self._model.device)

    def process_chunk(self, chunk_bytes, entropy_model, blt_encoder=None, device=None,
                      is_last_chunk=False):
        """pipeline.rs:111-238: runs the chunk, returns the patches it confirms."""
        del blt_encoder, device  # unused by the reference too (pipeline.rs:206)
        self._bind(entropy_model)
        data = np.frombuffer(bytes(chunk_bytes), np.uint8)
        cap = self.accumulated() + data.size
        start = np.empty(max(cap, 1), np.int64)
        length = np.empty(max(cap, 1), np.int64)
        prom = np.empty(max(cap, 1), np.float32)
        ent = np.empty(max(cap, 1), np.float32)
        n = ctypes.c_int64()
        check(_lib.lib().blt_pipeline_process_chunk(
            self._h, _ptr(data), data.size, 1 if is_last_chunk else 0, cap, start.ctypes.data,
            length.ctypes.data, prom.ctypes.data, ent.ctypes.data, ctypes.byref(n),
            self._stream()), "blt_pipeline_process_chunk")
        k = n.value
        if k == 0:
            return []
        lo = int(start[:k].min())
        hi = int((start[:k] + length[:k]).max())
        raw = self._read(lo, hi - lo)[2]
        return _patches(start[:k], length[:k], prom[:k], ent[:k], raw, base=-lo)

    def accumulated(self):
        if self._h is None:
            return 0
        n = ctypes.c_int64()
        check(_lib.lib().blt_pipeline_accumulated(self._h, ctypes.byref(n)),
              "blt_pipeline_accumulated")
        return n.value

    def _read(self, offset, n):
        H = np.empty(n, np.float32)
        N = np.empty(n, np.float32)
        raw = np.empty(n, np.uint8)
        if n:
            check(_lib.lib().blt_pipeline_read(self._h, offset, n, H.ctypes.data, N.ctypes.data,
                                               raw.ctypes.data, self._stream()),
                  "blt_pipeline_read")
        return H, N, raw

    def entropies(self):
        """pipeline.rs:260-263."""
        return self._read(0, self.accumulated())[0]

    def norms(self):
        """pipeline.rs:265-268."""
        return self._read(0, self.accumulated())[1]

    def raw_bytes(self):
        """pipeline.rs:270-273."""
        return self._read(0, self.accumulated())[2].tobytes()


def process_document(data, entropy_model, blt_encoder=None, device=None, threshold=1.335):
    """pipeline.rs:279-324: the chunk loop over one document, one forward per
    chunk through a PipelineBuffer (one kept per model and threshold, reset to
    PipelineBuffer::new's state for every document, so its device and pinned
    buffers are reused)."""
    buf = _buffer_for(entropy_model, threshold)
    check(_lib.lib().blt_pipeline_reset(buf._h), "blt_pipeline_reset")
    data = bytes(data)
    total = len(data)
    patches = []
    pos = 0
    while pos < total:
        chunk_end = min(pos + CHUNK_SIZE, total)
        is_last = chunk_end >= total
        start = max(pos - STRIDE, 0) if pos > 0 else 0
        patches.extend(buf.process_chunk(data[start:chunk_end], entropy_model, blt_encoder,
                                         device, is_last))
        if is_last:
            break
        pos = chunk_end
    H, N, _ = buf._read(0, buf.accumulated())
    return ProcessingResult(patches=patches, entropies=H, norms=N)


def process_documents(docs, entropy_model, threshold=1.335, rows=None, row_len=8192):
    """process_document for many documents at once -> [ProcessingResult].

    The chunks of every document run as independent segments of packed
    [rows, row_len] forwards (rows defaults to what the model's max_tokens
    holds); patches, entropies and norms are those of process_document, up to
    the forward's rounding differences between packed and separate runs."""
    docs = [bytes(d) for d in docs]
    rows = rows or max(1, entropy_model.max_tokens // row_len)
    lens = np.array([len(d) for d in docs], np.int64)
    off = np.zeros(len(docs) + 1, np.int64)
    off[1:] = np.cumsum(lens)
    flat = np.frombuffer(b"".join(docs), np.uint8)
    total = int(off[-1])
    cap = total + STRIDE * len(docs)
    H = np.zeros(max(total, 1), np.float32)
    N = np.zeros(max(total, 1), np.float32)
    start = np.zeros(max(cap, 1), np.int64)
    length = np.zeros(max(cap, 1), np.int64)
    prom = np.zeros(max(cap, 1), np.float32)
    ent = np.zeros(max(cap, 1), np.float32)
    poff = np.zeros(len(docs) + 1, np.int64)
    h = _buffer_for(entropy_model, threshold)._h
    check(_lib.lib().blt_pipeline_process_documents(
        h, _ptr(flat), off.ctypes.data, len(docs), rows, row_len, H.ctypes.data, N.ctypes.data,
        cap, start.ctypes.data, length.ctypes.data, prom.ctypes.data, ent.ctypes.data,
        poff.ctypes.data, stream_ptr(entropy_model.device)), "blt_pipeline_process_documents")
    out = []
    for d in range(len(docs)):
        a, b = int(off[d]), int(off[d + 1])
        p, q = int(poff[d]), int(poff[d + 1])
        out.append(ProcessingResult(
            patches=_patches(start[p:q], length[p:q], prom[p:q], ent[p:q], docs[d]),
            entropies=H[a:b].copy(), norms=N[a:b].copy()))
    return out


def _buffer_for(model, threshold):
    """The PipelineBuffer that process_document and process_documents use for
    this model and threshold, kept on the model (its device, pinned and ingest
    buffers are reused by later calls)."""
    cache = model.__dict__.setdefault("_pipeline_cache", {})
    key = float(threshold)
    buf = cache.get(key)
    if buf is None:
        buf = PipelineBuffer(threshold)
        buf._bind(model, weak=True)
        cache[key] = buf
    return buf


__all__ = ["CHUNK_SIZE", "STRIDE", "SAFE_ZONE_END", "PatchData", "ProcessingResult",
           "PipelineBuffer", "process_document", "process_documents"]
