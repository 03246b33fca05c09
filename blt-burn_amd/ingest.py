"""Document ingest of the entropy-patching path (blt_core.rs), on one GPU.

Mirrors the reference's BltConfig, BltExample, BltExampleWithEmbeddings,
process_bytes and process_bytes_with_embeddings (blt_core.rs:19-228), and
adds StreamingIngest, which runs many documents through the native driver
(blt_ingest_* in libblt_hip.so): chunks of every document are packed into
[rows, row_len] batches as independent attention/RoPE segments, with pinned
double-buffered uploads and downloads around the packed forward, the stitch
of overlapping chunks and the per-document boundary pass on the device.
"""
import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from ._lib import PATCH_GLOBAL, PATCH_MONOTONIC, BltError, IngestConfig, IngestStats, check
from .tokenizer import OFFSET, tokenize_bytes


@dataclass
class BltConfig:
    """blt_core.rs:53-81 (defaults included)."""
    threshold: float = 1.335
    monotonicity: bool = True
    max_seq_len: int = 1024
    chunk_overlap: int = 512
    add_bos: bool = False
    add_eos: bool = False


@dataclass
class BltExample:
    """blt_core.rs:19-34."""
    sample_id: str
    text: Optional[str]
    tokens: np.ndarray         # int32 [n]
    entropies: np.ndarray      # f32 [n]
    patch_lengths: np.ndarray  # int32 [patches]
    mask: np.ndarray           # bool [n]


@dataclass
class BltExampleWithEmbeddings:
    """blt_core.rs:36-51."""
    core: BltExample
    pre_norm_embeddings: np.ndarray  # f32 [n * dim] (flattened, as the reference)
    embedding_dim: int
    prominence: np.ndarray           # f32 [n], pre-norm L2 norms
    coherence_scores: np.ndarray     # f32 [n], prominence^2 / (entropy + 1e-6)
    patch_indices: np.ndarray        # int32 [patches]


def plan_chunks(doc_len, chunk_len, overlap):
    """[(start, len, skip)] of compute_all_signals_chunked's loop (blt_core.rs:300-356)."""
    cap = max(1, doc_len)
    starts = np.empty(cap, np.int64)
    lens = np.empty(cap, np.int32)
    skips = np.empty(cap, np.int32)
    n = _lib.lib().blt_ingest_plan_chunks(doc_len, chunk_len, overlap, starts.ctypes.data,
                                          lens.ctypes.data, skips.ctypes.data, cap)
    check(n if n < 0 else 0, "blt_ingest_plan_chunks")
    return [(int(starts[i]), int(lens[i]), int(skips[i])) for i in range(n)]


@dataclass
class IngestResult:
    """Outputs of StreamingIngest.run, indexed like the concatenated tokens."""
    offsets: np.ndarray       # int64 [n_docs + 1]
    entropies: np.ndarray     # f32 [total]
    norms: np.ndarray         # f32 [total]
    coherence: np.ndarray     # f32 [total]
    starts: np.ndarray        # int32 [total]: doc d's patch starts at offsets[d] .. + counts[d]
    lengths: np.ndarray       # int32 [total]
    counts: np.ndarray        # int32 [n_docs]
    embeddings: Optional[np.ndarray] = None  # f32 [total, dim]
    # per-patch means (run(..., patch_means=True)), laid out like starts
    patch_entropy: Optional[np.ndarray] = None
    patch_prominence: Optional[np.ndarray] = None
    patch_coherence: Optional[np.ndarray] = None

    def doc(self, d):
        """(entropies, norms, coherence, starts, lengths[, embeddings]) of document d."""
        a, b = int(self.offsets[d]), int(self.offsets[d + 1])
        n = int(self.counts[d])
        out = [self.entropies[a:b], self.norms[a:b], self.coherence[a:b],
               self.starts[a:a + n], self.lengths[a:a + n]]
        if self.embeddings is not None:
            out.append(self.embeddings[a:b])
        return tuple(out)

    def patches(self, d):
        """Document d's patches as the reference's PatchData fields
        (pipeline.rs:47-60): (start offsets, lengths, mean entropy, mean
        prominence, mean coherence); the means need run(..., patch_means=True)."""
        a, n = int(self.offsets[d]), int(self.counts[d])
        if self.patch_entropy is None:
            raise BltError("per-patch means were not computed (run with patch_means=True)")
        return (self.starts[a:a + n], self.lengths[a:a + n], self.patch_entropy[a:a + n],
                self.patch_prominence[a:a + n], self.patch_coherence[a:a + n])


class StreamingIngest:
    """Native ingest driver over one LMTransformer.

    rows x row_len is one packed batch (it must fit the model's max_tokens);
    chunk_len / overlap / threshold come from `config` (BltConfig), the
    boundary rule from `mode` (the reference's process_bytes always applies
    the monotonic rule, blt_core.rs:118-119, 185-186).  Documents may be of any
    length: one whose chunks do not fit a batch spans several; such a document
    is stitched on the device in `long_arena_tokens` of room (0: 2^22, negative:
    none, every such document then gathered on the host)."""

    def __init__(self, model, config=None, rows=None, row_len=None, mode=PATCH_MONOTONIC,
                 with_embeddings=False, long_arena_tokens=0):
        self.model = model
        self.config = config or BltConfig()
        self.row_len = row_len or max(self.config.max_seq_len,
                                      min(8192, model.cfg.max_seqlen))
        self.rows = rows or max(1, model.max_tokens // self.row_len)
        self.with_embeddings = bool(with_embeddings)
        self.mode = mode
        c = IngestConfig(self.rows, self.row_len, self.config.max_seq_len,
                         self.config.chunk_overlap, float(self.config.threshold), mode,
                         int(self.with_embeddings), int(long_arena_tokens))
        h = ctypes.c_void_p()
        check(_lib.lib().blt_ingest_create(model._h, ctypes.byref(c), ctypes.byref(h)),
              "blt_ingest_create")
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        # at interpreter exit the module globals may already be gone
        if h is not None and h.value and _lib is not None and _lib._lib is not None:
            _lib.lib().blt_ingest_destroy(h)
            self._h = None

    def run(self, tokens, offsets, patch_means=False):
        """tokens int32 [total] (host), offsets int64 [n_docs + 1] -> IngestResult
        (with the per-patch means of every document when patch_means)."""
        tok = np.ascontiguousarray(tokens, dtype=np.int32)
        off = np.ascontiguousarray(offsets, dtype=np.int64)
        if off.ndim != 1 or off.size < 1 or off[0] != 0 or off[-1] != tok.size:
            raise BltError("offsets must run from 0 to len(tokens)")
        nd = off.size - 1
        total = tok.size
        res = IngestResult(
            offsets=off, entropies=np.zeros(total, np.float32), norms=np.zeros(total, np.float32),
            coherence=np.zeros(total, np.float32), starts=np.zeros(total, np.int32),
            lengths=np.zeros(total, np.int32), counts=np.zeros(nd, np.int32),
            embeddings=(np.zeros((total, self.model.cfg.dim), np.float32)
                        if self.with_embeddings else None))
        if patch_means:
            res.patch_entropy = np.zeros(total, np.float32)
            res.patch_prominence = np.zeros(total, np.float32)
            res.patch_coherence = np.zeros(total, np.float32)
        p = lambda a: a.ctypes.data if a is not None and a.size else None  # noqa: E731
        check(_lib.lib().blt_ingest_run_patch_means(
            self._h, p(tok), off.ctypes.data, nd, p(res.entropies), p(res.norms),
            p(res.coherence), p(res.embeddings), p(res.starts), p(res.lengths), p(res.counts),
            p(res.patch_entropy), p(res.patch_prominence), p(res.patch_coherence)),
            "blt_ingest_run")
        return res

    def last_stats(self):
        """Counts of the last run(): dict(batches, documents, tokens, tokens_computed,
        row_tokens)."""
        st = IngestStats()
        check(_lib.lib().blt_ingest_last_stats(self._h, ctypes.byref(st)), "ingest_last_stats")
        return {n: int(getattr(st, n)) for n, _ in IngestStats._fields_}

    def stream(self, docs, segment_bytes=64 << 20, buffer_size=2, patch_means=False):
        """Run an iterable of (sample_id, bytes) documents (or bare bytes) in
        segments of about segment_bytes: a background thread reads and
        tokenizes segment i + 1 (the DocumentPrefetcher role, prefetch.rs:39-149)
        while segment i runs on the GPU.  Yields (sample_ids, tokens, IngestResult)
        per segment, results indexed like the segment's concatenated tokens."""
        from .prefetch import SegmentPrefetcher
        pf = SegmentPrefetcher(docs, segment_bytes, self.config.add_bos, self.config.add_eos,
                               buffer_size)
        try:
            for seg in pf:
                yield seg.sample_ids, seg.tokens, self.run(seg.tokens, seg.token_offsets,
                                                           patch_means=patch_means)
        finally:
            pf.close()

    def process(self, docs, sample_ids=None):
        """bytes documents -> [BltExampleWithEmbeddings] (process_bytes_with_embeddings
        for each, blt_core.rs:145-228).  pre_norm_embeddings is empty unless the
        ingest was made with_embeddings."""
        toks = [tokenize_bytes(d, self.config.add_bos, self.config.add_eos) for d in docs]
        off = np.zeros(len(docs) + 1, np.int64)
        off[1:] = np.cumsum([t.size for t in toks])
        flat = np.concatenate(toks) if toks else np.zeros(0, np.int32)
        r = self.run(flat, off)
        out = []
        for d, data in enumerate(docs):
            sid = sample_ids[d] if sample_ids is not None else str(d)
            parts = r.doc(d)
            H, N, C, S, Lp = (np.array(x) for x in parts[:5])
            emb = (np.array(parts[5]).reshape(-1) if self.with_embeddings
                   else np.zeros(0, np.float32))
            core = BltExample(sample_id=sid, text=bytes(data).decode("utf-8", errors="replace"),
                              tokens=toks[d], entropies=H, patch_lengths=Lp,
                              mask=np.ones(toks[d].size, dtype=bool))
            out.append(BltExampleWithEmbeddings(
                core=core, pre_norm_embeddings=emb, embedding_dim=self.model.cfg.dim,
                prominence=N, coherence_scores=C, patch_indices=S))
        return out


def ingest_for(model, config=None, with_embeddings=False, mode=PATCH_MONOTONIC):
    """The StreamingIngest that process_bytes* use for this model and config:
    rows of config.max_seq_len tokens, as many as the model's max_tokens holds,
    made once and kept on the model (its pinned and device buffers are reused
    by every later document)."""
    config = config or BltConfig()
    if config.max_seq_len > model.max_tokens:
        raise BltError("max_seq_len %d exceeds the model's max_tokens %d"
                       % (config.max_seq_len, model.max_tokens))
    key = (float(config.threshold), int(config.max_seq_len), int(config.chunk_overlap),
           bool(config.add_bos), bool(config.add_eos), int(mode), bool(with_embeddings))
    cache = model.__dict__.setdefault("_ingest_cache", {})
    ing = cache.get(key)
    if ing is None:
        ing = StreamingIngest(model, config, rows=max(1, model.max_tokens // config.max_seq_len),
                              row_len=config.max_seq_len, mode=mode,
                              with_embeddings=with_embeddings)
        cache[key] = ing
    return ing


def _process_one(data, sample_id, model, config, with_embeddings):
    # a document of any length: its chunks run in as many packed batches as
    # they need (blt_core.rs:286-370 loops over them one forward at a time)
    return ingest_for(model, config, with_embeddings).process([data], [sample_id])[0]


def process_bytes_with_embeddings(data, sample_id, model, config=None):
    """blt_core.rs:145-228 for one document."""
    return _process_one(data, sample_id, model, config, True)


def process_bytes(data, sample_id, model, config=None):
    """blt_core.rs:86-140 for one document (no embeddings)."""
    return _process_one(data, sample_id, model, config, False).core


def tokens_to_text(tokens):
    """blt_core.rs:373-387."""
    raw = bytes((int(t) - OFFSET) & 0xFF for t in tokens if int(t) >= OFFSET)
    return raw.decode("utf-8", errors="replace")


__all__ = ["BltConfig", "BltExample", "BltExampleWithEmbeddings", "IngestResult",
           "StreamingIngest", "ingest_for", "plan_chunks", "process_bytes",
           "process_bytes_with_embeddings", "tokens_to_text", "PATCH_MONOTONIC", "PATCH_GLOBAL"]
