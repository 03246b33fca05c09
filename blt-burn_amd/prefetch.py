"""Background document prefetching for streaming ingest (prefetch.rs:1-149).

DocumentPrefetcher mirrors the reference's: a thread walks an iterator of
(id, bytes) documents and hands them over through a bounded queue, so reading
the next documents overlaps the GPU work on the current ones (the bound is
the backpressure).  SegmentPrefetcher goes one step further for the packed
ingest driver: its thread also groups the documents into segments of about
`segment_bytes` and tokenizes each segment (blt_tokenize_documents, host C
code that runs without the interpreter lock), so segment i + 1 is read and
tokenized while segment i runs on the GPU.
"""
import queue
import threading
from dataclasses import dataclass
from typing import List

import numpy as np

from .tokenizer import tokenize_documents

__all__ = ["PrefetchedDoc", "DocumentPrefetcher", "Segment", "SegmentPrefetcher"]

_END = object()


@dataclass
class PrefetchedDoc:
    """prefetch.rs:15-23."""
    id: str
    bytes: bytes
    original_len: int


class _Worker:
    """A producer thread feeding a bounded queue; exceptions are re-raised in
    the consumer, close() stops the producer and joins it."""

    def __init__(self, produce, buffer_size):
        if buffer_size < 1:
            raise ValueError("buffer_size must be at least 1")
        self._q = queue.Queue(maxsize=buffer_size)
        self._stop = threading.Event()
        self._done = False
        self._thread = threading.Thread(target=self._main, args=(produce,), daemon=True)
        self._thread.start()

    def _put(self, item):
        while not self._stop.is_set():
            try:
                self._q.put(item, timeout=0.1)
                return True
            except queue.Full:
                continue
        return False

    def _main(self, produce):
        try:
            for item in produce():
                if not self._put(item):
                    return
        except BaseException as e:  # handed to the consumer
            self._put(("__error__", e))
            return
        self._put(_END)

    def get(self):
        """The next item, or _END when the producer is exhausted."""
        if self._done:
            return _END
        item = self._q.get()
        if item is _END:
            self._done = True
            return _END
        if isinstance(item, tuple) and len(item) == 2 and item[0] == "__error__":
            self._done = True
            raise item[1]
        return item

    def close(self):
        self._stop.set()
        while True:  # unblock a producer waiting for room
            try:
                self._q.get_nowait()
            except queue.Empty:
                break
        self._thread.join()
        self._done = True


def _as_doc(i, item):
    if isinstance(item, (bytes, bytearray, memoryview)):
        return str(i), bytes(item)
    sid, data = item
    return str(sid), bytes(data)


class DocumentPrefetcher:
    """DocumentPrefetcher::new(iter, buffer_size) (prefetch.rs:39-91): iter
    yields (id, bytes); recv() returns the next PrefetchedDoc or None at the end."""

    def __init__(self, docs, buffer_size=4):
        self._buffer_size = buffer_size
        self._n = 0

        def produce():
            for i, item in enumerate(docs):
                sid, data = _as_doc(i, item)
                yield PrefetchedDoc(sid, data, len(data))
        self._w = _Worker(produce, buffer_size)

    def recv(self):
        item = self._w.get()
        if item is _END:
            return None
        self._n += 1
        return item

    @property
    def buffer_size(self):
        return self._buffer_size

    @property
    def docs_prefetched(self):
        return self._n

    def __iter__(self):
        return self

    def __next__(self):
        d = self.recv()
        if d is None:
            raise StopIteration
        return d

    def close(self):
        self._w.close()

    def __del__(self):
        w = getattr(self, "_w", None)
        if w is not None:
            w.close()


@dataclass
class Segment:
    """Documents of one segment, tokenized: document d's tokens are
    tokens[token_offsets[d], token_offsets[d + 1])."""
    sample_ids: List[str]
    docs: List[bytes]
    tokens: np.ndarray         # int32 [total]
    token_offsets: np.ndarray  # int64 [n_docs + 1]
    n_bytes: int


class SegmentPrefetcher:
    """Reads (id, bytes) documents (or bare bytes) on a thread, groups them
    into segments of at least segment_bytes (the last may be smaller) and
    tokenizes each (tokenizer.rs on from_utf8_lossy text, with BOS / EOS as
    asked); iterating yields Segment objects, at most buffer_size ahead."""

    def __init__(self, docs, segment_bytes=64 << 20, add_bos=False, add_eos=False,
                 buffer_size=2):
        if segment_bytes < 1:
            raise ValueError("segment_bytes must be at least 1")

        def emit(ids, datas):
            offs = np.zeros(len(datas) + 1, np.int64)
            offs[1:] = np.cumsum([len(x) for x in datas])
            flat = np.frombuffer(b"".join(datas), np.uint8)
            toks, toff = tokenize_documents(flat, offs, add_bos, add_eos)
            return Segment(ids, datas, toks, toff, int(offs[-1]))

        def produce():
            ids, datas, have = [], [], 0
            for i, item in enumerate(docs):
                sid, data = _as_doc(i, item)
                ids.append(sid)
                datas.append(data)
                have += len(data)
                if have >= segment_bytes:
                    yield emit(ids, datas)
                    ids, datas, have = [], [], 0
            if ids:
                yield emit(ids, datas)
        self._w = _Worker(produce, buffer_size)

    def __iter__(self):
        return self

    def __next__(self):
        s = self._w.get()
        if s is _END:
            raise StopIteration
        return s

    def close(self):
        self._w.close()

    def __del__(self):
        w = getattr(self, "_w", None)
        if w is not None:
            w.close()
