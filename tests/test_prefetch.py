"""Background prefetchers of the ingest path (prefetch.rs:39-149), CPU only:
the reference's own DocumentPrefetcher tests (prefetch.rs:151-200) plus the
tokenizing SegmentPrefetcher, checked against tokenizing everything at once."""
import threading

import numpy as np
import pytest

from blt_burn_amd import prefetch as P
from blt_burn_amd import synth
from blt_burn_amd import tokenizer as tk


def test_prefetcher_basic():
    docs = [("doc1", b"hello"), ("doc2", b"world"), ("doc3", b"test")]
    pf = P.DocumentPrefetcher(iter(docs), 2)
    d1 = pf.recv()
    assert d1.id == "doc1" and d1.bytes == b"hello" and d1.original_len == 5
    assert pf.recv().id == "doc2"
    assert pf.recv().id == "doc3"
    assert pf.recv() is None and pf.recv() is None
    assert pf.docs_prefetched == 3 and pf.buffer_size == 2


def test_prefetcher_empty():
    assert P.DocumentPrefetcher(iter([]), 4).recv() is None


def test_prefetcher_as_iterator():
    got = list(P.DocumentPrefetcher(iter([("a", bytes([1, 2, 3])), ("b", bytes([4, 5, 6]))]), 2))
    assert [d.id for d in got] == ["a", "b"]


def test_prefetcher_backpressure_and_close():
    # the producer never runs more than buffer_size (+1 in hand) ahead, and
    # close() stops it while it waits for room
    produced = []
    gate = threading.Event()

    def gen():
        for i in range(1000):
            produced.append(i)
            yield ("d%d" % i, b"x")
    pf = P.DocumentPrefetcher(gen(), 3)
    assert pf.recv().id == "d0"
    gate.wait(0.3)
    assert len(produced) <= 1 + 3 + 1
    pf.close()
    assert len(produced) < 1000


def test_prefetcher_reraises_producer_error():
    def gen():
        yield ("a", b"1")
        raise ValueError("reader failed")
    pf = P.DocumentPrefetcher(gen(), 2)
    assert pf.recv().id == "a"
    with pytest.raises(ValueError, match="reader failed"):
        pf.recv()


@pytest.mark.parametrize("seg_bytes", [1, 5000, 1 << 30])
def test_segment_prefetcher_matches_one_tokenization(seg_bytes):
    data, off = synth.documents(synth.config_seed(5) + 3, 40 * 1024, max_len=8000)
    docs = [("id%d" % d, data[off[d]:off[d + 1]].tobytes()) for d in range(off.size - 1)]
    docs.insert(3, ("empty", b""))
    segs = list(P.SegmentPrefetcher(iter(docs), seg_bytes, add_bos=True, add_eos=False))
    assert [s for seg in segs for s in seg.sample_ids] == [d[0] for d in docs]
    for seg in segs[:-1]:
        assert seg.n_bytes >= seg_bytes
    if seg_bytes == 1:  # every non-empty document closes its own segment
        assert all(len(seg.docs) == 1 or seg.docs[0] == b"" for seg in segs)
    i = 0
    for seg in segs:
        for d, raw in enumerate(seg.docs):
            ref = tk.tokenize_bytes(raw, True, False)
            got = seg.tokens[seg.token_offsets[d]:seg.token_offsets[d + 1]]
            np.testing.assert_array_equal(got, ref)
            assert raw == docs[i][1]
            i += 1
    assert i == len(docs)


def test_segment_prefetcher_bare_bytes_and_close_early():
    pf = P.SegmentPrefetcher((bytes([65 + (i % 26)]) * 10 for i in range(100)), 30, buffer_size=1)
    first = next(pf)
    assert first.sample_ids == ["0", "1", "2"] and first.tokens.size == 30
    pf.close()
