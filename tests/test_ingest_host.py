"""Host half of the ingest path: the byte tokenizer (blt_tokenize_bytes) and the
chunk planner (blt_ingest_plan_chunks).  CPU only; these entry points never
touch the GPU."""
import json
import os

import numpy as np
import pytest

import oracle
from blt_burn_amd import BltError, synth
from blt_burn_amd import ingest as I
from blt_burn_amd import tokenizer as tk

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))


# ---- tokenizer ----------------------------------------------------------------

@pytest.mark.parametrize("case", KAT["tokens"], ids=lambda c: c["text"])
def test_tokenizer_kat(case):
    # tests/test_blt_core.rs:38-60
    assert tk.BltTokenizer().encode(case["text"]) == case["tokens"]
    assert I.tokens_to_text(case["tokens"]) == case["text"]
    assert tk.BltTokenizer().decode(case["tokens"]) == case["text"]


def test_tokenizer_constants():
    # tokenizer.rs:4-10
    assert (tk.BOE_ID, tk.BOS_ID, tk.EOS_ID, tk.BPE_ID, tk.OFFSET) == (0, 1, 2, 3, 4)


def test_tokenizer_bos_eos():
    assert tk.BltTokenizer(True, True).encode("AB") == [1, 69, 70, 2]
    assert tk.BltTokenizer(True, False).encode("") == [1]
    assert tk.BltTokenizer(False, True).encode("") == [2]
    assert tk.tokenize_bytes(b"").size == 0


def _lossy_ref(data):
    # Python's UTF-8 decoder with errors="replace" substitutes one U+FFFD per
    # maximal ill-formed subpart, the Unicode-recommended practice that
    # String::from_utf8_lossy also follows: an independent implementation.
    return [b + 4 for b in data.decode("utf-8", errors="replace").encode("utf-8")]


EDGE = [b"\x80", b"\xff", b"\xc0\xaf", b"\xc2", b"\xc2A", b"\xe0\x80\x80", b"\xe0\xa0",
        b"\xe0\xa0\x80", b"\xed\xa0\x80", b"\xed\x9f\xbf", b"\xef\xbf\xbd", b"\xf0\x80\x80\x80",
        b"\xf0\x90\x80", b"\xf0\x90\x80\x80", b"\xf4\x8f\xbf\xbf", b"\xf4\x90\x80\x80",
        b"\xf5\x80", b"\xe1\x80\xe1\x80\x80", "héllo wörld €𝄞".encode(), b"a\xf1\x80\x80"]


@pytest.mark.parametrize("data", EDGE, ids=lambda d: d.hex())
def test_tokenizer_lossy_edges(data):
    assert tk.tokenize_bytes(data).tolist() == _lossy_ref(data)


def test_tokenizer_lossy_random():
    rng = np.random.default_rng(7)
    for n in (1, 2, 3, 7, 64, 1000, 20000):
        for _ in range(5):
            data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
            assert tk.tokenize_bytes(data).tolist() == _lossy_ref(data)
    # bytes biased toward lead / continuation bytes: more multi-byte shapes
    for _ in range(50):
        data = rng.choice(np.array([0x41, 0x80, 0x9f, 0xa0, 0xbf, 0xc2, 0xdf, 0xe0, 0xed, 0xef,
                                    0xf0, 0xf4, 0xf5], np.uint8), 200).tobytes()
        assert tk.tokenize_bytes(data).tolist() == _lossy_ref(data)


def test_tokenizer_synthetic_corpus():
    # the config-4/5 content: printable Zipf bytes plus 5% uniform bytes
    toks = synth.tokens(1, 4096, 11).reshape(-1)
    data = (toks - 4).astype(np.uint8).tobytes()
    out = tk.tokenize_bytes(data)
    assert out.tolist() == _lossy_ref(data)
    assert out.size >= len(data)


# ---- chunk planner --------------------------------------------------------------

def test_plan_chunks_hand_case():
    # BltConfig defaults (1024 / 512) on a 2000-token document, worked by hand
    # from blt_core.rs:300-356
    assert I.plan_chunks(2000, 1024, 512) == [(0, 512, 0), (0, 1024, 512), (512, 1024, 512),
                                              (1024, 976, 512)]
    assert I.plan_chunks(100, 1024, 512) == [(0, 100, 0)]
    assert I.plan_chunks(0, 1024, 512) == []
    assert I.plan_chunks(8192, 8192, 512) == [(0, 7680, 0), (7168, 1024, 512)]


@pytest.mark.parametrize("chunk,overlap", [(1024, 512), (8192, 512), (64, 16), (5, 2), (7, 0),
                                           (1, 0)])
def test_plan_chunks_matches_reference_loop(chunk, overlap):
    for L in list(range(0, 3 * chunk + 3)) + [10 * chunk + 1, 31 * chunk + 7]:
        ref = oracle.chunk_plan(L, chunk, overlap)
        got = I.plan_chunks(L, chunk, overlap)
        assert [(s, s + n, k) for s, n, k in got] == ref
        # the kept outputs tile [0, L) once, in order
        kept = [t for s, n, k in got for t in range(s + k, s + n)]
        assert kept == list(range(L))
        assert all(n <= chunk for _, n, _ in got)


def test_plan_chunks_rejects_large_overlap():
    with pytest.raises(BltError):
        I.plan_chunks(100, 1024, 513)
    with pytest.raises(BltError):
        I.plan_chunks(100, 0, 0)


def test_tokenize_documents_matches_per_document():
    data, off = synth.documents(synth.config_seed(5), 200_000)
    toks, toff = tk.tokenize_documents(data, off, add_bos=True, add_eos=False)
    assert toff.size == off.size and toff[0] == 0
    raw = data.tobytes()
    for d in range(off.size - 1):
        one = tk.tokenize_bytes(raw[off[d]:off[d + 1]], add_bos=True)
        np.testing.assert_array_equal(toks[toff[d]:toff[d + 1]], one)
    # a truncated sequence at a document's end does not join the next document
    t2, o2 = tk.tokenize_documents(b"\xe2\x82\xac", np.array([0, 2, 3]))
    assert t2.tolist() == [0xEF + 4, 0xBF + 4, 0xBD + 4, 0xEF + 4, 0xBF + 4, 0xBD + 4]
    assert o2.tolist() == [0, 3, 6]
