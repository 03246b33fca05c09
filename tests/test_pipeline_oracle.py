"""The oracle's restatement of the streaming pipeline (pipeline.rs:111-324),
pinned on the CPU: the reference's own constant test (pipeline.rs:330-336),
a hand-worked document at chunk 4 / stride 2, the left-to-right f32 means of
compute_mean_* (pipeline.rs:241-258) on values where the summation order shows,
and the closed form of which patches the chunk loop emits at 4096 / 2048."""
import numpy as np
import pytest

import oracle


def test_pipeline_constants():
    # pipeline.rs:330-336
    from blt_burn_amd import pipeline as P
    assert P.CHUNK_SIZE == 4096 and P.STRIDE == 2048 and P.SAFE_ZONE_END == 2048
    assert P.CHUNK_SIZE - P.STRIDE == P.SAFE_ZONE_END
    import os
    h = open(os.path.join(os.path.dirname(__file__), "..", "include", "blt_hip.h")).read()
    for name, v in (("CHUNK_SIZE", 4096), ("STRIDE", 2048), ("SAFE_ZONE_END", 2048)):
        assert "#define BLT_PIPELINE_%s %d" % (name, v) in h


def test_mean_f32_left_to_right():
    big = np.float32(2 ** 24)
    # 2^24 + 1 rounds back to 2^24 at every step: the sum stays 2^24
    assert oracle.mean_f32(np.array([big, 1, 1, 1, 1], np.float32), 0, 5) == np.float32(big / 5)
    # the other order reaches 2^24 + 4 exactly
    assert oracle.mean_f32(np.array([1, 1, 1, 1, big], np.float32), 0, 5) == \
        np.float32((big + 4) / 5)
    x = np.arange(1, 11, dtype=np.float32)
    assert oracle.mean_f32(x, 3, 100) == np.float32(7.0)   # end clamped to len: 4..10
    assert oracle.mean_f32(x, 12, 100) == 0                 # start clamped to end: empty
    assert oracle.mean_f32(x, 4, 4) == 0


def _table_forward(Htab, Ntab, data):
    """A position-keyed stand-in for the model that also checks the tokens it
    is given are the raw byte values of the chunk (pipeline.rs:123)."""
    def fwd(tokens, start):
        n = tokens.size
        np.testing.assert_array_equal(tokens, np.frombuffer(data[start:start + n], np.uint8))
        return Htab[start:start + n], Ntab[start:start + n]
    return fwd


def test_pipeline_hand_worked_chunk4_stride2():
    # positions:   0  1  2  3  4  5  6  7  8  9
    H = np.array([0, 0, 0, 0, 0, 9, 9, 9, 0, 3], np.float32)
    N = np.arange(1, 11, dtype=np.float32)
    data = bytes(range(10, 20))
    r = oracle.pipeline_process_document(data, _table_forward(H, N, data), 1.0, 4, 2)
    # chunk 0 = [0,4): starts {0,1}, window [0, 2): (0,1), (1, acc 4)
    # chunk 1 = [2,8) keeps [4,8): starts {0,1,5}, window [0, 4): (0,1), (1,5)
    # chunk 2 = [6,10) keeps [8,10), last: starts {0,1,5,9}, window [4, inf): (5,9), (9,10)
    want = [(0, 1, 1.0, 0.0), (1, 3, 3.0, 0.0), (0, 1, 1.0, 0.0), (1, 4, 3.5, 0.0),
            (5, 4, 7.5, 6.75), (9, 1, 10.0, 3.0)]
    got = [(s, n, float(p), float(h)) for s, n, p, h, _ in r["patches"]]
    assert got == want
    assert [b for *_, b in r["patches"]] == [data[s:s + n] for s, n, _, _ in want]
    np.testing.assert_array_equal(r["entropies"], H)
    np.testing.assert_array_equal(r["norms"], N)


def _closed_form(H, thr):
    """Which (start, end) pairs process_document emits at 4096 / 2048, derived
    from the chunk geometry instead of stepping the loop: chunk k >= 1 covers
    [4096k - 2048, 4096k + 4096) and leaves min(4096(k + 1), L) accumulated;
    a start s is confirmed by chunk 0 when s < 2048 and L > 4096 (end clipped
    at 4096), and once more by chunk floor(s / 4096) + 1, or by the last chunk,
    with the end clipped at min(4096 (floor(s / 4096) + 2), L)."""
    L = H.size
    S = oracle.patch_indices(oracle.patch_mask(H[None, :], thr, 0))[0]
    nxt = {s: (S[i + 1] if i + 1 < len(S) else L) for i, s in enumerate(S)}
    if L <= 4096:
        return [(s, nxt[s]) for s in S]
    first = [(s, min(nxt[s], 4096)) for s in S if s < 2048]
    return first + [(s, min(nxt[s], min(4096 * (s // 4096 + 2), L))) for s in S]


@pytest.mark.parametrize("L", [1, 2, 3, 100, 2048, 4096, 4097, 6000, 6144, 8192, 8193, 12288,
                               12289, 20000])
@pytest.mark.parametrize("sparse", [False, True])
def test_pipeline_closed_form(L, sparse):
    rng = np.random.default_rng(L * 2 + sparse)
    if sparse:
        # a jump every ~5000 positions: patches longer than a chunk, clipped ends
        H = np.zeros(L, np.float32)
        H[rng.integers(0, max(L, 1), size=max(1, L // 5000))] = 5.0
    else:
        H = rng.gamma(2.0, 0.8, size=L).astype(np.float32)
    N = rng.uniform(0.5, 2.0, size=L).astype(np.float32)
    data = rng.integers(0, 256, size=L, dtype=np.uint8).tobytes()
    r = oracle.pipeline_process_document(data, _table_forward(H, N, data), 1.335)
    got = [(s, s + n) for s, n, *_ in r["patches"]]
    assert got == _closed_form(H, 1.335)
    for s, n, p, h, b in r["patches"]:
        assert b == data[s:s + n] and n >= 1
    np.testing.assert_array_equal(r["entropies"], H)


def _closed_form_general(H, thr, C, S):
    """The emitted (start, end) pairs for chunk C and stride S <= C, from the
    chunk geometry: chunk 0 keeps [0, C) and confirms starts below C - S (all
    when it is the last); chunk k >= 1 starts at kC - S, keeps [kC, (k + 1)C)
    and confirms starts in [max(kC - 2S, 0), (k + 1)C - 2S) (no upper end for
    the last chunk); every end is clipped at the accumulated end."""
    L = H.size
    S_ = oracle.patch_indices(oracle.patch_mask(H[None, :], thr, 0))[0] if L else []
    nxt = {s: (S_[i + 1] if i + 1 < len(S_) else L) for i, s in enumerate(S_)}
    out = []
    k = 0
    while k * C < L or (k == 0 and L > 0):
        acc = min((k + 1) * C, L)
        last = (k + 1) * C >= L
        lo = 0 if k == 0 else max(k * C - 2 * S, 0)
        hi = None if last else ((C - S) if k == 0 else (k + 1) * C - 2 * S)
        out += [(s, min(nxt[s], acc)) for s in S_
                if s >= lo and (hi is None or s < hi) and s < acc]
        if last:
            break
        k += 1
    return out


def test_pipeline_closed_form_any_chunking():
    rng = np.random.default_rng(77)
    for _ in range(400):
        C = int(rng.integers(2, 13))
        S = int(rng.integers(1, C + 1))
        L = int(rng.integers(0, 70))
        H = (rng.integers(0, 4, size=L) * rng.choice([0.0, 1.0, 2.5], size=L)).astype(np.float32)
        N = rng.uniform(0.5, 2.0, size=L).astype(np.float32)
        data = rng.integers(0, 256, size=L, dtype=np.uint8).tobytes()
        r = oracle.pipeline_process_document(data, _table_forward(H, N, data), 1.0, C, S)
        got = [(s, s + n) for s, n, *_ in r["patches"]]
        assert got == _closed_form_general(H, 1.0, C, S), (C, S, L)
        np.testing.assert_array_equal(r["entropies"], H)


def test_patch_data_embedding_is_per_patch():
    # pipeline.rs:46-60: every PatchData carries its own 768-float zero
    # embedding; the mirror allocates it on first access
    from blt_burn_amd.pipeline import EMBEDDING_DIM, PatchData
    a = PatchData(3, 4, None, 1.5, 2.5, b"abcd")
    b = PatchData(3, 4, None, 1.5, 2.5, b"abcd")
    assert a.embedding.shape == (EMBEDDING_DIM,) and a.embedding.dtype == np.float32
    assert not a.embedding.any()
    assert a == b
    a.embedding[0] = 1.0  # a patch's embedding is its own array
    assert not b.embedding.any() and a != b
    b.embedding = np.ones(EMBEDDING_DIM, np.float32)
    assert b.embedding.sum() == EMBEDDING_DIM
    c = PatchData(start_offset=0, length=1, prominence=0.5, entropy=0.25, bytes=b"x")
    assert (c.start_offset, c.length, c.prominence, c.entropy, c.bytes) == (0, 1, 0.5, 0.25, b"x")
    assert "start_offset=0" in repr(c)
