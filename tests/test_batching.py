"""Document batching helpers (batching.rs:1-204), host only: the reference's
own unit tests (batching.rs:205-300) restated."""
from blt_burn_amd.batching import (BatchStats, LengthSortedWindow, SizeBucket, bucket_by_size,
                                   sort_by_length, sort_by_length_desc)
from blt_burn_amd.prefetch import PrefetchedDoc


def _doc(i, n):
    return PrefetchedDoc(id=i, bytes=bytes(n), original_len=n)


def test_size_bucket_classification():
    cases = [(100, SizeBucket.TINY), (511, SizeBucket.TINY), (512, SizeBucket.SMALL),
             (2047, SizeBucket.SMALL), (2048, SizeBucket.MEDIUM), (8191, SizeBucket.MEDIUM),
             (8192, SizeBucket.LARGE), (32767, SizeBucket.LARGE), (32768, SizeBucket.HUGE),
             (100_000, SizeBucket.HUGE), (0, SizeBucket.TINY)]
    for n, b in cases:
        assert SizeBucket.from_len(n) is b, n
    assert SizeBucket.MEDIUM.name_str() == "medium (2KB-8KB)"


def test_sort_by_length():
    docs = [_doc("c", 3000), _doc("a", 100), _doc("b", 1000)]
    assert [d.id for d in sort_by_length(docs)] == ["a", "b", "c"]
    assert [d.id for d in sort_by_length_desc(docs)] == ["c", "b", "a"]
    # stable for equal lengths, both directions
    eq = [_doc("x", 5), _doc("y", 5), _doc("z", 1)]
    assert [d.id for d in sort_by_length(eq)] == ["z", "x", "y"]
    assert [d.id for d in sort_by_length_desc(eq)] == ["x", "y", "z"]


def test_bucket_by_size():
    b = bucket_by_size([_doc("tiny", 100), _doc("small", 1000), _doc("medium", 4000),
                        _doc("tiny2", 200)])
    assert len(b[SizeBucket.TINY]) == 2 and len(b[SizeBucket.SMALL]) == 1
    assert len(b[SizeBucket.MEDIUM]) == 1 and SizeBucket.LARGE not in b


def test_length_sorted_window():
    w = LengthSortedWindow(3)
    assert w.add(_doc("c", 3000)) is None
    assert w.add(_doc("a", 100)) is None
    batch = w.add(_doc("b", 500))
    assert [d.id for d in batch] == ["a", "b", "c"]
    w.add(_doc("d", 200))
    assert [d.id for d in w.flush()] == ["d"]
    assert w.flush() == []


def test_batch_stats():
    s = BatchStats()
    for i, n in (("a", 100), ("b", 1000), ("c", 4000), ("d", 50)):
        s.add(_doc(i, n))
    assert (s.tiny_count, s.small_count, s.medium_count, s.large_count, s.huge_count) == \
        (2, 1, 1, 0, 0)
    assert s.total_bytes == 5150
    lines = s.summary()
    assert lines[-1] == "   Total: 4 docs, 5150 bytes" and "(50.0%)" in lines[1]
