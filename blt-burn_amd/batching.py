"""Document batching utilities of the ingest path (batching.rs:1-204).

Mirrors SizeBucket, BatchStats, sort_by_length, sort_by_length_desc,
bucket_by_size and LengthSortedWindow over PrefetchedDoc.  In the reference
these order documents so that one-document forwards of similar length follow
each other; here the native ingest driver packs the chunks of many documents
into shared [rows, row_len] forwards (each chunk its own attention / RoPE
segment, so no document sees another), and these helpers order or summarise
the documents handed to it.
"""
import enum
from typing import Dict, List, Optional

from .prefetch import PrefetchedDoc

__all__ = ["SizeBucket", "BatchStats", "sort_by_length", "sort_by_length_desc",
           "bucket_by_size", "LengthSortedWindow"]


class SizeBucket(enum.Enum):
    """batching.rs:19-55."""
    TINY = "tiny (<512B)"
    SMALL = "small (512B-2KB)"
    MEDIUM = "medium (2KB-8KB)"
    LARGE = "large (8KB-32KB)"
    HUGE = "huge (>32KB)"

    @classmethod
    def from_len(cls, n):
        if n < 512:
            return cls.TINY
        if n < 2048:
            return cls.SMALL
        if n < 8192:
            return cls.MEDIUM
        if n < 32768:
            return cls.LARGE
        return cls.HUGE

    def name_str(self):
        """SizeBucket::name: the label used in summaries."""
        return self.value


class BatchStats:
    """batching.rs:58-117: document counts per size bucket and total bytes."""

    def __init__(self):
        self.tiny_count = self.small_count = self.medium_count = 0
        self.large_count = self.huge_count = 0
        self.total_bytes = 0

    def add(self, doc: PrefetchedDoc):
        self.total_bytes += doc.original_len
        b = SizeBucket.from_len(doc.original_len)
        attr = {SizeBucket.TINY: "tiny_count", SizeBucket.SMALL: "small_count",
                SizeBucket.MEDIUM: "medium_count", SizeBucket.LARGE: "large_count",
                SizeBucket.HUGE: "huge_count"}[b]
        setattr(self, attr, getattr(self, attr) + 1)

    def summary(self):
        """The lines print_summary writes (returned, not printed)."""
        counts = [self.tiny_count, self.small_count, self.medium_count, self.large_count,
                  self.huge_count]
        total = sum(counts)
        labels = ["Tiny (<512B):    ", "Small (512B-2KB):", "Medium (2KB-8KB):",
                  "Large (8KB-32KB):", "Huge (>32KB):    "]
        out = ["Document size distribution:"]
        for lab, c in zip(labels, counts):
            out.append("   %s %d (%.1f%%)" % (lab, c, 100.0 * c / max(total, 1)))
        out.append("   Total: %d docs, %d bytes" % (total, self.total_bytes))
        return out

    def print_summary(self):
        print("\n".join(self.summary()))


def sort_by_length(docs: List[PrefetchedDoc]) -> List[PrefetchedDoc]:
    """batching.rs:129-132 (stable, ascending original_len)."""
    return sorted(docs, key=lambda d: d.original_len)


def sort_by_length_desc(docs: List[PrefetchedDoc]) -> List[PrefetchedDoc]:
    """batching.rs:140-143 (stable, descending original_len)."""
    return sorted(docs, key=lambda d: -d.original_len)


def bucket_by_size(docs: List[PrefetchedDoc]) -> Dict[SizeBucket, List[PrefetchedDoc]]:
    """batching.rs:149-158."""
    out: Dict[SizeBucket, List[PrefetchedDoc]] = {}
    for d in docs:
        out.setdefault(SizeBucket.from_len(d.original_len), []).append(d)
    return out


class LengthSortedWindow:
    """batching.rs:165-204: buffers window_size documents and hands them back
    sorted by length once the window is full."""

    def __init__(self, window_size=100):
        self.window: List[PrefetchedDoc] = []
        self.window_size = window_size

    def add(self, doc: PrefetchedDoc) -> Optional[List[PrefetchedDoc]]:
        self.window.append(doc)
        if len(self.window) >= self.window_size:
            out = sort_by_length(self.window)
            self.window = []
            return out
        return None

    def flush(self) -> List[PrefetchedDoc]:
        out = sort_by_length(self.window)
        self.window = []
        return out
