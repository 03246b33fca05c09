"""Byte tokenizer of the entropy model (tokenizer.rs), over the C ABI.

encode() is BltTokenizer::encode applied to String::from_utf8_lossy(bytes),
which is how the reference builds token streams (blt_core.rs:93-96, 152-154):
ill-formed UTF-8 becomes U+FFFD before the bytes are offset by 4.  The work
is done by blt_tokenize_bytes in libblt_hip.so (host code, no GPU).
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import check

# tokenizer.rs:4-10
BOE_ID = 0
BOS_ID = 1
EOS_ID = 2
BPE_ID = 3
OFFSET = 4
BYTE_UNITS = 256


def tokenize_bytes(data, add_bos=False, add_eos=False):
    """bytes-like -> int32 numpy array of token ids."""
    buf = np.frombuffer(bytes(data), dtype=np.uint8)
    n = ctypes.c_int64()
    L = _lib.lib()
    ptr = buf.ctypes.data if buf.size else None
    # at most 3 tokens per input byte (one U+FFFD per ill-formed byte) + BOS/EOS
    out = np.empty(3 * buf.size + 2, dtype=np.int32)
    check(L.blt_tokenize_bytes(ptr, buf.size, int(add_bos), int(add_eos), out.ctypes.data,
                               out.size, ctypes.byref(n)), "blt_tokenize_bytes")
    return out[: n.value].copy()


def tokenize_documents(data, byte_offsets, add_bos=False, add_eos=False):
    """Concatenated documents data[byte_offsets[d]:byte_offsets[d + 1]] ->
    (tokens int32 [total], token_offsets int64 [n_docs + 1]); each document is
    tokenized on its own, as tokenize_bytes."""
    buf = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8) if isinstance(
        data, (bytes, bytearray)) else data, dtype=np.uint8)
    boff = np.ascontiguousarray(byte_offsets, dtype=np.int64)
    nd = boff.size - 1
    cap = 3 * buf.size + 2 * nd
    out = np.empty(max(cap, 1), dtype=np.int32)
    toff = np.zeros(nd + 1, dtype=np.int64)
    check(_lib.lib().blt_tokenize_documents(buf.ctypes.data if buf.size else None,
                                            boff.ctypes.data, nd, int(add_bos), int(add_eos),
                                            out.ctypes.data, cap, toff.ctypes.data),
          "blt_tokenize_documents")
    return out[: toff[-1]].copy(), toff


class BltTokenizer:
    """BltTokenizer::new(add_bos, add_eos) without BPE delimiters (tokenizer.rs:12-36)."""

    def __init__(self, add_bos=False, add_eos=False):
        self.add_bos = add_bos
        self.add_eos = add_eos
        self.offsetting_special_char = OFFSET
        self.bos_id = BOS_ID
        self.eos_id = EOS_ID

    def encode(self, text):
        """str (or bytes, decoded lossily first) -> list of token ids (tokenizer.rs:50-103)."""
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        return tokenize_bytes(data, self.add_bos, self.add_eos).tolist()

    def decode(self, tokens):
        """Drops ids below OFFSET, decodes the bytes lossily (tokenizer.rs:105-118)."""
        raw = bytes((t - OFFSET) & 0xFF for t in tokens if t >= OFFSET)
        return raw.decode("utf-8", errors="replace")
