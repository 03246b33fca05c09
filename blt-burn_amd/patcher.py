"""Patcher API of the reference (src/patcher.rs) on the GPU.

entropy / patch_start_mask_from_entropy_with_monotonicity keep the reference's
signatures; the device pass behind them also compacts start indices and
lengths (patch_boundaries), and patch_start_indices_cpu compacts a mask on the
device when it lives on a GPU, so only the results are copied to the host.

The pass runs many blocks per row and passes per-tile counts and flag words
between its kernels through a workspace.  Each call takes its own from torch's
caching allocator on the current stream, so calls on different streams or
threads never share one (the allocator hands a freed block out again only to
later work on the same stream).  Two rules (e.g. the global and the monotonic
mask) can share one read of the entropies (patch_boundaries_rules), and
entropy_patch_boundaries computes the entropies and the rules in one pass over
the logits.
"""
import torch

from . import _lib
from ._lib import PATCH_GLOBAL, PATCH_MONOTONIC, BltError, check
from ._torch import contiguous, require_cuda, stream_ptr
from .fused_ops import fused_entropy

__all__ = ["entropy", "patch_start_mask_from_entropy_with_monotonicity",
           "patch_start_mask_global", "patch_boundaries", "patch_boundaries_rules",
           "entropy_patch_boundaries", "patch_start_indices_cpu", "patch_mask_starts",
           "patch_lengths_from_start_indices", "patch_means", "PATCH_MONOTONIC",
           "PATCH_GLOBAL"]


def entropy(scores):
    """[batch, seq, vocab] logits -> [batch, seq] entropies (patcher.rs:15-22)."""
    return fused_entropy(scores, scores.shape[-1])


def _workspace(device, nbytes):
    """A workspace for one boundary pass on `device`, allocated on the current
    stream (where the pass runs): the caching allocator keeps this cheap, and
    the block returns to that stream's pool when the call's tensor is dropped,
    after the kernels queued on it."""
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


def _rule_outputs(B, T, device, out):
    i32 = torch.int32
    if out is not None:
        mask, starts, lengths, counts = out
        for t, shp in ((mask, (B, T)), (starts, (B, T)), (lengths, (B, T)), (counts, (B,))):
            require_cuda(t)
            if not (t.dtype == i32 and tuple(t.shape) == shp and t.is_contiguous() and
                    t.device == device):
                raise BltError("patch boundaries: out tensors must be contiguous int32 "
                               "[batch, seq] x3 and [batch] on the entropies' device")
        return tuple(out)
    return (torch.empty((B, T), dtype=i32, device=device),
            torch.empty((B, T), dtype=i32, device=device),
            torch.empty((B, T), dtype=i32, device=device),
            torch.empty((B,), dtype=i32, device=device))


def _rules_struct(rules, outs):
    if not 1 <= len(rules) <= 2:
        raise BltError("one or two boundary rules per pass")
    arr = (_lib.PatchRule * len(rules))()
    for r, ((mode, thr), (mask, starts, lengths, counts)) in enumerate(zip(rules, outs)):
        arr[r] = _lib.PatchRule(int(mode), float(thr), mask.data_ptr(), starts.data_ptr(),
                                lengths.data_ptr(), counts.data_ptr())
    return arr


def patch_boundaries_rules(entropies, rules, out=None):
    """One or two boundary rules over entropies [batch, seq] f32 in one read
    (patcher.rs:80-164 once per rule).  rules: [(mode, threshold), ...].
    Returns one (mask, starts, lengths, counts) per rule, laid out as
    patch_boundaries returns them; `out` may pass them preallocated."""
    require_cuda(entropies)
    if entropies.dim() != 2:
        raise BltError("patch_boundaries expects [batch, seq]")
    H = contiguous(entropies if entropies.dtype == torch.float32 else entropies.to(torch.float32))
    B, T = H.shape
    rules = list(rules)
    outs = [_rule_outputs(B, T, H.device, out[r] if out is not None else None)
            for r in range(len(rules))]
    arr = _rules_struct(rules, outs)
    L = _lib.lib()
    nbytes = L.blt_patch_workspace_bytes(B, T, len(rules))
    ws = _workspace(H.device, nbytes)
    check(L.blt_patch_boundaries_rules(H.data_ptr(), B, T, len(rules), arr, ws.data_ptr(),
                                       ws.numel(), stream_ptr(H.device)), "patch_boundaries")
    return outs


def entropy_patch_boundaries(logits, rules, out=None, entropies=None):
    """patcher::entropy (patcher.rs:15-22) and then the boundary rules, in one
    pass over logits [batch, seq, vocab] f32.  Returns (entropies [batch, seq]
    f32, [(mask, starts, lengths, counts) per rule])."""
    require_cuda(logits)
    if logits.dim() != 3 or logits.dtype != torch.float32:
        raise BltError("entropy_patch_boundaries expects f32 logits [batch, seq, vocab]")
    x = contiguous(logits)
    B, T, V = x.shape
    if entropies is None:
        entropies = torch.empty((B, T), dtype=torch.float32, device=x.device)
    else:
        require_cuda(entropies)
        if not (entropies.dtype == torch.float32 and tuple(entropies.shape) == (B, T) and
                entropies.is_contiguous() and entropies.device == x.device):
            raise BltError("entropy_patch_boundaries: entropies out must be contiguous f32 "
                           "[batch, seq] on the logits' device")
    rules = list(rules)
    outs = [_rule_outputs(B, T, x.device, out[r] if out is not None else None)
            for r in range(len(rules))]
    arr = _rules_struct(rules, outs)
    L = _lib.lib()
    nbytes = L.blt_patch_workspace_bytes(B, T, len(rules))
    ws = _workspace(x.device, nbytes)
    check(L.blt_entropy_patch_boundaries(x.data_ptr(), B, T, V, entropies.data_ptr(), len(rules),
                                         arr, ws.data_ptr(), ws.numel(), stream_ptr(x.device)),
          "entropy_patch_boundaries")
    return entropies, outs


class EntropyPatchPlan:
    """entropy_patch_boundaries prepared for repeated calls on logits of one
    shape, as a serving loop makes them: the entropies and rule outputs are
    allocated, the rule array and the workspace bound, once; each call checks
    the logits and makes the one library call (the per-call checks of a dozen
    tensors cost the function form more host time than the device pass).
    Calls return the same output tensors and reuse the plan's own workspace
    each time, so the calls of one plan must be stream-ordered (one plan per
    stream or thread); separate plans and the function forms share nothing."""

    def __init__(self, batch, seq, vocab, rules, device=None):
        dev = torch.device("cuda" if device is None else device)
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        rules = list(rules)
        self.shape = (int(batch), int(seq), int(vocab))
        self.device = dev
        self.entropies = torch.empty((batch, seq), dtype=torch.float32, device=dev)
        self.outs = [_rule_outputs(batch, seq, dev, None) for _ in rules]
        self._arr = _rules_struct(rules, self.outs)
        L = _lib.lib()
        self._ws = _workspace(dev, L.blt_patch_workspace_bytes(batch, seq, len(rules)))
        self._fn = L.blt_entropy_patch_boundaries
        self._tail = (self.entropies.data_ptr(), len(rules), self._arr, self._ws.data_ptr(),
                      self._ws.numel())

    def __call__(self, logits):
        """logits: f32 [batch, seq, vocab] on the plan's device, contiguous.
        Returns (entropies, [(mask, starts, lengths, counts) per rule])."""
        if not (isinstance(logits, torch.Tensor) and logits.dtype == torch.float32 and
                logits.shape == self.shape and logits.device == self.device and
                logits.is_contiguous()):
            raise BltError("EntropyPatchPlan expects contiguous f32 logits %s on %s"
                           % (list(self.shape), self.device))
        B, T, V = self.shape
        check(self._fn(logits.data_ptr(), B, T, V, *self._tail, stream_ptr(self.device)),
              "entropy_patch_boundaries")
        return self.entropies, self.outs


def patch_boundaries(entropies, threshold, mode=PATCH_MONOTONIC, out=None):
    """Device pass over entropies [batch, seq] f32.  Returns (mask, starts, lengths,
    counts): mask [B, T] int32, starts/lengths [B, T] int32 with counts[b] valid
    entries per row, counts [B] int32.  mode PATCH_MONOTONIC: patcher.rs:80-118;
    PATCH_GLOBAL: same layout with H[t] > threshold.  `out` may pass the four
    result tensors preallocated (reused as is)."""
    return patch_boundaries_rules(entropies, [(mode, threshold)],
                                  out=[out] if out is not None else None)[0]


def patch_start_mask_from_entropy_with_monotonicity(entropies, threshold):
    """[batch, seq] -> int32 mask [batch, seq]: positions 0 and 1 start patches,
    t >= 2 starts one iff H[t] - H[t-1] > threshold (patcher.rs:80-118)."""
    return patch_boundaries(entropies, threshold, PATCH_MONOTONIC)[0]


def patch_start_mask_global(entropies, threshold):
    """Global-threshold variant: [1, 1, H[t] > threshold for t >= 2]."""
    return patch_boundaries(entropies, threshold, PATCH_GLOBAL)[0]


def patch_start_indices_cpu(patch_start_mask):
    """Per-row lists of positions whose mask is exactly 1 (patcher.rs:124-142).

    A mask on a GPU is compacted there (blt_patch_mask_starts) and only the
    starts and counts come back; a host tensor is scanned on the host, which
    is what the reference's function does with the data it reads back."""
    if patch_start_mask.dim() != 2:
        raise BltError("patch_start_indices_cpu expects [batch, seq]")
    if not patch_start_mask.is_cuda:
        m = patch_start_mask.detach()
        return [torch.nonzero(row == 1).flatten().tolist() for row in m]
    m = contiguous(patch_start_mask if patch_start_mask.dtype == torch.int32
                   else patch_start_mask.to(torch.int32))
    B, T = m.shape
    starts = torch.empty((B, T), dtype=torch.int32, device=m.device)
    counts = torch.empty((B,), dtype=torch.int32, device=m.device)
    check(_lib.lib().blt_patch_mask_starts(m.data_ptr(), B, T, starts.data_ptr(), None,
                                           counts.data_ptr(), stream_ptr(m.device)),
          "patch_mask_starts")
    ct = counts.cpu().tolist()
    n = max(ct) if ct else 0
    st = starts[:, :n].cpu().tolist()
    return [st[b][:ct[b]] for b in range(B)]


def patch_mask_starts(patch_start_mask):
    """Device compaction of a start mask [batch, seq] (patcher.rs:124-164):
    (starts [B, T], lengths [B, T], counts [B]) int32 on the mask's GPU, laid
    out as patch_boundaries returns them."""
    require_cuda(patch_start_mask)
    if patch_start_mask.dim() != 2:
        raise BltError("patch_mask_starts expects [batch, seq]")
    m = contiguous(patch_start_mask if patch_start_mask.dtype == torch.int32
                   else patch_start_mask.to(torch.int32))
    B, T = m.shape
    starts = torch.empty((B, T), dtype=torch.int32, device=m.device)
    lengths = torch.empty((B, T), dtype=torch.int32, device=m.device)
    counts = torch.empty((B,), dtype=torch.int32, device=m.device)
    check(_lib.lib().blt_patch_mask_starts(m.data_ptr(), B, T, starts.data_ptr(),
                                           lengths.data_ptr(), counts.data_ptr(),
                                           stream_ptr(m.device)), "patch_mask_starts")
    return starts, lengths, counts


def patch_lengths_from_start_indices(start_indices, seq_len):
    """Per-row patch lengths from start lists: next start (or seq_len) minus start
    (patcher.rs:144-164)."""
    out = []
    for idx in start_indices:
        out.append([(idx[i + 1] if i + 1 < len(idx) else seq_len) - idx[i]
                    for i in range(len(idx))])
    return out


def patch_means(entropies, norms, starts, counts, coherence=None, out=None):
    """Per-patch means on the device (compute_mean_entropy /
    compute_mean_prominence, pipeline.rs:240-258; segment coherence,
    huggingface_loader.rs:265-295): for patch p of row b (starts / counts as
    patch_boundaries returns them) the left-to-right f32 mean of entropies,
    norms and (optionally) coherence over [starts[b, p], next start or seq).
    Returns (mean_entropy, mean_prominence, mean_coherence or None), each
    [B, T] f32 with counts[b] valid entries per row."""
    for t in (entropies, norms, starts, counts):
        require_cuda(t)
    H = contiguous(entropies.to(torch.float32))
    N = contiguous(norms.to(torch.float32))
    if H.dim() != 2 or N.shape != H.shape:
        raise BltError("patch_means expects entropies and norms [batch, seq]")
    B, T = H.shape
    st = contiguous(starts.to(torch.int32))
    ct = contiguous(counts.to(torch.int32))
    if tuple(st.shape) != (B, T) or tuple(ct.shape) != (B,):
        raise BltError("patch_means expects starts [batch, seq] and counts [batch]")
    C = None
    if coherence is not None:
        require_cuda(coherence)
        C = contiguous(coherence.to(torch.float32))
        if C.shape != H.shape:
            raise BltError("patch_means: coherence must match entropies")
    if out is not None:
        mH, mN, mC = out
        if (mC is None) != (C is None):
            raise BltError("patch_means: out must hold a coherence tensor exactly when "
                           "coherence is given")
        for t in (mH, mN, mC):
            if t is None:
                continue
            if not isinstance(t, torch.Tensor):
                raise TypeError("expected a torch.Tensor, got %r" % type(t))
            if not (t.is_cuda and t.device == H.device and t.dtype == torch.float32 and
                    tuple(t.shape) == (B, T) and t.is_contiguous()):
                raise BltError("patch_means: out tensors must be contiguous f32 [batch, seq] "
                               "on the entropies' device")
    else:
        mH = torch.empty((B, T), dtype=torch.float32, device=H.device)
        mN = torch.empty((B, T), dtype=torch.float32, device=H.device)
        mC = torch.empty((B, T), dtype=torch.float32, device=H.device) if C is not None else None
    check(_lib.lib().blt_patch_means(H.data_ptr(), N.data_ptr(),
                                     C.data_ptr() if C is not None else None, st.data_ptr(),
                                     ct.data_ptr(), B, T, mH.data_ptr(), mN.data_ptr(),
                                     mC.data_ptr() if mC is not None else None,
                                     stream_ptr(H.device)), "patch_means")
    return mH, mN, mC
