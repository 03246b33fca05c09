"""Patcher API of the reference (src/patcher.rs) on the GPU.

entropy / patch_start_mask_from_entropy_with_monotonicity keep the reference's
signatures; the device kernel behind them also compacts start indices and
lengths (patch_boundaries), so patch_start_indices_cpu only copies results.
"""
import torch

from . import _lib
from ._lib import PATCH_GLOBAL, PATCH_MONOTONIC, BltError, check
from ._torch import contiguous, require_cuda, stream_ptr
from .fused_ops import fused_entropy

__all__ = ["entropy", "patch_start_mask_from_entropy_with_monotonicity",
           "patch_start_mask_global", "patch_boundaries", "patch_start_indices_cpu",
           "patch_lengths_from_start_indices", "patch_means", "PATCH_MONOTONIC",
           "PATCH_GLOBAL"]


def entropy(scores):
    """[batch, seq, vocab] logits -> [batch, seq] entropies (patcher.rs:15-22)."""
    return fused_entropy(scores, scores.shape[-1])


def patch_boundaries(entropies, threshold, mode=PATCH_MONOTONIC, out=None):
    """Device pass over entropies [batch, seq] f32.  Returns (mask, starts, lengths,
    counts): mask [B, T] int32, starts/lengths [B, T] int32 with counts[b] valid
    entries per row, counts [B] int32.  mode PATCH_MONOTONIC: patcher.rs:80-118;
    PATCH_GLOBAL: same layout with H[t] > threshold.  `out` may pass the four
    result tensors preallocated (reused as is)."""
    require_cuda(entropies)
    if entropies.dim() != 2:
        raise BltError("patch_boundaries expects [batch, seq]")
    H = contiguous(entropies if entropies.dtype == torch.float32 else entropies.to(torch.float32))
    B, T = H.shape
    if out is not None:
        mask, starts, lengths, counts = out
        i32 = torch.int32
        for t, shp in ((mask, (B, T)), (starts, (B, T)), (lengths, (B, T)), (counts, (B,))):
            if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == i32 and
                    t.shape == shp and t.is_contiguous()):
                require_cuda(t)
                raise BltError("patch_boundaries: out tensors must be contiguous int32")
    else:
        mask = torch.empty((B, T), dtype=torch.int32, device=H.device)
        starts = torch.empty((B, T), dtype=torch.int32, device=H.device)
        lengths = torch.empty((B, T), dtype=torch.int32, device=H.device)
        counts = torch.empty((B,), dtype=torch.int32, device=H.device)
    check(_lib.lib().blt_patch_boundaries(H.data_ptr(), B, T, float(threshold), mode,
                                          mask.data_ptr(), starts.data_ptr(), lengths.data_ptr(),
                                          counts.data_ptr(), stream_ptr(H.device)),
          "patch_boundaries")
    return mask, starts, lengths, counts


def patch_start_mask_from_entropy_with_monotonicity(entropies, threshold):
    """[batch, seq] -> int32 mask [batch, seq]: positions 0 and 1 start patches,
    t >= 2 starts one iff H[t] - H[t-1] > threshold (patcher.rs:80-118)."""
    return patch_boundaries(entropies, threshold, PATCH_MONOTONIC)[0]


def patch_start_mask_global(entropies, threshold):
    """Global-threshold variant: [1, 1, H[t] > threshold for t >= 2]."""
    return patch_boundaries(entropies, threshold, PATCH_GLOBAL)[0]


def patch_start_indices_cpu(patch_start_mask):
    """Per-row lists of positions whose mask is 1 (patcher.rs:124-142)."""
    m = patch_start_mask.detach().to("cpu")
    if m.dim() != 2:
        raise BltError("patch_start_indices_cpu expects [batch, seq]")
    return [torch.nonzero(row == 1).flatten().tolist() for row in m]


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
