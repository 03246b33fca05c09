"""Device-memory plumbing: torch CUDA tensors carry the buffers and streams
handed to the C ABI (pointers, element counts, the current HIP stream)."""
import torch

from ._lib import BltError


# the raw current-stream handle without building a torch.cuda.Stream object
# (one per call otherwise: about 1.5 us of host time on every launch)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device=None):
    if _raw_stream is not None:
        if isinstance(device, torch.device) and device.index is not None:
            return _raw_stream(device.index)
        if device is None or isinstance(device, int):
            return _raw_stream(torch.cuda.current_device() if device is None else device)
    return torch.cuda.current_stream(device).cuda_stream


def require_cuda(*tensors):
    for t in tensors:
        if not isinstance(t, torch.Tensor):
            raise TypeError("expected a torch.Tensor, got %r" % type(t))
        if not t.is_cuda:
            raise BltError("tensor must live on a GPU (got device %s)" % t.device)


def contiguous(t):
    return t if t.is_contiguous() else t.contiguous()


def bf16_bits_to_tensor(arr, device):
    """numpy uint16 bf16 bits -> torch.bfloat16 tensor on `device`."""
    import numpy as np
    return torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(torch.bfloat16).to(device)
