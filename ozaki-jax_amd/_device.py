"""Device-memory plumbing for the ctypes calls.

PyTorch-ROCm provides the device allocations (its caching allocator) and the
current HIP stream; every computation is done by libozaki_amd.so.  Arrays
cross into the library as (device pointer, leading dimension) pairs.
"""

import numpy as np

from . import _lib

try:
    import torch
except ImportError:  # pragma: no cover - torch is part of the image
    torch = None


def is_torch(x):
    return torch is not None and isinstance(x, torch.Tensor)


def require_gpu():
    if torch is None or not torch.cuda.is_available():
        raise RuntimeError(
            "ozaki_jax_amd needs a ROCm GPU (torch.cuda.is_available() is "
            "False); there is no CPU implementation.")
    _lib.load()
    return torch.device("cuda", torch.cuda.current_device())


def stream_handle():
    """hipStream_t of torch's current stream, as an integer for ctypes."""
    return torch.cuda.current_stream().cuda_stream


def to_device_f64(x, dev):
    """Return a float64 device tensor whose rows are contiguous (stride 1 in
    the last dimension) holding the values of `x` (NumPy array, array-like or
    torch tensor).  Never aliases a NumPy input."""
    if is_torch(x):
        t = x.detach()
        if t.dtype != torch.float64:
            t = t.to(torch.float64)
        if t.device != dev:
            t = t.to(dev)
    else:
        a = np.ascontiguousarray(np.asarray(x, dtype=np.float64))
        t = torch.from_numpy(a).to(dev)
    if t.dim() >= 1 and t.numel() > 0 and t.stride(-1) != 1:
        t = t.contiguous()
    if t.dim() == 2 and t.numel() > 0 and t.stride(0) < max(t.shape[1], 1):
        t = t.contiguous()
    return t


def ld_of(t):
    """Leading dimension (row stride in elements) of a 2-D device tensor."""
    if t.dim() != 2:
        raise ValueError("expected a 2-D tensor")
    return max(int(t.stride(0)), int(t.shape[1]), 1)


def ptr(t):
    return ctypes_ptr(t.data_ptr()) if t is not None else None


def ctypes_ptr(v):
    return v if v else None


def workspace(nbytes, dev):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


def new_flags(dev):
    return torch.zeros(1, dtype=torch.int32, device=dev)


def read_flags(flags):
    """Synchronising read of the device flag word."""
    return int(flags.item())


def to_family(t, want_torch):
    """Return device tensor `t` as a torch tensor or as a NumPy array."""
    if want_torch:
        return t
    return t.cpu().numpy()
