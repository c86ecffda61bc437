"""Device memory, streams and FP64 helper products for the ctypes calls, per
array family.

NumPy family (NumPy arrays and array-likes): device arrays from the HIP
runtime (``_hip``), copies on the null stream, FP64 products by rocBLAS; no
PyTorch involved.  Torch family (torch tensors, the optional on-device
type): PyTorch-ROCm's allocator and current stream; FP64 products through
torch (rocBLAS underneath).  Every Ozaki computation is done by
libozaki_amd.so in both.  Arrays cross into the library as (device pointer,
leading dimension) pairs.
"""

import ctypes
import sys
import threading

import numpy as np

from . import _hip
from . import _lib

try:  # imported before the library loads, so both share torch's HIP runtime
    import torch
except ImportError:  # pragma: no cover - torch is optional
    torch = None


def is_torch(x):
    """A torch tensor (or a subclass of one)?  Checked against the torch
    module the program has imported, if any; this never imports it."""
    t = sys.modules.get("torch")
    return t is not None and isinstance(x, t.Tensor)


def ld_of(t):
    """Leading dimension (row stride in elements) of a 2-D device array."""
    if t.dim() != 2:
        raise ValueError("expected a 2-D array")
    return max(int(t.stride(0)), int(t.shape[1]), 1)


_NO_GPU = ("ozaki_jax_amd needs a ROCm GPU; there is no CPU implementation "
           "(no HIP device found).")


def _numpy_to_torch(a, dev):
    """A contiguous NumPy array as a device tensor.  Large ones go through
    the pinned staging buffers (_hip), after torch's current stream has
    drained (the copy runs on the null stream)."""
    if a.nbytes < _hip._STAGE_MIN:
        return torch.from_numpy(a).to(dev)
    t = torch.empty(a.shape, dtype=_TORCH_DTYPES[a.dtype], device=dev)
    torch.cuda.current_stream(dev).synchronize()
    _hip._stager().to_device(t.data_ptr(), a)
    return t


def _torch_to_numpy(t):
    """A device tensor as a new NumPy array, large contiguous ones through the
    pinned staging buffers."""
    if (not t.is_cuda or not t.is_contiguous() or t.dtype not in _NUMPY_DTYPES
            or t.numel() * t.element_size() < _hip._STAGE_MIN):
        return t.cpu().numpy()
    out = np.empty(tuple(t.shape), _NUMPY_DTYPES[t.dtype])
    torch.cuda.current_stream(t.device).synchronize()
    _hip._stager().to_host(out, t.data_ptr())
    return out


# Pinned host words and HIP events of the early flag reads, per device: a
# call takes one pair for the time of its read and gives it back, so the
# pairs are shared by all threads and never leak.
_early_free = {}
_early_lock = threading.Lock()


class _TorchFamily:
    """Torch tensors on torch's current device and stream."""

    def __init__(self):
        if torch is None or not torch.cuda.is_available():
            raise RuntimeError(
                "ozaki_jax_amd needs a ROCm GPU (torch.cuda.is_available() is "
                "False); there is no CPU implementation.")
        _lib.load()
        self.dev = torch.device("cuda", torch.cuda.current_device())

    def stream(self):
        return torch.cuda.current_stream().cuda_stream

    def f64(self, x):
        """float64 device tensor with contiguous rows holding x's values;
        never aliases a NumPy input."""
        if is_torch(x):
            t = x.detach()
            if t.dtype != torch.float64:
                t = t.to(torch.float64)
            if t.device != self.dev:
                t = t.to(self.dev)
        else:
            a = np.ascontiguousarray(np.asarray(x, dtype=np.float64))
            t = _numpy_to_torch(a, self.dev)
        if t.dim() >= 1 and t.numel() > 0 and t.stride(-1) != 1:
            t = t.contiguous()
        if t.dim() == 2 and t.numel() > 0 and t.stride(0) < max(t.shape[1], 1):
            t = t.contiguous()
        return t

    def empty(self, shape, dtype=np.float64):
        return torch.empty(shape, dtype=_TORCH_DTYPES[np.dtype(dtype)], device=self.dev)

    def workspace(self, nbytes):
        return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=self.dev)

    def flags(self):
        """A flag word for a call that clears it itself."""
        return torch.empty(1, dtype=torch.int32, device=self.dev)

    def zero_flags(self):
        return torch.zeros(1, dtype=torch.int32, device=self.dev)

    def zeros(self, shape, dtype):
        return torch.zeros(shape, dtype=_TORCH_DTYPES[np.dtype(dtype)], device=self.dev)

    def early_flags(self):
        """(host word, event, read) for ozk_matmul_early_flags: a pinned
        host word and a HIP event of this device, taken from a shared free
        list, and read() waiting for the event, returning the word and giving
        the pair back.  The product stays ordered on the current stream, as
        torch's own results are."""
        rt = _hip._rt()
        with _early_lock:
            free = _early_free.setdefault(self.dev.index, [])
            pair = free.pop() if free else None
        if pair is None:
            with torch.cuda.device(self.dev):
                pair = (rt.host_malloc(4), rt.event())
        word, ev = pair
        word_v = ctypes.c_uint32.from_address(word)

        def read():
            try:
                rt.wait(ev)
                return int(word_v.value)
            finally:
                with _early_lock:
                    _early_free[self.dev.index].append(pair)

        return word, ev, read

    def read_flags(self, f):
        """Synchronising read of a device flag word."""
        return int(f.item()) & 0xffffffff

    def column(self, v):
        return v[:, None].contiguous()

    def flat(self, v):
        return v[:, 0]

    def out(self, t, want_torch):
        return t if want_torch else _torch_to_numpy(t)

    def matmul(self, A, B):
        """FP64 A @ B."""
        return torch.matmul(A, B)

    def gram_f64(self, A):
        G = torch.matmul(A.T, A)
        return (G + G.T) * 0.5

    def residual_f64(self, A, x, b):
        return b - torch.matmul(A, x)


class _HipFamily:
    """NumPy inputs: device arrays of the HIP runtime on the null stream."""

    def __init__(self):
        if _hip.device_count() < 1:
            raise RuntimeError(_NO_GPU)

    def stream(self):
        return None

    def f64(self, x):
        if is_torch(x):  # matmul_numpy takes any array-like
            x = x.detach().cpu().numpy()
        return _hip.DeviceArray.from_numpy(np.asarray(x, dtype=np.float64))

    def empty(self, shape, dtype=np.float64):
        return _hip.DeviceArray(shape, dtype)

    def workspace(self, nbytes):
        return _hip.DeviceArray((max(int(nbytes), 1),), np.uint8)

    def flags(self):
        return _hip.DeviceArray((1,), np.int32)

    def zero_flags(self):
        return _hip.DeviceArray.zeros((1,), np.int32)

    def zeros(self, shape, dtype):
        return _hip.DeviceArray.zeros(shape, dtype)

    def read_flags(self, f):
        return int(f.numpy()[0]) & 0xffffffff

    def column(self, v):
        return v.column()

    def flat(self, v):
        return v.flat()

    def out(self, t, want_torch):
        if want_torch:
            raise TypeError("a NumPy-family result cannot be returned as a tensor")
        return t.numpy()

    def matmul(self, A, B):
        C = _hip.DeviceArray((A.shape[0], B.shape[1]))
        return _hip.blas().matmul(A, B, C)

    def gram_f64(self, A):
        n = A.shape[1]
        G = _hip.blas().gram(A, _hip.DeviceArray((n, n)))
        return _hip.blas().half_sum_transpose(G, _hip.DeviceArray((n, n)))

    def residual_f64(self, A, x, b):
        r = _hip.DeviceArray(b.shape)
        r.copy_from(b)
        return _hip.blas().matmul(A, x, r, alpha=-1.0, beta=1.0)


_TORCH_DTYPES = {}
_NUMPY_DTYPES = {}
if torch is not None:
    _TORCH_DTYPES = {np.dtype(np.float64): torch.float64, np.dtype(np.float32): torch.float32,
                     np.dtype(np.int32): torch.int32, np.dtype(np.int16): torch.int16,
                     np.dtype(np.int8): torch.int8, np.dtype(np.uint8): torch.uint8}
    _NUMPY_DTYPES = {v: k for k, v in _TORCH_DTYPES.items()}


def family(want_torch):
    """The device family of a call: torch tensors in -> torch, else the
    HIP-runtime NumPy family."""
    return _TorchFamily() if want_torch else _HipFamily()


# ---- helpers of the torch-only modules (solve, lstsq, norm, inv, extract,
# accumulate, lowlevel), which take their FP32 factorisations from torch.linalg

def require_gpu():
    fam = _TorchFamily()
    return fam.dev


def stream_handle():
    """hipStream_t of torch's current stream, as an integer for ctypes."""
    return torch.cuda.current_stream().cuda_stream


def to_device_f64(x, dev):
    """float64 device tensor with contiguous rows holding the values of `x`
    (NumPy array, array-like or torch tensor).  Never aliases NumPy input."""
    fam = _TorchFamily.__new__(_TorchFamily)
    fam.dev = dev
    return fam.f64(x)


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
    return _torch_to_numpy(t)


def ptr(t):
    return t.data_ptr() if t is not None else None
