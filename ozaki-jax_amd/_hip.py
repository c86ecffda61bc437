"""HIP runtime and rocBLAS through ctypes: device memory, copies and FP64
products for the NumPy array family, which therefore needs no PyTorch.

The HIP runtime is reached by its soname after libozaki_amd.so has been
loaded, so this module and the library always share the one copy of the
runtime in the process (PyTorch ships one under the same soname; whichever
was loaded first serves both).  All work runs on the null stream, in order
with the library's kernels, which this family launches there too.

Device memory comes from a caching pool: blocks are rounded to size classes
and kept for reuse after their arrays are garbage collected, so repeated
calls of one shape allocate nothing after the first.

Host copies of large arrays go through two pinned staging buffers: host
threads copy one chunk between the NumPy array and a staging buffer while
the DMA engine moves the other (a direct copy from pageable memory, and
the page faults of a fresh output array, are otherwise serial).
"""

import atexit
import ctypes
import os
import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import _lib

_ROCM_LIB = "/opt/rocm/lib"
_H2D, _D2H, _D2D = 1, 2, 3
_OP_N, _OP_T = 111, 112  # rocblas_operation_none / _transpose


def _open(soname):
    """The library of this soname already in the process, else ROCm's."""
    try:
        return ctypes.CDLL(soname)
    except OSError:
        return ctypes.CDLL(os.path.join(_ROCM_LIB, soname))


class _Runtime:
    def __init__(self):
        _lib.load()  # pulls libamdhip64.so.7 in through its runpath
        h = _open("libamdhip64.so.7")
        vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        for name, args in [("hipMalloc", [ctypes.POINTER(vp), sz]), ("hipFree", [vp]),
                           ("hipMemcpy", [vp, vp, sz, i]),
                           ("hipMemcpyAsync", [vp, vp, sz, i, vp]),
                           ("hipMemset", [vp, i, sz]),
                           ("hipHostFree", [vp]),
                           ("hipStreamDestroy", [vp]),
                           ("hipDeviceSynchronize", []),
                           ("hipHostMalloc", [ctypes.POINTER(vp), sz, ctypes.c_uint]),
                           ("hipEventCreate", [ctypes.POINTER(vp)]),
                           ("hipEventRecord", [vp, vp]),
                           ("hipEventSynchronize", [vp]),
                           ("hipEventDestroy", [vp]),
                           ("hipStreamSynchronize", [vp]),
                           ("hipStreamCreateWithFlags", [ctypes.POINTER(vp), ctypes.c_uint]),
                           ("hipGetDeviceCount", [ctypes.POINTER(i)]),
                           ("hipGetLastError", [])]:
            fn = getattr(h, name)
            fn.restype = i
            fn.argtypes = args
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipGetErrorString.argtypes = [i]
        self.h = h

    def check(self, rc, what):
        if rc != 0:
            msg = self.h.hipGetErrorString(rc).decode(errors="replace")
            self.h.hipGetLastError()  # leave no error behind for other users of the runtime
            raise _lib.OzakiError(f"{what} failed: {msg} ({rc})")

    def device_count(self):
        n = ctypes.c_int(0)
        rc = self.h.hipGetDeviceCount(ctypes.byref(n))
        if rc != 0:
            self.h.hipGetLastError()  # clear the sticky "no device" status
            return 0
        return n.value

    def malloc(self, nbytes):
        p = ctypes.c_void_p()
        self.check(self.h.hipMalloc(ctypes.byref(p), nbytes), f"hipMalloc({nbytes})")
        return p.value

    def free(self, ptr):
        self.check(self.h.hipFree(ptr), "hipFree")

    def copy(self, dst, src, nbytes, kind):
        if nbytes:
            self.check(self.h.hipMemcpy(dst, src, nbytes, kind), "hipMemcpy")

    def memset(self, dst, value, nbytes):
        if nbytes:
            self.check(self.h.hipMemset(dst, value, nbytes), "hipMemset")

    def sync(self, stream=None):
        self.check(self.h.hipStreamSynchronize(stream), "hipStreamSynchronize")

    def host_malloc(self, nbytes):
        p = ctypes.c_void_p()
        self.check(self.h.hipHostMalloc(ctypes.byref(p), nbytes, 0), f"hipHostMalloc({nbytes})")
        return p.value

    def copy_async(self, dst, src, nbytes, kind):
        self.check(self.h.hipMemcpyAsync(dst, src, nbytes, kind, None), "hipMemcpyAsync")

    def event(self):
        e = ctypes.c_void_p()
        self.check(self.h.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e.value

    def record(self, e, stream=None):
        self.check(self.h.hipEventRecord(e, stream), "hipEventRecord")

    def nonblocking_stream(self):
        """A stream that does not wait for the null stream's work, nor the
        null stream for its (hipStreamNonBlocking), at the default priority."""
        s = ctypes.c_void_p()
        self.check(self.h.hipStreamCreateWithFlags(ctypes.byref(s), 1),
                   "hipStreamCreateWithFlags")
        return s.value

    def wait(self, e):
        self.check(self.h.hipEventSynchronize(e), "hipEventSynchronize")

    def destroy_event(self, e):
        self.check(self.h.hipEventDestroy(e), "hipEventDestroy")


# Host copies of at least _STAGE_MIN bytes are staged in _STAGE_CHUNK pieces.
_STAGE_MIN = 32 << 20
_STAGE_CHUNK = 64 << 20


class _Stager:
    """Two pinned buffers of `chunk` bytes (allocated once, kept for the
    process), an event per buffer on the null stream, and a thread pool for
    the host-side copies.  One transfer at a time (a lock)."""

    def __init__(self, rt, chunk=_STAGE_CHUNK):
        self.rt, self.chunk = rt, int(chunk)
        self.buf = [rt.host_malloc(self.chunk) for _ in range(2)]
        self.ev = [rt.event() for _ in range(2)]
        self.nthreads = max(1, min(8, os.cpu_count() or 1))
        self.pool = ThreadPoolExecutor(self.nthreads)
        self.lock = threading.Lock()

    def _host_copy(self, dst, src):
        """dst[:] = src for two flat uint8 arrays, split over the threads."""
        n = dst.size
        step = -(-n // self.nthreads)
        parts = [(a, min(a + step, n)) for a in range(0, n, step)]
        list(self.pool.map(lambda ab: np.copyto(dst[ab[0]:ab[1]], src[ab[0]:ab[1]]), parts))

    def _staging(self, i, n):
        return np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(self.buf[i]))

    def to_device(self, dev_ptr, host):
        """host: a C-contiguous array; its bytes to dev_ptr."""
        src = host.reshape(-1).view(np.uint8)
        with self.lock:
            try:
                for k, a in enumerate(range(0, src.size, self.chunk)):
                    b = min(a + self.chunk, src.size)
                    i = k & 1
                    if k >= 2:
                        self.rt.wait(self.ev[i])  # the DMA of chunk k - 2 has read buffer i
                    self._host_copy(self._staging(i, b - a), src[a:b])
                    self.rt.copy_async(dev_ptr + a, self.buf[i], b - a, _H2D)
                    self.rt.record(self.ev[i])
            finally:  # no copy may still read the buffers once the lock is free
                self.rt.sync()

    def to_host(self, out, dev_ptr):
        """out: a C-contiguous array; its bytes from dev_ptr."""
        dst = out.reshape(-1).view(np.uint8)
        with self.lock:
            chunks = [(a, min(a + self.chunk, dst.size)) for a in range(0, dst.size, self.chunk)]
            try:
                for k, (a, b) in enumerate(chunks[:2]):
                    self.rt.copy_async(self.buf[k], dev_ptr + a, b - a, _D2H)
                    self.rt.record(self.ev[k])
                for k, (a, b) in enumerate(chunks):
                    i = k & 1
                    self.rt.wait(self.ev[i])
                    self._host_copy(dst[a:b], self._staging(i, b - a))
                    if k + 2 < len(chunks):  # buffer i is free again
                        a2, b2 = chunks[k + 2]
                        self.rt.copy_async(self.buf[i], dev_ptr + a2, b2 - a2, _D2H)
                        self.rt.record(self.ev[i])
            except BaseException:
                self.rt.sync()  # no copy may still write the buffers once the lock is free
                raise


class _Pool:
    """Device blocks by size class: powers of two below 1 MiB, multiples of
    2 MiB above.  Released blocks are kept up to `keep` bytes in all."""

    def __init__(self, rt, keep=64 << 30):
        self.rt, self.keep, self.cached = rt, keep, 0
        self.free = {}
        self.lock = threading.Lock()

    @staticmethod
    def size_class(n):
        n = max(int(n), 256)
        if n < (1 << 20):
            return 1 << (n - 1).bit_length()
        return -(-n // (2 << 20)) * (2 << 20)

    def take(self, n):
        c = self.size_class(n)
        with self.lock:
            lst = self.free.get(c)
            if lst:
                self.cached -= c
                return lst.pop(), c
        return self.rt.malloc(c), c

    def give(self, ptr, c):
        with self.lock:
            if self.cached + c <= self.keep:
                self.free.setdefault(c, []).append(ptr)
                self.cached += c
                return
        self.rt.free(ptr)


class _Block:
    """One pool block, returned to the pool when the last array using it is
    collected.  Work that still reads it was queued on the null stream
    before any later use of the block, so reuse on the null stream stays in
    order; a user that writes a block on another stream first synchronizes
    the null stream (matmul's two-halves path does)."""
    __slots__ = ("ptr", "cls", "__weakref__")

    def __init__(self, nbytes):
        self.ptr, self.cls = _pool().take(nbytes)

    def __del__(self):
        try:
            _pool().give(self.ptr, self.cls)
        except Exception:  # interpreter shutdown
            pass


class DeviceArray:
    """A device array of the NumPy family: a 2-D array has C-ordered rows
    with `ld` elements from one row to the next; other ranks are contiguous."""

    def __init__(self, shape, dtype=np.float64, ld=None, block=None, offset=0):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        if len(self.shape) == 2:
            rows, cols = self.shape
            self.ld = int(ld) if ld is not None else max(cols, 1)
            count = max(rows - 1, 0) * self.ld + cols if rows and cols else 0
        else:
            self.ld = None
            count = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = count * self.dtype.itemsize
        self._block = block if block is not None else _Block(max(self.nbytes, 1))
        self._offset = offset

    # the protocol the host layer uses (shared with torch tensors)
    def data_ptr(self):
        return self._block.ptr + self._offset

    def dim(self):
        return len(self.shape)

    @property
    def ndim(self):
        return len(self.shape)

    def numel(self):
        return int(np.prod(self.shape)) if self.shape else 1

    def stride(self, d):
        return (self.ld, 1)[d] if len(self.shape) == 2 else 1

    def element_size(self):
        return self.dtype.itemsize

    def column(self):
        """A 1-D array as its (n, 1) matrix (same memory)."""
        return DeviceArray((self.shape[0], 1), self.dtype, 1, self._block, self._offset)

    def flat(self):
        """An (n, 1) matrix as its 1-D array (same memory)."""
        return DeviceArray((self.shape[0],), self.dtype, None, self._block, self._offset)

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        assert d.nbytes == a.nbytes
        if a.nbytes >= _STAGE_MIN:
            _stager().to_device(d.data_ptr(), a)
        else:
            _rt().copy(d.data_ptr(), a.ctypes.data, a.nbytes, _H2D)
        return d

    def numpy(self):
        """Synchronising copy to a new NumPy array."""
        out = np.empty(self.shape, self.dtype)
        if out.size == 0:
            return out
        if self.dim() == 2 and self.ld != self.shape[1]:
            full = np.empty((self.shape[0], self.ld), self.dtype)
            _rt().copy(full.ctypes.data, self.data_ptr(), self.nbytes, _D2H)
            out[:] = full[:, :self.shape[1]]
        elif out.nbytes >= _STAGE_MIN:
            _stager().to_host(out, self.data_ptr())
        else:
            _rt().copy(out.ctypes.data, self.data_ptr(), out.nbytes, _D2H)
        return out

    @classmethod
    def zeros(cls, shape, dtype=np.float64):
        d = cls(shape, dtype)
        _rt().memset(d.data_ptr(), 0, d.nbytes)
        return d

    def copy_from(self, other):
        """Device-to-device copy of an array of the same shape and layout."""
        if other.shape != self.shape or other.nbytes != self.nbytes:
            raise ValueError("copy between arrays of different shape or layout")
        _rt().copy(self.data_ptr(), other.data_ptr(), self.nbytes, _D2D)


class _Blas:
    """rocBLAS FP64 products on the null stream.  Row-major matrices are
    column-major transposes, so C = A B is computed as C^T = B^T A^T."""

    def __init__(self):
        _rt()
        b = _open("librocblas.so.5")
        vp, i = ctypes.c_void_p, ctypes.c_int
        dp = ctypes.POINTER(ctypes.c_double)
        b.rocblas_create_handle.restype = i
        b.rocblas_create_handle.argtypes = [ctypes.POINTER(vp)]
        b.rocblas_set_stream.restype = i
        b.rocblas_set_stream.argtypes = [vp, vp]
        b.rocblas_dgemm.restype = i
        b.rocblas_dgemm.argtypes = [vp, i, i, i, i, i, dp, vp, i, vp, i, dp, vp, i]
        b.rocblas_dgeam.restype = i
        b.rocblas_dgeam.argtypes = [vp, i, i, i, i, dp, vp, i, dp, vp, i, vp, i]
        b.rocblas_destroy_handle.restype = i
        b.rocblas_destroy_handle.argtypes = [vp]
        h = vp()
        self._chk(b.rocblas_create_handle(ctypes.byref(h)), "rocblas_create_handle")
        self._chk(b.rocblas_set_stream(h, None), "rocblas_set_stream")
        self.b, self.h = b, h

    @staticmethod
    def _chk(rc, what):
        if rc != 0:
            raise _lib.OzakiError(f"{what} failed: rocblas status {rc}")

    @staticmethod
    def _c(x):
        return ctypes.byref(ctypes.c_double(x))

    def matmul(self, A, B, C, alpha=1.0, beta=0.0):
        """C = alpha A B + beta C (row-major A: N x K, B: K x M, C: N x M)."""
        N, K = A.shape
        M = B.shape[1]
        if N == 0 or M == 0:
            return C
        if K == 0:
            raise ValueError("contraction length 0")
        self._chk(self.b.rocblas_dgemm(self.h, _OP_N, _OP_N, M, N, K, self._c(alpha),
                                       B.data_ptr(), B.ld, A.data_ptr(), A.ld, self._c(beta),
                                       C.data_ptr(), C.ld), "rocblas_dgemm")
        return C

    def gram(self, A, G):
        """G = A^T A (row-major A: rows x cols, G: cols x cols)."""
        rows, cols = A.shape
        self._chk(self.b.rocblas_dgemm(self.h, _OP_N, _OP_T, cols, cols, rows, self._c(1.0),
                                       A.data_ptr(), A.ld, A.data_ptr(), A.ld, self._c(0.0),
                                       G.data_ptr(), G.ld), "rocblas_dgemm")
        return G

    def add(self, A, B, out):
        """out = A + B (row-major matrices of one shape; one rounding per
        element, as an FP64 add)."""
        n, m = A.shape
        if n and m:
            self._chk(self.b.rocblas_dgeam(self.h, _OP_N, _OP_N, m, n, self._c(1.0),
                                           A.data_ptr(), A.ld, self._c(1.0), B.data_ptr(),
                                           B.ld, out.data_ptr(), out.ld), "rocblas_dgeam")
        return out

    def half_sum_transpose(self, G, out):
        """out = G * 0.5 + G^T * 0.5, which equals (G + G^T) * 0.5 exactly
        (halving is exact, and one rounding of the same sum)."""
        n = G.shape[0]
        self._chk(self.b.rocblas_dgeam(self.h, _OP_N, _OP_T, n, n, self._c(0.5), G.data_ptr(),
                                       G.ld, self._c(0.5), G.data_ptr(), G.ld,
                                       out.data_ptr(), out.ld), "rocblas_dgeam")
        return out


_state = {}
# Re-entrant: a maker may create another singleton (the stager's and the
# pool's makers take the runtime), and any of them may be the first created.
_state_lock = threading.RLock()


def _get(name, make):
    v = _state.get(name)
    if v is None:
        with _state_lock:
            v = _state.get(name)
            if v is None:
                v = make()
                _state[name] = v
    return v


def _rt():
    return _get("rt", _Runtime)


def _release_at_exit():
    """At interpreter exit, before the runtime's own teardown: let queued
    work end, then release what this module holds in the runtime (the
    staging buffers and their events, the rocBLAS handle, the compute stream,
    the pool's cached blocks), so that none of it is left for the runtime's
    static destructors.  The runtime and the pool stay: blocks that arrays
    release later are freed at once.  Errors are ignored: the runtime may be
    unusable by then."""
    with _state_lock:
        st = dict(_state)
        for k in ("stager", "blas", "cstream"):
            _state.pop(k, None)
    rt = st.get("rt")
    if rt is None:
        return
    h = rt.h
    try:
        h.hipDeviceSynchronize()
        stager = st.get("stager")
        if stager is not None:
            stager.pool.shutdown(wait=True)
            for b in stager.buf:
                h.hipHostFree(b)
            for e in stager.ev:
                h.hipEventDestroy(e)
        blas_ = st.get("blas")
        if blas_ is not None:
            blas_.b.rocblas_destroy_handle(blas_.h)
        if st.get("cstream") is not None:
            h.hipStreamDestroy(st["cstream"])
        pool = st.get("pool")
        if pool is not None:
            with pool.lock:
                for ptrs in pool.free.values():
                    for ptr in ptrs:
                        h.hipFree(ptr)
                pool.free.clear()
                pool.cached = 0
                pool.keep = 0  # blocks released later are freed, not kept
        h.hipGetLastError()
    except Exception:
        pass


atexit.register(_release_at_exit)


def _pool():
    return _get("pool", lambda: _Pool(_rt()))


def _stager():
    return _get("stager", lambda: _Stager(_rt()))


def compute_stream():
    """The NumPy family's stream for work that overlaps its null-stream
    copies (kept for the process)."""
    return _get("cstream", lambda: _rt().nonblocking_stream())


def blas():
    return _get("blas", _Blas)


def device_count():
    return _rt().device_count()


def sync():
    _rt().sync()
