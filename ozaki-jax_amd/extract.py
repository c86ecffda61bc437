"""Slice extraction (Ozaki "Extract" sigma trick) on the GPU.

Mirrors the public helpers of ``ozaki_jax/extract.py``.  All six run the HIP
extraction kernels:

  extract_split_rows / extract_split_cols        FP64 path (extract.py:21-103)
  f32_extract_split_rows / f32_extract_split_cols FP32 path (extract.py:116-191)
  jax_extract_split_rows / jax_extract_split_cols stacked FP32 results
                                                  (extract.py:197-286)

Slices come back as float32 arrays (BF16-exact values), exponents as float
arrays (float64 for the FP64 path, float32 for the FP32 path), like the
reference.  NumPy inputs need only NumPy, as in the reference: their device
arrays come from the HIP runtime (``_hip``) and the planes are unpacked on
the host.  Torch tensors stay on torch's device and stream.
"""

import numpy as np

from . import _device as D
from . import _lib
from .lowlevel import CHUNK_BYTES, Planes, unit_swizzle


def _rho(K, m1):
    """max(ceil(m1 - (24 - ceil(log2 max(K, 2))) / 2), m1 + 1 - 8)."""
    k = max(int(K), 2)
    clog2 = (k - 1).bit_length()
    num = 2 * m1 - 24 + clog2
    return max(-((-num) // 2), m1 + 1 - 8)


def rho_f64(K):
    """extract.py:12-18 `_compute_rho` (m1=53, m2=8, m3=24)."""
    return _rho(K, 53)


def rho_f32(K):
    """extract.py:109-113 `_compute_rho_f32` (m1=24, m2=8, m3=24)."""
    return _rho(K, 24)


_compute_rho = rho_f64
_compute_rho_f32 = rho_f32


def _grid_numpy(s):
    """Host form of lowlevel.Planes.grid: chunk-major BF16 planes (P, L, ld)
    int16, the four 16-byte units of a line's chunk stored in the order
    u ^ unit_swizzle(line), as (P, L, ld) line-major."""
    P, L, ld = s.shape
    nch = ld * s.itemsize // CHUNK_BYTES
    raw = np.ascontiguousarray(s).reshape(-1).view(np.uint8).reshape(P, nch, L, 4, 16)
    r = np.arange(L)
    stored = np.arange(4)[None, :] ^ unit_swizzle(r)[:, None]
    raw = raw[:, :, r[:, None], stored, :]
    raw = raw.transpose(0, 2, 1, 3, 4).reshape(P, L, nch * CHUNK_BYTES)
    return np.ascontiguousarray(raw).view(s.dtype).reshape(P, L, ld)


def _extract(X, rho, n_slices, by_cols, f64):
    """Run one extraction on the device; return (slices (n, r, c) float32
    in the input orientation, exponents (n, lines) int32, input is torch),
    as torch tensors for torch input and NumPy arrays otherwise."""
    lib = _lib.load()
    want_torch = D.is_torch(X)
    fam = D.family(want_torch)
    if f64:
        Xt = fam.f64(X)
    elif want_torch:
        # FP32 input: widen exactly; the split then gives hi = X, lo = 0.
        Xt = fam.f64(X.to(D.torch.float32))
    else:
        Xt = fam.f64(np.asarray(X, dtype=np.float32))
    if Xt.dim() != 2:
        raise ValueError("expected a 2-D matrix")
    rows, cols = Xt.shape
    if (cols if not by_cols else rows) == 0 and (rows if not by_cols else cols) > 0:
        raise ValueError("zero-size array to reduction operation maximum "
                         "which has no identity")
    lines, length = (cols, rows) if by_cols else (rows, cols)
    lp = lib.ozk_slice_lines(max(lines, 1))
    ld = lib.ozk_slice_ld(max(length, 1))
    S = fam.zeros((n_slices, lp, ld), np.int16)
    E = fam.zeros((n_slices, lp), np.int32)
    if rows and cols:
        def once():
            flags = fam.zero_flags()  # the extraction entry points OR into the word
            wsb = lib.ozk_extract_workspace_bytes(rows, cols, int(by_cols))
            ws = fam.workspace(wsb)
            if f64:
                rc = lib.ozk_extract_f64(Xt.data_ptr(), rows, cols, D.ld_of(Xt),
                                         int(by_cols), int(rho), n_slices,
                                         S.data_ptr(), E.data_ptr(),
                                         flags.data_ptr(), ws.data_ptr(), wsb,
                                         fam.stream())
            else:
                rc = lib.ozk_extract_f32(Xt.data_ptr(), rows, cols, D.ld_of(Xt),
                                         int(by_cols), int(rho), n_slices, 0,
                                         S.data_ptr(), E.data_ptr(),
                                         flags.data_ptr(), ws.data_ptr(), wsb,
                                         fam.stream())
            _lib.check(rc)
            return fam.read_flags(flags)

        _lib.with_gang_retry(once)
    if want_torch:
        # chunk-major BF16 planes -> float32 values; back to the input orientation
        vals = Planes(S, E, lines, length, None).values()
        if by_cols:
            vals = vals.transpose(1, 2)
        return vals.contiguous(), E[:, :lines], True
    g = _grid_numpy(S.numpy())[:, :lines, :length]
    vals = (g.astype(np.int32) << 16).view(np.float32)
    if by_cols:
        vals = vals.transpose(0, 2, 1)
    return np.ascontiguousarray(vals), E.numpy()[:, :lines], False


def _as_lists(vals, E, want_torch, exp_dtype):
    n = vals.shape[0]
    if want_torch:
        return ([vals[i] for i in range(n)],
                [E[i].to(getattr(D.torch, exp_dtype)) for i in range(n)])
    e = E.astype(exp_dtype)
    return [vals[i] for i in range(n)], [e[i] for i in range(n)]


def extract_split_rows(X_f64, rho, n_slices=8):
    """extract.py:21-65: FP64 row extraction."""
    v, e, t = _extract(X_f64, rho, n_slices, False, True)
    return _as_lists(v, e, t, "float64")


def extract_split_cols(X_f64, rho, n_slices=8):
    """extract.py:68-103: FP64 column extraction."""
    v, e, t = _extract(X_f64, rho, n_slices, True, True)
    return _as_lists(v, e, t, "float64")


def f32_extract_split_rows(X_f32, rho, n_slices=5):
    """extract.py:116-154: FP32 row extraction."""
    v, e, t = _extract(X_f32, rho, n_slices, False, False)
    return _as_lists(v, e, t, "float32")


def f32_extract_split_cols(X_f32, rho, n_slices=5):
    """extract.py:157-191: FP32 column extraction."""
    v, e, t = _extract(X_f32, rho, n_slices, True, False)
    return _as_lists(v, e, t, "float32")


def jax_extract_split_rows(X_f32, rho, n_slices=5):
    """extract.py:197-242: stacked (n, N, K) slices and (n, N) exponents."""
    v, e, t = _extract(X_f32, rho, n_slices, False, False)
    if t:
        return v, e.to(D.torch.float32)
    return v, e.astype(np.float32)


def jax_extract_split_cols(X_f32, rho, n_slices=5):
    """extract.py:245-286: stacked (n, K, M) slices and (n, M) exponents."""
    v, e, t = _extract(X_f32, rho, n_slices, True, False)
    if t:
        return v, e.to(D.torch.float32)
    return v, e.astype(np.float32)
