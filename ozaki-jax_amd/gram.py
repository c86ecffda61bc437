"""FP64-accurate Gram matrix A^T @ A (mirror of ``ozaki_jax/gram.py``).

mode='ozaki' runs the Ozaki pipeline on the GPU: one column extraction of A
serves as both operands (row extraction of A^T equals column extraction of
A), the fused slice-pair kernel accumulates in the 2Sum order, and the result
is symmetrised as (G + G^T) * 0.5 (gram.py:19-37).  mode='f64' is the plain
FP64 product (gram.py:40-44), computed by rocBLAS DGEMM.
"""

from . import _device as D
from . import _lib
from .extract import rho_f32
from .matmul import _resolve_precision


def gram(A, precision="high", accumulation="bf16_interleaved", mode="f64"):
    """gram.py:47-99.  Returns the symmetric (K, K) matrix in A's family."""
    allowed_modes = {"f64", "ozaki"}
    if mode not in allowed_modes:
        raise ValueError(
            f"mode={mode!r}; expected one of {sorted(allowed_modes)}.")
    if mode == "ozaki":
        allowed_accum = {"bf16_interleaved", "fused"}
        if accumulation not in allowed_accum:
            raise ValueError(
                f"accumulation={accumulation!r}; expected one of "
                f"{sorted(allowed_accum)}.")
    if A.ndim != 2:
        raise ValueError(f"A must be 2D, got ndim={A.ndim}.")
    want_torch = D.is_torch(A)
    fam = D.family(want_torch)
    At = fam.f64(A)
    rows, cols = At.shape
    if mode == "f64":
        return fam.out(fam.gram_f64(At), want_torch)
    n_hi, n_lo = _resolve_precision(precision)
    lib = _lib.load()
    G = fam.empty((cols, cols))
    if cols == 0:
        return fam.out(G, want_torch)
    if rows == 0:
        raise ValueError("zero-size array to reduction operation maximum "
                         "which has no identity")
    # A NaN / Inf in A gives NaN rows and columns of G, as in the reference,
    # which runs no preflight here; the flag word is read only for
    # OZK_FLAG_WAIT_TIMEOUT.
    flags = fam.flags()
    early = getattr(fam, "early_flags", None)

    def once():
        wsb = lib.ozk_gram_workspace_bytes(rows, cols, n_hi, n_lo)
        ws = fam.workspace(wsb)
        args = (At.data_ptr(), D.ld_of(At), rows, cols, n_hi, n_lo, G.data_ptr(),
                D.ld_of(G), ws.data_ptr(), wsb, flags.data_ptr())
        if early is None:
            _lib.check(lib.ozk_gram(*args, fam.stream()))
            return fam.read_flags(flags)
        # torch tensors: the flags are read once the extraction has run; G is
        # returned while the GEMM is still queued on the current stream
        word, ev, read = early()
        _lib.check(lib.ozk_gram_early_flags(*args, word, ev, fam.stream()))
        return read()

    _lib.with_gang_retry(once)
    return fam.out(G, want_torch)


__all__ = ["gram", "rho_f32"]
