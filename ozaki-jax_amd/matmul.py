"""FP64-accurate matrix multiplication via the Ozaki scheme on MI355X.

Host-side mirror of ``ozaki_jax/matmul.py``: the same functions, arguments,
defaults, validation order and error messages, with every computation done by
the HIP kernels of libozaki_amd.so.

Array families.  The reference accepts NumPy or JAX arrays; here the second
family is PyTorch tensors.  NumPy in -> NumPy out; torch in -> torch (on the
GPU) out for pipeline='ondevice'; the host pipeline always returns NumPy
(matmul.py:826-851); mixed families raise ValueError (matmul.py:803-808).
"""

import numpy as np

from . import _device as D
from . import _hip
from . import _lib
from .extract import rho_f32, rho_f64

# matmul.py:168-172
_PRECISION_PRESETS = {
    "high": (4, 1),    # 24 GEMMs
    "medium": (3, 1),  # 15 GEMMs
    "max": (5, 4),     # 65 GEMMs
}

_ACCUMULATION_MODES = {"fused", "bf16_interleaved", "ondevice", "host"}


def _resolve_precision(precision):
    """matmul.py:175-194: preset name or a custom (n_hi, n_lo) tuple."""
    if isinstance(precision, tuple) and len(precision) == 2:
        n_hi, n_lo = precision
        if n_hi < 1 or n_lo < 1:
            raise ValueError(
                f"Custom precision tuple must have n_hi >= 1 and n_lo >= 1, "
                f"got ({n_hi}, {n_lo}).")
        return precision
    if precision not in _PRECISION_PRESETS:
        raise ValueError(
            f"Unknown precision={precision!r}; expected one of "
            f"{sorted(_PRECISION_PRESETS)} or a (n_hi, n_lo) tuple.")
    return _PRECISION_PRESETS[precision]


def _validate_accumulation_mode(accumulation):
    """matmul.py:138-144."""
    if accumulation not in _ACCUMULATION_MODES:
        raise ValueError(
            f"Unknown accumulation={accumulation!r}; expected one of "
            f"{sorted(_ACCUMULATION_MODES)}.")


def _validate_shapes(A, B):
    """matmul.py:67-74."""
    if A.ndim != 2 or B.ndim != 2:
        raise ValueError("Inputs must be rank-2 matrices.")
    if A.shape[1] != B.shape[0]:
        raise ValueError(
            f"Incompatible shapes for matmul: {tuple(A.shape)} and "
            f"{tuple(B.shape)}.")


def _kbound_reasons(K, bits, too_large):
    """Exactness-bound part of the preflight (matmul.py:89-100, :609-621)."""
    reasons = []
    if bits <= 0:
        reasons.append(
            f"non-positive bits per slice ({bits}); K={K} is too {too_large}")
    elif K * (2 ** bits - 1) ** 2 >= 2 ** 24:
        max_K = int(2 ** 24 / (2 ** bits - 1) ** 2)
        reasons.append(
            f"K={K} violates BF16->FP32 exact inner-product bound "
            f"(need K <= {max_K})")
    return reasons


def _check_safe_mode(safe_mode):
    """matmul.py:121-125."""
    allowed = {"raise", "fallback"}
    if safe_mode not in allowed:
        raise ValueError(
            f"Invalid safe_mode={safe_mode!r}; expected one of "
            f"{sorted(allowed)}.")


def _nonfinite(fam, tensors):
    """np.isfinite(...).all() on the device (matmul.py:108-109, :623-628)."""
    lib = _lib.load()
    flags = fam.zero_flags()
    for t in tensors:
        if t.numel() == 0:
            continue
        _lib.check(lib.ozk_check_finite(t.data_ptr(), t.shape[0], t.shape[1],
                                        D.ld_of(t), flags.data_ptr(), fam.stream()))
    return fam.read_flags(flags) & _lib.OZK_FLAG_NONFINITE


def _unsafe(fam, reasons, safe_mode, At, Bt):
    """matmul.py:127-135 once the reasons are known.  The fallback result is
    the plain FP64 product, computed on the GPU by rocBLAS DGEMM."""
    if not reasons:
        return None
    if safe_mode == "fallback":
        return fam.matmul(At, Bt)
    raise ValueError("Ozaki preflight marked this input as unsafe: "
                     + "; ".join(reasons))


def _run_matmul(fam, At, Bt, pipeline, n_hi, n_lo, order):
    """ozk_matmul on device arrays; returns (C, nonfinite flag).

    INT8 slice planes (K > 4096) store a slice that the reference's
    extraction makes non-finite as zeros with a NaN scale.  In the FP64 block
    order (accumulation='host') a slice of +-inf can give C = +-inf where
    that folds to NaN; the library flags such slices, and the call is then
    repeated on BF16 planes, which hold the infinities themselves."""
    lib = _lib.load()
    N, K = At.shape
    M = Bt.shape[1]
    C = fam.empty((N, M))
    if N == 0 or M == 0:
        return C, 0
    flags = fam.flags()  # cleared by the call
    early = getattr(fam, "early_flags", None)

    def once(pipe):
        wsb = lib.ozk_matmul_workspace_bytes(N, K, M, pipe, n_hi, n_lo)
        ws = fam.workspace(wsb)
        args = (At.data_ptr(), D.ld_of(At), Bt.data_ptr(), D.ld_of(Bt), C.data_ptr(),
                D.ld_of(C), N, K, M, pipe, n_hi, n_lo, order, ws.data_ptr(), wsb,
                flags.data_ptr())
        if early is None:
            _lib.check(lib.ozk_matmul(*args, fam.stream()))
            return fam.read_flags(flags)
        # torch tensors: the flags are read once the extraction has run, and
        # C is returned while the GEMM is still queued on the current stream
        word, ev, read = early()
        _lib.check(lib.ozk_matmul_early_flags(*args, word, ev, fam.stream()))
        return read()

    def run(pipe):
        return _lib.with_gang_retry(lambda: once(pipe))

    fl = run(pipeline)
    if (fl & _lib.OZK_FLAG_INF_SLICE and order == _lib.ORDER_BLOCK64
            and pipeline == _lib.PIPE_ONDEVICE):
        fl = run(_lib.PIPE_ONDEVICE_BF16)
    return C, fl & _lib.OZK_FLAG_NONFINITE


def _matmul_ondevice(fam, At, Bt, safe_mode, accumulation, n_hi, n_lo):
    """matmul.py:641-728: preflight, then split + FP32 extraction + fused
    slice GEMMs with the accumulation order of `accumulation`
    ('fused' / 'bf16_interleaved' / 'ondevice' -> 2Sum A4; 'host' -> A3)."""
    _validate_accumulation_mode(accumulation)
    _validate_shapes(At, Bt)
    K = At.shape[1]
    if K == 0:
        raise ValueError("zero-size array to reduction operation maximum "
                         "which has no identity")
    bits = 24 - rho_f32(K)
    reasons = _kbound_reasons(K, bits, "large for FP32 extraction")
    _check_safe_mode(safe_mode)
    if reasons:
        if _nonfinite(fam, (At, Bt)):
            reasons.append("inputs contain NaN or Inf")
        return _unsafe(fam, reasons, safe_mode, At, Bt)
    order = _lib.ORDER_BLOCK64 if accumulation == "host" else _lib.ORDER_2SUM
    C, bad = _run_matmul(fam, At, Bt, _lib.PIPE_ONDEVICE, n_hi, n_lo, order)
    if bad:
        return _unsafe(fam, ["inputs contain NaN or Inf"], safe_mode, At, Bt)
    return C


def _numpy_halves_ok(A, B):
    """NumPy operands for which the two-halves form pays: each half of A and
    of C at least _hip._STAGE_MIN bytes (the staged copies)."""
    if not (isinstance(A, np.ndarray) and isinstance(B, np.ndarray)
            and A.ndim == 2 and B.ndim == 2 and A.shape[1] == B.shape[0]):
        return False
    N, K = A.shape
    M = B.shape[1]
    half = 8 * (N // 2)
    return N >= 256 and half * K >= _hip._STAGE_MIN and half * M >= _hip._STAGE_MIN


def _matmul_ondevice_numpy(fam, A, B, safe_mode, accumulation, n_hi, n_lo):
    """_matmul_ondevice for large NumPy operands, as two ozk_matmul calls on
    the row halves of A on a stream of their own.  The second half's upload
    runs while the first half computes, and the first half's download while
    the second computes; B is uploaded once.  A's slice lines are its rows,
    so each half's slices, products and folds are those of the whole call,
    bit for bit.  Calls that the preflight marks, or whose flags ask for a
    rerun or a fallback (or whose extraction gangs gave up), take the
    one-call path."""
    A = np.ascontiguousarray(A, dtype=np.float64)
    B = np.ascontiguousarray(B, dtype=np.float64)
    _validate_accumulation_mode(accumulation)
    _validate_shapes(A, B)
    N, K = A.shape
    M = B.shape[1]
    _check_safe_mode(safe_mode)

    def whole():
        return _matmul_ondevice(fam, fam.f64(A), fam.f64(B), safe_mode, accumulation,
                                n_hi, n_lo).numpy()

    if _kbound_reasons(K, 24 - rho_f32(K), "large for FP32 extraction"):
        return whole()
    order = _lib.ORDER_BLOCK64 if accumulation == "host" else _lib.ORDER_2SUM
    lib, rt, st = _lib.load(), _hip._rt(), _hip.compute_stream()
    h = (N // 2 + 63) // 64 * 64
    Bt = fam.f64(B)
    held, done = [Bt], []
    out = np.empty((N, M))
    fl = 0
    try:
        for r0, r1 in ((0, h), (h, N)):
            At = fam.f64(A[r0:r1])  # null stream: overlaps the previous half's kernels
            C = fam.empty((r1 - r0, M))
            flags = fam.flags()
            wsb = lib.ozk_matmul_workspace_bytes(r1 - r0, K, M, _lib.PIPE_ONDEVICE, n_hi, n_lo)
            ws = fam.workspace(wsb)
            held += [At, C, flags, ws]
            # Pool blocks are reused in null-stream order; work queued there
            # before these blocks were taken (another thread's product that
            # still reads a block it released) must end before the compute
            # stream writes them.
            rt.sync()
            _lib.check(lib.ozk_matmul(
                At.data_ptr(), D.ld_of(At), Bt.data_ptr(), D.ld_of(Bt), C.data_ptr(),
                D.ld_of(C), r1 - r0, K, M, _lib.PIPE_ONDEVICE, n_hi, n_lo, order,
                ws.data_ptr(), wsb, flags.data_ptr(), st))
            ev = rt.event()
            done.append((r0, r1, C, flags, ev))
            rt.record(ev, st)
        for r0, r1, C, flags, ev in done:
            rt.wait(ev)  # then the download (null stream) overlaps the next half
            _hip._stager().to_host(out[r0:r1], C.data_ptr())
            fl |= fam.read_flags(flags)
    finally:
        rt.sync(st)  # no kernel may still use a block once it is released
        for *_, ev in done:
            rt.destroy_event(ev)
    if fl & _lib.OZK_FLAG_WAIT_TIMEOUT or fl & _lib.OZK_FLAG_NONFINITE or (
            fl & _lib.OZK_FLAG_INF_SLICE and order == _lib.ORDER_BLOCK64):
        return whole()  # repeats a call whose gangs gave up without them
    return out


def _matmul_host(fam, At, Bt, n_slices, safe_mode, order):
    """matmul.py:826-851 / :866-900: FP64 extraction (rho from
    `_compute_rho`), triangular slice pairs i + j <= n_slices - 1, FP64
    accumulation in order A2 (matmul) or A1 (matmul_numpy)."""
    if n_slices < 1:
        raise ValueError("n_slices must be >= 1.")
    _validate_shapes(At, Bt)
    K = At.shape[1]
    if K == 0:
        raise ValueError("zero-size array to reduction operation maximum "
                         "which has no identity")
    bits = 53 - rho_f64(K)
    reasons = _kbound_reasons(
        K, bits, "large for this BF16->FP32 exactness model")
    if n_slices * max(bits, 0) < 53:
        reasons.append(f"insufficient slice budget: n_slices*bits_per_slice="
                       f"{n_slices * max(bits, 0)} < 53")
    _check_safe_mode(safe_mode)
    if reasons:
        if _nonfinite(fam, (At, Bt)):
            reasons.append("inputs contain NaN or Inf")
        return _unsafe(fam, reasons, safe_mode, At, Bt)
    if n_slices > 32:
        raise NotImplementedError("n_slices > 32 is not supported")
    C, bad = _run_matmul(fam, At, Bt, _lib.PIPE_HOST, n_slices, 0, order)
    if bad:
        return _unsafe(fam, ["inputs contain NaN or Inf"], safe_mode, At, Bt)
    return C


def _families(A, B):
    a_t, b_t = D.is_torch(A), D.is_torch(B)
    if a_t != b_t:
        raise ValueError(
            "A and B must both be numpy arrays or both be torch tensors.")
    return a_t


def matmul(A, B, n_slices=8, safe_mode="raise", pipeline="host",
           accumulation="fused", precision="high"):
    """FP64 matmul via Ozaki Extract (matmul.py:781-851).

    pipeline='host': FP64 extraction, n_slices slices per operand, triangular
    pairs, FP64 accumulation (order of `_accumulate_products`); returns NumPy.
    pipeline='ondevice': FP64 -> FP32 hi/lo split, FP32 extraction with
    `precision` ('high' (4,1) 24 GEMMs, 'medium' (3,1) 15, 'max' (5,4) 65, or
    a custom (n_hi, n_lo)), one fused kernel for the slice GEMMs and the
    accumulation (`accumulation`: 'fused', 'bf16_interleaved', 'ondevice' ->
    double-float 2Sum; 'host' -> FP64 block accumulation); output family
    follows the input family.
    """
    want_torch = _families(A, B)
    fam = D.family(want_torch)
    if pipeline == "ondevice":
        n_hi, n_lo = _resolve_precision(precision)
        if not want_torch and _numpy_halves_ok(A, B):
            return _matmul_ondevice_numpy(fam, A, B, safe_mode, accumulation, n_hi, n_lo)
        At, Bt = fam.f64(A), fam.f64(B)
        C = _matmul_ondevice(fam, At, Bt, safe_mode, accumulation, n_hi, n_lo)
        return fam.out(C, want_torch)
    if pipeline != "host":
        raise ValueError(
            f"Unknown pipeline={pipeline!r}; expected 'host' or 'ondevice'.")
    At, Bt = fam.f64(A), fam.f64(B)
    C = _matmul_host(fam, At, Bt, n_slices, safe_mode, _lib.ORDER_HOST_JAX)
    return fam.out(C, False)


def matmul_numpy(A_f64, B_f64, n_slices=8, safe_mode="raise", pipeline="host",
                 precision="high"):
    """`matmul_numpy` (matmul.py:854-900): the results of the reference's
    NumPy pipeline -- accumulation order A1 for pipeline='host' and A3
    (`_accumulate_block_products`) for 'ondevice' -- computed by the same
    GPU kernels.  Accepts array-likes; returns NumPy."""
    want_torch = D.is_torch(A_f64) and D.is_torch(B_f64)
    fam = D.family(want_torch)
    if pipeline == "ondevice" and not want_torch and _numpy_halves_ok(A_f64, B_f64):
        n_hi, n_lo = _resolve_precision(precision)
        return _matmul_ondevice_numpy(fam, A_f64, B_f64, safe_mode, "host", n_hi, n_lo)
    At, Bt = fam.f64(A_f64), fam.f64(B_f64)
    if pipeline == "ondevice":
        n_hi, n_lo = _resolve_precision(precision)
        C = _matmul_ondevice(fam, At, Bt, safe_mode, "host", n_hi, n_lo)
        return fam.out(C, False)
    if pipeline != "host":
        raise ValueError(
            f"Unknown pipeline={pipeline!r}; expected 'host' or 'ondevice'.")
    C = _matmul_host(fam, At, Bt, n_slices, safe_mode, _lib.ORDER_HOST_NP)
    return fam.out(C, False)
