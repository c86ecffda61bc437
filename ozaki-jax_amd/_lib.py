"""ctypes binding of libozaki_amd.so (the C ABI declared in include/ozaki_amd.h).

The library is built in-tree by ``__graft_entry__.build()`` (or
``make -C ozaki-jax_amd/csrc``).  There is no fallback: if the shared library
is missing or fails to load, every entry point raises ``RuntimeError``.
"""

import ctypes
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libozaki_amd.so"

OZK_OK = 0
OZK_ERR_INVALID = -1
OZK_ERR_HIP = -2
OZK_ERR_UNSUPPORTED = -3
OZK_ERR_WORKSPACE = -4
OZK_FLAG_NONFINITE = 1
OZK_FLAG_WAIT_TIMEOUT = 2
OZK_FLAG_SINGULAR = 4
OZK_FLAG_INF_SLICE = 8
OZK_EXP_NONFINITE = -2 ** 31

ORDER_2SUM = 0       # A4  pallas_ops.py:178-239
ORDER_BLOCK64 = 1    # A3  matmul.py:543-597
ORDER_HOST_JAX = 2   # A2  matmul.py:35-64
ORDER_HOST_NP = 3    # A1  matmul.py:879-898

PIPE_ONDEVICE = 0
PIPE_HOST = 1
PIPE_ONDEVICE_BF16 = 2  # ozk_matmul only: on-device pipeline, BF16 planes at any K


def check_flags(fl):
    """Raise if a kernel's bounded wait gave up (OZK_FLAG_WAIT_TIMEOUT): the
    results of that call are not valid.  Returns the flag word."""
    if fl & OZK_FLAG_WAIT_TIMEOUT:
        raise RuntimeError("ozaki_amd: a bounded wait between workgroups gave up "
                           "(OZK_FLAG_WAIT_TIMEOUT); the result is not valid")
    return fl


# Calls repeated without extraction gangs after OZK_FLAG_WAIT_TIMEOUT.
gang_retries = 0


def with_gang_retry(call):
    """Run call() -> flag word.  When the extraction gangs' waits gave up
    (other work held the CUs that a gang needed), run it once more with the
    gangs switched off for this thread (ozk_set_gangs(0): transposed columns
    and streamed rows, no waits between workgroups; the same bits), then
    raise on the flag as check_flags does.  call() must query its workspace
    size itself, since the gang-free path needs a larger one."""
    global gang_retries
    fl = call()
    if fl & OZK_FLAG_WAIT_TIMEOUT:
        lib = load()
        gang_retries += 1
        lib.ozk_set_gangs(0)
        try:
            fl = call()
        finally:
            lib.ozk_set_gangs(1)
    return check_flags(fl)

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_c_vp = ctypes.c_void_p

# name -> (restype, argtypes); must match include/ozaki_amd.h exactly.
SIGNATURES = {
    "ozk_last_error": (ctypes.c_char_p, []),
    "ozk_abi_version": (_c_int, []),
    "ozk_set_wait_polls": (None, [ctypes.c_uint32]),
    "ozk_set_gangs": (None, [_c_int]),
    "ozk_device_info": (_c_int, [ctypes.c_char_p, _c_size, ctypes.POINTER(_c_int)]),
    "ozk_rho_f64": (_c_int, [_c_i64]),
    "ozk_rho_f32": (_c_int, [_c_i64]),
    "ozk_slice_ld": (_c_i64, [_c_i64]),
    "ozk_slice_lines": (_c_i64, [_c_i64]),
    "ozk_extract_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_int]),
    "ozk_extract_f32": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                 _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp,
                                 _c_size, _c_vp]),
    "ozk_extract_f32_i8": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                    _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                    _c_size, _c_vp]),
    "ozk_extract_f64": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                 _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_size,
                                 _c_vp]),
    "ozk_pair_count": (_c_int, [_c_int, _c_int, _c_int]),
    "ozk_gemm_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_int, _c_int, _c_int,
                                           _c_int]),
    "ozk_gemm": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                          _c_int, _c_int, _c_int, _c_int, _c_vp, _c_i64, _c_vp,
                          _c_size, _c_vp]),
    "ozk_gemm_i8": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64,
                             _c_i64, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_i64, _c_vp,
                             _c_size, _c_vp]),
    "ozk_gemm_2sum_pair": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64,
                                    _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_vp,
                                    _c_vp, _c_i64, _c_vp, _c_size, _c_vp]),
    "ozk_slice_products_i8": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                       _c_int, _c_int, _c_int, _c_vp, _c_i64, _c_vp]),
    "ozk_slice_products": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int,
                                    _c_int, _c_int, _c_vp, _c_i64, _c_vp]),
    "ozk_matmul_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_int,
                                             _c_int, _c_int]),
    "ozk_matmul_plane_bytes": (_c_int, [_c_int, _c_i64, _c_int, _c_int]),
    "ozk_matmul": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64,
                            _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
                            _c_vp, _c_size, _c_vp, _c_vp]),
    "ozk_matmul_early_flags": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,
                                        _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int,
                                        _c_int, _c_vp, _c_size, _c_vp, _c_vp, _c_vp,
                                        _c_vp]),
    "ozk_matmul_noalloc": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64,
                                    _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                    _c_vp, _c_vp]),
    "ozk_gram_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_int, _c_int]),
    "ozk_gram": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_vp,
                          _c_i64, _c_vp, _c_size, _c_vp, _c_vp]),
    "ozk_gram_early_flags": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                                      _c_vp, _c_i64, _c_vp, _c_size, _c_vp, _c_vp, _c_vp,
                                      _c_vp]),
    "ozk_residual_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_int,
                                               _c_int]),
    "ozk_residual": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp,
                              _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                              _c_vp, _c_size, _c_vp, _c_vp]),
    "ozk_lu_factor_max_n": (_c_i64, []),
    "ozk_lu_factor_workspace_bytes": (_c_size, [_c_i64]),
    "ozk_lu_factor_f32": (_c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_size, _c_vp,
                                   _c_vp]),
    "ozk_lu_solve_workspace_bytes": (_c_size, [_c_i64, _c_i64]),
    "ozk_lu_solve_f32": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp,
                                  _c_i64, _c_i64, _c_vp, _c_size, _c_vp, _c_vp]),
    "ozk_pivots_to_perm": (_c_int, [_c_vp, _c_i64, _c_vp]),
    "ozk_check_finite": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp]),
    "ozk_accumulate_2sum": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp,
                                     _c_vp, _c_int, _c_vp, _c_int, _c_vp, _c_vp,
                                     _c_vp]),
    "ozk_probe_mfma_layout": (_c_int, [_c_vp, _c_vp]),
}

_lib = None
_load_error = None


def load():
    """Load and bind the shared library once; raise RuntimeError if absent."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if _load_error is not None:
        raise RuntimeError(_load_error)
    path = os.environ.get("OZAKI_AMD_LIB", str(LIB_PATH))
    try:
        lib = ctypes.CDLL(path)
    except OSError as exc:
        _load_error = (f"ozaki_jax_amd: cannot load the HIP library {path} "
                       f"({exc}); build it with __graft_entry__.build() or "
                       f"`make -C ozaki-jax_amd/csrc`.  There is no CPU path.")
        raise RuntimeError(_load_error) from None
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class OzakiError(RuntimeError):
    """A non-argument failure reported by the HIP library."""


def check(rc):
    """Map a C status code to a Python exception."""
    if rc >= 0:
        return rc
    msg = _lib.ozk_last_error().decode(errors="replace") if _lib else ""
    if rc == OZK_ERR_INVALID:
        raise ValueError(msg)
    if rc == OZK_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise OzakiError(f"ozaki HIP library error {rc}: {msg}")
