"""ozaki_jax_amd: the Ozaki-scheme FP64 matmul of ozaki-jax, MI355X-native.

Drop-in for the hot path of ozaki_jax (``ozaki_jax/__init__.py:5-25``):
``matmul``, ``matmul_numpy``, ``gram``, ``residual``, ``solve``, ``inv``,
``lstsq``, ``norm``, the ``*extract_split_*`` helpers and
``accumulate_2sum`` / ``validate_accumulation_2sum``, same signatures and
defaults.  Every
Ozaki computation runs in hand-written HIP kernels for gfx950
(libozaki_amd.so, C ABI in include/ozaki_amd.h), bound with ctypes.  NumPy
in -> NumPy out: NumPy inputs take device memory from the HIP runtime and
FP64 products from rocBLAS, both through ctypes, so matmul, matmul_numpy,
gram, residual, the extraction helpers, solve and inv (n up to
ozk_lu_factor_max_n()) and norm need no PyTorch.  Torch tensors (PyTorch-ROCm
memory and current stream) play the role of the reference's JAX arrays;
lstsq and larger solves use torch.linalg for their FP32 factorisations.
"""

__version__ = "0.7.0"

from .matmul import matmul, matmul_numpy  # noqa: F401
from .gram import gram  # noqa: F401
from .solve import residual, solve  # noqa: F401
from .inv import inv  # noqa: F401
from .lstsq import lstsq  # noqa: F401
from .norm import norm  # noqa: F401
from .accumulate import accumulate_2sum, validate_accumulation_2sum  # noqa: F401
from .extract import (  # noqa: F401
    extract_split_rows, extract_split_cols,
    f32_extract_split_rows, f32_extract_split_cols,
    jax_extract_split_rows, jax_extract_split_cols,
    rho_f32, rho_f64,
)

__all__ = [
    "gram", "matmul", "matmul_numpy", "residual", "solve",
    "inv", "lstsq", "norm",
    "extract_split_rows", "extract_split_cols",
    "f32_extract_split_rows", "f32_extract_split_cols",
    "jax_extract_split_rows", "jax_extract_split_cols",
    "accumulate_2sum", "validate_accumulation_2sum",
]
