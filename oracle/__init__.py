"""CPU oracle for the Ozaki-scheme matmul path -- TEST INFRASTRUCTURE ONLY.

This package is a NumPy restatement of the reference's (Efithor/ozaki-jax)
arithmetic for the Ozaki-scheme FP64 matmul: the FP64 -> FP32 hi/lo split, the
sigma-trick slice extraction (FP32 and FP64), the slice-pair products and the
four accumulation orders, plus gram / residual / solve on top of them.  Every
function cites the reference file:line it restates.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import it, and only to check results against.  The product (``ozaki_jax_amd``) never
imports, links or executes anything under ``oracle/``.

How each part is pinned (a check that a plausible mistake would fail):
  * rho / presets / pair schedule: closed forms plus the reference's own
    tables (ondevice_validate.py:139-140, test_pallas_fused.py:26-50).
  * split: hi + lo reconstructs x to < 2^-47 relative; lo is the exact FP32
    rounding of x - hi (checked with exact rationals on samples).
  * extraction: sum_s slice_s * 2^c_s + final residual == input exactly,
    slices BF16-exact, |slice| <= 2, grid 2^(rho-p); exponent rule checked
    exhaustively over all positive float32 against np.log2.
  * slice products: exact integer sums (Python ints) on small shapes.
  * accumulate_2sum (A4 on explicit arrays): equal to accumulate_a4 for the
    schedules' own block/group sizes and scales.
  * orders A1..A4: brute-force scalar re-evaluation with Python floats /
    struct-rounded float32 on small shapes, and the reference's recorded
    known answers (tpu_full_results.json:77,93,109,157,173,189,
    tpu_results.json:8-28) replayed from RandomState(42).
  * end-to-end: exact rational products and the CI thresholds of
    ci_cpu_validate.py:35-65, ci_gram_validate.py:178-187,
    ci_solve_validate.py:49-60,139-144.
"""

from .extract import (  # noqa: F401
    rho_f64, rho_f32,
    extract_rows_f64, extract_cols_f64,
    extract_rows_f32, extract_cols_f32,
)
from .pipeline import (  # noqa: F401
    PRECISION_PRESETS, resolve_precision, split_hi_lo,
    ondevice_schedule, host_schedule,
    host_safety_report, ondevice_safety_report, handle_unsafe,
    slice_products, ondevice_slices, host_slices, scales_f32,
    accumulate_a1, accumulate_a2, accumulate_a3, accumulate_a4,
    accumulate_2sum, precompute_accumulation_scales, combine_f64,
    matmul_numpy, matmul_host_a2, matmul_ondevice_a4, matmul_ondevice_a3,
    gram_ozaki, residual_ozaki, solve_ozaki,
)
