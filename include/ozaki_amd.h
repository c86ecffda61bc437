/*
 * ozaki_amd.h -- C ABI of the MI355X (gfx950) Ozaki-scheme matmul engine.
 *
 * The reference (Efithor/ozaki-jax) has no FFI: its operator API is the Python
 * functions matmul / matmul_numpy / gram / residual / solve, each lowered by
 * jax.jit.  This header is the boundary that replaces those jitted programs;
 * every entry point names the reference code it stands in for.  The Python
 * host layer (ozaki_jax_amd) binds these symbols with ctypes.
 *
 * Conventions
 *  - All array arguments are DEVICE pointers (hipMalloc'd or equivalent);
 *    matrices are row-major with an explicit leading dimension in elements.
 *  - `stream` is a hipStream_t (NULL = default stream).  Calls enqueue work
 *    and return; they do not synchronise.
 *  - Returns OZK_OK (0) or a negative status; ozk_last_error() then holds a
 *    message (thread-local).  No call aborts the process.
 *  - The library keeps no device memory of its own.  Drivers take a caller
 *    workspace whose size the matching *_workspace_bytes() query returns.
 *  - `flags` (device uint32) receives OZK_FLAG_NONFINITE when an input holds
 *    NaN/Inf; drivers clear it first.  It replaces the host-side
 *    np.isfinite preflight scan (ozaki_jax/matmul.py:108-109, :623-628).
 *  - Slice planes: BF16 bit patterns (2 bytes) or INT8 grid counts (1 byte,
 *    offset: see ozk_extract_f32_i8), L = ozk_slice_lines(lines) lines of
 *    ld = ozk_slice_ld(len) elements per plane, planes back to back; padding
 *    holds zero slices.  Inside a plane the bytes
 *    are chunk-major: byte b of line r lies at
 *        ((b / 64) * L + r) * 64 + 16 * (((b % 64) / 16) ^ s(r)) + b % 16,
 *    s(r) = (((r & 15) >> 1) ^ ((r & 15) >> 2)) & 3, so the 64 lines of an
 *    output tile form one contiguous 4 KiB block per 64-byte chunk.
 *    Exponents: int32 [plane][L].
 */
#ifndef OZAKI_AMD_H
#define OZAKI_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OZK_OK 0
#define OZK_ERR_INVALID (-1)     /* bad argument (shape, mode, size) */
#define OZK_ERR_HIP (-2)         /* HIP runtime / launch failure */
#define OZK_ERR_UNSUPPORTED (-3) /* valid request the library does not serve */
#define OZK_ERR_WORKSPACE (-4)   /* workspace too small */

#define OZK_FLAG_NONFINITE 1u
#define OZK_FLAG_WAIT_TIMEOUT 2u /* a bounded wait between workgroups gave up (column
                                   extraction, ozk_lu_solve_f32): results not valid */

#define OZK_FLAG_SINGULAR 4u     /* ozk_lu_factor_f32: a zero pivot */
/* INT8 planes: a slice line overflowed with 2^-c > FLT_MAX (see
 * OZK_EXP_NONFINITE).  The reference's slice then holds +-inf (and NaN where
 * its value is zero); a product with it may be +-inf rather than NaN, which
 * the FP64 order OZK_ORDER_BLOCK64 can carry to C.  Rerun such a call with
 * OZK_PIPE_ONDEVICE_BF16 to get those values; the 2Sum order turns every
 * non-finite product into NaN, so its results are exact either way. */
#define OZK_FLAG_INF_SLICE 8u

/* Exponent stored for a slice that INT8 planes cannot represent.  The
 * reference's FP32 extraction (extract.py:130-148) gives a line non-finite
 * slices when sigma = 0.75 * 2^(rho + c) or 2^-c overflows FP32 (rho + c >=
 * 128 or c <= -128) or the line holds NaN/Inf; every product with such a
 * slice is NaN or +-inf, and its output row / column comes out NaN in the
 * 2Sum order.  On INT8 planes that slice and every later slice of its part
 * are stored as zeros with this exponent, and the slice GEMM folds each pair
 * product with it as NaN. */
#define OZK_EXP_NONFINITE (-2147483647 - 1)

/* Test hook, no counterpart in the reference: the limit of every bounded
 * wait between workgroups for the kernels launched after the call (ticks of
 * the 100 MHz real-time counter in the extraction gangs, polls in
 * ozk_lu_solve_f32); 0 restores the built-in limits (0.2 s per wait in the
 * gangs).  A tiny limit makes those waits give up, so that a test can check
 * OZK_FLAG_WAIT_TIMEOUT and the callers' handling of it while every kernel
 * still exits normally. */
void ozk_set_wait_polls(uint32_t polls);

/* No counterpart in the reference: the extraction strategy of the calling
 * thread's later calls (thread-local).  1 (the default): columns of 4097 to
 * 65536 rows, and FP32 rows of 32769 to 262144 elements, are extracted by
 * gangs of workgroups that exchange their partial maxima, with waits that
 * give up after 0.2 s (OZK_FLAG_WAIT_TIMEOUT) when other work keeps the
 * gang's members from running together; ozk_lu_solve_f32 spreads each
 * column's row blocks over several workgroups.  0: no waits between
 * workgroups; columns go through an FP64 transposed copy, long rows are
 * streamed (a larger workspace for columns: query the *_workspace_bytes
 * functions after the switch), and one workgroup solves each column.  The
 * Python layer repeats a call that reports OZK_FLAG_WAIT_TIMEOUT once with
 * 0; the results are bit-identical. */
void ozk_set_gangs(int enable);

/* Accumulation orders (the four orders of the reference). */
#define OZK_ORDER_2SUM 0     /* A4: pallas_ops.py:178-239 == matmul.py:382-488 */
#define OZK_ORDER_BLOCK64 1  /* A3: matmul.py:543-597 (accumulation="host")  */
#define OZK_ORDER_HOST_JAX 2 /* A2: matmul.py:35-64 (matmul, pipeline="host") */
#define OZK_ORDER_HOST_NP 3  /* A1: matmul.py:879-898 (matmul_numpy, "host")  */

/* Pipelines / pair schedules. */
#define OZK_PIPE_ONDEVICE 0 /* hh, hl, lh blocks: pallas_gemm_accum.py:26-87 */
#define OZK_PIPE_HOST 1     /* triangle i+j <= n-1: matmul.py:23-32           */
/* ozk_matmul / ozk_matmul_workspace_bytes only: the on-device pipeline on
 * BF16 planes at every contraction length (no INT8 planes).  Same results as
 * OZK_PIPE_ONDEVICE except where OZK_FLAG_INF_SLICE applies. */
#define OZK_PIPE_ONDEVICE_BF16 2

/* ---- library --------------------------------------------------------- */
const char* ozk_last_error(void);
int ozk_abi_version(void);
/* Writes the device name of the current device into buf (NUL-terminated)
 * and its compute-unit count into *cu_count. */
int ozk_device_info(char* buf, size_t len, int* cu_count);

/* ---- parameters ------------------------------------------------------ */
/* extract.py:12-18 `_compute_rho` (FP64 extraction, m1=53). */
int ozk_rho_f64(int64_t K);
/* extract.py:109-113 `_compute_rho_f32` (FP32 extraction, m1=24). */
int ozk_rho_f32(int64_t K);
/* Padded K stride / line count of slice planes. */
int64_t ozk_slice_ld(int64_t len);
int64_t ozk_slice_lines(int64_t lines);

/* ---- extraction ------------------------------------------------------ */
/* FP64 -> (FP32 hi, FP32 lo) split (matmul.py:204-213) fused with FP32
 * sigma-trick extraction: n_hi slices of hi then n_lo slices of lo
 * (extract.py:197-286; NumPy twin extract.py:116-191).  by_cols = 0 extracts
 * per row of X (rows x cols), by_cols = 1 per column; in both cases a line
 * is stored contiguously.  Columns of up to 4096 rows are extracted in place,
 * each by one workgroup (no workspace); columns of 4097 to 65536 rows in place
 * by groups of workgroups that exchange their column maxima through the
 * workspace (a bounded wait that gives up sets OZK_FLAG_WAIT_TIMEOUT in
 * flags: the planes are then not valid); longer columns are transposed
 * through the workspace.  Lines of 32769 to 262144 elements (rows, or the
 * transposed columns) are likewise held by groups of workgroups exchanging
 * their line maxima through the workspace, so row extraction needs one too.
 * ozk_extract_workspace_bytes covers both this and ozk_extract_f64 (whose
 * columns are always transposed).
 * Output planes: n_hi + n_lo. */
size_t ozk_extract_workspace_bytes(int64_t rows, int64_t cols, int by_cols);
int ozk_extract_f32(const double* X, int64_t rows, int64_t cols, int64_t ldx,
                    int by_cols, int rho, int n_hi, int n_lo,
                    uint16_t* slices, int32_t* exps, uint32_t* flags,
                    void* workspace, size_t workspace_bytes, void* stream);

/* As ozk_extract_f32, with INT8 planes: each slice is held as its integer
 * count of grid steps, q = slice * 2^(24 - rho), which needs
 * 19 <= rho <= 24 (|q| <= 2^(25 - rho) <= 64; OZK_ERR_UNSUPPORTED
 * otherwise), and stored as q + 2^(25 - rho) - 1 (in [-1, 127]: the INT8
 * matrix cores run at a higher clock on mostly non-negative operands).
 * sums (planes x ozk_slice_lines(lines), like exps) receives each plane
 * line's sum of q over its padded length; the INT8 GEMMs take it to remove
 * the offset exactly.  Same plane layout with 1-byte elements.  No
 * counterpart in the reference: an exact re-encoding of its BF16-exact
 * slices (extract.py:145-151) for the INT8 matrix cores.  Slices the
 * reference makes non-finite are stored as q = 0 with exponent
 * OZK_EXP_NONFINITE, and OZK_FLAG_INF_SLICE is set when one of them may hold
 * +-inf (2^-c overflow). */
int ozk_extract_f32_i8(const double* X, int64_t rows, int64_t cols,
                       int64_t ldx, int by_cols, int rho, int n_hi, int n_lo,
                       int8_t* slices, int32_t* exps, int32_t* sums, uint32_t* flags,
                       void* workspace, size_t workspace_bytes, void* stream);

/* FP64 sigma-trick extraction, n_slices planes (extract.py:21-103); slices
 * are the FP32 rounding of v * 2^-c (extract.py:57-60), stored as BF16. */
int ozk_extract_f64(const double* X, int64_t rows, int64_t cols, int64_t ldx,
                    int by_cols, int rho, int n_slices,
                    uint16_t* slices, int32_t* exps, uint32_t* flags,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ---- slice-pair GEMM + accumulation ---------------------------------- */
/* Number of slice pairs of a schedule (matmul.py:636; host: n(n+1)/2). */
int ozk_pair_count(int pipeline, int n_hi, int n_lo);

/* Fused slice-pair GEMMs (BF16 MFMA, FP32 accumulate) with the selected
 * accumulation order folded in registers; writes C (N x M, FP64).
 * Replaces `_fully_fused_f64_jit` / `_bf16_interleaved_f64_jit`
 * (matmul.py:514-540), the Pallas kernel `fused_gemm_accum`
 * (pallas_gemm_accum.py:191-275), `_ondevice_gemms_jit` + accumulate_2sum
 * (matmul.py:706-722), `_accumulate_block_products` (matmul.py:543-597),
 * `_ozaki_gemms_jit` + `_accumulate_products` (matmul.py:23-64) and the
 * matmul_numpy host loop (matmul.py:879-898).  A planes are rows of A
 * (N lines), B planes are columns of B (M lines); both of length K.
 * The drivers below use INT8 planes (ozk_gemm_i8) instead when the
 * contraction length gives rho >= 19 and the schedule is an all-pairs one.
 *
 * All-pairs schedules: every on-device (n_hi, n_lo) with both counts in
 * 1 .. 5, in one K sweep when n_hi + n_lo <= 5 (high (4,1), medium (3,1)),
 * else in two (hh + hl, then lh) or three (hh, hl, lh, as max (5,4);
 * matmul.py:670-674), keeping the fold state between the sweeps in the
 * workspace; every other on-device (n_hi, n_lo) with both counts up to 8
 * in the 2SUM and BLOCK64 orders (and ozk_gemm_2sum_pair), in sweeps over
 * rectangles of one block (consecutive groups x the block's B planes; a
 * block cut between groups carries its running sum in the fold state too);
 * and the host pipeline's triangle of up to 9 slices in the FP64 orders
 * (HOST_JAX, HOST_NP, BLOCK64), in sweeps over groups of A planes that keep
 * each element's FP64 running sum between them.  Other schedules run one
 * pair at a time on BF16 planes.
 * Workspace: ozk_gemm_workspace_bytes is the fold state (multi-sweep
 * schedules only) plus 4608 bytes of tile counters, with which the last
 * rounds of output tiles are handed out at run time to the workgroups that
 * finish first.  Any workspace from the fold state up (none for one-sweep
 * schedules) is accepted; below the full size the tiles run in a static
 * order. */
size_t ozk_gemm_workspace_bytes(int64_t N, int64_t M, int pipeline, int n_hi,
                                int n_lo, int order);
int ozk_gemm(const uint16_t* a_slices, const int32_t* a_exps,
             const uint16_t* b_slices, const int32_t* b_exps,
             int64_t N, int64_t M, int64_t K,
             int pipeline, int n_hi, int n_lo, int order,
             double* C, int64_t ldc, void* workspace, size_t workspace_bytes,
             void* stream);

/* ozk_gemm on INT8 planes (ozk_extract_f32_i8 with the same rho, with their
 * line sums): INT8 MFMA with exact INT32 sums, from which the offset's
 * terms are removed with the line sums; each pair product is the integer
 * sum times 2^(2 rho - 48), the FP32 product of the BF16 path whenever that
 * one is exact.  All-pairs on-device schedules (see ozk_gemm). */
int ozk_gemm_i8(const int8_t* a_slices, const int32_t* a_exps, const int32_t* a_sums,
                const int8_t* b_slices, const int32_t* b_exps, const int32_t* b_sums,
                int64_t N, int64_t M, int64_t K, int rho,
                int n_hi, int n_lo, int order,
                double* C, int64_t ldc, void* workspace, size_t workspace_bytes,
                void* stream);

/* The fused slice GEMM of `fused_gemm_accum` (pallas_gemm_accum.py:191-275):
 * the on-device (n_hi, n_lo) schedule in the 2Sum order, returning the
 * double-float pair (C_hi, C_lo) of pallas_gemm_accum.py:181-186 (whose FP64
 * sum ozk_gemm writes) as two FP32 N x M arrays with leading dimension ldc.
 * plane_bytes 2: BF16 planes (ozk_extract_f32; rho and the sums are not
 * used); 1: INT8 planes and their line sums (ozk_extract_f32_i8 with this
 * rho, all-pairs schedules).
 * Workspace: ozk_gemm_workspace_bytes(N, M, OZK_PIPE_ONDEVICE, n_hi, n_lo,
 * OZK_ORDER_2SUM). */
int ozk_gemm_2sum_pair(const void* a_slices, const int32_t* a_exps,
                       const int32_t* a_sums, const void* b_slices,
                       const int32_t* b_exps, const int32_t* b_sums,
                       int64_t N, int64_t M, int64_t K, int plane_bytes, int rho,
                       int n_hi, int n_lo, float* C_hi, float* C_lo, int64_t ldc,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Test hook: the per-pair FP32 products P[p] = S^A_a(p) . S^B_b(p) written
 * to P[p][N][ldp] in schedule order (matmul.py:216-233, :757-773, :885-887). */
int ozk_slice_products(const uint16_t* a_slices, const uint16_t* b_slices,
                       int64_t N, int64_t M, int64_t K,
                       int pipeline, int n_hi, int n_lo,
                       float* P, int64_t ldp, void* stream);

/* Test hook: ozk_slice_products on INT8 planes and their line sums. */
int ozk_slice_products_i8(const int8_t* a_slices, const int32_t* a_sums,
                          const int8_t* b_slices, const int32_t* b_sums,
                          int64_t N, int64_t M, int64_t K, int rho,
                          int n_hi, int n_lo, float* P, int64_t ldp,
                          void* stream);

/* accumulate_2sum(products, col_scales, row_scales, block_group_sizes)
 * (pallas_ops.py:178-239, dispatched by :372-396), the A4 order on products
 * the caller holds.  products: n_products x N x M FP32, contiguous;
 * col_scales: n_products x M; row_scales: n_groups x N.  Block b has
 * block_ngroups[b] groups (n_blocks <= 8) and group g has group_sizes[g]
 * products (n_groups <= 256; the sizes add up to n_products).  Per output
 * element: per group, 2Sum of product * column scale from zero, times the
 * group's row scale, hi then lo 2Sum-added into the block; then every
 * block's hi, then every block's lo, 2Sum-added into (C_hi, C_lo), N x M
 * FP32 each.  block_ngroups and group_sizes are host arrays. */
int ozk_accumulate_2sum(const float* products, int64_t n_products,
                        int64_t N, int64_t M, const float* col_scales,
                        const float* row_scales,
                        const int32_t* block_ngroups, int n_blocks,
                        const int32_t* group_sizes, int n_groups,
                        float* C_hi, float* C_lo, void* stream);

/* ---- drivers --------------------------------------------------------- */
/* matmul(A, B, pipeline, accumulation, precision) after preflight:
 * pipeline OZK_PIPE_ONDEVICE: split + FP32 extraction with
 *   rho = ozk_rho_f32(K), n_hi/n_lo slices, order 2SUM or BLOCK64
 *   (matmul.py:641-728); INT8 planes when rho >= 19 and the schedule is an
 *   all-pairs one (ozk_gemm; OZK_PIPE_ONDEVICE_BF16 keeps BF16 planes);
 * pipeline OZK_PIPE_HOST: FP64 extraction with rho = ozk_rho_f64(K),
 *   n_hi = n_slices (n_lo ignored), order HOST_JAX or HOST_NP
 *   (matmul.py:823-851, :866-900).
 * flags receives OZK_FLAG_NONFINITE (NaN/Inf in A or B) and, on INT8
 * planes, OZK_FLAG_INF_SLICE. */
size_t ozk_matmul_workspace_bytes(int64_t N, int64_t K, int64_t M,
                                  int pipeline, int n_hi, int n_lo);
/* Bytes per slice-plane element ozk_matmul uses for this shape: 1 (INT8
 * planes, ozk_gemm_i8's kernels) or 2 (BF16 planes); negative on a bad
 * pipeline or slice count.  No counterpart in the reference (whose slices
 * are always BF16-valued FP32). */
int ozk_matmul_plane_bytes(int pipeline, int64_t K, int n_hi, int n_lo);
int ozk_matmul(const double* A, int64_t lda, const double* B, int64_t ldb,
               double* C, int64_t ldc, int64_t N, int64_t K, int64_t M,
               int pipeline, int n_hi, int n_lo, int order,
               void* workspace, size_t workspace_bytes, uint32_t* flags,
               void* stream);
/* ozk_matmul, and also a copy of the call's final flag word to host_flags
 * (pinned host memory, e.g. from hipHostMalloc), then `event` (a hipEvent_t)
 * recorded on `stream`.  Both come as soon as the kernels that set flags
 * (the extraction) are queued, ahead of the GEMM.  A caller that waits for
 * `event` and reads *host_flags has the call's flags without waiting for
 * the product, so it can raise or fall back as matmul.py:127-135 does while
 * the GEMM still runs.  This serves callers whose result is ordered on the
 * stream, as a JAX or torch array is (the reference's calls return JAX
 * arrays, matmul.py:781-851).  It has no counterpart of its own in the
 * reference. */
int ozk_matmul_early_flags(const double* A, int64_t lda, const double* B,
                           int64_t ldb, double* C, int64_t ldc, int64_t N,
                           int64_t K, int64_t M, int pipeline, int n_hi,
                           int n_lo, int order, void* workspace,
                           size_t workspace_bytes, uint32_t* flags,
                           uint32_t* host_flags, void* event, void* stream);

/* ozk_matmul without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is the library's own device array of OZK_NOALLOC_SCRATCH_BYTES
 * (128 MiB), which each GPU the library runs on holds until the process
 * ends; shapes whose ozk_matmul_workspace_bytes exceeds it return
 * OZK_ERR_WORKSPACE (e.g. 2048^3 high needs 112 MiB and fits, 4096^3 high
 * needs 448 MiB and does not).  The call allocates nothing: no hipMalloc,
 * no hipFree.  All calls on one GPU share that GPU's array, so calls that
 * overlap on a GPU (other streams, other threads) race. */
#define OZK_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)
int ozk_matmul_noalloc(const double* A, int64_t lda, const double* B, int64_t ldb,
                       double* C, int64_t ldc, int64_t N, int64_t K, int64_t M,
                       int pipeline, int n_hi, int n_lo, int order,
                       uint32_t* flags, void* stream);

/* gram(A, mode="ozaki"): G = Ozaki(A^T, A) in order 2SUM with
 * rho = ozk_rho_f32(rows), then G = (G + G^T) * 0.5 (gram.py:19-37, :92-95).
 * A is rows x cols; G is cols x cols.  One column extraction of A serves
 * both operands. */
size_t ozk_gram_workspace_bytes(int64_t rows, int64_t cols, int n_hi,
                                int n_lo);
int ozk_gram(const double* A, int64_t lda, int64_t rows, int64_t cols,
             int n_hi, int n_lo, double* G, int64_t ldg,
             void* workspace, size_t workspace_bytes, uint32_t* flags,
             void* stream);
/* ozk_gram with the flag word copied to host_flags and `event` recorded
 * once the column extraction is queued, as ozk_matmul_early_flags does
 * (the reference's gram returns a JAX array, gram.py:47-99). */
int ozk_gram_early_flags(const double* A, int64_t lda, int64_t rows,
                         int64_t cols, int n_hi, int n_lo, double* G,
                         int64_t ldg, void* workspace, size_t workspace_bytes,
                         uint32_t* flags, uint32_t* host_flags, void* event,
                         void* stream);

/* residual(A, x, b, mode="ozaki"): r = b - Ozaki(A, x) in order 2SUM with
 * rho = ozk_rho_f32(K); x is K x ncols, b and r are N x ncols
 * (solve.py:38-53, :78-82, :91-151).  Up to 4 columns with K <= 16384 and
 * (n_hi, n_lo) = (4, 1) or (3, 1), or K <= 8192 and (5, 4), run fused row
 * kernels that read A once per column and need no workspace
 * (ozk_residual_workspace_bytes returns 0); other shapes extract A's slice
 * planes and run the slice GEMM. */
size_t ozk_residual_workspace_bytes(int64_t N, int64_t K, int64_t ncols,
                                    int n_hi, int n_lo);
int ozk_residual(const double* A, int64_t lda, const double* x, int64_t ldx,
                 const double* b, int64_t ldb, double* r, int64_t ldr,
                 int64_t N, int64_t K, int64_t ncols, int n_hi, int n_lo,
                 void* workspace, size_t workspace_bytes, uint32_t* flags,
                 void* stream);

/* FP32 LU factorisation with partial pivoting, in place: the factorisation
 * inside the reference's jnp.linalg.solve(A32, .) (solve.py:159).  A is
 * n x n FP32, row-major (lda); on return it holds the unit-diagonal L below
 * the diagonal and U on and above it, and perm (device int32, n entries)
 * the row permutation (row i of P A is row perm[i] of A), the form
 * ozk_lu_solve_f32 takes.  The pivot of a column is its largest |value| on
 * or below the diagonal (the lowest row on ties).  flags is cleared first
 * and receives OZK_FLAG_SINGULAR if a pivot is zero; as in LAPACK's getrf
 * the factorisation then completes and U has a zero on its diagonal.
 * n <= ozk_lu_factor_max_n(); larger n return OZK_ERR_UNSUPPORTED. */
int64_t ozk_lu_factor_max_n(void);
size_t ozk_lu_factor_workspace_bytes(int64_t n);
int ozk_lu_factor_f32(float* A, int64_t lda, int64_t n, int32_t* perm,
                      void* workspace, size_t workspace_bytes, uint32_t* flags,
                      void* stream);

/* The FP32 solves of solve(...) (solve.py:154-167): x0 = A32^-1 b and
 * d = A32^-1 r in each refinement step, which the reference computes with
 * jnp.linalg.solve(A32, .) (solve.py:159, :164) -- an LU factorisation with
 * partial pivoting and two triangular solves.  This entry point does the
 * triangular solves on an existing factor:
 *     X = U^-1 L^-1 P B   for ncols right-hand sides.
 * LU is n x n FP32, row-major (lda), as getrf leaves it: unit-diagonal L
 * below the diagonal, U on and above it.  perm (device int32) is the row
 * permutation: row i of P B is row perm[i] of B.  B and X are n x ncols FP64
 * (ldb, ldx); B is rounded to FP32 first (r.astype(float32)) and X is the
 * FP32 solution widened.  X may alias B.  flags is cleared first and
 * receives OZK_FLAG_WAIT_TIMEOUT if a row block gave up waiting for the
 * blocks it depends on (X is then invalid).  The workspace (8-byte aligned,
 * ozk_lu_solve_workspace_bytes(n, ncols) = 16 n ncols bytes) holds the
 * published solution words; each call clears it first, so calls that share
 * one must not overlap. */
size_t ozk_lu_solve_workspace_bytes(int64_t n, int64_t ncols);
int ozk_lu_solve_f32(const float* LU, int64_t lda, const int32_t* perm,
                     int64_t n, const double* B, int64_t ldb, double* X,
                     int64_t ldx, int64_t ncols, void* workspace,
                     size_t workspace_bytes, uint32_t* flags, void* stream);

/* LAPACK getrf pivots -> the permutation ozk_lu_solve_f32 takes.  ipiv is
 * 1-based: step i swapped rows i and ipiv[i] - 1, for i = 0 .. n-1 in order.
 * HOST arrays; no device work. */
int ozk_pivots_to_perm(const int32_t* ipiv, int64_t n, int32_t* perm);

/* np.isfinite(X).all() as a flag (matmul.py:108-109, :623-628). */
int ozk_check_finite(const double* X, int64_t rows, int64_t cols, int64_t ld,
                     uint32_t* flags, void* stream);

/* Test hook: runs one 32x32x16 and one 16x16x32 BF16 MFMA and one
 * 16x16x64 and one 32x32x32 INT8 MFMA on fixed patterns and writes their
 * accumulator registers as int32: out[0..1023] = 64 lanes x 16 registers
 * (32x32x16), out[1024..1279] and out[1280..1535] = 64 lanes x 4 registers
 * (16x16x32, 16x16x64), out[1536..2559] = 64 lanes x 16 registers
 * (32x32x32).  out must hold 2560 int32. */
int ozk_probe_mfma_layout(int32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OZAKI_AMD_H */
