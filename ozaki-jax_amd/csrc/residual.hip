// Fused residual r = b - Ozaki(A, x) for one right-hand side (solve.py:38-53,
// :78-82 with the 2Sum order of pallas_ops.py:178-239).
//
// The GEMM route extracts every slice plane of A to HBM and runs the slice
// GEMMs with a single useful output column.  Here one wave owns one row of A:
// it reads the row once (K <= 64 * EPL values in registers), splits and
// extracts its slices with the same arithmetic as the extraction kernels,
// and dots each A slice with the x slices it pairs with.  x's slices are
// decoded once to FP32.  A slice product is a sum of K exact products of
// BF16-exact values; accumulated in FP64 it is exact, and its rounding to
// FP32 is the reference's FP32 GEMM result whenever that one is exact
// (partial sums below 2^24 grid units).  The per-row pair products are then
// folded in schedule order; the workload is bound by the read of A.

#include "fold.h"
#include "sigma.h"

namespace ozk {

constexpr int kResRows = 4;  // rows (waves) per workgroup

// Slice values of line 0 of `planes` chunk-major planes (BF16 bits or INT8
// grid counts) -> FP32, xs[p * kp + k] for k < K, zero for K <= k < kp.
__global__ void decode_line0_kernel(const void* __restrict__ S, int i8,
                                    int64_t K, int64_t kp, int64_t ld,
                                    int64_t lpad, int rho,
                                    float* __restrict__ xs) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int p = blockIdx.y;
  if (k >= kp) return;
  float v = 0.0f;
  if (k < K) {
    const int64_t plane = lpad * ld;
    if (i8) {
      const int8_t q = ((const int8_t*)S)[p * plane + plane_offset<1>(0, k, lpad)];
      v = (float)q * ldexpf(1.0f, rho - 24);
    } else {
      const uint16_t h = ((const uint16_t*)S)[p * plane + plane_offset<2>(0, k, lpad)];
      v = bf16_bits_to_f32(h);
    }
  }
  xs[p * kp + k] = v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// One wave per row, rows strided over a persistent grid; x's slices (FP32,
// NT planes of kp values) sit in LDS for the workgroup's lifetime.  Phase 1
// extracts the row's NT slices into registers as packed BF16 pairs (the
// slices are BF16-exact); phase 2 walks k once and updates the pair sums;
// phase 3 reduces them across the wave and folds.  A pair sum adds exact
// products of BF16-exact values with FP32 fma, like the FP32-accumulating
// slice GEMM: exact whenever partial sums stay below 2^24 grid units.
template <int EPL, int NHI, int NLO>
__global__ __launch_bounds__(64 * kResRows) void residual_rows_kernel(
    const double* __restrict__ A, int64_t N, int64_t K, int64_t lda,
    const float* __restrict__ xs, const int32_t* __restrict__ xe,
    int64_t xe_stride, const double* __restrict__ b, int64_t ldb,
    double* __restrict__ r, int64_t ldr, int rho, uint32_t* __restrict__ flags) {
  constexpr int NT = NHI + NLO;
  constexpr int NP = pair_count(OZK_PIPE_ONDEVICE, NHI, NLO);
  constexpr int KP = 64 * EPL;
  static_assert(EPL % 2 == 0, "slices are packed in pairs");
  extern __shared__ float xl[];  // NT * KP
  for (int i = threadIdx.x; i < NT * KP; i += blockDim.x) xl[i] = xs[i];
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float cs[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) cs[t] = ldexpf(1.0f, xe[t * xe_stride]);

  for (int64_t row = (int64_t)blockIdx.x * kResRows + wave; row < N;
       row += (int64_t)gridDim.x * kResRows) {
    const double* a = A + row * lda;
    float R[2][EPL];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int64_t k = (int64_t)j * 64 + lane;
      const double v = k < K ? a[k] : 0.0;
      bad |= !isfinite(v);
      float p[2];
      split<float>(v, p);
      R[0][j] = p[0];
      R[1][j] = p[1];
    }
    if (bad) atomicOr(flags, OZK_FLAG_NONFINITE);

    // Phase 1: slices of A planes 0 .. NHI-1 (hi part) and NHI .. NT-1 (lo).
    uint32_t sl[NT][EPL / 2];
    int ea[NT];
#pragma unroll
    for (int s = 0; s < (NHI > NLO ? NHI : NLO); ++s) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (s >= (q == 0 ? NHI : NLO)) continue;
        const int t = q == 0 ? s : NHI + s;
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < EPL; ++j) m = fmaxf(m, fabsf(R[q][j]));
        m = wave_max(m);
        const SliceConst<float> kc = slice_const<float>(m, rho);
        ea[t] = kc.c;
#pragma unroll
        for (int j = 0; j < EPL; j += 2) {
          uint32_t pk = 0;
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float rr = R[q][j + e];
            float v = (rr + kc.sigma) - kc.sigma;
            if (kc.zero) v = 0.0f;
            R[q][j + e] = rr - v;
            pk |= (uint32_t)f32_to_bf16_bits(slice_value_f32(v, kc.inv)) << (16 * e);
          }
          sl[t][j / 2] = pk;
        }
      }
    }
    // Phase 2: pair sums.
    float acc[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) acc[p] = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      float xv[NT], av[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        xv[t] = xl[t * KP + j * 64 + lane];
        const uint32_t pk = sl[t][j / 2];
        av[t] = __uint_as_float((j & 1) ? (pk & 0xffff0000u) : (pk << 16));
      }
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const PairInfo q = pair_info(OZK_PIPE_ONDEVICE, NHI, NLO, p);
        acc[p] = fmaf(av[q.a], xv[q.b], acc[p]);
      }
      // keep the LDS reads of later k-steps from being hoisted (registers)
      __builtin_amdgcn_sched_barrier(0);
    }
    // Phase 3: reduce, then fold in schedule order.
#pragma unroll
    for (int p = 0; p < NP; ++p) acc[p] = wave_sum(acc[p]);
    Fold2Sum f;
    f.init();
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const PairInfo q = pair_info(OZK_PIPE_ONDEVICE, NHI, NLO, p);
      f.pair(q, acc[p], cs[q.b], ldexpf(1.0f, ea[q.a]), 0.0, 0.0);
    }
    const double c = f.finish(3);
    if (lane == 0) r[row * ldr] = b[row * ldb] - c;
  }
}

bool residual_rows_supported(int64_t K, int64_t ncols, int nhi, int nlo) {
  return ncols == 1 && K >= 1 && K <= 64 * 32 &&
         ((nhi == 4 && nlo == 1) || (nhi == 3 && nlo == 1));
}

// Values per lane (EPL) and padded length 64 * EPL of the decoded x slices.
static int residual_rows_epl(int64_t K) {
  int epl = 8;
  while (64 * epl < K) epl *= 2;
  return epl;
}

size_t residual_rows_xs_bytes(int64_t K, int nhi, int nlo) {
  return (size_t)(nhi + nlo) * (size_t)(64 * residual_rows_epl(K)) * sizeof(float);
}

// x's planes (chunk-major, `lpad` lines, `ld` elements per line) and
// exponents (plane stride xe_stride) -> r for the N rows of A.
int launch_residual_rows(const double* A, int64_t N, int64_t K, int64_t lda,
                         const void* xplanes, bool i8, int64_t ld, int64_t lpad,
                         const int32_t* xe, int64_t xe_stride, const double* b,
                         int64_t ldb, double* r, int64_t ldr, int rho, int nhi,
                         int nlo, float* xs, uint32_t* flags, hipStream_t st) {
  const int epl = residual_rows_epl(K);
  const int64_t kp = 64 * epl;  // the kernel reads xs[p * kp + j * 64 + lane], j < epl
  hipLaunchKernelGGL(decode_line0_kernel, dim3((unsigned)((kp + 255) / 256), nhi + nlo),
                     dim3(256), 0, st, xplanes, i8 ? 1 : 0, K, kp, ld, lpad, rho, xs);
  OZK_LAUNCH_CHECK();
  // persistent grid: two workgroups per CU, each holding x's slices in LDS
  const int cus = cu_count();
  const int64_t need = (N + kResRows - 1) / kResRows;
  const dim3 grid((unsigned)(need < 2 * cus ? need : 2 * cus));
  const size_t lds = (size_t)(nhi + nlo) * kp * sizeof(float);
#define OZK_RES(E, H, L)                                                              \
  hipLaunchKernelGGL((residual_rows_kernel<E, H, L>), grid, dim3(64 * kResRows), lds, \
                     st, A, N, K, lda, xs, xe, xe_stride, b, ldb, r, ldr, rho, flags)
#define OZK_RES_E(H, L)          \
  switch (epl) {                 \
    case 8: OZK_RES(8, H, L); break;   \
    case 16: OZK_RES(16, H, L); break; \
    default: OZK_RES(32, H, L); break; \
  }
  if (nhi == 4) {
    OZK_RES_E(4, 1);
  } else {
    OZK_RES_E(3, 1);
  }
#undef OZK_RES_E
#undef OZK_RES
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

}  // namespace ozk
