// Fused residual r = b - Ozaki(A, x) for one right-hand side (solve.py:38-53,
// :78-82 with the 2Sum order of pallas_ops.py:178-239).
//
// The GEMM route extracts every slice plane of A to HBM and runs the slice
// GEMMs with a single useful output column.  Here one wave owns one row of A
// at a time: it reads the row once (K <= 64 * EPL values in registers),
// splits and extracts its slices with the same arithmetic as the extraction
// kernels, and dots each A slice with the x slices it pairs with.  A slice
// product is a sum of K exact products of BF16-exact values on one grid; the
// slice exponent rule keeps every partial sum below 2^24 grid units, so the
// sum is exact in FP32 in any order and equals the reference's FP32 GEMM
// result.  The per-row pair products are then folded in schedule order.
// The work is bound by the read of A and the VALU work of the extraction.

#include <type_traits>

#include "fold.h"
#include "sigma.h"

namespace ozk {

// f(integral_constant<int, I>) for I = B .. E - 1, unrolled at compile time.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

constexpr int kResWaves = 8;   // waves per workgroup: two per SIMD
constexpr int kResBatch = 16;  // rows whose pair products are folded together

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// DPP source selections (gfx9 encoding).
constexpr int kDppQuad1032 = 0xB1;     // quad_perm [1, 0, 3, 2]
constexpr int kDppQuad2301 = 0x4E;     // quad_perm [2, 3, 0, 1]
constexpr int kDppRowMirror = 0x140;   // lane i <- lane 15 - i of its row
constexpr int kDppHalfMirror = 0x141;  // lane i <- lane 7 - i of its half row

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// The two halves of a permlane swap: (x, y) of rows of 32 (or 16) lanes.
// v_permlane32_swap exchanges the upper 32 lanes of its first operand with
// the lower 32 lanes of its second; v_permlane16_swap exchanges the odd rows
// of 16 lanes of its first operand with the even rows of its second.
__device__ __forceinline__ float swap32_sum(float x, float y) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y),
                                                  false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float swap16_sum(float x, float y) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y),
                                                  false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// old value 0, the identity of an unsigned max, so that the move folds into
// the max as one DPP instruction
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

// Maximum over the wave of non-negative floats (|R| values), returned
// wave-uniform.  Non-negative IEEE values order like their bit patterns, so
// the steps are integer maxima, which fold into DPP forms.  A NaN lane
// (bit pattern above +inf) wins where fmaxf would drop it; either way a row
// holding a NaN gives a NaN residual, since that element's slices are NaN.
__device__ __forceinline__ float wave_max_uniform(float v) {
  uint32_t u = __float_as_uint(v);
  u = max(u, dpp_u<kDppQuad1032>(u));
  u = max(u, dpp_u<kDppQuad2301>(u));
  u = max(u, dpp_u<kDppHalfMirror>(u));
  u = max(u, dpp_u<kDppRowMirror>(u));
  {
    const auto s = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    u = max((uint32_t)s[0], (uint32_t)s[1]);
  }
  {
    const auto s = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    u = max((uint32_t)s[0], (uint32_t)s[1]);
  }
  return __uint_as_float(__builtin_amdgcn_readfirstlane(u));
}

// m = max(m, |a|, |b|) as one v_max3_f32 (the compiler otherwise builds a
// tree that costs 1.5 instructions per pair of values).
__device__ __forceinline__ float max3_abs(float m, float a, float b) {
  float r;
  asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(a), "v"(b));
  return r;
}

// Sum over the 16 lanes of each row; every lane of the row gets it.
__device__ __forceinline__ float row_sum(float v) {
  v += dpp<kDppQuad1032>(v);
  v += dpp<kDppQuad2301>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppRowMirror>(v);
  return v;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  // the upper halves of two BF16-exact FP32 values
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                        __builtin_bit_cast(bf16x2, b), c, false);
}

// x's slices for the row kernel, by one workgroup of 4 waves: the split and
// sigma steps of the extraction kernels applied to x as a single line (x is
// one column, extract.py:157-191; split matmul.py:204-213).  Thread t holds
// elements k = 256 j + t.  Writes the FP32 slice values xs[t * kp + k] (zero
// for K <= k < kp, kp <= 2048), the exponents xe[t], and the flag word
// (OZK_FLAG_NONFINITE if x holds NaN/Inf, else 0).
constexpr int kResXThreads = 256;

__global__ __launch_bounds__(kResXThreads) void residual_x_kernel(
    const double* __restrict__ x, int64_t K, int64_t ldx, int rho, int nhi,
    int nlo, int64_t kp, float* __restrict__ xs, int32_t* __restrict__ xe,
    uint32_t* __restrict__ flags) {
  constexpr int E = 2048 / kResXThreads;
  constexpr int W = kResXThreads / 64;
  __shared__ uint32_t wmax[2][W];  // per-wave maxima, alternating buffers
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float R[2][E];
  bool bad = false;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int64_t k = (int64_t)j * kResXThreads + tid;
    const double v = k < K ? x[k * ldx] : 0.0;
    bad |= !isfinite(v);
    float pr[2];
    split<float>(v, pr);
    R[0][j] = pr[0];
    R[1][j] = pr[1];
  }
  if (__syncthreads_or(bad ? 1 : 0)) {
    if (tid == 0) flags[0] = OZK_FLAG_NONFINITE;
  } else if (tid == 0) {
    flags[0] = 0u;
  }
  int step = 0;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int n = q == 0 ? nhi : nlo;
    for (int s = 0; s < n; ++s, ++step) {
      float m = 0.0f;
#pragma unroll
      for (int j = 0; j < E; ++j) m = fmaxf(m, fabsf(R[q][j]));
      const float mw = wave_max_uniform(m);
      if (lane == 0) wmax[step & 1][wave] = __float_as_uint(mw);
      __syncthreads();
      uint32_t mb = 0;
#pragma unroll
      for (int w = 0; w < W; ++w) mb = max(mb, wmax[step & 1][w]);
      const SliceConst<float> kc = slice_const<float>(__uint_as_float(mb), rho);
      const int t = q == 0 ? s : nhi + s;
#pragma unroll
      for (int j = 0; j < E; ++j) {
        const float rr = R[q][j];
        float v = (rr + kc.sigma) - kc.sigma;
        if (kc.zero) v = 0.0f;
        R[q][j] = rr - v;
        const int64_t k = (int64_t)j * kResXThreads + tid;
        if (k < kp) xs[t * kp + k] = slice_value_f32(v, kc.inv);
      }
      if (tid == 0) xe[t] = kc.c;
    }
  }
}

// Per-row values kept for the batched fold, in LDS: the pair sums, then per
// A slice its row scale 2^c and the factor that turns the accumulated sum
// into the slice product (1, or 2^-c when the unnormalised slice values were
// summed).
template <int NP, int NT>
struct ResRow {
  float p[NP];
  float rs[NT];
  float un[NT];
};

// One wave per row, rows strided over a persistent grid (one workgroup of
// kResWaves waves per CU).  Lane l holds elements k = 64 j + l, j < EPL; x's
// slices live in registers as BF16 pairs (elements j, j + 1).  Per row:
//   split into hi / lo parts; lo slice first, so that its registers are free
//   when the next row's load is issued; then the hi slices.  Each slice is
//   extracted and immediately dotted (v_dot2_f32_bf16) with the x slices of
//   its pairs.  A slice whose exponent c lies in [-100, 100] is dotted in
//   unnormalised form v = slice * 2^c (BF16-exact, every product and partial
//   sum a normal FP32 value), so the sum is the slice product times 2^c
//   exactly; the fold multiplies by 2^-c.  Other slices are normalised first.
// The pair sums are reduced across the wave by a reduce-scatter (permlane
// swaps, then DPP within rows of 16), stored per row in LDS, and every
// kResBatch rows one lane per row folds them in schedule order.
template <int EPL, bool FULL, bool DMA, int NHI, int NLO>
__global__ __launch_bounds__(64 * kResWaves) void residual_rows_kernel(
    const double* __restrict__ A, int64_t N, int64_t K, int64_t lda,
    const float* __restrict__ xs, const int32_t* __restrict__ xe,
    int64_t xe_stride, const double* __restrict__ b, int64_t ldb,
    double* __restrict__ r, int64_t ldr, int rho, uint32_t* __restrict__ flags) {
  constexpr int NT = NHI + NLO;
  constexpr int NP = pair_count(OZK_PIPE_ONDEVICE, NHI, NLO);
  constexpr int NR = (NP + 3) / 4 * 4;  // pair sums padded for the reduce-scatter
  constexpr int KP = 64 * EPL, H = EPL / 2;
  static_assert(EPL % 2 == 0, "elements are paired");
  static_assert(!DMA || FULL, "the row buffer is filled by whole 1 KiB blocks");
  __shared__ ResRow<NP, NT> red[kResWaves][kResBatch];
  // DMA: each wave's next row, copied into LDS as it lies in memory
  __shared__ double rowbuf[DMA ? kResWaves * KP : 1];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  uint32_t xp[NT][H];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int i = 0; i < H; ++i)
      xp[t][i] = pack_bf16x2(xs[t * KP + (2 * i) * 64 + lane],
                             xs[t * KP + (2 * i + 1) * 64 + lane]);
  float cs[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) cs[t] = ldexpf(1.0f, xe[t * xe_stride]);

  const int64_t nw = (int64_t)gridDim.x * kResWaves;
  const int64_t first = (int64_t)blockIdx.x * kResWaves + wave;
  double nx[EPL];
  // FULL: rows of exactly 64 EPL elements, loaded without guards; shorter
  // rows read element min(k, K - 1) and replace it by zero past the end
  const int Ki = (int)K;
  auto load_row = [&](int64_t row) {
    // wave-uniform row base plus a 32-bit byte offset per lane; K passes an
    // empty asm so that the clamped offsets are recomputed per row instead of
    // being kept live across the loop
    const char* a = (const char*)(A + row * lda);
    int Kr = Ki;
    asm volatile("" : "+s"(Kr));
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int k = j * 64 + lane;
      if constexpr (FULL) {
        nx[j] = *(const double*)(a + (uint32_t)k * 8u);
      } else {
        const double v = *(const double*)(a + (uint32_t)(k < Kr ? k : Kr - 1) * 8u);
        nx[j] = k < Kr ? v : 0.0;
      }
    }
  };
  // Prefetch of the next row.  PF: into registers, issued once the current
  // row's lo part is done (up to 16 elements per lane).  DMA: into the
  // wave's LDS row buffer (global_load_lds_dwordx4, 1 KiB per instruction),
  // issued as soon as the current row has been read out of it; rows must be
  // 16-byte aligned.  Otherwise the other wave on the SIMD covers the load.
  constexpr bool PF = EPL <= 16 && !DMA;
  double* myrow = rowbuf + (DMA ? wave * KP : 0);
  const uint32_t myrow_lds = lds_offset(myrow);
  auto dma_row = [&](int64_t row) {
    const char* a = (const char*)(A + row * lda);
#pragma unroll
    for (int i = 0; i < KP * 8 / 1024; ++i)
      dma16(myrow_lds + i * 1024, a + i * 1024, 16u * (uint32_t)lane);
  };
  if (PF && first < N) load_row(first);
  if (DMA && first < N) dma_row(first);
  int nb = 0;
  int64_t row0 = first;
  ResRow<NP, NT>* rows = red[wave];
  // b of the batch's rows, lane i holding row row0 + i nw, loaded when the
  // batch starts
  auto load_b = [&](int64_t r0) {
    const int64_t ri = r0 + (int64_t)lane * nw;
    return lane < kResBatch && ri < N ? b[ri * ldb] : 0.0;
  };
  double bb = load_b(row0);

  for (int64_t row = first; row < N; row += nw) {
    if constexpr (DMA) {
      wait_vm<0>();  // this row's copy has landed in LDS
#pragma unroll
      for (int j = 0; j < EPL; ++j) nx[j] = myrow[j * 64 + lane];
      // the reads must complete before the buffer is refilled
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (row + nw < N) dma_row(row + nw);
    } else if constexpr (!PF) {
      load_row(row);
    }
    float Rh[EPL], Rl[EPL];
    bool bad = false;
    float mh = 0.0f, ml = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      bad |= !isfinite(nx[j]);
      float pr[2];
      split<float>(nx[j], pr);
      Rh[j] = pr[0];
      Rl[j] = pr[1];
      if (j & 1) {
        mh = max3_abs(mh, Rh[j - 1], Rh[j]);
        ml = max3_abs(ml, Rl[j - 1], Rl[j]);
      }
    }
    if (bad) atomicOr(flags, OZK_FLAG_NONFINITE);

    float acc[NR];
#pragma unroll
    for (int p = 0; p < NR; ++p) acc[p] = 0.0f;
    float rs[NT], un[NT];

    // Extract the slice of plane `a` from part R with constants kc and dot it
    // with the x slices of its pairs; NORM: normalised slice values, else
    // v = slice * 2^c.  Returns the lane's max of the new residual (MAXNEXT).
    auto slice_loop = [&](auto a_c, auto maxnext_c, auto norm_c, float (&R)[EPL],
                          const SliceConst<float>& kc) {
      constexpr int a = decltype(a_c)::value;
      constexpr bool MAXNEXT = decltype(maxnext_c)::value;
      constexpr bool NORM = decltype(norm_c)::value;
      float mn = 0.0f;
#pragma unroll
      for (int i = 0; i < H; ++i) {
        float v[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float rr = R[2 * i + e];
          v[e] = (rr + kc.sigma) - kc.sigma;
          if (MAXNEXT) R[2 * i + e] = rr - v[e];
          if (NORM) v[e] = slice_value_f32(v[e], kc.inv);
        }
        if (MAXNEXT) mn = max3_abs(mn, R[2 * i], R[2 * i + 1]);
        const uint32_t pk = pack_bf16x2(v[0], v[1]);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const PairInfo q = pair_info(OZK_PIPE_ONDEVICE, NHI, NLO, p);
          if (q.a == a) acc[p] = dot2(pk, xp[q.b][i], acc[p]);
        }
      }
      return mn;
    };
    // Slice of plane `a` from part R, whose max |R| over the row is mw; m
    // returns the lane's max of the new residual (when MAXNEXT; R is dead
    // otherwise).
    auto slice = [&](auto a_c, auto maxnext_c, float (&R)[EPL], float mw, float& m) {
      constexpr int a = decltype(a_c)::value;
      const SliceConst<float> kc = slice_const<float>(mw, rho);
      rs[a] = ldexpf(1.0f, kc.c);
      un[a] = 1.0f;
      if (kc.zero) {  // v = 0 for the whole line: R unchanged, products 0
        m = 0.0f;
        return;
      }
      if (kc.c >= -100 && kc.c <= 100) {
        un[a] = ldexpf(1.0f, -kc.c);
        m = slice_loop(a_c, maxnext_c, std::false_type{}, R, kc);
      } else {
        m = slice_loop(a_c, maxnext_c, std::true_type{}, R, kc);
      }
    };

    // lo part (planes NHI ..), then the next row's load, then the hi part.
    // The first maxima of both parts are reduced together, so that their
    // two dependent chains overlap.
    const float mwl0 = wave_max_uniform(ml);
    const float mwh0 = wave_max_uniform(mh);
    static_for<0, NLO>([&](auto s) {
      constexpr int S = decltype(s)::value;
      const float mw = S == 0 ? mwl0 : wave_max_uniform(ml);
      slice(std::integral_constant<int, NHI + S>{},
            std::integral_constant<bool, (S + 1 < NLO)>{}, Rl, mw, ml);
    });
    if (PF && row + nw < N) load_row(row + nw);
    static_for<0, NHI>([&](auto s) {
      constexpr int S = decltype(s)::value;
      const float mw = S == 0 ? mwh0 : wave_max_uniform(mh);
      slice(std::integral_constant<int, S>{},
            std::integral_constant<bool, (S + 1 < NHI)>{}, Rh, mw, mh);
    });

    // reduce-scatter: z[k] row q holds pair k + q * NR / 4
    float y[NR / 2], z[NR / 4];
#pragma unroll
    for (int k = 0; k < NR / 2; ++k) y[k] = swap32_sum(acc[k], acc[k + NR / 2]);
#pragma unroll
    for (int k = 0; k < NR / 4; ++k) z[k] = row_sum(swap16_sum(y[k], y[k + NR / 4]));
    ResRow<NP, NT>& rr = rows[nb];
    if ((lane & 15) == 0) {
#pragma unroll
      for (int k = 0; k < NR / 4; ++k) {
        const int p = k + (lane >> 4) * (NR / 4);
        if (p < NP) rr.p[p] = z[k];
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        rr.rs[t] = rs[t];
        rr.un[t] = un[t];
      }
    }
    ++nb;
    if (nb == kResBatch || row + nw >= N) {
      // LDS accesses of one wave complete in order; the clobber keeps the
      // compiler from moving them across this point
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane < nb) {
        const ResRow<NP, NT>& s = rows[lane];
        const int64_t ri = row0 + (int64_t)lane * nw;
        Fold2Sum f;
        f.init();
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const PairInfo q = pair_info(OZK_PIPE_ONDEVICE, NHI, NLO, p);
          f.pair(q, s.p[p] * s.un[q.a], cs[q.b], s.rs[q.a], 0.0, 0.0);
        }
        const double c = f.finish(3);
        r[ri * ldr] = bb - c;
      }
      asm volatile("" ::: "memory");
      nb = 0;
      row0 = row + nw;
      bb = load_b(row0);
    }
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

// Workspace of the row path: x's FP32 slice values, then their exponents.
size_t residual_rows_xs_bytes(int64_t K, int nhi, int nlo) {
  return (size_t)(nhi + nlo) * (size_t)(64 * residual_rows_epl(K)) * sizeof(float);
}
size_t residual_rows_xe_bytes(int nhi, int nlo) {
  return (size_t)(nhi + nlo) * sizeof(int32_t);
}

// r = b - Ozaki(A, x) for one right-hand side x (K elements, stride ldx):
// x's slices into xs / xe (workspace), then the row kernel.  Also clears
// `flags` and sets it for a non-finite x or A.
int launch_residual_rows(const double* A, int64_t N, int64_t K, int64_t lda,
                         const double* x, int64_t ldx, const double* b,
                         int64_t ldb, double* r, int64_t ldr, int rho, int nhi,
                         int nlo, float* xs, int32_t* xe, uint32_t* flags,
                         hipStream_t st) {
  const int epl = residual_rows_epl(K);
  const int64_t kp = 64 * epl;  // the kernel reads xs[p * kp + j * 64 + lane], j < epl
  const int64_t xe_stride = 1;
  hipLaunchKernelGGL(residual_x_kernel, dim3(1), dim3(kResXThreads), 0, st, x, K,
                     ldx, rho, nhi, nlo, kp, xs, xe, flags);
  OZK_LAUNCH_CHECK();
  // persistent grid: one workgroup of kResWaves waves per CU
  const int cus = cu_count();
  // every row start 16-byte aligned: the LDS row copy may be used
  const bool dma_ok = ((uintptr_t)A % 16 == 0) && (lda % 2 == 0 || N == 1);
  const int64_t need = (N + kResWaves - 1) / kResWaves;
  const dim3 grid((unsigned)(need < cus ? need : cus));
#define OZK_RES(E, H, L)                                                           \
  do {                                                                             \
    if (K == 64 * (E) && (E) == 32 && dma_ok)                                      \
      hipLaunchKernelGGL((residual_rows_kernel<E, true, (E) == 32, H, L>), grid,   \
                         dim3(64 * kResWaves), 0, st, A, N, K, lda, xs, xe,        \
                         xe_stride, b, ldb, r, ldr, rho, flags);                   \
    else if (K == 64 * (E))                                                        \
      hipLaunchKernelGGL((residual_rows_kernel<E, true, false, H, L>), grid,       \
                         dim3(64 * kResWaves), 0, st, A, N, K, lda, xs, xe,        \
                         xe_stride, b, ldb, r, ldr, rho, flags);                   \
    else                                                                           \
      hipLaunchKernelGGL((residual_rows_kernel<E, false, false, H, L>), grid,      \
                         dim3(64 * kResWaves), 0, st, A, N, K, lda, xs, xe,        \
                         xe_stride, b, ldb, r, ldr, rho, flags);                   \
  } while (0)
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
