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

#include "fold.h"
#include "sigma.h"

namespace ozk {

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

// Per-row values kept for the batched fold, in LDS: the row and its b, the
// pair sums, then per A slice its row scale 2^c and the factor that turns the
// accumulated sum into the slice product (1, or 2^-c when the unnormalised
// slice values were summed).
template <int NP, int NT>
struct ResRow {
  double b;     // b of the row
  int64_t row;  // the row
  float p[NP];
  float rs[NT];
  float un[NT];
};

// One wave per row over a persistent grid (one workgroup of kResWaves waves
// per CU; rows handed to the waves as described at the row loop).  Lane l
// holds elements k = 64 j + l, j < EPL; x's slices live in registers as BF16
// pairs (elements j, j + 1).  Per row:
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
    const double* __restrict__ x, int64_t ldx, const double* __restrict__ b,
    int64_t ldb, double* __restrict__ r, int64_t ldr, int rho,
    uint32_t* __restrict__ flags) {
  constexpr int NT = NHI + NLO;
  constexpr int NP = pair_count(OZK_PIPE_ONDEVICE, NHI, NLO);
  constexpr int NR = (NP + 3) / 4 * 4;  // pair sums padded for the reduce-scatter
  constexpr int KP = 64 * EPL, H = EPL / 2;
  static_assert(EPL % 2 == 0, "elements are paired");
  static_assert(!DMA || FULL, "the row buffer is filled by whole 1 KiB blocks");
  __shared__ ResRow<NP, NT> red[kResWaves][kResBatch];
  // DMA: each wave's next row, copied into LDS as it lies in memory
  __shared__ double rowbuf[DMA ? kResWaves * KP : 1];
  __shared__ int queue;  // the workgroup's next row index (see below)
  if (threadIdx.x == 0) queue = 0;
  __syncthreads();

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  uint32_t xp[NT][H];  // x's slices, BF16 pairs (elements j, j + 1)
  float cs[NT];        // their scales 2^c

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
  // Rows: workgroup g owns rows g + i G (G workgroups), i = 0, 1, ...  Wave
  // w starts with i = w and i = w + kResWaves; later indices come from the
  // workgroup's LDS counter in the order the waves ask, so that waves the
  // hardware serves unevenly (two share a SIMD) still finish together.  A
  // wave asks for the index after its next one while it works on the
  // current one and stops at the first row >= N it is given; indices are
  // handed out in increasing order, so every row is taken exactly once.
  const int64_t G = gridDim.x;
  auto row_of = [&](int64_t i) { return (int64_t)blockIdx.x + i * G; };
  int64_t cur = row_of(wave), nxt = row_of(wave + kResWaves);
  if (PF && cur < N) load_row(cur);
  if (DMA && cur < N) dma_row(cur);

  // x's slices (x is one column: extract.py:157-191, split matmul.py:204-213),
  // computed by every wave while its first row is in flight, with the split
  // and sigma steps of the extraction kernels; normalised slice values are
  // BF16-exact.  One wave reports a non-finite x.
  {
    float X[2][EPL];
    bool xbad = false;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int k = j * 64 + lane;
      const double v = k < Ki ? x[(int64_t)k * ldx] : 0.0;
      xbad |= !isfinite(v);
      float pr[2];
      split<float>(v, pr);
      X[0][j] = pr[0];
      X[1][j] = pr[1];
    }
    if (blockIdx.x == 0 && wave == 0 && xbad) atomicOr(flags, OZK_FLAG_NONFINITE);
    static_for<0, NT>([&](auto t_c) {
      constexpr int T = decltype(t_c)::value;
      constexpr int Q = T < NHI ? 0 : 1;  // hi part, then lo part
      float m = 0.0f;
#pragma unroll
      for (int j = 0; j < EPL; ++j) m = fmaxf(m, fabsf(X[Q][j]));
      const SliceConst<float> kc = slice_const<float>(wave_max_uniform(m), rho);
      cs[T] = ldexpf(1.0f, kc.c);
#pragma unroll
      for (int i = 0; i < H; ++i) {
        float s[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float rr = X[Q][2 * i + e];
          float v = (rr + kc.sigma) - kc.sigma;
          if (kc.zero) v = 0.0f;
          X[Q][2 * i + e] = rr - v;
          s[e] = slice_value_f32(v, kc.inv);
        }
        xp[T][i] = pack_bf16x2(s[0], s[1]);
      }
    });
  }
  int nb = 0;
  ResRow<NP, NT>* rows = red[wave];

  while (cur < N) {
    if constexpr (DMA) {
      wait_vm<0>();  // this row's copy has landed in LDS
#pragma unroll
      for (int j = 0; j < EPL; ++j) nx[j] = myrow[j * 64 + lane];
      // the reads must complete before the buffer is refilled
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (nxt < N) dma_row(nxt);
    } else if constexpr (!PF) {
      load_row(cur);
    }
    const bool take = nxt < N;
    int q = 0;
    if (take && lane == 0) q = atomicAdd(&queue, 1);
    const double bv = lane == 0 ? b[cur * ldb] : 0.0;
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
    if (PF && nxt < N) load_row(nxt);
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
      rr.b = bv;
      rr.row = cur;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        rr.rs[t] = rs[t];
        rr.un[t] = un[t];
      }
    }
    ++nb;
    if (nb == kResBatch || !take) {
      // LDS accesses of one wave complete in order; the clobber keeps the
      // compiler from moving them across this point
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane < nb) {
        const ResRow<NP, NT>& s = rows[lane];
        Fold2Sum f;
        f.init();
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const PairInfo q = pair_info(OZK_PIPE_ONDEVICE, NHI, NLO, p);
          f.pair(q, s.p[p] * s.un[q.a], cs[q.b], s.rs[q.a], 0.0, 0.0);
        }
        const double c = f.finish(3);
        r[s.row * ldr] = s.b - c;
      }
      asm volatile("" ::: "memory");
      nb = 0;
    }
    cur = nxt;
    nxt = take ? row_of(2 * kResWaves + __builtin_amdgcn_readfirstlane(q)) : N;
  }
}

// Rows longer than one wave holds (K up to 64 EPL W): a workgroup of W waves
// per row over a persistent grid, wave w holding elements k = 64 EPL w +
// 64 j + l, j < EPL, in lane l, with the arithmetic of residual_rows_kernel.
// What crosses waves goes through LDS: the row maxima of every slice (each
// wave's maximum as a bit pattern, then the maximum of the W, so every wave
// gets the same slice constants) and, per row, the waves' pair sums, which
// wave 0 adds and folds.  Every partial sum of a slice product lies on one
// grid below 2^24 units, so the sum over the waves is exact in any order.
// x's slices are extracted the same way, once.
//
// D > 0: the rows reach the waves through an LDS ring of D row buffers
// instead of a one-row register prefetch, so that D rows are in flight per
// workgroup while one is worked on.  Each wave copies its own KW elements of
// a row (global_load_lds_dwordx4, EPL / 2 loads of 1 KiB) and reads only
// those, so its own vmcnt orders the copy before the reads.  Needs 16-byte
// aligned rows and even K.
template <int EPL, bool FULL, int W, int NHI, int NLO, int D = 0, int WPE = 1>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(WPE))) void residual_split_kernel(
    const double* __restrict__ A, int64_t N, int64_t K, int64_t lda,
    const double* __restrict__ x, int64_t ldx, const double* __restrict__ b,
    int64_t ldb, double* __restrict__ r, int64_t ldr, int rho,
    uint32_t* __restrict__ flags) {
  constexpr int NT = NHI + NLO;
  constexpr int NP = pair_count(OZK_PIPE_ONDEVICE, NHI, NLO);
  constexpr int NR = (NP + 3) / 4 * 4;  // pair sums padded for the reduce-scatter
  constexpr int KW = 64 * EPL, H = EPL / 2;
  static_assert(EPL % 2 == 0 && NP <= 128, "elements are paired; one or two pairs per lane");
  __shared__ ResRow<NP, NT> rows[kResBatch];
  __shared__ uint32_t gm[2][W][2];  // the waves' maxima, alternating buffers
  __shared__ float part[W][NR];     // the waves' pair sums of the row

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int kw0 = wave * KW;  // this wave's first element
  const int Ki = (int)K;
  int ph = 0;
  // Maxima over the row of two wave-uniform values (non-negative floats or
  // NaN, compared as bit patterns like wave_max_uniform).  The buffers
  // alternate, so that one barrier per exchange suffices: a buffer is
  // rewritten two exchanges later, after every wave has read it.
  auto row_max2 = [&](float& u, float& v) {
    if (lane == 0) {
      gm[ph][wave][0] = __float_as_uint(u);
      gm[ph][wave][1] = __float_as_uint(v);
    }
    __syncthreads();
    uint32_t mu = 0u, mv = 0u;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      mu = max(mu, gm[ph][w][0]);
      mv = max(mv, gm[ph][w][1]);
    }
    u = __uint_as_float(__builtin_amdgcn_readfirstlane(mu));
    v = __uint_as_float(__builtin_amdgcn_readfirstlane(mv));
    ph ^= 1;
  };
  auto row_max = [&](float u) {
    float v = 0.0f;
    row_max2(u, v);
    return u;
  };

  // LDS ring (D > 0): buffer trow % D of this wave holds its elements of
  // the workgroup's row trow (rows cur = blockIdx.x + trow G).
  constexpr int kDmaPerRow = D > 0 ? KW * 8 / 1024 : 0;
  static_assert(D == 0 || KW % 128 == 0, "whole 1 KiB copies per wave");
  __shared__ double ring[D > 0 ? D : 1][D > 0 ? W : 1][D > 0 ? KW : 1];
  auto dma_row = [&](int64_t row, int slot) {
    // lane l copies elements e, e + 1 (e = 2 l + 128 i) of the wave's part;
    // past the end of a short row it copies the row's last pair instead
    const char* a = (const char*)(A + row * lda);
    const uint32_t base = lds_offset(&ring[slot][wave][0]);
#pragma unroll
    for (int i = 0; i < kDmaPerRow; ++i) {
      int e = kw0 + 128 * i + 2 * lane;
      if constexpr (!FULL) e = e < Ki ? e : Ki - 2;
      dma16(base + i * 1024, a, 8u * (uint32_t)e);
    }
  };
  int trow = 0;  // this workgroup's row counter
  int rslot = 0;  // the ring buffer of the row at hand
  if constexpr (D > 0) {  // the first D rows load while x is extracted
#pragma unroll
    for (int i = 0; i < D; ++i)
      if ((int64_t)blockIdx.x + i * (int64_t)gridDim.x < N)
        dma_row((int64_t)blockIdx.x + i * (int64_t)gridDim.x, i);
  }

  uint32_t xp[NT][H];  // x's slices, BF16 pairs (elements j, j + 1)
  float cs[NT];        // their scales 2^c
  {
    float X[2][EPL];
    bool xbad = false;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int k = kw0 + j * 64 + lane;
      const double v = k < Ki ? x[(int64_t)k * ldx] : 0.0;
      xbad |= !isfinite(v);
      float pr[2];
      split<float>(v, pr);
      X[0][j] = pr[0];
      X[1][j] = pr[1];
    }
    if (blockIdx.x == 0 && xbad) atomicOr(flags, OZK_FLAG_NONFINITE);
    static_for<0, NT>([&](auto t_c) {
      constexpr int T = decltype(t_c)::value;
      constexpr int Q = T < NHI ? 0 : 1;  // hi part, then lo part
      float m = 0.0f;
#pragma unroll
      for (int j = 0; j < EPL; ++j) m = fmaxf(m, fabsf(X[Q][j]));
      const SliceConst<float> kc = slice_const<float>(row_max(wave_max_uniform(m)), rho);
      cs[T] = ldexpf(1.0f, kc.c);
#pragma unroll
      for (int i = 0; i < H; ++i) {
        float s[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float rr = X[Q][2 * i + e];
          float v = (rr + kc.sigma) - kc.sigma;
          if (kc.zero) v = 0.0f;
          X[Q][2 * i + e] = rr - v;
          s[e] = slice_value_f32(v, kc.inv);
        }
        xp[T][i] = pack_bf16x2(s[0], s[1]);
      }
    });
  }

  double nx[EPL];
  auto load_row = [&](int64_t row) {
    const char* a = (const char*)(A + row * lda);
    int Kr = Ki;
    asm volatile("" : "+s"(Kr));
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int k = kw0 + j * 64 + lane;
      if constexpr (FULL) {
        nx[j] = *(const double*)(a + (uint32_t)k * 8u);
      } else {
        const double v = *(const double*)(a + (uint32_t)(k < Kr ? k : Kr - 1) * 8u);
        nx[j] = k < Kr ? v : 0.0;
      }
    }
  };
  // the next row's prefetch fits in registers (not beside max's 65 pair sums)
  constexpr bool PF = EPL <= 16 && D == 0 && NP <= 64;
  const int64_t G = gridDim.x;
  int64_t cur = blockIdx.x;
  if (PF && cur < N) load_row(cur);
  int nb = 0;

  while (cur < N) {  // uniform over the workgroup
    const int64_t nxt = cur + G;
    if constexpr (D > 0) {
      // rows copied after this one: min(D - 1, rows left after it); every
      // other vector memory operation of the wave only adds to the count
      static_assert(D <= 3, "waits for up to two later rows");
      const int64_t later = (N - 1 - cur) / G;
      const int slot = trow % D;
      if (later >= D - 1) wait_vm<(D - 1) * kDmaPerRow>();
      else if (later == 1) wait_vm<kDmaPerRow>();
      else wait_vm<0>();
      rslot = slot;
    } else if constexpr (!PF) {
      load_row(cur);
    }
    // a wave-uniform (scalar) load: a vector load would make the compiler
    // wait for every outstanding copy of the ring before its use
    const double bv = b[cur * ldb];
    float Rh[EPL], Rl[EPL];
    bool bad = false;
    float mh = 0.0f, ml = 0.0f;
    // element j of the row: from the ring (read as it is split, so the row
    // is never held as doubles) or from the register prefetch
    auto elem = [&](int j) -> double {
      if constexpr (D > 0) {
        const int k = kw0 + j * 64 + lane;
        const double v = ring[rslot][wave][j * 64 + lane];
        return (FULL || k < Ki) ? v : 0.0;
      } else {
        return nx[j];
      }
    };
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const double v = elem(j);
      bad |= !isfinite(v);
      float pr[2];
      split<float>(v, pr);
      Rh[j] = pr[0];
      Rl[j] = pr[1];
      if (j & 1) {
        mh = max3_abs(mh, Rh[j - 1], Rh[j]);
        ml = max3_abs(ml, Rl[j - 1], Rl[j]);
      }
    }
    if constexpr (D > 0) {
      // the reads complete before the buffer is refilled with row trow + D
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (cur + (int64_t)D * G < N) dma_row(cur + (int64_t)D * G, rslot);
      ++trow;
    }
    if (bad) atomicOr(flags, OZK_FLAG_NONFINITE);

    float acc[NR];
#pragma unroll
    for (int p = 0; p < NR; ++p) acc[p] = 0.0f;
    float rs[NT], un[NT];

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
    // The slice constants come from the row maximum mw, the same in every
    // wave, so the zero / normalised branches are uniform over the row.
    auto slice = [&](auto a_c, auto maxnext_c, float (&R)[EPL], float mw, float& m) {
      constexpr int a = decltype(a_c)::value;
      const SliceConst<float> kc = slice_const<float>(mw, rho);
      rs[a] = ldexpf(1.0f, kc.c);
      un[a] = 1.0f;
      if (kc.zero) {
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

    float mwl0 = wave_max_uniform(ml), mwh0 = wave_max_uniform(mh);
    row_max2(mwl0, mwh0);
    static_for<0, NLO>([&](auto s) {
      constexpr int S = decltype(s)::value;
      const float mw = S == 0 ? mwl0 : row_max(wave_max_uniform(ml));
      slice(std::integral_constant<int, NHI + S>{},
            std::integral_constant<bool, (S + 1 < NLO)>{}, Rl, mw, ml);
    });
    if (PF && nxt < N) load_row(nxt);
    static_for<0, NHI>([&](auto s) {
      constexpr int S = decltype(s)::value;
      const float mw = S == 0 ? mwh0 : row_max(wave_max_uniform(mh));
      slice(std::integral_constant<int, S>{},
            std::integral_constant<bool, (S + 1 < NHI)>{}, Rh, mw, mh);
    });

    // reduce-scatter within the wave (z[k] of row q of lanes holds pair
    // k + q * NR / 4), then the waves' sums meet in LDS
    float y[NR / 2], z[NR / 4];
#pragma unroll
    for (int k = 0; k < NR / 2; ++k) y[k] = swap32_sum(acc[k], acc[k + NR / 2]);
#pragma unroll
    for (int k = 0; k < NR / 4; ++k) z[k] = row_sum(swap16_sum(y[k], y[k + NR / 4]));
    if ((lane & 15) == 0) {
#pragma unroll
      for (int k = 0; k < NR / 4; ++k) part[wave][k + (lane >> 4) * (NR / 4)] = z[k];
    }
    __syncthreads();
    if (wave == 0) {
      ResRow<NP, NT>& rr = rows[nb];
#pragma unroll
      for (int i = 0; i < (NP + 63) / 64; ++i) {
        const int p = lane + 64 * i;
        if (p < NP) {
          float s = part[0][p];
#pragma unroll
          for (int w = 1; w < W; ++w) s += part[w][p];
          rr.p[p] = s;
        }
      }
      if (lane == 0) {
        rr.b = bv;
        rr.row = cur;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          rr.rs[t] = rs[t];
          rr.un[t] = un[t];
        }
      }
      ++nb;
      if (nb == kResBatch || nxt >= N) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane < nb) {
          const ResRow<NP, NT>& s = rows[lane];
          Fold2Sum f;
          f.init();
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            const PairInfo q = pair_info(OZK_PIPE_ONDEVICE, NHI, NLO, p);
            f.pair(q, s.p[p] * s.un[q.a], cs[q.b], s.rs[q.a], 0.0, 0.0);
          }
          const double c = f.finish(3);
          r[s.row * ldr] = s.b - c;
        }
        asm volatile("" ::: "memory");
        nb = 0;
      }
    }
    cur = nxt;
  }
}

// Right-hand sides and row lengths the fused kernels take: up to
// kResMaxCols columns, each a launch of its own (A is read once per column,
// 8 B an element, against the ~28 B of the slice-GEMM route's plane round
// trip), and K <= 64 * 32 * 8 (eight waves of 2048 elements per row).
constexpr int64_t kResMaxCols = 4;
constexpr int64_t kResMaxK = 64 * 32 * 8;

// The max preset (5, 4): 65 pair sums and 9 slices of x per lane need the
// registers of two waves per SIMD, so its rows run up to kResMaxKMax
// elements (eight waves of 1024).
constexpr int64_t kResMaxKMax = 64 * 16 * 8;

bool residual_rows_supported(int64_t K, int64_t ncols, int nhi, int nlo) {
  if (ncols < 1 || ncols > kResMaxCols || K < 1) return false;
  if (nhi == 5 && nlo == 4) return K <= kResMaxKMax;
  return K <= kResMaxK && ((nhi == 4 && nlo == 1) || (nhi == 3 && nlo == 1));
}

// Values per lane (EPL): rows (and x) of up to 64 EPL elements.
static int residual_rows_epl(int64_t K) {
  int epl = 8;
  while (64 * epl < K) epl *= 2;
  return epl;
}

int launch_fill_u32(uint32_t* p, uint32_t v, hipStream_t st);

// One right-hand side on the one-wave-per-row kernel (K <= 2048).
static void launch_rows_1(const double* A, int64_t N, int64_t K, int64_t lda,
                          const double* x, int64_t ldx, const double* b, int64_t ldb,
                          double* r, int64_t ldr, int rho, int nhi, uint32_t* flags,
                          hipStream_t st) {
  const int epl = residual_rows_epl(K);
  // persistent grid: one workgroup of kResWaves waves per CU
  const int cus = cu_count();
  // every row start 16-byte aligned: the LDS row copy may be used
  const bool dma_ok = ((uintptr_t)A % 16 == 0) && (lda % 2 == 0 || N == 1);
  const int64_t need = (N + kResWaves - 1) / kResWaves;
  const dim3 grid((unsigned)(need < cus ? need : cus));
#define OZK_RES(E, H, L)                                                         \
  do {                                                                           \
    if (K == 64 * (E) && (E) == 32 && dma_ok)                                    \
      hipLaunchKernelGGL((residual_rows_kernel<E, true, (E) == 32, H, L>), grid, \
                         dim3(64 * kResWaves), 0, st, A, N, K, lda, x, ldx, b,   \
                         ldb, r, ldr, rho, flags);                               \
    else if (K == 64 * (E))                                                      \
      hipLaunchKernelGGL((residual_rows_kernel<E, true, false, H, L>), grid,     \
                         dim3(64 * kResWaves), 0, st, A, N, K, lda, x, ldx, b,   \
                         ldb, r, ldr, rho, flags);                               \
    else                                                                         \
      hipLaunchKernelGGL((residual_rows_kernel<E, false, false, H, L>), grid,    \
                         dim3(64 * kResWaves), 0, st, A, N, K, lda, x, ldx, b,   \
                         ldb, r, ldr, rho, flags);                               \
  } while (0)
#define OZK_RES_E(H, L)          \
  switch (epl) {                 \
    case 8: OZK_RES(8, H, L); break;   \
    case 16: OZK_RES(16, H, L); break; \
    default: OZK_RES(32, H, L); break; \
  }
  if (nhi == 5) {  // max (5, 4): rows of up to 1024 elements
    if (epl == 8) OZK_RES(8, 5, 4);
    else OZK_RES(16, 5, 4);
  } else if (nhi == 4) {
    OZK_RES_E(4, 1);
  } else {
    OZK_RES_E(3, 1);
  }
#undef OZK_RES_E
#undef OZK_RES
}

// One right-hand side on the split-row kernel (2048 < K <= kResMaxK): W = 4
// waves of 1024 elements up to K = 4096, else 8 waves of 1024 or 2048.
// 16-byte aligned rows of even K come through an LDS ring of one row buffer
// per workgroup, others through the register prefetch.
static void launch_rows_split(const double* A, int64_t N, int64_t K, int64_t lda,
                              const double* x, int64_t ldx, const double* b, int64_t ldb,
                              double* r, int64_t ldr, int rho, int nhi, uint32_t* flags,
                              hipStream_t st) {
  // persistent grid: PER_CU workgroups per CU
  const int64_t cus = cu_count();
  const bool ring = (uintptr_t)A % 16 == 0 && lda % 2 == 0 && K % 2 == 0;
#define OZK_SPLIT_DL(E, W, H, L, D, WPE, PER_CU)                                     \
  do {                                                                               \
    const int64_t g = cus * (PER_CU);                                                \
    const dim3 grid((unsigned)(N < g ? N : g));                                      \
    if (K == 64 * (E) * (W))                                                         \
      hipLaunchKernelGGL((residual_split_kernel<E, true, W, H, L, D, WPE>), grid,    \
                         dim3(64 * (W)), 0, st, A, N, K, lda, x, ldx, b, ldb, r, ldr, \
                         rho, flags);                                                \
    else                                                                             \
      hipLaunchKernelGGL((residual_split_kernel<E, false, W, H, L, D, WPE>), grid,   \
                         dim3(64 * (W)), 0, st, A, N, K, lda, x, ldx, b, ldb, r, ldr, \
                         rho, flags);                                                \
  } while (0)
#define OZK_SPLIT_D(E, W, H, D, WPE, PER_CU) OZK_SPLIT_DL(E, W, H, 1, D, WPE, PER_CU)
  // Rows of up to 8192 elements that come through the ring keep one row
  // buffer per workgroup and at most 128 VGPRs, so that 16 waves share a CU
  // (4 workgroups of 4 waves, or 2 of 8): while one workgroup's waves wait
  // at a row-maximum barrier, another's run.  Others: 8 waves per CU.
#define OZK_SPLIT_K(H)                                                      \
  if (K <= 64 * 16 * 4) {                                                   \
    if (ring) OZK_SPLIT_D(16, 4, H, 1, 4, 4);                               \
    else OZK_SPLIT_D(16, 4, H, 0, 1, 2);                                    \
  } else if (K <= 64 * 16 * 8) {                                            \
    if (ring) OZK_SPLIT_D(16, 8, H, 1, 4, 2);                               \
    else OZK_SPLIT_D(16, 8, H, 0, 1, 1);                                    \
  } else {                                                                  \
    if (ring) OZK_SPLIT_D(32, 8, H, 1, 1, 1);                               \
    else OZK_SPLIT_D(32, 8, H, 0, 1, 1);                                    \
  }
  // max (5, 4): two waves per SIMD (its pair sums and x slices take about
  // 200 VGPRs), 1024 elements per wave
#define OZK_SPLIT_MAX(W, PER_CU)                       \
  if (ring) OZK_SPLIT_DL(16, W, 5, 4, 1, 2, PER_CU);   \
  else OZK_SPLIT_DL(16, W, 5, 4, 0, 2, PER_CU);
  if (nhi == 5) {
    if (K <= 64 * 16 * 2) {
      OZK_SPLIT_MAX(2, 4);
    } else if (K <= 64 * 16 * 4) {
      OZK_SPLIT_MAX(4, 2);
    } else {
      OZK_SPLIT_MAX(8, 1);
    }
  } else if (nhi == 4) {
    OZK_SPLIT_K(4);
  } else {
    OZK_SPLIT_K(3);
  }
#undef OZK_SPLIT_MAX
#undef OZK_SPLIT_K
#undef OZK_SPLIT_D
#undef OZK_SPLIT_DL
}

// r = b - Ozaki(A, x) for up to kResMaxCols right-hand sides (column j of x,
// b and r at x + j, b + j, r + j with strides ldx, ldb, ldr): clears `flags`,
// then runs the row kernel once per column; it sets the flag for a
// non-finite x or A.  Needs no workspace.
int launch_residual_rows(const double* A, int64_t N, int64_t K, int64_t lda,
                         const double* x, int64_t ldx, const double* b,
                         int64_t ldb, double* r, int64_t ldr, int64_t ncols, int rho,
                         int nhi, int nlo, uint32_t* flags, hipStream_t st) {
  (void)nlo;
  const int rc = launch_fill_u32(flags, 0u, st);
  if (rc) return rc;
  // one wave per row up to 2048 elements (max: 1024), else the split rows
  const int64_t k1 = nhi == 5 ? 64 * 16 : 64 * 32;
  for (int64_t j = 0; j < ncols; ++j) {
    if (K <= k1)
      launch_rows_1(A, N, K, lda, x + j, ldx, b + j, ldb, r + j, ldr, rho, nhi, flags, st);
    else
      launch_rows_split(A, N, K, lda, x + j, ldx, b + j, ldb, r + j, ldr, rho, nhi, flags,
                        st);
    OZK_LAUNCH_CHECK();
  }
  return OZK_OK;
}

}  // namespace ozk
