// FP32 LU factorisation with partial pivoting, in place and row-major: the
// factorisation inside the reference's FP32 solve (jnp.linalg.solve(A32, .),
// ozaki_jax/solve.py:159).  Right-looking and blocked by panels of 32
// columns; each panel step is three kernels:
//  1. lu_panel_kernel (one workgroup): factors the panel's rows c .. n-1 in
//     registers, 16 columns at a time (each column: a pivot search and the
//     rank-1 update of the rows not yet pivots; rows stay where they were
//     read and their final positions are composed after the panel), and
//     writes the permutation the panel's swaps make of the rows;
//  2. lu_rowfix_trsm_kernel (64 columns outside the panel per workgroup):
//     applies that permutation to its columns (and to the permutation
//     vector) and, right of the panel, solves the unit-lower 32 x 32
//     diagonal block for its rows c .. c+31 (the U12 block);
//  3. lu_update_kernel: trailing A22 -= L21 U12, 64 x 64 tiles, K = 32.
// The panel step is the critical path: 32 pivot searches, one workgroup
// barrier each.
#include <cfloat>

#include "common.h"

namespace ozk {

constexpr int kLuThreads = 512;                  // panel workgroup
constexpr int kLuRpt = 8;                        // rows per thread
constexpr int kLuSub = 16;                       // sub-panel columns, in registers
constexpr int kLuPanel = 2 * kLuSub;             // panel width
constexpr int kLuMaxRows = kLuThreads * kLuRpt;  // panel height the registers hold
constexpr int kLuPairs = 2 * kLuPanel;           // rows a panel's swaps can move
constexpr int kLuWaves = kLuThreads / 64;
constexpr int kLuMapInts = 1 + 2 * kLuPairs;

// ---------------------------------------------------------------- waves
template <int CTRL>
__device__ __forceinline__ uint32_t lu_dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

// Wave-uniform maximum (MAX) or minimum of u: quad, half-row and row
// mirrors, then the two permlane swaps across rows of 16 and 32 lanes.
template <bool MAX>
__device__ __forceinline__ uint32_t lu_wave_reduce(uint32_t u) {
  auto op = [](uint32_t x, uint32_t y) { return MAX ? max(x, y) : min(x, y); };
  u = op(u, lu_dpp<0xB1>(u));   // quad_perm [1, 0, 3, 2]
  u = op(u, lu_dpp<0x4E>(u));   // quad_perm [2, 3, 0, 1]
  u = op(u, lu_dpp<0x141>(u));  // half-row mirror
  u = op(u, lu_dpp<0x140>(u));  // row mirror
  {
    const auto s = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    u = op((uint32_t)s[0], (uint32_t)s[1]);
  }
  {
    const auto s = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    u = op((uint32_t)s[0], (uint32_t)s[1]);
  }
  return __builtin_amdgcn_readfirstlane(u);
}

// ---------------------------------------------------------------- panel
// The panel's rows stay where they were read: thread t holds physical rows
// t + i * kLuThreads (relative to row c).  A pivot is not moved in
// registers; the kernel tracks positions instead (LAPACK's row order after
// its swaps) and stores every row at its final position.
struct LuPanelShared {
  // per-wave candidates: (|value| bits + 1) << 32 | (INT_MAX - physical row),
  // so that the largest key is the largest value, then the lowest row
  uint64_t ckey[2][kLuWaves];
  float crow[2][kLuWaves][kLuSub];    //   and those rows' sub-panel values
  float la[kLuSub][kLuSub];           // the first sub-panel's pivot rows
  float lb[kLuSub][kLuSub];           //   and their second sub-panel columns
  float u01[kLuSub][kLuSub];          // U block right of the first sub-panel
  int piv[kLuPanel];                  // position swapped with column j's diagonal
  int prow_of[kLuPanel];              // physical pivot row of column j
  int smap[kLuMaxRows];               // position q holds physical row smap[q]
  int inv[kLuMaxRows];                // physical row x sits at position inv[x]
};

// Partial pivoting on one sub-panel in registers: r[i][k] is column OFF + k
// of physical row t + i * kLuThreads (rows < m); bit i of `used` marks the
// rows that are pivots already, and 6-bit field i of pcode receives 1 + the
// column (OFF + j) a row becomes the pivot of.  Column j's pivot is the unused row with the
// largest |value| (on ties the lowest row of the lowest lane); it takes
// position OFF + j, swapping with the row there as LAPACK's getf2 swaps
// (lu_compose_positions works those out from prow_of).  A zero pivot leaves the
// column as it is (its unused entries are zero too) and raises
// OZK_FLAG_SINGULAR.
template <int OFF>
__device__ __forceinline__ void lu_factor_sub(float (&r)[kLuRpt][kLuSub], uint32_t& used,
                                              uint64_t& pcode, int ncols, int m,
                                              LuPanelShared& sh, uint32_t* status) {
  const int t = threadIdx.x, wave = t / 64, lane = t % 64;
  uint32_t present = 0u;  // row slots below the panel's last row
#pragma unroll
  for (int i = 0; i < kLuRpt; ++i) present |= (t + i * kLuThreads < m) ? 1u << i : 0u;
  // (a compile-time column index: the loop body is too large for the
  // unroller, and a run-time j would index r through scratch memory)
  static_for<0, kLuSub>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if (j >= ncols) return;  // uniform
    const int dj = OFF + j;
    const int par = j & 1;
    const uint32_t avail = present & ~used;  // row slots that can still pivot
    // + 1: an unused row holding 0 still beats a lane with no row (bb = 0)
    uint32_t bb = 0u;
    int br = INT_MAX;
#pragma unroll
    for (int i = 0; i < kLuRpt; ++i) {
      if (i * kLuThreads >= m) break;  // uniform: no thread has row slot i
      const uint32_t bits = __float_as_uint(fabsf(r[i][j])) + 1u;
      if (((avail >> i) & 1u) && bits > bb) {
        bb = bits;
        br = t + i * kLuThreads;
      }
    }
    const uint32_t wb = lu_wave_reduce<true>(bb);
    const uint64_t tie = __ballot(bb == wb);
    const int wr = __builtin_amdgcn_readlane(br, (int)__builtin_ctzll(tie));
    if (lane == 0) sh.ckey[par][wave] = (uint64_t)wb << 32 | (uint32_t)(INT_MAX - wr);
    if (wr != INT_MAX && lane == (wr & 63)) {  // the candidate's lane
      const int iw = wr / kLuThreads;          // wave-uniform
      static_for<0, kLuRpt>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        if (i == iw) {
          float4* const d = (float4*)sh.crow[par][wave];
#pragma unroll
          for (int q = 0; q < kLuSub / 4; ++q)
            d[q] = make_float4(r[i][4 * q], r[i][4 * q + 1], r[i][4 * q + 2], r[i][4 * q + 3]);
          // (distinct per case: keeps the compiler from merging the cases
          // into one store of a run-time-indexed row)
          asm volatile("; lu candidate row %0" ::"n"(i));
        }
      });
    }
    __syncthreads();

    // all keys first, then the maximum: one LDS round trip
    uint64_t keys[kLuWaves];
#pragma unroll
    for (int q = 0; q < kLuWaves; ++q) keys[q] = sh.ckey[par][q];
    uint64_t best = keys[0];
#pragma unroll
    for (int q = 1; q < kLuWaves; ++q) best = keys[q] > best ? keys[q] : best;
    const int pr = __builtin_amdgcn_readfirstlane(INT_MAX - (int)(uint32_t)best);
    const int pw = (pr % kLuThreads) / 64;  // the wave holding that row
    float prow[kLuSub];
#pragma unroll
    for (int k = 0; k < kLuSub; ++k) prow[k] = sh.crow[par][pw][k];
    if (t == pr % kLuThreads) {  // the pivot's owner; its slot ip is uniform
      const int ip = pr / kLuThreads;
      used |= 1u << ip;
      pcode |= (uint64_t)(dj + 1) << (6 * ip);
    }
    if (t == 0) sh.prow_of[dj] = pr;  // positions are composed after the sub-panel
    const float pv = prow[j];
    if (pv != 0.0f) {  // uniform
      // LAPACK's getf2 scales by the reciprocal when it is representable.
      // Pivot rows (old and new) get l = 0, which leaves them as they are.
      const bool recip = fabsf(pv) >= FLT_MIN;  // uniform
      const float rinv = 1.0f / pv;
      const uint32_t act_bits = avail & ~used;  // the new pivot is out too
#pragma unroll
      for (int i = 0; i < kLuRpt; ++i) {
        if (i * kLuThreads >= m) break;  // uniform
        const bool act = (act_bits >> i) & 1u;
        float q;
        if (recip)  // uniform: the division is only paid for tiny pivots
          q = r[i][j] * rinv;
        else
          q = r[i][j] / pv;
        const float l = act ? q : 0.0f;
        r[i][j] = act ? q : r[i][j];
#pragma unroll
        for (int k = j + 1; k < kLuSub; ++k) r[i][k] = fmaf(-l, prow[k], r[i][k]);
      }
    } else if (t == 0) {
      atomicOr(status, OZK_FLAG_SINGULAR);
    }
  });
}

// LAPACK's swap sequence of the panel (column j swaps position j with the
// position its pivot row sits at) composed by wave 0 after the last column:
// only the physical rows 0 .. 31 and the pivot rows ever move, so lane k
// follows one of them (lanes 0-31: rows 0-31, lanes 32-63: the pivot row of
// column k - 32) through the w swaps.  Writes inv[row] and smap[position]
// for those rows and piv[j], the position column j swapped with.
__device__ __forceinline__ void lu_compose_positions(int w, int m, LuPanelShared& sh) {
  const int t = threadIdx.x;
  if (t >= 64) return;
  const int pf = t < kLuPanel && t < w ? sh.prow_of[t] : -1;  // lane j: column j's pivot
  int row = -1;
  if (t < kLuPanel) {
    if (t < m) row = t;
  } else if (t - kLuPanel < w) {
    row = sh.prow_of[t - kLuPanel];
  }
  int pos = row;
  for (int j = 0; j < w; ++j) {  // uniform
    const int pr = __builtin_amdgcn_readlane(pf, j);
    const uint64_t hit = __ballot(row == pr);  // lane kLuPanel + j at least
    const int pp = __builtin_amdgcn_readlane(pos, (int)__builtin_ctzll(hit));
    pos = pos == j ? pp : (pos == pp ? j : pos);
    if (t == 0) sh.piv[j] = pp;
  }
  if (row >= 0) {  // a row followed by two lanes gets the same values twice
    sh.inv[row] = pos;
    sh.smap[pos] = row;
  }
}

// Rows i in [I0, I1) of a sub-panel from global: r[i][k] = P[ph * lda +
// col0 + k] for physical row ph and k < ncols, zero elsewhere.  VEC: 16-byte
// loads (lda % 4 == 0, 16-byte aligned A; col0 is a multiple of 16).
template <bool VEC, int I0, int I1>
__device__ __forceinline__ void lu_load_rows(float (&r)[kLuRpt][kLuSub], const float* P,
                                             int64_t lda, int col0, int ncols, int m) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = I0; i < I1; ++i) {
    const int ph = t + i * kLuThreads;
    const bool live = ph < m;
    const float* const row = P + (int64_t)(live ? ph : 0) * lda + col0;
    if (VEC && ncols == kLuSub) {
#pragma unroll
      for (int q = 0; q < kLuSub / 4; ++q) {
        const float4 v = live ? ((const float4*)row)[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        r[i][4 * q] = v.x;
        r[i][4 * q + 1] = v.y;
        r[i][4 * q + 2] = v.z;
        r[i][4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int k = 0; k < kLuSub; ++k) r[i][k] = (live && k < ncols) ? row[k] : 0.0f;
    }
  }
}

// Stores the rows whose bit in `skip` is clear at position pos(ph).
template <bool VEC, class Pos>
__device__ __forceinline__ void lu_store_rows(const float (&r)[kLuRpt][kLuSub], float* P,
                                              int64_t lda, int col0, int ncols, int m,
                                              uint32_t skip, Pos pos) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < kLuRpt; ++i) {
    const int ph = t + i * kLuThreads;
    if (ph >= m || ((skip >> i) & 1u)) continue;
    float* const row = P + (int64_t)pos(ph) * lda + col0;
    if (VEC && ncols == kLuSub) {
#pragma unroll
      for (int q = 0; q < kLuSub / 4; ++q)
        ((float4*)row)[q] = make_float4(r[i][4 * q], r[i][4 * q + 1], r[i][4 * q + 2],
                                        r[i][4 * q + 3]);
    } else {
#pragma unroll
      for (int k = 0; k < kLuSub; ++k)
        if (k < ncols) row[k] = r[i][k];
    }
  }
}

// b[i] -= a[i] U01 for the rows that are not pivots of the first sub-panel,
// i in [I0, I1).
template <int I0, int I1>
__device__ __forceinline__ void lu_update_rows(float (&b)[kLuRpt][kLuSub],
                                               const float (&a)[kLuRpt][kLuSub], int m,
                                               uint32_t used, const LuPanelShared& sh) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = I0; i < I1; ++i) {
    const int ph = t + i * kLuThreads;
    if (ph >= m || ((used >> i) & 1u)) continue;
#pragma unroll
    for (int q = 0; q < kLuSub; ++q) {
      const float l = a[i][q];
#pragma unroll
      for (int k = 0; k < kLuSub; ++k) b[i][k] = fmaf(-l, sh.u01[q][k], b[i][k]);
    }
  }
}

// Factors panel columns [c, c + w) over rows [c, n) (m = n - c <= kLuMaxRows
// rows, w <= kLuPanel) and writes the row permutation its swaps make to
// maps: maps[0] = w, then kLuPairs destination rows (absolute, -1 = unused)
// and kLuPairs source rows.  Entries e < w are the diagonal positions c + e;
// entries kLuPanel + j are the positions column j's swap exchanged with the
// diagonal, when they lie below the diagonal block.
template <bool VEC>
__global__ __launch_bounds__(kLuThreads) void lu_panel_kernel(float* __restrict__ A,
                                                              int64_t lda, int n, int c, int w,
                                                              int* __restrict__ maps,
                                                              uint32_t* __restrict__ status) {
  __shared__ LuPanelShared sh;
  const int t = threadIdx.x;
  const int m = n - c;
  const int w0 = w < kLuSub ? w : kLuSub, w1 = w - w0;
  float* const P = A + (int64_t)c * lda + c;
  for (int q = t; q < m; q += kLuThreads) {  // (ordered by lu_factor_sub's barriers)
    sh.smap[q] = q;
    sh.inv[q] = q;
  }
  uint32_t used = 0u;
  uint64_t pcode = 0u;

  float a[kLuRpt][kLuSub];
  lu_load_rows<VEC, 0, kLuRpt>(a, P, lda, 0, w0, m);
  lu_factor_sub<0>(a, used, pcode, w0, m, sh, status);
  // The first sub-panel's columns go back to the rows they came from; the
  // panel's permutation moves them at the end.
  lu_store_rows<VEC>(a, P, lda, 0, w0, m, 0u, [](int ph) { return ph; });

  const uint32_t used0 = used;
  float b[kLuRpt][kLuSub];
  if (w1 > 0) {
#pragma unroll
    for (int i = 0; i < kLuRpt; ++i) {
      const int col = (int)((pcode >> (6 * i)) & 63u) - 1;
      if (col >= 0) {  // a pivot row of the first sub-panel: its L part
#pragma unroll
        for (int k = 0; k < kLuSub; ++k) sh.la[col][k] = a[i][k];
      }
    }
    __syncthreads();  // pivot rows staged; prow_of of the first sub-panel final
    if (t < 64) {
      // U01 = L00^-1 B0; lane j holds column j's pivot row (position j),
      // whose second sub-panel columns nothing has changed yet
      const int jl = t < kLuSub ? t : 0;
      const float* const src = P + (int64_t)sh.prow_of[jl] * lda + kLuSub;
      float lrow[kLuSub], u[kLuSub];
#pragma unroll
      for (int k = 0; k < kLuSub; ++k) {
        lrow[k] = sh.la[jl][k];
        u[k] = k < w1 ? src[k] : 0.0f;
      }
#pragma unroll
      for (int q = 0; q < kLuSub; ++q) {
#pragma unroll
        for (int k = 0; k < kLuSub; ++k) {
          const float uq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(u[k]), q));
          if (t > q && t < kLuSub) u[k] = fmaf(-lrow[q], uq, u[k]);
        }
      }
      if (t < kLuSub) {
#pragma unroll
        for (int k = 0; k < kLuSub; ++k) sh.u01[t][k] = u[k];
      }
    }
    __syncthreads();  // U01 in LDS
    // Half of the rows at a time, so that a and b do not both fill the
    // registers.  The first sub-panel's pivot rows are loaded but left alone.
    lu_load_rows<VEC, 0, kLuRpt / 2>(b, P, lda, kLuSub, w1, m);
    lu_update_rows<0, kLuRpt / 2>(b, a, m, used0, sh);
    lu_load_rows<VEC, kLuRpt / 2, kLuRpt>(b, P, lda, kLuSub, w1, m);
    lu_update_rows<kLuRpt / 2, kLuRpt>(b, a, m, used0, sh);
    lu_factor_sub<kLuSub>(b, used, pcode, w1, m, sh, status);  // its barriers follow every load
    if (t < kLuSub) {  // positions 0 .. 15 hold the first sub-panel's pivots
#pragma unroll
      for (int k = 0; k < kLuSub; ++k)
        if (k < w1) P[(int64_t)t * lda + kLuSub + k] = sh.u01[t][k];
    }
  }
  __syncthreads();  // prow_of final; the first sub-panel's stores done
  lu_compose_positions(w, m, sh);
  __syncthreads();  // inv, smap and piv final
  if (w1 > 0)
    lu_store_rows<VEC>(b, P, lda, kLuSub, w1, m, used0, [&](int ph) { return sh.inv[ph]; });

  // The first sub-panel's columns of the rows the permutation moves:
  // position q takes physical row smap[q].  Load all, then store.
  int dst = -1, src = 0;
  if (t < kLuPairs) {
    if (t < kLuPanel) {
      if (t < w) {
        dst = t;
        src = sh.smap[t];
      }
    } else if (t - kLuPanel < w) {
      const int p = sh.piv[t - kLuPanel];
      if (p >= w) {
        dst = p;
        src = sh.smap[p];
      }
    }
    maps[1 + t] = dst >= 0 ? c + dst : -1;
    maps[1 + kLuPairs + t] = c + src;
  }
  if (t == 0) maps[0] = w;
  // thread t moves entry t % kLuPairs, columns (t / kLuPairs) * 2 and + 1
  static_assert(kLuThreads * 2 == kLuPairs * kLuSub, "one thread per two elements");
  __shared__ int dst_s[kLuPairs], src_s[kLuPairs];
  if (t < kLuPairs) {
    dst_s[t] = dst;
    src_s[t] = src;
  }
  __syncthreads();
  const int e = t % kLuPairs, k0 = (t / kLuPairs) * 2;
  const int de = dst_s[e], se = src_s[e];
  float v[2];
#pragma unroll
  for (int k = 0; k < 2; ++k)
    v[k] = (de >= 0 && k0 + k < w0) ? P[(int64_t)se * lda + k0 + k] : 0.0f;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k)
    if (de >= 0 && k0 + k < w0) P[(int64_t)de * lda + k0 + k] = v[k];
}

// The columns outside the panel [c, c + w), 64 per workgroup (lane = column,
// wave = a sixteenth of the permutation's entries), and the permutation
// vector (the last workgroup): applies the panel's row permutation, every
// source value read before any is written.  Right of the panel, wave 0 then
// solves the unit-lower diagonal block for its 64 columns (rows c .. c+w-1
// become U12) from the values staged in LDS.
constexpr int kLuFixCols = 64;
constexpr int kLuFixThreads = 1024;  // 16 waves, 4 entries each

__global__ __launch_bounds__(kLuFixThreads) void lu_rowfix_trsm_kernel(
    float* __restrict__ A, int64_t lda, int n, int c, const int* __restrict__ maps,
    int32_t* __restrict__ perm) {
  __shared__ float L[kLuPanel][kLuPanel + 1];
  __shared__ float buf[kLuPairs][kLuFixCols + 1];
  const int t = threadIdx.x, lane = t % 64, wv = t / 64;
  const int w = maps[0];
  const int right = n - c - w;
  const int nleft = (c + kLuFixCols - 1) / kLuFixCols;
  const int nright = (right + kLuFixCols - 1) / kLuFixCols;
  constexpr int kPer = kLuPairs / (kLuFixThreads / 64);  // entries per wave

  if ((int)blockIdx.x == nleft + nright) {  // the permutation vector
    int v = 0;
    const int dst = t < kLuPairs ? maps[1 + t] : -1;
    if (dst >= 0) v = perm[maps[1 + kLuPairs + t]];
    __syncthreads();
    if (dst >= 0) perm[dst] = v;
    return;
  }
  const bool is_right = (int)blockIdx.x >= nleft;
  const int64_t x = is_right ? (int64_t)c + w + ((int)blockIdx.x - nleft) * kLuFixCols + lane
                             : (int64_t)blockIdx.x * kLuFixCols + lane;
  const bool live = is_right ? x < n : x < c;
  if (is_right) {
    for (int q = t; q < kLuPanel * kLuPanel; q += kLuFixThreads) {
      const int rr = q / kLuPanel, cc = q % kLuPanel;
      L[rr][cc] = (cc < rr && rr < w) ? A[(int64_t)(c + rr) * lda + c + cc] : 0.0f;
    }
  }
  float v[kPer];
  int dst[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int e = wv * kPer + k;
    dst[k] = maps[1 + e];
    v[k] = (live && dst[k] >= 0) ? A[(int64_t)maps[1 + kLuPairs + e] * lda + x] : 0.0f;
  }
  __syncthreads();  // every load before any store: rows move between waves
  if (is_right) {
#pragma unroll
    for (int k = 0; k < kPer; ++k) buf[wv * kPer + k][lane] = v[k];
    __syncthreads();
    if (wv == 0) {  // entries j < w are the diagonal rows c + j, in order
      // column-oriented: once u[q] is final it updates every later row, so
      // the dependent chain is 32 steps, not 496
      float u[kLuPanel];
#pragma unroll
      for (int j = 0; j < kLuPanel; ++j) u[j] = buf[j][lane];
#pragma unroll
      for (int q = 0; q < kLuPanel - 1; ++q) {
#pragma unroll
        for (int j = q + 1; j < kLuPanel; ++j) u[j] = fmaf(-L[j][q], u[q], u[j]);
      }
#pragma unroll
      for (int j = 0; j < kLuPanel; ++j) buf[j][lane] = u[j];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kPer; ++k) v[k] = buf[wv * kPer + k][lane];
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    if (live && dst[k] >= 0) A[(int64_t)dst[k] * lda + x] = v[k];
}

// Trailing update A[r][x] -= sum_q A[r][c + q] A[c + q][x] over rows and
// columns [c + w, n), q < w <= 32: one 64 x 64 tile per workgroup, 4 x 4
// outputs per thread.  K = 32 makes it bound by the read and write of A22.
template <bool VEC>
__global__ __launch_bounds__(256) void lu_update_kernel(float* __restrict__ A, int64_t lda,
                                                        int n, int c, int w) {
  __shared__ float As[64][kLuPanel + 1];
  __shared__ float4 Bs[kLuPanel][16];
  const int t = threadIdx.x;
  const int s = c + w;
  const int64_t r0 = s + (int64_t)blockIdx.y * 64, x0 = s + (int64_t)blockIdx.x * 64;
  for (int q = t; q < 64 * kLuPanel; q += 256) {
    const int rr = q / kLuPanel, kk = q % kLuPanel;
    As[rr][kk] = (r0 + rr < n && kk < w) ? A[(r0 + rr) * lda + c + kk] : 0.0f;
  }
  for (int q = t; q < kLuPanel * 16; q += 256) {
    const int kk = q / 16, cc = q % 16;
    const int64_t x = x0 + 4 * cc;
    const float* const src = A + (int64_t)(c + kk) * lda + x;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (kk < w) {
      if (VEC && x + 4 <= n) {
        v = *(const float4*)src;
      } else {
        if (x < n) v.x = src[0];
        if (x + 1 < n) v.y = src[1];
        if (x + 2 < n) v.z = src[2];
        if (x + 3 < n) v.w = src[3];
      }
    }
    Bs[kk][cc] = v;
  }
  __syncthreads();
  const int ty = t / 16, tx = t % 16;
  float acc[4][4] = {};
#pragma unroll 4
  for (int kk = 0; kk < kLuPanel; ++kk) {
    const float4 b = Bs[kk][tx];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float l = As[ty * 4 + i][kk];
      acc[i][0] = fmaf(l, b.x, acc[i][0]);
      acc[i][1] = fmaf(l, b.y, acc[i][1]);
      acc[i][2] = fmaf(l, b.z, acc[i][2]);
      acc[i][3] = fmaf(l, b.w, acc[i][3]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = r0 + ty * 4 + i;
    if (r >= n) continue;
    const int64_t x = x0 + 4 * tx;
    float* const dst = A + r * lda + x;
    if (VEC && x + 4 <= n) {
      float4 v = *(float4*)dst;
      v.x -= acc[i][0];
      v.y -= acc[i][1];
      v.z -= acc[i][2];
      v.w -= acc[i][3];
      *(float4*)dst = v;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (x + j < n) dst[j] -= acc[i][j];
    }
  }
}

__global__ void lu_iota_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = i;
}

int64_t lu_factor_max_n() { return kLuMaxRows; }
size_t lu_factor_workspace_bytes() { return kLuMapInts * sizeof(int); }

template <bool VEC>
static int lu_factor_steps(float* A, int64_t lda, int n, int32_t* perm, int* maps,
                           uint32_t* status, hipStream_t st) {
  for (int c = 0; c < n; c += kLuPanel) {
    const int w = n - c < kLuPanel ? n - c : kLuPanel;
    hipLaunchKernelGGL(lu_panel_kernel<VEC>, dim3(1), dim3(kLuThreads), 0, st, A, lda, n, c,
                       w, maps, status);
    OZK_LAUNCH_CHECK();
    const int right = n - c - w;
    const int groups = (c + kLuFixCols - 1) / kLuFixCols + (right + kLuFixCols - 1) / kLuFixCols;
    hipLaunchKernelGGL(lu_rowfix_trsm_kernel, dim3(groups + 1), dim3(kLuFixThreads), 0, st, A,
                       lda, n, c, maps, perm);
    OZK_LAUNCH_CHECK();
    if (right > 0) {
      const unsigned tiles = (unsigned)((right + 63) / 64);
      hipLaunchKernelGGL(lu_update_kernel<VEC>, dim3(tiles, tiles), dim3(256), 0, st, A, lda,
                         n, c, w);
      OZK_LAUNCH_CHECK();
    }
  }
  return OZK_OK;
}

int launch_lu_factor(float* A, int64_t lda, int64_t n, int32_t* perm, void* ws,
                     uint32_t* status, hipStream_t st) {
  hipLaunchKernelGGL(lu_iota_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, perm,
                     (int)n);
  OZK_LAUNCH_CHECK();
  const bool vec = ((uintptr_t)A % 16 == 0) && (lda % 4 == 0);
  return vec ? lu_factor_steps<true>(A, lda, (int)n, perm, (int*)ws, status, st)
             : lu_factor_steps<false>(A, lda, (int)n, perm, (int*)ws, status, st);
}

}  // namespace ozk
