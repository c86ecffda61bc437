// Pair schedules and accumulation orders of the Ozaki scheme, shared by the
// GEMM kernels and the fused residual.
#pragma once

#include "common.h"

namespace ozk {

// ---------------------------------------------------------------- schedule

struct PairInfo {
  int a, b;   // A / B slice (plane) index
  int blk;    // block id (0 hh, 1 hl, 2 lh; host: 0)
  bool gs;    // first pair of its group
  bool ge;    // last pair of its group
  bool bs;    // first pair of its block
  bool be;    // last pair of its block
  bool fg;    // in the first group of its block
};

__host__ __device__ constexpr int pair_count(int pipe, int nhi, int nlo) {
  return pipe == OZK_PIPE_ONDEVICE ? nhi * nhi + 2 * nhi * nlo
                                   : nhi * (nhi + 1) / 2;
}

// Pair p of the schedule.  Ondevice: hh (i, j), hl (i, n_hi + j), lh
// (n_hi + i, j), i-major (pallas_gemm_accum.py:39-53, groups :59-79).
// Host: (i, j) with i + j <= n - 1, i-major (matmul.py:27-31).
__host__ __device__ constexpr PairInfo pair_info(int pipe, int nhi, int nlo,
                                                 int p) {
  PairInfo r{0, 0, 0, false, false, false, false, false};
  if (pipe == OZK_PIPE_ONDEVICE) {
    const int hh = nhi * nhi, hl = nhi * nlo;
    if (p < hh) {
      const int i = p / nhi, j = p % nhi;
      r = PairInfo{i, j, 0, j == 0, j == nhi - 1, p == 0, p == hh - 1, i == 0};
    } else if (p < hh + hl) {
      const int q = p - hh, i = q / nlo, j = q % nlo;
      r = PairInfo{i, nhi + j, 1, j == 0, j == nlo - 1, q == 0, q == hl - 1, i == 0};
    } else {
      const int q = p - hh - hl, i = q / nhi, j = q % nhi;
      r = PairInfo{nhi + i, j, 2, j == 0, j == nhi - 1, q == 0, q == hl - 1, i == 0};
    }
  } else {
    // group i holds the pairs from i n - i (i - 1) / 2 on: count the group
    // starts at or below p (a loop of n - 1 steps, which folds away when n
    // and p are known at compile time)
    const int n = nhi;
    int i = 0;
    for (int t = 1; t < n; ++t) i += p >= t * n - t * (t - 1) / 2 ? 1 : 0;
    const int q = p - (i * n - i * (i - 1) / 2);
    const int np = n * (n + 1) / 2;
    r = PairInfo{i, q, 0, q == 0, q == n - 1 - i, p == 0, p == np - 1, i == 0};
  }
  return r;
}

// ---------------------------------------------------------------- fold

// Scale 2^e of a slice exponent, as the reference forms it (FP32:
// pallas_ops.py:126-164, matmul.py:558-561; FP64: matmul.py:553-556).  The
// exponent OZK_EXP_NONFINITE marks a slice the reference makes NaN / +-inf
// (INT8 planes store zeros there): its scale is NaN, so every product with
// the slice folds as NaN.
__device__ __forceinline__ float scale32(int e) {
  return e == OZK_EXP_NONFINITE ? __builtin_nanf("") : ldexpf(1.0f, e);
}
__device__ __forceinline__ double scale64(int e) {
  return e == OZK_EXP_NONFINITE ? __builtin_nan("") : ldexp(1.0, e);
}

__device__ __forceinline__ void twosum(float& s, float& l, float x) {
  const float t = s + x;
  const float e = (s - t) + x;
  s = t;
  l = l + e;
}

// twosum(s, l, x) from s = l = +0: s = 0 + x, and l = 0 + ((0 - s) + x),
// which is +0 for every finite x (also -0) and NaN for an infinite or NaN
// x, as is x - x.  Two operations instead of four, the same bits.
__device__ __forceinline__ void twosum_from_zero(float& s, float& l, float x) {
  s = x + 0.0f;
  l = x - x;
}

struct Fold2Sum {
  float it, il, bt, bl, ct, cl, p0, p1, p2;
  __device__ __forceinline__ void init() {
    it = il = bt = bl = ct = cl = p0 = p1 = p2 = 0.0f;
  }
  // Pair q's product at its column scale, x = P * 2^cb (pallas_ops.py:206-214).
  // A group's first product, a block's first group sum and block 0's sum
  // start from zeros (the reference's zero-initialised accumulators).
  __device__ __forceinline__ void pair_x(const PairInfo& q, float x, float rs32) {
    if (q.gs) twosum_from_zero(it, il, x);
    else twosum(it, il, x);
    if (q.ge) {
      const float ht = it * rs32, hl = il * rs32;
      if (q.fg) twosum_from_zero(bt, bl, ht);
      else twosum(bt, bl, ht);
      twosum(bt, bl, hl);
      if (q.be) {
        if (q.blk == 0) twosum_from_zero(ct, cl, bt);
        else twosum(ct, cl, bt);
        // value selects, not a store through a selected field: the block id
        // may be a run-time value, and the fold must stay in registers
        p0 = q.blk == 0 ? bl : p0;
        p1 = q.blk == 1 ? bl : p1;
        p2 = q.blk == 2 ? bl : p2;
      }
    }
  }
  __device__ __forceinline__ void pair(const PairInfo& q, float P, float cs32,
                                       float rs32, double, double) {
    pair_x(q, P * cs32, rs32);
  }
  // The blocks' lo parts after their hi parts (pallas_ops.py:230-237): the
  // double-float pair (C_hi, C_lo) ...
  __device__ __forceinline__ void finish_pair(int nblocks, float& hi, float& lo) {
    twosum(ct, cl, p0);
    if (nblocks > 1) twosum(ct, cl, p1);
    if (nblocks > 2) twosum(ct, cl, p2);
    hi = ct;
    lo = cl;
  }
  // ... and its FP64 combine (matmul.py:526, :540).
  __device__ __forceinline__ double finish(int nblocks) {
    float hi, lo;
    finish_pair(nblocks, hi, lo);
    return (double)hi + (double)lo;
  }
};

template <int ORDER>
struct Fold64 {
  double c, in;
  __device__ __forceinline__ void init() { c = 0.0; in = 0.0; }
  __device__ __forceinline__ void pair(const PairInfo& q, float P, float cs32,
                                       float, double cs64, double rs64) {
    if (ORDER == OZK_ORDER_HOST_NP) {
      double t = (double)P * rs64;
      t = t * cs64;
      c = c + t;
      return;
    }
    if (q.gs) in = 0.0;
    if (ORDER == OZK_ORDER_BLOCK64) {
      in = in + (double)(P * cs32);
    } else {  // OZK_ORDER_HOST_JAX
      in = in + (double)P * cs64;
    }
    if (q.ge) {
      in = in * rs64;
      c = c + in;
    }
  }
  __device__ __forceinline__ double finish(int) { return c; }
};

template <int ORDER> struct FoldOf { typedef Fold64<ORDER> type; };
template <> struct FoldOf<OZK_ORDER_2SUM> { typedef Fold2Sum type; };

}  // namespace ozk
