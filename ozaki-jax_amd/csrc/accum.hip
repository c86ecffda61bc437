// Standalone 2Sum accumulation of per-pair products (the reference's
// accumulate_2sum, pallas_ops.py:178-239 through :372-396).  The fused GEMM
// applies the same order inside its epilogue; this kernel serves callers
// that hold the products themselves.  HBM-bound: every product is read once.

#include "common.h"

namespace ozk {

constexpr int kAccMaxBlocks = 8, kAccMaxGroups = 256;

// Block / group structure of the products, passed by value.
struct GroupTable {
  int nblk;
  int ngrp[kAccMaxBlocks];   // groups of each block
  int size[kAccMaxGroups];   // products of each group, in order
};

__device__ __forceinline__ void two_sum_add(float& hi, float& lo, float x) {
  const float t = hi + x;
  const float e = (hi - t) + x;
  hi = t;
  lo = lo + e;
}

// One thread per output element (grid-stride).  For each block: per group,
// the products times their column scales are 2Sum-summed from zero, the
// group's (hi, lo) is multiplied by its row scale, and hi then lo are
// 2Sum-added into the block's pair; then the blocks' hi parts, followed by
// their lo parts, are 2Sum-added into (C_hi, C_lo) (pallas_ops.py:198-239).
__global__ __launch_bounds__(256) void accumulate_2sum_kernel(
    const float* __restrict__ P, int64_t N, int64_t M,
    const float* __restrict__ cs, const float* __restrict__ rs, GroupTable tab,
    float* __restrict__ Ch, float* __restrict__ Cl) {
  const int64_t nm = N * M;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < nm;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = e / M, m = e - n * M;
    float bh[kAccMaxBlocks], bl[kAccMaxBlocks];
    int64_t p = 0;
    int g = 0;
#pragma unroll
    for (int b = 0; b < kAccMaxBlocks; ++b) {
      float h = 0.0f, l = 0.0f;
      if (b < tab.nblk) {
        for (int gi = 0; gi < tab.ngrp[b]; ++gi, ++g) {
          float ih = 0.0f, il = 0.0f;
          for (int t = 0; t < tab.size[g]; ++t, ++p)
            two_sum_add(ih, il, P[p * nm + e] * cs[p * M + m]);
          const float r = rs[(int64_t)g * N + n];
          ih = ih * r;
          il = il * r;
          two_sum_add(h, l, ih);
          two_sum_add(h, l, il);
        }
      }
      bh[b] = h;
      bl[b] = l;
    }
    float ch = 0.0f, cl = 0.0f;
#pragma unroll
    for (int b = 0; b < kAccMaxBlocks; ++b)
      if (b < tab.nblk) two_sum_add(ch, cl, bh[b]);
#pragma unroll
    for (int b = 0; b < kAccMaxBlocks; ++b)
      if (b < tab.nblk) two_sum_add(ch, cl, bl[b]);
    Ch[e] = ch;
    Cl[e] = cl;
  }
}

}  // namespace ozk

extern "C" int ozk_accumulate_2sum(const float* products, int64_t n_products,
                                   int64_t N, int64_t M, const float* col_scales,
                                   const float* row_scales,
                                   const int32_t* block_ngroups, int n_blocks,
                                   const int32_t* group_sizes, int n_groups,
                                   float* C_hi, float* C_lo, void* stream) {
  using namespace ozk;
  clear_error();
  OZK_CHECK_ARG(N >= 0 && M >= 0 && n_products >= 0, "invalid shape");
  OZK_CHECK_ARG(n_blocks >= 0 && n_blocks <= kAccMaxBlocks,
                "at most %d blocks (got %d)", kAccMaxBlocks, n_blocks);
  OZK_CHECK_ARG(n_groups >= 0 && n_groups <= kAccMaxGroups,
                "at most %d groups (got %d)", kAccMaxGroups, n_groups);
  OZK_CHECK_ARG((n_blocks == 0 || block_ngroups) && (n_groups == 0 || group_sizes),
                "null group table");
  GroupTable tab{};
  tab.nblk = n_blocks;
  int64_t groups = 0, prods = 0;
  for (int b = 0; b < n_blocks; ++b) {
    OZK_CHECK_ARG(block_ngroups[b] >= 0, "negative group count in block %d", b);
    tab.ngrp[b] = block_ngroups[b];
    groups += block_ngroups[b];
  }
  OZK_CHECK_ARG(groups == n_groups, "blocks hold %lld groups, %d given",
                (long long)groups, n_groups);
  for (int g = 0; g < n_groups; ++g) {
    OZK_CHECK_ARG(group_sizes[g] >= 0, "negative size of group %d", g);
    tab.size[g] = group_sizes[g];
    prods += group_sizes[g];
  }
  OZK_CHECK_ARG(prods == n_products, "groups hold %lld products, %lld given",
                (long long)prods, (long long)n_products);
  OZK_CHECK_ARG(N * M == 0 || (C_hi && C_lo), "null output pointer");
  OZK_CHECK_ARG(N * M == 0 || n_products == 0 || (products && col_scales),
                "null products / column scales");
  OZK_CHECK_ARG(N * M == 0 || n_groups == 0 || row_scales, "null row scales");
  if (N * M == 0) return OZK_OK;
  int64_t blocks = (N * M + 255) / 256;
  const int64_t cap = (int64_t)cu_count() * 8;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(accumulate_2sum_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, products, N, M, col_scales, row_scales, tab,
                     C_hi, C_lo);
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}
