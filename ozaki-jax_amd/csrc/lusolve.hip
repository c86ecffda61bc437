// Triangular solves with an FP32 LU factor: the refinement steps of
// solve(residual_mode="ozaki") solve A32 d = r with the factor of A32
// (ozaki_jax/solve.py:159, :164, where jnp.linalg.solve re-solves with the
// same matrix).  Latency-bound: one right-hand side is a chain of n / 64
// dependent 64-row blocks.
#include <cfloat>

#include "common.h"

namespace ozk {

constexpr int kTsRows = 64;   // rows per block (one wave solves a block)
constexpr int kTsWaves = 4;   // waves per workgroup
constexpr int kTsThreads = kTsRows * kTsWaves;
// Polls of a block's words before the wait is abandoned: a poll takes about a
// microsecond (an agent-scope load plus s_sleep), a whole solve a few
// hundred, so this only ends waits that cannot finish.
constexpr uint32_t kTsSpinLimit = 1u << 21;

// Lane j's value, for every lane (the builtin moves 32-bit integers).
__device__ __forceinline__ float lane_value(float v, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

// A solution value is published as one 64-bit word, its FP32 bits below
// kTsTag: value and readiness arrive together, with no flag or fence.
constexpr uint32_t kTsTag = 1u;

// Forward (UPPER false: y = L^-1 P b, L unit lower) or backward (UPPER true:
// x = U^-1 y) substitution.  LU is n x n row-major with leading dimension
// lda.  Rows are cut into nb = ceil(n / 64) blocks; workgroup g of G handles
// blocks g, g + G, ... (counted from the bottom going backward) of
// right-hand side column c0 + blockIdx.y.
//
// Block k needs the solution of every block before it (after it, going
// backward).  Each wave takes every fourth of those blocks in the order they
// complete: it loads its 64 x 64 piece of LU (before waiting), polls the
// block's 64 published words until all carry kTsTag, and accumulates the
// product.  Wave 0 then sums the four partial products, solves the diagonal
// block (lane i holds row i; a step broadcasts x_j with lane_value) and
// publishes the block's solution (and writes x going backward).
// Dependencies point only to blocks a workgroup reaches earlier, so with all
// G workgroups resident every wait ends; a wait that still exceeds
// spin_limit polls (kTsSpinLimit unless a test set another limit with
// ozk_set_wait_polls), or sees another one fail, sets OZK_FLAG_WAIT_TIMEOUT
// and stops waiting, so that every wave exits.
template <bool UPPER>
__global__ __launch_bounds__(kTsThreads) void lu_trsv_kernel(
    const float* __restrict__ LU, int64_t n, int64_t lda, int vec,
    const int32_t* __restrict__ perm, const double* __restrict__ B, int64_t ldb,
    const uint64_t* __restrict__ win, uint64_t* __restrict__ wout, int64_t ldw,
    double* __restrict__ X, int64_t ldx, int64_t c0, uint32_t* __restrict__ status,
    uint32_t spin_limit) {
  const int nb = (int)((n + kTsRows - 1) / kTsRows);
  const int64_t col = c0 + blockIdx.y;
  __shared__ float part[kTsWaves][kTsRows];
  __shared__ float4 xs[kTsWaves][kTsRows / 4];  // a wave's copy of a finished block
  const int w = threadIdx.x / kTsRows, lane = threadIdx.x % kTsRows;
  bool failed = false;

  for (int g = blockIdx.x; g < nb; g += gridDim.x) {
    const int blk = UPPER ? nb - 1 - g : g;
    const int64_t row = (int64_t)blk * kTsRows + lane;
    const bool live = row < n;
    const float* const lrow = LU + (live ? row : 0) * lda;
    const int ndep = UPPER ? nb - 1 - blk : blk;

    // Wave 0's right-hand side and diagonal-block row, loaded ahead of the
    // waits so that the solve after the last one starts at once.
    float rhs = 0.0f, dg[kTsRows];
    // Going backward the row is scaled by 1/u (u its diagonal entry), so that
    // the diagonal block is unit upper triangular and its solve, like the
    // forward one, is a broadcast and an FMA per step: the division leaves
    // the chain of dependent steps.
    // A block with a diagonal entry below FLT_MIN, whose reciprocal can
    // overflow (0 * inf would then turn the row's zeros into NaN), is left
    // unscaled instead and divides in the chain (`plain`, wave-uniform).
    float ur = 0.0f, u = 1.0f;
    bool plain = false;
    if (w == 0) {
      if (live)
        rhs = UPPER ? __uint_as_float((uint32_t)win[row * ldw + col])
                    : (float)B[(int64_t)perm[row] * ldb + col];
      if (UPPER) {
        if (live) u = lrow[row];
        plain = __any(!(fabsf(u) >= FLT_MIN));
        if (live) ur = plain ? 1.0f : 1.0f / u;
      }
      const int64_t k0 = (int64_t)blk * kTsRows;
#pragma unroll
      for (int j = 0; j < kTsRows; ++j) {
        dg[j] = (live && k0 + j < n) ? lrow[k0 + j] : 0.0f;
        if (UPPER) dg[j] *= ur;
      }
    }

    float acc = 0.0f;
    for (int d = w; d < ndep; d += kTsWaves) {
      const int c = UPPER ? nb - 1 - d : d;
      const int64_t k0 = (int64_t)c * kTsRows;
      float a[kTsRows];
      if (vec && live && k0 + kTsRows <= n) {
        const float4* const p = (const float4*)(lrow + k0);
#pragma unroll
        for (int q = 0; q < kTsRows / 4; ++q) {
          const float4 v = p[q];
          a[4 * q] = v.x;
          a[4 * q + 1] = v.y;
          a[4 * q + 2] = v.z;
          a[4 * q + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < kTsRows; ++j) a[j] = (live && k0 + j < n) ? lrow[k0 + j] : 0.0f;
      }
      // poll the block's words until every lane's value has arrived
      float xv = 0.0f;
      bool ready = k0 + lane >= n || failed;
      uint32_t spins = 0;
      while (true) {
        if (!ready) {
          const uint64_t wd = __hip_atomic_load(wout + (k0 + lane) * ldw + col, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
          if ((uint32_t)(wd >> 32) == kTsTag) {
            ready = true;
            xv = __uint_as_float((uint32_t)wd);
          }
        }
        if (__all(ready)) break;
        if (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &
                OZK_FLAG_WAIT_TIMEOUT ||
            ++spins > spin_limit) {
          failed = true;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      // broadcast through LDS (one wave: no barrier), so that the 64 values
      // need no scalar registers
      ((float*)xs[w])[lane] = xv;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int q = 0; q < kTsRows / 4; ++q) {
        const float4 x4 = xs[w][q];
        acc = fmaf(a[4 * q], x4.x, acc);
        acc = fmaf(a[4 * q + 1], x4.y, acc);
        acc = fmaf(a[4 * q + 2], x4.z, acc);
        acc = fmaf(a[4 * q + 3], x4.w, acc);
      }
      __builtin_amdgcn_wave_barrier();  // the next block's write waits for these reads
    }
    part[w][lane] = acc;
    __syncthreads();

    if (w == 0) {
      float v = 0.0f;
      if (live) v = rhs - ((part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]));
      if (UPPER) v *= ur;  // the scaled row's right-hand side (0 past n)
      // d = lane - j, stepped with j and opaque to the compiler, so that the
      // lane tests are made at each step; otherwise all 64 lane masks are
      // hoisted into scalar registers and spilled
      if (UPPER && !plain) {
        int d = lane - (kTsRows - 1);
#pragma unroll
        for (int j = kTsRows - 1; j >= 0; --j, ++d) {
          asm volatile("" : "+v"(d));  // (opaque: see above)
          const float xj = lane_value(v, j);
          v = d < 0 ? fmaf(-dg[j], xj, v) : v;
        }
      } else if (UPPER) {  // unscaled rows: lane j divides by u before step j
        int d = lane - (kTsRows - 1);
#pragma unroll
        for (int j = kTsRows - 1; j >= 0; --j, ++d) {
          asm volatile("" : "+v"(d));
          v = d == 0 ? v / u : v;
          const float xj = lane_value(v, j);
          v = d < 0 ? fmaf(-dg[j], xj, v) : v;
        }
      } else {
        int d = lane;
#pragma unroll
        for (int j = 0; j < kTsRows; ++j, --d) {
          asm volatile("" : "+v"(d));
          const float xj = lane_value(v, j);
          v = d > 0 ? fmaf(-dg[j], xj, v) : v;
        }
      }
      if (live) {
        __hip_atomic_store(wout + row * ldw + col,
                           (uint64_t)kTsTag << 32 | __float_as_uint(v), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        if (UPPER) X[row * ldx + col] = (double)v;
      }
    }
    __syncthreads();  // part[] is rewritten by the next block
  }
  if (failed && lane == 0) atomicOr(status, OZK_FLAG_WAIT_TIMEOUT);
}

__global__ void fill_u64_array_kernel(uint64_t* p, int64_t count, uint64_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// Columns per launch: the G x chunk workgroups of a launch must be resident
// together (one per CU suffices).
static int64_t ts_chunk(int64_t ncols) {
  const int64_t cus = cu_count();
  return ncols < cus ? ncols : cus;
}

// Two arrays of published words, n x ncols each: the forward pass's and the
// backward pass's.
size_t lu_solve_workspace_bytes(int64_t n, int64_t ncols) {
  return (size_t)(2 * n * ncols) * sizeof(uint64_t);
}

int launch_lu_solve(const float* LU, int64_t lda, const int32_t* perm, int64_t n,
                    const double* B, int64_t ldb, double* X, int64_t ldx, int64_t ncols,
                    void* ws, uint32_t* status, hipStream_t st) {
  uint64_t* const wf = (uint64_t*)ws;
  uint64_t* const wb = wf + n * ncols;
  const int64_t nb = (n + kTsRows - 1) / kTsRows;
  const int64_t chunk = ts_chunk(ncols);
  const int vec = ((uintptr_t)LU % 16 == 0) && (lda % 4 == 0);
  const int64_t per = cu_count() / chunk;
  // Without gangs (ozk_set_gangs(0)) one workgroup solves all blocks of its
  // column: its waits are then only for words that its own wave 0 stored
  // before the barrier ending the previous block, and they take the
  // built-in limit.
  const bool one = !gangs_enabled();
  const unsigned G = one ? 1u : (unsigned)(nb < per ? nb : (per > 0 ? per : 1));
  const int64_t words = 2 * n * ncols;
  const int64_t fb = (words + 255) / 256;
  hipLaunchKernelGGL(fill_u64_array_kernel, dim3((unsigned)(fb < 4096 ? fb : 4096)), dim3(256), 0,
                     st, wf, words, (uint64_t)0);
  OZK_LAUNCH_CHECK();
  const uint32_t spin_limit = one ? kTsSpinLimit : wait_polls(kTsSpinLimit);
  for (int64_t c0 = 0; c0 < ncols; c0 += chunk) {
    const int64_t nc = ncols - c0 < chunk ? ncols - c0 : chunk;
    hipLaunchKernelGGL(lu_trsv_kernel<false>, dim3(G, (unsigned)nc), dim3(kTsThreads), 0, st,
                       LU, n, lda, vec, perm, B, ldb, nullptr, wf, ncols, X, ldx, c0, status,
                       spin_limit);
    OZK_LAUNCH_CHECK();
    hipLaunchKernelGGL(lu_trsv_kernel<true>, dim3(G, (unsigned)nc), dim3(kTsThreads), 0, st,
                       LU, n, lda, vec, perm, B, ldb, wf, wb, ncols, X, ldx, c0, status,
                       spin_limit);
    OZK_LAUNCH_CHECK();
  }
  return OZK_OK;
}

}  // namespace ozk
