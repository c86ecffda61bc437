// Slice-pair GEMMs on BF16 MFMA (FP32 accumulate) with the reference's
// accumulation order folded into registers.
//
// Products.  Slices are integers on the grid 2^(rho-p) with at most 8
// significant bits, so every BF16 x BF16 product is exact in FP32 and, while
// the partial sums stay below 2^24 grid units (the reference's exactness
// model, matmul.py:615-621), every FP32 sum is exact as well: the product of
// a slice pair is the same bit pattern whatever the summation order.  That is
// why the K loop may use any blocking and any k permutation inside an MFMA
// fragment, provided A and B fragments use the same one.
//
// Tiling (gfx950, 64-wide waves).  A workgroup of 4 waves owns a 64x64 output
// tile; each wave owns a 32x32 sub-tile and keeps one v_mfma_f32_32x32x16_bf16
// accumulator (16 VGPRs per lane) per slice pair.  Per 32-wide K stage the
// workgroup stages every slice plane it needs (A: 64 rows, B: 64 columns)
// into LDS in fragment order: each 1 KiB block holds exactly the 64 lanes'
// 16-byte operands of one MFMA, so fragment reads are conflict-free
// ds_read_b128.  A fragment of A slice a is loaded once per stage and reused
// by every pair (a, b) -- for precision="high" 10 fragments feed 24 MFMAs.
//
// Accumulation.  After the K loop each lane folds its 16 output elements'
// pair products in schedule order (pallas_gemm_accum.py:26-87):
//   2SUM     (A4) pallas_ops.py:195-237  double-float FP32 2Sum chain
//   BLOCK64  (A3) matmul.py:562-597      FP32 col scale, FP64 group sum
//   HOST_JAX (A2) matmul.py:47-64        FP64 col scale, FP64 group sum
//   HOST_NP  (A1) matmul.py:879-898      (f64(P) * row) * col, running sum
// All operations are single IEEE RN ops (-ffp-contract=off), so the result
// is bit-identical to the NumPy restatement of each order.

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
  PairInfo r{0, 0, 0, false, false, false, false};
  if (pipe == OZK_PIPE_ONDEVICE) {
    const int hh = nhi * nhi, hl = nhi * nlo;
    if (p < hh) {
      const int i = p / nhi, j = p % nhi;
      r = PairInfo{i, j, 0, j == 0, j == nhi - 1, p == 0, p == hh - 1};
    } else if (p < hh + hl) {
      const int q = p - hh, i = q / nlo, j = q % nlo;
      r = PairInfo{i, nhi + j, 1, j == 0, j == nlo - 1, q == 0, q == hl - 1};
    } else {
      const int q = p - hh - hl, i = q / nhi, j = q % nhi;
      r = PairInfo{nhi + i, j, 2, j == 0, j == nhi - 1, q == 0, q == hl - 1};
    }
  } else {
    const int n = nhi;
    int q = p, i = 0;
    while (q >= n - i) {
      q -= n - i;
      ++i;
    }
    const int np = n * (n + 1) / 2;
    r = PairInfo{i, q, 0, q == 0, q == n - 1 - i, p == 0, p == np - 1};
  }
  return r;
}

// ---------------------------------------------------------------- fold

__device__ __forceinline__ void twosum(float& s, float& l, float x) {
  const float t = s + x;
  const float e = (s - t) + x;
  s = t;
  l = l + e;
}

struct Fold2Sum {
  float it, il, bt, bl, ct, cl, p0, p1, p2;
  __device__ __forceinline__ void init() {
    it = il = bt = bl = ct = cl = p0 = p1 = p2 = 0.0f;
  }
  __device__ __forceinline__ void pair(const PairInfo& q, float P, float cs32,
                                       float rs32, double, double) {
    if (q.bs) { bt = 0.0f; bl = 0.0f; }
    if (q.gs) { it = 0.0f; il = 0.0f; }
    twosum(it, il, P * cs32);
    if (q.ge) {
      const float ht = it * rs32, hl = il * rs32;
      twosum(bt, bl, ht);
      twosum(bt, bl, hl);
      if (q.be) {
        twosum(ct, cl, bt);
        if (q.blk == 0) p0 = bl;
        else if (q.blk == 1) p1 = bl;
        else p2 = bl;
      }
    }
  }
  __device__ __forceinline__ double finish(int nblocks) {
    twosum(ct, cl, p0);
    if (nblocks > 1) twosum(ct, cl, p1);
    if (nblocks > 2) twosum(ct, cl, p2);
    return (double)ct + (double)cl;
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

// ---------------------------------------------------------------- tiling

constexpr int kBM = 64, kBN = 64, kBK = 32, kThreads = 256;

// Output-tile order: consecutive workgroups go round-robin to the 8 XCDs, so
// first gather each XCD's share into a contiguous range, then walk that range
// in groups of kGroupM tile-rows (column-major inside a group) so that the
// ~32 tiles resident on one XCD share A rows and B columns in its L2.
constexpr int kXcds = 8, kGroupM = 8;

__device__ __forceinline__ void tile_coords(int bid, int ntm, int ntn, int& tm,
                                            int& tn) {
  const int nt = ntm * ntn;
  const int q = nt / kXcds, rem = nt % kXcds;
  const int xcd = bid % kXcds, slot = bid / kXcds;
  const int L = (xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q) + slot;
  const int per_group = kGroupM * ntn;
  const int g = L / per_group, first_m = g * kGroupM;
  const int gsz = min(ntm - first_m, kGroupM);
  const int inner = L - g * per_group;
  tm = first_m + inner % gsz;
  tn = inner / gsz;
}

// LDS offset (in 16-byte units) of the operand of (slot, 32-row group, MFMA
// k-step, lane) inside one stage buffer.  Tile line r (0..63) and 8-wide k
// chunk c (0..3) of a stage go to lane (r & 31) + 32 * (c & 1) of block
// (slot, r >> 5, c >> 1).
__device__ __forceinline__ int frag_off(int slot, int rg, int ks, int lane) {
  return ((slot * 2 + rg) * 2 + ks) * 64 + lane;
}

// One operand side (A or B) of a stage: N slot tiles of 64 lines x 32 k,
// i.e. one 64-byte chunk of each of the tile's lines, which is a contiguous
// 4 KiB block of the plane.  Thread t moves the block's 16-byte unit t
// (line t / 4, stored unit t % 4, which holds logical unit
// (t % 4) ^ unit_swizzle(line)): one 16-byte global load and one 16-byte LDS
// store per slot.
template <int N>
struct HalfStage {
  uint4 v[N];
  __device__ __forceinline__ void load(const uint16_t* const (&ptr)[N],
                                       int64_t stage_stride, int64_t s) {
    const int64_t off = s * stage_stride + (int64_t)threadIdx.x * 8;
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = *(const uint4*)(ptr[i] + off);
  }
  __device__ __forceinline__ void store(uint4* buf, int slot0) const {
    const int t = threadIdx.x;
    const int r = t >> 2, c = (t & 3) ^ unit_swizzle(r);
    const int lane = (r & 31) + 32 * (c & 1);
#pragma unroll
    for (int i = 0; i < N; ++i) buf[frag_off(slot0 + i, r >> 5, c >> 1, lane)] = v[i];
  }
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

// Output element of accumulator register r of a 32x32 MFMA in lane `lane`:
// column lane % 32, row 8 * (r / 4) + 4 * (lane / 32) + r % 4.
__device__ __forceinline__ int acc_row(int r, int lane) {
  return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

// K sweep of the pairwise kernel: double-buffered LDS stages; while one
// buffer feeds the MFMAs the next stage is fetched half by half (A slots
// during k-step 0, B slots during k-step 1) through NA or NB registers.
// `mma(buf, ks)` issues the MFMAs of one 16-wide k-step.  a_ptr / b_ptr
// point at the tile's first line in chunk 0; chunk s lies s * a_stride /
// s * b_stride elements further.
template <int NA, int NB, class MMA>
__device__ __forceinline__ void k_sweep(const uint16_t* const (&a_ptr)[NA],
                                        const uint16_t* const (&b_ptr)[NB],
                                        int64_t a_stride, int64_t b_stride,
                                        int64_t nst, uint4* lds, MMA& mma) {
  constexpr int kBuf = (NA + NB) * 4 * 64;  // uint4 per stage buffer
  {
    HalfStage<NA> ha;
    ha.load(a_ptr, a_stride, 0);
    ha.store(lds, 0);
    HalfStage<NB> hb;
    hb.load(b_ptr, b_stride, 0);
    hb.store(lds, NA);
  }
  __syncthreads();
  for (int64_t s = 0; s < nst; ++s) {
    uint4* cur = lds + (s & 1) * kBuf;
    uint4* nxt = lds + ((s + 1) & 1) * kBuf;
    const bool more = s + 1 < nst;
    {
      HalfStage<NA> ha;
      if (more) ha.load(a_ptr, a_stride, s + 1);
      mma(cur, 0);
      if (more) ha.store(nxt, 0);
    }
    {
      HalfStage<NB> hb;
      if (more) hb.load(b_ptr, b_stride, s + 1);
      mma(cur, 1);
      if (more) hb.store(nxt, NA);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- kernels

// ---------------------------------------------------------------- all pairs
//
// The all-pairs kernel uses 8 waves (2 per SIMD).  Wave w owns rows
// 32 * (w >> 2) .. +31 and columns 16 * (w & 3) .. +15 of the 64x64 tile as
// two 16x16 MFMA blocks, so a pair costs 8 accumulator registers and the 24
// pairs of precision="high" fit with the operand registers in 256.
//
// Operands come in one of two plane formats, each 64 bytes of a line per
// MFMA k-step:
//   BF16  v_mfma_f32_16x16x32_bf16, FP32 accumulators.
//   I8    v_mfma_i32_16x16x64_i8 on q = slice * 2^(24 - rho) (rho >= 19:
//         |q| <= 64), INT32 accumulators; the product is the integer sum
//         scaled by 2^(2 rho - 48), i.e. the same FP32 value as the BF16
//         product whenever that one is exact (partial sums < 2^24 units).
//
// LDS: a ring of kRing stage buffers, one 64-byte chunk of every line each.
// Fragment (slot, 16-line group lg) is the 1 KiB block of lines
// 16 lg .. 16 lg + 15 of that chunk exactly as it lies in the plane (line r
// at byte 64 (r % 16), units swizzled).  Wave w fetches the fragments w,
// w + 8, ... of a stage with contiguous direct global->LDS loads, kRing - 1
// stages ahead of the MFMAs.  MFMA lane l reads line l % 16, logical unit
// l / 16 of a fragment (frag_lane); the swizzle spreads those 64 reads over
// all LDS banks.

constexpr int kThreads16 = 512;
constexpr int kRing = 4;       // stage buffers (kRing - 1 stages in flight)

typedef int int32x4 __attribute__((ext_vector_type(4)));
typedef int int32x16 __attribute__((ext_vector_type(16)));

struct OpBf16 {
  typedef floatx4 acc_t;
  static constexpr int kElemBytes = 2;
  static __device__ __forceinline__ acc_t mma(uint4 a, uint4 b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float product(float x, float) { return x; }
};

struct OpI8 {
  typedef int32x4 acc_t;
  static constexpr int kElemBytes = 1;
  static __device__ __forceinline__ acc_t mma(uint4 a, uint4 b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(
        __builtin_bit_cast(int32x4, a), __builtin_bit_cast(int32x4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float product(int x, float unit2) {
    return (float)x * unit2;
  }
};

// One 16-byte-per-lane direct load from global memory into LDS
// (global_load_lds_dwordx4): lane l's 16 bytes land at LDS offset
// `lds_addr` + 16 l.  `lds_addr` and `gbase` are wave-uniform; `voff` is the
// lane's byte offset from `gbase`.  Written as inline assembly so that the
// compiler does not order the K loop's LDS reads behind these loads: the
// kernel waits for them itself (wait_vm) before the barrier that publishes
// a stage.  M0 carries the LDS address; nothing else in these kernels uses
// M0.
__device__ __forceinline__ void dma16(uint32_t lds_addr, const void* gbase,
                                      uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2"
      :
      : "s"(lds_addr), "v"(voff), "s"(gbase)
      : "memory");
}

// Wait until at most N of this wave's vector-memory loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(size_t)((__attribute__((address_space(3))) const char*)p);
}

// Fetch stage `st` (chunk st of every line of the tile) into the LDS buffer
// at byte offset `buf_lds`: wave w moves fragments F = w + 8 i, i.e. slot
// 2 i + (w >> 2), line group w & 3, each a contiguous 1 KiB of the plane.
// At, Bt point at the tile's first line in chunk 0; chunk st lies
// st * a_stage / st * b_stage bytes further.  All addresses lie inside the
// zero-padded slice planes.
template <int NT>
__device__ __forceinline__ void stage_dma(const char* At, int64_t aplane,
                                          int64_t a_stage, const char* Bt,
                                          int64_t bplane, int64_t b_stage,
                                          int64_t st, uint32_t buf_lds,
                                          int wave, uint32_t lane_bytes) {
  const int64_t g = (int64_t)(wave & 3) * 1024;
  const int64_t qa = st * a_stage + g, qb = st * b_stage + g;
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const int slot = 2 * i + (wave >> 2);
    const char* base = slot < NT ? At + slot * aplane + qa : Bt + (slot - NT) * bplane + qb;
    const int F = 8 * i + wave;
    dma16(__builtin_amdgcn_readfirstlane(buf_lds + F * 1024), (const void*)base,
          lane_bytes);
  }
}

// uint4 index inside a 1 KiB fragment of the 16x16x64 operand of lane l:
// line l % 16, logical unit l / 16.
__device__ __forceinline__ int frag_lane(int lane) {
  return (lane & 15) * 4 + ((lane >> 4) ^ unit_swizzle(lane & 15));
}

template <class Op, int PIPE, int NHI, int NLO, int NT, int NP>
struct AllPairsMMA {
  typename Op::acc_t acc[NP][2];
  int fl, wr, wc;  // fl = frag_lane(lane)

  // MFMAs of one (A slot, row block) for every pair of that A slot.
  template <int SA, int H>
  __device__ __forceinline__ void block(uint4 af, const uint4 (&bf)[NT]) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const PairInfo q = pair_info(PIPE, NHI, NLO, p);
      if (q.a == SA) acc[p][H] = Op::mma(af, bf[q.b], acc[p][H]);
    }
  }

  // The NT * 2 blocks of a stage, A fragments software-pipelined through
  // kDepth + 1 registers: the read of block j + kDepth is issued before the
  // MFMAs of block j.  Scheduling barriers keep the reads where they are.
  static constexpr int kBlocks = NT * 2, kDepth = 3;

  __device__ __forceinline__ uint4 read_a(const uint4* buf, int j) const {
    return buf[((j >> 1) * 4 + 2 * wr + (j & 1)) * 64 + fl];
  }

  template <int J>
  __device__ __forceinline__ void pipe_step(const uint4* buf,
                                            uint4 (&af)[kDepth + 1],
                                            const uint4 (&bf)[NT]) {
    if constexpr (J < kBlocks) {
      if constexpr (J + kDepth < kBlocks)
        af[(J + kDepth) % (kDepth + 1)] = read_a(buf, J + kDepth);
      block<J / 2, J % 2>(af[J % (kDepth + 1)], bf);
      __builtin_amdgcn_sched_barrier(0);
      pipe_step<J + 1>(buf, af, bf);
    }
  }

  // Opening of a stage: the pairs of A slot 0 walk the B slots (both row
  // blocks per B slot), so the first MFMA needs only B0 and A0's two
  // fragments; later B fragments are read two pairs ahead and the A ring for
  // blocks 2.. is filled on the way.
  static constexpr int count_a0() {
    int n = 0;
    for (int p = 0; p < NP; ++p) n += pair_info(PIPE, NHI, NLO, p).a == 0;
    return n;
  }
  static constexpr int a0_pair(int k) {  // k-th pair of A slot 0
    for (int p = 0; p < NP; ++p)
      if (pair_info(PIPE, NHI, NLO, p).a == 0 && k-- == 0) return p;
    return -1;
  }
  static constexpr int kA0 = count_a0();

  __device__ __forceinline__ uint4 read_b(const uint4* buf, int s) const {
    return buf[((NT + s) * 4 + wc) * 64 + fl];
  }

  template <int K>
  __device__ __forceinline__ void opening(const uint4* buf, uint4 (&af)[kDepth + 1],
                                          uint4 (&bf)[NT]) {
    if constexpr (K < kA0) {
      constexpr int p = a0_pair(K);
      constexpr int b = pair_info(PIPE, NHI, NLO, p).b;
      if constexpr (K + 2 < kA0) {
        constexpr int b2 = pair_info(PIPE, NHI, NLO, a0_pair(K + 2)).b;
        bf[b2] = read_b(buf, b2);
      }
      if constexpr (K == kA0 - 2) af[2] = read_a(buf, 2);
      if constexpr (K == kA0 - 1) af[3] = read_a(buf, 3);
      acc[p][0] = Op::mma(af[0], bf[b], acc[p][0]);
      if constexpr (K == kA0 - 1) af[0] = read_a(buf, 4);
      acc[p][1] = Op::mma(af[1], bf[b], acc[p][1]);
      __builtin_amdgcn_sched_barrier(0);
      opening<K + 1>(buf, af, bf);
    }
  }

  __device__ __forceinline__ void operator()(const uint4* buf) {
    static_assert(kDepth == 3, "the opening fills ring slots 2, 3, 0");
    uint4 bf[NT];
    uint4 af[kDepth + 1];
    constexpr int b0 = pair_info(PIPE, NHI, NLO, a0_pair(0)).b;
    constexpr int b1 = pair_info(PIPE, NHI, NLO, a0_pair(1)).b;
    bf[b0] = read_b(buf, b0);
    af[0] = read_a(buf, 0);
    af[1] = read_a(buf, 1);
    bf[b1] = read_b(buf, b1);
    __builtin_amdgcn_sched_barrier(0);
    opening<0>(buf, af, bf);
    pipe_step<2>(buf, af, bf);
  }
};

// vmcnt wait before consuming stage s: the loads of the `later` stages
// already issued after it (each NT instructions per wave) may stay in flight.
template <int NT>
__device__ __forceinline__ void wait_stage(int64_t later) {
  if (later >= 2) wait_vm<2 * NT>();
  else if (later == 1) wait_vm<NT>();
  else wait_vm<0>();
}

// All pairs of the schedule in one K sweep (schedules whose accumulators fit
// in registers).  PIPE/NHI/NLO fix the schedule at compile time.  ORDER < 0
// writes the per-pair FP32 products P[p][row][col] instead of C (test hook).
// `unit2` is the product scale 2^(2 rho - 48) of the I8 format.
constexpr int kOrderProducts = -1;

template <class Op, int PIPE, int NHI, int NLO, int ORDER>
__global__ __launch_bounds__(kThreads16) void gemm_allpairs(
    const char* __restrict__ As, const int32_t* __restrict__ Ae,
    const char* __restrict__ Bs, const int32_t* __restrict__ Be,
    int64_t N, int64_t M, int64_t nst, int64_t a_lines, int64_t b_lines,
    float unit2, double* __restrict__ C, int64_t ldc, float* __restrict__ P,
    int64_t ldp) {
  constexpr int NT = PIPE == OZK_PIPE_ONDEVICE ? NHI + NLO : NHI;
  constexpr int NP = pair_count(PIPE, NHI, NLO);
  constexpr int NBLK = PIPE == OZK_PIPE_ONDEVICE ? 3 : 1;
  constexpr int kBuf = (NT + NT) * 4 * 64;  // uint4 per stage buffer
  static_assert(kRing == 4, "wait_stage assumes 4 stage buffers");
  // NT = 5: 4 x 40 KiB, the whole 160 KiB LDS of a gfx950 CU.
  __shared__ uint4 lds[kRing * kBuf];

  const int ntm = (int)(a_lines / kBM), ntn = (int)(b_lines / kBN);
  int tm, tn;
  tile_coords(blockIdx.x, ntm, ntn, tm, tn);
  const int64_t row0 = (int64_t)tm * kBM, col0 = (int64_t)tn * kBN;
  const int64_t a_stage = a_lines * kChunkBytes, b_stage = b_lines * kChunkBytes;
  const int64_t aplane = a_stage * nst, bplane = b_stage * nst;
  const char* At = As + row0 * kChunkBytes;
  const char* Bt = Bs + col0 * kChunkBytes;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  AllPairsMMA<Op, PIPE, NHI, NLO, NT, NP> mma;
  mma.fl = frag_lane(lane);
  mma.wr = wave >> 2;
  mma.wc = wave & 3;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    mma.acc[p][0] = typename Op::acc_t{};
    mma.acc[p][1] = typename Op::acc_t{};
  }

  // Per stage s: wait for this wave's loads of stage s, barrier (stage s is
  // complete in LDS and every wave has finished stage s - 1, whose buffer is
  // refilled next), fetch stage s + kRing - 1, run the MFMAs of stage s.
  const uint32_t lane_bytes = 16u * (uint32_t)lane;
  const uint32_t lds0 = lds_offset(lds);
  for (int i = 0; i < kRing - 1; ++i)
    if (i < nst)
      stage_dma<NT>(At, aplane, a_stage, Bt, bplane, b_stage, i,
                    lds0 + i * kBuf * 16, wave, lane_bytes);
  for (int64_t s = 0; s < nst; ++s) {
    const int64_t later = nst - 1 - s;
    wait_stage<NT>(later < kRing - 2 ? later : kRing - 2);
    __syncthreads();
    const int64_t fetch = s + kRing - 1;
    if (fetch < nst)
      stage_dma<NT>(At, aplane, a_stage, Bt, bplane, b_stage, fetch,
                    lds0 + (uint32_t)((fetch % kRing) * kBuf * 16), wave, lane_bytes);
    mma(lds + (s % kRing) * kBuf);
  }

  // Accumulator register r of lane l of a 16x16 block holds row
  // 4 * (l / 16) + r, column l % 16.
  const int64_t col = col0 + 16 * mma.wc + (lane & 15);
  if constexpr (ORDER == kOrderProducts) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = row0 + 32 * mma.wr + 16 * h + 4 * (lane >> 4) + r;
        if (row < N && col < M) {
#pragma unroll
          for (int p = 0; p < NP; ++p)
            P[((int64_t)p * N + row) * ldp + col] = Op::product(mma.acc[p][h][r], unit2);
        }
      }
    }
  } else {
    // Fold in schedule order and store.
    int eb[NT];
#pragma unroll
    for (int s = 0; s < NT; ++s) eb[s] = Be[s * b_lines + col];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = row0 + 32 * mma.wr + 16 * h + 4 * (lane >> 4) + r;
        int ea[NT];
#pragma unroll
        for (int s = 0; s < NT; ++s) ea[s] = Ae[s * a_lines + row];
        typename FoldOf<ORDER>::type f;
        f.init();
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const PairInfo q = pair_info(PIPE, NHI, NLO, p);
          f.pair(q, Op::product(mma.acc[p][h][r], unit2), ldexpf(1.0f, eb[q.b]),
                 ldexpf(1.0f, ea[q.a]), ldexp(1.0, eb[q.b]), ldexp(1.0, ea[q.a]));
        }
        const double out = f.finish(NBLK);
        if (row < N && col < M) C[row * ldc + col] = out;
      }
    }
  }
}

struct OnePairMMA {
  floatx16 acc;
  int lane, wm, wn;
  __device__ __forceinline__ void operator()(const uint4* buf, int ks) {
    const bf16x8 bf = as_bf16x8(buf[frag_off(1, wn, ks, lane)]);
    const bf16x8 af = as_bf16x8(buf[frag_off(0, wm, ks, lane)]);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf, acc, 0, 0, 0);
  }
};

// Any schedule: one pair per K sweep, the pair's slices chosen at run time.
// MODE 0: fold with ORDER and write C; MODE 1: write the raw FP32 products
// P[p][row][col] (test hook).  The fold state of the lane's 16 elements is
// kept as one register array per field.
template <int ORDER, int MODE>
__global__ __launch_bounds__(kThreads) void gemm_pairwise(
    const uint16_t* __restrict__ As, const int32_t* __restrict__ Ae,
    const uint16_t* __restrict__ Bs, const int32_t* __restrict__ Be,
    int64_t N, int64_t M, int64_t ld, int64_t a_lines, int64_t b_lines,
    int pipe, int nhi, int nlo, double* __restrict__ C, int64_t ldc,
    float* __restrict__ P, int64_t ldp) {
  __shared__ uint4 lds[2 * 2 * 4 * 64];
  const int ntm = (int)(a_lines / kBM), ntn = (int)(b_lines / kBN);
  int tm, tn;
  tile_coords(blockIdx.x, ntm, ntn, tm, tn);
  const int64_t row0 = (int64_t)tm * kBM, col0 = (int64_t)tn * kBN;
  const int64_t aplane = a_lines * ld, bplane = b_lines * ld;
  constexpr int64_t kPer = kChunkBytes / 2;  // BF16 values per chunk
  OnePairMMA mma;
  mma.lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  mma.wm = wave >> 1;
  mma.wn = wave & 1;
  const int lane = mma.lane;
  const int64_t col = col0 + 32 * mma.wn + (lane & 31);
  const int np = pair_count(pipe, nhi, nlo);
  const int nblocks = pipe == OZK_PIPE_ONDEVICE ? 3 : 1;

  typename FoldOf<ORDER>::type f[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) f[r].init();

  for (int p = 0; p < np; ++p) {
    const PairInfo q = pair_info(pipe, nhi, nlo, p);
    const uint16_t* a_ptr[1] = {As + q.a * aplane + row0 * kPer};
    const uint16_t* b_ptr[1] = {Bs + q.b * bplane + col0 * kPer};
    mma.acc = floatx16{};
    k_sweep<1, 1>(a_ptr, b_ptr, a_lines * kPer, b_lines * kPer, ld / kPer, lds, mma);
    if (MODE == 1) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row0 + 32 * mma.wm + acc_row(r, lane);
        if (row < N && col < M) P[((int64_t)p * N + row) * ldp + col] = mma.acc[r];
      }
      continue;
    }
    const int eb = Be[q.b * b_lines + col];
    const float cs32 = ldexpf(1.0f, eb);
    const double cs64 = ldexp(1.0, eb);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = row0 + 32 * mma.wm + acc_row(r, lane);
      const int ea = Ae[q.a * a_lines + row];
      f[r].pair(q, mma.acc[r], cs32, ldexpf(1.0f, ea), cs64, ldexp(1.0, ea));
    }
  }
  if (MODE == 1) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = row0 + 32 * mma.wm + acc_row(r, lane);
    const double out = f[r].finish(nblocks);
    if (row < N && col < M) C[row * ldc + col] = out;
  }
}

// One MFMA on a pattern that encodes (row, col) in the result:
// A[i][0] = i, A[i][1] = 1, B[0][j] = 1, B[1][j] = 64 j, all other k zero,
// under the operand layout lane l -> (row l % 32, k 8 * (l / 32) + e).
// Then C[i][j] = i + 64 j identifies every accumulator register.
__global__ void probe_mfma_kernel(int32_t* out) {
  const int l = threadIdx.x;
  bf16x8 a = bf16x8{}, b = bf16x8{};
  if (l < 32) {
    a[0] = (__bf16)(float)l;
    a[1] = (__bf16)1.0f;
    b[0] = (__bf16)1.0f;
    b[1] = (__bf16)(64.0f * (float)l);
  }
  floatx16 acc = floatx16{};
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 16; ++r) out[l * 16 + r] = (int32_t)acc[r];
}

// Same probe for v_mfma_f32_16x16x32_bf16: lane l -> (row l % 16, k 8 * (l / 16)
// + e); C[i][j] = i + 64 j.  Writes 64 lanes x 4 registers to out[1024..1279].
__global__ void probe_mfma16_kernel(int32_t* out) {
  const int l = threadIdx.x;
  bf16x8 a = bf16x8{}, b = bf16x8{};
  if (l < 16) {
    a[0] = (__bf16)(float)l;
    a[1] = (__bf16)1.0f;
    b[0] = (__bf16)1.0f;
    b[1] = (__bf16)(64.0f * (float)l);
  }
  floatx4 acc = floatx4{};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 4; ++r) out[1024 + l * 4 + r] = (int32_t)acc[r];
}

// ---------------------------------------------------------------- launch

// Schedules with an all-pairs instantiation (accumulators fit in registers).
static bool allpairs_schedule(int pipe, int nhi, int nlo) {
  return pipe == OZK_PIPE_ONDEVICE && ((nhi == 4 && nlo == 1) || (nhi == 3 && nlo == 1));
}

bool allpairs_supported(int pipe, int nhi, int nlo) {
  return allpairs_schedule(pipe, nhi, nlo);
}

template <class Op, int NHI, int NLO, int ORDER>
static void launch_ap(dim3 grid, hipStream_t st, const void* As,
                      const int32_t* Ae, const void* Bs, const int32_t* Be,
                      int64_t N, int64_t M, int64_t nst, int64_t al, int64_t bl,
                      float unit2, double* C, int64_t ldc, float* P,
                      int64_t ldp) {
  hipLaunchKernelGGL((gemm_allpairs<Op, OZK_PIPE_ONDEVICE, NHI, NLO, ORDER>),
                     grid, dim3(kThreads16), 0, st, (const char*)As, Ae,
                     (const char*)Bs, Be, N, M, nst, al, bl, unit2, C, ldc, P,
                     ldp);
}

template <class Op, int NHI, int NLO>
static void launch_ap_order(int order, dim3 grid, hipStream_t st,
                            const void* As, const int32_t* Ae, const void* Bs,
                            const int32_t* Be, int64_t N, int64_t M,
                            int64_t nst, int64_t al, int64_t bl, float unit2,
                            double* C, int64_t ldc, float* P, int64_t ldp) {
  switch (order) {
    case OZK_ORDER_2SUM:
      launch_ap<Op, NHI, NLO, OZK_ORDER_2SUM>(grid, st, As, Ae, Bs, Be, N, M, nst, al, bl, unit2, C, ldc, P, ldp);
      break;
    case OZK_ORDER_BLOCK64:
      launch_ap<Op, NHI, NLO, OZK_ORDER_BLOCK64>(grid, st, As, Ae, Bs, Be, N, M, nst, al, bl, unit2, C, ldc, P, ldp);
      break;
    case OZK_ORDER_HOST_JAX:
      launch_ap<Op, NHI, NLO, OZK_ORDER_HOST_JAX>(grid, st, As, Ae, Bs, Be, N, M, nst, al, bl, unit2, C, ldc, P, ldp);
      break;
    case OZK_ORDER_HOST_NP:
      launch_ap<Op, NHI, NLO, OZK_ORDER_HOST_NP>(grid, st, As, Ae, Bs, Be, N, M, nst, al, bl, unit2, C, ldc, P, ldp);
      break;
    default:
      launch_ap<Op, NHI, NLO, kOrderProducts>(grid, st, As, Ae, Bs, Be, N, M, nst, al, bl, unit2, C, ldc, P, ldp);
      break;
  }
}

// All-pairs launch for a preset schedule; `i8` selects the INT8 plane
// format (rho >= 19).  order = kOrderProducts writes P.
static int launch_allpairs(bool i8, const void* As, const int32_t* Ae,
                           const void* Bs, const int32_t* Be, int64_t N,
                           int64_t M, int64_t K, int rho, int nhi, int nlo,
                           int order, double* C, int64_t ldc, float* P,
                           int64_t ldp, hipStream_t st) {
  // chunks per line: round_up(K, kKPad) elements of 1 or 2 bytes
  const int64_t nst = round_up(K, kKPad) * (i8 ? 1 : 2) / kChunkBytes;
  const int64_t al = round_up(N, kLinePad), bl = round_up(M, kLinePad);
  const int64_t ntiles = (al / kBM) * (bl / kBN);
  OZK_CHECK_ARG(ntiles < (1ll << 31), "problem too large for one launch");
  const dim3 grid((unsigned)ntiles);
  const float unit2 = ldexpf(1.0f, 2 * rho - 48);
#define OZK_AP_ALL(Op)                                                              \
  do {                                                                              \
    if (nhi == 4)                                                                   \
      launch_ap_order<Op, 4, 1>(order, grid, st, As, Ae, Bs, Be, N, M, nst, al, bl, \
                                unit2, C, ldc, P, ldp);                             \
    else                                                                            \
      launch_ap_order<Op, 3, 1>(order, grid, st, As, Ae, Bs, Be, N, M, nst, al, bl, \
                                unit2, C, ldc, P, ldp);                             \
  } while (0)
  if (i8) OZK_AP_ALL(OpI8);
  else OZK_AP_ALL(OpBf16);
#undef OZK_AP_ALL
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

int launch_gemm(const void* As, const int32_t* Ae, const void* Bs,
                const int32_t* Be, int64_t N, int64_t M, int64_t K, int pipe,
                int nhi, int nlo, int order, double* C, int64_t ldc,
                hipStream_t st, bool i8, int rho) {
  if (allpairs_schedule(pipe, nhi, nlo))
    return launch_allpairs(i8, As, Ae, Bs, Be, N, M, K, rho, nhi, nlo, order,
                           C, ldc, nullptr, 0, st);
  if (i8) {
    set_error("int8 slice planes need a preset on-device schedule");
    return OZK_ERR_UNSUPPORTED;
  }
  const int64_t ld = round_up(K, kKPad);
  const int64_t al = round_up(N, kLinePad), bl = round_up(M, kLinePad);
  const int64_t ntiles = (al / kBM) * (bl / kBN);
  OZK_CHECK_ARG(ntiles < (1ll << 31), "problem too large for one launch");
  const dim3 grid((unsigned)ntiles);
  const uint16_t* A16 = (const uint16_t*)As;
  const uint16_t* B16 = (const uint16_t*)Bs;
#define OZK_PW(O)                                                              \
  hipLaunchKernelGGL((gemm_pairwise<O, 0>), grid, dim3(kThreads), 0, st, A16,  \
                     Ae, B16, Be, N, M, ld, al, bl, pipe, nhi, nlo, C, ldc,    \
                     (float*)nullptr, (int64_t)0)
  switch (order) {
    case OZK_ORDER_2SUM: OZK_PW(OZK_ORDER_2SUM); break;
    case OZK_ORDER_BLOCK64: OZK_PW(OZK_ORDER_BLOCK64); break;
    case OZK_ORDER_HOST_JAX: OZK_PW(OZK_ORDER_HOST_JAX); break;
    default: OZK_PW(OZK_ORDER_HOST_NP); break;
  }
#undef OZK_PW
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

// Per-pair products.  Preset schedules run the all-pairs kernel (the one the
// drivers use); other schedules (BF16 only) the pairwise kernel.
int launch_products(const void* As, const void* Bs, int64_t N, int64_t M,
                    int64_t K, int pipe, int nhi, int nlo, float* P,
                    int64_t ldp, hipStream_t st, bool i8, int rho) {
  if (allpairs_schedule(pipe, nhi, nlo))
    return launch_allpairs(i8, As, nullptr, Bs, nullptr, N, M, K, rho, nhi, nlo,
                           kOrderProducts, nullptr, 0, P, ldp, st);
  if (i8) {
    set_error("int8 slice planes need a preset on-device schedule");
    return OZK_ERR_UNSUPPORTED;
  }
  const int64_t ld = round_up(K, kKPad);
  const int64_t al = round_up(N, kLinePad), bl = round_up(M, kLinePad);
  const int64_t ntiles = (al / kBM) * (bl / kBN);
  OZK_CHECK_ARG(ntiles < (1ll << 31), "problem too large for one launch");
  hipLaunchKernelGGL((gemm_pairwise<OZK_ORDER_2SUM, 1>), dim3((unsigned)ntiles),
                     dim3(kThreads), 0, st, (const uint16_t*)As,
                     (const int32_t*)nullptr, (const uint16_t*)Bs,
                     (const int32_t*)nullptr, N, M, ld, al, bl, pipe, nhi, nlo,
                     (double*)nullptr, (int64_t)0, P, ldp);
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

// Probe for v_mfma_i32_16x16x64_i8: bytes 0 and 1 of lane l < 16 hold
// A[l][k0] = l, A[l][k1] = 16 and B[k0][l] = 1, B[k1][l] = l, so that
// C[i][j] = i + 16 j.  Writes 64 lanes x 4 registers to out[1280..1535].
__global__ void probe_mfma_i8_kernel(int32_t* out) {
  const int l = threadIdx.x;
  int32x4 a = int32x4{}, b = int32x4{};
  if (l < 16) {
    a[0] = l | (16 << 8);
    b[0] = 1 | (l << 8);
  }
  int32x4 acc = int32x4{};
  acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 4; ++r) out[1280 + l * 4 + r] = acc[r];
}

// Probe for v_mfma_i32_32x32x32_i8: bytes 0 and 1 of lane l < 32 hold
// A[l][k0] = l, A[l][k1] = 64 and B[k0][l] = 1, B[k1][l] = l, so that
// C[i][j] = i + 64 j.  Writes 64 lanes x 16 registers to out[1536..2559].
__global__ void probe_mfma_i8_32_kernel(int32_t* out) {
  const int l = threadIdx.x;
  int32x4 a = int32x4{}, b = int32x4{};
  if (l < 32) {
    a[0] = l | (64 << 8);
    b[0] = 1 | (l << 8);
  }
  int32x16 acc = int32x16{};
  acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 16; ++r) out[1536 + l * 16 + r] = acc[r];
}

int launch_probe_mfma(int32_t* out, hipStream_t st) {
  hipLaunchKernelGGL(probe_mfma_kernel, dim3(1), dim3(64), 0, st, out);
  OZK_LAUNCH_CHECK();
  hipLaunchKernelGGL(probe_mfma16_kernel, dim3(1), dim3(64), 0, st, out);
  OZK_LAUNCH_CHECK();
  hipLaunchKernelGGL(probe_mfma_i8_kernel, dim3(1), dim3(64), 0, st, out);
  OZK_LAUNCH_CHECK();
  hipLaunchKernelGGL(probe_mfma_i8_32_kernel, dim3(1), dim3(64), 0, st, out);
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

}  // namespace ozk
