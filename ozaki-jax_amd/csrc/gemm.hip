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

#include "fold.h"

namespace ozk {

// ---------------------------------------------------------------- tiling

constexpr int kBM = 64, kBN = 64, kThreads = 256;

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

// Upper-triangle tile order for a symmetric product (tm <= tn, T x T tiles).
// As in tile_coords, each XCD gets a contiguous range of the order.  The
// order walks groups of kGroupM tile-rows; inside a group, tile-columns
// ascend, and each column's tiles of the group (tm <= tn) are adjacent.
__device__ __forceinline__ void tile_coords_sym(int bid, int T, int& tm, int& tn) {
  const int nt = T * (T + 1) / 2;
  const int q = nt / kXcds, rem = nt % kXcds;
  const int xcd = bid % kXcds, slot = bid / kXcds;
  int L = (xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q) + slot;
  int g0 = 0;
  for (;;) {
    const int gsz = min(kGroupM, T - g0);
    const int cnt = gsz * (gsz + 1) / 2 + gsz * (T - g0 - gsz);
    if (L < cnt || g0 + gsz >= T) {
      const int tri = gsz * (gsz + 1) / 2;
      if (L < tri) {  // columns g0 .. g0 + gsz - 1: 1, 2, .., gsz tiles
        int c = 0;
        while ((c + 1) * (c + 2) / 2 <= L) ++c;
        tn = g0 + c;
        tm = g0 + (L - c * (c + 1) / 2);
      } else {  // later columns: gsz tiles each
        const int o = L - tri;
        tn = g0 + gsz + o / gsz;
        tm = g0 + o % gsz;
      }
      return;
    }
    L -= cnt;
    g0 += gsz;
  }
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
// at byte 64 (r % 16), units swizzled).  Waves 0..3 fetch every fragment of
// a stage with contiguous direct global->LDS loads, kRing - 1 stages ahead of
// the MFMAs, while waves 4..7 (one on each SIMD) already run theirs.  MFMA lane l reads line l % 16, logical unit
// l / 16 of a fragment (frag_lane); the swizzle spreads those 64 reads over
// all LDS banks.

constexpr int kThreads16 = 512;
constexpr int kRing = 4;       // stage buffers (kRing - 1 stages in flight)
// Dynamic-tail words (gemm_allpairs): kXcds counters per sweep (at most
// kDynSlot0 / kXcds sweeps), then one word per workgroup (at most
// kDynMaxGrid) that passes a claimed tile on.
constexpr int kDynSlot0 = 128, kDynMaxGrid = 1024;

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

// uint4 index inside a 1 KiB fragment of the 16x16x64 operand of lane l:
// line l % 16, logical unit l / 16.
__device__ __forceinline__ int frag_lane(int lane) {
  return (lane & 15) * 4 + ((lane >> 4) ^ unit_swizzle(lane & 15));
}

// Pairs and planes of one K sweep over the blocks B0..B1 of the on-device
// schedule (0 hh, 1 hl, 2 lh; each block is a contiguous pair range).  Block
// hh uses the hi planes of A and B, hl the hi planes of A and the lo planes
// of B, lh the lo planes of A and the hi planes of B; a sweep stages exactly
// the planes its blocks use.
// Row blocks of 16 lines per wave of an all-pairs tile: a workgroup's 8
// waves hold 2 x RB blocks of rows and 4 of columns, so its tile is
// 32 RB x 64.  RB = 3 (96-row tiles) where the sweep's pairs fit three
// blocks of accumulators (at most 16 pairs) and its stage buffer (2 RB
// fragments of 1 KiB per A plane, 4 per B plane) the 40 KiB slot of the
// four-stage ring: fewer staged bytes per MFMA.  Square 64-row tiles for the
// symmetric (gram) form.  The sweeps of one schedule may differ (the fold
// state between them is kept per element, whatever the tiles).
constexpr int ap_rb_of(int np, int na, int nb, bool sym) {
  return (!sym && np <= 16 && 6 * na + 4 * nb <= 40) ? 3 : 2;
}
constexpr int ap_rb(int nhi, int nlo, int b0, int b1, bool sym) {
  const int na = (b1 == 2 ? nhi + nlo : nhi) - (b0 == 2 ? nhi : 0);
  const int bb = (b0 == 1 && b1 == 1) ? nhi : 0;
  const int nb = ((b0 <= 1 && b1 >= 1) ? nhi + nlo : nhi) - bb;
  const int p0 = b0 == 0 ? 0 : (b0 == 1 ? nhi * nhi : nhi * nhi + nhi * nlo);
  const int p1 = b1 == 0 ? nhi * nhi
                         : (b1 == 1 ? nhi * nhi + nhi * nlo : nhi * nhi + 2 * nhi * nlo);
  return ap_rb_of(p1 - p0, na, nb, sym);
}

// Besides the planes and pairs, a sweep says whether it starts the schedule
// (kFirst: no fold state to load) and ends it (kLast: C is written, not the
// state), how many blocks the schedule folds (kNBlk) and, for the 2Sum
// state, the blocks folded before and after it (kDone0, kDone1).
template <int PIPE, int NHI, int NLO, int B0, int B1, bool SYM = false>
struct Sweep {
  static_assert(PIPE == OZK_PIPE_ONDEVICE, "sweeps cover the on-device schedule");
  static constexpr bool kRect = false, kFirst = B0 == 0, kLast = B1 == 2;
  static constexpr bool kMid0 = false, kMid1 = false;
  static constexpr int kNBlk = 3, kDone0 = B0, kDone1 = B1 + 1;
  static constexpr int A0 = B0 == 2 ? NHI : 0;                    // first A plane
  static constexpr int NA = (B1 == 2 ? NHI + NLO : NHI) - A0;     // A planes
  static constexpr int BB = (B0 == 1 && B1 == 1) ? NHI : 0;       // first B plane
  static constexpr int NB = ((B0 <= 1 && B1 >= 1) ? NHI + NLO : NHI) - BB;
  static constexpr int P0 = B0 == 0 ? 0 : (B0 == 1 ? NHI * NHI : NHI * NHI + NHI * NLO);
  static constexpr int P1 = B1 == 0 ? NHI * NHI
                                    : (B1 == 1 ? NHI * NHI + NHI * NLO
                                               : NHI * NHI + 2 * NHI * NLO);
  static constexpr int NP = P1 - P0;  // pairs of the sweep
  static constexpr int S = NA + NB;   // LDS slots per stage
  static constexpr int RB = ap_rb(NHI, NLO, B0, B1, SYM);  // row blocks per wave
  static constexpr int TM = 32 * RB;                     // tile rows
  static constexpr int FA = 2 * RB;                      // fragments per A slot
  static constexpr int NFRAG = NA * FA + NB * 4;         // fragments per stage
  static constexpr PairInfo pair(int k) { return pair_info(PIPE, NHI, NLO, P0 + k); }
  static constexpr int la(int k) { return pair(k).a - A0; }  // local A slot
  static constexpr int lb(int k) { return pair(k).b - BB; }  // local B slot
  // Index of pair (b, a) for pair k = (a, b), -1 if the sweep lacks it.
  static constexpr int tpair(int k) {
    for (int i = 0; i < NP; ++i)
      if (pair(i).a == pair(k).b && pair(i).b == pair(k).a) return i;
    return -1;
  }
};

// A sweep of the host schedule (pairs (i, j), i + j <= N - 1, i-major) over
// its groups G0..G1 (A planes G0..G1): B planes 0 .. N - 1 - G0, the planes
// of the first group's pairs.  The FP64 orders fold the products of a group
// into one running sum, so the sweeps, which cut between groups, carry that
// sum alone.
template <int N, int G0, int G1>
struct Sweep<OZK_PIPE_HOST, N, 0, G0, G1, false> {
  static constexpr bool kRect = false, kFirst = G0 == 0, kLast = G1 == N - 1;
  static constexpr bool kMid0 = false, kMid1 = false;
  static constexpr int kNBlk = 1, kDone0 = 0, kDone1 = 0;
  static constexpr int A0 = G0, NA = G1 - G0 + 1, BB = 0, NB = N - G0;
  static constexpr int P0 = G0 * N - G0 * (G0 - 1) / 2;
  static constexpr int P1 = (G1 + 1) * N - G1 * (G1 + 1) / 2;
  static constexpr int NP = P1 - P0;
  static constexpr int S = NA + NB;
  static constexpr int RB = ap_rb_of(NP, NA, NB, false);
  static constexpr int TM = 32 * RB;
  static constexpr int FA = 2 * RB;
  static constexpr int NFRAG = NA * FA + NB * 4;
  static constexpr PairInfo pair(int k) { return pair_info(OZK_PIPE_HOST, N, 0, P0 + k); }
  static constexpr int la(int k) { return pair(k).a - A0; }
  static constexpr int lb(int k) { return pair(k).b - BB; }
  static constexpr int tpair(int) { return -1; }
};

// Last group of the host sweep that starts at group g0: as many groups as
// keep the sweep within 10 planes and 25 pairs.
constexpr int host_sweep_end(int n, int g0) {
  int g1 = g0;
  while (g1 + 1 < n && (g1 + 2 - g0) + (n - g0) <= 10 &&
         ((g1 + 2) * n - (g1 + 1) * (g1 + 2) / 2) - (g0 * n - g0 * (g0 - 1) / 2) <= 25)
    ++g1;
  return g1;
}
constexpr int host_nsweeps(int n) {
  int k = 0;
  for (int g = 0; g < n; g = host_sweep_end(n, g) + 1) ++k;
  return k;
}

// Rectangle sweeps: the on-device schedules beyond the fixed ones (a count
// of 6 to 8) run as sweeps over rectangles of one block: NA consecutive
// groups of the block (A planes) times all NB B planes of its pairs, the
// NA x NB pairs i-major, as the block orders them.  The kernel is the same
// for every schedule and block with that shape: the host offsets the plane,
// exponent and line-sum pointers to the rectangle's first A and B plane,
// and the fold's block id, block-boundary flags and state boundaries come
// in a run-time word (kRf*).  Sweep<kPipeRect, NA, NB, 0, 0>.
constexpr int kPipeRect = 16;
constexpr int kRfBlk = 3;           // bits 0-1: block id
constexpr int kRfGFirst = 1 << 2;   // the rectangle starts its block
constexpr int kRfGLast = 1 << 3;    // ... and ends it
constexpr int kRfFirst = 1 << 4;    // starts the schedule: no state to load
constexpr int kRfLast = 1 << 5;     // ends it: C is written
constexpr int kRfPair = 1 << 6;     // 2Sum order: write the (hi, lo) pair
constexpr int kRfDone0 = 7;         // bits 7-8: blocks folded before it
constexpr int kRfDone1 = 9;         // bits 9-10: ... and after it

template <int NA_, int NB_>
struct Sweep<kPipeRect, NA_, NB_, 0, 0, false> {
  static constexpr bool kRect = true, kFirst = false, kLast = false;
  static constexpr bool kMid0 = false, kMid1 = false;
  static constexpr int kNBlk = 3, kDone0 = 0, kDone1 = 0;
  static constexpr int A0 = 0, NA = NA_, BB = 0, NB = NB_, P0 = 0;
  static constexpr int NP = NA * NB;
  static constexpr int S = NA + NB;
  static constexpr int RB = ap_rb_of(NP, NA, NB, false);
  static constexpr int TM = 32 * RB;
  static constexpr int FA = 2 * RB;
  static constexpr int NFRAG = NA * FA + NB * 4;
  // fg and be hold inside the rectangle; the run-time word says whether the
  // rectangle's first group and last pair are also its block's
  static constexpr PairInfo pair(int k) {
    return PairInfo{k / NB, k % NB, 0, k % NB == 0, k % NB == NB - 1, k == 0, k == NP - 1,
                    k / NB == 0};
  }
  static constexpr int la(int k) { return k / NB; }
  static constexpr int lb(int k) { return k % NB; }
  static constexpr int tpair(int) { return -1; }
};

// Most planes (A + B) and pairs of one sweep: the 160 KiB ring holds 10
// planes' fragments per stage, the registers 25 pairs' accumulators.
constexpr int kSweepPlanes = 10, kSweepPairs = 25;

template <class Op, class SW>
struct AllPairsMMA {
  static constexpr int NA = SW::NA, NB = SW::NB, NP = SW::NP, RB = SW::RB;
  typename Op::acc_t acc[NP][RB];
  int fl, wr, wc;  // fl = frag_lane(lane)

  // MFMAs of one (A slot, row block) for every pair of that A slot.
  template <int SA, int H>
  __device__ __forceinline__ void block(uint4 af, const uint4 (&bf)[NB]) {
#pragma unroll
    for (int k = 0; k < NP; ++k)
      if (SW::la(k) == SA) acc[k][H] = Op::mma(af, bf[SW::lb(k)], acc[k][H]);
  }

  // The RB NA blocks of a stage (A slot j / RB, row block j % RB), A
  // fragments software-pipelined through kDepth + 1 = RB + 2 registers: the
  // read of block j + kDepth is issued before the MFMAs of block j.
  // Scheduling barriers keep the reads where they are.
  static constexpr int kBlocks = NA * RB, kDepth = RB + 1;

  __device__ __forceinline__ uint4 read_a(const uint4* buf, int j) const {
    return buf[((j / RB) * SW::FA + RB * wr + (j % RB)) * 64 + fl];
  }
  __device__ __forceinline__ uint4 read_b(const uint4* buf, int s) const {
    return buf[(NA * SW::FA + s * 4 + wc) * 64 + fl];
  }

  template <int J>
  __device__ __forceinline__ void pipe_step(const uint4* buf,
                                            uint4 (&af)[kDepth + 1],
                                            const uint4 (&bf)[NB]) {
    if constexpr (J < kBlocks) {
      if constexpr (J + kDepth < kBlocks)
        af[(J + kDepth) % (kDepth + 1)] = read_a(buf, J + kDepth);
      block<J / RB, J % RB>(af[J % (kDepth + 1)], bf);
      __builtin_amdgcn_sched_barrier(0);
      pipe_step<J + 1>(buf, af, bf);
    }
  }

  // Opening of a stage: the pairs of A slot 0 walk the B slots (all RB row
  // blocks per B slot), so the first MFMA needs only one B and A slot 0's RB
  // fragments; later B fragments are read two pairs ahead and the A ring for
  // blocks RB .. 2 RB is filled on the way (blocks RB + 2 .. into the
  // registers of blocks 0 .. as the last pair leaves them).
  static constexpr int count_a0() {
    int n = 0;
    for (int k = 0; k < NP; ++k) n += SW::la(k) == 0;
    return n;
  }
  static constexpr int a0_pair(int i) {  // i-th pair of A slot 0
    for (int k = 0; k < NP; ++k)
      if (SW::la(k) == 0 && i-- == 0) return k;
    return -1;
  }
  static constexpr int kA0 = count_a0();
  // the B fragments are read by the pairs of A slot 0
  static_assert(kA0 == NB, "A slot 0 pairs with every B slot");

  template <int K>
  __device__ __forceinline__ void opening(const uint4* buf, uint4 (&af)[kDepth + 1],
                                          uint4 (&bf)[NB]) {
    if constexpr (K < kA0) {
      constexpr int k = a0_pair(K);
      constexpr int b = SW::lb(k);
      if constexpr (K + 2 < kA0) {
        constexpr int b2 = SW::lb(a0_pair(K + 2));
        bf[b2] = read_b(buf, b2);
      }
      // blocks RB and RB + 1 of the ring (both in the first pair when A
      // slot 0 has only one; none past the stage's last block)
      if constexpr (K == (kA0 >= 2 ? kA0 - 2 : 0) && RB < kBlocks) af[RB] = read_a(buf, RB);
      if constexpr (K == kA0 - 1 && RB + 1 < kBlocks) af[RB + 1] = read_a(buf, RB + 1);
#pragma unroll
      for (int h = 0; h < RB; ++h) {
        acc[k][h] = Op::mma(af[h], bf[b], acc[k][h]);
        if (K == kA0 - 1 && h + 1 < RB && RB + 2 + h < kBlocks) af[h] = read_a(buf, RB + 2 + h);
      }
      __builtin_amdgcn_sched_barrier(0);
      opening<K + 1>(buf, af, bf);
    }
  }

  __device__ __forceinline__ void operator()(const uint4* buf) {
    uint4 bf[NB];
    uint4 af[kDepth + 1];
    constexpr int b0 = SW::lb(a0_pair(0));
    bf[b0] = read_b(buf, b0);
#pragma unroll
    for (int h = 0; h < RB; ++h) af[h] = read_a(buf, h);
    if constexpr (kA0 >= 2) {
      constexpr int b1 = SW::lb(a0_pair(1));
      bf[b1] = read_b(buf, b1);
    }
    __builtin_amdgcn_sched_barrier(0);
    opening<0>(buf, af, bf);
    pipe_step<RB>(buf, af, bf);
  }
};

// Fetch stage `st` (chunk st of every line of the tile) into the LDS buffer
// at byte offset `buf_lds`.  Waves 0..3 move the whole stage: wave w moves
// line groups w and w + 4 (16 lines, a contiguous 1 KiB of the slot's
// plane) of every A slot, of FA groups, into its fragments FA slot + group,
// and line group w of every B slot into fragment NA FA + 4 slot + w.
// Waves 4..7 move nothing, so on every SIMD one wave issues MFMAs while the
// other waits on the texture addresser, which takes a stage's 40 loads one
// by one.  At, Bt point at the tile's first line of the sweep's first A / B
// plane in chunk 0; chunk st lies st * a_stage / st * b_stage bytes
// further.  A tile of 96 rows at the end of the lines has `agroups` < FA
// groups inside the planes: its later groups read the last of them again
// (their rows are never stored), so all addresses lie inside the
// zero-padded slice planes.
template <int NA, int NB, int FA>
__device__ __forceinline__ void stage_dma(const char* At, int64_t aplane,
                                          int64_t a_stage, const char* Bt,
                                          int64_t bplane, int64_t b_stage,
                                          int64_t st, uint32_t buf_lds,
                                          int wave, uint32_t lane_bytes, int agroups) {
  const int64_t qa = st * a_stage, qb = st * b_stage + (int64_t)wave * 1024;
#pragma unroll
  for (int slot = 0; slot < NA; ++slot) {
#pragma unroll
    for (int gg = 0; gg < (FA + 3) / 4; ++gg) {
      const int g = wave + 4 * gg;
      if (gg == 0 || g < FA) {  // uniform
        const int gs = g < agroups ? g : agroups - 1;
        dma16(__builtin_amdgcn_readfirstlane(buf_lds + (FA * slot + g) * 1024),
              (const void*)(At + slot * aplane + qa + (int64_t)gs * 1024), lane_bytes);
      }
    }
  }
#pragma unroll
  for (int slot = 0; slot < NB; ++slot)
    dma16(__builtin_amdgcn_readfirstlane(buf_lds + (NA * FA + 4 * slot + wave) * 1024),
          (const void*)(Bt + slot * bplane + qb), lane_bytes);
}

// Loads a DMA wave issues per stage: one per B slot and one or two per A
// slot (waves 0 .. FA - 5 take two A groups).
template <int NA, int NB, int FA>
__host__ __device__ constexpr int stage_loads(int wave) {
  return NB + NA * (wave + 4 < FA ? 2 : 1);
}

// vmcnt wait before consuming a stage: the loads of the `later` stages
// already issued after it (PER instructions per wave each) may stay in
// flight.
template <int PER>
__device__ __forceinline__ void wait_stage(int64_t later) {
  if (later >= 2) wait_vm<2 * PER>();
  else if (later == 1) wait_vm<PER>();
  else wait_vm<0>();
}

// Fold state at a block boundary, kept in a workspace between the sweeps of
// one product: 2Sum order (ct, cl, p0, p1, p2) as FP32 fields, the FP64
// block order the running sum c.  Field f of element (row, col) lies at
// state[f * N * M + row * M + col].  `done` = the blocks folded before the
// boundary: block lo parts p_done.. are still zero there, so they are
// neither stored nor loaded.
// MID: the boundary lies inside a block, between two of its groups; the
// 2Sum order then also carries the block's running sum (bt, bl).  The FP64
// orders' running sum covers every group folded so far either way.  `done`
// and `mid` are compile-time constants for the sweeps of the fixed
// schedules and run-time values for the rectangle sweeps.
template <int ORDER> struct FoldState {  // the FP64 orders: the running sum
  static constexpr int kBytes = 8, kBytesMid = 8;
  static __device__ __forceinline__ void load(Fold64<ORDER>& f, const char* st, int64_t e,
                                              int64_t, int, bool) {
    f.c = ((const double*)st)[e];
  }
  static __device__ __forceinline__ void store(const Fold64<ORDER>& f, char* st, int64_t e,
                                               int64_t, int, bool) {
    ((double*)st)[e] = f.c;
  }
};

template <> struct FoldState<OZK_ORDER_2SUM> {
  static constexpr int kBytes = 5 * 4, kBytesMid = 7 * 4;
  static __device__ __forceinline__ void load(Fold2Sum& f, const char* st, int64_t e,
                                              int64_t nm, int done, bool mid) {
    const float* s = (const float*)st;
    f.ct = s[e];
    f.cl = s[nm + e];
    if (done > 0) f.p0 = s[2 * nm + e];
    if (done > 1) f.p1 = s[3 * nm + e];
    if (done > 2) f.p2 = s[4 * nm + e];
    if (mid) {
      f.bt = s[5 * nm + e];
      f.bl = s[6 * nm + e];
    }
  }
  static __device__ __forceinline__ void store(const Fold2Sum& f, char* st, int64_t e,
                                               int64_t nm, int done, bool mid) {
    float* s = (float*)st;
    s[e] = f.ct;
    s[nm + e] = f.cl;
    if (done > 0) s[2 * nm + e] = f.p0;
    if (done > 1) s[3 * nm + e] = f.p1;
    if (done > 2) s[4 * nm + e] = f.p2;
    if (mid) {
      s[5 * nm + e] = f.bt;
      s[6 * nm + e] = f.bl;
    }
  }
};

constexpr int kOrderProducts = -1;
// ORDER value of the 2Sum order written as its double-float pair (C_hi,
// C_lo) (pallas_gemm_accum.py:181-186) instead of their FP64 sum: C_hi goes
// to P and C_lo to C, which then points at FP32 values; both use ldp.
constexpr int kOrderPair = -2;
template <> struct FoldOf<kOrderPair> { typedef Fold2Sum type; };
template <> struct FoldState<kOrderPair> : FoldState<OZK_ORDER_2SUM> {};

// INT8 planes store each grid count q with the offset o = 2^(25 - rho) - 1
// (q + o in [-1, 2^(26 - rho) - 1]: mostly non-negative operands, which the
// matrix cores multiply at a lower power, so a higher clock), and every
// plane line comes with its sum of q.  The exact sum of a pair's products
// is then
//   S = sum_k (qa + o)(qb + o) - o (sum_k qa + sum_k qb) - Kp o^2
// over the Kp padded positions (padding holds q = 0).  Under the rho rule
// every term is an integer below 2^31 in magnitude; the arithmetic is done
// modulo 2^32 (as the matrix cores add), which gives S exactly whenever S
// itself fits.  as / bs: sums per (plane, line), plane stride a_lines /
// b_lines; kpo2 = Kp o^2 modulo 2^32.
struct I8Fix {
  const int32_t* as;
  const int32_t* bs;
  uint32_t off, kpo2;
};

// Minus the INT8 offset's part (I8Fix) of a pair's sum at the lane's 4 rows
// (line sums sa) and its column (sb): the accumulator value a whole tile
// starts from.
__device__ __forceinline__ int32x4 i8_start(const I8Fix& fix, int32x4 sa, int sb) {
  const uint32_t c = fix.off * (uint32_t)sb + fix.kpo2;
  int32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (int32_t)(0u - (fix.off * (uint32_t)sa[i] + c));
  return r;
}

// Fold and store one output tile (tm, tn) from one wave's accumulators:
// wave (wr, wc) owns rows 16 RB wr .. + 16 RB - 1 and columns 16 wc .. +15
// of the tile as RB 16x16 blocks h.  Shared by the all-pairs kernel and the
// fixup of its K-split tail tiles.

template <class Op, class SW, int ORDER, int B0, int B1, bool SYM>
__device__ __forceinline__ void tile_epilogue(
    const typename Op::acc_t (&acc)[SW::NP][SW::RB], int tm, int tn, int wr, int wc,
    int lane, const int32_t* __restrict__ Ae, const int32_t* __restrict__ Be,
    int64_t N, int64_t M, int64_t a_lines, int64_t b_lines, float unit2,
    double* __restrict__ C, int64_t ldc, float* __restrict__ P, int64_t ldp,
    char* __restrict__ state, int rflags) {
  constexpr int NA = SW::NA, NB = SW::NB, NP = SW::NP, RB = SW::RB;
  constexpr int NBLK = SW::kNBlk;
  // where the sweep lies in its schedule: compile-time for the fixed
  // schedules, the run-time word (kRf*) for a rectangle
  const bool first = SW::kRect ? (rflags & kRfFirst) != 0 : SW::kFirst;
  const bool last = SW::kRect ? (rflags & kRfLast) != 0 : SW::kLast;
  const int done0 = SW::kRect ? (rflags >> kRfDone0) & 3 : SW::kDone0;
  const int done1 = SW::kRect ? (rflags >> kRfDone1) & 3 : SW::kDone1;
  const bool mid0 = SW::kRect ? (rflags & kRfGFirst) == 0 : SW::kMid0;
  const bool mid1 = SW::kRect ? (rflags & kRfGLast) == 0 : SW::kMid1;
  const int64_t row0 = (int64_t)tm * SW::TM, col0 = (int64_t)tn * kBN;

  // Accumulator register r of lane l of a 16x16 block holds row
  // 4 * (l / 16) + r, column l % 16.
  const int64_t col = col0 + 16 * wc + (lane & 15);
  if constexpr (ORDER == kOrderProducts) {
#pragma unroll
    for (int h = 0; h < RB; ++h) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = row0 + 16 * RB * wr + 16 * h + 4 * (lane >> 4) + r;
        if (row < N && col < M) {
#pragma unroll
          for (int k = 0; k < NP; ++k)
            P[((int64_t)(SW::P0 + k) * N + row) * ldp + col] =
                Op::product(acc[k][h][r], unit2);
        }
      }
    }
  } else {
    // Fold in schedule order; carry the state to the next sweep or store C.
    // The exponents of the lane's column, and per 16-row block those of its
    // 4 consecutive rows (one 16-byte load per A plane), are loaded
    // together, so the epilogue waits for memory twice.  Rows and columns
    // up to the padded line counts lie inside Ae / Be; the blocks of a
    // 96-row tile past them read the last 4 rows again (never stored).
    const int64_t rbase = row0 + 16 * RB * wr + 4 * (lane >> 4);
    int eb[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) eb[q] = Be[(SW::BB + q) * b_lines + col];
    const int64_t nm = N * M;
#pragma unroll
    for (int h = 0; h < RB; ++h) {
      int32x4 ea4[NA];
      const int64_t rh = rbase + 16 * h < a_lines ? rbase + 16 * h : a_lines - 4;
#pragma unroll
      for (int q = 0; q < NA; ++q)
        ea4[q] = *(const int32x4*)(Ae + (SW::A0 + q) * a_lines + rh);
      // A sweep that continues the schedule loads the fold state of the
      // block's 4 rows here too.
      typename FoldOf<ORDER>::type fr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        fr[r].init();
        if (!first) {
          const int64_t row = rbase + 16 * h + r;
          if (row < N && col < M)
            FoldState<ORDER>::load(fr[r], state, row * M + col, nm, done0, mid0);
        }
      }
      // One wait for all of them here: the folds below sit in branches on
      // `live`, and a wait placed inside them would also wait for the
      // previous row's store.  (s_waitcnt vmcnt(0), other counters free.)
      __builtin_amdgcn_s_waitcnt(0x0f70);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = rbase + 16 * h + r;
        const bool live = row < N && col < M;
        int ea[NA];
#pragma unroll
        for (int q = 0; q < NA; ++q) ea[q] = ea4[q][r];
        typename FoldOf<ORDER>::type& f = fr[r];
#pragma unroll
        for (int k = 0; k < NP; ++k) {
          PairInfo q = SW::pair(k);
          if constexpr (SW::kRect) {
            q.blk = rflags & kRfBlk;
            q.fg = q.fg && (rflags & kRfGFirst);
            q.be = q.be && (rflags & kRfGLast);
          }
          const int ia = ea[SW::la(k)], ib = eb[SW::lb(k)];
          f.pair(q, Op::product(acc[k][h][r], unit2), scale32(ib), scale32(ia),
                 scale64(ib), scale64(ia));
        }
        if constexpr (SYM) {
          // Element (col, row) of a gram matrix: its pair (a, b) product is
          // this lane's pair (b, a) product, its row-side exponents are the
          // column's and vice versa.  Fold it in schedule order too, then
          // store (C[i][j] + C[j][i]) * 0.5 at both places (gram.py:37).
          typename FoldOf<ORDER>::type f2;
          f2.init();
#pragma unroll
          for (int k = 0; k < NP; ++k) {
            const PairInfo q = SW::pair(k);
            const int ia = eb[SW::la(k)], ib = ea[SW::lb(k)];
            f2.pair(q, Op::product(acc[SW::tpair(k)][h][r], unit2), scale32(ib),
                    scale32(ia), scale64(ib), scale64(ia));
          }
          const double c1 = f.finish(NBLK), c2 = f2.finish(NBLK);
          const double out = (c1 + c2) * 0.5;
          if (live) {
            C[row * ldc + col] = out;
            if (tm != tn) C[col * ldc + row] = out;
          }
        } else if (!last) {
          if (live) FoldState<ORDER>::store(f, state, row * M + col, nm, done1, mid1);
        } else if (ORDER == kOrderPair ||
                   (ORDER == OZK_ORDER_2SUM && SW::kRect && (rflags & kRfPair))) {
          if constexpr (std::is_same<typename FoldOf<ORDER>::type, Fold2Sum>::value) {
            float hi, lo;
            f.finish_pair(NBLK, hi, lo);
            if (live) {
              P[row * ldp + col] = hi;
              ((float*)C)[row * ldp + col] = lo;
            }
          }
        } else {
          const double out = f.finish(NBLK);
          if (live) C[row * ldc + col] = out;
        }
      }
    }
  }
}

// One K sweep over blocks B0..B1 of the on-device schedule, every pair of
// those blocks accumulated in registers.  ORDER < 0 writes the per-pair FP32
// products P[p][row][col] instead (test hook).  A sweep that does not start
// the schedule reloads the fold state from `state`; one that does not end it
// stores the state there instead of writing C.  `nst` = chunks per line;
// `unit2` is the product scale 2^(2 rho - 48) of the I8 format.
//
// The grid is persistent (one workgroup per CU, gridDim.x <= tiles):
// workgroup b owns tiles b, b + gridDim.x, ... and runs their stages as one
// sequence through the LDS ring, so the loads of a tile's first stages are
// issued during the previous tile's last stages and epilogue.

template <class Op, int PIPE, int NHI, int NLO, int ORDER, int B0, int B1, bool SYM>
__global__ __launch_bounds__(kThreads16) void gemm_allpairs(
    const char* __restrict__ As, const int32_t* __restrict__ Ae,
    const char* __restrict__ Bs, const int32_t* __restrict__ Be,
    int64_t N, int64_t M, int64_t nst, int64_t a_lines, int64_t b_lines,
    float unit2, double* __restrict__ C, int64_t ldc, float* __restrict__ P,
    int64_t ldp, char* __restrict__ state, int tail_P, uint32_t* __restrict__ part,
    I8Fix fix, uint32_t* __restrict__ dyn, int dyn_nstat, int rflags) {
  typedef Sweep<PIPE, NHI, NLO, B0, B1, SYM> SW;
  constexpr int NA = SW::NA, NB = SW::NB, NP = SW::NP, RB = SW::RB, FA = SW::FA;
  constexpr int kBuf = SW::NFRAG * 64;  // uint4 per stage buffer
  static_assert(kRing == 4, "wait_stage assumes 4 stage buffers");
  static_assert(SW::NFRAG <= 40, "a stage holds at most 40 fragments (160 KiB ring)");
  // 40 fragments: 4 x 40 KiB, the whole 160 KiB LDS of a gfx950 CU.
  __shared__ uint4 lds[kRing * kBuf];

  const int ntm = (int)((a_lines + SW::TM - 1) / SW::TM), ntn = (int)(b_lines / kBN);
  const int bid = (int)blockIdx.x, nwg = (int)gridDim.x;
  // SYM: B's planes are A's (a gram matrix); only tiles tm <= tn are run
  // and each element folds both C[i][j] and C[j][i] (see the epilogue).
  static_assert(!SYM || (B0 == 0 && B1 == 2 && ORDER == OZK_ORDER_2SUM),
                "symmetric products need the single-sweep schedule");
  const int ntiles = SYM ? ntm * (ntm + 1) / 2 : ntm * ntn;
  auto coords = [&](int t, int& tm, int& tn) {
    if constexpr (SYM) tile_coords_sym(t, ntm, tm, tn);
    else tile_coords(t, ntm, ntn, tm, tn);
  };
  // Work items of this workgroup: whole tiles bid + j nwg, j < nstat.  With
  // tail_P > 1 (K-split tail) every workgroup runs the ntiles / nwg whole
  // rounds, and the ntiles % nwg tail tiles are split along K into tail_P
  // pieces of about nst / tail_P stages: workgroup bid < tail tiles * tail_P
  // runs piece bid % tail_P of tail tile bid / tail_P and stores its raw
  // sums in part (block bid) for gemm_tail_fixup.
  //
  // With dyn (dynamic tail, never together with tail_P) every workgroup runs
  // dyn_nstat whole rounds in the static order, and the tiles after them
  // are handed out at run time, so that workgroups on faster XCDs take more
  // of them: tile nstat nwg + d, d = x mod 8, comes from XCD x's counter
  // dyn[x] (d = 8 dyn[x]++ + x, which the static order would also have put
  // on XCD x), and a workgroup whose own counter is spent takes from the
  // other XCDs'.  Item j + 1 is claimed when item j starts, so the stage
  // ring's prefetch across the tile boundary is kept.  The LDS is all ring,
  // so the claimed tile reaches the other waves through the workgroup's
  // word dyn[kDynSlot0 + bid].
  const int nstat = dyn ? dyn_nstat : (tail_P ? ntiles / nwg : (ntiles - 1 - bid) / nwg + 1);
  const int ndyn = dyn ? ntiles - nstat * nwg : 0;  // dynamic tiles
  const bool has_piece = tail_P > 0 && bid < (ntiles % nwg) * tail_P;
  const int piece_tile = has_piece ? nstat * nwg + bid / tail_P : 0;
  const int64_t ps0 = has_piece ? (int64_t)(bid % tail_P) * nst / tail_P : 0;
  const int64_t ps1 = has_piece ? (int64_t)(bid % tail_P + 1) * nst / tail_P : 0;
  int nwhole = nstat;  // whole-tile items known so far (grows with claims)
  int nitems = nstat + (has_piece ? 1 : 0);
  int64_t total = (int64_t)nstat * nst + (ps1 - ps0);  // stages of this workgroup
  int dt0 = 0, dt1 = 0;  // claimed tiles of the even / odd dynamic items
  bool more = dyn != nullptr;
  auto item_tile = [&](int jj) {
    return jj < nstat ? bid + jj * nwg : (jj < nwhole ? ((jj & 1) ? dt1 : dt0) : piece_tile);
  };
  const int64_t a_stage = a_lines * kChunkBytes, b_stage = b_lines * kChunkBytes;
  const int64_t aplane = a_stage * nst, bplane = b_stage * nst;
  const char* Ab = As + SW::A0 * aplane;
  const char* Bb = Bs + SW::BB * bplane;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool dma_wave = wave < 4;
  AllPairsMMA<Op, SW> mma;
  mma.fl = frag_lane(lane);
  mma.wr = wave >> 2;
  mma.wc = wave & 3;
  // Accumulators of work item jj: zero, or on INT8 planes for a whole tile
  // minus the offset's part (I8Fix); a K-split piece stores raw sums and
  // its fixup removes that part once.
  auto start_item = [&](int jj) {
    // claim item jj + 1 (one workgroup-wide wait on the counter, per item)
    if (more && jj < nwhole && jj + 1 >= nstat) {
      if (threadIdx.x == 256) {  // a wave that issues no stage loads
        int t = -1;
        for (int i = 0; i < kXcds; ++i) {
          const int y = (bid + i) & (kXcds - 1);
          const int d = kXcds * (int)__hip_atomic_fetch_add(dyn + y, 1u, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT) + y;
          if (d < ndyn) {
            t = nstat * nwg + d;
            break;
          }
        }
        __hip_atomic_store(dyn + kDynSlot0 + bid, (uint32_t)t, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      const int t = __builtin_amdgcn_readfirstlane((int)__hip_atomic_load(
          dyn + kDynSlot0 + bid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      if (t >= 0) {
        if ((jj + 1) & 1) dt1 = t;
        else dt0 = t;
        ++nwhole;
        ++nitems;
        total += nst;
      } else {
        more = false;
      }
    }
    if constexpr (std::is_same<Op, OpI8>::value) {
      if (jj < nwhole) {
        int tm, tn;
        coords(item_tile(jj), tm, tn);
        const int64_t col = (int64_t)tn * kBN + 16 * mma.wc + (lane & 15);
        const int64_t rb = (int64_t)tm * SW::TM + 16 * RB * mma.wr + 4 * (lane >> 4);
        // per plane once: o sb + Kp o^2 and -o sa (modulo 2^32, as i8_start)
        uint32_t tb[NB];
#pragma unroll
        for (int q = 0; q < NB; ++q)
          tb[q] = fix.off * (uint32_t)fix.bs[(SW::BB + q) * b_lines + col] + fix.kpo2;
#pragma unroll
        for (int h = 0; h < RB; ++h) {
          uint32_t na[NA][4];
          // rows past the lines (a 96-row tile's last blocks) read the last 4
          const int64_t rh = rb + 16 * h < a_lines ? rb + 16 * h : a_lines - 4;
#pragma unroll
          for (int q = 0; q < NA; ++q) {
            const int32x4 sa = *(const int32x4*)(fix.as + (SW::A0 + q) * a_lines + rh);
#pragma unroll
            for (int i = 0; i < 4; ++i) na[q][i] = 0u - fix.off * (uint32_t)sa[i];
          }
#pragma unroll
          for (int k = 0; k < NP; ++k) {
            int32x4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = (int32_t)(na[SW::la(k)][i] - tb[SW::lb(k)]);
            mma.acc[k][h] = v;
          }
        }
        return;
      }
    }
#pragma unroll
    for (int k = 0; k < NP; ++k) {
#pragma unroll
      for (int h = 0; h < RB; ++h) mma.acc[k][h] = typename Op::acc_t{};
    }
  };
  start_item(0);

  // Load cursor: chunk fs of this workgroup's tile fj, whose first lines
  // are fA / fB.
  const uint32_t lane_bytes = 16u * (uint32_t)lane;
  const uint32_t lds0 = lds_offset(lds);
  int fj = 0;
  int64_t fs = 0, fe = 0;
  const char *fA = Ab, *fB = Bb;
  int fg = FA;  // line groups of the fetched tile inside the A planes
  auto load_tile = [&](int j) {
    int tm, tn;
    coords(item_tile(j), tm, tn);
    fA = Ab + (int64_t)tm * SW::TM * kChunkBytes;
    fB = Bb + (int64_t)tn * kBN * kChunkBytes;
    const int64_t left = (a_lines - (int64_t)tm * SW::TM) / 16;
    fg = left < FA ? (int)left : FA;
    fs = j < nwhole ? 0 : ps0;
    fe = j < nwhole ? nst : ps1;
  };
  // issue stage g of the sequence into ring buffer g % kRing
  auto fetch = [&](int64_t g) {
    if (dma_wave)
      stage_dma<NA, NB, FA>(fA, aplane, a_stage, fB, bplane, b_stage, fs,
                            lds0 + (uint32_t)((g & (kRing - 1)) * kBuf * 16), wave,
                            lane_bytes, fg);
    if (++fs == fe) {
      if (++fj < nitems) load_tile(fj);
    }
  };
  if (nitems > 0) load_tile(0);
  for (int64_t g = 0; g < kRing - 1 && g < total; ++g) fetch(g);

  // Per stage g: wait for this wave's loads of stage g, barrier (stage g is
  // complete in LDS and every wave has finished stage g - 1, whose buffer is
  // refilled next), fetch stage g + kRing - 1, run the MFMAs of stage g;
  // after a tile's last stage fold and store it (a tail piece: store its raw
  // sums).
  int j = 0;  // work item of the MFMA cursor
  int64_t s = 0;
  for (int64_t g = 0; g < total; ++g) {
    const int64_t later = total - 1 - g < kRing - 2 ? total - 1 - g : kRing - 2;
    if (dma_wave) {
      if (wave + 4 < FA) wait_stage<stage_loads<NA, NB, FA>(0)>(later);
      else wait_stage<stage_loads<NA, NB, FA>(3)>(later);
    }
    __syncthreads();
    if (g + kRing - 1 < total) fetch(g + kRing - 1);
    mma(lds + (g & (kRing - 1)) * kBuf);
    if (++s < (j < nwhole ? nst : ps1 - ps0)) continue;
    s = 0;
    if (j < nwhole) {
      int tm, tn;
      coords(item_tile(j), tm, tn);
      tile_epilogue<Op, SW, ORDER, B0, B1, SYM>(mma.acc, tm, tn, mma.wr, mma.wc, lane, Ae,
                                                Be, N, M, a_lines, b_lines, unit2, C, ldc,
                                                P, ldp, state, rflags);
    } else {
      // part[bid][thread][k][h]: each thread's sums are contiguous, so the
      // 16-byte stores take immediate offsets
      typename Op::acc_t* dst =
          (typename Op::acc_t*)part + ((int64_t)bid * kThreads16 + threadIdx.x) * NP * RB;
#pragma unroll
      for (int k = 0; k < NP; ++k) {
#pragma unroll
        for (int h = 0; h < RB; ++h) dst[RB * k + h] = mma.acc[k][h];
      }
    }
    ++j;
    start_item(j);
  }
}

// Tail tiles split along K: sums the tail_P pieces' raw sums (exact: integer
// sums, or FP32 sums below 2^24 grid units) and folds the tile like the
// all-pairs kernel.  One workgroup per (tail tile, wave of the all-pairs
// workgroup): blockIdx.x = 8 * tail tile + wave slot.  Each of its 8 waves
// adds up a sixth-or-so of the lane's 2 NP accumulator vectors over all
// pieces (several pieces' loads in flight), leaves the sums in LDS, and
// wave 0 folds them.  Tail tile t is tile tile0 + t of the all-pairs order.
template <class Op, int PIPE, int NHI, int NLO, int ORDER, int B0, int B1, bool SYM>
__global__ __launch_bounds__(kThreads16) void gemm_tail_fixup(
    const uint32_t* __restrict__ part, int tail_P, int tile0,
    const int32_t* __restrict__ Ae, const int32_t* __restrict__ Be, int64_t N,
    int64_t M, int64_t a_lines, int64_t b_lines, float unit2, double* __restrict__ C,
    int64_t ldc, float* __restrict__ P, int64_t ldp, char* __restrict__ state, I8Fix fix) {
  typedef Sweep<PIPE, NHI, NLO, B0, B1, SYM> SW;
  typedef typename Op::acc_t V;
  constexpr int NP = SW::NP, RB = SW::RB, NV = RB * NP;  // accumulator vectors per lane
  constexpr int PER = (NV + 7) / 8;                      // vectors per wave
  __shared__ V sum[NV][64];
  const int tl = blockIdx.x >> 3, w = blockIdx.x & 7;
  const int v = threadIdx.x >> 6, lane = threadIdx.x & 63;
  V s[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) s[i] = V{};
  // part[slot][thread][RB NP] with slot = tail tile * tail_P + piece and
  // thread = 64 w + lane of the all-pairs workgroup
  const V* src = (const V*)part + ((int64_t)tl * tail_P * kThreads16 + w * 64 + lane) * NV;
  const int64_t piece_stride = (int64_t)kThreads16 * NV;
#pragma unroll 4
  for (int q = 0; q < tail_P; ++q) {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (v * PER + i < NV) s[i] += src[q * piece_stride + v * PER + i];
  }
  const int ntm = (int)((a_lines + SW::TM - 1) / SW::TM), ntn = (int)(b_lines / kBN);
  int tm, tn;
  if constexpr (SYM) tile_coords_sym(tile0 + tl, ntm, tm, tn);
  else tile_coords(tile0 + tl, ntm, ntn, tm, tn);
  if constexpr (std::is_same<Op, OpI8>::value) {
    // the offset's part (I8Fix) out of the pieces' raw sums
    const int64_t col = (int64_t)tn * kBN + 16 * (w & 3) + (lane & 15);
    const int64_t rb = (int64_t)tm * SW::TM + 16 * RB * (w >> 2) + 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = v * PER + i;  // vector idx = RB k + h
      if (idx < NV) {
        const int k = idx / RB, h = idx % RB;
        const int64_t rh = rb + 16 * h < a_lines ? rb + 16 * h : a_lines - 4;
        const int32x4 sa = *(const int32x4*)(fix.as + (SW::A0 + SW::la(k)) * a_lines + rh);
        const int sb = fix.bs[(SW::BB + SW::lb(k)) * b_lines + col];
        s[i] += i8_start(fix, sa, sb);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (v * PER + i < NV) sum[v * PER + i][lane] = s[i];
  __syncthreads();
  if (v != 0) return;
  V acc[NP][RB];
#pragma unroll
  for (int k = 0; k < NP; ++k) {
#pragma unroll
    for (int h = 0; h < RB; ++h) acc[k][h] = sum[RB * k + h][lane];
  }
  tile_epilogue<Op, SW, ORDER, B0, B1, SYM>(acc, tm, tn, w >> 2, w & 3, lane, Ae, Be, N, M,
                                            a_lines, b_lines, unit2, C, ldc, P, ldp, state, 0);
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
    const float cs32 = scale32(eb);
    const double cs64 = scale64(eb);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = row0 + 32 * mma.wm + acc_row(r, lane);
      const int ea = Ae[q.a * a_lines + row];
      f[r].pair(q, mma.acc[r], cs32, scale32(ea), cs64, scale64(ea));
    }
  }
  if (MODE == 1) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = row0 + 32 * mma.wm + acc_row(r, lane);
    if constexpr (ORDER == kOrderPair) {
      float hi, lo;
      f[r].finish_pair(nblocks, hi, lo);
      if (row < N && col < M) {
        P[row * ldp + col] = hi;
        ((float*)C)[row * ldp + col] = lo;
      }
    } else {
      const double out = f[r].finish(nblocks);
      if (row < N && col < M) C[row * ldc + col] = out;
    }
  }
}

#ifndef OZK_GEMM_PART
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

__global__ void zero_u32_kernel(uint32_t* __restrict__ p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}
#endif  // OZK_GEMM_PART

// Schedules with an all-pairs instantiation: every (n_hi, n_lo) with both
// counts in 1 .. 5, in as few sweeps as fit the kernel (a sweep holds at
// most 25 pairs, the accumulators, and 10 planes, the 160 KiB ring).  One
// sweep when n_hi + n_lo <= 5 (high (4,1), medium (3,1)); else two (hh +
// hl, then lh) when hh + hl fit; else three (hh, hl, lh; max (5,4)).
// Custom schedules take the on-device orders only (2Sum, FP64 block, and
// the pair and per-product forms).
constexpr int allpairs_nsweeps(int nhi, int nlo) {
  return (nhi < 1 || nlo < 1 || nhi > 5 || nlo > 5) ? 0
         : nhi + nlo <= 5                            ? 1
         : (2 * nhi + nlo <= 10 && nhi * (nhi + nlo) <= 25) ? 2
                                                              : 3;
}
constexpr bool allpairs_two_sweeps(int nhi, int nlo) { return allpairs_nsweeps(nhi, nlo) == 2; }
constexpr bool allpairs_three_sweeps(int nhi, int nlo) {
  return allpairs_nsweeps(nhi, nlo) == 3;
}

constexpr bool allpairs_preset(int nhi, int nlo) {
  return (nhi == 4 && nlo == 1) || (nhi == 3 && nlo == 1) || (nhi == 5 && nlo == 4);
}


// Dynamic tail (gemm_allpairs): with R = ntiles / cus whole rounds, the
// last ceil(R / kDynDiv) of them are handed out at run time from one counter
// per XCD and sweep (kDynBytes, zeroed before the launch).  Needs at least
// kDynMinRounds rounds and kDynMinStages stages per tile, so that a claim
// made when a tile starts is known before the ring fetches the next tile.
constexpr int kDynDiv = 8, kDynMinRounds = 4, kDynMinStages = 8;
constexpr size_t kDynBytes = (kDynSlot0 + kDynMaxGrid) * sizeof(uint32_t);

static int dyn_static_rounds(int64_t ntiles, int grid, int64_t nst) {
  const int64_t R = ntiles / grid;
  if (grid % kXcds != 0 || grid > kDynMaxGrid || R < kDynMinRounds || nst < kDynMinStages)
    return 0;
  return (int)(R - (R + kDynDiv - 1) / kDynDiv);
}

// Tiles of an all-pairs sweep with tm-row tiles.
static int64_t allpairs_ntiles(int64_t N, int64_t M, bool sym, int tm) {
  const int64_t al = round_up(N, kLinePad), bl = round_up(M, kLinePad);
  return sym ? (al / kBM) * (al / kBM + 1) / 2 : ((al + tm - 1) / tm) * (bl / kBN);
}

struct ApArgs {
  dim3 grid;
  bool sym;
  int tail_P;
  int tile0;  // first tail tile
  int64_t tail_T;
  uint32_t* part;
  uint32_t* dyn;  // dynamic-tail counters: kXcds per sweep, or null
  int cus;        // the GPU's compute units
  hipStream_t st;
  const char *As, *Bs;
  const int32_t *Ae, *Be;
  int64_t N, M, nst, al, bl;
  float unit2;
  double* C;
  int64_t ldc;
  float* P;
  int64_t ldp;
  char* state;
  I8Fix fix;
};

// One sweep's kernel on operands As .. fix (the rectangle sweeps pass them
// offset to their first planes); `ordinal` picks the sweep's dynamic-tail
// counters.  Its grid (one workgroup per CU, at most one per tile) and
// dynamic tail follow its own tile rows.  A single sweep may split its tail
// along K instead, on the grid the plan of launch_allpairs chose, and then
// runs the fixup.  (Sweeps of multi-sweep schedules do not split: there the
// fixups cost about what the split saves.)
template <class Op, int PIPE, int NHI, int NLO, int ORDER, int B0, int B1, bool SYM>
static void launch_sweep_kernel(const ApArgs& a, const char* As, const int32_t* Ae,
                                const char* Bs, const int32_t* Be, const I8Fix& fix,
                                int ordinal, int rflags) {
  typedef Sweep<PIPE, NHI, NLO, B0, B1, SYM> SW;
  const int64_t nt = allpairs_ntiles(a.N, a.M, SYM, SW::TM);
  dim3 grid((unsigned)(nt < a.cus ? nt : a.cus));
  int tail_P = 0, tile0 = 0;
  int64_t tail_T = 0;
  uint32_t* part = nullptr;
  if constexpr (SW::kFirst && SW::kLast) {
    if (a.tail_P > 1) {
      grid = a.grid;
      tail_P = a.tail_P;
      tail_T = a.tail_T;
      tile0 = a.tile0;
      part = a.part;
    }
  }
  uint32_t* dyn = nullptr;
  int nstat = 0;
  if (tail_P == 0 && a.dyn) {
    nstat = dyn_static_rounds(nt, (int)grid.x, a.nst);
    if (nstat > 0) dyn = a.dyn + kXcds * ordinal;
  }
  hipLaunchKernelGGL((gemm_allpairs<Op, PIPE, NHI, NLO, ORDER, B0, B1, SYM>), grid,
                     dim3(kThreads16), 0, a.st, As, Ae, Bs, Be, a.N, a.M, a.nst, a.al, a.bl,
                     a.unit2, a.C, a.ldc, a.P, a.ldp, a.state, tail_P, part, fix, dyn, nstat,
                     rflags);
  if constexpr (SW::kFirst && SW::kLast) {
    if (tail_P > 1)
      hipLaunchKernelGGL((gemm_tail_fixup<Op, PIPE, NHI, NLO, ORDER, B0, B1, SYM>),
                         dim3((unsigned)(tail_T * 8)), dim3(kThreads16), 0, a.st, part, tail_P,
                         tile0, Ae, Be, a.N, a.M, a.al, a.bl, a.unit2, a.C, a.ldc, a.P, a.ldp,
                         a.state, fix);
  }
}

// One sweep of a fixed schedule (its dynamic-tail counters: those of its
// first block or group).
template <class Op, int PIPE, int NHI, int NLO, int ORDER, int B0, int B1, bool SYM = false>
static void launch_sweep_of(const ApArgs& a) {
  launch_sweep_kernel<Op, PIPE, NHI, NLO, ORDER, B0, B1, SYM>(a, a.As, a.Ae, a.Bs, a.Be, a.fix,
                                                              B0, 0);
}

template <class Op, int NHI, int NLO, int ORDER, int B0, int B1, bool SYM = false>
static void launch_sweep(const ApArgs& a) {
  launch_sweep_of<Op, OZK_PIPE_ONDEVICE, NHI, NLO, ORDER, B0, B1, SYM>(a);
}

// The host schedule's sweeps from group G0 on (host_sweep_end).
template <int N, int ORDER, int G0>
static void launch_host_sweeps(const ApArgs& a) {
  if constexpr (G0 < N) {
    constexpr int G1 = host_sweep_end(N, G0);
    launch_sweep_of<OpBf16, OZK_PIPE_HOST, N, 0, ORDER, G0, G1>(a);
    launch_host_sweeps<N, ORDER, G1 + 1>(a);
  }
}

// The host schedule on BF16 planes in the FP64 orders (and the per-product
// form of the test hook).
template <int N>
static void launch_host_order(int order, const ApArgs& a) {
  switch (order) {
    case OZK_ORDER_BLOCK64: launch_host_sweeps<N, OZK_ORDER_BLOCK64, 0>(a); break;
    case OZK_ORDER_HOST_JAX: launch_host_sweeps<N, OZK_ORDER_HOST_JAX, 0>(a); break;
    case OZK_ORDER_HOST_NP: launch_host_sweeps<N, OZK_ORDER_HOST_NP, 0>(a); break;
    default: launch_host_sweeps<N, kOrderProducts, 0>(a); break;
  }
}

// One rectangle sweep: planes a0.. of A and bb.. of B, the `ordinal`-th
// sweep of its schedule (its dynamic-tail counters), flags kRf*.
struct RectSweep {
  int na, nb, a0, bb, ordinal, rflags;
};

template <class Op, int NA, int NB, int ORDER>
static void launch_rect(const ApArgs& a, const RectSweep& r) {
  // the rectangle's first planes: slice planes, exponents and line sums
  const int64_t aplane = a.al * kChunkBytes * a.nst, bplane = a.bl * kChunkBytes * a.nst;
  I8Fix fix = a.fix;
  if (fix.as) {
    fix.as += (int64_t)r.a0 * a.al;
    fix.bs += (int64_t)r.bb * a.bl;
  }
  launch_sweep_kernel<Op, kPipeRect, NA, NB, ORDER, 0, 0, false>(
      a, a.As + r.a0 * aplane, a.Ae + r.a0 * a.al, a.Bs + r.bb * bplane, a.Be + r.bb * a.bl,
      fix, r.ordinal, r.rflags);
}

// The 2Sum order and its pair form share the 2Sum kernels (kRfPair).
template <class Op, int NA, int NB>
static void launch_rect_order(int order, const ApArgs& a, const RectSweep& r) {
  if (order == OZK_ORDER_BLOCK64) launch_rect<Op, NA, NB, OZK_ORDER_BLOCK64>(a, r);
  else launch_rect<Op, NA, NB, OZK_ORDER_2SUM>(a, r);
}

template <class Op, int NHI, int NLO, int ORDER>
static void launch_schedule(const ApArgs& a) {
  if constexpr (allpairs_three_sweeps(NHI, NLO)) {
    launch_sweep<Op, NHI, NLO, ORDER, 0, 0>(a);
    launch_sweep<Op, NHI, NLO, ORDER, 1, 1>(a);
    launch_sweep<Op, NHI, NLO, ORDER, 2, 2>(a);
  } else if constexpr (allpairs_two_sweeps(NHI, NLO)) {
    launch_sweep<Op, NHI, NLO, ORDER, 0, 1>(a);
    launch_sweep<Op, NHI, NLO, ORDER, 2, 2>(a);
  } else {
    launch_sweep<Op, NHI, NLO, ORDER, 0, 2>(a);
  }
}

template <class Op, int NHI, int NLO>
static void launch_ap_order(int order, const ApArgs& a) {
  switch (order) {
    case OZK_ORDER_2SUM:
      if constexpr (NLO == 1 && (NHI == 3 || NHI == 4)) {  // high, medium: symmetric form
        if (a.sym) {
          launch_sweep<Op, NHI, NLO, OZK_ORDER_2SUM, 0, 2, true>(a);
          break;
        }
      }
      launch_schedule<Op, NHI, NLO, OZK_ORDER_2SUM>(a);
      break;
    case OZK_ORDER_BLOCK64: launch_schedule<Op, NHI, NLO, OZK_ORDER_BLOCK64>(a); break;
    case OZK_ORDER_HOST_JAX:  // presets only (allpairs_order)
      if constexpr (allpairs_preset(NHI, NLO))
        launch_schedule<Op, NHI, NLO, OZK_ORDER_HOST_JAX>(a);
      break;
    case OZK_ORDER_HOST_NP:
      if constexpr (allpairs_preset(NHI, NLO))
        launch_schedule<Op, NHI, NLO, OZK_ORDER_HOST_NP>(a);
      break;
    case kOrderPair: launch_schedule<Op, NHI, NLO, kOrderPair>(a); break;
    default: launch_schedule<Op, NHI, NLO, kOrderProducts>(a); break;
  }
}


#if defined(OZK_GEMM_PART_HOST)
// The host schedules with 1 .. 9 slices (BF16 planes): false for any
// other count.
bool launch_ap_host(int n, int order, const ApArgs& a) {
  switch (n) {
    case 1: launch_host_order<1>(order, a); return true;
    case 2: launch_host_order<2>(order, a); return true;
    case 3: launch_host_order<3>(order, a); return true;
    case 4: launch_host_order<4>(order, a); return true;
    case 5: launch_host_order<5>(order, a); return true;
    case 6: launch_host_order<6>(order, a); return true;
    case 7: launch_host_order<7>(order, a); return true;
    case 8: launch_host_order<8>(order, a); return true;
    case 9: launch_host_order<9>(order, a); return true;
    default: return false;
  }
}
#elif defined(OZK_GEMM_PART_RECT)
// A part of the rectangle sweeps' instantiations: OZK_GEMM_RECT_SHAPES(X)
// names its (NA, NB).  Returns false for a shape of another part.
bool OZK_GEMM_PART_FN(bool i8, int order, const ApArgs& a, const RectSweep& r) {
#define OZK_RECT_CASE(A, B)                                 \
  if (r.na == A && r.nb == B) {                             \
    if (i8) launch_rect_order<OpI8, A, B>(order, a, r);     \
    else launch_rect_order<OpBf16, A, B>(order, a, r);      \
    return true;                                            \
  }
  OZK_GEMM_RECT_SHAPES(OZK_RECT_CASE)
#undef OZK_RECT_CASE
  return false;
}
#elif defined(OZK_GEMM_PART)
// A part of the schedules' instantiations, compiled as a translation unit
// of its own so that the parts build in parallel: OZK_GEMM_PART_TUPLES(X)
// names its (n_hi, n_lo).  Returns false for a schedule of another part.
bool OZK_GEMM_PART_FN(bool i8, int nhi, int nlo, int order, const ApArgs& a) {
#define OZK_PART_CASE(H, L)                                   \
  if (nhi == H && nlo == L) {                                 \
    if (i8) launch_ap_order<OpI8, H, L>(order, a);            \
    else launch_ap_order<OpBf16, H, L>(order, a);             \
    return true;                                              \
  }
  OZK_GEMM_PART_TUPLES(OZK_PART_CASE)
#undef OZK_PART_CASE
  return false;
}
#else
bool launch_ap_part1(bool i8, int nhi, int nlo, int order, const ApArgs& a);
bool launch_ap_part2(bool i8, int nhi, int nlo, int order, const ApArgs& a);
bool launch_ap_part3(bool i8, int nhi, int nlo, int order, const ApArgs& a);
bool launch_ap_part4(bool i8, int nhi, int nlo, int order, const ApArgs& a);
bool launch_ap_host(int n, int order, const ApArgs& a);
bool launch_ap_rect1(bool i8, int order, const ApArgs& a, const RectSweep& r);
bool launch_ap_rect2(bool i8, int order, const ApArgs& a, const RectSweep& r);

// The on-device schedules beyond the fixed ones, both counts up to
// kRectMaxSlices, as rectangle sweeps: each block (hh, hl, lh) is cut into
// as few rectangles of consecutive groups as fit a sweep (kSweepPlanes,
// kSweepPairs), the groups spread evenly over them.  rect_plan fills `out`
// (if given) and returns the number of sweeps; *mid says whether some
// block is cut (its running sum then crosses a sweep boundary).
constexpr int kRectMaxSlices = 8;
constexpr int kRectMaxSweeps = kDynSlot0 / kXcds;

// Sweeps of a rectangle schedule (as rect_plan cuts it), and a check that
// every schedule's sweeps fit the plan array and the dynamic-tail words.
constexpr int rect_nsweeps(int nhi, int nlo) {
  int n = 0;
  for (int blk = 0; blk < 3; ++blk) {
    const int ng = blk == 2 ? nlo : nhi, nb = blk == 1 ? nlo : nhi;
    int na = ng;
    while (na > 1 && (na + nb > kSweepPlanes || na * nb > kSweepPairs)) --na;
    n += (ng + na - 1) / na;
  }
  return n;
}
constexpr bool rect_sweeps_fit() {
  for (int h = 1; h <= kRectMaxSlices; ++h)
    for (int l = 1; l <= kRectMaxSlices; ++l)
      if (rect_nsweeps(h, l) > kRectMaxSweeps) return false;
  return true;
}
static_assert(rect_sweeps_fit(), "a rectangle schedule has more sweeps than the plan holds");

static bool rect_tuple(int nhi, int nlo) {
  return allpairs_nsweeps(nhi, nlo) == 0 && nhi >= 1 && nlo >= 1 && nhi <= kRectMaxSlices &&
         nlo <= kRectMaxSlices;
}

static int rect_plan(int nhi, int nlo, bool pair_out, RectSweep* out, bool* mid) {
  int n = 0;
  if (mid) *mid = false;
  for (int blk = 0; blk < 3; ++blk) {
    const int ng = blk == 2 ? nlo : nhi;       // groups: the block's A planes
    const int nb = blk == 1 ? nlo : nhi;       // B planes of every group
    const int a_base = blk == 2 ? nhi : 0, b_base = blk == 1 ? nhi : 0;
    int na = ng;
    while (na > 1 && (na + nb > kSweepPlanes || na * nb > kSweepPairs)) --na;
    const int nsw = (ng + na - 1) / na;
    if (nsw > 1 && mid) *mid = true;
    for (int sw = 0, g0 = 0; sw < nsw; ++sw) {
      const int cnt = ng / nsw + (sw < ng % nsw ? 1 : 0);
      const int g1 = g0 + cnt - 1;
      if (out) {
        RectSweep& r = out[n];
        r.na = cnt;
        r.nb = nb;
        r.a0 = a_base + g0;
        r.bb = b_base;
        r.ordinal = n;
        r.rflags = blk | (g0 == 0 ? kRfGFirst : 0) | (g1 == ng - 1 ? kRfGLast : 0) |
                   (blk == 0 && g0 == 0 ? kRfFirst : 0) |
                   (blk == 2 && g1 == ng - 1 ? kRfLast : 0) | (pair_out ? kRfPair : 0) |
                   (blk << kRfDone0) | ((g1 == ng - 1 ? blk + 1 : blk) << kRfDone1);
      }
      ++n;
      g0 = g1 + 1;
    }
  }
  return n;
}

// Host schedules (FP64 extraction, BF16 planes) of up to this many slices
// run on the all-pairs kernel, in sweeps over groups of A planes: group 0
// pairs A plane 0 with all n B planes, which fit one stage beside it for
// n <= 9.  (Nine slices of 6 bits are what the host pipeline needs for
// 2048 < K <= 4226, where rho = 47.)
constexpr int kHostMaxSlices = 9;

// Orders the all-pairs kernel runs for schedule (nhi, nlo): every order for
// the on-device presets, the on-device ones for the custom schedules (the
// rectangle sweeps: 2Sum, its pair form and the FP64 block order), the FP64
// ones (and the per-product form) for the host schedules.
static bool allpairs_order(int pipe, int nhi, int nlo, int order) {
  if (pipe == OZK_PIPE_HOST)
    return order == OZK_ORDER_BLOCK64 || order == OZK_ORDER_HOST_JAX ||
           order == OZK_ORDER_HOST_NP || order == kOrderProducts;
  if (rect_tuple(nhi, nlo))
    return order == OZK_ORDER_2SUM || order == OZK_ORDER_BLOCK64 || order == kOrderPair;
  return allpairs_preset(nhi, nlo) ||
         (order != OZK_ORDER_HOST_JAX && order != OZK_ORDER_HOST_NP);
}

static bool allpairs_schedule(int pipe, int nhi, int nlo) {
  if (pipe == OZK_PIPE_HOST) return nlo == 0 && nhi >= 1 && nhi <= kHostMaxSlices;
  return pipe == OZK_PIPE_ONDEVICE && (allpairs_nsweeps(nhi, nlo) > 0 || rect_tuple(nhi, nlo));
}

static int allpairs_sweeps(int pipe, int nhi, int nlo) {
  if (pipe == OZK_PIPE_HOST) return host_nsweeps(nhi);
  return rect_tuple(nhi, nlo) ? rect_plan(nhi, nlo, false, nullptr, nullptr)
                              : allpairs_nsweeps(nhi, nlo);
}

bool allpairs_supported(int pipe, int nhi, int nlo) {
  return allpairs_schedule(pipe, nhi, nlo);
}

// The per-pair products (test hook) on the all-pairs kernel: the fixed
// schedules only.
bool allpairs_products_supported(int pipe, int nhi, int nlo) {
  return allpairs_schedule(pipe, nhi, nlo) && allpairs_order(pipe, nhi, nlo, kOrderProducts);
}

// Bytes per element of the fold state between sweeps: the 2Sum order also
// carries a block's running sum where a rectangle sweep cuts a block.
static int fold_state_bytes(int pipe, int nhi, int nlo, int order) {
  if (order != OZK_ORDER_2SUM) return FoldState<OZK_ORDER_BLOCK64>::kBytes;
  bool mid = false;
  if (pipe == OZK_PIPE_ONDEVICE && rect_tuple(nhi, nlo))
    rect_plan(nhi, nlo, false, nullptr, &mid);
  return mid ? FoldState<OZK_ORDER_2SUM>::kBytesMid : FoldState<OZK_ORDER_2SUM>::kBytes;
}

// Workspace an all-pairs product cannot run without: the fold state kept
// between the sweeps of a multi-sweep schedule (0 for one sweep).
// The per-product form keeps no state; the pair form keeps the 2Sum state.
size_t gemm_state_bytes(int64_t N, int64_t M, int pipe, int nhi, int nlo, int order) {
  if (!allpairs_schedule(pipe, nhi, nlo) || !allpairs_order(pipe, nhi, nlo, order) ||
      allpairs_sweeps(pipe, nhi, nlo) == 1 || order == kOrderProducts)
    return 0;
  const int fold = order == kOrderPair ? OZK_ORDER_2SUM : order;
  return (size_t)N * (size_t)M * (size_t)fold_state_bytes(pipe, nhi, nlo, fold);
}

// K-split of the tail.  With R = ntiles / cus whole rounds of one tile per
// workgroup and T = ntiles % cus tiles left, the last round would keep T
// CUs busy while the others idle.  Instead each tail tile is split along K
// into P = min(cus / T, nst / kMinPieceStages) pieces, one per workgroup,
// whose raw sums gemm_tail_fixup adds up and folds.  Single-sweep schedules
// only; needs T * P * NP * RB * 4 * kThreads16 * 4 bytes of workspace.
constexpr int kMinPieceStages = 16;

struct TailPlan {
  int P = 0;        // pieces per tail tile (0: no split)
  int64_t T = 0;    // tail tiles
  int grid = 0;     // all-pairs workgroups
  size_t bytes = 0; // partial sums
};

static TailPlan plan_tail(int64_t ntiles, int cus, int64_t nst, int np, int rb) {
  TailPlan tp;
  const int64_t R = ntiles / cus, T = ntiles % cus;
  if (T == 0) return tp;
  const int64_t P = cus / T < nst / kMinPieceStages ? cus / T : nst / kMinPieceStages;
  if (P < 2) return tp;
  tp.P = (int)P;
  tp.T = T;
  tp.grid = R > 0 ? cus : (int)(T * P);
  tp.bytes = (size_t)(T * P) * (size_t)np * 4 * rb * kThreads16 * sizeof(uint32_t);
  return tp;
}

// Workspace of the fastest all-pairs launch: the fold state, then the
// dynamic-tail words.  (The K-split tail's partial sums, gemm_tail_bytes,
// follow them where a driver reserves those too.)
size_t gemm_workspace_bytes(int64_t N, int64_t M, int pipe, int nhi, int nlo,
                            int order) {
  if (!allpairs_schedule(pipe, nhi, nlo) || !allpairs_order(pipe, nhi, nlo, order)) return 0;
  return (size_t)round_up((int64_t)gemm_state_bytes(N, M, pipe, nhi, nlo, order), 256) +
         kDynBytes;
}

// Tile rows of the all-pairs launch of schedule (nhi, nlo): those of its
// single sweep; 64 for a multi-sweep schedule, whose sweeps size their own
// grids (64-row tiles give the most tiles, the bound the launch checks).
static int allpairs_tm(int pipe, int nhi, int nlo, bool sym) {
  if (allpairs_sweeps(pipe, nhi, nlo) != 1) return 64;
  return 32 * (pipe == OZK_PIPE_HOST ? ap_rb_of(pair_count(pipe, nhi, 0), nhi, nhi, false)
                                     : ap_rb(nhi, nlo, 0, 2, sym));
}

static int64_t allpairs_nst(int64_t K, bool i8) {
  // chunks per line: round_up(K, kKPad) elements of 1 or 2 bytes
  return round_up(K, kKPad) * (i8 ? 1 : 2) / kChunkBytes;
}

// Workspace of the K-split tail of an N x M (x K) all-pairs product: zero
// when the product does not split (multi-sweep schedules never do).
size_t gemm_tail_bytes(int64_t N, int64_t M, int64_t K, int pipe, int nhi, int nlo,
                       bool sym, bool i8) {
  if (!allpairs_schedule(pipe, nhi, nlo) || allpairs_sweeps(pipe, nhi, nlo) != 1) return 0;
  const int tm = allpairs_tm(pipe, nhi, nlo, sym);
  return plan_tail(allpairs_ntiles(N, M, sym, tm), cu_count(), allpairs_nst(K, i8),
                   pair_count(pipe, nhi, nlo), tm / 32)
      .bytes;
}

// All-pairs launch for an all-pairs schedule; `i8` selects the INT8 plane
// format (rho >= 19).  order = kOrderProducts writes P.  `state` holds at
// least gemm_state_bytes(); with gemm_workspace_bytes() the last rounds of
// tiles are handed out dynamically, and a single-sweep schedule splits its
// tail along K instead when `state` also holds gemm_tail_bytes().
static int launch_allpairs(bool i8, int pipe, const void* As, const int32_t* Ae,
                           const void* Bs, const int32_t* Be, int64_t N,
                           int64_t M, int64_t K, int rho, int nhi, int nlo,
                           int order, double* C, int64_t ldc, float* P,
                           int64_t ldp, void* state, size_t state_bytes,
                           hipStream_t st, const int32_t* Asum, const int32_t* Bsum,
                           bool sym = false) {
  if (i8 && (!Asum || !Bsum)) {
    set_error("int8 slice planes need their line sums");
    return OZK_ERR_INVALID;
  }
  const size_t need = gemm_state_bytes(N, M, pipe, nhi, nlo, order);
  if (state_bytes < need || (need && !state)) {
    set_error("gemm workspace of %zu bytes < %zu needed", state_bytes, need);
    return OZK_ERR_WORKSPACE;
  }
  ApArgs a;
  const int64_t al = round_up(N, kLinePad), bl = round_up(M, kLinePad);
  const int tmr = allpairs_tm(pipe, nhi, nlo, sym);
  const int64_t ntiles = allpairs_ntiles(N, M, sym, tmr);
  OZK_CHECK_ARG(ntiles < (1ll << 31), "problem too large for one launch");
  // persistent: one workgroup per CU (the 160 KiB ring fills its LDS)
  const int cus = cu_count();
  a.grid = dim3((unsigned)(ntiles < cus ? ntiles : cus));
  a.tail_P = 0;
  a.tile0 = 0;
  a.tail_T = 0;
  a.part = nullptr;
  a.dyn = nullptr;
  a.cus = cus;
  // workspace: fold state | dynamic-tail words | K-split partial sums
  const size_t off = round_up((int64_t)need, 256);
  if (allpairs_sweeps(pipe, nhi, nlo) == 1) {
    const TailPlan tp = plan_tail(ntiles, cus, allpairs_nst(K, i8),
                                  pair_count(pipe, nhi, nlo), tmr / 32);
    if (tp.P > 1 && state && state_bytes >= off + kDynBytes + tp.bytes) {
      a.grid = dim3((unsigned)tp.grid);
      a.tail_P = tp.P;
      a.tail_T = tp.T;
      a.tile0 = (int)(ntiles - tp.T);
      a.part = (uint32_t*)((char*)state + off + kDynBytes);
    }
  }
  // the dynamic tail's counters, when some sweep will use them (each sweep
  // decides for its own tiles in launch_sweep_kernel)
  if (!a.part && state && state_bytes >= off + kDynBytes &&
      (allpairs_sweeps(pipe, nhi, nlo) > 1 ||
       dyn_static_rounds(ntiles, (int)a.grid.x, allpairs_nst(K, i8)) > 0)) {
    a.dyn = (uint32_t*)((char*)state + off);
    hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(64), 0, st, a.dyn, kDynSlot0);
  }
  a.sym = sym;
  a.st = st;
  a.As = (const char*)As;
  a.Bs = (const char*)Bs;
  a.Ae = Ae;
  a.Be = Be;
  a.N = N;
  a.M = M;
  a.nst = allpairs_nst(K, i8);
  a.al = al;
  a.bl = bl;
  a.unit2 = ldexpf(1.0f, 2 * rho - 48);
  a.C = C;
  a.ldc = ldc;
  a.P = P;
  a.ldp = ldp;
  a.state = (char*)state;
  a.fix.as = Asum;
  a.fix.bs = Bsum;
  a.fix.off = i8 ? (uint32_t)i8_offset(rho) : 0u;
  a.fix.kpo2 = (uint32_t)((uint64_t)(a.nst * kChunkBytes) * a.fix.off * a.fix.off);
  if (pipe == OZK_PIPE_ONDEVICE && rect_tuple(nhi, nlo)) {
    RectSweep plan[kRectMaxSweeps];
    const int n = rect_plan(nhi, nlo, order == kOrderPair, plan, nullptr);
    const int ord = order == kOrderPair ? OZK_ORDER_2SUM : order;
    for (int i = 0; i < n; ++i) {
      if (!launch_ap_rect1(i8, ord, a, plan[i]) && !launch_ap_rect2(i8, ord, a, plan[i])) {
        set_error("rectangle sweep %d x %d has no instantiation", plan[i].na, plan[i].nb);
        return OZK_ERR_UNSUPPORTED;
      }
    }
    OZK_LAUNCH_CHECK();
    return OZK_OK;
  }
  if (pipe == OZK_PIPE_HOST) {
    if (!launch_ap_host(nhi, order, a)) {
      set_error("host schedule of %d slices has no all-pairs instantiation", nhi);
      return OZK_ERR_UNSUPPORTED;
    }
    OZK_LAUNCH_CHECK();
    return OZK_OK;
  }
  // the presets and the smallest custom schedules here, the others in the
  // parts (gemm_parts.h)
  bool done = true;
#define OZK_AP_MAIN(Op)                                                   \
  do {                                                                    \
    if (nhi == 4 && nlo == 1) launch_ap_order<Op, 4, 1>(order, a);        \
    else if (nhi == 3 && nlo == 1) launch_ap_order<Op, 3, 1>(order, a);   \
    else if (nhi == 5 && nlo == 4) launch_ap_order<Op, 5, 4>(order, a);   \
    else if (nhi == 1 && nlo == 1) launch_ap_order<Op, 1, 1>(order, a);   \
    else if (nhi == 2 && nlo == 1) launch_ap_order<Op, 2, 1>(order, a);   \
    else if (nhi == 2 && nlo == 2) launch_ap_order<Op, 2, 2>(order, a);   \
    else done = false;                                                    \
  } while (0)
  if (i8) OZK_AP_MAIN(OpI8);
  else OZK_AP_MAIN(OpBf16);
#undef OZK_AP_MAIN
  if (!done && !launch_ap_part1(i8, nhi, nlo, order, a) &&
      !launch_ap_part2(i8, nhi, nlo, order, a) && !launch_ap_part3(i8, nhi, nlo, order, a) &&
      !launch_ap_part4(i8, nhi, nlo, order, a)) {
    set_error("all-pairs schedule (%d, %d) has no instantiation", nhi, nlo);
    return OZK_ERR_UNSUPPORTED;
  }
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

// Gram matrix of one plane set (A's columns) with itself: only the tiles on
// and above the diagonal are computed, and the epilogue writes
// (C + C^T) * 0.5 to both halves (2Sum order; presets (4,1) and (3,1)).
bool gram_sym_supported(int nhi, int nlo) { return nlo == 1 && (nhi == 4 || nhi == 3); }

int launch_gram_sym(const void* S, const int32_t* E, int64_t n, int64_t K, int nhi,
                    int nlo, double* G, int64_t ldg, void* ws, size_t ws_bytes,
                    hipStream_t st, bool i8, int rho, const int32_t* Ssum) {
  if (!gram_sym_supported(nhi, nlo)) {
    set_error("symmetric gram needs the high or medium preset");
    return OZK_ERR_UNSUPPORTED;
  }
  return launch_allpairs(i8, OZK_PIPE_ONDEVICE, S, E, S, E, n, n, K, rho, nhi, nlo, OZK_ORDER_2SUM, G, ldg,
                         nullptr, 0, ws, ws_bytes, st, Ssum, Ssum, true);
}

int launch_gemm(const void* As, const int32_t* Ae, const void* Bs,
                const int32_t* Be, int64_t N, int64_t M, int64_t K, int pipe,
                int nhi, int nlo, int order, double* C, int64_t ldc,
                void* ws, size_t ws_bytes, hipStream_t st, bool i8, int rho,
                const int32_t* Asum, const int32_t* Bsum) {
  if (allpairs_schedule(pipe, nhi, nlo) && allpairs_order(pipe, nhi, nlo, order))
    return launch_allpairs(i8, pipe, As, Ae, Bs, Be, N, M, K, rho, nhi, nlo, order,
                           C, ldc, nullptr, 0, ws, ws_bytes, st, Asum, Bsum);
  if (i8) {
    set_error("int8 slice planes need an all-pairs on-device schedule");
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

// The on-device schedule of (nhi, nlo) in the 2Sum order, written as the
// pair (C_hi, C_lo), FP32, both with leading dimension ldc.
int launch_gemm_pair(const void* As, const int32_t* Ae, const void* Bs,
                     const int32_t* Be, int64_t N, int64_t M, int64_t K, int nhi,
                     int nlo, float* C_hi, float* C_lo, int64_t ldc, void* ws,
                     size_t ws_bytes, hipStream_t st, bool i8, int rho,
                     const int32_t* Asum, const int32_t* Bsum) {
  if (allpairs_schedule(OZK_PIPE_ONDEVICE, nhi, nlo))
    return launch_allpairs(i8, OZK_PIPE_ONDEVICE, As, Ae, Bs, Be, N, M, K, rho, nhi, nlo, kOrderPair,
                           (double*)C_lo, ldc, C_hi, ldc, ws, ws_bytes, st, Asum, Bsum);
  if (i8) {
    set_error("int8 slice planes need an all-pairs on-device schedule");
    return OZK_ERR_UNSUPPORTED;
  }
  const int64_t ld = round_up(K, kKPad);
  const int64_t al = round_up(N, kLinePad), bl = round_up(M, kLinePad);
  const int64_t ntiles = (al / kBM) * (bl / kBN);
  OZK_CHECK_ARG(ntiles < (1ll << 31), "problem too large for one launch");
  hipLaunchKernelGGL((gemm_pairwise<kOrderPair, 0>), dim3((unsigned)ntiles), dim3(kThreads),
                     0, st, (const uint16_t*)As, Ae, (const uint16_t*)Bs, Be, N, M, ld, al,
                     bl, (int)OZK_PIPE_ONDEVICE, nhi, nlo, (double*)C_lo, ldc, C_hi, ldc);
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

// Per-pair products.  All-pairs schedules run the all-pairs kernel (the one
// the drivers use); other schedules (BF16 only) the pairwise kernel.
int launch_products(const void* As, const void* Bs, int64_t N, int64_t M,
                    int64_t K, int pipe, int nhi, int nlo, float* P,
                    int64_t ldp, hipStream_t st, bool i8, int rho, const int32_t* Asum,
                    const int32_t* Bsum) {
  if (allpairs_schedule(pipe, nhi, nlo) && allpairs_order(pipe, nhi, nlo, kOrderProducts))
    return launch_allpairs(i8, pipe, As, nullptr, Bs, nullptr, N, M, K, rho, nhi, nlo,
                           kOrderProducts, nullptr, 0, P, ldp, nullptr, 0, st, Asum, Bsum);
  if (i8) {
    set_error("int8 slice planes need an all-pairs on-device schedule");
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

#endif  // OZK_GEMM_PART

}  // namespace ozk
