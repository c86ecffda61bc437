// Split + sigma-trick slice extraction kernels (bandwidth-bound).
//
// One workgroup owns one line (a row of X, or a row of X^T for column
// extraction) and keeps the whole line's residual on chip (registers, and
// for the longest lines the lo parts in LDS), so X is read from HBM once and
// every slice plane is written once.  Per slice the line
// maximum comes from a wavefront butterfly + an LDS combine across waves.
// Lines too long for one workgroup, and columns read in place, are held by
// gangs of workgroups that exchange their partial maxima through global
// memory; lines longer still are streamed.
//
// Arithmetic per slice (reference extract.py:124-152 for FP32, :28-63 for
// FP64; split matmul.py:204-213):
//   m = max|R|; c = m == 0 ? 0 : floor(RN(log2 m)); sigma = 0.75 * 2^(rho+c)
//   v = (R + sigma) - sigma (v = 0 when m == 0); R = R - v; slice = v * 2^-c
// All floating-point operations are single IEEE round-to-nearest operations
// (built with -ffp-contract=off, denormals kept).

#include "sigma.h"

#include <type_traits>

namespace ozk {

// Slice plane formats.  BF16: the FP32 slice value's BF16 bits.  I8: the
// slice as an integer count of its grid step, q = slice * 2^(24 - rho)
// (FP32 path only; |q| <= 2^(25 - rho) <= 64 for rho >= 19, so exact),
// stored as q + 2^(25 - rho) - 1 (i8_offset), with the sum of q over each
// plane line written beside the plane (see the slice GEMM's I8Fix).
constexpr int kFmtBf16 = 0, kFmtI8 = 1;
constexpr int kMaxSlices = 32;
constexpr int kMaxPlanes = 2 * kMaxSlices;

template <int FMT> struct PlaneElem;
template <> struct PlaneElem<kFmtBf16> {
  typedef uint16_t type;
  static __device__ __forceinline__ uint16_t make(float s, float) {
    return f32_to_bf16_bits(s);
  }
};
template <> struct PlaneElem<kFmtI8> {
  typedef int8_t type;
  // qscale = 2^(24 - rho), so 2 qscale - 1 is the offset
  static __device__ __forceinline__ int8_t make(float s, float qscale) {
    return (int8_t)((int)(s * qscale) + (int)(2.0f * qscale) - 1);
  }
};

// acc + the sum of the signed bytes of w (one dot product with ones)
__device__ __forceinline__ int byte_sum(uint32_t w, int acc) {
  return __builtin_amdgcn_sdot4((int)w, 0x01010101, acc, false);
}
__device__ __forceinline__ int byte_sum(uint16_t w, int acc) { return byte_sum((uint32_t)w, acc); }
__device__ __forceinline__ int byte_sum(uint2 w, int acc) { return byte_sum(w.y, byte_sum(w.x, acc)); }

// A value that every lane of the wave holds, as a scalar.
__device__ __forceinline__ float wave_uniform(float x) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}
__device__ __forceinline__ double wave_uniform(double x) {
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Slices the INT8 format cannot hold.  The reference's slice of a line is
// non-finite when sigma = 0.75 * 2^(rho + c) or 2^-c overflows FP32
// (extract.py:134-136, :145-148), and a NaN / Inf element makes every slice
// of its line non-finite.  Each product with such a slice is NaN or +-inf,
// so the output row / column is NaN in the 2Sum order whichever slice it
// was.  INT8 planes store the slice as zeros (v = 0, so the residual and
// with it the overflow carry into the next slice, which is stored the same
// way) with exponent OZK_EXP_NONFINITE; the slice GEMM folds every product
// with it as NaN.  A 2^-c overflow can leave the reference's slice all +-inf
// with no NaN, whose products may then be +-inf: OZK_FLAG_INF_SLICE.
// Returns the exponent to store; `leader` is one thread of the line.
template <int FMT, typename W>
__device__ __forceinline__ int plane_exponent(SliceConst<W>& kc, int rho,
                                              uint32_t* flags, bool leader) {
  if constexpr (FMT == kFmtI8) {
    if (!kc.zero && (rho + kc.c >= 128 || kc.c <= -128)) {
      if (kc.c <= -128 && leader) atomicOr(flags, OZK_FLAG_INF_SLICE);
      kc.zero = true;
      kc.inv = W(1);
      return OZK_EXP_NONFINITE;
    }
  }
  return kc.c;
}

// Line-maximum contribution of a thread that read a NaN / Inf element: on
// INT8 planes +inf, whose exponent plane_exponent classifies as overflow in
// every slice of the line.  (The BF16 format carries such values itself.)
template <int FMT, typename W>
__device__ __forceinline__ W line_max_input(W m, bool bad) {
  if constexpr (FMT == kFmtI8) return bad ? W(INFINITY) : m;
  return m;
}

// Line maxima of up to two parts at once: wave butterfly then LDS combine
// over the BLOCK / 64 waves of the thread's line (a workgroup holds LPB
// lines of BLOCK threads each).
template <typename W, int BLOCK, int LPB, int NP>
__device__ __forceinline__ void block_max2(W (&m)[NP], W* red) {
  constexpr int NW = BLOCK / 64;
#pragma unroll
  for (int q = 0; q < NP; ++q) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m[q] = max_w(m[q], __shfl_xor(m[q], off));
  }
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int w0 = (wid / NW) * NW;  // first wave of this line
  __syncthreads();  // previous readers of red are done
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < NP; ++q) red[q * NW * LPB + wid] = m[q];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    W r = red[q * NW * LPB + w0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r = max_w(r, red[q * NW * LPB + w0 + w]);
    m[q] = r;
  }
}

// Line group handled by workgroup `bid` of `n` (n a multiple of 8):
// consecutive workgroups go round-robin to the 8 XCDs, so groups are dealt
// out such that neighbouring groups, whose chunks share cache lines in the
// plane layout, are written from the same XCD.
__device__ __forceinline__ int64_t xcd_line(int64_t bid, int64_t n) {
  return (bid & 7) * (n >> 3) + (bid >> 3);
}

// Register-resident extraction.  A workgroup owns LPB consecutive lines,
// BLOCK threads each; thread t of a line owns the VEC consecutive elements
// k = (j * BLOCK + t) * VEC + v, j < EPT, v < VEC, which must cover the
// padded line (EPT * BLOCK * VEC >= ld).  With `vec_ok` (line starts 16-byte
// aligned, len a multiple of VEC) a thread reads its VEC doubles with 16-byte
// loads; it writes its
// VEC plane elements, which are adjacent in the plane, with one store.
// Planes: part 0 -> [0, n0), part 1 -> [n0, n0 + n1).
template <int FMT, int VEC> struct PlaneVec;
template <> struct PlaneVec<kFmtI8, 2> { typedef uint16_t type; };
template <> struct PlaneVec<kFmtI8, 4> { typedef uint32_t type; };
template <> struct PlaneVec<kFmtBf16, 2> { typedef uint32_t type; };
template <> struct PlaneVec<kFmtBf16, 4> { typedef uint2 type; };
template <> struct PlaneVec<kFmtI8, 8> { typedef uint2 type; };
template <> struct PlaneVec<kFmtBf16, 8> { typedef uint4 type; };

// Short-form plane words (fast_step): the carriers c[u] of the VEC
// elements (INT8: q + i8_magic(offset), whose low byte is the element; BF16:
// q * 2^(rho - 24), exact in BF16, whose high half is the element) packed
// as the elements' word.
template <int FMT, int VEC>
__device__ __forceinline__ typename PlaneVec<FMT, VEC>::type pack_fast(const float (&c)[VEC]) {
  typedef typename PlaneVec<FMT, VEC>::type TV;
  if constexpr (FMT == kFmtI8 && VEC == 2) {
    return (TV)pack_low_bytes(c[0], c[1], c[1], c[1]);
  } else {
    union {
      TV v;
      uint32_t w[sizeof(TV) / 4];
    } o;
    if constexpr (FMT == kFmtI8) {
#pragma unroll
      for (int i = 0; i < VEC / 4; ++i)
        o.w[i] = pack_low_bytes(c[4 * i], c[4 * i + 1], c[4 * i + 2], c[4 * i + 3]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC / 2; ++i) o.w[i] = pack_high_halves(c[2 * i], c[2 * i + 1]);
    }
    return o.v;
  }
}

// The carrier constant of pack_fast for a slice of grid count q.
template <int FMT>
__device__ __forceinline__ float fast_carrier(int rho) {
  return FMT == kFmtI8 ? i8_magic(i8_offset(rho)) : ldexpf(1.0f, rho - 24);
}
// BF16: q * 2^(rho - 24) + 0, so that q = -0 (rint of a small negative
// number) gives +0, as the plain form's (R + sigma) - sigma does.
template <int FMT>
__device__ __forceinline__ float fast_carry(float q, float k) {
  return FMT == kFmtI8 ? q + k : __builtin_fmaf(q, k, 0.0f);
}

template <typename W, int BLOCK, int EPT, int LPB, int FMT, int VEC>
__global__ __launch_bounds__(BLOCK * LPB) void extract_lines_reg(
    const double* __restrict__ X, int64_t lines, int64_t len, int64_t ldx,
    int vec_ok, int rho, int n0, int n1, typename PlaneElem<FMT>::type* __restrict__ S,
    int64_t ld, int64_t plane, int32_t* __restrict__ E, int64_t eplane,
    uint32_t* __restrict__ flags, int32_t* __restrict__ Sg) {
  static_assert(VEC == 2 || VEC == 4, "VEC doubles are read as 16-byte pairs");
  const float qscale = ldexpf(1.0f, 24 - rho);
  constexpr int NP = Parts<W>::N;
  __shared__ W red[NP * (BLOCK / 64) * LPB];
  // INT8: line sums of q per plane.  Every thread adds up the bytes it packs
  // (q + offset, the elements past the line's end included: their q is 0),
  // the waves meet in LDS, and offset x BLOCK * EPT * VEC comes off at the end.
  __shared__ int ssum[FMT == kFmtI8 ? kMaxPlanes * LPB : 1];
  if constexpr (FMT == kFmtI8) {
    for (int i = threadIdx.x; i < kMaxPlanes * LPB; i += BLOCK * LPB) ssum[i] = 0;
  }
  const int t = threadIdx.x % BLOCK;
  const int64_t grp = xcd_line(blockIdx.x, gridDim.x);
  const int64_t line = grp * LPB + threadIdx.x / BLOCK;
  const bool live = line < lines;
  // Plane offset of the thread's first element: BLOCK * VEC is a multiple of
  // the elements per chunk, so the in-chunk position (and its swizzle) is
  // fixed per thread and j only advances the chunk by BLOCK * VEC / kPer.
  typedef typename PlaneElem<FMT>::type T;
  typedef typename PlaneVec<FMT, VEC>::type TV;
  constexpr int kPer = kChunkBytes / (int)sizeof(T);
  static_assert((BLOCK * VEC) % kPer == 0, "BLOCK * VEC must hold whole chunks");
  const int64_t off0 = plane_offset<sizeof(T)>(line, (int64_t)t * VEC, eplane);
  const int64_t step = (int64_t)(BLOCK * VEC / kPer) * eplane * kPer;
  // 512-thread workgroups whose threads hold 32 elements keep the lo parts
  // in LDS (64 KiB) and only the hi parts in registers, so that two of them
  // fit on a CU rather than one.  (256 threads x 32 elements fit four per
  // CU in registers alone, which was faster than with the LDS traffic.)
  constexpr bool kLoLds = NP == 2 && BLOCK * LPB == 512 && EPT * VEC == 32;
  __shared__ float lo[kLoLds ? EPT * VEC : 1][kLoLds ? BLOCK * LPB : 1];
  W Rr[kLoLds ? 1 : NP][EPT * VEC];
  auto R = [&](int q, int i) -> W& {
    if constexpr (kLoLds) return q == 0 ? Rr[0][i] : lo[i][threadIdx.x];
    else return Rr[q][i];
  };
  bool bad = false;
  // Every load reads an address inside X (an element past the line's end
  // reads the line's first element, a line past the last reads line 0) and
  // its value is replaced by zero afterwards, so no branch separates the
  // chunks' loads and several are in flight at once.  vec_ok (16-byte
  // aligned lines, len a multiple of VEC): 16-byte loads, whole chunks.
  const double* xl = X + (live ? line : 0) * ldx;
  auto read_split = [&](auto vec) {
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int64_t k0 = ((int64_t)j * BLOCK + t) * VEC;
      double v[VEC];
      if constexpr (decltype(vec)::value) {
        const bool ok = live && k0 < len;
        const double* p = xl + (ok ? k0 : 0);
#pragma unroll
        for (int u = 0; u < VEC; u += 2) {
          const double2 d = *(const double2*)(p + u);
          v[u] = ok ? d.x : 0.0;
          v[u + 1] = ok ? d.y : 0.0;
        }
      } else {
#pragma unroll
        for (int u = 0; u < VEC; ++u) {
          const bool ok = live && k0 + u < len;
          const double d = xl[ok ? k0 + u : 0];
          v[u] = ok ? d : 0.0;
        }
      }
#pragma unroll
      for (int u = 0; u < VEC; ++u) {
        bad |= !isfinite(v[u]);
        W p[NP];
        split<W>(v[u], p);
#pragma unroll
        for (int q = 0; q < NP; ++q) R(q, j * VEC + u) = p[q];
      }
    }
  };
  if (vec_ok)
    read_split(std::true_type());
  else
    read_split(std::false_type());
  if (bad) atomicOr(flags, OZK_FLAG_NONFINITE);

  const int ns = NP == 2 ? max(n0, n1) : n0;
  for (int s = 0; s < ns; ++s) {
    W m[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      m[q] = W(0);
#pragma unroll
      for (int j = 0; j < EPT * VEC; ++j) m[q] = max_w(m[q], fabs(R(q, j)));
      m[q] = line_max_input<FMT>(m[q], bad);
    }
    block_max2<W, BLOCK, LPB, NP>(m, red);
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int nq = q == 0 ? n0 : n1;
      if (s >= nq) continue;  // uniform
      // the line maximum is the same in every lane of a wave: the slice
      // constants are computed once, by scalar instructions
      SliceConst<W> kc = slice_const<W>(wave_uniform(m[q]), rho);
      const int ce = plane_exponent<FMT>(kc, rho, flags, t == 0);
      const int pl = (q == 0 ? 0 : n0) + s;
      T* out = S + pl * plane + off0;
      int qs = 0;
      auto emit = [&](auto fastc) {
        constexpr bool FAST = decltype(fastc)::value;
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
          union {
            TV w;
            T e[VEC];
          } pk;
          if constexpr (FAST) {
            const FastSlice fs = fast_slice(kc, rho);
            const float carrier = fast_carrier<FMT>(rho);
            float c[VEC];
#pragma unroll
            for (int u = 0; u < VEC; ++u) {
              float r = R(q, j * VEC + u);
              const float qv = fast_step(r, fs);
              asm volatile("" : "+v"(r));
              R(q, j * VEC + u) = r;
              c[u] = fast_carry<FMT>(qv, carrier);
            }
            pk.w = pack_fast<FMT, VEC>(c);
          } else {
#pragma unroll
            for (int u = 0; u < VEC; ++u) {
              W r = R(q, j * VEC + u);
              W v = (r + kc.sigma) - kc.sigma;
              if (kc.zero) v = W(0);
              W rn = r - v;
              // pinned here: otherwise the residual updates sink below the
              // stores and every v stays live meanwhile
              asm volatile("" : "+v"(rn));
              R(q, j * VEC + u) = rn;
              const float sv = slice_value_f32(v, kc.inv);
              pk.e[u] = PlaneElem<FMT>::make(sv, qscale);
            }
          }
          if constexpr (FMT == kFmtI8) qs = byte_sum(pk.w, qs);
          if (((int64_t)j * BLOCK + t) * VEC < ld) *(TV*)(out + j * step) = pk.w;
        }
      };
      if constexpr (sizeof(W) == 4) {
        // uniform per wave: a wave's lanes hold one line
        if (__builtin_amdgcn_readfirstlane((int)fast_slice(kc, rho).ok))
          emit(std::true_type());
        else
          emit(std::false_type());
      } else {
        emit(std::false_type());
      }
      if constexpr (FMT == kFmtI8) {
        qs = wave_sum(qs);
        if ((threadIdx.x & 63) == 0) atomicAdd(&ssum[pl * LPB + threadIdx.x / BLOCK], qs);
      }
      if (t == 0) E[pl * eplane + line] = ce;
    }
  }
  if constexpr (FMT == kFmtI8) {
    __syncthreads();
    for (int i = threadIdx.x; i < (n0 + n1) * LPB; i += BLOCK * LPB)
      Sg[(i / LPB) * eplane + grp * LPB + i % LPB] =
          ssum[i] - i8_offset(rho) * (BLOCK * EPT * VEC);
  }
}

// Streaming extraction for lines too long for registers: every pass re-reads
// the line and replays the previous slices' sigma steps (R_s depends only on
// x and sigma_1..sigma_{s-1}), so only the per-slice constants are stored.

template <typename W, int BLOCK, int FMT>
__global__ __launch_bounds__(BLOCK) void extract_lines_stream(
    const double* __restrict__ X, int64_t lines, int64_t len, int64_t ldx,
    int rho, int n0, int n1, typename PlaneElem<FMT>::type* __restrict__ S,
    int64_t ld, int64_t plane, int32_t* __restrict__ E, int64_t eplane,
    uint32_t* __restrict__ flags) {
  const float qscale = ldexpf(1.0f, 24 - rho);
  constexpr int NP = Parts<W>::N;
  __shared__ W red[NP * (BLOCK / 64)];
  __shared__ W sig[NP][kMaxSlices];
  __shared__ W inv[NP][kMaxSlices];
  __shared__ int zero[NP][kMaxSlices];
  const int64_t line = xcd_line(blockIdx.x, gridDim.x);
  const bool live = line < lines;
  const double* x = X + line * ldx;
  const int ns = NP == 2 ? max(n0, n1) : n0;
  bool bad = false;

  // Passes 0..ns-1 determine slice constants; pass ns writes every plane.
  for (int s = 0; s <= ns; ++s) {
    W m[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) m[q] = W(0);
    for (int64_t k = threadIdx.x; k < ld; k += BLOCK) {
      double xv = (live && k < len) ? x[k] : 0.0;
      if (s == 0) bad |= !isfinite(xv);
      W p[NP];
      split<W>(xv, p);
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        const int nq = q == 0 ? n0 : n1;
        W r = p[q];
        const int upto = s < nq ? s : nq;
        for (int t = 0; t < upto; ++t) {
          W v = (r + sig[q][t]) - sig[q][t];
          if (zero[q][t]) v = W(0);
          if (s == ns) {
            const int pl = (q == 0 ? 0 : n0) + t;
            S[pl * plane + plane_offset<sizeof(*S)>(line, k, eplane)] =
                PlaneElem<FMT>::make(slice_value_f32(v, inv[q][t]), qscale);
          }
          r = r - v;
        }
        m[q] = max_w(m[q], fabs(r));
      }
    }
    if (s == ns) break;
#pragma unroll
    for (int q = 0; q < NP; ++q) m[q] = line_max_input<FMT>(m[q], bad);
    block_max2<W, BLOCK, 1, NP>(m, red);
    if (threadIdx.x == 0) {
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        const int nq = q == 0 ? n0 : n1;
        if (s >= nq) continue;
        SliceConst<W> kc = slice_const<W>(m[q], rho);
        const int ce = plane_exponent<FMT>(kc, rho, flags, true);
        sig[q][s] = kc.sigma;
        inv[q][s] = kc.inv;
        zero[q][s] = kc.zero;
        E[((q == 0 ? 0 : n0) + s) * eplane + line] = ce;
      }
    }
    __syncthreads();
  }
  if (bad) atomicOr(flags, OZK_FLAG_NONFINITE);
}

// Column extraction without a transposed copy of X.  The columns are cut
// into panels of kGangPW = 16 (a 128-byte row segment of X) and each panel's
// rows into runs of kGangRun; workgroup ("member") m of the panel's gang of
// G = ceil(rows / kGangRun) holds run m of all 16 columns on chip (thread
// t: column t % 16, rows 32 (t / 16) .. +31 of the run; hi parts in
// registers, lo parts in LDS), so X is read once, in whole 128-byte row
// segments, and every plane element is written once.  The arithmetic is extract_lines_reg's; only line maxima
// cross workgroups.
//
// Rounds.  A slice's exponent needs the maximum of the residual over the
// whole column, so each slice costs an exchange between the members.
// Round 0 settles slice 0 of both parts.  Round 1 settles up to three
// slices of a part at once: besides max |R| (slice j), each member sends the
// maxima of the next two residuals under the exponents they can have.  The
// residual after a slice with grid u is at most u / 2 in magnitude, so the
// next exponent is c' = rho + c - 25 unless the column's largest residual
// falls below 2^(rho + c - 25) (then c' <= rho + c - 26): the members send
// max |R_{j+1}| for c_j in {a, a - 1}, a = rho + c_{j-1} - 25, and
// max |R_{j+2}| for the four (c_j, c_{j+1}) pairs that follow (keys
// 0, 1..2, 3..6).  The combined maxima settle slice j exactly; slice j + 1
// when c_j is one of its two candidates, and slice j + 2 likewise.  The
// candidates' residuals are the short-form steps (fast_step) that the
// emission then takes, so a settled slice is the one the slice-by-slice
// procedure gives.  Candidates are taken only where the short form holds
// for them; other columns, and later rounds, settle one slice per part.
// For normally distributed columns the exponents step by -6 or -7
// (rho = 19), so the four hi slices of the high preset take two rounds.
//
// Exchange, per (panel, round): a record of G lines, zeroed before the
// launch (2 parts x 16 columns words a line; in round 1 the hi part sends
// 7 keys a column: 8 x 16 words).
// Member m stores its partial maxima as order keys, which are never 0,
// into line m, then waits until every line is complete and combines them.
// Every word is written once per launch, so a reader that sees a nonzero
// word sees its final value: relaxed agent-scope atomic loads and stores
// suffice (no fences, and no read-modify-write on shared words).  Every
// member settles the same slices (the same combined keys, the same rules),
// so all agree on the next round's record.
//
// Progress: a member's place (panel, m) comes from a ticket taken when it
// starts, so all members of the gangs before the first incomplete one have
// started, and those gangs finish; the incomplete gang's remaining members
// then need only free slots (G <= kGangMaxMembers = 128 workgroups resident
// at once, of the 1024 that 256 CUs hold).  Every wait is bounded all the same: after kGangWaitTicks ticks of
// the 100 MHz real-time counter (0.2 s, or the limit a test set with
// ozk_set_wait_polls) it sets OZK_FLAG_WAIT_TIMEOUT (the slices are then not
// valid) and the member waits no more in later rounds.  Other work that
// holds the CUs for longer (another process, or a persistent GEMM on
// another stream) can keep a gang's members apart that long; the caller
// then repeats the extraction without gangs (ozk_set_gangs).
constexpr int kGangPW = 16;
constexpr int kGangRowsPT = 32;
constexpr int kGangThreads = 256;
constexpr int kGangRun = kGangThreads / kGangPW * kGangRowsPT;  // 512 rows
constexpr int kGangMaxMembers = 128;
constexpr int kGangBatch = 8;  // exchange words a combining thread loads at once
constexpr uint32_t kGangWaitTicks = 20000000u;
constexpr int kGangSpecKeys = 7;        // keys per hi column in round 1
constexpr int kGangWords = 2 * kGangPW;  // words per record line (round 1: x 4)
constexpr int kGangSpecWords = (kGangSpecKeys + 1) * kGangPW;  // 128
constexpr int64_t kGangHeader = 256;    // the ticket word, padded

__host__ __device__ constexpr int gang_members(int64_t ld) {
  return (int)((ld + kGangRun - 1) / kGangRun);
}
// Words per member line in round r, and the word offset of round r's
// records in a panel's (rounds 0 .. r - 1 before it).
__host__ __device__ constexpr int gang_round_words(int r) {
  return r == 1 ? kGangSpecWords : kGangWords;
}
__host__ __device__ constexpr int64_t gang_round_offset(int r, int G) {
  return r == 0 ? 0
                : (int64_t)G * (kGangWords + (r >= 2 ? kGangSpecWords +
                                                           (int64_t)(r - 2) * kGangWords
                                                     : 0));
}
// Word of key k of part q, column col, in a record line of a round whose
// hi part sends nk keys a column (the lo part sends one).
__device__ __forceinline__ int gang_word(int q, int k, int nk, int col) {
  return (q == 0 ? k : nk) * kGangPW + col;
}

// Order key of a partial maximum (a non-negative float or NaN): the key of
// a maximum is the maximum of the keys under fmaxf's rule (NaN only when
// every part is NaN), and no key is 0.
__device__ __forceinline__ uint32_t max_key(float m) {
  return m != m ? 1u : __float_as_uint(m) + 2u;
}
__device__ __forceinline__ float key_max(uint32_t k) {
  return k == 1u ? __builtin_nanf("") : __uint_as_float(k - 2u);
}

// Bounded wait for a nonzero word; 0 (and the flag) once `ticks` ticks of
// the 100 MHz real-time counter have passed without it.
__device__ __forceinline__ uint32_t wait_key(const uint32_t* p, uint32_t* flags,
                                             uint32_t ticks) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    const uint32_t k = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (k) return k;
    if (__builtin_amdgcn_s_memrealtime() - t0 >= ticks) break;
    __builtin_amdgcn_s_sleep(1);
  }
  atomicOr(flags, OZK_FLAG_WAIT_TIMEOUT);
  return 0u;
}

// Bounded wait for the n <= N word pairs base[off + i * stride] (8-byte
// aligned), both words nonzero, with their loads in flight together; false
// (and the flag) on time-out.
template <int N>
__device__ __forceinline__ bool wait_pairs(const uint64_t* base, uint32_t off, uint32_t stride,
                                           uint64_t (&k)[N], int n, uint32_t* flags,
                                           uint32_t ticks) {
  auto whole = [](uint64_t v) { return (uint32_t)v != 0u && (uint32_t)(v >> 32) != 0u; };
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    bool all = true;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (i < n && !whole(k[i]))
        k[i] = __hip_atomic_load(base + off + i * stride, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) all &= i >= n || whole(k[i]);
    if (all) return true;
    if (__builtin_amdgcn_s_memrealtime() - t0 >= ticks) break;
    __builtin_amdgcn_s_sleep(1);
  }
  atomicOr(flags, OZK_FLAG_WAIT_TIMEOUT);
  return false;
}

// The short-form constants of exponent c (fast_slice for a known c).
__device__ __forceinline__ FastSlice fast_slice_c(int c, int rho) {
  SliceConst<float> k;
  k.zero = false;
  k.c = c;
  return fast_slice(k, rho);
}

// INT8: every member adds its sums of q over its rows, per plane pl and
// column, into sums[pl eplane + column] (zeroed before the launch): the
// packed bytes (q + offset) of all kGangRun rows, rows past the column's
// end included (q = 0 there), less offset x kGangRun.  Integer sums, so
// the order of the members' atomic adds does not matter.
// Four waves, up to 128 VGPRs each (four waves per SIMD), with the lo parts
// in LDS: four members per CU, which cover each other's exchange waits.
template <int FMT>
__global__ __launch_bounds__(kGangThreads) __attribute__((amdgpu_waves_per_eu(4))) void extract_cols_gang(
    const double* __restrict__ X, int64_t K, int64_t M, int64_t ldx, int rho, int n0,
    int n1, typename PlaneElem<FMT>::type* __restrict__ S, int64_t ld, int64_t plane,
    int32_t* __restrict__ E, int64_t eplane, uint32_t* __restrict__ flags,
    uint32_t* __restrict__ rec, uint32_t* __restrict__ ticket, int G, uint32_t wait_ticks,
    int32_t* __restrict__ sums) {
  typedef typename PlaneElem<FMT>::type T;
  constexpr int NP = 2, R = kGangRowsPT, NKS = kGangSpecKeys;
  constexpr int NWORD = R * (int)sizeof(T) / 4;  // plane words of a thread's rows
  constexpr int kMaxWords = kGangSpecWords;      // 128
  const float qscale = ldexpf(1.0f, 24 - rho);
  // per-workgroup key maxima of the round, then all members' (order keys,
  // LDS atomic max)
  __shared__ uint32_t wkey[kMaxWords], wall[kMaxWords];
  // per (part, column): slices settled so far, the last settled exponent,
  // whether round 1 may take candidates after it, this round's count, and
  // per slice settled in the round its constants (short form: s, u; plain
  // form: sigma, inv) and form (1: short form; 2: zero slice; 0: plain)
  struct GangCol {
    int done, c, spec, d;
    float a[3], b[3];
    int mode[3], pad;
  };
  __shared__ GangCol gc[NP][kGangPW];
  __shared__ uint32_t place;
  __shared__ int gave_up, more;
  __shared__ int ssum[FMT == kFmtI8 ? kMaxPlanes * kGangPW : 1];
  const int t = threadIdx.x, lane = t & 63;
  if constexpr (FMT == kFmtI8) {
    for (int i = t; i < kMaxPlanes * kGangPW; i += kGangThreads) ssum[i] = 0;
  }
  for (int i = t; i < kMaxWords; i += kGangThreads) wkey[i] = wall[i] = 0u;
  if (t < NP * kGangPW) {
    gc[t / kGangPW][t % kGangPW].done = 0;
    gc[t / kGangPW][t % kGangPW].spec = 0;
  }
  if (t == 0) {
    place = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    gave_up = 0;
  }
  __syncthreads();
  const int64_t panel = place / (uint32_t)G;
  const int member = (int)(place % (uint32_t)G);
  const int ns = max(n0, n1);
  uint32_t* const my = rec + panel * gang_round_offset(ns, G);
  const int col = t % kGangPW;
  const int64_t r0 = (int64_t)member * kGangRun + R * (t / kGangPW);
  const int64_t line = panel * kGangPW + col;  // the thread's column

  // The one read: hi parts in registers, lo parts in LDS (32 KiB): four
  // members per CU.  Every load reads an address inside X (a row past the
  // last reads row 0, a column past the last column 0) and its value is
  // replaced by zero afterwards, so no branch separates the R loads: all
  // of them are in flight at once.
  float Rh[R];
  __shared__ float lo_s[R][kGangThreads];
  bool bad = false;
  {
    double v[R];
    const bool cok = line < M;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t row = r0 + i;
      const bool ok = cok && row < K;
      const double d = X[(ok ? row : 0) * ldx + (ok ? line : 0)];
      v[i] = ok ? d : 0.0;
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      bad |= !isfinite(v[i]);
      float p[NP];
      split<float>(v[i], p);
      // pinned where made, so the doubles are not held until the check
      asm volatile("" : "+v"(p[0]), "+v"(p[1]));
      Rh[i] = p[0];
      lo_s[i][t] = p[1];
    }
  }
  if (bad) atomicOr(flags, OZK_FLAG_NONFINITE);

  // Lanes col, col + 16, col + 32, col + 48 of a wave hold the same column.
  auto wave_col_max = [&](float m) {
    m = max_w(m, __shfl_xor(m, 16));
    return max_w(m, __shfl_xor(m, 32));
  };
  const bool store = r0 < ld;  // the R rows lie in one padded unit
  for (int r = 0;; ++r) {
    const int words = gang_round_words(r);
    const int nk = r == 1 ? NKS : 1;  // keys per hi column
    uint32_t* const rs = my + gang_round_offset(r, G);  // this round's record
    // 1. The thread's partial maxima, reduced over the wave's lanes of the
    // column, then over the waves by LDS atomic max.  Candidates for the
    // hi part only (the lo part has one slice in the presets).
    auto publish_local = [&](int q, int k, float m) {
      m = wave_col_max(m);
      if (lane < kGangPW) atomicMax(&wkey[gang_word(q, k, nk, col)], max_key(m));
    };
    {
      const int left = n0 - gc[0][col].done;
      if (left > 0) {
        const int depth = (r == 1 && gc[0][col].spec) ? min(left, 3) : 1;
        float m0 = 0.0f;
#pragma unroll
        for (int i = 0; i < R; ++i) m0 = max_w(m0, fabsf(Rh[i]));
        publish_local(0, 0, line_max_input<FMT>(m0, bad));
        if (depth > 1) {
          // c_j in {a, a - 1}; then c_{j+1} in {rho + c_j - 25, that - 1}
          const int a = rho + gc[0][col].c - 25;
#pragma unroll 1
          for (int x = 0; x < 2; ++x) {
            const FastSlice f1 = fast_slice_c(a - x, rho);
            const FastSlice f2a = fast_slice_c(rho + a - x - 25, rho);
            const FastSlice f2b = fast_slice_c(rho + a - x - 26, rho);
            float m1 = 0.0f, m2a = 0.0f, m2b = 0.0f;
#pragma unroll
            for (int i = 0; i < R; ++i) {
              float r1 = Rh[i];
              fast_step(r1, f1);
              m1 = max_w(m1, fabsf(r1));
              float r2 = r1, r3 = r1;
              fast_step(r2, f2a);
              fast_step(r3, f2b);
              m2a = max_w(m2a, fabsf(r2));
              m2b = max_w(m2b, fabsf(r3));
            }
            publish_local(0, 1 + x, m1);
            if (depth > 2) {
              publish_local(0, 3 + 2 * x, m2a);
              publish_local(0, 4 + 2 * x, m2b);
            }
          }
        }
      }
      if (n1 - gc[1][col].done > 0) {
        float m0 = 0.0f;
#pragma unroll
        for (int i = 0; i < R; ++i) m0 = max_w(m0, fabsf(lo_s[i][t]));
        publish_local(1, 0, line_max_input<FMT>(m0, bad));
      }
    }
    __syncthreads();
    // 2. Publish (words never 0: keys unused this round are max_key(0)).
    if (t < words) {
      const uint32_t k = wkey[t];
      __hip_atomic_store(rs + member * words + t, k ? k : max_key(0.0f), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    // 3. Combine: thread t waits for word pair w = t % (words / 2) of
    // members t / (words / 2), that + ng, ... (kGangBatch 8-byte loads in
    // flight together), then the maxima meet in LDS.
    {
      const int pairs = words / 2;
      const int ng = kGangThreads / pairs;  // 16 groups, or 4 in round 1
      const int grp = t / pairs, w = t % pairs;
      if (grp < G) {
        const int n = (G - 1 - grp) / ng + 1;  // members grp, grp + ng, ... < G
        uint32_t k0 = 0u, k1 = 0u;
        for (int b = 0; b < n; b += kGangBatch) {
          uint64_t kk[kGangBatch];
#pragma unroll
          for (int i = 0; i < kGangBatch; ++i) kk[i] = 0u;
          if (!gave_up &&
              !wait_pairs((const uint64_t*)rs, (uint32_t)((grp + b * ng) * pairs + w),
                          (uint32_t)(ng * pairs), kk, min(n - b, kGangBatch), flags,
                          wait_ticks))
            gave_up = 1;
#pragma unroll
          for (int i = 0; i < kGangBatch; ++i) {
            k0 = max(k0, (uint32_t)kk[i]);
            k1 = max(k1, (uint32_t)(kk[i] >> 32));
          }
        }
        atomicMax(&wall[2 * w], k0);
        atomicMax(&wall[2 * w + 1], k1);
      }
    }
    __syncthreads();
    if (t == 0) more = 0;
    // 4. Settle: one thread per (part, column).
    if (t < NP * kGangPW) {
      const int q = t / kGangPW, cl = t % kGangPW;
      GangCol& g = gc[q][cl];
      auto key = [&](int k) { return key_max(wall[gang_word(q, k, nk, cl)]); };
      const int nq = q == 0 ? n0 : n1;
      const int done = g.done;
      const int left = nq - done;
      int d = 0;
      if (left > 0) {
        const int depth = (r == 1 && q == 0 && g.spec) ? min(left, 3) : 1;
        const int a = rho + g.c - 25;
        int kidx = 0;   // key of the slice at hand
        int cnext = a;  // largest candidate exponent of the next slice
        for (int j = 0; j < depth; ++j) {
          SliceConst<float> kc = slice_const<float>(key(kidx), rho);
          const int cexact = kc.c;
          const int ce = plane_exponent<FMT>(kc, rho, flags, member == 0);
          const int pl = (q == 0 ? 0 : n0) + done + j;
          if (member == 0) E[pl * eplane + panel * kGangPW + cl] = ce;
          const FastSlice fs = fast_slice(kc, rho);
          g.a[j] = fs.ok ? fs.s : kc.sigma;
          g.b[j] = fs.ok ? fs.u : kc.inv;
          g.mode[j] = fs.ok ? 1 : (kc.zero ? 2 : 0);
          g.c = cexact;
          g.spec = fs.ok;
          ++d;
          if (j + 1 >= depth || !fs.ok) break;
          // the next slice's key, if this exponent is one of its candidates
          const int x = cnext - cexact;
          if (x != 0 && x != 1) break;
          kidx = j == 0 ? 1 + x : 3 + 2 * (kidx - 1) + x;
          cnext = rho + cexact - 25;
        }
        if (done + d < nq) more = 1;
      }
      g.d = d;
    }
    __syncthreads();
    // 5. Emit the settled slices.
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const GangCol& g = gc[q][col];
      const int d = g.d, done = g.done;
      for (int j = 0; j < d; ++j) {
        const int pl = (q == 0 ? 0 : n0) + done + j;
        const int mode = g.mode[j];
        const float ka = g.a[j], kb = g.b[j];
        uint32_t w[NWORD];
        if (mode == 1) {  // every lane, but for exceptional columns
          const FastSlice fs = {ka, kb, true};
          const float carrier = fast_carrier<FMT>(rho);
          float cv[R];
#pragma unroll
          for (int i = 0; i < R; ++i) {
            float rv = q == 0 ? Rh[i] : lo_s[i][t];
            const float qv = fast_step(rv, fs);
            asm volatile("" : "+v"(rv));  // as in extract_lines_reg
            if (q == 0) Rh[i] = rv; else lo_s[i][t] = rv;
            cv[i] = fast_carry<FMT>(qv, carrier);
          }
          if constexpr (FMT == kFmtI8) {
#pragma unroll
            for (int u = 0; u < NWORD; ++u)
              w[u] = pack_low_bytes(cv[4 * u], cv[4 * u + 1], cv[4 * u + 2], cv[4 * u + 3]);
          } else {
#pragma unroll
            for (int u = 0; u < NWORD; ++u) w[u] = pack_high_halves(cv[2 * u], cv[2 * u + 1]);
          }
        } else {
          const bool zero = mode == 2;
          union {
            uint32_t w[NWORD];
            T e[R];
          } pk;
#pragma unroll
          for (int i = 0; i < R; ++i) {
            const float rv = q == 0 ? Rh[i] : lo_s[i][t];
            float vv = (rv + ka) - ka;
            if (zero) vv = 0.0f;
            float rn = rv - vv;
            asm volatile("" : "+v"(rn));  // as in extract_lines_reg
            if (q == 0) Rh[i] = rn; else lo_s[i][t] = rn;
            const float sv = slice_value_f32(vv, kb);
            pk.e[i] = PlaneElem<FMT>::make(sv, qscale);
          }
#pragma unroll
          for (int u = 0; u < NWORD; ++u) w[u] = pk.w[u];
        }
        if (store) {
          // 16-byte units of the chunk-major layout (8 or 16 rows each)
          constexpr int UR = 16 / (int)sizeof(T);
#pragma unroll
          for (int u = 0; u < NWORD / 4; ++u)
            *(uint4*)(S + pl * plane + plane_offset<sizeof(T)>(line, r0 + u * UR, eplane)) =
                make_uint4(w[4 * u], w[4 * u + 1], w[4 * u + 2], w[4 * u + 3]);
        }
        if constexpr (FMT == kFmtI8) {
          int qs = 0;
#pragma unroll
          for (int u = 0; u < NWORD; ++u) qs = byte_sum(w[u], qs);
          qs += __shfl_xor(qs, 16);
          qs += __shfl_xor(qs, 32);
          if (lane < kGangPW) atomicAdd(&ssum[pl * kGangPW + col], qs);
        }
      }
    }
    const int again = more;
    __syncthreads();  // the settled counts and constants are read; reset for the next round
    if (t < NP * kGangPW) gc[t / kGangPW][t % kGangPW].done += gc[t / kGangPW][t % kGangPW].d;
    for (int i = t; i < kMaxWords; i += kGangThreads) wkey[i] = wall[i] = 0u;
    if (!again) break;
    __syncthreads();
  }
  if constexpr (FMT == kFmtI8) {
    __syncthreads();
    for (int i = t; i < (n0 + n1) * kGangPW; i += kGangThreads) {
      const int64_t c = panel * kGangPW + i % kGangPW;
      if (c < M) atomicAdd(&sums[(i / kGangPW) * eplane + c], ssum[i] - i8_offset(rho) * kGangRun);
    }
  }
}

// Column extraction without a transposed copy of X and without exchanges
// between workgroups, for columns of up to 4096 rows: workgroup b holds a
// panel of kPanelCols = 2 whole columns of up to 256 RPT rows on chip
// (thread t: column t % 2, rows RPT (t / 2) .. + RPT - 1, hi and lo parts
// in registers), so every line maximum is a reduction inside the
// workgroup, X is read once and every plane element is written once.  Lanes 2 k and 2 k + 1 of a load read one
// 16-byte row segment; the panels that share X's 128-byte lines run on one
// XCD (xcd_line), whose L2 serves the segments of a line to all of them.
// The arithmetic is extract_lines_reg's (the short form of the slice step
// where it holds).  INT8: the line sums are complete in the workgroup.
constexpr int kPanelCols = 2;
constexpr int kPanelThreads = 512;
constexpr int kPanelGroups = kPanelThreads / kPanelCols;  // 256 row groups

template <int FMT, int RPT>
__global__ __launch_bounds__(kPanelThreads) __attribute__((amdgpu_waves_per_eu(4))) void extract_cols_panel(
    const double* __restrict__ X, int64_t K, int64_t M, int64_t ldx, int rho, int n0, int n1,
    typename PlaneElem<FMT>::type* __restrict__ S, int64_t ld, int64_t plane,
    int32_t* __restrict__ E, int64_t eplane, uint32_t* __restrict__ flags,
    int32_t* __restrict__ Sg) {
  typedef typename PlaneElem<FMT>::type T;
  constexpr int NP = 2, NW = kPanelThreads / 64;
  constexpr int BYTES = RPT * (int)sizeof(T);  // plane bytes of a thread's rows
  constexpr int NWORD = (BYTES + 3) / 4;
  const float qscale = ldexpf(1.0f, 24 - rho);
  __shared__ float red[NW][NP][kPanelCols];
  __shared__ int ssum[FMT == kFmtI8 ? kMaxPlanes * kPanelCols : 1];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  if constexpr (FMT == kFmtI8) {
    for (int i = t; i < kMaxPlanes * kPanelCols; i += kPanelThreads) ssum[i] = 0;
  }
  const int64_t panel = xcd_line(blockIdx.x, gridDim.x);
  const int cl = t % kPanelCols;
  const int64_t line = panel * kPanelCols + cl;  // the thread's column
  const int64_t r0 = (int64_t)RPT * (t / kPanelCols);

  // The one read.  Every load reads an address inside X (a row past the
  // last reads row 0, a column past the last column 0) and its value is
  // replaced by zero afterwards, so no branch separates the RPT loads.
  float Rr[NP][RPT];
  bool bad = false;
  {
    const bool cok = line < M;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int64_t row = r0 + i;
      const bool ok = cok && row < K;
      const double d = X[(ok ? row : 0) * ldx + (ok ? line : 0)];
      const double v = ok ? d : 0.0;
      bad |= !isfinite(v);
      float p[NP];
      split<float>(v, p);
      Rr[0][i] = p[0];
      Rr[1][i] = p[1];
    }
  }
  if (bad) atomicOr(flags, OZK_FLAG_NONFINITE);

  const bool store = r0 < ld;
  const int ns = max(n0, n1);
  for (int s = 0; s < ns; ++s) {
    // line maxima: the thread, the wave's lanes of the column, the waves
    float m[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      m[q] = 0.0f;
#pragma unroll
      for (int i = 0; i < RPT; ++i) m[q] = max_w(m[q], fabsf(Rr[q][i]));
      m[q] = line_max_input<FMT>(m[q], bad);
#pragma unroll
      for (int off = kPanelCols; off < 64; off <<= 1) m[q] = max_w(m[q], __shfl_xor(m[q], off));
    }
    __syncthreads();  // the previous slice's readers of red are done
    if (lane < kPanelCols) {
      red[wave][0][lane] = m[0];
      red[wave][1][lane] = m[1];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int nq = q == 0 ? n0 : n1;
      if (s >= nq) continue;  // uniform
      float mm = red[0][q][cl];
#pragma unroll
      for (int w = 1; w < NW; ++w) mm = max_w(mm, red[w][q][cl]);
      SliceConst<float> kc = slice_const<float>(mm, rho);
      const int ce = plane_exponent<FMT>(kc, rho, flags, t < kPanelCols);
      const int pl = (q == 0 ? 0 : n0) + s;
      uint32_t w[NWORD];
      const FastSlice fs = fast_slice(kc, rho);
      if (fs.ok) {  // every lane, but for exceptional columns
        const float carrier = fast_carrier<FMT>(rho);
        float cv[RPT];
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
          float rv = Rr[q][i];
          const float qv = fast_step(rv, fs);
          asm volatile("" : "+v"(rv));  // as in extract_lines_reg
          Rr[q][i] = rv;
          cv[i] = fast_carry<FMT>(qv, carrier);
        }
        if constexpr (FMT == kFmtI8) {
#pragma unroll
          for (int u = 0; u < NWORD; ++u)
            w[u] = pack_low_bytes(cv[4 * u], cv[(4 * u + 1) % RPT], cv[(4 * u + 2) % RPT],
                                  cv[(4 * u + 3) % RPT]);
        } else {
#pragma unroll
          for (int u = 0; u < NWORD; ++u) w[u] = pack_high_halves(cv[2 * u], cv[2 * u + 1]);
        }
      } else {
        union {
          uint32_t w[NWORD];
          T e[NWORD * 4 / sizeof(T)];
        } pk;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
          const float rv = Rr[q][i];
          float vv = (rv + kc.sigma) - kc.sigma;
          if (kc.zero) vv = 0.0f;
          float rn = rv - vv;
          asm volatile("" : "+v"(rn));  // as in extract_lines_reg
          Rr[q][i] = rn;
          const float sv = slice_value_f32(vv, kc.inv);
          pk.e[i] = PlaneElem<FMT>::make(sv, qscale);
        }
#pragma unroll
        for (int u = 0; u < NWORD; ++u) w[u] = pk.w[u];
      }
      if (store) {
        T* out = S + pl * plane;
        if constexpr (BYTES >= 16) {
          // whole 16-byte units of the chunk-major layout
#pragma unroll
          for (int u = 0; u < BYTES / 16; ++u)
            *(uint4*)(out + plane_offset<sizeof(T)>(line, r0 + u * (16 / (int)sizeof(T)),
                                                    eplane)) =
                make_uint4(w[4 * u], w[4 * u + 1], w[4 * u + 2], w[4 * u + 3]);
        } else if constexpr (BYTES == 8) {
          *(uint2*)(out + plane_offset<sizeof(T)>(line, r0, eplane)) = make_uint2(w[0], w[1]);
        } else {
          *(uint32_t*)(out + plane_offset<sizeof(T)>(line, r0, eplane)) = w[0];
        }
      }
      if constexpr (FMT == kFmtI8) {
        int qs = 0;
#pragma unroll
        for (int u = 0; u < NWORD; ++u) qs = byte_sum(w[u], qs);
#pragma unroll
        for (int off = kPanelCols; off < 64; off <<= 1) qs += __shfl_xor(qs, off);
        if (lane < kPanelCols) atomicAdd(&ssum[pl * kPanelCols + cl], qs);
      }
      if (t < kPanelCols) E[pl * eplane + line] = ce;
    }
  }
  if constexpr (FMT == kFmtI8) {
    __syncthreads();
    for (int i = t; i < (n0 + n1) * kPanelCols; i += kPanelThreads)
      Sg[(i / kPanelCols) * eplane + panel * kPanelCols + i % kPanelCols] =
          ssum[i] - i8_offset(rho) * (kPanelGroups * RPT);
  }
}

// Row extraction of lines longer than one workgroup holds (FP32 path,
// padded length 32769 .. kRowRun * kRowMaxMembers): each line is cut into
// runs of kRowRun elements, one per workgroup ("member") of the line's gang
// of G = ceil(ld / kRowRun), which holds its run on chip with
// extract_lines_reg's layout (thread t: elements base + (512 j + t) * 4 + v;
// hi parts in registers, lo parts in LDS) and arithmetic.  Per slice the members exchange the run maxima of both
// parts, as extract_cols_gang does: member m stores its two order keys
// into words 2 m, 2 m + 1 of the (line, slice) record (128 bytes, zeroed
// before the launch), then every member waits for all 2 G words.  Places
// come from a ticket, and every wait is bounded, as for the column gangs.
constexpr int kRowThreads = 512, kRowEPT = 8, kRowVEC = 4;
constexpr int kRowRun = kRowThreads * kRowEPT * kRowVEC;  // 16384 elements
constexpr int kRowMaxMembers = 16;
constexpr int64_t kRowRecBytes = 8 * kRowMaxMembers;  // two keys per member

// INT8: every member adds its run's sums of q per plane into
// sums[pl eplane + line] (zeroed before the launch): the packed bytes of its
// run, less offset x kRowRun, as in extract_lines_reg.
template <int FMT, bool VEC>
__global__ __launch_bounds__(kRowThreads) void extract_lines_gang(
    const double* __restrict__ X, int64_t lines, int64_t len, int64_t ldx, int rho, int n0,
    int n1,
    typename PlaneElem<FMT>::type* __restrict__ S, int64_t ld, int64_t plane,
    int32_t* __restrict__ E, int64_t eplane, uint32_t* __restrict__ flags,
    uint32_t* __restrict__ rec, uint32_t* __restrict__ ticket, int G, uint32_t wait_ticks,
    int32_t* __restrict__ sums) {
  typedef typename PlaneElem<FMT>::type T;
  typedef typename PlaneVec<FMT, kRowVEC>::type TV;
  constexpr int NP = 2, EPT = kRowEPT, V = kRowVEC;
  constexpr int kPer = kChunkBytes / (int)sizeof(T);
  static_assert(kRowRun % kPer == 0 && (kRowThreads * V) % kPer == 0, "whole chunks");
  constexpr int64_t kWords = kRowRecBytes / 4;
  const float qscale = ldexpf(1.0f, 24 - rho);
  __shared__ float red[NP * (kRowThreads / 64)];
  __shared__ uint32_t comb[2 * kRowMaxMembers];
  __shared__ uint32_t place;
  __shared__ int gave_up;
  __shared__ int ssum[FMT == kFmtI8 ? kMaxPlanes : 1];
  const int t = threadIdx.x;
  if constexpr (FMT == kFmtI8) {
    if (t < kMaxPlanes) ssum[t] = 0;
  }
  if (t == 0) {
    place = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    gave_up = 0;
  }
  __syncthreads();
  // the grid holds exactly G workgroups per padded line, so every place is a
  // member; the padding lines (no reads) store zero slices
  const int64_t line = place / (uint32_t)G;
  const int member = (int)(place % (uint32_t)G);
  const bool live = line < lines;
  const int ns = max(n0, n1);
  const int64_t base = (int64_t)member * kRowRun;
  const double* x = X + (live ? line : 0) * ldx;
  // base is a whole number of chunks, so as in extract_lines_reg the
  // in-chunk position is fixed per thread and j advances whole chunks
  const int64_t off0 = plane_offset<sizeof(T)>(line, base + (int64_t)t * V, eplane);
  const int64_t step = (int64_t)(kRowThreads * V / kPer) * eplane * kPer;
  uint32_t* const my = rec + line * ns * kWords;

  // The run's hi parts stay in registers and its lo parts in LDS (64 KiB),
  // so two workgroups fit on a CU.
  __shared__ float lo[EPT * V][kRowThreads];
  float hi[EPT * V];
  auto R = [&](int q, int i) -> float& { return q == 0 ? hi[i] : lo[i][t]; };
  bool bad = false;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int64_t k0 = base + ((int64_t)j * kRowThreads + t) * V;
    double v[V];
    if (VEC && live && k0 + V <= len) {
#pragma unroll
      for (int u = 0; u < V; u += 2) {
        const double2 d = *(const double2*)(x + k0 + u);
        v[u] = d.x;
        v[u + 1] = d.y;
      }
    } else {
#pragma unroll
      for (int u = 0; u < V; ++u) v[u] = live && k0 + u < len ? x[k0 + u] : 0.0;
    }
#pragma unroll
    for (int u = 0; u < V; ++u) {
      bad |= !isfinite(v[u]);
      float p[NP];
      split<float>(v[u], p);
#pragma unroll
      for (int q = 0; q < NP; ++q) R(q, j * V + u) = p[q];
    }
  }
  if (bad) atomicOr(flags, OZK_FLAG_NONFINITE);

  for (int s = 0; s < ns; ++s) {
    uint32_t* const rs = my + s * kWords;  // this slice's record
    float m[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      m[q] = 0.0f;
#pragma unroll
      for (int j = 0; j < EPT * V; ++j) m[q] = max_w(m[q], fabsf(R(q, j)));
      m[q] = line_max_input<FMT>(m[q], bad);
    }
    block_max2<float, kRowThreads, 1, NP>(m, red);  // the run's maxima
    if (t < NP)
      __hip_atomic_store(rs + 2 * member + t, max_key(m[t]), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (t < 2 * G) {  // every member's maxima
      uint32_t k = 0u;
      if (!gave_up) {
        k = wait_key(rs + t, flags, wait_ticks);
        if (!k) gave_up = 1;
      }
      comb[t] = k;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      uint32_t kk = 0u;
      for (int mb = 0; mb < G; ++mb) kk = max(kk, comb[2 * mb + q]);
      m[q] = key_max(kk);
    }
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int nq = q == 0 ? n0 : n1;
      if (s >= nq) continue;  // uniform
      SliceConst<float> kc = slice_const<float>(m[q], rho);
      const int ce = plane_exponent<FMT>(kc, rho, flags, t == 0 && member == 0);
      const int pl = (q == 0 ? 0 : n0) + s;
      T* out = S + pl * plane + off0;
      int qs = 0;
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        union {
          TV w;
          T e[V];
        } pk;
#pragma unroll
        for (int u = 0; u < V; ++u) {
          const float r = R(q, j * V + u);
          float v = (r + kc.sigma) - kc.sigma;
          if (kc.zero) v = 0.0f;
          float rn = r - v;
          asm volatile("" : "+v"(rn));  // as in extract_lines_reg
          R(q, j * V + u) = rn;
          const float sv = slice_value_f32(v, kc.inv);
          pk.e[u] = PlaneElem<FMT>::make(sv, qscale);
        }
        if constexpr (FMT == kFmtI8) qs = byte_sum(pk.w, qs);
        if (base + ((int64_t)j * kRowThreads + t) * V < ld) *(TV*)(out + j * step) = pk.w;
      }
      if constexpr (FMT == kFmtI8) {
        qs = wave_sum(qs);
        if ((t & 63) == 0) atomicAdd(&ssum[pl], qs);
      }
      if (t == 0 && member == 0) E[pl * eplane + line] = ce;
    }
  }
  if constexpr (FMT == kFmtI8) {
    __syncthreads();
    if (t < n0 + n1 && live)
      atomicAdd(&sums[(int64_t)t * eplane + line], ssum[t] - i8_offset(rho) * kRowRun);
  }
}

__global__ void zero_i32_kernel(int32_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

__global__ void zero_u32x4_kernel(uint4* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// X (rows x cols, ldx) -> XT (cols x rows, contiguous) through LDS tiles of
// 128 rows x 64 columns: each wave reads 512 contiguous bytes of a row of X
// and writes 512 contiguous bytes of a row of XT.
__global__ __launch_bounds__(512) void transpose_f64(
    const double* __restrict__ X, int64_t rows, int64_t cols, int64_t ldx,
    double* __restrict__ XT) {
  __shared__ double tile[128][65];
  const int64_t r0 = (int64_t)blockIdx.y * 128, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // ty in [0, 8)
  // Interior tiles skip the bounds checks: with them the compiler no longer
  // issues the 16 loads back to back (18% slower at 8192^2).
  const bool full = r0 + 128 <= rows && c0 + 64 <= cols;
  if (full) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int rr = ty + 8 * i;
      tile[rr][tx] = X[(r0 + rr) * ldx + c0 + tx];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int rr = ty + 8 * i;
      const int64_t r = r0 + rr, c = c0 + tx;
      tile[rr][tx] = (r < rows && c < cols) ? X[r * ldx + c] : 0.0;
    }
  }
  __syncthreads();
  if (full) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int cc = ty + 8 * i;
      double* o = XT + (c0 + cc) * rows + r0;
      o[tx] = tile[tx][cc];
      o[64 + tx] = tile[64 + tx][cc];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int cc = ty + 8 * i;
      const int64_t c = c0 + cc;
      if (c < cols) {
        if (r0 + tx < rows) XT[c * rows + r0 + tx] = tile[tx][cc];
        if (r0 + 64 + tx < rows) XT[c * rows + r0 + 64 + tx] = tile[64 + tx][cc];
      }
    }
  }
}

__global__ void check_finite_kernel(const double* __restrict__ X, int64_t rows,
                                    int64_t cols, int64_t ld,
                                    uint32_t* __restrict__ flags) {
  const int64_t total = rows * cols;
  bool bad = false;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols, c = i - r * cols;
    bad |= !isfinite(X[r * ld + c]);
  }
  if (bad) atomicOr(flags, OZK_FLAG_NONFINITE);
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v) { *p = v; }

// INT8 line sums read back from stored planes (the streaming path): 64
// lines per workgroup, four threads per line, each summing one 16-byte unit
// of every chunk; the stored values are q + off.
__global__ __launch_bounds__(256) void i8_plane_sums_kernel(const int8_t* __restrict__ S,
                                                            int64_t lp, int64_t ld, int off,
                                                            int32_t* __restrict__ sums) {
  const int t = threadIdx.x;
  const int64_t pl = blockIdx.y, line = (int64_t)blockIdx.x * 64 + t / 4;
  const int8_t* base = S + pl * lp * ld + line * kChunkBytes + 16 * (t % 4);
  int v = 0;
  for (int64_t c = 0; c < ld / kChunkBytes; ++c) {
    const int4 w = *(const int4*)(base + c * lp * kChunkBytes);
    const int ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v += (int)(int8_t)ws[i] + (int)(int8_t)(ws[i] >> 8) + (int)(int8_t)(ws[i] >> 16) +
           (ws[i] >> 24);
  }
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  if (t % 4 == 0) sums[pl * lp + line] = v - (int)ld * off;
}

// ---------------------------------------------------------------- launchers

// FP32 lines longer than one workgroup holds and at most
// kRowRun * kRowMaxMembers long run on row gangs.
static bool gang_rows(int64_t len) {
  const int64_t ld = round_up(len, kKPad);
  return ld > 32768 && ld <= (int64_t)kRowRun * kRowMaxMembers && gangs_enabled();
}

// Ticket and exchange records (zeroed per launch).
static size_t row_gang_bytes(int64_t lines, int64_t, int nslices) {
  return (size_t)round_up(kGangHeader + round_up(lines, kLinePad) * nslices * kRowRecBytes, 256);
}

template <int FMT>
static int launch_rows_gang(const double* X, int64_t lines, int64_t len, int64_t ldx,
                            int rho, int n0, int n1, void* Sv, int32_t* E, uint32_t* flags,
                            void* ws, size_t wsb, hipStream_t st, int32_t* Sg) {
  typedef typename PlaneElem<FMT>::type T;
  const int ns = n0 > n1 ? n0 : n1;
  const size_t need = row_gang_bytes(lines, len, ns);
  if (wsb < need || !ws) {
    set_error("extract: workspace of %zu bytes needed, %zu given", need, wsb);
    return OZK_ERR_WORKSPACE;
  }
  const int64_t ld = round_up(len, kKPad), lp = round_up(lines, kLinePad);
  const int64_t plane = lp * ld;
  const int G = (int)((ld + kRowRun - 1) / kRowRun);
  // the ticket, the exchange records and the INT8 line sums start at zero
  const int64_t n16 = (int64_t)need / 16;
  hipLaunchKernelGGL(zero_u32x4_kernel,
                     dim3((unsigned)((n16 + 255) / 256 < 1024 ? (n16 + 255) / 256 : 1024)),
                     dim3(256), 0, st, (uint4*)ws, n16);
  OZK_LAUNCH_CHECK();
  if constexpr (FMT == kFmtI8) {
    const int64_t ns32 = (int64_t)(n0 + n1) * lp;
    hipLaunchKernelGGL(zero_i32_kernel, dim3((unsigned)((ns32 + 255) / 256 < 1024 ? (ns32 + 255) / 256 : 1024)),
                       dim3(256), 0, st, Sg, ns32);
    OZK_LAUNCH_CHECK();
  }
  uint32_t* ticket = (uint32_t*)ws;
  uint32_t* rec = (uint32_t*)((char*)ws + kGangHeader);
  const dim3 grid((unsigned)(lp * G));
  const uint32_t wait_ticks = wait_polls(kGangWaitTicks);
  if (((uintptr_t)X % 16 == 0) && (ldx % 2 == 0))
    hipLaunchKernelGGL((extract_lines_gang<FMT, true>), grid, dim3(kRowThreads), 0, st, X,
                       lines, len, ldx, rho, n0, n1, (T*)Sv, ld, plane, E, lp, flags, rec,
                       ticket, G, wait_ticks, Sg);
  else
    hipLaunchKernelGGL((extract_lines_gang<FMT, false>), grid, dim3(kRowThreads), 0, st, X,
                       lines, len, ldx, rho, n0, n1, (T*)Sv, ld, plane, E, lp, flags, rec,
                       ticket, G, wait_ticks, Sg);
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

template <typename W, int FMT>
static int launch_lines(const double* X, int64_t lines, int64_t len,
                        int64_t ldx, int rho, int n0, int n1, void* Sv,
                        int32_t* E, uint32_t* flags, void* ws, size_t wsb, hipStream_t st,
                        int32_t* Sg) {
  if constexpr (sizeof(W) == 4) {
    if (gang_rows(len) && lines > 0)
      return launch_rows_gang<FMT>(X, lines, len, ldx, rho, n0, n1, Sv, E, flags, ws, wsb,
                                   st, Sg);
  }
  typedef typename PlaneElem<FMT>::type T;
  T* S = (T*)Sv;
  const int64_t ld = round_up(len, kKPad);
  const int64_t lp = round_up(lines, kLinePad);
  const int64_t plane = lp * ld;
  const dim3 grid((unsigned)lp);
  // 16-byte loads need 16-byte aligned line starts
  const int vec_ok = ((uintptr_t)X % 16 == 0) && (ldx % 2 == 0);
#define OZK_REG(B, EPT, LPB, V)                                                        \
  hipLaunchKernelGGL((extract_lines_reg<W, B, EPT, LPB, FMT, V>),                      \
                     dim3((unsigned)(lp / LPB)), dim3(B * LPB), 0, st, X, lines, len, ldx, \
                     vec_ok && len % V == 0, rho, n0, n1, S, ld, plane, E, lp, flags, Sg)
  // Shapes measured per line-length bucket (one or two lines per workgroup
  // so that several workgroups share a CU and overlap loads with stores).
  if (ld <= 256) {
    OZK_REG(64, 2, 4, 2);
  } else if (ld <= 1024) {
    OZK_REG(128, 4, 1, 2);
  } else if (ld <= 2048) {
    OZK_REG(128, 8, 1, 2);
  } else if (ld <= 4096) {
    OZK_REG(256, 8, 2, 2);
  } else if (ld <= 8192) {
    OZK_REG(256, 8, 1, 4);
  } else if (ld <= 16384) {
    OZK_REG(512, 16, 1, 2);
  } else {
    bool done = false;
    if constexpr (sizeof(W) == 4) {  // FP32 parts: 32768 elements still fit
      if (ld <= 32768) {
        OZK_REG(512, 16, 1, 4);
        done = true;
      }
    }
    if (!done) {  // FP64 lines, and FP32 lines longer than the row gangs take
      hipLaunchKernelGGL((extract_lines_stream<W, 1024, FMT>), grid, dim3(1024),
                         0, st, X, lines, len, ldx, rho, n0, n1, S, ld, plane, E,
                         lp, flags);
      if constexpr (FMT == kFmtI8) {
        OZK_LAUNCH_CHECK();
        hipLaunchKernelGGL(i8_plane_sums_kernel, dim3((unsigned)(lp / 64), (unsigned)(n0 + n1)),
                           dim3(256), 0, st, (const int8_t*)S, lp, ld, i8_offset(rho), Sg);
      }
    }
  }
#undef OZK_REG
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

int launch_fill_u32(uint32_t* p, uint32_t v, hipStream_t st) {
  hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(1), 0, st, p, v);
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

// FP32 column extraction of columns up to kGangRun * kGangMaxMembers =
// 65536 rows runs on gangs; FP64 column extraction, and longer columns, go
// through an FP64 transpose of X into the workspace.
static bool gang_columns(int64_t rows) {
  return round_up(rows, kKPad) <= (int64_t)kGangRun * kGangMaxMembers && gangs_enabled();
}

// FP32 columns of up to 256 x 16 rows: one panel per workgroup
// (extract_cols_panel).  Longer ones go to the gangs, whose members read
// whole 128-byte lines of X: a panel's 16-byte row segments cost as many
// L2 requests as whole lines do, which bounds it below the gangs there
// (8192 x 8192: 0.34 ms, the gangs 0.30 ms; 4096 x 4096: 0.095 ms, the
// gangs 0.104 ms).
static bool panel_columns(int64_t rows) {
  return round_up(rows, kKPad) <= (int64_t)kPanelGroups * 16;
}

template <int FMT>
static int launch_cols_panel(const double* X, int64_t rows, int64_t cols, int64_t ldx,
                             int rho, int n0, int n1, void* Sv, int32_t* E, uint32_t* flags,
                             hipStream_t st, int32_t* Sg) {
  typedef typename PlaneElem<FMT>::type T;
  if (rows <= 0 || cols <= 0) return OZK_OK;
  const int64_t ld = round_up(rows, kKPad), lp = round_up(cols, kLinePad);
  const int64_t plane = lp * ld;
  const dim3 grid((unsigned)(lp / kPanelCols));
#define OZK_PANEL_LAUNCH(RPT)                                                              \
  hipLaunchKernelGGL((extract_cols_panel<FMT, RPT>), grid, dim3(kPanelThreads), 0, st, X,  \
                     rows, cols, ldx, rho, n0, n1, (T*)Sv, ld, plane, E, lp, flags, Sg)
  if (ld <= kPanelGroups * 4)
    OZK_PANEL_LAUNCH(4);
  else if (ld <= kPanelGroups * 8)
    OZK_PANEL_LAUNCH(8);
  else
    OZK_PANEL_LAUNCH(16);
#undef OZK_PANEL_LAUNCH
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

// Ticket and exchange records (zeroed per launch).
static size_t gang_workspace_bytes(int64_t rows, int64_t cols, int nslices) {
  const int G = gang_members(round_up(rows, kKPad));
  return (size_t)round_up(kGangHeader + (round_up(cols, kLinePad) / kGangPW) *
                                            gang_round_offset(nslices, G) * 4,
                          256);
}

// Offset of the row-gang records after the transposed copy.
static size_t transpose_bytes(int64_t rows, int64_t cols) {
  return (size_t)round_up(rows * cols * (int64_t)sizeof(double), 256);
}

size_t extract_workspace_bytes(int64_t rows, int64_t cols, int by_cols, bool f64) {
  if (!by_cols) return !f64 && gang_rows(cols) ? row_gang_bytes(rows, cols, kMaxSlices) : 0;
  if (!f64 && panel_columns(rows)) return 0;
  if (!f64 && gang_columns(rows)) return gang_workspace_bytes(rows, cols, kMaxSlices);
  return transpose_bytes(rows, cols) +
         (!f64 && gang_rows(rows) ? row_gang_bytes(cols, rows, kMaxSlices) : 0);
}

template <int FMT>
static int launch_cols_gang(const double* X, int64_t rows, int64_t cols, int64_t ldx,
                            int rho, int n0, int n1, void* Sv, int32_t* E, uint32_t* flags,
                            void* ws, size_t wsb, hipStream_t st, int32_t* Sg) {
  typedef typename PlaneElem<FMT>::type T;
  if (rows <= 0 || cols <= 0) return OZK_OK;
  const int ns = n0 > n1 ? n0 : n1;
  const size_t need = gang_workspace_bytes(rows, cols, ns);
  if (wsb < need || !ws) {
    set_error("extract: workspace of %zu bytes needed, %zu given", need, wsb);
    return OZK_ERR_WORKSPACE;
  }
  const int64_t ld = round_up(rows, kKPad), lp = round_up(cols, kLinePad);
  const int64_t plane = lp * ld, npanels = lp / kGangPW;
  const int G = gang_members(ld);
  // the ticket, the exchange records and the INT8 line sums start at zero
  const int64_t n16 = (int64_t)need / 16;
  hipLaunchKernelGGL(zero_u32x4_kernel, dim3((unsigned)((n16 + 255) / 256 < 1024 ? (n16 + 255) / 256 : 1024)),
                     dim3(256), 0, st, (uint4*)ws, n16);
  OZK_LAUNCH_CHECK();
  if constexpr (FMT == kFmtI8) {
    const int64_t ns32 = (int64_t)(n0 + n1) * lp;
    hipLaunchKernelGGL(zero_i32_kernel, dim3((unsigned)((ns32 + 255) / 256 < 1024 ? (ns32 + 255) / 256 : 1024)),
                       dim3(256), 0, st, Sg, ns32);
    OZK_LAUNCH_CHECK();
  }
  uint32_t* ticket = (uint32_t*)ws;
  uint32_t* rec = (uint32_t*)((char*)ws + kGangHeader);
  const dim3 grid((unsigned)(npanels * G));
  const uint32_t wait_ticks = wait_polls(kGangWaitTicks);
  hipLaunchKernelGGL((extract_cols_gang<FMT>), grid, dim3(kGangThreads), 0, st, X, rows, cols,
                     ldx, rho, n0, n1, (T*)Sv, ld, plane, E, lp, flags, rec, ticket, G,
                     wait_ticks, Sg);
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

// Extraction entry shared by the FP32 and FP64 paths.  FP32 columns go to
// the gangs; other columns are first transposed into the workspace so each
// is contiguous.  int8 planes (FP32 path only) need rho >= 19 so that
// |q| <= 64.
template <typename W>
int extract(const double* X, int64_t rows, int64_t cols, int64_t ldx,
            int by_cols, int rho, int n0, int n1, void* S, int32_t* E,
            uint32_t* flags, void* ws, size_t wsb, hipStream_t st, bool i8,
            int32_t* sums) {
  if (i8 && (sizeof(W) != 4 || rho < 19 || rho > 24)) {
    set_error("int8 slice planes need the FP32 path with 19 <= rho <= 24 (rho=%d)", rho);
    return OZK_ERR_UNSUPPORTED;
  }
  if (i8 && !sums) {
    set_error("int8 slice planes need a line-sum array");
    return OZK_ERR_INVALID;
  }
  const double* src = X;
  int64_t lines = rows, len = cols, lds = ldx;
  if constexpr (sizeof(W) == 4) {
    if (by_cols && panel_columns(rows)) {
      if (i8)
        return launch_cols_panel<kFmtI8>(X, rows, cols, ldx, rho, n0, n1, S, E, flags, st,
                                         sums);
      return launch_cols_panel<kFmtBf16>(X, rows, cols, ldx, rho, n0, n1, S, E, flags, st,
                                         nullptr);
    }
    if (by_cols && gang_columns(rows)) {
      if (i8)
        return launch_cols_gang<kFmtI8>(X, rows, cols, ldx, rho, n0, n1, S, E, flags, ws,
                                        wsb, st, sums);
      return launch_cols_gang<kFmtBf16>(X, rows, cols, ldx, rho, n0, n1, S, E, flags, ws,
                                        wsb, st, nullptr);
    }
  }
  if (by_cols) {
    const size_t need = extract_workspace_bytes(rows, cols, 1, sizeof(W) == 8);
    if (wsb < need || (need && !ws)) {
      set_error("extract: workspace of %zu bytes needed, %zu given", need, wsb);
      return OZK_ERR_WORKSPACE;
    }
    double* XT = (double*)ws;
    const dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 127) / 128));
    hipLaunchKernelGGL(transpose_f64, grid, dim3(512), 0, st, X, rows, cols, ldx, XT);
    OZK_LAUNCH_CHECK();
    src = XT;
    lines = cols;
    len = rows;
    lds = rows;
    const size_t tb = transpose_bytes(rows, cols);  // the rest holds row-gang records
    ws = wsb > tb ? (void*)((char*)ws + tb) : nullptr;
    wsb = wsb > tb ? wsb - tb : 0;
  }
  if (i8)
    return launch_lines<W, kFmtI8>(src, lines, len, lds, rho, n0, n1, S, E, flags, ws, wsb, st,
                                   sums);
  return launch_lines<W, kFmtBf16>(src, lines, len, lds, rho, n0, n1, S, E, flags, ws, wsb,
                                   st, nullptr);
}

template int extract<float>(const double*, int64_t, int64_t, int64_t, int, int,
                            int, int, void*, int32_t*, uint32_t*, void*,
                            size_t, hipStream_t, bool, int32_t*);
template int extract<double>(const double*, int64_t, int64_t, int64_t, int, int,
                             int, int, void*, int32_t*, uint32_t*, void*,
                             size_t, hipStream_t, bool, int32_t*);

int launch_check_finite(const double* X, int64_t rows, int64_t cols,
                        int64_t ld, uint32_t* flags, hipStream_t st) {
  const int64_t total = rows * cols;
  if (total == 0) return OZK_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(check_finite_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     st, X, rows, cols, ld, flags);
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

}  // namespace ozk
