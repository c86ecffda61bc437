// Shared definitions for the Ozaki-scheme kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <type_traits>

#include "../../include/ozaki_amd.h"

namespace ozk {

// f(integral_constant<int, I>) for I = B .. E - 1, unrolled at compile time.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// ---------------------------------------------------------------- errors
// Thread-local message behind ozk_last_error(); every entry point clears it
// on entry and returns a negative status with a message on failure.
void set_error(const char* fmt, ...);
void clear_error();

#define OZK_CHECK_ARG(cond, ...)            \
  do {                                      \
    if (!(cond)) {                          \
      ::ozk::set_error(__VA_ARGS__);        \
      return OZK_ERR_INVALID;               \
    }                                       \
  } while (0)

#define OZK_HIP(call)                                                     \
  do {                                                                    \
    hipError_t e_ = (call);                                               \
    if (e_ != hipSuccess) {                                               \
      ::ozk::set_error("%s failed: %s", #call, hipGetErrorString(e_));    \
      return OZK_ERR_HIP;                                                 \
    }                                                                     \
  } while (0)

#define OZK_LAUNCH_CHECK()                                                \
  do {                                                                    \
    hipError_t e_ = hipGetLastError();                                    \
    if (e_ != hipSuccess) {                                               \
      ::ozk::set_error("kernel launch failed: %s", hipGetErrorString(e_)); \
      return OZK_ERR_HIP;                                                 \
    }                                                                     \
  } while (0)

// Compute units of the current device (cached per device; 256 if the
// query fails).  Persistent kernels size their grids with it.
int cu_count();

// Limit of the kernels' bounded waits between workgroups: `dflt`, or the
// limit a test set with ozk_set_wait_polls.
uint32_t wait_polls(uint32_t dflt);

// Whether the calling thread's extractions may use gangs of workgroups
// (ozk_set_gangs); without them, columns go through a transposed copy and
// long rows are streamed, with no waits between workgroups.
bool gangs_enabled();

// ---------------------------------------------------------------- layout
// Slice planes hold BF16 bit patterns or INT8 grid counts with lines padded
// to kLinePad and k padded to kKPad elements; padding holds zeros, so the
// GEMM needs no bounds checks in its K loop or its operand tiles.
//
// Inside a plane the bytes are chunk-major: k is cut into 64-byte chunks
// (32 BF16 or 64 INT8 values) and chunk c of every line is stored together,
// [c][line][64 bytes].  The 64 lines of an output tile therefore occupy one
// contiguous 4 KiB block per chunk, which the GEMM moves into LDS with
// fully contiguous 1 KiB loads.  Within a line's 64 bytes the four 16-byte
// units are stored in the order u ^ unit_swizzle(line), which spreads the
// MFMA fragment reads of 16 or 32 consecutive lines over all LDS banks.
constexpr int64_t kKPad = 64;
constexpr int64_t kLinePad = 64;
constexpr int kChunkBytes = 64;

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Offset of the INT8 plane format: a grid count q (|q| <= 2^(25 - rho),
// rho >= 19) is stored as q + i8_offset(rho), in [-1, 127].
__host__ __device__ inline int32_t i8_offset(int rho) { return (1 << (25 - rho)) - 1; }

__host__ __device__ __forceinline__ int unit_swizzle(int64_t line) {
  const int r = (int)(line & 15);
  return ((r >> 1) ^ (r >> 2)) & 3;
}

// Element offset of (line, k) inside one plane of `lpad` lines, for
// elements of `EB` bytes.
template <int EB>
__host__ __device__ __forceinline__ int64_t plane_offset(int64_t line, int64_t k,
                                                         int64_t lpad) {
  constexpr int kPer = kChunkBytes / EB;
  const int64_t c = k / kPer;
  const int b = (int)(k - c * kPer) * EB;
  const int u = b >> 4;
  return ((c * lpad + line) * kChunkBytes + 16 * (u ^ unit_swizzle(line)) + (b & 15)) / EB;
}

// ---------------------------------------------------------------- device
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// FP32 -> BF16 bits, round to nearest even.  Slices are BF16-exact by
// construction (at most 8 significant bits), so this is exact for them.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

// One 16-byte-per-lane direct load from global memory into LDS
// (global_load_lds_dwordx4): lane l's 16 bytes land at LDS offset
// `lds_addr` + 16 l.  `lds_addr` and `gbase` are wave-uniform; `voff` is the
// lane's byte offset from `gbase`, which must be 16-byte aligned.  Written as
// inline assembly so that the compiler does not order LDS reads behind these
// loads: the kernels wait for them themselves (wait_vm).  M0 carries the LDS
// address and is declared clobbered, so the compiler keeps no value of its
// own in M0 across the load.  (Clang warns that M0 is a reserved register
// whose value it will not save for the statement, which is not wanted here.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(uint32_t lds_addr, const void* gbase,
                                      uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2"
      :
      : "s"(lds_addr), "v"(voff), "s"(gbase)
      : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most N of this wave's vector-memory operations are
// outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(size_t)((__attribute__((address_space(3))) const char*)p);
}

}  // namespace ozk
