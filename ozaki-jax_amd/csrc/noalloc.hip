// ozk_matmul_noalloc: ozk_matmul for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).  Its workspace is a file-scope device array of
// OZK_NOALLOC_SCRATCH_BYTES, which every GPU the library runs on holds from
// the module's load until the process ends.
//
// In host code the array's name is a host-side stand-in, not a device
// address: the first call on each device, with that device current, asks the
// runtime for the array's address on that device (hipGetSymbolAddress), and
// every later use -- the workspace handed to the driver -- takes that
// pointer.  Each GPU holds its own copy of the array at its own address.
//
// Every call on one GPU uses that GPU's one array: calls that overlap on a
// GPU (other streams, other host threads) race.  Nothing in the array has
// to start at zero: every region the driver carves from it (slice planes,
// transpose, fold state, K-split partial sums) is written before it is
// read, and the flag word, which is cleared first, is the caller's.

#include <mutex>

#include "common.h"

namespace ozk {

constexpr size_t kScratchBytes = OZK_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch size");

static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, looked up once per
// device.
static int scratch_on_current_device(void** out) {
  int dev = 0;
  OZK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("matmul_noalloc: device %d beyond the %d devices tracked", dev, kMaxDevices);
    return OZK_ERR_UNSUPPORTED;
  }
  void* p = __atomic_load_n(&g_scratch_ptr[dev], __ATOMIC_ACQUIRE);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev];
    if (!p) {
      OZK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
      if (!p) {
        set_error("matmul_noalloc: no device address for the scratch array");
        return OZK_ERR_HIP;
      }
      __atomic_store_n(&g_scratch_ptr[dev], p, __ATOMIC_RELEASE);
    }
  }
  *out = p;
  return OZK_OK;
}

}  // namespace ozk

using namespace ozk;

extern "C" int ozk_matmul_noalloc(const double* A, int64_t lda, const double* B,
                                  int64_t ldb, double* C, int64_t ldc, int64_t N,
                                  int64_t K, int64_t M, int pipeline, int n_hi,
                                  int n_lo, int order, uint32_t* flags, void* stream) {
  clear_error();
  OZK_CHECK_ARG(N >= 0 && M >= 0 && K >= 1, "invalid shape N=%lld K=%lld M=%lld",
                (long long)N, (long long)K, (long long)M);
  const int pb = ozk_matmul_plane_bytes(pipeline, K, n_hi, n_lo);  // checks the counts
  if (pb < 0) return pb;
  const size_t need = ozk_matmul_workspace_bytes(N, K, M, pipeline, n_hi, n_lo);
  if (need > kScratchBytes) {
    set_error("matmul_noalloc: this shape needs %zu bytes of workspace, above the "
              "%zu bytes of the library's scratch array; use ozk_matmul",
              need, kScratchBytes);
    return OZK_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc) return rc;
  return ozk_matmul(A, lda, B, ldb, C, ldc, N, K, M, pipeline, n_hi, n_lo, order, ws,
                    kScratchBytes, flags, stream);
}
