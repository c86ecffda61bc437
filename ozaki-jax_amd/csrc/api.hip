// C ABI of the Ozaki-scheme engine: argument checks, workspace carving and
// the driver sequences (extract A, extract B, fused GEMM, epilogue kernels).

#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "common.h"

namespace ozk {

static thread_local std::string g_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}
void clear_error() { g_error.clear(); }

int cu_count() {
  static int cache[64];  // 0 = not queried yet; racing writers store the same value
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < 64 && cache[dev] > 0) return cache[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  if (dev >= 0 && dev < 64) cache[dev] = cus;
  return cus;
}

static std::atomic<uint32_t> g_wait_polls{0};

uint32_t wait_polls(uint32_t dflt) {
  const uint32_t v = g_wait_polls.load(std::memory_order_relaxed);
  return v ? v : dflt;
}

// Gang extraction on (1) or off (0) for the calling thread's calls.
static thread_local int t_gangs = 1;
bool gangs_enabled() { return t_gangs != 0; }

// Implemented in extract.hip / gemm.hip.
template <typename W>
int extract(const double* X, int64_t rows, int64_t cols, int64_t ldx,
            int by_cols, int rho, int n0, int n1, void* S, int32_t* E,
            uint32_t* flags, void* ws, size_t wsb, hipStream_t st, bool i8,
            int32_t* sums);
size_t extract_workspace_bytes(int64_t rows, int64_t cols, int by_cols, bool f64);
int launch_fill_u32(uint32_t* p, uint32_t v, hipStream_t st);
int launch_check_finite(const double* X, int64_t rows, int64_t cols,
                        int64_t ld, uint32_t* flags, hipStream_t st);
bool allpairs_supported(int pipe, int nhi, int nlo);
bool allpairs_products_supported(int pipe, int nhi, int nlo);
int launch_gemm(const void* As, const int32_t* Ae, const void* Bs,
                const int32_t* Be, int64_t N, int64_t M, int64_t K, int pipe,
                int nhi, int nlo, int order, double* C, int64_t ldc,
                void* ws, size_t ws_bytes, hipStream_t st, bool i8, int rho,
                const int32_t* Asum, const int32_t* Bsum);
size_t gemm_workspace_bytes(int64_t N, int64_t M, int pipe, int nhi, int nlo,
                            int order);
size_t gemm_state_bytes(int64_t N, int64_t M, int pipe, int nhi, int nlo, int order);
int launch_gemm_pair(const void* As, const int32_t* Ae, const void* Bs,
                     const int32_t* Be, int64_t N, int64_t M, int64_t K, int nhi,
                     int nlo, float* C_hi, float* C_lo, int64_t ldc, void* ws,
                     size_t ws_bytes, hipStream_t st, bool i8, int rho,
                     const int32_t* Asum, const int32_t* Bsum);
int launch_products(const void* As, const void* Bs, int64_t N, int64_t M,
                    int64_t K, int pipe, int nhi, int nlo, float* P,
                    int64_t ldp, hipStream_t st, bool i8, int rho, const int32_t* Asum,
                    const int32_t* Bsum);
int launch_probe_mfma(int32_t* out, hipStream_t st);
size_t lu_solve_workspace_bytes(int64_t n, int64_t ncols);
int64_t lu_factor_max_n();
size_t lu_factor_workspace_bytes();
int launch_lu_factor(float* A, int64_t lda, int64_t n, int32_t* perm, void* ws,
                     uint32_t* status, hipStream_t st);
int launch_lu_solve(const float* LU, int64_t lda, const int32_t* perm, int64_t n,
                    const double* B, int64_t ldb, double* X, int64_t ldx, int64_t ncols,
                    void* ws, uint32_t* status, hipStream_t st);
bool gram_sym_supported(int nhi, int nlo);
int launch_gram_sym(const void* S, const int32_t* E, int64_t n, int64_t K, int nhi,
                    int nlo, double* G, int64_t ldg, void* ws, size_t ws_bytes,
                    hipStream_t st, bool i8, int rho, const int32_t* Ssum);
size_t gemm_tail_bytes(int64_t N, int64_t M, int64_t K, int pipe, int nhi, int nlo,
                       bool sym, bool i8);
bool residual_rows_supported(int64_t K, int64_t ncols, int nhi, int nlo);
int launch_residual_rows(const double* A, int64_t N, int64_t K, int64_t lda,
                         const double* x, int64_t ldx, const double* b,
                         int64_t ldb, double* r, int64_t ldr, int64_t ncols, int rho,
                         int nhi, int nlo, uint32_t* flags, hipStream_t st);

constexpr int kMaxSlices = 32;
constexpr size_t kAlign = 256;

static int rho_generic(int64_t K, int m1) {
  // rho = max(ceil(m1 - (24 - ceil(log2 max(K, 2))) / 2), m1 + 1 - 8)
  const int64_t k = K < 2 ? 2 : K;
  int clog2 = 0;
  while (((int64_t)1 << clog2) < k) ++clog2;
  const int num = 2 * m1 - 24 + clog2;
  const int gamma = num >= 0 ? (num + 1) / 2 : -((-num) / 2);
  const int xi = m1 + 1 - 8;
  return gamma > xi ? gamma : xi;
}

// Sequential carving of one workspace into aligned regions.
struct Carver {
  char* base;
  size_t off = 0;
  explicit Carver(void* b) : base((char*)b) {}
  void* take(size_t bytes) {
    void* p = base ? base + off : nullptr;
    off += (bytes + kAlign - 1) / kAlign * kAlign;
    return p;
  }
};

// Slice planes, their exponents and, for INT8 planes, their line sums.
struct SliceSet {
  void* s;
  int32_t* e;
  int32_t* sum;
};

static SliceSet carve_slices(Carver& c, int planes, int64_t lines, int64_t len,
                             size_t elem_bytes) {
  const int64_t lp = round_up(lines, kLinePad), ld = round_up(len, kKPad);
  SliceSet r;
  r.s = c.take((size_t)planes * lp * ld * elem_bytes);
  r.e = (int32_t*)c.take((size_t)planes * lp * sizeof(int32_t));
  r.sum = elem_bytes == 1 ? (int32_t*)c.take((size_t)planes * lp * sizeof(int32_t)) : nullptr;
  return r;
}

// The drivers use INT8 slice planes (exact for rho >= 19, i.e. K > 4096)
// whenever the schedule has an all-pairs kernel, BF16 planes otherwise.
static bool use_i8(int pipe, int64_t contraction, int nhi, int nlo) {
  return pipe == OZK_PIPE_ONDEVICE && rho_generic(contraction, 24) >= 19 &&
         allpairs_supported(pipe, nhi, nlo);
}

static int check_counts(int pipe, int nhi, int nlo) {
  OZK_CHECK_ARG(pipe == OZK_PIPE_ONDEVICE || pipe == OZK_PIPE_HOST,
                "unknown pipeline %d", pipe);
  OZK_CHECK_ARG(nhi >= 1 && nhi <= kMaxSlices, "n_hi/n_slices=%d outside [1, %d]",
                nhi, kMaxSlices);
  if (pipe == OZK_PIPE_ONDEVICE)
    OZK_CHECK_ARG(nlo >= 1 && nlo <= kMaxSlices, "n_lo=%d outside [1, %d]", nlo,
                  kMaxSlices);
  return OZK_OK;
}

static int check_order(int order) {
  OZK_CHECK_ARG(order >= OZK_ORDER_2SUM && order <= OZK_ORDER_HOST_NP,
                "unknown accumulation order %d", order);
  return OZK_OK;
}

// y = b - y (residual epilogue), N x ncols with leading dimensions.
__global__ void sub_from_kernel(const double* __restrict__ b, int64_t ldb,
                                double* __restrict__ y, int64_t ldy,
                                double* __restrict__ r, int64_t ldr, int64_t n,
                                int64_t ncols) {
  const int64_t total = n * ncols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / ncols, c = i - row * ncols;
    r[row * ldr + c] = b[row * ldb + c] - y[row * ldy + c];
  }
}

// G = (G + G^T) * 0.5 in place (gram.py:37); each unordered pair once.
__global__ void symmetrize_kernel(double* __restrict__ G, int64_t n,
                                  int64_t ld) {
  const int64_t total = n * n;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / n, c = i - r * n;
    if (c < r) continue;
    const double a = G[r * ld + c], b = G[c * ld + r];
    const double s = (a + b) * 0.5;
    G[r * ld + c] = s;
    if (c != r) G[c * ld + r] = (b + a) * 0.5;
  }
}

static unsigned grid_for(int64_t total) {
  int64_t b = (total + 255) / 256;
  if (b < 1) b = 1;
  if (b > 8192) b = 8192;
  return (unsigned)b;
}

}  // namespace ozk

using namespace ozk;

extern "C" {

const char* ozk_last_error(void) { return g_error.c_str(); }

int ozk_abi_version(void) { return 3; }

void ozk_set_wait_polls(uint32_t polls) {
  ozk::g_wait_polls.store(polls, std::memory_order_relaxed);
}

void ozk_set_gangs(int enable) { ozk::t_gangs = enable ? 1 : 0; }

int ozk_device_info(char* buf, size_t len, int* cu_count) {
  clear_error();
  int dev = 0;
  OZK_HIP(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  OZK_HIP(hipGetDeviceProperties(&prop, dev));
  if (buf && len) {
    snprintf(buf, len, "%s (%s)", prop.name, prop.gcnArchName);
  }
  if (cu_count) *cu_count = prop.multiProcessorCount;
  return OZK_OK;
}

int ozk_rho_f64(int64_t K) { return rho_generic(K, 53); }
int ozk_rho_f32(int64_t K) { return rho_generic(K, 24); }
int64_t ozk_slice_ld(int64_t len) { return round_up(len, kKPad); }
int64_t ozk_slice_lines(int64_t lines) { return round_up(lines, kLinePad); }

int ozk_pair_count(int pipeline, int n_hi, int n_lo) {
  clear_error();
  int rc = check_counts(pipeline, n_hi, n_lo);
  if (rc) return rc;
  return pipeline == OZK_PIPE_ONDEVICE ? n_hi * n_hi + 2 * n_hi * n_lo
                                       : n_hi * (n_hi + 1) / 2;
}

size_t ozk_extract_workspace_bytes(int64_t rows, int64_t cols, int by_cols) {
  const size_t a = extract_workspace_bytes(rows, cols, by_cols, false);
  const size_t b = extract_workspace_bytes(rows, cols, by_cols, true);
  return a > b ? a : b;
}

int ozk_extract_f32(const double* X, int64_t rows, int64_t cols, int64_t ldx,
                    int by_cols, int rho, int n_hi, int n_lo,
                    uint16_t* slices, int32_t* exps, uint32_t* flags,
                    void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  OZK_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  OZK_CHECK_ARG(ldx >= cols || rows <= 1, "ldx=%lld < cols=%lld", (long long)ldx,
                (long long)cols);
  // n_lo = 0 extracts the hi part only (the FP32 helpers of the reference
  // take FP32 input, for which lo is identically zero).
  OZK_CHECK_ARG(n_hi >= 1 && n_hi <= kMaxSlices && n_lo >= 0 && n_lo <= kMaxSlices,
                "slice counts (%d, %d) outside [1, %d] x [0, %d]", n_hi, n_lo,
                kMaxSlices, kMaxSlices);
  if (rows == 0 || cols == 0) return OZK_OK;
  OZK_CHECK_ARG(X && slices && exps && flags, "null pointer");
  return extract<float>(X, rows, cols, ldx, by_cols, rho, n_hi, n_lo, slices,
                        exps, flags, workspace, workspace_bytes,
                        (hipStream_t)stream, false, nullptr);
}

int ozk_extract_f32_i8(const double* X, int64_t rows, int64_t cols,
                       int64_t ldx, int by_cols, int rho, int n_hi, int n_lo,
                       int8_t* slices, int32_t* exps, int32_t* sums, uint32_t* flags,
                       void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  OZK_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  OZK_CHECK_ARG(ldx >= cols || rows <= 1, "ldx=%lld < cols=%lld", (long long)ldx,
                (long long)cols);
  OZK_CHECK_ARG(n_hi >= 1 && n_hi <= kMaxSlices && n_lo >= 0 && n_lo <= kMaxSlices,
                "slice counts (%d, %d) outside [1, %d] x [0, %d]", n_hi, n_lo,
                kMaxSlices, kMaxSlices);
  if (rho < 19 || rho > 24) {
    set_error("int8 slice planes need 19 <= rho <= 24 (got %d)", rho);
    return OZK_ERR_UNSUPPORTED;
  }
  if (rows == 0 || cols == 0) return OZK_OK;
  OZK_CHECK_ARG(X && slices && exps && sums && flags, "null pointer");
  return extract<float>(X, rows, cols, ldx, by_cols, rho, n_hi, n_lo, slices,
                        exps, flags, workspace, workspace_bytes,
                        (hipStream_t)stream, true, sums);
}

int ozk_extract_f64(const double* X, int64_t rows, int64_t cols, int64_t ldx,
                    int by_cols, int rho, int n_slices, uint16_t* slices,
                    int32_t* exps, uint32_t* flags, void* workspace,
                    size_t workspace_bytes, void* stream) {
  clear_error();
  OZK_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  OZK_CHECK_ARG(ldx >= cols || rows <= 1, "ldx < cols");
  int rc = check_counts(OZK_PIPE_HOST, n_slices, 0);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return OZK_OK;
  OZK_CHECK_ARG(X && slices && exps && flags, "null pointer");
  return extract<double>(X, rows, cols, ldx, by_cols, rho, n_slices, 0, slices,
                         exps, flags, workspace, workspace_bytes,
                         (hipStream_t)stream, false, nullptr);
}

size_t ozk_gemm_workspace_bytes(int64_t N, int64_t M, int pipeline, int n_hi,
                                int n_lo, int order) {
  if (N < 0 || M < 0) return 0;
  return gemm_workspace_bytes(N, M, pipeline, n_hi, n_lo, order);
}

int ozk_gemm(const uint16_t* a_slices, const int32_t* a_exps,
             const uint16_t* b_slices, const int32_t* b_exps, int64_t N,
             int64_t M, int64_t K, int pipeline, int n_hi, int n_lo, int order,
             double* C, int64_t ldc, void* workspace, size_t workspace_bytes,
             void* stream) {
  clear_error();
  int rc = check_counts(pipeline, n_hi, n_lo);
  if (rc) return rc;
  if ((rc = check_order(order))) return rc;
  OZK_CHECK_ARG(N >= 0 && M >= 0 && K >= 1, "invalid shape N=%lld M=%lld K=%lld",
                (long long)N, (long long)M, (long long)K);
  OZK_CHECK_ARG(ldc >= M || N <= 1, "ldc < M");
  if (N == 0 || M == 0) return OZK_OK;
  return launch_gemm(a_slices, a_exps, b_slices, b_exps, N, M, K, pipeline,
                     n_hi, n_lo, order, C, ldc, workspace, workspace_bytes,
                     (hipStream_t)stream, false, 0, nullptr, nullptr);
}

int ozk_gemm_i8(const int8_t* a_slices, const int32_t* a_exps, const int32_t* a_sums,
                const int8_t* b_slices, const int32_t* b_exps, const int32_t* b_sums,
                int64_t N, int64_t M, int64_t K, int rho, int n_hi, int n_lo, int order,
                double* C, int64_t ldc, void* workspace, size_t workspace_bytes,
                void* stream) {
  clear_error();
  int rc = check_counts(OZK_PIPE_ONDEVICE, n_hi, n_lo);
  if (rc) return rc;
  if ((rc = check_order(order))) return rc;
  OZK_CHECK_ARG(N >= 0 && M >= 0 && K >= 1, "invalid shape N=%lld M=%lld K=%lld",
                (long long)N, (long long)M, (long long)K);
  OZK_CHECK_ARG(ldc >= M || N <= 1, "ldc < M");
  if (rho < 19 || rho > 24 || !allpairs_supported(OZK_PIPE_ONDEVICE, n_hi, n_lo)) {
    set_error("int8 planes need 19 <= rho <= 24 and an all-pairs schedule (rho=%d, (%d, %d))",
              rho, n_hi, n_lo);
    return OZK_ERR_UNSUPPORTED;
  }
  if (N == 0 || M == 0) return OZK_OK;
  OZK_CHECK_ARG(a_sums && b_sums, "null pointer");
  return launch_gemm(a_slices, a_exps, b_slices, b_exps, N, M, K,
                     OZK_PIPE_ONDEVICE, n_hi, n_lo, order, C, ldc, workspace,
                     workspace_bytes, (hipStream_t)stream, true, rho, a_sums, b_sums);
}

int ozk_gemm_2sum_pair(const void* a_slices, const int32_t* a_exps,
                       const int32_t* a_sums, const void* b_slices,
                       const int32_t* b_exps, const int32_t* b_sums, int64_t N,
                       int64_t M, int64_t K, int plane_bytes, int rho, int n_hi,
                       int n_lo, float* C_hi, float* C_lo, int64_t ldc,
                       void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_counts(OZK_PIPE_ONDEVICE, n_hi, n_lo);
  if (rc) return rc;
  OZK_CHECK_ARG(plane_bytes == 1 || plane_bytes == 2, "plane_bytes=%d is not 1 or 2",
                plane_bytes);
  OZK_CHECK_ARG(N >= 0 && M >= 0 && K >= 1, "invalid shape N=%lld M=%lld K=%lld",
                (long long)N, (long long)M, (long long)K);
  OZK_CHECK_ARG(ldc >= M || N <= 1, "ldc < M");
  const bool i8 = plane_bytes == 1;
  if (i8 && (rho < 19 || rho > 24 || !allpairs_supported(OZK_PIPE_ONDEVICE, n_hi, n_lo))) {
    set_error("int8 planes need 19 <= rho <= 24 and an all-pairs schedule (rho=%d, (%d, %d))",
              rho, n_hi, n_lo);
    return OZK_ERR_UNSUPPORTED;
  }
  if (N == 0 || M == 0) return OZK_OK;
  OZK_CHECK_ARG(a_slices && a_exps && b_slices && b_exps && C_hi && C_lo, "null pointer");
  OZK_CHECK_ARG(!i8 || (a_sums && b_sums), "null pointer");
  const size_t need = gemm_state_bytes(N, M, OZK_PIPE_ONDEVICE, n_hi, n_lo, OZK_ORDER_2SUM);
  if (workspace_bytes < need || (need && !workspace)) {
    set_error("gemm_2sum_pair: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
    return OZK_ERR_WORKSPACE;
  }
  return launch_gemm_pair(a_slices, a_exps, b_slices, b_exps, N, M, K, n_hi, n_lo, C_hi,
                          C_lo, ldc, workspace, workspace_bytes, (hipStream_t)stream, i8,
                          rho, i8 ? a_sums : nullptr, i8 ? b_sums : nullptr);
}

int ozk_slice_products(const uint16_t* a_slices, const uint16_t* b_slices,
                       int64_t N, int64_t M, int64_t K, int pipeline, int n_hi,
                       int n_lo, float* P, int64_t ldp, void* stream) {
  clear_error();
  int rc = check_counts(pipeline, n_hi, n_lo);
  if (rc) return rc;
  OZK_CHECK_ARG(N >= 0 && M >= 0 && K >= 1, "invalid shape");
  OZK_CHECK_ARG(ldp >= M, "ldp < M");
  if (N == 0 || M == 0) return OZK_OK;
  return launch_products(a_slices, b_slices, N, M, K, pipeline, n_hi, n_lo, P,
                         ldp, (hipStream_t)stream, false, 0, nullptr, nullptr);
}

int ozk_slice_products_i8(const int8_t* a_slices, const int32_t* a_sums,
                          const int8_t* b_slices, const int32_t* b_sums,
                          int64_t N, int64_t M, int64_t K, int rho, int n_hi,
                          int n_lo, float* P, int64_t ldp, void* stream) {
  clear_error();
  int rc = check_counts(OZK_PIPE_ONDEVICE, n_hi, n_lo);
  if (rc) return rc;
  OZK_CHECK_ARG(N >= 0 && M >= 0 && K >= 1, "invalid shape");
  OZK_CHECK_ARG(ldp >= M, "ldp < M");
  if (rho < 19 || rho > 24 || !allpairs_products_supported(OZK_PIPE_ONDEVICE, n_hi, n_lo)) {
    set_error("int8 per-pair products need 19 <= rho <= 24 and a fixed all-pairs schedule");
    return OZK_ERR_UNSUPPORTED;
  }
  if (N == 0 || M == 0) return OZK_OK;
  OZK_CHECK_ARG(a_sums && b_sums, "null pointer");
  return launch_products(a_slices, b_slices, N, M, K, OZK_PIPE_ONDEVICE, n_hi,
                         n_lo, P, ldp, (hipStream_t)stream, true, rho, a_sums, b_sums);
}

// OZK_PIPE_ONDEVICE_BF16 is the on-device pipeline with the INT8 planes
// switched off; `i8` says whether a matmul of this shape runs on INT8 planes.
static int matmul_pipe(int pipeline, int64_t K, int nhi, int nlo, bool* i8) {
  const bool bf16 = pipeline == OZK_PIPE_ONDEVICE_BF16;
  const int pipe = bf16 ? OZK_PIPE_ONDEVICE : pipeline;
  if (i8) *i8 = !bf16 && use_i8(pipe, K, nhi, nlo);
  return pipe;
}

// Extraction workspace of the rows of A (N x K) and the columns of B
// (K x M), extracted one after the other on one stream: one buffer serves
// both.
static size_t extract_pair_bytes(int64_t N, int64_t K, int64_t M, bool f64) {
  const size_t a = extract_workspace_bytes(N, K, 0, f64);
  const size_t b = extract_workspace_bytes(K, M, 1, f64);
  return a > b ? a : b;
}

static size_t matmul_ws(int64_t N, int64_t K, int64_t M, int pipeline, int nhi,
                        int nlo, bool carve, void* ws, SliceSet* a,
                        SliceSet* b, void** tws, void** gws = nullptr,
                        size_t* gwsb = nullptr) {
  bool i8;
  pipeline = matmul_pipe(pipeline, K, nhi, nlo, &i8);
  const int planes = pipeline == OZK_PIPE_ONDEVICE ? nhi + nlo : nhi;
  const size_t eb = i8 ? 1 : 2;
  Carver c(carve ? ws : nullptr);
  SliceSet sa = carve_slices(c, planes, N, K, eb);
  SliceSet sb = carve_slices(c, planes, M, K, eb);
  void* t = c.take(extract_pair_bytes(N, K, M, pipeline != OZK_PIPE_ONDEVICE));
  // fold state between sweeps (on device the 2Sum state bounds every
  // order's; the host pipeline's FP64 orders keep one running sum), then the
  // partial sums of a K-split tail
  const size_t gb = round_up(gemm_workspace_bytes(N, M, pipeline, nhi, nlo,
                                                  pipeline == OZK_PIPE_ONDEVICE
                                                      ? OZK_ORDER_2SUM
                                                      : OZK_ORDER_HOST_JAX),
                             256) +
                    gemm_tail_bytes(N, M, K, pipeline, nhi, nlo, false, eb == 1);
  void* g = c.take(gb);
  if (a) *a = sa;
  if (b) *b = sb;
  if (tws) *tws = t;
  if (gws) *gws = g;
  if (gwsb) *gwsb = gb;
  return c.off;
}

size_t ozk_matmul_workspace_bytes(int64_t N, int64_t K, int64_t M,
                                  int pipeline, int n_hi, int n_lo) {
  return matmul_ws(N, K, M, pipeline, n_hi, n_lo, false, nullptr, nullptr,
                   nullptr, nullptr);
}

int ozk_matmul_plane_bytes(int pipeline, int64_t K, int n_hi, int n_lo) {
  clear_error();
  bool i8 = false;
  const int pipe = matmul_pipe(pipeline, K, n_hi, n_lo, &i8);
  const int rc = check_counts(pipe, n_hi, n_lo);
  if (rc) return rc;
  return i8 ? 1 : 2;
}

// After the kernels that set flags (the fill and the extraction), copy the
// flag word to host_flags and record `event`, when given: the caller can
// then read the flags without waiting for the GEMM queued behind.
static int flags_to_host(const uint32_t* flags, uint32_t* host_flags, void* event,
                         hipStream_t st) {
  if (!host_flags) return OZK_OK;
  OZK_HIP(hipMemcpyAsync(host_flags, flags, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  OZK_HIP(hipEventRecord((hipEvent_t)event, st));
  return OZK_OK;
}

static int matmul_call(const double* A, int64_t lda, const double* B, int64_t ldb,
                       double* C, int64_t ldc, int64_t N, int64_t K, int64_t M,
                       int pipeline, int n_hi, int n_lo, int order, void* workspace,
                       size_t workspace_bytes, uint32_t* flags, uint32_t* host_flags,
                       void* event, void* stream) {
  clear_error();
  hipStream_t st = (hipStream_t)stream;
  const int pipe_arg = pipeline;
  bool i8 = false;
  pipeline = matmul_pipe(pipeline, K, n_hi, n_lo, &i8);
  int rc = check_counts(pipeline, n_hi, n_lo);
  if (rc) return rc;
  if ((rc = check_order(order))) return rc;
  OZK_CHECK_ARG(N >= 0 && M >= 0 && K >= 1, "invalid shape N=%lld K=%lld M=%lld",
                (long long)N, (long long)K, (long long)M);
  OZK_CHECK_ARG((lda >= K || N <= 1) && (ldb >= M || K <= 1) &&
                    (ldc >= M || N <= 1),
                "leading dimension smaller than the row length");
  OZK_CHECK_ARG(flags, "null flags pointer");
  if ((rc = launch_fill_u32(flags, 0u, st))) return rc;
  if (N == 0 || M == 0) return flags_to_host(flags, host_flags, event, st);
  const size_t need = ozk_matmul_workspace_bytes(N, K, M, pipe_arg, n_hi, n_lo);
  if (!workspace || workspace_bytes < need) {
    set_error("matmul: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
    return OZK_ERR_WORKSPACE;
  }
  SliceSet sa, sb;
  void *tws, *gws;
  size_t gwsb;
  matmul_ws(N, K, M, pipe_arg, n_hi, n_lo, true, workspace, &sa, &sb, &tws, &gws,
            &gwsb);
  const size_t tbytes = extract_pair_bytes(N, K, M, pipeline != OZK_PIPE_ONDEVICE);
  int rho;
  if (pipeline == OZK_PIPE_ONDEVICE) {
    rho = rho_generic(K, 24);
    if ((rc = extract<float>(A, N, K, lda, 0, rho, n_hi, n_lo, sa.s, sa.e, flags,
                             tws, tbytes, st, i8, sa.sum)))
      return rc;
    if ((rc = extract<float>(B, K, M, ldb, 1, rho, n_hi, n_lo, sb.s, sb.e, flags,
                             tws, tbytes, st, i8, sb.sum)))
      return rc;
  } else {
    rho = rho_generic(K, 53);
    if ((rc = extract<double>(A, N, K, lda, 0, rho, n_hi, 0, sa.s, sa.e, flags,
                              tws, tbytes, st, false, nullptr)))
      return rc;
    if ((rc = extract<double>(B, K, M, ldb, 1, rho, n_hi, 0, sb.s, sb.e, flags,
                              tws, tbytes, st, false, nullptr)))
      return rc;
  }
  if ((rc = flags_to_host(flags, host_flags, event, st))) return rc;
  return launch_gemm(sa.s, sa.e, sb.s, sb.e, N, M, K, pipeline, n_hi, n_lo,
                     order, C, ldc, gws, gwsb, st, i8, rho, sa.sum, sb.sum);
}

int ozk_matmul(const double* A, int64_t lda, const double* B, int64_t ldb,
               double* C, int64_t ldc, int64_t N, int64_t K, int64_t M,
               int pipeline, int n_hi, int n_lo, int order, void* workspace,
               size_t workspace_bytes, uint32_t* flags, void* stream) {
  return matmul_call(A, lda, B, ldb, C, ldc, N, K, M, pipeline, n_hi, n_lo, order,
                     workspace, workspace_bytes, flags, nullptr, nullptr, stream);
}

int ozk_matmul_early_flags(const double* A, int64_t lda, const double* B, int64_t ldb,
                           double* C, int64_t ldc, int64_t N, int64_t K, int64_t M,
                           int pipeline, int n_hi, int n_lo, int order, void* workspace,
                           size_t workspace_bytes, uint32_t* flags, uint32_t* host_flags,
                           void* event, void* stream) {
  clear_error();
  OZK_CHECK_ARG(host_flags && event, "null host flag word or event");
  return matmul_call(A, lda, B, ldb, C, ldc, N, K, M, pipeline, n_hi, n_lo, order,
                     workspace, workspace_bytes, flags, host_flags, event, stream);
}

static size_t gram_ws(int64_t rows, int64_t cols, int nhi, int nlo, void* ws,
                      SliceSet* s, void** tws, void** gws = nullptr,
                      size_t* gwsb = nullptr) {
  Carver c(ws);
  SliceSet ss = carve_slices(c, nhi + nlo, cols, rows,
                             use_i8(OZK_PIPE_ONDEVICE, rows, nhi, nlo) ? 1 : 2);
  void* t = c.take(extract_workspace_bytes(rows, cols, 1, false));
  const bool i8 = use_i8(OZK_PIPE_ONDEVICE, rows, nhi, nlo);
  const size_t gb = round_up(gemm_workspace_bytes(cols, cols, OZK_PIPE_ONDEVICE, nhi, nlo,
                                                  OZK_ORDER_2SUM),
                             256) +
                    gemm_tail_bytes(cols, cols, rows, OZK_PIPE_ONDEVICE, nhi, nlo,
                                    gram_sym_supported(nhi, nlo), i8);
  void* g = c.take(gb);
  if (s) *s = ss;
  if (tws) *tws = t;
  if (gws) *gws = g;
  if (gwsb) *gwsb = gb;
  return c.off;
}

size_t ozk_gram_workspace_bytes(int64_t rows, int64_t cols, int n_hi,
                                int n_lo) {
  return gram_ws(rows, cols, n_hi, n_lo, nullptr, nullptr, nullptr);
}

static int gram_call(const double* A, int64_t lda, int64_t rows, int64_t cols, int n_hi,
                     int n_lo, double* G, int64_t ldg, void* workspace,
                     size_t workspace_bytes, uint32_t* flags, uint32_t* host_flags,
                     void* event, void* stream) {
  clear_error();
  hipStream_t st = (hipStream_t)stream;
  int rc = check_counts(OZK_PIPE_ONDEVICE, n_hi, n_lo);
  if (rc) return rc;
  OZK_CHECK_ARG(rows >= 1 && cols >= 0, "invalid shape rows=%lld cols=%lld",
                (long long)rows, (long long)cols);
  OZK_CHECK_ARG((lda >= cols || rows <= 1) && (ldg >= cols || cols <= 1),
                "leading dimension too small");
  OZK_CHECK_ARG(flags, "null flags pointer");
  if ((rc = launch_fill_u32(flags, 0u, st))) return rc;
  if (cols == 0) return flags_to_host(flags, host_flags, event, st);
  const size_t need = ozk_gram_workspace_bytes(rows, cols, n_hi, n_lo);
  if (!workspace || workspace_bytes < need) {
    set_error("gram: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
    return OZK_ERR_WORKSPACE;
  }
  SliceSet s;
  void *tws, *gws;
  size_t gwsb;
  gram_ws(rows, cols, n_hi, n_lo, workspace, &s, &tws, &gws, &gwsb);
  // Row extraction of A^T == column extraction of A: one set of slices is
  // both operands (gram.py:22-35 extracts the same values twice).
  const int rho = rho_generic(rows, 24);
  const bool i8 = use_i8(OZK_PIPE_ONDEVICE, rows, n_hi, n_lo);
  if ((rc = extract<float>(A, rows, cols, lda, 1, rho, n_hi, n_lo, s.s, s.e,
                           flags, tws, extract_workspace_bytes(rows, cols, 1, false), st,
                           i8, s.sum)))
    return rc;
  if ((rc = flags_to_host(flags, host_flags, event, st))) return rc;
  // high / medium: upper tiles only, the symmetrisation folded into the
  // epilogue.  max (three K sweeps): full product, then symmetrise.
  if (gram_sym_supported(n_hi, n_lo))
    return launch_gram_sym(s.s, s.e, cols, rows, n_hi, n_lo, G, ldg, gws, gwsb, st, i8,
                           rho, s.sum);
  if ((rc = launch_gemm(s.s, s.e, s.s, s.e, cols, cols, rows, OZK_PIPE_ONDEVICE,
                        n_hi, n_lo, OZK_ORDER_2SUM, G, ldg, gws, gwsb, st, i8, rho, s.sum,
                        s.sum)))
    return rc;
  hipLaunchKernelGGL(symmetrize_kernel, dim3(grid_for(cols * cols)), dim3(256),
                     0, st, G, cols, ldg);
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

int ozk_gram(const double* A, int64_t lda, int64_t rows, int64_t cols,
             int n_hi, int n_lo, double* G, int64_t ldg, void* workspace,
             size_t workspace_bytes, uint32_t* flags, void* stream) {
  return gram_call(A, lda, rows, cols, n_hi, n_lo, G, ldg, workspace, workspace_bytes,
                   flags, nullptr, nullptr, stream);
}

int ozk_gram_early_flags(const double* A, int64_t lda, int64_t rows, int64_t cols,
                         int n_hi, int n_lo, double* G, int64_t ldg, void* workspace,
                         size_t workspace_bytes, uint32_t* flags, uint32_t* host_flags,
                         void* event, void* stream) {
  clear_error();
  OZK_CHECK_ARG(host_flags && event, "null host flag word or event");
  return gram_call(A, lda, rows, cols, n_hi, n_lo, G, ldg, workspace, workspace_bytes,
                   flags, host_flags, event, stream);
}

// Residual workspace.  Up to 4 right-hand sides with K <= 16384 (presets
// high and medium) take the fused row kernels, which need none; otherwise A
// and x are extracted to planes for the slice GEMM, whose FP64 product y is
// subtracted from b afterwards.
static size_t residual_ws(int64_t N, int64_t K, int64_t ncols, int nhi,
                          int nlo, void* ws, SliceSet* a, SliceSet* x,
                          double** y, void** tws, void** gws = nullptr,
                          size_t* gwsb = nullptr) {
  Carver c(ws);
  const size_t eb = use_i8(OZK_PIPE_ONDEVICE, K, nhi, nlo) ? 1 : 2;
  if (residual_rows_supported(K, ncols, nhi, nlo)) return 0;
  SliceSet sa = carve_slices(c, nhi + nlo, N, K, eb);
  SliceSet sx = carve_slices(c, nhi + nlo, ncols, K, eb);
  double* yy = (double*)c.take((size_t)N * ncols * sizeof(double));
  void* t = c.take(extract_pair_bytes(N, K, ncols, false));
  const size_t gb = gemm_workspace_bytes(N, ncols, OZK_PIPE_ONDEVICE, nhi, nlo,
                                         OZK_ORDER_2SUM);
  void* g = c.take(gb);
  if (a) *a = sa;
  if (x) *x = sx;
  if (y) *y = yy;
  if (tws) *tws = t;
  if (gws) *gws = g;
  if (gwsb) *gwsb = gb;
  return c.off;
}

size_t ozk_residual_workspace_bytes(int64_t N, int64_t K, int64_t ncols,
                                    int n_hi, int n_lo) {
  return residual_ws(N, K, ncols, n_hi, n_lo, nullptr, nullptr, nullptr,
                     nullptr, nullptr);
}

int ozk_residual(const double* A, int64_t lda, const double* x, int64_t ldx,
                 const double* b, int64_t ldb, double* r, int64_t ldr,
                 int64_t N, int64_t K, int64_t ncols, int n_hi, int n_lo,
                 void* workspace, size_t workspace_bytes, uint32_t* flags,
                 void* stream) {
  clear_error();
  hipStream_t st = (hipStream_t)stream;
  int rc = check_counts(OZK_PIPE_ONDEVICE, n_hi, n_lo);
  if (rc) return rc;
  OZK_CHECK_ARG(N >= 0 && K >= 1 && ncols >= 0, "invalid shape");
  OZK_CHECK_ARG((lda >= K || N <= 1) && (ldx >= ncols || K <= 1) &&
                    (ldb >= ncols || N <= 1) && (ldr >= ncols || N <= 1),
                "leading dimension too small");
  OZK_CHECK_ARG(flags, "null flags pointer");
  if (N == 0 || ncols == 0) return launch_fill_u32(flags, 0u, st);
  const size_t need = ozk_residual_workspace_bytes(N, K, ncols, n_hi, n_lo);
  if (need && (!workspace || workspace_bytes < need)) {
    set_error("residual: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
    return OZK_ERR_WORKSPACE;
  }
  const int rho = rho_generic(K, 24);
  if (residual_rows_supported(K, ncols, n_hi, n_lo))  // clears and sets flags
    return launch_residual_rows(A, N, K, lda, x, ldx, b, ldb, r, ldr, ncols, rho, n_hi,
                                n_lo, flags, st);
  SliceSet sa, sx;
  double* y;
  void *tws, *gws;
  size_t gwsb;
  residual_ws(N, K, ncols, n_hi, n_lo, workspace, &sa, &sx, &y, &tws, &gws, &gwsb);
  if ((rc = launch_fill_u32(flags, 0u, st))) return rc;
  const bool i8 = use_i8(OZK_PIPE_ONDEVICE, K, n_hi, n_lo);
  const size_t tbytes = extract_pair_bytes(N, K, ncols, false);
  if ((rc = extract<float>(x, K, ncols, ldx, 1, rho, n_hi, n_lo, sx.s, sx.e,
                           flags, tws, tbytes, st, i8, sx.sum)))
    return rc;
  if ((rc = extract<float>(A, N, K, lda, 0, rho, n_hi, n_lo, sa.s, sa.e, flags,
                           tws, tbytes, st, i8, sa.sum)))
    return rc;
  if ((rc = launch_gemm(sa.s, sa.e, sx.s, sx.e, N, ncols, K, OZK_PIPE_ONDEVICE,
                        n_hi, n_lo, OZK_ORDER_2SUM, y, ncols, gws, gwsb, st, i8, rho,
                        sa.sum, sx.sum)))
    return rc;
  hipLaunchKernelGGL(sub_from_kernel, dim3(grid_for(N * ncols)), dim3(256), 0,
                     st, b, ldb, y, ncols, r, ldr, N, ncols);
  OZK_LAUNCH_CHECK();
  return OZK_OK;
}

int64_t ozk_lu_factor_max_n(void) { return lu_factor_max_n(); }

size_t ozk_lu_factor_workspace_bytes(int64_t n) {
  return n > 0 ? lu_factor_workspace_bytes() : 0;
}

int ozk_lu_factor_f32(float* A, int64_t lda, int64_t n, int32_t* perm,
                      void* workspace, size_t workspace_bytes, uint32_t* flags,
                      void* stream) {
  clear_error();
  hipStream_t st = (hipStream_t)stream;
  OZK_CHECK_ARG(n >= 0, "invalid shape");
  OZK_CHECK_ARG(lda >= n || n <= 1, "leading dimension too small");
  OZK_CHECK_ARG(flags, "null flags pointer");
  if (n > lu_factor_max_n()) {
    set_error("lu_factor: n = %lld above the %lld rows a panel holds", (long long)n,
              (long long)lu_factor_max_n());
    return OZK_ERR_UNSUPPORTED;
  }
  int rc = launch_fill_u32(flags, 0u, st);
  if (rc || n == 0) return rc;
  OZK_CHECK_ARG(A && perm, "null pointer");
  const size_t need = ozk_lu_factor_workspace_bytes(n);
  if (!workspace || workspace_bytes < need) {
    set_error("lu_factor: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    return OZK_ERR_WORKSPACE;
  }
  return launch_lu_factor(A, lda, n, perm, workspace, flags, st);
}

size_t ozk_lu_solve_workspace_bytes(int64_t n, int64_t ncols) {
  if (n <= 0 || ncols <= 0) return 0;
  return lu_solve_workspace_bytes(n, ncols);
}

int ozk_lu_solve_f32(const float* LU, int64_t lda, const int32_t* perm,
                     int64_t n, const double* B, int64_t ldb, double* X,
                     int64_t ldx, int64_t ncols, void* workspace,
                     size_t workspace_bytes, uint32_t* flags, void* stream) {
  clear_error();
  hipStream_t st = (hipStream_t)stream;
  OZK_CHECK_ARG(n >= 0 && ncols >= 0, "invalid shape");
  OZK_CHECK_ARG(n <= INT32_MAX, "n above the int32 row indices of perm");
  OZK_CHECK_ARG((lda >= n || n <= 1) && (ldb >= ncols || n <= 1) &&
                    (ldx >= ncols || n <= 1),
                "leading dimension too small");
  OZK_CHECK_ARG(flags, "null flags pointer");
  int rc = launch_fill_u32(flags, 0u, st);
  if (rc || n == 0 || ncols == 0) return rc;
  OZK_CHECK_ARG(LU && perm && B && X, "null pointer");
  const size_t need = ozk_lu_solve_workspace_bytes(n, ncols);
  if (!workspace || workspace_bytes < need) {
    set_error("lu_solve: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
    return OZK_ERR_WORKSPACE;
  }
  OZK_CHECK_ARG((uintptr_t)workspace % 8 == 0, "workspace not 8-byte aligned");
  return launch_lu_solve(LU, lda, perm, n, B, ldb, X, ldx, ncols, workspace, flags, st);
}

int ozk_pivots_to_perm(const int32_t* ipiv, int64_t n, int32_t* perm) {
  clear_error();
  OZK_CHECK_ARG(n >= 0 && n <= INT32_MAX, "invalid size");
  OZK_CHECK_ARG(n == 0 || (ipiv && perm), "null pointer");
  for (int64_t i = 0; i < n; ++i) perm[i] = (int32_t)i;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t p = (int64_t)ipiv[i] - 1;
    OZK_CHECK_ARG(p >= i && p < n, "pivot %lld of step %lld outside [%lld, %lld)",
                  (long long)p, (long long)i, (long long)i, (long long)n);
    const int32_t s = perm[i];
    perm[i] = perm[p];
    perm[p] = s;
  }
  return OZK_OK;
}

int ozk_check_finite(const double* X, int64_t rows, int64_t cols, int64_t ld,
                     uint32_t* flags, void* stream) {
  clear_error();
  OZK_CHECK_ARG(rows >= 0 && cols >= 0, "negative shape");
  OZK_CHECK_ARG(flags, "null flags pointer");
  return launch_check_finite(X, rows, cols, ld, flags, (hipStream_t)stream);
}

int ozk_probe_mfma_layout(int32_t* out, void* stream) {
  clear_error();
  OZK_CHECK_ARG(out, "null pointer");
  return launch_probe_mfma(out, (hipStream_t)stream);
}

}  // extern "C"
