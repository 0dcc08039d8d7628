// gemm_bf16 without any allocation: myos_gemm_bf16_noalloc.
//
// myos_gemm_bf16 allocates its scratch on every call (the bf16 hi / lo planes
// of X and the f32 partials of the K splits, hipMallocAsync / hipFreeAsync).
// Callers that cannot allocate -- code under stream capture, tight serving
// loops -- use this variant instead: the same kernels, with the scratch in a
// file-scope device array of kScratchBytes per GPU, held until the process
// ends. Host code never passes the array's name to a kernel (on the host it
// is only a stand-in symbol): each device's address of it is looked up once
// with hipGetSymbolAddress, with that device current, and kept per device.
//
// Every call on one GPU shares that GPU's array; calls that overlap on one
// GPU (two streams, two threads) race on it. Nothing in it has to start at
// zero: each call writes every scratch word it reads (the split kernel both
// planes, each K split its own partial tile) before reading it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/myos_hip.h"
#include "myos_internal.h"

using namespace myos;

namespace {

constexpr size_t kScratchBytes = 32ull << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mu;
uint8_t *g_ptr[kMaxDevices] = {};

inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// this device's address of `scratch` (looked up on the device's first call)
int scratch_ptr(uint8_t **out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MYOS_E_HIP;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return MYOS_E_HIP;
    g_ptr[dev] = (uint8_t *)p;
  }
  *out = g_ptr[dev];
  return MYOS_OK;
}

inline bool mul_ok(size_t a, size_t b, size_t *out) {
  if (a && b > SIZE_MAX / a) return false;
  *out = a * b;
  return true;
}

}  // namespace

extern "C" {

size_t myos_gemm_bf16_noalloc_scratch(size_t batch, size_t m, size_t k) {
  if (!batch || !m || !k || batch > INT32_MAX || m > INT32_MAX || k > INT32_MAX) return 0;
  size_t x;
  if (!mul_ok(batch, k, &x) || x > SIZE_MAX / 4) return SIZE_MAX;
  return 2 * align256(x * 2) + align256(gemm_ws_floats((int)batch, (int)m, (int)k) * 4);
}

size_t myos_gemm_bf16_noalloc_max_scratch(void) { return kScratchBytes; }

// gemm_bf16, gemm_bf16.rs:73-110, with the same checks in the same order as
// myos_gemm_bf16, then MYOS_E_SCRATCH when the call needs more scratch than
// the static array holds
int myos_gemm_bf16_noalloc(float *y, size_t y_len, const uint16_t *w, size_t w_len,
                           const float *x, size_t x_len, size_t batch, size_t m, size_t k,
                           myos_stream_t stream) {
  size_t y_need, x_need, w_need;
  if (!mul_ok(batch, m, &y_need) || !mul_ok(batch, k, &x_need) || !mul_ok(m, k, &w_need))
    return MYOS_E_SHAPE;
  if (y_len != y_need || x_len != x_need || w_len != w_need) return MYOS_E_SHAPE;
  if (m == 0 || batch == 0) return MYOS_OK;
  hipStream_t s = (hipStream_t)stream;
  if (k == 0) return launch_fill_zero(y, y_need, s) == hipSuccess ? MYOS_OK : MYOS_E_HIP;
  if (batch > INT32_MAX || m > INT32_MAX || k > INT32_MAX) return MYOS_E_SHAPE;
  const size_t need = myos_gemm_bf16_noalloc_scratch(batch, m, k);
  if (need > kScratchBytes) return MYOS_E_SCRATCH;
  uint8_t *base = nullptr;
  int rc = scratch_ptr(&base);
  if (rc) return rc;
  uint16_t *hi = (uint16_t *)base;
  uint16_t *lo = (uint16_t *)(base + align256(x_need * 2));
  const size_t wsf = gemm_ws_floats((int)batch, (int)m, (int)k);
  float *ws = wsf ? (float *)(base + 2 * align256(x_need * 2)) : nullptr;
  hipError_t e = launch_split_rows(x, x_need, hi, lo, s);
  if (e == hipSuccess) {
    GemmArgs g{};
    g.a_hi = hi;
    g.a_lo = lo;
    g.w = w;
    g.M = (int)batch;
    g.N = (int)m;
    g.K = (int)k;
    g.y = y;
    g.ws = ws;
    g.ws_cap = wsf;
    e = launch_gemm(g, EPI_STORE, s);
    if (e == hipSuccess) e = launch_gemm_nan_repair(y, w, x, (int)batch, (int)m, (int)k, s);
  }
  return e == hipSuccess ? MYOS_OK : MYOS_E_HIP;
}

}  // extern "C"
