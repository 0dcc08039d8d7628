// Op tier of the C ABI: the tensor_core functions on device pointers.
// Every check the reference makes on its slices runs here, on the host, in
// the reference's order, before any launch; so a non-zero status means no
// output was touched (bf16.rs:36-38, gqa.rs:132-135, rope.rs:68-71).
#include <hip/hip_runtime.h>
#include <math.h>

#include <vector>

#include "../../include/myos_hip.h"
#include "myos_internal.h"

using namespace myos;

namespace {
inline hipStream_t S(myos_stream_t s) { return (hipStream_t)s; }
inline int hip_status(hipError_t e) { return e == hipSuccess ? MYOS_OK : MYOS_E_HIP; }
inline bool mul_ok(size_t a, size_t b, size_t *out) {
  if (a && b > SIZE_MAX / a) return false;
  *out = a * b;
  return true;
}
}  // namespace

extern "C" {

const char *myos_strerror(int status) {
  switch (status) {
    case MYOS_OK: return "ok";
    case MYOS_E_SHAPE: return "shape does not match the buffers";
    case MYOS_E_TOKEN: return "token id is out of range";
    case MYOS_E_ROW_OOB: return "bf16 row is out of bounds";
    case MYOS_E_POSITION: return "position does not match the kv cursor";
    case MYOS_E_KV_FULL: return "kv cache is full";
    case MYOS_E_KV_RANGE: return "kv index is out of range";
    case MYOS_E_W_MISSING: return "tensor not found";
    case MYOS_E_W_DTYPE: return "tensor dtype is not bf16";
    case MYOS_E_W_SHAPE: return "tensor shape does not match the layout";
    case MYOS_E_W_LENGTH: return "tensor byte length does not match shape";
    case MYOS_E_IO: return "weights file could not be opened or mapped";
    case MYOS_E_PARSE: return "weight buffer could not be parsed";
    case MYOS_E_HIP: return "HIP runtime error";
    case MYOS_E_ARG: return "invalid argument";
    case MYOS_E_SCRATCH: return "call needs more than the static scratch of the no-allocation entry point";
    default: return "unknown status";
  }
}

const char *myos_build_info(void) { return kernel_build_info(); }

int myos_stream_sync(myos_stream_t stream) {
  return hip_status(hipStreamSynchronize(S(stream)));
}

// bf16.rs:94-122
int myos_gemv_bf16(float *y, size_t y_len, const uint16_t *w, size_t w_len, const float *x,
                   size_t x_len, size_t m, size_t k, myos_stream_t stream) {
  if (y_len != m || x_len != k) return MYOS_E_SHAPE;
  if (k == 0) {
    if (w_len != 0) return MYOS_E_SHAPE;
    return hip_status(launch_fill_zero(y, m, S(stream)));
  }
  if (w_len / k < m) return MYOS_E_ROW_OOB;
  size_t need;
  if (!mul_ok(m, k, &need) || w_len != need) return MYOS_E_SHAPE;
  if (m == 0) return MYOS_OK;
  if (m > INT32_MAX || k > INT32_MAX) return MYOS_E_SHAPE;
  GemvArgs a;
  a.w = w;
  a.x = x;
  a.m = (int)m;
  a.k = (int)k;
  a.y = y;
  return hip_status(launch_gemv(a, X_PLAIN, EPI_STORE, S(stream)));
}

// gemm_bf16.rs:73-110 (the scratch argument is internal here)
int myos_gemm_bf16(float *y, size_t y_len, const uint16_t *w, size_t w_len, const float *x,
                   size_t x_len, size_t batch, size_t m, size_t k, myos_stream_t stream) {
  size_t y_need, x_need, w_need;
  if (!mul_ok(batch, m, &y_need) || !mul_ok(batch, k, &x_need) || !mul_ok(m, k, &w_need))
    return MYOS_E_SHAPE;
  if (y_len != y_need || x_len != x_need || w_len != w_need) return MYOS_E_SHAPE;
  if (m == 0 || batch == 0) return MYOS_OK;
  if (k == 0) return hip_status(launch_fill_zero(y, y_need, S(stream)));
  if (batch > INT32_MAX || m > INT32_MAX || k > INT32_MAX) return MYOS_E_SHAPE;
  hipStream_t s = S(stream);
  uint16_t *hi = nullptr, *lo = nullptr;
  if (hipMallocAsync((void **)&hi, x_need * 2, s) != hipSuccess) return MYOS_E_HIP;
  if (hipMallocAsync((void **)&lo, x_need * 2, s) != hipSuccess) {
    (void)hipFreeAsync(hi, s);
    return MYOS_E_HIP;
  }
  // partials of the K splits (none when the grid already fills the device)
  const size_t wsf = gemm_ws_floats((int)batch, (int)m, (int)k);
  float *ws = nullptr;
  if (wsf && hipMallocAsync((void **)&ws, wsf * 4, s) != hipSuccess) {
    (void)hipFreeAsync(hi, s);
    (void)hipFreeAsync(lo, s);
    return MYOS_E_HIP;
  }
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
  hipError_t f1 = hipFreeAsync(hi, s), f2 = hipFreeAsync(lo, s);
  hipError_t f3 = ws ? hipFreeAsync(ws, s) : hipSuccess;
  if (e == hipSuccess) e = f1 != hipSuccess ? f1 : f2 != hipSuccess ? f2 : f3;
  return hip_status(e);
}

// bf16.rs:147-158
int myos_add_bf16_bias(float *y, size_t y_len, const uint16_t *bias, size_t bias_len,
                       myos_stream_t stream) {
  if (bias_len != y_len) return MYOS_E_SHAPE;
  if (y_len == 0) return MYOS_OK;
  return hip_status(launch_add_bias(y, bias, y_len, S(stream)));
}

// bf16.rs:165-198
int myos_embed_gather_bf16(float *out, size_t out_len, const uint16_t *table, size_t table_len,
                           size_t vocab, size_t hidden, uint32_t token, myos_stream_t stream) {
  if (out_len != hidden) return MYOS_E_SHAPE;
  if ((size_t)token >= vocab) return MYOS_E_TOKEN;
  size_t start, end, need;
  if (!mul_ok((size_t)token, hidden, &start)) return MYOS_E_SHAPE;
  end = start + hidden;
  if (end > table_len) return MYOS_E_ROW_OOB;
  if (!mul_ok(vocab, hidden, &need) || table_len != need) return MYOS_E_SHAPE;
  if (hidden == 0) return MYOS_OK;
  return hip_status(launch_embed_gather(out, table, hidden, nullptr, token, S(stream)));
}

// bf16.rs:231-249
int myos_rmsnorm_bf16_weight(float *y, size_t y_len, const uint16_t *weight, size_t weight_len,
                             const float *x, size_t x_len, float eps, myos_stream_t stream) {
  if (x_len == 0 || y_len != x_len) return MYOS_E_SHAPE;
  if (weight_len != x_len) return MYOS_E_SHAPE;
  return hip_status(launch_rmsnorm(y, weight, x, x_len, eps, S(stream)));
}

// rope.rs:119-184. The table of (cos, sin) per pair is evaluated here with the
// reference's own expression and libm calls, so angles are bit-identical.
int myos_rope_f32_inplace(float *x, size_t len, uint32_t position, size_t head_dim, float theta,
                          myos_stream_t stream) {
  if (head_dim == 0 || head_dim % 2 != 0) return MYOS_E_SHAPE;
  if (len == 0 || len % head_dim != 0) return MYOS_E_SHAPE;
  const size_t half = head_dim / 2;
  std::vector<float2> cs(half);
  const float posf = (float)position;
  for (size_t p = 0; p < half; p++) {
    const float e = (float)(2 * p) / (float)head_dim;
    const float inv = 1.0f / powf(theta, e);
    const float ang = posf * inv;
    cs[p] = make_float2(cosf(ang), sinf(ang));
  }
  hipStream_t s = S(stream);
  float2 *dcs = nullptr;
  if (hipMallocAsync((void **)&dcs, half * sizeof(float2), s) != hipSuccess) return MYOS_E_HIP;
  hipError_t e = hipMemcpyAsync(dcs, cs.data(), half * sizeof(float2), hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = launch_rope_apply(x, len, head_dim, dcs, s);
  // the host table must outlive the copy
  hipError_t sy = hipStreamSynchronize(s);
  hipError_t f = hipFreeAsync(dcs, s);
  if (e == hipSuccess) e = sy != hipSuccess ? sy : f;
  return hip_status(e);
}

// gqa.rs:174-264
int myos_gqa_attn_f32(float *y, size_t y_len, const float *q, size_t q_len, const float *k,
                      size_t k_len, const float *v, size_t v_len, float *probs,
                      size_t probs_len, size_t num_q_heads, size_t num_kv_heads,
                      size_t head_dim, size_t seq_len, int mask, size_t query_pos,
                      myos_stream_t stream) {
  if (mask != 0 && mask != 1) return MYOS_E_ARG;
  if (!num_q_heads || !num_kv_heads || !head_dim || !seq_len) return MYOS_E_SHAPE;
  if (num_q_heads % num_kv_heads) return MYOS_E_SHAPE;
  size_t q_elems, kv_elems;
  if (!mul_ok(num_q_heads, head_dim, &q_elems)) return MYOS_E_SHAPE;
  if (!mul_ok(num_kv_heads, seq_len, &kv_elems) || !mul_ok(kv_elems, head_dim, &kv_elems))
    return MYOS_E_SHAPE;
  if (y_len != q_elems || q_len != q_elems || k_len != kv_elems || v_len != kv_elems)
    return MYOS_E_SHAPE;
  if (probs_len != seq_len) return MYOS_E_SHAPE;
  if (num_q_heads > INT32_MAX || seq_len > INT32_MAX || head_dim > INT32_MAX)
    return MYOS_E_SHAPE;
  hipStream_t s = S(stream);
  size_t scr_elems;
  if (!mul_ok(num_q_heads, seq_len, &scr_elems)) return MYOS_E_SHAPE;
  float *scr = nullptr;
  if (hipMallocAsync((void **)&scr, scr_elems * sizeof(float), s) != hipSuccess)
    return MYOS_E_HIP;
  hipError_t e = launch_gqa_general(y, q, k, v, probs, scr, (int)num_q_heads, (int)num_kv_heads,
                                    (int)head_dim, (int)seq_len, mask, query_pos, s);
  hipError_t f = hipFreeAsync(scr, s);
  return hip_status(e != hipSuccess ? e : f);
}

// swiglu.rs:125-131
int myos_swiglu_mul_f32(float *h, size_t h_len, const float *gate, size_t gate_len,
                        const float *up, size_t up_len, myos_stream_t stream) {
  if (gate_len == 0 || up_len != gate_len || h_len != gate_len) return MYOS_E_SHAPE;
  return hip_status(launch_swiglu_mul(h, gate, up, gate_len, S(stream)));
}

// swiglu.rs:184-213: gate = W_g x, up = W_u x, h = silu(gate) * up, y = W_d h
// (the three GEMVs and the product on the device; every check first, so on
// an error y, gate, up and h are unchanged)
int myos_swiglu_bf16(float *y, size_t y_len, const float *x, size_t x_len, const uint16_t *gate_w,
                     size_t gate_w_len, const uint16_t *up_w, size_t up_w_len, const uint16_t *down_w,
                     size_t down_w_len, float *gate, size_t gate_len, float *up, size_t up_len,
                     float *h, size_t h_len, size_t hidden, size_t intermediate,
                     myos_stream_t stream) {
  if (hidden == 0 || intermediate == 0) return MYOS_E_SHAPE;
  if (y_len != hidden || x_len != hidden) return MYOS_E_SHAPE;
  if (gate_len != intermediate || up_len != intermediate || h_len != intermediate) return MYOS_E_SHAPE;
  size_t wn;
  if (!mul_ok(hidden, intermediate, &wn)) return MYOS_E_SHAPE;
  if (gate_w_len != wn || up_w_len != wn || down_w_len != wn) return MYOS_E_SHAPE;
  if (hidden > INT32_MAX || intermediate > INT32_MAX) return MYOS_E_SHAPE;
  hipStream_t s = S(stream);
  GemvArgs a;
  a.x = x;
  a.k = (int)hidden;
  a.m = (int)intermediate;
  a.w = gate_w;
  a.y = gate;
  hipError_t e = launch_gemv(a, X_PLAIN, EPI_STORE, s);
  if (e == hipSuccess) {
    a.w = up_w;
    a.y = up;
    e = launch_gemv(a, X_PLAIN, EPI_STORE, s);
  }
  if (e == hipSuccess) e = launch_swiglu_mul(h, gate, up, intermediate, s);
  if (e == hipSuccess) {
    GemvArgs d;
    d.w = down_w;
    d.x = h;
    d.m = (int)hidden;
    d.k = (int)intermediate;
    d.y = y;
    e = launch_gemv(d, X_PLAIN, EPI_STORE, s);
  }
  return hip_status(e);
}

// swiglu.rs:113-115, elementwise: y[i] = z[i] / (1 + expf(-z[i]))
int myos_silu_f32(float *y, size_t y_len, const float *z, size_t z_len, myos_stream_t stream) {
  if (y_len != z_len) return MYOS_E_SHAPE;
  return hip_status(launch_silu(y, z, z_len, S(stream)));
}

// bf16.rs:200-216: rmsnorm_bf16_weight with an f32 gamma
int myos_rmsnorm_f32(float *y, size_t y_len, const float *weight, size_t weight_len, const float *x,
                     size_t x_len, float eps, myos_stream_t stream) {
  if (x_len == 0 || y_len != x_len || weight_len != x_len) return MYOS_E_SHAPE;
  return hip_status(launch_rmsnorm_f32(y, weight, x, x_len, eps, S(stream)));
}

// rope.rs:89-98: inv_freq[i] = 1 / powf(theta, f32(2 i) / f32(head_dim)),
// evaluated with the reference's expression and libm call (as the decode
// kernels' cos/sin tables are) and copied to the device
int myos_rope_inv_freqs(float *inv_freq, size_t len, size_t head_dim, float theta,
                        myos_stream_t stream) {
  if (head_dim == 0 || head_dim % 2 != 0 || len != head_dim / 2) return MYOS_E_SHAPE;
  std::vector<float> t(len);
  for (size_t i = 0; i < len; i++) t[i] = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
  hipStream_t s = S(stream);
  hipError_t e = hipMemcpyAsync(inv_freq, t.data(), len * sizeof(float), hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);  // the host table must outlive the copy
  return hip_status(e);
}

// gqa.rs:158-163: 1 / sqrtf(head_dim), the scale every attention kernel
// here multiplies a finished dot by
int myos_attn_scale_f32(size_t head_dim, float *out) {
  if (!out) return MYOS_E_ARG;
  if (head_dim == 0) return MYOS_E_SHAPE;
  *out = 1.0f / sqrtf((float)head_dim);
  return MYOS_OK;
}

// model_core/src/lib.rs:157-167
int myos_greedy_token(uint32_t *out, const float *logits, size_t n, myos_stream_t stream) {
  if (!out) return MYOS_E_ARG;
  hipStream_t s = S(stream);
  if (n == 0) return hip_status(hipMemsetAsync(out, 0, sizeof(uint32_t), s));
  if (n > UINT32_MAX) return MYOS_E_SHAPE;
  const int parts = argmax_parts(n);
  float2 *part = nullptr;
  if (hipMallocAsync((void **)&part, parts * sizeof(float2), s) != hipSuccess) return MYOS_E_HIP;
  hipError_t e = launch_argmax_partial(logits, n, part, s);
  if (e == hipSuccess) {
    ArgmaxFinalArgs a;
    a.part = part;
    a.nparts = parts;
    a.token_out = out;
    a.vocab = (uint32_t)n;
    e = launch_argmax_final(a, s);
  }
  hipError_t f = hipFreeAsync(part, s);
  return hip_status(e != hipSuccess ? e : f);
}

}  // extern "C"
