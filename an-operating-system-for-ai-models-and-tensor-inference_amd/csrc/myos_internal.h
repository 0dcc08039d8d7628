// Internal launcher API between the kernel translation unit (myos_kernels.hip)
// and the host code (op tier, model tier). Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace myos {

// ---- GEMV family: one launch streams a row-major BF16 matrix once ----------
// X_NORM: x goes through the RMSNorm with gains `gamma` as it is staged
enum GemvX { X_PLAIN = 0, X_NORM = 1 };
enum GemvEpi { EPI_STORE = 0, EPI_RESID = 1, EPI_QKV = 2, EPI_GU = 3, EPI_HEAD = 4 };

struct GemvArgs {
  const uint16_t *w = nullptr;  // [m, k]
  const float *x = nullptr;     // [k]
  const uint16_t *gamma = nullptr;  // X_NORM gains [k]
  float eps = 0.f;
  int m = 0, k = 0;
  float *y = nullptr;           // STORE/HEAD: out[m]; RESID: residual[m] += row
  float *normed_out = nullptr;  // X_NORM: block 0 also writes the normed vector here
  // EPI_QKV: rows permuted so RoPE pairs (p, p + d/2) are adjacent
  const float *bias = nullptr;  // f32 [m] in the permuted row order
  const float2 *rope = nullptr; // [max_seq][d/2] (cos, sin)
  const uint32_t *pos_ptr = nullptr;  // device position (decode state)
  float *q_out = nullptr;       // [q_dim], natural order
  void *kc = nullptr, *vc = nullptr;  // this layer's cache [nkv][max_seq][d]
  int kv_bf16 = 0, max_seq = 0, q_dim = 0, kv_dim = 0, head_dim = 0;
  // EPI_GU: rows (2i, 2i+1) = (gate_i, up_i); h[i] = silu(gate_i) * up_i
  float *h_out = nullptr;
  // EPI_HEAD: per-block (value, index) argmax partials
  float2 *part = nullptr;       // x = value, y = index bits
  int part_cap = 0;             // entries `part` holds; a larger grid is refused
  uint32_t *pos_inc = nullptr;  // EPI_HEAD: block 0 increments *pos_inc when set
};

// Launch the best kernel variant for (m, k, x mode, epilogue); returns the
// number of argmax partials written (EPI_HEAD) or 0.
hipError_t launch_gemv(const GemvArgs &a, GemvX xm, GemvEpi epi, hipStream_t s,
                       int *n_parts = nullptr);
int gemv_head_parts(int m, int k);  // partial count EPI_HEAD will produce

// ---- decode attention over the HBM cache (split positions + last-block merge)
struct AttnDecodeArgs {
  const float *q;          // [nq, d] (RoPE applied)
  const void *kc, *vc;     // this layer's cache [nkv][max_seq][d]
  int kv_bf16, max_seq, nq, nkv, head_dim;
  const uint32_t *pos_ptr; // attends positions 0..*pos_ptr
  float *part;             // out: [nq][nchunks][d + 2] per-chunk (o[d], m, l)
  float *att;              // out: [nq * d] the merged attention output
  int *cnt;                // [nkv] zero between launches: chunks finished per group
};
int attn_decode_chunks(int max_seq, int head_dim);
size_t attn_decode_part_floats(int nq, int max_seq, int head_dim);
hipError_t launch_attn_decode(const AttnDecodeArgs &a, hipStream_t s);

// ---- small ops --------------------------------------------------------------
hipError_t launch_fill_zero(float *y, size_t n, hipStream_t s);
// recompute NaN outputs of Y[batch, m] = X W^T as the reference's f32 chain
hipError_t launch_gemm_nan_repair(float *y, const uint16_t *w, const float *x, int batch, int m, int k,
                                  hipStream_t s);
hipError_t launch_add_bias(float *y, const uint16_t *b, size_t n, hipStream_t s);
hipError_t launch_embed_gather(float *out, const uint16_t *table, size_t hidden,
                               const uint32_t *token_dev, uint32_t token_host, hipStream_t s);
hipError_t launch_rmsnorm(float *y, const uint16_t *g, const float *x, size_t n, float eps,
                          hipStream_t s);
hipError_t launch_rope_apply(float *x, size_t len, size_t head_dim, const float2 *cs,
                             hipStream_t s);
hipError_t launch_gqa_general(float *y, const float *q, const float *k, const float *v,
                              float *probs, float *scratch, int nq, int nkv, int d, int seq,
                              int mask, size_t query_pos, hipStream_t s);
hipError_t launch_swiglu_mul(float *h, const float *g, const float *u, size_t n, hipStream_t s);
hipError_t launch_rmsnorm_f32(float *y, const float *g, const float *x, size_t n, float eps,
                              hipStream_t s);
hipError_t launch_silu(float *y, const float *z, size_t n, hipStream_t s);
int argmax_parts(size_t n);
hipError_t launch_argmax_partial(const float *logits, size_t n, float2 *part, hipStream_t s);

// final argmax reduction; optionally also the decode-step prologue:
// token -> state[1], out_ids[state[2]++] = token, x = embed[token]
struct ArgmaxFinalArgs {
  const float2 *part = nullptr;
  int nparts = 0;
  uint32_t *token_out = nullptr;       // plain result
  // [pos, token, step, mode]; mode 0 = feed the argmax, 1 = feed state[1],
  // 2 = feed force[step] (the argmax is still recorded in out_ids[step])
  uint32_t *state = nullptr;
  uint32_t *out_ids = nullptr;
  const uint32_t *force = nullptr;
  const uint16_t *embed = nullptr;
  float *x = nullptr;
  int hidden = 0;
  uint32_t vocab = 0;                  // indices >= vocab (none found) select id 0
};
hipError_t launch_argmax_final(const ArgmaxFinalArgs &a, hipStream_t s);

// ---- prefill ----------------------------------------------------------------
hipError_t launch_embed_rows(float *X, const uint16_t *embed, const uint32_t *tokens, int M,
                             int H, hipStream_t s);
// rows of X -> rmsnorm -> bf16 hi/lo planes (A operand of the MFMA GEMM)
hipError_t launch_rmsnorm_rows_split(const float *X, const uint16_t *g, float eps, int M, int H,
                                     uint16_t *hi, uint16_t *lo, hipStream_t s);
hipError_t launch_split_rows(const float *X, size_t n, uint16_t *hi, uint16_t *lo,
                             hipStream_t s);

struct GemmArgs {
  const uint16_t *a_hi, *a_lo;  // [M, K] bf16 planes
  const uint16_t *w;            // [N, K] bf16
  int M, N, K;
  float *y;                     // STORE: [M, N]; RESID: [M, N] +=
  // EPI_QKV (N = q_dim + 2 kv_dim, permuted rows)
  const float *bias;
  const float2 *rope;
  int start_pos;
  float *q_out;                 // [M, q_dim]
  void *kc, *vc;
  int kv_bf16, max_seq, q_dim, kv_dim, head_dim;
  // EPI_GU: writes h = silu(g)*u as hi/lo planes [M, N/2]
  uint16_t *h_hi, *h_lo;
  // K-split partials [splits][M][N] f32 (gemm_ws_floats); null: one split
  float *ws;
  size_t ws_cap;               // floats at ws
  int kps;                     // set by the launcher: K steps per split
};
// Launch plan of the pipelined MFMA GEMM: tile shape (cfg 0..3 = 128 x 32,
// 64, 128, 256) and K splits; cfg -1 takes the single-stage 128 x 64 kernel
// (shapes the pipelined one does not take, and wide short-K projections)
struct GemmPlan {
  int cfg = -1;
  int splits = 1;
};
GemmPlan pf_plan(int M, int N, int K);
// force every later plan to (cfg, splits); cfg < 0 restores the planner
void gemm_force_plan(int cfg, int splits);
// the partial-buffer floats launch_gemm needs for this shape (0: one split)
size_t gemm_ws_floats(int M, int N, int K);
hipError_t launch_gemm(const GemmArgs &a, GemvEpi epi, hipStream_t s);
// EPI_RESID GEMM (y += A W^T) followed by the RMSNorm of y with gains g into
// bf16 hi/lo planes, the split-K reduction and the norm in one pass when the
// shape allows (else launch_gemm + launch_rmsnorm_rows_split)
hipError_t launch_gemm_resid_norm(const GemmArgs &a, const uint16_t *g, float eps, uint16_t *hi,
                                  uint16_t *lo, hipStream_t s);

struct AttnPrefillArgs {
  const float *q;               // [M, nq*d]
  const void *kc, *vc;
  int kv_bf16, max_seq, nq, nkv, head_dim, M, start_pos;
  uint16_t *out_hi, *out_lo;    // [M, nq*d]
  float *part = nullptr;        // key-split partials (head_dim 128), part_cap floats
  size_t part_cap = 0;
};
hipError_t launch_attn_prefill(const AttnPrefillArgs &a, hipStream_t s);
// floats of the key-split partials for M queries of nq heads in ns splits
inline size_t attn_prefill_part_floats(int nq, int M, int ns) {
  return (size_t)nq * ns * M * (128 + 2);
}

hipError_t launch_permute_rows(uint16_t *dst, const uint16_t *src, const int *perm, int rows,
                               int cols, hipStream_t s);

// ---- persistent decode (myos_persistent.hip) ---------------------------------
// One cooperative launch runs `steps` greedy decode steps. Workgroups hand
// activations to each other as 64-bit (value, tag) words written and read with
// device-coherent (sc1) accesses; a consumer waits for exactly the words it
// needs to carry the expected tag, so there is no grid barrier or fence.
struct PersistLayer {
  const uint16_t *ln1, *wqkv, *wo, *ln2, *wgu, *wd;
  const float *bqkv;
  // down as column pairs [I/2][H]: word (j, r) = (wd[r][2j], wd[r][2j+1])
  const uint32_t *wdp;
};
struct PersistArgs {
  int H, I, V, L, nq, nkv, d, max_seq, qkv_rows;
  float eps;
  const PersistLayer *layers;  // device array [L]
  const uint16_t *embed, *final_norm, *head;
  const float2 *rope;
  float *kc, *vc;              // f32 cache base, layer stride = layer_kv
  size_t layer_kv;
  // tagged exchange buffers (zeroed once; tags only grow)
  uint64_t *tq, *tkv, *tpart, *tatt, *txo, *txd, *targ;
  uint64_t *tpr;               // down partials, [owner][grid][rows per owner]
  // outputs
  float *logits, *normed, *x_out;
  float2 *part_out;
  int part_cap;
  const float2 *part_in;       // argmax partials of the forward before the launch
  int nparts_in;
  uint32_t *state, *out_ids;
  const uint32_t *force;       // non-null: step s feeds force[s] (out_ids[s] keeps the argmax)
  uint32_t *err;
  uint32_t tag_base, steps, pos0;
  int lds_wd;                  // set by the launcher: LDS offset (floats) of the down block
  int kv_bf16;                 // the cache at kc / vc holds bf16
  uint64_t *trace;             // optional [grid][5 L + 3] phase timestamps of one step
  uint32_t trace_step;
  // streamed kernel: f32 activation buffers (wide_buffer_floats) and one
  // barrier flag word per workgroup, kWFlagStride words apart (zeroed once;
  // tags only grow)
  float *wide;
  uint64_t *wflags;
};
// words between two workgroups' barrier flags: one flag per 128-byte line, so
// flags published at the same moment do not queue on a shared line
constexpr int kWFlagStride = 16;
int persist_grid();                       // workgroups per launch
int persist_tags_per_step(int layers);
size_t persist_part_words(int nq, int max_seq, int d);
size_t persist_pr_words(int H, int nq);
bool persist_supported(int H, int I, int qdim, int d, int gq);
bool persist_device_ok(const PersistArgs &a);  // shape, LDS and the current device fit
hipError_t launch_decode_persistent(const PersistArgs &a, hipStream_t s);
// first-use set-up of the instantiation a launch with these arguments takes
// (launches do it themselves when it has not been done)
hipError_t persist_prepare(const PersistArgs &a);
// one empty cooperative launch on s (and a wait for it): the runtime's set-up
// for a stream's first cooperative launch
hipError_t coop_warm_launch(hipStream_t s);
// the streamed cooperative kernel, for layers larger than the chip holds
bool wide_supported(int H, int I, int qdim, int d, int gq, int max_seq);
size_t wide_buffer_floats(int H, int I, int nq, int d, int max_seq);
bool wide_device_ok(const PersistArgs &a);
hipError_t launch_decode_wide(const PersistArgs &a, hipStream_t s);
hipError_t wide_prepare(const PersistArgs &a);

// dst[c][r] = src[r][c] for a [rows, cols] matrix of 32-bit words
hipError_t launch_transpose_u32(uint32_t *dst, const uint32_t *src, int rows, int cols,
                                hipStream_t s);

const char *kernel_build_info();

}  // namespace myos
