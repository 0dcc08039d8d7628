/*
 * myos_hip.h -- C ABI of the MI355X (gfx950) implementation of the reference's
 * batch-1 BF16-weight / FP32-accumulate token loop.
 *
 * Two tiers, both plain C: pointers + sizes + int status codes, no C++ or torch
 * types. A caller that binds the reference's Rust API (a cgo/ctypes/Rust
 * `extern "C"` block) maps one function to one reference function:
 *
 *  - op tier: the `tensor_core` re-exports (crates/tensor_core/src/lib.rs:54-74),
 *    on DEVICE pointers, asynchronous on the given HIP stream (NULL = default
 *    stream). Every slice argument of the reference (`&[u8]`, `&[f32]`) is a
 *    (pointer, element count) pair here, and the reference's length checks
 *    run on the host before anything is launched, so on a non-zero return no
 *    output has been written ("on Err, outputs unchanged", bf16.rs:36-38).
 *  - model tier: `model_core` (crates/model_core/src/lib.rs:21-26): KvCache +
 *    BlockWorkspace + prefill / forward_token / greedy_decode over weights read
 *    once from a BF16 SafeTensors file (qwen25_layout keys) into HBM. On a
 *    non-zero return the KV cursor has not moved (qwen25_block.rs:129-135).
 */
#ifndef MYOS_HIP_H
#define MYOS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: one per variant of the reference's error enums ---- */
enum {
  MYOS_OK = 0,
  MYOS_E_SHAPE = 1,        /* Bf16OpError::Shape, GqaError/RopeError/SwigluError::Shape,
                              BlockError::Shape, KvError::Shape */
  MYOS_E_TOKEN = 2,        /* Bf16OpError::TokenOutOfBounds, BlockError::Token */
  MYOS_E_ROW_OOB = 3,      /* Bf16OpError::RowOutOfBounds */
  MYOS_E_POSITION = 4,     /* BlockError::Position, AttnError::Position */
  MYOS_E_KV_FULL = 5,      /* KvError::Full */
  MYOS_E_KV_RANGE = 6,     /* KvError::Range */
  MYOS_E_W_MISSING = 7,    /* QwenBf16Error::Missing (weight_loader WeightError::NotFound) */
  MYOS_E_W_DTYPE = 8,      /* QwenBf16Error::DType */
  MYOS_E_W_SHAPE = 9,      /* QwenBf16Error::Shape */
  MYOS_E_W_LENGTH = 10,    /* QwenBf16Error::Length / WeightError::LengthMismatch */
  MYOS_E_IO = 11,          /* WeightFileError::Io */
  MYOS_E_PARSE = 12,       /* WeightError::Parse / Duplicate / EmptyName / UnsupportedDType */
  MYOS_E_HIP = 13,         /* a HIP runtime call failed (no reference counterpart) */
  MYOS_E_ARG = 14,         /* NULL handle or pointer, unknown enum value */
  MYOS_E_SCRATCH = 15,     /* a no-allocation call needs more than its static scratch
                              (no reference counterpart) */
};

typedef void *myos_stream_t; /* a hipStream_t */

/* Text for a status code (static storage). */
const char *myos_strerror(int status);
/* Build identification: target arch and kernel variant names. */
const char *myos_build_info(void);

/* ======================= op tier (tensor_core) ======================= */

/* gemv_bf16, crates/tensor_core/src/bf16.rs:80-122.
 * y[m] = W[m,k] x[k]; W row-major little-endian BF16 with w_len ELEMENTS
 * (the reference's byte length / 2; an odd byte count is not representable
 * here). Checks in the reference's order: y_len != m or x_len != k -> SHAPE;
 * k == 0: w_len != 0 -> SHAPE, else y = 0; w_len / k < m -> ROW_OOB;
 * w_len != m*k -> SHAPE. f32 accumulate (the per-row sum order differs from
 * the reference's serial chain; see the parity tolerance of the tests). */
int myos_gemv_bf16(float *y, size_t y_len, const uint16_t *w, size_t w_len, const float *x,
                   size_t x_len, size_t m, size_t k, myos_stream_t stream);

/* gemm_bf16, crates/tensor_core/src/gemm_bf16.rs:51-110 (prefill projection).
 * Y[batch,m] = X[batch,k] W[m,k]^T on MFMA (v_mfma_f32_32x32x16_bf16) with X
 * split into two BF16 terms (hi + lo) so the f32 activations keep ~16 mantissa
 * bits. The reference's caller-provided scratch is internal here. */
int myos_gemm_bf16(float *y, size_t y_len, const uint16_t *w, size_t w_len, const float *x,
                   size_t x_len, size_t batch, size_t m, size_t k, myos_stream_t stream);

/* myos_gemm_bf16 without any allocation. No counterpart in the reference:
 * this is for callers that cannot allocate device memory (code under stream
 * capture, tight serving loops). Same arguments, checks, kernels and results
 * (bit for bit) as myos_gemm_bf16, whose scratch (the bf16 hi / lo planes of
 * X and the K-split partials) comes instead from one static device array of
 * myos_gemm_bf16_noalloc_max_scratch() bytes (32 MiB) per GPU, held until
 * the process ends. A call needing more (myos_gemm_bf16_noalloc_scratch)
 * returns MYOS_E_SCRATCH before anything is launched. All calls on one GPU
 * share that GPU's array: calls that overlap on one GPU race. The first call
 * on a device resolves the array's address (hipGetSymbolAddress) and sets the
 * tile kernels' LDS limits, which stream capture does not record: make one
 * call outside capture on each device before capturing this entry point.
 * Outputs that come out NaN (an infinite weight times a zero activation
 * part) are recomputed as the reference's f32 chain, as in myos_gemm_bf16. */
int myos_gemm_bf16_noalloc(float *y, size_t y_len, const uint16_t *w, size_t w_len,
                           const float *x, size_t x_len, size_t batch, size_t m, size_t k,
                           myos_stream_t stream);
/* Scratch bytes a myos_gemm_bf16_noalloc call of this shape needs (0 when it
 * launches nothing), and the static array's size. */
size_t myos_gemm_bf16_noalloc_scratch(size_t batch, size_t m, size_t k);
size_t myos_gemm_bf16_noalloc_max_scratch(void);

/* add_bf16_bias, bf16.rs:147-158: y[i] += bf16(bias[i]); bias_len != y_len -> SHAPE. */
int myos_add_bf16_bias(float *y, size_t y_len, const uint16_t *bias, size_t bias_len,
                       myos_stream_t stream);

/* embed_gather_bf16, bf16.rs:165-198: out[hidden] = table[token, :].
 * shape = [vocab, hidden]; out_len != hidden -> SHAPE; token >= vocab -> TOKEN;
 * row past table_len -> ROW_OOB; table_len != vocab*hidden -> SHAPE. */
int myos_embed_gather_bf16(float *out, size_t out_len, const uint16_t *table, size_t table_len,
                           size_t vocab, size_t hidden, uint32_t token, myos_stream_t stream);

/* rmsnorm_bf16_weight, bf16.rs:231-270: y = g * (x * 1/sqrtf(mean(x^2) + eps)).
 * n == 0 or length mismatch -> SHAPE. */
int myos_rmsnorm_bf16_weight(float *y, size_t y_len, const uint16_t *weight, size_t weight_len,
                             const float *x, size_t x_len, float eps, myos_stream_t stream);

/* rope_f32_inplace, crates/tensor_core/src/rope.rs:119-184 (NeoX half-rotate).
 * The per-pair angles are evaluated on the host exactly as the reference does
 * (f32 pos * 1/powf(theta, 2i/d), cosf/sinf) and applied on the device.
 * head_dim zero/odd, len zero or not a multiple of head_dim -> SHAPE. */
int myos_rope_f32_inplace(float *x, size_t len, uint32_t position, size_t head_dim, float theta,
                          myos_stream_t stream);

/* gqa_attn_f32, crates/tensor_core/src/gqa.rs:174-218. mask: 0 = Full,
 * 1 = Causal{query_pos}. q,y: [nq, d]; k,v: [nkv, seq, d]; probs: [seq]
 * (scratch; written with the last head's probabilities like the reference).
 * Shape rules of gqa.rs:231-264 -> SHAPE. */
int myos_gqa_attn_f32(float *y, size_t y_len, const float *q, size_t q_len, const float *k,
                      size_t k_len, const float *v, size_t v_len, float *probs,
                      size_t probs_len, size_t num_q_heads, size_t num_kv_heads,
                      size_t head_dim, size_t seq_len, int mask, size_t query_pos,
                      myos_stream_t stream);

/* swiglu_mul_f32, crates/tensor_core/src/swiglu.rs:125-131: h = silu(g) * u. */
int myos_swiglu_mul_f32(float *h, size_t h_len, const float *gate, size_t gate_len,
                        const float *up, size_t up_len, myos_stream_t stream);

/* swiglu_bf16, crates/tensor_core/src/swiglu.rs:184-213: gate = W_g x,
 * up = W_u x (W_g, W_u [intermediate, hidden] bf16), h = silu(gate) * up,
 * y = W_d h (W_d [hidden, intermediate]); gate / up / h are the caller's
 * scratch (the reference's argument order: activations, weights, scratch,
 * shape). hidden or intermediate zero, or any length mismatch -> SHAPE. */
int myos_swiglu_bf16(float *y, size_t y_len, const float *x, size_t x_len, const uint16_t *gate_w,
                     size_t gate_w_len, const uint16_t *up_w, size_t up_w_len, const uint16_t *down_w,
                     size_t down_w_len, float *gate, size_t gate_len, float *up, size_t up_len,
                     float *h, size_t h_len, size_t hidden, size_t intermediate,
                     myos_stream_t stream);

/* silu_f32, crates/tensor_core/src/swiglu.rs:113-115, elementwise on the
 * device: y[i] = z[i] / (1 + expf(-z[i])). y_len != z_len -> SHAPE. */
int myos_silu_f32(float *y, size_t y_len, const float *z, size_t z_len, myos_stream_t stream);

/* rmsnorm_f32, crates/tensor_core/src/bf16.rs:200-216: rmsnorm_bf16_weight
 * with an f32 gamma. n == 0 or length mismatch -> SHAPE. */
int myos_rmsnorm_f32(float *y, size_t y_len, const float *weight, size_t weight_len, const float *x,
                     size_t x_len, float eps, myos_stream_t stream);

/* rope_inv_freqs, crates/tensor_core/src/rope.rs:89-98: inv_freq[i] =
 * 1 / powf(theta, f32(2 i) / f32(head_dim)) into DEVICE memory, evaluated on
 * the host with the reference's expression (as every RoPE table here is).
 * head_dim zero or odd, or len != head_dim / 2 -> SHAPE. */
int myos_rope_inv_freqs(float *inv_freq, size_t len, size_t head_dim, float theta,
                        myos_stream_t stream);

/* attn_scale_f32, crates/tensor_core/src/gqa.rs:158-163: *out = 1 /
 * sqrtf(head_dim) (host), the factor the attention kernels apply to each
 * finished dot. head_dim == 0 -> SHAPE. */
int myos_attn_scale_f32(size_t head_dim, float *out);

/* greedy_token, crates/model_core/src/lib.rs:157-167: first index of the
 * strict maximum (ties -> lowest index, NaN never wins, all -inf/NaN -> 0).
 * Two-pass block argmax; the u32 result is written to DEVICE memory *out. */
int myos_greedy_token(uint32_t *out, const float *logits, size_t n, myos_stream_t stream);

/* Block until the stream's work is done; returns MYOS_E_HIP on a device error. */
int myos_stream_sync(myos_stream_t stream);

/* ======================= model tier (model_core) ===================== */

typedef struct myos_model myos_model;

/* BlockShape (qwen25_block.rs:53-75) + AttnShape (attn_wire.rs:44-63). */
typedef struct {
  size_t hidden, num_q_heads, num_kv_heads, head_dim, intermediate, vocab, num_layers;
  float rms_eps, rope_theta;
  int tied_head; /* 1: logits = embed_tokens (the reference); 0: lm_head.weight */
} myos_block_shape;

/* BlockShape::qwen25_1_5b (qwen25_block.rs:66-74) and the 7B analogue
 * (hidden 3584, intermediate 18944, 28/4 heads, vocab 152064, untied head). */
enum { MYOS_SHAPE_QWEN25_1_5B = 0, MYOS_SHAPE_QWEN25_7B = 1 };
int myos_block_shape_preset(int preset, myos_block_shape *out);

enum { MYOS_KV_F32 = 0, MYOS_KV_BF16 = 1 };

/* Open: map `path` (SafeTensors), check every tensor the shape needs
 * (preflight_weights, qwen25_block.rs:599-643), upload them once to HBM
 * through pinned staging, allocate the KV cache [layers][kv][max_seq][d]
 * (KvCache::new, kv_cache.rs:99-125) and the workspace (BlockWorkspace::new,
 * qwen25_block.rs:97-114). Errors: IO / PARSE / W_* / SHAPE / HIP. */
int myos_model_open(const char *path, const myos_block_shape *shape, int kv_dtype,
                    size_t max_seq, myos_model **out);
void myos_model_close(myos_model *m);

/* prefill, qwen25_block.rs:323-543: the prompt as one chunk (MFMA GEMMs),
 * causal attention, logits for the last id, cursor += n. A device error in a
 * persistent decode launch leaves the model refusing decode calls until the
 * next prefill or cache_clear (see myos_debug_raise_wait_error). */
int myos_prefill(myos_model *m, const uint32_t *tokens, size_t n);
/* forward_token, qwen25_block.rs:220-304. pos must equal the cursor. */
int myos_forward_token(myos_model *m, uint32_t token, size_t pos);
/* greedy_decode, qwen25_block.rs:765-780: token = argmax(logits), forward,
 * append; `out` receives `steps` ids (host memory). A KV-full stop returns
 * MYOS_E_KV_FULL after the steps that fit, like the reference's loop. Each
 * step is one hipGraph replay when graphs are enabled (the default). */
int myos_greedy_decode(myos_model *m, size_t steps, uint32_t *out);

/* Teacher-forced decode (no reference counterpart: the reference's runtime
 * compares free-running ids only, main.rs:672-686): `steps` steps from the
 * cursor, step s feeding ids[s] as forward_token(ids[s], cursor) would, on the
 * same path greedy_decode takes (one cooperative launch when persistent).
 * argmax_out[s] receives greedy_token of the logits step s started from, so
 * a caller can compare each step's greedy choice with a reference run fed the
 * same ids. Checks before any launch: ids[s] >= vocab -> TOKEN; steps past
 * max_seq -> KV_FULL (nothing runs). */
int myos_decode_forced(myos_model *m, const uint32_t *ids, size_t steps, uint32_t *argmax_out);

/* attention_layer, crates/model_core/src/attn_wire.rs:207-313, on the model's
 * weights: residual += o_proj(attention(proj_in)) for `layer` at `pos`, where
 * proj_in (the caller's normed vector) feeds q/k/v (+ bias, RoPE at pos) and
 * the layer's K/V row is stored at pos; the cursor does not move. residual
 * and proj_in are HOST vectors of len == hidden floats. Checks before any
 * launch: len -> SHAPE; layer >= layers -> KV_RANGE (KvError::Range); pos !=
 * cursor -> POSITION; pos >= max_seq -> KV_FULL. */
int myos_attention_layer(myos_model *m, size_t layer, size_t pos, float *residual,
                         const float *proj_in, size_t len);
/* KvCache::advance, kv_cache.rs:226-232: cursor += 1; at max_seq -> KV_FULL. */
int myos_kv_advance(myos_model *m);

size_t myos_cache_len(const myos_model *m);        /* KvCache::len */
/* KvCache::clear (kv_cache.rs:234-237): cursor back to 0, slots kept. */
int myos_cache_clear(myos_model *m);
size_t myos_max_seq(const myos_model *m);
/* Host copies of the last forward's outputs: logits[vocab] (BlockWorkspace::logits),
 * hidden[hidden] = residual stream after the last layer, normed[hidden] = final
 * RMSNorm output (the head's input). */
int myos_copy_logits(const myos_model *m, float *out, size_t n);
int myos_copy_hidden(const myos_model *m, float *out, size_t n);
int myos_copy_normed(const myos_model *m, float *out, size_t n);
/* KvCache::key_head / value_head (kv_cache.rs:240-252) as f32 host copies. */
int myos_kv_read(const myos_model *m, size_t layer, size_t head, size_t pos, float *k, float *v);
/* 1 = capture each decode step in a hipGraph (default), 0 = plain launches. */
int myos_set_graph(myos_model *m, int enabled);
/* Decode path of myos_greedy_decode (no reference counterpart; the reference
 * has one CPU path). PERSISTENT runs the whole call as one cooperative kernel
 * whose workgroups hand activations to each other through tagged words;
 * KERNELS replays per-step graphs of per-layer kernels; AUTO (default) takes
 * PERSISTENT when the model allows it (f32 or bf16 cache, hidden and q_dim <=
 * 1536 and multiples of 32 and 8, intermediate <= 9216, head_dim 32, 64 or
 * 128, at most 8 q heads per kv head, and the kernel's LDS budget) and the
 * device has >= 256 CUs with cooperative launch. Where that kernel does not
 * fit, AUTO and PERSISTENT take STREAMED: a cooperative kernel that streams
 * each phase's weight rows from HBM and meets at device-wide barriers (hidden
 * and q_dim <= 3584, intermediate <= 20480, head_dim 32, 64 or 128, at most 8
 * q heads per kv head, max_seq <= 2048, at most 128 layers; the 7B shape). STREAMED can also be asked for on any
 * model it fits. Setting PERSISTENT or STREAMED where neither is available
 * returns MYOS_E_SHAPE. myos_decode_path returns the path the next call takes
 * (KERNELS, PERSISTENT for the register-resident kernel, or STREAMED); the
 * decode trace records the register-resident kernel only. */
enum { MYOS_DECODE_AUTO = 0, MYOS_DECODE_KERNELS = 1, MYOS_DECODE_PERSISTENT = 2,
       MYOS_DECODE_STREAMED = 3 };
int myos_set_decode_mode(myos_model *m, int mode);
int myos_decode_path(const myos_model *m);
/* Measurement hook for the persistent path (no reference counterpart): from
 * the next greedy_decode on, decode step `step` of each call records, per
 * workgroup, the device wall clock (100 MHz ticks) at 5 layers + 3 phase
 * points: [0] token chosen; [1 + 5 l + p] layer l with p = 0 input ready,
 * 1 attention items done, 2 attention merged, 3 o output ready, 4 h ready;
 * [1 + 5 layers] head input ready; [2 + 5 layers] head done. step < 0 turns
 * it off. myos_copy_decode_trace copies [grid][5 layers + 3] values, where
 * grid is 256; n must equal that count. MYOS_E_SHAPE without the path. */
int myos_set_decode_trace(myos_model *m, int64_t step);
/* Test hook for the persistent path's error handling (no reference
 * counterpart): raises the kernel's error word, so every bounded wait of the
 * next launch gives up at once and the launch returns MYOS_E_HIP. After such
 * an error the model refuses forward_token / greedy_decode / decode_forced
 * (MYOS_E_HIP) until a prefill or cache_clear. MYOS_E_SHAPE without the path. */
int myos_debug_raise_wait_error(myos_model *m);
int myos_copy_decode_trace(const myos_model *m, uint64_t *out, size_t n);
/* Device time of the last prefill / greedy_decode (hipEvent, milliseconds). */
double myos_last_prefill_ms(const myos_model *m);
double myos_last_decode_ms(const myos_model *m);
/* Device bytes held by weights / KV cache / workspace. */
size_t myos_weight_bytes(const myos_model *m);
size_t myos_kv_bytes(const myos_model *m);

/* Measurement hook (no reference counterpart): average device time of one
 * decode-step kernel class, from a hipGraph holding that kernel once per
 * layer (distinct weights, so no cache reuse across launches), replayed
 * `reps` times between two hipEvents on the model's stream. Clobbers the
 * decode activations (x, q, h) and the cache slot at the cursor: call it
 * after the decode being measured. which: MYOS_K_* below. */
enum { MYOS_K_QKV = 0, MYOS_K_ATTN = 1, MYOS_K_O = 2, MYOS_K_GATE_UP = 3, MYOS_K_DOWN = 4,
       MYOS_K_HEAD = 5 };
int myos_time_kernel(myos_model *m, int which, int reps, double *avg_ms);
/* Algorithmic HBM bytes one launch of that kernel class moves at the current
 * cursor (weights + biases + norm gains + KV read/written + activations). */
double myos_kernel_bytes(const myos_model *m, int which);

/* Seeded random-init writer for the benchmark models (no reference
 * counterpart; the reference reads real checkpoints): every matrix and bias
 * ~ N(0, std) rounded to BF16 (RNE), norm gains 1.0, qwen25_layout keys
 * (+ lm_head.weight when untied). Generator: per tensor a SplitMix64 counter
 * stream seeded with seed ^ FNV-1a64(name), Box-Muller in double. */
int myos_write_random_qwen25(const char *path, const myos_block_shape *shape, uint64_t seed,
                             float std_dev, int threads);

/* SHA-256 of a file as 64 lowercase hex digits + NUL in out_hex[65], for the
 * run fingerprint's model_sha256 field (fingerprint.rs:63-206, which the
 * reference leaves null). Host only. MYOS_E_IO if the file cannot be read. */
int myos_sha256_file(const char *path, char *out_hex);

#ifdef __cplusplus
}
#endif
#endif
