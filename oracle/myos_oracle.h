/*
 * CPU oracle for the batch-1 BF16-weight / FP32-accumulate token loop.
 *
 * TEST INFRASTRUCTURE ONLY. This is a restatement of the reference's CPU
 * path (crates/tensor_core and crates/model_core), kept bit-faithful: every
 * f32 operation is one IEEE rounding in the reference's order, products are
 * formed before they are added (built with -ffp-contract=off), and the
 * transcendental functions are the same glibc libm entry points the reference
 * links (sqrtf, expf, powf, sinf, cosf). It is used by tests/, by the smoke
 * check and as the bench's CPU baseline. The product path never links it.
 *
 * Parity pins (what fixes each function independently of this file):
 *   orc_bf16_to_f32          bf16.rs:316-320 known bits
 *   orc_gemv_bf16(_mt)       bf16.rs:350-362 hand values; gemv_bf16_kernel.rs:929-951
 *                            2^24 cancellation order; AVX2 == scalar bit-equality;
 *                            brute-force f64 error bound
 *   orc_add_bf16_bias        bf16.rs:324-347 hand values
 *   orc_embed_gather_bf16    bf16.rs:381-396 hand values
 *   orc_rmsnorm_bf16_weight  bf16.rs:311,488-544 bits (eps, serial order, 0x3f7ffff8)
 *   orc_rope_*               rope.rs:230-360 bits
 *   orc_gqa_attn_f32         gqa.rs:357-608 bits
 *   orc_silu_f32 / swiglu    swiglu.rs:362-452 bits
 *   orc_greedy_token         model_core/src/lib.rs:157-167 spec (ties, NaN)
 *   orc_attention_layer      attn_wire.rs:450-704 hand fixtures (grouped step, bias after
 *                            the GEMV, second-token mix, RoPE on k not v)
 *   orc_model_*              qwen25_block.rs:1011-1071 block fixture [1,2,0,-1] / [1,1,1,1];
 *                            :1423-1478 chunk prefill == serial forward bits; block errors
 *                            leave the cursor; two layers advance once per token; untied
 *                            head copy == tied; the post-attention norm feeds the MLP;
 *                            the MLP residual changes the logits
 *   orc_model_* (wiring)     an independent float64 numpy Qwen2 forward written from the
 *                            architecture's definition (tests/qwen2_textbook.py) agrees
 *                            on random small models
 *   orc_model_* (mutations)  tests/test_oracle_mutations.py rebuilds this file with one
 *                            plausible wiring mistake each (MLP norm reads ln1, MLP
 *                            residual dropped, KV store ignores the layer, untied head
 *                            ignored, prefill attends layer 0's cache, RoPE on v, and the
 *                            three bf16-cache mistakes below) and requires a pin to fail
 *   orc_round_bf16           closed forms: representable values unchanged, halfway cases
 *                            to even, above / below half, overflow to inf, NaN kept,
 *                            tiny denormals to zero
 *   orc_set_kv_bf16          hand fixture whose hidden state depends only on how v is
 *                            rounded (1 + 3*2^-8 -> 1 + 2^-6, 1 + 2^-9 -> 1); every
 *                            layer-0 cache row equals RNE of the f32 mode's row;
 *                            chunk prefill == serial decode bits in bf16 mode
 */
#ifndef MYOS_ORACLE_H
#define MYOS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes mirror the reference error enums (one code per variant) */
enum {
  ORC_OK = 0,
  ORC_E_SHAPE = 1,
  ORC_E_TOKEN = 2,
  ORC_E_ROW_OOB = 3,
  ORC_E_POSITION = 4,
  ORC_E_KV_FULL = 5,
  ORC_E_KV_RANGE = 6,
  ORC_E_NOMEM = 7, /* a scratch allocation failed (no reference counterpart) */
};

float orc_bf16_to_f32(uint16_t bits);

/* tensor_core ops (reference semantics, host pointers) */
int orc_gemv_bf16(float *y, const uint16_t *w, const float *x, size_t m, size_t k);
int orc_gemv_bf16_mt(float *y, const uint16_t *w, const float *x, size_t m, size_t k,
                     int threads);
int orc_gemm_bf16_mt(float *y, const uint16_t *w, const float *x, size_t batch, size_t m,
                     size_t k, int threads);
void orc_add_bf16_bias(float *y, const uint16_t *bias, size_t n);
int orc_embed_gather_bf16(float *out, const uint16_t *table, size_t vocab, size_t hidden,
                          uint32_t token);
int orc_rmsnorm_bf16_weight(float *y, const uint16_t *gamma, const float *x, size_t n,
                            float eps);
int orc_rope_inv_freqs(float *inv_freq, size_t head_dim, float theta);
int orc_rope_f32_inplace(float *x, size_t len, uint32_t position, size_t head_dim,
                         float theta);
float orc_attn_scale_f32(size_t head_dim);
/* mask: 0 = Full, 1 = Causal{query_pos} */
int orc_gqa_attn_f32(float *y, const float *q, const float *k, const float *v, float *probs,
                     size_t nq, size_t nkv, size_t head_dim, size_t seq, int mask,
                     size_t query_pos);
float orc_silu_f32(float z);
void orc_swiglu_mul_f32(float *h, const float *gate, const float *up, size_t n);
uint32_t orc_greedy_token(const float *logits, size_t n);

/* model_core: one Qwen2.5-shaped decoder over caller-owned BF16 weights */
typedef struct {
  size_t hidden, num_q_heads, num_kv_heads, head_dim, intermediate, vocab, num_layers;
  float rms_eps, rope_theta;
} orc_shape;

typedef struct {
  const uint16_t *ln1, *wq, *bq, *wk, *bk, *wv, *bv, *wo, *ln2, *wg, *wu, *wd;
} orc_layer;

typedef struct orc_model orc_model;

/* lm_head == NULL means the head is tied to embed (the reference's only form) */
orc_model *orc_model_new(const orc_shape *shape, size_t max_seq, const orc_layer *layers,
                         const uint16_t *embed, const uint16_t *final_norm,
                         const uint16_t *lm_head, int threads);
void orc_model_free(orc_model *m);
int orc_forward_token(orc_model *m, uint32_t token, size_t pos);
int orc_prefill(orc_model *m, const uint32_t *tokens, size_t n);
int orc_greedy_decode(orc_model *m, size_t steps, uint32_t *out);
size_t orc_cache_len(const orc_model *m);
const float *orc_logits(const orc_model *m);
const float *orc_hidden(const orc_model *m);  /* residual stream after the last layer */
const float *orc_normed(const orc_model *m);  /* final-norm output fed to the head */
int orc_kv_read(const orc_model *m, size_t layer, size_t head, size_t pos, float *k, float *v);
void orc_set_threads(orc_model *m, int threads);
/* bf16 KV cache mode (the reference's cache is f32, kv_cache.rs:93-94): every
 * K/V value is rounded to bf16 (nearest, ties to even) when stored, and the
 * decode step's own row is rounded the same way before attention, so every
 * attention read sees the value a bf16 cache slot holds. Only while the cache
 * is empty (ORC_E_KV_RANGE otherwise). */
int orc_set_kv_bf16(orc_model *m, int on);
float orc_round_bf16(float x);
int orc_attention_layer(orc_model *m, size_t layer, size_t pos, float *residual,
                        const float *proj_in);
int orc_kv_advance(orc_model *m);

#ifdef __cplusplus
}
#endif
#endif
