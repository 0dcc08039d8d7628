/*
 * CPU oracle for the batch-1 BF16-weight / FP32-accumulate token loop.
 * TEST INFRASTRUCTURE ONLY (tests/, the smoke check, the bench's CPU baseline).
 *
 * Restates the reference's CPU path bit-for-bit. Build flags matter:
 * -O2 -ffp-contract=off -fno-fast-math (no FMA contraction, no reassociation),
 * glibc libm for sqrtf/expf/powf/sinf/cosf (the functions the reference binds
 * through `extern "C"`, e.g. crates/tensor_core/src/bf16.rs:274-283,
 * rope.rs:199-220, gqa.rs:311-326, swiglu.rs:265-273).
 *
 * The AVX2 GEMV keeps one accumulator lane per row and walks the columns left
 * to right, so it is bit-equal to the scalar chain (the property the reference
 * asserts in crates/tensor_core/src/gemv_bf16_kernel.rs:878-1048). Rows are
 * split across a persistent thread pool in contiguous spans of whole 32-row
 * panels (gemv_bf16_kernel.rs:119-162, gemv_pool.rs:130-189).
 */
#define _GNU_SOURCE
#include "myos_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* bf16_le_to_f32, crates/tensor_core/src/bf16.rs:61-63 */
float orc_bf16_to_f32(uint16_t bits) {
  uint32_t u = (uint32_t)bits << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ---------------------------------------------------------------- GEMV --- */

/* one row, left to right, multiply then add: bf16.rs:64-79 contract */
static float dot_row_scalar(const uint16_t *w, const float *x, size_t k) {
  float acc = 0.0f;
  for (size_t j = 0; j < k; j++) {
    float p = orc_bf16_to_f32(w[j]) * x[j];
    acc = acc + p;
  }
  return acc;
}

/* gemv_bf16, bf16.rs:80-122 (k == 0 fills zero, :105-111) */
int orc_gemv_bf16(float *y, const uint16_t *w, const float *x, size_t m, size_t k) {
  for (size_t i = 0; i < m; i++) y[i] = k ? dot_row_scalar(w + i * k, x, k) : 0.0f;
  return ORC_OK;
}

__attribute__((target("avx2"))) static inline __m256 bf16x8_to_f32(const uint16_t *p) {
  __m128i h = _mm_loadu_si128((const __m128i *)p);
  return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
}

/* in-register 8x8 transpose: r[i] = row i -> r[j] = column j */
__attribute__((target("avx2"))) static inline void transpose8(__m256 r[8]) {
  __m256 t0 = _mm256_unpacklo_ps(r[0], r[1]), t1 = _mm256_unpackhi_ps(r[0], r[1]);
  __m256 t2 = _mm256_unpacklo_ps(r[2], r[3]), t3 = _mm256_unpackhi_ps(r[2], r[3]);
  __m256 t4 = _mm256_unpacklo_ps(r[4], r[5]), t5 = _mm256_unpackhi_ps(r[4], r[5]);
  __m256 t6 = _mm256_unpacklo_ps(r[6], r[7]), t7 = _mm256_unpackhi_ps(r[6], r[7]);
  __m256 s0 = _mm256_shuffle_ps(t0, t2, 0x44), s1 = _mm256_shuffle_ps(t0, t2, 0xEE);
  __m256 s2 = _mm256_shuffle_ps(t1, t3, 0x44), s3 = _mm256_shuffle_ps(t1, t3, 0xEE);
  __m256 s4 = _mm256_shuffle_ps(t4, t6, 0x44), s5 = _mm256_shuffle_ps(t4, t6, 0xEE);
  __m256 s6 = _mm256_shuffle_ps(t5, t7, 0x44), s7 = _mm256_shuffle_ps(t5, t7, 0xEE);
  r[0] = _mm256_permute2f128_ps(s0, s4, 0x20);
  r[1] = _mm256_permute2f128_ps(s1, s5, 0x20);
  r[2] = _mm256_permute2f128_ps(s2, s6, 0x20);
  r[3] = _mm256_permute2f128_ps(s3, s7, 0x20);
  r[4] = _mm256_permute2f128_ps(s0, s4, 0x31);
  r[5] = _mm256_permute2f128_ps(s1, s5, 0x31);
  r[6] = _mm256_permute2f128_ps(s2, s6, 0x31);
  r[7] = _mm256_permute2f128_ps(s3, s7, 0x31);
}

/* NP panels of 8 rows at once; lane r of acc[p] is row p*8+r. The chain per
 * row is j = 0..k-1, multiply then add, then a scalar tail for k % 8. */
#define DEF_PANELS(NP)                                                                 \
  __attribute__((target("avx2"))) static void dot_panels##NP(                          \
      float *y, const uint16_t *w, size_t k, const float *x) {                         \
    __m256 acc[NP];                                                                    \
    for (int p = 0; p < NP; p++) acc[p] = _mm256_setzero_ps();                         \
    size_t j = 0;                                                                      \
    for (; j + 8 <= k; j += 8) {                                                       \
      __m256 xb[8];                                                                    \
      for (int c = 0; c < 8; c++) xb[c] = _mm256_set1_ps(x[j + c]);                    \
      for (int p = 0; p < NP; p++) {                                                   \
        __m256 r[8];                                                                   \
        for (int q = 0; q < 8; q++) r[q] = bf16x8_to_f32(w + (size_t)(p * 8 + q) * k + j); \
        transpose8(r);                                                                 \
        for (int c = 0; c < 8; c++) acc[p] = _mm256_add_ps(acc[p], _mm256_mul_ps(r[c], xb[c])); \
      }                                                                                \
    }                                                                                  \
    float lanes[NP * 8];                                                               \
    for (int p = 0; p < NP; p++) _mm256_storeu_ps(lanes + p * 8, acc[p]);              \
    for (int r = 0; r < NP * 8; r++) {                                                 \
      float a = lanes[r];                                                              \
      const uint16_t *row = w + (size_t)r * k;                                         \
      for (size_t t = j; t < k; t++) {                                                 \
        float prod = orc_bf16_to_f32(row[t]) * x[t];                                   \
        a = a + prod;                                                                  \
      }                                                                                \
      y[r] = a;                                                                        \
    }                                                                                  \
  }
DEF_PANELS(4)
DEF_PANELS(1)

static int have_avx2(void) {
  static int cached = -1;
  if (cached < 0) cached = __builtin_cpu_supports("avx2") ? 1 : 0;
  return cached;
}

/* rows [r0, r1) of y = W x */
static void gemv_span(float *y, const uint16_t *w, const float *x, size_t k, size_t r0,
                      size_t r1) {
  size_t i = r0;
  if (have_avx2() && k > 0) {
    for (; i + 32 <= r1; i += 32) dot_panels4(y + i, w + i * k, k, x);
    for (; i + 8 <= r1; i += 8) dot_panels1(y + i, w + i * k, k, x);
  }
  for (; i < r1; i++) y[i] = k ? dot_row_scalar(w + i * k, x, k) : 0.0f;
}

/* ------------------------------------------------------- thread pool --- */

typedef void (*pool_fn)(void *arg, int part, int nparts);
#define POOL_MAX 64
static struct {
  pthread_mutex_t mu;
  pthread_cond_t start, done;
  pthread_t th[POOL_MAX];
  int nworkers;
  unsigned gen;
  int pending;
  pool_fn fn;
  void *arg;
  int nparts;
} g_pool = {.mu = PTHREAD_MUTEX_INITIALIZER,
            .start = PTHREAD_COND_INITIALIZER,
            .done = PTHREAD_COND_INITIALIZER};
static pthread_mutex_t g_pool_call = PTHREAD_MUTEX_INITIALIZER;

typedef struct {
  int id;
  unsigned born_gen; /* generation current when the worker was created */
} worker_arg;
static worker_arg g_wargs[POOL_MAX];

static void *pool_worker(void *p) {
  int id = ((worker_arg *)p)->id; /* handles part id (part 0 is the caller) */
  unsigned seen = ((worker_arg *)p)->born_gen;
  pthread_mutex_lock(&g_pool.mu);
  for (;;) {
    while (g_pool.gen == seen) pthread_cond_wait(&g_pool.start, &g_pool.mu);
    seen = g_pool.gen;
    pool_fn fn = g_pool.fn;
    void *arg = g_pool.arg;
    int nparts = g_pool.nparts;
    pthread_mutex_unlock(&g_pool.mu);
    if (id < nparts) fn(arg, id, nparts);
    pthread_mutex_lock(&g_pool.mu);
    if (id < nparts && --g_pool.pending == 0) pthread_cond_signal(&g_pool.done);
  }
  return NULL;
}

static void pool_run(pool_fn fn, void *arg, int nparts) {
  if (nparts <= 1) {
    fn(arg, 0, 1);
    return;
  }
  if (nparts > POOL_MAX) nparts = POOL_MAX;
  pthread_mutex_lock(&g_pool_call);
  pthread_mutex_lock(&g_pool.mu);
  while (g_pool.nworkers < nparts - 1) {
    int id = ++g_pool.nworkers;
    g_wargs[id].id = id;
    g_wargs[id].born_gen = g_pool.gen;
    pthread_create(&g_pool.th[id], NULL, pool_worker, &g_wargs[id]);
  }
  g_pool.fn = fn;
  g_pool.arg = arg;
  g_pool.nparts = nparts;
  g_pool.pending = nparts - 1;
  g_pool.gen++;
  pthread_cond_broadcast(&g_pool.start);
  pthread_mutex_unlock(&g_pool.mu);
  fn(arg, 0, nparts);
  pthread_mutex_lock(&g_pool.mu);
  while (g_pool.pending > 0) pthread_cond_wait(&g_pool.done, &g_pool.mu);
  pthread_mutex_unlock(&g_pool.mu);
  pthread_mutex_unlock(&g_pool_call);
}

/* contiguous span of whole 32-row panels per part (gemv_bf16_kernel.rs:119-162) */
static void span_of(size_t m, int part, int nparts, size_t *r0, size_t *r1) {
  size_t panels = (m + 31) / 32;
  size_t per = panels / (size_t)nparts, extra = panels % (size_t)nparts;
  size_t p0 = (size_t)part * per + ((size_t)part < extra ? (size_t)part : extra);
  size_t p1 = p0 + per + ((size_t)part < extra ? 1 : 0);
  *r0 = p0 * 32 < m ? p0 * 32 : m;
  *r1 = p1 * 32 < m ? p1 * 32 : m;
}

typedef struct {
  float *y;
  const uint16_t *w;
  const float *x;
  size_t batch, m, k;
} gemm_job;

static void gemm_part(void *p, int part, int nparts) {
  gemm_job *j = (gemm_job *)p;
  size_t r0, r1;
  span_of(j->m, part, nparts, &r0, &r1);
  if (r0 >= r1) return;
  /* 32-row panels outermost so a panel stays in cache across the tokens */
  for (size_t a = r0; a < r1; a += 32) {
    size_t b1 = a + 32 < r1 ? a + 32 : r1;
    for (size_t b = 0; b < j->batch; b++)
      gemv_span(j->y + b * j->m, j->w, j->x + b * j->k, j->k, a, b1);
  }
}

int orc_gemv_bf16_mt(float *y, const uint16_t *w, const float *x, size_t m, size_t k,
                     int threads) {
  gemm_job j = {y, w, x, 1, m, k};
  size_t panels = (m + 31) / 32;
  int parts = threads < 1 ? 1 : threads;
  if ((size_t)parts > panels) parts = panels ? (int)panels : 1;
  pool_run(gemm_part, &j, parts);
  return ORC_OK;
}

/* gemm_bf16, crates/tensor_core/src/gemm_bf16.rs:51-110: Y[b,i] is the same
 * f32 chain as the per-token GEMV (bit-identical, gemm_bf16.rs:517-572). */
int orc_gemm_bf16_mt(float *y, const uint16_t *w, const float *x, size_t batch, size_t m,
                     size_t k, int threads) {
  gemm_job j = {y, w, x, batch, m, k};
  size_t panels = (m + 31) / 32;
  int parts = threads < 1 ? 1 : threads;
  if ((size_t)parts > panels) parts = panels ? (int)panels : 1;
  pool_run(gemm_part, &j, parts);
  return ORC_OK;
}

/* ------------------------------------------------------ small ops ----- */

/* add_bf16_bias, bf16.rs:147-158 */
void orc_add_bf16_bias(float *y, const uint16_t *bias, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = y[i] + orc_bf16_to_f32(bias[i]);
}

/* embed_gather_bf16, bf16.rs:165-198 */
int orc_embed_gather_bf16(float *out, const uint16_t *table, size_t vocab, size_t hidden,
                          uint32_t token) {
  if ((size_t)token >= vocab) return ORC_E_TOKEN;
  const uint16_t *row = table + (size_t)token * hidden;
  for (size_t j = 0; j < hidden; j++) out[j] = orc_bf16_to_f32(row[j]);
  return ORC_OK;
}

/* rmsnorm_bf16_weight + inv_rms_serial, bf16.rs:231-270 */
int orc_rmsnorm_bf16_weight(float *y, const uint16_t *gamma, const float *x, size_t n,
                            float eps) {
  if (n == 0) return ORC_E_SHAPE;
  float sum_sq = 0.0f;
  for (size_t i = 0; i < n; i++) {
    float sq = x[i] * x[i];
    sum_sq = sum_sq + sq;
  }
  float mean = sum_sq / (float)n;
  float inv = 1.0f / sqrtf(mean + eps);
  for (size_t i = 0; i < n; i++) {
    float xs = x[i] * inv;
    y[i] = orc_bf16_to_f32(gamma[i]) * xs;
  }
  return ORC_OK;
}

/* inv_freq_at, rope.rs:186-189 */
static float inv_freq_at(size_t pair, size_t head_dim, float theta) {
  float exponent = (float)(2 * pair) / (float)head_dim;
  return 1.0f / powf(theta, exponent);
}

/* rope_inv_freqs, rope.rs:89-98 */
int orc_rope_inv_freqs(float *inv_freq, size_t head_dim, float theta) {
  if (head_dim == 0 || head_dim % 2) return ORC_E_SHAPE;
  for (size_t i = 0; i < head_dim / 2; i++) inv_freq[i] = inv_freq_at(i, head_dim, theta);
  return ORC_OK;
}

/* rope_f32_inplace -> rotate, rope.rs:119-184 (NeoX half-rotate) */
int orc_rope_f32_inplace(float *x, size_t len, uint32_t position, size_t head_dim,
                         float theta) {
  if (head_dim == 0 || head_dim % 2 || len == 0 || len % head_dim) return ORC_E_SHAPE;
  size_t heads = len / head_dim, half = head_dim / 2;
  float posf = (float)position;
  for (size_t pair = 0; pair < half; pair++) {
    float angle = posf * inv_freq_at(pair, head_dim, theta);
    float c = cosf(angle), s = sinf(angle);
    for (size_t h = 0; h < heads; h++) {
      size_t i0 = h * head_dim + pair, i1 = i0 + half;
      float x0 = x[i0], x1 = x[i1];
      float x0c = x0 * c, x1s = x1 * s, x1c = x1 * c, x0s = x0 * s;
      x[i0] = x0c - x1s;
      x[i1] = x1c + x0s;
    }
  }
  return ORC_OK;
}

/* attn_scale_f32, gqa.rs:158-163 */
float orc_attn_scale_f32(size_t head_dim) { return 1.0f / sqrtf((float)head_dim); }

/* gqa_attn_f32, gqa.rs:174-218, softmax_kept :283-307 */
int orc_gqa_attn_f32(float *y, const float *q, const float *k, const float *v, float *probs,
                     size_t nq, size_t nkv, size_t head_dim, size_t seq, int mask,
                     size_t query_pos) {
  if (!nq || !nkv || !head_dim || !seq || nq % nkv) return ORC_E_SHAPE;
  size_t q_per_kv = nq / nkv;
  float scale = orc_attn_scale_f32(head_dim);
#define KEPT(t) (mask == 0 || (t) <= query_pos)
  for (size_t h = 0; h < nq; h++) {
    size_t g = h / q_per_kv;
    const float *qr = q + h * head_dim;
    for (size_t t = 0; t < seq; t++) {
      if (!KEPT(t)) continue;
      const float *kr = k + (g * seq + t) * head_dim;
      float acc = 0.0f;
      for (size_t d = 0; d < head_dim; d++) {
        float p = qr[d] * kr[d];
        acc = acc + p;
      }
      probs[t] = acc * scale;
    }
    float mx = probs[0];
    for (size_t t = 1; t < seq; t++)
      if (KEPT(t) && probs[t] > mx) mx = probs[t];
    float sum = 0.0f;
    for (size_t t = 0; t < seq; t++) {
      if (!KEPT(t)) continue;
      float e = expf(probs[t] - mx);
      probs[t] = e;
      sum = sum + e;
    }
    for (size_t t = 0; t < seq; t++) probs[t] = KEPT(t) ? probs[t] / sum : 0.0f;
    float *yr = y + h * head_dim;
    for (size_t d = 0; d < head_dim; d++) {
      float acc = 0.0f;
      for (size_t t = 0; t < seq; t++) {
        if (!KEPT(t)) continue;
        float p = probs[t] * v[(g * seq + t) * head_dim + d];
        acc = acc + p;
      }
      yr[d] = acc;
    }
  }
#undef KEPT
  return ORC_OK;
}

/* silu_f32, swiglu.rs:113-115 */
float orc_silu_f32(float z) { return z / (1.0f + expf(-z)); }

/* swiglu_mul_f32 -> mul_ltr, swiglu.rs:125-131,254-261 */
void orc_swiglu_mul_f32(float *h, const float *gate, const float *up, size_t n) {
  for (size_t i = 0; i < n; i++) {
    float a = orc_silu_f32(gate[i]);
    h[i] = a * up[i];
  }
}

/* greedy_token, crates/model_core/src/lib.rs:157-167 */
uint32_t orc_greedy_token(const float *logits, size_t n) {
  size_t best_i = 0;
  float best = -INFINITY;
  for (size_t i = 0; i < n; i++) {
    if (logits[i] > best) {
      best = logits[i];
      best_i = i;
    }
  }
  return (uint32_t)best_i;
}

/* ------------------------------------------------------------ model --- */

struct orc_model {
  orc_shape s;
  size_t max_seq, len, q_dim, kv_dim;
  int threads;
  int kv_bf16; /* cache holds bf16 values (RNE on store); every attention read sees them */
  orc_layer *layers;
  const uint16_t *embed, *final_norm, *head;
  /* kv_cache.rs:89-125: [layer][kv_head][max_seq][head_dim] f32, zeroed */
  float *kc, *vc;
  /* workspace, qwen25_block.rs:81-114 / attn_wire.rs:65-105 */
  float *x, *normed, *mlp, *gate, *up, *act, *logits;
  float *q, *k, *v, *att, *proj, *probs, *pack_k, *pack_v;
};

static float *zalloc(size_t n) { return (float *)calloc(n ? n : 1, sizeof(float)); }

orc_model *orc_model_new(const orc_shape *shape, size_t max_seq, const orc_layer *layers,
                         const uint16_t *embed, const uint16_t *final_norm,
                         const uint16_t *lm_head, int threads) {
  const orc_shape *s = shape;
  if (!max_seq || !s->num_layers || !s->vocab || !s->intermediate || !s->hidden ||
      !s->num_q_heads || !s->num_kv_heads || !s->head_dim || s->head_dim % 2 ||
      s->num_q_heads % s->num_kv_heads)
    return NULL;
  orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
  m->s = *s;
  m->max_seq = max_seq;
  m->threads = threads < 1 ? 1 : threads;
  m->q_dim = s->num_q_heads * s->head_dim;
  m->kv_dim = s->num_kv_heads * s->head_dim;
  m->layers = (orc_layer *)malloc(sizeof(orc_layer) * s->num_layers);
  memcpy(m->layers, layers, sizeof(orc_layer) * s->num_layers);
  m->embed = embed;
  m->final_norm = final_norm;
  m->head = lm_head ? lm_head : embed;
  size_t kvn = s->num_layers * s->num_kv_heads * max_seq * s->head_dim;
  m->kc = zalloc(kvn);
  m->vc = zalloc(kvn);
  m->x = zalloc(s->hidden);
  m->normed = zalloc(s->hidden);
  m->mlp = zalloc(s->hidden);
  m->gate = zalloc(s->intermediate);
  m->up = zalloc(s->intermediate);
  m->act = zalloc(s->intermediate);
  m->logits = zalloc(s->vocab);
  m->q = zalloc(m->q_dim);
  m->k = zalloc(m->kv_dim);
  m->v = zalloc(m->kv_dim);
  m->att = zalloc(m->q_dim);
  m->proj = zalloc(s->hidden);
  m->probs = zalloc(max_seq);
  m->pack_k = zalloc(s->num_kv_heads * max_seq * s->head_dim);
  m->pack_v = zalloc(s->num_kv_heads * max_seq * s->head_dim);
  return m;
}

void orc_model_free(orc_model *m) {
  if (!m) return;
  float *bufs[] = {m->kc, m->vc, m->x, m->normed, m->mlp, m->gate, m->up, m->act,
                   m->logits, m->q, m->k, m->v, m->att, m->proj, m->probs, m->pack_k,
                   m->pack_v};
  for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++) free(bufs[i]);
  free(m->layers);
  free(m);
}

void orc_set_threads(orc_model *m, int threads) { m->threads = threads < 1 ? 1 : threads; }
size_t orc_cache_len(const orc_model *m) { return m->len; }
const float *orc_logits(const orc_model *m) { return m->logits; }
const float *orc_hidden(const orc_model *m) { return m->x; }
const float *orc_normed(const orc_model *m) { return m->normed; }

/* KvCache::offset, kv_cache.rs:311-335 */
static size_t kv_off(const orc_model *m, size_t layer, size_t head, size_t pos) {
  return ((layer * m->s.num_kv_heads + head) * m->max_seq + pos) * m->s.head_dim;
}

int orc_kv_read(const orc_model *m, size_t layer, size_t head, size_t pos, float *k,
                float *v) {
  if (layer >= m->s.num_layers || head >= m->s.num_kv_heads || pos >= m->max_seq)
    return ORC_E_KV_RANGE;
  size_t o = kv_off(m, layer, head, pos);
  memcpy(k, m->kc + o, m->s.head_dim * sizeof(float));
  memcpy(v, m->vc + o, m->s.head_dim * sizeof(float));
  return ORC_OK;
}

/* f32 -> nearest bf16 (ties to even), widened back to f32; NaN stays a quiet
 * NaN. The reference's cache is f32 (kv_cache.rs:93-94); this is the value a
 * bf16 cache slot holds. */
float orc_round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    u = (u | 0x00400000u) & 0xffff0000u;
  else
    u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

static void round_bf16_n(float *x, size_t n) {
  for (size_t i = 0; i < n; i++) x[i] = orc_round_bf16(x[i]);
}

int orc_set_kv_bf16(orc_model *m, int on) {
  if (m->len) return ORC_E_KV_RANGE; /* only while the cache is empty */
  m->kv_bf16 = on != 0;
  return ORC_OK;
}

/* KvCache::store_at, kv_cache.rs:158-183 (rounded to bf16 in the bf16 mode) */
static void kv_store(orc_model *m, size_t layer, size_t pos, const float *k, const float *v) {
  size_t d = m->s.head_dim;
  for (size_t h = 0; h < m->s.num_kv_heads; h++) {
    size_t o = kv_off(m, layer, h, pos);
    memcpy(m->kc + o, k + h * d, d * sizeof(float));
    memcpy(m->vc + o, v + h * d, d * sizeof(float));
    if (m->kv_bf16) {
      round_bf16_n(m->kc + o, d);
      round_bf16_n(m->vc + o, d);
    }
  }
}

/* KvCache::pack_prefix, kv_cache.rs:191-223 (slots 0..seq into [kv, seq, d]) */
static void kv_pack(orc_model *m, size_t layer, size_t seq) {
  size_t d = m->s.head_dim;
  for (size_t h = 0; h < m->s.num_kv_heads; h++)
    for (size_t t = 0; t < seq; t++) {
      size_t src = kv_off(m, layer, h, t), dst = (h * seq + t) * d;
      memcpy(m->pack_k + dst, m->kc + src, d * sizeof(float));
      memcpy(m->pack_v + dst, m->vc + src, d * sizeof(float));
    }
}

/* KvCache::pack_prefix_with_token, kv_cache.rs:259-302 */
static void kv_pack_with_token(orc_model *m, size_t layer, size_t pos) {
  size_t d = m->s.head_dim, seq = pos + 1;
  for (size_t h = 0; h < m->s.num_kv_heads; h++) {
    for (size_t t = 0; t < pos; t++) {
      size_t src = kv_off(m, layer, h, t), dst = (h * seq + t) * d;
      memcpy(m->pack_k + dst, m->kc + src, d * sizeof(float));
      memcpy(m->pack_v + dst, m->vc + src, d * sizeof(float));
    }
    size_t dst = (h * seq + pos) * d;
    memcpy(m->pack_k + dst, m->k + h * d, d * sizeof(float));
    memcpy(m->pack_v + dst, m->v + h * d, d * sizeof(float));
  }
}

static void add_assign(float *y, const float *x, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = y[i] + x[i];
}

/* attention_layer, crates/model_core/src/attn_wire.rs:207-313 */
static void attention_layer(orc_model *m, size_t layer, size_t pos) {
  const orc_layer *L = &m->layers[layer];
  size_t H = m->s.hidden, qd = m->q_dim, kd = m->kv_dim;
  orc_gemv_bf16_mt(m->q, L->wq, m->normed, qd, H, m->threads);
  orc_add_bf16_bias(m->q, L->bq, qd);
  orc_gemv_bf16_mt(m->k, L->wk, m->normed, kd, H, m->threads);
  orc_add_bf16_bias(m->k, L->bk, kd);
  orc_gemv_bf16_mt(m->v, L->wv, m->normed, kd, H, m->threads);
  orc_add_bf16_bias(m->v, L->bv, kd);
  orc_rope_f32_inplace(m->q, qd, (uint32_t)pos, m->s.head_dim, m->s.rope_theta);
  orc_rope_f32_inplace(m->k, kd, (uint32_t)pos, m->s.head_dim, m->s.rope_theta);
  if (m->kv_bf16) { /* the token's own row as its cache slot will hold it */
    round_bf16_n(m->k, kd);
    round_bf16_n(m->v, kd);
  }
  kv_pack_with_token(m, layer, pos);
  orc_gqa_attn_f32(m->att, m->q, m->pack_k, m->pack_v, m->probs, m->s.num_q_heads,
                   m->s.num_kv_heads, m->s.head_dim, pos + 1, 0, 0);
  orc_gemv_bf16_mt(m->proj, L->wo, m->att, H, qd, m->threads);
  kv_store(m, layer, pos, m->k, m->v);
  add_assign(m->x, m->proj, H);
}

/* attention_layer on caller vectors: residual += o_proj(attn(proj_in)); stores
 * this layer's K/V at pos, does not advance (attn_wire.rs:207-313) */
int orc_attention_layer(orc_model *m, size_t layer, size_t pos, float *residual,
                        const float *proj_in) {
  if (layer >= m->s.num_layers) return ORC_E_KV_RANGE;
  if (pos != m->len) return ORC_E_POSITION;
  if (pos >= m->max_seq) return ORC_E_KV_FULL;
  memcpy(m->normed, proj_in, m->s.hidden * sizeof(float));
  memcpy(m->x, residual, m->s.hidden * sizeof(float));
  attention_layer(m, layer, pos);
  memcpy(residual, m->x, m->s.hidden * sizeof(float));
  return ORC_OK;
}

/* KvCache::advance, kv_cache.rs:226-232 */
int orc_kv_advance(orc_model *m) {
  if (m->len >= m->max_seq) return ORC_E_KV_FULL;
  m->len += 1;
  return ORC_OK;
}

/* forward_token, crates/model_core/src/qwen25_block.rs:220-304 */
int orc_forward_token(orc_model *m, uint32_t token, size_t pos) {
  if (pos != m->len) return ORC_E_POSITION;
  if (pos >= m->max_seq) return ORC_E_KV_FULL;
  if ((size_t)token >= m->s.vocab) return ORC_E_TOKEN;
  size_t H = m->s.hidden, I = m->s.intermediate;
  orc_embed_gather_bf16(m->x, m->embed, m->s.vocab, H, token);
  for (size_t l = 0; l < m->s.num_layers; l++) {
    const orc_layer *L = &m->layers[l];
    orc_rmsnorm_bf16_weight(m->normed, L->ln1, m->x, H, m->s.rms_eps);
    attention_layer(m, l, pos);
    orc_rmsnorm_bf16_weight(m->normed, L->ln2, m->x, H, m->s.rms_eps);
    /* swiglu_bf16, swiglu.rs:184-213 */
    orc_gemv_bf16_mt(m->gate, L->wg, m->normed, I, H, m->threads);
    orc_gemv_bf16_mt(m->up, L->wu, m->normed, I, H, m->threads);
    orc_swiglu_mul_f32(m->act, m->gate, m->up, I);
    orc_gemv_bf16_mt(m->mlp, L->wd, m->act, H, I, m->threads);
    add_assign(m->x, m->mlp, H);
  }
  orc_rmsnorm_bf16_weight(m->normed, m->final_norm, m->x, H, m->s.rms_eps);
  orc_gemv_bf16_mt(m->logits, m->head, m->normed, m->s.vocab, H, m->threads);
  m->len += 1;
  return ORC_OK;
}

/* attend_chunk's per-position loop (qwen25_block.rs:737-756): positions are
 * independent and each is the serial gqa_attn_f32, so spreading them over the
 * pool changes no bit; every part has its own probs scratch. */
typedef struct {
  orc_model *m;
  float *A;
  const float *Q;
  size_t n, start, end;
  float *probs; /* [nparts][end] */
} attend_job;

static void attend_part(void *p, int part, int nparts) {
  attend_job *j = (attend_job *)p;
  orc_model *m = j->m;
  size_t qd = m->q_dim, d = m->s.head_dim;
  float *probs = j->probs + (size_t)part * j->end;
  for (size_t i = (size_t)part; i < j->n; i += (size_t)nparts)
    orc_gqa_attn_f32(j->A + i * qd, j->Q + i * qd, m->pack_k, m->pack_v, probs,
                     m->s.num_q_heads, m->s.num_kv_heads, d, j->end, 1, j->start + i);
}

/* prefill, crates/model_core/src/qwen25_block.rs:323-543 */
int orc_prefill(orc_model *m, const uint32_t *tokens, size_t n) {
  if (n == 0) return ORC_E_SHAPE;
  size_t start = m->len;
  if (start >= m->max_seq) return ORC_E_KV_FULL;
  size_t end = start + n;
  if (end > m->max_seq) return ORC_E_KV_FULL;
  for (size_t i = 0; i < n; i++)
    if ((size_t)tokens[i] >= m->s.vocab) return ORC_E_TOKEN;
  size_t H = m->s.hidden, I = m->s.intermediate, qd = m->q_dim, kd = m->kv_dim;
  size_t d = m->s.head_dim;
  float *X = zalloc(n * H), *N = zalloc(n * H), *Q = zalloc(n * qd), *K = zalloc(n * kd);
  float *V = zalloc(n * kd), *A = zalloc(n * qd), *P = zalloc(n * H), *G = zalloc(n * I);
  float *U = zalloc(n * I), *F = zalloc(n * I);
  {
    float *bufs[] = {X, N, Q, K, V, A, P, G, U, F};
    int bad = 0;
    for (size_t i = 0; i < 10; i++) bad |= bufs[i] == NULL;
    if (bad) {
      for (size_t i = 0; i < 10; i++) free(bufs[i]);
      return ORC_E_NOMEM;
    }
  }
  for (size_t i = 0; i < n; i++) orc_embed_gather_bf16(X + i * H, m->embed, m->s.vocab, H, tokens[i]);
  for (size_t l = 0; l < m->s.num_layers; l++) {
    const orc_layer *L = &m->layers[l];
    for (size_t i = 0; i < n; i++)
      orc_rmsnorm_bf16_weight(N + i * H, L->ln1, X + i * H, H, m->s.rms_eps);
    orc_gemm_bf16_mt(Q, L->wq, N, n, qd, H, m->threads);
    orc_gemm_bf16_mt(K, L->wk, N, n, kd, H, m->threads);
    orc_gemm_bf16_mt(V, L->wv, N, n, kd, H, m->threads);
    /* bias_rope_store, qwen25_block.rs:679-712 */
    for (size_t i = 0; i < n; i++) {
      orc_add_bf16_bias(Q + i * qd, L->bq, qd);
      orc_add_bf16_bias(K + i * kd, L->bk, kd);
      orc_add_bf16_bias(V + i * kd, L->bv, kd);
      orc_rope_f32_inplace(Q + i * qd, qd, (uint32_t)(start + i), d, m->s.rope_theta);
      orc_rope_f32_inplace(K + i * kd, kd, (uint32_t)(start + i), d, m->s.rope_theta);
      kv_store(m, l, start + i, K + i * kd, V + i * kd);
    }
    /* attend_chunk, qwen25_block.rs:714-758 */
    kv_pack(m, l, end);
    {
      int parts = n < 8 ? 1 : m->threads;
      attend_job job = {m, A, Q, n, start, end, zalloc((size_t)parts * end)};
      if (!job.probs) {
        float *bufs[] = {X, N, Q, K, V, A, P, G, U, F};
        for (size_t i = 0; i < 10; i++) free(bufs[i]);
        return ORC_E_NOMEM;
      }
      pool_run(attend_part, &job, parts);
      free(job.probs);
    }
    orc_gemm_bf16_mt(P, L->wo, A, n, H, qd, m->threads);
    for (size_t i = 0; i < n; i++) add_assign(X + i * H, P + i * H, H);
    for (size_t i = 0; i < n; i++)
      orc_rmsnorm_bf16_weight(N + i * H, L->ln2, X + i * H, H, m->s.rms_eps);
    orc_gemm_bf16_mt(G, L->wg, N, n, I, H, m->threads);
    orc_gemm_bf16_mt(U, L->wu, N, n, I, H, m->threads);
    for (size_t i = 0; i < n; i++) orc_swiglu_mul_f32(F + i * I, G + i * I, U + i * I, I);
    orc_gemm_bf16_mt(P, L->wd, F, n, H, I, m->threads);
    for (size_t i = 0; i < n; i++) add_assign(X + i * H, P + i * H, H);
  }
  const float *last = X + (n - 1) * H;
  orc_rmsnorm_bf16_weight(m->normed, m->final_norm, last, H, m->s.rms_eps);
  memcpy(m->x, last, H * sizeof(float));
  orc_gemv_bf16_mt(m->logits, m->head, m->normed, m->s.vocab, H, m->threads);
  m->len = end;
  float *bufs[] = {X, N, Q, K, V, A, P, G, U, F};
  for (size_t i = 0; i < 10; i++) free(bufs[i]);
  return ORC_OK;
}

/* greedy_decode, crates/model_core/src/qwen25_block.rs:765-780 */
int orc_greedy_decode(orc_model *m, size_t steps, uint32_t *out) {
  for (size_t s = 0; s < steps; s++) {
    uint32_t token = orc_greedy_token(m->logits, m->s.vocab);
    int rc = orc_forward_token(m, token, m->len);
    if (rc) return rc;
    out[s] = token;
  }
  return ORC_OK;
}
