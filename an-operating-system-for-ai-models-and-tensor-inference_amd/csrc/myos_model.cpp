// Model tier of the C ABI: model_core's KvCache + BlockWorkspace + prefill /
// forward_token / greedy_decode (crates/model_core/src/qwen25_block.rs) over
// weights uploaded once into HBM.
//
// HBM layout per layer (one arena, 256-byte aligned sub-buffers):
//   wqkv [q_dim + 2 kv_dim, hidden]  q, k, v rows fused; q and k rows reordered
//                                    so each RoPE pair (p, p + d/2) of a head is
//                                    two adjacent rows (the GEMV epilogue rotates
//                                    a pair it holds in registers), v in order
//   bqkv [q_dim + 2 kv_dim] f32      biases in the same row order
//   wo   [hidden, q_dim]
//   wgu  [2 intermediate, hidden]    gate_i and up_i interleaved (SwiGLU epilogue)
//   wd   [hidden, intermediate]
//   ln1, ln2 [hidden] bf16
// plus embed [vocab, hidden] (also the tied head), final norm, lm_head (untied).
// KV cache: [layer][kv_head][max_seq][head_dim], f32 (the reference's
// kv_cache.rs:84-87 layout) or bf16.
//
// A decode step is 2 + 5 * layers launches, all reading the device-resident
// state {pos, token, step, mode}, so one captured hipGraph replays every step.
// greedy_decode instead runs the whole call as one persistent cooperative
// kernel (myos_persistent.hip) when the shape, an f32 cache and the device
// allow it; both paths leave the same state, logits and cache behind.
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <string>
#include <vector>

#include "../../include/myos_hip.h"
#include "myos_internal.h"
#include "myos_safetensors.h"

using namespace myos;

namespace {

constexpr size_t kStage = 64ull << 20;  // pinned staging buffer size

struct DevLayer {
  uint16_t *ln1, *wqkv, *wo, *ln2, *wgu, *wd;
  float *bqkv;
};

std::string lkey(size_t l, const char *suffix) {
  return "model.layers." + std::to_string(l) + "." + suffix;
}

inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

}  // namespace

struct myos_model {
  myos_block_shape s{};
  int kv_bf16 = 0;
  size_t max_seq = 0, len = 0;
  size_t q_dim = 0, kv_dim = 0, qkv_rows = 0, gu_rows = 0;
  hipStream_t stream = nullptr;
  uint8_t *wbuf = nullptr;
  size_t wbytes = 0;
  std::vector<DevLayer> layers;
  uint16_t *embed = nullptr, *final_norm = nullptr, *head = nullptr;
  uint8_t *kc = nullptr, *vc = nullptr;
  size_t kv_bytes = 0, layer_kv_elems = 0;
  float2 *rope = nullptr;
  // decode workspace
  uint8_t *ws = nullptr;
  size_t ws_bytes = 0;
  float *x = nullptr, *q = nullptr, *att = nullptr, *h = nullptr, *logits = nullptr,
        *normed = nullptr, *attn_part = nullptr;
  int *attn_cnt = nullptr;  // per kv group: chunk workgroups finished (decode attention merge)
  float2 *part = nullptr;
  int nparts = 0;
  uint32_t *state = nullptr, *out_ids = nullptr;
  uint32_t *force_ids = nullptr;  // teacher-forced ids of myos_decode_forced
  uint32_t *host_state = nullptr;  // pinned [4]
  // prefill workspace, grown on demand
  uint8_t *pf = nullptr;
  size_t pf_rows = 0;
  float *pX = nullptr, *pQ = nullptr;
  uint16_t *pAhi = nullptr, *pAlo = nullptr, *pHhi = nullptr, *pHlo = nullptr;
  uint32_t *ptok = nullptr;
  float *pws = nullptr;           // GEMM K-split partials
  size_t pws_cap = 0;
  // graph + timing
  bool use_graph = true;
  hipGraphExec_t graph = nullptr;   // one decode step
  hipGraphExec_t graph_n = nullptr; // kGraphSteps decode steps back to back
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  double prefill_ms = 0, decode_ms = 0;
  // persistent decode: one cooperative launch per greedy_decode call
  int decode_mode = MYOS_DECODE_AUTO;
  bool persist_ok = false;        // the register-resident cooperative kernel fits
  bool wide_ok = false;           // the streamed cooperative kernel fits
  uint8_t *pbuf = nullptr;        // tagged exchange words + error word, zeroed
  size_t pbuf_bytes = 0;
  PersistLayer *dlayers = nullptr;
  PersistArgs pargs{};            // all but tag_base / steps / pos0
  uint32_t *wdp = nullptr;        // down as column pairs, [L][I/2][H] words
  uint32_t tag_base = 1;          // tags below this value are spent
  uint32_t *err = nullptr;
  uint64_t *trace = nullptr;      // phase timestamps (myos_set_decode_trace)
  int64_t trace_step = -1;
  // a persistent launch gave up on a wait: logits, argmax partials and the
  // residual are garbage; decode calls are refused until prefill or cache_clear
  bool poisoned = false;

  void *kc_layer(size_t l) const {
    return kc + l * layer_kv_elems * (kv_bf16 ? 2 : 4);
  }
  void *vc_layer(size_t l) const {
    return vc + l * layer_kv_elems * (kv_bf16 ? 2 : 4);
  }
};

namespace {

int hs(hipError_t e) { return e == hipSuccess ? MYOS_OK : MYOS_E_HIP; }

#define HIP_TRY(expr)                   \
  do {                                  \
    hipError_t _e = (expr);             \
    if (_e != hipSuccess) return MYOS_E_HIP; \
  } while (0)

// host -> device through two pinned staging buffers (double buffered)
struct Uploader {
  hipStream_t s;
  uint8_t *stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int cur = 0;
  bool ok = true;

  int init(hipStream_t st) {
    s = st;
    for (int i = 0; i < 2; i++) {
      HIP_TRY(hipHostMalloc((void **)&stage[i], kStage, hipHostMallocDefault));
      HIP_TRY(hipEventCreateWithFlags(&done[i], hipEventDisableTiming));
      HIP_TRY(hipEventRecord(done[i], s));
    }
    return MYOS_OK;
  }
  int put(void *dst, const void *src, size_t n) {
    const uint8_t *p = (const uint8_t *)src;
    uint8_t *d = (uint8_t *)dst;
    while (n) {
      const size_t c = n < kStage ? n : kStage;
      HIP_TRY(hipEventSynchronize(done[cur]));
      memcpy(stage[cur], p, c);
      HIP_TRY(hipMemcpyAsync(d, stage[cur], c, hipMemcpyHostToDevice, s));
      HIP_TRY(hipEventRecord(done[cur], s));
      cur ^= 1;
      p += c;
      d += c;
      n -= c;
    }
    return MYOS_OK;
  }
  ~Uploader() {
    if (s) (void)hipStreamSynchronize(s);
    for (int i = 0; i < 2; i++) {
      if (stage[i]) (void)hipHostFree(stage[i]);
      if (done[i]) (void)hipEventDestroy(done[i]);
    }
  }
};

float bf16_to_f32_host(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// fused row r of wqkv -> source row of the [q; k; v] concatenation
int qkv_source_row(size_t r, size_t q_dim, size_t kv_dim, size_t d) {
  const size_t half = d / 2;
  if (r < q_dim + kv_dim) {
    const bool is_q = r < q_dim;
    const size_t rr = is_q ? r : r - q_dim;
    const size_t u = rr / 2, member = rr % 2, head = u / half, p = u % half;
    const size_t src = head * d + p + member * half;
    return (int)(is_q ? src : q_dim + src);
  }
  return (int)r;
}

// One decode-step kernel class for layer l (or the head), on the model stream.
int enq_kernel(myos_model *m, int which, size_t l, bool advance_pos) {
  const myos_block_shape &s = m->s;
  hipStream_t st = m->stream;
  const DevLayer &L = m->layers[l < m->layers.size() ? l : 0];
  GemvArgs g;
  switch (which) {
    case MYOS_K_QKV:
      g.w = L.wqkv;
      g.x = m->x;
      g.gamma = L.ln1;
      g.eps = s.rms_eps;
      g.m = (int)m->qkv_rows;
      g.k = (int)s.hidden;
      g.bias = L.bqkv;
      g.rope = m->rope;
      g.pos_ptr = m->state;
      g.q_out = m->q;
      g.kc = m->kc_layer(l);
      g.vc = m->vc_layer(l);
      g.kv_bf16 = m->kv_bf16;
      g.max_seq = (int)m->max_seq;
      g.q_dim = (int)m->q_dim;
      g.kv_dim = (int)m->kv_dim;
      g.head_dim = (int)s.head_dim;
      return hs(launch_gemv(g, X_NORM, EPI_QKV, st));
    case MYOS_K_ATTN: {
      AttnDecodeArgs ad;
      ad.q = m->q;
      ad.kc = m->kc_layer(l);
      ad.vc = m->vc_layer(l);
      ad.kv_bf16 = m->kv_bf16;
      ad.max_seq = (int)m->max_seq;
      ad.nq = (int)s.num_q_heads;
      ad.nkv = (int)s.num_kv_heads;
      ad.head_dim = (int)s.head_dim;
      ad.pos_ptr = m->state;
      ad.part = m->attn_part;
      ad.att = m->att;
      ad.cnt = m->attn_cnt;
      return hs(launch_attn_decode(ad, st));
    }
    case MYOS_K_O:  // the attention kernel left the merged heads in att
      g.w = L.wo;
      g.x = m->att;
      g.m = (int)s.hidden;
      g.k = (int)m->q_dim;
      g.y = m->x;
      return hs(launch_gemv(g, X_PLAIN, EPI_RESID, st));
    case MYOS_K_GATE_UP:
      g.w = L.wgu;
      g.x = m->x;
      g.gamma = L.ln2;
      g.eps = s.rms_eps;
      g.m = (int)m->gu_rows;
      g.k = (int)s.hidden;
      g.h_out = m->h;
      return hs(launch_gemv(g, X_NORM, EPI_GU, st));
    case MYOS_K_DOWN:
      g.w = L.wd;
      g.x = m->h;
      g.m = (int)s.hidden;
      g.k = (int)s.intermediate;
      g.y = m->x;
      return hs(launch_gemv(g, X_PLAIN, EPI_RESID, st));
    case MYOS_K_HEAD:
      g.w = m->head;
      g.x = m->x;
      g.gamma = m->final_norm;
      g.eps = s.rms_eps;
      g.m = (int)s.vocab;
      g.k = (int)s.hidden;
      g.y = m->logits;
      g.part = m->part;
      g.part_cap = m->nparts;
      g.normed_out = m->normed;
      g.pos_inc = advance_pos ? m->state : nullptr;
      return hs(launch_gemv(g, X_NORM, EPI_HEAD, st));
    default:
      return MYOS_E_ARG;
  }
}

// argmax of the previous logits (or the forced token) -> embed -> every
// layer (QKV+RoPE+KV store, attention, o + residual, gate/up + SwiGLU,
// down + residual) -> final norm + head + argmax partials -> pos += 1
int enqueue_step(myos_model *m) {
  ArgmaxFinalArgs af;
  af.part = m->part;
  af.nparts = m->nparts;
  af.state = m->state;
  af.out_ids = m->out_ids;
  af.force = m->force_ids;
  af.embed = m->embed;
  af.x = m->x;
  af.hidden = (int)m->s.hidden;
  af.vocab = (uint32_t)m->s.vocab;
  HIP_TRY(launch_argmax_final(af, m->stream));
  static const int order[5] = {MYOS_K_QKV, MYOS_K_ATTN, MYOS_K_O, MYOS_K_GATE_UP, MYOS_K_DOWN};
  for (size_t l = 0; l < m->s.num_layers; l++)
    for (int k : order) {
      int rc = enq_kernel(m, k, l, false);
      if (rc) return rc;
    }
  return enq_kernel(m, MYOS_K_HEAD, 0, true);
}

// Decode steps replay from graphs: one holding a single step and one holding
// kGraphSteps steps, so a long greedy decode pays one graph launch per
// kGraphSteps tokens (every step reads its position/token from device state).
constexpr size_t kGraphSteps = 8;

hipGraphExec_t capture_steps(myos_model *m, size_t steps) {
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  if (hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal) == hipSuccess) {
    int rc = MYOS_OK;
    for (size_t i = 0; i < steps && rc == MYOS_OK; i++) rc = enqueue_step(m);
    hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (rc == MYOS_OK && e == hipSuccess && g) {
      if (hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) ge = nullptr;
    }
    if (g) (void)hipGraphDestroy(g);
  }
  (void)hipGetLastError();
  return ge;
}

void prepare_graph(myos_model *m) {
  if (m->use_graph && !m->graph) {
    m->graph = capture_steps(m, 1);
    if (m->graph) m->graph_n = capture_steps(m, kGraphSteps);
    if (!m->graph) m->use_graph = false;  // capture failed: plain launches from here on
  }
}

// run n decode steps on the model stream
int run_steps(myos_model *m, size_t n) {
  prepare_graph(m);
  while (n) {
    if (m->use_graph && m->graph_n && n >= kGraphSteps) {
      HIP_TRY(hipGraphLaunch(m->graph_n, m->stream));
      n -= kGraphSteps;
    } else if (m->use_graph && m->graph) {
      HIP_TRY(hipGraphLaunch(m->graph, m->stream));
      n -= 1;
    } else {
      int rc = enqueue_step(m);
      if (rc) return rc;
      n -= 1;
    }
  }
  return MYOS_OK;
}

int write_state(myos_model *m, uint32_t pos, uint32_t token, uint32_t step, uint32_t mode) {
  HIP_TRY(hipStreamSynchronize(m->stream));  // host_state may still be in flight
  m->host_state[0] = pos;
  m->host_state[1] = token;
  m->host_state[2] = step;
  m->host_state[3] = mode;
  HIP_TRY(hipMemcpyAsync(m->state, m->host_state, 4 * sizeof(uint32_t), hipMemcpyHostToDevice,
                         m->stream));
  return MYOS_OK;
}

int ensure_prefill(myos_model *m, size_t rows) {
  if (rows <= m->pf_rows) return MYOS_OK;
  if (m->pf) {
    HIP_TRY(hipStreamSynchronize(m->stream));
    HIP_TRY(hipFree(m->pf));
    m->pf = nullptr;
    m->pf_rows = 0;
  }
  const size_t H = m->s.hidden, I = m->s.intermediate, Q = m->q_dim;
  const size_t bx = align256(rows * H * 4), bq = align256(rows * Q * 4);
  const size_t ba = align256(rows * (H > Q ? H : Q) * 2), bh = align256(rows * I * 2);
  const size_t bt = align256(rows * 4);
  // K-split partials of the four projections
  const int R = (int)rows;
  size_t wsf = gemm_ws_floats(R, (int)m->qkv_rows, (int)H);
  wsf = std::max(wsf, gemm_ws_floats(R, (int)H, (int)Q));
  wsf = std::max(wsf, gemm_ws_floats(R, (int)m->gu_rows, (int)H));
  wsf = std::max(wsf, gemm_ws_floats(R, (int)H, (int)I));
  // the attention's key-split partials use the same space (between GEMMs)
  if (m->s.head_dim == 128) wsf = std::max(wsf, attn_prefill_part_floats((int)m->s.num_q_heads, R, 4));
  const size_t bw = align256(wsf * 4);
  const size_t total = bx + bq + 2 * ba + 2 * bh + bt + bw;
  HIP_TRY(hipMalloc((void **)&m->pf, total));
  uint8_t *p = m->pf;
  m->pX = (float *)p;
  p += bx;
  m->pQ = (float *)p;
  p += bq;
  m->pAhi = (uint16_t *)p;
  p += ba;
  m->pAlo = (uint16_t *)p;
  p += ba;
  m->pHhi = (uint16_t *)p;
  p += bh;
  m->pHlo = (uint16_t *)p;
  p += bh;
  m->ptok = (uint32_t *)p;
  p += bt;
  m->pws = wsf ? (float *)p : nullptr;
  m->pws_cap = wsf;
  m->pf_rows = rows;
  return MYOS_OK;
}

int validate_shape(const myos_block_shape *s, size_t max_seq) {
  if (!s->hidden || !s->num_q_heads || !s->num_kv_heads || !s->head_dim || s->head_dim % 2 ||
      s->num_q_heads % s->num_kv_heads || !s->intermediate || !s->vocab || !s->num_layers ||
      !max_seq)
    return MYOS_E_SHAPE;
  // device limits of this build: q heads per kv head <= 8, head_dim <= 256,
  // 32-bit row indices
  if (s->num_q_heads / s->num_kv_heads > 8 || s->head_dim > 256) return MYOS_E_SHAPE;
  if (s->num_q_heads * s->head_dim > 4096) return MYOS_E_SHAPE;  // o-projection merge width
  if (s->vocab > (1u << 30) || s->hidden > (1u << 20) || s->intermediate > (1u << 24) ||
      max_seq > (1u << 24))
    return MYOS_E_SHAPE;
  return MYOS_OK;
}

// Persistent decode buffers, when the shape, the f32 cache and the device fit
// the cooperative kernel: tagged words for q, this step's k/v, attention
// partials, the residual after o and after down, h, and the head's argmax
// partials; all zero, so no tag >= 1 matches before it is written.
int setup_persistent(myos_model *m) {
  const myos_block_shape &s = m->s;
  PersistArgs &a = m->pargs;
  a.H = (int)s.hidden;
  a.I = (int)s.intermediate;
  a.V = (int)s.vocab;
  a.L = (int)s.num_layers;
  a.nq = (int)s.num_q_heads;
  a.nkv = (int)s.num_kv_heads;
  a.d = (int)s.head_dim;
  a.max_seq = (int)m->max_seq;
  a.qkv_rows = (int)m->qkv_rows;
  a.eps = s.rms_eps;
  a.kv_bf16 = m->kv_bf16;
  a.tpr = nullptr;
  const bool reg = persist_device_ok(a);
  const bool wide = wide_device_ok(a);
  if (!reg && !wide) return MYOS_OK;
  // the register kernel's tagged words (none without it), the streamed
  // kernel's f32 buffers and barrier flags (none without it), the error word
  size_t words[8] = {m->q_dim, 2 * m->kv_dim, persist_part_words(a.nq, a.max_seq, a.d),
                     m->q_dim, s.hidden, s.hidden, 2 * (size_t)persist_grid(),
                     persist_pr_words((int)s.hidden, (int)s.num_q_heads)};
  if (!reg)
    for (size_t &w : words) w = 0;
  const size_t wide_f = wide ? wide_buffer_floats(a.H, a.I, a.nq, a.d, a.max_seq) : 0;
  const size_t flags = wide ? (size_t)persist_grid() * kWFlagStride : 0;
  size_t total = 0;
  for (size_t w : words) total += align256(w * 8);
  total += align256(wide_f * 4) + align256(flags * 8) + 256;
  HIP_TRY(hipMalloc((void **)&m->pbuf, total));
  HIP_TRY(hipMemsetAsync(m->pbuf, 0, total, m->stream));
  m->pbuf_bytes = total;
  uint64_t **dst[8] = {&a.tq, &a.tkv, &a.tpart, &a.tatt, &a.txo, &a.txd, &a.targ, &a.tpr};
  uint8_t *p = m->pbuf;
  for (int i = 0; i < 8; i++) {
    *dst[i] = words[i] ? (uint64_t *)p : nullptr;
    p += align256(words[i] * 8);
  }
  a.wide = wide ? (float *)p : nullptr;
  p += align256(wide_f * 4);
  a.wflags = wide ? (uint64_t *)p : nullptr;
  p += align256(flags * 8);
  m->err = (uint32_t *)p;
  a.err = m->err;
  std::vector<PersistLayer> hl(s.num_layers);
  const size_t dsz = s.intermediate * s.hidden;  // elements of one down matrix
  // the register kernel reads down by columns: a copy of it as column pairs
  // (one 32-bit word per row of a pair); the streamed kernel reads rows
  if (reg) {
    HIP_TRY(hipMalloc((void **)&m->wdp, s.num_layers * dsz * 2));
    for (size_t l = 0; l < s.num_layers; l++)
      HIP_TRY(launch_transpose_u32(m->wdp + l * dsz / 2, (const uint32_t *)m->layers[l].wd,
                                   (int)s.hidden, (int)s.intermediate / 2, m->stream));
  }
  for (size_t l = 0; l < s.num_layers; l++) {
    const DevLayer &L = m->layers[l];
    hl[l] = PersistLayer{L.ln1, L.wqkv, L.wo, L.ln2, L.wgu, L.wd, L.bqkv,
                         reg ? m->wdp + l * dsz / 2 : nullptr};
  }
  HIP_TRY(hipMalloc((void **)&m->dlayers, hl.size() * sizeof(PersistLayer)));
  HIP_TRY(hipMemcpy(m->dlayers, hl.data(), hl.size() * sizeof(PersistLayer),
                    hipMemcpyHostToDevice));
  a.layers = m->dlayers;
  a.embed = m->embed;
  a.final_norm = m->final_norm;
  a.head = m->head;
  a.rope = m->rope;
  a.kc = (float *)m->kc;
  a.vc = (float *)m->vc;
  a.layer_kv = m->layer_kv_elems;
  a.logits = m->logits;
  a.normed = m->normed;
  a.x_out = m->x;
  a.part_out = m->part;
  a.part_cap = m->nparts;
  a.part_in = m->part;
  a.nparts_in = m->nparts;
  a.state = m->state;
  a.out_ids = m->out_ids;
  a.force = nullptr;
  // the kernels' first-use set-up (code object load, LDS limit) belongs to
  // load time, not to the first decode call's timed region
  if (reg) HIP_TRY(persist_prepare(a));
  if (wide) HIP_TRY(wide_prepare(a));
  HIP_TRY(coop_warm_launch(m->stream));
  m->persist_ok = reg;
  m->wide_ok = wide;
  return MYOS_OK;
}

constexpr int kLaunchRefused = -1;

// the streamed kernel runs when asked for, or when the register kernel does
// not fit the model
bool use_wide(const myos_model *m) {
  if (m->decode_mode == MYOS_DECODE_KERNELS) return false;
  if (m->decode_mode == MYOS_DECODE_STREAMED) return m->wide_ok;
  return !m->persist_ok && m->wide_ok;
}

bool use_persistent(const myos_model *m) {
  if (m->decode_mode == MYOS_DECODE_KERNELS) return false;
  return use_wide(m) || m->persist_ok;
}

// n greedy steps from the cursor in one cooperative launch; the error word
// is checked after the stream synchronizes
int persist_decode(myos_model *m, size_t n, bool forced = false) {
  const uint64_t tps = (uint64_t)persist_tags_per_step((int)m->s.num_layers);
  if ((uint64_t)m->tag_base + n * tps >= 0xffffffffull) {
    // the next tags would wrap: start again from zeroed words
    HIP_TRY(hipMemsetAsync(m->pbuf, 0, m->pbuf_bytes, m->stream));
    m->tag_base = 1;
  }
  PersistArgs a = m->pargs;
  a.tag_base = m->tag_base;
  a.steps = (uint32_t)n;
  a.pos0 = (uint32_t)m->len;
  a.force = forced ? m->force_ids : nullptr;
  if (m->trace_step >= 0 && (size_t)m->trace_step < n && !use_wide(m)) {
    a.trace = m->trace;
    a.trace_step = (uint32_t)m->trace_step;
  }
  const hipError_t e = use_wide(m) ? launch_decode_wide(a, m->stream)
                                    : launch_decode_persistent(a, m->stream);
  if (e == hipErrorCooperativeLaunchTooLarge || e == hipErrorInvalidConfiguration) {
    (void)hipGetLastError();
    return kLaunchRefused;  // nothing ran: the caller takes the per-kernel path
  }
  HIP_TRY(e);
  m->tag_base += (uint32_t)(n * tps);
  return MYOS_OK;
}

int persist_check_error(myos_model *m) {
  uint32_t e = 0;
  HIP_TRY(hipMemcpy(&e, m->err, 4, hipMemcpyDeviceToHost));
  if (e) {
    // a wait timed out: the run's ids, logits and cache rows are not
    // trustworthy, so nothing continues from them
    HIP_TRY(hipMemset(m->err, 0, 4));
    m->poisoned = true;
    return MYOS_E_HIP;
  }
  return MYOS_OK;
}

// n decode steps from the cursor on the selected path: greedy (mode 0) or
// fed from force_ids (mode 2); out receives the argmax of each step's input
// logits; the cursor advances by n
int decode_run(myos_model *m, size_t n, uint32_t mode, uint32_t *out) {
  bool persist = use_persistent(m);
  if (!persist) prepare_graph(m);  // capture (once) outside the timed region
  int rc = write_state(m, (uint32_t)m->len, 0, 0, mode);
  if (rc) return rc;
  HIP_TRY(hipEventRecord(m->ev0, m->stream));
  rc = persist ? persist_decode(m, n, mode == 2) : run_steps(m, n);
  if (rc == kLaunchRefused) {
    // the device cannot hold the cooperative grid: per-kernel path from now on
    m->persist_ok = false;
    m->wide_ok = false;
    persist = false;
    prepare_graph(m);
    HIP_TRY(hipEventRecord(m->ev0, m->stream));
    rc = run_steps(m, n);
  }
  if (rc) return rc;
  HIP_TRY(hipEventRecord(m->ev1, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  if (persist) {
    rc = persist_check_error(m);
    if (rc) return rc;
  }
  HIP_TRY(hipMemcpy(out, m->out_ids, n * 4, hipMemcpyDeviceToHost));
  float ms = 0;
  HIP_TRY(hipEventElapsedTime(&ms, m->ev0, m->ev1));
  m->decode_ms = ms;
  m->len += n;
  return MYOS_OK;
}
}  // namespace

extern "C" {

int myos_block_shape_preset(int preset, myos_block_shape *out) {
  if (!out) return MYOS_E_ARG;
  myos_block_shape s{};
  s.head_dim = 128;
  s.num_layers = 28;
  s.rms_eps = 1e-6f;
  s.rope_theta = 1000000.0f;
  if (preset == MYOS_SHAPE_QWEN25_1_5B) {
    s.hidden = 1536;
    s.num_q_heads = 12;
    s.num_kv_heads = 2;
    s.intermediate = 8960;
    s.vocab = 151936;
    s.tied_head = 1;
  } else if (preset == MYOS_SHAPE_QWEN25_7B) {
    s.hidden = 3584;
    s.num_q_heads = 28;
    s.num_kv_heads = 4;
    s.intermediate = 18944;
    s.vocab = 152064;
    s.tied_head = 0;
  } else {
    return MYOS_E_ARG;
  }
  *out = s;
  return MYOS_OK;
}

void myos_model_close(myos_model *m) {
  if (!m) return;
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  if (m->graph) (void)hipGraphExecDestroy(m->graph);
  if (m->graph_n) (void)hipGraphExecDestroy(m->graph_n);
  if (m->ev0) (void)hipEventDestroy(m->ev0);
  if (m->ev1) (void)hipEventDestroy(m->ev1);
  if (m->wbuf) (void)hipFree(m->wbuf);
  if (m->kc) (void)hipFree(m->kc);
  if (m->vc) (void)hipFree(m->vc);
  if (m->rope) (void)hipFree(m->rope);
  if (m->ws) (void)hipFree(m->ws);
  if (m->pf) (void)hipFree(m->pf);
  if (m->pbuf) (void)hipFree(m->pbuf);
  if (m->dlayers) (void)hipFree(m->dlayers);
  if (m->wdp) (void)hipFree(m->wdp);
  if (m->trace) (void)hipFree(m->trace);
  if (m->host_state) (void)hipHostFree(m->host_state);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

static int open_impl(myos_model *m, const char *path, const myos_block_shape *shape, int kv_dtype,
                     size_t max_seq) {
  const myos_block_shape &s = *shape;
  int rc = validate_shape(shape, max_seq);
  if (rc) return rc;
  if (kv_dtype != MYOS_KV_F32 && kv_dtype != MYOS_KV_BF16) return MYOS_E_ARG;
  m->s = s;
  m->kv_bf16 = kv_dtype == MYOS_KV_BF16;
  m->max_seq = max_seq;
  m->q_dim = s.num_q_heads * s.head_dim;
  m->kv_dim = s.num_kv_heads * s.head_dim;
  m->qkv_rows = m->q_dim + 2 * m->kv_dim;
  m->gu_rows = 2 * s.intermediate;
  const size_t H = s.hidden, I = s.intermediate, V = s.vocab, Q = m->q_dim, KD = m->kv_dim;

  SafeTensorsFile f;
  rc = f.open(path);
  if (rc) return rc;
  // preflight_weights order (qwen25_block.rs:599-643), then the untied head
  struct Need {
    std::string name;
    std::vector<size_t> shape;
  };
  std::vector<Need> need;
  need.push_back({"model.embed_tokens.weight", {V, H}});
  need.push_back({"model.norm.weight", {H}});
  for (size_t l = 0; l < s.num_layers; l++) {
    need.push_back({lkey(l, "input_layernorm.weight"), {H}});
    need.push_back({lkey(l, "self_attn.q_proj.weight"), {Q, H}});
    need.push_back({lkey(l, "self_attn.q_proj.bias"), {Q}});
    need.push_back({lkey(l, "self_attn.k_proj.weight"), {KD, H}});
    need.push_back({lkey(l, "self_attn.k_proj.bias"), {KD}});
    need.push_back({lkey(l, "self_attn.v_proj.weight"), {KD, H}});
    need.push_back({lkey(l, "self_attn.v_proj.bias"), {KD}});
    need.push_back({lkey(l, "self_attn.o_proj.weight"), {H, Q}});
    need.push_back({lkey(l, "post_attention_layernorm.weight"), {H}});
    need.push_back({lkey(l, "mlp.gate_proj.weight"), {I, H}});
    need.push_back({lkey(l, "mlp.up_proj.weight"), {I, H}});
    need.push_back({lkey(l, "mlp.down_proj.weight"), {H, I}});
  }
  if (!s.tied_head) need.push_back({"lm_head.weight", {V, H}});
  for (auto &n : need) {
    rc = f.bf16(n.name, n.shape, nullptr);
    if (rc) return rc;
  }
  auto host = [&](const std::string &name) {
    return (const uint16_t *)f.find(name)->data;
  };

  HIP_TRY(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
  HIP_TRY(hipEventCreate(&m->ev0));
  HIP_TRY(hipEventCreate(&m->ev1));

  // weight arena
  const size_t b_ln = align256(H * 2), b_qkv = align256(m->qkv_rows * H * 2);
  const size_t b_bias = align256(m->qkv_rows * 4), b_o = align256(H * Q * 2);
  const size_t b_gu = align256(m->gu_rows * H * 2), b_d = align256(H * I * 2);
  const size_t per_layer = 2 * b_ln + b_qkv + b_bias + b_o + b_gu + b_d;
  const size_t b_emb = align256(V * H * 2);
  m->wbytes = per_layer * s.num_layers + b_emb + b_ln + (s.tied_head ? 0 : b_emb);
  HIP_TRY(hipMalloc((void **)&m->wbuf, m->wbytes));
  uint8_t *p = m->wbuf;
  m->layers.resize(s.num_layers);
  for (auto &L : m->layers) {
    L.ln1 = (uint16_t *)p;
    p += b_ln;
    L.ln2 = (uint16_t *)p;
    p += b_ln;
    L.wqkv = (uint16_t *)p;
    p += b_qkv;
    L.bqkv = (float *)p;
    p += b_bias;
    L.wo = (uint16_t *)p;
    p += b_o;
    L.wgu = (uint16_t *)p;
    p += b_gu;
    L.wd = (uint16_t *)p;
    p += b_d;
  }
  m->embed = (uint16_t *)p;
  p += b_emb;
  m->final_norm = (uint16_t *)p;
  p += b_ln;
  m->head = m->embed;
  if (!s.tied_head) {
    m->head = (uint16_t *)p;
    p += b_emb;
  }

  // row permutations (same for every layer)
  std::vector<int> perm_qkv(m->qkv_rows), perm_gu(m->gu_rows);
  for (size_t r = 0; r < m->qkv_rows; r++)
    perm_qkv[r] = qkv_source_row(r, Q, KD, s.head_dim);
  for (size_t i = 0; i < I; i++) {
    perm_gu[2 * i] = (int)i;
    perm_gu[2 * i + 1] = (int)(I + i);
  }
  int *dperm = nullptr;
  uint16_t *tmp = nullptr;
  const size_t tmp_bytes = (m->gu_rows > m->qkv_rows ? m->gu_rows : m->qkv_rows) * H * 2;
  HIP_TRY(hipMalloc((void **)&dperm, (m->qkv_rows + m->gu_rows) * sizeof(int)));
  HIP_TRY(hipMalloc((void **)&tmp, tmp_bytes));
  int up_rc = MYOS_OK;
  {
    Uploader up;
    up_rc = up.init(m->stream);
    if (!up_rc) up_rc = up.put(dperm, perm_qkv.data(), m->qkv_rows * sizeof(int));
    if (!up_rc) up_rc = up.put(dperm + m->qkv_rows, perm_gu.data(), m->gu_rows * sizeof(int));
    std::vector<float> bias(m->qkv_rows);
    for (size_t l = 0; l < s.num_layers && !up_rc; l++) {
      DevLayer &L = m->layers[l];
      up_rc = up.put(L.ln1, host(lkey(l, "input_layernorm.weight")), H * 2);
      if (!up_rc) up_rc = up.put(L.ln2, host(lkey(l, "post_attention_layernorm.weight")), H * 2);
      if (!up_rc) up_rc = up.put(tmp, host(lkey(l, "self_attn.q_proj.weight")), Q * H * 2);
      if (!up_rc) up_rc = up.put(tmp + Q * H, host(lkey(l, "self_attn.k_proj.weight")), KD * H * 2);
      if (!up_rc)
        up_rc = up.put(tmp + (Q + KD) * H, host(lkey(l, "self_attn.v_proj.weight")), KD * H * 2);
      if (!up_rc)
        up_rc = hs(launch_permute_rows(L.wqkv, tmp, dperm, (int)m->qkv_rows, (int)H, m->stream));
      // tmp is reused next: the permute must finish reading it first
      if (!up_rc) up_rc = hs(hipStreamSynchronize(m->stream));
      const uint16_t *bq = host(lkey(l, "self_attn.q_proj.bias"));
      const uint16_t *bk = host(lkey(l, "self_attn.k_proj.bias"));
      const uint16_t *bv = host(lkey(l, "self_attn.v_proj.bias"));
      for (size_t r = 0; r < m->qkv_rows; r++) {
        const size_t src = (size_t)perm_qkv[r];
        const uint16_t b = src < Q ? bq[src] : src < Q + KD ? bk[src - Q] : bv[src - Q - KD];
        bias[r] = bf16_to_f32_host(b);
      }
      if (!up_rc) up_rc = up.put(L.bqkv, bias.data(), m->qkv_rows * 4);
      if (!up_rc) up_rc = up.put(L.wo, host(lkey(l, "self_attn.o_proj.weight")), H * Q * 2);
      if (!up_rc) up_rc = up.put(tmp, host(lkey(l, "mlp.gate_proj.weight")), I * H * 2);
      if (!up_rc) up_rc = up.put(tmp + I * H, host(lkey(l, "mlp.up_proj.weight")), I * H * 2);
      if (!up_rc)
        up_rc = hs(launch_permute_rows(L.wgu, tmp, dperm + m->qkv_rows, (int)m->gu_rows, (int)H,
                                       m->stream));
      if (!up_rc) up_rc = hs(hipStreamSynchronize(m->stream));
      if (!up_rc) up_rc = up.put(L.wd, host(lkey(l, "mlp.down_proj.weight")), H * I * 2);
    }
    if (!up_rc) up_rc = up.put(m->embed, host("model.embed_tokens.weight"), V * H * 2);
    if (!up_rc) up_rc = up.put(m->final_norm, host("model.norm.weight"), H * 2);
    if (!up_rc && !s.tied_head) up_rc = up.put(m->head, host("lm_head.weight"), V * H * 2);
  }
  (void)hipStreamSynchronize(m->stream);
  (void)hipFree(dperm);
  (void)hipFree(tmp);
  if (up_rc) return up_rc;

  // KV cache, zeroed like KvCache::new
  m->layer_kv_elems = s.num_kv_heads * max_seq * s.head_dim;
  m->kv_bytes = s.num_layers * m->layer_kv_elems * (m->kv_bf16 ? 2 : 4);
  HIP_TRY(hipMalloc((void **)&m->kc, m->kv_bytes));
  HIP_TRY(hipMalloc((void **)&m->vc, m->kv_bytes));
  HIP_TRY(hipMemsetAsync(m->kc, 0, m->kv_bytes, m->stream));
  HIP_TRY(hipMemsetAsync(m->vc, 0, m->kv_bytes, m->stream));

  // RoPE table: the reference's per-position angles (rope.rs:186-193) with libm
  const size_t half = s.head_dim / 2;
  std::vector<float2> tab(max_seq * half);
  std::vector<float> inv(half);
  for (size_t p2 = 0; p2 < half; p2++) {
    const float e = (float)(2 * p2) / (float)s.head_dim;
    inv[p2] = 1.0f / powf(s.rope_theta, e);
  }
  for (size_t pos = 0; pos < max_seq; pos++)
    for (size_t p2 = 0; p2 < half; p2++) {
      const float ang = (float)pos * inv[p2];
      tab[pos * half + p2] = make_float2(cosf(ang), sinf(ang));
    }
  HIP_TRY(hipMalloc((void **)&m->rope, tab.size() * sizeof(float2)));
  HIP_TRY(hipMemcpy(m->rope, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice));

  // decode workspace
  m->nparts = gemv_head_parts((int)V, (int)H);
  const size_t b_x = align256(H * 4), b_q = align256(Q * 4), b_h = align256(I * 4);
  const size_t b_lg = align256(V * 4), b_part = align256(m->nparts * sizeof(float2));
  const size_t b_ap =
      align256(attn_decode_part_floats((int)s.num_q_heads, (int)max_seq, (int)s.head_dim) * 4);
  const size_t b_st = align256(16);
  const size_t b_ids = align256(max_seq * 4);
  const size_t b_cnt = align256(s.num_kv_heads * 4);
  m->ws_bytes = 2 * b_x + 2 * b_q + b_h + b_lg + b_part + b_ap + b_st + 2 * b_ids + b_cnt;
  HIP_TRY(hipMalloc((void **)&m->ws, m->ws_bytes));
  HIP_TRY(hipMemsetAsync(m->ws, 0, m->ws_bytes, m->stream));
  p = m->ws;
  m->x = (float *)p;
  p += b_x;
  m->normed = (float *)p;
  p += b_x;
  m->q = (float *)p;
  p += b_q;
  m->att = (float *)p;
  p += b_q;
  m->h = (float *)p;
  p += b_h;
  m->logits = (float *)p;
  p += b_lg;
  m->part = (float2 *)p;
  p += b_part;
  m->attn_part = (float *)p;
  p += b_ap;
  m->state = (uint32_t *)p;
  p += b_st;
  m->out_ids = (uint32_t *)p;
  p += b_ids;
  m->force_ids = (uint32_t *)p;
  p += b_ids;
  m->attn_cnt = (int *)p;  // zero (the memset above); each attention launch leaves it zero
  // argmax of the all-zero logits BlockWorkspace starts with is id 0
  std::vector<float2> part0(m->nparts);
  uint32_t none = 0xffffffffu, zero = 0;
  float none_f, zero_f;
  memcpy(&none_f, &none, 4);
  memcpy(&zero_f, &zero, 4);
  for (auto &q2 : part0) q2 = make_float2(-INFINITY, none_f);
  part0[0] = make_float2(0.0f, zero_f);
  HIP_TRY(hipMemcpyAsync(m->part, part0.data(), part0.size() * sizeof(float2),
                         hipMemcpyHostToDevice, m->stream));
  HIP_TRY(hipHostMalloc((void **)&m->host_state, 4 * sizeof(uint32_t), hipHostMallocDefault));
  rc = setup_persistent(m);
  if (rc) return rc;
  HIP_TRY(hipStreamSynchronize(m->stream));
  return MYOS_OK;
}

int myos_model_open(const char *path, const myos_block_shape *shape, int kv_dtype,
                    size_t max_seq, myos_model **out) {
  if (!path || !shape || !out) return MYOS_E_ARG;
  *out = nullptr;
  myos_model *m = new myos_model();
  int rc = open_impl(m, path, shape, kv_dtype, max_seq);
  if (rc) {
    myos_model_close(m);
    return rc;
  }
  *out = m;
  return MYOS_OK;
}

// qwen25_block.rs:323-543
int myos_prefill(myos_model *m, const uint32_t *tokens, size_t n) {
  if (!m || (!tokens && n)) return MYOS_E_ARG;
  if (n == 0) return MYOS_E_SHAPE;
  const size_t start = m->len;
  if (start >= m->max_seq) return MYOS_E_KV_FULL;
  if (n > m->max_seq - start) return MYOS_E_KV_FULL;
  for (size_t i = 0; i < n; i++)
    if ((size_t)tokens[i] >= m->s.vocab) return MYOS_E_TOKEN;
  int rc = ensure_prefill(m, n);
  if (rc) return rc;
  const myos_block_shape &s = m->s;
  const int H = (int)s.hidden, I = (int)s.intermediate, M = (int)n;
  hipStream_t st = m->stream;
  HIP_TRY(hipMemcpyAsync(m->ptok, tokens, n * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipEventRecord(m->ev0, st));
  HIP_TRY(launch_embed_rows(m->pX, m->embed, m->ptok, M, H, st));
  // layer 0's ln1 here; every later norm rides on the GEMM before it
  HIP_TRY(launch_rmsnorm_rows_split(m->pX, m->layers[0].ln1, s.rms_eps, M, H, m->pAhi, m->pAlo, st));
  for (size_t l = 0; l < s.num_layers; l++) {
    const DevLayer &L = m->layers[l];
    GemmArgs g{};
    g.a_hi = m->pAhi;
    g.a_lo = m->pAlo;
    g.w = L.wqkv;
    g.M = M;
    g.N = (int)m->qkv_rows;
    g.K = H;
    g.bias = L.bqkv;
    g.rope = m->rope;
    g.start_pos = (int)start;
    g.q_out = m->pQ;
    g.kc = m->kc_layer(l);
    g.vc = m->vc_layer(l);
    g.kv_bf16 = m->kv_bf16;
    g.max_seq = (int)m->max_seq;
    g.q_dim = (int)m->q_dim;
    g.kv_dim = (int)m->kv_dim;
    g.head_dim = (int)s.head_dim;
    g.ws = m->pws;
    g.ws_cap = m->pws_cap;
    HIP_TRY(launch_gemm(g, EPI_QKV, st));

    AttnPrefillArgs ap;
    ap.q = m->pQ;
    ap.kc = m->kc_layer(l);
    ap.vc = m->vc_layer(l);
    ap.kv_bf16 = m->kv_bf16;
    ap.max_seq = (int)m->max_seq;
    ap.nq = (int)s.num_q_heads;
    ap.nkv = (int)s.num_kv_heads;
    ap.head_dim = (int)s.head_dim;
    ap.M = M;
    ap.start_pos = (int)start;
    ap.out_hi = m->pAhi;  // the normed planes are dead after the QKV GEMM
    ap.out_lo = m->pAlo;
    ap.part = m->pws;     // the QKV GEMM's partials are reduced by now
    ap.part_cap = m->pws_cap;
    HIP_TRY(launch_attn_prefill(ap, st));

    GemmArgs o{};
    o.a_hi = m->pAhi;
    o.a_lo = m->pAlo;
    o.w = L.wo;
    o.M = M;
    o.N = H;
    o.K = (int)m->q_dim;
    o.y = m->pX;
    o.ws = m->pws;
    o.ws_cap = m->pws_cap;
    HIP_TRY(launch_gemm_resid_norm(o, L.ln2, s.rms_eps, m->pAhi, m->pAlo, st));

    GemmArgs gu{};
    gu.a_hi = m->pAhi;
    gu.a_lo = m->pAlo;
    gu.w = L.wgu;
    gu.M = M;
    gu.N = (int)m->gu_rows;
    gu.K = H;
    gu.h_hi = m->pHhi;
    gu.h_lo = m->pHlo;
    gu.ws = m->pws;
    gu.ws_cap = m->pws_cap;
    HIP_TRY(launch_gemm(gu, EPI_GU, st));

    GemmArgs dn{};
    dn.a_hi = m->pHhi;
    dn.a_lo = m->pHlo;
    dn.w = L.wd;
    dn.M = M;
    dn.N = H;
    dn.K = I;
    dn.y = m->pX;
    dn.ws = m->pws;
    dn.ws_cap = m->pws_cap;
    if (l + 1 < s.num_layers)
      HIP_TRY(launch_gemm_resid_norm(dn, m->layers[l + 1].ln1, s.rms_eps, m->pAhi, m->pAlo, st));
    else
      HIP_TRY(launch_gemm(dn, EPI_RESID, st));
  }
  const float *last = m->pX + (size_t)(M - 1) * H;
  HIP_TRY(hipMemcpyAsync(m->x, last, (size_t)H * 4, hipMemcpyDeviceToDevice, st));
  GemvArgs hd;
  hd.w = m->head;
  hd.x = m->x;
  hd.gamma = m->final_norm;
  hd.eps = s.rms_eps;
  hd.m = (int)s.vocab;
  hd.k = H;
  hd.y = m->logits;
  hd.part = m->part;
  hd.part_cap = m->nparts;
  hd.normed_out = m->normed;
  HIP_TRY(launch_gemv(hd, X_NORM, EPI_HEAD, st));
  HIP_TRY(hipEventRecord(m->ev1, st));
  const size_t end = start + n;
  rc = write_state(m, (uint32_t)end, 0, 0, 0);  // synchronizes the prefill first
  if (rc) return rc;
  float ms = 0;
  HIP_TRY(hipEventElapsedTime(&ms, m->ev0, m->ev1));
  m->prefill_ms = ms;
  m->len = end;
  m->poisoned = false;  // logits, argmax partials and residual are fresh again
  return MYOS_OK;
}

// qwen25_block.rs:220-304
int myos_forward_token(myos_model *m, uint32_t token, size_t pos) {
  if (!m) return MYOS_E_ARG;
  if (m->poisoned) return MYOS_E_HIP;
  if (pos != m->len) return MYOS_E_POSITION;
  if (pos >= m->max_seq) return MYOS_E_KV_FULL;
  if ((size_t)token >= m->s.vocab) return MYOS_E_TOKEN;
  int rc = write_state(m, (uint32_t)pos, token, 0, 1);
  if (rc) return rc;
  rc = run_steps(m, 1);
  if (rc) return rc;
  HIP_TRY(hipStreamSynchronize(m->stream));
  m->len += 1;
  return MYOS_OK;
}

// qwen25_block.rs:765-780
int myos_greedy_decode(myos_model *m, size_t steps, uint32_t *out) {
  if (!m || (!out && steps)) return MYOS_E_ARG;
  if (m->poisoned) return MYOS_E_HIP;
  const size_t room = m->max_seq - m->len;
  const size_t n = steps < room ? steps : room;
  if (n) {
    int rc = decode_run(m, n, 0, out);
    if (rc) return rc;
  }
  return n < steps ? MYOS_E_KV_FULL : MYOS_OK;
}

int myos_decode_forced(myos_model *m, const uint32_t *ids, size_t steps, uint32_t *argmax_out) {
  if (!m || (steps && (!ids || !argmax_out))) return MYOS_E_ARG;
  if (m->poisoned) return MYOS_E_HIP;
  if (steps > m->max_seq - m->len) return MYOS_E_KV_FULL;
  for (size_t i = 0; i < steps; i++)
    if ((size_t)ids[i] >= m->s.vocab) return MYOS_E_TOKEN;
  if (!steps) return MYOS_OK;
  HIP_TRY(hipStreamSynchronize(m->stream));
  HIP_TRY(hipMemcpy(m->force_ids, ids, steps * 4, hipMemcpyHostToDevice));
  return decode_run(m, steps, 2, argmax_out);
}

size_t myos_cache_len(const myos_model *m) { return m ? m->len : 0; }

// attention_layer, attn_wire.rs:207-313: residual += o_proj(attention(q, k, v
// of proj_in)) for one layer at position pos = the cache cursor, storing the
// layer's K/V row at pos; the cursor does not move (myos_kv_advance moves
// it). residual and proj_in are host vectors of `hidden` floats. Every check
// runs before anything is launched, so on an error residual and the cache
// are unchanged.
int myos_attention_layer(myos_model *m, size_t layer, size_t pos, float *residual, const float *proj_in,
                         size_t len) {
  if (!m || !residual || !proj_in) return MYOS_E_ARG;
  if (m->poisoned) return MYOS_E_HIP;
  if (len != m->s.hidden) return MYOS_E_SHAPE;
  if (layer >= m->s.num_layers) return MYOS_E_KV_RANGE;
  if (pos != m->len) return MYOS_E_POSITION;
  if (pos >= m->max_seq) return MYOS_E_KV_FULL;
  const myos_block_shape &s = m->s;
  const DevLayer &L = m->layers[layer];
  int rc = write_state(m, (uint32_t)pos, 0, 0, 1);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(m->x, residual, len * sizeof(float), hipMemcpyHostToDevice, m->stream));
  HIP_TRY(hipMemcpyAsync(m->normed, proj_in, len * sizeof(float), hipMemcpyHostToDevice, m->stream));
  // q/k/v GEMV of the caller's vector (no norm prologue) + bias, RoPE, K/V store
  GemvArgs g;
  g.w = L.wqkv;
  g.x = m->normed;
  g.m = (int)m->qkv_rows;
  g.k = (int)s.hidden;
  g.bias = L.bqkv;
  g.rope = m->rope;
  g.pos_ptr = m->state;
  g.q_out = m->q;
  g.kc = m->kc_layer(layer);
  g.vc = m->vc_layer(layer);
  g.kv_bf16 = m->kv_bf16;
  g.max_seq = (int)m->max_seq;
  g.q_dim = (int)m->q_dim;
  g.kv_dim = (int)m->kv_dim;
  g.head_dim = (int)s.head_dim;
  HIP_TRY(launch_gemv(g, X_PLAIN, EPI_QKV, m->stream));
  rc = enq_kernel(m, MYOS_K_ATTN, layer, false);
  if (!rc) rc = enq_kernel(m, MYOS_K_O, layer, false);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(residual, m->x, len * sizeof(float), hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  return MYOS_OK;
}

// KvCache::advance, kv_cache.rs:226-232: one step of the shared cursor
int myos_kv_advance(myos_model *m) {
  if (!m) return MYOS_E_ARG;
  if (m->len >= m->max_seq) return MYOS_E_KV_FULL;
  m->len += 1;
  return write_state(m, (uint32_t)m->len, 0, 0, 0);
}

int myos_cache_clear(myos_model *m) {
  if (!m) return MYOS_E_ARG;
  m->len = 0;
  m->poisoned = false;
  return write_state(m, 0, 0, 0, 0);
}

int myos_time_kernel(myos_model *m, int which, int reps, double *avg_ms) {
  if (!m || !avg_ms || reps <= 0 || which < MYOS_K_QKV || which > MYOS_K_HEAD) return MYOS_E_ARG;
  // a valid position for the kernels that read it (the cursor may be at max_seq)
  const uint32_t pos = (uint32_t)(m->len < m->max_seq ? m->len : m->max_seq - 1);
  int rc = write_state(m, pos, 0, 0, 0);
  if (rc) return rc;
  const size_t n = which == MYOS_K_HEAD ? 1 : m->s.num_layers;
  if (!m->use_graph) {
    // plain launches (for tools that do not follow graph replays)
    for (size_t l = 0; l < n && !rc; l++) rc = enq_kernel(m, which, l, false);  // warm
    if (!rc) rc = hs(hipEventRecord(m->ev0, m->stream));
    for (int r = 0; r < reps && !rc; r++)
      for (size_t l = 0; l < n && !rc; l++) rc = enq_kernel(m, which, l, false);
    if (!rc) rc = hs(hipEventRecord(m->ev1, m->stream));
    if (!rc) rc = hs(hipStreamSynchronize(m->stream));
    float ms = 0;
    if (!rc) rc = hs(hipEventElapsedTime(&ms, m->ev0, m->ev1));
    if (rc) return rc;
    *avg_ms = (double)ms / ((double)reps * (double)n);
    return MYOS_OK;
  }
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  HIP_TRY(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
  for (size_t l = 0; l < n && !rc; l++) rc = enq_kernel(m, which, l, false);
  hipError_t e = hipStreamEndCapture(m->stream, &g);
  if (rc || e != hipSuccess || !g) {
    if (g) (void)hipGraphDestroy(g);
    return rc ? rc : MYOS_E_HIP;
  }
  e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return MYOS_E_HIP;
  rc = hs(hipGraphLaunch(ge, m->stream));  // warm
  if (!rc) rc = hs(hipEventRecord(m->ev0, m->stream));
  for (int r = 0; r < reps && !rc; r++) rc = hs(hipGraphLaunch(ge, m->stream));
  if (!rc) rc = hs(hipEventRecord(m->ev1, m->stream));
  if (!rc) rc = hs(hipStreamSynchronize(m->stream));
  float ms = 0;
  if (!rc) rc = hs(hipEventElapsedTime(&ms, m->ev0, m->ev1));
  (void)hipGraphExecDestroy(ge);
  if (rc) return rc;
  *avg_ms = (double)ms / ((double)reps * (double)n);
  return MYOS_OK;
}

double myos_kernel_bytes(const myos_model *m, int which) {
  if (!m) return 0.0;
  const double H = (double)m->s.hidden, I = (double)m->s.intermediate, V = (double)m->s.vocab;
  const double Q = (double)m->q_dim, KD = (double)m->kv_dim, R = (double)m->qkv_rows;
  const double skv = m->kv_bf16 ? 2.0 : 4.0;
  const double seq = (double)(m->len < m->max_seq ? m->len : m->max_seq - 1) + 1.0;
  switch (which) {
    case MYOS_K_QKV: return R * H * 2 + R * 4 + H * 2 + H * 4 + Q * 4 + 2 * KD * skv;
    case MYOS_K_ATTN: return Q * 4 + 2 * KD * seq * skv + Q * 4;
    case MYOS_K_O: return H * Q * 2 + Q * 4 + 2 * H * 4;
    case MYOS_K_GATE_UP: return 2 * I * H * 2 + H * 2 + H * 4 + I * 4;
    case MYOS_K_DOWN: return H * I * 2 + I * 4 + 2 * H * 4;
    case MYOS_K_HEAD: return V * H * 2 + H * 2 + H * 4 + V * 4;
    default: return 0.0;
  }
}
size_t myos_max_seq(const myos_model *m) { return m ? m->max_seq : 0; }

static int copy_out(const myos_model *m, const float *src, size_t have, float *out, size_t n) {
  if (!m || !out) return MYOS_E_ARG;
  if (n != have) return MYOS_E_SHAPE;
  HIP_TRY(hipStreamSynchronize(m->stream));
  HIP_TRY(hipMemcpy(out, src, n * 4, hipMemcpyDeviceToHost));
  return MYOS_OK;
}

int myos_copy_logits(const myos_model *m, float *out, size_t n) {
  return copy_out(m, m ? m->logits : nullptr, m ? m->s.vocab : 0, out, n);
}
int myos_copy_hidden(const myos_model *m, float *out, size_t n) {
  return copy_out(m, m ? m->x : nullptr, m ? m->s.hidden : 0, out, n);
}
int myos_copy_normed(const myos_model *m, float *out, size_t n) {
  return copy_out(m, m ? m->normed : nullptr, m ? m->s.hidden : 0, out, n);
}

int myos_kv_read(const myos_model *m, size_t layer, size_t head, size_t pos, float *k, float *v) {
  if (!m || !k || !v) return MYOS_E_ARG;
  if (layer >= m->s.num_layers || head >= m->s.num_kv_heads || pos >= m->max_seq)
    return MYOS_E_KV_RANGE;
  const size_t d = m->s.head_dim, off = (head * m->max_seq + pos) * d;
  HIP_TRY(hipStreamSynchronize(m->stream));
  if (!m->kv_bf16) {
    HIP_TRY(hipMemcpy(k, (const float *)m->kc_layer(layer) + off, d * 4, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(v, (const float *)m->vc_layer(layer) + off, d * 4, hipMemcpyDeviceToHost));
  } else {
    std::vector<uint16_t> tk(d), tv(d);
    HIP_TRY(hipMemcpy(tk.data(), (const uint16_t *)m->kc_layer(layer) + off, d * 2,
                      hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(tv.data(), (const uint16_t *)m->vc_layer(layer) + off, d * 2,
                      hipMemcpyDeviceToHost));
    for (size_t i = 0; i < d; i++) {
      k[i] = bf16_to_f32_host(tk[i]);
      v[i] = bf16_to_f32_host(tv[i]);
    }
  }
  return MYOS_OK;
}

int myos_set_decode_mode(myos_model *m, int mode) {
  if (!m || mode < MYOS_DECODE_AUTO || mode > MYOS_DECODE_STREAMED) return MYOS_E_ARG;
  if (mode == MYOS_DECODE_PERSISTENT && !m->persist_ok && !m->wide_ok) return MYOS_E_SHAPE;
  if (mode == MYOS_DECODE_STREAMED && !m->wide_ok) return MYOS_E_SHAPE;
  m->decode_mode = mode;
  return MYOS_OK;
}

int myos_set_decode_trace(myos_model *m, int64_t step) {
  if (!m) return MYOS_E_ARG;
  if (step < 0) {
    m->trace_step = -1;
    return MYOS_OK;
  }
  if (!m->persist_ok) return MYOS_E_SHAPE;
  if (!m->trace) {
    const size_t n = (size_t)persist_grid() * (5 * m->s.num_layers + 3);
    HIP_TRY(hipMalloc((void **)&m->trace, n * sizeof(uint64_t)));
    HIP_TRY(hipMemset(m->trace, 0, n * sizeof(uint64_t)));
  }
  m->trace_step = step;
  return MYOS_OK;
}

int myos_debug_raise_wait_error(myos_model *m) {
  if (!m) return MYOS_E_ARG;
  if (!m->persist_ok && !m->wide_ok) return MYOS_E_SHAPE;
  const uint32_t one = 1;
  HIP_TRY(hipMemcpyAsync(m->err, &one, 4, hipMemcpyHostToDevice, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  return MYOS_OK;
}

int myos_copy_decode_trace(const myos_model *m, uint64_t *out, size_t n) {
  if (!m || !out) return MYOS_E_ARG;
  if (!m->trace) return MYOS_E_SHAPE;
  if (n != (size_t)persist_grid() * (5 * m->s.num_layers + 3)) return MYOS_E_SHAPE;
  HIP_TRY(hipStreamSynchronize(m->stream));
  HIP_TRY(hipMemcpy(out, m->trace, n * sizeof(uint64_t), hipMemcpyDeviceToHost));
  return MYOS_OK;
}

int myos_decode_path(const myos_model *m) {
  if (!m) return MYOS_E_ARG;
  if (!use_persistent(m)) return MYOS_DECODE_KERNELS;
  return use_wide(m) ? MYOS_DECODE_STREAMED : MYOS_DECODE_PERSISTENT;
}

int myos_set_graph(myos_model *m, int enabled) {
  if (!m) return MYOS_E_ARG;
  m->use_graph = enabled != 0;
  return MYOS_OK;
}

double myos_last_prefill_ms(const myos_model *m) { return m ? m->prefill_ms : 0.0; }
double myos_last_decode_ms(const myos_model *m) { return m ? m->decode_ms : 0.0; }
size_t myos_weight_bytes(const myos_model *m) { return m ? m->wbytes : 0; }
size_t myos_kv_bytes(const myos_model *m) { return m ? 2 * m->kv_bytes : 0; }

}  // extern "C"
