// Persistent greedy-decode kernel for MI355X (gfx950).
//
// One cooperative launch of 256 workgroups (one per CU, 512 threads) runs a
// whole run of decode steps. Every workgroup owns fixed rows of every
// projection (QKV, o, gate/up, down, head) and a fixed slice of the residual
// stream; attention work items (kv head, 32-position chunk) are dealt round
// robin. Activations cross workgroups as 64-bit words (value, tag), stored and
// loaded with device-coherent (sc1) accesses; the tag names the step, layer
// and phase that produced the value. A consumer re-polls exactly the words it
// needs until they carry the expected tag, so the only synchronisation is the
// data dependency itself: no grid barrier, no fence, no read-modify-write
// atomic (all three cost microseconds on this part). Each workgroup issues the
// next phase's weight loads before it waits for that phase's inputs, which
// keeps HBM streaming across the dependency chain.
//
// Every wait is bounded: after ~1 s of spinning a workgroup raises the error
// word, and every wait returns at once when that word is set, so the grid
// always drains. The reference's numerics are the same as the per-kernel path
// (crates/model_core/src/qwen25_block.rs:220-304 per step).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "myos_internal.h"

namespace myos {
namespace {

constexpr int NT = 512;              // threads per workgroup
constexpr int NW = NT / 64;          // wavefronts per workgroup
constexpr int NB = 256;              // workgroups (one per CU)
constexpr int HC = 3;                // 8-column chunks per lane, k <= 1536
constexpr int MAXI = 9216;           // intermediate limit (down rows staged in LDS)
constexpr int GPMAX = 5;             // gate/up row pairs per wavefront
constexpr int AC = 32;               // attention positions per work item
constexpr int HT = 2;                // head rows per tile
constexpr int MAXH = 1536;           // hidden / q_dim limit of this kernel
constexpr int MAXD = 128;            // head_dim limit
constexpr int KV4 = (AC * MAXD / 4 + NT - 1) / NT;      // cached-row loads per thread
constexpr int QW = (8 * MAXD + 2 * MAXD + NT - 1) / NT;  // q + k + v words per thread
constexpr unsigned kSpinMax = 1u << 20;
// A word's tag is its step's base + kTPL * layer + phase; the head's partials
// take base + kTPL * layers; a step spans kTPL * layers + 2 tags.
constexpr uint32_t kTPL = 6;
constexpr uint32_t P_QKV = 0, P_PART = 1, P_XO = 2, P_H = 3, P_XD = 4, P_ATT = 5;
constexpr size_t kMaxLds = 159 * 1024;  // dynamic LDS: 160 KB per workgroup on gfx950 less the static part

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
__device__ __forceinline__ float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Cross-lane reductions with DPP lane moves (a few cycles each; a
// __shfl_xor is an LDS permute round trip). gfx9 DPP controls: quad_perm
// [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, row_half_mirror 0x141, row_mirror
// 0x140, row_bcast:15 0x142, row_bcast:31 0x143. Rows outside ROW_MASK keep
// `old`, the identity of the reduction.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float v, float old) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL,
                                                    ROW_MASK, 0xF, false));
}
// sum / max over the wavefront, returned to every lane
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v, 0.f);
  v += dpp<0x4E>(v, 0.f);
  v += dpp<0x141>(v, 0.f);
  v += dpp<0x140>(v, 0.f);
  v += dpp<0x142, 0xA>(v, 0.f);  // row 0 into row 1, row 2 into row 3
  v += dpp<0x143, 0xC>(v, 0.f);  // rows 0 + 1 into rows 2, 3: lane 63 holds the total
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v, -INFINITY));
  v = fmaxf(v, dpp<0x4E>(v, -INFINITY));
  v = fmaxf(v, dpp<0x141>(v, -INFINITY));
  v = fmaxf(v, dpp<0x140>(v, -INFINITY));
  v = fmaxf(v, dpp<0x142, 0xA>(v, -INFINITY));
  v = fmaxf(v, dpp<0x143, 0xC>(v, -INFINITY));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ bool beats(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && v != -INFINITY && i < bi);
}

// ---- device-coherent exchange ------------------------------------------------
__device__ __forceinline__ void tput(uint64_t *p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tload(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cstore(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool err_raised(const PersistArgs &a) {
  return __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}

// Called every spin of a wait: every 64 spins, past the limit raise the error
// word, and report whether it is raised (then every wait gives up at once).
__device__ __forceinline__ bool spin_fail(const PersistArgs &a, unsigned spins) {
  if ((spins & 63) != 63) return false;
  if (spins > kSpinMax) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return err_raised(a);
}

// Gather n tagged words (index i -> src[map(i)]) into dst[i]; the whole
// workgroup waits until every word carries `tag`. Returns false (and leaves
// garbage in dst) when the wait failed or an earlier one did.
template <int U, class Map>
__device__ bool tgather(const uint64_t *src, Map map, int n, uint32_t tag, float *dst,
                        const PersistArgs &a, int *fail) {
  bool ok = *fail == 0;
  for (int i0 = threadIdx.x; i0 < n && ok; i0 += NT * U) {
    uint64_t w[U];
    for (unsigned spins = 0;; spins++) {
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int i = i0 + u * NT;
        w[u] = i < n ? tload(src + map(i)) : ((uint64_t)tag << 32);
      }
      bool ready = true;
#pragma unroll
      for (int u = 0; u < U; u++) ready = ready && (uint32_t)(w[u] >> 32) == tag;
      if (ready) break;
      if (spin_fail(a, spins)) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = i0 + u * NT;
      if (i < n) dst[i] = __uint_as_float((uint32_t)w[u]);
    }
  }
  if (!ok) *fail = 1;
  __syncthreads();
  return *fail == 0;
}

struct Linear {
  __device__ int operator()(int i) const { return i; }
};

// tgather for src[0, n) in order: one buffer descriptor, one lane offset and
// per-unroll constant offsets keep the address cost at one register. The
// loads are sc1 (device-coherent) and volatile, so a spin re-reads memory.
template <int U>
__device__ bool tgather_lin(const uint64_t *src, int n, uint32_t tag, float *dst,
                            const PersistArgs &a, int *fail) {
  constexpr int kAux = 16 | (1 << 31);  // sc1, volatile
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, n * 8, 0x00020000);
  bool ok = *fail == 0;
  for (int i0 = threadIdx.x; i0 < n && ok; i0 += NT * U) {
    uint64_t w[U];
    for (unsigned spins = 0;; spins++) {
#pragma unroll
      for (int u = 0; u < U; u++)
        if (i0 + u * NT < n) {
          const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, i0 * 8, u * NT * 8, kAux);
          w[u] = ((uint64_t)v.y << 32) | v.x;
        } else {
          w[u] = (uint64_t)tag << 32;
        }
      bool ready = true;
#pragma unroll
      for (int u = 0; u < U; u++) ready = ready && (uint32_t)(w[u] >> 32) == tag;
      if (ready) break;
      if (spin_fail(a, spins)) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = i0 + u * NT;
      if (i < n) dst[i] = __uint_as_float((uint32_t)w[u]);
    }
  }
  if (!ok) *fail = 1;
  __syncthreads();
  return *fail == 0;
}

// ---- row tiles -----------------------------------------------------------------
template <int C>
__device__ __forceinline__ void ldrow(u32x4 (&t)[C], const uint16_t *W, int k, int row, bool valid,
                                      int lane) {
  const int nch = k >> 3;
  const u32x4 *rp = (const u32x4 *)(W + (size_t)(valid ? row : 0) * k);
#pragma unroll
  for (int i = 0; i < C; i++) {
    const int c = lane + i * 64;
    const u32x4 zero = {0u, 0u, 0u, 0u};
    t[i] = (valid && c < nch) ? __builtin_nontemporal_load(rp + c) : zero;
  }
}

// Stream one row into LDS with direct (DMA) loads: chunk c of the row lands at
// dst + 16 c. `dst` must be wave-uniform; no registers hold the row meanwhile.
// The compiler waits for these loads before the wave's next LDS read.
__device__ __forceinline__ void dma_row(const uint16_t *W, int k, int row, bool valid, uint8_t *dst,
                                        int lane) {
  const int nch = k >> 3;
  const u32x4 *rp = (const u32x4 *)(W + (size_t)(valid ? row : 0) * k);
  for (int i = 0; i * 64 < nch; i++) {
    const int c = lane + i * 64;
    if (valid && c < nch)
      __builtin_amdgcn_global_load_lds((const void *)(rp + c),
                                       (__attribute__((address_space(3))) void *)(dst + i * 1024),
                                       16, 0, 2 /* nt */);
  }
}

// row held in LDS (16 bytes per 8-column chunk) dotted with x in LDS
__device__ __forceinline__ float dotrow_lds(const uint8_t *wl, const float *x, int k, int lane) {
  const int nch = k >> 3;
  float s = 0.f;
  for (int c = lane; c < nch; c += 64) {
    const u32x4 w = *(const u32x4 *)(wl + c * 16);
    const float4 x0 = *(const float4 *)(x + c * 8), x1 = *(const float4 *)(x + c * 8 + 4);
    s = fmaf(bf_lo(w.x), x0.x, s);
    s = fmaf(bf_hi(w.x), x0.y, s);
    s = fmaf(bf_lo(w.y), x0.z, s);
    s = fmaf(bf_hi(w.y), x0.w, s);
    s = fmaf(bf_lo(w.z), x1.x, s);
    s = fmaf(bf_hi(w.z), x1.y, s);
    s = fmaf(bf_lo(w.w), x1.z, s);
    s = fmaf(bf_hi(w.w), x1.w, s);
  }
  return wave_sum(s);
}

// one row (held 8 columns per chunk per lane) dotted with x in LDS; all lanes
// get the sum
template <int C>
__device__ __forceinline__ float dotrow(const u32x4 (&t)[C], const float *x, int k, int lane) {
  const int nch = k >> 3;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < C; i++) {
    const int c = lane + i * 64;
    if (c < nch) {
      const float4 x0 = *(const float4 *)(x + c * 8), x1 = *(const float4 *)(x + c * 8 + 4);
      const u32x4 w = t[i];
      s = fmaf(bf_lo(w.x), x0.x, s);
      s = fmaf(bf_hi(w.x), x0.y, s);
      s = fmaf(bf_lo(w.y), x0.z, s);
      s = fmaf(bf_hi(w.y), x0.w, s);
      s = fmaf(bf_lo(w.z), x1.x, s);
      s = fmaf(bf_hi(w.z), x1.y, s);
      s = fmaf(bf_lo(w.w), x1.z, s);
      s = fmaf(bf_hi(w.w), x1.w, s);
    }
  }
  return wave_sum(s);
}

// x <- g * (x * 1/sqrt(mean(x^2) + eps)) in LDS (rmsnorm_bf16_weight,
// crates/tensor_core/src/bf16.rs:231-270, with a tree sum)
__device__ void rmsnorm_lds(float *x, const uint16_t *g, int n, float eps, float *red) {
  float ss = 0.f;
  for (int j = threadIdx.x; j < n; j += NT) ss += x[j] * x[j];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < NW; w++) tot += red[w];
  const float inv = 1.0f / sqrtf(tot / (float)n + eps);
  for (int j = threadIdx.x; j < n; j += NT) x[j] = bf16f(g[j]) * (x[j] * inv);
  __syncthreads();
}

__device__ __forceinline__ float silu(float z) { return z / (1.0f + expf(-z)); }

// phase timestamps of one step (100 MHz device clock), thread 0 of each
// workgroup: slot 0 token chosen; 1 + 5 l + {0 x ready, 1 attention items
// done, 2 attention merged, 3 X_o ready, 4 h ready}; 1 + 5 L head input ready;
// 2 + 5 L head done
__device__ __forceinline__ void mark(const PersistArgs &a, uint32_t s, int slot) {
  if (a.trace && s == a.trace_step && threadIdx.x == 0)
    a.trace[(size_t)blockIdx.x * (5 * a.L + 3) + slot] = wall_clock64();
}

__global__ void __launch_bounds__(NT) decode_persistent_kernel(PersistArgs a) {
  extern __shared__ float4 sm4[];
  float *xs = (float *)sm4;     // [MAXH] activation for the current phase
  float *att = xs + MAXH;       // [MAXH] attention output
  float *big = att + MAXH;      // phase scratch: h [I] / attention staging / merge weights
  uint8_t *wdl = (uint8_t *)(xs + a.lds_wd);  // [rows per workgroup][I] bf16 down rows
  __shared__ float red[NW * 2];
  __shared__ float xl[NW];      // this workgroup's rows of the residual stream
  __shared__ int fail_s;
  __shared__ uint32_t tok_s;
  __shared__ float2 best_s[NW];

  const int tid = threadIdx.x, lane = tid & 63, wg = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, I = a.I, d = a.d, half = d >> 1, gq = a.nq / a.nkv;
  const int qdim = a.nq * d, kvdim = a.nkv * d;
  const uint32_t TPS = (uint32_t)a.L * kTPL + 2;
  const int nchmax = (a.max_seq + AC - 1) / AC;
  // ownership
  const int qper = (((a.qkv_rows + NB - 1) / NB) + 1) & ~1;
  const int q0 = wg * qper, q1 = min(q0 + qper, a.qkv_rows);
  const int xper = (H + NB - 1) / NB;
  const int x0 = wg * xper, x1 = min(x0 + xper, H);
  const int gper = (((2 * I + NB - 1) / NB) + 1) & ~1;
  const int g0 = wg * gper, g1 = min(g0 + gper, 2 * I);
  const int vper = (a.V + NB - 1) / NB;
  const int v0 = wg * vper, v1 = min(v0 + vper, a.V);
  const int qrow = q0 + 2 * wave;      // this wave's QKV pair
  const int xrow = x0 + wave;          // this wave's residual row (o and down)
  const bool has_q = qrow < q1, has_x = xrow < x1;

  if (tid == 0) fail_s = 0;
  if (tid < NW) xl[tid] = 0.f;
  __syncthreads();

  // weight tiles held in registers across phases
  u32x4 wq0[HC], wq1[HC], wo[HC];
  u32x4 gA0[HC], gA1[HC], gB0[HC], gB1[HC];  // gate/up pairs, two stages in flight

  auto issue_qo = [&](int l) {
    const PersistLayer &L = a.layers[l];
    ldrow<HC>(wq0, L.wqkv, H, qrow, has_q, lane);
    ldrow<HC>(wq1, L.wqkv, H, qrow + 1, has_q, lane);
    ldrow<HC>(wo, L.wo, qdim, xrow, has_x, lane);
  };
  // gate/up pair p of this wavefront (rows 2i, 2i+1 = gate_i, up_i)
  auto gu_row = [&](int p) { return g0 + 2 * (wave + p * NW); };

  issue_qo(0);
  for (uint32_t s = 0; s < a.steps; s++) {
    const uint32_t pos = a.pos0 + s;
    const int seq = (int)pos + 1;
    const uint32_t tstep = a.tag_base + s * TPS;

    // ---- greedy token: argmax of the previous logits --------------------
    {
      float bv = -INFINITY;
      uint32_t bi = 0xffffffffu;
      if (s == 0) {
        for (int i = tid; i < a.nparts_in; i += NT) {
          const float2 p = a.part_in[i];
          if (beats(p.x, __float_as_uint(p.y), bv, bi)) {
            bv = p.x;
            bi = __float_as_uint(p.y);
          }
        }
      } else {
        float *pp = big;  // [2 * NB]: value, index bits
        tgather_lin<1>(a.targ, 2 * NB, tstep - TPS + (uint32_t)a.L * kTPL, pp, a, &fail_s);
        if (tid < NB) {
          bv = pp[2 * tid];
          bi = __float_as_uint(pp[2 * tid + 1]);
        }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        if (beats(ov, oi, bv, bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (lane == 0) best_s[wave] = make_float2(bv, __uint_as_float(bi));
      __syncthreads();
      if (tid == 0) {
        float2 b = best_s[0];
        for (int w = 1; w < NW; w++)
          if (beats(best_s[w].x, __float_as_uint(best_s[w].y), b.x, __float_as_uint(b.y)))
            b = best_s[w];
        const uint32_t idx = __float_as_uint(b.y);
        tok_s = idx < (uint32_t)a.V ? idx : 0u;  // no candidate (all NaN / -inf) -> 0
        if (wg == 0) a.out_ids[s] = tok_s;
      }
      __syncthreads();
      const uint16_t *erow = a.embed + (size_t)tok_s * H;
      for (int j = tid; j < H; j += NT) xs[j] = bf16f(erow[j]);
      if (tid < NW && x0 + tid < x1) xl[tid] = bf16f(erow[x0 + tid]);
      __syncthreads();
      mark(a, s, 0);
    }

    for (int l = 0; l < a.L; l++) {
      const PersistLayer &L = a.layers[l];
      const uint32_t T = tstep + (uint32_t)l * kTPL;
      float *kc = a.kc + (size_t)l * a.layer_kv, *vc = a.vc + (size_t)l * a.layer_kv;

      // ---- QKV + bias + RoPE + KV store (tag T + P_QKV) ---------------------
      if (l > 0) tgather_lin<3>(a.txd, H, T - kTPL + P_XD, xs, a, &fail_s);
      mark(a, s, 1 + 5 * l);
      rmsnorm_lds(xs, L.ln1, H, a.eps, red);
      if (has_q) {
        const float y0 = dotrow<HC>(wq0, xs, H, lane), y1 = dotrow<HC>(wq1, xs, H, lane);
        if (lane == 0) {
          const float b0 = y0 + L.bqkv[qrow], b1 = y1 + L.bqkv[qrow + 1];
          if (qrow < qdim + kvdim) {
            const bool is_q = qrow < qdim;
            const int rr = is_q ? qrow : qrow - qdim;
            const int u = rr >> 1, head = u / half, p = u - head * half;
            const float2 cs = a.rope[(size_t)pos * half + p];
            const float o0 = b0 * cs.x - b1 * cs.y, o1 = b1 * cs.x + b0 * cs.y;
            if (is_q) {
              tput(a.tq + head * d + p, o0, T + P_QKV);
              tput(a.tq + head * d + p + half, o1, T + P_QKV);
            } else {
              const size_t base = ((size_t)head * a.max_seq + pos) * d;
              cstore(kc + base + p, o0);
              cstore(kc + base + p + half, o1);
              tput(a.tkv + head * d + p, o0, T + P_QKV);
              tput(a.tkv + head * d + p + half, o1, T + P_QKV);
            }
          } else {
            const int rr = qrow - qdim - kvdim, head = rr / d, j = rr - head * d;
            const size_t base = ((size_t)head * a.max_seq + pos) * d + j;
            cstore(vc + base, b0);
            cstore(vc + base + 1, b1);
            tput(a.tkv + kvdim + head * d + j, b0, T + P_QKV);
            tput(a.tkv + kvdim + head * d + j + 1, b1, T + P_QKV);
          }
          // the cache rows must be complete before anything this workgroup
          // publishes later: later steps read them without tags
          __builtin_amdgcn_s_waitcnt(0);
        }
      }

      // ---- attention partials for (kv head, chunk) items (tag T + P_PART) ----
      const int nch = (seq + AC - 1) / AC;
      for (int it = wg; it < a.nkv * nch; it += NB) {
        const int g = it % a.nkv, c = it / a.nkv;
        const int t0 = c * AC, n = min(AC, seq - t0);
        const bool has_cur = (int)pos < t0 + n;  // this step's row ends the chunk
        const int nold = has_cur ? n - 1 : n;
        float *q_s = big;                    // [gq][d]
        float *k_s = q_s + gq * d;           // [AC][d + 1]
        float *v_s = k_s + AC * (d + 1);     // [AC][d]
        float *p_s = v_s + AC * d;           // [gq][AC]
        float *ml = p_s + gq * AC;           // [gq][2]
        // cached rows (positions < pos, complete before this step) and the
        // tagged q heads + this step's k, v of head g, all in one round trip
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            kc, (short)0, (int)(a.layer_kv * sizeof(float)), 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            vc, (short)0, (int)(a.layer_kv * sizeof(float)), 0x00020000);
        const int dq = d >> 2;
        u32x4 kr[KV4], vr[KV4];
#pragma unroll
        for (int u = 0; u < KV4; u++) {
          const int i = tid + u * NT;
          if (i < nold * dq) {
            const int t = i / dq, j4 = i - t * dq;
            const uint32_t off = (uint32_t)((((size_t)g * a.max_seq + t0 + t) * d + j4 * 4) * 4);
            kr[u] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 16);
            vr[u] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 16);
          }
        }
        const int nqw = gq * d, nw = nqw + (has_cur ? 2 * d : 0);
        const uint64_t *srcw[QW];
#pragma unroll
        for (int u = 0; u < QW; u++) {
          const int i = tid + u * NT, r = i - nqw;
          srcw[u] = i < nqw ? a.tq + g * gq * d + i
                            : r < d ? a.tkv + g * d + r : a.tkv + kvdim + g * d + (r - d);
        }
        uint64_t w[QW];
        for (unsigned spins = 0; fail_s == 0; spins++) {
          bool ready = true;
#pragma unroll
          for (int u = 0; u < QW; u++) {
            w[u] = tid + u * NT < nw ? tload(srcw[u]) : ((uint64_t)(T + P_QKV) << 32);
            ready = ready && (uint32_t)(w[u] >> 32) == T + P_QKV;
          }
          if (ready) break;
          if (spin_fail(a, spins)) {
            fail_s = 1;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int u = 0; u < KV4; u++) {
          const int i = tid + u * NT;
          if (i < nold * dq) {
            const int t = i / dq, j4 = i - t * dq;
            float *kd = k_s + t * (d + 1) + j4 * 4;
            kd[0] = __uint_as_float(kr[u].x);
            kd[1] = __uint_as_float(kr[u].y);
            kd[2] = __uint_as_float(kr[u].z);
            kd[3] = __uint_as_float(kr[u].w);
            *(float4 *)(v_s + t * d + j4 * 4) =
                make_float4(__uint_as_float(vr[u].x), __uint_as_float(vr[u].y),
                            __uint_as_float(vr[u].z), __uint_as_float(vr[u].w));
          }
        }
#pragma unroll
        for (int u = 0; u < QW; u++) {
          const int i = tid + u * NT, r = i - nqw;
          const float v = __uint_as_float((uint32_t)w[u]);
          if (i < nqw) q_s[i] = v;
          else if (i < nw) {
            if (r < d) k_s[nold * (d + 1) + r] = v;
            else v_s[nold * d + r - d] = v;
          }
        }
        __syncthreads();
        const float scale = 1.0f / sqrtf((float)d);
        for (int i = tid; i < gq * n; i += NT) {
          const int h = i / n, t = i - h * n;
          const float *qh = q_s + h * d, *kt = k_s + t * (d + 1);
          float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
          for (int j = 0; j < d; j += 4) {
            s0 = fmaf(qh[j], kt[j], s0);
            s1 = fmaf(qh[j + 1], kt[j + 1], s1);
            s2 = fmaf(qh[j + 2], kt[j + 2], s2);
            s3 = fmaf(qh[j + 3], kt[j + 3], s3);
          }
          p_s[h * AC + t] = ((s0 + s1) + (s2 + s3)) * scale;
        }
        __syncthreads();
        for (int h = wave; h < gq; h += NW) {
          const float sc = lane < n ? p_s[h * AC + lane] : -INFINITY;
          const float mx = wave_max(sc);
          const float e = lane < n ? expf(sc - mx) : 0.f;
          const float lsum = wave_sum(e);
          if (lane < n) p_s[h * AC + lane] = e;
          if (lane == 0) {
            ml[2 * h] = mx;
            ml[2 * h + 1] = lsum;
          }
        }
        __syncthreads();
        for (int i = tid; i < gq * d; i += NT) {
          const int h = i / d, j = i - h * d;
          float o = 0.f;
          for (int t = 0; t < n; t++) o = fmaf(p_s[h * AC + t], v_s[t * d + j], o);
          uint64_t *dst = a.tpart + ((size_t)(g * gq + h) * nchmax + c) * (d + 2);
          tput(dst + j, o, T + P_PART);
          if (j == 0) {
            tput(dst + d, ml[2 * h], T + P_PART);
            tput(dst + d + 1, ml[2 * h + 1], T + P_PART);
          }
        }
        __syncthreads();
      }

      // ---- merge: q head h's chunks -> att[h] (tag T + P_ATT), on the last
      // workgroups (attention items start at the first) --------------------
      const int mh = NB - 1 - wg;
      if (mh < a.nq) {
        const int dd = d + 2;
        float *pc = big;                     // [nch][d + 2] gathered partials
        float *wc = big + nch * dd;          // [nch] chunk weights
        const int base = mh * nchmax * dd;
        tgather<2>(a.tpart, [base](int i) { return base + i; }, nch * dd, T + P_PART, pc, a, &fail_s);
        if (tid == 0) {
          // w_c = e^(m_c - M) / sum_c e^(m_c - M) l_c
          float mx = -INFINITY;
          for (int c = 0; c < nch; c++) mx = fmaxf(mx, pc[c * dd + d]);
          float lsum = 0.f;
          for (int c = 0; c < nch; c++) {
            const float e = expf(pc[c * dd + d] - mx);
            wc[c] = e;
            lsum = fmaf(e, pc[c * dd + d + 1], lsum);
          }
          const float inv = 1.0f / lsum;
          for (int c = 0; c < nch; c++) wc[c] *= inv;
        }
        __syncthreads();
        for (int j = tid; j < d; j += NT) {
          float acc = 0.f;
          for (int c = 0; c < nch; c++) acc = fmaf(wc[c], pc[c * dd + j], acc);
          tput(a.tatt + mh * d + j, acc, T + P_ATT);
        }
        __syncthreads();
      }
      mark(a, s, 2 + 5 * l);

      // ---- o projection + residual (tag T + P_XO) -----------------------------
      tgather_lin<3>(a.tatt, qdim, T + P_ATT, att, a, &fail_s);
      mark(a, s, 3 + 5 * l);
      if (has_x) {
        const float y = dotrow<HC>(wo, att, qdim, lane);
        if (lane == 0) {
          xl[wave] += y;
          tput(a.txo + xrow, xl[wave], T + P_XO);
        }
      }

      // ---- gate/up + SwiGLU (tag T + P_H) -------------------------------------
      // pairs 0 and 1 load while X_o is awaited; pair p + 2 loads while p computes
      ldrow<HC>(gA0, L.wgu, H, gu_row(0), gu_row(0) < g1, lane);
      ldrow<HC>(gA1, L.wgu, H, gu_row(0) + 1, gu_row(0) < g1, lane);
      ldrow<HC>(gB0, L.wgu, H, gu_row(1), gu_row(1) < g1, lane);
      ldrow<HC>(gB1, L.wgu, H, gu_row(1) + 1, gu_row(1) < g1, lane);
      tgather_lin<3>(a.txo, H, T + P_XO, xs, a, &fail_s);
      mark(a, s, 4 + 5 * l);
      rmsnorm_lds(xs, L.ln2, H, a.eps, red);
#pragma unroll
      for (int p = 0; p < GPMAX; p++) {
        const int row = gu_row(p), nrow = gu_row(p + 2);
        const bool nv2 = p + 2 < GPMAX && nrow < g1;
        float y0 = 0.f, y1 = 0.f;
        if (p % 2 == 0) {
          if (row < g1) {
            y0 = dotrow<HC>(gA0, xs, H, lane);
            y1 = dotrow<HC>(gA1, xs, H, lane);
          }
          ldrow<HC>(gA0, L.wgu, H, nrow, nv2, lane);
          ldrow<HC>(gA1, L.wgu, H, nrow + 1, nv2, lane);
        } else {
          if (row < g1) {
            y0 = dotrow<HC>(gB0, xs, H, lane);
            y1 = dotrow<HC>(gB1, xs, H, lane);
          }
          ldrow<HC>(gB0, L.wgu, H, nrow, nv2, lane);
          ldrow<HC>(gB1, L.wgu, H, nrow + 1, nv2, lane);
        }
        if (row < g1 && lane == 0) tput(a.th + (row >> 1), silu(y0) * y1, T + P_H);
      }
      // next weights: down of this layer, QKV and o of the next layer
      uint8_t *wd_s = wdl + (size_t)wave * I * 2;
      dma_row(L.wd, I, xrow, has_x, wd_s, lane);
      if (l + 1 < a.L) issue_qo(l + 1);

      // ---- down + residual (tag T + P_XD) -------------------------------------
      tgather_lin<18>(a.th, I, T + P_H, big, a, &fail_s);
      mark(a, s, 5 + 5 * l);
      if (has_x) {
        const float y = dotrow_lds(wd_s, big, I, lane);
        if (lane == 0) {
          xl[wave] += y;
          tput(a.txd + xrow, xl[wave], T + P_XD);
        }
      }
    }

    // ---- final norm + head + argmax partial (tag tstep + 5L) -----------------
    const uint32_t TH = tstep + (uint32_t)a.L * kTPL;
    tgather_lin<3>(a.txd, H, TH - kTPL + P_XD, xs, a, &fail_s);
    mark(a, s, 1 + 5 * a.L);
    rmsnorm_lds(xs, a.final_norm, H, a.eps, red);
    if (wg == 0)
      for (int j = tid; j < H; j += NT) a.normed[j] = xs[j];
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    {
      // this wave's rows v0 + wave*HT + k*NW*HT, two tiles in flight
      u32x4 ta[HT][HC], tb[HT][HC];
      const int stride = NW * HT;
      int r0 = v0 + wave * HT;
#pragma unroll
      for (int r = 0; r < HT; r++) ldrow<HC>(ta[r], a.head, H, r0 + r, r0 + r < v1, lane);
      for (; r0 < v1; r0 += 2 * stride) {
        const int r1 = r0 + stride;
#pragma unroll
        for (int r = 0; r < HT; r++) ldrow<HC>(tb[r], a.head, H, r1 + r, r1 + r < v1, lane);
#pragma unroll
        for (int r = 0; r < HT; r++)
          if (r0 + r < v1) {
            const float y = dotrow<HC>(ta[r], xs, H, lane);
            if (lane == 0) a.logits[r0 + r] = y;
            if (beats(y, (uint32_t)(r0 + r), bv, bi)) {
              bv = y;
              bi = (uint32_t)(r0 + r);
            }
          }
        const int r2 = r1 + stride;
#pragma unroll
        for (int r = 0; r < HT; r++) ldrow<HC>(ta[r], a.head, H, r2 + r, r2 + r < v1, lane);
#pragma unroll
        for (int r = 0; r < HT; r++)
          if (r1 + r < v1) {
            const float y = dotrow<HC>(tb[r], xs, H, lane);
            if (lane == 0) a.logits[r1 + r] = y;
            if (beats(y, (uint32_t)(r1 + r), bv, bi)) {
              bv = y;
              bi = (uint32_t)(r1 + r);
            }
          }
      }
    }
    if (s + 1 < a.steps) issue_qo(0);
    if (lane == 0) best_s[wave] = make_float2(bv, __uint_as_float(bi));
    __syncthreads();
    if (tid == 0) {
      float2 b = best_s[0];
      for (int w = 1; w < NW; w++)
        if (beats(best_s[w].x, __float_as_uint(best_s[w].y), b.x, __float_as_uint(b.y)))
          b = best_s[w];
      tput(a.targ + 2 * wg, b.x, TH);
      tput(a.targ + 2 * wg + 1, b.y, TH);
      mark(a, s, 2 + 5 * a.L);
    }
    __syncthreads();
  }

  // ---- hand the state back to the per-kernel path ---------------------------
  if (tid < NW && x0 + tid < x1) a.x_out[x0 + tid] = xl[tid];
  if (wg == 0) {
    const uint32_t TH = a.tag_base + (a.steps - 1) * TPS + (uint32_t)a.L * kTPL;
    float *pp = big;
    tgather_lin<1>(a.targ, 2 * NB, TH, pp, a, &fail_s);
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    if (tid < NB) {
      bv = pp[2 * tid];
      bi = __float_as_uint(pp[2 * tid + 1]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const uint32_t oi = __shfl_xor(bi, o, 64);
      if (beats(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) best_s[wave] = make_float2(bv, __uint_as_float(bi));
    __syncthreads();
    if (tid == 0) {
      float2 b = best_s[0];
      for (int w = 1; w < NW; w++)
        if (beats(best_s[w].x, __float_as_uint(best_s[w].y), b.x, __float_as_uint(b.y)))
          b = best_s[w];
      best_s[0] = b;
      a.state[0] = a.pos0 + a.steps;
      a.state[1] = a.out_ids[a.steps - 1];
      a.state[2] = a.steps;
    }
    __syncthreads();
    const float2 none = make_float2(-INFINITY, __uint_as_float(0xffffffffu));
    for (int i = tid; i < a.part_cap; i += NT) a.part_out[i] = i == 0 ? best_s[0] : none;
  }
}

}  // namespace

int persist_grid() { return NB; }
int persist_tags_per_step(int layers) { return layers * (int)kTPL + 2; }
size_t persist_part_words(int nq, int max_seq, int d) {
  return (size_t)nq * ((max_seq + AC - 1) / AC) * (size_t)(d + 2);
}

bool persist_supported(int H, int I, int qdim, int d, int gq) {
  if (H % 8 || I % 8 || qdim % 8) return false;
  if (H > MAXH || qdim > MAXH || I > MAXI) return false;
  if (d % 8 || d > MAXD || gq > 8) return false;
  // each workgroup's gate/up pairs fit GPMAX per wavefront, residual rows and
  // QKV pairs one per wavefront
  const int gper = (((2 * I + NB - 1) / NB) + 1) & ~1;
  if (gper / 2 > GPMAX * NW) return false;
  if ((H + NB - 1) / NB > NW) return false;
  const int qkv_rows = qdim + 2 * (qdim / gq);
  if ((((qkv_rows + NB - 1) / NB) + 1) / 2 > NW) return false;
  return true;
}

// LDS bytes one workgroup needs: activations, the largest phase scratch, and
// this workgroup's down rows; sets the down-row offset in `a`
static size_t persist_lds(PersistArgs &a) {
  const int gq = a.nq / a.nkv;
  const size_t attn = (size_t)gq * a.d + AC * (a.d + 1) + AC * a.d + gq * AC + 2 * gq + 2 * a.d;
  const size_t nchm = (size_t)(a.max_seq + AC - 1) / AC;
  const size_t merge = nchm * (a.d + 2) + nchm;
  size_t big = (size_t)a.I;
  if (attn > big) big = attn;
  if (merge > big) big = merge;
  if ((size_t)2 * NB > big) big = 2 * NB;
  const size_t wd_off = 2 * MAXH + ((big + 3) & ~(size_t)3);  // floats
  const size_t xper = (size_t)(a.H + NB - 1) / NB;
  a.lds_wd = (int)wd_off;
  return wd_off * sizeof(float) + xper * (size_t)a.I * 2;
}

bool persist_device_ok(const PersistArgs &a) {
  if (!persist_supported(a.H, a.I, a.nq * a.d, a.d, a.nq / a.nkv)) return false;
  PersistArgs t = a;
  if (persist_lds(t) > kMaxLds) return false;
  int dev = 0, coop = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess) return false;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
  return coop != 0 && cus >= NB;
}

hipError_t launch_decode_persistent(const PersistArgs &a, hipStream_t s) {
  if (!persist_supported(a.H, a.I, a.nq * a.d, a.d, a.nq / a.nkv)) return hipErrorInvalidValue;
  if (a.steps == 0) return hipSuccess;
  if (a.pos0 + a.steps > (uint32_t)a.max_seq) return hipErrorInvalidValue;
  PersistArgs args = a;
  const size_t smem = persist_lds(args);
  if (smem > kMaxLds) return hipErrorInvalidValue;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)decode_persistent_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  void *params[] = {&args};
  return hipLaunchCooperativeKernel((const void *)decode_persistent_kernel, dim3(NB), dim3(NT),
                                    params, (unsigned)smem, s);
}

}  // namespace myos
