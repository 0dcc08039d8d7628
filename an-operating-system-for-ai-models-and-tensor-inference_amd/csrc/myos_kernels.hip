// HIP kernels for the batch-1 BF16-weight / FP32-accumulate token loop on
// MI355X (gfx950, CDNA4): 64-wide wavefronts, 256 CUs in 8 XCDs, HBM3E.
//
// Decode is a weight stream: every projection reads its BF16 matrix from HBM
// exactly once per token, so each GEMV kernel is written to keep many 16-byte
// loads in flight per lane and to fuse the surrounding elementwise work
// (RMSNorm prologue; bias + RoPE + KV-store, SwiGLU, residual and argmax
// epilogues) so no activation round-trips through HBM between launches.
// Prefill's projections run on MFMA (v_mfma_f32_32x32x16_bf16).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "myos_internal.h"

namespace myos {
namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
__device__ __forceinline__ float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// round to nearest even; NaN stays a quiet NaN
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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
// sum / max over aligned groups of W lanes (W = 2, 4, 8, 16 or the whole
// 64-lane wavefront); every lane of a group gets the result
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(W == 2 || W == 4 || W == 8 || W == 16 || W == 64, "group width");
  if (W >= 2) v += dpp<0xB1>(v, 0.f);
  if (W >= 4) v += dpp<0x4E>(v, 0.f);
  if (W >= 8) v += dpp<0x141>(v, 0.f);
  if (W >= 16) v += dpp<0x140>(v, 0.f);
  if (W == 64) {
    v += dpp<0x142, 0xA>(v, 0.f);  // row 0 into row 1, row 2 into row 3
    v += dpp<0x143, 0xC>(v, 0.f);  // rows 0 + 1 into rows 2, 3: lane 63 holds the total
    v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  }
  return v;
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
  static_assert(W == 2 || W == 4 || W == 8 || W == 16 || W == 64, "group width");
  if (W >= 2) v = fmaxf(v, dpp<0xB1>(v, -INFINITY));
  if (W >= 4) v = fmaxf(v, dpp<0x4E>(v, -INFINITY));
  if (W >= 8) v = fmaxf(v, dpp<0x141>(v, -INFINITY));
  if (W >= 16) v = fmaxf(v, dpp<0x140>(v, -INFINITY));
  if (W == 64) {
    v = fmaxf(v, dpp<0x142, 0xA>(v, -INFINITY));
    v = fmaxf(v, dpp<0x143, 0xC>(v, -INFINITY));
    v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  }
  return v;
}

// SiLU as the reference spells it: z / (1 + expf(-z)) (swiglu.rs:113-115)
__device__ __forceinline__ float silu(float z) { return z / (1.0f + expf(-z)); }

// greedy_token ordering (model_core/src/lib.rs:157-167): a candidate wins on a
// strictly larger value, or on an equal value at a lower index; -inf and NaN
// never win, so an all -inf/NaN vector ends with index UINT32_MAX -> 0.
__device__ __forceinline__ bool beats(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && v != -INFINITY && i < bi);
}

__device__ __forceinline__ float load_kv(const void *base, size_t idx, int bf16) {
  return bf16 ? bf16f(((const uint16_t *)base)[idx]) : ((const float *)base)[idx];
}
__device__ __forceinline__ void store_kv(void *base, size_t idx, float v, int bf16) {
  if (bf16)
    ((uint16_t *)base)[idx] = f2bf(v);
  else
    ((float *)base)[idx] = v;
}

// (u / n, u % n) for n > 0: shifts when n is a power of two (every head dim
// in use; n is uniform, so the branch is too), a division otherwise
__device__ __forceinline__ int2 divmod_n(int u, int n) {
  if ((n & (n - 1)) == 0) return make_int2(u >> __builtin_ctz(n), u & (n - 1));
  const int q = u / n;
  return make_int2(q, u - q * n);
}

// Block-wide sum over 256 threads in a fixed order (wave partials, then 0..3).
__device__ float block_sum(float v, float *scratch4) {
  v = group_sum<kWave>(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) scratch4[wave] = v;
  __syncthreads();
  return ((scratch4[0] + scratch4[1]) + scratch4[2]) + scratch4[3];
}

// --------------------------------------------------------------- GEMV -----
//
// One "team" (a wavefront, TEAM = 64, or the whole 256-thread workgroup,
// TEAM = 256) computes ROWS consecutive rows. Thread t of a team owns the
// 8-column chunks t, t + TEAM, ... (CPT of them at most), so its slice of x
// is loaded from LDS into registers once and reused for every row, and the
// ROWS x CPT 16-byte weight loads are all issued before the first FMA.
// x is staged through LDS once per workgroup; with X_NORM the workgroup also
// applies the RMSNorm there (sum of squares over the whole vector, then
// g * (x * inv_rms)), which fuses rmsnorm_bf16_weight into the projection.

// decode attention splits positions into chunks of this many
__host__ __device__ constexpr int attn_chunk(int d) { return d <= 128 ? 32 : 16; }

template <int XM>
__device__ void stage_x(const GemvArgs &a, float *xs, float *red4) {
  const int k = a.k, tid = threadIdx.x;
  float ss = 0.f;
  for (int j = tid * 4; j < k; j += kBlock * 4) {
    float4 v = *(const float4 *)(a.x + j);
    *(float4 *)(xs + j) = v;
    if (XM == X_NORM) ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  if (XM == X_NORM) {
    float tot = block_sum(ss, red4);
    float mean = tot / (float)k;
    float inv = 1.0f / sqrtf(mean + a.eps);
    for (int j = tid * 4; j < k; j += kBlock * 4) {
      float4 v = *(float4 *)(xs + j);
      uint2 g = *(const uint2 *)(a.gamma + j);
      v.x = bf_lo(g.x) * (v.x * inv);
      v.y = bf_hi(g.x) * (v.y * inv);
      v.z = bf_lo(g.y) * (v.z * inv);
      v.w = bf_hi(g.y) * (v.w * inv);
      *(float4 *)(xs + j) = v;
      if (a.normed_out && blockIdx.x == 0) *(float4 *)(a.normed_out + j) = v;
    }
  }
  __syncthreads();
}

// Epilogue for one team's ROWS results (run by the team's thread 0).
template <int EPI, int ROWS>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs &a, int row0, const float *v,
                                              uint32_t pos, float2 *team_best) {
  if (EPI == EPI_STORE) {
#pragma unroll
    for (int r = 0; r < ROWS; r++)
      if (row0 + r < a.m) a.y[row0 + r] = v[r];
  } else if (EPI == EPI_RESID) {
#pragma unroll
    for (int r = 0; r < ROWS; r++)
      if (row0 + r < a.m) a.y[row0 + r] += v[r];
  } else if (EPI == EPI_GU) {
#pragma unroll
    for (int r = 0; r < ROWS; r += 2)
      if (row0 + r < a.m) a.h_out[(row0 + r) >> 1] = silu(v[r]) * v[r + 1];
  } else if (EPI == EPI_HEAD) {
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      int row = row0 + r;
      if (row < a.m) {
        a.y[row] = v[r];
        if (beats(v[r], (uint32_t)row, bv, bi)) {
          bv = v[r];
          bi = (uint32_t)row;
        }
      }
    }
    *team_best = make_float2(bv, __uint_as_float(bi));
  } else if (EPI == EPI_QKV) {
    const int d = a.head_dim, half = d >> 1;
#pragma unroll
    for (int r = 0; r < ROWS; r += 2) {
      const int row = row0 + r;
      if (row >= a.m) break;
      float y0 = v[r] + a.bias[row], y1 = v[r + 1] + a.bias[row + 1];
      if (row < a.q_dim + a.kv_dim) {
        const bool is_q = row < a.q_dim;
        const int rr = is_q ? row : row - a.q_dim;
        const int u = rr >> 1, head = u / half, p = u - head * half;
        const float2 cs = a.rope[(size_t)pos * half + p];
        const float o0 = y0 * cs.x - y1 * cs.y;
        const float o1 = y1 * cs.x + y0 * cs.y;
        if (is_q) {
          a.q_out[head * d + p] = o0;
          a.q_out[head * d + p + half] = o1;
        } else {
          size_t base = ((size_t)head * a.max_seq + pos) * d;
          store_kv(a.kc, base + p, o0, a.kv_bf16);
          store_kv(a.kc, base + p + half, o1, a.kv_bf16);
        }
      } else {
        const int rr = row - a.q_dim - a.kv_dim;
        const int head = rr / d, j = rr - head * d;
        size_t base = ((size_t)head * a.max_seq + pos) * d + j;
        store_kv(a.vc, base, y0, a.kv_bf16);
        store_kv(a.vc, base + 1, y1, a.kv_bf16);
      }
    }
  }
}

template <int TEAM, int ROWS, int CPT, int XM, int EPI>
__global__ void __launch_bounds__(kBlock) gemv_kernel(GemvArgs a) {
  extern __shared__ float4 xs4[];
  float *xs = (float *)xs4;
  __shared__ float red4[4];
  __shared__ float red[4][ROWS];
  __shared__ float2 best[4];
  constexpr int TEAMS = kBlock / TEAM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int team = TEAMS == 1 ? 0 : wave;
  const int tt = TEAMS == 1 ? tid : lane;
  const int k = a.k, m = a.m, nch = k >> 3;
  const int row0 = (blockIdx.x * TEAMS + team) * ROWS;
  uint32_t pos = 0;
  if (EPI == EPI_QKV) pos = *a.pos_ptr;

  // weight loads first: they do not depend on x, so they overlap the staging
  u32x4 wv[ROWS][CPT];
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    const int row = min(row0 + r, m - 1);
    const u32x4 *rowp = (const u32x4 *)(a.w + (size_t)row * k);
#pragma unroll
    for (int i = 0; i < CPT; i++) {
      const int c = tt + i * TEAM;
      const u32x4 zero = {0u, 0u, 0u, 0u};
      wv[r][i] = c < nch ? __builtin_nontemporal_load(rowp + c) : zero;
    }
  }

  stage_x<XM>(a, xs, red4);

  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; i++) {
    const int c = tt + i * TEAM;
    if (c < nch) {
      const float4 x0 = xs4[c * 2], x1 = xs4[c * 2 + 1];
#pragma unroll
      for (int r = 0; r < ROWS; r++) {
        const u32x4 w = wv[r][i];
        float s = acc[r];
        s = fmaf(bf_lo(w.x), x0.x, s);
        s = fmaf(bf_hi(w.x), x0.y, s);
        s = fmaf(bf_lo(w.y), x0.z, s);
        s = fmaf(bf_hi(w.y), x0.w, s);
        s = fmaf(bf_lo(w.z), x1.x, s);
        s = fmaf(bf_hi(w.z), x1.y, s);
        s = fmaf(bf_lo(w.w), x1.z, s);
        s = fmaf(bf_hi(w.w), x1.w, s);
        acc[r] = s;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = group_sum<kWave>(acc[r]);
  if (TEAMS == 1) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < ROWS; r++) red[wave][r] = acc[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < ROWS; r++) acc[r] = ((red[0][r] + red[1][r]) + red[2][r]) + red[3][r];
  }
  if (tt == 0) gemv_epilogue<EPI, ROWS>(a, row0, acc, pos, &best[team]);
  if (EPI == EPI_HEAD) {
    __syncthreads();
    if (tid == 0) {
      float2 b = best[0];
#pragma unroll
      for (int t = 1; t < TEAMS; t++)
        if (beats(best[t].x, __float_as_uint(best[t].y), b.x, __float_as_uint(b.y))) b = best[t];
      a.part[blockIdx.x] = b;
      if (blockIdx.x == 0 && a.pos_inc) *a.pos_inc += 1u;
    }
  }
}

// Streaming GEMV for large matrices: about two workgroups per CU, each
// staging x once (with the fused RMSNorm for X_NORM) and then walking a
// contiguous range of rows, RB rows per team at a time, while the team's
// loads for its next RB rows are in flight. A one-shot launch (gemv_kernel)
// stages x in every workgroup: with 16 or fewer rows per workgroup that
// re-reads as many x bytes as weight bytes once k is large (a 3584 x 18944
// down projection reads its 74 KB h vector 1792 times). The next batch is
// always loaded (past the range: the range's first row again), so the
// compiler's wait for the current batch leaves the next one in flight.
template <int TEAM, int RB, int CPT, int XM, int EPI>
__global__ void __launch_bounds__(kBlock) gemv_stream_kernel(GemvArgs a, int rows_per_wg) {
  extern __shared__ float4 xs4[];
  float *xs = (float *)xs4;
  __shared__ float red4[4];
  __shared__ float red[2][4][RB];
  __shared__ float2 best[4];
  constexpr int TEAMS = kBlock / TEAM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int team = TEAMS == 1 ? 0 : wave;
  const int tt = TEAMS == 1 ? tid : lane;
  const int k = a.k, m = a.m, nch = k >> 3;
  const int r0 = blockIdx.x * rows_per_wg, r1 = min(m, r0 + rows_per_wg);
  const int nb = (r1 - r0 + RB - 1) / RB;  // batches of this workgroup
  uint32_t pos = 0;
  if (EPI == EPI_QKV) pos = *a.pos_ptr;

  auto load = [&](u32x4 (&w)[RB][CPT], int b) {
    const int rb = b < nb ? r0 + b * RB : r0;
#pragma unroll
    for (int r = 0; r < RB; r++) {
      const u32x4 *rowp = (const u32x4 *)(a.w + (size_t)min(rb + r, m - 1) * k);
#pragma unroll
      for (int i = 0; i < CPT; i++) {
        const int c = tt + i * TEAM;
        const u32x4 zero = {0u, 0u, 0u, 0u};
        w[r][i] = c < nch ? __builtin_nontemporal_load(rowp + c) : zero;
      }
    }
  };
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  int parity = 0;
  auto mult = [&](const u32x4 (&w)[RB][CPT], int b) {
    float acc[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) acc[r] = 0.f;
#pragma unroll
    for (int i = 0; i < CPT; i++) {
      const int c = tt + i * TEAM;
      if (c < nch) {
        const float4 x0 = xs4[c * 2], x1 = xs4[c * 2 + 1];
#pragma unroll
        for (int r = 0; r < RB; r++) {
          const u32x4 v = w[r][i];
          float s = acc[r];
          s = fmaf(bf_lo(v.x), x0.x, s);
          s = fmaf(bf_hi(v.x), x0.y, s);
          s = fmaf(bf_lo(v.y), x0.z, s);
          s = fmaf(bf_hi(v.y), x0.w, s);
          s = fmaf(bf_lo(v.z), x1.x, s);
          s = fmaf(bf_hi(v.z), x1.y, s);
          s = fmaf(bf_lo(v.w), x1.z, s);
          s = fmaf(bf_hi(v.w), x1.w, s);
          acc[r] = s;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RB; r++) acc[r] = group_sum<kWave>(acc[r]);
    if (TEAMS == 1) {
      // the four waves' sums through LDS; two buffers, so one barrier per batch
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RB; r++) red[parity][wave][r] = acc[r];
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < RB; r++)
        acc[r] = ((red[parity][0][r] + red[parity][1][r]) + red[parity][2][r]) + red[parity][3][r];
      parity ^= 1;
    }
    if (tt == 0 && b < nb) {
      const int row0 = r0 + b * RB;
      float2 tb;
      gemv_epilogue<EPI, RB>(a, row0, acc, pos, &tb);
      if (EPI == EPI_HEAD && beats(tb.x, __float_as_uint(tb.y), bv, bi)) {
        bv = tb.x;
        bi = __float_as_uint(tb.y);
      }
    }
  };

  // weight loads first: they do not depend on x, so they overlap the staging
  u32x4 wa[RB][CPT], wb[RB][CPT];
  load(wa, team);
  stage_x<XM>(a, xs, red4);
  // every team runs the same number of batch pairs (the TEAM = 256 barrier)
  const int steps = (nb + TEAMS - 1) / TEAMS;
  for (int s = 0; s < steps; s += 2) {
    const int b = team + s * TEAMS;
    load(wb, b + TEAMS);
    mult(wa, b);
    if (s + 1 < steps) {
      load(wa, b + 2 * TEAMS);
      mult(wb, b + TEAMS);
    }
  }
  if (EPI == EPI_HEAD) {
    if (tt == 0) best[team] = make_float2(bv, __uint_as_float(bi));
    __syncthreads();
    if (tid == 0) {
      float2 bb = best[0];
#pragma unroll
      for (int t = 1; t < TEAMS; t++)
        if (beats(best[t].x, __float_as_uint(best[t].y), bb.x, __float_as_uint(bb.y))) bb = best[t];
      a.part[blockIdx.x] = bb;
      if (blockIdx.x == 0 && a.pos_inc) *a.pos_inc += 1u;
    }
  }
}

// Any k (including k % 8 != 0): one wavefront per row pair, element loads.
template <int XM, int EPI>
__global__ void __launch_bounds__(kBlock) gemv_generic_kernel(GemvArgs a) {
  extern __shared__ float4 xs4[];
  float *xs = (float *)xs4;
  __shared__ float red4[4];
  __shared__ float2 best[4];
  constexpr int ROWS = 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int k = a.k, m = a.m;
  const int row0 = (blockIdx.x * 4 + wave) * ROWS;
  uint32_t pos = 0;
  if (EPI == EPI_QKV) pos = *a.pos_ptr;
  // scalar staging (k may not be a multiple of 4)
  float ss = 0.f;
  for (int j = tid; j < k; j += kBlock) {
    float v = a.x[j];
    xs[j] = v;
    ss += v * v;
  }
  if (XM == X_NORM) {
    float tot = block_sum(ss, red4);
    float inv = 1.0f / sqrtf(tot / (float)k + a.eps);
    for (int j = tid; j < k; j += kBlock) {
      float v = bf16f(a.gamma[j]) * (xs[j] * inv);
      xs[j] = v;
      if (a.normed_out && blockIdx.x == 0) a.normed_out[j] = v;
    }
  }
  __syncthreads();
  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    const int row = min(row0 + r, m - 1);
    const uint16_t *rowp = a.w + (size_t)row * k;
    float s = 0.f;
    for (int j = lane; j < k; j += kWave) s = fmaf(bf16f(rowp[j]), xs[j], s);
    acc[r] = group_sum<kWave>(s);
  }
  if (lane == 0) gemv_epilogue<EPI, ROWS>(a, row0, acc, pos, &best[wave]);
  if (EPI == EPI_HEAD) {
    __syncthreads();
    if (tid == 0) {
      float2 b = best[0];
      for (int t = 1; t < 4; t++)
        if (beats(best[t].x, __float_as_uint(best[t].y), b.x, __float_as_uint(b.y))) b = best[t];
      a.part[blockIdx.x] = b;
      if (blockIdx.x == 0 && a.pos_inc) *a.pos_inc += 1u;
    }
  }
}

// ------------------------------------------------------ decode attention ---
//
// Workgroup (kv head g, chunk c of attn_chunk(d) positions) scores the chunk
// for the q_per_kv query heads that share g (K/V read once per group), keeps a
// chunk-local softmax (max m, sum l, unnormalised mix o), and the last
// workgroup of the group to finish (atomic counter) merges the chunks:
// y = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c. The serial reference
// (gqa.rs:174-218) is the same quantity with one chunk. K, V (chunk x d each)
// and q stay under the 64 KiB workgroup LDS limit: 32 positions up to d = 128,
// 16 up to d = 256.
constexpr int kMaxQPerKv = 8;
constexpr int kMaxHeadDim = 256;

// The last of a group's nv chunk workgroups to finish merges the group's
// heads. Each thread first waits until its partial stores have completed
// (vmcnt counts stores on gfx9; the asm is also a compiler barrier), then one
// thread counts the workgroup in with a relaxed device-scope add. The merging
// workgroup reads the partials with device-coherent loads. No device-scope
// fence: on this part that writes back and invalidates the whole L2.
__device__ bool attn_last_in_group(const AttnDecodeArgs &a, int g, int nv) {
  __shared__ int last_s;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    last_s = __hip_atomic_fetch_add(&a.cnt[g], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nv - 1;
  __syncthreads();
  return last_s != 0;
}

// Device-coherent (sc1, the cache policy of a relaxed agent-scope atomic
// load) 32-bit load of element i through a buffer descriptor. To the
// compiler it is an ordinary load, so a run of them goes out back to back:
// every atomic load orders the memory operations around it, which put a full
// wait after each one (a merge of 30 partials took 30 round trips).
__device__ __forceinline__ float attn_cload(__amdgpu_buffer_rsrc_t rs, size_t i) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (int)(i * 4), 0, 16));
}

// Merge of group g's nv chunk partials ([nq][nchunks][d + 2]: o, m, l):
// att[h] = sum_c w_c o_c with w_c = e^(m_c - M) / sum_c' e^(m_c' - M) l_c'
// (gqa.rs:283-307 is the one-chunk case), chunks added in order, so the
// result does not depend on which workgroup merges. The counter is reset for
// the next launch. With at most kFastMerge chunks every load is issued in one
// round trip (this thread's o values into registers, every (m, l) into LDS);
// longer runs load the weights first and the o values in batches of 8.
constexpr int kFastMerge = 16;
__device__ void attn_merge(const AttnDecodeArgs &a, int g, int gq, int d, int nv, int nchunks,
                           float *smem) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t stride = (size_t)d + 2;
  const float *part = a.part + (size_t)g * gq * nchunks * stride;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)part, (short)0, (int)((size_t)gq * nchunks * stride * 4), 0x00020000);
  const int nout = gq * d;
  float *wm = smem, *lm = smem + gq * nv;  // [gq][nv] (m, l) -> weights
  auto load_ml = [&]() {
    for (int i = tid; i < gq * nv; i += kBlock) {
      const int h = i / nv, cc = i - h * nv;
      const size_t src = ((size_t)h * nchunks + cc) * stride + d;
      wm[i] = attn_cload(rs, src);
      lm[i] = attn_cload(rs, src + 1);
    }
  };
  if (nv <= kFastMerge && nout <= 4 * kBlock) {
    float ov[4][kFastMerge];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int i = tid + r * kBlock, h = i / d, j = i - h * d;
#pragma unroll
      for (int cc = 0; cc < kFastMerge; cc++)
        ov[r][cc] = i < nout && cc < nv ? attn_cload(rs, ((size_t)h * nchunks + cc) * stride + j) : 0.f;
    }
    load_ml();
    __syncthreads();
    // one wave per head: lane cc holds chunk cc
    for (int h = wave; h < gq; h += kBlock / kWave) {
      const float m = lane < nv ? wm[h * nv + lane] : -INFINITY;
      const float mx = group_max<kWave>(m);
      const float e = lane < nv ? expf(m - mx) : 0.f;
      const float l = group_sum<kWave>(lane < nv ? e * lm[h * nv + lane] : 0.f);
      if (lane < nv) wm[h * nv + lane] = e * (1.0f / l);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int i = tid + r * kBlock, h = i / d, j = i - h * d;
      if (i < nout) {
        float acc = 0.f;
#pragma unroll
        for (int cc = 0; cc < kFastMerge; cc++)
          if (cc < nv) acc = fmaf(wm[h * nv + cc], ov[r][cc], acc);
        a.att[(size_t)(g * gq + h) * d + j] = acc;
      }
    }
  } else {
    load_ml();
    __syncthreads();
    for (int h = tid; h < gq; h += kBlock) {
      float *w = wm + h * nv;
      const float *lh = lm + h * nv;
      float mx = -INFINITY;
      for (int cc = 0; cc < nv; cc++) mx = fmaxf(mx, w[cc]);
      float l = 0.f;
      for (int cc = 0; cc < nv; cc++) {
        const float e = expf(w[cc] - mx);
        w[cc] = e;
        l = fmaf(e, lh[cc], l);
      }
      const float inv = 1.0f / l;
      for (int cc = 0; cc < nv; cc++) w[cc] *= inv;
    }
    __syncthreads();
    for (int i = tid; i < nout; i += kBlock) {
      const int h = i / d, j = i - h * d;
      const float *w = wm + h * nv;
      const size_t base = (size_t)h * nchunks * stride + j;
      float acc = 0.f;
      int cc = 0;
      for (; cc + 8 <= nv; cc += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = attn_cload(rs, base + (size_t)(cc + u) * stride);
#pragma unroll
        for (int u = 0; u < 8; u++) acc = fmaf(w[cc + u], v[u], acc);
      }
      for (; cc < nv; cc++) acc = fmaf(w[cc], attn_cload(rs, base + (size_t)cc * stride), acc);
      a.att[(size_t)(g * gq + h) * d + j] = acc;
    }
  }
  if (tid == 0) a.cnt[g] = 0;
}

// Decode attention at head_dim 128 with the chunk in registers: workgroup
// (kv head g, chunk c of 32 positions); thread (wave w, lane l) holds
// positions t = 8 w + 4 (l >> 5) + u, u < 4, columns [4 (l & 31), +4) of K
// and V, and the same columns of the group's gq query heads. A score is a
// 32-lane sum (DPP); wave w then takes the softmax of heads w, w + 4; the V
// sum runs on the same registers, its 8 partial sums per column (two lane
// halves x four waves) added through LDS in a fixed order. Same partial
// layout and merge as attn_decode_kernel.
template <bool KB>
__global__ void __launch_bounds__(kBlock) attn_decode_d128_kernel(AttnDecodeArgs a) {
  constexpr int D = 128, CH = 32;
  extern __shared__ float smem[];
  float4 *o_s = (float4 *)smem;                // [4 waves][2 halves][gq][32]: V-sum partials
  float *p_s = smem + 4 * 2 * kMaxQPerKv * D;  // [gq][CH] scores -> weights
  float *ml_s = p_s + kMaxQPerKv * CH;         // [gq][2]
  const int gq = a.nq / a.nkv, g = blockIdx.x, c = blockIdx.y, nchunks = gridDim.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5, j4 = lane & 31;
  const int seq = (int)*a.pos_ptr + 1, t0 = c * CH, n = min(CH, seq - t0);
  if (n <= 0) return;  // past the cursor: the merge takes chunks < seq only
  const size_t row0 = (size_t)g * a.max_seq + t0;
  // positions past the chunk's end are read at its last row (in range) and
  // zeroed: unconditional loads go out together, where loads under a lane
  // branch were each waited for where the branch joined
  float4 kr[4], vr[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int t = 8 * wave + 4 * half + u;
    const size_t e = (row0 + min(t, n - 1)) * D + 4 * j4;
    float4 kx, vx;
    if (KB) {
      const uint2 k2 = *(const uint2 *)((const uint16_t *)a.kc + e);
      const uint2 v2 = *(const uint2 *)((const uint16_t *)a.vc + e);
      kx = make_float4(bf_lo(k2.x), bf_hi(k2.x), bf_lo(k2.y), bf_hi(k2.y));
      vx = make_float4(bf_lo(v2.x), bf_hi(v2.x), bf_lo(v2.y), bf_hi(v2.y));
    } else {
      kx = *(const float4 *)((const float *)a.kc + e);
      vx = *(const float4 *)((const float *)a.vc + e);
    }
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    kr[u] = t < n ? kx : zero;
    vr[u] = t < n ? vx : zero;
  }
  float4 q4[kMaxQPerKv];
#pragma unroll
  for (int h = 0; h < kMaxQPerKv; h++)
    if (h < gq) q4[h] = *(const float4 *)(a.q + (size_t)(g * gq + h) * D + 4 * j4);
  const float scale = 1.0f / sqrtf((float)D);
#pragma unroll
  for (int h = 0; h < kMaxQPerKv; h++) {
    if (h >= gq) break;
#pragma unroll
    for (int u = 0; u < 4; u++) {
      float s = q4[h].x * kr[u].x;
      s = fmaf(q4[h].y, kr[u].y, s);
      s = fmaf(q4[h].z, kr[u].z, s);
      s = fmaf(q4[h].w, kr[u].w, s);
      s = group_sum<16>(s);
      s += dpp<0x142, 0xA>(s, 0.f);  // rows 1, 3 add rows 0, 2: lanes 16-31, 48-63 hold the 32-lane sums
      const int t = 8 * wave + 4 * half + u;
      if ((lane & 31) == 16 && t < n) p_s[h * CH + t] = s * scale;
    }
  }
  __syncthreads();
  for (int h = wave; h < gq; h += kBlock / kWave) {
    const float s = lane < n ? p_s[h * CH + lane] : -INFINITY;
    const float mx = group_max<kWave>(s);
    const float e = lane < n ? expf(s - mx) : 0.f;
    const float l = group_sum<kWave>(e);
    if (lane < CH) p_s[h * CH + lane] = e;
    if (lane == 0) {
      ml_s[2 * h] = mx;
      ml_s[2 * h + 1] = l;
    }
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < kMaxQPerKv; h++) {
    if (h >= gq) break;
    const float4 e4 = *(const float4 *)(p_s + h * CH + 8 * wave + 4 * half);
    const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < 4; u++) {
      acc.x = fmaf(ev[u], vr[u].x, acc.x);
      acc.y = fmaf(ev[u], vr[u].y, acc.y);
      acc.z = fmaf(ev[u], vr[u].z, acc.z);
      acc.w = fmaf(ev[u], vr[u].w, acc.w);
    }
    o_s[((wave * 2 + half) * kMaxQPerKv + h) * 32 + j4] = acc;
  }
  __syncthreads();
  const size_t stride = (size_t)D + 2;
  for (int i = tid; i < gq * 32; i += kBlock) {
    const int h = i >> 5, jj = i & 31;
    float4 o = o_s[h * 32 + jj];
#pragma unroll
    for (int p = 1; p < 8; p++) {
      const float4 v = o_s[(p * kMaxQPerKv + h) * 32 + jj];
      o.x += v.x;
      o.y += v.y;
      o.z += v.z;
      o.w += v.w;
    }
    // device-coherent stores (they reach the coherence point, not this XCD's
    // L2), so the merging workgroup on any XCD reads them with no cache flush
    float *dst = a.part + ((size_t)(g * gq + h) * nchunks + c) * stride;
    __hip_atomic_store(dst + 4 * jj, o.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(dst + 4 * jj + 1, o.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(dst + 4 * jj + 2, o.z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(dst + 4 * jj + 3, o.w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (jj == 0) {
      __hip_atomic_store(dst + D, ml_s[2 * h], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(dst + D + 1, ml_s[2 * h + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  const int nv = (seq + CH - 1) / CH;
  if (attn_last_in_group(a, g, nv)) attn_merge(a, g, gq, D, nv, nchunks, smem);
}

__global__ void __launch_bounds__(kBlock) attn_decode_kernel(AttnDecodeArgs a) {
  extern __shared__ float smem[];
  const int d = a.head_dim, gq = a.nq / a.nkv, dp = d + 1, ch = attn_chunk(d);
  float *q_s = smem;                        // [gq][d]
  float *k_s = q_s + gq * d;                // [chunk][d + 1]
  float *v_s = k_s + ch * dp;               // [chunk][d]
  float *p_s = v_s + ch * d;                // [gq][chunk]
  float *ml_s = p_s + gq * ch;              // [gq][2]
  const int g = blockIdx.x, c = blockIdx.y, nchunks = gridDim.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int seq = (int)*a.pos_ptr + 1;
  const int t0 = c * ch;
  const int n = min(ch, seq - t0);
  if (n <= 0) return;  // past the cursor: the merge takes chunks < seq only
  const float scale = 1.0f / sqrtf((float)d);
  for (int i = tid; i < gq * d; i += kBlock) q_s[i] = a.q[(size_t)g * gq * d + i];
  const size_t kv0 = ((size_t)g * a.max_seq + t0) * d;
  if (!a.kv_bf16 && (d & 3) == 0) {
    const float4 *k4 = (const float4 *)((const float *)a.kc + kv0);
    const float4 *v4 = (const float4 *)((const float *)a.vc + kv0);
    for (int i = tid; i < (n * d) >> 2; i += kBlock) {
      const float4 kv = k4[i], vv = v4[i];
      const int e = i << 2, t = e / d, j = e - t * d;
      float *kd = k_s + t * dp + j;
      kd[0] = kv.x;
      kd[1] = kv.y;
      kd[2] = kv.z;
      kd[3] = kv.w;
      *(float4 *)(v_s + e) = vv;
    }
  } else {
    for (int i = tid; i < n * d; i += kBlock) {
      const int t = i / d, j = i - t * d;
      k_s[t * dp + j] = load_kv(a.kc, kv0 + i, a.kv_bf16);
      v_s[i] = load_kv(a.vc, kv0 + i, a.kv_bf16);
    }
  }
  __syncthreads();
  for (int i = tid; i < gq * n; i += kBlock) {
    const int h = i / n, t = i - h * n;
    const float *qh = q_s + h * d, *kt = k_s + t * dp;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int j = 0;
#pragma unroll 4
    for (; j + 3 < d; j += 4) {
      s0 = fmaf(qh[j], kt[j], s0);
      s1 = fmaf(qh[j + 1], kt[j + 1], s1);
      s2 = fmaf(qh[j + 2], kt[j + 2], s2);
      s3 = fmaf(qh[j + 3], kt[j + 3], s3);
    }
    for (; j < d; j++) s0 = fmaf(qh[j], kt[j], s0);
    p_s[h * ch + t] = ((s0 + s1) + (s2 + s3)) * scale;
  }
  __syncthreads();
  for (int h = wave; h < gq; h += 4) {
    float s = lane < n ? p_s[h * ch + lane] : -INFINITY;
    const float mx = group_max<kWave>(s);
    const float e = lane < n ? expf(s - mx) : 0.f;
    const float l = group_sum<kWave>(e);
    if (lane < n) p_s[h * ch + lane] = e;
    if (lane == 0) {
      ml_s[2 * h] = mx;
      ml_s[2 * h + 1] = l;
    }
  }
  __syncthreads();
  const size_t stride_part = (size_t)d + 2;
  for (int i = tid; i < gq * d; i += kBlock) {
    const int h = i / d, j = i - h * d;
    const float *ph = p_s + h * ch;
    float o = 0.f;
    for (int t = 0; t < n; t++) o = fmaf(ph[t], v_s[t * d + j], o);
    // device-coherent stores (they reach the coherence point, not this XCD's
    // L2), so the merging workgroup on any XCD reads them with no cache flush
    float *dst = a.part + ((size_t)(g * gq + h) * nchunks + c) * stride_part;
    __hip_atomic_store(dst + j, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (j == 0) {
      __hip_atomic_store(dst + d, ml_s[2 * h], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(dst + d + 1, ml_s[2 * h + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  if (attn_last_in_group(a, g, (seq + ch - 1) / ch)) attn_merge(a, g, gq, d, (seq + ch - 1) / ch, nchunks, smem);
}

// ----------------------------------------------------------- small ops ----

__global__ void fill_zero_kernel(float *y, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) y[i] = 0.f;
}

__global__ void add_bias_kernel(float *y, const uint16_t *b, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) y[i] = y[i] + bf16f(b[i]);
}

__global__ void embed_gather_kernel(float *out, const uint16_t *table, size_t hidden,
                                    const uint32_t *token_dev, uint32_t token_host) {
  const uint32_t tok = token_dev ? *token_dev : token_host;
  const uint16_t *row = table + (size_t)tok * hidden;
  for (size_t j = blockIdx.x * (size_t)blockDim.x + threadIdx.x; j < hidden;
       j += (size_t)gridDim.x * blockDim.x)
    out[j] = bf16f(row[j]);
}

__device__ __forceinline__ float gain(const uint16_t *g, size_t j) { return bf16f(g[j]); }
__device__ __forceinline__ float gain(const float *g, size_t j) { return g[j]; }

// rmsnorm_bf16_weight (bf16 gains) and rmsnorm_f32 (f32 gains)
template <class G>
__global__ void __launch_bounds__(kBlock)
    rmsnorm_kernel(float *y, const G *g, const float *x, size_t n, float eps) {
  __shared__ float red4[4];
  float ss = 0.f;
  for (size_t j = threadIdx.x; j < n; j += kBlock) ss += x[j] * x[j];
  const float tot = block_sum(ss, red4);
  const float inv = 1.0f / sqrtf(tot / (float)n + eps);
  for (size_t j = threadIdx.x; j < n; j += kBlock) y[j] = gain(g, j) * (x[j] * inv);
}

// cs[p] = (cos, sin) of pair p, evaluated on the host (rope.rs:186-193)
__global__ void rope_apply_kernel(float *x, size_t len, size_t head_dim, const float2 *cs) {
  const size_t half = head_dim / 2, pairs = len / 2;
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= pairs) return;
  const size_t head = i / half, p = i - head * half;
  const size_t i0 = head * head_dim + p, i1 = i0 + half;
  const float x0 = x[i0], x1 = x[i1];
  const float2 c = cs[p];
  x[i0] = x0 * c.x - x1 * c.y;
  x[i1] = x1 * c.x + x0 * c.y;
}

// Op-tier gqa_attn_f32 for any shape: one workgroup per query head; scores
// in a global scratch row of length seq; the last head's probabilities are
// also written to `probs` (gqa.rs:26-30).
__global__ void __launch_bounds__(kBlock)
    gqa_general_kernel(float *y, const float *q, const float *k, const float *v, float *probs,
                       float *scr, int nq, int nkv, int d, int seq, int mask,
                       unsigned long long qpos) {
  __shared__ float red4[4];
  const int h = blockIdx.x, g = h / (nq / nkv), tid = threadIdx.x;
  const float scale = 1.0f / sqrtf((float)d);
  float *s = scr + (size_t)h * seq;
  const float *qh = q + (size_t)h * d;
  auto kept = [&](int t) { return mask == 0 || (unsigned long long)t <= qpos; };
  float mx = -INFINITY;
  for (int t = tid; t < seq; t += kBlock) {
    if (!kept(t)) continue;
    const float *kt = k + ((size_t)g * seq + t) * d;
    float acc = 0.f;
    for (int j = 0; j < d; j++) acc = fmaf(qh[j], kt[j], acc);
    s[t] = acc * scale;
    mx = fmaxf(mx, s[t]);
  }
  // block max
  mx = group_max<kWave>(mx);
  __syncthreads();
  if ((tid & 63) == 0) red4[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
  float sum = 0.f;
  for (int t = tid; t < seq; t += kBlock) {
    if (!kept(t)) continue;
    const float e = expf(s[t] - mx);
    s[t] = e;
    sum += e;
  }
  sum = block_sum(sum, red4);
  for (int t = tid; t < seq; t += kBlock) {
    const float p = kept(t) ? s[t] / sum : 0.f;
    s[t] = p;
    if (h == nq - 1) probs[t] = p;
  }
  __syncthreads();
  for (int j = tid; j < d; j += kBlock) {
    float acc = 0.f;
    for (int t = 0; t < seq; t++)
      if (kept(t)) acc = fmaf(s[t], v[((size_t)g * seq + t) * d + j], acc);
    y[(size_t)h * d + j] = acc;
  }
}

__global__ void swiglu_mul_kernel(float *h, const float *g, const float *u, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) h[i] = silu(g[i]) * u[i];
}

__global__ void silu_kernel(float *y, const float *z, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) y[i] = silu(z[i]);
}

constexpr int kArgmaxPerBlock = 4096;

__device__ float2 block_best(float bv, uint32_t bi, float2 *sh) {
  // wave reduce then waves 0..3 in order
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, kWave);
    const uint32_t oi = __shfl_xor(bi, o, kWave);
    if (beats(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) sh[wave] = make_float2(bv, __uint_as_float(bi));
  __syncthreads();
  float2 b = sh[0];
  for (int t = 1; t < (int)(blockDim.x >> 6); t++)
    if (beats(sh[t].x, __float_as_uint(sh[t].y), b.x, __float_as_uint(b.y))) b = sh[t];
  return b;
}

__global__ void __launch_bounds__(kBlock)
    argmax_partial_kernel(const float *logits, size_t n, float2 *part) {
  __shared__ float2 sh[4];
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  const size_t base = (size_t)blockIdx.x * kArgmaxPerBlock;
  for (size_t i = base + threadIdx.x; i < min(n, base + kArgmaxPerBlock); i += kBlock)
    if (beats(logits[i], (uint32_t)i, bv, bi)) {
      bv = logits[i];
      bi = (uint32_t)i;
    }
  float2 b = block_best(bv, bi, sh);
  if (threadIdx.x == 0) part[blockIdx.x] = b;
}

__global__ void __launch_bounds__(1024) argmax_final_kernel(ArgmaxFinalArgs a) {
  __shared__ float2 sh[16];
  __shared__ uint32_t tok_s;
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  const uint32_t mode = a.state ? a.state[3] : 0u;
  if (mode != 1u) {
    // 8 partials per thread per round, all loaded before any compare
    for (int i0 = threadIdx.x; i0 < a.nparts; i0 += blockDim.x * 8) {
      float2 p[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int i = i0 + u * (int)blockDim.x;
        p[u] = i < a.nparts ? a.part[i] : make_float2(-INFINITY, __uint_as_float(0xffffffffu));
      }
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (beats(p[u].x, __float_as_uint(p[u].y), bv, bi)) {
          bv = p[u].x;
          bi = __float_as_uint(p[u].y);
        }
    }
    float2 b = block_best(bv, bi, sh);
    if (threadIdx.x == 0) {
      uint32_t idx = __float_as_uint(b.y);
      idx = idx < a.vocab ? idx : 0u;  // no candidate (all NaN / -inf) -> 0
      // teacher forcing: record the argmax, feed the given id
      if (mode == 2u) {
        if (a.out_ids) a.out_ids[a.state[2]] = idx;
        idx = a.force[a.state[2]];
      }
      tok_s = idx;
    }
  } else if (threadIdx.x == 0) {
    tok_s = a.state[1];
  }
  __syncthreads();
  const uint32_t tok = tok_s;
  if (threadIdx.x == 0) {
    if (a.token_out) *a.token_out = tok;
    if (a.state) {
      a.state[1] = tok;
      if (a.out_ids && mode != 2u) a.out_ids[a.state[2]] = tok;
      a.state[2] += 1u;
    }
  }
  if (a.embed)
    for (int j = threadIdx.x; j < a.hidden; j += blockDim.x)
      a.x[j] = bf16f(a.embed[(size_t)tok * a.hidden + j]);
}

// ------------------------------------------------------------- prefill ----

__global__ void embed_rows_kernel(float *X, const uint16_t *embed, const uint32_t *tokens,
                                  int H) {
  const int r = blockIdx.x;
  const uint16_t *src = embed + (size_t)tokens[r] * H;
  for (int j = threadIdx.x; j < H; j += blockDim.x) X[(size_t)r * H + j] = bf16f(src[j]);
}

__device__ __forceinline__ void split2(float x, uint16_t *hi, uint16_t *lo) {
  const uint16_t h = f2bf(x);
  *hi = h;
  *lo = f2bf(x - bf16f(h));
}

// four consecutive normalised values g[e] * (x[e] * inv), as split2 writes
// them, stored as one 8-byte word per plane (hi, lo 8-byte aligned)
__device__ __forceinline__ void split4_store(float4 x, uint2 g, float inv, uint16_t *hi, uint16_t *lo) {
  const float y[4] = {bf16f((uint16_t)(g.x & 0xffffu)) * (x.x * inv), bf16f((uint16_t)(g.x >> 16)) * (x.y * inv),
                      bf16f((uint16_t)(g.y & 0xffffu)) * (x.z * inv), bf16f((uint16_t)(g.y >> 16)) * (x.w * inv)};
  uint32_t h[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const uint16_t hb = f2bf(y[e]);
    h[e] = hb;
    l[e] = f2bf(y[e] - bf16f(hb));
  }
  *(uint2 *)hi = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
  *(uint2 *)lo = make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
}

// rmsnorm_rows_split_kernel for H % 4 == 0 and H <= 4 NV kBlock: the row's
// values and gains are loaded once, up front, as float4 / 8-byte words
template <int NV>
__global__ void __launch_bounds__(kBlock)
    rmsnorm_rows_split4_kernel(const float *X, const uint16_t *g, float eps, int H, uint16_t *hi,
                               uint16_t *lo) {
  __shared__ float red4[4];
  const size_t r = blockIdx.x;
  const int n4 = H >> 2;
  float4 xv[NV];
  uint2 gv[NV];
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int c4 = threadIdx.x + v * kBlock;
    xv[v] = c4 < n4 ? *(const float4 *)(X + r * H + 4 * c4) : make_float4(0.f, 0.f, 0.f, 0.f);
    gv[v] = c4 < n4 ? *(const uint2 *)(g + 4 * c4) : make_uint2(0u, 0u);
    ss += xv[v].x * xv[v].x + xv[v].y * xv[v].y + xv[v].z * xv[v].z + xv[v].w * xv[v].w;
  }
  const float tot = block_sum(ss, red4);
  const float inv = 1.0f / sqrtf(tot / (float)H + eps);
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int c4 = threadIdx.x + v * kBlock;
    if (c4 < n4) split4_store(xv[v], gv[v], inv, hi + r * H + 4 * c4, lo + r * H + 4 * c4);
  }
}

__global__ void __launch_bounds__(kBlock)
    rmsnorm_rows_split_kernel(const float *X, const uint16_t *g, float eps, int H, uint16_t *hi,
                              uint16_t *lo) {
  __shared__ float red4[4];
  const size_t r = blockIdx.x;
  const float *x = X + r * H;
  float ss = 0.f;
  for (int j = threadIdx.x; j < H; j += kBlock) ss += x[j] * x[j];
  const float tot = block_sum(ss, red4);
  const float inv = 1.0f / sqrtf(tot / (float)H + eps);
  for (int j = threadIdx.x; j < H; j += kBlock)
    split2(bf16f(g[j]) * (x[j] * inv), hi + r * H + j, lo + r * H + j);
}

__global__ void split_kernel(const float *X, size_t n, uint16_t *hi, uint16_t *lo) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i < n) split2(X[i], hi + i, lo + i);
}

// MFMA GEMM, C[M,N] = (A_hi + A_lo)[M,K] . W[N,K]^T, both operands K-contiguous.
// Workgroup tile 128 (M) x 64 (N) x 64 (K); wave w owns rows 32w..32w+31 and
// both 32-column halves: 2 accumulators of v_mfma_f32_32x32x16_bf16, each fed
// by the hi and the lo term of A. Operand fragments: lane l holds row/col
// (l % 32) and K-octet (l / 32) of a 16-wide K step, so A and W share the K
// mapping; the 32x32 result sits at row 8*(i/4) + 4*(l/32) + i%4, col l%32.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBN = 64, GBK = 64, GLD = GBK + 8;  // LDS row pitch (bf16)

__device__ __forceinline__ u32x4 load_tile8(const uint16_t *src, int row, int rows, int kk,
                                            int K, bool vec) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (row >= rows) return v;
  const uint16_t *p = src + (size_t)row * K + kk;
  if (vec && kk + 8 <= K) return *(const u32x4 *)p;
  uint16_t t[8];
#pragma unroll
  for (int e = 0; e < 8; e++) t[e] = kk + e < K ? p[e] : (uint16_t)0;
  v[0] = t[0] | ((uint32_t)t[1] << 16);
  v[1] = t[2] | ((uint32_t)t[3] << 16);
  v[2] = t[4] | ((uint32_t)t[5] << 16);
  v[3] = t[6] | ((uint32_t)t[7] << 16);
  return v;
}

// One output element of the GEMM epilogues; `partner` is column col ^ 1 of
// the same row (the gate/up pair, the RoPE pair)
template <int EPI>
__device__ __forceinline__ void gemm_store(const GemmArgs &a, int row, int col, float c,
                                           float partner) {
  const int N = a.N;
  if (EPI == EPI_STORE) {
    a.y[(size_t)row * N + col] = c;
  } else if (EPI == EPI_RESID) {
    a.y[(size_t)row * N + col] += c;
  } else if (EPI == EPI_GU) {
    if ((col & 1) == 0) {
      const size_t o = (size_t)row * (N >> 1) + (col >> 1);
      split2(silu(c) * partner, a.h_hi + o, a.h_lo + o);
    }
  } else if (EPI == EPI_QKV) {
    if ((col & 1) == 0) {
      const int d = a.head_dim, half = d >> 1;
      const int pos = a.start_pos + row;
      const float y0 = c + a.bias[col], y1 = partner + a.bias[col + 1];
      if (col < a.q_dim + a.kv_dim) {
        const bool is_q = col < a.q_dim;
        const int rr = is_q ? col : col - a.q_dim;
        const int2 hp = divmod_n(rr >> 1, half);
        const int head = hp.x, p = hp.y;
        const float2 cs = a.rope[(size_t)pos * half + p];
        const float o0 = y0 * cs.x - y1 * cs.y;
        const float o1 = y1 * cs.x + y0 * cs.y;
        if (is_q) {
          float *qrow = a.q_out + (size_t)row * a.q_dim;
          qrow[head * d + p] = o0;
          qrow[head * d + p + half] = o1;
        } else {
          const size_t base = ((size_t)head * a.max_seq + pos) * d;
          store_kv(a.kc, base + p, o0, a.kv_bf16);
          store_kv(a.kc, base + p + half, o1, a.kv_bf16);
        }
      } else {
        const int2 hj = divmod_n(col - a.q_dim - a.kv_dim, d);
        const size_t base = ((size_t)hj.x * a.max_seq + pos) * d + hj.y;
        store_kv(a.vc, base, y0, a.kv_bf16);
        store_kv(a.vc, base + 1, y1, a.kv_bf16);
      }
    }
  }
}

// The global reads of gemm_store for one element, issued ahead of the stores
// of a batch (the stores may alias them to the compiler, so each element's
// read would otherwise wait for the previous element's stores): EPI_RESID's
// residual; EPI_QKV's bias pair and RoPE (cos, sin)
struct EpiIn {
  float2 u, v;
};
template <int EPI>
__device__ __forceinline__ EpiIn gemm_epi_load(const GemmArgs &a, int row, int col) {
  // branch-free: a load under a divergent branch makes the compiler wait for
  // it where the branch joins, one round trip per element. (row, col) must be
  // in range; odd columns load their pair's values, which go unused.
  EpiIn in;
  in.u = make_float2(0.f, 0.f);
  in.v = make_float2(1.f, 0.f);
  if (EPI == EPI_RESID) {
    in.u.x = a.y[(size_t)row * a.N + col];
  } else if (EPI == EPI_QKV) {
    const int ce = col & ~1, half = a.head_dim >> 1;
    in.u = make_float2(a.bias[ce], a.bias[ce + 1]);
    // v columns (past q and k) use no RoPE factor; any in-range one is read
    const int rr = ce < a.q_dim ? ce : ce - a.q_dim;
    in.v = a.rope[(size_t)(a.start_pos + row) * half + divmod_n(rr >> 1, half).y];
  }
  return in;
}
// gemm_store with the element's reads from gemm_epi_load
template <int EPI>
__device__ __forceinline__ void gemm_store_in(const GemmArgs &a, int row, int col, float c,
                                              float partner, const EpiIn &in) {
  if (EPI == EPI_RESID) {
    a.y[(size_t)row * a.N + col] = in.u.x + c;
  } else if (EPI == EPI_QKV) {
    if ((col & 1) == 0) {
      const int d = a.head_dim, half = d >> 1;
      const int pos = a.start_pos + row;
      const float y0 = c + in.u.x, y1 = partner + in.u.y;
      if (col < a.q_dim + a.kv_dim) {
        const bool is_q = col < a.q_dim;
        const int rr = is_q ? col : col - a.q_dim;
        const int2 hp = divmod_n(rr >> 1, half);
        const int head = hp.x, p = hp.y;
        const float2 cs = in.v;
        const float o0 = y0 * cs.x - y1 * cs.y;
        const float o1 = y1 * cs.x + y0 * cs.y;
        if (is_q) {
          float *qrow = a.q_out + (size_t)row * a.q_dim;
          qrow[head * d + p] = o0;
          qrow[head * d + p + half] = o1;
        } else {
          const size_t base = ((size_t)head * a.max_seq + pos) * d;
          store_kv(a.kc, base + p, o0, a.kv_bf16);
          store_kv(a.kc, base + p + half, o1, a.kv_bf16);
        }
      } else {
        const int2 hj = divmod_n(col - a.q_dim - a.kv_dim, d);
        const size_t base = ((size_t)hj.x * a.max_seq + pos) * d + hj.y;
        store_kv(a.vc, base, y0, a.kv_bf16);
        store_kv(a.vc, base + 1, y1, a.kv_bf16);
      }
    }
  } else {
    gemm_store<EPI>(a, row, col, c, partner);
  }
}

// One K tile of both operands: A (hi, lo) 128 rows x 8 octets, W 64 x 8;
// thread tid holds octets tid + it * kBlock
struct GemmTile {
  u32x4 ah[4], al[4], w[2];
};
__device__ __forceinline__ void gemm_load_tile(const GemmArgs &a, int m0, int n0, int k0, bool vec,
                                               int tid, GemmTile &t) {
#pragma unroll
  for (int it = 0; it < 4; it++) {
    const int v = tid + it * kBlock, r = v >> 3, o = v & 7;
    t.ah[it] = load_tile8(a.a_hi, m0 + r, a.M, k0 + o * 8, a.K, vec);
    t.al[it] = load_tile8(a.a_lo, m0 + r, a.M, k0 + o * 8, a.K, vec);
  }
#pragma unroll
  for (int it = 0; it < 2; it++) {
    const int v = tid + it * kBlock, r = v >> 3, o = v & 7;
    t.w[it] = load_tile8(a.w, n0 + r, a.N, k0 + o * 8, a.K, vec);
  }
}

// MFMA GEMM, C[M,N] = (A_hi + A_lo)[M,K] . W[N,K]^T, both operands K-contiguous.
// Workgroup tile 128 (M) x 64 (N) x 64 (K); wave w owns rows 32w..32w+31 and
// both 32-column halves: 2 accumulators of v_mfma_f32_32x32x16_bf16, each fed
// by the hi and the lo term of A. Operand fragments: lane l holds row/col
// (l % 32) and K-octet (l / 32) of a 16-wide K step, so A and W share the K
// mapping; the 32x32 result sits at row 8*(i/4) + 4*(l/32) + i%4, col l%32.
// The next K tile loads into registers while the current one is multiplied
// (a deeper register pipeline measured slower: it halves occupancy).
// blockIdx.z takes the K steps [z * kps, (z + 1) * kps): with more than one
// split the tile goes to the partial buffer a.ws[z] and gemm_reduce_kernel
// adds the splits in order and applies the epilogue.
template <int EPI>
__global__ void __launch_bounds__(kBlock) gemm_mfma_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t ahi_s[GBM * GLD];
  __shared__ __attribute__((aligned(16))) uint16_t alo_s[GBM * GLD];
  __shared__ __attribute__((aligned(16))) uint16_t w_s[GBN * GLD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * GBN, m0 = blockIdx.y * GBM;
  const int M = a.M, N = a.N, K = a.K;
  const int kbeg = blockIdx.z * a.kps * GBK, kend = min(K, kbeg + a.kps * GBK);
  // 16-byte operand loads need K % 8 == 0 and 16-byte aligned bases
  const bool vec = (K & 7) == 0 && (((uintptr_t)a.a_hi | (uintptr_t)a.a_lo | (uintptr_t)a.w) & 15) == 0;
  f32x16 acc0, acc1;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    acc0[i] = 0.f;
    acc1[i] = 0.f;
  }
  GemmTile t;
  if (kbeg < kend) gemm_load_tile(a, m0, n0, kbeg, vec, tid, t);
  for (int k0 = kbeg; k0 < kend; k0 += GBK) {
#pragma unroll
    for (int it = 0; it < 4; it++) {
      const int v = tid + it * kBlock, r = v >> 3, o = v & 7;
      *(u32x4 *)&ahi_s[r * GLD + o * 8] = t.ah[it];
      *(u32x4 *)&alo_s[r * GLD + o * 8] = t.al[it];
    }
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int v = tid + it * kBlock, r = v >> 3, o = v & 7;
      *(u32x4 *)&w_s[r * GLD + o * 8] = t.w[it];
    }
    __syncthreads();
    if (k0 + GBK < kend) gemm_load_tile(a, m0, n0, k0 + GBK, vec, tid, t);
#pragma unroll
    for (int ks = 0; ks < GBK; ks += 16) {
      const int kk = ks + (lane >> 5) * 8;
      const int ar = wave * 32 + (lane & 31);
      const bf16x8 ah = __builtin_bit_cast(bf16x8, *(const u32x4 *)&ahi_s[ar * GLD + kk]);
      const bf16x8 al = __builtin_bit_cast(bf16x8, *(const u32x4 *)&alo_s[ar * GLD + kk]);
      const bf16x8 b0 = __builtin_bit_cast(bf16x8, *(const u32x4 *)&w_s[(lane & 31) * GLD + kk]);
      const bf16x8 b1 =
          __builtin_bit_cast(bf16x8, *(const u32x4 *)&w_s[(32 + (lane & 31)) * GLD + kk]);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, b0, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, b1, acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, b0, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, b1, acc1, 0, 0, 0);
    }
    __syncthreads();
  }
  const bool split = gridDim.z > 1;
  float *ws = a.ws + (size_t)blockIdx.z * M * N;
#pragma unroll
  for (int nh = 0; nh < 2; nh++) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float c = nh ? acc1[i] : acc0[i];
      const int row = m0 + wave * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
      const int col = n0 + nh * 32 + (lane & 31);
      const float partner = __shfl_xor(c, 1, kWave);  // column col ^ 1, same row
      if (row >= M || col >= N) continue;
      if (split) ws[(size_t)row * N + col] = c;
      else gemm_store<EPI>(a, row, col, c, partner);
    }
  }
}

// ---- prefill GEMM with a two-stage LDS pipeline (K % 64 == 0) ---------------
//
// C[M,N] = (A_hi + A_lo)[M,K] . W[N,K]^T on v_mfma_f32_32x32x16_bf16. The
// workgroup is WGM x WGN wavefronts; wave (wm, wn) owns a (32 MB) x (32 NB)
// block of the (32 MB WGM) x (32 NB WGN) workgroup tile, MB x NB accumulators.
// Per 64-wide K stage every thread loads its share of the A hi/lo and W rows
// as 16-byte chunks (a wavefront load covers 8 rows x 128 B) into one of
// three register sets, through buffer descriptors whose range ends at the
// matrix, so rows past M or N read as zero; a set goes to one of two LDS
// stages while the other stage is multiplied, one barrier per stage. Loads run
// two stages ahead of their LDS store, and every stage issues its loads
// unconditionally (a stage past the split reads out of range: zeros, no
// traffic), so the compiler's wait before a store leaves the younger stages in
// flight. An LDS row is the 128 B of one matrix row with chunk c at slot
// c ^ (row & 7) ^ ((row >> 3) & 1): the 8 or 16 consecutive rows an MFMA
// fragment read serves per LDS cycle (32 or 64 banks) hit distinct banks, and
// so do the chunk stores. The next 16-wide K step's fragments are read from
// LDS while the current step's MFMAs run.
// LDS bytes per MFMA fall with MB and NB: (2 MB + NB) 1 KB fragments feed
// 2 MB NB MFMAs (the hi and the lo term share each W fragment).
template <int MB_, int NB_, int WGM_, int WGN_>
struct PfCfg {
  static constexpr int MB = MB_, NB = NB_, WGM = WGM_, WGN = WGN_;
  static constexpr int NTH = 64 * WGM * WGN;
  static constexpr int BM = 32 * MB * WGM, BN = 32 * NB * WGN;
  static constexpr int ACH = BM * 8, WCH = BN * 8;  // 16-byte chunks per stage
  static constexpr int ALD = (ACH + NTH - 1) / NTH, WLD = (WCH + NTH - 1) / NTH;
  static constexpr int AL_OFF = ACH * 16, W_OFF = 2 * ACH * 16;
  static constexpr int STAGE = (2 * ACH + WCH) * 16;
  static constexpr int LDS = 2 * STAGE;
  static constexpr int R = 3;  // register sets: loads run R - 1 stages ahead
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pf_rsrc(const uint16_t *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}

// gemm_pf_kernel's QKV epilogue (bias, RoPE, q / K / V stores) by column
// pairs: lane pair index pi takes columns (2j, 2j + 1) of tile row pi / (BN/2)
// from the accumulator tile cs in LDS, so every lane works; a batch of pairs'
// bias and RoPE reads goes out before its stores. REG 0 / 1 / 2: a full tile
// of q / k / v columns with power-of-two head dims (shifts, no bounds or
// region tests; KB: bf16 cache); REG 3: any tile, every test per pair. Same
// arithmetic as gemm_store<EPI_QKV> for each element.
template <class C, int REG, bool KB>
__device__ __forceinline__ void qkv_pairs(const GemmArgs &a, const float *cs, int tid, int m0, int n0) {
  // one batch of up to 32 pairs: with one wave per SIMD nothing hides a
  // batch's read latency, so the reads go out together
  constexpr int HB = C::BN / 2, NIT2 = C::BM * HB / C::NTH;
  constexpr int EB2 = NIT2 <= 32 ? NIT2 : (NIT2 % 8 == 0 ? 8 : 1);
  static_assert(C::BM * HB % C::NTH == 0, "whole epilogue iterations");
  const int M = a.M, N = a.N, d = a.head_dim, half = d >> 1, qd = a.q_dim, qkd = a.q_dim + a.kv_dim;
  const int lh = __builtin_ctz(half), ld = lh + 1;
  for (int it0 = 0; it0 < NIT2; it0 += EB2) {
    float2 bv[EB2], rv[EB2];
#pragma unroll
    for (int e = 0; e < EB2; e++) {
      const int pi = tid + (it0 + e) * C::NTH;
      const int row = REG < 3 ? m0 + pi / HB : min(m0 + pi / HB, M - 1);
      const int col = REG < 3 ? n0 + 2 * (pi % HB) : min(n0 + 2 * (pi % HB), N - 2);
      bv[e] = make_float2(a.bias[col], a.bias[col + 1]);
      if (REG == 0 || REG == 1) {
        const int rr = REG == 0 ? col : col - qd;
        rv[e] = a.rope[(size_t)(a.start_pos + row) * half + ((rr >> 1) & (half - 1))];
      } else if (REG == 3) {
        const int rr = col < qd ? col : col - qd;  // v columns read an unused factor
        rv[e] = a.rope[(size_t)(a.start_pos + row) * half + divmod_n(rr >> 1, half).y];
      }
    }
#pragma unroll
    for (int e = 0; e < EB2; e++) {
      const int pi = tid + (it0 + e) * C::NTH;
      const int tr = pi / HB, tc = 2 * (pi % HB);
      const int row = m0 + tr, col = n0 + tc;
      if (REG == 3 && !(row < M && col < N)) continue;
      const float2 yv = *(const float2 *)(cs + tr * C::BN + tc);
      const float y0 = yv.x + bv[e].x, y1 = yv.y + bv[e].y;
      const int pos = a.start_pos + row;
      if (REG == 0) {
        const int u = col >> 1;
        const float o0 = y0 * rv[e].x - y1 * rv[e].y;
        const float o1 = y1 * rv[e].x + y0 * rv[e].y;
        float *qr = a.q_out + (size_t)row * qd + ((u >> lh) << ld) + (u & (half - 1));
        qr[0] = o0;
        qr[half] = o1;
      } else if (REG == 1) {
        const int u = (col - qd) >> 1;
        const float o0 = y0 * rv[e].x - y1 * rv[e].y;
        const float o1 = y1 * rv[e].x + y0 * rv[e].y;
        const size_t base = ((size_t)(u >> lh) * a.max_seq + pos) * d + (u & (half - 1));
        if (KB) {
          ((uint16_t *)a.kc)[base] = f2bf(o0);
          ((uint16_t *)a.kc)[base + half] = f2bf(o1);
        } else {
          ((float *)a.kc)[base] = o0;
          ((float *)a.kc)[base + half] = o1;
        }
      } else if (REG == 2) {
        const int rr = col - qkd;
        const size_t base = ((size_t)(rr >> ld) * a.max_seq + pos) * d + (rr & (d - 1));
        if (KB) {
          *(uint32_t *)((uint16_t *)a.vc + base) = (uint32_t)f2bf(y0) | ((uint32_t)f2bf(y1) << 16);
        } else {
          *(float2 *)((float *)a.vc + base) = make_float2(y0, y1);
        }
      } else {
        if (col < qkd) {
          const bool is_q = col < qd;
          const int2 hp = divmod_n((is_q ? col : col - qd) >> 1, half);
          const float o0 = y0 * rv[e].x - y1 * rv[e].y;
          const float o1 = y1 * rv[e].x + y0 * rv[e].y;
          if (is_q) {
            float *qr = a.q_out + (size_t)row * qd + hp.x * d + hp.y;
            qr[0] = o0;
            qr[half] = o1;
          } else {
            const size_t base = ((size_t)hp.x * a.max_seq + pos) * d + hp.y;
            store_kv(a.kc, base, o0, a.kv_bf16);
            store_kv(a.kc, base + half, o1, a.kv_bf16);
          }
        } else {
          const int2 hj = divmod_n(col - qkd, d);
          const size_t base = ((size_t)hj.x * a.max_seq + pos) * d + hj.y;
          store_kv(a.vc, base, y0, a.kv_bf16);
          store_kv(a.vc, base + 1, y1, a.kv_bf16);
        }
      }
    }
  }
}

// TAIL: the launch covers the last gridDim.x * BN columns of N (a tail
// launch after one over the first columns).
template <class C, int EPI, bool TAIL = false>
__global__ void __launch_bounds__(C::NTH) gemm_pf_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t pf_sm[];
  constexpr int R = C::R;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % C::WGM, wn = wave / C::WGM;
  // Tile order. Workgroup L (in launch order) runs on XCD L % 8, and each XCD
  // has its own L2. With 8 or more M tiles, XCD c takes the c-th contiguous
  // run of tiles in an order that walks groups of 4 M tiles along N, so the
  // workgroups resident on one XCD share their A and W panels: at 2048 rows
  // the L2 hit rate goes from 44 % to 76 % (bit-identical output; each tile
  // is computed the same way wherever it runs).
  const int gx = gridDim.x, gy = gridDim.y, gxy = gx * gy;
  int tn = blockIdx.x, tm = blockIdx.y, z = blockIdx.z;
  if (gy >= 8) {
    const int T = gxy * gridDim.z, L = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const int xc = L & 7, t = xc * (T >> 3) + min(xc, T & 7) + (L >> 3);
    z = t / gxy;
    const int t2 = t - z * gxy, g = t2 / (4 * gx), r = t2 - g * 4 * gx, gm = min(4, gy - 4 * g);
    tn = r / gm;
    tm = 4 * g + (r - tn * gm);
  }
  const int nb = TAIL ? a.N - gx * C::BN : 0;
  const int n0 = nb + tn * C::BN, m0 = tm * C::BM;
  const int M = a.M, N = a.N, K = a.K;
  const int nks = K >> 6, S = gridDim.z;
  const int ks0 = (int)((long)z * nks / S), ks1 = (int)((long)(z + 1) * nks / S);
  const int nst = ks1 - ks0;
  // descriptors start at the tile's first row; rows past the matrix read 0
  const __amdgpu_buffer_rsrc_t rah = pf_rsrc(a.a_hi + (size_t)m0 * K, (uint32_t)(M - m0) * K * 2);
  const __amdgpu_buffer_rsrc_t ral = pf_rsrc(a.a_lo + (size_t)m0 * K, (uint32_t)(M - m0) * K * 2);
  const __amdgpu_buffer_rsrc_t rw = pf_rsrc(a.w + (size_t)n0 * K, (uint32_t)(N - n0) * K * 2);

  u32x4 ra[R][C::ALD], rl[R][C::ALD], rb[R][C::WLD];
  // stage ks into register set `set`; a stage past the split sits at byte
  // offset 2^31 of each row, beyond every descriptor's range (< 2^31 bytes)
  auto gload = [&](int set, int ks) {
    const uint32_t kb = ks < ks1 ? (uint32_t)ks * 128u : 0x80000000u;
#pragma unroll
    for (int i = 0; i < C::ALD; i++) {
      const int q = tid + i * C::NTH;
      if (C::ACH % C::NTH == 0 || q < C::ACH) {
        const int off = (int)((uint32_t)((q >> 3) * K * 2) + kb + (uint32_t)((q & 7) << 4));
        ra[set][i] = __builtin_amdgcn_raw_buffer_load_b128(rah, off, 0, 0);
        rl[set][i] = __builtin_amdgcn_raw_buffer_load_b128(ral, off, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < C::WLD; i++) {
      const int q = tid + i * C::NTH;
      if (C::WCH % C::NTH == 0 || q < C::WCH) {
        const int off = (int)((uint32_t)((q >> 3) * K * 2) + kb + (uint32_t)((q & 7) << 4));
        rb[set][i] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0);
      }
    }
  };
  // the register set's chunks into LDS stage `st`: the thread's stores are
  // numbered e = 0 .. NW - 1 (A hi, A lo, W) and part p of np takes those with
  // e * np / NW == p
  constexpr int NW = 2 * C::ALD + C::WLD;
  auto swrite = [&](int set, int st, int p, int np) {
    uint8_t *base = pf_sm + st * C::STAGE;
#pragma unroll
    for (int i = 0; i < C::ALD; i++) {
      const int q = tid + i * C::NTH;
      if (C::ACH % C::NTH == 0 || q < C::ACH) {
        const int r = q >> 3, slot = ((q & 7) ^ (r & 7) ^ ((r >> 3) & 1)) << 4;
        if ((2 * i) * np / NW == p) *(u32x4 *)(base + r * 128 + slot) = ra[set][i];
        if ((2 * i + 1) * np / NW == p) *(u32x4 *)(base + C::AL_OFF + r * 128 + slot) = rl[set][i];
      }
    }
#pragma unroll
    for (int i = 0; i < C::WLD; i++) {
      const int q = tid + i * C::NTH;
      if (C::WCH % C::NTH == 0 || q < C::WCH) {
        const int r = q >> 3, slot = ((q & 7) ^ (r & 7) ^ ((r >> 3) & 1)) << 4;
        if ((2 * C::ALD + i) * np / NW == p) *(u32x4 *)(base + C::W_OFF + r * 128 + slot) = rb[set][i];
      }
    }
  };

  f32x16 acc[C::MB][C::NB];
#pragma unroll
  for (int i = 0; i < C::MB; i++)
#pragma unroll
    for (int j = 0; j < C::NB; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  const int arow = (wm * C::MB * 32 + (lane & 31)) * 128;
  const int wrow = (wn * C::NB * 32 + (lane & 31)) * 128;
  // the 64-wide stage in LDS stage `st`: 4 K steps of 16, each step's
  // fragments read while the previous step's MFMAs run. After each step's
  // MFMAs a quarter of register set `wset` goes to the other LDS stage (last
  // read before the previous barrier), so the next stage's stores share the
  // LDS with this stage's reads instead of stalling every wave after the
  // barrier.
  auto mult = [&](int st, int wset) {
    const uint8_t *base = pf_sm + st * C::STAGE;
    bf16x8 fh[2][C::MB], fl[2][C::MB], fw[2][C::NB];
    auto ldfrag = [&](int buf, int ks) {
      const int swz = ((2 * ks + (lane >> 5)) ^ (lane & 7) ^ ((lane >> 3) & 1)) << 4;
#pragma unroll
      for (int i = 0; i < C::MB; i++) {
        fh[buf][i] = __builtin_bit_cast(bf16x8, *(const u32x4 *)(base + arow + i * 4096 + swz));
        fl[buf][i] = __builtin_bit_cast(bf16x8, *(const u32x4 *)(base + C::AL_OFF + arow + i * 4096 + swz));
      }
#pragma unroll
      for (int j = 0; j < C::NB; j++)
        fw[buf][j] = __builtin_bit_cast(bf16x8, *(const u32x4 *)(base + C::W_OFF + wrow + j * 4096 + swz));
    };
    ldfrag(0, 0);
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
      const int b = ks & 1;
      if (ks + 1 < 4) ldfrag(b ^ 1, ks + 1);
#pragma unroll
      for (int i = 0; i < C::MB; i++)
#pragma unroll
        for (int j = 0; j < C::NB; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fh[b][i], fw[b][j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < C::MB; i++)
#pragma unroll
        for (int j = 0; j < C::NB; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fl[b][i], fw[b][j], acc[i][j], 0, 0, 0);
      swrite(wset, st ^ 1, ks, 4);
      // schedule of the step: one MFMA, then one of the next step's fragment
      // reads, then one of the next stage's LDS stores, in turn (the reads
      // stay ahead of their MFMAs, which the scheduler otherwise moves each
      // read next to; against all reads first, then every MFMA: 2048-id
      // prefill 14.98 -> 14.70 ms), and a fence at the step's end. In the
      // stage's first step the global loads issued at the stage start go out
      // two after each MFMA instead of in one burst (2048 ids a further
      // 0.7 %; one or four after each MFMA, or two before it, no better).
#pragma unroll
      for (int g = 0; g < 2 * C::MB * C::NB; g++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if (ks == 0) __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // global loads
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // stage s lives in register set s % R and LDS stage s & 1
  if (nst > 0) {
    gload(0, ks0);
    swrite(0, 0, 0, 1);
#pragma unroll
    for (int s = 1; s < R; s++) gload(s, ks0 + s);
  }
  __syncthreads();
  const int nfull = nst / R * R;
  for (int it0 = 0; it0 < nfull; it0 += R) {
#pragma unroll
    for (int u = 0; u < R; u++) {
      const int it = it0 + u;
      gload(u, ks0 + it + R);
      mult(it & 1, (u + 1) % R);
      __syncthreads();
    }
  }
#pragma unroll
  for (int u = 0; u < R; u++) {
    const int it = nfull + u;
    if (it < nst) {
      mult(it & 1, (u + 1) % R);
      __syncthreads();
    }
  }

  // the accumulator tile goes through LDS (free after the last stage's
  // barrier), then each thread takes elements tid, tid + NTH, ... in row-major
  // order: coalesced stores, and the epilogue's partner column (col ^ 1) is a
  // plain LDS read
  static_assert(C::BM * C::BN * 4 <= C::LDS, "accumulator tile exceeds the LDS stages");
  float *cs = (float *)pf_sm;
#pragma unroll
  for (int i = 0; i < C::MB; i++)
#pragma unroll
    for (int j = 0; j < C::NB; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int tr = wm * C::MB * 32 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        const int tc = wn * C::NB * 32 + j * 32 + (lane & 31);
        cs[tr * C::BN + tc] = acc[i][j][e];
      }
  __syncthreads();
  const bool split = S > 1;
  float *ws = a.ws + (size_t)z * M * N;
  if (EPI == EPI_GU && !split) {
    // h = silu(gate) * up by column pairs (gate 2j, up 2j + 1), one pair per
    // lane: every lane works and consecutive lanes write consecutive h
    constexpr int HB = C::BN / 2;
    for (int pi = tid; pi < C::BM * HB; pi += C::NTH) {
      const int tr = pi / HB, tc = 2 * (pi % HB);
      const int row = m0 + tr, col = n0 + tc;
      if (row < M && col < N) {
        const float2 gu = *(const float2 *)(cs + tr * C::BN + tc);
        const size_t o = (size_t)row * (N >> 1) + (col >> 1);
        split2(silu(gu.x) * gu.y, a.h_hi + o, a.h_lo + o);
      }
    }
    return;
  }
  if (split || EPI == EPI_STORE || EPI == EPI_GU) {
    for (int idx = tid; idx < C::BM * C::BN; idx += C::NTH) {
      const int tr = idx / C::BN, tc = idx % C::BN;
      const int row = m0 + tr, col = n0 + tc;
      if (row < M && col < N) {
        const float c = cs[idx];
        if (split) ws[(size_t)row * N + col] = c;
        else gemm_store<EPI>(a, row, col, c, cs[idx ^ 1]);
      }
    }
    return;
  }
  if constexpr (EPI == EPI_QKV) {
    // Decisions that are uniform for the tile are taken once here: a full
    // tile whose columns are all q, all k or all v, with power-of-two head
    // dims, runs a branch-free pair loop (see qkv_pairs).
    const int half = a.head_dim >> 1, qd = a.q_dim, qkd = a.q_dim + a.kv_dim;
    const bool fast = (half & (half - 1)) == 0 && m0 + C::BM <= M && n0 + C::BN <= N;
    const int reg = !fast ? 3 : n0 + C::BN <= qd ? 0 : (n0 >= qd && n0 + C::BN <= qkd) ? 1 : n0 >= qkd ? 2 : 3;
    const bool kb = a.kv_bf16 != 0;
    switch (reg * 2 + (kb ? 1 : 0)) {
      case 0: qkv_pairs<C, 0, false>(a, cs, tid, m0, n0); break;
      case 1: qkv_pairs<C, 0, true>(a, cs, tid, m0, n0); break;
      case 2: qkv_pairs<C, 1, false>(a, cs, tid, m0, n0); break;
      case 3: qkv_pairs<C, 1, true>(a, cs, tid, m0, n0); break;
      case 4: qkv_pairs<C, 2, false>(a, cs, tid, m0, n0); break;
      case 5: qkv_pairs<C, 2, true>(a, cs, tid, m0, n0); break;
      default: qkv_pairs<C, 3, false>(a, cs, tid, m0, n0); break;
    }
    return;
  }
  // the epilogues that read global memory: a batch of EB elements' reads
  // first, then their stores
  constexpr int NIT = C::BM * C::BN / C::NTH, EB = NIT % 8 == 0 ? 8 : 1;
  static_assert(C::BM * C::BN % C::NTH == 0, "whole epilogue iterations");
  for (int it0 = 0; it0 < NIT; it0 += EB) {
    EpiIn in[EB];
#pragma unroll
    for (int e = 0; e < EB; e++) {
      const int idx = tid + (it0 + e) * C::NTH;
      const int row = m0 + idx / C::BN, col = n0 + idx % C::BN;
      in[e] = gemm_epi_load<EPI>(a, min(row, M - 1), min(col, N - 1));  // clamped, unconditional
    }
#pragma unroll
    for (int e = 0; e < EB; e++) {
      const int idx = tid + (it0 + e) * C::NTH;
      const int row = m0 + idx / C::BN, col = n0 + idx % C::BN;
      if (row < M && col < N) gemm_store_in<EPI>(a, row, col, cs[idx], cs[idx ^ 1], in[e]);
    }
  }
}

// EPI_RESID's K splits fused with the RMSNorm that reads the result: row r of
// y += (the splits of row r, added in split order), then the normalised row
// (gains g) as bf16 hi/lo planes, as rmsnorm_rows_split_kernel writes them.
// One workgroup per row, NV 4-column groups per thread.
template <int NV>
__global__ void __launch_bounds__(kBlock) gemm_resid_norm_kernel(GemmArgs a, int splits,
                                                                 const uint16_t *g, float eps,
                                                                 uint16_t *hi, uint16_t *lo) {
  __shared__ float red4[4];
  const int r = blockIdx.x, H = a.N, n4 = H >> 2;
  const size_t MN = (size_t)a.M * H;
  const float *ws = a.ws + (size_t)r * H;
  float *y = a.y + (size_t)r * H;
  // the residual and a batch of up to 8 splits for all NV column groups are
  // loaded before any is added (one memory round trip per batch); each
  // group's splits are added in split order
  constexpr int ZB = 8;
  float4 xv[NV], c[NV];
  uint2 gv[NV];  // the group's four gains, loaded before any store
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int c4 = threadIdx.x + v * kBlock;
    c[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    xv[v] = c4 < n4 ? *(const float4 *)(y + 4 * c4) : make_float4(0.f, 0.f, 0.f, 0.f);
    gv[v] = c4 < n4 ? *(const uint2 *)(g + 4 * c4) : make_uint2(0u, 0u);
  }
  for (int z0 = 0; z0 < splits; z0 += ZB) {
    float4 w[ZB][NV];
#pragma unroll
    for (int dz = 0; dz < ZB; dz++)
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const int c4 = threadIdx.x + v * kBlock;
        w[dz][v] = z0 + dz < splits && c4 < n4 ? *(const float4 *)(ws + (z0 + dz) * MN + 4 * c4)
                                               : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
    for (int dz = 0; dz < ZB; dz++)
#pragma unroll
      for (int v = 0; v < NV; v++)
        if (z0 + dz < splits) {
          c[v].x += w[dz][v].x;
          c[v].y += w[dz][v].y;
          c[v].z += w[dz][v].z;
          c[v].w += w[dz][v].w;
        }
  }
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int c4 = threadIdx.x + v * kBlock;
    if (c4 < n4) {
      float4 x = xv[v];
      x.x += c[v].x;
      x.y += c[v].y;
      x.z += c[v].z;
      x.w += c[v].w;
      *(float4 *)(y + 4 * c4) = x;
      xv[v] = x;
      ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
    } else {
      xv[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  const float tot = block_sum(ss, red4);
  const float inv = 1.0f / sqrtf(tot / (float)H + eps);
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int c4 = threadIdx.x + v * kBlock;
    if (c4 < n4) split4_store(xv[v], gv[v], inv, hi + (size_t)r * H + 4 * c4, lo + (size_t)r * H + 4 * c4);
  }
}

// gemm_reduce_kernel for N % 4 == 0: one thread per two column pairs, float4 loads
template <int EPI>
__global__ void __launch_bounds__(kBlock) gemm_reduce4_kernel(GemmArgs a, int splits) {
  const int n4 = a.N >> 2;
  const size_t i = blockIdx.x * (size_t)kBlock + threadIdx.x;
  if (i >= (size_t)a.M * n4) return;
  const int row = (int)(i / (size_t)n4), col = 4 * (int)(i % (size_t)n4);
  const size_t MN = (size_t)a.M * a.N, off = (size_t)row * a.N + col;
  // a batch of up to 8 splits is loaded before any is added (one memory round
  // trip per batch); the splits are added in split order
  constexpr int ZB = 8;
  float4 c = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int z0 = 0; z0 < splits; z0 += ZB) {
    float4 w[ZB];
#pragma unroll
    for (int dz = 0; dz < ZB; dz++)
      w[dz] = z0 + dz < splits ? *(const float4 *)(a.ws + (z0 + dz) * MN + off) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int dz = 0; dz < ZB; dz++)
      if (z0 + dz < splits) {
        c.x += w[dz].x;
        c.y += w[dz].y;
        c.z += w[dz].z;
        c.w += w[dz].w;
      }
  }
  if constexpr (EPI == EPI_RESID || EPI == EPI_QKV) {
    // the epilogue's global reads for all four columns ahead of their stores
    EpiIn in[4];
#pragma unroll
    for (int e = 0; e < 4; e++) in[e] = gemm_epi_load<EPI>(a, row, col + e);
    gemm_store_in<EPI>(a, row, col, c.x, c.y, in[0]);
    gemm_store_in<EPI>(a, row, col + 1, c.y, c.x, in[1]);
    gemm_store_in<EPI>(a, row, col + 2, c.z, c.w, in[2]);
    gemm_store_in<EPI>(a, row, col + 3, c.w, c.z, in[3]);
  } else {
    gemm_store<EPI>(a, row, col, c.x, c.y);
    gemm_store<EPI>(a, row, col + 1, c.y, c.x);
    gemm_store<EPI>(a, row, col + 2, c.z, c.w);
    gemm_store<EPI>(a, row, col + 3, c.w, c.z);
  }
}

// the K splits of gemm_mfma_kernel, added in split order, then the epilogue;
// one thread per column pair (a last odd column stands alone)
template <int EPI>
__global__ void __launch_bounds__(kBlock) gemm_reduce_kernel(GemmArgs a, int splits) {
  const int np = (a.N + 1) >> 1;
  const size_t i = blockIdx.x * (size_t)kBlock + threadIdx.x;
  if (i >= (size_t)a.M * np) return;
  const int row = (int)(i / (size_t)np), col = 2 * (int)(i % (size_t)np);
  const bool two = col + 1 < a.N;
  const size_t MN = (size_t)a.M * a.N, off = (size_t)row * a.N + col;
  float c0 = 0.f, c1 = 0.f;
  for (int z = 0; z < splits; z++) {
    c0 += a.ws[z * MN + off];
    if (two) c1 += a.ws[z * MN + off + 1];
  }
  gemm_store<EPI>(a, row, col, c0, c1);
  if (two) gemm_store<EPI>(a, row, col + 1, c1, c0);
}

// Causal prefill attention: workgroup = (query head, 32 queries); 8 lanes per
// query each own dims j, j+8, ...; keys stream through LDS in tiles of 32 with
// an online softmax. Query i sits at position start + i and sees keys <= it
// (GqaMask::Causal, gqa.rs:80-86).
constexpr int kPqPerBlock = 32, kPkTile = 32, kPdPerLane = kMaxHeadDim / 8;

__global__ void __launch_bounds__(kBlock) attn_prefill_kernel(AttnPrefillArgs a) {
  extern __shared__ float psm[];
  const int d = a.head_dim;
  float *k_s = psm;                   // [tile][d]
  float *v_s = psm + kPkTile * d;     // [tile][d]
  const int h = blockIdx.x, g = h / (a.nq / a.nkv);
  const int tid = threadIdx.x, qi = blockIdx.y * kPqPerBlock + (tid >> 3), j = tid & 7;
  const bool active = qi < a.M;
  const int qpos = a.start_pos + (active ? qi : a.M - 1);
  const int last_pos = a.start_pos + min(a.M - 1, (int)(blockIdx.y + 1) * kPqPerBlock - 1);
  const float scale = 1.0f / sqrtf((float)d);
  const int qd = a.nq * d;
  float q[kPdPerLane], o[kPdPerLane];
#pragma unroll
  for (int e = 0; e < kPdPerLane; e++) {
    const int dd = j + e * 8;
    q[e] = (active && dd < d) ? a.q[(size_t)qi * qd + h * d + dd] : 0.f;
    o[e] = 0.f;
  }
  float mx = -INFINITY, l = 0.f;
  for (int t0 = 0; t0 <= last_pos; t0 += kPkTile) {
    const int nt = min(kPkTile, last_pos + 1 - t0);
    __syncthreads();
    const size_t kv0 = ((size_t)g * a.max_seq + t0) * d;
    for (int i = tid; i < nt * d; i += kBlock) {
      k_s[i] = load_kv(a.kc, kv0 + i, a.kv_bf16);
      v_s[i] = load_kv(a.vc, kv0 + i, a.kv_bf16);
    }
    __syncthreads();
    for (int t = 0; t < nt; t++) {
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < kPdPerLane; e++) {
        const int dd = j + e * 8;
        if (dd < d) s = fmaf(q[e], k_s[t * d + dd], s);
      }
      s = group_sum<8>(s) * scale;
      if (t0 + t <= qpos) {
        const float mnew = fmaxf(mx, s);
        const float corr = expf(mx - mnew);
        const float p = expf(s - mnew);
        l = l * corr + p;
#pragma unroll
        for (int e = 0; e < kPdPerLane; e++) {
          const int dd = j + e * 8;
          if (dd < d) o[e] = fmaf(p, v_s[t * d + dd], o[e] * corr);
        }
        mx = mnew;
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int e = 0; e < kPdPerLane; e++) {
    const int dd = j + e * 8;
    if (dd < d) {
      const size_t idx = (size_t)qi * qd + h * d + dd;
      split2(o[e] / l, a.out_hi + idx, a.out_lo + idx);
    }
  }
}

__global__ void permute_rows_kernel(uint16_t *dst, const uint16_t *src, const int *perm,
                                    int cols) {
  const int r = blockIdx.x;
  const uint16_t *s = src + (size_t)perm[r] * cols;
  uint16_t *o = dst + (size_t)r * cols;
  for (int j = threadIdx.x; j < cols; j += blockDim.x) o[j] = s[j];
}

// dst[c][r] = src[r][c] for a [rows, cols] matrix of 32-bit words, 32x32 tiles
// through LDS (one-time layout change at load)
__global__ void transpose_u32_kernel(uint32_t *dst, const uint32_t *src, int rows, int cols) {
  __shared__ uint32_t t[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: 8 rows a pass
  for (int y = ty; y < 32; y += 8) {
    const int r = r0 + y, c = c0 + tx;
    if (r < rows && c < cols) t[y][tx] = src[(size_t)r * cols + c];
  }
  __syncthreads();
  for (int y = ty; y < 32; y += 8) {
    const int c = c0 + y, r = r0 + tx;
    if (r < rows && c < cols) dst[(size_t)c * rows + r] = t[tx][y];
  }
}

// Causal prefill attention for head_dim D in {32, 64, 128}: workgroup = (query
// head, 16 queries) x KG key groups, 8 lanes per query each own D / 8 adjacent
// dims; keys and values stream through LDS in tiles of 32. Per tile all 32
// scores are formed first, then the running max, the rescale of the partial
// output and the probabilities (one online-softmax step per tile). Key group
// kg takes tiles kg, kg + KG, ... of the visible keys, each group into its own
// LDS tile, so a short prompt's few workgroups walk 1 / KG of the tiles one
// after another; the groups' (max, sum, output) states then merge through LDS
// in a fixed order. Query i sits at position start + i and sees keys <= it
// (GqaMask::Causal, gqa.rs:80-86).
constexpr int kTq = 16, kTk = 32;
template <int D, int KG>
__global__ void __launch_bounds__(kTq * 8 * KG) attn_prefill_tiled_kernel(AttnPrefillArgs a) {
  constexpr int DL = D / 8, NTG = kTq * 8;
  extern __shared__ float4 attn_sm[];
  const int tid = threadIdx.x, kg = tid / NTG, gt = tid - kg * NTG;
  float *k_s = (float *)attn_sm + kg * 2 * kTk * D;
  float *v_s = k_s + kTk * D;
  const int h = blockIdx.x, g = h / (a.nq / a.nkv);
  const int qi = blockIdx.y * kTq + (gt >> 3), j = gt & 7;
  const bool active = qi < a.M;
  const int qpos = a.start_pos + (active ? qi : a.M - 1);
  const int last_pos = a.start_pos + min(a.M - 1, (int)(blockIdx.y + 1) * kTq - 1);
  const float scale = 1.0f / sqrtf((float)D);
  const int qd = a.nq * D;
  float q[DL], o[DL];
#pragma unroll
  for (int e = 0; e < DL; e++) {
    q[e] = active ? a.q[(size_t)qi * qd + h * D + j * DL + e] : 0.f;
    o[e] = 0.f;
  }
  float mx = -INFINITY, l = 0.f;
  // every group runs the same rounds (the barriers), a group past the
  // visible keys idles
  for (int r0 = 0; r0 <= last_pos; r0 += KG * kTk) {
    const int t0 = r0 + kg * kTk;
    const int nt = max(0, min(kTk, last_pos + 1 - t0));
    __syncthreads();
    // the tile's K and V rows, 4 floats per load
    const size_t kv0 = ((size_t)g * a.max_seq + t0) * D;
    for (int i = gt * 4; i < nt * D; i += NTG * 4) {
      float4 kv, vv;
      if (a.kv_bf16) {
        const uint2 kb = *(const uint2 *)((const uint16_t *)a.kc + kv0 + i);
        const uint2 vb = *(const uint2 *)((const uint16_t *)a.vc + kv0 + i);
        kv = make_float4(bf_lo(kb.x), bf_hi(kb.x), bf_lo(kb.y), bf_hi(kb.y));
        vv = make_float4(bf_lo(vb.x), bf_hi(vb.x), bf_lo(vb.y), bf_hi(vb.y));
      } else {
        kv = *(const float4 *)((const float *)a.kc + kv0 + i);
        vv = *(const float4 *)((const float *)a.vc + kv0 + i);
      }
      *(float4 *)(k_s + i) = kv;
      *(float4 *)(v_s + i) = vv;
    }
    __syncthreads();
    if (nt == 0) continue;
    float sc[kTk];
    float tmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < kTk; t++) {
      float s = 0.f;
      if (t < nt) {
        const float *kr = k_s + t * D + j * DL;
#pragma unroll
        for (int e = 0; e < DL; e++) s = fmaf(q[e], kr[e], s);
      }
      s = group_sum<8>(s) * scale;
      sc[t] = (t < nt && t0 + t <= qpos) ? s : -INFINITY;
      tmax = fmaxf(tmax, sc[t]);
    }
    const float mnew = fmaxf(mx, tmax);
    if (mnew == -INFINITY) continue;  // nothing visible yet
    const float corr = expf(mx - mnew);
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < DL; e++) o[e] *= corr;
#pragma unroll
    for (int t = 0; t < kTk; t++) {
      const float p = expf(sc[t] - mnew);  // masked: exp(-inf) = 0
      psum += p;
      if (t < nt) {
        const float *vr = v_s + t * D + j * DL;
#pragma unroll
        for (int e = 0; e < DL; e++) o[e] = fmaf(p, vr[e], o[e]);
      }
    }
    l = l * corr + psum;
    mx = mnew;
  }
  if (KG > 1) {
    // merge: group 0 combines the KG states of its query in group order
    __syncthreads();
    float *mo = (float *)attn_sm;                 // [KG][NTG][DL] outputs
    float *ml = mo + KG * NTG * DL;               // [KG][NTG] (max, sum)
    if (kg > 0) {
#pragma unroll
      for (int e = 0; e < DL; e++) mo[(kg * NTG + gt) * DL + e] = o[e];
      ml[2 * (kg * NTG + gt)] = mx;
      ml[2 * (kg * NTG + gt) + 1] = l;
    }
    __syncthreads();
    if (kg > 0) return;
    float M = mx;
#pragma unroll
    for (int k = 1; k < KG; k++) M = fmaxf(M, ml[2 * (k * NTG + gt)]);
    // every query sees key 0, so M is finite
    const float c0 = expf(mx - M);
    l *= c0;
#pragma unroll
    for (int e = 0; e < DL; e++) o[e] *= c0;
#pragma unroll
    for (int k = 1; k < KG; k++) {
      const float mk = ml[2 * (k * NTG + gt)];
      const float ck = mk == -INFINITY ? 0.f : expf(mk - M);
      l = fmaf(ml[2 * (k * NTG + gt) + 1], ck, l);
#pragma unroll
      for (int e = 0; e < DL; e++) o[e] = fmaf(mo[(k * NTG + gt) * DL + e], ck, o[e]);
    }
  }
  if (!active) return;
#pragma unroll
  for (int e = 0; e < DL; e++) {
    const size_t idx = (size_t)qi * qd + h * D + j * DL + e;
    split2(o[e] / l, a.out_hi + idx, a.out_lo + idx);
  }
}

// Causal prefill attention on MFMA, head_dim 128 (v_mfma_f32_32x32x16_bf16).
// Workgroup = (query head h, 128 queries): four waves of 32 queries; the
// head's key/value rows stream through LDS in blocks of 32 keys (two stages,
// the next block loaded into registers while the current one is multiplied).
// Per block and wave:
//   S^T = K Q^T (32 keys x 32 queries, 8 steps over the head dims): lane l
//     then holds 16 scores of query l % 32 (keys 8 (i / 4) + 4 (l / 32) +
//     i % 4), so a query's max and sum over the block are its lane's 16
//     values and one exchange with lane l ^ 32;
//   O^T += V^T P^T (4 tiles of 32 dims, 2 steps over the keys): the B
//     operand is the lane's own probabilities, because V^T sits in LDS with
//     each 16-key step's keys in the order the S^T layout hands them out
//     (position 8 half + 4 (j / 4) + j % 4 holds key 8 (j / 4) + 4 half +
//     j % 4), and the lane's O^T column is its own query, so the online
//     softmax rescale is lane-local.
// f32 operands enter as bf16 hi + lo pairs, three products each (hi hi,
// lo hi, hi lo), about 16 significant bits, accumulated in f32. Query i sits
// at position start + i and sees keys <= it (GqaMask::Causal, gqa.rs:80-86).
constexpr int kFaQ = 128, kFaK = 32, kFaD = 128;
constexpr int kFaStage = 4 * kFaK * kFaD * 2;  // K hi, K lo, V^T hi, V^T lo (bf16)
constexpr int kFaLds = 2 * kFaStage + kFaK * kFaD * 4;  // + the f32 V staging tile

// Two workgroups per CU (80 KB of LDS each): the bound caps the kernel at 256
// registers a lane (248 VGPRs, no spills), where it otherwise took 340 and fit
// one wave per SIMD; one workgroup's MFMAs then overlap the other's staging
// and barriers.
__global__ void __launch_bounds__(256, 2) attn_prefill_mfma_kernel(AttnPrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t fa_sm[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Workgroups start in linear grid order (x fastest). A query block's work
  // grows with its index under the causal mask, so linear id w takes query
  // block nqb - 1 - w / (heads * splits) and, within it, head w % heads and
  // key split (w / heads) % splits: the longest workgroups start first and
  // the short ones fill the tail.
  const int nh = gridDim.x, nqb = gridDim.y, ns = gridDim.z;
  const int w = blockIdx.x + nh * (blockIdx.y + nqb * blockIdx.z);
  const int rem = w % (nh * ns), h = rem % nh, zs = rem / nh;
  const int g = h / (a.nq / a.nkv);
  const int q0 = (nqb - 1 - w / (nh * ns)) * kFaQ;
  const int qi = q0 + wave * 32 + (lane & 31);  // this lane's query
  const bool active = qi < a.M;
  const int qpos = a.start_pos + (active ? qi : a.M - 1);
  const int last_pos = a.start_pos + min(a.M - 1, q0 + kFaQ - 1);  // the workgroup's last query
  const int wave_last = a.start_pos + min(a.M - 1, q0 + wave * 32 + 31);
  // key split z of gridDim.z takes key blocks [b0, b1) of the query block's
  // blocks [0, last_pos / kFaK]; with more than one split the workgroup writes
  // f32 partials (o, max, sum) for attn_prefill_merge_kernel
  const int nball = last_pos / kFaK + 1, bps = (nball + ns - 1) / ns;
  const int b0 = min(zs * bps, nball), nblk = min(b0 + bps, nball);
  // scores scaled by log2(e) / sqrt(d): the softmax runs on exp2
  const float scale2 = 1.4426950408889634f / sqrtf((float)kFaD);
  const int qd = a.nq * kFaD;

  // Q^T operand of the score MFMA: lane l, step ks -> query l % 32, dims
  // 16 ks + 8 (l / 32) .. + 7
  bf16x8 qh[8], ql[8];
  {
    const float *qrow = a.q + (size_t)(active ? qi : a.M - 1) * qd + h * kFaD + 8 * (lane >> 5);
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
      const float4 x0 = *(const float4 *)(qrow + 16 * ks), x1 = *(const float4 *)(qrow + 16 * ks + 4);
      const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const __bf16 hb = (__bf16)v[e];
        qh[ks][e] = hb;
        ql[ks][e] = (__bf16)(v[e] - (float)hb);
      }
    }
  }

  // block loader: thread t takes key t / 8 of the block, dims (t % 8) 16 .. + 15.
  // Buffer loads: a block past this split's range reads at byte offset 2^31,
  // out of the descriptor's range (zeros, no traffic), so the pipeline's
  // look-ahead loads cost nothing there and every load is still issued.
  const int lkey = tid >> 3, ldim = (tid & 7) * 16;
  const uint32_t kvbytes = (uint32_t)((size_t)a.nkv * a.max_seq * kFaD * (a.kv_bf16 ? 2 : 4));
  const __amdgpu_buffer_rsrc_t rkc =
      __builtin_amdgcn_make_buffer_rsrc((void *)a.kc, (short)0, (int)kvbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rvc =
      __builtin_amdgcn_make_buffer_rsrc((void *)a.vc, (short)0, (int)kvbytes, 0x00020000);
  float kr[16], vr[16];
  auto gload = [&](int b) {
    const int kpos = min(b * kFaK + lkey, last_pos);
    const size_t base = ((size_t)g * a.max_seq + kpos) * kFaD + ldim;
    const uint32_t esz = a.kv_bf16 ? 2u : 4u;
    const int boff = b < nblk ? (int)(base * esz) : (int)0x80000000u;
    if (a.kv_bf16) {
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const u32x4 kb = __builtin_amdgcn_raw_buffer_load_b128(rkc, boff, 16 * u, 0);
        const u32x4 vb = __builtin_amdgcn_raw_buffer_load_b128(rvc, boff, 16 * u, 0);
        const uint32_t kw[4] = {kb.x, kb.y, kb.z, kb.w}, vw[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          kr[8 * u + 2 * e] = bf_lo(kw[e]);
          kr[8 * u + 2 * e + 1] = bf_hi(kw[e]);
          vr[8 * u + 2 * e] = bf_lo(vw[e]);
          vr[8 * u + 2 * e + 1] = bf_hi(vw[e]);
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const u32x4 k4 = __builtin_amdgcn_raw_buffer_load_b128(rkc, boff, 16 * u, 0);
        const u32x4 v4 = __builtin_amdgcn_raw_buffer_load_b128(rvc, boff, 16 * u, 0);
        kr[4 * u] = __uint_as_float(k4.x); kr[4 * u + 1] = __uint_as_float(k4.y);
        kr[4 * u + 2] = __uint_as_float(k4.z); kr[4 * u + 3] = __uint_as_float(k4.w);
        vr[4 * u] = __uint_as_float(v4.x); vr[4 * u + 1] = __uint_as_float(v4.y);
        vr[4 * u + 2] = __uint_as_float(v4.z); vr[4 * u + 3] = __uint_as_float(v4.w);
      }
    }
  };
  // K rows: 256 B (16 chunks of 8 dims), chunk c at slot c ^ (key & 15).
  // V goes through an f32 row-major staging tile (float4 stores), then each
  // thread gathers 16 keys of one dim from it (lanes on consecutive dims, no
  // bank conflicts) into two 8-key octets of the V^T row.
  // V^T rows: 64 B (4 octets of keys), octet o at slot o ^ ((dim >> 2) & 3).
  float *vstage = (float *)(fa_sm + 2 * kFaStage);  // [kFaK][kFaD] f32
  auto sstore_k = [&](int st) {
    uint8_t *kh = fa_sm + st * kFaStage, *kl = kh + kFaK * kFaD * 2;
#pragma unroll
    for (int u = 0; u < 2; u++) {
      bf16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float v = kr[8 * u + e];
        const __bf16 hb = (__bf16)v;
        hi[e] = hb;
        lo[e] = (__bf16)(v - (float)hb);
      }
      const int c = (ldim >> 3) + u, off = lkey * 256 + ((c ^ (lkey & 15)) << 4);
      *(bf16x8 *)(kh + off) = hi;
      *(bf16x8 *)(kl + off) = lo;
    }
#pragma unroll
    for (int u = 0; u < 4; u++)
      *(float4 *)(vstage + lkey * kFaD + ldim + 4 * u) =
          make_float4(vr[4 * u], vr[4 * u + 1], vr[4 * u + 2], vr[4 * u + 3]);
  };
  // thread t: dim t / 2, key step t & 1 (keys 16 s .. 16 s + 15); octet 0 of
  // the step holds keys {0..3, 8..11}, octet 1 keys {4..7, 12..15}
  auto sstore_vt = [&](int st) {
    uint8_t *vh = fa_sm + st * kFaStage + 2 * kFaK * kFaD * 2, *vl = vh + kFaK * kFaD * 2;
    const int dim = tid >> 1, s2 = tid & 1;
#pragma unroll
    for (int oc = 0; oc < 2; oc++) {
      bf16x8 hi, lo;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int key = 16 * s2 + 8 * (j >> 2) + 4 * oc + (j & 3);
        const float v = vstage[key * kFaD + dim];
        const __bf16 hb = (__bf16)v;
        hi[j] = hb;
        lo[j] = (__bf16)(v - (float)hb);
      }
      const int off = dim * 64 + (((2 * s2 + oc) ^ ((dim >> 2) & 3)) << 4);
      *(bf16x8 *)(vh + off) = hi;
      *(bf16x8 *)(vl + off) = lo;
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int n = 0; n < 4; n++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[n][e] = 0.f;
  float mx = -INFINITY, l = 0.f;

  gload(b0);
  sstore_k(0);
  gload(b0 + 1);
  __syncthreads();
  sstore_vt(0);
  __syncthreads();
  for (int b = b0; b < nblk; b++) {
    const int st = (b - b0) & 1;
    const int kb = b * kFaK;
    if (kb <= wave_last) {  // some query of the wave sees a key of the block
      const uint8_t *kh = fa_sm + st * kFaStage, *kl = kh + kFaK * kFaD * 2;
      const uint8_t *vh = kl + kFaK * kFaD * 2, *vl = vh + kFaK * kFaD * 2;
      // three independent chains (hi hi, lo hi, hi lo) keep the MFMA pipe busy
      f32x16 s0, s1, s2;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        s0[e] = 0.f;
        s1[e] = 0.f;
        s2[e] = 0.f;
      }
      const int krow = (lane & 31) * 256;
#pragma unroll
      for (int ks = 0; ks < 8; ks++) {
        const int c = 2 * ks + (lane >> 5), off = krow + ((c ^ (lane & 15)) << 4);
        const bf16x8 ah = *(const bf16x8 *)(kh + off), al = *(const bf16x8 *)(kl + off);
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, qh[ks], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, qh[ks], s1, 0, 0, 0);
        s2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, ql[ks], s2, 0, 0, 0);
      }
      // scores in the base-2 domain: s log2(e) / sqrt(d), masked; block max
      float sc[16];
      float bm = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int key = kb + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        sc[i] = key <= qpos ? ((s0[i] + s1[i]) + s2[i]) * scale2 : -INFINITY;
        bm = fmaxf(bm, sc[i]);
      }
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float mnew = fmaxf(mx, bm);
      float p[16];
      float ps = 0.f;
      if (mnew != -INFINITY) {
        const float corr = __builtin_amdgcn_exp2f(mx - mnew);  // mx = -inf: 0
#pragma unroll
        for (int i = 0; i < 16; i++) {
          p[i] = __builtin_amdgcn_exp2f(sc[i] - mnew);  // masked: 2^-inf = 0
          ps += p[i];
        }
        ps += __shfl_xor(ps, 32, 64);
        l = l * corr + ps;
        mx = mnew;
        // the accumulators leave the matrix registers only when some query of
        // the wave raised its max
        if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
          for (int n = 0; n < 4; n++)
#pragma unroll
            for (int e = 0; e < 16; e++) o[n][e] *= corr;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; i++) p[i] = 0.f;
      }
      // P^T operand for key step s2: the lane's probabilities 8 s2 .. 8 s2 + 7
#pragma unroll
      for (int s2 = 0; s2 < 2; s2++) {
        bf16x8 ph, pl;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float v = p[8 * s2 + e];
          const __bf16 hb = (__bf16)v;
          ph[e] = hb;
          pl[e] = (__bf16)(v - (float)hb);
        }
        const int oct = 2 * s2 + (lane >> 5);
#pragma unroll
        for (int n = 0; n < 4; n++) {
          const int dim = 32 * n + (lane & 31);
          const int off = dim * 64 + ((oct ^ ((dim >> 2) & 3)) << 4);
          const bf16x8 vah = *(const bf16x8 *)(vh + off), val = *(const bf16x8 *)(vl + off);
          o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vah, ph, o[n], 0, 0, 0);
          o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(val, ph, o[n], 0, 0, 0);
          o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vah, pl, o[n], 0, 0, 0);
        }
      }
    }
    // block b + 1 into the other stage (its last readers passed the previous
    // barrier); the V staging tile is free again after each transpose's barrier
    if (b + 1 < nblk) sstore_k(st ^ 1);
    gload(b + 2);  // always issued (clamped past the last block)
    __syncthreads();
    if (b + 1 < nblk) {
      sstore_vt(st ^ 1);
      __syncthreads();
    }
  }
  // O^T tile n: lane l holds dims 32 n + 8 (i / 4) + 4 (l / 32) + i % 4 of
  // its query. The normalised rows go to LDS (the stages are free after the
  // last barrier), then each lane writes 8 consecutive dims of one query as
  // 16-byte hi / lo stores.
  float *orow = (float *)fa_sm + wave * 32 * (kFaD + 4);  // [32][d + 4] f32 per wave
  const float inv = ns > 1 ? 1.0f : 1.0f / l;
#pragma unroll
  for (int n = 0; n < 4; n++)
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int dim = 32 * n + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
      orow[(lane & 31) * (kFaD + 4) + dim] = o[n][i] * inv;
    }
  __syncthreads();
  if (ns > 1) {
    // partial [h][z][query]: o (unnormalised, relative to the max) then (max, sum)
    float *pbase = a.part + ((size_t)h * ns + zs) * a.M * (kFaD + 2);
    if (lane < 32 && active) {
      pbase[(size_t)qi * (kFaD + 2) + kFaD] = mx;
      pbase[(size_t)qi * (kFaD + 2) + kFaD + 1] = l;
    }
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const int qq = r * 4 + (lane >> 4), c8 = (lane & 15) * 8;
      const int qrow = q0 + wave * 32 + qq;
      if (qrow < a.M) {
        const float *src = orow + qq * (kFaD + 4) + c8;
        float *dst = pbase + (size_t)qrow * (kFaD + 2) + c8;  // 8-byte aligned: d + 2 is even
#pragma unroll
        for (int e = 0; e < 8; e += 2) *(float2 *)(dst + e) = *(const float2 *)(src + e);
      }
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 8; r++) {
    const int qq = r * 4 + (lane >> 4), c8 = (lane & 15) * 8;  // query of the wave, dims c8 .. + 7
    const int qrow = q0 + wave * 32 + qq;
    if (qrow < a.M) {
      const float *src = orow + qq * (kFaD + 4) + c8;
      const float4 x0 = *(const float4 *)src, x1 = *(const float4 *)(src + 4);
      const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      bf16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const __bf16 hb = (__bf16)v[e];
        hi[e] = hb;
        lo[e] = (__bf16)(v[e] - (float)hb);
      }
      const size_t idx = (size_t)qrow * qd + h * kFaD + c8;
      *(bf16x8 *)(a.out_hi + idx) = hi;
      *(bf16x8 *)(a.out_lo + idx) = lo;
    }
  }
}

// The key splits of attn_prefill_mfma_kernel merged in split order: thread t
// takes 4 dims of one (query, head); out = sum_z 2^(m_z - M) o_z /
// sum_z 2^(m_z - M) l_z with M = max_z m_z, as bf16 hi / lo planes.
__global__ void __launch_bounds__(256) attn_prefill_merge_kernel(AttnPrefillArgs a, int ns) {
  const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t nvec = (size_t)a.M * a.nq * (kFaD / 4);
  if (t >= nvec) return;
  const int d4 = (int)(t % (kFaD / 4));
  const size_t qh = t / (kFaD / 4);
  const int h = (int)(qh % a.nq), q = (int)(qh / a.nq);
  const size_t zs = (size_t)a.M * (kFaD + 2);  // one split's partials of a head
  const float *p = a.part + (size_t)h * ns * zs + (size_t)q * (kFaD + 2);
  // every split's (max, sum) and outputs in one round trip (ns <= 4); the
  // loads are unconditional (split min(z, ns - 1) for z >= ns, unused): a
  // load under a branch would be waited for where the branch joins
  float2 ml[4], x0[4], x1[4];
#pragma unroll
  for (int z = 0; z < 4; z++) {
    const float *pz = p + min(z, ns - 1) * zs;
    ml[z] = *(const float2 *)(pz + kFaD);
    x0[z] = *(const float2 *)(pz + 4 * d4);
    x1[z] = *(const float2 *)(pz + 4 * d4 + 2);
  }
  float mmax = -INFINITY;
#pragma unroll
  for (int z = 0; z < 4; z++)
    if (z < ns) mmax = fmaxf(mmax, ml[z].x);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float lsum = 0.f;
#pragma unroll
  for (int z = 0; z < 4; z++) {
    if (z < ns) {
      const float e = ml[z].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[z].x - mmax);
      lsum = fmaf(e, ml[z].y, lsum);
      acc.x = fmaf(e, x0[z].x, acc.x);
      acc.y = fmaf(e, x0[z].y, acc.y);
      acc.z = fmaf(e, x1[z].x, acc.z);
      acc.w = fmaf(e, x1[z].y, acc.w);
    }
  }
  const float inv = 1.0f / lsum;
  const float v[4] = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
  uint16_t hi[4], lo[4];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const __bf16 hb = (__bf16)v[e];
    hi[e] = __builtin_bit_cast(uint16_t, hb);
    lo[e] = __builtin_bit_cast(uint16_t, (__bf16)(v[e] - (float)hb));
  }
  const size_t idx = (size_t)q * a.nq * kFaD + h * kFaD + 4 * d4;
  *(uint2 *)(a.out_hi + idx) = make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
  *(uint2 *)(a.out_lo + idx) = make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
}

// Causal prefill attention for short prompts (head_dim 128, at most 128
// queries, at most 256 keys): workgroup (q head h, 32 queries), wave w takes
// key blocks w, w + 4, ... of the queries' causal range. A key block is used
// by one wave only, so its K and V go straight from the cache into MFMA
// operand registers, with no LDS staging and no barrier per block:
//   S^T = K Q^T as in attn_prefill_mfma_kernel (lane l holds key l % 32,
//     dims 16 ks + 8 (l / 32) .. + 7 of the block as the A operand);
//   O^T += V^T P^T with the lane's own probabilities as the B operand: its
//     probability j of key step s belongs to key 16 s + 8 (j / 4) +
//     4 (l / 32) + j % 4, so the A operand holds V[that key][32 n + l % 32]
//     (each load a 128-byte row segment per half-wave).
// Each wave keeps an online softmax over its blocks (scores in base 2); the
// waves' (max, sum, unnormalised o) are merged through LDS in wave order,
// out = sum_w 2^(m_w - M) o_w / sum_w 2^(m_w - M) l_w, and written as bf16
// hi / lo planes. One launch, no partials in global memory, and Q is read
// once per wave: at 128 ids the key-split kernel's four splits each pulled
// their block's 64 KB of Q and left a merge launch behind them. A wave
// issues its block's K and V loads together, so the V round trip overlaps
// the score MFMAs (that alone took the 128-id prefill 2.65 -> 2.59 ms).
constexpr int kFsQ = 32;
constexpr int kFsLds = (4 * kFsQ * (kFaD + 4) + 4 * kFsQ * 2) * (int)sizeof(float);

// KB: the cache holds bf16 (else f32). A compile-time choice: under a run-time
// flag every V load sat behind its own branch and was waited for where the
// branch joined, 64 round trips in a row per key block.
template <bool KB>
__global__ void __launch_bounds__(256) attn_prefill_small_kernel(AttnPrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t fs_sm[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x, g = h / (a.nq / a.nkv);
  const int q0 = blockIdx.y * kFsQ;
  const int qi = q0 + (lane & 31);  // this lane's query
  const bool active = qi < a.M;
  const int qpos = a.start_pos + (active ? qi : a.M - 1);
  const int last_pos = a.start_pos + min(a.M - 1, q0 + kFsQ - 1);  // the workgroup's last query
  const int nball = last_pos / kFaK + 1;
  const float scale2 = 1.4426950408889634f / sqrtf((float)kFaD);
  const int qd = a.nq * kFaD;

  // Q^T operand: lane l, step ks -> query l % 32, dims 16 ks + 8 (l / 32) .. + 7
  bf16x8 qh[8], ql[8];
  {
    const float *qrow = a.q + (size_t)(active ? qi : a.M - 1) * qd + h * kFaD + 8 * (lane >> 5);
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
      const float4 x0 = *(const float4 *)(qrow + 16 * ks), x1 = *(const float4 *)(qrow + 16 * ks + 4);
      const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const __bf16 hb = (__bf16)v[e];
        qh[ks][e] = hb;
        ql[ks][e] = (__bf16)(v[e] - (float)hb);
      }
    }
  }
  // 8 consecutive cached values from element offset i (f32 or bf16 cache)
  auto kv8 = [&](const void *base, size_t i, float *v) {
    if constexpr (KB) {
      const uint4 w = *(const uint4 *)((const uint16_t *)base + i);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[2 * e] = bf_lo(ww[e]);
        v[2 * e + 1] = bf_hi(ww[e]);
      }
    } else {
      const float4 x0 = *(const float4 *)((const float *)base + i), x1 = *(const float4 *)((const float *)base + i + 4);
      v[0] = x0.x, v[1] = x0.y, v[2] = x0.z, v[3] = x0.w, v[4] = x1.x, v[5] = x1.y, v[6] = x1.z, v[7] = x1.w;
    }
  };
  auto kv1 = [&](const void *base, size_t i) {
    if constexpr (KB)
      return bf16f(((const uint16_t *)base)[i]);
    else
      return ((const float *)base)[i];
  };
  const size_t head_base = (size_t)g * a.max_seq * kFaD;

  f32x16 o[4];
#pragma unroll
  for (int n = 0; n < 4; n++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[n][e] = 0.f;
  float mx = -INFINITY, l = 0.f;

  for (int b = wave; b < nball; b += 4) {
    const int kb = b * kFaK;
    // K rows past the last query are read at the last query's row (in range;
    // their scores are masked)
    const int kpos = min(kb + (lane & 31), last_pos);
    f32x16 s0, s1, s2;
#pragma unroll
    for (int e = 0; e < 16; e++) {
      s0[e] = 0.f;
      s1[e] = 0.f;
      s2[e] = 0.f;
    }
    float kv[8][8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) kv8(a.kc, head_base + (size_t)kpos * kFaD + 16 * ks + 8 * (lane >> 5), kv[ks]);
    // the block's V operand values, loaded with K so that their round trip
    // overlaps the score MFMAs; keys past the last query read as zero (their
    // probabilities are zero too)
    float vv[2][4][8];
#pragma unroll
    for (int s2i = 0; s2i < 2; s2i++)
#pragma unroll
      for (int n = 0; n < 4; n++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int key = kb + 16 * s2i + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
          const float x = kv1(a.vc, head_base + (size_t)min(key, last_pos) * kFaD + 32 * n + (lane & 31));
          vv[s2i][n][j] = key <= last_pos ? x : 0.f;
        }
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
      bf16x8 kh, kl;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const __bf16 hb = (__bf16)kv[ks][e];
        kh[e] = hb;
        kl[e] = (__bf16)(kv[ks][e] - (float)hb);
      }
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qh[ks], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl, qh[ks], s1, 0, 0, 0);
      s2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, ql[ks], s2, 0, 0, 0);
    }
    float sc[16];
    float bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int key = kb + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
      sc[i] = key <= qpos ? ((s0[i] + s1[i]) + s2[i]) * scale2 : -INFINITY;
      bm = fmaxf(bm, sc[i]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mnew = fmaxf(mx, bm);
    float p[16];
    if (mnew != -INFINITY) {
      const float corr = __builtin_amdgcn_exp2f(mx - mnew);  // mx = -inf: 0
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        p[i] = __builtin_amdgcn_exp2f(sc[i] - mnew);  // masked: 2^-inf = 0
        ps += p[i];
      }
      ps += __shfl_xor(ps, 32, 64);
      l = l * corr + ps;
      mx = mnew;
#pragma unroll
      for (int n = 0; n < 4; n++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[n][e] *= corr;
    } else {
#pragma unroll
      for (int i = 0; i < 16; i++) p[i] = 0.f;
    }
#pragma unroll
    for (int s2i = 0; s2i < 2; s2i++) {
      bf16x8 ph, pl;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float v = p[8 * s2i + e];
        const __bf16 hb = (__bf16)v;
        ph[e] = hb;
        pl[e] = (__bf16)(v - (float)hb);
      }
#pragma unroll
      for (int n = 0; n < 4; n++) {
        bf16x8 vah, val;
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const float x = vv[s2i][n][j];
          const __bf16 hb = (__bf16)x;
          vah[j] = hb;
          val[j] = (__bf16)(x - (float)hb);
        }
        o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vah, ph, o[n], 0, 0, 0);
        o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(val, ph, o[n], 0, 0, 0);
        o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vah, pl, o[n], 0, 0, 0);
      }
    }
  }

  // merge the waves: o^T tile n, lane l holds dims 32 n + 8 (i / 4) +
  // 4 (l / 32) + i % 4 of query l % 32
  float *om = (float *)fs_sm;                  // [wave][query][kFaD + 4]
  float *mlp = om + 4 * kFsQ * (kFaD + 4);     // [wave][query][2]
#pragma unroll
  for (int n = 0; n < 4; n++)
#pragma unroll
    for (int i = 0; i < 16; i++)
      om[(wave * kFsQ + (lane & 31)) * (kFaD + 4) + 32 * n + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)] = o[n][i];
  if (lane < 32) {
    mlp[(wave * kFsQ + lane) * 2] = mx;
    mlp[(wave * kFsQ + lane) * 2 + 1] = l;
  }
  __syncthreads();
  // thread t: query t / 8, dims 16 (t % 8) .. + 15
  const int qq = tid >> 3, d0 = (tid & 7) * 16;
  float mw[4], lw[4], mall = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; w++) {
    mw[w] = mlp[(w * kFsQ + qq) * 2];
    lw[w] = mlp[(w * kFsQ + qq) * 2 + 1];
    mall = fmaxf(mall, mw[w]);
  }
  float ew[4], lsum = 0.f;
#pragma unroll
  for (int w = 0; w < 4; w++) {
    ew[w] = mw[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw[w] - mall);
    lsum = fmaf(ew[w], lw[w], lsum);
  }
  const float inv = 1.0f / lsum;
  const int qrow = q0 + qq;
  if (qrow < a.M) {
#pragma unroll
    for (int half = 0; half < 2; half++) {
      bf16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int d = d0 + 8 * half + e;
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) acc = fmaf(ew[w], om[(w * kFsQ + qq) * (kFaD + 4) + d], acc);
        const float v = acc * inv;
        const __bf16 hb = (__bf16)v;
        hi[e] = hb;
        lo[e] = (__bf16)(v - (float)hb);
      }
      const size_t idx = (size_t)qrow * qd + h * kFaD + d0 + 8 * half;
      *(bf16x8 *)(a.out_hi + idx) = hi;
      *(bf16x8 *)(a.out_lo + idx) = lo;
    }
  }
}

inline unsigned nblk(size_t n, unsigned b) { return (unsigned)((n + b - 1) / b); }
constexpr long kCUsGemv = 256;

}  // namespace

// ============================================================ launchers ====

namespace {
// dynamic LDS of a GEMV launch: x (k floats, rounded to 4)
size_t stage_bytes(const GemvArgs &a, int) { return (size_t)((a.k + 3) & ~3) * sizeof(float); }

template <int TEAM, int ROWS, int CPT, int XM, int EPI>
hipError_t go_gemv(const GemvArgs &a, hipStream_t s, int *nparts) {
  const int rows_per_block = ROWS * (kBlock / TEAM);
  const unsigned grid = nblk((size_t)a.m, rows_per_block);
  if (nparts) *nparts = (int)grid;
  if (EPI == EPI_HEAD && (int)grid > a.part_cap) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemv_kernel<TEAM, ROWS, CPT, XM, EPI>), dim3(grid), dim3(kBlock),
                     stage_bytes(a, XM), s, a);
  return hipGetLastError();
}

template <int XM, int EPI>
hipError_t go_gemv_generic(const GemvArgs &a, hipStream_t s, int *nparts) {
  const unsigned grid = nblk((size_t)a.m, 8);
  if (nparts) *nparts = (int)grid;
  if (EPI == EPI_HEAD && (int)grid > a.part_cap) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemv_generic_kernel<XM, EPI>), dim3(grid), dim3(kBlock),
                     stage_bytes(a, XM), s, a);
  return hipGetLastError();
}

// Streaming launch plan: each workgroup takes a contiguous range of whole
// batches. Taken for rows of >= 2048 columns in matrices of >= 32M weights
// (measured on MI355X with the weights streamed from HBM: 3584 x 18944
// 37.6 -> 31.5 us, 152064 x 3584 179 -> 169 us, 37888 x 3584 51.4 -> 50.5
// us); smaller matrices and k = 1536 rows are faster one-shot (151936 x
// 1536: 71.9 one-shot, 79.3 streaming).
struct StreamPlan {
  int team = 0, rb = 0, cpt = 0, grid = 0, rows_per_wg = 0;
};
int g_gemv_force = -1;  // -1 planner, 0 one-shot only, 1 streaming where it applies
static StreamPlan stream_plan(int m, int k) {
  StreamPlan p;
  if (g_gemv_force == 0 || k % 8 != 0 || k < 8 || k > 24576 || m < 512) return p;
  if (g_gemv_force < 0 && (k < 2048 || (size_t)m * k < (32u << 20))) return p;
  // a workgroup team per row batch; measured best on MI355X: rows of <= 512
  // chunks two at a time with ~4 workgroups per CU (37888 x 3584: 46.7 us),
  // longer rows one at a time with 2 per CU (3584 x 18944: 29.9 us)
  const int nch = k / 8;
  p.team = 256;
  long cap;
  if (nch <= 512) {
    p.cpt = (nch + 255) / 256;
    p.rb = 2;
    cap = 4 * kCUsGemv;
  } else {
    const int c = (nch + 255) / 256;
    p.cpt = c <= 5 ? 5 : c <= 10 ? 10 : 12;
    p.rb = 1;
    cap = 2 * kCUsGemv;
  }
  const long batches = (m + p.rb - 1) / p.rb;
  const long wgs = std::min<long>(cap, batches);
  const long per = (batches + wgs - 1) / wgs;  // batches per workgroup
  p.rows_per_wg = (int)(per * p.rb);
  p.grid = (int)((m + p.rows_per_wg - 1) / p.rows_per_wg);
  return p;
}

template <int TEAM, int RB, int CPT, int XM, int EPI>
hipError_t go_stream(const GemvArgs &a, const StreamPlan &p, hipStream_t s, int *nparts) {
  if (nparts) *nparts = p.grid;
  if (EPI == EPI_HEAD && p.grid > a.part_cap) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemv_stream_kernel<TEAM, RB, CPT, XM, EPI>), dim3(p.grid), dim3(kBlock),
                     stage_bytes(a, XM), s, a, p.rows_per_wg);
  return hipGetLastError();
}

template <int XM, int EPI>
hipError_t pick_stream(const GemvArgs &a, const StreamPlan &p, hipStream_t s, int *nparts) {
  switch (p.cpt) {
    case 1: return go_stream<256, 2, 1, XM, EPI>(a, p, s, nparts);
    case 2: return go_stream<256, 2, 2, XM, EPI>(a, p, s, nparts);
    case 5: return go_stream<256, 1, 5, XM, EPI>(a, p, s, nparts);
    case 10: return go_stream<256, 1, 10, XM, EPI>(a, p, s, nparts);
    default: return go_stream<256, 1, 12, XM, EPI>(a, p, s, nparts);
  }
}

// Variant choice: rows per team grow with m (more independent loads in flight
// per lane); a wavefront team while one wave's chunks cover the row in <= 8
// steps, else the whole workgroup splits the row (k up to 24576).
template <int XM, int EPI>
hipError_t pick_gemv(const GemvArgs &a, hipStream_t s, int *nparts) {
  const int nch = a.k / 8;
  const bool vec = (a.k % 8) == 0 && a.k >= 8 && ((uintptr_t)a.w % 16) == 0 &&
                   ((uintptr_t)a.x % 16) == 0 && (XM == X_PLAIN || ((uintptr_t)a.gamma % 8) == 0);
  if (!vec || a.k > 24576) return go_gemv_generic<XM, EPI>(a, s, nparts);
  const StreamPlan p = stream_plan(a.m, a.k);
  if (p.grid > 0) return pick_stream<XM, EPI>(a, p, s, nparts);
  const bool big = a.m >= 16384;
  if (nch <= 64 * 8) {
    const int cpt = (nch + 63) / 64;
#define WAVE_CASE(C)                                                                     \
  case C:                                                                                \
    return big ? go_gemv<64, 4, C, XM, EPI>(a, s, nparts) : go_gemv<64, 2, C, XM, EPI>(a, s, nparts);
    switch (cpt) {
      WAVE_CASE(1)
      WAVE_CASE(2)
      WAVE_CASE(3)
      WAVE_CASE(4)
      case 5:
      WAVE_CASE(6)
      case 7:
      WAVE_CASE(8)
      default:
        break;
    }
#undef WAVE_CASE
  }
  const int cpt = (nch + 255) / 256;
  if (cpt <= 3) return go_gemv<256, 2, 3, XM, EPI>(a, s, nparts);
  if (cpt <= 5) return go_gemv<256, 2, 5, XM, EPI>(a, s, nparts);
  if (cpt <= 8) return go_gemv<256, 2, 8, XM, EPI>(a, s, nparts);
  if (cpt <= 10) return go_gemv<256, 2, 10, XM, EPI>(a, s, nparts);
  return go_gemv<256, 2, 12, XM, EPI>(a, s, nparts);
}
}  // namespace

hipError_t launch_gemv(const GemvArgs &a, GemvX xm, GemvEpi epi, hipStream_t s, int *nparts) {
  if (a.m <= 0) return hipSuccess;
  if (xm == X_PLAIN && epi == EPI_STORE) return pick_gemv<X_PLAIN, EPI_STORE>(a, s, nparts);
  if (xm == X_PLAIN && epi == EPI_RESID) return pick_gemv<X_PLAIN, EPI_RESID>(a, s, nparts);
  if (xm == X_NORM && epi == EPI_QKV) return pick_gemv<X_NORM, EPI_QKV>(a, s, nparts);
  if (xm == X_PLAIN && epi == EPI_QKV) return pick_gemv<X_PLAIN, EPI_QKV>(a, s, nparts);
  if (xm == X_NORM && epi == EPI_GU) return pick_gemv<X_NORM, EPI_GU>(a, s, nparts);
  if (xm == X_NORM && epi == EPI_HEAD) return pick_gemv<X_NORM, EPI_HEAD>(a, s, nparts);
  return hipErrorInvalidValue;
}

int gemv_head_parts(int m, int k) {
  const int nch = k / 8;
  if (k % 8 != 0 || k < 8 || k > 24576) return (int)nblk((size_t)m, 8);
  const StreamPlan p = stream_plan(m, k);
  if (p.grid > 0) return p.grid;
  const bool big = m >= 16384;
  if (nch <= 64 * 8) return (int)nblk((size_t)m, big ? 16 : 8);
  return (int)nblk((size_t)m, 2);
}

int attn_decode_chunks(int max_seq, int head_dim) {
  return (max_seq + attn_chunk(head_dim) - 1) / attn_chunk(head_dim);
}

size_t attn_decode_part_floats(int nq, int max_seq, int head_dim) {
  return (size_t)nq * attn_decode_chunks(max_seq, head_dim) * ((size_t)head_dim + 2);
}

hipError_t launch_attn_decode(const AttnDecodeArgs &a, hipStream_t s) {
  const int gq = a.nq / a.nkv, d = a.head_dim;
  if (gq > kMaxQPerKv || d > kMaxHeadDim) return hipErrorInvalidValue;
  const int ch = attn_chunk(d), nchunks = attn_decode_chunks(a.max_seq, d);
  const size_t merge = sizeof(float) * 2 * (size_t)gq * nchunks;  // the merge's (m, l) table
  dim3 grid(a.nkv, nchunks);
  if (d == 128) {
    const size_t smem = std::max(merge, sizeof(float) * (4 * 2 * kMaxQPerKv * 128 + kMaxQPerKv * 34));
    if (smem > 65536) return hipErrorInvalidValue;
    if (a.kv_bf16)
      hipLaunchKernelGGL(attn_decode_d128_kernel<true>, grid, dim3(kBlock), smem, s, a);
    else
      hipLaunchKernelGGL(attn_decode_d128_kernel<false>, grid, dim3(kBlock), smem, s, a);
    return hipGetLastError();
  }
  const size_t smem = std::max(merge, sizeof(float) * ((size_t)gq * d + (size_t)ch * (d + 1) +
                                                       (size_t)ch * d + (size_t)gq * ch + 2 * gq));
  if (smem > 65536) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attn_decode_kernel, grid, dim3(kBlock), smem, s, a);
  return hipGetLastError();
}

// The MFMA GEMM multiplies every weight by the activation's bf16 hi and lo
// parts. An infinite weight times a zero lo part is NaN where the
// reference's f32 chain (gemm_bf16.rs:337-378, bit-identical to the per-token
// GEMV) gives +-inf, so a NaN output is recomputed here as that chain: left
// to right from +0, each product rounded before it is added. Outputs that
// are not NaN are left as they are; with finite weights and activations no
// output is NaN and the pass only reads Y.
__global__ void gemm_nan_repair_kernel(float *y, const uint16_t *w, const float *x, int batch, int m, int k) {
  const size_t n = (size_t)batch * m;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    if (!__builtin_isnan(y[i])) continue;
    const size_t b = i / m, r = i - b * m;
    const uint16_t *wr = w + r * k;
    const float *xb = x + b * k;
    float acc = 0.f;
    for (int j = 0; j < k; j++) acc = __fadd_rn(acc, __fmul_rn(bf16f(wr[j]), xb[j]));
    y[i] = acc;
  }
}

hipError_t launch_gemm_nan_repair(float *y, const uint16_t *w, const float *x, int batch, int m, int k,
                                  hipStream_t s) {
  const size_t n = (size_t)batch * m;
  if (!n) return hipSuccess;
  const size_t blocks = std::min<size_t>(nblk(n, 256), 2048);
  hipLaunchKernelGGL(gemm_nan_repair_kernel, dim3((unsigned)blocks), dim3(256), 0, s, y, w, x, batch, m, k);
  return hipGetLastError();
}

hipError_t launch_fill_zero(float *y, size_t n, hipStream_t s) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(nblk(n, 256)), dim3(256), 0, s, y, n);
  return hipGetLastError();
}

hipError_t launch_add_bias(float *y, const uint16_t *b, size_t n, hipStream_t s) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(add_bias_kernel, dim3(nblk(n, 256)), dim3(256), 0, s, y, b, n);
  return hipGetLastError();
}

hipError_t launch_embed_gather(float *out, const uint16_t *table, size_t hidden,
                               const uint32_t *token_dev, uint32_t token_host, hipStream_t s) {
  hipLaunchKernelGGL(embed_gather_kernel, dim3(nblk(hidden, 256) > 64 ? 64 : nblk(hidden, 256)),
                     dim3(256), 0, s, out, table, hidden, token_dev, token_host);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(float *y, const uint16_t *g, const float *x, size_t n, float eps,
                          hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel<uint16_t>, dim3(1), dim3(kBlock), 0, s, y, g, x, n, eps);
  return hipGetLastError();
}

hipError_t launch_rope_apply(float *x, size_t len, size_t head_dim, const float2 *cs,
                             hipStream_t s) {
  hipLaunchKernelGGL(rope_apply_kernel, dim3(nblk(len / 2, 256)), dim3(256), 0, s, x, len,
                     head_dim, cs);
  return hipGetLastError();
}

hipError_t launch_gqa_general(float *y, const float *q, const float *k, const float *v,
                              float *probs, float *scratch, int nq, int nkv, int d, int seq,
                              int mask, size_t query_pos, hipStream_t s) {
  hipLaunchKernelGGL(gqa_general_kernel, dim3(nq), dim3(kBlock), 0, s, y, q, k, v, probs,
                     scratch, nq, nkv, d, seq, mask, (unsigned long long)query_pos);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_f32(float *y, const float *g, const float *x, size_t n, float eps,
                              hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel<float>, dim3(1), dim3(kBlock), 0, s, y, g, x, n, eps);
  return hipGetLastError();
}

hipError_t launch_silu(float *y, const float *z, size_t n, hipStream_t s) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(silu_kernel, dim3(nblk(n, 256)), dim3(256), 0, s, y, z, n);
  return hipGetLastError();
}

hipError_t launch_swiglu_mul(float *h, const float *g, const float *u, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(swiglu_mul_kernel, dim3(nblk(n, 256)), dim3(256), 0, s, h, g, u, n);
  return hipGetLastError();
}

int argmax_parts(size_t n) { return (int)nblk(n, kArgmaxPerBlock); }

hipError_t launch_argmax_partial(const float *logits, size_t n, float2 *part, hipStream_t s) {
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(argmax_parts(n)), dim3(kBlock), 0, s, logits, n,
                     part);
  return hipGetLastError();
}

hipError_t launch_argmax_final(const ArgmaxFinalArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_embed_rows(float *X, const uint16_t *embed, const uint32_t *tokens, int M,
                             int H, hipStream_t s) {
  hipLaunchKernelGGL(embed_rows_kernel, dim3(M), dim3(256), 0, s, X, embed, tokens, H);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rows_split(const float *X, const uint16_t *g, float eps, int M, int H,
                                     uint16_t *hi, uint16_t *lo, hipStream_t s) {
  const int n4 = H >> 2;
  const bool vec = (H & 3) == 0 && n4 <= 4 * kBlock && ((uintptr_t)X & 15) == 0 &&
                   (((uintptr_t)g | (uintptr_t)hi | (uintptr_t)lo) & 7) == 0;
  if (!vec)
    hipLaunchKernelGGL(rmsnorm_rows_split_kernel, dim3(M), dim3(kBlock), 0, s, X, g, eps, H, hi, lo);
  else if (n4 <= kBlock)
    hipLaunchKernelGGL(rmsnorm_rows_split4_kernel<1>, dim3(M), dim3(kBlock), 0, s, X, g, eps, H, hi, lo);
  else if (n4 <= 2 * kBlock)
    hipLaunchKernelGGL(rmsnorm_rows_split4_kernel<2>, dim3(M), dim3(kBlock), 0, s, X, g, eps, H, hi, lo);
  else
    hipLaunchKernelGGL(rmsnorm_rows_split4_kernel<4>, dim3(M), dim3(kBlock), 0, s, X, g, eps, H, hi, lo);
  return hipGetLastError();
}

hipError_t launch_split_rows(const float *X, size_t n, uint16_t *hi, uint16_t *lo,
                             hipStream_t s) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(split_kernel, dim3(nblk(n, 256)), dim3(256), 0, s, X, n, hi, lo);
  return hipGetLastError();
}

// ---- GEMM launch plans ------------------------------------------------------
// The pipelined kernel's tile shapes (M x N): 128 x 32, 128 x 64, 128 x 128,
// 128 x 256. Wider tiles read fewer A bytes per weight byte (the A tile is
// re-read by every N tile) and fewer LDS bytes per MFMA; narrower ones give
// more workgroups when N is small.
using PfT32 = PfCfg<1, 1, 4, 1>;
using PfT64 = PfCfg<1, 2, 4, 1>;
using PfT128 = PfCfg<2, 2, 2, 2>;
using PfT256 = PfCfg<2, 4, 2, 2>;
// 128 x 256 with eight waves (two per SIMD, 64 x 64 each): one wave's MFMAs
// run while the other waits on LDS, which the four-wave 128 x 256 tile cannot
using PfW256 = PfCfg<2, 2, 2, 4>;
// 128 x 192 with eight waves (32 x 96 each): 8 N tiles of a 1536-wide
// projection, so 16 M tiles x 2 splits fill the 256 CUs exactly
using PfW192 = PfCfg<1, 3, 4, 2>;
// Short prompts (at most 128 rows): 64-row tiles halve the activation bytes
// each workgroup pulls per weight byte. 64 x 64 with four waves for the
// narrow projections, 64 x 128 with eight waves for gate/up.
using PfS64 = PfCfg<1, 1, 2, 2>;
using PfS128 = PfCfg<1, 1, 2, 4>;
// 64 x 160 with ten waves: a 17920-row gate/up at 65-128 rows is 224
// workgroups, one round over the CUs, where the 64 x 128 tile's 280 put two
// workgroups on 24 CUs
using PfS160 = PfCfg<1, 1, 2, 5>;
// 128 x 128 with eight waves (32 x 64 each): over 256 rows it takes the
// 128 x 128 plans of the cost model (qkv 40.0 -> 32.4 us, o 38.0 -> 29.9 at
// 2048 rows of the 1.5B shape)
using PfW128 = PfCfg<1, 2, 4, 2>;
constexpr int kPfCfgs = 10;
constexpr int kPfPlanCfgs = 4;  // the cost model's candidates (the others are picked by shape)
constexpr int kPfBN[kPfCfgs] = {PfT32::BN, PfT64::BN, PfT128::BN, PfT256::BN, PfW256::BN, PfW192::BN, PfS64::BN, PfS128::BN,
                                PfS160::BN, PfW128::BN};
constexpr int kCUs = 256;

int g_force_cfg = -1, g_force_splits = 0;

// Tile shape and K splits for the pipelined kernel, from a cost model fitted
// to measurements of this kernel on MI355X over the prefill shapes (1.5B and
// 7B projections at 128 and 2048 rows). A workgroup is bound by what its CU
// can pull from L2: about 64 outstanding 128-byte L2 requests at ~520 cycles
// each, 14 B/clk, so a 64-wide K stage costs (A hi/lo 128 x 256 B + W
// BN x 128 B) / 14 clocks; workgroups beyond one per CU run in further
// rounds; K splits add their f32 partials written and read back at ~2 TB/s
// and a reduction launch. Wider tiles re-read the A tile fewer times per
// weight byte; split K fills the CUs when N has few tiles.
GemmPlan pf_plan(int M, int N, int K) {
  GemmPlan best;
  if (K <= 0 || (K & 63) || M <= 0 || N <= 0) return best;
  if (g_force_cfg >= 0) {
    best.cfg = g_force_cfg;
    best.splits = g_force_splits > 0 ? std::min(g_force_splits, K >> 6) : 1;
    return best;
  }
  // Wide, short-K projections (gate/up: N >= 8192 rows of K <= 4096), and
  // long-K ones (down) over many rows, take the eight-wave 128 x 256 tile.
  // Measured per launch with the split reduction, weights from HBM (1.5B
  // shapes): gate/up at 128 rows 48.3 us on the single-stage 128 x 64 kernel
  // -> 45.4 (three splits), at 2048 rows 380 -> 326; down at 2048 rows 175
  // (128 x 256, four waves, two splits) -> 140. The small projections and
  // down at 128 rows stay on the cost model's choice (the eight-wave tiles
  // measured no better there).
  // Up to 128 rows, measured per launch with the split reduction (1.5B
  // shapes, weights from HBM): gate/up without a split on the 64 x 160
  // ten-wave tile where its grid fits one round (34.2 -> 26.7 us at 128
  // rows), else on the 64 x 128 eight-wave tile (29.1 -> 23.5 us at 64 rows,
  // 26.1 -> 19.7 at 32); where that grid would exceed ~1.25 rounds (the 7B
  // gate/up, 592 workgroups) the 128 x 256 tile stays ahead.
  if (N >= 8192 && K <= 4096) {
    const long mt64 = (M + 63) / 64;
    if (M > 64 && M <= 128 && mt64 * ((N + 159) / 160) <= kCUs) {
      best.cfg = 8;
      best.splits = 1;
      return best;
    }
    if (M <= 128 && mt64 * ((N + 127) / 128) <= 320) {
      best.cfg = 7;
      best.splits = 1;
      return best;
    }
    // (the 7B gate/up at 128 rows: 110.8 us with three splits, 107.5 with none)
    best.cfg = 4;
    best.splits = M > 128 && M <= 256 ? std::min(3, K >> 6) : 1;
    return best;
  }
  // The other projections at up to 128 rows, except long-K ones wider than
  // 2048 (the 7B down keeps the cost model's plan): a 64-row tile split so
  // the grid fills one round over the CUs, the 64 x 64 four-wave tile or the
  // 64 x 128 eight-wave one, whichever comes closer to 256 workgroups (the
  // 64 x 64 on a tie). At 128 rows qkv 12.7 -> 11.0 us, o 11.6 -> 10.1,
  // down 21.9 -> 19.7 (1.5B); 7B qkv 26.3 -> 22.6 (64 x 128, 3 splits), 7B
  // o 21.5 -> 19.6 (64 x 64, 2 splits); at 32-64 rows qkv and o 1.8-3 us
  // faster.
  if (M <= 128 && (N <= 2048 || K <= 4096)) {
    const long mt64 = (M + 63) / 64;
    auto fill = [&](int bn, int *sp) {
      const long tiles = mt64 * ((N + bn - 1) / bn);
      *sp = (int)std::max(1L, std::min<long>({kCUs / tiles, 16L, (long)(K >> 6)}));
      return tiles * *sp;
    };
    int s64 = 1, s128 = 1;
    const long w64 = fill(64, &s64), w128 = fill(128, &s128);
    if (w128 > w64 && w128 <= kCUs) {
      best.cfg = 7;
      best.splits = s128;
    } else {
      best.cfg = 6;
      best.splits = s64;
    }
    return best;
  }
  if (M > 256 && N <= 4096 && K >= 4096) {
    // the 128 x 192 tile when its two-split grid fits the CUs in one round
    // (down at 2048 rows: 256 workgroups, 139 -> 121 us against 192 of the
    // 128 x 256 tile)
    const long t192 = ((M + 127) / 128) * (long)(N / 192);
    best.cfg = N % 192 == 0 && 2 * t192 <= kCUs ? 5 : 4;
    best.splits = 2;
    return best;
  }
  const int nks = K >> 6;
  const long mt = (M + 127) / 128;
  double best_t = 1e30;
  for (int c = 0; c < kPfPlanCfgs; c++) {
    const long tiles = mt * ((N + kPfBN[c] - 1) / kPfBN[c]);
    const double stage = (32768.0 + 128.0 * kPfBN[c]) / 14.0;  // clocks per K stage
    for (int sp = 1; sp <= std::min(nks, 64); sp++) {
      const long rounds = (tiles * sp + kCUs - 1) / kCUs;
      const int kst = (nks + sp - 1) / sp;
      double t = rounds * (kst * stage + 1500.0) / 2400.0;  // us at 2.4 GHz
      if (sp > 1) t += 2.0 * sp * (double)M * N * 4.0 / 2.0e6 + 1.0;
      if (t < best_t - 1e-9) {
        best_t = t;
        best.cfg = c;
        best.splits = sp;
      }
    }
  }
  if (M > 256 && best.cfg == 2) best.cfg = 9;  // the eight-wave 128 x 128 tile
  return best;
}

void gemm_force_plan(int cfg, int splits) {
  g_force_cfg = cfg;
  g_force_splits = splits;
}

// the pipelined kernel takes the shape: K stages of 64, 16-byte aligned
// operands, 32-bit buffer ranges
static bool pf_ok(const GemmArgs &a) {
  return a.K > 0 && (a.K & 63) == 0 && a.M > 0 && a.N > 0 &&
         (((uintptr_t)a.a_hi | (uintptr_t)a.a_lo | (uintptr_t)a.w) & 15) == 0 &&
         (size_t)a.M * a.K * 2 < (1ull << 31) && (size_t)a.N * a.K * 2 < (1ull << 31);
}

int gemm_splits_old(int M, int N, int K) {
  const int tiles = (int)(nblk((size_t)N, GBN) * nblk((size_t)M, GBM));
  const int ksteps = (K + GBK - 1) / GBK;
  // about two workgroups per CU, so one's operand loads overlap the other's
  // MFMAs (measured at M = 128: one per CU 4 % slower, three 11 % slower)
  int sp = (512 + tiles - 1) / tiles;
  // partials (sp M N f32) no larger than the weights (N K bf16)
  if (sp > K / (2 * M)) sp = K / (2 * M);
  if (sp > ksteps) sp = ksteps;
  if (sp < 1) sp = 1;
  const int kps = (ksteps + sp - 1) / sp;
  return (ksteps + kps - 1) / kps;
}

// Gate/up over many rows on the 128 x 256 tile: when the tiles fill some
// rounds over the CUs and leave a partial round of at most half the CUs, the
// N tiles that fill whole rounds run in one launch (returned: that many N
// tiles) and the rest in a tail launch on 128 x 128 tiles, at most one round.
// 2048 rows of the 1.5B gate/up: 1120 tiles = 4.375 rounds, 243 us ->
// 1024 tiles (203-207 us), then 192 128 x 128 tiles (30 us), bit-identical.
// (The tail as 96 x 2 half-K tiles took 28 us and their reduction 7.5.)
// 0: one launch.
static int gu_tail_plan(int M, int N, int K) {
  static_assert(PfW256::BN % PfW128::BN == 0 && PfW256::BM == PfW128::BM, "tail tiles split the wide ones");
  if (g_force_cfg >= 0 || K <= 0 || (K & 63) || M <= 0 || N % PfW256::BN) return 0;
  const GemmPlan p = pf_plan(M, N, K);
  if (p.cfg != 4 || p.splits != 1) return 0;
  const long mt = (M + PfW256::BM - 1) / PfW256::BM, nt = N / PfW256::BN, tiles = mt * nt;
  if (tiles <= kCUs || tiles % kCUs == 0) return 0;
  const long nm = tiles / kCUs * kCUs / mt, tail = mt * (nt - nm);
  return nm >= 1 && 2 * tail <= kCUs ? (int)nm : 0;
}

size_t gemm_ws_floats(int M, int N, int K) {
  const GemmPlan p = pf_plan(M, N, K);
  const int sp = std::max(p.cfg >= 0 ? p.splits : 1, gemm_splits_old(M, N, K));
  return sp > 1 ? (size_t)sp * M * N : 0;
}

// the fallback kernel's launch shape: K splits (1 when the partial buffer is
// short) and K steps per split in a.kps
static int gemm_plan_old(GemmArgs &a) {
  const int ksteps = (a.K + GBK - 1) / GBK;
  int splits = gemm_splits_old(a.M, a.N, a.K);
  if (!a.ws || a.ws_cap < (size_t)splits * a.M * a.N) splits = 1;  // no room for partials
  a.kps = (ksteps + splits - 1) / splits;
  if (a.kps < 1) a.kps = 1;
  return splits;
}

// gx > 0: a grid gx tiles wide (the first gx tiles of N, or with TAIL the
// last gx)
template <class C, int EPI, bool TAIL = false>
static hipError_t go_pf(const GemmArgs &a, int splits, hipStream_t s, int gx = 0) {
  static bool attr_done = false;
  const void *fn = (const void *)gemm_pf_kernel<C, EPI, TAIL>;
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
    if (e != hipSuccess) return e;
    attr_done = true;
  }
  dim3 grid(gx > 0 ? (unsigned)gx : nblk((size_t)a.N, C::BN), nblk((size_t)a.M, C::BM), splits);
  GemmArgs args = a;
  void *params[] = {&args};
  return hipLaunchKernel(fn, grid, dim3(C::NTH), params, C::LDS, s);
}

template <int EPI>
static hipError_t go_pf_cfg(const GemmArgs &a, int cfg, int splits, hipStream_t s) {
  switch (cfg) {
    case 0: return go_pf<PfT32, EPI>(a, splits, s);
    case 1: return go_pf<PfT64, EPI>(a, splits, s);
    case 2: return go_pf<PfT128, EPI>(a, splits, s);
    case 3: return go_pf<PfT256, EPI>(a, splits, s);
    case 4: return go_pf<PfW256, EPI>(a, splits, s);
    case 5: return go_pf<PfW192, EPI>(a, splits, s);
    case 6: return go_pf<PfS64, EPI>(a, splits, s);
    case 7: return go_pf<PfS128, EPI>(a, splits, s);
    case 8: return go_pf<PfS160, EPI>(a, splits, s);
    case 9: return go_pf<PfW128, EPI>(a, splits, s);
    default: return hipErrorInvalidValue;
  }
}

// Launch the GEMM (partials into a.ws when split) with epilogue EPI, or with
// EPI_STORE into the partials; returns the split count used in *splits_out.
template <int EPI>
static hipError_t gemm_main(GemmArgs &a, hipStream_t s, int *splits_out) {
  const GemmPlan p = pf_plan(a.M, a.N, a.K);
  if (p.cfg >= 0 && p.cfg < kPfCfgs && pf_ok(a) &&
      (p.splits == 1 || (a.ws && a.ws_cap >= (size_t)p.splits * a.M * a.N))) {
    *splits_out = p.splits;
    return go_pf_cfg<EPI>(a, p.cfg, p.splits, s);
  }
  const int splits = gemm_plan_old(a);
  *splits_out = splits;
  dim3 grid(nblk((size_t)a.N, GBN), nblk((size_t)a.M, GBM), splits);
  hipLaunchKernelGGL(gemm_mfma_kernel<EPI>, grid, dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gemm_resid_norm(const GemmArgs &args, const uint16_t *g, float eps,
                                  uint16_t *hi, uint16_t *lo, hipStream_t s) {
  if (args.M <= 0 || args.N <= 0) return hipSuccess;
  GemmArgs a = args;
  const int n4 = a.N >> 2;
  const bool can_fuse = (a.N & 3) == 0 && n4 <= 4 * kBlock &&
                        (((uintptr_t)a.ws | (uintptr_t)a.y) & 15) == 0 &&
                        (((uintptr_t)g | (uintptr_t)hi | (uintptr_t)lo) & 7) == 0;
  int splits = 1;
  hipError_t e = gemm_main<EPI_RESID>(a, s, &splits);
  if (e != hipSuccess) return e;
  if (splits == 1 || !can_fuse) {
    if (splits > 1) {  // plain split reduction into y, then the norm
      const unsigned rgrid = nblk((size_t)a.M * ((a.N + 1) >> 1), kBlock);
      hipLaunchKernelGGL(gemm_reduce_kernel<EPI_RESID>, dim3(rgrid), dim3(kBlock), 0, s, a, splits);
    }
    return launch_rmsnorm_rows_split(a.y, g, eps, a.M, a.N, hi, lo, s);
  }
  if (n4 <= kBlock)
    hipLaunchKernelGGL(gemm_resid_norm_kernel<1>, dim3(a.M), dim3(kBlock), 0, s, a, splits, g, eps, hi, lo);
  else if (n4 <= 2 * kBlock)
    hipLaunchKernelGGL(gemm_resid_norm_kernel<2>, dim3(a.M), dim3(kBlock), 0, s, a, splits, g, eps, hi, lo);
  else
    hipLaunchKernelGGL(gemm_resid_norm_kernel<4>, dim3(a.M), dim3(kBlock), 0, s, a, splits, g, eps, hi, lo);
  return hipGetLastError();
}

template <int EPI>
static hipError_t launch_gemm_epi(const GemmArgs &args, hipStream_t s) {
  GemmArgs a = args;
  if constexpr (EPI == EPI_GU) {
    const int nm = gu_tail_plan(a.M, a.N, a.K);
    if (nm > 0 && pf_ok(a)) {
      hipError_t e = go_pf<PfW256, EPI_GU>(a, 1, s, nm);
      if (e != hipSuccess) return e;
      return go_pf<PfW128, EPI_GU, true>(a, 1, s, (a.N - nm * PfW256::BN) / PfW128::BN);
    }
  }
  int splits = 1;
  hipError_t e = gemm_main<EPI>(a, s, &splits);
  if (e != hipSuccess || splits == 1) return e;
  const bool r4 = (a.N & 3) == 0 && ((uintptr_t)a.ws & 15) == 0;
  if (r4) {
    const unsigned rgrid4 = nblk((size_t)a.M * (a.N >> 2), kBlock);
    hipLaunchKernelGGL(gemm_reduce4_kernel<EPI>, dim3(rgrid4), dim3(kBlock), 0, s, a, splits);
  } else {
    const unsigned rgrid = nblk((size_t)a.M * ((a.N + 1) >> 1), kBlock);
    hipLaunchKernelGGL(gemm_reduce_kernel<EPI>, dim3(rgrid), dim3(kBlock), 0, s, a, splits);
  }
  return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs &args, GemvEpi epi, hipStream_t s) {
  if (args.M <= 0 || args.N <= 0) return hipSuccess;
  switch (epi) {
    case EPI_STORE: return launch_gemm_epi<EPI_STORE>(args, s);
    case EPI_RESID: return launch_gemm_epi<EPI_RESID>(args, s);
    case EPI_GU: return launch_gemm_epi<EPI_GU>(args, s);
    case EPI_QKV: return launch_gemm_epi<EPI_QKV>(args, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_attn_prefill(const AttnPrefillArgs &a, hipStream_t s) {
  if (a.head_dim > kMaxHeadDim) return hipErrorInvalidValue;
  // the MFMA kernel's buffer loads address the layer's cache with 32-bit
  // offsets and use 2^31 as the out-of-range offset
  const size_t kv_bytes = (size_t)a.nkv * a.max_seq * a.head_dim * (a.kv_bf16 ? 2 : 4);
  if (a.head_dim == kFaD && a.nq % a.nkv == 0 && a.M > kFsQ && a.M <= 128 && a.start_pos + a.M <= 256) {
    // short prompts: one launch, a key block per wave. Measured per prefill
    // (1.5B shape, same box): 128 ids 2.70 -> 2.59 ms, 64 ids 2.19 -> 2.13;
    // at 32 ids or fewer a single wave would carry all the keys, and the
    // key-split kernel, whose four waves stage each block together, stays
    // ahead (1.86 against 1.88 ms)
    static bool small_attr[2] = {false, false};
    const int kb = a.kv_bf16 ? 1 : 0;
    const void *fn = kb ? (const void *)attn_prefill_small_kernel<true> : (const void *)attn_prefill_small_kernel<false>;
    if (!small_attr[kb]) {
      hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kFsLds);
      if (e != hipSuccess) return e;
      small_attr[kb] = true;
    }
    AttnPrefillArgs args = a;
    void *params[] = {&args};
    return hipLaunchKernel(fn, dim3(a.nq, (unsigned)nblk((size_t)a.M, kFsQ)), dim3(256), params, kFsLds, s);
  }
  if (a.head_dim == kFaD && a.nq % a.nkv == 0 && kv_bytes < (size_t(1) << 31)) {
    static bool attr_done = false;
    const void *fn = (const void *)attn_prefill_mfma_kernel;
    if (!attr_done) {
      hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kFaLds);
      if (e != hipSuccess) return e;
      attr_done = true;
    }
    AttnPrefillArgs args = a;
    void *params[] = {&args};
    // fewer query-block workgroups than twice the CUs: split each block's keys
    // four ways (when the workspace holds the partials)
    const int nqb = (int)nblk((size_t)a.M, kFaQ);
    const int nb_max = (a.start_pos + a.M - 1) / kFaK + 1;
    int ns = a.nq * nqb < 512 ? std::min(4, nb_max) : 1;
    if (ns > 1 && (!a.part || attn_prefill_part_floats(a.nq, a.M, ns) > a.part_cap)) ns = 1;
    hipError_t e = hipLaunchKernel(fn, dim3(a.nq, nqb, ns), dim3(256), params, kFaLds, s);
    if (e != hipSuccess || ns == 1) return e;
    const size_t nvec = (size_t)a.M * a.nq * (kFaD / 4);
    hipLaunchKernelGGL(attn_prefill_merge_kernel, dim3((unsigned)((nvec + 255) / 256)), dim3(256), 0, s,
                       args, ns);
    return hipGetLastError();
  }
  // 16-byte tile loads: the cache rows and q must be aligned to 4 elements
  if (a.head_dim == 128 || a.head_dim == 64 || a.head_dim == 32) {
    dim3 tg(a.nq, nblk((size_t)a.M, kTq));
    // fewer workgroups than CUs: four key groups per workgroup
    const bool split = tg.x * tg.y < 256;
    const size_t smem = (split ? 4 : 1) * 2 * kTk * a.head_dim * sizeof(float);
    const void *fn;
    switch (a.head_dim) {
      case 128:
        fn = split ? (const void *)attn_prefill_tiled_kernel<128, 4>
                   : (const void *)attn_prefill_tiled_kernel<128, 1>;
        break;
      case 64:
        fn = split ? (const void *)attn_prefill_tiled_kernel<64, 4>
                   : (const void *)attn_prefill_tiled_kernel<64, 1>;
        break;
      default:
        fn = split ? (const void *)attn_prefill_tiled_kernel<32, 4>
                   : (const void *)attn_prefill_tiled_kernel<32, 1>;
        break;
    }
    if (smem >= 64 * 1024) {  // the 4-group d = 64 and d = 128 instantiations
      static bool attr_done[2] = {false, false};
      bool &done = attr_done[a.head_dim == 128];
      if (!done) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        done = true;
      }
    }
    AttnPrefillArgs args = a;
    void *params[] = {&args};
    return hipLaunchKernel(fn, tg, dim3(kTq * 8 * (split ? 4 : 1)), params, smem, s);
  }
  dim3 grid(a.nq, nblk((size_t)a.M, kPqPerBlock));
  const size_t smem = sizeof(float) * 2 * kPkTile * a.head_dim;
  hipLaunchKernelGGL(attn_prefill_kernel, grid, dim3(kBlock), smem, s, a);
  return hipGetLastError();
}

hipError_t launch_permute_rows(uint16_t *dst, const uint16_t *src, const int *perm, int rows,
                               int cols, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(permute_rows_kernel, dim3(rows), dim3(256), 0, s, dst, src, perm, cols);
  return hipGetLastError();
}

hipError_t launch_transpose_u32(uint32_t *dst, const uint32_t *src, int rows, int cols,
                                hipStream_t s) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  hipLaunchKernelGGL(transpose_u32_kernel, dim3(nblk(cols, 32), nblk(rows, 32)), dim3(256), 0, s,
                     dst, src, rows, cols);
  return hipGetLastError();
}

const char *kernel_build_info() {
  return "gfx950; gemv: wave/workgroup teams, 16B nontemporal bf16 loads, fused "
         "rmsnorm/bias+rope+kv/swiglu/residual/argmax epilogues; attention: split-position "
         "decode partials merged by the last chunk workgroup of each kv group; streaming GEMV for "
         "large projections; prefill: v_mfma_f32_32x32x16_bf16 hi/lo GEMM, LDS-pipelined, planned tiles";
}

}  // namespace myos
