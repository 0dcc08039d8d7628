// Persistent greedy-decode kernel for MI355X (gfx950).
//
// One cooperative launch of 256 workgroups (one per CU, 512 threads) runs a
// whole run of decode steps. Every workgroup owns fixed rows of the QKV, o,
// gate/up and head projections and a fixed slice of the residual stream; a
// gate/up owner also owns the down columns of its h values, so down runs as
// per-workgroup partial sums that the residual-row owners add up. Attention
// work items (kv head, 32-position chunk) are dealt round robin. Activations cross workgroups as 64-bit words (value, tag), stored and
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

#include <algorithm>
#include <math.h>
#include <stdint.h>

#include "myos_internal.h"

namespace myos {
namespace {

constexpr int NT = 512;              // threads per workgroup
constexpr int NW = NT / 64;          // wavefronts per workgroup
constexpr int NB = 256;              // workgroups (one per CU)
constexpr int HC = 3;                // 8-column chunks per lane, k <= 1536
constexpr int MAXI = 9216;           // intermediate limit
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
constexpr uint32_t P_QKV = 0, P_PART = 1, P_XO = 2, P_PD = 3, P_XD = 4, P_ATT = 5;
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

// tgather for src[0, n) in order: one buffer descriptor, one lane offset and
// per-unroll constant offsets keep the address cost at one register. The
// loads are sc1 (device-coherent) and volatile, so a spin re-reads memory.
// A wait that starts before its producers have published would otherwise
// re-read all U words per spin from every workgroup at once, which costs
// bandwidth the weight stream needs: each thread first spins on its last
// word alone, then reads the rest once, re-reading only words still untagged.
template <int U, class Put>
__device__ bool tgather_lin_to(const uint64_t *src, int n, uint32_t tag, Put put,
                               const PersistArgs &a, int *fail) {
  constexpr int kAux = 16 | (1 << 31);  // sc1, volatile
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, n * 8, 0x00020000);
  bool ok = *fail == 0;
  for (int i0 = threadIdx.x; i0 < n && ok; i0 += NT * U) {
    const int last = min(U - 1, (n - 1 - i0) / NT);
    for (unsigned spins = 0;; spins++) {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, (i0 + last * NT) * 8, 0, kAux);
      if (v.y == tag) break;
      if (spin_fail(a, spins)) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    uint64_t w[U];
    uint32_t pend = 0;
#pragma unroll
    for (int u = 0; u < U; u++) {
      w[u] = (uint64_t)tag << 32;
      if (i0 + u * NT < n) pend |= 1u << u;
    }
    for (unsigned spins = 0; ok; spins++) {
#pragma unroll
      for (int u = 0; u < U; u++)
        if (pend & (1u << u)) {
          const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, i0 * 8, u * NT * 8, kAux);
          w[u] = ((uint64_t)v.y << 32) | v.x;
        }
#pragma unroll
      for (int u = 0; u < U; u++)
        if ((uint32_t)(w[u] >> 32) == tag) pend &= ~(1u << u);
      if (!pend) break;
      if (spin_fail(a, spins)) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = i0 + u * NT;
      if (i < n) put(i, __uint_as_float((uint32_t)w[u]));
    }
  }
  if (!ok) *fail = 1;
  __syncthreads();
  return *fail == 0;
}

template <int U>
__device__ bool tgather_lin(const uint64_t *src, int n, uint32_t tag, float *dst,
                            const PersistArgs &a, int *fail) {
  return tgather_lin_to<U>(src, n, tag, [dst](int i, float v) { dst[i] = v; }, a, fail);
}

// ---- row tiles -----------------------------------------------------------------
// Weight rows load through a buffer descriptor of the matrix with the row's
// byte offset in a scalar register and one shared lane offset, so no per-row
// 64-bit lane address stays live while a row is in flight.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wrsrc(const uint16_t *W) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)W, (short)0, 0x7fffffff, 0x00020000);
}

// row `row` of a [rows, k] bf16 matrix, 8 columns per chunk, chunk lane + 64 i
// in t[i]; `valid` and `row` are wave-uniform
template <int C>
__device__ __forceinline__ void ldrow(u32x4 (&t)[C], const uint16_t *W, int k, int row, bool valid,
                                      int lane) {
  const int nch = k >> 3;
  const __amdgpu_buffer_rsrc_t rs = wrsrc(W);
  const int soff = valid ? row * k * 2 : 0;
#pragma unroll
  for (int i = 0; i < C; i++) {
    const int c = lane + i * 64;
    const u32x4 zero = {0u, 0u, 0u, 0u};
    t[i] = (valid && c < nch) ? __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16 + i * 1024, soff, 2)
                              : zero;
  }
}

// ldrow with every load issued: the row is clamped to `last` and each lane's
// chunk to the row's last one (dotrow ignores chunks past the row), so the
// number of loads in flight is the same on every path and a wait for an
// older tile can leave the younger ones in flight.
template <int C>
__device__ __forceinline__ void ldrow_all(u32x4 (&t)[C], const uint16_t *W, int k, int row, int last,
                                          int lane) {
  const int nch = k >> 3;
  const __amdgpu_buffer_rsrc_t rs = wrsrc(W);
  const int soff = min(row, last) * k * 2;
#pragma unroll
  for (int i = 0; i < C; i++) {
    const int c = min(lane + i * 64, nch - 1);
    t[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, c * 16, soff, 2);
  }
}

// Part `part` of 3 of a block of the column-pair matrix P (rows of `ld`
// words) streamed into LDS with direct (DMA) loads: rows [j0, j0 + kv),
// columns [c0, c0 + cw) land row-major at dst (word q = row * cw + col), 1 KB
// per wave load, and part p covers loads [p per, (p + 1) per), so a block can
// be spread over several waits. cw % 4 == 0; `dst` is wave-uniform; no
// registers hold the block meanwhile. The compiler waits for these loads
// before the wave's next LDS access.
__device__ __forceinline__ void dma_block(const uint32_t *P, int ld, int j0, int kv, int c0, int cw,
                                          uint8_t *dst, int lane, int part) {
  const int tot = kv * cw, nld = (tot + 255) >> 8, per = (nld + 2) / 3;
  const int i0 = part * per, i1 = min(i0 + per, nld);
  const __amdgpu_buffer_rsrc_t rs = wrsrc((const uint16_t *)P);
  const int soff = (j0 * ld + c0) * 4;
  for (int i = i0; i < i1; i++) {
    const int q = i * 256 + lane * 4;
    if (q < tot) {
      const int row = q / cw, col = q - row * cw;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void *)(dst + i * 1024), 16,
          (row * ld + col) * 4, soff, 0, 2 /* nt */);
    }
  }
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

// Sum over aligned groups of S lanes, S = 8, 16 or 32 (wave-uniform), for N
// values at once: each DPP step runs over all of them, so the steps'
// latencies overlap. For S <= 16 every lane of a group holds its total; for
// S = 32 lanes 16-31 and 48-63 do.
template <int N>
__device__ __forceinline__ void seg_sum_n(float (&v)[N], int S) {
#pragma unroll
  for (int i = 0; i < N; i++) v[i] += dpp<0xB1>(v[i], 0.f);
#pragma unroll
  for (int i = 0; i < N; i++) v[i] += dpp<0x4E>(v[i], 0.f);
#pragma unroll
  for (int i = 0; i < N; i++) v[i] += dpp<0x141>(v[i], 0.f);
  if (S >= 16) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp<0x140>(v[i], 0.f);
  }
  if (S >= 32) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp<0x142, 0xA>(v[i], 0.f);
  }
}
__device__ __forceinline__ bool seg_leader(int lane, int S) {
  return (lane & (S - 1)) == (S == 32 ? 16 : 0);
}
// wave_sum of N values at once (the DPP steps overlap); lane 63 holds the totals
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
  seg_sum_n<N>(v, 32);
#pragma unroll
  for (int i = 0; i < N; i++) v[i] += dpp<0x143, 0xC>(v[i], 0.f);
}

// this lane's chunks of x (chunk lane + 64 i, 8 floats each) in registers,
// read from LDS once for every row a phase multiplies
template <int C>
__device__ __forceinline__ void load_x(float4 (&xr)[C][2], const float *x, int k, int lane) {
  const int nch = k >> 3;
#pragma unroll
  for (int i = 0; i < C; i++) {
    const int c = lane + i * 64;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    xr[i][0] = c < nch ? *(const float4 *)(x + c * 8) : z;
    xr[i][1] = c < nch ? *(const float4 *)(x + c * 8 + 4) : z;
  }
}

// dotrow with x from load_x
template <int C>
__device__ __forceinline__ float dotrow_x(const u32x4 (&t)[C], const float4 (&xr)[C][2], int k,
                                          int lane) {
  const int nch = k >> 3;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < C; i++) {
    const int c = lane + i * 64;
    if (c < nch) {
      const float4 x0 = xr[i][0], x1 = xr[i][1];
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

// ---- normalised x in registers, split for bf16 dot products -------------------
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, x),
                                         acc, false);
}
typedef float f32x2 __attribute__((ext_vector_type(2)));
// (a, b) -> bf16 pair (a low, b high), round to nearest even: one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const f32x2 f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}
// This lane's chunks of x (chunk lane + 64 i, 8 columns each) as bf16 pairs
// x = hi + lo: hi is x rounded to bf16, lo the remainder rounded to bf16, so
// hi + lo carries 16 significant bits of x. A weight pair times (hi + lo) is
// two v_dot2 steps accumulated in f32: half the VALU work of unpacking the
// weights and multiplying in f32.
template <int C>
struct XPairs {
  uint32_t h[C][4], l[C][4];
};

// Wave-local RMSNorm of x (rmsnorm_bf16_weight, crates/tensor_core/src/bf16.rs:
// 231-270, with a tree sum): the wave's lanes hold every column of x (lane +
// 64 i covers all chunks when k <= 512 C), so one wave_sum gives the mean
// square without a barrier. `gw` holds the gains of this lane's chunks.
// Returns the normalised chunks in f32 (xr) and split into pairs (xp).
template <int C>
__device__ __forceinline__ void norm_x(float4 (&xr)[C][2], XPairs<C> &xp, const float *x,
                                       const u32x4 (&gw)[C], int k, float eps, int lane) {
  load_x<C>(xr, x, k, lane);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < C; i++) {
    const float4 a = xr[i][0], b = xr[i][1];
    ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w + b.x * b.x + b.y * b.y + b.z * b.z +
          b.w * b.w;
  }
  const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)k + eps);
#pragma unroll
  for (int i = 0; i < C; i++) {
    float v[8] = {xr[i][0].x, xr[i][0].y, xr[i][0].z, xr[i][0].w,
                  xr[i][1].x, xr[i][1].y, xr[i][1].z, xr[i][1].w};
    const uint32_t g[4] = {gw[i].x, gw[i].y, gw[i].z, gw[i].w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float a = bf_lo(g[j]) * (v[2 * j] * inv), b = bf_hi(g[j]) * (v[2 * j + 1] * inv);
      v[2 * j] = a;
      v[2 * j + 1] = b;
      const uint32_t hp = pack_bf16(a, b);
      xp.h[i][j] = hp;
      xp.l[i][j] = pack_bf16(a - bf_lo(hp), b - bf_hi(hp));
    }
    xr[i][0] = make_float4(v[0], v[1], v[2], v[3]);
    xr[i][1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// gains of this lane's chunks (8 bf16 per chunk), loaded ahead of the wait
template <int C>
__device__ __forceinline__ void load_gw(u32x4 (&gw)[C], const uint16_t *g, int k, int lane) {
  const int nch = k >> 3;
#pragma unroll
  for (int i = 0; i < C; i++) {
    const int c = lane + i * 64;
    const u32x4 zero = {0u, 0u, 0u, 0u};
    gw[i] = c < nch ? *(const u32x4 *)(g + c * 8) : zero;
  }
}

// one row (held 8 columns per chunk per lane) times the split x
template <int C>
__device__ __forceinline__ float dotrow_p(const u32x4 (&t)[C], const XPairs<C> &xp) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < C; i++) {
    const u32x4 w = t[i];
    s = dot2(w.x, xp.h[i][0], s);
    s = dot2(w.x, xp.l[i][0], s);
    s = dot2(w.y, xp.h[i][1], s);
    s = dot2(w.y, xp.l[i][1], s);
    s = dot2(w.z, xp.h[i][2], s);
    s = dot2(w.z, xp.l[i][2], s);
    s = dot2(w.w, xp.h[i][3], s);
    s = dot2(w.w, xp.l[i][3], s);
  }
  return wave_sum(s);
}

__device__ __forceinline__ float silu(float z) { return z / (1.0f + expf(-z)); }

// A pointer read from LDS, made provably wave-uniform: kept in scalar
// registers, so a buffer descriptor built from it needs no per-lane loop.
template <class T>
__device__ __forceinline__ T *uni(T *p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (T *)(((uint64_t)hi << 32) | lo);
}

// The value itself, through an empty volatile asm: the compiler cannot treat
// it (or anything computed from it) as loop-invariant.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// phase timestamps of one step (100 MHz device clock), thread 0 of each
// workgroup: slot 0 token chosen; 1 + 5 l + {0 x ready, 1 attention items
// done, 2 attention merged, 3 X_o ready, 4 down partials ready}; 1 + 5 L head input ready;
// 2 + 5 L head done
__device__ __forceinline__ void mark(const PersistArgs &a, uint32_t s, int slot) {
  if (a.trace && s == a.trace_step && threadIdx.x == 0)
    a.trace[(size_t)blockIdx.x * (5 * a.L + 3) + slot] = wall_clock64();
}

// A cache value of this step (f32, or bf16 rounded to nearest even),
// stored device-coherently.
template <bool KB>
__device__ __forceinline__ void kvstore(uint8_t *base, size_t idx, float v) {
  if (KB)
    __hip_atomic_store((uint16_t *)base + idx, (uint16_t)pack_bf16(v, 0.f), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  else
    cstore((float *)base + idx, v);
}

// Gate/up ownership: h values [np * (wg - gst), np * (wg - gst + 1)) go to
// workgroup wg in [gst, gen), np even so a workgroup's share is whole column
// pairs of down. The workgroups that run no attention item (the first
// nkv * nchmax) and no merge (the last nq) take them when they can hold
// them: the attention chain's workgroups then carry almost no weight loads
// into their waits. Otherwise every workgroup takes a share. With head
// attention (na > 0 workgroups at the end run attention and hold its K rows
// where the others hold gate/up rows) the first NB - na take them, or np
// exceeds the cap and the launcher does not pick that mode. Returns np.
__host__ __device__ inline int gu_share(int I, int nkv, int nchmax, int nq, int na, int *gst,
                                        int *gen) {
  const int cap = GPMAX * NW;
  if (na > 0) {
    *gst = 0;
    *gen = NB - na;
    return 2 * ((I + 2 * (NB - na) - 1) / (2 * (NB - na)));
  }
  int a = nkv * nchmax, b = NB - nq;
  int np = b - a > 0 ? 2 * ((I + 2 * (b - a) - 1) / (2 * (b - a))) : cap + 1;
  if (np > cap) {
    a = 0;
    b = NB;
    np = 2 * ((I + 2 * NB - 1) / (2 * NB));
  }
  *gst = a;
  *gen = b;
  return np;
}

// Every dimension of the model is a template constant, or 0 to read it from
// the launch arguments: the launcher picks the Qwen2.5-1.5B instantiation for
// that shape, where folding the dimensions frees the scalar registers that
// the generic build would spill, and the generic one for every other shape.
// KB: the KV cache holds bf16 (else f32). AM, the attention mode: 0 work
// items (kv head, 32-position chunk) merged per q head on one workgroup; 1
// the same with more than 16 chunks per head (max_seq > 512), each head's
// merge split over four workgroups; 2 head attention (head dim 128, at most
// 256 positions): 2 nq workgroups at the end of the grid each own a q head
// and one half of its value columns, hold the head's cached K rows in
// registers and its value half in LDS (loaded a layer ahead), and publish
// their share of the attention output with no merge step.
template <int kH, int kI, int kV, int kNQ, int kNKV, int kD, bool KB, int AM>
__global__ void __launch_bounds__(NT) decode_persistent_kernel(PersistArgs a) {
  extern __shared__ float4 sm4[];
  float *xs = (float *)sm4;     // [MAXH] activation for the current phase
  float *att = xs + MAXH;       // [MAXH] attention output
  float *big = att + MAXH;      // phase scratch: attention staging / merge / h share
  uint8_t *wdl = (uint8_t *)(xs + a.lds_wd);  // [NW][kp][cw] down column pairs
  __shared__ float xl[NW];      // this workgroup's rows of the residual stream
  __shared__ int fail_s;
  __shared__ uint32_t tok_s;
  __shared__ float2 best_s[NW];

  // tid and lane are re-derived at the top of every step and layer (see
  // opaque), so per-lane values computed from them are not hoisted out of
  // the loops and held in registers for the whole launch
  int tid = threadIdx.x, lane = tid & 63;
  const int wg = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = kH ? kH : a.H, I = kI ? kI : a.I, V = kV ? kV : a.V, d = kD ? kD : a.d;
  const int nq = kNQ ? kNQ : a.nq, nkv = kNKV ? kNKV : a.nkv;
  const int half = d >> 1, gq = nq / nkv;
  const int qdim = nq * d, kvdim = nkv * d, qkv_rows = qdim + 2 * kvdim;
  const uint32_t TPS = (uint32_t)a.L * kTPL + 2;
  const int nchmax = (a.max_seq + AC - 1) / AC;
  // head attention: workgroups [NBW, NB) run attention, the others own the
  // QKV, residual (o, down) and gate/up rows
  constexpr bool HA = AM == 2;
  const int NA = HA ? 2 * nq : 0, NBW = NB - NA;
  const bool is_att = HA && wg >= NBW;
  // attention workgroup i = wg - NBW takes q head ah, value half avh. The
  // dispatcher deals workgroups to the 8 XCDs round robin (XCD = wg % 8),
  // and each XCD's L2 fetches the cached rows its workgroups read: with 12 q
  // heads over 2 kv heads, kv head g goes to XCDs 4 g .. 4 g + 3 (3
  // workgroups each), so its K rows are fetched by 4 L2s and each value half
  // by 2, where i -> (i / 2, i % 2) spreads every kv head over all 8.
  int ah = 0, avh = 0;
  if (HA) {
    const int i = max(wg - NBW, 0);
    if (nq == 12 && nkv == 2 && NBW % 8 == 0) {
      const int x = i & 7, li = (i >> 3) * 4 + (x & 3);
      ah = (x >> 2) * 6 + (li >> 1);
      avh = li & 1;
    } else {
      ah = i >> 1;
      avh = i & 1;
    }
  }
  const int ag = ah / gq;  // its kv head
  // ownership
  const int qper = (((qkv_rows + NBW - 1) / NBW) + 1) & ~1;
  const int q0 = wg < NBW ? wg * qper : qkv_rows, q1 = min(q0 + qper, qkv_rows);
  const int xper = (H + NBW - 1) / NBW;
  const int x0 = wg < NBW ? min(wg * xper, H) : H, x1 = min(x0 + xper, H);
  int gst, gen;
  const int np = gu_share(I, nkv, nchmax, nq, NA, &gst, &gen);
  const int gper = 2 * np;  // gate/up rows
  const int g0 = wg >= gst && wg < gen ? (wg - gst) * gper : 2 * I;
  const int g1 = min(g0 + gper, 2 * I);
  const int nact = (I + np - 1) / np;  // workgroups gst .. gst + nact - 1 hold h values
  // down as column pairs: this workgroup's h values pair up into kv rows of
  // P = [I / 2][H], from row j0; wave w takes columns [w cw, (w + 1) cw)
  const int kp = np >> 1, j0 = g0 >> 2;
  const int kv = max(0, min(kp, (I >> 1) - j0));
  const int cw = H / NW;
  const int vper = (V + NB - 1) / NB;
  const int v0 = wg * vper, v1 = min(v0 + vper, V);
  const int qrow = q0 + 2 * wave;      // this wave's QKV pair
  const int xrow = x0 + wave;          // this wave's residual row (o and down)
  const bool has_q = qrow < q1, has_x = xrow < x1;

  // The layer table, copied to LDS once: a weight pointer read from global
  // memory inside the loop would be a vector load whose wait (vmcnt 0) also
  // waits for every weight load in flight.
  PersistLayer *lay = (PersistLayer *)(wdl + (size_t)NW * kp * cw * 4);
  for (int i = tid; i < a.L * (int)(sizeof(PersistLayer) / 8); i += NT)
    ((uint64_t *)lay)[i] = ((const uint64_t *)a.layers)[i];
  if (tid == 0) fail_s = 0;
  if (tid < NW) xl[tid] = 0.f;
  __syncthreads();

  // Weight rows held on chip across phases: this wave's QKV pair, o row and
  // gate/up pairs in registers, its block of down column pairs in LDS. A
  // wait re-polls with vector loads, which queue behind every load the CU
  // issued before them, so loads go out right after a wait returns and drain
  // while the next phase computes, each batch as soon as its registers are
  // free:
  //   after the items of l (before the merge): gate/up slots 1-3 of l
  //   after the X_o wait of l:                 gate/up slot 4 of l
  //   during gate/up(l), after slot 0's dots:  gate/up slot 0 of l+1
  //   after the gate/up dots of l:             o(l+1) with head attention
  //   after the down partials of l:            QKV(l+1) (and o(l+1) in the
  //                                            item modes)
  // A wave that issues more loads than its memory queue holds stalls at the
  // issue, so big batches go out where the wave would wait anyway. Loads into
  // LDS make the compiler wait for them before the wave's next LDS access,
  // so the down block goes in three parts, each just before a wait: before
  // the x wait of l, after QKV(l) (with head attention, between gate/up
  // slots 2 and 3) and after o(l). (One batch after QKV(l) is 9 % slower:
  // the attention-output wait then drains all of it.)
  // Layer 0's first share loads after the head, so that no weight row is
  // live across the head's own tiles.
  u32x4 wq0[HC], wq1[HC], wo[HC];
  u32x4 gu[GPMAX][2][HC];  // gate/up slot p: rows (2i, 2i+1) = (gate_i, up_i)
  uint8_t *wp_s = wdl + (size_t)wave * kp * cw * 4;  // this wave's down block

  // gate/up pair in slot p of this wavefront
  auto gu_row = [&](int p) { return g0 + 2 * (wave + p * NW); };
  auto issue_q = [&](int l, bool v) {
    const uint16_t *w = uni(lay[l].wqkv);
    ldrow<HC>(wq0, w, H, qrow, v && has_q, lane);
    ldrow<HC>(wq1, w, H, qrow + 1, v && has_q, lane);
  };
  auto issue_o = [&](int l, bool v) { ldrow<HC>(wo, uni(lay[l].wo), qdim, xrow, v && has_x, lane); };
  auto issue_gu = [&](int l, bool v, int p) {
    const int row = gu_row(p);
    const bool ok = v && row < g1;
    const uint16_t *w = uni(lay[l].wgu);
    ldrow<HC>(gu[p][0], w, H, row, ok, lane);
    ldrow<HC>(gu[p][1], w, H, row + 1, ok, lane);
  };
  auto issue_wdp = [&](int l, int part) {
    if (kv > 0) dma_block(uni(lay[l].wdp), H, j0, kv, wave * cw, cw, wp_s, lane, part);
  };

  // ---- head attention (HA): K rows in the gate/up slot registers, value half
  // in LDS where the others hold their down block -----------------------------
  // Thread (r = tid / 8, j8 = tid % 8) holds columns [16 j8, 16 j8 + 16) of
  // cached positions r + 64 i, i < 4: f32 in kreg(4 i + c), c < 4, or bf16 in
  // kreg(2 i + c), c < 2.
  auto kreg = [&](int i) -> u32x4 & { return gu[i / (2 * HC)][(i / HC) & 1][i % HC]; };
  constexpr int HAD = 128, HAP = 256;                  // head dim, positions
  constexpr int hvb = HAD / 2 * (KB ? 2 : 4);          // bytes of a value half row
  // value half rows in LDS as 16-byte chunks, chunk c of row t at slot
  // t * hvc + (c ^ (t % hvc)): the V sum reads one chunk column of 64
  // consecutive rows at once, and the swizzle spreads them over the banks
  constexpr int hvc = hvb / 16;                        // chunks per row
  uint8_t *hv_s = wdl;                                 // [HAP][HAD / 2] value half
  float *hq_s = (float *)(wdl + HAP * hvb);            // [HAD] q head
  float *hk_s = hq_s + HAD;                            // [HAD] this step's k row
  float *hp_s = hk_s + HAD;                            // [HAP] scaled scores
  float *ho_s = hp_s + HAP;                            // [HAD / 2] this workgroup's output
  auto att_kv_rsrc = [&](const float *base, int l) {
    constexpr int kvb = KB ? 2 : 4;
    return __builtin_amdgcn_make_buffer_rsrc((void *)((const uint8_t *)base + (size_t)l * a.layer_kv * kvb),
                                             (short)0, (int)(a.layer_kv * kvb), 0x00020000);
  };
  // cached K rows [0, npos) of layer l into kreg; a row past npos reads at
  // an offset past the buffer (zeros, no traffic), so every load is issued
  auto att_load_k = [&](int l, int npos) {
    if (!HA) return;
    constexpr int kvb = KB ? 2 : 4, nc = KB ? 2 : 4;
    const __amdgpu_buffer_rsrc_t rk = att_kv_rsrc(a.kc, l);
    const int r = tid >> 3, j8 = tid & 7;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int t = r + 64 * i;
      const uint32_t off = t < npos ? (uint32_t)(((ag * a.max_seq + t) * HAD + 16 * j8) * kvb) : 0x80000000u;
#pragma unroll
      for (int c = 0; c < nc; c++) kreg(nc * i + c) = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 16 * c, 16);
    }
  };
  // cached value-half rows [0, npos) of layer l into hv_s with direct (DMA)
  // loads, 1 KB per wave instruction: lane l fills slot 64 i + l, so it
  // fetches the chunk the swizzle puts there
  auto att_load_v = [&](int l, int npos) {
    if (!HA) return;
    constexpr int kvb = KB ? 2 : 4, rpl = 1024 / hvb;  // rows per load
    const __amdgpu_buffer_rsrc_t rv = att_kv_rsrc(a.vc, l);
    const int nld = (npos + rpl - 1) / rpl;
    for (int i = wave; i < nld; i += NW) {
      const int t = i * rpl + lane / hvc, c = (lane % hvc) ^ (t % hvc);
      const uint32_t off = t < npos ? (uint32_t)((((ag * a.max_seq + t) * HAD) + avh * (HAD / 2)) * kvb + c * 16)
                                    : 0x80000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (__attribute__((address_space(3))) void *)(hv_s + i * 1024), 16, off, 0, 0, 16);
    }
  };

  // what layer l needs loaded before its first wait
  auto issue_first = [&](int l) {
    issue_wdp(l, 0);
    issue_q(l, true);
    issue_o(l, true);
    issue_gu(l, true, 0);
  };

  // ---- final norm + head + argmax partial of step s (tag tstep + kTPL L);
  // `next` issues the next step's first loads once the head's tiles are out
  // pre: the wave's first head tile was issued at the end of the last layer
  // into the QKV pair's registers (the item modes: the last layer has no
  // next-layer loads, so the head's first round trip would otherwise start
  // after the x wait; long-context launch 204.0-204.2 -> 199.6-200.0 ms; with
  // head attention it cost S1 1.5 %)
  auto head_phase = [&](uint32_t s, uint32_t tstep, auto next, bool pre) {
    const uint32_t TH = tstep + (uint32_t)a.L * kTPL;
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    {
      XPairs<HC> xp;
      {
        u32x4 gw[HC];
        load_gw<HC>(gw, a.final_norm, H, lane);
        tgather_lin<3>(a.txd, H, TH - kTPL + P_XD, xs, a, &fail_s);
        mark(a, s, 1 + 5 * a.L);
        float4 xr[HC][2];
        norm_x<HC>(xr, xp, xs, gw, H, a.eps, lane);
        if (wg == 0 && wave == 0) {
#pragma unroll
          for (int i = 0; i < HC; i++) {
            const int c = lane + i * 64;
            if (c < (H >> 3)) {
              *(float4 *)(a.normed + c * 8) = xr[i][0];
              *(float4 *)(a.normed + c * 8 + 4) = xr[i][1];
            }
          }
        }
      }
      // this wave's rows v0 + wave*HT + k*NW*HT, two tiles in flight
      u32x4 ta[HT][HC], tb[HT][HC];
      const int stride = NW * HT;
      int r0 = v0 + wave * HT;
      static_assert(HT == 2, "the preloaded first tile is the QKV pair's two rows");
      if (pre) {
#pragma unroll
        for (int i = 0; i < HC; i++) {
          ta[0][i] = wq0[i];
          ta[1][i] = wq1[i];
        }
      } else {
#pragma unroll
        for (int r = 0; r < HT; r++) ldrow_all<HC>(ta[r], a.head, H, r0 + r, v1 - 1, lane);
      }
      for (; r0 < v1; r0 += 2 * stride) {
        const int r1 = r0 + stride;
#pragma unroll
        for (int r = 0; r < HT; r++) ldrow_all<HC>(tb[r], a.head, H, r1 + r, v1 - 1, lane);
#pragma unroll
        for (int r = 0; r < HT; r++)
          if (r0 + r < v1) {
            const float y = dotrow_p<HC>(ta[r], xp);
            if (lane == 0) a.logits[r0 + r] = y;
            if (beats(y, (uint32_t)(r0 + r), bv, bi)) {
              bv = y;
              bi = (uint32_t)(r0 + r);
            }
          }
        const int r2 = r1 + stride;
#pragma unroll
        for (int r = 0; r < HT; r++) ldrow_all<HC>(ta[r], a.head, H, r2 + r, v1 - 1, lane);
#pragma unroll
        for (int r = 0; r < HT; r++)
          if (r1 + r < v1) {
            const float y = dotrow_p<HC>(tb[r], xp);
            if (lane == 0) a.logits[r1 + r] = y;
            if (beats(y, (uint32_t)(r1 + r), bv, bi)) {
              bv = y;
              bi = (uint32_t)(r1 + r);
            }
          }
      }
    }
    if (s + 1 < a.steps) next();
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
  };

  // ---- the head-attention workgroups' own loop: per layer, wait for the
  // head's q and this step's k / value half, attend over every position,
  // publish, then load the next layer's cached rows; per step, a share of the
  // head. Their registers hold K, so they run apart from the loop below. --
  if (HA && is_att) {
    att_load_k(0, (int)a.pos0);
    att_load_v(0, (int)a.pos0);
    for (uint32_t s = 0; s < a.steps; s++) {
      const uint32_t pos = a.pos0 + s;
      const int seq = (int)pos + 1;
      const uint32_t tstep = a.tag_base + s * TPS;
      for (int l = 0; l < a.L; l++) {
        tid = opaque(tid);
        lane = tid & 63;
        const uint32_t T = tstep + (uint32_t)l * kTPL;
        // ---- head attention (tag T + P_ATT): q head ah, value columns
        // [64 avh, 64 avh + 64) of kv head ag, all positions at once ----------
        // Every wave's direct-to-LDS loads of this layer's value rows have
        // landed before any wave writes this step's row: a load for a row
        // past the cached ones (out of range, it writes zeros) could land on
        // it otherwise. They were issued a layer ago, so this costs no wait.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        // q of the head, this step's k and value half: one tagged word a thread
        constexpr int nw = 2 * HAD + HAD / 2;
        if (tid < nw) {
          const uint64_t *src = tid < HAD       ? a.tq + ah * HAD + tid
                                : tid < 2 * HAD ? a.tkv + ag * HAD + (tid - HAD)
                                                : a.tkv + kvdim + ag * HAD + avh * (HAD / 2) + (tid - 2 * HAD);
          uint64_t w = 0;
          for (unsigned spins = 0; fail_s == 0; spins++) {
            w = tload(src);
            if ((uint32_t)(w >> 32) == T + P_QKV) break;
            if (spin_fail(a, spins)) {
              fail_s = 1;
              break;
            }
            __builtin_amdgcn_s_sleep(1);
          }
          const float v = __uint_as_float((uint32_t)w);
          const uint32_t vb = pack_bf16(v, 0.f);  // this step's k and v as its cache slot holds them
          if (tid < HAD) hq_s[tid] = v;
          else if (tid < 2 * HAD) hk_s[tid - HAD] = KB ? bf_lo(vb) : v;
          else {
            constexpr int per = 16 / (KB ? 2 : 4);  // values per chunk
            const int j = tid - 2 * HAD, c = j / per;
            uint8_t *dst = hv_s + (pos * hvc + (c ^ (pos % hvc))) * 16;
            if (KB) ((uint16_t *)dst)[j % per] = (uint16_t)vb;
            else ((float *)dst)[j % per] = v;
          }
        }
        __syncthreads();
        // scores: 16-column partial dots of positions r + 64 i, summed over
        // the 8 lanes of a position
        {
          const int r = tid >> 3, j8 = tid & 7;
          float4 q4[4], c4[4];
#pragma unroll
          for (int c = 0; c < 4; c++) {
            q4[c] = *(const float4 *)(hq_s + 16 * j8 + 4 * c);
            c4[c] = *(const float4 *)(hk_s + 16 * j8 + 4 * c);
          }
          float sc[4];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int t = r + 64 * i;
            const bool cur = t == (int)pos;
            float kf[16];
#pragma unroll
            for (int c = 0; c < 4; c++) {
              if (KB) {
                const u32x4 kw = kreg(2 * i + (c >> 1));
                const uint32_t w0 = (c & 1) ? kw.z : kw.x, w1 = (c & 1) ? kw.w : kw.y;
                kf[4 * c] = bf_lo(w0);
                kf[4 * c + 1] = bf_hi(w0);
                kf[4 * c + 2] = bf_lo(w1);
                kf[4 * c + 3] = bf_hi(w1);
              } else {
                const u32x4 kw = kreg(4 * i + c);
                kf[4 * c] = __uint_as_float(kw.x);
                kf[4 * c + 1] = __uint_as_float(kw.y);
                kf[4 * c + 2] = __uint_as_float(kw.z);
                kf[4 * c + 3] = __uint_as_float(kw.w);
              }
            }
            float v = 0.f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
              const float4 q = q4[c], k = cur ? c4[c] : make_float4(kf[4 * c], kf[4 * c + 1],
                                                                    kf[4 * c + 2], kf[4 * c + 3]);
              v = fmaf(q.x, k.x, v);
              v = fmaf(q.y, k.y, v);
              v = fmaf(q.z, k.z, v);
              v = fmaf(q.w, k.w, v);
            }
            sc[i] = v;
          }
          seg_sum_n<4>(sc, 8);
          const float scale = 1.0f / sqrtf((float)HAD);
          if (j8 == 0) {
#pragma unroll
            for (int i = 0; i < 4; i++)
              if (r + 64 * i < seq) hp_s[r + 64 * i] = sc[i] * scale;
          }
        }
        __syncthreads();
        // softmax over the positions in every wave: lane l holds positions
        // l + 64 i, the rows whose values it multiplies in the V sum. Wave w
        // sums columns [8 w, 8 w + 8) of the value half over every position
        // into LDS, and wave 0 publishes the 64 columns with one store (eight
        // single-lane stores per wave to one line serialise in the memory
        // pipeline, and the next layer's loads queue behind them).
        {
          float ev[4], mloc = -INFINITY;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int t = lane + 64 * i;
            ev[i] = t < seq ? hp_s[t] : -INFINITY;
            mloc = fmaxf(mloc, ev[i]);
          }
          const float mx = wave_max(mloc);
          float lsum = 0.f;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            ev[i] = lane + 64 * i < seq ? expf(ev[i] - mx) : 0.f;
            lsum += ev[i];
          }
          const float inv = 1.0f / wave_sum(lsum);
          float acc[8];
#pragma unroll
          for (int j = 0; j < 8; j++) acc[j] = 0.f;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int t = lane + 64 * i;
            const bool in = t < seq;  // rows past seq hold stale LDS: masked, not just weighted by 0
            float v[8];
            if (KB) {
              const u32x4 w = *(const u32x4 *)(hv_s + (t * hvc + (wave ^ (t % hvc))) * 16);
              v[0] = bf_lo(w.x), v[1] = bf_hi(w.x), v[2] = bf_lo(w.y), v[3] = bf_hi(w.y);
              v[4] = bf_lo(w.z), v[5] = bf_hi(w.z), v[6] = bf_lo(w.w), v[7] = bf_hi(w.w);
            } else {
              const float4 w0 = *(const float4 *)(hv_s + (t * hvc + ((2 * wave) ^ (t % hvc))) * 16);
              const float4 w1 = *(const float4 *)(hv_s + (t * hvc + ((2 * wave + 1) ^ (t % hvc))) * 16);
              v[0] = w0.x, v[1] = w0.y, v[2] = w0.z, v[3] = w0.w;
              v[4] = w1.x, v[5] = w1.y, v[6] = w1.z, v[7] = w1.w;
            }
#pragma unroll
            for (int j = 0; j < 8; j++) acc[j] = fmaf(ev[i], in ? v[j] : 0.f, acc[j]);
          }
          wave_sum_n<8>(acc);
          if (lane == 63) {
#pragma unroll
            for (int j = 0; j < 8; j++) ho_s[8 * wave + j] = acc[j] * inv;
          }
        }
        // (every wave has also read the value rows before the next layer's land)
        __syncthreads();
        if (tid < HAD / 2) tput(a.tatt + ah * HAD + avh * (HAD / 2) + tid, ho_s[tid], T + P_ATT);
        // the next layer's cached rows (this step), or the value half of the
        // next step's layer 0 (its K rows load after the head, so that no K
        // register is live across the head's tiles)
        if (l + 1 < a.L) {
          att_load_k(l + 1, (int)pos);
          att_load_v(l + 1, (int)pos);
        } else if (s + 1 < a.steps) {
          att_load_v(0, (int)pos + 1);
        }
        mark(a, s, 2 + 5 * l);
      }
      head_phase(s, tstep, [&] { att_load_k(0, (int)pos + 1); }, false);
    }
    return;
  }

  issue_first(0);
  for (uint32_t s = 0; s < a.steps; s++) {
    tid = opaque(tid);
    lane = tid & 63;
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
        const uint32_t best = idx < (uint32_t)V ? idx : 0u;  // no candidate (all NaN / -inf) -> 0
        if (wg == 0) a.out_ids[s] = best;
        tok_s = a.force ? a.force[s] : best;  // teacher forcing feeds the given id
        if (wg == 0 && s + 1 == a.steps) a.state[1] = tok_s;
      }
      __syncthreads();
      const uint16_t *erow = a.embed + (size_t)tok_s * H;
      for (int j = tid; j < H; j += NT) xs[j] = bf16f(erow[j]);
      if (tid < NW && x0 + tid < x1) xl[tid] = bf16f(erow[x0 + tid]);
      __syncthreads();
      mark(a, s, 0);
    }

    for (int l = 0; l < a.L; l++) {
      tid = opaque(tid);
      lane = tid & 63;
      const uint16_t *Lln1 = uni(lay[l].ln1), *Lln2 = uni(lay[l].ln2);
      const float *Lbqkv = uni(lay[l].bqkv);
      const uint32_t T = tstep + (uint32_t)l * kTPL;
      constexpr int kvb = KB ? 2 : 4;  // bytes per cached value
      uint8_t *kc = (uint8_t *)a.kc + (size_t)l * a.layer_kv * kvb;
      uint8_t *vc = (uint8_t *)a.vc + (size_t)l * a.layer_kv * kvb;

      // ---- QKV + bias + RoPE + KV store (tag T + P_QKV) ---------------------
      // gains, bias and this pair's (cos, sin) load while x is awaited
      u32x4 gw[HC];
      load_gw<HC>(gw, Lln1, H, lane);
      const bool roped = qrow < qdim + kvdim;
      const int qu = (roped && qrow >= qdim ? qrow - qdim : qrow) >> 1;
      const int qhead = qu / half, qp = qu - qhead * half;
      float qb0 = 0.f, qb1 = 0.f;
      float2 qcs = make_float2(1.f, 0.f);
      if (has_q) {
        qb0 = Lbqkv[qrow];
        qb1 = Lbqkv[qrow + 1];
        if (roped) qcs = a.rope[(size_t)pos * half + qp];
      }
      if (l > 0) tgather_lin<3>(a.txd, H, T - kTPL + P_XD, xs, a, &fail_s);
      mark(a, s, 1 + 5 * l);
      if (has_q) {
        float4 xr[HC][2];
        XPairs<HC> xp;
        norm_x<HC>(xr, xp, xs, gw, H, a.eps, lane);
        const float y0 = dotrow_x<HC>(wq0, xr, H, lane), y1 = dotrow_x<HC>(wq1, xr, H, lane);
        if (lane == 0) {
          const float b0 = y0 + qb0, b1 = y1 + qb1;
          if (roped) {
            const bool is_q = qrow < qdim;
            const int head = qhead, p = qp;
            const float2 cs = qcs;
            const float o0 = b0 * cs.x - b1 * cs.y, o1 = b1 * cs.x + b0 * cs.y;
            if (is_q) {
              tput(a.tq + head * d + p, o0, T + P_QKV);
              tput(a.tq + head * d + p + half, o1, T + P_QKV);
            } else {
              const size_t base = ((size_t)head * a.max_seq + pos) * d;
              kvstore<KB>(kc, base + p, o0);
              kvstore<KB>(kc, base + p + half, o1);
              tput(a.tkv + head * d + p, o0, T + P_QKV);
              tput(a.tkv + head * d + p + half, o1, T + P_QKV);
            }
          } else {
            const int rr = qrow - qdim - kvdim, head = rr / d, j = rr - head * d;
            const size_t base = ((size_t)head * a.max_seq + pos) * d + j;
            kvstore<KB>(vc, base, b0);
            kvstore<KB>(vc, base + 1, b1);
            tput(a.tkv + kvdim + head * d + j, b0, T + P_QKV);
            tput(a.tkv + kvdim + head * d + j + 1, b1, T + P_QKV);
          }
          // Later steps read the cache rows without tags, so they must be
          // complete before anything this wave publishes later. Every later
          // publish follows one of the wave's gathers, and the wait for a
          // gather's loads (vmcnt 0) also waits for these stores (gfx9 counts
          // stores in vmcnt). The empty asm with a memory clobber keeps the
          // compiler from sinking the stores past that wait.
          asm volatile("" ::: "memory");
        }
      }

      if (!HA) issue_wdp(l, 1);

      // ---- attention partials for (kv head, chunk) items (tag T + P_PART) ----
      // (AM 0 and 1; head attention follows below)
      // Thread i = tid + u NT holds columns [4 j4, 4 j4 + 4) of position
      // t = i / dq of the chunk (dq = d / 4 lanes per position), K in
      // registers and V staged in LDS. A score is a dq-lane segmented sum;
      // then wave h takes q head h: softmax over the chunk in its lanes and
      // the V sum with each weight read back from the lane that holds it.
      const int nch = (seq + AC - 1) / AC;
      for (int it = HA ? NB : wg; it < nkv * nch; it += NB) {
        const int g = it % nkv, c = it / nkv;
        const int t0 = c * AC, n = min(AC, seq - t0);
        const bool has_cur = (int)pos < t0 + n;  // this step's row ends the chunk
        const int nold = has_cur ? n - 1 : n;
        float *q_s = big;                    // [gq][d]
        float *kcur = q_s + gq * d;          // [d] this step's k row of head g
        float *v_s = kcur + d;               // [AC][d]
        float *p_s = v_s + AC * d;           // [gq][AC] scaled scores
        const int dq = d >> 2, j4 = tid & (dq - 1);
        // cached rows (positions < pos, complete before this step) and the
        // tagged q heads + this step's k, v of head g, all in one round trip
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            kc, (short)0, (int)(a.layer_kv * kvb), 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            vc, (short)0, (int)(a.layer_kv * kvb), 0x00020000);
        u32x4 kr[KV4], vr[KV4];
#pragma unroll
        for (int u = 0; u < KV4; u++) {
          const int t = (tid + u * NT) / dq;
          const u32x4 zero = {0u, 0u, 0u, 0u};
          kr[u] = zero;
          vr[u] = zero;
          if (t < nold) {
            const uint32_t off = (uint32_t)((((size_t)g * a.max_seq + t0 + t) * d + j4 * 4) * kvb);
            if (KB) {  // four bf16 -> four f32 bit patterns
              const u32x2 k2 = __builtin_amdgcn_raw_buffer_load_b64(rk, off, 0, 16);
              const u32x2 v2 = __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 16);
              kr[u] = (u32x4){k2.x << 16, k2.x & 0xffff0000u, k2.y << 16, k2.y & 0xffff0000u};
              vr[u] = (u32x4){v2.x << 16, v2.x & 0xffff0000u, v2.y << 16, v2.y & 0xffff0000u};
            } else {
              kr[u] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 16);
              vr[u] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 16);
            }
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
          const int t = (tid + u * NT) / dq;
          if (t < nold)
            *(float4 *)(v_s + t * d + j4 * 4) =
                make_float4(__uint_as_float(vr[u].x), __uint_as_float(vr[u].y),
                            __uint_as_float(vr[u].z), __uint_as_float(vr[u].w));
        }
#pragma unroll
        for (int u = 0; u < QW; u++) {
          const int i = tid + u * NT, r = i - nqw;
          const float v = __uint_as_float((uint32_t)w[u]);
          // this step's k and v as its cache slot holds them
          const float kvv = KB ? bf_lo(pack_bf16(v, 0.f)) : v;
          if (i < nqw) q_s[i] = v;
          else if (i < nw) {
            if (r < d) kcur[r] = kvv;
            else v_s[nold * d + r - d] = kvv;
          }
        }
        __syncthreads();
        const float scale = 1.0f / sqrtf((float)d);
#pragma unroll
        for (int u = 0; u < KV4; u++) {
          const int t = (tid + u * NT) / dq;
          float4 k4 = make_float4(__uint_as_float(kr[u].x), __uint_as_float(kr[u].y),
                                  __uint_as_float(kr[u].z), __uint_as_float(kr[u].w));
          if (t >= nold) k4 = t < n ? *(const float4 *)(kcur + j4 * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
          // every head's partial dot, then the segmented sums over all heads
          // at once (heads past gq are zeros and not stored)
          float sc[8];
#pragma unroll
          for (int h = 0; h < 8; h++) {
            sc[h] = 0.f;
            if (h < gq) {
              const float4 q4 = *(const float4 *)(q_s + h * d + j4 * 4);
              float v = q4.x * k4.x;
              v = fmaf(q4.y, k4.y, v);
              v = fmaf(q4.z, k4.z, v);
              sc[h] = fmaf(q4.w, k4.w, v);
            }
          }
          seg_sum_n<8>(sc, dq);
          if (t < n && seg_leader(lane, dq)) {
#pragma unroll
            for (int h = 0; h < 8; h++)
              if (h < gq) p_s[h * AC + t] = sc[h] * scale;
          }
        }
        __syncthreads();
        if (wave < gq) {
          const int h = wave;
          const float sc = lane < n ? p_s[h * AC + lane] : -INFINITY;
          const float mx = wave_max(sc);
          const float e = lane < n ? expf(sc - mx) : 0.f;
          const float lsum = wave_sum(e);
          // the weights go back through LDS and are read four at a time as
          // broadcasts; lanes past the head's columns read in-row duplicates
          // and drop them
          if (lane < AC) p_s[h * AC + lane] = e;
          // lane l sums columns 2l and 2l + 1 (one 8-byte LDS read per position)
          const int c2 = 2 * lane < d ? 2 * lane : 0;
          float o0 = 0.f, o1 = 0.f;
          if (n == AC) {
#pragma unroll
            for (int t4 = 0; t4 < AC; t4 += 4) {
              const float4 e4 = *(const float4 *)(p_s + h * AC + t4);
              const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
              for (int k = 0; k < 4; k++) {
                const float2 v2 = *(const float2 *)(v_s + (t4 + k) * d + c2);
                o0 = fmaf(ev[k], v2.x, o0);
                o1 = fmaf(ev[k], v2.y, o1);
              }
            }
          } else {
#pragma unroll
            for (int t4 = 0; t4 < AC; t4 += 4) {
              if (t4 < n) {
                const float4 e4 = *(const float4 *)(p_s + h * AC + t4);
                const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                  // rows past n hold stale LDS: masked, not just weighted by 0
                  const bool in = t4 + k < n;
                  const float2 v2 = *(const float2 *)(v_s + (t4 + k) * d + c2);
                  o0 = fmaf(ev[k], in ? v2.x : 0.f, o0);
                  o1 = fmaf(ev[k], in ? v2.y : 0.f, o1);
                }
              }
            }
          }
          uint64_t *dst = a.tpart + ((size_t)(g * gq + h) * nchmax + c) * (d + 2);
          if (2 * lane < d) {
            tput(dst + 2 * lane, o0, T + P_PART);
            tput(dst + 2 * lane + 1, o1, T + P_PART);
          }
          if (lane == 0) {
            tput(dst + d, mx, T + P_PART);
            tput(dst + d + 1, lsum, T + P_PART);
          }
        }
        __syncthreads();
      }

      issue_gu(l, true, 1);
      issue_gu(l, true, 2);
      // With head attention the down block's second part goes between slots
      // 2 and 3 rather than ahead of slot 1 (S1 91.3 -> 90.0 ms per launch;
      // after slot 3 90.2-90.4, after the attention-output wait 99); the item
      // modes keep it right after QKV (after their slots it cost the
      // long-context launch 203.4 -> 207.2 ms).
      if (HA) issue_wdp(l, 1);
      issue_gu(l, true, 3);

      // ---- merge: q head h's chunks -> att[h] (tag T + P_ATT), on the last
      // workgroups (attention items start at the first); one wave combines
      // att = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c. Launches with
      // more than 16 chunks per head (MS) split a head over four workgroups of
      // d / 4 columns each, so no merge gathers more than about 5 words a thread.
      constexpr int mp = AM == 1 ? 4 : 1;
      const int mi = NB - 1 - wg, mh = mi / mp, mq = mi - mh * mp;
      if (!HA && mh < nq) {
        const int dd = d + 2, dw = d / mp, dpw = dw + 2, j0 = mq * dw;
        float *pc = big;                     // [nch][dw + 2]: columns j0 .. j0 + dw, then m, l
        float *wc = big + nch * dpw;         // [nch] chunk weights
        const int base = mh * nchmax * dd;
        if (AM != 1)
          tgather<2>(a.tpart, [base](int i) { return base + i; }, nch * dd, T + P_PART, pc, a, &fail_s);
        else
          tgather<2>(
              a.tpart,
              [=](int i) {
                const int c = i / dpw, r = i - c * dpw;
                return base + c * dd + (r < dw ? j0 + r : d + (r - dw));
              },
              nch * dpw, T + P_PART, pc, a, &fail_s);
        if (wave == 0) {
          float mloc = -INFINITY;
          for (int c = lane; c < nch; c += 64) mloc = fmaxf(mloc, pc[c * dpw + dw]);
          const float mx = wave_max(mloc);
          float lloc = 0.f;
          for (int c = lane; c < nch; c += 64) {
            const float e = expf(pc[c * dpw + dw] - mx);
            wc[c] = e;
            lloc = fmaf(e, pc[c * dpw + dw + 1], lloc);
          }
          const float inv = 1.0f / wave_sum(lloc);
          for (int j = lane; j < dw; j += 64) {
            float acc = 0.f;
#pragma unroll 4
            for (int c = 0; c < nch; c++) acc = fmaf(wc[c], pc[c * dpw + j], acc);
            tput(a.tatt + mh * d + j0 + j, acc * inv, T + P_ATT);
          }
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

      issue_wdp(l, 2);
      // ---- gate/up + SwiGLU + down partials (tag T + P_PD) ----------------------
      load_gw<HC>(gw, Lln2, H, lane);
      tgather_lin<3>(a.txo, H, T + P_XO, xs, a, &fail_s);
      mark(a, s, 4 + 5 * l);
      // The last gate/up slot goes out only now: issued with slots 1-3 (or,
      // with head attention, before the X_o wait) it held the waits behind it
      // (the X_o wait 1.3 us with head attention). Its dots come last, so the
      // first four slots' dots cover its round trip.
      issue_gu(l, true, 4);
      // every dot first, then the stores
      float gy[GPMAX][2];
      {
        float4 xr[HC][2];
        XPairs<HC> xp;
        norm_x<HC>(xr, xp, xs, gw, H, a.eps, lane);
#pragma unroll
        for (int p = 0; p < GPMAX; p++) {
          gy[p][0] = gu_row(p) < g1 ? dotrow_p<HC>(gu[p][0], xp) : 0.f;
          gy[p][1] = gu_row(p) < g1 ? dotrow_p<HC>(gu[p][1], xp) : 0.f;
          if (p == 0 && l + 1 < a.L) issue_gu(l + 1, true, 0);
        }
      }
      // the next layer's o row, with head attention: issued after the
      // residual publish it queued ahead of the x wait; here its round trip
      // passes while the partials are computed and gathered (92.1-92.4 ->
      // 91.2-91.7 ms per S1 launch; issued between the slots' dots it cost
      // 0.7-5 ms). The item modes keep it after the publish: here it cost the
      // long-context launch 204.3-204.7 -> 205.9-206.6 ms.
      if (HA && l + 1 < a.L) issue_o(l + 1, true);
      // this workgroup's h values, local index wave + p NW, land in LDS; lane
      // p takes slot p, so a wave evaluates one SwiGLU instead of GPMAX in a row
      float *hs = big;
      {
        float g = gy[0][0], u = gy[0][1];
#pragma unroll
        for (int p = 1; p < GPMAX; p++)
          if (lane == p) {
            g = gy[p][0];
            u = gy[p][1];
          }
        if (lane < GPMAX && gu_row(lane) < g1) hs[wave + lane * NW] = silu(g) * u;
      }
      __syncthreads();
      // down partials: column r of the wave's block times the workgroup's h,
      // h split into bf16 hi + lo pairs (see XPairs), one word per row pair.
      // Lane j < kv packs pair j once; the unrolled loop takes pair j from
      // lane j into scalar registers, so every LDS read of the block can be in
      // flight at once. Rows past kv re-read row kv - 1 against a zero pair.
      if (kv > 0) {
        constexpr int CWC = (MAXH / NW + 63) / 64, KPM = GPMAX * NW / 2;
        float acc[CWC];
#pragma unroll
        for (int i = 0; i < CWC; i++) acc[i] = 0.f;
        const float2 h2 = lane < kv ? *(const float2 *)(hs + 2 * lane) : make_float2(0.f, 0.f);
        const uint32_t hpl = pack_bf16(h2.x, h2.y);
        const uint32_t lpl = pack_bf16(h2.x - bf_lo(hpl), h2.y - bf_hi(hpl));
        const uint32_t *wp = (const uint32_t *)wp_s;
        const int kvm = opaque(kv - 1);  // not hoisted: per-row offsets stay unspilled
        constexpr int RB = KPM / 2;      // rows per batch: reads first, then the dots
#pragma unroll
        for (int jb = 0; jb < KPM; jb += RB) {
          uint32_t wv[RB][CWC];
#pragma unroll
          for (int j = 0; j < RB; j++) {
            const int jj = min(jb + j, kvm);
#pragma unroll
            for (int i = 0; i < CWC; i++) {
              const int c = lane + i * 64;
              wv[j][i] = c < cw ? wp[jj * cw + c] : 0u;
            }
          }
#pragma unroll
          for (int j = 0; j < RB; j++) {
            const uint32_t hp = __builtin_amdgcn_readlane(hpl, jb + j);
            const uint32_t lp = __builtin_amdgcn_readlane(lpl, jb + j);
#pragma unroll
            for (int i = 0; i < CWC; i++) acc[i] = dot2(wv[j][i], lp, dot2(wv[j][i], hp, acc[i]));
          }
        }
        // row r goes to its owner b = r / xper: tpr[b][wg][r - b xper], the
        // block of b holding nx_b = min(xper, H - b xper) words per workgroup
#pragma unroll
        for (int i = 0; i < CWC; i++) {
          const int c = lane + i * 64;
          if (c < cw) {
            const int r = wave * cw + c, b = r / xper, nxb = min(xper, H - b * xper);
            tput(a.tpr + (size_t)b * NB * xper + wg * nxb + (r - b * xper), acc[i], T + P_PD);
          }
        }
      }

      // ---- down + residual (tag T + P_XD) -------------------------------------
      // this workgroup's block: nact partials of each of its nx rows, in one
      // contiguous gather; wave w sums row x0 + w in a fixed order
      {
        const int nx = x1 - x0;
        float *pr = big + 64;  // past the h share, which other waves may still read
        if (nx > 0)
          tgather_lin<3>(a.tpr + (size_t)wg * NB * xper + (size_t)gst * nx, nact * nx, T + P_PD, pr, a,
                         &fail_s);
        if (has_x) {
          float sum = 0.f;
          for (int k = lane; k < nact; k += 64) sum += pr[k * nx + wave];
          const float y = wave_sum(sum);
          if (lane == 0) {
            xl[wave] += y;
            tput(a.txd + xrow, xl[wave], T + P_XD);
          }
        }
      }
      mark(a, s, 5 + 5 * l);
      if (l + 1 < a.L) {
        issue_wdp(l + 1, 0);
        issue_q(l + 1, true);
        if (!HA) issue_o(l + 1, true);
      } else if (!HA) {
        // the head's first tile (see head_phase)
        ldrow_all<HC>(wq0, a.head, H, v0 + wave * HT, v1 - 1, lane);
        ldrow_all<HC>(wq1, a.head, H, v0 + wave * HT + 1, v1 - 1, lane);
      }

    }

    head_phase(s, tstep, [&] { issue_first(0); }, !HA);
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
      a.state[2] = a.steps;
    }
    __syncthreads();
    const float2 none = make_float2(-INFINITY, __uint_as_float(0xffffffffu));
    for (int i = tid; i < a.part_cap; i += NT) a.part_out[i] = i == 0 ? best_s[0] : none;
  }
}

// ============================================================================
// Streamed cooperative decode, for shapes whose layer the chip cannot hold
// (the 7B shape: 466 MB of weights per layer, 1.8 MB per CU).
//
// One cooperative launch of 256 workgroups (512 threads) runs a greedy_decode
// call like decode_persistent_kernel, but every phase streams its weight rows
// from HBM with the next row batch in flight, and phases meet at device-wide
// barriers: a workgroup waits until its own stores have completed, publishes
// a tagged flag word (one per 128-byte line), issues the loads of the next
// phase's first row batch (weights do not depend on the data, so the weight
// stream keeps running across the wait), and waits until all 256 flags carry
// the tag or a later one. Activations cross workgroups through f32 buffers
// with device-coherent (sc1) stores and loads. A layer is five phases:
//   RMSNorm + QKV rows (+ bias, RoPE, KV-cache store) | attention items (kv
//   head, 32-position chunk) on workgroups of their own, the last item of a
//   kv group merging its heads | o rows (+ residual) | RMSNorm + gate/up rows
//   (+ SwiGLU), in tiles handed out by ticket past a fixed share | down rows
//   (+ residual)
// then per step the final norm, the head rows with per-workgroup argmax
// partials and the argmax, which every workgroup takes from the partials.
// Numerics follow the per-kernel path: f32 FMAs over the bf16 weights in the
// same row orders (qwen25_block.rs:220-304 per step), except that a QKV row
// pair past one pair per wave is summed by columns over the waves.
constexpr int WDC = 5;    // 8-column chunks per thread of a down row: I <= 20480
constexpr int WMR = 16;   // residual rows per workgroup: H <= 4096
constexpr int WRB = 2;    // rows per wave batch
constexpr int WXMAX = 4096;  // LDS floats of the phase input vector
constexpr int WMAXQ = 8;     // q heads per kv head
constexpr int WQP = 64;      // QKV rows per workgroup
constexpr int WMCH = 64;     // attention chunks per head (one lane each in the merge)
constexpr int WOR = 32;      // o rows per workgroup
constexpr int WLMAX = 128;   // layers (the layer table sits in LDS)
// barrier tags of a layer, in the order the phases run (a flag is compared
// with >=, so they must grow)
constexpr uint32_t W_QKV = 0, W_ATT = 1, W_XO = 2, W_H = 3, W_X = 4;
static_assert(W_X < kTPL, "five barriers per layer");

__host__ __device__ inline size_t wide_al(size_t n) { return (n + 63) & ~(size_t)63; }

// LDS floats of the attention staging (q, V, scores)
__host__ __device__ inline int wide_big_floats(int d, int max_seq) {
  (void)d;
  (void)max_seq;
  return WMAXQ * MAXD + AC * MAXD + WMAXQ * AC;
}

// workgroups [0, n) run the attention items and hold no o rows, when every
// step's items fit in a quarter of the grid (else 0: o rows everywhere)
__host__ __device__ inline int wide_item_wgs(int nkv, int nchmax) {
  return nkv * nchmax <= NB / 4 ? nkv * nchmax : 0;
}

// f32 activation buffers of the streamed kernel, carved from one allocation
struct WideBufs {
  float *q, *att, *x, *xo, *h, *part, *arg;
  int *cnt;        // per kv group: attention items done this layer (the last one merges)
  uint32_t *tick;  // gate/up tile tickets handed out this launch
};
__host__ __device__ inline size_t wide_part_floats(int nq, int max_seq, int d) {
  return (size_t)nq * ((max_seq + AC - 1) / AC) * (size_t)(d + 2);
}
__host__ __device__ inline WideBufs wide_bufs(float *base, int H, int I, int nq, int d, int max_seq,
                                             size_t *total) {
  WideBufs b;
  const size_t qd = (size_t)nq * d;
  size_t o = 0;
  b.q = base + o;    o += wide_al(qd);
  b.att = base + o;  o += wide_al(qd);
  b.x = base + o;    o += wide_al(H);
  b.xo = base + o;   o += wide_al(H);
  b.h = base + o;    o += wide_al(I);
  b.part = base + o; o += wide_al(wide_part_floats(nq, max_seq, d));
  b.arg = base + o;  o += wide_al(2 * NB);
  b.cnt = (int *)(base + o); o += wide_al(WMAXQ * 64);
  b.tick = (uint32_t *)(base + o); o += wide_al(1);
  if (total) *total = o;
  return b;
}

// device-coherent (sc1) 32-bit load of float i of the buffer at p: an
// ordinary load to the compiler, so a run of them goes out back to back (a
// relaxed atomic load would take a full wait after each one)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t crsrc(const void *p) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, 0x7fffffff, 0x00020000);
}
// a plain buffer descriptor over p (loads through it are scalar-addressed)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gsrc(const void *p) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ float cldb(__amdgpu_buffer_rsrc_t rs, int byte_off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, byte_off, 0, 16));
}
__device__ __forceinline__ float cld(__amdgpu_buffer_rsrc_t rs, int i) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, i * 4, 0, 16));
}

// Device-wide barrier `tag`: this workgroup's stores are complete (vmcnt
// counts stores on gfx9) before thread 0 publishes the flag; `pf` then issues
// the next phase's weight loads (after the flag, so the wait for the stores
// does not also wait for them), and thread t < NB waits until flag t carries
// the tag or a later one (a workgroup can be one barrier ahead, never two).
// Returns false when a wait gave up.
template <class Pf>
__device__ __forceinline__ bool wide_barrier(const PersistArgs &a, uint32_t tag, int *fail, Pf pf) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) tput(a.wflags + blockIdx.x * kWFlagStride, 0.f, tag);
  pf();
  bool ok = *fail == 0;
  if (threadIdx.x < NB && ok) {
    for (unsigned spins = 0;; spins++) {
      const uint64_t w = tload(a.wflags + threadIdx.x * kWFlagStride);
      if ((uint32_t)(w >> 32) >= tag) break;
      if (spin_fail(a, spins)) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  if (!ok) *fail = 1;
  __syncthreads();
  return *fail == 0;
}

// n floats of a device-coherent buffer into LDS, every load issued first
// (n <= 8 NT)
__device__ __forceinline__ void cload_vec(float *dst, const float *src, int n, int tid) {
  const __amdgpu_buffer_rsrc_t rs = crsrc(src);
  float v[8];
#pragma unroll
  for (int u = 0; u < 8; u++) {
    const int i = tid + u * NT;
    v[u] = cld(rs, i < n ? i : 0);
  }
#pragma unroll
  for (int u = 0; u < 8; u++) {
    const int i = tid + u * NT;
    if (i < n) dst[i] = v[u];
  }
}

// a batch of WRB consecutive rows from `row` (clamped to `last`), 8 columns
// per chunk per lane; every load is issued on every path
template <int C>
__device__ __forceinline__ void wld(u32x4 (&t)[WRB][C], const uint16_t *W, int k, int row, int last,
                                    int lane) {
#pragma unroll
  for (int rb = 0; rb < WRB; rb++) ldrow_all<C>(t[rb], W, k, row + rb, last, lane);
}

// this lane's chunks of x (chunk lane + 64 i, 8 floats each) from LDS as
// 16-byte reads (x is 16-byte aligned)
template <int C>
__device__ __forceinline__ void wload_x(float4 (&xr)[C][2], const float *x, int k, int lane) {
  const int nch = k >> 3;
  const float4 *x4 = (const float4 *)__builtin_assume_aligned(x, 16);
  if (nch == 64 * C) {  // every lane holds C whole chunks: no guards
#pragma unroll
    for (int i = 0; i < C; i++) {
      const int c = lane + i * 64;
      xr[i][0] = x4[2 * c];
      xr[i][1] = x4[2 * c + 1];
    }
    return;
  }
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < C; i++) {
    const int c = lane + i * 64;
    xr[i][0] = c < nch ? x4[2 * c] : z;
    xr[i][1] = c < nch ? x4[2 * c + 1] : z;
  }
}

// RMSNorm of x (LDS, k floats) into this lane's chunks (lane + 64 i), f32;
// the bf16 gains g in global memory or LDS. Returns the 1 / rms factor
template <int C>
__device__ __forceinline__ float wnorm(float4 (&xr)[C][2], const float *x, const uint16_t *g, int k,
                                      float eps, int lane) {
  wload_x<C>(xr, x, k, lane);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < C; i++) {
    const float4 p = xr[i][0], q = xr[i][1];
    ss += p.x * p.x + p.y * p.y + p.z * p.z + p.w * p.w + q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w;
  }
  const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)k + eps);
  const int nch = k >> 3;
  const bool full = nch == 64 * C;
#pragma unroll
  for (int i = 0; i < C; i++) {
    const int c = lane + i * 64;
    if (full || c < nch) {
      const u32x4 gw = *(const u32x4 *)(g + c * 8);
      xr[i][0] = make_float4(bf_lo(gw.x) * (xr[i][0].x * inv), bf_hi(gw.x) * (xr[i][0].y * inv),
                             bf_lo(gw.y) * (xr[i][0].z * inv), bf_hi(gw.y) * (xr[i][0].w * inv));
      xr[i][1] = make_float4(bf_lo(gw.z) * (xr[i][1].x * inv), bf_hi(gw.z) * (xr[i][1].y * inv),
                             bf_lo(gw.w) * (xr[i][1].z * inv), bf_hi(gw.w) * (xr[i][1].w * inv));
    }
  }
  return inv;
}

// Rows [r0, r1) of W [rows, k]: wave w takes the row pairs r0 + 2 (w + NW j).
// `pre` holds the wave's first pair, issued by the caller (before a
// barrier); each pair's dot products are followed at once by the next pair's
// loads into the same registers, so they are in flight during the epilogue
// and the other waves' work (eight waves keep about 112 KB requested per CU
// at the 7B shape, above the CU's intake rate times the memory latency).
// epi(row, y_row, y_row+1) runs on every lane of the wave; rows past r1 are
// skipped (their loads re-read row r1 - 1).
template <int C, class Epi>
__device__ __forceinline__ void wstream(u32x4 (&pre)[WRB][C], const uint16_t *W, int k, int r0, int r1,
                                        const float4 (&xr)[C][2], int wave, int lane, Epi epi) {
  if (r0 >= r1) return;
  const int nb = (r1 - r0 + 2 * NW - 1) / (2 * NW);
  for (int j = 0; j < nb; j++) {
    const int ra = r0 + 2 * (wave + NW * j);
    const float y0 = dotrow_x<C>(pre[0], xr, k, lane);
    const float y1 = dotrow_x<C>(pre[1], xr, k, lane);
    if (j + 1 < nb) wld<C>(pre, W, k, ra + 2 * NW, r1 - 1, lane);
    if (ra < r1) epi(ra, y0, ra + 1 < r1 ? y1 : 0.f);
  }
}

// gate/up tiles (a pair per wave) a workgroup owns; the rest are handed out
// by ticket, so workgroups whose loads come in faster take more of them
__host__ __device__ inline int wide_gu_static(int I) {
  const int t = (3 * ((2 * I + 2 * NW - 1) / (2 * NW))) / (4 * NB);
  return t > 1 ? t : 1;
}

// Rows of W [rows, k] in tiles of 2 NW rows, wave w taking rows 2w, 2w + 1 of
// a tile: first this workgroup's tiles [t0, t0 + ns) (ns >= 1; `pre` holds
// tile t0's pair; rows past `rows` are read clamped and skipped), then tile
// dyn0 + i for each ticket base + i (i < ndyn)
// that thread 0 draws from *tick. A ticket is drawn one tile ahead, so its
// round trip overlaps a tile's loads; thread 0 posts the tile in tile_s
// (two slots, alternating) for the other waves. Each workgroup draws exactly
// one ticket past the last tile, so a pass advances the counter by
// ndyn + NB. epi(row, y_row, y_row+1) runs on every lane of the wave.
template <int C, class Epi>
__device__ __forceinline__ void wstream_tiles(u32x4 (&pre)[WRB][C], const uint16_t *W, int k, int rows,
                                              int t0, int ns, int dyn0, int ndyn, uint32_t *tick,
                                              uint32_t base, int *tile_s, const float4 (&xr)[C][2],
                                              int wave, int lane, int tid, Epi epi) {
  int cur = t0, left = ns, slot = 0;
  uint32_t tk = 0;
  if (ns == 1 && tid == 0) tk = __hip_atomic_fetch_add(tick, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    const int ra = cur * 2 * NW + 2 * wave;
    const float y0 = dotrow_x<C>(pre[0], xr, k, lane);
    const float y1 = dotrow_x<C>(pre[1], xr, k, lane);
    int nxt;
    if (left > 1) {
      nxt = cur + 1;
    } else {
      if (tid == 0) {
        const uint32_t i = tk - base;
        tile_s[slot] = i < (uint32_t)ndyn ? dyn0 + (int)i : -1;
      }
      __syncthreads();
      nxt = __builtin_amdgcn_readfirstlane(tile_s[slot]);
      slot ^= 1;
    }
    if (nxt >= 0) {
      wld<C>(pre, W, k, nxt * 2 * NW + 2 * wave, rows - 1, lane);
      if (left <= 2 && tid == 0)
        tk = __hip_atomic_fetch_add(tick, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (ra < rows) epi(ra, y0, ra + 1 < rows ? y1 : 0.f);
    if (nxt < 0) break;
    cur = nxt;
    left--;
  }
}

// first pair of the wave's rows in [r0, r1) into `pre`. Every load is issued:
// an empty range reads at byte offset 2^31, past the descriptor's range
// (zeros, no traffic), so the count of loads in flight after it does not
// depend on the range and the compiler's waits on earlier loads stay exact.
template <int C>
__device__ __forceinline__ void wpre(u32x4 (&pre)[WRB][C], const uint16_t *W, int k, int r0, int r1,
                                     int wave, int lane) {
  const int nch = k >> 3;
  const __amdgpu_buffer_rsrc_t rs = wrsrc(W);
#pragma unroll
  for (int rb = 0; rb < WRB; rb++) {
    const int soff = r0 < r1 ? min(r0 + 2 * wave + rb, r1 - 1) * k * 2 : (int)0x80000000u;
#pragma unroll
    for (int i = 0; i < C; i++) {
      const int c = min(lane + i * 64, nch - 1);
      pre[rb][i] = __builtin_amdgcn_raw_buffer_load_b128(rs, c * 16, soff, 2);
    }
  }
}

// a down row pair: each thread's WDC chunks (tid + NT i) of rows `row`,
// `row` + 1 (clamped to `last`, chunks clamped to the row)
__device__ __forceinline__ void dld(u32x4 (&t)[2][WDC], const uint16_t *W, int k, int row, int last,
                                    int tid) {
  const int nch = k >> 3;
  const __amdgpu_buffer_rsrc_t rs = wrsrc(W);
#pragma unroll
  for (int rb = 0; rb < 2; rb++) {
    const int soff = min(row + rb, last) * k * 2;
#pragma unroll
    for (int i = 0; i < WDC; i++) {
      const int c = min(tid + i * NT, nch - 1);
      t[rb][i] = __builtin_amdgcn_raw_buffer_load_b128(rs, c * 16, soff, 2);
    }
  }
}
__device__ __forceinline__ float ddot(const u32x4 (&w)[WDC], const float4 (&hr)[WDC][2]) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < WDC; i++) {
    const u32x4 q = w[i];
    const float4 a = hr[i][0], b = hr[i][1];
    s = fmaf(bf_lo(q.x), a.x, s);
    s = fmaf(bf_hi(q.x), a.y, s);
    s = fmaf(bf_lo(q.y), a.z, s);
    s = fmaf(bf_hi(q.y), a.w, s);
    s = fmaf(bf_lo(q.z), b.x, s);
    s = fmaf(bf_hi(q.z), b.y, s);
    s = fmaf(bf_lo(q.w), b.z, s);
    s = fmaf(bf_hi(q.w), b.w, s);
  }
  return s;
}

template <int C, bool KB>
__global__ void __launch_bounds__(NT) decode_wide_kernel(PersistArgs a) {
  extern __shared__ float4 wsm4[];
  float *xs = (float *)wsm4;   // [WXMAX] the phase's input vector
  float *big = xs + WXMAX;     // attention staging / merge partials / argmax partials
  uint16_t *gn_s = (uint16_t *)(big + wide_big_floats(a.d, a.max_seq));  // [WXMAX] next RMSNorm gains
  // the layer table, copied to LDS once (a pointer read from global memory
  // would be a vector load, and its wait would also wait for the weight loads
  // in flight); layer(l) gives its pointers in scalar registers
  PersistLayer *lay = (PersistLayer *)(gn_s + WXMAX);
  __shared__ float xl[WMR];    // this workgroup's down rows of the residual stream
  __shared__ float xol[WOR];   // the residual at its o rows
  __shared__ float red[NW][WMR];
  __shared__ int fail_s;
  __shared__ uint32_t tok_s;
  __shared__ float2 best_s[NW];
  __shared__ float qb_s[WQP];      // this workgroup's QKV biases, loaded ahead
  __shared__ float2 qcs_s[WQP / 2];  // RoPE (cos, sin) of its pairs at the step's position
  __shared__ int last_s;
  __shared__ int tile_s[2];
  __shared__ float2 red2_s[NW];

  // tid and lane are re-derived at the top of every step and layer (see
  // opaque), so per-lane addresses are not hoisted out of the loops and held
  // in registers (spilled) for the whole launch
  int tid = threadIdx.x, lane = tid & 63;
  const int wg = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, I = a.I, V = a.V, d = a.d, nq = a.nq, nkv = a.nkv;
  const int half = d >> 1, gq = nq / nkv, qdim = nq * d, kvdim = nkv * d;
  const int qkv_rows = qdim + 2 * kvdim;
  const uint32_t TPS = (uint32_t)a.L * kTPL + 2;
  const int nchmax = (a.max_seq + AC - 1) / AC;
  const WideBufs B = wide_bufs(a.wide, H, I, nq, d, a.max_seq, nullptr);
  // ownership: QKV row pairs, residual rows (o and down), gate/up row pairs,
  // head rows
  const int qper = 2 * ((qkv_rows + 2 * NB - 1) / (2 * NB));
  const int q0 = min(wg * qper, qkv_rows), q1 = min(q0 + qper, qkv_rows);
  const int xper = (H + NB - 1) / NB;
  const int x0 = min(wg * xper, H), x1 = min(x0 + xper, H), nx = x1 - x0;
  // o rows: when the attention items fit in the first quarter of the grid,
  // those workgroups hold none, so nothing but their item waits on their loads
  const int ow0 = wide_item_wgs(nkv, nchmax);
  const int oper = (H + (NB - ow0) - 1) / (NB - ow0);
  const int o0r = wg < ow0 ? H : min((wg - ow0) * oper, H), o1r = min(o0r + oper, H);
  // gate/up: static tiles of 2 NW rows, then tiles by ticket
  const int gns = wide_gu_static(I), gtiles = (2 * I + 2 * NW - 1) / (2 * NW);
  const int gdyn0 = NB * gns, gndyn = max(gtiles - gdyn0, 0);
  const int g0 = min(wg * gns * 2 * NW, 2 * I), g1 = min(g0 + gns * 2 * NW, 2 * I);
  const int vper = (V + NB - 1) / NB;
  const int v0 = min(wg * vper, V), v1 = min(v0 + vper, V);
  // biases and RoPE factors of this workgroup's QKV rows for layer l at
  // position p, into LDS ahead of the phase (the epilogue then loads nothing)
  auto gains_ld = [&](const uint16_t *g) {
    return __builtin_amdgcn_raw_buffer_load_b128(gsrc(g), tid < (H >> 3) ? tid * 16 : 0x7fffffff, 0, 0);
  };
  auto layer = [&](int l) {
    const PersistLayer &q = lay[l];
    PersistLayer p;
    p.ln1 = uni(q.ln1);
    p.wqkv = uni(q.wqkv);
    p.wo = uni(q.wo);
    p.ln2 = uni(q.ln2);
    p.wgu = uni(q.wgu);
    p.wd = uni(q.wd);
    p.bqkv = uni(q.bqkv);
    p.wdp = nullptr;
    return p;
  };
  struct Consts {
    float b;
    float2 cs;
    u32x4 g;
  };
  // loads of layer l's constants at position p: this thread's QKV bias and
  // RoPE pair, and its 8 RMSNorm gains (ln1); consts_st puts them in LDS, so
  // the loads can go out ahead of a phase's weight loads
  auto consts_ld = [&](int l, uint32_t p) {
    // buffer loads: an offset past the range (2^31) reads 0 and fetches nothing
    Consts c;
    const int r = q0 + 2 * tid;
    const int ib = tid < q1 - q0 ? (q0 + tid) * 4 : 0x7fffffff;
    const int ir = tid < (q1 - q0) / 2 && r < qdim + kvdim
                       ? (int)(((size_t)p * half + (((r < qdim ? r : r - qdim) >> 1) % half)) * 8)
                       : 0x7fffffff;
    c.b = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(gsrc(uni(lay[l].bqkv)), ib, 0, 0));
    const u32x2 cs = __builtin_amdgcn_raw_buffer_load_b64(gsrc(a.rope), ir, 0, 0);
    c.cs = ir == 0x7fffffff ? make_float2(1.f, 0.f) : make_float2(__uint_as_float(cs.x), __uint_as_float(cs.y));
    c.g = gains_ld(uni(lay[l].ln1));
    return c;
  };
  auto consts_st = [&](const Consts &c) {
    if (tid < q1 - q0) qb_s[tid] = c.b;
    if (tid < (q1 - q0) / 2) qcs_s[tid] = c.cs;
    if (tid < (H >> 3)) *(u32x4 *)(gn_s + tid * 8) = c.g;
  };

  auto gains_st = [&](const u32x4 &g) {
    if (tid < (H >> 3)) *(u32x4 *)(gn_s + tid * 8) = g;
  };
  for (int i = tid; i < a.L * (int)(sizeof(PersistLayer) / 8); i += NT)
    ((uint64_t *)lay)[i] = ((const uint64_t *)a.layers)[i];
  if (tid == 0) fail_s = 0;
  if (tid < WMR) xl[tid] = 0.f;
  // the ticket counter starts at 0; the first barrier orders this store
  // before every draw
  if (wg == 0 && tid == 0) __hip_atomic_store(B.tick, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();

  u32x4 pre[WRB][C];          // the next wave-row phase's first pair
  u32x4 dpre[2][WDC];         // the down phase's first pair
  wpre<C>(pre, uni(lay[0].wqkv), H, q0, q1, wave, lane);

  for (uint32_t s = 0; s < a.steps; s++) {
    tid = opaque(tid);
    lane = tid & 63;
    const uint32_t pos = a.pos0 + s;
    const int seq = (int)pos + 1;
    const uint32_t tstep = a.tag_base + s * TPS;

    // ---- token: argmax of the previous logits; embedding row -----------------
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
      } else if (tid < NB) {
        const __amdgpu_buffer_rsrc_t rs = crsrc(B.arg);
        bv = cld(rs, 2 * tid);
        bi = __float_as_uint(cld(rs, 2 * tid + 1));
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
          if (beats(best_s[w].x, __float_as_uint(best_s[w].y), b.x, __float_as_uint(b.y))) b = best_s[w];
        const uint32_t idx = __float_as_uint(b.y);
        const uint32_t best = idx < (uint32_t)V ? idx : 0u;  // no candidate (all NaN / -inf) -> 0
        if (wg == 0) a.out_ids[s] = best;
        tok_s = a.force ? a.force[s] : best;  // teacher forcing feeds the given id
        if (wg == 0 && s + 1 == a.steps) a.state[1] = tok_s;
      }
      __syncthreads();
      const uint16_t *erow = a.embed + (size_t)tok_s * H;
      for (int j = tid; j < H; j += NT) xs[j] = bf16f(erow[j]);
      if (tid < nx) xl[tid] = bf16f(erow[x0 + tid]);
      consts_st(consts_ld(0, pos));
      __syncthreads();
    }

    for (int l = 0; l < a.L; l++) {
      tid = opaque(tid);
      lane = tid & 63;
      const PersistLayer Ly = layer(l);
      const uint32_t T = tstep + (uint32_t)l * kTPL;
      constexpr int kvb = KB ? 2 : 4;
      uint8_t *kc = (uint8_t *)a.kc + (size_t)l * a.layer_kv * kvb;
      uint8_t *vc = (uint8_t *)a.vc + (size_t)l * a.layer_kv * kvb;

      // ---- QKV + bias + RoPE + KV store ----------------------------------------
      {
        // one row pair past a pair per wave (18 rows at the 7B shape) is
        // split by columns over the waves instead of a second round trip on
        // wave 0: wave w takes chunks [w spc, (w + 1) spc), loaded before x;
        // rows past the split read at byte offset 2^31 (zeros, no traffic)
        const int qs1 = min(q1, q0 + 2 * NW), nsp = q1 - qs1;
        const bool split = nsp > 0 && nsp <= 2;
        const int nchh = H >> 3, spc = (nchh + NW - 1) / NW, sc = wave * spc + lane;
        const bool sl = split && lane < spc && sc < nchh;
        const __amdgpu_buffer_rsrc_t rsq = wrsrc(Ly.wqkv);
        const u32x4 sw0 =
            __builtin_amdgcn_raw_buffer_load_b128(rsq, sc * 16, sl ? qs1 * H * 2 : (int)0x80000000u, 2);
        const u32x4 sw1 =
            __builtin_amdgcn_raw_buffer_load_b128(rsq, sc * 16, sl ? (q1 - 1) * H * 2 : (int)0x80000000u, 2);
        if (l > 0) cload_vec(xs, B.x, H, tid);
        __syncthreads();
        if (tid < o1r - o0r) xol[tid] = xs[o0r + tid];
        float4 xr[C][2];
        const float inv = wnorm<C>(xr, xs, gn_s, H, a.eps, lane);
        auto qepi = [&](int r, float y0, float y1) {
          if (lane != 0) return;
          const float b0 = y0 + qb_s[r - q0], b1 = y1 + qb_s[r - q0 + 1];
          if (r < qdim + kvdim) {
            const bool is_q = r < qdim;
            const int qu = (is_q ? r : r - qdim) >> 1, head = qu / half, p = qu - head * half;
            const float2 cs = qcs_s[(r - q0) >> 1];
            const float o0 = b0 * cs.x - b1 * cs.y, o1 = b1 * cs.x + b0 * cs.y;
            if (is_q) {
              cstore(B.q + head * d + p, o0);
              cstore(B.q + head * d + p + half, o1);
            } else {
              const size_t base = ((size_t)head * a.max_seq + pos) * d;
              kvstore<KB>(kc, base + p, o0);
              kvstore<KB>(kc, base + p + half, o1);
            }
          } else {
            const int rr = r - qdim - kvdim, head = rr / d, j = rr - head * d;
            const size_t base = ((size_t)head * a.max_seq + pos) * d + j;
            kvstore<KB>(vc, base, b0);
            kvstore<KB>(vc, base + 1, b1);
          }
        };
        wstream<C>(pre, Ly.wqkv, H, q0, split ? qs1 : q1, xr, wave, lane, qepi);
        if (split) {
          float p0 = 0.f, p1 = 0.f;
          if (sl) {
            const float4 *x4 = (const float4 *)__builtin_assume_aligned(xs, 16);
            const u32x4 gw = *(const u32x4 *)(gn_s + sc * 8);
            const float4 a0 = x4[2 * sc], a1 = x4[2 * sc + 1];
            const float xv[8] = {bf_lo(gw.x) * (a0.x * inv), bf_hi(gw.x) * (a0.y * inv),
                                 bf_lo(gw.y) * (a0.z * inv), bf_hi(gw.y) * (a0.w * inv),
                                 bf_lo(gw.z) * (a1.x * inv), bf_hi(gw.z) * (a1.y * inv),
                                 bf_lo(gw.w) * (a1.z * inv), bf_hi(gw.w) * (a1.w * inv)};
            const uint32_t w0[4] = {sw0.x, sw0.y, sw0.z, sw0.w}, w1[4] = {sw1.x, sw1.y, sw1.z, sw1.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
              p0 = fmaf(bf_lo(w0[e]), xv[2 * e], p0);
              p0 = fmaf(bf_hi(w0[e]), xv[2 * e + 1], p0);
              p1 = fmaf(bf_lo(w1[e]), xv[2 * e], p1);
              p1 = fmaf(bf_hi(w1[e]), xv[2 * e + 1], p1);
            }
          }
          p0 = wave_sum(p0);
          p1 = wave_sum(p1);
          if (lane == 0) red2_s[wave] = make_float2(p0, p1);
          __syncthreads();
          if (tid == 0) {
            float y0 = 0.f, y1 = 0.f;
            for (int w = 0; w < NW; w++) {
              y0 += red2_s[w].x;
              y1 += red2_s[w].y;
            }
            qepi(qs1, y0, nsp > 1 ? y1 : 0.f);
          }
        }
      }

      // ---- attention partials for (kv head, chunk) items, merged by the last
      // item of each kv group -------------------------------------------------
      // Thread i = tid + u NT holds columns [4 j4, 4 j4 + 4) of position
      // t = i / dq of the chunk (dq = d / 4 lanes per position), K in
      // registers and V staged in LDS; a score is a dq-lane segmented sum; wave
      // h then takes q head h (softmax over the chunk, the V sum). The first
      // item's cached rows (positions before this step's) load ahead of the
      // barrier; this step's row (written by the QKV phase) after it.
      const int nch = (seq + AC - 1) / AC;
      const int dq = d >> 2, j4 = tid & (dq - 1);
      const int ld = __builtin_ctz(d), ldq = ld - 2;  // d is a power of two
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
          kc, (short)0, (int)(a.layer_kv * kvb), 0x00020000);
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
          vc, (short)0, (int)(a.layer_kv * kvb), 0x00020000);
      u32x4 kr[KV4], vr[KV4];
      // rows t in [tmin, tmax) of item it into kr / vr
      auto item_rows = [&](int it, int tmin, int tmax) {
        const int g = it % nkv, t0 = (it / nkv) * AC;
#pragma unroll
        for (int u = 0; u < KV4; u++) {
          const int t = (tid + u * NT) >> ldq;
          if (t >= tmin && t < tmax) {
            const uint32_t off = (uint32_t)((((size_t)g * a.max_seq + t0 + t) * d + j4 * 4) * kvb);
            if (KB) {
              const u32x2 k2 = __builtin_amdgcn_raw_buffer_load_b64(rk, off, 0, 16);
              const u32x2 v2 = __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 16);
              kr[u] = (u32x4){k2.x << 16, k2.x & 0xffff0000u, k2.y << 16, k2.y & 0xffff0000u};
              vr[u] = (u32x4){v2.x << 16, v2.x & 0xffff0000u, v2.y << 16, v2.y & 0xffff0000u};
            } else {
              kr[u] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 16);
              vr[u] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 16);
            }
          }
        }
      };
      // positions of item it: n; cached ones: nold (the last chunk ends at pos)
      auto item_n = [&](int it) { return min(AC, seq - (it / nkv) * AC); };
      auto item_nold = [&](int it) { return (it / nkv) == nch - 1 ? item_n(it) - 1 : item_n(it); };
#pragma unroll
      for (int u = 0; u < KV4; u++) {
        const u32x4 zero = {0u, 0u, 0u, 0u};
        kr[u] = zero;
        vr[u] = zero;
      }
      wide_barrier(a, T + W_QKV, &fail_s, [&] {
        if (wg < nkv * nch) item_rows(wg, 0, item_nold(wg));
      });

      for (int it = wg; it < nkv * nch; it += NB) {
        const int g = it % nkv, c = it / nkv;
        const int n = item_n(it);
        float *q_s = big;                 // [gq][d]
        float *v_s = q_s + WMAXQ * MAXD;  // [AC][d]
        float *p_s = v_s + AC * MAXD;     // [gq][AC] scaled scores -> weights
        if (it == wg) {
          item_rows(it, item_nold(it), n);
        } else {
#pragma unroll
          for (int u = 0; u < KV4; u++) {
            const u32x4 zero = {0u, 0u, 0u, 0u};
            kr[u] = zero;
            vr[u] = zero;
          }
          item_rows(it, 0, n);
        }
        {
          const __amdgpu_buffer_rsrc_t rq = crsrc(B.q);
          float qv[2];
#pragma unroll
          for (int u = 0; u < 2; u++) {
            const int i = tid + u * NT;
            qv[u] = cld(rq, i < gq * d ? g * gq * d + i : 0);
          }
#pragma unroll
          for (int u = 0; u < 2; u++) {
            const int i = tid + u * NT;
            if (i < gq * d) q_s[(i >> ld) * MAXD + (i & (d - 1))] = qv[u];
          }
        }
#pragma unroll
        for (int u = 0; u < KV4; u++) {
          const int t = (tid + u * NT) >> ldq;
          if (t < n)
            *(float4 *)(v_s + t * MAXD + j4 * 4) =
                make_float4(__uint_as_float(vr[u].x), __uint_as_float(vr[u].y),
                            __uint_as_float(vr[u].z), __uint_as_float(vr[u].w));
        }
        __syncthreads();
        const float scale = 1.0f / sqrtf((float)d);
        // every head's partial dot first (rows past gq read stale LDS and are
        // not stored), then the segmented sums over all heads at once
#pragma unroll
        for (int u = 0; u < KV4; u++) {
          const int t = (tid + u * NT) >> ldq;
          const float4 k4 = make_float4(__uint_as_float(kr[u].x), __uint_as_float(kr[u].y),
                                        __uint_as_float(kr[u].z), __uint_as_float(kr[u].w));
          float sc[WMAXQ];
#pragma unroll
          for (int h = 0; h < WMAXQ; h++) {
            const float4 q4 = *(const float4 *)(q_s + h * MAXD + j4 * 4);
            float v = q4.x * k4.x;
            v = fmaf(q4.y, k4.y, v);
            v = fmaf(q4.z, k4.z, v);
            sc[h] = fmaf(q4.w, k4.w, v);
          }
          seg_sum_n<WMAXQ>(sc, dq);
          if (t < n && seg_leader(lane, dq)) {
#pragma unroll
            for (int h = 0; h < WMAXQ; h++)
              if (h < gq) p_s[h * AC + t] = sc[h] * scale;
          }
        }
        __syncthreads();
        if (wave < gq) {
          const int h = wave;
          const float sc = lane < n ? p_s[h * AC + lane] : -INFINITY;
          const float mx = wave_max(sc);
          const float e = lane < n ? expf(sc - mx) : 0.f;
          const float lsum = wave_sum(e);
          if (lane < AC) p_s[h * AC + lane] = e;
          // lane l sums columns 2l and 2l + 1 (one 8-byte LDS read per position)
          const int c2 = 2 * lane < d ? 2 * lane : 0;
          float o0 = 0.f, o1 = 0.f;
          if (n == AC) {
#pragma unroll
            for (int t4 = 0; t4 < AC; t4 += 4) {
              const float4 e4 = *(const float4 *)(p_s + h * AC + t4);
              const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
              for (int k = 0; k < 4; k++) {
                const float2 v2 = *(const float2 *)(v_s + (t4 + k) * MAXD + c2);
                o0 = fmaf(ev[k], v2.x, o0);
                o1 = fmaf(ev[k], v2.y, o1);
              }
            }
          } else {
#pragma unroll
            for (int t4 = 0; t4 < AC; t4 += 4) {
              if (t4 < n) {
                const float4 e4 = *(const float4 *)(p_s + h * AC + t4);
                const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                  // rows past n hold stale LDS: masked, not just weighted by 0
                  const bool in = t4 + k < n;
                  const float2 v2 = *(const float2 *)(v_s + (t4 + k) * MAXD + c2);
                  o0 = fmaf(ev[k], in ? v2.x : 0.f, o0);
                  o1 = fmaf(ev[k], in ? v2.y : 0.f, o1);
                }
              }
            }
          }
          float *dst = B.part + ((size_t)(g * gq + h) * nchmax + c) * (d + 2);
          if (2 * lane < d) {
            cstore(dst + 2 * lane, o0);
            cstore(dst + 2 * lane + 1, o1);
          }
          if (lane == 0) {
            cstore(dst + d, mx);
            cstore(dst + d + 1, lsum);
          }
        }
        // count the item in once its partial stores have completed; the
        // group's last item merges the group's heads, wave h taking head h:
        // att = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c, chunks in order
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0)
          last_s = __hip_atomic_fetch_add(&B.cnt[g], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   nch - 1;
        __syncthreads();
        if (last_s) {
          for (int h = wave; h < gq; h += NW) {
            const int hh = g * gq + h, dd = d + 2;
            const __amdgpu_buffer_rsrc_t rp = crsrc(B.part + (size_t)hh * nchmax * dd);
            const int ja = lane < d ? lane : 0, jb = lane + 64 < d ? lane + 64 : 0;
            // a batch of 8 chunks' outputs per round trip, the first one
            // issued with the (m, l) pairs; chunks past nch read at byte
            // offset 2^31 (zeros, no traffic) and carry weight 0
            float v0[8], v1[8];
            auto batch = [&](int cb) {
#pragma unroll
              for (int u = 0; u < 8; u++) {
                const int cc = cb + u;
                v0[u] = cldb(rp, cc < nch ? (cc * dd + ja) * 4 : (int)0x80000000u);
                v1[u] = cldb(rp, cc < nch ? (cc * dd + jb) * 4 : (int)0x80000000u);
              }
            };
            const float m = lane < nch ? cld(rp, lane * dd + d) : -INFINITY;
            const float lw = lane < nch ? cld(rp, lane * dd + d + 1) : 0.f;
            batch(0);
            const float mx = wave_max(m);
            const float e = lane < nch ? expf(m - mx) : 0.f;
            const float inv = 1.0f / wave_sum(e * lw);
            float acc0 = 0.f, acc1 = 0.f;
            for (int cb = 0;;) {
#pragma unroll
              for (int u = 0; u < 8; u++) {
                const float ec = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), cb + u));
                acc0 = fmaf(ec, v0[u], acc0);
                acc1 = fmaf(ec, v1[u], acc1);
              }
              cb += 8;
              if (cb >= nch) break;
              batch(cb);
            }
            if (lane < d) cstore(B.att + hh * d + lane, acc0 * inv);
            if (lane + 64 < d) cstore(B.att + hh * d + lane + 64, acc1 * inv);
          }
          if (tid == 0) __hip_atomic_store(&B.cnt[g], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
      }
      // the o rows' loads (a workgroup with none takes its gate/up loads):
      // `pre` is then written on every path here, so it holds nothing live
      // through the attention items
      wide_barrier(a, T + W_ATT, &fail_s, [&] {
        const u32x4 g = gains_ld(Ly.ln2);
        asm volatile("" ::: "memory");  // the gains' load goes out first
        const bool has_o = o0r < o1r;
        wpre<C>(pre, has_o ? Ly.wo : Ly.wgu, has_o ? qdim : H, has_o ? o0r : g0, has_o ? o1r : g1, wave,
                lane);
        gains_st(g);
      });

      // ---- o projection + residual ------------------------------------------
      {
        cload_vec(xs, B.att, qdim, tid);
        __syncthreads();
        float4 xr[C][2];
        wload_x<C>(xr, xs, qdim, lane);
        wstream<C>(pre, Ly.wo, qdim, o0r, o1r, xr, wave, lane, [&](int r, float y0, float y1) {
          if (lane != 0) return;
          cstore(B.xo + r, xol[r - o0r] + y0);
          if (r + 1 < o1r) cstore(B.xo + r + 1, xol[r + 1 - o0r] + y1);
        });
      }
      wide_barrier(a, T + W_XO, &fail_s, [&] {
        if (o0r < o1r) wpre<C>(pre, Ly.wgu, H, g0, g1, wave, lane);
      });

      // ---- RMSNorm + gate/up + SwiGLU -------------------------------------------
      {
        cload_vec(xs, B.xo, H, tid);
        __syncthreads();
        if (tid < nx) xl[tid] = xs[x0 + tid];
        float4 xr[C][2];
        wnorm<C>(xr, xs, gn_s, H, a.eps, lane);
        const uint32_t tbase = (s * (uint32_t)a.L + (uint32_t)l) * (uint32_t)(gndyn + NB);
        wstream_tiles<C>(pre, Ly.wgu, H, 2 * I, wg * gns, gns, gdyn0, gndyn, B.tick, tbase, tile_s, xr,
                         wave, lane, tid, [&](int r, float y0, float y1) {
                           if (lane == 0) cstore(B.h + (r >> 1), silu(y0) * y1);
                         });
      }
      wide_barrier(a, T + W_H, &fail_s, [&] {
        if (nx > 0) dld(dpre, Ly.wd, I, x0, x1 - 1, tid);
      });

      // ---- down + residual: whole-workgroup rows, h slice in registers ---------
      {
        const int nchi = I >> 3;
        float4 hr[WDC][2];
        {
          const __amdgpu_buffer_rsrc_t rh = crsrc(B.h);
#pragma unroll
          for (int i = 0; i < WDC; i++) {
            const int c = tid + i * NT;
            const int cc = c < nchi ? c : 0;
            const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            const u32x4 p = __builtin_amdgcn_raw_buffer_load_b128(rh, cc * 32, 0, 16);
            const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rh, cc * 32 + 16, 0, 16);
            hr[i][0] = c < nchi ? make_float4(__uint_as_float(p.x), __uint_as_float(p.y),
                                              __uint_as_float(p.z), __uint_as_float(p.w)) : z;
            hr[i][1] = c < nchi ? make_float4(__uint_as_float(q.x), __uint_as_float(q.y),
                                              __uint_as_float(q.z), __uint_as_float(q.w)) : z;
          }
        }
        // row pair p from set A (even p, first one issued before the
        // barrier) or B (odd p), the next pair's loads issued before the
        // current pair's dot products; a compiler memory barrier after each
        // pair keeps later pairs' loads from being hoisted (which would hold
        // every pair in registers at once)
        u32x4 dn[2][WDC];
        auto pair = [&](int r, u32x4 (&cur)[2][WDC], u32x4 (&nxt)[2][WDC]) {
          if (r + 2 < nx) dld(nxt, Ly.wd, I, x0 + r + 2, x1 - 1, tid);
          const float y0 = wave_sum(ddot(cur[0], hr)), y1 = wave_sum(ddot(cur[1], hr));
          if (lane == 0) {
            red[wave][r] = y0;
            if (r + 1 < nx) red[wave][r + 1] = y1;
          }
          asm volatile("" ::: "memory");
        };
#pragma unroll
        for (int r = 0; r < WMR; r += 4) {
          if (r < nx) pair(r, dpre, dn);
          if (r + 2 < nx) pair(r + 2, dn, dpre);
        }
        __syncthreads();
        if (tid < nx) {
          float sum = 0.f;
#pragma unroll
          for (int w = 0; w < NW; w++) sum += red[w][tid];
          const float v = xl[tid] + sum;
          xl[tid] = v;
          cstore(B.x + x0 + tid, v);
        }
      }
      wide_barrier(a, T + W_X, &fail_s, [&] {
        if (l + 1 < a.L) {
          const Consts c = consts_ld(l + 1, pos);
          asm volatile("" ::: "memory");  // the constants' loads go out first
          wpre<C>(pre, uni(lay[l + 1].wqkv), H, q0, q1, wave, lane);
          consts_st(c);
        } else
          wpre<C>(pre, a.head, H, v0, v1, wave, lane);
      });
    }

    // ---- final norm + head + argmax partial (tag tstep + 6 L) --------------------
    const uint32_t TH = tstep + (uint32_t)a.L * kTPL;
    {
      cload_vec(xs, B.x, H, tid);
      __syncthreads();
      float4 xr[C][2];
      wnorm<C>(xr, xs, a.final_norm, H, a.eps, lane);
      if (wg == 0 && wave == 0) {
#pragma unroll
        for (int i = 0; i < C; i++) {
          const int c = lane + i * 64;
          if (c < (H >> 3)) {
            *(float4 *)(a.normed + c * 8) = xr[i][0];
            *(float4 *)(a.normed + c * 8 + 4) = xr[i][1];
          }
        }
      }
      float bv = -INFINITY;
      uint32_t bi = 0xffffffffu;
      wstream<C>(pre, a.head, H, v0, v1, xr, wave, lane, [&](int r, float y0, float y1) {
        if (lane == 0) a.logits[r] = y0;
        if (beats(y0, (uint32_t)r, bv, bi)) {
          bv = y0;
          bi = (uint32_t)r;
        }
        if (r + 1 < v1) {
          if (lane == 0) a.logits[r + 1] = y1;
          if (beats(y1, (uint32_t)(r + 1), bv, bi)) {
            bv = y1;
            bi = (uint32_t)(r + 1);
          }
        }
      });
      if (lane == 0) best_s[wave] = make_float2(bv, __uint_as_float(bi));
      __syncthreads();
      if (tid == 0) {
        float2 b = best_s[0];
        for (int w = 1; w < NW; w++)
          if (beats(best_s[w].x, __float_as_uint(best_s[w].y), b.x, __float_as_uint(b.y))) b = best_s[w];
        cstore(B.arg + 2 * wg, b.x);
        cstore(B.arg + 2 * wg + 1, b.y);
      }
    }
    wide_barrier(a, TH, &fail_s, [&] {
      if (s + 1 < a.steps) wpre<C>(pre, uni(lay[0].wqkv), H, q0, q1, wave, lane);
    });
  }

  // ---- hand the state back to the per-kernel path ---------------------------
  if (tid < nx) a.x_out[x0 + tid] = xl[tid];
  if (wg == 0) {
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    if (tid < NB) {
      const __amdgpu_buffer_rsrc_t rs = crsrc(B.arg);
      bv = cld(rs, 2 * tid);
      bi = __float_as_uint(cld(rs, 2 * tid + 1));
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
        if (beats(best_s[w].x, __float_as_uint(best_s[w].y), b.x, __float_as_uint(b.y))) b = best_s[w];
      best_s[0] = b;
      a.state[0] = a.pos0 + a.steps;
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
// down partials, [owner][source][rows per owner]: rows per owner are largest
// when head attention leaves NB - 2 nq workgroups to own them
size_t persist_pr_words(int H, int nq) {
  const int own = NB - 2 * nq > 0 ? NB - 2 * nq : NB;
  return (size_t)NB * NB * (size_t)((H + own - 1) / own);
}

bool persist_supported(int H, int I, int qdim, int d, int gq) {
  // H % 32: each wave's H / 8 down columns load 4 words a lane
  if (H % 32 || I % 8 || qdim % 8) return false;
  if (H > MAXH || qdim > MAXH || I > MAXI) return false;
  // the attention items sum a score over d / 4 lanes: d in {32, 64, 128}
  if ((d & (d - 1)) || d < 32 || d > MAXD || gq > 8) return false;
  // each workgroup's gate/up pairs fit GPMAX per wavefront, residual rows and
  // QKV pairs one per wavefront
  if (2 * ((I + 2 * NB - 1) / (2 * NB)) > GPMAX * NW) return false;
  if ((H + NB - 1) / NB > NW) return false;
  const int qkv_rows = qdim + 2 * (qdim / gq);
  if ((((qkv_rows + NB - 1) / NB) + 1) / 2 > NW) return false;
  return true;
}

// LDS bytes one workgroup needs: activations, the largest phase scratch
// (attention item staging, merge partials, argmax partials, h share), this
// workgroup's down column pairs and the layer table; sets the down block's
// offset in `a`
static bool persist_head_attention(const PersistArgs &a);

static size_t persist_lds(PersistArgs &a) {
  const int gq = a.nq / a.nkv;
  const size_t attn = (size_t)gq * a.d + a.d + (size_t)AC * a.d + (size_t)gq * AC;
  const int nchm = (a.max_seq + AC - 1) / AC;
  const size_t merge = (size_t)nchm * (a.d + 2) + nchm;
  int gst, gen;
  const bool ha = persist_head_attention(a);
  const int np = gu_share(a.I, a.nkv, nchm, a.nq, ha ? 2 * a.nq : 0, &gst, &gen);
  size_t big = attn;
  if (merge > big) big = merge;
  if ((size_t)2 * NB > big) big = 2 * NB;
  if ((size_t)np > big) big = np;
  const size_t xper = (size_t)(a.H + (NB - (ha ? 2 * a.nq : 0)) - 1) / (NB - (ha ? 2 * a.nq : 0));
  if (64 + NB * xper > big) big = 64 + NB * xper;  // h share, then the down partials
  // the h share sits in the 64 floats before the gathered partials (np is at
  // most GPMAX * NW = 40 on every supported shape; larger would not fit)
  if (np > 64) return kMaxLds + 1;
  const size_t wd_off = 2 * MAXH + ((big + 3) & ~(size_t)3);  // floats
  a.lds_wd = (int)wd_off;
  return wd_off * sizeof(float) + (size_t)NW * (np / 2) * (a.H / NW) * 4 +
         (size_t)a.L * sizeof(PersistLayer);
}

// LDS bytes of a head-attention workgroup (value half, q, k, the scores and
// its output), which it keeps where the others keep their down block
static size_t head_attention_lds(int kv_bf16) {
  return (size_t)256 * 64 * (kv_bf16 ? 2 : 4) + (128 + 128 + 256 + 64) * sizeof(float);
}

// Head attention (AM 2) runs on the Qwen2.5-1.5B instantiation when every
// position of the launch fits one workgroup's registers and LDS (max_seq <=
// 256) and the other 232 workgroups can hold the gate/up rows.
static bool persist_head_attention(const PersistArgs &a) {
  const bool qwen15 = a.H == 1536 && a.I == 8960 && a.V == 151936 && a.nq == 12 && a.nkv == 2 &&
                      a.d == 128;
  if (!qwen15 || a.max_seq > 256) return false;
  int gst, gen;
  const int np = gu_share(a.I, a.nkv, 0, a.nq, 2 * a.nq, &gst, &gen);
  if (np > GPMAX * NW) return false;
  return (size_t)NW * (np / 2) * (a.H / NW) * 4 >= head_attention_lds(a.kv_bf16);
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

// The instantiation a launch with these arguments runs, and its first-use
// set-up: the dynamic LDS limit, and the function's attributes, whose query
// loads the kernel's code object onto the device. Done once per
// instantiation; launch_decode_persistent does it on its first call, and
// persist_prepare lets a caller do it before it starts timing (a first
// launch otherwise spends about 6 ms of host time between a stream event
// recorded before it and the kernel's start).
static hipError_t persist_fn(const PersistArgs &a, const void **out) {
  const bool qwen15 = a.H == 1536 && a.I == 8960 && a.V == 151936 && a.nq == 12 && a.nkv == 2 &&
                      a.d == 128;
  const bool kb = a.kv_bf16 != 0;
  const bool ms = (a.max_seq + AC - 1) / AC > 16;
  const bool ha = persist_head_attention(a);
  const void *const fns[10] = {
      (const void *)decode_persistent_kernel<0, 0, 0, 0, 0, 0, false, 0>,
      (const void *)decode_persistent_kernel<0, 0, 0, 0, 0, 0, true, 0>,
      (const void *)decode_persistent_kernel<1536, 8960, 151936, 12, 2, 128, false, 0>,
      (const void *)decode_persistent_kernel<1536, 8960, 151936, 12, 2, 128, true, 0>,
      (const void *)decode_persistent_kernel<0, 0, 0, 0, 0, 0, false, 1>,
      (const void *)decode_persistent_kernel<0, 0, 0, 0, 0, 0, true, 1>,
      (const void *)decode_persistent_kernel<1536, 8960, 151936, 12, 2, 128, false, 1>,
      (const void *)decode_persistent_kernel<1536, 8960, 151936, 12, 2, 128, true, 1>,
      (const void *)decode_persistent_kernel<1536, 8960, 151936, 12, 2, 128, false, 2>,
      (const void *)decode_persistent_kernel<1536, 8960, 151936, 12, 2, 128, true, 2>};
  const int which = ha ? 8 + kb : 4 * ms + 2 * qwen15 + kb;
  const void *fn = fns[which];
  static bool attr_set[10] = {false, false, false, false, false, false, false, false, false, false};
  if (!attr_set[which]) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
    if (e != hipSuccess) return e;
    hipFuncAttributes fa;
    e = hipFuncGetAttributes(&fa, fn);
    if (e != hipSuccess) return e;
    attr_set[which] = true;
  }
  *out = fn;
  return hipSuccess;
}

hipError_t persist_prepare(const PersistArgs &a) {
  if (!persist_supported(a.H, a.I, a.nq * a.d, a.d, a.nq / a.nkv)) return hipErrorInvalidValue;
  const void *fn = nullptr;
  return persist_fn(a, &fn);
}

// An empty kernel, launched cooperatively with the decode kernels' grid: the
// runtime's own set-up for a stream's first cooperative launch (about 4 ms of
// host time before the kernel starts, measured on MI355X) then happens here.
__global__ void __launch_bounds__(NT) coop_warm_kernel() {}

hipError_t coop_warm_launch(hipStream_t s) {
  hipError_t e = hipLaunchCooperativeKernel((const void *)coop_warm_kernel, dim3(NB), dim3(NT), nullptr, 0, s);
  if (e != hipSuccess) return e;
  return hipStreamSynchronize(s);
}

hipError_t launch_decode_persistent(const PersistArgs &a, hipStream_t s) {
  if (!persist_supported(a.H, a.I, a.nq * a.d, a.d, a.nq / a.nkv)) return hipErrorInvalidValue;
  if (a.steps == 0) return hipSuccess;
  if (a.pos0 + a.steps > (uint32_t)a.max_seq) return hipErrorInvalidValue;
  PersistArgs args = a;
  const size_t smem = persist_lds(args);
  if (smem > kMaxLds) return hipErrorInvalidValue;
  const void *fn = nullptr;
  hipError_t e = persist_fn(args, &fn);
  if (e != hipSuccess) return e;
  void *params[] = {&args};
  return hipLaunchCooperativeKernel(fn, dim3(NB), dim3(NT), params, (unsigned)smem, s);
}


// ---- streamed cooperative decode: support and launch ---------------------------
static size_t wide_lds_bytes(int d, int max_seq) {
  return (WXMAX + wide_big_floats(d, max_seq) + WXMAX / 2) * sizeof(float) + WLMAX * sizeof(PersistLayer);
}

bool wide_supported(int H, int I, int qdim, int d, int gq, int max_seq) {
  // 8-column chunks; rows of at most 64 x 8 x 7 columns held in a wave,
  // down rows of at most 512 x 8 x WDC columns held in a workgroup
  if (H % 8 || I % 8 || qdim % 8) return false;
  if (H > 64 * 8 * 7 || qdim > 64 * 8 * 7 || I > NT * 8 * WDC || H > WXMAX) return false;
  if ((H + NB - 1) / NB > WMR) return false;
  // the attention items sum a score over d / 4 lanes: d in {32, 64, 128};
  // the merge takes a head's chunks one per lane; QKV rows per workgroup
  if ((d & (d - 1)) || d < 32 || d > MAXD || gq > WMAXQ) return false;
  if ((max_seq + AC - 1) / AC > WMCH) return false;
  const int qkv_rows = qdim + 2 * (qdim / gq);
  if (2 * ((qkv_rows + 2 * NB - 1) / (2 * NB)) > WQP || qdim / gq / d > WMAXQ * 64) return false;
  const int ow0 = wide_item_wgs(qdim / gq / d, (max_seq + AC - 1) / AC);
  if ((H + (NB - ow0) - 1) / (NB - ow0) > WOR) return false;
  return wide_lds_bytes(d, max_seq) <= kMaxLds - 2048;  // room for the static LDS
}

size_t wide_buffer_floats(int H, int I, int nq, int d, int max_seq) {
  size_t total = 0;
  (void)wide_bufs(nullptr, H, I, nq, d, max_seq, &total);
  return total;
}

bool wide_device_ok(const PersistArgs &a) {
  if (!wide_supported(a.H, a.I, a.nq * a.d, a.d, a.nq / a.nkv, a.max_seq) || a.L > WLMAX) return false;
  int dev = 0, coop = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess) return false;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
  return coop != 0 && cus >= NB;
}

// the streamed kernel's instantiation for these arguments and its first-use
// set-up (as persist_fn)
static hipError_t wide_fn(const PersistArgs &a, const void **out) {
  const size_t smem = wide_lds_bytes(a.d, a.max_seq);
  const bool narrow = a.H <= 64 * 8 * 3 && a.nq * a.d <= 64 * 8 * 3;
  const bool kb = a.kv_bf16 != 0;
  const void *const fns[4] = {(const void *)decode_wide_kernel<7, false>,
                              (const void *)decode_wide_kernel<7, true>,
                              (const void *)decode_wide_kernel<3, false>,
                              (const void *)decode_wide_kernel<3, true>};
  const int which = 2 * narrow + kb;
  // the dynamic LDS this launch needs (the kernel's static LDS comes on top
  // of it, within the 160 KB a workgroup can hold)
  static size_t attr_set[4] = {0, 0, 0, 0};
  if (attr_set[which] < smem) {
    hipError_t e = hipFuncSetAttribute(fns[which], hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return e;
    hipFuncAttributes fa;
    e = hipFuncGetAttributes(&fa, fns[which]);
    if (e != hipSuccess) return e;
    attr_set[which] = smem;
  }
  *out = fns[which];
  return hipSuccess;
}

hipError_t wide_prepare(const PersistArgs &a) {
  if (!wide_supported(a.H, a.I, a.nq * a.d, a.d, a.nq / a.nkv, a.max_seq)) return hipErrorInvalidValue;
  const void *fn = nullptr;
  return wide_fn(a, &fn);
}

hipError_t launch_decode_wide(const PersistArgs &a, hipStream_t s) {
  if (!wide_supported(a.H, a.I, a.nq * a.d, a.d, a.nq / a.nkv, a.max_seq)) return hipErrorInvalidValue;
  if (a.steps == 0) return hipSuccess;
  if (a.pos0 + a.steps > (uint32_t)a.max_seq) return hipErrorInvalidValue;
  const void *fn = nullptr;
  hipError_t e = wide_fn(a, &fn);
  if (e != hipSuccess) return e;
  const size_t smem = wide_lds_bytes(a.d, a.max_seq);
  PersistArgs args = a;
  void *params[] = {&args};
  return hipLaunchCooperativeKernel(fn, dim3(NB), dim3(NT), params, (unsigned)smem, s);
}

}  // namespace myos
