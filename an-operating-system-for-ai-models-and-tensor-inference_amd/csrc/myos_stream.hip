// Streamed persistent greedy-decode kernel for MI355X (gfx950): the
// alternative to myos_persistent.hip, selected with MYOS_PERSIST_KERNEL=stream.
//
// One cooperative launch of 256 workgroups (one per CU) runs a whole
// greedy_decode call. Each workgroup splits its waves by role so that no wave
// that waits for a cross-workgroup input has weight loads queued in front of
// that wait:
//
//  * two loader waves stream the workgroup's weight bytes, in the exact order
//    the consumers use them (q/k/v, o, gate/up, down of every layer, then the
//    head, then the next step), into an LDS ring of 1 KB slots with direct
//    (global_load_lds) loads. One wave's direct loads top out near 4 TB/s
//    chip-wide; two reach ~7 TB/s.
//  * six consumer waves own the workgroup's rows, read them from the ring and
//    reduce; they issue no global loads at all, only stores.
//  * one poller wave does the cross-workgroup gathers (residual stream,
//    attention output, last step's argmax), the RMSNorms, and the reduction
//    of the down partials of this workgroup's residual rows; it hands inputs
//    to the consumers through LDS flags.
//  * one attention wave runs the decode-attention items (one q head over a
//    32-position chunk) and the per-head merge.
//
// The down projection is split by columns: workgroup c owns gate/up pairs
// [c*hp, (c+1)*hp) and multiplies its own h values with the matching columns
// of down (stored transposed at load time), so h never leaves the workgroup;
// the workgroup that owns a residual row reduces its 256 partials in a fixed
// order.
//
// Measured on MI355X it is slower than myos_persistent.hip (~100 us vs ~37 us
// per layer of the 1.5B shape): the ring is bounded by LDS (~86 slots), which
// must hold the loads in flight, the consumers' working span and any buffer
// for dependency stalls, so HBM idles through most of each layer's exchange
// chain; and a single-wave gather or attention item is slower than the
// 512-thread ones of the first kernel.
//
// Activations cross workgroups as 64-bit (value, tag) words written and read
// device-coherently (sc1); the tag names the step, layer and phase. Every wait
// is bounded: after ~1 s a wave raises the error word and every wait gives up,
// so the grid always drains.
//
// Numerics follow forward_token (crates/model_core/src/qwen25_block.rs:
// 220-304) per step of greedy_decode (:765-780), with f32 accumulation in
// this kernel's own summation order.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "myos_internal.h"

namespace myos {
namespace {

constexpr int NS = 6;              // consumer waves
constexpr int NL = 2;              // loader waves (one wave's direct loads cap near 4 TB/s)
constexpr int WAVE_L = NS, WAVE_P = NS + NL;  // the attention wave follows the poller
constexpr int NT = 64 * (NS + NL + 2);  // threads per workgroup
constexpr int NB = 256;            // workgroups (one per CU)
constexpr int SLOT = 512;          // bf16 columns per slot
constexpr int MAXP = 3;            // slots per row: k <= 1536
constexpr int MAXK = MAXP * SLOT;  // padded row length of the LDS vectors
constexpr int AC = 32;             // positions per attention work item
constexpr int MAXD = 128;          // head_dim limit
constexpr int MAXHP = 64;          // gate/up pairs per workgroup
constexpr int MAXXR = 8;           // residual rows per workgroup
constexpr int MAXPQ = 8;           // q/k/v row pairs per workgroup
constexpr unsigned kSpinMax = 1u << 20;
constexpr uint32_t kTPL = 6;       // tags per layer
constexpr uint32_t P_QKV = 0, P_PART = 1, P_ATT = 2, P_XO = 3, P_PD = 4, P_XD = 5;
constexpr int kAuxCoherent = 16 | (1 << 31);  // sc1, volatile
constexpr size_t kMaxLds = 160 * 1024;
// s_waitcnt lgkmcnt(0) alone (gfx9 encoding: vmcnt and expcnt at their maxima)
constexpr int kLgkm0 = 0xC07F;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
__device__ __forceinline__ float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ float silu(float z) { return z / (1.0f + expf(-z)); }

// Cross-lane reductions with DPP lane moves. gfx9 DPP controls: quad_perm
// [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, row_half_mirror 0x141, row_mirror
// 0x140, row_bcast:15 0x142, row_bcast:31 0x143. Rows outside ROW_MASK keep
// `old`, the identity of the reduction.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float v, float old) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL,
                                                    ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v, 0.f);
  v += dpp<0x4E>(v, 0.f);
  v += dpp<0x141>(v, 0.f);
  v += dpp<0x140>(v, 0.f);
  v += dpp<0x142, 0xA>(v, 0.f);
  v += dpp<0x143, 0xC>(v, 0.f);
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

// greedy_token's order (crates/model_core/src/lib.rs:157-167): larger value
// wins, ties go to the lower index, NaN never wins
__device__ __forceinline__ bool beats(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && v != -INFINITY && i < bi);
}

// ---- device-coherent exchange --------------------------------------------
__device__ __forceinline__ void tput(uint64_t *p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cstore(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// wave-uniform reads (readfirstlane): a branch on them is a scalar branch, so
// the waves' loop state stays in SGPRs
__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ bool err_raised(const PersistArgs &a) {
  return uni(__hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) != 0u;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)bytes, 0x00020000);
}

// ---- LDS hand-off between the waves of a workgroup ---------------------------
// LDS pointers carry address space 3 so every access is a ds_* instruction
// (a generic pointer would compile to flat accesses, which also count against
// vmcnt and so would wait for the streaming waves' weight loads).
typedef __attribute__((address_space(3))) float lf32;
typedef __attribute__((address_space(3))) f32x2 lf32x2;
typedef __attribute__((address_space(3))) f32x4 lf32x4;
typedef __attribute__((address_space(3))) uint32_t lu32;
typedef __attribute__((address_space(3))) uint8_t lu8;

// Flags only grow. A writer stores its data, then the flag; LDS operations of
// one wave complete in order, so a reader that sees the flag sees the data.
__device__ __forceinline__ void lds_flag_set(lu32 *f, uint32_t v) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  *(volatile lu32 *)f = v;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ void lds_flag_add(lu32 *f, uint32_t v) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __atomic_fetch_add(f, v, __ATOMIC_RELAXED);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

struct Lds {
  lf32 *xn, *att, *xn2, *xf;  // [MAXK] inputs of the q/k/v, o, gate/up, head phases;
                              // xf is xn (the next step's xn is written only
                              // after every workgroup's head is done)
  lf32 *xg;                   // [MAXK] the P wave's gathered (raw) vector
  lf32 *comb;                 // [NS][SLOT] down partials of the non-leading waves
  lf32 *hbuf;                 // [MAXHP] this workgroup's h values
  lf32 *xl;                   // [MAXXR] this workgroup's residual rows
  lf32 *bq;                   // [2 MAXPQ] q/k/v bias of this workgroup's rows
  lf32x2 *rope;               // [MAXD / 2] (cos, sin) at this step's position
  lf32 *qb, *pb, *kb, *vb;    // attention: q [MAXD], p [AC], K, V [AC][MAXD]
  lf32 *msc;                  // merge: [nchmax][d + 2]
  lf32x2 *best;               // [NS] head argmax per streaming wave
  lu32 *flag;                 // [16]
  lu32 *filled;               // [NL] loader k has landed its slots (i % NL == k)
                              // below filled[k]
  lu32 *cnext;                // [NS] consumer w has consumed every one of its
                              // slots below cnext[w]
  lu32 *ring;                 // [ring_slots][256] 1 KB weight slots
};
enum Flag { F_XN = 0, F_ATT, F_XN2, F_XF, C_H, C_COMB, C_HEAD, F_ABORT, F_NFLAGS = 16 };

__device__ __forceinline__ Lds carve(lu8 *base, int nchmax, int d, int ring_slots) {
  Lds s;
  lf32 *f = (lf32 *)base;
  s.xn = f;
  s.att = s.xn + MAXK;
  s.xn2 = s.att + MAXK;
  s.xf = s.xn;
  s.xg = s.xn2 + MAXK;
  s.comb = s.xg + MAXK;
  s.hbuf = s.comb + NS * SLOT;
  s.xl = s.hbuf + MAXHP;
  s.bq = s.xl + MAXXR;
  s.rope = (lf32x2 *)(s.bq + 2 * MAXPQ);
  s.qb = (lf32 *)(s.rope + MAXD / 2);
  s.pb = s.qb + MAXD;
  s.kb = s.pb + AC;
  s.vb = s.kb + AC * MAXD;
  s.msc = s.vb + AC * MAXD;
  s.best = (lf32x2 *)(s.msc + nchmax * (d + 2));
  s.flag = (lu32 *)(s.best + NS);
  s.filled = s.flag + F_NFLAGS;
  s.cnext = s.filled + NL;
  // the ring starts 1 KB-aligned past the rest
  const size_t off = (size_t)((lu8 *)(s.cnext + NS) - base);
  s.ring = (lu32 *)(base + ((off + 1023) & ~(size_t)1023));
  return s;
}
// LDS bytes without the ring
__host__ __device__ constexpr size_t lds_fixed_bytes(int nchmax, int d) {
  return sizeof(float) * (4 * MAXK + NS * SLOT + MAXHP + MAXXR + 2 * MAXPQ + MAXD + MAXD + AC +
                          2 * AC * MAXD + (size_t)nchmax * (d + 2) + 2 * NS + F_NFLAGS + NL + NS);
}
__host__ __device__ constexpr size_t lds_bytes(int nchmax, int d, int ring_slots) {
  return ((lds_fixed_bytes(nchmax, d) + 1023) & ~(size_t)1023) + 1024 * (size_t)ring_slots;
}

// wait for an LDS flag to reach `want`; false when the workgroup aborted
// (streaming waves: no global loads, so the bound raises the error word with
// a store only)
__device__ bool lds_wait(const PersistArgs &a, const Lds &s, int f, uint32_t want) {
  volatile lu32 *p = s.flag + f;
  volatile lu32 *ab = s.flag + F_ABORT;
  for (unsigned spins = 0; uni(*p) < want; spins++) {
    if (uni(*ab)) return false;
    if (spins > 64u * kSpinMax) {
      __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *ab = 1u;
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return true;
}
// the same for the P and A waves, which may also poll the global error word
__device__ bool lds_wait_global(const PersistArgs &a, const Lds &s, int f, uint32_t want) {
  volatile lu32 *p = s.flag + f;
  for (unsigned spins = 0; uni(*p) < want; spins++) {
    if ((spins & 63) == 63) {
      if (spins > kSpinMax) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (err_raised(a)) return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return true;
}

// ---- one-wave gathers of tagged words ------------------------------------------
// A poll loads every word the wave waits for, and repeats until all carry the
// tag; each word is 8-byte aligned, so a 16-byte load returns two whole words.
__device__ __forceinline__ bool spin_check(const PersistArgs &a, unsigned spins) {
  if ((spins & 63) != 63) return true;
  if (spins > kSpinMax) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return !err_raised(a);
}

constexpr int PC = MAXK / 64;  // words per lane of a linear gather (chunk)

// dst[0, n) <- src[0, n) once every word carries `tag`; lane l takes words
// [l C, l C + C), C even and C <= PC
__device__ bool pgather(const PersistArgs &a, const uint64_t *src, int n, int C, uint32_t tag,
                        lf32 *dst, int lane) {
  const __amdgpu_buffer_rsrc_t rs = rsrc(src, (size_t)n * 8);
  const int i0 = lane * C;
  for (unsigned spins = 0;; spins++) {
    u32x4 w[PC / 2];
    bool ready = true;
#pragma unroll
    for (int m = 0; m < PC / 2; m++) {
      const int i = i0 + 2 * m;
      if (2 * m < C && i < n) {
        w[m] = __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)i * 8u, 0, kAuxCoherent);
        ready = ready && w[m].y == tag && (i + 1 >= n || w[m].w == tag);
      }
    }
    if (__builtin_amdgcn_ballot_w64(!ready) == 0) {
#pragma unroll
      for (int m = 0; m < PC / 2; m++) {
        const int i = i0 + 2 * m;
        if (2 * m < C && i < n) {
          dst[i] = __uint_as_float(w[m].x);
          if (i + 1 < n) dst[i + 1] = __uint_as_float(w[m].z);
        }
      }
      return true;
    }
    if (!spin_check(a, spins)) return false;
    __builtin_amdgcn_s_sleep(1);
  }
}

// chunk per lane for a linear gather of n words
__device__ __forceinline__ int chunk_of(int n) { return ((n + 63) / 64 + 7) & ~7; }

__device__ __forceinline__ void mark(const PersistArgs &a, uint32_t s, int slot) {
  if (a.trace && s == a.trace_step && (threadIdx.x & 63) == 0)
    a.trace[(size_t)blockIdx.x * (5 * a.L + 3) + slot] = wall_clock64();
}

// ---- ownership -------------------------------------------------------------
struct Own {
  int P, Po;           // slots per row of a k = H and a k = q_dim row
  int pc0, pc1;        // q/k/v row pairs [pc0, pc1)
  int x0, x1;          // residual rows (o rows) [x0, x1)
  int g0, g1;          // gate/up pairs = h columns = down columns [g0, g1)
  int v0, v1;          // head rows [v0, v1)
};
__device__ __forceinline__ Own own_of(const PersistArgs &a, int c) {
  Own o;
  o.P = (a.H + SLOT - 1) / SLOT;
  o.Po = (a.nq * a.d + SLOT - 1) / SLOT;
  const int np = a.qkv_rows / 2, pq = (np + NB - 1) / NB;
  o.pc0 = min(c * pq, np);
  o.pc1 = min(o.pc0 + pq, np);
  const int xr = (a.H + NB - 1) / NB;
  o.x0 = min(c * xr, a.H);
  o.x1 = min(o.x0 + xr, a.H);
  const int hp = (a.I + NB - 1) / NB;
  o.g0 = min(c * hp, a.I);
  o.g1 = min(o.g0 + hp, a.I);
  const int vr = (a.V + NB - 1) / NB;
  o.v0 = min(c * vr, a.V);
  o.v1 = min(o.v0 + vr, a.V);
  return o;
}

// ---- the workgroup's slot stream -----------------------------------------------
// Phases of a layer: q/k/v pairs, o rows, gate/up pairs, down columns; after
// the last layer the head rows; then the next step. The workgroup's weight
// bytes of a phase are its units in order (a unit is a row pair, a row or a
// down column), each unit `rows` rows of P slots of 1 KB (512 columns, the
// last one partial). The loader streams every slot in this order; consumer
// wave w takes units w, w + NS, ... of the dot phases, and of down the slot
// (block) w % P of columns w / P, w / P + NS / P, ...
enum Ph { PH_QKV = 0, PH_O, PH_GU, PH_DOWN, PH_HEAD, PH_END };

struct Phase {
  uint32_t s;          // step
  int l, ph;           // layer, phase
  int nu, rows, P;     // units, rows per unit, slots per row
  int rowlen;          // columns of a row
  const uint8_t *m;    // the workgroup's first unit, first row
  uint32_t rowbytes;
};

__device__ __forceinline__ void phase_setup(const PersistArgs &a, const Own &o, Phase &f) {
  const PersistLayer *L = a.layers + f.l;
  const int H = a.H, qd = a.nq * a.d;
  const uint16_t *m = nullptr;
  f.rows = 1;
  f.rowlen = H;
  switch (f.ph) {
    case PH_QKV:
      m = L->wqkv + (size_t)2 * o.pc0 * H, f.nu = o.pc1 - o.pc0, f.rows = 2;
      break;
    case PH_O:
      m = L->wo + (size_t)o.x0 * qd, f.nu = o.x1 - o.x0, f.rowlen = qd;
      break;
    case PH_GU:
      m = L->wgu + (size_t)2 * o.g0 * H, f.nu = o.g1 - o.g0, f.rows = 2;
      break;
    case PH_DOWN:
      m = L->wdT + (size_t)o.g0 * H, f.nu = o.g1 - o.g0;
      break;
    default:  // PH_HEAD
      m = a.head + (size_t)o.v0 * H, f.nu = o.v1 - o.v0;
      break;
  }
  f.m = (const uint8_t *)m;
  f.P = (f.rowlen + SLOT - 1) / SLOT;
  f.rowbytes = (uint32_t)f.rowlen * 2u;
}
__device__ __forceinline__ void phase_next(const PersistArgs &a, Phase &f) {
  if (f.ph == PH_HEAD) {
    f.s++;
    f.l = 0;
    f.ph = f.s < a.steps ? PH_QKV : PH_END;
  } else if (f.ph == PH_DOWN) {
    if (f.l + 1 < a.L) {
      f.l++;
      f.ph = PH_QKV;
    } else {
      f.ph = PH_HEAD;
    }
  } else {
    f.ph++;
  }
}
__device__ __forceinline__ int phase_slots(const Phase &f) { return f.nu * f.rows * f.P; }

// ---- the loader wave --------------------------------------------------------------
// Its LDS accesses are inline assembly: the compiler would otherwise make
// every LDS access of this wave wait for all of its direct loads (they write
// LDS), and the loader tracks their completion itself with vmcnt.
__device__ __forceinline__ uint32_t lds_addr(const void __attribute__((address_space(3))) *p) {
  return (uint32_t)(uintptr_t)p;
}
__device__ __forceinline__ uint32_t asm_lds_read(uint32_t addr) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ void asm_lds_write(uint32_t addr, uint32_t v) {
  asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
// s_waitcnt vmcnt(N) alone (gfx9: vmcnt [3:0] and [15:14], expcnt [6:4],
// lgkmcnt [11:8])
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

constexpr int DMAX = 12;  // direct loads in flight per loader: enough for HBM
                          // bandwidth; more only lengthens the CU's memory
                          // queue, which every exchange poll waits behind

// smallest cnext over the consumer waves (lanes 0..NS-1 read one each)
__device__ __forceinline__ uint32_t min_cnext(uint32_t cnext0, int lane) {
  const uint32_t v = asm_lds_read(cnext0 + 4u * (uint32_t)(lane < NS ? lane : 0));
  uint32_t m = uni(v);
#pragma unroll
  for (int w = 1; w < NS; w++) m = min(m, (uint32_t)__builtin_amdgcn_readlane(v, w));
  return m;
}

// Loader k issues the slots i with i % NL == k, in order. After its c-th
// issue and a vmcnt(DMAX) wait, its slots k + j NL with j < c - DMAX have
// landed: it publishes filled[k] = k + (c - DMAX) NL.
__device__ __forceinline__ void loader_wave(const PersistArgs &a, const Own &o, const Lds &s,
                                            int k, int lane) {
  const uint32_t R = (uint32_t)a.ring_slots;
  const uint32_t filled0 = lds_addr(s.filled + k), cnext0 = lds_addr(s.cnext);
  const uint32_t abort0 = lds_addr(s.flag + F_ABORT);
  uint32_t i = 0, c = 0;  // stream index, slots issued by this loader
  uint32_t limit = R;     // slots below limit have a free ring position
  Phase f;
  f.s = 0, f.l = 0, f.ph = a.steps ? PH_QKV : PH_END;
  for (; f.ph != PH_END; phase_next(a, f)) {
    phase_setup(a, o, f);
    // one slot: row r of unit u, 512-column piece p
    auto issue = [&](int u, int r, int p) -> bool {
      const bool mine = i % NL == (uint32_t)k;
      const uint32_t at = i++;
      if (!mine) return true;
      if (at >= limit) {
        limit = min_cnext(cnext0, lane) + R;
        if (at >= limit) {
          // the ring is full: everything issued lands, then wait for space
          wait_vm<0>();
          if (lane == 0) asm_lds_write(filled0, k + c * NL);
          for (unsigned spins = 0;; spins++) {
            limit = min_cnext(cnext0, lane) + R;
            if (at < limit) break;
            if (uni(asm_lds_read(abort0))) return false;
            if ((spins & 255) == 255) {
              if (spins > 64u * kSpinMax)
                __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              if (err_raised(a)) {
                if (lane == 0) asm_lds_write(abort0, 1u);
                return false;
              }
            }
            __builtin_amdgcn_s_sleep(1);
          }
        }
      }
      // past the row's end a lane reads the row start (finite weights; the
      // consumers' inputs are zero there)
      const uint8_t *row = f.m + ((size_t)u * f.rows + r) * f.rowbytes;
      const int col = p * SLOT + lane * 8;
      const uint8_t *src = col < f.rowlen ? row + (size_t)col * 2 : row;
      __builtin_amdgcn_global_load_lds(
          (const void *)src,
          (__attribute__((address_space(3))) void *)(s.ring + (size_t)(at % R) * 256u), 16, 0,
          2 /* nt */);
      if (++c > (uint32_t)DMAX) {
        wait_vm<DMAX>();
        if (lane == 0) asm_lds_write(filled0, k + (c - DMAX) * NL);
      }
      return true;
    };
    if (f.ph == PH_DOWN) {
      // unit-major: consumer w takes block w % P of every (NS / P)-th column,
      // so the waves' slots of a round of NS columns are adjacent
      for (int u = 0; u < f.nu; u++)
        for (int p = 0; p < f.P; p++)
          if (!issue(u, 0, p)) return;
    } else {
      // round by round (NS units, one per consumer wave), slot q of every
      // unit of the round before slot q + 1: the waves stay a few slots apart
      const int spu = f.rows * f.P;
      for (int u0 = 0; u0 < f.nu; u0 += NS) {
        const int nw = min(NS, f.nu - u0);
        for (int q = 0; q < spu; q++)
          for (int wq = 0; wq < nw; wq++) {
            const int r = q >= f.P ? 1 : 0;
            if (!issue(u0 + wq, r, q - r * f.P)) return;
          }
      }
    }
  }
  wait_vm<0>();
  if (lane == 0) asm_lds_write(filled0, 0xffffffffu);
}

// ---- the consumer waves -------------------------------------------------------------
struct SState {
  float acc0, acc1;    // dot phases: the unit's two rows
  float dacc[8];       // down: this wave's partial of rows 512 (w % P) + 8 lane + e
  float bv;            // head argmax of this wave
  uint32_t bi;
};

__device__ __forceinline__ uint32_t epoch(const PersistArgs &a, uint32_t s, int l) {
  return s * (uint32_t)a.L + (uint32_t)l + 1u;
}
__device__ __forceinline__ uint32_t tagof(const PersistArgs &a, uint32_t s, int l, uint32_t ph) {
  return a.tag_base + s * ((uint32_t)a.L * kTPL + 2u) + (uint32_t)l * kTPL + ph;
}

// wait until slots [0, n) of the stream are in LDS; `seen` caches the last
// value read (the smallest loader watermark)
__device__ __forceinline__ uint32_t filled_min(const Lds &s) {
  uint32_t m = 0xffffffffu;
#pragma unroll
  for (int k = 0; k < NL; k++) m = min(m, uni(*(volatile lu32 *)(s.filled + k)));
  return m;
}
__device__ __forceinline__ bool wait_filled(const PersistArgs &a, const Lds &s, uint32_t n,
                                            uint32_t &seen) {
  if (seen >= n) return true;
  volatile lu32 *ab = s.flag + F_ABORT;
  for (unsigned spins = 0;; spins++) {
    seen = filled_min(s);
    if (seen >= n) break;
    if (uni(*ab)) return false;
    if (spins > 64u * kSpinMax) {
      __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *ab = 1u;
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return true;
}
// this lane's 16 bytes of slot i (in LDS)
__device__ __forceinline__ u32x4 slot_read(const Lds &s, uint32_t i, uint32_t R, int lane) {
  return *(const __attribute__((address_space(3))) u32x4 *)(s.ring + (size_t)(i % R) * 256u +
                                                              lane * 4);
}
// every slot of consumer w below n is consumed (its reads are done: they
// precede this store in the wave's LDS order)
__device__ __forceinline__ void publish_next(const Lds &s, int w, uint32_t n, int lane) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (lane == 0) *(volatile lu32 *)(s.cnext + w) = n;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// the unit u of phase f is done: reduce and publish
__device__ __forceinline__ void s_finish_unit(const PersistArgs &a, const Own &o, const Lds &s,
                                              const Phase &f, int u, int lane, SState &st) {
  const int qd = a.nq * a.d, kvd = a.nkv * a.d, half = a.d >> 1;
  switch (f.ph) {
    case PH_QKV: {
      const float y0 = wave_sum(st.acc0), y1 = wave_sum(st.acc1);
      st.acc0 = st.acc1 = 0.f;
      if (lane == 0) {
        const int row = 2 * (o.pc0 + u);  // permuted q/k/v row pair
        const uint32_t T = tagof(a, f.s, f.l, P_QKV);
        const float b0 = y0 + s.bq[2 * u], b1 = y1 + s.bq[2 * u + 1];
        if (row < qd + kvd) {
          // q or k: the pair is (p, p + d/2) of one head; rotate it
          const bool is_q = row < qd;
          const int rr = is_q ? row : row - qd;
          const int uu = rr >> 1, head = uu / half, p = uu - head * half;
          const f32x2 cs = s.rope[p];
          const float o0 = b0 * cs.x - b1 * cs.y, o1 = b1 * cs.x + b0 * cs.y;
          uint64_t *dst = is_q ? a.tq + head * a.d : a.tkv + head * a.d;
          tput(dst + p, o0, T);
          tput(dst + p + half, o1, T);
        } else {
          const int j = row - qd - kvd;
          tput(a.tkv + kvd + j, b0, T);
          tput(a.tkv + kvd + j + 1, b1, T);
        }
      }
      break;
    }
    case PH_O: {
      const float y = wave_sum(st.acc0);
      st.acc0 = 0.f;
      if (lane == 0) {
        const float xo = s.xl[u] + y;
        s.xl[u] = xo;
        __builtin_amdgcn_s_waitcnt(kLgkm0);  // the LDS row lands before the publish
        tput(a.txo + o.x0 + u, xo, tagof(a, f.s, f.l, P_XO));
      }
      break;
    }
    case PH_GU: {
      const float g = wave_sum(st.acc0), up = wave_sum(st.acc1);
      st.acc0 = st.acc1 = 0.f;
      if (lane == 0) {
        s.hbuf[u] = silu(g) * up;
        lds_flag_add(s.flag + C_H, 1u);
      }
      break;
    }
    default: {  // PH_HEAD
      const float y = wave_sum(st.acc0);
      st.acc0 = 0.f;
      const uint32_t row = (uint32_t)(o.v0 + u);
      if (lane == 0) a.logits[row] = y;
      if (beats(y, row, st.bv, st.bi)) {
        st.bv = y;
        st.bi = row;
      }
      break;
    }
  }
}

// number of consumer waves with down columns that are not the first wave of
// their block (w >= P); each adds one to C_COMB per layer
__device__ __forceinline__ int down_followers(const Own &o) {
  const int ncols = o.g1 - o.g0;
  int n = 0;
  for (int w = o.P; w < NS; w++) n += w / o.P < ncols;
  return n;
}

// this wave's down columns are done: the waves of each 512-row block are
// combined in a fixed order by the block's first wave (w < P), which
// publishes the workgroup's partial of every row of the block
__device__ __forceinline__ bool s_finish_down(const PersistArgs &a, const Own &o, const Lds &s,
                                              uint32_t step, int l, int w, int lane, SState &st) {
  const int P = o.P, piece = w % P, ncols = o.g1 - o.g0;
  const uint32_t e = epoch(a, step, l);
  if (w >= P) {
    lf32 *dst = s.comb + w * SLOT + lane * 8;
    *(lf32x4 *)dst = (f32x4){st.dacc[0], st.dacc[1], st.dacc[2], st.dacc[3]};
    *(lf32x4 *)(dst + 4) = (f32x4){st.dacc[4], st.dacc[5], st.dacc[6], st.dacc[7]};
    if (lane == 0) lds_flag_add(s.flag + C_COMB, 1u);
  } else {
    if (!lds_wait(a, s, C_COMB, e * (uint32_t)down_followers(o))) return false;
    for (int v = w + P; v < NS && v / P < ncols; v += P) {
      const lf32 *src = s.comb + v * SLOT + lane * 8;
      const f32x4 p0 = *(const lf32x4 *)src, p1 = *(const lf32x4 *)(src + 4);
      st.dacc[0] += p0.x;
      st.dacc[1] += p0.y;
      st.dacc[2] += p0.z;
      st.dacc[3] += p0.w;
      st.dacc[4] += p1.x;
      st.dacc[5] += p1.y;
      st.dacc[6] += p1.z;
      st.dacc[7] += p1.w;
    }
    const uint32_t T = tagof(a, step, l, P_PD);
    uint64_t *dst = a.tpd + (size_t)blockIdx.x * a.H;
    const int r0 = piece * SLOT + lane * 8;
#pragma unroll
    for (int e8 = 0; e8 < 8; e8++)
      if (r0 + e8 < a.H) tput(dst + r0 + e8, st.dacc[e8], T);
  }
#pragma unroll
  for (int e8 = 0; e8 < 8; e8++) st.dacc[e8] = 0.f;
  return true;
}

// a dot phase with P slots per row: the wave's slice of x stays in registers;
// two units per iteration, so one unit's LDS reads overlap the other's math
template <int P>
__device__ __forceinline__ bool dot_phase(const PersistArgs &a, const Own &o, const Lds &s,
                                          const Phase &f, uint32_t base, uint32_t end, int w,
                                          int lane, uint32_t &seen, SState &st) {
  const uint32_t R = (uint32_t)a.ring_slots;
  const lf32 *x = f.ph == PH_QKV ? s.xn : f.ph == PH_O ? s.att : f.ph == PH_GU ? s.xn2 : s.xf;
  f32x4 xr[P][2];
#pragma unroll
  for (int p = 0; p < P; p++) {
    xr[p][0] = *(const lf32x4 *)(x + p * SLOT + lane * 8);
    xr[p][1] = *(const lf32x4 *)(x + p * SLOT + lane * 8 + 4);
  }
  auto dot = [&](const u32x4 v, int p) {
    const f32x4 x0 = xr[p][0], x1 = xr[p][1];
    float d = bf_lo(v.x) * x0.x;
    d = fmaf(bf_hi(v.x), x0.y, d);
    d = fmaf(bf_lo(v.y), x0.z, d);
    d = fmaf(bf_hi(v.y), x0.w, d);
    d = fmaf(bf_lo(v.z), x1.x, d);
    d = fmaf(bf_hi(v.z), x1.y, d);
    d = fmaf(bf_lo(v.w), x1.z, d);
    d = fmaf(bf_hi(v.w), x1.w, d);
    return d;
  };
  const int rows = f.rows, spu = rows * P;
  for (int u = w; u < f.nu; u += 2 * NS) {
    // units u and u + NS (rounds u0 and u0 + NS): slot q of unit u0 + w of a
    // round of nw units sits at round start + q nw + w
    const int u0 = u - w, nw = min(NS, f.nu - u0);
    const bool two = u + NS < f.nu;
    const int nw2 = two ? min(NS, f.nu - u0 - NS) : 0;
    const uint32_t i0 = base + (uint32_t)(u0 * spu + w);
    const uint32_t i1 = base + (uint32_t)((u0 + NS) * spu + w);
    const uint32_t last = two ? i1 + (uint32_t)((spu - 1) * nw2) : i0 + (uint32_t)((spu - 1) * nw);
    if (!wait_filled(a, s, last + 1u, seen)) return false;
    u32x4 v0[2 * P], v1[2 * P];
#pragma unroll
    for (int k = 0; k < 2 * P; k++)
      if (k < spu) {
        v0[k] = slot_read(s, i0 + (uint32_t)(k * nw), R, lane);
        if (two) v1[k] = slot_read(s, i1 + (uint32_t)(k * nw2), R, lane);
      }
    float a0[2] = {0.f, 0.f}, a1[2] = {0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 2 * P; k++)
      if (k < spu) {
        a0[k / P] += dot(v0[k], k % P);
        if (two) a1[k / P] += dot(v1[k], k % P);
      }
    const int un = u + 2 * NS;  // the wave's next unit
    publish_next(s, w, un < f.nu ? base + (uint32_t)((u0 + 2 * NS) * spu + w) : end, lane);
    st.acc0 = a0[0];
    st.acc1 = a0[1];
    s_finish_unit(a, o, s, f, u, lane, st);
    if (two) {
      st.acc0 = a1[0];
      st.acc1 = a1[1];
      s_finish_unit(a, o, s, f, u + NS, lane, st);
    }
  }
  return true;
}

__device__ __forceinline__ void consumer_wave(const PersistArgs &a, const Own &o, const Lds &s,
                                              int w, int lane) {
  const uint32_t R = (uint32_t)a.ring_slots;
  SState st;
  st.acc0 = st.acc1 = 0.f;
#pragma unroll
  for (int e8 = 0; e8 < 8; e8++) st.dacc[e8] = 0.f;
  st.bv = -INFINITY;
  st.bi = 0xffffffffu;
  uint32_t base = 0;  // stream index of the phase's first slot
  uint32_t seen = 0;  // cached smallest loader watermark
  Phase f;
  f.s = 0, f.l = 0, f.ph = a.steps ? PH_QKV : PH_END;
  for (; f.ph != PH_END; base += (uint32_t)phase_slots(f), phase_next(a, f)) {
    phase_setup(a, o, f);
    const uint32_t e = epoch(a, f.s, f.l), end = base + (uint32_t)phase_slots(f);
    if (f.ph == PH_DOWN) {
      const int P = f.P, ncols = f.nu;
      const int j0 = w / P, jstep = NS / P, piece = w % P;
      if (j0 >= ncols) {  // no columns: no part in the combine
        publish_next(s, w, end, lane);
        continue;
      }
      publish_next(s, w, base + (uint32_t)(j0 * P + piece), lane);
      if (!lds_wait(a, s, C_H, e * (uint32_t)ncols)) return;
      // up to DB columns per batch
      constexpr int DB = 6;
      for (int j = j0; j < ncols; j += DB * jstep) {
        const int nb = min(DB, (ncols - j + jstep - 1) / jstep);
        const uint32_t ib = base + (uint32_t)(j * P + piece);
        if (!wait_filled(a, s, ib + (uint32_t)((nb - 1) * jstep * P) + 1u, seen)) return;
        u32x4 v[DB];
        float h[DB];
#pragma unroll
        for (int b = 0; b < DB; b++)
          if (b < nb) {
            v[b] = slot_read(s, ib + (uint32_t)(b * jstep * P), R, lane);
            h[b] = s.hbuf[j + b * jstep];
          }
        const int jn = j + DB * jstep;
        publish_next(s, w, jn < ncols ? base + (uint32_t)(jn * P + piece) : end, lane);
#pragma unroll
        for (int b = 0; b < DB; b++)
          if (b < nb) {
            st.dacc[0] = fmaf(bf_lo(v[b].x), h[b], st.dacc[0]);
            st.dacc[1] = fmaf(bf_hi(v[b].x), h[b], st.dacc[1]);
            st.dacc[2] = fmaf(bf_lo(v[b].y), h[b], st.dacc[2]);
            st.dacc[3] = fmaf(bf_hi(v[b].y), h[b], st.dacc[3]);
            st.dacc[4] = fmaf(bf_lo(v[b].z), h[b], st.dacc[4]);
            st.dacc[5] = fmaf(bf_hi(v[b].z), h[b], st.dacc[5]);
            st.dacc[6] = fmaf(bf_lo(v[b].w), h[b], st.dacc[6]);
            st.dacc[7] = fmaf(bf_hi(v[b].w), h[b], st.dacc[7]);
          }
      }
      if (!s_finish_down(a, o, s, f.s, f.l, w, lane, st)) return;
      continue;
    }
    if (w >= f.nu) {  // no unit of this phase
      publish_next(s, w, end, lane);
      continue;
    }
    publish_next(s, w, base + (uint32_t)w, lane);
    bool ok;
    switch (f.ph) {
      case PH_QKV: ok = lds_wait(a, s, F_XN, e); break;
      case PH_O: ok = lds_wait(a, s, F_ATT, e); break;
      case PH_GU: ok = lds_wait(a, s, F_XN2, e); break;
      default: ok = lds_wait(a, s, F_XF, f.s + 1); break;
    }
    if (!ok) return;
    switch (f.P) {
      case 1: ok = dot_phase<1>(a, o, s, f, base, end, w, lane, seen, st); break;
      case 2: ok = dot_phase<2>(a, o, s, f, base, end, w, lane, seen, st); break;
      default: ok = dot_phase<3>(a, o, s, f, base, end, w, lane, seen, st); break;
    }
    if (!ok) return;
    if (f.ph == PH_HEAD) {
      if (lane == 0) {
        s.best[w] = (f32x2){st.bv, __uint_as_float(st.bi)};
        lds_flag_add(s.flag + C_HEAD, 1u);
      }
      st.bv = -INFINITY;
      st.bi = 0xffffffffu;
    }
  }
  publish_next(s, w, 0xffffffffu, lane);
}

// ---- the attention wave ---------------------------------------------------------
__device__ __forceinline__ bool attention_item(const PersistArgs &a, const Lds &s, uint32_t step, int l, int h,
                               int ci, int lane) {
  const int d = a.d, gq = a.nq / a.nkv, g = h / gq, kvd = a.nkv * a.d;
  const uint32_t pos = a.pos0 + step;
  const int seq = (int)pos + 1, t0 = ci * AC, n = min(AC, seq - t0);
  const bool has_cur = (int)pos < t0 + n;
  const int nold = has_cur ? n - 1 : n;
  float *kc = a.kc + (size_t)l * a.layer_kv, *vc = a.vc + (size_t)l * a.layer_kv;
  // cached rows [t0, t0 + nold): contiguous in the [kv][seq][d] layout
  {
    const uint8_t *ks = (const uint8_t *)(kc + ((size_t)g * a.max_seq + t0) * d);
    const uint8_t *vs = (const uint8_t *)(vc + ((size_t)g * a.max_seq + t0) * d);
    const int bytes = nold * d * 4;
    for (int off = 0; off < bytes; off += 1024) {
      const int lo = off + lane * 16;
      if (lo < bytes) {
        __builtin_amdgcn_global_load_lds((const void *)(ks + lo),
                                         (__attribute__((address_space(3))) void *)((lu8 *)s.kb + off),
                                         16, 0, 16);
        __builtin_amdgcn_global_load_lds((const void *)(vs + lo),
                                         (__attribute__((address_space(3))) void *)((lu8 *)s.vb + off),
                                         16, 0, 16);
      }
    }
  }
  // q of head h and, in the last chunk, this step's k and v of head g
  constexpr int QM = 3 * MAXD / 64;
  float qv[QM];
  const int nw = d + (has_cur ? 2 * d : 0);
  const uint64_t *tq = a.tq + h * d;
  const uint32_t T = tagof(a, step, l, P_QKV);
  // words 0..d-1 from tq, d..2d-1 from tkv (k of g), 2d..3d-1 from tkv (v of g)
  bool ok;
  {
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc((void *)tq, (short)0, d * 8, 0x00020000);
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void *)(a.tkv + g * d), (short)0, d * 8, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.tkv + kvd + g * d), (short)0, d * 8, 0x00020000);
    ok = false;
    for (unsigned spins = 0;; spins++) {
      bool ready = true;
#pragma unroll
      for (int m = 0; m < QM; m++) {
        const int i = lane + 64 * m;
        if (i < nw) {
          const int part = i / d, j = i - part * d;
          const __amdgpu_buffer_rsrc_t rs = part == 0 ? rq : part == 1 ? rk : rv;
          const u32x2 wv = __builtin_amdgcn_raw_buffer_load_b64(rs, (uint32_t)j * 8u, 0, kAuxCoherent);
          qv[m] = __uint_as_float(wv.x);
          ready = ready && wv.y == T;
        }
      }
      if (__builtin_amdgcn_ballot_w64(!ready) == 0) {
        ok = true;
        break;
      }
      if ((spins & 63) == 63) {
        if (spins > kSpinMax) __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (err_raised(a)) break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  if (!ok) return false;
#pragma unroll
  for (int m = 0; m < QM; m++) {
    const int i = lane + 64 * m;
    if (i < nw) {
      const int part = i / d, j = i - part * d;
      if (part == 0) s.qb[j] = qv[m];
      else if (part == 1) s.kb[nold * d + j] = qv[m];
      else s.vb[nold * d + j] = qv[m];
    }
  }
  // the first q head of the group stores this step's k/v row into the cache;
  // it must be complete before this item publishes (later steps read it)
  if (has_cur && h % gq == 0) {
#pragma unroll
    for (int m = 0; m < QM; m++) {
      const int i = lane + 64 * m;
      if (i >= d && i < nw) {
        const int part = i / d, j = i - part * d;
        float *dst = (part == 1 ? kc : vc) + ((size_t)g * a.max_seq + pos) * d + j;
        cstore(dst, qv[m]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the direct loads into K/V are complete
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // scores: lane t = lane % 32 over the d/2 dims of half lane / 32, the
  // dims rotated by t so the 32 rows read distinct LDS banks
  const int t = lane & 31, hf = lane >> 5, dh = d >> 1;
  float sc = 0.f;
  if (t < n) {
    const lf32 *kr = s.kb + t * d + hf * dh, *qr = s.qb + hf * dh;
    int j = t % dh;
    for (int jj = 0; jj < dh; jj++) {
      sc = fmaf(qr[j], kr[j], sc);
      j = j + 1 == dh ? 0 : j + 1;
    }
  }
  sc += __shfl_xor(sc, 32, 64);
  const float scale = 1.0f / sqrtf((float)d);
  sc = t < n ? sc * scale : -INFINITY;
  const float mx = wave_max(sc);
  const float ex = (lane < 32 && t < n) ? expf(sc - mx) : 0.f;
  const float lsum = wave_sum(ex);
  if (lane < 32) s.pb[lane] = ex;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const uint32_t TP = tagof(a, step, l, P_PART);
  const int nchmax = (a.max_seq + AC - 1) / AC;
  uint64_t *dst = a.tpart + ((size_t)h * nchmax + ci) * (d + 2);
  for (int j = lane; j < d; j += 64) {
    float acc = 0.f;
    for (int tt = 0; tt < n; tt++) acc = fmaf(s.pb[tt], s.vb[tt * d + j], acc);
    tput(dst + j, acc, TP);
  }
  if (lane == 0) {
    tput(dst + d, mx, TP);
    tput(dst + d + 1, lsum, TP);
  }
  return true;
}

// q head h: merge its chunks' partials into att[h]
__device__ __forceinline__ bool attention_merge(const PersistArgs &a, const Lds &s, uint32_t step, int l, int h,
                                int lane) {
  const int d = a.d, dd = d + 2;
  const uint32_t pos = a.pos0 + step;
  const int nch = ((int)pos + AC) / AC;
  const int nchmax = (a.max_seq + AC - 1) / AC;
  const uint64_t *src = a.tpart + (size_t)h * nchmax * dd;
  const int n = nch * dd;
  const uint32_t TP = tagof(a, step, l, P_PART);
  for (int base = 0; base < n; base += 64 * PC) {
    const int cnt = min(n - base, 64 * PC);
    if (!pgather(a, src + base, cnt, chunk_of(cnt), TP, s.msc + base, lane)) return false;
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // w_c = e^(m_c - M) / sum_c e^(m_c - M) l_c; att = sum_c w_c o_c
  float mx = -INFINITY;
  for (int c = 0; c < nch; c++) mx = fmaxf(mx, s.msc[c * dd + d]);
  float lsum = 0.f;
  for (int c = 0; c < nch; c++) lsum = fmaf(expf(s.msc[c * dd + d] - mx), s.msc[c * dd + d + 1], lsum);
  const float inv = 1.0f / lsum;
  const uint32_t TA = tagof(a, step, l, P_ATT);
  for (int j = lane; j < d; j += 64) {
    float acc = 0.f;
    for (int c = 0; c < nch; c++) acc = fmaf(expf(s.msc[c * dd + d] - mx) * inv, s.msc[c * dd + j], acc);
    tput(a.tatt + h * d + j, acc, TA);
  }
  return true;
}

__device__ __forceinline__ void attention_wave(const PersistArgs &a, const Lds &s, int lane) {
  const int c = blockIdx.x;
  const int mh = NB - 1 - c;
  for (uint32_t step = 0; step < a.steps; step++) {
    const uint32_t pos = a.pos0 + step;
    const int nch = ((int)pos + AC) / AC;
    const int items = a.nq * nch;
    for (int l = 0; l < a.L; l++) {
      for (int it = c; it < items; it += NB)
        if (!attention_item(a, s, step, l, it % a.nq, it / a.nq, lane)) goto fail;
      if (mh < a.nq)
        if (!attention_merge(a, s, step, l, mh, lane)) goto fail;
    }
  }
  return;
fail:
  if (lane == 0) lds_flag_set(s.flag + F_ABORT, 1u);
}

// ---- the poller wave ------------------------------------------------------------
// dst = rmsnorm(s.xg[0, H)) with gains g (rmsnorm_bf16_weight,
// crates/tensor_core/src/bf16.rs:231-270, in this wave's summation order);
// lane l takes elements [l C, l C + C)
__device__ void p_norm(const PersistArgs &a, const Lds &s, const uint16_t *g, lf32 *dst, int C,
                       int lane) {
  const int H = a.H, i0 = lane * C;
  const __amdgpu_buffer_rsrc_t rg = rsrc(g, (size_t)H * 2);
  u32x4 gw[PC / 8];
#pragma unroll
  for (int m = 0; m < PC / 8; m++)
    if (8 * m < C && i0 + 8 * m < H)
      gw[m] = __builtin_amdgcn_raw_buffer_load_b128(rg, (uint32_t)(i0 + 8 * m) * 2u, 0, 0);
  float xv[PC];
  float ss = 0.f;
#pragma unroll
  for (int m = 0; m < PC; m++) {
    const int i = i0 + m;
    xv[m] = (m < C && i < H) ? s.xg[i] : 0.f;
    ss = fmaf(xv[m], xv[m], ss);
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)H + a.eps);
#pragma unroll
  for (int m = 0; m < PC / 8; m++)
    if (8 * m < C && i0 + 8 * m < H) {
      const u32x4 gg = gw[m];
      const float gv[8] = {bf_lo(gg.x), bf_hi(gg.x), bf_lo(gg.y), bf_hi(gg.y),
                           bf_lo(gg.z), bf_hi(gg.z), bf_lo(gg.w), bf_hi(gg.w)};
#pragma unroll
      for (int e = 0; e < 8; e++)
        if (i0 + 8 * m + e < H) dst[i0 + 8 * m + e] = gv[e] * (xv[8 * m + e] * inv);
    }
}

// best (value, index) over the 2 NB words (value, index bits) of targ
__device__ bool p_argmax(const PersistArgs &a, const Lds &s, uint32_t tag, float &bv,
                         uint32_t &bi, int lane) {
  if (!pgather(a, a.targ, 2 * NB, chunk_of(2 * NB), tag, s.xg, lane)) return false;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  for (int k = lane; k < NB; k += 64) {
    const float v = s.xg[2 * k];
    const uint32_t ix = __float_as_uint(s.xg[2 * k + 1]);
    if (beats(v, ix, bv, bi)) {
      bv = v;
      bi = ix;
    }
  }
  return true;
}
__device__ __forceinline__ void wave_best(float &bv, uint32_t &bi) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const uint32_t oi = __shfl_xor(bi, off, 64);
    if (beats(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
}

// the down partials of this workgroup's rows x0 + i (i < nx) from workgroups
// k < nkp, summed in a fixed order (lane over workgroups, then the wave tree)
__device__ bool p_down_sum(const PersistArgs &a, const Own &o, uint32_t tag, float (&part)[MAXXR],
                           int lane) {
  constexpr int RM = NB / 64;
  const int nx = o.x1 - o.x0, H = a.H;
  const int hp = (a.I + NB - 1) / NB, nkp = (a.I + hp - 1) / hp;
  const __amdgpu_buffer_rsrc_t rs = rsrc(a.tpd, (size_t)NB * H * 8);
  float t[MAXXR];
  for (unsigned spins = 0;; spins++) {
    bool ready = true;
#pragma unroll
    for (int i = 0; i < MAXXR; i++) t[i] = 0.f;
#pragma unroll
    for (int m = 0; m < RM; m++) {
      const int k = lane + 64 * m;
      if (k < nkp) {
        const uint32_t off = ((uint32_t)k * (uint32_t)H + (uint32_t)o.x0) * 8u;
#pragma unroll
        for (int i = 0; i < MAXXR; i++)
          if (i < nx) {
            const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rs, off + 8u * i, 0, kAuxCoherent);
            t[i] += __uint_as_float(w.x);
            ready = ready && w.y == tag;
          }
      }
    }
    if (__builtin_amdgcn_ballot_w64(!ready) == 0) break;
    if (!spin_check(a, spins)) return false;
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int i = 0; i < MAXXR; i++) part[i] = i < nx ? wave_sum(t[i]) : 0.f;
  return true;
}

__device__ __forceinline__ void poll_wave(const PersistArgs &a, const Own &o, const Lds &s, int lane) {
  const int c = blockIdx.x, H = a.H, qd = a.nq * a.d, half = a.d >> 1;
  const int nx = o.x1 - o.x0;
  const int CH = chunk_of(H), CQ = chunk_of(qd);
  for (uint32_t step = 0; step < a.steps; step++) {
    const uint32_t pos = a.pos0 + step;
    // ---- the step's token: argmax of the previous logits ------------------
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    if (step == 0) {
      for (int i = lane; i < a.nparts_in; i += 64) {
        const float2 p = a.part_in[i];
        if (beats(p.x, __float_as_uint(p.y), bv, bi)) {
          bv = p.x;
          bi = __float_as_uint(p.y);
        }
      }
    } else if (!p_argmax(a, s, tagof(a, step - 1, a.L, 0), bv, bi, lane)) {
      goto fail;
    }
    wave_best(bv, bi);
    {
      const uint32_t tok = bi < (uint32_t)a.V ? bi : 0u;  // no candidate -> id 0
      if (c == 0 && lane == 0) a.out_ids[step] = tok;
      mark(a, step, 0);
      const uint16_t *erow = a.embed + (size_t)tok * H;
      for (int i = lane; i < H; i += 64) s.xg[i] = bf16f(erow[i]);
    }
    for (int p = lane; p < half; p += 64) {
      const float2 cs = a.rope[(size_t)pos * half + p];
      s.rope[p] = (f32x2){cs.x, cs.y};
    }

    for (int l = 0; l < a.L; l++) {
      const PersistLayer &L = a.layers[l];
      const uint32_t e = epoch(a, step, l);
      if (l > 0 && !pgather(a, a.txd, H, CH, tagof(a, step, l - 1, P_XD), s.xg, lane)) goto fail;
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      mark(a, step, 1 + 5 * l);
      // this workgroup's residual rows, and the q/k/v bias of its rows (the
      // previous layer's q/k/v phase here is over: its output reached every
      // owner of the gathered rows)
      for (int i = lane; i < nx; i += 64) s.xl[i] = s.xg[o.x0 + i];
      for (int i = lane; i < 2 * (o.pc1 - o.pc0); i += 64) s.bq[i] = L.bqkv[2 * o.pc0 + i];
      p_norm(a, s, L.ln1, s.xn, CH, lane);
      lds_flag_set(s.flag + F_XN, e);
      // attention output -> o
      if (!pgather(a, a.tatt, qd, CQ, tagof(a, step, l, P_ATT), s.att, lane)) goto fail;
      lds_flag_set(s.flag + F_ATT, e);
      mark(a, step, 2 + 5 * l);
      // residual after o -> gate/up
      if (!pgather(a, a.txo, H, CH, tagof(a, step, l, P_XO), s.xg, lane)) goto fail;
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      mark(a, step, 3 + 5 * l);
      p_norm(a, s, L.ln2, s.xn2, CH, lane);
      lds_flag_set(s.flag + F_XN2, e);
      // down: the workgroups' partials of this workgroup's rows + residual
      if (nx > 0) {
        float part[MAXXR];
        if (!p_down_sum(a, o, tagof(a, step, l, P_PD), part, lane)) goto fail;
        const uint32_t TX = tagof(a, step, l, P_XD);
        if (lane == 0)
#pragma unroll
          for (int i = 0; i < MAXXR; i++)
            if (i < nx) {
              const float x = s.xl[i] + part[i];
              s.xl[i] = x;
              tput(a.txd + o.x0 + i, x, TX);
            }
      }
      mark(a, step, 4 + 5 * l);
    }
    // ---- final norm + head ----------------------------------------------------
    if (!pgather(a, a.txd, H, CH, tagof(a, step, a.L - 1, P_XD), s.xg, lane)) goto fail;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    mark(a, step, 1 + 5 * a.L);
    p_norm(a, s, a.final_norm, s.xf, CH, lane);
    if (c == 0)
      for (int i = lane; i < H; i += 64) a.normed[i] = s.xf[i];
    lds_flag_set(s.flag + F_XF, step + 1);
    {
      // every consumer wave with head rows reports; the others never do
      int nhw = 0;
      for (int w = 0; w < NS; w++) nhw += w < o.v1 - o.v0;
      if (!lds_wait_global(a, s, C_HEAD, (step + 1) * (uint32_t)nhw)) goto fail;
      float hv = -INFINITY;
      uint32_t hi = 0xffffffffu;
      for (int w = 0; w < nhw; w++) {
        const f32x2 c2 = s.best[w];
        if (beats(c2.x, __float_as_uint(c2.y), hv, hi)) {
          hv = c2.x;
          hi = __float_as_uint(c2.y);
        }
      }
      const uint32_t TH = tagof(a, step, a.L, 0);
      if (lane == 0) {
        tput(a.targ + 2 * c, hv, TH);
        tput(a.targ + 2 * c + 1, __uint_as_float(hi), TH);
      }
      mark(a, step, 2 + 5 * a.L);
    }
  }
  // ---- hand the state back to the per-kernel path ------------------------------
  if (lane == 0)
    for (int i = 0; i < nx; i++) a.x_out[o.x0 + i] = s.xl[i];
  if (c == 0) {
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    if (!p_argmax(a, s, tagof(a, a.steps - 1, a.L, 0), bv, bi, lane)) goto fail;
    wave_best(bv, bi);
    if (lane == 0) {
      a.state[0] = a.pos0 + a.steps;
      a.state[1] = a.out_ids[a.steps - 1];
      a.state[2] = a.steps;
    }
    const float2 none = make_float2(-INFINITY, __uint_as_float(0xffffffffu));
    for (int i = lane; i < a.part_cap; i += 64)
      a.part_out[i] = i == 0 ? make_float2(bv, __uint_as_float(bi)) : none;
  }
  return;
fail:
  if (lane == 0) lds_flag_set(s.flag + F_ABORT, 1u);
}

__global__ void __launch_bounds__(NT, 1) decode_stream_kernel(PersistArgs a) {
  extern __shared__ float4 sm4[];
  const int nchmax = (a.max_seq + AC - 1) / AC;
  const Lds s = carve((lu8 *)sm4, nchmax, a.d, a.ring_slots);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Own o = own_of(a, blockIdx.x);
  // zero the LDS vectors (their padding past k must read as 0) and the flags;
  // every ring position starts free
  for (int i = tid; i < 4 * MAXK; i += NT) s.xn[i] = 0.f;
  for (int i = tid; i < F_NFLAGS; i += NT) s.flag[i] = 0u;
  for (int i = tid; i < MAXXR; i += NT) s.xl[i] = 0.f;
  for (int i = tid; i < NL + NS; i += NT) s.filled[i] = 0u;  // filled[NL], cnext[NS]
  __syncthreads();
  if (wave < NS) consumer_wave(a, o, s, wave, lane);
  else if (wave < WAVE_L + NL) loader_wave(a, o, s, wave - WAVE_L, lane);
  else if (wave == WAVE_P) poll_wave(a, o, s, lane);
  else attention_wave(a, s, lane);
}

// ring slots that fit beside the rest of the LDS
int ring_slots_for(int max_seq, int d) {
  const size_t fixed = lds_fixed_bytes((max_seq + AC - 1) / AC, d);
  if (fixed + 2048 > kMaxLds) return 0;
  int r = (int)((kMaxLds - fixed - 1024) / (1024 + 8));
  while (r > 0 && lds_bytes((max_seq + AC - 1) / AC, d, r) > kMaxLds) r--;
  return r;
}

}  // namespace

bool stream_supported(int H, int I, int V, int qdim, int d, int gq, int nkv, int max_seq,
                      int qkv_rows) {
  if (H % 8 || I % 8 || qdim % 8 || d % 8) return false;
  if (H > MAXK || qdim > MAXK || d > MAXD || d < 8 || gq > 8) return false;
  const int P = (H + SLOT - 1) / SLOT;
  if (NS % P) return false;  // the down pieces split the streaming waves evenly
  if ((I + NB - 1) / NB > MAXHP || (H + NB - 1) / NB > MAXXR) return false;
  if ((qkv_rows / 2 + NB - 1) / NB > MAXPQ || qkv_rows % 2) return false;
  (void)V;
  (void)nkv;
  if (ring_slots_for(max_seq, d) < NL * DMAX + 24) return false;
  return true;
}

bool stream_device_ok(const PersistArgs &a) {
  if (!stream_supported(a.H, a.I, a.V, a.nq * a.d, a.d, a.nq / a.nkv, a.nkv, a.max_seq,
                        a.qkv_rows))
    return false;
  int dev = 0, coop = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess) return false;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
  return coop != 0 && cus >= NB;
}

size_t stream_tpd_words(int H) { return (size_t)NB * H; }
size_t stream_part_words(int nq, int max_seq, int d) {
  return (size_t)nq * ((max_seq + AC - 1) / AC) * (size_t)(d + 2);
}

hipError_t launch_decode_stream(const PersistArgs &a, hipStream_t s) {
  if (!stream_supported(a.H, a.I, a.V, a.nq * a.d, a.d, a.nq / a.nkv, a.nkv, a.max_seq,
                        a.qkv_rows))
    return hipErrorInvalidValue;
  if (a.steps == 0) return hipSuccess;
  if (a.pos0 + a.steps > (uint32_t)a.max_seq) return hipErrorInvalidValue;
  PersistArgs args = a;
  args.ring_slots = ring_slots_for(a.max_seq, a.d);
  const size_t smem = lds_bytes((a.max_seq + AC - 1) / AC, a.d, args.ring_slots);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)decode_stream_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  void *params[] = {&args};
  return hipLaunchCooperativeKernel((const void *)decode_stream_kernel, dim3(NB), dim3(NT), params,
                                    (unsigned)smem, s);
}

}  // namespace myos
