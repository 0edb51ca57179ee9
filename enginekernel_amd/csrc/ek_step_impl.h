// The whole Qwen3 decode step as one persistent launch (gfx950).
//
// One 512-thread workgroup per CU runs every phase of the step in order --
// per layer: RMSNorm + qkv projection, attention, o projection, residual add
// + RMSNorm + gate/up projection + SwiGLU, down projection; then the final
// add + norm, lm_head and argmax, and the step's bookkeeping -- with a grid
// barrier between phases instead of a kernel boundary. What a kernel boundary
// cannot do and this does: while a workgroup finishes one phase, its waves
// already load the first weight chunks of the next phase (weights never depend
// on activations), so the HBM stream does not stop at the ~180 phase
// boundaries of a step.
//
// Projections. A phase's output units (rows; gate/up row pairs for SwiGLU)
// are split evenly over the workgroups; a workgroup's (row, 1 KiB chunk)
// items are split evenly over its 8 waves, so no wave idles on a short row
// count. Each lane streams 16 B of a chunk (a wave reads 1 KiB per load
// instruction, fully coalesced) through an 8-deep register ring that crosses
// row and phase boundaries; fp32 FMA accumulation (bf16 products are exact),
// a butterfly per row segment, and a fixed-order sum of the waves' segment
// partials in LDS. Activations (at most 2 rows of <= 9728 bf16) are staged
// once per phase in LDS.
//
// Data between workgroups. The eight XCD L2 caches are not coherent with each
// other. Every activation a phase hands to the next lives in a per-layer
// buffer of an arena that each launch writes exactly once per element, with
// device-scope stores (write-through past the L2), and is read with
// device-scope loads. A workgroup's stores are complete (s_waitcnt) before it
// arrives at the barrier; the barrier is a counter per XCD group plus a top
// counter and a generation word (each on its own 256-byte line), reset by its
// last arrivers, so it needs no clearing between launches. Every wait is
// bounded: a workgroup that spins past the limit sets the error word and
// leaves, and so does every other workgroup at its next wait.
//
// Rounding points are the reference fallback's (engine/ek_model.py:360-416,
// 475-493): bf16 residual adds, fp32 norm statistics rounded to bf16 before
// the bf16 gain, projections accumulated in fp32 and rounded once,
// bf16(silu(bf16 g)) * bf16(u), bf16 probabilities before PV, first-index
// argmax of the bf16 logits.

#pragma once

#include "ek_common.h"
#include "ek_attn_impl.h"

namespace eks {

constexpr int SNT = eka::FNT;          // 512 threads
constexpr int SNW = SNT / EK_WAVE;     // 8 waves
constexpr int NB = 8;                  // weight chunks in flight per wave
constexpr int CH = 8 * EK_WAVE;        // bf16 elements per chunk (1 KiB)
constexpr int LW_FIELDS = 10;          // per-layer pointer table row
constexpr int STU = 2;                 // attention: 16-key score tiles in flight per wave
constexpr int SPT = 1;                 // attention: 32-key PV tiles in flight per wave

// per-layer pointer table: [n_layers][LW_FIELDS] device addresses
enum { LW_QKV = 0, LW_O, LW_GU, LW_DOWN, LW_LN1, LW_LN2, LW_QN, LW_KN, LW_KC, LW_VC };

struct Bar { unsigned sub[8][64]; unsigned top[64]; unsigned gen[64]; };

struct StepArgs {
  const int64_t* lw;
  int nl, h, inter, nq, nkv, vocab;
  float eps, sm_scale;
  const bf16_t* embed; int64_t lde;
  const bf16_t* lm_head; const bf16_t* fnorm;
  const bf16_t* cos; const bf16_t* sin; int64_t ld_cs, rope_len;
  int64_t csb, csh, css, s_cap;
  int64_t* tokens; int64_t* positions; int64_t* len_t; int64_t* slot_t; const int32_t* start_t;
  int32_t* out_buf; int64_t* step_idx; int64_t max_steps; int64_t* out_tok;
  bf16_t* arena;
  float* am_val; int32_t* am_idx;
  Bar* bar; int* err; int64_t spin;
  int kpad_max, part_max, o_rows;      // LDS plan (host-computed, see make_plan in ek_step.hip)
};

__host__ __device__ constexpr int cdiv_i(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ constexpr int kpad_of(int k) { return cdiv_i(k, CH) * CH; }

// largest unit count of one workgroup over the step's projections, times the
// rows per unit (2 for the gate/up pairs)
__host__ __device__ inline int part_rows_max(int h, int inter, int qkvw, int vocab, int nwg) {
  int r = cdiv_i(qkvw, nwg);
  r = r > cdiv_i(h, nwg) ? r : cdiv_i(h, nwg);
  r = r > 2 * cdiv_i(inter, nwg) ? r : 2 * cdiv_i(inter, nwg);
  r = r > cdiv_i(vocab, nwg) ? r : cdiv_i(vocab, nwg);
  return r;
}

// elements per layer of the activation arena at batch bm
__host__ __device__ inline int64_t arena_layer_elems(int bm, int h, int inter, int qkvw, int qw) {
  return (int64_t)bm * (4 * h + qkvw + qw + inter);
}

// ---------------------------------------------------------------------------
// device-scope (cross-XCD) loads and stores
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint4 ld16_dev(const bf16_t* p) {
  const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
  const uint64_t x = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t y = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint4((uint32_t)x, (uint32_t)(x >> 32), (uint32_t)y, (uint32_t)(y >> 32));
}

__device__ __forceinline__ void st16_dev(bf16_t* p, uint4 v) {
  uint64_t* q = reinterpret_cast<uint64_t*>(p);
  __hip_atomic_store(q, (uint64_t)v.x | ((uint64_t)v.y << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, (uint64_t)v.z | ((uint64_t)v.w << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void st_bf16_dev(bf16_t* p, float v) {
  __hip_atomic_store(p, (bf16_t)f2bf(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// grid barrier (all workgroups co-resident: one per CU). Every thread calls
// drain() first, so that its stores are performed before thread 0 arrives.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void drain() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0);
  __asm__ volatile("" ::: "memory");
}

__device__ __forceinline__ bool grid_sync(Bar* b, unsigned& gen, int* err, int64_t spin, bool wait, int* s_ok) {
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned nb = gridDim.x;
    const unsigned grp = blockIdx.x & 7u;
    const unsigned gsize = (nb - grp + 7u) / 8u;
    const unsigned ngrp = nb < 8u ? nb : 8u;
    const unsigned target = gen + 1u;
    const unsigned a = __hip_atomic_fetch_add(&b->sub[grp][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a == gsize - 1u) {
      __hip_atomic_store(&b->sub[grp][0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      const unsigned t = __hip_atomic_fetch_add(&b->top[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (t == ngrp - 1u) {
        __hip_atomic_store(&b->top[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        __hip_atomic_store(&b->gen[0], target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    int ok = 1;
    if (wait) {
      int64_t it = 0;
      while ((int)(__hip_atomic_load(&b->gen[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
        if ((++it & 1023) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) { ok = 0; break; }
        if (it > spin) {
          __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    gen = target;
    *s_ok = ok;
  }
  __syncthreads();
  return *s_ok != 0;
}

// ---------------------------------------------------------------------------
// projections
// ---------------------------------------------------------------------------
struct Gp {
  const bf16_t* w;   // [rows, K] row-major
  int K, C;          // reduction length, 1 KiB chunks per row
  int units;         // output units
  int pair;          // 1: unit u is rows u and up_off + u (gate/up)
  int up_off;
  int wg0, nwg;      // the units are spread over workgroups [wg0, wg0 + nwg)
};

__device__ __forceinline__ Gp make_gp(const bf16_t* w, int k, int units, int pair) {
  Gp g;
  g.w = w; g.K = k; g.C = cdiv_i(k, CH); g.units = units; g.pair = pair; g.up_off = units;
  g.wg0 = 0; g.nwg = gridDim.x;
  return g;
}

// this workgroup's units [u0, u1) (empty outside the phase's workgroups)
__device__ __forceinline__ void unit_range(const Gp& g, int& u0, int& u1) {
  const int w = (int)blockIdx.x - g.wg0;
  if (w < 0 || w >= g.nwg) { u0 = u1 = 0; return; }
  u0 = (int)((int64_t)g.units * w / g.nwg);
  u1 = (int)((int64_t)g.units * (w + 1) / g.nwg);
}

struct WaveItems { int i0, n; };

__device__ __forceinline__ WaveItems wave_items(const Gp& g, int nu, int wave) {
  const int n_items = nu * (g.pair ? 2 : 1) * g.C;
  const int i0 = (int)((int64_t)n_items * wave / SNW);
  const int i1 = (int)((int64_t)n_items * (wave + 1) / SNW);
  WaveItems w;
  w.i0 = i0; w.n = i1 - i0;
  return w;
}

// A wave's items of one phase. Rows are K = C * 1 KiB long (the plan
// requires K % 512 == 0), so the items of a workgroup's rows are one
// contiguous byte range per half (the gate rows, then the up rows, for a
// pair phase): item i sits at base + i KiB, or up + (i - half) KiB.
struct Span {
  const bf16_t* base;   // item 0 of the workgroup
  const bf16_t* up;     // item `half` (pair phases)
  int half;             // items before `up` (all of them for a plain phase)
  int i0, n;            // this wave's items [i0, i0 + n)
};

__device__ __forceinline__ Span make_span(const Gp& g, int wave) {
  int u0, u1;
  unit_range(g, u0, u1);
  const int nu = u1 - u0;
  const WaveItems w = wave_items(g, nu, wave);
  Span s;
  s.base = g.w + (int64_t)u0 * g.K;
  s.up = g.pair ? g.w + (int64_t)(g.up_off + u0) * g.K : s.base;
  s.half = g.pair ? nu * g.C : 0x7fffffff;
  s.i0 = w.i0; s.n = w.n;
  return s;
}

// first element of item i (wave-uniform)
__device__ __forceinline__ const bf16_t* span_item(const Span& s, int i) {
  return i < s.half ? s.base + (int64_t)i * CH : s.up + (int64_t)(i - s.half) * CH;
}

// The wave's ring: when `ready`, r[u] holds item u of the coming phase.
struct Ring {
  uint4 r[NB];
  bool ready;
};

// The first NB items of phase `pn` into this wave's ring, issued ahead of a
// barrier so that they load while the workgroup waits. Wave 0 runs the
// barrier's atomics, whose results would wait behind these loads (vector
// memory counts drain in order), so it loads its items after the barrier.
__device__ __forceinline__ void prefetch_phase(const Gp* pn, Ring& ring) {
  ring.ready = false;
  const int wave = wave_id();
  if (!pn || wave == 0) return;
  const Span sn = make_span(*pn, wave);
  const int loff = (threadIdx.x & 63) * 8;
#pragma unroll
  for (int u = 0; u < NB; ++u) ring.r[u] = ld16(span_item(sn, sn.i0 + (u < sn.n ? u : 0)) + loff);
  ring.ready = true;
}

// One projection phase: partial dot products of this wave's items into
// part[(row_local * SNW + wave) * BM + b]. Items go in blocks of NB: the
// loads of block i + 1 are issued (all NB at once) before block i is
// consumed, so NB to 2 NB chunks are always in flight. The ring holds block 0
// on entry when prefetch_phase loaded it. Loads past the end re-read item 0
// (never consumed).
template <int BM>
__device__ __forceinline__ void gemv_phase(const Gp& P, Ring& ring, const bf16_t* xs, int kpad, float* part) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const Span sp = make_span(P, wave);
  const int n = sp.n;
  const int loff = lane * 8;
  if (!ring.ready) {
#pragma unroll
    for (int u = 0; u < NB; ++u) ring.r[u] = ld16(span_item(sp, sp.i0 + (u < n ? u : 0)) + loff);
  }
  const int nblk = (n + NB - 1) / NB;
  int r = sp.i0 / P.C, ch = sp.i0 - (sp.i0 / P.C) * P.C;   // consume position (row-local, chunk)

  float acc[BM];
#pragma unroll
  for (int b = 0; b < BM; ++b) acc[b] = 0.f;
  for (int blk = 0; blk < nblk; ++blk) {
    const int nb0 = (blk + 1) * NB;   // first item of the next block
    uint4 nx[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) nx[u] = ld16(span_item(sp, sp.i0 + (nb0 + u < n ? nb0 + u : 0)) + loff);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int k = blk * NB + u;
      if (k < n) {
        const uint4 wv = ring.r[u];
#pragma unroll
        for (int b = 0; b < BM; ++b)
          acc[b] = dot8_acc(wv, *reinterpret_cast<const uint4*>(xs + b * kpad + ch * CH + loff), acc[b]);
        if (ch == P.C - 1 || k == n - 1) {
#pragma unroll
          for (int b = 0; b < BM; ++b) {
            const float sum = wave_sum(acc[b]);
            if (lane == 0) part[(r * SNW + wave) * BM + b] = sum;
            acc[b] = 0.f;
          }
        }
        if (++ch == P.C) { ch = 0; ++r; }
      }
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) ring.r[u] = nx[u];
  }
  ring.ready = false;
}

// Copy this workgroup's rows of a plain phase into LDS (row-major, K per row):
// 8 chunks of 16 B per thread in flight per round.
__device__ __forceinline__ void stage_rows_lds(const Gp& P, bf16_t* wl) {
  int u0, u1;
  unit_range(P, u0, u1);
  const int n16 = (u1 - u0) * P.K / 8;
  const bf16_t* src = P.w + (int64_t)u0 * P.K;
  for (int i0 = threadIdx.x; i0 < n16; i0 += 8 * SNT) {
    uint4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = i0 + j * SNT;
      v[j] = ld16(src + (int64_t)(i < n16 ? i : 0) * 8);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = i0 + j * SNT;
      if (i < n16) *reinterpret_cast<uint4*>(wl + (int64_t)i * 8) = v[j];
    }
  }
}

// A plain projection phase whose rows stage_rows_lds put in LDS: same item
// split and partials as gemv_phase, weights read from LDS.
template <int BM>
__device__ __forceinline__ void gemv_lds_phase(const Gp& P, const bf16_t* wl, const bf16_t* xs, int kpad, float* part) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  int u0, u1;
  unit_range(P, u0, u1);
  const WaveItems wr = wave_items(P, u1 - u0, wave);
  const int loff = lane * 8;
  int r = wr.i0 / P.C, ch = wr.i0 - (wr.i0 / P.C) * P.C;
  float acc[BM];
#pragma unroll
  for (int b = 0; b < BM; ++b) acc[b] = 0.f;
#pragma unroll 4
  for (int k = 0; k < wr.n; ++k) {
    const uint4 wv = *reinterpret_cast<const uint4*>(wl + (int64_t)r * P.K + ch * CH + loff);
#pragma unroll
    for (int b = 0; b < BM; ++b)
      acc[b] = dot8_acc(wv, *reinterpret_cast<const uint4*>(xs + b * kpad + ch * CH + loff), acc[b]);
    if (ch == P.C - 1 || k == wr.n - 1) {
#pragma unroll
      for (int b = 0; b < BM; ++b) {
        const float sum = wave_sum(acc[b]);
        if (lane == 0) part[(r * SNW + wave) * BM + b] = sum;
        acc[b] = 0.f;
      }
    }
    if (++ch == P.C) { ch = 0; ++r; }
  }
}

// sum of the waves' partials of row_local r, fixed order
template <int BM>
__device__ __forceinline__ float row_sum(const float* part, int r, int b) {
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < SNW; ++w) s += part[(r * SNW + w) * BM + b];
  return s;
}

// y = bf16(sum) for this workgroup's units
template <int BM>
__device__ __forceinline__ void epilogue_bf16(const Gp& P, const float* part, bf16_t* out, int ldo) {
  int u0, u1;
  unit_range(P, u0, u1);
  const int nu = u1 - u0;
  for (int i = threadIdx.x; i < nu * BM; i += SNT) {
    const int ul = i / BM, b = i - ul * BM;
    st_bf16_dev(out + (int64_t)b * ldo + u0 + ul, row_sum<BM>(part, ul, b));
  }
}

// act = bf16(bf16(silu(bf16 g)) * bf16 u)   (ek_kernels.py:1247-1261, :1062-1076)
template <int BM>
__device__ __forceinline__ void epilogue_swiglu(const Gp& P, const float* part, bf16_t* out, int ldo) {
  int u0, u1;
  unit_range(P, u0, u1);
  const int nu = u1 - u0;
  for (int i = threadIdx.x; i < nu * BM; i += SNT) {
    const int ul = i / BM, b = i - ul * BM;
    const float gt = rbf(row_sum<BM>(part, ul, b));
    const float up = rbf(row_sum<BM>(part, nu + ul, b));
    const float s = rbf(gt / (1.0f + expf(-gt)));
    st_bf16_dev(out + (int64_t)b * ldo + u0 + ul, s * up);
  }
}

// (a better, b) under "larger value, then lower index"; index 0x7fffffff = none
__device__ __forceinline__ bool am_better(float v, int i, float cv, int ci) {
  return i != 0x7fffffff && (ci == 0x7fffffff || v > cv || (v == cv && i < ci));
}

// this workgroup's first-index argmax of the bf16 logits -> am_val/am_idx[wg * BM + b]
template <int BM>
__device__ __forceinline__ void epilogue_argmax(const Gp& P, const float* part, float* sv, int* si, float* am_val, int32_t* am_idx) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  int u0, u1;
  unit_range(P, u0, u1);
  const int nu = u1 - u0;
  float bv[BM];
  int bi[BM];
#pragma unroll
  for (int b = 0; b < BM; ++b) { bv[b] = -INFINITY; bi[b] = 0x7fffffff; }
  for (int ul = tid; ul < nu; ul += SNT) {
#pragma unroll
    for (int b = 0; b < BM; ++b) {
      const float v = rbf(row_sum<BM>(part, ul, b));
      if (am_better(v, u0 + ul, bv[b], bi[b])) { bv[b] = v; bi[b] = u0 + ul; }
    }
  }
#pragma unroll
  for (int b = 0; b < BM; ++b) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float v = __shfl_xor(bv[b], o, EK_WAVE);
      const int i = __shfl_xor(bi[b], o, EK_WAVE);
      if (am_better(v, i, bv[b], bi[b])) { bv[b] = v; bi[b] = i; }
    }
    if (lane == 0) { sv[wave * BM + b] = bv[b]; si[wave * BM + b] = bi[b]; }
  }
  __syncthreads();
  if (tid < BM) {
    float v = sv[tid];
    int i = si[tid];
    for (int w = 1; w < SNW; ++w)
      if (am_better(sv[w * BM + tid], si[w * BM + tid], v, i)) { v = sv[w * BM + tid]; i = si[w * BM + tid]; }
    __hip_atomic_store(am_val + blockIdx.x * BM + tid, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(am_idx + blockIdx.x * BM + tid, i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// prologues: the phase's activation rows -> xs [BM][kpad] (bf16, zero-padded)
// ---------------------------------------------------------------------------
template <int BM>
__device__ __forceinline__ void zero_part(float* part, int n) {
  for (int i = threadIdx.x; i < n; i += SNT) part[i] = 0.f;
}

template <int BM>
__device__ __forceinline__ void zero_pad(bf16_t* xs, int k, int kpad) {
  for (int i = threadIdx.x; i < BM * (kpad - k); i += SNT) {
    const int b = i / (kpad - k), e = i - b * (kpad - k);
    xs[b * kpad + k + e] = 0;
  }
}

// x as given (device-scope loads of another phase's output)
template <int BM>
__device__ __forceinline__ void plain_prologue(const bf16_t* src, int k, int kpad, bf16_t* xs) {
  const int nch = k / 8;
  for (int i = threadIdx.x; i < BM * nch; i += SNT) {
    const int b = i / nch, c = i - b * nch;
    *reinterpret_cast<uint4*>(xs + b * kpad + c * 8) = ld16_dev(src + (int64_t)b * k + c * 8);
  }
  zero_pad<BM>(xs, k, kpad);
}

// r = embed[token] (ra == nullptr) or bf16(ra + rb); r -> r_out (writer);
// xs = bf16(w * bf16(r * rsqrt(mean(r^2) + eps)))     (ek_kernels.py:1025-1059, 1296-1304)
template <int BM>
__device__ __forceinline__ void norm_prologue(const StepArgs& a, const bf16_t* ra, const bf16_t* rb, const bf16_t* nw,
                                              int k, int kpad, bf16_t* xs, bf16_t* r_out, float* red) {
  constexpr int NCH = 2;   // chunks of 8 per thread: k <= 2 * 8 * SNT (checked by the plan)
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int nch = k / 8;
  // the gain's chunks load with the activations (one memory round trip)
  uint4 gw[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = tid + j * SNT;
    gw[j] = c < nch ? ld16(nw + c * 8) : make_uint4(0, 0, 0, 0);
  }
  float ss[BM];
#pragma unroll
  for (int b = 0; b < BM; ++b) ss[b] = 0.f;
#pragma unroll
  for (int b = 0; b < BM; ++b) {
    const bf16_t* erow = nullptr;
    if (!ra) {
      int64_t t = a.tokens[b];
      t = t < 0 ? 0 : (t >= a.vocab ? a.vocab - 1 : t);
      erow = a.embed + t * a.lde;
    }
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = tid + j * SNT;
      if (c >= nch) continue;
      float r[8];
      if (!ra) {
        unpack8(ld16(erow + c * 8), r);
      } else {
        float x0[8], x1[8];
        unpack8(ld16_dev(ra + (int64_t)b * k + c * 8), x0);
        unpack8(ld16_dev(rb + (int64_t)b * k + c * 8), x1);
#pragma unroll
        for (int q = 0; q < 8; ++q) r[q] = rbf(x0[q] + x1[q]);
      }
      const uint4 pk = make_uint4(pack2(r[0], r[1]), pack2(r[2], r[3]), pack2(r[4], r[5]), pack2(r[6], r[7]));
      *reinterpret_cast<uint4*>(xs + b * kpad + c * 8) = pk;
      if (r_out) st16_dev(r_out + (int64_t)b * k + c * 8, pk);
#pragma unroll
      for (int q = 0; q < 8; ++q) ss[b] = fmaf(r[q], r[q], ss[b]);
    }
  }
#pragma unroll
  for (int b = 0; b < BM; ++b) {
    const float v = wave_sum(ss[b]);
    if (lane == 0) red[wave * BM + b] = v;
  }
  __syncthreads();
  float rstd[BM];
#pragma unroll
  for (int b = 0; b < BM; ++b) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < SNW; ++w) t += red[w * BM + b];
    rstd[b] = 1.0f / sqrtf(t / (float)k + a.eps);
  }
#pragma unroll
  for (int b = 0; b < BM; ++b) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = tid + j * SNT;
      if (c >= nch) continue;
      uint4* dst = reinterpret_cast<uint4*>(xs + b * kpad + c * 8);
      float r[8], g[8], o[8];
      unpack8(*dst, r);
      unpack8(gw[j], g);
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] = rbf(g[q] * rbf(r[q] * rstd[b]));
      *dst = make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
    }
  }
  zero_pad<BM>(xs, k, kpad);
}

// ---------------------------------------------------------------------------
// attention phase: workgroup w < B * n_kv * D / 32 runs unit w
// ---------------------------------------------------------------------------
template <int BM, int D, int G>
__device__ __forceinline__ void attention_phase(const StepArgs& a, const int64_t* lw, const bf16_t* qkv, bf16_t* att, int64_t hi,
                                unsigned char* smem) {
  const int bhn = BM * a.nkv;
  const int bh = blockIdx.x % bhn, c = blockIdx.x / bhn;
  const int b = bh / a.nkv, h = bh - b * a.nkv;
  const int qkvw = (a.nq + 2 * a.nkv) * D;
  // this unit's q heads, new key and new value -> LDS
  bf16_t* qrow = reinterpret_cast<bf16_t*>(smem);
  const bf16_t* src = qkv + (int64_t)b * qkvw;
  for (int i = threadIdx.x; i < (G + 2) * D / 8; i += SNT) {
    const int hh = i / (D / 8), c8 = i - hh * (D / 8);
    const int64_t off = hh < G ? (int64_t)(h * G + hh) * D
                               : (hh == G ? (int64_t)(a.nq + h) * D : (int64_t)(a.nq + a.nkv + h) * D);
    *reinterpret_cast<uint4*>(qrow + hh * D + c8 * 8) = ld16_dev(src + off + c8 * 8);
  }
  __syncthreads();
  eka::AttnUnit u;
  u.qh = qrow; u.q_stride = D;
  u.kh = qrow + G * D; u.vh = qrow + (G + 1) * D;
  u.rope = 1;
  u.qn = reinterpret_cast<const bf16_t*>(lw[LW_QN]);
  u.kn = reinterpret_cast<const bf16_t*>(lw[LW_KN]);
  int64_t crow = a.positions[b];
  crow = crow < 0 ? 0 : (crow >= a.rope_len ? a.rope_len - 1 : crow);
  u.cr = a.cos + crow * a.ld_cs;
  u.sr = a.sin + crow * a.ld_cs;
  u.eps = a.eps; u.sm_scale = a.sm_scale;
  u.kc = reinterpret_cast<bf16_t*>(lw[LW_KC]) + b * a.csb + h * a.csh;
  u.vc = reinterpret_cast<bf16_t*>(lw[LW_VC]) + b * a.csb + h * a.csh;
  u.css = a.css;
  u.cap = a.s_cap;
  int64_t lo = a.start_t[b];
  u.lo = lo < 0 ? 0 : lo;
  u.hi = hi;
  u.writer = c == 0;
  u.d0 = c * eka::FDC;
  u.out = att + (int64_t)b * a.nq * D + (int64_t)h * G * D;
  u.out_stride = D;
  u.coherent_out = true;
  eka::attn_unit<D, G, STU, SPT>(u, smem + eka::align16((size_t)(G + 2) * D * 2));
}

// ---------------------------------------------------------------------------
// the step
// ---------------------------------------------------------------------------
template <int BM, int D, int G>
__global__ __launch_bounds__(SNT) void step_kernel(StepArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_ok;
  __shared__ float s_red[SNW * BM];
  __shared__ int s_redi[SNW * BM];

  const int tid = threadIdx.x;
  unsigned gen = 0;
  if (tid == 0) gen = __hip_atomic_load(&a.bar->gen[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  const int h = a.h, inter = a.inter;
  const int qw = a.nq * D, qkvw = (a.nq + 2 * a.nkv) * D;
  const int64_t ls = arena_layer_elems(BM, h, inter, qkvw, qw);
  const int64_t len_old = *a.len_t;
  int64_t hi = len_old + 1;
  hi = hi < 0 ? 0 : (hi > a.s_cap ? a.s_cap : hi);

  bf16_t* xs = reinterpret_cast<bf16_t*>(smem);
  float* part = reinterpret_cast<float*>(smem + eka::align16((size_t)BM * a.kpad_max * 2));
  const int part_n = a.part_max * SNW * BM;
  bf16_t* wl = reinterpret_cast<bf16_t*>(smem + eka::align16((size_t)BM * a.kpad_max * 2) +
                                         eka::align16((size_t)part_n * 4));   // staged o_proj rows

  Ring ring;
  ring.ready = false;
#pragma unroll
  for (int u = 0; u < NB; ++u) ring.r[u] = make_uint4(0, 0, 0, 0);

  const bf16_t* prev_mid = nullptr;
  const bf16_t* prev_dn = nullptr;
  for (int l = 0; l < a.nl; ++l) {
    const int64_t* lw = a.lw + (int64_t)l * LW_FIELDS;
    bf16_t* base = a.arena + (int64_t)l * ls;
    bf16_t* r_in = base;
    bf16_t* r_mid = r_in + BM * h;
    bf16_t* qkv = r_mid + BM * h;
    bf16_t* att = qkv + BM * qkvw;
    bf16_t* o = att + BM * qw;
    bf16_t* act = o + BM * h;
    bf16_t* dn = act + BM * inter;
    const int n_attn = BM * a.nkv * (D / eka::FDC);   // attention units = workgroups [0, n_attn)
    const Gp gq = make_gp(reinterpret_cast<const bf16_t*>(lw[LW_QKV]), h, qkvw, 0);
    Gp go = make_gp(reinterpret_cast<const bf16_t*>(lw[LW_O]), qw, h, 0);
    go.wg0 = n_attn;                                 // o_proj rows go to the other workgroups,
    go.nwg = (int)gridDim.x - n_attn;                //   which stage them in LDS during attention
    const Gp gg = make_gp(reinterpret_cast<const bf16_t*>(lw[LW_GU]), h, inter, 1);
    const Gp gd = make_gp(reinterpret_cast<const bf16_t*>(lw[LW_DOWN]), inter, h, 0);
    Gp gnext;
    if (l + 1 < a.nl) gnext = make_gp(reinterpret_cast<const bf16_t*>(a.lw[(int64_t)(l + 1) * LW_FIELDS + LW_QKV]), h, qkvw, 0);
    else gnext = make_gp(a.lm_head, h, a.vocab, 0);

    // ---- r = (layer 0) embed[token] | r_mid(l-1) + down(l-1); norm; qkv
    zero_part<BM>(part, part_n);
    norm_prologue<BM>(a, prev_mid, prev_dn, reinterpret_cast<const bf16_t*>(lw[LW_LN1]), h, kpad_of(h), xs,
                      blockIdx.x == 0 ? r_in : nullptr, s_red);
    __syncthreads();
    gemv_phase<BM>(gq, ring, xs, kpad_of(h), part);
    __syncthreads();
    epilogue_bf16<BM>(gq, part, qkv, qkvw);
    const bool attn_wg = (int)blockIdx.x < n_attn;
    drain();
    if (!grid_sync(a.bar, gen, a.err, a.spin, true, &s_ok)) return;

    // ---- attention (QK-norm, RoPE, KV write, softmax, PV) on workgroups
    //      [0, n_attn); meanwhile the others copy their o_proj rows to LDS
    if (attn_wg) attention_phase<BM, D, G>(a, lw, qkv, att, hi, smem);
    else stage_rows_lds(go, wl);
    drain();
    if (!grid_sync(a.bar, gen, a.err, a.spin, true, &s_ok)) return;

    // ---- o projection (weights from LDS)
    zero_part<BM>(part, part_n);
    plain_prologue<BM>(att, qw, kpad_of(qw), xs);
    __syncthreads();
    gemv_lds_phase<BM>(go, wl, xs, kpad_of(qw), part);
    __syncthreads();
    epilogue_bf16<BM>(go, part, o, h);
    drain();
    prefetch_phase(&gg, ring);
    if (!grid_sync(a.bar, gen, a.err, a.spin, true, &s_ok)) return;

    // ---- r' = r + o; norm; gate/up; SwiGLU
    zero_part<BM>(part, part_n);
    norm_prologue<BM>(a, r_in, o, reinterpret_cast<const bf16_t*>(lw[LW_LN2]), h, kpad_of(h), xs,
                      blockIdx.x == 0 ? r_mid : nullptr, s_red);
    __syncthreads();
    gemv_phase<BM>(gg, ring, xs, kpad_of(h), part);
    __syncthreads();
    epilogue_swiglu<BM>(gg, part, act, inter);
    drain();
    prefetch_phase(&gd, ring);
    if (!grid_sync(a.bar, gen, a.err, a.spin, true, &s_ok)) return;

    // ---- down projection
    zero_part<BM>(part, part_n);
    plain_prologue<BM>(act, inter, kpad_of(inter), xs);
    __syncthreads();
    gemv_phase<BM>(gd, ring, xs, kpad_of(inter), part);
    __syncthreads();
    epilogue_bf16<BM>(gd, part, dn, h);
    drain();
    prefetch_phase(&gnext, ring);
    if (!grid_sync(a.bar, gen, a.err, a.spin, true, &s_ok)) return;
    prev_mid = r_mid;
    prev_dn = dn;
  }

  // ---- final add + norm, lm_head, per-workgroup argmax
  zero_part<BM>(part, part_n);
  norm_prologue<BM>(a, prev_mid, prev_dn, a.fnorm, h, kpad_of(h), xs, nullptr, s_red);
  __syncthreads();
  const Gp gl = make_gp(a.lm_head, h, a.vocab, 0);
  gemv_phase<BM>(gl, ring, xs, kpad_of(h), part);
  __syncthreads();
  epilogue_argmax<BM>(gl, part, s_red, s_redi, a.am_val, a.am_idx);
  drain();
  // every workgroup arrives; only workgroup 0 waits and finishes the step
  if (!grid_sync(a.bar, gen, a.err, a.spin, blockIdx.x == 0, &s_ok) || blockIdx.x != 0) return;

  // ---- token = first-index argmax over the partials; step bookkeeping
  //      (engine.py:289-292; slot/len advance of ek_model.py:375-388)
  const int lane = tid & 63, wave = wave_id();
#pragma unroll
  for (int b = 0; b < BM; ++b) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int w = tid; w < (int)gridDim.x; w += SNT) {
      const float v = __hip_atomic_load(a.am_val + w * BM + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int i = __hip_atomic_load(a.am_idx + w * BM + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float v = __shfl_xor(bv, o, EK_WAVE);
      const int i = __shfl_xor(bi, o, EK_WAVE);
      if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    if (lane == 0) { s_red[wave * BM + b] = bv; s_redi[wave * BM + b] = bi; }
  }
  __syncthreads();
  if (tid == 0) {
    const int64_t step = *a.step_idx;
    for (int b = 0; b < BM; ++b) {
      float v = s_red[b];
      int i = s_redi[b];
      for (int w = 1; w < SNW; ++w)
        if (am_better(s_red[w * BM + b], s_redi[w * BM + b], v, i)) { v = s_red[w * BM + b]; i = s_redi[w * BM + b]; }
      const int64_t tok = i == 0x7fffffff ? 0 : i;
      if (a.out_tok) a.out_tok[b] = tok;
      a.tokens[b] = tok;
      a.positions[b] += 1;
      a.slot_t[b] = len_old;
      if (step >= 0 && step < a.max_steps) a.out_buf[step * BM + b] = (int32_t)tok;
    }
    *a.len_t = len_old + 1;
    *a.step_idx = step + 1;
  }
}

// LDS bytes of step_kernel<BM, D, G> (o_rows: the most o_proj rows of one workgroup, qw = n_q * D)
template <int BM, int D, int G>
inline size_t step_lds_bytes(int kpad_max, int part_max, int64_t s_cap, int o_rows, int qw) {
  const size_t gemv = eka::align16((size_t)BM * kpad_max * 2) + eka::align16((size_t)part_max * SNW * BM * 4) +
                      (size_t)o_rows * qw * 2;
  const size_t attn = eka::align16((size_t)(G + 2) * D * 2) + eka::AttnLds<D, G>::bytes(s_cap);
  return gemv > attn ? gemv : attn;
}

// launch of one (BM, D) instantiation for any G (ek_step_inst.hip)
template <int BM, int D>
hipError_t launch_step(const StepArgs& a, int g, int nwg, hipStream_t st);

}  // namespace eks
