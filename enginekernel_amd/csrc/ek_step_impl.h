// The whole Qwen3 decode step (batch 1) as one persistent launch (gfx950).
//
// One 512-thread workgroup per CU runs every phase of the step -- per layer:
// residual add + RMSNorm + qkv projection, attention, o projection, residual
// add + RMSNorm + gate/up projection + SwiGLU, down projection; then the
// final add + norm, lm_head and argmax, and the step's bookkeeping.
//
// No grid barriers. Every activation one workgroup hands to another travels
// in dense 8-byte words of four bf16 values, each stored with one
// device-scope store with its sign bits flipped, so that no stored word is
// zero; the consumer polls the words themselves until they are nonzero. A
// hand-over therefore costs one store-to-load trip (about a microsecond
// under full HBM load) instead of a store drain, a barrier round trip and a
// separate load, and it reads 8 values per 16-byte load. The arena holds
// two halves: a launch with epoch e hands over through half e & 1 and, at
// entry, zeroes the whole of half (e + 1) & 1 for the next launch (the
// launches of one stream run one after another: nothing reads that half
// meanwhile, and the kernel boundary makes the zeros visible before the next
// launch starts). Every location of a half is written at most once per
// launch (one region per layer), so a nonzero word is always this launch's.
// Every workgroup keeps its own copy of the residual row in LDS and applies
// the same bf16 adds to it, so the residual never travels. The eight XCD L2
// caches are not coherent with each other: the words are stored and loaded
// with device scope (past the L2). Each workgroup advances its own epoch
// counter at entry, so all workgroups of a launch agree on it without
// talking. Every wait is bounded: a workgroup that polls past the limit sets
// the error word and leaves, and every other workgroup leaves at its next
// wait.
//
// Weights never depend on activations: before each wait a workgroup's waves
// load the first weight chunks of the coming phase into a register ring
// (which holds a workgroup's whole o_proj share at the Qwen3-4B shape), and
// while attention runs they also pull their first gate/up chunks into L2, so
// the HBM stream keeps going across the hand-overs. Every weight is read once
// per step, and its loads are marked non-temporal (ld16_nt): that streams
// them measurably faster (Qwen3-4B: 2.04 -> 1.93 ms per step) and leaves the
// L2 to the lines l2_touch places there.
//
// Projections: a phase's output rows (gate/up row pairs for SwiGLU) are split
// evenly over the workgroups in units of four rows (so that every output word
// is produced by one workgroup, its two 32-bit halves by two threads); a
// workgroup's (row, 1 KiB chunk) items are split evenly over its 8 waves.
// Lanes stream 16 B of a chunk (a wave reads 1 KiB per load instruction); fp32
// accumulation of exact bf16 products, a butterfly per row segment, and a
// fixed-order sum of the waves' partials in LDS.
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
// Weight chunks in flight per wave (the ring of a projection phase) and how
// many of them are prefetched ahead of a hand-over wait, per form of the
// step: loads return in order, so every chunk in flight when a wait begins is
// one its polls return behind. Short contexts: a ring of 6 with 3 prefetched
// measured 0.4 % faster than 8 with 4 (rings of 4, 5 or 7, or 2-4 ahead, no
// better); before the dense hand-over words 6 ahead had been the best.
// The split-attention form: 10 with 10 ahead (0.2-0.55 % faster than 8 with
// 8 from 1.7 K to 32 K contexts; 10 with 8, or 12 with 12, 2 % slower; 8 with
// 8 had been 0.6 % faster than 8 with 6; a ring of 6 there 0.4 % slower).
#ifndef EK_STEP_NB
#define EK_STEP_NB 6
#endif
#ifndef EK_STEP_PF
#define EK_STEP_PF 3
#endif
#ifndef EK_STEP_NB_LONG
#define EK_STEP_NB_LONG 10
#endif
#ifndef EK_STEP_PF_LONG
#define EK_STEP_PF_LONG 10
#endif
constexpr int NB = EK_STEP_NB;
constexpr int PF = EK_STEP_PF;
constexpr int NB_LONG = EK_STEP_NB_LONG;
constexpr int PF_LONG = EK_STEP_PF_LONG;
constexpr int OB = 12;                 // o_proj chunks per wave held in registers through attention
constexpr int CH = 8 * EK_WAVE;        // bf16 elements per chunk (1 KiB)
constexpr int LW_FIELDS = 10;          // per-layer pointer table row
constexpr int ATU = 6;                 // attention: 16-key score tiles per wave held in registers
constexpr int APT = 3;                 // attention: 32-key PV tiles per wave held in registers
constexpr int LLW = 10;                // tagged words in flight per thread
constexpr int HW = 1;                  // dense 16-byte units in flight per thread: rows up to 4096 wide
constexpr int AW = 3;                  // the same for the act row (up to 12288 wide)
constexpr int NGW = 4;                 // norm gain words per thread (hidden <= 2 * NGW * SNT)
constexpr int MAX_WG = 1024;
constexpr int MAX_LAYERS = 64;          // layer table rows held in LDS
constexpr size_t kStepDynLds = 160 * 1024 - 8 * 1024;   // dynamic LDS limit (the static arrays take the rest)

typedef unsigned long long llw_t;

// per-layer pointer table: [n_layers][LW_FIELDS] device addresses
enum { LW_QKV = 0, LW_O, LW_GU, LW_DOWN, LW_LN1, LW_LN2, LW_QN, LW_KN, LW_KC, LW_VC };

// launch state, zeroed once by the host
struct Bar {
  unsigned ep[MAX_WG];   // per-workgroup launch epoch
  int64_t* trace;        // -DEK_STEP_TRACE builds: per-phase timestamps [wg][layer][48]
  int64_t pad[7];
};

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
  bf16_t* logits;                      // optional [vocab] bf16 logits of the step (null on the hot path)
  llw_t* arena;                        // two halves of `half` words (the launch uses half ep & 1)
  int64_t half;
  Bar* bar; int* err; int64_t spin;
  int kpad_max, part_max, o_rows;      // LDS plan (host-computed, see make_plan in ek_step.hip)
  // long contexts (kernels with LONG set): every workgroup runs attention unit
  // (kv head w % nkv, key split w / nkv) of lsplit splits of at most lchunk keys;
  // lx words after the argmax words hold the splits' statistics and partial
  // outputs (one region for every layer: its words carry the layer in their tag)
  int lsplit, lchunk;
  int64_t lx;
  int m;                               // batch rows (the batch kernel, ek_bstep_impl.h; 0 for batch 1)
};

__host__ __device__ constexpr int cdiv_i(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ constexpr int kpad_of(int k) { return cdiv_i(k, CH) * CH; }

// dense words (4 values each) per layer and batch row of a half: qkv,
// attention out, o out, act, down out (every count a multiple of 8 values,
// so each region starts on 16 bytes)
__host__ __device__ inline int64_t arena_layer_words(int h, int inter, int qkvw, int qw) {
  return (int64_t)(qkvw + qw + h + inter + h) / 4;
}

// long-context mode's exchange words: (max, sum) per query head of every
// split, then every split's partial output
__host__ __device__ inline int64_t long_words(int nkv, int splits, int g, int d) {
  return (int64_t)nkv * splits * (2 * g + g * d);
}
// words of one half: every layer (mb batch rows each), two tagged argmax
// words per workgroup and row, then the long-context exchange (lx words, 0
// for the attention-unit kernel), rounded up to 256 bytes
__host__ __device__ inline int64_t arena_half_words(int nl, int h, int inter, int qkvw, int qw, int nwg, int mb,
                                                    int64_t lx) {
  const int64_t w = nl * mb * arena_layer_words(h, inter, qkvw, qw) + 2 * (int64_t)nwg * mb + lx;
  return (w + 31) / 32 * 32;
}
// the half a launch uses, from an arena of `bytes` (the caller's whole
// buffer: every launch on one buffer splits it the same way, whatever its plan)
__host__ __device__ inline int64_t arena_half_of(int64_t bytes) { return bytes / 2 / 256 * 32; }

// rows of one workgroup's largest phase share (units in quads, or single
// rows for lm_head), times two for the gate/up phase
__host__ __device__ inline int part_rows_max(int h, int inter, int qkvw, int vocab, int nwg, int o_rows) {
  int r = 4 * cdiv_i(qkvw / 4, nwg);
  r = r > 4 * cdiv_i(h / 4, nwg) ? r : 4 * cdiv_i(h / 4, nwg);
  r = r > 8 * cdiv_i(inter / 4, nwg) ? r : 8 * cdiv_i(inter / 4, nwg);
  r = r > cdiv_i(vocab, nwg) ? r : cdiv_i(vocab, nwg);
  r = r > o_rows ? r : o_rows;
  return r;
}

// -DEK_STEP_TRACE builds stamp phase events into LDS (a global store would
// delay the memory waits that follow it) and copy one layer's stamps to
// bar->trace[wg][layer][48] at the layer's end.
#ifdef EK_STEP_TRACE
#define EK_TS(ev) do { if (threadIdx.x == 0) ts_lds[ev] = wall_clock64(); } while (0)
#define EK_TS_FLUSH(layer) do { if (a.bar->trace && threadIdx.x < 48) \
    a.bar->trace[((int64_t)blockIdx.x * 40 + (layer)) * 48 + threadIdx.x] = ts_lds[threadIdx.x]; } while (0)
#define EK_TS_FLUSH_SYNC(layer) do { __syncthreads(); EK_TS_FLUSH(layer); } while (0)
#else
#define EK_TS_FLUSH_SYNC(layer) do { } while (0)
#define EK_TS(ev) do { } while (0)
#define EK_TS_FLUSH(layer) do { } while (0)
#endif

// ---------------------------------------------------------------------------
// hand-over words
// ---------------------------------------------------------------------------
// Tagged words {32-bit data, 32-bit tag}, for the few values that are not
// bf16 activations: the argmax words (written once per launch, tag AM_TAG)
// and the long-context exchange (one region reused by every layer, tag
// layer + 1). They live in the launch's half too, so a zeroed word never
// matches a tag.
constexpr uint32_t AM_TAG = 1;

__device__ __forceinline__ void ll_put(llw_t* p, uint32_t data, uint32_t tag) {
  __hip_atomic_store(p, ((llw_t)tag << 32) | data, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ llw_t ll_get(const llw_t* p) {
  return __hip_atomic_load(const_cast<llw_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool ll_ok(llw_t v, uint32_t tag) { return (uint32_t)(v >> 32) == tag; }

// Wait until the n words src(i), i < n, carry tag `ep` and store their data
// halves in dst[i] (LDS). Thread t handles i = t + k * SNT; up to LLW words
// per thread are in flight at once, and only the words not yet valid are
// loaded again. False (the error word set) when a wait runs out.
struct LinDst {   // word i -> LDS word i
  __device__ int operator()(int i) const { return i; }
};

template <int W = LLW, typename SRC, typename DST = LinDst>
__device__ __forceinline__ bool ll_read(SRC src, int n, uint32_t ep, uint32_t* dst, int* err, int64_t spin,
                                        int64_t* rounds = nullptr, DST dix = DST()) {
  const int tid = threadIdx.x;
  for (int base = 0; base < n; base += W * SNT) {
    llw_t v[W];
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const int i = base + tid + k * SNT;
      v[k] = i < n ? ll_get(src(i)) : ((llw_t)ep << 32);
    }
    int64_t it = 0;
    while (true) {
      bool done = true;
#pragma unroll
      for (int k = 0; k < W; ++k) done = done && ll_ok(v[k], ep);
      if (done) break;
      if (rounds) ++*rounds;
      if (++it > spin) {
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
      if ((it & 63) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        const int i = base + tid + k * SNT;
        if (!ll_ok(v[k], ep)) v[k] = ll_get(src(i));
      }
    }
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const int i = base + tid + k * SNT;
      if (i < n) dst[dix(i)] = (uint32_t)v[k];
    }
  }
  return true;
}

// True when every thread of the workgroup passed ok. A failing thread sets
// the LDS flag before the barrier; the flag is zeroed at kernel entry and a
// workgroup that sees it set leaves the step, so it never needs clearing.
// (__syncthreads_and reads the dispatch packet from memory and takes three
// barriers.)
__device__ __forceinline__ bool wg_all(bool ok, int* s_fail) {
  if (!ok) *s_fail = 1;
  __syncthreads();
  return *s_fail == 0;   // the barrier's fences order this read after every thread's write
}

struct LinSrc {   // words [0, n) of one region
  const llw_t* p;
  __device__ const llw_t* operator()(int i) const { return p + i; }
};

// One thread's wait for one word (the data half into `out`); false (the
// error word set) when the wait runs out or another wait gave up.
__device__ __forceinline__ bool ll_wait1(const llw_t* p, uint32_t tag, uint32_t& out, int* err, int64_t spin) {
  llw_t v = ll_get(p);
  int64_t it = 0;
  while (!ll_ok(v, tag)) {
    if (++it > spin) {
      __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    if ((it & 63) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
    v = ll_get(p);
  }
  out = (uint32_t)v;
  return true;
}

// Two words (16 bytes) at byte offset `off` of a region, loaded with device
// scope: the cache-policy bits of the agent-scope atomic load (sc1) on a
// buffer load, since a 16-byte load has no atomic form. Each 32-bit quarter
// is checked on its own: a word is one producer store, or two half-word
// stores from two producers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dw_rsrc(const llw_t* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<llw_t*>(base), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ u32x4_t dw_get2(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
}
// (every quarter nonzero, as one unsigned min and one compare per unit: the
// same test as four compares, which measured 0.6 % / 1.7 % slower at 1 / 8
// rows; the min form measured faster than the older per-word test)
__device__ __forceinline__ bool dw_ok2(const u32x4_t& v) {
  return __builtin_elementwise_min(__builtin_elementwise_min(v.x, v.y), __builtin_elementwise_min(v.z, v.w)) != 0u;
}

// Wait until the n units j < n (16 bytes at byte offset src(j) of the region
// at base, 8 values) are written, and store their values in LDS at
// dst + dix(j) (a u32 index, a multiple of 4). Thread t handles j = t + k SNT;
// up to W units per thread are in flight at once, and only the units not
// yet whole are loaded again. False (the error word set) when a wait runs out.
struct LinUnits {   // unit j of one region -> byte 16 j; LDS u32 4 j
  __device__ int operator()(int j) const { return 16 * j; }
};
struct LinLds {
  __device__ int operator()(int j) const { return 4 * j; }
};

// units j of a map shifted by b0 (a later round of a read)
template <typename F>
struct OffUnits {
  F f;
  int b0;
  __device__ int operator()(int j) const { return f(b0 + j); }
};

// dw_read of at most W SNT units in two halves, for a wait whose loads go
// out early (ahead of other work): dw_issue loads every unit once into v;
// dw_finish polls the units not yet whole and stores all of them in LDS.
template <int W, typename SRC>
__device__ __forceinline__ void dw_issue(const llw_t* base, SRC src, int n, u32x4_t* v) {
  const __amdgpu_buffer_rsrc_t r = dw_rsrc(base);
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const int j = (int)threadIdx.x + k * SNT;
    v[k] = dw_get2(r, src(j < n ? j : 0));
  }
}

// dw_wait: the wait alone, the words left in v (for a reader that uses them
// in registers). dw_finish repeats its loop rather than calling it: the
// batch kernel measured 0.5 % slower with the call.
template <int W, typename SRC>
__device__ __forceinline__ bool dw_wait(const llw_t* base, SRC src, int n, u32x4_t* v, int* err, int64_t spin,
                                        int64_t* rounds = nullptr) {
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t r = dw_rsrc(base);
  int64_t it = 0;
  while (true) {
    bool done = true;
#pragma unroll
    for (int k = 0; k < W; ++k) done = done && (tid + k * SNT >= n || dw_ok2(v[k]));
    if (done) break;
    if (rounds) ++*rounds;
    if (++it > spin) {
      __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    if ((it & 63) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
    // the buffer-load builtin reads as ordinary memory: without this
    // compiler barrier a re-poll may be merged with the earlier load of the
    // same word (the loop's only other memory operation, the error word's
    // load, runs once in 64 rounds)
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const int j = tid + k * SNT;
      if (j < n && !dw_ok2(v[k])) v[k] = dw_get2(r, src(j));
    }
  }
  return true;
}

template <int W, typename SRC, typename DST>
__device__ __forceinline__ bool dw_finish(const llw_t* base, SRC src, int n, u32x4_t* v, uint32_t* dst, DST dix,
                                          int* err, int64_t spin, int64_t* rounds = nullptr) {
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t r = dw_rsrc(base);
  int64_t it = 0;
  while (true) {
    bool done = true;
#pragma unroll
    for (int k = 0; k < W; ++k) done = done && (tid + k * SNT >= n || dw_ok2(v[k]));
    if (done) break;
    if (rounds) ++*rounds;
    if (++it > spin) {
      __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    if ((it & 63) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
    // the buffer-load builtin reads as ordinary memory: without this
    // compiler barrier a re-poll may be merged with the earlier load of the
    // same word (the loop's only other memory operation, the error word's
    // load, runs once in 64 rounds)
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const int j = tid + k * SNT;
      if (j < n && !dw_ok2(v[k])) v[k] = dw_get2(r, src(j));
    }
  }
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const int j = tid + k * SNT;
    if (j < n)
      *reinterpret_cast<uint4*>(dst + dix(j)) =
          make_uint4(v[k].x ^ DW_FLIP32, v[k].y ^ DW_FLIP32, v[k].z ^ DW_FLIP32, v[k].w ^ DW_FLIP32);
  }
  return true;
}

// dw_issue for a wait that follows at once: a slot past the last unit loads
// nothing (dw_issue loads unit 0 there, so that a wait issued ahead of other
// loads can count its own)
template <int W, typename SRC>
__device__ __forceinline__ void dw_issue_now(const llw_t* base, SRC src, int n, u32x4_t* v) {
  const __amdgpu_buffer_rsrc_t r = dw_rsrc(base);
#pragma unroll
  for (int k = 0; k < W; ++k) {
    const int j = (int)threadIdx.x + k * SNT;
    v[k] = u32x4_t{0u, 0u, 0u, 0u};
    if (j < n) v[k] = dw_get2(r, src(j));
  }
}

// MASK: the first loads through dw_issue_now. The batch-1 step's reads use it
// (1.6 % faster at 4 K and 16 K contexts, 0.1 % at short ones, where a 2560-
// value row leaves 192 of 512 slots empty); the batch kernel's reads, whose
// slots are nearly all units, measured 0.45 % slower with it.
template <int W, bool MASK = false, typename SRC, typename DST>
__device__ __forceinline__ bool dw_read(const llw_t* base, SRC src, int n, uint32_t* dst, DST dix, int* err,
                                        int64_t spin, int64_t* rounds = nullptr) {
  for (int b0 = 0; b0 < n; b0 += W * SNT) {
    const OffUnits<SRC> s2{src, b0};
    const OffUnits<DST> d2{dix, b0};
    u32x4_t v[W];
    if constexpr (MASK) dw_issue_now<W>(base, s2, n - b0, v);
    else dw_issue<W>(base, s2, n - b0, v);
    if (!dw_finish<W>(base, s2, n - b0, v, dst, d2, err, spin, rounds)) return false;
  }
  return true;
}

// Zero this workgroup's share of the half the next launch uses (16-byte
// global stores spread over the grid; a.half is a multiple of 32 words).
typedef __attribute__((address_space(1))) u32x4_t global_w_u32x4_t;
__device__ __forceinline__ void clear_next_half(const StepArgs& a, uint32_t ep) {
  global_w_u32x4_t* h = (global_w_u32x4_t*)(a.arena + (int64_t)((ep + 1u) & 1u) * a.half);
  const int64_t n = a.half / 2;
  const u32x4_t z = {0u, 0u, 0u, 0u};
  for (int64_t i = (int64_t)blockIdx.x * SNT + threadIdx.x; i < n; i += (int64_t)gridDim.x * SNT) h[i] = z;
}

// the half this launch hands over through
__device__ __forceinline__ llw_t* cur_half(const StepArgs& a, uint32_t ep) {
  return a.arena + (int64_t)(ep & 1u) * a.half;
}

// ---------------------------------------------------------------------------
// projections
// ---------------------------------------------------------------------------
// The chunk dot product of the projections: on the bf16 dot instruction
// (the phases after a hand-over are bound by these instructions, not by
// memory, when their weights are already in registers).
__device__ __forceinline__ float step_dot8(const uint4& w, const uint4& x, float acc) {
  return dot8_acc_d2(w, x, acc);
}
struct Gp {
  const bf16_t* w;   // [rows, K] row-major
  int K, C;          // reduction length, 1 KiB chunks per row
  int units;         // output units
  int pair;          // 1: unit u is rows u and up_off + u (gate/up)
  int up_off;
  int gran;          // units per workgroup share come in multiples of gran
  int wg0, nwg;      // the units are spread over workgroups [wg0, wg0 + nwg)
};

__device__ __forceinline__ Gp make_gp(const bf16_t* w, int k, int units, int pair, int gran) {
  Gp g;
  g.w = w; g.K = k; g.C = cdiv_i(k, CH); g.units = units; g.pair = pair; g.up_off = units; g.gran = gran;
  g.wg0 = 0; g.nwg = gridDim.x;
  return g;
}

// this workgroup's units [u0, u1) (empty outside the phase's workgroups)
__device__ __forceinline__ void unit_range(const Gp& g, int& u0, int& u1) {
  const int w = (int)blockIdx.x - g.wg0;
  if (w < 0 || w >= g.nwg) { u0 = u1 = 0; return; }
  // 32-bit arithmetic (the plan bounds units / gran * workgroups below 2^31):
  // a 64-bit division is a long emulated sequence
  const uint32_t n = (uint32_t)(g.units / g.gran);
  u0 = g.gran * (int)(n * (uint32_t)w / (uint32_t)g.nwg);
  u1 = g.gran * (int)(n * (uint32_t)(w + 1) / (uint32_t)g.nwg);
}

struct WaveItems { int i0, n; };

__device__ __forceinline__ WaveItems wave_items(const Gp& g, int nu, int wave) {
  const int n_items = nu * (g.pair ? 2 : 1) * g.C;
  const int i0 = (int)((uint32_t)n_items * (uint32_t)wave / (uint32_t)SNW);
  const int i1 = (int)((uint32_t)n_items * (uint32_t)(wave + 1) / (uint32_t)SNW);
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

// The wave's ring: slots [0, nready) hold items 0 .. nready-1 of the coming
// phase (loaded ahead by prefetch_phase).
template <int N>
struct RingN {
  uint4 r[N];
  int nready;
};

// The first `cnt` items of phase `pn` into this wave's ring, issued ahead of
// a wait so that they load while the workgroup waits for its inputs. Loads
// retire in order, so every item prefetched here is also a load the wait's
// own polls queue behind: ahead of a short hand-over only a few are worth it.
template <int CNT, int R>
__device__ __forceinline__ void prefetch_phase(const Gp& pn, RingN<R>& ring) {
  static_assert(CNT <= R, "prefetch within the ring");
  const Span sn = make_span(pn, wave_id());
  const int loff = (threadIdx.x & 63) * 8;
#pragma unroll
  for (int u = 0; u < CNT; ++u) ring.r[u] = ld16_nt(span_item(sn, sn.i0 + (u < sn.n ? u : 0)) + loff);
  ring.nready = CNT;
}

// The o projection's chunks, loaded into registers while attention runs and
// consumed once its output arrives. When a row is exactly SNW chunks long
// and the workgroup's rows fit the OB registers (the Qwen3-4B shape: 4096 /
// 512 = 8 chunks, at most 12 rows), wave w holds chunk w of every row
// ("by column"): its products then need one activation chunk from LDS
// instead of one per item, and its rows' sums run as one interleaved DPP
// reduction. Otherwise a wave holds its first OB items (row-major order)
// and items past OB (larger shapes) load one by one.
__device__ __forceinline__ bool held_by_column(const Gp& P, int& u0, int& nr) {
  int u1;
  unit_range(P, u0, u1);
  nr = u1 - u0;
  return !P.pair && P.C == SNW && nr <= OB;
}

__device__ __forceinline__ void hold_phase(const Gp& P, uint4* ob) {
  const int loff = (threadIdx.x & 63) * 8;
  int u0, nr;
  if (held_by_column(P, u0, nr)) {
    const bf16_t* col = P.w + (int64_t)u0 * P.K + wave_id() * CH + loff;
#pragma unroll
    for (int u = 0; u < OB; ++u) ob[u] = ld16_nt(col + (int64_t)(u < nr ? u : 0) * P.K);
    return;
  }
  const Span sn = make_span(P, wave_id());
#pragma unroll
  for (int u = 0; u < OB; ++u) ob[u] = ld16_nt(span_item(sn, sn.i0 + (u < sn.n ? u : 0)) + loff);
}

// The held-by-column products: row u's partial over chunk `wave` (this
// lane's 8 values of it in xw) -> part[u * SNW + wave]
__device__ __forceinline__ void held_col_products(const uint4* ob, const uint4& xw, float* part, int nr) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  float acc[OB];
#pragma unroll
  for (int u = 0; u < OB; ++u) acc[u] = step_dot8(ob[u], xw, 0.f);
  wave_sums_dpp_lane63<OB>(acc);
  if (lane == 63) {
#pragma unroll
    for (int u = 0; u < OB; ++u)
      if (u < nr) part[u * SNW + wave] = acc[u];
  }
}

__device__ __forceinline__ void gemv_held_phase(const Gp& P, const uint4* ob, const bf16_t* xs, float* part) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  {
    int u0, nr;
    if (held_by_column(P, u0, nr)) {
      held_col_products(ob, *reinterpret_cast<const uint4*>(xs + wave * CH + lane * 8), part, nr);
      return;
    }
  }
  const Span sp = make_span(P, wave);
  const int n = sp.n;
  const int loff = lane * 8;
  int r = sp.i0 / P.C, ch = sp.i0 - (sp.i0 / P.C) * P.C;
  // the activation chunk of every held item, read from LDS up front (item k
  // of the wave uses chunk (ch + k) mod C of x): one LDS wait for all of
  // them instead of one per item
  uint4 xr[OB];
  {
    int c = ch;
#pragma unroll
    for (int u = 0; u < OB; ++u) {
      xr[u] = *reinterpret_cast<const uint4*>(xs + c * CH + loff);
      if (++c == P.C) c = 0;
    }
  }
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < OB; ++u) {
    if (u < n) {
      acc = step_dot8(ob[u], xr[u], acc);
      if (ch == P.C - 1 || u == n - 1) {
        const float sum = wave_sum_dpp(acc);
        if (lane == 0) part[r * SNW + wave] = sum;
        acc = 0.f;
      }
      if (++ch == P.C) { ch = 0; ++r; }
    }
  }
  for (int k = OB; k < n; ++k) {
    acc = step_dot8(ld16_nt(span_item(sp, sp.i0 + k) + loff), *reinterpret_cast<const uint4*>(xs + ch * CH + loff), acc);
    if (ch == P.C - 1 || k == n - 1) {
      const float sum = wave_sum_dpp(acc);
      if (lane == 0) part[r * SNW + wave] = sum;
      acc = 0.f;
    }
    if (++ch == P.C) { ch = 0; ++r; }
  }
}

// Bring items [PF, PF + L2T) of this wave's share of phase `pn` (the ones
// after its ring prefetch) into the L2 (one 4-byte load per 64-byte sector),
// so that the phase later reads them from L2 instead of HBM. The loaded words are
// folded into `sink`, which the caller consumes where it waits anyway.
#ifndef EK_STEP_L2T
#define EK_STEP_L2T 8
#endif
constexpr int L2T = EK_STEP_L2T;

__device__ __forceinline__ void l2_touch(const Gp& pn, uint32_t& sink) {
  const Span sn = make_span(pn, wave_id());
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < L2T / 4; ++j) {
    const int i = PF + 4 * j + (lane >> 4);
    // clamped, not conditional: a load under a lane condition is a branch that waits for it
    sink ^= ld4(span_item(sn, sn.i0 + (i < sn.n ? i : 0)) + (lane & 15) * 32);
  }
}

// One projection phase: partial dot products of this wave's items into
// part[row_local * SNW + wave]. The ring is consumed in order and each slot
// is refilled, right after its chunk is consumed, with the item R places
// ahead, so R chunks stay in flight and a refill never waits for anything
// but its own slot's previous load. The ring holds items 0 .. R-1 on entry
// when prefetch_phase loaded them. Refills past the wave's last item (every
// slot is refilled, so that the loads stay countable at compile time and R
// stay in flight) re-read that last item, which the L2 has just fetched.
template <int R>
__device__ __forceinline__ void gemv_phase(const Gp& P, RingN<R>& ring, const bf16_t* xs, float* part) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const Span sp = make_span(P, wave);
  const int n = sp.n;
  const int loff = lane * 8;
#pragma unroll
  for (int u = 0; u < R; ++u)
    if (u >= ring.nready) ring.r[u] = ld16_nt(span_item(sp, sp.i0 + (u < n ? u : 0)) + loff);
  int r = sp.i0 / P.C, ch = sp.i0 - (sp.i0 / P.C) * P.C;   // consume position (row-local, chunk)
  // the activation chunk of the current item; the next item's chunk is read
  // from LDS before the current item's products, so the LDS round trip
  // overlaps them instead of stalling every item
  uint4 xc = *reinterpret_cast<const uint4*>(xs + ch * CH + loff);
  float acc = 0.f;
  int k0 = 0;
  for (; k0 + R <= n; k0 += R) {
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int chn = ch + 1 == P.C ? 0 : ch + 1;
      const uint4 xn = *reinterpret_cast<const uint4*>(xs + chn * CH + loff);
      acc = step_dot8(ring.r[u], xc, acc);
      const int kn = k0 + u + R;
      ring.r[u] = ld16_nt(span_item(sp, sp.i0 + (kn < n ? kn : n - 1)) + loff);
      if (ch == P.C - 1) {
        const float sum = wave_sum_dpp(acc);
        if (lane == 0) part[r * SNW + wave] = sum;
        acc = 0.f;
      }
      if (++ch == P.C) { ch = 0; ++r; }
      xc = xn;
    }
  }
#pragma unroll
  for (int u = 0; u < R; ++u) {
    if (k0 + u < n) {
      const int chn = ch + 1 == P.C ? 0 : ch + 1;
      const uint4 xn = *reinterpret_cast<const uint4*>(xs + chn * CH + loff);
      acc = step_dot8(ring.r[u], xc, acc);
      xc = xn;
      if (ch == P.C - 1 || k0 + u == n - 1) {
        const float sum = wave_sum_dpp(acc);
        if (lane == 0) part[r * SNW + wave] = sum;
        acc = 0.f;
      }
      if (++ch == P.C) { ch = 0; ++r; }
    }
  }
  if (k0 == n && n > 0 && ch != 0) {   // the wave's items ended inside a row at a block edge
    const float sum = wave_sum_dpp(acc);
    if (lane == 0) part[r * SNW + wave] = sum;
  }
  ring.nready = 0;
}

// sum of the waves' partials of row_local r, fixed order
__device__ __forceinline__ float row_sum(const float* part, int r) {
  static_assert(SNW == 8, "two 16-byte reads per row sum");
  const float4* p = reinterpret_cast<const float4*>(part + r * SNW);
  const float4 a = p[0], b = p[1];
  return ((((((a.x + a.y) + a.z) + a.w) + b.x) + b.y) + b.z) + b.w;   // in wave order
}

// out word (u0 + 4i) / 4 = bf16 rows u0 + 4i .. u0 + 4i + 3 of this
// workgroup's rows (units in quads)
__device__ __forceinline__ void epilogue_ll(const Gp& P, const float* part, llw_t* out) {
  int u0, u1;
  unit_range(P, u0, u1);
  // a thread per row pair (32-bit halves of the words): twice the threads of
  // a thread per word, each with half the row sums on its path
  const int np = (u1 - u0) / 2;
  for (int i = threadIdx.x; i < np; i += SNT)
    dw_put1(reinterpret_cast<uint32_t*>(out) + u0 / 2 + i, pack2(row_sum(part, 2 * i), row_sum(part, 2 * i + 1)));
}

// act = bf16(bf16(silu(bf16 g)) * bf16 u)   (ek_kernels.py:1247-1261, :1062-1076)
__device__ __forceinline__ float swiglu_one(const float* part, int nu, int ul) {
  const float gt = rbf(row_sum(part, ul));
  const float up = rbf(row_sum(part, nu + ul));
  const float s = rbf(gt / (1.0f + expf(-gt)));
  return s * up;
}

__device__ __forceinline__ void epilogue_swiglu_ll(const Gp& P, const float* part, llw_t* out) {
  int u0, u1;
  unit_range(P, u0, u1);
  const int nu = u1 - u0, np = nu / 2;
  for (int i = threadIdx.x; i < np; i += SNT)
    dw_put1(reinterpret_cast<uint32_t*>(out) + u0 / 2 + i,
            pack2(swiglu_one(part, nu, 2 * i), swiglu_one(part, nu, 2 * i + 1)));
}

// (a better, b) under "larger value, then lower index"; index 0x7fffffff = none
__device__ __forceinline__ bool am_better(float v, int i, float cv, int ci) {
  return i != 0x7fffffff && (ci == 0x7fffffff || v > cv || (v == cv && i < ci));
}

// this workgroup's first-index argmax of the bf16 logits -> two words at am
__device__ __forceinline__ void wg_argmax(float bv, int bi, float* sv, int* si, float& ov, int& oi) {
  const int lane = threadIdx.x & 63, wave = wave_id();
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v = __shfl_xor(bv, o, EK_WAVE);
    const int i = __shfl_xor(bi, o, EK_WAVE);
    if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
  }
  if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
  __syncthreads();
  ov = sv[0]; oi = si[0];
  for (int w = 1; w < SNW; ++w)
    if (am_better(sv[w], si[w], ov, oi)) { ov = sv[w]; oi = si[w]; }
}

__device__ __forceinline__ void epilogue_argmax_ll(const Gp& P, const float* part, float* sv, int* si, llw_t* am,
                                                   bf16_t* logits) {
  int u0, u1;
  unit_range(P, u0, u1);
  const int nu = u1 - u0;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int ul = threadIdx.x; ul < nu; ul += SNT) {
    const float v = rbf(row_sum(part, ul));
    if (logits) logits[u0 + ul] = (bf16_t)f2bf(v);
    if (am_better(v, u0 + ul, bv, bi)) { bv = v; bi = u0 + ul; }
  }
  float ov;
  int oi;
  wg_argmax(bv, bi, sv, si, ov, oi);
  if (threadIdx.x == 0) {
    ll_put(am + 2 * blockIdx.x, __float_as_uint(ov), AM_TAG);
    ll_put(am + 2 * blockIdx.x + 1, (uint32_t)oi, AM_TAG);
  }
}

// ---------------------------------------------------------------------------
// prologues
// ---------------------------------------------------------------------------
__device__ __forceinline__ void zero_part(float* part, int n) {
  for (int i = threadIdx.x; i < n; i += SNT) part[i] = 0.f;
}

__device__ __forceinline__ void zero_pad(bf16_t* xs, int k, int kpad) {
  for (int i = k + threadIdx.x; i < kpad; i += SNT) xs[i] = 0;
}

// the norm gain's words of this thread (i = tid + j * SNT), loaded ahead of a wait
// (every load issued, at a clamped index, then masked: a load under a lane
// condition becomes a branch that waits for it)
__device__ __forceinline__ void load_gain(const bf16_t* nw, int k, uint32_t* gw) {
  const uint32_t* g32 = reinterpret_cast<const uint32_t*>(nw);
  const int nwd = k / 2;
#pragma unroll
  for (int j = 0; j < NGW; ++j) {
    const int i = threadIdx.x + j * SNT;
    const uint32_t v = ld4(g32 + (i < nwd ? i : 0));
    gw[j] = i < nwd ? v : 0u;
  }
}

__device__ __forceinline__ uint32_t add2_bf(uint32_t r, uint32_t x) { return pack2(lo_bf(r) + lo_bf(x), hi_bf(r) + hi_bf(x)); }
// ss + the squares of both halves of a word, on the bf16 dot instruction
// (the bf16 squares are exact in fp32; one instruction instead of two
// unpacks and two FMAs)
__device__ __forceinline__ float sq2(uint32_t r, float ss) {
  const ek_bf16x2 v = __builtin_bit_cast(ek_bf16x2, r);
  return __builtin_amdgcn_fdot2_f32_bf16(v, v, ss, false);
}
// bf16(g * bf16(r * rstd)) for both halves of a word: each rounding converts
// the two values in one instruction (rounding an already rounded value is
// exact, so the result is that of rounding each value on its own)
__device__ __forceinline__ uint32_t norm2(uint32_t r, uint32_t g, float rstd) {
  const uint32_t t = pack2(lo_bf(r) * rstd, hi_bf(r) * rstd);
  return pack2(lo_bf(g) * lo_bf(t), hi_bf(g) * hi_bf(t));
}


// 16 bytes from global memory (a global, not flat, load)
typedef const __attribute__((address_space(1))) u32x4_t global_u4_t;
__device__ __forceinline__ uint4 ld16g(const void* p) {
  const u32x4_t v = *(global_u4_t*)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// the norm gain's unit of this thread (values 8 tid .. +7; loaded at a
// clamped index, used only by the threads that own a unit)
__device__ __forceinline__ uint4 load_gain_u(const bf16_t* nw, int k) {
  const int t = threadIdx.x, nu = k / 8;
  return ld16g(nw + 8 * (t < nu ? t : 0));
}

// The residual row held by unit: thread t < k / 8 keeps values 8 t .. +7
// (bf16 pairs, exact: every add rounds to bf16). rres = bf16(rres + x) when
// x is given (the hand-over unit this thread waited for, flipped words); the
// squares' sum of the row (per thread, wave, then the workgroup in wave order
// through red) and the wait's vote share one barrier; xs's unit t =
// bf16(g * bf16(r * rsqrt(mean(r^2) + eps))). False when a wait gave up.
__device__ __forceinline__ bool add_norm_u(uint4& rres, const u32x4_t* x, const uint4& g, int k, int kpad,
                                           float eps, bf16_t* xs, float* red, bool ok, int* s_fail) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const bool mine = tid < k / 8;
  float ss = 0.f;
  if (mine) {
    if (x) {
      rres.x = add2_bf(rres.x, x->x ^ DW_FLIP32);
      rres.y = add2_bf(rres.y, x->y ^ DW_FLIP32);
      rres.z = add2_bf(rres.z, x->z ^ DW_FLIP32);
      rres.w = add2_bf(rres.w, x->w ^ DW_FLIP32);
    }
    ss = sq2(rres.w, sq2(rres.z, sq2(rres.y, sq2(rres.x, 0.f))));
  }
  ss = wave_sum_dpp(ss);
  if (lane == 0) red[wave] = ss;
  if (!ok) *s_fail = 1;
  __syncthreads();
  if (*s_fail) return false;
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < SNW; ++w) t += red[w];
  const float rstd = 1.0f / sqrtf(t / (float)k + eps);
  if (mine)
    reinterpret_cast<uint4*>(xs)[tid] = make_uint4(norm2(rres.x, g.x, rstd), norm2(rres.y, g.y, rstd),
                                                   norm2(rres.z, g.z, rstd), norm2(rres.w, g.w, rstd));
  zero_pad(xs, k, kpad);
  return true;
}

// the residual unit of this thread's hand-over words: waited for into registers
__device__ __forceinline__ bool wait_res(const llw_t* src, int k, u32x4_t* v, const StepArgs& a) {
  dw_issue_now<1>(src, LinUnits{}, k / 8, v);
  return dw_wait<1>(src, LinUnits{}, k / 8, v, a.err, a.spin);
}


// The qkv units (8 values) an attention unit of kv head h reads, in its LDS
// order: its G query heads, the new key, the new value (byte offsets in the
// qkv region of one batch row)
template <int D, int G>
struct HeadUnits {
  int h, nq, nkv;
  __device__ int operator()(int j) const {
    const int t = j / (D / 8), r = j - t * (D / 8);
    const int head = t < G ? h * G + t : (t == G ? nq + h : nq + nkv + h);
    return head * D * 2 + r * 16;
  }
};

// ---------------------------------------------------------------------------
// attention phase: workgroup w < n_kv * D / 32 runs unit w
// ---------------------------------------------------------------------------
template <int D, int G>
__device__ __forceinline__ bool attention_phase(const StepArgs& a, const int64_t* lw, const llw_t* qkv, llw_t* att,
                                                int64_t hi, unsigned char* smem, int* s_fail, int layer
#ifdef EK_STEP_TRACE
                                                , int64_t* ts_lds
#endif
                                                ) {
  (void)layer;
  const int h = (int)blockIdx.x % a.nkv, c = (int)blockIdx.x / a.nkv;
  // this unit's q heads, new key and new value -> LDS (bf16 rows)
  bf16_t* qrow = reinterpret_cast<bf16_t*>(smem);
  const HeadUnits<D, G> src{h, a.nq, a.nkv};
  // the q/k norm gains and this position's cos/sin rows, copied to LDS while
  // the unit waits, so that the RoPE work after the wait reads only LDS
  bf16_t* rope_lds = qrow + (G + 2) * D;   // [q gain | k gain | cos | sin] x D
  const bf16_t* qn = reinterpret_cast<const bf16_t*>(lw[LW_QN]);
  const bf16_t* kn = reinterpret_cast<const bf16_t*>(lw[LW_KN]);
  int64_t crow = a.positions[0];
  crow = crow < 0 ? 0 : (crow >= a.rope_len ? a.rope_len - 1 : crow);
  const bf16_t* cr = a.cos + crow * a.ld_cs;
  const bf16_t* sr = a.sin + crow * a.ld_cs;
  eka::AttnUnit u;
  u.qh = qrow; u.q_stride = D;
  u.kh = qrow + G * D; u.vh = qrow + (G + 1) * D;
  u.rope = 1;
  u.qn = rope_lds;
  u.kn = rope_lds + D;
  u.cr = rope_lds + 2 * D;
  u.sr = rope_lds + 3 * D;
  u.eps = a.eps; u.sm_scale = a.sm_scale;
  u.kc = reinterpret_cast<bf16_t*>(lw[LW_KC]) + h * a.csh;
  u.vc = reinterpret_cast<bf16_t*>(lw[LW_VC]) + h * a.csh;
  u.css = a.css;
  u.cap = a.s_cap;
  int64_t lo = a.start_t[0];
  u.lo = lo < 0 ? 0 : lo;
  u.hi = hi;
  u.writer = c == 0;
  u.d0 = c * eka::FDC;
  u.out = nullptr;
  u.out_stride = D;
  u.ll_out = att + (int64_t)h * G * (D / 4);
#ifdef EK_STEP_TRACE
  u.trace_lds = ts_lds;
#endif
  // the cached keys/values are already loading when the unit waits for its heads
  auto wait_heads = [&]() -> bool {
    for (int i = threadIdx.x; i < 4 * D; i += SNT) {
      const int t = i / D, d = i - t * D;
      rope_lds[i] = (t == 0 ? qn : t == 1 ? kn : t == 2 ? cr : sr)[d];
    }
    const bool ok = dw_read<1, true>(qkv, src, (G + 2) * (D / 8), reinterpret_cast<uint32_t*>(qrow), LinLds{}, a.err,
                               a.spin);
    return wg_all(ok, s_fail);
  };
  return eka::attn_unit<D, G, ATU, APT>(u, smem + eka::align16((size_t)(G + 6) * D * 2), wait_heads);
}

// ---------------------------------------------------------------------------
// long contexts: the attention phase on every workgroup
// ---------------------------------------------------------------------------
// Beyond the score row one attention workgroup holds in LDS, every workgroup
// takes part in attention: unit (kv head h, split s) = workgroup h + nkv * s
// attends the keys [k0, k1) = [lo + s c, lo + (s + 1) c) of its row's range
// [lo, hi), c = ceil((hi - lo) / S):
//   scores   QK-norm + RoPE of the G query heads (and of the new key, which
//            stands in for the cache row at the new slot), S^T = K_tile . Q^T
//            per 16-key tile on the matrix cores, scaled, into an LDS row per
//            head; the split's max m_s, e = exp(s - m_s) (fp32) in place and
//            l_s = sum e per head
//   PV       the split's unnormalised partial output sum e v over its keys,
//            every head dim, in fp32 -- the reference's split decode kernel
//            (engine/ek_kernels.py:535-616, the hot path of ek_model.py:401),
//            whose p stays fp32; only its torch fallback rounds p to bf16
//            after the global normalisation, which would cost a round of
//            statistics between the splits before any PV work
//   publish  (m_s, l_s) per head and the partial output travel as tagged
//            words (tag: the layer + 1, since every layer of the launch
//            reuses the region: a layer's words are overwritten only by a
//            workgroup past that layer's o projection wait, which needs every
//            unit's combine, hence every read of them, done)
//   combine  unit s owns head dims [s D/S, (s+1) D/S) of the G query heads
//            (S <= D / 4: whole dense words): the log-sum-exp merge of the S
//            splits (ek_kernels.py:989-1019), M = max m_j, out = sum
//            exp(m_j - M) o_j / sum exp(m_j - M) l_j in split order, stored
//            as the bf16 attention words the o projection awaits.
// The split holding the new slot stores the new key and value rows last.
// long contexts: 16-key score tiles per wave and value rows per thread in
// flight. Shallow rings: the first tiles load ahead of the heads' wait, whose
// polls return behind them, and a split of a batch row is often short (1 and
// 4 measured 3.6 % faster than 2 and 8 on the 8-row batch step, and the same
// or faster at one row: 4 K / 16 K contexts)
#ifndef EK_STEP_LUT
#define EK_STEP_LUT 1
#endif
#ifndef EK_STEP_LVR
#define EK_STEP_LVR 4
#endif
constexpr int LUT = EK_STEP_LUT;
constexpr int LVR = EK_STEP_LVR;

template <int D, int G>
struct LongLds {
  static constexpr size_t HEADS = eka::align16((size_t)(G + 2) * D * 2);   // raw q heads, new k, new v (bf16)
  static constexpr size_t ROPE = eka::align16((size_t)4 * D * 2);          // q gain, k gain, cos, sin
  static constexpr size_t QS = eka::align16((size_t)G * D * 4);            // normed, rotated q (fp32)
  static constexpr size_t KNF = eka::align16((size_t)D * 4);               // the new key (fp32)
  static constexpr size_t KNB = eka::align16((size_t)D * 2);               // the new key (bf16)
  static constexpr size_t ST = eka::align16((size_t)SNW * 8 * 4);          // per-wave max / sum
  static constexpr size_t RED = eka::align16((size_t)SNW * G * D * 4);     // per-wave partial outputs
  static constexpr size_t CMB = eka::align16((size_t)G * D * 4);           // the combined outputs
  static __host__ __device__ constexpr int64_t stride(int64_t chunk) { return chunk | 1; }
  static __host__ __device__ constexpr size_t bytes(int64_t chunk) {
    return HEADS + ROPE + QS + KNF + KNB + 2 * ST + RED + CMB + eka::align16((size_t)G * stride(chunk) * 4);
  }
};

// Where a split unit's q heads come from and its output goes. The step's
// (StepIO): the qkv hand-over words of batch row b (q heads raw, QK-normed
// and rotated by the unit, which also writes the new key and value) and the
// dense attention words. An IO type provides rope() (false: the q heads are
// already rotated, no new row), cs_row(a, b) (the cos/sin row),
// read_heads(a, h, heads, s_fail) (the G q heads, then with rope the new key
// and value, as bf16 rows into LDS; false when a wait gave up),
// put4(h, g, d, v) (the combined output of head h G + g, dims d .. d + 3),
// tag(t) (the exchange words' tag after read_heads: t, or one the IO read
// before), start(a, b) (row b's first key), kLateTiles (key tiles per wave
// that load once the heads are in, beyond the LUT loaded before them) and
// kTrim: whether the key and value rings stop refilling at the wave's last
// rows. A refill past them loads row `last`, a load that the code after the
// ring, which takes its registers, then waits for (a memory round trip);
// skipping them costs the rings' last rounds a condition. The one-launch
// attention kernel gains (config 3 at 4 K keys: 12.2 -> 10.7 us with the
// entry loads), the step kernels lose (8 rows at config 5: 2 % slower).

struct StepIO {
  const llw_t* qkv;
  llw_t* att;
  static constexpr bool kTrim = false;
  static constexpr int kLateTiles = 0;
  __device__ uint32_t tag(uint32_t t) const { return t; }
  __device__ int64_t start(const StepArgs& a, int b) const { return a.start_t[b]; }
  __device__ bool rope() const { return true; }
  __device__ int64_t cs_row(const StepArgs& a, int b) const { return a.positions[b]; }
  template <int D, int G>
  __device__ bool read_heads(const StepArgs& a, int h, bf16_t* heads, int* s_fail) const {
    const bool ok = dw_read<1>(qkv, HeadUnits<D, G>{h, a.nq, a.nkv}, (G + 2) * (D / 8),
                               reinterpret_cast<uint32_t*>(heads), LinLds{}, a.err, a.spin);
    return wg_all(ok, s_fail);
  }
  template <int D, int G>
  __device__ void put4(int h, int g, int d, const float* v) const {
    dw_put(att + ((int64_t)(h * G + g) * D + d) / 4, pack2(v[0], v[1]), pack2(v[2], v[3]));
  }
};

// The batch kernel's: at 8 rows a second key tile per wave, loaded once the
// heads are in, so that its round trip overlaps QK-norm/RoPE and the first
// tile's products (config 5: 2.388 -> 2.361 ms per step, 6 rows 2.349 ->
// 2.313). Where splits hold about one tile per wave it costs: 2 and 4 rows
// ran 1.1 % slower with it, the batch-1 split step at 4 K keys 2.5 %.
template <int MB>
struct BStepIO : StepIO {
  static constexpr int kLateTiles = MB == 8 ? 1 : 0;
};

template <int D, int G, typename IO>
// Unit (kv head h, split s of S) of batch row b; io holds row b's inputs and
// output, lx its nkv S units' exchange words; ltag tags these words. The
// row's keys per split must be at most a.lchunk.
__device__ __forceinline__ bool long_attention(const StepArgs& a, const int64_t* lw, const IO& io,
                                               llw_t* lx, int b, int h, int s, int S, int64_t hi, uint32_t ltag,
                                               unsigned char* lds, int* s_fail
#ifdef EK_STEP_TRACE
                                               , int64_t* ts_lds
#endif
                                               ) {
  using L = LongLds<D, G>;
  constexpr int KS = D / 32;       // 32-dim k-steps of a score tile
  // 16-key score tiles per wave in flight: LUT from the start, IO::kLateTiles
  // more once the heads are in (loads issued ahead of a hand-over's polls
  // delay them)
  constexpr int UT = LUT + IO::kLateTiles;
  constexpr int DCH = D / 8;       // 16-byte chunks per key row
  constexpr int NKG = SNT / DCH;   // key groups of the PV product
  constexpr int VR = LVR;          // value rows per thread in flight
  const int tid = opaque_tid(), lane = tid & 63, wave = wave_id();
  const int r16 = lane & 15, q4 = lane >> 4;
  if (s >= S) return true;
  const int dpu = D / S;   // dims this unit combines

  bf16_t* heads = reinterpret_cast<bf16_t*>(lds);
  bf16_t* rope = reinterpret_cast<bf16_t*>(lds + L::HEADS);
  bf16_t (*qs)[D] = reinterpret_cast<bf16_t (*)[D]>(lds + L::HEADS + L::ROPE);   // normed, rotated q (bf16)
  float* knf = reinterpret_cast<float*>(lds + L::HEADS + L::ROPE + L::QS);
  bf16_t* knew_bf = reinterpret_cast<bf16_t*>(lds + L::HEADS + L::ROPE + L::QS + L::KNF);
  unsigned char* p0 = lds + L::HEADS + L::ROPE + L::QS + L::KNF + L::KNB;
  float (*stm)[8] = reinterpret_cast<float (*)[8]>(p0);
  float (*stl)[8] = reinterpret_cast<float (*)[8]>(p0 + L::ST);
  float* red = reinterpret_cast<float*>(p0 + 2 * L::ST);                  // [SNW][G][D]
  float* cmb = reinterpret_cast<float*>(p0 + 2 * L::ST + L::RED);         // [G dpu]
  float* sc = reinterpret_cast<float*>(p0 + 2 * L::ST + L::RED + L::CMB);   // [G][stride]
  const int64_t cstride = L::stride(a.lchunk);

  int64_t lo = io.start(a, b);
  lo = lo < 0 ? 0 : lo;
  const int64_t nrel = hi > lo ? hi - lo : 0;
  const int64_t chunk = (nrel + S - 1) / S;   // <= a.lchunk (the caller's split count ensures it)
  const int64_t k0 = lo + (int64_t)s * chunk;
  int64_t k1 = k0 + chunk;
  k1 = k1 < hi ? k1 : hi;
  const int64_t nk = k1 > k0 ? k1 - k0 : 0;
  const int64_t slot = hi - 1;
  const bool own = io.rope() && nk > 0 && slot >= k0 && slot < k1;
  // loads past the split's keys (the last tiles' tails, an empty split) read
  // row `last` instead: k0 itself may lie past the cache's last row. Their
  // products are never used, nor is the cache row at the new slot (the new
  // key and value stand in for it), so no load is masked: a select on a
  // loaded value would wait for the load where it stands.
  const int64_t last = slot > 0 ? slot : 0;
  const bf16_t* kc = reinterpret_cast<const bf16_t*>(lw[LW_KC]) + b * a.csb + h * a.csh;
  const bf16_t* vc = reinterpret_cast<const bf16_t*>(lw[LW_VC]) + b * a.csb + h * a.csh;

  // key tiles, a ring of UT per wave: slot u holds tile wave + (u + UT j) SNW
  // of the split; lane holds key r16 of a tile, dims 32 i + 8 q4 .. +7
  // (32-bit key indices: the plan bounds a split's keys by 65536)
  const int nk32 = (int)nk;
  const int ntile = (nk32 + 15) >> 4;
  uint4 kt[UT][KS];
  const bf16_t* kbase = kc + k0 * a.css + 8 * q4;
  const bf16_t* klast = kc + last * a.css + 8 * q4;
  const int kcs = (int)a.css;
  auto load_tile = [&](int u, int t) {
    const int rel = (t << 4) + r16;
    const bf16_t* src = rel < nk32 ? kbase + rel * kcs : klast;
#pragma unroll
    for (int i = 0; i < KS; ++i) kt[u][i] = ld16_nt(src + 32 * i);
  };
  // the first tiles load before the heads are awaited (they do not depend on them)
#pragma unroll
  for (int u = 0; u < LUT; ++u) load_tile(u, wave + u * SNW);

  // the unit's q heads, new key and new value, and the gains / cos / sin rows
  {
    if (io.rope()) {
      const bf16_t* qn = reinterpret_cast<const bf16_t*>(lw[LW_QN]);
      const bf16_t* kn = reinterpret_cast<const bf16_t*>(lw[LW_KN]);
      int64_t crow = io.cs_row(a, b);
      crow = crow < 0 ? 0 : (crow >= a.rope_len ? a.rope_len - 1 : crow);
      const bf16_t* cr = a.cos + crow * a.ld_cs;
      const bf16_t* sr = a.sin + crow * a.ld_cs;
      for (int i = tid; i < 4 * D; i += SNT) {
        const int t = i / D, d = i - t * D;
        rope[i] = (t == 0 ? qn : t == 1 ? kn : t == 2 ? cr : sr)[d];
      }
    }
    if (!io.template read_heads<D, G>(a, h, heads, s_fail)) return false;
  }
  ltag = io.tag(ltag);
#pragma unroll
  for (int u = LUT; u < UT; ++u) load_tile(u, wave + u * SNW);
  EK_TS(28);
  if (io.rope()) {
    // QK-norm + RoPE: head u < G the query heads, u = G the new key (wave u % 8)
    for (int u = wave; u <= G; u += SNW) {
      if (u < G) eka::head_norm_rope<D, false>(heads + u * D, rope, rope + 2 * D, rope + 3 * D, a.eps, nullptr, qs[u]);
      else eka::head_norm_rope<D>(heads + G * D, rope + D, rope + 2 * D, rope + 3 * D, a.eps, knf, knew_bf);
    }
  } else {
    for (int i = tid; i < G * D; i += SNT) qs[i / D][i % D] = heads[i];
  }
  __syncthreads();

  // ---- scores. B operand = Q^T: q[g = r16][32 i + 8 q4 .. +7], zero for g >= G
  uint4 qb[KS];
  {
    const uint32_t qmask = r16 < G ? 0xffffffffu : 0u;
    const int g = r16 < G ? r16 : 0;
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(&qs[g][32 * i + 8 * q4]);
      qb[i] = make_uint4(v.x & qmask, v.y & qmask, v.z & qmask, v.w & qmask);
    }
  }
  // The wave's tiles run in rounds of UT with no early exit (an exit inside
  // the unrolled ring would roll it into a loop over one register set, one
  // tile in flight): tiles past the split's end compute on re-read rows and
  // their scores are dropped.
  float mrun = -INFINITY;
  const int ntw = wave < ntile ? (int)((ntile - 1 - wave) / SNW) + 1 : 0;   // this wave's tiles
  const int srel = own ? (int)(slot - k0) : -1;                              // the new slot's key
  auto score_tile = [&](int u, int k, bool refill) {
    const int t = wave + (k + u) * SNW;
    const int tb = t << 4;
    if (tb + r16 == srel) {   // the new key, from LDS
#pragma unroll
      for (int i = 0; i < KS; ++i) kt[u][i] = *reinterpret_cast<const uint4*>(&knew_bf[32 * i + 8 * q4]);
    }
    eka::f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KS; ++i) c = eka::mfma16x16x32(kt[u][i], qb[i], c);
    if (refill) load_tile(u, t + SNW * UT);   // refill the slot
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rel = tb + 4 * q4 + e;
      const float sv = c[e] * a.sm_scale;
      const bool ok = r16 < G && rel < nk32;
      if (ok) sc[r16 * cstride + rel] = sv;
      mrun = ok ? fmaxf(mrun, sv) : mrun;
    }
  };
  if constexpr (IO::kTrim) {
    // rounds whose refills all lie within the wave's tiles, then the last
    // one or two, which refill only tiles the wave has
    int k = 0;
    for (; k + 2 * UT <= ntw; k += UT) {
#pragma unroll
      for (int u = 0; u < UT; ++u) score_tile(u, k, true);
    }
    for (; k < ntw; k += UT) {
#pragma unroll
      for (int u = 0; u < UT; ++u) score_tile(u, k, k + u + UT < ntw);
    }
  } else {
    for (int k = 0; k < ntw; k += UT) {
#pragma unroll
      for (int u = 0; u < UT; ++u) {
        const int t = wave + (k + u) * SNW;
        const int tb = t << 4;
        if (tb + r16 == srel) {   // the new key, from LDS
#pragma unroll
          for (int i = 0; i < KS; ++i) kt[u][i] = *reinterpret_cast<const uint4*>(&knew_bf[32 * i + 8 * q4]);
        }
        eka::f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < KS; ++i) c = eka::mfma16x16x32(kt[u][i], qb[i], c);
        load_tile(u, t + SNW * UT);   // refill the slot
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int rel = tb + 4 * q4 + e;
          const float sv = c[e] * a.sm_scale;
          const bool ok = r16 < G && rel < nk32;
          if (ok) sc[r16 * cstride + rel] = sv;
          mrun = ok ? fmaxf(mrun, sv) : mrun;
        }
      }
    }
  }
  // the first value rows of the PV product load while the statistics travel:
  // thread -> head dims 8 dc .. +7 of keys kg, kg + NKG, ... (16-byte loads,
  // lane-contiguous across a key row), a ring of VR rows per thread
  const int dc = tid % DCH, kg = tid / DCH;
  const int nper = nk32 > kg ? (nk32 - kg + NKG - 1) / NKG : 0;
  // the wave's most and fewest rows (its first and last lanes' key groups)
  const int kgf = (tid & ~(EK_WAVE - 1)) / DCH, kgl = (tid | (EK_WAVE - 1)) / DCH;
  const int nperw = nk32 > kgf ? (nk32 - kgf + NKG - 1) / NKG : 0;
  const int npermin = nk32 > kgl ? (nk32 - kgl + NKG - 1) / NKG : 0;
  const bf16_t* vbase = vc + (k0 + kg) * a.css + 8 * dc;
  const bf16_t* vlast = vc + last * a.css + 8 * dc;
  const int vstep = NKG * (int)a.css;
  auto vaddr = [&](int j) { return j < nper ? vbase + j * vstep : vlast; };
  // the key row j of this thread that is the new slot (-1: none)
  int jslot = -1;
  if (own) {
    const int r = srel - kg;
    jslot = (r >= 0 && r % NKG == 0) ? r / NKG : -1;
  }
  uint4 vr[VR];
#pragma unroll
  for (int u = 0; u < VR; ++u) vr[u] = ld16_nt(vaddr(u));

  mrun = fmaxf(mrun, __shfl_xor(mrun, 16, EK_WAVE));
  mrun = fmaxf(mrun, __shfl_xor(mrun, 32, EK_WAVE));
  if (q4 == 0 && r16 < G) stm[wave][r16] = mrun;
  __syncthreads();
  EK_TS(31);

  // ---- the split's statistics per head (thread -> head tid % G): its max
  // m_s, e = exp(s - m_s) in place (fp32, unnormalised) and l_s = sum e;
  // they travel with the split's partial output, so PV starts at once
  llw_t* st_ll = lx;                                          // [nkv][S][2G]
  llw_t* pt_ll = lx + (int64_t)a.nkv * S * 2 * G;             // [nkv][S][G][D]
  {
    const int g = tid % G;
    float ms = stm[0][g];
#pragma unroll
    for (int w = 1; w < SNW; ++w) ms = fmaxf(ms, stm[w][g]);
    float ls = 0.f;
    for (int n = tid / G; n < nk32; n += SNT / G) {
      const float ev = expf(sc[g * cstride + n] - ms);
      sc[g * cstride + n] = ev;
      ls += ev;
    }
#pragma unroll
    for (int o = G; o < EK_WAVE; o <<= 1) ls += __shfl_xor(ls, o, EK_WAVE);
    if (lane < G) stl[wave][lane] = ls;
    __syncthreads();
    if (tid < G) {
      float lt = 0.f;
#pragma unroll
      for (int w = 0; w < SNW; ++w) lt += stl[w][tid];
      llw_t* my = st_ll + ((int64_t)h * S + s) * 2 * G;
      ll_put(my + 2 * tid, __float_as_uint(ms), ltag);
      ll_put(my + 2 * tid + 1, __float_as_uint(lt), ltag);
    }
  }
  EK_TS(29);
  EK_TS(32);

  // ---- PV: the split's partial output sum p v over its keys, every head dim, fp32
  {
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    const uint4 vnew = *reinterpret_cast<const uint4*>(heads + (G + 1) * D + 8 * dc);
    auto use = [&](const uint4& vv, int j) {
      const int n = kg + NKG * j;
      const uint4 v = j == jslot ? vnew : vv;
      float vf[8];
      unpack8(v, vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pg = sc[g * cstride + n];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(pg, vf[e], acc[g][e]);
      }
    };
    // the ring: each slot is consumed, then refilled (refilling first would
    // copy every slot at the loop's head, which waits for all of them); the
    // scheduling barrier keeps each refill where it stands (the scheduler
    // otherwise sinks all of them to the loop's end, and every round then
    // waits for the whole ring)
    if constexpr (IO::kTrim) {
      // rounds whose rows and refills exist for every lane run unconditioned;
      // the last one or two use each lane's own rows and refill only rows
      // the wave has
      int j0 = 0;
      for (; j0 + 2 * VR <= npermin; j0 += VR) {
#pragma unroll
        for (int u = 0; u < VR; ++u) {
          use(vr[u], j0 + u);
          vr[u] = ld16_nt(vaddr(j0 + u + VR));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      for (; j0 < nperw; j0 += VR) {
        const bool whole = j0 + VR <= npermin;
#pragma unroll
        for (int u = 0; u < VR; ++u) {
          if (whole || j0 + u < nper) use(vr[u], j0 + u);
          if (j0 + u + VR < nperw) vr[u] = ld16_nt(vaddr(j0 + u + VR));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else {
      int j0 = 0;
      for (; j0 + VR <= nper; j0 += VR) {
#pragma unroll
        for (int u = 0; u < VR; ++u) {
          use(vr[u], j0 + u);
          vr[u] = ld16_nt(vaddr(j0 + u + VR));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int u = 0; u < VR; ++u)
        if (j0 + u < nper) use(vr[u], j0 + u);
    }
    EK_TS(33);
    // key groups with the same dims: lanes dc, dc + DCH, ... of the wave, then
    // the waves. Lanes under 16 apart add by shuffles, 16 and 32 apart by row
    // swaps (v_permlane16_swap, v_permlane32_swap), which also transpose: the
    // N = 8 G sums end in N / 4 registers, row r of register i holding sum
    // i + (r & 1) N / 2 + (r >> 1) N / 4 (the same additions in the same
    // order as a butterfly over 16 then 32 lanes)
    constexpr int N = 8 * G;
    float* av = &acc[0][0];
#pragma unroll
    for (int o = DCH; o < 16; o <<= 1)
#pragma unroll
      for (int i = 0; i < N; ++i) av[i] += __shfl_xor(av[i], o, EK_WAVE);
    float t16[N / 2], t32[N / 4];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(av[i]), __float_as_uint(av[i + N / 2]), false, false);
      t16[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(t16[i]), __float_as_uint(t16[i + N / 4]), false, false);
      t32[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    if ((lane & 15) < DCH) {
      const int r = lane >> 4;
      const int off = (r & 1) * (N / 2) + (r >> 1) * (N / 4);
#pragma unroll
      for (int i = 0; i < N / 4; ++i) red[(wave * G + (i + off) / 8) * D + 8 * dc + ((i + off) & 7)] = t32[i];
    }
  }
  EK_TS(34);
  __syncthreads();
  EK_TS(35);
  // the split's partial output -> tagged words
  for (int i = tid; i < G * D; i += SNT) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < SNW; ++w) t += red[w * G * D + i];
    ll_put(pt_ll + ((int64_t)h * S + s) * G * D + i, __float_as_uint(t), ltag);
  }
  EK_TS(30);
  // ---- combine this unit's dims [s dpu, (s+1) dpu) of every query head,
  // the log-sum-exp merge of the splits (engine/ek_kernels.py:989-1019):
  // thread t -> output o = t / S (head g = o / dpu, dim o % dpu), split j =
  // t % S polls that split's partial word and its (m_j, l_j) of head g; the
  // S lanes of an output (S <= 64, a power of two, so they sit in one wave)
  // form M = max m_j, then sum exp(m_j - M) o_j and exp(m_j - M) l_j by
  // butterflies in a fixed order (a split without keys has m_j = -inf)
  {
    bool ok = true;
    for (int t = tid; t < G * D; t += SNT) {   // G * dpu * S = G * D
      const int o = t / S, j = t - o * S;
      const int g = o / dpu, dd = o - g * dpu;
      const llw_t* sj = st_ll + ((int64_t)h * S + j) * 2 * G + 2 * g;
      uint32_t w = 0u, mw = 0u, lw32 = 0u;
      ok = ok && ll_wait1(sj, ltag, mw, a.err, a.spin) && ll_wait1(sj + 1, ltag, lw32, a.err, a.spin) &&
           ll_wait1(pt_ll + (((int64_t)h * S + j) * G + g) * D + s * dpu + dd, ltag, w, a.err, a.spin);
      const float mj = __uint_as_float(mw);
      float M = mj;
      for (int m = 1; m < S; m <<= 1) M = fmaxf(M, __shfl_xor(M, m, EK_WAVE));
      const float sj_w = mj == -INFINITY ? 0.f : expf(mj - M);
      float num = sj_w * __uint_as_float(w), den = sj_w * __uint_as_float(lw32);
      for (int m = 1; m < S; m <<= 1) {
        num += __shfl_xor(num, m, EK_WAVE);
        den += __shfl_xor(den, m, EK_WAVE);
      }
      if (j == 0) cmb[o] = num / den;
    }
    if (!wg_all(ok, s_fail)) return false;
    EK_TS(5);
    for (int i = tid; i < G * dpu / 4; i += SNT) {
      const int g = (4 * i) / dpu, dd = 4 * i - g * dpu;
      io.template put4<D, G>(h, g, s * dpu + dd, cmb + 4 * i);
    }
  }
  // the new key and value rows (normed and rotated key, raw value)
  if (own && wave == SNW - 1) {
    bf16_t* kdst = const_cast<bf16_t*>(kc) + slot * a.css;
    bf16_t* vdst = const_cast<bf16_t*>(vc) + slot * a.css;
    for (int d = lane; d < D; d += EK_WAVE) {
      kdst[d] = knew_bf[d];
      vdst[d] = heads[(G + 1) * D + d];
    }
  }
  return true;
}

// ---------------------------------------------------------------------------
// the step
// ---------------------------------------------------------------------------
// Workgroups [0, n_attn) run only attention, one unit (kv head, 32 head dims)
// each, layer after layer: they enter a layer's unit as soon as the previous
// one is done, so its cached keys and values (up to ATU * 8 * 16 keys) load
// into registers while the projections of the layer before run elsewhere,
// and only QK-norm/RoPE, the two MFMA products and the softmax remain once
// the layer's q/k/v arrive. The other workgroups run every projection and
// the lm_head. The two roles share no state, so neither's registers are
// live in the other's code.
// LDS of a projection workgroup: [activation row][wave partials] (the
// residual row is held by unit in registers: add_norm_u)

template <int D, int G>
__device__ __forceinline__ void attention_loop(const StepArgs& a, const int64_t* lwt, uint32_t ep, int64_t hi,
                                               unsigned char* smem, int* s_fail
#ifdef EK_STEP_TRACE
                                               , int64_t* ts_lds
#endif
                                               ) {
  const int qw = a.nq * D, qkvw = (a.nq + 2 * a.nkv) * D;
  const int64_t lwords = arena_layer_words(a.h, a.inter, qkvw, qw);
  llw_t* half = cur_half(a, ep);
  for (int l = 0; l < a.nl; ++l) {
    const int64_t* lw = lwt + l * LW_FIELDS;
    const llw_t* qkv_ll = half + (int64_t)l * lwords;
    llw_t* att_ll = half + (int64_t)l * lwords + qkvw / 4;
    if (!attention_phase<D, G>(a, lw, qkv_ll, att_ll, hi, smem, s_fail, l
#ifdef EK_STEP_TRACE
                                , ts_lds
#endif
                                )) return;
    EK_TS(5);
    __syncthreads();
    EK_TS_FLUSH(l);
  }
}

__device__ __forceinline__ Gp on_gemv_wgs(Gp g, int n_attn) {
  g.wg0 = n_attn;
  g.nwg = (int)gridDim.x - n_attn;
  return g;
}

// The projection workgroups' part of the step: every layer's projections,
// then the final add + norm, lm_head and this workgroup's argmax words.
// False when a hand-over wait gave up (the error word is then set).
template <int D, int G, bool LONG>
__device__ __forceinline__ bool projection_pass(const StepArgs& a, const int64_t* lwt, uint32_t ep, int64_t hi,
                                                unsigned char* smem, float* s_red, int* s_redi, int* s_fail
#ifdef EK_STEP_TRACE
                                                , int64_t* ts_lds
#endif
                                                ) {
  const int tid = threadIdx.x;
  const int h = a.h, inter = a.inter;
  const int qw = a.nq * D, qkvw = (a.nq + 2 * a.nkv) * D;
  const int64_t lwords = arena_layer_words(h, inter, qkvw, qw);
  const int n_attn = LONG ? 0 : a.nkv * (D / eka::FDC);
  constexpr int PFM = LONG ? PF_LONG : PF;

  unsigned char* ph = smem;
  bf16_t* xs = reinterpret_cast<bf16_t*>(ph);
  uint32_t* xs32 = reinterpret_cast<uint32_t*>(ph);
  float* part = reinterpret_cast<float*>(ph + eka::align16((size_t)a.kpad_max * 2));
  const int part_n = a.part_max * SNW;

  RingN<LONG ? NB_LONG : NB> ring;
  ring.nready = 0;
#pragma unroll
  for (int u = 0; u < (LONG ? NB_LONG : NB); ++u) ring.r[u] = make_uint4(0, 0, 0, 0);
  // norm gains, loaded a phase ahead of their use: gw1 = input norm of the
  // coming layer (the final norm after the last), gw2 = post-attention norm
  uint4 gw1 = load_gain_u(reinterpret_cast<const bf16_t*>(lwt[LW_LN1]), h), gw2 = gw1;
  uint4 rres = make_uint4(0u, 0u, 0u, 0u);   // this thread's residual unit (add_norm_u)

  llw_t* half = cur_half(a, ep);
  const llw_t* dn_prev = nullptr;
  for (int l = 0; l < a.nl; ++l) {
    EK_TS(0);
    const int64_t* lw = lwt + l * LW_FIELDS;
    llw_t* qkv_ll = half + (int64_t)l * lwords;
    llw_t* att_ll = qkv_ll + qkvw / 4;
    llw_t* o_ll = att_ll + qw / 4;
    llw_t* act_ll = o_ll + h / 4;
    llw_t* dn_ll = act_ll + inter / 4;
    const Gp gq = on_gemv_wgs(make_gp(reinterpret_cast<const bf16_t*>(lw[LW_QKV]), h, qkvw, 0, 4), n_attn);
    const Gp go = on_gemv_wgs(make_gp(reinterpret_cast<const bf16_t*>(lw[LW_O]), qw, h, 0, 4), n_attn);
    const Gp gg = on_gemv_wgs(make_gp(reinterpret_cast<const bf16_t*>(lw[LW_GU]), h, inter, 1, 4), n_attn);
    const Gp gd = on_gemv_wgs(make_gp(reinterpret_cast<const bf16_t*>(lw[LW_DOWN]), inter, h, 0, 4), n_attn);

    // ---- r = (layer 0) embed[token] | r + down(l-1); norm; qkv
    zero_part(part, part_n);
    if (l == 0) {
      int64_t t = a.tokens[0];
      t = t < 0 ? 0 : (t >= a.vocab ? a.vocab - 1 : t);
      if (tid < h / 8) rres = ld16g(a.embed + t * a.lde + 8 * tid);
      add_norm_u(rres, nullptr, gw1, h, kpad_of(h), a.eps, xs, s_red, true, s_fail);
    } else {
      EK_TS(22);
      u32x4_t v[1];
      const bool ok = wait_res(dn_prev, h, v, a);
      if (!add_norm_u(rres, v, gw1, h, kpad_of(h), a.eps, xs, s_red, ok, s_fail)) return false;
    }
    EK_TS(26);
    __syncthreads();
    EK_TS(1);
    gemv_phase(gq, ring, xs, part);
    __syncthreads();
    EK_TS(2);
    epilogue_ll(gq, part, qkv_ll);
    EK_TS(3);
    __syncthreads();

    if constexpr (LONG) {
      // ---- attention on every workgroup (its LDS overlays the activation
      //      row and the partials), then the o projection from the ring
      llw_t* lx_ll = half + (int64_t)a.nl * lwords + 2 * (int64_t)gridDim.x;
      if (!long_attention<D, G>(a, lw, StepIO{qkv_ll, att_ll}, lx_ll, 0, (int)blockIdx.x % a.nkv,
                                (int)blockIdx.x / a.nkv, a.lsplit, hi, (uint32_t)l + 1u, ph, s_fail
#ifdef EK_STEP_TRACE
                                , ts_lds
#endif
                                ))
        return false;
      EK_TS(4);
      prefetch_phase<PFM>(go, ring);
      gw2 = load_gain_u(reinterpret_cast<const bf16_t*>(lw[LW_LN2]), h);
      __syncthreads();
      zero_part(part, part_n);
      {
        const bool ok = dw_read<HW, true>(att_ll, LinUnits{}, qw / 8, xs32, LinLds{}, a.err, a.spin);
        if (!wg_all(ok, s_fail)) return false;
      }
      zero_pad(xs, qw, kpad_of(qw));
      EK_TS(6);
      __syncthreads();
      gemv_phase(go, ring, xs, part);
      __syncthreads();
      EK_TS(7);
      epilogue_ll(go, part, o_ll);
      prefetch_phase<PFM>(gg, ring);
      EK_TS(8);
    } else {
      (void)hi;
      // ---- while attention runs: this workgroup's o_proj rows into registers
      //      (all of them at the Qwen3-4B shape) and its first gate/up rows into L2
      uint4 ob[OB];
      hold_phase(go, ob);
      prefetch_phase<PFM>(gg, ring);
      uint32_t sink = 0;
      l2_touch(gg, sink);
      gw2 = load_gain_u(reinterpret_cast<const bf16_t*>(lw[LW_LN2]), h);
      EK_TS(4);
      // ---- o projection
      int hu0, hnr;
      if (held_by_column(go, hu0, hnr) && qw == SNT * 8) {
        // held by column, wave w's chunk of the attention row is its lanes'
        // 16-byte units (thread t: unit t), the output of kv head w's
        // attention units: each wave waits for its own chunk into registers
        // and runs its products at once; the workgroup meets (and votes)
        // only before the epilogue
        u32x4_t v[1];
        const bool ok = wait_res(att_ll, qw, v, a);
        if (sink == 0x9e3779b9u) s_redi[0] = 0;   // keeps the L2 loads; their data is not used
        EK_TS(6);
        held_col_products(ob, make_uint4(v[0].x ^ DW_FLIP32, v[0].y ^ DW_FLIP32, v[0].z ^ DW_FLIP32,
                                          v[0].w ^ DW_FLIP32), part, hnr);
        EK_TS(30);
        if (!wg_all(ok, s_fail)) return false;
      } else {
        zero_part(part, part_n);
        {
          const bool ok = dw_read<HW, true>(att_ll, LinUnits{}, qw / 8, xs32, LinLds{}, a.err, a.spin);
          if (sink == 0x9e3779b9u) s_redi[0] = 0;   // keeps the L2 loads; their data is not used
          if (!wg_all(ok, s_fail)) return false;
        }
        zero_pad(xs, qw, kpad_of(qw));
        EK_TS(6);
        __syncthreads();
        EK_TS(29);
        gemv_held_phase(go, ob, xs, part);
        EK_TS(30);
        __syncthreads();
      }
      EK_TS(7);
      epilogue_ll(go, part, o_ll);
      EK_TS(8);
    }

    // ---- r = r + o; norm; gate/up; SwiGLU
    __syncthreads();
    zero_part(part, part_n);
    {
      EK_TS(15);
      u32x4_t v[1];
      const bool ok = wait_res(o_ll, h, v, a);
      EK_TS(17);
      if (!add_norm_u(rres, v, gw2, h, kpad_of(h), a.eps, xs, s_red, ok, s_fail)) return false;
    }
    EK_TS(24);
    // the next input norm's gain loads with the gate/up stream
    gw1 = load_gain_u(l + 1 < a.nl ? reinterpret_cast<const bf16_t*>(lwt[(l + 1) * LW_FIELDS + LW_LN1]) : a.fnorm,
                      h);
    EK_TS(25);
    __syncthreads();
    EK_TS(9);
    gemv_phase(gg, ring, xs, part);
    __syncthreads();
    EK_TS(10);
    epilogue_swiglu_ll(gg, part, act_ll);
    EK_TS(11);
    prefetch_phase<PFM>(gd, ring);
    EK_TS(27);

    // ---- down projection
    __syncthreads();
    zero_part(part, part_n);
    {
      EK_TS(19);
#ifdef EK_STEP_TRACE
      int64_t rounds = 0;
      const bool ok = dw_read<AW, true>(act_ll, LinUnits{}, inter / 8, xs32, LinLds{}, a.err, a.spin, &rounds);
      EK_TS(20);
      if (threadIdx.x == 0) ts_lds[21] = rounds;
#else
      const bool ok = dw_read<AW, true>(act_ll, LinUnits{}, inter / 8, xs32, LinLds{}, a.err, a.spin);
#endif
      if (!wg_all(ok, s_fail)) return false;
    }
    zero_pad(xs, inter, kpad_of(inter));
    __syncthreads();
    EK_TS(12);
    gemv_phase(gd, ring, xs, part);
    __syncthreads();
    EK_TS(13);
    epilogue_ll(gd, part, dn_ll);
    EK_TS(14);
    if (l + 1 < a.nl)
      prefetch_phase<PFM>(on_gemv_wgs(make_gp(reinterpret_cast<const bf16_t*>(lwt[(l + 1) * LW_FIELDS + LW_QKV]),
                                         h, qkvw, 0, 4), n_attn), ring);
    else
      prefetch_phase<PFM>(on_gemv_wgs(make_gp(a.lm_head, h, a.vocab, 0, 1), n_attn), ring);
    dn_prev = dn_ll;
    __syncthreads();
    EK_TS_FLUSH(l);
  }

  // ---- final add + norm, lm_head, per-workgroup argmax
  EK_TS(0);
  llw_t* am_ll = half + (int64_t)a.nl * lwords;
  zero_part(part, part_n);
  {
    u32x4_t v[1];
    const bool ok = wait_res(dn_prev, h, v, a);
    if (!add_norm_u(rres, v, gw1, h, kpad_of(h), a.eps, xs, s_red, ok, s_fail)) return false;
  }
  __syncthreads();
  EK_TS(1);
  const Gp gl = on_gemv_wgs(make_gp(a.lm_head, h, a.vocab, 0, 1), n_attn);
  gemv_phase(gl, ring, xs, part);
  __syncthreads();
  EK_TS(2);
  epilogue_argmax_ll(gl, part, s_red, s_redi, am_ll, a.logits);
  EK_TS(3);
  EK_TS_FLUSH_SYNC(a.nl);
  return true;
}

// Workgroup n_attn's end of the step: the token = first-index argmax over
// the projection workgroups' words, then the step's bookkeeping
// (engine.py:289-292; the slot/len advance of ek_model.py:375-388). A step
// that gave up (ok false, or a wait here runs out) still advances the step
// counter and writes the sentinel -1 as its token (out_buf, out_tok), and
// leaves tokens, positions, slot and length as they were, so the host reads
// the failure at this step's own row and every later row stays aligned.
template <int D>
__device__ __forceinline__ void finish_step(const StepArgs& a, uint32_t ep, bool ok, int64_t len_old, int n_attn,
                                            unsigned char* smem, float* s_red, int* s_redi, int* s_fail) {
  const int tid = threadIdx.x;
  const int h = a.h;
  const int qw = a.nq * D, qkvw = (a.nq + 2 * a.nkv) * D;
  const int n_gemv = (int)gridDim.x - n_attn;
  const llw_t* am_ll = cur_half(a, ep) + (int64_t)a.nl * arena_layer_words(h, a.inter, qkvw, qw);
  uint32_t* amw = reinterpret_cast<uint32_t*>(smem + eka::align16((size_t)a.kpad_max * 2));
  __syncthreads();
  if (ok) ok = wg_all(ll_read(LinSrc{am_ll + 2 * n_attn}, 2 * n_gemv, AM_TAG, amw, a.err, a.spin), s_fail);
  float ov = 0.f;
  int oi = 0x7fffffff;
  if (ok) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int w = tid; w < n_gemv; w += SNT) {
      const float v = __uint_as_float(amw[2 * w]);
      const int i = (int)amw[2 * w + 1];
      if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    wg_argmax(bv, bi, s_red, s_redi, ov, oi);
  }
  if (tid == 0) {
    const int64_t step = *a.step_idx;
    const int64_t tok = !ok ? -1 : (oi == 0x7fffffff ? 0 : oi);
    if (a.out_tok) a.out_tok[0] = tok;
    if (step >= 0 && step < a.max_steps) a.out_buf[step] = (int32_t)tok;
    if (ok) {
      a.tokens[0] = tok;
      a.positions[0] += 1;
      a.slot_t[0] = len_old;
      *a.len_t = len_old + 1;
    }
    *a.step_idx = step + 1;
  }
}

template <int D, int G, bool LONG>
__global__ __launch_bounds__(SNT) void step_kernel(StepArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float s_red[SNW];
  __shared__ int s_redi[SNW];
  __shared__ unsigned s_ep;
  __shared__ int s_abort;
  __shared__ int s_fail;
  __shared__ int64_t s_lw[MAX_LAYERS * LW_FIELDS];   // the layer table, read from LDS in every phase

  const int tid = threadIdx.x;
  for (int i = tid; i < a.nl * LW_FIELDS; i += SNT) s_lw[i] = a.lw[i];
  if (tid == 0) {
    s_fail = 0;
    const unsigned e = __hip_atomic_load(&a.bar->ep[blockIdx.x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    __hip_atomic_store(&a.bar->ep[blockIdx.x], e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_ep = e;
    // the error word is sticky: once a launch gave up, later launches only
    // advance the step counter (with the sentinel) until the host clears it
    s_abort = __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#ifdef EK_STEP_TRACE
  __shared__ int64_t s_ts[48];
  int64_t* ts_lds = s_ts;
#endif
  __syncthreads();
  const uint32_t ep = __builtin_amdgcn_readfirstlane(s_ep);   // wave-uniform: the halves' addresses stay scalar
  const bool aborted = s_abort != 0;
  clear_next_half(a, ep);   // also in a launch that gives up: the next one needs it
  const int64_t len_old = *a.len_t;
  int64_t hi = len_old + 1;
  hi = hi < 0 ? 0 : (hi > a.s_cap ? a.s_cap : hi);
  // attention-only workgroups [0, n_attn) (none for long contexts)
  const int n_attn = LONG ? 0 : a.nkv * (D / eka::FDC);
  if ((int)blockIdx.x < n_attn) {
    if (aborted) return;
    attention_loop<D, G>(a, s_lw, ep, hi, smem, &s_fail
#ifdef EK_STEP_TRACE
                         , ts_lds
#endif
                         );
    return;
  }
  bool ok = !aborted;
  if (ok)
    ok = projection_pass<D, G, LONG>(a, s_lw, ep, hi, smem, s_red, s_redi, &s_fail
#ifdef EK_STEP_TRACE
                               , ts_lds
#endif
                               );
  if ((int)blockIdx.x != n_attn) return;
  finish_step<D>(a, ep, ok, len_old, n_attn, smem, s_red, s_redi, &s_fail);
#ifdef EK_STEP_TRACE
  EK_TS(4);
  EK_TS_FLUSH_SYNC(a.nl);
#endif
}

// LDS bytes of step_kernel<D, G, LONG>: the projection layout, and either
// an attention unit's (the attention-only workgroups') or, for long
// contexts, the split attention's, which overlays the projection layout
// (lchunk: keys per split)
template <int D, int G, bool LONG>
inline size_t step_lds_bytes(int h, int kpad_max, int part_max, int64_t s_cap, int lchunk) {
  (void)h;
  const size_t gemv = eka::align16((size_t)kpad_max * 2) + eka::align16((size_t)part_max * SNW * 4);
  const size_t attn = LONG ? LongLds<D, G>::bytes(lchunk)
                           : eka::align16((size_t)(G + 6) * D * 2) + eka::AttnLds<D, G>::bytes(s_cap);
  return gemv > attn ? gemv : attn;
}

// launch of one head-dim instantiation for any G (ek_step_inst.hip); the
// long-context kernel when a.lsplit > 0
template <int D>
hipError_t launch_step(const StepArgs& a, int g, int nwg, hipStream_t st);
// workgroups of step_kernel<D, g, lng> with `lds` dynamic LDS bytes resident per CU
template <int D>
int step_occupancy(int g, bool lng, size_t lds);

}  // namespace eks
