// Decode attention over the static KV cache, for gfx950: a two-launch
// split-K pair over a (split, kv head, batch row) grid for any length, a
// one-launch split form when the whole grid fits on the device at once
// (attn_onepass_kernel, the split unit of the persistent decode step), and a
// single-launch variant for rows whose scores fit in LDS (attn_fused_kernel,
// below) when the plan asks for one split.
//
// The reference's fallback (engine/ek_model.py:475-488) rounds the softmax
// probabilities to bf16 before the PV product: p = bf16(exp(s - M) / L) with
// M, L the max and sum over ALL keys of the row; its GPU kernels (the split
// decode kernel, engine/ek_kernels.py:535-616, 989-1019) keep p in fp32 and
// merge the splits by log-sum-exp. The single-launch kernel and the
// two-launch pair round p where the fallback does; the one-launch split form
// (below) follows the split decode kernel, which saves the round of split
// statistics that the fallback's rounding point needs before any PV work.
// The pair takes two launches over the same grid:
//
//   scores   [rope_attn_decode's prologue] QK-norm + RoPE of the G query
//            heads of this kv head (and, in the split owning the new slot,
//            of the new key, which is written to the cache with the raw
//            value); then S^T[16 keys x 16] = K_tile . Q^T on the matrix
//            cores (v_mfma_f32_16x16x32_bf16, the G heads in the first G
//            columns) for the split's keys -> fp32 scores in a scratch row,
//            plus the split's max m and sum l = sum exp(s - m) per head.
//   pv       M = max_s m_s, L = sum_s l_s exp(m_s - M) from the statistics;
//            p_n = bf16(exp(s_n - M) / L) for the split's keys into LDS;
//            the split's partial out = sum_n p_n v_n (fp32, all head dims)
//            with FMAs on lane-contiguous value rows; then the splits'
//            partials are added in split order by the last workgroup of the
//            (batch row, kv head) to start, and rounded to bf16 once.
//
// Cached keys and values are read once per launch: their loads are marked
// non-temporal (ld16_nt), which measurably shortens the split launches.
//
// The split combine needs no third launch and no memory fence: a
// workgroup takes an arrival ticket (atomic add at agent scope) when it
// starts and writes its partial as 64-bit words {fp32 value, launch tag},
// where the tag is one more than the (batch row, kv head)'s epoch word that
// the previous launch left. The workgroup with the last ticket reads every
// split's words until their tags match (all other workgroups of its row
// have started, so they are resident and finish), sums them, then resets
// the ticket counter and advances the epoch for the next launch. Launches
// on one workspace are stream-ordered, so the epoch and counter always
// describe the previous launch.
//
// Streaming: key and value rows are loaded lane-contiguously (lanes
// (D / 8) r .. (D / 8) r + D / 8 - 1 read row r), the layout the memory
// pipeline coalesces best; the scores kernel re-lays each 16-key tile
// through a per-wave LDS tile into the MFMA operand layout. Keys below
// start[b] (left padding) are never read. The owner split uses the new key
// from LDS rather than re-reading the slot it just wrote.

#include "ek_common.h"
#include "ek_abi_internal.h"
#include "ek_attn_impl.h"
#include "ek_step_impl.h"
#include "ek_hip.h"

#include <map>
#include <mutex>
#include <tuple>

namespace {

constexpr int NT = 256;
constexpr int NW = NT / EK_WAVE;

struct AttnParams {
  const bf16_t* q; int64_t ldq_b; int64_t ldq_h;
  int rope;
  const bf16_t* qn; const bf16_t* kn;
  const bf16_t* cos; const bf16_t* sin; int64_t ld_cs; const int64_t* positions; int64_t rope_len;
  bf16_t* kc; bf16_t* vc; int64_t csb, csh, css, s_cap;
  const int64_t* seq_len; const int32_t* start;
  float* scores; int64_t score_ss;
  float* lsum; float* mmax; int64_t sp, gp;
  bf16_t* out; int64_t ldo_b, ldo_h;
  int nq, nkv, splits; int64_t chunk;
  float sm_scale, eps;
  unsigned long long* part;   // [B, nkv, splits, G, D] {fp32 bits, tag} words
  uint32_t* ticket;           // [B * nkv][2]: arrivals of this launch, epoch
  int* err;                   // set to 1 when the combine's wait for a split gives up (may be null)
  int64_t spin;               // polls of that wait before it gives up
  int qvec;                   // q rows and heads 16-byte aligned (the one-launch form loads them whole)
};

struct Range { int64_t lo, hi, len; };

__device__ __forceinline__ Range key_range(const AttnParams& p, int s, int b) {
  int64_t len = *p.seq_len;
  len = len < 0 ? 0 : (len > p.s_cap ? p.s_cap : len);
  int64_t st = p.start[b];
  st = st < 0 ? 0 : st;
  int64_t lo = (int64_t)s * p.chunk;
  int64_t hi = (s == p.splits - 1) ? len : (lo + p.chunk < len ? lo + p.chunk : len);
  Range r;
  r.len = len;
  r.lo = lo;
  r.hi = hi;
  return r;
}

// ---------------------------------------------------------------------------
// launch 1: scores and the split's statistics
// ---------------------------------------------------------------------------
constexpr int KT = 16;   // keys per MFMA tile
constexpr int UT = 4;    // key tiles in flight per wave

template <int D>
struct RowShape {
  static constexpr int LPK = D / 8;          // lanes per key row (16 B each)
  static constexpr int KPI = EK_WAVE / LPK;  // keys per load instruction
  static constexpr int TL = KT / KPI;        // load instructions per 16-key tile
  static constexpr int DS = D / 32;          // MFMA steps per tile
  static constexpr int ROWB = 2 * D + 16;    // LDS tile row stride (bytes): conflict-free operand reads
};

// merge of two (max, sum-of-exp) statistics
__device__ __forceinline__ void ml_merge(float& m, float& l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  l = l * expf(m - mn) + l2 * expf(m2 - mn);
  m = mn;
}

template <int D, int G>
__global__ __launch_bounds__(NT) void attn_qk_kernel(AttnParams p) {
  using S = RowShape<D>;
  __shared__ float qs[G][D];
  __shared__ float knew[D];
  __shared__ __align__(16) unsigned char ktile[NW][KT * S::ROWB];
  __shared__ float stm[NW][G], stl[NW][G];

  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, q4 = lane >> 4;
  const Range rg = key_range(p, s, b);
  const int64_t slot = rg.len - 1;
  const bool owns = p.rope && slot >= rg.lo && slot < rg.hi;
  int64_t st = p.start[b];
  st = st < 0 ? 0 : st;
  const int64_t lo = rg.lo > st ? rg.lo : st;
  const int64_t hi = rg.hi;
  const int64_t ntile = hi > lo ? (hi - lo + KT - 1) / KT : 0;

  // the first key tiles in flight before the QK-norm/RoPE work; rows past
  // the split's end re-read its last row (their scores are dropped)
  const int lrow = lane / S::LPK, lpc = lane % S::LPK;
  const bf16_t* kb = p.kc + b * p.csb + h * p.csh + lpc * 8;
  auto krow = [&](int64_t t, int i) -> const bf16_t* {
    int64_t n = lo + t * KT + i * S::KPI + lrow;
    n = n < hi ? n : hi - 1;
    n = n < 0 ? 0 : n;
    return kb + n * p.css;
  };
  uint4 ring[UT][S::TL];
#pragma unroll
  for (int u = 0; u < UT; ++u)
#pragma unroll
    for (int i = 0; i < S::TL; ++i) ring[u][i] = ld16_nt(krow(wave + (int64_t)u * NW, i));

  if (p.rope) {
    const bf16_t* row = p.q + b * p.ldq_b;
    int64_t crow = p.positions ? p.positions[b] : b;
    crow = crow < 0 ? 0 : (crow >= p.rope_len ? p.rope_len - 1 : crow);
    const bf16_t* cr = p.cos + crow * p.ld_cs;
    const bf16_t* sr = p.sin + crow * p.ld_cs;
    const int units = G + (owns ? 2 : 0);
    for (int u = wave; u < units; u += NW) {
      if (u < G) {
        eka::head_norm_rope<D>(row + (int64_t)(h * G + u) * D, p.qn, cr, sr, p.eps, qs[u], nullptr);
      } else if (u == G) {
        bf16_t* kdst = p.kc + b * p.csb + h * p.csh + slot * p.css;
        eka::head_norm_rope<D>(row + (int64_t)(p.nq + h) * D, p.kn, cr, sr, p.eps, knew, kdst);
      } else {
        const bf16_t* vsrc = row + (int64_t)(p.nq + p.nkv + h) * D;
        bf16_t* vdst = p.vc + b * p.csb + h * p.csh + slot * p.css;
        for (int d = lane; d < D; d += EK_WAVE) vdst[d] = vsrc[d];
      }
    }
  } else {
    for (int i = tid; i < G * D; i += NT)
      qs[i / D][i % D] = bf2f(p.q[b * p.ldq_b + (int64_t)(h * G + i / D) * p.ldq_h + i % D]);
  }
  __syncthreads();

  // B operand: the G query heads in columns 0..G-1 (bf16, zero elsewhere)
  uint4 qb[S::DS];
  {
    const int g = r16 < G ? r16 : 0;
    const float keep = r16 < G ? 1.f : 0.f;
#pragma unroll
    for (int i = 0; i < S::DS; ++i) {
      const float* q = &qs[g][32 * i + 8 * q4];
      qb[i] = make_uint4(pack2(keep * q[0], keep * q[1]), pack2(keep * q[2], keep * q[3]),
                         pack2(keep * q[4], keep * q[5]), pack2(keep * q[6], keep * q[7]));
    }
  }
  // the new key's row as four 16-byte pieces per lane group (owner split)
  uint4 kn16 = make_uint4(0, 0, 0, 0);
  if (owns) {
    const float* k = &knew[lpc * 8];
    kn16 = make_uint4(pack2(k[0], k[1]), pack2(k[2], k[3]), pack2(k[4], k[5]), pack2(k[6], k[7]));
  }

  unsigned char* tile = ktile[wave];
  float* scb = p.scores + ((int64_t)b * p.nq + h * G + (r16 < G ? r16 : 0)) * p.score_ss;
  float m_run = -1e30f, l_run = 0.f;
  // this wave's tiles: wave, wave + NW, ...; a round takes UT of them (tiles
  // past the split's end are re-reads of its last row, fully masked)
  const int64_t nt_w = ntile > wave ? (ntile - wave + NW - 1) / NW : 0;
  for (int64_t k0 = 0; k0 < nt_w; k0 += UT) {
#pragma unroll
    for (int u = 0; u < UT; ++u) {
      const int64_t t = wave + (k0 + u) * NW;
      const int64_t tb = lo + t * KT;
      // stage the tile row-major (lane-contiguous), the new key in its slot
#pragma unroll
      for (int i = 0; i < S::TL; ++i) {
        const int r = i * S::KPI + lrow;
        // a bitwise blend: a select of the two would become a load through a
        // lane-dependent pointer and move the ring to scratch memory
        const uint32_t nm = (owns && tb + r == slot) ? 0xffffffffu : 0u;
        const uint4 v = ring[u][i];
        *reinterpret_cast<uint4*>(tile + r * S::ROWB + lpc * 16) =
            make_uint4((v.x & ~nm) | (kn16.x & nm), (v.y & ~nm) | (kn16.y & nm), (v.z & ~nm) | (kn16.z & nm),
                       (v.w & ~nm) | (kn16.w & nm));
      }
#pragma unroll
      for (int i = 0; i < S::TL; ++i) ring[u][i] = ld16_nt(krow(t + (int64_t)UT * NW, i));
      __builtin_amdgcn_sched_barrier(0);
      eka::f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < S::DS; ++i) {
        const uint4 a = *reinterpret_cast<const uint4*>(tile + r16 * S::ROWB + (32 * i + 8 * q4) * 2);
        c = eka::mfma16x16x32(a, qb[i], c);
      }
      // lanes r16 < G hold keys tb + 4 q4 + e of head r16
      float sc[4], mt = -1e30f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t n = tb + 4 * q4 + e;
        const bool ok = r16 < G && n < hi;
        sc[e] = c[e] * p.sm_scale;
        if (ok) scb[n] = sc[e];
        sc[e] = ok ? sc[e] : -1e30f;
        mt = fmaxf(mt, sc[e]);
      }
      const float mn = fmaxf(m_run, mt);
      float lt = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) lt += sc[e] > -1e29f ? expf(sc[e] - mn) : 0.f;
      l_run = l_run * expf(m_run - mn) + lt;
      m_run = mn;
    }
  }
  // merge the four lane groups of a head, then the waves
#pragma unroll
  for (int o = 16; o < EK_WAVE; o <<= 1) {
    const float m2 = __shfl_xor(m_run, o, EK_WAVE), l2 = __shfl_xor(l_run, o, EK_WAVE);
    ml_merge(m_run, l_run, m2, l2);
  }
  if (q4 == 0 && r16 < G) {
    stm[wave][r16] = m_run;
    stl[wave][r16] = l_run;
  }
  __syncthreads();
  if (tid < G) {
    float m = stm[0][tid], l = stl[0][tid];
    for (int w = 1; w < NW; ++w) ml_merge(m, l, stm[w][tid], stl[w][tid]);
    const int64_t o = (((int64_t)b * p.nkv + h) * p.sp + s) * p.gp + tid;
    p.mmax[o] = m;
    p.lsum[o] = l;
  }
}

// ---------------------------------------------------------------------------
// launch 2: the softmax-weighted value sum of a split, and the combine
// ---------------------------------------------------------------------------
constexpr int PB = 256;   // keys per probability block (one per thread)

__device__ __forceinline__ unsigned long long tagged(float v, uint32_t tag) {
  return ((unsigned long long)tag << 32) | __float_as_uint(v);
}

template <int D, int G>
__global__ __launch_bounds__(NT) void attn_pvs_kernel(AttnParams p) {
  using S = RowShape<D>;
  constexpr int KPW = PB / NW;                 // keys per wave per block
  constexpr int VL = KPW / S::KPI;             // value loads per lane per block
  __shared__ float Ms[G], Ls[G];
  __shared__ float wm[NW][G], wl[NW][G];
  __shared__ __align__(16) float pl[PB][G];
  __shared__ float red[NW][G][D];
  __shared__ uint32_t s_tag;
  __shared__ int s_last;

  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t bh = (int64_t)b * p.nkv + h;
  // the arrival ticket and the epoch, taken now; their values are first
  // needed at the end, so the round trip overlaps the work
  uint32_t t_old = 0, t_ep = 0;
  if (tid == 0) {
    t_old = __hip_atomic_fetch_add(p.ticket + 2 * bh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    t_ep = __hip_atomic_load(p.ticket + 2 * bh + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const Range rg = key_range(p, s, b);
  int64_t st = p.start[b];
  st = st < 0 ? 0 : st;
  const int64_t lo = rg.lo > st ? rg.lo : st;
  const int64_t hi = rg.hi;
  const int lrow = lane / S::LPK, lpc = lane % S::LPK;
  const bf16_t* vb = p.vc + b * p.csb + h * p.csh + lpc * 8;
  const float* scb = p.scores + ((int64_t)b * p.nq + h * G) * p.score_ss;

  // one block of PB keys: this thread's key's scores (issued first: loads
  // retire in order, so the probabilities wait only for them), then this
  // wave's value rows (rows past the end re-read the split's last row and
  // get p = 0). Blocks are double-buffered: the next block's loads are in
  // flight while the current one is consumed.
  auto load_blk = [&](int64_t kb, float (&sv)[G], uint4 (&vv)[VL]) {
    int64_t n = kb + tid;
    n = n < hi ? n : hi - 1;
    n = n < 0 ? 0 : n;
#pragma unroll
    for (int g = 0; g < G; ++g) sv[g] = scb[(int64_t)g * p.score_ss + n];
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      int64_t nv = kb + wave * KPW + i * S::KPI + lrow;
      nv = nv < hi ? nv : hi - 1;
      nv = nv < 0 ? 0 : nv;
      vv[i] = ld16_nt(vb + nv * p.css);
    }
  };
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;
  auto use_blk = [&](int64_t kb, const float (&sv)[G], const uint4 (&vv)[VL]) {
    const bool ok = kb + tid < hi;
#pragma unroll
    for (int g = 0; g < G; ++g) pl[tid][g] = ok ? rbf(expf(sv[g] - Ms[g]) / Ls[g]) : 0.f;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int kl = wave * KPW + i * S::KPI + lrow;
      float pv[G];
#pragma unroll
      for (int g = 0; g < G; ++g) pv[g] = pl[kl][g];
      float vf[8];
      unpack8(vv[i], vf);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] = fmaf(pv[g], vf[j], acc[g][j]);
    }
    __syncthreads();
  };

  // M and L of each head over all splits: thread t merges splits t, t + NT,
  // ..., then the lanes and the waves merge in a fixed order. The first
  // round's statistics are loaded before the first block's rows, which then
  // stay in flight while the statistics are merged.
  const int64_t base = bh * p.sp;
  float m[G], l[G];
  {
    const int s2 = tid < p.splits ? tid : 0;
    const float keep = tid < p.splits ? 0.f : -1e30f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = p.mmax[(base + s2) * p.gp + g];
      l[g] = p.lsum[(base + s2) * p.gp + g];
      m[g] = keep < 0.f ? -1e30f : m[g];
      l[g] = keep < 0.f ? 0.f : l[g];
    }
  }
  float s0[G], s1[G];
  uint4 v0[VL], v1[VL];
  load_blk(lo, s0, v0);
  for (int s2 = tid + NT; s2 < p.splits; s2 += NT)
#pragma unroll
    for (int g = 0; g < G; ++g) ml_merge(m[g], l[g], p.mmax[(base + s2) * p.gp + g], p.lsum[(base + s2) * p.gp + g]);
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int o = 1; o < EK_WAVE; o <<= 1)
      ml_merge(m[g], l[g], __shfl_xor(m[g], o, EK_WAVE), __shfl_xor(l[g], o, EK_WAVE));
    if (lane == 0) { wm[wave][g] = m[g]; wl[wave][g] = l[g]; }
  }
  __syncthreads();
  if (tid < G) {
    float mm = wm[0][tid], ll = wl[0][tid];
    for (int w = 1; w < NW; ++w) ml_merge(mm, ll, wm[w][tid], wl[w][tid]);
    Ms[tid] = mm;
    Ls[tid] = ll;
  }
  __syncthreads();

  for (int64_t kb = lo; kb < hi; kb += 2 * PB) {
    load_blk(kb + PB, s1, v1);
    use_blk(kb, s0, v0);
    if (kb + PB >= hi) break;
    load_blk(kb + 2 * PB, s0, v0);
    use_blk(kb + PB, s1, v1);
  }
  // fold the key rows of the wave (lanes with equal lpc), then the waves
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = acc[g][j];
#pragma unroll
      for (int o = S::LPK; o < EK_WAVE; o <<= 1) v += __shfl_xor(v, o, EK_WAVE);
      acc[g][j] = v;
    }
  if (lrow == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < 8; ++j) red[wave][g][lpc * 8 + j] = acc[g][j];
  }
  if (tid == 0) {
    s_tag = t_ep + 1;
    s_last = t_old == (uint32_t)(p.splits - 1);
  }
  __syncthreads();
  const uint32_t tag = s_tag;
  unsigned long long* part = p.part + (bh * p.splits) * (int64_t)(G * D);
  for (int i = tid; i < G * D; i += NT) {
    float t = red[0][i / D][i % D];
#pragma unroll
    for (int w = 1; w < NW; ++w) t += red[w][i / D][i % D];
    __hip_atomic_store(part + (int64_t)s * G * D + i, tagged(t, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!s_last) return;

  // the last workgroup to start: every split's partial, added in split
  // order; the words are read CB splits at a time with all loads in flight,
  // and a word whose tag is not yet this launch's is polled on its own
  constexpr int CB = 16;
  for (int i = tid; i < G * D; i += NT) {
    float t = 0.f;
    for (int s0 = 0; s0 < p.splits; s0 += CB) {
      unsigned long long v[CB];
#pragma unroll
      for (int k = 0; k < CB; ++k) {
        const int s2 = s0 + k < p.splits ? s0 + k : p.splits - 1;
        v[k] = __hip_atomic_load(part + (int64_t)s2 * G * D + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int k = 0; k < CB; ++k) {
        if (s0 + k < p.splits) {
          unsigned long long x = v[k];
          unsigned long long* w = part + (int64_t)(s0 + k) * G * D + i;
          for (int64_t spin = 0; (uint32_t)(x >> 32) != tag; ++spin) {
            if (spin >= p.spin) {   // a split never delivered: flag the output as invalid
              if (p.err) __hip_atomic_store(p.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              break;
            }
            __builtin_amdgcn_s_sleep(1);
            x = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          t += __uint_as_float((uint32_t)x);
        }
      }
    }
    p.out[b * p.ldo_b + (int64_t)(h * G + i / D) * p.ldo_h + i % D] = (bf16_t)f2bf(t);
  }
  __syncthreads();
  if (tid == 0) {
    __hip_atomic_store(p.ticket + 2 * bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p.ticket + 2 * bh + 1, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Single-launch variant (rows whose scores fit in LDS): one 512-thread
// workgroup per (batch row, kv head, 32 head dims), the unit of
// ek_attn_impl.h.
template <int D, int G>
__global__ __launch_bounds__(eka::FNT) void attn_fused_kernel(AttnParams p) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int bh = blockIdx.x;
  const int b = bh / p.nkv, h = bh % p.nkv;
  int64_t len = *p.seq_len;
  len = len < 0 ? 0 : (len > p.s_cap ? p.s_cap : len);
  int64_t lo = p.start[b];
  lo = lo < 0 ? 0 : lo;
  eka::AttnUnit u;
  if (p.rope) {
    const bf16_t* row = p.q + b * p.ldq_b;
    u.qh = row + (int64_t)h * G * D;
    u.q_stride = D;
    u.kh = row + (int64_t)(p.nq + h) * D;
    u.vh = row + (int64_t)(p.nq + p.nkv + h) * D;
    int64_t crow = p.positions ? p.positions[b] : b;
    crow = crow < 0 ? 0 : (crow >= p.rope_len ? p.rope_len - 1 : crow);
    u.cr = p.cos + crow * p.ld_cs;
    u.sr = p.sin + crow * p.ld_cs;
  } else {
    u.qh = p.q + b * p.ldq_b + (int64_t)h * G * p.ldq_h;
    u.q_stride = p.ldq_h;
    u.kh = u.vh = nullptr;
    u.cr = u.sr = nullptr;
  }
  u.rope = p.rope;
  u.qn = p.qn; u.kn = p.kn;
  u.eps = p.eps; u.sm_scale = p.sm_scale;
  u.kc = p.kc + b * p.csb + h * p.csh;
  u.vc = p.vc + b * p.csb + h * p.csh;
  u.css = p.css;
  u.cap = p.s_cap;
  u.lo = lo; u.hi = len;
  u.writer = blockIdx.y == 0;
  u.d0 = blockIdx.y * eka::FDC;
  u.out = p.out + b * p.ldo_b + (int64_t)h * G * p.ldo_h;
  u.out_stride = p.ldo_h;
  u.ll_out = nullptr;
#ifdef EK_STEP_TRACE
  u.trace_lds = nullptr;
#endif
  eka::attn_unit<D, G>(u, lds);
}

// Score rows up to this many bytes per workgroup take the single-launch path
// (with the kernel's static LDS, at most 64 KiB per workgroup) when the plan
// asks for one split.
// ---------------------------------------------------------------------------
// one launch: the persistent step's split unit
// ---------------------------------------------------------------------------
// When every workgroup of the (split, kv head, row) grid can be resident at
// once, one launch does it all: unit (b, h, s) is eks::long_attention --
// scores of its keys on the matrix cores into LDS, its max m and e = exp(s -
// m) (fp32) per head, its unnormalised partial sum e v, both published as
// tagged words with l = sum e, and the log-sum-exp merge of head dims
// [s D / S, (s + 1) D / S) from every split's words, stored as bf16. Split s takes the keys [lo + s c, lo + (s + 1) c)
// of the row's range [lo, len), c = ceil((len - lo) / S). The words go to
// `part` (per row: n_kv S (2G + G D) of them); their tag is one more than
// the (row, kv head)'s epoch word in the ticket block, which split 0 moves on
// once its combine has seen every split's words (so every workgroup of the
// pair has read it), as the pair's last workgroup does.
struct PlainIO {
  const bf16_t* q;           // row b: rope: the raw fused qkv row; else the rotated heads, ldq_h apart
  int64_t ldq_h;
  int rope_on;
  const int64_t* positions;  // cos/sin row of row b (row b when null)
  bf16_t* out;               // row b's output heads, ldo_h apart
  int64_t ldo_h;
  int nq, nkv;
  // loaded at the kernel's entry, ahead of everything that depends on the
  // row's length (no wait until the length's, which returns behind them):
  uint32_t ep;               // the (row, kv head)'s epoch word; the words' tag is one more
  uint32_t* tag_lds;         // where read_heads leaves the tag for the workgroup
  int hvec;                  // the heads as 16-byte pieces, hv (aligned rows)
  uint4 hv;                  // (thread i: elements 8 i .. 8 i + 7 of the heads' LDS rows)
  int64_t st;                // the row's first key
  static constexpr bool kTrim = true;
  static constexpr int kLateTiles = 0;
  __device__ uint32_t tag(uint32_t) const { return *tag_lds; }
  __device__ int64_t start(const eks::StepArgs&, int) const { return st; }
  __device__ bool rope() const { return rope_on != 0; }
  __device__ int64_t cs_row(const eks::StepArgs&, int b) const { return positions ? positions[b] : b; }
  template <int D, int G>
  __device__ bool read_heads(const eks::StepArgs&, int h, bf16_t* heads, int*) const {
    if (threadIdx.x == 0) *tag_lds = ep + 1u;
    if (hvec) {
      if ((int)threadIdx.x < (rope_on ? G + 2 : G) * D / 8) *reinterpret_cast<uint4*>(heads + 8 * threadIdx.x) = hv;
    } else if (rope_on) {
      for (int i = threadIdx.x; i < (G + 2) * D; i += eks::SNT) {
        const int t = i / D, d = i - t * D;
        const int head = t < G ? h * G + t : (t == G ? nq + h : nq + nkv + h);
        heads[i] = q[(int64_t)head * D + d];
      }
    } else {
      for (int i = threadIdx.x; i < G * D; i += eks::SNT) heads[i] = q[(int64_t)(h * G + i / D) * ldq_h + i % D];
    }
    __syncthreads();
    return true;
  }
  template <int D, int G>
  __device__ void put4(int h, int g, int d, const float* v) const {
    bf16_t* o = out + (int64_t)(h * G + g) * ldo_h + d;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (bf16_t)f2bf(v[e]);
  }
};

template <int D, int G>
__global__ __launch_bounds__(eks::SNT) void attn_onepass_kernel(AttnParams p, int lchunk) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int s_fail;
  __shared__ uint32_t s_tag;
  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * p.nkv + h;
  // s_fail is first read after read_heads' barrier, s_tag is written there
  if (threadIdx.x == 0) s_fail = 0;
  eks::StepArgs a = {};
  a.nq = p.nq; a.nkv = p.nkv; a.eps = p.eps; a.sm_scale = p.sm_scale;
  a.cos = p.cos; a.sin = p.sin; a.ld_cs = p.ld_cs; a.rope_len = p.rope_len;
  a.csb = p.csb; a.csh = p.csh; a.css = p.css; a.s_cap = p.s_cap;
  a.start_t = p.start; a.err = p.err; a.spin = p.spin; a.lchunk = lchunk;
  int64_t lw[eks::LW_FIELDS] = {};
  lw[eks::LW_QN] = (int64_t)p.qn;
  lw[eks::LW_KN] = (int64_t)p.kn;
  lw[eks::LW_KC] = (int64_t)p.kc;
  lw[eks::LW_VC] = (int64_t)p.vc;
  int64_t hi = *p.seq_len;
  hi = hi < 0 ? 0 : (hi > p.s_cap ? p.s_cap : hi);
  PlainIO io{p.q + b * p.ldq_b, p.ldq_h, p.rope, p.positions, p.out + b * p.ldo_b, p.ldo_h, p.nq, p.nkv,
             0u, &s_tag, p.qvec, make_uint4(0u, 0u, 0u, 0u), (int64_t)p.start[b]};
  io.ep = __hip_atomic_load(p.ticket + 2 * bh + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (p.qvec && (int)threadIdx.x < (((p.rope ? G + 2 : G) * D / 8 + 63) & ~63)) {   // whole waves
    // piece i: the q heads (rope: then the new key and value heads) in order
    const int n16 = (p.rope ? G + 2 : G) * D / 8;
    const int e = 8 * ((int)threadIdx.x < n16 ? (int)threadIdx.x : 0), t = e / D, d = e - t * D;
    const bf16_t* src = p.rope ? io.q + (int64_t)(t < G ? h * G + t : (t == G ? p.nq + h : p.nq + p.nkv + h)) * D + d
                               : io.q + (int64_t)(h * G + t) * p.ldq_h + d;
    io.hv = *reinterpret_cast<const uint4*>(src);
  }
  eks::long_attention<D, G>(a, lw, io, p.part + b * eks::long_words(p.nkv, p.splits, G, D), b, h, s, p.splits, hi,
                            0u, lds, &s_fail);
  // also after a wait gave up (the error word is then set): the next launch
  // must not take this launch's words for its own
  if (s == 0 && threadIdx.x == 0)
    __hip_atomic_store(p.ticket + 2 * bh + 1, s_tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The one-launch form's LDS (keys per split at most lchunk), and whether its
// (splits, n_kv, b) grid is resident at once on the current device
template <int D, int G>
size_t onepass_lds(int lchunk) { return eks::LongLds<D, G>::bytes(lchunk); }

int device_cus() {
  static int n = -1;
  if (n < 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 0;
  }
  return n;
}

template <int D, int G>
bool onepass_fits(int64_t grid, size_t lds) {
  static std::mutex mu;
  static std::map<size_t, int> cache;
  int per_cu = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(lds);
    if (it != cache.end()) {
      per_cu = it->second;
    } else {
      if (hipFuncSetAttribute((const void*)attn_onepass_kernel<D, G>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)eks::kStepDynLds) != hipSuccess ||
          hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_onepass_kernel<D, G>, eks::SNT, lds) != hipSuccess)
        per_cu = 0;
      cache[lds] = per_cu;
    }
  }
  return grid <= (int64_t)per_cu * device_cus();
}

constexpr size_t kFusedScoreLds = 32 * 1024;

template <int D, int G>
hipError_t launch_attn(const AttnParams& p, int b, int64_t part_words, hipStream_t st) {
  if (p.splits == 1 && (size_t)G * p.s_cap * sizeof(float) <= kFusedScoreLds) {
    dim3 grid((unsigned)(b * p.nkv), (unsigned)(D / eka::FDC));
    const size_t lds = eka::AttnLds<D, G>::bytes(p.s_cap);
    hipLaunchKernelGGL((attn_fused_kernel<D, G>), grid, dim3(eka::FNT), lds, st, p);
    return hipGetLastError();
  }
  dim3 grid((unsigned)p.splits, (unsigned)p.nkv, (unsigned)b);
  // the one-launch form: splits a power of two up to min(32, D / 4) (each
  // split combines whole 4-dim groups; the combine's lanes sit in one wave),
  // an error word for its bounded waits, room for its words, its score rows
  // in LDS, and the whole grid resident at once
  const int64_t lchunk = (p.s_cap + p.splits - 1) / p.splits;
  const int smax = D / 4 < 32 ? D / 4 : 32;
  if (p.err && p.splits <= smax && (p.splits & (p.splits - 1)) == 0 && lchunk <= 65536 &&
      part_words >= (int64_t)b * eks::long_words(p.nkv, p.splits, G, D)) {
    const size_t lds = onepass_lds<D, G>((int)lchunk);
    if (lds <= eks::kStepDynLds && onepass_fits<D, G>((int64_t)p.splits * p.nkv * b, lds)) {
      hipLaunchKernelGGL((attn_onepass_kernel<D, G>), grid, dim3(eks::SNT), lds, st, p, (int)lchunk);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((attn_qk_kernel<D, G>), grid, dim3(NT), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_pvs_kernel<D, G>), grid, dim3(NT), 0, st, p);
  return hipGetLastError();
}

template <int D>
hipError_t launch_attn_g(const AttnParams& p, int g, int b, int64_t part_words, hipStream_t st) {
  switch (g) {
    case 1: return launch_attn<D, 1>(p, b, part_words, st);
    case 2: return launch_attn<D, 2>(p, b, part_words, st);
    case 4: return launch_attn<D, 4>(p, b, part_words, st);
    case 8: return launch_attn<D, 8>(p, b, part_words, st);
    default: return ek_fail(hipErrorInvalidValue, "attn: query heads per kv head must be 1, 2, 4 or 8");
  }
}

}  // namespace

extern "C" {

int ek_attn_decode(const void* q, int64_t ldq_b, int64_t ldq_h, int rope, const void* qn, const void* kn,
                   const void* cos, const void* sin, int64_t ld_cs, const int64_t* positions, int64_t rope_len,
                   void* k_cache, void* v_cache, int64_t csb, int64_t csh, int64_t css, int64_t s_cap,
                   const int64_t* seq_len, const int32_t* start, float* scores, int64_t score_ss, float* lsum,
                   float* mmax, int64_t sp, int64_t gp, void* out, int64_t ldo_b,
                   int64_t ldo_h, int64_t b, int64_t n_q, int64_t n_kv, int64_t head_dim, int64_t splits,
                   int64_t chunk, float sm_scale, float eps, void* part, int64_t part_words, uint32_t* ticket,
                   int* err, void* stream) {
  EK_GUARD();
  if (b < 1 || b * n_kv > 0x7fffffff || n_kv < 1 || n_q < n_kv || n_q % n_kv || b > 65535)
    return ek_fail(hipErrorInvalidValue, "attn: bad batch or head counts");
  const int64_t g = n_q / n_kv;
  if (splits < 1 || splits > sp || chunk < 1 || g > gp)
    return ek_fail(hipErrorInvalidValue, "attn: splits/chunk exceed the workspace");
  if (score_ss < s_cap) return ek_fail(hipErrorInvalidValue, "attn: score scratch shorter than the cache");
  const bool fused = splits == 1 && (size_t)g * s_cap * sizeof(float) <= kFusedScoreLds;
  if (!fused && (!part || !ticket || part_words < b * n_kv * splits * g * head_dim))
    return ek_fail(hipErrorInvalidValue, "attn: the split path needs the partial words and the ticket block");
  if (splits > 65535) return ek_fail(hipErrorInvalidValue, "attn: too many splits");
  if (rope && (!qn || !kn || !cos || !sin || rope_len < 1))
    return ek_fail(hipErrorInvalidValue, "attn: rope mode needs qn, kn, cos, sin");
  if (css % 8 || csh % 8 || csb % 8 || (reinterpret_cast<uintptr_t>(k_cache) & 15) ||
      (reinterpret_cast<uintptr_t>(v_cache) & 15))
    return ek_fail(hipErrorInvalidValue, "attn: cache rows must be 16-byte aligned");
  AttnParams p;
  memset(&p, 0, sizeof(p));
  p.q = (const bf16_t*)q; p.ldq_b = ldq_b; p.ldq_h = ldq_h; p.rope = rope;
  p.qn = (const bf16_t*)qn; p.kn = (const bf16_t*)kn;
  p.cos = (const bf16_t*)cos; p.sin = (const bf16_t*)sin; p.ld_cs = ld_cs; p.positions = positions;
  p.rope_len = rope_len;
  p.kc = (bf16_t*)k_cache; p.vc = (bf16_t*)v_cache; p.csb = csb; p.csh = csh; p.css = css; p.s_cap = s_cap;
  p.seq_len = seq_len; p.start = start;
  p.scores = scores; p.score_ss = score_ss;
  p.lsum = lsum; p.mmax = mmax; p.sp = sp; p.gp = gp;
  p.out = (bf16_t*)out; p.ldo_b = ldo_b; p.ldo_h = ldo_h;
  p.nq = (int)n_q; p.nkv = (int)n_kv; p.splits = (int)splits; p.chunk = chunk;
  p.sm_scale = sm_scale; p.eps = eps;
  p.part = (unsigned long long*)part; p.ticket = ticket;
  p.err = err; p.spin = ek_wait_limit(int64_t(1) << 22);
  p.qvec = (reinterpret_cast<uintptr_t>(q) & 15) == 0 && ldq_b % 8 == 0 && (rope || ldq_h % 8 == 0);
  hipStream_t st = (hipStream_t)stream;
  switch (head_dim) {
    case 32: return launch_attn_g<32>(p, (int)g, (int)b, part_words, st);
    case 64: return launch_attn_g<64>(p, (int)g, (int)b, part_words, st);
    case 128: return launch_attn_g<128>(p, (int)g, (int)b, part_words, st);
    default: return ek_fail(hipErrorInvalidValue, "attn: head_dim must be 32, 64 or 128");
  }
}

}  // extern "C"
