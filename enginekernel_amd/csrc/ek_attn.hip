// Decode attention over the static KV cache, for gfx950. Rows whose scores
// fit in LDS take a single launch (attn_fused_kernel, below); longer rows the
// two-phase split-K pair described here.
//
// The reference's fallback (engine/ek_model.py:475-488) rounds the softmax
// probabilities to bf16 before the PV product: p = bf16(exp(s - M) / L) with
// M, L the max and sum over ALL keys of the row. A one-pass flash-decode
// cannot round there (it only knows M and L at the end), so the build splits
// the work into two launches over the same (split, kv-head, batch) grid:
//
//   phase 1  [rope_attn_decode's prologue] QK-norm + RoPE of the G query
//            heads of this kv head (and, in the split owning the new slot,
//            of the new key, which is written to the cache with the raw
//            value), then fp32 scores s_n = (q . k_n) * scale for the
//            split's keys -> a score scratch row, plus the split's running
//            max m and sum l = sum exp(s - m).
//   phase 2  one workgroup per (batch, kv head, chunk of DC head dims) over
//            ALL keys: M = max_s m_s, L = sum_s l_s exp(m_s - M) from the
//            splits' statistics; p_n = bf16(exp(s_n - M) / L); out =
//            bf16(sum_n p_n v_n[chunk]) (fp32 sum). Splitting the head
//            dimension instead of the keys leaves nothing to combine, so no
//            workgroup waits on another: the eight L2s of the chip are not
//            coherent, and a cross-workgroup handoff inside a kernel would
//            need a full L2 write-back per workgroup.
//
// Bytes: K is read once (phase 1), V once (phase 2); the score scratch adds
// 4 bytes per key per query head written, and read once per dim chunk (at
// G = 4, D = 128, DC = 32: 16 B written + 64 B read per key, against 512 B
// of K+V). Lane layout: a key row's chunk of 16 B per lane, so a wave reads
// 64/(D/8) keys per load instruction in phase 1 (4 keys, 1 KiB at D = 128)
// and 64/(DC/8) keys in phase 2 (16 keys at DC = 32); dot products are
// folded over the lanes of a key with a butterfly.
//
// Keys below start[b] (left padding) are never read. The owner split uses
// the new key from LDS rather than re-reading the slot it just wrote. The
// first key loads are issued before the QK-norm/RoPE work so that their
// latency overlaps it.

#include "ek_common.h"
#include "ek_abi_internal.h"
#include "ek_hip.h"

namespace {

constexpr int NT = 256;
constexpr int NW = NT / EK_WAVE;
constexpr int UNR = 4;   // key steps in flight per lane

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

// QK-norm + rotate-half RoPE of one head (one wave); writes the bf16-valued
// result as fp32 to `dst` (LDS) and, if `gdst`, as bf16 to global memory.
template <int D>
__device__ __forceinline__ void head_norm_rope(const bf16_t* x, const bf16_t* w, const bf16_t* cr,
                                               const bf16_t* sr, float eps, float* dst, bf16_t* gdst) {
  constexpr int PER = D > 64 ? D / 64 : 1;
  constexpr int HALF = D / 2;
  const int lane = threadIdx.x & 63;
  float xv[PER], xp[PER];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = lane + 64 * i;
    const bool ok = d < D;
    const int pd = d < HALF ? d + HALF : d - HALF;
    xv[i] = ok ? bf2f(x[d]) : 0.f;
    xp[i] = ok ? bf2f(x[pd]) : 0.f;
    ss = fmaf(xv[i], xv[i], ss);
  }
  ss = wave_sum(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = lane + 64 * i;
    if (d >= D) continue;
    const int pd = d < HALF ? d + HALF : d - HALF;
    const float tn = rbf(bf2f(w[d]) * rbf(xv[i] * rstd));
    const float tp = rbf(bf2f(w[pd]) * rbf(xp[i] * rstd));
    const float rot = d < HALF ? -tp : tp;
    const float o = rbf(rbf(tn * bf2f(cr[d])) + rbf(rot * bf2f(sr[d])));
    dst[d] = o;
    if (gdst) gdst[d] = (bf16_t)f2bf(o);
  }
}

template <int D, int G>
__global__ __launch_bounds__(NT) void attn_scores_kernel(AttnParams p) {
  constexpr int LPK = D / 8;         // lanes per key row
  constexpr int KPW = EK_WAVE / LPK; // keys per wave per load
  constexpr int KPB = NW * KPW;      // keys per workgroup per load
  __shared__ float qs[G][D];
  __shared__ float knew[D];
  __shared__ float stm[NW * KPW][G];
  __shared__ float stl[NW * KPW][G];

  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const Range rg = key_range(p, s, b);
  const int64_t slot = rg.len - 1;
  const bool owns = p.rope && slot >= rg.lo && slot < rg.hi;
  int64_t st = p.start[b];
  st = st < 0 ? 0 : st;
  const int64_t lo = rg.lo > st ? rg.lo : st;
  const int64_t hi = rg.hi;

  const int sub = lane % LPK, grp = lane / LPK;
  const bf16_t* kb = p.kc + b * p.csb + h * p.csh + sub * 8;
  // first key tiles in flight before the QK-norm/RoPE work
  uint4 kv[UNR];
  const int64_t first = lo + wave * KPW + grp;
#pragma unroll
  for (int u = 0; u < UNR; ++u) {
    const int64_t n = first + (int64_t)u * KPB;
    kv[u] = (n < hi) ? ld16(kb + n * p.css) : make_uint4(0, 0, 0, 0);
  }

  if (p.rope) {
    const bf16_t* row = p.q + b * p.ldq_b;
    int64_t crow = p.positions ? p.positions[b] : b;
    crow = crow < 0 ? 0 : (crow >= p.rope_len ? p.rope_len - 1 : crow);
    const bf16_t* cr = p.cos + crow * p.ld_cs;
    const bf16_t* sr = p.sin + crow * p.ld_cs;
    const int units = G + (owns ? 2 : 0);
    for (int u = wave; u < units; u += NW) {
      if (u < G) {
        head_norm_rope<D>(row + (int64_t)(h * G + u) * D, p.qn, cr, sr, p.eps, qs[u], nullptr);
      } else if (u == G) {
        bf16_t* kdst = p.kc + b * p.csb + h * p.csh + slot * p.css;
        head_norm_rope<D>(row + (int64_t)(p.nq + h) * D, p.kn, cr, sr, p.eps, knew, kdst);
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

  float qr[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) qr[g][j] = qs[g][sub * 8 + j];
  float kn8[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) kn8[j] = owns ? knew[sub * 8 + j] : 0.f;

  float mr[G], lr[G];
#pragma unroll
  for (int g = 0; g < G; ++g) { mr[g] = -1e30f; lr[g] = 0.f; }

  float* scb = p.scores + ((int64_t)b * p.nq + h * G) * p.score_ss;
  for (int64_t n0 = first; n0 < hi; n0 += (int64_t)KPB * UNR) {
    if (n0 != first) {
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int64_t n = n0 + (int64_t)u * KPB;
        kv[u] = (n < hi) ? ld16(kb + n * p.css) : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t n = n0 + (int64_t)u * KPB;
      const bool valid = n < hi;
      float kf[8];
      unpack8(kv[u], kf);
      if (owns && n == slot) {
#pragma unroll
        for (int j = 0; j < 8; ++j) kf[j] = kn8[j];
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) d = fmaf(qr[g][j], kf[j], d);
        d = group_sum<LPK>(d);
        const float sc = d * p.sm_scale;
        if (valid) {
          if (sub == (g % LPK)) scb[(int64_t)g * p.score_ss + n] = sc;
          const float mn = fmaxf(mr[g], sc);
          lr[g] = lr[g] * expf(mr[g] - mn) + expf(sc - mn);
          mr[g] = mn;
        }
      }
    }
  }
  if (sub == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      stm[wave * KPW + grp][g] = mr[g];
      stl[wave * KPW + grp][g] = lr[g];
    }
  }
  __syncthreads();
  if (tid < G) {
    float M = -1e30f;
    for (int i = 0; i < NW * KPW; ++i) M = fmaxf(M, stm[i][tid]);
    float L = 0.f;
    for (int i = 0; i < NW * KPW; ++i) L += stl[i][tid] * expf(stm[i][tid] - M);
    const int64_t o = (((int64_t)b * p.nkv + h) * p.sp + s) * p.gp + tid;
    p.mmax[o] = M;
    p.lsum[o] = L;
  }
}

template <int D, int G, int DC>
__global__ __launch_bounds__(NT) void attn_pv_kernel(AttnParams p) {
  constexpr int LPK = DC / 8;          // lanes per key (16 B of the chunk each)
  constexpr int KPW = EK_WAVE / LPK;   // keys per wave per load
  constexpr int KPB = NW * KPW;
  __shared__ float Ms[G], Ls[G];
  __shared__ float red[NW][G][DC];

  const int bh = blockIdx.x;
  const int b = bh / p.nkv, h = bh % p.nkv;
  const int d0 = blockIdx.y * DC;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int64_t len = *p.seq_len;
  len = len < 0 ? 0 : (len > p.s_cap ? p.s_cap : len);
  int64_t lo = p.start[b];
  lo = lo < 0 ? 0 : lo;
  const int64_t hi = len;

  const int sub = lane % LPK, grp = lane / LPK;
  const bf16_t* vb = p.vc + b * p.csb + h * p.csh + d0 + sub * 8;
  const float* scb = p.scores + ((int64_t)b * p.nq + h * G) * p.score_ss;
  const int64_t first = lo + wave * KPW + grp;
  uint4 vv[UNR];
  float sv[UNR][G];
#pragma unroll
  for (int u = 0; u < UNR; ++u) {
    const int64_t n = first + (int64_t)u * KPB;
    const bool valid = n < hi;
    vv[u] = valid ? ld16(vb + n * p.css) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int g = 0; g < G; ++g) sv[u][g] = valid ? scb[(int64_t)g * p.score_ss + n] : 0.f;
  }

  const int64_t hbase = ((int64_t)b * p.nkv + h) * p.sp;
  if (tid < G) {
    float M = -1e30f;
    for (int s2 = 0; s2 < p.splits; ++s2) M = fmaxf(M, p.mmax[(hbase + s2) * p.gp + tid]);
    float L = 0.f;
    for (int s2 = 0; s2 < p.splits; ++s2) {
      const int64_t o = (hbase + s2) * p.gp + tid;
      L += p.lsum[o] * expf(p.mmax[o] - M);
    }
    Ms[tid] = M;
    Ls[tid] = L;
  }
  __syncthreads();
  float Mr[G], Lr[G];
#pragma unroll
  for (int g = 0; g < G; ++g) { Mr[g] = Ms[g]; Lr[g] = Ls[g]; }

  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;

  for (int64_t n0 = first; n0 < hi; n0 += (int64_t)KPB * UNR) {
    if (n0 != first) {
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int64_t n = n0 + (int64_t)u * KPB;
        const bool valid = n < hi;
        vv[u] = valid ? ld16(vb + n * p.css) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int g = 0; g < G; ++g) sv[u][g] = valid ? scb[(int64_t)g * p.score_ss + n] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t n = n0 + (int64_t)u * KPB;
      if (n >= hi) continue;
      float vf[8];
      unpack8(vv[u], vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pr = rbf(expf(sv[u][g] - Mr[g]) / Lr[g]);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] = fmaf(pr, vf[j], acc[g][j]);
      }
    }
  }
  // fold the key groups of the wave (lanes with equal `sub`), then the waves
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = acc[g][j];
#pragma unroll
      for (int o = LPK; o < EK_WAVE; o <<= 1) v += __shfl_xor(v, o, EK_WAVE);
      acc[g][j] = v;
    }
  if (grp == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < 8; ++j) red[wave][g][sub * 8 + j] = acc[g][j];
  }
  __syncthreads();
  for (int i = tid; i < G * DC; i += NT) {
    const int g = i / DC, d = i % DC;
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) t += red[w][g][d];
    p.out[b * p.ldo_b + (int64_t)(h * G + g) * p.ldo_h + d0 + d] = (bf16_t)f2bf(t);
  }
}

// ----------------------------------------------------------------------------
// Single-launch variant for short rows (the score row of a head fits in LDS):
// one workgroup per (batch, kv head, chunk of 32 head dims), both products on
// the matrix cores (v_mfma_f32_16x16x32_bf16: bf16 products are exact in
// fp32, sums are fp32).
//
//   scores   per tile of 16 keys, S^T[16 x 16] = K_tile[16 x D] . Q^T[D x 16]
//            with the G query heads in the first G columns, scaled, into an
//            LDS row per head. Each lane also keeps the running max and
//            exp-sum of the scores it produced; the lanes and waves merge
//            them into the row's M and L. Every chunk workgroup of a head
//            computes all of the head's scores; when B * n_kv is a multiple of
//            8 those workgroups sit on one XCD (workgroups are dealt
//            round-robin over the 8 XCDs by linear id), so the repeated K
//            reads hit its L2.
//   softmax  p = bf16(exp(s - M) / L) in place, one exp per score, spread
//            over all threads.
//   PV       per tile of 32 keys, O[16 x 16] += P[16 x 32] . V[32 x 16] per
//            16 head dims, the heads in the first G rows. V arrives as 16 B per
//            lane and is re-laid through a per-wave LDS tile into the B
//            operand (8 keys of one dim per lane), so the key sum happens
//            inside the MFMA. The waves' partial outputs are added through
//            LDS and rounded to bf16 once.
//
// Nothing crosses workgroups, so attention is one launch with no score
// scratch. In rope mode every workgroup norms/rotates its query heads and the
// new key (which stands in for the cache row at the new slot), takes the raw
// new value from the qkv row (likewise), and the chunk-0 workgroup also
// stores both in the cache. Rounding points are those of the two-phase
// kernels. The first K tiles are loaded at entry, before the QK-norm/RoPE
// work, and the first V tiles right after it, so both overlap the work
// before their use.
//
// MFMA lane layout (16x16x32): lane l = r + 16 q (r < 16, q < 4) holds
// A[row r][k = 8q .. 8q+7], B[k = 8q .. 8q+7][col r] and C[rows 4q .. 4q+3][col r].
// ----------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int FNT = 512;
constexpr int FNW = FNT / EK_WAVE;
constexpr int FTU = 4;     // 16-key score tiles in flight per wave
constexpr int FPT = 2;     // 32-key PV tiles in flight per wave
constexpr int FDC = 32;    // head dims per workgroup
constexpr int VTS = FDC + 4;   // LDS row of a staged V tile (bf16; 72 B keeps reads conflict-free)

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

__device__ __forceinline__ f32x4_t mfma16x16x32(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// merge a (max, sum of exp(s - max)) pair into another
__device__ __forceinline__ void merge_ml(float& m, float& l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  l = l * expf(m - mn) + l2 * expf(m2 - mn);
  m = mn;
}

template <int D, int G>
__global__ __launch_bounds__(FNT) void attn_fused_kernel(AttnParams p) {
  constexpr int KS = D / 32;   // 32-dim k-steps of a score tile
  static_assert(G <= 8 && D % 32 == 0, "tile shape");
  extern __shared__ float sc_lds[];   // [G][s_cap] scores by key - lo
  __shared__ float qs[G][D];
  __shared__ float knew[D];
  __shared__ __align__(16) uint16_t vnew[FDC];
  __shared__ float stm[FNW][8], stl[FNW][8];
  __shared__ __align__(16) uint16_t vt[FNW][32][VTS];
  __shared__ float outp[FNW][G][FDC];

  const int bh = blockIdx.x;
  const int b = bh / p.nkv, h = bh % p.nkv;
  const int d0 = blockIdx.y * FDC;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, q4 = lane >> 4;
  const int64_t cap = p.s_cap;
  int64_t len = *p.seq_len;
  len = len < 0 ? 0 : (len > cap ? cap : len);
  int64_t lo = p.start[b];
  lo = lo < 0 ? 0 : lo;
  const int64_t hi = len;
  const int64_t nrel = hi > lo ? hi - lo : 0;   // keys attended
  const int64_t slot = len - 1;
  const bool fresh = p.rope && slot >= lo;      // the new key/value come from the qkv row
  const int64_t srel = slot - lo;

  // first K tiles in flight before any other work: lane holds key row r16
  // of the tile, dims 32 i + 8 q4 .. +7
  const bf16_t* kb = p.kc + b * p.csb + h * p.csh + 8 * q4;
  const int64_t ntile = (nrel + 15) >> 4;
  uint4 kt[FTU][KS];
#pragma unroll
  for (int u = 0; u < FTU; ++u) {
    const int64_t rel = ((int64_t)(wave + u * FNW) << 4) + r16;
#pragma unroll
    for (int i = 0; i < KS; ++i)
      kt[u][i] = rel < nrel ? ld16(kb + (lo + rel) * p.css + 32 * i) : make_uint4(0, 0, 0, 0);
  }

  if (p.rope) {
    const bf16_t* row = p.q + b * p.ldq_b;
    int64_t crow = p.positions ? p.positions[b] : b;
    crow = crow < 0 ? 0 : (crow >= p.rope_len ? p.rope_len - 1 : crow);
    const bf16_t* cr = p.cos + crow * p.ld_cs;
    const bf16_t* sr = p.sin + crow * p.ld_cs;
    const bool writer = blockIdx.y == 0 && slot >= 0;
    const int units = G + ((fresh || writer) ? 1 : 0);
    for (int u = wave; u < units; u += FNW) {
      if (u < G) {
        head_norm_rope<D>(row + (int64_t)(h * G + u) * D, p.qn, cr, sr, p.eps, qs[u], nullptr);
      } else {
        bf16_t* kdst = writer ? p.kc + b * p.csb + h * p.csh + slot * p.css : nullptr;
        head_norm_rope<D>(row + (int64_t)(p.nq + h) * D, p.kn, cr, sr, p.eps, knew, kdst);
      }
    }
    if (writer && wave == FNW - 1) {
      const bf16_t* vsrc = row + (int64_t)(p.nq + p.nkv + h) * D;
      bf16_t* vdst = p.vc + b * p.csb + h * p.csh + slot * p.css;
      for (int d = lane; d < D; d += EK_WAVE) vdst[d] = vsrc[d];
    }
    if (fresh && tid < FDC) vnew[tid] = row[(int64_t)(p.nq + p.nkv + h) * D + d0 + tid];
  } else {
    for (int i = tid; i < G * D; i += FNT)
      qs[i / D][i % D] = bf2f(p.q[b * p.ldq_b + (int64_t)(h * G + i / D) * p.ldq_h + i % D]);
  }

  // first V tiles in flight: 16 B chunks c = lane + 64 m of the 32 x 32 tile,
  // key c / 4, dims 8 (c % 4) .. +7
  const int vkey = lane >> 2, vsub = lane & 3;
  const bf16_t* vb = p.vc + b * p.csb + h * p.csh + d0 + 8 * vsub;
  const int64_t ntile32 = (nrel + 31) >> 5;
  uint4 vreg[FPT][2];
#pragma unroll
  for (int u = 0; u < FPT; ++u) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int64_t rel = ((int64_t)(wave + u * FNW) << 5) + vkey + 16 * m;
      vreg[u][m] = (rel < nrel && !(fresh && rel == srel)) ? ld16(vb + (lo + rel) * p.css) : make_uint4(0, 0, 0, 0);
    }
  }
  __syncthreads();

  // ---- scores. B operand = Q^T: q[g = r16][32 i + 8 q4 .. +7], zero for g >= G
  uint4 qb[KS];
#pragma unroll
  for (int i = 0; i < KS; ++i) {
    const int g = r16 < G ? r16 : 0;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int dd = 32 * i + 8 * q4 + 2 * e;
      w[e] = r16 < G ? (f2bf(qs[g][dd]) | (f2bf(qs[g][dd + 1]) << 16)) : 0u;
    }
    qb[i] = make_uint4(w[0], w[1], w[2], w[3]);
  }
  float mrun = -1e30f, lrun = 0.f;   // this lane's scores: head r16, running max / exp-sum
  for (int64_t t0 = wave; t0 < ntile; t0 += (int64_t)FNW * FTU) {
    if (t0 != wave) {
#pragma unroll
      for (int u = 0; u < FTU; ++u) {
        const int64_t rel = ((t0 + u * FNW) << 4) + r16;
#pragma unroll
        for (int i = 0; i < KS; ++i)
          kt[u][i] = rel < nrel ? ld16(kb + (lo + rel) * p.css + 32 * i) : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < FTU; ++u) {
      const int64_t tb = (t0 + u * FNW) << 4;
      if (tb >= nrel) break;
      if (fresh && tb + r16 == srel) {   // the new key, not the cache row
#pragma unroll
        for (int i = 0; i < KS; ++i) {
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int dd = 32 * i + 8 * q4 + 2 * e;
            w[e] = f2bf(knew[dd]) | (f2bf(knew[dd + 1]) << 16);
          }
          kt[u][i] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KS; ++i) c = mfma16x16x32(kt[u][i], qb[i], c);
      if (r16 < G) {
        float sv[4];
        float mx = mrun;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t rel = tb + 4 * q4 + e;
          sv[e] = c[e] * p.sm_scale;
          if (rel < nrel) {
            sc_lds[(int64_t)r16 * cap + rel] = sv[e];
            mx = fmaxf(mx, sv[e]);
          }
        }
        float add = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (tb + 4 * q4 + e < nrel) add += expf(sv[e] - mx);
        lrun = lrun * expf(mrun - mx) + add;
        mrun = mx;
      }
    }
  }
  // merge over the four lane rows of a head, then over the waves
#pragma unroll
  for (int o = 16; o < EK_WAVE; o <<= 1) {
    const float m2 = __shfl_xor(mrun, o, EK_WAVE);
    const float l2 = __shfl_xor(lrun, o, EK_WAVE);
    merge_ml(mrun, lrun, m2, l2);
  }
  if (q4 == 0 && r16 < G) {
    stm[wave][r16] = mrun;
    stl[wave][r16] = lrun;
  }
  __syncthreads();
  // p = bf16(exp(s - M) / L) in place, once per score: thread -> head tid % G
  {
    const int g = tid % G;
    float M = stm[0][g], L = stl[0][g];
#pragma unroll
    for (int w = 1; w < FNW; ++w) merge_ml(M, L, stm[w][g], stl[w][g]);
    float* row = sc_lds + (int64_t)g * cap;
    for (int64_t n = tid / G; n < nrel; n += FNT / G) row[n] = rbf(expf(row[n] - M) / L);
  }
  __syncthreads();

  // ---- PV. A operand = P: p[head r16][keys 8 q4 .. +7 of the tile], zero for
  // r16 >= G and past the last key.
  f32x4_t acc[2];
  acc[0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  acc[1] = acc[0];
  const float* prow = sc_lds + (int64_t)(r16 < G ? r16 : 0) * cap;
  uint16_t (*vtw)[VTS] = vt[wave];
  for (int64_t t0 = wave; t0 < ntile32; t0 += (int64_t)FNW * FPT) {
    if (t0 != wave) {
#pragma unroll
      for (int u = 0; u < FPT; ++u) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const int64_t rel = ((t0 + u * FNW) << 5) + vkey + 16 * m;
          vreg[u][m] = (rel < nrel && !(fresh && rel == srel)) ? ld16(vb + (lo + rel) * p.css) : make_uint4(0, 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < FPT; ++u) {
      const int64_t tb = (t0 + u * FNW) << 5;
      if (tb >= nrel) break;
      // stage the V tile: key rows of 32 dims (the new value at the new slot)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        uint4 v = vreg[u][m];
        if (fresh && tb + vkey + 16 * m == srel) v = *reinterpret_cast<const uint4*>(&vnew[8 * vsub]);
        uint2* dst = reinterpret_cast<uint2*>(&vtw[vkey + 16 * m][8 * vsub]);
        dst[0] = make_uint2(v.x, v.y);
        dst[1] = make_uint2(v.z, v.w);
      }
      const int64_t rel0 = tb + 8 * q4;
      uint32_t pw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t ra = rel0 + 2 * e;
        const float pa = (r16 < G && ra < nrel) ? prow[ra] : 0.f;        // exact bf16 values
        const float pb = (r16 < G && ra + 1 < nrel) ? prow[ra + 1] : 0.f;
        pw[e] = (__float_as_uint(pa) >> 16) | (__float_as_uint(pb) & 0xffff0000u);
      }
      const uint4 pa4 = make_uint4(pw[0], pw[1], pw[2], pw[3]);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        uint32_t bw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          bw[e] = (uint32_t)vtw[8 * q4 + 2 * e][16 * j + r16] | ((uint32_t)vtw[8 * q4 + 2 * e + 1][16 * j + r16] << 16);
        acc[j] = mfma16x16x32(pa4, make_uint4(bw[0], bw[1], bw[2], bw[3]), acc[j]);
      }
    }
  }
  // C rows 4 q4 + e are heads; add the waves' partial outputs through LDS
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int g = 4 * q4 + e;
    if (g < G) {
#pragma unroll
      for (int j = 0; j < 2; ++j) outp[wave][g][16 * j + r16] = acc[j][e];
    }
  }
  __syncthreads();
  for (int i = tid; i < G * FDC; i += FNT) {
    const int g = i / FDC, d = i % FDC;
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < FNW; ++w) t += outp[w][g][d];
    p.out[b * p.ldo_b + (int64_t)(h * G + g) * p.ldo_h + d0 + d] = (bf16_t)f2bf(t);
  }
}

// Score rows up to this many bytes per workgroup take the single-launch path
// (with the kernel's static LDS, at most 64 KiB per workgroup).
constexpr size_t kFusedScoreLds = 32 * 1024;

template <int D, int G>
hipError_t launch_attn(const AttnParams& p, int b, hipStream_t st) {
  constexpr int DC = D >= 32 ? 32 : D;
  // short rows: one fused launch (the whole score row of a head in LDS)
  const size_t lds = (size_t)G * p.s_cap * sizeof(float);
  if (lds <= kFusedScoreLds) {
    dim3 grid((unsigned)(b * p.nkv), (unsigned)(D / FDC));
    hipLaunchKernelGGL((attn_fused_kernel<D, G>), grid, dim3(FNT), lds, st, p);
    return hipGetLastError();
  }
  dim3 grid1((unsigned)p.splits, (unsigned)p.nkv, (unsigned)b);
  hipLaunchKernelGGL((attn_scores_kernel<D, G>), grid1, dim3(NT), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // (b, kv head) in x: the D/DC chunk workgroups of one head share an XCD
  // (workgroups are dealt round-robin over the 8 XCDs by linear id)
  dim3 grid2((unsigned)(b * p.nkv), (unsigned)(D / DC));
  hipLaunchKernelGGL((attn_pv_kernel<D, G, DC>), grid2, dim3(NT), 0, st, p);
  return hipGetLastError();
}

template <int D>
hipError_t launch_attn_g(const AttnParams& p, int g, int b, hipStream_t st) {
  switch (g) {
    case 1: return launch_attn<D, 1>(p, b, st);
    case 2: return launch_attn<D, 2>(p, b, st);
    case 4: return launch_attn<D, 4>(p, b, st);
    case 8: return launch_attn<D, 8>(p, b, st);
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
                   int64_t chunk, float sm_scale, float eps, void* stream) {
  EK_GUARD();
  if (b < 1 || b * n_kv > 0x7fffffff || n_kv < 1 || n_q < n_kv || n_q % n_kv || b > 65535)
    return ek_fail(hipErrorInvalidValue, "attn: bad batch or head counts");
  const int64_t g = n_q / n_kv;
  if (splits < 1 || splits > sp || chunk < 1 || g > gp)
    return ek_fail(hipErrorInvalidValue, "attn: splits/chunk exceed the workspace");
  if (score_ss < s_cap) return ek_fail(hipErrorInvalidValue, "attn: score scratch shorter than the cache");
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
  hipStream_t st = (hipStream_t)stream;
  switch (head_dim) {
    case 32: return launch_attn_g<32>(p, (int)g, (int)b, st);
    case 64: return launch_attn_g<64>(p, (int)g, (int)b, st);
    case 128: return launch_attn_g<128>(p, (int)g, (int)b, st);
    default: return ek_fail(hipErrorInvalidValue, "attn: head_dim must be 32, 64 or 128");
  }
}

}  // extern "C"
