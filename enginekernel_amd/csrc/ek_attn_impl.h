// The single-launch decode attention of one (batch row, kv head, 32 head
// dims) unit, as a device function over one 512-thread workgroup and an LDS
// region it is handed. ek_attn.hip launches it as a kernel of its own (one
// workgroup per unit); the persistent decode-step kernel (ek_step.hip) runs it
// as one phase of the step.
//
//   scores   per tile of 16 keys, S^T[16 x 16] = K_tile[16 x D] . Q^T[D x 16]
//            on the matrix cores (v_mfma_f32_16x16x32_bf16: bf16 products are
//            exact in fp32, sums are fp32), the G query heads in the first G
//            columns; scaled into an LDS row per head, with each lane's
//            running max; the lanes and waves merge the maxima into M.
//   softmax  e = exp(s - M) in place, L = sum of e (fixed order), then
//            p = bf16(e / L): one exp per score, spread over all threads
//            (the reference fallback's rounding point, engine/ek_model.py:475-488).
//   PV       per tile of 32 keys, O[16 x 16] += P[16 x 32] . V[32 x 16] per
//            16 head dims, the heads in the first G rows. V arrives as 16 B
//            per lane and is re-laid through a per-wave LDS tile into the B
//            operand (8 keys of one dim per lane), so the key sum happens
//            inside the MFMA. The waves' partial outputs are added through
//            LDS and rounded to bf16 once.
//
// In rope mode the unit norms/rotates its query heads and the new key (which
// stands in for the cache row at the new slot), takes the raw new value
// (likewise), and the writer unit stores both in the cache at its end. The first K
// and V tiles are loaded on entry, before the q/k/v heads are awaited and
// before the QK-norm/RoPE work, so both overlap the work before their use.
//
// MFMA lane layout (16x16x32): lane l = r + 16 q (r < 16, q < 4) holds
// A[row r][k = 8q .. 8q+7], B[k = 8q .. 8q+7][col r] and C[rows 4q .. 4q+3][col r].

#pragma once

#include "ek_common.h"

namespace eka {

// QK-norm + rotate-half RoPE of one head (one wave); writes the bf16-valued
// result as fp32 to `dst` (LDS) and, if `gdst`, as bf16 to global memory.
template <int D, bool F32 = true>
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
  ss = wave_sum_dpp(ss);
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
    if constexpr (F32) dst[d] = o;
    if (gdst) gdst[d] = (bf16_t)f2bf(o);
  }
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int FNT = 512;            // threads of the unit's workgroup
constexpr int FNW = FNT / EK_WAVE;
constexpr int FTU = 4;              // default 16-key score tiles in flight per wave
constexpr int FPT = 2;              // default 32-key PV tiles in flight per wave
constexpr int FDC = 32;             // head dims per unit
constexpr int VTS = FDC + 4;        // LDS row of a staged V tile (bf16; 72 B keeps reads conflict-free)

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

__device__ __forceinline__ f32x4_t mfma16x16x32(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

struct AttnUnit {
  // rope == 0: q heads already rotated, head g at qh + g * q_stride.
  // rope != 0: raw heads of the qkv row: q head g at qh + g * q_stride, the
  // new key at kh, the new value at vh; cr/sr the cos/sin row.
  const bf16_t* qh; int64_t q_stride;
  const bf16_t* kh; const bf16_t* vh;
  int rope;
  const bf16_t* qn; const bf16_t* kn; const bf16_t* cr; const bf16_t* sr;
  float eps, sm_scale;
  bf16_t* kc; bf16_t* vc; int64_t css;   // this (b, kv head)'s cache rows
  int64_t cap;                           // LDS score row length (>= hi - lo)
  int64_t lo, hi;                        // keys attended: [lo, hi); new slot hi - 1 in rope mode
  bool writer;                           // stores the new key/value at slot hi - 1
  int d0;                                // first head dim of this unit
  bf16_t* out; int64_t out_stride;       // out[g * out_stride + d0 + d]
  // When set, the output goes instead to dense 8-byte words of four bf16 at
  // ll_out[(g * out_stride + d0 + d) / 4] (dw_put: device scope, read by
  // other workgroups of the same launch, which poll for them)
  unsigned long long* ll_out;
#ifdef EK_STEP_TRACE
  int64_t* trace_lds;                    // per-stage timestamps of this unit, in LDS (trace builds)
#endif
};

#ifdef EK_STEP_TRACE
#define EK_ATTN_MARK(ev) do { if (threadIdx.x == 0 && a.trace_lds) a.trace_lds[ev] = wall_clock64(); } while (0)
#else
#define EK_ATTN_MARK(ev) do { } while (0)
#endif

__host__ __device__ constexpr size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }

// LDS layout of one unit: the score rows, then the fixed-size arrays
template <int D, int G>
struct AttnLds {
  // score rows of an odd stride: with a stride that is a multiple of the 32
  // LDS banks, the G rows' same-key entries would share a bank
  static __host__ __device__ constexpr int64_t stride(int64_t cap) { return cap | 1; }
  static __host__ __device__ constexpr size_t scores(int64_t cap) { return align16((size_t)G * stride(cap) * 4); }
  static constexpr size_t QS = align16((size_t)G * D * 4);
  static constexpr size_t KNEW = align16((size_t)D * 4);
  static constexpr size_t VNEW = align16((size_t)FDC * 2);
  static constexpr size_t ST = align16((size_t)FNW * 8 * 4);
  static constexpr size_t VT = align16((size_t)FNW * 32 * VTS * 2);
  static constexpr size_t OUTP = align16((size_t)FNW * G * FDC * 4);
  static constexpr size_t KNB = align16((size_t)D * 2);
  static __host__ __device__ constexpr size_t bytes(int64_t cap) {
    return scores(cap) + QS + KNEW + VNEW + 2 * ST + VT + OUTP + KNB;
  }
};

struct NoPre {
  __device__ bool operator()() const { return true; }
};

// `pre` runs once the first K and V tiles are in flight and before the q/k/v
// heads are read (the persistent step waits there for them); false abandons
// the unit.
template <int D, int G, int FTU = eka::FTU, int FPT = eka::FPT, typename PRE = NoPre>
__device__ __forceinline__ bool attn_unit(const AttnUnit& a, unsigned char* lds, PRE pre = PRE()) {
  constexpr int KS = D / 32;   // 32-dim k-steps of a score tile
  static_assert(G <= 8 && D % 32 == 0, "tile shape");
  using L = AttnLds<D, G>;
  float* sc_lds = reinterpret_cast<float*>(lds);                       // [G][cap] by key - lo
  unsigned char* fx = lds + L::scores(a.cap);
  bf16_t (*qs)[D] = reinterpret_cast<bf16_t (*)[D]>(fx);   // the q heads, normed and rotated (bf16)
  float* knew = reinterpret_cast<float*>(fx + L::QS);
  uint16_t* vnew = reinterpret_cast<uint16_t*>(fx + L::QS + L::KNEW);
  float (*stm)[8] = reinterpret_cast<float (*)[8]>(fx + L::QS + L::KNEW + L::VNEW);
  float (*stl)[8] = reinterpret_cast<float (*)[8]>(fx + L::QS + L::KNEW + L::VNEW + L::ST);
  uint16_t (*vt)[32][VTS] = reinterpret_cast<uint16_t (*)[32][VTS]>(fx + L::QS + L::KNEW + L::VNEW + 2 * L::ST);
  float (*outp)[G][FDC] = reinterpret_cast<float (*)[G][FDC]>(fx + L::QS + L::KNEW + L::VNEW + 2 * L::ST + L::VT);
  bf16_t* knew_bf = reinterpret_cast<bf16_t*>(fx + L::QS + L::KNEW + L::VNEW + 2 * L::ST + L::VT + L::OUTP);

  // the thread index is made opaque here so that the per-lane offsets below
  // are computed per call rather than hoisted out of a caller's loop (where
  // they would stay live, in registers, across everything else it does)
  int tid_o = threadIdx.x;
  __asm__ volatile("" : "+v"(tid_o));
  const int tid = tid_o, lane = tid & 63, wave = wave_id();
  const int r16 = lane & 15, q4 = lane >> 4;
  const int64_t cap = a.cap;
  const int64_t lo = a.lo, hi = a.hi;
  const int64_t nrel = hi > lo ? hi - lo : 0;   // keys attended
  const int64_t slot = hi - 1;
  const bool fresh = a.rope && slot >= lo;      // the new key/value come from the qkv row
  const int64_t srel = slot - lo;
  const int d0 = a.d0;

  // first K tiles in flight before any other work: lane holds key row r16
  // of the tile, dims 32 i + 8 q4 .. +7
  const bf16_t* kb = a.kc + 8 * q4;
  const int64_t ntile = (nrel + 15) >> 4;
  uint4 kt[FTU][KS];
#pragma unroll
  for (int u = 0; u < FTU; ++u) {
    const int64_t rel = ((int64_t)(wave + u * FNW) << 4) + r16;
#pragma unroll
    for (int i = 0; i < KS; ++i)
      kt[u][i] = rel < nrel ? ld16(kb + (lo + rel) * a.css + 32 * i) : make_uint4(0, 0, 0, 0);
  }

  // first V tiles in flight: 16 B chunks c = lane + 64 m of the 32 x 32 tile,
  // key c / 4, dims 8 (c % 4) .. +7
  const int vkey = lane >> 2, vsub = lane & 3;
  const bf16_t* vb = a.vc + d0 + 8 * vsub;
  const int64_t ntile32 = (nrel + 31) >> 5;
  uint4 vreg[FPT][2];
#pragma unroll
  for (int u = 0; u < FPT; ++u) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int64_t rel = ((int64_t)(wave + u * FNW) << 5) + vkey + 16 * m;
      vreg[u][m] = (rel < nrel && !(fresh && rel == srel)) ? ld16(vb + (lo + rel) * a.css) : make_uint4(0, 0, 0, 0);
    }
  }
  // the writer unit stores the new key (normed, rotated) and value at the
  // new slot once its own work is done: a store issued earlier would hold up
  // the memory waits that follow it
  auto store_new_row = [&]() {
    if (a.rope && a.writer && slot >= 0 && wave == FNW - 1) {
      bf16_t* kdst = a.kc + slot * a.css;
      bf16_t* vdst = a.vc + slot * a.css;
      for (int d = lane; d < D; d += EK_WAVE) {
        kdst[d] = knew_bf[d];
        vdst[d] = a.vh[d];
      }
    }
  };
  if (!pre()) return false;
  EK_ATTN_MARK(15);

  if (a.rope) {
    const bool writer = a.writer && slot >= 0;
    const int units = G + ((fresh || writer) ? 1 : 0);
    for (int u = wave; u < units; u += FNW) {
      if (u < G) {
        head_norm_rope<D, false>(a.qh + u * a.q_stride, a.qn, a.cr, a.sr, a.eps, nullptr, qs[u]);
      } else {
        head_norm_rope<D>(a.kh, a.kn, a.cr, a.sr, a.eps, knew, knew_bf);
      }
    }
    if (fresh && tid < FDC) vnew[tid] = a.vh[d0 + tid];
  } else {
    for (int i = tid; i < G * D; i += FNT) qs[i / D][i % D] = a.qh[(i / D) * a.q_stride + i % D];
  }

  __syncthreads();
  EK_ATTN_MARK(16);

  // ---- scores. B operand = Q^T: q[g = r16][32 i + 8 q4 .. +7], zero for g >= G
  // (every lane reads a valid row and masks afterwards: a read under a lane
  // condition becomes a branch with its own wait, serialising the reads)
  uint4 qb[KS];
  const uint32_t qmask = r16 < G ? 0xffffffffu : 0u;
#pragma unroll
  for (int i = 0; i < KS; ++i) {
    const int g = r16 < G ? r16 : 0;
    const uint4 v = *reinterpret_cast<const uint4*>(&qs[g][32 * i + 8 * q4]);
    qb[i] = make_uint4(v.x & qmask, v.y & qmask, v.z & qmask, v.w & qmask);
  }
  EK_ATTN_MARK(20);
  // pass 1: scores into the LDS rows and each lane's running max (no
  // exponentials yet, no read under a lane condition)
  float mrun = -INFINITY;            // this lane's scores: head r16
  for (int64_t t0 = wave; t0 < ntile; t0 += (int64_t)FNW * FTU) {
    if (t0 != wave) {
#pragma unroll
      for (int u = 0; u < FTU; ++u) {
        const int64_t rel = ((t0 + u * FNW) << 4) + r16;
#pragma unroll
        for (int i = 0; i < KS; ++i)
          kt[u][i] = rel < nrel ? ld16(kb + (lo + rel) * a.css + 32 * i) : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < FTU; ++u) {
      const int64_t tb = (t0 + u * FNW) << 4;
      if (tb >= nrel) break;
      if (fresh && tb + r16 == srel) {   // the new key (packed bf16 in LDS), not the cache row
#pragma unroll
        for (int i = 0; i < KS; ++i) kt[u][i] = *reinterpret_cast<const uint4*>(&knew_bf[32 * i + 8 * q4]);
      }
      f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KS; ++i) c = mfma16x16x32(kt[u][i], qb[i], c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t rel = tb + 4 * q4 + e;
        const float sv = c[e] * a.sm_scale;
        const bool ok = r16 < G && rel < nrel;
        if (ok) sc_lds[(int64_t)r16 * L::stride(cap) + rel] = sv;
        mrun = ok ? fmaxf(mrun, sv) : mrun;
      }
    }
  }
  EK_ATTN_MARK(21);
  // row max: over the four lane rows of a head, then over the waves
  mrun = fmaxf(mrun, __shfl_xor(mrun, 16, EK_WAVE));
  mrun = fmaxf(mrun, __shfl_xor(mrun, 32, EK_WAVE));
  EK_ATTN_MARK(22);
  if (q4 == 0 && r16 < G) stm[wave][r16] = mrun;
  __syncthreads();
  EK_ATTN_MARK(17);
  // pass 2: e = exp(s - M) in place and its sum L (thread -> head tid % G,
  // keys tid / G + k FNT / G; the sum in a fixed order), then
  // p = bf16(e / L) -- the reference fallback's rounding point
  {
    const int g = tid % G;
    float M = stm[0][g];
#pragma unroll
    for (int w = 1; w < FNW; ++w) M = fmaxf(M, stm[w][g]);
    float* row = sc_lds + (int64_t)g * L::stride(cap);
    float lsum = 0.f;
    for (int64_t n = tid / G; n < nrel; n += FNT / G) {
      const float ev = expf(row[n] - M);
      row[n] = ev;
      lsum += ev;
    }
    // threads with the same head: lanes l, l + G, l + 2G, ... of each wave
#pragma unroll
    for (int o = G; o < EK_WAVE; o <<= 1) lsum += __shfl_xor(lsum, o, EK_WAVE);
    if (lane < G) stl[wave][lane] = lsum;
    __syncthreads();
    float Lsum = stl[0][g];
#pragma unroll
    for (int w = 1; w < FNW; ++w) Lsum += stl[w][g];
    for (int64_t n = tid / G; n < nrel; n += FNT / G) row[n] = rbf(row[n] / Lsum);
  }
  __syncthreads();
  EK_ATTN_MARK(18);

  // ---- PV. A operand = P: p[head r16][keys 8 q4 .. +7 of the tile], zero for
  // r16 >= G and past the last key.
  f32x4_t acc[2];
  acc[0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  acc[1] = acc[0];
  const float* prow = sc_lds + (int64_t)(r16 < G ? r16 : 0) * L::stride(cap);
  uint16_t (*vtw)[VTS] = vt[wave];
  for (int64_t t0 = wave; t0 < ntile32; t0 += (int64_t)FNW * FPT) {
    if (t0 != wave) {
#pragma unroll
      for (int u = 0; u < FPT; ++u) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const int64_t rel = ((t0 + u * FNW) << 5) + vkey + 16 * m;
          vreg[u][m] = (rel < nrel && !(fresh && rel == srel)) ? ld16(vb + (lo + rel) * a.css) : make_uint4(0, 0, 0, 0);
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
        // p values are exact bf16; reads are clamped to the last key and masked
        const int64_t ra = rel0 + 2 * e;
        const float pa = prow[ra < nrel ? ra : nrel - 1];
        const float pb = prow[ra + 1 < nrel ? ra + 1 : nrel - 1];
        const uint32_t ma = (r16 < G && ra < nrel) ? 0xffffu : 0u;
        const uint32_t mb = (r16 < G && ra + 1 < nrel) ? 0xffff0000u : 0u;
        pw[e] = ((__float_as_uint(pa) >> 16) & ma) | (__float_as_uint(pb) & mb);
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
  EK_ATTN_MARK(19);
  if (a.ll_out) {
    // a thread per pair of dims (32-bit halves of the words): half the sums
    // on each thread's path
    for (int i = tid; i < G * FDC / 2; i += FNT) {
      const int g = i / (FDC / 2), d = 2 * (i % (FDC / 2));
      float t0 = 0.f, t1 = 0.f;
#pragma unroll
      for (int w = 0; w < FNW; ++w) {
        const float2 v = *reinterpret_cast<const float2*>(&outp[w][g][d]);
        t0 += v.x;
        t1 += v.y;
      }
      dw_put1(reinterpret_cast<uint32_t*>(a.ll_out) + (g * a.out_stride + d0 + d) / 2, pack2(t0, t1));
    }
    store_new_row();
    return true;
  }
  for (int i = tid; i < G * FDC; i += FNT) {
    const int g = i / FDC, d = i % FDC;
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < FNW; ++w) t += outp[w][g][d];
    a.out[g * a.out_stride + d0 + d] = (bf16_t)f2bf(t);
  }
  store_new_row();
  return true;
}

}  // namespace eka
