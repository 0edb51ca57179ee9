// Decode-shaped projections for gfx950: y[m, n] = sum_k x[m, k] * W[n, k].
//
// Batch-1..8 decode is a pure weight stream (2 bytes of W per multiply-add
// per batch row), so the kernel is built around HBM: each wave owns RPW
// output rows, each lane streams 16-byte chunks of them (a wave reads 1 KiB
// of one row per load instruction, fully coalesced), all KPL chunks of a
// block are issued before any is consumed, and the fp32 partial sums are
// folded with a butterfly over the wave. No LDS staging of W: every byte of
// W is used exactly once, and its loads are marked non-temporal (ld16_nt),
// which streams them measurably faster (lm_head: 11% less time). The
// activation rows (x, at most 8 x K bf16) are staged once per workgroup in LDS.
//
// Prologues fuse the reference's small consumer kernels into the projection
// that follows them (the weight loads are issued first, so the prologue's
// latency hides under the HBM stream):
//   PRO_X          x as given                            (ek_kernels.py:1322 gemv)
//   PRO_NORM       RMSNorm(x) * w                        (:1031 rms_norm)
//   PRO_ADD_NORM   r = x (+) res; RMSNorm(r) * w          (:1045 add_rms_norm, :1220 norm_gemv)
//   PRO_PARTS      r = bf16(sum_s P_s) (+) res; norm      (:1296 add_rms_norm_parts)
//   PRO_EMBED      r = E[token]; norm; advance slot/len   (ek_model.py:375-382)
// Epilogues:
//   EPI_BF16       bf16 output
//   EPI_PARTS      fp32 split-K partials P[split, m, n]   (ek_kernels.py:1277 gemv_parts)
//   EPI_SWIGLU     gate row n and up row n+I in one wave,
//                  bf16(silu(bf16 g)) (x) bf16 u          (:1247 gemv_swiglu, :1062 silu_mul)
//   EPI_ARGMAX     bf16 logits -> first-index argmax over the vocabulary via
//                  per-workgroup partials and a last-arriving reduction, then
//                  the decode-step bookkeeping            (ek_model.py:490-493, engine.py:289-292)
// Rounding points are the reference fallback's: bf16 residual add, fp32
// norm statistics rounded to bf16 before the bf16 gain, fp32 accumulation
// rounded once to bf16.

#pragma once

#include "ek_common.h"

namespace ekg {

enum { PRO_X = 0, PRO_NORM = 1, PRO_ADD_NORM = 2, PRO_PARTS = 3, PRO_EMBED = 4 };
enum { EPI_BF16 = 0, EPI_PARTS = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };

constexpr int NWAVE = 4;                  // waves per workgroup
constexpr int NTHR = NWAVE * EK_WAVE;

struct GemvParams {
  const bf16_t* w; int64_t ldw;
  int64_t n;         // output rows (activations for SWIGLU)
  int64_t ks;        // reduction length handled by one blockIdx.y
  int m;             // batch rows (<= BM)
  // prologue inputs
  const bf16_t* x; int64_t ldx;
  const float* parts; int sk_in; int64_t parts_ss;     // parts[s * parts_ss + b * ks + e]
  const bf16_t* res; int64_t ldr;
  bf16_t* res_out; int64_t ldro;
  const bf16_t* nw; float eps;
  const int64_t* tokens; const bf16_t* embed; int64_t lde; int64_t vocab;
  int64_t* slot_t; int64_t* len_t;
  // outputs
  bf16_t* y; int64_t ldy;
  float* p_out;      // [gridDim.y][m][n]
  int64_t up_off;    // SWIGLU: first row of the up half
  // argmax partials, one (value, index) per workgroup and batch row
  float* am_val; int32_t* am_idx;
};

// The FMA kernel's prologue (one workgroup of NTHR threads per group of
// output rows, weights of a whole block already in flight): rows one after
// another, each thread's sum of squares folded with one barrier. At batch 1
// it is measured faster than the bulk form below (per-kernel batch-1 step
// 2.46 against 2.96 ms: the bulk form's second barrier and one-wave row
// statistics sit on the path after the weights land).
template <int PRO, int BM>
__device__ __forceinline__ void prologue_rows(const GemvParams& p, bf16_t* xs, float (*red)[BM]) {
  const int tid = threadIdx.x;
  const int64_t ks = p.ks;
  const int64_t nch = ks >> 3;
  const int64_t kbase = (int64_t)blockIdx.y * ks;
  if constexpr (PRO == PRO_X) {
    for (int b = 0; b < BM; ++b) {
      for (int64_t c = tid; c < nch; c += NTHR) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (b < p.m) v = ld16(p.x + b * p.ldx + kbase + c * 8);
        *reinterpret_cast<uint4*>(xs + b * ks + c * 8) = v;
      }
    }
    return;
  } else {
    // pass 1: r (the pre-norm row, bf16) into xs, sum of squares per row
    const bool writer = (blockIdx.x == 0 && blockIdx.y == 0);
    float ss[BM];
#pragma unroll
    for (int b = 0; b < BM; ++b) ss[b] = 0.f;
#pragma unroll
    for (int b = 0; b < BM; ++b) {
      if (b >= p.m) continue;
      const bf16_t* src = nullptr;
      if constexpr (PRO == PRO_EMBED) {
        int64_t t = p.tokens[b];
        t = t < 0 ? 0 : (t >= p.vocab ? p.vocab - 1 : t);
        src = p.embed + t * p.lde;
      }
      for (int64_t c = tid; c < nch; c += NTHR) {
        float r[8];
        if constexpr (PRO == PRO_EMBED) {
          unpack8(ld16(src + c * 8), r);
        } else if constexpr (PRO == PRO_NORM) {
          unpack8(ld16(p.x + b * p.ldx + c * 8), r);
        } else if constexpr (PRO == PRO_ADD_NORM) {
          float xv[8], rv[8];
          unpack8(ld16(p.x + b * p.ldx + c * 8), xv);
          unpack8(ld16(p.res + b * p.ldr + c * 8), rv);
#pragma unroll
          for (int j = 0; j < 8; ++j) r[j] = rbf(rv[j] + xv[j]);
        } else {  // PRO_PARTS
          float sum[8];
          const float* pp = p.parts + b * ks + c * 8;
          float4 a0 = *reinterpret_cast<const float4*>(pp);
          float4 a1 = *reinterpret_cast<const float4*>(pp + 4);
          sum[0] = a0.x; sum[1] = a0.y; sum[2] = a0.z; sum[3] = a0.w;
          sum[4] = a1.x; sum[5] = a1.y; sum[6] = a1.z; sum[7] = a1.w;
          for (int s = 1; s < p.sk_in; ++s) {
            const float* q = pp + s * p.parts_ss;
            float4 b0 = *reinterpret_cast<const float4*>(q);
            float4 b1 = *reinterpret_cast<const float4*>(q + 4);
            sum[0] += b0.x; sum[1] += b0.y; sum[2] += b0.z; sum[3] += b0.w;
            sum[4] += b1.x; sum[5] += b1.y; sum[6] += b1.z; sum[7] += b1.w;
          }
          float rv[8];
          unpack8(ld16(p.res + b * p.ldr + c * 8), rv);
#pragma unroll
          for (int j = 0; j < 8; ++j) r[j] = rbf(rv[j] + rbf(sum[j]));
        }
        uint4 pk = make_uint4(pack2(r[0], r[1]), pack2(r[2], r[3]), pack2(r[4], r[5]), pack2(r[6], r[7]));
        *reinterpret_cast<uint4*>(xs + b * ks + c * 8) = pk;
        if (PRO != PRO_NORM && writer && p.res_out)
          *reinterpret_cast<uint4*>(p.res_out + b * p.ldro + c * 8) = pk;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss[b] = fmaf(r[j], r[j], ss[b]);
      }
    }
    if constexpr (PRO == PRO_EMBED) {
      if (writer && tid == 0 && p.len_t) {
        int64_t len = *p.len_t;
        for (int b = 0; b < p.m; ++b) p.slot_t[b] = len;
        *p.len_t = len + 1;
      }
    }
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int b = 0; b < BM; ++b) {
      float v = wave_sum(ss[b]);
      if (lane == 0) red[wave][b] = v;
    }
    __syncthreads();
    float rstd[BM];
#pragma unroll
    for (int b = 0; b < BM; ++b) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < NWAVE; ++w) t += red[w][b];
      float mean = t / (float)ks;
      rstd[b] = 1.0f / sqrtf(mean + p.eps);
    }
    // pass 2: xn = bf16(w * bf16(r * rstd)); zero rows >= m
#pragma unroll
    for (int b = 0; b < BM; ++b) {
      for (int64_t c = tid; c < nch; c += NTHR) {
        uint4* dst = reinterpret_cast<uint4*>(xs + b * ks + c * 8);
        if (b >= p.m) { *dst = make_uint4(0, 0, 0, 0); continue; }
        float r[8], g[8];
        unpack8(*dst, r);
        unpack8(ld16(p.nw + c * 8), g);
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = rbf(g[j] * rbf(r[j] * rstd[b]));
        *dst = make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
      }
    }
  }
}


// ----------------------------------------------------------------------------
// prologue: xs[b * xld + e] (bf16) for b < BM, e < ks -- the matrix-core
// kernel's (2..8 rows; the FMA kernel takes prologue_rows above).
//
// The BM x ks/8 chunks of 8 elements are dealt out flat over the threads
// (job j -> row j / nch, chunk j % nch) and taken GJ jobs at a time with
// every load of the group issued before any is used, so a whole stage costs
// a few memory round trips rather than one per row. Addresses of jobs past
// the end are clamped to a valid chunk (read, never stored), so no load sits
// under a lane condition. The norm variants store the pre-norm row r first,
// then take each row's sum of squares from the stage (one wave per row) and
// normalise in place.
// ----------------------------------------------------------------------------
constexpr int GJ = 4;   // jobs per thread in flight

template <int PRO, int BM, int NT = NTHR>
__device__ __forceinline__ void prologue(const GemvParams& p, bf16_t* xs, int64_t xld, float (*red)[BM]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int64_t ks = p.ks;
  const int64_t nch = ks >> 3;
  const int64_t kbase = (int64_t)blockIdx.y * ks;
  const int64_t jobs = (int64_t)BM * nch;
  const bool writer = (blockIdx.x == 0 && blockIdx.y == 0);

  // pass 1: x (PRO_X) or the pre-norm row r into the stage
  for (int64_t j0 = tid; j0 < jobs; j0 += (int64_t)GJ * NT) {
    int bj[GJ];
    int64_t cj[GJ];
    bool ok[GJ];
#pragma unroll
    for (int g = 0; g < GJ; ++g) {
      int64_t j = j0 + (int64_t)g * NT;
      ok[g] = j < jobs;
      j = ok[g] ? j : jobs - 1;
      bj[g] = (int)(j / nch);
      cj[g] = j - (int64_t)bj[g] * nch;
      ok[g] = ok[g] && bj[g] < p.m;
    }
    // rows >= m read row 0 (zeroed below)
    int br[GJ];
#pragma unroll
    for (int g = 0; g < GJ; ++g) br[g] = bj[g] < p.m ? bj[g] : 0;
    uint4 out[GJ];
    if constexpr (PRO == PRO_X) {
      uint4 v[GJ];
#pragma unroll
      for (int g = 0; g < GJ; ++g) v[g] = ld16(p.x + br[g] * p.ldx + kbase + cj[g] * 8);
#pragma unroll
      for (int g = 0; g < GJ; ++g) out[g] = ok[g] ? v[g] : make_uint4(0, 0, 0, 0);
    } else if constexpr (PRO == PRO_NORM || PRO == PRO_EMBED) {
      uint4 v[GJ];
#pragma unroll
      for (int g = 0; g < GJ; ++g) {
        const bf16_t* src;
        if constexpr (PRO == PRO_EMBED) {
          int64_t t = p.tokens[br[g]];
          t = t < 0 ? 0 : (t >= p.vocab ? p.vocab - 1 : t);
          src = p.embed + t * p.lde;
        } else {
          src = p.x + br[g] * p.ldx;
        }
        v[g] = ld16(src + cj[g] * 8);
      }
#pragma unroll
      for (int g = 0; g < GJ; ++g) out[g] = ok[g] ? v[g] : make_uint4(0, 0, 0, 0);
    } else if constexpr (PRO == PRO_ADD_NORM) {
      uint4 xv[GJ], rv[GJ];
#pragma unroll
      for (int g = 0; g < GJ; ++g) {
        xv[g] = ld16(p.x + br[g] * p.ldx + cj[g] * 8);
        rv[g] = ld16(p.res + br[g] * p.ldr + cj[g] * 8);
      }
#pragma unroll
      for (int g = 0; g < GJ; ++g) {
        float a[8], r[8], o[8];
        unpack8(xv[g], a);
        unpack8(rv[g], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = rbf(r[e] + a[e]);
        out[g] = ok[g] ? make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]))
                       : make_uint4(0, 0, 0, 0);
      }
    } else {  // PRO_PARTS: r = bf16(res + bf16(sum_s parts_s)), two splits per round trip
      float sum[GJ][8];
      uint4 rv[GJ];
#pragma unroll
      for (int g = 0; g < GJ; ++g) {
        rv[g] = ld16(p.res + br[g] * p.ldr + cj[g] * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) sum[g][e] = 0.f;
      }
      for (int s0 = 0; s0 < p.sk_in; s0 += 2) {
        const bool two = s0 + 1 < p.sk_in;
        float4 a[GJ][2], b2[GJ][2];
#pragma unroll
        for (int g = 0; g < GJ; ++g) {
          const float* pp = p.parts + (int64_t)s0 * p.parts_ss + br[g] * ks + cj[g] * 8;
          const float* pq = two ? pp + p.parts_ss : pp;
          a[g][0] = *reinterpret_cast<const float4*>(pp);
          a[g][1] = *reinterpret_cast<const float4*>(pp + 4);
          b2[g][0] = *reinterpret_cast<const float4*>(pq);
          b2[g][1] = *reinterpret_cast<const float4*>(pq + 4);
        }
#pragma unroll
        for (int g = 0; g < GJ; ++g) {
          sum[g][0] += a[g][0].x; sum[g][1] += a[g][0].y; sum[g][2] += a[g][0].z; sum[g][3] += a[g][0].w;
          sum[g][4] += a[g][1].x; sum[g][5] += a[g][1].y; sum[g][6] += a[g][1].z; sum[g][7] += a[g][1].w;
          if (two) {
            sum[g][0] += b2[g][0].x; sum[g][1] += b2[g][0].y; sum[g][2] += b2[g][0].z; sum[g][3] += b2[g][0].w;
            sum[g][4] += b2[g][1].x; sum[g][5] += b2[g][1].y; sum[g][6] += b2[g][1].z; sum[g][7] += b2[g][1].w;
          }
        }
      }
#pragma unroll
      for (int g = 0; g < GJ; ++g) {
        float r[8], o[8];
        unpack8(rv[g], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = rbf(r[e] + rbf(sum[g][e]));
        out[g] = ok[g] ? make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]))
                       : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int g = 0; g < GJ; ++g) {
      if (j0 + (int64_t)g * NT >= jobs) continue;
      *reinterpret_cast<uint4*>(xs + bj[g] * xld + cj[g] * 8) = out[g];
      if (PRO != PRO_X && PRO != PRO_NORM && writer && p.res_out && ok[g])
        *reinterpret_cast<uint4*>(p.res_out + bj[g] * p.ldro + cj[g] * 8) = out[g];
    }
  }
  if constexpr (PRO == PRO_X) return;

  if constexpr (PRO == PRO_EMBED) {
    if (writer && tid == 0 && p.len_t) {
      int64_t len = *p.len_t;
      for (int b = 0; b < p.m; ++b) p.slot_t[b] = len;
      *p.len_t = len + 1;
    }
  }
  __syncthreads();
  // row statistics from the stage: wave w takes rows w, w + NT/64, ...
  for (int b = wave; b < BM; b += NT / EK_WAVE) {
    float ss = 0.f;
    for (int64_t c = lane; c < nch; c += EK_WAVE) {
      float r[8];
      unpack8(*reinterpret_cast<const uint4*>(xs + b * xld + c * 8), r);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(r[e], r[e], ss);
    }
    ss = wave_sum(ss);
    if (lane == 0) red[0][b] = ss;
  }
  __syncthreads();
  float rstd[BM];
#pragma unroll
  for (int b = 0; b < BM; ++b) rstd[b] = 1.0f / sqrtf(red[0][b] / (float)ks + p.eps);
  // pass 2: xn = bf16(w * bf16(r * rstd)); rows >= m stay zero
  for (int64_t j = tid; j < jobs; j += NT) {
    const int b = (int)(j / nch);
    const int64_t c = j - (int64_t)b * nch;
    if (b >= p.m) continue;
    uint4* dst = reinterpret_cast<uint4*>(xs + b * xld + c * 8);
    float r[8], g[8], o[8];
    unpack8(*dst, r);
    unpack8(ld16(p.nw + c * 8), g);
    float rs = rstd[0];
#pragma unroll
    for (int bb = 1; bb < BM; ++bb) rs = b == bb ? rstd[bb] : rs;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = rbf(g[e] * rbf(r[e] * rs));
    *dst = make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
  }
}

// ----------------------------------------------------------------------------
// the kernel
//
// Rows are dealt out in groups of NWAVE * RPW (RPW consecutive rows per
// wave). A workgroup handles groups blockIdx.x, blockIdx.x + gridDim.x, ...
// so a grid of a few workgroups per CU streams the whole matrix after one
// prologue. When a row fits one block of KPL chunks per lane (every decode
// shape), the loads of the next group are issued chunk by chunk as the
// current group's chunks are consumed, so the HBM stream never drains
// between groups.
// ----------------------------------------------------------------------------
template <int PRO, int EPI, int BM, int KPL, int RPW>
__global__ __launch_bounds__(NTHR) void gemv_kernel(GemvParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16_t* xs = reinterpret_cast<bf16_t*>(smem_raw);
  __shared__ float red[NWAVE][BM];
  constexpr int R2 = (EPI == EPI_SWIGLU) ? 2 * RPW : RPW;
  constexpr int ROWS = NWAVE * RPW;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t ks = p.ks;
  const int64_t nch = ks >> 3;
  const int64_t kbase = (int64_t)blockIdx.y * ks;
  const int64_t ngroups = (p.n + ROWS - 1) / ROWS;
  const bool one_block = nch <= (int64_t)KPL * EK_WAVE;

  // row r of this wave in group g (out-of-range rows read row 0; dropped)
  auto wrow = [&](int64_t g, int r) -> const bf16_t* {
    const int rr = (EPI == EPI_SWIGLU && r >= RPW) ? r - RPW : r;
    int64_t n = g * ROWS + wave * RPW + rr;
    if (n >= p.n) n = 0;
    if (EPI == EPI_SWIGLU && r >= RPW) n += p.up_off;
    return p.w + n * p.ldw + kbase;
  };

  float best_v[BM];
  int best_i[BM];
#pragma unroll
  for (int b = 0; b < BM; ++b) { best_v[b] = -INFINITY; best_i[b] = 0x7fffffff; }

  int64_t g = blockIdx.x;
  uint4 wv[R2][KPL];
  if (one_block && g < ngroups) {
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const int64_t c = j * EK_WAVE + lane;
#pragma unroll
      for (int r = 0; r < R2; ++r) wv[r][j] = (c < nch) ? ld16_nt(wrow(g, r) + c * 8) : make_uint4(0, 0, 0, 0);
    }
  }
  prologue_rows<PRO, BM>(p, xs, red);
  __syncthreads();

  for (; g < ngroups; g += gridDim.x) {
    const int64_t gn = g + gridDim.x;
    const bool more = gn < ngroups;
    float acc[R2][BM];
#pragma unroll
    for (int r = 0; r < R2; ++r)
#pragma unroll
      for (int b = 0; b < BM; ++b) acc[r][b] = 0.f;

    if (one_block) {
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int64_t c = j * EK_WAVE + lane;
        uint4 cur[R2];
#pragma unroll
        for (int r = 0; r < R2; ++r) cur[r] = wv[r][j];
        if (more && c < nch) {
#pragma unroll
          for (int r = 0; r < R2; ++r) wv[r][j] = ld16_nt(wrow(gn, r) + c * 8);
        }
        if (c < nch) {
#pragma unroll
          for (int b = 0; b < BM; ++b) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xs + b * ks + c * 8);
#pragma unroll
            for (int r = 0; r < R2; ++r) acc[r][b] = dot8_acc(cur[r], xv, acc[r][b]);
          }
        }
      }
    } else {
      for (int64_t cb = 0; cb < nch; cb += KPL * EK_WAVE) {
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
          const int64_t c = cb + j * EK_WAVE + lane;
#pragma unroll
          for (int r = 0; r < R2; ++r) wv[r][j] = (c < nch) ? ld16_nt(wrow(g, r) + c * 8) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < KPL; ++j) {
          const int64_t c = cb + j * EK_WAVE + lane;
          if (c < nch) {
#pragma unroll
            for (int b = 0; b < BM; ++b) {
              const uint4 xv = *reinterpret_cast<const uint4*>(xs + b * ks + c * 8);
#pragma unroll
              for (int r = 0; r < R2; ++r) acc[r][b] = dot8_acc(wv[r][j], xv, acc[r][b]);
            }
          }
        }
      }
    }

#pragma unroll
    for (int r = 0; r < R2; ++r)
#pragma unroll
      for (int b = 0; b < BM; ++b) acc[r][b] = wave_sum(acc[r][b]);

    const int64_t row0 = g * ROWS + wave * RPW;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int64_t n = row0 + r;
#pragma unroll
      for (int b = 0; b < BM; ++b) {
        if constexpr (EPI == EPI_ARGMAX) {
          // rows reach a wave in increasing order: strict > keeps the first max
          const float v = rbf(acc[r][b]);
          if (n < p.n && (v > best_v[b] || best_i[b] == 0x7fffffff)) { best_v[b] = v; best_i[b] = (int)n; }
        }
        if (lane != ((r * BM + b) & 63) || n >= p.n || b >= p.m) continue;
        if constexpr (EPI == EPI_BF16 || EPI == EPI_ARGMAX) {
          if (EPI == EPI_BF16 || p.y) p.y[b * p.ldy + n] = (bf16_t)f2bf(acc[r][b]);
        } else if constexpr (EPI == EPI_PARTS) {
          p.p_out[((int64_t)blockIdx.y * p.m + b) * p.n + n] = acc[r][b];
        } else {
          const float gt = rbf(acc[r][b]);
          const float u = rbf(acc[RPW + r][b]);
          const float s = rbf(gt / (1.0f + expf(-gt)));
          p.y[b * p.ldy + n] = (bf16_t)f2bf(s * u);
        }
      }
    }
  }

  if constexpr (EPI == EPI_ARGMAX) {
    // per-workgroup (value, index) partials; ek_argmax_reduce finishes
    __shared__ float wbv[NWAVE][BM];
    __shared__ int wbi[NWAVE][BM];
    if (lane == 0) {
#pragma unroll
      for (int b = 0; b < BM; ++b) { wbv[wave][b] = best_v[b]; wbi[wave][b] = best_i[b]; }
    }
    __syncthreads();
    if (threadIdx.x < (unsigned)p.m) {
      const int b = threadIdx.x;
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int w = 0; w < NWAVE; ++w) {
        const float v = wbv[w][b];
        const int i = wbi[w][b];
        if (i != 0x7fffffff && (bi == 0x7fffffff || v > bv || (v == bv && i < bi))) { bv = v; bi = i; }
      }
      p.am_val[(int64_t)blockIdx.x * p.m + b] = bv;
      p.am_idx[(int64_t)blockIdx.x * p.m + b] = bi;
    }
  }
}

// ----------------------------------------------------------------------------
// the matrix-core kernel, for 2..8 batch rows
//
// At 2..8 rows the FMA kernel above runs out of issue slots (each weight
// element costs a conversion and BM FMAs, each x element an LDS read per
// row). Here v_mfma_f32_4x4x4_16b_bf16 does the products. Its 64 lanes are
// 16 blocks of 4: lane l = 4 blk + j holds A[blk][row j][4 k], B[blk][4 k]
// [column j] and C[blk][rows 0..3][column j]. A tile is 4 weight rows; lane
// l loads 16 B of row j at k offset 8 blk of each 128-wide chunk, so one
// load instruction reads 256 contiguous bytes of each of the 4 rows (a
// pattern that streams HBM as well as whole 1 KiB rows do, where the 16x16
// MFMA layout's 64-byte row pieces reach only about 60% of that), and two
// MFMAs take its two halves. Block blk accumulates the k offsets 8 blk .. 8
// blk + 7 of every chunk; at the tile's end the 16 blocks are added with
// DPP row rotations and two cross-row shuffles, and lane (blk = e, j) holds
// output row e of column j. The B operand is the batch rows' 16 bytes at the
// same k from the LDS stage: columns 0..3 per MFMA, so 8 rows take two
// column groups. Batch columns >= BM repeat a real row; their outputs are
// dropped.
//
// The loads themselves are lane-contiguous (lanes 16 r .. 16 r + 15 read the
// 256 B of row r, the pattern the memory pipeline coalesces best: with rows
// interleaved over neighbouring lanes, as the MFMA layout has them, the
// same bytes stream markedly slower), and four ds_bpermute per load move
// piece blk of row j to lane 4 blk + j.
//
// Each wave streams whole tiles (no cross-wave reduction, no barrier after
// the prologue): tiles gw, gw + W, ... for wave gw of W. A ring of NB loads
// (per row tile) stays in flight: a slot is refilled right after its MFMAs
// with the chunk NB places ahead in the wave's sequence (the next tile's
// once this one runs out). NB divides the chunks per tile, so a tile always
// ends at the last slot of a ring round. The norm prologues run before the
// ring is filled (their loads would otherwise retire behind the weight
// loads, which complete in order); the plain-x stage runs after it.
// ----------------------------------------------------------------------------
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// threads of a matrix-core workgroup: 256 for the split-K partials (whose
// launches have the most tiles per CU: smaller workgroups stay co-resident),
// 512 otherwise (one stage of x serves more tiles)
__host__ __device__ constexpr int mfma_threads(int epi) { return epi == EPI_PARTS ? 256 : 512; }
constexpr int MT = 4;                    // weight rows per tile
constexpr int MCH = 128;                 // K per chunk (one load instruction)

__device__ __forceinline__ f32x4_t mfma4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f32x4_t c) {
  const s16x4_t a = __builtin_bit_cast(s16x4_t, make_uint2(a0, a1));
  const s16x4_t b = __builtin_bit_cast(s16x4_t, make_uint2(b0, b1));
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 0, 0, 0);
}

// the stage's row stride (elements): rows 64 B apart modulo 256 B, so the
// lanes of one k offset and different rows hit different banks
__host__ __device__ inline int64_t mfma_xld(int64_t ks) { return ks + 32; }

// sum over the 16 blocks of a wave (lanes with equal l % 4); every lane
// gets the total of its column
__device__ __forceinline__ float block_sum(float v) {
  v = dpp_plus<0x128>(v);   // row_ror:8
  v = dpp_plus<0x124>(v);   // row_ror:4
  v += __shfl_xor(v, 16, EK_WAVE);
  v += __shfl_xor(v, 32, EK_WAVE);
  return v;
}

template <int PRO, int EPI, int BM, int NB, int NT = mfma_threads(EPI)>
__global__ __launch_bounds__(NT) void gemv_mfma_kernel(GemvParams p) {
  constexpr int NWV = NT / EK_WAVE;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16_t* xs = reinterpret_cast<bf16_t*>(smem_raw);
  constexpr int RT = (EPI == EPI_SWIGLU) ? 2 : 1;   // gate and up tiles side by side
  constexpr int CG = BM > 4 ? 2 : 1;                // column groups of 4 batch rows
  __shared__ float red[NWV][BM];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int blk = lane >> 2, j4 = lane & 3;
  const int lrow = lane >> 4, lpc = lane & 15;      // row and 16-byte piece this lane loads
  const int src = (16 * j4 + blk) * 4;              // ds_bpermute source: row j4, piece blk
  const int64_t ks = p.ks;
  const int64_t xld = mfma_xld(ks);
  const int C = (int)(ks / MCH);                    // chunks per tile
  const int64_t ntiles = (p.n + MT - 1) / MT;
  const int64_t W = (int64_t)gridDim.x * NWV;
  const int64_t gw = (int64_t)blockIdx.x * NWV + wave;
  const int64_t my_tiles = gw < ntiles ? (ntiles - 1 - gw) / W + 1 : 0;
  const int64_t rounds = my_tiles * (C / NB);
  const bf16_t* wbase = p.w + (int64_t)blockIdx.y * ks + lpc * 8;

  // the weight row this lane loads in tile j (of this wave) and row tile t;
  // rows past the end re-read the last row (their outputs are dropped)
  auto wrow = [&](int64_t j, int t) -> const bf16_t* {
    int64_t n = (gw + j * W) * MT + lrow;
    n = n < p.n ? n : p.n - 1;
    if (t == 1) n += p.up_off;
    return wbase + n * p.ldw;
  };

  if constexpr (PRO != PRO_X) prologue<PRO, BM, NT>(p, xs, xld, red);
  // the first round in the order the ring refills it (slot-major), so each
  // slot's wait counts the same loads behind it as in every later round
  uint4 ring[RT][NB];
  if (rounds > 0) {
    const bf16_t* w0[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) w0[t] = wrow(0, t);
#pragma unroll
    for (int u = 0; u < NB; ++u)
#pragma unroll
      for (int t = 0; t < RT; ++t) ring[t][u] = ld16_nt(w0[t] + u * MCH);
  }
  if constexpr (PRO == PRO_X) prologue<PRO, BM, NT>(p, xs, xld, red);
  __syncthreads();

  const bf16_t* xr[CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) xr[c] = xs + ((4 * c + j4) & (BM - 1)) * xld + blk * 8;
  float best_v[CG];
  int best_i[CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) { best_v[c] = -INFINITY; best_i[c] = 0x7fffffff; }
  f32x4_t acc[RT][CG];
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int c = 0; c < CG; ++c) acc[t][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int R = C / NB;   // ring rounds per tile
  for (int64_t rd = 0; rd < rounds; ++rd) {
    const int64_t j = rd / R;
    const int c0 = (int)(rd - j * R) * NB;
    const int64_t rn = rd + 1 < rounds ? rd + 1 : rd;   // the last round re-reads itself
    const int64_t jn = rn / R;
    const int cn0 = (int)(rn - jn * R) * NB;
    const bf16_t* wn[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) wn[t] = wrow(jn, t) + cn0 * MCH;
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      uint4 xv[CG];
#pragma unroll
      for (int c = 0; c < CG; ++c) xv[c] = *reinterpret_cast<const uint4*>(xr[c] + (c0 + u) * MCH);
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        const uint4 g = ring[t][u];
        uint4 w;
        w.x = __builtin_amdgcn_ds_bpermute(src, (int)g.x);
        w.y = __builtin_amdgcn_ds_bpermute(src, (int)g.y);
        w.z = __builtin_amdgcn_ds_bpermute(src, (int)g.z);
        w.w = __builtin_amdgcn_ds_bpermute(src, (int)g.w);
        ring[t][u] = ld16_nt(wn[t] + u * MCH);
#pragma unroll
        for (int c = 0; c < CG; ++c) {
          acc[t][c] = mfma4(w.x, w.y, xv[c].x, xv[c].y, acc[t][c]);
          acc[t][c] = mfma4(w.z, w.w, xv[c].z, xv[c].w, acc[t][c]);
        }
      }
      // keep each slot's refill where it is: the scheduler would otherwise
      // sink all refills below the round's MFMAs and drain the ring
      __builtin_amdgcn_sched_barrier(0);
    }
    if (c0 + NB < C) continue;

    // ---- tile end: lane (blk = e < 4, j) takes row e of batch columns j, 4 + j
    const int64_t n0 = (gw + j * W) * MT;
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      float v[RT];
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        float mine = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float tot = block_sum(acc[t][c][e]);
          mine = blk == e ? tot : mine;
        }
        v[t] = mine;
        acc[t][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
      const int64_t n = n0 + blk;
      const int b = 4 * c + j4;
      if (blk < 4 && n < p.n && b < p.m) {
        if constexpr (EPI == EPI_BF16) {
          p.y[b * p.ldy + n] = (bf16_t)f2bf(v[0]);
        } else if constexpr (EPI == EPI_PARTS) {
          p.p_out[((int64_t)blockIdx.y * p.m + b) * p.n + n] = v[0];
        } else if constexpr (EPI == EPI_SWIGLU) {
          const float gt = rbf(v[0]);
          const float u = rbf(v[RT - 1]);
          const float sl = rbf(gt / (1.0f + expf(-gt)));
          p.y[b * p.ldy + n] = (bf16_t)f2bf(sl * u);
        } else {   // EPI_ARGMAX: this lane's rows of batch row b arrive in increasing order
          const float lv = rbf(v[0]);
          if (p.y) p.y[b * p.ldy + n] = (bf16_t)f2bf(lv);
          if (lv > best_v[c] || best_i[c] == 0x7fffffff) { best_v[c] = lv; best_i[c] = (int)n; }
        }
      }
    }
  }

  if constexpr (EPI == EPI_ARGMAX) {
    // per-workgroup (value, index) partials: batch row b's candidates are
    // lanes blk < 4, j = b % 4, column group b / 4 of every wave;
    // ek_argmax_reduce finishes
    __shared__ float abv[NWV][16][CG];
    __shared__ int abi[NWV][16][CG];
    if (lane < 16) {
#pragma unroll
      for (int c = 0; c < CG; ++c) { abv[wave][lane][c] = best_v[c]; abi[wave][lane][c] = best_i[c]; }
    }
    __syncthreads();
    if (threadIdx.x < (unsigned)p.m) {
      const int b = threadIdx.x;
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int w = 0; w < NWV; ++w)
        for (int e = 0; e < 4; ++e) {
          const float vv = abv[w][4 * e + (b & 3)][b >> 2];
          const int ii = abi[w][4 * e + (b & 3)][b >> 2];
          if (ii != 0x7fffffff && (bi == 0x7fffffff || vv > bv || (vv == bv && ii < bi))) { bv = vv; bi = ii; }
        }
      p.am_val[(int64_t)blockIdx.x * p.m + b] = bv;
      p.am_idx[(int64_t)blockIdx.x * p.m + b] = bi;
    }
  }
}

// ----------------------------------------------------------------------------
// per-(prologue, epilogue) launchers, each defined in its own translation unit
// (ek_gemv_inst.hip compiled once per pair)
// ----------------------------------------------------------------------------
template <int PRO, int EPI>
hipError_t launch_pair(const GemvParams& p, int bm, int kpl, int rpw, dim3 grid, size_t lds, hipStream_t st);
template <int PRO, int EPI>
hipError_t launch_mfma_pair(const GemvParams& p, int bm, int nb, dim3 grid, size_t lds, hipStream_t st);

// the pairs that exist (the build compiles ek_gemv_inst.hip once for each)
#define EK_GEMV_PAIRS(X) \
  X(0, 0) X(0, 1) X(0, 2) X(0, 3) X(1, 0) X(1, 2) X(2, 0) X(2, 2) X(3, 0) X(3, 2) X(3, 3) X(4, 0)
#define EK_DECL_PAIR(PR, EP)                                                                \
  template <>                                                                               \
  hipError_t launch_pair<PR, EP>(const GemvParams&, int, int, int, dim3, size_t, hipStream_t); \
  template <>                                                                               \
  hipError_t launch_mfma_pair<PR, EP>(const GemvParams&, int, int, dim3, size_t, hipStream_t);
EK_GEMV_PAIRS(EK_DECL_PAIR)
#undef EK_DECL_PAIR

}  // namespace ekg
