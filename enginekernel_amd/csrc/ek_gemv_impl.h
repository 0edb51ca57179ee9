// Decode-shaped projections for gfx950: y[m, n] = sum_k x[m, k] * W[n, k].
//
// Batch-1..8 decode is a pure weight stream (2 bytes of W per multiply-add
// per batch row), so the kernel is built around HBM: each wave owns RPW
// output rows, each lane streams 16-byte chunks of them (a wave reads 1 KiB
// of one row per load instruction, fully coalesced), all KPL chunks of a
// block are issued before any is consumed, and the fp32 partial sums are
// folded with a butterfly over the wave. No LDS staging of W: every byte of
// W is used exactly once. The activation rows (x, at most 8 x K bf16) are
// staged once per workgroup in LDS.
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

// ----------------------------------------------------------------------------
// prologue: xs[b][e] (bf16) for b < BM, e < ks
// ----------------------------------------------------------------------------
template <int PRO, int BM>
__device__ __forceinline__ void prologue(const GemvParams& p, bf16_t* xs, float (*red)[BM]) {
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
      for (int r = 0; r < R2; ++r) wv[r][j] = (c < nch) ? ld16(wrow(g, r) + c * 8) : make_uint4(0, 0, 0, 0);
    }
  }
  prologue<PRO, BM>(p, xs, red);
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
          for (int r = 0; r < R2; ++r) wv[r][j] = ld16(wrow(gn, r) + c * 8);
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
          for (int r = 0; r < R2; ++r) wv[r][j] = (c < nch) ? ld16(wrow(g, r) + c * 8) : make_uint4(0, 0, 0, 0);
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
// per-(prologue, epilogue) launchers, each defined in its own translation unit
// (ek_gemv_inst.hip compiled once per pair)
// ----------------------------------------------------------------------------
template <int PRO, int EPI>
hipError_t launch_pair(const GemvParams& p, int bm, int kpl, int rpw, dim3 grid, size_t lds, hipStream_t st);

// the pairs that exist (the build compiles ek_gemv_inst.hip once for each)
#define EK_GEMV_PAIRS(X) \
  X(0, 0) X(0, 1) X(0, 2) X(0, 3) X(1, 0) X(1, 2) X(2, 0) X(2, 2) X(3, 0) X(3, 2) X(3, 3) X(4, 0)
#define EK_DECL_PAIR(PR, EP) \
  template <>              \
  hipError_t launch_pair<PR, EP>(const GemvParams&, int, int, int, dim3, size_t, hipStream_t);
EK_GEMV_PAIRS(EK_DECL_PAIR)
#undef EK_DECL_PAIR

}  // namespace ekg
