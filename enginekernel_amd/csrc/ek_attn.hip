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
#include "ek_attn_impl.h"
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
  u.ll_ep = 0;
#ifdef EK_STEP_TRACE
  u.trace_lds = nullptr;
#endif
  eka::attn_unit<D, G>(u, lds);
}

// Score rows up to this many bytes per workgroup take the single-launch path
// (with the kernel's static LDS, at most 64 KiB per workgroup).
constexpr size_t kFusedScoreLds = 32 * 1024;

template <int D, int G>
hipError_t launch_attn(const AttnParams& p, int b, hipStream_t st) {
  constexpr int DC = D >= 32 ? 32 : D;
  // short rows: one fused launch (the whole score row of a head in LDS)
  if ((size_t)G * p.s_cap * sizeof(float) <= kFusedScoreLds) {
    dim3 grid((unsigned)(b * p.nkv), (unsigned)(D / eka::FDC));
    const size_t lds = eka::AttnLds<D, G>::bytes(p.s_cap);
    hipLaunchKernelGGL((attn_fused_kernel<D, G>), grid, dim3(eka::FNT), lds, st, p);
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
