// Prefill attention for gfx950: causal GQA flash attention over the prompt's
// keys, on the matrix cores. The reference runs torch SDPA here
// (engine/ek_model.py:315-323) with the prompt's additive mask: key <= query
// and key >= start[b] (left padding, engine.py:541-570); query rows with no
// visible key (the padding rows) attend to themselves, as this build's torch
// path does, so that their K/V rows stay finite (no decode step reads them).
//
// The same kernel scores a speculative verify step (ek_attn_verify; the
// reference's flash_verify, engine/ek_kernels.py:1419, restated by its torch
// fallback attn_torch, :1451): the row's S query tokens then sit at cache
// positions q0[b] .. q0[b] + S - 1 (after the row's cached keys), query j
// sees keys [start[b], q0[b] + j].
//
// One workgroup per (batch row, kv head, block of 16 query tokens), one wave
// per query head of the group (G waves), so the G heads share each K/V tile:
//
//   S[16 tokens x 32 keys] = Q . K^T      two v_mfma_f32_16x16x32_bf16 chains
//                                         of D/32 steps (16 keys each)
//   online softmax per token row in fp32  (max, rescale, sum of exp)
//   O[16 x D] += P . V                    D/16 MFMAs, P rounded to bf16
//
// Operand layouts (lane l = r + 16 q): A[row r][k 8q..8q+7], B[k 8q..8q+7]
// [col r], C[rows 4q..4q+3][col r]. Q rows stay in registers (A operand);
// K tiles are stored row-major in LDS (the B operand of QK^T is 16 B of a key
// row); V tiles are stored transposed ([dim][key], so the B operand of PV is
// 16 B of one dim over 8 keys); P goes from the C layout of S to the A layout
// through a per-wave LDS tile. The next K/V tile is loaded into registers
// while the current one is consumed. O is divided by the row sum and rounded
// to bf16 once.

#include <cstring>

#include "ek_abi_internal.h"
#include "ek_attn_impl.h"
#include "ek_common.h"
#include "ek_hip.h"

namespace {

constexpr int QT = 16;   // query tokens per workgroup
constexpr int KB = 32;   // keys per tile

struct PrefillParams {
  const bf16_t* q; int64_t ldq;       // q of token t, head j: q + (b * S + t) * ldq + j * D
  const bf16_t* kc; const bf16_t* vc; int64_t csb, csh, css;
  const int32_t* start;               // [B] first visible key (left padding)
  const int64_t* q0;                  // [B] cache position of query token 0 (verify), or null (prefill: 0)
  bf16_t* out; int64_t ldo;           // out row (b * S + t), head j at j * D
  int64_t s;                          // query tokens per row (prefill: the padded prompt length)
  int64_t s_cap;                      // cache rows per (batch row, kv head)
  int nkv;
  float scale;
  // key splits (verify): split sp of a query block takes keys [k0 + sp * kchunk,
  // + kchunk) and writes its unnormalised output and (max, sum) to po / pml
  int nsplit;                         // 1: no split, the normalised output goes to out
  int64_t kchunk;                     // keys per split (a multiple of KB)
  float* po;                          // [nsplit][B*S][n_q][D]
  float* pml;                         // [nsplit][B*S][n_q][2]
  int nq;                             // query heads (n_kv * G)
};

template <int D, int G>
struct PfLds {
  static constexpr int KROW = D + 8;       // bf16 per K tile row (16 B pad)
  static constexpr int VROW = KB + 8;      // bf16 per transposed V row
  static constexpr int PROW = KB + 8;      // bf16 per P tile row
};

template <int D, int G>
__global__ __launch_bounds__(64 * G) void attn_prefill_kernel(PrefillParams p) {
  using L = PfLds<D, G>;
  constexpr int NTH = 64 * G;
  constexpr int DS = D / 32;               // MFMA steps of QK^T
  constexpr int DB = D / 16;               // 16-dim blocks of O
  constexpr int TCH = KB * D / 8;          // 16-byte chunks of one K (or V) tile
  constexpr int CPT = (TCH + NTH - 1) / NTH;
  __shared__ __align__(16) bf16_t ks[KB * L::KROW];
  __shared__ __align__(16) bf16_t vt[D * L::VROW];
  __shared__ __align__(16) bf16_t ps[G][QT * L::PROW];

  const int tid = threadIdx.x, lane = tid & 63, g = tid >> 6;
  const int r16 = lane & 15, q4 = lane >> 4;
  const int h = blockIdx.y, b = blockIdx.z;
  // query token t of this row sits at cache position qb + t; keys [0, kend)
  int64_t qb = p.q0 ? p.q0[b] : 0;
  qb = qb < 0 ? 0 : (qb > p.s_cap - p.s ? p.s_cap - p.s : qb);
  const int64_t kend = qb + p.s;
  const int qblk = (int)blockIdx.x / p.nsplit, sp = (int)blockIdx.x - qblk * p.nsplit;
  const int64_t t0 = (int64_t)qblk * QT;
  int64_t pad = p.start[b];
  pad = pad < 0 ? 0 : (pad > kend ? kend : pad);
  const int64_t tend = t0 + QT < p.s ? t0 + QT : p.s;   // tokens [t0, tend)
  // keys [k0, qb + tend): padding rows see only themselves, the others keys >= pad
  const int64_t kb0 = (qb + t0 < pad ? qb + t0 : pad) & ~(int64_t)(KB - 1);
  // this split's keys [k0, k1)
  const int64_t k0 = p.nsplit == 1 ? kb0 : kb0 + sp * p.kchunk;
  int64_t k1 = p.nsplit == 1 ? qb + tend : k0 + p.kchunk;
  k1 = k1 < qb + tend ? k1 : qb + tend;
  const int64_t ntile = k1 > k0 ? (k1 - k0 + KB - 1) / KB : 0;

  const bf16_t* kb = p.kc + b * p.csb + h * p.csh;
  const bf16_t* vb = p.vc + b * p.csb + h * p.csh;
  // tile chunk c: key c / (D / 8), 16-byte piece c % (D / 8); keys past the
  // last query's position re-read that key (masked below)
  auto tile_ld = [&](int64_t kt, uint4 (&kr)[CPT], uint4 (&vr)[CPT]) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      int c = tid + i * NTH;
      c = c < TCH ? c : TCH - 1;
      int64_t key = kt + c / (D / 8);
      key = key < kend ? key : kend - 1;
      kr[i] = ld16(kb + key * p.css + (c % (D / 8)) * 8);
      vr[i] = ld16(vb + key * p.css + (c % (D / 8)) * 8);
    }
  };

  // this wave's query rows (head h * G + g), A operand of QK^T
  uint4 qa[DS];
  {
    int64_t t = t0 + r16;
    t = t < p.s ? t : p.s - 1;
    const bf16_t* qrow = p.q + ((int64_t)b * p.s + t) * p.ldq + (int64_t)(h * G + g) * D;
#pragma unroll
    for (int i = 0; i < DS; ++i) qa[i] = ld16(qrow + 32 * i + 8 * q4);
  }
  uint4 kr[CPT], vr[CPT];
  tile_ld(k0, kr, vr);

  eka::f32x4_t o[DB];
#pragma unroll
  for (int j = 0; j < DB; ++j) o[j] = eka::f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_row[4], l_row[4];                // rows 4 q4 + e of this lane group
#pragma unroll
  for (int e = 0; e < 4; ++e) { m_row[e] = -1e30f; l_row[e] = 0.f; }
  bf16_t* pw = ps[g];

  for (int64_t it = 0; it < ntile; ++it) {
    const int64_t kt = k0 + it * KB;
    __syncthreads();   // the previous tile is no longer read
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * NTH;
      if (c >= TCH) continue;
      const int key = c / (D / 8), pc = c % (D / 8);
      *reinterpret_cast<uint4*>(ks + key * L::KROW + pc * 8) = kr[i];
      const uint32_t w4[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vt[(pc * 8 + 2 * e) * L::VROW + key] = (bf16_t)(w4[e] & 0xffffu);
        vt[(pc * 8 + 2 * e + 1) * L::VROW + key] = (bf16_t)(w4[e] >> 16);
      }
    }
    __syncthreads();
    if (it + 1 < ntile) tile_ld(kt + KB, kr, vr);   // in flight while this tile is consumed

    // S for keys kt + 16 kb + r16 (two blocks), rows 4 q4 + e
    float sv[2][4];
#pragma unroll
    for (int kbk = 0; kbk < 2; ++kbk) {
      eka::f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < DS; ++i) {
        const uint4 kf = *reinterpret_cast<const uint4*>(ks + (16 * kbk + r16) * L::KROW + 32 * i + 8 * q4);
        c = eka::mfma16x16x32(qa[i], kf, c);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t tok = qb + t0 + 4 * q4 + e;   // the query's cache position
        const int64_t key = kt + 16 * kbk + r16;
        const bool ok = key < k1 && ((key <= tok && key >= pad) || (tok < pad && key == tok));
        sv[kbk][e] = ok ? c[e] * p.scale : -1e30f;
      }
    }
    // online softmax: rows are spread over the 16 lanes of a lane group
    float scale_o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float mt = fmaxf(sv[0][e], sv[1][e]);
#pragma unroll
      for (int o2 = 1; o2 < 16; o2 <<= 1) mt = fmaxf(mt, __shfl_xor(mt, o2, EK_WAVE));
      const float mn = fmaxf(m_row[e], mt);
      float ls = 0.f;
#pragma unroll
      for (int kbk = 0; kbk < 2; ++kbk) {
        const float pv = sv[kbk][e] > -1e29f ? expf(sv[kbk][e] - mn) : 0.f;
        sv[kbk][e] = pv;
        ls += pv;
      }
#pragma unroll
      for (int o2 = 1; o2 < 16; o2 <<= 1) ls += __shfl_xor(ls, o2, EK_WAVE);
      scale_o[e] = expf(m_row[e] - mn);
      l_row[e] = l_row[e] * scale_o[e] + ls;
      m_row[e] = mn;
    }
#pragma unroll
    for (int j = 0; j < DB; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) o[j][e] *= scale_o[e];
    // P (bf16) from the C layout to the A layout through this wave's tile
#pragma unroll
    for (int kbk = 0; kbk < 2; ++kbk)
#pragma unroll
      for (int e = 0; e < 4; ++e) pw[(4 * q4 + e) * L::PROW + 16 * kbk + r16] = (bf16_t)f2bf(sv[kbk][e]);
    const uint4 pa = *reinterpret_cast<const uint4*>(pw + r16 * L::PROW + 8 * q4);
#pragma unroll
    for (int j = 0; j < DB; ++j) {
      const uint4 vf = *reinterpret_cast<const uint4*>(vt + (16 * j + r16) * L::VROW + 8 * q4);
      o[j] = eka::mfma16x16x32(pa, vf, o[j]);
    }
  }
  // out rows 4 q4 + e, dims 16 j + r16
  if (p.nsplit > 1) {   // this split's unnormalised rows and their (max, sum)
    const int64_t rows = (int64_t)gridDim.z * p.s;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t tok = t0 + 4 * q4 + e;
      if (tok >= p.s) continue;
      const int64_t idx = ((int64_t)sp * rows + (int64_t)b * p.s + tok) * p.nq + (h * G + g);
      float* prow = p.po + idx * D;
#pragma unroll
      for (int j = 0; j < DB; ++j) prow[16 * j + r16] = o[j][e];
      if (r16 == 0) {
        p.pml[2 * idx] = m_row[e];
        p.pml[2 * idx + 1] = l_row[e];
      }
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t tok = t0 + 4 * q4 + e;
    if (tok >= p.s) continue;
    const float inv = l_row[e] > 0.f ? 1.f / l_row[e] : 0.f;
    bf16_t* orow = p.out + ((int64_t)b * p.s + tok) * p.ldo + (int64_t)(h * G + g) * D;
#pragma unroll
    for (int j = 0; j < DB; ++j) orow[16 * j + r16] = (bf16_t)f2bf(o[j][e] * inv);
  }
}

// The key splits' rows combined: M = max m_s, out = sum_s o_s e^(m_s - M) /
// sum_s l_s e^(m_s - M), rounded to bf16 once. One workgroup of D threads
// per (query row, head).
template <int D>
__global__ __launch_bounds__(D) void attn_split_combine_kernel(PrefillParams p) {
  const int64_t row = blockIdx.x, head = blockIdx.y;
  const int64_t rows = (int64_t)gridDim.x;
  const int d = threadIdx.x;
  float mx = -1e30f;
  for (int s = 0; s < p.nsplit; ++s) mx = fmaxf(mx, p.pml[2 * ((s * rows + row) * p.nq + head)]);
  float l = 0.f, acc = 0.f;
  for (int s = 0; s < p.nsplit; ++s) {
    const int64_t idx = (s * rows + row) * p.nq + head;
    const float ms = p.pml[2 * idx];
    const float w = ms > -1e29f ? expf(ms - mx) : 0.f;
    l += p.pml[2 * idx + 1] * w;
    acc += p.po[idx * D + d] * w;
  }
  p.out[row * p.ldo + head * D + d] = (bf16_t)f2bf(l > 0.f ? acc / l : 0.f);
}

template <int D, int G>
hipError_t launch_prefill(const PrefillParams& p, int64_t b, hipStream_t st) {
  dim3 grid((unsigned)((p.s + QT - 1) / QT * p.nsplit), (unsigned)p.nkv, (unsigned)b);
  hipLaunchKernelGGL((attn_prefill_kernel<D, G>), grid, dim3(64 * G), 0, st, p);
  if (p.nsplit > 1) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((attn_split_combine_kernel<D>), dim3((unsigned)(b * p.s), (unsigned)p.nq), dim3(D), 0, st,
                       p);
  }
  return hipGetLastError();
}

template <int D>
hipError_t launch_prefill_g(const PrefillParams& p, int g, int64_t b, hipStream_t st) {
  switch (g) {
    case 1: return launch_prefill<D, 1>(p, b, st);
    case 2: return launch_prefill<D, 2>(p, b, st);
    case 4: return launch_prefill<D, 4>(p, b, st);
    case 8: return launch_prefill<D, 8>(p, b, st);
    default: return ek_fail(hipErrorInvalidValue, "attn_prefill: query heads per kv head must be 1, 2, 4 or 8");
  }
}

}  // namespace

namespace {

hipError_t attn_flash(const void* q, int64_t ldq, const void* k_cache, const void* v_cache, int64_t csb, int64_t csh,
                      int64_t css, int64_t s_cap, const int32_t* start, const int64_t* q0, void* out, int64_t ldo,
                      int64_t b, int64_t s, int64_t n_q, int64_t n_kv, int64_t head_dim, float sm_scale,
                      void* stream, float* part = nullptr, int64_t part_floats = 0, int64_t splits = 1) {
  if (b < 1 || b > 65535 || s < 1 || s > s_cap || n_kv < 1 || n_kv > 65535 || n_q % n_kv)
    return ek_fail(hipErrorInvalidValue, "attn_prefill/attn_verify: bad batch, length or head counts");
  if (splits < 1 || splits > 256 || (s + QT - 1) / QT * splits > 65535)
    return ek_fail(hipErrorInvalidValue, "attn_verify: splits must be 1..256");
  if (splits > 1 && (!part || part_floats < splits * b * s * n_q * (head_dim + 2)))
    return ek_fail(hipErrorInvalidValue, "attn_verify: the split workspace is too small");
  if (ldq % 8 || ldo % 8 || css % 8 || csh % 8 || csb % 8 || (reinterpret_cast<uintptr_t>(q) & 15) ||
      (reinterpret_cast<uintptr_t>(k_cache) & 15) || (reinterpret_cast<uintptr_t>(v_cache) & 15))
    return ek_fail(hipErrorInvalidValue, "attn_prefill/attn_verify: rows must be 16-byte aligned");
  PrefillParams p;
  memset(&p, 0, sizeof(p));
  p.q = (const bf16_t*)q; p.ldq = ldq;
  p.kc = (const bf16_t*)k_cache; p.vc = (const bf16_t*)v_cache; p.csb = csb; p.csh = csh; p.css = css;
  p.start = start; p.q0 = q0;
  p.out = (bf16_t*)out; p.ldo = ldo;
  p.s = s; p.s_cap = s_cap; p.nkv = (int)n_kv; p.scale = sm_scale;
  p.nq = (int)n_q;
  p.nsplit = (int)splits;
  // keys per split: the cache's rows spread evenly, in whole 32-key tiles
  p.kchunk = ((s_cap + splits - 1) / splits + KB - 1) / KB * KB;
  p.po = part;
  p.pml = part ? part + splits * b * s * n_q * head_dim : nullptr;
  hipStream_t st = (hipStream_t)stream;
  const int g = (int)(n_q / n_kv);
  switch (head_dim) {
    case 32: return launch_prefill_g<32>(p, g, b, st);
    case 64: return launch_prefill_g<64>(p, g, b, st);
    case 128: return launch_prefill_g<128>(p, g, b, st);
    default: return ek_fail(hipErrorInvalidValue, "attn_prefill/attn_verify: head_dim must be 32, 64 or 128");
  }
}

}  // namespace

extern "C" {

int ek_attn_prefill(const void* q, int64_t ldq, const void* k_cache, const void* v_cache, int64_t csb, int64_t csh,
                    int64_t css, int64_t s_cap, const int32_t* start, void* out, int64_t ldo, int64_t b, int64_t s,
                    int64_t n_q, int64_t n_kv, int64_t head_dim, float sm_scale, void* stream) {
  EK_GUARD();
  return attn_flash(q, ldq, k_cache, v_cache, csb, csh, css, s_cap, start, nullptr, out, ldo, b, s, n_q, n_kv,
                    head_dim, sm_scale, stream);
}

int ek_attn_verify(const void* q, int64_t ldq, const void* k_cache, const void* v_cache, int64_t csb, int64_t csh,
                   int64_t css, int64_t s_cap, const int32_t* start, const int64_t* len_b, void* out, int64_t ldo,
                   int64_t b, int64_t nq, int64_t n_q, int64_t n_kv, int64_t head_dim, float sm_scale,
                   float* part, int64_t part_floats, int64_t splits, void* stream) {
  EK_GUARD();
  if (!len_b) return ek_fail(hipErrorInvalidValue, "attn_verify: len_b is required");
  return attn_flash(q, ldq, k_cache, v_cache, csb, csh, css, s_cap, start, len_b, out, ldo, b, nq, n_q, n_kv,
                    head_dim, sm_scale, stream, part, part_floats, splits);
}

}  // extern "C"
