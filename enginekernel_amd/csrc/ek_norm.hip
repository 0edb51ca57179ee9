// Row-wise kernels of the decode step that are not fused into a projection:
// RMSNorm (K1), add+RMSNorm (K2), split-K-sum+add+RMSNorm (K11), SiLU*up
// (K3) and per-head QK-norm + RoPE + KV-cache write (K6). The decode graph
// uses the fused forms (ek_gemv.hip, ek_attn.hip); these serve the
// reference's call surface and the prefill.
//
// Rounding points follow the reference torch fallbacks
// (engine/ek_kernels.py:1025-1028, 1047-1049, 1064-1066, 1119-1136).

#include "ek_common.h"
#include "ek_abi_internal.h"
#include "ek_hip.h"

namespace {

constexpr int NT = 256;

// one workgroup per row; MODE 0 = norm, 1 = add+norm, 2 = parts-sum+add+norm.
// A thread owns chunks tid, tid + NT, ... (8 elements each, at most CPT of
// them: rows up to CPT * NT * 8 elements). Every load of the row -- inputs,
// residual, partials, gain -- is issued before any is used, and the row
// stays in registers between the statistics and the output, so the launch
// costs about two memory round trips.
constexpr int CPT = 4;

template <int MODE>
__global__ __launch_bounds__(NT) void row_norm_kernel(const bf16_t* __restrict__ x, int64_t ldx,
                                                      const float* __restrict__ parts, int sk, int64_t parts_ss,
                                                      bf16_t* residual, int64_t ldr,
                                                      const bf16_t* __restrict__ w, bf16_t* __restrict__ y,
                                                      int64_t ldy, int64_t n, float eps) {
  __shared__ float red[NT / EK_WAVE];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t nch = n >> 3;
  // chunk i of this thread, clamped (reads of a missing chunk are dropped)
  int64_t cc[CPT];
  bool ok[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = tid + (int64_t)i * NT;
    ok[i] = c < nch;
    cc[i] = ok[i] ? c : nch - 1;
  }
  uint4 gv[CPT], xv[CPT], rv[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    gv[i] = ld16(w + cc[i] * 8);
    if (MODE != 2) xv[i] = ld16(((MODE == 0) ? x : x) + row * ldx + cc[i] * 8);
    if (MODE != 0) rv[i] = ld16(residual + row * ldr + cc[i] * 8);
  }
  float r[CPT][8];
  if (MODE == 2) {
    float a[CPT][8];
#pragma unroll
    for (int i = 0; i < CPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) a[i][j] = 0.f;
#pragma unroll 2
    for (int s = 0; s < sk; ++s) {
      float4 p0[CPT], p1[CPT];
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const float* pp = parts + s * parts_ss + row * n + cc[i] * 8;
        p0[i] = *reinterpret_cast<const float4*>(pp);
        p1[i] = *reinterpret_cast<const float4*>(pp + 4);
      }
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        a[i][0] += p0[i].x; a[i][1] += p0[i].y; a[i][2] += p0[i].z; a[i][3] += p0[i].w;
        a[i][4] += p1[i].x; a[i][5] += p1[i].y; a[i][6] += p1[i].z; a[i][7] += p1[i].w;
      }
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      float rr[8];
      unpack8(rv[i], rr);
#pragma unroll
      for (int j = 0; j < 8; ++j) r[i][j] = rbf(rr[j] + rbf(a[i][j]));
    }
  } else if (MODE == 1) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      float aa[8], rr[8];
      unpack8(xv[i], aa);
      unpack8(rv[i], rr);
#pragma unroll
      for (int j = 0; j < 8; ++j) r[i][j] = rbf(rr[j] + aa[j]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < CPT; ++i) unpack8(xv[i], r[i]);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    if (!ok[i]) continue;
    if (MODE != 0)   // the row is read (above) and written (here) by this thread only
      *reinterpret_cast<uint4*>(residual + row * ldr + cc[i] * 8) =
          make_uint4(pack2(r[i][0], r[i][1]), pack2(r[i][2], r[i][3]), pack2(r[i][4], r[i][5]),
                     pack2(r[i][6], r[i][7]));
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(r[i][j], r[i][j], ss);
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < NT / EK_WAVE; ++i) t += red[i];
  const float rstd = 1.0f / sqrtf(t / (float)n + eps);
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    if (!ok[i]) continue;
    float g[8], o[8];
    unpack8(gv[i], g);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = rbf(g[j] * rbf(r[i][j] * rstd));
    *reinterpret_cast<uint4*>(y + row * ldy + cc[i] * 8) =
        make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
  }
}

__global__ __launch_bounds__(NT) void silu_mul_kernel(const bf16_t* __restrict__ gu, int64_t ldgu,
                                                      bf16_t* __restrict__ y, int64_t ldy, int64_t n) {
  const int64_t row = blockIdx.y;
  const int64_t c = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (c >= (n >> 3)) return;
  float g[8], u[8], o[8];
  unpack8(ld16(gu + row * ldgu + c * 8), g);
  unpack8(ld16(gu + row * ldgu + n + c * 8), u);
  for (int j = 0; j < 8; ++j) {
    const float s = rbf(g[j] / (1.0f + expf(-g[j])));
    o[j] = s * u[j];
  }
  *reinterpret_cast<uint4*>(y + row * ldy + c * 8) =
      make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
}

// One wave per (row, head): heads [0, nq) are q (rotated in place), [nq,
// nq+nkv) are k (rotated, written to the cache), the rest v (copied raw).
template <int D>
__global__ __launch_bounds__(NT) void qk_norm_rope_kv_kernel(
    bf16_t* qkv, int64_t ld_qkv, const bf16_t* __restrict__ qn, const bf16_t* __restrict__ kn,
    const bf16_t* __restrict__ cos, const bf16_t* __restrict__ sin, int64_t ld_cs,
    bf16_t* kc, bf16_t* vc, int64_t csb, int64_t csh, int64_t css, int64_t s_cap,
    const int64_t* __restrict__ slot_base, int64_t m, int nq, int nkv, int64_t m_per_batch, float eps) {
  constexpr int PER = D > 64 ? D / 64 : 1;
  constexpr int HALF = D / 2;
  const int lane = threadIdx.x & 63;
  const int nh = nq + 2 * nkv;
  const int64_t unit = (int64_t)blockIdx.x * (NT / EK_WAVE) + (threadIdx.x >> 6);
  if (unit >= m * nh) return;
  const int64_t row = unit / nh;
  const int h = (int)(unit % nh);
  bf16_t* x = qkv + row * ld_qkv + (int64_t)h * D;
  const int64_t bi = row / m_per_batch;
  const int64_t slot = slot_base[bi] + row % m_per_batch;
  const bool to_cache = h >= nq && slot >= 0 && slot < s_cap;
  if (h >= nq + nkv) {  // v: raw copy into the cache
    if (!to_cache) return;
    bf16_t* dst = vc + bi * csb + (int64_t)(h - nq - nkv) * csh + slot * css;
    for (int i = 0; i < PER; ++i) {
      const int d = lane + 64 * i;
      if (d < D) dst[d] = x[d];
    }
    return;
  }
  const bf16_t* w = h < nq ? qn : kn;
  float xv[PER], xp[PER];
  float ss = 0.f;
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
  float out[PER];
  for (int i = 0; i < PER; ++i) {
    const int d = lane + 64 * i;
    if (d >= D) continue;
    const int pd = d < HALF ? d + HALF : d - HALF;
    const float tn = rbf(bf2f(w[d]) * rbf(xv[i] * rstd));
    const float tp = rbf(bf2f(w[pd]) * rbf(xp[i] * rstd));
    const float rot = d < HALF ? -tp : tp;
    const int64_t crow = row * ld_cs;
    out[i] = rbf(rbf(tn * bf2f(cos[crow + d])) + rbf(rot * bf2f(sin[crow + d])));
  }
  if (h < nq) {
    for (int i = 0; i < PER; ++i) {
      const int d = lane + 64 * i;
      if (d < D) x[d] = (bf16_t)f2bf(out[i]);
    }
  } else if (to_cache) {
    bf16_t* dst = kc + bi * csb + (int64_t)(h - nq) * csh + slot * css;
    for (int i = 0; i < PER; ++i) {
      const int d = lane + 64 * i;
      if (d < D) dst[d] = (bf16_t)f2bf(out[i]);
    }
  }
}

bool bad_row(int64_t n, const void* a) {
  return n <= 0 || (n % 8) != 0 || (reinterpret_cast<uintptr_t>(a) & 15) != 0;
}

}  // namespace

extern "C" {

int ek_rms_norm(const void* x, const void* w, void* y, int64_t m, int64_t n, int64_t ldx, int64_t ldy,
                float eps, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 0x7fffffff || bad_row(n, x) || ldx % 8 || ldy % 8)
    return ek_fail(hipErrorInvalidValue, "rms_norm: rows must be a multiple of 8 elements, 16-byte aligned");
  if (n > (int64_t)CPT * NT * 8) return ek_fail(hipErrorInvalidValue, "rms_norm: row longer than 8192 elements");
  hipLaunchKernelGGL((row_norm_kernel<0>), dim3((unsigned)m), dim3(NT), 0, (hipStream_t)stream,
                     (const bf16_t*)x, ldx, (const float*)nullptr, 0, (int64_t)0, (bf16_t*)nullptr, (int64_t)0,
                     (const bf16_t*)w, (bf16_t*)y, ldy, n, eps);
  return hipGetLastError();
}

int ek_add_rms_norm(const void* x, void* residual, const void* w, void* y, int64_t m, int64_t n, int64_t ldx,
                    int64_t ldr, int64_t ldy, float eps, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 0x7fffffff || bad_row(n, x) || bad_row(n, residual) || ldx % 8 || ldr % 8 || ldy % 8)
    return ek_fail(hipErrorInvalidValue, "add_rms_norm: rows must be a multiple of 8 elements, 16-byte aligned");
  if (n > (int64_t)CPT * NT * 8) return ek_fail(hipErrorInvalidValue, "add_rms_norm: row longer than 8192 elements");
  hipLaunchKernelGGL((row_norm_kernel<1>), dim3((unsigned)m), dim3(NT), 0, (hipStream_t)stream,
                     (const bf16_t*)x, ldx, (const float*)nullptr, 0, (int64_t)0, (bf16_t*)residual, ldr,
                     (const bf16_t*)w, (bf16_t*)y, ldy, n, eps);
  return hipGetLastError();
}

int ek_add_rms_norm_parts(const float* parts, void* residual, const void* w, void* y, int64_t sk, int64_t m,
                          int64_t n, int64_t ldr, int64_t ldy, float eps, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 0x7fffffff || sk < 1 || bad_row(n, residual) || ldr % 8 || ldy % 8 || n > (int64_t)CPT * NT * 8)
    return ek_fail(hipErrorInvalidValue, "add_rms_norm_parts: bad shape (rows up to 8192 elements)");
  hipLaunchKernelGGL((row_norm_kernel<2>), dim3((unsigned)m), dim3(NT), 0, (hipStream_t)stream,
                     (const bf16_t*)nullptr, (int64_t)0, parts, (int)sk, m * n, (bf16_t*)residual, ldr,
                     (const bf16_t*)w, (bf16_t*)y, ldy, n, eps);
  return hipGetLastError();
}

int ek_silu_mul(const void* gu, void* y, int64_t m, int64_t n, int64_t ldgu, int64_t ldy, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 65535 || bad_row(n, gu) || ldgu % 8 || ldy % 8)
    return ek_fail(hipErrorInvalidValue, "silu_mul: bad shape");
  const int64_t nch = n / 8;
  dim3 grid((unsigned)((nch + NT - 1) / NT), (unsigned)m);
  hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(NT), 0, (hipStream_t)stream, (const bf16_t*)gu, ldgu,
                     (bf16_t*)y, ldy, n);
  return hipGetLastError();
}

int ek_qk_norm_rope_kv(void* qkv, const void* qn, const void* kn, const void* cos, const void* sin,
                       void* k_cache, void* v_cache, const int64_t* slot_base, int64_t m, int64_t ld_qkv,
                       int64_t ld_cs, int64_t n_q, int64_t n_kv, int64_t head_dim, int64_t csb, int64_t csh,
                       int64_t css, int64_t s_cap, int64_t m_per_batch, float eps, void* stream) {
  EK_GUARD();
  if (m < 1 || n_q < 1 || n_kv < 1 || m_per_batch < 1 || m % m_per_batch)
    return ek_fail(hipErrorInvalidValue, "qk_norm_rope_kv: bad shape");
  const int64_t units = m * (n_q + 2 * n_kv);
  const int64_t blocks = (units + 3) / 4;
  if (blocks > 0x7fffffff) return ek_fail(hipErrorInvalidValue, "qk_norm_rope_kv: too many rows");
  hipStream_t st = (hipStream_t)stream;
#define EK_QK(DD)                                                                                        \
  hipLaunchKernelGGL((qk_norm_rope_kv_kernel<DD>), dim3((unsigned)blocks), dim3(NT), 0, st, (bf16_t*)qkv, \
                     ld_qkv, (const bf16_t*)qn, (const bf16_t*)kn, (const bf16_t*)cos, (const bf16_t*)sin, \
                     ld_cs, (bf16_t*)k_cache, (bf16_t*)v_cache, csb, csh, css, s_cap, slot_base, m,      \
                     (int)n_q, (int)n_kv, m_per_batch, eps)
  switch (head_dim) {
    case 32: EK_QK(32); break;
    case 64: EK_QK(64); break;
    case 128: EK_QK(128); break;
    case 256: EK_QK(256); break;
    default: return ek_fail(hipErrorInvalidValue, "qk_norm_rope_kv: head_dim must be 32, 64, 128 or 256");
  }
#undef EK_QK
  return hipGetLastError();
}

}  // extern "C"
