// C-ABI entry points of the GEMV family (kernel template: ek_gemv_impl.h;
// instantiations: ek_gemv_inst.hip, one object per prologue/epilogue pair).
//
// Every entry point takes two tuning arguments: rpw (output rows per wave,
// 1, 2 or 4; 0 = default) and blocks (the grid cap: workgroups loop over row
// groups, so a grid of a few workgroups per CU streams any height; 0 =
// default of 4 per CU). Both apply to the FMA kernel. Launches of 2..8 batch
// rows whose per-split K is a multiple of 128 take the matrix-core kernel
// (own tiles and grid; the tuning arguments are ignored) unless rpw < 0,
// which forces the FMA kernel. Neither changes results beyond fp32 summation
// order.

#include <cstring>

#include "ek_abi_internal.h"
#include "ek_gemv_impl.h"
#include "ek_hip.h"

namespace ekg {
namespace {

int pick_kpl(int64_t nch) {
  if (nch <= 64) return 1;
  if (nch == 320) return 5;    // K = 2560
  if (nch == 512) return 8;    // K = 4096
  if (nch == 1216) return 19;  // K = 9728
  return 4;
}

constexpr size_t kMaxLds = 48 * 1024;   // activation stage per workgroup (bytes)

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

int bm_for(int m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8; }

// compute units of the current device (cached per device index)
int cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cache[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// The matrix-core kernel's grid: at most eight waves per CU (all
// co-resident), every wave the same number of 4-row tiles.
int64_t mfma_grid(int64_t n, int epi) {
  const int64_t ntiles = (n + MT - 1) / MT;
  const int64_t cap = (int64_t)cu_count() * 8;     // waves
  const int64_t per = (ntiles + cap - 1) / cap;    // tiles per wave
  const int64_t wpg = mfma_threads(epi) / EK_WAVE;
  return (ntiles + per * wpg - 1) / (per * wpg);
}

// whether a launch takes the matrix-core kernel
bool use_mfma(int m, int64_t ks, int64_t rpw) { return m >= 2 && rpw >= 0 && ks % MCH == 0; }

// ring depth of the matrix-core kernel: the deepest that divides the chunks
// per tile, at most 20 loads in flight per wave (10 per row tile for the
// gate/up pairs)
int mfma_nb(int64_t chunks, bool pair) {
  static const int deep[] = {20, 19, 16, 10, 8, 5, 4};
  for (int nb : deep)
    if ((!pair || nb <= 10) && chunks % nb == 0) return nb;
  return 1;
}

// Launch one GEMV-family kernel. sk > 1 splits the reduction over
// blockIdx.y (EPI_PARTS only). The grid width used goes to *gx_out.
hipError_t run_gemv(int pro, int epi, GemvParams p, int64_t k, int64_t sk, int64_t rpw, int64_t blocks,
                    hipStream_t st, int64_t* gx_out = nullptr) {
  if (p.m < 1 || p.m > 8) return ek_fail(hipErrorInvalidValue, "gemv: batch rows must be 1..8 per launch");
  if (k <= 0 || k % 8 || sk < 1 || k % (8 * sk))
    return ek_fail(hipErrorInvalidValue, "gemv: K must be a positive multiple of 8*splits");
  if (sk > 1 && epi != EPI_PARTS) return ek_fail(hipErrorInvalidValue, "gemv: split-K needs the partials epilogue");
  if (sk > 1 && pro != PRO_X) return ek_fail(hipErrorInvalidValue, "gemv: split-K needs a plain x prologue");
  if (sk > 65535) return ek_fail(hipErrorInvalidValue, "gemv: too many splits");
  p.ks = k / sk;
  if (!aligned16(p.w) || p.ldw % 8 || (p.x && (!aligned16(p.x) || p.ldx % 8)) ||
      (p.res && (!aligned16(p.res) || p.ldr % 8)) || (p.res_out && (!aligned16(p.res_out) || p.ldro % 8)) ||
      (p.parts && !aligned16(p.parts)) || (p.nw && !aligned16(p.nw)) || (p.embed && (!aligned16(p.embed) || p.lde % 8)))
    return ek_fail(hipErrorInvalidValue, "gemv: operand rows must be 16-byte aligned (strides multiples of 8)");
  const int bm = bm_for(p.m);
  const size_t lds = (size_t)bm * p.ks * sizeof(bf16_t);
  if (lds > kMaxLds)
    return ek_fail(hipErrorInvalidValue, "gemv: batch rows x K exceed the 48 KiB activation stage (split K)");
  if (use_mfma(p.m, p.ks, rpw)) {
    const int64_t gx = mfma_grid(p.n, epi);
    if (gx_out) *gx_out = gx;
    const int nb = mfma_nb(p.ks / MCH, epi == EPI_SWIGLU);
    const size_t mlds = (size_t)bm * mfma_xld(p.ks) * sizeof(bf16_t);
    dim3 grid((unsigned)gx, (unsigned)sk);
#define EK_CASE(PR, EP) \
  if (pro == PR && epi == EP) return launch_mfma_pair<PR, EP>(p, bm, nb, grid, mlds, st);
    EK_CASE(PRO_X, EPI_BF16)
    EK_CASE(PRO_X, EPI_PARTS)
    EK_CASE(PRO_X, EPI_SWIGLU)
    EK_CASE(PRO_X, EPI_ARGMAX)
    EK_CASE(PRO_NORM, EPI_BF16)
    EK_CASE(PRO_NORM, EPI_SWIGLU)
    EK_CASE(PRO_ADD_NORM, EPI_BF16)
    EK_CASE(PRO_ADD_NORM, EPI_SWIGLU)
    EK_CASE(PRO_PARTS, EPI_BF16)
    EK_CASE(PRO_PARTS, EPI_SWIGLU)
    EK_CASE(PRO_PARTS, EPI_ARGMAX)
    EK_CASE(PRO_EMBED, EPI_BF16)
#undef EK_CASE
    return ek_fail(hipErrorInvalidValue, "gemv: unsupported prologue/epilogue pair");
  }
  if (rpw < 0) rpw = -rpw;   // -r: the FMA kernel forced, r rows per wave
  if (rpw == 0) rpw = (epi == EPI_ARGMAX) ? 4 : 1;
  if (rpw != 1 && rpw != 2 && rpw != 4) return ek_fail(hipErrorInvalidValue, "gemv: rows per wave must be 1, 2 or 4");
  const int64_t rows_per_grp = (int64_t)NWAVE * rpw;
  const int64_t ngroups = (p.n + rows_per_grp - 1) / rows_per_grp;
  if (blocks <= 0) blocks = 4 * (int64_t)cu_count();
  const int64_t gx = ngroups < blocks ? ngroups : blocks;
  if (gx <= 0 || gx > 0x7fffffff) return ek_fail(hipErrorInvalidValue, "gemv: bad grid");
  if (gx_out) *gx_out = gx;
  dim3 grid((unsigned)gx, (unsigned)sk);
  const int kpl = pick_kpl(p.ks / 8);
#define EK_CASE(PR, EP) \
  if (pro == PR && epi == EP) return launch_pair<PR, EP>(p, bm, kpl, (int)rpw, grid, lds, st);
  EK_CASE(PRO_X, EPI_BF16)
  EK_CASE(PRO_X, EPI_PARTS)
  EK_CASE(PRO_X, EPI_SWIGLU)
  EK_CASE(PRO_X, EPI_ARGMAX)
  EK_CASE(PRO_NORM, EPI_BF16)
  EK_CASE(PRO_NORM, EPI_SWIGLU)
  EK_CASE(PRO_ADD_NORM, EPI_BF16)
  EK_CASE(PRO_ADD_NORM, EPI_SWIGLU)
  EK_CASE(PRO_PARTS, EPI_BF16)
  EK_CASE(PRO_PARTS, EPI_SWIGLU)
  EK_CASE(PRO_PARTS, EPI_ARGMAX)
  EK_CASE(PRO_EMBED, EPI_BF16)
#undef EK_CASE
  return ek_fail(hipErrorInvalidValue, "gemv: unsupported prologue/epilogue pair");
}

// One workgroup: the first-index argmax over `parts` per-workgroup partials
// of each of m rows, then the optional decode-step bookkeeping.
__global__ __launch_bounds__(NTHR) void argmax_reduce_kernel(const float* __restrict__ am_val,
                                                             const int32_t* __restrict__ am_idx, int64_t parts,
                                                             int m, int64_t* out_tok, int64_t* st_tokens,
                                                             int64_t* st_positions, int32_t* st_out,
                                                             int64_t* st_step, int64_t max_steps) {
  __shared__ float tbv[NTHR];
  __shared__ int tbi[NTHR];
  for (int b = 0; b < m; ++b) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int64_t blk = threadIdx.x; blk < parts; blk += NTHR) {
      const float v = am_val[blk * m + b];
      const int i = am_idx[blk * m + b];
      if (i != 0x7fffffff && (bi == 0x7fffffff || v > bv || (v == bv && i < bi))) { bv = v; bi = i; }
    }
    tbv[threadIdx.x] = bv;
    tbi[threadIdx.x] = bi;
    __syncthreads();
    for (int s = NTHR / 2; s > 0; s >>= 1) {
      if (threadIdx.x < (unsigned)s) {
        const float v = tbv[threadIdx.x + s];
        const int i = tbi[threadIdx.x + s];
        const float cv = tbv[threadIdx.x];
        const int ci = tbi[threadIdx.x];
        if (i != 0x7fffffff && (ci == 0x7fffffff || v > cv || (v == cv && i < ci))) {
          tbv[threadIdx.x] = v;
          tbi[threadIdx.x] = i;
        }
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      const int64_t tok = tbi[0] == 0x7fffffff ? 0 : tbi[0];
      if (out_tok) out_tok[b] = tok;
      if (st_tokens) {
        st_tokens[b] = tok;
        st_positions[b] += 1;
        const int64_t step = *st_step;
        if (step >= 0 && step < max_steps) st_out[step * m + b] = (int32_t)tok;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0 && st_tokens) *st_step += 1;
}

GemvParams zero_params() {
  GemvParams p;
  memset(&p, 0, sizeof(p));
  return p;
}

}  // namespace
}  // namespace ekg

using namespace ekg;

// ============================================================================
// C ABI
// ============================================================================
extern "C" {

int ek_gemv(const void* x, const void* w, void* y, int64_t m, int64_t n, int64_t k, int64_t ldx, int64_t ldw,
            int64_t ldy, int64_t rpw, int64_t blocks, void* stream) {
  EK_GUARD();
  if (m < 1 || n < 1) return ek_fail(hipErrorInvalidValue, "gemv: empty shape");
  hipStream_t st = (hipStream_t)stream;
  for (int64_t m0 = 0; m0 < m;) {
    int64_t mt = m - m0 < 8 ? m - m0 : 8;
    while (mt > 1 && (size_t)bm_for((int)mt) * k * 2 > kMaxLds) mt = mt > 4 ? 4 : mt > 2 ? 2 : 1;
    GemvParams p = zero_params();
    p.w = (const bf16_t*)w; p.ldw = ldw; p.n = n; p.m = (int)mt;
    p.x = (const bf16_t*)x + m0 * ldx; p.ldx = ldx;
    p.y = (bf16_t*)y + m0 * ldy; p.ldy = ldy;
    hipError_t e = run_gemv(PRO_X, EPI_BF16, p, k, 1, rpw, blocks, st);
    if (e != hipSuccess) return e;
    m0 += mt;
  }
  return hipSuccess;
}

int ek_gemv_parts(const void* x, const void* w, float* parts, int64_t m, int64_t n, int64_t k, int64_t ldx,
                  int64_t ldw, int64_t sk, int64_t rpw, int64_t blocks, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || n < 1) return ek_fail(hipErrorInvalidValue, "gemv_parts: m must be 1..8");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = n; p.m = (int)m;
  p.x = (const bf16_t*)x; p.ldx = ldx;
  p.p_out = parts;
  return run_gemv(PRO_X, EPI_PARTS, p, k, sk, rpw, blocks, (hipStream_t)stream);
}

int ek_gemv_swiglu(const void* x, const void* w, void* y, int64_t m, int64_t inter, int64_t k, int64_t ldx,
                   int64_t ldw, int64_t ldy, int64_t rpw, int64_t blocks, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || inter < 1) return ek_fail(hipErrorInvalidValue, "gemv_swiglu: m must be 1..8");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = inter; p.m = (int)m; p.up_off = inter;
  p.x = (const bf16_t*)x; p.ldx = ldx;
  p.y = (bf16_t*)y; p.ldy = ldy;
  return run_gemv(PRO_X, EPI_SWIGLU, p, k, 1, rpw, blocks, (hipStream_t)stream);
}

int ek_norm_gemv(const void* x, const void* residual, void* residual_out, const void* norm_w, const void* w,
                 void* y, int64_t m, int64_t n, int64_t k, int64_t ldx, int64_t ldr, int64_t ldro, int64_t ldw,
                 int64_t ldy, float eps, int silu, int64_t rpw, int64_t blocks, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || n < 1) return ek_fail(hipErrorInvalidValue, "norm_gemv: m must be 1..8");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = n; p.m = (int)m; p.up_off = n;
  p.x = (const bf16_t*)x; p.ldx = ldx;
  p.res = (const bf16_t*)residual; p.ldr = ldr;
  p.res_out = (bf16_t*)residual_out; p.ldro = ldro;
  p.nw = (const bf16_t*)norm_w; p.eps = eps;
  p.y = (bf16_t*)y; p.ldy = ldy;
  const int pro = residual ? PRO_ADD_NORM : PRO_NORM;
  return run_gemv(pro, silu ? EPI_SWIGLU : EPI_BF16, p, k, 1, rpw, blocks, (hipStream_t)stream);
}

int ek_parts_norm_gemv(const float* parts, int64_t sk_in, const void* residual, void* residual_out,
                       const void* norm_w, const void* w, void* y, int64_t m, int64_t n, int64_t k, int64_t ldr,
                       int64_t ldro, int64_t ldw, int64_t ldy, float eps, int silu, int64_t rpw, int64_t blocks,
                       void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || n < 1 || sk_in < 1) return ek_fail(hipErrorInvalidValue, "parts_norm_gemv: bad shape");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = n; p.m = (int)m; p.up_off = n;
  p.parts = parts; p.sk_in = (int)sk_in; p.parts_ss = m * k;
  p.res = (const bf16_t*)residual; p.ldr = ldr;
  p.res_out = (bf16_t*)residual_out; p.ldro = ldro;
  p.nw = (const bf16_t*)norm_w; p.eps = eps;
  p.y = (bf16_t*)y; p.ldy = ldy;
  return run_gemv(PRO_PARTS, silu ? EPI_SWIGLU : EPI_BF16, p, k, 1, rpw, blocks, (hipStream_t)stream);
}

int ek_embed_norm_gemv(const int64_t* tokens, const void* embed, int64_t lde, int64_t vocab, void* residual_out,
                       const void* norm_w, const void* w, void* y, int64_t m, int64_t n, int64_t k, int64_t ldro,
                       int64_t ldw, int64_t ldy, float eps, int64_t* slot_t, int64_t* len_t, int64_t rpw,
                       int64_t blocks, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || n < 1) return ek_fail(hipErrorInvalidValue, "embed_norm_gemv: m must be 1..8");
  if (len_t && !slot_t) return ek_fail(hipErrorInvalidValue, "embed_norm_gemv: len_t needs slot_t");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = n; p.m = (int)m;
  p.tokens = tokens; p.embed = (const bf16_t*)embed; p.lde = lde; p.vocab = vocab;
  p.res_out = (bf16_t*)residual_out; p.ldro = ldro;
  p.nw = (const bf16_t*)norm_w; p.eps = eps;
  p.slot_t = slot_t; p.len_t = len_t;
  p.y = (bf16_t*)y; p.ldy = ldy;
  return run_gemv(PRO_EMBED, EPI_BF16, p, k, 1, rpw, blocks, (hipStream_t)stream);
}

int ek_lm_head_argmax(const void* x, const float* parts, int64_t sk_in, const void* residual, const void* norm_w,
                      float eps, const void* w, int64_t m, int64_t vocab, int64_t k, int64_t ldx, int64_t ldr,
                      int64_t ldw, void* logits, int64_t ld_logits, float* am_val, int32_t* am_idx, int64_t am_cap,
                      int64_t* out_tok, int64_t* st_tokens, int64_t* st_positions, int32_t* st_out,
                      int64_t* st_step, int64_t max_steps, int64_t rpw, int64_t blocks, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || vocab < 1) return ek_fail(hipErrorInvalidValue, "lm_head_argmax: m must be 1..8");
  if (st_tokens && (!st_positions || !st_out || !st_step))
    return ek_fail(hipErrorInvalidValue, "lm_head_argmax: step state needs tokens, positions, out and step");
  const bool force_fma = rpw < 0;
  int64_t r = rpw < 0 ? -rpw : rpw == 0 ? 4 : rpw;
  if (r != 1 && r != 2 && r != 4) return ek_fail(hipErrorInvalidValue, "lm_head_argmax: rpw must be 1, 2 or 4");
  if (blocks <= 0) blocks = 4 * (int64_t)cu_count();
  const int64_t groups = (vocab + NWAVE * r - 1) / (NWAVE * r);
  const int64_t gx =
      use_mfma((int)m, k, force_fma ? -r : r) ? mfma_grid(vocab, EPI_ARGMAX) : groups < blocks ? groups : blocks;
  if (gx * m > am_cap) return ek_fail(hipErrorInvalidValue, "lm_head_argmax: partial buffer too small");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = vocab; p.m = (int)m;
  p.x = (const bf16_t*)x; p.ldx = ldx;
  p.parts = parts; p.sk_in = (int)sk_in; p.parts_ss = m * k;
  p.res = (const bf16_t*)residual; p.ldr = ldr;
  p.nw = (const bf16_t*)norm_w; p.eps = eps;
  p.y = (bf16_t*)logits; p.ldy = ld_logits;
  p.am_val = am_val; p.am_idx = am_idx;
  const int pro = parts ? PRO_PARTS : PRO_X;
  hipStream_t st = (hipStream_t)stream;
  int64_t used = 0;
  hipError_t e = run_gemv(pro, EPI_ARGMAX, p, k, 1, force_fma ? -r : r, blocks, st, &used);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(argmax_reduce_kernel, dim3(1), dim3(NTHR), 0, st, (const float*)am_val,
                     (const int32_t*)am_idx, used, (int)m, out_tok, st_tokens, st_positions, st_out, st_step,
                     max_steps);
  return hipGetLastError();
}

}  // extern "C"
