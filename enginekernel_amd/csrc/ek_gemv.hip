// C-ABI entry points of the GEMV family (kernel template: ek_gemv_impl.h;
// instantiations: ek_gemv_inst.hip, one object per prologue/epilogue pair).

#include <cstring>

#include "ek_abi_internal.h"
#include "ek_gemv_impl.h"
#include "ek_hip.h"

namespace ekg {
namespace {


// ----------------------------------------------------------------------------
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

// Launch one GEMV-family kernel. sk > 1 splits the reduction over
// blockIdx.y (EPI_PARTS only). rpw == 0 picks the default rows per wave.
hipError_t run_gemv(int pro, int epi, GemvParams p, int64_t k, int64_t sk, int rpw, hipStream_t st) {
  if (p.m < 1 || p.m > 8) return ek_fail(hipErrorInvalidValue, "gemv: batch rows must be 1..8 per launch");
  if (k <= 0 || k % 8 || sk < 1 || k % (8 * sk))
    return ek_fail(hipErrorInvalidValue, "gemv: K must be a positive multiple of 8*splits");
  if (sk > 1 && epi != EPI_PARTS) return ek_fail(hipErrorInvalidValue, "gemv: split-K needs the partials epilogue");
  if (sk > 1 && pro != PRO_X) return ek_fail(hipErrorInvalidValue, "gemv: split-K needs a plain x prologue");
  p.ks = k / sk;
  if (!aligned16(p.w) || p.ldw % 8 || (p.x && (!aligned16(p.x) || p.ldx % 8)) ||
      (p.res && (!aligned16(p.res) || p.ldr % 8)) || (p.res_out && (!aligned16(p.res_out) || p.ldro % 8)) ||
      (p.parts && !aligned16(p.parts)) || (p.nw && !aligned16(p.nw)) || (p.embed && (!aligned16(p.embed) || p.lde % 8)))
    return ek_fail(hipErrorInvalidValue, "gemv: operand rows must be 16-byte aligned (strides multiples of 8)");
  const int bm = bm_for(p.m);
  const size_t lds = (size_t)bm * p.ks * sizeof(bf16_t);
  if (lds > kMaxLds) return ek_fail(hipErrorInvalidValue, "gemv: batch rows x K exceed the 48 KiB activation stage (split K)");
  if (rpw <= 0) rpw = (epi == EPI_ARGMAX) ? 4 : 1;
  const int64_t rows_per_blk = (int64_t)NWAVE * rpw;
  const int64_t gx = (p.n + rows_per_blk - 1) / rows_per_blk;
  if (gx <= 0 || gx > 0x7fffffff) return ek_fail(hipErrorInvalidValue, "gemv: bad grid");
  dim3 grid((unsigned)gx, (unsigned)sk);
  const int kpl = pick_kpl(p.ks / 8);
#define EK_CASE(PR, EP) if (pro == PR && epi == EP) return launch_pair<PR, EP>(p, bm, kpl, rpw, grid, lds, st);
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

int ek_gemv(const void* x, const void* w, void* y, int64_t m, int64_t n, int64_t k,
            int64_t ldx, int64_t ldw, int64_t ldy, void* stream) {
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
    hipError_t e = run_gemv(PRO_X, EPI_BF16, p, k, 1, 0, st);
    if (e != hipSuccess) return e;
    m0 += mt;
  }
  return hipSuccess;
}

int ek_gemv_parts(const void* x, const void* w, float* parts, int64_t m, int64_t n, int64_t k,
                  int64_t ldx, int64_t ldw, int64_t sk, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || n < 1) return ek_fail(hipErrorInvalidValue, "gemv_parts: m must be 1..8");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = n; p.m = (int)m;
  p.x = (const bf16_t*)x; p.ldx = ldx;
  p.p_out = parts;
  return run_gemv(PRO_X, EPI_PARTS, p, k, sk, 0, (hipStream_t)stream);
}

int ek_gemv_swiglu(const void* x, const void* w, void* y, int64_t m, int64_t inter, int64_t k,
                   int64_t ldx, int64_t ldw, int64_t ldy, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || inter < 1) return ek_fail(hipErrorInvalidValue, "gemv_swiglu: m must be 1..8");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = inter; p.m = (int)m; p.up_off = inter;
  p.x = (const bf16_t*)x; p.ldx = ldx;
  p.y = (bf16_t*)y; p.ldy = ldy;
  return run_gemv(PRO_X, EPI_SWIGLU, p, k, 1, 0, (hipStream_t)stream);
}

int ek_norm_gemv(const void* x, const void* residual, void* residual_out, const void* norm_w,
                 const void* w, void* y, int64_t m, int64_t n, int64_t k, int64_t ldx, int64_t ldr,
                 int64_t ldro, int64_t ldw, int64_t ldy, float eps, int silu, void* stream) {
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
  return run_gemv(pro, silu ? EPI_SWIGLU : EPI_BF16, p, k, 1, 0, (hipStream_t)stream);
}

int ek_parts_norm_gemv(const float* parts, int64_t sk_in, const void* residual, void* residual_out,
                       const void* norm_w, const void* w, void* y, int64_t m, int64_t n, int64_t k,
                       int64_t ldr, int64_t ldro, int64_t ldw, int64_t ldy, float eps, int silu,
                       int64_t rpw, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || n < 1 || sk_in < 1) return ek_fail(hipErrorInvalidValue, "parts_norm_gemv: bad shape");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = n; p.m = (int)m; p.up_off = n;
  p.parts = parts; p.sk_in = (int)sk_in; p.parts_ss = m * k;
  p.res = (const bf16_t*)residual; p.ldr = ldr;
  p.res_out = (bf16_t*)residual_out; p.ldro = ldro;
  p.nw = (const bf16_t*)norm_w; p.eps = eps;
  p.y = (bf16_t*)y; p.ldy = ldy;
  return run_gemv(PRO_PARTS, silu ? EPI_SWIGLU : EPI_BF16, p, k, 1, (int)rpw, (hipStream_t)stream);
}

int ek_embed_norm_gemv(const int64_t* tokens, const void* embed, int64_t lde, int64_t vocab,
                       void* residual_out, const void* norm_w, const void* w, void* y, int64_t m,
                       int64_t n, int64_t k, int64_t ldro, int64_t ldw, int64_t ldy, float eps,
                       int64_t* slot_t, int64_t* len_t, int64_t rpw, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || n < 1) return ek_fail(hipErrorInvalidValue, "embed_norm_gemv: m must be 1..8");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = n; p.m = (int)m;
  p.tokens = tokens; p.embed = (const bf16_t*)embed; p.lde = lde; p.vocab = vocab;
  p.res_out = (bf16_t*)residual_out; p.ldro = ldro;
  p.nw = (const bf16_t*)norm_w; p.eps = eps;
  p.slot_t = slot_t; p.len_t = len_t;
  p.y = (bf16_t*)y; p.ldy = ldy;
  return run_gemv(PRO_EMBED, EPI_BF16, p, k, 1, (int)rpw, (hipStream_t)stream);
}

int ek_lm_head_argmax(const void* x, const float* parts, int64_t sk_in, const void* residual,
                      const void* norm_w, float eps, const void* w, int64_t m, int64_t vocab, int64_t k,
                      int64_t ldx, int64_t ldr, int64_t ldw, void* logits, int64_t ld_logits,
                      float* am_val, int32_t* am_idx, int64_t am_cap, int32_t* counter, int64_t* out_tok,
                      int64_t* st_tokens, int64_t* st_positions, int32_t* st_out, int64_t* st_step,
                      int64_t max_steps, int64_t rpw, void* stream) {
  EK_GUARD();
  if (m < 1 || m > 8 || vocab < 1) return ek_fail(hipErrorInvalidValue, "lm_head_argmax: m must be 1..8");
  if (rpw <= 0) rpw = 4;
  const int64_t blocks = (vocab + NWAVE * rpw - 1) / (NWAVE * rpw);
  if (blocks * m > am_cap) return ek_fail(hipErrorInvalidValue, "lm_head_argmax: partial buffer too small");
  GemvParams p = zero_params();
  p.w = (const bf16_t*)w; p.ldw = ldw; p.n = vocab; p.m = (int)m;
  p.x = (const bf16_t*)x; p.ldx = ldx;
  p.parts = parts; p.sk_in = (int)sk_in; p.parts_ss = m * k;
  p.res = (const bf16_t*)residual; p.ldr = ldr;
  p.nw = (const bf16_t*)norm_w; p.eps = eps;
  p.y = (bf16_t*)logits; p.ldy = ld_logits;
  p.am_val = am_val; p.am_idx = am_idx; p.counter = counter; p.out_tok = out_tok;
  p.st_tokens = st_tokens; p.st_positions = st_positions; p.st_out = st_out; p.st_step = st_step;
  p.max_steps = max_steps;
  const int pro = parts ? PRO_PARTS : PRO_X;
  return run_gemv(pro, EPI_ARGMAX, p, k, 1, (int)rpw, (hipStream_t)stream);
}

}  // extern "C"
