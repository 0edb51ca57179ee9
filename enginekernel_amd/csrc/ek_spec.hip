// Speculative decoding's two integer kernels for gfx950: the n-gram draft
// and the accept step (the reference's _ngram_draft_kernel and
// _spec_accept_kernel, engine/ek_kernels.py:618-680, wrapped at :1510-1523;
// their torch form is engine.py:357-383). Per row, int64 token ids:
//
//   draft    tokens[row] = [last emitted token, Q-1 drafts]. The drafts
//            continue the most recent earlier occurrence of the history's
//            trailing 3-gram (else 2-gram, else token): position j <= hl - 2
//            scores (j + 1) + 2^20 [2-gram matches] + 2^21 [3-gram matches];
//            p = max score mod 2^20 (0: no match), span = max(hl - p, 1),
//            draft i = hist[min(p + i mod span, H - 1)].
//   accept   nacc = length of the prefix of drafts equal to the model's
//            argmax at the position before them, adv = min(nacc + 1,
//            remaining); the step's Q argmax tokens and adv go to the output
//            ring at step_idx, all Q argmax tokens to hist[hl ..] (those past
//            hl + adv are overwritten by the next step), and hist_len, len_b,
//            pos_b advance by adv, remaining falls by it.
//
// One workgroup per row: the draft's scan is spread over the workgroup (one
// position per thread and pass, a max-reduction over the waves); the accept
// step is one wave.

#include <cstring>

#include "ek_abi_internal.h"
#include "ek_common.h"
#include "ek_hip.h"

namespace {

constexpr int DNT = 256;                  // draft threads per row
constexpr int64_t BIG = int64_t(1) << 20; // score weight of one n-gram order (positions < 2^20)

__global__ __launch_bounds__(DNT) void ngram_draft_kernel(const int64_t* __restrict__ hist,
                                                          const int64_t* __restrict__ hist_len,
                                                          int64_t* __restrict__ tokens, int64_t h, int q) {
  __shared__ int64_t red[DNT / EK_WAVE];
  const int row = blockIdx.x, tid = threadIdx.x;
  const int64_t* base = hist + (int64_t)row * h;
  int64_t hl = hist_len[row];
  hl = hl < 1 ? 1 : (hl > h ? h : hl);
  const int64_t k_last = base[hl - 1];
  const int64_t k_prev = base[hl - 2 > 0 ? hl - 2 : 0];
  const int64_t k_pp = base[hl - 3 > 0 ? hl - 3 : 0];
  int64_t best = 0;
  for (int64_t j = tid; j <= hl - 2; j += DNT) {
    const bool m1 = base[j] == k_last;
    const bool m2 = m1 && j >= 1 && base[j - 1] == k_prev;
    const bool m3 = m2 && j >= 2 && base[j - 2] == k_pp;
    const int64_t sc = (m1 ? j + 1 : 0) + (m2 ? BIG : 0) + (m3 ? 2 * BIG : 0);
    best = sc > best ? sc : best;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const int64_t v = __shfl_xor(best, o, EK_WAVE);
    best = v > best ? v : best;
  }
  if ((tid & 63) == 0) red[tid >> 6] = best;
  __syncthreads();
  if (tid < q) {
    int64_t m = red[0];
#pragma unroll
    for (int w = 1; w < DNT / EK_WAVE; ++w) m = red[w] > m ? red[w] : m;
    const int64_t p = m % BIG;
    const int64_t span = hl - p > 1 ? hl - p : 1;
    int64_t src = p + (tid >= 1 ? (int64_t)(tid - 1) % span : 0);
    src = src < h - 1 ? src : h - 1;
    tokens[(int64_t)row * q + tid] = tid == 0 ? k_last : base[src];
  }
}

__global__ __launch_bounds__(EK_WAVE) void spec_accept_kernel(
    const int64_t* __restrict__ tokens, const int64_t* __restrict__ am, int64_t* __restrict__ hist,
    int64_t* __restrict__ hist_len, int64_t* __restrict__ len_b, int64_t* __restrict__ pos_b,
    int64_t* __restrict__ remaining, int32_t* __restrict__ out_tok, int32_t* __restrict__ out_adv,
    const int64_t* __restrict__ step_idx, int64_t h, int64_t b, int q, int64_t max_steps) {
  const int row = blockIdx.x, j = threadIdx.x;
  const bool inq = j < q;
  const int64_t a = inq ? am[(int64_t)row * q + j] : 0;
  const int64_t nxt = j < q - 1 ? tokens[(int64_t)row * q + j + 1] : -1;
  const bool match = j < q - 1 && nxt == a;
  // nacc = the first j < q - 1 whose draft does not match (q - 1 if all do)
  int first = match ? q - 1 : (j < q - 1 ? j : q - 1);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const int v = __shfl_xor(first, o, EK_WAVE);
    first = v < first ? v : first;
  }
  const int64_t rem = remaining[row];
  const int64_t adv = (int64_t)first + 1 < rem ? (int64_t)first + 1 : rem;
  const int64_t step = *step_idx;
  const int64_t hl = hist_len[row];
  if (step >= 0 && step < max_steps) {
    if (inq) out_tok[(step * b + row) * q + j] = (int32_t)a;
    if (j == 0) out_adv[step * b + row] = (int32_t)adv;
  }
  if (inq && hl >= 0 && hl + j < h) hist[(int64_t)row * h + hl + j] = a;
  if (j == 0) {
    hist_len[row] = hl + adv;
    len_b[row] += adv;
    pos_b[row] += adv;
    remaining[row] = rem - adv;
  }
}

}  // namespace

extern "C" {

int ek_ngram_draft(const int64_t* hist, const int64_t* hist_len, int64_t* tokens, int64_t b, int64_t h, int64_t q,
                   void* stream) {
  EK_GUARD();
  if (b < 1 || b > 65535 || h < 1 || h >= BIG || q < 1 || q > DNT)
    return ek_fail(hipErrorInvalidValue, "ngram_draft: need 1 <= b <= 65535, 1 <= H < 2^20, 1 <= Q <= 256");
  hipLaunchKernelGGL(ngram_draft_kernel, dim3((unsigned)b), dim3(DNT), 0, (hipStream_t)stream, hist, hist_len,
                     tokens, h, (int)q);
  return hipGetLastError();
}

int ek_spec_accept(const int64_t* tokens, const int64_t* am, int64_t* hist, int64_t* hist_len, int64_t* len_b,
                   int64_t* pos_b, int64_t* remaining, int32_t* out_tok, int32_t* out_adv, const int64_t* step_idx,
                   int64_t b, int64_t h, int64_t q, int64_t max_steps, void* stream) {
  EK_GUARD();
  if (b < 1 || b > 65535 || h < 1 || q < 1 || q > EK_WAVE || max_steps < 1)
    return ek_fail(hipErrorInvalidValue, "spec_accept: need 1 <= b <= 65535, H >= 1, 1 <= Q <= 64");
  hipLaunchKernelGGL(spec_accept_kernel, dim3((unsigned)b), dim3(EK_WAVE), 0, (hipStream_t)stream, tokens, am,
                     hist, hist_len, len_b, pos_b, remaining, out_tok, out_adv, step_idx, h, b, (int)q, max_steps);
  return hipGetLastError();
}

}  // extern "C"
