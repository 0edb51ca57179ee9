/* C ABI of libek_hip.so: the gfx950 kernels of the Qwen3 decode hot path.
 *
 * Every entry point takes raw device pointers, element counts and strides
 * (in elements), scalars by value, and the hipStream_t to launch on (as a
 * void*). It launches asynchronously and returns a hipError_t as int: 0 on
 * success; on a rejected argument, hipErrorInvalidValue (1) and a message
 * readable through ek_last_error(). No entry point allocates or
 * synchronizes, so every one of them may be recorded into a HIP graph. A
 * launch's status is read with hipGetLastError() after the launch: that
 * reports (and consumes) a failed launch, and also an error an earlier HIP
 * call on the calling thread left pending, which is then returned by this
 * entry point instead of by the caller's own next check. A failed attribute
 * or occupancy query inside an entry point is consumed the same way, so
 * that it is not reported by a later launch. Device scalars that a graph replay must re-read (sequence
 * length, start offsets, tokens, positions, step index) are passed as
 * pointers. bf16 tensors are raw 16-bit patterns; rows handed to 16-byte
 * loads must be 16-byte aligned with lengths that are multiples of 8.
 *
 * Citations name the reference interface each entry point replaces
 * (jeojdi1/EngineKernel, paths relative to its root).
 */
#ifndef EK_HIP_H
#define EK_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library identification and the last argument-check message of this thread. */
const char* ek_version(void);
const char* ek_last_error(void);
/* Compute units and gfx architecture name of the current device. */
int ek_device_info(int* n_cu, char* arch, int arch_len);
/* set_wait_limit: the number of polls after which a bounded device-side wait
 * (the decode step's hand-overs, the split attention's combine) gives up and
 * sets its error word; polls <= 0 restores each kernel's default (about a
 * second). Read when a launch is issued, so a captured graph keeps the bound
 * it was captured with. Returns the previous setting. No counterpart in the
 * reference (its kernels have no device-side waits); it lets tests and
 * callers with a latency budget bound how long a failed step takes. */
int64_t ek_set_wait_limit(int64_t polls);

/* rms_norm: y[m,:] = w (x) bf16(x * rsqrt(mean(x^2) + eps)).
 * Replaces engine/ek_kernels.py:1031-1042 (rms_norm, kernel :89-103). */
int ek_rms_norm(const void* x, const void* w, void* y, int64_t m, int64_t n, int64_t ldx, int64_t ldy,
                float eps, void* stream);

/* add_rms_norm: residual = bf16(residual + x) in place; y = rms_norm(residual).
 * Replaces engine/ek_kernels.py:1045-1059 (kernel :105-123). */
int ek_add_rms_norm(const void* x, void* residual, const void* w, void* y, int64_t m, int64_t n, int64_t ldx,
                    int64_t ldr, int64_t ldy, float eps, void* stream);

/* add_rms_norm_parts: x = bf16(sum_s parts[s]) over fp32 partials [sk, m, n];
 * residual = bf16(residual + x) in place; y = rms_norm(residual).
 * Replaces engine/ek_kernels.py:1296-1304 (kernel :447-470). */
int ek_add_rms_norm_parts(const float* parts, void* residual, const void* w, void* y, int64_t sk, int64_t m,
                          int64_t n, int64_t ldr, int64_t ldy, float eps, void* stream);

/* silu_mul: y[m, :n] = bf16(silu_fp32(gu[m, :n])) (x) gu[m, n:2n].
 * Replaces engine/ek_kernels.py:1062-1076 (kernel :125-143). */
int ek_silu_mul(const void* gu, void* y, int64_t m, int64_t n, int64_t ldgu, int64_t ldy, void* stream);

/* qk_norm_rope_kv: per-head RMSNorm + rotate-half RoPE on fused qkv rows
 * [m, (n_q + 2 n_kv) * head_dim]; q rotated in place; rotated k and raw v
 * written to caches [B, n_kv, S, D] at slot_base[row / m_per_batch] + row %
 * m_per_batch (slots outside [0, s_cap) are skipped). cos/sin rows are
 * indexed by qkv row with stride ld_cs.
 * Replaces engine/ek_kernels.py:1110-1146 (kernel :223-279). */
int ek_qk_norm_rope_kv(void* qkv, const void* qn, const void* kn, const void* cos, const void* sin,
                       void* k_cache, void* v_cache, const int64_t* slot_base, int64_t m, int64_t ld_qkv,
                       int64_t ld_cs, int64_t n_q, int64_t n_kv, int64_t head_dim, int64_t csb, int64_t csh,
                       int64_t css, int64_t s_cap, int64_t m_per_batch, float eps, void* stream);

/* GEMV-family tuning arguments (results do not depend on them beyond the
 * fp32 summation order): rpw = output rows per wave of the FMA kernel (1, 2
 * or 4; 0 = default), blocks = its grid cap (0 = four workgroups per CU;
 * workgroups loop over row groups). Launches of 2..8 batch rows whose
 * per-split K is a multiple of 128 run on the matrix cores (16-row MFMA
 * tiles, their own grid) and ignore both, unless rpw is negative: -r forces
 * the FMA kernel with r rows per wave. */

/* gemv: y[m, n] = bf16(sum_k x[m, k] * w[n, k]) with fp32 accumulation.
 * Replaces engine/ek_kernels.py:1322-1347 (gemv, kernel :281-308). */
int ek_gemv(const void* x, const void* w, void* y, int64_t m, int64_t n, int64_t k, int64_t ldx, int64_t ldw,
            int64_t ldy, int64_t rpw, int64_t blocks, void* stream);

/* gemv_parts: fp32 split-K partials parts[s, m, n] over sk equal K slices (m <= 8).
 * Replaces engine/ek_kernels.py:1277-1293 (kernel :413-445). */
int ek_gemv_parts(const void* x, const void* w, float* parts, int64_t m, int64_t n, int64_t k, int64_t ldx,
                  int64_t ldw, int64_t sk, int64_t rpw, int64_t blocks, void* stream);

/* gemv_swiglu: w is the fused [2*inter, k] gate-over-up matrix;
 * y[m, i] = bf16(silu(bf16 gate_i)) (x) bf16(up_i) (m <= 8).
 * Replaces engine/ek_kernels.py:1247-1261 (kernel :375-411). */
int ek_gemv_swiglu(const void* x, const void* w, void* y, int64_t m, int64_t inter, int64_t k, int64_t ldx,
                   int64_t ldw, int64_t ldy, int64_t rpw, int64_t blocks, void* stream);

/* norm_gemv: [residual add] + RMSNorm prologue + projection [+ SwiGLU epilogue].
 * residual == NULL: no add (the normalised input is x itself). Otherwise
 * r = bf16(x + residual) is written to residual_out (which must not alias x
 * or residual) and normalised. silu != 0: w is [2n, k] gate-over-up (m <= 8).
 * Replaces engine/ek_kernels.py:1220-1244 (kernel :310-373). */
int ek_norm_gemv(const void* x, const void* residual, void* residual_out, const void* norm_w, const void* w,
                 void* y, int64_t m, int64_t n, int64_t k, int64_t ldx, int64_t ldr, int64_t ldro, int64_t ldw,
                 int64_t ldy, float eps, int silu, int64_t rpw, int64_t blocks, void* stream);

/* parts_norm_gemv: the decode layer's consumer projection. r = bf16(residual +
 * bf16(sum_s parts[s])) over fp32 partials [sk_in, m, k]; r -> residual_out;
 * y = projection of rms_norm(r) [+ SwiGLU]. The composition
 * add_rms_norm_parts (engine/ek_kernels.py:1296) -> gemv (:1322) /
 * gemv_swiglu (:1247), as one launch. rpw: output rows per wave (0: default). */
int ek_parts_norm_gemv(const float* parts, int64_t sk_in, const void* residual, void* residual_out,
                       const void* norm_w, const void* w, void* y, int64_t m, int64_t n, int64_t k, int64_t ldr,
                       int64_t ldro, int64_t ldw, int64_t ldy, float eps, int silu, int64_t rpw, int64_t blocks,
                       void* stream);

/* embed_norm_gemv: the decode step's first layer. r = embed[tokens[b]] ->
 * residual_out; y = projection of rms_norm(r). When len_t != NULL it also
 * performs the step's slot/length advance (slot_t[b] = *len_t; *len_t += 1).
 * The composition F.embedding -> rms_norm -> qkv projection and the
 * slot_t/len_t update of engine/ek_model.py:375-388, as one launch. */
int ek_embed_norm_gemv(const int64_t* tokens, const void* embed, int64_t lde, int64_t vocab, void* residual_out,
                       const void* norm_w, const void* w, void* y, int64_t m, int64_t n, int64_t k, int64_t ldro,
                       int64_t ldw, int64_t ldy, float eps, int64_t* slot_t, int64_t* len_t, int64_t rpw,
                       int64_t blocks, void* stream);

/* attn_decode: split-K decode attention over caches [B, n_kv, S, D] (D in
 * {32, 64, 128}, n_q / n_kv in {1, 2, 4, 8}) for keys [start[b], *seq_len).
 * rope != 0: q is the raw fused qkv row (stride ldq_b); the query heads are
 * QK-normed and rotated, and the new key (rotated) and value (raw) are
 * written at slot *seq_len - 1 -- rope_attn_decode, engine/ek_kernels.py:
 * 1476-1507 (kernel :678-780). rope == 0: q [B, n_q, D] is already rotated
 * -- flash_decode, engine/ek_kernels.py:1389-1416 (kernel :534-615).
 * With splits == 1 and n_q / n_kv * s_cap * 4 <= 32 KiB, one launch per
 * (b, kv head, 32 head dims) keeps the row's scores in LDS (scores, lsum,
 * mmax, chunk, part and ticket are then unused). Otherwise two launches over
 * (split, kv head, b), split s taking keys [s * chunk, (s + 1) * chunk) (the
 * last split up to *seq_len): per-split scores into the scratch [B, n_q,
 * score_ss] with the split's max/sum in mmax/lsum [B, n_kv, sp, gp]; then
 * each split's softmax-weighted value sum, written as {fp32, tag} words to
 * part (at least B * n_kv * splits * (n_q / n_kv) * D of them), which the
 * last workgroup of each (b, kv head) adds in split order -- the reference's
 * split combine (kernel :988-1019), deterministic. ticket holds two words
 * per (b, kv head) (an arrival count and an epoch), zeroed once with the
 * workspace and kept by the kernel; launches sharing a workspace must not
 * overlap. err (may be NULL) is set to 1 if the combine's bounded wait for a
 * split's words gives up (the output row is then invalid). Probabilities are
 * rounded to bf16 before the PV product, as in engine/ek_model.py:475-488.
 * cos/sin rows: positions[b] when positions != NULL, else row b. */
int ek_attn_decode(const void* q, int64_t ldq_b, int64_t ldq_h, int rope, const void* qn, const void* kn,
                   const void* cos, const void* sin, int64_t ld_cs, const int64_t* positions, int64_t rope_len,
                   void* k_cache, void* v_cache, int64_t csb, int64_t csh, int64_t css, int64_t s_cap,
                   const int64_t* seq_len, const int32_t* start, float* scores, int64_t score_ss, float* lsum,
                   float* mmax, int64_t sp, int64_t gp, void* out, int64_t ldo_b, int64_t ldo_h, int64_t b,
                   int64_t n_q, int64_t n_kv, int64_t head_dim, int64_t splits, int64_t chunk, float sm_scale,
                   float eps, void* part, int64_t part_words, uint32_t* ticket, int* err, void* stream);

/* attn_prefill: the prompt's causal GQA attention, engine/ek_model.py:315-323
 * (torch SDPA with the prompt mask of engine/engine.py:541-570): for each
 * row b and token t < s, query head j (q at q + (b * s + t) * ldq + j * D),
 * keys/values of kv head j / (n_q / n_kv) at cache slots [start[b], t]
 * (caches [B, n_kv, s_cap, D], strides csb/csh/css); a padding token
 * (t < start[b]) attends to itself only. out row (b * s + t), head j at
 * j * D, bf16. Flash attention on the matrix cores (fp32 online softmax,
 * probabilities rounded to bf16 for the value product). D in {32, 64, 128},
 * n_q / n_kv in {1, 2, 4, 8}. */
int ek_attn_prefill(const void* q, int64_t ldq, const void* k_cache, const void* v_cache, int64_t csb, int64_t csh,
                    int64_t css, int64_t s_cap, const int32_t* start, void* out, int64_t ldo, int64_t b, int64_t s,
                    int64_t n_q, int64_t n_kv, int64_t head_dim, float sm_scale, void* stream);

/* attn_verify: the attention of a speculative verify step, engine/ek_kernels.py:1419
 * (flash_verify; its torch form attn_torch, :1451): row b's nq query tokens
 * (q rows b * nq + j, as in attn_prefill) sit at cache slots len_b[b] + j
 * (their keys/values already written there), and query j sees the keys at
 * slots [start[b], len_b[b] + j]. Same kernel, layouts and arithmetic as
 * attn_prefill; len_b is a device int64 [B], clamped to [0, s_cap - nq].
 * splits > 1 spreads each row's keys over that many workgroups (s_cap / splits
 * keys each, in 32-key tiles) whose unnormalised rows and (max, sum) go to
 * part (fp32, at least splits * B * nq * n_q * (head_dim + 2) floats) and
 * are combined by a second launch; splits = 1 needs no part. */
int ek_attn_verify(const void* q, int64_t ldq, const void* k_cache, const void* v_cache, int64_t csb, int64_t csh,
                   int64_t css, int64_t s_cap, const int32_t* start, const int64_t* len_b, void* out, int64_t ldo,
                   int64_t b, int64_t nq, int64_t n_q, int64_t n_kv, int64_t head_dim, float sm_scale,
                   float* part, int64_t part_floats, int64_t splits, void* stream);

/* ngram_draft: engine/ek_kernels.py:1510 (ngram_draft, its kernel :618):
 * per row b, tokens[b][0..q) = [hist[b][hl - 1], q - 1 drafts] with hl =
 * hist_len[b]: the drafts continue the most recent earlier occurrence of the
 * trailing 3-gram of hist[b][0..hl) (else 2-gram, else token), wrapping around
 * a short cycle (see csrc/ek_spec.hip). hist [B, h] int64 (h < 2^20),
 * hist_len [B], tokens [B, q] int64 (q <= 256). */
int ek_ngram_draft(const int64_t* hist, const int64_t* hist_len, int64_t* tokens, int64_t b, int64_t h, int64_t q,
                   void* stream);

/* spec_accept: engine/ek_kernels.py:1519 (spec_accept, its kernel :652):
 * per row b, with am [B, q] the model's argmax after each of tokens[b]:
 * adv = min(1 + the number of leading drafts tokens[b][j + 1] == am[b][j],
 * remaining[b]); out_tok[step][b][0..q) = am[b] (int32), out_adv[step][b] =
 * adv (step = *step_idx, stores skipped unless 0 <= step < max_steps);
 * hist[b][hist_len[b] + j] = am[b][j] (j < q, inside the row); hist_len,
 * len_b, pos_b += adv; remaining -= adv. *step_idx is not advanced. q <= 64. */
int ek_spec_accept(const int64_t* tokens, const int64_t* am, int64_t* hist, int64_t* hist_len, int64_t* len_b,
                   int64_t* pos_b, int64_t* remaining, int32_t* out_tok, int32_t* out_adv, const int64_t* step_idx,
                   int64_t b, int64_t h, int64_t q, int64_t max_steps, void* stream);

/* lm_head_argmax: logits = bf16(h . w^T) over the vocabulary and the
 * first-index argmax per row -> out_tok[b] (int64). The hidden row h is x
 * (parts == NULL) or, fused, rms_norm(bf16(residual + bf16(sum_s parts[s])))
 * with gain norm_w (the decode's final add + norm, engine/ek_model.py:413-416).
 * logits (nullable) receives the bf16 logits. am_val/am_idx (am_cap entries,
 * at least grid width * m) hold per-workgroup partials, which a second
 * one-workgroup launch reduces. When st_tokens != NULL that launch also
 * advances the decode state: st_tokens[b] = token,
 * st_positions[b] += 1, st_out[*st_step * m + b] = token (if *st_step <
 * max_steps), *st_step += 1.
 * Replaces engine/ek_model.py:490-493 (argmax_token) and the step bookkeeping
 * of engine/engine.py:289-292. */
int ek_lm_head_argmax(const void* x, const float* parts, int64_t sk_in, const void* residual, const void* norm_w,
                      float eps, const void* w, int64_t m, int64_t vocab, int64_t k, int64_t ldx, int64_t ldr,
                      int64_t ldw, void* logits, int64_t ld_logits, float* am_val, int32_t* am_idx, int64_t am_cap,
                      int64_t* out_tok, int64_t* st_tokens, int64_t* st_positions, int32_t* st_out,
                      int64_t* st_step, int64_t max_steps, int64_t rpw, int64_t blocks, void* stream);

/* decode_step_plan: whether the persistent decode-step kernel handles this
 * shape (returns 0) and, in sizes[4], the bytes of the hand-over arena, the
 * long-context key split (0 when s_cap <= 1024 and n_q / n_kv * s_cap * 4 <=
 * 32 KiB: attention then runs on n_kv * head_dim / 32 workgroups of its own
 * beside the projections; otherwise every workgroup attends 1 / split of one
 * kv head's keys), the bytes of the launch-state block and the grid (one workgroup per
 * CU). It handles batch m = 1..8 (2..8 rows: head_dim 128, every workgroup
 * attending a key split of one (row, kv head)), up to 64 layers, head_dim 32/64/128, n_q / n_kv of
 * 2 or 4 (the Qwen3 dense models up to hidden 4096; other groups take the
 * per-kernel step), hidden (<= 4096), intermediate and n_q * head_dim multiples
 * of 512, and s_cap up to what one split's score rows fit in LDS (about
 * 260 K keys at n_q / n_kv = 4 on 256 CUs at one row), on a device where one workgroup
 * of the kernel fits on every CU at once (its waits need the whole grid
 * resident).
 * Plans engine/engine.py:273-282 (_make_ws) for the step below. */
int ek_decode_step_plan(int64_t hidden, int64_t inter, int64_t n_q, int64_t n_kv, int64_t head_dim, int64_t vocab,
                        int64_t m, int64_t s_cap, int64_t n_layers, int64_t* sizes);

/* decode_step: the whole greedy decode step as ONE persistent launch -- per
 * layer RMSNorm + qkv, QK-norm + RoPE + KV write + attention, o_proj, add +
 * RMSNorm + gate/up + SwiGLU, down_proj; then the final add + norm, lm_head,
 * first-index argmax and the step bookkeeping (tokens[b] = token,
 * positions[b] += 1, slot_t[b] = *len_t, *len_t += 1, out_buf[*step_idx * m +
 * b] = token if *step_idx < max_steps, *step_idx += 1, out_tok[b] = token if
 * out_tok; logits[b * vocab ..) = row b's bf16 logits if logits is not
 * NULL), for the m rows of the batch (b < m). One workgroup per CU; workgroups hand activations to each other
 * through the arena as dense words of four bf16 that the consumer polls
 * until they are nonzero, with no grid barrier: the arena is two halves,
 * each launch hands over through one and zeroes the other for the next.
 * layer_ptrs: device int64 [n_layers][10] = addresses of qkv [(n_q + 2 n_kv) D,
 * hidden], o [hidden, n_q D], gate/up [2 inter, hidden], down [hidden, inter],
 * ln1, ln2 [hidden], q_norm, k_norm [D], k_cache, v_cache [B, n_kv, S, D] of
 * each layer (bf16, all caches with strides csb/csh/css). arena: the
 * hand-over arena (at least decode_step_plan sizes[0] bytes; every launch on
 * one arena must pass the same arena_bytes, which fixes where its halves
 * lie) and barrier: the launch-state block (sizes[2] bytes), both zero before
 * the first launch and kept between launches (they hold the launch epoch and
 * the next launch's cleared half); err: set to 1 (and the
 * launch abandoned) if a hand-over wait exceeds its bound. An abandoned
 * launch, and every launch that starts while err is set, still advances
 * *step_idx and writes -1 as its token to out_buf and out_tok, leaving
 * tokens, positions, slot_t and len_t unchanged, so the failure shows in the
 * step's own output row; zero err, the arena and the barrier block before
 * decoding again.
 * Launches that overlap on one device race on the arena and the barrier.
 * Replaces engine/ek_model.py:360-416 (decode) + :490-493 (argmax_token) and
 * the bookkeeping of engine/engine.py:288-292, i.e. the whole captured step
 * body engine.py:284-292 (_step_body). */
int ek_decode_step(const int64_t* layer_ptrs, int64_t n_layers, int64_t hidden, int64_t inter, int64_t n_q,
                   int64_t n_kv, int64_t head_dim, int64_t vocab, int64_t m, float eps, float sm_scale,
                   const void* embed, int64_t lde, const void* lm_head, const void* final_norm, const void* cos,
                   const void* sin, int64_t ld_cs, int64_t rope_len, int64_t csb, int64_t csh, int64_t css,
                   int64_t s_cap, int64_t* tokens, int64_t* positions, int64_t* len_t, int64_t* slot_t,
                   const int32_t* start_t, int32_t* out_buf, int64_t* step_idx, int64_t max_steps, int64_t* out_tok,
                   void* logits, void* arena, int64_t arena_bytes, void* barrier, int* err, void* stream);

/* decode_step_noalloc: decode_step without the caller's arena and barrier
 * block -- the launch uses a static per-device array of this library (the
 * launch-state block, about 4.3 KiB -- sizeof(eks::Bar), 4160 bytes, padded
 * to 256-byte alignment -- plus a hand-over arena of at most 16 MiB,
 * zero at load and held by each device until the process ends), so a call
 * allocates nothing and needs no workspace from the caller. Shapes whose
 * arena (decode_step_plan sizes[0]) exceeds 16 MiB are rejected with
 * hipErrorInvalidValue. Every call on one device shares that device's array:
 * calls that overlap on a device (other streams, other threads) race and must
 * not be issued. The array never needs clearing (each launch moves its
 * epoch on and clears the half the next launch uses); after an abandoned
 * launch zero only *err. Same arguments,
 * results and error behaviour as decode_step otherwise.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). */
int ek_decode_step_noalloc(const int64_t* layer_ptrs, int64_t n_layers, int64_t hidden, int64_t inter, int64_t n_q,
                           int64_t n_kv, int64_t head_dim, int64_t vocab, int64_t m, float eps, float sm_scale,
                           const void* embed, int64_t lde, const void* lm_head, const void* final_norm,
                           const void* cos, const void* sin, int64_t ld_cs, int64_t rope_len, int64_t csb,
                           int64_t csh, int64_t css, int64_t s_cap, int64_t* tokens, int64_t* positions,
                           int64_t* len_t, int64_t* slot_t, const int32_t* start_t, int32_t* out_buf,
                           int64_t* step_idx, int64_t max_steps, int64_t* out_tok, void* logits, int* err,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EK_HIP_H */
