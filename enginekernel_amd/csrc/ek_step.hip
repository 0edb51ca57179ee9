// C ABI of the persistent decode-step kernel (ek_step_impl.h): the plan query
// and the launch.

#include "ek_bstep_impl.h"
#include "ek_abi_internal.h"
#include "ek_hip.h"

#include <map>
#include <mutex>
#include <tuple>

namespace eks {
template <> hipError_t launch_step<32>(const StepArgs&, int, int, hipStream_t);
template <> hipError_t launch_step<64>(const StepArgs&, int, int, hipStream_t);
template <> hipError_t launch_step<128>(const StepArgs&, int, int, hipStream_t);
template <> int step_occupancy<32>(int, bool, size_t);
template <> int step_occupancy<64>(int, bool, size_t);
template <> int step_occupancy<128>(int, bool, size_t);
template <> hipError_t launch_bstep<2>(const StepArgs&, int, int, hipStream_t);
template <> hipError_t launch_bstep<4>(const StepArgs&, int, int, hipStream_t);
template <> hipError_t launch_bstep<8>(const StepArgs&, int, int, hipStream_t);
template <> int bstep_occupancy<2>(int, size_t);
template <> int bstep_occupancy<4>(int, size_t);
template <> int bstep_occupancy<8>(int, size_t);
}  // namespace eks

// The no-allocation entry point's state: the launch-state block (Bar,
// padded to 256 bytes) followed by the hand-over arena, at most
// kStaticArenaBytes. Each device holds its own copy of this array, zero at
// load and kept until the process ends; its address on a device comes from
// hipGetSymbolAddress (the array's name is not a device address in host
// code). Nothing in it needs clearing between calls: every launch bumps the
// per-workgroup epochs in the Bar and zeroes the half of the arena that the
// next launch hands over through, whatever the shapes of the two calls.
constexpr size_t kStaticBarBytes = (sizeof(eks::Bar) + 255) / 256 * 256;
constexpr size_t kStaticArenaBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticBarBytes + kStaticArenaBytes];

namespace {

constexpr int64_t kSpin = int64_t(1) << 20;           // default polls of one hand-over wait before giving up (~1 s)
constexpr size_t kLdsLimit = eks::kStepDynLds;        // dynamic LDS per workgroup (the static arrays take the rest)
// Rows of at most kUnitMaxKeys keys whose scores fit kFusedScoreLds bytes
// run on the attention units beside the projections; longer ones on the
// split kernel. At the Qwen3-4B shape the split kernel is the faster one
// from a 1024-key bucket on (ms per step at contexts ~940, split vs units:
// 1.824 vs 1.854; at ~640, a 768-key bucket, 1.818 vs 1.702; the split
// kernel stays at ~1.825 from 1024 to 2048 keys, the units reach 1.953 at
// 1280 and 2.104 at 1536): the 32 attention units then stream more keys than
// the projections take to run, while the split kernel's attention is on the
// critical path of every workgroup.
#ifndef EK_STEP_UNIT_MAX_KEYS
#define EK_STEP_UNIT_MAX_KEYS 768
#endif
constexpr int64_t kFusedScoreLds = 32 * 1024;
constexpr int64_t kUnitMaxKeys = EK_STEP_UNIT_MAX_KEYS;

int step_grid() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 0;
  }
  return n;
}

struct Plan {
  int mb;               // batch rows of the kernel (1, or m rounded up to 2, 4, 8: the batch kernel)
  int nwg, kpad_max, part_max, o_rows;
  int lsplit, lchunk;   // long contexts: key splits per kv head and keys per split (0: the attention-unit kernel)
  int64_t lx;           // long contexts: hand-over words of the splits' exchange
  int64_t half;         // words of one arena half the kernel needs
  int64_t arena_bytes;
  size_t lds;
};

template <int D>
size_t long_lds_d(int g, int64_t chunk) {
  switch (g) {
    case 1: return eks::LongLds<D, 1>::bytes(chunk);
    case 2: return eks::LongLds<D, 2>::bytes(chunk);
    case 4: return eks::LongLds<D, 4>::bytes(chunk);
    default: return eks::LongLds<D, 8>::bytes(chunk);
  }
}

size_t long_lds(int d, int g, int64_t chunk) {
  return d == 32 ? long_lds_d<32>(g, chunk) : d == 64 ? long_lds_d<64>(g, chunk) : long_lds_d<128>(g, chunk);
}

size_t attn_lds(int d, int g, int64_t s_cap) {
  size_t attn = eka::align16((size_t)(g + 6) * d * 2) + eka::align16((size_t)g * (s_cap | 1) * 4);   // AttnLds
  attn += eka::align16((size_t)g * d * 4) + eka::align16((size_t)d * 4) + eka::align16((size_t)eka::FDC * 2) +
          2 * eka::align16((size_t)eka::FNW * 8 * 4) + eka::align16((size_t)eka::FNW * 32 * eka::VTS * 2) +
          eka::align16((size_t)eka::FNW * g * eka::FDC * 4) + eka::align16((size_t)d * 2);
  return attn;
}

// Workgroups of step_kernel<d, g> with `lds` bytes of dynamic LDS that one CU
// holds at once (the occupancy query, cached per instantiation and size).
int resident_per_cu(int d, int g, bool lng, size_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, int, bool, size_t>, int> cache;
  const auto key = std::make_tuple(d, g, lng, lds);
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int n = 0;
  switch (d) {
    case 32: n = eks::step_occupancy<32>(g, lng, lds); break;
    case 64: n = eks::step_occupancy<64>(g, lng, lds); break;
    default: n = eks::step_occupancy<128>(g, lng, lds); break;
  }
  cache[key] = n;
  return n;
}

int resident_batch(int mb, int g, size_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, int, size_t>, int> cache;
  const auto key = std::make_tuple(mb, g, lds);
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  const int n = mb == 2 ? eks::bstep_occupancy<2>(g, lds) : mb == 4 ? eks::bstep_occupancy<4>(g, lds)
                                                                     : eks::bstep_occupancy<8>(g, lds);
  cache[key] = n;
  return n;
}

hipError_t make_plan(int64_t hidden, int64_t inter, int64_t n_q, int64_t n_kv, int64_t head_dim, int64_t vocab,
                     int64_t m, int64_t s_cap, int64_t n_layers, Plan& p);

// The batch kernel's plan (2..8 rows, ek_bstep_impl.h): every workgroup runs
// the projections of all rows and one attention unit (row, kv head, key
// split); the shape checks common to both kernels are done by the caller.
// sp is the split count that bounds a split's keys (lchunk) for any row of
// the bucket with every row split alike; the kernel gives each row at least
// the splits its own keys need (never more than sp) and shares the remaining
// nwg / n_kv slots per kv head out by keys (split_rows).
hipError_t make_batch_plan(int64_t hidden, int64_t inter, int64_t n_q, int64_t n_kv, int64_t head_dim, int64_t vocab,
                           int64_t m, int64_t s_cap, int64_t n_layers, Plan& p) {
  if (head_dim != 128) return ek_fail(hipErrorInvalidValue, "decode_step: batches of 2-8 rows need head_dim 128");
  const int g = (int)(n_q / n_kv);
  p.mb = m <= 2 ? 2 : m <= 4 ? 4 : 8;
  const int mb = p.mb;
  int sp = 1;
  while (2 * sp <= 32 && 2 * sp <= head_dim / 4 && (int64_t)2 * sp * n_kv * mb <= p.nwg) sp *= 2;
  if ((int64_t)sp * n_kv * mb > p.nwg) return ek_fail(hipErrorInvalidValue, "decode_step: too many attention units");
  const int64_t chunk = (s_cap + sp - 1) / sp;
  if (chunk > (1 << 16))
    return ek_fail(hipErrorInvalidValue, "decode_step: the context's score rows exceed the LDS of one split");
  p.lsplit = sp;
  p.lchunk = (int)chunk;
  p.lx = eks::long_words((int)n_kv, (int)(p.nwg / n_kv), g, 128);   // every slot's unit, whatever its row
  const int qw = (int)(n_q * head_dim), qkvw = (int)((n_q + 2 * n_kv) * head_dim);
  p.kpad_max = eks::bstep_xld((int)hidden, qw, mb);
  p.part_max = eks::bstep_part_rows((int)hidden, (int)inter, qkvw, p.nwg);
  p.o_rows = 0;
  size_t lds = 0;
  switch (mb) {
    case 2: lds = g == 2 ? eks::bstep_lds_bytes<128, 2, 2>((int)hidden, qw, p.part_max, p.lchunk, p.nwg)
                         : eks::bstep_lds_bytes<128, 4, 2>((int)hidden, qw, p.part_max, p.lchunk, p.nwg);
            break;
    case 4: lds = g == 2 ? eks::bstep_lds_bytes<128, 2, 4>((int)hidden, qw, p.part_max, p.lchunk, p.nwg)
                         : eks::bstep_lds_bytes<128, 4, 4>((int)hidden, qw, p.part_max, p.lchunk, p.nwg);
            break;
    default: lds = g == 2 ? eks::bstep_lds_bytes<128, 2, 8>((int)hidden, qw, p.part_max, p.lchunk, p.nwg)
                          : eks::bstep_lds_bytes<128, 4, 8>((int)hidden, qw, p.part_max, p.lchunk, p.nwg);
  }
  p.lds = lds;
  if (p.lds > kLdsLimit)
    return ek_fail(hipErrorInvalidValue, "decode_step: this batch's rows or context exceed the workgroup's LDS");
  p.half = eks::arena_half_words((int)n_layers, (int)hidden, (int)inter, qkvw, qw, p.nwg, mb, p.lx);
  p.arena_bytes = 16 * p.half;
  if (resident_batch(mb, g, p.lds) < 1)
    return ek_fail(hipErrorInvalidValue, "decode_step: one workgroup per CU does not fit (registers or LDS)");
  (void)vocab;
  return hipSuccess;
}

// Returns an error (with a message) when the shape is outside what the kernel handles.
hipError_t make_plan(int64_t hidden, int64_t inter, int64_t n_q, int64_t n_kv, int64_t head_dim, int64_t vocab,
                     int64_t m, int64_t s_cap, int64_t n_layers, Plan& p) {
  if (m < 1 || m > 8) return ek_fail(hipErrorInvalidValue, "decode_step: batch must be 1 to 8 rows");
  p.mb = 1;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128)
    return ek_fail(hipErrorInvalidValue, "decode_step: head_dim must be 32, 64 or 128");
  if (n_kv < 1 || n_q < n_kv || n_q % n_kv) return ek_fail(hipErrorInvalidValue, "decode_step: bad head counts");
  const int64_t g = n_q / n_kv;
  // the Qwen3 dense models the plan's other bounds admit (hidden <= 4096:
  // 0.6B and 1.7B at 2, 4B and 8B at 4); other groups run the per-kernel step
  if (g != 2 && g != 4)
    return ek_fail(hipErrorInvalidValue, "decode_step: query heads per kv head must be 2 or 4");
  if (n_layers > eks::MAX_LAYERS)
    return ek_fail(hipErrorInvalidValue, "decode_step: at most 64 layers (the layer table is held in LDS)");
  if (n_layers < 1 || hidden < eks::CH || inter < eks::CH || vocab < 1 || hidden % eks::CH || inter % eks::CH ||
      (n_q * head_dim) % eks::CH)
    return ek_fail(hipErrorInvalidValue, "decode_step: hidden, intermediate and n_q * head_dim must be multiples of 512");
  if (hidden > 2 * eks::NGW * eks::SNT)
    return ek_fail(hipErrorInvalidValue, "decode_step: hidden must be at most 4096");
  if (hidden > (1 << 20) || inter > (1 << 20) || vocab > (1 << 30) || n_q * head_dim > (1 << 20))
    return ek_fail(hipErrorInvalidValue, "decode_step: sizes too large");
  if (s_cap < 1) return ek_fail(hipErrorInvalidValue, "decode_step: empty cache");
  p.nwg = step_grid();
  if (p.nwg < 1 || p.nwg > eks::MAX_WG) return ek_fail(hipErrorInvalidValue, "decode_step: unsupported device");
  if (m > 1) return make_batch_plan(hidden, inter, n_q, n_kv, head_dim, vocab, m, s_cap, n_layers, p);
  // Short rows run on attention-only workgroups beside the projections
  // (kUnitMaxKeys above); longer ones on every workgroup, the
  // keys of each kv head split S ways (S a power of two, at most 32 and at
  // most head_dim / 4, so that each split owns whole 4-value words of the
  // combined output)
  p.lsplit = p.lchunk = 0;
  p.lx = 0;
  if (s_cap > kUnitMaxKeys || g * s_cap * 4 > kFusedScoreLds) {
    int sp = 1;
    while (2 * sp <= 32 && 2 * sp <= head_dim / 4 && 2 * sp * n_kv <= p.nwg) sp *= 2;
    if (sp < 2) return ek_fail(hipErrorInvalidValue, "decode_step: too few workgroups for the long-context split");
    const int64_t chunk = (s_cap + sp - 1) / sp;
    if (chunk > (1 << 16))
      return ek_fail(hipErrorInvalidValue, "decode_step: the context's score rows exceed the LDS of the long-context split");
    p.lsplit = sp;
    p.lchunk = (int)chunk;
    p.lx = eks::long_words((int)n_kv, sp, (int)g, (int)head_dim);
  }
  const bool lng = p.lsplit > 0;
  const int n_attn = lng ? 0 : (int)(n_kv * (head_dim / eka::FDC));
  if (4 * n_attn > p.nwg) return ek_fail(hipErrorInvalidValue, "decode_step: too many attention units for the grid");
  const int qw = (int)(n_q * head_dim), qkvw = (int)((n_q + 2 * n_kv) * head_dim);
  int kmax = (int)hidden;
  kmax = kmax > qw ? kmax : qw;
  kmax = kmax > (int)inter ? kmax : (int)inter;
  p.kpad_max = eks::kpad_of(kmax);
  const int n_gemv = p.nwg - n_attn;   // projection workgroups
  p.o_rows = 4 * eks::cdiv_i((int)hidden / 4, n_gemv);
  p.part_max = eks::part_rows_max((int)hidden, (int)inter, qkvw, (int)vocab, n_gemv, p.o_rows);
  const size_t gemv = eka::align16((size_t)p.kpad_max * 2) + eka::align16((size_t)p.part_max * eks::SNW * 4);
  const size_t attn = lng ? long_lds((int)head_dim, (int)g, p.lchunk) : attn_lds((int)head_dim, (int)g, s_cap);
  p.lds = gemv > attn ? gemv : attn;
  if (p.lds > kLdsLimit)
    return ek_fail(hipErrorInvalidValue, lng ? "decode_step: the context's score rows exceed the LDS of the long-context split"
                                             : "decode_step: LDS plan exceeds the workgroup limit");
  p.half = eks::arena_half_words((int)n_layers, (int)hidden, (int)inter, qkvw, qw, p.nwg, 1, p.lx);
  p.arena_bytes = 16 * p.half;
  // every workgroup must be resident at once (the hand-over waits of one
  // need the others running): at least one workgroup of this instantiation,
  // with this LDS, per CU -- registers, scratch and LDS all counted
  if (resident_per_cu((int)head_dim, (int)g, lng, p.lds) < 1)
    return ek_fail(hipErrorInvalidValue, "decode_step: one workgroup per CU does not fit (registers or LDS)");
  return hipSuccess;
}

}  // namespace

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, resolved once per device (with
// that device current) and kept.
hipError_t static_scratch(unsigned char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return ek_fail(e, "decode_step_noalloc: no current device");
  if (dev < 0 || dev >= kMaxDevices) return ek_fail(hipErrorInvalidValue, "decode_step_noalloc: device index too large");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return ek_fail(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                                "decode_step_noalloc: the static scratch has no device address");
    g_scratch_ptr[dev] = static_cast<unsigned char*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

// The launch behind both decode-step entry points; arena/barrier: the
// hand-over arena and launch-state block (the caller's, or the static scratch).
hipError_t decode_step_impl(const int64_t* layer_ptrs, int64_t n_layers, int64_t hidden,
                            int64_t inter, int64_t n_q, int64_t n_kv, int64_t head_dim, int64_t vocab, int64_t m,
                            float eps, float sm_scale, const void* embed, int64_t lde, const void* lm_head,
                            const void* final_norm, const void* cos, const void* sin, int64_t ld_cs, int64_t rope_len,
                            int64_t csb, int64_t csh, int64_t css, int64_t s_cap, int64_t* tokens,
                            int64_t* positions, int64_t* len_t, int64_t* slot_t, const int32_t* start_t,
                            int32_t* out_buf, int64_t* step_idx, int64_t max_steps, int64_t* out_tok, void* logits,
                            void* arena, int64_t arena_bytes, void* barrier, int* err, hipStream_t st) {
  Plan p;
  hipError_t e = make_plan(hidden, inter, n_q, n_kv, head_dim, vocab, m, s_cap, n_layers, p);
  if (e != hipSuccess) return e;
  if (!layer_ptrs || !embed || !lm_head || !final_norm || !cos || !sin || !tokens || !positions || !len_t ||
      !slot_t || !start_t || !out_buf || !step_idx || !arena || !barrier || !err)
    return ek_fail(hipErrorInvalidValue, "decode_step: null pointer argument");
  const int64_t half = eks::arena_half_of(arena_bytes);
  if (half < p.half) return ek_fail(hipErrorInvalidValue, "decode_step: arena smaller than the plan");
  if (rope_len < 1 || ld_cs < head_dim || lde < hidden || css % 8 || csh % 8 || csb % 8 ||
      (reinterpret_cast<uintptr_t>(arena) & 15) || (reinterpret_cast<uintptr_t>(embed) & 15))
    return ek_fail(hipErrorInvalidValue, "decode_step: bad strides or alignment");
  eks::StepArgs a;
  memset(&a, 0, sizeof(a));
  a.lw = layer_ptrs; a.nl = (int)n_layers; a.h = (int)hidden; a.inter = (int)inter; a.nq = (int)n_q;
  a.nkv = (int)n_kv; a.vocab = (int)vocab; a.eps = eps; a.sm_scale = sm_scale;
  a.embed = (const bf16_t*)embed; a.lde = lde; a.lm_head = (const bf16_t*)lm_head;
  a.fnorm = (const bf16_t*)final_norm; a.cos = (const bf16_t*)cos; a.sin = (const bf16_t*)sin;
  a.ld_cs = ld_cs; a.rope_len = rope_len; a.csb = csb; a.csh = csh; a.css = css; a.s_cap = s_cap;
  a.tokens = tokens; a.positions = positions; a.len_t = len_t; a.slot_t = slot_t; a.start_t = start_t;
  a.out_buf = out_buf; a.step_idx = step_idx; a.max_steps = max_steps; a.out_tok = out_tok;
  a.logits = (bf16_t*)logits;
  a.arena = (eks::llw_t*)arena;
  a.half = half;
  a.bar = (eks::Bar*)barrier; a.err = err; a.spin = ek_wait_limit(kSpin);
  a.kpad_max = p.kpad_max; a.part_max = p.part_max; a.o_rows = p.o_rows;
  a.lsplit = p.lsplit; a.lchunk = p.lchunk; a.lx = p.lx;
  a.m = (int)m;
  const int g = (int)(n_q / n_kv);
  if (p.mb > 1) {
    switch (p.mb) {
      case 2: return eks::launch_bstep<2>(a, g, p.nwg, st);
      case 4: return eks::launch_bstep<4>(a, g, p.nwg, st);
      default: return eks::launch_bstep<8>(a, g, p.nwg, st);
    }
  }
  switch (head_dim) {
    case 32: return eks::launch_step<32>(a, g, p.nwg, st);
    case 64: return eks::launch_step<64>(a, g, p.nwg, st);
    default: return eks::launch_step<128>(a, g, p.nwg, st);
  }
}

}  // namespace

extern "C" {

int ek_decode_step_plan(int64_t hidden, int64_t inter, int64_t n_q, int64_t n_kv, int64_t head_dim, int64_t vocab,
                        int64_t m, int64_t s_cap, int64_t n_layers, int64_t* sizes) {
  EK_GUARD();
  Plan p;
  hipError_t e = make_plan(hidden, inter, n_q, n_kv, head_dim, vocab, m, s_cap, n_layers, p);
  if (e != hipSuccess) return e;
  if (sizes) {
    sizes[0] = p.arena_bytes;
    sizes[1] = p.lsplit;
    sizes[2] = (int64_t)sizeof(eks::Bar);
    sizes[3] = p.nwg;
  }
  return hipSuccess;
}


int ek_decode_step(const int64_t* layer_ptrs, int64_t n_layers, int64_t hidden, int64_t inter, int64_t n_q,
                   int64_t n_kv, int64_t head_dim, int64_t vocab, int64_t m, float eps, float sm_scale,
                   const void* embed, int64_t lde, const void* lm_head, const void* final_norm, const void* cos,
                   const void* sin, int64_t ld_cs, int64_t rope_len, int64_t csb, int64_t csh, int64_t css,
                   int64_t s_cap, int64_t* tokens, int64_t* positions, int64_t* len_t, int64_t* slot_t,
                   const int32_t* start_t, int32_t* out_buf, int64_t* step_idx, int64_t max_steps, int64_t* out_tok,
                   void* logits, void* arena, int64_t arena_bytes, void* barrier, int* err, void* stream) {
  EK_GUARD();
  return decode_step_impl(layer_ptrs, n_layers, hidden, inter, n_q, n_kv, head_dim, vocab, m, eps,
                          sm_scale, embed, lde, lm_head, final_norm, cos, sin, ld_cs, rope_len, csb, csh, css, s_cap,
                          tokens, positions, len_t, slot_t, start_t, out_buf, step_idx, max_steps, out_tok, logits,
                          arena, arena_bytes, barrier, err, (hipStream_t)stream);
}

int ek_decode_step_noalloc(const int64_t* layer_ptrs, int64_t n_layers, int64_t hidden, int64_t inter, int64_t n_q,
                           int64_t n_kv, int64_t head_dim, int64_t vocab, int64_t m, float eps, float sm_scale,
                           const void* embed, int64_t lde, const void* lm_head, const void* final_norm,
                           const void* cos, const void* sin, int64_t ld_cs, int64_t rope_len, int64_t csb,
                           int64_t csh, int64_t css, int64_t s_cap, int64_t* tokens, int64_t* positions,
                           int64_t* len_t, int64_t* slot_t, const int32_t* start_t, int32_t* out_buf,
                           int64_t* step_idx, int64_t max_steps, int64_t* out_tok, void* logits, int* err,
                           void* stream) {
  EK_GUARD();
  Plan p;
  hipError_t e = make_plan(hidden, inter, n_q, n_kv, head_dim, vocab, m, s_cap, n_layers, p);
  if (e != hipSuccess) return e;
  if ((size_t)p.arena_bytes > kStaticArenaBytes)
    return ek_fail(hipErrorInvalidValue, "decode_step_noalloc: this shape's hand-over arena exceeds the static 16 MiB "
                                         "(use decode_step with an arena)");
  unsigned char* base = nullptr;
  e = static_scratch(&base);
  if (e != hipSuccess) return e;
  return decode_step_impl(layer_ptrs, n_layers, hidden, inter, n_q, n_kv, head_dim, vocab, m, eps, sm_scale, embed,
                          lde, lm_head, final_norm, cos, sin, ld_cs, rope_len, csb, csh, css, s_cap, tokens,
                          positions, len_t, slot_t, start_t, out_buf, step_idx, max_steps, out_tok, logits,
                          base + kStaticBarBytes, (int64_t)kStaticArenaBytes, base, err, (hipStream_t)stream);
}

}  // extern "C"
