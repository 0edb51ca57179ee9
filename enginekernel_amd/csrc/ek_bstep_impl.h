// The persistent decode step at 2..8 batch rows: one launch per step, every
// workgroup running every phase (engine.py:284-292 for B rows, the body the
// reference captures: ek_model.py:360-416 decode + :490-493 argmax_token +
// the tokens/positions/out_buf/step_idx advance).
//
// Per layer, on every workgroup (one per CU), for MB rows at once:
//   wait dn words of the MB rows; r += dn; RMSNorm   (layer 0: the embedding rows)
//   qkv rows: each weight chunk against the MB activation chunks in LDS -> qkv words
//   split attention: unit (row b, kv head h, key split s) = workgroup
//     b (n_kv S) + s n_kv + h, the batch-1 split kernel's unit (long_attention)
//   wait att words; o rows -> o words; wait o words; r += o; RMSNorm
//   gate/up rows + SwiGLU -> act words
//   down rows over the act row in K slices of bstep_slice(MB) chunks (up to
//     4 rows the whole of a 9728-wide act row; 8 such rows do not fit the
//     LDS at once): wait the slice's act words, its partial products added
//     into the same per-wave partials
//   -> dn words
// then the final add + norm, the lm_head rows (whole rows per wave, so each
// wave keeps a running first-index argmax per batch row instead of per-row
// partials) and the argmax words; workgroup 0 reduces them and advances the
// step state of every row.
//
// Weights are read once per step whatever MB is: from 4 rows up each 1 KiB
// weight load (4 rows x 256 B) meets the MB activation rows (LDS) on
// v_mfma_f32_4x4x4_16b_bf16; at 2 rows each 16-byte weight chunk meets the
// 2 activation chunks on the bf16 dot instruction. The residual rows are
// kept in LDS as bf16 (every add rounds to bf16, so this is exact), one per
// batch row. Rows past the launch's m (MB is m rounded up to 2, 4 or 8)
// compute on whatever their LDS rows hold and are never stored.
#pragma once

#include "ek_step_impl.h"

namespace eks {

constexpr int BLLW = 16;      // tagged (argmax) words in flight per thread
// Weight items in flight per wave (the batch kernel's ring; the batch-1
// kernel's is NB), and how many of them are prefetched ahead of a hand-over
// wait. Config 5 (8 rows, the ring / the prefetch): 5 / 5 measured 2.50 ms,
// 4 / 4 2.51, 6 / 6 2.51, 6 / 4 2.56, 8 / 8 2.54, 8 / 6 2.64; rings of 10 or
// 12 items, 3.8-4.4 % slower than 8. Fewer bytes in flight per wave leave
// the hand-over polls, which return behind them, less to wait for.
#ifndef EK_BSTEP_NB
#define EK_BSTEP_NB 5
#endif
#ifndef EK_BSTEP_PF
#define EK_BSTEP_PF 5
#endif
// units of a projection's share come in pairs of rows: 2560 rows over 256
// workgroups are then 10 rows each, where 4-row units gave 8 or 12 (the
// phase ends with the 12-row shares: 0.7-1.1 us later than the 8-row ones)
constexpr int BGRAN = 2;
constexpr int BNB = EK_BSTEP_NB;
constexpr int BPF = EK_BSTEP_PF;
using BRing = RingN<BNB>;
// activation chunks per LDS slice of a row in the down projection: up to 4
// rows 20 (10240 bf16: a 9728-wide act row in one slice, so the phase has no
// slice boundary, where the ring drains and the next act words make a round
// trip: 3.3-3.7 us each); 8 rows hold 10 (5120 bf16) beside their residual rows
#ifndef EK_BSTEP_SLICE
#define EK_BSTEP_SLICE 10
#endif
#ifndef EK_BSTEP_SLICE_NARROW
#define EK_BSTEP_SLICE_NARROW 20
#endif
__host__ __device__ constexpr int bstep_slice(int mb) { return mb <= 4 ? EK_BSTEP_SLICE_NARROW : EK_BSTEP_SLICE; }
// a K slice's act words are loaded ahead of the previous slice's products
// when they take at most this many 16-byte units per thread and a kv head has
// at most 4 q heads (beyond either, the extra registers spill)
#ifndef EK_BSTEP_EARLY_UNITS
#define EK_BSTEP_EARLY_UNITS 5
#endif
// dense 16-byte units in flight per thread: MB for the rows up to 4096 wide,
// and one K slice of MB act rows in one round
template <int MB>
constexpr int bstep_slice_units() { return (MB * bstep_slice(MB) * CH / 8 + SNT - 1) / SNT; }

// ---------------------------------------------------------------------------
// projections over 2 activation rows, on the bf16 dot instruction
// ---------------------------------------------------------------------------
// (2 rows would fill half of every matrix-core product's columns: the dot
// instruction does their products in fewer issue slots.) A wave's items of
// one phase: item i -> (row i / C, chunk i % C) of the workgroup's share,
// gate rows then up rows for a pair phase; rows are ldw elements apart (ldw
// > K for a K slice of a wider matrix).
struct BSpan {
  const bf16_t* g;    // row u0 of the share
  const bf16_t* up;   // row up_off + u0 (pair phases)
  int nu;             // rows of the first half (every row of a plain phase)
  int C;
  int64_t ldw;
  int i0, n;          // this wave's items [i0, i0 + n)
};

// by_rows: the wave's items are whole rows (rows split evenly over the waves)
__device__ __forceinline__ BSpan make_bspan(const Gp& P, int64_t ldw, int wave, bool by_rows) {
  int u0, u1;
  unit_range(P, u0, u1);
  const int nu = u1 - u0;
  BSpan s;
  s.g = P.w + (int64_t)u0 * ldw;
  s.up = P.pair ? P.w + (int64_t)(P.up_off + u0) * ldw : s.g;
  s.nu = P.pair ? nu : 0x7fffffff;
  s.C = P.C;
  s.ldw = ldw;
  if (by_rows) {
    const int r0 = (int)((uint32_t)nu * (uint32_t)wave / (uint32_t)SNW);
    const int r1 = (int)((uint32_t)nu * (uint32_t)(wave + 1) / (uint32_t)SNW);
    s.i0 = r0 * P.C;
    s.n = (r1 - r0) * P.C;
  } else {
    const WaveItems w = wave_items(P, nu, wave);
    s.i0 = w.i0;
    s.n = w.n;
  }
  return s;
}

__device__ __forceinline__ const bf16_t* bspan_at(const BSpan& s, int r, int c) {
  return (r < s.nu ? s.g + (int64_t)r * s.ldw : s.up + (int64_t)(r - s.nu) * s.ldw) + c * CH;
}

template <int CNT>
__device__ __forceinline__ void prefetch_rows(const Gp& P, int64_t ldw, bool by_rows, BRing& ring) {
  static_assert(CNT <= BNB, "prefetch within the ring");
  const BSpan s = make_bspan(P, ldw, wave_id(), by_rows);
  const int loff = (opaque_tid() & 63) * 8;
  int r = s.i0 / s.C, c = s.i0 - (s.i0 / s.C) * s.C;
#pragma unroll
  for (int u = 0; u < CNT; ++u) {
    ring.r[u] = ld16_nt(bspan_at(s, r, c) + loff);
    if (u + 1 < s.n && ++c == s.C) { c = 0; ++r; }
  }
  ring.nready = CNT;
}

// The wave's row sums over MB activation rows, handed per finished row (or
// row part, where a wave's items start or end inside a row) to
// sink.row(row, acc), in lane 63. Each weight chunk meets the MB rows'
// chunks at the same k, read from LDS one item ahead. The ring works as in
// gemv_phase.
template <int MB, typename SINK>
__device__ __forceinline__ void gemv_rows(const Gp& P, int64_t ldw, bool by_rows, BRing& ring, const bf16_t* xs,
                                          int xstride, SINK& sink) {
  const int lane = opaque_tid() & 63, wave = wave_id();
  const BSpan sp = make_bspan(P, ldw, wave, by_rows);
  const int n = sp.n, C = sp.C;
  const int loff = lane * 8;
  // refill cursor: the item BNB places ahead of the one consumed (the last
  // item again past the end)
  int rf = sp.i0 / C, cf = sp.i0 - (sp.i0 / C) * C;
#pragma unroll
  for (int u = 0; u < BNB; ++u) {
    if (u >= ring.nready) ring.r[u] = ld16_nt(bspan_at(sp, rf, cf) + loff);
    if (u + 1 < n && ++cf == C) { cf = 0; ++rf; }
  }
  int kf = BNB < n ? BNB : n - 1;   // item index of the cursor
  int r = sp.i0 / C, ch = sp.i0 - (sp.i0 / C) * C;
  uint4 xc[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) xc[m] = *reinterpret_cast<const uint4*>(xs + m * xstride + ch * CH + loff);
  float acc[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) acc[m] = 0.f;
  auto flush = [&](int row) {
    wave_sums_dpp_lane63<MB>(acc);
    if (lane == 63) sink.row(row, acc);
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[m] = 0.f;
  };
  auto step = [&](const uint4& w) {
    const int chn = ch + 1 == C ? 0 : ch + 1;
    uint4 xn[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) xn[m] = *reinterpret_cast<const uint4*>(xs + m * xstride + chn * CH + loff);
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[m] = step_dot8(w, xc[m], acc[m]);
#pragma unroll
    for (int m = 0; m < MB; ++m) xc[m] = xn[m];
  };
  int k0 = 0;
  for (; k0 + BNB <= n; k0 += BNB) {
#pragma unroll
    for (int u = 0; u < BNB; ++u) {
      step(ring.r[u]);
      ring.r[u] = ld16_nt(bspan_at(sp, rf, cf) + loff);
      if (kf + 1 < n) {
        ++kf;
        if (++cf == C) { cf = 0; ++rf; }
      }
      if (ch == C - 1) flush(r);
      if (++ch == C) { ch = 0; ++r; }
    }
  }
#pragma unroll
  for (int u = 0; u < BNB; ++u) {
    if (k0 + u < n) {
      step(ring.r[u]);
      if (ch == C - 1 || k0 + u == n - 1) flush(r);
      if (++ch == C) { ch = 0; ++r; }
    }
  }
  if (k0 == n && n > 0 && ch != 0) flush(r);   // the wave's items ended inside a row at a ring edge
  ring.nready = 0;
}

// ---------------------------------------------------------------------------
// projections over MB activation rows, on the matrix cores
// ---------------------------------------------------------------------------
// v_mfma_f32_4x4x4_16b_bf16: 16 blocks of 4 lanes, lane l = 4 blk + j holds
// A[blk][row j][4 k], B[blk][4 k][column j] and C[blk][rows 0..3][column j].
// A tile is 4 weight rows of the workgroup's share and an item one 128-wide
// K chunk of a tile: lanes 16 r .. 16 r + 15 load the 256 contiguous bytes
// of row r (1 KiB per load instruction, the pattern HBM streams best; the
// MFMA layout's interleaved rows stream markedly slower), and four
// ds_bpermute move piece blk of row j to lane 4 blk + j. Two MFMAs per
// column group (4 batch rows) take the piece's two 4-k halves against the
// batch rows' 16 bytes at the same k, read from the LDS activation rows
// (rows >= MB repeat a real row; their outputs are dropped). Block blk
// accumulates k offsets 8 blk .. 8 blk + 7 of every chunk of the tile; at
// the tile's end (or at the wave's last item inside it) tile_sum adds the
// 16 blocks. A phase has as many items as 1 KiB chunks of its rows, split
// over the waves as evenly as the rows' chunks were.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
using eka::f32x4_t;
constexpr int MT = 4;      // weight rows per tile
constexpr int MCH = 128;   // K per tile chunk (one 16-byte load per lane)

__device__ __forceinline__ f32x4_t mfma4x4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f32x4_t c) {
  const s16x4_t a = __builtin_bit_cast(s16x4_t, make_uint2(a0, a1));
  const s16x4_t b = __builtin_bit_cast(s16x4_t, make_uint2(b0, b1));
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 0, 0, 0);
}

// The 16 blocks' sum of one column group's accumulator: lane l gets row
// l / 16 of column l % 4. Rows 0 / 2 and 1 / 3 meet across the wave's
// halves (blocks b and b + 8, one permlane32 swap each), then 0 / 1 and 2 / 3
// across 16-lane rows (blocks b and b + 4, one permlane16 swap), then the 4
// blocks of a 16-lane row (two DPP rotations). The order is fixed.
__device__ __forceinline__ float tile_sum(f32x4_t a) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[0]), __float_as_uint(a[2]), false, false);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[1]), __float_as_uint(a[3]), false, false);
  const float s0 = __uint_as_float(p[0]) + __uint_as_float(p[1]);   // lanes < 32: row 0, else row 2
  const float s1 = __uint_as_float(q[0]) + __uint_as_float(q[1]);   // lanes < 32: row 1, else row 3
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(s0), __float_as_uint(s1), false, false);
  float v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  v = dpp_plus<0x128>(v);   // row_ror:8
  v = dpp_plus<0x124>(v);   // row_ror:4
  return v;
}

// A wave's items of one phase: item i -> (tile i / C4, chunk i % C4) of the
// workgroup's share, gate tiles then up tiles for a pair phase; rows are ldw
// elements apart (ldw > K for a K slice of a wider matrix). Rows past rmax
// (relative to their half) re-read it: a share's rows past the matrix (the
// lm_head's last tile) and the clamped cursors past a wave's last item.
struct TSpan {
  const bf16_t* g;    // row u0 of the share, this lane's k offset (16-byte piece lane % 16)
  const bf16_t* up;   // row up_off + u0 (pair phases), the same offset
  int tg;             // tiles of the first half (every tile of a plain phase)
  int C4;             // chunks per tile
  int rmax;
  int64_t ldw;
  int i0, n;          // this wave's items [i0, i0 + n)
};

// by_rows: the wave's items are whole tiles (tiles split evenly over the
// waves); rows_end: the matrix's rows (the lm_head's share may pass them)
// (Every count is pinned to a scalar register: the compiler cannot prove
// them wave-uniform after the kernel's earlier divergent loops, and would
// otherwise keep the cursors in vector registers behind exec-mask branches.)
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ TSpan make_tspan(const Gp& P, int64_t ldw, int wave, bool by_rows, int rows_end) {
  int u0, u1;
  unit_range(P, u0, u1);
  u0 = uni(u0);
  u1 = uni(u1);
  // the share's rows: a multiple of the phase's granularity (2 rows, or MT
  // for the lm_head); a last tile past them re-reads the share's last row
  // (an L2 hit) and its sums are dropped
  const int nu = u1 - u0;
  const int nt = cdiv_i(nu, MT);   // tiles of a half
  TSpan s;
  const int lpc = opaque_tid() & 15;
  s.g = P.w + (int64_t)u0 * ldw + lpc * 8;
  s.up = P.pair ? P.w + (int64_t)(P.up_off + u0) * ldw + lpc * 8 : s.g;
  s.tg = uni(P.pair ? nt : 0x7fffffff);
  s.C4 = uni(P.K / MCH);
  const int re = (rows_end < u1 ? rows_end : u1) - u0 - 1;
  s.rmax = uni(re > 0 ? re : 0);   // a share without rows re-reads its first row
  s.ldw = ldw;
  if (by_rows) {
    const int t0 = (int)((uint32_t)nt * (uint32_t)wave / (uint32_t)SNW);
    const int t1 = (int)((uint32_t)nt * (uint32_t)(wave + 1) / (uint32_t)SNW);
    s.i0 = uni(t0 * s.C4);
    s.n = uni((t1 - t0) * s.C4);
  } else {
    // the (tile, chunk) items of both halves, split evenly over the waves
    const uint32_t ni = (uint32_t)((P.pair ? 2 : 1) * nt * s.C4);
    const int i0 = (int)(ni * (uint32_t)wave / (uint32_t)SNW);
    const int i1 = (int)(ni * (uint32_t)(wave + 1) / (uint32_t)SNW);
    s.i0 = uni(i0);
    s.n = uni(i1 - i0);
  }
  return s;
}

// this lane's load address in tile t (chunk 0): row 4 t + lane / 16
__device__ __forceinline__ const bf16_t* tile_at(const TSpan& s, int t) {
  const bool gate = t < s.tg;
  int r = MT * (gate ? t : t - s.tg) + ((opaque_tid() & 63) >> 4);
  r = r < s.rmax ? r : s.rmax;
  return (gate ? s.g : s.up) + (int64_t)r * s.ldw;
}

template <int CNT>
__device__ __forceinline__ void prefetch_tiles(const Gp& P, int64_t ldw, bool by_rows, BRing& ring, int rows_end) {
  static_assert(CNT <= BNB, "prefetch within the ring");
  const TSpan s = make_tspan(P, ldw, wave_id(), by_rows, rows_end);
  int t = s.i0 / s.C4, c = s.i0 - (s.i0 / s.C4) * s.C4;
  const bf16_t* tp = tile_at(s, t);
#pragma unroll
  for (int u = 0; u < CNT; ++u) {
    ring.r[u] = ld16_nt(tp + c * MCH);
    if (u + 1 < s.n && ++c == s.C4) { c = 0; ++t; tp = tile_at(s, t); }
  }
  ring.nready = CNT;
}

// The wave's sums over MB activation rows, handed per finished tile (or
// tile part, where a wave's items start or end inside a tile) to sink(t,
// v): lane l holds v[c] = row 4 t + l / 16 (of the share), batch row 4 c +
// l % 4. PartWriter stores (or, for the K slices of one matrix, adds) them
// as per-wave partials, ArgmaxSink (lm_head, whole tiles per wave) keeps a
// running argmax. The ring works as in gemv_phase: slot u holds the item
// BNB places ahead, refilled as soon as its words are moved to the MFMA
// layout.
template <int MB, typename SINK>
__device__ __forceinline__ void gemv_tiles(const Gp& P, int64_t ldw, bool by_rows, BRing& ring, const bf16_t* xs,
                                           int xld, SINK& sink, int rows_end) {
  constexpr int CG = MB > 4 ? 2 : 1;   // column groups of 4 batch rows
  const int lane = opaque_tid() & 63;
  const int blk = lane >> 2, j4 = lane & 3;
  const int src = (16 * j4 + blk) * 4;   // ds_bpermute source: row j4's piece blk
  const TSpan sp = make_tspan(P, ldw, wave_id(), by_rows, rows_end);
  const int n = sp.n, C4 = sp.C4;
  // refill cursor: the item BNB places ahead of the one consumed (the last
  // item again past the end)
  int tf = sp.i0 / C4, cf = sp.i0 - (sp.i0 / C4) * C4;
  const bf16_t* tpf = tile_at(sp, tf);
#pragma unroll
  for (int u = 0; u < BNB; ++u) {
    if (u >= ring.nready) ring.r[u] = ld16_nt(tpf + cf * MCH);
    if (u + 1 < n && ++cf == C4) { cf = 0; ++tf; tpf = tile_at(sp, tf); }
  }
  int kf = BNB < n ? BNB : n - 1;   // item index of the cursor
  int t = sp.i0 / C4, ch = sp.i0 - (sp.i0 / C4) * C4;
  const bf16_t* xr[CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) xr[c] = xs + ((4 * c + j4) & (MB - 1)) * xld + blk * 8;
  f32x4_t acc[CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto flush = [&](int tile) {
    float v[CG];
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      v[c] = tile_sum(acc[c]);
      acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    sink.tile(tile, v);
  };
  // one item: its weights into the MFMA layout, then the slot's refill,
  // then the products
  auto step = [&](uint4& slot, bool refill) {
    uint4 xv[CG];
#pragma unroll
    for (int c = 0; c < CG; ++c) xv[c] = *reinterpret_cast<const uint4*>(xr[c] + ch * MCH);
    uint4 w;
    w.x = __builtin_amdgcn_ds_bpermute(src, (int)slot.x);
    w.y = __builtin_amdgcn_ds_bpermute(src, (int)slot.y);
    w.z = __builtin_amdgcn_ds_bpermute(src, (int)slot.z);
    w.w = __builtin_amdgcn_ds_bpermute(src, (int)slot.w);
    if (refill) {
      slot = ld16_nt(tpf + cf * MCH);
      if (kf + 1 < n) {
        ++kf;
        if (++cf == C4) { cf = 0; ++tf; tpf = tile_at(sp, tf); }
      }
    }
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      acc[c] = mfma4x4(w.x, w.y, xv[c].x, xv[c].y, acc[c]);
      acc[c] = mfma4x4(w.z, w.w, xv[c].z, xv[c].w, acc[c]);
    }
  };
  int k0 = 0;
  for (; k0 + BNB <= n; k0 += BNB) {
#pragma unroll
    for (int u = 0; u < BNB; ++u) {
      step(ring.r[u], true);
      if (ch == C4 - 1) flush(t);
      if (++ch == C4) { ch = 0; ++t; }
      // keep each slot's refill where it is: the scheduler would otherwise
      // sink the refills below later items' products and drain the ring
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int u = 0; u < BNB; ++u) {
    if (k0 + u < n) {
      step(ring.r[u], false);
      if (ch == C4 - 1 || k0 + u == n - 1) flush(t);
      if (++ch == C4) { ch = 0; ++t; }
    }
  }
  if (k0 == n && n > 0 && ch != 0) flush(t);   // the wave's items ended inside a tile at a ring edge
  ring.nready = 0;
}

// the batch's projections: matrix-core tiles from 4 rows up, the dot
// instruction at 2 rows; rows_end: the matrix's rows, where a tile share
// may pass them (the lm_head's)
template <int MB>
constexpr bool bstep_mfma() { return MB >= 4; }

template <int MB, int CNT>
__device__ __forceinline__ void prefetch_phase_b(const Gp& P, int64_t ldw, bool by_rows, BRing& ring,
                                                 int rows_end = 0x7fffffff) {
  if constexpr (bstep_mfma<MB>()) prefetch_tiles<CNT>(P, ldw, by_rows, ring, rows_end);
  else prefetch_rows<CNT>(P, ldw, by_rows, ring);
}

template <int MB, typename SINK>
__device__ __forceinline__ void gemv_phase_b(const Gp& P, int64_t ldw, bool by_rows, BRing& ring, const bf16_t* xs,
                                             int xld, SINK& sink, int rows_end = 0x7fffffff) {
  if constexpr (bstep_mfma<MB>()) gemv_tiles<MB>(P, ldw, by_rows, ring, xs, xld, sink, rows_end);
  else gemv_rows<MB>(P, ldw, by_rows, ring, xs, xld, sink);
}

template <int MB, bool ACC>
struct PartWriter {   // part[(row * MB + m) * SNW + wave] (+)= the row's sum for batch row m
  float* part;
  int wave;
  __device__ void row(int r, const float* acc) {   // lane 63: acc[m] of batch row m
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      float* p = part + (r * MB + m) * SNW + wave;
      *p = ACC ? *p + acc[m] : acc[m];
    }
  }
  __device__ void tile(int t, const float* v) {    // every lane: v[c] of row 4 t + lane / 16, batch row 4 c + lane % 4
    const int lane = opaque_tid() & 63;
    if ((lane & 12) != 0) return;   // one lane of each 16-lane row
    const int r = MT * t + (lane >> 4);
#pragma unroll
    for (int c = 0; c < (MB > 4 ? 2 : 1); ++c) {
      const int m = 4 * c + (lane & 3);
      if (m < MB) {
        float* p = part + (r * MB + m) * SNW + wave;
        *p = ACC ? *p + v[c] : v[c];
      }
    }
  }
};

template <int MB>
// the waves' partials of one (row, batch row), contiguous: two 16-byte LDS
// reads, added in wave order
__device__ __forceinline__ float row_sum_b(const float* part, int r, int m) {
  static_assert(SNW == 8, "two 16-byte reads per row sum");
  const float4* p = reinterpret_cast<const float4*>(part + (r * MB + m) * SNW);
  const float4 a = p[0], b = p[1];
  return ((((((a.x + a.y) + a.z) + a.w) + b.x) + b.y) + b.z) + b.w;
}

// row m's dense word (u0 + 4i) / 4 at out + m * rw + u0 / 4 + i, rows m < nrows
template <int MB>
// The share's rows [u0, u1) come in pairs (the phases' granularity is 2
// rows): pair q of batch row m is the half-word of values u0 + 2 q, +1 of
// that row's words, stored on its own (a word's other half may be another
// workgroup's).
__device__ __forceinline__ void epilogue_ll_b(const Gp& P, const float* part, llw_t* out, int64_t rw, int nrows) {
  int u0, u1;
  unit_range(P, u0, u1);
  const int np = (u1 - u0) / 2;
  for (int i = threadIdx.x; i < np * nrows; i += SNT) {
    const int m = i / np, q = i - m * np;
    dw_put1(reinterpret_cast<uint32_t*>(out + m * rw) + u0 / 2 + q,
            pack2(row_sum_b<MB>(part, 2 * q, m), row_sum_b<MB>(part, 2 * q + 1, m)));
  }
}

template <int MB>
__device__ __forceinline__ float swiglu_one_b(const float* part, int nu, int ul, int m) {
  const float gt = rbf(row_sum_b<MB>(part, ul, m));
  const float up = rbf(row_sum_b<MB>(part, nu + ul, m));
  const float s = rbf(gt / (1.0f + expf(-gt)));
  return s * up;
}

// The up rows' partials start at row `nu` of the share on the dot path
// and at its gate tiles' rows (nu rounded up to MT) on the tiles.
template <int MB>
__device__ __forceinline__ void epilogue_swiglu_ll_b(const Gp& P, const float* part, llw_t* out, int64_t rw,
                                                     int nrows) {
  int u0, u1;
  unit_range(P, u0, u1);
  const int nu = u1 - u0, np = nu / 2;
  const int upo = bstep_mfma<MB>() ? MT * cdiv_i(nu, MT) : nu;
  for (int i = threadIdx.x; i < np * nrows; i += SNT) {
    const int m = i / np, q = i - m * np;
    dw_put1(reinterpret_cast<uint32_t*>(out + m * rw) + u0 / 2 + q,
            pack2(swiglu_one_b<MB>(part, upo, 2 * q, m), swiglu_one_b<MB>(part, upo, 2 * q + 1, m)));
  }
}

// rr (bf16 pairs, [MB][k / 2]) = bf16(rr + x) for rows m < nrows (x pairs
// [m][k / 2] in xw, or no add when xw is null); xs row m (xstride apart) =
// bf16(w * bf16(rr * rsqrt(mean(rr^2) + eps)))   (ek_kernels.py:1025-1059).
// Row m belongs to the WPR = 8 / MB waves m WPR .. m WPR + WPR - 1, which take
// its 16-byte pieces (8 values) in turn, 64 at a time (k is a multiple of
// 512, so every round is whole for a wave). One barrier: it separates the
// residual update and the row sums of squares (pass 1, which reads the
// staged words in xw) from the output (pass 2, which may overwrite them: xs
// and xw share the LDS), and carries the waves' partial sums (red, fixed
// order). The gain words come from the registers gw (thread t: words
// t + j SNT) via the LDS row gl.
template <int MB>
__device__ __forceinline__ void add_norm_rows(uint32_t* rr, const uint32_t* xw, const uint32_t* gw, uint32_t* gl,
                                              int k, int nrows, float eps, bf16_t* xs, int xstride, float* red) {
  static_assert(MB <= SNW && SNW % MB == 0, "whole waves per row");
  constexpr int WPR = SNW / MB;
  const int tid = opaque_tid(), lane = tid & 63, wave = wave_id();
  const int m = wave / WPR, part = wave - m * WPR;
  const int nw = k / 2, n4 = k / 8;   // words, 16-byte pieces of a row
#pragma unroll
  for (int j = 0; j < NGW; ++j) {
    const int i = tid + j * SNT;
    if (i < nw) gl[i] = gw[j];
  }
  const int i0 = part * EK_WAVE + lane;
  if (m < nrows) {
    uint4* rrow = reinterpret_cast<uint4*>(rr + m * nw);
    const uint4* xrow = reinterpret_cast<const uint4*>(xw + m * nw);
    float ss = 0.f;
#pragma unroll 4
    for (int i = i0; i < n4; i += WPR * EK_WAVE) {
      uint4 r = rrow[i];
      if (xw) {
        const uint4 x = xrow[i];
        r = make_uint4(add2_bf(r.x, x.x), add2_bf(r.y, x.y), add2_bf(r.z, x.z), add2_bf(r.w, x.w));
        rrow[i] = r;
      }
      ss = sq2(r.w, sq2(r.z, sq2(r.y, sq2(r.x, ss))));
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0) red[wave] = ss;
  }
  __syncthreads();
  if (m < nrows) {
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < WPR; ++q) t += red[m * WPR + q];
    const float rstd = 1.0f / sqrtf(t / (float)k + eps);
    const uint4* rrow = reinterpret_cast<const uint4*>(rr + m * nw);
    const uint4* grow = reinterpret_cast<const uint4*>(gl);
    uint4* xrow = reinterpret_cast<uint4*>(xs + m * xstride);
#pragma unroll 4
    for (int i = i0; i < n4; i += WPR * EK_WAVE) {
      const uint4 r = rrow[i], g = grow[i];
      xrow[i] = make_uint4(norm2(r.x, g.x, rstd), norm2(r.y, g.y, rstd), norm2(r.z, g.z, rstd), norm2(r.w, g.w, rstd));
    }
  }
}

// The residual hand-over and add_norm_rows in one pass over registers: thread
// t waits for units j = t + q SNT of the words at base (16 bytes, 8 values of
// row j / (k / 8); every unit once, so nrows * k / 8 <= W * SNT), adds each
// to its residual piece (rr, the same flat order) and sums the squares of the
// wave's 64 units of round q. k is a multiple of 512, so those 64 units lie
// in one row: their sum is chunk c = j / 64 of red, and row m's sum of
// squares is that of its k / 512 chunks, in order. The barrier of the error
// vote carries the chunk sums; the waited words never pass through LDS
// (config 5: 0.7 % faster than staging them for add_norm_rows; 2-6 rows
// 1.6-1.8 %). False (the error word set) when a wait runs out.
template <int MB, int W>
__device__ __forceinline__ bool dw_add_norm(const llw_t* base, uint32_t* rr, const uint32_t* gw, uint32_t* gl, int k,
                                            int nrows, float eps, bf16_t* xs, int xstride, float* red, int* s_fail,
                                            int* err, int64_t spin) {
  const int tid = opaque_tid(), lane = tid & 63;
  const int u_r = k / 8, n = nrows * u_r;
#pragma unroll
  for (int j = 0; j < NGW; ++j) {
    const int i = tid + j * SNT;
    if (i < k / 2) gl[i] = gw[j];
  }
  u32x4_t v[W];
  dw_issue<W>(base, LinUnits{}, n, v);
  const bool ok = dw_wait<W>(base, LinUnits{}, n, v, err, spin);
  uint4* rr4 = reinterpret_cast<uint4*>(rr);
  uint4 r[W];
  float ss[W];
#pragma unroll
  for (int q = 0; q < W; ++q) {
    const int j = tid + q * SNT;
    ss[q] = 0.f;
    if (j < n) {
      const uint4 o = rr4[j];
      r[q] = make_uint4(add2_bf(o.x, v[q].x ^ DW_FLIP32), add2_bf(o.y, v[q].y ^ DW_FLIP32),
                        add2_bf(o.z, v[q].z ^ DW_FLIP32), add2_bf(o.w, v[q].w ^ DW_FLIP32));
      rr4[j] = r[q];
      ss[q] = sq2(r[q].w, sq2(r[q].z, sq2(r[q].y, sq2(r[q].x, 0.f))));
    }
  }
  wave_sums_dpp_lane63<W>(ss);
  if (lane == 63) {
#pragma unroll
    for (int q = 0; q < W; ++q)
      if (tid + q * SNT < n) red[(tid + q * SNT) >> 6] = ss[q];
  }
  if (!wg_all(ok, s_fail)) return false;
  const int cpr = u_r >> 6;
  float rs = 0.f;
  if (lane < nrows) {
    float t = 0.f;
    for (int c = 0; c < cpr; ++c) t += red[lane * cpr + c];
    rs = 1.0f / sqrtf(t / (float)k + eps);
  }
  const uint4* g4 = reinterpret_cast<const uint4*>(gl);
  const int xs4 = xstride / 8;
  const uint32_t inv = (65536u + (uint32_t)cpr - 1u) / (uint32_t)cpr;
#pragma unroll
  for (int q = 0; q < W; ++q) {
    const int j = __builtin_amdgcn_readfirstlane(tid - lane + q * SNT);
    if (j < n) {
      const int m = (int)(((uint32_t)j >> 6) * inv >> 16);
      const float rstd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rs), m));
      const int c = j - m * u_r + lane;
      const uint4 g = g4[c];
      reinterpret_cast<uint4*>(xs)[m * xs4 + c] =
          make_uint4(norm2(r[q].x, g.x, rstd), norm2(r[q].y, g.y, rstd), norm2(r[q].z, g.z, rstd),
                     norm2(r[q].w, g.w, rstd));
    }
  }
  return true;
}

// lm_head rows of this wave (whole rows, or whole tiles): a running
// first-index argmax per batch row over the rows the lane receives (lane 63
// every row of the wave on the dot path; on the tiles, row 4 t + lane / 16
// of batch row 4 c + lane % 4 in one lane of each 16-lane row), and the
// optional logits. A lane's slot k holds batch row k (dot path) or 4 k +
// lane % 4 (tiles).
template <int MB>
struct ArgmaxSink {
  static constexpr int NS = bstep_mfma<MB>() ? (MB > 4 ? 2 : 1) : MB;
  float bv[NS];
  int bi[NS];
  bf16_t* logits;      // [nrows][vocab] or null
  int vocab, nrows, u0;
  __device__ void take(int k, int m, int idx, float v) {
    const float lv = rbf(v);
    if (logits && m < nrows) logits[(int64_t)m * vocab + idx] = (bf16_t)f2bf(lv);
    if (am_better(lv, idx, bv[k], bi[k])) { bv[k] = lv; bi[k] = idx; }
  }
  __device__ void row(int r, const float* acc) {
#pragma unroll
    for (int m = 0; m < MB; ++m) take(m, m, u0 + r, acc[m]);
  }
  __device__ void tile(int t, const float* v) {
    const int lane = opaque_tid() & 63;
    const int idx = u0 + MT * t + (lane >> 4);
    if ((lane & 12) != 0 || idx >= vocab) return;
#pragma unroll
    for (int c = 0; c < NS; ++c) take(c, 4 * c + (lane & 3), idx, v[c]);
  }
};

// ---------------------------------------------------------------------------
// the batch step
// ---------------------------------------------------------------------------
__host__ __device__ inline size_t bstep_rr_bytes(int mb, int h) { return eka::align16((size_t)mb * h * 2); }
// activation rows: MB rows of the widest LDS row (hidden, n_q D or a slice)
__host__ __device__ inline int bstep_xcols(int h, int qw, int mb) {
  int x = kpad_of(h);
  x = x > qw ? x : qw;
  x = x > bstep_slice(mb) * CH ? x : bstep_slice(mb) * CH;
  return x;
}
// their LDS stride (elements): rows EK_BSTEP_XPAD elements past a multiple
// of 512, so that the 4 batch rows one B-operand read takes at one k fall in
// different banks
#ifndef EK_BSTEP_XPAD
#define EK_BSTEP_XPAD 32
#endif
__host__ __device__ inline int bstep_xld(int h, int qw, int mb) { return bstep_xcols(h, qw, mb) + EK_BSTEP_XPAD; }
// part rows of the largest projection share (lm_head keeps no partials)
// partial rows of a workgroup: its share of a phase's units (BGRAN rows per
// unit) rounded up to whole tiles, twice for the gate/up pair
__host__ __device__ inline int bstep_share_rows(int units, int nwg) {
  return 4 * cdiv_i(BGRAN * cdiv_i(units / BGRAN, nwg), 4);
}
__host__ __device__ inline int bstep_part_rows(int h, int inter, int qkvw, int nwg) {
  int r = bstep_share_rows(qkvw, nwg);
  r = r > bstep_share_rows(h, nwg) ? r : bstep_share_rows(h, nwg);
  r = r > 2 * bstep_share_rows(inter, nwg) ? r : 2 * bstep_share_rows(inter, nwg);
  return r;
}

// Units (16 bytes) of nrows rows (rw dense words apart, the first su units
// of each) into LDS rows xw u32 apart: unit j -> row j / su, unit j % su
struct RowsUnits {
  int rw, su;
  __device__ int operator()(int j) const {
    const int m = j / su;
    return 8 * m * rw + 16 * (j - m * su);
  }
};
struct RowsLds {
  int su, xw;
  __device__ int operator()(int j) const {
    const int m = j / su;
    return m * xw + 4 * (j - m * su);
  }
};

// Key splits of the batch rows' attention (slots nwg / nkv per kv head, the
// rows taking consecutive slots): every
// row first takes the fewest splits that keep its keys per split within the
// plan's score row (a.lchunk; the plan guarantees that these fit the slots),
// then, while slots remain, the row with the most keys per split (the lowest
// row on ties) doubles its splits, up to min(32, D / 4). Every workgroup
// computes the same from the step's row ranges (one thread, 32-bit shifts:
// the key counts are below 2^31), then its own unit: unit[] = {row (nrows:
// none), split, the row's splits, the row's first slot} of slot w / nkv.
template <int D>
__device__ __forceinline__ void split_rows(const StepArgs& a, int64_t hi, int nrows, int* unit) {
  constexpr int SMAX = D / 4 < 32 ? D / 4 : 32;
  const int slots = (int)gridDim.x / a.nkv;
  uint32_t nk[8];
  int lg[8];
  int used = 0;
  for (int b = 0; b < nrows; ++b) {
    int64_t lo = a.start_t[b];
    lo = lo < 0 ? 0 : lo;
    nk[b] = (uint32_t)(hi > lo ? hi - lo : 0);
    lg[b] = 0;
    while (((nk[b] + (1u << lg[b]) - 1) >> lg[b]) > (uint32_t)a.lchunk && (1 << lg[b]) < SMAX) ++lg[b];
    used += 1 << lg[b];
  }
  while (true) {
    int best = -1;
    uint32_t bl = 1;   // a row down to one key per split gains nothing
    for (int b = 0; b < nrows; ++b) {
      const uint32_t l = (nk[b] + (1u << lg[b]) - 1) >> lg[b];
      if ((2 << lg[b]) <= SMAX && used + (1 << lg[b]) <= slots && l > bl) { bl = l; best = b; }
    }
    if (best < 0) break;
    used += 1 << lg[best];
    ++lg[best];
  }
  const int uj = (int)blockIdx.x / a.nkv;
  unit[0] = nrows; unit[1] = 0; unit[2] = 1; unit[3] = 0;
  for (int b = 0, p = 0; b < nrows; p += 1 << lg[b], ++b)
    if (uj >= p && uj < p + (1 << lg[b])) { unit[0] = b; unit[1] = uj - p; unit[2] = 1 << lg[b]; unit[3] = p; }
}

template <int D, int G, int MB>
__device__ __forceinline__ bool batch_pass(const StepArgs& a, const int64_t* lwt, uint32_t ep, int64_t hi,
                                           const int* s_unit, unsigned char* smem, float* s_red, int* s_fail
#ifdef EK_STEP_TRACE
                                           , int64_t* ts_lds
#endif
                                           ) {
  const int tid = threadIdx.x;
  const int h = a.h, inter = a.inter, nrows = a.m;
  const int qw = a.nq * D, qkvw = (a.nq + 2 * a.nkv) * D;
  const int64_t lwords = (int64_t)MB * arena_layer_words(h, inter, qkvw, qw);
  constexpr int BSLICE = bstep_slice(MB);
  const int xld = bstep_xld(h, qw, MB);

  uint32_t* rr = reinterpret_cast<uint32_t*>(smem);
  unsigned char* ph = smem + bstep_rr_bytes(MB, h);
  bf16_t* xs = reinterpret_cast<bf16_t*>(ph);
  uint32_t* xs32 = reinterpret_cast<uint32_t*>(ph);
  float* part = reinterpret_cast<float*>(ph + eka::align16((size_t)MB * xld * 2));
  const int part_n = a.part_max * SNW * MB;
  uint32_t* gain_lds = reinterpret_cast<uint32_t*>(reinterpret_cast<unsigned char*>(part) +
                                                   eka::align16((size_t)a.part_max * SNW * MB * 4));   // the norm's gain row
  PartWriter<MB, false> put{part, wave_id()};
  PartWriter<MB, true> add{part, wave_id()};
  // the residual rows' words into LDS: every 16-byte unit slot of a thread
  // is loaded (a slot past the last unit re-reads unit 0), so at 8 rows 5
  // slots per thread, which cover hidden 2560 (2560 units) in one round (8
  // measured 1 % slower at config 5; 4 rows keep 4: 3 measured slower);
  // wider rows take more rounds
  auto read_res = [&](const llw_t* src) -> bool {
    constexpr int WR = MB == 8 ? 5 : MB;
    return dw_read<WR>(src, LinUnits{}, nrows * (h / 8), xs32, LinLds{}, a.err, a.spin);
  };

  // attention unit of this workgroup (s_unit: row, split, splits, the row's
  // first slot; wave-uniform)
  const int uh = (int)blockIdx.x % a.nkv;
  const int ub = __builtin_amdgcn_readfirstlane(s_unit[0]), us = __builtin_amdgcn_readfirstlane(s_unit[1]);
  const int uS = __builtin_amdgcn_readfirstlane(s_unit[2]), upre = __builtin_amdgcn_readfirstlane(s_unit[3]);
  const bool attends = ub < nrows;

  BRing ring;
  ring.nready = 0;
#pragma unroll
  for (int u = 0; u < BNB; ++u) ring.r[u] = make_uint4(0, 0, 0, 0);
  uint32_t gw1[NGW], gw2[NGW];
  load_gain(reinterpret_cast<const bf16_t*>(lwt[LW_LN1]), h, gw1);

  llw_t* half = cur_half(a, ep);
  // the unit's row's exchange words: its slots' units, after the rows before
  llw_t* lx_row = half + (int64_t)a.nl * lwords + 2 * (int64_t)gridDim.x * MB + long_words(a.nkv, upre, G, D);
  const int nsl = cdiv_i(inter, BSLICE * CH);   // K slices of the down projection
  // the lm_head's share: whole tiles (the rows past vocab re-read its last), or rows
  const Gp glm = bstep_mfma<MB>() ? make_gp(a.lm_head, h, MT * cdiv_i(a.vocab, MT), 0, MT)
                                  : make_gp(a.lm_head, h, a.vocab, 0, 1);

  const llw_t* dn_prev = nullptr;
  for (int l = 0; l < a.nl; ++l) {
    const int64_t* lw = lwt + l * LW_FIELDS;
    llw_t* qkv_ll = half + (int64_t)l * lwords;
    llw_t* att_ll = qkv_ll + (int64_t)MB * qkvw / 4;
    llw_t* o_ll = att_ll + (int64_t)MB * qw / 4;
    llw_t* act_ll = o_ll + (int64_t)MB * h / 4;
    llw_t* dn_ll = act_ll + (int64_t)MB * inter / 4;
    const Gp gq = make_gp(reinterpret_cast<const bf16_t*>(lw[LW_QKV]), h, qkvw, 0, BGRAN);
    const Gp go = make_gp(reinterpret_cast<const bf16_t*>(lw[LW_O]), qw, h, 0, BGRAN);
    const Gp gg = make_gp(reinterpret_cast<const bf16_t*>(lw[LW_GU]), h, inter, 1, BGRAN);
    const bf16_t* wdown = reinterpret_cast<const bf16_t*>(lw[LW_DOWN]);
    auto down_slice = [&](int sl) {
      const int c0 = sl * BSLICE, c1 = (sl + 1) * BSLICE < inter / CH ? (sl + 1) * BSLICE : inter / CH;
      return make_gp(wdown + c0 * CH, (c1 - c0) * CH, h, 0, BGRAN);
    };

    // ---- r = (layer 0) embed[token] | r + down(l-1); norm; qkv
    EK_TS(0);
    zero_part(part, part_n);
    if (l == 0) {
      for (int m = 0; m < nrows; ++m) {
        int64_t t = a.tokens[m];
        t = t < 0 ? 0 : (t >= a.vocab ? a.vocab - 1 : t);
        const uint32_t* e32 = reinterpret_cast<const uint32_t*>(a.embed + t * a.lde);
        for (int i = tid; i < h / 2; i += SNT) rr[m * (h / 2) + i] = e32[i];
      }
      __syncthreads();
      add_norm_rows<MB>(rr, nullptr, gw1, gain_lds, h, nrows, a.eps, xs, xld, s_red);
    } else {
      constexpr int WR = MB == 8 ? 5 : MB;
      if (nrows * (h / 8) <= WR * SNT) {
        if (!dw_add_norm<MB, WR>(dn_prev, rr, gw1, gain_lds, h, nrows, a.eps, xs, xld, s_red, s_fail, a.err, a.spin))
          return false;
      } else {
        const bool ok = read_res(dn_prev);
        if (!wg_all(ok, s_fail)) return false;
        add_norm_rows<MB>(rr, xs32, gw1, gain_lds, h, nrows, a.eps, xs, xld, s_red);
      }
      EK_TS(23);
    }
    __syncthreads();
    EK_TS(1);
    gemv_phase_b<MB>(gq, h, false, ring, xs, xld, put);
    __syncthreads();
    EK_TS(2);
    epilogue_ll_b<MB>(gq, part, qkv_ll, qkvw / 4, nrows);
    __syncthreads();
    EK_TS(3);

    // ---- split attention (its LDS overlays the activation rows and partials)
    if (attends) {
      if (!long_attention<D, G>(a, lw, BStepIO<MB>{StepIO{qkv_ll + (int64_t)ub * (qkvw / 4), att_ll + (int64_t)ub * (qw / 4)}},
                                lx_row, ub, uh, us, uS, hi, (uint32_t)l + 1u, ph, s_fail
#ifdef EK_STEP_TRACE
                                , ts_lds
#endif
                                ))
        return false;
    }
    EK_TS(4);
    prefetch_phase_b<MB, BPF>(go, qw, false, ring);
    load_gain(reinterpret_cast<const bf16_t*>(lw[LW_LN2]), h, gw2);
    __syncthreads();

    // ---- o projection
    zero_part(part, part_n);
    {
      // row m's values land xld apart
      const bool ok = dw_read<MB>(att_ll, RowsUnits{qw / 4, qw / 8}, nrows * (qw / 8), xs32,
                                  RowsLds{qw / 8, xld / 2}, a.err, a.spin);
      if (!wg_all(ok, s_fail)) return false;
    }
    EK_TS(6);
    __syncthreads();
    gemv_phase_b<MB>(go, qw, false, ring, xs, xld, put);
    __syncthreads();
    EK_TS(7);
    epilogue_ll_b<MB>(go, part, o_ll, h / 4, nrows);
    EK_TS(8);
    prefetch_phase_b<MB, BPF>(gg, h, false, ring);

    // ---- r = r + o; norm; gate/up; SwiGLU
    __syncthreads();
    zero_part(part, part_n);
    {
      constexpr int WR = MB == 8 ? 5 : MB;
      if (nrows * (h / 8) <= WR * SNT) {
        if (!dw_add_norm<MB, WR>(o_ll, rr, gw2, gain_lds, h, nrows, a.eps, xs, xld, s_red, s_fail, a.err, a.spin))
          return false;
      } else {
        const bool ok = read_res(o_ll);
        if (!wg_all(ok, s_fail)) return false;
        add_norm_rows<MB>(rr, xs32, gw2, gain_lds, h, nrows, a.eps, xs, xld, s_red);
      }
    }
    EK_TS(17);
    load_gain(l + 1 < a.nl ? reinterpret_cast<const bf16_t*>(lwt[(l + 1) * LW_FIELDS + LW_LN1]) : a.fnorm, h, gw1);
    EK_TS(18);
    __syncthreads();
    EK_TS(9);
    gemv_phase_b<MB>(gg, h, false, ring, xs, xld, put);
    __syncthreads();
    EK_TS(10);
    epilogue_swiglu_ll_b<MB>(gg, part, act_ll, inter / 4, nrows);
    EK_TS(11);
    prefetch_phase_b<MB, BPF>(down_slice(0), inter, false, ring);

    // ---- down projection, one K slice of the act rows at a time (one slice
    //      for a 9728-wide act row up to 4 rows); when their registers fit,
    //      each slice's words are loaded (once) before the previous slice's
    //      products, so that their round trip overlaps them
    __syncthreads();
    zero_part(part, part_n);
    constexpr int SW = bstep_slice_units<MB>();
    constexpr bool EARLY = SW <= EK_BSTEP_EARLY_UNITS && G <= 4;
    u32x4_t nx[SW];
    for (int sl = 0; sl < nsl; ++sl) {
      const Gp gd = down_slice(sl);
      const int c0 = sl * BSLICE;
      const int su = gd.K / 8;   // units of a row's slice
      const RowsUnits src{inter / 4, su};
      if (sl > 0) __syncthreads();   // the previous slice's products have read their LDS rows
      {
        if (sl == 0 || !EARLY) dw_issue<SW>(act_ll + c0 * (CH / 4), src, nrows * su, nx);
        const bool ok = dw_finish<SW>(act_ll + c0 * (CH / 4), src, nrows * su, nx, xs32, RowsLds{su, xld / 2},
                                      a.err, a.spin);
        if (!wg_all(ok, s_fail)) return false;
      }
      if (EARLY && sl + 1 < nsl) {
        const int sun = down_slice(sl + 1).K / 8;
        dw_issue<SW>(act_ll + (c0 + BSLICE) * (CH / 4), RowsUnits{inter / 4, sun}, nrows * sun, nx);
      }
      if (sl == 0) EK_TS(20);
      else EK_TS(21);
      __syncthreads();
      gemv_phase_b<MB>(gd, inter, false, ring, xs, xld, add);
      if (sl == 0) EK_TS(12);
      else EK_TS(13);
      // the next slice's first chunks, or the next phase's (every iteration
      // leaves the ring in the same state, so the products above see a
      // prefetched ring at compile time)
      if (sl + 1 < nsl)
        prefetch_phase_b<MB, BPF>(down_slice(sl + 1), inter, false, ring);
      else if (l + 1 < a.nl)
        prefetch_phase_b<MB, BPF>(make_gp(reinterpret_cast<const bf16_t*>(lwt[(l + 1) * LW_FIELDS + LW_QKV]), h, qkvw,
                                     0, BGRAN), h, false, ring);
      else
        prefetch_phase_b<MB, BPF>(glm, h, true, ring, a.vocab);
    }
    __syncthreads();
    epilogue_ll_b<MB>(down_slice(0), part, dn_ll, h / 4, nrows);
    EK_TS(14);
    dn_prev = dn_ll;
    __syncthreads();
    EK_TS_FLUSH(l);
  }

  // ---- final add + norm, lm_head, per-workgroup argmax per row
  {
    const bool ok = read_res(dn_prev);
    if (!wg_all(ok, s_fail)) return false;
  }
  add_norm_rows<MB>(rr, xs32, gw1, gain_lds, h, nrows, a.eps, xs, xld, s_red);
  __syncthreads();
  int u0, u1;
  unit_range(glm, u0, u1);
  ArgmaxSink<MB> am;
#pragma unroll
  for (int k = 0; k < ArgmaxSink<MB>::NS; ++k) { am.bv[k] = -INFINITY; am.bi[k] = 0x7fffffff; }
  am.logits = a.logits;
  am.vocab = a.vocab;
  am.nrows = nrows;
  am.u0 = u0;
  gemv_phase_b<MB>(glm, h, true, ring, xs, xld, am, a.vocab);
  // the lanes' bests -> the workgroup's, per row -> two words per row: the
  // candidates of batch row m in slots [SNW][4][MB] (the activation rows are
  // no longer read), every slot no lane fills a -inf sentinel
  float* sv = reinterpret_cast<float*>(ph);
  int* si = reinterpret_cast<int*>(ph) + SNW * 4 * MB;
  __syncthreads();
  for (int i = tid; i < SNW * 4 * MB; i += SNT) { sv[i] = -INFINITY; si[i] = 0x7fffffff; }
  __syncthreads();
  {
    const int lane = tid & 63;
    if constexpr (bstep_mfma<MB>()) {
      if ((lane & 12) == 0) {
#pragma unroll
        for (int c = 0; c < ArgmaxSink<MB>::NS; ++c) {
          const int m = 4 * c + (lane & 3);
          if (m < MB) {
            sv[(wave_id() * 4 + (lane >> 4)) * MB + m] = am.bv[c];
            si[(wave_id() * 4 + (lane >> 4)) * MB + m] = am.bi[c];
          }
        }
      }
    } else if (lane == 63) {
#pragma unroll
      for (int m = 0; m < MB; ++m) { sv[wave_id() * 4 * MB + m] = am.bv[m]; si[wave_id() * 4 * MB + m] = am.bi[m]; }
    }
  }
  __syncthreads();
  llw_t* am_ll = half + (int64_t)a.nl * lwords;
  if (tid < nrows) {
    float ov = sv[tid];
    int oi = si[tid];
    for (int w = 1; w < SNW * 4; ++w)
      if (am_better(sv[w * MB + tid], si[w * MB + tid], ov, oi)) { ov = sv[w * MB + tid]; oi = si[w * MB + tid]; }
    ll_put(am_ll + 2 * ((int64_t)blockIdx.x * MB + tid), __float_as_uint(ov), AM_TAG);
    ll_put(am_ll + 2 * ((int64_t)blockIdx.x * MB + tid) + 1, (uint32_t)oi, AM_TAG);
  }
  return true;
}

// Workgroup 0's end of the step: per row, the first-index argmax over every
// workgroup's words, then the step's bookkeeping for every row (as the
// batch-1 finish_step; a step that gave up writes -1 for every row).
template <int MB>
__device__ __forceinline__ void finish_step_b(const StepArgs& a, uint32_t ep, bool ok, int64_t len_old, int qw,
                                              int qkvw, unsigned char* smem, float* s_red, int* s_redi, int* s_fail) {
  const int tid = threadIdx.x, nrows = a.m;
  const int64_t lwords = (int64_t)MB * arena_layer_words(a.h, a.inter, qkvw, qw);
  const llw_t* am_ll = cur_half(a, ep) + (int64_t)a.nl * lwords;
  const int nwg = (int)gridDim.x;
  uint32_t* amw = reinterpret_cast<uint32_t*>(smem + bstep_rr_bytes(MB, a.h));
  int* toks = reinterpret_cast<int*>(amw + 2 * nwg * MB);
  __syncthreads();
  if (ok) {
    struct Src {   // workgroup w's two words of row m at 2 (w MB + m)
      const llw_t* p; int nrows;
      __device__ const llw_t* operator()(int i) const {
        const int w = i / (2 * nrows), j = i - w * (2 * nrows);
        return p + 2 * (int64_t)w * MB + j;
      }
    };
    ok = wg_all(ll_read<BLLW>(Src{am_ll, nrows}, 2 * nwg * nrows, AM_TAG, amw, a.err, a.spin), s_fail);
  }
  if (ok) {
    for (int m = 0; m < nrows; ++m) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int w = tid; w < nwg; w += SNT) {
        const float v = __uint_as_float(amw[2 * (w * nrows + m)]);
        const int i = (int)amw[2 * (w * nrows + m) + 1];
        if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
      }
      float ov;
      int oi;
      wg_argmax(bv, bi, s_red, s_redi, ov, oi);
      if (tid == 0) toks[m] = oi == 0x7fffffff ? 0 : oi;
      __syncthreads();
    }
  }
  if (tid == 0) {
    const int64_t step = *a.step_idx;
    for (int m = 0; m < nrows; ++m) {
      const int64_t tok = !ok ? -1 : toks[m];
      if (a.out_tok) a.out_tok[m] = tok;
      if (step >= 0 && step < a.max_steps) a.out_buf[step * nrows + m] = (int32_t)tok;
      if (ok) {
        a.tokens[m] = tok;
        a.positions[m] += 1;
        a.slot_t[m] = len_old;
      }
    }
    if (ok) *a.len_t = len_old + 1;
    *a.step_idx = step + 1;
  }
}

template <int D, int G, int MB>
__global__ __launch_bounds__(SNT) void batch_step_kernel(StepArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float s_red[SNW * MB];
  __shared__ int s_redi[SNW];
  __shared__ unsigned s_ep;
  __shared__ int s_abort;
  __shared__ int s_fail;
  __shared__ int64_t s_lw[MAX_LAYERS * LW_FIELDS];
  __shared__ int s_unit[4];
#ifdef EK_STEP_TRACE
  __shared__ int64_t s_ts[48];
  int64_t* ts_lds = s_ts;
#endif

  const int tid = threadIdx.x;
  const int64_t len_old = *a.len_t;
  int64_t hi = len_old + 1;
  hi = hi < 0 ? 0 : (hi > a.s_cap ? a.s_cap : hi);
  for (int i = tid; i < a.nl * LW_FIELDS; i += SNT) s_lw[i] = a.lw[i];
  if (tid == 0) {
    s_fail = 0;
    const unsigned e = __hip_atomic_load(&a.bar->ep[blockIdx.x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    __hip_atomic_store(&a.bar->ep[blockIdx.x], e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_ep = e;
    s_abort = __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    split_rows<D>(a, hi, a.m, s_unit);
  }
  __syncthreads();
  const uint32_t ep = __builtin_amdgcn_readfirstlane(s_ep);   // wave-uniform: the halves' addresses stay scalar
  clear_next_half(a, ep);   // also in a launch that gives up: the next one needs it
  bool ok = s_abort == 0;
  if (ok) ok = batch_pass<D, G, MB>(a, s_lw, ep, hi, s_unit, smem, s_red, &s_fail
#ifdef EK_STEP_TRACE
                                     , ts_lds
#endif
                                     );
  if (blockIdx.x != 0) return;
  finish_step_b<MB>(a, ep, ok, len_old, a.nq * D, (a.nq + 2 * a.nkv) * D, smem, s_red, s_redi, &s_fail);
}

// LDS bytes of batch_step_kernel<D, G, MB>
template <int D, int G, int MB>
inline size_t bstep_lds_bytes(int h, int qw, int part_rows, int lchunk, int nwg) {
  const size_t rr = bstep_rr_bytes(MB, h);
  const size_t gemv = eka::align16((size_t)MB * bstep_xld(h, qw, MB) * 2) + eka::align16((size_t)part_rows * SNW * MB * 4) +
                      eka::align16((size_t)h / 2 * 4);
  const size_t attn = LongLds<D, G>::bytes(lchunk);
  const size_t fin = (size_t)2 * nwg * MB * 4 + (size_t)MB * 4;
  size_t x = gemv > attn ? gemv : attn;
  x = x > fin ? x : fin;
  return rr + x;
}

// launch / occupancy of one batch instantiation (ek_bstep_inst.hip, one per MB)
template <int MB>
hipError_t launch_bstep(const StepArgs& a, int g, int nwg, hipStream_t st);
template <int MB>
int bstep_occupancy(int g, size_t lds);

}  // namespace eks
