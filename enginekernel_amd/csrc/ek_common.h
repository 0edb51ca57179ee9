// Shared device helpers for the gfx950 decode kernels.
//
// bf16 values travel as raw 16-bit patterns (uint16_t) so that every
// rounding point is explicit: bf2f widens exactly, f2bf rounds to nearest
// even once. bf16 x bf16 products are exact in fp32 (8+8 significant bits),
// so an fp32 FMA chain over bf16 operands rounds only the running sum.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define EK_WAVE 64

typedef uint16_t bf16_t;

__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

// gfx950's conversion instruction (v_cvt_pk_bf16_f32): round to nearest
// even, one instruction for two values (the bit arithmetic it replaces --
// NaN test, add 0x7fff plus the lsb, shift -- took six per value)
typedef __bf16 ek_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float ek_f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// round an fp32 value to the nearest bf16 and widen it back
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// the low / high bf16 of a packed 32-bit word, widened
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = lo_bf(v.x); f[1] = hi_bf(v.x);
  f[2] = lo_bf(v.y); f[3] = hi_bf(v.y);
  f[4] = lo_bf(v.z); f[5] = hi_bf(v.z);
  f[6] = lo_bf(v.w); f[7] = hi_bf(v.w);
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const ek_f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, ek_bf16x2_t));
}

// sum of 8 products of two packed-bf16 chunks, added to acc in order
__device__ __forceinline__ float dot8_acc(const uint4& w, const uint4& x, float acc) {
  acc = fmaf(lo_bf(w.x), lo_bf(x.x), acc);
  acc = fmaf(hi_bf(w.x), hi_bf(x.x), acc);
  acc = fmaf(lo_bf(w.y), lo_bf(x.y), acc);
  acc = fmaf(hi_bf(w.y), hi_bf(x.y), acc);
  acc = fmaf(lo_bf(w.z), lo_bf(x.z), acc);
  acc = fmaf(hi_bf(w.z), hi_bf(x.z), acc);
  acc = fmaf(lo_bf(w.w), lo_bf(x.w), acc);
  acc = fmaf(hi_bf(w.w), hi_bf(x.w), acc);
  return acc;
}

// The same sum on gfx950's bf16 dot instruction (v_dot2c_f32_bf16: two bf16
// products added to an fp32 accumulator per instruction): 4 instructions per
// chunk instead of 8 FMAs and 16 unpacking shifts/masks. The bf16 products
// are exact in fp32; only the fp32 summation order differs from dot8_acc.
typedef __bf16 ek_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot8_acc_d2(const uint4& w, const uint4& x, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ek_bf16x2, w.x), __builtin_bit_cast(ek_bf16x2, x.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ek_bf16x2, w.y), __builtin_bit_cast(ek_bf16x2, x.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ek_bf16x2, w.z), __builtin_bit_cast(ek_bf16x2, x.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ek_bf16x2, w.w), __builtin_bit_cast(ek_bf16x2, x.w), acc, false);
  return acc;
}

// butterfly sum over all 64 lanes of a wave (every lane gets the total)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, EK_WAVE);
  return v;
}

// butterfly sum over aligned groups of `width` lanes (width a power of two)
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, EK_WAVE);
  return v;
}

// Sum over all 64 lanes through DPP moves (no LDS traffic): pairs and quads
// by quad permutes, rows of 16 by row rotates, then rows 0+1 and 2+3 by
// row broadcasts; the total is exact in lane 63 (other lanes hold partial
// sums) and is returned wave-uniform. The summation order is fixed.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_plus(float v) {
  const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false);
  return v + __int_as_float(moved);
}
// The same sum for N independent values, step by step across all of them
// (each DPP step's result is needed two instructions later: interleaving the
// N chains fills the waits that one chain alone spends in s_nop). The
// totals are exact in lane 63; returns nothing, leaves them there.
template <int N>
__device__ __forceinline__ void wave_sums_dpp_lane63(float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = dpp_plus<0xB1>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = dpp_plus<0x4E>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = dpp_plus<0x124>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = dpp_plus<0x128>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = dpp_plus<0x142, 0xa>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = dpp_plus<0x143, 0xc>(v[i]);
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_plus<0xB1>(v);        // quad_perm [1,0,3,2]
  v = dpp_plus<0x4E>(v);        // quad_perm [2,3,0,1]
  v = dpp_plus<0x124>(v);       // row_ror:4
  v = dpp_plus<0x128>(v);       // row_ror:8  -> every lane holds its row's sum
  v = dpp_plus<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
  v = dpp_plus<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, EK_WAVE));
  return v;
}

// The thread index, opaque to the optimizer: per-lane offsets derived from
// it are then computed where they are used instead of hoisted out of a
// caller's loop (where they would stay live, in registers, across
// everything else the loop does).
__device__ __forceinline__ int opaque_tid() {
  int t = threadIdx.x;
  __asm__ volatile("" : "+v"(t));
  return t;
}

// index of this thread's wave in the workgroup, as a wave-uniform (scalar) value
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// 16-byte load of 8 bf16 from global memory. The pointer is taken as a
// global (not flat) address, so the load is a global_load_dwordx4 even when
// the pointer itself was read from memory; callers pass device memory only.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4_t global_u32x4_t;
__device__ __forceinline__ uint4 ld16(const bf16_t* p) {
  const u32x4_t v = *(global_u32x4_t*)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// The same load marked non-temporal, for data read once per pass (weights,
// cached keys and values): the L2 then keeps the lines that are reused.
__device__ __forceinline__ uint4 ld16_nt(const bf16_t* p) {
  const u32x4_t v = __builtin_nontemporal_load((global_u32x4_t*)(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 4-byte load from global memory as a global (not flat) load: a flat load
// also counts against the LDS wait counter, so every later LDS access (and
// every barrier) would wait for it.
typedef const __attribute__((address_space(1))) uint32_t global_u32_t;
__device__ __forceinline__ uint32_t ld4(const void* p) { return *(global_u32_t*)(p); }

// Dense hand-over words of the persistent step kernels: word i of a region
// holds its values 4i .. 4i + 3 (value 4i + j in bits 16j .. 16j + 15, so a
// region is its bf16 row in memory order), sign bits flipped so that no
// stored 32-bit half is zero (zero means "not written yet"). A word is one
// device-scope store, or two: a producer that owns only values 2i, 2i + 1 of
// a region stores that half alone (dw_put1), so readers check each half.
constexpr unsigned long long DW_FLIP = 0x8000800080008000ull;
constexpr uint32_t DW_FLIP32 = 0x80008000u;

// a half of (-0.0, -0.0) would read as unwritten: its first value travels as +0.0
__device__ __forceinline__ uint32_t dw_half(uint32_t v01) {
  const uint32_t w = v01 ^ DW_FLIP32;
  return w ? w : 0x8000u;
}
__device__ __forceinline__ void dw_put(unsigned long long* p, uint32_t v01, uint32_t v23) {
  const unsigned long long w = ((unsigned long long)dw_half(v23) << 32) | dw_half(v01);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// values 2i, 2i + 1 of a region, at its 32-bit index i
__device__ __forceinline__ void dw_put1(uint32_t* p, uint32_t v01) {
  __hip_atomic_store(p, dw_half(v01), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
