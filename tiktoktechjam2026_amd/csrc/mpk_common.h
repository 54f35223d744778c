// Shared device helpers for the gfx950 (CDNA4) mixed-precision Transformer kernels.
//
// Conventions used by every kernel in this library
// ------------------------------------------------
// * Wavefronts are 64 lanes.  A lane index l splits as r = l % 16 (MFMA row/col)
//   and g = l / 16 (the lane group that owns a k-slice of an MFMA operand).
// * All matrix products use v_mfma_f32_16x16x32_f16 (FP16 x FP16 -> FP32) or, for
//   16-wide head dims, v_mfma_f32_16x16x16_f16.  Operand layouts (every GEMM and
//   attention parity test in tests/test_kernels_gpu.py depends on them):
//     A (16 x K): lane l holds row r, k = 8g .. 8g+7          (16x16x32)
//     B (K x 16): lane l holds col r, k = 8g .. 8g+7
//     C (16 x 16): lane l holds col r, rows 4g .. 4g+3
//   The k -> slot assignment only has to agree between A and B, which lets a
//   kernel feed one MFMA's result straight into the next one's B operand.
// * "Transposed" products: every GEMM here computes C^T = W * X^T, i.e. the
//   weight rows (output features n) are the MFMA rows and the token rows m are
//   the MFMA columns.  A lane then owns one token row and a run of output
//   features, which makes row-wise epilogues (bias, GELU, residual, LayerNorm)
//   lane-local and gives 16-byte stores.
// * "Paired" row mapping: two consecutive 16-row MFMA tiles (t = 0, 1) cover 32
//   output features; MFMA row q of tile t is mapped to feature
//       pair_row(q, t) = 8 * (q / 4) + 4 * t + (q % 4)
//   so lane group g ends up holding features 8g .. 8g+7 of the pair in one
//   contiguous run: acc[t][i] is feature 8g + 4t + i.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mpk.h"  // the exported C ABI (include/mpk.h); definitions are checked against it

namespace mpk {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

enum DType : int { kF32 = 0, kF16 = 1 };

constexpr int kWave = 64;
constexpr int kBlock = 256;  // four waves per workgroup everywhere

__device__ __forceinline__ f4 mfma32(const h8& a, const h8& b, const f4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 mfma16(const h4& a, const h4& b, const f4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int pair_row(int q, int t) { return 8 * (q >> 2) + 4 * t + (q & 3); }

// LDS slot of weight row j: within each 32-row group, row pair_row(r, tt) goes
// to slot 16 tt + r, so the 16 lanes of one fragment read consecutive padded
// rows (no bank conflicts) instead of pair_row's strided set.
__device__ __forceinline__ int w_slot(int j) {
  return (j & ~31) | (((j >> 2) & 1) << 4) | ((j >> 3) & 3) << 2 | (j & 3);
}

// ---- 32x32x16 products ----
// Operand layouts of v_mfma_f32_32x32x16_f16 (lane l, i = l % 32, h = l / 32):
//   A (32 x 16): row i, k = 8h .. 8h+7     B (16 x 32): column i, k = 8h .. 8h+7
//   C (32 x 32): column i, rows 8J + 4h + I in register 4J + I  (J, I = 0..3)
// A kernel that feeds MFMA row rho of a 32-row block from row kappa32(rho) of its
// operand,
//   kappa32(8J + 4h + I) = 16 (J >> 1) + 8h + 4 (J & 1) + I,
// finds in accumulator register e = 8s + j (s = 0, 1; j = 0..7) of lane (i, h) the
// operand row 16s + 8h + j: two runs of 8 consecutive rows per lane, which is the
// B operand of the two 16-deep k-steps of a following product over those rows.
typedef float f16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f16v mfma32x32(const h8& a, const h8& b, const f16v& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int kappa32(int rho) {
  const int J = rho >> 3, hh = (rho >> 2) & 1, I = rho & 3;
  return 16 * (J >> 1) + 8 * hh + 4 * (J & 1) + I;
}

// Sum of v over lanes l and l ^ 32 (the two halves of a 32x32 C column), bit-identical in both.
__device__ __forceinline__ float sum_over_halves(float v) {
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Index of the calling wave in its workgroup, as a wave-uniform (scalar) value:
// branches on quantities derived from it compile to scalar branches instead of
// exec-mask divergence, and its address arithmetic stays on the scalar unit.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

__device__ __forceinline__ f4 zero4() { return f4{0.f, 0.f, 0.f, 0.f}; }

// ---- global loads of 8 consecutive elements as FP16 (round-to-nearest-even) ----
__device__ __forceinline__ h8 load8_as_half(const _Float16* p) { return *reinterpret_cast<const h8*>(p); }

__device__ __forceinline__ h8 load8_as_half(const float* p) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  h8 r;
  r[0] = (_Float16)a.x; r[1] = (_Float16)a.y; r[2] = (_Float16)a.z; r[3] = (_Float16)a.w;
  r[4] = (_Float16)b.x; r[5] = (_Float16)b.y; r[6] = (_Float16)b.z; r[7] = (_Float16)b.w;
  return r;
}

// Hardware bounds-checked loads.  A raw buffer resource over [base, base + bytes)
// returns zeros for a 16-byte chunk that starts at or past `bytes`, so tile loads
// that run off the end of a sequence need no per-lane predication or zero fill.
// (0x00020000: the gfx9 buffer format word for 32-bit untyped data.)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ h8 buffer_load8_as_half(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, const _Float16*) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  const u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
  return __builtin_bit_cast(h8, v);
}

__device__ __forceinline__ h8 buffer_load8_as_half(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, const float*) {
  typedef float v4 __attribute__((ext_vector_type(4)));
  const v4 a = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
  const v4 b = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off + 16, 0, 0));
  h8 h;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = (_Float16)a[j];
    h[4 + j] = (_Float16)b[j];
  }
  return h;
}

// Bounds-checked stores through the same kind of buffer resource: a store whose
// 16-byte (8-byte) chunk starts at or past the resource's size is dropped by the
// hardware, so row tiles that run past the last row need no per-lane branch.
__device__ __forceinline__ void buffer_store8(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, const float* v,
                                              _Float16*) {
  h8 h;
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = (_Float16)v[j];
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, h), r, byte_off, 0, 0);
}

__device__ __forceinline__ void buffer_store8(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, const float* v, float*) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  typedef float v4 __attribute__((ext_vector_type(4)));
  const v4 a = {v[0], v[1], v[2], v[3]};
  const v4 b = {v[4], v[5], v[6], v[7]};
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, a), r, byte_off, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, b), r, byte_off + 16, 0, 0);
}

__device__ __forceinline__ void buffer_store4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, const float* v) {
  h4 h;
#pragma unroll
  for (int j = 0; j < 4; ++j) h[j] = (_Float16)v[j];
  typedef unsigned int u2 __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, h), r, byte_off, 0, 0);
}

__device__ __forceinline__ h8 zero_h8() {
  h8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = (_Float16)0.f;
  return r;
}

__device__ __forceinline__ void load8_f32(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void load8_f16_to_f32(const _Float16* p, float* v) {
  const h8 h = *reinterpret_cast<const h8*>(p);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (float)h[j];
}

// ---- stores of 8 consecutive FP32 values, as FP32 or rounded to FP16 ----
__device__ __forceinline__ void store8(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ void store8(_Float16* p, const float* v) {
  h8 h;
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = (_Float16)v[j];
  *reinterpret_cast<h8*>(p) = h;
}

// Exact-erf GELU, x * Phi(x) = 0.5 x (1 + erf(x / sqrt 2)), in FP32.  erf comes from
// Abramowitz & Stegun, Handbook of Mathematical Functions, formula 7.1.26:
//   erf(z) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-z^2),  t = 1 / (1 + p z),  z >= 0,
// |error| <= 1.5e-7 for all z (about one FP32 ulp of 1).  With the a_i halved,
// q = (a1 t + ... + a5 t^5) exp(-z^2) is erfc(|x| / sqrt 2) / 2 = Phi(-|x|), and
//   GELU(x) = x (1 - q) for x >= 0,  x q for x < 0,  i.e.  max(x, 0) - |x| q
// (one FMA).  The variable is u = z sqrt(log2 e), so exp(-z^2) = exp2(-u u) and
// p becomes p / sqrt(log2 e).  Per element: one reciprocal, one exp2 and 11 other
// VALU operations.  Over x in [-12, 12] the result differs from the float64 GELU
// by at most 3.4e-7 (FP32 emulation of these steps), below the rounding error of
// evaluating 0.5 x (1 + erff(x / sqrt 2)) in FP32 (4.5e-7).
// Pin an FP32 value in a register (an empty asm), so that a later conversion to FP16 rounds
// this FP32 value: otherwise the compiler may fuse the producing multiply or FMA and the
// conversion into v_fma_mix, which rounds the exact result once - in some kernel
// instantiations and not in others, so the same arithmetic would round differently
// depending on the tile shape.  The reference rounds its FP32 results, then casts.
__device__ __forceinline__ void pin_f32(float& x) { __asm__("" : "+v"(x)); }
// the same for four / eight values in one statement (fewer scheduling boundaries)
__device__ __forceinline__ void pin_f32x4(float* x) { __asm__("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3])); }
__device__ __forceinline__ void pin_f32x8(float* x) {
  __asm__("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7]));
}

__device__ __forceinline__ float gelu_erf(float x) {
  constexpr float kU = 0.84932180028801904f;  // sqrt(log2 e) / sqrt 2
  constexpr float kP = 0.2727374808792225f;   // 0.3275911 / sqrt(log2 e)
  constexpr float kA1 = 0.5f * 0.254829592f, kA2 = 0.5f * -0.284496736f, kA3 = 0.5f * 1.421413741f;
  constexpr float kA4 = 0.5f * -1.453152027f, kA5 = 0.5f * 1.061405429f;
  const float ax = fabsf(x);
  const float u = ax * kU;
  const float t = __builtin_amdgcn_rcpf(fmaf(u, kP, 1.0f));
  const float poly = t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, kA5, kA4), kA3), kA2), kA1);
  const float q = poly * __builtin_amdgcn_exp2f(-(u * u));
  float r = fmaf(-ax, q, fmaxf(x, 0.0f));
  // r is rounded to FP32 here.  A caller's FP16 conversion then rounds that value, as
  // the reference's FP32 GELU followed by a cast does; without the (empty) asm the
  // compiler may fuse the FMA and the conversion into v_fma_mix, which rounds the
  // unrounded result once - in some kernels and not in others, so identical rows
  // would get different FP16 hidden activations depending on the tile shape.
  __asm__("" : "+v"(r));
  return r;
}

// Reductions over the four lane groups g that share one MFMA column (lanes l,
// l^16, l^32, l^48), with the gfx950 row-swap instructions: permlane16_swap
// exchanges rows 1/3 of one operand with rows 0/2 of the other and
// permlane32_swap the upper and lower 32-lane halves, so calling them with the
// same value twice yields (own, partner) pairs in every lane.  Both partners
// evaluate the same commutative expression, so all four lanes end bit-identical.
__device__ __forceinline__ float sum_over_groups(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float max_over_groups(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Flash attention's running row max (log2 units) is raised only when a tile exceeds it by
// more than this (attention.hip, and the attention stage of layer_tail.hip).
constexpr float kRescaleLog2 = 8.0f;

// ---- LDS-DMA copies (global -> LDS without registers) ----
typedef __attribute__((address_space(3))) void lds_void;

// One 16-byte-per-lane LDS-DMA copy: lane l's 16 bytes at base + voff (base
// wave-uniform, voff per lane) land at LDS byte address lds_base + 16 l
// (lds_base wave-uniform, in M0).  Issued as inline assembly: the compiler does
// not track it, so it neither counts it in its own vmcnt waits nor drains every
// LDS read behind it (it cannot tell the copy's target buffer from the ones being
// read).  Its completion is awaited explicitly with wait_copies.  M0 is declared
// clobbered, so the compiler keeps no value of its own there across a copy.
__device__ __forceinline__ void dma16(uint32_t voff, const void* base, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(base), "s"(lds_base)
               : "m0");
}

// Wait until at most N of this wave's vector-memory operations are outstanding
// (they complete in issue order), and for all of its LDS operations.  gfx9
// s_waitcnt encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14.
template <int N>
__device__ __forceinline__ void wait_copies() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier after wait_copies (which has also drained this wave's LDS
// reads).  __syncthreads() would add a release fence, which waits for every
// outstanding load and LDS-DMA copy - including the chunk copies meant to stay in
// flight across it; the acquire fence keeps later LDS reads below the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Map a linear workgroup id so that consecutive tile indices land on the same
// XCD (workgroups are dispatched round-robin over the 8 XCDs, each with its own
// L2).  Identity when the grid is not a multiple of 8.
__device__ __forceinline__ int xcd_local_tile(int wg, int nwg) {
  if ((nwg & 7) != 0) return wg;
  return (wg & 7) * (nwg >> 3) + (wg >> 3);
}

}  // namespace mpk
