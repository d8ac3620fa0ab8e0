// Device helpers shared by the 4-bit weight GEMM kernels (INT4 decode stream and
// prefill tile, MXFP4 stream).
#pragma once

#include "common.h"

namespace xk {

// A wave-uniform constant held in a VGPR. A VOP3 instruction may read at most one
// SGPR or literal on gfx950, so with the nibble mask in a VGPR the compiler
// selects one v_and_or_b32 for (x & mask) | k instead of v_and_b32 + v_or_b32,
// and the unpack stays plain code the scheduler can interleave with MFMAs.
__device__ __forceinline__ uint32_t in_vgpr(uint32_t x) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "s"(x));
  return r;
}

// (x & m) | k with k & m == 0 (one v_and_or_b32 when m is in a VGPR).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t k) {
  return (x & m) | k;
}

// Per-scale constants of dequant_rne_nat (two VALU per scale, shared by every word
// of the group).
struct RneScale {
  float s, m1032, m72;  // s, -1032 s, -72 s
};
__device__ __forceinline__ RneScale rne_scale(float s) {
  return RneScale{s, -1032.0f * s, -72.0f * s};
}

// 8 nibbles of `w` (low nibble = lowest k) -> 8 bf16 = bf16_rne((n - 8) * s),
// the reference's dequant rounding, in natural k order n0 .. n7. Nibble pairs
// (d, d + 4) become two fp16 values with one v_and_or_b32 each: pairs 0 and 2
// (nibbles at bits 0-3 of a half word, mask `mlo` = 0x000F000F, exponent bits
// 0x6400) read 1024 + n, pairs 1 and 3 (bits 4-7, mask `mhi` = 0x00F000F0,
// exponent bits 0x5400) read 64 + n, so one shift of the word serves all four
// pairs and every pair uses the same multiplier. v_fma_mix_f32 then forms
// (1024 + n) s - 1032 s, resp. (64 + n) s - 72 s, both exactly (n - 8) s in
// fp32 (every term fits 24 bits), and v_cvt_pk_bf16_f32 rounds to nearest
// even, pairing the results of nibbles (2d, 2d + 1). 17 VALU per 8 weights.
__device__ __forceinline__ bf16x8 dequant_rne_nat(uint32_t w, const RneScale& k, uint32_t mlo,
                                                  uint32_t mhi) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const uint32_t w8 = w >> 8;
  // x[d] holds nibbles (d, d + 4) in natural order of d: x0 (n0, n4), x1 (n1, n5),
  // x2 (n2, n6), x3 (n3, n7)
  const h2 x[4] = {__builtin_bit_cast(h2, and_or(w, mlo, 0x64006400u)),
                   __builtin_bit_cast(h2, and_or(w, mhi, 0x54005400u)),
                   __builtin_bit_cast(h2, and_or(w8, mlo, 0x64006400u)),
                   __builtin_bit_cast(h2, and_or(w8, mhi, 0x54005400u))};
  float v[8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const float c = (d & 1) ? k.m72 : k.m1032;
    v[d] = fmaf(static_cast<float>(x[d][0]), k.s, c);      // nibble d
    v[d + 4] = fmaf(static_cast<float>(x[d][1]), k.s, c);  // nibble d + 4
  }
  u32x4 b;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    b[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{v[2 * e], v[2 * e + 1]}), b2));
  return __builtin_bit_cast(bf16x8, b);
}

// dequant_rne_nat's exact fp32 products (n - 8) s as a bf16 pair hi + lo ==
// (n - 8) s exactly: hi rounds the product to nearest even, lo is the
// remainder (the product has at most 12 significant bits, so the remainder
// has at most 5 and is exact in bf16). For fp32 activations, whose reference
// contraction uses the unrounded products.
__device__ __forceinline__ void dequant_split_nat(uint32_t w, const RneScale& k, uint32_t mlo,
                                                  uint32_t mhi, bf16x8& hi, bf16x8& lo) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const uint32_t w8 = w >> 8;
  const h2 x[4] = {__builtin_bit_cast(h2, and_or(w, mlo, 0x64006400u)),
                   __builtin_bit_cast(h2, and_or(w, mhi, 0x54005400u)),
                   __builtin_bit_cast(h2, and_or(w8, mlo, 0x64006400u)),
                   __builtin_bit_cast(h2, and_or(w8, mhi, 0x54005400u))};
  float v[8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const float c = (d & 1) ? k.m72 : k.m1032;
    v[d] = fmaf(static_cast<float>(x[d][0]), k.s, c);
    v[d + 4] = fmaf(static_cast<float>(x[d][1]), k.s, c);
  }
  u32x4 bh, bl;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{v[2 * e], v[2 * e + 1]}), b2));
    const float r0 = v[2 * e] - __uint_as_float(h << 16);
    const float r1 = v[2 * e + 1] - __uint_as_float(h & 0xFFFF0000u);
    bh[e] = h;
    bl[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{r0, r1}), b2));
  }
  hi = __builtin_bit_cast(bf16x8, bh);
  lo = __builtin_bit_cast(bf16x8, bl);
}

// e8m0 byte -> the scale operand of v_cvt_scalef32_pk_bf16_fp4, which applies
// only the exponent field of its f32 operand: the byte placed there gives
// 2^(b-127), byte 0 included (2^-127, as in the reference). Byte 0xFF (the
// reserved NaN code, which the reference reads as 0) is handled by zeroing the
// weight word instead (and the scale operand then must not be the inf/nan
// exponent, which would turn 0 * scale into nan).
__device__ __forceinline__ float e8m0_scale(uint32_t b) {
  return __uint_as_float((b == 0xFFu ? 127u : b) << 23);
}

// 8 e2m1 nibbles of `w` (low nibble = lower k) times `s` -> 8 bf16.
__device__ __forceinline__ bf16x8 fp4x8_to_bf16(uint32_t w, float s) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 0);
  const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 1);
  const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 2);
  const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 3);
  bf16x8 r;
  r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
  r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
  return r;
}

// The MXFP4 MoE's clamped SwiGLU of one column j of a slot (mxfp4_reference.py,
// gu = bf16(A @ w13^T) (+ b13 -> bf16), act = bf16(silu(min(g, L)) *
// clamp(u, -L, L))): g and u are the fp32 sums of gate column j and up column
// ispp + j, b13e the expert's bias row (nullable), limit <= 0 no clamp. Every
// kernel that finishes the gate/up projection calls this, so they agree bit
// for bit.
__device__ __forceinline__ uint16_t mxfp4_swiglu(float g, float u, const uint16_t* b13e, int j,
                                                 int ispp, float limit) {
  g = round_bf16(g);
  u = round_bf16(u);
  if (b13e != nullptr) {
    g = round_bf16(g + bf16_to_f32(b13e[j]));
    u = round_bf16(u + bf16_to_f32(b13e[ispp + j]));
  }
  if (limit > 0.f) {
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
  }
  return f32_to_bf16((g / (1.0f + __expf(-g))) * u);
}

}  // namespace xk
