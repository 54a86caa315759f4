// Shared device helpers for the ConvNN-Attention HIP library (gfx950 only).
//
// Storage types: float for fp32 tensors, uint16_t holding the bf16 bit
// pattern for bf16 tensors, _Float16 for fp16 tensors.  All arithmetic is
// fp32; 16-bit values are rounded to nearest-even when stored, the same
// rounding torch applies.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include "../../include/cnna.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint16_t bf16_t;
// first-class 16-byte vector (HIP's uint4 is a struct and can defeat register promotion)
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

#define CNNA_DEV __device__ __forceinline__

CNNA_DEV float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// round to nearest even (v_cvt_pk_bf16_f32)
CNNA_DEV uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// two floats -> packed bf16 pair (lo, hi)
CNNA_DEV uint32_t f2bf2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

CNNA_DEV float ldf(const float* p) { return *p; }
CNNA_DEV float ldf(const uint16_t* p) { return bf2f(*p); }
CNNA_DEV float ldf(const _Float16* p) { return (float)*p; }
CNNA_DEV void stf(float* p, float v) { *p = v; }
CNNA_DEV void stf(uint16_t* p, float v) { *p = f2bf(v); }
CNNA_DEV void stf(_Float16* p, float v) { *p = (_Float16)v; }

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// Pairs of 16-bit values packed in a 32-bit word (element 0 in the low half),
// for either 16-bit storage type.
template <typename T> struct Pair16;
template <> struct Pair16<uint16_t> {
  static CNNA_DEV float lo(uint32_t u) { return __uint_as_float(u << 16); }
  static CNNA_DEV float hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
  static CNNA_DEV uint32_t pack(float lo, float hi) { return f2bf2(lo, hi); }
};
template <> struct Pair16<_Float16> {
  static CNNA_DEV float lo(uint32_t u) { return (float)__builtin_bit_cast(f16x2_t, u)[0]; }
  static CNNA_DEV float hi(uint32_t u) { return (float)__builtin_bit_cast(f16x2_t, u)[1]; }
  static CNNA_DEV uint32_t pack(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
  }
};
// v rounded to the storage type T and back (what storing a T and reading it gives)
CNNA_DEV float rnd_to(float v, float) { return v; }
CNNA_DEV float rnd_to(float v, uint16_t) { return bf2f(f2bf(v)); }
CNNA_DEV float rnd_to(float v, _Float16) { return (float)(_Float16)v; }

// Smallest float strictly greater than x (x not NaN).
CNNA_DEV float next_up(float x) {
  if (x == INFINITY) return x;
  if (x == 0.0f) return __uint_as_float(1u);
  uint32_t u = __float_as_uint(x);
  u = (x > 0.0f) ? u + 1u : u - 1u;
  return __uint_as_float(u);
}

// MFMA 32x32 traits.  Operand layout of v_mfma_f32_32x32x{16_bf16,16_f16,2_f32}:
//   A (32 x KC): lane l supplies A[l % 32][(l / 32) * KL + 0..KL-1]
//   B (KC x 32): lane l supplies B[(l / 32) * KL + 0..KL-1][l % 32]
//   D (32 x 32): lane l, register v holds D[(v/4)*8 + (l/32)*4 + v%4][l % 32]
template <typename T> struct Mfma;

template <> struct Mfma<uint16_t> {
  static constexpr int KC = 16;   // reduction depth of one instruction
  static constexpr int KL = 8;    // elements per lane
  typedef bf16x8_t frag;
  static CNNA_DEV frag load(const uint16_t* p) {
    uint4 u = *reinterpret_cast<const uint4*>(p);
    return __builtin_bit_cast(frag, u);
  }
  static CNNA_DEV frag zero() { return __builtin_bit_cast(frag, make_uint4(0, 0, 0, 0)); }
  // exact negation: flip the eight sign bits
  static CNNA_DEV frag neg(frag a) {
    u32x4_t u = __builtin_bit_cast(u32x4_t, a);
    u ^= 0x80008000u;
    return __builtin_bit_cast(frag, u);
  }
  static CNNA_DEV f32x16_t mma(frag a, frag b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma<_Float16> {
  static constexpr int KC = 16;
  static constexpr int KL = 8;
  typedef f16x8_t frag;
  static CNNA_DEV frag load(const _Float16* p) {
    uint4 u = *reinterpret_cast<const uint4*>(p);
    return __builtin_bit_cast(frag, u);
  }
  static CNNA_DEV frag zero() { return __builtin_bit_cast(frag, make_uint4(0, 0, 0, 0)); }
  static CNNA_DEV frag neg(frag a) {
    u32x4_t u = __builtin_bit_cast(u32x4_t, a);
    u ^= 0x80008000u;
    return __builtin_bit_cast(frag, u);
  }
  static CNNA_DEV f32x16_t mma(frag a, frag b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma<float> {
  static constexpr int KC = 2;
  static constexpr int KL = 1;
  typedef float frag;
  static CNNA_DEV frag load(const float* p) { return *p; }
  static CNNA_DEV frag zero() { return 0.0f; }
  static CNNA_DEV frag neg(frag a) { return -a; }
  static CNNA_DEV f32x16_t mma(frag a, frag b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

// nn.GELU() (erf form): 0.5 x (1 + erf(x / sqrt 2)) with erf from Abramowitz &
// Stegun, Handbook of Mathematical Functions (1964), formula 7.1.26:
//   erfc(z) = (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-z^2),  t = 1 / (1 + p z),
// absolute error <= 1.5e-7 for z >= 0.  Written as
//   gelu(x) = max(x, 0) - |x| h,  h = Phi(-|x|) = erfc(|x| / sqrt 2) / 2,
// which holds for either sign and needs no cancellation-prone 1 - h: the
// 1 / sqrt 2 goes into p, the 1/2 into the a_i, and exp(-x^2 / 2) is
// exp2(-x^2 log2(e) / 2).  Fifteen VALU operations as compiled, two of them
// transcendental (eighteen for 0.5 x (2 - erfc) or 0.5 x erfc by sign); +inf
// is passed through (the product would be inf * 0), -inf and NaN give NaN as
// the erf form does.
CNNA_DEV float gelu_erf(float x) {
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f * 0.70710678118654752f, ax, 1.0f));
  float p = __builtin_fmaf(0.5f * 1.061405429f, t, 0.5f * -1.453152027f);
  p = __builtin_fmaf(p, t, 0.5f * 1.421413741f);
  p = __builtin_fmaf(p, t, 0.5f * -0.284496736f);
  p = __builtin_fmaf(p, t, 0.5f * 0.254829592f);
  const float e = __builtin_amdgcn_exp2f(x * (x * -0.72134752044448170f));
  float pos;   // max(x, 0) without the operand canonicalisation fmaxf adds
  asm("v_max_f32 %0, 0, %1" : "=v"(pos) : "v"(x));
  const float g = __builtin_fmaf(-ax, (p * t) * e, pos);
  return x == INFINITY ? x : g;
}

// The value of lane l ^ 32 (the other half of the wave) without a trip through
// LDS: v_permlane32_swap exchanges lanes 32..63 of its first operand with lanes
// 0..31 of its second; with both operands x, the lower half finds the upper
// half's values in the second result and the upper half the lower half's in
// the first.
CNNA_DEV uint32_t xor32(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return __lane_id() < 32 ? r[1] : r[0];
}
CNNA_DEV float xor32(float x) { return __uint_as_float(xor32(__float_as_uint(x))); }
// lanes 32..63 take the value of lane l - 32, lanes 0..31 keep their own
CNNA_DEV float from_lower(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __lane_id() < 32 ? x : __uint_as_float(r[0]);
}

// c ? t : f as one v_cndmask_b32 on the wave's lane mask of c.  A plain ?: on
// a value just loaded from LDS can be compiled into an exec-masked branch per
// select (the load sunk into it); this form stays one VALU instruction.
CNNA_DEV uint32_t vsel(bool c, uint32_t t, uint32_t f) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(c);
  uint32_t r;
  asm("v_cndmask_b32 %0, %1, %2, %3" : "=v"(r) : "v"(f), "v"(t), "s"(m));
  return r;
}

// Sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15), every lane gets
// it; no LDS traffic.  All 16 lanes must be active.
template <int CTRL>
CNNA_DEV float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
CNNA_DEV float row16_sum(float v) {
  v += dpp_f<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);   // row_half_mirror
  v += dpp_f<0x140>(v);   // row_mirror
  return v;
}

CNNA_DEV int mfma_row(int v, int lane) { return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3); }

// Map a linear block id so that consecutive work items land on the same XCD
// (blocks are dealt to the 8 XCDs round-robin; each XCD has its own L2).
CNNA_DEV int xcd_swizzle(int L, int total) {
  if ((total & 7) != 0) return L;
  const int per = total >> 3;
  return (L & 7) * per + (L >> 3);
}

// torch.linspace(start, end, steps) in float32 (symmetric evaluation).
CNNA_DEV float linspace_f32(float start, float end, int steps, int i) {
  if (steps == 1) return start;
  const float step = (end - start) / (float)(steps - 1);
  const int halfway = steps / 2;
  return (i < halfway) ? start + step * (float)i : end - step * (float)(steps - i - 1);
}

__host__ __device__ inline size_t cnna_round_up(size_t a, size_t b) { return (a + b - 1) / b * b; }
