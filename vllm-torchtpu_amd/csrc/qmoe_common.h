// Shared device helpers for the qmoe gfx950 kernels.
//
// Conventions used by every kernel in this library:
//  * activations are row-major [rows, K]; weights are N-major [N, K] (each
//    output channel's K values contiguous), the checkpoint layout, so both
//    MFMA operands stream along K with 16-byte loads;
//  * bf16 is carried as uint16_t bit patterns;
//  * MFMA 16x16 tiles: lane l feeds row/column (l & 15) of its operand and
//    k-group (l >> 4); the output element (4*(l>>4) + r, l & 15) sits in
//    accumulator register r.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define QMOE_HD __host__ __device__ __forceinline__

// ----------------------------------------------------------------- bf16

QMOE_HD float bf16_to_f32(uint16_t b) {
  union { uint32_t u; float f; } c;
  c.u = (uint32_t)b << 16;
  return c.f;
}

QMOE_HD uint32_t f32_bits(float f) {
  union { uint32_t u; float f; } c;
  c.f = f;
  return c.u;
}

QMOE_HD float bits_f32(uint32_t u) {
  union { uint32_t u; float f; } c;
  c.u = u;
  return c.f;
}

// Round-to-nearest-even float32 -> bf16 (NaN stays a quiet NaN).
QMOE_HD uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

QMOE_HD float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ----------------------------------------------------------------- e4m3fn

// float32 -> OCP e4m3fn code, round-to-nearest-even. Callers clip to +-448
// first (as the reference does); NaN -> 0x7f with the input's sign.
QMOE_HD uint32_t f32_to_e4m3(float f) {
  uint32_t u = f32_bits(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  if (a >= (121u << 23)) {  // |f| >= 2^-6: normal e4m3 binade
    uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;
    r -= 120u << 3;  // rebias 127 -> 7
    if (r > 0x7eu) r = 0x7fu;
    return sign | r;
  }
  // subnormal quantum 2^-9; a * 512 is exact and < 8, rint is RNE; a result
  // of 8 is the code of 2^-6 (exponent field 1), which is what 8 encodes.
  float v = bits_f32(a) * 512.0f;
  return sign | (uint32_t)rintf(v);
}

// OCP e4m3fn code -> float32 (exact).
QMOE_HD float e4m3_to_f32(uint32_t c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xfu;
  uint32_t m = c & 0x7u;
  if (e == 0xfu && m == 0x7u) return bits_f32(s | 0x7fc00000u);
  if (e == 0) return bits_f32(s | f32_bits((float)m * 0.001953125f));
  return bits_f32(s | ((e + 120u) << 23) | (m << 20));
}

// ----------------------------------------------------------------- e5m2

// float32 -> OCP e5m2 code, round-to-nearest-even (bias 15, two mantissa
// bits; magnitudes rounding above 57344 give inf; NaN -> 0x7f with the
// input's sign). Callers clip to +-57344 first, as the reference does.
QMOE_HD uint32_t f32_to_e5m2(float f) {
  uint32_t u = f32_bits(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  if (a >= (113u << 23)) {  // |f| >= 2^-14: normal e5m2 binade
    uint32_t r = (a + 0xfffffu + ((a >> 21) & 1u)) >> 21;
    r -= 112u << 2;  // rebias 127 -> 15
    if (r > 0x7bu) r = 0x7cu;  // inf
    return sign | r;
  }
  // subnormal quantum 2^-16: a * 65536 is exact and < 4; rint is RNE, and
  // 4 is the code of 2^-14
  float v = bits_f32(a) * 65536.0f;
  return sign | (uint32_t)rintf(v);
}

// OCP e5m2 code -> float32 (exact).
QMOE_HD float e5m2_to_f32(uint32_t c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 2) & 0x1fu;
  uint32_t m = c & 0x3u;
  if (e == 0x1fu) return bits_f32(s | (m ? 0x7fc00000u : 0x7f800000u));
  if (e == 0) return bits_f32(s | f32_bits((float)m * 1.52587890625e-05f));
  return bits_f32(s | ((e + 112u) << 23) | (m << 21));
}

// ----------------------------------------------------------------- e8m0

// e8m0 byte -> float32 2^(b-127). b == 0 is the f32 subnormal 2^-127 and
// b == 255 is +inf, matching the reference's ldexp-based decoder.
// Branch-free: 255 << 23 is already the +inf pattern, and every b >= 1
// gives a pattern above the subnormal's, so one unsigned max covers b == 0.
QMOE_HD float e8m0_to_f32(uint32_t b) {
  const uint32_t bits = (b & 0xffu) << 23;
  return bits_f32(bits > 0x00400000u ? bits : 0x00400000u);
}

// ----------------------------------------------------------------- misc

template <typename T>
QMOE_HD T cdiv(T a, T b) { return (a + b - 1) / b; }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Status codes returned by every extern "C" entry point.
enum {
  QMOE_OK = 0,
  QMOE_ERR_ARG = 1,        // bad shape / unsupported combination
  QMOE_ERR_WORKSPACE = 2,  // workspace too small
  QMOE_ERR_LAUNCH = 3,     // hipGetLastError after launch
  QMOE_ERR_SCRATCH = 4,    // qmoe_gemm_static: the problem's split-K partials exceed the static scratch
};
