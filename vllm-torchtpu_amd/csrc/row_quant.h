// Per-element arithmetic of the row quantizers, shared by the quantizer
// kernels (act_quant.hip) and the streaming GEMM's fused per-token
// quantization (gemm_skinny.hip), so that both produce the same codes bit
// for bit. The recipes (runtime division, load-time reciprocal multiply,
// int8 in bf16 arithmetic) are described at the top of act_quant.hip.
#pragma once

#include "qmoe_common.h"

namespace qmoe_rq {

struct Row8 {
  float v[8];
};

// 8 bf16 values (one 16-byte chunk, low half of each dword first) as f32
__device__ __forceinline__ Row8 row8_bf16(const uint4& q) {
  Row8 r;
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r.v[2 * i] = bits_f32(w[i] << 16);
    r.v[2 * i + 1] = bits_f32(w[i] & 0xffff0000u);
  }
  return r;
}

template <bool kInF32>
__device__ __forceinline__ Row8 load8(const void* base, int64_t idx) {
  if (kInF32) {
    Row8 r;
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    float4 a = p[0], b = p[1];
    r.v[0] = a.x; r.v[1] = a.y; r.v[2] = a.z; r.v[3] = a.w;
    r.v[4] = b.x; r.v[5] = b.y; r.v[6] = b.z; r.v[7] = b.w;
    return r;
  }
  return row8_bf16(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + idx));
}

// mode: 0 runtime (division), 1 load-time (reciprocal multiply)
// qdt : 0 e4m3fn, 1 int8, 2 e5m2 (float targets run in f32, qmax 448 /
// 57344; int8 in bf16 arithmetic at runtime)
template <int kQdt>
__device__ __forceinline__ constexpr float qmax_of() {
  return kQdt == 0 ? 448.0f : (kQdt == 2 ? 57344.0f : 127.0f);
}

template <int kQdt>
__device__ __forceinline__ uint32_t float_code(float q) {
  return kQdt == 2 ? f32_to_e5m2(q) : f32_to_e4m3(q);
}

template <int kQdt, int kMode>
__device__ __forceinline__ float make_scale(float amax) {
  if (kMode == 0) {
    if (kQdt != 1) {
      float s = amax / qmax_of<kQdt>();
      return s == 0.0f ? 1.0f : s;
    }
    float s = bf16_round(amax / 127.0f);
    return s == 0.0f ? 1.0f : s;
  }
  const float recip = kQdt == 0 ? (float)(1.0 / 448.0) : (kQdt == 2 ? (float)(1.0 / 57344.0) : (float)(1.0 / 127.0));
  return amax * recip;
}

// x / scale rounded to nearest even, from inv = RN(1 / scale): q = RN(x*inv)
// is within one ulp of the quotient, so r = x - q*scale is exact (one FMA)
// and RN(q + r*inv) is the correctly rounded quotient (Markstein's theorem;
// |x / scale| <= qmax rules out overflow, and a quotient in the f32
// subnormal range encodes to a signed zero whatever its last bits). A zero
// quotient takes x's sign, as the division gives it.
__device__ __forceinline__ float div_rn(float x, float scale, float inv) {
  const float q = x * inv;
  const float r = __builtin_fmaf(-q, scale, x);
  return __builtin_copysignf(__builtin_fmaf(r, inv, q), x);
}

template <int kQdt, int kMode>
__device__ __forceinline__ uint32_t quant1(float x, float scale, float inv) {
  if (kMode == 0) {
    if (kQdt != 1) {
      constexpr float mx = qmax_of<kQdt>();
      float d = x / scale;
      float q = d != d ? d : fminf(fmaxf(d, -mx), mx);  // clip keeps NaN
      return float_code<kQdt>(q);
    }
    float q = rintf(bf16_round(x / scale));
    q = q != q ? 0.0f : fminf(fmaxf(q, -128.0f), 127.0f);  // NaN -> 0, saturate
    return (uint32_t)(int32_t)q & 0xffu;
  }
  float q = x * inv;
  if (kQdt != 1) {
    constexpr float mx = qmax_of<kQdt>();
    float c = fminf(fmaxf(q, -mx), mx);
    if (q != q) c = q;
    return float_code<kQdt>(c);
  }
  float c = q != q ? 0.0f : fminf(fmaxf(q, -128.0f), 127.0f);
  return (uint32_t)(int32_t)rintf(c) & 0xffu;
}

// Runtime codes of 8 values of a row whose scale is finite (so are the
// values: the absmax is NaN- and inf-sticky): division as div_rn, clip,
// then the hardware RNE conversion (e4m3 / e5m2 pairs) or rint (int8).
// Returns the 8 code bytes, the first value in the low byte.
template <int kQdt>
__device__ __forceinline__ uint2 codes8_fast(const Row8& r, float scale, float inv) {
  if (kQdt != 1) {
    constexpr float mx = qmax_of<kQdt>();
    float d[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = fminf(fmaxf(div_rn(r.v[i], scale, inv), -mx), mx);
    int lo, hi;
    if (kQdt == 0) {
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(d[0], d[1], 0, false);
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(d[2], d[3], lo, true);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(d[4], d[5], 0, false);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(d[6], d[7], hi, true);
    } else {
      lo = __builtin_amdgcn_cvt_pk_bf8_f32(d[0], d[1], 0, false);
      lo = __builtin_amdgcn_cvt_pk_bf8_f32(d[2], d[3], lo, true);
      hi = __builtin_amdgcn_cvt_pk_bf8_f32(d[4], d[5], 0, false);
      hi = __builtin_amdgcn_cvt_pk_bf8_f32(d[6], d[7], hi, true);
    }
    return make_uint2((uint32_t)lo, (uint32_t)hi);
  }
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float q = fminf(fmaxf(rintf(bf16_round(div_rn(r.v[i], scale, inv))), -128.0f), 127.0f);
    const uint32_t c = (uint32_t)(int32_t)q & 0xffu;
    if (i < 4) lo |= c << (8 * i);
    else hi |= c << (8 * (i - 4));
  }
  return make_uint2(lo, hi);
}

// Codes of 8 values of a row with scale `scale` (the mode's recipe; the
// runtime mode's rows with a finite scale take the fast path above).
template <int kQdt, int kMode>
__device__ __forceinline__ uint2 codes8(const Row8& r, float scale) {
  if (kMode == 0 && __builtin_isfinite(scale)) return codes8_fast<kQdt>(r, scale, 1.0f / scale);
  float inv = 0.0f;
  if (kMode == 1) inv = scale == 0.0f ? 0.0f : 1.0f / scale;
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) lo |= quant1<kQdt, kMode>(r.v[i], scale, inv) << (8 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) hi |= quant1<kQdt, kMode>(r.v[4 + i], scale, inv) << (8 * i);
  return make_uint2(lo, hi);
}

template <int kQdt, int kMode>
__device__ __forceinline__ void store8(uint8_t* dst, const Row8& r, float scale) {
  *reinterpret_cast<uint2*>(dst) = codes8<kQdt, kMode>(r, scale);
}

// max that keeps NaN sticky, like a jnp/np reduction (fmaxf drops NaN)
__device__ __forceinline__ float nanmax(float a, float b) {
  float r = fmaxf(a, b);
  return a != a ? a : (b != b ? b : r);
}

__device__ __forceinline__ float amax8(const Row8& r) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = nanmax(m, fabsf(r.v[i]));
  return m;
}

}  // namespace qmoe_rq
