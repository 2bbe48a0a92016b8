// Problem description shared by the skinny (decode) and tiled (prefill)
// grouped GEMM kernels.
//
// A grouped GEMM computes, for every group g and every compact row R in
// [group_offs[g], group_offs[g+1]):
//     acc[R, n] = sum_k A[arow(R), k] * W[g, n, k]          (n < N)
// then the epilogue applies the format's scales, the optional bias, the
// optional fused gate/up activation (gate = column n, up = column
// n + N/2, output column n < N/2), the optional per-row routing weight, and
// stores bf16 at Y[yrow(R), n_out].
// A dense linear is the one-group case (group_offs == nullptr, rows [0, M)).
#pragma once

#include "qmoe_common.h"

enum QmoeKind {
  QK_W8A8_PC = 0,   // A e4m3/int8 codes + per-row f32 scale; W codes + per-channel f32 scale
  QK_W8A8_BLK = 1,  // A e4m3 + per-(row,128) f32 scale; W e4m3 + per-(n/bn, 128) f32 scale
  QK_W8A16_PC = 2,  // A bf16; W e4m3 + per-channel f32 scale
  QK_W4A16_MX = 3,  // A bf16; W e2m1 (2 per byte, low nibble = even k) + e8m0 per 32 k
  QK_W16A16 = 4,    // A bf16; W bf16
  QK_W4A16_NV = 5,  // A bf16; W e2m1 (as QK_W4A16_MX) + bf16 scale per 16 k
  QK_W4A16_I4 = 6,  // A bf16; W 4-bit integers, offset binary (nibble = v + 8), packed as
                    // QK_W4A16_MX, + bf16 scale per wq_group k (32, 64 or 128)
  QK_W8A16_BLK = 8,  // A bf16; W e4m3 + f32 scale per (n / bn, 128 k), dequantized in bf16:
                     // each weight is bf16(code * bf16(scale))
  QK_W4A4_MX = 9,    // A e2m1 (packed as W) + e8m0 byte per (row, 32 k) in a_scale; W as
                     // QK_W4A16_MX; both scales applied by the MFMA (the 1-byte tile kernels' MX
                     // modes, dense and grouped)
};
// The host maps the descriptor kind QMOE_W8A8_GMM (7) onto QK_W8A8_BLK with
// a_kshift = 2 (activation scales per 512 columns) and w_kshift = 31 (one
// weight scale per row: per-channel); wfmt 1 runs it on int8 codes.

// bf16 activations (the other kinds take 1-byte activation codes)
QMOE_HD constexpr bool kind_abf16(int kind) {
  return kind == QK_W8A16_PC || kind == QK_W4A16_MX || kind == QK_W16A16 || kind == QK_W4A16_NV ||
         kind == QK_W4A16_I4 || kind == QK_W8A16_BLK;
}

// 4-bit weights (two codes per byte, the even k in the low nibble)
QMOE_HD constexpr bool kind_w4(int kind) {
  return kind == QK_W4A16_MX || kind == QK_W4A16_NV || kind == QK_W4A16_I4;
}

typedef float f32x2 __attribute__((ext_vector_type(2)));

// 8 e2m1 codes (one dword, low nibble first) times a bf16-valued scale ->
// 8 bf16, each the round-to-nearest-even of code * scale: the product of a
// 2-bit and an 8-bit significand is exact in float32, so this is the one
// rounding of the reference's bf16 multiply (`kernels/megablox/gmm_v2.py:
// 452-462`). The scaled conversion instructions apply only the exponent of
// their scale operand, so the codes are converted unscaled and multiplied.
__device__ __forceinline__ uint4 nvfp4x8_to_bf16(uint32_t d, float s) {
  const f32x2 f0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 0);
  const f32x2 f1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 1);
  const f32x2 f2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 2);
  const f32x2 f3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 3);
  union {
    bf16x2 h[4];
    uint4 u;
  } r;
  r.h[0] = __builtin_convertvector(f32x2{f0[0] * s, f0[1] * s}, bf16x2);
  r.h[1] = __builtin_convertvector(f32x2{f1[0] * s, f1[1] * s}, bf16x2);
  r.h[2] = __builtin_convertvector(f32x2{f2[0] * s, f2[1] * s}, bf16x2);
  r.h[3] = __builtin_convertvector(f32x2{f3[0] * s, f3[1] * s}, bf16x2);
  return r.u;
}

// 8 offset-binary 4-bit integers (one dword, low nibble first; value =
// nibble - 8) times a bf16-valued scale -> 8 bf16, each the
// round-to-nearest-even of value * scale (the reference's bf16 multiply of
// the int4 weight by its bf16 scale). nibble * s + (-8 s) is computed by one
// fma whose exact result (a 4-bit by 8-bit significand product) is
// representable, so the only rounding is the final bf16 one.
__device__ __forceinline__ uint4 int4x8_to_bf16(uint32_t d, float s) {
  const uint32_t lo = d & 0x0f0f0f0fu;         // nibbles 0, 2, 4, 6 in bytes 0..3
  const uint32_t hi = (d >> 4) & 0x0f0f0f0fu;  // nibbles 1, 3, 5, 7
  const float ns = -8.0f * s;
  union {
    bf16x2 h[4];
    uint4 u;
  } r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = fmaf((float)((lo >> (8 * j)) & 0xffu), s, ns);
    const float b = fmaf((float)((hi >> (8 * j)) & 0xffu), s, ns);
    r.h[j] = __builtin_convertvector(f32x2{a, b}, bf16x2);
  }
  return r.u;
}

enum QmoeAct {
  QA_NONE = 0,
  QA_SILU = 1,
  QA_SWIGLUOAI = 2,  // alpha = p0 (1.702), limit = p1 (7.0)
  QA_GELU_TANH = 3,
  QA_SILU_CLAMP = 4,  // limit = p0 (10.0)
  QA_SITU = 5,        // beta = p0, linear_beta = p1 (<= 0: none)
};

struct GemmParams {
  // A operand
  const void* a;           // codes (1 byte) or bf16, row-major
  int64_t lda;             // row stride in elements
  const float* a_scale;    // W8A8: per-row [rows] or per-(row,kb) [rows, lds_a];
                           // QK_W4A4_MX: e8m0 bytes [rows, lds_a]
  int64_t lds_a;           // row stride of a_scale (1 for per-row; bytes for QK_W4A4_MX)
  const int32_t* a_rows;   // optional gather: physical A row of compact row R
  // W operand, group g at w + g * w_gstride (bytes); row n at + n * ldw
  const uint8_t* w;
  int64_t ldw;             // bytes per weight row
  int64_t w_gstride;
  const void* w_scale;     // f32 [N] | f32 [N/bn, ldws] | u8 [N, ldws] | bf16 [N, ldws] (NVFP4, INT4)
  int64_t ldws;            // row stride of w_scale (elements)
  int64_t ws_gstride;      // group stride of w_scale (elements)
  int32_t ws_bn;           // rows of W sharing one block-scale row (1 or 128)
  // QK_W8A8_BLK: the scale of 128-k step s is a_scale[row, s >> a_kshift]
  // and w_scale[n / ws_bn, s >> w_kshift] (0: 128-column blocks; 2: 512;
  // 31: one scale for the whole row)
  int32_t a_kshift;
  int32_t w_kshift;
  int32_t wq_group;        // QK_W4A16_I4: k values per scale (32, 64 or 128)
  const float* bias;       // optional f32 [G, N]
  int64_t bias_gstride;
  // rows / groups
  const int32_t* group_offs;  // [G+1] compact row offsets, or nullptr (one group)
  const int32_t* active;      // optional list of non-empty groups (slot -> group)
  const int32_t* num_active;  // device scalar: number of valid slots in `active`
  int32_t slots;              // number of groups (or capacity of `active`)
  int32_t M;                  // total compact rows
  int32_t N;                  // weight rows (2*I when an activation is fused)
  int32_t K;
  int32_t wfmt;               // QK_W8A8_PC only: 0 e4m3, 1 int8
  int32_t a_quant;            // QK_W8A8_PC, streaming kernel: A holds bf16 rows that the kernel
                              // quantizes per row (runtime recipe, wfmt's codes) before the MFMAs;
                              // a_scale then receives the row scales (for the split-K finish)
  // epilogue
  int32_t act;
  float act_p0, act_p1;
  const uint16_t* row_weight;  // optional bf16 per compact row
  uint16_t* y;
  int64_t ldy;
  const int32_t* y_rows;       // optional scatter: destination row of compact row R
  // split-K workspace (skinny kernel only)
  float* partial;
  int32_t ksplit;
  // dense streaming kernel only: gridDim.z slices of row_split rows each
  // (slice z: rows [z * row_split, +row_split)), all reading the one weight
  // matrix; 0: the grid's z dimension is the groups
  int32_t row_split;
  // Fused decode MoE (skinny kernel only, ksplit 1, no bias). x0 != 0: group
  // 0 is the layer's shared expert, with its own weights w_x / scales ws_x
  // (same layout, n_x weight rows), and group g >= 1 is expert g - 1 of w /
  // w_scale. y32 != nullptr: the epilogue multiplies by row_coeff[R] and
  // stores float32 at y32[R * ldy + n], folding the absolute maximum of each
  // (row, 2^bshift columns) block into bmax[R * ldb + n >> bshift] (float32
  // bits, atomic max; the values are non-negative, so integer order is float
  // order). The extra group needs no dispatch metadata: its workgroups start
  // streaming without waiting for the active list.
  int32_t x0;
  int32_t n_x;
  int32_t rows_x;  // rows of the extra group: compact rows [0, rows_x), always slot 0
  const uint8_t* w_x;
  const void* ws_x;
  const float* row_coeff;
  float* y32;
  uint32_t* bmax;
  int32_t bshift;
  int32_t ldb;
};

// Group g's slice of a per-group array with group stride gs (elements); with
// p.x0, group 0 is the extra group's own array and the others shift down.
template <typename T>
__device__ __forceinline__ const T* group_slice(const GemmParams& p, const T* base, const void* xbase, int64_t gs,
                                                int g) {
  if (p.x0) return g == 0 ? static_cast<const T*>(xbase) : base + (int64_t)(g - 1) * gs;
  return base + (int64_t)g * gs;
}

__device__ __forceinline__ float qmoe_sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Fused gate/up activations, `kernels/megablox/gmm_v2.py:30-58, 84-122` of the
// reference (gelu is jax.nn.gelu's default tanh approximation).
__device__ __forceinline__ float qmoe_act(int act, float g, float u, float p0, float p1) {
  switch (act) {
    case QA_SILU:
      return g * qmoe_sigmoid(g) * u;
    case QA_SWIGLUOAI: {
      g = fminf(g, p1);
      u = fminf(fmaxf(u, -p1), p1);
      return (u + 1.0f) * (g * qmoe_sigmoid(p0 * g));
    }
    case QA_GELU_TANH: {
      const float c = 0.7978845608028654f;  // sqrt(2/pi)
      float t = tanhf(c * (g + 0.044715f * g * g * g));
      return 0.5f * g * (1.0f + t) * u;
    }
    case QA_SILU_CLAMP: {
      g = fminf(g, p0);
      u = fminf(fmaxf(u, -p0), p0);
      return g * qmoe_sigmoid(g) * u;
    }
    case QA_SITU: {
      float gg = p0 * tanhf(g / p0) * qmoe_sigmoid(g);
      if (p1 > 0.0f) u = p1 * tanhf(u / p1);
      return gg * u;
    }
    default:
      return g;
  }
}
