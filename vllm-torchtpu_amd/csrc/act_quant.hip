// Row quantizer: bf16/f32 rows -> e4m3 or int8 codes + float32 scales.
//
// One kernel covers the two quantizers of the reference, which round
// differently (both restated from the reference source):
//  * RUNTIME activation quant, kernels/quantized_matmul/util.py:294-318
//    (quantize_block): scale = absmax / qmax (a division), codes x / scale.
//    fp8 target: float32 arithmetic; int8 target: bf16 arithmetic (the
//    reference's qmax is a weakly typed Python int, so JAX stays in bf16):
//    scale = bf16(absmax / 127), codes = rint(bf16(x / scale)). A zero scale
//    becomes 1.
//  * LOAD-TIME weight quant, layers/core/quantization.py:232-318
//    (quantize_tensor): scale = absmax * f32(1/qmax) (reciprocal multiply),
//    inv = scale == 0 ? 0 : 1/scale, codes clamp(x * inv); int rounds half to
//    even. A zero scale stays 0.
//  * GROUPED-GEMM activation quant, kernels/megablox/gmm_v2.py:508-536
//    (the quantized-lhs regime of gmm_v2, taken for weight blocks of 256 or
//    more columns, per-channel weights included): per (row, 512-column
//    block) from column 0, the last block partial, in bf16 arithmetic (the
//    block's dtype_max is a Python float): scale = bf16(absmax / qmax),
//    inv = scale == 0 ? 0 : bf16(1 / scale), codes = e4m3 RNE of
//    bf16(x * inv) (no clip), or for int8 that bf16 value truncated toward
//    zero (`.astype(int8)`). A zero scale stays 0.
// Granularity: one scale per row, or per (row, 128-column block); the
// grouped-GEMM mode per (row, 512-column block).
//
// Launch: one 256-thread workgroup per row (per-row scale; 128 threads for
// many rows of 2049-8192 columns); thread t owns 8 consecutive columns per
// 8 x (threads)-column stride, so a 128-column block is
// exactly 16 adjacent lanes of one wavefront (reduced with shuffles, no LDS).
// Per-block scales need no row-wide reduction, so a row's 2048-column spans
// go to separate workgroups (grid.y): a decode row is quantized in one
// memory round trip instead of one per span. Per-row scales of a few rows
// (decode) also spread a row's spans over grid.y: every workgroup reads the
// whole row for the absmax (from L2 after the first) and encodes only its
// own span, so the per-element division and encode run on S CUs instead of
// one.

#include <algorithm>

#include "qmoe_common.h"
#include "row_quant.h"

namespace {

constexpr int kThreads = 256;

using namespace qmoe_rq;

template <int kQdt, int kMode, bool kInF32, bool kBlock, int kNT, bool kSpan = false>
__global__ __launch_bounds__(kNT) void row_quant_kernel(
    const void* __restrict__ x, int64_t ldx, int64_t K, uint8_t* __restrict__ q,
    int64_t ldq, float* __restrict__ scales, int64_t lds) {
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t xbase = row * ldx;
  uint8_t* qrow = q + row * ldq;
  if (kBlock) {
    // 16 lanes per 128-column block; this workgroup's 2048-column span
    const int64_t c = (int64_t)blockIdx.y * (kNT * 8) + (int64_t)tid * 8;
    if (c < K) {
      Row8 r = load8<kInF32>(x, xbase + c);
      float m = amax8(r);
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) m = nanmax(m, __shfl_xor(m, o, 64));
      float s = make_scale<kQdt, kMode>(m);
      store8<kQdt, kMode>(qrow + c, r, s);
      if ((tid & 15) == 0) scales[row * lds + c / 128] = s;
    }
    return;
  }
  __shared__ float red[kNT / 64];
  float m = 0.0f;
  // rows of up to kHeld spans stay in registers: all their loads are in
  // flight at once and the codes are written from the registers
  constexpr int kHeld = kNT >= 1024 ? 4 : 8;
  const bool held = K <= (int64_t)kHeld * kNT * 8;
  Row8 r[kHeld];
  if (held) {
#pragma unroll
    for (int i = 0; i < kHeld; ++i) {
      const int64_t c = (int64_t)(i * kNT + tid) * 8;
      if (c < K) {
        r[i] = load8<kInF32>(x, xbase + c);
        m = nanmax(m, amax8(r[i]));
      }
    }
  } else {
    for (int64_t c = (int64_t)tid * 8; c < K; c += kNT * 8)
      m = nanmax(m, amax8(load8<kInF32>(x, xbase + c)));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = nanmax(m, __shfl_xor(m, o, 64));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (int w = 1; w < kNT / 64; ++w) m = nanmax(m, red[w]);
  float s = make_scale<kQdt, kMode>(m);
  if (kSpan) {
    // held rows only (the host checks); span i of the row is this
    // workgroup's when i == blockIdx.y
#pragma unroll
    for (int i = 0; i < kHeld; ++i) {
      const int64_t c = (int64_t)(i * kNT + tid) * 8;
      if (i == (int)blockIdx.y && c < K) store8<kQdt, kMode>(qrow + c, r[i], s);
    }
    if (tid == 0 && blockIdx.y == 0) scales[row * lds] = s;
    return;
  }
  if (held) {
#pragma unroll
    for (int i = 0; i < kHeld; ++i) {
      const int64_t c = (int64_t)(i * kNT + tid) * 8;
      if (c < K) store8<kQdt, kMode>(qrow + c, r[i], s);
    }
  } else {
    for (int64_t c = (int64_t)tid * 8; c < K; c += kNT * 8)
      store8<kQdt, kMode>(qrow + c, load8<kInF32>(x, xbase + c), s);
  }
  if (tid == 0) scales[row * lds] = s;
}

// Grouped-GEMM quant (mode 2): one wavefront per 512-column block, lane l
// holding columns [8 l, 8 l + 8) of it; every lane takes part in the
// reduction (lanes past K contribute 0), only lanes inside K store.
template <int kQdt>
__global__ __launch_bounds__(kThreads) void gmm_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                             int64_t K, uint8_t* __restrict__ q, int64_t ldq,
                                                             float* __restrict__ scales, int64_t lds) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int64_t blk = (int64_t)blockIdx.y * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t c = blk * 512 + lane * 8;
  if (blk * 512 >= K) return;  // the whole wavefront is past K
  const bool live = c < K;
  Row8 r;
  if (live) r = load8<false>(x, row * ldx + c);
  else
#pragma unroll
    for (int i = 0; i < 8; ++i) r.v[i] = 0.0f;
  float m = amax8(r);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = nanmax(m, __shfl_xor(m, o, 64));
  const float qmax = kQdt == 0 ? 448.0f : 127.0f;
  const float scale = bf16_round(m / qmax);
  const float inv = scale == 0.0f ? 0.0f : bf16_round(1.0f / scale);
  if (live) {
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = bf16_round(r.v[i] * inv);
      uint32_t code;
      if (kQdt == 0) {
        code = f32_to_e4m3(v);
      } else {
        float t = v != v ? 0.0f : fminf(fmaxf(truncf(v), -128.0f), 127.0f);
        code = (uint32_t)(int32_t)t & 0xffu;
      }
      w[i >> 2] |= code << (8 * (i & 3));
    }
    *reinterpret_cast<uint2*>(q + row * ldq + c) = make_uint2(w[0], w[1]);
  }
  if (lane == 0) scales[row * lds + blk] = scale;
}

// ---- MX activation quant (e2m1 codes + e8m0 byte per 32 columns) ----
// The reference's ue8m0 block quantizer, layers/core/quantization.py:232-318
// (quantize_tensor with use_ue8m0) with e2m1 as the target: per 32-column
// block scale = amax * f32(1/6), snapped up to the smallest power of two 2^e
// >= scale (the value its ceil(log2) + repair step computes; e clamped to
// [-127, 127], byte e + 127); values x * 2^-e clamped to +-6 and encoded by
// the reference's e2m1 encoder, compressed_tensors_moe/utils.py:167-183
// (magnitude = number of the edges 0.25 0.75 1.25 1.75 2.5 3.5 5 strictly
// below |v|, sign 8 for v < 0). Thread t owns 8 consecutive columns per
// 2048-column span (grid.y), so a block is 4 adjacent lanes; columns K..Kp-1
// are zero blocks (codes 0, byte 0). Outputs: packed codes (low nibble = even
// column, one dword per lane) + scale bytes, and/or the dequantized values
// as bf16 (exact: an e2m1 value times a power of two), for callers that run
// the 4-bit activations through a bf16-activation kernel.
__device__ __forceinline__ int mx_exponent_ceil(float scale) {
  const uint32_t b = f32_bits(scale);
  const int be = (int)((b >> 23) & 0xffu);
  const uint32_t mant = b & 0x7fffffu;
  if (be == 255) return 127;
  // subnormal scales: 2^-127 = 2^22 ulps; at or below it the clamp gives -127
  if (be == 0) return mant > (1u << 22) ? -126 : -127;
  const int e = be - 127 + (mant != 0u ? 1 : 0);
  return e < -127 ? -127 : (e > 127 ? 127 : e);
}

// Work split: the (row, 8-column group) pairs in row-major order, one group
// per lane per step, kMxIter groups kThreads apart per loop trip (several
// 16-byte loads in flight), a grid-stride loop over all of them: rows of any
// length keep every lane busy (a per-row grid would leave most of a row's
// last 2048-column span idle at K = 2880). Kp % 32 == 0 keeps the 4 groups
// of a 32-column block in one row and in 4 adjacent lanes, which are live or
// past the end together.
constexpr int kMxIter = 4;
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// e2m1 magnitude code (0..7) of |v| <= 6 by the reference encoder's edges
// (ties to the lower magnitude), from the f32 bits ab = bits(|v|): at 1.0 and
// above, the f32 rounded to one mantissa bit with ties toward zero (add
// 2^21 - 1, drop 22 bits; the carry moves 1.75+ to 2.0, 5.0 stays 4.0) is
// 254 + 2 (exponent) + mantissa bit = code + 252. Below 1.0 the same rounding
// of |v| + 1 (exact for the codes that matter: |v| > 2^-8) gives 254, 255
// and 256 for codes 0, 1 and 2 (edges 0.25 and 0.75).
__device__ __forceinline__ uint32_t e2m1_mag(uint32_t ab) {
  const bool small = ab < 0x3f800000u;
  const float t = small ? bits_f32(ab) + 1.0f : bits_f32(ab);
  return ((f32_bits(t) + 0x1fffffu) >> 22) - (small ? 254u : 252u);
}

template <bool kCodes, bool kFake>
__global__ __launch_bounds__(kThreads) void mx_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx, int K,
                                                            int Kp, int total, uint8_t* __restrict__ q, int64_t ldq,
                                                            uint8_t* __restrict__ scales, int64_t lds,
                                                            uint16_t* __restrict__ xq, int64_t ldxq) {
  const uint32_t gpr = (uint32_t)Kp / 8u;  // groups per row
  const int step = (int)gridDim.x * kThreads * kMxIter;
  for (int g0 = (int)blockIdx.x * kThreads * kMxIter + (int)threadIdx.x; g0 < total; g0 += step) {
    uint4 raw[kMxIter];  // 8 bf16 values
    int64_t row[kMxIter];
    int c[kMxIter];
#pragma unroll
    for (int it = 0; it < kMxIter; ++it) {
      const int g = g0 + it * kThreads;
      const uint32_t rr = (uint32_t)g / gpr;
      row[it] = rr;
      c[it] = (int)(((uint32_t)g - rr * gpr) * 8u);
      raw[it] = g < total && c[it] < K ? *reinterpret_cast<const uint4*>(x + row[it] * ldx + c[it])
                                       : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int it = 0; it < kMxIter; ++it) {
      const uint32_t wd[4] = {raw[it].x, raw[it].y, raw[it].z, raw[it].w};
      // block amax on the absolute-value bits of the bf16 pairs (ordered
      // like the values, inf and NaN above every finite value): packed
      // 16-bit maxima
      u16x2 m2 = __builtin_bit_cast(u16x2, wd[0] & 0x7fff7fffu);
#pragma unroll
      for (int i = 1; i < 4; ++i) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, wd[i] & 0x7fff7fffu));
      uint32_t mb = (uint32_t)max(m2.x, m2.y) << 16;
      mb = max(mb, (uint32_t)__shfl_xor((int)mb, 1, 64));
      mb = max(mb, (uint32_t)__shfl_xor((int)mb, 2, 64));
      // a block holding an inf or NaN: codes 0 and scale byte 255 (the e8m0
      // NaN encoding), so the block reads back as NaN and its neighbours
      // keep their own codes
      const bool bad = mb >= 0x7f800000u;
      const int e = mx_exponent_ceil(bits_f32(bad ? 0u : mb) * (1.0f / 6.0f));
      const float inv = __builtin_amdgcn_ldexpf(1.0f, -e);
      if (g0 + it * kThreads >= total) continue;
      uint32_t w = 0;
      uint32_t d[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float xv = bits_f32(i & 1 ? wd[i >> 1] & 0xffff0000u : wd[i >> 1] << 16);
        // |x| 2^-e <= amax 2^-e <= 6: the reference's clamp to +-6 never
        // binds; + 0.0f turns -0 into +0 (the encoder's sign is v < 0)
        const uint32_t vb = f32_bits(xv * inv + 0.0f);
        const uint32_t mag = bad ? 0u : e2m1_mag(vb & 0x7fffffffu);
        const uint32_t code = bad ? 0u : mag | ((vb >> 28) & 8u);
        const float v = bits_f32(vb);
        w |= code << (4 * i);
        if (kFake) {
          // e2m1 magnitude of the code, times 2^e: exact in bf16 (3 significant bits)
          const float mv =
              mag < 4u ? 0.5f * (float)mag : (mag < 6u ? (float)(mag - 2u) : (mag == 6u ? 4.0f : 6.0f));
          const float dv = __builtin_amdgcn_ldexpf(v < 0.0f ? -mv : mv, e);
          d[i >> 1] |= (bad ? 0x7fc0u : f32_bits(dv) >> 16) << (16 * (i & 1));
        }
      }
      if (kCodes) {
        *reinterpret_cast<uint32_t*>(q + row[it] * ldq + c[it] / 2) = w;
        if ((threadIdx.x & 3) == 0) scales[row[it] * lds + c[it] / 32] = bad ? (uint8_t)255 : (uint8_t)(e + 127);
      }
      if (kFake && c[it] < K)
        *reinterpret_cast<uint4*>(xq + row[it] * ldxq + c[it]) = make_uint4(d[0], d[1], d[2], d[3]);
    }
  }
}

template <int kQdt, int kMode, bool kInF32, bool kBlock>
void launch_rq(const void* x, int64_t ldx, int64_t M, int64_t K, uint8_t* q, int64_t ldq,
               float* s, int64_t lds, hipStream_t st) {
  const unsigned spans = kBlock ? (unsigned)cdiv<int64_t>(K, kThreads * 8) : 1u;
  // a few long rows (decode): each row's 2048-column spans are encoded by
  // separate workgroups (rows of up to 8 spans, held in registers), or, for
  // longer rows, 1024 threads per row
  if (!kBlock && M <= 256 && K > kThreads * 8 && K <= 8 * kThreads * 8)
    hipLaunchKernelGGL((row_quant_kernel<kQdt, kMode, kInF32, kBlock, kThreads, true>),
                       dim3((unsigned)M, (unsigned)cdiv<int64_t>(K, kThreads * 8)), dim3(kThreads), 0, st, x, ldx,
                       K, q, ldq, s, lds);
  else if (!kBlock && M <= 64 && K > kThreads * 8)
    hipLaunchKernelGGL((row_quant_kernel<kQdt, kMode, kInF32, kBlock, 1024>), dim3((unsigned)M), dim3(1024), 0,
                       st, x, ldx, K, q, ldq, s, lds);
  else if (!kBlock && M > 256 && K > 2048 && K <= 128 * 8 * 8)
    // many rows of 2049-8192 columns: 128 threads per row, the row still held
    // in registers (measured on MI355X, 4096 rows of 4096 / 7168 columns,
    // FP8: 14.7 / 19.5 -> 12.6 / 18.6 us; 8192 rows of 4096: 24.5 -> 20.7 us;
    // 512 threads and more are slower, and rows of 14336 columns, which 128
    // threads would stream twice, stay on 256)
    hipLaunchKernelGGL((row_quant_kernel<kQdt, kMode, kInF32, kBlock, 128>), dim3((unsigned)M), dim3(128), 0, st, x,
                       ldx, K, q, ldq, s, lds);
  else
    hipLaunchKernelGGL((row_quant_kernel<kQdt, kMode, kInF32, kBlock, kThreads>), dim3((unsigned)M, spans),
                       dim3(kThreads), 0, st, x, ldx, K, q, ldq, s, lds);
}

}  // namespace

// See include/qmoe.h for the contract.
extern "C" int qmoe_row_quant(const void* x, int64_t ldx, int in_f32, int64_t M, int64_t K,
                              int qdtype, int mode, int block, void* q, int64_t ldq,
                              float* scales, int64_t lds, hipStream_t stream) {
  if (M < 0 || K <= 0 || (K % 8) != 0) return QMOE_ERR_ARG;
  if (qdtype < 0 || qdtype > 2) return QMOE_ERR_ARG;
  if (mode == 2) {  // grouped-GEMM activation quant: bf16 rows, 512-column blocks
    if (qdtype == 2) return QMOE_ERR_ARG;  // float weights meet e4m3 activations there
    if (block != 512 || in_f32 || lds < cdiv<int64_t>(K, 512)) return QMOE_ERR_ARG;
    if (M == 0) return QMOE_OK;
    const dim3 grid((unsigned)M, (unsigned)cdiv<int64_t>(K, 512 * (kThreads / 64)));
    if (qdtype == 0)
      hipLaunchKernelGGL(gmm_quant_kernel<0>, grid, dim3(kThreads), 0, stream, static_cast<const uint16_t*>(x),
                         ldx, K, static_cast<uint8_t*>(q), ldq, scales, lds);
    else
      hipLaunchKernelGGL(gmm_quant_kernel<1>, grid, dim3(kThreads), 0, stream, static_cast<const uint16_t*>(x),
                         ldx, K, static_cast<uint8_t*>(q), ldq, scales, lds);
    return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
  }
  if (mode != 0 && mode != 1) return QMOE_ERR_ARG;
  if (block != 0 && block != 128) return QMOE_ERR_ARG;
  if (block == 128 && (K % 128) != 0) return QMOE_ERR_ARG;
  if (in_f32 && mode == 0) return QMOE_ERR_ARG;  // runtime path takes bf16 activations
  if (M == 0) return QMOE_OK;
  uint8_t* qq = static_cast<uint8_t*>(q);
  const bool blk = block == 128;
#define QMOE_RQ(QD, MD, F32, BLK) launch_rq<QD, MD, F32, BLK>(x, ldx, M, K, qq, ldq, scales, lds, stream)
  if (qdtype == 2) {  // e5m2: per-row scales (runtime, or load time from f32 / bf16)
    if (blk) return QMOE_ERR_ARG;
    if (mode == 0) QMOE_RQ(2, 0, false, false);
    else if (in_f32) QMOE_RQ(2, 1, true, false);
    else QMOE_RQ(2, 1, false, false);
  } else if (mode == 0) {
    if (qdtype == 0) { if (blk) QMOE_RQ(0, 0, false, true); else QMOE_RQ(0, 0, false, false); }
    else { if (blk) QMOE_RQ(1, 0, false, true); else QMOE_RQ(1, 0, false, false); }
  } else if (in_f32) {
    if (qdtype == 0) { if (blk) QMOE_RQ(0, 1, true, true); else QMOE_RQ(0, 1, true, false); }
    else { if (blk) QMOE_RQ(1, 1, true, true); else QMOE_RQ(1, 1, true, false); }
  } else {
    if (qdtype == 0) { if (blk) QMOE_RQ(0, 1, false, true); else QMOE_RQ(0, 1, false, false); }
    else { if (blk) QMOE_RQ(1, 1, false, true); else QMOE_RQ(1, 1, false, false); }
  }
#undef QMOE_RQ
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}

// See include/qmoe.h for the contract.
extern "C" int qmoe_mx_quant(const void* x, int64_t ldx, int64_t M, int64_t K, int64_t Kp, void* q, int64_t ldq,
                             void* scales, int64_t lds, void* xq, int64_t ldxq, hipStream_t stream) {
  if (!x || M < 0 || K <= 0 || (K % 32) != 0 || Kp < K || (Kp % 32) != 0) return QMOE_ERR_ARG;
  if (ldx < K || (ldx % 8) != 0 || (reinterpret_cast<uintptr_t>(x) & 15)) return QMOE_ERR_ARG;
  const bool codes = q != nullptr;
  if (!codes && !xq) return QMOE_ERR_ARG;
  if (codes && (!scales || ldq < Kp / 2 || (ldq % 4) != 0 || lds < Kp / 32 || (reinterpret_cast<uintptr_t>(q) & 3)))
    return QMOE_ERR_ARG;
  if (xq && (ldxq < K || (ldxq % 8) != 0 || (reinterpret_cast<uintptr_t>(xq) & 15))) return QMOE_ERR_ARG;
  if (M == 0) return QMOE_OK;
  // group indices in 32 bits, including the last loop trip's overshoot
  const int64_t total = M * (Kp / 8);
  if (total + (int64_t)kThreads * kMxIter * 4096 > 0x7fffffffLL) return QMOE_ERR_ARG;
  // enough workgroups for every CU several times over, at most one loop trip
  // of groups each when that is fewer
  const dim3 grid((unsigned)std::min<int64_t>(cdiv<int64_t>(total, kThreads * kMxIter), 4096));
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  uint8_t* qb = static_cast<uint8_t*>(q);
  uint8_t* sb = static_cast<uint8_t*>(scales);
  uint16_t* fb = static_cast<uint16_t*>(xq);
  if (codes && xq)
    hipLaunchKernelGGL((mx_quant_kernel<true, true>), grid, dim3(kThreads), 0, stream, xb, ldx, (int)K, (int)Kp,
                       (int)total, qb, ldq, sb, lds, fb, ldxq);
  else if (codes)
    hipLaunchKernelGGL((mx_quant_kernel<true, false>), grid, dim3(kThreads), 0, stream, xb, ldx, (int)K, (int)Kp,
                       (int)total, qb, ldq, sb, lds, fb, ldxq);
  else
    hipLaunchKernelGGL((mx_quant_kernel<false, true>), grid, dim3(kThreads), 0, stream, xb, ldx, (int)K, (int)Kp,
                       (int)total, qb, ldq, sb, lds, fb, ldxq);
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
