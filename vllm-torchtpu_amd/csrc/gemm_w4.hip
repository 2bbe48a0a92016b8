// Tiled (prefill) GEMM for bf16 activations x 4-bit weights (W4A16: codes
// two per byte with the even k in the low nibble; MXFP4: e2m1 + one e8m0
// scale per 32 k; NVFP4: e2m1 + one bf16 scale per 16 k; INT4: offset-binary
// integers + one bf16 scale per 32 / 64 / 128 k), dense or grouped.
//
// Restates the reference's W4A16 path (`layers/adapter/linear_common.py:
// 188-209` -> `kernels/megablox/gmm_v2.py:452-462`: blocks below 256 k are
// dequantized to the activation dtype and multiplied in bf16 with f32
// accumulation). Expanding the codes on the fly gives the same bf16 weights
// as dequantizing the whole matrix first: exact for e8m0 scales, one
// round-to-nearest-even of value * scale for the bf16 NVFP4 / INT4 scales.
//
// Design for gfx950 (one workgroup of 4 wavefronts per CU), on the machinery
// of the 1-byte tiled kernel (gemm_tile.h):
//  * output tile BM tokens x 256 weight rows of 32 x 32 MFMA blocks (weight
//    block first, activation block second: v_mfma_f32_32x32x16_bf16);
//  * a stage is 64 k: 128 bytes of each activation row and 32 bytes of each
//    weight row, copied straight into a ring of four LDS stages (distinct
//    arrays) four stages ahead; each lane loads the scale bytes it needs
//    with the copies (bounded buffer loads into a 4-deep register ring);
//  * in a stage, lane l (row l % 32, half h = l / 32) feeds k in
//    [32h, 32h + 32): that is one e8m0 block (two NVFP4 blocks), 16
//    contiguous code bytes (one LDS read for all four 16-k MFMA steps) and
//    one scale byte (NVFP4: one 4-byte bf16 pair; INT4: one bf16 group
//    scale). Each 16-k step expands 8 codes to bf16 with the scale applied
//    (v_cvt_scalef32_pk_bf16_fp4 for e8m0; unscaled conversion, f32 product
//    and bf16 rounding for NVFP4 and INT4);
//    activation and weight use the same lane -> k assignment, so the
//    products pair up whatever order the MFMA sums;
//  * every operand of stage s+1 is read into the second register set during
//    the MFMAs of stage s; the activation rows are stored with the 16-byte
//    chunk c of row r at slot c ^ ((r & 7) ^ ((r >> 3) & 1)) so that the
//    MFMA operand reads are conflict-free;
//  * the shared epilogue applies bias, fused activation and routing weight
//    (the weights carry no other scale).

#include <algorithm>
#include <cstdlib>

#include "gemm_tile.h"

namespace {

using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr int kW4BN = 256;  // weight rows per tile

// The wavefronts split the 256 weight rows (each expands its own 64 rows
// once per stage and reuses them for all BM tokens); WN = 4 always.
template <int BM>
struct W4Shape {
  static constexpr int WN = 4;                  // wavefronts along weight rows
  static constexpr int WM = 1;                  // along tokens
  static constexpr int TN = kW4BN / WN;         // weight rows per wavefront
  static constexpr int TM = BM / WM;            // tokens per wavefront
  static constexpr int NI = TN / 32;
  static constexpr int MJ = TM / 32;
  static_assert(NI >= 1 && MJ >= 1, "tile too small");
};

__device__ __forceinline__ int w4_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// 8 e2m1 codes (one dword, low nibble first) -> 8 bf16 times `scale`
__device__ __forceinline__ bf16x8 w4_expand(uint32_t d, float scale) {
  union {
    bf16x2 h[4];
    bf16x8 v;
  } u;
  u.h[0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 0);
  u.h[1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 1);
  u.h[2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 2);
  u.h[3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 3);
  return u.v;
}

__device__ __forceinline__ bf16x8 as_bf16x8_u4(const uint4& x) {
  union {
    uint4 u;
    bf16x8 v;
  } c;
  c.u = x;
  return c.v;
}

// FMT: 0 MXFP4, 1 NVFP4, 2 INT4
template <int BM, bool ACT, int FMT>
__global__ __launch_bounds__(kThreads) void w4_gemm_kernel(const GemmParams p, int m_tiles, int n_tiles) {
  constexpr bool NV = FMT == 1, I4 = FMT == 2;
  using S = W4Shape<BM>;
  constexpr int BN = kW4BN;
  constexpr int NI = S::NI, MJ = S::MJ, TN = S::TN, TM = S::TM;
  constexpr int BNO = ACT ? BN / 2 : BN;  // output channels per tile
  static_assert(!ACT || NI % 2 == 0, "fused activation pairs gate and up blocks");

  // four LDS stages of 64 k: activations [BM][128 B], codes [BN][32 B]
  __shared__ __align__(1024) uint8_t sA0[BM * 128], sA1[BM * 128], sA2[BM * 128], sA3[BM * 128];
  __shared__ __align__(1024) uint8_t sW0[BN * 32], sW1[BN * 32], sW2[BN * 32], sW3[BN * 32];
  __shared__ int s_info[4];
  __shared__ float s_sx[BM], s_rw[BM], s_ws[BN], s_bs[BN];
  __shared__ int s_yr[BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave % S::WN, wm = wave / S::WN;

  int g, row0, rows, ntile;
  if (p.group_offs) {
    if (!tile_group<BM>(p, blockIdx.y, g, row0, rows, s_info)) return;
    ntile = blockIdx.x;
  } else {
    int mt;
    if (!tile_dense(blockIdx.x, m_tiles, n_tiles, mt, ntile)) return;
    g = 0;
    row0 = mt * BM;
    rows = min(BM, p.M - row0);
  }
  const int n0 = ntile * BNO;
  const int nlim = ACT ? p.N / 2 : p.N;
  // global weight row of tile LDS row r (gate rows, then up rows with ACT);
  // rows past the end are clamped (their outputs are never stored)
  auto wrow_global = [&](int r) {
    if (ACT) return (r < BN / 2 ? 0 : p.N / 2) + min(n0 + (r % (BN / 2)), nlim - 1);
    return min(n0 + r, nlim - 1);
  };

  // epilogue inputs (loaded now, staged in LDS at the end): token routing
  // weight and output row; weight-row bias. No activation / channel scales.
  float e_rw = 1.0f, e_bs = 0.0f;
  int e_yr = 0;
  if (tid < BM) {
    const int R = row0 + min(tid, rows - 1);
    if (p.row_weight) e_rw = bf16_to_f32(p.row_weight[R]);
    e_yr = p.y_rows ? p.y_rows[R] : R;
  }
  if (tid < BN && p.bias) e_bs = p.bias[(int64_t)g * p.bias_gstride + wrow_global(tid)];

  // ---- LDS copies (16 bytes per lane) ----
  // activations: one instruction = 8 rows x 128 bytes (lane -> row l >> 3,
  // slot l & 7, fetching the chunk that the row's swizzle stores there);
  // codes: 32 rows x 32 bytes (lane -> row l >> 1, half l & 1). Scales:
  // lane (row l % 32, half h) of weight block i needs e8m0 byte 2*stage + h
  // of its row (NVFP4: bf16 scales 4*stage + 2h and + 1, one 4-byte load;
  // INT4: bf16 scale (64*stage + 32h) / group).
  constexpr int kSB = NV || I4 ? 2 : 1;  // bytes per scale
  constexpr int XI = BM / 32;  // activation copies per wavefront
  constexpr int WI = 2;        // code copies per wavefront
  const uint8_t* xbase = static_cast<const uint8_t*>(p.a);
  const uint8_t* wbase = p.w + (int64_t)g * p.w_gstride;
  const rsrc_t eres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(static_cast<const void*>(static_cast<const uint8_t*>(p.w_scale) + (int64_t)g * p.ws_gstride * kSB)),
      (short)0, (int)std::min<int64_t>((int64_t)p.N * p.ldws * kSB, 0x7fffffff), 0x00020000);
  const uint64_t lda_b = (uint64_t)p.lda * 2;
  uint32_t xrow[XI], woff[WI];
  int xcx[XI];
#pragma unroll
  for (int j = 0; j < XI; ++j) {
    const int r = (wave + 4 * j) * 8 + (lane >> 3);
    const int R = row0 + min(r, rows - 1);
    xrow[j] = (uint32_t)(p.a_rows ? p.a_rows[R] : R);
    xcx[j] = ((lane & 7) ^ w4_swz(r)) * 16;
  }
#pragma unroll
  for (int j = 0; j < WI; ++j) {
    const int r = (wave + 4 * j) * 32 + (lane >> 1);
    woff[j] = (uint32_t)wrow_global(r) * (uint32_t)p.ldw + (lane & 1) * 16;
  }

  // split-K: this workgroup's K range in 64-k stages
  const int NU = p.K / 64;
  const int u0 = (int)((int64_t)NU * blockIdx.z / p.ksplit);
  const int u1 = (int)((int64_t)NU * (blockIdx.z + 1) / p.ksplit);
  const int KS = u1 - u0;
  const int rl = lane & 31, kh = lane >> 5;
  auto wrow = [&](int i) { return tile_wrow<BN, TN, NI, ACT>(wn, i); };
  uint32_t eoff[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i)
    eoff[i] = (uint32_t)wrow_global(wrow(i) + rl) * (uint32_t)(p.ldws * kSB) + (NV ? kh * 4 : (I4 ? 0 : kh));
  const int lg = I4 ? (p.wq_group == 32 ? 5 : (p.wq_group == 64 ? 6 : 7)) : 0;  // log2(group)
  uint32_t we[4][NI];  // scales of the stages in flight (stage s in set s % 4)
  auto copy_stage = [&](uint8_t* dA, uint8_t* dW, int e, int ks) {
    const uint32_t st = (uint32_t)(u0 + ks);
#pragma unroll
    for (int j = 0; j < WI; ++j) {
      uint32_t o = woff[j];
      asm volatile("" : "+v"(o));
      __builtin_amdgcn_global_load_lds(wbase + (o + st * 32u), QMOE_LDS(dW + (wave + 4 * j) * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < XI; ++j) {
      uint32_t r = xrow[j];
      asm volatile("" : "+v"(r));
      const uint8_t* src = xbase + (uint64_t)r * lda_b + (st * 128u + xcx[j]);
      __builtin_amdgcn_global_load_lds(src, QMOE_LDS(dA + (wave + 4 * j) * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      if constexpr (NV) {
        we[e][i] = __builtin_amdgcn_raw_buffer_load_b32(eres, eoff[i], st * 8u, 0);
      } else if constexpr (I4) {
        const uint32_t gi = (st * 64u + (uint32_t)kh * 32u) >> lg;  // group of the lane's 32 k
        we[e][i] = __builtin_amdgcn_raw_buffer_load_b16(eres, eoff[i] + gi * 2u, 0, 0);
      } else {
        we[e][i] = __builtin_amdgcn_raw_buffer_load_b8(eres, eoff[i], st * 2u, 0);
      }
    }
  };

  uint4 wc[2][NI];  // codes: dword q feeds 16-k step q
  uint4 xa[2][MJ][4];  // activations: [block][16-k step]
  f32x16 acc[NI][MJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // The K pipeline over the first MJE 32-token blocks of the tile (MJ: all
  // of them); the accumulators of the others keep their zeros.
  auto pipeline = [&](auto mje_c) {
    constexpr int MJE = decltype(mje_c)::value;
    // ---- operands of one stage into register set t ----
    auto read_stage = [&](const uint8_t* sA, const uint8_t* sW, int t) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int r = wrow(i) + rl;
        wc[t][i] = *reinterpret_cast<const uint4*>(sW + r * 32 + kh * 16);
      }
#pragma unroll
      for (int j = 0; j < MJE; ++j) {
        const int r = wm * TM + j * 32 + rl;
        const uint8_t* row = sA + r * 128;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          xa[t][j][q] = *reinterpret_cast<const uint4*>(row + (((kh * 4 + q) ^ w4_swz(r)) * 16));
      }
    };

    // k-step outer, blocks inner: consecutive MFMAs go to different
    // accumulators, and a step's expansions overlap the previous step's MFMAs
    auto mma_stage = [&](int t, const uint32_t (&eb)[NI]) {
      float scale[NI], scale1[NI];  // NVFP4: scale for 16-k steps 0-1, scale1 for 2-3
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        if constexpr (NV) {
          scale[i] = bits_f32(eb[i] << 16);
          scale1[i] = bits_f32(eb[i] & 0xffff0000u);
        } else if constexpr (I4) {
          scale[i] = bits_f32(eb[i] << 16);
        } else {
          scale[i] = e8m0_to_f32(eb[i]);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        bf16x8 wv[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const uint32_t d = q == 0 ? wc[t][i].x : (q == 1 ? wc[t][i].y : (q == 2 ? wc[t][i].z : wc[t][i].w));
          if constexpr (NV) wv[i] = as_bf16x8_u4(nvfp4x8_to_bf16(d, q < 2 ? scale[i] : scale1[i]));
          else if constexpr (I4) wv[i] = as_bf16x8_u4(int4x8_to_bf16(d, scale[i]));
          else wv[i] = w4_expand(d, scale[i]);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < MJE; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wv[i], as_bf16x8_u4(xa[t][j][q]), acc[i][j], 0, 0, 0);
      }
    };

    constexpr int CPS = WI + XI + NI;        // vector-memory loads per wavefront per stage
    constexpr int NM = NI * MJE * 4;         // MFMAs per stage
    constexpr int NR = NI + MJE * 4;         // LDS operand reads per stage
    // Stage s lives in buffer s % 4 and is copied four stages ahead. Stage s:
    // wait for the own copy of stage s+1 -> barrier (stage s+1 has landed
    // everywhere, and every wavefront holds stage s in registers, so buffer
    // s % 4 is free) -> copy stage s+4 into it -> MFMAs of stage s with the
    // operand reads of stage s+1 among the first half and the copies among
    // the second. Copies past the end refetch the last stage into a consumed
    // buffer (never read again).
    // (stage s's scale bytes are register set s % 4; they are taken before
    // the set is reloaded with stage s+4)
    auto stage = [&](uint8_t* fA, uint8_t* fW, const uint8_t* nA, const uint8_t* nW, int e, int s, int t) {
      wait_copies_upto<2 * CPS>();
      stage_barrier();
      uint32_t eb[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) eb[i] = we[e][i];
      copy_stage(fA, fW, e, min(s + 4, KS - 1));
      mma_stage(t, eb);
      read_stage(nA, nW, t ^ 1);
      interleave<0, NM, NR, CPS>();
    };
    if (KS > 0) {
      copy_stage(sA0, sW0, 0, 0);
      copy_stage(sA1, sW1, 1, min(1, KS - 1));
      copy_stage(sA2, sW2, 2, min(2, KS - 1));
      copy_stage(sA3, sW3, 3, min(3, KS - 1));
      wait_copies_upto<3 * CPS>();
      __syncthreads();
      read_stage(sA0, sW0, 0);
      int s = 0;
      for (; s + 4 <= KS; s += 4) {
        stage(sA0, sW0, sA1, sW1, 0, s, 0);
        stage(sA1, sW1, sA2, sW2, 1, s + 1, 1);
        stage(sA2, sW2, sA3, sW3, 2, s + 2, 0);
        stage(sA3, sW3, sA0, sW0, 3, s + 3, 1);
      }
      if (s < KS) stage(sA0, sW0, sA1, sW1, 0, s, 0);
      if (s + 1 < KS) stage(sA1, sW1, sA2, sW2, 1, s + 1, 1);
      if (s + 2 < KS) stage(sA2, sW2, sA3, sW3, 2, s + 2, 0);
    }

  };
  // A tile with at most 32 (64) valid tokens -- a routed expert's last tile
  // -- runs the MFMAs of its first one (two) 32-token blocks only: the
  // others' sums belong to no token. The expansion of the weight codes, the
  // copies and the barriers are the same.
  const int rows_u = __builtin_amdgcn_readfirstlane(rows);
  if constexpr (MJ == 4) {
    if (rows_u <= 32) pipeline(std::integral_constant<int, 1>{});
    else if (rows_u <= 64) pipeline(std::integral_constant<int, 2>{});
    else pipeline(std::integral_constant<int, 4>{});
  } else if constexpr (MJ == 2) {
    if (rows_u <= 32) pipeline(std::integral_constant<int, 1>{});
    else pipeline(std::integral_constant<int, 2>{});
  } else {
    pipeline(std::integral_constant<int, MJ>{});
  }
  if (p.ksplit > 1) {
    tile_store_partials<BN, TN, TM, NI, MJ, ACT, false>(p, acc, row0, rows, n0, nlim, wn, wm, lane);
    return;
  }
  wait_copies_upto<0>();
  __syncthreads();  // every wavefront is done with the stage buffers
  if (tid < BM) {
    s_sx[tid] = 1.0f;
    s_rw[tid] = e_rw;
    s_yr[tid] = e_yr;
  }
  if (tid < BN) {
    s_ws[tid] = 1.0f;
    s_bs[tid] = e_bs;
  }
  __syncthreads();
  // a wavefront's f32 region [32 tokens][TN rows]: an activation stage for
  // 64- and 128-token tiles, a code stage for 32-token tiles
  static_assert(32 * TN * 4 <= (BM >= 64 ? BM * 128 : BN * 32), "epilogue region");
  uint8_t* regb;
  if constexpr (BM >= 64) regb = wave == 0 ? sA0 : wave == 1 ? sA1 : wave == 2 ? sA2 : sA3;
  else regb = wave == 0 ? sW0 : wave == 1 ? sW1 : wave == 2 ? sW2 : sW3;
  tile_epilogue<BN, TN, TM, NI, MJ, ACT>(p, acc, reinterpret_cast<float*>(regb), s_sx, s_rw, s_yr, s_ws, s_bs,
                                        n0, nlim, rows, wn, wm, lane);
}

template <int BM, bool ACT, int FMT>
void w4_launch_shape(const GemmParams& p, hipStream_t st) {
  const int nout = ACT ? p.N / 2 : p.N;
  const int n_tiles = cdiv(nout, ACT ? kW4BN / 2 : kW4BN);
  const unsigned ks = (unsigned)std::max(1, p.ksplit);
  if (p.group_offs) {
    const int m_tiles = cdiv(p.M, BM) + std::min(p.slots, p.M);
    hipLaunchKernelGGL((w4_gemm_kernel<BM, ACT, FMT>), dim3(n_tiles, m_tiles, ks), dim3(kThreads), 0, st, p,
                       m_tiles, n_tiles);
  } else {
    const int m_tiles = cdiv(p.M, BM);
    const int grid = cdiv(m_tiles * n_tiles, kXcds) * kXcds;
    hipLaunchKernelGGL((w4_gemm_kernel<BM, ACT, FMT>), dim3(grid, 1, ks), dim3(kThreads), 0, st, p, m_tiles,
                       n_tiles);
  }
}

template <int BM, int FMT>
void w4_launch_act(const GemmParams& p, hipStream_t st) {
  if (p.act != QA_NONE) w4_launch_shape<BM, true, FMT>(p, st);
  else w4_launch_shape<BM, false, FMT>(p, st);
}

template <int BM>
void w4_launch_fmt(const GemmParams& p, int fmt, hipStream_t st) {
  if (fmt == 1) w4_launch_act<BM, 1>(p, st);
  else if (fmt == 2) w4_launch_act<BM, 2>(p, st);
  else w4_launch_act<BM, 0>(p, st);
}

}  // namespace

// Whether the W4A16 tiled kernel takes the problem (K % 64, 16-byte aligned
// rows, even scale rows, codes < 4 GiB per group), and its plan: token-tile
// height (the largest of 128 / 64 / 32 that still fills the CUs, or that fits
// the average group), K split (dense problems with few tiles) and the f32
// workspace the split needs ([ksplit][M][N]). `fmt`: 0 MXFP4 (e8m0 per
// 32 k), 1 NVFP4 (bf16 per 16 k), 2 INT4 (bf16 per wq_group k).
bool qmoe_w4_plan(const GemmParams& p, int fmt, int* bm_out, int* ksplit_out, int64_t* ws_bytes) {
  if (p.M <= 0 || p.K <= 0 || (p.K % 64) != 0 || p.N <= 0) return false;
  if (p.act != QA_NONE && (p.N % 2) != 0) return false;
  if ((p.lda % 8) != 0 || (p.ldw % 16) != 0 || (fmt != 2 && (p.ldws % 2) != 0)) return false;
  if (fmt == 2 && ((p.wq_group != 32 && p.wq_group != 64 && p.wq_group != 128) || (p.K % p.wq_group) != 0))
    return false;
  // scale alignment mask: 4-byte bf16 pairs (NVFP4), 2-byte e8m0 pairs (MXFP4), bf16 (INT4)
  const int sal = fmt == 1 ? 3 : 1;
  if ((reinterpret_cast<uintptr_t>(p.a) & 15) || (reinterpret_cast<uintptr_t>(p.w) & 15) ||
      (p.w_gstride % 16) != 0 || (reinterpret_cast<uintptr_t>(p.w_scale) & sal) ||
      (fmt != 2 && (p.ws_gstride % 2) != 0))
    return false;
  if ((int64_t)p.ldw * p.N >= ((int64_t)1 << 32) || (int64_t)p.ldws * (fmt ? 2 : 1) * p.N >= ((int64_t)1 << 31))
    return false;
  const int nout = p.act != QA_NONE ? p.N / 2 : p.N;
  const int n_tiles = cdiv(nout, p.act != QA_NONE ? kW4BN / 2 : kW4BN);
  int bm = 32;
  const char* env = getenv("QMOE_W4_BM");  // tuning knob
  if (env && (atoi(env) == 128 || atoi(env) == 64 || atoi(env) == 32)) {
    bm = atoi(env);
  } else if (p.group_offs) {
    // measured on MI355X (GPT-OSS MoE, 128 experts): 64-token tiles up to
    // ~96 rows per routed expert (32-token tiles lose ~25% at 32 rows), 128
    // above
    const int avg = std::max(1, p.M / std::max(1, std::min(p.slots, p.M)));
    bm = avg > 96 ? 128 : 64;
  } else {
    // measured on MI355X (K 2880, N 5760): 128-token tiles once they fill the
    // CUs, else 64 with a K split (32-token tiles are slower at every M)
    bm = (int64_t)cdiv(p.M, 128) * n_tiles >= 200 ? 128 : 64;
  }
  const int m_tiles0 = p.group_offs ? cdiv(p.M, bm) + std::min(p.slots, p.M) : cdiv(p.M, bm);
  if (p.group_offs && m_tiles0 > 65535) return false;
  // dense problems with fewer than ~200 tiles split K (every slice keeps at
  // least 8 stages)
  int ksplit = 1;
  if (!p.group_offs) {
    const int tiles = m_tiles0 * n_tiles;
    if (tiles < 200) ksplit = std::min(cdiv(256, tiles), std::max(1, (p.K / 64) / 8));
  }
  // e2m1 (MXFP4 / NVFP4) dense problems too small for 200 128-token tiles:
  // measured on MI355X (K 2880, N 5760), 32-token tiles with a K split that
  // shrinks as the tokens grow (MXFP4 64 tokens: 15.5 vs 20.0 us; 256: 25.5
  // vs 32.2 us). INT4's costlier expansion keeps the larger tiles.
  if (!p.group_offs && fmt != 2 && !env && (int64_t)cdiv(p.M, 128) * n_tiles < 200 && p.M <= 512) {
    if (p.M <= 256) {
      bm = 32;
      ksplit = p.M <= 64 ? 4 : (p.M <= 128 ? 2 : 1);
    } else {
      bm = 64;
      ksplit = 1;
    }
    ksplit = std::max(1, std::min(ksplit, p.K / 64));
  }
  // INT4 from 129 to 512 tokens in the same regime: 128-token tiles split
  // 4 / 2 ways (measured on MI355X, K 2880, N 5760: 256 tokens 33.9 vs 38.2
  // us, 512 tokens 45.6 vs 48.1 us)
  if (!p.group_offs && fmt == 2 && !env && (int64_t)cdiv(p.M, 128) * n_tiles < 200 && p.M > 128 && p.M <= 512) {
    bm = 128;
    ksplit = std::max(1, std::min(p.M <= 256 ? 4 : 2, p.K / 64));
  }
  const char* ks_env = getenv("QMOE_W4_KSPLIT");  // tuning knob
  if (ks_env && atoi(ks_env) > 0) ksplit = std::max(1, std::min(atoi(ks_env), p.K / 64));
  *bm_out = bm;
  *ksplit_out = ksplit;
  *ws_bytes = ksplit > 1 ? (int64_t)ksplit * p.M * p.N * 4 : 0;
  return true;
}

// Launch per the plan (the caller sized the workspace); with a K split the
// finishing kernel runs the epilogue.
int qmoe_w4_launch(GemmParams p, int fmt, void* workspace, int64_t ws_bytes, hipStream_t st) {
  int bm = 0, ksplit = 1;
  int64_t need = 0;
  if (!qmoe_w4_plan(p, fmt, &bm, &ksplit, &need)) return QMOE_ERR_ARG;
  p.ksplit = ksplit;
  if (ksplit > 1) {
    if (!workspace || ws_bytes < need) return QMOE_ERR_WORKSPACE;
    p.partial = static_cast<float*>(workspace);
  }
  switch (bm) {
    case 128: w4_launch_fmt<128>(p, fmt, st); break;
    case 64: w4_launch_fmt<64>(p, fmt, st); break;
    default: w4_launch_fmt<32>(p, fmt, st); break;
  }
  if (ksplit > 1) {
    const int nout = p.act != QA_NONE ? p.N / 2 : p.N;
    const dim3 rg((unsigned)cdiv(nout, 512), (unsigned)cdiv(p.M, 4), 1);
    if (p.act != QA_NONE)
      hipLaunchKernelGGL((tile_splitk_finish_kernel<false, true, kScNone>), rg, dim3(kThreads), 0, st, p);
    else
      hipLaunchKernelGGL((tile_splitk_finish_kernel<false, false, kScNone>), rg, dim3(kThreads), 0, st, p);
  }
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
