// Tiled (prefill) GEMM for 1-byte activations x 1-byte weights (FP8 e4m3 and
// INT8 W8A8, per-token x per-channel scales), dense or grouped.
//
// Design for gfx950 (one workgroup of 4 wavefronts per CU):
//  * output tile BM tokens x BN weight rows; the wavefronts form a WN x WM
//    grid, each owning (BN/WN) x (BM/WM) outputs as 32 x 32 MFMA blocks.
//    The MFMA's first operand is the weight block (32 output channels) and
//    the second the activation block (32 tokens), so each lane ends with 4
//    consecutive output channels of one token per register quad;
//  * K advances in stages of 64 bytes (one MFMA k-step): FP8 runs
//    v_mfma_scale_f32_32x32x64_f8f6f4 (unit scales), INT8 two
//    v_mfma_i32_32x32x32_i8;
//  * global -> LDS copies are direct (global_load_lds_dwordx4: each lane moves
//    16 bytes, a wavefront instruction fills 1 KB = 16 LDS rows of 64 bytes)
//    into a ring of four LDS stages held in eight distinct LDS arrays, so the
//    compiler can tell the stage being read from the stages being filled and
//    does not wait on the copies; the 16-byte chunk c of row r is stored at
//    slot c ^ ((r >> 2) & 3), so the MFMA operand reads (lane l -> row
//    l & 31, 32 bytes) hit every bank once per 16 lanes;
//  * copies run four stages ahead of the MFMAs (three stages of latency
//    slack): per stage, wait for the own copy of the next stage, barrier,
//    refill the buffer just consumed, MFMAs of this stage with the next
//    stage's operand reads (into the second register set) scheduled among
//    the first MFMAs and the copies among the rest;
//  * epilogue: the f32 sums go through a per-wavefront LDS region (float4
//    quads, slot-swizzled) so that a compact loop can finish 8 contiguous
//    output channels per lane (scales, bias, fused activation, routing
//    weight) and store them as one 16-byte bf16 chunk.
// Tile order: dense problems use a 1-D grid remapped so that each XCD walks
// groups of 8 m-tiles column by column; grouped problems enumerate m-tiles of
// all groups on grid.y (wave-wide scan of the group sizes).

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "gemm_tile.h"
#include "stream_load.h"


namespace {

template <int BM, int BN>
struct F8Shape {
  static constexpr int WN = BM >= 128 ? 2 : 4;  // wavefronts along weight rows
  static constexpr int WM = 4 / WN;             // along tokens
  static constexpr int TN = BN / WN;            // weight rows per wavefront
  static constexpr int TM = BM / WM;            // tokens per wavefront
  static constexpr int NI = TN / 32;            // 32-row weight blocks per wavefront
  static constexpr int MJ = TM / 32;            // 32-token blocks per wavefront
  // LDS-copy instructions per wavefront per 64-byte stage (16 rows each). A
  // 32-token tile still has every wavefront copy 16 rows: the LDS array has
  // 64 rows and rows 32..63 (clamped duplicates) are never read, which keeps
  // the copy free of divergent branches.
  static constexpr int XI = BM >= 64 ? BM / 64 : 1;
  static constexpr int XR = XI * 64;  // rows of an activation LDS stage
  static constexpr int WI = BN / 64;
  static_assert(NI >= 1 && MJ >= 1 && XI >= 1 && WI >= 1, "tile too small");
};


__device__ __forceinline__ i32x8 lds_frag(const uint8_t* p0, const uint8_t* p1) {
  const uint4 a = *reinterpret_cast<const uint4*>(p0);
  const uint4 b = *reinterpret_cast<const uint4*>(p1);
  i32x8 r;
  r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
  r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
  return r;
}

__device__ __forceinline__ i32x4 lo4(const i32x8& v) { return i32x4{v[0], v[1], v[2], v[3]}; }

// `interleave` (gemm_tile.h) with NV vector-ALU instructions after every MFMA
// but the first, and NV after the last: the block-scaled tiles' scaling of
// the previous block pair runs while the next MFMA executes
template <int K, int NM, int NR, int NC, int NV>
__device__ __forceinline__ void interleave_v() {
  if constexpr (NV == 0) {
    interleave<K, NM, NR, NC>();
  } else if constexpr (K < NM) {
    constexpr int H = NM / 2 > 0 ? NM / 2 : 1;
    constexpr int r0 = K < H ? K * NR / H : NR, r1 = K < H ? (K + 1) * NR / H : NR;
    constexpr int c0 = K < H ? 0 : (K - H) * NC / (NM - H), c1 = K < H ? 0 : (K - H + 1) * NC / (NM - H);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    if constexpr (K > 0) __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);  // VALU
    if constexpr (r1 > r0) __builtin_amdgcn_sched_group_barrier(0x100, r1 - r0, 0);  // DS read
    if constexpr (c1 > c0) __builtin_amdgcn_sched_group_barrier(0x020, c1 - c0, 0);  // VMEM read
    interleave_v<K + 1, NM, NR, NC, NV>();
  } else {
    __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);  // VALU
  }
}
__device__ __forceinline__ i32x4 hi4(const i32x8& v) { return i32x4{v[4], v[5], v[6], v[7]}; }
// e2m1 MFMA operand: 4 registers (32 codes) in the low half of the 8-register
// operand; the undefined upper half lets the compiler pass a 4-register tuple
__device__ __forceinline__ i32x8 fp4_op(const i32x4& v) {
  return __builtin_shufflevector(v, v, 0, 1, 2, 3, -1, -1, -1, -1);
}

// E5: e5m2 operands (bit 0 the weights, bit 1 the activations; the others
// e4m3): the MFMA's operand format codes
template <bool INT, int BM, int BN, bool ACT, int KB, bool BLK, bool WPC = false, bool MX = false, int E5 = 0>
__global__ __launch_bounds__(kThreads) void f8_gemm_kernel(const GemmParams p, int m_tiles, int n_tiles) {
  static_assert(E5 == 0 || (!INT && !MX), "e5m2 operands: float codes only");
  constexpr int kFw = E5 & 1, kFx = (E5 >> 1) & 1;  // weight (A) / activation (B) format codes
  static_assert(KB == 64 || KB == 128, "K bytes per LDS stage");
  // MX (QK_W4A4_MX): e2m1 codes of both operands in the 128-byte stages (256
  // k), their e8m0 bytes ([row][8] per stage) copied beside them; the MFMA
  // applies both scales, so the epilogue's token and weight scales are 1
  // (the persistent kernel's mode 2 describes the operand layout)
  static_assert(!MX || (KB == 128 && !INT && !BLK && BM >= 128), "MX: 128-byte stages, tiles of >= 128 tokens");
  // BLK: block scales (W8A8_BLK): one 128-byte stage is one 128-column K step;
  // the token scale of step s is a_scale[row, s >> a_kshift]. Without WPC the
  // weight scale is that of the tile's 128-row block and K block s >> w_kshift;
  // WPC (per-channel weights, the grouped-matmul recipe) applies one scale per
  // weight row in the epilogue instead.
  static_assert(!BLK || (KB == 128 && (BN == 256 || (BN == 128 && BM <= 128))),
                "block scales: 128-byte stages, 256-row tiles or 128-row tiles of <= 128 tokens");
  static_assert(!WPC || BLK, "per-channel weight scales with block activation scales");
  using S = F8Shape<BM, BN>;
  constexpr int NI = S::NI, MJ = S::MJ, TN = S::TN, TM = S::TM;
  constexpr int BNO = ACT ? BN / 2 : BN;  // output channels per tile
  constexpr int TNO = ACT ? TN / 2 : TN;  // output channels per wavefront
  static_assert(!ACT || NI % 2 == 0, "fused activation pairs gate and up blocks");

  // LDS stages, each operand of each stage in its own array: four stages of
  // 64 K-bytes (KB = 64) or two of 128 (KB = 128; arrays 2 and 3 unused)
  // (KB = 128 with tiles of at most 128 tokens: three stages fit in LDS,
  // array 2 holds the third)
  constexpr bool TRI = KB == 128 && BM <= 128;
  constexpr int XRS = KB == 64 ? S::XR : BM;  // activation rows per stage array
  constexpr int B2 = KB == 64 ? 64 : (TRI ? 128 : 0);  // bytes per row of array 2
  constexpr int B3 = KB == 64 ? 64 : 0;                // and of array 3
  __shared__ __align__(1024) uint8_t sW0[BN * KB], sW1[BN * KB], sW2[B2 ? BN * B2 : 16], sW3[B3 ? BN * B3 : 16];
  __shared__ __align__(1024) uint8_t sX0[XRS * KB], sX1[XRS * KB], sX2[B2 ? XRS * B2 : 16], sX3[B3 ? XRS * B3 : 16];
  // MX scale bytes of stage buffers 0..2
  constexpr int QWB = MX ? BN * 8 : 16, QXB = MX ? BM * 8 : 16, QB2 = MX && TRI;
  __shared__ __align__(16) uint8_t sQW0[QWB], sQW1[QWB], sQW2[QB2 ? QWB : 16];
  __shared__ __align__(16) uint8_t sQX0[QXB], sQX1[QXB], sQX2[QB2 ? QXB : 16];
  __shared__ int s_info[4];
  __shared__ float s_sx[BM], s_rw[BM], s_ws[BN], s_bs[BN];
  // BLK: per-stage scales, one 64-float slot per wavefront: [0, BM) token
  // scales of the stage's K block, [BM, BM + 2) the scales of the tile's two
  // 128-row weight blocks (LDS rows 0..127 and 128..255), the rest unused
  __shared__ __align__(16) float sS0[BLK ? 256 : 1], sS1[BLK ? 256 : 1], sS2[BLK && TRI ? 256 : 1];
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

  // ---- epilogue inputs, loaded now (their latency hides under the first
  // copies) and kept in registers until the epilogue stages them in LDS:
  // thread t < BM holds token t's activation scale, routing weight and
  // output row; thread t < BN holds weight row t's scale and bias.
  float e_sx = 0.0f, e_rw = 1.0f, e_ws = 0.0f, e_bs = 0.0f;
  int e_yr = 0;
  if (tid < BM) {
    const int R = row0 + min(tid, rows - 1);
    const int ar = p.a_rows ? p.a_rows[R] : R;
    e_sx = BLK || MX ? 1.0f : p.a_scale[(int64_t)ar * p.lds_a];
    if (p.row_weight) e_rw = bf16_to_f32(p.row_weight[R]);
    e_yr = p.y_rows ? p.y_rows[R] : R;
  }
  if (tid < BN) {
    int n;
    if (ACT) {
      const int cidx = min(n0 + (tid % (BN / 2)), nlim - 1);
      n = (tid < BN / 2 ? 0 : p.N / 2) + cidx;
    } else {
      n = min(n0 + tid, nlim - 1);
    }
    e_ws = (BLK && !WPC) || MX ? 1.0f : static_cast<const float*>(p.w_scale)[(int64_t)g * p.ws_gstride + n];
    if (p.bias) e_bs = p.bias[(int64_t)g * p.bias_gstride + n];
  }

  // ---- LDS copies: one wavefront instruction moves 1 KB: 16 rows x 64
  // bytes (KB = 64: lane -> row lane >> 2, chunk lane & 3) or 8 rows x 128
  // bytes (KB = 128: lane -> row lane >> 3, chunk lane & 7, whole 128-byte
  // lines, which halves the L1 -> L2 requests per byte). A lane fetches the
  // chunk that the row's swizzle stores in its slot. Activation rows are kept
  // as 32-bit indices (a gathered row may lie anywhere, so the 64-bit address
  // is formed at the copy), weight rows as 32-bit offsets.
  constexpr int RPI = KB == 64 ? 16 : 8;                       // rows per copy instruction
  constexpr int WI = BN / (4 * RPI);                           // weight copies per wavefront
  constexpr int XI = KB == 64 ? S::XI : BM / (4 * RPI);        // activation copies per wavefront
  static_assert(XI >= 1 && WI >= 1, "copy geometry");
  const uint8_t* xbase = static_cast<const uint8_t*>(p.a);
  const uint8_t* wbase = p.w + (int64_t)g * p.w_gstride;
  auto chunk_of = [&](int r) {  // byte offset of the chunk lane fetches for LDS row r
    if (KB == 64) return ((lane & 3) ^ ((r >> 2) & 3)) * 16;
    return ((lane & 7) ^ ((r & 7) ^ ((r >> 3) & 1))) * 16;
  };
  uint32_t xrow[XI], woff[WI];
  int xcx[XI];
#pragma unroll
  for (int j = 0; j < XI; ++j) {
    const int r = (wave + 4 * j) * RPI + (KB == 64 ? lane >> 2 : lane >> 3);
    const int R = row0 + min(r, rows - 1);
    xrow[j] = (uint32_t)(p.a_rows ? p.a_rows[R] : R);
    xcx[j] = chunk_of(r);
  }
#pragma unroll
  for (int j = 0; j < WI; ++j) {
    const int r = (wave + 4 * j) * RPI + (KB == 64 ? lane >> 2 : lane >> 3);
    int n;
    if (ACT) {
      const int cidx = min(n0 + (r % (BN / 2)), nlim - 1);
      n = (r < BN / 2 ? 0 : p.N / 2) + cidx;
    } else {
      n = min(n0 + r, nlim - 1);
    }
    woff[j] = (uint32_t)n * (uint32_t)p.ldw + chunk_of(r);
  }
  // MX scale copies: 32 rows x 8 bytes per instruction, lane -> row lane & 31,
  // dword lane >> 5, so that the instruction's 256 LDS bytes are [dword][row]
  // and the reads (32 consecutive rows, one dword) hit 32 consecutive banks;
  // QW weight and QX activation instructions per wavefront
  constexpr int QW = MX ? BN / 128 : 0, QX = MX ? BM / 128 : 0;
  const uint8_t* wqbase = static_cast<const uint8_t*>(p.w_scale) + (int64_t)g * p.ws_gstride;
  const uint8_t* xqbase = reinterpret_cast<const uint8_t*>(p.a_scale);
  uint32_t qwoff[QW ? QW : 1], qxrow[QX ? QX : 1];
  if constexpr (MX) {
#pragma unroll
    for (int j = 0; j < QW; ++j) {
      const int r = (wave * QW + j) * 32 + (lane & 31);
      int n;
      if (ACT) {
        const int cidx = min(n0 + (r % (BN / 2)), nlim - 1);
        n = (r < BN / 2 ? 0 : p.N / 2) + cidx;
      } else {
        n = min(n0 + r, nlim - 1);
      }
      qwoff[j] = (uint32_t)n * (uint32_t)p.ldws + (uint32_t)(lane >> 5) * 4u;
    }
#pragma unroll
    for (int j = 0; j < QX; ++j) {
      const int r = (wave * QX + j) * 32 + (lane & 31);
      const int R = row0 + min(r, rows - 1);
      qxrow[j] = (uint32_t)(p.a_rows ? p.a_rows[R] : R);
    }
  }
  // BLK: this lane's source for the per-stage scale copy (4 bytes; the K
  // block index is added per stage): LDS slot wave*64 + lane holds token
  // scale `slot` for slot < BM, the scale of LDS weight rows
  // [(slot-BM)*128, +128) for slot < BM + 2, a duplicate elsewhere
  const float* sc_src = p.a_scale;
  int sc_shift = 0;  // K-block shift of this lane's scale stream
  if constexpr (BLK) {
    const int slot = wave * 64 + lane;
    sc_shift = p.a_kshift;
    if (!WPC && slot >= BM && slot < BM + 2) {
      sc_shift = p.w_kshift;
      const int b = slot - BM;
      const int n = ACT ? (b == 0 ? 0 : p.N / 2) + min(n0, nlim - 1) : min(n0 + b * 128, nlim - 1);
      sc_src = static_cast<const float*>(p.w_scale) + (int64_t)g * p.ws_gstride + (int64_t)(n / 128) * p.ldws;
    } else {
      const int R = row0 + min(slot < BM ? slot : 0, rows - 1);
      const int ar = p.a_rows ? p.a_rows[R] : R;
      sc_src = p.a_scale + (int64_t)ar * p.lds_a;
    }
  }
  // The row terms pass through an empty asm so that the compiler forms the
  // 64-bit addresses at each copy instead of keeping them alive across the
  // MFMA loop.
  // split-K: this workgroup's K range, in units of 256 bytes (two 128-byte
  // or four 64-byte stages, so every pipeline below runs whole loops)
  const int NU = (MX ? p.K / 2 : p.K) / 256;
  const int u0 = (int)((int64_t)NU * blockIdx.z / p.ksplit);
  const int u1 = (int)((int64_t)NU * (blockIdx.z + 1) / p.ksplit);
  const uint32_t kbase = (uint32_t)u0 * 256u;
  auto copy_stage = [&](uint8_t* dW, uint8_t* dX, float* dS, uint8_t* dQW, uint8_t* dQX, int ks) {
    const uint32_t kb = kbase + (uint32_t)ks * (uint32_t)KB;
    if constexpr (BLK)
      __builtin_amdgcn_global_load_lds(sc_src + ((kb / 128) >> sc_shift), QMOE_LDS(dS + wave * 64), 4, 0, 0);
    if constexpr (MX) {
      const uint32_t kq = kb / 16;  // one scale byte per 16 code bytes
#pragma unroll
      for (int j = 0; j < QW; ++j) {
        uint32_t o = qwoff[j];
        asm volatile("" : "+v"(o));
        __builtin_amdgcn_global_load_lds(wqbase + (o + kq), QMOE_LDS(dQW + (wave * QW + j) * 256), 4, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < QX; ++j) {
        uint32_t r = qxrow[j];
        asm volatile("" : "+v"(r));
        const uint8_t* src = xqbase + (uint64_t)r * (uint64_t)p.lds_a + (kq + (uint32_t)(lane >> 5) * 4u);
        __builtin_amdgcn_global_load_lds(src, QMOE_LDS(dQX + (wave * QX + j) * 256), 4, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < WI; ++j) {
      uint32_t o = woff[j];
      asm volatile("" : "+v"(o));
      __builtin_amdgcn_global_load_lds(wbase + (o + kb), QMOE_LDS(dW + (wave + 4 * j) * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < XI; ++j) {
      uint32_t r = xrow[j];
      asm volatile("" : "+v"(r));
      const uint8_t* src = xbase + (uint64_t)r * (uint64_t)p.lda + (kb + xcx[j]);
      __builtin_amdgcn_global_load_lds(src, QMOE_LDS(dX + (wave + 4 * j) * 1024), 16, 0, 0);
    }
  };

  // ---- operand reads: lane -> row (l & 31), 32 bytes at k-step t ----
  // (chunks 2 kh, 2 kh + 1 of the k-step's 64 bytes; the block rows start at
  // multiples of 32, so the swizzle depends on l & 31 only)
  const int rl = lane & 31, kh = lane >> 5;
  int po[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (KB == 64) po[t][h] = rl * 64 + (((2 * kh + h) ^ ((rl >> 2) & 3)) * 16);
      else  // MX: 16 bytes of 64-k step h of the half (chunk 4t + 2h + kh)
        po[t][h] = rl * 128 + (((MX ? 4 * t + 2 * h + kh : 4 * t + 2 * kh + h) ^ ((rl & 7) ^ ((rl >> 3) & 1))) * 16);
    }
  auto wrow = [&](int i) {  // LDS row of this wavefront's weight block i
    if (ACT) return (i < NI / 2 ? 0 : BN / 2) + wn * (TN / 2) + (i % (NI / 2)) * 32;
    return wn * TN + i * 32;
  };
  i32x8 wf[2][NI], xf[2][MJ];
  // MX: scale dword of half t (32-k blocks 4t + 2h + kh), shifted so that
  // byte 2h is the lane's block of step h
  uint32_t wsc[2][MX ? NI : 1], xsc[2][MX ? MJ : 1];
  // BLK: the scaled block sums accumulate in f32 for INT8 codes too
  using Acc = typename std::conditional<INT && !BLK, i32x16, f32x16>::type;
  Acc acc[NI][MJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // BLK: the stage's block sums go to tmp, then acc += tmp * (sx * sw)
  // (INT8 codes: an exact int32 block sum, |sum| < 2^21, converted to f32)
  using Tmp = typename std::conditional<INT, i32x16, f32x16>::type;
  Tmp tmp[BLK ? NI : 1][BLK ? MJ : 1];
  float scl[BLK ? NI : 1][BLK ? MJ : 1];
  // The K pipeline over the wavefront's first MJE 32-token blocks (MJ: all
  // of them); the accumulators of the others keep their zeros.
  auto pipeline = [&](auto mje_c) {
    constexpr int MJE = decltype(mje_c)::value;
    // operands of k-step `ks` of the stage in (sW, sX) into register set t
    auto read_frags = [&](const uint8_t* sW, const uint8_t* sX, const uint8_t* sQW, const uint8_t* sQX, int ks,
                          int t) {
      if constexpr (MX) {
        // block of 32 rows at 8 (first row) bytes, dword plane ks, row rl
#pragma unroll
        for (int i = 0; i < NI; ++i)
          wsc[t][i] = *reinterpret_cast<const uint32_t*>(sQW + wrow(i) * 8 + ks * 128 + rl * 4) >> (8 * kh);
#pragma unroll
        for (int j = 0; j < MJE; ++j)
          xsc[t][j] =
              *reinterpret_cast<const uint32_t*>(sQX + (wm * TM + j * 32) * 8 + ks * 128 + rl * 4) >> (8 * kh);
      }
      const int h0 = KB == 64 ? po[0][0] : po[ks][0], h1 = KB == 64 ? po[0][1] : po[ks][1];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const uint8_t* b = sW + wrow(i) * KB;
        wf[t][i] = lds_frag(b + h0, b + h1);
      }
#pragma unroll
      for (int j = 0; j < MJE; ++j) {
        const uint8_t* b = sX + (wm * TM + j * 32) * KB;
        xf[t][j] = lds_frag(b + h0, b + h1);
      }
    };

    auto read_scales = [&](const float* sS) {
      if constexpr (BLK) {
        float sx[MJE];
#pragma unroll
        for (int j = 0; j < MJE; ++j) sx[j] = sS[wm * TM + j * 32 + rl];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          // the tile's 128-row weight blocks: LDS rows 0..127 and 128..255 of a
          // 256-row tile; with an activation the gate and the up half
          const int wb = ACT ? (wrow(i) >= BN / 2 ? 1 : 0) : wrow(i) / 128;
          const float sw = WPC ? 1.0f : sS[BM + wb];
#pragma unroll
          for (int j = 0; j < MJE; ++j) scl[i][j] = sx[j] * sw;
        }
      }
    };
    auto mma = [&](int t) {
      if constexpr (MX) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < MJE; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fp4_op(lo4(wf[t][i])), fp4_op(lo4(xf[t][j])),
                                                                        acc[i][j], 4, 4, 0, (int)wsc[t][i], 0,
                                                                        (int)xsc[t][j]);
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < MJE; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fp4_op(hi4(wf[t][i])), fp4_op(hi4(xf[t][j])),
                                                                        acc[i][j], 4, 4, 2, (int)wsc[t][i], 2,
                                                                        (int)xsc[t][j]);
        return;
      }
      if constexpr (INT && !BLK) {
        // the two 32-k halves of the k-step go to every accumulator in turn:
        // the second MFMA of an accumulator comes NI * MJE MFMAs after its first,
        // so no MFMA waits on the result of the one before it
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < MJE; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(h ? hi4(wf[t][i]) : lo4(wf[t][i]),
                                                                h ? hi4(xf[t][j]) : lo4(xf[t][j]), acc[i][j], 0, 0,
                                                                0);
        return;
      }
      if constexpr (BLK) {
        if (t == 1) {
          // the stage's last k-step: block pair p's MFMA, then the scaling
          // acc += tmp * (sx * sw) of pair p - 1, whose MFMA has completed by
          // then, so the FMAs run on the vector ALU while the matrix core runs
          // the next MFMA (each accumulator still sees the same operations in
          // the same order). INT8: every pair's first 32-k half first, then
          // the second halves with the scaling behind them.
          if constexpr (INT) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
              for (int j = 0; j < MJE; ++j)
                tmp[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(lo4(wf[1][i]), lo4(xf[1][j]), tmp[i][j], 0, 0, 0);
          }
#pragma unroll
          for (int q = 0; q <= NI * MJE; ++q) {
            if (q < NI * MJE) {
              const int i = q / MJE, j = q % MJE;
              if constexpr (INT)
                tmp[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(hi4(wf[1][i]), hi4(xf[1][j]), tmp[i][j], 0, 0, 0);
              else
                tmp[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[1][i], xf[1][j], tmp[i][j], kFw, kFx,
                                                                            0, 127, 0, 127);
            }
            if (q > 0) {
              const int i = (q - 1) / MJE, j = (q - 1) % MJE;
#pragma unroll
              for (int r = 0; r < 16; ++r) acc[i][j][r] += (float)tmp[i][j][r] * scl[i][j];
            }
          }
          return;
        }
        if constexpr (INT) {
          // the stage's first k-step: fresh block sums, halves as above
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
              for (int j = 0; j < MJE; ++j)
                tmp[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(h ? hi4(wf[0][i]) : lo4(wf[0][i]),
                                                                  h ? hi4(xf[0][j]) : lo4(xf[0][j]),
                                                                  h ? tmp[i][j] : i32x16{}, 0, 0, 0);
          return;
        }
      }
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < MJE; ++j) {
          if constexpr (BLK) {
            tmp[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[t][i], xf[t][j], f32x16{}, kFw, kFx, 0,
                                                                        127, 0, 127);
          } else {
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[t][i], xf[t][j], acc[i][j], kFw, kFx, 0,
                                                                        127, 0, 127);
          }
        }
    };


    constexpr int CPS = WI + XI + (BLK ? 1 : 0) + QW + QX;  // copy instructions per wavefront per stage
    constexpr int NM = NI * MJE * (INT || MX ? 2 : 1);       // MFMAs per k-step
    constexpr int NR = (MX ? 3 : 2) * (NI + MJE);            // LDS operand reads per k-step
    if constexpr (KB == 64) {
      // ---- four stages of one k-step (KS % 4 == 0) ----
      // Stage s lives in LDS buffer s % 4 and is copied four stages ahead.
      // Stage s: wait for the own copy of stage s+1 -> barrier (every copy of
      // stage s+1 has landed, and every wavefront holds the operands of stage
      // s in registers, so buffer s % 4 is free) -> copy stage s+4 into it ->
      // MFMAs of stage s, with the operand reads of stage s+1 issued among the
      // first MFMAs (so they have landed by the next barrier) and the copies
      // among the rest. The copy is unconditional (past the end it refetches
      // the last stage into a consumed buffer, which is never read again), so
      // the loop body has no branch.
      const int KS = (u1 - u0) * 4;
      copy_stage(sW0, sX0, sS0, sQW0, sQX0, 0);
      copy_stage(sW1, sX1, sS0, sQW0, sQX0, 1);
      copy_stage(sW2, sX2, sS0, sQW0, sQX0, 2);
      copy_stage(sW3, sX3, sS0, sQW0, sQX0, 3);
      wait_copies_upto<3 * CPS>();
      __syncthreads();
      read_frags(sW0, sX0, sQW0, sQX0, 0, 0);
      auto stage = [&](uint8_t* fW, uint8_t* fX, uint8_t* nW, uint8_t* nX, int s, int t) {
        wait_copies_upto<2 * CPS>();  // copies issued after stage s+1's: s+2, s+3
        stage_barrier();
        // the operand reads of stage s+1 come before the copies in program
        // order: the compiler treats an LDS copy as a write that may alias any
        // LDS read after it, so reads placed after the copies could not be
        // interleaved with this stage's MFMAs
        read_frags(nW, nX, sQW0, sQX0, 0, t ^ 1);
        copy_stage(fW, fX, sS0, sQW0, sQX0, min(s + 4, KS - 1));
        mma(t);
        interleave<0, NM, NR, CPS>();
      };
      for (int s = 0; s < KS; s += 4) {
        stage(sW0, sX0, sW1, sX1, s, 0);
        stage(sW1, sX1, sW2, sX2, s + 1, 1);
        stage(sW2, sX2, sW3, sX3, s + 2, 0);
        stage(sW3, sX3, sW0, sX0, s + 3, 1);
      }
    } else {
      // ---- two stages of two k-steps (KS % 2 == 0) ----
      // Stage s lives in LDS buffer s % 2. Its first half runs the MFMAs of
      // k-step 0 while k-step 1 is read; then: wait for the own copy of stage
      // s+1 -> barrier (stage s+1 has landed everywhere, and stage s has been
      // read everywhere, so its buffer is free) -> copy stage s+2 into it ->
      // MFMAs of k-step 1 while k-step 0 of stage s+1 is read. A copy has one
      // stage (two k-steps of MFMAs) to land.
      // BLK: the stage's scales are read with its second k-step (before the
      // barrier that frees its buffer) and applied after the k-step's MFMAs.
      // With three buffers (TRI) the buffer freed at stage s's barrier takes
      // stage s+3, so a copy has two stages to land.
      const int KS = (u1 - u0) * 2;
      constexpr int AHEAD = TRI ? 3 : 2;
      auto stage = [&](uint8_t* cW, uint8_t* cX, float* cS, uint8_t* cQW, uint8_t* cQX, uint8_t* nW, uint8_t* nX,
                       uint8_t* nQW, uint8_t* nQX, int s) {
        mma(0);
        read_frags(cW, cX, cQW, cQX, 1, 1);
        read_scales(cS);
        interleave<0, NM, NR + (BLK ? MJE + NI : 0), 0>();
        // every MFMA of k-step 0 is issued before the wait (the wait has no
        // data dependence on them, so the scheduler would otherwise hoist it
        // above half of them and cut the copies' latency slack)
        __builtin_amdgcn_sched_barrier(0);
        wait_copies_upto<(AHEAD - 2) * CPS>();  // stage s+1 has landed
        stage_barrier();
        // k-step 0 of stage s+1 is read before the copies are issued (an LDS
        // copy may alias any later LDS read for the compiler, which would keep
        // the reads behind every copy and expose their latency)
        read_frags(nW, nX, nQW, nQX, 0, 0);
        copy_stage(cW, cX, cS, cQW, cQX, min(s + AHEAD, KS - 1));
        mma(1);
        // BLK: each MFMA followed by the previous block pair's 16 scaling FMAs
        interleave_v<0, NM, NR, CPS, BLK ? 16 : 0>();
      };
      copy_stage(sW0, sX0, sS0, sQW0, sQX0, 0);
      copy_stage(sW1, sX1, sS1, sQW1, sQX1, 1);
      if constexpr (TRI) copy_stage(sW2, sX2, sS2, sQW2, sQX2, min(2, KS - 1));
      wait_copies_upto<(AHEAD - 1) * CPS>();
      __syncthreads();
      read_frags(sW0, sX0, sQW0, sQX0, 0, 0);
      if constexpr (TRI) {
        int s = 0;
        for (; s + 3 <= KS; s += 3) {
          stage(sW0, sX0, sS0, sQW0, sQX0, sW1, sX1, sQW1, sQX1, s);
          stage(sW1, sX1, sS1, sQW1, sQX1, sW2, sX2, sQW2, sQX2, s + 1);
          stage(sW2, sX2, sS2, sQW2, sQX2, sW0, sX0, sQW0, sQX0, s + 2);
        }
        if (s < KS) stage(sW0, sX0, sS0, sQW0, sQX0, sW1, sX1, sQW1, sQX1, s);
        if (s + 1 < KS) stage(sW1, sX1, sS1, sQW1, sQX1, sW2, sX2, sQW2, sQX2, s + 1);
      } else {
        for (int s = 0; s < KS; s += 2) {
          stage(sW0, sX0, sS0, sQW0, sQX0, sW1, sX1, sQW1, sQX1, s);
          stage(sW1, sX1, sS1, sQW1, sQX1, sW0, sX0, sQW0, sQX0, s + 1);
        }
      }
    }

  };
  // A block-scaled tile whose wavefront holds at most 32 of its tokens (the
  // last tile of a routed expert, a ragged last token tile) runs the MFMAs
  // and block scaling of its first 32-token block only: the other block's
  // sums belong to no token. Every wavefront still makes the same copies
  // and reaches the same barriers.
  if constexpr (BLK && MJ == 2) {
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    if (rows - (wave_u / S::WN) * TM <= 32) pipeline(std::integral_constant<int, 1>{});
    else pipeline(std::integral_constant<int, MJ>{});
  } else {
    pipeline(std::integral_constant<int, MJ>{});
  }
  if (p.ksplit > 1) {
    tile_store_partials<BN, TN, TM, NI, MJ, ACT, INT && !BLK>(p, acc, row0, rows, n0, nlim, wn, wm, lane);
    return;
  }
  wait_copies_upto<0>();
  if (tid < BM) {
    s_sx[tid] = e_sx;
    s_rw[tid] = e_rw;
    s_yr[tid] = e_yr;
  }
  if (tid < BN) {
    s_ws[tid] = e_ws;
    s_bs[tid] = e_bs;
  }
  __syncthreads();
  float* reg;
  if constexpr (KB == 64) reg = reinterpret_cast<float*>(wave == 0 ? sW0 : wave == 1 ? sW1 : wave == 2 ? sW2 : sW3);
  else reg = reinterpret_cast<float*>((wave < 2 ? sW0 : sW1) + (wave & 1) * (BN * 64));
  static_assert(32 * TN * 4 <= BN * 64, "a wavefront region fits a quarter of the weight stages");
  tile_epilogue<BN, TN, TM, NI, MJ, ACT>(p, acc, reg, s_sx, s_rw, s_yr, s_ws, s_bs, n0, nlim, rows, wn, wm, lane);

}

// Persistent dense form of the 1-byte tiles (256 x 256 and the shapes below;
// 128-byte K stages in two LDS buffers, per-token x per-channel scales, no K
// split, bias or row maps).
// Measured on MI355X: the one-tile-per-workgroup kernel spends ~14 us per
// tile outside its K loop (launch, the first stages' copy latency, the
// LDS-staged epilogue), which on the up projection of Llama-3-8B (896 tiles
// of 32 stages) is a fifth of the time. Here each workgroup walks tiles b,
// b + G, b + 2G, ... (G the grid, a multiple of the 8 XCDs, so a workgroup
// stays on its XCD's tile range) and the stage pipeline runs on across
// tiles: the copies of the next tile's first two stages are issued during
// the current tile's last two stages, so they are in flight while this
// tile's epilogue runs. The epilogue therefore cannot stage through the
// stage buffers: it stores from registers, with the tile's token and
// channel scales in small double-buffered LDS arrays of their own.
//
// MODE 0: FP8 e4m3 codes; 1: INT8 codes; 2: MX (QK_W4A4_MX): e2m1 codes of
// both operands with their e8m0 bytes. An MX stage is the same 128 bytes per
// row (256 k values, 8 scale bytes); its MFMAs are
// v_mfma_scale_f32_32x32x64_f8f6f4 with e2m1 operands (16 bytes per lane:
// row l & 31, k values 32 (l >> 5) .. + 31 of the 64-k step) and the scale
// bytes of the lane's row and 32-k block selected by opsel from a dword, so
// the sums come out scaled and the epilogue adds only the bias. The stage's
// scale bytes ([256 rows][8 bytes] per operand) ride in the stage's copies
// (dword LDS copies) into LDS arrays beside the code buffers.
//
// BN (weight rows per tile) is 256, or 224 for 1-byte codes: the wavefronts
// then form a 1 x 4 grid of 224 weight rows x 64 tokens each (7 x 2 blocks).
// Measured on MI355X (FP8, 4096 tokens): a 256-wide tile's MFMA loop alone
// (no copies, no operand reads, no barriers) runs at ~3.6 PFLOP/s, so the
// tile count per round matters as much as the loop: N = 14336 makes 896
// tiles of 256 x 256 -- 4 rounds on 224 of the 256 CUs -- but 1024 tiles of
// 256 x 224, 4 rounds on all 256.
//
// BM (tokens per tile) is 256, or 128 for 1-byte codes (mid-size problems
// whose 128 x 256 tiles leave CUs idle: 512 tokens of Llama-3-8B's up
// projection make 224 such tiles, but 256 of 128 x 224).
template <int MODE, int BN = 256, int BM = 256>
__global__ __launch_bounds__(kThreads) void f8_persistent_kernel(const GemmParams p, int m_tiles, int n_tiles,
                                                                 int tile_slots, int wide) {
  constexpr bool INT = MODE == 1, MX = MODE == 2;
  constexpr bool ACT = false;  // fused activations take the one-tile kernel
  constexpr int KB = 128;
  static_assert(BN == 256 || (BN == 224 && !MX), "weight tile height");
  static_assert(BM == 256 || (BM == 128 && !MX), "token tile height");
  constexpr int WN = BN == 256 ? 2 : 1, WM = 4 / WN;  // wavefront grid (weight rows x tokens)
  constexpr int TN = BN / WN, TM = BM / WM, NI = TN / 32, MJ = TM / 32;
  __shared__ __align__(1024) uint8_t sW0[BN * KB], sW1[BN * KB];
  __shared__ __align__(1024) uint8_t sX0[BM * KB], sX1[BM * KB];
  // MX scale bytes of the two stage buffers ([row][8], 32 k per byte)
  constexpr int QB = MX ? BN * 8 : 16;
  __shared__ __align__(16) uint8_t sQW0[QB], sQW1[QB], sQX0[QB], sQX1[QB];
  // per-tile epilogue vectors, double-buffered by tile parity: written after
  // the tile's first stage, read by its epilogue while the next tile's are
  // written to the other set (MX: s_ws holds the bias, s_sx is unused)
  __shared__ __align__(16) float s_sx[2][BM], s_ws[2][BN];

  const int tid = threadIdx.x;
  // the wavefront index in an SGPR: the LDS destinations of the copies are
  // then scalar (M0) values instead of VGPRs held across the K loop
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % WN, wm = wave / WN;
  const int nlim = ACT ? p.N / 2 : p.N;
  constexpr int BNO = ACT ? BN / 2 : BN;
  constexpr int RPI = 8;                   // rows per copy instruction (128-byte rows)
  constexpr int WI = BN / (4 * RPI);       // weight copies per wavefront per stage
  constexpr int XI = BM / (4 * RPI);       // activation copies per wavefront per stage
  constexpr int QI = MX ? BN / (4 * 32) : 0;  // MX scale copies per operand (32 rows of 8 bytes each)
  constexpr int CPS = WI + XI + 2 * QI;
  // stages per tile (the host keeps the row bytes a multiple of 256, >= 512)
  const int KS = (MX ? p.K / 2 : p.K) / KB;
  const uint8_t* xbase = static_cast<const uint8_t*>(p.a);
  const uint8_t* wbase = p.w;
  const uint8_t* xqbase = reinterpret_cast<const uint8_t*>(p.a_scale);
  const uint8_t* wqbase = static_cast<const uint8_t*>(p.w_scale);

  // A tile's copies: this lane moves row r_j = rbase + 32 j of the weight
  // and activation stages (j < 8), 16-byte chunk `chunk` of the row's 128
  // bytes (the chunk its slot holds under the row swizzle, the same for
  // every j); the row offsets are formed at each copy from the tile's
  // (uniform) origin, so no per-tile offsets stay live across the K loop.
  struct Src {
    int row0, rows, n0;
  };
  const int rbase = wave * RPI + (lane >> 3);
  const int chunk = ((lane & 7) ^ (lane >> 3) ^ (wave & 1)) * 16;
  auto make_src = [&](int row0, int rows, int n0, Src& sc) {
    sc.row0 = row0;
    sc.rows = rows;
    sc.n0 = n0;
  };
  auto copy_stage = [&](uint8_t* dW, uint8_t* dX, uint8_t* dQW, uint8_t* dQX, const Src& sc, int ks) {
    const uint32_t kb = (uint32_t)ks * (uint32_t)KB;
#pragma unroll
    for (int j = 0; j < WI; ++j) {
      const int n = min(sc.n0 + rbase + 32 * j, nlim - 1);
      uint32_t o = (uint32_t)n * (uint32_t)p.ldw + (uint32_t)chunk;
      asm volatile("" : "+v"(o));
      __builtin_amdgcn_global_load_lds(wbase + (o + kb), QMOE_LDS(dW + (wave + 4 * j) * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < XI; ++j) {
      uint32_t r = (uint32_t)(sc.row0 + min(rbase + 32 * j, sc.rows - 1));
      asm volatile("" : "+v"(r));
      const uint8_t* src = xbase + (uint64_t)r * (uint64_t)p.lda + (kb + (uint32_t)chunk);
      __builtin_amdgcn_global_load_lds(src, QMOE_LDS(dX + (wave + 4 * j) * 1024), 16, 0, 0);
    }
    if constexpr (MX) {
      // copy q moves scale rows 32q .. 32q + 31 of the stage (lane -> row
      // lane & 31, dword lane >> 5 of the row's 8 bytes) into 256 LDS bytes
      // laid out [dword][row]: the reads (32 consecutive rows, one dword)
      // then hit 32 consecutive banks
      const uint32_t kq = (uint32_t)ks * 8u + (uint32_t)(lane >> 5) * 4u;
#pragma unroll
      for (int j = 0; j < QI; ++j) {
        const int rr = (wave * QI + j) * 32 + (lane & 31);
        const int n = min(sc.n0 + rr, nlim - 1);
        uint32_t o = (uint32_t)n * (uint32_t)p.ldws + kq;
        asm volatile("" : "+v"(o));
        __builtin_amdgcn_global_load_lds(wqbase + o, QMOE_LDS(dQW + (wave * QI + j) * 256), 4, 0, 0);
        uint32_t r = (uint32_t)(sc.row0 + min(rr, sc.rows - 1));
        asm volatile("" : "+v"(r));
        const uint8_t* src = xqbase + (uint64_t)r * (uint64_t)p.lds_a + kq;
        __builtin_amdgcn_global_load_lds(src, QMOE_LDS(dQX + (wave * QI + j) * 256), 4, 0, 0);
      }
    }
  };

  // operand reads: lane -> row (l & 31), 32 bytes of half t of the stage:
  // 1-byte codes: bytes 32 (l >> 5) .. + 31 of the 64-byte k-step t (chunks
  // 4t + 2 kh + h); MX: the 16 bytes of 64-k step h of the half (chunks
  // 4t + 2h + kh), one MFMA each
  const int rl = lane & 31, kh = lane >> 5;
  int po[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      po[t][h] = rl * 128 + (((MX ? 4 * t + 2 * h + kh : 4 * t + 2 * kh + h) ^ ((rl & 7) ^ ((rl >> 3) & 1))) * 16);
  auto wrow = [&](int i) { return tile_wrow<BN, TN, NI, ACT>(wn, i); };
  i32x8 wf[2][NI], xf[2][MJ];
  // MX: scale dword of half t (bytes 4t .. 4t + 3 of the row: 32-k blocks
  // 4t + 2h + kh), shifted so that byte 2h is the lane's block of step h
  uint32_t wsc[2][MX ? NI : 1], xsc[2][MX ? MJ : 1];
  auto read_frags = [&](const uint8_t* sW, const uint8_t* sX, const uint8_t* sQW, const uint8_t* sQX, int ks,
                        int t) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const uint8_t* b = sW + wrow(i) * KB;
      wf[t][i] = lds_frag(b + po[ks][0], b + po[ks][1]);
    }
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
      const uint8_t* b = sX + (wm * TM + j * 32) * KB;
      xf[t][j] = lds_frag(b + po[ks][0], b + po[ks][1]);
    }
    if constexpr (MX) {
      // block of 32 rows at 8 (first row) bytes, dword plane ks, row rl
#pragma unroll
      for (int i = 0; i < NI; ++i)
        wsc[t][i] = *reinterpret_cast<const uint32_t*>(sQW + wrow(i) * 8 + ks * 128 + rl * 4) >> (8 * kh);
#pragma unroll
      for (int j = 0; j < MJ; ++j)
        xsc[t][j] =
            *reinterpret_cast<const uint32_t*>(sQX + (wm * TM + j * 32) * 8 + ks * 128 + rl * 4) >> (8 * kh);
    }
  };
  using Acc = typename std::conditional<INT, i32x16, f32x16>::type;
  Acc acc[NI][MJ];
  auto mma = [&](int t) {
    if constexpr (MX) {
      // opsel 0 / 2 picks byte 0 / 2 of the shifted scale dword: the lane's
      // 32-k block of 64-k step 0 / 1 of the half
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fp4_op(lo4(wf[t][i])), fp4_op(lo4(xf[t][j])),
                                                                      acc[i][j], 4, 4, 0, (int)wsc[t][i], 0,
                                                                      (int)xsc[t][j]);
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fp4_op(hi4(wf[t][i])), fp4_op(hi4(xf[t][j])),
                                                                      acc[i][j], 4, 4, 2, (int)wsc[t][i], 2,
                                                                      (int)xsc[t][j]);
    } else if constexpr (INT) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < MJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(h ? hi4(wf[t][i]) : lo4(wf[t][i]),
                                                              h ? hi4(xf[t][j]) : lo4(xf[t][j]), acc[i][j], 0, 0,
                                                              0);
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[t][i], xf[t][j], acc[i][j], 0, 0, 0, 127,
                                                                      0, 127);
    }
  };
  constexpr int NM = NI * MJ * (INT || MX ? 2 : 1);
  constexpr int NR = (MX ? 3 : 2) * (NI + MJ);

  // tiles of this workgroup: b = blockIdx.x + i * gridDim.x over the
  // XCD-ordered slots [0, tile_slots), or in plain order (wide: rows of a
  // multiple of 32 KB)
  auto tile_of = [&](int bb, int& m, int& n) {
    return wide ? tile_wide(bb, m_tiles, n_tiles, m, n) : tile_dense(bb, m_tiles, n_tiles, m, n);
  };
  int b = blockIdx.x;
  int mt, nt;
  if (!tile_of(b, mt, nt)) return;
  Src cur;
  int row0 = mt * BM, rows = min(BM, p.M - row0), n0 = nt * BNO;
  make_src(row0, rows, n0, cur);
  copy_stage(sW0, sX0, sQW0, sQX0, cur, 0);
  copy_stage(sW1, sX1, sQW1, sQX1, cur, 1);
  wait_copies_upto<CPS>();
  __syncthreads();

  for (int par = 0;; par ^= 1) {
    // the next tile (or none: the last copies then refetch this tile's last
    // stage into buffers that are never read again)
    int mt2 = 0, nt2 = 0;
    const bool has_next = b + (int)gridDim.x < tile_slots && tile_of(b + gridDim.x, mt2, nt2);
    const int row0n = mt2 * BM, rowsn = has_next ? min(BM, p.M - row0n) : 0, n0n = nt2 * BNO;

    // stage 0 has landed everywhere (prologue / end of the previous tile)
    read_frags(sW0, sX0, sQW0, sQX0, 0, 0);
    // epilogue inputs of this tile (token tid's activation scale, weight row
    // tid's scale; MX: weight row tid's bias), loaded now and stored to LDS
    // after stage 0
    float e_sx = 0.0f, e_ws = 0.0f;
    if constexpr (MX) {
      if (p.bias) e_ws = p.bias[min(n0 + tid, nlim - 1)];
    } else {
      e_sx = p.a_scale[(int64_t)(row0 + min(tid, rows - 1)) * p.lds_a];
      e_ws = static_cast<const float*>(p.w_scale)[min(n0 + tid, nlim - 1)];
    }
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < MJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    // Stage s lives in LDS buffer s % 2 (as in f8_gemm_kernel with 128-byte
    // stages) and copies stage kc of the tile in `cur`: s + 2 of this tile,
    // and in the last two stages the next tile's stages 0 and 1 (`cur` is
    // switched to the next tile before them), or this tile's last stage
    // again when there is no next tile (into a buffer never read again).
    // The last stage reads no operands ahead and does not wait for the
    // copies: the next tile's first stage lands while the epilogue runs.
    auto stage = [&](uint8_t* cW, uint8_t* cX, uint8_t* cQW, uint8_t* cQX, uint8_t* nW, uint8_t* nX,
                     uint8_t* nQW, uint8_t* nQX, int kc, bool last) {
      mma(0);
      read_frags(cW, cX, cQW, cQX, 1, 1);
      interleave<0, NM, NR, 0>();
      __builtin_amdgcn_sched_barrier(0);
      if (!last) wait_copies_upto<0>();  // stage s + 1 has landed
      stage_barrier();
      if (!last) read_frags(nW, nX, nQW, nQX, 0, 0);
      copy_stage(cW, cX, cQW, cQX, cur, kc);
      mma(1);
      interleave<0, NM, NR, CPS>();
    };
    stage(sW0, sX0, sQW0, sQX0, sW1, sX1, sQW1, sQX1, 2, false);
    // the epilogue vectors have landed (the wait in stage 0 covers every
    // earlier load); the stage barriers ahead make them visible
    if (BM == 256 || tid < BM) s_sx[par][tid] = e_sx;
    if (BN == 256 || tid < BN) s_ws[par][tid] = e_ws;
    stage(sW1, sX1, sQW1, sQX1, sW0, sX0, sQW0, sQX0, 3, false);
    for (int s = 2; s < KS - 2; s += 2) {
      stage(sW0, sX0, sQW0, sQX0, sW1, sX1, sQW1, sQX1, s + 2, false);
      stage(sW1, sX1, sQW1, sQX1, sW0, sX0, sQW0, sQX0, s + 3, false);
    }
    if (has_next) make_src(row0n, rowsn, n0n, cur);
    stage(sW0, sX0, sQW0, sQX0, sW1, sX1, sQW1, sQX1, has_next ? 0 : KS - 1, false);
    stage(sW1, sX1, sQW1, sQX1, sW0, sX0, sQW0, sQX0, has_next ? 1 : KS - 1, true);
    // the epilogue starts after the last MFMAs: the empty asm takes every
    // accumulator, so no MFMA can be sunk into the epilogue (interleaving
    // the two keeps the last stage's operands alive across it)
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < MJ; ++j) asm volatile("" : "+a"(acc[i][j]));
    __builtin_amdgcn_sched_barrier(0);

    // ---- epilogue (the next tile's first two stages are in flight) ----
    // A register quad holds 4 consecutive output channels of one token; the
    // lane 32 apart holds the next 4 (kh = 1). The two exchange one quad of
    // each pair (q even, q odd), so lane kh = 0 stores the 8 channels of the
    // even quad and lane kh = 1 those of the odd one: one 16-byte bf16 store
    // per lane per pair (the host guarantees N % 8 == 0 and 16-byte aligned
    // output rows), bf16 by the hardware round-to-nearest-even conversion.
    const qmoe_stream::rsrc_t yres = qmoe_stream::make_rsrc(p.y, (int64_t)p.M * p.ldy * 2);
    float sxa[MJ];
    bool tok_ok[MJ];
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
      const int tr = wm * TM + j * 32 + rl;
      tok_ok[j] = tr < rows;
      sxa[j] = s_sx[par][min(tr, rows - 1)];
    }
    // Stores in token-major order: the four stores (i, qp) of blocks i = 2c,
    // 2c + 1 cover 128 contiguous bytes of a token's row back to back, so
    // the L2 assembles whole lines before writing them out.
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int qp = 0; qp < 2; ++qp) {
          const int lr_out = wrow(i) + (2 * qp + kh) * 8;  // first tile row of this lane's 8 channels
          const bool ch_ok = n0 + lr_out < nlim;
          uint32_t pk[2][2];  // [quad of the pair][dword]
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int q = 2 * qp + h;
            const float4 cs = *reinterpret_cast<const float4*>(s_ws[par] + wrow(i) + q * 8 + kh * 4);
            const float csv[4] = {cs.x, cs.y, cs.z, cs.w};
            float o[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
              o[t] = MX ? (float)acc[i][j][q * 4 + t] + csv[t] : ((float)acc[i][j][q * 4 + t] * sxa[j]) * csv[t];
            union { bf16x2 b; uint32_t u; } lo, hi;
            lo.b = __builtin_convertvector(f32x2{o[0], o[1]}, bf16x2);
            hi.b = __builtin_convertvector(f32x2{o[2], o[3]}, bf16x2);
            pk[h][0] = lo.u;
            pk[h][1] = hi.u;
          }
          // kh = 0 sends its odd quad and keeps the even one; kh = 1 the reverse
          const uint32_t s0 = kh ? pk[0][0] : pk[1][0], s1 = kh ? pk[0][1] : pk[1][1];
          const uint32_t r0 = (uint32_t)__shfl_xor((int)s0, 32, 64), r1 = (uint32_t)__shfl_xor((int)s1, 32, 64);
          i32x4 out;
          out[0] = (int)(kh ? r0 : pk[0][0]);
          out[1] = (int)(kh ? r1 : pk[0][1]);
          out[2] = (int)(kh ? pk[1][0] : r0);
          out[3] = (int)(kh ? pk[1][1] : r1);
          // outputs past the tile's tokens or channels store at an offset
          // past the buffer: the store is dropped, with no branch
          const uint32_t yoff = tok_ok[j] && ch_ok
                                    ? (uint32_t)((row0 + wm * TM + j * 32 + rl) * (uint32_t)p.ldy + n0 + lr_out) * 2u
                                    : qmoe_stream::kOob;
          __builtin_amdgcn_raw_buffer_store_b128(out, yres, yoff, 0, 0);
        }
    if (!has_next) {
      // no LDS copy may still be landing when the workgroup's LDS is freed
      wait_copies_upto<0>();
      break;
    }
    // the next tile's stage 0 has landed everywhere (its copies are older
    // than stage 1's and than the stores: at most CPS operations newer)
    wait_copies_upto<CPS>();
    stage_barrier();
    b += gridDim.x;
    row0 = row0n;
    rows = rowsn;
    n0 = n0n;
  }
}

// CUs the persistent kernel may use, a multiple of the 8 XCDs: 0 when the
// tuning knob QMOE_F8_PERSIST=0 turns the kernel off; another value of the
// knob caps them.
int f8_persistent_cus() {
  const char* env = getenv("QMOE_F8_PERSIST");  // tuning knob
  if (env && atoi(env) == 0) return 0;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess)
    return 0;
  if (env && atoi(env) >= kXcds) cus = std::min(cus, atoi(env));
  return cus / kXcds * kXcds;
}

// Workgroups of the persistent tile kernel for `tiles` tiles: as few tile
// rounds as the CUs allow, spread evenly (896 tiles on 256 CUs: 4 rounds on
// 224 workgroups, not 3.5 on 256; measured on MI355X, 216 vs 222 us for
// Llama-3-8B's up projection at 4096 tokens), rounded up to a multiple of
// the 8 XCDs. 0 when the tiles fit one round (the one-tile kernel then runs)
// or the kernel is off.
int f8_persistent_grid(int tiles) {
  const int cus = f8_persistent_cus();
  if (cus <= 0 || tiles <= cus / 2) return 0;
  const int rounds = cdiv(tiles, cus);
  return std::min(cus, cdiv(cdiv(tiles, rounds), kXcds) * kXcds);
}

// Weight rows per persistent tile: 224 where its tile rounds times rows,
// weighted by 17/16, are fewer than 256's on this device's CUs, else 256. A
// round's time follows the tile height, and a 224-row tile does ~6 % less
// per row than a 256-row one (7 x 2 blocks per wavefront instead of 4 x 4:
// more operand reads per MFMA). Measured on MI355X, Llama-3-8B's up
// projection (N 14336) at 4096 tokens, 1024 tiles in 4 rounds of 224 rows
// instead of 896 in 4 rounds of 256: 222.0 -> 207.8 us (FP8), 233.6 ->
// 216.7 us (INT8); at 8192 tokens (7 rounds of 256 against 8 of 224) 394 vs
// 418 us. The tuning knob QMOE_F8_PERSIST_BN (224 or 256) forces one.
int f8_persistent_bn(const GemmParams& p) {
  const char* env = getenv("QMOE_F8_PERSIST_BN");  // tuning knob
  if (env && (atoi(env) == 224 || atoi(env) == 256)) return atoi(env);
  const int cus = f8_persistent_cus();
  if (cus <= 0) return 256;
  const int mt = cdiv(p.M, 256);
  const int64_t c256 = (int64_t)cdiv(mt * cdiv(p.N, 256), cus) * 256;
  const int64_t c224 = (int64_t)cdiv(mt * cdiv(p.N, 224), cus) * 224;
  return c224 * 17 < c256 * 16 ? 224 : 256;
}

// Whether a dense problem with this plan runs the persistent kernel: 256 x
// 256 tiles of per-channel W8A8 without a fused activation or K split,
// 128-byte stages (the default of the QMOE_F8_KB knob), K >= 512, plain
// row-major output with N % 8 == 0 and 16-byte aligned rows below 2 GiB, no
// bias, row gather / scatter or routing weights, and more tiles than CUs.
bool f8_persistent_form_ok(const GemmParams& p, bool blk, int ksplit) {
  if (blk || ksplit != 1 || p.group_offs || p.act != QA_NONE || p.K < 512 || p.wfmt > 1) return false;
  const char* env = getenv("QMOE_F8_KB");
  if (env && atoi(env) == 64) return false;
  if ((p.N % 8) != 0 || (p.ldy % 8) != 0 || (reinterpret_cast<uintptr_t>(p.y) & 15) != 0) return false;
  return !(p.a_rows || p.y_rows || p.row_weight || p.bias || (int64_t)p.M * p.ldy * 2 >= 0x7fffffffLL);
}

bool f8_persistent_ok(const GemmParams& p, bool blk, int bm, int ksplit) {
  return bm == 256 && f8_persistent_form_ok(p, blk, ksplit) && f8_persistent_grid(cdiv(p.M, 256) * cdiv(p.N, 256)) > 0;
}

// Whether a problem planned on one-tile 64- or 128-token x 256-row tiles
// runs the persistent kernel in tiles of 128 tokens x 224 weight rows
// instead: the same form, and fewer tile rounds times tile area (the 224-row
// tile weighted as in f8_persistent_bn). Measured on MI355X, Llama-3-8B's up
// projection (K 4096, N 14336): 512 tokens 39.7 -> 36.0 us (256 tiles on 256
// CUs instead of 224 one-tile workgroups), 640 67.1 -> 58.5, 768 67.4 ->
// 59.7; 1000 x 7000 (K 2048) 25.4 -> 20.7 us.
bool f8_persistent_mid_ok(const GemmParams& p, bool blk, int bm, int bn, int ksplit) {
  if ((bm != 128 && bm != 64) || bn != 256 || !f8_persistent_form_ok(p, blk, ksplit)) return false;
  const char* env = getenv("QMOE_F8_PERSIST_BN");  // tuning knob: 256 keeps the one-tile kernel
  if (env && atoi(env) == 256) return false;
  const int cus = f8_persistent_cus();
  if (cus <= 0) return false;
  const int mid = cdiv(p.M, 128) * cdiv(p.N, 224);
  const int64_t c_cur = (int64_t)cdiv(cdiv(p.M, bm) * cdiv(p.N, 256), cus) * bm * 256 * 16;
  const int64_t c_mid = (int64_t)cdiv(mid, cus) * 128 * 224 * 17;
  return c_mid < c_cur && f8_persistent_grid(mid) > 0;
}

// Whether the persistent kernel walks its tiles in plain order (tile_wide):
// output rows of a multiple of 32 KB and K up to 1024, where it was
// measured (the QMOE_F8_PERSIST_ORDER knob forces 0: XCD runs, 1: plain
// order).
int f8_persistent_wide(const GemmParams& p) {
  const char* env = getenv("QMOE_F8_PERSIST_ORDER");  // tuning knob
  if (env && (atoi(env) == 0 || atoi(env) == 1)) return atoi(env);
  return ((int64_t)p.ldy * 2) % 32768 == 0 && p.K <= 1024 ? 1 : 0;
}

// The persistent kernel in 128 x 224 tiles (f8_persistent_mid_ok holds).
template <bool INT>
void f8_launch_mid(const GemmParams& p, hipStream_t st) {
  const int mt = cdiv(p.M, 128), pn = cdiv(p.N, 224), tiles = mt * pn;
  hipLaunchKernelGGL((f8_persistent_kernel<INT ? 1 : 0, 224, 128>), dim3(f8_persistent_grid(tiles)), dim3(kThreads),
                     0, st, p, mt, pn, cdiv(tiles, kXcds) * kXcds, f8_persistent_wide(p));
}

template <bool INT, int BM, int BN, bool ACT, bool BLK, bool WPC = false, int E5 = 0>
void f8_launch_shape(const GemmParams& p, hipStream_t st) {
  const char* env = getenv("QMOE_F8_KB");  // tuning knob: K bytes per LDS stage
  const int kb = BLK ? 128 : (env ? atoi(env) : 128);
  auto kern = kb == 64 ? f8_gemm_kernel<INT, BM, BN, ACT, BLK ? 128 : 64, BLK, WPC, false, E5>
                       : f8_gemm_kernel<INT, BM, BN, ACT, 128, BLK, WPC, false, E5>;
  const int nout = ACT ? p.N / 2 : p.N;
  const int n_tiles = cdiv(nout, ACT ? BN / 2 : BN);
  const unsigned ks = (unsigned)std::max(1, p.ksplit);
  if (p.group_offs) {
    const int m_tiles = cdiv(p.M, BM) + std::min(p.slots, p.M);
    hipLaunchKernelGGL(kern, dim3(n_tiles, m_tiles, ks), dim3(kThreads), 0, st, p, m_tiles, n_tiles);
  } else {
    const int m_tiles = cdiv(p.M, BM);
    const int grid = cdiv(m_tiles * n_tiles, kXcds) * kXcds;
    if constexpr (BM == 256 && BN == 256 && !BLK && !ACT && E5 == 0) {
      if (kb == 128 && f8_persistent_ok(p, BLK, BM, (int)ks)) {
        const int pbn = f8_persistent_bn(p);
        const int pn = cdiv(p.N, pbn), tiles = m_tiles * pn, slots = cdiv(tiles, kXcds) * kXcds;
        const int wide = f8_persistent_wide(p);
        if (pbn == 224)
          hipLaunchKernelGGL((f8_persistent_kernel<INT ? 1 : 0, 224>), dim3(f8_persistent_grid(tiles)),
                             dim3(kThreads), 0, st, p, m_tiles, pn, slots, wide);
        else
          hipLaunchKernelGGL((f8_persistent_kernel<INT ? 1 : 0>), dim3(f8_persistent_grid(tiles)), dim3(kThreads),
                             0, st, p, m_tiles, pn, slots, wide);
        return;
      }
    }
    hipLaunchKernelGGL(kern, dim3(grid, 1, ks), dim3(kThreads), 0, st, p, m_tiles, n_tiles);
  }
}

template <bool INT, int BM, int BN, bool BLK, bool WPC = false, int E5 = 0>
void f8_launch_act(const GemmParams& p, hipStream_t st) {
  if (p.act != QA_NONE) f8_launch_shape<INT, BM, BN, true, BLK, WPC, E5>(p, st);
  else f8_launch_shape<INT, BM, BN, false, BLK, WPC, E5>(p, st);
}

template <bool INT, int E5 = 0>
void f8_launch_bm(const GemmParams& p, int bm, int bn, hipStream_t st) {
  if (bn == 128 && p.act == QA_NONE) {  // narrow weight tiles (twice the workgroups)
    switch (bm) {
      case 256: f8_launch_shape<INT, 256, 128, false, false, false, E5>(p, st); break;
      case 128: f8_launch_shape<INT, 128, 128, false, false, false, E5>(p, st); break;
      case 64: f8_launch_shape<INT, 64, 128, false, false, false, E5>(p, st); break;
      default: f8_launch_shape<INT, 32, 128, false, false, false, E5>(p, st); break;
    }
    return;
  }
  switch (bm) {
    case 256: f8_launch_act<INT, 256, 256, false, false, E5>(p, st); break;
    case 128: f8_launch_act<INT, 128, 256, false, false, E5>(p, st); break;
    case 64: f8_launch_act<INT, 64, 256, false, false, E5>(p, st); break;
    default: f8_launch_act<INT, 32, 256, false, false, E5>(p, st); break;
  }
}

// block-scaled tiles: at most 128 tokens (the per-block sums need a second
// accumulator set); E5 1: e5m2 weights against e4m3 activations; INT: int8
// codes (the grouped-matmul recipe for int8 weights)
template <bool INT, bool WPC, int E5 = 0>
void f8_launch_bm_blk(const GemmParams& p, int bm, int bn, hipStream_t st) {
  if (bn == 128) {
    // 128-row weight tiles: a fused activation (gate and up halves of 64
    // rows) needs two weight blocks per wavefront, so 128-token tiles
    if (bm == 128) f8_launch_act<INT, 128, 128, true, WPC, E5>(p, st);
    else if (bm == 64) f8_launch_shape<INT, 64, 128, false, true, WPC, E5>(p, st);
    else f8_launch_shape<INT, 32, 128, false, true, WPC, E5>(p, st);
    return;
  }
  switch (bm) {
    case 128: f8_launch_act<INT, 128, 256, true, WPC, E5>(p, st); break;
    case 64: f8_launch_act<INT, 64, 256, true, WPC, E5>(p, st); break;
    default: f8_launch_act<INT, 32, 256, true, WPC, E5>(p, st); break;
  }
}

// per-channel weight scales with block activation scales (the grouped-matmul
// recipe): one weight scale for the whole row
bool f8_wpc(const GemmParams& p) { return p.w_kshift >= 31; }

}  // namespace

// Token-tile height: the largest of 256 / 128 / 64 / 32 whose tile count
// still fills the CUs (dense), or that fits the average group (grouped).
static int f8_pick_bm_any(const GemmParams& p) {
  const char* env = getenv("QMOE_F8_BM");  // tuning knob
  if (env) {
    const int v = atoi(env);
    if (v == 256 || v == 128 || v == 64 || v == 32) return v;
  }
  const int nout = p.act != QA_NONE ? p.N / 2 : p.N;
  const int n_tiles = cdiv(nout, p.act != QA_NONE ? 128 : 256);
  if (p.group_offs) {
    // measured on MI355X (DeepSeek-V3 MoE, 256 experts): 64-token tiles
    // also below 48 rows per routed expert (32-token tiles lose ~5%)
    const int avg = std::max(1, p.M / std::max(1, std::min(p.slots, p.M)));
    if (avg > 192) return 256;
    if (avg > 96) return 128;
    return 64;
  }
  for (int bm : {256, 128, 64}) {
    if ((int64_t)cdiv(p.M, bm) * n_tiles >= 200) return bm;
  }
  return 32;
}

// Whether this kernel takes the problem (K % 256, 16-byte alignment,
// weights < 4 GiB per group), and its plan: token-tile height, K split and
// the f32 workspace the split needs ([ksplit][M][N]).
bool qmoe_f8_plan(const GemmParams& p, bool blk, int* bm_out, int* ksplit_out, int64_t* ws_bytes, int* bn_out) {
  if (p.M <= 0 || p.K <= 0 || (p.K % 256) != 0 || p.N <= 0) return false;
  if (p.act != QA_NONE && (p.N % 2) != 0) return false;
  // block scales: 128-row weight blocks aligned with the tile's halves
  // (per-channel weight scales need no alignment); 1-byte FP8 codes only
  if (blk && !f8_wpc(p) && (p.ws_bn != 128 || (p.act != QA_NONE && ((p.N / 2) % 128) != 0))) return false;
  // block scales take e4m3 codes, e5m2 weights against e4m3 activations or
  // int8 codes on both operands (the last two: the grouped-matmul recipe)
  if ((p.lda % 16) != 0 || (p.ldw % 16) != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.a) & 15) || (reinterpret_cast<uintptr_t>(p.w) & 15) ||
      (p.w_gstride % 16) != 0)
    return false;
  if ((int64_t)p.ldw * p.N >= ((int64_t)1 << 32)) return false;
  int bm = f8_pick_bm_any(p);
  int ksplit = 1;
  const bool env_bm = getenv("QMOE_F8_BM") != nullptr;
  // dense block-scaled problems with at least 64 weight-row tiles (16384
  // output channels: DeepSeek-V3's wide projections) take the tile height
  // and K split measured best on MI355X (K 7168, N 18432 / 24576)
  const int nout = p.act != QA_NONE ? p.N / 2 : p.N;
  const bool blk_wide = blk && !p.group_offs && cdiv(nout, p.act != QA_NONE ? 128 : 256) >= 64;
  if (blk && !env_bm) {
    // block-scaled tiles hold at most 128 tokens; measured on MI355X (K 7168,
    // N 18432): 128-token tiles up to 256 and from 2048 tokens, 64 between
    bm = p.group_offs ? std::min(bm, 128) : (p.M > 256 && p.M < 2048 ? 64 : 128);
    // grouped: 32-token tiles up to 12 rows per routed expert (measured on
    // MI355X, DeepSeek-V3 experts: 4-12 rows 3-16% faster than 64)
    if (p.group_offs && p.M <= 12 * std::max(1, std::min(p.slots, p.M))) bm = 32;
    if (blk_wide) {
      // (tokens: tile, split) 32: 32/2 (27 vs 34 us streaming), 64: 64/2
      // (33 vs 60 us), 128: 64/1 (49 vs 85 us), 256: 128/1, 512: 64/1,
      // 1024: 128/1 (254 vs 296 us at N 24576)
      if (p.M <= 32) { bm = 32; ksplit = 2; }
      else if (p.M <= 64) { bm = 64; ksplit = 2; }
      else if (p.M <= 128) bm = 64;
      else if (p.M <= 256) bm = 128;
      else if (p.M <= 512) bm = 64;
      else bm = 128;
      ksplit = std::min(ksplit, p.K / 256);
    }
  }
  const int m_tiles = p.group_offs ? cdiv(p.M, bm) + std::min(p.slots, p.M) : cdiv(p.M, bm);
  if (p.group_offs && m_tiles > 65535) return false;
  // Dense problems whose largest CU-filling tile is small (tall-K, few
  // tokens) are split over K, with the tile and split that measured best on
  // MI355X: (32 rows, 4 slices) up to 128 tokens, (64, 4) up to 256 (K 14336,
  // N 4096: 30 vs 39 us), (128, 4) up to 512, (128, 2) above.
  if (!p.group_offs && !blk_wide && bm <= 64 && p.K >= 8192 && !env_bm) {
    if (p.M <= 128) { bm = 32; ksplit = 4; }
    else if (p.M <= 256) { bm = 64; ksplit = 4; }
    else if (p.M <= 512) { bm = 128; ksplit = 4; }
    else { bm = 128; ksplit = 2; }
  }
  // Dense per-channel problems (no fused activation) whose 256-row weight
  // tiles leave CUs idle take 128-row weight tiles (twice the workgroups),
  // with the token tile and split measured best on MI355X (Llama-3-8B MLP
  // shapes): K 4096, N 14336: 64 tokens 32 / 1 (14.9 vs 18.5 us), 128
  // tokens 64 / 1 (17.1 vs 19.1), 256 tokens 128 / 1 (22.9 vs 24.2); K
  // 14336, N 4096: 512 tokens 128 / 2 (42.2 vs 44.9), 1024 tokens 128 / 1
  // (59.6 vs 70.0).
  int bn = 256;
  if (!blk && !p.group_offs && p.act == QA_NONE && !env_bm) {
    const int n256 = cdiv(p.N, 256);
    if (p.K < 8192 && p.M <= 256) {
      const int b = p.M <= 64 ? 32 : (p.M <= 128 ? 64 : 128);
      if (cdiv(p.M, b) * n256 < 256) { bm = b; bn = 128; ksplit = 1; }
    } else if (p.K >= 8192 && p.M > 256 && p.M <= 1024 && cdiv(p.M, 128) * n256 < 256) {
      bm = 128;
      bn = 128;
      ksplit = p.M <= 512 ? 2 : 1;
    } else if (p.K < 8192 && p.M > 256 && n256 <= 4 && cdiv(p.M, 128) * cdiv(p.N, 128) <= 256) {
      // at most 1024 channels (DeepSeek-V3's kv_a projection, 576): 64- or
      // 128-token tiles of 128 rows, the larger once the smaller would make
      // over 256 tiles. Measured on MI355X: K 7168, N 576, 512 / 1024 / 2048
      // / 4096 tokens 26.3 / 25.3 / 26.6 / 48.4 -> 20.9 / 21.7 / 21.6 / 28.6
      // us; N 512, 4096 / 8192 tokens 28.6 / 37.2 -> 24.1 / 34.2; K 4096,
      // N 1024, 2048 / 4096 tokens 19.1 / 25.0 -> 15.3 / 23.6
      bm = cdiv(p.M, 64) * cdiv(p.N, 128) <= 256 ? 64 : 128;
      bn = 128;
      ksplit = 1;
    }
  }
  // Dense wide block-scaled problems (the blk_wide rule above) take 128-row
  // weight tiles where they measured faster on MI355X (K 7168, N 18432 /
  // 24576): 64 tokens 64 / 1 (35.5 / 39.6 -> 32.6 / 33.7 us), 128 tokens
  // 128 / 1 (48.8 / 49.5 -> 44.5 / 47.3), 257-512 tokens 64 / 1 (142.0 /
  // 158.1 -> 121.0 / 147.0); 256 and 1024 tokens keep 256-row tiles
  if (blk_wide && !env_bm && p.act == QA_NONE && ((p.M > 32 && p.M <= 128) || (p.M > 256 && p.M <= 512))) {
    bm = p.M <= 64 || p.M > 256 ? 64 : 128;
    bn = 128;
    ksplit = 1;
  }
  // Grouped 128 x 128-tile problems without an activation (the MoE down
  // projection) in 32- or 64-token tiles: 128-row weight tiles, measured on
  // MI355X (DeepSeek-V3 layer, native tiles) T = 256 / 512 1373.6 / 1566.8
  // -> 1319.1 / 1517.9 us; 128-token tiles (T = 4096) lose with them
  if (blk && p.group_offs && !f8_wpc(p) && p.act == QA_NONE && !env_bm && bm <= 64) bn = 128;
  const char* env_bn = getenv("QMOE_F8_BN");  // tuning knob: 128 or 256
  if (env_bn && (p.act == QA_NONE || (blk && bm == 128))) bn = atoi(env_bn) == 128 ? 128 : 256;
  if (blk && bn == 128 && bm > 128) bn = 256;
  const char* env = getenv("QMOE_F8_KSPLIT");  // tuning knob
  if (env && atoi(env) > 0) ksplit = std::max(1, std::min(atoi(env), p.K / 256));
  if (bn_out) *bn_out = bn;
  *bm_out = bm;
  *ksplit_out = ksplit;
  *ws_bytes = ksplit > 1 ? (int64_t)ksplit * p.M * p.N * 4 : 0;
  return true;
}

// Whether the planned problem runs the persistent kernel (256 x 256 / 256 x 224
// tiles, or 128 x 224 for mid-size problems).
bool qmoe_f8_persistent(const GemmParams& p, bool blk) {
  int bm = 0, ksplit = 1, bn = 256;
  int64_t ws = 0;
  return qmoe_f8_plan(p, blk, &bm, &ksplit, &ws, &bn) && bn == 256 &&
         (f8_persistent_ok(p, blk, bm, ksplit) || f8_persistent_mid_ok(p, blk, bm, bn, ksplit));
}

// K-split finish of the generic tiled kernel's f32 partials (no fused
// activation): the partials carry every scale, or all but the per-channel
// weight scale (weight_scale: bf16 activations against e4m3 weights).
int qmoe_tile_splitk_finish(const GemmParams& p, bool weight_scale, hipStream_t st) {
  if (p.act != QA_NONE || p.ksplit < 2 || !p.partial) return QMOE_ERR_ARG;
  const dim3 rg((unsigned)cdiv(p.N, 512), (unsigned)cdiv(p.M, 4), 1);
  if (weight_scale) hipLaunchKernelGGL((tile_splitk_finish_kernel<false, false, kScWeight>), rg, dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL((tile_splitk_finish_kernel<false, false, kScNone>), rg, dim3(kThreads), 0, st, p);
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}

// Launch per the plan (the caller checked qmoe_f8_plan and sized the
// workspace); with a K split the reduce kernel finishes the epilogue.
int qmoe_f8_launch(GemmParams p, bool blk, void* workspace, int64_t ws_bytes, hipStream_t st) {
  int bm = 0, ksplit = 1;
  int64_t need = 0;
  int bn = 256;
  if (!qmoe_f8_plan(p, blk, &bm, &ksplit, &need, &bn)) return QMOE_ERR_ARG;
  p.ksplit = ksplit;
  if (ksplit > 1) {
    if (!workspace || ws_bytes < need) return QMOE_ERR_WORKSPACE;
    p.partial = static_cast<float*>(workspace);
  }
  // e5m2 weights (wfmt 2): against e5m2 activations for per-channel W8A8,
  // e4m3 ones for the grouped-matmul recipe; int8 (wfmt 1) block-scaled
  // tiles: the grouped-matmul recipe for int8 weights
  if (blk && f8_wpc(p) && p.wfmt == 2) f8_launch_bm_blk<false, true, 1>(p, bm, bn, st);
  else if (blk && f8_wpc(p) && p.wfmt == 1) f8_launch_bm_blk<true, true>(p, bm, bn, st);
  else if (blk && f8_wpc(p)) f8_launch_bm_blk<false, true>(p, bm, bn, st);
  else if (blk && p.wfmt == 2) f8_launch_bm_blk<false, false, 1>(p, bm, bn, st);
  else if (blk && p.wfmt == 1) f8_launch_bm_blk<true, false>(p, bm, bn, st);
  else if (blk) f8_launch_bm_blk<false, false>(p, bm, bn, st);
  else if (f8_persistent_mid_ok(p, blk, bm, bn, ksplit) && p.wfmt == 1) f8_launch_mid<true>(p, st);
  else if (f8_persistent_mid_ok(p, blk, bm, bn, ksplit)) f8_launch_mid<false>(p, st);
  else if (p.wfmt == 1) f8_launch_bm<true>(p, bm, bn, st);
  else if (p.wfmt == 2) f8_launch_bm<false, 3>(p, bm, bn, st);
  else f8_launch_bm<false>(p, bm, bn, st);
  if (ksplit > 1) {
    const int nout = p.act != QA_NONE ? p.N / 2 : p.N;
    const dim3 rg((unsigned)cdiv(nout, 512), (unsigned)cdiv(p.M, 4), 1);
    const bool act = p.act != QA_NONE;
    if (blk && f8_wpc(p)) {
      if (act) hipLaunchKernelGGL((tile_splitk_finish_kernel<false, true, kScWeight>), rg, dim3(kThreads), 0, st, p);
      else hipLaunchKernelGGL((tile_splitk_finish_kernel<false, false, kScWeight>), rg, dim3(kThreads), 0, st, p);
    } else if (blk) {
      if (act) hipLaunchKernelGGL((tile_splitk_finish_kernel<false, true, kScNone>), rg, dim3(kThreads), 0, st, p);
      else hipLaunchKernelGGL((tile_splitk_finish_kernel<false, false, kScNone>), rg, dim3(kThreads), 0, st, p);
    } else if (p.wfmt == 1) {
      if (act) hipLaunchKernelGGL((tile_splitk_finish_kernel<true, true, kScAll>), rg, dim3(kThreads), 0, st, p);
      else hipLaunchKernelGGL((tile_splitk_finish_kernel<true, false, kScAll>), rg, dim3(kThreads), 0, st, p);
    } else {
      if (act) hipLaunchKernelGGL((tile_splitk_finish_kernel<false, true, kScAll>), rg, dim3(kThreads), 0, st, p);
      else hipLaunchKernelGGL((tile_splitk_finish_kernel<false, false, kScAll>), rg, dim3(kThreads), 0, st, p);
    }
  }
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}

// ---- MX (QK_W4A4_MX) ----
// Dense problems: the persistent 256 x 256 kernel in mode 2 (no fused
// activation, bias only). Grouped problems (MoE): the one-tile kernel in MX
// mode with 256- or 128-token tiles (the average rows per routed group above
// or below 192), fused activation, bias, routing weight and row maps, no K
// split. Both: K % 512 == 0 and K >= 1024 (128-byte stages of packed codes,
// an even count of at least 4), 16-byte aligned code rows and operands,
// 4-byte aligned scale rows, weights within the kernels' 32-bit offsets.
// Returns the token-tile height, 0 when no MX kernel takes the problem.
int qmoe_mx_plan(const GemmParams& p) {
  if (p.M <= 0 || p.N <= 0 || (p.K % 512) != 0 || p.K < 1024 || !p.a_scale || !p.w_scale) return 0;
  if (p.act != QA_NONE && (p.N % 2) != 0) return 0;
  if ((p.lda % 16) != 0 || (p.ldw % 16) != 0 || (p.lds_a % 4) != 0 || (p.ldws % 4) != 0) return 0;
  if ((reinterpret_cast<uintptr_t>(p.a) & 15) || (reinterpret_cast<uintptr_t>(p.w) & 15) ||
      (reinterpret_cast<uintptr_t>(p.a_scale) & 3) || (reinterpret_cast<uintptr_t>(p.w_scale) & 3) ||
      (p.w_gstride % 16) != 0 || (p.ws_gstride % 4) != 0)
    return 0;
  if ((int64_t)p.ldw * p.N >= ((int64_t)1 << 32) || (int64_t)p.ldws * p.N >= ((int64_t)1 << 32)) return 0;
  if (p.group_offs) {
    const int avg = std::max(1, p.M / std::max(1, std::min(p.slots, p.M)));
    int bm = avg > 192 ? 256 : 128;
    const char* env = getenv("QMOE_MX_BM");  // tuning knob: 128 or 256
    if (env && (atoi(env) == 128 || atoi(env) == 256)) bm = atoi(env);
    return cdiv(p.M, bm) + std::min(p.slots, p.M) > 65535 ? 0 : bm;
  }
  if (p.act != QA_NONE || p.a_rows || p.y_rows || p.row_weight) return 0;
  if ((p.N % 8) != 0 || (p.ldy % 8) != 0 || (reinterpret_cast<uintptr_t>(p.y) & 15) != 0) return 0;
  return (int64_t)p.M * p.ldy * 2 < 0x7fffffffLL ? 256 : 0;
}

namespace {

template <int BM, bool ACT>
void mx_launch_grouped(const GemmParams& p, hipStream_t st) {
  const int nout = ACT ? p.N / 2 : p.N;
  const int n_tiles = cdiv(nout, ACT ? 128 : 256);
  const int m_tiles = cdiv(p.M, BM) + std::min(p.slots, p.M);
  hipLaunchKernelGGL((f8_gemm_kernel<false, BM, 256, ACT, 128, false, false, true>), dim3(n_tiles, m_tiles, 1),
                     dim3(kThreads), 0, st, p, m_tiles, n_tiles);
}

}  // namespace

// Dense: as few tile rounds as the CUs allow, spread evenly over a multiple
// of the 8 XCDs (also for fewer tiles than CUs: one tile each). Grouped: one
// workgroup per (weight tile, token tile of a group), as the FP8 tiles.
int qmoe_mx_launch(GemmParams p, hipStream_t st) {
  const int bm = qmoe_mx_plan(p);
  if (!bm) return QMOE_ERR_ARG;
  p.ksplit = 1;
  if (p.group_offs) {
    p.active = nullptr;  // the tiles enumerate every group
    p.num_active = nullptr;
    const bool act = p.act != QA_NONE;
    if (bm == 256) act ? mx_launch_grouped<256, true>(p, st) : mx_launch_grouped<256, false>(p, st);
    else act ? mx_launch_grouped<128, true>(p, st) : mx_launch_grouped<128, false>(p, st);
    return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
  }
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return QMOE_ERR_LAUNCH;
  cus = std::max(kXcds, cus / kXcds * kXcds);
  const int m_tiles = cdiv(p.M, 256), n_tiles = cdiv(p.N, 256);
  const int tiles = m_tiles * n_tiles;
  const int rounds = cdiv(tiles, cus);
  const int grid = std::min(cus, cdiv(cdiv(tiles, rounds), kXcds) * kXcds);
  hipLaunchKernelGGL((f8_persistent_kernel<2>), dim3(grid), dim3(kThreads), 0, st, p, m_tiles, n_tiles,
                     cdiv(tiles, kXcds) * kXcds, 0);
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
