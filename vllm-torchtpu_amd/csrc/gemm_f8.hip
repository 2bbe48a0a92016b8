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

#include "gemm_common.h"


namespace {

constexpr int kThreads = 256;
constexpr int kXcds = 8;
constexpr int kGroupM = 8;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

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


#define QMOE_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// Wait until at most N of this wavefront's vector-memory operations (here:
// LDS copies) are outstanding; expcnt and lgkmcnt are left alone. A
// workgroup barrier alone does not wait for them: the compiler orders only
// ordinary global accesses at workgroup scope, and an LDS copy's data is in
// LDS only once its vector-memory count retires (they retire in order).
// Workgroup barrier between stages. It waits for this wavefront's LDS
// operand reads (lgkmcnt(0)) but, unlike __syncthreads, not for its LDS
// copies in flight: a workgroup-scope fence would count those as pending LDS
// writes and drain them all, which would remove the copies' latency slack.
// Scheduler fences keep the MFMAs -- which touch no memory -- from drifting
// into a neighbouring stage; the empty asm keeps the compiler's memory
// accesses on their side of the barrier.
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt untouched
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Scheduling pattern of one stage: NM MFMAs; the NR LDS operand reads are
// spread over the first half of them, the NC LDS copies (vector-memory
// reads) over the second half.
template <int K, int NM, int NR, int NC>
__device__ __forceinline__ void interleave() {
  if constexpr (K < NM) {
    constexpr int H = NM / 2 > 0 ? NM / 2 : 1;
    constexpr int r0 = K < H ? K * NR / H : NR, r1 = K < H ? (K + 1) * NR / H : NR;
    constexpr int c0 = K < H ? 0 : (K - H) * NC / (NM - H), c1 = K < H ? 0 : (K - H + 1) * NC / (NM - H);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    if constexpr (r1 > r0) __builtin_amdgcn_sched_group_barrier(0x100, r1 - r0, 0);  // DS read
    if constexpr (c1 > c0) __builtin_amdgcn_sched_group_barrier(0x020, c1 - c0, 0);  // VMEM read
    interleave<K + 1, NM, NR, NC>();
  }
}

template <int N>
__device__ __forceinline__ void wait_copies_upto() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ i32x8 lds_frag(const uint8_t* p0, const uint8_t* p1) {
  const uint4 a = *reinterpret_cast<const uint4*>(p0);
  const uint4 b = *reinterpret_cast<const uint4*>(p1);
  i32x8 r;
  r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
  r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
  return r;
}

__device__ __forceinline__ i32x4 lo4(const i32x8& v) { return i32x4{v[0], v[1], v[2], v[3]}; }
__device__ __forceinline__ i32x4 hi4(const i32x8& v) { return i32x4{v[4], v[5], v[6], v[7]}; }

template <int BM>
__device__ __forceinline__ bool f8_group_tile(const GemmParams& p, int y, int& g, int& row0, int& rows,
                                              int* s_info) {
  const int G = p.slots;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int done = 0, found = -1, fr0 = 0, frows = 0;
    for (int g0 = 0; g0 < G && found < 0; g0 += 64) {
      const int gg = g0 + lane;
      int cnt = 0, r0 = 0;
      if (gg < G) {
        r0 = p.group_offs[gg];
        cnt = p.group_offs[gg + 1] - r0;
      }
      const int nt = (cnt + BM - 1) / BM;
      int incl = nt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
      }
      const int excl = done + incl - nt;
      const uint64_t bal = __ballot(gg < G && y >= excl && y < excl + nt);
      if (bal) {
        const int src = __ffsll((unsigned long long)bal) - 1;
        const int mt = y - __shfl(excl, src, 64);
        found = __shfl(gg, src, 64);
        fr0 = __shfl(r0, src, 64) + mt * BM;
        frows = min(BM, __shfl(cnt, src, 64) - mt * BM);
      }
      done += __shfl(incl, 63, 64);
    }
    if (lane == 0) {
      s_info[0] = found;
      s_info[1] = fr0;
      s_info[2] = frows;
    }
  }
  __syncthreads();
  g = s_info[0];
  row0 = s_info[1];
  rows = s_info[2];
  return g >= 0;
}

__device__ __forceinline__ bool f8_dense_tile(int b, int m_tiles, int n_tiles, int& mt, int& nt) {
  const int total = m_tiles * n_tiles;
  const int per = (total + kXcds - 1) / kXcds;
  const int t = (b % kXcds) * per + b / kXcds;
  if (t >= total) return false;
  const int group = t / (kGroupM * n_tiles);
  const int first_m = group * kGroupM;
  const int gm = min(kGroupM, m_tiles - first_m);
  const int in = t - group * kGroupM * n_tiles;
  mt = first_m + in % gm;
  nt = in / gm;
  return true;
}

template <bool INT, int BM, int BN, bool ACT, int KB, bool BLK>
__global__ __launch_bounds__(kThreads) void f8_gemm_kernel(const GemmParams p, int m_tiles, int n_tiles) {
  static_assert(KB == 64 || KB == 128, "K bytes per LDS stage");
  // BLK: 128x128 block scales (W8A8_BLK): one 128-byte stage is one K block
  static_assert(!BLK || (KB == 128 && !INT && BN == 256), "block scales: FP8, 128-byte stages, 256-row tiles");
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
    if (!f8_group_tile<BM>(p, blockIdx.y, g, row0, rows, s_info)) return;
    ntile = blockIdx.x;
  } else {
    int mt;
    if (!f8_dense_tile(blockIdx.x, m_tiles, n_tiles, mt, ntile)) return;
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
    e_sx = BLK ? 1.0f : p.a_scale[(int64_t)ar * p.lds_a];
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
    e_ws = BLK ? 1.0f : static_cast<const float*>(p.w_scale)[(int64_t)g * p.ws_gstride + n];
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
  // BLK: this lane's source for the per-stage scale copy (4 bytes; the K
  // block index is added per stage): LDS slot wave*64 + lane holds token
  // scale `slot` for slot < BM, the scale of LDS weight rows
  // [(slot-BM)*128, +128) for slot < BM + 2, a duplicate elsewhere
  const float* sc_src = p.a_scale;
  if constexpr (BLK) {
    const int slot = wave * 64 + lane;
    if (slot >= BM && slot < BM + 2) {
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
  const int NU = p.K / 256;
  const int u0 = (int)((int64_t)NU * blockIdx.z / p.ksplit);
  const int u1 = (int)((int64_t)NU * (blockIdx.z + 1) / p.ksplit);
  const uint32_t kbase = (uint32_t)u0 * 256u;
  auto copy_stage = [&](uint8_t* dW, uint8_t* dX, float* dS, int ks) {
    const uint32_t kb = kbase + (uint32_t)ks * (uint32_t)KB;
    if constexpr (BLK)
      __builtin_amdgcn_global_load_lds(sc_src + kb / 128, QMOE_LDS(dS + wave * 64), 4, 0, 0);
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
      else po[t][h] = rl * 128 + (((4 * t + 2 * kh + h) ^ ((rl & 7) ^ ((rl >> 3) & 1))) * 16);
    }
  auto wrow = [&](int i) {  // LDS row of this wavefront's weight block i
    if (ACT) return (i < NI / 2 ? 0 : BN / 2) + wn * (TN / 2) + (i % (NI / 2)) * 32;
    return wn * TN + i * 32;
  };
  i32x8 wf[2][NI], xf[2][MJ];
  // operands of k-step `ks` of the stage in (sW, sX) into register set t
  auto read_frags = [&](const uint8_t* sW, const uint8_t* sX, int ks, int t) {
    const int h0 = KB == 64 ? po[0][0] : po[ks][0], h1 = KB == 64 ? po[0][1] : po[ks][1];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const uint8_t* b = sW + wrow(i) * KB;
      wf[t][i] = lds_frag(b + h0, b + h1);
    }
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
      const uint8_t* b = sX + (wm * TM + j * 32) * KB;
      xf[t][j] = lds_frag(b + h0, b + h1);
    }
  };

  using Acc = typename std::conditional<INT, i32x16, f32x16>::type;
  Acc acc[NI][MJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // BLK: the stage's block sums go to tmp, then acc += tmp * (sx * sw)
  f32x16 tmp[BLK ? NI : 1][BLK ? MJ : 1];
  float scl[BLK ? NI : 1][BLK ? MJ : 1];
  auto read_scales = [&](const float* sS) {
    if constexpr (BLK) {
      float sx[MJ];
#pragma unroll
      for (int j = 0; j < MJ; ++j) sx[j] = sS[wm * TM + j * 32 + rl];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const float sw = sS[BM + wrow(i) / 128];
#pragma unroll
        for (int j = 0; j < MJ; ++j) scl[i][j] = sx[j] * sw;
      }
    }
  };
  auto mma = [&](int t) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < MJ; ++j) {
        if constexpr (BLK) {
          const f32x16 c = t == 0 ? f32x16{} : tmp[i][j];
          tmp[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[t][i], xf[t][j], c, 0, 0, 0, 127, 0, 127);
        } else if constexpr (INT) {
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(lo4(wf[t][i]), lo4(xf[t][j]), acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(hi4(wf[t][i]), hi4(xf[t][j]), acc[i][j], 0, 0, 0);
        } else {
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[t][i], xf[t][j], acc[i][j], 0, 0, 0,
                                                                      127, 0, 127);
        }
      }
  };

  auto apply_scales = [&]() {
    if constexpr (BLK) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += tmp[i][j][r] * scl[i][j];
    }
  };

  constexpr int CPS = WI + XI + (BLK ? 1 : 0);  // copy instructions per wavefront per stage
  constexpr int NM = NI * MJ * (INT ? 2 : 1);  // MFMAs per k-step
  constexpr int NR = 2 * (NI + MJ);            // LDS operand reads per k-step
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
    copy_stage(sW0, sX0, sS0, 0);
    copy_stage(sW1, sX1, sS0, 1);
    copy_stage(sW2, sX2, sS0, 2);
    copy_stage(sW3, sX3, sS0, 3);
    wait_copies_upto<3 * CPS>();
    __syncthreads();
    read_frags(sW0, sX0, 0, 0);
    auto stage = [&](uint8_t* fW, uint8_t* fX, uint8_t* nW, uint8_t* nX, int s, int t) {
      wait_copies_upto<2 * CPS>();  // copies issued after stage s+1's: s+2, s+3
      stage_barrier();
      copy_stage(fW, fX, sS0, min(s + 4, KS - 1));
      mma(t);
      read_frags(nW, nX, 0, t ^ 1);
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
    auto stage = [&](uint8_t* cW, uint8_t* cX, float* cS, uint8_t* nW, uint8_t* nX, int s) {
      mma(0);
      read_frags(cW, cX, 1, 1);
      read_scales(cS);
      interleave<0, NM, NR + (BLK ? MJ + NI : 0), 0>();
      wait_copies_upto<(AHEAD - 2) * CPS>();  // stage s+1 has landed
      stage_barrier();
      copy_stage(cW, cX, cS, min(s + AHEAD, KS - 1));
      mma(1);
      apply_scales();
      read_frags(nW, nX, 0, 0);
      interleave<0, NM, NR, CPS>();
    };
    copy_stage(sW0, sX0, sS0, 0);
    copy_stage(sW1, sX1, sS1, 1);
    if constexpr (TRI) copy_stage(sW2, sX2, sS2, min(2, KS - 1));
    wait_copies_upto<(AHEAD - 1) * CPS>();
    __syncthreads();
    read_frags(sW0, sX0, 0, 0);
    if constexpr (TRI) {
      int s = 0;
      for (; s + 3 <= KS; s += 3) {
        stage(sW0, sX0, sS0, sW1, sX1, s);
        stage(sW1, sX1, sS1, sW2, sX2, s + 1);
        stage(sW2, sX2, sS2, sW0, sX0, s + 2);
      }
      if (s < KS) stage(sW0, sX0, sS0, sW1, sX1, s);
      if (s + 1 < KS) stage(sW1, sX1, sS1, sW2, sX2, s + 1);
    } else {
      for (int s = 0; s < KS; s += 2) {
        stage(sW0, sX0, sS0, sW1, sX1, s);
        stage(sW1, sX1, sS1, sW0, sX0, s + 1);
      }
    }
  }

  // ---- split-K: raw sums (int32 bit patterns for INT8) to the f32
  // workspace [ksplit][M][N]; the reduce kernel adds the slices in order and
  // runs the epilogue. A lane holds 4 consecutive weight rows of one token.
  if (p.ksplit > 1) {
    float* plane = p.partial + (int64_t)blockIdx.z * p.M * p.N;
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
      const int tr = wm * TM + j * 32 + rl;
      if (tr >= rows) continue;
      float* dst = plane + (int64_t)(row0 + tr) * p.N;
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int lr = wrow(i) + q * 8 + kh * 4;  // tile weight row of the quad
          int n;
          if (ACT) n = (lr < BN / 2 ? n0 + lr : p.N / 2 + n0 + (lr - BN / 2));
          else n = n0 + lr;
          const int nl = ACT ? (lr < BN / 2 ? n0 + lr : n0 + (lr - BN / 2)) : n;  // output column
          float v[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            if constexpr (INT) v[t] = __int_as_float(acc[i][j][q * 4 + t]);
            else v[t] = acc[i][j][q * 4 + t];
          }
          if (nl + 4 <= nlim && (p.N & 3) == 0) {
            *reinterpret_cast<float4*>(dst + n) = make_float4(v[0], v[1], v[2], v[3]);
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
              if (nl + t < nlim) dst[n + t] = v[t];
          }
        }
    }
    return;
  }

  // ---- epilogue ----
  // Every wavefront passed the last barrier after its final LDS operand read
  // and no copy is in flight. Per 32-token block j, each wavefront dumps its
  // f32 sums (4 consecutive weight rows of one token per register quad) into
  // a private LDS region [32 tokens][TN rows], float4 slot s of token row t at
  // s ^ (t & (TN/4 - 1)), then a rolled loop finishes 8 output channels per
  // lane (scales, bias, activation, routing weight) and stores 16 bytes. The
  // per-token and per-channel inputs come from LDS (staged here from the
  // registers loaded in the prologue), so the loop issues no global loads.
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
  constexpr int SLOTS = TN / 4;  // float4 slots per token row
  static_assert(32 * TN * 4 <= BN * 64, "a wavefront region fits a quarter of the weight stages");
  float* reg;
  if constexpr (KB == 64) reg = reinterpret_cast<float*>(wave == 0 ? sW0 : wave == 1 ? sW1 : wave == 2 ? sW2 : sW3);
  else reg = reinterpret_cast<float*>((wave < 2 ? sW0 : sW1) + (wave & 1) * (BN * 64));
  const bool has_bias = p.bias != nullptr;
  const bool vec_ok = ((p.ldy & 7) == 0) && ((reinterpret_cast<uintptr_t>(p.y) & 15) == 0);
  constexpr int CH = TNO / 8;  // 8-channel output chunks per token
  static_assert(64 % CH == 0, "a lane keeps its channel chunk across the finish loop");
  float cs_g[8], cs_u[8], cb_g[8], cb_u[8];
  {
    // tile weight row of this lane's first output channel (gate half with ACT)
    const int wr = (ACT ? wn * (TN / 2) : wn * TN) + (lane % CH) * 8;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      cs_g[k] = s_ws[wr + k];
      cb_g[k] = s_bs[wr + k];
      cs_u[k] = ACT ? s_ws[BN / 2 + wr + k] : 0.0f;
      cb_u[k] = ACT ? s_bs[BN / 2 + wr + k] : 0.0f;
    }
  }
#pragma unroll
  for (int j = 0; j < MJ; ++j) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int slot = (i * 32 + q * 8 + kh * 4) >> 2;
        float4 v;
        v.x = (float)acc[i][j][q * 4 + 0];
        v.y = (float)acc[i][j][q * 4 + 1];
        v.z = (float)acc[i][j][q * 4 + 2];
        v.w = (float)acc[i][j][q * 4 + 3];
        *reinterpret_cast<float4*>(reg + rl * TN + ((slot ^ (rl & (SLOTS - 1))) * 4)) = v;
      }
    // the wavefront reads back only its own region: LDS is in order per
    // wavefront. 64 % CH == 0, so a lane always finishes the same 8 channels
    // (c = lane % CH): their scales and biases are loaded once per tile.
    for (int e = lane; e < 32 * CH; e += 64) {
      const int t = e / CH, c = e % CH;
      const int tr = wm * TM + j * 32 + t;   // token within the tile
      const int nb = n0 + wn * TNO + c * 8;  // first global output channel
      if (tr >= rows || nb >= nlim) continue;
      const float sxa = s_sx[tr];
      const float rwt = s_rw[tr];
      const int sw = t & (SLOTS - 1);
      const float* rowp = reg + t * TN;
      const int s0 = c * 2;  // float4 slot of local weight row c * 8
      const float4 g0 = *reinterpret_cast<const float4*>(rowp + ((s0 ^ sw) * 4));
      const float4 g1 = *reinterpret_cast<const float4*>(rowp + (((s0 + 1) ^ sw) * 4));
      const float vg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
      float vu[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (ACT) {
        const int s1 = s0 + SLOTS / 2;  // matching up row: TN/2 rows later
        const float4 u0 = *reinterpret_cast<const float4*>(rowp + ((s1 ^ sw) * 4));
        const float4 u1 = *reinterpret_cast<const float4*>(rowp + (((s1 + 1) ^ sw) * 4));
        vu[0] = u0.x; vu[1] = u0.y; vu[2] = u0.z; vu[3] = u0.w;
        vu[4] = u1.x; vu[5] = u1.y; vu[6] = u1.z; vu[7] = u1.w;
      }
      uint32_t packed[4];
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        float o2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float v = vg[k + h] * sxa;
          v = v * cs_g[k + h];
          if (has_bias) v += cb_g[k + h];
          if (ACT) {
            float u = vu[k + h] * sxa;
            u = u * cs_u[k + h];
            if (has_bias) u += cb_u[k + h];
            v = qmoe_act(p.act, v, u, p.act_p0, p.act_p1);
          }
          o2[h] = v * rwt;
        }
        packed[k / 2] = (uint32_t)f32_to_bf16(o2[0]) | ((uint32_t)f32_to_bf16(o2[1]) << 16);
      }
      const int64_t yr = s_yr[tr];
      uint16_t* dst = p.y + yr * p.ldy + nb;
      if (vec_ok && nb + 8 <= nlim) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
      } else {
        for (int k = 0; k < 8 && nb + k < nlim; ++k)
          dst[k] = (uint16_t)(packed[k / 2] >> ((k & 1) * 16));
      }
    }
  }
}

// Split-K finish for the tiled kernel: one lane = 8 consecutive output
// channels of one compact row; a wavefront covers 512 channels of a row, a
// workgroup 4 rows. The slices are added in slice order (deterministic),
// then scales, bias, activation and routing weight are applied as in the
// single-pass epilogue. A grouped problem finds the row's group by binary
// search over group_offs.
template <bool INT, bool ACT, bool BLK>
__global__ __launch_bounds__(kThreads) void f8_splitk_finish_kernel(const GemmParams p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int R = blockIdx.y * 4 + wave;
  if (R >= p.M) return;
  const int nlim = ACT ? p.N / 2 : p.N;
  const int c0 = (blockIdx.x * 64 + lane) * 8;
  if (c0 >= nlim) return;
  int g = 0;
  if (p.group_offs) {
    int lo = 0, hi = p.slots;  // group_offs[lo] <= R < group_offs[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (p.group_offs[mid] <= R) lo = mid;
      else hi = mid;
    }
    g = lo;
  }
  const int ar = p.a_rows ? p.a_rows[R] : R;
  // block-scaled partials already carry their scales
  const float sxa = BLK ? 1.0f : p.a_scale[(int64_t)ar * p.lds_a];
  const float rwt = p.row_weight ? bf16_to_f32(p.row_weight[R]) : 1.0f;
  const float* wsc = static_cast<const float*>(p.w_scale) + (int64_t)g * p.ws_gstride;
  const float* bias = p.bias ? p.bias + (int64_t)g * p.bias_gstride : nullptr;
  const int64_t plane = (int64_t)p.M * p.N;
  const float* src = p.partial + (int64_t)R * p.N;
  const bool vec = (p.N & 3) == 0 && c0 + 8 <= nlim;
  float vg[8], vu[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) vg[k] = vu[k] = 0.0f;
  int ig[8], iu[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) ig[k] = iu[k] = 0;
  for (int j = 0; j < p.ksplit; ++j) {
    const float* sj = src + j * plane;
    float a[8], b[8];
    if (vec) {
      const float4 a0 = *reinterpret_cast<const float4*>(sj + c0);
      const float4 a1 = *reinterpret_cast<const float4*>(sj + c0 + 4);
      a[0] = a0.x; a[1] = a0.y; a[2] = a0.z; a[3] = a0.w; a[4] = a1.x; a[5] = a1.y; a[6] = a1.z; a[7] = a1.w;
      if (ACT) {
        const float4 b0 = *reinterpret_cast<const float4*>(sj + p.N / 2 + c0);
        const float4 b1 = *reinterpret_cast<const float4*>(sj + p.N / 2 + c0 + 4);
        b[0] = b0.x; b[1] = b0.y; b[2] = b0.z; b[3] = b0.w; b[4] = b1.x; b[5] = b1.y; b[6] = b1.z; b[7] = b1.w;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int c = min(c0 + k, nlim - 1);
        a[k] = sj[c];
        b[k] = ACT ? sj[p.N / 2 + c] : 0.0f;
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if constexpr (INT) {
        ig[k] += __float_as_int(a[k]);
        if (ACT) iu[k] += __float_as_int(b[k]);
      } else {
        vg[k] += a[k];
        if (ACT) vu[k] += b[k];
      }
    }
  }
  uint32_t packed[4];
#pragma unroll
  for (int k = 0; k < 8; k += 2) {
    float o2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int n = min(c0 + k + h, nlim - 1);
      float v = INT ? (float)ig[k + h] : vg[k + h];
      v = v * sxa;
      if (!BLK) v = v * wsc[n];
      if (bias) v += bias[n];
      if (ACT) {
        float u = INT ? (float)iu[k + h] : vu[k + h];
        u = u * sxa;
        if (!BLK) u = u * wsc[p.N / 2 + n];
        if (bias) u += bias[p.N / 2 + n];
        v = qmoe_act(p.act, v, u, p.act_p0, p.act_p1);
      }
      o2[h] = v * rwt;
    }
    packed[k / 2] = (uint32_t)f32_to_bf16(o2[0]) | ((uint32_t)f32_to_bf16(o2[1]) << 16);
  }
  const int64_t yr = p.y_rows ? p.y_rows[R] : R;
  uint16_t* dst = p.y + yr * p.ldy + c0;
  if (c0 + 8 <= nlim && ((p.ldy & 7) == 0) && ((reinterpret_cast<uintptr_t>(p.y) & 15) == 0)) {
    *reinterpret_cast<uint4*>(dst) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  } else {
    for (int k = 0; k < 8 && c0 + k < nlim; ++k) dst[k] = (uint16_t)(packed[k / 2] >> ((k & 1) * 16));
  }
}

template <bool INT, int BM, int BN, bool ACT, bool BLK>
void f8_launch_shape(const GemmParams& p, hipStream_t st) {
  const char* env = getenv("QMOE_F8_KB");  // tuning knob: K bytes per LDS stage
  const int kb = BLK ? 128 : (env ? atoi(env) : 128);
  auto kern = kb == 64 ? f8_gemm_kernel<INT, BM, BN, ACT, BLK ? 128 : 64, BLK>
                       : f8_gemm_kernel<INT, BM, BN, ACT, 128, BLK>;
  const int nout = ACT ? p.N / 2 : p.N;
  const int n_tiles = cdiv(nout, ACT ? BN / 2 : BN);
  const unsigned ks = (unsigned)std::max(1, p.ksplit);
  if (p.group_offs) {
    const int m_tiles = cdiv(p.M, BM) + std::min(p.slots, p.M);
    hipLaunchKernelGGL(kern, dim3(n_tiles, m_tiles, ks), dim3(kThreads), 0, st, p, m_tiles, n_tiles);
  } else {
    const int m_tiles = cdiv(p.M, BM);
    const int grid = cdiv(m_tiles * n_tiles, kXcds) * kXcds;
    hipLaunchKernelGGL(kern, dim3(grid, 1, ks), dim3(kThreads), 0, st, p, m_tiles, n_tiles);
  }
}

template <bool INT, int BM, int BN, bool BLK>
void f8_launch_act(const GemmParams& p, hipStream_t st) {
  if (p.act != QA_NONE) f8_launch_shape<INT, BM, BN, true, BLK>(p, st);
  else f8_launch_shape<INT, BM, BN, false, BLK>(p, st);
}

template <bool INT>
void f8_launch_bm(const GemmParams& p, int bm, hipStream_t st) {
  switch (bm) {
    case 256: f8_launch_act<INT, 256, 256, false>(p, st); break;
    case 128: f8_launch_act<INT, 128, 256, false>(p, st); break;
    case 64: f8_launch_act<INT, 64, 256, false>(p, st); break;
    default: f8_launch_act<INT, 32, 256, false>(p, st); break;
  }
}

// block-scaled FP8: tiles of at most 128 tokens (the per-block sums need a
// second accumulator set)
void f8_launch_bm_blk(const GemmParams& p, int bm, hipStream_t st) {
  switch (bm) {
    case 128: f8_launch_act<false, 128, 256, true>(p, st); break;
    case 64: f8_launch_act<false, 64, 256, true>(p, st); break;
    default: f8_launch_act<false, 32, 256, true>(p, st); break;
  }
}

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
    const int avg = std::max(1, p.M / std::max(1, std::min(p.slots, p.M)));
    if (avg > 192) return 256;
    if (avg > 96) return 128;
    if (avg > 48) return 64;
    return 32;
  }
  for (int bm : {256, 128, 64}) {
    if ((int64_t)cdiv(p.M, bm) * n_tiles >= 200) return bm;
  }
  return 32;
}

// Whether this kernel takes the problem (K % 256, 16-byte alignment,
// weights < 4 GiB per group), and its plan: token-tile height, K split and
// the f32 workspace the split needs ([ksplit][M][N]).
bool qmoe_f8_plan(const GemmParams& p, bool blk, int* bm_out, int* ksplit_out, int64_t* ws_bytes) {
  if (p.M <= 0 || p.K <= 0 || (p.K % 256) != 0 || p.N <= 0) return false;
  if (p.act != QA_NONE && (p.N % 2) != 0) return false;
  // block scales: 128-row weight blocks aligned with the tile's halves
  if (blk && (p.ws_bn != 128 || (p.act != QA_NONE && ((p.N / 2) % 128) != 0))) return false;
  if ((p.lda % 16) != 0 || (p.ldw % 16) != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.a) & 15) || (reinterpret_cast<uintptr_t>(p.w) & 15) ||
      (p.w_gstride % 16) != 0)
    return false;
  if ((int64_t)p.ldw * p.N >= ((int64_t)1 << 32)) return false;
  int bm = f8_pick_bm_any(p);
  if (blk && !getenv("QMOE_F8_BM")) {
    // block-scaled tiles hold at most 128 tokens; measured on MI355X (K 7168,
    // N 18432): 128-token tiles up to 256 and from 2048 tokens, 64 between
    bm = p.group_offs ? std::min(bm, 128) : (p.M > 256 && p.M < 2048 ? 64 : 128);
  }
  const int m_tiles = p.group_offs ? cdiv(p.M, bm) + std::min(p.slots, p.M) : cdiv(p.M, bm);
  if (p.group_offs && m_tiles > 65535) return false;
  // Dense problems whose largest CU-filling tile is small (tall-K, few
  // tokens) are split over K, with the tile and split that measured best on
  // MI355X: (32 rows, 4 slices) up to 256 tokens, (128, 4) up to 512,
  // (128, 2) above.
  int ksplit = 1;
  const bool env_bm = getenv("QMOE_F8_BM") != nullptr;
  if (!p.group_offs && bm <= 64 && p.K >= 8192 && !env_bm) {
    if (p.M <= 256) { bm = 32; ksplit = 4; }
    else if (p.M <= 512) { bm = 128; ksplit = 4; }
    else { bm = 128; ksplit = 2; }
  }
  const char* env = getenv("QMOE_F8_KSPLIT");  // tuning knob
  if (env && atoi(env) > 0) ksplit = std::max(1, std::min(atoi(env), p.K / 256));
  *bm_out = bm;
  *ksplit_out = ksplit;
  *ws_bytes = ksplit > 1 ? (int64_t)ksplit * p.M * p.N * 4 : 0;
  return true;
}

// Launch per the plan (the caller checked qmoe_f8_plan and sized the
// workspace); with a K split the reduce kernel finishes the epilogue.
int qmoe_f8_launch(GemmParams p, bool blk, void* workspace, int64_t ws_bytes, hipStream_t st) {
  int bm = 0, ksplit = 1;
  int64_t need = 0;
  if (!qmoe_f8_plan(p, blk, &bm, &ksplit, &need)) return QMOE_ERR_ARG;
  p.ksplit = ksplit;
  if (ksplit > 1) {
    if (!workspace || ws_bytes < need) return QMOE_ERR_WORKSPACE;
    p.partial = static_cast<float*>(workspace);
  }
  if (blk) f8_launch_bm_blk(p, bm, st);
  else if (p.wfmt == 1) f8_launch_bm<true>(p, bm, st);
  else f8_launch_bm<false>(p, bm, st);
  if (ksplit > 1) {
    const int nout = p.act != QA_NONE ? p.N / 2 : p.N;
    const dim3 rg((unsigned)cdiv(nout, 512), (unsigned)cdiv(p.M, 4), 1);
    const bool act = p.act != QA_NONE;
    if (blk) {
      if (act) hipLaunchKernelGGL((f8_splitk_finish_kernel<false, true, true>), rg, dim3(kThreads), 0, st, p);
      else hipLaunchKernelGGL((f8_splitk_finish_kernel<false, false, true>), rg, dim3(kThreads), 0, st, p);
    } else if (p.wfmt == 1) {
      if (act) hipLaunchKernelGGL((f8_splitk_finish_kernel<true, true, false>), rg, dim3(kThreads), 0, st, p);
      else hipLaunchKernelGGL((f8_splitk_finish_kernel<true, false, false>), rg, dim3(kThreads), 0, st, p);
    } else {
      if (act) hipLaunchKernelGGL((f8_splitk_finish_kernel<false, true, false>), rg, dim3(kThreads), 0, st, p);
      else hipLaunchKernelGGL((f8_splitk_finish_kernel<false, false, false>), rg, dim3(kThreads), 0, st, p);
    }
  }
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
