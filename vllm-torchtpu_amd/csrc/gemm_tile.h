// Shared machinery of the tiled (prefill) GEMM kernels -- 1-byte x 1-byte
// in gemm_f8.hip, bf16 x e2m1 in gemm_w4.hip: 4-wavefront workgroups fed by
// direct global->LDS copies with explicit vector-memory waits, tile
// enumeration (XCD-aware dense order, grouped m-tiles), the output tile
// layout of 32x32 MFMA blocks (weight rows x tokens) with its LDS-staged
// epilogue, and the split-K finishing kernel.
#pragma once

#include "gemm_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kXcds = 8;
constexpr int kGroupM = 8;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

#define QMOE_LDS(p) ((__attribute__((address_space(3))) void*)(p))

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

// Wait until at most N of this wavefront's vector-memory operations (here:
// LDS copies) are outstanding; expcnt and lgkmcnt are left alone. A
// workgroup barrier alone does not wait for them: the compiler orders only
// ordinary global accesses at workgroup scope, and an LDS copy's data is in
// LDS only once its vector-memory count retires (they retire in order).
template <int N>
__device__ __forceinline__ void wait_copies_upto() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int BM>
__device__ __forceinline__ bool tile_group(const GemmParams& p, int y, int& g, int& row0, int& rows,
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

__device__ __forceinline__ bool tile_dense(int b, int m_tiles, int n_tiles, int& mt, int& nt) {
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

// Dense tile of a persistent grid in plain order, channel tiles fastest:
// the tiles in flight at once then cover the whole width of the output
// rows. For rows whose byte stride is a multiple of 32 KB, the XCD runs of
// tile_dense put every in-flight store on the few column ranges of a few
// channel tiles, which maps them to few HBM channels (measured on MI355X,
// 4096 tokens, FP8: K 512, N 32768 178 -> 106 us; K 1024, N 16384 108 ->
// 77 us; 8 KB rows lose 2-7 % with it: the weight tiles leave the L2).
__device__ __forceinline__ bool tile_wide(int b, int m_tiles, int n_tiles, int& mt, int& nt) {
  if (b >= m_tiles * n_tiles) return false;
  mt = b / n_tiles;
  nt = b % n_tiles;
  return true;
}

// ---- output tile of 32x32 MFMA blocks ----
// The wavefronts form a WN x WM grid; wavefront (wn, wm) owns NI 32-row weight
// blocks (LDS rows wrow(i)) and MJ 32-token blocks (tile tokens wm*TM +
// j*32 + ...). Block (i, j) is an MFMA D matrix with weight rows down and
// tokens across: lane l, register r holds weight row 8*(r/4) + 4*(l/32) +
// (r%4) of the block and token l % 32, so a register quad q holds 4
// consecutive weight rows (q*8 + 4*(l/32) + 0..3) of one token. With a fused
// activation the tile's LDS rows [0, BN/2) are gate rows and [BN/2, BN) the
// matching up rows; a wavefront's gate blocks are i < NI/2.
template <int BN, int TN, int NI, bool ACT>
__device__ __forceinline__ int tile_wrow(int wn, int i) {
  if (ACT) return (i < NI / 2 ? 0 : BN / 2) + wn * (TN / 2) + (i % (NI / 2)) * 32;
  return wn * TN + i * 32;
}

// Split-K: raw sums (int32 bit patterns for INT8) to the f32 workspace
// [ksplit][M][N]; the finishing kernel adds the slices in order and runs the
// epilogue. A lane holds 4 consecutive weight rows of one token.
template <int BN, int TN, int TM, int NI, int MJ, bool ACT, bool INT, typename AccT>
__device__ __forceinline__ void tile_store_partials(const GemmParams& p, const AccT (&acc)[NI][MJ], int row0,
                                                    int rows, int n0, int nlim, int wn, int wm, int lane) {
  const int rl = lane & 31, kh = lane >> 5;
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
        const int lr = tile_wrow<BN, TN, NI, ACT>(wn, i) + q * 8 + kh * 4;  // tile weight row of the quad
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
}

// Epilogue. Every wavefront has passed the last barrier after its final LDS
// operand read and no copy is in flight; the per-token inputs (activation
// scale, routing weight, output row) and per-weight-row inputs (scale, bias)
// of the tile are staged in LDS. Per 32-token block j, each wavefront dumps
// its f32 sums (register quads) into its private LDS region `reg` [32
// tokens][TN rows], float4 slot s of token row t at s ^ (t & (TN/4 - 1)),
// then a rolled loop finishes 8 output channels per lane (scales, bias,
// activation, routing weight) and stores 16 bytes, so the loop issues no
// global loads.
template <int BN, int TN, int TM, int NI, int MJ, bool ACT, typename AccT>
__device__ __forceinline__ void tile_epilogue(const GemmParams& p, const AccT (&acc)[NI][MJ], float* reg,
                                              const float* s_sx, const float* s_rw, const int* s_yr,
                                              const float* s_ws, const float* s_bs, int n0, int nlim,
                                              int rows, int wn, int wm, int lane) {
  const int rl = lane & 31, kh = lane >> 5;
  constexpr int TNO = ACT ? TN / 2 : TN;  // output channels per wavefront
  constexpr int SLOTS = TN / 4;           // float4 slots per token row
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
// SC: which scales the finish applies -- kScAll (per-row activation and
// per-channel weight scales), kScNone (the partials carry every scale:
// block-scaled FP8, e2m1) or kScWeight (block activation scales are in the
// partials, the per-channel weight scale is not: the grouped-matmul recipe).
enum { kScAll = 0, kScNone = 1, kScWeight = 2 };

template <bool INT, bool ACT, int SC>
__global__ __launch_bounds__(kThreads) void tile_splitk_finish_kernel(const GemmParams p) {
  constexpr bool SCALED = SC == kScNone;
  constexpr bool ASCALE = SC == kScAll;
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
  const float sxa = ASCALE ? p.a_scale[(int64_t)ar * p.lds_a] : 1.0f;
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
      if (!SCALED) v = v * wsc[n];
      if (bias) v += bias[n];
      if (ACT) {
        float u = INT ? (float)iu[k + h] : vu[k + h];
        u = u * sxa;
        if (!SCALED) u = u * wsc[p.N / 2 + n];
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

}  // namespace
