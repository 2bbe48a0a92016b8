// Tiled (prefill) grouped GEMM: LDS-staged, double-buffered MFMA tiles.
//
// Workgroup = 256 threads (2x2 wavefronts) owning a BM x BN output tile;
// each wavefront owns (BM/2) x (BN/2) = MF x NF MFMA 16x16 tiles (128 x 128
// for the 256 x 256 tile: every 2 KB fragment read from LDS feeds 8 MFMAs,
// which keeps LDS reads at about half the MFMA time). K advances in stages
// of 128 bytes per row (128 e4m3/int8 values, 64 bf16 values):
//  1. every thread issues the global loads of stage s+1 into registers
//     (16-byte loads; 8 threads cover a 128-byte row, so rows are read with
//     full coalescing) -- e2m1 / e4m3 weights of the bf16-activation kinds
//     are expanded to bf16 on the way into LDS, once per element per tile;
//  2. the wavefronts run stage s out of LDS: lane l reads 32 bytes at column
//     32*(l>>4) of row (l & 15) of each A and B fragment (2 x ds_read_b128)
//     and issues MF*NF MFMA groups (one 16x16x128 f8f6f4, two 16x16x64 i8 or
//     two 16x16x32 bf16 per fragment pair);
//  3. registers -> the other LDS buffer (free since the last barrier),
//     barrier.
// LDS rows are padded to 144 bytes: 16 lanes reading 16 consecutive rows at
// one column hit 16 disjoint 4-bank groups of the 64 banks.
// The epilogue applies scales / bias / activation / routing weight in
// registers, stages the bf16 tile in LDS and writes whole rows with 16-byte
// stores.
//
// Tile order: a dense GEMM runs a 1-D grid; consecutive workgroups are dealt
// round-robin to the 8 XCDs, so the block index is remapped to give each XCD
// a contiguous run of tiles that share a weight (B) column block, which its
// L2 then serves to all of them. A grouped GEMM enumerates the m-tiles of all
// groups in order (ceil(rows_g / BM) per group) on grid.y; a wavefront-wide
// scan of the group sizes maps y to (group, m-tile). Rows past a group's end
// and weight rows past N load as zeros and are not stored.
// A fused activation pairs gate rows [n0, n0+BN/2) with up rows
// [N/2+n0, ...): in a wavefront, fragment j < NF/2 is gate and j + NF/2 the
// matching up fragment, so the epilogue combines them in registers.

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "gemm_common.h"

extern __shared__ __align__(16) uint8_t qmoe_tiled_smem[];

namespace {

constexpr int kThreads = 256;
constexpr int kRowBytes = 128;  // K bytes per row per stage
constexpr int kPitch = 144;     // padded LDS row pitch
constexpr int kXcds = 8;

template <int KIND, int WF>
struct TTraits {
  static constexpr bool kAbf16 = KIND == QK_W8A16_PC || KIND == QK_W4A16_MX || KIND == QK_W16A16 ||
                                 KIND == QK_W8A16_BLK;
  static constexpr bool kInt = KIND == QK_W8A8_PC && WF == 1;
  static constexpr int kKPerStage = kAbf16 ? 64 : 128;
  // bytes of one weight row per stage in HBM
  static constexpr int kWRowBytes =
      KIND == QK_W4A16_MX ? 32 : (KIND == QK_W8A16_PC || KIND == QK_W8A16_BLK ? 64 : 128);
};

template <int BM, int BN, bool ACT>
constexpr size_t tiled_smem_bytes() {
  const size_t pipe = 2 * (BM + BN) * kPitch + 2 * (BM + BN) * sizeof(float);
  const size_t out = (size_t)BM * ((ACT ? BN / 2 : BN) * 2 + 16);
  return pipe > out ? pipe : out;
}

__device__ __forceinline__ i32x8 pack8(uint4 a, uint4 b) {
  i32x8 r;
  r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
  r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
  return r;
}

__device__ __forceinline__ i32x4 as_i4(uint4 u) {
  i32x4 r;
  r[0] = u.x; r[1] = u.y; r[2] = u.z; r[3] = u.w;
  return r;
}

__device__ __forceinline__ bf16x8 as_b8(uint4 u) {
  union { uint4 u; bf16x8 b; } c;
  c.u = u;
  return c.b;
}

__device__ __forceinline__ uint4 fp4x8_bf16(uint32_t d, float scale) {
  bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 0);
  bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 1);
  bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 2);
  bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 3);
  union { bf16x2 b; uint32_t u; } c0, c1, c2, c3;
  c0.b = p0; c1.b = p1; c2.b = p2; c3.b = p3;
  return make_uint4(c0.u, c1.u, c2.u, c3.u);
}

// e4m3 codes times a bf16-valued scale, each product rounded to bf16 once
// (exact in f32: a 4-bit by 8-bit significand product)
__device__ __forceinline__ uint2 fp8x4_bf16_scaled(uint32_t d, float s) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, false);
  const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, true);
  union { bf16x2 h; uint32_t u; } a, b;
  a.h = __builtin_convertvector(f32x2{lo[0] * s, lo[1] * s}, bf16x2);
  b.h = __builtin_convertvector(f32x2{hi[0] * s, hi[1] * s}, bf16x2);
  return make_uint2(a.u, b.u);
}

__device__ __forceinline__ uint2 fp8x4_bf16(uint32_t d) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, false);
  v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, true);
  return make_uint2((f32_bits(lo[0]) >> 16) | (f32_bits(lo[1]) & 0xffff0000u),
                    (f32_bits(hi[0]) >> 16) | (f32_bits(hi[1]) & 0xffff0000u));
}

// Map a grouped workgroup's y index to (group, first compact row, rows in
// tile). Returns false if y is past the last tile.
template <int BM>
__device__ __forceinline__ bool map_group_tile(const GemmParams& p, int y, int& g, int& row0, int& rows,
                                               int* s_info) {
  const int G = p.slots;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int done = 0;  // tiles of groups already passed
    int found = -1, fr0 = 0, frows = 0;
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
        int v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
      }
      const int excl = done + incl - nt;
      const bool mine = gg < G && y >= excl && y < excl + nt;
      const uint64_t bal = __ballot(mine);
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

// Dense tile of a 1-D grid, XCD-aware: workgroup b runs on XCD b % 8, and
// the 8 XCDs each take one contiguous run of the tile order. The order walks
// groups of kGroupM m-tiles column by column (n-tile after n-tile), so the
// ~64 workgroups an XCD runs at once cover about 8 m-tiles x 8 n-tiles:
// each A row block and each weight column block fetched into that XCD's L2
// is then shared by ~8 tiles instead of being re-fetched per tile.
constexpr int kGroupM = 8;

__device__ __forceinline__ bool map_dense_tile(int b, int m_tiles, int n_tiles, int& mt, int& nt) {
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

template <int KIND, int WF, int BM, int BN, bool ACT>
__global__ __launch_bounds__(kThreads) void tiled_gemm_kernel(const GemmParams p, int m_tiles, int n_tiles) {
  using Tr = TTraits<KIND, WF>;
  constexpr int MF = BM / 32;  // 16-row fragments per wavefront (2x2 waves)
  constexpr int NF = BN / 32;
  constexpr int A_CH = BM * 8 / kThreads;                    // 16-byte chunks per thread (A)
  constexpr int W_CH = BN * Tr::kWRowBytes / 16 / kThreads;  // 16-byte global chunks (W)
  constexpr int BNO = ACT ? BN / 2 : BN;                     // output columns of the tile
  static_assert(A_CH >= 1 && W_CH >= 1, "tile too small");
  static_assert(BM + BN <= 2 * kThreads, "block-scale staging holds two scales per thread");

  uint8_t* smem = qmoe_tiled_smem;
  auto sA = [&](int b) { return smem + b * (BM * kPitch); };
  auto sB = [&](int b) { return smem + 2 * BM * kPitch + b * (BN * kPitch); };
  float* sSc = reinterpret_cast<float*>(smem + 2 * (BM + BN) * kPitch);  // [2][BM + BN]
  __shared__ int s_info[4];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int col = lane & 15, kg = lane >> 4;

  int g, row0, rows, ntile;
  if (p.group_offs) {
    if (!map_group_tile<BM>(p, blockIdx.y, g, row0, rows, s_info)) return;
    ntile = blockIdx.x;
  } else {
    int mt;
    if (!map_dense_tile(blockIdx.x, m_tiles, n_tiles, mt, ntile)) return;
    g = 0;
    row0 = mt * BM;
    rows = min(BM, p.M - row0);
  }

  const int n0 = ntile * BNO;
  const int nlim = ACT ? p.N / 2 : p.N;
  const uint8_t* wg = p.w + (int64_t)g * p.w_gstride;
  const uint8_t* abase = static_cast<const uint8_t*>(p.a);
  const int64_t lda_b = p.lda * (Tr::kAbf16 ? 2 : 1);

  // per-thread source rows for the global loads
  int64_t a_off[A_CH];
  bool a_ok[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int c = tid + i * kThreads;
    const int r = c >> 3;
    a_ok[i] = r < rows;
    const int R = row0 + (a_ok[i] ? r : 0);
    const int ar = p.a_rows ? p.a_rows[R] : R;
    a_off[i] = (int64_t)ar * lda_b + (c & 7) * 16;
  }
  // weight rows: tile row tr -> weight row
  constexpr int W_PER_ROW = Tr::kWRowBytes / 16;  // 16-byte chunks per weight row per stage
  int w_row[W_CH];
  bool w_ok[W_CH];
#pragma unroll
  for (int i = 0; i < W_CH; ++i) {
    const int c = tid + i * kThreads;
    const int tr = c / W_PER_ROW;
    int n;
    bool ok;
    if (ACT) {
      const int half = BN / 2;
      const int cidx = n0 + (tr % half);
      ok = cidx < nlim;
      n = (tr < half ? 0 : p.N / 2) + cidx;
    } else {
      n = n0 + tr;
      ok = n < nlim;
    }
    w_ok[i] = ok;
    w_row[i] = ok ? n : 0;
  }

  // K stages [ks0, ks1): all of them, or slice blockIdx.z of a K split
  // (dense, no fused activation: the slices' f32 sums go to the partials)
  const int ks_all = p.K / Tr::kKPerStage;
  const int ks0 = (int)((int64_t)blockIdx.z * ks_all / gridDim.z);
  const int ks1 = (int)((int64_t)(blockIdx.z + 1) * ks_all / gridDim.z);

  uint4 ra[A_CH];
  uint4 rw[W_CH];
  float rsc[2] = {0.0f, 0.0f};  // block-scale staging

  auto gload = [&](int ks) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i)
      ra[i] = a_ok[i] ? *reinterpret_cast<const uint4*>(abase + a_off[i] + (int64_t)ks * kRowBytes)
                      : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < W_CH; ++i) {
      const int c = tid + i * kThreads;
      const int64_t off = (int64_t)w_row[i] * p.ldw + (int64_t)ks * Tr::kWRowBytes + (c % W_PER_ROW) * 16;
      rw[i] = w_ok[i] ? *reinterpret_cast<const uint4*>(wg + off) : make_uint4(0, 0, 0, 0);
    }
    if constexpr (KIND == QK_W8A8_BLK) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int idx = tid + h * kThreads;
        if (idx < BM) {
          const int R = row0 + (idx < rows ? idx : 0);
          const int ar = p.a_rows ? p.a_rows[R] : R;
          rsc[h] = p.a_scale[(int64_t)ar * p.lds_a + (ks >> p.a_kshift)];
        } else if (idx < BM + BN) {
          const int tr = idx - BM;
          int n;
          if (ACT) {
            const int half = BN / 2;
            const int cidx = min(n0 + (tr % half), nlim - 1);
            n = (tr < half ? 0 : p.N / 2) + cidx;
          } else {
            n = min(n0 + tr, nlim - 1);
          }
          rsc[h] = static_cast<const float*>(p.w_scale)[(int64_t)g * p.ws_gstride +
                                                        (int64_t)(n / p.ws_bn) * p.ldws + (ks >> p.w_kshift)];
        }
      }
    }
  };

  auto sstore = [&](int buf, int ks) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<uint4*>(sA(buf) + (c >> 3) * kPitch + (c & 7) * 16) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < W_CH; ++i) {
      const int c = tid + i * kThreads;
      const int tr = c / W_PER_ROW;
      const int cc = c % W_PER_ROW;
      uint8_t* dst = sB(buf) + tr * kPitch;
      if constexpr (KIND == QK_W4A16_MX) {
        // 32 e2m1 codes = k [ks*64 + cc*32, +32): one e8m0 block
        const uint8_t* sp = static_cast<const uint8_t*>(p.w_scale) + (int64_t)g * p.ws_gstride +
                            (int64_t)w_row[i] * p.ldws + ks * 2 + cc;
        const float scl = e8m0_to_f32(*sp);
        uint4* d = reinterpret_cast<uint4*>(dst + cc * 64);
        d[0] = fp4x8_bf16(rw[i].x, scl);
        d[1] = fp4x8_bf16(rw[i].y, scl);
        d[2] = fp4x8_bf16(rw[i].z, scl);
        d[3] = fp4x8_bf16(rw[i].w, scl);
      } else if constexpr (KIND == QK_W8A16_PC) {
        uint4* d = reinterpret_cast<uint4*>(dst + cc * 32);
        const uint2 a0 = fp8x4_bf16(rw[i].x), a1 = fp8x4_bf16(rw[i].y);
        const uint2 a2 = fp8x4_bf16(rw[i].z), a3 = fp8x4_bf16(rw[i].w);
        d[0] = make_uint4(a0.x, a0.y, a1.x, a1.y);
        d[1] = make_uint4(a2.x, a2.y, a3.x, a3.y);
      } else if constexpr (KIND == QK_W8A16_BLK) {
        // the stage's 64 k lie in 128-k block ks >> 1 (scale rounded to bf16)
        const float scl = bf16_round(static_cast<const float*>(p.w_scale)[
            (int64_t)g * p.ws_gstride + (int64_t)(w_row[i] / p.ws_bn) * p.ldws + ((ks >> 1) >> p.w_kshift)]);
        uint4* d = reinterpret_cast<uint4*>(dst + cc * 32);
        const uint2 a0 = fp8x4_bf16_scaled(rw[i].x, scl), a1 = fp8x4_bf16_scaled(rw[i].y, scl);
        const uint2 a2 = fp8x4_bf16_scaled(rw[i].z, scl), a3 = fp8x4_bf16_scaled(rw[i].w, scl);
        d[0] = make_uint4(a0.x, a0.y, a1.x, a1.y);
        d[1] = make_uint4(a2.x, a2.y, a3.x, a3.y);
      } else {
        *reinterpret_cast<uint4*>(dst + cc * 16) = rw[i];
      }
    }
    if constexpr (KIND == QK_W8A8_BLK) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
        if (tid + h * kThreads < BM + BN) sSc[buf * (BM + BN) + tid + h * kThreads] = rsc[h];
    }
    (void)ks;
  };

  // LDS row of B fragment j of this wavefront
  auto b_row = [&](int j) {
    if (ACT) {
      constexpr int half = NF / 2;
      return (j < half ? 0 : BN / 2) + wn * (BN / 4) + (j % half) * 16 + col;
    }
    return wn * (BN / 2) + j * 16 + col;
  };

  using AccT = typename std::conditional<Tr::kInt, i32x4, f32x4>::type;
  AccT acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) acc[i][j] = AccT{0, 0, 0, 0};

  if (ks1 > ks0) {
    gload(ks0);
    sstore(0, ks0);
  }
  __syncthreads();

  for (int ks = ks0; ks < ks1; ++ks) {
    const int buf = (ks - ks0) & 1;
    if (ks + 1 < ks1) gload(ks + 1);

    const uint8_t* A = sA(buf);
    const uint8_t* Bt = sB(buf);
    uint4 bfr[NF][2];
#pragma unroll
    for (int j = 0; j < NF; ++j) {
      const uint4* src = reinterpret_cast<const uint4*>(Bt + b_row(j) * kPitch + kg * 32);
      bfr[j][0] = src[0];
      bfr[j][1] = src[1];
    }
    float sbv[NF];
    if constexpr (KIND == QK_W8A8_BLK) {
      const float* sc = sSc + buf * (BM + BN) + BM;
#pragma unroll
      for (int j = 0; j < NF; ++j) sbv[j] = sc[b_row(j)];
    }
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      const int ar = wm * (BM / 2) + i * 16;
      const uint4* src = reinterpret_cast<const uint4*>(A + (ar + col) * kPitch + kg * 32);
      const uint4 a0 = src[0], a1 = src[1];
      if constexpr (KIND == QK_W8A8_PC && WF == 0) {
        const i32x8 av = pack8(a0, a1);
#pragma unroll
        for (int j = 0; j < NF; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, pack8(bfr[j][0], bfr[j][1]),
                                                                       acc[i][j], 0, 0, 0, 127, 0, 127);
      } else if constexpr (KIND == QK_W8A8_PC && WF == 1) {
        // both 64-k halves of every fragment pair, the second NF MFMAs after
        // the first (no MFMA waits on the one before it)
#pragma unroll
        for (int j = 0; j < NF; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i4(a0), as_i4(bfr[j][0]), acc[i][j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < NF; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i4(a1), as_i4(bfr[j][1]), acc[i][j], 0, 0, 0);
      } else if constexpr (KIND == QK_W8A8_BLK) {
        const i32x8 av = pack8(a0, a1);
        const float* sc = sSc + buf * (BM + BN);
        float sa[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sa[r] = sc[ar + kg * 4 + r];
#pragma unroll
        for (int j = 0; j < NF; ++j) {
          f32x4 d;
          if constexpr (WF == 1) {  // int8 codes: the stage's int32 dot is exact in f32
            i32x4 di = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i4(a0), as_i4(bfr[j][0]), i32x4{0, 0, 0, 0}, 0, 0, 0);
            di = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i4(a1), as_i4(bfr[j][1]), di, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) d[r] = (float)di[r];
          } else {
            d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, pack8(bfr[j][0], bfr[j][1]),
                                                                 f32x4{0, 0, 0, 0}, 0, 0, 0, 127, 0, 127);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] += d[r] * (sa[r] * sbv[j]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < NF; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(a0), as_b8(bfr[j][0]), acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(a1), as_b8(bfr[j][1]), acc[i][j], 0, 0, 0);
        }
      }
    }
    // buf ^ 1 was last read in the previous stage, which every wavefront
    // finished before the previous barrier
    if (ks + 1 < ks1) sstore(buf ^ 1, ks + 1);
    __syncthreads();
  }

  if constexpr (!Tr::kInt && !ACT && BM == 128) {
    if (gridDim.z > 1) {  // K split: this slice's sums, [slice][M][N] f32
      float* dst = p.partial + (int64_t)blockIdx.z * p.M * p.N;
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int rr = wm * (BM / 2) + i * 16 + kg * 4 + r;
          if (rr >= rows) continue;
          float* drow = dst + (int64_t)(row0 + rr) * p.N;
#pragma unroll
          for (int j = 0; j < NF; ++j) {
            const int n = n0 + wn * (BN / 2) + j * 16 + col;
            if (n < nlim) drow[n] = acc[i][j][r];
          }
        }
      return;
    }
  }

  // ---- epilogue: finish in registers, stage bf16 in LDS, 16-byte stores ----
  constexpr int OP = BNO * 2 + 16;  // padded LDS pitch of the output tile (bytes)
  uint8_t* sOut = smem;
  const float* wsc = static_cast<const float*>(p.w_scale);
  auto fin = [&](float v, float sxa, int n) {
    if (KIND == QK_W8A8_PC) {
      v = v * sxa;
      v = v * wsc[(int64_t)g * p.ws_gstride + n];
    } else if (KIND == QK_W8A16_PC) {
      v = v * wsc[(int64_t)g * p.ws_gstride + n];
    }
    if (p.bias) v += p.bias[(int64_t)g * p.bias_gstride + n];
    return v;
  };
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rr = wm * (BM / 2) + i * 16 + kg * 4 + r;
      const int R = row0 + (rr < rows ? rr : 0);
      const int ar = p.a_rows ? p.a_rows[R] : R;
      const float sxa = KIND == QK_W8A8_PC ? p.a_scale[(int64_t)ar * p.lds_a] : 1.0f;
      const float rwt = p.row_weight ? bf16_to_f32(p.row_weight[R]) : 1.0f;
      constexpr int JN = ACT ? NF / 2 : NF;
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const int tc = ACT ? wn * (BN / 4) + j * 16 + col : wn * (BN / 2) + j * 16 + col;
        const int ccol = min(n0 + tc, nlim - 1);
        float v0, v1 = 0.0f;
        if constexpr (Tr::kInt) v0 = (float)acc[i][j][r];
        else v0 = acc[i][j][r];
        float out;
        if (ACT) {
          if constexpr (Tr::kInt) v1 = (float)acc[i][j + NF / 2][r];
          else v1 = acc[i][j + NF / 2][r];
          out = qmoe_act(p.act, fin(v0, sxa, ccol), fin(v1, sxa, p.N / 2 + ccol), p.act_p0, p.act_p1);
        } else {
          out = fin(v0, sxa, ccol);
        }
        *reinterpret_cast<uint16_t*>(sOut + rr * OP + tc * 2) = f32_to_bf16(out * rwt);
      }
    }
  __syncthreads();
  // copy rows out: 8 bf16 (16 bytes) per thread per chunk
  constexpr int CPR = BNO / 8;  // chunks per row
  const bool vec_ok = ((p.ldy & 7) == 0) && ((reinterpret_cast<uintptr_t>(p.y) & 15) == 0);
  for (int c = tid; c < BM * CPR; c += kThreads) {
    const int rr = c / CPR;
    const int cc = (c % CPR) * 8;
    if (rr >= rows) continue;
    const int R = row0 + rr;
    const int64_t yr = p.y_rows ? p.y_rows[R] : R;
    uint16_t* dst = p.y + yr * p.ldy + n0 + cc;
    const uint8_t* src = sOut + rr * OP + cc * 2;
    if (vec_ok && n0 + cc + 8 <= nlim) {
      *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
    } else {
      for (int e = 0; e < 8 && n0 + cc + e < nlim; ++e) dst[e] = reinterpret_cast<const uint16_t*>(src)[e];
    }
  }
}

template <int KIND, int WF, int BM, int BN, bool ACT>
void launch_tiled(const GemmParams& p, int ksplit, hipStream_t st) {
  constexpr size_t smem = tiled_smem_bytes<BM, BN, ACT>();
  auto kern = tiled_gemm_kernel<KIND, WF, BM, BN, ACT>;
  static bool attr_set = false;  // once per instantiation (process-wide)
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    attr_set = true;
  }
  const int nout = ACT ? p.N / 2 : p.N;
  const int n_tiles = cdiv(nout, ACT ? BN / 2 : BN);
  if (p.group_offs) {
    const int m_tiles = cdiv(p.M, BM) + std::min(p.slots, p.M);
    hipLaunchKernelGGL(kern, dim3(n_tiles, m_tiles, 1), dim3(kThreads), smem, st, p, m_tiles, n_tiles);
  } else {
    const int m_tiles = cdiv(p.M, BM);
    const int total = m_tiles * n_tiles;
    const int grid = cdiv(total, kXcds) * kXcds;
    hipLaunchKernelGGL(kern, dim3(grid, 1, ksplit), dim3(kThreads), smem, st, p, m_tiles, n_tiles);
  }
}

template <int KIND, int WF, int BM, int BN>
void launch_tiled_act(const GemmParams& p, int ksplit, hipStream_t st) {
  // K splits: 128 x 128 tiles without a fused activation only
  if (p.act != QA_NONE) launch_tiled<KIND, WF, BM, BN, true>(p, 1, st);
  else launch_tiled<KIND, WF, BM, BN, false>(p, BM == 128 ? ksplit : 1, st);
}

// 256 x 256 tiles only for the kinds whose 128 x 128 wavefront tile fits the
// register file without spilling (the block-scale and bf16-expanding kinds
// need extra registers per MFMA group)
template <int KIND>
constexpr bool has_big_tile() {
  return KIND == QK_W8A8_PC || KIND == QK_W8A16_PC;
}

template <int KIND, int WF>
void launch_shape(const GemmParams& p, bool big, int ksplit, hipStream_t st) {
  if constexpr (has_big_tile<KIND>()) {
    if (big) {
      launch_tiled_act<KIND, WF, 256, 256>(p, ksplit, st);
      return;
    }
  }
  launch_tiled_act<KIND, WF, 128, 128>(p, ksplit, st);
}

}  // namespace

// K-split finish for this kernel's partials (defined with the other tiled
// kernels' finish): sums the slices in order, then the per-channel weight
// scale (weight_scale), bias and routing weight, bf16 out.
int qmoe_tile_splitk_finish(const GemmParams& p, bool weight_scale, hipStream_t st);

// Whether the generic tiled kernel takes the problem (QMOE_OK) and its plan:
// tile edge (128, or 256 with the QMOE_TILED_BIG knob), K split and the f32
// workspace the split needs ([ksplit][M][N]). Dense bf16-activation problems
// without a fused activation and under 256 tiles of 128 x 128 are split over
// K into about 512 workgroups (at most 8 slices of at least 8 stages).
// Measured on MI355X, DeepSeek-V3's router gate (K 7168, N 256): 128 / 1024
// / 4096 / 8192 tokens 94.3 / 98.6 / 98.3 / 98.6 us in one pass, 22.2 / 23.9
// / 35.0 / 49.8 in 8 / 8 / 8 / 4 slices.
int qmoe_tiled_plan(int kind, const GemmParams& p, int* tile, int* ksplit, int64_t* ws_bytes) {
  const bool abf16 = kind == QK_W8A16_PC || kind == QK_W4A16_MX || kind == QK_W16A16 || kind == QK_W8A16_BLK;
  const int kstage = abf16 ? 64 : 128;
  if (kind != QK_W8A8_PC && kind != QK_W8A8_BLK && !abf16) return QMOE_ERR_ARG;
  if (p.wfmt != 0 && p.wfmt != 1) return QMOE_ERR_ARG;  // no e5m2 form
  if (kind == QK_W8A16_BLK && (p.K % 128) != 0) return QMOE_ERR_ARG;
  if (p.K <= 0 || (p.K % kstage) != 0 || p.N <= 0) return QMOE_ERR_ARG;
  if (p.act != QA_NONE && (p.N % 2) != 0) return QMOE_ERR_ARG;
  bool big = false;  // 128 x 128 measured faster or equal on every config shape
  const char* env = getenv("QMOE_TILED_BIG");  // tuning knob: force 1 / 0
  if (env) big = atoi(env) != 0;
  if (kind != QK_W8A8_PC && kind != QK_W8A16_PC) big = false;
  if (p.group_offs) {
    const int m_tiles = cdiv(p.M, big ? 256 : 128) + std::min(p.slots, p.M);
    if (m_tiles > 65535) return QMOE_ERR_ARG;
  }
  int ks = 1;
  if (abf16 && !big && !p.group_offs && p.act == QA_NONE && p.M > 0) {
    const int64_t tiles = (int64_t)cdiv(p.M, 128) * cdiv(p.N, 128);
    if (tiles < 256) ks = (int)std::min<int64_t>(std::min<int64_t>(8, 512 / tiles), p.K / kstage / 8);
    const char* ks_env = getenv("QMOE_TILED_KSPLIT");  // tuning knob
    if (ks_env && atoi(ks_env) > 0) ks = std::min(atoi(ks_env), p.K / kstage);
    ks = std::max(ks, 1);
  }
  *tile = big ? 256 : 128;
  if (ksplit) *ksplit = ks;
  if (ws_bytes) *ws_bytes = ks > 1 ? (int64_t)ks * p.M * p.N * 4 : 0;
  return QMOE_OK;
}

int qmoe_tiled_launch(int kind, GemmParams p, void* workspace, int64_t ws_bytes, hipStream_t st) {
  if (p.M <= 0) return QMOE_OK;
  int tile = 128, ks = 1;
  int64_t need = 0;
  const int chk = qmoe_tiled_plan(kind, p, &tile, &ks, &need);
  if (chk != QMOE_OK) return chk;
  p.ksplit = ks;
  if (ks > 1) {
    if (!workspace || ws_bytes < need) return QMOE_ERR_WORKSPACE;
    p.partial = static_cast<float*>(workspace);
  }
  const bool big = tile == 256;
  switch (kind) {
    case QK_W8A8_PC:
      if (p.wfmt == 0) launch_shape<QK_W8A8_PC, 0>(p, big, 1, st);
      else launch_shape<QK_W8A8_PC, 1>(p, big, 1, st);
      break;
    case QK_W8A8_BLK:
      if (p.wfmt == 0) launch_shape<QK_W8A8_BLK, 0>(p, big, 1, st);
      else launch_shape<QK_W8A8_BLK, 1>(p, big, 1, st);
      break;
    case QK_W8A16_BLK: launch_shape<QK_W8A16_BLK, 0>(p, big, ks, st); break;
    case QK_W8A16_PC: launch_shape<QK_W8A16_PC, 0>(p, big, ks, st); break;
    case QK_W4A16_MX: launch_shape<QK_W4A16_MX, 0>(p, big, ks, st); break;
    case QK_W16A16: launch_shape<QK_W16A16, 0>(p, big, ks, st); break;
    default: return QMOE_ERR_ARG;
  }
  if (ks > 1) {
    const int fin = qmoe_tile_splitk_finish(p, kind == QK_W8A16_PC, st);
    if (fin != QMOE_OK) return fin;
  }
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
