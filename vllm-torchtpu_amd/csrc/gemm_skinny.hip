// Skinny (decode) grouped GEMM: few rows per group, weights streamed from HBM
// exactly once.
//
// Small-M linears and decode MoE are weight-bandwidth bound, so the design
// goal is to keep enough 16-byte weight loads in flight to saturate HBM3E:
//  * workgroup = W wavefronts (4 or 8); it owns NS 16-row MFMA B tiles
//    of weight rows (NS/2 gate tiles + the matching up tiles when an
//    activation is fused) and a slice of K. NS = 2 (4 is kept for e2m1
//    weights as a tuning option);
//  * K is cut into 128-wide steps; the workgroup's steps are dealt out to its
//    W wavefronts, and further across `ksplit` workgroups (grid.y) when
//    the grid is small;
//  * a wavefront issues the loads of U steps back to back, unconditionally
//    (weight rows past N are clamped to valid rows, activation rows past the
//    group read zeros from an out-of-range offset -- both only feed outputs
//    that are never stored), and only then waits and issues the MFMAs, so U
//    steps of weights are in flight per wavefront. Only a K tail
//    (K % 128 != 0) uses masked loads;
//  * weight loads are coalesced: 4 adjacent lanes read the 4 x 16 B of one
//    row's 64 B segment (16 rows per load instruction; measured on MI355X,
//    17% more bandwidth than one row per lane), and ds_bpermute then moves
//    the data into MFMA fragment order;
//  * in a step, lane l holds 32 k values of weight row (l & 15)
//    (32 B of e4m3/int8, 16 B of e2m1, 64 B of bf16) and the same k values of
//    activation row (l & 15) of each 16-row M tile, and issues the matching
//    MFMA(s): one
//    v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3), two v_mfma_i32_16x16x64_i8
//    (int8) or four v_mfma_f32_16x16x32_bf16 (bf16 activations; e2m1 weights
//    are expanded with v_cvt_scalef32_pk_bf16_fp4, which also applies the e8m0
//    block scale; e4m3 with v_cvt_pk_f32_fp8). A and W use the same
//    lane -> k assignment, so products pair up whatever order the MFMA walks k;
//  * the W wavefronts' sums are added in LDS in a fixed order; with
//    ksplit > 1 each workgroup stores its raw sums to a float32 workspace and
//    a second kernel adds the slices in order and runs the epilogue (kernel
//    boundaries order the memory traffic, so no cache-flushing fence runs).

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "gemm_common.h"
#include "row_quant.h"
#include "stream_load.h"

namespace {

using namespace qmoe_stream;

// cache-policy bits of the weight stream's loads (read once per launch).
// The non-temporal bit (2) keeps the small tensors and code of the next
// launches cached but cut the DeepSeek-V3 decode GEMMs' bandwidth by 15%
// on MI355X, so the default policy stays.
constexpr int kWeightAux = 0;

constexpr int kWaves = 4;  // wavefronts per workgroup (streaming and split-K finishing kernels)
// QA: the most dynamic LDS a workgroup's activation codes may take (two
// workgroups still fit one CU's 160 KB)
constexpr int64_t kQaMaxLds = 64 << 10;
constexpr int kThreads = kWaves * 64;

// QA: the kernel reads bf16 activation rows and quantizes them per row
// itself (QK_W8A8_PC only); its A fragments then come from the codes it
// wrote to LDS, not from global memory.
template <int KIND, int WF, bool QA = false>
struct Traits {
  static constexpr bool kAbf16 = kind_abf16(KIND) || QA;
  static constexpr bool kW4 = kind_w4(KIND);
  static constexpr bool kInt = KIND == QK_W8A8_PC && WF == 1;
  // bytes per lane per 128-k step (32 k values)
  static constexpr int kWBytes = kW4 ? 16 : (KIND == QK_W16A16 ? 64 : 32);
  static constexpr int kABytes = kAbf16 ? 64 : 32;
  // Weight chunk j (16 B) of lane (column c, k-group kg) sits at byte
  // j*64 + kg*16 of the row's step (4 lanes x 16 B = one 64 B segment per
  // load instruction and row); the k values of each 16 B activation chunk i
  // match the weight data they meet in the MFMA:
  //   1-byte A (e4m3/int8) and bf16 A with bf16 W: byte kg*16 + i*64
  //   bf16 A with e4m3 W: byte kg*32 + (i/2)*128 + (i%2)*16
  //   bf16 A with e2m1 W: byte kg*64 + i*16
  static constexpr bool kW8A16 = KIND == QK_W8A16_PC || KIND == QK_W8A16_BLK || QA;
  static constexpr int kAOffBase = kW4 ? 64 : (kW8A16 ? 32 : 16);
  static __device__ __forceinline__ constexpr int a_off(int i) {
    return kW4 ? i * 16 : (kW8A16 ? (i >> 1) * 128 + (i & 1) * 16 : i * 64);
  }
  // first k (within the step) of weight chunk (j, kg) / activation chunk (i, kg)
  static __device__ __forceinline__ constexpr int w_k0(int j, int kg) {
    return kW4 ? kg * 32 : (KIND == QK_W16A16 ? j * 32 + kg * 8 : j * 64 + kg * 16);
  }
  static __device__ __forceinline__ constexpr int a_k0(int i, int kg) {
    return (kg * kAOffBase + a_off(i)) / (kAbf16 ? 2 : 1);
  }
};

// 128-k steps per pipeline chunk (two chunks are in flight per wavefront):
// one. Measured on MI355X: deeper chunks (2 or 4 steps) add clamped duplicate
// loads at the end of the short per-wavefront K slices and lose 5-30%, so
// only the one-step form is instantiated.
constexpr int kUnroll = 1;

// activation chunks of one step at the offsets of Traits::a_off
template <typename Tr>
__device__ __forceinline__ void lda_chunks(Frag& f, rsrc_t r, uint32_t voff, uint32_t soff) {
#pragma unroll
  for (int i = 0; i < Tr::kABytes / 16; ++i) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff + Tr::a_off(i), soff, 0);
    f.v[i] = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

__device__ __forceinline__ i32x4 as_i32x4(const uint4& u) {
  i32x4 r;
  r[0] = u.x; r[1] = u.y; r[2] = u.z; r[3] = u.w;
  return r;
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& u) {
  union { uint4 u; bf16x8 b; } c;
  c.u = u;
  return c.b;
}

// 8 e2m1 codes (one dword, low nibble first) -> 8 bf16 times 2^(e-127)
__device__ __forceinline__ uint4 fp4x8_to_bf16(uint32_t d, float scale) {
  bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 0);
  bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 1);
  bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 2);
  bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 3);
  union { bf16x2 b; uint32_t u; } c0, c1, c2, c3;
  c0.b = p0; c1.b = p1; c2.b = p2; c3.b = p3;
  return make_uint4(c0.u, c1.u, c2.u, c3.u);
}

// 4 e4m3 codes (one dword) times a bf16-valued scale -> 4 bf16, each the
// round-to-nearest-even of code * scale (a 4-bit by 8-bit significand
// product, exact in f32): the reference's bf16 dequantization of a block-
// scaled FP8 weight, `kernels/megablox/gmm_v2.py:452-462`.
__device__ __forceinline__ uint2 fp8x4_to_bf16_scaled(uint32_t d, float s) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, false);
  const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, true);
  union { bf16x2 h; uint32_t u; } a, b;
  a.h = __builtin_convertvector(f32x2{lo[0] * s, lo[1] * s}, bf16x2);
  b.h = __builtin_convertvector(f32x2{hi[0] * s, hi[1] * s}, bf16x2);
  return make_uint2(a.u, b.u);
}

// 4 e4m3 codes (one dword) -> 4 bf16 bit patterns packed in two dwords
// (e4m3 values are exact in f32 and in bf16, so truncation is exact).
__device__ __forceinline__ uint2 fp8x4_to_bf16(uint32_t d) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, false);
  v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, true);
  uint32_t a = (f32_bits(lo[0]) >> 16) | (f32_bits(lo[1]) & 0xffff0000u);
  uint32_t b = (f32_bits(hi[0]) >> 16) | (f32_bits(hi[1]) & 0xffff0000u);
  return make_uint2(a, b);
}

template <int KIND, int WF, int MS, int NS>
struct Acc {
  using T = typename std::conditional<Traits<KIND, WF>::kInt, i32x4, f32x4>::type;
  T v[MS][NS];
};

// Per-step side data: per-(row, block) and per-(n, block) scales (W8A8_BLK),
// e8m0 block scale of the lane's weight row (W4A16_MX), the two bf16 block
// scales of the lane's 32 k (W4A16_NV, low half first), the bf16 group
// scale of the lane's 32 k (W4A16_I4).
template <int MS, int NS>
struct StepScales {
  float sa[MS][4];
  float sb[NS];
  uint32_t eb[NS];  // raw e8m0 bytes / bf16 pairs, decoded where they are used
};

// One 128-k step of MFMAs for all (M tile, weight tile) pairs.
template <int KIND, int WF, int MS, int NS>
__device__ __forceinline__ void mma_step(Acc<KIND, WF, MS, NS>& acc, const Frag (&fa)[MS],
                                         const Frag (&bw)[NS], const StepScales<MS, NS>& sc) {
  if constexpr (KIND == QK_W8A8_PC && WF != 1) {
    // e4m3 (WF 0) or e5m2 (WF 2) on both operands (format codes 0 / 1)
    constexpr int kF = WF == 2 ? 1 : 0;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int s = 0; s < NS; ++s)
        acc.v[ms][s] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            as_i32x8(fa[ms]), as_i32x8(bw[s]), acc.v[ms][s], kF, kF, 0, 127, 0, 127);
  } else if constexpr (KIND == QK_W8A8_PC && WF == 1) {
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        acc.v[ms][s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i32x4(fa[ms].v[0]), as_i32x4(bw[s].v[0]),
                                                             acc.v[ms][s], 0, 0, 0);
        acc.v[ms][s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i32x4(fa[ms].v[1]), as_i32x4(bw[s].v[1]),
                                                             acc.v[ms][s], 0, 0, 0);
      }
  } else if constexpr (KIND == QK_W8A8_BLK) {
    // one 128-k step lies in one scale block: scale the step's dot, then add
    // (int8 codes: the step's int32 dot is exact in f32, |dot| < 2^21)
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        f32x4 d;
        if constexpr (WF == 1) {
          i32x4 di = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i32x4(fa[ms].v[0]), as_i32x4(bw[s].v[0]),
                                                           i32x4{0, 0, 0, 0}, 0, 0, 0);
          di = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_i32x4(fa[ms].v[1]), as_i32x4(bw[s].v[1]), di, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) d[r] = (float)di[r];
        } else {
          // e4m3 activations; e4m3 (WF 0) or e5m2 (WF 2) weights
          d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(as_i32x8(fa[ms]), as_i32x8(bw[s]),
                                                               f32x4{0, 0, 0, 0}, 0, WF == 2 ? 1 : 0, 0, 127, 0,
                                                               127);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc.v[ms][s][r] += d[r] * (sc.sa[ms][r] * sc.sb[s]);
      }
  } else {
    // bf16 activations: expand each weight fragment to 4 x 8 bf16 right
    // before its MFMAs (one tile's expansion live at a time)
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint4 wb[4];
      if constexpr (KIND == QK_W16A16) {
#pragma unroll
        for (int q = 0; q < 4; ++q) wb[q] = bw[s].v[q];
      } else if constexpr (KIND == QK_W8A16_PC) {
        const uint32_t d[8] = {bw[s].v[0].x, bw[s].v[0].y, bw[s].v[0].z, bw[s].v[0].w,
                               bw[s].v[1].x, bw[s].v[1].y, bw[s].v[1].z, bw[s].v[1].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint2 lo = fp8x4_to_bf16(d[2 * q]);
          const uint2 hi = fp8x4_to_bf16(d[2 * q + 1]);
          wb[q] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
      } else if constexpr (KIND == QK_W8A16_BLK) {  // bf16(code * bf16(scale)), the step's block scale
        const uint32_t d[8] = {bw[s].v[0].x, bw[s].v[0].y, bw[s].v[0].z, bw[s].v[0].w,
                               bw[s].v[1].x, bw[s].v[1].y, bw[s].v[1].z, bw[s].v[1].w};
        const float sc1 = bf16_round(sc.sb[s]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint2 lo = fp8x4_to_bf16_scaled(d[2 * q], sc1);
          const uint2 hi = fp8x4_to_bf16_scaled(d[2 * q + 1], sc1);
          wb[q] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
      } else if constexpr (KIND == QK_W4A16_MX) {
        const uint32_t d[4] = {bw[s].v[0].x, bw[s].v[0].y, bw[s].v[0].z, bw[s].v[0].w};
        const float scale = e8m0_to_f32(sc.eb[s]);
#pragma unroll
        for (int q = 0; q < 4; ++q) wb[q] = fp4x8_to_bf16(d[q], scale);
      } else if constexpr (KIND == QK_W4A16_I4) {  // one group scale for the lane's 32 k
        const uint32_t d[4] = {bw[s].v[0].x, bw[s].v[0].y, bw[s].v[0].z, bw[s].v[0].w};
        const float sc1 = bits_f32(sc.eb[s] << 16);
#pragma unroll
        for (int q = 0; q < 4; ++q) wb[q] = int4x8_to_bf16(d[q], sc1);
      } else {  // QK_W4A16_NV: dwords 0-1 are the first 16-k block, 2-3 the second
        const uint32_t d[4] = {bw[s].v[0].x, bw[s].v[0].y, bw[s].v[0].z, bw[s].v[0].w};
        const float s0 = bits_f32(sc.eb[s] << 16), s1 = bits_f32(sc.eb[s] & 0xffff0000u);
#pragma unroll
        for (int q = 0; q < 4; ++q) wb[q] = nvfp4x8_to_bf16(d[q], q < 2 ? s0 : s1);
      }
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc.v[ms][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(fa[ms].v[q]), as_bf16x8(wb[q]),
                                                                 acc.v[ms][s], 0, 0, 0);
    }
  }
}

// Per-format scale + bias for one accumulator element (before activation).
// QA: the activation row's scale is `asc` (computed in the kernel).
template <int KIND, bool QA = false>
__device__ __forceinline__ float finish_elem(const GemmParams& p, float acc, int arow, int g, int n,
                                             float asc = 0.0f) {
  float v = acc;
  if (KIND == QK_W8A8_PC) {
    v = v * (QA ? asc : p.a_scale[(int64_t)arow * p.lds_a]);
    v = v * group_slice(p, static_cast<const float*>(p.w_scale), p.ws_x, p.ws_gstride, g)[n];
  } else if (KIND == QK_W8A16_PC) {
    v = v * group_slice(p, static_cast<const float*>(p.w_scale), p.ws_x, p.ws_gstride, g)[n];
  }
  if (p.bias) v += p.bias[(int64_t)g * p.bias_gstride + n];
  return v;
}

template <int KIND, bool ACT, bool QA = false>
__device__ __forceinline__ void store_out(const GemmParams& p, int g, int R, int arow, int ncol_out,
                                          int n0, int n1, float v0, float v1, float asc = 0.0f) {
  float out;
  if (ACT) {
    const float gte = finish_elem<KIND, QA>(p, v0, arow, g, n0, asc);
    const float up = finish_elem<KIND, QA>(p, v1, arow, g, n1, asc);
    out = qmoe_act(p.act, gte, up, p.act_p0, p.act_p1);
  } else {
    out = finish_elem<KIND, QA>(p, v0, arow, g, n0, asc);
  }
  if (p.row_weight) out *= bf16_to_f32(p.row_weight[R]);
  const int64_t yr = p.y_rows ? p.y_rows[R] : R;
  p.y[yr * p.ldy + ncol_out] = f32_to_bf16(out);
}

// group of this workgroup's slot; false if the slot is empty
__device__ __forceinline__ bool slot_group(const GemmParams& p, int slot, int& g, int& row0, int& rows) {
  if (p.row_split) {  // dense: slice `slot` of the rows
    g = 0;
    row0 = slot * p.row_split;
    rows = min(p.row_split, p.M - row0);
    return rows > 0;
  }
  if (p.x0 && slot == 0) {
    g = 0;
    row0 = 0;
    rows = p.rows_x;
    return rows > 0;
  }
  g = slot;
  if (p.active) {
    // both loads at once (the list has an entry for every slot of the grid:
    // its capacity), then the count decides
    const int na = *p.num_active;
    const int ga = p.active[slot];
    if (slot >= na) return false;
    g = ga;
  }
  row0 = p.group_offs ? p.group_offs[g] : 0;
  rows = p.group_offs ? p.group_offs[g + 1] - row0 : p.M;
  return rows > 0;
}

template <int KIND, int WF, int MS, bool ACT, int U, int NS, int W, bool QA = false>
__global__ __launch_bounds__(W * 64) void skinny_gemm_kernel(const GemmParams p) {
  using Tr = Traits<KIND, WF, QA>;
  static_assert(!QA || KIND == QK_W8A8_PC, "in-kernel activation quantization is per-channel W8A8 only");
  constexpr int NT = W * 64;
  const int lane = threadIdx.x & 63;
  // wave-uniform in an SGPR, so K-slice bounds and loop tests are scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;
  const int kg = lane >> 4;

  int g, row0, rows;
  if (!slot_group(p, blockIdx.z, g, row0, rows)) return;

  // weight rows of the NS B tiles (clamped copies feed the loads); with an
  // activation, tile s < NS/2 holds gate rows and tile s + NS/2 the
  // matching up rows
  constexpr int NH = NS / 2;
  const int tile = blockIdx.x;
  // weight rows of this group (the extra group of a fused decode layer may
  // have fewer; its surplus tiles have no work)
  const int NG = (p.x0 && g == 0) ? p.n_x : p.N;
  const int nlim = ACT ? (NG >> 1) : NG;
  if (tile * (ACT ? 16 * NH : 16 * NS) >= nlim) return;
  int nw[NS];
  bool nok[NS];
  if (ACT) {
#pragma unroll
    for (int s = 0; s < NH; ++s) {
      const int c = tile * (16 * NH) + s * 16 + col;
      nok[s] = nok[s + NH] = c < nlim;
      nw[s] = c;
      nw[s + NH] = (NG >> 1) + c;
    }
  } else {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      nw[s] = tile * (16 * NS) + s * 16 + col;
      nok[s] = nw[s] < nlim;
    }
  }
  g = __builtin_amdgcn_readfirstlane(g);
  const rsrc_t wres = make_rsrc(group_slice(p, p.w, p.w_x, p.w_gstride, g), (int64_t)NG * p.ldw);
  auto row_of = [&](int s, int c) {  // clamped global row of tile s, column c
    if (ACT) {
      const int r = min(tile * (16 * NH) + (s % NH) * 16 + c, nlim - 1);
      return s < NH ? r : (NG >> 1) + r;
    }
    return min(tile * (16 * NS) + s * 16 + c, NG - 1);
  };
  // weight loads: lane l reads row (l >> 2) of each tile, 16 B column (l & 3)
  uint32_t woff[NS];
  int nclamp[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    nclamp[s] = nok[s] ? nw[s] : (ACT ? (s < NH ? nlim - 1 : NG - 1) : NG - 1);
    woff[s] = (uint32_t)(row_of(s, lane >> 2) * p.ldw + (lane & 3) * 16);
  }
  const int perm_src = (4 * col + kg) * 4;
  // scale streams: e8m0 bytes [N][K/32] (W4A16_MX: one byte per lane, tile
  // and step, for the lane's row and 32 k, loaded with the step's weights;
  // measured on MI355X, faster than staging the rows in LDS first), bf16
  // [N][K/16] (W4A16_NV: one 4-byte pair per lane and step, for the lane's
  // row and 32 k), per-step f32 [N/bn][K/128] weight blocks and [rows][K/128]
  // activation blocks (W8A8_BLK)
  rsrc_t sres = wres, ares = wres;  // placeholders for kinds without scale streams
  uint32_t soffw[NS];
  if constexpr (KIND == QK_W4A16_MX) {
    sres = make_rsrc(group_slice(p, static_cast<const uint8_t*>(p.w_scale), p.ws_x, p.ws_gstride, g), (int64_t)NG * p.ldws);
#pragma unroll
    for (int s = 0; s < NS; ++s) soffw[s] = (uint32_t)(nclamp[s] * p.ldws + kg);
  } else if constexpr (KIND == QK_W4A16_NV) {
    sres = make_rsrc(group_slice(p, static_cast<const uint16_t*>(p.w_scale), p.ws_x, p.ws_gstride, g),
                     (int64_t)NG * p.ldws * 2);
#pragma unroll
    for (int s = 0; s < NS; ++s) soffw[s] = (uint32_t)(nclamp[s] * p.ldws * 2 + kg * 4);
  } else if constexpr (KIND == QK_W4A16_I4) {
    // bf16 [N][K/group]: the lane's 32 k sit in group (128 step + 32 kg) / group
    sres = make_rsrc(group_slice(p, static_cast<const uint16_t*>(p.w_scale), p.ws_x, p.ws_gstride, g),
                     (int64_t)NG * p.ldws * 2);
#pragma unroll
    for (int s = 0; s < NS; ++s) soffw[s] = (uint32_t)(nclamp[s] * p.ldws * 2 + (kg * 32 / p.wq_group) * 2);
  } else if constexpr (KIND == QK_W8A8_BLK || KIND == QK_W8A16_BLK) {
    sres = make_rsrc(group_slice(p, static_cast<const float*>(p.w_scale), p.ws_x, p.ws_gstride, g),
                     (int64_t)cdiv(NG, p.ws_bn) * p.ldws * 4);
    if (KIND == QK_W8A8_BLK) ares = make_rsrc(p.a_scale, (int64_t)p.M * p.lds_a * 4);
#pragma unroll
    for (int s = 0; s < NS; ++s) soffw[s] = (uint32_t)((nclamp[s] / p.ws_bn) * p.ldws * 4);
  }
  // block index of 128-k step ks: ks >> shift (the activation's and the
  // weight's; 31 for one scale per row)
  const int a_kshift = p.a_kshift, w_kshift = p.w_kshift;
  const uint32_t i4_step = KIND == QK_W4A16_I4 ? (uint32_t)(256 / p.wq_group) : 0u;  // INT4 scale bytes per step
  // K steps: KSF full 128-wide steps, plus a tail step when K % 128 != 0
  const int KSF = p.K >> 7;
  const bool tail = (p.K & 127) != 0;
  const int KS = KSF + (tail ? 1 : 0);
  // this wavefront's full steps are sbase + j, j < nj (a contiguous run of
  // the workgroup's K slice); the wavefront whose run ends at K takes the tail
  // (q or q + 1 steps per slice: the first KS % nsl slices take one more)
  const int nsl = p.ksplit * W;
  const int sl = blockIdx.y * W + wave;
  const int q = (int)((uint32_t)KS / (uint32_t)nsl), rem = KS - q * nsl;
  const int sbase = sl * q + min(sl, rem);
  const int send = sbase + q + (sl < rem ? 1 : 0);
  const int nj = max(0, min(send, KSF) - sbase);
  const bool tail_mine = tail && send == KS && sbase < send;

  const int64_t lda_b = p.lda * (Tr::kAbf16 ? 2 : 1);
  const rsrc_t xres = make_rsrc(p.a, (int64_t)p.M * lda_b);
  constexpr int NV = MS * NS * 4;
  __shared__ float red[W - 1][NV][64];
  // QA: the rows' absolute maxima (as integer bits), the row scales, and
  // the rows' codes over this workgroup's K range (dynamic LDS: rows x
  // (range bytes + 16), the pad spreading rows over the banks)
  __shared__ float s_amax[1][QA ? 16 * MS : 1];
  __shared__ float s_sx[QA ? 16 * MS : 1];
  extern __shared__ __align__(16) uint8_t s_codes[];
  const int64_t plane = (int64_t)p.M * p.N;

  // Rows are taken 16*MS at a time (one pass when the host's row bound
  // holds; more passes re-read this workgroup's weight slice from cache).
  // Lanes of rows past the group load with kOob set in their offset: zeros,
  // and no memory request (at M = 1, 15 of the 16 copies of the activation
  // row a 16-row tile would otherwise read).
  for (int mp = 0; mp < rows; mp += 16 * MS) {
    uint32_t aoff[MS];
    uint32_t soffa[MS][4];  // scale offsets of the 4 accumulator rows (block scales)
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      const int r = mp + ms * 16 + col;
      const int R = row0 + (r < rows ? r : 0);
      const int ar = p.a_rows ? p.a_rows[R] : R;
      aoff[ms] = r < rows ? (uint32_t)(ar * lda_b + kg * Tr::kAOffBase) : kOob;
      if constexpr (KIND == QK_W8A8_BLK) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int rr = mp + ms * 16 + kg * 4 + r4;
          const int R2 = row0 + (rr < rows ? rr : 0);
          soffa[ms][r4] = rr < rows ? (uint32_t)((p.a_rows ? p.a_rows[R2] : R2) * p.lds_a * 4) : kOob;
        }
      }
    }

    Acc<KIND, WF, MS, NS> acc;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int s = 0; s < NS; ++s) acc.v[ms][s] = {0, 0, 0, 0};
    // QA: rows of the codes in LDS, their first step and row stride (bytes)
    int qa_rows = 0, qa_s0 = 0, qa_stride = 0;

    auto load_scales = [&](int ks, bool live, StepScales<MS, NS>& sc) {
      if constexpr (KIND == QK_W8A8_BLK) {
        const uint32_t oob = live ? 0u : kOob;
#pragma unroll
        for (int s = 0; s < NS; ++s) sc.sb[s] = ldb_f32(sres, soffw[s] | oob, (uint32_t)(ks >> w_kshift) * 4);
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4)
            sc.sa[ms][r4] = ldb_f32(ares, soffa[ms][r4] | oob, (uint32_t)(ks >> a_kshift) * 4);
      } else if constexpr (KIND == QK_W8A16_BLK) {
        const uint32_t oob = live ? 0u : kOob;
#pragma unroll
        for (int s = 0; s < NS; ++s) sc.sb[s] = ldb_f32(sres, soffw[s] | oob, (uint32_t)(ks >> w_kshift) * 4);
      } else if constexpr (KIND == QK_W4A16_MX) {
        const uint32_t oob = live ? 0u : kOob;
#pragma unroll
        for (int s = 0; s < NS; ++s)
          sc.eb[s] = __builtin_amdgcn_raw_buffer_load_b8(sres, soffw[s] | oob, (uint32_t)ks * 4, 0);
      } else if constexpr (KIND == QK_W4A16_NV) {
        const uint32_t oob = live ? 0u : kOob;
#pragma unroll
        for (int s = 0; s < NS; ++s)
          sc.eb[s] = __builtin_amdgcn_raw_buffer_load_b32(sres, soffw[s] | oob, (uint32_t)ks * 16, 0);
      } else if constexpr (KIND == QK_W4A16_I4) {
        const uint32_t oob = live ? 0u : kOob;
#pragma unroll
        for (int s = 0; s < NS; ++s)
          sc.eb[s] = __builtin_amdgcn_raw_buffer_load_b16(sres, soffw[s] | oob, (uint32_t)ks * i4_step, 0);
      }
    };

    // Full steps, U at a time, double-buffered: the loads of chunk c+1 are
    // issued before the MFMAs of chunk c, so 1-2 chunks are always in flight.
    // Steps past the run issue loads that return zeros without a memory
    // request; their MFMAs are skipped.
    struct Chunk {
      Frag bw[U][NS];
      Frag fa[U][MS];
      StepScales<MS, NS> sc[U];
    };
    // steps past the run are issued with kOob set in the lane offsets: the
    // load instructions still count in vmcnt (so every path waits alike) but
    // return zeros without a memory request
    auto issue_mem = [&](int j, Chunk& c) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool live = j + u < nj;
        const uint32_t kk = live ? (uint32_t)(sbase + j + u) : 0u;
        const uint32_t oob = live ? 0u : kOob;
#pragma unroll
        for (int s = 0; s < NS; ++s)
          ldw_seg<Tr::kWBytes, kWeightAux>(c.bw[u][s], wres, woff[s] | oob, kk * (4 * Tr::kWBytes));
        if constexpr (!QA) {
#pragma unroll
          for (int ms = 0; ms < MS; ++ms) lda_chunks<Tr>(c.fa[u][ms], xres, aoff[ms] | oob, kk * (4 * Tr::kABytes));
        }
      }
    };
    auto issue_sc = [&](int j, Chunk& c) {
#pragma unroll
      for (int u = 0; u < U; ++u) load_scales(sbase + min(j + u, nj - 1), j + u < nj, c.sc[u]);
    };
    auto issue = [&](int j, Chunk& c) {
      issue_mem(j, c);
      issue_sc(j, c);
    };
    auto consume = [&](int j, Chunk& c) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int s = 0; s < NS; ++s) permute_w<Tr::kWBytes>(c.bw[u][s], perm_src);
        if (j + u < nj) {
          if constexpr (QA) {
            // the step's codes of the lane's row: k kg*16 .. +16 and 64 +
            // kg*16 .. +16 of the step, from LDS (rows past the group: 0)
            const int off = (sbase + j + u - qa_s0) * 128 + kg * 16;
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
              const int r = ms * 16 + col;
              const bool live = r < qa_rows;
              const uint8_t* src = s_codes + (live ? r : 0) * qa_stride + off;
              const uint4 c0 = *reinterpret_cast<const uint4*>(src);
              const uint4 c1 = *reinterpret_cast<const uint4*>(src + 64);
              c.fa[u][ms].v[0] = live ? c0 : make_uint4(0, 0, 0, 0);
              c.fa[u][ms].v[1] = live ? c1 : make_uint4(0, 0, 0, 0);
            }
          }
          mma_step<KIND, WF, MS, NS>(acc, c.fa[u], c.bw[u], c.sc[u]);
        }
      }
    };
    // Issues are unconditional (clamped step indices): a load issued only on
    // some paths would make the wait before the next MFMAs assume the
    // shorter path and drain the chunk just issued as well. The scheduling
    // barriers keep the compiler from sinking a chunk's loads below the
    // MFMAs of the previous one.
    Chunk ca, cb;
    const bool run = nj > 0;
    if (run) issue_mem(0, ca);
    if constexpr (QA) {
      // Phase 1, while the first weight chunk is in flight: each row's
      // absolute maximum over the whole K. The rows' 16-byte chunks are
      // dealt to all threads (from L2 after the first workgroup's read),
      // eight independent loads per batch; each chunk's maximum is folded
      // into its row's LDS slot by an integer atomic max (|x| bit patterns
      // order like the values, NaN above inf: NaN-sticky).
      const int np = min(16 * MS, rows - mp);
      const int cpr = p.K >> 3;  // 16-byte chunks per row
      unsigned* s_amax_u = reinterpret_cast<unsigned*>(&s_amax[0][0]);
      if ((int)threadIdx.x < 16 * MS) s_amax_u[threadIdx.x] = 0u;
      __syncthreads();
      {
        constexpr int kIt = 8;
        const int items = np * cpr;
        for (int i0 = (int)threadIdx.x; i0 < items; i0 += NT * kIt) {
          uint4 v[kIt];
          int rr[kIt];
#pragma unroll
          for (int it = 0; it < kIt; ++it) {
            const int i = i0 + it * NT;
            const int r = i / cpr;
            rr[it] = i < items ? r : -1;
            const uint32_t o = i < items ? (uint32_t)((row0 + mp + r) * lda_b) + (uint32_t)(i - r * cpr) * 16u : kOob;
            const auto t = __builtin_amdgcn_raw_buffer_load_b128(xres, o, 0, 0);
            v[it] = make_uint4(t[0], t[1], t[2], t[3]);
          }
#pragma unroll
          for (int it = 0; it < kIt; ++it)
            if (rr[it] >= 0) atomicMax(&s_amax_u[rr[it]], __float_as_uint(qmoe_rq::amax8(qmoe_rq::row8_bf16(v[it]))));
        }
      }
      __syncthreads();
      if ((int)threadIdx.x < 16 * MS) {
        const float m = (int)threadIdx.x < np ? __uint_as_float(s_amax_u[threadIdx.x]) : 0.0f;
        s_sx[threadIdx.x] = qmoe_rq::make_scale<WF, 0>(m);
      }
      __syncthreads();
      // the row scales for the split-K finishing kernel's epilogue
      if (p.a_scale && blockIdx.x == 0 && blockIdx.y == 0 && (int)threadIdx.x < np)
        const_cast<float*>(p.a_scale)[(int64_t)(row0 + mp + (int)threadIdx.x) * p.lds_a] = s_sx[threadIdx.x];
      // Phase 2: the codes of this workgroup's K range (the union of its
      // wavefronts' step runs) into LDS, 16 codes per thread per trip,
      // with the arithmetic of qmoe_row_quant mode 0 (row_quant.h)
      const int sl0 = blockIdx.y * W, sl1 = sl0 + W - 1;
      qa_s0 = sl0 * q + min(sl0, rem);
      const int qa_s1 = sl1 * q + min(sl1, rem) + q + (sl1 < rem ? 1 : 0);
      const int nc = (qa_s1 - qa_s0) * 8;  // 16-code chunks per row
      qa_rows = np;
      qa_stride = (qa_s1 - qa_s0) * 128 + 16;
      constexpr int kJt = 4;  // 16-code chunks per batch (eight loads)
      for (int i0 = (int)threadIdx.x; i0 < np * nc; i0 += NT * kJt) {
        uint4 v[kJt][2];
#pragma unroll
        for (int jt = 0; jt < kJt; ++jt) {
          const int i = i0 + jt * NT;
          const int rr = i / nc;
          const uint32_t o = i < np * nc ? (uint32_t)((row0 + mp + rr) * lda_b) +
                                               (uint32_t)(qa_s0 * 128 + (i - rr * nc) * 16) * 2u
                                         : kOob;
          const auto t0 = __builtin_amdgcn_raw_buffer_load_b128(xres, o, 0, 0);
          const auto t1 = __builtin_amdgcn_raw_buffer_load_b128(xres, o + 16u, 0, 0);
          v[jt][0] = make_uint4(t0[0], t0[1], t0[2], t0[3]);
          v[jt][1] = make_uint4(t1[0], t1[1], t1[2], t1[3]);
        }
#pragma unroll
        for (int jt = 0; jt < kJt; ++jt) {
          const int i = i0 + jt * NT;
          if (i >= np * nc) continue;
          const int rr = i / nc, c16 = i - rr * nc;
          const float sc = s_sx[rr];
          const uint2 a0 = qmoe_rq::codes8<WF, 0>(qmoe_rq::row8_bf16(v[jt][0]), sc);
          const uint2 a1 = qmoe_rq::codes8<WF, 0>(qmoe_rq::row8_bf16(v[jt][1]), sc);
          *reinterpret_cast<uint4*>(s_codes + rr * qa_stride + c16 * 16) = make_uint4(a0.x, a0.y, a1.x, a1.y);
        }
      }
      __syncthreads();
    }
    if (run) {
      issue_sc(0, ca);
      for (int j = 0; j < nj; j += 2 * U) {
        issue(j + U, cb);
        __builtin_amdgcn_sched_barrier(0);
        consume(j, ca);
        __builtin_amdgcn_sched_barrier(0);
        issue(j + 2 * U, ca);
        __builtin_amdgcn_sched_barrier(0);
        consume(j + U, cb);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // K tail (t = K % 128 valid k, a multiple of 32): a chunk whose k values
    // start past K is loaded with kOob (zeros) and fed as zeros
    if constexpr (!QA) if (tail_mine) {
      const int kk = KSF;
      const int t = p.K - KSF * 128;
      Frag bw[NS];
      Frag fa[MS];
      StepScales<MS, NS> sc;
      const int lc = lane & 3;  // 16 B column of this lane's weight loads
#pragma unroll
      for (int s = 0; s < NS; ++s) {
#pragma unroll
        for (int j = 0; j < Tr::kWBytes / 16; ++j) {
          const uint32_t o = Tr::w_k0(j, lc) < t ? woff[s] + j * 64 : kOob;
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(wres, o, (uint32_t)kk * (4 * Tr::kWBytes), 0);
          bw[s].v[j] = make_uint4(v[0], v[1], v[2], v[3]);
        }
        permute_w<Tr::kWBytes>(bw[s], perm_src);
#pragma unroll
        for (int j = 0; j < Tr::kWBytes / 16; ++j)
          if (Tr::w_k0(j, kg) >= t) bw[s].v[j] = make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
        for (int i = 0; i < Tr::kABytes / 16; ++i) {
          const bool ok = Tr::a_k0(i, kg) < t;
          const uint32_t o = ok ? aoff[ms] + Tr::a_off(i) : kOob;
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(xres, o, (uint32_t)kk * (4 * Tr::kABytes), 0);
          fa[ms].v[i] = ok ? make_uint4(v[0], v[1], v[2], v[3]) : make_uint4(0, 0, 0, 0);
        }
      }
      if constexpr (KIND == QK_W4A16_MX) {
        const bool ok = kg * 32 < t;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const uint32_t b = __builtin_amdgcn_raw_buffer_load_b8(sres, ok ? soffw[s] : kOob, (uint32_t)kk * 4, 0);
          sc.eb[s] = ok ? b : 127u;
        }
      } else if constexpr (KIND == QK_W4A16_NV) {
        // blocks past K read zeros (the weights there are zero as well)
        const uint32_t oob = kg * 32 < t ? 0u : kOob;
#pragma unroll
        for (int s = 0; s < NS; ++s)
          sc.eb[s] = __builtin_amdgcn_raw_buffer_load_b32(sres, soffw[s] | oob, (uint32_t)kk * 16, 0);
      } else if constexpr (KIND == QK_W4A16_I4) {
        // zero weights past K: their scale is read as zero too (0 * 0 + -8 * 0)
        const uint32_t oob = kg * 32 < t ? 0u : kOob;
#pragma unroll
        for (int s = 0; s < NS; ++s)
          sc.eb[s] = __builtin_amdgcn_raw_buffer_load_b16(sres, soffw[s] | oob, (uint32_t)kk * i4_step, 0);
      }
      mma_step<KIND, WF, MS, NS>(acc, fa, bw, sc);
    }

    // ---- reduce the 4 wavefronts' sums (fixed order) ----
    __syncthreads();  // the previous pass has finished reading `red`
    if (wave > 0) {
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float v;
            if constexpr (Tr::kInt) v = __int_as_float(acc.v[ms][s][r]);
            else v = acc.v[ms][s][r];
            red[wave - 1][(ms * NS + s) * 4 + r][lane] = v;
          }
    }
    __syncthreads();
    if (wave != 0) continue;
#pragma unroll
    for (int w = 0; w < W - 1; ++w)
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float v = red[w][(ms * NS + s) * 4 + r][lane];
            if constexpr (Tr::kInt) acc.v[ms][s][r] += __float_as_int(v);
            else acc.v[ms][s][r] += v;
          }
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rr = mp + ms * 16 + kg * 4 + r;
        if (rr >= rows) continue;
        const int R = row0 + rr;
        float v[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          if constexpr (Tr::kInt) v[s] = __int_as_float(acc.v[ms][s][r]);
          else v[s] = acc.v[ms][s][r];
        }
        if (p.ksplit > 1) {
          // raw sums (int32 bit patterns for int8) for the reduce kernel
          float* dst = p.partial + (int64_t)blockIdx.y * plane + (int64_t)R * p.N;
#pragma unroll
          for (int s = 0; s < NS; ++s)
            if (nok[s]) dst[nw[s]] = v[s];
          continue;
        }
        if constexpr (Tr::kInt) {
#pragma unroll
          for (int s = 0; s < NS; ++s) v[s] = (float)acc.v[ms][s][r];
        }
        const int ar = p.a_rows ? p.a_rows[R] : R;
        const float asc = QA ? s_sx[ms * 16 + kg * 4 + r] : 0.0f;
        if (p.y32) {
          // fused decode epilogue: float32 out times the row coefficient,
          // and the row's absolute maximum over this workgroup's columns
          // (one quantization block: 16 * NS columns from a multiple of 32)
          // folded into the block maximum. The 16 lanes of a row share kg,
          // so the row test above is uniform across them.
          const float coef = p.row_coeff ? p.row_coeff[R] : 1.0f;
          float mx = 0.0f;
#pragma unroll
          for (int s = 0; s < (ACT ? NH : NS); ++s) {
            if (!nok[s]) continue;
            float o;
            if constexpr (ACT)
              o = qmoe_act(p.act, finish_elem<KIND, QA>(p, v[s], ar, g, nw[s], asc),
                           finish_elem<KIND, QA>(p, v[s + NH], ar, g, nw[s + NH], asc), p.act_p0, p.act_p1);
            else
              o = finish_elem<KIND, QA>(p, v[s], ar, g, nw[s], asc);
            o = o * coef;
            p.y32[(int64_t)R * p.ldy + nw[s]] = o;
            mx = fmaxf(mx, fabsf(o));
          }
#pragma unroll
          for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
          if (col == 0)
            atomicMax(p.bmax + (int64_t)R * p.ldb + ((tile * (ACT ? 16 * NH : 16 * NS)) >> p.bshift),
                      __float_as_uint(mx));
        } else if (ACT) {
#pragma unroll
          for (int s = 0; s < NH; ++s)
            if (nok[s]) store_out<KIND, true, QA>(p, g, R, ar, nw[s], nw[s], nw[s + NH], v[s], v[s + NH], asc);
        } else {
#pragma unroll
          for (int s = 0; s < NS; ++s)
            if (nok[s]) store_out<KIND, false, QA>(p, g, R, ar, nw[s], nw[s], 0, v[s], 0.0f, asc);
        }
      }
  }
}

// Split-K finish: sum the ksplit slices in order, then the epilogue.
// grid = (ceil(nout / 64), 1, slots); thread = one output column, rows
// strided over the 4 wavefronts.
template <int KIND, int WF, bool ACT>
__global__ __launch_bounds__(kThreads) void skinny_reduce_kernel(const GemmParams p) {
  using Tr = Traits<KIND, WF>;
  int g, row0, rows;
  if (!slot_group(p, blockIdx.z, g, row0, rows)) return;
  const int nout = ACT ? p.N / 2 : p.N;
  const int c = blockIdx.x * 64 + (threadIdx.x & 63);
  if (c >= nout) return;
  const int64_t plane = (int64_t)p.M * p.N;
  for (int r = threadIdx.x >> 6; r < rows; r += kWaves) {
    const int R = row0 + r;
    const float* src = p.partial + (int64_t)R * p.N;
    float v0, v1 = 0.0f;
    if constexpr (Tr::kInt) {
      int s0 = 0, s1 = 0;
      for (int j = 0; j < p.ksplit; ++j) {
        s0 += __float_as_int(src[j * plane + c]);
        if (ACT) s1 += __float_as_int(src[j * plane + p.N / 2 + c]);
      }
      v0 = (float)s0;
      v1 = (float)s1;
    } else {
      float s0 = 0.0f, s1 = 0.0f;
      for (int j = 0; j < p.ksplit; ++j) {
        s0 += src[j * plane + c];
        if (ACT) s1 += src[j * plane + p.N / 2 + c];
      }
      v0 = s0;
      v1 = s1;
    }
    const int ar = p.a_rows ? p.a_rows[R] : R;
    store_out<KIND, ACT>(p, g, R, ar, c, c, ACT ? p.N / 2 + c : c, v0, v1);
  }
}

template <int KIND, int WF, int MS, bool ACT, int NS, bool QA = false>
void launch_skinny(const GemmParams& p, dim3 grid, hipStream_t st, unsigned lds = 0) {
  hipLaunchKernelGGL((skinny_gemm_kernel<KIND, WF, MS, ACT, kUnroll, NS, kWaves, QA>), grid, dim3(kWaves * 64), lds,
                     st, p);
  if (p.ksplit > 1) {
    const int nout = ACT ? p.N / 2 : p.N;
    dim3 rg((unsigned)cdiv(nout, 64), 1, grid.z);
    hipLaunchKernelGGL((skinny_reduce_kernel<KIND, WF, ACT>), rg, dim3(kThreads), 0, st, p);
  }
}

template <int KIND, int WF, bool ACT>
void launch_ms(const GemmParams& p, int ms, int ns, dim3 grid, hipStream_t st) {
  if (ms == 1) {
    if constexpr (KIND == QK_W4A16_MX) {
      if (ns == 4) {
        launch_skinny<KIND, WF, 1, ACT, 4>(p, grid, st);
        return;
      }
    }
    if constexpr (!ACT) {
      if (ns == 1) {
        launch_skinny<KIND, WF, 1, false, 1>(p, grid, st);
        return;
      }
    }
    launch_skinny<KIND, WF, 1, ACT, 2>(p, grid, st);
  } else if (ms == 2) {
    launch_skinny<KIND, WF, 2, ACT, 2>(p, grid, st);
  } else {
    launch_skinny<KIND, WF, 4, ACT, 2>(p, grid, st);
  }
}

// QA (per-channel W8A8 with the activation quantization inside): no fused
// activation, 16 or 32 rows per pass (the host's row limit is below that)
template <int WF>
void launch_qa(const GemmParams& p, int ms, int ns, dim3 grid, hipStream_t st, unsigned lds) {
  if (ms == 1 && ns == 1) launch_skinny<QK_W8A8_PC, WF, 1, false, 1, true>(p, grid, st, lds);
  else if (ms == 1) launch_skinny<QK_W8A8_PC, WF, 1, false, 2, true>(p, grid, st, lds);
  else launch_skinny<QK_W8A8_PC, WF, 2, false, 2, true>(p, grid, st, lds);
}

template <int KIND, int WF>
void launch_act(const GemmParams& p, int ms, int ns, dim3 grid, hipStream_t st) {
  if (p.act != QA_NONE) launch_ms<KIND, WF, true>(p, ms, ns, grid, st);
  else launch_ms<KIND, WF, false>(p, ms, ns, grid, st);
}

// 16-row M tiles per pass for a problem whose groups hold `rows` rows
int skinny_ms(int rows) {
  int ms = rows <= 16 ? 1 : (rows <= 32 ? 2 : 4);
  const char* env_ms = getenv("QMOE_SKINNY_MS");  // tuning knob: 1, 2 or 4
  if (env_ms && (atoi(env_ms) == 1 || atoi(env_ms) == 2 || atoi(env_ms) == 4)) ms = atoi(env_ms);
  return ms;
}

// 16-row weight tiles per workgroup: 2 (measured on MI355X: 4 tiles for
// e2m1 weights gain a few percent on grouped decode and lose a third on
// dense decode, where the workgroup count halves)
int skinny_ns(int kind, int ms, int act) {
  const char* env = getenv("QMOE_SKINNY_NS");  // tuning knob: 1 (no fused activation), 2 or 4 (e2m1)
  const int v = env ? atoi(env) : 2;
  if (ms == 1 && act == QA_NONE && v == 1) return 1;
  if (kind != QK_W4A16_MX || ms != 1) return 2;
  return v == 4 ? 4 : 2;
}

int skinny_tiles(int64_t N, int act, int ns) {
  return act != QA_NONE ? (int)cdiv<int64_t>(N / 2, 8 * ns) : (int)cdiv<int64_t>(N, 16 * ns);
}

}  // namespace

namespace {

struct SkinnyPlan {
  int ksplit;  // K slices over grid.y
  int64_t ws_bytes;
  int ns;      // 16-row weight tiles per workgroup
};

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && atoi(v) > 0 ? atoi(v) : dflt;
}

// Launch shape of the skinny kernel. Measured on MI355X: 4 wavefronts per
// workgroup stream best (8 or 16, i.e. shorter K runs per wavefront, lose
// 10-60%, so only 4 is instantiated); K is split across workgroups only when there are fewer than ~160
// workgroups (one per 32 weight rows), which costs a second launch and the
// [ksplit][M][N] float32 partial sums in the workspace; every wavefront keeps
// at least two 128-k steps.
//
// Weight tiles per workgroup: two 16-row tiles, or one for dense 1-byte
// weights without a fused activation when there is a single row or when
// two-tile workgroups would split K (measured on MI355X: the FP8 down
// projection K 14336, N 4096 at 1 / 8 / 16 rows 13.0 / 14.8 / 16.7 -> 11.0 /
// 12.3 / 12.6 us with one tile, which needs no split and so no second
// launch; 128x128 block FP8 N 18432 at one row 25.2 -> 23.5 us; e2m1
// weights are slower with one tile).
SkinnyPlan skinny_plan(int kind, int64_t M, int64_t N, int64_t K, int act, int slots, int rows,
                       int ksplit_hint) {
  const int ms = skinny_ms(rows);
  const int KS = (int)cdiv<int64_t>(K, 128);
  // tuning knobs (read per call): forced K split, workgroup count the split
  // planner aims for
  const int w = kWaves;
  const int target = env_int("QMOE_SKINNY_TARGET_WG", 160);
  const int ks_env = ksplit_hint > 0 ? ksplit_hint : env_int("QMOE_SKINNY_KSPLIT", 0);
  auto split_for = [&](int ns) {
    int ks = ks_env > 0 ? ks_env : (int)cdiv<int64_t>(target, skinny_tiles(N, act, ns) * std::max(slots, 1));
    return std::max(1, std::min(ks, std::max(1, KS / (2 * w))));
  };
  int ns = skinny_ns(kind, ms, act);
  const bool one_byte_w = kind == QK_W8A8_PC || kind == QK_W8A8_BLK;
  if (!getenv("QMOE_SKINNY_NS") && one_byte_w && ms == 1 && act == QA_NONE && slots == 1 && ns == 2 &&
      (M == 1 || split_for(2) > 1))
    ns = 1;
  const int ksplit = split_for(ns);
  return SkinnyPlan{ksplit, ksplit <= 1 ? 0 : (int64_t)ksplit * M * N * 4, ns};
}

}  // namespace

// Workspace of the skinny kernel for this problem (see skinny_plan).
void qmoe_skinny_plan(int kind, int64_t M, int64_t N, int64_t K, int act, int slots, int rows,
                      int ksplit_hint, int* ksplit_out, int64_t* ws_bytes) {
  const SkinnyPlan pl = skinny_plan(kind, M, N, K, act, slots, rows, ksplit_hint);
  *ksplit_out = pl.ksplit;
  *ws_bytes = pl.ws_bytes;
}

// Whether the skinny kernel takes the problem: QMOE_OK, or QMOE_ERR_ARG for
// shapes outside its envelope (K granule, operands of 2 GiB or more, scale
// alignment), which the generic tiled kernel takes.
int qmoe_skinny_check(int kind, const GemmParams& p) {
  if (p.K <= 0 || (p.K % 32) != 0 || p.N <= 0) return QMOE_ERR_ARG;
  if (p.act != QA_NONE && (p.N % 2) != 0) return QMOE_ERR_ARG;
  if ((kind == QK_W8A8_BLK || kind == QK_W8A16_BLK) && (p.K % 128) != 0) return QMOE_ERR_ARG;
  // 32-bit buffer offsets: every operand stream stays below 2 GiB
  const bool abf16 = kind_abf16(kind) || p.a_quant;
  constexpr int64_t kLim = 0x7fffffff;
  if ((int64_t)p.N * p.ldw > kLim || p.M * p.lda * (abf16 ? 2 : 1) > kLim) return QMOE_ERR_ARG;
  if (kind == QK_W4A16_MX && (int64_t)p.N * p.ldws > kLim) return QMOE_ERR_ARG;
  if (kind == QK_W4A16_NV && ((int64_t)p.N * p.ldws * 2 > kLim || (p.ldws % 2) != 0 ||
                              (reinterpret_cast<uintptr_t>(p.w_scale) & 3) || (p.ws_gstride % 2) != 0))
    return QMOE_ERR_ARG;
  if (kind == QK_W4A16_I4 && ((int64_t)p.N * p.ldws * 2 > kLim || (reinterpret_cast<uintptr_t>(p.w_scale) & 1) ||
                              (p.wq_group != 32 && p.wq_group != 64 && p.wq_group != 128) ||
                              (p.K % p.wq_group) != 0))
    return QMOE_ERR_ARG;
  if (kind == QK_W8A8_BLK &&
      ((int64_t)cdiv(p.N, p.ws_bn) * p.ldws * 4 > kLim || p.M * p.lds_a * 4 > kLim))
    return QMOE_ERR_ARG;
  if (kind == QK_W8A16_BLK && (int64_t)cdiv(p.N, p.ws_bn) * p.ldws * 4 > kLim) return QMOE_ERR_ARG;
  return QMOE_OK;
}

// QA: dynamic LDS of a workgroup's codes, rows x (its K range + 16 bytes);
// a workgroup's range is W wavefront runs of at most ceil(steps / slices)
// 128-k steps each.
int64_t qmoe_skinny_qa_lds(int64_t M, int64_t K, int ksplit) {
  const int64_t ks = cdiv<int64_t>(K, 128);
  const int64_t nsl = (int64_t)std::max(1, ksplit) * kWaves;
  return M * (kWaves * cdiv<int64_t>(ks, nsl) * 128 + 16);
}

// Whether the in-kernel activation quantization takes an M x K problem
// split `ksplit` ways over K (its codes fit the workgroup's LDS).
bool qmoe_skinny_qa_fits(int64_t M, int64_t K, int ksplit) {
  return qmoe_skinny_qa_lds(M, K, ksplit) <= kQaMaxLds;
}

// Token rows one pass of the skinny kernel covers (16, 32 or 64).
int qmoe_skinny_tile_rows(int max_rows) { return 16 * skinny_ms(max_rows); }

// Host-side launcher shared by the dense and MoE entry points.
//   max_rows : rows the M tile is sized for (groups with more rows are
//              still correct, in more passes)
//   slots    : gridDim.z (groups, or the capacity of the active list)
// Returns a QMOE_* status.
int qmoe_skinny_launch(int kind, GemmParams p, int max_rows, int slots, void* workspace,
                       int64_t ws_bytes, int ksplit_hint, hipStream_t st) {
  if (max_rows <= 0 || slots <= 0 || p.M <= 0) return QMOE_OK;
  const int chk = qmoe_skinny_check(kind, p);
  if (chk != QMOE_OK) return chk;
  const int ms = skinny_ms(max_rows);
  const SkinnyPlan pl = skinny_plan(kind, p.M, p.N, p.K, p.act, slots, max_rows, ksplit_hint);
  const int ns = pl.ns;
  const int n_tiles = skinny_tiles(p.N, p.act, ns);
  p.ksplit = pl.ksplit;
  if (pl.ksplit > 1) {
    if (!workspace || ws_bytes < pl.ws_bytes) return QMOE_ERR_WORKSPACE;
    p.partial = static_cast<float*>(workspace);
  }
  dim3 grid(n_tiles, pl.ksplit, slots);
  if (p.row_split) {
    // row slices: one pass each, no K split, and the weight-tile dimension a
    // multiple of the 8 XCDs so that every slice's workgroup of a tile runs
    // on the same XCD (workgroups are dealt to XCDs round robin) and finds
    // the tile's bytes in that XCD's L2
    if (p.group_offs || p.active || p.x0 || p.a_quant || pl.ksplit != 1 || p.row_split > 16 * ms ||
        cdiv(p.M, p.row_split) != slots)
      return QMOE_ERR_ARG;
    grid.x = (unsigned)cdiv(n_tiles, 8) * 8;
  }
  switch (kind) {
    case QK_W8A8_PC:
      if (p.a_quant) {
        const int64_t lds = qmoe_skinny_qa_lds(p.M, p.K, pl.ksplit);
        if (p.act != QA_NONE || ms > 2 || (p.K % 128) != 0 || p.group_offs || lds > kQaMaxLds) return QMOE_ERR_ARG;
        if (p.wfmt == 0) launch_qa<0>(p, ms, ns, grid, st, (unsigned)lds);
        else if (p.wfmt == 1) launch_qa<1>(p, ms, ns, grid, st, (unsigned)lds);
        else launch_qa<2>(p, ms, ns, grid, st, (unsigned)lds);
      } else if (p.wfmt == 0) {
        launch_act<QK_W8A8_PC, 0>(p, ms, ns, grid, st);
      } else if (p.wfmt == 1) {
        launch_act<QK_W8A8_PC, 1>(p, ms, ns, grid, st);
      } else {
        launch_act<QK_W8A8_PC, 2>(p, ms, ns, grid, st);
      }
      break;
    case QK_W8A8_BLK:
      if (p.wfmt == 0) launch_act<QK_W8A8_BLK, 0>(p, ms, ns, grid, st);
      else if (p.wfmt == 1) launch_act<QK_W8A8_BLK, 1>(p, ms, ns, grid, st);
      else launch_act<QK_W8A8_BLK, 2>(p, ms, ns, grid, st);
      break;
    case QK_W8A16_PC: launch_act<QK_W8A16_PC, 0>(p, ms, ns, grid, st); break;
    case QK_W8A16_BLK: launch_act<QK_W8A16_BLK, 0>(p, ms, ns, grid, st); break;
    case QK_W4A16_MX: launch_act<QK_W4A16_MX, 0>(p, ms, ns, grid, st); break;
    case QK_W4A16_NV: launch_act<QK_W4A16_NV, 0>(p, ms, ns, grid, st); break;
    case QK_W4A16_I4: launch_act<QK_W4A16_I4, 0>(p, ms, ns, grid, st); break;
    case QK_W16A16: launch_act<QK_W16A16, 0>(p, ms, ns, grid, st); break;
    default: return QMOE_ERR_ARG;
  }
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
