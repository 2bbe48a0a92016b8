// Skinny (decode) grouped GEMM: at most 64 rows per group, weights streamed
// from HBM exactly once.
//
// Small-M linears and decode MoE are weight-bandwidth bound, so the design
// goal is to keep enough 16-byte weight loads in flight to saturate HBM3E:
//  * workgroup = 4 wavefronts; it owns 32 weight rows (two 16-row MFMA
//    B tiles, or one 16-column gate tile + the matching up tile when an
//    activation is fused) and a slice of K;
//  * K is cut into 128-wide steps; the steps of the workgroup's slice are
//    dealt out to its 4 wavefronts, and further across `ksplit` workgroups
//    (a split-K reduction through a float32 workspace, finished by the last
//    workgroup to arrive, in a fixed order, so results are deterministic);
//  * in a step, lane l reads 32 consecutive k values of weight row (l & 15)
//    (32 B of e4m3/int8, 16 B of e2m1, 64 B of bf16) and 32 k values of
//    activation row (l & 15) of each 16-row M tile, and issues the matching
//    MFMA(s): one v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3), two
//    v_mfma_i32_16x16x64_i8 (int8) or four v_mfma_f32_16x16x32_bf16 (bf16
//    activations; e2m1 weights are expanded with v_cvt_scalef32_pk_bf16_fp4,
//    which also applies the e8m0 block scale, e4m3 with v_cvt_pk_f32_fp8).
//    A and W use the same lane -> k assignment, so the products pair up
//    correctly whatever order the MFMA unit walks k in.
// Rows beyond the group's count and k beyond K are fed as zeros.

#include <algorithm>
#include <type_traits>

#include "gemm_common.h"

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kNSub = 2;  // 16-row weight tiles per workgroup

struct Frag {
  uint4 v[4];
};

template <int KIND, int WF>
struct Traits {
  static constexpr bool kAbf16 = KIND == QK_W8A16_PC || KIND == QK_W4A16_MX || KIND == QK_W16A16;
  static constexpr bool kInt = KIND == QK_W8A8_PC && WF == 1;
  // weight bytes per lane per 128-k step (32 k values)
  static constexpr int kWBytes = KIND == QK_W4A16_MX ? 16 : (KIND == QK_W16A16 ? 64 : 32);
  static constexpr int kABytes = kAbf16 ? 64 : 32;
};

template <int NB>
__device__ __forceinline__ void load_frag(Frag& f, const uint8_t* p, bool ok) {
#pragma unroll
  for (int i = 0; i < NB / 16; ++i) {
    f.v[i] = ok ? reinterpret_cast<const uint4*>(p)[i] : make_uint4(0, 0, 0, 0);
  }
}

__device__ __forceinline__ i32x8 as_i32x8(const Frag& f) {
  i32x8 r;
  r[0] = f.v[0].x; r[1] = f.v[0].y; r[2] = f.v[0].z; r[3] = f.v[0].w;
  r[4] = f.v[1].x; r[5] = f.v[1].y; r[6] = f.v[1].z; r[7] = f.v[1].w;
  return r;
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
__device__ __forceinline__ bf16x8 fp4x8_to_bf16(uint32_t d, float scale) {
  bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 0);
  bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 1);
  bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 2);
  bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 3);
  bf16x8 r;
  r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
  r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
  return r;
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

template <int KIND, int WF, int MS>
struct Acc {
  using T = typename std::conditional<Traits<KIND, WF>::kInt, i32x4, f32x4>::type;
  T v[MS][kNSub];
};

__device__ __forceinline__ float ldf(const float* p) { return *p; }

// Per-format scale + bias for one accumulator element (before activation).
template <int KIND>
__device__ __forceinline__ float finish_elem(const GemmParams& p, float acc, int arow, int g, int n) {
  float v = acc;
  if (KIND == QK_W8A8_PC) {
    v = v * p.a_scale[(int64_t)arow * p.lds_a];
    v = v * static_cast<const float*>(p.w_scale)[(int64_t)g * p.ws_gstride + n];
  } else if (KIND == QK_W8A16_PC) {
    v = v * static_cast<const float*>(p.w_scale)[(int64_t)g * p.ws_gstride + n];
  }
  if (p.bias) v += p.bias[(int64_t)g * p.bias_gstride + n];
  return v;
}

template <int KIND, bool ACT>
__device__ __forceinline__ void store_out(const GemmParams& p, int g, int R, int arow, int ncol_out,
                                          int n0, int n1, float v0, float v1) {
  float out;
  if (ACT) {
    float gte = finish_elem<KIND>(p, v0, arow, g, n0);
    float up = finish_elem<KIND>(p, v1, arow, g, n1);
    out = qmoe_act(p.act, gte, up, p.act_p0, p.act_p1);
  } else {
    out = finish_elem<KIND>(p, v0, arow, g, n0);
  }
  if (p.row_weight) out *= bf16_to_f32(p.row_weight[R]);
  int64_t yr = p.y_rows ? p.y_rows[R] : R;
  p.y[yr * p.ldy + ncol_out] = f32_to_bf16(out);
}

template <int KIND, int WF, int MS, bool ACT>
__device__ __forceinline__ void epilogue_pass(const GemmParams& p, const Acc<KIND, WF, MS>& acc, int g,
                                              int row0, int rows, int mp, int kg, int col, int tile,
                                              const int (&nw)[kNSub], const bool (&nok)[kNSub]) {
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rr = mp + ms * 16 + kg * 4 + r;
      if (rr >= rows) continue;
      const int R = row0 + rr;
      const int ar = p.a_rows ? p.a_rows[R] : R;
      float v0, v1;
      if constexpr (Traits<KIND, WF>::kInt) {
        v0 = (float)acc.v[ms][0][r];
        v1 = (float)acc.v[ms][1][r];
      } else {
        v0 = acc.v[ms][0][r];
        v1 = acc.v[ms][1][r];
      }
      if (ACT) {
        if (nok[0]) store_out<KIND, true>(p, g, R, ar, tile * 16 + col, nw[0], nw[1], v0, v1);
      } else {
        if (nok[0]) store_out<KIND, false>(p, g, R, ar, nw[0], nw[0], 0, v0, 0.0f);
        if (nok[1]) store_out<KIND, false>(p, g, R, ar, nw[1], nw[1], 0, v1, 0.0f);
      }
    }
}

template <int KIND, int WF, int MS, bool ACT>
__global__ __launch_bounds__(kThreads) void skinny_gemm_kernel(const GemmParams p) {
  using Tr = Traits<KIND, WF>;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int kg = lane >> 4;

  const int slot = blockIdx.z;
  int g = slot;
  if (p.active) {
    if (slot >= *p.num_active) return;
    g = p.active[slot];
  }
  const int row0 = p.group_offs ? p.group_offs[g] : 0;
  const int rows = p.group_offs ? p.group_offs[g + 1] - row0 : p.M;
  if (rows <= 0) return;

  // weight rows of the two B tiles
  const int tile = blockIdx.x;
  int nw[kNSub];
  if (ACT) {
    nw[0] = tile * 16 + col;
    nw[1] = (p.N >> 1) + tile * 16 + col;
  } else {
    nw[0] = tile * 32 + col;
    nw[1] = tile * 32 + 16 + col;
  }
  const int nlim = ACT ? (p.N >> 1) : p.N;
  bool nok[kNSub];
  nok[0] = (ACT ? tile * 16 + col : nw[0]) < nlim;
  nok[1] = ACT ? nok[0] : nw[1] < nlim;

  const uint8_t* wg = p.w + (int64_t)g * p.w_gstride;
  const int KS = (p.K + 127) >> 7;
  const int nsl = p.ksplit * kWaves;
  const int sl = blockIdx.y * kWaves + wave;
  const int ks0 = (int)((int64_t)KS * sl / nsl);
  const int ks1 = (int)((int64_t)KS * (sl + 1) / nsl);

  const uint8_t* abase = static_cast<const uint8_t*>(p.a);
  const int64_t lda_b = p.lda * (Tr::kAbf16 ? 2 : 1);
  constexpr int NV = MS * kNSub * 4;
  __shared__ float red[kWaves - 1][NV][64];
  const int64_t plane = (int64_t)p.M * p.N;

  // Rows are taken 16*MS at a time (one pass when the host's row bound
  // holds; more passes re-read this workgroup's weight slice from cache).
  for (int mp = 0; mp < rows; mp += 16 * MS) {
    // activation rows of this lane, per M tile
    int arow[MS];
    bool aok[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      const int r = mp + ms * 16 + col;
      aok[ms] = r < rows;
      const int R = row0 + (aok[ms] ? r : 0);
      arow[ms] = p.a_rows ? p.a_rows[R] : R;
    }

    Acc<KIND, WF, MS> acc;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int s = 0; s < kNSub; ++s) acc.v[ms][s] = {0, 0, 0, 0};

    for (int ks = ks0; ks < ks1; ++ks) {
      const int k0 = ks * 128 + kg * 32;
      const bool kok = k0 < p.K;
      Frag bw[kNSub];
#pragma unroll
      for (int s = 0; s < kNSub; ++s) {
        const int64_t off = (int64_t)nw[s] * p.ldw + (int64_t)k0 * Tr::kWBytes / 32;
        load_frag<Tr::kWBytes>(bw[s], wg + off, kok && nok[s]);
      }
      Frag fa[MS];
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
        const int64_t off = (int64_t)arow[ms] * lda_b + (int64_t)k0 * Tr::kABytes / 32;
        load_frag<Tr::kABytes>(fa[ms], abase + off, kok && aok[ms]);
      }

      if constexpr (KIND == QK_W8A8_PC && WF == 0) {
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
#pragma unroll
          for (int s = 0; s < kNSub; ++s)
            acc.v[ms][s] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                as_i32x8(fa[ms]), as_i32x8(bw[s]), acc.v[ms][s], 0, 0, 0, 127, 0, 127);
      } else if constexpr (KIND == QK_W8A8_PC && WF == 1) {
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
#pragma unroll
          for (int s = 0; s < kNSub; ++s) {
            acc.v[ms][s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                as_i32x4(fa[ms].v[0]), as_i32x4(bw[s].v[0]), acc.v[ms][s], 0, 0, 0);
            acc.v[ms][s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                as_i32x4(fa[ms].v[1]), as_i32x4(bw[s].v[1]), acc.v[ms][s], 0, 0, 0);
          }
      } else if constexpr (KIND == QK_W8A8_BLK) {
        // one 128-k step == one scale block: scale the block's dot, then add
        const int kb = ks;
        float sb[kNSub];
#pragma unroll
        for (int s = 0; s < kNSub; ++s) {
          const int nn = nok[s] ? nw[s] : 0;
          sb[s] = static_cast<const float*>(p.w_scale)[(int64_t)g * p.ws_gstride +
                                                       (int64_t)(nn / p.ws_bn) * p.ldws + kb];
        }
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
          float sa[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int rr = mp + ms * 16 + kg * 4 + r;
            const int R = row0 + (rr < rows ? rr : 0);
            const int ar = p.a_rows ? p.a_rows[R] : R;
            sa[r] = p.a_scale[(int64_t)ar * p.lds_a + kb];
          }
#pragma unroll
          for (int s = 0; s < kNSub; ++s) {
            f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                as_i32x8(fa[ms]), as_i32x8(bw[s]), f32x4{0, 0, 0, 0}, 0, 0, 0, 127, 0, 127);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc.v[ms][s][r] += d[r] * (sa[r] * sb[s]);
          }
        }
      } else {
        // bf16 activations: expand the weight fragment to 4 x 8 bf16
        uint4 wb[kNSub][4];
#pragma unroll
        for (int s = 0; s < kNSub; ++s) {
          if constexpr (KIND == QK_W16A16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) wb[s][q] = bw[s].v[q];
          } else if constexpr (KIND == QK_W8A16_PC) {
            uint32_t d[8] = {bw[s].v[0].x, bw[s].v[0].y, bw[s].v[0].z, bw[s].v[0].w,
                             bw[s].v[1].x, bw[s].v[1].y, bw[s].v[1].z, bw[s].v[1].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              uint2 lo = fp8x4_to_bf16(d[2 * q]);
              uint2 hi = fp8x4_to_bf16(d[2 * q + 1]);
              wb[s][q] = make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
          } else {  // QK_W4A16_MX
            const int nn = nok[s] ? nw[s] : 0;
            const uint8_t* sp = static_cast<const uint8_t*>(p.w_scale) + (int64_t)g * p.ws_gstride +
                                (int64_t)nn * p.ldws + (kok ? (k0 >> 5) : 0);
            const float scl = e8m0_to_f32(*sp);
            uint32_t d[4] = {bw[s].v[0].x, bw[s].v[0].y, bw[s].v[0].z, bw[s].v[0].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              union { bf16x8 b; uint4 u; } c;
              c.b = fp4x8_to_bf16(d[q], scl);
              wb[s][q] = c.u;
            }
          }
        }
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
#pragma unroll
          for (int s = 0; s < kNSub; ++s)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              acc.v[ms][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  as_bf16x8(fa[ms].v[q]), as_bf16x8(wb[s][q]), acc.v[ms][s], 0, 0, 0);
      }
    }

    // ---- reduce the 4 wavefronts' partial sums (fixed order) ----
    __syncthreads();  // the previous pass has finished reading `red`
    if (wave > 0) {
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int s = 0; s < kNSub; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float v;
            if constexpr (Tr::kInt) v = __int_as_float(acc.v[ms][s][r]);
            else v = acc.v[ms][s][r];
            red[wave - 1][(ms * kNSub + s) * 4 + r][lane] = v;
          }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int w = 0; w < kWaves - 1; ++w)
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
#pragma unroll
          for (int s = 0; s < kNSub; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float v = red[w][(ms * kNSub + s) * 4 + r][lane];
              if constexpr (Tr::kInt) acc.v[ms][s][r] += __float_as_int(v);
              else acc.v[ms][s][r] += v;
            }
      if (p.ksplit > 1) {
        // publish this slice's partial sums
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int rr = mp + ms * 16 + kg * 4 + r;
            if (rr >= rows) continue;
            const int64_t base = (int64_t)blockIdx.y * plane + (int64_t)(row0 + rr) * p.N;
#pragma unroll
            for (int s = 0; s < kNSub; ++s) {
              if (!nok[s]) continue;
              float v;
              if constexpr (Tr::kInt) v = __int_as_float(acc.v[ms][s][r]);
              else v = acc.v[ms][s][r];
              p.partial[base + nw[s]] = v;
            }
          }
      } else {
        epilogue_pass<KIND, WF, MS, ACT>(p, acc, g, row0, rows, mp, kg, col, tile, nw, nok);
      }
    }
  }
  if (wave > 0 || p.ksplit <= 1) return;

  // ---- split-K: the last workgroup to arrive sums the slices in order ----
  __threadfence();
  uint32_t* ctr = p.counters + (int64_t)slot * gridDim.x + tile;
  uint32_t prev = 0;
  if (lane == 0) prev = atomicAdd(ctr, 1u);
  prev = __shfl(prev, 0, 64);
  if (prev != (uint32_t)(p.ksplit - 1)) return;
  __threadfence();
  for (int mp = 0; mp < rows; mp += 16 * MS) {
    Acc<KIND, WF, MS> acc;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rr = mp + ms * 16 + kg * 4 + r;
        const int64_t rowoff = (int64_t)(row0 + (rr < rows ? rr : 0)) * p.N;
#pragma unroll
        for (int s = 0; s < kNSub; ++s) {
          const int64_t idx = rowoff + (nok[s] ? nw[s] : 0);
          if constexpr (Tr::kInt) {
            int t = 0;
            for (int j = 0; j < p.ksplit; ++j)
              t += __float_as_int(__builtin_nontemporal_load(&p.partial[j * plane + idx]));
            acc.v[ms][s][r] = t;
          } else {
            float t = 0.0f;
            for (int j = 0; j < p.ksplit; ++j) t += __builtin_nontemporal_load(&p.partial[j * plane + idx]);
            acc.v[ms][s][r] = t;
          }
        }
      }
    epilogue_pass<KIND, WF, MS, ACT>(p, acc, g, row0, rows, mp, kg, col, tile, nw, nok);
  }
  if (lane == 0) *ctr = 0u;  // leave the counter ready for the next call
}

template <int KIND, int WF, int MS, bool ACT>
void launch_skinny(const GemmParams& p, dim3 grid, hipStream_t st) {
  hipLaunchKernelGGL((skinny_gemm_kernel<KIND, WF, MS, ACT>), grid, dim3(kThreads), 0, st, p);
}

template <int KIND, int WF, bool ACT>
void launch_ms(const GemmParams& p, int ms, dim3 grid, hipStream_t st) {
  if (ms == 1) launch_skinny<KIND, WF, 1, ACT>(p, grid, st);
  else if (ms == 2) launch_skinny<KIND, WF, 2, ACT>(p, grid, st);
  else launch_skinny<KIND, WF, 4, ACT>(p, grid, st);
}

template <int KIND, int WF>
void launch_act(const GemmParams& p, int ms, dim3 grid, hipStream_t st) {
  if (p.act != QA_NONE) launch_ms<KIND, WF, true>(p, ms, grid, st);
  else launch_ms<KIND, WF, false>(p, ms, grid, st);
}

}  // namespace

// Split-K workspace layout: a FIXED counter area (so a call never reads as a
// counter what an earlier call of another shape wrote as a partial sum),
// then the float32 partial planes [ksplit][M][N].
constexpr int64_t kCounterBytes = 256 * 1024;
constexpr int64_t kMaxCounters = kCounterBytes / 4;

// Split-K plan of the skinny kernel: the number of K slices and the workspace
// bytes they need.
void qmoe_skinny_plan(int64_t M, int64_t N, int64_t K, int act, int slots, int ksplit_hint,
                      int* ksplit_out, int64_t* ws_bytes) {
  const int n_tiles = act != QA_NONE ? (int)cdiv<int64_t>(N / 2, 16) : (int)cdiv<int64_t>(N, 32);
  const int KS = (int)cdiv<int64_t>(K, 128);
  int ksplit = ksplit_hint;
  if (ksplit <= 0) ksplit = (int)cdiv<int64_t>(1024, (int64_t)n_tiles * std::max(slots, 1));
  ksplit = std::max(1, std::min(ksplit, std::max(1, KS / kWaves)));
  if ((int64_t)n_tiles * slots > kMaxCounters) ksplit = 1;
  *ksplit_out = ksplit;
  *ws_bytes = ksplit <= 1 ? 0 : kCounterBytes + (int64_t)ksplit * M * N * 4;
}

// Host-side launcher shared by the dense and MoE entry points.
//   max_rows : upper bound of rows in any group (<= 64)
//   slots    : gridDim.z (groups, or the capacity of the active list)
// The workspace's counter area must be zero on first use; the kernel leaves
// it zero again. Returns a QMOE_* status.
int qmoe_skinny_launch(int kind, GemmParams p, int max_rows, int slots, void* workspace,
                       int64_t ws_bytes, int ksplit_hint, hipStream_t st) {
  if (max_rows <= 0 || slots <= 0 || p.M <= 0) return QMOE_OK;
  if (max_rows > 64) return QMOE_ERR_ARG;
  if (p.K <= 0 || (p.K % 32) != 0 || p.N <= 0) return QMOE_ERR_ARG;
  if (p.act != QA_NONE && (p.N % 2) != 0) return QMOE_ERR_ARG;
  if (kind == QK_W8A8_BLK && (p.K % 128) != 0) return QMOE_ERR_ARG;
  const int ms = max_rows <= 16 ? 1 : (max_rows <= 32 ? 2 : 4);
  const int n_tiles = p.act != QA_NONE ? cdiv(p.N / 2, 16) : cdiv(p.N, 32);
  int ksplit = 1;
  int64_t need = 0;
  qmoe_skinny_plan(p.M, p.N, p.K, p.act, slots, ksplit_hint, &ksplit, &need);
  p.ksplit = ksplit;
  if (ksplit > 1) {
    if (!workspace || ws_bytes < need) return QMOE_ERR_WORKSPACE;
    p.counters = static_cast<uint32_t*>(workspace);
    p.partial = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kCounterBytes);
  }
  dim3 grid(n_tiles, ksplit, slots);
  switch (kind) {
    case QK_W8A8_PC:
      if (p.wfmt == 0) launch_act<QK_W8A8_PC, 0>(p, ms, grid, st);
      else launch_act<QK_W8A8_PC, 1>(p, ms, grid, st);
      break;
    case QK_W8A8_BLK: launch_act<QK_W8A8_BLK, 0>(p, ms, grid, st); break;
    case QK_W8A16_PC: launch_act<QK_W8A16_PC, 0>(p, ms, grid, st); break;
    case QK_W4A16_MX: launch_act<QK_W4A16_MX, 0>(p, ms, grid, st); break;
    case QK_W16A16: launch_act<QK_W16A16, 0>(p, ms, grid, st); break;
    default: return QMOE_ERR_ARG;
  }
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
