// MoE router: scores -> top-k experts (plain or grouped) -> renormalize,
// scale -> (bf16 weights, int32 ids).
//
// Restates `layers/adapter/moe_routing.py:189-323` (select_experts) and the
// sort-free top-k of `layers/core/rowmax_topk.py:28-61`: k passes of
// (row max -> lowest expert attaining it -> mask it), scores <= -3e38 (and
// NaN) clamped to -3e38, a row with no score above that gets NaN weights.
//
// One wavefront per token; expert e lives in lane e % 64, slot e / 64.
// Scores are evaluated in float64 and rounded once to float32 (the correctly
// rounded score), so that a bias-corrected choice score -- compared exactly
// -- is reproducible on any host that evaluates the same definition.
//
// The kernel is instantiated per (slots, scoring rule, grouped): a decode
// step runs it on one CU with a cold instruction cache, so its time is
// mostly instruction fetch, and each instantiation carries only the code of
// its own rule.

#include "moe_common.h"

namespace {

constexpr int kMaxSlots = 8;  // E <= 512
constexpr float kNeg = -3.0e38f;

// scoring rules: 0 softmax (over the row), 1 sigmoid, 2 sqrtsoftplus,
// 3 scores given
template <int SCORING>
__device__ __forceinline__ float score_of(float x) {
  if constexpr (SCORING == 3) {
    return x;
  } else if constexpr (SCORING == 1) {
    return (float)(1.0 / (1.0 + exp(-(double)x)));
  } else {
    // sqrtsoftplus: sqrt(log(1 + e^x)), evaluated stably
    const double d = (double)x;
    const double sp = d > 0.0 ? d + log1p(exp(-d)) : log1p(exp(d));
    return (float)sqrt(sp);
  }
}

// (largest, second largest) of two pairs, duplicates counted
__device__ __forceinline__ void top2_merge(float& m1, float& m2, float o1, float o2) {
  const float hi = fmaxf(m1, o1);
  const float lo = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
  m1 = hi;
  m2 = lo;
}

using qmoe_moe::wave_lds_sync;

// Cross-lane reductions without LDS round trips: DPP moves inside each
// 16-lane row (xor-1 and xor-2 inside quads, then the half-row and row
// mirrors; each step pairs lanes holding disjoint partial results, so every
// lane of a row ends with the row's result), then the four row results read
// into scalars. The results are wave-uniform.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__device__ __forceinline__ float wave_max_u(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

__device__ __forceinline__ int wave_min_u(int v) {
  v = min(v, dpp_i<0xB1>(v));
  v = min(v, dpp_i<0x4E>(v));
  v = min(v, dpp_i<0x141>(v));
  v = min(v, dpp_i<0x140>(v));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

__device__ __forceinline__ float wave_sum_u(float v) {
  v = v + dpp_f<0xB1>(v);
  v = v + dpp_f<0x4E>(v);
  v = v + dpp_f<0x141>(v);
  v = v + dpp_f<0x140>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// (value, index) argmax over the wavefront: largest value, lowest index
// among the lanes holding it (values are never NaN here). Uniform result.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  const float m = wave_max_u(v);
  i = wave_min_u(v == m ? i : 0x7fffffff);
  v = m;
}

// Top-2 all-reduce inside aligned groups of G = 2^n <= 64 lanes.
__device__ __forceinline__ void group_top2(float& m1, float& m2, int G) {
  if (G > 1) top2_merge(m1, m2, dpp_f<0xB1>(m1), dpp_f<0xB1>(m2));
  if (G > 2) top2_merge(m1, m2, dpp_f<0x4E>(m1), dpp_f<0x4E>(m2));
  if (G > 4) top2_merge(m1, m2, dpp_f<0x141>(m1), dpp_f<0x141>(m2));
  if (G > 8) top2_merge(m1, m2, dpp_f<0x140>(m1), dpp_f<0x140>(m2));
  if (G > 16) top2_merge(m1, m2, __shfl_xor(m1, 16, 64), __shfl_xor(m2, 16, 64));
  if (G > 32) top2_merge(m1, m2, __shfl_xor(m1, 32, 64), __shfl_xor(m2, 32, 64));
}

// One rowmax pass over the lane's slots (values already clamped to >= kNeg,
// masked entries hold -FLT_MAX). Returns the wave-wide max and its lowest id.
template <int S>
__device__ __forceinline__ void rowmax_pass(const float (&cur)[kMaxSlots], int lane, int E, float& mv,
                                            int& mi) {
  float v = -3.402823466e38f;
  int idx = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const int e = j * 64 + lane;
    if (e < E && (cur[j] > v)) {
      v = cur[j];
      idx = e;
    }
  }
  // lanes with no expert contribute (-FLT_MAX, INT_MAX); a real expert
  // holding -FLT_MAX ties on value and wins on index
  wave_argmax(v, idx);
  mv = v;
  mi = idx;
}

// Scores of token t's row, expert e in lane e % 64, slot e / 64 (calling
// wavefront, all lanes): softmax over the row or the elementwise rule, in
// float64 rounded once to float32.
template <int S, int SCORING>
__device__ __forceinline__ void row_scores(const void* __restrict__ logits, int logits_f32, int64_t t, int E,
                                           float (&s)[kMaxSlots]) {
  const int lane = threadIdx.x & 63;
  float x[kMaxSlots];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const int e = j * 64 + lane;
    float v = 0.0f;
    if (e < E) {
      v = logits_f32 ? static_cast<const float*>(logits)[t * E + e]
                     : bf16_to_f32(static_cast<const uint16_t*>(logits)[t * E + e]);
    }
    x[j] = v;
  }
  if constexpr (SCORING == 0) {  // softmax in float64
    float mx = -__builtin_inff();
    bool nan = false;
#pragma unroll
    for (int j = 0; j < S; ++j)
      if (j * 64 + lane < E) {
        nan |= x[j] != x[j];
        mx = fmaxf(mx, x[j]);
      }
    mx = wave_max_u(mx);
    double ex[kMaxSlots];
    double sum = 0.0;
#pragma unroll
    for (int j = 0; j < S; ++j) {
      ex[j] = (j * 64 + lane < E) ? exp((double)x[j] - (double)mx) : 0.0;
      sum += ex[j];
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    const int anynan = __any(nan);
#pragma unroll
    for (int j = 0; j < S; ++j) s[j] = anynan ? __builtin_nanf("") : (float)(ex[j] / sum);
  } else {
#pragma unroll
    for (int j = 0; j < S; ++j) s[j] = score_of<SCORING>(x[j]);
  }

}

// Routes token t with the calling wavefront (all 64 lanes). `ch` is this
// wavefront's LDS scratch (kMaxSlots * 64 floats, grouped selection with
// groups that are not a power of two <= 64). When lds_ids is given, the
// token's ids and bf16 weights also go to lds_ids / lds_w [t * topk + j].
template <int S, int SCORING, bool GROUPED>
__device__ __forceinline__ void route_token(const void* __restrict__ logits, int logits_f32, int64_t t, int E,
                                            int topk, const float* __restrict__ bias, int renormalize, float rsf,
                                            int num_group, int topk_group, void* __restrict__ out_w, int w_f32,
                                            int32_t* __restrict__ out_ids, float* ch, int32_t* lds_ids,
                                            uint16_t* lds_w) {
  const int lane = threadIdx.x & 63;

  float s[kMaxSlots];
  row_scores<S, SCORING>(logits, logits_f32, t, E, s);

  // choice scores
  float c[kMaxSlots];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const int e = j * 64 + lane;
    c[j] = (bias && e < E) ? s[j] + bias[e] : s[j];
  }

  float cur[kMaxSlots];
#pragma unroll
  for (int j = 0; j < S; ++j) cur[j] = c[j] > kNeg ? c[j] : kNeg;

  if constexpr (GROUPED) {
    const int gsize = E / num_group;
    // group score: the top choice score, or the sum of the top two when a
    // correction bias is given
    float gs = -3.402823466e38f;
    if (gsize <= 64 && (gsize & (gsize - 1)) == 0) {
      // power-of-two groups inside a slot: top-2 by a butterfly over the
      // group's lanes, then lane g fetches group g's result
      float res[S];
#pragma unroll
      for (int j = 0; j < S; ++j) {
        float m1 = j * 64 + lane < E ? cur[j] : -__builtin_inff();
        float m2 = -__builtin_inff();
        group_top2(m1, m2, gsize);
        res[j] = bias ? (gsize >= 2 ? m1 + m2 : m1) : m1;
      }
      const int first = (lane < num_group ? lane : 0) * gsize;  // group's first expert
      float v = 0.0f;
#pragma unroll
      for (int j = 0; j < S; ++j) {
        const float r = __shfl(res[j], first & 63, 64);
        if (j == (first >> 6)) v = r;
      }
      if (lane < num_group) gs = v;
    } else {
#pragma unroll
      for (int j = 0; j < S; ++j)
        if (j * 64 + lane < E) ch[j * 64 + lane] = cur[j];
      wave_lds_sync();
      if (lane < num_group) {
        float m1 = -__builtin_inff(), m2 = -__builtin_inff();
        for (int i = 0; i < gsize; ++i) top2_merge(m1, m2, ch[lane * gsize + i], -__builtin_inff());
        gs = bias ? (gsize >= 2 ? m1 + m2 : m1) : m1;
      }
    }
    // top `topk_group` groups (rowmax order over group scores)
    float gcur = lane < num_group ? (gs > kNeg ? gs : kNeg) : -3.402823466e38f;
    bool keep = false;
    for (int p = 0; p < topk_group; ++p) {
      float v = gcur;
      int i = lane < num_group ? lane : 0x7fffffff;
      wave_argmax(v, i);
      if (lane == i) {
        keep = true;
        gcur = -3.402823466e38f;
      }
    }
    const uint64_t kept_groups = __ballot(keep);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int e = j * 64 + lane;
      if (e < E && !((kept_groups >> (e / gsize)) & 1)) cur[j] = kNeg;
    }
  }
  const bool gather = bias != nullptr || GROUPED;

  float first = 0.0f;
  float myw = 0.0f;
  int myid = 0;
  for (int p = 0; p < topk; ++p) {
    float mv;
    int mi;
    rowmax_pass<S>(cur, lane, E, mv, mi);  // wave-uniform results
    if (p == 0) first = mv;
    // weight: the pass value for plain top-k, the unbiased score otherwise
    float w = mv;
    if (gather) {
      const int src_slot = mi >> 6;
      float sv = 0.0f;
#pragma unroll
      for (int j = 0; j < S; ++j)
        if (j == src_slot) sv = s[j];
      w = lane_f(sv, mi & 63);
    }
    if (lane == p) {
      myid = mi;
      myw = w;
    }
#pragma unroll
    for (int j = 0; j < S; ++j)
      if (j * 64 + lane == mi) cur[j] = -3.402823466e38f;
  }
  if (lane < topk) out_ids[t * topk + lane] = myid;
  // a plain top-k row with no score above the sentinel is poisoned (NaN)
  if (!gather && first <= kNeg) myw = __builtin_nanf("");
  const float sum = wave_sum_u(lane < topk ? myw : 0.0f);
  if (lane < topk) {
    float v = myw;
    if (renormalize) v = v / (sum != sum ? sum : fmaxf(sum, 1e-20f));
    if (rsf != 1.0f) v = v * rsf;
    if (w_f32) {
      static_cast<float*>(out_w)[t * topk + lane] = v;
    } else {
      const uint16_t b = f32_to_bf16(v);
      static_cast<uint16_t*>(out_w)[t * topk + lane] = b;
      if (lds_w) lds_w[t * topk + lane] = b;
    }
    if (lds_ids) lds_ids[t * topk + lane] = myid;
  }
}

template <int S, int SCORING, bool GROUPED>
__global__ __launch_bounds__(256) void route_kernel(const void* __restrict__ logits, int logits_f32,
                                                    int64_t T, int E, int topk,
                                                    const float* __restrict__ bias, int renormalize,
                                                    float rsf, int num_group, int topk_group,
                                                    void* __restrict__ out_w, int w_f32,
                                                    int32_t* __restrict__ out_ids) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  __shared__ float choice_lds[GROUPED ? 4 : 1][GROUPED ? kMaxSlots * 64 : 1];
  if (t >= T) return;
  route_token<S, SCORING, GROUPED>(logits, logits_f32, t, E, topk, bias, renormalize, rsf, num_group, topk_group,
                                   out_w, w_f32, out_ids, choice_lds[GROUPED ? threadIdx.x >> 6 : 0], nullptr,
                                   nullptr);
}

// Decode form of routing + dispatch in one launch (T <= 16 tokens, T * topk
// <= 64 routes): one workgroup, wavefront t routes token t (ids and bf16
// weights to global and to LDS), then wavefront 0 runs the single-wavefront
// dispatch on the routes in LDS.
template <int S, int SCORING, bool GROUPED>
__global__ __launch_bounds__(1024) void route_dispatch_kernel(
    const void* __restrict__ logits, int logits_f32, int T, int E, int topk, const float* __restrict__ bias,
    int renormalize, float rsf, int num_group, int topk_group, uint16_t* __restrict__ out_w,
    int32_t* __restrict__ out_ids, int skip_padded, int32_t* __restrict__ sorted_idx, int32_t* __restrict__ revert,
    int32_t* __restrict__ token_sorted, int32_t* __restrict__ group_offs, int32_t* __restrict__ active,
    int32_t* __restrict__ num_active, uint16_t* __restrict__ sorted_weight) {
  __shared__ float choice_lds[GROUPED ? 16 : 1][GROUPED ? kMaxSlots * 64 : 1];
  __shared__ int32_t s_ids[64];
  __shared__ uint16_t s_w[64];
  __shared__ int cnt[64 * qmoe_moe::kPer];
  __shared__ int offs[64 * qmoe_moe::kPer];
  const int wave = threadIdx.x >> 6;
  route_token<S, SCORING, GROUPED>(logits, logits_f32, wave, E, topk, bias, renormalize, rsf, num_group, topk_group,
                                   out_w, 0, out_ids, choice_lds[GROUPED ? wave : 0], s_ids, s_w);
  __syncthreads();
  if (wave == 0)
    qmoe_moe::dispatch_wave(s_ids, s_w, T * topk, topk, E, skip_padded, sorted_idx, revert, token_sorted,
                            group_offs, active, num_active, sorted_weight, cnt, offs);
}

// FUSED: the route + dispatch kernel, one workgroup of 64 * grid.x threads
template <int S, int SCORING, bool GROUPED, bool FUSED = false, typename... A>
void launch_route3(dim3 grid, hipStream_t st, A... a) {
  if constexpr (FUSED)
    hipLaunchKernelGGL((route_dispatch_kernel<S, SCORING, GROUPED>), dim3(1), dim3(64 * grid.x), 0, st, a...);
  else
    hipLaunchKernelGGL((route_kernel<S, SCORING, GROUPED>), grid, dim3(256), 0, st, a...);
}

template <int S, bool FUSED, typename... A>
void launch_route2(int scoring, bool grouped, dim3 grid, hipStream_t st, A... a) {
  switch (scoring * 2 + (grouped ? 1 : 0)) {
    case 0: launch_route3<S, 0, false, FUSED>(grid, st, a...); break;
    case 1: launch_route3<S, 0, true, FUSED>(grid, st, a...); break;
    case 2: launch_route3<S, 1, false, FUSED>(grid, st, a...); break;
    case 3: launch_route3<S, 1, true, FUSED>(grid, st, a...); break;
    case 4: launch_route3<S, 2, false, FUSED>(grid, st, a...); break;
    case 5: launch_route3<S, 2, true, FUSED>(grid, st, a...); break;
    case 6: launch_route3<S, 3, false, FUSED>(grid, st, a...); break;
    default: launch_route3<S, 3, true, FUSED>(grid, st, a...); break;
  }
}

template <bool FUSED = false, typename... A>
void launch_route(int S, int scoring, bool grouped, dim3 grid, hipStream_t st, A... a) {
  if (S == 1) launch_route2<1, FUSED>(scoring, grouped, grid, st, a...);
  else if (S == 2) launch_route2<2, FUSED>(scoring, grouped, grid, st, a...);
  else if (S == 4) launch_route2<4, FUSED>(scoring, grouped, grid, st, a...);
  else launch_route2<8, FUSED>(scoring, grouped, grid, st, a...);
}

// DeepSeek-V4 hash routing, `layers/adapter/moe_routing.py:204-229`
// (_hash_moe_select): the ids are the table row of the token's input id,
// the weights the row's scores at those ids (no bias), renormalized and
// scaled. One wavefront per token; lane j < topk owns route j.
template <int S, int SCORING>
__global__ __launch_bounds__(256) void route_hash_kernel(const void* __restrict__ logits, int logits_f32, int64_t T,
                                                         int E, int topk, const int32_t* __restrict__ table,
                                                         int64_t table_rows, const void* __restrict__ input_ids,
                                                         int ids_i64,
                                                         int renormalize, float rsf, uint16_t* __restrict__ out_w,
                                                         int32_t* __restrict__ out_ids) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float s[kMaxSlots];
  row_scores<S, SCORING>(logits, logits_f32, t, E, s);
  // an input id outside the table, or a table entry outside [0, E), gives
  // the invalid route id -1 with a NaN weight (the dispatch sorts it last)
  int id = 0;
  bool ok = false;
  if (lane < topk) {
    const int64_t row = ids_i64 ? static_cast<const int64_t*>(input_ids)[t] : static_cast<const int32_t*>(input_ids)[t];
    if (row >= 0 && row < table_rows) {
      id = table[row * topk + lane];
      ok = id >= 0 && id < E;
    }
  }
  const int idc = ok ? id : 0;
  float w = 0.0f;
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const float v = __shfl(s[j], idc & 63, 64);
    if ((idc >> 6) == j) w = v;
  }
  if (!ok) w = __builtin_nanf("");
  const float sum = wave_sum_u(lane < topk ? w : 0.0f);
  if (lane < topk) {
    float v = w;
    if (renormalize) v = v / (sum != sum ? sum : fmaxf(sum, 1e-20f));
    if (rsf != 1.0f) v = v * rsf;
    out_w[t * topk + lane] = f32_to_bf16(v);
    out_ids[t * topk + lane] = ok ? id : -1;
  }
}

template <int S>
void launch_hash2(int scoring, dim3 grid, hipStream_t st, const void* logits, int logits_f32, int64_t T, int E,
                  int topk, const int32_t* table, int64_t table_rows, const void* input_ids, int ids_i64,
                  int renormalize, float rsf, uint16_t* out_w, int32_t* out_ids) {
#define QMOE_HASH(SC)                                                                                            \
  hipLaunchKernelGGL((route_hash_kernel<S, SC>), grid, dim3(256), 0, st, logits, logits_f32, T, E, topk, table, \
                     table_rows, input_ids, ids_i64, renormalize, rsf, out_w, out_ids)
  if (scoring == 0) QMOE_HASH(0);
  else if (scoring == 1) QMOE_HASH(1);
  else if (scoring == 2) QMOE_HASH(2);
  else QMOE_HASH(3);
#undef QMOE_HASH
}

// argument checks shared by both entry points
int route_args_ok(int64_t T, int E, int topk, int scoring, int num_group, int topk_group) {
  if (T < 0 || E <= 0 || E > kMaxSlots * 64 || topk <= 0 || topk > E || topk > 64) return 0;
  if (scoring < 0 || scoring > 3) return 0;
  const bool grouped = num_group > 1 && topk_group < num_group;
  if (grouped) {
    if (E % num_group != 0 || num_group > 64 || topk_group <= 0) return 0;
    if (topk > topk_group * (E / num_group)) return 0;
  }
  return 1;
}

}  // namespace

extern "C" int qmoe_moe_route(const void* logits, int logits_f32, int64_t T, int E, int topk,
                              int scoring, const float* bias, int renormalize,
                              float routed_scaling_factor, int num_group, int topk_group,
                              void* topk_weights, int weights_f32, int32_t* topk_ids,
                              hipStream_t stream) {
  if (!route_args_ok(T, E, topk, scoring, num_group, topk_group)) return QMOE_ERR_ARG;
  const bool grouped = num_group > 1 && topk_group < num_group;
  if (T == 0) return QMOE_OK;
  const int S = (E + 63) / 64;
  launch_route(S <= 1 ? 1 : (S <= 2 ? 2 : (S <= 4 ? 4 : 8)), scoring, grouped, dim3((unsigned)((T + 3) / 4)),
               stream, logits, logits_f32, T, E, topk, bias, renormalize, routed_scaling_factor, num_group,
               topk_group, topk_weights, weights_f32, topk_ids);
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}

// See include/qmoe.h for the contract.
extern "C" int qmoe_moe_route_dispatch(const void* logits, int logits_f32, int64_t T, int E, int topk, int scoring,
                                       const float* bias, int renormalize, float routed_scaling_factor,
                                       int num_group, int topk_group, uint16_t* topk_weights, int32_t* topk_ids,
                                       int skip_padded, int32_t* sorted_idx, int32_t* revert,
                                       int32_t* token_sorted, int32_t* group_offs, int32_t* active,
                                       int32_t* num_active, uint16_t* sorted_weight, hipStream_t stream) {
  if (!route_args_ok(T, E, topk, scoring, num_group, topk_group)) return QMOE_ERR_ARG;
  if (T < 1 || T > 16 || T * topk > 64 || E > qmoe_moe::kMaxE) return QMOE_ERR_ARG;
  const bool grouped = num_group > 1 && topk_group < num_group;
  const int S = (E + 63) / 64;
  launch_route<true>(S <= 1 ? 1 : (S <= 2 ? 2 : (S <= 4 ? 4 : 8)), scoring, grouped, dim3((unsigned)T), stream,
                     logits, logits_f32, (int)T, E, topk, bias, renormalize, routed_scaling_factor, num_group,
                     topk_group, topk_weights, topk_ids, skip_padded, sorted_idx, revert, token_sorted,
                     group_offs, active, num_active, sorted_weight);
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}

// See include/qmoe.h for the contract.
extern "C" int qmoe_moe_route_hash(const void* logits, int logits_f32, int64_t T, int E, int topk, int scoring,
                                   const int32_t* hash_table, int64_t table_rows, const void* input_ids,
                                   int ids_i64, int renormalize,
                                   float routed_scaling_factor, uint16_t* topk_weights, int32_t* topk_ids,
                                   hipStream_t stream) {
  if (!route_args_ok(T, E, topk, scoring, 1, 1) || !hash_table || !input_ids) return QMOE_ERR_ARG;
  if (T == 0) return QMOE_OK;
  const int S = (E + 63) / 64;
  const dim3 grid((unsigned)((T + 3) / 4));
  const int Sp = S <= 1 ? 1 : (S <= 2 ? 2 : (S <= 4 ? 4 : 8));
#define QMOE_HASH_S(SS)                                                                                        \
  launch_hash2<SS>(scoring, grid, stream, logits, logits_f32, T, E, topk, hash_table, table_rows, input_ids, \
                   ids_i64, renormalize, routed_scaling_factor, topk_weights, topk_ids)
  if (Sp == 1) QMOE_HASH_S(1);
  else if (Sp == 2) QMOE_HASH_S(2);
  else if (Sp == 4) QMOE_HASH_S(4);
  else QMOE_HASH_S(8);
#undef QMOE_HASH_S
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
