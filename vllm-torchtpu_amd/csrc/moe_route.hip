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
// The kernel is instantiated per (slots, scoring rule, grouped). A decode
// step routes one token with one wavefront, so the time is the latency of a
// dependent chain of cross-lane steps: those are DPP moves and readlanes (no
// LDS shuffles), the expert holding a pass's max comes from ballots, and
// lane-dependent choices are selects rather than divergent branches.

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

// The selection compares order keys: the int whose signed order is the
// float order (non-NaN input; -0.0 is taken as +0.0, so equal floats give
// equal keys). Integer max / min need no NaN quieting, so a DPP move folds
// into the max, and uniform keys reduce with scalar instructions.
__device__ __forceinline__ int fkey(float f) {
  const int b = __float_as_int(f + 0.0f);
  return b >= 0 ? b : b ^ 0x7fffffff;
}
__device__ __forceinline__ float kfloat(int k) { return __int_as_float(k >= 0 ? k : k ^ 0x7fffffff); }
constexpr int kMinKey = (int)0x80800000u;  // fkey(-FLT_MAX): taken, or no expert
constexpr int kNoKey = (int)0x80000000u;   // below every key: the empty side of a top-2

__device__ __forceinline__ void top2_merge_k(int& m1, int& m2, int o1, int o2) {
  const int hi = max(m1, o1);
  const int lo = max(min(m1, o1), max(m2, o2));
  m1 = hi;
  m2 = lo;
}

using qmoe_moe::wave_lds_sync;

// Cross-lane steps are DPP moves (a VALU operand, no LDS round trip) and
// v_readlane into scalars. DPP controls used here:
//   0xB1 quad_perm [1,0,3,2] (lane ^ 1), 0x4E quad_perm [2,3,0,1] (lane ^ 2),
//   0x141 row_half_mirror (i <-> 7 - i inside 8 lanes), 0x140 row_mirror
//   (i <-> 15 - i inside a 16-lane row), 0x142 row_bcast:15 (lane 15 of a row
//   to the whole next row), 0x143 row_bcast:31 (lane 31 to rows 2 and 3).
// The first four pair lanes holding disjoint partial results, so after them
// every lane of a row holds the row's result; rows disabled by the row mask
// receive `old`.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_f(float v, float old = 0.0f) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROWS, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp_i(int v, int old = 0) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double lane_d(double v, int l) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Wave-uniform max / sum over all 64 lanes (row all-reduce by DPP, then the
// four row results read into scalars).
__device__ __forceinline__ float wave_max_u(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
__device__ __forceinline__ int wave_max_k(int v) {
  v = max(v, dpp_i<0xB1>(v));
  v = max(v, dpp_i<0x4E>(v));
  v = max(v, dpp_i<0x141>(v));
  v = max(v, dpp_i<0x140>(v));
  return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ float wave_sum_u(float v) {
  v = v + dpp_f<0xB1>(v);
  v = v + dpp_f<0x4E>(v);
  v = v + dpp_f<0x141>(v);
  v = v + dpp_f<0x140>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ double wave_sum_du(double v) {
  v = v + dpp_d<0xB1>(v);
  v = v + dpp_d<0x4E>(v);
  v = v + dpp_d<0x141>(v);
  v = v + dpp_d<0x140>(v);
  return (lane_d(v, 0) + lane_d(v, 16)) + (lane_d(v, 32) + lane_d(v, 48));
}

// Per slot, the lanes that hold an expert (e = 64 * slot + lane < E).
template <int S>
__device__ __forceinline__ void expert_lanes(int E, uint64_t (&vm)[kMaxSlots]) {
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const int n = E - j * 64;
    vm[j] = n >= 64 ? ~0ull : (n <= 0 ? 0ull : ((1ull << n) - 1ull));
  }
}

// One pass of the sort-free top-k over order keys: the row max m
// (wave-uniform) and the lowest expert holding it, found from one ballot per
// slot (the lowest slot with a hit, then its lowest lane). Lanes without an
// expert hold the key of -FLT_MAX and are left out of the ballots, so a real
// expert holding -FLT_MAX wins a tie with them.
template <int S>
__device__ __forceinline__ void top_pass(const int (&cur)[kMaxSlots], const uint64_t (&vm)[kMaxSlots], int& m,
                                         int& mi) {
  int v = cur[0];
#pragma unroll
  for (int j = 1; j < S; ++j) v = max(v, cur[j]);
  m = wave_max_k(v);
  mi = 0x7fffffff;
#pragma unroll
  for (int j = S - 1; j >= 0; --j) {
    const uint64_t b = __ballot(cur[j] == m) & vm[j];
    if (b) mi = j * 64 + (int)__builtin_ctzll(b);
  }
}

// Scores of token t's row, expert e in lane e % 64, slot e / 64 (calling
// wavefront, all lanes): softmax over the row or the elementwise rule, in
// float64 rounded once to float32.
template <int S, int SCORING>
__device__ __forceinline__ void row_scores(const void* __restrict__ logits, int logits_f32, int64_t t, int E,
                                           float (&s)[kMaxSlots]) {
  const int lane = threadIdx.x & 63;
  // every load of the row issued before the first use (the dtype branch is
  // uniform and outside the slot loop); lanes past E load expert E - 1 and
  // drop it
  float x[kMaxSlots];
  if (logits_f32) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int e = j * 64 + lane;
      x[j] = static_cast<const float*>(logits)[t * E + (e < E ? e : E - 1)];
    }
  } else {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int e = j * 64 + lane;
      x[j] = bf16_to_f32(static_cast<const uint16_t*>(logits)[t * E + (e < E ? e : E - 1)]);
    }
  }
#pragma unroll
  for (int j = 0; j < S; ++j)
    if (j * 64 + lane >= E) x[j] = 0.0f;
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
    sum = wave_sum_du(sum);
    const int anynan = __any(nan);
#pragma unroll
    for (int j = 0; j < S; ++j) s[j] = anynan ? __builtin_nanf("") : (float)(ex[j] / sum);
  } else {
#pragma unroll
    for (int j = 0; j < S; ++j) s[j] = score_of<SCORING>(x[j]);
  }
}

constexpr int kChoiceLds = kMaxSlots * 64 + 64;  // floats of LDS scratch per wavefront

// Routes token t with the calling wavefront (all 64 lanes). `ch` is this
// wavefront's LDS scratch of kChoiceLds floats (grouped selection: the
// group scores, and the choice scores when groups are not a power of two).
// When lds_ids is given, the token's ids and bf16 weights also go to
// lds_ids / lds_w [t * topk + j]. The selection is branch-free per lane:
// lane-dependent choices are selects, the remaining branches are uniform.
template <int S, int SCORING, bool GROUPED>
__device__ __forceinline__ void route_token(const void* __restrict__ logits, int logits_f32, int64_t t, int E,
                                            int topk, const float* __restrict__ bias, int renormalize, float rsf,
                                            int num_group, int topk_group, void* __restrict__ out_w, int w_f32,
                                            int32_t* __restrict__ out_ids, float* ch, int32_t* lds_ids,
                                            uint16_t* lds_w) {
  const int lane = threadIdx.x & 63;
  constexpr float kMin = -3.402823466e38f;  // -FLT_MAX
  const int neg_key = fkey(kNeg);

  uint64_t vm[kMaxSlots];
  expert_lanes<S>(E, vm);
  // bias loads issued with the row's loads
  float bv[kMaxSlots];
  if (bias) {
#pragma unroll
    for (int j = 0; j < S; ++j) bv[j] = bias[j * 64 + lane < E ? j * 64 + lane : E - 1];
  }
  float s[kMaxSlots];
  row_scores<S, SCORING>(logits, logits_f32, t, E, s);

  // keys of the choice scores, clamped to >= kNeg (NaN included)
  int cur[kMaxSlots];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const float c = bias ? s[j] + bv[j] : s[j];
    cur[j] = j * 64 + lane < E ? fkey(c > kNeg ? c : kNeg) : kMinKey;
  }

  if constexpr (GROUPED) {
    const int gsize = E / num_group;
    float* gsl = ch + kMaxSlots * 64;  // group scores
    // group score: the top choice score, or the sum of the top two when a
    // correction bias is given
    const bool two = bias != nullptr && gsize >= 2;
    const bool pow2 = gsize <= 64 && (gsize & (gsize - 1)) == 0;
    int gl = 0;
    if (pow2) {
      gl = __builtin_ctz((unsigned)gsize);
      // power-of-two groups are aligned inside a slot: top-2 all-reduce over
      // the group's lanes by DPP (rows, then row_bcast into the later rows),
      // leaving the group's result in its last lane
      int m1[kMaxSlots], m2[kMaxSlots];
#pragma unroll
      for (int j = 0; j < S; ++j) {
        m1[j] = cur[j];
        m2[j] = kNoKey;
      }
#define QMOE_GROUP_STEP(CTRL, ROWS)                                                                  \
  _Pragma("unroll") for (int j = 0; j < S; ++j) {                                                    \
    const int o1 = dpp_i<CTRL, ROWS>(m1[j], kNoKey), o2 = dpp_i<CTRL, ROWS>(m2[j], kNoKey);          \
    top2_merge_k(m1[j], m2[j], o1, o2);                                                              \
  }
      if (gsize > 1) { QMOE_GROUP_STEP(0xB1, 0xF) }
      if (gsize > 2) { QMOE_GROUP_STEP(0x4E, 0xF) }
      if (gsize > 4) { QMOE_GROUP_STEP(0x141, 0xF) }
      if (gsize > 8) { QMOE_GROUP_STEP(0x140, 0xF) }
      if (gsize > 16) { QMOE_GROUP_STEP(0x142, 0xA) }
      if (gsize > 32) { QMOE_GROUP_STEP(0x143, 0x8) }
#undef QMOE_GROUP_STEP
      const bool last = ((lane + 1) & (gsize - 1)) == 0;
#pragma unroll
      for (int j = 0; j < S; ++j) {
        const int g = (j * 64 + lane) >> gl;
        if (last && g < num_group) gsl[g] = two ? kfloat(m1[j]) + kfloat(m2[j]) : kfloat(m1[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < S; ++j)
        if (j * 64 + lane < E) ch[j * 64 + lane] = kfloat(cur[j]);
      wave_lds_sync();
      if (lane < num_group) {
        float m1 = -__builtin_inff(), m2 = -__builtin_inff();
        for (int i = 0; i < gsize; ++i) top2_merge(m1, m2, ch[lane * gsize + i], -__builtin_inff());
        gsl[lane] = two ? m1 + m2 : m1;
      }
    }
    wave_lds_sync();
    // the `topk_group` best groups: rank by (score desc, group asc), scores
    // clamped to >= kNeg -- the set k row-max passes over the groups pick
    const float mine = lane < num_group ? fmaxf(gsl[lane], kNeg) : kMin;
    int rank = 0;
    for (int h = 0; h < num_group; ++h) {
      const float o = fmaxf(gsl[h], kNeg);
      rank += (o > mine || (o == mine && h < lane)) ? 1 : 0;
    }
    const uint64_t kept = __ballot(lane < num_group && rank < topk_group);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int e = j * 64 + lane;
      const int g = pow2 ? (e >> gl) : e / gsize;
      if (e < E && !((kept >> g) & 1)) cur[j] = neg_key;
    }
  }
  const bool gather = bias != nullptr || GROUPED;

  float first = 0.0f;
  float myw = 0.0f;
  int myid = 0;
  for (int p = 0; p < topk; ++p) {
    int mk, mi;
    top_pass<S>(cur, vm, mk, mi);  // wave-uniform results
    const float mv = kfloat(mk);
    if (p == 0) first = mv;
    myid = lane == p ? mi : myid;
    myw = lane == p ? mv : myw;
#pragma unroll
    for (int j = 0; j < S; ++j) cur[j] = j * 64 + lane == mi ? kMinKey : cur[j];
  }
  // weight: the pass value for plain top-k, the unbiased score otherwise
  // (lane p fetches its expert's score from the lane that holds it)
  if (gather) {
    float sv = 0.0f;
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const float v = __shfl(s[j], myid & 63, 64);
      sv = (myid >> 6) == j ? v : sv;
    }
    myw = sv;
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
  __shared__ float choice_lds[GROUPED ? 4 : 1][GROUPED ? kChoiceLds : 1];
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
  __shared__ float choice_lds[GROUPED ? 16 : 1][GROUPED ? kChoiceLds : 1];
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
