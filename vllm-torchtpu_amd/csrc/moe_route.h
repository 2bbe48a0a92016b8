// Routing device code: scores -> top-k experts (plain or grouped) ->
// renormalize, scale, for one token per wavefront. Shared by the router
// kernels (moe_route.hip) and the fused decode layer's prep launch, which
// routes a decode step's tokens itself (moe_decode.hip).
#pragma once

#include "moe_common.h"

namespace qmoe_route {

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

// route_token with the scoring rule and grouping chosen at run time (one
// instantiation per slot count for a kernel that serves every rule)
template <int S>
__device__ __forceinline__ void route_token_any(int scoring, bool grouped, const void* __restrict__ logits,
                                                int logits_f32, int64_t t, int E, int topk,
                                                const float* __restrict__ bias, int renormalize, float rsf,
                                                int num_group, int topk_group, uint16_t* __restrict__ out_w,
                                                int32_t* __restrict__ out_ids, float* ch, int32_t* lds_ids,
                                                uint16_t* lds_w) {
#define QMOE_ROUTE_CASE(SC, G)                                                                               \
  route_token<S, SC, G>(logits, logits_f32, t, E, topk, bias, renormalize, rsf, num_group, topk_group, out_w, 0, \
                        out_ids, ch, lds_ids, lds_w)
  switch (scoring * 2 + (grouped ? 1 : 0)) {
    case 0: QMOE_ROUTE_CASE(0, false); break;
    case 1: QMOE_ROUTE_CASE(0, true); break;
    case 2: QMOE_ROUTE_CASE(1, false); break;
    case 3: QMOE_ROUTE_CASE(1, true); break;
    case 4: QMOE_ROUTE_CASE(2, false); break;
    case 5: QMOE_ROUTE_CASE(2, true); break;
    case 6: QMOE_ROUTE_CASE(3, false); break;
    default: QMOE_ROUTE_CASE(3, true); break;
  }
#undef QMOE_ROUTE_CASE
}

// argument checks shared by both entry points
inline int route_args_ok(int64_t T, int E, int topk, int scoring, int num_group, int topk_group) {
  if (T < 0 || E <= 0 || E > kMaxSlots * 64 || topk <= 0 || topk > E || topk > 64) return 0;
  if (scoring < 0 || scoring > 3) return 0;
  const bool grouped = num_group > 1 && topk_group < num_group;
  if (grouped) {
    if (E % num_group != 0 || num_group > 64 || topk_group <= 0) return 0;
    if (topk > topk_group * (E / num_group)) return 0;
  }
  return 1;
}

// slots of a row of E experts, rounded up to an instantiated count
inline int route_slots(int E) {
  const int S = (E + 63) / 64;
  return S <= 1 ? 1 : (S <= 2 ? 2 : (S <= 4 ? 4 : 8));
}

}  // namespace qmoe_route
