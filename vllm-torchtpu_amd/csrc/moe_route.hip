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

#include "moe_route.h"

namespace {

using namespace qmoe_route;

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
