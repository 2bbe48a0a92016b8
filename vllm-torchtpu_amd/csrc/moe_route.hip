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

#include "qmoe_common.h"

namespace {

constexpr int kMaxSlots = 8;  // E <= 512
constexpr float kNeg = -3.0e38f;

__device__ __forceinline__ float score_of(float x, int scoring) {
  if (scoring == 3) return x;  // scores given
  double d = (double)x;
  if (scoring == 1) return (float)(1.0 / (1.0 + exp(-d)));
  // sqrtsoftplus: sqrt(log(1 + e^x)), evaluated stably
  double sp = d > 0.0 ? d + log1p(exp(-d)) : log1p(exp(d));
  return (float)sqrt(sp);
}

// Make this wavefront's LDS writes visible to its own later LDS reads.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// (value, index) argmax over the wavefront: largest value, lowest index.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(v, o, 64);
    int oi = __shfl_xor(i, o, 64);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
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

template <int S>
__global__ __launch_bounds__(256) void route_kernel(const void* __restrict__ logits, int logits_f32,
                                                    int64_t T, int E, int topk, int scoring,
                                                    const float* __restrict__ bias, int renormalize,
                                                    float rsf, int num_group, int topk_group,
                                                    void* __restrict__ out_w, int w_f32,
                                                    int32_t* __restrict__ out_ids) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  __shared__ float choice_lds[4][kMaxSlots * 64];
  if (t >= T) return;
  float* ch = choice_lds[threadIdx.x >> 6];

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
  float s[kMaxSlots];
  if (scoring == 0) {  // softmax in float64
    float mx = -__builtin_inff();
    bool nan = false;
#pragma unroll
    for (int j = 0; j < S; ++j)
      if (j * 64 + lane < E) {
        nan |= x[j] != x[j];
        mx = fmaxf(mx, x[j]);
      }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
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
    for (int j = 0; j < S; ++j) s[j] = score_of(x[j], scoring);
  }

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

  if (num_group > 1 && topk_group < num_group) {
    const int gsize = E / num_group;
#pragma unroll
    for (int j = 0; j < S; ++j)
      if (j * 64 + lane < E) ch[j * 64 + lane] = cur[j];
    wave_lds_sync();
    float gs = -3.402823466e38f;
    if (lane < num_group) {
      float m1 = -__builtin_inff(), m2 = -__builtin_inff();
      for (int i = 0; i < gsize; ++i) {
        const float v = ch[lane * gsize + i];
        if (v > m1) {
          m2 = m1;
          m1 = v;
        } else if (v > m2) {
          m2 = v;
        }
      }
      gs = bias ? (gsize >= 2 ? m1 + m2 : m1) : m1;
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
    const int keep_i = keep ? 1 : 0;
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int e = j * 64 + lane;
      const int kept = __shfl(keep_i, e < E ? e / gsize : 0, 64);
      if (e < E && !kept) cur[j] = kNeg;
    }
  }
  const bool gather = bias != nullptr || (num_group > 1 && topk_group < num_group);

  float first = 0.0f;
  float myw = 0.0f;
  for (int p = 0; p < topk; ++p) {
    float mv;
    int mi;
    rowmax_pass<S>(cur, lane, E, mv, mi);
    if (p == 0) first = mv;
    // weight: the pass value for plain top-k, the unbiased score otherwise
    float w = mv;
    if (gather) {
      const int src_lane = mi & 63;
      const int src_slot = mi >> 6;
      float sv = 0.0f;
#pragma unroll
      for (int j = 0; j < S; ++j)
        if (j == src_slot) sv = s[j];
      w = __shfl(sv, src_lane, 64);
    }
    if (lane == p) {
      out_ids[t * topk + p] = mi;
      myw = w;
    }
#pragma unroll
    for (int j = 0; j < S; ++j)
      if (j * 64 + lane == mi) cur[j] = -3.402823466e38f;
  }
  // a plain top-k row with no score above the sentinel is poisoned (NaN)
  if (!gather && first <= kNeg) myw = __builtin_nanf("");
  float sum = lane < topk ? myw : 0.0f;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if (lane < topk) {
    float v = myw;
    if (renormalize) v = v / (sum != sum ? sum : fmaxf(sum, 1e-20f));
    if (rsf != 1.0f) v = v * rsf;
    if (w_f32) static_cast<float*>(out_w)[t * topk + lane] = v;
    else static_cast<uint16_t*>(out_w)[t * topk + lane] = f32_to_bf16(v);
  }
}

}  // namespace

extern "C" int qmoe_moe_route(const void* logits, int logits_f32, int64_t T, int E, int topk,
                              int scoring, const float* bias, int renormalize,
                              float routed_scaling_factor, int num_group, int topk_group,
                              void* topk_weights, int weights_f32, int32_t* topk_ids,
                              hipStream_t stream) {
  if (T < 0 || E <= 0 || E > kMaxSlots * 64 || topk <= 0 || topk > E || topk > 64) return QMOE_ERR_ARG;
  if (scoring < 0 || scoring > 3) return QMOE_ERR_ARG;
  const bool grouped = num_group > 1 && topk_group < num_group;
  if (grouped) {
    if (E % num_group != 0 || num_group > 64 || topk_group <= 0) return QMOE_ERR_ARG;
    if (topk > topk_group * (E / num_group)) return QMOE_ERR_ARG;
  }
  if (T == 0) return QMOE_OK;
  const int S = (E + 63) / 64;
  dim3 grid((unsigned)((T + 3) / 4));
#define QMOE_ROUTE(SS)                                                                              \
  hipLaunchKernelGGL((route_kernel<SS>), grid, dim3(256), 0, stream, logits, logits_f32, T, E, topk, \
                     scoring, bias, renormalize, routed_scaling_factor, num_group, topk_group,      \
                     topk_weights, weights_f32, topk_ids)
  if (S <= 1) QMOE_ROUTE(1);
  else if (S <= 2) QMOE_ROUTE(2);
  else if (S <= 4) QMOE_ROUTE(4);
  else QMOE_ROUTE(8);
#undef QMOE_ROUTE
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
