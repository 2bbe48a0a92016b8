// Single-wavefront MoE dispatch (T*k <= 64 routes), shared by the dispatch
// entry point (moe_dispatch.hip) and the fused route + dispatch kernel
// (moe_route.hip).
#pragma once

#include "qmoe_common.h"

namespace qmoe_moe {

constexpr int kMaxE = 512;
constexpr int kMaxB = kMaxE + 1;          // + the "invalid" bucket
constexpr int kPer = (kMaxB + 63) / 64;   // buckets per lane

// Make this wavefront's LDS writes visible to its own later LDS reads.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Exclusive prefix sum over the wavefront (and the total), by DPP: row_shr
// 1, 2, 4, 8 inside each 16-lane row (lanes whose source falls outside the
// row add the `old` 0), then row_bcast:15 adds a row's last lane to the next
// row (rows 1, 3) and row_bcast:31 adds lane 31 to rows 2 and 3.
__device__ __forceinline__ int wave_excl_scan(int v, int lane, int& total) {
  (void)lane;
  int x = v;
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
  total = __builtin_amdgcn_readlane(x, 63);
  return x - v;
}

// Restates `layers/core/fused_moe_gmm.py:288-408` (prepare_routed_gmm_inputs)
// for at most 64 routes, run by ONE whole wavefront (lane = route f): bucket
// counts by LDS atomics; lane l owns buckets kPer*l .. kPer*l + kPer-1, whose
// exclusive prefix gives the group offsets and the active list; a route's
// rank is its bucket's offset plus the routes of the same bucket in lower
// lanes (ballot match), i.e. the stable order. `ids` and `wts` may point to
// global memory or LDS; cnt and offs are LDS scratch of 64 * kPer ints.
__device__ __forceinline__ void dispatch_wave(const int32_t* ids, const uint16_t* wts, int Nf, int topk, int E,
                                              int skip_padded, int32_t* sorted_idx, int32_t* revert,
                                              int32_t* token_sorted, int32_t* group_offs, int32_t* active,
                                              int32_t* num_active, uint16_t* sorted_weight, int* cnt, int* offs) {
  const int lane = threadIdx.x & 63;
  const bool in = lane < Nf;
  int b = 0;
  uint16_t w = 0;
  if (in) {
    const int id = ids[lane];
    w = wts[lane];
    bool ok = id >= 0 && id < E;
    if (skip_padded && ok) ok = (w & 0x7fffu) != 0;
    b = ok ? id : E;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) cnt[lane * kPer + j] = 0;
  wave_lds_sync();
  if (in) atomicAdd(&cnt[b], 1);
  wave_lds_sync();
  int c[kPer], pre[kPer], t = 0, fa = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    c[j] = cnt[lane * kPer + j];
    pre[j] = t;
    t += c[j];
    fa += (lane * kPer + j < E && c[j] > 0) ? 1 : 0;
  }
  int total = 0, nact = 0;
  const int base = wave_excl_scan(t, lane, total);
  int apos = wave_excl_scan(fa, lane, nact);
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * kPer + j;
    offs[e] = base + pre[j];
    if (e <= E) group_offs[e] = base + pre[j];  // group_offs[E] = valid routes
    if (e < E && c[j] > 0) active[apos++] = e;
  }
  if (lane == 0) *num_active = nact;
  wave_lds_sync();
  // routes of the same bucket in lower lanes (10 ballots resolve a bucket id)
  uint64_t m = __ballot(in);
#pragma unroll
  for (int bit = 0; bit < 10; ++bit) {
    const bool s = (b >> bit) & 1;
    const uint64_t bal = __ballot(s);
    m &= s ? bal : ~bal;
  }
  const uint64_t lower = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  if (in) {
    const int rank = offs[b] + __popcll(m & lower);
    sorted_idx[rank] = lane;
    revert[lane] = rank;
    token_sorted[rank] = lane / topk;
    sorted_weight[rank] = w;
  }
}

}  // namespace qmoe_moe
