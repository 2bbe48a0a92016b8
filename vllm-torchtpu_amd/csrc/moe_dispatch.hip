// MoE token permutation (dispatch) and weighted unpermute (combine).
//
// Dispatch restates `layers/core/fused_moe_gmm.py:288-408`
// (prepare_routed_gmm_inputs, non-EP): routes are ordered by expert with a
// STABLE tie order by flat route index f = t*k + slot (the reference's stable
// argsort / single packed sort), invalid routes last. It is one workgroup of
// 1024 threads doing histogram (LDS atomics), exclusive scan, and a stable
// scatter. LDS atomics alone would give a nondeterministic order, so the
// scatter walks the routes in chunks of 1024 and ranks equal buckets inside
// a wavefront with a ballot match (10 ballots resolve a 10-bit bucket id),
// across wavefronts with per-wave counts, and across chunks with a running
// base per bucket.
//
// Many routes (prefill): the same order from three launches over chunks of
// the routes (1024 each, the last one taking the remainder, so every chunk
// holds at least 1024): per-chunk LDS histograms, one workgroup scanning them
// into per-(chunk, bucket) bases, and the stable scatter per chunk starting
// from its chunk's bases. The library allocates nothing, so a chunk's
// histogram row (then its bases) lives in the chunk's own stretch of `revert`,
// which only that chunk's scatter overwrites, after reading the row.
//
// Combine restates `fused_moe_gmm.py:572-577`: the down GEMM has already
// multiplied each row by its routing weight and scattered it to its flat
// route slot, so out[t] = sum of the token's valid slots.

#include "moe_common.h"

namespace {

constexpr int kDT = 1024;
constexpr int kWaves = kDT / 64;
using qmoe_moe::kMaxB;
using qmoe_moe::kMaxE;

__device__ __forceinline__ int block_excl_scan(int v, int* tmp, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kWaves ? tmp[lane] : 0;
#pragma unroll
    for (int o = 1; o < kWaves; o <<= 1) {
      int y = __shfl_up(w, o, 64);
      if (lane >= o) w += y;
    }
    if (lane < kWaves) tmp[kWaves + lane] = w;  // inclusive wave totals
  }
  __syncthreads();
  const int before = wave > 0 ? tmp[kWaves + wave - 1] : 0;
  total = tmp[2 * kWaves - 1];
  __syncthreads();
  return before + x - v;
}

__global__ __launch_bounds__(kDT) void dispatch_kernel(
    const int32_t* __restrict__ ids, const uint16_t* __restrict__ wts, int Nf, int topk, int E,
    int skip_padded, int32_t* __restrict__ sorted_idx, int32_t* __restrict__ revert,
    int32_t* __restrict__ token_sorted, int32_t* __restrict__ group_offs,
    int32_t* __restrict__ active, int32_t* __restrict__ num_active,
    uint16_t* __restrict__ sorted_weight) {
  __shared__ int base[kMaxB];
  __shared__ int wcnt[kWaves][kMaxB];
  __shared__ int tmp[2 * kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = E + 1;

  auto bucket = [&](int f) -> int {
    const int id = ids[f];
    bool ok = id >= 0 && id < E;
    if (skip_padded && ok) ok = (wts[f] & 0x7fffu) != 0;
    return ok ? id : E;
  };

  for (int i = tid; i < B; i += kDT) base[i] = 0;
  for (int i = tid; i < kWaves * kMaxB; i += kDT) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  for (int f = tid; f < Nf; f += kDT) atomicAdd(&base[bucket(f)], 1);
  __syncthreads();

  // bucket bases (exclusive scan of counts) and the list of non-empty experts
  const int c = tid < B ? base[tid] : 0;
  int total = 0;
  const int start = block_excl_scan(c, tmp, total);
  const int flag = (tid < E && c > 0) ? 1 : 0;
  int nact = 0;
  const int apos = block_excl_scan(flag, tmp, nact);
  if (tid < B) {
    base[tid] = start;
    group_offs[tid] = start;  // group_offs[E] = number of valid routes
  }
  if (flag) active[apos] = tid;
  if (tid == 0) *num_active = nact;
  __syncthreads();

  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int c0 = 0; c0 < Nf; c0 += kDT) {
    const int f = c0 + tid;
    const bool in = f < Nf;
    const int b = in ? bucket(f) : 0;
    uint64_t m = __ballot(in);
#pragma unroll
    for (int bit = 0; bit < 10; ++bit) {
      const bool s = (b >> bit) & 1;
      const uint64_t bal = __ballot(s);
      m &= s ? bal : ~bal;
    }
    const int rank = __popcll(m & lt);
    if (in && rank == 0) wcnt[wave][b] = __popcll(m);
    __syncthreads();
    if (in) {
      int pos = base[b] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][b];
      sorted_idx[pos] = f;
      revert[f] = pos;
      token_sorted[pos] = f / topk;
      sorted_weight[pos] = wts[f];
    }
    __syncthreads();
    for (int i = tid; i < B; i += kDT) {
      int s = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        s += wcnt[w][i];
        wcnt[w][i] = 0;
      }
      base[i] += s;
    }
    __syncthreads();
  }
}

// ---- many routes: chunked dispatch ----
constexpr int kChunk = 1024;
constexpr int kChunkedMinRoutes = 8192;

__device__ __forceinline__ int route_bucket(const int32_t* ids, const uint16_t* wts, int f, int E, int skip_padded) {
  const int id = ids[f];
  bool ok = id >= 0 && id < E;
  if (skip_padded && ok) ok = (wts[f] & 0x7fffu) != 0;
  return ok ? id : E;
}

// Chunk c = blockIdx.x covers routes [c * kChunk, c == C - 1 ? Nf : (c + 1) * kChunk).
__device__ __forceinline__ void chunk_range(int Nf, int& f0, int& f1) {
  const int C = Nf / kChunk;
  f0 = (int)blockIdx.x * kChunk;
  f1 = (int)blockIdx.x == C - 1 ? Nf : f0 + kChunk;
}

__global__ __launch_bounds__(kDT) void dispatch_count_kernel(const int32_t* __restrict__ ids,
                                                             const uint16_t* __restrict__ wts, int Nf, int E,
                                                             int skip_padded, int32_t* __restrict__ rows) {
  __shared__ int cnt[kMaxB];
  const int B = E + 1;
  int f0, f1;
  chunk_range(Nf, f0, f1);
  for (int i = threadIdx.x; i < B; i += kDT) cnt[i] = 0;
  __syncthreads();
  for (int f = f0 + threadIdx.x; f < f1; f += kDT) atomicAdd(&cnt[route_bucket(ids, wts, f, E, skip_padded)], 1);
  __syncthreads();
  // the row sits at the start of the chunk's own stretch (B <= kChunk)
  for (int i = threadIdx.x; i < B; i += kDT) rows[f0 + i] = cnt[i];
}

__global__ __launch_bounds__(kDT) void dispatch_scan_kernel(int Nf, int E, int32_t* __restrict__ rows,
                                                            int32_t* __restrict__ group_offs,
                                                            int32_t* __restrict__ active,
                                                            int32_t* __restrict__ num_active) {
  __shared__ int tmp[2 * kWaves];
  const int tid = threadIdx.x;
  const int B = E + 1, C = Nf / kChunk;
  // bucket tid's total over the chunks (8 rows per step, so that the loads
  // are in flight together)
  constexpr int kStep = 8;
  int c_tot = 0;
  if (tid < B) {
    for (int c0 = 0; c0 < C; c0 += kStep) {
      int v[kStep];
#pragma unroll
      for (int u = 0; u < kStep; ++u) v[u] = c0 + u < C ? rows[(c0 + u) * kChunk + tid] : 0;
#pragma unroll
      for (int u = 0; u < kStep; ++u) c_tot += v[u];
    }
  }
  int total = 0;
  const int start = block_excl_scan(c_tot, tmp, total);
  const int flag = (tid < E && c_tot > 0) ? 1 : 0;
  int nact = 0;
  const int apos = block_excl_scan(flag, tmp, nact);
  if (tid < B) {
    group_offs[tid] = start;  // group_offs[E] = number of valid routes
    // chunk c's first slot in bucket tid: the bucket start plus the earlier chunks' counts
    int run = start;
    for (int c0 = 0; c0 < C; c0 += kStep) {
      int v[kStep];
#pragma unroll
      for (int u = 0; u < kStep; ++u) v[u] = c0 + u < C ? rows[(c0 + u) * kChunk + tid] : 0;
#pragma unroll
      for (int u = 0; u < kStep; ++u) {
        if (c0 + u < C) rows[(c0 + u) * kChunk + tid] = run;
        run += v[u];
      }
    }
  }
  if (flag) active[apos] = tid;
  if (tid == 0) *num_active = nact;
}

__global__ __launch_bounds__(kDT) void dispatch_scatter_kernel(
    const int32_t* __restrict__ ids, const uint16_t* __restrict__ wts, int Nf, int topk, int E, int skip_padded,
    int32_t* __restrict__ sorted_idx, int32_t* __restrict__ revert, int32_t* __restrict__ token_sorted,
    uint16_t* __restrict__ sorted_weight) {
  __shared__ int base[kMaxB];
  __shared__ int wcnt[kWaves][kMaxB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = E + 1;
  int f0, f1;
  chunk_range(Nf, f0, f1);
  for (int i = tid; i < B; i += kDT) base[i] = revert[f0 + i];
  for (int i = tid; i < kWaves * kMaxB; i += kDT) (&wcnt[0][0])[i] = 0;
  __syncthreads();  // the bases are read before any revert entry of the chunk is written
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int c0 = f0; c0 < f1; c0 += kDT) {
    const int f = c0 + tid;
    const bool in = f < f1;
    const int b = in ? route_bucket(ids, wts, f, E, skip_padded) : 0;
    uint64_t m = __ballot(in);
#pragma unroll
    for (int bit = 0; bit < 10; ++bit) {
      const bool sb = (b >> bit) & 1;
      const uint64_t bal = __ballot(sb);
      m &= sb ? bal : ~bal;
    }
    const int rank = __popcll(m & lt);
    if (in && rank == 0) wcnt[wave][b] = __popcll(m);
    __syncthreads();
    if (in) {
      int pos = base[b] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][b];
      sorted_idx[pos] = f;
      revert[f] = pos;
      token_sorted[pos] = f / topk;
      sorted_weight[pos] = wts[f];
    }
    __syncthreads();
    for (int i = tid; i < B; i += kDT) {
      int sum = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        sum += wcnt[w][i];
        wcnt[w][i] = 0;
      }
      base[i] += sum;
    }
    __syncthreads();
  }
}

// Decode form (T*k <= 64): one wavefront, route f in lane f; see
// qmoe_moe::dispatch_wave. Same outputs as dispatch_kernel.
__global__ __launch_bounds__(64) void dispatch_small_kernel(
    const int32_t* __restrict__ ids, const uint16_t* __restrict__ wts, int Nf, int topk, int E,
    int skip_padded, int32_t* __restrict__ sorted_idx, int32_t* __restrict__ revert,
    int32_t* __restrict__ token_sorted, int32_t* __restrict__ group_offs,
    int32_t* __restrict__ active, int32_t* __restrict__ num_active,
    uint16_t* __restrict__ sorted_weight) {
  __shared__ int cnt[64 * qmoe_moe::kPer];
  __shared__ int offs[64 * qmoe_moe::kPer];
  qmoe_moe::dispatch_wave(ids, wts, Nf, topk, E, skip_padded, sorted_idx, revert, token_sorted, group_offs,
                          active, num_active, sorted_weight, cnt, offs);
}

__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ rows,
                                                      const int32_t* __restrict__ ids,
                                                      const uint16_t* __restrict__ wts, int topk,
                                                      int E, int64_t H, int skip_padded,
                                                      uint16_t* __restrict__ out, int64_t ldo) {
  const int64_t t = blockIdx.x;
  const int64_t h = ((int64_t)blockIdx.y * 256 + threadIdx.x) * 8;
  if (h >= H) return;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int j = 0; j < topk; ++j) {
    const int64_t f = t * topk + j;
    const int id = ids[f];
    // the dispatch kernels' validity rule: ids outside [0, E) sort into the
    // invalid bucket, so the down GEMM never wrote their rows
    bool ok = id >= 0 && id < E;
    if (skip_padded && ok) ok = (wts[f] & 0x7fffu) != 0;
    if (!ok) continue;
    const uint4 v = *reinterpret_cast<const uint4*>(rows + f * H + h);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += bits_f32(w[i] << 16);
      acc[2 * i + 1] += bits_f32(w[i] & 0xffff0000u);
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = (uint32_t)f32_to_bf16(acc[2 * i]) | ((uint32_t)f32_to_bf16(acc[2 * i + 1]) << 16);
  *reinterpret_cast<uint4*>(out + t * ldo + h) = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace

extern "C" int qmoe_moe_dispatch(const int32_t* topk_ids, const uint16_t* topk_weights, int64_t T,
                                 int topk, int E, int skip_padded, int32_t* sorted_idx,
                                 int32_t* revert, int32_t* token_sorted, int32_t* group_offs,
                                 int32_t* active, int32_t* num_active, uint16_t* sorted_weight,
                                 hipStream_t stream) {
  if (T < 0 || topk <= 0 || E <= 0 || E > kMaxE) return QMOE_ERR_ARG;
  const int64_t nf = T * topk;
  if (nf >= (int64_t)1 << 30) return QMOE_ERR_ARG;
  if (nf <= 64)
    hipLaunchKernelGGL(dispatch_small_kernel, dim3(1), dim3(64), 0, stream, topk_ids, topk_weights, (int)nf, topk,
                       E, skip_padded, sorted_idx, revert, token_sorted, group_offs, active, num_active,
                       sorted_weight);
  else if (nf < kChunkedMinRoutes)
    hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(kDT), 0, stream, topk_ids, topk_weights,
                       (int)nf, topk, E, skip_padded, sorted_idx, revert, token_sorted, group_offs,
                       active, num_active, sorted_weight);
  else {
    const unsigned chunks = (unsigned)(nf / kChunk);
    hipLaunchKernelGGL(dispatch_count_kernel, dim3(chunks), dim3(kDT), 0, stream, topk_ids, topk_weights, (int)nf,
                       E, skip_padded, revert);
    hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(kDT), 0, stream, (int)nf, E, revert, group_offs, active,
                       num_active);
    hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(chunks), dim3(kDT), 0, stream, topk_ids, topk_weights,
                       (int)nf, topk, E, skip_padded, sorted_idx, revert, token_sorted, sorted_weight);
  }
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}

extern "C" int qmoe_moe_combine(const uint16_t* rows, const int32_t* topk_ids,
                                const uint16_t* topk_weights, int64_t T, int topk, int E, int64_t H,
                                int skip_padded, uint16_t* out, int64_t ldo, hipStream_t stream) {
  if (T < 0 || topk <= 0 || E <= 0 || H <= 0 || (H % 8) != 0 || ldo < H || (ldo % 8) != 0) return QMOE_ERR_ARG;
  if (T == 0) return QMOE_OK;
  if (cdiv<int64_t>(H, 256 * 8) > 65535) return QMOE_ERR_ARG;
  dim3 grid((unsigned)T, (unsigned)cdiv<int64_t>(H, 256 * 8));
  hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, stream, rows, topk_ids, topk_weights, topk,
                     E, H, skip_padded, out, ldo);
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
