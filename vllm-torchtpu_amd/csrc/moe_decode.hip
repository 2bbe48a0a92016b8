// Fused decode MoE layer on one GPU: the shared expert and the routed
// experts of a decode step (1..64 tokens) in four launches, restating
// `kernels/experimental/fused_moe_decode/fused_moe_decode_kernel.py:552-740`
// (route-weight table, active experts, shared gate) and `:200-336` (the
// activation quantization, the two matmuls, the float32 accumulator).
//
//  1. prep (1 + T workgroups): workgroup 0 builds the dispatch -- group 0 is
//     the shared expert (every token, rows 0..T-1), group e + 1 routed expert
//     e (its tokens in order, rows after the shared ones), the active list
//     (shared first, then routed experts in increasing id: the reference's
//     accumulation order), each row's float32 coefficient and the (slot,
//     token) -> row map; workgroup 1 + t quantizes token t's hidden state per
//     (row, 512 | 128 columns) in float32 and computes its shared-expert
//     coefficient (sigmoid of the gate dot, or 1); every workgroup clears a
//     share of the block-maximum table;
//  2. gate_up: the skinny grouped GEMM over the active groups, silu(gate) *
//     up times the row coefficient stored as float32 rows, each (row, block)
//     absolute maximum folded into the table by atomic max;
//  3. intermediate quantization: codes e4m3(v * (1 / (max / 448))) per
//     (row, block), the reference's float32 recipe;
//  4. down: one workgroup per 16 (or 32) output columns walks every active
//     slot, streams that expert's weight slab once, and adds each token's
//     term into registers (tokens are MFMA rows, a token the expert does not
//     serve reads zeros without a memory request), so the per-token sum over
//     experts -- the combine -- happens in the workgroup, in slot order, and
//     the bf16 output is written directly.
//
// Weights are N-major (checkpoint layout): w1 [E][2I][H] (gate rows then
// up rows), w2 [E][H][I]; scales per channel ([E][2I], [E][H]) or per
// 128x128 tile ([E][2I/128][H/128], [E][H/128][I/128]). The shared expert's
// tensors have the same layouts without the E axis and I_s <= I.

#include <algorithm>
#include <cstdlib>

#include "gemm_common.h"
#include "moe_route.h"
#include "stream_load.h"

#include "qmoe.h"

int qmoe_skinny_launch(int kind, GemmParams p, int max_rows, int slots, void* workspace, int64_t ws_bytes,
                       int ksplit_hint, hipStream_t st);

namespace {

using namespace qmoe_stream;

constexpr int kPrep = 256;        // threads of the prep and quantization workgroups
constexpr int kMaxTokens = 64;    // tokens of one fused decode call
constexpr int kMaxExperts = 512;
constexpr int kRouteInPrep = 8;   // tokens the prep launch routes itself (2 per wavefront)

// Workspace carve-up (byte offsets, 256-aligned), shared by host and kernels.
struct DecodeLayout {
  int64_t xq, xs, goffs, active, nact, arows, coeff, map, mid, bmax, mq, msc, part, total;
  int R;      // rows: T shared + T * topk routed (upper bound)
  int slots;  // 1 + min(E, T * topk)
  int xb;     // hidden-state quantization block (512 or 128)
  int qb;     // intermediate quantization block: 512 (the last one partial when
              // I % 512 != 0, the reference's min(512, I) blocks) or 128
  int nbx, nbm;
  int splits;  // down: contiguous ranges of the active list over grid.y
};

int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

// Workgroups of the down kernel per column block: above 16 tokens a step
// touches ~100-250 experts, and one workgroup walking all of them in turn
// (two in flight) is latency bound, so the active list is cut into
// contiguous ranges whose float32 partial sums are added in range order by
// a last launch.
int down_splits(int64_t T) {
  const char* env = std::getenv("QMOE_DECODE_DOWN_SPLITS");  // tuning knob: 1..16
  if (env && std::atoi(env) >= 1 && std::atoi(env) <= 16) return T > 16 ? std::atoi(env) : 1;
  return T > 16 ? 4 : 1;
}

DecodeLayout decode_layout(const qmoe_moe_decode_desc* d) {
  DecodeLayout L{};
  L.R = (int)(d->T * (d->topk + 1));
  L.slots = 1 + (int)std::min<int64_t>(d->E, d->T * d->topk);
  L.xb = d->weight_blocks ? 128 : 512;
  L.qb = d->weight_blocks ? 128 : 512;
  L.nbx = (int)(d->H / L.xb);
  L.nbm = (int)cdiv<int64_t>(d->I, L.qb);
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o = align256(o + bytes);
    return at;
  };
  L.xq = take(d->T * d->H);
  L.xs = take(d->T * L.nbx * 4);
  L.goffs = take((int64_t)(d->E + 2) * 4);
  L.active = take((int64_t)L.slots * 4);
  L.nact = take(4);
  L.arows = take((int64_t)L.R * 4);
  L.coeff = take((int64_t)L.R * 4);
  L.map = take((int64_t)L.slots * d->T * 4);
  L.mid = take((int64_t)L.R * d->I * 4);
  L.bmax = take((int64_t)L.R * L.nbm * 4);
  L.mq = take((int64_t)L.R * d->I);
  L.msc = take((int64_t)L.R * L.nbm * 4);
  L.splits = down_splits(d->T);
  L.part = take(L.splits > 1 ? (int64_t)L.splits * d->T * d->H * 4 : 0);
  L.total = o;
  return L;
}

struct PrepArgs {
  const uint16_t* x;
  int T, H, E, topk;
  const int32_t* ids;
  const void* tw;
  int tw_f32;
  float routed_scale;
  const uint16_t* gate;  // bf16 [H] or nullptr
  int xb;
  uint8_t* xq;
  float* xs;
  int32_t* goffs;
  int32_t* active;
  int32_t* nact;
  int32_t* arows;
  float* coeff;
  int32_t* map;
  uint32_t* bmax;
  int64_t bmax_words;
  // in-launch routing (prep instantiations with S > 0 slots): the router's
  // arguments, and where the ids and bf16 weights go
  const void* logits;
  int logits_f32, scoring, renormalize, num_group, topk_group;
  const float* bias;
  float rsf;
  int32_t* ids_out;
  uint16_t* w_out;
};

// The reference's route weight: rounded to the activation dtype (bf16), then
// times routed_scale in float32 (`fused_moe_decode_kernel.py:639-641`).
__device__ __forceinline__ float scaled_route_weight(const PrepArgs& a, float w_bf16) {
  return a.routed_scale != 1.0f ? w_bf16 * a.routed_scale : w_bf16;
}
__device__ __forceinline__ float route_weight(const PrepArgs& a, int f) {
  return scaled_route_weight(a, a.tw_f32 ? bf16_round(static_cast<const float*>(a.tw)[f])
                                         : bf16_to_f32(static_cast<const uint16_t*>(a.tw)[f]));
}

// Route f's row coefficient from the staged ids / weights, or 0 when it
// yields no row: an id outside [0, E), a later route of its token naming the
// same expert (folded into the first: the reference's table sums them in
// route order, `:642-645`), or a zero sum (`where(coeff != 0, ..., 0)` makes
// such a row zero).
__device__ __forceinline__ float route_coeff(const int* ids, const float* w, int topk, int E, int f) {
  const int t = f / topk, j = f - t * topk;
  const int id = ids[f];
  if (id < 0 || id >= E) return 0.0f;
  const int* row = ids + t * topk;
  for (int j2 = 0; j2 < j; ++j2)
    if (row[j2] == id) return 0.0f;
  float c = w[f];
  for (int j2 = j + 1; j2 < topk; ++j2)
    if (row[j2] == id) c = c + w[t * topk + j2];
  return c;
}

// Exclusive scan of one int per thread over the workgroup (kPrep threads):
// the wavefront scans by DPP, then the wavefront totals through LDS.
__device__ __forceinline__ int prep_scan(int v, int* tmp, int& total) {
  constexpr int kW = kPrep / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int wtot = 0;
  const int ex = qmoe_moe::wave_excl_scan(v, lane, wtot);
  if (lane == 0) tmp[wave] = wtot;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kW; ++w) {
    const int c = tmp[w];
    before += w < wave ? c : 0;
    total += c;
  }
  __syncthreads();
  return before + ex;
}

// Token t's hidden-state codes per (row, XB columns) in float32 (scale =
// max|x| / 448, inv = 0 where the scale is 0 else 1 / scale, codes e4m3(x *
// inv) rounded to nearest even, `:216-223`) and its shared-expert gate dot.
// Thread i holds 8-value chunks i, i + 256, ...: the XB / 8 lanes of a block
// are adjacent, all loads are issued before any reduction.
template <int XB>
__device__ __forceinline__ void quant_token(const PrepArgs& a, int t) {
  constexpr int L = XB / 8;  // lanes per block (16 or 64)
  constexpr int kMaxChunks = 8;  // H <= 16384
  const int tid = threadIdx.x;
  const int nch = a.H / 8;
  const uint4* xr = reinterpret_cast<const uint4*>(a.x + (int64_t)t * a.H);
  const uint4* gr = reinterpret_cast<const uint4*>(a.gate);
  uint4 xv[kMaxChunks], gv[kMaxChunks];
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int c = tid + i * kPrep;
    if (c < nch) {
      xv[i] = xr[c];
      if (a.gate) gv[i] = gr[c];
    }
  }
  float dsum = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int c = tid + i * kPrep;
    if (i * kPrep >= nch) break;  // uniform: whole blocks per iteration
    const bool in = c < nch;
    const uint32_t w[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bits_f32(w[j] << 16);
      v[2 * j + 1] = bits_f32(w[j] & 0xffff0000u);
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = in ? fmaxf(m, fabsf(v[j])) : m;
#pragma unroll
    for (int o = 1; o < L; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, L));
    const float s = m / 448.0f;
    const float inv = s == 0.0f ? 0.0f : 1.0f / s;
    if (in) {
      float q[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) q[j] = fminf(fmaxf(v[j] * inv, -448.0f), 448.0f);
      int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
      int hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
      *reinterpret_cast<uint2*>(a.xq + (int64_t)t * a.H + (int64_t)c * 8) = make_uint2((uint32_t)lo, (uint32_t)hi);
      if ((c % L) == 0) a.xs[(int64_t)t * (a.H / XB) + c / L] = s;
      if (a.gate) {
        const uint32_t g[4] = {gv[i].x, gv[i].y, gv[i].z, gv[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          dsum += v[2 * j] * bits_f32(g[j] << 16) + v[2 * j + 1] * bits_f32(g[j] & 0xffff0000u);
      }
    }
  }
  // shared gate: sigmoid of the float32-accumulated dot of bf16 values
  __shared__ float part[kPrep / 64];
  dsum = wave_sum(dsum);
  if ((tid & 63) == 0) part[tid >> 6] = dsum;
  __syncthreads();
  if (tid == 0) {
    float d = 0.0f;
    for (int w = 0; w < kPrep / 64; ++w) d += part[w];
    a.coeff[t] = a.gate ? 1.0f / (1.0f + expf(-d)) : 1.0f;
  }
}

constexpr int kMaxRoutes = kMaxTokens * 64;

// S > 0: workgroup 0 first routes the step's tokens (S 64-expert slots per
// row, at most kRouteInPrep tokens: wavefront w routes tokens w, w + 4), the
// routes going to LDS for the dispatch and to ids_out / w_out.
template <int S>
__global__ __launch_bounds__(kPrep) void decode_prep_kernel(const PrepArgs a) {
  const int tid = threadIdx.x;
  // every workgroup clears its share of the block-maximum table
  for (int64_t i = (int64_t)blockIdx.x * kPrep + tid; i < a.bmax_words; i += (int64_t)gridDim.x * kPrep)
    a.bmax[i] = 0u;

  if (blockIdx.x > 0) {
    if (a.xb == 512) quant_token<512>(a, blockIdx.x - 1);
    else quant_token<128>(a, blockIdx.x - 1);
    return;
  }

  // workgroup 0: dispatch, from routes staged in LDS
  __shared__ int s_ids[kMaxRoutes];
  __shared__ float s_w[kMaxRoutes];
  __shared__ int cnt[kMaxExperts];
  __shared__ int cursor[kMaxExperts];
  __shared__ int slotpos[kMaxExperts];
  __shared__ int tmp[kPrep / 64];
  const int Nf = a.T * a.topk;
  if constexpr (S > 0) {
    __shared__ float route_lds[kPrep / 64][qmoe_route::kChoiceLds];
    __shared__ uint16_t s_w16[kRouteInPrep * 64];
    const int wave = tid >> 6;
    const bool grouped = a.num_group > 1 && a.topk_group < a.num_group;
    for (int t = wave; t < a.T; t += kPrep / 64)
      qmoe_route::route_token_any<S>(a.scoring, grouped, a.logits, a.logits_f32, t, a.E, a.topk, a.bias,
                                     a.renormalize, a.rsf, a.num_group, a.topk_group, a.w_out, a.ids_out,
                                     route_lds[wave], s_ids, s_w16);
    __syncthreads();
    for (int f = tid; f < Nf; f += kPrep) s_w[f] = scaled_route_weight(a, bf16_to_f32(s_w16[f]));
  } else {
    for (int f = tid; f < Nf; f += kPrep) {
      s_ids[f] = a.ids[f];
      s_w[f] = route_weight(a, f);
    }
  }
  for (int e = tid; e < a.E; e += kPrep) cnt[e] = 0;
  __syncthreads();
  for (int f = tid; f < Nf; f += kPrep) {
    const float c = route_coeff(s_ids, s_w, a.topk, a.E, f);
    if (c != 0.0f) atomicAdd(&cnt[s_ids[f]], 1);
  }
  __syncthreads();
  // two consecutive experts per thread (E <= 512)
  const int e0 = 2 * tid;
  const int c0 = e0 < a.E ? cnt[e0] : 0, c1 = e0 + 1 < a.E ? cnt[e0 + 1] : 0;
  int rows_total = 0, nact_routed = 0;
  const int rbase = prep_scan(c0 + c1, tmp, rows_total);
  const int abase = prep_scan((c0 > 0) + (c1 > 0), tmp, nact_routed);
  if (e0 < a.E) {
    a.goffs[e0 + 1] = a.T + rbase;
    cursor[e0] = a.T + rbase;
    slotpos[e0] = c0 > 0 ? 1 + abase : -1;
    if (c0 > 0) a.active[1 + abase] = e0 + 1;
  }
  if (e0 + 1 < a.E) {
    a.goffs[e0 + 2] = a.T + rbase + c0;
    cursor[e0 + 1] = a.T + rbase + c0;
    slotpos[e0 + 1] = c1 > 0 ? 1 + abase + (c0 > 0) : -1;
    if (c1 > 0) a.active[1 + abase + (c0 > 0)] = e0 + 2;
  }
  if (tid == 0) {
    a.goffs[0] = 0;
    a.goffs[a.E + 1] = a.T + rows_total;
    a.active[0] = 0;
    *a.nact = 1 + nact_routed;
  }
  // the shared group: row t is token t (its coefficient comes from
  // workgroup 1 + t); routed slots start with no token
  for (int i = tid; i < a.T; i += kPrep) {
    a.arows[i] = i;
    a.map[i] = i;
  }
  for (int i = a.T + tid; i < (1 + nact_routed) * a.T; i += kPrep) a.map[i] = -1;
  __syncthreads();
  // routed rows: positions inside a group come from LDS atomics, so their
  // order varies from call to call; every row is computed on its own and
  // the down projection sums a token's terms in slot order, so the output
  // does not depend on it
  for (int f = tid; f < Nf; f += kPrep) {
    const float c = route_coeff(s_ids, s_w, a.topk, a.E, f);
    if (c == 0.0f) continue;
    const int e = s_ids[f];
    const int r = atomicAdd(&cursor[e], 1);
    const int t = f / a.topk;
    a.arows[r] = t;
    a.coeff[r] = c;
    a.map[slotpos[e] * a.T + t] = r;
  }
}

// Step 3: codes of the float32 intermediate rows, per (row, qb columns).
__global__ __launch_bounds__(kPrep) void decode_mid_quant_kernel(const float* __restrict__ mid,
                                                                 const uint32_t* __restrict__ bmax,
                                                                 const int32_t* __restrict__ goffs, int E, int T,
                                                                 int I, int Is, int qb, int nbm,
                                                                 uint8_t* __restrict__ mq, float* __restrict__ msc) {
  // every row bound R (no wait on the group offsets first): rows past the
  // used count have block maxima 0 (cleared by prep) and their codes are
  // never read
  (void)goffs;
  (void)E;
  const int R = blockIdx.x;
  const int width = R < T ? Is : I;
  const float* src = mid + (int64_t)R * I;
  uint8_t* dst = mq + (int64_t)R * I;
  for (int c = threadIdx.x * 8; c < width; c += kPrep * 8) {
    // 8 columns inside one block (qb is a multiple of 128)
    const int b = c / qb;
    const float s = __uint_as_float(bmax[(int64_t)R * nbm + b]) / 448.0f;
    const float inv = s == 0.0f ? 0.0f : 1.0f / s;
    const float4 v0 = *reinterpret_cast<const float4*>(src + c);
    const float4 v1 = *reinterpret_cast<const float4*>(src + c + 4);
    const float f[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = fminf(fmaxf(f[i] * inv, -448.0f), 448.0f);
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
    int hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
    *reinterpret_cast<uint2*>(dst + c) = make_uint2((uint32_t)lo, (uint32_t)hi);
    if ((c % qb) == 0) msc[(int64_t)R * nbm + b] = s;
  }
}

struct DownArgs {
  const uint8_t* mq;  // [R][I] e4m3 codes
  const float* msc;   // [R][nbm]
  int nbm, qsh;       // block of 128-step s: s >> qsh
  int R;
  const int32_t* map;  // [slot][T] -> row or -1
  const int32_t* active;
  const int32_t* nact;
  int slots;  // capacity of `active`
  int T, H, I, Is;
  const uint8_t* w2;  // [E][H][I]
  const uint8_t* w2x; // [H][Is]
  const float* ws2;   // [E][H] or [E][H/128][I/128]
  const float* ws2x;  // [H] or [H/128][Is/128]
  uint16_t* out;
  int64_t ldo;
  int splits;      // grid.y: contiguous ranges of the active list
  float* partial;  // splits > 1: float32 [splits][T][H] partial sums
};

// One workgroup: output columns [n0, n0 + 16 * NS) for every token (MT
// tiles of 16 tokens), W wavefronts. Each active slot is one item: wavefront
// w takes its share of the slot's 128-k steps (at most CH); the next slot's
// weight, code and scale loads are issued before the current slot's MFMAs,
// so two slots of loads are in flight per wavefront.
template <int MT, int NS, int CH, int W, bool TILES>
__global__ __launch_bounds__(W * 64) void decode_down_kernel(const DownArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * 16 * NS;
  const int perm_src = (4 * col + kg) * 4;

  __shared__ int s_active[kMaxExperts + 1];
  // the (slot, token) -> row map of the active slots, staged once: slot
  // setup then reads LDS instead of waiting on a global load per slot
  extern __shared__ int16_t s_map[];
  const rsrc_t ares = make_rsrc(a.mq, (int64_t)a.R * a.I);
  const rsrc_t sres = make_rsrc(a.msc, (int64_t)a.R * a.nbm * 4);

  struct Slot {
    rsrc_t wres;
    uint32_t woff[NS];
    uint32_t aoff[MT];  // the lane's code row (token mt*16 + col) or kOob
    uint32_t soff[MT];  // its scale row
    float wsv[NS];      // per-channel scales of the lane's columns
    int g, j0, n;       // group, this wavefront's first step and step count
    uint32_t live;      // M tiles holding a token the expert serves
  };
  struct Item {
    uint4 bw[CH][NS][2];
    uint4 fa[CH][MT][2];
    float ms[CH][MT];  // the lane's code-row scale at the step's block
    float wt[CH];      // tile scale (TILES)
  };

  // slot 0 is the shared expert, whose rows are the tokens themselves: it
  // needs no dispatch metadata, so its loads go out before the active list
  // is read
  auto setup_issue = [&](int s, Slot& S, Item& it) {
    const int g = s == 0 ? 0 : s_active[s];
    const int K = g == 0 ? a.Is : a.I;
    const int steps = K >> 7;
    S.g = g;
    S.j0 = steps * wave / W;
    S.n = steps * (wave + 1) / W - S.j0;
    const uint8_t* wb = g == 0 ? a.w2x : a.w2 + (int64_t)(g - 1) * a.H * a.I;
    S.wres = make_rsrc(wb + (int64_t)n0 * K, (int64_t)16 * NS * K);
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) S.woff[ns] = (uint32_t)((ns * 16 + (lane >> 2)) * K + (lane & 3) * 16);
    S.live = 0;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int tok = mt * 16 + col;
      const int r = tok < a.T ? (s == 0 ? tok : (int)s_map[s * a.T + tok]) : -1;
      S.aoff[mt] = r >= 0 ? (uint32_t)(r * a.I + kg * 16) : kOob;
      S.soff[mt] = r >= 0 ? (uint32_t)(r * a.nbm * 4) : kOob;
      if (__ballot(r >= 0)) S.live |= 1u << mt;
    }
    if constexpr (!TILES) {
      const float* ws = g == 0 ? a.ws2x : a.ws2 + (int64_t)(g - 1) * a.H;
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) S.wsv[ns] = ws[n0 + ns * 16 + col];
    }
    // loads of this wavefront's steps; steps past its share return zeros
    // without a memory request
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const bool in = c < S.n;
      const uint32_t ks = (uint32_t)(S.j0 + (in ? c : 0));
      const uint32_t oob = in ? 0u : kOob;
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        Frag f;
        ldw_seg<32>(f, S.wres, S.woff[ns] | oob, ks * 128);
        it.bw[c][ns][0] = f.v[0];
        it.bw[c][ns][1] = f.v[1];
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint32_t o = S.aoff[mt] | oob;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(ares, o + i * 64, ks * 128, 0);
          it.fa[c][mt][i] = make_uint4(v[0], v[1], v[2], v[3]);
        }
        it.ms[c][mt] = ldb_f32(sres, S.soff[mt] | oob, (ks >> a.qsh) * 4);
      }
      if constexpr (TILES) {
        const float* wt = g == 0 ? a.ws2x : a.ws2 + (int64_t)(g - 1) * (a.H >> 7) * (a.I >> 7);
        it.wt[c] = in ? wt[(n0 >> 7) * (K >> 7) + ks] : 0.0f;
      }
    }
  };

  f32x4 acc[MT][NS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) acc[mt][ns] = f32x4{0, 0, 0, 0};

  // one slot's term: per step, the MFMA of codes from zero times the
  // accumulator rows' scales (and the tile scale); per-channel scales once
  // per slot
  auto consume = [&](const Slot& S, Item& it) {
    f32x4 te[MT][NS];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) te[mt][ns] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      i32x8 bw[NS];
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        Frag f;
        f.v[0] = it.bw[c][ns][0];
        f.v[1] = it.bw[c][ns][1];
        permute_w<32>(f, perm_src);
        bw[ns] = as_i32x8(f);
      }
      if (c >= S.n) continue;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (!((S.live >> mt) & 1)) continue;
        Frag fa;
        fa.v[0] = it.fa[c][mt][0];
        fa.v[1] = it.fa[c][mt][1];
        // accumulator row q holds token mt*16 + 4kg + q: the code lane of
        // that token (column 4kg + q) has its scale
        float sr[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) sr[q] = __shfl(it.ms[c][mt], 4 * kg + q, 64);
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          const f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(as_i32x8(fa), bw[ns],
                                                                           f32x4{0, 0, 0, 0}, 0, 0, 0, 127, 0, 127);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if constexpr (TILES) te[mt][ns][q] += d[q] * (sr[q] * it.wt[c]);
            else te[mt][ns][q] += d[q] * sr[q];
          }
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (TILES) acc[mt][ns][q] += te[mt][ns][q];
          else acc[mt][ns][q] += te[mt][ns][q] * S.wsv[ns];
        }
  };

  Slot sa, sb;
  Item ia, ib;
  // range y of the active list: the shared slot 0, then the routed slots
  // 1..nact-1 cut into `splits` contiguous pieces, [1 + (nact-1) y / splits,
  // 1 + (nact-1) (y+1) / splits), range 0 also taking slot 0 -- so range 0
  // is never empty and the shared slot's loads go out first
  const int ys = blockIdx.y;
  if (ys == 0) setup_issue(0, sa, ia);
  const int nact = min(*a.nact, a.slots);
  for (int i = threadIdx.x; i < nact; i += W * 64) s_active[i] = a.active[i];
  for (int i = threadIdx.x; i < nact * a.T; i += W * 64) s_map[i] = (int16_t)a.map[i];
  __syncthreads();
  const int sb0 = ys == 0 ? 0 : 1 + (int)((int64_t)(nact - 1) * ys / a.splits);
  const int se = 1 + (int)((int64_t)(nact - 1) * (ys + 1) / a.splits);
  if (ys != 0 && sb0 < se) setup_issue(sb0, sa, ia);
  for (int s = sb0; s < se; s += 2) {
    if (s + 1 < se) setup_issue(s + 1, sb, ib);
    __builtin_amdgcn_sched_barrier(0);
    consume(sa, ia);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 >= se) break;
    if (s + 2 < se) setup_issue(s + 2, sa, ia);
    __builtin_amdgcn_sched_barrier(0);
    consume(sb, ib);
    __builtin_amdgcn_sched_barrier(0);
  }

  // sum the wavefronts in a fixed order, then bf16 out
  __shared__ float red[W - 1][MT * NS * 4][64];
  if (wave > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns)
#pragma unroll
        for (int q = 0; q < 4; ++q) red[wave - 1][(mt * NS + ns) * 4 + q][lane] = acc[mt][ns][q];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < W - 1; ++w)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[mt][ns][q] += red[w][(mt * NS + ns) * 4 + q][lane];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int tok = mt * 16 + 4 * kg + q;
      if (tok >= a.T) continue;
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        if (a.splits > 1)
          a.partial[((int64_t)ys * a.T + tok) * a.H + n0 + ns * 16 + col] = acc[mt][ns][q];
        else
          a.out[(int64_t)tok * a.ldo + n0 + ns * 16 + col] = f32_to_bf16(acc[mt][ns][q]);
      }
    }
}

// The down kernel's range partial sums added in range order, bf16 out.
__global__ __launch_bounds__(256) void decode_down_sum_kernel(const float* __restrict__ partial, int splits, int T,
                                                              int H, uint16_t* __restrict__ out, int64_t ldo) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)T * H) return;
  const int tok = (int)(i / H), n = (int)(i - (int64_t)tok * H);
  float v = partial[i];
  for (int y = 1; y < splits; ++y) v += partial[(int64_t)y * T * H + i];
  out[(int64_t)tok * ldo + n] = f32_to_bf16(v);
}

template <int MT, int NS, int CH, int W>
void launch_down(const DownArgs& a, bool tiles, hipStream_t st) {
  const dim3 grid((unsigned)(a.H / (16 * NS)), (unsigned)a.splits);
  const size_t lds = (size_t)a.slots * a.T * sizeof(int16_t);  // s_map
  if (tiles)
    hipLaunchKernelGGL((decode_down_kernel<MT, NS, CH, W, true>), grid, dim3(W * 64), lds, st, a);
  else
    hipLaunchKernelGGL((decode_down_kernel<MT, NS, CH, W, false>), grid, dim3(W * 64), lds, st, a);
}

// 128-k steps of the routed down projection per wavefront, and whether the
// down kernel's instantiations cover them: T <= 16 with 4 wavefronts (up to
// 8 steps each: I <= 4096), T <= 64 with 8 wavefronts (up to 2 steps each:
// I <= 2048)
bool down_fits(int64_t T, int64_t I) {
  const int64_t steps = I / 128;
  return T <= 16 ? steps <= 32 : steps <= 16;
}

int decode_check(const qmoe_moe_decode_desc* d) {
  if (!d || !d->x || !d->topk_ids || !d->topk_weights || !d->w1 || !d->w2 || !d->w1_scale || !d->w2_scale ||
      !d->shared_w1 || !d->shared_w2 || !d->shared_w1_scale || !d->shared_w2_scale || !d->out)
    return QMOE_ERR_ARG;
  if (d->T < 1 || d->T > kMaxTokens || d->E < 1 || d->E > kMaxExperts || d->topk < 1 || d->topk > 64)
    return QMOE_ERR_ARG;
  if (d->weight_blocks != 0 && d->weight_blocks != 128) return QMOE_ERR_ARG;
  // 16-byte loads of the hidden states and the gate weight
  if ((reinterpret_cast<uintptr_t>(d->x) & 15) || (reinterpret_cast<uintptr_t>(d->shared_gate) & 15))
    return QMOE_ERR_ARG;
  if (d->H <= 0 || d->H % 512 || d->H > 16384 || d->I <= 0 || d->I % 128 || d->I_shared <= 0 || d->I_shared % 128 ||
      d->I_shared > d->I || d->ldo < d->H || !down_fits(d->T, d->I))
    return QMOE_ERR_ARG;
  // the down kernel stages the (slot, token) -> row map in LDS (int16)
  if ((1 + std::min<int64_t>(d->E, d->T * d->topk)) * d->T * 2 > 65536) return QMOE_ERR_ARG;
  // 32-bit buffer offsets per expert slab and for the row buffers
  constexpr int64_t kLim = 0x7fffffff;
  if (2 * d->I * d->H > kLim || d->T * (d->topk + 1) * d->I * 4 > kLim) return QMOE_ERR_ARG;
  // routing by the call: the router's envelope, bf16 weights written out
  if (d->router_logits &&
      (d->weights_f32 || !qmoe_route::route_args_ok(d->T, d->E, d->topk, d->scoring, d->num_group, d->topk_group)))
    return QMOE_ERR_ARG;
  return QMOE_OK;
}

}  // namespace

extern "C" int qmoe_moe_decode_workspace_size(const qmoe_moe_decode_desc* d, int64_t* bytes) {
  if (!bytes || decode_check(d) != QMOE_OK) return QMOE_ERR_ARG;
  *bytes = decode_layout(d).total;
  return QMOE_OK;
}

// See include/qmoe.h for the contract.
extern "C" int qmoe_moe_decode(const qmoe_moe_decode_desc* d, void* workspace, int64_t ws_bytes,
                               hipStream_t stream) {
  const int chk = decode_check(d);
  if (chk != QMOE_OK) return chk;
  const DecodeLayout L = decode_layout(d);
  if (!workspace || ws_bytes < L.total) return QMOE_ERR_WORKSPACE;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const int T = (int)d->T, H = (int)d->H, I = (int)d->I, Is = (int)d->I_shared;
  const bool tiles = d->weight_blocks != 0;

  PrepArgs pa{};
  pa.x = static_cast<const uint16_t*>(d->x);
  pa.T = T;
  pa.H = H;
  pa.E = d->E;
  pa.topk = d->topk;
  pa.ids = d->topk_ids;
  pa.tw = d->topk_weights;
  pa.tw_f32 = d->weights_f32;
  pa.routed_scale = d->routed_scale;
  pa.gate = d->shared_gate;
  pa.xb = L.xb;
  pa.xq = ws + L.xq;
  pa.xs = reinterpret_cast<float*>(ws + L.xs);
  pa.goffs = reinterpret_cast<int32_t*>(ws + L.goffs);
  pa.active = reinterpret_cast<int32_t*>(ws + L.active);
  pa.nact = reinterpret_cast<int32_t*>(ws + L.nact);
  pa.arows = reinterpret_cast<int32_t*>(ws + L.arows);
  pa.coeff = reinterpret_cast<float*>(ws + L.coeff);
  pa.map = reinterpret_cast<int32_t*>(ws + L.map);
  pa.bmax = reinterpret_cast<uint32_t*>(ws + L.bmax);
  pa.bmax_words = (int64_t)L.R * L.nbm;
  // routing by the call: inside the prep launch for up to kRouteInPrep
  // tokens, else the router's own launch first (same results either way)
  int route_slots = 0;
  if (d->router_logits) {
    int32_t* ids = const_cast<int32_t*>(d->topk_ids);
    uint16_t* tw = static_cast<uint16_t*>(const_cast<void*>(d->topk_weights));
    if (T <= kRouteInPrep) {
      route_slots = qmoe_route::route_slots(d->E);
      pa.logits = d->router_logits;
      pa.logits_f32 = d->logits_f32;
      pa.scoring = d->scoring;
      pa.renormalize = d->renormalize;
      pa.num_group = d->num_group;
      pa.topk_group = d->topk_group;
      pa.bias = d->correction_bias;
      pa.rsf = d->routed_scaling_factor;
      pa.ids_out = ids;
      pa.w_out = tw;
    } else {
      const int rc = qmoe_moe_route(d->router_logits, d->logits_f32, T, d->E, d->topk, d->scoring,
                                    d->correction_bias, d->renormalize, d->routed_scaling_factor, d->num_group,
                                    d->topk_group, tw, 0, ids, stream);
      if (rc != QMOE_OK) return rc;
    }
  }
  const dim3 pgrid((unsigned)(1 + T));
  switch (route_slots) {
    case 1: hipLaunchKernelGGL(decode_prep_kernel<1>, pgrid, dim3(kPrep), 0, stream, pa); break;
    case 2: hipLaunchKernelGGL(decode_prep_kernel<2>, pgrid, dim3(kPrep), 0, stream, pa); break;
    case 4: hipLaunchKernelGGL(decode_prep_kernel<4>, pgrid, dim3(kPrep), 0, stream, pa); break;
    case 8: hipLaunchKernelGGL(decode_prep_kernel<8>, pgrid, dim3(kPrep), 0, stream, pa); break;
    default: hipLaunchKernelGGL(decode_prep_kernel<0>, pgrid, dim3(kPrep), 0, stream, pa); break;
  }
  if (hipGetLastError() != hipSuccess) return QMOE_ERR_LAUNCH;

  // gate_up: silu(gate) * up * coefficient, float32 rows + block maxima
  GemmParams g{};
  g.a = pa.xq;
  g.lda = H;
  g.a_scale = pa.xs;
  g.lds_a = L.nbx;
  g.a_rows = pa.arows;
  g.w = static_cast<const uint8_t*>(d->w1);
  g.ldw = H;
  g.w_gstride = 2 * d->I * d->H;
  g.w_scale = d->w1_scale;
  g.ws_bn = tiles ? 128 : 1;
  g.ldws = tiles ? H / 128 : 1;
  g.ws_gstride = tiles ? (2 * d->I / 128) * (d->H / 128) : 2 * d->I;
  g.a_kshift = tiles ? 0 : 2;
  g.w_kshift = tiles ? 0 : 31;
  g.group_offs = pa.goffs;
  g.active = pa.active;
  g.num_active = pa.nact;
  g.slots = L.slots;
  g.M = L.R;
  g.N = 2 * I;
  g.K = H;
  g.act = QA_SILU;
  g.x0 = 1;
  g.n_x = 2 * Is;
  g.rows_x = T;
  g.w_x = static_cast<const uint8_t*>(d->shared_w1);
  g.ws_x = d->shared_w1_scale;
  g.row_coeff = pa.coeff;
  g.y32 = reinterpret_cast<float*>(ws + L.mid);
  g.ldy = I;
  g.bmax = pa.bmax;
  g.bshift = L.qb == 512 ? 9 : 7;
  g.ldb = L.nbm;
  // the M tile sized for 16 rows whatever T is: routed experts hold about
  // T * topk / E rows, and a 64-row tile's activation loads and MFMAs cost
  // more than the shared expert's extra passes over its weights
  int rc = qmoe_skinny_launch(QK_W8A8_BLK, g, std::min(T, 16), L.slots, nullptr, 0, 1, stream);
  if (rc != QMOE_OK) return rc;

  hipLaunchKernelGGL(decode_mid_quant_kernel, dim3((unsigned)L.R), dim3(kPrep), 0, stream, g.y32, pa.bmax,
                     pa.goffs, d->E, T, I, Is, L.qb, L.nbm, ws + L.mq, reinterpret_cast<float*>(ws + L.msc));
  if (hipGetLastError() != hipSuccess) return QMOE_ERR_LAUNCH;

  DownArgs da{};
  da.mq = ws + L.mq;
  da.msc = reinterpret_cast<const float*>(ws + L.msc);
  da.nbm = L.nbm;
  da.qsh = L.qb == 512 ? 2 : 0;
  da.R = L.R;
  da.map = pa.map;
  da.active = pa.active;
  da.nact = pa.nact;
  da.slots = L.slots;
  da.T = T;
  da.H = H;
  da.I = I;
  da.Is = Is;
  da.w2 = static_cast<const uint8_t*>(d->w2);
  da.w2x = static_cast<const uint8_t*>(d->shared_w2);
  da.ws2 = d->w2_scale;
  da.ws2x = d->shared_w2_scale;
  da.out = d->out;
  da.ldo = d->ldo;
  da.splits = L.splits;
  da.partial = L.splits > 1 ? reinterpret_cast<float*>(ws + L.part) : nullptr;
  if (T <= 16) {
    if (I <= 2048) launch_down<1, 1, 4, 4>(da, tiles, stream);
    else launch_down<1, 1, 8, 4>(da, tiles, stream);
  } else {
    launch_down<4, 1, 2, 8>(da, tiles, stream);
  }
  if (hipGetLastError() != hipSuccess) return QMOE_ERR_LAUNCH;
  if (L.splits > 1) {
    const int64_t n = (int64_t)T * H;
    hipLaunchKernelGGL(decode_down_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       da.partial, L.splits, T, H, d->out, d->ldo);
  }
  return hipGetLastError() == hipSuccess ? QMOE_OK : QMOE_ERR_LAUNCH;
}
