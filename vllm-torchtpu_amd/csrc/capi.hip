// C ABI of the grouped GEMM: validates the descriptor and picks the skinny
// (weight-streaming, <= 64 rows per group) or the tiled (LDS/MFMA) kernel.

#include <algorithm>
#include <cstdlib>

#include "gemm_route.h"

// defined in gemm_skinny.hip / gemm_tiled.hip / gemm_f8.hip
void qmoe_skinny_plan(int kind, int64_t M, int64_t N, int64_t K, int act, int slots, int rows,
                      int ksplit_hint, int* ksplit_out, int64_t* ws_bytes);
int qmoe_skinny_launch(int kind, GemmParams p, int max_rows, int slots, void* workspace,
                       int64_t ws_bytes, int ksplit_hint, hipStream_t st);
int qmoe_skinny_check(int kind, const GemmParams& p);
int qmoe_skinny_tile_rows(int max_rows);
bool qmoe_skinny_qa_fits(int64_t M, int64_t K, int ksplit);
int qmoe_tiled_launch(int kind, GemmParams p, void* workspace, int64_t ws_bytes, hipStream_t st);
int qmoe_tiled_plan(int kind, const GemmParams& p, int* tile, int* ksplit, int64_t* ws_bytes);
bool qmoe_f8_plan(const GemmParams& p, bool blk, int* bm_out, int* ksplit_out, int64_t* ws_bytes, int* bn_out);
int qmoe_f8_launch(GemmParams p, bool blk, void* workspace, int64_t ws_bytes, hipStream_t st);
int qmoe_mx_plan(const GemmParams& p);
int qmoe_mx_launch(GemmParams p, hipStream_t st);
bool qmoe_f8_persistent(const GemmParams& p, bool blk);
bool qmoe_w4_plan(const GemmParams& p, int fmt, int* bm_out, int* ksplit_out, int64_t* ws_bytes);
int qmoe_w4_launch(GemmParams p, int fmt, void* workspace, int64_t ws_bytes, hipStream_t st);

namespace {

constexpr int kSkinnyMaxRows = 64;
constexpr int kSkinnyMaxGroupRows = 8;
constexpr int kSkinnyMaxGroupRowsBlk = 3;
constexpr int kSkinnyMaxRowsW8A8 = 32;  // also dense e2m1
constexpr int kSkinnyMaxRowsBlkWide = 16;

}  // namespace

int qmoe_to_params(const qmoe_gemm_desc* d, GemmParams* p) {
  if (!d) return QMOE_ERR_ARG;
  if (d->kind < QMOE_W8A8_PC || d->kind > QMOE_W8A8_PC_DYN) return QMOE_ERR_ARG;
  // weight codes: 0 e4m3, 1 int8, 2 e5m2 (the per-channel and grouped-matmul
  // W8A8 kinds); the other kinds name their formats themselves
  if (d->kind == QMOE_W8A8_PC || d->kind == QMOE_W8A8_GMM || d->kind == QMOE_W8A8_PC_DYN) {
    if (d->wfmt < 0 || d->wfmt > 2) return QMOE_ERR_ARG;
  } else if (d->wfmt != 0) {
    return QMOE_ERR_ARG;
  }
  // bf16 rows quantized inside: dense problems only
  if (d->kind == QMOE_W8A8_PC_DYN && (d->group_offs || d->a_rows)) return QMOE_ERR_ARG;
  if (d->act < QMOE_ACT_NONE || d->act > QMOE_ACT_SITU) return QMOE_ERR_ARG;
  if (d->M < 0 || d->N <= 0 || d->K <= 0 || d->slots <= 0) return QMOE_ERR_ARG;
  if (!d->a || !d->w || !d->y) return QMOE_ERR_ARG;
  if ((d->kind == QMOE_W8A8_PC || d->kind == QMOE_W8A8_BLK || d->kind == QMOE_W8A8_GMM ||
       d->kind == QMOE_W4A4_MX) && !d->a_scale)
    return QMOE_ERR_ARG;
  // MX activations: e8m0 bytes per (row, 32 k) on both operands
  if (d->kind == QMOE_W4A4_MX && (d->lds_a < d->K / 32 || d->ldws < d->K / 32)) return QMOE_ERR_ARG;
  if (d->kind != QMOE_W16A16 && !d->w_scale) return QMOE_ERR_ARG;
  if (d->kind == QMOE_W8A8_BLK && (d->ws_bn <= 0 || (d->K % 128) != 0)) return QMOE_ERR_ARG;
  // grouped-matmul recipe: activation scales per 512 columns, per-channel weights
  if (d->kind == QMOE_W8A8_GMM && ((d->K % 128) != 0 || d->lds_a < (d->K + 511) / 512)) return QMOE_ERR_ARG;
  if (d->kind == QMOE_W8A16_BLK && (d->ws_bn <= 0 || (d->K % 128) != 0 || d->ldws < d->K / 128))
    return QMOE_ERR_ARG;
  if (d->act != QMOE_ACT_NONE && (d->N % 2) != 0) return QMOE_ERR_ARG;
  if (d->active && (!d->num_active || !d->group_offs)) return QMOE_ERR_ARG;
  if (!d->group_offs && d->slots != 1) return QMOE_ERR_ARG;
  // 16-byte loads along K
  const bool w4 = kind_w4(d->kind) || d->kind == QMOE_W4A4_MX;
  const int wbytes = w4 ? d->K / 2 : (d->kind == QMOE_W16A16 ? 2 * d->K : d->K);
  if (d->ldw < wbytes || (d->ldw % 16) != 0 || (d->K % 32) != 0) return QMOE_ERR_ARG;
  // NVFP4 scales: bf16 [N][ldws >= K/16], 4-byte aligned pairs
  if (d->kind == QMOE_W4A16_NV && (d->ldws < d->K / 16 || (d->ldws % 2) != 0 || (d->ws_gstride % 2) != 0 ||
                                   (reinterpret_cast<uintptr_t>(d->w_scale) & 3)))
    return QMOE_ERR_ARG;
  // INT4 scales: bf16 [N][ldws >= K/group], group 32, 64 or 128
  if (d->kind == QMOE_W4A16_I4 &&
      ((d->wq_group != 32 && d->wq_group != 64 && d->wq_group != 128) || (d->K % d->wq_group) != 0 ||
       d->ldws < d->K / d->wq_group || (reinterpret_cast<uintptr_t>(d->w_scale) & 1)))
    return QMOE_ERR_ARG;
  const bool abf16 = kind_abf16(d->kind) || d->kind == QMOE_W8A8_PC_DYN;
  // packed e2m1 activations: lda counts bytes (two codes each)
  const int abytes = d->kind == QMOE_W4A4_MX ? d->K / 2 : d->K;
  if (d->lda < abytes || ((d->lda * (abf16 ? 2 : 1)) % 16) != 0) return QMOE_ERR_ARG;
  const int nout = d->act != QMOE_ACT_NONE ? d->N / 2 : d->N;
  if (d->ldy < nout) return QMOE_ERR_ARG;
  *p = GemmParams{};
  p->a = d->a;
  p->lda = d->lda;
  p->a_scale = d->a_scale;
  p->lds_a = d->lds_a;
  p->a_rows = d->a_rows;
  p->w = static_cast<const uint8_t*>(d->w);
  p->ldw = d->ldw;
  p->w_gstride = d->w_gstride;
  p->w_scale = d->w_scale;
  p->ldws = d->ldws;
  p->ws_gstride = d->ws_gstride;
  p->ws_bn = d->ws_bn > 0 ? d->ws_bn : 1;
  p->a_kshift = 0;
  p->w_kshift = 0;
  if (d->kind == QMOE_W8A8_GMM) {
    // onto the block-scale kernels: 512-column activation blocks; one weight
    // scale per row ([G][N], ldws <= 1) or per (row, B columns) with
    // B = K / ldws a power-of-two multiple of 512 ([G][N][K/B])
    p->a_kshift = 2;
    p->ws_bn = 1;
    if (d->ldws <= 1) {
      p->w_kshift = 31;
      p->ldws = 1;
    } else {
      if (d->K % d->ldws != 0) return QMOE_ERR_ARG;
      const int B = d->K / (int)d->ldws;
      int sh = -1;
      for (int j = 2; j < 20; ++j)
        if (B == (128 << j)) sh = j;
      if (sh < 0) return QMOE_ERR_ARG;
      p->w_kshift = sh;
    }
  }
  p->wq_group = d->wq_group;
  p->bias = d->bias;
  p->bias_gstride = d->bias_gstride;
  p->group_offs = d->group_offs;
  p->active = d->active;
  p->num_active = d->num_active;
  p->slots = d->slots;
  p->M = d->M;
  p->N = d->N;
  p->K = d->K;
  p->wfmt = d->wfmt;
  p->act = d->act;
  p->act_p0 = d->act_p0;
  p->act_p1 = d->act_p1;
  p->row_weight = d->row_weight;
  p->y = static_cast<uint16_t*>(d->y);
  p->ldy = d->ldy;
  p->y_rows = d->y_rows;
  p->ksplit = 1;
  return QMOE_OK;
}

namespace {

// Kernel kind of a descriptor kind: the grouped-matmul recipe runs on the
// block-scale kernels (its shifts are set in qmoe_to_params); bf16 rows
// quantized inside run on the per-channel kernels
int kernel_kind(const qmoe_gemm_desc* d) {
  if (d->kind == QMOE_W8A8_PC_DYN) return QK_W8A8_PC;
  return d->kind == QMOE_W8A8_GMM ? QK_W8A8_BLK : d->kind;
}

// Grid depth of the skinny kernel: every group, or -- with an active list --
// at most one slot per row (a listed group has at least one row).
int skinny_slots(const qmoe_gemm_desc* d) {
  return d->active ? std::max(1, std::min(d->slots, d->M)) : d->slots;
}

// Rows the skinny kernel's M tile is sized for: all rows of a dense
// problem; for a grouped one the average rows per routed group (groups
// above it take extra 16-row passes over their weight slice, from cache).
int skinny_rows(const qmoe_gemm_desc* d) {
  if (!d->group_offs) return d->M;
  const int groups = std::max(1, std::min(skinny_slots(d), d->M));
  const int avg = (d->M + groups - 1) / groups;
  return std::max(1, std::min(std::min(d->max_rows, d->M), avg));
}

// Dense problems take the skinny kernel up to 64 rows (32 for W8A8, whose
// tiled kernel is faster from there on); grouped ones while the routed
// experts average at most 8 rows (measured on MI355X: beyond that the tiled
// kernel's weight reuse across rows wins).
bool use_skinny(const qmoe_gemm_desc* d) {
  const char* env = getenv("QMOE_SKINNY_MAX_ROWS");  // tuning knob
  int lim = d->group_offs ? kSkinnyMaxGroupRows : kSkinnyMaxRows;
  if (!d->group_offs && (d->kind == QMOE_W8A8_PC || d->kind == QMOE_W8A8_GMM)) lim = kSkinnyMaxRowsW8A8;
  // wide dense block-scaled problems (>= 16384 output channels): the tiled
  // kernel with a K split wins from 17 rows (measured on MI355X, K 7168)
  const int nout = d->act != QMOE_ACT_NONE ? d->N / 2 : d->N;
  if (!d->group_offs && d->kind == QMOE_W8A8_BLK && nout >= 16384) lim = kSkinnyMaxRowsBlkWide;
  // grouped block-scaled (DeepSeek-V3 experts): the tiled kernel's 32-token
  // tiles win from 4 rows per routed expert (measured on MI355X, 256 experts,
  // top 8: 192 tokens 1309 vs 1466 us, 256 tokens 1432 vs 1704 us)
  if (d->group_offs && (d->kind == QMOE_W8A8_BLK || d->kind == QMOE_W8A8_GMM)) lim = kSkinnyMaxGroupRowsBlk;
  // dense e2m1 (MXFP4 / NVFP4): the tiled kernel's 32-token tiles with a K
  // split win from 33 rows (measured on MI355X, K 2880, N 5760)
  if (!d->group_offs && (d->kind == QMOE_W4A16_MX || d->kind == QMOE_W4A16_NV)) lim = kSkinnyMaxRowsW8A8;
  if (env) lim = atoi(env);
  return skinny_rows(d) <= lim;
}

// the W4A16 tiled kernel's format code: 0 MXFP4, 1 NVFP4, 2 INT4
int w4_fmt(const qmoe_gemm_desc* d) {
  return d->kind == QMOE_W4A16_NV ? 1 : (d->kind == QMOE_W4A16_I4 ? 2 : 0);
}

bool use_w4(const qmoe_gemm_desc* d) {
  // the generic kernel has no NVFP4 / INT4 form
  if (d->kind == QMOE_W4A16_NV || d->kind == QMOE_W4A16_I4) return true;
  return d->kind == QMOE_W4A16_MX && !getenv("QMOE_W4_OFF");  // tuning knob: generic kernel only
}

bool use_f8(const qmoe_gemm_desc* d) {
  if (getenv("QMOE_F8_OFF")) return false;  // tuning knob: generic kernel only
  const bool blk = d->kind == QMOE_W8A8_BLK || d->kind == QMOE_W8A8_GMM;
  return d->kind == QMOE_W8A8_PC || (blk && !getenv("QMOE_F8_BLK_OFF"));
}

// Kernel paths of qmoe_gemm (reported by qmoe_gemm_plan).
enum Path {
  kPathSkinny = 0,      // weight streaming (decode)
  kPathF8 = 1,          // 1-byte x 1-byte tiles
  kPathW4 = 2,          // bf16 x 4-bit tiles
  kPathTiled = 3,       // generic tiles
  kPathSkinnyPass = 4,  // weight streaming in 64-row passes (K outside every tiled granule)
  kPathF8Persistent = 5,  // 1-byte x 1-byte tiles (256 or 128 tokens), persistent workgroups
  kPathMx = 6,            // e2m1 x e2m1 with e8m0 scales on both, 256 x 256 persistent tiles
  kPathMxTiles = 7,       // the same operands, grouped tiles (one tile per workgroup)
  kPathSkinnyDyn = 8,     // weight streaming with the per-row activation quantization inside
  kPathF8Narrow = 9,      // 1-byte x 1-byte tiles of 128 weight rows
  kPathSkinnyRows = 10,   // weight streaming, one slice of rows per grid.z index
};

// Dense problems of a few dozen rows can stream the weights once per slice
// of 16 rows: one slice per grid.z index, every slice's workgroups
// streaming the whole weight matrix (the slices of one weight tile meet its
// bytes in one XCD's L2). Measured on MI355X: e2m1 weights (K 2880, N 5760)
// at 17 / 32 / 64 rows 8.4 / 11.0 / 15.8 -> 8.0 / 10.5 / 13.8 us (slower
// from 128 rows); 1-byte weights only while the slices keep the grid near
// one workgroup per CU -- the FP8 down projection (K 14336, N 4096, 128
// tiles per slice) at 32 rows 21.2 -> 14.8 us with no K split, while the up
// projection (448 tiles per slice) loses 17.1 -> 20.3 us. 0: not this route.
int dense_row_split(const qmoe_gemm_desc* d) {
  if (d->group_offs || d->active || d->M <= 16) return 0;
  const char* env = getenv("QMOE_SKINNY_ROW_SPLIT");  // tuning knob: 0 off, 16 / 32 / 64 forced up to 256 rows
  if (env) {
    const int rs = atoi(env);
    const bool ok = (rs == 16 || rs == 32 || rs == 64) && d->M > rs && d->M <= 256 && d->kind != QMOE_W4A4_MX &&
                    d->kind != QMOE_W8A8_PC_DYN;
    return ok ? rs : 0;
  }
  if (d->kind == QMOE_W4A16_MX || d->kind == QMOE_W4A16_NV) return d->M <= 64 ? 16 : 0;
  if (d->kind == QMOE_W8A8_PC && d->M <= 32) {
    const int64_t nout = d->act != QMOE_ACT_NONE ? d->N / 2 : d->N;
    const int64_t tiles = d->act != QMOE_ACT_NONE ? cdiv<int64_t>(nout, 16) : cdiv<int64_t>(nout, 32);
    return tiles * cdiv<int64_t>(d->M, 16) <= 320 ? 16 : 0;
  }
  return 0;
}

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

// QMOE_W8A8_PC_DYN: whether the streaming kernel quantizes the activations
// itself. Each of its workgroups reads every row for the absmax and then
// its K range again for the codes (two dependent L2 round trips before its
// first MFMA) instead of a separate quantizer launch; measured on MI355X
// (Llama-3-8B MLP shapes, FP8 and INT8) that pays for one row (up / down
// projection 14.3 -> 12.8 us / 16.5 -> 15.4 us) and for two rows of K 4096
// (15.0 -> 14.2 us), and loses for two rows of K 14336 and from four rows.
// Short rows over many channels lose too: DeepSeek-V3's kv_b projection (K
// 512, N 32768: 2048 workgroups each quantizing the row) 10.3 -> 8.3 us in
// two launches, so K of at least 1024 is required.
bool dyn_fused(const qmoe_gemm_desc* d, const GemmParams& p, int ksplit) {
  const char* env = getenv("QMOE_DYN_FUSE_ROWS");  // tuning knob: row limit
  const int lim = env ? std::min(atoi(env), 32) : (ksplit == 1 && d->K < 8192 ? 2 : 1);
  return d->M <= lim && d->act == QMOE_ACT_NONE && (d->K % 128) == 0 && d->K >= 1024 &&
         qmoe_skinny_check(QK_W8A8_PC, p) == QMOE_OK;
}

// K slices of the in-kernel form: one for a single row (measured on MI355X,
// DeepSeek-V3's q_a / kv_a projections, K 7168, N 1536 / 576: the 2 / 5
// slices the streaming planner picks for their few weight tiles, and the
// finishing launch they need, 8.7 / 8.5 -> 7.6 / 7.5 us), else the
// streaming planner's choice (0).
int dyn_split_hint(const qmoe_gemm_desc* d) { return d->M == 1 ? 1 : 0; }

// The two-step form of a QMOE_W8A8_PC_DYN problem: codes [M][K] and scales
// [M] at the start of the workspace (qmoe_row_quant mode 0), then the
// QMOE_W8A8_PC problem over them with the rest of the workspace.
int64_t dyn_prefix(const qmoe_gemm_desc* d) {
  return align256((int64_t)d->M * d->K) + align256(4 * (int64_t)std::max(d->M, 1));
}

qmoe_gemm_desc dyn_inner(const qmoe_gemm_desc* d, uint8_t* ws) {
  qmoe_gemm_desc e = *d;
  e.kind = QMOE_W8A8_PC;
  e.a = ws;
  e.lda = d->K;
  e.a_scale = reinterpret_cast<const float*>(ws + align256((int64_t)d->M * d->K));
  e.lds_a = 1;
  return e;
}

// The one place that decides which kernel runs a problem: the streaming
// kernel within its row limits (unless it declines the operands), else the
// format's tiled kernel, else the generic tiled kernel, else the streaming
// kernel in 64-row passes. The tiled kernels enumerate m-tiles over all
// groups; the active list is a streaming-path device (it bounds the grid by
// the number of routed experts), so `p` has it cleared for them.
}  // namespace

int qmoe_route_of(const qmoe_gemm_desc* d, GemmParams& p, QmoeRoute* r) {
  const int kind = kernel_kind(d);
  if (d->kind == QMOE_W8A8_PC_DYN) {
    int ks = 1;
    int64_t ws = 0;
    qmoe_skinny_plan(QK_W8A8_PC, d->M, d->N, d->K, d->act, 1, d->M, dyn_split_hint(d), &ks, &ws);
    if (dyn_fused(d, p, ks)) {  // one launch; the row scales first in the workspace
      if (qmoe_skinny_qa_fits(d->M, d->K, ks)) {
        *r = QmoeRoute{kPathSkinnyDyn, qmoe_skinny_tile_rows(d->M), ks, ws + align256(4 * (int64_t)d->M)};
        return QMOE_OK;
      }
    }
    // placeholder workspace address (256-aligned, as device allocations
    // are): the plan reads no memory; the launch plans again with the real one
    const qmoe_gemm_desc e = dyn_inner(d, reinterpret_cast<uint8_t*>((uintptr_t)1 << 24));
    GemmParams pe;
    int st = qmoe_to_params(&e, &pe);
    if (st == QMOE_OK) st = qmoe_route_of(&e, pe, r);
    if (st == QMOE_OK) r->ws_bytes += dyn_prefix(d);
    return st;
  }
  if (kind == QK_W4A4_MX) {  // the MX kernels take MX activations, nothing else does
    const int bm = qmoe_mx_plan(p);
    if (!bm) return QMOE_ERR_ARG;
    *r = QmoeRoute{p.group_offs ? kPathMxTiles : kPathMx, bm, 1, 0};
    return QMOE_OK;
  }
  if (const int rs = dense_row_split(d)) {
    if (qmoe_skinny_check(kind, p) == QMOE_OK) {
      *r = QmoeRoute{kPathSkinnyRows, rs, 1, 0};
      return QMOE_OK;
    }
  }
  if (use_skinny(d) && qmoe_skinny_check(kind, p) == QMOE_OK) {
    r->path = kPathSkinny;
    r->tile_m = qmoe_skinny_tile_rows(skinny_rows(d));
    qmoe_skinny_plan(kind, d->M, d->N, d->K, d->act, skinny_slots(d), skinny_rows(d), 0, &r->ksplit,
                     &r->ws_bytes);
    return QMOE_OK;
  }
  const bool skinny_first = use_skinny(d);
  p.active = nullptr;
  p.num_active = nullptr;
  if (!skinny_first) {
    int bm = 0, ks = 1;
    int64_t ws = 0;
    int bn = 256;
    if (use_f8(d) && qmoe_f8_plan(p, kind == QK_W8A8_BLK, &bm, &ks, &ws, &bn)) {
      const int path = bn == 128 ? kPathF8Narrow
                                 : (qmoe_f8_persistent(p, kind == QK_W8A8_BLK) ? kPathF8Persistent : kPathF8);
      // persistent tiles hold 128 or 256 tokens (a 64-token plan runs 128)
      *r = QmoeRoute{path, path == kPathF8Persistent ? std::max(bm, 128) : bm, ks, ws};
      return QMOE_OK;
    }
    if (!use_f8(d) && use_w4(d) && qmoe_w4_plan(p, w4_fmt(d), &bm, &ks, &ws)) {
      *r = QmoeRoute{kPathW4, bm, ks, ws};
      return QMOE_OK;
    }
  }
  int tile = 128, tks = 1;
  int64_t tws = 0;
  if (qmoe_tiled_plan(kind, p, &tile, &tks, &tws) == QMOE_OK) {
    *r = QmoeRoute{kPathTiled, tile, tks, tws};
    return QMOE_OK;
  }
  // bf16 activations with K % 64 == 32 (no tiled granule): the streaming
  // kernel takes any K % 32 == 0, in passes of 64 rows per group
  if (!skinny_first && qmoe_skinny_check(kind, p) == QMOE_OK) {
    *r = QmoeRoute{kPathSkinnyPass, qmoe_skinny_tile_rows(kSkinnyMaxRows), 1, 0};
    return QMOE_OK;
  }
  return QMOE_ERR_ARG;
}

int qmoe_run_route(const qmoe_gemm_desc* d, const QmoeRoute& r, GemmParams p, void* workspace,
                   int64_t ws_bytes, hipStream_t stream) {
  const int kind = kernel_kind(d);
  if (d->kind == QMOE_W8A8_PC_DYN) {
    uint8_t* w8 = static_cast<uint8_t*>(workspace);
    if (!w8 || ws_bytes < r.ws_bytes) return QMOE_ERR_WORKSPACE;
    if (r.path == kPathSkinnyDyn) {
      const int64_t sc = align256(4 * (int64_t)d->M);
      p.a_quant = 1;
      p.a_scale = reinterpret_cast<const float*>(w8);
      p.lds_a = 1;
      return qmoe_skinny_launch(QK_W8A8_PC, p, d->M, 1, w8 + sc, ws_bytes - sc, dyn_split_hint(d), stream);
    }
    const qmoe_gemm_desc e = dyn_inner(d, w8);
    int st = qmoe_row_quant(d->a, d->lda, 0, d->M, d->K, d->wfmt, 0, 0, w8, d->K, const_cast<float*>(e.a_scale), 1,
                            stream);
    if (st != QMOE_OK) return st;
    GemmParams pe;
    QmoeRoute re;
    st = qmoe_to_params(&e, &pe);
    if (st == QMOE_OK) st = qmoe_route_of(&e, pe, &re);
    if (st != QMOE_OK) return st;
    const int64_t pre = dyn_prefix(d);
    return qmoe_run_route(&e, re, pe, w8 + pre, ws_bytes - pre, stream);
  }
  switch (r.path) {
    case kPathSkinnyRows: {
      GemmParams q;
      qmoe_to_params(d, &q);
      q.row_split = r.tile_m;
      return qmoe_skinny_launch(kind, q, r.tile_m, (int)cdiv<int64_t>(d->M, r.tile_m), workspace, ws_bytes, 1, stream);
    }
    case kPathSkinny: {
      GemmParams q;
      qmoe_to_params(d, &q);  // keeps the active list
      return qmoe_skinny_launch(kind, q, skinny_rows(d), skinny_slots(d), workspace, ws_bytes, 0, stream);
    }
    case kPathF8:
    case kPathF8Narrow:
    case kPathF8Persistent: return qmoe_f8_launch(p, kind == QK_W8A8_BLK, workspace, ws_bytes, stream);
    case kPathW4: return qmoe_w4_launch(p, w4_fmt(d), workspace, ws_bytes, stream);
    case kPathTiled: return qmoe_tiled_launch(kind, p, workspace, ws_bytes, stream);
    case kPathMx:
    case kPathMxTiles: return qmoe_mx_launch(p, stream);
    default: {
      GemmParams q;
      qmoe_to_params(d, &q);
      return qmoe_skinny_launch(kind, q, kSkinnyMaxRows, skinny_slots(d), workspace, ws_bytes, 1, stream);
    }
  }
}

extern "C" int qmoe_abi_version(void) { return 8; }

extern "C" int qmoe_gemm_workspace_size(const qmoe_gemm_desc* d, int64_t* bytes) {
  GemmParams p;
  const int st = qmoe_to_params(d, &p);
  if (st != QMOE_OK) return st;
  QmoeRoute r;
  *bytes = qmoe_route_of(d, p, &r) == QMOE_OK ? r.ws_bytes : 0;
  return QMOE_OK;
}

extern "C" int qmoe_gemm_plan(const qmoe_gemm_desc* d, int32_t* path, int32_t* tile_m, int32_t* ksplit) {
  GemmParams p;
  const int st = qmoe_to_params(d, &p);
  if (st != QMOE_OK) return st;
  QmoeRoute r;
  const int rc = qmoe_route_of(d, p, &r);
  if (rc != QMOE_OK) return rc;
  if (path) *path = r.path;
  if (tile_m) *tile_m = r.tile_m;
  if (ksplit) *ksplit = r.ksplit;
  return QMOE_OK;
}

extern "C" int qmoe_gemm(const qmoe_gemm_desc* d, void* workspace, int64_t ws_bytes,
                         hipStream_t stream) {
  GemmParams p;
  const int st = qmoe_to_params(d, &p);
  if (st != QMOE_OK) return st;
  if (d->M == 0) return QMOE_OK;
  QmoeRoute r;
  const int rc = qmoe_route_of(d, p, &r);
  if (rc != QMOE_OK) return rc;
  return qmoe_run_route(d, r, p, workspace, ws_bytes, stream);
}

