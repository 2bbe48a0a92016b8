/*
 * qmoe — C ABI of the MI355X (gfx950) quantized-GEMM / fused-MoE library.
 *
 * Every entry point takes raw device pointers, sizes and a hipStream_t, is
 * asynchronous on that stream, allocates nothing, and returns a status:
 *   0 QMOE_OK, 1 QMOE_ERR_ARG (bad shape / unsupported combination),
 *   2 QMOE_ERR_WORKSPACE (workspace too small), 3 QMOE_ERR_LAUNCH,
 *   4 QMOE_ERR_SCRATCH (qmoe_gemm_static: partial sums exceed its scratch).
 * Layouts (all row-major):
 *   activations  [rows, K]            bf16 (uint16 bit patterns) or 1-byte codes
 *   weights      [G][N][K]            N-major: each output channel's K contiguous
 *                                     (e2m1: [G][N][K/2], low nibble = even k)
 *   scales       per-channel f32 [G][N]; block f32 [G][N/bn][K/128];
 *                MX e8m0 bytes [G][N][K/32]; NVFP4 bf16 [G][N][K/16];
 *                INT4 bf16 [G][N][K/wq_group]
 * Reference paths below are relative to the reference plugin's
 * src/vllm_torchtpu/.
 */
#ifndef QMOE_H_
#define QMOE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* qmoe_stream_t; /* == hipStream_t */

/* GEMM kinds (qmoe_gemm_desc.kind) */
enum {
  QMOE_W8A8_PC = 0,  /* A e4m3|int8|e5m2 (wfmt) + per-row f32 scale; W same dtype + per-channel
                        f32 scale */
  QMOE_W8A8_BLK = 1, /* A e4m3 + per-(row,128) scale; W e4m3 + per-(n/bn, 128) scale */
  QMOE_W8A16_PC = 2, /* A bf16; W e4m3 + per-channel scale */
  QMOE_W4A16_MX = 3, /* A bf16; W e2m1 + e8m0 scale per 32 k */
  QMOE_W16A16 = 4,   /* A bf16; W bf16 */
  QMOE_W4A16_NV = 5, /* A bf16; W e2m1 + bf16 scale per 16 k (NVFP4: the checkpoint's e4m3
                        block scale times its f32 global scale, rounded to bf16 as the
                        reference's `kernels/megablox/gmm_v2.py:452-462` dequantization
                        does; each weight is bf16(code * scale)) */
  QMOE_W8A8_GMM = 7, /* A e4m3|int8 codes + f32 scale per (row, 512 columns, the last
                        block partial) from qmoe_row_quant mode 2; W e4m3|int8|e5m2 (wfmt; A is
                        int8 for int8 W, e4m3 for float W) + per-channel f32
                        scale [G][N] (ldws <= 1) or one per (row, B columns) [G][N][K/B] with
                        ldws = K/B, B a power-of-two multiple of 512. The quantized-lhs regime
                        of the reference's grouped
                        matmul, `kernels/megablox/gmm_v2.py:500-548, 1198-1237` (weights with
                        quant blocks of 256 or more columns: per-channel experts) */
  QMOE_W8A16_BLK = 8, /* A bf16; W e4m3 + f32 scale per (n / ws_bn, 128 k) [G][N/bn][K/128];
                        each weight is bf16(code * bf16(scale)) before the product: the
                        dequantize-before-matmul regime of `kernels/megablox/gmm_v2.py:452-462`
                        (quant blocks below 256 columns) */
  QMOE_W4A16_I4 = 6, /* A bf16; W symmetric 4-bit integers in the compressed-tensors
                        encoding (nibble = value + 8, two per byte, even k in the low
                        nibble: the int32 carriers of `compressed_tensors_moe_w4a16.py`
                        read as bytes) + bf16 scale per wq_group k; each weight is
                        bf16(value * scale), `kernels/megablox/gmm_v2.py:452-462` */
  QMOE_W4A4_MX = 9,  /* A e2m1 codes packed as W (lda in bytes >= K/2) + e8m0 bytes per
                        (row, 32 k) in a_scale [M, lds_a >= K/32] (qmoe_mx_quant); W as
                        QMOE_W4A16_MX. Both scales go to the MFMA. Opt-in MX activations
                        (no counterpart in the reference, whose W4A4 method runs W4A16,
                        `compressed_tensors_moe_w4an_mxfp4.py:49-55`). Dense: bias only;
                        grouped: fused activation, bias, row maps and routing weight as
                        the other kinds (a_rows also gathers the scale rows); no K split;
                        K % 512 == 0 and K >= 1024 (pad with zero codes) */
  QMOE_W8A8_PC_DYN = 10 /* A bf16 rows (lda in elements, a multiple of 8), quantized per row
                        inside the call with the runtime recipe of
                        `kernels/quantized_matmul/util.py:294-318` (quantize_block: scale =
                        absmax / qmax, e4m3 / e5m2 in f32 or int8 in bf16 arithmetic per wfmt;
                        qmoe_row_quant mode 0 computes the same codes); W and w_scale as
                        QMOE_W8A8_PC; a_scale unused. The whole xla_quantized_matmul of
                        `:80-124` in one call. Dense only (no group_offs). Decode-size
                        problems quantize inside the weight-streaming kernel (one launch: each
                        workgroup reads its rows' absmax from L2 while its first weight loads
                        are in flight); the rest quantize into the workspace first. The
                        workspace also holds the row scales, so it is needed whatever the
                        plan (qmoe_gemm_workspace_size) */
};

/* Fused gate/up activations (qmoe_gemm_desc.act) */
enum {
  QMOE_ACT_NONE = 0,
  QMOE_ACT_SILU = 1,
  QMOE_ACT_SWIGLUOAI = 2, /* p0 = alpha (1.702), p1 = limit (7.0) */
  QMOE_ACT_GELU_TANH = 3,
  QMOE_ACT_SILU_CLAMP = 4, /* p0 = limit (10.0) */
  QMOE_ACT_SITU = 5        /* p0 = beta, p1 = linear_beta (<= 0: none) */
};

/*
 * Grouped GEMM problem. For each group g (one group when group_offs is NULL)
 * and compact row R in [group_offs[g], group_offs[g+1]):
 *   acc[R, n] = sum_k A[a_rows ? a_rows[R] : R, k] * W[g, n, k]
 *   v = scales(acc) (+ bias[g, n]); with act: out[n] = act(v[n], v[n + N/2])
 *   out *= row_weight[R] (bf16, optional)
 *   Y[y_rows ? y_rows[R] : R, n] = bf16(out)
 */
typedef struct qmoe_gemm_desc {
  int32_t kind;           /* QMOE_W8A8_PC ... */
  int32_t wfmt;           /* QMOE_W8A8_PC, _GMM, _PC_DYN: 0 e4m3, 1 int8, 2 e5m2; other kinds 0 */
  const void* a;          /* activation codes or bf16 */
  int64_t lda;            /* elements (W4A4_MX: bytes of packed codes) */
  const float* a_scale;   /* W8A8: [rows] or [rows, lds_a]; W4A4_MX: e8m0 bytes [rows, lds_a] */
  int64_t lds_a;
  const int32_t* a_rows;  /* optional gather map [M] */
  const void* w;
  int64_t ldw;            /* bytes per weight row */
  int64_t w_gstride;      /* bytes per group */
  const void* w_scale;
  int64_t ldws;           /* elements per scale row */
  int64_t ws_gstride;     /* elements per group */
  int32_t ws_bn;          /* W8A8_BLK: weight rows per scale row (1 or 128) */
  const float* bias;      /* optional [G, N] */
  int64_t bias_gstride;
  const int32_t* group_offs; /* optional [G+1] */
  const int32_t* active;     /* optional slot -> group list (non-empty groups) */
  const int32_t* num_active; /* device scalar, valid slots in `active` */
  int32_t slots;          /* number of groups (or capacity of `active`) */
  int32_t max_rows;       /* host bound on rows of any one group */
  int32_t M;              /* total compact rows */
  int32_t N;              /* weight rows (2*I with a fused activation) */
  int32_t K;
  int32_t act;
  float act_p0, act_p1;
  const uint16_t* row_weight; /* optional bf16 [M] */
  void* y;                /* bf16 output */
  int64_t ldy;
  const int32_t* y_rows;  /* optional scatter map [M] */
  int32_t wq_group;       /* QMOE_W4A16_I4: k values per scale (32, 64 or 128) */
} qmoe_gemm_desc;

/* ABI revision of this header (bumped on any layout change). */
int qmoe_abi_version(void);

/*
 * Row quantizer: rows of x (bf16, or f32 when in_f32) -> 1-byte codes q and
 * f32 scales (one per row, or per (row, 128 columns) when block == 128).
 *   qdtype 0 e4m3fn, 1 int8, 2 e5m2 (per-row scales only; not mode 2, whose codes are
 *   e4m3 for any float weight: `kernels/megablox/gmm_v2.py:1198-1218`).
 *   mode 0: runtime activation quant, replaces the reference's
 *           `kernels/quantized_matmul/util.py:47-64` quantize_tensor /
 *           `:294-318` quantize_block (fp8 in f32, int8 in bf16 arithmetic);
 *   mode 1: load-time weight quant, replaces
 *           `layers/core/quantization.py:232-318` quantize_tensor
 *           (reciprocal-multiply scale, zero rows keep scale 0).
 */
int qmoe_row_quant(const void* x, int64_t ldx, int in_f32, int64_t M, int64_t K, int qdtype,
                   int mode, int block, void* q, int64_t ldq, float* scales, int64_t lds,
                   qmoe_stream_t stream);

/*
 * MX activation quantizer: bf16 rows x [M, K] (K % 32 == 0) -> e2m1 codes
 * packed two per byte (low nibble = even column) q [M, ldq >= Kp/2] and e8m0
 * bytes scales [M, lds >= Kp/32], columns K..Kp-1 (Kp % 32 == 0) as zero
 * blocks (codes 0, byte 0); and/or (xq != NULL) the dequantized values as
 * bf16 [M, ldxq >= K], exact. Per 32-column block: the reference's ue8m0
 * block rule, `layers/core/quantization.py:232-318` (`quantize_tensor` with
 * use_ue8m0, scale = amax * f32(1/6) snapped up to a power of two) and its
 * e2m1 encoder `compressed_tensors_moe/utils.py:167-183`
 * (`quantize_to_fp4_e2m1_nibbles`). The reference's W4A4 MXFP4 method runs
 * its activations unquantized; this is the activation side of the opt-in
 * QMOE_W4A4_MX GEMM. At least one of q, xq. A block holding an inf or NaN
 * (the reference's rule has no answer for it) gets codes 0 and byte 255,
 * the e8m0 NaN encoding: it reads back as NaN (xq: bf16 NaN) and the row's
 * other blocks keep their own codes.
 */
int qmoe_mx_quant(const void* x, int64_t ldx, int64_t M, int64_t K, int64_t Kp, void* q, int64_t ldq,
                  void* scales, int64_t lds, void* xq, int64_t ldxq, qmoe_stream_t stream);

/* Workspace bytes qmoe_gemm needs for this problem (split-K partials). */
int qmoe_gemm_workspace_size(const qmoe_gemm_desc* d, int64_t* bytes);

/*
 * The kernel choice qmoe_gemm makes for this problem, computed on the host
 * from the descriptor alone (no device memory is read): path 0 weight
 * streaming, 1 1-byte x 1-byte tiles, 2 bf16 x 4-bit tiles, 3 generic
 * tiles, 4 weight streaming in 64-row passes, 5 1-byte x 1-byte tiles of
 * 256 tokens x 256 or 224 weight rows, or 128 tokens x 224 rows, on
 * persistent workgroups (at most one per CU of the current device), 6 MX
 * 256 x 256 persistent tiles, 7 MX grouped tiles, 8 weight streaming with
 * the per-row activation quantization inside (QMOE_W8A8_PC_DYN; for the
 * kind's other problems the path of the GEMM after its separate
 * quantization), 9 1-byte x 1-byte tiles of 128 weight rows, 10 weight
 * streaming in slices of tile_m rows of a dense problem (one slice per
 * grid.z index, each streaming the whole weight matrix); tile_m = token rows
 * per tile (or per streaming pass or slice); ksplit = K slices. No counterpart in the
 * reference (its tiling is chosen inside the Pallas call,
 * `kernels/megablox/gmm_v2.py:922-1055`); it lets tests assert which kernel
 * instances they exercise. Any output pointer may be NULL.
 */
int qmoe_gemm_plan(const qmoe_gemm_desc* d, int32_t* path, int32_t* tile_m, int32_t* ksplit);

/*
 * Quantized (grouped) GEMM. One group replaces the dense runtime matmul of
 * `layers/adapter/linear_common.py:69-128` (_quantized_matmul_jax ->
 * `kernels/quantized_matmul/util.py:80-124` xla_quantized_matmul, and the
 * single-group gmm_v2 call for rank-4 scales) and `:188-209`
 * (_quantized_matmul_fp4_jax). Several groups replace the grouped matmul
 * `kernels/megablox/gmm_v2.py:1280-1443` (gmm_v2, incl. its fused
 * activation epilogue `:84-122`). The workspace holds split-K partial sums
 * of the small-M path; every call writes before it reads, so it needs no
 * initialisation, and calls that share one workspace must be ordered on one
 * stream.
 */
int qmoe_gemm(const qmoe_gemm_desc* d, void* workspace, int64_t ws_bytes, qmoe_stream_t stream);

/*
 * qmoe_gemm for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. Same kernels and results as qmoe_gemm; the
 * split-K partial sums go to a static device array of the library
 * (qmoe_gemm_static_scratch_bytes(), 64 MiB, held per GPU until the process
 * ends) instead of a caller workspace, and no call allocates or frees
 * anything. A problem whose partials exceed it returns QMOE_ERR_SCRATCH
 * before any launch. Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (other streams, other threads) race.
 */
int qmoe_gemm_static(const qmoe_gemm_desc* d, qmoe_stream_t stream);
int64_t qmoe_gemm_static_scratch_bytes(void);

/*
 * MoE routing for T tokens over E experts: scores, top-k, renormalize and
 * scale; weights written as bf16 (or f32 with weights_f32), ids int32 [T, k].
 * Replaces `layers/adapter/moe_routing.py:232-323` (select_experts) with the
 * sort-free top-k of `layers/core/rowmax_topk.py:28-61` (ties -> lowest id;
 * a row with no score above -3e38 gets NaN weights and ids 0..k-1).
 *   logits   : bf16 [T, E] (logits_f32 = 0) or f32 [T, E] (logits_f32 = 1)
 *   scoring  : 0 softmax, 1 sigmoid, 2 sqrtsoftplus, 3 none (logits are the
 *              scores: the reference's `layers/adapter/router_topk.py:42-50`
 *              rowmax_select)
 *   bias     : optional f32 [E] (choice = score + bias, weight = score)
 *   num_group/topk_group > 1: grouped selection (sum of top-2 per group with
 *   a bias, max without), the DeepSeek-V3 rule; upstream vLLM grouped_topk,
 *   called at `moe_routing.py:276-299`.
 */
int qmoe_moe_route(const void* logits, int logits_f32, int64_t T, int E, int topk, int scoring,
                   const float* bias, int renormalize, float routed_scaling_factor, int num_group,
                   int topk_group, void* topk_weights, int weights_f32, int32_t* topk_ids,
                   qmoe_stream_t stream);

/*
 * DeepSeek-V4 hash routing, replaces `layers/adapter/moe_routing.py:204-229`
 * (_hash_moe_select, taken by select_experts when the layer has a
 * hash_indices_table and input ids are given, `:259-274`): ids =
 * hash_table[input_ids[t]] (int32 [table_rows, topk]; input ids int32, or
 * int64 with ids_i64), weights = the row's scores (scoring as in
 * qmoe_moe_route, no bias) at those ids, renormalized, scaled, as bf16. An
 * input id outside the table or a table entry outside [0, E) gives id -1
 * and a NaN weight.
 */
int qmoe_moe_route_hash(const void* logits, int logits_f32, int64_t T, int E, int topk, int scoring,
                        const int32_t* hash_table, int64_t table_rows, const void* input_ids, int ids_i64,
                        int renormalize, float routed_scaling_factor, uint16_t* topk_weights, int32_t* topk_ids,
                        qmoe_stream_t stream);

/*
 * Token permutation by expert, replaces `layers/core/fused_moe_gmm.py:288-408`
 * (prepare_routed_gmm_inputs, non-EP): stable order by (expert, flat route
 * index t*k + slot); invalid routes (id < 0, or weight == 0 with
 * skip_padded) sort last. Outputs (int32):
 *   sorted_idx [T*k]  flat route index of each sorted row
 *   revert     [T*k]  sorted position of each flat route (inverse permutation)
 *   token_sorted [T*k] token of each sorted row (sorted_idx / k)
 *   group_offs [E+1]  row offsets per expert (group_sizes = diff)
 *   active     [min(E, T*k)] ids of experts with rows, ascending; num_active [1]
 *   sorted_weight [T*k] bf16 routing weight of each sorted row
 * One workgroup; histogram + exclusive scan + stable scatter in LDS.
 */
int qmoe_moe_dispatch(const int32_t* topk_ids, const uint16_t* topk_weights, int64_t T, int topk,
                      int E, int skip_padded, int32_t* sorted_idx, int32_t* revert,
                      int32_t* token_sorted, int32_t* group_offs, int32_t* active,
                      int32_t* num_active, uint16_t* sorted_weight, qmoe_stream_t stream);

/*
 * Routing and dispatch of a decode step in one launch (1 <= T <= 16 tokens,
 * T * topk <= 64 routes, E <= 512): the outputs of qmoe_moe_route (bf16
 * weights) followed by those of qmoe_moe_dispatch on its routes, written by
 * one workgroup. Replaces `layers/adapter/moe_routing.py:232-323`
 * (select_experts) followed by `layers/core/fused_moe_gmm.py:288-408`
 * (prepare_routed_gmm_inputs), which the reference runs back to back in
 * its MoE entry (`layers/adapter/quantization/fp8.py:1108-1222`). Returns
 * QMOE_ERR_ARG outside those bounds (the caller then makes the two calls).
 */
int qmoe_moe_route_dispatch(const void* logits, int logits_f32, int64_t T, int E, int topk, int scoring,
                            const float* bias, int renormalize, float routed_scaling_factor, int num_group,
                            int topk_group, uint16_t* topk_weights, int32_t* topk_ids, int skip_padded,
                            int32_t* sorted_idx, int32_t* revert, int32_t* token_sorted,
                            int32_t* group_offs, int32_t* active, int32_t* num_active,
                            uint16_t* sorted_weight, qmoe_stream_t stream);

/*
 * Weighted unpermute, replaces `layers/core/fused_moe_gmm.py:572-577`:
 * out[t] = bf16( sum over valid slots j of rows[t*k + j] ), where `rows`
 * holds the already weighted down-projection rows in flat route order
 * (written by qmoe_gemm with row_weight and y_rows = sorted_idx). A slot is
 * valid under the dispatch rule: 0 <= id < E (and weight != 0 with
 * skip_padded); the rows of other slots were never written and are skipped.
 */
int qmoe_moe_combine(const uint16_t* rows, const int32_t* topk_ids, const uint16_t* topk_weights,
                     int64_t T, int topk, int E, int64_t H, int skip_padded, uint16_t* out, int64_t ldo,
                     qmoe_stream_t stream);

/*
 * Fused decode MoE layer: the shared expert plus the routed experts of a
 * decode step, one call. Replaces the kernel call of
 * `layers/adapter/fused_moe_decode.py:249-339` (`_build_op` -> `_layer`),
 * i.e. `kernels/experimental/fused_moe_decode/fused_moe_decode_kernel.py:
 * 552-740` (`fused_moe_decode`) on one rank: n_ranks = 1 (the all-reduce is
 * the identity), expert_start = None, scatter_rows = False; the caller's
 * router supplies topk_ids / topk_weights.
 *
 * Numerics (all float32, output bf16): hidden states quantized to e4m3 per
 * (row, 512 columns) as scale = max|x| / 448, codes e4m3(x * (1 / scale));
 * each block's code dot times its row scale, summed, times the per-channel
 * w1 scale; mid = silu(gate) * up * coeff, coeff = bf16(route weight) *
 * routed_scale summed over the token's routes to that expert, or for the
 * shared expert sigmoid(x . shared_gate) (1 when shared_gate is NULL);
 * mid quantized per (row, 512 columns) the same way; second dot per block
 * times its row scale, summed, times the per-channel w2 scale; the shared
 * expert and the active routed experts added into one float32 sum per
 * token.
 *
 * weight_blocks = 128 (this build's variant, no reference counterpart):
 * 128x128 weight tiles kept as checkpointed, activations quantized per
 * (row, 128 columns), each block's dot times the activation block scale
 * times the tile scale.
 */
typedef struct qmoe_moe_decode_desc {
  const void* x;           /* bf16 [T][H] hidden states */
  int64_t T;               /* tokens, 1..64 */
  int64_t H;               /* hidden size, a multiple of 512 */
  int64_t I;               /* routed intermediate size, a multiple of 128 */
  int64_t I_shared;        /* shared intermediate size, a multiple of 128, <= I */
  int E;                   /* routed experts, 1..512 */
  int topk;                /* routes per token, 1..64 */
  const int32_t* topk_ids; /* [T][topk]; ids outside [0, E) select nothing */
  const void* topk_weights;/* [T][topk] bf16 (weights_f32 = 0) or f32 */
  int weights_f32;
  float routed_scale;      /* multiplies the routed experts only */
  int weight_blocks;       /* 0: per-channel scales; 128: 128x128 tile scales */
  const void* w1;          /* e4m3 [E][2I][H]: gate rows then up rows */
  const void* w2;          /* e4m3 [E][H][I] */
  const float* w1_scale;   /* [E][2I] | [E][2I/128][H/128] */
  const float* w2_scale;   /* [E][H]  | [E][H/128][I/128] */
  const void* shared_w1;   /* e4m3 [2 I_shared][H] */
  const void* shared_w2;   /* e4m3 [H][I_shared] */
  const float* shared_w1_scale; /* [2 I_shared] | [2 I_shared/128][H/128] */
  const float* shared_w2_scale; /* [H] | [H/128][I_shared/128] */
  const uint16_t* shared_gate;  /* bf16 [H], or NULL for an ungated shared expert */
  uint16_t* out;           /* bf16 [T][ldo] */
  int64_t ldo;
  /* Routing by the call (optional; no counterpart in the reference, whose
   * router runs before the decode kernel). With router_logits not NULL the
   * call first routes the tokens -- qmoe_moe_route's rule and results for
   * these arguments, bf16 weights -- and writes topk_ids / topk_weights,
   * which are then outputs (weights_f32 must be 0). Up to 8 tokens are
   * routed inside the first launch, more by a routing launch before it. */
  const void* router_logits;     /* [T][E] bf16 (logits_f32 = 0) or f32 */
  int logits_f32;
  int scoring;                   /* as qmoe_moe_route */
  const float* correction_bias;  /* [E] or NULL */
  int renormalize;
  float routed_scaling_factor;
  int num_group;
  int topk_group;
} qmoe_moe_decode_desc;

/* Workspace bytes of qmoe_moe_decode for this descriptor. */
int qmoe_moe_decode_workspace_size(const qmoe_moe_decode_desc* d, int64_t* bytes);

/* Four launches on `stream` (five when more than 8 tokens are routed by the
 * call); QMOE_ERR_ARG outside the envelope above, QMOE_ERR_WORKSPACE when
 * ws_bytes is below qmoe_moe_decode_workspace_size. */
int qmoe_moe_decode(const qmoe_moe_decode_desc* d, void* workspace, int64_t ws_bytes, qmoe_stream_t stream);

/*
 * Plain read of `bytes` (a multiple of 16, 16-byte aligned) at `src` by at
 * most `workgroups` 256-thread workgroups; `sink` receives at most one dword
 * per workgroup ([workgroups] uint32, normally untouched). No counterpart in
 * the reference: a measurement helper giving the HBM read floor (time vs
 * size, launch included) that the weight-streaming GEMMs are compared with.
 */
int qmoe_stream_read(const void* src, int64_t bytes, int32_t workgroups, void* sink, qmoe_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QMOE_H_ */
