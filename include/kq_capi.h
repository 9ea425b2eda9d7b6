/*
 * kq_capi.h -- C ABI of libgmlx_amd.so, the MI355X (gfx950) K-quant
 * batched-decode hot path: GGUF Q4_K / Q6_K / IQ2_XXS dequant-fused matmuls
 * (dense, grouped, MoE expert gather) and ragged GQA decode attention.
 *
 * Every entry point replaces one op of the un-vendored mlx-kquant package that
 * gmlx binds (pyproject.toml:26-34); the reference call site each replaces is
 * cited beside it.  Conventions:
 *   - all pointers are device pointers unless stated; the caller owns every
 *     buffer (outputs and workspace included); the library never allocates,
 *     frees or synchronizes;
 *   - weights are GGUF wire bytes, consumed unchanged: row n of a matrix
 *     starts at w + n * w_row_bytes and holds K/256 consecutive super-blocks;
 *   - every call takes a hipStream_t (pass the caller's current stream) and
 *     launches asynchronously;
 *   - return value: KQ_OK (0) or a negative kq_status; kq_strerror() names it.
 *     Validation happens on the host before any launch, so a rejected call
 *     launches nothing.
 */
#ifndef KQ_CAPI_H
#define KQ_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *kq_stream_t; /* == hipStream_t */

typedef enum {
    KQ_OK = 0,
    KQ_ERR_NULL_POINTER = -1,
    KQ_ERR_BAD_SHAPE = -2,
    KQ_ERR_BAD_ALIGN = -3,
    KQ_ERR_UNSUPPORTED_CODEC = -4,
    KQ_ERR_UNSUPPORTED_DTYPE = -5,
    KQ_ERR_WORKSPACE_TOO_SMALL = -6,
    KQ_ERR_LAUNCH_FAILED = -7,
    KQ_ERR_TOO_MANY_PROBLEMS = -8,
    KQ_ERR_BAD_ARGUMENT = -9,
    KQ_ERR_IO = -10,         /* a file could not be opened or mapped (kq_gguf.h) */
    KQ_ERR_BAD_FORMAT = -11  /* a malformed GGUF header (kq_gguf.h) */
} kq_status;

/* Codec ids are the GGML type ids (gguf GGMLQuantizationType). */
enum { KQ_CODEC_Q4_K = 12, KQ_CODEC_Q6_K = 14, KQ_CODEC_IQ2_XXS = 16 };
/* Element types of activations / outputs. */
enum { KQ_DTYPE_F32 = 0, KQ_DTYPE_F16 = 1, KQ_DTYPE_BF16 = 2 };
/* Op ids for kq_supports. */
enum {
    KQ_OP_DEQUANTIZE = 0,
    KQ_OP_QUANTIZE = 1,
    KQ_OP_MATMUL = 2,
    KQ_OP_GATHER = 3,
    KQ_OP_MOE_GLU = 4,
    KQ_OP_SDPA = 5
};

/* ---- identity and capability probes ---------------------------------- */
/* Capability probes replace kq.codecs() / kq.codec_has_matmul(c) /
 * kq.codec_has_moe_glu(c) (gmlx/modules.py:179-181, gmlx/loader.py:1443-1456). */
const char *kq_version(void);
const char *kq_strerror(int code);
/* Bytes per 256-value super-block of a codec (144 / 210 / 66), else 0. */
int kq_codec_block_bytes(int codec);
/* 1 when `op` supports `codec` (ignored for KQ_OP_SDPA) with activation
 * `dtype`, else 0. */
int kq_supports(int op, int codec, int dtype);
/* Host copy of the IQ2_XXS grid the kernels use (256 x u64, byte j = value j). */
const uint64_t *kq_iq2xxs_grid_host(void);

/* ---- dequantize / quantize ------------------------------------------- */
/* kq.dequantize(w, scales, codec, dtype) (gmlx/modules.py:1461,
 * gmlx/dsv32_patches.py:229): n_blocks super-blocks at `wire` (contiguous)
 * -> n_blocks*256 values of out_dtype.  fp32 output is bit-exact to the GGML
 * dequantize_row_* definition; f16/bf16 outputs are that value rounded to
 * nearest even. */
int kq_dequantize(const void *wire, int64_t n_blocks, int codec, void *out, int out_dtype,
                  kq_stream_t stream);

/* kq.quantize(w, codec) (tests/test_dequant_unattachable.py:36,
 * gmlx/mtp_load.py:290): fp32 w [n_rows, K] (row stride w_row_stride
 * elements), K % 256 == 0 -> wire [n_rows, K/256*block_bytes].  Q4_K / Q6_K
 * follow llama.cpp's reference quantizers; IQ2_XXS uses an exhaustive-grid
 * search.  Deterministic. */
int kq_quantize(const float *w, int64_t n_rows, int64_t K, int64_t w_row_stride, int codec,
                void *wire, kq_stream_t stream);

/* ---- dense quantized matmul ------------------------------------------ */
/* One problem y[M, N] = x[M, K] . dequant(W[N, K])^T, fp32 accumulation. */
typedef struct {
    const void *w;       /* wire bytes */
    int64_t w_row_bytes; /* byte stride between weight rows (>= K/256*bpb) */
    const void *x;       /* activations [M, K] of x_dtype */
    int64_t x_row_stride;/* elements, K <= stride <= 2^22 */
    void *y;             /* output [M, N] of y_dtype */
    int64_t y_row_stride;/* elements */
    int32_t M, N, K;
    int32_t codec;
} kq_matmul_problem;

/* Every non-empty workspace of kq_quantized_matmul_grouped and of the
 * gathers below begins with KQ_MATMUL_COUNTER_BYTES of arrival counters:
 * zero them once when the buffer is allocated (any fill); each call leaves
 * them zero, and nothing else may write them (do not hand such a workspace
 * to the attention entry points).  Calls sharing a workspace must be
 * ordered (same stream). */
#define KQ_MATMUL_COUNTER_BYTES ((size_t)16 << 10)

/* Workspace bytes kq_quantized_matmul_grouped needs for these problems and
 * activation dtype, 0 when it needs none: the counter region above, then
 *  - for bf16 / fp32 activations an fp16 copy of each problem's rows
 *    (problems sharing x share one) and one int32 exponent per row.  Every
 *    kernel computes with fp16 operands: a bf16 / fp32 row enters as
 *    fp16(x * 2^-e) with e chosen per row so its largest magnitude lands in
 *    [2^14, 2^15), and the fp32 results are scaled back by 2^e before
 *    rounding to y_dtype -- no overflow past 65504, no flush below 2^-14,
 *    bf16 values exact;
 *  - fp32 partial tiles of K slices for the launches that cut K: groups of
 *    at most 16 rows whose K runs past 16 super-blocks (the down
 *    projections: slices of 8 super-blocks up to 8 rows, 12 past 8) and
 *    Q4_K + Q6_K groups of at most 16 rows (q|k|v: two slices); 17..64-row
 *    groups that the mid-batch streaming kernel takes in slices (the down
 *    projection, q|k|v: 2 or 4 KB per 16-row tile and slice).  The last
 *    slice of each 16-row tile to finish sums the slices in slice order
 *    (results stay independent of scheduling).  With fp16 activations a
 *    workspace smaller than this (none included) takes the unsplit kernels
 *    instead. */
size_t kq_matmul_workspace_bytes(const kq_matmul_problem *problems, int n_problems, int x_dtype);

/* kq.quantized_matmul(x, w, scales, codec, transpose=True) -- the
 * KQuantLinear forward (gmlx/modules.py:1535-1539; direct calls at
 * gmlx/occupancy_fuse.py:162-165, 224-227, 290-293, 312-315).  Up to
 * KQ_MAX_GROUP independent problems (any codec mix, shared x_dtype/y_dtype)
 * run in one call: the row-concatenated q|k|v and gate|up wires of
 * gmlx/occupancy_fuse.py:141-344 become one call without concatenating
 * bytes.  The call is one launch (problems sharing x with M <= 16 whose
 * codecs mix beyond Q4_K with Q6_K may take one launch per codec).
 * x_dtype: f16, bf16 or f32 (bf16 /
 * f32 need the workspace above; one extra launch prepares the rows).
 * y_dtype: f16, bf16 or f32.  Results do not depend on scheduling: repeated
 * calls on the same inputs are bitwise identical. */
#define KQ_MAX_GROUP 8
int kq_quantized_matmul_grouped(const kq_matmul_problem *problems, int n_problems,
                                int x_dtype, int y_dtype, void *workspace,
                                size_t workspace_bytes, kq_stream_t stream);

/* ---- Fused dense MLP ----------------------------------------------------- */
/* gmlx's _FusedMLP forward (gmlx/occupancy_fuse.py:270-316): the grouped
 * gate|up call kq.quantized_matmul(x, w_gate|w_up), its SwiGLU
 * h = act(x . Wg^T) * (x . Wu^T), then down_proj(h) = h . Wd^T -- in one
 * launch: the down projection's weight stream starts while gate|up is
 * finishing, and h never leaves the device's caches as a separate
 * activation pass.  x [M, K] fp16, gate / up [I, K] wire rows of gu_codec,
 * down [N, I] wire rows of down_codec, y [M, N] of y_dtype.  h is computed in
 * fp32 and held as fp16 (the activation dtype the reference's swiglu feeds
 * down_proj).  act: KQ_ACT_SILU or KQ_ACT_GELU.
 * Served: fp16 x, M <= 8, Q4_K gate / up with K of 2048 or 4096, Q6_K or
 * Q4_K down with I a multiple of 2048 up to 16384.  Other shapes and dtypes
 * (bf16 / f32 activations keep h in their own dtype) and a workspace
 * below kq_fused_mlp_workspace_bytes, 256-byte aligned) return
 * KQ_ERR_BAD_SHAPE / KQ_ERR_WORKSPACE_TOO_SMALL before any launch; callers
 * then run the three steps as separate calls.  The workspace starts with
 * the KQ_MATMUL_COUNTER_BYTES counter region (zeroed once, left zero by
 * every call); the uint32 at byte KQ_FUSED_MLP_STATUS_OFFSET is set to 1 if
 * a wait for h gave up (the launch then did not complete normally: only
 * possible when the GPU cannot hold one workgroup per CU of this launch at
 * once), and is never cleared by the library.  Results do not depend on
 * scheduling. */
#define KQ_FUSED_MLP_STATUS_OFFSET (KQ_MATMUL_COUNTER_BYTES - 64)
size_t kq_fused_mlp_workspace_bytes(int32_t M, int32_t K, int32_t I, int32_t N, int x_dtype);
int kq_fused_mlp(const void *x, int x_dtype, int64_t x_row_stride, int32_t M, int32_t K, const void *w_gate,
                 const void *w_up, int64_t gu_row_bytes, int gu_codec, int32_t I, const void *w_down,
                 int64_t down_row_bytes, int down_codec, int32_t N, int act, void *y, int y_dtype,
                 int64_t y_row_stride, void *workspace, size_t workspace_bytes, kq_stream_t stream);

/* ---- MoE expert gather ------------------------------------------------- */
/* Device-side routing of (token, slot) pairs to experts.  idx [n_pairs]
 * int32 expert ids (row-major [T, k]).  Writes:
 *   seg_info  int32 [2 + 2*n_experts]: [0] = number of non-empty experts S,
 *             then seg_expert[n_experts], seg_start[n_experts + 1];
 *   pair_order int32 [2 * n_pairs]: pair ids grouped by expert (ascending
 *             expert, ascending pair id inside an expert) -- the stable sort
 *             gmlx's SwitchGLU applies at indices.size >= 64
 *             (gmlx/modules.py:1308-1310) -- then each pair's expert id, or
 *             -1 for an id out of range.
 * Expert ids outside [0, n_experts) are rejected on device: they are routed
 * to no segment and their outputs are written as zeros. */
int kq_moe_route(const int32_t *idx, int32_t n_pairs, int32_t n_experts, int32_t *seg_info,
                 int32_t *pair_order, kq_stream_t stream);

/* KQuantSwitchLinear / kq.gather_qmm (gmlx/modules.py:1549-1552,
 * tests/test_native_fp.py:420-428) and kq.gather_qmv_kq (gmlx/modules.py:595-597):
 * for every pair p = t*k + s with expert e = idx[p]:
 *   y[p, :] = x_row(p) . dequant(W[e])^T
 * x_row(p) = x[p / x_pair_div]: x_pair_div = top_k for gather_qmm (one x row
 * per token), 1 for gather_qmv (one h row per pair).  W: [n_experts, N, K]
 * wire with expert stride w_expert_bytes.  seg_info / pair_order come from
 * kq_moe_route.  y [n_pairs, N] of y_dtype (f32/f16/bf16). */
int kq_gather_qmm(const void *x, int x_dtype, int64_t x_row_stride, int32_t x_pair_div,
                  const void *w, int64_t w_expert_bytes, int64_t w_row_bytes, int32_t N,
                  int32_t K, int codec, const int32_t *seg_info, const int32_t *pair_order,
                  int32_t n_pairs, int32_t n_experts, void *y, int y_dtype,
                  int64_t y_row_stride, void *workspace, size_t workspace_bytes,
                  kq_stream_t stream);

/* kq.moe_glu_gather_kq(x, gate_w, up_w, codec, idx, act) (gmlx/modules.py:557-588):
 * h[p, :] = act(x_row(p) . Wg[e]^T) * (x_row(p) . Wu[e]^T) in fp32, act 0 =
 * silu, 1 = gelu (tanh approximation).  h [n_pairs, N] fp32. */
int kq_moe_glu_gather(const void *x, int x_dtype, int64_t x_row_stride, int32_t x_pair_div,
                      const void *w_gate, const void *w_up, int64_t w_expert_bytes,
                      int64_t w_row_bytes, int32_t N, int32_t K, int codec, int act,
                      const int32_t *seg_info, const int32_t *pair_order, int32_t n_pairs,
                      int32_t n_experts, float *h, void *workspace, size_t workspace_bytes,
                      kq_stream_t stream);

/* GLU activations of the fused gathers (the act= strings of
 * gmlx/modules.py:263-291, 557-566). */
enum {
    KQ_ACT_SILU = 0,        /* silu(g) * u */
    KQ_ACT_GELU = 1,        /* gelu_tanh(g) * u */
    KQ_ACT_SILU_LIMIT = 2,  /* silu(min(g, limit)) * clip(u, -limit, limit)
                               (gmlx/deepseek_v4_model.py:740-744) */
    KQ_ACT_SWIGLU_CLAMP = 3 /* g' = min(g + gate_bias, limit),
                               u' = clip(u + up_bias, -limit, limit):
                               (u' + 1) * g' * sigmoid(alpha * g')
                               (gmlx/minimax_m3_model.py:134-138) */
};

/* Epilogue of kq_moe_gather_rows, all in fp32.  Fused GLU (w1 != NULL): act
 * with limit / alpha, bias0 / bias1 the gate / up biases of swiglu_clamp.
 * Plain gather (w1 == NULL): bias0 is added to the output (the bias= of
 * kq.gather_qmv_kq, gmlx/modules.py:595-597).  Biases are fp32 rows of N
 * values per expert, bias_expert_stride elements apart; NULL for none. */
typedef struct {
    int32_t act;
    float limit, alpha;
    const float *bias0, *bias1;
    int64_t bias_expert_stride;
} kq_gather_epilogue;

/* The general form of the two gathers above, for pair rows laid out with a
 * spare row every few pairs: kq.moe_glu_gather_shexp_kq(x, gate_w, up_w,
 * shexp_gate_w, shexp_up_w, codec, idx, act=) and kq.gather_qmv_mix_kq(h,
 * down_w, shexp_down_w, codec, idx, scores) (gmlx/modules.py:571-584,
 * 777-787) keep the shared expert in slot k of [t, k + 1, N] blocks.
 * Pair p reads x row p / x_pair_div + p / x_skip and writes y row
 * p + p / y_skip (a skip of 0 adds nothing).  w1 == NULL: plain gather;
 * w1 != NULL: fused GLU, computed in fp32.  Either way y is of y_dtype (f32,
 * f16 or bf16; an f16 GLU output is what the down gather reads without
 * preparing its rows).  ep == NULL means silu and no biases.  The shared
 * expert itself is a one-expert gather (n_experts 1, every pair routed to
 * it). */
int kq_moe_gather_rows(const void *x, int x_dtype, int64_t x_row_stride, int32_t x_pair_div,
                       int32_t x_skip, const void *w0, const void *w1, int64_t w_expert_bytes,
                       int64_t w_row_bytes, int32_t N, int32_t K, int codec,
                       const kq_gather_epilogue *ep, const int32_t *seg_info,
                       const int32_t *pair_order, int32_t n_pairs, int32_t n_experts, void *y,
                       int y_dtype, int64_t y_row_stride, int32_t y_skip, void *workspace,
                       size_t workspace_bytes, kq_stream_t stream);

/* Workspace of the three gathers above: 0 for fp16 activations; for bf16 /
 * fp32 ones the counter region (KQ_MATMUL_COUNTER_BYTES, zeroed once, so one
 * buffer may serve matmuls and gathers), then an fp16 copy of the rows the
 * pairs read (row p / x_pair_div + p / x_skip) with one int32 exponent per
 * row, prepared as for kq_quantized_matmul_grouped (x_skip 0 for
 * kq_gather_qmm / kq_moe_glu_gather).  Results are scaled back in fp32
 * before the GLU and biases. */
size_t kq_gather_workspace_bytes(int32_t n_pairs, int32_t x_pair_div, int32_t x_skip, int32_t K,
                                 int x_dtype);

/* The routing mix of kq.gather_qmv_mix_ns_kq (gmlx/modules.py:591-593):
 * y[t, :] = sum_s scores[t, s] * y_pairs[t*k + s, :], fp32, slots summed in
 * order s = 0..k-1.  y_pairs fp32 [T*k, N]; scores fp32 [T, k]; y of y_dtype. */
int kq_moe_mix(const float *y_pairs, const float *scores, int32_t T, int32_t top_k, int32_t N,
               void *y, int y_dtype, kq_stream_t stream);

/* Scoring functions of the router (gmlx/deepseek_v4_model.py:690-697). */
enum { KQ_SCORE_SOFTMAX = 0, KQ_SCORE_SIGMOID = 1, KQ_SCORE_SQRTSOFTPLUS = 2 };

/* Keywords of kq.moe_router_topk(logits, k, norm_topk_prob, shared_gate=,
 * per_expert_scale=, bias=, scoring=, scale=). */
typedef struct {
    int32_t norm_topk_prob;   /* divide the k picked scores by their sum (+1e-20) */
    int32_t shared_gate;      /* logits carry one more column, the shared expert's gate */
    int32_t scoring;          /* KQ_SCORE_* */
    float scale;              /* routed scaling factor applied to every pick */
    const void *bias;         /* [E] selection-only bias (e_score_correction_bias), or NULL */
    int32_t bias_dtype;
    const void *per_expert_scale; /* [E] multiplies pick e's weight, or NULL */
    int32_t per_expert_scale_dtype;
} kq_router_options;

/* kq.moe_router_topk (gmlx/modules.py:750-752, 1043-1046, 1208-1211;
 * gmlx/deepseek_v4_model.py:1179-1187), in fp32, per token:
 *   score_e  = softmax over the E routed logits, sigmoid(logit), or
 *              sqrt(softplus(logit));
 *   picks    = the k experts with the largest score_e + bias[e] (descending,
 *              ties to the lower expert id), weighted by their score_e;
 *   weights  = picks / (sum of picks + 1e-20) when norm_topk_prob, then
 *              times per_expert_scale[e] and scale;
 *   shared_gate: logits [T, E + 1] whose last column is the shared expert's
 *              gate logit (the router-cat rows of gmlx/modules.py:300-312);
 *              sigmoid(it) is appended as weight k (the stock form
 *              gmlx/modules.py:754-763).
 * logits rows logits_row_stride elements apart (>= E + shared_gate); inds
 * int32 [T, k]; scores fp32 [T, k + shared_gate].  E <= 1024, k <= 32,
 * k <= E.  opts == NULL: softmax, renormalised, no shared gate, scale 1. */
int kq_moe_router_topk(const void *logits, int logits_dtype, int64_t logits_row_stride, int32_t T,
                       int32_t E, int32_t k, const kq_router_options *opts, int32_t *inds,
                       float *scores, kq_stream_t stream);

/* ---- ragged GQA decode attention ----------------------------------------- */
/* Workspace of kq_sdpa_decode_ragged: fp32 split partials (O, m, l) for
 * B * Hkv * ceil(max_len / split) splits; no zero-fill needed.  Calls that
 * share a workspace must be ordered (same stream).
 *
 * ragged_decode_attention(q, k, v, pads, scale) (gmlx/qwen35_attn.py:395-493)
 * and kq.sdpa_decode_gqa(q, k, v, scale, starts=) (gmlx/gemma4_batched_sdpa.py:
 * 210-226), one query token per row:
 *   out[b, hq, :] = softmax(scale * q[b, hq] . K_b,h^T) . V_b,h,  h = hq / (Hq/Hkv)
 * over the row's visible keys.  Row b's keys for kv head h are the row_len[b]
 * tokens starting at element kv_off[b] + h * head_stride[b] of k (and v), each
 * token D contiguous elements.  Both the packed per-row slab layout
 * ([Hkv, len_b, D] at a row offset) and the reference's padded
 * [B, Hkv, L, D] + per-row start layout are expressible.
 * q [B, Hq, D] (contiguous), out [B, Hq, D]; q/k/v/out share dtype (f16 or
 * bf16).  D in {64, 96, 128, 256, 512} (512 walks 16-token tiles); Hq % Hkv
 * == 0; Hq/Hkv <= 16.
 * max_len >= every row_len[b] (sizes the split table and workspace). */
size_t kq_sdpa_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t max_len);
int kq_sdpa_decode_ragged(const void *q, const void *k, const void *v, const int64_t *kv_off,
                          const int64_t *head_stride, const int32_t *row_len, int32_t B,
                          int32_t Hq, int32_t Hkv, int32_t D, int32_t max_len, float scale,
                          int dtype, void *out, void *workspace, size_t workspace_bytes,
                          kq_stream_t stream);

/* 8-bit affine KV cache, group 64 (the quantized-KV form of
 * kq.sdpa_decode_gqa(q, kw, vw, scale, starts=, k_scales=, k_biases=,
 * v_scales=, v_biases=), gmlx/quantized_sdpa_fix.py:170-182, as mlx's
 * BatchQuantizedKVCache holds it: bits 8, group_size 64): k / v hold uint8
 * values (an mlx uint32 word packs four, lowest byte first), a token row is
 * D bytes; value = scale * q + bias with one 16-bit (q's dtype) scale and
 * bias per 64 values, at element index (byte offset) / 64 of k_scales /
 * k_biases (v_*).  kv_off and head_stride are in bytes and multiples of 64;
 * D in {64, 128, 256, 512}; k / v 8-byte aligned.  Same workspace as above. */
int kq_sdpa_decode_ragged_q8(const void *q, const void *k, const void *v, const void *k_scales,
                             const void *k_biases, const void *v_scales, const void *v_biases,
                             const int64_t *kv_off, const int64_t *head_stride,
                             const int32_t *row_len, int32_t B, int32_t Hq, int32_t Hkv,
                             int32_t D, int32_t max_len, float scale, int dtype, void *out,
                             void *workspace, size_t workspace_bytes, kq_stream_t stream);

/* kq.sdpa_decode_gqa(q, k, v, scale, starts=) on the reference's padded
 * cache layout (gmlx/gemma4_batched_sdpa.py:210-226, the ragged route of
 * gmlx/qwen35_attn.py:395-493 with pads as starts): k / v [B, Hkv, L, D]
 * with D contiguous elements per token, batch_stride / head_stride elements
 * apart (multiples of 8); row b attends keys [starts[b], L) (starts: device
 * int32 [B], read on the device and clamped to [0, L]; NULL means 0).  No
 * per-row tables and no host synchronisation: a decode loop passes the same
 * starts at every L.  Same outputs, dtypes, head dims and workspace
 * (kq_sdpa_workspace_bytes(B, Hq, Hkv, D, L)) as kq_sdpa_decode_ragged. */
int kq_sdpa_decode_gqa(const void *q, const void *k, const void *v, int64_t batch_stride,
                       int64_t head_stride, int32_t L, const int32_t *starts, int32_t B, int32_t Hq,
                       int32_t Hkv, int32_t D, float scale, int dtype, void *out, void *workspace,
                       size_t workspace_bytes, kq_stream_t stream);

/* kq_sdpa_decode_gqa with no workspace argument; it allocates nothing.  No
 * counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The split partials live in a device array the library
 * holds on each GPU it runs on (KQ_SDPA_NOALLOC_SCRATCH_BYTES, until the
 * process ends); calls needing more (kq_sdpa_workspace_bytes(B, Hq, Hkv, D,
 * L) above the limit) return KQ_ERR_WORKSPACE_TOO_SMALL and launch nothing.
 * Same outputs as kq_sdpa_decode_gqa (the same kernels and split plan).  All
 * calls on one GPU share the array: calls that overlap there (other streams
 * or threads) race; order them. */
#define KQ_SDPA_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int kq_sdpa_decode_gqa_noalloc(const void *q, const void *k, const void *v, int64_t batch_stride,
                               int64_t head_stride, int32_t L, const int32_t *starts, int32_t B, int32_t Hq,
                               int32_t Hkv, int32_t D, float scale, int dtype, void *out, kq_stream_t stream);

/* The 8-bit affine form of kq_sdpa_decode_gqa (k_scales=, k_biases=,
 * v_scales=, v_biases=, gmlx/quantized_sdpa_fix.py:76-93, 170-182): k / v
 * uint8 [B, Hkv, L, D] with byte strides (multiples of 64), kv_scales =
 * {k_scales, k_biases, v_scales, v_biases} laid out as
 * kq_sdpa_decode_ragged_q8 describes (index = byte offset / 64). */
int kq_sdpa_decode_gqa_q8(const void *q, const void *k, const void *v, const void *const *kv_scales,
                          int64_t batch_stride, int64_t head_stride, int32_t L, const int32_t *starts,
                          int32_t B, int32_t Hq, int32_t Hkv, int32_t D, float scale, int dtype,
                          void *out, void *workspace, size_t workspace_bytes, kq_stream_t stream);

/* ---- cascade (shared-prefix) decode attention ---------------------------- */
/* kq.sdpa_decode_gqa_cascade(q, k_shared, v_shared, k_priv, v_priv, scale,
 * starts=) as called at gmlx/cascade_sdpa.py:238-248 (claim gates :171-215):
 * B sequences share a prefix of P tokens held once; each has a private slab
 * of S tokens after it.  Query token i < qL of sequence b attends
 *   the whole prefix k_shared/v_shared [Hkv, P, D] (element h * shared_head_stride
 *   + t * D), then private keys [starts[b], S - qL + i] of k_priv/v_priv
 *   (element b * priv_batch_stride + h * priv_head_stride + t * D):
 * left padding plus the end-aligned causal mask of the query block.
 * starts == NULL means 0 for every sequence; starts are clamped to [0, S].
 * q, out [B, Hq, qL, D] contiguous; all tensors share dtype (f16 or bf16).
 * qL in 1..64, D in {64, 96, 128, 256, 512}, Hq % Hkv == 0, Hq/Hkv <= 16.
 * Each prefix tile is loaded once per 16 / (Hq/Hkv) query rows (the rows'
 * heads share the MFMA's 16 columns), so the prefix costs P, not B * P,
 * bytes per head in the common case (B * qL * Hq / Hkv <= 16). */
size_t kq_sdpa_cascade_workspace_bytes(int32_t B, int32_t qL, int32_t Hq, int32_t Hkv, int32_t D,
                                       int32_t P, int32_t S);
int kq_sdpa_decode_gqa_cascade(const void *q, const void *k_shared, const void *v_shared,
                               int64_t shared_head_stride, int32_t P, const void *k_priv,
                               const void *v_priv, int64_t priv_batch_stride,
                               int64_t priv_head_stride, int32_t S, const int32_t *starts,
                               int32_t B, int32_t qL, int32_t Hq, int32_t Hkv, int32_t D,
                               float scale, int dtype, void *out, void *workspace,
                               size_t workspace_bytes, kq_stream_t stream);

/* The 8-bit affine KV form of the cascade (gmlx/cascade_sdpa.py:216-236:
 * bits 8, group 64, wire plus scales / biases for the shared prefix and the
 * private slab), as kq_sdpa_decode_ragged_q8 describes the format:
 * shared_scales / priv_scales = {k_scales, k_biases, v_scales, v_biases} of
 * the prefix and of the slabs; strides in bytes, multiples of 64. */
int kq_sdpa_decode_gqa_cascade_q8(const void *q, const void *k_shared, const void *v_shared,
                                  const void *const *shared_scales, int64_t shared_head_stride,
                                  int32_t P, const void *k_priv, const void *v_priv,
                                  const void *const *priv_scales, int64_t priv_batch_stride,
                                  int64_t priv_head_stride, int32_t S, const int32_t *starts,
                                  int32_t B, int32_t qL, int32_t Hq, int32_t Hkv, int32_t D,
                                  float scale, int dtype, void *out, void *workspace,
                                  size_t workspace_bytes, kq_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* KQ_CAPI_H */
