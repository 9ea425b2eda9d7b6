// Dequant-fused quantized matmul: dense grouped problems (KQuantLinear /
// kq.quantized_matmul) and the MoE expert gather family (kq.gather_qmm,
// kq.moe_glu_gather_kq, kq.gather_qmv_kq, mix, router top-k).
//
// Dense work decomposition: one workgroup per (problem, 16-row weight tile,
// 64-row batch chunk).  The WV waves of a workgroup split the tile's K range
// (wave w takes super-blocks w, w+WV, ...), each wave keeps its own MFMA
// accumulators, and the workgroup sums them through LDS in wave order.  The
// reduction never leaves the workgroup, so there are no global partials,
// counters or device-scope fences, and the result does not depend on
// scheduling.  Small batches (one 16-row m-tile) use 16 waves per tile: each
// wave then holds one or a few blocks and little register state, and the many
// resident waves hide the memory latency behind the dequant work; wider batch
// chunks use 4 waves with more m-tiles each.
#include <stdlib.h>

#include "kq_mma.h"

// kq_mv.hip: LDS-staged small-batch launch (problems validated, all live,
// one codec, sharing x / M <= 16, x rows fitting in LDS).
bool kq_mv_eligible(const kq_matmul_problem *ps, int n, int x_dtype, int y_dtype);
int kq_mv_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, hipStream_t s);
// kq_stream.hip: weight-streaming launch for M <= 8 (problems validated, all
// live, fp16 x shared, one codec or Q4_K with Q6_K, K as its slab plan allows).
int kq_stream_split_want(const kq_matmul_problem *ps, int n);
size_t kq_stream_part_bytes(const kq_matmul_problem *ps, int n, int split);
bool kq_stream_eligible(const kq_matmul_problem *ps, int n, int split);
int kq_stream_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, int split,
                     uint32_t *ctr, float *part, hipStream_t s);
// kq_stream.hip: the one-shot kernel (a workgroup's tiles and x in LDS at once).
bool kq_shot_eligible(const kq_matmul_problem *ps, int n);
int kq_shot_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, hipStream_t s);
bool kq_sgather_eligible(int codec, bool glu, int32_t N, int32_t K, int64_t w_row_bytes, int32_t n_experts);
int kq_sgather_launch(const void *x, const int32_t *x_exp, int64_t x_row_stride, int32_t x_pair_div, int32_t x_skip,
                      const void *w0, const void *w1, int64_t w_expert_bytes, int64_t w_row_bytes, int32_t N,
                      int32_t K, int codec, int act, float limit, float alpha, const float *b0, const float *b1,
                      int64_t b_stride, const int32_t *seg_info, const int32_t *pair_order, int32_t n_pairs,
                      int32_t n_experts, void *y, int y_dtype, int64_t y_row_stride, int32_t y_skip, hipStream_t s);
// kq_mm.hip: batches of 17..64 rows (problems validated, all live, Q4_K /
// Q6_K, sharing x / M / K).
bool kq_mms_eligible(const kq_matmul_problem *ps, int n, bool room);
size_t kq_mms_part_bytes(const kq_matmul_problem *ps, int n);
int kq_mms_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, uint32_t *ctr,
                  float *part, hipStream_t s);
bool kq_mm_eligible(const kq_matmul_problem *ps, int n, int x_dtype);
// kq_stream.hip: the fused dense MLP (one launch).
bool kq_mlp_eligible(int32_t M, int32_t K, int32_t I, int32_t N, int gu_codec, int d_codec, int64_t gu_row,
                     int64_t d_row);
size_t kq_mlp_work_bytes(int32_t I, int32_t N);
int kq_mlp_launch(const void *x, const int32_t *x_exp, int64_t x_row_stride, int32_t M, int32_t K,
                  const void *w_gate, const void *w_up, int64_t gu_row, int32_t I, const void *w_down,
                  int64_t d_row, int d_codec, int32_t N, int act, void *y, int y_dtype, int64_t y_row_stride,
                  void *workspace, hipStream_t s);
int kq_mm_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, hipStream_t s);
int device_cus();

namespace {

using namespace kqmma;

constexpr int kMaxChunk = 64;  // batch rows per grid.y chunk (4 m-tiles)

int env_int(const char *name, int dflt) {
    const char *s = getenv(name);
    return (s && *s) ? atoi(s) : dflt;
}


struct DenseProblem {
    const uint8_t *w;
    const char *x;
    const int32_t *x_exp;  // per-row exponents of prepared activations (results * 2^e), or null
    void *y;
    int64_t w_row_bytes, x_stride, y_stride;
    int32_t M, N, K, codec;
    int32_t n_tiles;
    int32_t unit_begin;   // first workgroup id of this problem
};

struct DenseArgs {
    DenseProblem p[KQ_MAX_GROUP];
    int32_t n_problems;
    int32_t y_dtype;
};

__device__ __forceinline__ void store_tile(void *y, int y_dtype, int64_t y_stride, int m0, int M,
                                           int n, bool n_valid, const floatx4 &c, const int32_t *x_exp) {
    const int lane = kq_lane();
    if (!n_valid) return;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = m0 + 4 * (lane >> 4) + e;
        if (m < M) kq_store_out(y, y_dtype, (int64_t)m * y_stride + n, x_exp ? ldexpf(c[e], x_exp[m]) : c[e]);
    }
}

// Wave `wave` of the workgroup takes super-blocks wave, wave + WV, ... of
// NW column tiles (16 * NW output columns); the activation fragments of a
// super-block are loaded once for all NW tiles.
template <int CODEC, int MT, int XT, int WV, int NW>
__device__ __forceinline__ void dense_tile(const DenseProblem &p, int nt, int wave, floatx4 (&acc)[NW][MT],
                                           const Iq2Tables &tab) {
    const int lane = kq_lane();
    const int r = lane & 15;
    const int m0 = blockIdx.y * kMaxChunk;
    const int nb = p.K / KQ_QK;
    const uint8_t *wrow[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) wrow[i] = p.w + (int64_t)min((nt * NW + i) * 16 + r, p.N - 1) * p.w_row_bytes;
    const XRowsBuf<MT> xrow = x_rows_buf<MT, XT>(p.x, p.x_stride, p.M, p.K, m0, r);
#pragma unroll
    for (int i = 0; i < NW; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[i][mt] = floatx4{0, 0, 0, 0};
    tile_accumulate<CODEC, MT, XT, NW, XRowsBuf<MT>, (WV < 16)>(wrow, wave, WV, nb, xrow, acc, tab);
}

template <int MT, int XT, int WV, int NW>
__global__ __launch_bounds__(64 * WV) void kq_dense_grouped_kernel(DenseArgs a) {
    __shared__ floatx4 red[WV - 1][NW * MT][64];
    __shared__ Iq2Tables iq2_tab;
    const int unit = blockIdx.x;
    // Select the problem with static indices only: dynamic indexing of the
    // by-value argument array would copy it to scratch memory.
    DenseProblem p = a.p[0];
#pragma unroll
    for (int i = 1; i < KQ_MAX_GROUP; ++i)
        if (i < a.n_problems && unit >= a.p[i].unit_begin) p = a.p[i];
    const int nt = unit - p.unit_begin;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = kq_lane();
    const int m0 = blockIdx.y * kMaxChunk;
    if (m0 >= p.M) return;  // uniform over the workgroup
    floatx4 acc[NW][MT];
    switch (p.codec) {
    case KQ_CODEC_Q4_K: dense_tile<KQ_CODEC_Q4_K, MT, XT, WV, NW>(p, nt, wave, acc, iq2_tab); break;
    case KQ_CODEC_Q6_K: dense_tile<KQ_CODEC_Q6_K, MT, XT, WV, NW>(p, nt, wave, acc, iq2_tab); break;
    default:
        load_iq2_tables(iq2_tab);
        dense_tile<KQ_CODEC_IQ2_XXS, MT, XT, WV, NW>(p, nt, wave, acc, iq2_tab);
        break;
    }
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < NW; ++i)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) red[wave - 1][i * MT + mt][lane] = acc[i][mt];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < WV - 1; ++w)
#pragma unroll
        for (int i = 0; i < NW; ++i)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[i][mt] += red[w][i * MT + mt][lane];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int n = (nt * NW + i) * 16 + (lane & 15);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            store_tile(p.y, a.y_dtype, p.y_stride, m0 + 16 * mt, p.M, n, n < p.N, acc[i][mt], p.x_exp);
    }
}

// ---------------------------------------------------------------- MoE

struct GatherArgs {
    const char *x;
    const uint8_t *w0, *w1;   // expert stacks (w1: up for the fused GLU)
    void *y;                  // [n_pairs, N] (f32 for the GLU)
    const int32_t *seg_info;  // [0] = S, then seg_expert[E], seg_start[E+1]
    const int32_t *pair_order;
    int64_t x_stride, w_expert_bytes, w_row_bytes, y_stride;
    int32_t x_pair_div, N, K, n_pairs, n_experts, n_tiles, y_dtype, act;
    // row of pair p: x  p / x_pair_div + p / x_skip,  y  p + p / y_skip
    // (a skip of 0 adds nothing): one spare row per x_skip / y_skip pairs,
    // e.g. the shared expert's slot k of an [t, k + 1, N] block
    int32_t x_skip, y_skip;
    // epilogue: GLU clamp / slope, fp32 biases [expert][N] (b0: gate bias of
    // the GLU, or the output bias of a plain gather; b1: up bias), or null
    float limit, alpha;
    const float *b0, *b1;
    int64_t b_stride;
    const int32_t *x_exp;  // per-row exponents of prepared activations (results * 2^e), or null
};

__device__ __forceinline__ int64_t gather_x_row(const GatherArgs &a, int pair) {
    return pair / a.x_pair_div + (a.x_skip ? pair / a.x_skip : 0);
}
__device__ __forceinline__ int64_t gather_y_row(const GatherArgs &a, int pair) {
    return pair + (a.y_skip ? pair / a.y_skip : 0);
}

// Output of pair rows for weight row n of `expert`: acc[0] (gate, or the
// plain product) and acc[1] (up) in fp32: plain v = g (+ b0[n]); the GLU
// forms are kq_glu (kq_common.h).
template <int NW>
__device__ __forceinline__ float gather_epilogue(const GatherArgs &a, int expert, int n, float g, float u) {
    const int64_t bo = (int64_t)expert * a.b_stride + n;
    if constexpr (NW == 1) {
        return a.b0 ? g + a.b0[bo] : g;
    } else {
        const bool clamp = a.act == KQ_ACT_SWIGLU_CLAMP;
        return kq_glu(a.act, g, u, a.limit, a.alpha, clamp && a.b0 ? a.b0[bo] : 0.f, clamp && a.b1 ? a.b1[bo] : 0.f);
    }
}

// One workgroup of kGatherWaves waves per (expert segment, 16-row weight
// tile): the waves split the super-blocks (wave w takes w, w + kGatherWaves,
// ...) like the dense kernel, and wave 0 sums their tiles in wave order (so
// the result is deterministic) before the epilogue.  A segment longer than
// 16 * MT rows is walked in chunks.
constexpr int kGatherWaves = 4;

// Register budget (tighter budgets spill to scratch): four waves per SIMD
// (128 VGPRs) for one 16-row tile of one matrix with fp16/bf16 rows; three
// (168) up to two such tiles or fp32 rows; two (256) up to four tiles (and
// Q6_K pairs of fp32 rows); one (AGPRs too) beyond, and for four tiles of
// fp32 rows.  Q4_K tiles, which also carry the activations' sub-block sums
// for the minimum term, take the next budget up.
template <int CODEC, int MT, int NW, int XT>
constexpr int gather_waves_per_simd() {
    constexpr int t = MT * NW * (CODEC == KQ_CODEC_Q4_K ? 2 : 1);
    if (t == 1 && XT != 2) return 4;
    if (t <= 2 && !(CODEC == KQ_CODEC_Q6_K && XT == 2 && t == 2)) return 3;
    return (t <= 4 && !(XT == 2 && t == 4)) ? 2 : 1;
}

template <int CODEC, int MT, int XT, int NW>
__global__ __launch_bounds__(64 * kGatherWaves)
__attribute__((amdgpu_waves_per_eu(gather_waves_per_simd<CODEC, MT, NW, XT>()))) void kq_gather_kernel(GatherArgs a) {
    __shared__ floatx4 red[kGatherWaves - 1][NW][MT][64];
    __shared__ Iq2Tables iq2_tab;
    if constexpr (CODEC == KQ_CODEC_IQ2_XXS) load_iq2_tables(iq2_tab);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = kq_lane();
    const int r = lane & 15;
    const int slot = blockIdx.x / a.n_tiles;
    const int nt = blockIdx.x - slot * a.n_tiles;
    if (slot == 0 && wave == 0) {
        // pairs whose expert id is out of range (never routed) get zeros in
        // this tile's columns
        const int c = nt * 16 + (lane & 15);
        kq_for_unrouted(a.pair_order + a.n_pairs, a.n_pairs, [&](int p) {
            if (lane < 16 && c < a.N) kq_store_out(a.y, a.y_dtype, gather_y_row(a, p) * a.y_stride + c, 0.f);
        });
    }
    const int S = a.seg_info[0];
    if (slot >= S) return;  // uniform over the workgroup
    const int expert = a.seg_info[1 + slot];
    const int seg_begin = a.seg_info[1 + a.n_experts + slot];
    const int seg_end = a.seg_info[1 + a.n_experts + slot + 1];
    const int n = nt * 16 + r;
    const bool n_valid = n < a.N;
    const int nc = n_valid ? n : a.N - 1;
    const int nb = a.K / KQ_QK;
    const uint8_t *wrow[NW];
    wrow[0] = a.w0 + (int64_t)expert * a.w_expert_bytes + (int64_t)nc * a.w_row_bytes;
    if constexpr (NW == 2)
        wrow[1] = a.w1 + (int64_t)expert * a.w_expert_bytes + (int64_t)nc * a.w_row_bytes;
    for (int c0 = seg_begin; c0 < seg_end; c0 += 16 * MT) {
        XRowPtrs<MT> xrow;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int ri = min(c0 + 16 * mt + r, seg_end - 1);
            xrow.row[mt] = a.x + gather_x_row(a, a.pair_order[ri]) * a.x_stride * x_elem_bytes<XT>();
        }
        floatx4 acc[NW][MT];
#pragma unroll
        for (int i = 0; i < NW; ++i)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[i][mt] = floatx4{0, 0, 0, 0};
        // no prefetch stage: resident waves hide the latency
        tile_accumulate<CODEC, MT, XT, NW, XRowPtrs<MT>, false>(wrow, wave, kGatherWaves, nb, xrow, acc, iq2_tab);
        if (wave > 0) {
#pragma unroll
            for (int i = 0; i < NW; ++i)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) red[wave - 1][i][mt][lane] = acc[i][mt];
        }
        __syncthreads();
        if (wave == 0 && n_valid) {
#pragma unroll
            for (int w = 0; w < kGatherWaves - 1; ++w)
#pragma unroll
                for (int i = 0; i < NW; ++i)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[i][mt] += red[w][i][mt][lane];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int ri = c0 + 16 * mt + 4 * (lane >> 4) + e;
                    if (ri >= seg_end) continue;
                    const int pair = a.pair_order[ri];
                    const int ex = a.x_exp ? a.x_exp[gather_x_row(a, pair)] : 0;
                    const float v = gather_epilogue<NW>(a, expert, n, ldexpf(acc[0][mt][e], ex),
                                                        ldexpf(acc[NW - 1][mt][e], ex));
                    kq_store_out(a.y, a.y_dtype, gather_y_row(a, pair) * a.y_stride + n, v);
                }
            }
        }
        __syncthreads();  // red is reused by the next chunk
    }
}


// Activation rows of one segment staged in LDS as fp16 (converted the way the
// global loaders convert), row i at base + i * stride bytes.
struct XRowsLds {
    uint32_t base;  // LDS byte address of the lane's row
    template <int XT>
    __device__ __forceinline__ half8_t load(int, int elem) const {
        return __builtin_bit_cast(half8_t,
                                  *(const __attribute__((address_space(3))) u32x4 *)(uintptr_t)(base + (uint32_t)elem * 2));
    }
};

// Staged activation rows per workgroup: 32 KB, or 24 KB where the kernel runs
// five waves per SIMD (five workgroups per CU then fit the 160 KB of LDS with
// the IQ2_XXS tables; at K = 2048 that still stages segments of five rows).
template <int CODEC, int MT, int NW, int XT>
constexpr int gather_wave_waves_per_simd() {
    // single-tile fp16 forms (the per-pair down gathers): five waves in 96
    // VGPRs, with 20 (IQ2_XXS) and 52 (Q6_K) bytes per lane spilled outside
    // the block loop; measured 1.5 % (C4 down, Q6_K) and 3 % (C5, IQ2_XXS)
    // faster than four waves
    if (MT * NW * (CODEC == KQ_CODEC_Q4_K ? 2 : 1) == 1 && XT == 0) return 5;
    return gather_waves_per_simd<CODEC, MT, NW, XT>();
}
template <int CODEC, int MT, int NW, int XT>
constexpr int gather_lds_bytes() {
    return gather_wave_waves_per_simd<CODEC, MT, NW, XT>() == 5 ? 24 * 1024 : 32 * 1024;
}

// Short K: one wave per (segment slot, tile) unit, kGatherWaves units per
// workgroup (consecutive tiles of one expert), the whole K in the wave; no
// cross-wave reduction.  When the workgroup's units share one segment of at
// most 16 rows whose activations fit gather_lds_bytes, the rows are staged in
// LDS once for the four waves (their fragments are read from LDS instead of
// once per tile from L2); otherwise each wave loads them from memory.
template <int CODEC, int MT, int XT, int NW>
__global__ __launch_bounds__(64 * kGatherWaves)
__attribute__((amdgpu_waves_per_eu(gather_wave_waves_per_simd<CODEC, MT, NW, XT>()))) void kq_gather_wave_kernel(GatherArgs a) {
    __shared__ Iq2Tables iq2_tab;
    __shared__ __attribute__((aligned(16))) uint8_t xs_lds[MT == 1 ? gather_lds_bytes<CODEC, MT, NW, XT>() : 16];
    if constexpr (CODEC == KQ_CODEC_IQ2_XXS) load_iq2_tables(iq2_tab);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = kq_lane();
    const int r = lane & 15;
    const int unit = blockIdx.x * kGatherWaves + wave;
    const int slot = unit / a.n_tiles;
    const int nt = unit - slot * a.n_tiles;
    const int S = a.seg_info[0];
    const int nb = a.K / KQ_QK;
    // ---- staging decision, uniform over the workgroup
    bool staged = false;
    uint32_t xrow_bytes = 0;
    if constexpr (MT == 1) {
        const int u0 = blockIdx.x * kGatherWaves;
        const int s0 = u0 / a.n_tiles, s3 = (u0 + kGatherWaves - 1) / a.n_tiles;
        if (s0 == s3 && s0 < S) {
            const int rows = a.seg_info[1 + a.n_experts + s0 + 1] - a.seg_info[1 + a.n_experts + s0];
            xrow_bytes = (uint32_t)a.K * 2 + 16;  // padded: rows start on different banks
            staged = rows <= 16 && (uint32_t)rows * xrow_bytes <= (uint32_t)gather_lds_bytes<CODEC, MT, NW, XT>();
            if (staged) {
                const int begin = a.seg_info[1 + a.n_experts + s0];
                const int per_row = a.K / 8;  // 8 activations (16 bytes of fp16) per item
                for (int i = threadIdx.x; i < rows * per_row; i += 64 * kGatherWaves) {
                    const int row = i / per_row, c = i - row * per_row;
                    const char *src = a.x + (gather_x_row(a, a.pair_order[begin + row]) * a.x_stride +
                                             (int64_t)c * 8) * x_elem_bytes<XT>();
                    *(__attribute__((address_space(3))) half8_t *)(uintptr_t)(
                        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)xs_lds + row * xrow_bytes + c * 16) =
                        load_x8<XT>(src);
                }
            }
            __syncthreads();
        }
    }
    if (slot == 0) {
        // pairs whose expert id is out of range (never routed) get zeros in
        // this tile's columns
        const int c = nt * 16 + r;
        kq_for_unrouted(a.pair_order + a.n_pairs, a.n_pairs, [&](int p) {
            if (lane < 16 && c < a.N) kq_store_out(a.y, a.y_dtype, gather_y_row(a, p) * a.y_stride + c, 0.f);
        });
    }
    if (slot >= S) return;  // uniform over the wave
    const int expert = a.seg_info[1 + slot];
    const int seg_begin = a.seg_info[1 + a.n_experts + slot];
    const int seg_end = a.seg_info[1 + a.n_experts + slot + 1];
    const int n = nt * 16 + r;
    const bool n_valid = n < a.N;
    const int nc = n_valid ? n : a.N - 1;
    const uint8_t *wrow[NW];
    wrow[0] = a.w0 + (int64_t)expert * a.w_expert_bytes + (int64_t)nc * a.w_row_bytes;
    if constexpr (NW == 2)
        wrow[1] = a.w1 + (int64_t)expert * a.w_expert_bytes + (int64_t)nc * a.w_row_bytes;
    auto epilogue = [&](const floatx4 (&acc)[NW][MT], int c0) {
        if (!n_valid) return;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int ri = c0 + 16 * mt + 4 * (lane >> 4) + e;
                if (ri >= seg_end) continue;
                const int pair = a.pair_order[ri];
                const int ex = a.x_exp ? a.x_exp[gather_x_row(a, pair)] : 0;
                const float v = gather_epilogue<NW>(a, expert, n, ldexpf(acc[0][mt][e], ex),
                                                    ldexpf(acc[NW - 1][mt][e], ex));
                kq_store_out(a.y, a.y_dtype, gather_y_row(a, pair) * a.y_stride + n, v);
            }
        }
    };
    if constexpr (MT == 1) {
        if (staged) {
            XRowsLds xl;
            xl.base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)xs_lds +
                      (uint32_t)min(r, seg_end - seg_begin - 1) * xrow_bytes;
            floatx4 acc[NW][MT];
#pragma unroll
            for (int i = 0; i < NW; ++i) acc[i][0] = floatx4{0, 0, 0, 0};
            tile_accumulate<CODEC, MT, XT, NW, XRowsLds, false>(wrow, 0, 1, nb, xl, acc, iq2_tab);
            epilogue(acc, seg_begin);
            return;
        }
    }
    for (int c0 = seg_begin; c0 < seg_end; c0 += 16 * MT) {
        XRowPtrs<MT> xrow;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int ri = min(c0 + 16 * mt + r, seg_end - 1);
            xrow.row[mt] = a.x + gather_x_row(a, a.pair_order[ri]) * a.x_stride * x_elem_bytes<XT>();
        }
        floatx4 acc[NW][MT];
#pragma unroll
        for (int i = 0; i < NW; ++i)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[i][mt] = floatx4{0, 0, 0, 0};
        // no prefetch stage (two would not fit 128 VGPRs): resident waves hide the latency
        tile_accumulate<CODEC, MT, XT, NW, XRowPtrs<MT>, false>(wrow, 0, 1, nb, xrow, acc, iq2_tab);
        epilogue(acc, c0);
    }
}

// Routing: one workgroup, counting sort of pairs by expert (stable by pair id).
// seg_info = [S, seg_expert[E], seg_start[E+1]]; pair_order[n_pairs];
// valid_flag[n_pairs] (appended after pair_order) = expert or -1.
constexpr int kRouteThreads = 1024;
constexpr int kRouteLdsInts = 15360;  // counts, starts and (when they fit) the pairs' expert ids: 60 KB

__host__ __device__ inline bool route_staged(int n_pairs, int n_experts) {
    return 2 * n_experts + n_pairs <= kRouteLdsInts;
}

// Exclusive prefix sum of one int per thread over the workgroup
// (kRouteThreads threads); *total receives the sum.
__device__ int route_block_scan(int v, int *wsum, int *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int NWAVE = kRouteThreads / 64;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0;
        for (int w = 0; w < NWAVE; ++w) {
            const int t = wsum[w];
            wsum[w] = acc;
            acc += t;
        }
        *total = acc;
    }
    __syncthreads();
    const int r = x - v + wsum[wave];
    __syncthreads();  // wsum is reused by the next scan
    return r;
}

// Stable counting sort of (token, slot) pairs by expert id (the SwitchGLU
// order): counts in LDS, one workgroup-wide scan for the segment starts and
// the segment list, then one wave per expert walks the pairs in order and
// writes its segment, so pairs keep their original order within it.  `ids`
// holds the pairs' expert ids in LDS, or is null (they are read from idx and
// then from the flag array).  Called by all kRouteThreads threads of the
// workgroup.
__device__ void route_pairs(const int32_t *__restrict__ idx, const int32_t *ids, int32_t n_pairs,
                            int32_t n_experts, int32_t *count, int32_t *start, int32_t *__restrict__ seg_info,
                            int32_t *__restrict__ pair_order) {
    __shared__ int wsum[kRouteThreads / 64];
    __shared__ int tot_pairs, tot_segs;
    const int tid = threadIdx.x;
    for (int e = tid; e < n_experts; e += kRouteThreads) count[e] = 0;
    __syncthreads();
    int32_t *flag = pair_order + n_pairs;
    for (int p = tid; p < n_pairs; p += kRouteThreads) {
        int e = ids ? ids[p] : idx[p];
        if (e < 0 || e >= n_experts) e = -1;
        else atomicAdd(&count[e], 1);
        flag[p] = e;
    }
    __syncthreads();
    // thread t owns experts [t * per, t * per + per)
    const int per = (n_experts + kRouteThreads - 1) / kRouteThreads;
    const int e0 = tid * per, e1 = min(e0 + per, n_experts);
    int c = 0, nz = 0;
    for (int e = e0; e < e1; ++e) {
        c += count[e];
        nz += count[e] > 0;
    }
    int acc = route_block_scan(c, wsum, &tot_pairs);
    int sg = route_block_scan(nz, wsum, &tot_segs);
    for (int e = e0; e < e1; ++e) {
        start[e] = acc;
        if (count[e] > 0) {
            seg_info[1 + sg] = e;
            seg_info[1 + n_experts + sg] = acc;
            ++sg;
        }
        acc += count[e];
    }
    const int S = tot_segs, P = tot_pairs;
    if (tid == 0) seg_info[0] = S;
    for (int i = S + tid; i <= n_experts; i += kRouteThreads) seg_info[1 + n_experts + i] = P;
    for (int i = S + tid; i < n_experts; i += kRouteThreads) seg_info[1 + i] = -1;
    __syncthreads();
    // wave w writes the segments of experts w, w + 16, ...: 64 pairs per step,
    // each hit at its rank among the step's hits (ballot prefix count)
    const int wave = tid >> 6, lane = tid & 63;
    const uint64_t below = (lane ? ~0ull >> (64 - lane) : 0ull);
    for (int e = wave; e < n_experts; e += kRouteThreads / 64) {
        if (count[e] == 0) continue;  // uniform over the wave
        int w = start[e];
        for (int q0 = 0; q0 < n_pairs; q0 += 64) {
            const int q = q0 + lane;
            int id = -1;
            if (q < n_pairs) {
                id = ids ? ids[q] : flag[q];
                if (id < 0 || id >= n_experts) id = -1;
            }
            const bool hit = id == e;
            const uint64_t m = __ballot(hit);
            if (hit) pair_order[w + __popcll(m & below)] = q;
            w += __popcll(m);
        }
    }
}

// The same sort with O(1) passes over the pairs, when the chunk histograms fit
// LDS (C = ceil(n_pairs / 64) chunks x n_experts counts beside the counts and
// starts).  Chunk c (64 consecutive pairs) is one wave's step: ballots over
// the bits of each lane's expert id give every lane the mask of lanes with
// the same expert, its rank among them and the chunk's count for that expert
// (written by the expert's first lane).  Per expert, the counts turn into
// exclusive prefixes over the chunks; a pair's position is then
// start[e] + prefix[c][e] + rank, so pairs keep their order within an expert.
constexpr int kRouteFastMaxPairs = 4 * kRouteThreads;

__host__ __device__ inline bool route_fast(int n_pairs, int n_experts) {
    const int chunks = (n_pairs + 63) / 64;
    return n_pairs <= kRouteFastMaxPairs && (int64_t)chunks * n_experts + 2 * n_experts <= kRouteLdsInts;
}

__device__ void route_pairs_fast(const int32_t *__restrict__ idx, int32_t n_pairs, int32_t n_experts,
                                 int32_t *count, int32_t *start, int32_t *hist, int32_t *__restrict__ seg_info,
                                 int32_t *__restrict__ pair_order) {
    __shared__ int wsum[kRouteThreads / 64];
    __shared__ int tot_pairs, tot_segs;
    constexpr int NW = kRouteThreads / 64;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int chunks = (n_pairs + 63) / 64;
    for (int i = tid; i < chunks * n_experts; i += kRouteThreads) hist[i] = 0;
    // the lane's pairs: chunk wave + NW * j, j < 4 (n_pairs <= 4 * kRouteThreads)
    int ex[4], rank[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int p = (wave + NW * j) * 64 + lane;
        int e = -1;
        if (p < n_pairs) {
            e = idx[p];
            if (e < 0 || e >= n_experts) e = -1;
            pair_order[n_pairs + p] = e;
        }
        ex[j] = e;
    }
    // bits of e + 1 (0 for a pair routed nowhere, or past n_pairs)
    const int nbits = 32 - __builtin_clz((unsigned)n_experts);
    const uint64_t below = lane ? ~0ull >> (64 - lane) : 0ull;
    __syncthreads();  // hist zeroed
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = wave + NW * j;
        rank[j] = 0;
        if (c >= chunks) continue;  // uniform over the wave
        const uint32_t v = (uint32_t)(ex[j] + 1);
        uint64_t same = ~0ull;
        for (int b = 0; b < nbits; ++b) {
            const bool bit = (v >> b) & 1u;
            const uint64_t m = __ballot(bit);
            same &= bit ? m : ~m;
        }
        rank[j] = __popcll(same & below);
        if (ex[j] >= 0 && rank[j] == 0) hist[c * n_experts + ex[j]] = __popcll(same);
    }
    __syncthreads();
    // per expert: exclusive prefix over the chunks, and the total
    const int per = (n_experts + kRouteThreads - 1) / kRouteThreads;
    const int e0 = tid * per, e1 = min(e0 + per, n_experts);
    int tot = 0, nz = 0;
    for (int e = e0; e < e1; ++e) {
        int run = 0;
        for (int c = 0; c < chunks; ++c) {
            const int h = hist[c * n_experts + e];
            hist[c * n_experts + e] = run;
            run += h;
        }
        count[e] = run;
        tot += run;
        nz += run > 0;
    }
    int acc = route_block_scan(tot, wsum, &tot_pairs);
    int sg = route_block_scan(nz, wsum, &tot_segs);
    for (int e = e0; e < e1; ++e) {
        start[e] = acc;
        if (count[e] > 0) {
            seg_info[1 + sg] = e;
            seg_info[1 + n_experts + sg] = acc;
            ++sg;
        }
        acc += count[e];
    }
    const int S = tot_segs, P = tot_pairs;
    if (tid == 0) seg_info[0] = S;
    for (int i = S + tid; i <= n_experts; i += kRouteThreads) seg_info[1 + n_experts + i] = P;
    for (int i = S + tid; i < n_experts; i += kRouteThreads) seg_info[1 + i] = -1;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = wave + NW * j;
        if (c < chunks && ex[j] >= 0)
            pair_order[start[ex[j]] + hist[c * n_experts + ex[j]] + rank[j]] = c * 64 + lane;
    }
}

__global__ __launch_bounds__(kRouteThreads) void kq_route_kernel(const int32_t *__restrict__ idx, int32_t n_pairs,
                                                                 int32_t n_experts, int32_t *__restrict__ seg_info,
                                                                 int32_t *__restrict__ pair_order) {
    extern __shared__ int32_t sm[];
    int32_t *count = sm;                    // [E]
    int32_t *start = sm + n_experts;        // [E]
    int32_t *rest = sm + 2 * n_experts;     // chunk histograms, or the pairs' ids when staged
    if (route_fast(n_pairs, n_experts)) {
        route_pairs_fast(idx, n_pairs, n_experts, count, start, rest, seg_info, pair_order);
        return;
    }
    const bool staged = route_staged(n_pairs, n_experts);
    if (staged) {
        for (int p = threadIdx.x; p < n_pairs; p += kRouteThreads) rest[p] = idx[p];
        // route_pairs' first barrier orders these writes before any read
    }
    route_pairs(idx, staged ? rest : nullptr, n_pairs, n_experts, count, start, seg_info, pair_order);
}

__global__ void kq_mix_kernel(const float *__restrict__ yp, const float *__restrict__ sc, int32_t T,
                              int32_t k, int32_t N, void *y, int y_dtype) {
    const int t = blockIdx.y;
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    float acc = 0.f;
    for (int s = 0; s < k; ++s) acc += sc[t * k + s] * yp[((int64_t)t * k + s) * N + n];
    kq_store_out(y, y_dtype, (int64_t)t * N + n, acc);
}

// Router arguments (kq_router_options resolved on the host).
struct RouterArgs {
    const void *logits;
    int64_t ld;              // elements between tokens' logit rows
    int32_t ldt, E, k;       // logits dtype; routed experts; picks
    int32_t norm, shared_gate, scoring;
    float scale;
    const void *bias;        // [E] selection bias or null
    const void *pes;         // [E] per-expert scale or null
    int32_t bias_dt, pes_dt;
    int32_t *inds;
    float *scores;           // row stride k + shared_gate
};

__device__ __forceinline__ float router_load(const void *p, int dt, int64_t i) {
    return dt == KQ_DTYPE_F32 ? ((const float *)p)[i]
           : dt == KQ_DTYPE_F16 ? (float)((const _Float16 *)p)[i]
                                : kq_bf16_bits_to_f32(((const uint16_t *)p)[i]);
}

// Cross-lane steps of the router's reductions: DPP moves inside each row of
// 16 lanes (pair swap, quad swap, half-row mirror, row mirror), after which
// every lane of a row holds the row's result, and four lane reads combine the
// rows in row order.  DPP moves are VALU operations with a few cycles of
// latency, against an LDS round trip per step for a lane shuffle.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_row(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, __uint_as_float(dpp_row<0xB1>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_row<0x4E>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_row<0x141>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_row<0x140>(__float_as_uint(v))));
    float r = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
#pragma unroll
    for (int q = 1; q < 4; ++q) r = fmaxf(r, __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16 * q)));
    return r;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    v += __uint_as_float(dpp_row<0xB1>(__float_as_uint(v)));
    v += __uint_as_float(dpp_row<0x4E>(__float_as_uint(v)));
    v += __uint_as_float(dpp_row<0x141>(__float_as_uint(v)));
    v += __uint_as_float(dpp_row<0x140>(__float_as_uint(v)));
    float r = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
#pragma unroll
    for (int q = 1; q < 4; ++q) r += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16 * q));
    return r;
}

// A pick candidate as a 64-bit key (hi, lo): hi orders the selection score
// (larger float -> larger key; NaN lowest), lo = ~expert so that equal scores
// rank the lower expert id first.  Key (0, 0) is below every candidate.
__device__ __forceinline__ uint32_t f32_order(float f) {
    const uint32_t b = __float_as_uint(f);
    if (f != f) return 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ void key_max(uint32_t &hi, uint32_t &lo, uint32_t ohi, uint32_t olo) {
    const bool t = ohi > hi || (ohi == hi && olo > lo);
    hi = t ? ohi : hi;
    lo = t ? olo : lo;
}

template <int CTRL>
__device__ __forceinline__ void key_dpp(uint32_t &hi, uint32_t &lo) {
    const uint32_t ohi = dpp_row<CTRL>(hi), olo = dpp_row<CTRL>(lo);
    key_max(hi, lo, ohi, olo);
}

// The wave's largest key, uniform over the wave.
__device__ __forceinline__ void wave_max_key(uint32_t &hi, uint32_t &lo) {
    key_dpp<0xB1>(hi, lo);
    key_dpp<0x4E>(hi, lo);
    key_dpp<0x141>(hi, lo);
    key_dpp<0x140>(hi, lo);
    uint32_t bh = __builtin_amdgcn_readlane(hi, 0), bl = __builtin_amdgcn_readlane(lo, 0);
#pragma unroll
    for (int q = 1; q < 4; ++q)
        key_max(bh, bl, __builtin_amdgcn_readlane(hi, 16 * q), __builtin_amdgcn_readlane(lo, 16 * q));
    hi = bh;
    lo = bl;
}

// Router of one token on one wave, in fp32 (E <= 64 * NPER experts, expert
// lane + 64 i in slot i of each lane).
//   score_e = softmax over the E routed logits (max-subtracted), sigmoid, or
//             sqrt(softplus) with softplus(x) = max(x, 0) + log1p(exp(-|x|));
//   picks   = top-k of score_e + bias_e by repeated arg-max (ties -> lower
//             expert id), reported with their unbiased scores;
//   weights = picks / (sum of picks, in pick order, + 1e-20) when
//             normalising, then times per_expert_scale[e] and scale;
//   shared_gate: logit column E is the shared expert's gate, appended to the
//             weights as sigmoid(logit) (k + 1 weights per token).
template <int NPER>
__device__ __forceinline__ void router_token(const RouterArgs &a, int t, int lane) {
    const int E = a.E;
    const int64_t row = (int64_t)t * a.ld;
    float v[NPER], bias[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        const int e = lane + 64 * i;
        v[i] = e < E ? router_load(a.logits, a.ldt, row + e) : -INFINITY;
        bias[i] = (a.bias && e < E) ? router_load(a.bias, a.bias_dt, e) : 0.f;
    }
    if (a.scoring == KQ_SCORE_SOFTMAX) {
        float mx = v[0];
#pragma unroll
        for (int i = 1; i < NPER; ++i) mx = fmaxf(mx, v[i]);
        mx = wave_max_f32(mx);
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < NPER; ++i) {
            const int e = lane + 64 * i;
            v[i] = e < E ? expf(v[i] - mx) : 0.f;
            sum += v[i];
        }
        sum = wave_sum_f32(sum);
#pragma unroll
        for (int i = 0; i < NPER; ++i) v[i] = v[i] / sum;
    } else if (a.scoring == KQ_SCORE_SIGMOID) {
#pragma unroll
        for (int i = 0; i < NPER; ++i) v[i] = 1.f / (1.f + expf(-v[i]));
    } else {
#pragma unroll
        for (int i = 0; i < NPER; ++i) {
            const float x = v[i];
            v[i] = sqrtf(fmaxf(x, 0.f) + log1pf(expf(-fabsf(x))));
        }
    }
    uint32_t khi[NPER], klo[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        const int e = lane + 64 * i;
        khi[i] = e < E ? f32_order(v[i] + bias[i]) : 0u;
        klo[i] = e < E ? ~(uint32_t)e : 0u;
    }
    float picked_sum = 0.f, my_score = 0.f;
    int my_ind = 0;
    for (int j = 0; j < a.k; ++j) {
        uint32_t bh = khi[0], bl = klo[0];
#pragma unroll
        for (int i = 1; i < NPER; ++i) key_max(bh, bl, khi[i], klo[i]);
        wave_max_key(bh, bl);
        const int e = (int)~bl;  // uniform
        float sv = 0.f;
#pragma unroll
        for (int i = 0; i < NPER; ++i) {
            if (lane + 64 * i == e) {
                sv = v[i];
                khi[i] = 0u;
                klo[i] = 0u;
            }
        }
        const float best_v = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(sv), e & 63));
        picked_sum += best_v;
        if (lane == j) {
            my_score = best_v;
            my_ind = e;
        }
    }
    // one store per output array; picks are renormalised from registers
    const int sld = a.k + a.shared_gate;
    if (lane < a.k) {
        float w = a.norm ? my_score / (picked_sum + 1e-20f) : my_score;
        if (a.pes) w *= router_load(a.pes, a.pes_dt, my_ind);
        w *= a.scale;
        a.inds[(int64_t)t * a.k + lane] = my_ind;
        a.scores[(int64_t)t * sld + lane] = w;
    }
    if (a.shared_gate && lane == 0) {
        const float g = router_load(a.logits, a.ldt, row + E);
        a.scores[(int64_t)t * sld + a.k] = 1.f / (1.f + expf(-g));
    }
}

// One wave per token.
template <int NPER>
__global__ __launch_bounds__(64) void kq_router_kernel(RouterArgs a) {
    router_token<NPER>(a, blockIdx.x, kq_lane());
}

// ---------------------------------------------------------------- host


struct Plan {
    int n_tiles, mt, chunks;
};

Plan plan_problem(const kq_matmul_problem &q) {
    Plan pl;
    pl.n_tiles = (q.N + 15) / 16;
    const int mrows = q.M < kMaxChunk ? q.M : kMaxChunk;
    pl.mt = (mrows + 15) / 16;
    pl.chunks = (q.M + kMaxChunk - 1) / kMaxChunk;
    return pl;
}

int validate_problem(const kq_matmul_problem &q) {
    if (!q.w || !q.x || !q.y) return KQ_ERR_NULL_POINTER;
    if (kq_block_bytes(q.codec) == 0) return KQ_ERR_UNSUPPORTED_CODEC;
    if (q.M < 0 || q.N < 0 || q.K <= 0) return KQ_ERR_BAD_SHAPE;
    if (q.K % KQ_QK) return KQ_ERR_BAD_SHAPE;
    const int64_t need = (int64_t)(q.K / KQ_QK) * kq_block_bytes(q.codec);
    if (q.w_row_bytes < need) return KQ_ERR_BAD_SHAPE;
    if (q.x_row_stride < q.K || q.y_row_stride < q.N) return KQ_ERR_BAD_SHAPE;
    // activation rows are addressed with 32-bit byte offsets inside a 64-row chunk
    if (q.x_row_stride > (1 << 22)) return KQ_ERR_BAD_SHAPE;
    if (((uintptr_t)q.x & 15) || (q.x_row_stride & 7)) return KQ_ERR_BAD_ALIGN;
    if (q.codec == KQ_CODEC_Q4_K && (((uintptr_t)q.w & 15) || (q.w_row_bytes & 15))) return KQ_ERR_BAD_ALIGN;
    if (((uintptr_t)q.w & 1) || (q.w_row_bytes & 1)) return KQ_ERR_BAD_ALIGN;
    return KQ_OK;
}

// m-tiles per wave of one grouped launch: the largest any live problem needs
// (the kernel is instantiated once for the whole group).
int group_mt(const kq_matmul_problem *ps, int n) {
    int mt = 1;
    for (int i = 0; i < n; ++i) {
        if (ps[i].M == 0 || ps[i].N == 0) continue;
        const Plan pl = plan_problem(ps[i]);
        if (pl.mt > mt) mt = pl.mt;
    }
    return mt <= 1 ? 1 : mt <= 2 ? 2 : 4;
}

// "0" -> 0, "2" -> 2, anything else set -> 1, unset -> dflt
int env_int_flag(const char *name, int dflt) {
    const char *s = getenv(name);
    if (!s || !*s) return dflt;
    if (s[1] == 0 && (s[0] == '0' || s[0] == '2')) return s[0] - '0';
    return 1;
}

// 16 waves per tile for one m-tile, 4 waves for wider chunks
template <int MT, int XT, int NW>
void launch_dense(const DenseArgs &a, int units, int chunks, hipStream_t s) {
    constexpr int WV = MT == 1 ? 16 : 4;
    hipLaunchKernelGGL((kq_dense_grouped_kernel<MT, XT, WV, NW>), dim3(units, chunks), dim3(64 * WV), 0, s, a);
}

// Column tiles per dense workgroup: one m-tile keeps 1; wider chunks read
// their activation fragments once per super-block for NW tiles
// (GMLX_KQ_DENSE_NW: 1, 2 or 4).
int dense_nw(int mt) {
    if (mt == 1) return 1;
    const int nw = env_int("GMLX_KQ_DENSE_NW", 2);
    return nw >= 4 ? 4 : (nw >= 2 ? 2 : 1);
}

template <int MT, int XT>
void launch_dense_nw(int nw, const DenseArgs &a, int units, int chunks, hipStream_t s) {
    if constexpr (MT == 1) {
        launch_dense<MT, XT, 1>(a, units, chunks, s);
    } else {
        if (nw == 4) launch_dense<MT, XT, 4>(a, units, chunks, s);
        else if (nw == 2) launch_dense<MT, XT, 2>(a, units, chunks, s);
        else launch_dense<MT, XT, 1>(a, units, chunks, s);
    }
}

// One wave per unit (the whole K of a 16-column tile) for rows of at most 8
// super-blocks, and for longer rows when the launch's units (its grid: the
// experts it can touch times the tiles) give every CU 16 waves: the waves
// then stream their rows without the split's reduction (measured on C5,
// IQ2_XXS K = 7168, 51 touched experts, alternating in one process: 0.272
// against 0.285 ms); smaller batches split K over the workgroup's waves for
// parallelism.
// GMLX_KQ_GATHER_WAVE_NB = n forces the rule "at most n super-blocks" (0: always split).
bool gather_use_wave(const GatherArgs &a, int grid) {
    const int forced = env_int("GMLX_KQ_GATHER_WAVE_NB", -1);
    const int nb = a.K / KQ_QK;
    if (forced >= 0) return nb <= forced;
    return nb <= 8 || grid >= 16 * device_cus();
}

template <int CODEC, int XT, int NW>
void launch_gather_codec(int mt, const GatherArgs &a, int grid, hipStream_t s) {
    if (gather_use_wave(a, grid)) {
        const int g = (grid + kGatherWaves - 1) / kGatherWaves;
        switch (mt) {
        case 1: hipLaunchKernelGGL((kq_gather_wave_kernel<CODEC, 1, XT, NW>), dim3(g), dim3(64 * kGatherWaves), 0, s, a); break;
        case 2: hipLaunchKernelGGL((kq_gather_wave_kernel<CODEC, 2, XT, NW>), dim3(g), dim3(64 * kGatherWaves), 0, s, a); break;
        default: hipLaunchKernelGGL((kq_gather_wave_kernel<CODEC, 4, XT, NW>), dim3(g), dim3(64 * kGatherWaves), 0, s, a); break;
        }
        return;
    }
    switch (mt) {
    case 1: hipLaunchKernelGGL((kq_gather_kernel<CODEC, 1, XT, NW>), dim3(grid), dim3(64 * kGatherWaves), 0, s, a); break;
    case 2: hipLaunchKernelGGL((kq_gather_kernel<CODEC, 2, XT, NW>), dim3(grid), dim3(64 * kGatherWaves), 0, s, a); break;
    default: hipLaunchKernelGGL((kq_gather_kernel<CODEC, 4, XT, NW>), dim3(grid), dim3(64 * kGatherWaves), 0, s, a); break;
    }
}

template <int XT, int NW>
void launch_gather(int codec, int mt, const GatherArgs &a, int grid, hipStream_t s) {
    if (codec == KQ_CODEC_Q4_K) launch_gather_codec<KQ_CODEC_Q4_K, XT, NW>(mt, a, grid, s);
    else if (codec == KQ_CODEC_Q6_K) launch_gather_codec<KQ_CODEC_Q6_K, XT, NW>(mt, a, grid, s);
    else launch_gather_codec<KQ_CODEC_IQ2_XXS, XT, NW>(mt, a, grid, s);
}

// Activation rows a gather reads: pair p uses row p / x_pair_div + p / x_skip.
int32_t gather_x_rows(int32_t n_pairs, int32_t x_pair_div, int32_t x_skip) {
    if (n_pairs <= 0) return 0;
    return (n_pairs - 1) / x_pair_div + (x_skip ? (n_pairs - 1) / x_skip : 0) + 1;
}

int gather_common(const void *x, int x_dtype, int64_t x_row_stride, int32_t x_pair_div, const void *w0,
                  const void *w1, int64_t w_expert_bytes, int64_t w_row_bytes, int32_t N, int32_t K,
                  int codec, const kq_gather_epilogue *ep, const int32_t *seg_info, const int32_t *pair_order,
                  int32_t n_pairs, int32_t n_experts, void *y, int y_dtype, int64_t y_row_stride,
                  void *workspace, size_t workspace_bytes, hipStream_t s, int32_t x_skip = 0,
                  int32_t y_skip = 0) {
    if (!x || !w0 || !seg_info || !pair_order || !y) return KQ_ERR_NULL_POINTER;
    if (kq_block_bytes(codec) == 0) return KQ_ERR_UNSUPPORTED_CODEC;
    if (x_dtype != KQ_DTYPE_F16 && x_dtype != KQ_DTYPE_BF16 && x_dtype != KQ_DTYPE_F32)
        return KQ_ERR_UNSUPPORTED_DTYPE;
    if (y_dtype != KQ_DTYPE_F32 && y_dtype != KQ_DTYPE_F16 && y_dtype != KQ_DTYPE_BF16)
        return KQ_ERR_UNSUPPORTED_DTYPE;
    if (N <= 0 || K <= 0 || K % KQ_QK || n_pairs < 0 || n_experts <= 0 || x_pair_div <= 0 || x_skip < 0 ||
        y_skip < 0)
        return KQ_ERR_BAD_SHAPE;
    if (n_pairs == 0) return KQ_OK;
    const int64_t need = (int64_t)(K / KQ_QK) * kq_block_bytes(codec);
    if (w_row_bytes < need || w_expert_bytes < w_row_bytes * N) return KQ_ERR_BAD_SHAPE;
    if (x_row_stride < K || y_row_stride < N) return KQ_ERR_BAD_SHAPE;
    if (((uintptr_t)x & 15) || (x_row_stride & (x_dtype == KQ_DTYPE_F32 ? 3 : 7))) return KQ_ERR_BAD_ALIGN;
    if (codec == KQ_CODEC_Q4_K && (((uintptr_t)w0 & 15) || (w_row_bytes & 15) || (w_expert_bytes & 15) ||
                                   (w1 && ((uintptr_t)w1 & 15))))
        return KQ_ERR_BAD_ALIGN;
    if (((uintptr_t)w0 & 1) || (w_row_bytes & 1) || (w_expert_bytes & 1)) return KQ_ERR_BAD_ALIGN;
    const kq_gather_epilogue plain{KQ_ACT_SILU, 0.f, 0.f, nullptr, nullptr, 0};
    if (!ep) ep = &plain;
    if (w1 && (ep->act < KQ_ACT_SILU || ep->act > KQ_ACT_SWIGLU_CLAMP)) return KQ_ERR_BAD_ARGUMENT;
    if (!w1 && ep->bias1) return KQ_ERR_BAD_ARGUMENT;
    if (w1 && ep->act != KQ_ACT_SWIGLU_CLAMP && (ep->bias0 || ep->bias1)) return KQ_ERR_BAD_ARGUMENT;
    if ((ep->bias0 || ep->bias1) && ep->bias_expert_stride < N) return KQ_ERR_BAD_SHAPE;
    if (((uintptr_t)ep->bias0 | (uintptr_t)ep->bias1) & 3) return KQ_ERR_BAD_ALIGN;
    if ((ep->act == KQ_ACT_SILU_LIMIT || ep->act == KQ_ACT_SWIGLU_CLAMP) && w1 && !(ep->limit > 0.f))
        return KQ_ERR_BAD_ARGUMENT;
    // bf16 / fp32 activations: fp16 rows with a power of two per row first
    const int32_t *x_exp = nullptr;
    if (x_dtype != KQ_DTYPE_F16) {
        const int32_t rows = gather_x_rows(n_pairs, x_pair_div, x_skip);
        if (!workspace || workspace_bytes < KQ_MATMUL_COUNTER_BYTES + kq_prepared_bytes(rows, K))
            return KQ_ERR_WORKSPACE_TOO_SMALL;
        const void *x16 = nullptr;
        if (const int rc = kq_prepare_rows(x, x_dtype, x_row_stride, rows, K,
                                           (char *)workspace + KQ_MATMUL_COUNTER_BYTES, &x_exp, &x16, s))
            return rc;
        x = x16;
        x_row_stride = K;
        x_dtype = KQ_DTYPE_F16;
    }
    // the streaming gather: weight tiles by row-contiguous direct-to-LDS
    // copies, one persistent workgroup per CU
    if (kq_sgather_eligible(codec, w1 != nullptr, N, K, w_row_bytes, n_experts))
        return kq_sgather_launch(x, x_exp, x_row_stride, x_pair_div, x_skip, w0, w1, w_expert_bytes, w_row_bytes, N,
                                 K, codec, w1 ? ep->act : KQ_ACT_SILU, ep->limit, ep->alpha, ep->bias0,
                                 w1 ? ep->bias1 : nullptr, ep->bias_expert_stride, seg_info, pair_order, n_pairs,
                                 n_experts, y, y_dtype, y_row_stride, y_skip, s);
    GatherArgs a;
    a.x = (const char *)x;
    a.x_exp = x_exp;
    a.w0 = (const uint8_t *)w0;
    a.w1 = (const uint8_t *)w1;
    a.y = y;
    a.seg_info = seg_info;
    a.pair_order = pair_order;
    a.x_stride = x_row_stride;
    a.w_expert_bytes = w_expert_bytes;
    a.w_row_bytes = w_row_bytes;
    a.y_stride = y_row_stride;
    a.x_pair_div = x_pair_div;
    a.x_skip = x_skip;
    a.y_skip = y_skip;
    a.N = N;
    a.K = K;
    a.n_pairs = n_pairs;
    a.n_experts = n_experts;
    a.n_tiles = (N + 15) / 16;
    a.y_dtype = y_dtype;
    a.act = w1 ? ep->act : KQ_ACT_SILU;
    a.limit = ep->limit;
    a.alpha = ep->alpha;
    a.b0 = ep->bias0;
    a.b1 = w1 ? ep->bias1 : nullptr;
    a.b_stride = ep->bias_expert_stride;
    // m-tiles per chunk from the mean segment length (pairs spread over the
    // experts): decode batches leave a few rows per expert; longer segments
    // are walked in chunks of 16 * mt rows
    const int slots = n_experts < n_pairs ? n_experts : n_pairs;
    const int rows = (n_pairs + slots - 1) / slots;
    const int mt = rows <= 16 ? 1 : rows <= 32 ? 2 : 4;
    const int grid = slots * a.n_tiles;
    if (w1) launch_gather<0, 2>(codec, mt, a, grid, s);
    else launch_gather<0, 1>(codec, mt, a, grid, s);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

// Bytes of prepared activation rows (a copy per problem; problems sharing x share one).
size_t prepared_total(const kq_matmul_problem *problems, int n_problems, int x_dtype) {
    if (x_dtype == KQ_DTYPE_F16) return 0;
    size_t b = 0;
    for (int i = 0; i < n_problems && i < KQ_MAX_GROUP; ++i)
        if (problems[i].M > 0 && problems[i].N > 0) b += kq_prepared_bytes(problems[i].M, problems[i].K);
    return b;
}

// Partial-tile bytes of a split launch of the group's live problems (0: none).
size_t split_bytes(const kq_matmul_problem *problems, int n_problems) {
    kq_matmul_problem all[KQ_MAX_GROUP];
    int na = 0;
    for (int i = 0; i < n_problems && i < KQ_MAX_GROUP; ++i)
        if (problems[i].M > 0 && problems[i].N > 0) all[na++] = problems[i];
    if (na == 0) return 0;
    const size_t a = kq_stream_part_bytes(all, na, kq_stream_split_want(all, na)), b = kq_mms_part_bytes(all, na);
    return a > b ? a : b;
}

}  // namespace

// Compute units of the current device (cached per device id; 256 on MI355X).
int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

extern "C" {

size_t kq_matmul_workspace_bytes(const kq_matmul_problem *problems, int n_problems, int x_dtype) {
    if (!problems || n_problems <= 0) return 0;
    const size_t b = prepared_total(problems, n_problems, x_dtype) + split_bytes(problems, n_problems);
    return b ? KQ_MATMUL_COUNTER_BYTES + b : 0;
}

int kq_quantized_matmul_grouped(const kq_matmul_problem *problems, int n_problems, int x_dtype,
                                int y_dtype, void *workspace, size_t workspace_bytes,
                                kq_stream_t stream) {
    if (!problems) return KQ_ERR_NULL_POINTER;
    if (n_problems <= 0) return KQ_ERR_BAD_ARGUMENT;
    if (n_problems > KQ_MAX_GROUP) return KQ_ERR_TOO_MANY_PROBLEMS;
    if (x_dtype != KQ_DTYPE_F16 && x_dtype != KQ_DTYPE_BF16 && x_dtype != KQ_DTYPE_F32)
        return KQ_ERR_UNSUPPORTED_DTYPE;
    if (y_dtype != KQ_DTYPE_F32 && y_dtype != KQ_DTYPE_F16 && y_dtype != KQ_DTYPE_BF16)
        return KQ_ERR_UNSUPPORTED_DTYPE;
    for (int i = 0; i < n_problems; ++i) {
        const int rc = validate_problem(problems[i]);
        if (rc != KQ_OK) return rc;
    }
    // bf16 / fp32 activations: fp16 rows with a power of two per row, once per
    // distinct x; every kernel below then reads fp16 and scales its fp32
    // results back (x_exp)
    kq_matmul_problem prep[KQ_MAX_GROUP];
    const int32_t *exps[KQ_MAX_GROUP] = {};
    // workspace: arrival counters, prepared rows, then split partial tiles
    size_t used = KQ_MATMUL_COUNTER_BYTES;
    if (x_dtype != KQ_DTYPE_F16) {
        if (!workspace || workspace_bytes < used + prepared_total(problems, n_problems, x_dtype))
            return KQ_ERR_WORKSPACE_TOO_SMALL;
        size_t off = used;
        for (int i = 0; i < n_problems; ++i) {
            prep[i] = problems[i];
            if (prep[i].M == 0 || prep[i].N == 0) continue;
            int j = 0;
            for (; j < i; ++j)
                if (exps[j] && problems[j].x == problems[i].x && problems[j].x_row_stride == problems[i].x_row_stride &&
                    problems[j].M == problems[i].M && problems[j].K == problems[i].K)
                    break;
            if (j < i) {
                prep[i].x = prep[j].x;
                prep[i].x_row_stride = prep[j].x_row_stride;
                exps[i] = exps[j];
                continue;
            }
            const void *x16 = nullptr;
            const int rc = kq_prepare_rows(problems[i].x, x_dtype, problems[i].x_row_stride, problems[i].M,
                                           problems[i].K, (char *)workspace + off, &exps[i], &x16,
                                           (hipStream_t)stream);
            if (rc != KQ_OK) return rc;
            prep[i].x = x16;
            prep[i].x_row_stride = problems[i].K;
            off += kq_prepared_bytes(problems[i].M, problems[i].K);
        }
        used = off;
        problems = prep;
        x_dtype = KQ_DTYPE_F16;
    }
    // live problems by codec (the small-batch paths launch once per codec)
    int by_codec[3][KQ_MAX_GROUP], cnt[3] = {0, 0, 0};
    int live = 0;
    {
        const int codecs[3] = {KQ_CODEC_Q4_K, KQ_CODEC_Q6_K, KQ_CODEC_IQ2_XXS};
        for (int i = 0; i < n_problems; ++i) {
            if (problems[i].M == 0 || problems[i].N == 0) continue;
            ++live;
            for (int c = 0; c < 3; ++c)
                if (problems[i].codec == codecs[c]) by_codec[c][cnt[c]++] = i;
        }
    }
    const int32_t *xe0 = nullptr;  // exponents of the first live problem's rows (shared-x launches)
    for (int i = 0; i < n_problems; ++i)
        if (problems[i].M != 0 && problems[i].N != 0) {
            xe0 = exps[i];
            break;
        }
    // small batches with activations that fit in LDS: the LDS-staged path.
    // Other codec mixes (IQ2_XXS with K-quants) take one launch per codec
    // only when every codec's launch is large (four tiles per CU); otherwise
    // one dense launch serves the whole group (GMLX_KQ_MV=2 forces the path).
    const int mv_mode = env_int_flag("GMLX_KQ_MV", 1);
    if (live > 0 && mv_mode) {
        // one launch for the whole group: one codec, or Q4_K with Q6_K
        kq_matmul_problem all[KQ_MAX_GROUP];
        int na = 0;
        for (int i = 0; i < n_problems; ++i)
            if (problems[i].M != 0 && problems[i].N != 0) all[na++] = problems[i];
        // at most two tiles per CU that fit in LDS with x: every byte at once
        if (kq_shot_eligible(all, na)) return kq_shot_launch(all, na, xe0, y_dtype, (hipStream_t)stream);
        // K past 16 super-blocks: K slices, given room for their partial tiles
        int split = kq_stream_split_want(all, na);
        if (split > 1 && (!workspace || ((uintptr_t)workspace & 255) ||
                          workspace_bytes < used + kq_stream_part_bytes(all, na, split)))
            split = 1;
        if (kq_stream_eligible(all, na, split))
            return kq_stream_launch(all, na, xe0, y_dtype, split, (uint32_t *)workspace,
                                    split > 1 ? (float *)((char *)workspace + used) : nullptr, (hipStream_t)stream);
        if (kq_mv_eligible(all, na, x_dtype, y_dtype)) return kq_mv_launch(all, na, xe0, y_dtype, (hipStream_t)stream);
    }
    if (live > 0 && mv_mode) {
        bool ok = true;
        const int n_codecs = (cnt[0] > 0) + (cnt[1] > 0) + (cnt[2] > 0);
        kq_matmul_problem sub[3][KQ_MAX_GROUP];
        for (int c = 0; c < 3 && ok; ++c) {
            if (!cnt[c]) continue;
            int tiles = 0;
            for (int i = 0; i < cnt[c]; ++i) {
                sub[c][i] = problems[by_codec[c][i]];
                tiles += (sub[c][i].N + 15) / 16;
            }
            ok = kq_mv_eligible(sub[c], cnt[c], x_dtype, y_dtype) &&
                 (mv_mode == 2 || n_codecs == 1 || tiles >= 4 * device_cus());
        }
        if (ok) {
            for (int c = 0; c < 3; ++c) {
                if (!cnt[c]) continue;
                const int rc = kq_mv_launch(sub[c], cnt[c], exps[by_codec[c][0]], y_dtype, (hipStream_t)stream);
                if (rc != KQ_OK) return rc;
            }
            return KQ_OK;
        }
    }
    // 17..64 rows sharing their activations: the mid-batch streaming kernel
    // (K in stages, the activations read once per CU and unit; GMLX_KQ_MMS=0
    // declines); else one launch with the activations streamed through LDS
    // once per group of weight tiles (GMLX_KQ_MM=0: the dense kernel instead)
    if (live > 0) {
        kq_matmul_problem all[KQ_MAX_GROUP];
        int na = 0;
        for (int i = 0; i < n_problems; ++i)
            if (problems[i].M != 0 && problems[i].N != 0) all[na++] = problems[i];
        // K slices given room for their partial tiles
        const size_t pb = kq_mms_part_bytes(all, na);
        const bool room = pb && workspace && !((uintptr_t)workspace & 255) && workspace_bytes >= used + pb;
        if (kq_mms_eligible(all, na, room))
            return kq_mms_launch(all, na, xe0, y_dtype, room ? (uint32_t *)workspace : nullptr,
                                 room ? (float *)((char *)workspace + used) : nullptr, (hipStream_t)stream);
        if (env_int_flag("GMLX_KQ_MM", 1) && kq_mm_eligible(all, na, x_dtype))
            return kq_mm_launch(all, na, xe0, y_dtype, (hipStream_t)stream);
    }
    DenseArgs a;
    int units = 0, max_chunks = 0, np = 0;
    const int mt = group_mt(problems, n_problems);
    const int nw = dense_nw(mt);
    for (int i = 0; i < n_problems; ++i) {
        const kq_matmul_problem &q = problems[i];
        if (q.M == 0 || q.N == 0) continue;
        const Plan pl = plan_problem(q);
        DenseProblem &p = a.p[np++];
        p.w = (const uint8_t *)q.w;
        p.x = (const char *)q.x;
        p.x_exp = exps[i];
        p.y = q.y;
        p.w_row_bytes = q.w_row_bytes;
        p.x_stride = q.x_row_stride;
        p.y_stride = q.y_row_stride;
        p.M = q.M;
        p.N = q.N;
        p.K = q.K;
        p.codec = q.codec;
        p.n_tiles = (pl.n_tiles + nw - 1) / nw;
        p.unit_begin = units;
        units += p.n_tiles;
        if (pl.chunks > max_chunks) max_chunks = pl.chunks;
    }
    if (np == 0) return KQ_OK;
    if (max_chunks > 65535) return KQ_ERR_BAD_SHAPE;
    a.n_problems = np;
    a.y_dtype = y_dtype;
    hipStream_t s = (hipStream_t)stream;
    if (mt == 1) launch_dense_nw<1, 0>(nw, a, units, max_chunks, s);
    else if (mt == 2) launch_dense_nw<2, 0>(nw, a, units, max_chunks, s);
    else launch_dense_nw<4, 0>(nw, a, units, max_chunks, s);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

size_t kq_fused_mlp_workspace_bytes(int32_t M, int32_t K, int32_t I, int32_t N, int x_dtype) {
    (void)x_dtype;
    if (M <= 0 || K <= 0 || I <= 0 || N <= 0) return 0;
    return KQ_MATMUL_COUNTER_BYTES + kq_mlp_work_bytes(I, N);
}

int kq_fused_mlp(const void *x, int x_dtype, int64_t x_row_stride, int32_t M, int32_t K, const void *w_gate,
                 const void *w_up, int64_t gu_row_bytes, int gu_codec, int32_t I, const void *w_down,
                 int64_t down_row_bytes, int down_codec, int32_t N, int act, void *y, int y_dtype,
                 int64_t y_row_stride, void *workspace, size_t workspace_bytes, kq_stream_t stream) {
    if (!x || !w_gate || !w_up || !w_down || !y) return KQ_ERR_NULL_POINTER;
    if (kq_block_bytes(gu_codec) == 0 || kq_block_bytes(down_codec) == 0) return KQ_ERR_UNSUPPORTED_CODEC;
    if (x_dtype != KQ_DTYPE_F16 && x_dtype != KQ_DTYPE_BF16 && x_dtype != KQ_DTYPE_F32)
        return KQ_ERR_UNSUPPORTED_DTYPE;
    if (y_dtype != KQ_DTYPE_F32 && y_dtype != KQ_DTYPE_F16 && y_dtype != KQ_DTYPE_BF16)
        return KQ_ERR_UNSUPPORTED_DTYPE;
    if (act != KQ_ACT_SILU && act != KQ_ACT_GELU) return KQ_ERR_BAD_ARGUMENT;
    if (M < 0 || K <= 0 || I <= 0 || N <= 0 || K % KQ_QK || I % KQ_QK) return KQ_ERR_BAD_SHAPE;
    if (M == 0) return KQ_OK;
    if (gu_row_bytes < (int64_t)(K / KQ_QK) * kq_block_bytes(gu_codec) ||
        down_row_bytes < (int64_t)(I / KQ_QK) * kq_block_bytes(down_codec) || x_row_stride < K || y_row_stride < N)
        return KQ_ERR_BAD_SHAPE;
    if (((uintptr_t)x & 15) || (x_row_stride & (x_dtype == KQ_DTYPE_F32 ? 3 : 7))) return KQ_ERR_BAD_ALIGN;
    if (((uintptr_t)w_gate & 15) || ((uintptr_t)w_up & 15) || (gu_row_bytes & 15)) return KQ_ERR_BAD_ALIGN;
    if (((uintptr_t)w_down & 1) || (down_row_bytes & 1) ||
        (down_codec == KQ_CODEC_Q4_K && (((uintptr_t)w_down & 15) || (down_row_bytes & 15))))
        return KQ_ERR_BAD_ALIGN;
    // h is held as fp16: the single launch serves fp16 activations (other
    // dtypes keep h in their own dtype, as the reference's swiglu does)
    if (x_dtype != KQ_DTYPE_F16 ||
        !kq_mlp_eligible(M, K, I, N, gu_codec, down_codec, gu_row_bytes, down_row_bytes))
        return KQ_ERR_BAD_SHAPE;
    if (!workspace || ((uintptr_t)workspace & 255) ||
        workspace_bytes < kq_fused_mlp_workspace_bytes(M, K, I, N, x_dtype))
        return KQ_ERR_WORKSPACE_TOO_SMALL;
    return kq_mlp_launch(x, nullptr, x_row_stride, M, K, w_gate, w_up, gu_row_bytes, I, w_down, down_row_bytes,
                         down_codec, N, act, y, y_dtype, y_row_stride, workspace, (hipStream_t)stream);
}

int kq_moe_route(const int32_t *idx, int32_t n_pairs, int32_t n_experts, int32_t *seg_info,
                 int32_t *pair_order, kq_stream_t stream) {
    if (!idx || !seg_info || !pair_order) return KQ_ERR_NULL_POINTER;
    if (n_pairs < 0 || n_experts <= 0 || n_experts > 4096) return KQ_ERR_BAD_SHAPE;
    const size_t rest = route_fast(n_pairs, n_experts) ? (size_t)((n_pairs + 63) / 64) * n_experts
                        : route_staged(n_pairs, n_experts) ? (size_t)n_pairs : 0;
    const size_t smem = ((size_t)2 * n_experts + rest) * sizeof(int32_t);
    hipLaunchKernelGGL(kq_route_kernel, dim3(1), dim3(kRouteThreads), smem, (hipStream_t)stream, idx, n_pairs,
                       n_experts, seg_info, pair_order);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

int kq_gather_qmm(const void *x, int x_dtype, int64_t x_row_stride, int32_t x_pair_div, const void *w,
                  int64_t w_expert_bytes, int64_t w_row_bytes, int32_t N, int32_t K, int codec,
                  const int32_t *seg_info, const int32_t *pair_order, int32_t n_pairs,
                  int32_t n_experts, void *y, int y_dtype, int64_t y_row_stride, void *workspace,
                  size_t workspace_bytes, kq_stream_t stream) {
    return gather_common(x, x_dtype, x_row_stride, x_pair_div, w, nullptr, w_expert_bytes, w_row_bytes,
                         N, K, codec, nullptr, seg_info, pair_order, n_pairs, n_experts, y, y_dtype,
                         y_row_stride, workspace, workspace_bytes, (hipStream_t)stream);
}

int kq_moe_glu_gather(const void *x, int x_dtype, int64_t x_row_stride, int32_t x_pair_div,
                      const void *w_gate, const void *w_up, int64_t w_expert_bytes, int64_t w_row_bytes,
                      int32_t N, int32_t K, int codec, int act, const int32_t *seg_info,
                      const int32_t *pair_order, int32_t n_pairs, int32_t n_experts, float *h,
                      void *workspace, size_t workspace_bytes, kq_stream_t stream) {
    if (!w_up) return KQ_ERR_NULL_POINTER;
    if (act != KQ_ACT_SILU && act != KQ_ACT_GELU) return KQ_ERR_BAD_ARGUMENT;
    const kq_gather_epilogue ep{act, 0.f, 0.f, nullptr, nullptr, 0};
    return gather_common(x, x_dtype, x_row_stride, x_pair_div, w_gate, w_up, w_expert_bytes, w_row_bytes,
                         N, K, codec, &ep, seg_info, pair_order, n_pairs, n_experts, h, KQ_DTYPE_F32, N,
                         workspace, workspace_bytes, (hipStream_t)stream);
}

int kq_moe_gather_rows(const void *x, int x_dtype, int64_t x_row_stride, int32_t x_pair_div, int32_t x_skip,
                       const void *w0, const void *w1, int64_t w_expert_bytes, int64_t w_row_bytes, int32_t N,
                       int32_t K, int codec, const kq_gather_epilogue *ep, const int32_t *seg_info,
                       const int32_t *pair_order, int32_t n_pairs, int32_t n_experts, void *y, int y_dtype,
                       int64_t y_row_stride, int32_t y_skip, void *workspace, size_t workspace_bytes,
                       kq_stream_t stream) {
    return gather_common(x, x_dtype, x_row_stride, x_pair_div, w0, w1, w_expert_bytes, w_row_bytes, N, K, codec,
                         ep, seg_info, pair_order, n_pairs, n_experts, y, y_dtype, y_row_stride, workspace,
                         workspace_bytes, (hipStream_t)stream, x_skip, y_skip);
}

size_t kq_gather_workspace_bytes(int32_t n_pairs, int32_t x_pair_div, int32_t x_skip, int32_t K, int x_dtype) {
    if (x_dtype == KQ_DTYPE_F16 || n_pairs <= 0 || x_pair_div <= 0 || x_skip < 0 || K <= 0) return 0;
    return KQ_MATMUL_COUNTER_BYTES + kq_prepared_bytes(gather_x_rows(n_pairs, x_pair_div, x_skip), K);
}

int kq_moe_mix(const float *y_pairs, const float *scores, int32_t T, int32_t top_k, int32_t N, void *y,
               int y_dtype, kq_stream_t stream) {
    if (!y_pairs || !scores || !y) return KQ_ERR_NULL_POINTER;
    if (T < 0 || top_k <= 0 || N <= 0) return KQ_ERR_BAD_SHAPE;
    if (y_dtype != KQ_DTYPE_F32 && y_dtype != KQ_DTYPE_F16 && y_dtype != KQ_DTYPE_BF16)
        return KQ_ERR_UNSUPPORTED_DTYPE;
    if (T == 0) return KQ_OK;
    hipLaunchKernelGGL(kq_mix_kernel, dim3((N + 255) / 256, T), dim3(256), 0, (hipStream_t)stream, y_pairs,
                       scores, T, top_k, N, y, y_dtype);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

}  // extern "C"

// Validates a router call and fills its arguments (KQ_OK or a status).
static int router_args(const void *logits, int logits_dtype, int64_t logits_row_stride, int32_t T, int32_t E,
                       int32_t k, const kq_router_options *opts, int32_t *inds, float *scores, RouterArgs &a) {
    if (!logits || !inds || !scores) return KQ_ERR_NULL_POINTER;
    const kq_router_options dflt{1, 0, KQ_SCORE_SOFTMAX, 1.f, nullptr, KQ_DTYPE_F32, nullptr, KQ_DTYPE_F32};
    const kq_router_options &o = opts ? *opts : dflt;
    const int sg = o.shared_gate ? 1 : 0;
    if (T < 0 || E <= 0 || E > 1024 || k <= 0 || k > 32 || k > E || logits_row_stride < E + sg)
        return KQ_ERR_BAD_SHAPE;
    auto dt_ok = [](int d) { return d == KQ_DTYPE_F32 || d == KQ_DTYPE_F16 || d == KQ_DTYPE_BF16; };
    if (!dt_ok(logits_dtype) || (o.bias && !dt_ok(o.bias_dtype)) ||
        (o.per_expert_scale && !dt_ok(o.per_expert_scale_dtype)))
        return KQ_ERR_UNSUPPORTED_DTYPE;
    if (o.scoring < KQ_SCORE_SOFTMAX || o.scoring > KQ_SCORE_SQRTSOFTPLUS) return KQ_ERR_BAD_ARGUMENT;
    a.logits = logits;
    a.ld = logits_row_stride;
    a.ldt = logits_dtype;
    a.E = E;
    a.k = k;
    a.norm = o.norm_topk_prob ? 1 : 0;
    a.shared_gate = sg;
    a.scoring = o.scoring;
    a.scale = o.scale;
    a.bias = o.bias;
    a.bias_dt = o.bias_dtype;
    a.pes = o.per_expert_scale;
    a.pes_dt = o.per_expert_scale_dtype;
    a.inds = inds;
    a.scores = scores;
    return KQ_OK;
}

extern "C" {

int kq_moe_router_topk(const void *logits, int logits_dtype, int64_t logits_row_stride, int32_t T, int32_t E,
                       int32_t k, const kq_router_options *opts, int32_t *inds, float *scores,
                       kq_stream_t stream) {
    RouterArgs a;
    const int st = router_args(logits, logits_dtype, logits_row_stride, T, E, k, opts, inds, scores, a);
    if (st != KQ_OK) return st;
    if (T == 0) return KQ_OK;
    const hipStream_t s = (hipStream_t)stream;
    if (E <= 64) hipLaunchKernelGGL(kq_router_kernel<1>, dim3(T), dim3(64), 0, s, a);
    else if (E <= 128) hipLaunchKernelGGL(kq_router_kernel<2>, dim3(T), dim3(64), 0, s, a);
    else if (E <= 256) hipLaunchKernelGGL(kq_router_kernel<4>, dim3(T), dim3(64), 0, s, a);
    else if (E <= 512) hipLaunchKernelGGL(kq_router_kernel<8>, dim3(T), dim3(64), 0, s, a);
    else hipLaunchKernelGGL(kq_router_kernel<16>, dim3(T), dim3(64), 0, s, a);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

}  // extern "C"
