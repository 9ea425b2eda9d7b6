// Dequant-fused matmul for batches of 17..64 activation rows that share their
// activations (the q|k|v, o, gate|up and down calls of a decode step at
// B = 17..64, the ragged batch widths past the small-batch path).
//
// y[M, N] = x[M, K] . dequant(W[N, K])^T,   Q4_K and Q6_K weights.
//
// At these widths every weight value feeds 17..64 products, so the cost that
// grows with M is the activation traffic, not the weights: a workgroup that
// computes 16 output columns must see all of x (M * K * 2 bytes, 512 KB at
// M = 64, K = 4096).  Work decomposition:
//   - one persistent workgroup of 4 waves per CU (one wave per SIMD, the
//     whole register file for it) walks groups of T consecutive 16-row weight
//     tiles of one problem;
//   - wave w takes super-blocks w, w + 4, ... of every tile of the group, so
//     each activation byte is loaded by one wave of the CU once per group and
//     multiplied against T tiles;
//   - a wave streams its activations in quarter-block stages (64 columns of
//     every activation row): each stage is read with row-contiguous loads
//     (8 rows x 128 bytes per instruction; the MFMA fragment layout would
//     touch 16 rows per instruction, which measured twice as slow), three
//     stages ahead through a register ring, then written to a per-wave LDS
//     double buffer one quarter before its multiply and read back as MFMA
//     fragments.  The weights go through the register lane views of
//     kq_mma.h one super-block ahead.  All global reads are ordinary vector
//     loads, so the compiler's wait counts follow the ring exactly; a wave
//     reads back only what it wrote itself, so no barrier runs in the K loop;
//   - after the K loop the four waves' partial tiles are summed through LDS
//     in wave order (deterministic results) and stored.
#include <stdlib.h>

#include <type_traits>

#include "kq_mma.h"

int device_cus();

namespace {

using namespace kqmma;

constexpr int kMmWaves = 4;  // waves per workgroup, one per SIMD
constexpr int kStages = 4;   // activation stages in a wave's register ring

enum { kSetQ4K = 0, kSetQ6K = 1, kSetMix = 2 };

struct MmProblem {
    const uint8_t *w;
    void *y;
    int64_t w_row_bytes, y_stride;  // bytes, elements
    int32_t N, codec;
};

struct MmArgs {
    int32_t group_begin[KQ_MAX_GROUP];  // first group of each problem; unused: INT_MAX
    MmProblem p[KQ_MAX_GROUP];
    const char *x;
    const int32_t *x_exp;  // per-row exponents of prepared activations (results * 2^e), or null
    int64_t x_stride;  // elements
    int32_t M, K, y_dtype, total_groups, n_problems;
};

// Kernel arguments read in place through the constant address space.
typedef const __attribute__((address_space(4))) MmArgs *KArgs;

// One group: tiles tile0 .. tile0 + T - 1 of a problem, all M rows.
template <int CODEC, int MT, int XT, int T>
__device__ __forceinline__ void mm_group(KArgs A, const uint8_t *w, int64_t w_row_bytes, void *y,
                                         int64_t y_stride, int N, int tile0, floatx4 *red, u32x4 *xstage) {
    constexpr int BPB = kq_block_bytes(CODEC);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = kq_lane(), r = lane & 15, g = lane >> 4;
    const int M = A->M, K = A->K, nb = K / KQ_QK;

    floatx4 acc[T][MT];
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[i][mt] = floatx4{0, 0, 0, 0};

    const int my_blocks = nb > wave ? (nb - wave + kMmWaves - 1) / kMmWaves : 0;  // uniform
    if (my_blocks > 0) {
        const uint8_t *wrow[T];
#pragma unroll
        for (int i = 0; i < T; ++i) wrow[i] = w + (int64_t)min((tile0 + i) * 16 + r, N - 1) * w_row_bytes;
        // coalesced activation loads: instruction (mt, v) reads rows
        // 16 mt + 8 v + lane / 8, piece lane % 8 (16 B) of the stage's 128 B
        // per row; rows past M lie outside the buffer and read zeros
        const __amdgpu_buffer_rsrc_t xrs = kq_buffer(A->x, (uint32_t)(((int64_t)(M - 1) * A->x_stride + K) * 2));
        const uint32_t x_oob = (uint32_t)(((int64_t)(M - 1) * A->x_stride + K) * 2);
        uint32_t row_off[MT][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                const int m = 16 * mt + 8 * v + (lane >> 3);
                row_off[mt][v] = m < M ? (uint32_t)((int64_t)m * A->x_stride * 2 + 16 * (lane & 7)) : x_oob;
            }
        const int n_stages = 4 * my_blocks;
        // stage s: quarter s % 4 (MFMA steps 2q, 2q + 1) of super-block
        // wave + 4 (s / 4).  Stages past the end re-load the last stage
        // (uniform loads, exact wait counts).
        u32x4 raw[kStages][MT][2];
        auto load_stage = [&](u32x4 (&dst)[MT][2], int s) {
            const int sc = min(s, n_stages - 1);
            const uint32_t colb = (uint32_t)(((wave + kMmWaves * (sc >> 2)) * KQ_QK + 64 * (sc & 3)) * 2);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 2; ++v)
                    dst[mt][v] = __builtin_bit_cast(  // lane row offset + wave-uniform column (scalar offset)
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, row_off[mt][v], (int)colb, 0));
        };
        // LDS stage buffers of this wave: row m at 128 m, piece c at
        // 16 (c ^ (m & 7)) (conflict-free for the row-wise writes and the
        // fragment reads)
        u32x4 *stage_buf = xstage + wave * 2 * (16 * MT * 8);
        const int wr_row = lane >> 3, wr_piece = lane & 7;
        auto write_stage = [&](const u32x4 (&src)[MT][2], int buf) {
            u32x4 *b = stage_buf + buf * (16 * MT * 8);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 2; ++v) {
                    const int m = 16 * mt + 8 * v + wr_row;
                    b[m * 8 + (wr_piece ^ (m & 7))] = src[mt][v];
                }
        };
        // super-block bi: the next one's weights requested first (past the
        // end: this one again); quarter q requests stage s + 3 (register
        // ring), writes stage s + 1 (loaded two quarters ago) to the free LDS
        // buffer and multiplies stage s (written one quarter ago)
        auto do_block = [&](Block<CODEC> (&cur)[T], Block<CODEC> (&nxt)[T], int bi, auto slot0) {
            constexpr int j0 = decltype(slot0)::value;
            const int kb_next = wave + kMmWaves * min(bi + 1, my_blocks - 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < T; ++i) nxt[i].load(wrow[i] + (int64_t)kb_next * BPB, g);
#pragma unroll
            for (int i = 0; i < T; ++i) cur[i].prep(g);
            floatx4 P[T][MT];                // the super-block's chains (exact integer weights)
            [[maybe_unused]] floatx4 Sm[MT];  // Q4_K: its activation sub-block sums
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int jq = j0 + q;
                // the requests stay ahead of this quarter's multiplies (the
                // scheduler would otherwise sink them next to their use)
                __builtin_amdgcn_sched_barrier(0);
                load_stage(raw[(jq + kStages - 1) % kStages], 4 * bi + q + kStages - 1);
                __builtin_amdgcn_sched_barrier(0);
                write_stage(raw[(jq + 1) % kStages], (q + 1) & 1);
                const u32x4 *b = stage_buf + (q & 1) * (16 * MT * 8);
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int t = 2 * q + u;
                    half8_t xf[MT];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const int m = 16 * mt + r;
                        xf[mt] = x8_from_bits<XT>(b[m * 8 + ((4 * u + g) ^ (m & 7))]);
                    }
                    if constexpr (CODEC == KQ_CODEC_Q4_K) {
                        const half8_t sel = sum_sel(r, sum_row(t, 0));
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            Sm[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, xf[mt], t == 0 ? fzero4() : Sm[mt], 0,
                                                                            0, 0);
                    }
#pragma unroll
                    for (int i = 0; i < T; ++i) {
                        const half8_t bw = cur[i].frag(t, g, kIq2);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            P[i][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[mt], bw, t == 0 ? fzero4() : P[i][mt],
                                                                              0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < T; ++i) {
                const float f = cur[i].dscale();
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) acc[i][mt] = fold4(f, P[i][mt], acc[i][mt]);
                if constexpr (CODEC == KQ_CODEC_Q4_K) {
                    float b0, b1;
                    cur[i].min_b(g, b0, b1);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[i][mt] = min_accumulate(Sm[mt][0], Sm[mt][1], b0, b1, acc[i][mt]);
                }
            }
        };
        Block<CODEC> b0[T], b1[T];
#pragma unroll
        for (int i = 0; i < T; ++i) b0[i].load(wrow[i] + (int64_t)wave * BPB, g);
#pragma unroll
        for (int s = 0; s < kStages - 1; ++s) load_stage(raw[s], s);
        write_stage(raw[0], 0);
        for (int bi = 0;;) {
            do_block(b0, b1, bi, std::integral_constant<int, 0>{});
            if (++bi >= my_blocks) {
                kq_mfma_drain();
                break;
            }
            do_block(b1, b0, bi, std::integral_constant<int, 4>{});
            if (++bi >= my_blocks) {
                kq_mfma_drain();
                break;
            }
        }
    }
    // ---- sum the four waves' partial tiles in wave order and store
#pragma unroll
    for (int i = 0; i < T; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) red[(wave * T * MT + i * MT + mt) * 64 + lane] = acc[i][mt];
    __syncthreads();
    const int y_dtype = A->y_dtype;
    for (int f = (int)threadIdx.x; f < T * MT * 64; f += 64 * kMmWaves) {
        floatx4 s = red[f];
#pragma unroll
        for (int w2 = 1; w2 < kMmWaves; ++w2) s += red[w2 * T * MT * 64 + f];
        const int fl = f & 63, im = f >> 6, i = im / MT, mt = im - i * MT;
        const int n = (tile0 + i) * 16 + (fl & 15);
        if (n < N) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = 16 * mt + 4 * (fl >> 4) + e;
                if (m < M) kq_store_out(y, y_dtype, (int64_t)m * y_stride + n, A->x_exp ? ldexpf(s[e], A->x_exp[m]) : s[e]);
            }
        }
    }
    __syncthreads();  // the next group writes its partials over these
}

// SET: kSetQ4K / kSetQ6K (one codec) or kSetMix (Q4_K and Q6_K problems).
// MT: 16-row activation tiles (2: M <= 32, 4: M <= 64).  XT: 0 fp16, 1 bf16.
// T: weight tiles per group.
template <int SET, int MT, int XT, int T>
__global__ __launch_bounds__(64 * kMmWaves) __attribute__((amdgpu_waves_per_eu(1, 1))) void kq_mm_kernel(MmArgs a_) {
    __shared__ floatx4 red[kMmWaves * T * MT * 64];
    __shared__ u32x4 xstage[kMmWaves * 2 * 16 * MT * 8];  // two activation stages per wave
    const KArgs A = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
    const int total = A->total_groups, np = A->n_problems;
    for (int grp = (int)blockIdx.x; grp < total; grp += (int)gridDim.x) {  // uniform
        int pi = 0;
        for (int i = 1; i < np; ++i)
            if (grp >= A->group_begin[i]) pi = i;
        const uint8_t *w = A->p[pi].w;
        void *y = A->p[pi].y;
        const int64_t wrb = A->p[pi].w_row_bytes, ys = A->p[pi].y_stride;
        const int N = A->p[pi].N;
        const int tile0 = (grp - A->group_begin[pi]) * T;
        if constexpr (SET == kSetQ4K) {
            mm_group<KQ_CODEC_Q4_K, MT, XT, T>(A, w, wrb, y, ys, N, tile0, red, xstage);
        } else if constexpr (SET == kSetQ6K) {
            mm_group<KQ_CODEC_Q6_K, MT, XT, T>(A, w, wrb, y, ys, N, tile0, red, xstage);
        } else {
            if (A->p[pi].codec == KQ_CODEC_Q6_K) mm_group<KQ_CODEC_Q6_K, MT, XT, T>(A, w, wrb, y, ys, N, tile0, red, xstage);
            else mm_group<KQ_CODEC_Q4_K, MT, XT, T>(A, w, wrb, y, ys, N, tile0, red, xstage);
        }
    }
}

template <int SET, int MT, int XT, int T>
int mm_launch_one(const MmArgs &a, int grid, hipStream_t s) {
    hipLaunchKernelGGL((kq_mm_kernel<SET, MT, XT, T>), dim3(grid), dim3(64 * kMmWaves), 0, s, a);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

// Instantiated: Q4_K alone with T = 1..4 and 6 at two m-tiles, 1..3 at four
// (six spill there); Q6_K alone or mixed with T = 1..2 (a Q6_K super-block
// holds more registers per tile).
template <int SET, int MT, int XT>
int mm_launch_t(const MmArgs &a, int t, int grid, hipStream_t s) {
    if constexpr (SET == kSetQ4K) {
        switch (t) {
        case 1: return mm_launch_one<SET, MT, XT, 1>(a, grid, s);
        case 2: return mm_launch_one<SET, MT, XT, 2>(a, grid, s);
        case 3: return mm_launch_one<SET, MT, XT, 3>(a, grid, s);
        default:  // t is 4 or 6 here, and only at two m-tiles (the host caps four m-tiles at 3)
            if constexpr (MT == 2) {
                return t == 4 ? mm_launch_one<SET, MT, XT, 4>(a, grid, s) : mm_launch_one<SET, MT, XT, 6>(a, grid, s);
            } else {
                return KQ_ERR_BAD_SHAPE;
            }
        }
    } else {
        return t == 1 ? mm_launch_one<SET, MT, XT, 1>(a, grid, s) : mm_launch_one<SET, MT, XT, 2>(a, grid, s);
    }
}

template <int SET>
int mm_launch_set(const MmArgs &a, int mt, int t, int grid, hipStream_t s) {
    if (mt == 2) return mm_launch_t<SET, 2, 0>(a, t, grid, s);
    return mm_launch_t<SET, 4, 0>(a, t, grid, s);
}

int mm_env_int(const char *name, int dflt) {
    const char *s = getenv(name);
    if (!s || !*s) return dflt;
    char *end = nullptr;
    const long v = strtol(s, &end, 10);
    return (end && *end == 0 && v > 0 && v < (1 << 24)) ? (int)v : dflt;
}

}  // namespace

// Eligibility: problems validated and live, Q4_K / Q6_K only, fp16 or bf16
// activations shared by every problem (same x, stride, M, K), 17 <= M <= 64,
// x and its row stride 16-byte aligned, x addressable with 31-bit offsets.
bool kq_mm_eligible(const kq_matmul_problem *ps, int n, int x_dtype) {
    if (n <= 0) return false;
    if (x_dtype != KQ_DTYPE_F16) return false;
    const kq_matmul_problem &q0 = ps[0];
    if (q0.M < 17 || q0.M > 64) return false;
    // 16-byte activation pieces: x and its row stride 16-byte aligned
    if (((uintptr_t)q0.x & 15) != 0 || q0.x_row_stride % 8 != 0) return false;
    // activation reads are 32-bit buffer offsets (rows past M sit just past the end)
    if (((int64_t)(q0.M - 1) * q0.x_row_stride + 2 * (int64_t)q0.K) * 2 >= ((int64_t)1 << 31)) return false;
    for (int i = 0; i < n; ++i) {
        const kq_matmul_problem &q = ps[i];
        if (q.codec != KQ_CODEC_Q4_K && q.codec != KQ_CODEC_Q6_K) return false;
        if (q.x != q0.x || q.x_row_stride != q0.x_row_stride || q.M != q0.M || q.K != q0.K) return false;
    }
    return true;
}

// Problems eligible (kq_mm_eligible).  T (tiles per group) from the tiles per
// CU: as many tiles per group as one round of groups over the CUs needs, up
// to the register limit (Q4_K 6 at M <= 32, 3 above; any Q6_K 2); more tiles
// take several rounds of equal groups (GMLX_KQ_MM_T forces T; a T between the
// instantiated sizes takes the next larger one).
int kq_mm_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, hipStream_t s) {
    bool any4 = false, any6 = false;
    int tiles = 0;
    for (int i = 0; i < n; ++i) {
        any4 |= ps[i].codec == KQ_CODEC_Q4_K;
        any6 |= ps[i].codec == KQ_CODEC_Q6_K;
        tiles += (ps[i].N + 15) / 16;
    }
    const int set = any4 && any6 ? kSetMix : (any6 ? kSetQ6K : kSetQ4K);
    const int mt = ps[0].M <= 32 ? 2 : 4;
    const int tmax = set == kSetQ4K ? (mt == 2 ? 6 : 3) : 2;
    const int cus = device_cus();
    int t = (tiles + cus - 1) / cus;
    if (t > tmax) {
        const int rounds = (tiles + tmax * cus - 1) / (tmax * cus);
        t = (tiles + rounds * cus - 1) / (rounds * cus);
    }
    t = mm_env_int("GMLX_KQ_MM_T", t);
    if (t < 1) t = 1;
    if (t > tmax) t = tmax;
    if (t == 5) t = 6;  // instantiated sizes: the groups below use the kernel's own T

    MmArgs a;
    int groups = 0;
    for (int i = 0; i < n; ++i) {
        MmProblem &p = a.p[i];
        p.w = (const uint8_t *)ps[i].w;
        p.y = ps[i].y;
        p.w_row_bytes = ps[i].w_row_bytes;
        p.y_stride = ps[i].y_row_stride;
        p.N = ps[i].N;
        p.codec = ps[i].codec;
        a.group_begin[i] = groups;
        groups += ((ps[i].N + 15) / 16 + t - 1) / t;
    }
    for (int i = n; i < KQ_MAX_GROUP; ++i) {
        a.p[i] = a.p[0];
        a.group_begin[i] = 0x7FFFFFFF;
    }
    a.x = (const char *)ps[0].x;
    a.x_exp = x_exp;
    a.x_stride = ps[0].x_row_stride;
    a.M = ps[0].M;
    a.K = ps[0].K;
    a.y_dtype = y_dtype;
    a.total_groups = groups;
    a.n_problems = n;
    const int grid = groups < cus ? groups : cus;
    switch (set) {
    case kSetQ4K: return mm_launch_set<kSetQ4K>(a, mt, t, grid, s);
    case kSetQ6K: return mm_launch_set<kSetQ6K>(a, mt, t, grid, s);
    default: return mm_launch_set<kSetMix>(a, mt, t, grid, s);
    }
}
