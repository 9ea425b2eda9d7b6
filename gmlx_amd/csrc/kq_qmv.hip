// Persistent small-batch quantized matmul (M <= 16 activation rows).
//
// y[M, N] = x[M, K] . dequant(W[N, K])^T for problems that share x (the
// q|k|v and gate|up groups of one layer), one codec per launch.
//
// Decomposition: a workgroup has S waves, S = ceil(K / 1024); wave s owns the
// fixed k-step s (super-blocks 4s .. 4s+3) for the whole launch, so it loads
// its 32 activation fragments (16 rows x 1024 values, fp16) ONCE into
// registers.  The workgroup then walks 16-row weight tiles t = blockIdx.x,
// blockIdx.x + gridDim.x, ... ; for each tile every wave dequantizes its
// step's 4 blocks and runs 32 MFMAs, while the NEXT tile's blocks are already
// in flight (register double buffer).  The S partial tiles are summed through
// LDS in wave order (deterministic), and wave 0 stores the 16 x M outputs.
//
// Lane l = 16*g + r of a wave owns ONE super-block: weight row 16t + r,
// block 4s + g; its scales are decoded once per block.  An MFMA sums over the
// 4 lane groups, i.e. over 4 different blocks at once, which is valid because
// the fragments are fully dequantized (fp16) before the MFMA.
#include <stdlib.h>

#include "kq_mma.h"

namespace {

using namespace kqmma;

constexpr int kMaxSteps = 8;     // waves per workgroup (K <= 8192)
constexpr int kMaxProblems = KQ_MAX_GROUP;

// ---- lane-owns-block decoders ------------------------------------------------

template <int CODEC>
struct BlockL;

// Q4_K: 144 B, 16-B aligned.  Nibbles become exact fp16 integers through the
// fp8 (E4M3) converter: a byte q in [0, 15] read as E4M3 is q * 2^-9, and a
// scale of 2^9 (an exact power of two, which is all the converter applies)
// returns q.  Then w = fma(q, d*sc, -dmin*m) with one rounding.
template <>
struct BlockL<KQ_CODEC_Q4_K> {
    u32x4 raw[9];
    half2_t dsc[8], ndm[8];

    __device__ __forceinline__ void load(const uint8_t *blk) {
        const u32x4 *p = (const u32x4 *)blk;
#pragma unroll
        for (int i = 0; i < 9; ++i) raw[i] = p[i];
    }
    __device__ __forceinline__ void prep(bool valid) {
        const uint32_t h0 = raw[0].x;
        const float d = valid ? kq_f16_bits_to_f32(h0 & 0xFFFF) : 0.f;
        const float dmin = valid ? kq_f16_bits_to_f32(h0 >> 16) : 0.f;
        const uint32_t s0 = raw[0].y, s1 = raw[0].z, s2 = raw[0].w;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t sc, mn;
            if (j < 4) {
                sc = (s0 >> (8 * j)) & 63;
                mn = (s1 >> (8 * j)) & 63;
            } else {
                const uint32_t bj4 = (s2 >> (8 * (j - 4))) & 0xFF;   // s[j+4]
                const uint32_t bjm4 = (s0 >> (8 * (j - 4))) & 0xFF;  // s[j-4]
                const uint32_t bj = (s1 >> (8 * (j - 4))) & 0xFF;    // s[j]
                sc = (bj4 & 0xF) | ((bjm4 >> 6) << 4);
                mn = (bj4 >> 4) | ((bj >> 6) << 4);
            }
            dsc[j] = bcast((_Float16)(d * (float)sc));
            ndm[j] = bcast((_Float16)(-(dmin * (float)mn)));
        }
    }
    // values 8t .. 8t+7 of the block (t = 0..31)
    __device__ __forceinline__ half8_t frag(int t, const Iq2Tables &) const {
        const int sub = t >> 2, c = sub >> 1, j = t & 3;
        const uint32_t *qs = (const uint32_t *)&raw[1];
        uint32_t w0 = qs[8 * c + 2 * j], w1 = qs[8 * c + 2 * j + 1];
        if (sub & 1) {
            w0 >>= 4;
            w1 >>= 4;
        }
        w0 &= 0x0F0F0F0Fu;
        w1 &= 0x0F0F0F0Fu;
        const half2_t q0 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 512.f, false));
        const half2_t q1 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 512.f, true));
        const half2_t q2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 512.f, false));
        const half2_t q3 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 512.f, true));
        return cat8(__builtin_elementwise_fma(q0, dsc[sub], ndm[sub]), __builtin_elementwise_fma(q1, dsc[sub], ndm[sub]),
                    __builtin_elementwise_fma(q2, dsc[sub], ndm[sub]), __builtin_elementwise_fma(q3, dsc[sub], ndm[sub]));
    }
};

// Q6_K: 210 B, only 2-byte aligned.
template <>
struct BlockL<KQ_CODEC_Q6_K> {
    u32x4 raw[13];  // bytes 0..207
    uint32_t dbits;
    half2_t dsc[16];

    __device__ __forceinline__ void load(const uint8_t *blk) {
        const u32x4_a2 *p = (const u32x4_a2 *)blk;
#pragma unroll
        for (int i = 0; i < 13; ++i) {
            const u32x4_a2 v = p[i];
            raw[i] = u32x4{v.x, v.y, v.z, v.w};
        }
        dbits = (uint32_t)*(const uint16_t *)(blk + 208);
    }
    __device__ __forceinline__ void prep(bool valid) {
        const float d = valid ? kq_f16_bits_to_f32(dbits) : 0.f;
        const uint32_t *sw = (const uint32_t *)&raw[12];  // bytes 192..207
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int8_t sc = (int8_t)((sw[i >> 2] >> (8 * (i & 3))) & 0xFF);
            dsc[i] = bcast((_Float16)(d * (float)sc));
        }
    }
    __device__ __forceinline__ half8_t frag(int t, const Iq2Tables &) const {
        const int h = t >> 4, quarter = (t >> 2) & 3, j = t & 3;
        const uint32_t *ql = (const uint32_t *)&raw[0];  // 32 dwords
        const uint32_t *qh = (const uint32_t *)&raw[8];  // 16 dwords
        uint32_t l0 = ql[16 * h + 8 * (quarter & 1) + 2 * j];
        uint32_t l1 = ql[16 * h + 8 * (quarter & 1) + 2 * j + 1];
        const uint32_t q0 = qh[8 * h + 2 * j], q1 = qh[8 * h + 2 * j + 1];
        if (quarter >= 2) {
            l0 >>= 4;
            l1 >>= 4;
        }
        const int hs = 2 * quarter;
        uint32_t c0, c1;
        if (hs <= 4) {
            c0 = (l0 & 0x0F0F0F0Fu) | ((q0 << (4 - hs)) & 0x30303030u);
            c1 = (l1 & 0x0F0F0F0Fu) | ((q1 << (4 - hs)) & 0x30303030u);
        } else {
            c0 = (l0 & 0x0F0F0F0Fu) | ((q0 >> (hs - 4)) & 0x30303030u);
            c1 = (l1 & 0x0F0F0F0Fu) | ((q1 >> (hs - 4)) & 0x30303030u);
        }
        const Bias8 b(c0, c1);
        const half2_t k1056 = {(_Float16)1056.f, (_Float16)1056.f};
        const half2_t s = dsc[t >> 1];
        return cat8((b.p0 - k1056) * s, (b.p1 - k1056) * s, (b.p2 - k1056) * s, (b.p3 - k1056) * s);
    }
};

// IQ2_XXS: 66 B; grid / sign tables in LDS.
template <>
struct BlockL<KQ_CODEC_IQ2_XXS> {
    u32x4 raw[4];  // bytes 2..65 (the 8 groups)
    uint32_t dbits;
    half2_t db[8];

    __device__ __forceinline__ void load(const uint8_t *blk) {
        const u32x4_a2 *p = (const u32x4_a2 *)(blk + 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4_a2 v = p[i];
            raw[i] = u32x4{v.x, v.y, v.z, v.w};
        }
        dbits = (uint32_t)*(const uint16_t *)blk;
    }
    __device__ __forceinline__ void prep(bool valid) {
        const float d = valid ? kq_f16_bits_to_f32(dbits) : 0.f;
        const uint32_t *g = (const uint32_t *)&raw[0];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float v = d * (0.5f + (float)(g[2 * i + 1] >> 28)) * 0.25f;
            db[i] = bcast((_Float16)v);
        }
    }
    __device__ __forceinline__ half8_t frag(int t, const Iq2Tables &tab) const {
        const int grp = t >> 2, l = t & 3;
        const uint32_t *g = (const uint32_t *)&raw[0];
        const uint32_t idx = (g[2 * grp] >> (8 * l)) & 0xFF;
        const uint32_t s7 = (g[2 * grp + 1] >> (7 * l)) & 127u;
        const u32x4 gm = *(const u32x4 *)tab.grid_h2[idx];
        const u32x4 sm = *(const u32x4 *)tab.sign_x2[s7];
        const half2_t s = db[grp];
        return cat8(h2b(gm.x ^ sm.x) * s, h2b(gm.y ^ sm.y) * s, h2b(gm.z ^ sm.z) * s, h2b(gm.w ^ sm.w) * s);
    }
};

// ---- kernel ---------------------------------------------------------------------

struct QmvProblem {
    const uint8_t *w;
    void *y;
    int64_t w_row_bytes, y_stride;
    int32_t N, tile_begin;
};

struct QmvArgs {
    QmvProblem p[kMaxProblems];
    const char *x;
    const int32_t *x_exp;  // per-row exponents of prepared activations (results * 2^e), or null
    int64_t x_stride;  // elements
    int32_t n_problems, M, K, y_dtype, total_tiles;
};

template <int CODEC>
__device__ __forceinline__ const uint8_t *tile_block(const QmvArgs &a, int tile, int r, int kb, QmvProblem &p) {
    p = a.p[0];
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
        if (i < a.n_problems && tile >= a.p[i].tile_begin) p = a.p[i];
    const int n = min((tile - p.tile_begin) * 16 + r, p.N - 1);
    return p.w + (int64_t)n * p.w_row_bytes + (int64_t)kb * kq_block_bytes(CODEC);
}

template <int CODEC, int XT>
__device__ __forceinline__ void tile_mma(const BlockL<CODEC> &b, const half8_t (&xa)[32], floatx4 &acc,
                                         const Iq2Tables &tab) {
    acc = floatx4{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 32; ++t) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[t], b.frag(t, tab), acc, 0, 0, 0);
    kq_mfma_drain();
}

// Q6_K's two 210-B blocks do not fit beside the activations at two waves per
// SIMD: its launches are limited to 4 waves (K <= 4096), one wave per SIMD.
template <int CODEC>
constexpr int max_waves() { return CODEC == KQ_CODEC_Q6_K ? 4 : kMaxSteps; }

template <int CODEC, int XT>
__global__ __launch_bounds__(64 * max_waves<CODEC>()) void kq_qmv_persistent_kernel(QmvArgs a) {
    __shared__ floatx4 red[2][kMaxSteps - 1][64];
    __shared__ Iq2Tables iq2_tab;
    if constexpr (CODEC == KQ_CODEC_IQ2_XXS) load_iq2_tables(iq2_tab);
    const int S = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6;
    const int lane = kq_lane();
    const int r = lane & 15, g = lane >> 4;
    const int nb = a.K / KQ_QK;
    const int kb = 4 * wave + g;
    const bool kvalid = kb < nb;
    const int kb_c = kvalid ? kb : nb - 1;
    int tile = blockIdx.x;
    if (tile >= a.total_tiles) return;  // uniform over the workgroup

    // this wave's activation fragments: row r (zeros for r >= M, no memory
    // access), block kb_c, values 8t..8t+7
    half8_t xa[32];
    {
        const XRowsBuf<1> xr = x_rows_buf<1, XT>(a.x, a.x_stride, a.M, a.K, 0, r);
#pragma unroll
        for (int t = 0; t < 32; ++t) xa[t] = xr.template load<XT>(0, kb_c * KQ_QK + 8 * t);
    }
    QmvProblem pc, pn;
    BlockL<CODEC> b0, b1;
    b0.load(tile_block<CODEC>(a, tile, r, kb_c, pc));
    int it = 0;
    for (;;) {
        // ---- even half: compute b0 while b1 loads
        // unconditional prefetch (the last one re-reads the current tile): a
        // load under a branch makes the compiler wait for it before the math
        int tn = tile + gridDim.x;
        bool more = tn < a.total_tiles;
        b1.load(tile_block<CODEC>(a, more ? tn : tile, r, kb_c, pn));
        __builtin_amdgcn_sched_barrier(0);
        floatx4 acc;
        b0.prep(kvalid);
        tile_mma<CODEC, XT>(b0, xa, acc, iq2_tab);
        // ---- reduce the S partial tiles in wave order
        if (wave > 0) red[it & 1][wave - 1][lane] = acc;
        __syncthreads();
        if (wave == 0) {
            for (int w = 0; w < S - 1; ++w) acc += red[it & 1][w][lane];
            const int n = (tile - pc.tile_begin) * 16 + r;
            if (n < pc.N) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = 4 * g + e;
                    if (m < a.M)
                        kq_store_out(pc.y, a.y_dtype, (int64_t)m * pc.y_stride + n,
                                     a.x_exp ? ldexpf(acc[e], a.x_exp[m]) : acc[e]);
                }
            }
        }
        ++it;
        if (!more) break;
        tile = tn;
        pc = pn;
        // ---- odd half: compute b1 while b0 loads
        tn = tile + gridDim.x;
        more = tn < a.total_tiles;
        b0.load(tile_block<CODEC>(a, more ? tn : tile, r, kb_c, pn));
        __builtin_amdgcn_sched_barrier(0);
        b1.prep(kvalid);
        tile_mma<CODEC, XT>(b1, xa, acc, iq2_tab);
        if (wave > 0) red[it & 1][wave - 1][lane] = acc;
        __syncthreads();
        if (wave == 0) {
            for (int w = 0; w < S - 1; ++w) acc += red[it & 1][w][lane];
            const int n = (tile - pc.tile_begin) * 16 + r;
            if (n < pc.N) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = 4 * g + e;
                    if (m < a.M)
                        kq_store_out(pc.y, a.y_dtype, (int64_t)m * pc.y_stride + n,
                                     a.x_exp ? ldexpf(acc[e], a.x_exp[m]) : acc[e]);
                }
            }
        }
        ++it;
        if (!more) break;
        tile = tn;
        pc = pn;
    }
}

int env_int(const char *name, int dflt) {
    const char *s = getenv(name);
    if (!s || !*s) return dflt;
    char *end = nullptr;
    const long v = strtol(s, &end, 10);
    return (end && *end == 0 && v > 0 && v < (1 << 24)) ? (int)v : dflt;
}

template <int CODEC>
void launch_codec(const QmvArgs &a, int S, int grid, hipStream_t s) {
    hipLaunchKernelGGL((kq_qmv_persistent_kernel<CODEC, 0>), dim3(grid), dim3(64 * S), 0, s, a);
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

int kq_qmv_persistent_grid(const kq_matmul_problem &q) {
    const int S = (q.K / KQ_QK + 3) / 4;
    // waves per CU the register budget allows: 8 (4 for Q6_K)
    const int waves_cu = q.codec == KQ_CODEC_Q6_K ? 4 : 8;
    const int per_cu = S >= waves_cu ? 1 : waves_cu / S;
    return env_int("GMLX_KQ_QMV_WGS", device_cus() * per_cu);
}

// Internal entry used by kq_quantized_matmul_grouped: problems already
// validated, all live, sharing x / x_row_stride / M / K / codec, M <= 16,
// K <= 8192 (K <= 4096 for Q6_K).  Returns KQ_OK or KQ_ERR_LAUNCH_FAILED.
int kq_qmv_persistent_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, hipStream_t s) {
    QmvArgs a;
    int tiles = 0;
    for (int i = 0; i < n; ++i) {
        QmvProblem &p = a.p[i];
        p.w = (const uint8_t *)ps[i].w;
        p.y = ps[i].y;
        p.w_row_bytes = ps[i].w_row_bytes;
        p.y_stride = ps[i].y_row_stride;
        p.N = ps[i].N;
        p.tile_begin = tiles;
        tiles += (ps[i].N + 15) / 16;
    }
    for (int i = n; i < kMaxProblems; ++i) a.p[i] = a.p[0];
    a.x = (const char *)ps[0].x;
    a.x_exp = x_exp;
    a.x_stride = ps[0].x_row_stride;
    a.n_problems = n;
    a.M = ps[0].M;
    a.K = ps[0].K;
    a.y_dtype = y_dtype;
    a.total_tiles = tiles;
    const int S = (ps[0].K / KQ_QK + 3) / 4;
    int grid = kq_qmv_persistent_grid(ps[0]);
    if (grid > tiles) grid = tiles;
    switch (ps[0].codec) {
    case KQ_CODEC_Q4_K: launch_codec<KQ_CODEC_Q4_K>(a, S, grid, s); break;
    case KQ_CODEC_Q6_K: launch_codec<KQ_CODEC_Q6_K>(a, S, grid, s); break;
    default: launch_codec<KQ_CODEC_IQ2_XXS>(a, S, grid, s); break;
    }
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}
