// Small-batch dequant-fused matmul (M <= 16 activation rows) for problems that
// share their activations (the q|k, o, gate|up calls of a decode step).
//
// y[M, N] = x[M, K] . dequant(W[N, K])^T
//
// One persistent workgroup of 16 waves per CU.  The workgroup first copies x
// into LDS with coalesced direct-to-LDS loads (1 KB per instruction, rows
// padded by 16 bytes so that the 16 rows of an MFMA operand fall in different
// LDS banks), so activations cost the memory pipeline one pass per workgroup
// instead of one pass per weight tile.  It then walks 16-row weight tiles
// t = blockIdx.x, blockIdx.x + gridDim.x, ...; wave w dequantizes super-blocks
// w, w + 16, ... of the tile, reads the matching activation fragments from
// LDS and runs v_mfma_f32_16x16x32_f16.  A wave always works on the same
// super-blocks, so when x does not fit in LDS (K = 12288 at M = 5..8) the
// last 4096 columns stay in registers instead (XR): each wave loads its
// fragments of them once.  Lanes of rows M..15 read row M - 1: they feed only
// output rows that are never stored.  Each wave keeps a register ring of
// DEPTH tiles, so DEPTH - 1 tiles are in flight while one is multiplied (the
// host picks DEPTH from the tiles per workgroup: a ring deeper than the work
// only adds dead requests to the first wait).
//
// The weights are read with buffer loads whose range is the problem's matrix:
// rows past N and the ring's requests past the workgroup's last tile use an
// offset outside the range, which reads zeros without a memory access.  So
// every ring step issues the same loads and stores with no branch around
// them, and the compiler's wait counts follow the ring exactly.  The 16
// partial tiles are summed through LDS in wave order (each wave sums and
// stores one sixteenth of the tile, again with out-of-range offsets for the
// lanes that store nothing), so results are deterministic.
//
// Lane views (lane l = 16g + r feeds weight row r):
//   Q4_K, IQ2_XXS : lane group g owns the quarter 64g .. 64g+63 of a block;
//                   MFMA step t covers values 64g + 8t .. +7.
//   Q6_K          : lane group g owns half h = g/2 of the block and the
//                   positions l = 16(g%2) .. +15 of its four 32-value runs;
//                   step t covers run t/2, positions 16(g%2) + 8(t%2) .. +7.
#include <stdlib.h>

#include "kq_mma.h"

int device_cus();

namespace {

using namespace kqmma;

constexpr int kWaves = 16;             // waves per CU (one 16-wave or two 8-wave workgroups)
constexpr int kLdsBytes = 160 * 1024;  // LDS of one CU
constexpr uint32_t kOut = 0x80000000u; // buffer offset past every range (reads 0, writes dropped)
#define LDSP(T) __attribute__((address_space(3))) T *

struct MvProblem {
    const uint8_t *w;
    void *y;
    int64_t y_stride;        // elements
    uint32_t w_bytes;        // N * row_bytes (< 2^31)
    uint32_t row_bytes;
    uint32_t y_bytes;        // ((M - 1) * y_stride + N) * element size (< 2^31)
    int32_t N;
    int32_t codec;           // KQ_CODEC_*
};

struct MvArgs {
    int32_t tile_begin[KQ_MAX_GROUP];  // first tile of each problem; unused: INT_MAX
    MvProblem p[KQ_MAX_GROUP];
    const char *x;
    const int32_t *x_exp;              // per-row exponents of prepared activations (results * 2^e), or null
    int64_t x_stride;                  // elements
    int32_t M, K, y_dtype, total_tiles;
    int32_t n_problems;
    int32_t kl;                        // columns of x staged in LDS (K, or K - 4096 with XR)
    int32_t xrow;                      // LDS bytes per staged activation row (2 kl + 16)
    int32_t red_off, red_bufs;         // reduction area: byte offset in LDS, 1 or 2 buffers
};

// Kernel arguments read in place through the constant address space, so the
// compiler may keep them in scalar registers across the loop.
typedef const __attribute__((address_space(4))) MvArgs *KArgs;


__device__ __forceinline__ u32x4 ld128(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
}

// ---- lane views ----------------------------------------------------------------

template <int CODEC>
struct WB;

// Q4_K quarter view: header (d, dmin, scales) + qs bytes 32g .. 32g+31.
// Sub-block 2g in the low nibbles, 2g+1 in the high nibbles.  Scales and mins
// are unpacked as bytes four at a time (sub-blocks 0..3 and 4..7), the lane's
// two are picked with a lane-constant mask and become exact fp16 integers
// through the 1024-bias.  Nibble bytes become exact fp16 integers through the
// fp8 converter (q <= 15 read as E4M3 is q * 2^-9, scale 2^9), and the
// fragment is q * sc, exact.  The block's chain is folded with d in fp32 and
// the minimum term comes from the wave's activation sub-block sums xs
// (sub-blocks 2g, 2g + 1 of the lane's row) on the fp32 MFMA.
template <>
struct WB<KQ_CODEC_Q4_K> {
    u32x4 hdr, q0, q1;
    __device__ static constexpr int x_elem(int t, int g) { return 64 * g + 8 * t; }
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t off, int g, bool) {
        hdr = ld128(rs, off);
        q0 = ld128(rs, off + 16 + 32 * g);
        q1 = ld128(rs, off + 32 + 32 * g);
    }
    template <class XF>
    __device__ __forceinline__ void mma(floatx4 &acc, const XF &xf, int g, const Iq2Tables &, bool,
                                        const float (&xs)[2]) const {
        const uint32_t hmask = g >= 2 ? 0xFFFFFFFFu : 0u;
        const uint32_t ssel = (g & 1) ? KQ_SEL_B23 : KQ_SEL_B01;
        const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
        const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
        const uint32_t m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
        const uint32_t scb = (sc_hi & hmask) | (s0 & 0x3F3F3F3Fu & ~hmask);
        const uint32_t mb = (m_hi & hmask) | (s1 & 0x3F3F3F3Fu & ~hmask);
        const half2_t k1024 = {(_Float16)1024.f, (_Float16)1024.f};
        const half2_t sc = h2b(__builtin_amdgcn_perm(0x64646464u, scb, ssel)) - k1024;
        const half2_t mh = h2b(__builtin_amdgcn_perm(0x64646464u, mb, ssel)) - k1024;
        const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        floatx4 P;
#pragma unroll
        for (int tp = 0; tp < 4; ++tp) {
            const uint32_t lo0 = qw[2 * tp] & 0x0F0F0F0Fu, lo1 = qw[2 * tp + 1] & 0x0F0F0F0Fu;
            const uint32_t hi0 = (qw[2 * tp] >> 4) & 0x0F0F0F0Fu, hi1 = (qw[2 * tp + 1] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t w0 = e ? hi0 : lo0, w1 = e ? hi1 : lo1;
                const half2_t s = bcast(e ? sc.y : sc.x);
                const half2_t a0 = h2b(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 512.f, false)));
                const half2_t a1 = h2b(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 512.f, true)));
                const half2_t a2 = h2b(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 512.f, false)));
                const half2_t a3 = h2b(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 512.f, true)));
                const half8_t bf = cat8(a0 * s, a1 * s, a2 * s, a3 * s);
                P = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf(4 * e + tp, x_elem(4 * e + tp, g)), bf,
                                                           tp == 0 && e == 0 ? fzero4() : P, 0, 0, 0);
            }
        }
        const float dmin = kq_f16_bits_to_f32(hdr.x >> 16);
        acc = fold4(kq_f16_bits_to_f32(hdr.x & 0xFFFFu), P, acc);
        acc = min_accumulate(xs[0], xs[1], -dmin * (float)mh.x, -dmin * (float)mh.y, acc);
    }
};

// Q6_K half view (210 B: ql[128], qh[64], scales[16], d).  Lane group g:
// h = g / 2, c = g % 2.  Value 128h + 32q + l (l = 16c .. 16c+15) is
// (ql[64h + 32(q%2) + l] nibble q/2) | (qh[32h + l] bits 2q, 2q+1) << 4,
// minus 32, times scales[8h + 2q + c] (the fragment, an integer), times d in
// fp32 after the chain.  Loads: the two ql runs and the qh run of the lane
// (16 B each), the 16 scales and d.
template <>
struct WB<KQ_CODEC_Q6_K> {
    u32x4 qa, qb, qh, sc;
    uint32_t dbits;
    __device__ static constexpr int x_elem(int t, int g) {
        return 128 * (g >> 1) + 32 * (t >> 1) + 16 * (g & 1) + 8 * (t & 1);
    }
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t off, int g, bool) {
        const uint32_t h = (uint32_t)(g >> 1), c = (uint32_t)(g & 1);
        qa = ld128(rs, off + 64 * h + 16 * c);
        qb = ld128(rs, off + 64 * h + 32 + 16 * c);
        qh = ld128(rs, off + 128 + 32 * h + 16 * c);
        sc = ld128(rs, off + 192);
        dbits = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off + 208, 0, 0);
    }
    template <class XF>
    __device__ __forceinline__ void mma(floatx4 &acc, const XF &xf, int g, const Iq2Tables &, bool = false,
                                        const float (&)[2] = {}) const {
        // scales 8h + 2q + c: q = 0, 1 in word 2h, q = 2, 3 in word 2h + 1, byte 2(q%2) + c
        const uint32_t sw0 = g >= 2 ? sc.z : sc.x, sw1 = g >= 2 ? sc.w : sc.y;
        const uint32_t cs = 8u * (uint32_t)(g & 1);
        half2_t isc[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t w = q < 2 ? sw0 : sw1;
            const int s = __builtin_amdgcn_sbfe((int)w, (int)(16u * (q & 1) + cs), 8);
            isc[q] = bcast((_Float16)(float)s);
        }
        const half2_t k1056 = {(_Float16)1056.f, (_Float16)1056.f};
        floatx4 P;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int q = t >> 1, sub = t & 1;
            const u32x4 &lq = (q & 1) ? qb : qa;
            uint32_t l0 = sub ? lq.z : lq.x, l1 = sub ? lq.w : lq.y;
            if (q >= 2) {
                l0 >>= 4;
                l1 >>= 4;
            }
            const uint32_t h0 = sub ? qh.z : qh.x, h1 = sub ? qh.w : qh.y;
            uint32_t c0, c1;
            if (q <= 2) {
                c0 = (l0 & 0x0F0F0F0Fu) | ((h0 << (4 - 2 * q)) & 0x30303030u);
                c1 = (l1 & 0x0F0F0F0Fu) | ((h1 << (4 - 2 * q)) & 0x30303030u);
            } else {
                c0 = (l0 & 0x0F0F0F0Fu) | ((h0 >> 2) & 0x30303030u);
                c1 = (l1 & 0x0F0F0F0Fu) | ((h1 >> 2) & 0x30303030u);
            }
            const Bias8 b(c0, c1);
            const half2_t s = isc[q];
            const half8_t bf = cat8((b.p0 - k1056) * s, (b.p1 - k1056) * s, (b.p2 - k1056) * s, (b.p3 - k1056) * s);
            P = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf(t, x_elem(t, g)), bf, t == 0 ? fzero4() : P, 0, 0, 0);
        }
        acc = fold4(kq_f16_bits_to_f32(dbits), P, acc);
    }
};

// IQ2_XXS quarter view: groups 2g, 2g+1 (bytes 2 + 16g .. +15) and d; grid and
// sign tables from LDS.  Fragment (2s + 1) * grid * sign (an integer), times
// d / 8 in fp32 after the chain.
template <>
struct WB<KQ_CODEC_IQ2_XXS> {
    u32x4 raw;
    uint32_t dbits;
    __device__ static constexpr int x_elem(int t, int g) { return 64 * g + 8 * t; }
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t off, int g, bool) {
        raw = ld128(rs, off + 2 + 16 * g);
        dbits = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
    }
    template <class XF>
    __device__ __forceinline__ void mma(floatx4 &acc, const XF &xf, int g, const Iq2Tables &tab, bool = false,
                                        const float (&)[2] = {}) const {
        (void)g;
        const half2_t os0 = bcast((_Float16)(float)(2u * (raw.y >> 28) + 1u));
        const half2_t os1 = bcast((_Float16)(float)(2u * (raw.w >> 28) + 1u));
        floatx4 P;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int e = t >> 2, l = t & 3;
            const uint32_t gw = e ? raw.z : raw.x, aux = e ? raw.w : raw.y;
            const uint32_t idx = (gw >> (8 * l)) & 0xFF;
            const uint32_t s7 = (aux >> (7 * l)) & 127u;
            const u32x4 gm = *(const u32x4 *)tab.grid_h2[idx];
            const u32x4 sm = *(const u32x4 *)tab.sign_x2[s7];
            const half2_t s = e ? os1 : os0;
            const half8_t bf =
                cat8(h2b(gm.x ^ sm.x) * s, h2b(gm.y ^ sm.y) * s, h2b(gm.z ^ sm.z) * s, h2b(gm.w ^ sm.w) * s);
            P = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf(t, x_elem(t, g)), bf, t == 0 ? fzero4() : P, 0, 0, 0);
        }
        acc = fold4(kq_f16_bits_to_f32(dbits) * 0.125f, P, acc);
    }
};

// Q4_K and Q6_K problems in one launch (the q|k and v of a Q4_K_M layer).
// Every ring slot issues the loads of the Q6_K view (four 16-B runs and d);
// a Q4_K tile fills the first three with the Q4_K view and sends the other
// two out of range, so both codecs issue the same instructions and the wait
// counts do not depend on the tile.  The tile's codec (uniform over the
// workgroup) picks the dequantization.
constexpr int KQ_MIX = 0x7F;

template <>
struct WB<KQ_MIX> {
    u32x4 v0, v1, v2, v3;
    uint32_t dbits;
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t off, int g, bool q6) {
        const uint32_t h = (uint32_t)(g >> 1), c = (uint32_t)(g & 1);
        const bool dead = off >= kOut;
        v0 = ld128(rs, q6 ? off + 64 * h + 16 * c : off);
        v1 = ld128(rs, q6 ? off + 64 * h + 32 + 16 * c : off + 16 + 32 * g);
        v2 = ld128(rs, q6 ? off + 128 + 32 * h + 16 * c : off + 32 + 32 * g);
        v3 = ld128(rs, q6 && !dead ? off + 192 : kOut);
        dbits = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, q6 && !dead ? off + 208 : kOut, 0, 0);
    }
    template <class XF>
    __device__ __forceinline__ void mma(floatx4 &acc, const XF &xf, int g, const Iq2Tables &tab, bool q6,
                                        const float (&xs)[2]) const {
        if (q6) {
            WB<KQ_CODEC_Q6_K> b;
            b.qa = v0;
            b.qb = v1;
            b.qh = v2;
            b.sc = v3;
            b.dbits = dbits;
            b.mma(acc, xf, g, tab, true, xs);
        } else {
            WB<KQ_CODEC_Q4_K> b;
            b.hdr = v0;
            b.q0 = v1;
            b.q1 = v2;
            b.mma(acc, xf, g, tab, false, xs);
        }
    }
};

// IQ2_XXS kernels keep the fp16 grid / sign tables in LDS; other codecs
// allocate nothing.
template <int CODEC>
struct Tables {
    __device__ static const Iq2Tables *get() { return nullptr; }
};
template <>
struct Tables<KQ_CODEC_IQ2_XXS> {
    __device__ static const Iq2Tables *get() {
        __shared__ Iq2Tables t;
        load_iq2_tables(t);
        return &t;
    }
};

// ---- kernel ---------------------------------------------------------------------

// WV: waves per workgroup (16: one workgroup per CU; 8: two, which are not
// phase-locked by each other's per-tile barrier).  NBW: blocks per wave per
// tile (K <= 256 * WV * NBW).  XT: 0 fp16, 1 bf16.  DEPTH: register ring
// depth in tiles.  XR: block NBW - 1 of every wave takes its activations
// from registers.
template <int CODEC, int XT, int NBW, int DEPTH, bool XR, int WV>
__global__ __launch_bounds__(64 * WV) __attribute__((amdgpu_waves_per_eu(4))) void kq_mv_kernel(MvArgs a_) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const KArgs A = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
    const Iq2Tables *tab = Tables<CODEC>::get();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = kq_lane(), r = lane & 15, g = lane >> 4;
    const int G = (int)gridDim.x, B0 = (int)blockIdx.x;
    const int my_tiles = (A->total_tiles - B0 + G - 1) / G;
    if (my_tiles <= 0) return;  // uniform over the workgroup
    const int M = A->M, K = A->K, nb = K / KQ_QK;
    const int xrow = A->xrow;

    // ---- stage columns [0, kl) of x rows [0, M) into LDS (1 KB per
    //      instruction, row m at m * xrow)
    {
        const int rowb = 2 * A->kl, segs = (rowb + 1023) >> 10;
        const int total = M * segs;
        for (int i = wave; i < total; i += WV) {
            const int m = i / segs, sg = i - m * segs;
            const int off = sg * 1024 + lane * 16;
            if (off < rowb)
                __builtin_amdgcn_global_load_lds(A->x + (int64_t)m * A->x_stride * 2 + off,
                                                 (LDSP(void))(smem + m * xrow + sg * 1024), 16, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // the copies go first (see the wait below)
    // ---- XR: this wave's fragments of block wave + WV * (NBW - 1) (rows >= M read zeros)
    half8_t xreg[XR ? 8 : 1];
    if constexpr (XR) {
        const XRowsBuf<1> xb = x_rows_buf<1, XT>(A->x, A->x_stride, M, K, 0, r);
        const int kb = wave + WV * (NBW - 1);
#pragma unroll
        for (int t = 0; t < 8; ++t)
            xreg[t] = xb.template load<XT>(0, min(kb, nb - 1) * KQ_QK + WB<CODEC>::x_elem(t, g));
    }

    // ---- ring step k: tile B0 + k * G, this wave's blocks kb = wave + WV * i
    // Tiles are walked in increasing order, so the problem of the next tile is
    // found by advancing a cursor from the previous one, and the fields a step
    // needs stay in scalar registers, reloaded only when the cursor moves (at
    // most once per problem).  The load side (tile k + DEPTH - 1) and the
    // multiply/store side (tile k) keep a cursor each.
    struct LoadCursor {
        int pi, begin, next;  // problem, its first tile, the next problem's first tile
        const uint8_t *w;
        uint32_t w_bytes, row_bytes;
        int codec;
    };
    struct StoreCursor {
        int pi, begin, next;
        void *y;
        int64_t y_stride;
        uint32_t y_bytes;
        int N, codec;
    };
    auto next_begin = [&](int pi) { return pi + 1 < A->n_problems ? A->tile_begin[pi + 1] : 0x7FFFFFFF; };
    LoadCursor lc{0, 0, next_begin(0), A->p[0].w, A->p[0].w_bytes, A->p[0].row_bytes, A->p[0].codec};
    StoreCursor sc{0, 0, next_begin(0), A->p[0].y, A->p[0].y_stride, A->p[0].y_bytes, A->p[0].N, A->p[0].codec};
    auto load_at = [&](int tile) {
        while (tile >= lc.next) {  // uniform over the workgroup
            ++lc.pi;
            lc.begin = lc.next;
            lc.next = next_begin(lc.pi);
            lc.w = A->p[lc.pi].w;
            lc.w_bytes = A->p[lc.pi].w_bytes;
            lc.row_bytes = A->p[lc.pi].row_bytes;
            lc.codec = A->p[lc.pi].codec;
        }
    };
    auto store_at = [&](int tile) {
        while (tile >= sc.next) {
            ++sc.pi;
            sc.begin = sc.next;
            sc.next = next_begin(sc.pi);
            sc.y = A->p[sc.pi].y;
            sc.y_stride = A->p[sc.pi].y_stride;
            sc.y_bytes = A->p[sc.pi].y_bytes;
            sc.N = A->p[sc.pi].N;
            sc.codec = A->p[sc.pi].codec;
        }
    };
    auto load_tile = [&](WB<CODEC> (&b)[NBW], int k) {
        const bool live = k < my_tiles;
        const int tile = B0 + min(k, my_tiles - 1) * G;
        load_at(tile);
        const int row0 = (tile - lc.begin) * 16;
        const __amdgpu_buffer_rsrc_t rs = kq_buffer(lc.w, lc.w_bytes);
        const bool q6 = CODEC == KQ_MIX && lc.codec == KQ_CODEC_Q6_K;
        const uint32_t bpb = CODEC == KQ_MIX ? (q6 ? 210u : 144u) : (uint32_t)kq_block_bytes(CODEC);
        // rows past N fall outside the range; so does every row of a dead step
        const uint32_t base = live ? (uint32_t)(row0 + r) * lc.row_bytes : kOut;
#pragma unroll
        for (int i = 0; i < NBW; ++i) {
            const int kb = wave + WV * i;  // past nb: out of range too
            b[i].load(rs, kb < nb ? base + (uint32_t)kb * bpb : kOut, g, q6);
        }
    };

    float *red = (float *)(smem + A->red_off);  // [bufs][WV][64 lanes][4]
    const int bufs = A->red_bufs;
    const uint32_t xr_base = (uint32_t)(uintptr_t)(LDSP(const void))(smem + min(r, M - 1) * xrow);
    // reduction slice of this wave: source lane SL * wave + lane / 4, element
    // lane % 4 (SL = 64 / WV; lanes 4 * SL .. 63 store nothing)
    constexpr int SL = 64 / WV;
    const int src_lane = SL * wave + ((lane >> 2) & (SL - 1)), src_e = lane & 3;
    const int out_n = src_lane & 15, out_m = 4 * (src_lane >> 4) + src_e;
    const bool out_lane = lane < 4 * SL && out_m < M;

    const bool y_f32 = A->y_dtype == KQ_DTYPE_F32, y_bf16 = A->y_dtype == KQ_DTYPE_BF16;
    // Q4_K: activation sub-block sums of the wave's blocks (filled below, once x is in LDS)
    [[maybe_unused]] float xsum[NBW][2] = {};
    auto compute_tile = [&](WB<CODEC> (&b)[NBW], int k) {
        const int tile = B0 + k * G;
        store_at(tile);
        const bool q6 = CODEC == KQ_MIX && sc.codec == KQ_CODEC_Q6_K;
        floatx4 acc = floatx4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < NBW; ++i) {
            const int kb = wave + WV * i;
            if (kb < nb) {
                if (XR && i == NBW - 1) {
                    auto xf = [&](int t, int) -> half8_t { return xreg[XR ? t : 0]; };
                    b[i].mma(acc, xf, g, *tab, q6, xsum[i]);
                } else {
                    // activation fragment at element e of the block: x[r][kb * 256 + e]
                    auto xf = [&](int, int e) -> half8_t {
                        return x8_from_bits<XT>(*(const LDSP(u32x4))(uintptr_t)(xr_base + (kb * KQ_QK + e) * 2));
                    };
                    b[i].mma(acc, xf, g, *tab, q6, xsum[i]);
                }
            }
        }
        kq_mfma_drain();
        // ---- sum the WV partials in wave order; every wave stores its slice
        const int buf = bufs == 2 ? (k & 1) : 0;
        float *rb = red + (size_t)buf * WV * 256;
        *(floatx4 *)(rb + 4 * (wave * 64 + lane)) = acc;
        __syncthreads();
        float sum = rb[4 * src_lane + src_e];
#pragma unroll
        for (int w = 1; w < WV; ++w) sum += rb[4 * (w * 64 + src_lane) + src_e];
        if (A->x_exp && out_lane) sum = ldexpf(sum, A->x_exp[out_m]);
        const int n = (tile - sc.begin) * 16 + out_n;
        const __amdgpu_buffer_rsrc_t ys = kq_buffer(sc.y, sc.y_bytes);
        const uint32_t yo = (out_lane && n < sc.N) ? (uint32_t)(out_m * sc.y_stride + n) * (y_f32 ? 4u : 2u) : kOut;
        if (y_f32)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sum), ys, yo, 0, 0);
        else
            __builtin_amdgcn_raw_buffer_store_b16(
                y_bf16 ? kq_f32_to_bf16_bits(sum) : __builtin_bit_cast(uint16_t, (_Float16)sum), ys, yo, 0, 0);
        if (bufs == 1) __syncthreads();  // the buffer is reused by the next tile
    };

    WB<CODEC> bq[DEPTH][NBW];
    // A ring requests its first DEPTH - 1 tiles before the wait for the x
    // copies, so their latency overlaps the staging.  A single slot requests
    // its tile after the staging (measured faster for one tile per
    // workgroup).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d) load_tile(bq[d], d);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // Q4_K: the activation sub-block sums of this wave's blocks, once per
    // launch (the wave's blocks never change): element e of lane (g, r) of an
    // MFMA whose selection A takes, at step t, the k values of lane group
    // r / 4 for row r when (r & 1) == (t >= 4), row r = 4g + (r & 3) only in
    // the first two of each four: sum of row r over sub-block 2g + e
    if constexpr (CODEC == KQ_CODEC_Q4_K || CODEC == KQ_MIX) {
        const _Float16 one = (_Float16)1.f, zero = (_Float16)0.f;
#pragma unroll
        for (int i = 0; i < NBW; ++i) {
            const int kb = wave + WV * i;
            floatx4 S = fzero4();
            if (kb < nb) {  // uniform over the wave
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const _Float16 v = (r >> 2) == g && (r & 2) == 0 && (r & 1) == (t >= 4 ? 1 : 0) ? one : zero;
                    const half8_t sel = {v, v, v, v, v, v, v, v};
                    const half8_t xf = (XR && i == NBW - 1)
                                           ? xreg[XR ? t : 0]
                                           : x8_from_bits<XT>(*(const LDSP(u32x4))(uintptr_t)(
                                                 xr_base + (kb * KQ_QK + WB<KQ_CODEC_Q4_K>::x_elem(t, g)) * 2));
                    S = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, xf, S, 0, 0, 0);
                }
                kq_mfma_drain();
            }
            xsum[i][0] = S[0];
            xsum[i][1] = S[1];
        }
    }
    // ring step k requests tile k + DEPTH - 1 and multiplies tile k; the loop
    // runs whole rounds of DEPTH steps (steps past the last tile only issue
    // their out-of-range requests)
    const int rounds = (my_tiles + DEPTH - 1) / DEPTH;
    for (int k0 = 0; k0 < rounds * DEPTH; k0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int k = k0 + d;
            load_tile(bq[(d + DEPTH - 1) % DEPTH], k + DEPTH - 1);
            __builtin_amdgcn_sched_barrier(0);
            if (k < my_tiles) compute_tile(bq[d], k);  // uniform over the workgroup
        }
    }
}

// Launch with `lds` bytes of dynamic LDS; the kernel's limit is raised to the
// CU's LDS once per instantiation (the default limit is lower).
template <int CODEC, int XT, int NBW, int DEPTH, bool XR, int WV>
int launch_one(const MvArgs &a, int grid, size_t lds, hipStream_t s) {
    static bool raised = false;
    if (!raised) {
        const size_t tables = CODEC == KQ_CODEC_IQ2_XXS ? sizeof(Iq2Tables) : 0;
        if (hipFuncSetAttribute((const void *)kq_mv_kernel<CODEC, XT, NBW, DEPTH, XR, WV>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kLdsBytes - tables)) != hipSuccess)
            return KQ_ERR_LAUNCH_FAILED;
        raised = true;
    }
    hipLaunchKernelGGL((kq_mv_kernel<CODEC, XT, NBW, DEPTH, XR, WV>), dim3(grid), dim3(64 * WV), lds, s, a);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

// Instantiated shapes (registers of a lane at 16 waves per CU: 128): one
// block per wave with rings of 1..3 tiles; two or three blocks per wave with
// rings of 1..2 tiles, except three Q6_K blocks and the XR form (ring of 1);
// the mixed Q4_K / Q6_K form as below.
template <int CODEC, int XT, int WV>
int launch_shape(const MvArgs &a, int nbw, int depth, bool xr, int grid, size_t lds, hipStream_t s) {
    if constexpr (CODEC == KQ_MIX) {
        // mixed Q4_K / Q6_K: up to two blocks per wave, x in LDS; rings of
        // one tile at two blocks and of two at one (deeper rings of both
        // codecs' views spilled: 20 / 40 bytes per lane)
        if (xr || nbw > 2) return KQ_ERR_BAD_SHAPE;
        if (nbw == 2) return launch_one<CODEC, XT, 2, 1, false, WV>(a, grid, lds, s);
        if (depth == 1) return launch_one<CODEC, XT, 1, 1, false, WV>(a, grid, lds, s);
        return launch_one<CODEC, XT, 1, 2, false, WV>(a, grid, lds, s);
    } else {
        if (nbw == 1) {
            if (depth == 1) return launch_one<CODEC, XT, 1, 1, false, WV>(a, grid, lds, s);
            if (depth == 2) return launch_one<CODEC, XT, 1, 2, false, WV>(a, grid, lds, s);
            return launch_one<CODEC, XT, 1, 3, false, WV>(a, grid, lds, s);
        }
        if (nbw == 2) {
            if constexpr (WV == kWaves) {
                if (xr) return launch_one<CODEC, XT, 2, 1, true, WV>(a, grid, lds, s);
            }
            if (depth == 1) return launch_one<CODEC, XT, 2, 1, false, WV>(a, grid, lds, s);
            return launch_one<CODEC, XT, 2, 2, false, WV>(a, grid, lds, s);
        }
        if constexpr (WV == kWaves) {  // 8-wave workgroups take K <= 4096
            if (nbw == 3) {
                if (xr) return launch_one<CODEC, XT, 3, 1, true, WV>(a, grid, lds, s);
                if constexpr (CODEC != KQ_CODEC_Q6_K) {
                    if (depth >= 2) return launch_one<CODEC, XT, 3, 2, false, WV>(a, grid, lds, s);
                }
                return launch_one<CODEC, XT, 3, 1, false, WV>(a, grid, lds, s);
            }
        }
    }
    return KQ_ERR_BAD_SHAPE;
}

int env_int(const char *name, int dflt) {
    const char *s = getenv(name);
    if (!s || !*s) return dflt;
    char *end = nullptr;
    const long v = strtol(s, &end, 10);
    return (end && *end == 0 && v > 0 && v < (1 << 24)) ? (int)v : dflt;
}

// Columns of x staged in LDS: all of K, or with XR all but the last block
// of every wave.
int mv_kl(const kq_matmul_problem &q, bool xr, int wv = kWaves) {
    const int nbw = (q.K / KQ_QK + wv - 1) / wv;
    return xr ? (nbw - 1) * wv * KQ_QK : q.K;
}

// Bytes of LDS the launch needs: staged x rows and the reduction buffers.
size_t mv_lds(const kq_matmul_problem &q, bool xr, int bufs, int wv = kWaves) {
    const size_t xrow = 2 * (size_t)mv_kl(q, xr, wv) + 16;
    return (size_t)q.M * xrow + (size_t)bufs * wv * 64 * sizeof(floatx4);
}

size_t mv_tables(const kq_matmul_problem &q) { return q.codec == KQ_CODEC_IQ2_XXS ? sizeof(Iq2Tables) : 0; }

// x in LDS when it fits with one reduction buffer, else XR (two or more
// blocks per wave); -1: neither fits.
int mv_xr(const kq_matmul_problem &q) {
    const size_t avail = (size_t)kLdsBytes - mv_tables(q);
    if (mv_lds(q, false, 1) <= avail) return 0;
    if (q.K / KQ_QK > kWaves && mv_lds(q, true, 1) <= avail) return 1;
    return -1;
}

int y_elem_bytes(int y_dtype) { return y_dtype == KQ_DTYPE_F32 ? 4 : 2; }

// A set of problems of one codec, or of Q4_K and Q6_K together (KQ_MIX).
bool mv_mixed(const kq_matmul_problem *ps, int n) {
    for (int i = 1; i < n; ++i)
        if (ps[i].codec != ps[0].codec) return true;
    return false;
}

}  // namespace

// Eligibility of a set of problems for the LDS-staged small-batch path: one
// codec (or Q4_K and Q6_K together, K <= 8192, x all in LDS), shared x /
// stride / M / K, M <= 16, fp16 activations, x rows that fit in LDS
// (all but the last 4096 columns, when K > 4096), at most 3 blocks per wave,
// weights and outputs addressable with 31-bit buffer offsets.
bool kq_mv_eligible(const kq_matmul_problem *ps, int n, int x_dtype, int y_dtype) {
    if (n <= 0) return false;
    if (x_dtype != KQ_DTYPE_F16) return false;
    const kq_matmul_problem &q0 = ps[0];
    if (q0.M < 1 || q0.M > 16) return false;
    const int nb = q0.K / KQ_QK;
    if (nb > 3 * kWaves) return false;
    const int xr = mv_xr(q0);
    if (xr < 0) return false;
    const bool mixed = mv_mixed(ps, n);
    if (mixed && (xr || nb > 2 * kWaves)) return false;
    for (int i = 0; i < n; ++i) {
        const kq_matmul_problem &q = ps[i];
        if (q.x != q0.x || q.x_row_stride != q0.x_row_stride || q.M != q0.M || q.K != q0.K) return false;
        if (mixed ? (q.codec != KQ_CODEC_Q4_K && q.codec != KQ_CODEC_Q6_K) : q.codec != q0.codec) return false;
        if ((int64_t)(q.N + 16) * q.w_row_bytes >= (int64_t)kOut) return false;
        if (((int64_t)(q.M - 1) * q.y_row_stride + q.N) * y_elem_bytes(y_dtype) >= (int64_t)kOut) return false;
    }
    return true;
}

// Problems validated and eligible (kq_mv_eligible), all live.
int kq_mv_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, hipStream_t s) {
    MvArgs a;
    int tiles = 0;
    for (int i = 0; i < n; ++i) {
        MvProblem &p = a.p[i];
        p.w = (const uint8_t *)ps[i].w;
        p.y = ps[i].y;
        p.y_stride = ps[i].y_row_stride;
        p.row_bytes = (uint32_t)ps[i].w_row_bytes;
        p.w_bytes = (uint32_t)(ps[i].N * ps[i].w_row_bytes);
        p.y_bytes = (uint32_t)(((int64_t)(ps[i].M - 1) * ps[i].y_row_stride + ps[i].N) * y_elem_bytes(y_dtype));
        p.N = ps[i].N;
        p.codec = ps[i].codec;
        a.tile_begin[i] = tiles;
        tiles += (ps[i].N + 15) / 16;
    }
    for (int i = n; i < KQ_MAX_GROUP; ++i) {
        a.p[i] = a.p[0];
        a.tile_begin[i] = 0x7FFFFFFF;
    }
    const kq_matmul_problem &q0 = ps[0];
    a.x = (const char *)q0.x;
    a.x_exp = x_exp;
    a.x_stride = q0.x_row_stride;
    a.M = q0.M;
    a.K = q0.K;
    a.y_dtype = y_dtype;
    a.total_tiles = tiles;
    a.n_problems = n;
    const bool xr = mv_xr(q0) == 1;
    const bool mixed = mv_mixed(ps, n);
    const int nb = q0.K / KQ_QK;
    // two 8-wave workgroups per CU for launches of at most two tiles per CU
    // (measured: q|k|v and o of a Q4_K_M layer 1-3 % faster, gate|up at six
    // tiles per CU 7 % slower), when x and one reduction buffer fit in half
    // the LDS and every wave keeps at most two blocks per tile;
    // GMLX_KQ_MV_WAVES=8 / 16 forces the choice
    const size_t half = (size_t)kLdsBytes / 2 - mv_tables(q0);
    const int want = env_int("GMLX_KQ_MV_WAVES", tiles <= 2 * device_cus() ? 8 : kWaves);
    const bool w8 = want == 8 && !xr && nb <= 16 && mv_lds(q0, false, 1, 8) <= half;
    const int wv = w8 ? 8 : kWaves;
    a.kl = mv_kl(q0, xr, wv);
    a.xrow = 2 * a.kl + 16;
    a.red_off = q0.M * a.xrow;
    a.red_bufs = w8 ? (mv_lds(q0, false, 2, 8) <= half ? 2 : 1)
                    : (mv_lds(q0, xr, 2) + mv_tables(q0) <= (size_t)kLdsBytes ? 2 : 1);
    const size_t lds = mv_lds(q0, xr, a.red_bufs, wv);
    int grid = env_int("GMLX_KQ_MV_WGS", device_cus() * (kWaves / wv));
    if (grid > tiles) grid = tiles;
    const int nbw = (nb + wv - 1) / wv;
    // ring depth: the tiles each workgroup walks, at most 3 (one block per
    // wave) or 2 (more blocks: register budget; launch_shape lowers it further
    // where the registers run out)
    const int per_wg = (tiles + grid - 1) / grid;
    const int depth = env_int("GMLX_KQ_MV_DEPTH", per_wg >= 4 ? 3 : per_wg >= 2 ? 2 : 1);
    const int d = min(depth, nbw == 1 ? 3 : 2);
    if (w8) {
        if (mixed) return launch_shape<KQ_MIX, 0, 8>(a, nbw, d, false, grid, lds, s);
        switch (q0.codec) {
        case KQ_CODEC_Q4_K: return launch_shape<KQ_CODEC_Q4_K, 0, 8>(a, nbw, d, false, grid, lds, s);
        case KQ_CODEC_Q6_K: return launch_shape<KQ_CODEC_Q6_K, 0, 8>(a, nbw, d, false, grid, lds, s);
        default: return launch_shape<KQ_CODEC_IQ2_XXS, 0, 8>(a, nbw, d, false, grid, lds, s);
        }
    }
    if (mixed) return launch_shape<KQ_MIX, 0, 16>(a, nbw, d, xr, grid, lds, s);
    switch (q0.codec) {
    case KQ_CODEC_Q4_K: return launch_shape<KQ_CODEC_Q4_K, 0, 16>(a, nbw, d, xr, grid, lds, s);
    case KQ_CODEC_Q6_K: return launch_shape<KQ_CODEC_Q6_K, 0, 16>(a, nbw, d, xr, grid, lds, s);
    default: return launch_shape<KQ_CODEC_IQ2_XXS, 0, 16>(a, nbw, d, xr, grid, lds, s);
    }
}
