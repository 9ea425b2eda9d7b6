// Weight-streaming small-batch matmul (M <= 16 activation rows) for problems
// that share their activations: the decode-step projections at batch 1..16
// (the MFMA computes 16 rows either way; 8-row launches keep half the
// partial-tile LDS and epilogue work).
//
//   y[M, N] = x[M, K] . dequant(W[N, K])^T,  fp32 accumulation
//
// Producer / consumer workgroups, one per CU, walking 16-row weight tiles
// t = blockIdx.x + k gridDim.x:
//  - 2 producer waves copy whole tiles (16 rows x K) from HBM into a ring of
//    R tile slots in LDS with direct-to-LDS buffer loads (no registers hold
//    the data), up to R tiles ahead of the compute;
//  - C consumer waves each own a K-slab of SB super-blocks for the whole
//    launch: their activation fragments of that slab are loaded once and stay
//    in registers; per tile a consumer reads its slab of the 16 rows from the
//    slot in the MFMA lane layout of kq_mma.h, dequantizes in registers, runs
//    v_mfma_f32_16x16x32_f16 and leaves its partial tile in LDS.
// One workgroup barrier per tile hands a landed slot to the consumers and a
// consumed slot back to the producers (the producers wait for their own loads
// with explicit vmcnt counts, so the later tiles stay in flight across it).
// The C partial tiles of a round are summed in consumer order
// (deterministic) and stored.  Dequantization (about 1.9 VALU instructions
// per weight per lane) runs on the consumers while the producers keep the HBM
// stream going; with one kind of wave alternating between loads and math the
// math added to the stream time instead of hiding under it (measured).
//
// Tile slot layout in LDS: row r at r * RC 16-byte chunks, RC = nb * SLOT / 16
// + 1 (the spare chunk staggers the rows over the LDS banks, so the 16 rows
// of an MFMA operand are read without conflicts); super-block kb of the row
// at kb * SLOT bytes.  The copy is row-contiguous: each 1 KB load covers 64
// consecutive chunks of the slot, one or two long runs of consecutive bytes of
// one or two weight rows (measured on this part: streaming the gate|up bytes
// this way takes 10.5 us against 14.1 us for per-lane row views, and 4.1
// against 8.4 us at q|k|v size).  A Q4_K + Q6_K group (the q|k|v of a Q4_K_M
// layer) runs in one launch with Q6_K-sized slots.
#include <stdlib.h>

#include <type_traits>

#include "kq_mma.h"

int device_cus();

namespace {

using namespace kqmma;

#define LDSP(T) __attribute__((address_space(3))) T *

constexpr int KQ_MIX = 0x7F;  // Q4_K and Q6_K problems in one launch
constexpr int kProducers = 2;
#ifndef KQ_STREAM_START_TILES
#define KQ_STREAM_START_TILES 2
#endif
// MR activation rows per launch (8, or 16 for M = 9..16): tiles per
// workgroup per round (the partial tiles of a round fill the same LDS)
__host__ __device__ constexpr int tiles_per_round(int MR) { return MR == 8 ? 8 : 4; }

// A super-block's LDS slot is SLOT bytes (16-aligned), filled by SLOT / 16
// chunk loads; chunk cb reads the 16 block bytes from src(cb), always inside
// the block (a load that crosses the end of a buffer range reads zeros whole).
//   Q4_K    : the 144 bytes in order.
//   Q6_K    : bytes 0..207 in order, then 194..209 (d lands at slot 222).
//   IQ2_XXS : bytes 0..15 (d at slot 0), then the 64 bytes of groups from
//             byte 2 (slot 16..79, 16-aligned).
template <int CODEC>
struct Geo;
template <>
struct Geo<KQ_CODEC_Q4_K> {
    static constexpr int BPB = 144, SLOT = 144;
    __device__ static constexpr int src(int cb) { return 16 * cb; }
};
template <>
struct Geo<KQ_CODEC_Q6_K> {
    static constexpr int BPB = 210, SLOT = 224, D_AT = 222;
    __device__ static constexpr int src(int cb) { return cb < 13 ? 16 * cb : 194; }
};
template <>
struct Geo<KQ_CODEC_IQ2_XXS> {
    static constexpr int BPB = 66, SLOT = 80;
    __device__ static constexpr int src(int cb) { return cb == 0 ? 0 : 2 + 16 * (cb - 1); }
};

__device__ __forceinline__ u32x4 lds128(uint32_t a) { return *(const LDSP(u32x4))(uintptr_t)a; }
__device__ __forceinline__ u32x2 lds64(uint32_t a) { return *(const LDSP(u32x2))(uintptr_t)a; }
__device__ __forceinline__ uint32_t lds16(uint32_t a) { return (uint32_t) * (const LDSP(uint16_t))(uintptr_t)a; }

// Lane views of kq_mma.h's Block<> filled from an LDS slot (layout above).
template <int CODEC>
__device__ __forceinline__ void load_slot(Block<CODEC> &b, uint32_t slot, int g);

template <>
__device__ __forceinline__ void load_slot<KQ_CODEC_Q4_K>(Block<KQ_CODEC_Q4_K> &b, uint32_t slot, int g) {
    b.hdr = lds128(slot);
#pragma unroll
    for (int c = 0; c < 4; ++c) b.q[c] = lds64(slot + 16 + 32 * c + 8 * g);
}

template <>
__device__ __forceinline__ void load_slot<KQ_CODEC_Q6_K>(Block<KQ_CODEC_Q6_K> &b, uint32_t slot, int g) {
#pragma unroll
    for (int i = 0; i < 4; ++i) b.ql[i] = lds64(slot + 64 * (i >> 1) + 32 * (i & 1) + 8 * g);
#pragma unroll
    for (int h = 0; h < 2; ++h) b.qh[h] = lds64(slot + 128 + 32 * h + 8 * g);
    b.sc = lds128(slot + 192);
    b.dbits = lds16(slot + Geo<KQ_CODEC_Q6_K>::D_AT);
}

template <>
__device__ __forceinline__ void load_slot<KQ_CODEC_IQ2_XXS>(Block<KQ_CODEC_IQ2_XXS> &b, uint32_t slot, int g) {
    b.raw = lds128(slot + 16 + 16 * g);
    b.dbits = lds16(slot);
}

struct StreamProblem {
    const uint8_t *w;
    void *y;
    int64_t y_stride;   // elements
    uint32_t w_bytes;   // N * row_bytes (< 2^31)
    uint32_t row_bytes;
    int32_t N;
    int32_t codec;
};

struct StreamArgs {
    int32_t tile_begin[KQ_MAX_GROUP];  // first tile of each problem; unused: INT_MAX
    StreamProblem p[KQ_MAX_GROUP];
    const char *x;                     // fp16 [M, K]
    const int32_t *x_exp;              // per-row exponents of prepared activations (results * 2^e), or null
    uint32_t *ctr;                     // split launches: arrivals per tile (zero on entry, left zero)
    float *part;                       // split launches: partial tiles [tile][slice][MR rows][16 columns]
    int64_t x_stride;                  // elements
    int32_t M, K, y_dtype, total_tiles, n_problems;
    int32_t split;                     // K slices per tile (1: the whole K in one item)
    int32_t pairs;                     // one-shot launches: workgroups holding two tiles
};

// K slices per tile at most (the last arrival loads them all at once).
constexpr int kMaxSplit = 8;

typedef const __attribute__((address_space(4))) StreamArgs *KArgs;

// Problems per launch (the eligibility test declines larger groups).
constexpr int kStreamProblems = 4;

// The problem of a tile, from the kernel arguments by constant indices only:
// the loads have fixed addresses, so they issue together (and then hit the
// scalar cache) instead of forming a chain of dependent scalar-cache misses
// (index, then fields) in front of every tile's first load.
__device__ __forceinline__ int problem_of(KArgs A, int tile) {
    int pi = 0;
#pragma unroll
    for (int i = 1; i < kStreamProblems; ++i) pi += tile >= A->tile_begin[i];  // unused entries: INT_MAX
    return pi;
}

__device__ __forceinline__ StreamProblem problem_at(KArgs A, int pi, int32_t &begin) {
    StreamProblem p;
#pragma unroll
    for (int i = 0; i < kStreamProblems; ++i)
        if (i == 0 || pi == i) {
            p.w = A->p[i].w;
            p.y = A->p[i].y;
            p.y_stride = A->p[i].y_stride;
            p.w_bytes = A->p[i].w_bytes;
            p.row_bytes = A->p[i].row_bytes;
            p.N = A->p[i].N;
            p.codec = A->p[i].codec;
            begin = A->tile_begin[i];
        }
    return p;
}

// Slot geometry of one codec for NB super-blocks per row.
template <int CODEC, int NB>
struct SlotGeo {
    static constexpr int CPB = Geo<CODEC>::SLOT / 16;  // chunks per super-block
    static constexpr int RC = NB * CPB + 1;            // chunks per (padded) row
    static constexpr int CHUNKS = 16 * RC;
};

// Byte offset in the weight matrix of slot chunk q of the tile whose first
// row is row0 (rows past last_row read last_row: their outputs are never
// stored).  The row pads and the chunks past the codec's geometry (a Q4_K
// tile in Q6_K-sized slots) are never read: their offset lies past the
// buffer, so the load writes zeros and makes no memory request (pointing them
// all at one address made a 16-row copy several times slower, measured).
template <int CODEC, int NB>
__device__ __forceinline__ uint32_t slot_src(int q, uint32_t row0, uint32_t last_row, uint32_t row_bytes) {
    using SG = SlotGeo<CODEC, NB>;
    const int row = q / SG::RC, w = q - row * SG::RC;
    if (w >= NB * SG::CPB || row >= 16) return 0x80000000u;
    const int blk = w / SG::CPB, cb = w - blk * SG::CPB;
    const uint32_t rr = min(row0 + (uint32_t)row, last_row);
    return rr * row_bytes + (uint32_t)(blk * Geo<CODEC>::BPB + Geo<CODEC>::src(cb));
}

// 1 KB loads per slot row (its NB super-blocks of chunks, without the pad).
template <int CODEC, int NB>
constexpr int row_parts() {
    return (NB * SlotGeo<CODEC, NB>::CPB + 63) / 64;
}

// Offset within a weight row of slot chunk w of the row (w < valid; others
// past the buffer, which reads zeros with no memory request).
template <int CODEC, int NB>
__device__ __forceinline__ uint32_t row_chunk_src(int w, int valid) {
    using SG = SlotGeo<CODEC, NB>;
    const int blk = w / SG::CPB, cb = w - blk * SG::CPB;
    return w < valid ? (uint32_t)(blk * Geo<CODEC>::BPB + Geo<CODEC>::src(cb)) : 0x80000000u;
}

// The slot geometry a launch allocates: its codec's, or Q6_K's for Q4_K + Q6_K.
template <int CODEC>
struct SlotCodec {
    static constexpr int C = CODEC;
};
template <>
struct SlotCodec<KQ_MIX> {
    static constexpr int C = KQ_CODEC_Q6_K;
};

// Loads per producer per tile: the slot's chunks in 1 KB loads, split evenly
// over the producers (the slot is allocated for all of them).
template <int SC, int NB>
constexpr int producer_loads() {
    return ((SlotGeo<SC, NB>::CHUNKS + 63) / 64 + kProducers - 1) / kProducers;
}
template <int SC, int NB>
constexpr int slot_bytes() {
    return producer_loads<SC, NB>() * kProducers * 1024;
}

// Wait until at most `newer` tiles of PL loads each are still in flight
// (K: the most the ring can hold, within the counter's 63).
template <int PL, int K>
__device__ __forceinline__ void wait_tiles_left(int newer) {
    if constexpr (K <= 0) {
        __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));
    } else {
        if (newer >= K) __builtin_amdgcn_s_waitcnt(KQ_VMCNT(K * PL));
        else wait_tiles_left<PL, K - 1>(newer);
    }
}

// IQ2_XXS kernels keep the fp16 grid / sign tables in LDS; other codecs
// allocate none (their views never read the tables).
template <int CODEC>
struct IqTables {
    __device__ static const Iq2Tables *get() { return nullptr; }
};
template <>
struct IqTables<KQ_CODEC_IQ2_XXS> {
    __device__ static const Iq2Tables *get() {
        __shared__ Iq2Tables t;
        load_iq2_tables(t);
        return &t;
    }
};

// ---- Q4_K with owned sub-blocks (launches of Q4_K problems only) ---------
// Lane group g owns sub-blocks 2g and 2g+1 of every super-block: qs bytes
// 32g + l (l = 0..31), whose low nibbles are values 64g + l and high nibbles
// values 64g + 32 + l.  Step t takes qs dword t of that run: the values
// l = 4t + (0, 2, 1, 3) of both sub-blocks.  A byte pair (b0, b2) or (b1, b3)
// becomes two biased fp16 values with one v_and_or_b32:
//   (w & 0x000F000F) | 0x64006400 = 1024 + low nibble (exponent 10: unit 1)
//   (w & 0x00F000F0) | 0x54005400 =   64 + high nibble (exponent 6: unit 16/16)
// and one fma against the exact constant -1024 sc (-64 sc) removes the bias:
// fma(1024 + q, sc, -1024 sc) = q sc, an integer of at most 945, exact (sc
// <= 63, so the constant, at most 64512, is exact as well).  The chain of a
// super-block is folded into the accumulator with d in fp32, and the minimum
// term -dmin m_j sum_{l in j} x_l enters through two fp32 MFMAs
// (min_accumulate) from the per-sub-block activation sums (fp32, q4own_x).
struct Q4Prep {
    half2_t sc;   // (sc_2g, sc_2g+1), exact integers
    half2_t nb;   // (-1024 sc_2g, -64 sc_2g+1)
    float d;
    float b0, b1; // -dmin m_2g, -dmin m_2g+1
};

// Constants of the owned view held in VGPRs: gfx9 VOP3 encodings take no
// literal and at most one SGPR, so v_and_or_b32 needs its mask and bias in
// vector registers (kept opaque to the compiler, which would otherwise fold
// them back into literal v_and / v_or pairs).
struct Q4Consts {
    uint32_t lo_mask, lo_bias, hi_mask, hi_bias, upper;  // upper: ~0 in lane groups 2, 3
    uint32_t sel;                                         // perm selector of the lane's scale byte pair
};

__device__ __forceinline__ Q4Consts q4own_consts(int g) {
    Q4Consts k = {0x000F000Fu, 0x64006400u, 0x00F000F0u, 0x54005400u, g >= 2 ? ~0u : 0u,
                  (g & 1) ? KQ_SEL_B23 : KQ_SEL_B01};
    asm volatile("" : "+v"(k.lo_mask), "+v"(k.lo_bias), "+v"(k.hi_mask), "+v"(k.hi_bias), "+v"(k.upper));
    return k;
}

__device__ __forceinline__ Q4Prep q4own_prep(u32x4 hdr, const Q4Consts &k) {
    const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;  // scale bytes 0..3, 4..7, 8..11
    // sub-blocks 0..3: sc = s[j] & 63, m = s[j+4] & 63; 4..7: low nibbles from
    // s[j+4], the two high bits from the top of s[j-4] / s[j]; the lane's
    // pair is picked by bit masks (a select would become a branch)
    const uint32_t sc_lo = s0 & 0x3F3F3F3Fu, m_lo = s1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
    const uint32_t scw = (sc_hi & k.upper) | (sc_lo & ~k.upper);
    const uint32_t mw = (m_hi & k.upper) | (m_lo & ~k.upper);
    const half2_t k1024 = {(_Float16)1024.f, (_Float16)1024.f};
    Q4Prep p;
    p.sc = h2b(__builtin_amdgcn_perm(0x64646464u, scw, k.sel)) - k1024;
    p.nb = p.sc * half2_t{(_Float16)-1024.f, (_Float16)-64.f};
    const half2_t m = h2b(__builtin_amdgcn_perm(0x64646464u, mw, k.sel)) - k1024;
    const float dmin = kq_f16_bits_to_f32(hdr.x >> 16);
    p.d = kq_f16_bits_to_f32(hdr.x & 0xFFFFu);
    p.b0 = -dmin * (float)m.x;
    p.b1 = -dmin * (float)m.y;
    return p;
}

__device__ __forceinline__ half8_t q4own_frag(uint32_t w, const Q4Prep &p, const Q4Consts &k) {
    const uint32_t w8 = w >> 8;
    const half2_t l0 = h2b((w & k.lo_mask) | k.lo_bias), l1 = h2b((w8 & k.lo_mask) | k.lo_bias);
    const half2_t u0 = h2b((w & k.hi_mask) | k.hi_bias), u1 = h2b((w8 & k.hi_mask) | k.hi_bias);
    const half2_t s0 = bcast(p.sc.x), s1 = bcast(p.sc.y);
    const half2_t c0 = bcast(p.nb.x), c1 = bcast(p.nb.y);
    return cat8(__builtin_elementwise_fma(l0, s0, c0), __builtin_elementwise_fma(l1, s0, c0),
                __builtin_elementwise_fma(u0, s1, c1), __builtin_elementwise_fma(u1, s1, c1));
}

// Activation fragments of the owned view for super-blocks kb0 .. kb0+SB-1:
// xr[s][t] = x[e + (0, 2, 1, 3)], x[e + 32 + (0, 2, 1, 3)] with e = 256 (kb0 + s)
// + 64 g + 4 t, and the sub-block sums (fp32): element 2 s + i of lane (g, r)
// = sum of activation row r over sub-block 2g + i of super-block s.
// Input: the lane's runs c[s][2 w + a] = x[256 (kb0 + s) + 64 g + 32 a + 8 w .. +7].
//
// The sums come from MFMAs with the fragments as the B operand (column r =
// batch row r) against a 0 / 1 selection A: row m = 4 g' + e of the result
// selects sub-block 2 g' + (e & 1) of super-block e >> 1, so lane (g, r)
// ends with the sums of its own row (exact products, fp32 accumulation).
template <int SB>
__device__ __forceinline__ void q4own_x(half8_t (&xr)[SB][8], floatx4 &xsum, const u32x4 (&cin)[SB][8], int lane) {
    static_assert(SB <= 2, "one accumulator holds two super-blocks of sums");
    const int g = lane >> 4, m = lane & 15;
    floatx4 sum = fzero4();
#pragma unroll
    for (int s = 0; s < SB; ++s) {
        // selection of super-block s: element i of lane (g, m) is 1 where row
        // m takes sub-block 2 g + (i >= 4) of super-block s
        const bool mine = (m >> 2) == g && ((m >> 1) & 1) == s;
        const _Float16 one = (_Float16)1.f, zero = (_Float16)0.f;
        const _Float16 lo = mine && (m & 1) == 0 ? one : zero, hi = mine && (m & 1) == 1 ? one : zero;
        const half8_t sel = {lo, lo, lo, lo, hi, hi, hi, hi};
        const u32x4(&c)[8] = cin[s];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const u32x4 &l = c[2 * (t >> 1)], &h = c[2 * (t >> 1) + 1];
            const int d = 2 * (t & 1);
            const u32x4 v = {__builtin_amdgcn_perm(l[d + 1], l[d], 0x05040100u),
                             __builtin_amdgcn_perm(l[d + 1], l[d], 0x07060302u),
                             __builtin_amdgcn_perm(h[d + 1], h[d], 0x05040100u),
                             __builtin_amdgcn_perm(h[d + 1], h[d], 0x07060302u)};
            xr[s][t] = __builtin_bit_cast(half8_t, v);
            sum = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, xr[s][t], sum, 0, 0, 0);
        }
    }
    xsum = sum;
}

// One K-slab of a tile in the owned view: row_p points at the lane's row,
// super-block kb0, in the slot.
template <int SB>
__device__ __forceinline__ void q4own_slab(floatx4 &acc, LDSP(const uint8_t) row_p, const half8_t (&xr)[SB][8],
                                           const floatx4 &xsum, const Q4Consts &k) {
    u32x4 hdr[SB], qa[SB], qb[SB];
#pragma unroll
    for (int s = 0; s < SB; ++s) {
        hdr[s] = *(const LDSP(u32x4))(row_p + s * 144);
        qa[s] = *(const LDSP(u32x4))(row_p + s * 144 + 16 + 32 * (kq_lane() >> 4));
        qb[s] = *(const LDSP(u32x4))(row_p + s * 144 + 32 + 32 * (kq_lane() >> 4));
    }
#pragma unroll
    for (int s = 0; s < SB; ++s) {
        const Q4Prep p = q4own_prep(hdr[s], k);
        const uint32_t q[8] = {qa[s].x, qa[s].y, qa[s].z, qa[s].w, qb[s].x, qb[s].y, qb[s].z, qb[s].w};
        floatx4 P;
#pragma unroll
        for (int t = 0; t < 8; ++t)
            P = __builtin_amdgcn_mfma_f32_16x16x32_f16(xr[s][t], q4own_frag(q[t], p, k), t == 0 ? fzero4() : P, 0, 0, 0);
        acc = fold4(p.d, P, acc);
        acc = min_accumulate(xsum[2 * s], xsum[2 * s + 1], p.b0, p.b1, acc);
    }
}

// One K-slab of a tile in kq_mma.h's Block<> views (xsum: the slab's
// activation sub-block sums, read by Q4_K tiles only).
template <int CODEC, int SB>
__device__ __forceinline__ void mma_slab(floatx4 &acc, uint32_t row_lds, const half8_t (&xr)[SB][8],
                                         const floatx4 &xsum, int g, const Iq2Tables &tab) {
#pragma unroll
    for (int s = 0; s < SB; ++s) {
        Block<CODEC> b;
        load_slot<CODEC>(b, row_lds + s * Geo<CODEC>::SLOT, g);
        b.prep(g);
        floatx4 P;
#pragma unroll
        for (int t = 0; t < 8; ++t)
            P = __builtin_amdgcn_mfma_f32_16x16x32_f16(xr[s][t], b.frag(t, g, tab), t == 0 ? fzero4() : P, 0, 0, 0);
        acc = fold4(b.dscale(), P, acc);
        if constexpr (CODEC == KQ_CODEC_Q4_K) {
            float b0, b1;
            b.min_b(g, b0, b1);
            acc = min_accumulate(xsum[2 * s], xsum[2 * s + 1], b0, b1, acc);
        }
    }
}

// CODEC: KQ_CODEC_* or KQ_MIX.  SB: super-blocks per consumer, C consumers
// (K = 256 SB C).  R: tile slots in the ring.  MR: activation rows (8 or 16).
template <int CODEC, int SB, int C, int R, int MR>
__global__ __launch_bounds__(64 * (kProducers + C)) void kq_stream_kernel(StreamArgs a_) {
    constexpr int NB = SB * C;
    constexpr int SC = SlotCodec<CODEC>::C;
    // Rows of at least 64 chunks load by rows (PR loads each); shorter ones
    // by the slot's consecutive 1 KB runs with per-lane row offsets.
    constexpr int kRowChunks = NB * SlotGeo<SC, NB>::CPB;
    constexpr bool kByRows = kRowChunks >= 64;
    constexpr int PR = row_parts<SC, NB>();  // loads per slot row
    constexpr int PL = kByRows ? (16 / kProducers) * PR : producer_loads<SC, NB>();  // loads per producer per tile
    // row pitch of a mixed launch's Q4_K tiles: the Q6_K slot's when loading by rows
    constexpr int kMixQ4Pitch = (kByRows ? SlotGeo<SC, NB>::RC : SlotGeo<KQ_CODEC_Q4_K, NB>::RC) * 16;
    constexpr int SLOTB = slot_bytes<SC, NB>();
    constexpr int XC = CODEC == KQ_MIX ? KQ_CODEC_Q4_K : CODEC;  // activation layout (Q4_K / Q6_K alike)
    static_assert(PL <= 63, "vmcnt counts at most 63 loads");
    constexpr int kTmax = tiles_per_round(MR);
    constexpr int LR = 4 * MR;  // lanes of a partial tile that hold live rows (MFMA row 4g + e in lane 16g + n)
    // Activation staging: C regions of 8 rows of kXPitch bytes (1 KB and 16:
    // rows on different banks) from ring slot kXSlot on, which the producers
    // fill only after the first hand-off (it may reach into the partial-tile
    // area, free until the round ends).  Forms where it does not fit load the
    // fragments straight into registers.
    constexpr int kXPitch = 1040;
    constexpr size_t kXRegion = (size_t)C * 8 * kXPitch;
    constexpr size_t kRedBytes = (size_t)kTmax * C * LR * 16;
    constexpr int kXSlot = (size_t)(R - 2) * SLOTB + kRedBytes >= kXRegion && R >= 3   ? 2
                           : (size_t)(R - 1) * SLOTB + kRedBytes >= kXRegion && R >= 2 ? 1
                                                                                      : 0;
    // Staging halves a two-block slab's load instructions (one 1 KB row each
    // instead of eight 16-byte runs per block and lane); a one-block slab
    // gains nothing at 8 rows and gives up a start tile (the down slices:
    // 16.0 against 15.4 us, measured).  At 16 rows (two passes through the
    // region) it pays for Q4_K (gate|up at 9..16 rows: 16.2-17.0 against
    // 16.9-18.8 us), not for the Q4_K + Q6_K form (q|k|v: 10.4-11.5 against
    // 10.3-11.3 us); the Q6_K form would spill.
    constexpr bool kXStaged = kXSlot > 0 && SB == 2 && (MR == 8 || CODEC == KQ_CODEC_Q4_K);
    // tiles issued before the first hand-off (below the staging region)
    constexpr int kStartTiles = kXStaged ? (KQ_STREAM_START_TILES < kXSlot ? KQ_STREAM_START_TILES : kXSlot)
                                         : (KQ_STREAM_START_TILES < R ? KQ_STREAM_START_TILES : R);
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const KArgs A = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
    const Iq2Tables &iq2_tab = *IqTables<CODEC>::get();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = kq_lane(), r = lane & 15, g = lane >> 4;
    const int G = (int)gridDim.x, B0 = (int)blockIdx.x;
    const int M = A->M;
    // item i = (tile i / S, K-slice i % S); workgroup B0 takes items B0 + j G,
    // which with G a multiple of S are slice q of tiles T0 + j Gs
    const int S = A->split, q = B0 % S, Gs = G / S, T0 = B0 / S;
    const int my_tiles = (A->total_tiles - T0 + Gs - 1) / Gs;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(LDSP(void))smem;
    floatx4 *red = (floatx4 *)(smem + R * SLOTB);  // [kTmax][C][LR lanes]

    if (wave < kProducers) {
        // ================= producer: tiles into slots, up to R ahead.  The
        // ring runs across rounds: the workgroup's tile j goes to slot j % R,
        // and the next round's first tiles are in flight while the consumers
        // sum a round's partial tiles.
        {
            // Rows of 64 chunks or more: one load per (row, 1 KB part of the
            // row's slot chunks).  The row's offset goes in the load's scalar
            // offset (rows past N clamped by scalar code) and the lane's
            // offset within the row comes from a table of PR registers made
            // once, so a load costs no VALU instruction (per-lane row offsets
            // cost about ten, much of the launch's start).  The last part
            // covers the row's last 64 chunks: where it overlaps the part
            // before, both write the same bytes.  (The tables reach copy as
            // arguments: captured by the lambda, the host pass dropped the
            // kernel's instantiations.)
            uint32_t tab[PR];     // the launch's slot geometry
            uint32_t tab_q4[PR];  // Q4_K tiles in Q6_K-sized slots (mixed launch)
#pragma unroll
            for (int p = 0; p < PR; ++p) {
                const int w = (p == PR - 1 ? kRowChunks - 64 : 64 * p) + lane;
                tab[p] = kByRows ? row_chunk_src<SC, NB>(w, kRowChunks) : 0u;
                tab_q4[p] = kByRows && CODEC == KQ_MIX ? row_chunk_src<KQ_CODEC_Q4_K, NB>(w, NB * 9) : 0u;
            }
            auto copy = [&](int j, const uint32_t *tb, const uint32_t *tb4) {
                const int tile = T0 + j * Gs;
                int32_t begin;
                const StreamProblem pr = problem_at(A, problem_of(A, tile), begin);
                const uint32_t rb = pr.row_bytes;
                const uint32_t row0 = (uint32_t)(tile - begin) * 16;
                const uint32_t last = (uint32_t)pr.N - 1;
                const __amdgpu_buffer_rsrc_t rs = kq_buffer(pr.w, pr.w_bytes);
                const bool q6 = CODEC == KQ_MIX && pr.codec == KQ_CODEC_Q6_K;
                const uint32_t slot = ring_lds + (uint32_t)(j % R) * SLOTB;
                // the slice's first super-block in each row
                const uint32_t kofs = (uint32_t)(q * NB) * (uint32_t)(q6 ? Geo<KQ_CODEC_Q6_K>::BPB : Geo<XC>::BPB);
                if constexpr (kByRows) {
                    // producer w copies rows w, w + 2, ...
                    auto issue = [&](const uint32_t *t) {
#pragma unroll
                        for (int i = 0; i < 16 / kProducers; ++i) {
                            const int row = i * kProducers + wave;
                            const uint32_t rr = min(row0 + (uint32_t)row, last);
                            const int soff = (int)(rr * rb + kofs);
                            const uint32_t m0 = slot + (uint32_t)(row * SlotGeo<SC, NB>::RC * 16);
#pragma unroll
                            for (int p2 = 0; p2 < PR; ++p2)
                                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                                    rs, (LDSP(void))(uintptr_t)(m0 + 16 * (p2 == PR - 1 ? kRowChunks - 64 : 64 * p2)),
                                    16, t[p2], soff, 0, 0);
                        }
                    };
                    if constexpr (CODEC == KQ_MIX) {
                        if (q6) issue(tb);
                        else issue(tb4);
                    } else {
                        issue(tb);
                    }
                } else {
                    // load i of this wave fills slot chunks 64 (i P + wave) .. +63
                    auto issue = [&](auto geo) {
                        constexpr int GC = decltype(geo)::C;
#pragma unroll
                        for (int i = 0; i < PL; ++i) {
                            const int li = i * kProducers + wave;
                            const uint32_t off = slot_src<GC, NB>(64 * li + lane, row0, last, rb);
                            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDSP(void))(uintptr_t)(slot + 1024 * li),
                                                                     16, off + kofs, 0, 0, 0);
                        }
                    };
                    // a mixed launch branches once per tile (uniform), so only
                    // one geometry's offsets are live
                    if constexpr (CODEC == KQ_MIX) {
                        if (q6) issue(SlotCodec<KQ_CODEC_Q6_K>{});
                        else issue(SlotCodec<KQ_CODEC_Q4_K>{});
                    } else {
                        issue(SlotCodec<CODEC>{});
                    }
                }
            };
            // The start is bound by the memory system, which every CU floods
            // at once: the consumers' activation loads go first (they issue
            // them before this barrier), then kStartTiles tiles; the rest of
            // the ring follows once tile 0 is with the consumers (the whole
            // ring issued together delayed tile 0 by about 2 us; two tiles
            // beat one by 0.25 us at gate|up size, measured).
            __builtin_amdgcn_s_barrier();
            const int first = min(kStartTiles, my_tiles);
            for (int j = 0; j < first; ++j) copy(j, tab, tab_q4);
            for (int b = 0; b < my_tiles; ++b) {
                // wait for tile b's loads; the tiles copied after it stay in flight
                const int newer = b == 0 ? first - 1 : min(R - 2, my_tiles - 1 - b);
                wait_tiles_left<PL, (R - 1 < 63 / PL ? R - 1 : 63 / PL)>(newer);
                __builtin_amdgcn_s_barrier();  // slot b % R to the consumers; slot (b - 1) % R back
                if (b == 0) {
                    for (int j = first; j < min(R, my_tiles); ++j) copy(j, tab, tab_q4);
                } else if (b + R - 1 < my_tiles) {
                    copy(b + R - 1, tab, tab_q4);
                }
                if ((b + 1) % kTmax == 0 || b + 1 == my_tiles) {
                    __builtin_amdgcn_s_barrier();  // the round's partial tiles are in LDS
                    if (b + 1 < my_tiles)
                        __builtin_amdgcn_s_barrier();  // the round's outputs are summed: red is free
                }
            }
        }
        return;
    }

    // ================= consumer c: K-slab [c SB, c SB + SB) of every tile
    const int c = wave - kProducers;
    const int kb0 = c * SB;
    half8_t xr[SB][8];
    // Q4_K tiles: the slab's activation sub-block sums (fp32)
    [[maybe_unused]] floatx4 xsum = fzero4();
    {
        const uint32_t xbytes = (uint32_t)(((int64_t)(M - 1) * A->x_stride + A->K) * 2);
        const __amdgpu_buffer_rsrc_t xs = kq_buffer(A->x, xbytes);
        const uint32_t col0 = (uint32_t)((q * NB + kb0) * KQ_QK * 2);
        if constexpr (kXStaged) {
            // The slab's rows arrive by direct-to-LDS loads, one row (SB x
            // 512 bytes) per instruction, into ring slots the producers fill
            // only after the first hand-off; then each lane reads its
            // fragments.  Lanes past the slab read zeros into the row's unused
            // bytes.  16 rows take two passes through the region.
            const uint32_t xreg = ring_lds + kXSlot * SLOTB + (uint32_t)(c * 8 * kXPitch);
            const uint32_t lsrc = 16u * lane < 512u * SB ? 16u * lane + col0 : 0x80000000u;
            const uint32_t rowa = xreg + (uint32_t)((r & 7) * kXPitch);
            [[maybe_unused]] u32x4 cin[SB][8];
            const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int p = 0; p < MR / 8; ++p) {
                if (p > 0) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the region's reads are done
#pragma unroll
                for (int m = 0; m < 8; ++m)
                    if (8 * p + m < M)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            xs, (LDSP(void))(uintptr_t)(xreg + m * kXPitch), 16,
                            lsrc + (uint32_t)((8 * p + m) * A->x_stride * 2), 0, 0, 0);
                if (p == 0) __builtin_amdgcn_s_barrier();  // the loads are issued: the producers may start
                __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));
                const bool mine = (r >> 3) == p && r < M;
#pragma unroll
                for (int s2 = 0; s2 < SB; ++s2)
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        if constexpr (CODEC == KQ_CODEC_Q4_K) {
                            // owned view: c[2 w + a] = x[64 g + 32 a + 8 w .. +7]
                            const u32x4 v =
                                lds128(rowa + (uint32_t)(2 * (256 * s2 + 64 * g + 32 * (t & 1) + 8 * (t >> 1))));
                            cin[s2][t] = mine ? v : (p == 0 ? zero : cin[s2][t]);
                        } else {
                            const u32x4 v = lds128(rowa + (uint32_t)(2 * (256 * s2 + Block<XC>::x_elem(t, g))));
                            const u32x4 old = p == 0 ? zero : __builtin_bit_cast(u32x4, xr[s2][t]);
                            xr[s2][t] = __builtin_bit_cast(half8_t, mine ? v : old);
                        }
                    }
            }
            if constexpr (CODEC == KQ_CODEC_Q4_K) q4own_x<SB>(xr, xsum, cin, lane);
        } else {
            // The slab's activation fragments straight from global memory into
            // registers: lane (g, r) reads 16-byte runs of row r, rows >= M
            // past the buffer (zeros).
            const uint32_t xrow = r < M ? (uint32_t)(r * A->x_stride * 2) + col0 : 0x80000000u;
            if constexpr (CODEC == KQ_CODEC_Q4_K) {
                // owned view: lane group g needs values 64 g .. 64 g + 63 of each
                // super-block, as 16-byte runs c[2 w + a] = x[64 g + 32 a + 8 w .. +7]
                u32x4 cin[SB][8];
#pragma unroll
                for (int s2 = 0; s2 < SB; ++s2)
#pragma unroll
                    for (int w = 0; w < 4; ++w)
#pragma unroll
                        for (int a2 = 0; a2 < 2; ++a2)
                            cin[s2][2 * w + a2] = __builtin_bit_cast(
                                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           xs, xrow + (uint32_t)(2 * (256 * s2 + 64 * g + 32 * a2 + 8 * w)), 0, 0));
                __builtin_amdgcn_s_barrier();  // the loads are issued: the producers may start
                q4own_x<SB>(xr, xsum, cin, lane);
            } else {
#pragma unroll
                for (int s2 = 0; s2 < SB; ++s2)
#pragma unroll
                    for (int t = 0; t < 8; ++t)
                        xr[s2][t] = __builtin_bit_cast(
                            half8_t, __builtin_amdgcn_raw_buffer_load_b128(
                                         xs, xrow + (uint32_t)(2 * (256 * s2 + Block<XC>::x_elem(t, g))), 0, 0));
                __builtin_amdgcn_s_barrier();  // the loads are issued: the producers may start
            }
        }
    }
    // a mixed launch's Q4_K tiles: the sums in the Block<> layout
    if constexpr (CODEC == KQ_MIX) xsum = xsum_generic<SB>(xr, r);
    // owned Q4_K view: the lane's row at super-block kb0 in slot 0
    [[maybe_unused]] const Q4Consts q4k = q4own_consts(g);
    [[maybe_unused]] LDSP(const uint8_t) own_p =
        (LDSP(const uint8_t))smem + r * SlotGeo<KQ_CODEC_Q4_K, NB>::RC * 16 + kb0 * 144;
    // The epilogue's parameters are read ahead of the tiles: per-row exponents
    // of prepared activations once, the output of the consumer's first tile of
    // a round before the round (its kernel-argument loads, a chain of scalar
    // loads, took about 1 us at the end of a launch, measured).
    const int n = lane & 15, mq = lane >> 4;
    const bool has_xe = A->x_exp != nullptr;
    int xe[MR / 4];
#pragma unroll
    for (int h = 0; h < MR / 4; ++h) xe[h] = has_xe && 4 * h + mq < M ? A->x_exp[4 * h + mq] : 0;
    // (arguments, not captures: a lambda capturing a local array dropped the
    // kernel's host-side instantiations)
    // kept in registers (the compiler would reload them at their use)
    int ydt = A->y_dtype;
    uint64_t part_b = (uint64_t)(uintptr_t)A->part, ctr_b = (uint64_t)(uintptr_t)A->ctr;
    asm volatile("" : "+s"(ydt), "+s"(part_b), "+s"(ctr_b));
    float *const part = (float *)(uintptr_t)part_b;
    uint32_t *const ctr0 = (uint32_t *)(uintptr_t)ctr_b;
    // arrival counters spread over the counter region (up to one per 128-byte
    // line): the slices of a launch's tiles arrive at nearly the same time
    const int cstride = min(32, 1 << (31 - __builtin_clz(
                                          (int)(KQ_MATMUL_COUNTER_BYTES / 4) / max(A->total_tiles, 1))));
    auto store = [&](const StreamProblem &pr, int32_t begin, int tile, int m, int e, float sum) {
        if (m >= M) return;
        if (has_xe) sum = ldexpf(sum, e);
        const int nn = (tile - begin) * 16 + n;
        if (nn < pr.N) kq_store_out(pr.y, ydt, (int64_t)m * pr.y_stride + nn, sum);
    };
    for (int round0 = 0; round0 < my_tiles; round0 += kTmax) {
        const int nt = min(kTmax, my_tiles - round0);
        const int etile = T0 + (round0 + c) * Gs;  // this consumer's first tile of the round (if c < nt)
        int32_t ebegin = 0;
        StreamProblem epr = problem_at(A, problem_of(A, c < nt ? etile : T0), ebegin);
        {
            // held in registers from here (left to itself, the compiler
            // sinks these kernel-argument loads to their use at the store)
            uint64_t yb = (uint64_t)(uintptr_t)epr.y;
            int64_t ys = epr.y_stride;
            asm volatile("" : "+s"(yb), "+s"(ys), "+s"(epr.N), "+s"(ebegin));
            epr.y = (void *)(uintptr_t)yb;
            epr.y_stride = ys;
        }
        for (int b = 0; b < nt; ++b) {
            const int gb = round0 + b;  // the workgroup's tile count: slot gb % R
            __builtin_amdgcn_s_barrier();  // tile gb has landed in its slot
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            const int tile = T0 + gb * Gs;
            const uint32_t slot = ring_lds + (uint32_t)(gb % R) * SLOTB;
            floatx4 acc = {0, 0, 0, 0};
            if constexpr (CODEC == KQ_MIX) {
                int32_t begin;
                if (problem_at(A, problem_of(A, tile), begin).codec == KQ_CODEC_Q6_K)
                    mma_slab<KQ_CODEC_Q6_K, SB>(acc, slot + r * SlotGeo<KQ_CODEC_Q6_K, NB>::RC * 16 + kb0 * 224, xr,
                                                xsum, g, iq2_tab);
                else
                    mma_slab<KQ_CODEC_Q4_K, SB>(acc, slot + r * kMixQ4Pitch + kb0 * 144, xr, xsum, g,
                                                iq2_tab);
            } else if constexpr (CODEC == KQ_CODEC_Q4_K) {
                q4own_slab<SB>(acc, own_p + (gb % R) * SLOTB, xr, xsum, q4k);
            } else {
                mma_slab<CODEC, SB>(acc, slot + r * SlotGeo<CODEC, NB>::RC * 16 + kb0 * Geo<CODEC>::SLOT, xr, xsum, g,
                                    iq2_tab);
            }
            kq_mfma_drain();
            // batch rows 4g + e < MR live in lanes g < MR / 4
            if (g < MR / 4) red[(b * C + c) * LR + lane] = acc;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // slot reads and red writes done
        }
        __builtin_amdgcn_s_barrier();  // every partial tile of the round is in LDS
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // ---- consumer c sums tiles b = c, c + C, ... of the round over the C
        // partial tiles in consumer order (deterministic).  Lane l holds
        // outputs o = 64 h + l (h < MR / 4) of the tile: row m = o >> 4,
        // column l & 15.
        for (int b = c; b < nt; b += C) {
            const int tile = T0 + (round0 + b) * Gs;
            int32_t begin = ebegin;
            const StreamProblem pr = b == c ? epr : problem_at(A, problem_of(A, tile), begin);
#pragma unroll
            for (int h = 0; h < MR / 4; ++h) {
                // one float per lane and partial tile: element mq of lane 16 h + n
                const float *rf = (const float *)red + 4 * (b * C * LR + 16 * h + n) + mq;
                float sum = rf[0];
#pragma unroll
                for (int c2 = 1; c2 < C; ++c2) sum += rf[4 * c2 * LR];
                if (S == 1) store(pr, begin, tile, 4 * h + mq, xe[h], sum);
                else if (4 * h + mq < M)
                    __hip_atomic_store(part + ((size_t)tile * S + q) * (16 * MR) + 64 * h + lane, sum,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (S > 1) {
            // Split launches: the slice's partial tiles out, then one arrival
            // per tile (lane i: the wave's i-th tile of the round); the last
            // of a tile's S arrivals sums the S partials in slice order
            // (deterministic), stores, and clears the count for the next call.
            // The partials move by agent-scope stores and loads, which are
            // coherent across the XCDs' L2s by themselves; an agent-scope
            // fence would write back and invalidate whole L2s instead (it
            // made a split launch slower than the unsplit one, measured).
            // Ordering: the stores have completed (vmcnt 0) before the
            // arrival is counted, and the loads issue only after the count
            // returns.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));
            const int bl = c + lane * C;
            bool last = false;
            if (bl < nt) {
                uint32_t *ctr = ctr0 + (T0 + (round0 + bl) * Gs) * cstride;
                last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(S - 1);
                if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            uint64_t mine = __builtin_amdgcn_ballot_w64(last);
            if (mine) {
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                while (mine) {
                    const int i = __builtin_ctzll(mine);
                    mine &= mine - 1;
                    const int tile = T0 + (round0 + c + i * C) * Gs;
                    int32_t begin = ebegin;
                    const StreamProblem pr = i == 0 ? epr : problem_at(A, problem_of(A, tile), begin);
                    const float *pp = part + (size_t)tile * S * (16 * MR);
#pragma unroll
                    for (int h = 0; h < MR / 4; ++h) {
                        const int o = 64 * h + lane;
                        if (4 * h + mq >= M) continue;
                        float v[kMaxSplit];
#pragma unroll
                        for (int s2 = 0; s2 < kMaxSplit; ++s2)
                            v[s2] = s2 < S ? __hip_atomic_load(pp + s2 * (16 * MR) + o, __ATOMIC_RELAXED,
                                                               __HIP_MEMORY_SCOPE_AGENT)
                                           : 0.f;
                        float sum = v[0];
#pragma unroll
                        for (int s2 = 1; s2 < kMaxSplit; ++s2)
                            if (s2 < S) sum += v[s2];
                        store(pr, begin, tile, 4 * h + mq, xe[h], sum);
                    }
                }
            }
        }
        if (round0 + kTmax < my_tiles) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_barrier();  // red is free for the next round
        }
    }
}

template <int CODEC, int SB, int C, int MR>
int launch(const StreamArgs &a, int grid, hipStream_t s) {
    constexpr int NB = SB * C;
    constexpr int SC = SlotCodec<CODEC>::C;
    // as many tile slots as fit beside the partial tiles, 2 to 6: the bytes a
    // CU keeps in flight set its share of the bandwidth, so small slots (K
    // slices, short K) take deeper rings
    constexpr size_t red = (size_t)tiles_per_round(MR) * C * (4 * MR) * 16;
    constexpr size_t budget = 150 * 1024 - (CODEC == KQ_CODEC_IQ2_XXS ? sizeof(Iq2Tables) : 0);
    constexpr size_t sb = slot_bytes<SC, NB>();
    constexpr auto need = [](size_t ring) { return ring + red; };
    constexpr int R = need(6 * sb) <= budget   ? 6
                      : need(5 * sb) <= budget ? 5
                      : need(4 * sb) <= budget ? 4
                      : need(3 * sb) <= budget ? 3
                                               : 2;
    constexpr size_t lds = need((size_t)R * sb);
    static_assert(lds <= budget, "stream kernel LDS");
    static bool raised = false;
    if (!raised) {
        if (hipFuncSetAttribute((const void *)kq_stream_kernel<CODEC, SB, C, R, MR>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return KQ_ERR_LAUNCH_FAILED;
        raised = true;
    }
    hipLaunchKernelGGL((kq_stream_kernel<CODEC, SB, C, R, MR>), dim3(grid), dim3(64 * (kProducers + C)), lds, s, a);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

// Consumers for K = 256 nb (one K-slab of SB super-blocks each): as many as
// the slab count allows up to 12, so that two or more share each SIMD and
// hide each other's LDS and MFMA latency (8 consumers of one super-block beat
// 4 of two by 1-2 us on the 8-block slices of a split down projection,
// measured); 16 blocks take 8 consumers of two.  The mixed Q4_K + Q6_K form
// keeps two super-blocks per consumer where one would spill.
template <int CODEC, int MR>
int launch_codec(const StreamArgs &a, int nb, int grid, hipStream_t s) {
    constexpr bool mix = CODEC == KQ_MIX;
    switch (nb) {
    case 2: return launch<CODEC, 1, 2, MR>(a, grid, s);
    case 4: return launch<CODEC, 1, 4, MR>(a, grid, s);
    case 6: return launch<CODEC, 1, 6, MR>(a, grid, s);
    case 8:
        if constexpr (mix) return launch<CODEC, 2, 4, MR>(a, grid, s);
        else return launch<CODEC, 1, 8, MR>(a, grid, s);
    case 12:
        if constexpr (mix) return launch<CODEC, 2, 6, MR>(a, grid, s);
        else return launch<CODEC, 1, 12, MR>(a, grid, s);
    case 16: return launch<CODEC, 2, 8, MR>(a, grid, s);
    default: return KQ_ERR_BAD_SHAPE;
    }
}

template <int CODEC>
int launch_rows(const StreamArgs &a, int nb, int grid, hipStream_t s) {
    return a.M <= 8 ? launch_codec<CODEC, 8>(a, nb, grid, s) : launch_codec<CODEC, 16>(a, nb, grid, s);
}

bool stream_k_ok(int K) {
    const int nb = K / KQ_QK;
    return nb == 2 || nb == 4 || nb == 6 || nb == 8 || nb == 12 || nb == 16;
}

// ---- One-shot kernel: a workgroup's whole share in LDS at once --------------
// Launches of at most two 16-row tiles per CU (the o and q|k|v projections of
// a decode step at up to 32 rows).  Every wave owns one super-block column of
// the workgroup's tiles (NB = 16: super-block `wave` of each tile; NB = 8:
// unit `wave` = tile wave / 8, super-block wave % 8): at entry it copies that
// column of each tile (16 rows) and the 8 activation rows of that
// super-block into its own LDS region with direct-to-LDS loads, waits for its
// own loads only, and multiplies at once, so the math of the columns that
// land first overlaps the loads of the others (after one barrier for the
// whole tile, the math ran after the last byte: 1-1.9 us more per launch,
// measured with in-kernel stamps).  The partial tiles are then written into
// the waves' regions, and after the launch's only barrier 128 threads per
// tile sum them in super-block order (deterministic) and store.
// Tiles: T over G = min(CUs, T) workgroups (T <= 2 G): workgroup b < P = T - G
// takes tiles 2b and 2b + 1, the others tile P + b.  The host orders Q4_K
// problems before Q6_K ones (a workgroup then holds two Q4_K tiles or one of
// either codec) and checks that every workgroup fits in LDS.
// A wave's region: the activation slab (8 rows x 512 bytes, each row's
// 16-byte chunks XOR-swizzled by the row so the fragment reads of 8 rows hit
// different banks; rows >= M read as zeros; a 16-row launch copies rows
// 8..15 into it once lanes 0..7 hold theirs; a 32-row launch then runs rows
// 16..31 as a second block through the same slab after the first block's
// sums, reading and decoding the columns again), then its columns: Q4_K rows of
// 144 bytes, Q6_K rows of 240 (the streaming kernel's 224-byte slot with d at
// 222, and a spare chunk: 15 chunks, an odd count, so the 16 rows of an MFMA
// operand hit different banks).
constexpr int kShotWaves = 16;
constexpr int kShotRows = 8;
constexpr int kShotSlab = kShotRows * 512;

__host__ __device__ constexpr int shot_col_bytes(int codec) { return codec == KQ_CODEC_Q6_K ? 16 * 240 : 16 * 144; }

// Bytes of a wave's region for tiles of column sizes c0 and c1 (0: none).
__host__ __device__ constexpr int shot_region(int nb, int c0, int c1) {
    return kShotSlab + (nb == 16 ? c0 + c1 : (c0 > c1 ? c0 : c1));
}

// Direct-to-LDS buffer loads of 16 and 4 bytes per lane.  Plain functions, not
// templates: the builtin exists for the device target only, and the host pass
// marks a function template whose body uses it invalid after its first
// instantiation, so a second kernel instance calling the same specialization
// would not compile.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDSP(void))(uintptr_t)lds, 16, voff, (int)soff, 0, 0);
}
__device__ __forceinline__ void lds_dma4(__amdgpu_buffer_rsrc_t rs, uint32_t lds, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDSP(void))(uintptr_t)lds, 4, voff, (int)soff, 0, 0);
}

// Column kb of a 16-row tile (codec C) into LDS at dst: 64-chunk loads of 16
// bytes per lane, then the rest in loads of 4 bytes per lane (a 16-byte load
// writes 1 KB whatever its range, which would run into the next column).
// voffset: the row's offset within the tile's rows (row r, clamped to rlast)
// plus the column's bytes; soff: the tile's first row.
template <int C, int NB>
__device__ __forceinline__ void shot_copy_col(__amdgpu_buffer_rsrc_t rs, uint32_t dst, uint32_t row_bytes,
                                              uint32_t kofs, int rlast, uint32_t soff, int lane) {
    constexpr int RCH = C == KQ_CODEC_Q6_K ? 15 : 9;  // chunks per LDS row
    constexpr int CH = 16 * RCH;
    constexpr int FULL = CH / 64;
    constexpr int TAIL = (CH - 64 * FULL) * 4 / 64;   // dword loads
    auto src = [&](int q, int byte) -> uint32_t {
        const int row = q / RCH, c = q - row * RCH;
        int off;
        if constexpr (C == KQ_CODEC_Q6_K) off = c < 13 ? 16 * c : c == 13 ? 194 : -1;
        else off = 16 * c;
        return off < 0 ? 0x80000000u
                       : (uint32_t)min(row, rlast) * row_bytes + kofs + (uint32_t)(off + byte);
    };
#pragma unroll
    for (int p = 0; p < FULL; ++p) lds_dma16(rs, dst + 1024u * p, src(64 * p + lane, 0), soff);
#pragma unroll
    for (int t = 0; t < TAIL; ++t) {
        const int d = 64 * t + lane;
        lds_dma4(rs, dst + 1024u * FULL + 256u * t, src(64 * FULL + d / 4, 4 * (d & 3)), soff);
    }
}

template <int NB, int MR>
__global__ __launch_bounds__(64 * kShotWaves) void kq_shot_kernel(StreamArgs a_) {
    static_assert(NB == 8 || NB == 16, "one super-block column per wave and tile");
    static_assert(MR == 8 || MR == 16 || MR == 32, "8, 16 or 32 activation rows");
    constexpr int MB = MR > 16 ? MR / 16 : 1;  // 16-row blocks of the MFMA
    constexpr int UPW = NB == 16 ? 2 : 1;  // units per wave at most
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const KArgs A = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = kq_lane(), r = lane & 15, g = lane >> 4;
    // Every argument the kernel reads, loaded at entry and held in SGPRs:
    // independent scalar loads at fixed offsets issue together (one round
    // trip), and each tile's problem is picked by scalar selects.  (Left to
    // itself, the compiler moved the problems' loads behind the branches that
    // pick them: a chain of scalar-cache misses ahead of the first vector load.)
    uint64_t aw[kStreamProblems], ay[kStreamProblems];
    int64_t ays[kStreamProblems];
    uint32_t awb[kStreamProblems], arb[kStreamProblems];
    int32_t an[kStreamProblems], ac[kStreamProblems], tb[kStreamProblems];
#pragma unroll
    for (int i = 0; i < kStreamProblems; ++i) {
        aw[i] = (uint64_t)(uintptr_t)A->p[i].w;
        ay[i] = (uint64_t)(uintptr_t)A->p[i].y;
        ays[i] = A->p[i].y_stride;
        awb[i] = A->p[i].w_bytes;
        arb[i] = A->p[i].row_bytes;
        an[i] = A->p[i].N;
        ac[i] = A->p[i].codec;
        tb[i] = A->tile_begin[i];
    }
    int P = A->pairs, M = A->M, xstride = (int)A->x_stride, K = A->K;
    uint64_t xb = (uint64_t)(uintptr_t)A->x;
    asm volatile("" : "+s"(P), "+s"(M), "+s"(xstride), "+s"(K), "+s"(xb));
    StreamProblem all[kStreamProblems];
#pragma unroll
    for (int i = 0; i < kStreamProblems; ++i) {
        asm volatile("" : "+s"(aw[i]), "+s"(ay[i]), "+s"(ays[i]), "+s"(awb[i]), "+s"(arb[i]), "+s"(an[i]), "+s"(ac[i]),
                     "+s"(tb[i]));
        all[i].w = (const uint8_t *)(uintptr_t)aw[i];
        all[i].y = (void *)(uintptr_t)ay[i];
        all[i].y_stride = ays[i];
        all[i].w_bytes = awb[i];
        all[i].row_bytes = arb[i];
        all[i].N = an[i];
        all[i].codec = ac[i];
    }
    const int b = (int)blockIdx.x;
    const int nt = b < P ? 2 : 1;
    const int t0 = b < P ? 2 * b : P + b;
    // the workgroup's tiles: problem, first row, codec
    StreamProblem pr[2];
    int32_t begin[2];
    bool q6[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = j < nt ? t0 + j : t0;
        const int pi = (t >= tb[1]) + (t >= tb[2]) + (t >= tb[3]);  // unused entries: INT_MAX
        pr[j] = all[0];
        begin[j] = tb[0];
#pragma unroll
        for (int i = 1; i < kStreamProblems; ++i)
            if (pi == i) {
                pr[j] = all[i];
                begin[j] = tb[i];
            }
        q6[j] = pr[j].codec == KQ_CODEC_Q6_K;
    }
    const int cb0 = shot_col_bytes(q6[0] ? KQ_CODEC_Q6_K : KQ_CODEC_Q4_K);
    const int cb1 = nt > 1 ? shot_col_bytes(q6[1] ? KQ_CODEC_Q6_K : KQ_CODEC_Q4_K) : 0;
    const uint32_t region = (uint32_t)(uintptr_t)(LDSP(void))smem + (uint32_t)(wave * shot_region(NB, cb0, cb1));
    // the wave's units: (tile uj[i], super-block kb)
    const int kb = NB == 16 ? wave : wave % NB;
    int uj[UPW];
    bool live[UPW], uq6[UPW];
    uint32_t ucol[UPW];
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
        uj[i] = NB == 16 ? i : wave / NB;
        live[i] = uj[i] < nt;
        uq6[i] = uj[i] == 1 ? q6[1] : q6[0];
        ucol[i] = region + kShotSlab + (uint32_t)(NB == 16 && i == 1 ? cb0 : 0);
    }
    const bool any = live[0];

    // ---- loads: the activation slab of super-block kb (rows 0..7), then the
    // columns; 16-row launches copy rows 8..15 into the same slab once lanes
    // 0..7 hold their fragments (two slabs would not fit beside the columns)
    const uint32_t xbytes = (uint32_t)(((int64_t)(M - 1) * xstride + K) * 2);
    const __amdgpu_buffer_rsrc_t xs = kq_buffer((const void *)(uintptr_t)xb, xbytes);
    auto copy_slab = [&](int m0) {
#pragma unroll
        for (int i = 0; i < kShotRows / 2; ++i) {
            const int m = m0 + 2 * i + (lane >> 5), c = (lane & 31) ^ (m & 7);
            const uint32_t off =
                m < M ? (uint32_t)m * (uint32_t)xstride * 2u + (uint32_t)(kb * 512 + 16 * c) : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xs, (LDSP(void))(uintptr_t)(region + 1024u * i), 16, off, 0, 0, 0);
        }
    };
    if (any) {
        copy_slab(0);
#pragma unroll
        for (int i = 0; i < UPW; ++i) {
            if (!live[i]) continue;
            // (selects, not array indices: a runtime index puts the arrays in scratch)
            const bool u1 = uj[i] == 1;
            const StreamProblem &pj = u1 ? pr[1] : pr[0];
            const int row0 = (t0 + uj[i] - (u1 ? begin[1] : begin[0])) * 16;
            const int rlast = min(15, pj.N - 1 - row0);
            const __amdgpu_buffer_rsrc_t rs = kq_buffer(pj.w, pj.w_bytes);
            const uint32_t soff = (uint32_t)row0 * pj.row_bytes;
            if (u1 ? q6[1] : q6[0])
                shot_copy_col<KQ_CODEC_Q6_K, NB>(rs, ucol[i], pj.row_bytes, (uint32_t)(kb * Geo<KQ_CODEC_Q6_K>::BPB),
                                                 rlast, soff, lane);
            else
                shot_copy_col<KQ_CODEC_Q4_K, NB>(rs, ucol[i], pj.row_bytes, (uint32_t)(kb * Geo<KQ_CODEC_Q4_K>::BPB),
                                                 rlast, soff, lane);
        }
    }
    // epilogue parameters ahead of the wait (held in registers)
    const bool has_xe = A->x_exp != nullptr;
    int ydt = A->y_dtype;
    asm volatile("" : "+s"(ydt));
    // ---- the activation fragments of block 0 (rows 0..15)
    const uint32_t xrow = region + (uint32_t)((r & 7) * 512);
    const int sw = r & 7;
    const bool use4 = (live[0] && !uq6[0]) || (UPW > 1 && live[UPW - 1] && !uq6[UPW - 1]);
    const bool use6 = (live[0] && uq6[0]) || (UPW > 1 && live[UPW - 1] && uq6[UPW - 1]);
    half8_t x4[1][8], x6[1][8];
    floatx4 xsum = fzero4();
    u32x4 cin[1][8];
    Q4Consts q4k;
    // 32-row launches: a wave's units share one codec (the host declines
    // workgroups that pair a Q4_K tile with a Q6_K one), so one register set
    // holds either codec's fragments (the Q4_K runs, or the Q6_K fragments)
    [[maybe_unused]] u32x4 xr[1][8];
    // the lane's raw fragments from the slab (lanes of rows 8..15 of a 16-row
    // block take theirs from the block's second pass)
    auto read_slab = [&](bool mine) {
        if constexpr (MR > 16) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int ch = use6 ? 4 * i + g : 8 * g + 4 * (i & 1) + (i >> 1);
                const u32x4 v = lds128(xrow + 16u * (uint32_t)(ch ^ sw));
                xr[0][i] = mine ? v : xr[0][i];
            }
            return;
        }
        if (use4) {
#pragma unroll
            for (int w = 0; w < 4; ++w)
#pragma unroll
                for (int a2 = 0; a2 < 2; ++a2) {
                    const u32x4 v = lds128(xrow + 16u * (uint32_t)((8 * g + 4 * a2 + w) ^ sw));
                    cin[0][2 * w + a2] = mine ? v : cin[0][2 * w + a2];
                }
        }
        if (use6) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const u32x4 v = lds128(xrow + 16u * (uint32_t)((4 * t + g) ^ sw));
                x6[0][t] = mine ? __builtin_bit_cast(half8_t, v) : x6[0][t];
            }
        }
    };
    if (any) {
        int col_loads = 0;  // loads issued after the slab (they return in order)
#pragma unroll
        for (int i = 0; i < UPW; ++i) col_loads += live[i] ? (uq6[i] ? 6 : 3) : 0;
        wait_tiles_left<1, 12>(col_loads);
        read_slab(true);
        if constexpr (MR >= 16) {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the first pass's reads are done
            copy_slab(8);
            __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));  // (the columns too: they were issued first)
            read_slab(r >= 8);
        }
        q4k = q4own_consts(g);
    }
    // ---- per 16-row block (two for 32-row launches: rows 16..31 are copied
    // into the slab once block 0's partial tiles have been summed, then the
    // columns are read and decoded again): math on the wave's units, the
    // partial tiles into its region, one barrier, the sums.  The activation
    // part (fragment permutes, the Q4_K sub-block sums) runs as soon as the
    // slab has landed, while the columns (issued after it) are in flight.
    constexpr int RB = MR < 16 ? MR : 16;  // rows per block
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        // (the scheduler would otherwise mix the blocks' live ranges: spills)
        __builtin_amdgcn_sched_barrier(0);
        if (any) {
            if (mb >= 1) {
                copy_slab(16 * mb);
                __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));
                read_slab(true);
                __builtin_amdgcn_s_waitcnt(0xC07F);
                copy_slab(16 * mb + 8);
                __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));
                read_slab(r >= 8);
            }
            const Iq2Tables &no_tab = *IqTables<KQ_CODEC_Q4_K>::get();
            floatx4 acc[UPW];
#pragma unroll
            for (int i = 0; i < UPW; ++i) acc[i] = fzero4();
            // the lane's row, opaque per block: left to itself, the compiler kept
            // its products live across the blocks and spilled them
            int r = lane & 15;
            asm volatile("" : "+v"(r));
            if constexpr (MR > 16) {
                // one codec per wave: the branch keeps one fragment set live
                if (use6) {
                    half8_t xf[1][8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) xf[0][t] = __builtin_bit_cast(half8_t, xr[0][t]);
                    __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));  // the columns
#pragma unroll
                    for (int i = 0; i < UPW; ++i)
                        if (live[i])
                            mma_slab<KQ_CODEC_Q6_K, 1>(acc[i], ucol[i] + (uint32_t)(r * 240), xf, xsum, g, no_tab);
                } else {
                    q4own_x<1>(x4, xsum, xr, lane);
                    __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));  // the columns
#pragma unroll
                    for (int i = 0; i < UPW; ++i)
                        if (live[i])
                            q4own_slab<1>(acc[i], (LDSP(const uint8_t))(uintptr_t)(ucol[i] + (uint32_t)(r * 144)), x4,
                                          xsum, q4k);
                }
            } else {
                if (use4) q4own_x<1>(x4, xsum, cin, lane);
                __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));  // the columns
#pragma unroll
                for (int i = 0; i < UPW; ++i) {
                    if (!live[i]) continue;
                    if (uq6[i])
                        mma_slab<KQ_CODEC_Q6_K, 1>(acc[i], ucol[i] + (uint32_t)(r * 240), x6, xsum, g, no_tab);
                    else
                        q4own_slab<1>(acc[i], (LDSP(const uint8_t))(uintptr_t)(ucol[i] + (uint32_t)(r * 144)), x4,
                                      xsum, q4k);
                }
            }
            kq_mfma_drain();
            // block rows 4 g + e < RB live in lanes g < RB / 4; partial of tile j
            // at region + 64 RB j (in the slab, whose fragments are in registers)
#pragma unroll
            for (int i = 0; i < UPW; ++i)
                if (live[i] && g < RB / 4)
                    *(LDSP(floatx4))(uintptr_t)(region + (uint32_t)(64 * RB) * (uint32_t)uj[i] + 16u * lane) = acc[i];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // ---- tile j: threads 16 RB j .. 16 RB j + 16 RB - 1, output (m, n) =
        // (16 mb + (t >> 4), t & 15) of the tile, summed over its super-blocks in order
        int tid = (int)threadIdx.x;
        asm volatile("" : "+v"(tid));  // (recomputed per block, as r above)
        const int j = tid / (16 * RB), tt = tid % (16 * RB);
        if (j < nt) {
            const int mr = tt >> 4, n = tt & 15, m = 16 * mb + mr;
            const uint32_t at =
                (uint32_t)(64 * RB) * (uint32_t)j + 16u * (uint32_t)((mr >> 2) * 16 + n) + 4u * (uint32_t)(mr & 3);
            const uint32_t rb = (uint32_t)shot_region(NB, cb0, cb1);
            const uint32_t base = (uint32_t)(uintptr_t)(LDSP(void))smem + at;
            float sum = 0.f;
#pragma unroll
            for (int k = 0; k < NB; ++k) {
                const int w = (j * NB + k) & (kShotWaves - 1);  // the wave holding unit (j, k)
                const float v = *(const LDSP(float))(uintptr_t)(base + (uint32_t)w * rb);
                sum = k == 0 ? v : sum + v;
            }
            const StreamProblem &p = j == 0 ? pr[0] : pr[1];
            const int col = (t0 + j - (j == 0 ? begin[0] : begin[1])) * 16 + n;
            if (m < M && col < p.N) {
                if (has_xe) sum = ldexpf(sum, A->x_exp[m]);
                kq_store_out(p.y, ydt, (int64_t)m * p.y_stride + col, sum);
            }
        }
        if (mb + 1 < MB) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_barrier();  // the partial tiles are read: the slab is free
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

template <int NB, int MR>
int launch_shot(const StreamArgs &a, int grid, size_t lds, hipStream_t s) {
    static bool raised = false;
    if (!raised) {
        if (hipFuncSetAttribute((const void *)kq_shot_kernel<NB, MR>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024) != hipSuccess)
            return KQ_ERR_LAUNCH_FAILED;
        raised = true;
    }
    hipLaunchKernelGGL((kq_shot_kernel<NB, MR>), dim3(grid), dim3(64 * kShotWaves), lds, s, a);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

// ---- Mid-batch streaming kernel (17..64 rows) -------------------------------
// Work units: a group of up to C (six) consecutive 16-row weight tiles of one
// problem against one K slice (split launches cut K in S slices; unit u is
// group u mod groups, slice u / groups, so the CUs walk one slice of the
// activations at a time).  One workgroup per CU walks its units with K in
// stages of one super-block.  kMmsProducers waves copy each stage into a ring
// of R stage buffers in LDS with direct-to-LDS loads: the stage's activation
// rows (two 512-byte rows per 1 KB load, their 16-byte chunks XOR-swizzled by
// row so the consumers' fragment reads of 16 rows hit different banks) and the
// group's weight rows of that super-block (RCW chunks per row: odd, so the 16
// rows of a tile start in different banks).  Consumer c owns tile c of the
// unit and accumulates its MT 16-row blocks of activations on MFMA, reading
// every activation byte from HBM / L2 once per CU and unit.  Unsplit launches
// store the results; split ones write the unit's partial tile, and the last
// of a tile's S arrivals sums the S partials in slice order (deterministic)
// and stores.  The weight views are kq_mma.h's Block<> (exact integer
// fragments, the block's chain folded in with d), the activation fragments
// x[32 t + 8 g .. +7] of rows 16 m + r.  The Q4_K minimum term needs the
// stage's activation sub-block sums: producer wave p (p < MT) computes those
// of 16-row block p from the stage in LDS (eight selection MFMAs; the
// producers are otherwise idle between copies) into one of two LDS buffers
// (stage parity), and the consumers add -dmin m_j S_j of stage b on the fp32
// MFMA after the next barrier they pass anyway (stage b + 1's); the last
// stage of a unit takes one extra barrier before the unit's results leave.  The Q4_K + Q6_K form (q|k|v)
// lays each stage out for the larger Q6_K rows and picks the codec per unit.
constexpr int kMmsProducers = 4;
constexpr int kMmsTiles = 6;  // tiles per group: consumers
constexpr int kMmsMaxSplit = 16;

// Chunks per super-block and per LDS weight row of a codec.
__host__ __device__ constexpr int mms_cpb(int codec) { return codec == KQ_CODEC_Q6_K ? 14 : 9; }
__host__ __device__ constexpr int mms_rcw(int codec) { return mms_cpb(codec) | 1; }

template <int CODEC, int MT, int C>
struct MmsGeo {
    static constexpr int RCW = mms_rcw(CODEC == KQ_MIX ? KQ_CODEC_Q6_K : CODEC);  // largest row of the form
    static constexpr int XL = MT * 8;                                             // activation loads per stage
    static constexpr int WL = (C * 16 * RCW + 63) / 64;                           // weight loads per stage
    static constexpr int PL = (XL + WL + kMmsProducers - 1) / kMmsProducers;     // loads per producer
    static constexpr int XB = MT * 16 * 512;                                      // activation bytes per stage
    static constexpr int SB = XB + WL * 1024;                                     // stage bytes
    // Q4_K forms: the stage's activation sub-block sums, float2 per lane per
    // 16-row block (sub-blocks 2g, 2g + 1 of the lane's row), after the ring
    static constexpr bool SUMS = CODEC != KQ_CODEC_Q6_K && MT == 4;
    // two-block forms: the minimum term as a second MFMA chain against the
    // integer minimums (mms_tile_stage), no sums
    static constexpr bool MINC = CODEC != KQ_CODEC_Q6_K && MT != 4;
    static constexpr int SUMB = SUMS ? 2 * MT * 64 * 8 : 0;  // two stages (parity)
};

// Unit u of a launch: problem pi, its tiles t0 .. t0 + nt - 1 (global tile
// numbers), super-blocks kb0 .. kb1 - 1.  Groups: each problem's tiles in runs
// of C (its last run partial).
struct MmsUnit {
    int pi, t0, nt, kb0, kb1;
};

__device__ __forceinline__ int mms_ngroups(KArgs A, int C) {
    int ng = 0;
    for (int i = 0; i < A->n_problems; ++i)
        ng += ((i + 1 < A->n_problems ? A->tile_begin[i + 1] : A->total_tiles) - A->tile_begin[i] + C - 1) / C;
    return ng;
}

__device__ __forceinline__ MmsUnit mms_unit(KArgs A, int C, int ngroups, int nb, int u) {
    MmsUnit w{0, 0, 0, 0, 0};
    const int gp = u % ngroups, q = u / ngroups, S = A->split;
    w.kb0 = q * nb / S;
    w.kb1 = (q + 1) * nb / S;
    int gb = 0;
    for (int i = 0; i < A->n_problems; ++i) {
        const int tb = A->tile_begin[i];
        const int te = i + 1 < A->n_problems ? A->tile_begin[i + 1] : A->total_tiles;
        const int ng = (te - tb + C - 1) / C;
        if (gp >= gb && gp < gb + ng) {
            w.pi = i;
            w.t0 = tb + (gp - gb) * C;
            w.nt = min(C, te - w.t0);
        }
        gb += ng;
    }
    return w;
}

inline int mms_groups_host(const int32_t *tile_begin, int n, int total, int C) {
    int ng = 0;
    for (int i = 0; i < n; ++i) ng += ((i + 1 < n ? tile_begin[i + 1] : total) - tile_begin[i] + C - 1) / C;
    return ng;
}

// The producers' place in their unit walk: the unit and its next super-block.
struct MmsCursor {
    int u, kb, kb1;
    uint32_t bpb;  // weight bytes per super-block of the unit's codec
};

// A producer's per-lane offsets for a unit: activation loads (rows 2 li,
// 2 li + 1; lane l: row 2 li + l / 32, LDS chunk l % 32 holding activation
// chunk (l % 32) ^ (row % 16)), weight loads (chunk f = 64 (li - XL) + l of
// the stage's [tile][row][rcw chunks] block; rows past N clamped, pads, tiles
// past the unit and chunks past the codec's part of the stage past the buffer).
template <int CODEC, int MT, int C>
__device__ __forceinline__ void mms_setup(KArgs A, const MmsUnit &w, int wave, int lane, int M,
                                          uint32_t (&o)[MmsGeo<CODEC, MT, C>::PL], StreamProblem &pr,
                                          uint32_t &bpb) {
    using MG = MmsGeo<CODEC, MT, C>;
    constexpr int NL = MG::XL + MG::WL;
    int32_t begin;
    pr = problem_at(A, w.pi, begin);
    const bool q6 = CODEC == KQ_CODEC_Q6_K || (CODEC == KQ_MIX && pr.codec == KQ_CODEC_Q6_K);
    const int cpb = q6 ? mms_cpb(KQ_CODEC_Q6_K) : mms_cpb(KQ_CODEC_Q4_K);
    const int rcw = q6 ? mms_rcw(KQ_CODEC_Q6_K) : mms_rcw(KQ_CODEC_Q4_K);
    bpb = q6 ? Geo<KQ_CODEC_Q6_K>::BPB : Geo<KQ_CODEC_Q4_K>::BPB;
    const uint32_t row0 = (uint32_t)(w.t0 - begin) * 16, last = (uint32_t)pr.N - 1, rb = pr.row_bytes;
#pragma unroll
    for (int i = 0; i < MG::PL; ++i) {
        const int li = min(wave + kMmsProducers * i, NL - 1);
        if (li < MG::XL) {
            const int row = 2 * li + (lane >> 5);
            const int ch = (lane & 31) ^ (row & 15);
            o[i] = row < M ? (uint32_t)(row * A->x_stride * 2 + 16 * ch) : 0x80000000u;
        } else {
            const int f = 64 * (li - MG::XL) + lane;
            const int tile = f / (16 * rcw), rem = f - tile * (16 * rcw);
            const int row = rem / rcw, ck = rem - row * rcw;
            const uint32_t rr = min(row0 + (uint32_t)(tile * 16 + row), last);
            const uint32_t src = q6 ? (uint32_t)Geo<KQ_CODEC_Q6_K>::src(ck) : (uint32_t)(16 * ck);
            o[i] = ck < cpb && tile < w.nt ? rr * rb + src : 0x80000000u;
        }
    }
}

// Copy stage j (the cursor's next super-block) into ring slot j % R; moves
// to the workgroup's next unit when the current one is done.
template <int CODEC, int MT, int C, int R>
__device__ __forceinline__ void mms_copy(KArgs A, int j, int wave, int lane, int M, int ngroups, int nb,
                                         uint32_t ring, uint32_t xbytes, uint32_t (&o)[MmsGeo<CODEC, MT, C>::PL],
                                         StreamProblem &pr, MmsCursor &cur) {
    using MG = MmsGeo<CODEC, MT, C>;
    constexpr int NL = MG::XL + MG::WL;
    if (cur.kb == cur.kb1) {
        cur.u += (int)gridDim.x;
        const MmsUnit w = mms_unit(A, C, ngroups, nb, cur.u);
        mms_setup<CODEC, MT, C>(A, w, wave, lane, M, o, pr, cur.bpb);
        cur.kb = w.kb0;
        cur.kb1 = w.kb1;
    }
    const int kb = cur.kb++;
    const __amdgpu_buffer_rsrc_t ws = kq_buffer(pr.w, pr.w_bytes);
    const __amdgpu_buffer_rsrc_t xs = kq_buffer(A->x, xbytes);
    const uint32_t base = ring + (uint32_t)(j % R) * MG::SB;
#pragma unroll
    for (int i = 0; i < MG::PL; ++i) {
        const int li = min(wave + kMmsProducers * i, NL - 1);
        if (li < MG::XL)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xs, (LDSP(void))(uintptr_t)(base + 1024 * li), 16, o[i],
                                                     kb * 512, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ws, (LDSP(void))(uintptr_t)(base + MG::XB + 1024 * (li - MG::XL)),
                                                     16, o[i], kb * (int)cur.bpb, 0, 0);
    }
}

// One stage of one tile: the chains P[m] = x rows 16 m .. 16 m + 15
// (super-block of the stage) . the tile's integer weight fragments (rows at
// wrow, RCW chunks apart) and the block's factor d.  Q4_K's minimum term:
// with MINC, a second chain Pm[m] = the same rows . the integer minimums
// (Block::min_frag) and its factor nd = -dmin; otherwise the B operand of
// the sums' form (-dmin m of sub-blocks 2g, 2g + 1) in b0, b1.  The caller
// folds them into its accumulators after the next barrier, when the chains
// have long completed.
template <int CODEC, int MT, bool MINC>
__device__ __forceinline__ void mms_tile_stage(floatx4 (&P)[MT], floatx4 (&Pm)[MT], uint32_t base, uint32_t wrow,
                                               int r, int g, const Iq2Tables &iq2_tab, float &d, float &nd, float &b0,
                                               float &b1) {
    // activation fragments one step ahead of their MFMAs (the reads of step
    // t + 1 in flight while step t multiplies)
    const uint32_t xrow = base + (uint32_t)(r * 512);
    u32x4 xq[2][MT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
        xq[0][m] = lds128(xrow + (uint32_t)(m * 8192 + 16 * ((Block<CODEC>::x_elem(0, g) / 8) ^ r)));
    Block<CODEC> blk;
    load_slot<CODEC>(blk, wrow, g);
    blk.prep(g);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        if (t < 7) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
                xq[(t + 1) & 1][m] =
                    lds128(xrow + (uint32_t)(m * 8192 + 16 * ((Block<CODEC>::x_elem(t + 1, g) / 8) ^ r)));
        }
        __builtin_amdgcn_sched_barrier(0);  // (left alone, the scheduler sinks the reads to their use)
        const half8_t wf = blk.frag(t, g, iq2_tab);
#pragma unroll
        for (int m = 0; m < MT; ++m)
            P[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, xq[t & 1][m]), wf,
                                                          t == 0 ? fzero4() : P[m], 0, 0, 0);
        if constexpr (CODEC == KQ_CODEC_Q4_K && MINC) {
            const half8_t mf = blk.min_frag(t);
#pragma unroll
            for (int m = 0; m < MT; ++m)
                Pm[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, xq[t & 1][m]), mf,
                                                               t == 0 ? fzero4() : Pm[m], 0, 0, 0);
        }
    }
    d = blk.dscale();
    if constexpr (CODEC == KQ_CODEC_Q4_K) {
        if constexpr (MINC) nd = -blk.dmin;
        else blk.min_b(g, b0, b1);
    }
}

// Producer side of the Q4_K minimum term: the sub-block sums of 16-row
// activation block m of the stage at `base` (Block<Q4_K> layout), as float2
// per lane at `dst` (element e of lane (g, r): sub-block 2g + e of row r).
__device__ __forceinline__ void mms_stage_sums(uint32_t base, int m, float2 *dst, int r, int g) {
    const uint32_t xrow = base + (uint32_t)(r * 512 + m * 8192);
    floatx4 S = fzero4();
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const half8_t xf = __builtin_bit_cast(
            half8_t, lds128(xrow + (uint32_t)(16 * ((Block<KQ_CODEC_Q4_K>::x_elem(t, g) / 8) ^ r))));
        S = __builtin_amdgcn_mfma_f32_16x16x32_f16(sum_sel(r, sum_row(t, 0)), xf, S, 0, 0, 0);
    }
    kq_mfma_drain();
    dst[kq_lane()] = float2{S[0], S[1]};
}

template <int CODEC, int MT, int C, int R>
__global__ __launch_bounds__(64 * (kMmsProducers + C)) void kq_mms_kernel(StreamArgs a_) {
    using MG = MmsGeo<CODEC, MT, C>;
    constexpr int PL = MG::PL;
    static_assert(PL * (R - 1) <= 63, "vmcnt counts at most 63 loads");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const KArgs A = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
    const Iq2Tables &iq2_tab = *IqTables<CODEC == KQ_MIX ? KQ_CODEC_Q4_K : CODEC>::get();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = kq_lane(), r = lane & 15, g = lane >> 4;
    const int M = A->M, nb = A->K / KQ_QK, S = A->split;
    const int ngroups = mms_ngroups(A, C);
    const int U = ngroups * S, G = (int)gridDim.x;
    int stages = 0;
    for (int u = (int)blockIdx.x; u < U; u += G) {
        const int q = u / ngroups;
        stages += (q + 1) * nb / S - q * nb / S;
    }
    const uint32_t ring = (uint32_t)(uintptr_t)(LDSP(void))smem;

    if (wave < kMmsProducers) {
        // ================= producers: load li = wave + kMmsProducers i of a
        // stage (activation loads first, then weight loads); a producer with
        // fewer than PL repeats its last load (the same bytes again)
        const uint32_t xbytes = (uint32_t)(((int64_t)(M - 1) * A->x_stride + A->K) * 2);
        uint32_t off[PL];  // per-lane offsets of the producer's loads (weights: for the current unit)
        StreamProblem prob;  // set by the first unit's set-up
        MmsCursor cur{(int)blockIdx.x - G, 0, 0, 0};
        // the consumers' unit walk (the extra barrier after each unit's last stage)
        [[maybe_unused]] int su = (int)blockIdx.x, unit_left = 0;
        if constexpr (MG::SUMS) {
            if (su < U) {
                const MmsUnit w = mms_unit(A, C, ngroups, nb, su);
                unit_left = w.kb1 - w.kb0;
            }
        }
        const int pre = min(R, stages);
        for (int j = 0; j < pre; ++j)
            mms_copy<CODEC, MT, C, R>(A, j, wave, lane, M, ngroups, nb, ring, xbytes, off, prob, cur);
        for (int b = 0; b < stages; ++b) {
            const int newer = min(b == 0 ? R - 1 : R - 2, stages - 1 - b);
            wait_tiles_left<PL, R - 1>(newer);
            __builtin_amdgcn_s_barrier();  // stage b to the consumers; stage b - 1 back
            if (b >= 1 && b + R - 1 < stages)
                mms_copy<CODEC, MT, C, R>(A, b + R - 1, wave, lane, M, ngroups, nb, ring, xbytes, off, prob, cur);
            if constexpr (MG::SUMS) {
                // the stage's activation sub-block sums (every stage of a
                // mixed launch: its codec is known to the consumers only),
                // read by the consumers after the next barrier
                if (wave < MT) {
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                    mms_stage_sums(ring + (uint32_t)(b % R) * MG::SB, wave,
                                   (float2 *)(smem + R * MG::SB) + ((b & 1) * MT + wave) * 64, r, g);
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                }
                if (--unit_left == 0) {
                    __builtin_amdgcn_s_barrier();  // the last stage's sums of the consumers' unit
                    su += G;
                    if (su < U) {
                        const MmsUnit w = mms_unit(A, C, ngroups, nb, su);
                        unit_left = w.kb1 - w.kb0;
                    }
                }
            }
        }
        return;
    }

    // ================= consumer c: tile c of each unit
    const int c = wave - kMmsProducers;
    const bool has_xe = A->x_exp != nullptr;
    int ydt = A->y_dtype;
    uint64_t part_b = (uint64_t)(uintptr_t)A->part, ctr_b = (uint64_t)(uintptr_t)A->ctr;
    asm volatile("" : "+s"(ydt), "+s"(part_b), "+s"(ctr_b));
    float *const part = (float *)(uintptr_t)part_b;
    uint32_t *const ctr0 = (uint32_t *)(uintptr_t)ctr_b;
    // arrival counters spread over the counter region (up to one per 128-byte line)
    const int cstride = min(32, 1 << (31 - __builtin_clz((int)(KQ_MATMUL_COUNTER_BYTES / 4) / max(A->total_tiles, 1))));
    int j = 0;
    for (int u = (int)blockIdx.x; u < U; u += G) {
        const MmsUnit w = mms_unit(A, C, ngroups, nb, u);
        int32_t begin;
        const StreamProblem pr = problem_at(A, w.pi, begin);
        const bool q6 = CODEC == KQ_CODEC_Q6_K || (CODEC == KQ_MIX && pr.codec == KQ_CODEC_Q6_K);
        const uint32_t pitch = (uint32_t)(q6 ? mms_rcw(KQ_CODEC_Q6_K) : mms_rcw(KQ_CODEC_Q4_K)) * 16;
        floatx4 acc[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = floatx4{0, 0, 0, 0};
        // The previous stage's chains, folded in after the next barrier (the
        // MFMAs have completed by then); Q4_K: its minimum term too, whose
        // sums the producers wrote during that stage
        floatx4 P[MT], Pm[MT];
        float pd = 0.f, pnd = 0.f;
        [[maybe_unused]] float pb0 = 0.f, pb1 = 0.f;
        bool pending = false;
        [[maybe_unused]] bool pmin = false;
        auto fold_prev = [&](int stage) {
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[m] = fold4(pd, P[m], acc[m]);
            if constexpr (MG::MINC) {
                if (pmin) {
#pragma unroll
                    for (int m = 0; m < MT; ++m) acc[m] = fold4(pnd, Pm[m], acc[m]);
                }
            }
            if constexpr (MG::SUMS) {
                if (pmin) {
                    const float2 *sums = (const float2 *)(smem + R * MG::SB) + (stage & 1) * MT * 64;
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const float2 sv = sums[m * 64 + lane];
                        acc[m] = min_accumulate(sv.x, sv.y, pb0, pb1, acc[m]);
                    }
                }
            }
        };
        for (int kb = w.kb0; kb < w.kb1; ++kb, ++j) {
            __builtin_amdgcn_s_barrier();  // stage j has landed (and stage j - 1's sums)
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            if (pending) fold_prev(j - 1);
            const uint32_t base = ring + (uint32_t)(j % R) * MG::SB;
            if (c < w.nt) {
                const uint32_t wrow = base + MG::XB + (uint32_t)(c * 16 + r) * pitch;
                if constexpr (CODEC == KQ_MIX) {
                    if (q6)
                        mms_tile_stage<KQ_CODEC_Q6_K, MT, false>(P, Pm, base, wrow, r, g, iq2_tab, pd, pnd, pb0, pb1);
                    else
                        mms_tile_stage<KQ_CODEC_Q4_K, MT, MG::MINC>(P, Pm, base, wrow, r, g, iq2_tab, pd, pnd, pb0,
                                                                     pb1);
                } else {
                    mms_tile_stage<CODEC, MT, MG::MINC>(P, Pm, base, wrow, r, g, iq2_tab, pd, pnd, pb0, pb1);
                }
                kq_mfma_drain();
            }
            pending = c < w.nt;
            pmin = pending && !q6;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // stage reads done
        }
        if constexpr (MG::SUMS) {
            __builtin_amdgcn_s_barrier();  // the unit's last sums
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        }
        if (pending) fold_prev(j - 1);
        kq_mfma_drain();
        if constexpr (MG::SUMS) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (c >= w.nt) continue;
        const int tile = w.t0 + c;
        const int nn = (tile - begin) * 16 + r;
        if (S == 1) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = 16 * m + 4 * g + e;
                    if (row < M && nn < pr.N) {
                        float v = acc[m][e];
                        if (has_xe) v = ldexpf(v, A->x_exp[row]);
                        kq_store_out(pr.y, ydt, (int64_t)row * pr.y_stride + nn, v);
                    }
                }
            continue;
        }
        // Split launches: the unit's partial tile out ([m][e][lane] floats),
        // then one arrival on the tile's counter; the last of its S arrivals
        // sums the S partials in slice order, stores, and clears the count
        // for the next call.  The partials move by agent-scope stores and
        // loads (coherent across the XCDs' L2s by themselves); the stores
        // have completed (vmcnt 0) before the arrival is counted, and the
        // loads issue only after the count returns.
        const int q = u / ngroups;
        // (an opaque lane offset: left alone, the compiler hoists these
        // addresses out of the stage loop and holds them in registers)
        int lo = lane;
        asm volatile("" : "+v"(lo));
        float *const pq = part + ((size_t)tile * S + q) * (MT * 256) + lo;
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (16 * m < M)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    __hip_atomic_store(pq + m * 256 + e * 64, acc[m][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));
        uint32_t *const ctr = ctr0 + tile * cstride;
        uint32_t prev = 0;
        if (lane == 0) prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = (uint32_t)__builtin_amdgcn_readfirstlane((int)prev);
        if (prev != (uint32_t)(S - 1)) continue;
        if (lane == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // the partials of four slices at a time in flight (one load of each
        // after another would wait out a round trip per load), summed in
        // slice order
        const float *const pt = part + (size_t)tile * S * (MT * 256) + lo;
        floatx4 sum[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) sum[m] = floatx4{0, 0, 0, 0};
        for (int s0 = 0; s0 < S; s0 += 4) {
            floatx4 v[4][MT];
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[d][m][e] = s0 + d < S && 16 * m < M
                                         ? __hip_atomic_load(pt + (s0 + d) * (MT * 256) + m * 256 + e * 64,
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                         : 0.f;
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int m = 0; m < MT; ++m) sum[m] += v[d][m];
        }
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = 16 * m + 4 * g + e;
                if (row < M && nn < pr.N) {
                    float y = sum[m][e];
                    if (has_xe) y = ldexpf(y, A->x_exp[row]);
                    kq_store_out(pr.y, ydt, (int64_t)row * pr.y_stride + nn, y);
                }
            }
    }
}

template <int CODEC, int MT, int C>
int launch_mms(const StreamArgs &a, int grid, hipStream_t s) {
    using MG = MmsGeo<CODEC, MT, C>;
    constexpr size_t budget = 160 * 1024;
    constexpr int R0 = (budget - MG::SUMB) / MG::SB > 4 ? 4 : (int)((budget - MG::SUMB) / MG::SB);
    constexpr int R = MG::PL * (R0 - 1) <= 63 ? R0 : 63 / MG::PL + 1;
    static_assert(R >= 2, "mid-batch stream kernel LDS");
    constexpr size_t lds = (size_t)R * MG::SB + MG::SUMB;
    static bool raised = false;
    if (!raised) {
        if (hipFuncSetAttribute((const void *)kq_mms_kernel<CODEC, MT, C, R>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
            return KQ_ERR_LAUNCH_FAILED;
        raised = true;
    }
    hipLaunchKernelGGL((kq_mms_kernel<CODEC, MT, C, R>), dim3(grid), dim3(64 * (kMmsProducers + C)), lds, s, a);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

template <int CODEC>
int launch_mms_rows(const StreamArgs &a, int grid, hipStream_t s) {
    return a.M <= 32 ? launch_mms<CODEC, 2, kMmsTiles>(a, grid, s) : launch_mms<CODEC, 4, kMmsTiles>(a, grid, s);
}

// K slices of a launch: the split that leaves the fewest stages per CU
// (rounds of units over the CUs, times the super-blocks of a slice plus, for
// a split launch, about one stage's worth of partial tiles).  GMLX_KQ_MMS_S
// forces the count (tests and tuning).
int mms_split(const kq_matmul_problem *ps, int n, int max_split) {
    const int nb = ps[0].K / KQ_QK, cus = device_cus();
    int32_t tb[KQ_MAX_GROUP];
    int tiles = 0;
    for (int i = 0; i < n; ++i) {
        tb[i] = tiles;
        tiles += (ps[i].N + 15) / 16;
    }
    const int ng = mms_groups_host(tb, n, tiles, kMmsTiles);
    const int smax = min(min(max_split, kMmsMaxSplit), nb);
    if (const char *e = getenv("GMLX_KQ_MMS_S")) {
        const int s = atoi(e);
        return s >= 1 && s <= smax ? s : 1;
    }
    int64_t best = -1;
    int split = 1;
    for (int s = 1; s <= smax; ++s) {
        const int64_t cost = (int64_t)((ng * s + cus - 1) / cus) * ((nb + s - 1) / s + (s > 1));
        if (best < 0 || cost < best) {
            best = cost;
            split = s;
        }
    }
    return split;
}

}  // namespace

namespace {

// The shapes the kernel serves: 17..64 rows of fp16 activations (16-byte
// aligned rows), one codec (Q4_K or Q6_K) or Q4_K with Q6_K, at most 4
// problems sharing x / stride / M / K, weights and x addressable with 31-bit
// buffer offsets.
bool mms_shape_ok(const kq_matmul_problem *ps, int n) {
    if (n <= 0 || n > kStreamProblems) return false;
    const kq_matmul_problem &q0 = ps[0];
    if (q0.M < 17 || q0.M > 64 || q0.K % KQ_QK || q0.K < KQ_QK) return false;
    // 16-byte activation pieces: x and its row stride 16-byte aligned
    if (((uintptr_t)q0.x & 15) != 0 || q0.x_row_stride % 8 != 0) return false;
    for (int i = 0; i < n; ++i) {
        const kq_matmul_problem &q = ps[i];
        if (q.codec != KQ_CODEC_Q4_K && q.codec != KQ_CODEC_Q6_K) return false;
        if (q.x != q0.x || q.x_row_stride != q0.x_row_stride || q.M != q0.M || q.K != q0.K) return false;
        if ((int64_t)(q.N + 16) * q.w_row_bytes >= (int64_t)0x80000000LL) return false;
    }
    if ((int64_t)(q0.M - 1) * q0.x_row_stride * 2 + (int64_t)q0.K * 2 >= (int64_t)0x80000000LL) return false;
    return true;
}

int64_t mms_tiles(const kq_matmul_problem *ps, int n) {
    int64_t tiles = 0;
    for (int i = 0; i < n; ++i) tiles += (ps[i].N + 15) / 16;
    return tiles;
}

// K slices the launch may take: split launches need one arrival counter per
// tile in the counter region (and room for the partial tiles).
int mms_max_split(const kq_matmul_problem *ps, int n, bool room) {
    return room && mms_tiles(ps, n) * 4 <= (int64_t)KQ_MATMUL_COUNTER_BYTES ? kMmsMaxSplit : 1;
}

// Routing (measured at the Qwen3-8B shapes, 17..64 rows): the kernel pays off
// when its planned units (tile groups times K slices) cover three quarters of
// the CUs or more: gate|up (256 groups, unsplit: 21.0-28.9 us against
// 29.5-44.3 for the tile kernel), the down projection (43 groups in 5 slices:
// 22.6-27.8 against 24.1-37.1), q|k|v (65 groups in 3 slices: 16.8-19.5
// against 17.1-21.4); not o (43 groups in 4 slices, 172 units: 11.5-15.6
// against 9.3-12.8).  GMLX_KQ_MMS=0 declines, =2 takes every shape it serves
// (tests).
bool mms_worth(const kq_matmul_problem *ps, int n, bool room) {
    const char *env = getenv("GMLX_KQ_MMS");
    if (env && env[0] == '0' && env[1] == 0) return false;
    if (env && env[0] == '2' && env[1] == 0) return true;
    int32_t tb[KQ_MAX_GROUP];
    int tiles = 0;
    for (int i = 0; i < n; ++i) {
        tb[i] = tiles;
        tiles += (ps[i].N + 15) / 16;
    }
    const int64_t units = (int64_t)mms_groups_host(tb, n, tiles, kMmsTiles) * mms_split(ps, n, mms_max_split(ps, n, room));
    return 4 * units >= 3 * (int64_t)device_cus();
}

}  // namespace

// Whether the mid-batch streaming kernel takes the launch (room: the
// workspace holds kq_mms_part_bytes after the counter region).
bool kq_mms_eligible(const kq_matmul_problem *ps, int n, bool room) {
    return mms_shape_ok(ps, n) && mms_worth(ps, n, room);
}

// Bytes of partial tiles the launch writes when it is taken and given room
// for them (after the counter region): MT 1 KB blocks per tile and slice.
size_t kq_mms_part_bytes(const kq_matmul_problem *ps, int n) {
    if (!kq_mms_eligible(ps, n, true)) return 0;
    const int S = mms_split(ps, n, mms_max_split(ps, n, true));
    const size_t mt = ps[0].M <= 32 ? 2 : 4;
    return S > 1 ? ((size_t)mms_tiles(ps, n) * S * mt * 1024 + 255) & ~(size_t)255 : 0;
}

// Problems validated and eligible (for this room); x fp16, x_exp its per-row
// exponents or null.  ctr / part: the arrival counters (zero on entry; left
// zero) and room for kq_mms_part_bytes, or null (no split).
int kq_mms_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, uint32_t *ctr,
                  float *part, hipStream_t s) {
    StreamArgs a;
    int tiles = 0;
    bool mixed = false;
    for (int i = 0; i < n; ++i) {
        StreamProblem &p = a.p[i];
        p.w = (const uint8_t *)ps[i].w;
        p.y = ps[i].y;
        p.y_stride = ps[i].y_row_stride;
        p.row_bytes = (uint32_t)ps[i].w_row_bytes;
        p.w_bytes = (uint32_t)(ps[i].N * ps[i].w_row_bytes);
        p.N = ps[i].N;
        p.codec = ps[i].codec;
        a.tile_begin[i] = tiles;
        tiles += (ps[i].N + 15) / 16;
        if (ps[i].codec != ps[0].codec) mixed = true;
    }
    for (int i = n; i < KQ_MAX_GROUP; ++i) {
        a.p[i] = a.p[0];
        a.tile_begin[i] = 0x7FFFFFFF;
    }
    const kq_matmul_problem &q0 = ps[0];
    const int S = mms_split(ps, n, mms_max_split(ps, n, ctr && part));
    a.x = (const char *)q0.x;
    a.x_exp = x_exp;
    a.ctr = S > 1 ? ctr : nullptr;
    a.part = S > 1 ? part : nullptr;
    a.x_stride = q0.x_row_stride;
    a.M = q0.M;
    a.K = q0.K;
    a.y_dtype = y_dtype;
    a.total_tiles = tiles;
    a.n_problems = n;
    a.split = S;
    const int units = mms_groups_host(a.tile_begin, n, tiles, kMmsTiles) * S;
    int grid = device_cus();
    if (const char *e = getenv("GMLX_KQ_STREAM_WGS")) {
        const int w = atoi(e);
        if (w > 0 && w < grid) grid = w;
    }
    if (grid > units) grid = units;
    if (mixed) return launch_mms_rows<KQ_MIX>(a, grid, s);
    return q0.codec == KQ_CODEC_Q6_K ? launch_mms_rows<KQ_CODEC_Q6_K>(a, grid, s)
                                     : launch_mms_rows<KQ_CODEC_Q4_K>(a, grid, s);
}

namespace {

// ---- Streaming expert gather ------------------------------------------------
// The MoE expert matmuls (kq_gather_qmm, kq_moe_glu_gather, kq_moe_gather_rows)
// on the same producer / consumer ring: a work item is one 16-row weight tile
// of one matrix (gate, up, or the plain one) of one expert, against one chunk
// of at most kSgRows (8) of the expert's routed rows (a segment of the
// route's seg_info / pair_order, cut into chunks of 8).  Items are ordered chunk,
// tile, matrix (gate before up), and each workgroup takes a contiguous range
// of (chunk, tile) pairs, so it meets few chunk changes.  The consumers load
// their activation fragments straight from the chunk's rows (fp16, gathered
// through pair_order) when the chunk changes; the producers stream each
// item's tile into the ring from its expert's matrix.  A round's partial
// tiles are summed in consumer order and the epilogue (plain bias, or the GLU
// of gate and up) writes the pairs' output rows.
struct SGatherArgs {
    const uint8_t *w0, *w1;            // expert stacks: gate (or the plain matrix), up
    const char *x;                     // fp16 activation rows
    const int32_t *x_exp;              // per-row exponents of prepared activations (results * 2^e), or null
    void *y;
    const int32_t *seg_info;           // [0] = S, seg_expert[E], seg_start[E + 1]
    const int32_t *pair_order;         // pair ids by segment, then per pair its expert or -1
    const float *b0, *b1;              // GLU biases, or the plain gather's output bias [expert][N], or null
    int64_t x_stride, w_expert_bytes, y_stride, b_stride;
    uint32_t w_row_bytes, w_bytes;     // one expert's matrix: N * row bytes (< 2^31)
    int32_t x_pair_div, x_skip, y_skip, N, K, n_pairs, n_experts, n_tiles, y_dtype, act;
    float limit, alpha;
};

typedef const __attribute__((address_space(4))) SGatherArgs *GArgs;

constexpr int kSGatherMaxSegs = 1024;  // experts per launch (the router's bound)

__device__ __forceinline__ int64_t sg_x_row(GArgs A, int pair) {
    return pair / A->x_pair_div + (A->x_skip ? pair / A->x_skip : 0);
}
__device__ __forceinline__ int64_t sg_y_row(GArgs A, int pair) {
    return pair + (A->y_skip ? pair / A->y_skip : 0);
}

constexpr int kSgRows = 8;  // activation rows per chunk (MFMA rows 0..7: lane groups 0, 1)

// TM: items per round (a multiple of NW: a gate / up pair shares its round).
// Items are small (16 rows of 3..28 super-blocks), so the ring is deep: the
// bytes in flight per CU, not the item count, set its share of the bandwidth.
// CPB: consumers per super-block (2: each takes four of its eight MFMA
// steps, for short K, where one wave per super-block left the MFMA chains
// latency-bound; not the owned Q4_K view, whose minimum term spans the block).
template <int CODEC, int SB, int C, int R, int NW, int TM, int CPB>
__global__ __launch_bounds__(64 * (kProducers + C)) void kq_sgather_kernel(SGatherArgs a_) {
    static_assert(CPB == 1 || (CPB == 2 && SB == 1 && CODEC != KQ_CODEC_Q4_K), "split super-blocks: K-quant views");
    constexpr int NB = SB * C / CPB;
    constexpr int TS = 8 / CPB;  // MFMA steps per consumer and super-block
    constexpr int PL = producer_loads<CODEC, NB>();
    constexpr int SLOTB = slot_bytes<CODEC, NB>();
    constexpr int kThreads = 64 * (kProducers + C);
    static_assert(PL <= 63, "vmcnt counts at most 63 loads");
    static_assert(TM % NW == 0, "rounds hold whole gate / up pairs");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // the route's segments in LDS: chunks before segment s, its first pair
    // position, its expert (no global loads on the per-item paths)
    __shared__ int32_t cstart[kSGatherMaxSegs + 1];
    __shared__ int32_t sbeg[kSGatherMaxSegs + 1];
    __shared__ int32_t sexp[kSGatherMaxSegs];
    __shared__ int32_t wsum[16];
    const GArgs A = (GArgs)__builtin_amdgcn_kernarg_segment_ptr();
    const Iq2Tables &iq2_tab = *IqTables<CODEC>::get();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = kq_lane(), r = lane & 15, g = lane >> 4;
    const int S = A->seg_info[0];
    const int32_t *sstart = A->seg_info + 1 + A->n_experts;
    // ---- chunk table (segment s: ceil(len / 8) chunks), a workgroup scan
    {
        const int per = (S + kThreads - 1) / kThreads;
        const int s0 = min(S, (int)threadIdx.x * per), s1 = min(S, s0 + per);
        int v = 0;
        for (int s = s0; s < s1; ++s) v += (sstart[s + 1] - sstart[s] + kSgRows - 1) / kSgRows;
        int incl = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int y = __shfl_up(incl, d, 64);
            if (lane >= d) incl += y;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int base = 0, total = 0;
        for (int w2 = 0; w2 < kProducers + C; ++w2) {
            base += w2 < wave ? wsum[w2] : 0;
            total += wsum[w2];
        }
        int acc = base + incl - v;
        for (int s = s0; s < s1; ++s) {
            cstart[s] = acc;
            sbeg[s] = sstart[s];
            sexp[s] = A->seg_info[1 + s];
            acc += (sstart[s + 1] - sstart[s] + kSgRows - 1) / kSgRows;
        }
        if (threadIdx.x == 0) {
            cstart[S] = total;
            sbeg[S] = sstart[S];
        }
        __syncthreads();
    }
    // (chunk, tile) pairs of this workgroup: [p0, p1); item j is pair p0 + j / NW, matrix j % NW
    const int G = (int)gridDim.x;
    const int pairs_total = cstart[S] * A->n_tiles;
    const int per_wg = (pairs_total + G - 1) / G;
    const int p0 = min(pairs_total, (int)blockIdx.x * per_wg), p1 = min(pairs_total, p0 + per_wg);
    const int my_items = (p1 - p0) * NW;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(LDSP(void))smem;
    floatx4 *red = (floatx4 *)(smem + R * SLOTB);  // [TM][C][32 lanes]
    auto chunk_of = [&](int j) { return (p0 + j / NW) / A->n_tiles; };
    // segment of a chunk, advancing monotonically from the previous answer
    auto seg_of = [&](int chunk, int &s) {
        while (s + 1 < S && cstart[s + 1] <= chunk) ++s;
        return s;
    };
    int s_start = 0;
    {  // first segment by bisection
        const int chunk0 = p0 / max(A->n_tiles, 1);
        int lo = 0, hi = max(S - 1, 0);
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (cstart[mid] <= chunk0) lo = mid;
            else hi = mid - 1;
        }
        s_start = lo;
    }

    if (wave < kProducers) {
        // ================= producer: item tiles into slots
        int ps = s_start;
        auto copy = [&](int j) {
            const int pt = p0 + j / NW;
            const int chunk = pt / A->n_tiles, t = pt - chunk * A->n_tiles;
            const int expert = sexp[seg_of(chunk, ps)];
            const uint8_t *wm = (NW == 2 && j % NW) ? A->w1 : A->w0;
            const __amdgpu_buffer_rsrc_t rs = kq_buffer(wm + (int64_t)expert * A->w_expert_bytes, A->w_bytes);
            const uint32_t row0 = (uint32_t)t * 16, last = (uint32_t)A->N - 1, rb = A->w_row_bytes;
            const uint32_t slot = ring_lds + (uint32_t)(j % R) * SLOTB;
#pragma unroll
            for (int i = 0; i < PL; ++i) {
                const int li = i * kProducers + wave;
                const uint32_t off = slot_src<CODEC, NB>(64 * li + lane, row0, last, rb);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (LDSP(void))(uintptr_t)(slot + 1024 * li), 16, off, 0,
                                                         0, 0);
            }
        };
        // KQ_STREAM_START_TILES items first, the rest of the ring once item 0
        // is with the consumers (every CU issuing its whole ring at once
        // delayed the first item, as in kq_stream_kernel)
        const int pre = min(min(KQ_STREAM_START_TILES, R), my_items);
        for (int j = 0; j < pre; ++j) copy(j);
        for (int b = 0; b < my_items; ++b) {
            const int newer = b == 0 ? pre - 1 : min(R - 2, my_items - 1 - b);
            wait_tiles_left<PL, (R - 1 < 63 / PL ? R - 1 : 63 / PL)>(newer);
            __builtin_amdgcn_s_barrier();  // slot b % R to the consumers; slot (b - 1) % R back
            if (b == 0) {
                for (int j = pre; j < min(R, my_items); ++j) copy(j);
            } else if (b + R - 1 < my_items) {
                copy(b + R - 1);
            }
            if ((b + 1) % TM == 0 || b + 1 == my_items) {
                __builtin_amdgcn_s_barrier();  // the round's partial tiles are in LDS
                if (b + 1 < my_items) __builtin_amdgcn_s_barrier();  // the round's outputs are stored: red is free
            }
        }
        return;
    }

    // ================= consumer c: K-slab [c SB, c SB + SB) of every item (or
    // steps t0 .. t0 + TS - 1 of super-block c / CPB)
    const int c = wave - kProducers;
    const int kb0 = (c / CPB) * SB;
    const int t0 = (c % CPB) * TS;
    constexpr int XC = CODEC;
    half8_t xr[SB][8];
    [[maybe_unused]] floatx4 xsum = fzero4();  // Q4_K: the slab's activation sub-block sums
    [[maybe_unused]] const Q4Consts q4k = q4own_consts(g);
    [[maybe_unused]] LDSP(const uint8_t) own_p =
        (LDSP(const uint8_t))smem + r * SlotGeo<KQ_CODEC_Q4_K, NB>::RC * 16 + kb0 * 144;
    int cs = s_start, es = s_start;
    int cur_chunk = -1;
    // the chunk's activation fragments of this consumer's slab, from its rows
    auto load_x = [&](int chunk) {
        const int s = seg_of(chunk, cs);
        const int seg_begin = sbeg[s], seg_len = sbeg[s + 1] - seg_begin;
        const int row0 = (chunk - cstart[s]) * kSgRows;
        const int rows = min(kSgRows, seg_len - row0);
        const bool live = r < rows;
        const int pair = A->pair_order[seg_begin + row0 + min(r, rows - 1)];
        const char *xrow = A->x + sg_x_row(A, pair) * A->x_stride * 2;
        const u32x4 zero = {0u, 0u, 0u, 0u};
        if constexpr (CODEC == KQ_CODEC_Q4_K) {
            u32x4 ch[SB][8];
#pragma unroll
            for (int s2 = 0; s2 < SB; ++s2)
#pragma unroll
                for (int w = 0; w < 4; ++w)
#pragma unroll
                    for (int a2 = 0; a2 < 2; ++a2) {
                        const u32x4 v =
                            *(const u32x4 *)(xrow + (256 * (kb0 + s2) + 64 * g + 32 * a2 + 8 * w) * 2);
                        ch[s2][2 * w + a2] = live ? v : zero;
                    }
            q4own_x<SB>(xr, xsum, ch, lane);
        } else {
#pragma unroll
            for (int s2 = 0; s2 < SB; ++s2)
#pragma unroll
                for (int i = 0; i < TS; ++i) {
                    const int elem = 256 * (kb0 + s2) + Block<XC>::x_elem(t0 + i, g);
                    const u32x4 v = *(const u32x4 *)(xrow + elem * 2);
                    xr[s2][i] = __builtin_bit_cast(half8_t, live ? v : zero);
                }
        }
    };
    // steps T0 .. T0 + TS - 1 of the consumer's super-block (CPB 2)
    auto half_slab = [&](floatx4 &acc, uint32_t row_lds, auto t0c) {
        constexpr int T0 = decltype(t0c)::value;
        Block<CODEC> blk;
        load_slot<CODEC>(blk, row_lds, g);
        blk.prep(g);
        floatx4 P;
#pragma unroll
        for (int i = 0; i < TS; ++i)
            P = __builtin_amdgcn_mfma_f32_16x16x32_f16(xr[0][i], blk.frag(T0 + i, g, iq2_tab), i == 0 ? fzero4() : P,
                                                       0, 0, 0);
        acc = fold4(blk.dscale(), P, acc);
    };
    auto slab = [&](floatx4 &acc, int gb) {
        const uint32_t slot = ring_lds + (uint32_t)(gb % R) * SLOTB;
        const uint32_t row_lds = slot + r * SlotGeo<CODEC, NB>::RC * 16 + kb0 * Geo<CODEC>::SLOT;
        if constexpr (CODEC == KQ_CODEC_Q4_K) {
            q4own_slab<SB>(acc, own_p + (gb % R) * SLOTB, xr, xsum, q4k);
        } else if constexpr (CPB == 2) {
            if (t0 == 0) half_slab(acc, row_lds, std::integral_constant<int, 0>{});  // uniform
            else half_slab(acc, row_lds, std::integral_constant<int, 4>{});
        } else {
            mma_slab<CODEC, SB>(acc, row_lds, xr, xsum, g, iq2_tab);
        }
    };
    const int n = lane & 15, mq = lane >> 4;
    // the epilogue's view of a chunk: lane l stores rows 4h + (l >> 4), h < 2;
    // their pairs and exponents are loaded once per chunk
    int ep_chunk = -1, ep_expert = 0, ep_rows = 0;
    int ep_pair[2], ep_ex[2];
    auto ep_load = [&](int chunk) {
        const int s = seg_of(chunk, es);
        const int seg_begin = sbeg[s];
        const int row0 = (chunk - cstart[s]) * kSgRows;
        ep_rows = min(kSgRows, sbeg[s + 1] - seg_begin - row0);
        ep_expert = sexp[s];
#pragma unroll
        for (int h = 0; h < 2; ++h) ep_pair[h] = A->pair_order[seg_begin + row0 + min(4 * h + mq, ep_rows - 1)];
#pragma unroll
        for (int h = 0; h < 2; ++h) ep_ex[h] = A->x_exp ? A->x_exp[sg_x_row(A, ep_pair[h])] : 0;
        ep_chunk = chunk;
    };
    const float *redf = (const float *)red;
    for (int round0 = 0; round0 < my_items; round0 += TM) {
        const int nt = min(TM, my_items - round0);
        for (int b = 0; b < nt; ++b) {
            const int gb = round0 + b;
            const int chunk = chunk_of(gb);
            if (chunk != cur_chunk) {  // uniform; before the wait, so the loads overlap the tile's
                load_x(chunk);
                cur_chunk = chunk;
            }
            __builtin_amdgcn_s_barrier();  // item gb has landed in slot gb % R
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            floatx4 acc = {0, 0, 0, 0};
            slab(acc, gb);
            kq_mfma_drain();
            if (g < 2) red[(b * C + c) * 32 + lane] = acc;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // slot reads and red writes done
        }
        __builtin_amdgcn_s_barrier();  // every partial tile of the round is in LDS
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // ---- the round's outputs: units (item pair qq, row group h < 2)
        // spread over the consumers (a unit is 4 rows x 16 columns: one value
        // per lane); the C partial tiles summed in consumer order, then the
        // epilogue.  Spreading keeps each consumer's chain of LDS reads short.
        for (int unit = c; unit < (nt / NW) * 2; unit += C) {
            const int qq = unit >> 1, h = unit & 1;
            const int b0 = qq * NW;
            const int pt = p0 + (round0 + b0) / NW;
            const int chunk = pt / A->n_tiles, t = pt - chunk * A->n_tiles;
            if (chunk != ep_chunk) ep_load(chunk);  // uniform
            const int nn = t * 16 + n;
            const int m = 4 * h + mq;
            float v[NW];
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) {
                // reads in groups of (at most) 8 in flight, summed in consumer order
                constexpr int GR = C > 8 ? 4 : C;
                float sum = 0.f;
#pragma unroll
                for (int c0 = 0; c0 < C; c0 += GR) {
                    float pv[GR];
#pragma unroll
                    for (int i = 0; i < GR; ++i)
                        pv[i] = c0 + i < C ? redf[(((b0 + w2) * C + c0 + i) * 32 + 16 * h + n) * 4 + mq] : 0.f;
#pragma unroll
                    for (int i = 0; i < GR; ++i)
                        if (c0 + i < C) sum = (c0 + i == 0) ? pv[i] : sum + pv[i];
                }
                v[w2] = sum;
            }
            if (m >= ep_rows || nn >= A->N) continue;
            const int pair = h ? ep_pair[1] : ep_pair[0];
            const int ex = h ? ep_ex[1] : ep_ex[0];
            const int64_t bo = (int64_t)ep_expert * A->b_stride + nn;
            float out;
            if constexpr (NW == 1) {
                out = ldexpf(v[0], ex);
                if (A->b0) out += A->b0[bo];
            } else {
                const bool clamp = A->act == KQ_ACT_SWIGLU_CLAMP;
                out = kq_glu(A->act, ldexpf(v[0], ex), ldexpf(v[NW - 1], ex), A->limit, A->alpha,
                             clamp && A->b0 ? A->b0[bo] : 0.f, clamp && A->b1 ? A->b1[bo] : 0.f);
            }
            kq_store_out(A->y, A->y_dtype, sg_y_row(A, pair) * A->y_stride + nn, out);
        }
        if (round0 + TM < my_items) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_barrier();  // red is free for the next round
        }
    }
    // pairs whose expert id is out of range (never routed): zeros in their
    // rows, columns of tiles blockIdx.x, blockIdx.x + G, ...
    if (c == 0 && (int)blockIdx.x < A->n_tiles) {
        kq_for_unrouted(A->pair_order + A->n_pairs, A->n_pairs, [&](int p) {
            if (lane >= 16) return;
            for (int t = blockIdx.x; t < A->n_tiles; t += G) {
                const int nn = t * 16 + n;
                if (nn < A->N) kq_store_out(A->y, A->y_dtype, sg_y_row(A, p) * A->y_stride + nn, 0.f);
            }
        });
    }
}

// Items per round: 8 (a multiple of NW) down to 2, the first whose partial
// tiles leave room for a ring of four slots (three at 2); 0: no fit.  The
// ring takes the rest of the LDS, up to 16 slots.  Each round ends in a
// workgroup-wide epilogue (about 0.8 us), so rounds are as long as fits.
constexpr int sgather_tm(size_t sb, size_t budget, int C) {
    for (int tm = 8; tm >= 2; tm -= 2)
        if ((tm == 2 ? 3 : 4) * sb + (size_t)tm * C * 32 * 16 <= budget) return tm;
    return 0;
}
constexpr int sgather_ring(size_t sb, size_t red, size_t budget) {
    for (int r = 16; r >= 3; --r)
        if (r * sb + red <= budget) return r;
    return 0;
}

// dry: only report whether this form fits (KQ_OK) or not (KQ_ERR_BAD_SHAPE).
template <int CODEC, int SB, int C, int NW, int CPB = 1>
int launch_sgather(const SGatherArgs &a, hipStream_t s, bool dry) {
    constexpr int NB = SB * C / CPB;
    constexpr size_t sb = slot_bytes<CODEC, NB>();
    constexpr size_t budget = 150 * 1024 - (CODEC == KQ_CODEC_IQ2_XXS ? sizeof(Iq2Tables) : 0) -
                              (3 * kSGatherMaxSegs + 2 + 16) * 4;
    constexpr int TM = sgather_tm(sb, budget, C);
    if constexpr (TM == 0) {
        return KQ_ERR_BAD_SHAPE;
    } else {
        constexpr size_t red = (size_t)TM * C * 32 * 16;
        constexpr int R = sgather_ring(sb, red, budget);
        constexpr size_t lds = R * sb + red;
        static_assert(R >= 3 && lds <= budget, "stream gather LDS");
        if (dry) return KQ_OK;
        static bool raised = false;
        if (!raised) {
            if (hipFuncSetAttribute((const void *)kq_sgather_kernel<CODEC, SB, C, R, NW, TM, CPB>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
                return KQ_ERR_LAUNCH_FAILED;
            raised = true;
        }
        hipLaunchKernelGGL((kq_sgather_kernel<CODEC, SB, C, R, NW, TM, CPB>), dim3(device_cus()),
                           dim3(64 * (kProducers + C)), lds, s, a);
        return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
    }
}

// Consumers for K = 256 nb: one super-block each up to 12; two for 16,
// IQ2_XXS only (the K-quant views of two super-blocks, with their activation
// reload inside the loop, run out of registers; those calls keep the
// per-tile gather kernels).  Forms whose workgroup of 14 or 16 waves (a
// 128-VGPR cap) spilled to scratch decline as well: Q4_K at 12 super-blocks
// (116 / 64 bytes per lane, GLU / plain) and IQ2_XXS at 28 (184 / 80).
template <int CODEC, int NW>
int sgather_codec(const SGatherArgs &a, int nb, hipStream_t s, bool dry) {
    // up to 4 super-blocks, two consumers share each (Q6_K, IQ2_XXS)
    constexpr int CPB = CODEC == KQ_CODEC_Q4_K ? 1 : 2;
    switch (nb) {
    case 2: return launch_sgather<CODEC, 1, 2 * CPB, NW, CPB>(a, s, dry);
    case 3: return launch_sgather<CODEC, 1, 3 * CPB, NW, CPB>(a, s, dry);
    case 4: return launch_sgather<CODEC, 1, 4 * CPB, NW, CPB>(a, s, dry);
    case 6: return launch_sgather<CODEC, 1, 6, NW>(a, s, dry);
    case 8: return launch_sgather<CODEC, 1, 8, NW>(a, s, dry);
    case 12:
        if constexpr (CODEC != KQ_CODEC_Q4_K) return launch_sgather<CODEC, 1, 12, NW>(a, s, dry);
        else return KQ_ERR_BAD_SHAPE;
    case 16:
        if constexpr (CODEC == KQ_CODEC_IQ2_XXS) return launch_sgather<CODEC, 2, 8, NW>(a, s, dry);
        else return KQ_ERR_BAD_SHAPE;
    default: return KQ_ERR_BAD_SHAPE;
    }
}

int sgather_dispatch(const SGatherArgs &a, int codec, bool glu, int nb, hipStream_t s, bool dry) {
    switch (codec) {
    case KQ_CODEC_Q4_K:
        return glu ? sgather_codec<KQ_CODEC_Q4_K, 2>(a, nb, s, dry) : sgather_codec<KQ_CODEC_Q4_K, 1>(a, nb, s, dry);
    case KQ_CODEC_Q6_K:
        return glu ? sgather_codec<KQ_CODEC_Q6_K, 2>(a, nb, s, dry) : sgather_codec<KQ_CODEC_Q6_K, 1>(a, nb, s, dry);
    default:
        return glu ? sgather_codec<KQ_CODEC_IQ2_XXS, 2>(a, nb, s, dry)
                   : sgather_codec<KQ_CODEC_IQ2_XXS, 1>(a, nb, s, dry);
    }
}

int64_t group_tiles(const kq_matmul_problem *ps, int n) {
    int64_t tiles = 0;
    for (int i = 0; i < n; ++i) tiles += (ps[i].N + 15) / 16;
    return tiles;
}

// One-shot plan: the problems with Q4_K ones first (ord), the tiles, the
// workgroups holding two tiles, the grid and the LDS of the largest
// workgroup.  False when the launch is not served: more than 32 rows (16 at
// K = 2048), K not 8
// or 16 super-blocks, another codec, more than two tiles per CU, a
// workgroup past 160 KB of LDS (two Q6_K tiles at K = 4096), 31-bit offsets.
// GMLX_KQ_SHOT=0 declines every launch (tests and comparisons), and so does
// a route forced with GMLX_KQ_STREAM or GMLX_KQ_MV (tests of those kernels).
bool shot_plan(const kq_matmul_problem *ps, int n, kq_matmul_problem *ord, int &tiles, int &pairs, int &grid,
               size_t &lds) {
    if (n <= 0 || n > kStreamProblems) return false;
    const char *env = getenv("GMLX_KQ_SHOT");
    if (env && env[0] == '0' && env[1] == 0) return false;
    for (const char *forced : {"GMLX_KQ_STREAM", "GMLX_KQ_MV"}) {
        const char *e = getenv(forced);
        if (e && *e) return false;
    }
    const kq_matmul_problem &q0 = ps[0];
    // (four 16-row blocks measured slower than the mid-batch kernels at 64 rows:
    // q|k|v 20.5 against 20.4 us, o 16.0 against 14.6)
    if (q0.M < 1 || q0.M > 4 * kShotRows || q0.K % KQ_QK) return false;
    const int nb = q0.K / KQ_QK;
    if (nb != 8 && nb != 16) return false;
    if (q0.M > 16 && nb != 16) return false;  // 17..32 rows: K = 4096 only
    if (((uintptr_t)q0.x & 15) != 0 || q0.x_row_stride % 8 != 0) return false;
    int no = 0;
    for (const int codec : {KQ_CODEC_Q4_K, KQ_CODEC_Q6_K})
        for (int i = 0; i < n; ++i)
            if (ps[i].codec == codec) ord[no++] = ps[i];
    if (no != n) return false;
    for (int i = 0; i < n; ++i) {
        const kq_matmul_problem &q = ord[i];
        if (q.x != q0.x || q.x_row_stride != q0.x_row_stride || q.M != q0.M || q.K != q0.K) return false;
        if ((int64_t)(q.N + 16) * q.w_row_bytes >= (int64_t)0x80000000LL) return false;
    }
    if ((int64_t)(q0.M - 1) * q0.x_row_stride * 2 + (int64_t)q0.K * 2 >= (int64_t)0x80000000LL) return false;
    const int64_t t64 = group_tiles(ord, n);
    if (t64 > 2 * (int64_t)device_cus()) return false;
    tiles = (int)t64;
    grid = tiles < device_cus() ? tiles : device_cus();
    pairs = tiles - grid;
    auto codec_of = [&](int t) {
        int first = 0;
        for (int i = 0; i < n; ++i) {
            first += (ord[i].N + 15) / 16;
            if (t < first) return ord[i].codec;
        }
        return ord[n - 1].codec;
    };
    size_t worst = 0;
    for (int b = 0; b < grid; ++b) {
        // 17..32-row launches: a workgroup's tiles share one codec
        if (q0.M > 16 && b < pairs && codec_of(2 * b) != codec_of(2 * b + 1)) return false;
        const int c0 = shot_col_bytes(codec_of(b < pairs ? 2 * b : pairs + b));
        const int c1 = b < pairs ? shot_col_bytes(codec_of(2 * b + 1)) : 0;
        const size_t s = (size_t)kShotWaves * (size_t)shot_region(nb, c0, c1);
        worst = s > worst ? s : worst;
    }
    lds = worst;
    return lds <= (size_t)160 * 1024;
}

}  // namespace

// Whether the one-shot kernel serves this group (fp16 activations; see shot_plan).
bool kq_shot_eligible(const kq_matmul_problem *ps, int n) {
    kq_matmul_problem ord[KQ_MAX_GROUP];
    int tiles, pairs, grid;
    size_t lds;
    return shot_plan(ps, n, ord, tiles, pairs, grid, lds);
}

// Problems validated, eligible and all live; x fp16, x_exp its per-row
// exponents or null.
int kq_shot_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, hipStream_t s) {
    kq_matmul_problem ord[KQ_MAX_GROUP];
    int tiles, pairs, grid;
    size_t lds;
    if (!shot_plan(ps, n, ord, tiles, pairs, grid, lds)) return KQ_ERR_BAD_SHAPE;
    StreamArgs a;
    int t = 0;
    for (int i = 0; i < n; ++i) {
        StreamProblem &p = a.p[i];
        p.w = (const uint8_t *)ord[i].w;
        p.y = ord[i].y;
        p.y_stride = ord[i].y_row_stride;
        p.row_bytes = (uint32_t)ord[i].w_row_bytes;
        p.w_bytes = (uint32_t)(ord[i].N * ord[i].w_row_bytes);
        p.N = ord[i].N;
        p.codec = ord[i].codec;
        a.tile_begin[i] = t;
        t += (ord[i].N + 15) / 16;
    }
    for (int i = n; i < KQ_MAX_GROUP; ++i) {
        a.p[i] = a.p[0];
        a.tile_begin[i] = 0x7FFFFFFF;
    }
    a.x = (const char *)ord[0].x;
    a.x_exp = x_exp;
    a.ctr = nullptr;
    a.part = nullptr;
    a.x_stride = ord[0].x_row_stride;
    a.M = ord[0].M;
    a.K = ord[0].K;
    a.y_dtype = y_dtype;
    a.total_tiles = tiles;
    a.n_problems = n;
    a.split = 1;
    a.pairs = pairs;
    const bool nb8 = ord[0].K / KQ_QK == 8;
    const int m = ord[0].M;
    if (nb8) return m <= 8 ? launch_shot<8, 8>(a, grid, lds, s) : launch_shot<8, 16>(a, grid, lds, s);
    return m <= 8 ? launch_shot<16, 8>(a, grid, lds, s)
           : m <= 16 ? launch_shot<16, 16>(a, grid, lds, s) : launch_shot<16, 32>(a, grid, lds, s);
}

// K slices a launch of this group would take given the workspace (1: whole
// K).  K past 16 super-blocks (the down projections) is cut into at most 8
// slices of 8 super-blocks, else 12, 6 or 4 (the first that divides K); at
// 9..16 rows slices of 12 come first (the Qwen3-8B down projection at 16
// rows: 19.8 us in 4 slices against 22.8 in 6; at 8 rows 16.7 in 6 against
// 17.4 in 4, measured).  A Q4_K + Q6_K group of shorter K is cut in two
// (q|k|v at 1..16 rows: 9.4-11.7 us against 9.6-12.7 for the LDS-staged
// path, measured).  GMLX_KQ_SPLITK=s asks for s slices (tests and tuning; 1
// turns splitting off).
int kq_stream_split_want(const kq_matmul_problem *ps, int n) {
    if (n <= 0 || n > kStreamProblems || ps[0].M < 1 || ps[0].M > 16 || ps[0].K % KQ_QK) return 1;
    const int nb = ps[0].K / KQ_QK;
    if (group_tiles(ps, n) * 4 > (int64_t)KQ_MATMUL_COUNTER_BYTES) return 1;
    if (const char *e = getenv("GMLX_KQ_SPLITK")) {
        const int s = atoi(e);
        return s >= 1 && s <= kMaxSplit && nb % s == 0 && stream_k_ok(ps[0].K / s) ? s : 1;
    }
    if (stream_k_ok(ps[0].K)) {
        // a Q4_K + Q6_K group (the q|k|v of a Q4_K_M layer) takes two slices
        bool q4 = false, q6 = false, other = false;
        for (int i = 0; i < n; ++i) {
            q4 |= ps[i].codec == KQ_CODEC_Q4_K;
            q6 |= ps[i].codec == KQ_CODEC_Q6_K;
            other |= ps[i].codec != KQ_CODEC_Q4_K && ps[i].codec != KQ_CODEC_Q6_K;
        }
        return q4 && q6 && !other && nb % 2 == 0 && stream_k_ok(ps[0].K / 2) ? 2 : 1;
    }
    static constexpr int kWidths[2][4] = {{8, 12, 6, 4}, {12, 8, 6, 4}};
    for (const int w : kWidths[ps[0].M > 8])
        if (nb % w == 0 && nb / w <= kMaxSplit) return nb / w;
    return 1;
}

// Bytes of partial tiles a split launch writes (after the counter region):
// 16 columns of 8 or 16 rows (M <= 8 / 9..16) per tile and slice.
size_t kq_stream_part_bytes(const kq_matmul_problem *ps, int n, int split) {
    const size_t tile_bytes = ps[0].M <= 8 ? 512 : 1024;
    return split > 1 ? ((size_t)group_tiles(ps, n) * split * tile_bytes + 255) & ~(size_t)255 : 0;
}

// Eligibility (the dispatcher also requires fp16 activations): M <= 16, at
// most 4 problems sharing x / stride / M / K, one codec or Q4_K with Q6_K,
// K / split of 2, 4, 6, 8, 12 or 16 super-blocks, weights and x addressable with
// 31-bit buffer offsets.  GMLX_KQ_STREAM=0 declines, =2 forces every eligible
// launch here; GMLX_KQ_STREAM_WGS=n caps the grid at n workgroups (tests).
bool kq_stream_eligible(const kq_matmul_problem *ps, int n, int split) {
    if (n <= 0 || n > kStreamProblems || split < 1 || split > kMaxSplit) return false;
    const char *env = getenv("GMLX_KQ_STREAM");
    if (env && env[0] == '0' && env[1] == 0) return false;
    const kq_matmul_problem &q0 = ps[0];
    if (q0.M < 1 || q0.M > 16 || q0.K % (KQ_QK * split) || !stream_k_ok(q0.K / split)) return false;
    bool mixed = false;
    for (int i = 0; i < n; ++i) {
        const kq_matmul_problem &q = ps[i];
        if (q.x != q0.x || q.x_row_stride != q0.x_row_stride || q.M != q0.M || q.K != q0.K) return false;
        if (q.codec != q0.codec) mixed = true;
        if ((int64_t)(q.N + 16) * q.w_row_bytes >= (int64_t)0x80000000LL) return false;
    }
    if (mixed)
        for (int i = 0; i < n; ++i)
            if (ps[i].codec != KQ_CODEC_Q4_K && ps[i].codec != KQ_CODEC_Q6_K) return false;
    if ((int64_t)(q0.M - 1) * q0.x_row_stride * 2 + (int64_t)q0.K * 2 >= (int64_t)0x80000000LL) return false;
    const int64_t tiles = group_tiles(ps, n);
    if (split > 1 && tiles * 4 > (int64_t)KQ_MATMUL_COUNTER_BYTES) return false;
    // Routing (measured at the Qwen3-8B shapes, B = 1..8): the kernel's fixed
    // cost (ten waves per CU, the activation slab, the partial-tile sums) pays
    // off from about four items (tiles, or tile slices of a split launch) per
    // CU (gate|up: 15.4-16.6 us against 17.5-18.2 us for the LDS-staged
    // path); at one per CU (o) the LDS-staged path is faster (5.5-7.6 us
    // against 6.5-8.6 at 1..16 rows).  GMLX_KQ_STREAM=2 takes every eligible
    // launch (tests).  At 9..16 rows likewise (gate|up: 18.4 / 18.7 us at 12
    // / 16 rows against 19.1 / 20.4; the down projection in 12-block slices:
    // 18.1 / 19.2 against 22.1 / 23.8 for the general kernel).  A Q4_K + Q6_K
    // group comes here split in two (768 items, 3 per CU, for a q|k|v group);
    // the one-shot kernel, tried first, now takes q|k|v and o at 1..16 rows.
    if (!(env && env[0] == '2' && env[1] == 0)) {
        if (mixed) {
            if (split < 2 || tiles * split < 2 * (int64_t)device_cus()) return false;
        } else {
            if (tiles * split < 4 * (int64_t)device_cus()) return false;
        }
    }
    return true;
}

// Problems validated, eligible (for this split) and all live; x is fp16,
// x_exp its per-row exponents or null.  Split launches (split > 1) take the
// arrival counters ctr (one per tile, zero on entry; left zero) and room for
// kq_stream_part_bytes at part.
int kq_stream_launch(const kq_matmul_problem *ps, int n, const int32_t *x_exp, int y_dtype, int split,
                     uint32_t *ctr, float *part, hipStream_t s) {
    StreamArgs a;
    int tiles = 0;
    bool mixed = false;
    for (int i = 0; i < n; ++i) {
        StreamProblem &p = a.p[i];
        p.w = (const uint8_t *)ps[i].w;
        p.y = ps[i].y;
        p.y_stride = ps[i].y_row_stride;
        p.row_bytes = (uint32_t)ps[i].w_row_bytes;
        p.w_bytes = (uint32_t)(ps[i].N * ps[i].w_row_bytes);
        p.N = ps[i].N;
        p.codec = ps[i].codec;
        a.tile_begin[i] = tiles;
        tiles += (ps[i].N + 15) / 16;
        if (ps[i].codec != ps[0].codec) mixed = true;
    }
    for (int i = n; i < KQ_MAX_GROUP; ++i) {
        a.p[i] = a.p[0];
        a.tile_begin[i] = 0x7FFFFFFF;
    }
    const kq_matmul_problem &q0 = ps[0];
    a.x = (const char *)q0.x;
    a.x_exp = x_exp;
    a.ctr = ctr;
    a.part = part;
    a.x_stride = q0.x_row_stride;
    a.M = q0.M;
    a.K = q0.K;
    a.y_dtype = y_dtype;
    a.total_tiles = tiles;
    a.n_problems = n;
    a.split = split;
    int grid = device_cus();
    if (const char *e = getenv("GMLX_KQ_STREAM_WGS")) {  // smaller grids: more tiles and rounds per workgroup
        const int w = atoi(e);
        if (w > 0 && w < grid) grid = w;
    }
    // a multiple of the split (each workgroup keeps one K slice), at most one item each
    grid = grid / split * split;
    if (grid < split) grid = split;
    if (grid > tiles * split) grid = tiles * split;
    const int nb = q0.K / KQ_QK / split;
    if (mixed) return launch_rows<KQ_MIX>(a, nb, grid, s);
    switch (q0.codec) {
    case KQ_CODEC_Q4_K: return launch_rows<KQ_CODEC_Q4_K>(a, nb, grid, s);
    case KQ_CODEC_Q6_K: return launch_rows<KQ_CODEC_Q6_K>(a, nb, grid, s);
    default: return launch_rows<KQ_CODEC_IQ2_XXS>(a, nb, grid, s);
    }
}

// Streaming expert gather (see kq_sgather_kernel).  Forms: K of 2, 3, 4, 6, 8
// or 12 super-blocks (16 and 28 for IQ2_XXS), at most 1024 experts, one
// expert's matrix below 2^31 bytes.  Routing (measured at the C4 / C5
// layers): the K-quant GLU gathers come here (C4 gate|up 61 us against 67
// for the per-tile kernels); the per-pair down gathers (C4 67 against 65) and
// the IQ2_XXS gathers (C5 256 / 116 against 165 / 88) stay on the per-tile
// kernels.  GMLX_KQ_SGATHER=0 declines every call, =2 takes every form.
bool kq_sgather_eligible(int codec, bool glu, int32_t N, int32_t K, int64_t w_row_bytes, int32_t n_experts) {
    const char *env = getenv("GMLX_KQ_SGATHER");
    if (env && env[0] == '0' && env[1] == 0) return false;
    if (K % KQ_QK || K <= 0) return false;
    if (codec != KQ_CODEC_Q4_K && codec != KQ_CODEC_Q6_K && codec != KQ_CODEC_IQ2_XXS) return false;
    if (n_experts < 1 || n_experts > kSGatherMaxSegs) return false;
    if ((int64_t)(N + 16) * w_row_bytes >= (int64_t)0x80000000LL) return false;
    SGatherArgs none{};
    if (sgather_dispatch(none, codec, glu, K / KQ_QK, nullptr, true) != KQ_OK) return false;
    if (env && env[0] == '2' && env[1] == 0) return true;
    return glu && codec != KQ_CODEC_IQ2_XXS;
}

// x: fp16 rows (16-byte aligned, x_row_stride a multiple of 8), x_exp their
// exponents or null; the other arguments as for the per-tile gathers.
int kq_sgather_launch(const void *x, const int32_t *x_exp, int64_t x_row_stride, int32_t x_pair_div, int32_t x_skip,
                      const void *w0, const void *w1, int64_t w_expert_bytes, int64_t w_row_bytes, int32_t N,
                      int32_t K, int codec, int act, float limit, float alpha, const float *b0, const float *b1,
                      int64_t b_stride, const int32_t *seg_info, const int32_t *pair_order, int32_t n_pairs,
                      int32_t n_experts, void *y, int y_dtype, int64_t y_row_stride, int32_t y_skip, hipStream_t s) {
    SGatherArgs a;
    a.w0 = (const uint8_t *)w0;
    a.w1 = (const uint8_t *)w1;
    a.x = (const char *)x;
    a.x_exp = x_exp;
    a.y = y;
    a.seg_info = seg_info;
    a.pair_order = pair_order;
    a.b0 = b0;
    a.b1 = b1;
    a.x_stride = x_row_stride;
    a.w_expert_bytes = w_expert_bytes;
    a.y_stride = y_row_stride;
    a.b_stride = b_stride;
    a.w_row_bytes = (uint32_t)w_row_bytes;
    a.w_bytes = (uint32_t)((int64_t)N * w_row_bytes);
    a.x_pair_div = x_pair_div;
    a.x_skip = x_skip;
    a.y_skip = y_skip;
    a.N = N;
    a.K = K;
    a.n_pairs = n_pairs;
    a.n_experts = n_experts;
    a.n_tiles = (N + 15) / 16;
    a.y_dtype = y_dtype;
    a.act = act;
    a.limit = limit;
    a.alpha = alpha;
    return sgather_dispatch(a, codec, w1 != nullptr, K / KQ_QK, s, false);
}

// ---- Fused dense MLP at M <= 8 ----------------------------------------------
// gmlx's _FusedMLP (gmlx/occupancy_fuse.py:270-316): the grouped gate|up call,
// the SwiGLU h = act(gate . x) * (up . x), then the down projection -- here in
// one persistent launch of one producer / consumer workgroup per CU, so the
// down projection's weight stream starts while gate|up is finishing instead
// of after a launch boundary and a fresh ramp.
//  Phase A (gate|up): items are 16-row tile pairs (gate tile p, then up tile
//    p), workgroup b taking pairs b, b + G, ...; the consumers own K-slabs of
//    the Q4_K rows as in the streaming kernel (owned view), and a round's
//    epilogue forms h[m][16p + n] = act(g, u) in fp32 and stores it as fp16
//    with device-coherent stores (they reach the point of coherence past the
//    XCDs' L2s), then counts one arrival per (pair, row group) on the counter
//    of the down K-slice the columns belong to.
//  Phase B (down): K = I is cut into S slices of 8 super-blocks; workgroup b
//    keeps slice q = b mod S and walks down tiles b / S + j G_q (G_q: the
//    workgroups of slice q, G / S or one more), like a
//    split launch of the streaming kernel (partial tiles, per-tile arrival
//    counters, the last slice sums in slice order).  The producers copy the
//    first down tiles into the ring while the consumers finish phase A; the
//    consumers wait once, before their first down tile, until the h columns
//    of their own super-block of the slice have all arrived (a bounded spin
//    on its counter), then load their h fragments with device-coherent loads.
// Every phase-A item is finished by a running workgroup that never waits
// before it, and the grid is at most one workgroup per CU (LDS), so every
// wait ends; past kMlpSpinLimit polls a wait gives up and sets the status
// word instead of hanging (the results are then invalid).  The slice counters
// return to zero: the last of a slice's waiting workgroups to pass its wait
// clears them.
namespace {

constexpr int kMlpC = 8;           // consumer waves
constexpr int kMlpRows = 8;        // activation rows (M <= 8)
constexpr int kMlpSliceNb = 8;     // down super-blocks per slice (one per consumer)
constexpr uint32_t kMlpSpinLimit = 1u << 22;
// counter region (uint32 index): per-tile split counters below kMlpSbBase;
// per h super-block sb (sb < I / 256 <= 64) the arrivals at kMlpSbBase + 32 sb
// and, for the slice's first super-block, the slice's readers at + 16; the
// status word at kMlpStatus
constexpr int kMlpSbBase = (int)(KQ_MATMUL_COUNTER_BYTES / 4) - 2048 - 32;
constexpr int kMlpStatus = (int)(KQ_MATMUL_COUNTER_BYTES / 4) - 16;

struct MlpArgs {
    const uint8_t *wg, *wu, *wd;
    const char *x;           // fp16 [M, K]
    const int32_t *x_exp;    // per-row exponents of prepared activations, or null
    uint16_t *h;             // fp16 bits [kMlpRows][I]
    uint32_t *ctr;           // counter region
    float *part;             // partial tiles [tiles][S][8 rows][16 columns]
    void *y;
    int64_t x_stride, y_stride;
    uint32_t gu_bytes, gu_row, d_bytes, d_row;
    int32_t M, K, I, N, y_dtype, act, S, pairs, tiles;
};

typedef const __attribute__((address_space(4))) MlpArgs *MArgs;

template <int SBA, int CD>
struct MlpGeo {
    static constexpr int NBA = SBA * kMlpC;                          // gate / up super-blocks (K / 256)
    static constexpr int RCA = SlotGeo<KQ_CODEC_Q4_K, NBA>::RC;      // chunks per slot row
    static constexpr int RCB = SlotGeo<CD, kMlpSliceNb>::RC;
    static constexpr int ROWA = NBA * SlotGeo<KQ_CODEC_Q4_K, NBA>::CPB;  // chunks a row copies
    static constexpr int ROWB = kMlpSliceNb * SlotGeo<CD, kMlpSliceNb>::CPB;
    static constexpr int PRA = row_parts<KQ_CODEC_Q4_K, NBA>(), PRB = row_parts<CD, kMlpSliceNb>();
    static constexpr int PR = PRA > PRB ? PRA : PRB;                 // 1 KB loads per row, both phases
    static constexpr int PL = (16 / kProducers) * PR;                // loads per producer per tile
    static constexpr int SLOTB = 16 * 16 * (RCA > RCB ? RCA : RCB);
    static constexpr int RED = 8 * kMlpC * 32 * 16;                  // a round's partial tiles
    static constexpr int JUNK = 1024;                                // target of padding loads
};

template <int SBA, int CD, int R>
__global__ __launch_bounds__(64 * (kProducers + kMlpC)) void kq_mlp_kernel(MlpArgs a_) {
    using MG = MlpGeo<SBA, CD>;
    constexpr int C = kMlpC, LR = 32, kTmax = 8;
    static_assert(MG::PL * (R - 1) <= 63, "vmcnt counts at most 63 loads");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const MArgs A = (MArgs)__builtin_amdgcn_kernarg_segment_ptr();
    const Iq2Tables &iq2_tab = *IqTables<CD>::get();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = kq_lane(), r = lane & 15, g = lane >> 4;
    const int G = (int)gridDim.x, B0 = (int)blockIdx.x, S = A->S;
    const int M = A->M;
    const int nA = B0 < A->pairs ? 2 * ((A->pairs - B0 + G - 1) / G) : 0;  // phase-A tiles (gate, up alternating)
    // slice q = B0 mod S has Gs workgroups (G need not be a multiple of S)
    const int q = B0 % S, Gs = G / S + (q < G % S ? 1 : 0), T0 = B0 / S;
    const int nB = T0 < A->tiles ? (A->tiles - T0 + Gs - 1) / Gs : 0;     // phase-B tiles
    const int n = nA + nB;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(LDSP(void))smem;
    floatx4 *red = (floatx4 *)(smem + R * MG::SLOTB);
    const uint32_t junk = ring_lds + R * MG::SLOTB + MG::RED;
    // a workgroup's round boundaries: rounds of kTmax tiles within each phase
    auto round_end = [&](int b) { return b < nA ? ((b + 1) % kTmax == 0 || b + 1 == nA) : ((b + 1 - nA) % kTmax == 0 || b + 1 == n); };

    if (wave < kProducers) {
        uint32_t tabA[MG::PR], tabB[MG::PR];
#pragma unroll
        for (int p = 0; p < MG::PR; ++p) {
            tabA[p] = p < MG::PRA ? row_chunk_src<KQ_CODEC_Q4_K, MG::NBA>(
                                        (p == MG::PRA - 1 ? MG::ROWA - 64 : 64 * p) + lane, MG::ROWA)
                                  : 0x80000000u;
            tabB[p] = p < MG::PRB ? row_chunk_src<CD, kMlpSliceNb>(
                                        (p == MG::PRB - 1 ? MG::ROWB - 64 : 64 * p) + lane, MG::ROWB)
                                  : 0x80000000u;
        }
        const uint32_t kofsB = (uint32_t)(q * kMlpSliceNb) * (uint32_t)Geo<CD>::BPB;
        // (the tables reach copy as arguments: a lambda capturing a local
        // array made the host pass drop the kernel's instantiations)
        auto copy = [&](int j, const uint32_t *ta, const uint32_t *tb) {
            const uint32_t slot = ring_lds + (uint32_t)(j % R) * MG::SLOTB;
            if (j < nA) {
                const int pair = B0 + (j >> 1) * G;
                const __amdgpu_buffer_rsrc_t rs = kq_buffer((j & 1) ? A->wu : A->wg, A->gu_bytes);
                const uint32_t row0 = (uint32_t)pair * 16, last = (uint32_t)A->I - 1, rb = A->gu_row;
#pragma unroll
                for (int i = 0; i < 16 / kProducers; ++i) {
                    const int row = i * kProducers + wave;
                    const int soff = (int)(min(row0 + (uint32_t)row, last) * rb);
                    const uint32_t m0 = slot + (uint32_t)(row * MG::RCA * 16);
#pragma unroll
                    for (int p = 0; p < MG::PR; ++p)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            rs,
                            (LDSP(void))(uintptr_t)(p < MG::PRA ? m0 + 16 * (p == MG::PRA - 1 ? MG::ROWA - 64 : 64 * p)
                                                                : junk),
                            16, ta[p], soff, 0, 0);
                }
            } else {
                const int tile = T0 + (j - nA) * Gs;
                const __amdgpu_buffer_rsrc_t rs = kq_buffer(A->wd, A->d_bytes);
                const uint32_t row0 = (uint32_t)tile * 16, last = (uint32_t)A->N - 1, rb = A->d_row;
#pragma unroll
                for (int i = 0; i < 16 / kProducers; ++i) {
                    const int row = i * kProducers + wave;
                    const int soff = (int)(min(row0 + (uint32_t)row, last) * rb + kofsB);
                    const uint32_t m0 = slot + (uint32_t)(row * MG::RCB * 16);
#pragma unroll
                    for (int p = 0; p < MG::PR; ++p)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            rs,
                            (LDSP(void))(uintptr_t)(p < MG::PRB ? m0 + 16 * (p == MG::PRB - 1 ? MG::ROWB - 64 : 64 * p)
                                                                : junk),
                            16, tb[p], soff, 0, 0);
                }
            }
        };
        __builtin_amdgcn_s_barrier();  // the consumers' activation loads are issued
        const int first = min(2, n);
        for (int j = 0; j < first; ++j) copy(j, tabA, tabB);
        for (int b = 0; b < n; ++b) {
            const int newer = b == 0 ? first - 1 : min(R - 2, n - 1 - b);
            wait_tiles_left<MG::PL, (R - 1 < 63 / MG::PL ? R - 1 : 63 / MG::PL)>(newer);
            __builtin_amdgcn_s_barrier();  // tile b to the consumers; tile b - 1's slot back
            if (b == 0) {
                for (int j = first; j < min(R, n); ++j) copy(j, tabA, tabB);
            } else if (b + R - 1 < n) {
                copy(b + R - 1, tabA, tabB);
            }
            if (round_end(b)) {
                __builtin_amdgcn_s_barrier();  // the round's partial tiles are in LDS
                if (b + 1 < n) __builtin_amdgcn_s_barrier();  // the round's outputs are out: red is free
            }
        }
        return;
    }

    // ================= consumers
    const int c = wave - kProducers;
    const int n16 = lane & 15, mq = lane >> 4;
    // phase A: the owned Q4_K view of super-blocks [c SBA, c SBA + SBA) of x
    half8_t xr[SBA][8];
    floatx4 xsum;
    {
        const uint32_t xbytes = (uint32_t)(((int64_t)(M - 1) * A->x_stride + A->K) * 2);
        const __amdgpu_buffer_rsrc_t xs = kq_buffer(A->x, xbytes);
        const uint32_t xrow = r < M ? (uint32_t)(r * A->x_stride * 2) + (uint32_t)(c * SBA * KQ_QK * 2) : 0x80000000u;
        u32x4 cin[SBA][8];
#pragma unroll
        for (int s2 = 0; s2 < SBA; ++s2)
#pragma unroll
            for (int w = 0; w < 4; ++w)
#pragma unroll
                for (int a2 = 0; a2 < 2; ++a2)
                    cin[s2][2 * w + a2] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                   xs, xrow + (uint32_t)(2 * (256 * s2 + 64 * g + 32 * a2 + 8 * w)), 0, 0));
        __builtin_amdgcn_s_barrier();  // the loads are issued: the producers may start
        q4own_x<SBA>(xr, xsum, cin, lane);
    }
    const Q4Consts q4k = q4own_consts(g);
    const bool has_xe = A->x_exp != nullptr;
    int xe[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) xe[h] = has_xe && 4 * h + mq < M ? A->x_exp[4 * h + mq] : 0;
    const __amdgpu_buffer_rsrc_t hrs = kq_buffer(A->h, (uint32_t)(kMlpRows * A->I * 2));
    uint32_t *const ctr0 = A->ctr;
    const float *redf = (const float *)red;
    for (int round0 = 0; round0 < nA; round0 += kTmax) {
        const int nt = min(kTmax, nA - round0);
        for (int b = 0; b < nt; ++b) {
            const int gb = round0 + b;
            __builtin_amdgcn_s_barrier();  // tile gb has landed
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            floatx4 acc = fzero4();
            q4own_slab<SBA>(acc,
                            (LDSP(const uint8_t))smem + (gb % R) * MG::SLOTB + r * MG::RCA * 16 + c * SBA * 144, xr,
                            xsum, q4k);
            kq_mfma_drain();
            if (g < 2) red[(b * C + c) * LR + lane] = acc;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        }
        __builtin_amdgcn_s_barrier();  // the round's partial tiles are in LDS
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // units (pair qq, row group h): one output per lane, the C partial
        // tiles of gate and of up summed in consumer order, then act(g, u)
        for (int unit = c; unit < nt; unit += C) {
            const int qq = unit >> 1, h = unit & 1;
            const int pair = B0 + ((round0 >> 1) + qq) * G;
            float v[2];
#pragma unroll
            for (int w2 = 0; w2 < 2; ++w2) {
                float sum = 0.f;
#pragma unroll
                for (int c2 = 0; c2 < C; ++c2) {
                    const float pv = redf[((((2 * qq + w2) * C + c2) * LR) + 16 * h + n16) * 4 + mq];
                    sum = c2 == 0 ? pv : sum + pv;
                }
                v[w2] = sum;
            }
            const int m = 4 * h + mq;
            const float hv = kq_glu(A->act, ldexpf(v[0], xe[h]), ldexpf(v[1], xe[h]), 0.f, 0.f, 0.f, 0.f);
            const uint32_t off = m < M ? (uint32_t)((m * A->I + pair * 16 + n16) * 2) : 0x80000000u;
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)hv), hrs, off, 0, 16);
            __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));  // the stores have reached the point of coherence
            if (lane == 0)  // the h super-block of the pair's columns
                __hip_atomic_fetch_add(ctr0 + kMlpSbBase + 32 * ((pair * 16) / KQ_QK), 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
        if (round0 + nt < n) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_barrier();  // red is free for the next round
        }
    }
    if (nB == 0) return;
    // ---- phase B: wait until slice q's h columns have all arrived (two per
    // pair: the pair's two row groups), then the consumer's fragments of
    // super-block q * 8 + c of h
    // Each consumer waits for its own h super-block sb = q * 8 + c: 16 pairs,
    // two arrivals each (one lane polls, spaced: every poll is a
    // device-coherent load of a line the arrivals also write).
    {
        const int sb = q * kMlpSliceNb + c;
        const uint32_t want = (uint32_t)(2 * min(KQ_QK / 16, max(0, A->pairs - sb * (KQ_QK / 16))));
        uint32_t *const sc = ctr0 + kMlpSbBase + 32 * sb;
        uint32_t seen = 0, spins = 0;
        if (lane == 0) {
            while ((seen = __hip_atomic_load(sc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) < want) {
                __builtin_amdgcn_s_sleep(4);
                if (++spins >= kMlpSpinLimit) {
                    __hip_atomic_store(ctr0 + kMlpStatus, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
        }
        (void)__builtin_amdgcn_readfirstlane((int)seen);
    }
    half8_t hr[1][8];
    [[maybe_unused]] floatx4 hsum = fzero4();
    {
        const uint32_t hrow = r < M ? (uint32_t)((r * A->I + (q * kMlpSliceNb + c) * KQ_QK) * 2) : 0x80000000u;
#pragma unroll
        for (int t = 0; t < 8; ++t)
            hr[0][t] = __builtin_bit_cast(
                half8_t, __builtin_amdgcn_raw_buffer_load_b128(hrs, hrow + (uint32_t)(2 * Block<CD>::x_elem(t, g)), 0, 16));
        if constexpr (CD == KQ_CODEC_Q4_K) hsum = xsum_generic<1>(hr, r);
    }
    int ydt = A->y_dtype;
    float *const part = A->part;
    const int cstride = min(32, 1 << (31 - __builtin_clz(kMlpSbBase / max(A->tiles, 1))));
    for (int round0 = nA; round0 < n; round0 += kTmax) {
        const int nt = min(kTmax, n - round0);
        for (int b = 0; b < nt; ++b) {
            const int gb = round0 + b;
            __builtin_amdgcn_s_barrier();  // tile gb has landed
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            if (gb == nA && c == 0 && lane == 0) {
                // every consumer of this workgroup has passed its wait: the
                // last of the slice's waiting workgroups (those with down
                // tiles: min(Gs, tiles)) clears the slice's counters
                uint32_t *const sc = ctr0 + kMlpSbBase + 32 * (q * kMlpSliceNb);
                if (__hip_atomic_fetch_add(sc + 16, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    (uint32_t)(min(Gs, A->tiles) - 1)) {
                    __hip_atomic_store(sc + 16, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                    for (int i = 0; i < kMlpSliceNb; ++i)
                        __hip_atomic_store(sc + 32 * i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            floatx4 acc = fzero4();
            mma_slab<CD, 1>(acc, ring_lds + (uint32_t)(gb % R) * MG::SLOTB + r * MG::RCB * 16 + c * Geo<CD>::SLOT, hr,
                            hsum, g, iq2_tab);
            kq_mfma_drain();
            if (g < 2) red[(b * C + c) * LR + lane] = acc;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        }
        __builtin_amdgcn_s_barrier();  // the round's partial tiles are in LDS
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // the round's tiles b = c, c + C, ...: partial of slice q over the C
        // consumers (consumer order), out with device-coherent stores
        for (int b = c; b < nt; b += C) {
            const int tile = T0 + (round0 - nA + b) * Gs;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float *rf = redf + 4 * (b * C * LR + 16 * h + n16) + mq;
                float sum = rf[0];
#pragma unroll
                for (int c2 = 1; c2 < C; ++c2) sum += rf[4 * c2 * LR];
                if (4 * h + mq < M)
                    __hip_atomic_store(part + ((size_t)tile * S + q) * 128 + 64 * h + lane, sum, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(KQ_VMCNT(0));
        const int bl = c + lane * C;
        bool last = false;
        if (bl < nt) {
            uint32_t *const ctr = ctr0 + (T0 + (round0 - nA + bl) * Gs) * cstride;
            last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(S - 1);
            if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        uint64_t mine = __builtin_amdgcn_ballot_w64(last);
        while (mine) {
            const int i = __builtin_ctzll(mine);
            mine &= mine - 1;
            const int tile = T0 + (round0 - nA + c + i * C) * Gs;
            const float *pp = part + (size_t)tile * S * 128;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int m = 4 * h + mq, col = tile * 16 + n16;
                if (m >= M) continue;
                float v[kMaxSplit];
#pragma unroll
                for (int s2 = 0; s2 < kMaxSplit; ++s2)
                    v[s2] = s2 < S ? __hip_atomic_load(pp + s2 * 128 + 64 * h + lane, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT)
                                   : 0.f;
                float sum = v[0];
#pragma unroll
                for (int s2 = 1; s2 < kMaxSplit; ++s2)
                    if (s2 < S) sum += v[s2];
                if (col < A->N) kq_store_out(A->y, ydt, (int64_t)m * A->y_stride + col, sum);
            }
        }
        if (round0 + nt < n) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_barrier();  // red is free for the next round
        }
    }
}

template <int SBA, int CD>
int launch_mlp(const MlpArgs &a, int grid, hipStream_t s) {
    using MG = MlpGeo<SBA, CD>;
    constexpr size_t budget = 160 * 1024 - (CD == KQ_CODEC_IQ2_XXS ? sizeof(Iq2Tables) : 0);
    constexpr size_t fixed = MG::RED + MG::JUNK;
    constexpr int R = (budget - fixed) / MG::SLOTB >= 4 ? 4 : (int)((budget - fixed) / MG::SLOTB);
    static_assert(R >= 2, "fused MLP LDS");
    constexpr size_t lds = (size_t)R * MG::SLOTB + fixed;
    static bool raised = false;
    if (!raised) {
        if (hipFuncSetAttribute((const void *)kq_mlp_kernel<SBA, CD, R>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess)
            return KQ_ERR_LAUNCH_FAILED;
        raised = true;
    }
    hipLaunchKernelGGL((kq_mlp_kernel<SBA, CD, R>), dim3(grid), dim3(64 * (kProducers + kMlpC)), lds, s, a);
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

}  // namespace

// Shapes the fused MLP kernel serves (fp16 activations; the caller prepares
// bf16 / fp32 rows): M 1..8, Q4_K gate / up with K of 8 or 16 super-blocks,
// Q6_K or Q4_K down whose K = I is whole slices of 8 super-blocks (at most
// kMaxSplit), byte offsets within 31 bits.
bool kq_mlp_eligible(int32_t M, int32_t K, int32_t I, int32_t N, int gu_codec, int d_codec, int64_t gu_row,
                     int64_t d_row) {
    if (M < 1 || M > kMlpRows || gu_codec != KQ_CODEC_Q4_K) return false;
    if (d_codec != KQ_CODEC_Q6_K && d_codec != KQ_CODEC_Q4_K) return false;
    if (K != 8 * KQ_QK && K != 16 * KQ_QK) return false;  // one or two super-blocks per consumer
    if (I <= 0 || I % (kMlpSliceNb * KQ_QK) || I / (kMlpSliceNb * KQ_QK) > kMaxSplit) return false;
    if (N <= 0) return false;
    const int64_t tiles = (N + 15) / 16;
    if (tiles > kMlpSbBase) return false;  // one split counter per down tile
    if ((int64_t)(I + 16) * gu_row >= 0x80000000LL || (int64_t)(N + 16) * d_row >= 0x80000000LL) return false;
    if ((int64_t)kMlpRows * I * 2 >= 0x80000000LL) return false;
    return true;
}

// Workspace after the counter region: fp16 h [8][I], then the partial tiles.
size_t kq_mlp_work_bytes(int32_t I, int32_t N) {
    const size_t hb = ((size_t)kMlpRows * I * 2 + 255) & ~(size_t)255;
    const size_t pb = (size_t)((N + 15) / 16) * (I / (kMlpSliceNb * KQ_QK)) * 512;
    return hb + pb;
}

int kq_mlp_launch(const void *x, const int32_t *x_exp, int64_t x_row_stride, int32_t M, int32_t K,
                  const void *w_gate, const void *w_up, int64_t gu_row, int32_t I, const void *w_down,
                  int64_t d_row, int d_codec, int32_t N, int act, void *y, int y_dtype, int64_t y_row_stride,
                  void *workspace, hipStream_t s) {
    MlpArgs a;
    a.wg = (const uint8_t *)w_gate;
    a.wu = (const uint8_t *)w_up;
    a.wd = (const uint8_t *)w_down;
    a.x = (const char *)x;
    a.x_exp = x_exp;
    a.ctr = (uint32_t *)workspace;
    a.h = (uint16_t *)((char *)workspace + KQ_MATMUL_COUNTER_BYTES);
    a.part = (float *)((char *)workspace + KQ_MATMUL_COUNTER_BYTES +
                       (((size_t)kMlpRows * I * 2 + 255) & ~(size_t)255));
    a.y = y;
    a.x_stride = x_row_stride;
    a.y_stride = y_row_stride;
    a.gu_row = (uint32_t)gu_row;
    a.gu_bytes = (uint32_t)(I * gu_row);
    a.d_row = (uint32_t)d_row;
    a.d_bytes = (uint32_t)(N * d_row);
    a.M = M;
    a.K = K;
    a.I = I;
    a.N = N;
    a.y_dtype = y_dtype;
    a.act = act;
    a.S = I / (kMlpSliceNb * KQ_QK);
    a.pairs = I / 16;
    a.tiles = (N + 15) / 16;
    const int grid = device_cus();
    const bool k16 = K == 16 * KQ_QK;
    if (d_codec == KQ_CODEC_Q6_K) return k16 ? launch_mlp<2, KQ_CODEC_Q6_K>(a, grid, s) : launch_mlp<1, KQ_CODEC_Q6_K>(a, grid, s);
    return k16 ? launch_mlp<2, KQ_CODEC_Q4_K>(a, grid, s) : launch_mlp<1, KQ_CODEC_Q4_K>(a, grid, s);
}
