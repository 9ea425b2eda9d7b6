// Wave-level dequant-fused MFMA tile for GGUF K-quant weights (gfx950).
//
// Tile: one wave computes C[16*MT batch rows, 16 weight rows] over a range of
// super-blocks with v_mfma_f32_16x16x32_f16 (A = activations, B = weights^T).
// Lane l = 16*g + r: r selects the weight row (B column) and the activation
// row (A row) the lane feeds; g selects WHICH super-block of the current
// 4-block step the lane owns.  A lane therefore decodes one whole super-block
// per step -- all of its scales are local -- and feeds 32 MFMAs of 8 values
// each (values 8t..8t+7 of its block).  The MFMA sums over the 4 lane groups,
// i.e. over 4 different blocks at once; that is valid because every weight
// fragment is already fully scaled (w = dequant(q) in fp16), so no per-block
// factor has to be applied to the accumulator.
//
// Dequant to fp16 in registers, per pair of values:
//   Q4_K : h = perm(0x64.., nibbles)  (= 1024+q, exact)
//          w = fma(h - 1024, dsc, -dm)          single rounding
//   Q6_K : w = (h - 1056) * dsc                 single rounding (q-32 exact)
//   IQ2  : w = (grid ^ signmask) * db           single rounding
// dsc / dm / db are the fp32 sub-block scales rounded once to fp16.
#pragma once
#include "kq_common.h"
#include "kq_tables.h"

namespace kqmma {

// ---- IQ2_XXS tables in fp16 form, built at compile time ------------------
constexpr uint32_t mag_to_f16_bits(uint32_t b) { return b == 0x08 ? 0x4800u : b == 0x19 ? 0x4E40u : 0x5160u; }

struct Iq2Tables {
    uint32_t grid_h2[256][4];  // 8 fp16 magnitudes per grid entry
    uint32_t sign_x2[128][4];  // XOR masks (0x8000 per negative value)
};

constexpr Iq2Tables make_iq2_tables() {
    Iq2Tables t{};
    constexpr uint64_t grid[256] = KQ_IQ2XXS_GRID_INIT;
    for (int e = 0; e < 256; ++e) {
        for (int p = 0; p < 4; ++p) {
            const uint32_t lo = mag_to_f16_bits((uint32_t)((grid[e] >> (16 * p)) & 0xFF));
            const uint32_t hi = mag_to_f16_bits((uint32_t)((grid[e] >> (16 * p + 8)) & 0xFF));
            t.grid_h2[e][p] = lo | (hi << 16);
        }
    }
    for (int i = 0; i < 128; ++i) {
        int pc = 0;
        for (int b = 0; b < 7; ++b) pc += (i >> b) & 1;
        const uint32_t s = (uint32_t)i | ((uint32_t)(pc & 1) << 7);
        for (int p = 0; p < 4; ++p) {
            const uint32_t lo = ((s >> (2 * p)) & 1) ? 0x8000u : 0u;
            const uint32_t hi = ((s >> (2 * p + 1)) & 1) ? 0x80000000u : 0u;
            t.sign_x2[i][p] = lo | hi;
        }
    }
    return t;
}

__device__ const Iq2Tables kIq2 = make_iq2_tables();

// ---- per-codec block decoders --------------------------------------------

__device__ __forceinline__ half2_t h2b(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t b2h(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2_t bcast(_Float16 v) { return half2_t{v, v}; }

template <int CODEC>
struct Block;

// Q4_K: 144 B = header (d, dmin, 12 B scales) + 128 B qs; 16-B aligned.
template <>
struct Block<KQ_CODEC_Q4_K> {
    u32x4 raw[9];
    half2_t dsc[8], ndm[8];

    __device__ __forceinline__ void load(const uint8_t *blk) {
        const u32x4 *p = (const u32x4 *)blk;
#pragma unroll
        for (int i = 0; i < 9; ++i) raw[i] = p[i];
    }
    // valid == false zeroes every weight of the block (a padding block).
    __device__ __forceinline__ void prep(bool valid) {
        const uint32_t h0 = raw[0].x;
        const float d = valid ? kq_f16_bits_to_f32(h0 & 0xFFFF) : 0.f;
        const float dmin = valid ? kq_f16_bits_to_f32(h0 >> 16) : 0.f;
        // scales bytes s[0..11] = raw[0].y, .z, .w
        const uint32_t s0 = raw[0].y, s1 = raw[0].z, s2 = raw[0].w;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t sc, mn;
            if (j < 4) {
                sc = (s0 >> (8 * j)) & 63;
                mn = (s1 >> (8 * j)) & 63;
            } else {
                const uint32_t bj4 = (s2 >> (8 * (j - 4))) & 0xFF;     // s[j+4]
                const uint32_t bjm4 = (s0 >> (8 * (j - 4))) & 0xFF;    // s[j-4]
                const uint32_t bj = (s1 >> (8 * (j - 4))) & 0xFF;      // s[j]
                sc = (bj4 & 0xF) | ((bjm4 >> 6) << 4);
                mn = (bj4 >> 4) | ((bj >> 6) << 4);
            }
            dsc[j] = bcast((_Float16)(d * (float)sc));
            ndm[j] = bcast((_Float16)(-(dmin * (float)mn)));
        }
    }
    // values 8t .. 8t+7 of the block (t = 0..31)
    __device__ __forceinline__ half8_t frag(int t) const {
        const int sub = t >> 2, c = sub >> 1, j = t & 3;
        const uint32_t *qs = (const uint32_t *)&raw[1];
        uint32_t w0 = qs[8 * c + 2 * j], w1 = qs[8 * c + 2 * j + 1];
        if (sub & 1) {
            w0 >>= 4;
            w1 >>= 4;
        }
        w0 &= 0x0F0F0F0Fu;
        w1 &= 0x0F0F0F0Fu;
        const half2_t k1024 = {(_Float16)1024.f, (_Float16)1024.f};
        half2_t p0 = h2b(kq_bytes_to_h2_biased(w0, KQ_SEL_B01)) - k1024;
        half2_t p1 = h2b(kq_bytes_to_h2_biased(w0, KQ_SEL_B23)) - k1024;
        half2_t p2 = h2b(kq_bytes_to_h2_biased(w1, KQ_SEL_B01)) - k1024;
        half2_t p3 = h2b(kq_bytes_to_h2_biased(w1, KQ_SEL_B23)) - k1024;
        p0 = __builtin_elementwise_fma(p0, dsc[sub], ndm[sub]);
        p1 = __builtin_elementwise_fma(p1, dsc[sub], ndm[sub]);
        p2 = __builtin_elementwise_fma(p2, dsc[sub], ndm[sub]);
        p3 = __builtin_elementwise_fma(p3, dsc[sub], ndm[sub]);
        return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    }
};

// Q6_K: 210 B = ql[128] qh[64] scales[16] d; only 2-byte aligned.
template <>
struct Block<KQ_CODEC_Q6_K> {
    u32x4 raw[13];        // bytes 0..207
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
    __device__ __forceinline__ half8_t frag(int t) const {
        const int h = t >> 4, quarter = (t >> 2) & 3, j = t & 3;
        const uint32_t *ql = (const uint32_t *)&raw[0];   // 32 dwords
        const uint32_t *qh = (const uint32_t *)&raw[8];   // 16 dwords
        uint32_t l0 = ql[16 * h + 8 * (quarter & 1) + 2 * j];
        uint32_t l1 = ql[16 * h + 8 * (quarter & 1) + 2 * j + 1];
        uint32_t q0 = qh[8 * h + 2 * j], q1 = qh[8 * h + 2 * j + 1];
        if (quarter >= 2) {
            l0 >>= 4;
            l1 >>= 4;
        }
        // 6-bit codes: low nibble | (2 high bits << 4)
        const int hs = 2 * quarter;
        uint32_t c0, c1;
        if (hs <= 4) {
            c0 = (l0 & 0x0F0F0F0Fu) | ((q0 << (4 - hs)) & 0x30303030u);
            c1 = (l1 & 0x0F0F0F0Fu) | ((q1 << (4 - hs)) & 0x30303030u);
        } else {
            c0 = (l0 & 0x0F0F0F0Fu) | ((q0 >> (hs - 4)) & 0x30303030u);
            c1 = (l1 & 0x0F0F0F0Fu) | ((q1 >> (hs - 4)) & 0x30303030u);
        }
        const half2_t k1056 = {(_Float16)1056.f, (_Float16)1056.f};
        const half2_t s = dsc[t >> 1];
        const half2_t p0 = (h2b(kq_bytes_to_h2_biased(c0, KQ_SEL_B01)) - k1056) * s;
        const half2_t p1 = (h2b(kq_bytes_to_h2_biased(c0, KQ_SEL_B23)) - k1056) * s;
        const half2_t p2 = (h2b(kq_bytes_to_h2_biased(c1, KQ_SEL_B01)) - k1056) * s;
        const half2_t p3 = (h2b(kq_bytes_to_h2_biased(c1, KQ_SEL_B23)) - k1056) * s;
        return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    }
};

// IQ2_XXS: 66 B = d + 8 groups x (4 grid indices, u32 signs|scale).
template <>
struct Block<KQ_CODEC_IQ2_XXS> {
    u32x4 raw[4];         // bytes 2..65 (the 8 groups)
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
    __device__ __forceinline__ half8_t frag(int t) const {
        const int grp = t >> 2, l = t & 3;
        const uint32_t *g = (const uint32_t *)&raw[0];
        const uint32_t idx = (g[2 * grp] >> (8 * l)) & 0xFF;
        const uint32_t s7 = (g[2 * grp + 1] >> (7 * l)) & 127u;
        const u32x4 gm = *(const u32x4 *)kIq2.grid_h2[idx];
        const u32x4 sm = *(const u32x4 *)kIq2.sign_x2[s7];
        const half2_t s = db[grp];
        const half2_t p0 = h2b(gm.x ^ sm.x) * s;
        const half2_t p1 = h2b(gm.y ^ sm.y) * s;
        const half2_t p2 = h2b(gm.z ^ sm.z) * s;
        const half2_t p3 = h2b(gm.w ^ sm.w) * s;
        return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    }
};

// ---- activation fragments -------------------------------------------------

// Activation element types: 0 = fp16, 1 = bf16, 2 = fp32.
template <int XT>
constexpr int x_elem_bytes() { return XT == 2 ? 4 : 2; }

// 8 consecutive activations as fp16.  bf16 / fp32 inputs are converted
// (exact for bf16 in the fp16 normal range; fp32 rounds to nearest).
template <int XT>
__device__ __forceinline__ half8_t load_x8(const char *p) {
    if constexpr (XT == 0) {
        return __builtin_bit_cast(half8_t, *(const u32x4 *)p);
    } else if constexpr (XT == 1) {
        const u32x4 v = *(const u32x4 *)p;
        half8_t h;
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h[2 * i] = (_Float16)__builtin_bit_cast(float, w[i] << 16);
            h[2 * i + 1] = (_Float16)__builtin_bit_cast(float, w[i] & 0xFFFF0000u);
        }
        return h;
    } else {
        const float4 a = *(const float4 *)p;
        const float4 b = *(const float4 *)(p + 16);
        return half8_t{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                       (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
    }
}

// Accumulate over super-blocks [kb_begin, kb_end) of NW weight matrices
// (NW = 2: gate and up share the activations).  wrow[i] points at this
// lane's weight row (row n0 + lane%16 of matrix i, clamped to a valid row by
// the caller).  xrow[mt] points (as bytes) at this lane's activation row of
// m-tile mt, clamped to a valid row: rows past M compute throw-away outputs
// that are never stored, so no load is conditional.  Blocks past kb_end (the
// last, partial 4-block step) are read from a clamped valid address and
// zeroed through their scales.
template <int CODEC, int MT, int XT, int NW>
__device__ __forceinline__ void tile_accumulate(const uint8_t *const (&wrow)[NW], int kb_begin,
                                                int kb_end, const char *const (&xrow)[MT],
                                                floatx4 (&acc)[NW][MT]) {
    constexpr int XS = x_elem_bytes<XT>();
    constexpr int BPB = kq_block_bytes(CODEC);
    const int g = kq_lane() >> 4;
    for (int kb = kb_begin; kb < kb_end; kb += 4) {
        const int blk = kb + g;
        const bool bvalid = blk < kb_end;
        const int blk_c = bvalid ? blk : kb_end - 1;
        Block<CODEC> wb[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) wb[i].load(wrow[i] + (int64_t)blk_c * BPB);
#pragma unroll
        for (int i = 0; i < NW; ++i) wb[i].prep(bvalid);
        const int64_t xoff = (int64_t)blk_c * KQ_QK * XS;
        // Activation fragments are issued in chunks of TC MFMA steps (128
        // VGPRs of fp16 operands) before any of them is consumed, so their
        // L2 latency overlaps instead of stalling every MFMA.
        constexpr int TC = 32 / MT;
#pragma unroll
        for (int t0 = 0; t0 < 32; t0 += TC) {
            half8_t a[TC][MT];
#pragma unroll
            for (int tt = 0; tt < TC; ++tt)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    a[tt][mt] = load_x8<XT>(xrow[mt] + xoff + 8 * (t0 + tt) * XS);
            // keep the whole batch of loads ahead of the first consumer (the
            // scheduler would otherwise sink each load next to its MFMA)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int tt = 0; tt < TC; ++tt) {
#pragma unroll
                for (int i = 0; i < NW; ++i) {
                    const half8_t b = wb[i].frag(t0 + tt);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        acc[i][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tt][mt], b, acc[i][mt], 0, 0, 0);
                }
            }
        }
        // inside the loop: the accumulator copies at the loop exit must come
        // after these wait states
        kq_mfma_drain();
    }
}

}  // namespace kqmma
