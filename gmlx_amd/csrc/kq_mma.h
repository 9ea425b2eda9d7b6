// Wave-level dequant-fused MFMA tile for GGUF K-quant weights (gfx950).
//
// Tile: one wave computes C[16*MT batch rows, 16 weight rows] over a set of
// super-blocks with v_mfma_f32_16x16x32_f16 (A = activations, B = weights^T).
// Lane l = 16*g + r: r selects the weight row (B column) and the activation
// row (A row) the lane feeds; g selects which 8 of the MFMA's 32 k values.
// One super-block takes 8 MFMA steps t = 0..7.  Q4_K and Q6_K: step t covers
// the 32 values 32t .. 32t+31 of the block and lane group g feeds values
// 32t + 8g .. +7, so the 4 lane groups of one activation row read one
// contiguous 64-byte run.  IQ2_XXS: lane group g owns the quarter 64g .. 64g+63
// (one 16-byte load of the block per lane) and feeds 64g + 8t .. +7.  The
// activation fragment of a step is the 8 activations at the same value
// indices (Block<>::x_elem).
//
// Exact weights.  The MFMA's B operand is an exact integer in fp16, the
// block's integer codes times its integer sub-block scales:
//   Q4_K : q * sc                 (q <= 15, sc <= 63: at most 945)
//   Q6_K : (q - 32) * sc          (|.| <= 4096; exact up to 2048, beyond that
//                                  an odd product rounds to the nearest even)
//   IQ2  : +-grid * (2 s + 1)     (grid in {8, 25, 43}, s <= 15: at most 1333)
// Each super-block's eight steps run as their own MFMA chain P (exact
// products, fp32 sums), and the chain is folded into the fp32 accumulator
// with the block's fp32 factor: acc += d * P (IQ2_XXS: d / 8).  The Q4_K
// minimum term -dmin * m_j * sum_{l in j} x_l takes fp32 sub-block sums of
// the activations (sub-block j of the super-block, from a 0 / 1 selection
// MFMA, sum_sel below) against -dmin * m_j (exact in fp32) on the fp32 MFMA
// v_mfma_f32_16x16x4_f32 (min_accumulate).  No scale is rounded to fp16, so
// the only rounding left is fp32 accumulation (and Q6_K's even rounding of
// products past 2048, unbiased and independent per weight).
#pragma once
#include "kq_common.h"
#include "kq_tables.h"

namespace kqmma {

// ---- IQ2_XXS tables in fp16 form, built at compile time ------------------
constexpr uint32_t mag_to_f16_bits(uint32_t b) { return b == 0x08 ? 0x4800u : b == 0x19 ? 0x4E40u : 0x5160u; }

// 16-byte aligned rows: an entry is one ds_read_b128 (with 4-byte alignment
// the compiler splits it into two ds_read2_b32).
struct alignas(16) Iq2Tables {
    alignas(16) uint32_t grid_h2[256][4];  // 8 fp16 magnitudes per grid entry
    alignas(16) uint32_t sign_x2[128][4];  // XOR masks (0x8000 per negative value)
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

// Copy the IQ2_XXS tables into a workgroup's LDS (6 KB); every thread of the
// workgroup must call it, and it ends with a workgroup barrier.
__device__ __forceinline__ void load_iq2_tables(Iq2Tables &dst) {
    const u32x4 *src = (const u32x4 *)&kIq2;
    u32x4 *d = (u32x4 *)&dst;
    constexpr int n = (int)(sizeof(Iq2Tables) / 16);
    for (int i = threadIdx.x; i < n; i += blockDim.x) d[i] = src[i];
    __syncthreads();
}

// ---- per-codec block decoders (the lane's view of one super-block) -------

__device__ __forceinline__ half2_t h2b(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ half2_t bcast(_Float16 v) { return half2_t{v, v}; }

// 8 bytes (two dwords, each value in [0, 63]) -> 8 fp16 (1024 + byte)
struct Bias8 {
    half2_t p0, p1, p2, p3;
    __device__ __forceinline__ Bias8(uint32_t w0, uint32_t w1)
        : p0(h2b(kq_bytes_to_h2_biased(w0, KQ_SEL_B01))), p1(h2b(kq_bytes_to_h2_biased(w0, KQ_SEL_B23))),
          p2(h2b(kq_bytes_to_h2_biased(w1, KQ_SEL_B01))), p3(h2b(kq_bytes_to_h2_biased(w1, KQ_SEL_B23))) {}
};

__device__ __forceinline__ half8_t cat8(half2_t a, half2_t b, half2_t c, half2_t d) {
    return half8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

template <int CODEC>
struct Block;

// Q4_K (144 B = d, dmin, 12 B packed scales, 128 B qs; 16-B aligned).
// Step t = sub-block t: qs chunk c = t/2 (bytes 32c .. 32c+31), low nibbles for
// even t, high for odd t; lane group g takes bytes 32c + 8g .. +7.
// The 8 six-bit scales and mins are unpacked four at a time as bytes:
//   sub-blocks 0..3: sc = s[j] & 63,                    m = s[j+4] & 63
//   sub-blocks 4..7: sc = s[j+4] & 15 | (s[j-4] >> 6) << 4,
//                    m  = s[j+4] >> 4 | (s[j] >> 6) << 4
// and the scales become exact fp16 integers through the 1024-bias.  A nibble
// byte q <= 15 read as fp8 E4M3 is q * 2^-9; the converter's scale 2^9 (a
// power of two, the only part of the scale it applies) returns q exactly, and
// q * sc (at most 945) is exact in fp16.
template <>
struct Block<KQ_CODEC_Q4_K> {
    u32x4 hdr;
    u32x2 q[4];
    half2_t sc[4];          // [i] = integer scales of sub-blocks 2i, 2i+1
    uint32_t mlo, mhi;      // integer mins, one byte per sub-block (0..3, 4..7)
    float d, dmin;

    __device__ static constexpr int x_elem(int t, int g) { return 32 * t + 8 * g; }
    __device__ __forceinline__ void load(const uint8_t *blk, int g) {
        hdr = *(const u32x4 *)blk;
#pragma unroll
        for (int c = 0; c < 4; ++c) q[c] = *(const u32x2 *)(blk + 16 + 32 * c + 8 * g);
    }
    __device__ __forceinline__ void prep(int g) {
        (void)g;
        const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;  // scale bytes 0..3, 4..7, 8..11
        const uint32_t sc_lo = s0 & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
        mlo = s1 & 0x3F3F3F3Fu;
        mhi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
        const half2_t k1024 = {(_Float16)1024.f, (_Float16)1024.f};
        const uint32_t scw[2] = {sc_lo, sc_hi};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            sc[i] = h2b(__builtin_amdgcn_perm(0x64646464u, scw[i >> 1], (i & 1) ? KQ_SEL_B23 : KQ_SEL_B01)) - k1024;
        d = kq_f16_bits_to_f32(hdr.x & 0xFFFFu);
        dmin = kq_f16_bits_to_f32(hdr.x >> 16);
    }
    __device__ __forceinline__ half8_t frag(int t, int g, const Iq2Tables &) const {
        (void)g;
        uint32_t w0 = q[t >> 1].x, w1 = q[t >> 1].y;
        if (t & 1) {
            w0 >>= 4;
            w1 >>= 4;
        }
        w0 &= 0x0F0F0F0Fu;
        w1 &= 0x0F0F0F0Fu;
        const half2_t s = bcast((t & 1) ? sc[t >> 1].y : sc[t >> 1].x);
        const half2_t a0 = h2b(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 512.f, false)));
        const half2_t a1 = h2b(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 512.f, true)));
        const half2_t a2 = h2b(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 512.f, false)));
        const half2_t a3 = h2b(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 512.f, true)));
        return cat8(a0 * s, a1 * s, a2 * s, a3 * s);
    }
    __device__ __forceinline__ float dscale() const { return d; }
    // The integer minimum m of sub-block t (0..63, exact in fp16) in all eight
    // values: as the B operand of step t against the activation fragment it
    // gives m_t * (sum of the step's 32 activations) per row, a chain that
    // folds in with -dmin.
    __device__ __forceinline__ half8_t min_frag(int t) const {
        const uint32_t b = (uint32_t)(t & 3);
        const half2_t k1024 = {(_Float16)1024.f, (_Float16)1024.f};
        const uint32_t sel = b | (4u << 8) | (b << 16) | (4u << 24);  // byte t of the word under 0x64 bytes
        const half2_t m = h2b(__builtin_amdgcn_perm(0x64646464u, t < 4 ? mlo : mhi, sel)) - k1024;
        return cat8(m, m, m, m);
    }
    // -dmin * m of sub-blocks 2g and 2g + 1 (exact in fp32): the B operand of
    // the minimum MFMAs (min_accumulate)
    __device__ __forceinline__ void min_b(int g, float &b0, float &b1) const {
        const uint32_t w = (g >= 2 ? mhi : mlo) >> (16 * (g & 1));
        b0 = -dmin * (float)(w & 0xFFu);
        b1 = -dmin * (float)((w >> 8) & 0xFFu);
    }
};

// Q6_K (210 B = ql[128] qh[64] scales[16] d; only 2-byte aligned).
// Step t: half h = t/4, quarter q = t%4 (values 128h + 32q + l, l = 0..31);
// lane group g takes l = 8g .. 8g+7: ql bytes 64h + 32(q&1) + 8g (high
// nibbles for q >= 2), qh bytes 32h + 8g (bits 2q, 2q+1), one int8 scale
// sc[8h + 2q + g/2].  The fragment is (q6 - 32) * sc (an integer of at most
// 4096 in magnitude), times d in fp32 after the chain.
template <>
struct Block<KQ_CODEC_Q6_K> {
    u32x2 ql[4];  // [2h + p]
    u32x2 qh[2];  // [h]
    u32x4 sc;     // scales[16]
    uint32_t dbits;
    half2_t isc[8];  // the lane's int8 scale of step t, as fp16
    float d;

    __device__ static constexpr int x_elem(int t, int g) { return 32 * t + 8 * g; }
    __device__ __forceinline__ void load(const uint8_t *blk, int g) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x2_a2 v = *(const u32x2_a2 *)(blk + 64 * (i >> 1) + 32 * (i & 1) + 8 * g);
            ql[i] = u32x2{v.x, v.y};
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const u32x2_a2 v = *(const u32x2_a2 *)(blk + 128 + 32 * h + 8 * g);
            qh[h] = u32x2{v.x, v.y};
        }
        const u32x4_a2 s = *(const u32x4_a2 *)(blk + 192);
        sc = u32x4{s.x, s.y, s.z, s.w};
        dbits = (uint32_t)*(const uint16_t *)(blk + 208);
    }
    __device__ __forceinline__ void prep(int g) {
        d = kq_f16_bits_to_f32(dbits);
        const int sh = 8 * (g >> 1);
        const uint32_t w[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            // scale index 8h + 2q + g/2 = 2t + g/2: byte (2t + g/2) of the 16
            const int bi = 2 * t;
            const int8_t s = (int8_t)((w[bi >> 2] >> (8 * (bi & 3) + sh)) & 0xFF);
            isc[t] = bcast((_Float16)(float)s);
        }
    }
    __device__ __forceinline__ half8_t frag(int t, int g, const Iq2Tables &) const {
        (void)g;
        const int h = t >> 2, q = t & 3;
        uint32_t l0 = ql[2 * h + (q & 1)].x, l1 = ql[2 * h + (q & 1)].y;
        if (q >= 2) {
            l0 >>= 4;
            l1 >>= 4;
        }
        const uint32_t hq0 = qh[h].x, hq1 = qh[h].y;
        const int hs = 2 * q;
        uint32_t c0, c1;
        if (hs <= 4) {
            c0 = (l0 & 0x0F0F0F0Fu) | ((hq0 << (4 - hs)) & 0x30303030u);
            c1 = (l1 & 0x0F0F0F0Fu) | ((hq1 << (4 - hs)) & 0x30303030u);
        } else {
            c0 = (l0 & 0x0F0F0F0Fu) | ((hq0 >> (hs - 4)) & 0x30303030u);
            c1 = (l1 & 0x0F0F0F0Fu) | ((hq1 >> (hs - 4)) & 0x30303030u);
        }
        const Bias8 b(c0, c1);
        const half2_t k1056 = {(_Float16)1056.f, (_Float16)1056.f};
        const half2_t s = isc[t];
        return cat8((b.p0 - k1056) * s, (b.p1 - k1056) * s, (b.p2 - k1056) * s, (b.p3 - k1056) * s);
    }
    __device__ __forceinline__ float dscale() const { return d; }
};

// IQ2_XXS (66 B = d + 8 groups of 8 B: 4 grid indices, u32 signs|scale).
// Lane group g owns groups 2g and 2g+1 (bytes 2 + 16g .. +15: one 16-B load
// per lane) and the values 64g .. 64g+63; step t covers values 64g + 8t .. +7
// (group 2g + t/4, grid index t%4).  The grid and sign tables are read from
// LDS.  Value = d * (0.5 + s) * 0.25 * grid * sign = (d / 8) * (2s + 1) * grid
// * sign: the fragment is the integer (2s + 1) * grid * sign, times d / 8 in
// fp32 after the chain.
template <>
struct Block<KQ_CODEC_IQ2_XXS> {
    u32x4 raw;  // index word, sign|scale word of group 2g, then of group 2g+1
    uint32_t dbits;
    half2_t os[2];  // 2 s + 1 of groups 2g, 2g + 1
    float d8;

    __device__ static constexpr int x_elem(int t, int g) { return 64 * g + 8 * t; }
    __device__ __forceinline__ void load(const uint8_t *blk, int g) {
        const u32x4_a2 v = *(const u32x4_a2 *)(blk + 2 + 16 * g);
        raw = u32x4{v.x, v.y, v.z, v.w};
        dbits = (uint32_t)*(const uint16_t *)blk;
    }
    __device__ __forceinline__ void prep(int g) {
        (void)g;
        d8 = kq_f16_bits_to_f32(dbits) * 0.125f;
        os[0] = bcast((_Float16)(float)(2u * (raw.y >> 28) + 1u));
        os[1] = bcast((_Float16)(float)(2u * (raw.w >> 28) + 1u));
    }
    __device__ __forceinline__ half8_t frag(int t, int g, const Iq2Tables &tab) const {
        (void)g;
        const int e = t >> 2, l = t & 3;
        const uint32_t gw = e ? raw.z : raw.x, aux = e ? raw.w : raw.y;
        const uint32_t idx = (gw >> (8 * l)) & 0xFF;
        const uint32_t s7 = (aux >> (7 * l)) & 127u;
        const u32x4 gm = *(const u32x4 *)tab.grid_h2[idx];
        const u32x4 sm = *(const u32x4 *)tab.sign_x2[s7];
        const half2_t s = os[e];
        return cat8(h2b(gm.x ^ sm.x) * s, h2b(gm.y ^ sm.y) * s, h2b(gm.z ^ sm.z) * s, h2b(gm.w ^ sm.w) * s);
    }
    __device__ __forceinline__ float dscale() const { return d8; }
};

// ---- exact-weight accumulation helpers --------------------------------------

__device__ __forceinline__ floatx4 fzero4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }

// acc += f * p (one rounding per element)
__device__ __forceinline__ floatx4 fold4(float f, const floatx4 &p, const floatx4 &acc) {
    return floatx4{__builtin_fmaf(f, p[0], acc[0]), __builtin_fmaf(f, p[1], acc[1]), __builtin_fmaf(f, p[2], acc[2]),
                   __builtin_fmaf(f, p[3], acc[3])};
}

// Activation sub-block sums by MFMA: S = mfma(sum_sel(r, row), x fragment, S)
// with the fragment as the B operand (column = activation row of its lane)
// and a 0 / 1 selection as A: only A-row `row` takes this step's 32 values,
// so the lane (g, r) of the result accumulates in element e the sum of
// activation row r over the values whose steps selected row 4g + e (exact
// products, fp32 sums).  For the layout above (step t = sub-block t) the
// selection row of sub-block t in super-block slot s is sum_row(t, s):
// element e of lane (g, r) is then the sum of sub-block 2g + (e & 1) of slot
// e >> 1, which is what min_accumulate pairs with min_b.
__device__ __forceinline__ half8_t sum_sel(int r, int row) {
    const _Float16 v = r == row ? (_Float16)1.f : (_Float16)0.f;
    return half8_t{v, v, v, v, v, v, v, v};
}
__device__ __forceinline__ constexpr int sum_row(int t, int s) { return 4 * (t >> 1) + (t & 1) + 2 * s; }

// Sub-block sums of SB super-blocks of activation fragments in the layout
// above (xr[s][t]: step t of super-block slot s): element e of lane (g, r) =
// sum of activation row r over sub-block 2g + (e & 1) of slot e >> 1.
template <int SB>
__device__ __forceinline__ floatx4 xsum_generic(const half8_t (&xr)[SB][8], int r) {
    static_assert(SB <= 2, "one accumulator holds two super-blocks of sums");
    floatx4 S = fzero4();
#pragma unroll
    for (int s = 0; s < SB; ++s)
#pragma unroll
        for (int t = 0; t < 8; ++t) S = __builtin_amdgcn_mfma_f32_16x16x32_f16(sum_sel(r, sum_row(t, s)), xr[s][t], S, 0, 0, 0);
    return S;
}

// acc += sum_j S_j * (-dmin m_j) over the 8 sub-blocks of one super-block:
// two fp32 MFMAs with k = lane group g, A = the sums of sub-blocks 2g + i of
// the lane's activation row (s0, s1), B = -dmin m of the same sub-blocks of
// its weight row (b0, b1).
__device__ __forceinline__ floatx4 min_accumulate(float s0, float s1, float b0, float b1, floatx4 acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(s0, b0, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(s1, b1, acc, 0, 0, 0);
}

// ---- activation fragments -------------------------------------------------

// Activation element types: 0 = fp16, 1 = bf16, 2 = fp32.
template <int XT>
constexpr int x_elem_bytes() { return XT == 2 ? 4 : 2; }

// Raw 16 bytes -> 8 activations as fp16 (bf16 is converted, exact in the fp16
// normal range).
template <int XT>
__device__ __forceinline__ half8_t x8_from_bits(u32x4 v) {
    if constexpr (XT == 0) {
        return __builtin_bit_cast(half8_t, v);
    } else {
        half8_t h;
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h[2 * i] = (_Float16)__builtin_bit_cast(float, w[i] << 16);
            h[2 * i + 1] = (_Float16)__builtin_bit_cast(float, w[i] & 0xFFFF0000u);
        }
        return h;
    }
}

// 8 consecutive activations as fp16.  bf16 / fp32 inputs are converted
// (fp32 rounds to nearest).
template <int XT>
__device__ __forceinline__ half8_t load_x8(const char *p) {
    if constexpr (XT != 2) {
        return x8_from_bits<XT>(*(const u32x4 *)p);
    } else {
        const float4 a = *(const float4 *)p;
        const float4 b = *(const float4 *)(p + 16);
        return half8_t{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                       (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
    }
}

// Activation rows addressed by pointer (one per m-tile, already clamped to a
// valid row): the MoE gather, whose rows come from a pair table.
template <int MT>
struct XRowPtrs {
    const char *row[MT];
    template <int XT>
    __device__ __forceinline__ half8_t load(int mt, int elem) const {
        return load_x8<XT>(row[mt] + (int64_t)elem * x_elem_bytes<XT>());
    }
};

// Activation rows of a contiguous [rows, K] block read through a buffer
// resource whose size covers only the valid rows: a lane whose row is past
// the end gets an offset at the end of the buffer, and the hardware returns
// zeros without touching memory, so padding rows of a 16-row tile cost no
// memory traffic and need no branch.  Offsets are 32-bit bytes.
template <int MT>
struct XRowsBuf {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t row_off[MT];
    template <int XT>
    __device__ __forceinline__ half8_t load(int mt, int elem) const {
        const uint32_t off = row_off[mt] + (uint32_t)elem * (uint32_t)x_elem_bytes<XT>();
        if constexpr (XT != 2) {
            return x8_from_bits<XT>(__builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0)));
        } else {
            const u32x4 a = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
            const u32x4 b = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off + 16, 0, 0));
            return half8_t{(_Float16)__builtin_bit_cast(float, a.x), (_Float16)__builtin_bit_cast(float, a.y),
                           (_Float16)__builtin_bit_cast(float, a.z), (_Float16)__builtin_bit_cast(float, a.w),
                           (_Float16)__builtin_bit_cast(float, b.x), (_Float16)__builtin_bit_cast(float, b.y),
                           (_Float16)__builtin_bit_cast(float, b.z), (_Float16)__builtin_bit_cast(float, b.w)};
        }
    }
};

// Buffer resource over `bytes` bytes at `base` (raw, 32-bit data format).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t kq_buffer(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// XRowsBuf for rows [m0, m0 + 16*MT) of x[M, K] (row stride in elements):
// lane row m0 + 16*mt + r; rows >= M read as zeros.
template <int MT, int XT>
__device__ __forceinline__ XRowsBuf<MT> x_rows_buf(const char *x, int64_t stride, int M, int K, int m0, int r) {
    constexpr int XS = x_elem_bytes<XT>();
    XRowsBuf<MT> xr;
    const int rows = min(M - m0, 16 * MT);
    const uint32_t bytes = (uint32_t)(((int64_t)(rows - 1) * stride + K) * XS);
    xr.rsrc = kq_buffer(x + (int64_t)m0 * stride * XS, bytes);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r;
        xr.row_off[mt] = m < rows ? (uint32_t)((int64_t)m * stride * XS) : bytes;
    }
    return xr;
}

// One super-block's operands for a wave: NW weight blocks and the 8 MFMA
// steps' activation fragments of MT m-tiles.
template <int CODEC, int MT, int XT, int NW>
struct Stage {
    Block<CODEC> w[NW];
    half8_t x[8][MT];

    template <class XS>
    __device__ __forceinline__ void load(const uint8_t *const (&wrow)[NW], const XS &xs, int kb, int g) {
        constexpr int BPB = kq_block_bytes(CODEC);
#pragma unroll
        for (int i = 0; i < NW; ++i) w[i].load(wrow[i] + (int64_t)kb * BPB, g);
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                x[t][mt] = xs.template load<XT>(mt, kb * KQ_QK + Block<CODEC>::x_elem(t, g));
    }

    __device__ __forceinline__ void compute(floatx4 (&acc)[NW][MT], int g, const Iq2Tables &tab) {
#pragma unroll
        for (int i = 0; i < NW; ++i) w[i].prep(g);
        // Q4_K: the activations' sub-block sums, once for the NW tiles
        [[maybe_unused]] floatx4 sums[MT];
        if constexpr (CODEC == KQ_CODEC_Q4_K) {
            const int r = kq_lane() & 15;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) sums[mt] = fzero4();
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const half8_t sel = sum_sel(r, sum_row(t, 0));
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    sums[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, x[t][mt], sums[mt], 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            floatx4 p[MT];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const half8_t b = w[i].frag(t, g, tab);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    p[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[t][mt], b, t == 0 ? fzero4() : p[mt], 0, 0, 0);
            }
            const float f = w[i].dscale();
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[i][mt] = fold4(f, p[mt], acc[i][mt]);
            if constexpr (CODEC == KQ_CODEC_Q4_K) {
                float b0, b1;
                w[i].min_b(g, b0, b1);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) acc[i][mt] = min_accumulate(sums[mt][0], sums[mt][1], b0, b1, acc[i][mt]);
            }
        }
    }
};

// Accumulate super-blocks kb_first, kb_first + kb_step, ... < kb_end of NW
// weight matrices (NW = 2: gate and up share the activations).  wrow[i]
// points at this lane's weight row (row n0 + lane%16 of matrix i, clamped to
// a valid row by the caller).  xrow (XRowPtrs / XRowsBuf) yields this lane's
// activation fragments of each m-tile; rows past M feed outputs that are
// never stored.  With PREFETCH (and MT * NW <= 2) the next block's loads are
// issued before the current block is multiplied (register double buffer);
// without it each block is loaded and multiplied in turn, and the latency is
// hidden by the other resident waves.
template <int CODEC, int MT, int XT, int NW, class XS, bool PREFETCH = true>
__device__ __forceinline__ void tile_accumulate(const uint8_t *const (&wrow)[NW], int kb_first, int kb_step,
                                                int kb_end, const XS &xrow, floatx4 (&acc)[NW][MT],
                                                const Iq2Tables &tab) {
    const int g = kq_lane() >> 4;
    int kb = kb_first;
    if (kb >= kb_end) return;
    if (kb + kb_step >= kb_end) {
        // a single block for this wave: no prefetch stage
        Stage<CODEC, MT, XT, NW> st;
        st.load(wrow, xrow, kb, g);
        __builtin_amdgcn_sched_barrier(0);
        st.compute(acc, g, tab);
        kq_mfma_drain();
        return;
    }
    if constexpr (MT * NW > 2 || !PREFETCH) {
        // wide tiles: one stage (two would not fit the register file); or the
        // caller relies on many resident waves instead of a prefetch stage
        Stage<CODEC, MT, XT, NW> st;
        for (;;) {
            st.load(wrow, xrow, kb, g);
            __builtin_amdgcn_sched_barrier(0);
            st.compute(acc, g, tab);
            kb += kb_step;
            if (kb >= kb_end) {
                kq_mfma_drain();
                break;
            }
        }
        return;
    }
    // The prefetch loads are unconditional (past the end they re-read the
    // current block): a load under a branch makes the compiler's wait-count
    // merge at the join assume the short path and wait for the prefetch
    // before the current block's math, which serialises the pipeline.
    Stage<CODEC, MT, XT, NW> s0, s1;
    s0.load(wrow, xrow, kb, g);
    for (;;) {
        const int k1 = kb + kb_step;
        s1.load(wrow, xrow, k1 < kb_end ? k1 : kb, g);
        __builtin_amdgcn_sched_barrier(0);
        s0.compute(acc, g, tab);
        // at the exits: wait out the last MFMA's result latency inside the
        // loop body, ahead of the accumulator copies the compiler places at
        // the loop exit
        if (k1 >= kb_end) {
            kq_mfma_drain();
            break;
        }
        const int k2 = k1 + kb_step;
        s0.load(wrow, xrow, k2 < kb_end ? k2 : k1, g);
        __builtin_amdgcn_sched_barrier(0);
        s1.compute(acc, g, tab);
        if (k2 >= kb_end) {
            kq_mfma_drain();
            break;
        }
        kb = k2;
    }
}

}  // namespace kqmma
