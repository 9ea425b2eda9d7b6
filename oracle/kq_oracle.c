/*
 * CPU ORACLE -- test infrastructure only.
 *
 * Plain-C restatement of the GGUF K-quant codecs that gmlx binds through the
 * un-vendored `mlx-kquant` package (pinned >=0.3.13,<0.4 at
 * /root/reference/pyproject.toml:26-34).  That package is absent from the
 * reference tree, so the arithmetic follows the public GGML block definitions
 * (ggml-common.h block layouts, ggml-quants.c dequantize_row_* and the
 * *_ref quantizers of llama.cpp), restated here in this file's own code:
 *
 *   - dequantization (Q4_K, Q6_K, IQ2_XXS): the GGML evaluation order in
 *     fp32 with no FMA contraction (build with -ffp-contract=off).  This is the
 *     bit-exact target for every GPU dequant.  Call sites it stands in for:
 *     kq.dequantize at gmlx/modules.py:1461, gmlx/dsv32_patches.py:229.
 *   - quantization (Q4_K, Q6_K): llama.cpp's reference quantizers
 *     (make_qkx2_quants / make_qx_quants search).  kq.quantize call sites:
 *     tests/test_dequant_unattachable.py:36, gmlx/mtp_load.py:290.
 *     mlx-kquant's own quantizer choices are NOT pinned (no import possible).
 *   - quantization (IQ2_XXS): this build's own nearest-lattice search; it
 *     produces valid blocks but is not llama.cpp's iq2xs_init_impl search.
 *   - an OpenMP fp32 dequant-fused GEMM and a ragged decode attention used
 *     only as the reported CPU baseline (the reference's CPU path, MLX CPU /
 *     mlx-kquant NEON kernels, cannot run on x86).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library.  The product never does.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "kq_oracle_tables.h"

#define QK_K 256

/* ---------------------------------------------------------------- fp16 */

float kqo_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24, exact in fp32 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Round-to-nearest-even fp32 -> fp16, subnormals and overflow to inf. */
uint16_t kqo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* inf / nan */
        return sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u);
    }
    if (ax >= 0x477FF000u) { /* rounds to >= 65520 -> inf */
        return sign | 0x7C00u;
    }
    if (ax < 0x38800000u) { /* below 2^-14: fp16 subnormal or zero */
        if (ax < 0x33000000u) return sign; /* < 2^-25 rounds to 0 */
        const uint32_t e = ax >> 23;              /* biased fp32 exponent */
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;          /* 14 + (127 - e) - 1 ... */
        /* value = m * 2^(e-150); fp16 subnormal unit = 2^-24 -> m >> (126 - e) */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return sign | (uint16_t)q;
    }
    /* normal */
    uint32_t r = ax + 0xC8000000u; /* rebias exponent: -112 << 23 */
    const uint32_t lsb = (r >> 13) & 1u;
    r += 0xFFFu + lsb;
    return sign | (uint16_t)(r >> 13);
}

static inline int rne_int(float v) { return (int)rintf(v); }

/* ---------------------------------------------------------------- Q4_K */
/* Block (144 B): d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16. */

static inline void q4k_scale_min(int j, const uint8_t *s, uint8_t *sc, uint8_t *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

void kqo_dequant_q4_k(const uint8_t *wire, int64_t nblocks, float *out) {
    for (int64_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = wire + b * 144;
        uint16_t dh, mh;
        memcpy(&dh, blk, 2);
        memcpy(&mh, blk + 2, 2);
        const float d = kqo_f16_to_f32(dh);
        const float dmin = kqo_f16_to_f32(mh);
        const uint8_t *sc = blk + 4;
        const uint8_t *qs = blk + 16;
        float *y = out + b * QK_K;
        for (int c = 0; c < 4; ++c) {
            uint8_t s0, m0, s1, m1;
            q4k_scale_min(2 * c, sc, &s0, &m0);
            q4k_scale_min(2 * c + 1, sc, &s1, &m1);
            const float d1 = d * (float)s0, n1 = dmin * (float)m0;
            const float d2 = d * (float)s1, n2 = dmin * (float)m1;
            for (int l = 0; l < 32; ++l) {
                y[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0xF) - n1;
                y[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - n2;
            }
        }
    }
}

/* llama.cpp make_qkx2_quants: weighted min/scale search for an asymmetric
 * nmax-level quantizer of n values.  Returns scale, writes -min. */
static float qkx2_search(int n, int nmax, const float *x, const float *w, uint8_t *L,
                         float *neg_min, uint8_t *Laux, float rmin, float rdelta, int nstep) {
    float lo = x[0], hi = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (lo > 0) lo = 0;
    if (hi == lo) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *neg_min = -lo;
        return 0.f;
    }
    float iscale = (float)nmax / (hi - lo);
    float scale = 1.f / iscale;
    float best = 0;
    for (int i = 0; i < n; ++i) {
        int l = rne_int(iscale * (x[i] - lo));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t)l;
        float diff = scale * (float)L[i] + lo - x[i];
        diff = diff * diff;
        best += w[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (hi - lo);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = rne_int(iscale * (x[i] - lo));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            const float fl = (float)l;
            sum_l += w[i] * fl;
            sum_l2 += w[i] * fl * fl;
            sum_xl += w[i] * fl * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float err = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * (float)Laux[i] + this_min - x[i];
                diff = diff * diff;
                err += w[i] * diff;
            }
            if (err < best) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best = err;
                scale = this_scale;
                lo = this_min;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

void kqo_quantize_q4_k(const float *xin, int64_t nblocks, uint8_t *wire) {
    for (int64_t b = 0; b < nblocks; ++b) {
        const float *x = xin + b * QK_K;
        uint8_t *blk = wire + b * 144;
        uint8_t L[QK_K], Laux[32];
        float w[32], mins[8], scales[8];
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32.f);
            for (int l = 0; l < 32; ++l) w[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = qkx2_search(32, 15, x + 32 * j, w, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        uint8_t *sc = blk + 4;
        memset(sc, 0, 12);
        for (int j = 0; j < 8; ++j) {
            int ls = rne_int(inv_scale * scales[j]);
            int lm = rne_int(inv_min * mins[j]);
            ls = ls > 63 ? 63 : ls;
            lm = lm > 63 ? 63 : lm;
            if (j < 4) {
                sc[j] = (uint8_t)ls;
                sc[j + 4] = (uint8_t)lm;
            } else {
                sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
                sc[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        const uint16_t dh = kqo_f32_to_f16(max_scale / 63.f);
        const uint16_t mh = kqo_f32_to_f16(max_min / 63.f);
        memcpy(blk, &dh, 2);
        memcpy(blk + 2, &mh, 2);
        const float d = kqo_f16_to_f32(dh), dmin = kqo_f16_to_f32(mh);
        for (int j = 0; j < 8; ++j) {
            uint8_t s, m;
            q4k_scale_min(j, sc, &s, &m);
            const float dd = d * (float)s;
            if (dd == 0.f) continue;
            const float dm = dmin * (float)m;
            for (int i = 0; i < 32; ++i) {
                int l = rne_int((x[32 * j + i] + dm) / dd);
                l = l < 0 ? 0 : (l > 15 ? 15 : l);
                L[32 * j + i] = (uint8_t)l;
            }
        }
        uint8_t *qs = blk + 16;
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 32; ++l)
                qs[32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
    }
}

/* ---------------------------------------------------------------- Q6_K */
/* Block (210 B): ql[128] @0, qh[64] @128, scales int8[16] @192, d f16 @208. */

void kqo_dequant_q6_k(const uint8_t *wire, int64_t nblocks, float *out) {
    for (int64_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = wire + b * 210;
        uint16_t dh;
        memcpy(&dh, blk + 208, 2);
        const float d = kqo_f16_to_f32(dh);
        float *y = out + b * QK_K;
        for (int h = 0; h < 2; ++h) {
            const uint8_t *ql = blk + 64 * h;
            const uint8_t *qh = blk + 128 + 32 * h;
            const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[128 * h + l] = d * (float)sc[is + 0] * (float)q1;
                y[128 * h + l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[128 * h + l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[128 * h + l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
}

/* llama.cpp make_qx_quants with rmse_type 1 (weights x^2), no importance. */
static float qx_search(int n, int nmax, const float *x, int8_t *L) {
    float vmax = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            vmax = x[i];
        }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -(float)nmax / vmax;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = rne_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0.f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / vmax;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = rne_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = rne_int(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                L[i] = (int8_t)(l + nmax);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

void kqo_quantize_q6_k(const float *xin, int64_t nblocks, uint8_t *wire) {
    for (int64_t b = 0; b < nblocks; ++b) {
        const float *x = xin + b * QK_K;
        uint8_t *blk = wire + b * 210;
        int8_t L[QK_K];
        float scales[16];
        float max_scale = 0, max_abs = 0;
        for (int ib = 0; ib < 16; ++ib) {
            const float s = qx_search(16, 32, x + 16 * ib, L + 16 * ib);
            scales[ib] = s;
            if (fabsf(s) > max_abs) {
                max_abs = fabsf(s);
                max_scale = s;
            }
        }
        memset(blk, 0, 210);
        if (max_abs < 1e-15f) continue; /* all-zero block: d = +0 */
        const float iscale = -128.f / max_scale;
        const uint16_t dh = kqo_f32_to_f16(1.f / iscale);
        memcpy(blk + 208, &dh, 2);
        int8_t *sc = (int8_t *)(blk + 192);
        for (int ib = 0; ib < 16; ++ib) {
            int v = rne_int(iscale * scales[ib]);
            sc[ib] = (int8_t)(v > 127 ? 127 : v);
        }
        const float d = kqo_f16_to_f32(dh);
        for (int j = 0; j < 16; ++j) {
            const float dd = d * (float)sc[j];
            if (dd == 0.f) continue;
            for (int i = 0; i < 16; ++i) {
                int l = rne_int(x[16 * j + i] / dd);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                L[16 * j + i] = (int8_t)(l + 32);
            }
        }
        uint8_t *ql = blk, *qh = blk + 128;
        for (int h = 0; h < 2; ++h) {
            const int8_t *Lh = L + 128 * h;
            for (int l = 0; l < 32; ++l) {
                const uint8_t a = (uint8_t)Lh[l], bq = (uint8_t)Lh[l + 32];
                const uint8_t c = (uint8_t)Lh[l + 64], e = (uint8_t)Lh[l + 96];
                ql[64 * h + l] = (uint8_t)((a & 0xF) | ((c & 0xF) << 4));
                ql[64 * h + l + 32] = (uint8_t)((bq & 0xF) | ((e & 0xF) << 4));
                qh[32 * h + l] = (uint8_t)((a >> 4) | ((bq >> 4) << 2) | ((c >> 4) << 4) | ((e >> 4) << 6));
            }
        }
    }
}

/* ------------------------------------------------------------- IQ2_XXS */
/* Block (66 B): d f16 @0, qs[64] @2 = 8 groups x (4 grid-index bytes,
 * u32 with four 7-bit sign indices at bits 7l and a 4-bit scale at 28). */

static inline uint8_t iq2_signs(uint32_t idx7) {
    return (uint8_t)(idx7 | ((uint32_t)(__builtin_popcount(idx7) & 1) << 7));
}

void kqo_dequant_iq2_xxs(const uint8_t *wire, int64_t nblocks, float *out) {
    for (int64_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = wire + b * 66;
        uint16_t dh;
        memcpy(&dh, blk, 2);
        const float d = kqo_f16_to_f32(dh);
        float *y = out + b * QK_K;
        for (int g = 0; g < 8; ++g) {
            uint32_t aux[2];
            memcpy(aux, blk + 2 + 8 * g, 8);
            const float db = d * (0.5f + (float)(aux[1] >> 28)) * 0.25f;
            for (int l = 0; l < 4; ++l) {
                const uint64_t gv = KQO_IQ2XXS_GRID[(aux[0] >> (8 * l)) & 0xFF];
                const uint8_t s = iq2_signs((aux[1] >> (7 * l)) & 127);
                for (int j = 0; j < 8; ++j) {
                    const float gj = (float)((gv >> (8 * j)) & 0xFF);
                    y[32 * g + 8 * l + j] = db * gj * ((s >> j) & 1 ? -1.f : 1.f);
                }
            }
        }
    }
}

/* This build's own IQ2_XXS quantizer (the GPU kernel quant_iq2xxs_kernel
 * runs the same operations in the same order):
 *   d = fp16(amax / (43 * 15.5 * 0.25)) per block;
 *   per 32-value group and 8-value sub-group: signs folded so that an even
 *   number are negative (the smallest magnitude gives way), the 7-bit sign
 *   index kept, values multiplied by their folded sign;
 *   per scale field s (db = d (0.5 + s) / 4): every folded value takes the
 *   nearest grid level (8, 25, 43: below 16.5 db level 0, below 34 db level
 *   1, else 2), the sub-group's lattice point u = sum l_j 3^j maps to the
 *   grid entry nearest in level values (integer squared distance, ties to
 *   the lower entry), and the squared error of the 32 values is summed;
 *   the least error wins (ties to the lower s). */
static uint8_t iq2_near[6561];
static int iq2_near_ready = 0;

static void iq2_build_near(void) {
    static const int val[3] = {8, 25, 43};
    for (int u = 0; u < 6561; ++u) {
        int lv[8];
        for (int j = 0, r = u; j < 8; ++j, r /= 3) lv[j] = r % 3;
        int best = 0x7FFFFFFF, bk = 0;
        for (int k = 0; k < 256; ++k) {
            const uint64_t gv = KQO_IQ2XXS_GRID[k];
            int dsum = 0;
            for (int j = 0; j < 8; ++j) {
                const int dd = val[lv[j]] - (int)((gv >> (8 * j)) & 0xFF);
                dsum += dd * dd;
            }
            if (dsum < best) {
                best = dsum;
                bk = k;
            }
        }
        iq2_near[u] = (uint8_t)bk;
    }
    iq2_near_ready = 1;
}

const uint8_t *kqo_iq2_near_table(void) {
    if (!iq2_near_ready) iq2_build_near();
    return iq2_near;
}

void kqo_quantize_iq2_xxs(const float *xin, int64_t nblocks, uint8_t *wire) {
    const uint8_t *near = kqo_iq2_near_table();
    for (int64_t b = 0; b < nblocks; ++b) {
        const float *x = xin + b * QK_K;
        uint8_t *blk = wire + b * 66;
        memset(blk, 0, 66);
        float amax = 0;
        for (int i = 0; i < QK_K; ++i)
            if (fabsf(x[i]) > amax) amax = fabsf(x[i]);
        if (amax < 1e-30f) continue;
        /* grid magnitudes reach 43; scale field 15 gives db = d * 15.5 / 4 */
        const float dguess = amax / (43.f * 15.5f * 0.25f);
        const uint16_t dh = kqo_f32_to_f16(dguess);
        memcpy(blk, &dh, 2);
        const float d = kqo_f16_to_f32(dh);
        for (int g = 0; g < 8; ++g) {
            const float *xg = x + 32 * g;
            float folded[32], wt[32];
            uint32_t sign_idx[4];
            for (int i = 0; i < 32; ++i) wt[i] = fabsf(xg[i]); /* sign-flip cost */
            for (int l = 0; l < 4; ++l) {
                uint32_t s = 0;
                int nneg = 0, jmin = 0;
                for (int j = 0; j < 8; ++j) {
                    if (xg[8 * l + j] < 0) {
                        s |= 1u << j;
                        nneg++;
                    }
                    if (wt[8 * l + j] < wt[8 * l + jmin]) jmin = j;
                }
                if (nneg & 1) s ^= 1u << jmin; /* parity: flip cheapest */
                sign_idx[l] = s & 127u;
                /* the folded sign of element 7 is implied by parity */
                const uint8_t full = iq2_signs(sign_idx[l]);
                for (int j = 0; j < 8; ++j) folded[8 * l + j] = (full >> j) & 1 ? -xg[8 * l + j] : xg[8 * l + j];
            }
            float best_err = INFINITY;
            uint32_t best_s = 0, best_idx = 0;
            for (uint32_t sfield = 0; sfield < 16; ++sfield) {
                const float db = d * (0.5f + (float)sfield) * 0.25f;
                const float t01 = db * 16.5f, t12 = db * 34.f;
                float err_tot = 0;
                uint32_t idx_word = 0;
                for (int l = 0; l < 4; ++l) {
                    int u = 0;
                    for (int j = 7; j >= 0; --j) {
                        const float f = folded[8 * l + j];
                        u = 3 * u + (f < t01 ? 0 : (f < t12 ? 1 : 2));
                    }
                    const uint32_t k = near[u];
                    const uint64_t gv = KQO_IQ2XXS_GRID[k];
                    float e = 0;
                    for (int j = 0; j < 8; ++j) {
                        const float q = db * (float)((gv >> (8 * j)) & 0xFF);
                        const float diff = q - folded[8 * l + j];
                        e += diff * diff;
                    }
                    err_tot += e;
                    idx_word |= k << (8 * l);
                }
                if (err_tot < best_err) {
                    best_err = err_tot;
                    best_s = sfield;
                    best_idx = idx_word;
                }
            }
            uint32_t aux1 = best_s << 28;
            for (int l = 0; l < 4; ++l) aux1 |= sign_idx[l] << (7 * l);
            memcpy(blk + 2 + 8 * g, &best_idx, 4);
            memcpy(blk + 2 + 8 * g + 4, &aux1, 4);
        }
    }
}

/* ------------------------------------------------------ CPU baselines */

typedef void (*dequant_fn)(const uint8_t *, int64_t, float *);

static dequant_fn pick_dequant(int codec, int *bpb) {
    switch (codec) {
    case 12: *bpb = 144; return kqo_dequant_q4_k;
    case 14: *bpb = 210; return kqo_dequant_q6_k;
    case 16: *bpb = 66; return kqo_dequant_iq2_xxs;
    default: return 0;
    }
}

/* y[M,N] (fp32) = x[M,K] (fp16) . dequant(W[N,K])^T, fp32 accumulation,
 * one weight row dequantized at a time (fused, no materialized matrix).
 * Returns 0, or -1 for an unknown codec. */
int kqo_qmm_f32(const uint16_t *x, int M, int K, const uint8_t *wire, int N, int codec,
                float *y, int nthreads) {
    int bpb = 0;
    dequant_fn deq = pick_dequant(codec, &bpb);
    if (!deq || K % QK_K) return -1;
    const int nb = K / QK_K;
    const int64_t row_bytes = (int64_t)nb * bpb;
#pragma omp parallel num_threads(nthreads)
    {
        float wrow[K];
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            deq(wire + (int64_t)n * row_bytes, nb, wrow);
            for (int m = 0; m < M; ++m) {
                const uint16_t *xm = x + (int64_t)m * K;
                float acc = 0.f;
                for (int k = 0; k < K; ++k) acc += kqo_f16_to_f32(xm[k]) * wrow[k];
                y[(int64_t)m * N + n] = acc;
            }
        }
    }
    return 0;
}

/* Ragged GQA decode attention, fp32 online softmax over each row's keys.
 * q [B, Hq, D] fp16; per row b the keys of kv head h start at element
 * k + kv_off[b] + h * head_stride[b] with D-contiguous tokens; row_len[b]
 * tokens.  out [B, Hq, D] fp32. */
void kqo_ragged_attn_f32(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                         const int64_t *kv_off, const int64_t *head_stride,
                         const int32_t *row_len, int B, int Hq, int Hkv, int D, float scale,
                         float *out, int nthreads) {
    const int G = Hq / Hkv;
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(nthreads)
    for (int b = 0; b < B; ++b) {
        for (int hq = 0; hq < Hq; ++hq) {
            const int h = hq / G;
            float qf[D], o[D];
            for (int i = 0; i < D; ++i) {
                qf[i] = kqo_f16_to_f32(q[((int64_t)b * Hq + hq) * D + i]) * scale;
                o[i] = 0.f;
            }
            const uint16_t *kb = k + kv_off[b] + (int64_t)h * head_stride[b];
            const uint16_t *vb = v + kv_off[b] + (int64_t)h * head_stride[b];
            float mx = -INFINITY, l = 0.f;
            for (int t = 0; t < row_len[b]; ++t) {
                float s = 0.f;
                for (int i = 0; i < D; ++i) s += qf[i] * kqo_f16_to_f32(kb[(int64_t)t * D + i]);
                const float nm = s > mx ? s : mx;
                const float f = expf(mx - nm), p = expf(s - nm);
                l = l * f + p;
                for (int i = 0; i < D; ++i) o[i] = o[i] * f + p * kqo_f16_to_f32(vb[(int64_t)t * D + i]);
                mx = nm;
            }
            for (int i = 0; i < D; ++i)
                out[((int64_t)b * Hq + hq) * D + i] = l > 0.f ? o[i] / l : 0.f;
        }
    }
}

int kqo_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
